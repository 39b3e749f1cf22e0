"""GPU: the DiT block (src/dit.h:183-247) and the DiT graph head
(src/dit.h:250-268) built with the restated ggml API and run through
ggml_backend_graph_compute on the MI355X backend, against a CPU float32
restatement of the same math with dequantized weights (torch on the CPU).

Tolerance (stated): cosine >= 0.9999 and relative RMS error <= 5e-3 on the
block output.  The backend follows ggml's arithmetic: activations are
quantized to Q8_0 before each Q8_0 dot and K/V are rounded to f16, both of
which the reference does in exact arithmetic except the f16 rounding of K/V,
which it applies too.  The first compute runs eagerly, later ones replay the
captured HIP graph: every replay must equal the eager result bit for bit."""
import ctypes
import importlib

import numpy as np
import pytest
import torch

from conftest import cosine

pytestmark = pytest.mark.gpu


def _mods(pkg):
    return importlib.import_module(pkg.__name__ + ".opgraph"), importlib.import_module(pkg.__name__ + ".ditgraph")


def _deq(orc, rows, k):
    if rows.dtype == np.uint16:  # BF16 rows: the f32 of each bf16
        return torch.from_numpy((rows.astype(np.uint32) << 16).view(np.float32))
    return torch.from_numpy(orc.dequantize(8, rows, k, rows.shape[0]).reshape(rows.shape[0], k))


def _ln(x, w, b, eps):
    m = x.mean(-1, keepdim=True)
    v = ((x - m) ** 2).mean(-1, keepdim=True)
    return (x - m) / torch.sqrt(v + eps) * w + b


def _rope(x, pos, n_dims, base):
    """x [B, S, H, D]: NeoX pairs (i, i + n_dims/2) of the first n_dims dims
    rotate by pos * base^(-2i/n_dims)."""
    half = n_dims // 2
    inv = base ** (-2.0 * torch.arange(half, dtype=torch.float64) / n_dims)
    ang = (pos.to(torch.float64)[:, None] * inv[None, :]).to(torch.float32)  # [S, half]
    c, s = torch.cos(ang)[None, :, None, :], torch.sin(ang)[None, :, None, :]
    y = x.clone()
    x0, x1 = x[..., :half], x[..., half:n_dims]
    y[..., :half] = x0 * c - x1 * s
    y[..., half:n_dims] = x0 * s + x1 * c
    return y


def ref_block(orc, dg, w, x, pos, ff):
    """x [B, S, dim] f32 on the CPU."""
    B, S, dim = x.shape
    Nh, D = dg.N_HEADS, dg.HEAD_DIM
    W = {n: _deq(orc, w[n], dim if n != "ff_out_w" else ff) for n in ("wq", "wk", "wv", "wo", "ff_in_w", "ff_out_w")}
    t = {n: torch.from_numpy(w[n]) for n in ("norm1_w", "norm1_b", "norm2_w", "norm2_b", "ff_in_b", "ff_out_b")}
    h = _ln(x, t["norm1_w"], t["norm1_b"], dg.LN_EPS)
    q = (h @ W["wq"].T).reshape(B, S, Nh, D)
    k = (h @ W["wk"].T).reshape(B, S, Nh, D)
    v = (h @ W["wv"].T).reshape(B, S, Nh, D)
    q = _rope(q, pos, dg.ROTARY_DIM, dg.ROPE_BASE)
    k = _rope(k, pos, dg.ROTARY_DIM, dg.ROPE_BASE).half().float()
    v = v.half().float()
    qh, kh, vh = (a.permute(0, 2, 1, 3).contiguous() for a in (q, k, v))
    p = torch.softmax((qh @ kh.transpose(-1, -2).contiguous()) / np.sqrt(D), dim=-1)
    a = (p @ vh).permute(0, 2, 1, 3).reshape(B, S, Nh * D)
    x = x + a @ W["wo"].T
    h = _ln(x, t["norm2_w"], t["norm2_b"], dg.LN_EPS)
    f = h @ W["ff_in_w"].T + t["ff_in_b"]
    value, gate = f[..., :ff], f[..., ff:]
    return x + (torch.nn.functional.silu(gate) * value) @ W["ff_out_w"].T + t["ff_out_b"]


@pytest.mark.parametrize("S,B,seed,wt", [(690, 2, 51, 8), (37, 1, 52, 8), (690, 2, 54, 30), (37, 1, 55, 30)])
def test_dit_block_through_backend(pkg, orc, S, B, seed, wt):
    """One DiT block at the model's shape (S = T + 1 = 690 tokens, CFG B = 2)
    and a ragged small case, with Q8_0 weights (wt 8) and with BF16 weights
    (wt 30, the native-BF16 files: every projection on the bf16 MFMA GEMM,
    activations rounded to bf16 as ggml's BF16 dot does)."""
    og, dg = _mods(pkg)
    torch.set_num_threads(16)
    w = dg.synth_block(seed, wtype=wt)
    rng = np.random.default_rng(seed + 100)
    x = rng.standard_normal((B, S, dg.DIM)).astype(np.float32)
    pos = np.arange(S, dtype=np.int32)
    g = og.OpGraph()
    try:
        blk = dg.Block(g, wtype=wt)
        tx = g.tensor(og.F32, [dg.DIM, S, B])
        tp = g.tensor(26, [S])  # GGML_TYPE_I32
        out = dg.build_block(g, blk, tx, tp, S, B)
        g.build([out])
        blk.upload(g, w)
        g.set(tx, x)
        g.set(tp, pos)
        g.compute()
        y0 = g.get(out).reshape(B, S, dg.DIM)
        for _ in range(2):
            g.compute()
            assert np.array_equal(g.get(out).reshape(B, S, dg.DIM), y0)
        replays, _ = g.graph_stats()
    finally:
        g.close()
    ref = ref_block(orc, dg, w, torch.from_numpy(x), torch.from_numpy(pos), dg.FF_INNER).numpy()
    assert np.isfinite(y0).all()
    rel_rms = float(np.sqrt(((y0.astype(np.float64) - ref) ** 2).mean() / (ref.astype(np.float64) ** 2).mean()))
    assert cosine(y0, ref) >= 0.9999 and rel_rms <= 5e-3, (cosine(y0, ref), rel_rms)
    assert replays >= 1


def test_dit_graph_head_through_backend(pkg, orc):
    """src/dit.h:250-268: concat [latent, zeros, condition], residual
    preprocess projection, proj_in, timestep token prepended (T = 689)."""
    og, dg = _mods(pkg)
    torch.set_num_threads(16)
    T, B = 689, 2
    rng = np.random.default_rng(53)
    xt = rng.standard_normal((B, T, dg.IN_CH)).astype(np.float32)
    cond = rng.standard_normal((B, T, dg.COND_DIM)).astype(np.float32)
    temb = rng.standard_normal((B, 1, dg.DIM)).astype(np.float32)
    pre = dg.q8_0_rows(rng, dg.CONCAT_CH, dg.CONCAT_CH)
    inw = dg.q8_0_rows(rng, dg.DIM, dg.CONCAT_CH)
    g = og.OpGraph()
    try:
        t_xt = g.tensor(og.F32, [dg.IN_CH, T, B])
        t_c = g.tensor(og.F32, [dg.COND_DIM, T, B])
        t_e = g.tensor(og.F32, [dg.DIM, 1, B])
        t_pre = g.tensor(og.Q8_0, [dg.CONCAT_CH, dg.CONCAT_CH])
        t_in = g.tensor(og.Q8_0, [dg.CONCAT_CH, dg.DIM])
        out = dg.build_input(g, t_xt, t_c, t_e, t_pre, t_in)
        g.build([out])
        for t, a in ((t_xt, xt), (t_c, cond), (t_e, temb), (t_pre, pre), (t_in, inw)):
            g.set(t, a)
        g.compute()
        y = g.get(out).reshape(B, T + 1, dg.DIM)
    finally:
        g.close()
    x = torch.cat([torch.from_numpy(xt), torch.zeros(B, T, dg.IN_CH), torch.from_numpy(cond)], dim=-1)
    x = x @ _deq(orc, pre, dg.CONCAT_CH).T + x
    x = x @ _deq(orc, inw, dg.CONCAT_CH).T
    ref = torch.cat([torch.from_numpy(temb), x], dim=1).numpy()
    # the timestep row is copied exactly
    assert np.array_equal(y[:, 0], temb[:, 0])
    rel_rms = float(np.sqrt(((y.astype(np.float64) - ref) ** 2).mean() / (ref.astype(np.float64) ** 2).mean()))
    assert cosine(y, ref) >= 0.9999 and rel_rms <= 5e-3, (cosine(y, ref), rel_rms)


@pytest.mark.parametrize("S,B", [(690, 2), (37, 1)])
def test_rope_f16_equals_rope_then_cast(pkg, S, B):
    """mmhip_rope_neox_f16 (the DiT's K rope and its f16 cast in one launch)
    writes the bytes of mmhip_rope_neox followed by the CPY of the permuted
    view to f16: [D, Nh, S, B] rows in, [D, S, Nh, B] f16 rows out."""
    mm = importlib.import_module(pkg.__name__ + ".mmhip")
    L = mm.load()
    _, dg = _mods(pkg)
    D, H = dg.DIM // dg.N_HEADS, dg.N_HEADS
    g = torch.Generator().manual_seed(S + B)
    x = torch.randn((B, S, H, D), generator=g).cuda()          # ggml [D, H, S, B]
    pos = torch.arange(S, dtype=torch.int32, device="cuda")
    theta = ctypes.c_float(dg.ROPE_BASE ** (-2.0 / dg.ROTARY_DIM))
    V = lambda t: ctypes.byref(mm.view_of(t))
    P = lambda t: ctypes.c_void_p(t.data_ptr())
    r = torch.empty_like(x)
    assert L.mmhip_rope_neox(V(x), P(pos), dg.ROTARY_DIM, theta, P(r), None) == 0
    ref = r.permute(0, 2, 1, 3).contiguous().half()           # ggml [D, S, H, B] f16 (CPY rounds to nearest)
    out = torch.full((B, H, S, D), float("nan"), dtype=torch.float16, device="cuda")
    dv = out.permute(0, 2, 1, 3)                               # the cast's rows in the rope's dim order
    assert L.mmhip_rope_neox_f16(V(x), P(pos), dg.ROTARY_DIM, theta, V(dv), None) == 0
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), ref.view(torch.int16))


def test_dit_block_rope_cast_fusion_gives_the_same_bits(pkg, monkeypatch):
    """The DiT block with K's rope storing f16 into the cast's rows equals the
    same graph with that fusion off, bit for bit."""
    og, dg = _mods(pkg)
    S, B = 690, 2
    w = dg.synth_block(61)
    x = np.random.default_rng(62).standard_normal((B, S, dg.DIM)).astype(np.float32)

    def run():
        g = og.OpGraph()
        try:
            blk = dg.Block(g)
            tx = g.tensor(og.F32, [dg.DIM, S, B])
            tp = g.tensor(26, [S])
            out = dg.build_block(g, blk, tx, tp, S, B)
            g.build([out])
            blk.upload(g, w)
            g.set(tx, x)
            g.set(tp, np.arange(S, dtype=np.int32))
            g.compute()
            return g.get(out)
        finally:
            g.close()

    fused = run()
    monkeypatch.setenv("GGML_MI355X_DISABLE_ROPE_F16", "1")
    plain = run()
    assert np.array_equal(fused, plain)


@pytest.mark.parametrize("D,H,S,B,n_dims", [(64, 32, 690, 2, 32), (128, 8, 37, 1, 128), (96, 4, 20, 2, 32)])
def test_rope_in_place(pkg, D, H, S, B, n_dims):
    """ggml runs ROPE in place when its allocator lets it (dst == x): the
    position-parallel kernel at the DiT's shape (a row's D / 4 chunks divide
    a wave), the LM's head dim, and a head dim whose rows straddle waves (the
    pair-per-thread kernel then runs) all give the out-of-place bytes."""
    mm = importlib.import_module(pkg.__name__ + ".mmhip")
    L = mm.load()
    g = torch.Generator().manual_seed(D + S)
    x = torch.randn((B, S, H, D), generator=g).cuda()          # ggml [D, H, S, B]
    pos = torch.arange(S, dtype=torch.int32, device="cuda") * 3
    theta = ctypes.c_float(1e4 ** (-2.0 / n_dims))
    V = lambda t: ctypes.byref(mm.view_of(t))
    P = lambda t: ctypes.c_void_p(t.data_ptr())
    ref = torch.empty_like(x)
    assert L.mmhip_rope_neox(V(x), P(pos), n_dims, theta, P(ref), None) == 0
    y = x.clone()
    assert L.mmhip_rope_neox(V(y), P(pos), n_dims, theta, P(y), None) == 0
    torch.cuda.synchronize()
    assert torch.equal(y.view(torch.int32), ref.view(torch.int32))
    # a destination overlapping x without being x is refused
    assert L.mmhip_rope_neox(V(y), P(pos), n_dims, theta, ctypes.c_void_p(y.data_ptr() + 16), None) != 0


def test_rope_cast_into_the_rope_input_is_not_fused(pkg):
    """K's rope + f16 cast (plan step ROPE_H) is not fused when the cast's
    destination overlaps the rope's input, which an allocator may do since
    the input is dead after the rope in the unfused order: the fused launch
    would read x while writing over it.  The graph then runs ROPE and CPY
    apart and writes the rope-then-cast bytes."""
    og, dg = _mods(pkg)
    mm = importlib.import_module(pkg.__name__ + ".mmhip")
    L = mm.load()
    D, H, S, B = dg.DIM // dg.N_HEADS, dg.N_HEADS, 690, 2
    G = og._load()[0]
    G.ggml_cpy.restype, G.ggml_cpy.argtypes = og._T, [ctypes.c_void_p, og._T, og._T]
    xs = torch.randn((B, S, H, D), generator=torch.Generator().manual_seed(77))
    g = og.OpGraph()
    try:
        tx = g.tensor(og.F32, [D, H, S, B])
        tp = g.tensor(26, [S])
        r = g.rope_neox(tx, tp, dg.ROTARY_DIM, dg.ROPE_BASE)
        p = g.permute(r, 0, 2, 1, 3)
        dst = g.tensor(og.F16, [D, S, H, B])
        c = G.ggml_cpy(g.ctx, p, dst)
        g.build([c])
        # the cast writes into the first half of x's memory
        dst.contents.data = tx.contents.data
        c.contents.data = tx.contents.data
        g.set(tx, xs.numpy())
        g.set(tp, np.arange(S, dtype=np.int32))
        g.compute()
        got = g.get(c, np.float16)
    finally:
        g.close()
    xr = xs.cuda()
    rr = torch.empty_like(xr)
    theta = ctypes.c_float(dg.ROPE_BASE ** (-2.0 / dg.ROTARY_DIM))
    pos = torch.arange(S, dtype=torch.int32, device="cuda")
    assert L.mmhip_rope_neox(ctypes.byref(mm.view_of(xr)), ctypes.c_void_p(pos.data_ptr()), dg.ROTARY_DIM, theta,
                             ctypes.c_void_p(rr.data_ptr()), None) == 0
    ref = rr.permute(0, 2, 1, 3).contiguous().half().cpu().numpy().ravel()  # ggml [D, S, H, B]
    assert np.array_equal(got.view(np.int16), ref.view(np.int16))
