"""GPU: the RVQ depth decoder's transformer layer (src/depth-decoder.h:196-236)
built with the restated ggml API and run through ggml_backend_graph_compute
on the MI355X backend, against a CPU float32 restatement with dequantized
weights (torch on the CPU); plus the three ops it adds to the backend
(f32 x f32 MUL_MAT, DIAG_MASK_INF, SOFT_MAX) through the C-ABI.

Tolerances (stated): layer output cosine >= 0.9999 and relative RMS error
<= 5e-3 (the Q8_0 GEMV / GEMM quantize or round the activations as ggml
does; the reference does not); f32 MUL_MAT max-rel 1e-6 against float64
(double accumulation of f32 products); SOFT_MAX max-abs 1e-6 against
float64; DIAG_MASK_INF bit-exact."""
import ctypes
import importlib

import numpy as np
import pytest
import torch

from conftest import cosine

pytestmark = pytest.mark.gpu


def st():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def ptr(t):
    return ctypes.c_void_p(t.data_ptr())


def _deq(orc, rows, k):
    return torch.from_numpy(orc.dequantize(8, rows, k, rows.shape[0]).reshape(rows.shape[0], k))


def ref_layer(orc, dg, w, x):
    """x [B, S, dim] f32 on the CPU; causal attention over S, no RoPE."""
    B, S, dim = x.shape
    Nh, D = dg.N_HEADS, dg.HEAD_DIM
    W = {n: _deq(orc, w[n], dim if n != "w_down" else dg.FF_INNER)
         for n in ("wq", "wk", "wv", "wo", "w_gate", "w_up", "w_down")}

    def rms(a, g_):
        return a / torch.sqrt((a * a).mean(-1, keepdim=True) + dg.RMS_EPS) * torch.from_numpy(g_)

    h = rms(x, w["attn_norm"])
    q, k, v = ((h @ W[n].T).reshape(B, S, Nh, D).permute(0, 2, 1, 3) for n in ("wq", "wk", "wv"))
    s = (q @ k.transpose(-1, -2).contiguous()) / np.sqrt(D)
    s = s.masked_fill(torch.triu(torch.ones(S, S, dtype=torch.bool), 1), float("-inf"))
    a = (torch.softmax(s, -1) @ v).permute(0, 2, 1, 3).reshape(B, S, Nh * D)
    x = x + a @ W["wo"].T
    h = rms(x, w["ffn_norm"])
    return x + (torch.nn.functional.silu(h @ W["w_gate"].T) * (h @ W["w_up"].T)) @ W["w_down"].T


@pytest.mark.parametrize("S,B", [(2, 1), (8, 1), (5, 2), (8, 2)])
def test_depth_layer_through_backend(pkg, orc, S, B):
    """S steps (2..8) x B streams (1, or the CFG pair): M = S * B tokens from
    2 (GEMVs with the norm / SwiGLU prologues) to 16 (GEMM)."""
    og = importlib.import_module(pkg.__name__ + ".opgraph")
    dg = importlib.import_module(pkg.__name__ + ".depthgraph")
    torch.set_num_threads(16)
    w = dg.synth_layer(61 + S)
    x = np.random.default_rng(70 + S * B).standard_normal((B, S, dg.DIM)).astype(np.float32)
    g = og.OpGraph()
    try:
        lw = dg.Layer(g)
        tx = g.tensor(og.F32, [dg.DIM, S, B])
        out = dg.build_layer(g, lw, tx, S, B)
        g.build([out])
        lw.upload(g, w)
        g.set(tx, x)
        g.compute()
        y0 = g.get(out).reshape(B, S, dg.DIM)
        for _ in range(2):
            g.compute()
            assert np.array_equal(g.get(out).reshape(B, S, dg.DIM), y0)
    finally:
        g.close()
    ref = ref_layer(orc, dg, w, torch.from_numpy(x)).numpy()
    assert np.isfinite(y0).all()
    rel_rms = float(np.sqrt(((y0.astype(np.float64) - ref) ** 2).mean() / (ref.astype(np.float64) ** 2).mean()))
    assert cosine(y0, ref) >= 0.9999 and rel_rms <= 5e-3, (cosine(y0, ref), rel_rms)


def test_mul_mat_f32_broadcast_and_views(mm):
    """dst[i, j, i2, i3] = sum_k a[k, i, i2/r2, i3/r3] b[k, j, i2, i3] with a
    permuted (non-contiguous) b and a broadcast over dim 2."""
    L = mm.load()
    g = torch.Generator().manual_seed(62)
    a = torch.randn((2, 4, 7, 256), generator=g)            # ggml [256, 7, 4, 2]
    bq = torch.randn((2, 5, 8, 256), generator=g)           # [B, S, H, D]
    b = bq.permute(0, 2, 1, 3)                              # ggml [256, 5, 8, 2], strided
    ta, tb = a.cuda(), b.cuda()
    out = torch.empty((2, 8, 5, 7), device="cuda")          # ggml [7, 5, 8, 2]
    assert L.mmhip_mul_mat_f32(ctypes.byref(mm.view_of(ta)), ctypes.byref(mm.view_of(tb)), ptr(out), st()) == 0
    a64 = a.double().repeat_interleave(2, dim=1)            # head h uses a's head h // 2
    ref = torch.einsum("bhik,bhjk->bhji", a64, b.double())
    assert float((out.cpu().double() - ref).abs().max() / ref.abs().max()) < 1e-6


def test_diag_mask_inf_and_soft_max(mm):
    L = mm.load()
    g = torch.Generator().manual_seed(63)
    x = torch.randn((3, 16, 8, 8), generator=g) * 4         # ggml [8 keys, 8 queries, 16, 3]
    tx = x.cuda()
    m = torch.empty_like(tx)
    assert L.mmhip_diag_mask_inf(ctypes.byref(mm.view_of(tx)), 0, ptr(m), st()) == 0
    tri = torch.triu(torch.ones(8, 8, dtype=torch.bool), 1)
    assert torch.equal(m.cpu(), x.masked_fill(tri, float("-inf")))
    m2 = torch.empty_like(tx)
    assert L.mmhip_diag_mask_inf(ctypes.byref(mm.view_of(tx)), 3, ptr(m2), st()) == 0
    assert torch.equal(m2.cpu(), x.masked_fill(torch.triu(torch.ones(8, 8, dtype=torch.bool), 4), float("-inf")))
    p = torch.empty_like(tx)
    assert L.mmhip_soft_max(ctypes.byref(mm.view_of(m)), ptr(p), st()) == 0
    ref = torch.softmax(m.cpu().double(), -1)
    assert float((p.cpu().double() - ref).abs().max()) < 1e-6
    # a long row (the sampler's 1024-entry vocabulary) and a strided view
    v = torch.randn((2, 1024), generator=g).cuda() * 8
    pv = torch.empty((2, 1000), device="cuda")
    assert L.mmhip_soft_max(ctypes.byref(mm.view_of(v[:, 24:])), ptr(pv), st()) == 0
    assert float((pv.cpu().double() - torch.softmax(v[:, 24:].cpu().double(), -1)).abs().max()) < 1e-6


def _small_attn_chain(mm, q, k, v, scale, bias, n_past):
    """The seven separate ops of src/depth-decoder.h:214-221 through the C-ABI:
    MUL_MAT(k, q), SCALE, DIAG_MASK_INF, SOFT_MAX, CONT(TRANSPOSE(v)),
    MUL_MAT(vt, P), CONT(PERMUTE(.., 0, 2, 1, 3)).  q, k, v: torch [B, H, S, D]
    views (ggml [D, S, H, B])."""
    L = mm.load()
    V = lambda t: ctypes.byref(mm.view_of(t))
    B, H, Sq, D = q.shape
    Sk = k.shape[2]
    sc = torch.empty((B, H, Sq, Sk), device="cuda")         # ggml [Sk, Sq, H, B]
    assert L.mmhip_mul_mat_f32(V(k), V(q), ptr(sc), st()) == 0
    s2 = torch.empty_like(sc)
    assert L.mmhip_scale(V(sc), ctypes.c_float(scale), ctypes.c_float(bias), ptr(s2), st()) == 0
    dm = torch.empty_like(sc)
    assert L.mmhip_diag_mask_inf(V(s2), n_past, ptr(dm), st()) == 0
    p = torch.empty_like(sc)
    assert L.mmhip_soft_max(V(dm), ptr(p), st()) == 0
    vt = v.transpose(2, 3).contiguous()                     # ggml [Sk, D, Hv, Bv] (a copy: the CONT)
    o = torch.empty((B, H, Sq, D), device="cuda")           # ggml [D, Sq, H, B]
    assert L.mmhip_mul_mat_f32(V(vt), V(p), ptr(o), st()) == 0
    return o.permute(0, 2, 1, 3).contiguous()               # ggml [D, H, Sq, B]


@pytest.mark.parametrize("B,H,Hkv,S,D,scale,bias,n_past",
                         [(2, 16, 16, 8, 256, 0.0625, 0.0, 0), (1, 16, 16, 2, 256, 0.0625, 0.0, 0),
                          (2, 16, 16, 16, 256, 0.0625, 0.0, 0), (2, 4, 2, 5, 64, 0.125, 0.5, 0),
                          (1, 3, 3, 13, 96, 0.1, 0.0, 2), (2, 2, 1, 16, 128, 0.08, 0.0, 0)])
def test_small_attn_equals_the_op_chain(mm, B, H, Hkv, S, D, scale, bias, n_past):
    """mmhip_small_attn (the depth decoder's manual causal attention in one
    launch) gives the bits of the seven separate ops: q / k / v as permuted
    views of projection rows, k / v heads broadcast (Hkv < H), a SCALE bias,
    n_past > 0, two to 16 keys, head dims up to 256."""
    L = mm.load()
    g = torch.Generator().manual_seed(900 + S * H + D)
    # projection rows [B, S, H, D] permuted to [B, H, S, D]: strided views
    q = (torch.randn((B, S, H, D), generator=g)).cuda().permute(0, 2, 1, 3)
    k = (torch.randn((B, S, Hkv, D), generator=g)).cuda().permute(0, 2, 1, 3)
    v = (torch.randn((B, S, Hkv, D), generator=g)).cuda().permute(0, 2, 1, 3)
    ref = _small_attn_chain(mm, q, k, v, scale, bias, n_past)
    out = torch.empty((B, S, H, D), device="cuda")
    V = lambda t: ctypes.byref(mm.view_of(t))
    assert L.mmhip_small_attn(V(q), V(k), V(v), ctypes.c_float(scale), ctypes.c_float(bias), n_past, ptr(out),
                              st()) == 0
    assert torch.equal(out, ref)
    if D % 32 == 0:
        # the quantising form: the same f32 rows, and their Q8_0 activation
        # blocks byte-equal to mmhip_quantize_act over those rows
        K, M = H * D, S * B
        xq = torch.full((L.mmhip_act_bytes(8, K, M),), 0x5A, dtype=torch.uint8, device="cuda")
        ref_q = torch.full_like(xq, 0x5A)
        out2 = torch.full_like(out, float("nan"))
        assert L.mmhip_small_attn_q(V(q), V(k), V(v), ctypes.c_float(scale), ctypes.c_float(bias), n_past,
                                    ptr(out2), 8, ptr(xq), st()) == 0
        assert L.mmhip_quantize_act(8, ptr(out), K, K, M, ptr(ref_q), st()) == 0
        torch.cuda.synchronize()
        assert torch.equal(out2, ref)
        assert torch.equal(xq, ref_q)
    # and against float64 (causal softmax attention)
    q64, k64, v64 = (t.cpu().double().repeat_interleave(H // t.shape[1], dim=1) for t in (q, k, v))
    s64 = (q64 @ k64.transpose(-1, -2)) * np.float32(scale) + bias
    s64 = s64.masked_fill(torch.triu(torch.ones(S, S, dtype=torch.bool), 1 + n_past), float("-inf"))
    o64 = (torch.softmax(s64, -1) @ v64).permute(0, 2, 1, 3)
    assert float((out.cpu().double() - o64).abs().max()) < 1e-5


def test_small_attn_rejects_long_rows(mm):
    L = mm.load()
    q = torch.zeros((1, 1, 17, 64), device="cuda")
    out = torch.empty((1, 17, 1, 64), device="cuda")
    V = lambda t: ctypes.byref(mm.view_of(t))
    assert L.mmhip_small_attn(V(q), V(q), V(q), ctypes.c_float(1.0), ctypes.c_float(0.0), 0, ptr(out), st()) == \
        mm.ERR_UNSUPPORTED
    # quantisation only for Q8_0 weights and head dims of whole blocks
    q = torch.zeros((1, 1, 4, 48), device="cuda")
    out = torch.empty((1, 4, 1, 48), device="cuda")
    xq = torch.empty(4096, dtype=torch.uint8, device="cuda")
    assert L.mmhip_small_attn_q(V(q), V(q), V(q), ctypes.c_float(1.0), ctypes.c_float(0.0), 0, ptr(out), 8, ptr(xq),
                                st()) == mm.ERR_UNSUPPORTED
    q = torch.zeros((1, 1, 4, 64), device="cuda")
    out = torch.empty((1, 4, 1, 64), device="cuda")
    assert L.mmhip_small_attn_q(V(q), V(q), V(q), ctypes.c_float(1.0), ctypes.c_float(0.0), 0, ptr(out), 12,
                                ptr(xq), st()) == mm.ERR_UNSUPPORTED


@pytest.mark.parametrize("S,B", [(8, 2), (3, 1)])
def test_depth_layer_fusions_give_the_same_bits(pkg, S, B, monkeypatch):
    """The depth layer through the backend with the manual attention as one
    launch (and the output / down projections' residual ADDs in the GEMV
    store over the [DIM, S, B] rows) equals the same graph with those two
    fusions off, bit for bit."""
    og = importlib.import_module(pkg.__name__ + ".opgraph")
    dg = importlib.import_module(pkg.__name__ + ".depthgraph")
    w = dg.synth_layer(81 + S)
    x = np.random.default_rng(90 + S * B).standard_normal((B, S, dg.DIM)).astype(np.float32)

    def run():
        g = og.OpGraph()
        try:
            lw = dg.Layer(g)
            tx = g.tensor(og.F32, [dg.DIM, S, B])
            out = dg.build_layer(g, lw, tx, S, B)
            g.build([out])
            lw.upload(g, w)
            g.set(tx, x)
            g.compute()
            return g.get(out)
        finally:
            g.close()

    fused = run()
    monkeypatch.setenv("GGML_MI355X_DISABLE_SMALL_ATTN", "1")
    monkeypatch.setenv("GGML_MI355X_DISABLE_FUSION", "1")
    plain = run()
    assert np.array_equal(fused, plain)
