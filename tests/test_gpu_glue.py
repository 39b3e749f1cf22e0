"""GPU: decode-step glue kernels against the oracle / closed forms.

Tolerances (stated): binary ops, copies, set_rows, get_rows bit-exact;
rms_norm and swiglu max-rel 1e-5 (f32 reduction order, libm expf vs device
expf); rope max-abs 2e-5 at positions up to 5000 (libm vs device cosf/sinf of
the same f32 angle)."""
import ctypes

import numpy as np
import pytest
import torch

from conftest import rel_err

pytestmark = pytest.mark.gpu


def st():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def ptr(t):
    return ctypes.c_void_p(t.data_ptr())


def test_binary_broadcast(mm):
    L = mm.load()
    rng = np.random.default_rng(1)
    a = rng.standard_normal((2, 3, 5, 64)).astype(np.float32)
    b = rng.standard_normal((1, 3, 1, 64)).astype(np.float32)
    ta, tb = torch.from_numpy(a).cuda(), torch.from_numpy(b).cuda()
    for op, ref in ((0, a + b), (1, a - b), (2, a * b)):
        out = torch.empty_like(ta)
        assert L.mmhip_binary(op, ctypes.byref(mm.view_of(ta)), ctypes.byref(mm.view_of(tb)), ptr(out), st()) == 0
        assert np.array_equal(out.cpu().numpy(), ref)


@pytest.mark.parametrize("with_w", [False, True])
def test_rms_norm(mm, orc, with_w):
    L = mm.load()
    rng = np.random.default_rng(2)
    x = (rng.standard_normal((2, 32, 128)) * 3).astype(np.float32)
    w = (1 + 0.02 * rng.standard_normal(128)).astype(np.float32)
    tx, tw = torch.from_numpy(x).cuda(), torch.from_numpy(w).cuda()
    out = torch.empty_like(tx)
    wv = ctypes.byref(mm.view_of(tw)) if with_w else None
    assert L.mmhip_rms_norm(ctypes.byref(mm.view_of(tx)), wv, 1e-6, ptr(out), st()) == 0
    ref = orc.rms_norm_mul(x, w if with_w else None, 1e-6)
    assert rel_err(out.cpu().numpy(), ref) < 1e-5


def test_rope_neox(mm, orc):
    L = mm.load()
    rng = np.random.default_rng(3)
    T, H, D = 4, 8, 128
    x = rng.standard_normal((T, H, D)).astype(np.float32)
    pos = np.array([0, 1, 4095, 5000], np.int32)
    tx, tp = torch.from_numpy(x).cuda(), torch.from_numpy(pos).cuda()
    out = torch.empty_like(tx)
    # the backend computes powf(base, -2/n_dims) on the host, as ggml-CPU does
    theta_scale = float(np.power(np.float32(1e6), np.float32(-2.0) / np.float32(D)))
    assert L.mmhip_rope_neox(ctypes.byref(mm.view_of(tx)), ptr(tp), D, ctypes.c_float(theta_scale), ptr(out), st()) == 0
    ref = orc.rope_neox(x, pos, D, 1e6)
    assert np.abs(out.cpu().numpy() - ref).max() < 2e-5
    # partial rotation (DiT: 32 of 64 dims) leaves the tail unchanged
    x2 = rng.standard_normal((3, 4, 64)).astype(np.float32)
    t2 = torch.from_numpy(x2).cuda()
    o2 = torch.empty_like(t2)
    p2 = torch.tensor([5, 6, 7], dtype=torch.int32, device="cuda")
    ts2 = float(np.power(np.float32(1e4), np.float32(-2.0) / np.float32(32)))
    assert L.mmhip_rope_neox(ctypes.byref(mm.view_of(t2)), ptr(p2), 32, ctypes.c_float(ts2), ptr(o2), st()) == 0
    r2 = orc.rope_neox(x2, np.array([5, 6, 7], np.int32), 32, 1e4)
    assert np.abs(o2.cpu().numpy() - r2).max() < 2e-5
    assert np.array_equal(o2.cpu().numpy()[..., 32:], x2[..., 32:])


@pytest.mark.parametrize("split", [False, True])
def test_swiglu(mm, orc, split):
    L = mm.load()
    rng = np.random.default_rng(4)
    a = (rng.standard_normal((2, 1024)) * 4).astype(np.float32)
    ta = torch.from_numpy(a).cuda()
    if split:
        out = torch.empty((2, 512), device="cuda")
        g, u = ta[:, :512].contiguous(), ta[:, 512:].contiguous()
        assert L.mmhip_swiglu(ctypes.byref(mm.view_of(g)), ctypes.byref(mm.view_of(u)), 0, ptr(out), st()) == 0
    else:
        out = torch.empty((2, 512), device="cuda")
        assert L.mmhip_swiglu(ctypes.byref(mm.view_of(ta)), None, 0, ptr(out), st()) == 0
    assert rel_err(out.cpu().numpy(), orc.swiglu(a)) < 1e-5


def test_set_rows_into_f16_cache(mm):
    """KV write of src/qwen3-lm.h:803-804: rows [D, 1, Nkv, N] into the
    [D, max_seq, Nkv, N] f16 cache at per-set positions (int64)."""
    L = mm.load()
    D, S, Nkv, N = 128, 64, 8, 2
    cache = torch.zeros((N, Nkv, S, D), dtype=torch.float16, device="cuda")
    src = torch.randn((N, Nkv, 1, D), device="cuda")
    ids = torch.tensor([[[5]], [[17]]], dtype=torch.int64, device="cuda").view(N, 1, 1)
    sv = mm.view_of(src)
    iv = mm.view_of(ids, ne=[1, 1, N, 1], nb=[8, 8, 8, 8 * N])
    dv = mm.view_of(cache)
    assert L.mmhip_set_rows(ctypes.byref(sv), ctypes.byref(iv), 27, ctypes.byref(dv), 1, st()) == 0
    c = cache.cpu()
    assert torch.equal(c[0, :, 5], src[0, :, 0].half().cpu()) and torch.equal(c[1, :, 17], src[1, :, 0].half().cpu())
    c[0, :, 5] = 0
    c[1, :, 17] = 0
    assert not c.any()


@pytest.mark.parametrize("t", [8, 12, 13, 14])
def test_get_rows_quantized(mm, orc, pkg, t):
    L = mm.load()
    V, K = 50, 512
    raw = pkg.synth.gguf_blocks_np(t, V, K, 30 + t)
    W = mm.QuantWeight.from_gguf(t, raw, V, K)
    ids = torch.tensor([3, 49, 0, 3], dtype=torch.int32, device="cuda")
    out = torch.empty((4, K), device="cuda")
    rs = W.row_bytes
    wv = mm.view_of(W.data, ne=[K, V, 1, 1], nb=[1, rs, rs * V, rs * V])
    assert L.mmhip_get_rows(t, ctypes.byref(wv), ctypes.byref(mm.view_of(ids)), ptr(out), st()) == 0
    ref = orc.dequantize(t, raw, K, V)[[3, 49, 0, 3]]
    assert np.array_equal(out.cpu().numpy().view(np.uint32), ref.view(np.uint32))


def test_cpy_strided_to_f16(mm):
    L = mm.load()
    a = torch.randn((3, 40, 64), device="cuda")
    src = a.permute(1, 0, 2)  # strided view
    dst = torch.empty((40, 3, 64), dtype=torch.float16, device="cuda")
    assert L.mmhip_cpy(ctypes.byref(mm.view_of(src)), 0, ctypes.byref(mm.view_of(dst)), 1, st()) == 0
    assert torch.equal(dst, src.half())


def _act(mm, L, wt, x):
    """Separate-pass activation quantisation of x [M, K] (reference for the fused forms)."""
    M, K = x.shape
    n = L.mmhip_act_bytes(wt, K, M)
    buf = torch.zeros(n, dtype=torch.uint8, device="cuda")
    assert L.mmhip_quantize_act(wt, ptr(x), K, K, M, ptr(buf), st()) == 0
    return buf


@pytest.mark.parametrize("shape", [(3, 4096), (2, 2, 1024), (1, 256)])
def test_rms_norm_rows(mm, orc, shape):
    """Row kernel (n % 256 == 0), also on rows read through a strided view."""
    L = mm.load()
    rng = np.random.default_rng(20)
    n = shape[-1]
    big = (rng.standard_normal(shape[:-1] + (n + 64,)) * 2).astype(np.float32)
    w = (1 + 0.02 * rng.standard_normal(n)).astype(np.float32)
    tb, tw = torch.from_numpy(big).cuda(), torch.from_numpy(w).cuda()
    tx = tb[..., 32:32 + n]  # row stride n + 64, 16-byte aligned start
    out = torch.empty(shape, dtype=torch.float32, device="cuda")
    assert L.mmhip_rms_norm(ctypes.byref(mm.view_of(tx)), ctypes.byref(mm.view_of(tw)), 1e-6, ptr(out), st()) == 0
    ref = orc.rms_norm_mul(np.ascontiguousarray(big[..., 32:32 + n]), w, 1e-6)
    assert rel_err(out.cpu().numpy(), ref) < 1e-5


@pytest.mark.parametrize("wt", [8, 12, 13, 14])
def test_rms_norm_quant_equals_two_pass(mm, wt):
    """Fused norm + quantisation is byte-identical to norm then quantize_act."""
    L = mm.load()
    rng = np.random.default_rng(21)
    M, K = 2, 4096
    x = torch.from_numpy((rng.standard_normal((M, K)) * 3).astype(np.float32)).cuda()
    w = torch.from_numpy((1 + 0.02 * rng.standard_normal(K)).astype(np.float32)).cuda()
    y1 = torch.empty_like(x)
    assert L.mmhip_rms_norm(ctypes.byref(mm.view_of(x)), ctypes.byref(mm.view_of(w)), 1e-6, ptr(y1), st()) == 0
    ref_q = _act(mm, L, wt, y1)
    y2 = torch.empty_like(x)
    q2 = torch.zeros_like(ref_q)
    assert L.mmhip_rms_norm_quant(ctypes.byref(mm.view_of(x)), ctypes.byref(mm.view_of(w)), 1e-6, ptr(y2), wt,
                                  ptr(q2), st()) == 0
    q3 = torch.zeros_like(ref_q)
    assert L.mmhip_rms_norm_quant(ctypes.byref(mm.view_of(x)), ctypes.byref(mm.view_of(w)), 1e-6, None, wt,
                                  ptr(q3), st()) == 0
    torch.cuda.synchronize()
    assert torch.equal(y1, y2)
    assert torch.equal(q2, ref_q) and torch.equal(q3, ref_q)


@pytest.mark.parametrize("wt", [8, 14])
def test_swiglu_quant_equals_two_pass(mm, wt):
    L = mm.load()
    rng = np.random.default_rng(22)
    M, F = 2, 1024
    a = torch.from_numpy((rng.standard_normal((M, 2 * F)) * 2).astype(np.float32)).cuda()
    y1 = torch.empty((M, F), dtype=torch.float32, device="cuda")
    assert L.mmhip_swiglu(ctypes.byref(mm.view_of(a)), None, 0, ptr(y1), st()) == 0
    ref_q = _act(mm, L, wt, y1)
    y2 = torch.empty_like(y1)
    q2 = torch.zeros_like(ref_q)
    assert L.mmhip_swiglu_quant(ctypes.byref(mm.view_of(a)), None, 0, ptr(y2), wt, ptr(q2), st()) == 0
    torch.cuda.synchronize()
    assert torch.equal(y1, y2) and torch.equal(q2, ref_q)


def _head_args(mm, src, D, H, T, nb_t, norm_w=None, eps=1e-6, pos=None, theta=1e6, dst=None, ids=None,
               cache=None):
    a = mm.HeadRowsArgs()
    a.src = src.data_ptr()
    a.src_nb_h, a.src_nb_t = D * 4, nb_t
    a.D, a.H, a.T = D, H, T
    a.norm = 1 if norm_w is not None else 0
    a.norm_w = norm_w.data_ptr() if norm_w is not None else None
    a.eps = eps
    a.pos = pos.data_ptr() if pos is not None else None
    a.theta_scale = float(np.power(np.float32(theta), np.float32(-2.0) / np.float32(D)))
    if ids is None:
        a.dst, a.dst_type = dst.data_ptr(), 0
    else:
        # cache [T(sets), H, S, D] f16; ids [T] i64: row ids[t] of set t
        a.dst, a.dst_type = cache.data_ptr(), 1
        a.ids, a.ids_type = ids.data_ptr(), 27
        a.ids_nb1, a.ids_nb2, a.ids_ne1, a.ids_ne2 = 8, 8, 1, T
        a.dst_nb1, a.dst_nb2, a.dst_nb3 = D * 2, cache.stride(1) * 2, cache.stride(0) * 2
    return a


@pytest.mark.parametrize("D", [64, 128])
def test_head_rows_q_and_k(mm, orc, D):
    """QK-norm + NeoX RoPE of the heads of a fused QKV row (src/qwen3-lm.h:
    764-772), then Q as contiguous f32 and K stored into an f16 cache."""
    L = mm.load()
    rng = np.random.default_rng(23)
    T, Hq, Hk, S = 2, 8, 2, 64
    C = (Hq + 2 * Hk) * D
    qkv = (rng.standard_normal((T, C)) * 2).astype(np.float32)
    wq = (1 + 0.02 * rng.standard_normal(D)).astype(np.float32)
    wk = (1 + 0.02 * rng.standard_normal(D)).astype(np.float32)
    pos = np.array([17, 4095], np.int32)
    tqkv, twq, twk, tpos = (torch.from_numpy(v).cuda() for v in (qkv, wq, wk, pos))
    qout = torch.empty((T, Hq, D), dtype=torch.float32, device="cuda")
    a = _head_args(mm, tqkv, D, Hq, T, C * 4, norm_w=twq, pos=tpos, dst=qout)
    assert L.mmhip_head_rows(ctypes.byref(a), st()) == 0
    cache = torch.zeros((T, Hk, S, D), dtype=torch.float16, device="cuda")
    ids = torch.tensor([5, 40], dtype=torch.int64, device="cuda")
    kview = tqkv[:, Hq * D:]
    a = _head_args(mm, kview, D, Hk, T, C * 4, norm_w=twk, pos=tpos, ids=ids, cache=cache)
    assert L.mmhip_head_rows(ctypes.byref(a), st()) == 0
    torch.cuda.synchronize()
    qr = orc.rope_neox(orc.rms_norm_mul(qkv[:, :Hq * D].reshape(T * Hq, D), wq, 1e-6).reshape(T, Hq, D), pos, D, 1e6)
    assert np.abs(qout.cpu().numpy() - qr).max() < 5e-5
    kr = orc.rope_neox(orc.rms_norm_mul(qkv[:, Hq * D:(Hq + Hk) * D].reshape(T * Hk, D), wk, 1e-6).reshape(T, Hk, D),
                       pos, D, 1e6)
    c = cache.cpu().numpy().astype(np.float32)
    for t, r in enumerate((5, 40)):
        got = c[t, :, r, :]
        assert np.abs(got - kr[t]).max() <= 2e-3 * np.abs(kr[t]).max()
        # every other row untouched
        assert not np.any(np.delete(c[t], r, axis=1))


def test_head_rows_v_store(mm):
    """V rows: no norm, no rope, f32 -> f16 into the cache rows (bit-exact)."""
    L = mm.load()
    rng = np.random.default_rng(24)
    T, Hk, D, S = 2, 8, 128, 16
    C = 48 * D
    qkv = torch.from_numpy(rng.standard_normal((T, C)).astype(np.float32)).cuda()
    vview = qkv[:, 40 * D:]
    cache = torch.zeros((T, Hk, S, D), dtype=torch.float16, device="cuda")
    ids = torch.tensor([3, 9], dtype=torch.int64, device="cuda")
    a = _head_args(mm, vview, D, Hk, T, C * 4, ids=ids, cache=cache)
    assert L.mmhip_head_rows(ctypes.byref(a), st()) == 0
    torch.cuda.synchronize()
    want = vview.reshape(T, Hk, D).half()
    assert torch.equal(cache[0, :, 3], want[0]) and torch.equal(cache[1, :, 9], want[1])


@pytest.mark.parametrize("wt", [8, 12, 13, 14])
def test_mul_mat_q_add(mm, pkg, wt):
    """GEMV with the residual ADD in its store equals GEMV then a separate f32 add."""
    L = mm.load()
    synth = pkg.synth
    N, K, M = 1000, 4096, 2
    Wq = mm.QuantWeight.from_gguf(wt, synth.gguf_blocks_np(wt, N, K, 3), N, K)
    rng = np.random.default_rng(25)
    x = torch.from_numpy(rng.standard_normal((M, K)).astype(np.float32)).cuda()
    r = torch.from_numpy(rng.standard_normal((M, N)).astype(np.float32)).cuda()
    xq = _act(mm, L, wt, x)
    y = torch.empty((M, N), dtype=torch.float32, device="cuda")
    assert L.mmhip_mul_mat_q(wt, ptr(Wq.data), N, K, Wq.row_bytes, ptr(xq), M, ptr(y), N, st()) == 0
    y2 = torch.empty_like(y)
    assert L.mmhip_mul_mat_q_add(wt, ptr(Wq.data), N, K, Wq.row_bytes, ptr(xq), M, ptr(r), N, ptr(y2), N, st()) == 0
    # in place: r and y the same buffer
    r3 = r.clone()
    assert L.mmhip_mul_mat_q_add(wt, ptr(Wq.data), N, K, Wq.row_bytes, ptr(xq), M, ptr(r3), N, ptr(r3), N, st()) == 0
    torch.cuda.synchronize()
    assert torch.equal(y2, y + r) and torch.equal(r3, y + r)


def test_head_rows_three_chains_one_launch(mm, orc):
    """mmhip_head_rows_n with the Q, K and V chains of one attention block gives
    exactly what three separate calls give."""
    L = mm.load()
    rng = np.random.default_rng(26)
    T, Hq, Hk, D, S = 2, 32, 8, 128, 32
    C = (Hq + 2 * Hk) * D
    qkv = torch.from_numpy((rng.standard_normal((T, C)) * 2).astype(np.float32)).cuda()
    wq = torch.from_numpy((1 + 0.02 * rng.standard_normal(D)).astype(np.float32)).cuda()
    wk = torch.from_numpy((1 + 0.02 * rng.standard_normal(D)).astype(np.float32)).cuda()
    pos = torch.tensor([7, 1234], dtype=torch.int32, device="cuda")
    ids = torch.tensor([3, 17], dtype=torch.int64, device="cuda")
    outs = []
    for merged in (False, True):
        qout = torch.zeros((T, Hq, D), dtype=torch.float32, device="cuda")
        kc = torch.zeros((T, Hk, S, D), dtype=torch.float16, device="cuda")
        vc = torch.zeros((T, Hk, S, D), dtype=torch.float16, device="cuda")
        a = [_head_args(mm, qkv, D, Hq, T, C * 4, norm_w=wq, pos=pos, dst=qout),
             _head_args(mm, qkv[:, Hq * D:], D, Hk, T, C * 4, norm_w=wk, pos=pos, ids=ids, cache=kc),
             _head_args(mm, qkv[:, (Hq + Hk) * D:], D, Hk, T, C * 4, ids=ids, cache=vc)]
        if merged:
            arr = (mm.HeadRowsArgs * 3)(*a)
            assert L.mmhip_head_rows_n(ctypes.byref(arr), 3, st()) == 0
        else:
            for x in a:
                assert L.mmhip_head_rows(ctypes.byref(x), st()) == 0
        torch.cuda.synchronize()
        outs.append((qout, kc, vc))
    for x, y in zip(outs[0], outs[1]):
        assert torch.equal(x, y)


@pytest.mark.parametrize("D,nkv,ids_", [(128, 512, (300, 45)), (128, 4096, (4095, 4095)), (64, 700, (699, 0)),
                                        (128, 256, (900, 3))])
@pytest.mark.parametrize("quant", [0, 8, 14])
def test_flash_attn_head_equals_separate(mm, D, nkv, ids_, quant):
    """Decode attention with the Q/K/V head chains in its prologue equals
    mmhip_head_rows_n then the attention: the same caches (the new rows
    written), the same output (and quantised output: Q8_0 blocks for Q8_0
    weights, Q8_K super-blocks for Q6_K weights) bit for bit.  At D = 128 the
    fused call runs k_fa_dec_dma (the split's K / V DMA'd into LDS while the
    prologue runs, the new rows substituted there), the separate one
    k_fa_dec_mfma.  Both run the inputs A, B, A in a row through one
    workspace.  Cases: new rows inside the window, at its last key, and past
    it (900 > nkv: written, not attended)."""
    L = mm.load()
    rng = np.random.default_rng(31)
    T, Hq, Hk, S = 2, 32, 8, 4608
    C = (Hq + 2 * Hk) * D
    qkvs = [torch.from_numpy((rng.standard_normal((T, C)) * 2).astype(np.float32)).cuda() for _ in range(2)]
    wq = torch.from_numpy((1 + 0.02 * rng.standard_normal(D)).astype(np.float32)).cuda()
    wk = torch.from_numpy((1 + 0.02 * rng.standard_normal(D)).astype(np.float32)).cuda()
    pos = torch.tensor(list(ids_), dtype=torch.int32, device="cuda")
    ids = torch.tensor(list(ids_), dtype=torch.int64, device="cuda")
    kc0s = [torch.from_numpy(rng.standard_normal((T, Hk, S, D)).astype(np.float16)).cuda() for _ in range(2)]
    vc0s = [torch.from_numpy(rng.standard_normal((T, Hk, S, D)).astype(np.float16)).cuda() for _ in range(2)]
    keys = np.arange(nkv)[None, :]
    allow = keys <= np.minimum(np.array(ids_), nkv - 1)[:, None]
    mask = torch.from_numpy(np.where(allow, 0, -np.inf).astype(np.float16).reshape(T, 1, 1, nkv)).cuda()
    kvne, kvnb = [D, nkv, Hk, T], [2, 2 * D, 2 * D * S, 2 * D * S * Hk]
    K = Hq * D
    qout = torch.zeros((T, Hq, D), dtype=torch.float32, device="cuda")
    qv = mm.view_of(qout, [D, 1, Hq, T], [4, 4 * D * Hq, 4 * D, 4 * D * Hq])
    kc, vc = kc0s[0].clone(), vc0s[0].clone()
    kv, vv = mm.view_of(kc, kvne, kvnb), mm.view_of(vc, kvne, kvnb)
    mv = mm.view_of(mask)
    need = L.mmhip_flash_attn_workspace(ctypes.byref(qv), ctypes.byref(kv), ctypes.byref(vv))
    ws = torch.empty(max(need, 256), dtype=torch.uint8, device="cuda")
    res = {}
    for fused in (False, True):
        for rep, sel in enumerate((0, 1, 0)):
            qkv = qkvs[sel]
            kc.copy_(kc0s[sel])
            vc.copy_(vc0s[sel])
            qout.zero_()
            a = (mm.HeadRowsArgs * 3)(
                _head_args(mm, qkv, D, Hq, T, C * 4, norm_w=wq, pos=pos, dst=qout),
                _head_args(mm, qkv[:, Hq * D:], D, Hk, T, C * 4, norm_w=wk, pos=pos, ids=ids, cache=kc),
                _head_args(mm, qkv[:, (Hq + Hk) * D:], D, Hk, T, C * 4, ids=ids, cache=vc))
            out = torch.full((T, 1, Hq, D), float("nan"), device="cuda")
            xq = torch.zeros(L.mmhip_act_bytes(quant, K, T), dtype=torch.uint8, device="cuda") if quant else None
            args = (ctypes.byref(qv), ctypes.byref(kv), ctypes.byref(vv), ctypes.byref(mv), float(1 / np.sqrt(D)),
                    ptr(out), ptr(ws), need)
            if fused:
                assert L.mmhip_flash_attn_ext_head_supported(ctypes.byref(qv), ctypes.byref(kv),
                                                             ctypes.byref(vv)) == 1
                assert L.mmhip_flash_attn_ext_head(*args, quant, ptr(xq) if quant else None,
                                                   ctypes.byref(a), st()) == 0
            else:
                assert L.mmhip_head_rows_n(ctypes.byref(a), 3, st()) == 0
                if quant:
                    assert L.mmhip_flash_attn_ext_q(*args, quant, ptr(xq), st()) == 0
                else:
                    assert L.mmhip_flash_attn_ext(*args, st()) == 0
            torch.cuda.synchronize()
            assert not torch.equal(kc, kc0s[sel])  # the new rows were written
            res[fused, rep] = (out, kc.clone(), vc.clone(), xq)
    assert not torch.equal(res[False, 0][0], res[False, 1][0])  # A and B differ
    for rep in range(3):
        (o1, k1, v1, x1), (o2, k2, v2, x2) = res[False, rep], res[True, rep]
        assert torch.equal(k1, k2) and torch.equal(v1, v2)
        assert torch.equal(o1, o2), rep
        if quant:
            assert torch.equal(x1, x2), rep


def test_flash_attn_head_rejects_prefill_shapes(mm):
    """Too many query columns per KV head for the prologue's waves (nq = 4
    tokens x 4 heads): not taken, so the caller keeps the separate chains."""
    L = mm.load()
    D, nq, Hq, Hk, T, S = 128, 4, 32, 8, 2, 64
    q = torch.zeros((T, Hq, nq, D), device="cuda")
    kc = torch.zeros((T, Hk, S, D), dtype=torch.float16, device="cuda")
    qv, kv = mm.view_of(q), mm.view_of(kc)
    assert L.mmhip_flash_attn_ext_head_supported(ctypes.byref(qv), ctypes.byref(kv), ctypes.byref(kv)) == 0


@pytest.mark.parametrize("wt,M,K,N,ldx", [(8, 2, 4096, 6144, 4096), (8, 1, 1024, 300, 1088), (8, 2, 2048, 9000, 2048),
                                          (8, 2, 4096, 30000, 4096), (8, 1, 256, 77, 320), (8, 2, 1024, 70001, 1024),
                                          (14, 2, 4096, 6144, 4096), (14, 1, 2048, 300, 2112),
                                          (14, 2, 4096, 30000, 4096), (14, 2, 2048, 9001, 2048),
                                          (14, 2, 4096, 24576, 4096), (13, 2, 4096, 6144, 4096),
                                          (13, 1, 4096, 300, 4160), (13, 2, 4096, 30000, 4096),
                                          (13, 2, 4096, 24576, 4096), (12, 2, 4096, 9001, 4096),
                                          (12, 1, 4096, 5120, 4096)])
def test_rms_norm_mul_mat_equals_two_pass(mm, pkg, wt, M, K, N, ldx):
    """GEMV with the RMS norm + quantisation in its prologue is bit-identical
    to rms_norm_quant then mul_mat_q (and mul_mat_q_add with a residual);
    N from one to eight row iterations of the persistent grid, odd tails.
    Q8_0 weights (Q8_0 activation blocks), Q6_K weights (Q8_K super-blocks,
    the persistent Q6_K kernel) and Q5_K / Q4_K weights (Q8_K, the
    persistent Q4_K / Q5_K kernel, whose quantised-row form mul_mat_q takes
    at 1-2 columns)."""
    L = mm.load()
    Wq = mm.QuantWeight.from_gguf(wt, pkg.synth.gguf_blocks_np(wt, N, K, 5), N, K)
    rng = np.random.default_rng(26)
    xb = torch.from_numpy((rng.standard_normal((M, ldx)) * 3).astype(np.float32)).cuda()
    x = xb[:, :K]
    w = torch.from_numpy((1 + 0.05 * rng.standard_normal(K)).astype(np.float32)).cuda()
    r = torch.from_numpy(rng.standard_normal((M, N)).astype(np.float32)).cuda()
    assert L.mmhip_rms_norm_mul_mat_supported(wt, N, K, M) == 1
    xn = torch.empty((M, K), dtype=torch.float32, device="cuda")
    xq = torch.zeros(L.mmhip_act_bytes(wt, K, M), dtype=torch.uint8, device="cuda")
    assert L.mmhip_rms_norm_quant(ctypes.byref(mm.view_of(x)), ctypes.byref(mm.view_of(w)), 1e-6, ptr(xn), wt,
                                  ptr(xq), st()) == 0
    y1 = torch.empty((M, N), dtype=torch.float32, device="cuda")
    assert L.mmhip_mul_mat_q(wt, ptr(Wq.data), N, K, Wq.row_bytes, ptr(xq), M, ptr(y1), N, st()) == 0
    y2 = torch.full((M, N), float("nan"), device="cuda")
    xn2 = torch.full((M, K), float("nan"), device="cuda")
    assert L.mmhip_rms_norm_mul_mat(wt, ptr(Wq.data), N, K, Wq.row_bytes, ptr(x), ldx, M, ptr(w), 1e-6, ptr(xn2),
                                    None, 0, ptr(y2), N, st()) == 0
    y3 = torch.empty_like(y1)
    assert L.mmhip_rms_norm_mul_mat(wt, ptr(Wq.data), N, K, Wq.row_bytes, ptr(x), ldx, M, ptr(w), 1e-6, None,
                                    ptr(r), N, ptr(y3), N, st()) == 0
    torch.cuda.synchronize()
    assert torch.equal(y2, y1)
    assert torch.equal(xn2, xn)
    assert torch.equal(y3, y1 + r)


def test_rms_norm_mul_mat_rejects_unsupported(mm):
    """Shapes outside the fused kernel's limits are refused before any launch."""
    L = mm.load()
    assert L.mmhip_rms_norm_mul_mat_supported(8, 4096, 4352, 2) == 0   # K > 4096
    assert L.mmhip_rms_norm_mul_mat_supported(8, 4096, 4096, 3) == 0   # M > 2
    assert L.mmhip_rms_norm_mul_mat_supported(12, 4096, 2048, 2) == 0  # Q4_K / Q5_K: K = 4096 only
    assert L.mmhip_rms_norm_mul_mat_supported(13, 4096, 8192, 2) == 0
    assert L.mmhip_rms_norm_mul_mat_supported(14, 4096, 1024, 2) == 0  # Q6_K rows not 16-byte sized
    assert L.mmhip_rms_norm_mul_mat_supported(8, 4096, 1000, 2) == 0   # K % 256
    dummy = torch.zeros(16, dtype=torch.float32, device="cuda")
    rc = L.mmhip_rms_norm_mul_mat(8, ptr(dummy), 4096, 4352, 4624, ptr(dummy), 4352, 2, ptr(dummy), 1e-6, None,
                                  None, 0, ptr(dummy), 4096, st())
    assert rc != 0


@pytest.mark.parametrize("wt,M,F,N,mode", [(8, 2, 12288, 4096, "fused"), (8, 1, 3072, 1000, "split"),
                                           (8, 2, 2048, 9001, "swapped"), (8, 2, 12288, 5000, "fused"),
                                           (8, 1, 256, 77, "fused"), (14, 2, 4096, 4096, "fused"),
                                           (14, 1, 4096, 1000, "split"), (14, 2, 2048, 9001, "swapped"),
                                           (14, 2, 4096, 30000, "fused")])
def test_swiglu_mul_mat_equals_two_pass(mm, pkg, wt, M, F, N, mode):
    """GEMV with the SwiGLU + quantisation in its prologue is bit-identical to
    swiglu_quant then mul_mat_q / mul_mat_q_add: fused gate|up rows (also
    swapped) and split gate / up tensors; one and two row iterations of the
    persistent grid for the long (K = 12288) rows.  Q8_0 and Q6_K weights
    (Q6_K up to K = 4096)."""
    L = mm.load()
    Wq = mm.QuantWeight.from_gguf(wt, pkg.synth.gguf_blocks_np(wt, N, F, 6), N, F)
    rng = np.random.default_rng(27)
    a = torch.from_numpy((rng.standard_normal((M, 2 * F)) * 2).astype(np.float32)).cuda()
    r = torch.from_numpy(rng.standard_normal((M, N)).astype(np.float32)).cuda()
    swapped = 1 if mode == "swapped" else 0
    if mode == "split":
        g, u = a[:, :F].contiguous(), a[:, F:].contiguous()
        b_view = ctypes.byref(mm.view_of(u))
        a_view = ctypes.byref(mm.view_of(g))
        gp, ldg, up, ldu = g, F, u, F
    else:
        a_view, b_view = ctypes.byref(mm.view_of(a)), None
        first, second = a[:, :F], a[:, F:]
        gp, up = (second, first) if swapped else (first, second)
        ldg = ldu = 2 * F
    assert L.mmhip_swiglu_mul_mat_supported(wt, N, F, M) == 1
    h = torch.empty((M, F), dtype=torch.float32, device="cuda")
    xq = torch.zeros(L.mmhip_act_bytes(wt, F, M), dtype=torch.uint8, device="cuda")
    assert L.mmhip_swiglu_quant(a_view, b_view, swapped, ptr(h), wt, ptr(xq), st()) == 0
    y1 = torch.empty((M, N), dtype=torch.float32, device="cuda")
    assert L.mmhip_mul_mat_q(wt, ptr(Wq.data), N, F, Wq.row_bytes, ptr(xq), M, ptr(y1), N, st()) == 0
    y2 = torch.full((M, N), float("nan"), device="cuda")
    h2 = torch.full((M, F), float("nan"), device="cuda")
    assert L.mmhip_swiglu_mul_mat(wt, ptr(Wq.data), N, F, Wq.row_bytes, ptr(gp), ldg, ptr(up), ldu, M, ptr(h2), None,
                                  0, ptr(y2), N, st()) == 0
    y3 = torch.empty_like(y1)
    assert L.mmhip_swiglu_mul_mat(wt, ptr(Wq.data), N, F, Wq.row_bytes, ptr(gp), ldg, ptr(up), ldu, M, None, ptr(r),
                                  N, ptr(y3), N, st()) == 0
    torch.cuda.synchronize()
    assert torch.equal(h2, h)
    assert torch.equal(y2, y1)
    assert torch.equal(y3, y1 + r)


@pytest.mark.parametrize("M,K,F,swapped", [(2, 4096, 12288, 0), (1, 1024, 512, 0), (2, 2048, 256 * 65, 1),
                                           (1, 256, 256, 1), (2, 4096, 256 * 90, 0)])
def test_rms_norm_mul_mat_glu_equals_two_pass(mm, pkg, M, K, F, swapped):
    """gate_up GEMV with the RMS norm in its prologue and the SwiGLU + the
    down GEMV's Q8_0 quantisation in its epilogue: the quantised activations
    (bytes and scales) and the f32 SwiGLU rows equal rms_norm_mul_mat then
    swiglu_quant bit for bit; one to three blocks per workgroup, a last
    workgroup with one block (520 blocks over 256 CUs), gate / up halves in
    either order."""
    L = mm.load()
    N = 2 * F
    Wq = mm.QuantWeight.from_gguf(8, pkg.synth.gguf_blocks_np(8, N, K, 7), N, K)
    rng = np.random.default_rng(28)
    x = torch.from_numpy((rng.standard_normal((M, K)) * 3).astype(np.float32)).cuda()
    w = torch.from_numpy((1 + 0.05 * rng.standard_normal(K)).astype(np.float32)).cuda()
    assert L.mmhip_rms_norm_mul_mat_glu_supported(8, N, K, M) == 1
    y = torch.empty((M, N), dtype=torch.float32, device="cuda")
    assert L.mmhip_rms_norm_mul_mat(8, ptr(Wq.data), N, K, Wq.row_bytes, ptr(x), K, M, ptr(w), 1e-6, None, None, 0,
                                    ptr(y), N, st()) == 0
    h1 = torch.empty((M, F), dtype=torch.float32, device="cuda")
    xq1 = torch.zeros(L.mmhip_act_bytes(8, F, M), dtype=torch.uint8, device="cuda")
    assert L.mmhip_swiglu_quant(ctypes.byref(mm.view_of(y)), None, swapped, ptr(h1), 8, ptr(xq1), st()) == 0
    h2 = torch.full((M, F), float("nan"), device="cuda")
    xq2 = torch.full_like(xq1, 0x5A)
    assert L.mmhip_rms_norm_mul_mat_glu(8, ptr(Wq.data), N, K, Wq.row_bytes, ptr(x), K, M, ptr(w), 1e-6, swapped,
                                        ptr(xq2), ptr(h2), st()) == 0
    xq3 = torch.full_like(xq1, 0xA5)
    assert L.mmhip_rms_norm_mul_mat_glu(8, ptr(Wq.data), N, K, Wq.row_bytes, ptr(x), K, M, ptr(w), 1e-6, swapped,
                                        ptr(xq3), None, st()) == 0
    torch.cuda.synchronize()
    assert torch.equal(h2, h1)
    # the layout's padding bytes are never written: compare the qs and d fields
    qs_n, d_off = M * F, (M * F + 255) // 256 * 256
    for xq in (xq2, xq3):
        assert torch.equal(xq[:qs_n], xq1[:qs_n])
        assert torch.equal(xq[d_off:d_off + 4 * M * (F // 32)], xq1[d_off:d_off + 4 * M * (F // 32)])


def test_rms_norm_mul_mat_glu_rejects_unsupported(mm):
    L = mm.load()
    assert L.mmhip_rms_norm_mul_mat_glu_supported(8, 24576, 4096, 2) == 1
    assert L.mmhip_rms_norm_mul_mat_glu_supported(8, 24576, 8192, 2) == 0   # the norm: K <= 4096
    assert L.mmhip_rms_norm_mul_mat_glu_supported(8, 24576, 4096, 3) == 0   # M > 2
    assert L.mmhip_rms_norm_mul_mat_glu_supported(14, 24576, 4096, 2) == 0  # Q6_K weights
    assert L.mmhip_rms_norm_mul_mat_glu_supported(8, 24320, 4096, 2) == 0   # N / 2 not whole 256-chunks
    assert L.mmhip_rms_norm_mul_mat_glu_supported(8, 1 << 22, 4096, 2) == 0  # too many blocks per workgroup
    dummy = torch.zeros(16, dtype=torch.float32, device="cuda")
    rc = L.mmhip_rms_norm_mul_mat_glu(8, ptr(dummy), 24576, 8192, 8704, ptr(dummy), 8192, 2, ptr(dummy), 1e-6, 0,
                                      ptr(dummy), None, st())
    assert rc != 0


def test_swiglu_mul_mat_rejects_unsupported(mm):
    L = mm.load()
    assert L.mmhip_swiglu_mul_mat_supported(8, 4096, 12544, 2) == 0  # K > 12288
    assert L.mmhip_swiglu_mul_mat_supported(8, 4096, 12288, 3) == 0  # M > 2
    assert L.mmhip_swiglu_mul_mat_supported(12, 4096, 12288, 2) == 0  # Q4_K weights
    assert L.mmhip_swiglu_mul_mat_supported(14, 4096, 4096, 2) == 1   # Q6_K weights
    assert L.mmhip_swiglu_mul_mat_supported(14, 4096, 12288, 2) == 0  # Q6_K: the FFN width goes the two-pass way
    assert L.mmhip_swiglu_mul_mat_supported(14, 4096, 3072, 2) == 0   # Q6_K rows not 16-byte sized
    assert L.mmhip_rms_norm_mul_mat_supported(8, 4096, 8192, 2) == 0  # the norm: K <= 4096


# ---- DiT glue: LayerNorm, CONCAT, CLAMP ----

@pytest.mark.parametrize("shape", [(3, 2048), (2, 5, 300), (4, 1), (1, 4096 + 7)])
def test_layer_norm(mm, orc, shape):
    """GGML_OP_NORM vs the oracle: max-rel 1e-5 (f32 steps, double sums in
    another order); a strided view reads the same rows."""
    L = mm.load()
    rng = np.random.default_rng(31)
    x = (rng.standard_normal(shape) * 4 + 10).astype(np.float32)
    tx = torch.from_numpy(x).cuda()
    out = torch.empty_like(tx)
    assert L.mmhip_norm(ctypes.byref(mm.view_of(tx)), 1e-6, ptr(out), st()) == 0
    ref = orc.layer_norm(x, 1e-6)
    assert rel_err(out.cpu().numpy(), ref) < 1e-5
    # rows of a wider tensor (nb[1] = 2 * ne[0] * 4)
    wide = torch.from_numpy(np.concatenate([x, -x], axis=-1)).cuda()
    vw = wide[..., : shape[-1]]
    out2 = torch.empty_like(tx)
    assert L.mmhip_norm(ctypes.byref(mm.view_of(vw)), 1e-6, ptr(out2), st()) == 0
    assert torch.equal(out2, out)


def test_layer_norm_in_place_and_constant_rows(mm):
    L = mm.load()
    t = torch.full((3, 512), 2.5, device="cuda")
    assert L.mmhip_norm(ctypes.byref(mm.view_of(t)), 1e-6, ptr(t), st()) == 0
    assert torch.equal(t, torch.zeros_like(t))
    a = torch.tensor([1.0, -1.0], device="cuda").repeat(2, 64) + 7.0
    assert L.mmhip_norm(ctypes.byref(mm.view_of(a)), 3.0, ptr(a), st()) == 0
    exp = torch.tensor([0.5, -0.5], device="cuda").repeat(2, 64)
    assert torch.allclose(a, exp, rtol=1e-6, atol=0)


@pytest.mark.parametrize("dim", [0, 1, 2])
def test_concat(mm, dim):
    """GGML_OP_CONCAT, bit-exact against torch.cat (ggml dim d is torch dim 2-d
    for 3-d tensors)."""
    L = mm.load()
    g = torch.Generator().manual_seed(32 + dim)
    base = [4, 6, 40]
    sa, sb = list(base), list(base)
    sb[2 - dim] = 3
    a = torch.randn(sa, generator=g).cuda()
    b = torch.randn(sb, generator=g).cuda()
    ref = torch.cat([a, b], dim=2 - dim)
    out = torch.empty_like(ref)
    assert L.mmhip_concat(ctypes.byref(mm.view_of(a)), ctypes.byref(mm.view_of(b)), dim, ptr(out), st()) == 0
    assert torch.equal(out, ref)
    # a transposed (non-contiguous) first operand
    at_ = torch.randn([sa[0], sa[2], sa[1]], generator=g).cuda().transpose(1, 2)
    ref2 = torch.cat([at_, b], dim=2 - dim)
    out2 = torch.empty_like(ref2)
    assert L.mmhip_concat(ctypes.byref(mm.view_of(at_)), ctypes.byref(mm.view_of(b)), dim, ptr(out2), st()) == 0
    assert torch.equal(out2, ref2)


def test_concat_rejects_mismatched_shapes(mm):
    L = mm.load()
    a = torch.zeros(4, 8, device="cuda")
    b = torch.zeros(5, 7, device="cuda")
    out = torch.zeros(64, device="cuda")
    assert L.mmhip_concat(ctypes.byref(mm.view_of(a)), ctypes.byref(mm.view_of(b)), 0, ptr(out), st()) != 0
    assert L.mmhip_concat(ctypes.byref(mm.view_of(a)), ctypes.byref(mm.view_of(a)), 4, ptr(out), st()) != 0


def test_clamp(mm):
    """GGML_OP_CLAMP: MAX(MIN(x, hi), lo) with ggml's comparison macros,
    bit-exact; NaN becomes hi (x < hi is false, then hi > lo)."""
    L = mm.load()

    def ref(a, lo, hi):
        t = np.where(a < np.float32(hi), a, np.float32(hi))
        return np.where(t > np.float32(lo), t, np.float32(lo))

    rng = np.random.default_rng(33)
    x = (rng.standard_normal((3, 7, 129)) * 10).astype(np.float32)
    x[0, 0, :5] = [np.inf, -np.inf, 0.0, -0.0, np.nan]
    tx = torch.from_numpy(x).cuda()
    out = torch.empty_like(tx)
    assert L.mmhip_clamp(ctypes.byref(mm.view_of(tx)), -3.5, 2.25, ptr(out), st()) == 0
    o = out.cpu().numpy()
    assert np.array_equal(o, ref(x, -3.5, 2.25)) and o[0, 0, 4] == np.float32(2.25)
    # strided input; then in place on a contiguous tensor
    tv = tx.transpose(1, 2)
    o2 = torch.empty(tv.shape, device="cuda")
    assert L.mmhip_clamp(ctypes.byref(mm.view_of(tv)), -1.0, 1.0, ptr(o2), st()) == 0
    assert np.array_equal(o2.cpu().numpy(), ref(x.transpose(0, 2, 1), -1.0, 1.0))
    assert L.mmhip_clamp(ctypes.byref(mm.view_of(tx)), -1.0, 1.0, ptr(tx), st()) == 0
    assert np.array_equal(tx.cpu().numpy(), ref(x, -1.0, 1.0))


def test_norm_affine_equals_three_ops(mm, orc):
    """mmhip_norm_affine (dit_layer_norm fused) is bit-identical to
    mmhip_norm followed by the MUL by w and the ADD of b in f32."""
    L = mm.load()
    rng = np.random.default_rng(34)
    x = (rng.standard_normal((5, 2048)) * 3 + 1).astype(np.float32)
    w = (1 + 0.1 * rng.standard_normal(2048)).astype(np.float32)
    b = (0.1 * rng.standard_normal(2048)).astype(np.float32)
    tx, tw, tb = (torch.from_numpy(a).cuda() for a in (x, w, b))
    n = torch.empty_like(tx)
    assert L.mmhip_norm(ctypes.byref(mm.view_of(tx)), 1e-5, ptr(n), st()) == 0
    out = torch.empty_like(tx)
    assert L.mmhip_norm_affine(ctypes.byref(mm.view_of(tx)), 1e-5, ptr(tw), ptr(tb), ptr(out), st()) == 0
    assert torch.equal(out, n * tw + tb)
    assert rel_err(out.cpu().numpy(), orc.layer_norm(x, 1e-5) * w + b) < 1e-5


@pytest.mark.parametrize("case", ["dit_kv_cast", "f16_to_f32", "odd_inner", "misaligned"])
def test_cpy_row_paths(mm, case):
    """CPY / CONT over views with contiguous inner rows (the DiT's K/V cast of
    the permuted projections, src/dit.h:219-220, and the value / gate conts,
    :239-241): bit-exact against torch, including the generic fallback cases
    (inner size not a multiple of 4, misaligned start)."""
    L = mm.load()
    g = torch.Generator().manual_seed(35)
    if case == "dit_kv_cast":
        k = torch.randn((2, 37, 32, 64), generator=g).cuda()      # [B, S, H, D]
        src, dt = k.permute(0, 2, 1, 3), torch.float16            # [B, H, S, D] view
    elif case == "f16_to_f32":
        src, dt = torch.randn((5, 6, 128), generator=g).half().cuda().transpose(0, 1), torch.float32
    elif case == "odd_inner":
        src, dt = torch.randn((7, 9, 30), generator=g).cuda().transpose(0, 1), torch.float16
    else:
        src, dt = torch.randn((4, 6, 65), generator=g).cuda()[:, :, 1:], torch.float32
    dst = torch.empty(src.shape, dtype=dt, device="cuda")
    stype = 0 if src.dtype == torch.float32 else 1
    dtype_ = 0 if dt == torch.float32 else 1
    assert L.mmhip_cpy(ctypes.byref(mm.view_of(src)), stype, ctypes.byref(mm.view_of(dst)), dtype_, st()) == 0
    assert torch.equal(dst, src.to(dt))


def test_norm_affine_h_and_gemm_on_f16_rows(mm, pkg):
    """mmhip_norm_affine_h writes the f32 rows' f16 rounding, and
    mmhip_mul_mat_bias_add_h on those rows equals mmhip_mul_mat_bias_add on
    the f32 rows (which rounds them to f16 itself), bit for bit."""
    L = mm.load()
    rng = np.random.default_rng(36)
    M, K, N = 96, 2048, 384
    x = (rng.standard_normal((M, K)) * 2).astype(np.float32)
    w = (1 + 0.1 * rng.standard_normal(K)).astype(np.float32)
    b = (0.1 * rng.standard_normal(K)).astype(np.float32)
    tx, tw, tb = (torch.from_numpy(a).cuda() for a in (x, w, b))
    f32 = torch.empty_like(tx)
    h16 = torch.empty((M, K), dtype=torch.float16, device="cuda")
    assert L.mmhip_norm_affine_h(ctypes.byref(mm.view_of(tx)), 1e-5, ptr(tw), ptr(tb), ptr(f32), ptr(h16), st()) == 0
    ref = torch.empty_like(tx)
    assert L.mmhip_norm_affine(ctypes.byref(mm.view_of(tx)), 1e-5, ptr(tw), ptr(tb), ptr(ref), st()) == 0
    assert torch.equal(f32, ref) and torch.equal(h16, ref.half())
    raw = pkg.synth.gguf_blocks_np(8, N, K, 37)
    W = mm.QuantWeight.from_gguf(8, raw, N, K)
    bias = torch.randn(N, device="cuda")
    y1 = torch.empty((M, N), device="cuda")
    y2 = torch.empty((M, N), device="cuda")
    need = L.mmhip_mul_mat_workspace(8, N, K, M)
    ws = torch.empty(need, dtype=torch.uint8, device="cuda")
    assert L.mmhip_mul_mat_bias_add(8, ptr(W.data), N, K, W.row_bytes, ptr(f32), K, M, ptr(bias), None, 0, ptr(y1), N,
                                    ptr(ws), need, st()) == 0
    assert L.mmhip_mul_mat_bias_add_h(8, ptr(W.data), N, K, W.row_bytes, ptr(h16), M, ptr(bias), None, 0, ptr(y2), N,
                                      st()) == 0
    torch.cuda.synchronize()
    assert torch.equal(y1, y2)
