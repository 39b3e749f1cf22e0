"""GPU: the fused GEMM forms the DiT block runs.

1. The feed-forward input with its SwiGLU in the GEMM epilogue
(mmhip_mul_mat_bias_swiglu(_h), src/dit.h:236-242).

The fused form must equal the separate ops bit for bit: the GEMM with the
bias ADD in its store (mmhip_mul_mat_bias_add, itself checked against the
oracle in test_gpu_mul_mat.py), then GGML_OP_GLU swiglu_split(gate, value) on
the two halves (mmhip_swiglu).  The f16 output equals the f32 output rounded
to f16 (the next GEMM's activation copy).  An oracle check at fp64 closes the
loop on a small shape (cosine >= 0.9999: the GEMM rounds activations and
dequantised weights to f16).

2. Several MUL_MATs of one activation tensor in one launch
(mmhip_mul_mat_multi(_h), the q / k / v projections, src/dit.h:197-199):
bit for bit the separate calls.

3. Split-K for few output tiles and a long K (mmhip_mul_mat_bias_add_hw,
ff_out, src/dit.h:243-246): the parts' sums are added in another order than
the single pass, so the result is checked against the unsplit GEMM (max
|diff| <= 1e-5 x max |y|) and the fp64 oracle (cosine >= 0.9999), and the f32
and f16 entry points (which split the same way) bit for bit."""
import ctypes

import numpy as np
import pytest
import torch

from conftest import cosine

pytestmark = pytest.mark.gpu


def ptr(t):
    return ctypes.c_void_p(t.data_ptr())


def separate(mm, W, x, bias, swapped):
    ff = mm.mul_mat_bias_add(W, x, bias)
    F = W.N // 2
    value, gate = (ff[:, F:], ff[:, :F]) if swapped else (ff[:, :F], ff[:, F:])
    out = torch.empty((x.shape[0], F), dtype=torch.float32, device="cuda")
    L = mm.load()
    rc = L.mmhip_swiglu(ctypes.byref(mm.view_of(gate)), ctypes.byref(mm.view_of(value)), 0, ptr(out),
                        ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert rc == 0
    return out


@pytest.mark.parametrize("t,F,K,M,swapped,with_bias", [
    (8, 8192, 2048, 1380, False, True),   # the DiT's ff_in at its real shape (256 x 256 tiles)
    (8, 384, 512, 100, False, True),      # small grid: 64 x 128 tiles
    (8, 200, 256, 70, True, True),        # F not a multiple of the tile's columns; gate first
    (12, 512, 1024, 300, False, False),   # Q4_K, no bias
    (14, 256, 2048, 33, True, True),      # Q6_K (rows of 1680 bytes)
])
def test_fused_equals_separate_ops(mm, pkg, t, F, K, M, swapped, with_bias):
    raw = pkg.synth.gguf_blocks_np(t, 2 * F, K, 5000 + F)
    W = mm.QuantWeight.from_gguf(t, raw, 2 * F, K)
    x = torch.from_numpy(pkg.synth.normal_np((M, K), 5100 + M)).cuda()
    bias = torch.from_numpy(pkg.synth.normal_np((2 * F,), 5200)).cuda() if with_bias else None
    h, hh = mm.mul_mat_bias_swiglu(W, x, bias, swapped, f32_out=True, f16_out=True)
    ref = separate(mm, W, x, bias, swapped)
    torch.cuda.synchronize()
    assert torch.isfinite(h).all()
    assert torch.equal(h.view(torch.int32), ref.view(torch.int32))
    assert torch.equal(hh.view(torch.int16), ref.half().view(torch.int16))
    # f16 activations in: the same values (the f32 path rounds x to f16 first)
    h2, hh2 = mm.mul_mat_bias_swiglu(W, x.half().contiguous(), bias, swapped, f32_out=True, f16_out=True)
    assert torch.equal(h2.view(torch.int32), h.view(torch.int32))
    assert torch.equal(hh2.view(torch.int16), hh.view(torch.int16))
    # f16 output alone
    _, hh3 = mm.mul_mat_bias_swiglu(W, x, bias, swapped, f32_out=False, f16_out=True)
    assert torch.equal(hh3.view(torch.int16), hh.view(torch.int16))


def test_fused_against_oracle(mm, orc, pkg):
    t, F, K, M = 8, 160, 256, 40
    raw = pkg.synth.gguf_blocks_np(t, 2 * F, K, 6000)
    W = mm.QuantWeight.from_gguf(t, raw, 2 * F, K)
    xn = pkg.synth.normal_np((M, K), 6001)
    bn = pkg.synth.normal_np((2 * F,), 6002)
    h, _ = mm.mul_mat_bias_swiglu(W, torch.from_numpy(xn).cuda(), torch.from_numpy(bn).cuda())
    ff = orc.mul_mat_f64(t, raw, 2 * F, K, xn).astype(np.float64) + bn.astype(np.float64)
    v, g = ff[:, :F], ff[:, F:]
    ref = g / (1.0 + np.exp(-g)) * v
    assert cosine(h.cpu().numpy(), ref) > 0.9999


def test_rejects_bad_arguments(mm):
    L = mm.load()
    P = ctypes.c_void_p(16)
    # odd N, no output, a GEMV token count
    assert L.mmhip_mul_mat_bias_swiglu_h(8, P, 257, 256, 272, P, 64, None, 0, P, None, None) != 0
    assert L.mmhip_mul_mat_bias_swiglu_h(8, P, 256, 256, 272, P, 64, None, 0, None, None, None) != 0
    assert L.mmhip_mul_mat_bias_swiglu_h(8, P, 256, 256, 272, P, 4, None, 0, P, None, None) != 0


# ---------------------------------------------------------------------------
# several MUL_MATs of one activation tensor in one launch (the DiT's q / k / v)

def _arr(ctype, vals):
    return (ctype * len(vals))(*vals)


@pytest.mark.parametrize("t,n,N,K,M,with_bias", [
    (8, 3, 2048, 2048, 1380, False),  # the DiT's q / k / v: 144 tiles of 256 x 256 in one launch
    (8, 2, 512, 512, 300, True),      # a small grid: 64 x 128 tiles
    (12, 3, 256, 1024, 77, True),     # Q4_K
])
def test_multi_equals_separate_calls(mm, pkg, t, n, N, K, M, with_bias):
    Ws = [mm.QuantWeight.from_gguf(t, pkg.synth.gguf_blocks_np(t, N, K, 7000 + i), N, K) for i in range(n)]
    x = torch.from_numpy(pkg.synth.normal_np((M, K), 7100)).cuda()
    bs = [torch.from_numpy(pkg.synth.normal_np((N,), 7200 + i)).cuda() for i in range(n)] if with_bias else None
    refs = [mm.mul_mat_bias_add(W, x, bs[i] if bs else None) for i, W in enumerate(Ws)]
    L = mm.load()
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    W_p = _arr(ctypes.c_void_p, [W.data.data_ptr() for W in Ws])
    b_p = _arr(ctypes.c_void_p, [b.data_ptr() for b in bs]) if bs else None
    ld = _arr(ctypes.c_int64, [N] * n)
    for f16 in (False, True):
        ys = [torch.full((M, N), float("nan"), device="cuda") for _ in range(n)]
        y_p = _arr(ctypes.c_void_p, [y.data_ptr() for y in ys])
        if f16:
            xh = x.half().contiguous()
            rc = L.mmhip_mul_mat_multi_h(t, n, W_p, N, K, Ws[0].row_bytes, ptr(xh), M, b_p, y_p, ld, st)
        else:
            need = L.mmhip_mul_mat_workspace(t, N, K, M)
            ws = torch.empty(need, dtype=torch.uint8, device="cuda")
            rc = L.mmhip_mul_mat_multi(t, n, W_p, N, K, Ws[0].row_bytes, ptr(x), K, M, b_p, y_p, ld, ptr(ws), need, st)
        assert rc == 0, L.mmhip_last_error()
        torch.cuda.synchronize()
        for y, r in zip(ys, refs):
            assert torch.equal(y.view(torch.int32), r.view(torch.int32))


def test_multi_rejects_bad_arguments(mm):
    L = mm.load()
    P = ctypes.c_void_p(16)
    W_p = _arr(ctypes.c_void_p, [16, 16, 16])
    ld = _arr(ctypes.c_int64, [256] * 3)
    y_p = _arr(ctypes.c_void_p, [16, 16, 16])
    # n out of range, N not a multiple of 256, a GEMV token count
    assert L.mmhip_mul_mat_multi_h(8, 4, W_p, 256, 256, 272, P, 64, None, y_p, ld, None) != 0
    assert L.mmhip_mul_mat_multi_h(8, 3, W_p, 200, 256, 272, P, 64, None, y_p, ld, None) != 0
    assert L.mmhip_mul_mat_multi_h(8, 3, W_p, 256, 256, 272, P, 4, None, y_p, ld, None) != 0


# ---------------------------------------------------------------------------
# split-K (the DiT's ff_out: 2048 rows, K = 8192, 1380 tokens, bias + residual)

@pytest.mark.parametrize("t,N,K,M", [(8, 2048, 8192, 1380), (12, 1024, 4096, 300)])
def test_split_k(mm, orc, pkg, t, N, K, M):
    raw = pkg.synth.gguf_blocks_np(t, N, K, 8000 + N)
    W = mm.QuantWeight.from_gguf(t, raw, N, K)
    xn = pkg.synth.normal_np((M, K), 8100)
    x = torch.from_numpy(xn).cuda()
    bias = torch.from_numpy(pkg.synth.normal_np((N,), 8200)).cuda()
    res = torch.from_numpy(pkg.synth.normal_np((M, N), 8300)).cuda()
    L = mm.load()
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    need = L.mmhip_mul_mat_h_workspace(t, N, K, M)
    assert need == 4 * M * N * 4  # four K parts of f32 partial sums
    xh = x.half().contiguous()
    ws = torch.empty(need, dtype=torch.uint8, device="cuda")
    y_split = torch.empty((M, N), device="cuda")
    y_one = torch.empty((M, N), device="cuda")
    assert L.mmhip_mul_mat_bias_add_hw(t, ptr(W.data), N, K, W.row_bytes, ptr(xh), M, ptr(bias), ptr(res), N,
                                       ptr(y_split), N, ptr(ws), need, st) == 0
    assert L.mmhip_mul_mat_bias_add_h(t, ptr(W.data), N, K, W.row_bytes, ptr(xh), M, ptr(bias), ptr(res), N,
                                      ptr(y_one), N, st) == 0
    # the f32 entry point splits the same way (its workspace holds the f16 copy and the parts)
    y_f32 = mm.mul_mat_bias_add(W, x, bias, res)
    torch.cuda.synchronize()
    assert torch.isfinite(y_split).all()
    assert torch.equal(y_f32.view(torch.int32), y_split.view(torch.int32))
    assert (y_split - y_one).abs().max().item() <= 1e-5 * y_one.abs().max().item()
    rows = np.arange(0, M, 97)
    ref = orc.mul_mat_f64(t, raw, N, K, xn[rows]) + pkg.synth.normal_np((N,), 8200)[None] + res.cpu().numpy()[rows]
    assert cosine(y_split.cpu().numpy()[rows], ref) > 0.9999


# f16 weight copies registered under the quantised weight (the backend's
# copies for repeating graphs, such as the DiT's per diffusion step)

@pytest.mark.parametrize("t,N,K,M,kind", [
    (8, 2048, 2048, 1380, "bias_res_h"),   # the DiT's o projection: 64 x 128 ring tiles
    (8, 16384, 2048, 1380, "swiglu_h"),    # ff_in with the SwiGLU epilogue: 256 x 256 ring tiles
    (8, 2048, 8192, 1380, "split_h"),      # ff_out: split-K on the ring, then the ordered reduce
    (8, 2048, 2048, 690, "multi_h"),       # q / k / v in one launch
    (12, 6144, 2048, 300, "plain"),        # f32 activations below the per-call copy threshold
    (14, 3000, 2048, 2100, "plain"),       # f32 activations above it (the registered copy replaces it)
])
def test_registered_f16_weights_give_the_same_bits(mm, pkg, t, N, K, M, kind):
    """GEMMs above 16 tokens on weights with a registered f16 copy
    (mmhip_weights_to_f16 + mmhip_register_weights_f16) read the copy through
    the DMA ring and return the unregistered call's bits in every form; once
    unregistered the same call takes its own path again.  A copy registered
    for another shape is not used."""
    L = mm.load()
    nm = 3 if kind == "multi_h" else 1
    Ws = [mm.QuantWeight.from_gguf(t, pkg.synth.gguf_blocks_np(t, N, K, 7300 + t + i), N, K) for i in range(nm)]
    x = torch.from_numpy(pkg.synth.normal_np((M, K), 7400 + t)).cuda()
    xh = x.half().contiguous()
    b = torch.from_numpy(pkg.synth.normal_np((N,), 7500)).cuda()
    r = torch.from_numpy(pkg.synth.normal_np((M, N), 7600)).cuda()
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    rs = Ws[0].row_bytes

    def run():
        if kind == "swiglu_h":
            h = torch.full((M, N // 2), float("nan"), device="cuda")
            hh = torch.zeros((M, N // 2), dtype=torch.float16, device="cuda")
            rc = L.mmhip_mul_mat_bias_swiglu_h(t, ptr(Ws[0].data), N, K, rs, ptr(xh), M, ptr(b), 0, ptr(h), ptr(hh), st)
            outs = [h, hh]
        elif kind == "multi_h":
            ys = [torch.full((M, N), float("nan"), device="cuda") for _ in range(nm)]
            rc = L.mmhip_mul_mat_multi_h(t, nm, _arr(ctypes.c_void_p, [W.data.data_ptr() for W in Ws]), N, K, rs,
                                         ptr(xh), M, None, _arr(ctypes.c_void_p, [y.data_ptr() for y in ys]),
                                         _arr(ctypes.c_int64, [N] * nm), st)
            outs = ys
        else:
            y = torch.full((M, N), float("nan"), device="cuda")
            if kind == "bias_res_h":
                rc = L.mmhip_mul_mat_bias_add_h(t, ptr(Ws[0].data), N, K, rs, ptr(xh), M, ptr(b), ptr(r), N, ptr(y), N, st)
            elif kind == "split_h":
                need = L.mmhip_mul_mat_h_workspace(t, N, K, M)
                assert need > 0
                ws = torch.empty(need, dtype=torch.uint8, device="cuda")
                rc = L.mmhip_mul_mat_bias_add_hw(t, ptr(Ws[0].data), N, K, rs, ptr(xh), M, ptr(b), ptr(r), N, ptr(y),
                                                 N, ptr(ws), need, st)
            else:
                need = L.mmhip_mul_mat_workspace(t, N, K, M)
                ws = torch.empty(need, dtype=torch.uint8, device="cuda")
                rc = L.mmhip_mul_mat(t, ptr(Ws[0].data), N, K, rs, ptr(x), K, M, ptr(y), N, ptr(ws), need, st)
            outs = [y]
        assert rc == 0, L.mmhip_last_error()
        torch.cuda.synchronize()
        return outs

    base = run()
    copies = [torch.empty(L.mmhip_weights_f16_bytes(N, K), dtype=torch.uint8, device="cuda") for _ in Ws]
    for W, c in zip(Ws, copies):
        assert L.mmhip_weights_to_f16(t, ptr(W.data), N, K, rs, ptr(c), st) == 0, L.mmhip_last_error()
        assert L.mmhip_register_weights_f16(ptr(W.data), N + 256, K, ptr(c)) == 0  # another shape: ignored
    assert all(torch.equal(a, b_) for a, b_ in zip(run(), base))
    try:
        for W, c in zip(Ws, copies):
            assert L.mmhip_register_weights_f16(ptr(W.data), N, K, ptr(c)) == 0
        reg = run()
    finally:
        for W in Ws:
            assert L.mmhip_unregister_weights_f16(ptr(W.data)) == 0
    assert L.mmhip_unregister_weights_f16(ptr(Ws[0].data)) != 0  # already gone
    after = run()
    for a, c, d in zip(base, reg, after):
        assert torch.equal(a.view(torch.int16 if a.dtype == torch.float16 else torch.int32),
                           c.view(torch.int16 if c.dtype == torch.float16 else torch.int32))
        assert torch.equal(a.view(torch.int16 if a.dtype == torch.float16 else torch.int32),
                           d.view(torch.int16 if d.dtype == torch.float16 else torch.int32))
    assert torch.isfinite(base[0]).all()
