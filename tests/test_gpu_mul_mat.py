"""GPU: GGML_OP_MUL_MAT over Q8_0 / Q4_K / Q5_K / Q6_K weights against the oracle.

Tolerances (stated): against the ggml-CPU-semantics oracle, which quantises
activations the same way and differs only in f32 summation order,
max|y - y_ggml| <= 2e-5 * max|y_ggml|; against the exact fp64 oracle,
cosine >= 0.9999 (ggml-CPU's own activation-quantisation error)."""
import ctypes

import numpy as np
import pytest
import torch

from conftest import cosine, rel_err

pytestmark = pytest.mark.gpu


def run(mm, orc, pkg, t, N, K, M, seed):
    raw = pkg.synth.gguf_blocks_np(t, N, K, seed)
    x = pkg.synth.normal_np((M, K), seed + 1)
    W = mm.QuantWeight.from_gguf(t, raw, N, K)
    y = mm.mul_mat(W, torch.from_numpy(x).cuda()).cpu().numpy()
    return y, orc.mul_mat_ggml(t, raw, N, K, x), orc.mul_mat_f64(t, raw, N, K, x)


@pytest.mark.parametrize("t", [8, 12, 13, 14])
@pytest.mark.parametrize("M", [1, 2, 3, 5, 8, 12, 16])
def test_gemv_small(mm, orc, pkg, t, M):
    y, yg, yf = run(mm, orc, pkg, t, 1000, 2048, M, 2000 + 10 * t + M)
    assert rel_err(y, yg) < 2e-5
    assert cosine(y, yf) > 0.9999


@pytest.mark.parametrize("t", [8, 12, 13, 14])
@pytest.mark.parametrize("N,K", [(6144, 4096), (4096, 12288), (2048, 2304), (3, 256), (513, 1280), (256, 512),
                                 (1000, 256), (1024, 256)])
def test_gemv_decode_shapes(mm, orc, pkg, t, N, K):
    y, yg, yf = run(mm, orc, pkg, t, N, K, 2, 3000 + t + N)
    assert rel_err(y, yg) < 2e-5
    assert cosine(y, yf) > 0.9999


def test_gemv_q8_0_benchmark_shape(mm, orc, pkg):
    """The Q8_0 decode GEMV workload at full size: W 12288 x 4096, x [2 x 4096]."""
    y, yg, yf = run(mm, orc, pkg, 8, 12288, 4096, 2, 1002)
    assert rel_err(y, yg) < 2e-5
    assert cosine(y, yf) > 0.9999
    # swapping the two CFG rows swaps the outputs exactly
    raw = pkg.synth.gguf_blocks_np(8, 12288, 4096, 1002)
    x = pkg.synth.normal_np((2, 4096), 1003)
    W = mm.QuantWeight.from_gguf(8, raw, 12288, 4096)
    a = mm.mul_mat(W, torch.from_numpy(x).cuda())
    b = mm.mul_mat(W, torch.from_numpy(x[::-1].copy()).cuda())
    assert torch.equal(a, b.flip(0))


def test_gemv_rejects_bad_shapes(mm, pkg):
    raw = pkg.synth.gguf_blocks_np(8, 4, 96, 1)
    W = mm.QuantWeight.from_gguf(8, raw, 4, 96)
    with pytest.raises(mm.MmhipError) as e:
        mm.mul_mat(W, torch.zeros((2, 96), device="cuda"))
    assert e.value.code == mm.ERR_UNSUPPORTED


# ---------------------------------------------------------------------------
# token counts (M > 16): MFMA GEMM on f16-rounded dequantised weights and
# f16-rounded activations with f32 accumulation.  Stated tolerance against
# the exact fp64 oracle: relative RMS error <= 2e-3 and cosine >= 0.99999;
# against the ggml-CPU-semantics oracle: cosine >= 0.9999.

def rel_rms(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / np.linalg.norm(b))


@pytest.mark.parametrize("t", [8, 12, 13, 14])
@pytest.mark.parametrize("N,K,M", [(384, 2048, 200), (100, 4096, 17), (130, 2048, 1380)])
def test_gemm_shapes(mm, orc, pkg, t, N, K, M):
    y, yg, yf = run(mm, orc, pkg, t, N, K, M, 5000 + t + M)
    assert rel_rms(y, yf) < 2e-3
    assert cosine(y, yf) > 0.99999
    assert cosine(y, yg) > 0.9999


@pytest.mark.parametrize("N,K,M", [(96, 2304, 40), (300, 768, 600), (2048, 2048, 1380)])
def test_gemm_q8_0_k_steps(mm, orc, pkg, N, K, M):
    """Q8_0 GEMMs on small grids (128-wide K steps): the DiT preprocess K,
    a short K and the DiT projection shape.  (16-byte weight rows make K a
    multiple of 256 on this path.)"""
    y, yg, yf = run(mm, orc, pkg, 8, N, K, M, 5100 + K + M)
    assert rel_rms(y, yf) < 2e-3
    assert cosine(y, yf) > 0.99999
    assert cosine(y, yg) > 0.9999


def test_gemm_q4_K_benchmark_shape_sampled(mm, orc, pkg):
    """DiT QKV projection workload: W 6144 x 2048 Q4_K, 8192 tokens; checked
    on 40 sampled tokens."""
    N, K, M = 6144, 2048, 8192
    raw = pkg.synth.gguf_blocks_np(12, N, K, 1005)
    x = pkg.synth.normal_np((M, K), 1006)
    W = mm.QuantWeight.from_gguf(12, raw, N, K)
    y = mm.mul_mat(W, torch.from_numpy(x).cuda()).cpu().numpy()
    rows = np.array([0, 1, 127, 128, 4095, 8191] + list(np.random.default_rng(8).choice(M, 34, replace=False)))
    yf = orc.mul_mat_f64(12, raw, N, K, x[rows])
    assert rel_rms(y[rows], yf) < 2e-3
    assert cosine(y[rows], yf) > 0.99999


def test_gemm_matches_gemv_semantics_closely(mm, pkg):
    """M = 16 (GEMV in two column groups, activation-quantised) and M = 17
    (GEMM, f16) agree on the shared rows to the activation-quantisation
    error."""
    N, K = 512, 2048
    raw = pkg.synth.gguf_blocks_np(8, N, K, 77)
    x = torch.from_numpy(pkg.synth.normal_np((17, K), 78)).cuda()
    W = mm.QuantWeight.from_gguf(8, raw, N, K)
    a = mm.mul_mat(W, x[:16].contiguous()).cpu().numpy()
    b = mm.mul_mat(W, x).cpu().numpy()[:16]
    assert cosine(a, b) > 0.9999


@pytest.mark.parametrize("t", [8, 12, 13, 14])
@pytest.mark.parametrize("bias,res", [(True, False), (False, True), (True, True)])
def test_gemm_bias_add_equals_separate_ops(mm, pkg, t, bias, res):
    """mmhip_mul_mat_bias_add (the DiT's projection + bias, + residual) is
    bit-identical to mmhip_mul_mat followed by the two ADDs in f32; the
    residual may be the output buffer itself."""
    import ctypes

    N, K, M = 300, 2048, 77  # Q6_K rows of 2048 are 16-byte multiples (GEMM loads)
    raw = pkg.synth.gguf_blocks_np(t, N, K, 4100 + t)
    W = mm.QuantWeight.from_gguf(t, raw, N, K)
    x = torch.from_numpy(pkg.synth.normal_np((M, K), 4200 + t)).cuda()
    b = torch.randn(N, device="cuda") if bias else None
    r = torch.randn(M, N, device="cuda") if res else None
    y0 = mm.mul_mat(W, x)
    ref = y0 + b if bias else y0
    ref = r + ref if res else ref
    L = mm.load()
    need = L.mmhip_mul_mat_workspace(t, N, K, M)
    ws = torch.empty(need, dtype=torch.uint8, device="cuda")
    P = lambda a: ctypes.c_void_p(a.data_ptr()) if a is not None else None
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    out = r.clone() if res else torch.empty(M, N, device="cuda")
    rc = L.mmhip_mul_mat_bias_add(t, P(W.data), N, K, W.row_bytes, P(x), K, M, P(b), P(out) if res else None,
                                  N, P(out), N, P(ws), need, st)
    assert rc == 0, L.mmhip_last_error()
    torch.cuda.synchronize()
    assert torch.equal(out, ref)


def test_gemm_bias_add_rejects_gemv_token_counts(mm):
    import ctypes

    L = mm.load()
    d = torch.zeros(1 << 16, device="cuda")
    P = ctypes.c_void_p(d.data_ptr())
    assert L.mmhip_mul_mat_bias_add(8, P, 64, 256, 272, P, 256, 16, P, None, 0, P, 64, P, 1 << 18, None) != 0


@pytest.mark.parametrize("N,K,M", [(4096, 4096, 2), (1000, 2048, 16), (37, 520, 5), (6144, 4096, 16), (300, 1024, 1)])
def test_mul_mat_bf16_weights(mm, N, K, M):
    """MUL_MAT over BF16 weights at 1..16 tokens (ggml's BF16 dot: the
    activations rounded to bf16 -- torch's bfloat16 rounding, nearest-even
    -- and the products summed in f32) against float64 of the same bf16
    operands: max-rel 1e-5."""
    import ctypes

    g = torch.Generator().manual_seed(N + K + M)
    W = (torch.randn((N, K), generator=g) * 0.02).bfloat16()
    x = torch.randn((M, K), generator=g)
    ref = x.bfloat16().double() @ W.double().T
    L = mm.load()
    tw, tx = W.cuda(), x.cuda()
    y = torch.empty((M, N), device="cuda")
    P = lambda t: ctypes.c_void_p(t.data_ptr())
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    assert L.mmhip_mul_mat_bf16(P(tw), N, K, K, P(tx), K, M, P(y), N, st) == 0, L.mmhip_last_error()
    torch.cuda.synchronize()
    assert float((y.cpu().double() - ref).abs().max() / ref.abs().max()) < 1e-5


def test_mul_mat_bf16_rejects_and_backend(mm, pkg):
    """Over 16 tokens or K % 8 != 0 is refused; through the backend a BF16
    MUL_MAT node gives the C-ABI result bit for bit."""
    import ctypes
    import importlib

    L = mm.load()
    d = torch.zeros(1 << 16, device="cuda")
    P = ctypes.c_void_p(d.data_ptr())
    assert L.mmhip_mul_mat_bf16(P, 64, 256, 256, P, 256, 17, P, 64, None) != 0
    assert L.mmhip_mul_mat_bf16(P, 64, 250, 256, P, 256, 4, P, 64, None) != 0
    og = importlib.import_module(pkg.__name__ + ".opgraph")
    N, K, M = 512, 2048, 6
    g = torch.Generator().manual_seed(5)
    W = (torch.randn((N, K), generator=g) * 0.02).bfloat16()
    x = torch.randn((M, K), generator=g)
    gr = og.OpGraph()
    try:
        tw = gr.tensor(30, [K, N])  # GGML_TYPE_BF16
        tx = gr.tensor(og.F32, [K, M])
        out = gr.mul_mat(tw, tx)
        gr.build([out])
        gr.set(tw, W.view(torch.int16).numpy())
        gr.set(tx, x.numpy())
        gr.compute()
        yb = gr.get(out).reshape(M, N)
    finally:
        gr.close()
    y = torch.empty((M, N), device="cuda")
    Q = lambda t: ctypes.c_void_p(t.data_ptr())
    assert L.mmhip_mul_mat_bf16(Q(W.cuda()), N, K, K, Q(x.cuda()), K, M, Q(y), N, None) == 0
    torch.cuda.synchronize()
    assert np.array_equal(yb, y.cpu().numpy())


@pytest.mark.parametrize("N,K,M,pad", [(2048, 2048, 1380, 0), (6144, 4096, 100, 0), (37, 544, 33, 32),
                                       (4096, 2048, 8192, 0), (300, 1024, 17, 64), (1000, 8192, 257, 0),
                                       (16384, 2048, 1380, 0)])
def test_mul_mat_bf16_gemm(mm, N, K, M, pad):
    """MUL_MAT over BF16 weights above 16 tokens: the bf16 MFMA GEMM reading
    the weight rows in place (row stride K + pad elements) through the 16-bit
    DMA ring, on a bf16 copy of the activations.  ggml's BF16 arithmetic --
    activations rounded to bf16 (torch's rounding, nearest-even), exact
    products, f32 sums -- against float64 of the same bf16 operands, max-rel
    2e-5 (f32 sums over K <= 8192).  Shapes cover the three tile
    configurations (64 x 128 tiles on small grids, 256 x 256 at 8192 tokens,
    192 x 256 at 1380 tokens x 16384 rows), ragged N and M, and padded rows; the
    workspace is the bf16 copy and a smaller one is refused."""
    import ctypes

    g = torch.Generator().manual_seed(N + K + M)
    Wp = (torch.randn((N, K + pad), generator=g) * 0.02).bfloat16()
    W = Wp[:, :K]
    x = torch.randn((M, K), generator=g)
    ref = (x.bfloat16().double().cuda() @ W.double().cuda().T).cpu()
    L = mm.load()
    need = L.mmhip_mul_mat_workspace(30, N, K, M)
    assert need == M * K * 2
    ws = torch.empty(need, dtype=torch.uint8, device="cuda")
    tw, tx = Wp.cuda(), x.cuda()
    y = torch.full((M, N), float("nan"), device="cuda")
    P = lambda t: ctypes.c_void_p(t.data_ptr())
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    rs = (K + pad) * 2
    assert L.mmhip_mul_mat(30, P(tw), N, K, rs, P(tx), K, M, P(y), N, P(ws), need - 16, st) == -4
    assert L.mmhip_mul_mat(30, P(tw), N, K, rs, P(tx), K, M, P(y), N, P(ws), need, st) == 0, L.mmhip_last_error()
    torch.cuda.synchronize()
    yc = y.cpu().double()
    assert torch.isfinite(yc).all()
    assert float((yc - ref).abs().max() / ref.abs().max()) < 2e-5


def test_mul_mat_bf16_gemm_backend(mm, pkg):
    """A BF16 MUL_MAT node at 100 tokens runs on the backend (supports_op
    takes BF16 above 16 tokens at K % 32 == 0) and gives the C-ABI GEMM's
    result bit for bit; at K % 32 != 0 above 16 tokens the C-ABI refuses."""
    import ctypes
    import importlib

    L = mm.load()
    d = torch.zeros(1 << 16, device="cuda")
    Pd = ctypes.c_void_p(d.data_ptr())
    assert L.mmhip_mul_mat(30, Pd, 64, 272, 544, Pd, 272, 17, Pd, 64, Pd, 1 << 18, None) != 0
    og = importlib.import_module(pkg.__name__ + ".opgraph")
    N, K, M = 512, 2048, 100
    g = torch.Generator().manual_seed(6)
    W = (torch.randn((N, K), generator=g) * 0.02).bfloat16()
    x = torch.randn((M, K), generator=g)
    gr = og.OpGraph()
    try:
        tw = gr.tensor(30, [K, N])  # GGML_TYPE_BF16
        tx = gr.tensor(og.F32, [K, M])
        out = gr.mul_mat(tw, tx)
        gr.build([out])
        gr.set(tw, W.view(torch.int16).numpy())
        gr.set(tx, x.numpy())
        gr.compute()
        yb = gr.get(out).reshape(M, N)
    finally:
        gr.close()
    need = L.mmhip_mul_mat_workspace(30, N, K, M)
    ws = torch.empty(need, dtype=torch.uint8, device="cuda")
    y = torch.empty((M, N), device="cuda")
    Q = lambda t: ctypes.c_void_p(t.data_ptr())
    tw_, tx_ = W.cuda(), x.cuda()
    assert L.mmhip_mul_mat(30, Q(tw_), N, K, K * 2, Q(tx_), K, M, Q(y), N, Q(ws), need, None) == 0
    torch.cuda.synchronize()
    assert np.array_equal(yb, y.cpu().numpy())


@pytest.mark.parametrize("N,K,M", [(4096, 12288, 2), (4096, 4096, 2), (1000, 8192, 1), (6144, 4096, 2),
                                   (30000, 2048, 2), (77, 4096, 1)])
def test_gemv_q6_K_persistent_equals_wave_kernel(mm, pkg, monkeypatch, N, K, M):
    """Q6_K GEMV at 1-2 tokens through the persistent kernel (Q8_K rows in
    LDS, 16-wave workgroups streaming rows) equals the one-wave-per-row-pair
    kernel (GGML_MI355X_DISABLE_Q6_PRO) bit for bit, with and without the
    residual: each lane adds the same units in the same order and the sums
    reduce by the same butterfly.  K = 8192 leaves a third of the lanes
    without a third unit; N from a partial to several row iterations."""
    import ctypes
    L = mm.load()
    W = mm.QuantWeight.from_gguf(14, pkg.synth.gguf_blocks_np(14, N, K, 7), N, K)
    x = torch.from_numpy(pkg.synth.normal_np((M, K), 8)).cuda()
    r = torch.from_numpy(pkg.synth.normal_np((M, N), 9)).cuda()
    xq = torch.zeros(L.mmhip_act_bytes(14, K, M), dtype=torch.uint8, device="cuda")
    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    p = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    assert L.mmhip_quantize_act(14, p(x), K, K, M, p(xq), s) == 0
    outs = []
    for wave_kernel in (False, True):
        if wave_kernel:
            monkeypatch.setenv("GGML_MI355X_DISABLE_Q6_PRO", "1")
        y = torch.full((M, N), float("nan"), device="cuda")
        ya = torch.full((M, N), float("nan"), device="cuda")
        assert L.mmhip_mul_mat_q(14, p(W.data), N, K, W.row_bytes, p(xq), M, p(y), N, s) == 0
        assert L.mmhip_mul_mat_q_add(14, p(W.data), N, K, W.row_bytes, p(xq), M, p(r), N, p(ya), N, s) == 0
        torch.cuda.synchronize()
        outs.append((y, ya))
    monkeypatch.delenv("GGML_MI355X_DISABLE_Q6_PRO")
    assert torch.equal(outs[0][0], outs[1][0])
    assert torch.equal(outs[0][1], outs[1][1])
    assert torch.isfinite(outs[0][0]).all()


@pytest.mark.parametrize("t", [12, 13])
@pytest.mark.parametrize("N,K", [(6144, 4096), (4097, 4096), (37, 8192), (4096, 12288), (5000, 12288), (151, 4096)])
@pytest.mark.parametrize("M", [1, 2])
def test_gemv_q45_persistent(mm, orc, pkg, monkeypatch, t, N, K, M):
    """Q4_K / Q5_K at 1-2 columns and K = 4096 / 8192 / 12288 take the
    persistent kernel (the quantised Q8_K rows copied into LDS once per
    workgroup, 64-element units per lane, two rows in flight at K = 4096):
    within the ggml-semantics oracle's 2e-5, and within 1e-5 of the
    one-wave-per-row-pair kernel (GGML_MI355X_DISABLE_Q45_PRO), which sums in
    another order; ragged N (one to several rows per wave)."""
    raw = pkg.synth.gguf_blocks_np(t, N, K, 7100 + t + K + M)
    x = pkg.synth.normal_np((M, K), 7200 + M)
    W = mm.QuantWeight.from_gguf(t, raw, N, K)
    xt = torch.from_numpy(x).cuda()
    y = mm.mul_mat(W, xt).cpu().numpy()
    monkeypatch.setenv("GGML_MI355X_DISABLE_Q45_PRO", "1")
    yp = mm.mul_mat(W, xt).cpu().numpy()
    monkeypatch.delenv("GGML_MI355X_DISABLE_Q45_PRO")
    yg = orc.mul_mat_ggml(t, raw, N, K, x)
    assert rel_err(y, yg) < 2e-5
    assert rel_err(y, yp) < 1e-5
    assert np.isfinite(y).all()


@pytest.mark.parametrize("t,N,K,M,kind", [(12, 6144, 2048, 2048, "plain"), (8, 2048, 2048, 2100, "plain"),
                                          (14, 3000, 2048, 2051, "bias_res"), (8, 2048, 8192, 2200, "bias_res"),
                                          (12, 1024, 2048, 2077, "swiglu"), (8, 16384, 2048, 2048, "swiglu"),
                                          (8, 512, 2048, 2049, "plain"), (13, 4096, 2048, 2048, "plain"),
                                          (13, 1024, 2048, 2077, "swiglu")])
def test_gemm_f16_weight_copy_equals_register_path(mm, pkg, monkeypatch, t, N, K, M, kind):
    """At 2048+ tokens the GEMM first writes the weights to f16 rows
    (k_w_to_f16, the in-kernel dequantisation's arithmetic) and streams both
    tiles by DMA through a 4-stage ring; the MFMAs run in the same k order, so
    the output equals the register-staged kernel's (GGML_MI355X_DISABLE_GEMM_WH)
    bit for bit: plain, with bias + residual (K = 8192 also takes split-K),
    and with the SwiGLU epilogue; ragged N and M tails; 256 x 256 tiles and
    (few tiles) 64 x 128 tiles."""
    import ctypes

    L = mm.load()
    raw = pkg.synth.gguf_blocks_np(t, N, K, 5100 + t)
    W = mm.QuantWeight.from_gguf(t, raw, N, K)
    x = torch.from_numpy(pkg.synth.normal_np((M, K), 5200 + t)).cuda()
    b = torch.randn(N, device="cuda")
    r = torch.randn(M, N, device="cuda")
    P = lambda a: ctypes.c_void_p(a.data_ptr()) if a is not None else None  # noqa: E731
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    outs = []
    for reg in (False, True):
        if reg:
            monkeypatch.setenv("GGML_MI355X_DISABLE_GEMM_WH", "1")
        need = L.mmhip_mul_mat_workspace(t, N, K, M)
        ws = torch.empty(max(need, 256), dtype=torch.uint8, device="cuda")
        if kind == "swiglu":
            h = torch.full((M, N // 2), float("nan"), device="cuda")
            hh = torch.zeros((M, N // 2), dtype=torch.float16, device="cuda")
            rc = L.mmhip_mul_mat_bias_swiglu(t, P(W.data), N, K, W.row_bytes, P(x), K, M, P(b), 0, P(h), P(hh),
                                             P(ws), need, st)
            out = (h, hh)
        else:
            y = torch.full((M, N), float("nan"), device="cuda")
            rc = L.mmhip_mul_mat_bias_add(t, P(W.data), N, K, W.row_bytes, P(x), K, M,
                                          P(b) if kind == "bias_res" else None, P(r) if kind == "bias_res" else None,
                                          N, P(y), N, P(ws), need, st)
            out = (y,)
        assert rc == 0, L.mmhip_last_error()
        torch.cuda.synchronize()
        outs.append(out)
    monkeypatch.delenv("GGML_MI355X_DISABLE_GEMM_WH")
    for a, c in zip(outs[0], outs[1]):
        assert torch.equal(a, c)
    assert torch.isfinite(outs[0][0]).all()


@pytest.mark.parametrize("N,K", [(6144, 4096), (4096, 6144), (2048, 1024), (37, 256), (1000, 4096), (4106, 2048)])
@pytest.mark.parametrize("M", [3, 4, 7, 9, 16])
def test_gemv_q8_0_int8_mfma_columns(mm, orc, pkg, N, K, M):
    """Q8_0 at 3..16 activation columns (the int8-MFMA GEMV: 16-row groups,
    K split over the waves by block pairs, each block's int32 sum scaled as
    ggml scales it): the depth decoder's projection shapes, a row count that
    is not a multiple of 16 (last group partial, 10 of 16 rows), one-chunk
    and uneven K splits, against the ggml-semantics and float64 oracles."""
    y, yg, yf = run(mm, orc, pkg, 8, N, K, M, 7000 + N + K + M)
    assert rel_err(y, yg) < 2e-5
    assert cosine(y, yf) > 0.9999


@pytest.mark.parametrize("N,K,T,B,pad", [(2304, 2304, 689, 2, 0), (128, 128, 689, 2, 0), (100, 96, 45, 1, 0),
                                         (64, 256, 32, 1, 8), (257, 512, 70, 3, 4)])
def test_mul_mat_f32_weights_at_token_counts(mm, N, K, T, B, pad):
    """F32 weight rows against f32 activations at >= 32 tokens (the DiT's
    k = 1 convs, src/dit.h:258 and :285, stored F32 by the quantiser): the f32
    MFMA GEMM, 3-D activations collapsed to K x (T*B), partial 64-row / 64-token
    tiles, and weight rows `pad` floats longer than K (a view).  Tolerance:
    max|y - y64| <= 1e-5 * max|y64| against float64 (f32 products, f32 sums)."""
    L = mm.load()
    g = torch.Generator().manual_seed(N + K + T)
    wfull = torch.randn((N, K + pad), generator=g) / np.sqrt(K)
    x = torch.randn((B, T, K), generator=g)
    tw = wfull.cuda()[:, :K]                                  # ggml [K, N], row stride K + pad
    tx = x.cuda()                                             # ggml [K, T, B]
    out = torch.full((B, T, N), float("nan"), device="cuda")  # ggml [N, T, B]
    va, vb = mm.view_of(tw), mm.view_of(tx)
    assert L.mmhip_mul_mat_f32(ctypes.byref(va), ctypes.byref(vb), ctypes.c_void_p(out.data_ptr()),
                               ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)) == 0, L.mmhip_last_error()
    ref = x.double() @ wfull[:, :K].double().T
    y = out.cpu().double()
    assert torch.isfinite(y).all()
    assert float((y - ref).abs().max() / ref.abs().max()) < 1e-5


def _bf16_rows(rng, N, K):
    """bf16 weight rows (uint16) ~ N(0, 0.02) and their exact f32 values."""
    import lm_reference

    w = lm_reference.round_bf16((0.02 * rng.standard_normal((N, K))).astype(np.float32))
    return (w.view(np.uint32) >> 16).astype(np.uint16), w


@pytest.mark.parametrize("N,K,M,mode", [(6144, 4096, 2, "norm"), (24576, 4096, 2, "norm_glu"), (4096, 12288, 2, "add"),
                                        (4096, 4096, 1, "add"), (1000, 4096, 2, "plain"), (1030, 8192, 1, "norm"),
                                        (24576, 4096, 1, "norm_glu"), (6, 4096, 2, "norm_glu")])
def test_bf16_decode_gemv(mm, N, K, M, mode):
    """The persistent BF16 decode GEMV (mmhip_mul_mat_bf16_dec) at the LM's
    projection shapes: RMS-norm prologue (QKV, gate_up), SwiGLU pairs (gate_up),
    residual ADD (O, down).  Against float64 of the same bf16 operands (weights
    exact, activations rounded to bf16 after the norm, as ggml's BF16 MUL_MAT
    rounds its src1): max|y - y64| <= 1e-5 max|y64| (f32 sums); the
    residual / SwiGLU epilogues restated from the f64 dot products."""
    import lm_reference

    L = mm.load()
    assert L.mmhip_mul_mat_bf16_dec_supported(N, 2048, M, 0) == 0  # K % 4096 != 0: the plain BF16 GEMV's shapes
    assert L.mmhip_mul_mat_bf16_dec_supported(N, K, 3, 0) == 0
    rng = np.random.default_rng(N + K + M)
    Wb, Wf = _bf16_rows(rng, N, K)
    x = rng.standard_normal((M, K)).astype(np.float32)
    nw = (1.0 + 0.05 * rng.standard_normal(K)).astype(np.float32)
    r = rng.standard_normal((M, N)).astype(np.float32)
    eps = 1e-6
    norm = mode.startswith("norm")
    glu = mode.endswith("glu")
    if norm:
        x64 = x.astype(np.float64)
        sc = (1.0 / np.sqrt(np.float32((x64 * x64).mean(axis=1)) + np.float32(eps))).astype(np.float32)
        xa = (x * sc[:, None]).astype(np.float32) * nw
    else:
        xa = x
    xa = lm_reference.round_bf16(xa).astype(np.float64)
    d = xa @ Wf.astype(np.float64).T                          # [M, N]
    if glu:
        g, u = d[:, :N // 2], d[:, N // 2:]
        ref = g / (1.0 + np.exp(-g)) * u
    elif mode == "add":
        ref = r.astype(np.float64) + d
    else:
        ref = d
    tW, tx, tn, tr = (torch.from_numpy(a).cuda() for a in (Wb.view(np.int16), x, nw, r))
    nout = N // 2 if glu else N
    y = torch.full((M, nout), float("nan"), device="cuda")
    P = lambda t: ctypes.c_void_p(t.data_ptr())
    assert L.mmhip_mul_mat_bf16_dec_supported(N, K, M, int(glu)) == 1
    rc = L.mmhip_mul_mat_bf16_dec(P(tW), N, K, K, P(tx), K, M, P(tn) if norm else None, eps,
                                  P(tr) if mode == "add" else None, N, int(glu), P(y), nout,
                                  ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert rc == 0, L.mmhip_last_error()
    out = y.cpu().numpy().astype(np.float64)
    assert np.isfinite(out).all()
    scale = np.abs(d).max() if mode == "add" else np.abs(ref).max()
    assert np.abs(out - ref).max() <= 1e-5 * max(scale, np.abs(ref).max() * 1e-2), np.abs(out - ref).max() / scale
