"""GPU: GGML_OP_FLASH_ATTN_EXT against the oracle.

Tolerances (stated): against the fp64 oracle max-abs <= 2e-3 and cosine >=
0.9999; against the ggml-CPU-semantics oracle (f16 V accumulator) max-abs
<= that oracle's own max-abs distance from fp64 + 1e-3 (the GPU accumulates
in f32, so it sits closer to fp64 than ggml-CPU does)."""
import numpy as np
import pytest
import torch

from conftest import cosine

pytestmark = pytest.mark.gpu


def rnd(shape, seed, dt=np.float32):
    return np.random.default_rng(seed).standard_normal(shape).astype(dt)


def check(out, ref64, refg=None):
    assert np.isfinite(out).all()
    assert np.abs(out - ref64).max() < 2e-3
    assert cosine(out, ref64) > 0.9999
    if refg is not None:
        assert np.abs(out - refg).max() <= np.abs(refg - ref64).max() + 1e-3


def test_decode_benchmark_shape(mm, orc):
    """B=2 (CFG), 32 q heads / 8 KV heads, D=128, KV 2048, no mask."""
    B, Hq, Hkv, D, nkv = 2, 32, 8, 128, 2048
    q = rnd((B, Hq, 1, D), 1001)
    k = rnd((B, Hkv, nkv, D), 1002, np.float16)
    v = rnd((B, Hkv, nkv, D), 1003, np.float16)
    s = float(np.float32(1 / np.sqrt(D)))
    out = mm.flash_attn_ext(torch.from_numpy(q).cuda(), torch.from_numpy(k).cuda(), torch.from_numpy(v).cuda(),
                            None, s).cpu().numpy()
    check(out, orc.flash_attn_ext(q, k, v, None, s, "f64"), orc.flash_attn_ext(q, k, v, None, s, "ggml"))


def test_decode_real_cache_views_and_mask(mm, orc):
    """The batched decode of src/qwen3-lm.h:793-821: K/V are windows of the 4-D
    f16 cache [D, max_seq, Nkv, sets] (n_kv_pad = 2304 of max_seq 4096), the
    mask is [n_kv_pad, 1, 1, 2] with -inf past each set's kv_len."""
    D, Hq, Hkv, sets, max_seq, pad = 128, 32, 8, 2, 4096, 2304
    kv_len = [2049, 2111]
    cache_k = torch.from_numpy(rnd((sets, Hkv, max_seq, D), 11, np.float16)).cuda()
    cache_v = torch.from_numpy(rnd((sets, Hkv, max_seq, D), 12, np.float16)).cuda()
    kw, vw = cache_k[:, :, :pad], cache_v[:, :, :pad]  # strided windows of the cache
    q = rnd((sets, Hq, 1, D), 13)
    mask = np.zeros((sets, 1, 1, pad), np.float16)
    for i, L in enumerate(kv_len):
        mask[i, ..., L:] = -np.inf
    s = float(np.float32(1 / np.sqrt(D)))
    out = mm.flash_attn_ext(torch.from_numpy(q).cuda(), kw, vw, torch.from_numpy(mask).cuda(), s).cpu().numpy()
    kn, vn = kw.cpu().numpy(), vw.cpu().numpy()
    check(out, orc.flash_attn_ext(q, kn, vn, mask, s, "f64"), orc.flash_attn_ext(q, kn, vn, mask, s, "ggml"))


@pytest.mark.parametrize("B,Bk,Hq,Hkv,nq,nkv,D", [
    (1, 1, 4, 4, 1, 1, 64), (2, 1, 8, 2, 3, 333, 64), (1, 1, 2, 1, 2, 1000, 256), (2, 2, 16, 16, 1, 77, 128),
    (1, 1, 32, 8, 4, 129, 128)])
def test_decode_shapes(mm, orc, B, Bk, Hq, Hkv, nq, nkv, D):
    q = rnd((B, Hq, nq, D), 21)
    k = rnd((Bk, Hkv, nkv, D), 22, np.float16)
    v = rnd((Bk, Hkv, nkv, D), 23, np.float16)
    mask = np.where(np.random.default_rng(24).random((1, 1, nq, nkv)) < 0.2, -np.inf, 0).astype(np.float16)
    s = float(np.float32(1 / np.sqrt(D)))  # the graphs' scale, src/qwen3-lm.h:785, src/dit.h:216
    out = mm.flash_attn_ext(torch.from_numpy(q).cuda(), torch.from_numpy(k).cuda(), torch.from_numpy(v).cuda(),
                            torch.from_numpy(mask).cuda(), s).cpu().numpy()
    check(out, orc.flash_attn_ext(q, k, v, mask, s, "f64"), orc.flash_attn_ext(q, k, v, mask, s, "ggml"))


def test_decode_sharp_softmax(mm, orc):
    """A larger scale sharpens the softmax; Q rounded to f16 (ggml's Q->f16
    conversion) then dominates the error: bounded by 5e-3 against fp64."""
    q = rnd((1, 8, 2, 128), 25)
    k = rnd((1, 2, 500, 128), 26, np.float16)
    v = rnd((1, 2, 500, 128), 27, np.float16)
    out = mm.flash_attn_ext(torch.from_numpy(q).cuda(), torch.from_numpy(k).cuda(), torch.from_numpy(v).cuda(),
                            None, 0.3).cpu().numpy()
    ref = orc.flash_attn_ext(q, k, v, None, 0.3, "f64")
    assert np.abs(out - ref).max() < 5e-3 and cosine(out, ref) > 0.9999
    # the f16 V accumulator of the ggml-semantics oracle drifts further from
    # fp64 than the f32 accumulation here: bound by its own error + 2e-3
    refg = orc.flash_attn_ext(q, k, v, None, 0.3, "ggml")
    assert np.abs(out - refg).max() < np.abs(refg - ref).max() + 2e-3


def test_fully_masked_rows_are_zero(mm):
    q = torch.randn((1, 4, 2, 128), device="cuda")
    k = torch.randn((1, 1, 64, 128), device="cuda").half()
    mask = torch.zeros((1, 1, 2, 64), device="cuda").half()
    mask[0, 0, 1] = float("-inf")
    out = mm.flash_attn_ext(q, k, k, mask, 0.1)
    assert torch.all(out[0, 1] == 0) and torch.all(torch.isfinite(out))


def test_permuted_query_view(mm, orc):
    """Q as the permuted view the graphs pass (src/qwen3-lm.h:401,
    src/dit.h:212): stored [B, S, H, D], viewed as ggml [D, S, H, B]."""
    B, S, H, D = 2, 3, 4, 64
    qs = rnd((B, S, H, D), 31)
    k = rnd((B, H, 50, D), 32, np.float16)
    v = rnd((B, H, 50, D), 33, np.float16)
    qt = torch.from_numpy(qs).cuda()
    qview = mm.view_of(qt, ne=[D, S, H, B], nb=[4, H * D * 4, D * 4, S * H * D * 4])
    out = mm.flash_attn_ext(qt, torch.from_numpy(k).cuda(), torch.from_numpy(v).cuda(), None, 0.125,
                            q_view=qview).cpu().numpy()
    qn = np.ascontiguousarray(qs.transpose(0, 2, 1, 3))  # [B, H, S, D]
    check(out, orc.flash_attn_ext(qn, k, v, None, 0.125, "f64"))


# ---------------------------------------------------------------------------
# many query rows: the MFMA kernel (causal prefill, DiT bidirectional)

def oracle_rows(orc, q, k, v, mask, scale, rows, flavour="f64"):
    """Oracle on a subset of query rows (q [B, Hq, nq, D]); returns [B, len, Hq, D]."""
    qs = np.ascontiguousarray(q[:, :, rows])
    ms = None if mask is None else np.ascontiguousarray(mask[:, :, rows])
    return orc.flash_attn_ext(qs, k, v, ms, scale, flavour)


def test_dit_real_shape_permuted_views(mm, orc):
    """DiT attention at its real shape (src/dit.h:54-55, T = 689 + 1): 32 heads
    x 64 dims, 690 tokens, B = 2, no mask.  Q is the permuted view of the
    [D, Nh, S, B] projection (src/dit.h:212); K/V are the contiguous f16 casts
    (src/dit.h:219-220)."""
    B, S, H, D = 2, 690, 32, 64
    qst = rnd((B, S, H, D), 41)                      # ggml [D, H, S, B]
    k = rnd((B, H, S, D), 42, np.float16)            # ggml [D, S, H, B]
    v = rnd((B, H, S, D), 43, np.float16)
    s = float(np.float32(1 / np.sqrt(D)))
    qt = torch.from_numpy(qst).cuda()
    qview = mm.view_of(qt, ne=[D, S, H, B], nb=[4, H * D * 4, D * 4, S * H * D * 4])
    out = mm.flash_attn_ext(qt, torch.from_numpy(k).cuda(), torch.from_numpy(v).cuda(), None, s,
                            q_view=qview).cpu().numpy()
    qn = np.ascontiguousarray(qst.transpose(0, 2, 1, 3))
    check(out, orc.flash_attn_ext(qn, k, v, None, s, "f64"))


def test_dit_benchmark_shape_sampled(mm, orc):
    """B=2, 4096 latent tokens, 16 heads x 128, no mask; Q drawn N(0,1) and
    rounded to f16 (passed as f32).  Checked on 48 sampled query rows."""
    B, S, H, D = 2, 4096, 16, 128
    q = rnd((B, H, S, D), 1004).astype(np.float16).astype(np.float32)
    k = rnd((B, H, S, D), 1005, np.float16)
    v = rnd((B, H, S, D), 1006, np.float16)
    s = float(np.float32(1 / np.sqrt(D)))
    out = mm.flash_attn_ext(torch.from_numpy(q).cuda(), torch.from_numpy(k).cuda(), torch.from_numpy(v).cuda(),
                            None, s).cpu().numpy()
    rows = np.array([0, 1, 127, 128, 129, 1000, 2047, 2048, 3071, 4094, 4095] +
                    list(np.random.default_rng(7).choice(4096, 37, replace=False)))
    ref = oracle_rows(orc, q, k, v, None, s, rows)
    check(out[:, rows], ref)


def causal_mask(S, n_kv):
    m = np.full((S, n_kv), -np.inf, np.float32)
    for i in range(S):
        m[i, : i + 1] = 0
    return m.astype(np.float16)[None, None]


def test_causal_prefill_benchmark_shape_sampled(mm, orc):
    """B=2 (CFG), 1024 tokens, 32 q / 8 KV heads, D=128, causal f16 mask."""
    B, S, Hq, Hkv, D = 2, 1024, 32, 8, 128
    q = rnd((B, Hq, S, D), 1003).astype(np.float16).astype(np.float32)
    k = rnd((B, Hkv, S, D), 1013, np.float16)
    v = rnd((B, Hkv, S, D), 1023, np.float16)
    mask = causal_mask(S, S)
    s = float(np.float32(1 / np.sqrt(D)))
    out = mm.flash_attn_ext(torch.from_numpy(q).cuda(), torch.from_numpy(k).cuda(), torch.from_numpy(v).cuda(),
                            torch.from_numpy(mask).cuda(), s).cpu().numpy()
    rows = np.array([0, 1, 2, 63, 64, 127, 128, 129, 511, 512, 700, 1022, 1023])
    ref = oracle_rows(orc, q, k, v, mask, s, rows)
    check(out[:, rows], ref, oracle_rows(orc, q, k, v, mask, s, rows, "ggml"))


def test_lm_prefill_real_path(mm, orc):
    """qw3lm_build_attn (src/qwen3-lm.h:346-443): Q is the permuted view of
    [D, Nh, S]; K/V are [0, n_kv_pad) windows of the [D, max_seq, Nkv] f16
    cache; the mask is [n_kv_pad, S] with -inf above the diagonal and on the
    padded tail."""
    S, Hq, Hkv, D, max_seq, pad = 200, 32, 8, 128, 1024, 256
    qst = rnd((S, Hq, D), 51)                               # ggml [D, Nh, S]
    cache_k = torch.from_numpy(rnd((Hkv, max_seq, D), 52, np.float16)).cuda()
    cache_v = torch.from_numpy(rnd((Hkv, max_seq, D), 53, np.float16)).cuda()
    kw, vw = cache_k[:, :pad], cache_v[:, :pad]
    mask = causal_mask(S, pad)
    s = float(np.float32(1 / np.sqrt(D)))
    qt = torch.from_numpy(qst).cuda()
    qview = mm.view_of(qt, ne=[D, S, Hq, 1], nb=[4, Hq * D * 4, D * 4, S * Hq * D * 4])
    out = mm.flash_attn_ext(qt, kw, vw, torch.from_numpy(mask).cuda(), s, q_view=qview).cpu().numpy()
    qn = np.ascontiguousarray(qst.transpose(1, 0, 2))[None]
    kn, vn = kw.cpu().numpy()[None], vw.cpu().numpy()[None]
    check(out, orc.flash_attn_ext(qn, kn, vn, mask, s, "f64"), orc.flash_attn_ext(qn, kn, vn, mask, s, "ggml"))


@pytest.mark.parametrize("B,Bk,Hq,Hkv,nq,nkv,D", [(2, 1, 8, 2, 130, 77, 64), (1, 1, 4, 1, 257, 300, 128),
                                                 (2, 2, 2, 2, 33, 1, 128), (1, 1, 16, 16, 64, 640, 64)])
def test_mfma_odd_shapes_with_mask(mm, orc, B, Bk, Hq, Hkv, nq, nkv, D):
    q = rnd((B, Hq, nq, D), 61)
    k = rnd((Bk, Hkv, nkv, D), 62, np.float16)
    v = rnd((Bk, Hkv, nkv, D), 63, np.float16)
    rng = np.random.default_rng(64)
    mask = np.where(rng.random((B, 1, nq, nkv + 3)) < 0.3, -np.inf, rng.normal(0, 1, (B, 1, nq, nkv + 3)))
    mask[:, :, 5] = -np.inf  # a fully masked query row -> 0
    mask = mask.astype(np.float16)
    s = float(np.float32(1 / np.sqrt(D)))
    out = mm.flash_attn_ext(torch.from_numpy(q).cuda(), torch.from_numpy(k).cuda(), torch.from_numpy(v).cuda(),
                            torch.from_numpy(mask).cuda(), s).cpu().numpy()
    mk = np.ascontiguousarray(mask)
    check(out, orc.flash_attn_ext(q, k, v, mk, s, "f64"))
    assert not out[:, 5].any()


@pytest.mark.parametrize("B,Bk,Hq,Hkv,nq,nkv,D", [(2, 1, 8, 2, 130, 77, 64), (1, 1, 4, 1, 257, 300, 128),
                                                 (2, 2, 2, 2, 33, 1, 128), (1, 1, 16, 16, 64, 640, 64),
                                                 (1, 1, 8, 2, 96, 31, 128), (1, 1, 2, 2, 40, 33, 64)])
def test_mfma_odd_shapes_no_mask(mm, orc, B, Bk, Hq, Hkv, nq, nkv, D):
    """Unmasked attention (the DiT path) with partial key tiles (nkv % 32 != 0),
    a single key, GQA and both head sizes."""
    q = rnd((B, Hq, nq, D), 71)
    k = rnd((Bk, Hkv, nkv, D), 72, np.float16)
    v = rnd((Bk, Hkv, nkv, D), 73, np.float16)
    s = float(np.float32(1 / np.sqrt(D)))
    out = mm.flash_attn_ext(torch.from_numpy(q).cuda(), torch.from_numpy(k).cuda(), torch.from_numpy(v).cuda(),
                            None, s).cpu().numpy()
    check(out, orc.flash_attn_ext(q, k, v, None, s, "f64"))


@pytest.mark.parametrize("B,Bk,Hq,Hkv,nq,nkv", [(1, 1, 64, 8, 1000, 333), (2, 1, 32, 32, 1100, 97),
                                              (1, 1, 64, 64, 1024, 1)])
def test_dma_kernel_shapes(mm, orc, B, Bk, Hq, Hkv, nq, nkv):
    """Unmasked D = 128 on at least 256 workgroups of 256 query rows, the
    shapes that take the DMA-fed kernel: GQA, a broadcast K/V batch, a partial
    last query tile, partial 32-key units and 64-key tiles, a single key."""
    q = rnd((B, Hq, nq, 128), 81)
    k = rnd((Bk, Hkv, nkv, 128), 82, np.float16)
    v = rnd((Bk, Hkv, nkv, 128), 83, np.float16)
    s = float(np.float32(1 / np.sqrt(128)))
    out = mm.flash_attn_ext(torch.from_numpy(q).cuda(), torch.from_numpy(k).cuda(), torch.from_numpy(v).cuda(),
                            None, s).cpu().numpy()
    check(out, orc.flash_attn_ext(q, k, v, None, s, "f64"))


def test_dma_kernel_running_max_moves(mm, orc):
    """K rows grow with the key index (x0.25 at the first key to x3.25 at the
    last), so the row max keeps rising along the sequence and the running max
    is moved (O and l rescaled) many times.  48 sampled rows against fp64."""
    B, S, H, D = 2, 2048, 16, 128
    q = rnd((B, H, S, D), 91)
    grow = (0.25 + 3.0 * np.arange(S) / S).astype(np.float32)[None, None, :, None]
    k = (rnd((B, H, S, D), 92) * grow).astype(np.float16)
    v = rnd((B, H, S, D), 93, np.float16)
    s = float(np.float32(1 / np.sqrt(D)))
    out = mm.flash_attn_ext(torch.from_numpy(q).cuda(), torch.from_numpy(k).cuda(), torch.from_numpy(v).cuda(),
                            None, s).cpu().numpy()
    rows = np.array([0, 1, 255, 256, 1023, 2046, 2047] + list(np.random.default_rng(9).choice(S, 41, replace=False)))
    ref = oracle_rows(orc, q, k, v, None, s, rows)
    assert np.isfinite(out).all()
    # a sharp softmax: Q's f16 rounding dominates, as in the decode sharp case
    assert np.abs(out[:, rows] - ref).max() < 5e-3 and cosine(out[:, rows], ref) > 0.9999


@pytest.mark.parametrize("wt", [8, 14])
def test_decode_with_quantised_output(mm, orc, wt):
    """mmhip_flash_attn_ext_q (the attention feeding the output projection,
    src/qwen3-lm.h:816-826): the output matches the oracle, and its quantised
    copy is byte-identical to quantize_act of that output."""
    import ctypes

    L = mm.load()
    D, Hq, Hkv, sets, max_seq, pad = 128, 32, 8, 2, 4096, 2304
    kv_len = [2049, 2111]
    cache_k = torch.from_numpy(rnd((sets, Hkv, max_seq, D), 31, np.float16)).cuda()
    cache_v = torch.from_numpy(rnd((sets, Hkv, max_seq, D), 32, np.float16)).cuda()
    kw, vw = cache_k[:, :, :pad], cache_v[:, :, :pad]
    q = rnd((sets, Hq, 1, D), 33)
    mask = np.zeros((sets, 1, 1, pad), np.float16)
    for i, n in enumerate(kv_len):
        mask[i, ..., n:] = -np.inf
    s = float(np.float32(1 / np.sqrt(D)))
    tq, tm = torch.from_numpy(q).cuda(), torch.from_numpy(mask).cuda()
    qv, kv, vv, mv = mm.view_of(tq), mm.view_of(kw), mm.view_of(vw), mm.view_of(tm)
    out = torch.empty((sets, 1, Hq, D), dtype=torch.float32, device="cuda")
    need = L.mmhip_flash_attn_workspace(ctypes.byref(qv), ctypes.byref(kv), ctypes.byref(vv))
    ws = torch.empty(max(need, 1), dtype=torch.uint8, device="cuda")
    K, M = Hq * D, sets
    xq = torch.zeros(L.mmhip_act_bytes(wt, K, M), dtype=torch.uint8, device="cuda")
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    assert L.mmhip_flash_attn_ext_q(ctypes.byref(qv), ctypes.byref(kv), ctypes.byref(vv), ctypes.byref(mv), s,
                                    ctypes.c_void_p(out.data_ptr()), ctypes.c_void_p(ws.data_ptr()), need, wt,
                                    ctypes.c_void_p(xq.data_ptr()), st) == 0
    ref_q = torch.zeros_like(xq)
    assert L.mmhip_quantize_act(wt, ctypes.c_void_p(out.data_ptr()), K, K, M, ctypes.c_void_p(ref_q.data_ptr()),
                                st) == 0
    torch.cuda.synchronize()
    assert torch.equal(xq, ref_q)
    kn, vn = kw.cpu().numpy(), vw.cpu().numpy()
    check(out.cpu().numpy(), orc.flash_attn_ext(q, kn, vn, mask, s, "f64"), orc.flash_attn_ext(q, kn, vn, mask, s, "ggml"))


@pytest.mark.parametrize("B,Bk,Hq,Hkv,nq,nkv,kind", [(1, 1, 64, 8, 1000, 1100, "random"),
                                                   (2, 2, 32, 8, 1100, 1300, "causal"),
                                                   (2, 1, 64, 64, 257, 333, "random"),
                                                   (1, 1, 256, 32, 130, 130, "causal"),
                                                   (1, 1, 64, 8, 1000, 1000, "prefix")])
def test_dma_kernel_masked(mm, orc, B, Bk, Hq, Hkv, nq, nkv, kind):
    """Masked D = 128 on >= 256 workgroups: the DMA-fed kernel with the mask
    prepass's row ends, one 128-row query tile per workgroup (the longest
    first), waves that stop before the workgroup's last staged key, the mask
    added past each wave's all-zero prefix.  Random masks (-inf, biases, a
    fully masked row -> 0), causal masks behind a 170-key visible prefix, and
    a 100-key prefix for every row (every workgroup stages two tiles); 48
    sampled rows against fp64."""
    q = rnd((B, Hq, nq, 128), 111)
    k = rnd((Bk, Hkv, nkv, 128), 112, np.float16)
    v = rnd((Bk, Hkv, nkv, 128), 113, np.float16)
    rng = np.random.default_rng(114)
    if kind == "random":
        mask = np.where(rng.random((B, 1, nq, nkv)) < 0.3, -np.inf, rng.normal(0, 1, (B, 1, nq, nkv)))
        mask[:, :, 5] = -np.inf
    elif kind == "prefix":
        mask = np.full((1, 1, nq, nkv), -np.inf)
        mask[..., :100] = 0
    else:
        off = nkv - nq if nkv > nq else 0
        mask = np.full((1, 1, nq, nkv), -np.inf)
        for i in range(nq):
            mask[0, 0, i, :off + i + 1] = 0
    mask = mask.astype(np.float16)
    s = float(np.float32(1 / np.sqrt(128)))
    out = mm.flash_attn_ext(torch.from_numpy(q).cuda(), torch.from_numpy(k).cuda(), torch.from_numpy(v).cuda(),
                            torch.from_numpy(mask).cuda(), s).cpu().numpy()
    rows = np.unique(np.array([0, 1, 5, 31, 32, 127, 128, nq // 2, nq - 2, nq - 1] +
                              list(rng.choice(nq, 38, replace=False))))
    check(out[:, rows], oracle_rows(orc, q, k, v, mask, s, rows))
    if kind == "random":
        assert not out[:, 5].any()


def test_replay_prefill_9000_tokens(mm, orc):
    """The replay prefill (src/pipeline.cpp:288, one qw3lm_forward over up to
    9000 feedback frames; qw3lm_build_attn, src/qwen3-lm.h:346-443) for one
    CFG set: Q the permuted view of [D, Nh, S], K / V the [0, n_kv_pad = 9216)
    windows of the [D, max_seq, Nkv] f16 cache, the [n_kv_pad, S] f16 causal
    mask with its -inf padded tail (166 MB).  32 sampled rows against fp64."""
    S, Hq, Hkv, D, max_seq, pad = 9000, 32, 8, 128, 9472, 9216
    qst = rnd((S, Hq, D), 121)                                       # ggml [D, Nh, S]
    cache_k = torch.from_numpy(rnd((Hkv, max_seq, D), 122, np.float16)).cuda()
    cache_v = torch.from_numpy(rnd((Hkv, max_seq, D), 123, np.float16)).cuda()
    kw, vw = cache_k[:, :pad], cache_v[:, :pad]
    mask = np.triu(np.full((S, pad), -np.inf, np.float32), 1).astype(np.float16)[None, None]
    s = float(np.float32(1 / np.sqrt(D)))
    qt = torch.from_numpy(qst).cuda()
    qview = mm.view_of(qt, ne=[D, S, Hq, 1], nb=[4, Hq * D * 4, D * 4, S * Hq * D * 4])
    out = mm.flash_attn_ext(qt, kw, vw, torch.from_numpy(mask).cuda(), s, q_view=qview).cpu().numpy()
    rows = np.unique(np.array([0, 1, 127, 128, 4499, 4500, 8191, 8999] +
                              list(np.random.default_rng(124).choice(S, 24, replace=False))))
    qn = np.ascontiguousarray(qst.transpose(1, 0, 2))[None]
    kn, vn = kw.cpu().numpy()[None], vw.cpu().numpy()[None]
    check(out[:, rows], oracle_rows(orc, qn, kn, vn, mask, s, rows))
