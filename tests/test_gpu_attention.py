"""GPU: GGML_OP_FLASH_ATTN_EXT against the oracle.

Tolerances (stated): against the fp64 oracle max-abs <= 2e-3 and cosine >=
0.9999; against the ggml-CPU-semantics oracle (f16 V accumulator) max-abs
<= 3e-3."""
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
        assert np.abs(out - refg).max() < 3e-3


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
