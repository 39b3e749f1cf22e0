"""Pins the oracle's flash_attn_ext flavours (oracle/oracle.c)."""
import numpy as np
import pytest
import torch

from conftest import cosine


def sdpa_f64(q, k, v, mask):
    """torch scaled_dot_product_attention in float64 on the CPU; q [B,Hq,nq,D],
    k/v [Bk,Hkv,nkv,D]; mask f16 [M3,M2,nq',nkv'] (additive) or None."""
    B, Hq, nq, D = q.shape
    Bk, Hkv, nkv, _ = k.shape
    qt = torch.from_numpy(q.astype(np.float64))
    kt = torch.from_numpy(k.astype(np.float64)).repeat_interleave(Hq // Hkv, dim=1).repeat_interleave(B // Bk, dim=0)
    vt = torch.from_numpy(v.astype(np.float64)).repeat_interleave(Hq // Hkv, dim=1).repeat_interleave(B // Bk, dim=0)
    am = None
    if mask is not None:
        m = torch.from_numpy(mask.astype(np.float64))[:, :, :nq, :nkv]
        am = m.repeat(B // m.shape[0], Hq // m.shape[1], 1, 1)
    # the op's scale is an f32 op_param
    o = torch.nn.functional.scaled_dot_product_attention(qt, kt, vt, attn_mask=am,
                                                         scale=float(np.float32(1.0 / np.sqrt(D))))
    return o.permute(0, 2, 1, 3).numpy()  # [B, nq, Hq, D]


def rnd(shape, seed, dt=np.float32):
    return np.random.default_rng(seed).standard_normal(shape).astype(dt)


@pytest.mark.parametrize("B,Bk,Hq,Hkv,nq,nkv,D", [(2, 2, 8, 2, 1, 300, 128), (1, 1, 4, 4, 5, 64, 64),
                                                 (2, 1, 4, 1, 3, 97, 256)])
def test_f64_matches_torch_sdpa(orc, B, Bk, Hq, Hkv, nq, nkv, D):
    q = rnd((B, Hq, nq, D), 1)
    k = rnd((Bk, Hkv, nkv, D), 2, np.float16)
    v = rnd((Bk, Hkv, nkv, D), 3, np.float16)
    s = 1.0 / np.sqrt(D)
    got = orc.flash_attn_ext(q, k, v, None, s, flavour="f64")
    ref = sdpa_f64(q, k, v, None)
    assert np.abs(got - ref).max() < 1e-12
    # with a random 0/-inf mask (every row keeps key 0)
    mask = np.where(np.random.default_rng(4).random((1, 1, nq, nkv)) < 0.3, -np.inf, 0).astype(np.float16)
    mask[..., 0] = 0
    got = orc.flash_attn_ext(q, k, v, mask, s, flavour="f64")
    ref = sdpa_f64(q, k, v, mask)
    assert np.abs(got - ref).max() < 1e-12


def test_closed_forms(orc):
    D, nkv = 128, 50
    q = rnd((1, 2, 1, D), 5)
    v = rnd((1, 1, nkv, D), 6, np.float16)
    k_const = np.repeat(rnd((1, 1, 1, D), 7, np.float16), nkv, axis=2)
    for fl in ("f64", "ggml"):
        out = orc.flash_attn_ext(q, k_const, v, None, 0.1, flavour=fl)
        np.testing.assert_allclose(out[0, 0, 0], v[0, 0].astype(np.float64).mean(0), atol=2e-3 if fl == "ggml" else 1e-12)
        # a mask that allows one key returns that V row exactly
        mask = np.full((1, 1, 1, nkv), -np.inf, np.float16)
        mask[..., 17] = 0
        out = orc.flash_attn_ext(q, rnd((1, 1, nkv, D), 8, np.float16), v, mask, 0.1, flavour=fl)
        assert np.array_equal(out[0, 0, 1].astype(np.float32), v[0, 0, 17].astype(np.float32))
        # fully masked rows give 0
        out = orc.flash_attn_ext(q, k_const, v, np.full((1, 1, 1, nkv), -np.inf, np.float16), 0.1, flavour=fl)
        assert not out.any()


def test_gqa_map_and_padding_invariance(orc):
    D, nkv = 64, 80
    q = rnd((2, 8, 1, D), 9)
    k = rnd((2, 2, nkv, D), 10, np.float16)
    v = rnd((2, 2, nkv, D), 11, np.float16)
    full = orc.flash_attn_ext(q, k, v, None, 0.125, flavour="f64")
    for h in range(8):
        one = orc.flash_attn_ext(np.ascontiguousarray(q[:, h:h + 1]), np.ascontiguousarray(k[:, h // 4:h // 4 + 1]),
                                 np.ascontiguousarray(v[:, h // 4:h // 4 + 1]), None, 0.125, flavour="f64")
        assert np.abs(one[:, :, 0] - full[:, :, h]).max() < 1e-12
    # padding the cache with masked garbage keys changes nothing (n_kv_pad window)
    pad = 176
    kp = np.concatenate([k, rnd((2, 2, pad - nkv, D), 12, np.float16) * 100], axis=2)
    vp = np.concatenate([v, rnd((2, 2, pad - nkv, D), 13, np.float16) * 100], axis=2)
    mask = np.zeros((2, 1, 1, pad), np.float16)
    mask[..., nkv:] = -np.inf
    for fl in ("f64", "ggml"):
        a = orc.flash_attn_ext(q, k, v, None, 0.125, flavour=fl)
        b = orc.flash_attn_ext(q, kp, vp, mask, 0.125, flavour=fl)
        assert np.array_equal(a, b)


def test_causal_prefix_invariance(orc):
    D, S = 64, 40
    q = rnd((1, 2, S, D), 14)
    k = rnd((1, 2, S, D), 15, np.float16)
    v = rnd((1, 2, S, D), 16, np.float16)
    causal = np.triu(np.full((S, S), -np.inf, np.float32), 1).astype(np.float16)[None, None]
    full = orc.flash_attn_ext(q, k, v, causal, 0.125, flavour="f64")
    for i in (0, 7, 39):
        pre = orc.flash_attn_ext(np.ascontiguousarray(q[:, :, i:i + 1]), np.ascontiguousarray(k[:, :, :i + 1]),
                                 np.ascontiguousarray(v[:, :, :i + 1]), None, 0.125, flavour="f64")
        assert np.abs(pre[:, 0] - full[:, i]).max() < 1e-12


def test_ggml_flavour_error_bound(orc):
    """The f16 V accumulator of ggml-CPU stays within the stated bound of the
    exact result at the decode shape."""
    B, Hq, Hkv, D, nkv = 2, 8, 2, 128, 2048
    q = rnd((B, Hq, 1, D), 17)
    k = rnd((B, Hkv, nkv, D), 18, np.float16)
    v = rnd((B, Hkv, nkv, D), 19, np.float16)
    s = 1.0 / np.sqrt(D)
    g = orc.flash_attn_ext(q, k, v, None, s, flavour="ggml")
    e = orc.flash_attn_ext(q, k, v, None, s, flavour="f64")
    assert np.abs(g - e).max() < 2e-3
    assert cosine(g, e) > 0.9999
