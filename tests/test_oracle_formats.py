"""Pins the oracle's scalar conversions, block decoders and activation
quantisers (oracle/oracle.c) against independent checks."""
import json
import pathlib

import numpy as np
import pytest

GOLDEN = pathlib.Path(__file__).resolve().parent / "golden" / "known_blocks.json"


def test_fp16_to_fp32_exhaustive(orc):
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = orc.fp16_bits_to_fp32(h)
    ref = h.view(np.float16).astype(np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def test_fp32_to_fp16_matches_ieee_rne(orc):
    rng = np.random.default_rng(7)
    bits = rng.integers(0, 2**32, size=1 << 20, dtype=np.uint64).astype(np.uint32)
    x = bits.view(np.float32)
    # add edge cases: ties, overflow boundary, subnormal boundaries, signed zero
    edges = np.array([0.0, -0.0, 65504.0, 65519.99, 65520.0, 1e9, -1e9, 6.1035156e-05, 6.0975552e-05,
                      2.9802322e-08, 2.9802326e-08, 5.9604645e-08, 1.0 + 2**-11, 1.0 + 3 * 2**-11,
                      np.inf, -np.inf], dtype=np.float32)
    x = np.concatenate([x, edges, (np.arange(-70000, 70000, 0.37)).astype(np.float32)])
    got = orc.fp32_to_fp16_bits(x)
    with np.errstate(over="ignore"):
        ref = x.astype(np.float16)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got.view(np.float16)), nan)
    assert np.array_equal(got[~nan], ref.view(np.uint16)[~nan])


def test_bf16_rounding_matches_torch(orc):
    import torch

    rng = np.random.default_rng(8)
    x = rng.standard_normal(4096).astype(np.float32) * 1e3
    got = np.array([orc.lib().orc_fp32_to_bf16(float(v)) for v in x], dtype=np.uint16)
    ref = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got, ref)


def test_known_answer_blocks(orc):
    data = json.loads(GOLDEN.read_text())
    assert len(data["blocks"]) >= 8
    for b in data["blocks"]:
        raw = np.frombuffer(bytes.fromhex(b["hex"]), dtype=np.uint8)
        got = orc.dequantize(b["type"], raw, b["ne0"])[0]
        exp = np.array(b["expected"], dtype=np.float32)
        assert np.array_equal(got.view(np.uint32), exp.view(np.uint32)), b["name"]


# --- an independent vectorised decoder written from the format description ---
def np_decode(t, raw, ne0):
    raw = raw.reshape(-1)
    if t == 8:
        blk = raw.reshape(-1, 34)
        d = blk[:, 0:2].copy().view(np.float16).astype(np.float32)
        q = blk[:, 2:].view(np.int8).astype(np.float32)
        return (d * q).reshape(-1)
    if t in (12, 13):
        blk = raw.reshape(-1, 144 if t == 12 else 176)
        d = blk[:, 0:2].copy().view(np.float16).astype(np.float32)
        dmin = blk[:, 2:4].copy().view(np.float16).astype(np.float32)
        s = blk[:, 4:16].astype(np.int32)
        qs = blk[:, 16:].astype(np.int32) if t == 12 else blk[:, 48:].astype(np.int32)
        sc = np.zeros((blk.shape[0], 8), np.int32)
        mn = np.zeros((blk.shape[0], 8), np.int32)
        sc[:, :4] = s[:, 0:4] & 63
        mn[:, :4] = s[:, 4:8] & 63
        sc[:, 4:] = (s[:, 8:12] & 15) | ((s[:, 0:4] >> 6) << 4)
        mn[:, 4:] = (s[:, 8:12] >> 4) | ((s[:, 4:8] >> 6) << 4)
        q = np.zeros((blk.shape[0], 256), np.int32)
        for c in range(4):
            q[:, 64 * c: 64 * c + 32] = qs[:, 32 * c: 32 * c + 32] & 15
            q[:, 64 * c + 32: 64 * c + 64] = qs[:, 32 * c: 32 * c + 32] >> 4
        if t == 13:
            # fifth bit of element e: bit e // 32 of qh[e % 32]
            qh = blk[:, 16:48].astype(np.int32)
            e = np.arange(256)
            q |= ((qh[:, e % 32] >> (e // 32)) & 1) << 4
        j = np.arange(256) // 32
        d1 = (d * sc[:, j].astype(np.float32)).astype(np.float32)
        m1 = (dmin * mn[:, j].astype(np.float32)).astype(np.float32)
        return ((d1 * q.astype(np.float32)).astype(np.float32) - m1).reshape(-1)
    if t == 14:
        blk = raw.reshape(-1, 210)
        ql = blk[:, 0:128].astype(np.int32)
        qh = blk[:, 128:192].astype(np.int32)
        sc = blk[:, 192:208].view(np.int8).astype(np.float32)
        d = blk[:, 208:210].copy().view(np.float16).astype(np.float32)
        q = np.zeros((blk.shape[0], 256), np.int32)
        for h in range(2):
            for t in range(4):
                lo_src = ql[:, 64 * h + 32 * (t & 1): 64 * h + 32 * (t & 1) + 32]
                lo = (lo_src & 15) if t < 2 else (lo_src >> 4)
                hi = (qh[:, 32 * h: 32 * h + 32] >> (2 * t)) & 3
                q[:, 128 * h + 32 * t: 128 * h + 32 * t + 32] = lo | (hi << 4)
        ds = (d * sc[:, np.arange(256) // 16]).astype(np.float32)
        return (ds * (q - 32).astype(np.float32)).reshape(-1)
    raise ValueError(t)


@pytest.mark.parametrize("t", [8, 12, 13, 14])
def test_dequant_vs_independent_decoder(orc, pkg, t):
    K, N = 1024, 9
    raw = pkg.synth.gguf_blocks_np(t, N, K, 100 + t)
    got = orc.dequantize(t, raw, K, N).reshape(-1)
    ref = np_decode(t, raw, K)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


def _q8_0_fields(buf):
    blk = buf.reshape(-1, 34)
    return blk[:, 0:2].copy().view(np.float16).astype(np.float32).ravel(), blk[:, 2:].view(np.int8)


def _q8_K_fields(buf):
    blk = buf.reshape(-1, 292)
    d = blk[:, 0:4].copy().view(np.float32).ravel()
    qs = blk[:, 4:260].view(np.int8)
    bs = blk[:, 260:292].copy().view(np.int16)
    return d, qs, bs


def test_quantize_q8_0_closed_forms(orc):
    rng = np.random.default_rng(3)
    # exactly representable: q in [-127,127] with |q|max = 127, d = 2^-k
    q = rng.integers(-127, 128, size=(64, 32))
    q[:, 5] = 127 * np.where(rng.random(64) < 0.5, 1, -1)
    k = rng.integers(0, 10, size=(64, 1))
    x = (q * (2.0 ** -k)).astype(np.float32)
    d, qs = _q8_0_fields(orc.quantize_q8_0(x))
    assert np.array_equal(qs, q.astype(np.int8))
    assert np.array_equal(d, (2.0 ** -k).ravel().astype(np.float32))
    # zero block
    d, qs = _q8_0_fields(orc.quantize_q8_0(np.zeros(32, np.float32)))
    assert d[0] == 0 and not qs.any()
    # general: q = round(x / d32); the stored d is f16(d32), so
    # |x - d16*q| <= d/2 + 127*|d16 - d32| <= d * (1/2 + 127 * 2^-11)
    x = rng.standard_normal(32 * 100).astype(np.float32)
    d, qs = _q8_0_fields(orc.quantize_q8_0(x))
    err = np.abs(x.reshape(-1, 32) - d[:, None] * qs)
    assert (err <= d[:, None] * (0.5 + 127 * 2.0**-11) * 1.001).all()
    amax = np.abs(x.reshape(-1, 32)).max(axis=1)
    assert (np.abs(qs).max(axis=1) == 127).all() and np.allclose(d, amax / 127, rtol=2**-11)


def test_quantize_q8_K_closed_forms(orc):
    rng = np.random.default_rng(4)
    x = rng.standard_normal(256 * 20).astype(np.float32)
    d, qs, bs = _q8_K_fields(orc.quantize_q8_K(x))
    xb = x.reshape(-1, 256)
    imax = np.abs(xb).argmax(axis=1)
    assert (qs[np.arange(20), imax] == -127).all()
    assert np.array_equal(bs, qs.astype(np.int32).reshape(-1, 16, 16).sum(-1).astype(np.int16))
    assert (np.abs(xb - d[:, None] * qs) <= np.abs(d)[:, None] * 0.5001).all()
    # exactly representable with a negative extreme
    q = rng.integers(-126, 127, size=(4, 256))
    q[:, 17] = -127
    x = (q * 2.0 ** -3).astype(np.float32)
    d, qs, bs = _q8_K_fields(orc.quantize_q8_K(x))
    assert np.array_equal(qs, q.astype(np.int8)) and np.all(d == 0.125)
    d, qs, bs = _q8_K_fields(orc.quantize_q8_K(np.zeros(256, np.float32)))
    assert d[0] == 0 and not qs.any() and not bs.any()


def test_lm_reference_round_bf16_matches_the_oracle(orc):
    """tests/lm_reference.round_bf16 (numpy, used by the BF16 restatement)
    equals the oracle's f32 -> bf16 conversion, ties and near-ties included."""
    import lm_reference

    rng = np.random.default_rng(5)
    u = rng.integers(0, 1 << 31, 4000, dtype=np.uint64).astype(np.uint32)
    u[:1000] = (u[:1000] & 0xFFFF0000) | 0x8000          # exact ties
    u[1000:1500] = (u[1000:1500] & 0xFFFF0000) | 0x7FFF  # just below a tie
    u = u[(u & 0x7F800000) != 0x7F800000]                # finite values
    x = u.view(np.float32)
    got = lm_reference.round_bf16(x).view(np.uint32) >> 16
    exp = np.array([orc.lib().orc_fp32_to_bf16(float(v)) for v in x], dtype=np.uint32)
    assert np.array_equal(got, exp)
