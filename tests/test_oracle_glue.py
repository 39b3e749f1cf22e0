"""Pin the oracle's glue restatements (oracle.c orc_rms_norm_mul,
orc_layer_norm, orc_rope_neox, orc_swiglu) against closed forms and numpy
float64 forms written independently of oracle.c.  Each check is chosen so a
plausible slip fails it: a dropped eps, an n-1 divisor, mean(x) for mean(x^2),
GPT-J pairing for NeoX pairing, a flipped rotation sign, silu on the wrong
half."""
import numpy as np
import pytest


def _f64_rms(x, w, eps):
    x = x.astype(np.float64)
    y = x / np.sqrt((x * x).mean(-1, keepdims=True) + eps)
    return y * w if w is not None else y


def _f64_layer(x, eps):
    x = x.astype(np.float64)
    v = x - x.mean(-1, keepdims=True)
    return v / np.sqrt((v * v).mean(-1, keepdims=True) + eps)


def test_rms_norm_closed_forms(orc):
    # constant row c: y = c / sqrt(c^2 + eps)
    for c, eps in ((1.0, 1.0), (3.0, 1e-6), (-2.0, 0.5)):
        y = orc.rms_norm_mul(np.full((1, 64), c, np.float32), None, eps)
        assert np.allclose(y, c / np.sqrt(c * c + eps), rtol=1e-6, atol=0)
    # alternating +-a: mean(x^2) = a^2 (a mean(x) slip gives 0)
    x = np.tile(np.array([2.0, -2.0], np.float32), 128)[None]
    y = orc.rms_norm_mul(x, None, 0.0)
    assert np.array_equal(y, np.sign(x))
    # weight multiplies element-wise after the normalisation
    w = np.arange(1, 257, dtype=np.float32) / 256
    yw = orc.rms_norm_mul(x, w, 0.0)
    assert np.allclose(yw, np.sign(x) * w, rtol=1e-7, atol=0)
    # one non-zero element in n: y = sqrt(n) exactly (n divisor, not n-1)
    e = np.zeros((1, 256), np.float32)
    e[0, 17] = 5.0
    assert abs(orc.rms_norm_mul(e, None, 0.0)[0, 17] - 16.0) < 1e-5


def test_rms_norm_vs_f64(orc):
    rng = np.random.default_rng(11)
    x = (rng.standard_normal((6, 4096)) * rng.uniform(0.01, 100, (6, 1))).astype(np.float32)
    w = (1 + 0.1 * rng.standard_normal(4096)).astype(np.float32)
    for ww in (None, w):
        y = orc.rms_norm_mul(x, ww, 1e-6)
        ref = _f64_rms(x, ww, 1e-6)
        assert np.abs(y - ref).max() / np.abs(ref).max() < 1e-6


def test_layer_norm_closed_forms(orc):
    # constant row: v = 0 everywhere
    y = orc.layer_norm(np.full((2, 128), 7.25, np.float32), 1e-6)
    assert np.array_equal(y, np.zeros_like(y))
    # alternating +-a around an offset m: y = +-a / sqrt(a^2 + eps)
    a, m, eps = 3.0, 40.0, 1e-6
    x = (m + a * np.tile(np.array([1.0, -1.0]), 64)).astype(np.float32)[None]
    y = orc.layer_norm(x, eps)
    assert np.allclose(y, np.tile([1.0, -1.0], 64) * a / np.sqrt(a * a + eps), rtol=1e-6, atol=0)
    # eps enters under the root: a = 1, eps = 3 gives +-1/2
    x1 = np.tile(np.array([1.0, -1.0], np.float32), 8)[None]
    assert np.allclose(orc.layer_norm(x1, 3.0), x1 / 2, rtol=1e-7, atol=0)
    # one non-zero element in n (mean x/n, variance x^2 (n-1)/n^2):
    # y_k = sqrt(n-1) for the element, -1/sqrt(n-1) for the rest
    n = 65
    e = np.zeros((1, n), np.float32)
    e[0, 3] = 2.0
    y = orc.layer_norm(e, 0.0)[0]
    assert abs(y[3] - np.sqrt(n - 1)) < 1e-5
    assert np.allclose(np.delete(y, 3), -1 / np.sqrt(n - 1), rtol=1e-5, atol=0)


def test_layer_norm_invariances_and_f64(orc):
    rng = np.random.default_rng(12)
    x = rng.standard_normal((4, 2048)).astype(np.float32)
    y = orc.layer_norm(x, 1e-6)
    # shift and positive scale invariance (eps small against the variance)
    assert np.abs(orc.layer_norm(x + np.float32(5.0), 1e-6) - y).max() < 1e-5
    assert np.abs(orc.layer_norm(x * np.float32(4.0), 1e-6) - y).max() < 1e-5
    # zero mean, unit variance per row
    assert np.abs(y.astype(np.float64).mean(-1)).max() < 1e-6
    assert np.abs((y.astype(np.float64) ** 2).mean(-1) - 1).max() < 1e-5
    xs = (rng.standard_normal((3, 1536)) * 30 + 100).astype(np.float32)
    assert np.abs(orc.layer_norm(xs, 1e-6) - _f64_layer(xs, 1e-6)).max() < 2e-5


def _f64_rope(x, pos, n_dims, base):
    """Direct NeoX form: pair (i, i + n_dims/2) rotates by pos * base^(-2i/n_dims)."""
    x = x.astype(np.float64)
    y = x.copy()
    half = n_dims // 2
    inv = base ** (-2.0 * np.arange(half) / n_dims)
    ang = pos.astype(np.float64)[:, None, None] * inv[None, None, :]
    c, s = np.cos(ang), np.sin(ang)
    x0, x1 = x[..., :half], x[..., half:n_dims]
    y[..., :half] = x0 * c - x1 * s
    y[..., half:n_dims] = x0 * s + x1 * c
    return y


@pytest.mark.parametrize("D,n_dims,base", [(128, 128, 1e6), (64, 32, 1e4)])
def test_rope_neox_vs_direct_form(orc, D, n_dims, base):
    rng = np.random.default_rng(13)
    pos = np.array([0, 1, 2, 7, 31, 64, 1000, 4095, 8192], np.int32)
    x = rng.standard_normal((len(pos), 4, D)).astype(np.float32)
    y = orc.rope_neox(x, pos, n_dims, base)
    ref = _f64_rope(x, pos, n_dims, base)
    # the angle theta_i is built by i f32 multiplies: relative error <= (i+1) 2^-23
    half = n_dims // 2
    i = np.arange(half)
    ang = pos.astype(np.float64)[:, None] * base ** (-2.0 * i / n_dims)[None, :]
    dang = ang * (i[None, :] + 2) * 2.0 ** -23 + 1e-6
    amp = np.abs(x.astype(np.float64)[..., :half]) + np.abs(x.astype(np.float64)[..., half:n_dims])
    bound = amp * dang[:, None, :] + 1e-6
    assert np.all(np.abs(y[..., :half] - ref[..., :half]) <= bound)
    assert np.all(np.abs(y[..., half:n_dims] - ref[..., half:n_dims]) <= bound)
    # small positions: within 1e-5 absolute
    small = pos <= 64
    assert np.abs(y[small] - ref[small]).max() < 1e-5
    # pos 0 is the identity; the tail past n_dims is copied
    assert np.array_equal(y[0], x[0])
    assert np.array_equal(y[..., n_dims:], x[..., n_dims:])


def test_rope_neox_rotation_properties(orc):
    rng = np.random.default_rng(14)
    D = 64
    q = rng.standard_normal((1, 1, D)).astype(np.float32)
    k = rng.standard_normal((1, 1, D)).astype(np.float32)
    # pair norms are preserved
    y = orc.rope_neox(q, np.array([123], np.int32), D, 1e4)
    n0 = q[0, 0, :32] ** 2 + q[0, 0, 32:] ** 2
    n1 = y[0, 0, :32] ** 2 + y[0, 0, 32:] ** 2
    assert np.allclose(n0, n1, rtol=1e-5, atol=1e-6)
    # q.k depends on the position difference only
    dots = []
    for m, n in ((10, 3), (20, 13), (107, 100)):
        qm = orc.rope_neox(q, np.array([m], np.int32), D, 1e4)
        kn = orc.rope_neox(k, np.array([n], np.int32), D, 1e4)
        dots.append(float((qm.astype(np.float64) * kn).sum()))
    assert max(dots) - min(dots) < 1e-4
    # position 1, pair 0 rotates by exactly 1 radian, counter-clockwise
    e = np.zeros((1, 1, D), np.float32)
    e[0, 0, 0] = 1.0
    r = orc.rope_neox(e, np.array([1], np.int32), D, 1e4)
    assert abs(r[0, 0, 0] - np.cos(1.0)) < 1e-7 and abs(r[0, 0, 32] - np.sin(1.0)) < 1e-7


def test_swiglu_closed_forms_and_f64(orc):
    n = 256
    g = np.linspace(-20, 20, n, dtype=np.float32)
    u = np.full(n, 3.0, np.float32)
    y = orc.swiglu(np.concatenate([g, u])[None])[0]
    # gate 0 -> 0; large positive gate -> gate * up; large negative -> 0
    assert np.allclose(y, 3.0 * g.astype(np.float64) / (1 + np.exp(-g.astype(np.float64))), rtol=1e-6, atol=1e-30)
    zero = np.zeros(n, np.float32)
    assert np.array_equal(orc.swiglu(np.concatenate([zero, u])[None])[0], zero)
    # silu acts on the first half only: swapping halves changes the result
    ys = orc.swiglu(np.concatenate([u, g])[None])[0]
    assert not np.allclose(ys, y)
    rng = np.random.default_rng(15)
    x = (rng.standard_normal((5, 2 * 1024)) * 4).astype(np.float32)
    gg, uu = x[:, :1024].astype(np.float64), x[:, 1024:].astype(np.float64)
    ref = gg / (1 + np.exp(-gg)) * uu
    assert np.abs(orc.swiglu(x) - ref).max() < 1e-5 * np.abs(ref).max()
