"""Pins the oracle's mul_mat flavours (oracle/oracle.c)."""
import numpy as np
import pytest

from conftest import cosine, rel_err
from test_oracle_formats import np_decode

TYPES = [8, 12, 13, 14]


@pytest.mark.parametrize("t", TYPES)
def test_mul_mat_f64_vs_numpy(orc, pkg, t):
    N, K, M = 37, 512, 3
    raw = pkg.synth.gguf_blocks_np(t, N, K, 200 + t)
    x = pkg.synth.normal_np((M, K), 201)
    W = np_decode(t, raw, K).reshape(N, K).astype(np.float64)
    ref = x.astype(np.float64) @ W.T
    got = orc.mul_mat_f64(t, raw, N, K, x)
    assert rel_err(got, ref) < 1e-12


@pytest.mark.parametrize("t", TYPES)
def test_mul_mat_ggml_exact_when_activations_representable(orc, pkg, t):
    """When every activation block is exactly representable in the activation
    format (power-of-two scale, max |q| = 127), the ggml flavour is exact up to
    f32 rounding of the block sums."""
    N, K, M = 23, 1024, 2
    raw = pkg.synth.gguf_blocks_np(t, N, K, 300 + t)
    rng = np.random.default_rng(301)
    blk = 32 if t == 8 else 256
    q = rng.integers(-126, 127, size=(M, K // blk, blk))
    q[:, :, 0] = -127
    e = rng.integers(0, 6, size=(M, K // blk, 1))
    x = (q * 2.0 ** -e).reshape(M, K).astype(np.float32)
    got = orc.mul_mat_ggml(t, raw, N, K, x)
    ref = orc.mul_mat_f64(t, raw, N, K, x)
    assert rel_err(got, ref) < 2e-6


@pytest.mark.parametrize("t", TYPES)
def test_mul_mat_ggml_error_vs_f64(orc, pkg, t):
    N, K, M = 64, 4096, 2
    raw = pkg.synth.gguf_blocks_np(t, N, K, 400 + t)
    x = pkg.synth.normal_np((M, K), 401)
    got = orc.mul_mat_ggml(t, raw, N, K, x)
    ref = orc.mul_mat_f64(t, raw, N, K, x)
    # activation quantisation error of ggml-CPU itself
    assert cosine(got, ref) > 0.9999
    assert rel_err(got, ref) < 3e-2


@pytest.mark.parametrize("t", TYPES)
def test_mul_mat_one_hot_and_row_swap(orc, pkg, t):
    N, K = 16, 512
    raw = pkg.synth.gguf_blocks_np(t, N, K, 500 + t)
    W = orc.dequantize(t, raw, K, N)
    x = np.zeros((2, K), np.float32)
    # one-hot values 127 * 2^-k quantise exactly (q = +-127, d = 2^-k)
    x[0, 77] = 127.0 / 64
    x[1, 300] = -127.0 / 32
    y = orc.mul_mat_ggml(t, raw, N, K, x)
    np.testing.assert_allclose(y[0], W[:, 77] * (127.0 / 64), rtol=1e-6, atol=0)
    np.testing.assert_allclose(y[1], W[:, 300] * (-127.0 / 32), rtol=1e-6, atol=0)
    ys = orc.mul_mat_ggml(t, raw, N, K, x[::-1].copy())
    assert np.array_equal(ys, y[::-1])
    # linearity of the exact flavour
    a = pkg.synth.normal_np((1, K), 502)
    b = pkg.synth.normal_np((1, K), 503)
    lin = orc.mul_mat_f64(t, raw, N, K, (a + b).astype(np.float32))
    sep = orc.mul_mat_f64(t, raw, N, K, a) + orc.mul_mat_f64(t, raw, N, K, b)
    assert rel_err(lin, sep) < 1e-6


def test_vec_dot_zero_blocks(orc, pkg):
    K = 256
    for t in TYPES:
        raw = np.zeros(orc.row_size(t, K), np.uint8)
        x = pkg.synth.normal_np((1, K), 600)
        assert np.all(orc.mul_mat_ggml(t, raw, 1, K, x) == 0)
