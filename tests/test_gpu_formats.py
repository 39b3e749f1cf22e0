"""GPU: weight-format kernels (repack / unpack / dequant) and the activation
quantisers are bit-exact with the oracle."""
import json
import pathlib

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu
GOLDEN = pathlib.Path(__file__).resolve().parent / "golden" / "known_blocks.json"


@pytest.mark.parametrize("t", [8, 12, 13, 14])
@pytest.mark.parametrize("N,K", [(37, 512), (5, 4096), (64, 2304)])
def test_repack_roundtrip_and_dequant_bit_exact(mm, orc, pkg, t, N, K):
    raw = pkg.synth.gguf_blocks_np(t, N, K, 1000 + t + K)
    W = mm.QuantWeight.from_gguf(t, raw, N, K)
    assert not torch.equal(W.data.cpu(), torch.from_numpy(raw)), "row-grouped layout should differ from GGUF"
    back = W.to_gguf().cpu().numpy()
    assert np.array_equal(back, raw)
    got = W.dequantize().cpu().numpy()
    ref = orc.dequantize(t, raw, K, N)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


def test_known_answer_blocks_on_gpu(mm):
    for b in json.loads(GOLDEN.read_text())["blocks"]:
        raw = np.frombuffer(bytes.fromhex(b["hex"]), dtype=np.uint8).copy()
        W = mm.QuantWeight.from_gguf(b["type"], raw, 1, b["ne0"])
        got = W.dequantize().cpu().numpy()[0]
        exp = np.array(b["expected"], dtype=np.float32)
        assert np.array_equal(got.view(np.uint32), exp.view(np.uint32)), b["name"]


@pytest.mark.parametrize("t", [8, 12])
def test_activation_quantisers_bit_exact(mm, orc, pkg, t):
    M, K = 3, 2048
    x = pkg.synth.normal_np((M, K), 1100 + t) * np.array([[1.0], [1e-3], [300.0]], np.float32)
    x[1, :256] = 0.0  # an all-zero block / super-block
    x[2, 5] = -x[2].__abs__().max() * 1.5  # negative extreme
    buf = mm.quantize_act(t, torch.from_numpy(x).cuda()).cpu().numpy()
    L = mm.load()
    if t == 8:
        qs = buf[: M * K].view(np.int8).reshape(M, K)
        d_off = (M * K + 255) // 256 * 256
        d = buf[d_off: d_off + 4 * M * K // 32].view(np.float32).reshape(M, K // 32)
        for m in range(M):
            ref = orc.quantize_q8_0(x[m]).reshape(-1, 34)
            assert np.array_equal(qs[m].reshape(-1, 32), ref[:, 2:].view(np.int8))
            assert np.array_equal(d[m], ref[:, 0:2].copy().view(np.float16).astype(np.float32).ravel())
    else:
        qs = buf[: M * K].view(np.int8).reshape(M, K)
        d_off = (M * K + 255) // 256 * 256
        d = buf[d_off: d_off + 4 * M * K // 256].view(np.float32).reshape(M, K // 256)
        b_off = (d_off + 4 * M * K // 256 + 255) // 256 * 256
        bs = buf[b_off: b_off + 2 * M * K // 16].view(np.int16).reshape(M, K // 16)
        for m in range(M):
            ref = orc.quantize_q8_K(x[m]).reshape(-1, 292)
            assert np.array_equal(qs[m].reshape(-1, 256), ref[:, 4:260].view(np.int8))
            assert np.array_equal(d[m], ref[:, 0:4].copy().view(np.float32).ravel())
            assert np.array_equal(bs[m], ref[:, 260:].copy().view(np.int16).ravel())
    assert L.mmhip_act_bytes(t, K, M) == buf.size
