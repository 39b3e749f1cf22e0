"""GPU: the ggml-backend boundary.  The MI355X backend registers, stores
quantized weights in its own layout behind set/get_tensor, and runs the LM
batched CFG decode graph of src/qwen3-lm.h:645-934 (built with the ggml API)
through ggml_backend_graph_compute, matching a CPU evaluation of the same op
sequence with the oracle.

Stated tolerance for logits and final hidden states: cosine >= 0.9999
against the ggml-CPU-semantics reference (the GPU differs in its attention
accumulator precision and f32 summation order), argmax equal on both CFG
rows; cosine >= 0.999 against the exact (fp64 matmul / fp64 attention)
reference, which differs by ggml's activation quantisation."""
import numpy as np
import pytest

from conftest import cosine

pytestmark = pytest.mark.gpu

SMALL = dict(n_layers=2, hidden=256, n_heads=4, n_kv_heads=2, head_dim=64, ffn=512, vocab=1000, max_seq=768,
             n_sets=2, rms_eps=1e-6, rope_theta=1e6)


@pytest.fixture(scope="module")
def lmmod(pkg, mm):
    import importlib

    return importlib.import_module(pkg.__name__ + ".lm")


def test_registry_and_weight_roundtrip(lmmod, pkg):
    lm = lmmod.Lm(seed=3, wtype=8, **SMALL)
    raw = lm.get("blk.0.qkv")
    assert raw.size == 256 // 32 * 34 * (4 * 64 + 2 * 2 * 64)
    # host bytes in == host bytes out (row-grouped device layout in between)
    new = pkg.synth.gguf_blocks_np(8, 4 * 64 + 2 * 2 * 64, 256, 11)
    lm.set("blk.0.qkv", new)
    assert np.array_equal(lm.get("blk.0.qkv"), new)
    lm.close()


@pytest.mark.parametrize("wtype", [8, 14, 12])
def test_lm_decode_matches_reference(lmmod, wtype):
    import lm_reference

    lm = lmmod.Lm(seed=5 + wtype, wtype=wtype, **SMALL)
    lm.fill_kv(0, 300, seed=21)
    lm.fill_kv(1, 287, seed=22)
    st = lm_reference.LmState(lm)
    st64 = lm_reference.LmState(lm)
    kv_pos = {0: 300, 1: 287}
    rng = np.random.default_rng(wtype)
    for step in range(4):  # eager, eager, captured, replayed
        emb = rng.standard_normal((2, SMALL["hidden"])).astype(np.float32)
        lg, hid = lm.decode(emb, [0, 1])
        rl, rh = lm_reference.decode(st, emb, [0, 1], kv_pos, "ggml")
        el, eh = lm_reference.decode(st64, emb, [0, 1], kv_pos, "f64")
        kv_pos = {0: kv_pos[0] + 1, 1: kv_pos[1] + 1}
        assert np.isfinite(lg).all()
        print(f"step {step}: logits cos vs ggml-ref {[cosine(lg[r], rl[r]) for r in range(2)]}, "
              f"vs exact {[cosine(lg[r], el[r]) for r in range(2)]}, ggml-ref vs exact "
              f"{[cosine(rl[r], el[r]) for r in range(2)]}; hidden vs ggml-ref {[cosine(hid[r], rh[r]) for r in range(2)]}"
              f", vs exact {[cosine(hid[r], eh[r]) for r in range(2)]}", flush=True)
        for r in range(2):
            assert cosine(lg[r], rl[r]) > 0.9999, (step, r)
            assert cosine(hid[r], rh[r]) > 0.9999, (step, r)
            assert np.argmax(lg[r]) == np.argmax(rl[r])
            # at least as close to the exact result as ggml-CPU's arithmetic is
            assert 1 - cosine(lg[r], el[r]) <= 1.5 * (1 - cosine(rl[r], el[r])) + 1e-6
        assert lm.pos(0) == kv_pos[0] and lm.pos(1) == kv_pos[1]
    replays, eager = lm.graph_stats()
    assert eager == 1 and replays == 3, (replays, eager)
    # the device KV cache received this step's rows at the right positions
    k0 = lm.get("kv_k4_1", np.float16).reshape(2, 2, SMALL["max_seq"], 64)
    assert np.array_equal(k0[0, :, 300:304], st.k[1][0, :, 300:304]) or \
        np.abs(k0[0, :, 300:304].astype(np.float32) - st.k[1][0, :, 300:304].astype(np.float32)).max() < 2e-2
    lm.close()


def test_lm_decode_window_crosses_256(lmmod):
    """kv_len 255 -> 256 -> 257 changes n_kv_pad from 256 to 512: the graph is
    rebuilt (src/qwen3-lm.h:688-693) and results stay consistent."""
    import lm_reference

    lm = lmmod.Lm(seed=9, wtype=8, **SMALL)
    lm.fill_kv(0, 254, seed=1)
    lm.fill_kv(1, 254, seed=2)
    st = lm_reference.LmState(lm)
    kv_pos = {0: 254, 1: 254}
    rng = np.random.default_rng(4)
    for step in range(3):
        emb = rng.standard_normal((2, SMALL["hidden"])).astype(np.float32)
        lg, _ = lm.decode(emb, [0, 1])
        rl, _ = lm_reference.decode(st, emb, [0, 1], kv_pos, "ggml")
        kv_pos = {k: v + 1 for k, v in kv_pos.items()}
        assert min(cosine(lg[r], rl[r]) for r in range(2)) > 0.9999
    lm.close()


def test_lm_decode_benchmark_shape(lmmod):
    """The Qwen3-8B-shape decode step (36 layers, Q8_0, vocab 151936) at KV
    4096 on both CFG sets: finite, deterministic, graph replayed."""
    cfg = dict(lmmod.QWEN3_8B)
    lm = lmmod.Lm(seed=1005, **cfg)
    lm.fill_kv(0, 4095, seed=1)
    lm.fill_kv(1, 4095, seed=2)
    emb = np.random.default_rng(1005).standard_normal((2, cfg["hidden"])).astype(np.float32)
    lg1, h1 = lm.decode(emb, [0, 1])
    assert lm.graph_nodes() > 36 * 20
    assert np.isfinite(lg1).all() and np.isfinite(h1).all()
    for _ in range(3):
        lm.set_pos(0, 4095)
        lm.set_pos(1, 4095)
        lg, h = lm.decode(emb, [0, 1])
        assert np.array_equal(lg, lg1)
    replays, eager = lm.graph_stats()
    assert replays >= 2
    lm.close()
