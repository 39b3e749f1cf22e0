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


# (weight type, bumped type): Q8_0, Q6_K, Q4_K, and Q5_K_M (Q5_K with the
# V / down projections of the bumped layers in Q6_K, tools/quantize.cpp:47-48)
WTYPES = [(8, 0), (14, 0), (12, 0), (13, 14)]


@pytest.mark.parametrize("wtype,bump", WTYPES, ids=["q8_0", "q6_k", "q4_k", "q5_k_m"])
def test_lm_decode_matches_reference(lmmod, wtype, bump):
    import lm_reference

    lm = lmmod.Lm(seed=5 + wtype, wtype=wtype, bump_type=bump, **SMALL)
    if bump:
        # two layers: layer 0 is bumped (l % 3 == 0), layer 1 is not
        assert lm.type_of("blk.0.v") == bump and lm.type_of("blk.0.down") == bump
        assert lm.type_of("blk.0.qk") == wtype and lm.type_of("blk.0.qkv") is None
        assert lm.type_of("blk.1.qkv") == wtype and lm.type_of("blk.1.down") == wtype
    lm.fill_kv(0, 300, seed=21)
    lm.fill_kv(1, 287, seed=22)
    st = lm_reference.LmState(lm)
    st64 = lm_reference.LmState(lm)
    kv_pos = {0: 300, 1: 287}
    rng = np.random.default_rng(wtype)
    err_dev = err_ref = 0.0
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
            err_dev += 1 - cosine(lg[r], el[r])
            err_ref += 1 - cosine(rl[r], el[r])
        assert lm.pos(0) == kv_pos[0] and lm.pos(1) == kv_pos[1]
    # as close to the exact result as ggml-CPU's arithmetic is, over the 8
    # logits rows together: a single row moves either way by the few int8
    # activation codes that round differently once the layers' f32 inputs
    # differ in their last bits (chained, not teacher-forced)
    print(f"logits 1 - cosine vs exact, summed: device {err_dev:.3e}, ggml-ref {err_ref:.3e}", flush=True)
    assert err_dev <= 1.5 * err_ref + 1e-6
    replays, eager = lm.graph_stats()
    assert eager == 1 and replays == 3, (replays, eager)
    # the device KV cache received this step's rows at the right positions
    _check_kv_rows(lm, st, SMALL, {0: (300, 304), 1: (287, 291)})
    lm.close()


def _check_kv_rows(lm, st, cfg, written, teacher_forced=False):
    """The device caches equal the reference's.  Every layer: rows the steps
    did not write byte for byte.  Layer 0, and every layer of a teacher-forced
    reference (inputs identical to the reference's): the written rows at
    least 95 % byte-equal, the rest within
    one f16 ulp or, for elements near zero, 1e-4 of the row's largest
    magnitude (they come out of the QKV GEMV, whose f32 block sums differ from
    the reference's in order before the f16 rounding).  Later layers: within
    2e-2 of the row's largest magnitude (their inputs carry the earlier
    layers' differences, and one step of the activation quantisation is 1/127
    of a block's largest value)."""
    shp = (cfg["n_sets"], cfg["n_kv_heads"], cfg["max_seq"], cfg["head_dim"])
    for layer in range(cfg["n_layers"]):
        for name, ref in ((f"kv_k4_{layer}", st.k[layer]), (f"kv_v4_{layer}", st.v[layer])):
            dev = lm.get(name, np.float16).reshape(shp)
            for s, (p0, p1) in written.items():
                a, b = dev[s, :, p0:p1].astype(np.float32), ref[s, :, p0:p1].astype(np.float32)
                err = np.abs(a - b)
                if layer == 0 or teacher_forced:
                    ulp = np.spacing(np.abs(b).astype(np.float16)).astype(np.float32)
                    tol = np.maximum(ulp, 1e-4 * np.abs(b).max(axis=-1, keepdims=True))
                    assert (err <= tol).all(), (name, s, float(err.max()))
                    same = dev[s, :, p0:p1].view(np.uint16) == ref[s, :, p0:p1].view(np.uint16)
                    assert same.mean() >= 0.95, (name, s, float(same.mean()))
                else:
                    assert (err <= 2e-2 * np.abs(b).max(axis=-1, keepdims=True)).all(), (name, s, float(err.max()))
                assert np.array_equal(dev[s, :, :p0].view(np.uint16), ref[s, :, :p0].view(np.uint16)), (name, s)
                assert np.array_equal(dev[s, :, p1:].view(np.uint16), ref[s, :, p1:].view(np.uint16)), (name, s)


@pytest.mark.parametrize("wtype,bump", [(8, 0), (14, 0), (30, 0), (13, 14)], ids=["q8_0", "q6_k", "bf16", "q5_k_m"])
def test_lm_decode_headline_width_matches_reference(lmmod, wtype, bump):
    """Oracle parity at the Qwen3-8B width of the decode benchmark: hidden
    4096, 32 / 8 heads of 128, FFN 12288, vocab 151936, f16 KV caches of 4096
    positions on both CFG sets (Q8_0, and the Q6_K variant), 2 layers of the
    36 (every layer runs the same kernels), for the eager step and the
    captured one; and with BF16 weights (type 30, the native-BF16 files: the
    persistent BF16 decode GEMV with the norm, residual and SwiGLU fused);
    and Q5_K_M (layer 0 with a Q6_K V / down projection, layer 1 all Q5_K).

    Stated tolerance, teacher-forced (each layer restated from the device's
    own input rows of that layer and the device's caches, the logits from its
    last layer's rows, so that no earlier difference is carried in): cosine
    >= 0.9999 per layer output and on the logits and final hidden states, and
    equal argmax on both CFG rows.  Chained from the embeddings alone: equal
    argmax, and, summed over the steps' logits rows, at most 1.5x as far from
    exact (f64) arithmetic as the ggml-CPU-semantics restatement is
    (activation codes that round the other way in one layer move the next
    layers' inputs; the chained cosines are printed).  The last step's KV rows
    of every layer against the teacher-forced restatement's, to the first
    layer's bar of _check_kv_rows (identical inputs)."""
    import lm_reference

    cfg = dict(lmmod.QWEN3_8B, n_layers=2, wtype=wtype, bump_type=bump)
    lm = lmmod.Lm(seed=77 + wtype, **cfg)
    lm.fill_kv(0, 4094, seed=31)  # both steps in the 4096-key window
    lm.fill_kv(1, 4093, seed=32)
    st = lm_reference.LmState(lm)
    st64 = lm_reference.LmState(lm)
    stf = lm_reference.LmState(lm)
    kv_pos = {0: 4094, 1: 4093}
    rng = np.random.default_rng(1005 + wtype)
    err_dev = err_ref = 0.0
    for step in range(2):
        print(f"headline-width decode wtype {wtype} step {step}", flush=True)
        emb = rng.standard_normal((2, cfg["hidden"])).astype(np.float32)
        stf.refresh_kv(lm)
        lg, hid = lm.decode(emb, [0, 1])
        outs = [lm.get(f"layer_out-{l}", np.float32).reshape(2, cfg["hidden"]) for l in range(cfg["n_layers"])]
        tl, tlg, thid = lm_reference.decode_teacher_forced(stf, emb, outs, [0, 1], kv_pos, "ggml")
        rl, rh = lm_reference.decode(st, emb, [0, 1], kv_pos, "ggml")
        el, eh = lm_reference.decode(st64, emb, [0, 1], kv_pos, "f64")
        kv_pos = {k: v + 1 for k, v in kv_pos.items()}
        layer_cos = [[cosine(outs[l][r], tl[l][r]) for r in range(2)] for l in range(cfg["n_layers"])]
        tf_cos = [cosine(lg[r], tlg[r]) for r in range(2)]
        print(f"  teacher-forced: layer outputs cosine {layer_cos}, logits cosine {tf_cos}, hidden cosine "
              f"{[cosine(hid[r], thid[r]) for r in range(2)]}", flush=True)
        print(f"  chained: logits cosine {[cosine(lg[r], rl[r]) for r in range(2)]}, hidden cosine "
              f"{[cosine(hid[r], rh[r]) for r in range(2)]}; vs exact {[cosine(lg[r], el[r]) for r in range(2)]}, "
              f"ggml-ref vs exact {[cosine(rl[r], el[r]) for r in range(2)]}", flush=True)
        for r in range(2):
            for l in range(cfg["n_layers"]):
                assert layer_cos[l][r] >= 0.9999, (step, l, r, layer_cos[l][r])
            assert tf_cos[r] >= 0.9999, (step, r, tf_cos[r])
            assert cosine(hid[r], thid[r]) >= 0.9999, (step, r)
            assert np.argmax(lg[r]) == np.argmax(tlg[r]), (step, r)
            assert np.argmax(lg[r]) == np.argmax(rl[r]), (step, r)
            err_dev += 1 - cosine(lg[r], el[r])
            err_ref += 1 - cosine(rl[r], el[r])
    print(f"logits 1 - cosine vs exact, summed: device {err_dev:.3e}, ggml-ref {err_ref:.3e}", flush=True)
    assert err_dev <= 1.5 * err_ref + 1e-6
    replays, eager = lm.graph_stats()
    assert eager == 1 and replays == 1, (replays, eager)
    _check_kv_rows(lm, stf, cfg, {0: (4095, 4096), 1: (4094, 4095)}, teacher_forced=True)
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


@pytest.mark.parametrize("wtype,bump", [(8, 0), (14, 0), (30, 0), (13, 14)], ids=["q8_0", "q6_k", "bf16", "q5_k_m"])
def test_lm_decode_benchmark_shape(lmmod, wtype, bump):
    """The Qwen3-8B-shape decode step (36 layers, Q8_0, the Q6_K variant, BF16
    and Q5_K_M, vocab 151936) at KV 4096 on both CFG sets: finite,
    deterministic, graph replayed."""
    cfg = dict(lmmod.QWEN3_8B, wtype=wtype, bump_type=bump)
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
