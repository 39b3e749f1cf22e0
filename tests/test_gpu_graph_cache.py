"""GPU: the backend's graph cache and teardown.

- Several graphs alternate on one backend, as the reference's frame loop
  alternates the depth decoder's frame graph and the LM's decode graph on one
  shared backend (src/pipeline.cpp:458, :545-547; src/backend.h:21-23): both
  are captured on their second sight and replayed from then on, with results
  bit-identical to a backend that runs every graph eagerly.
- A graph rebuilt at the same addresses with different op_params (the depth
  decoder rebuilds its frame graph when cfg changes, src/depth-decoder.h:
  439-447) is not served by the stale capture.
- A backend is created, captures, replays and is freed three times in one
  process with bit-identical results (teardown order: the stream drains, the
  captures go, then the buffers).
"""
import ctypes
import importlib
import os
import struct

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

SMALL_LM = dict(n_layers=2, hidden=256, n_heads=4, n_kv_heads=2, head_dim=64, ffn=512, vocab=1000, max_seq=768,
                n_sets=2, wtype=8, rms_eps=1e-6, rope_theta=1e6)
DIM, FF, NH, HD = 512, 768, 2, 256


@pytest.fixture(scope="module")
def mods(pkg, mm):
    return (importlib.import_module(pkg.__name__ + ".opgraph"), importlib.import_module(pkg.__name__ + ".depthgraph"),
            importlib.import_module(pkg.__name__ + ".lm"))


def _eager_backend(og):
    """A backend that never captures (GGML_MI355X_DISABLE_GRAPHS is read at init)."""
    _, MI = og._load()
    os.environ["GGML_MI355X_DISABLE_GRAPHS"] = "1"
    try:
        b = MI.ggml_backend_mi355x_init(0)
    finally:
        del os.environ["GGML_MI355X_DISABLE_GRAPHS"]
    assert b
    return b


def _depth_graph(og, dg, backend, S, B, w):
    g = og.OpGraph(n_tensors=200, backend=backend)
    lw = dg.Layer(g, dim=DIM, ff=FF)
    tx = g.tensor(og.F32, [DIM, S, B])
    out = dg.build_layer(g, lw, tx, S, B, n_heads=NH, head_dim=HD)
    g.build([out])
    lw.upload(g, w)
    return g, tx, out


def _run_frames(og, dg, lmmod, backend, frames=5):
    """Alternate a depth-layer graph and the LM decode graph on `backend`."""
    S, B = 4, 2
    w = dg.synth_layer(7, dim=DIM, ff=FF)
    g, tx, out = _depth_graph(og, dg, backend, S, B, w)
    lm = lmmod.Lm(seed=9, backend=backend, **SMALL_LM)
    lm.fill_kv(0, 300, seed=21)
    lm.fill_kv(1, 287, seed=22)
    rng = np.random.default_rng(5)
    x = rng.standard_normal((B, S, DIM)).astype(np.float32)
    depth_out, logits = [], []
    try:
        for _ in range(frames):
            g.set(tx, x)
            g.compute()
            depth_out.append(g.get(out))
            emb = rng.standard_normal((2, SMALL_LM["hidden"])).astype(np.float32)
            lg, _ = lm.decode(emb, [0, 1])
            logits.append(lg)
        stats = g.graph_stats()
        info = g.graph_cache_info()
    finally:
        lm.close()
        g.close()
    return depth_out, logits, stats, info


def test_alternating_graphs_replay_on_one_backend(mods):
    og, dg, lmmod = mods
    _, MI = og._load()
    G, _ = og._load()
    shared = MI.ggml_backend_mi355x_init(0)
    eager = _eager_backend(og)
    try:
        d_rep, l_rep, (replays, n_eager), (entries, captured, captures) = _run_frames(og, dg, lmmod, shared)
        d_ref, l_ref, (replays_e, _), _ = _run_frames(og, dg, lmmod, eager)
    finally:
        G.ggml_backend_free(shared)
        G.ggml_backend_free(eager)
    print(f"shared backend: replays {replays}, eager {n_eager}, entries {entries}, captured {captured}, "
          f"captures {captures}")
    # 5 frames x 2 graphs: each graph eager once, captured on its second sight,
    # replayed from then on (the LM's decode graph keeps its addresses)
    assert entries == 2 and captured == 2 and captures == 2
    assert replays == 8 and n_eager == 2
    assert replays_e == 0
    for a, b in zip(d_rep, d_ref):
        assert np.array_equal(a, b)
    for a, b in zip(l_rep, l_ref):
        assert np.array_equal(a, b)
    for a in d_rep[1:]:
        assert np.array_equal(a, d_rep[0])


def _set_f32_param(t, i, v):
    t.contents.op_params[i] = struct.unpack("<i", struct.pack("<f", v))[0]


def test_op_params_change_is_not_replayed(mods):
    """The CFG SCALE of the sampler chain (src/depth-decoder.h:331-338) is
    changed in place after the graph was captured: the next compute must use
    the new scale (a new capture), equal to a fresh graph built with it."""
    og, _, _ = mods
    V, k = 1024, 64
    rng = np.random.default_rng(12)
    logits = (rng.standard_normal((2, V)) * 3).astype(np.float32)

    def build(g, cfg):
        tl = g.tensor(og.F32, [V, 2])
        cond = g.view_1d(tl, V, 0)
        uncond = g.view_1d(tl, V, V * 4)
        sc = g.scale(g.sub(cond, uncond), cfg)
        guided = g.add(uncond, sc)
        idxk = g.cont(g.argsort_top_k(guided, k))
        g.build([guided, idxk])
        g.set(tl, logits)
        return sc, guided, idxk

    def expect(cfg):
        gd = logits[1] + (logits[0] - logits[1]) * np.float32(cfg)
        return gd, np.lexsort((np.arange(V), -gd))[:k].astype(np.int32)

    g = og.OpGraph(n_tensors=64)
    try:
        sc, guided, idxk = build(g, 3.0)
        for _ in range(3):  # eager, capture, replay
            g.compute()
            gd, order = expect(3.0)
            assert np.array_equal(g.get(idxk, np.int32), order)
        _set_f32_param(sc, 0, 1.5)
        for _ in range(3):  # new signature: eager, capture, replay
            g.compute()
            gd, order = expect(1.5)
            assert np.array_equal(g.get(idxk, np.int32), order)
            np.testing.assert_allclose(g.get(guided), gd, rtol=0, atol=1e-5)
        replays, n_eager = g.graph_stats()
        entries, captured, captures = g.graph_cache_info()
    finally:
        g.close()
    assert n_eager == 2 and replays == 4 and entries == 2 and captures == 2


def test_backend_teardown_three_times(mods):
    """Create a backend, build a depth-layer graph, run it eagerly, capture,
    replay twice, free it (backend first), three times in one process."""
    og, dg, _ = mods
    S, B = 8, 1
    w = dg.synth_layer(11, dim=DIM, ff=FF)
    x = np.random.default_rng(3).standard_normal((B, S, DIM)).astype(np.float32)
    outs = []
    for rnd in range(3):
        print(f"teardown round {rnd}", flush=True)
        g, tx, out = _depth_graph(og, dg, None, S, B, w)
        try:
            g.set(tx, x)
            res = []
            for _ in range(4):
                g.compute()
                res.append(g.get(out))
            assert g.graph_stats() == (3, 1)
        finally:
            g.close()
        for r in res[1:]:
            assert np.array_equal(r, res[0])
        outs.append(res[0])
    assert np.array_equal(outs[0], outs[1]) and np.array_equal(outs[0], outs[2])


def test_f16_weight_copies_of_a_repeating_graph(mods, pkg, mm):
    """A graph computed three or more times gets f16 copies of the weights its
    token-count GEMMs multiply (registered with the kernel library, so the
    GEMMs read them through the DMA ring): the results stay bit-identical
    across the eager run, the first capture, the copies' creation with the
    recapture it forces, and replays.  Uploading new weights afterwards
    refreshes the copy in place: the next replay equals the C-ABI product of
    the new weights.  Freeing the graph's buffers frees the copies."""
    og = mods[0]
    N, K, M = 2048, 2048, 300
    g = og.OpGraph()
    before = g.f16_weight_bytes()
    try:
        tw = g.tensor(og.Q8_0, [K, N])
        tx = g.tensor(og.F32, [K, M])
        tb = g.tensor(og.F32, [N])
        out = g.add(g.mul_mat(tw, tx), tb)
        g.build([out])
        raw = pkg.synth.gguf_blocks_np(8, N, K, 7700)
        x = pkg.synth.normal_np((M, K), 7701)
        bias = pkg.synth.normal_np((N,), 7702)
        g.set(tw, raw)
        g.set(tx, x)
        g.set(tb, bias)
        ys = []
        for _ in range(5):
            g.compute()
            ys.append(g.get(out))
        assert all(np.array_equal(y.view(np.int32), ys[0].view(np.int32)) for y in ys)
        assert g.f16_weight_bytes() >= before + N * K * 2
        replays, _ = g.graph_stats()
        assert replays >= 3
        raw2 = pkg.synth.gguf_blocks_np(8, N, K, 7703)
        g.set(tw, raw2)
        g.compute()
        y2 = g.get(out).reshape(M, N)
    finally:
        g.close()
    assert g.f16_weight_bytes() == before
    W2 = mm.QuantWeight.from_gguf(8, raw2, N, K)
    ref = (mm.mul_mat(W2, __import__("torch").from_numpy(x).cuda()) +
           __import__("torch").from_numpy(bias).cuda()).cpu().numpy()
    assert np.array_equal(y2.view(np.int32), ref.view(np.int32))
    assert not np.array_equal(y2.view(np.int32), ys[0].reshape(M, N).view(np.int32))


def test_f16_weight_copies_follow_copy_memset_and_clear(mods, pkg, mm):
    """Every buffer write into a weight that has an f16 copy refreshes the
    copy: ggml_backend_tensor_copy (cpy_tensor) of other weights into it,
    ggml_backend_tensor_memset (zero weights: the GEMM then gives the bias),
    and ggml_backend_buffer_clear of the whole buffer; each next replay equals
    what the written weights give."""
    import torch

    og = mods[0]
    N, K, M = 1024, 2048, 300
    g = og.OpGraph()
    G = g.G
    for n, r, a in [("ggml_backend_tensor_copy", None, [og._T, og._T]),
                    ("ggml_backend_tensor_memset", None, [og._T, ctypes.c_uint8, ctypes.c_size_t, ctypes.c_size_t]),
                    ("ggml_backend_buffer_clear", None, [ctypes.c_void_p, ctypes.c_uint8])]:
        getattr(G, n).restype, getattr(G, n).argtypes = r, a
    try:
        tw = g.tensor(og.Q8_0, [K, N])
        tw2 = g.tensor(og.Q8_0, [K, N])  # the copy's source, not in the graph
        tx = g.tensor(og.F32, [K, M])
        tb = g.tensor(og.F32, [N])
        out = g.add(g.mul_mat(tw, tx), tb)
        g.build([out])
        raw, raw2 = pkg.synth.gguf_blocks_np(8, N, K, 7710), pkg.synth.gguf_blocks_np(8, N, K, 7711)
        x, bias = pkg.synth.normal_np((M, K), 7712), pkg.synth.normal_np((N,), 7713)
        for t, a in ((tw, raw), (tw2, raw2), (tx, x), (tb, bias)):
            g.set(t, a)
        for _ in range(4):
            g.compute()
        y1 = g.get(out).reshape(M, N)
        assert g.f16_weight_bytes() > 0

        def product(r):
            W = mm.QuantWeight.from_gguf(8, r, N, K)
            return (mm.mul_mat(W, torch.from_numpy(x).cuda()) + torch.from_numpy(bias).cuda()).cpu().numpy()

        assert np.array_equal(y1.view(np.int32), product(raw).view(np.int32))
        G.ggml_backend_tensor_copy(tw2, tw)
        g.compute()
        assert np.array_equal(g.get(out).reshape(M, N).view(np.int32), product(raw2).view(np.int32))
        G.ggml_backend_tensor_memset(tw, 0, 0, G.ggml_nbytes(tw))
        g.compute()
        assert np.array_equal(g.get(out).reshape(M, N), np.broadcast_to(bias, (M, N)))
        g.set(tw, raw)
        g.compute()
        assert np.array_equal(g.get(out).reshape(M, N).view(np.int32), y1.view(np.int32))
        G.ggml_backend_buffer_clear(g.buf, 0)
        g.set(tx, x)
        g.set(tb, bias)
        g.compute()
        assert np.array_equal(g.get(out).reshape(M, N), np.broadcast_to(bias, (M, N)))
    finally:
        g.close()
