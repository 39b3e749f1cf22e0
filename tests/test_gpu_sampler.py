"""GPU: the depth decoder's in-graph CFG sampler (src/depth-decoder.h:331-361)
built with the restated ggml API and run through ggml_backend_graph_compute,
plus its ops through the C-ABI.

Expected values come from numpy restatements of the same ops: ARGSORT
descending (equal values in ascending index order) and the integer ops
bit-exact; CUMSUM / SUM / STEP bit-exact on values exactly representable in
f32; the sampler's chosen code exact, with the uniform draws placed away
from every CDF entry (margin 1e-3) so the f32 softmax's last-bit differences
cannot move the pick."""
import ctypes
import importlib

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def st():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def ptr(t):
    return ctypes.c_void_p(t.data_ptr())


def test_argsort_cumsum_sum_step_casts(mm):
    L = mm.load()
    rng = np.random.default_rng(81)
    x = rng.standard_normal((3, 1000)).astype(np.float32)
    x[1, 10:20] = 0.5  # ties: ascending index order
    tx = torch.from_numpy(x).cuda()
    idx = torch.empty((3, 1000), dtype=torch.int32, device="cuda")
    assert L.mmhip_argsort_desc(ctypes.byref(mm.view_of(tx)), ptr(idx), st()) == 0
    ref = np.stack([np.lexsort((np.arange(1000), -r)) for r in x]).astype(np.int32)
    assert np.array_equal(idx.cpu().numpy(), ref)
    # integers and quarters: every partial sum exact in f32
    q = (rng.integers(-40, 41, (4, 37)) / 4).astype(np.float32)
    tq = torch.from_numpy(q).cuda()
    cs = torch.empty_like(tq)
    assert L.mmhip_cumsum(ctypes.byref(mm.view_of(tq)), ptr(cs), st()) == 0
    assert np.array_equal(cs.cpu().numpy(), np.cumsum(q, axis=1, dtype=np.float64).astype(np.float32))
    sm = torch.empty(1, device="cuda")
    assert L.mmhip_sum(ctypes.byref(mm.view_of(tq)), ptr(sm), st()) == 0
    assert sm.item() == float(q.astype(np.float64).sum())
    stp = torch.empty_like(tq)
    assert L.mmhip_step(ctypes.byref(mm.view_of(tq)), ptr(stp), st()) == 0
    assert np.array_equal(stp.cpu().numpy(), (q > 0).astype(np.float32))
    f = torch.tensor([-2.7, -0.5, 0.0, 0.99, 3.5, 49.0], device="cuda")
    i32 = torch.empty(6, dtype=torch.int32, device="cuda")
    assert L.mmhip_cast_i32(ctypes.byref(mm.view_of(f)), ptr(i32), st()) == 0
    assert i32.cpu().tolist() == [-2, 0, 0, 0, 3, 49]
    back = torch.empty(6, device="cuda")
    assert L.mmhip_cast_f32_of_i32(ctypes.byref(mm.view_of(i32)), ptr(back), st()) == 0
    assert back.cpu().tolist() == [-2.0, 0.0, 0.0, 0.0, 3.0, 49.0]
    big = torch.zeros(4097, device="cuda")
    assert L.mmhip_argsort_desc(ctypes.byref(mm.view_of(big)), ptr(idx), st()) != 0


def _sampler_graph(g, og, logits, rand, V, k, cfg, slot):
    """One stream's sampler chain (src/depth-decoder.h:331-358): returns the
    top-k index view (cont) and the chosen code (I32 [1, 1])."""
    cond = g.view_1d(logits, V, 0)
    uncond = g.view_1d(logits, V, V * 4)
    guided_full = g.add(uncond, g.scale(g.sub(cond, uncond), cfg))
    idxk = g.cont(g.argsort_top_k(guided_full, k))
    guided = g.reshape_1d(g.get_rows(g.reshape_2d(guided_full, 1, V), idxk), k)
    cdf = g.cumsum(g.soft_max(guided))
    u = g.view_1d(rand, 1, slot * 4)
    idxf = g.scale_bias(g.sum(g.step(g.sub(cdf, u))), -1.0, float(k))
    pick = g.cast(g.clamp(idxf, 0.0, float(k - 1)), 26)  # GGML_TYPE_I32
    code = g.get_rows(g.reshape_2d(idxk, 1, k), pick)
    code_f = g.get_rows(g.reshape_2d(g.cast(idxk, og.F32), 1, k), pick)
    return idxk, code, code_f


@pytest.mark.parametrize("k,cfg", [(50, 3.0), (1, 1.5), (1024, 2.0)])
def test_sampler_chain_through_backend(pkg, k, cfg):
    og = importlib.import_module(pkg.__name__ + ".opgraph")
    V = 1024
    rng = np.random.default_rng(82 + k)
    logits = (rng.standard_normal((2, V)) * 3).astype(np.float32)
    cond, uncond = logits[0], logits[1]
    guided = uncond + (cond - uncond) * np.float32(cfg)
    order = np.lexsort((np.arange(V), -guided))[:k].astype(np.int32)
    gk = guided[order].astype(np.float64)
    p = np.exp(gk - gk.max())
    cdf = np.cumsum(p / p.sum())
    # draws away from every CDF entry (and one past the tail: clamped)
    draws = []
    for target in (0.05, 0.5, 0.93):
        cand = np.linspace(0.0, 1.0, 20001)
        ok = cand[np.min(np.abs(cand[:, None] - cdf[None, :]), axis=1) > 1e-3]
        draws.append(float(ok[np.argmin(np.abs(ok - target))]) if len(ok) else target)
    draws.append(1.5)
    rand = np.array(draws, np.float32)
    g = og.OpGraph(n_tensors=512)
    try:
        tl = g.tensor(og.F32, [V, 2])
        tr = g.tensor(og.F32, [len(draws)])
        outs = [_sampler_graph(g, og, tl, tr, V, k, cfg, i) for i in range(len(draws))]
        g.build([t for o in outs for t in o])
        g.set(tl, logits)
        g.set(tr, rand)
        g.compute()
        got = [(g.get(a, np.int32), g.get(b, np.int32), g.get(c)) for a, b, c in outs]
    finally:
        g.close()
    for (idxk, code, code_f), u in zip(got, draws):
        assert np.array_equal(idxk, order)
        pick = min(max(k - int((cdf > u).sum()), 0), k - 1)
        assert code[0] == order[pick] and code_f[0] == float(order[pick])
