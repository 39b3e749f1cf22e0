"""GPU: the RVQ depth decoder's transformer layer (src/depth-decoder.h:196-236)
built with the restated ggml API and run through ggml_backend_graph_compute
on the MI355X backend, against a CPU float32 restatement with dequantized
weights (torch on the CPU); plus the three ops it adds to the backend
(f32 x f32 MUL_MAT, DIAG_MASK_INF, SOFT_MAX) through the C-ABI.

Tolerances (stated): layer output cosine >= 0.9999 and relative RMS error
<= 5e-3 (the Q8_0 GEMV / GEMM quantize or round the activations as ggml
does; the reference does not); f32 MUL_MAT max-rel 1e-6 against float64
(double accumulation of f32 products); SOFT_MAX max-abs 1e-6 against
float64; DIAG_MASK_INF bit-exact."""
import ctypes
import importlib

import numpy as np
import pytest
import torch

from conftest import cosine

pytestmark = pytest.mark.gpu


def st():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def ptr(t):
    return ctypes.c_void_p(t.data_ptr())


def _deq(orc, rows, k):
    return torch.from_numpy(orc.dequantize(8, rows, k, rows.shape[0]).reshape(rows.shape[0], k))


def ref_layer(orc, dg, w, x):
    """x [B, S, dim] f32 on the CPU; causal attention over S, no RoPE."""
    B, S, dim = x.shape
    Nh, D = dg.N_HEADS, dg.HEAD_DIM
    W = {n: _deq(orc, w[n], dim if n != "w_down" else dg.FF_INNER)
         for n in ("wq", "wk", "wv", "wo", "w_gate", "w_up", "w_down")}

    def rms(a, g_):
        return a / torch.sqrt((a * a).mean(-1, keepdim=True) + dg.RMS_EPS) * torch.from_numpy(g_)

    h = rms(x, w["attn_norm"])
    q, k, v = ((h @ W[n].T).reshape(B, S, Nh, D).permute(0, 2, 1, 3) for n in ("wq", "wk", "wv"))
    s = (q @ k.transpose(-1, -2).contiguous()) / np.sqrt(D)
    s = s.masked_fill(torch.triu(torch.ones(S, S, dtype=torch.bool), 1), float("-inf"))
    a = (torch.softmax(s, -1) @ v).permute(0, 2, 1, 3).reshape(B, S, Nh * D)
    x = x + a @ W["wo"].T
    h = rms(x, w["ffn_norm"])
    return x + (torch.nn.functional.silu(h @ W["w_gate"].T) * (h @ W["w_up"].T)) @ W["w_down"].T


@pytest.mark.parametrize("S,B", [(2, 1), (8, 1), (5, 2), (8, 2)])
def test_depth_layer_through_backend(pkg, orc, S, B):
    """S steps (2..8) x B streams (1, or the CFG pair): M = S * B tokens from
    2 (GEMVs with the norm / SwiGLU prologues) to 16 (GEMM)."""
    og = importlib.import_module(pkg.__name__ + ".opgraph")
    dg = importlib.import_module(pkg.__name__ + ".depthgraph")
    torch.set_num_threads(16)
    w = dg.synth_layer(61 + S)
    x = np.random.default_rng(70 + S * B).standard_normal((B, S, dg.DIM)).astype(np.float32)
    g = og.OpGraph()
    try:
        lw = dg.Layer(g)
        tx = g.tensor(og.F32, [dg.DIM, S, B])
        out = dg.build_layer(g, lw, tx, S, B)
        g.build([out])
        lw.upload(g, w)
        g.set(tx, x)
        g.compute()
        y0 = g.get(out).reshape(B, S, dg.DIM)
        for _ in range(2):
            g.compute()
            assert np.array_equal(g.get(out).reshape(B, S, dg.DIM), y0)
    finally:
        g.close()
    ref = ref_layer(orc, dg, w, torch.from_numpy(x)).numpy()
    assert np.isfinite(y0).all()
    rel_rms = float(np.sqrt(((y0.astype(np.float64) - ref) ** 2).mean() / (ref.astype(np.float64) ** 2).mean()))
    assert cosine(y0, ref) >= 0.9999 and rel_rms <= 5e-3, (cosine(y0, ref), rel_rms)


def test_mul_mat_f32_broadcast_and_views(mm):
    """dst[i, j, i2, i3] = sum_k a[k, i, i2/r2, i3/r3] b[k, j, i2, i3] with a
    permuted (non-contiguous) b and a broadcast over dim 2."""
    L = mm.load()
    g = torch.Generator().manual_seed(62)
    a = torch.randn((2, 4, 7, 256), generator=g)            # ggml [256, 7, 4, 2]
    bq = torch.randn((2, 5, 8, 256), generator=g)           # [B, S, H, D]
    b = bq.permute(0, 2, 1, 3)                              # ggml [256, 5, 8, 2], strided
    ta, tb = a.cuda(), b.cuda()
    out = torch.empty((2, 8, 5, 7), device="cuda")          # ggml [7, 5, 8, 2]
    assert L.mmhip_mul_mat_f32(ctypes.byref(mm.view_of(ta)), ctypes.byref(mm.view_of(tb)), ptr(out), st()) == 0
    a64 = a.double().repeat_interleave(2, dim=1)            # head h uses a's head h // 2
    ref = torch.einsum("bhik,bhjk->bhji", a64, b.double())
    assert float((out.cpu().double() - ref).abs().max() / ref.abs().max()) < 1e-6


def test_diag_mask_inf_and_soft_max(mm):
    L = mm.load()
    g = torch.Generator().manual_seed(63)
    x = torch.randn((3, 16, 8, 8), generator=g) * 4         # ggml [8 keys, 8 queries, 16, 3]
    tx = x.cuda()
    m = torch.empty_like(tx)
    assert L.mmhip_diag_mask_inf(ctypes.byref(mm.view_of(tx)), 0, ptr(m), st()) == 0
    tri = torch.triu(torch.ones(8, 8, dtype=torch.bool), 1)
    assert torch.equal(m.cpu(), x.masked_fill(tri, float("-inf")))
    m2 = torch.empty_like(tx)
    assert L.mmhip_diag_mask_inf(ctypes.byref(mm.view_of(tx)), 3, ptr(m2), st()) == 0
    assert torch.equal(m2.cpu(), x.masked_fill(torch.triu(torch.ones(8, 8, dtype=torch.bool), 4), float("-inf")))
    p = torch.empty_like(tx)
    assert L.mmhip_soft_max(ctypes.byref(mm.view_of(m)), ptr(p), st()) == 0
    ref = torch.softmax(m.cpu().double(), -1)
    assert float((p.cpu().double() - ref).abs().max()) < 1e-6
    # a long row (the sampler's 1024-entry vocabulary) and a strided view
    v = torch.randn((2, 1024), generator=g).cuda() * 8
    pv = torch.empty((2, 1000), device="cuda")
    assert L.mmhip_soft_max(ctypes.byref(mm.view_of(v[:, 24:])), ptr(pv), st()) == 0
    assert float((pv.cpu().double() - torch.softmax(v[:, 24:].cpu().double(), -1)).abs().max()) < 1e-6
