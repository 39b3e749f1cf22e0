"""The RVQ depth decoder's transformer layer as a ggml graph on the MI355X
backend.

build_layer() makes the same nodes as the reference's depth_layer
(src/depth-decoder.h:196-236) with the restated ggml API (opgraph.OpGraph):
RMSNorm (eps 1e-6) times the norm weight, Q/K/V projections, causal manual
attention without RoPE (scores = K.Q as an f32 MUL_MAT, scale 1/sqrt(256),
DIAG_MASK_INF, SOFT_MAX, P.V against the transposed V), the output
projection and residual, then the split SwiGLU MLP (gate, up, down) and its
residual.  Token counts are tiny (S <= 8 steps x B streams), so the Q8_0
projections take the GEMV path (M <= 8) or the GEMM (M <= 16).  Weights are
synthesised GGUF Q8_0 rows (int8 quants uniform in [-127, 127], fp16 scales
|N(0, 0.02)| / 127), as in ditgraph.
"""
import numpy as np

from . import ditgraph, opgraph

DIM, N_HEADS, HEAD_DIM, FF_INNER = 4096, 16, 256, 6144
RMS_EPS = 1e-6


def synth_layer(seed, dim=DIM, ff=FF_INNER):
    rng = np.random.default_rng(seed)
    w = {}
    for n, (rows, k) in {"wq": (dim, dim), "wk": (dim, dim), "wv": (dim, dim), "wo": (dim, dim),
                         "w_gate": (ff, dim), "w_up": (ff, dim), "w_down": (dim, ff)}.items():
        w[n] = ditgraph.q8_0_rows(rng, rows, k)
    for n in ("attn_norm", "ffn_norm"):
        w[n] = (1.0 + 0.05 * rng.standard_normal(dim)).astype(np.float32)
    return w


class Layer:
    """Graph tensors of one layer's weights, created in g."""

    def __init__(self, g, dim=DIM, ff=FF_INNER):
        t = g.tensor
        self.wq, self.wk, self.wv, self.wo = (t(opgraph.Q8_0, [dim, dim]) for _ in range(4))
        self.w_gate = t(opgraph.Q8_0, [dim, ff])
        self.w_up = t(opgraph.Q8_0, [dim, ff])
        self.w_down = t(opgraph.Q8_0, [ff, dim])
        self.attn_norm = t(opgraph.F32, [dim])
        self.ffn_norm = t(opgraph.F32, [dim])

    def upload(self, g, w):
        for n, arr in w.items():
            g.set(getattr(self, n), arr)


def build_layer(g, lw, x, S, B, n_heads=N_HEADS, head_dim=HEAD_DIM):
    """x [dim, S, B] f32 -> [dim, S, B] (src/depth-decoder.h:196-236)."""
    D, Nh = head_dim, n_heads
    h = g.mul(g.rms_norm(x, RMS_EPS), lw.attn_norm)
    q = g.permute(g.reshape(g.mul_mat(lw.wq, h), [D, Nh, S, B]), 0, 2, 1, 3)
    k = g.permute(g.reshape(g.mul_mat(lw.wk, h), [D, Nh, S, B]), 0, 2, 1, 3)
    v = g.permute(g.reshape(g.mul_mat(lw.wv, h), [D, Nh, S, B]), 0, 2, 1, 3)
    scores = g.scale(g.mul_mat(k, q), float(np.float32(1.0) / np.sqrt(np.float32(D))))
    scores = g.soft_max(g.diag_mask_inf(scores, 0))
    vt = g.cont(g.transpose(v))
    attn = g.cont(g.permute(g.mul_mat(vt, scores), 0, 2, 1, 3))
    attn = g.reshape(attn, [Nh * D, S, B])
    x = g.add(x, g.mul_mat(lw.wo, attn))
    h = g.mul(g.rms_norm(x, RMS_EPS), lw.ffn_norm)
    act = g.swiglu_split(g.mul_mat(lw.w_gate, h), g.mul_mat(lw.w_up, h))
    return g.add(x, g.mul_mat(lw.w_down, act))
