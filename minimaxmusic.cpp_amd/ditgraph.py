"""The DiT transformer block as a ggml graph on the MI355X backend.

build_block() makes the same nodes as the reference's dit_block
(src/dit.h:183-247) with the restated ggml API (opgraph.OpGraph): LayerNorm
with weight and bias (src/dit.h:161-167), Q/K/V projections, partial NeoX RoPE
on the first 32 dims of each head (theta 1e4), K/V cast to f16 into
FLASH_ATTN_EXT (prec F32), the output projection and residual, then the
SwiGLU feed-forward whose ff_in emits [value | gate] with biases.
build_input() makes the graph head (src/dit.h:250-268): the channel concat
[latent, zeros, condition], the residual preprocess projection, proj_in and
the prepended timestep token.  Weights are GGUF Q8_0 rows (the default DiT
file), synthesised here: int8 quants uniform in [-127, 127], fp16 scales
|N(0, 0.02)| / 127; or BF16 rows (the native-BF16 files), N(0, 0.02)
rounded to bf16.
"""
import numpy as np

from . import opgraph

DIM, N_HEADS, HEAD_DIM, FF_INNER, ROTARY_DIM = 2048, 32, 64, 8192, 32
IN_CH, COND_DIM = 128, 2048
CONCAT_CH = 2 * IN_CH + COND_DIM
LN_EPS, ROPE_BASE = 1e-5, 10000.0


def q8_0_rows(rng, n, k):
    """n GGUF Q8_0 rows of k elements (34-byte blocks: fp16 d, 32 int8)."""
    if k % 32:
        raise ValueError("Q8_0 rows need k % 32 == 0")
    blk = np.zeros((n, k // 32), dtype=[("d", "<f2"), ("qs", "i1", (32,))])
    blk["d"] = (np.abs(rng.standard_normal((n, k // 32))) * 0.02 / 127).astype(np.float16)
    blk["qs"] = rng.integers(-127, 128, (n, k // 32, 32), dtype=np.int8)
    return blk.view(np.uint8).reshape(n, k // 32 * 34)


def bf16_rows(rng, n, k):
    """n BF16 rows of k elements (uint16 bit patterns): N(0, 0.02) rounded
    to the nearest bf16, ties to even."""
    u = (rng.standard_normal((n, k)) * 0.02).astype(np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def synth_block(seed, dim=DIM, ff=FF_INNER, wtype=opgraph.Q8_0):
    """Host arrays of one block's tensors: Q8_0 rows [N, K/32*34] (or BF16
    rows [N, K]) for the projections, f32 vectors for norms and biases."""
    rng = np.random.default_rng(seed)
    w = {}
    rows_of = q8_0_rows if wtype == opgraph.Q8_0 else bf16_rows
    for n, (rows, k) in {"wq": (dim, dim), "wk": (dim, dim), "wv": (dim, dim), "wo": (dim, dim),
                         "ff_in_w": (2 * ff, dim), "ff_out_w": (dim, ff)}.items():
        w[n] = rows_of(rng, rows, k)
    for n, size in {"norm1_w": dim, "norm1_b": dim, "norm2_w": dim, "norm2_b": dim,
                    "ff_in_b": 2 * ff, "ff_out_b": dim}.items():
        base = 1.0 if n.endswith("_w") else 0.0
        w[n] = (base + 0.05 * rng.standard_normal(size)).astype(np.float32)
    return w


class Block:
    """Graph tensors of one block's weights, created in g."""

    def __init__(self, g, dim=DIM, ff=FF_INNER, wtype=opgraph.Q8_0):
        t = g.tensor
        self.wq, self.wk, self.wv, self.wo = (t(wtype, [dim, dim]) for _ in range(4))
        self.ff_in_w = t(wtype, [dim, 2 * ff])
        self.ff_out_w = t(wtype, [ff, dim])
        self.norm1_w, self.norm1_b, self.norm2_w, self.norm2_b = (t(opgraph.F32, [dim]) for _ in range(4))
        self.ff_in_b = t(opgraph.F32, [2 * ff])
        self.ff_out_b = t(opgraph.F32, [dim])

    def upload(self, g, w):
        for n, arr in w.items():
            g.set(getattr(self, n), arr)


def layer_norm(g, x, w, b):
    """src/dit.h:161-167: ggml_norm(eps 1e-5) * w + b."""
    return g.add(g.mul(g.norm(x, LN_EPS), w), b)


def build_block(g, blk, x, pos, S, B, n_heads=N_HEADS, head_dim=HEAD_DIM, ff=FF_INNER):
    """x [dim, S, B] f32 -> [dim, S, B] (src/dit.h:183-247, flash-attention
    branch)."""
    D, Nh = head_dim, n_heads
    h = layer_norm(g, x, blk.norm1_w, blk.norm1_b)
    q = g.reshape(g.mul_mat(blk.wq, h), [D, Nh, S, B])
    k = g.reshape(g.mul_mat(blk.wk, h), [D, Nh, S, B])
    v = g.reshape(g.mul_mat(blk.wv, h), [D, Nh, S, B])
    q = g.rope_neox(q, pos, ROTARY_DIM, ROPE_BASE)
    k = g.rope_neox(k, pos, ROTARY_DIM, ROPE_BASE)
    q = g.permute(q, 0, 2, 1, 3)
    k = g.cast(g.permute(k, 0, 2, 1, 3), opgraph.F16)
    v = g.cast(g.permute(v, 0, 2, 1, 3), opgraph.F16)
    scale = float(np.float32(1.0) / np.sqrt(np.float32(D)))
    attn = g.reshape(g.flash_attn(q, k, v, None, scale), [Nh * D, S, B])
    x = g.add(x, g.mul_mat(blk.wo, attn))
    h = layer_norm(g, x, blk.norm2_w, blk.norm2_b)
    f = g.add(g.mul_mat(blk.ff_in_w, h), blk.ff_in_b)
    nb = f.contents.nb
    value = g.cont(g.view_3d(f, [ff, S, B], nb[1], nb[2], 0))
    gate = g.cont(g.view_3d(f, [ff, S, B], nb[1], nb[2], ff * nb[0]))
    out = g.add(g.mul_mat(blk.ff_out_w, g.swiglu_split(gate, value)), blk.ff_out_b)
    return g.add(x, out)


def build_input(g, xt, cond, temb, pre_w, in_w):
    """src/dit.h:250-268: [latent, zeros, condition] along channels, the
    residual preprocess projection, proj_in, then the timestep token
    prepended along the sequence."""
    zeros = g.scale(xt, 0.0)
    x = g.concat(g.concat(xt, zeros, 0), cond, 0)
    x = g.add(g.mul_mat(pre_w, x), x)
    x = g.mul_mat(in_w, x)
    return g.concat(temb, x, 1)
