"""CPU reference of the LM batched decode step (test infrastructure): the
op sequence of qw3lm_forward_batch (src/qwen3-lm.h:695-856) evaluated with the
oracle (oracle/), on weights and KV caches read back from the device."""
import numpy as np

import oracle


class LmState:
    """Host copies of the model (GGUF bytes / f32) and of the f16 KV caches."""

    @classmethod
    def from_arrays(cls, cfg, weights, k, v):
        """cfg: an object with the mm_lm config fields; weights: name -> GGUF
        bytes / f32 array under the mm_lm names (plus "embed_tokens" for the
        prefill); k, v: per layer f16 [n_sets, Nkv, max_seq, D]."""
        st = cls.__new__(cls)
        st.c, st.w = cfg, dict(weights)
        st.t = {}
        st.k = [np.array(a, dtype=np.float16, copy=True) for a in k]
        st.v = [np.array(a, dtype=np.float16, copy=True) for a in v]
        return st

    def __init__(self, lm):
        c = lm.cfg
        self.c = c
        self.w = {}
        self.t = {}  # GGML type of each linear weight (absent: c.wtype)
        for l in range(c.n_layers):
            for n in ("attn_norm", "q_norm", "k_norm", "ffn_norm"):
                self.w[f"blk.{l}.{n}"] = lm.get(f"blk.{l}.{n}", np.float32)
            for n in ("qkv", "qk", "v", "o_proj", "gate_up", "down"):
                name = f"blk.{l}.{n}"
                if lm.has(name):
                    self.w[name] = lm.get(name)
                    self.t[name] = lm.type_of(name)
        self.w["output_norm"] = lm.get("output_norm", np.float32)
        self.w["lm_head"] = lm.get("lm_head")
        self.t["lm_head"] = lm.type_of("lm_head")
        # caches: ggml [D, max_seq, Nkv, n_sets] -> numpy [n_sets, Nkv, max_seq, D]
        self.refresh_kv(lm)

    def refresh_kv(self, lm):
        """Take the device's KV caches as they are now."""
        c = self.c
        shp = (c.n_sets, c.n_kv_heads, c.max_seq, c.head_dim)
        self.k = [lm.get(f"kv_k4_{l}", np.float16).reshape(shp).copy() for l in range(c.n_layers)]
        self.v = [lm.get(f"kv_v4_{l}", np.float16).reshape(shp).copy() for l in range(c.n_layers)]


def _qkv(st, p, mm, x):
    """The Q | K | V rows of the normed rows x: one fused weight, or the
    fused Q | K weight and a separate V of another type (src/qwen3-lm.h:742-757)."""
    c = st.c
    q_dim, kv_dim, H = c.n_heads * c.head_dim, c.n_kv_heads * c.head_dim, c.hidden
    if p + "qkv" in st.w:
        return mm(p + "qkv", q_dim + 2 * kv_dim, H, x)
    return np.concatenate([mm(p + "qk", q_dim + kv_dim, H, x), mm(p + "v", kv_dim, H, x)], axis=1)


def _qkv_rows(st, l, h, pos, sets_rows, mm):
    """The attention block's head rows for the token rows h [T, H]: the norm,
    the QKV projection, q/k-norm and RoPE; writes K / V of token i into cache
    row sets_rows[i] = (set, row) and returns q [T, Nh, D]."""
    c = st.c
    D, Nh, Nkv = c.head_dim, c.n_heads, c.n_kv_heads
    q_dim, kv_dim, H = Nh * D, Nkv * D, c.hidden
    T = h.shape[0]
    p = f"blk.{l}."
    x = oracle.rms_norm_mul(h, st.w[p + "attn_norm"], c.rms_eps)
    qkv = _qkv(st, p, mm, x)
    q = oracle.rms_norm_mul(qkv[:, :q_dim].reshape(T, Nh, D), st.w[p + "q_norm"], c.rms_eps)
    k = oracle.rms_norm_mul(qkv[:, q_dim:q_dim + kv_dim].reshape(T, Nkv, D), st.w[p + "k_norm"], c.rms_eps)
    v = qkv[:, q_dim + kv_dim:].reshape(T, Nkv, D)
    q = oracle.rope_neox(q, pos, D, c.rope_theta)
    k = oracle.rope_neox(k, pos, D, c.rope_theta)
    for i, (s, r) in enumerate(sets_rows):
        st.k[l][s, :, r] = k[i].astype(np.float16)
        st.v[l][s, :, r] = v[i].astype(np.float16)
    return q


def prefill(st, tokens, kv_set, kv_pos, flavour="ggml"):
    """qw3lm_forward (src/qwen3-lm.h:451-643) for one set from token ids:
    embedding rows (GET_ROWS of embed_tokens), the layers with causal attention
    over the padded window [0, n_kv_pad) of the set's cache, the final norm;
    returns (logits of the last token [V], final-norm hidden states [T, H])
    and writes the prompt's K / V rows into st's caches."""
    c = st.c
    H, D, Nh = c.hidden, c.head_dim, c.n_heads
    q_dim = Nh * D
    T = len(tokens)
    t = c.wtype
    mm = _mm_fn(st, flavour)

    rs = oracle.row_size(t, H)
    emb = np.asarray(st.w["embed_tokens"], np.uint8).reshape(-1, rs)
    h = oracle.dequantize(t, emb[np.asarray(tokens)], H, T)
    kv_len = kv_pos + T
    n_kv_pad = min((kv_len + 255) // 256 * 256, c.max_seq)
    mask = np.full((1, 1, T, n_kv_pad), -np.inf, np.float16)
    for i in range(T):
        mask[0, 0, i, :kv_pos + i + 1] = 0
    pos = np.arange(kv_pos, kv_pos + T, dtype=np.int32)
    scale = float(np.float32(1.0 / np.sqrt(D)))
    for l in range(c.n_layers):
        p = f"blk.{l}."
        q = _qkv_rows(st, l, h, pos, [(kv_set, int(r)) for r in pos], mm)
        kw = np.ascontiguousarray(st.k[l][kv_set:kv_set + 1, :, :n_kv_pad])
        vw = np.ascontiguousarray(st.v[l][kv_set:kv_set + 1, :, :n_kv_pad])
        q4 = np.ascontiguousarray(q.transpose(1, 0, 2)[None])  # [1, Hq, T, D]
        o = oracle.flash_attn_ext(q4, kw, vw, mask, scale, "ggml" if flavour == "ggml" else "f64")
        h = h + mm(p + "o_proj", H, q_dim, np.asarray(o, np.float32).reshape(T, q_dim))
        x = oracle.rms_norm_mul(h, st.w[p + "ffn_norm"], c.rms_eps)
        h = h + mm(p + "down", H, c.ffn, oracle.swiglu(mm(p + "gate_up", 2 * c.ffn, H, x)))
    hid = oracle.rms_norm_mul(h, st.w["output_norm"], c.rms_eps)
    return mm("lm_head", c.vocab, H, hid[-1:])[0], hid


def round_bf16(x):
    """f32 -> bf16 -> f32 as ggml rounds (nearest-even on the upper 16 bits;
    finite inputs)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000).astype(np.uint32)
    return r.view(np.float32).reshape(np.shape(x))


def _mm_fn(st, flavour):
    """The MUL_MAT of a weight by name.  Quantised weights: ggml-CPU's
    activation quantisation and integer dots ("ggml") or exact f64 ("f64").
    BF16 weights (type 30): ggml's BF16 dot multiplies bf16 weights by the
    activations rounded to bf16, each product exact, and sums them ("ggml":
    in f64 here, as the generic C path does), or the unrounded activations
    ("f64").  Each weight in its own type (st.t; c.wtype where absent)."""

    def mm(name, n_out, k_in, x):
        t = st.t.get(name, st.c.wtype)
        if t == 30:
            xr = round_bf16(x) if flavour == "ggml" else np.asarray(x, np.float32)
            return oracle.mul_mat_f64(t, st.w[name], n_out, k_in, xr).astype(np.float32)
        if flavour == "ggml":
            return oracle.mul_mat_ggml(t, st.w[name], n_out, k_in, x)
        return oracle.mul_mat_f64(t, st.w[name], n_out, k_in, x).astype(np.float32)

    return mm


def _decode_setup(st, sets, kv_pos, flavour):
    c = st.c
    N = len(sets)
    mm = _mm_fn(st, flavour)

    max_len = max(kv_pos[s] + 1 for s in sets)
    n_kv_pad = min((max_len + 255) // 256 * 256, c.max_seq)
    mask = np.zeros((N, 1, 1, n_kv_pad), np.float16)
    for i, s in enumerate(sets):
        mask[i, ..., kv_pos[s] + 1:] = -np.inf
    pos = np.array([kv_pos[s] for s in sets], np.int32)
    return mm, mask, pos, n_kv_pad


def _decode_layer(st, l, h, sets, mm, mask, pos, n_kv_pad, flavour):
    """One layer of qw3lm_forward_batch (src/qwen3-lm.h:730-840) on the rows
    h [N, H]; writes the step's K / V rows into st's caches."""
    c = st.c
    H, D, Nh, Nkv = c.hidden, c.head_dim, c.n_heads, c.n_kv_heads
    q_dim, kv_dim = Nh * D, Nkv * D
    N = len(sets)
    scale = float(np.float32(1.0 / np.sqrt(D)))
    p = f"blk.{l}."
    x = oracle.rms_norm_mul(h, st.w[p + "attn_norm"], c.rms_eps)
    qkv = _qkv(st, p, mm, x)
    q = qkv[:, :q_dim].reshape(N, Nh, D)
    k = qkv[:, q_dim:q_dim + kv_dim].reshape(N, Nkv, D)
    v = qkv[:, q_dim + kv_dim:].reshape(N, Nkv, D)
    q = oracle.rms_norm_mul(q, st.w[p + "q_norm"], c.rms_eps)
    k = oracle.rms_norm_mul(k, st.w[p + "k_norm"], c.rms_eps)
    q = oracle.rope_neox(q, pos, D, c.rope_theta)
    k = oracle.rope_neox(k, pos, D, c.rope_theta)
    for i, s in enumerate(sets):
        st.k[l][s, :, pos[i]] = k[i].astype(np.float16)
        st.v[l][s, :, pos[i]] = v[i].astype(np.float16)
    s0 = sets[0]
    kw = np.ascontiguousarray(st.k[l][s0:s0 + N, :, :n_kv_pad])
    vw = np.ascontiguousarray(st.v[l][s0:s0 + N, :, :n_kv_pad])
    q4 = np.ascontiguousarray(q[:, :, None, :])  # [B=N, Hq, nq=1, D]
    o = oracle.flash_attn_ext(q4, kw, vw, mask, scale, "ggml" if flavour == "ggml" else "f64")
    attn = np.asarray(o, np.float32).reshape(N, q_dim)
    h = h + mm(p + "o_proj", H, q_dim, attn)
    x = oracle.rms_norm_mul(h, st.w[p + "ffn_norm"], c.rms_eps)
    gu = mm(p + "gate_up", 2 * c.ffn, H, x)
    ff = oracle.swiglu(gu)
    return h + mm(p + "down", H, c.ffn, ff)


def _decode_head(st, h, mm):
    """Final norm and lm_head (src/qwen3-lm.h:843-856): (logits, hidden)."""
    c = st.c
    hid = oracle.rms_norm_mul(h, st.w["output_norm"], c.rms_eps)
    return mm("lm_head", c.vocab, c.hidden, hid), hid


def decode(st, embeds, sets, kv_pos, flavour="ggml"):
    """One step; updates st's caches. kv_pos: positions of the sets before the step."""
    mm, mask, pos, n_kv_pad = _decode_setup(st, sets, kv_pos, flavour)
    h = np.asarray(embeds, np.float32)
    for l in range(st.c.n_layers):
        h = _decode_layer(st, l, h, sets, mm, mask, pos, n_kv_pad, flavour)
    return _decode_head(st, h, mm)


def decode_teacher_forced(st, embeds, layer_outs, sets, kv_pos, flavour="ggml"):
    """The step with each layer restated from the device's own input rows of
    that layer: layer l starts from layer_outs[l - 1] (the device's rows after
    layer l - 1; the embeddings for layer 0), the final norm and lm_head from
    layer_outs[-1].  A difference in one layer is therefore not carried into
    the next (a few int8 activation codes rounding the other way when their
    f32 inputs differ in the last bits would otherwise cascade).  Returns
    (restated layer outputs, logits, hidden); updates st's caches."""
    mm, mask, pos, n_kv_pad = _decode_setup(st, sets, kv_pos, flavour)
    outs = []
    for l in range(st.c.n_layers):
        h = np.asarray(embeds if l == 0 else layer_outs[l - 1], np.float32)
        outs.append(_decode_layer(st, l, h, sets, mm, mask, pos, n_kv_pad, flavour))
    logits, hid = _decode_head(st, np.asarray(layer_outs[-1], np.float32), mm)
    return outs, logits, hid
