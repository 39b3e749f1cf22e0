"""CPU reference of the LM batched decode step (test infrastructure): the
op sequence of qw3lm_forward_batch (src/qwen3-lm.h:695-856) evaluated with the
oracle (oracle/), on weights and KV caches read back from the device."""
import numpy as np

import oracle


class LmState:
    """Host copies of the model (GGUF bytes / f32) and of the f16 KV caches."""

    def __init__(self, lm):
        c = lm.cfg
        self.c = c
        self.w = {}
        for l in range(c.n_layers):
            for n in ("attn_norm", "q_norm", "k_norm", "ffn_norm"):
                self.w[f"blk.{l}.{n}"] = lm.get(f"blk.{l}.{n}", np.float32)
            for n in ("qkv", "o_proj", "gate_up", "down"):
                self.w[f"blk.{l}.{n}"] = lm.get(f"blk.{l}.{n}")
        self.w["output_norm"] = lm.get("output_norm", np.float32)
        self.w["lm_head"] = lm.get("lm_head")
        # caches: ggml [D, max_seq, Nkv, n_sets] -> numpy [n_sets, Nkv, max_seq, D]
        shp = (c.n_sets, c.n_kv_heads, c.max_seq, c.head_dim)
        self.k = [lm.get(f"kv_k4_{l}", np.float16).reshape(shp).copy() for l in range(c.n_layers)]
        self.v = [lm.get(f"kv_v4_{l}", np.float16).reshape(shp).copy() for l in range(c.n_layers)]


def decode(st, embeds, sets, kv_pos, flavour="ggml"):
    """One step; updates st's caches. kv_pos: positions of the sets before the step."""
    c = st.c
    H, D, Nh, Nkv = c.hidden, c.head_dim, c.n_heads, c.n_kv_heads
    q_dim, kv_dim = Nh * D, Nkv * D
    N = len(sets)
    t = c.wtype

    def mm(name, n_out, k_in, x):
        if flavour == "ggml":
            return oracle.mul_mat_ggml(t, st.w[name], n_out, k_in, x)
        return oracle.mul_mat_f64(t, st.w[name], n_out, k_in, x).astype(np.float32)

    max_len = max(kv_pos[s] + 1 for s in sets)
    n_kv_pad = min((max_len + 255) // 256 * 256, c.max_seq)
    mask = np.zeros((N, 1, 1, n_kv_pad), np.float16)
    for i, s in enumerate(sets):
        mask[i, ..., kv_pos[s] + 1:] = -np.inf
    pos = np.array([kv_pos[s] for s in sets], np.int32)
    scale = float(np.float32(1.0 / np.sqrt(D)))
    h = np.asarray(embeds, np.float32)
    for l in range(c.n_layers):
        p = f"blk.{l}."
        x = oracle.rms_norm_mul(h, st.w[p + "attn_norm"], c.rms_eps)
        qkv = mm(p + "qkv", q_dim + 2 * kv_dim, H, x)
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
        h = h + mm(p + "down", H, c.ffn, ff)
    hid = oracle.rms_norm_mul(h, st.w["output_norm"], c.rms_eps)
    logits = mm("lm_head", c.vocab, H, hid)
    return logits, hid
