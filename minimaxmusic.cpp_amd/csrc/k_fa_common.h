// k_fa_common.h - argument block shared by the flash-attention kernels.
#pragma once
#include <stdint.h>
#include <stddef.h>
#include <hip/hip_runtime.h>

namespace mmhip {

// ggml FLASH_ATTN_EXT operands: q f32 [D, nq, Hq, B], k/v f16 [D, nkv, Hkv, Bk],
// mask f16 [>=nkv, >=nq, mne2, mne3] (or null); strides in bytes.
struct FaArgs {
    const char * q;
    int64_t      qnb1, qnb2, qnb3;
    const char * k;
    int64_t      knb1, knb2, knb3;
    const char * v;
    int64_t      vnb1, vnb2, vnb3;
    const char * mask;
    int64_t      mnb1, mnb2, mnb3;
    int          mne2, mne3;
    int          nq, Hq, Hkv, B, Bk, nkv;
    float        scale;
};

// The per-head work between the QKV projection and a decode attention, done
// in the attention's prologue: the query rows' RMS norm (times the weight) and
// NeoX RoPE, and the new key / value rows (the key normed and roped the same
// way) written into the caches at row ids[t] - the arithmetic of
// k_head_rows.  Attention batch b is token t = b, KV head g is head h = g.
struct FaHead {
    const char *    q_src;  // raw query rows: row (h, t) at q_src + t q_nbt + h q_nbh (bytes)
    int64_t         q_nbh, q_nbt;
    int             q_H;
    const float *   q_w;  // norm weight (nullptr: none)
    float           q_eps;
    int             q_norm;
    const int32_t * q_pos;  // rope positions [t] (nullptr: no rope)
    float           q_ts;
    int64_t         qr0, qr1, qr2, qr3;  // attention q element (iq, hq, b) -> row qr0 + iq qr1 + hq qr2 + b qr3
    const char *    k_src;
    int64_t         k_nbh, k_nbt;
    const float *   k_w;
    float           k_eps;
    int             k_norm;
    const int32_t * k_pos;
    float           k_ts;
    const char *    v_src;
    int64_t         v_nbh, v_nbt;
    const char *    ids;  // cache row of (h, t): ids + (h % ids_ne1) ids_nb1 + (t % ids_ne2) ids_nb2
    int             ids_type;
    int64_t         ids_nb1, ids_nb2, ids_ne1, ids_ne2;
};

size_t fa_decode_workspace(const FaArgs & a, int D);
// With xq != nullptr the split combine also quantises the output rows into
// the activation layout for weights of qtype; *quantised reports whether it
// did (it does not when the decode runs in one split).
int    fa_decode(const FaArgs & a, int D, float * out, void * ws, size_t ws_bytes, hipStream_t stream,
                 int qtype = 0, void * xq = nullptr, bool * quantised = nullptr, const FaHead * hd = nullptr);
// Whether fa_decode takes a FaHead for these arguments (the MFMA decode
// kernel with its query columns and the two new rows one wave each).
bool   fa_decode_head_supported(const FaArgs & a, int D);

size_t fa_mfma_workspace(const FaArgs & a);
bool   fa_mfma_supported(const FaArgs & a, int D);
int    fa_mfma(const FaArgs & a, int D, float * out, void * ws, size_t ws_bytes, hipStream_t stream);

// Kernel choice: the split-KV decode kernel while the query rows of one KV head
// fit one workgroup (the LM decode, the depth decoder's few rows), the MFMA
// kernel beyond (prefill, DiT).
inline bool fa_use_mfma(const FaArgs & a, int D) {
    return fa_mfma_supported(a, D) && (a.Hq / a.Hkv) * a.nq > 8;
}

}  // namespace mmhip
