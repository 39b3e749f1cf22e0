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

size_t fa_decode_workspace(const FaArgs & a, int D);
// With xq != nullptr the split combine also quantises the output rows into
// the activation layout for weights of qtype; *quantised reports whether it
// did (it does not when the decode runs in one split).
int    fa_decode(const FaArgs & a, int D, float * out, void * ws, size_t ws_bytes, hipStream_t stream,
                 int qtype = 0, void * xq = nullptr, bool * quantised = nullptr);

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
