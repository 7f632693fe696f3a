// Internal launch arguments shared by the kernels and the C-ABI entry points (not part of the public ABI).
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "../../include/bifrost.h"

namespace bf {

constexpr int DT_F32 = BF_DTYPE_F32;
constexpr int DT_BF16 = BF_DTYPE_BF16;
constexpr int BF_ERR_UNSUPPORTED = BF_STATUS_UNSUPPORTED;
constexpr int GDN_PHASE_PREP = BF_GDN_PHASE_PREP;
constexpr int GDN_PHASE_SCAN = BF_GDN_PHASE_SCAN;

struct GdnArgs {
    const void* q;           // [N_tok][G*R][D]  in_dtype
    const void* k;           // [N_tok][G][D]    in_dtype
    const void* v;           // [N_tok][G][D]    in_dtype
    const float* g;          // [N_tok][G]
    const float* beta;       // [N_tok][G]
    const int32_t* cu_seqlens;  // [num_seqs + 1] or null (uniform sequences of seq_len tokens)
    int num_seqs;
    int seq_len;
    long total_tokens;
    int G, R, D;
    int in_dtype, o_dtype;
    float scale;
    const float* s0;         // [num_seqs][G][D][D] or null
    void* o;                 // [N_tok][G*R][D]  o_dtype
    float* s_out;            // [num_seqs][G][D][D] or null
    int max_chunks;          // grid bound for the per-chunk kernel
    // workspace carve-up
    float* ws_gcum;
    void* ws_w;
    float* ws_uT;
    void* ws_kt;
    void* ws_attn;
};

int gdn_dispatch(const GdnArgs& a, int phases, hipStream_t stream);

}  // namespace bf
