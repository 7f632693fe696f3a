/*
 * bifrost.h — C ABI of libbifrost_hip.so, the MI355X (gfx950) kernels of the Bifrost converted-layer core.
 *
 * Conventions
 *   - Every pointer argument is a device pointer unless stated otherwise; tensors are dense and row-major in the
 *     layouts given per function (no strides). "N_tok" is the number of packed tokens: B equal-length sequences of
 *     T tokens are simply N_tok = B*T with num_seqs = B.
 *   - dtype codes: BF_DTYPE_F32 (fp32) and BF_DTYPE_BF16 (bf16, stored as 16-bit words).
 *   - Work is enqueued on `stream` (a hipStream_t passed as void*; null = the default stream) and is not
 *     synchronised; results are ready when the stream reaches that point.
 *   - Return value: 0 on success, a negative BF_STATUS_* code for an argument error (nothing was launched), or a
 *     positive hipError_t from the launch. bf_status_string() names every code. No exceptions cross the ABI.
 *   - No entry point allocates device memory: scratch space is a caller-provided workspace whose size comes from
 *     the matching *_workspace_size() query. Calls on one stream are ordered; calls that share a workspace must
 *     not overlap.
 *   - Supported head dims: D = 64, 128, 256 (D_k = D_v = D).
 */
#ifndef BIFROST_H
#define BIFROST_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define BF_DTYPE_F32 0
#define BF_DTYPE_BF16 1

#define BF_STATUS_OK 0
#define BF_STATUS_INVALID (-1)     /* null pointer, non-positive size, inconsistent shape */
#define BF_STATUS_UNSUPPORTED (-2) /* head dim, dtype or chunk size outside the supported set */
#define BF_STATUS_WORKSPACE (-3)   /* workspace missing or smaller than the size query returned */

/* Phases of bf_gdn_fwd (bit mask); BF_GDN_PHASE_ALL runs the whole operator. */
#define BF_GDN_PHASE_PREP 1
#define BF_GDN_PHASE_SCAN 2
#define BF_GDN_PHASE_ALL 3

/* Library version (major * 10000 + minor * 100 + patch). */
int bf_version(void);

/* Static description of a status code (never null). */
const char* bf_status_string(int status);

/*
 * Chunked gated delta rule, forward, in GQA form with packed variable-length sequences.
 *
 * Replaces the reference operator kernels.delta_rule(q, k, v, g, beta, chunk_size=64, initial_state)
 * (Heimdall/heimdall/kernels.py:152-155 -> delta_rule_reference, kernels.py:94-129) when R = 1, and
 * motor.delta_rule_gqa(q, k, v, g, beta, chunk=64, state) (Heimdall/heimdall/motor.py:70-102) for R > 1; it also
 * covers the native op GGML_OP_GATED_DELTA_NET at D = 256 (Heimdall/llamacpp/bifrost.patch:5-18).
 *
 * Per KV head g and token t (alpha = exp(g_t)):
 *     S_t = alpha S_{t-1} + beta_t k_t (v_t - alpha S_{t-1}^T k_t)^T,   o_{t,h} = S_t^T (scale * q_{t,h})
 * for the R query heads h = g*R + r of the group. Each sequence starts from its initial state (zeros if
 * initial_state is null) and its final state is written to final_state (if non-null).
 *
 *   q [N_tok][G*R][D], k [N_tok][G][D], v [N_tok][G][D]   in_dtype (k expected L2-normalised per head)
 *   g, beta [N_tok][G] fp32   (log-decay, write strength)
 *   cu_seqlens [num_seqs + 1] int32 (device), or null for num_seqs equal sequences of N_tok / num_seqs tokens
 *   initial_state [num_seqs][G][D][D] fp32 or null;  final_state [num_seqs][G][D][D] fp32 or null
 *   o [N_tok][G*R][D] in o_dtype (fp32 or bf16)
 *   phases: BF_GDN_PHASE_ALL, or PREP then SCAN in two calls with the same arguments and workspace.
 * Chunk length is 64. Arithmetic: MFMA in in_dtype with fp32 accumulation; state, decay and the triangular
 * inverse in fp32.
 */
int bf_gdn_workspace_size(int64_t total_tokens, int num_seqs, int G, int R, int D, int in_dtype, size_t* bytes);

int bf_gdn_fwd(const void* q, const void* k, const void* v, const float* g, const float* beta,
               const int32_t* cu_seqlens, int num_seqs, int64_t total_tokens, int G, int R, int D, int in_dtype,
               float scale, const float* initial_state, void* o, int o_dtype, float* final_state, void* workspace,
               size_t workspace_bytes, int phases, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* BIFROST_H */
