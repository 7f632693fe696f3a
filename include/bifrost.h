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
#define BF_STATUS_SCRATCH (-4)     /* problem needs more than the static scratch of an allocation-free entry point */

/* Phases of bf_gdn_fwd (bit mask), run in the order PREP, SUMMARY, COMBINE, OUTPUT; BF_GDN_PHASE_ALL runs the whole
 * operator.
 *   PREP     per-chunk quantities that do not depend on the state (decay, (I + A)^-1, masked q.k^T)
 *   SUMMARY  per-segment affine maps S_end = Phi S_start + N (skipped when every sequence is a single segment)
 *   COMBINE  their sequential composition per sequence: the state entering every segment (same condition)
 *   OUTPUT   per-segment scan from the segment's entry state: outputs and the final state
 * BF_GDN_PHASE_STATES is SUMMARY | COMBINE. */
#define BF_GDN_PHASE_PREP 1
#define BF_GDN_PHASE_SUMMARY 2
#define BF_GDN_PHASE_OUTPUT 4
#define BF_GDN_PHASE_COMBINE 8
#define BF_GDN_PHASE_STATES (BF_GDN_PHASE_SUMMARY | BF_GDN_PHASE_COMBINE)
#define BF_GDN_PHASE_ALL 15

/* Library version (major * 10000 + minor * 100 + patch). */
int bf_version(void);

/* Static description of a status code (never null). */
const char* bf_status_string(int status);

/*
 * Chunked gated delta rule, forward, in GQA form with packed variable-length sequences.
 *
 * Replaces the reference operator kernels.delta_rule(q, k, v, g, beta, chunk_size=64, initial_state)
 * (Heimdall/heimdall/kernels.py:152-155 -> delta_rule_reference, kernels.py:94-129) when R = 1, and
 * motor.delta_rule_gqa(q, k, v, g, beta, chunk=64, state) (Heimdall/heimdall/motor.py:70-102) for R > 1. It computes
 * the same recurrence as the native op GGML_OP_GATED_DELTA_NET (Heimdall/llamacpp/bifrost.patch:5-18) but is not a
 * drop-in for that op's launcher: it takes dense layouts and a [dk][dv] state, not ggml's per-tensor strides,
 * state-slot stride, KDA variant or transposed [dv][dk] state.
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
 *   segment_chunks: each sequence is cut into segments of this many 64-token chunks that are scanned in parallel
 *     (their entry states come from the STATES phase); 0 picks a length from the problem size. The result does not
 *     depend on it beyond rounding.
 *   phases: BF_GDN_PHASE_ALL, or PREP, SUMMARY, COMBINE, OUTPUT in separate calls (in that order) with the same
 *     arguments and workspace.
 * Chunk length is 64. Arithmetic: MFMA in in_dtype with fp32 accumulation; state, decay and the triangular
 * inverse in fp32; segment entry states composed in fp32 (split-bf16 MFMA for bf16 runs).
 */
/* Segment length (64-token chunks) that bf_gdn_fwd uses when segment_chunks is 0, or a negative status. */
int bf_gdn_segment_chunks(int64_t total_tokens, int num_seqs, int G, int R, int D);

int bf_gdn_workspace_size(int64_t total_tokens, int num_seqs, int G, int R, int D, int in_dtype,
                          int segment_chunks, size_t* bytes);

int bf_gdn_fwd(const void* q, const void* k, const void* v, const float* g, const float* beta,
               const int32_t* cu_seqlens, int num_seqs, int64_t total_tokens, int G, int R, int D, int in_dtype,
               float scale, const float* initial_state, void* o, int o_dtype, float* final_state,
               int segment_chunks, void* workspace, size_t workspace_bytes, int phases, void* stream);

/*
 * Single-token gated delta rule (GQA): kernels.delta_rule_step(q, k, v, g, beta, state)
 * (Heimdall/heimdall/kernels.py:132-138) and the inline rank-1 decode update of Heimdall/heimdall/hibrit.py:398-403.
 *   S' = e^g S + k (beta (v - e^g S^T k))^T,   o_h = S'^T q_h for the R query heads of each KV head.
 *   q [B][G*R][D], k, v [B][G][D], g, beta [B][G], state_in, state_out [B][G][D][D], o [B][G*R][D]; all fp32.
 *   state_out may equal state_in (in-place update). R <= 8.
 */
int bf_gdn_step(const float* q, const float* k, const float* v, const float* g, const float* beta,
                const float* state_in, float* state_out, float* o, int B, int G, int R, int D, void* stream);

/*
 * One decode step of the converted layer for B sequences, all at absolute position `pos`: the core of
 * HybridAttention._student with t == 1 (Heimdall/heimdall/hibrit.py:363-424) and of the llama.cpp decode graph
 * build_layer_bifrost (Heimdall/llamacpp/bifrost.patch:1039-1054,1118-1166), as one bandwidth-bound pass.
 *   window: softmax over the sinks, the ring entries with max(sinks, pos-W+1) <= position <= pos-1 and the new token
 *           (if pos >= sinks), scores qr.k / sqrt(D); lse written to `lse` (if non-null).
 *   memory (memory != 0 and pos >= W): the ring row of position pos - W (slot pos mod W; ignored unless
 *           ring_pos[slot] == pos - W) is written into the per-KV-head state (decay, delta rule), then read with qm.
 *   mix:    gamma = sigmoid(z + mix_lse (lse - ln W)) when the memory is active; o = o_win + gamma (mem_scale o_mem - o_win).
 *   cache:  ring slot pos mod W receives (kr, v, km, g_new, beta_new) and ring_pos[slot] = pos. Sinks are passed in
 *           already holding the new token when pos < sinks (the caller appends it, as the reference does).
 * Layouts: qr [B][H][D] (q_dtype), qm [B][H][D] f32 (normalised, scaled by 1/sqrt(D)), kr, v [B][G][D] (kv_dtype),
 * km [B][G][D] f32, g_new, beta_new [B][G] f32, z [B][H] f32, mix_lse, mem_scale [H] f32, sink_k/sink_v
 * [B][G][n_sinks][D] (kv_dtype), ring_k/ring_v [B][G][W][D] (kv_dtype), ring_km [B][W][G][D] f32,
 * ring_g/ring_beta [B][W][G] f32, ring_pos [W] int64, state [B][G][D][D] f32 (updated in place), o [B][H][D] f32,
 * lse [B][H] f32 or null. H = G*R, R <= 8, n_sinks <= 63.
 */
int bf_decode_workspace_size(int B, int G, int R, int D, int W, size_t* bytes);

int bf_decode_fwd(int B, int G, int R, int D, int W, int sinks, int64_t pos, int memory, int kv_dtype, int q_dtype,
                  const void* qr, const float* qm, const void* kr, const void* v, const float* km, const float* g_new,
                  const float* beta_new, const float* z, const float* mix_lse, const float* mem_scale,
                  const void* sink_k, const void* sink_v, int n_sinks, void* ring_k, void* ring_v, float* ring_km,
                  float* ring_g, float* ring_beta, int64_t* ring_pos, float* state, float* o, float* lse,
                  void* workspace, size_t workspace_bytes, void* stream);

/*
 * One decode step for B sequences each at its own position (continuous batching): the step of bf_decode_fwd for
 * sequence b at position pos[b], with a per-sequence cache. Replaces the batched-ubatch form of llama.cpp's
 * build_layer_bifrost, whose set_input takes each sequence's own positions and state row
 * (Heimdall/llamacpp/bifrost.patch:841-884; multi-sequence check llamacpp/bifrost_multiseq.cpp:48-98); per
 * sequence the result equals the reference's _student with t == 1 (Heimdall/heimdall/hibrit.py:363-424) on that
 * sequence's own cache.
 *   pos [B] int64 on the device; sequence b: ring rows [b] as in bf_decode_fwd, ring_pos [B][W] (its own slot
 *   positions, -1 empty), sink_k / sink_v [B][G][sinks][D] kv_dtype with rows 0 .. min(pos[b], sinks) - 1 present:
 *   the new token is written to sink row pos[b] when pos[b] < sinks (and to ring slot pos[b] mod W as always);
 *   state [B][G][D][D] f32, updated when memory and pos[b] >= W. The memory inputs (qm, z, mix_lse, mem_scale,
 *   state) are required when memory is set, since the positions are not read on the host.
 * Workspace: bf_decode_workspace_size bytes. sinks <= 63, R <= 8.
 */
int bf_decode_fwd_batch(int B, int G, int R, int D, int W, int sinks, const int64_t* pos, int memory, int kv_dtype,
                        int q_dtype, const void* qr, const float* qm, const void* kr, const void* v, const float* km,
                        const float* g_new, const float* beta_new, const float* z, const float* mix_lse,
                        const float* mem_scale, void* sink_k, void* sink_v, void* ring_k, void* ring_v, float* ring_km,
                        float* ring_g, float* ring_beta, int64_t* ring_pos, float* state, float* o, float* lse,
                        void* workspace, size_t workspace_bytes, void* stream);

/*
 * One decode step of the converted layer from the layer's own inputs, for bf16 activations: _student with t == 1
 * (Heimdall/heimdall/hibrit.py:363-424) including its _mem_inputs (:327-334) and the gamma logit mix(x) (:409), in
 * one call. It runs the kernels of bf_gate_project (ab and mix), bf_mem_project (qm with scale D^-1/2 and km, fp32),
 * bf_mem_gates and then bf_decode_fwd (pos_arr null: all sequences at pos) or bf_decode_fwd_batch (pos_arr [B]
 * int64 on the device: sequence b at pos_arr[b]) on `stream`, so results equal those entry points' chained (bit for
 * bit). The caller keeps the cache bookkeeping of those entry points: with one position, the new token appended to
 * the sinks while pos < sinks (n_sinks counts it) and a zero state before the memory is first written; with
 * pos_arr, the fixed per-sequence sink blocks and ring_pos rows of bf_decode_fwd_batch.
 *   x [B][d_model] bf16 (d_model a multiple of 8, 16-byte aligned); q [B][H][D], k, v [B][G][D], qr [B][H][D],
 *   kr [B][G][D] bf16, dense; fq [H][D][D], fk [G][D][D] f32 (the module's projections); w_ab [2G][d_model], w_mix
 *   [H][d_model] f32 (16-byte aligned), b_ab [2G], b_mix [H] f32 or null; A_log, dt_bias, decay_mask [G],
 *   mix_lse, mem_scale [H] f32; the cache and o as in bf_decode_fwd / bf_decode_fwd_batch (bf16 ring and sinks).
 *   2G + H <= 64, H = G * R with R <= 8, sinks <= 63.
 * Workspace: bf_student_decode_workspace_size bytes.
 */
int bf_student_decode_workspace_size(int B, int H, int G, int D, int W, int d_model, size_t* bytes);

int bf_student_decode(int B, int H, int G, int D, int W, int sinks, int64_t pos, const int64_t* pos_arr, int memory,
                      int d_model, const void* x, const void* q, const void* k, const void* v, const void* qr,
                      const void* kr, const float* fq, const float* fk, const float* w_ab, const float* b_ab,
                      const float* w_mix, const float* b_mix, const float* A_log, const float* dt_bias,
                      const float* decay_mask, const float* mix_lse, const float* mem_scale, void* sink_k,
                      void* sink_v, int n_sinks, void* ring_k, void* ring_v, float* ring_km, float* ring_g,
                      float* ring_beta, int64_t* ring_pos, float* state, float* o, void* workspace,
                      size_t workspace_bytes, void* stream);

/*
 * bf_decode_fwd without a workspace argument: the same kernels and results, with their scratch (the memory read and
 * the window-split partials, bf_decode_workspace_size bytes) in a static device buffer of
 * BF_DECODE_STATIC_SCRATCH_BYTES that the library holds on each GPU it runs on until the process ends. No counterpart
 * in the reference: it is for callers that cannot allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid allocation); the call allocates and frees nothing. Runs on the current device; its
 * buffer's address is looked up once per device, on the first call there. Returns BF_STATUS_SCRATCH, launching
 * nothing, when bf_decode_workspace_size exceeds the buffer (e.g. B = 64, H = 16, G = 4, D = 256, W = 2048 needs
 * 5.3 MB). Every call on one GPU shares that GPU's buffer: calls that overlap in time on one GPU (other streams,
 * other threads) race and must be serialised by the caller.
 */
#define BF_DECODE_STATIC_SCRATCH_BYTES (16u << 20)
int bf_decode_fwd_noalloc(int B, int G, int R, int D, int W, int sinks, int64_t pos, int memory, int kv_dtype,
                          int q_dtype, const void* qr, const float* qm, const void* kr, const void* v, const float* km,
                          const float* g_new, const float* beta_new, const float* z, const float* mix_lse,
                          const float* mem_scale, const void* sink_k, const void* sink_v, int n_sinks, void* ring_k,
                          void* ring_v, float* ring_km, float* ring_g, float* ring_beta, int64_t* ring_pos,
                          float* state, float* o, float* lse, void* stream);

/*
 * Sliding-window + sink attention over a prefill chunk, with per-row log-sum-exp and the fused gamma mix:
 * HybridAttention._window_fp32 (Heimdall/heimdall/hibrit.py:341-361) plus the mix of hibrit.py:409-411; covers the
 * soft_max_ext + LSE + mix part of the llama.cpp prefill graph (Heimdall/llamacpp/bifrost.patch:1095-1148).
 *   Query i (position start + i) sees the sinks j < n_sinks with j <= its position, and the window keys at positions
 *   kp with sinks <= kp <= position, position - kp < W: kp >= start from the chunk (k, v), kp < start from the ring
 *   (slot kp mod W, used only if ring_pos[slot] == kp; ring_k may be null when there is no history).
 *   s = q.k / sqrt(D); lse = ln sum e^s; o_win = softmax(s) V.
 *   mix != 0: gamma = sigmoid(z + mix_lse (lse - ln W)) for positions >= W, else 0;
 *             o = o_win + gamma (mem_scale o_mem - o_win). mix == 0: o = o_win.
 * Layouts: q, k, v given by element strides (batch, head, token) with D contiguous: q over the H = G*R query heads,
 * k and v over the G KV heads (e.g. q [B][H][T][D] -> strides (H*T*D, T*D, D); v [B][T][G][D] -> (T*G*D, D, G*D)).
 * ring_k/ring_v [B][G][W][D], ring_pos [W] int64, sink_k/sink_v [B][G][n_sinks][D], all in in_dtype.
 * o_mem [B][T][H][D] in o_mem_dtype (fp32 or bf16), z [B][T][H] f32, mix_lse/mem_scale [H] f32; o [B][T][H][D] in o_dtype; lse [B][H][T] f32 or
 * null. Arithmetic: MFMA in in_dtype (bf16 probabilities for bf16 inputs) with fp32 accumulation and softmax.
 */
int bf_window_fwd(int B, int G, int R, int D, int T, int W, int sinks, int64_t start, int in_dtype, const void* q,
                  int64_t q_sb, int64_t q_sh, int64_t q_st, const void* k, int64_t k_sb, int64_t k_sh, int64_t k_st,
                  const void* v, int64_t v_sb, int64_t v_sh, int64_t v_st, const void* ring_k, const void* ring_v,
                  const int64_t* ring_pos, const void* sink_k, const void* sink_v, int n_sinks, int mix,
                  const void* o_mem, int o_mem_dtype, const float* z, const float* mix_lse, const float* mem_scale,
                  void* o,
                  int o_dtype, float* lse, void* stream);

/*
 * Memory-branch keys of the converted layer, bf16 activations:
 *     out[t][h] = scale * normalize(x[t][h] F_h),   normalize(u) = u / max(||u||_2, 1e-12)
 * Replaces the two projections of HybridAttention._mem_inputs (Heimdall/heimdall/hibrit.py:327-334):
 * qm = normalize(q_h fq_h) * D^-1/2 (x = q, scale = D^-1/2) and km = normalize(k_g fk_g) (x = k, scale = 1).
 *
 *   x: bf16, token t / head h at x + t * x_st + h * x_sh elements, D contiguous; n_tok tokens, nh heads
 *   f [nh][D][D] f32: the projections as the module holds them (fq, fk), f[h][i][j] = F_h[i][j]
 *   out [n_tok][nh][D] in out_dtype (bf16 or f32)
 * Arithmetic: F_h rounded to bf16 (nearest even), bf16 MFMA with fp32 accumulation, norm and scale in fp32.
 * in_dtype must be BF_DTYPE_BF16 (fp32 runs keep the reference's fp32 projections).
 */
int bf_mem_project(const void* x, int64_t n_tok, int nh, int D, int64_t x_st, int64_t x_sh, const float* f,
                   float scale, void* out, int in_dtype, int out_dtype, void* stream);

/*
 * Memory-branch gates of the converted layer, replacing the gate lines of HybridAttention._mem_inputs
 * (Heimdall/heimdall/hibrit.py:331-333):
 *     g[i][j]    = -exp(A_log[j]) * softplus(ab[i][j] + dt_bias[j]) * decay_mask[j]     (softplus threshold 20)
 *     beta[i][j] = sigmoid(ab[i][G + j]) * [pos_i >= sinks],   pos_i = start + i mod T
 *   ab: f32 rows of the ab projection (x W_ab^T + b_ab, columns [a | b], 2G wide) at ab + i * ab_st for the
 *   n_tok = B * T tokens (T tokens per sequence); A_log, dt_bias, decay_mask [G] f32; g, beta [n_tok][G] f32.
 */
int bf_mem_gates(const float* ab, int64_t n_tok, int64_t T, int G, int64_t ab_st, const float* A_log,
                 const float* dt_bias, const float* decay_mask, int64_t start, int sinks, float* g, float* beta,
                 void* stream);

/*
 * Gate projections of the converted layer for bf16 activations: the two small Linear layers applied to x,
 *     out0[t] = x_t W0^T + b0   (ab(x), HybridAttention._mem_inputs, Heimdall/heimdall/hibrit.py:330)
 *     out1[t] = x_t W1^T + b1   (mix(x), the gamma logit, hibrit.py:409)
 * in one pass over x.
 *   x: bf16 rows, token t at x + t * x_st elements, d contiguous, d a multiple of 8, 16-byte aligned rows
 *   w0 [n0][d], w1 [n1][d] f32; b0 [n0], b1 [n1] f32 or null; out0 [n_tok][n0], out1 [n_tok][n1] f32;
 *   n0 + n1 <= 64 (n1 may be 0)
 * Arithmetic: x exact (bf16), W as bf16 high + low parts (relative residual <= 2^-18), fp32 accumulation: the fp32
 * product to ~4e-6 relative (the reference runs these layers under bf16 autocast, i.e. with W rounded to bf16).
 * Workspace: bf_gate_project_workspace_size(n_tok, d, n0 + n1) bytes, always required. Up to 4096 tokens the d range
 * is split over workgroups and the partial sums are added in a fixed order, so results are reproducible. Above that
 * it holds W split into bf16 high and low parts (4 bytes per weight, with d rounded up to a multiple of 256 and
 * n0 + n1 to a multiple of 16), which the call writes before it reads x.
 */
int bf_gate_project_workspace_size(int64_t n_tok, int d, int nout, size_t* bytes);

int bf_gate_project(const void* x, int64_t n_tok, int d, int64_t x_st, const float* w0, const float* b0, int n0,
                    float* out0, const float* w1, const float* b1, int n1, float* out1, void* workspace,
                    size_t workspace_bytes, void* stream);

/*
 * Native Gated DeltaNet layer, the pass before the delta rule: GatedDeltaNet.forward up to delta_rule
 * (Heimdall/heimdall/hibrit.py:159-179) with causal_conv (Heimdall/heimdall/kernels.py:29-37) and l2norm
 * (hibrit.py:132-133), for packed sequences.
 *   y = SiLU(causal depthwise conv of z), y_c[t] = sum_j conv_w[c][K-1-j] z[t-j][c], rows before a sequence's first
 *       token taken from `prefix` (the reference's cache["conv"]) or zero;
 *   q_h = q_scale * l2norm(y_q[h / r]), k_h = l2norm(y_k[h / r]), v_h = y_v[h] for the HV value heads (r = HV / HK,
 *       the reference's repeat_interleave), l2norm(x) = x / sqrt(sum x^2 + eps);
 *   beta = sigmoid(b), g = -exp(A_log) * softplus(a + dt_bias) (softplus threshold 20).
 * Layouts: z [n_tok][C] in in_dtype with C = (2 HK + HV) D channels ordered [q | k | v] and z_st >= C elements
 * between tokens; prefix [num_seqs][K-1][C] in in_dtype or null; conv_w [C][K] f32 (column K-1 = the current token); a, b
 * [n_tok][HV] f32; A_log, dt_bias [HV] f32; cu_seqlens [num_seqs + 1] int32 (device); q, k, v [n_tok][HV][D] in
 * out_dtype; g, beta [n_tok][HV] f32. D_k = D_v = D. z, prefix, conv_w, q, k, v 16-byte aligned and z_st a multiple
 * of 8. The new conv cache (the last K-1 rows of [prefix; z] per
 * sequence) is the caller's slice.
 */
int bf_gdn_conv_inputs(const void* z, int64_t z_st, const void* prefix, int in_dtype, const float* conv_w, int K,
                       const float* a, const float* b, const float* A_log, const float* dt_bias,
                       const int32_t* cu_seqlens, int num_seqs, int64_t n_tok, int HK, int HV, int D, float eps,
                       float q_scale, void* q, void* k, void* v, float* g, float* beta, int out_dtype, void* stream);

/*
 * GatedNorm of the native layer's output (Heimdall/heimdall/hibrit.py:118-129, applied at :183), per row of D:
 *   io_dtype fp32: out = w * o * rsqrt(mean(o^2) + eps) * SiLU(z);
 *   io_dtype bf16: out = bf16(bf16(w * bf16(o_b * rsqrt(mean(o_b^2) + eps))) * SiLU(z)), o_b = o rounded to bf16
 *                  (the rounding points of the reference's bf16 layer).
 * o [rows][D] in o_dtype, z [rows][D] and out [rows][D] in io_dtype (o, z, out 16-byte aligned), w [D] f32.
 */
int bf_gated_norm(const void* o, int o_dtype, const void* z, const float* w, int64_t rows, int D, float eps,
                  void* out, int io_dtype, void* stream);

/*
 * The native layer's delta rule and GatedNorm in one call (Heimdall/heimdall/hibrit.py:180-183: delta_rule, then
 * self.norm(o, z)), for a bf16 layer with D <= 128: bf_gdn_fwd with in_dtype = o_dtype = bf16, whose output row of
 * each (token, head) goes through bf_gated_norm's bf16 arithmetic before it is stored, so out holds the same bits as
 * bf_gdn_fwd into o followed by bf_gated_norm(o, BF16, norm_z, norm_w, ..., out, BF16); o itself is never written.
 *   norm_z [N_tok][G*R][D] bf16 (the z_g rows), norm_w [D] f32, out [N_tok][G*R][D] bf16 (norm_z, out 16-byte aligned);
 *   the other arguments, the workspace (bf_gdn_workspace_size with in_dtype bf16) and the phases as for bf_gdn_fwd.
 * BF_STATUS_UNSUPPORTED for D = 256 (a head's row spans two of the output scan's workgroups there).
 */
int bf_gdn_fwd_gated(const void* q, const void* k, const void* v, const float* g, const float* beta,
                     const int32_t* cu_seqlens, int num_seqs, int64_t total_tokens, int G, int R, int D,
                     float scale, const float* initial_state, const void* norm_z, const float* norm_w,
                     float norm_eps, void* out, float* final_state, int segment_chunks, void* workspace,
                     size_t workspace_bytes, int phases, void* stream);

/*
 * One prefill chunk of the converted layer: HybridAttention._student with t > 1 (Heimdall/heimdall/hibrit.py:363-424)
 * on the student cache, in one call: the delta-rule write stream (the ring rows leaving the window, then the chunk's
 * own rows; from an empty cache the chunk shifted by W), bf_gdn_fwd on it from the cached state, bf_window_fwd with
 * the gamma mix (memory active when memory != 0 and start + T > W), then the write-back of the last min(T, W) tokens
 * into the ring (slot = position mod W, ring_pos) and of the new state. qr, kr, v as bf_window_fwd (in_dtype, element
 * strides); qm [B][T][H][D] and km [B][T][G][D] in qm_dtype / km_dtype (normalised, qm scaled by 1/sqrt(D)); g, beta
 * [B][T][G] f32; z [B][T][H] f32 (mix logits); mix_lse, mem_scale [H]; sink_k / sink_v [B][G][n_sinks][D] already
 * holding this chunk's sinks; ring_k / ring_v [B][G][W][D] in in_dtype, ring_km [B][W][G][D], ring_g / ring_beta
 * [B][W][G], ring_pos [W], state [B][G][D][D] f32 (state_valid 0: no state yet) — all updated in place. o [B][T][H][D]
 * f32, lse [B][H][T] f32 or null. Workspace from bf_layer_prefill_workspace_size, 256-byte aligned.
 */
int bf_layer_prefill_workspace_size(int B, int G, int R, int D, int T, int in_dtype, size_t* bytes);
int bf_layer_prefill_fwd(int B, int G, int R, int D, int T, int W, int sinks, int64_t start, int memory, int in_dtype,
                         const void* qr, int64_t q_sb, int64_t q_sh, int64_t q_st, const void* kr, int64_t k_sb,
                         int64_t k_sh, int64_t k_st, const void* v, int64_t v_sb, int64_t v_sh, int64_t v_st,
                         const void* qm, int qm_dtype, const void* km, int km_dtype, const float* g,
                         const float* beta, const float* z, const float* mix_lse, const float* mem_scale,
                         const void* sink_k, const void* sink_v, int n_sinks, void* ring_k, void* ring_v,
                         float* ring_km, float* ring_g, float* ring_beta, int64_t* ring_pos, float* state,
                         int state_valid, float* o, float* lse, void* workspace, size_t workspace_bytes,
                         void* stream);

/*
 * The llama.cpp per-sequence Bifrost state row (Heimdall/llamacpp/bifrost.patch:221-239, the views of
 * build_layer_bifrost :1000-1013) <-> the student cache (sink_k, sink_v, ring_k, ring_v, ring_km, ring_g, ring_beta,
 * ring_pos, S of HybridAttention._student, Heimdall/heimdall/hibrit.py:363-424), so a llama.cpp build and these
 * kernels can hand sequences to each other. Row (f32, bf_llama_state_floats floats): region [LR][C] (LR =
 * ceil((S + W + 2) / 32) * 32 slots: sinks, ring slot S + p mod (W + 1), scratch; C = 3 G D + 2 G channels
 * [k_rope | v | k_mem | g | beta]), K plane [G][LR][D], transposed V plane [G][D][LR], delta [G][dv][dk].
 * Cache layouts as bf_decode_fwd (ring of W slots, slot p mod W), n = tokens seen, n_sinks sink rows (unpack:
 * min(S, n)), state [B][G][D][D] f32. Rows [B][floats]. A sink slot's k_mem / g / beta are packed from the ring while
 * the sink is still in it, else 0 (never read by the layer).
 */
int bf_llama_state_floats(int G, int D, int W, int S, int64_t* floats);
int bf_llama_state_pack(int B, int G, int D, int W, int S, int64_t n, int kv_dtype, const void* ring_k,
                        const void* ring_v, const float* ring_km, const float* ring_g, const float* ring_beta,
                        const int64_t* ring_pos, const void* sink_k, const void* sink_v, int n_sinks,
                        const float* state, float* rows, void* stream);
int bf_llama_state_unpack(int B, int G, int D, int W, int S, int64_t n, int kv_dtype, const float* rows, void* ring_k,
                          void* ring_v, float* ring_km, float* ring_g, float* ring_beta, int64_t* ring_pos,
                          void* sink_k, void* sink_v, int n_sinks, float* state, void* stream);

/*
 * Backward of the chunked GQA gated delta rule: the gradients that autograd takes through motor.delta_rule_gqa
 * (Heimdall/heimdall/motor.py:70-102) in the conversion training's loss (motor.seq_loss, :149-193), fp32 like the
 * reference's training path. Inputs as bf_gdn_fwd with fp32 q, k, v for num_seqs sequences of seq_len tokens each
 * (seq_len a multiple of 64; pad with zeros and g = beta = 0 as the reference does): q, dO [N][G*R][D], k, v
 * [N][G][D], g, beta [N][G], s0 and ds_final [num_seqs][G][D][D] or null (zero), o = forward(q * scale, ...). dO is
 * the gradient of o, ds_final that of the final state. Writes dq, dk, dv [same layouts], dg, dbeta [N][G] and, if
 * non-null, ds0 [num_seqs][G][D][D]. Pointers 16-byte aligned; workspace from bf_gdn_bwd_workspace_size, 256-byte
 * aligned.
 */
int bf_gdn_bwd_workspace_size(int num_seqs, int64_t seq_len, int G, int R, int D, size_t* bytes);
int bf_gdn_bwd(const float* q, const float* k, const float* v, const float* g, const float* beta, const float* s0,
               float scale, const float* dO, const float* ds_final, int num_seqs, int64_t seq_len, int G, int R, int D,
               float* dq, float* dk, float* dv, float* dg, float* dbeta, float* ds0, void* workspace,
               size_t workspace_bytes, void* stream);

/*
 * Attention of the kept full-attention layers over a dense KV cache, for the T most recent queries of each sequence
 * (T = 1: one decode step), with optional retrieval (Quest-style block selection): HybridAttention._teacher
 * (Heimdall/heimdall/hibrit.py:275-290) and _retrieval_mask (:301-324). Key (b, g) row of position p at
 * k + (b * G + g) * k_sbg + p * k_st (elements; v likewise, D contiguous); the cache holds positions 0 .. n - 1 and
 * query i of a sequence sits at position p = n - T + i. With S = sinks, W = window, L = block length, block j holds the
 * keys S + j L .. S + j L + L - 1 and nb = (n - S) / L.
 *   retrieval == 0: query p attends to the keys 0 .. p.
 *   retrieval != 0: query p attends to the keys 0 .. S - 1, the selected blocks (sel) among its candidates
 *                   j < nc = min(max(p - W + 1 - S, 0) / L, nb), and the window S + nc L .. p.
 *
 * bf_kv_block_summary: per-dimension key min / max of blocks [first_block, nb) into kmin / kmax, in the key dtype
 *   (exact: each is one of the key values) with the layout [B][G][D / GS][nb_cap][GS], GS = 16 bytes / element (dims
 *   GS c .. GS c + GS - 1 of block j at ((b G + g) D / GS + c) nb_cap + j); a growing cache summarises only its new
 *   full blocks.
 * bf_kv_select: per (b, query, g), the K candidate blocks with the highest upper bound
 *   max_r sum_d max(q_rd kmin_jd, q_rd kmax_jd) (fp32) over the R query heads of the KV head, into sel [B][T][G][K]
 *   int32 in descending bound order (-1 past the candidates; ties to the lower block id). K <= 64, nb <= 16384. q and
 *   the summaries share dtype. bf_kv_attention reads the valid ids of sel in any order.
 * bf_kv_attention: softmax(q . k * scale) v per query head over the attended keys. q [B][T][G*R][D] in dtype, o
 *   [B][T][G*R][D] in o_dtype; sel as bf_kv_select wrote it (retrieval only); workspace from
 *   bf_kv_attention_workspace_size with the same geometry.
 * q, k, v, kmin, kmax 16-byte aligned; k / v strides multiples of 8 elements. R <= 8.
 */
/* bf_kv_append: the t new rows k_new / v_new (row (b, g, i) at b k_sb + g k_sg + i k_st elements) written to
 * positions n0 .. n0 + t - 1 of the cache buffers k_buf / v_buf [B][G][cap][D] (the torch.cat of _teacher,
 * hibrit.py:277-279, into preallocated capacity). One launch for both tensors. */
int bf_kv_append(const void* k_new, int64_t k_sb, int64_t k_sg, int64_t k_st, const void* v_new, int64_t v_sb,
                 int64_t v_sg, int64_t v_st, int dtype, int B, int G, int t, int D, void* k_buf, void* v_buf,
                 int64_t cap, int64_t n0, void* stream);
int bf_kv_block_summary(const void* k, int dtype, int B, int G, int D, int64_t k_sbg, int64_t k_st, int sinks, int L,
                        int first_block, int nb, int nb_cap, void* kmin, void* kmax, void* stream);
int bf_kv_select(const void* q, int dtype, int B, int T, int G, int R, int D, int64_t n, int sinks, int window, int L,
                 const void* kmin, const void* kmax, int nb_cap, int K, int* sel, void* stream);
int bf_kv_attention_workspace_size(int B, int T, int G, int R, int D, int64_t n, int retrieval, int sinks, int window,
                                   int L, int K, size_t* bytes);
int bf_kv_attention(const void* q, const void* k, const void* v, int dtype, int B, int T, int G, int R, int D,
                    int64_t n, int64_t k_sbg, int64_t k_st, int64_t v_sbg, int64_t v_st, int retrieval, int sinks,
                    int window, int L, const int* sel, int K, float scale, void* workspace, size_t workspace_bytes,
                    void* o, int o_dtype, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* BIFROST_H */
