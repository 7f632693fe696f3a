// C-ABI entry points of libbifrost_hip.so: argument checks, workspace carve-up, dispatch to the kernels.
#include <hip/hip_runtime.h>

#include <mutex>

#include "bf_internal.h"

// The scratch of the allocation-free decode entry point: one copy of this array on every GPU the library runs on,
// held until the process ends. Host code never uses its name as an address: the device address comes from
// hipGetSymbolAddress, once per device (scratch_on_current_device).
static __device__ __align__(256) unsigned char scratch[BF_DECODE_STATIC_SCRATCH_BYTES];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// Device address of `scratch` on the current device, looked up on the first call there (with that device current).
int scratch_on_current_device(void** out) {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return (int)e;
    if (dev < 0 || dev >= kMaxDevices) return BF_STATUS_UNSUPPORTED;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return (int)e;
        if (!p) return BF_STATUS_INVALID;
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return BF_STATUS_OK;
}

constexpr int kChunk = 64;

size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

bool supported_dim(int D) { return D == 64 || D == 128 || D == 256; }
bool supported_dtype(int dt) { return dt == BF_DTYPE_F32 || dt == BF_DTYPE_BF16; }
size_t esize(int dt) { return dt == BF_DTYPE_BF16 ? 2 : 4; }

struct GdnLayout {
    size_t gcum, T, phi, c, n, sin, total;
    int max_chunks, seg_chunks, max_segs;
};

// Segment length (chunks) when the caller passes 0: the L that minimises a cost model of the three sequential-part
// kernels on an MI355X (256 CUs, one scan workgroup per CU), with per-chunk and per-step times measured at D = 256:
//   output   ceil(segments x G x D/128 / 256) rounds of L chunks, ~(4.6 + 2.8 R) us per chunk (R query heads per KV
//            head; 7.4 us at R = 1, 21.5 us at R = 6)
//   summary  ceil((segments - 1) x G x 2D/128 / 256) rounds of L chunks, ~3.7 us per chunk
//   combine  (segments - 1) sequential steps, ~2.1 us each
// Times scale with D^2 for the scan kernels and D^3 for the combine, which only shifts the balance for D < 256.
// The chunk count of the model is ceil(tokens / 64) + sequences - 1 (exact for one sequence; each further sequence
// adds at most one partial chunk), so that e.g. one sequence of 32768 tokens gets 32 segments of 16 chunks: one
// round of 256 output workgroups at G = 4. Short streams (a 2048-token chunk of a long prompt at R = 6) get L = 2:
// measured 5.9 ms per 32768-token prefill as 16 such calls, against 6.2 ms at L = 4 and 6.25 ms at L = 1.
constexpr int kSegMinChunks = 2;

int model_chunks(int64_t total_tokens, int num_seqs) { return (int)((total_tokens + kChunk - 1) / kChunk) + num_seqs - 1; }

int auto_segment_chunks(int max_chunks, int G, int R, int D) {
    const double f = (double)D / 256.0;
    const double t_out = (4.6 + 2.8 * R) * f * f, t_sum = 3.7 * f * f, t_comb = 2.1 * f * f * f;
    const int cg = D >= 128 ? D / 128 : 1;
    int best_L = max_chunks > kSegMinChunks ? max_chunks : kSegMinChunks;
    double best = 1e300;
    for (int L = kSegMinChunks; L <= (max_chunks > kSegMinChunks ? max_chunks : kSegMinChunks); ++L) {
        const long nseg = (max_chunks + L - 1) / L;
        const long out_rounds = (nseg * G * cg + 255) / 256;
        const long sum_rounds = ((nseg - 1) * G * 2 * cg + 255) / 256;
        const double t = out_rounds * L * t_out + sum_rounds * L * t_sum + (nseg - 1) * t_comb;
        if (t < best - 1e-9) {
            best = t;
            best_L = L;
        }
    }
    return best_L;
}

GdnLayout gdn_layout(int64_t total_tokens, int num_seqs, int G, int R, int D, int in_dtype, int segment_chunks) {
    GdnLayout L;
    // every sequence contributes ceil(len / C) chunks: at most total/C + num_seqs overall
    L.max_chunks = (int)(total_tokens / kChunk) + num_seqs;
    L.seg_chunks = segment_chunks > 0 ? segment_chunks
                                      : auto_segment_chunks(model_chunks(total_tokens, num_seqs), G, R, D);
    // every sequence contributes max(1, ceil(chunks / L)) segments
    L.max_segs = (L.max_chunks + L.seg_chunks - 1) / L.seg_chunks + num_seqs;
    const size_t nc = (size_t)L.max_chunks, ns = (size_t)L.max_segs, e = esize(in_dtype);
    size_t off = 0;
    L.gcum = off; off = align256(off + nc * G * kChunk * sizeof(float));
    L.T = off;    off = align256(off + nc * G * kChunk * kChunk * e);
    L.phi = off;  off = align256(off + ns * G * D * D * e);
    L.c = off;    off = align256(off + ns * G * sizeof(float));
    L.n = off;    off = align256(off + ns * G * D * D * sizeof(float));
    L.sin = off;  off = align256(off + ns * G * D * D * sizeof(float));
    L.total = off;
    return L;
}

}  // namespace

extern "C" {

int bf_version(void) { return 100; }

const char* bf_status_string(int status) {
    switch (status) {
        case BF_STATUS_OK: return "ok";
        case BF_STATUS_INVALID: return "invalid argument (null pointer, bad size or inconsistent shape)";
        case BF_STATUS_UNSUPPORTED: return "unsupported head dim, dtype or chunk size";
        case BF_STATUS_WORKSPACE: return "workspace missing or too small";
        case BF_STATUS_SCRATCH: return "problem larger than the static scratch of the allocation-free entry point";
        default: break;
    }
    return status > 0 ? hipGetErrorString((hipError_t)status) : "unknown status";
}

int bf_gdn_segment_chunks(int64_t total_tokens, int num_seqs, int G, int R, int D) {
    if (total_tokens < 0 || num_seqs <= 0 || G <= 0 || R <= 0) return BF_STATUS_INVALID;
    if (!supported_dim(D)) return BF_STATUS_UNSUPPORTED;
    return auto_segment_chunks(model_chunks(total_tokens, num_seqs), G, R, D);
}

int bf_gdn_workspace_size(int64_t total_tokens, int num_seqs, int G, int R, int D, int in_dtype,
                          int segment_chunks, size_t* bytes) {
    if (!bytes || total_tokens < 0 || num_seqs <= 0 || G <= 0 || R <= 0 || segment_chunks < 0)
        return BF_STATUS_INVALID;
    if (!supported_dim(D) || !supported_dtype(in_dtype)) return BF_STATUS_UNSUPPORTED;
    *bytes = gdn_layout(total_tokens, num_seqs, G, R, D, in_dtype, segment_chunks).total;
    return BF_STATUS_OK;
}

}  // extern "C"

namespace {

// bf_gdn_fwd, with the output scan's fused GatedNorm when gn_z is set (bf_gdn_fwd_gated)
int gdn_fwd(const void* q, const void* k, const void* v, const float* g, const float* beta, const int32_t* cu_seqlens,
            int num_seqs, int64_t total_tokens, int G, int R, int D, int in_dtype, float scale,
            const float* initial_state, void* o, int o_dtype, float* final_state, int segment_chunks, void* workspace,
            size_t workspace_bytes, int phases, const void* gn_z, const float* gn_w, float gn_eps, void* stream) {
    if (num_seqs <= 0 || total_tokens < 0 || G <= 0 || R <= 0 || segment_chunks < 0 ||
        (phases & ~BF_GDN_PHASE_ALL) || !phases)
        return BF_STATUS_INVALID;
    if (!supported_dim(D) || !supported_dtype(in_dtype) || !supported_dtype(o_dtype)) return BF_STATUS_UNSUPPORTED;
    if (!cu_seqlens && total_tokens % num_seqs) return BF_STATUS_INVALID;
    if (total_tokens > 0 && (!q || !k || !v || !g || !beta || !o)) return BF_STATUS_INVALID;
    const GdnLayout L = gdn_layout(total_tokens, num_seqs, G, R, D, in_dtype, segment_chunks);
    if (!workspace || workspace_bytes < L.total) return BF_STATUS_WORKSPACE;
    bf::GdnArgs a{};
    a.q = q; a.k = k; a.v = v; a.g = g; a.beta = beta;
    a.cu_seqlens = cu_seqlens;
    a.num_seqs = num_seqs;
    a.seq_len = cu_seqlens ? 0 : (int)(total_tokens / num_seqs);
    a.total_tokens = total_tokens;
    a.G = G; a.R = R; a.D = D;
    a.in_dtype = in_dtype; a.o_dtype = o_dtype;
    a.scale = scale;
    a.s0 = initial_state; a.o = o; a.s_out = final_state;
    a.max_chunks = L.max_chunks;
    a.seg_chunks = L.seg_chunks;
    a.max_segs = L.max_segs;
    // equal sequences: known segment count; packed sequences: any of them may be long
    a.multi_seg = cu_seqlens ? (L.max_chunks > L.seg_chunks)
                             : ((total_tokens / num_seqs + kChunk - 1) / kChunk > L.seg_chunks);
    char* ws = static_cast<char*>(workspace);
    a.ws_gcum = reinterpret_cast<float*>(ws + L.gcum);
    a.ws_T = ws + L.T;
    a.ws_phi = ws + L.phi;
    a.ws_c = reinterpret_cast<float*>(ws + L.c);
    a.ws_n = reinterpret_cast<float*>(ws + L.n);
    a.ws_sin = reinterpret_cast<float*>(ws + L.sin);
    a.gn_z = gn_z; a.gn_w = gn_w; a.gn_eps = gn_eps;
    if (total_tokens == 0 && !final_state) return BF_STATUS_OK;
    const hipStream_t st = static_cast<hipStream_t>(stream);
    int rc = 0;
    if ((phases & BF_GDN_PHASE_PREP) && total_tokens > 0 && (rc = bf::gdn_prep(a, st))) return rc;
    if ((phases & BF_GDN_PHASE_STATES) &&
        (rc = bf::gdn_states(a, st, phases & BF_GDN_PHASE_SUMMARY, phases & BF_GDN_PHASE_COMBINE)))
        return rc;
    if (phases & BF_GDN_PHASE_OUTPUT) return bf::gdn_output(a, st);
    return BF_STATUS_OK;
}

}  // namespace

extern "C" {

int bf_gdn_fwd(const void* q, const void* k, const void* v, const float* g, const float* beta,
               const int32_t* cu_seqlens, int num_seqs, int64_t total_tokens, int G, int R, int D, int in_dtype,
               float scale, const float* initial_state, void* o, int o_dtype, float* final_state,
               int segment_chunks, void* workspace, size_t workspace_bytes, int phases, void* stream) {
    return gdn_fwd(q, k, v, g, beta, cu_seqlens, num_seqs, total_tokens, G, R, D, in_dtype, scale, initial_state, o,
                   o_dtype, final_state, segment_chunks, workspace, workspace_bytes, phases, nullptr, nullptr, 0.f,
                   stream);
}

int bf_gdn_fwd_gated(const void* q, const void* k, const void* v, const float* g, const float* beta,
                     const int32_t* cu_seqlens, int num_seqs, int64_t total_tokens, int G, int R, int D,
                     float scale, const float* initial_state, const void* norm_z, const float* norm_w,
                     float norm_eps, void* out, float* final_state, int segment_chunks, void* workspace,
                     size_t workspace_bytes, int phases, void* stream) {
    if (D > 128) return BF_STATUS_UNSUPPORTED;
    if (total_tokens > 0 && (phases & BF_GDN_PHASE_OUTPUT) &&
        (!norm_z || !norm_w || ((uintptr_t)norm_z & 15) || ((uintptr_t)out & 15)))
        return BF_STATUS_INVALID;
    return gdn_fwd(q, k, v, g, beta, cu_seqlens, num_seqs, total_tokens, G, R, D, BF_DTYPE_BF16, scale,
                   initial_state, out, BF_DTYPE_BF16, final_state, segment_chunks, workspace, workspace_bytes, phases,
                   norm_z, norm_w, norm_eps, stream);
}

int bf_gdn_step(const float* q, const float* k, const float* v, const float* g, const float* beta,
                const float* state_in, float* state_out, float* o, int B, int G, int R, int D, void* stream) {
    if (B <= 0 || G <= 0 || R <= 0 || R > 8) return BF_STATUS_INVALID;
    if (!supported_dim(D)) return BF_STATUS_UNSUPPORTED;
    if (!q || !k || !v || !g || !beta || !state_in || !state_out || !o) return BF_STATUS_INVALID;
    bf::StepArgs a{};
    a.B = B; a.G = G; a.R = R; a.D = D;
    a.q = q; a.k = k; a.v = v; a.g = g; a.beta = beta;
    a.s_in = state_in; a.s_out = state_out; a.o = o;
    return bf::step_dispatch(a, static_cast<hipStream_t>(stream));
}

int bf_decode_workspace_size(int B, int G, int R, int D, int W, size_t* bytes) {
    if (!bytes || B <= 0 || G <= 0 || R <= 0 || W <= 0) return BF_STATUS_INVALID;
    if (!supported_dim(D) || R > 8) return BF_STATUS_UNSUPPORTED;
    int nsplit = 0, slots = 0;
    bf::decode_split(B, G, W, nsplit, slots);
    *bytes = align256((size_t)B * G * R * D * sizeof(float)) +
             align256((size_t)B * G * nsplit * R * (D + 2) * sizeof(float)) +
             align256((size_t)B * G * (2 * D + 4) * sizeof(float));
    return BF_STATUS_OK;
}

int bf_decode_fwd(int B, int G, int R, int D, int W, int sinks, int64_t pos, int memory, int kv_dtype, int q_dtype,
                  const void* qr, const float* qm, const void* kr, const void* v, const float* km, const float* g_new,
                  const float* beta_new, const float* z, const float* mix_lse, const float* mem_scale,
                  const void* sink_k, const void* sink_v, int n_sinks, void* ring_k, void* ring_v, float* ring_km,
                  float* ring_g, float* ring_beta, int64_t* ring_pos, float* state, float* o, float* lse,
                  void* workspace, size_t workspace_bytes, void* stream) {
    if (B <= 0 || G <= 0 || R <= 0 || W <= 0 || sinks < 0 || pos < 0) return BF_STATUS_INVALID;
    if (!supported_dim(D) || R > 8 || !supported_dtype(kv_dtype) || !supported_dtype(q_dtype))
        return BF_STATUS_UNSUPPORTED;
    if (n_sinks < 0 || n_sinks > 63 || n_sinks > sinks || (n_sinks > 0 && (!sink_k || !sink_v)))
        return BF_STATUS_INVALID;
    if (!qr || !kr || !v || !km || !g_new || !beta_new || !ring_k || !ring_v || !ring_km || !ring_g || !ring_beta ||
        !ring_pos || !o)
        return BF_STATUS_INVALID;
    const int mem_on = memory && pos >= W;
    if (mem_on && (!qm || !z || !mix_lse || !mem_scale || !state)) return BF_STATUS_INVALID;
    size_t need = 0;
    const int st = bf_decode_workspace_size(B, G, R, D, W, &need);
    if (st) return st;
    if (!workspace || workspace_bytes < need) return BF_STATUS_WORKSPACE;
    bf::DecodeArgs a{};
    a.B = B; a.G = G; a.R = R; a.D = D; a.W = W; a.sinks = sinks; a.pos = pos; a.mem_on = mem_on;
    a.kv_dtype = kv_dtype; a.q_dtype = q_dtype;
    a.qr = qr; a.qm = qm; a.kr = kr; a.v = v; a.km = km; a.g_new = g_new; a.beta_new = beta_new;
    a.z = z; a.mix_lse = mix_lse; a.mem_scale = mem_scale;
    a.sink_k = const_cast<void*>(sink_k); a.sink_v = const_cast<void*>(sink_v); a.n_sinks = n_sinks;
    a.ring_k = ring_k; a.ring_v = ring_v; a.ring_km = ring_km; a.ring_g = ring_g; a.ring_beta = ring_beta;
    a.ring_pos = ring_pos; a.state = state; a.o = o; a.lse = lse;
    bf::decode_split(B, G, W, a.nsplit, a.slots);
    char* ws = static_cast<char*>(workspace);
    a.ws_om = reinterpret_cast<float*>(ws);
    a.ws_part = reinterpret_cast<float*>(ws + align256((size_t)B * G * R * D * sizeof(float)));
    a.ws_ev = reinterpret_cast<float*>(reinterpret_cast<char*>(a.ws_part) +
                                       align256((size_t)B * G * a.nsplit * R * (D + 2) * sizeof(float)));
    return bf::decode_dispatch(a, static_cast<hipStream_t>(stream));
}

int bf_decode_fwd_batch(int B, int G, int R, int D, int W, int sinks, const int64_t* pos, int memory, int kv_dtype,
                        int q_dtype, const void* qr, const float* qm, const void* kr, const void* v, const float* km,
                        const float* g_new, const float* beta_new, const float* z, const float* mix_lse,
                        const float* mem_scale, void* sink_k, void* sink_v, void* ring_k, void* ring_v, float* ring_km,
                        float* ring_g, float* ring_beta, int64_t* ring_pos, float* state, float* o, float* lse,
                        void* workspace, size_t workspace_bytes, void* stream) {
    if (B <= 0 || G <= 0 || R <= 0 || W <= 0 || sinks < 0 || sinks > 63 || !pos) return BF_STATUS_INVALID;
    if (!supported_dim(D) || R > 8 || !supported_dtype(kv_dtype) || !supported_dtype(q_dtype))
        return BF_STATUS_UNSUPPORTED;
    if (sinks > 0 && (!sink_k || !sink_v)) return BF_STATUS_INVALID;
    if (!qr || !kr || !v || !km || !g_new || !beta_new || !ring_k || !ring_v || !ring_km || !ring_g || !ring_beta ||
        !ring_pos || !o)
        return BF_STATUS_INVALID;
    // the positions live on the device: any sequence may read its memory, so its inputs must be given
    if (memory && (!qm || !z || !mix_lse || !mem_scale || !state)) return BF_STATUS_INVALID;
    size_t need = 0;
    const int st = bf_decode_workspace_size(B, G, R, D, W, &need);
    if (st) return st;
    if (!workspace || workspace_bytes < need) return BF_STATUS_WORKSPACE;
    bf::DecodeArgs a{};
    a.B = B; a.G = G; a.R = R; a.D = D; a.W = W; a.sinks = sinks; a.pos = 0; a.pos_arr = pos; a.mem_on = memory != 0;
    a.kv_dtype = kv_dtype; a.q_dtype = q_dtype;
    a.qr = qr; a.qm = qm; a.kr = kr; a.v = v; a.km = km; a.g_new = g_new; a.beta_new = beta_new;
    a.z = z; a.mix_lse = mix_lse; a.mem_scale = mem_scale;
    a.sink_k = sink_k; a.sink_v = sink_v; a.n_sinks = sinks;
    a.ring_k = ring_k; a.ring_v = ring_v; a.ring_km = ring_km; a.ring_g = ring_g; a.ring_beta = ring_beta;
    a.ring_pos = ring_pos; a.state = state; a.o = o; a.lse = lse;
    bf::decode_split(B, G, W, a.nsplit, a.slots);
    char* ws = static_cast<char*>(workspace);
    a.ws_om = reinterpret_cast<float*>(ws);
    a.ws_part = reinterpret_cast<float*>(ws + align256((size_t)B * G * R * D * sizeof(float)));
    a.ws_ev = reinterpret_cast<float*>(reinterpret_cast<char*>(a.ws_part) +
                                       align256((size_t)B * G * a.nsplit * R * (D + 2) * sizeof(float)));
    return bf::decode_dispatch(a, static_cast<hipStream_t>(stream));
}

// One decode step of the converted layer from the layer's own inputs (bf16 activations): the gate projections, the
// memory projections and gates, then the decode kernels, on one stream and one workspace. Intermediates (ab, z, qm,
// km, g, beta: the same values the separate entry points produce) sit at the head of the workspace, the decode
// workspace after them.
namespace {
struct StudentDecodeWs {
    size_t ab, z, qm, km, g, beta, gp, dec, total;
};
int student_decode_layout(int B, int H, int G, int D, int W, int d_model, StudentDecodeWs& l) {
    if (B <= 0 || G <= 0 || H <= 0 || H % G || W <= 0 || d_model <= 0) return BF_STATUS_INVALID;
    size_t dec = 0;
    const int st = bf_decode_workspace_size(B, G, H / G, D, W, &dec);
    if (st) return st;
    size_t o = 0;
    auto take = [&](size_t n) { const size_t at = o; o += align256(n); return at; };
    l.ab = take((size_t)B * 2 * G * sizeof(float));
    l.z = take((size_t)B * H * sizeof(float));
    l.qm = take((size_t)B * H * D * sizeof(float));
    l.km = take((size_t)B * G * D * sizeof(float));
    l.g = take((size_t)B * G * sizeof(float));
    l.beta = take((size_t)B * G * sizeof(float));
    l.gp = take(bf::gate_project_workspace(B, d_model, 2 * G + H));
    l.dec = take(dec);
    l.total = o;
    return BF_STATUS_OK;
}
}  // namespace

int bf_student_decode_workspace_size(int B, int H, int G, int D, int W, int d_model, size_t* bytes) {
    if (!bytes) return BF_STATUS_INVALID;
    StudentDecodeWs l{};
    const int st = student_decode_layout(B, H, G, D, W, d_model, l);
    if (st) return st;
    *bytes = l.total;
    return BF_STATUS_OK;
}

int bf_student_decode(int B, int H, int G, int D, int W, int sinks, int64_t pos, const int64_t* pos_arr, int memory,
                      int d_model, const void* x, const void* q, const void* k, const void* v, const void* qr,
                      const void* kr, const float* fq, const float* fk, const float* w_ab, const float* b_ab,
                      const float* w_mix, const float* b_mix, const float* A_log, const float* dt_bias,
                      const float* decay_mask, const float* mix_lse, const float* mem_scale, void* sink_k,
                      void* sink_v, int n_sinks, void* ring_k, void* ring_v, float* ring_km, float* ring_g,
                      float* ring_beta, int64_t* ring_pos, float* state, float* o, void* workspace,
                      size_t workspace_bytes, void* stream) {
    StudentDecodeWs l{};
    int st = student_decode_layout(B, H, G, D, W, d_model, l);
    if (st) return st;
    if (!supported_dim(D)) return BF_STATUS_UNSUPPORTED;
    if (d_model <= 0 || d_model % 8 || 2 * G + H > bf::GP_MAX_OUT || sinks < 0 || sinks > 63 || (!pos_arr && pos < 0))
        return BF_STATUS_INVALID;
    if (!x || !q || !k || !v || !qr || !kr || !fq || !fk || !w_ab || !w_mix || !A_log || !dt_bias || !decay_mask ||
        !mix_lse || !mem_scale || !ring_k || !ring_v || !ring_km || !ring_g || !ring_beta || !ring_pos || !o)
        return BF_STATUS_INVALID;
    auto al16 = [](const void* p) { return ((uintptr_t)p & 15) == 0; };
    if (!al16(x) || !al16(w_ab) || !al16(w_mix)) return BF_STATUS_INVALID;
    if (!workspace || workspace_bytes < l.total) return BF_STATUS_WORKSPACE;
    char* ws = static_cast<char*>(workspace);
    float *ab = reinterpret_cast<float*>(ws + l.ab), *z = reinterpret_cast<float*>(ws + l.z);
    float *qm = reinterpret_cast<float*>(ws + l.qm), *km = reinterpret_cast<float*>(ws + l.km);
    float *g = reinterpret_cast<float*>(ws + l.g), *beta = reinterpret_cast<float*>(ws + l.beta);
    const hipStream_t s = static_cast<hipStream_t>(stream);
    {
        bf::GateProjArgs a{};
        a.x = static_cast<const uint16_t*>(x); a.n_tok = B; a.x_st = d_model; a.d = d_model;
        a.w0 = w_ab; a.b0 = b_ab; a.n0 = 2 * G; a.out0 = ab; a.w1 = w_mix; a.b1 = b_mix; a.n1 = H; a.out1 = z;
        a.part = reinterpret_cast<float*>(ws + l.gp);
        if ((st = bf::gate_project_dispatch(a, s))) return st;
    }
    {
        bf::MemProjArgs a{};
        a.x = q; a.n_tok = B; a.nh = H; a.D = D; a.x_st = (long)H * D; a.x_sh = D;
        a.f = fq; a.scale = 1.f / sqrtf((float)D); a.out = qm; a.out_dtype = BF_DTYPE_F32;
        if ((st = bf::mem_project_dispatch(a, s))) return st;
        a.x = k; a.nh = G; a.x_st = (long)G * D; a.f = fk; a.scale = 1.f; a.out = km;
        if ((st = bf::mem_project_dispatch(a, s))) return st;
    }
    {
        bf::MemGatesArgs a{};
        a.ab = ab; a.n_tok = B; a.T = 1; a.ab_st = 2 * G; a.G = G; a.sinks = sinks; a.start = pos_arr ? 0 : pos;
        a.pos_arr = pos_arr; a.A_log = A_log; a.dt_bias = dt_bias; a.decay_mask = decay_mask; a.g = g; a.beta = beta;
        if ((st = bf::mem_gates_dispatch(a, s))) return st;
    }
    void* dws = ws + l.dec;
    const size_t dn = workspace_bytes - l.dec;
    if (pos_arr)
        return bf_decode_fwd_batch(B, G, H / G, D, W, sinks, pos_arr, memory, BF_DTYPE_BF16, BF_DTYPE_BF16, qr, qm,
                                   kr, v, km, g, beta, z, mix_lse, mem_scale, sink_k, sink_v, ring_k, ring_v, ring_km,
                                   ring_g, ring_beta, ring_pos, state, o, nullptr, dws, dn, stream);
    return bf_decode_fwd(B, G, H / G, D, W, sinks, pos, memory, BF_DTYPE_BF16, BF_DTYPE_BF16, qr, qm, kr, v, km, g,
                         beta, z, mix_lse, mem_scale, sink_k, sink_v, n_sinks, ring_k, ring_v, ring_km, ring_g,
                         ring_beta, ring_pos, state, o, nullptr, dws, dn, stream);
}

int bf_decode_fwd_noalloc(int B, int G, int R, int D, int W, int sinks, int64_t pos, int memory, int kv_dtype,
                          int q_dtype, const void* qr, const float* qm, const void* kr, const void* v, const float* km,
                          const float* g_new, const float* beta_new, const float* z, const float* mix_lse,
                          const float* mem_scale, const void* sink_k, const void* sink_v, int n_sinks, void* ring_k,
                          void* ring_v, float* ring_km, float* ring_g, float* ring_beta, int64_t* ring_pos,
                          float* state, float* o, float* lse, void* stream) {
    size_t need = 0;
    const int st = bf_decode_workspace_size(B, G, R, D, W, &need);
    if (st) return st;
    if (need > sizeof(scratch)) return BF_STATUS_SCRATCH;
    void* ws = nullptr;
    const int rc = scratch_on_current_device(&ws);
    if (rc) return rc;
    return bf_decode_fwd(B, G, R, D, W, sinks, pos, memory, kv_dtype, q_dtype, qr, qm, kr, v, km, g_new, beta_new, z,
                         mix_lse, mem_scale, sink_k, sink_v, n_sinks, ring_k, ring_v, ring_km, ring_g, ring_beta,
                         ring_pos, state, o, lse, ws, sizeof(scratch), stream);
}

// bf_window_fwd with an optional partial-row buffer of window_split_bytes(window_map(...), D) bytes: with it, bf16
// inputs run the work items of a last, at most half-full round on each XCD as two key halves, or a grid of a few
// items as up to 8 key parts (merged after).
static int window_fwd(int B, int G, int R, int D, int T, int W, int sinks, int64_t start, int in_dtype, const void* q,
                      int64_t q_sb, int64_t q_sh, int64_t q_st, const void* k, int64_t k_sb, int64_t k_sh, int64_t k_st,
                      const void* v, int64_t v_sb, int64_t v_sh, int64_t v_st, const void* ring_k, const void* ring_v,
                      const int64_t* ring_pos, const void* sink_k, const void* sink_v, int n_sinks, int mix,
                      const void* o_mem, int o_mem_dtype, const float* z, const float* mix_lse, const float* mem_scale,
                      void* o, int o_dtype, float* lse, float* part, void* stream) {
    if (B <= 0 || G <= 0 || R <= 0 || T <= 0 || W <= 0 || sinks < 0 || start < 0) return BF_STATUS_INVALID;
    if (!supported_dim(D) || !supported_dtype(in_dtype) || !supported_dtype(o_dtype)) return BF_STATUS_UNSUPPORTED;
    if (!q || !k || !v || !o) return BF_STATUS_INVALID;
    if ((ring_k == nullptr) != (ring_v == nullptr) || (ring_k && !ring_pos)) return BF_STATUS_INVALID;
    if (n_sinks < 0 || n_sinks > sinks || (n_sinks && (!sink_k || !sink_v))) return BF_STATUS_INVALID;
    if (mix && (!o_mem || !z || !mix_lse || !mem_scale)) return BF_STATUS_INVALID;
    if (mix && !supported_dtype(o_mem_dtype)) return BF_STATUS_UNSUPPORTED;
    bf::WinArgs a{};
    a.B = B; a.G = G; a.R = R; a.D = D; a.T = T; a.W = W; a.sinks = sinks; a.start = start;
    a.in_dtype = in_dtype; a.o_dtype = o_dtype;
    a.q = q; a.q_sb = q_sb; a.q_sh = q_sh; a.q_st = q_st;
    a.k = k; a.k_sb = k_sb; a.k_sh = k_sh; a.k_st = k_st;
    a.v = v; a.v_sb = v_sb; a.v_sh = v_sh; a.v_st = v_st;
    a.ring_k = ring_k; a.ring_v = ring_v; a.ring_pos = ring_pos;
    a.sink_k = sink_k; a.sink_v = sink_v; a.n_sinks = n_sinks;
    a.mix_on = mix; a.o_mem = o_mem; a.o_mem_dtype = o_mem_dtype; a.z = z; a.mix_lse = mix_lse; a.mem_scale = mem_scale;
    a.o = o; a.lse = lse;
    if (part && in_dtype == BF_DTYPE_BF16) {
        const bf::WinMap wm = bf::window_map(B, G, R, T, W, start);
        a.split_x = bf::window_split_x(wm);
        a.split_p = bf::window_split_p(wm);
        a.part = part;
    }
    return bf::window_dispatch(a, static_cast<hipStream_t>(stream));
}

int bf_window_fwd(int B, int G, int R, int D, int T, int W, int sinks, int64_t start, int in_dtype, const void* q,
                  int64_t q_sb, int64_t q_sh, int64_t q_st, const void* k, int64_t k_sb, int64_t k_sh, int64_t k_st,
                  const void* v, int64_t v_sb, int64_t v_sh, int64_t v_st, const void* ring_k, const void* ring_v,
                  const int64_t* ring_pos, const void* sink_k, const void* sink_v, int n_sinks, int mix,
                  const void* o_mem, int o_mem_dtype, const float* z, const float* mix_lse, const float* mem_scale, void* o,
                  int o_dtype, float* lse, void* stream) {
    return window_fwd(B, G, R, D, T, W, sinks, start, in_dtype, q, q_sb, q_sh, q_st, k, k_sb, k_sh, k_st, v, v_sb,
                      v_sh, v_st, ring_k, ring_v, ring_pos, sink_k, sink_v, n_sinks, mix, o_mem, o_mem_dtype, z,
                      mix_lse, mem_scale, o, o_dtype, lse, nullptr, stream);
}

int bf_mem_project(const void* x, int64_t n_tok, int nh, int D, int64_t x_st, int64_t x_sh, const float* f,
                   float scale, void* out, int in_dtype, int out_dtype, void* stream) {
    if (n_tok < 0 || nh <= 0 || x_st <= 0 || x_sh < 0) return BF_STATUS_INVALID;
    if (!supported_dim(D) || in_dtype != BF_DTYPE_BF16 || !supported_dtype(out_dtype)) return BF_STATUS_UNSUPPORTED;
    if (n_tok == 0) return BF_STATUS_OK;
    if (!x || !f || !out) return BF_STATUS_INVALID;
    if (x_st * 16 * 2 > 0xffffffffLL) return BF_STATUS_INVALID;     // 16 token rows per 32-bit buffer range
    bf::MemProjArgs a{};
    a.x = x; a.n_tok = n_tok; a.nh = nh; a.D = D; a.x_st = x_st; a.x_sh = x_sh;
    a.f = f; a.scale = scale; a.out = out; a.out_dtype = out_dtype;
    return bf::mem_project_dispatch(a, static_cast<hipStream_t>(stream));
}

int bf_mem_gates(const float* ab, int64_t n_tok, int64_t T, int G, int64_t ab_st, const float* A_log,
                 const float* dt_bias, const float* decay_mask, int64_t start, int sinks, float* g, float* beta,
                 void* stream) {
    if (n_tok < 0 || T <= 0 || G <= 0 || ab_st < 2 * G || start < 0 || sinks < 0 || (n_tok % T)) return BF_STATUS_INVALID;
    if (n_tok == 0) return BF_STATUS_OK;
    if (!ab || !A_log || !dt_bias || !decay_mask || !g || !beta) return BF_STATUS_INVALID;
    bf::MemGatesArgs a{};
    a.ab = ab; a.n_tok = n_tok; a.T = T; a.ab_st = ab_st; a.G = G; a.sinks = sinks; a.start = start;
    a.A_log = A_log; a.dt_bias = dt_bias; a.decay_mask = decay_mask; a.g = g; a.beta = beta;
    return bf::mem_gates_dispatch(a, static_cast<hipStream_t>(stream));
}

int bf_gate_project_workspace_size(int64_t n_tok, int d, int nout, size_t* bytes) {
    if (!bytes || n_tok < 0 || d <= 0 || nout <= 0 || nout > bf::GP_MAX_OUT) return BF_STATUS_INVALID;
    *bytes = bf::gate_project_workspace(n_tok, d, nout);
    return BF_STATUS_OK;
}

int bf_gate_project(const void* x, int64_t n_tok, int d, int64_t x_st, const float* w0, const float* b0, int n0,
                    float* out0, const float* w1, const float* b1, int n1, float* out1, void* workspace,
                    size_t workspace_bytes, void* stream) {
    if (n_tok < 0 || d <= 0 || d % 8 || x_st < d || x_st % 8 || n0 < 0 || n1 < 0 || n0 + n1 <= 0 ||
        n0 + n1 > bf::GP_MAX_OUT)
        return BF_STATUS_INVALID;
    if (n_tok == 0) return BF_STATUS_OK;
    if (!x || (n0 && (!w0 || !out0)) || (n1 && (!w1 || !out1))) return BF_STATUS_INVALID;
    auto al16 = [](const void* p) { return ((uintptr_t)p & 15) == 0; };
    if (!al16(x) || !al16(w0) || !al16(w1)) return BF_STATUS_INVALID;
    bf::GateProjArgs a{};
    a.x = static_cast<const uint16_t*>(x); a.n_tok = n_tok; a.x_st = x_st; a.d = d;
    a.w0 = w0; a.b0 = b0; a.n0 = n0; a.out0 = out0; a.w1 = w1; a.b1 = b1; a.n1 = n1; a.out1 = out1;
    const size_t need = bf::gate_project_workspace(n_tok, d, n0 + n1);
    if (need && (!workspace || workspace_bytes < need)) return BF_STATUS_WORKSPACE;
    a.part = static_cast<float*>(workspace);
    return bf::gate_project_dispatch(a, static_cast<hipStream_t>(stream));
}

int bf_gdn_conv_inputs(const void* z, int64_t z_st, const void* prefix, int in_dtype, const float* conv_w, int K,
                       const float* a, const float* b, const float* A_log, const float* dt_bias,
                       const int32_t* cu_seqlens, int num_seqs, int64_t n_tok, int HK, int HV, int D, float eps,
                       float q_scale, void* q, void* k, void* v, float* g, float* beta, int out_dtype, void* stream) {
    if (n_tok < 0 || num_seqs <= 0 || HK <= 0 || HV <= 0 || HV % HK || K < 1 || K > 16) return BF_STATUS_INVALID;
    if (!supported_dim(D) || !supported_dtype(in_dtype) || !supported_dtype(out_dtype)) return BF_STATUS_UNSUPPORTED;
    if (n_tok == 0) return BF_STATUS_OK;
    if (!z || !conv_w || !a || !b || !A_log || !dt_bias || !cu_seqlens || !q || !k || !v || !g || !beta)
        return BF_STATUS_INVALID;
    if (z_st < (int64_t)(2 * HK + HV) * D || z_st % 8) return BF_STATUS_INVALID;
    // 16-byte vector accesses: rows of 8 elements start 16-byte aligned
    auto al16 = [](const void* p) { return ((uintptr_t)p & 15) == 0; };
    if (!al16(z) || !al16(prefix) || !al16(conv_w) || !al16(q) || !al16(k) || !al16(v)) return BF_STATUS_INVALID;
    bf::GdnInArgs x{};
    x.z = z; x.z_st = z_st; x.prefix = prefix; x.in_dtype = in_dtype;
    x.w = conv_w; x.a = a; x.b = b; x.A_log = A_log; x.dt_bias = dt_bias;
    x.cu_seqlens = cu_seqlens; x.num_seqs = num_seqs; x.n_tok = n_tok;
    x.HK = HK; x.HV = HV; x.D = D; x.K = K; x.out_dtype = out_dtype; x.eps = eps; x.q_scale = q_scale;
    x.q = q; x.k = k; x.v = v; x.g = g; x.beta = beta;
    return bf::gdn_conv_inputs_dispatch(x, static_cast<hipStream_t>(stream));
}

int bf_gated_norm(const void* o, int o_dtype, const void* z, const float* w, int64_t rows, int D, float eps,
                  void* out, int io_dtype, void* stream) {
    if (rows < 0) return BF_STATUS_INVALID;
    if (!supported_dim(D) || !supported_dtype(o_dtype) || !supported_dtype(io_dtype)) return BF_STATUS_UNSUPPORTED;
    if (rows == 0) return BF_STATUS_OK;
    if (!o || !z || !w || !out) return BF_STATUS_INVALID;
    auto al16 = [](const void* p) { return ((uintptr_t)p & 15) == 0; };
    if (!al16(o) || !al16(z) || !al16(out)) return BF_STATUS_INVALID;
    bf::GatedNormArgs x{};
    x.o = o; x.o_dtype = o_dtype; x.z = z; x.w = w; x.out = out; x.io_dtype = io_dtype;
    x.rows = rows; x.D = D; x.eps = eps;
    return bf::gated_norm_dispatch(x, static_cast<hipStream_t>(stream));
}

static bool kv_aligned(const void* p, int64_t s1, int64_t s2) {
    return (reinterpret_cast<uintptr_t>(p) & 15) == 0 && s1 % 8 == 0 && s2 % 8 == 0;
}

// workspace of bf_layer_prefill_fwd: the GDN inputs and outputs for up to B T memory queries, o_mem, the new state
// and the GDN workspace. The GDN part is laid out for B T tokens with the segment length chosen for B T tokens; the
// inner call runs on at most B T tokens with that same segment length, and every buffer of the GDN layout grows
// monotonically with the token count at a fixed segment length, so the reservation always suffices.
struct LayerWs {
    size_t wq, wk, wv, wg, wb, om, o_mem, s_new, part, gdn, total;
    int seg_chunks;
};
static LayerWs layer_ws(int B, int G, int R, int D, int T, int in_dtype) {
    LayerWs w{};
    const size_t esz = in_dtype == BF_DTYPE_BF16 ? 2 : 4, H = (size_t)G * R, BT = (size_t)B * T;
    size_t at = 0;
    auto put = [&](size_t& f, size_t n) { f = at; at += align256(n); };
    put(w.wq, BT * H * D * esz);
    put(w.wk, BT * G * D * esz);
    put(w.wv, BT * G * D * esz);
    put(w.wg, BT * G * 4);
    put(w.wb, BT * G * 4);
    put(w.om, BT * H * D * esz);
    put(w.o_mem, BT * H * D * esz);
    put(w.s_new, (size_t)B * G * D * D * 4);
    // the item map's slot count does not depend on the window or the position
    put(w.part, in_dtype == BF_DTYPE_BF16 ? bf::window_split_bytes(bf::window_map(B, G, R, T, 1, 0), D) : 0);
    const GdnLayout gl = gdn_layout((int64_t)B * T, B, G, R, D, in_dtype, 0);
    w.seg_chunks = gl.seg_chunks;
    put(w.gdn, gl.total);
    w.total = at;
    return w;
}

int bf_layer_prefill_workspace_size(int B, int G, int R, int D, int T, int in_dtype, size_t* bytes) {
    if (!bytes || B <= 0 || G <= 0 || R <= 0 || T <= 0) return BF_STATUS_INVALID;
    if (!supported_dim(D) || !supported_dtype(in_dtype)) return BF_STATUS_UNSUPPORTED;
    *bytes = layer_ws(B, G, R, D, T, in_dtype).total;
    return BF_STATUS_OK;
}

int bf_layer_prefill_fwd(int B, int G, int R, int D, int T, int W, int sinks, int64_t start, int memory, int in_dtype,
                         const void* qr, int64_t q_sb, int64_t q_sh, int64_t q_st, const void* kr, int64_t k_sb,
                         int64_t k_sh, int64_t k_st, const void* v, int64_t v_sb, int64_t v_sh, int64_t v_st,
                         const void* qm, int qm_dtype, const void* km, int km_dtype, const float* g,
                         const float* beta, const float* z, const float* mix_lse, const float* mem_scale,
                         const void* sink_k, const void* sink_v, int n_sinks, void* ring_k, void* ring_v,
                         float* ring_km, float* ring_g, float* ring_beta, int64_t* ring_pos, float* state,
                         int state_valid, float* o, float* lse, void* workspace, size_t workspace_bytes,
                         void* stream) {
    if (B <= 0 || G <= 0 || R <= 0 || T <= 0 || W <= 0 || sinks < 0 || start < 0) return BF_STATUS_INVALID;
    if (!supported_dim(D) || !supported_dtype(in_dtype) || !supported_dtype(qm_dtype) || !supported_dtype(km_dtype))
        return BF_STATUS_UNSUPPORTED;
    if (!qr || !kr || !v || !qm || !km || !g || !beta || !ring_k || !ring_v || !ring_km || !ring_g || !ring_beta ||
        !ring_pos || !state || !o)
        return BF_STATUS_INVALID;
    const bool use_mem = memory && start + T > W;
    if (use_mem && (!z || !mix_lse || !mem_scale)) return BF_STATUS_INVALID;
    const LayerWs L = layer_ws(B, G, R, D, T, in_dtype);
    if (!workspace || workspace_bytes < L.total || (reinterpret_cast<uintptr_t>(workspace) & 255))
        return BF_STATUS_WORKSPACE;
    char* ws = static_cast<char*>(workspace);
    const hipStream_t st = static_cast<hipStream_t>(stream);
    bf::LayerArgs a{};
    a.B = B; a.G = G; a.R = R; a.D = D; a.T = T; a.W = W; a.start = start;
    a.in_dtype = in_dtype; a.qm_dtype = qm_dtype; a.km_dtype = km_dtype;
    a.qm = qm; a.km = km; a.kr = kr; a.v = v; a.g = g; a.beta = beta;
    a.k_sb = k_sb; a.k_sh = k_sh; a.k_st = k_st; a.v_sb = v_sb; a.v_sh = v_sh; a.v_st = v_st;
    a.ring_v = ring_v; a.ring_km = ring_km; a.ring_g = ring_g; a.ring_beta = ring_beta; a.ring_pos = ring_pos;
    a.wq = ws + L.wq; a.wk = ws + L.wk; a.wv = ws + L.wv;
    a.wg = reinterpret_cast<float*>(ws + L.wg); a.wb = reinterpret_cast<float*>(ws + L.wb);
    a.om = ws + L.om; a.o_mem = ws + L.o_mem;
    a.ring_k_w = ring_k; a.ring_v_w = ring_v; a.ring_km_w = ring_km; a.ring_g_w = ring_g; a.ring_beta_w = ring_beta;
    a.ring_pos_w = ring_pos;
    a.s_new = reinterpret_cast<float*>(ws + L.s_new); a.state = state;
    int rc;
    const void* o_mem = nullptr;
    if (use_mem) {
        // from an empty cache the queries before W never mix the memory in: the stream is the chunk shifted by W
        const bool fresh = start == 0 && !state_valid;
        a.qoff = fresh ? W : 0;
        a.Tq = T - a.qoff;
        const size_t esz = in_dtype == BF_DTYPE_BF16 ? 2 : 4, H = (size_t)G * R;
        // a single sequence, or no shift, keeps the query and output rows contiguous: no staging copies
        const bool rows = B == 1 || a.qoff == 0;
        const void* wq = a.wq;
        if (rows && qm_dtype == in_dtype) wq = static_cast<const char*>(qm) + a.qoff * H * D * esz;
        else if ((rc = bf::layer_launch(a, 4, st))) return rc;
        const void *wk = a.wk, *wv = a.wv;
        const float *wg = a.wg, *wb = a.wb;
        if (fresh && B == 1 && km_dtype == in_dtype && v_sh == D && v_st == (int64_t)G * D) {
            wk = km; wv = v; wg = g; wb = beta;                 // the stream is the chunk's own rows 0 .. T - W - 1
        } else if ((rc = bf::layer_launch(a, 0, st))) {
            return rc;
        }
        void* om = rows ? static_cast<char*>(a.o_mem) + a.qoff * H * D * esz : ws + L.om;
        a.om = om;
        rc = bf_gdn_fwd(wq, wk, wv, wg, wb, nullptr, B, (int64_t)B * a.Tq, G, R, D, in_dtype, 1.f,
                        state_valid ? state : nullptr, om, in_dtype, reinterpret_cast<float*>(ws + L.s_new), L.seg_chunks,
                        ws + L.gdn, L.total - L.gdn,
                        BF_GDN_PHASE_ALL, stream);
        if (rc) return rc;
        if (!rows && (rc = bf::layer_launch(a, 1, st))) return rc;
        o_mem = a.o_mem;
    }
    rc = window_fwd(B, G, R, D, T, W, sinks, start, in_dtype, qr, q_sb, q_sh, q_st, kr, k_sb, k_sh, k_st, v, v_sb,
                    v_sh, v_st, ring_k, ring_v, ring_pos, sink_k, sink_v, n_sinks, use_mem ? 1 : 0, o_mem,
                    in_dtype, use_mem ? z : nullptr, use_mem ? mix_lse : nullptr, use_mem ? mem_scale : nullptr, o,
                    BF_DTYPE_F32, lse, reinterpret_cast<float*>(ws + L.part), stream);
    if (rc) return rc;
    if ((rc = bf::layer_launch(a, 2, st))) return rc;         // ring write-back after every read of the ring
    if (use_mem && (rc = bf::layer_launch(a, 3, st))) return rc;
    return BF_STATUS_OK;
}

int bf_gdn_bwd_workspace_size(int num_seqs, int64_t seq_len, int G, int R, int D, size_t* bytes) {
    if (!bytes || num_seqs <= 0 || seq_len <= 0 || G <= 0 || R <= 0) return BF_STATUS_INVALID;
    if (!supported_dim(D) || seq_len % 64) return BF_STATUS_UNSUPPORTED;
    *bytes = bf::gdn_bwd_workspace(num_seqs, seq_len, G, R, D);
    return BF_STATUS_OK;
}

int bf_gdn_bwd(const float* q, const float* k, const float* v, const float* g, const float* beta, const float* s0,
               float scale, const float* dO, const float* ds_final, int num_seqs, int64_t seq_len, int G, int R, int D,
               float* dq, float* dk, float* dv, float* dg, float* dbeta, float* ds0, void* workspace,
               size_t workspace_bytes, void* stream) {
    if (num_seqs <= 0 || seq_len <= 0 || G <= 0 || R <= 0) return BF_STATUS_INVALID;
    if (!supported_dim(D) || seq_len % 64) return BF_STATUS_UNSUPPORTED;
    if ((int64_t)num_seqs * (seq_len / 64) * G * R > INT32_MAX) return BF_STATUS_UNSUPPORTED;
    if (!q || !k || !v || !g || !beta || !dO || !dq || !dk || !dv || !dg || !dbeta) return BF_STATUS_INVALID;
    for (const void* p : {(const void*)q, (const void*)k, (const void*)v, (const void*)dO, (const void*)s0,
                          (const void*)ds_final, (const void*)dq, (const void*)dk, (const void*)dv, (const void*)ds0})
        if (reinterpret_cast<uintptr_t>(p) & 15) return BF_STATUS_INVALID;
    const size_t need = bf::gdn_bwd_workspace(num_seqs, seq_len, G, R, D);
    if (!workspace || workspace_bytes < need || (reinterpret_cast<uintptr_t>(workspace) & 255)) return BF_STATUS_WORKSPACE;
    bf::GdnBwdArgs a{};
    a.q = q; a.k = k; a.v = v; a.g = g; a.beta = beta; a.s0 = s0; a.dO = dO; a.dsf = ds_final; a.scale = scale;
    a.num_seqs = num_seqs; a.n_chunks = (int)(seq_len / 64); a.G = G; a.R = R; a.D = D;
    a.dq = dq; a.dk = dk; a.dv = dv; a.dg = dg; a.dbeta = dbeta; a.ds0 = ds0;
    return bf::gdn_bwd(a, workspace, static_cast<hipStream_t>(stream));
}

int bf_llama_state_floats(int G, int D, int W, int S, int64_t* floats) {
    if (!floats || G <= 0 || D <= 0 || W <= 0 || S < 0) return BF_STATUS_INVALID;
    *floats = bf::llama_state_floats(G, D, W, S);
    return BF_STATUS_OK;
}

static int llama_geometry(bf::LlamaStateArgs& a, int B, int G, int D, int W, int S, int64_t n, int kv_dtype,
                          int n_sinks) {
    if (B <= 0 || G <= 0 || W <= 0 || S < 0 || n < 0 || n_sinks < 0 || n_sinks > S || n_sinks > n)
        return BF_STATUS_INVALID;
    if (!supported_dim(D) || !supported_dtype(kv_dtype)) return BF_STATUS_UNSUPPORTED;
    a.B = B; a.G = G; a.D = D; a.W = W; a.S = S; a.n = n; a.kv_dtype = kv_dtype; a.n_sinks = n_sinks;
    a.LR = (S + W + 2 + 31) / 32 * 32;
    a.row = bf::llama_state_floats(G, D, W, S);
    return BF_STATUS_OK;
}

int bf_llama_state_pack(int B, int G, int D, int W, int S, int64_t n, int kv_dtype, const void* ring_k,
                        const void* ring_v, const float* ring_km, const float* ring_g, const float* ring_beta,
                        const int64_t* ring_pos, const void* sink_k, const void* sink_v, int n_sinks,
                        const float* state, float* rows, void* stream) {
    bf::LlamaStateArgs a{};
    const int st = llama_geometry(a, B, G, D, W, S, n, kv_dtype, n_sinks);
    if (st != BF_STATUS_OK) return st;
    if (!ring_k || !ring_v || !ring_km || !ring_g || !ring_beta || !ring_pos || !state || !rows ||
        (n_sinks && (!sink_k || !sink_v)))
        return BF_STATUS_INVALID;
    a.ring_k = ring_k; a.ring_v = ring_v; a.ring_km = ring_km; a.ring_g = ring_g; a.ring_beta = ring_beta;
    a.ring_pos = ring_pos; a.sink_k = sink_k; a.sink_v = sink_v; a.state = state; a.rows = rows;
    return bf::llama_state(a, true, static_cast<hipStream_t>(stream));
}

int bf_llama_state_unpack(int B, int G, int D, int W, int S, int64_t n, int kv_dtype, const float* rows, void* ring_k,
                          void* ring_v, float* ring_km, float* ring_g, float* ring_beta, int64_t* ring_pos,
                          void* sink_k, void* sink_v, int n_sinks, float* state, void* stream) {
    bf::LlamaStateArgs a{};
    const int st = llama_geometry(a, B, G, D, W, S, n, kv_dtype, n_sinks);
    if (st != BF_STATUS_OK) return st;
    if (n_sinks != (n < S ? n : S)) return BF_STATUS_INVALID;
    if (!rows || !ring_k || !ring_v || !ring_km || !ring_g || !ring_beta || !ring_pos || !state ||
        (n_sinks && (!sink_k || !sink_v)))
        return BF_STATUS_INVALID;
    a.rows = const_cast<float*>(rows);
    a.ring_k_out = ring_k; a.ring_v_out = ring_v; a.ring_km_out = ring_km; a.ring_g_out = ring_g;
    a.ring_beta_out = ring_beta; a.ring_pos_out = ring_pos; a.sink_k_out = sink_k; a.sink_v_out = sink_v;
    a.state_out = state;
    return bf::llama_state(a, false, static_cast<hipStream_t>(stream));
}

int bf_kv_append(const void* k_new, int64_t k_sb, int64_t k_sg, int64_t k_st, const void* v_new, int64_t v_sb,
                 int64_t v_sg, int64_t v_st, int dtype, int B, int G, int t, int D, void* k_buf, void* v_buf,
                 int64_t cap, int64_t n0, void* stream) {
    if (B <= 0 || G <= 0 || t < 0 || cap <= 0 || n0 < 0 || n0 + t > cap) return BF_STATUS_INVALID;
    if (!supported_dim(D) || !supported_dtype(dtype)) return BF_STATUS_UNSUPPORTED;
    if (t == 0) return BF_STATUS_OK;
    if (!k_new || !v_new || !k_buf || !v_buf) return BF_STATUS_INVALID;
    if (!kv_aligned(k_new, k_sb, k_sg) || !kv_aligned(v_new, v_sb, v_sg) || k_st % 8 || v_st % 8 ||
        !kv_aligned(k_buf, 0, 0) || !kv_aligned(v_buf, 0, 0))
        return BF_STATUS_INVALID;
    bf::KvAppendArgs a{};
    a.k_new = k_new; a.v_new = v_new; a.k_sb = k_sb; a.k_sg = k_sg; a.k_st = k_st; a.v_sb = v_sb; a.v_sg = v_sg;
    a.v_st = v_st; a.B = B; a.G = G; a.t = t; a.D = D; a.esz = dtype == BF_DTYPE_BF16 ? 2 : 4;
    a.k_buf = k_buf; a.v_buf = v_buf; a.cap = cap; a.n0 = n0;
    return bf::kv_append(a, static_cast<hipStream_t>(stream));
}

int bf_kv_block_summary(const void* k, int dtype, int B, int G, int D, int64_t k_sbg, int64_t k_st, int sinks, int L,
                        int first_block, int nb, int nb_cap, void* kmin, void* kmax, void* stream) {
    if (B <= 0 || G <= 0 || L <= 0 || sinks < 0 || first_block < 0 || nb < first_block || nb > nb_cap || k_st <= 0 ||
        k_sbg < 0)
        return BF_STATUS_INVALID;
    if (!supported_dim(D) || !supported_dtype(dtype)) return BF_STATUS_UNSUPPORTED;
    if (nb == first_block) return BF_STATUS_OK;
    if (!k || !kmin || !kmax || !kv_aligned(k, k_sbg, k_st) || !kv_aligned(kmin, 0, 0) || !kv_aligned(kmax, 0, 0))
        return BF_STATUS_INVALID;
    bf::KvArgs a{};
    a.B = B; a.T = 1; a.G = G; a.R = 1; a.D = D; a.dtype = dtype; a.k = k; a.k_sbg = k_sbg; a.k_st = k_st;
    a.sinks = sinks; a.L = L; a.sum_first = first_block; a.nb = nb; a.nb_cap = nb_cap; a.kmin = kmin; a.kmax = kmax;
    return bf::kv_dispatch(a, 0, static_cast<hipStream_t>(stream));
}

// the shared checks of the selection and the attention; fills the geometry fields of a
static int kv_geometry(bf::KvArgs& a, int B, int T, int G, int R, int D, int64_t n, int dtype, int retrieval, int sinks,
                       int window, int L, int K) {
    if (B <= 0 || T <= 0 || G <= 0 || R <= 0 || n <= 0 || T > n || K < 0) return BF_STATUS_INVALID;
    if ((int64_t)B * T > (int64_t)1 << 22 || (int64_t)B * G > 65535 || n > INT32_MAX) return BF_STATUS_UNSUPPORTED;
    if (R > 8 || !supported_dim(D) || !supported_dtype(dtype) || K > bf::kv_max_k()) return BF_STATUS_UNSUPPORTED;
    a.B = B; a.T = T; a.G = G; a.R = R; a.D = D; a.dtype = dtype; a.n = n; a.retrieval = retrieval ? 1 : 0;
    if (a.retrieval) {
        if (sinks < 0 || window <= 0 || L <= 0 || sinks > n) return BF_STATUS_INVALID;
        a.sinks = sinks; a.window = window; a.L = L; a.K = K;
        const int64_t nb = (n - sinks) / L;
        if (nb > bf::kv_max_blocks()) return BF_STATUS_UNSUPPORTED;
        a.nb = (int)nb;
    } else {
        a.sinks = 0; a.window = 0; a.L = 1; a.K = 0; a.nb = 0;
    }
    return BF_STATUS_OK;
}

int bf_kv_select(const void* q, int dtype, int B, int T, int G, int R, int D, int64_t n, int sinks, int window, int L,
                 const void* kmin, const void* kmax, int nb_cap, int K, int* sel, void* stream) {
    bf::KvArgs a{};
    const int st = kv_geometry(a, B, T, G, R, D, n, dtype, 1, sinks, window, L, K);
    if (st != BF_STATUS_OK) return st;
    if (a.nb > nb_cap) return BF_STATUS_INVALID;
    if (K == 0) return BF_STATUS_OK;
    if (!q || !sel || !kv_aligned(q, 0, 0) || (a.nb > 0 && (!kmin || !kmax || !kv_aligned(kmin, 0, 0) ||
                                                             !kv_aligned(kmax, 0, 0))))
        return BF_STATUS_INVALID;
    a.q = q; a.kmin = const_cast<void*>(kmin); a.kmax = const_cast<void*>(kmax); a.nb_cap = nb_cap; a.sel = sel;
    return bf::kv_dispatch(a, 1, static_cast<hipStream_t>(stream));
}

int bf_kv_attention_workspace_size(int B, int T, int G, int R, int D, int64_t n, int retrieval, int sinks, int window,
                                   int L, int K, size_t* bytes) {
    if (!bytes) return BF_STATUS_INVALID;
    bf::KvArgs a{};
    const int st = kv_geometry(a, B, T, G, R, D, n, BF_DTYPE_F32, retrieval, sinks, window, L, K);
    if (st != BF_STATUS_OK) return st;
    int sl = 0, ns = 0;
    bf::kv_split_plan(a, &sl, &ns);
    if (ns > bf::kv_max_splits()) return BF_STATUS_UNSUPPORTED;
    *bytes = (size_t)B * T * G * ns * R * (D + 2) * sizeof(float);
    return BF_STATUS_OK;
}

int bf_kv_attention(const void* q, const void* k, const void* v, int dtype, int B, int T, int G, int R, int D,
                    int64_t n, int64_t k_sbg, int64_t k_st, int64_t v_sbg, int64_t v_st, int retrieval, int sinks,
                    int window, int L, const int* sel, int K, float scale, void* workspace, size_t workspace_bytes,
                    void* o, int o_dtype, void* stream) {
    bf::KvArgs a{};
    const int st = kv_geometry(a, B, T, G, R, D, n, dtype, retrieval, sinks, window, L, K);
    if (st != BF_STATUS_OK) return st;
    if (!supported_dtype(o_dtype)) return BF_STATUS_UNSUPPORTED;
    if (k_st <= 0 || v_st <= 0 || k_sbg < 0 || v_sbg < 0) return BF_STATUS_INVALID;
    if (!q || !k || !v || !o || (a.retrieval && K > 0 && !sel)) return BF_STATUS_INVALID;
    if (!kv_aligned(q, 0, 0) || !kv_aligned(k, k_sbg, k_st) || !kv_aligned(v, v_sbg, v_st)) return BF_STATUS_INVALID;
    int slen = 0, nsplit = 0;
    bf::kv_split_plan(a, &slen, &nsplit);
    if (nsplit > bf::kv_max_splits()) return BF_STATUS_UNSUPPORTED;
    const size_t need = (size_t)B * T * G * nsplit * R * (D + 2) * sizeof(float);
    if (!workspace || workspace_bytes < need) return BF_STATUS_WORKSPACE;
    a.q = q; a.k = k; a.v = v; a.k_sbg = k_sbg; a.k_st = k_st; a.v_sbg = v_sbg; a.v_st = v_st;
    a.sel = const_cast<int*>(sel); a.scale = scale; a.slen = slen; a.nsplit = nsplit;
    a.ws_part = static_cast<float*>(workspace);
    a.o = o; a.o_dtype = o_dtype;
    return bf::kv_dispatch(a, 2, static_cast<hipStream_t>(stream));
}

}  // extern "C"
