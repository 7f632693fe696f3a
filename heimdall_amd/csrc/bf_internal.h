// Internal launch arguments shared by the kernels and the C-ABI entry points (not part of the public ABI).
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "../../include/bifrost.h"

namespace bf {

// Ring slots per window split of the decode step (at B = 64, G = 4, W = 2048: 1024 slots 129.1 us per step, 512 130.4,
// 2048 134.0, 256 141).
constexpr int DECODE_SLOTS = 1024;

constexpr int DT_F32 = BF_DTYPE_F32;
constexpr int DT_BF16 = BF_DTYPE_BF16;
constexpr int BF_ERR_UNSUPPORTED = BF_STATUS_UNSUPPORTED;
constexpr int GDN_PHASE_PREP = BF_GDN_PHASE_PREP;
constexpr int GDN_PHASE_STATES = BF_GDN_PHASE_STATES;
constexpr int GDN_PHASE_OUTPUT = BF_GDN_PHASE_OUTPUT;

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
    int seg_chunks;          // chunks per segment (L)
    int max_segs;            // grid bound on segments over all sequences
    int multi_seg;           // some sequence may span more than one segment (STATES phase needed)
    // workspace carve-up (cid = chunk id, sid = segment id; C = 64)
    float* ws_gcum;          // [cid][G][C]        in-chunk cumulative log-decay
    void* ws_T;              // [cid][G][C*C]      (I + A)^-1 diag(beta), in_dtype, MFMA A-fragment order (tfrag_index)
    void* ws_phi;            // [sid][G][D*D]      Psi = Phi - c I of each segment map (in_dtype, fragment order)
    float* ws_c;             // [sid][G]           c = e^{sum of g over the segment}
    float* ws_n;             // [sid][G][D*D]      segment state from a zero entry state (fp32, accumulator-fragment order)
    float* ws_sin;           // [sid][G][D*D]      entry state of each segment (fp32, accumulator-fragment order; segments > 0)
    // the output scan's fused GatedNorm (null: o is stored as computed): z rows [N_tok][G*R][D] bf16, w [D] f32
    const void* gn_z;
    const float* gn_w;
    float gn_eps;
};

int gdn_prep(const GdnArgs& a, hipStream_t stream);
int gdn_states(const GdnArgs& a, hipStream_t stream, bool summary, bool combine);
int gdn_output(const GdnArgs& a, hipStream_t stream);


struct DecodeArgs {
    int B, G, R, D, W, sinks;
    long pos;                 // absolute position of the new token (same for all sequences; pos_arr == null)
    const int64_t* pos_arr;   // [B] positions of the sequences (device), or null: one position for all
    int mem_on;               // shared position: memory branch active (pos >= W and memory enabled); with pos_arr:
                              // memory enabled (sequence b's branch is active when pos_arr[b] >= W)
    int kv_dtype, q_dtype;
    const void* qr;           // [B][H][D] q_dtype
    const float* qm;          // [B][H][D]
    const void* kr;           // [B][G][D] kv_dtype
    const void* v;            // [B][G][D] kv_dtype
    const float* km;          // [B][G][D]
    const float* g_new;       // [B][G]
    const float* beta_new;    // [B][G]
    const float* z;           // [B][H] mix logits
    const float* mix_lse;     // [H]
    const float* mem_scale;   // [H]
    void* sink_k;             // [B][G][n_sinks][D] kv_dtype; with pos_arr [B][G][sinks][D], the first
    void* sink_v;             //   min(pos, sinks) rows valid and the new token written to row pos if pos < sinks
    int n_sinks;              // sink rows per (sequence, KV head): present sinks, or the capacity `sinks` with pos_arr
    void* ring_k;             // [B][G][W][D] kv_dtype
    void* ring_v;
    float* ring_km;           // [B][W][G][D]
    float* ring_g;            // [B][W][G]
    float* ring_beta;         // [B][W][G]
    int64_t* ring_pos;        // [W]; with pos_arr [B][W], one per sequence
    float* state;             // [B][G][D][D]
    float* o;                 // [B][H][D]
    float* lse;               // [B][H] or null
    int nsplit, slots;        // window splits of `slots` ring slots (decode_split)
    float* ws_om;             // [B][H][D] memory read
    float* ws_part;           // [B][G][nsplit][R][D + 2] window partials
    float* ws_ev;             // [B][G][2 D + 4] the ring row leaving the window: v, km, g, beta, valid
};

int decode_dispatch(const DecodeArgs& a, hipStream_t stream);

// Window splits of a decode step: at least two workgroups per CU over the B * G (sequence, KV head) pairs, splits of
// at most DECODE_SLOTS and at least 16 ring slots (a multiple of 16), at most 64 splits (the merge keeps 64 in LDS).
// B = 64, G = 4, W = 2048: 2 splits of 1024 slots; B = 1: 64 splits of 32.
inline void decode_split(int B, int G, int W, int& nsplit, int& slots) {
    const long bg = (long)B * G;
    const long need = (W + DECODE_SLOTS - 1) / DECODE_SLOTS;
    long n = (512 + bg - 1) / bg;
    const long most = (W + 15) / 16 < 64 ? (W + 15) / 16 : 64;
    if (n > most) n = most;
    if (n < need) n = need;
    slots = (int)(((W + n - 1) / n + 15) / 16 * 16);
    if (slots > DECODE_SLOTS) slots = DECODE_SLOTS;
    nsplit = (W + slots - 1) / slots;
}

struct StepArgs {
    int B, G, R, D;
    const float* q;           // [B][G*R][D]
    const float* k;           // [B][G][D]
    const float* v;           // [B][G][D]
    const float* g;           // [B][G]
    const float* beta;        // [B][G]
    const float* s_in;        // [B][G][D][D]
    float* s_out;             // [B][G][D][D] (may equal s_in)
    float* o;                 // [B][G*R][D]
};

int step_dispatch(const StepArgs& a, hipStream_t stream);

// Work items of the bf16 window kernel: 128 consecutive queries x one query head. Row u = (b G + g) nqb + j holds
// the R heads of query block nqb - 1 - j (later blocks first within each (b, g)); item u R + r is head r of row u.
// The 8 XCDs form 8 / f groups of f XCDs: group q takes the contiguous rows [q rpg, (q + 1) rpg), and XCD e of the
// group every f-th row of them from row q rpg + e. The XCDs of a group read about the same key range (each into its
// own L2), and query blocks of unequal length (causal attention, the first W positions) spread evenly over them.
// Each XCD takes its items in order, its last rot items first; workgroup x runs on XCD x mod 8 as dispatch slot
// x / 8 of per.
struct WinMap {
    long nrow, rpg, per;
    int R, f, rot;
};
__host__ __device__ inline WinMap window_map_make(int B, int G, int R, int T, int f, int rot) {
    WinMap m{};
    m.nrow = (long)B * G * ((T + 127) / 128);
    m.R = R;
    m.f = f;
    m.rot = rot;
    m.rpg = (m.nrow + 8 / f - 1) / (8 / f);
    m.per = (m.rpg + f - 1) / f * R;
    return m;
}
// item u R + r of dispatch slot k on XCD x, -1 past the XCD's items
__host__ __device__ inline long window_item(const WinMap& m, int x, long k) {
    const int q = x / m.f, e = x % m.f;
    const long u0 = q * m.rpg + e, u1 = m.nrow < (q + 1) * m.rpg ? m.nrow : (q + 1) * m.rpg;
    if (u0 >= u1) return -1;
    const long n = (u1 - u0 + m.f - 1) / m.f * m.R;
    if (k >= n) return -1;
    const long rot = m.rot < n ? m.rot : n;
    const long pos = k < rot ? n - rot + k : k - rot;
    return (u0 + m.f * (pos / m.R)) * m.R + pos % m.R;
}

struct WinArgs {
    int B, G, R, D, T, W, sinks;
    long start;               // absolute position of the chunk's first token
    int in_dtype, o_dtype;
    const void* q;            // queries, element strides (batch, head, token), D contiguous
    long q_sb, q_sh, q_st;
    const void* k;            // chunk keys
    long k_sb, k_sh, k_st;
    const void* v;            // chunk values
    long v_sb, v_sh, v_st;
    const void* ring_k;       // [B][G][W][D] or null
    const void* ring_v;
    const int64_t* ring_pos;  // [W]
    const void* sink_k;       // [B][G][n_sinks][D]
    const void* sink_v;
    int n_sinks;
    int mix_on;
    const void* o_mem;        // [B][T][H][D] in o_mem_dtype
    int o_mem_dtype;
    const float* z;           // [B][T][H]
    const float* mix_lse;     // [H]
    const float* mem_scale;   // [H]
    void* o;                  // [B][T][H][D] o_dtype
    float* lse;               // [B][H][T] or null
    int split_x;              // bf16 kernel: slots per XCD split into key parts (window_split_x), 0: none
    int split_p;              // key parts per split slot (window_split_p)
    float* part;              // their partial rows [8 split_x][split_p][128][D + 4] (m, l, -, -, unnormalised o)
    WinMap map;               // bf16 kernel: set by its launcher from window_map
};

// The bf16 window kernel's item map for B sequences of T queries, G KV heads of R query heads each, window W from
// position start. The slot count per XCD, ceil(ceil(rows / (8 / f)) / f) R = ceil(rows / 8) R, does not depend on f.
// When queries before position W see fewer keys (start < W: a prefill's first chunk, causal attention), XCDs are
// paired (f = 2) so that both take long and short query blocks: causal attention over 32768 queries (H = 24, G = 4,
// D = 256) 12.6 ms against 18.8 ms with contiguous ranges per XCD (f = 1), which gave one XCD of each pair the 128
// longest query blocks of its KV head and the other the 128 shortest; f = 4 12.7 ms, f = 8 13.1 ms. With rot = 32
// each XCD starts with its shortest items, so its workgroups do not reach their epilogues (the o stores) in
// lockstep: sliding window 2048 over 32768 queries 1955-1965 us against 1975-1990 us without the rotation. Chunks
// past the first W positions (every item as long) keep contiguous ranges (f = 1), whose concurrent items share
// one L2's keys: 16 chunks of 2048 at 5.61-5.66 ms against 5.68-5.72 ms paired.
inline WinMap window_map(int B, int G, int R, int T, int W, long start) {
    return start < W ? window_map_make(B, G, R, T, 2, 32) : window_map_make(B, G, R, T, 1, 0);
}

// Dispatch slots past the last full round of an XCD (32 CUs) are split into two key halves when they fill at most
// half a round: the XCD then runs one full round and a round of halves instead of two full rounds.
inline int window_split_x(const WinMap& m) {
    const long rem = m.per % 32;
    return rem > 0 && rem <= 16 ? (int)rem : 0;
}
// Key parts per split slot: two, unless every slot of an XCD is split and there are few (a chunk of a few tokens,
// such as an MTP verification step), then as many as keep the XCD's parts within one round on its 32 CUs.
inline int window_split_p(const WinMap& m) {
    if (m.per > 16) return 2;
    const long p = 32 / (m.per > 0 ? m.per : 1);
    return (int)(p < 2 ? 2 : (p > 8 ? 8 : p));
}
inline size_t window_split_bytes(const WinMap& m, int D) {
    return (size_t)8 * window_split_x(m) * window_split_p(m) * 128 * (D + 4) * sizeof(float);
}

int window_dispatch(const WinArgs& a, hipStream_t stream);

// 4 consecutive elements of the memory read (fp32 or bf16) at element index i (a multiple of 4) as fp32.
// om[j] = o_mem elements i + 16 j .. + 3 as fp32. The N reads are issued back to back under one dtype branch: with
// the dtype tested per read, each read sat in its own basic block and the compiler waited for it before the next.
template <int N>
__device__ __forceinline__ void load_om(const WinArgs& a, long i, float4 (&om)[N]) {
    if (a.o_mem_dtype == DT_BF16) {
        const uint16_t* p = reinterpret_cast<const uint16_t*>(a.o_mem) + i;
        uint2 raw[N];
#pragma unroll
        for (int j = 0; j < N; ++j) raw[j] = *reinterpret_cast<const uint2*>(p + 16 * j);
#pragma unroll
        for (int j = 0; j < N; ++j)
            om[j] = make_float4(__uint_as_float(raw[j].x << 16), __uint_as_float(raw[j].x & 0xffff0000u),
                                __uint_as_float(raw[j].y << 16), __uint_as_float(raw[j].y & 0xffff0000u));
    } else {
        const float* p = reinterpret_cast<const float*>(a.o_mem) + i;
#pragma unroll
        for (int j = 0; j < N; ++j) om[j] = *reinterpret_cast<const float4*>(p + 16 * j);
    }
}

struct MemProjArgs {
    const void* x;            // bf16 rows: token t, head h at x + t * x_st + h * x_sh (elements), D contiguous
    long n_tok;
    int nh, D;
    long x_st, x_sh;
    const float* f;           // [nh][D][D] fp32, the projections as the module holds them: f[h][i][j] = F_h[i][j]
    float scale;
    void* out;                // [n_tok][nh][D] in out_dtype
    int out_dtype;            // DT_BF16 or DT_F32
};

struct MemGatesArgs {
    const float* ab;                // [n_tok][ab_st]: columns [a (G) | b (G)]
    long n_tok, T, ab_st;           // tokens, tokens per sequence, row stride
    int G, sinks;
    long start;                     // position of each sequence's first token
    const int64_t* pos_arr;         // or null: sequence b's first token at pos_arr[b] (device memory)
    const float *A_log, *dt_bias, *decay_mask;
    float *g, *beta;                // [n_tok][G]
};
int mem_gates_dispatch(const MemGatesArgs& a, hipStream_t stream);

constexpr int GP_MAX_OUT = 64;      // gate projection: n0 + n1 output columns at most
struct GateProjArgs {
    const uint16_t* x;              // bf16 rows: token t at x + t * x_st, d contiguous (d a multiple of 8)
    long n_tok, x_st;
    int d;
    const float *w0, *b0;           // [n0][d], [n0] (b0 may be null)
    int n0;
    float* out0;                    // [n_tok][n0]
    const float *w1, *b1;           // [n1][d], [n1]
    int n1;
    float* out1;                    // [n_tok][n1]
    float* part;                    // split-d partial sums [nsplit][n_tok][n0 + n1] (gate_project_split)
};
// Split-d form of the gate projection for up to GP_SPLIT_MAX_TOK tokens: its d splits, whose partial sums
// [nsplit][n_tok][nout] fp32 are the workspace. Above that the workspace holds W^T split into bf16 high and low parts
// in MFMA B-fragment order: 2 ceil(d / 256) sub-steps of 128 elements, 8 KB per 16 outputs each.
constexpr long GP_SPLIT_MAX_TOK = 4096;
inline int gate_project_nsplit(long n_tok, int d) {
    if (n_tok > GP_SPLIT_MAX_TOK) return 0;
    const long tiles = (n_tok + 15) / 16, steps = (d + 127) / 128;
    long ns = 1024 / (tiles > 0 ? tiles : 1);
    return (int)(ns < 1 ? 1 : (ns > steps ? steps : ns));
}
inline int gate_project_wsplit_substeps(int d) { return 2 * ((d + 255) / 256); }
inline size_t gate_project_workspace(long n_tok, int d, int nout) {
    if (n_tok > GP_SPLIT_MAX_TOK)
        return (size_t)gate_project_wsplit_substeps(d) * (size_t)((nout + 15) / 16) * 8 * 1024;
    return (size_t)gate_project_nsplit(n_tok, d) * (size_t)n_tok * (size_t)nout * sizeof(float);
}
int gate_project_dispatch(const GateProjArgs& a, hipStream_t stream);
int mem_project_dispatch(const MemProjArgs& a, hipStream_t stream);
int window_fa_dispatch(const WinArgs& a, hipStream_t stream);

struct KvArgs {
    int B, T, G, R, D, dtype;       // T queries per sequence at positions n - T .. n - 1; q, k, v dtype (f32 / bf16)
    const void* q;                  // [B][T][G*R][D]
    const void* k;                  // key (b, g) rows at k + (b * G + g) * k_sbg + pos * k_st
    const void* v;                  // value rows, same addressing with v_sbg / v_st
    long k_sbg, k_st, v_sbg, v_st;
    long n;                         // cached keys (positions 0 .. n - 1)
    int retrieval;                  // 0: each query attends to every key up to its position
    int sinks, window, L;           // S, W, block length; blocks start after the first S keys
    int nb;                         // full blocks after the sinks, (n - S) / L
    // summaries
    int sum_first, nb_cap;          // summarise blocks [sum_first, nb); arrays hold nb_cap blocks per (b, g)
    void* kmin;                     // key dtype, [B][G][D / GS][nb_cap][GS], GS = 16 bytes / element
    void* kmax;
    // selection
    int K;                          // blocks to select
    int* sel;                       // [B][T][G][K] block ids, -1 = none
    // attention
    float scale;
    int slen, nsplit;               // keys per split (<= 512), splits
    float* ws_part;                 // [B][T][G][nsplit][R][D + 2]
    void* o;                        // [B][T][G*R][D] o_dtype
    int o_dtype;
};
int kv_dispatch(const KvArgs& a, int what, hipStream_t stream);   // what: 0 summaries, 1 selection, 2 attention

struct GdnBwdArgs {
    // inputs, fp32, token-major: q, dO [N_tok][G*R][D]; k, v [N_tok][G][D]; g, beta [N_tok][G]; N_tok = num_seqs *
    // n_chunks * 64; s0, dsf [num_seqs][G][D][D] or null (zero)
    const float *q, *k, *v, *g, *beta, *s0, *dO, *dsf;
    float scale;
    int num_seqs, n_chunks, G, R, D;
    // outputs (same layouts); ds0 may be null
    float *dq, *dk, *dv, *dg, *dbeta, *ds0;
    // workspace, chunk-major [chunk][g][...] (cg = chunk * G + g)
    float *gam, *eg, *dgz, *Am, *Mi, *dA, *kb, *vb, *kbe, *ktl, *ktlF, *ktlTF, *u, *w, *wF, *wTF, *attn, *dattn, *qdot, *zr, *zc, *zrA, *zcA;
    float *Sc, *E2, *dSx, *part, *psd;
    float *E1, *dvn, *vn, *dkt, *dw, *dvb, *dkbe, *dkb, *dkacc;
};
size_t gdn_bwd_workspace(int num_seqs, long T, int G, int R, int D);
int gdn_bwd(GdnBwdArgs a, void* ws, hipStream_t stream);

struct LlamaStateArgs {
    int B, G, D, W, S, kv_dtype, n_sinks;
    long n, LR, row;                // tokens seen; region slots; floats per row
    const void *ring_k, *ring_v, *sink_k, *sink_v;
    const float *ring_km, *ring_g, *ring_beta, *state;
    const int64_t* ring_pos;
    float* rows;                    // [B][row]: written by pack, read by unpack
    void *ring_k_out, *ring_v_out, *sink_k_out, *sink_v_out;
    float *ring_km_out, *ring_g_out, *ring_beta_out, *state_out;
    int64_t* ring_pos_out;
};
long llama_state_floats(int G, int D, int W, int S);
int llama_state(const LlamaStateArgs& a, bool pack, hipStream_t stream);

struct LayerArgs {
    int B, G, R, D, T, W, Tq, qoff;     // chunk of T tokens; Tq memory queries from chunk token qoff on
    long start;
    int in_dtype, qm_dtype, km_dtype;
    const void *qm, *km, *kr, *v;
    const float *g, *beta;
    long k_sb, k_sh, k_st, v_sb, v_sh, v_st;
    const void* ring_v;
    const float *ring_km, *ring_g, *ring_beta;
    const int64_t* ring_pos;
    void *wq, *wk, *wv;                 // the GDN inputs [B Tq][H | G][D]
    float *wg, *wb;
    const void* om;                     // the GDN output [B Tq][H][D]
    void* o_mem;                        // [B][T][H][D]
    void *ring_k_w, *ring_v_w;
    float *ring_km_w, *ring_g_w, *ring_beta_w;
    int64_t* ring_pos_w;
    const float* s_new;
    float* state;
};
int layer_launch(const LayerArgs& a, int what, hipStream_t s);   // 0 stream, 1 place, 2 write-back, 3 state, 4 query

struct KvAppendArgs {
    const void* k_new;              // row (b, g, i) at k_new + b * k_sb + g * k_sg + i * k_st (elements)
    const void* v_new;
    long k_sb, k_sg, k_st, v_sb, v_sg, v_st;
    int B, G, t, D, esz;            // esz: bytes per element
    void* k_buf;                    // [B][G][cap][D]
    void* v_buf;
    long cap, n0;                   // rows go to positions n0 .. n0 + t - 1
};
int kv_append(const KvAppendArgs& a, hipStream_t stream);
long kv_max_keys(const KvArgs& a);   // attended keys of one query at most
void kv_split_plan(const KvArgs& a, int* slen, int* nsplit);
int kv_max_k();
int kv_max_blocks();
int kv_max_splits();


struct GdnInArgs {
    const void* z;            // [N_tok][C] in_dtype rows (C = (2 HK + HV) D channels [q | k | v]), z_st elements apart
    long z_st;
    const void* prefix;       // [num_seqs][K - 1][C] in_dtype: the rows before each sequence's start, or null (zeros)
    int in_dtype;
    const float* w;           // [C][K] conv weights, column K - 1 = the current token
    const float* a;           // [N_tok][HV]
    const float* b;           // [N_tok][HV]
    const float* A_log;       // [HV]
    const float* dt_bias;     // [HV]
    const int32_t* cu_seqlens;  // [num_seqs + 1]
    int num_seqs;
    long n_tok;
    int HK, HV, D, K;
    int out_dtype;
    float eps, q_scale;
    void* q;                  // [N_tok][HV][D] out_dtype
    void* k;                  // [N_tok][HV][D] out_dtype
    void* v;                  // [N_tok][HV][D] out_dtype
    float* g;                 // [N_tok][HV]
    float* beta;              // [N_tok][HV]
};
int gdn_conv_inputs_dispatch(const GdnInArgs& a, hipStream_t stream);

struct GatedNormArgs {
    const void* o;            // [rows][D] o_dtype
    int o_dtype;
    const void* z;            // [rows][D] io_dtype gate
    const float* w;           // [D]
    void* out;                // [rows][D] io_dtype
    int io_dtype;
    long rows;
    int D;
    float eps;
};
int gated_norm_dispatch(const GatedNormArgs& a, hipStream_t stream);
   // bf16 operands

}  // namespace bf
