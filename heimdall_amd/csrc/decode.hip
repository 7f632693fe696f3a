// K3: one decode step of the converted layer for B sequences (one new token each, all at absolute position p), and
// the single-token gated delta-rule step.
//
// Reference semantics (Heimdall/heimdall/hibrit.py:363-424 with t == 1; kernels.py:132-138):
//   window  : keys = sinks (j < ns) + ring entries with max(S, p-W+1) <= pos <= p-1 + the new token (if p >= S);
//             s = qr.k / sqrt(D), lse = log sum exp s, o_win = softmax(s) V
//   memory  : (p >= W) the ring row leaving the window (position p - W, slot p mod W) is written into the state:
//             S <- e^g S;  delta = beta (v - S^T km);  S <- S + km delta^T;   then o_mem = S^T qm per query head
//   mix     : gamma = sigmoid(z + mix_lse (lse - ln W)) [p >= W];  o = o_win + gamma (mem_scale o_mem - o_win)
//   cache   : slot p mod W <- (kr, v, km, g, beta, p)
//
// Layout (row-major): state [B][G][D][D] f32; ring_k, ring_v [B][G][W][D]; ring_km [B][W][G][D] f32;
// ring_g, ring_beta [B][W][G] f32; ring_pos [W] int64; sinks [B][G][ns][D]; qr, qm, o [B][H][D]; kr, v, km [B][G][D].
// Per-sequence positions (pos_arr, the llama.cpp multi-sequence setting): sequence b at position pos_arr[b] with its
// own ring_pos row [b][W] and a fixed sink block [b][g][S][D] whose first min(pos, S) rows are present; the new token
// is written to sink row pos when pos < S, and the memory branch of b is active when pos >= W.
//
// Kernels (two launches per step):
//   decode_main    grid (nsplit, G, B): window split x (a.slots ring slots, decode_split; split 0 also takes the
//                  sinks and the new token, saves the ring row leaving the window and writes the new token's values
//                  into its slot)
//   decode_tail    grid (D/64, G, B): state slab x (64 columns): memory write of the saved row, memory read; then
//                  the merge of the window splits, the gamma mix and o for the slab's 64 dims; the new ring_pos entry
//   gdn_step       grid (D/64, G, B): the state slab pass alone (delta_rule_step)
#include "bf_common.h"
#include "bf_internal.h"

namespace bf {

constexpr int NT_DEC = 256;
constexpr int SLOTS = DECODE_SLOTS;   // ring slots per window split at most (LDS sizing)
constexpr int SCG = 16;          // 4-column groups per state slab (64 columns: 1024 slab workgroups at B = 64, G = 4
                                 // fit one round; 16 / 32 / 128 columns measured 150 / 133 / 134 us per step, 64 131)
constexpr int SCOL = 4 * SCG;    // state columns per slab
constexpr int RMAX = 8;          // query heads per KV head supported by the decode kernels

template <class KV>
__device__ __forceinline__ float kv_ld(const typename KV::T* p) { return KV::to_f(*p); }

// Load 16 consecutive elements (as fp32) starting at p (16-byte aligned).
template <class KV>
__device__ __forceinline__ void ld16f(const typename KV::T* p, float (&out)[16]);
template <>
__device__ __forceinline__ void ld16f<BF16>(const uint16_t* p, float (&out)[16]) {
    const uint4 a = ld16(p), b = ld16(p + 8);
    const uint32_t w[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        out[2 * i] = __uint_as_float(w[i] << 16);
        out[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
    }
}
template <>
__device__ __forceinline__ void ld16f<F32>(const float* p, float (&out)[16]) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float4 v = *reinterpret_cast<const float4*>(p + 4 * i);
        out[4 * i] = v.x; out[4 * i + 1] = v.y; out[4 * i + 2] = v.z; out[4 * i + 3] = v.w;
    }
}

// Sum over the threads of a block that share (tid % SCG): lanes l, l + SCG, .. of each wave, then the 4 waves.
// red: shared scratch of 4 * SCG * NV floats. Returns the total in every thread of the group (tid % SCG).
template <int NV>
__device__ __forceinline__ void reduce_colgroups(float (&v)[NV], float* red) {
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        float x = v[i];
#pragma unroll
        for (int off = SCG; off < 64; off <<= 1) x += __shfl_xor(x, off);
        v[i] = x;
    }
    if (lane < SCG) {
#pragma unroll
        for (int i = 0; i < NV; ++i) red[(wv * SCG + lane) * NV + i] = v[i];
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        const int c = tid & (SCG - 1);
        v[i] = red[(0 * SCG + c) * NV + i] + red[(1 * SCG + c) * NV + i] + red[(2 * SCG + c) * NV + i] +
               red[(3 * SCG + c) * NV + i];
    }
    __syncthreads();
}

// State slab pass for one (b, g): columns [j0, j0 + SCOL). Thread tid owns columns j0 + 4 (tid % SCG) .. +3 of rows
// tid / SCG + (256 / SCG) i. Applies S <- e^{wg} S; delta = wb (wv - S^T wk); S <- S + wk delta^T (skipped when !write), then
// writes o[r][j] = sum_d qm_r[d] S[d][j] for the R query heads. S is updated in place (s_in == s_out allowed).
template <int D, int RMAX>
__device__ __forceinline__ void state_slab(const float* s_in, float* s_out, const float* wk, const float* wv,
                                           float wg, float wb, bool write, const float* qm, int R, long q_stride,
                                           float* om, long o_stride, int j0, float* red) {
    constexpr int RSTEP = 256 / SCG, RPT = D / RSTEP;   // row step, rows per thread
    const int tid = threadIdx.x, cg = tid & (SCG - 1), r0 = tid / SCG;
    const int jc = j0 + 4 * cg;
    float4 s[RPT];
#pragma unroll
    for (int i = 0; i < RPT; ++i) s[i] = nt_ldf4(s_in + (long)(r0 + RSTEP * i) * D + jc);    // streamed: read once
    if (write) {
        const float a = __expf(wg);
        float rc[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int i = 0; i < RPT; ++i) {
            const float k = wk[r0 + RSTEP * i];
            rc[0] += k * s[i].x; rc[1] += k * s[i].y; rc[2] += k * s[i].z; rc[3] += k * s[i].w;
        }
        reduce_colgroups<4>(rc, red);
        const float4 v4 = *reinterpret_cast<const float4*>(wv + jc);
        const float dl[4] = {wb * (v4.x - a * rc[0]), wb * (v4.y - a * rc[1]), wb * (v4.z - a * rc[2]),
                             wb * (v4.w - a * rc[3])};
#pragma unroll
        for (int i = 0; i < RPT; ++i) {
            const float k = wk[r0 + RSTEP * i];
            s[i].x = a * s[i].x + k * dl[0];
            s[i].y = a * s[i].y + k * dl[1];
            s[i].z = a * s[i].z + k * dl[2];
            s[i].w = a * s[i].w + k * dl[3];
        }
    }
#pragma unroll
    for (int i = 0; i < RPT; ++i) nt_stf4(s_out + (long)(r0 + RSTEP * i) * D + jc, s[i]);
    if (!om) return;
    float acc[RMAX * 4];
#pragma unroll
    for (int r = 0; r < RMAX; ++r) {
        float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
        if (r < R) {
#pragma unroll
            for (int i = 0; i < RPT; ++i) {
                const float qv = qm[r * q_stride + r0 + RSTEP * i];
                a0 += qv * s[i].x; a1 += qv * s[i].y; a2 += qv * s[i].z; a3 += qv * s[i].w;
            }
        }
        acc[4 * r] = a0; acc[4 * r + 1] = a1; acc[4 * r + 2] = a2; acc[4 * r + 3] = a3;
    }
    reduce_colgroups<RMAX * 4>(acc, red);
    if (r0 == 0) {
#pragma unroll
        for (int r = 0; r < RMAX; ++r)
            if (r < R) *reinterpret_cast<float4*>(om + r * o_stride + jc) =
                make_float4(acc[4 * r], acc[4 * r + 1], acc[4 * r + 2], acc[4 * r + 3]);
    }
}

// ------------------------------------------------------------------------------------------------------- decode
template <class KV, int D, int RM>
__global__ __launch_bounds__(NT_DEC) void decode_main_kernel(DecodeArgs a) {
    using T = typename KV::T;
    constexpr int RMAX = RM;                    // query heads per KV head this instance supports (R <= RM)
    constexpr int LPS = D / 16;                 // lanes per key slot (16 dims each)
    constexpr int SPW = 64 / LPS;               // slots per wave per iteration
    __shared__ float sc[RMAX][SLOTS + 64];      // scores, then probabilities (ring slots + sinks + new token)
    __shared__ int vis[SLOTS + 64];             // key visible to the query (ring validity and window range)
    __shared__ float part[4][RMAX][D];          // per-wave PV partials
    __shared__ float mx[RMAX], sm[RMAX];

    const int x = blockIdx.x, g = blockIdx.y, b = blockIdx.z;
    const int G = a.G, R = a.R, H = G * R, W = a.W;
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const long bg = (long)b * G + g;

    // ---- this sequence's position, ring positions and present sinks
    const long pos = a.pos_arr ? a.pos_arr[b] : a.pos;
    int64_t* RPOS = a.ring_pos + (a.pos_arr ? (long)b * W : 0L);
    const int nsk = a.pos_arr ? (int)min((long)a.n_sinks, pos) : a.n_sinks;
    // the new token: its own key (with pos_arr always; otherwise the caller appended it to the sinks while pos < S)
    const bool new_vis = a.pos_arr ? true : pos >= a.sinks;

    // ---- window split x
    const int s0 = x * a.slots, s1 = min(W, s0 + a.slots);
    const int nring = s1 - s0;
    const int nextra = x == 0 ? nsk + 1 : 0;            // sinks and the new token ride on split 0
    const int nkeys = nring + nextra;
    const float scale = rsqrtf((float)D);
    const long lo = max((long)a.sinks, pos - W + 1);    // oldest visible window position

    const int sl = lane / LPS, dl = (lane % LPS) * 16;  // slot within the wave step, dims dl..dl+15
    // bf16 V rows: a lane takes dims 8 lq .. + 7 and D / 2 + 8 lq .. + 7 (each load instruction reads whole 256-byte
    // halves of SPW rows)
    const int lq = lane % LPS;
    auto vdim = [&](int i) { return sizeof(T) == 2 ? (i < 8 ? 8 * lq + i : D / 2 + 8 * lq + i - 8) : dl + i; };
    const T* RK = reinterpret_cast<const T*>(a.ring_k) + bg * W * D;
    const T* RV = reinterpret_cast<const T*>(a.ring_v) + bg * W * D;
    const T* SK = reinterpret_cast<const T*>(a.sink_k) + bg * a.n_sinks * D;
    const T* SV = reinterpret_cast<const T*>(a.sink_v) + bg * a.n_sinks * D;
    const T* NK = reinterpret_cast<const T*>(a.kr) + bg * D;
    const T* NV = reinterpret_cast<const T*>(a.v) + bg * D;

    // key index k in [0, nkeys): ring slot s0 + k, then sinks, then the new token
    auto key_row = [&](int k, const T* ring, const T* sink, const T* nw) -> const T* {
        if (k < nring) return ring + (long)(s0 + k) * D;
        if (k < nring + nsk) return sink + (long)(k - nring) * D;
        return nw;
    };
    // visibility of every key of the split, read once into LDS (its ring_pos loads overlap the first K loads). The
    // loads are issued together, unconditionally (indices clamped to the split): a load under a per-key branch is
    // waited for before the next one.
    {
        constexpr int VI = (SLOTS + 64 + NT_DEC - 1) / NT_DEC;
        long rpv[VI];
#pragma unroll
        for (int u = 0; u < VI; ++u) rpv[u] = RPOS[s0 + min(tid + u * NT_DEC, nring - 1)];
#pragma unroll
        for (int u = 0; u < VI; ++u) {
            const int k = tid + u * NT_DEC;
            if (k < nkeys) {
                const bool v_ = k < nring ? rpv[u] >= lo && rpv[u] <= pos - 1 : (k < nring + nsk ? true : new_vis);
                vis[k] = v_;
            }
        }
    }
    __syncthreads();
    auto visible = [&](int k) -> bool { return vis[k] != 0; };

    // Scores. bf16: MFMA, S^T = K Q^T with 16-key groups of K rows straight from global memory as A fragments and the
    // R query heads as the first R columns of the B fragment (no cross-lane reduction). fp32: a lane-parallel dot
    // product over the LPS lanes of a slot.
    if constexpr (sizeof(T) == 2) {
        constexpr int NKD = D / 32;
        const int l16 = lane & 15, lg = lane >> 4;
        uint4 qf[NKD];
        {
            // all NKD loads issued before any is used, under one dtype branch (lanes past R read head 0, then zero)
            const int r = l16 < R ? l16 : 0;
            const long qrow = ((long)b * H + g * R + r) * D;
            if (a.q_dtype == DT_BF16) {
                const uint16_t* qp = reinterpret_cast<const uint16_t*>(a.qr) + qrow + 8 * lg;
#pragma unroll
                for (int ks = 0; ks < NKD; ++ks) qf[ks] = ld16(qp + 32 * ks);
            } else {
                const float* qp = reinterpret_cast<const float*>(a.qr) + qrow + 8 * lg;
                float4 q0[NKD], q1[NKD];
#pragma unroll
                for (int ks = 0; ks < NKD; ++ks) {
                    q0[ks] = *reinterpret_cast<const float4*>(qp + 32 * ks);
                    q1[ks] = *reinterpret_cast<const float4*>(qp + 32 * ks + 4);
                }
#pragma unroll
                for (int ks = 0; ks < NKD; ++ks)
                    qf[ks] = make_uint4(pack_bf16x2(q0[ks].x, q0[ks].y), pack_bf16x2(q0[ks].z, q0[ks].w),
                                        pack_bf16x2(q1[ks].x, q1[ks].y), pack_bf16x2(q1[ks].z, q1[ks].w));
            }
            if (l16 >= R) {
#pragma unroll
                for (int ks = 0; ks < NKD; ++ks) qf[ks] = zero16();
            }
        }
        // ring keys: two 16-key groups per wave iteration (addresses past the last ring key clamped to it)
        const int ngrp = (nring + 15) / 16;
        const uint16_t* rk16 = reinterpret_cast<const uint16_t*>(RK) + (long)s0 * D + 8 * lg;
        constexpr int KG = D <= 128 ? 4 : 2;              // 16-key groups per wave iteration; the next KG loaded ahead
        auto ldk = [&](int t0, uint4 (&ka)[KG][NKD]) {
#pragma unroll
            for (int u = 0; u < KG; ++u) {
                const int key = min(16 * (t0 + 4 * u) + l16, nring - 1);
#pragma unroll
                for (int ks = 0; ks < NKD; ++ks) ka[u][ks] = ld16(rk16 + (long)key * D + 32 * ks);
            }
        };
        uint4 kc[KG][NKD];
        ldk(wv, kc);
        for (int t0 = wv; t0 < ngrp; t0 += 4 * KG) {
            uint4 kn[KG][NKD];
            ldk(t0 + 4 * KG, kn);
#pragma unroll
            for (int u = 0; u < KG; ++u) {
                const int t = t0 + 4 * u;
                f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int ks = 0; ks < NKD; ++ks) mma<BF16>(acc, kc[u][ks], qf[ks]);
                if (t < ngrp && l16 < R) {
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const int k = 16 * t + 4 * lg + i;
                        if (k < nring) sc[l16][k] = visible(k) ? acc[i] * scale : -INFINITY;
                    }
                }
            }
#pragma unroll
            for (int u = 0; u < KG; ++u)
#pragma unroll
                for (int ks = 0; ks < NKD; ++ks) kc[u][ks] = kn[u][ks];
        }
        // extra keys of split 0 (sinks, new token), wave 0, 16 at a time
        if (nextra > 0 && wv == 0) {
            for (int e0 = 0; e0 < nextra; e0 += 16) {
                const int k = nring + min(e0 + l16, nextra - 1);
                const uint16_t* row = reinterpret_cast<const uint16_t*>(key_row(k, RK, SK, NK)) + 8 * lg;
                uint4 kx[NKD];
#pragma unroll
                for (int ks = 0; ks < NKD; ++ks) kx[ks] = ld16(row + 32 * ks);
                f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int ks = 0; ks < NKD; ++ks) mma<BF16>(acc, kx[ks], qf[ks]);
                if (l16 < R) {
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const int ke = nring + e0 + 4 * lg + i;
                        if (ke < nkeys) sc[l16][ke] = visible(ke) ? acc[i] * scale : -INFINITY;
                    }
                }
            }
        }
    } else {
        float q[RMAX][16];
#pragma unroll
        for (int r = 0; r < RMAX; ++r) {
            if (r < R) {
                if (a.q_dtype == DT_BF16) ld16f<BF16>(reinterpret_cast<const uint16_t*>(a.qr) + ((long)b * H + g * R + r) * D + dl, q[r]);
                else ld16f<F32>(reinterpret_cast<const float*>(a.qr) + ((long)b * H + g * R + r) * D + dl, q[r]);
#pragma unroll
                for (int i = 0; i < 16; ++i) q[r][i] *= scale;
            } else {
#pragma unroll
                for (int i = 0; i < 16; ++i) q[r][i] = 0.f;
            }
        }
        for (int k0 = wv * SPW; k0 < nkeys; k0 += 4 * SPW) {
            const int k = k0 + sl;
            float kv[16];
            ld16f<KV>(key_row(min(k, nkeys - 1), RK, SK, NK) + dl, kv);
            float d[RMAX];
#pragma unroll
            for (int r = 0; r < RMAX; ++r) {
                d[r] = 0.f;
#pragma unroll
                for (int i = 0; i < 16; ++i) d[r] += q[r][i] * kv[i];
            }
#pragma unroll
            for (int r = 0; r < RMAX; ++r)
#pragma unroll
                for (int off = 1; off < LPS; off <<= 1) d[r] += __shfl_xor(d[r], off);
            if (k < nkeys && (lane % LPS) == 0) {
                const bool vis = visible(k);
#pragma unroll
                for (int r = 0; r < RMAX; ++r)
                    if (r < R) sc[r][k] = vis ? d[r] : -INFINITY;
            }
        }
    }
    // bf16: this wave's first V rows are loaded before the softmax barrier, so the V stream starts while the scores
    // finish
    constexpr int U = RM <= 4 ? 4 : 2;
    const uint16_t* rv16 = reinterpret_cast<const uint16_t*>(RV) + (long)s0 * D + 8 * lq;
    auto ldv = [&](int k0, uint4 (&vr)[U][2]) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int k = min(k0 + u * SPW + sl, nring - 1);
            vr[u][0] = ld16(rv16 + (long)k * D);
            vr[u][1] = ld16(rv16 + (long)k * D + D / 2);
        }
    };
    uint4 cur[U][2];
    if constexpr (sizeof(T) == 2) ldv(wv * SPW * U, cur);
    __syncthreads();
    // max and exp-sum per head (wave r handles head r, r + 4, ...)
    for (int r = wv; r < R; r += 4) {
        float m = -INFINITY;
        for (int k = lane; k < nkeys; k += 64) m = fmaxf(m, sc[r][k]);
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off));
        float l = 0.f;
        for (int k = lane; k < nkeys; k += 64) {
            const float p = m == -INFINITY ? 0.f : __expf(sc[r][k] - m);
            sc[r][k] = p;
            l += p;
        }
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) l += __shfl_xor(l, off);
        if (lane == 0) { mx[r] = m; sm[r] = l; }
    }
    __syncthreads();
    // P V
    float acc[RMAX][16];
#pragma unroll
    for (int r = 0; r < RMAX; ++r)
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[r][i] = 0.f;
    // ring keys: U slot steps per wave iteration, every lane's U rows loaded before use (addresses past the last
    // ring key are clamped to it and their probabilities taken as zero). bf16: the rows stay packed in registers and
    // the next iteration's rows are loaded while the current ones are accumulated.
    if constexpr (sizeof(T) == 2) {
        int k0 = wv * SPW * U;
        for (; k0 < nring; k0 += 4 * SPW * U) {
            uint4 nxt[U][2];
            ldv(min(k0 + 4 * SPW * U, nring - 1), nxt);
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int k = k0 + u * SPW + sl;
                const uint32_t w[8] = {cur[u][0].x, cur[u][0].y, cur[u][0].z, cur[u][0].w,
                                       cur[u][1].x, cur[u][1].y, cur[u][1].z, cur[u][1].w};
#pragma unroll
                for (int r = 0; r < RMAX; ++r) {
                    const float p = (r < R && k < nring) ? sc[r][k < nring ? k : 0] : 0.f;
#pragma unroll
                    for (int i = 0; i < 8; ++i) {
                        acc[r][2 * i] += p * __uint_as_float(w[i] << 16);
                        acc[r][2 * i + 1] += p * __uint_as_float(w[i] & 0xffff0000u);
                    }
                }
            }
#pragma unroll
            for (int u = 0; u < U; ++u) { cur[u][0] = nxt[u][0]; cur[u][1] = nxt[u][1]; }
        }
    } else
    for (int k0 = wv * SPW * U; k0 < nring; k0 += 4 * SPW * U) {
        float vv[U][16];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int k = min(k0 + u * SPW + sl, nring - 1);
            ld16f<KV>(RV + (long)(s0 + k) * D + dl, vv[u]);
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int k = k0 + u * SPW + sl;
#pragma unroll
            for (int r = 0; r < RMAX; ++r) {
                const float p = (r < R && k < nring) ? sc[r][k < nring ? k : 0] : 0.f;
#pragma unroll
                for (int i = 0; i < 16; ++i) acc[r][i] += p * vv[u][i];
            }
        }
    }
    // extra keys of split 0 (sinks, new token)
    for (int k0 = nring + wv * SPW; k0 < nkeys; k0 += 4 * SPW) {
        const int k = k0 + sl;
        float vv[16];
        if constexpr (sizeof(T) == 2) {
            const T* row = key_row(min(k, nkeys - 1), RV, SV, NV);
            const uint4 h0 = ld16(row + 8 * lq), h1 = ld16(row + D / 2 + 8 * lq);
            const uint32_t w[8] = {h0.x, h0.y, h0.z, h0.w, h1.x, h1.y, h1.z, h1.w};
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                vv[2 * i] = __uint_as_float(w[i] << 16);
                vv[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
            }
        } else {
            ld16f<KV>(key_row(min(k, nkeys - 1), RV, SV, NV) + dl, vv);
        }
#pragma unroll
        for (int r = 0; r < RMAX; ++r) {
            const float p = (r < R && k < nkeys) ? sc[r][k < nkeys ? k : 0] : 0.f;
#pragma unroll
            for (int i = 0; i < 16; ++i) acc[r][i] += p * vv[i];
        }
    }
    // reduce over the SPW slot groups of the wave (lanes with equal lane % LPS), then over the 4 waves
#pragma unroll
    for (int r = 0; r < RMAX; ++r)
#pragma unroll
        for (int i = 0; i < 16; ++i)
#pragma unroll
            for (int off = LPS; off < 64; off <<= 1) acc[r][i] += __shfl_xor(acc[r][i], off);
    if (lane < LPS) {
#pragma unroll
        for (int r = 0; r < RMAX; ++r)
            if (r < R) {
#pragma unroll
                for (int i = 0; i < 16; ++i) part[wv][r][vdim(i)] = acc[r][i];
            }
    }
    __syncthreads();
    // partial record for this split: [m, l, o[0..D)] per head
    float* out = a.ws_part + ((bg * a.nsplit + x) * R) * (D + 2);
    for (int idx = tid; idx < R * D; idx += NT_DEC) {
        const int r = idx / D, dd = idx % D;
        out[r * (D + 2) + 2 + dd] = part[0][r][dd] + part[1][r][dd] + part[2][r][dd] + part[3][r][dd];
    }
    if (tid < R) {
        out[tid * (D + 2)] = mx[tid];
        out[tid * (D + 2) + 1] = sm[tid];
    }
    if (x != 0) return;
    // Split 0: the ring row of slot pos mod W (position pos - W, leaving the window) into ws_ev for the state update
    // of decode_tail_kernel, then the new token into that slot. No split reads the slot's values: its ring_pos
    // (pos - W or older, rewritten by the tail) keeps it out of every window, so its scores are masked.
    const int slot = (int)(pos % W);
    const long pe = pos - W, rg = ((long)b * W + slot) * G + g;
    T* RKs = reinterpret_cast<T*>(a.ring_k) + (bg * W + slot) * D;
    T* RVs = reinterpret_cast<T*>(a.ring_v) + (bg * W + slot) * D;
    float* KM = a.ring_km + rg * D;
    float* ev = a.ws_ev + bg * (2 * D + 4);
    for (int d = tid; d < D; d += NT_DEC) {
        const float vv = KV::to_f(RVs[d]), kk = KM[d];
        ev[d] = vv;
        ev[D + d] = kk;
        RKs[d] = NK[d];
        RVs[d] = NV[d];
        KM[d] = a.km[bg * D + d];
    }
    if (a.pos_arr && pos < a.n_sinks) {                 // the new token becomes sink row pos (no split reads it)
        T* sk = reinterpret_cast<T*>(a.sink_k) + (bg * a.n_sinks + pos) * D;
        T* sv = reinterpret_cast<T*>(a.sink_v) + (bg * a.n_sinks + pos) * D;
        for (int d = tid; d < D; d += NT_DEC) {
            sk[d] = NK[d];
            sv[d] = NV[d];
        }
    }
    if (tid == 0) {
        const bool valid = pe >= 0 && RPOS[slot] == pe;
        ev[2 * D] = a.ring_g[rg];
        ev[2 * D + 1] = a.ring_beta[rg];
        ev[2 * D + 2] = valid ? 1.f : 0.f;
        a.ring_g[rg] = a.g_new[bg];
        a.ring_beta[rg] = a.beta_new[bg];
    }
}

// After the window splits: state slab x (SCOL columns) of (b, g) and the output dims of those columns.
//  - memory on: the write of the ring row that left the window (from ws_ev), then the memory read of the R query
//    heads for the slab's columns (into ws_om);
//  - the merge of the window splits for the slab's dims and every query head, the gamma mix, o and lse;
//  - the ring_pos entry of the new token (its values were written by split 0 of the window kernel).
template <class KV, int D, int RM>
__global__ __launch_bounds__(NT_DEC) void decode_tail_kernel(DecodeArgs a) {
    constexpr int MAXS = 64;                            // window splits held in LDS (W <= 65536)
    __shared__ float red[4 * SCG * RM * 4];
    __shared__ float fs[RM][MAXS];
    __shared__ float st2[RM][2];
    const int x = blockIdx.x, g = blockIdx.y, b = blockIdx.z;
    const int G = a.G, R = a.R, H = G * R, W = a.W, NS = a.nsplit;
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const long bg = (long)b * G + g;
    const int j0 = x * SCOL;
    const long pos = a.pos_arr ? a.pos_arr[b] : a.pos;
    const bool mem_on = a.mem_on && (!a.pos_arr || pos >= W);
    float* om = a.ws_om + ((long)b * H + g * R) * D;
    if (mem_on) {
        const float* ev = a.ws_ev + bg * (2 * D + 4);
        const bool valid = ev[2 * D + 2] != 0.f;
        const float wg = valid ? ev[2 * D] : 0.f, wb = valid ? ev[2 * D + 1] : 0.f;
        float* S = a.state + bg * D * D;
        state_slab<D, RM>(S, S, ev + D, ev, wg, wb, valid, a.qm + ((long)b * H + g * R) * D, R, D, om, D, j0, red);
    }
    // split statistics per head (wave w takes heads w, w + 4): M = max m_s, f_s = e^{m_s - M}, L = sum f_s l_s
    const float* part = a.ws_part + bg * NS * R * (D + 2);
    for (int r = wv; r < R; r += NT_DEC / 64) {
        const float ms = lane < NS ? part[(lane * R + r) * (D + 2)] : -INFINITY;
        const float ls = lane < NS ? part[(lane * R + r) * (D + 2) + 1] : 0.f;
        float M = ms;
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) M = fmaxf(M, __shfl_xor(M, off));
        const float f = ms == -INFINITY ? 0.f : __expf(ms - M);
        float L = f * ls;
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) L += __shfl_xor(L, off);
        if (lane < NS) fs[r][lane] = f;
        if (lane == 0) { st2[r][0] = M; st2[r][1] = L; }
    }
    __syncthreads();                                    // also orders the slab's om stores before their reads below
    const float lnW = logf((float)W);
    for (int i = tid; i < R * SCOL; i += NT_DEC) {
        const int r = i / SCOL, d = j0 + i % SCOL, h = g * R + r;
        const float M = st2[r][0], L = st2[r][1];
        float ow = 0.f;
        for (int s_ = 0; s_ < NS; ++s_) ow += fs[r][s_] * part[(s_ * R + r) * (D + 2) + 2 + d];
        ow /= L;
        const float lse = M + logf(L);
        float o = ow;
        if (mem_on) {
            const float gam = 1.f / (1.f + __expf(-(a.z[(long)b * H + h] + a.mix_lse[h] * (lse - lnW))));
            o = ow + gam * (a.mem_scale[h] * om[r * D + d] - ow);
        }
        a.o[((long)b * H + h) * D + d] = o;
        if (x == 0 && i % SCOL == 0 && a.lse) a.lse[(long)b * H + h] = lse;
    }
    if (x == 0 && g == 0 && tid == 0 && (a.pos_arr || b == 0)) a.ring_pos[(a.pos_arr ? (long)b * W : 0L) + pos % W] = pos;
}

// ----------------------------------------------------------------------------------------------- single-token GDN
template <int D>
__global__ __launch_bounds__(NT_DEC) void gdn_step_kernel(StepArgs a) {
    __shared__ float red[4 * SCG * RMAX * 4];
    const int x = blockIdx.x, g = blockIdx.y, b = blockIdx.z;
    const int G = a.G, R = a.R, H = G * R;
    const long bg = (long)b * G + g;
    state_slab<D, RMAX>(a.s_in + bg * D * D, a.s_out + bg * D * D, a.k + bg * D, a.v + bg * D, a.g[bg], a.beta[bg], true,
                  a.q + ((long)b * H + g * R) * D, R, D, a.o + ((long)b * H + g * R) * D, D, x * SCOL, red);
}

// ------------------------------------------------------------------------------------------------ host launchers
template <class KV, int D>
static int launch_decode(const DecodeArgs& a, hipStream_t stream) {
    if (a.nsplit > 64) return BF_STATUS_UNSUPPORTED;
    hipError_t e;
    if (a.R <= 4) hipLaunchKernelGGL((decode_main_kernel<KV, D, 4>), dim3(a.nsplit, a.G, a.B), dim3(NT_DEC), 0, stream, a);
    else hipLaunchKernelGGL((decode_main_kernel<KV, D, 8>), dim3(a.nsplit, a.G, a.B), dim3(NT_DEC), 0, stream, a);
    if ((e = hipGetLastError()) != hipSuccess) return (int)e;
    if (a.R <= 4) hipLaunchKernelGGL((decode_tail_kernel<KV, D, 4>), dim3(D / SCOL, a.G, a.B), dim3(NT_DEC), 0, stream, a);
    else hipLaunchKernelGGL((decode_tail_kernel<KV, D, 8>), dim3(D / SCOL, a.G, a.B), dim3(NT_DEC), 0, stream, a);
    e = hipGetLastError();
    return e == hipSuccess ? 0 : (int)e;
}

int decode_dispatch(const DecodeArgs& a, hipStream_t stream) {
    const bool bf = a.kv_dtype == DT_BF16;
    switch (a.D) {
        case 64: return bf ? launch_decode<BF16, 64>(a, stream) : launch_decode<F32, 64>(a, stream);
        case 128: return bf ? launch_decode<BF16, 128>(a, stream) : launch_decode<F32, 128>(a, stream);
        case 256: return bf ? launch_decode<BF16, 256>(a, stream) : launch_decode<F32, 256>(a, stream);
        default: return BF_ERR_UNSUPPORTED;
    }
}

template <int D>
static int launch_step(const StepArgs& a, hipStream_t stream) {
    hipLaunchKernelGGL((gdn_step_kernel<D>), dim3(D / SCOL, a.G, a.B), dim3(NT_DEC), 0, stream, a);
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? 0 : (int)e;
}

int step_dispatch(const StepArgs& a, hipStream_t stream) {
    switch (a.D) {
        case 64: return launch_step<64>(a, stream);
        case 128: return launch_step<128>(a, stream);
        case 256: return launch_step<256>(a, stream);
        default: return BF_ERR_UNSUPPORTED;
    }
}

}  // namespace bf
