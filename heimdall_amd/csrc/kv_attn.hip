// Attention of the kept full-attention layers over a dense KV cache (reference: HybridAttention._teacher,
// Heimdall/heimdall/hibrit.py:275-290), for the T most recent queries of each sequence (T = 1: decode), with or
// without retrieval (Quest-style block selection, _retrieval_mask hibrit.py:301-324). Query i sits at position
// p = n - T + i and attends to
//   retrieval off:  the keys 0 .. p
//   retrieval on:   the sinks 0 .. S - 1, the K key blocks (L keys each, block j = keys S + j L ..) with the highest
//                   upper bound on q.k among the nc = min(max(p - W + 1 - S, 0) / L, nb) blocks that end before the
//                   window, and the window S + nc L .. p.
// The upper bound of block j for query head r is sum_d max(q_rd kmin_jd, q_rd kmax_jd) with the per-dimension key
// minimum and maximum of the block; one selection per KV head takes the maximum over its R query heads.
//
// kv_summary_kernel   per (block, G, B): the key min / max of a block, one wave per block (kept by the caller for
//                     the full blocks of a growing cache, so a decode step summarises only new blocks).
// kv_select_kernel    per (query, G): upper bounds of the candidate blocks into LDS, then K rounds of a block-wide
//                     arg max (ties to the lower block index) -> the selected block ids.
// kv_split_kernel     per (query, split, G): KV_SPLIT consecutive keys of the attended list (sinks, selected blocks
//                     in ascending order, window); scores for the R heads with 16 lanes per key, the split's max / sum
//                     / unnormalised output per head into the workspace. Every K and V row is one 16-byte-vector
//                     read per lane.
// kv_combine_kernel   per (query, head): the splits merged into o.
#include "bf_common.h"
#include "bf_internal.h"

namespace bf {

namespace {

constexpr int KV_SPLIT = 512;       // attended keys per split at most (the split length is chosen per launch)
constexpr int KV_NT = 256;          // threads per workgroup
constexpr int KV_NW = KV_NT / 64;   // waves per workgroup
constexpr int KV_MAXR = 8;          // query heads per KV head at most
constexpr int KV_MAXK = 64;         // selected blocks at most
constexpr int KV_MAXNB = 16384;     // candidate blocks at most (upper bounds held in LDS)
constexpr int KV_MAXSPLIT = 2048;   // splits at most (attended keys <= 2048 * 512)

// N consecutive elements from element index i of a row, as fp32; i is a multiple of min(N, 16 bytes / element)
template <class E, int N>
__device__ __forceinline__ void ldv(const void* base, long i, float (&x)[N]) {
    if constexpr (sizeof(typename E::T) == 2) {
        const uint16_t* s = reinterpret_cast<const uint16_t*>(base) + i;
        if constexpr (N % 8 == 0) {
#pragma unroll
            for (int c = 0; c < N / 8; ++c) {
                const uint4 u = *reinterpret_cast<const uint4*>(s + 8 * c);
                const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    x[8 * c + 2 * j] = __uint_as_float(w[j] << 16);
                    x[8 * c + 2 * j + 1] = __uint_as_float(w[j] & 0xffff0000u);
                }
            }
        } else if constexpr (N == 4) {
            const uint2 u = *reinterpret_cast<const uint2*>(s);
            x[0] = __uint_as_float(u.x << 16);
            x[1] = __uint_as_float(u.x & 0xffff0000u);
            x[2] = __uint_as_float(u.y << 16);
            x[3] = __uint_as_float(u.y & 0xffff0000u);
        } else if constexpr (N == 2) {
            const uint32_t u = *reinterpret_cast<const uint32_t*>(s);
            x[0] = __uint_as_float(u << 16);
            x[1] = __uint_as_float(u & 0xffff0000u);
        } else {
#pragma unroll
            for (int e = 0; e < N; ++e) x[e] = bf2f(s[e]);
        }
    } else {
        const float* s = reinterpret_cast<const float*>(base) + i;
        if constexpr (N % 4 == 0) {
#pragma unroll
            for (int c = 0; c < N / 4; ++c) {
                const float4 u = *reinterpret_cast<const float4*>(s + 4 * c);
                x[4 * c] = u.x; x[4 * c + 1] = u.y; x[4 * c + 2] = u.z; x[4 * c + 3] = u.w;
            }
        } else if constexpr (N == 2) {
            const float2 u = *reinterpret_cast<const float2*>(s);
            x[0] = u.x; x[1] = u.y;
        } else {
#pragma unroll
            for (int e = 0; e < N; ++e) x[e] = s[e];
        }
    }
}

template <int N>
__device__ __forceinline__ void ldf(const float* s, float (&x)[N]) {
    if constexpr (N % 4 == 0) {
#pragma unroll
        for (int c = 0; c < N / 4; ++c) {
            const float4 u = *reinterpret_cast<const float4*>(s + 4 * c);
            x[4 * c] = u.x; x[4 * c + 1] = u.y; x[4 * c + 2] = u.z; x[4 * c + 3] = u.w;
        }
    } else {
#pragma unroll
        for (int e = 0; e < N; ++e) x[e] = s[e];
    }
}

// the DPL dims of one of LPK lanes sharing a row of D elements: with whole 16-byte chunks per lane, lane l takes chunks
// l, l + LPK, l + 2 LPK, ... (each load instruction of the LPK lanes reads a contiguous span of the row); with less
// than a chunk per lane, the DPL consecutive dims from l DPL.
template <class E, int D, int LPK>
__device__ __forceinline__ void ld_rowpart(const void* base, long row, int l, float (&x)[D / LPK]) {
    constexpr int DPL = D / LPK, VE = 16 / (int)sizeof(typename E::T);
    if constexpr (DPL >= VE) {
#pragma unroll
        for (int c = 0; c < DPL / VE; ++c) {
            float y[VE];
            ldv<E, VE>(base, row + (long)(l + LPK * c) * VE, y);
#pragma unroll
            for (int e = 0; e < VE; ++e) x[c * VE + e] = y[e];
        }
    } else {
        ldv<E, DPL>(base, row + (long)l * DPL, x);
    }
}

// the 16 / sizeof(T) elements of a 16-byte vector as fp32
template <class E>
__device__ __forceinline__ void unpack16(const uint4& u, float (&x)[16 / sizeof(typename E::T)]) {
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
    if constexpr (sizeof(typename E::T) == 2) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            x[2 * j] = __uint_as_float(w[j] << 16);
            x[2 * j + 1] = __uint_as_float(w[j] & 0xffff0000u);
        }
    } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) x[j] = __uint_as_float(w[j]);
    }
}

// the attended key list of query i: ns sinks, the selected blocks, the window win0 .. end - 1
struct KvQuery {
    long end, win0;
    int ns, nc;
};

__device__ __forceinline__ KvQuery kv_query(const KvArgs& a, int i) {
    KvQuery q;
    const long p = a.n - a.T + i;
    q.end = p + 1;
    if (a.retrieval) {
        const long c = max(p - a.window + 1 - a.sinks, 0L) / a.L;
        q.nc = (int)min(c, (long)a.nb);
        q.ns = a.sinks;
        q.win0 = a.sinks + (long)q.nc * a.L;
    } else {
        q.nc = 0;
        q.ns = 0;
        q.win0 = 0;
    }
    return q;
}

// cache position of attended key v (the list: sinks, selected blocks in ascending order, window)
__device__ __forceinline__ long kv_key_pos(const KvArgs& a, const KvQuery& qi, const int* blk, int nsel, long v) {
    if (v < qi.ns) return v;
    v -= qi.ns;
    if (v < (long)nsel * a.L) return a.sinks + (long)blk[v / a.L] * a.L + v % a.L;
    return qi.win0 + (v - (long)nsel * a.L);
}

}  // namespace

// ---- block summaries: wave w of the workgroup summarises block sum_first + blockIdx.x * 4 + w. kmin / kmax hold the
// key dtype (the min / max of a key dimension is one of its values, so no rounding) in the layout
// [B][G][D / GS][nb_cap][GS], GS = 16 bytes / element: the GS consecutive dims of one block are one 16-byte vector and
// the blocks of one dim group are consecutive, so the selection reads them as coalesced vectors, one lane per block.
template <class E, int D>
__global__ __launch_bounds__(KV_NT) void kv_summary_kernel(KvArgs a) {
    using T = typename E::T;
    constexpr int DPL = D / 64;                           // dims per lane
    constexpr int GS = 16 / (int)sizeof(T);
    const int lane = lane_id(), wv = wave_id();
    const int g = blockIdx.y, b = blockIdx.z;
    const int j = a.sum_first + blockIdx.x * KV_NW + wv;  // block id
    if (j >= a.nb) return;
    const long bg = (long)b * a.G + g;
    const long key0 = a.sinks + (long)j * a.L;
    float mn[DPL], mx[DPL];
#pragma unroll
    for (int e = 0; e < DPL; ++e) { mn[e] = INFINITY; mx[e] = -INFINITY; }
    for (int r = 0; r < a.L; ++r) {
        float x[DPL];
        ldv<E, DPL>(a.k, bg * a.k_sbg + (key0 + r) * a.k_st + lane * DPL, x);
#pragma unroll
        for (int e = 0; e < DPL; ++e) {
            mn[e] = fminf(mn[e], x[e]);
            mx[e] = fmaxf(mx[e], x[e]);
        }
    }
    T* smin = reinterpret_cast<T*>(a.kmin);
    T* smax = reinterpret_cast<T*>(a.kmax);
#pragma unroll
    for (int e = 0; e < DPL; ++e) {
        const int d = lane * DPL + e;
        const long at = ((bg * (D / GS) + d / GS) * a.nb_cap + j) * GS + d % GS;
        smin[at] = E::from_f(mn[e]);
        smax[at] = E::from_f(mx[e]);
    }
}

// ---- selection: the K candidate blocks with the highest upper bound, per (query, g); KV_SNT threads.
// Bounds: lane per block, each thread walks the D / 4 dim groups of its block in batches of 16 (coalesced 16-byte
// summary vectors, all loads of a batch in flight together), q of the R heads from LDS.
// Top K, ordered by (bound descending, block id ascending): each wave takes K rounds over its slice of the bounds with
// shuffles only (a per-lane mask marks the taken entries), then one wave merges the waves' K-lists the same way.
constexpr int KV_SNT = 512;
constexpr int KV_SNW = KV_SNT / 64;
constexpr int KV_SPL = KV_MAXNB / KV_SNT;                 // bounds per lane in a wave's slice, at most

__device__ __forceinline__ bool kv_better(float v, int i, float bv, int bi) { return v > bv || (v == bv && i < bi); }

// wave-wide arg max of (v, i) by kv_better; every lane returns the winner
__device__ __forceinline__ void kv_wave_argmax(float& v, int& i) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const float ov = __shfl_xor(v, off);
        const int oi = __shfl_xor(i, off);
        if (kv_better(ov, oi, v, i)) { v = ov; i = oi; }
    }
}

template <class E, int D, int RM>
__global__ __launch_bounds__(KV_SNT) void kv_select_kernel(KvArgs a) {
    constexpr int GS = 16 / (int)sizeof(typename E::T);  // dims per 16-byte summary vector
    constexpr int NCG = D / GS, CB = NCG / 2 < 16 ? NCG / 2 : 16;   // >= 2 batches: q reads stay inside the loop
    constexpr int NC4 = D / 4;
    __shared__ float ub[KV_MAXNB];
    __shared__ float4 qs[RM][NC4];
    __shared__ float cv[KV_SNW * KV_MAXK];
    __shared__ int ci[KV_SNW * KV_MAXK];
    const int lane = lane_id(), wv = threadIdx.x / 64, tid = threadIdx.x;
    const int bt = blockIdx.x, g = blockIdx.y;
    const int b = bt / a.T;
    const int R = a.R, H = a.G * R, K = a.K;
    const long bg = (long)b * a.G + g;
    const int nc = kv_query(a, bt % a.T).nc;

    for (int i = tid; i < RM * NC4; i += KV_SNT) {        // heads past R: zero q, bound 0 (never taken)
        const int r = i / NC4, c = i % NC4;
        float x[4] = {0.f, 0.f, 0.f, 0.f};
        if (r < R) ldv<E, 4>(a.q, ((long)bt * H + g * R + r) * D + 4 * c, x);
        qs[r][c] = make_float4(x[0], x[1], x[2], x[3]);
    }
    __syncthreads();
    const long sbase = bg * NCG * a.nb_cap * GS;           // element offset of (b, g)'s summaries
    for (int j = tid; j < nc; j += KV_SNT) {
        float s[RM];
#pragma unroll
        for (int r = 0; r < RM; ++r) s[r] = 0.f;
#pragma unroll 1
        for (int c0 = 0; c0 < NCG; c0 += CB) {
            uint4 lo[CB], hi[CB];
#pragma unroll
            for (int u = 0; u < CB; ++u) {
                const long at = (sbase + ((long)(c0 + u) * a.nb_cap + j) * GS) * (long)sizeof(typename E::T);
                lo[u] = ld16(reinterpret_cast<const char*>(a.kmin) + at);
                hi[u] = ld16(reinterpret_cast<const char*>(a.kmax) + at);
            }
#pragma unroll
            for (int u = 0; u < CB; ++u) {
                float l[GS], h[GS];
                unpack16<E>(lo[u], l);
                unpack16<E>(hi[u], h);
#pragma unroll
                for (int r = 0; r < RM; ++r) {
#pragma unroll
                    for (int q4 = 0; q4 < GS / 4; ++q4) {
                        const float4 q = qs[r][(c0 + u) * (GS / 4) + q4];
                        const float* lq = l + 4 * q4;
                        const float* hq = h + 4 * q4;
                        s[r] += fmaxf(q.x * lq[0], q.x * hq[0]) + fmaxf(q.y * lq[1], q.y * hq[1]) +
                                fmaxf(q.z * lq[2], q.z * hq[2]) + fmaxf(q.w * lq[3], q.w * hq[3]);
                    }
                }
            }
        }
        float best = s[0];
#pragma unroll
        for (int r = 1; r < RM; ++r)
            if (r < R) best = fmaxf(best, s[r]);
        ub[j] = best;
    }
    __syncthreads();
    if (K == 0) return;

    // per-wave top K over the slice [w SL, (w + 1) SL); lane l holds the entries w SL + l + 64 e
    const int SL = (nc + KV_SNW - 1) / KV_SNW;
    const int lo_j = wv * SL, hi_j = min(nc, lo_j + SL);
    uint32_t taken = 0;
    for (int it = 0; it < K; ++it) {
        float bv = -INFINITY;
        int bi = 0x7fffffff;
        int be = -1;
#pragma unroll 4
        for (int e = 0; e < KV_SPL; ++e) {
            const int j = lo_j + lane + 64 * e;
            if (j >= hi_j) break;
            const float v = ub[j];
            if (!((taken >> e) & 1u) && kv_better(v, j, bv, bi)) { bv = v; bi = j; be = e; }
        }
        float wv_ = bv;
        int wi = bi;
        kv_wave_argmax(wv_, wi);
        if (wi == bi && be >= 0 && wv_ > -INFINITY) taken |= 1u << be;
        if (lane == 0) {
            cv[wv * K + it] = wv_;
            ci[wv * K + it] = wv_ > -INFINITY ? wi : 0x7fffffff;
        }
    }
    __syncthreads();
    if (wv != 0) return;
    // merge: wave 0, lane l holds candidates l + 64 e of the KV_SNW x K lists
    const int NCAND = KV_SNW * K;
    uint32_t mt = 0;
    int* sel = a.sel + ((long)bt * a.G + g) * K;
    for (int it = 0; it < K; ++it) {
        float bv = -INFINITY;
        int bi = 0x7fffffff;
        int be = -1;
#pragma unroll
        for (int e = 0; e < KV_SNW * KV_MAXK / 64; ++e) {
            const int c = lane + 64 * e;
            if (c >= NCAND) break;
            const float v = cv[c];
            const int i = ci[c];
            if (!((mt >> e) & 1u) && kv_better(v, i, bv, bi)) { bv = v; bi = i; be = e; }
        }
        float mv = bv;
        int mi = bi;
        kv_wave_argmax(mv, mi);
        if (mi == bi && be >= 0 && mv > -INFINITY) mt |= 1u << be;
        if (lane == 0) sel[it] = (mv > -INFINITY && mi < nc) ? mi : -1;
    }
}

// ---- one split of one query's attended keys; RM >= R query heads per KV head (their q in registers). Each lane
// issues the loads of several keys (score pass) or value rows (P V pass) before using any of them.
template <class E, int D, int RM>
__global__ __launch_bounds__(KV_NT) void kv_split_kernel(KvArgs a) {
    constexpr int LPK = 16, KPW = 64 / LPK;               // score pass: lanes per key, keys per wave step
    constexpr int DPL = D / LPK;                          // dims per lane in the dot product
    constexpr int US = RM * DPL >= 128 ? 2 : 4;           // keys in flight per lane (register budget)
    constexpr int VW = 16 / (int)sizeof(typename E::T);  // value pass: dims per lane (one 16-byte read)
    constexpr int LPV = D / VW < 64 ? D / VW : 64;        // lanes per value row
    constexpr int KPV = 64 / LPV;                         // value rows per wave step
    constexpr int VPL = D / LPV;                          // dims per lane in the value pass
    constexpr int UV = 4;                                 // value rows in flight per lane
    __shared__ float p[RM][KV_SPLIT];                     // scores, then probabilities
    __shared__ int kpos[KV_SPLIT];                        // cache position of each key of the split
    __shared__ int blk[KV_MAXK];
    __shared__ float part[KV_NW][RM][D];
    __shared__ float mxs[RM], sms[RM];
    __shared__ int nsel_s;
    const int lane = lane_id(), wv = wave_id(), tid = threadIdx.x;
    const int bt = blockIdx.x, x = blockIdx.y, g = blockIdx.z;
    const int b = bt / a.T;
    const int R = a.R, H = a.G * R;
    const long bg = (long)b * a.G + g;
    const KvQuery qi = kv_query(a, bt % a.T);

    // the valid selected blocks of (query, g) (ids in [0, nc); their order does not matter), compacted by one wave
    int nsel = 0;
    if (a.retrieval && a.K > 0) {
        if (wv == 0) {
            const int* sel = a.sel + ((long)bt * a.G + g) * a.K;
            const int s = lane < a.K ? sel[lane] : -1;
            const bool ok = s >= 0 && s < qi.nc;
            const unsigned long long m = __ballot(ok);
            if (ok) blk[__popcll(m & ((1ull << lane) - 1ull))] = s;
            if (lane == 0) nsel_s = __popcll(m);
        }
        __syncthreads();
        nsel = nsel_s;
    }
    const long nv = qi.ns + (long)nsel * a.L + max(0L, qi.end - qi.win0);
    const long v0 = (long)x * a.slen;
    const int nk = (int)max(0L, min((long)a.slen, nv - v0));
    float* out = a.ws_part + (((long)bt * a.G + g) * a.nsplit + x) * R * (D + 2);
    if (nk == 0) {                                        // empty split: weight zero in the combine
        for (int i = tid; i < R * (D + 2); i += KV_NT) {
            const int c = i % (D + 2);
            out[i] = c == 0 ? -INFINITY : 0.f;
        }
        return;
    }
    for (int k = tid; k < KV_SPLIT; k += KV_NT)          // positions < n < 2^31; past nk: the last key again
        kpos[k] = (int)kv_key_pos(a, qi, blk, nsel, v0 + (k < nk ? k : nk - 1));
    __syncthreads();

    // scores: 16 lanes per key (dims of lane l: ld_rowpart)
    {
        const int kl = lane / LPK, ll = lane % LPK;
        float q[RM][DPL];
#pragma unroll
        for (int r = 0; r < RM; ++r) {
            if (r < R) {
                ld_rowpart<E, D, LPK>(a.q, ((long)bt * H + g * R + r) * D, ll, q[r]);
#pragma unroll
                for (int e = 0; e < DPL; ++e) q[r][e] *= a.scale;
            } else {
#pragma unroll
                for (int e = 0; e < DPL; ++e) q[r][e] = 0.f;
            }
        }
        constexpr int STEP = KV_NW * KPW;                 // keys per workgroup step
        for (int k0 = wv * KPW + kl; k0 - kl < nk; k0 += STEP * US) {
            float kx[US][DPL];
#pragma unroll
            for (int u = 0; u < US; ++u) {
                const int k = k0 + u * STEP;
                const long pos = kpos[k < KV_SPLIT ? k : KV_SPLIT - 1];
                ld_rowpart<E, D, LPK>(a.k, bg * a.k_sbg + pos * a.k_st, ll, kx[u]);
            }
#pragma unroll
            for (int u = 0; u < US; ++u) {
                const int k = k0 + u * STEP;
#pragma unroll
                for (int r = 0; r < RM; ++r) {
                    if (r >= R) break;
                    float s = 0.f;
#pragma unroll
                    for (int e = 0; e < DPL; ++e) s += q[r][e] * kx[u][e];
#pragma unroll
                    for (int off = LPK / 2; off > 0; off >>= 1) s += __shfl_xor(s, off);
                    if ((lane % LPK) == 0 && k < nk) p[r][k] = s;
                }
            }
        }
    }
    __syncthreads();
    // split max and probabilities per head (wave w handles heads w, w + 4)
    for (int r = wv; r < R; r += KV_NW) {
        float m = -INFINITY;
        for (int k = lane; k < nk; k += 64) m = fmaxf(m, p[r][k]);
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off));
        float l = 0.f;
        for (int k = lane; k < nk; k += 64) {
            const float e = __expf(p[r][k] - m);
            p[r][k] = e;
            l += e;
        }
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) l += __shfl_xor(l, off);
        if (lane == 0) { mxs[r] = m; sms[r] = l; }
    }
    __syncthreads();
    // P V: LPV lanes per value row, KPV rows per wave step
    {
        const int kv = lane / LPV, dv = (lane % LPV) * VPL;
        float acc[RM][VPL];
#pragma unroll
        for (int r = 0; r < RM; ++r)
#pragma unroll
            for (int e = 0; e < VPL; ++e) acc[r][e] = 0.f;
        constexpr int STEP = KV_NW * KPV;                 // value rows per workgroup step
        for (int k0 = wv * KPV + kv; k0 - kv < nk; k0 += STEP * UV) {
            float vx[UV][VPL];
#pragma unroll
            for (int u = 0; u < UV; ++u) {
                const int k = k0 + u * STEP;
                const long pos = kpos[k < KV_SPLIT ? k : KV_SPLIT - 1];
                ldv<E, VPL>(a.v, bg * a.v_sbg + pos * a.v_st + dv, vx[u]);
            }
#pragma unroll
            for (int u = 0; u < UV; ++u) {
                const int k = k0 + u * STEP;
                const bool ok = k < nk;
#pragma unroll
                for (int r = 0; r < RM; ++r) {
                    if (r >= R) break;
                    const float pr = ok ? p[r][k] : 0.f;
#pragma unroll
                    for (int e = 0; e < VPL; ++e) acc[r][e] += pr * vx[u][e];
                }
            }
        }
#pragma unroll
        for (int r = 0; r < RM; ++r) {
            if (r >= R) break;
#pragma unroll
            for (int e = 0; e < VPL; ++e) {
#pragma unroll
                for (int off = LPV; off < 64; off <<= 1) acc[r][e] += __shfl_xor(acc[r][e], off);
            }
            if (kv == 0)
#pragma unroll
                for (int e = 0; e < VPL; ++e) part[wv][r][dv + e] = acc[r][e];
        }
    }
    __syncthreads();
    for (int i = tid; i < R * D; i += KV_NT) {
        const int r = i / D, d = i % D;
        float s = 0.f;
#pragma unroll
        for (int w = 0; w < KV_NW; ++w) s += part[w][r][d];
        out[r * (D + 2) + 2 + d] = s;
    }
    if (tid < R) {
        out[tid * (D + 2)] = mxs[tid];
        out[tid * (D + 2) + 1] = sms[tid];
    }
}

// ---- append: the t new rows of k and v into the cache buffers, 16 bytes per thread
__global__ __launch_bounds__(KV_NT) void kv_append_kernel(KvAppendArgs a) {
    const int cpr = a.D * a.esz / 16;                     // 16-byte chunks per row
    const long rows = (long)a.B * a.G * a.t;
    const long idx = (long)blockIdx.x * KV_NT + threadIdx.x;
    if (idx >= 2 * rows * cpr) return;
    const int c = (int)(idx % cpr);
    long r = idx / cpr;
    const bool is_v = r >= rows;
    if (is_v) r -= rows;
    const int i = (int)(r % a.t);
    const long bg = r / a.t;
    const int g = (int)(bg % a.G), b = (int)(bg / a.G);
    const char* src = reinterpret_cast<const char*>(is_v ? a.v_new : a.k_new) +
                      ((long)b * (is_v ? a.v_sb : a.k_sb) + (long)g * (is_v ? a.v_sg : a.k_sg) +
                       (long)i * (is_v ? a.v_st : a.k_st)) * a.esz + c * 16;
    char* dst = reinterpret_cast<char*>(is_v ? a.v_buf : a.k_buf) + ((bg * a.cap + a.n0 + i) * a.D) * a.esz + c * 16;
    st16(dst, ld16(src));
}

int kv_append(const KvAppendArgs& a, hipStream_t stream) {
    const long total = 2L * a.B * a.G * a.t * (a.D * a.esz / 16);
    hipLaunchKernelGGL(kv_append_kernel, dim3((unsigned)((total + KV_NT - 1) / KV_NT)), dim3(KV_NT), 0, stream, a);
    return (int)hipGetLastError();
}

// ---- the splits of one (query, head) merged
template <int D>
__global__ __launch_bounds__(KV_NT) void kv_combine_kernel(KvArgs a) {
    __shared__ float fs[KV_MAXSPLIT];
    __shared__ float red[KV_NW];
    const int bt = blockIdx.x, h = blockIdx.y;
    const int R = a.R, H = a.G * R, NS = a.nsplit;
    const int g = h / R, r = h % R;
    const int tid = threadIdx.x, lane = lane_id(), wv = wave_id();
    const float* part = a.ws_part + ((long)bt * a.G + g) * NS * R * (D + 2) + r * (D + 2);
    const long sst = (long)R * (D + 2);                   // split stride
    auto block_reduce = [&](float v, bool is_max) {
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) {
            const float o = __shfl_xor(v, off);
            v = is_max ? fmaxf(v, o) : v + o;
        }
        if (lane == 0) red[wv] = v;
        __syncthreads();
        float t = red[0];
        for (int w = 1; w < KV_NW; ++w) t = is_max ? fmaxf(t, red[w]) : t + red[w];
        __syncthreads();
        return t;
    };
    float m = -INFINITY;
    for (int s = tid; s < NS; s += KV_NT) m = fmaxf(m, part[s * sst]);
    const float M = block_reduce(m, true);
    float l = 0.f;
    for (int s = tid; s < NS; s += KV_NT) {
        const float ms = part[s * sst];
        const float f = ms == -INFINITY ? 0.f : __expf(ms - M);
        fs[s] = f;
        l += f * part[s * sst + 1];
    }
    const float L = block_reduce(l, false);               // also orders the fs writes before their reads
    const float inv = 1.f / L;
    const long orow = ((long)bt * H + h) * D;
    for (int d = tid; d < D; d += KV_NT) {
        float o = 0.f;
        for (int s = 0; s < NS; ++s) o += fs[s] * part[s * sst + 2 + d];
        o *= inv;
        if (a.o_dtype == DT_BF16) reinterpret_cast<uint16_t*>(a.o)[orow + d] = f2bf(o);
        else reinterpret_cast<float*>(a.o)[orow + d] = o;
    }
}

namespace {

template <class E, int D>
int launch_kv(const KvArgs& a, int what, hipStream_t stream) {
    const dim3 blk(KV_NT);
    if (what == 0) {
        const int nnew = a.nb - a.sum_first;
        if (nnew <= 0) return 0;
        hipLaunchKernelGGL((kv_summary_kernel<E, D>), dim3((nnew + KV_NW - 1) / KV_NW, a.G, a.B), blk, 0, stream, a);
    } else if (what == 1) {
        const dim3 grid(a.B * a.T, a.G), sblk(KV_SNT);
        if (a.R <= 1) hipLaunchKernelGGL((kv_select_kernel<E, D, 1>), grid, sblk, 0, stream, a);
        else if (a.R <= 2) hipLaunchKernelGGL((kv_select_kernel<E, D, 2>), grid, sblk, 0, stream, a);
        else if (a.R <= 4) hipLaunchKernelGGL((kv_select_kernel<E, D, 4>), grid, sblk, 0, stream, a);
        else hipLaunchKernelGGL((kv_select_kernel<E, D, 8>), grid, sblk, 0, stream, a);
    } else {
        const dim3 grid(a.B * a.T, a.nsplit, a.G);
        if (a.R <= 1) hipLaunchKernelGGL((kv_split_kernel<E, D, 1>), grid, blk, 0, stream, a);
        else if (a.R <= 2) hipLaunchKernelGGL((kv_split_kernel<E, D, 2>), grid, blk, 0, stream, a);
        else if (a.R <= 4) hipLaunchKernelGGL((kv_split_kernel<E, D, 4>), grid, blk, 0, stream, a);
        else hipLaunchKernelGGL((kv_split_kernel<E, D, 8>), grid, blk, 0, stream, a);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return (int)e;
        hipLaunchKernelGGL((kv_combine_kernel<D>), dim3(a.B * a.T, a.G * a.R), blk, 0, stream, a);
    }
    return (int)hipGetLastError();
}

}  // namespace

long kv_max_keys(const KvArgs& a) {
    if (!a.retrieval) return a.n;
    // the window holds at most W + L - 1 keys; sinks, blocks and window are disjoint positions of the cache
    const long m = (long)a.sinks + (long)a.K * a.L + (long)a.window + a.L - 1;
    return m < a.n ? m : a.n;
}
// split length: at most KV_SPLIT keys, shorter (down to 64) until a launch has about 2048 workgroups, so that the
// last round of workgroups is not a small fraction of a full one
void kv_split_plan(const KvArgs& a, int* slen, int* nsplit) {
    const long mk = kv_max_keys(a) > 0 ? kv_max_keys(a) : 1;
    const long rows = (long)a.B * a.T * a.G;
    long want = (mk * rows + 1023) / 1024;                 // keys per split for 1024 workgroups
    want = (want + 63) / 64 * 64;
    const int sl = (int)(want < 64 ? 64 : want > KV_SPLIT ? KV_SPLIT : want);
    *slen = sl;
    *nsplit = (int)((mk + sl - 1) / sl);
}
int kv_max_k() { return KV_MAXK; }
int kv_max_blocks() { return KV_MAXNB; }
int kv_max_splits() { return KV_MAXSPLIT; }

int kv_dispatch(const KvArgs& a, int what, hipStream_t stream) {
    const bool bf = a.dtype == DT_BF16;
    switch (a.D) {
        case 64: return bf ? launch_kv<BF16, 64>(a, what, stream) : launch_kv<F32, 64>(a, what, stream);
        case 128: return bf ? launch_kv<BF16, 128>(a, what, stream) : launch_kv<F32, 128>(a, what, stream);
        case 256: return bf ? launch_kv<BF16, 256>(a, what, stream) : launch_kv<F32, 256>(a, what, stream);
        default: return BF_ERR_UNSUPPORTED;
    }
}

}  // namespace bf
