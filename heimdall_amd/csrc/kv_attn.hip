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

constexpr int KV_SPLIT = 512;       // attended keys per split
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

// ---- block summaries: wave w of the workgroup summarises block sum_first + blockIdx.x * 4 + w
template <class E, int D>
__global__ __launch_bounds__(KV_NT) void kv_summary_kernel(KvArgs a) {
    constexpr int DPL = D / 64;                           // dims per lane
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
    float* smin = a.kmin + (bg * a.nb_cap + j) * D + lane * DPL;
    float* smax = a.kmax + (bg * a.nb_cap + j) * D + lane * DPL;
#pragma unroll
    for (int e = 0; e < DPL; ++e) { smin[e] = mn[e]; smax[e] = mx[e]; }
}

// ---- selection: the K candidate blocks with the highest upper bound, per (query, g)
template <class E, int D>
__global__ __launch_bounds__(KV_NT) void kv_select_kernel(KvArgs a) {
    constexpr int DPL = D / 64;
    __shared__ float ub[KV_MAXNB];
    __shared__ float rv[KV_NW];
    __shared__ int ri[KV_NW];
    const int lane = lane_id(), wv = wave_id(), tid = threadIdx.x;
    const int bt = blockIdx.x, g = blockIdx.y;
    const int b = bt / a.T;
    const int R = a.R, H = a.G * R;
    const long bg = (long)b * a.G + g;
    const int nc = kv_query(a, bt % a.T).nc;

    float q[KV_MAXR][DPL];
#pragma unroll
    for (int r = 0; r < KV_MAXR; ++r) {
        if (r < R) ldv<E, DPL>(a.q, ((long)bt * H + g * R + r) * D + lane * DPL, q[r]);
        else
#pragma unroll
            for (int e = 0; e < DPL; ++e) q[r][e] = 0.f;
    }
    for (int j = wv; j < nc; j += KV_NW) {
        float lo[DPL], hi[DPL];
        ldf<DPL>(a.kmin + (bg * a.nb_cap + j) * D + lane * DPL, lo);
        ldf<DPL>(a.kmax + (bg * a.nb_cap + j) * D + lane * DPL, hi);
        float best = -INFINITY;
#pragma unroll
        for (int r = 0; r < KV_MAXR; ++r) {
            if (r >= R) break;
            float s = 0.f;
#pragma unroll
            for (int e = 0; e < DPL; ++e) s += fmaxf(q[r][e] * lo[e], q[r][e] * hi[e]);
#pragma unroll
            for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off);
            best = fmaxf(best, s);
        }
        if (lane == 0) ub[j] = best;
    }
    __syncthreads();
    int* sel = a.sel + ((long)bt * a.G + g) * a.K;
    for (int it = 0; it < a.K; ++it) {
        float bv = -INFINITY;
        int bi = 0x7fffffff;
        for (int j = tid; j < nc; j += KV_NT) {
            const float v = ub[j];
            if (v > bv || (v == bv && j < bi)) { bv = v; bi = j; }
        }
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) {
            const float ov = __shfl_xor(bv, off);
            const int oi = __shfl_xor(bi, off);
            if (ov > bv || (ov == bv && oi < bi)) { bv = ov; bi = oi; }
        }
        if (lane == 0) { rv[wv] = bv; ri[wv] = bi; }
        __syncthreads();
        if (tid == 0) {
            float v0 = rv[0];
            int i0 = ri[0];
            for (int w = 1; w < KV_NW; ++w)
                if (rv[w] > v0 || (rv[w] == v0 && ri[w] < i0)) { v0 = rv[w]; i0 = ri[w]; }
            const bool ok = i0 < nc && v0 > -INFINITY;
            sel[it] = ok ? i0 : -1;
            if (ok) ub[i0] = -INFINITY;
        }
        __syncthreads();
    }
}

// ---- one split of one query's attended keys
template <class E, int D>
__global__ __launch_bounds__(KV_NT) void kv_split_kernel(KvArgs a) {
    constexpr int LPK = 16, KPW = 64 / LPK;               // score pass: lanes per key, keys per wave step
    constexpr int DPL = D / LPK;                          // dims per lane in the dot product
    constexpr int VW = 16 / (int)sizeof(typename E::T);  // value pass: dims per lane (one 16-byte read)
    constexpr int LPV = D / VW < 64 ? D / VW : 64;        // lanes per value row
    constexpr int KPV = 64 / LPV;                         // value rows per wave step
    constexpr int VPL = D / LPV;                          // dims per lane in the value pass
    __shared__ float p[KV_MAXR][KV_SPLIT];                // scores, then probabilities
    __shared__ int blk[KV_MAXK];
    __shared__ float part[KV_NW][KV_MAXR][D];
    __shared__ float mxs[KV_MAXR], sms[KV_MAXR];
    __shared__ int nsel_s;
    const int lane = lane_id(), wv = wave_id(), tid = threadIdx.x;
    const int bt = blockIdx.x, x = blockIdx.y, g = blockIdx.z;
    const int b = bt / a.T;
    const int R = a.R, H = a.G * R;
    const long bg = (long)b * a.G + g;
    const KvQuery qi = kv_query(a, bt % a.T);

    // selected blocks of (query, g), ascending, and their count
    int nsel = 0;
    if (a.retrieval && a.K > 0) {
        if (tid == 0) {
            const int* sel = a.sel + ((long)bt * a.G + g) * a.K;
            int m = 0;
            for (int i = 0; i < a.K; ++i) {
                const int s = sel[i];
                if (s >= 0 && s < qi.nc) blk[m++] = s;
            }
            for (int i = 1; i < m; ++i)                   // insertion sort (K <= 64)
                for (int jj = i; jj > 0 && blk[jj - 1] > blk[jj]; --jj) {
                    const int t = blk[jj]; blk[jj] = blk[jj - 1]; blk[jj - 1] = t;
                }
            nsel_s = m;
        }
        __syncthreads();
        nsel = nsel_s;
    }
    const long nv = qi.ns + (long)nsel * a.L + max(0L, qi.end - qi.win0);
    const long v0 = (long)x * KV_SPLIT;
    const int nk = (int)max(0L, min((long)KV_SPLIT, nv - v0));
    float* out = a.ws_part + (((long)bt * a.G + g) * a.nsplit + x) * R * (D + 2);
    if (nk == 0) {                                        // empty split: weight zero in the combine
        for (int i = tid; i < R * (D + 2); i += KV_NT) {
            const int c = i % (D + 2);
            out[i] = c == 0 ? -INFINITY : 0.f;
        }
        return;
    }

    // scores: 16 lanes per key, dims (lane % 16) * DPL .. + DPL - 1
    {
        const int kl = lane / LPK, dl = (lane % LPK) * DPL;
        float q[KV_MAXR][DPL];
#pragma unroll
        for (int r = 0; r < KV_MAXR; ++r) {
            if (r < R) {
                ldv<E, DPL>(a.q, ((long)bt * H + g * R + r) * D + dl, q[r]);
#pragma unroll
                for (int e = 0; e < DPL; ++e) q[r][e] *= a.scale;
            } else {
#pragma unroll
                for (int e = 0; e < DPL; ++e) q[r][e] = 0.f;
            }
        }
        for (int k0 = wv * KPW; k0 < nk; k0 += KV_NW * KPW) {
            const int k = k0 + kl;
            const long pos = kv_key_pos(a, qi, blk, nsel, v0 + (k < nk ? k : nk - 1));
            float kx[DPL];
            ldv<E, DPL>(a.k, bg * a.k_sbg + pos * a.k_st + dl, kx);
#pragma unroll
            for (int r = 0; r < KV_MAXR; ++r) {
                if (r >= R) break;
                float s = 0.f;
#pragma unroll
                for (int e = 0; e < DPL; ++e) s += q[r][e] * kx[e];
#pragma unroll
                for (int off = LPK / 2; off > 0; off >>= 1) s += __shfl_xor(s, off);
                if ((lane % LPK) == 0 && k < nk) p[r][k] = s;
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
        float acc[KV_MAXR][VPL];
#pragma unroll
        for (int r = 0; r < KV_MAXR; ++r)
#pragma unroll
            for (int e = 0; e < VPL; ++e) acc[r][e] = 0.f;
        for (int k0 = wv * KPV; k0 < nk; k0 += KV_NW * KPV) {
            const int k = k0 + kv;
            const bool ok = k < nk;
            const long pos = kv_key_pos(a, qi, blk, nsel, v0 + (ok ? k : nk - 1));
            float vx[VPL];
            ldv<E, VPL>(a.v, bg * a.v_sbg + pos * a.v_st + dv, vx);
#pragma unroll
            for (int r = 0; r < KV_MAXR; ++r) {
                if (r >= R) break;
                const float pr = ok ? p[r][k] : 0.f;
#pragma unroll
                for (int e = 0; e < VPL; ++e) acc[r][e] += pr * vx[e];
            }
        }
#pragma unroll
        for (int r = 0; r < KV_MAXR; ++r) {
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
        hipLaunchKernelGGL((kv_select_kernel<E, D>), dim3(a.B * a.T, a.G), blk, 0, stream, a);
    } else {
        hipLaunchKernelGGL((kv_split_kernel<E, D>), dim3(a.B * a.T, a.nsplit, a.G), blk, 0, stream, a);
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
int kv_nsplit(long max_keys) { return (int)((max_keys + KV_SPLIT - 1) / KV_SPLIT); }
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
