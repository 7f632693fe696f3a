// K2: exact sliding-window + sink attention over a prefill chunk, with per-row log-sum-exp and the fused gamma mix.
//
// Reference: HybridAttention._window_fp32 (Heimdall/heimdall/hibrit.py:341-361) and the mix of :409-411.
// Query i of the chunk sits at absolute position p = start + i. Visible keys (mask of hibrit.py:356):
//   sinks j < n_sinks with j <= p, and window keys at positions kp with S <= kp <= p, p - kp < W, where
//   kp < start comes from the ring (slot kp mod W, valid iff ring_pos[slot] == kp) and kp >= start from the chunk.
// s = (q . k) / sqrt(D); lse = ln sum_visible e^s; o_win = softmax(s) V.
// Mix (when enabled): gamma = sigmoid(z + mix_lse (lse - ln W)) [p >= W]; o = o_win + gamma (mem_scale o_mem - o_win).
//
// One workgroup = 64 queries of one query head (4 waves x 16). Per key block (64 positions for bf16 operands, 32
// for fp32) the block's K rows (row-major) and V rows (transposed) are staged in LDS; the next block is prefetched
// into registers while the current one is consumed. Scores are computed transposed (S^T = K Q^T) so each lane's
// softmax statistics belong to its own query column, and P feeds the P.V MFMA straight from registers.
#include "bf_common.h"
#include "bf_internal.h"

namespace bf {

constexpr int NT_WIN = 256;
constexpr int NQT = 1;           // 16-query tiles per wave
constexpr int QW = 16 * NQT;     // queries per wave
constexpr int BQ = 4 * QW;       // queries per workgroup

template <class E>
struct WinKB {
    static constexpr int value = sizeof(typename E::T) == 2 ? 64 : 32;
};

template <class E, int D>
struct WinShared {
    static constexpr int KB = WinKB<E>::value;
    typename E::T ks[KB][D + E::VEC];        // key rows of the block
    typename E::T vt[D][KB + E::VEC];        // value rows of the block, transposed [d][key]
    int valid[KB];                           // key row holds a real key (else its scores are masked)
    int krel[KB];                            // key position minus the workgroup's first query position
};

template <class E, int D>
struct WinPrefetch {
    static constexpr int KB = WinKB<E>::value;
    static constexpr int CPR = D * (int)sizeof(typename E::T) / 16;    // 16-byte chunks per row
    static constexpr int KCH = KB * CPR / NT_WIN;                      // K chunks per thread
    static constexpr int VBT = KB / E::VEC, VBD = D / E::VEC;          // V transpose blocks
    static constexpr int VPT = (VBT * VBD + NT_WIN - 1) / NT_WIN;      // V blocks per thread
    uint4 k[KCH];
    uint4 v[VPT][E::VEC];
    uint2 rp;          // ring_pos of row (thread % KB) for ring blocks, read with the rows
};

// The keys of a workgroup are split into segments that each come from one contiguous source: the sinks, the ring
// up to its wrap point, the ring after it, and the chunk. A key block never straddles two segments, so the address
// of every row is base + min(row, last) * stride with no per-row branching.
template <class T>
struct KeySeg {
    const T* kb;       // first key row of the segment
    const T* vb;       // first value row
    long ks, vs;       // row strides (elements)
    long pos0;         // position of the first row (sinks: 0)
    int count;         // rows
    int slot0;         // ring slot of the first row, or -1 outside the ring
    int sink;          // sink rows: visible to every query at or after their position, no window limit
};

// Load the rows of one key block into registers. Rows past the segment's end re-read its last row; their scores are
// masked to -inf so they add nothing (exec-masked loads would make the compiler wait for the whole prefetch early).
template <class E, int D>
__device__ __forceinline__ void win_fetch(WinPrefetch<E, D>& f, const KeySeg<typename E::T>& br, rsrc_t rpos) {
    using P = WinPrefetch<E, D>;
    constexpr int VEC = E::VEC;
    const int tid = threadIdx.x;
    const int last = min(br.count, P::KB) - 1;
    // out-of-range offset (outside the ring) reads 0
    f.rp = buf_ld8(rpos, br.slot0 >= 0 ? (uint32_t)(br.slot0 + min(tid % P::KB, last)) * 8u : 0xFFFFFFF0u);
#pragma unroll
    for (int j = 0; j < P::KCH; ++j) {
        const int c = tid + NT_WIN * j, row = c / P::CPR, col = (c % P::CPR) * VEC;
        f.k[j] = ld16(br.kb + min(row, last) * br.ks + col);
    }
#pragma unroll
    for (int j = 0; j < P::VPT; ++j) {
        const int blk = tid + NT_WIN * j;
        const int bt = blk % P::VBT, bd = (blk / P::VBT) % P::VBD;
#pragma unroll
        for (int i = 0; i < VEC; ++i) f.v[j][i] = ld16(br.vb + min(bt * VEC + i, last) * br.vs + bd * VEC);
    }
}

template <class E, int D>
__device__ __forceinline__ void win_park(WinShared<E, D>& sm, WinPrefetch<E, D>& f, const WinArgs& a,
                                         const KeySeg<typename E::T>& br, long p_first) {
    using P = WinPrefetch<E, D>;
    constexpr int VEC = E::VEC, KB = P::KB;
    const int tid = threadIdx.x;
#pragma unroll
    for (int j = 0; j < P::KCH; ++j) {
        const int c = tid + NT_WIN * j, row = c / P::CPR, col = (c % P::CPR) * VEC;
        st16(&sm.ks[row][col], f.k[j]);
    }
#pragma unroll
    for (int j = 0; j < P::VPT; ++j) {
        const int blk = tid + NT_WIN * j;
        if (blk < P::VBT * P::VBD) {
            const int bt = blk % P::VBT, bd = blk / P::VBT;
            transpose_block<E>(f.v[j]);
#pragma unroll
            for (int i = 0; i < VEC; ++i) st16(&sm.vt[bd * VEC + i][bt * VEC], f.v[j][i]);
        }
    }
    if (tid < KB) {
        const long kp = br.pos0 + tid;
        bool val = tid < br.count;
        if (br.slot0 >= 0) val = val && (long)(((uint64_t)f.rp.y << 32) | f.rp.x) == kp;
        sm.valid[tid] = val;
        const long rel = kp - p_first;                      // sinks far behind the chunk clamp (always visible)
        sm.krel[tid] = (int)max(rel, -(1L << 30));
    }
}

template <class E, int D, bool BO>
__global__ __launch_bounds__(NT_WIN) void window_kernel(WinArgs a) {
    using T = typename E::T;
    using P = WinPrefetch<E, D>;
    constexpr int VEC = E::VEC, KF = E::KF, KB = P::KB;
    constexpr int NKD = D / KF;           // fragments along D
    constexpr int NKT = KB / 16;          // key tiles per block
    constexpr int NDT = D / 16;           // d tiles of the output
    constexpr int PF = KB / KF;           // P fragments per query tile per block
    __shared__ WinShared<E, D> sm;

    const int qb = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
    const int R = a.R, G = a.G, H = G * R, g = h / R;
    const int lane = lane_id(), wv = wave_id(), l16 = lane & 15, lg = lane >> 4;
    const long qi0 = (long)qb * BQ;                       // first query index of the workgroup
    const int nq = (int)min((long)BQ, (long)a.T - qi0);
    const long p_first = a.start + qi0, p_last = a.start + qi0 + nq - 1;
    const float scale = rsqrtf((float)D);

    const T* Qb = reinterpret_cast<const T*>(a.q) + b * a.q_sb + h * a.q_sh;
    const T* rk = a.ring_k ? reinterpret_cast<const T*>(a.ring_k) + ((long)b * G + g) * a.W * D : nullptr;
    const T* rv = a.ring_v ? reinterpret_cast<const T*>(a.ring_v) + ((long)b * G + g) * a.W * D : nullptr;
    const T* ck = reinterpret_cast<const T*>(a.k) + b * a.k_sb + g * a.k_sh;
    const T* cv = reinterpret_cast<const T*>(a.v) + b * a.v_sb + g * a.v_sh;
    const T* sk = a.n_sinks ? reinterpret_cast<const T*>(a.sink_k) + ((long)b * G + g) * a.n_sinks * D : nullptr;
    const T* sv = a.n_sinks ? reinterpret_cast<const T*>(a.sink_v) + ((long)b * G + g) * a.n_sinks * D : nullptr;

    // Q fragments (B operand of S^T = K Q^T): query tile qt, column l16, k range VEC*lg of each KF step
    uint4 fq[NQT][NKD];
#pragma unroll
    for (int qt = 0; qt < NQT; ++qt) {
        const int qi = QW * wv + 16 * qt + l16;
        const T* qrow = Qb + (qi0 + qi) * a.q_st;
#pragma unroll
        for (int kf = 0; kf < NKD; ++kf) fq[qt][kf] = qi < nq ? ld16(qrow + kf * KF + VEC * lg) : zero16();
    }
    int qrel[NQT];                                        // query position minus p_first
    f32x4 o[NDT][NQT];
    float m[NQT], l[NQT];
#pragma unroll
    for (int qt = 0; qt < NQT; ++qt) {
        qrel[qt] = QW * wv + 16 * qt + l16;
        m[qt] = -INFINITY;
        l[qt] = 0.f;
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt) o[dt][qt] = f32x4{0.f, 0.f, 0.f, 0.f};
    }

    // key segments (sinks, ring before its wrap point, ring after it, chunk), consumed in blocks of KB rows
    using Seg = KeySeg<T>;
    const long kp_lo = max((long)a.sinks, p_first - a.W + 1);
    Seg sg[4];
    int nb[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        sg[j] = Seg{ck, cv, 0, 0, 0, 0, -1, 0};
        nb[j] = 0;
    }
    if (a.n_sinks) sg[0] = Seg{sk, sv, D, D, 0, a.n_sinks, -1, 1};
    const long rhi = min(p_last, a.start - 1);
    if (rk && kp_lo <= rhi) {
        const int sa = (int)(kp_lo % a.W);                  // one division per workgroup
        const long n = rhi - kp_lo + 1;
        const long n1 = min(n, (long)(a.W - sa));
        sg[1] = Seg{rk + (long)sa * D, rv + (long)sa * D, D, D, kp_lo, (int)n1, sa, 0};
        if (n > n1) sg[2] = Seg{rk, rv, D, D, kp_lo + n1, (int)(n - n1), 0, 0};
    }
    const long clo = max(kp_lo, a.start);
    if (clo <= p_last)
        sg[3] = Seg{ck + (clo - a.start) * a.k_st, cv + (clo - a.start) * a.v_st, a.k_st, a.v_st, clo,
                    (int)(p_last - clo + 1), -1, 0};
    int nblk = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        nb[j] = (sg[j].count + KB - 1) / KB;
        nblk += nb[j];
    }
    // block i as a segment of its own: the KB rows starting at row KB * (i - first block of its segment)
    auto block_ref = [&](int i) {
        Seg r = sg[3];
        int base = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            if (i >= base && i < base + nb[j]) {
                const int off = (i - base) * KB;
                r = sg[j];
                r.kb += off * sg[j].ks;
                r.vb += off * sg[j].vs;
                r.pos0 += off;
                r.count -= off;
                if (r.slot0 >= 0) r.slot0 += off;
            }
            base += nb[j];
        }
        return r;
    };

    const rsrc_t rpos = make_rsrc(a.ring_pos, a.ring_pos ? (uint32_t)a.W * 8u : 0u);
    P pf;
    Seg br;
    if (nblk > 0) {
        br = block_ref(0);
        win_fetch<E, D>(pf, br, rpos);
    }
    for (int i = 0; i < nblk; ++i) {
        const bool sb = br.sink;
        __syncthreads();                                   // previous block fully consumed
        win_park<E, D>(sm, pf, a, br, p_first);
        __syncthreads();
        if (i + 1 < nblk) {                                // uniform: the next block's loads fly during this one
            br = block_ref(i + 1);
            win_fetch<E, D>(pf, br, rpos);
        }
        // S^T = K Q^T for this block
        f32x4 s[NKT][NQT];
#pragma unroll
        for (int kt = 0; kt < NKT; ++kt)
#pragma unroll
            for (int qt = 0; qt < NQT; ++qt) s[kt][qt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kf = 0; kf < NKD; ++kf)
#pragma unroll
            for (int kt = 0; kt < NKT; ++kt) {
                const uint4 ak = ld16(&sm.ks[16 * kt + l16][kf * KF + VEC * lg]);
#pragma unroll
                for (int qt = 0; qt < NQT; ++qt) mma<E>(s[kt][qt], ak, fq[qt][kf]);
            }
        // mask, online softmax per query column
#pragma unroll
        for (int qt = 0; qt < NQT; ++qt) {
            const int qp = qrel[qt];
            float bm = -INFINITY;
#pragma unroll
            for (int kt = 0; kt < NKT; ++kt)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int kr = 16 * kt + 4 * lg + e;
                    const int kp = sm.krel[kr];
                    const bool vis = sm.valid[kr] && kp <= qp && (sb || qp - kp < a.W);
                    const float x = vis ? s[kt][qt][e] * scale : -INFINITY;
                    s[kt][qt][e] = x;
                    bm = fmaxf(bm, x);
                }
            bm = fmaxf(bm, __shfl_xor(bm, 16));
            bm = fmaxf(bm, __shfl_xor(bm, 32));
            const float mn = fmaxf(m[qt], bm);
            const float corr = mn == -INFINITY ? 1.f : __expf(m[qt] - mn);
            float ls = 0.f;
#pragma unroll
            for (int kt = 0; kt < NKT; ++kt)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float p = mn == -INFINITY ? 0.f : __expf(s[kt][qt][e] - mn);
                    s[kt][qt][e] = p;
                    ls += p;
                }
            ls += __shfl_xor(ls, 16);
            ls += __shfl_xor(ls, 32);
            l[qt] = l[qt] * corr + ls;
            m[qt] = mn;
#pragma unroll
            for (int dt = 0; dt < NDT; ++dt) {
                o[dt][qt][0] *= corr; o[dt][qt][1] *= corr; o[dt][qt][2] *= corr; o[dt][qt][3] *= corr;
            }
        }
        // O^T += V^T P^T. P fragment f of query tile qt: keys {KF*f + 4*lg + e} of key tiles covered by the fragment
#pragma unroll
        for (int f = 0; f < PF; ++f) {
            uint4 pb[NQT];
#pragma unroll
            for (int qt = 0; qt < NQT; ++qt) {
                if constexpr (sizeof(T) == 2) {
                    const f32x4 x0 = s[2 * f][qt], x1 = s[2 * f + 1][qt];
                    pb[qt].x = (uint32_t)f2bf(x0[0]) | ((uint32_t)f2bf(x0[1]) << 16);
                    pb[qt].y = (uint32_t)f2bf(x0[2]) | ((uint32_t)f2bf(x0[3]) << 16);
                    pb[qt].z = (uint32_t)f2bf(x1[0]) | ((uint32_t)f2bf(x1[1]) << 16);
                    pb[qt].w = (uint32_t)f2bf(x1[2]) | ((uint32_t)f2bf(x1[3]) << 16);
                } else {
                    const f32x4 x0 = s[f][qt];
                    pb[qt] = make_uint4(__float_as_uint(x0[0]), __float_as_uint(x0[1]), __float_as_uint(x0[2]),
                                        __float_as_uint(x0[3]));
                }
            }
#pragma unroll
            for (int dt = 0; dt < NDT; ++dt) {
                uint4 av;
                if constexpr (sizeof(T) == 2) {
                    const uint2 lo = *reinterpret_cast<const uint2*>(&sm.vt[16 * dt + l16][KF * f + 4 * lg]);
                    const uint2 hi = *reinterpret_cast<const uint2*>(&sm.vt[16 * dt + l16][KF * f + 16 + 4 * lg]);
                    av = make_uint4(lo.x, lo.y, hi.x, hi.y);
                } else {
                    av = ld16(&sm.vt[16 * dt + l16][KF * f + 4 * lg]);
                }
#pragma unroll
                for (int qt = 0; qt < NQT; ++qt) mma<E>(o[dt][qt], av, pb[qt]);
            }
        }
    }

    // epilogue: normalise, lse, gamma mix, store o [B][T][H][D]
    const float lnW = logf((float)a.W);
#pragma unroll
    for (int qt = 0; qt < NQT; ++qt) {
        const int qi = QW * wv + 16 * qt + l16;
        if (qi >= nq) continue;
        const long tq = qi0 + qi;
        const float inv = 1.f / l[qt];
        const float lse = m[qt] + logf(l[qt]);
        if (a.lse && lg == 0) a.lse[((long)b * H + h) * a.T + tq] = lse;
        float gam = 0.f;
        if (a.mix_on && p_first + qrel[qt] >= a.W)
            gam = 1.f / (1.f + __expf(-(a.z[((long)b * a.T + tq) * H + h] + a.mix_lse[h] * (lse - lnW))));
        const float ms = a.mix_on ? a.mem_scale[h] : 0.f;
        const long orow = (((long)b * a.T + tq) * H + h) * D;
        // memory reads issued together (every row of o_mem exists); rows with gam = 0 keep the window output by
        // selection, so rows the delta rule never wrote cannot leak in
        const bool on = gam != 0.f;
        float4 om[NDT];
        if (a.mix_on) load_om<NDT>(a, orow + 4 * lg, om);
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt) {
            const int d0 = 16 * dt + 4 * lg;
            float r4[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) r4[e] = o[dt][qt][e] * inv;
            if (a.mix_on) {
                const float mv[4] = {om[dt].x, om[dt].y, om[dt].z, om[dt].w};
#pragma unroll
                for (int e = 0; e < 4; ++e) r4[e] = on ? r4[e] + gam * (ms * mv[e] - r4[e]) : r4[e];
            }
            if constexpr (BO) store4<BF16>(reinterpret_cast<uint16_t*>(a.o) + orow + d0, r4[0], r4[1], r4[2], r4[3]);
            else store4<F32>(reinterpret_cast<float*>(a.o) + orow + d0, r4[0], r4[1], r4[2], r4[3]);
        }
    }
}

template <class E, int D>
static int launch_window(const WinArgs& a, hipStream_t stream) {
    const dim3 grid((a.T + BQ - 1) / BQ, a.G * a.R, a.B);
    if (a.o_dtype == DT_BF16) hipLaunchKernelGGL((window_kernel<E, D, true>), grid, dim3(NT_WIN), 0, stream, a);
    else hipLaunchKernelGGL((window_kernel<E, D, false>), grid, dim3(NT_WIN), 0, stream, a);
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? 0 : (int)e;
}

int window_dispatch(const WinArgs& a, hipStream_t stream) {
    if (a.in_dtype == DT_BF16) return window_fa_dispatch(a, stream);
    switch (a.D) {
        case 64: return launch_window<F32, 64>(a, stream);
        case 128: return launch_window<F32, 128>(a, stream);
        case 256: return launch_window<F32, 256>(a, stream);
        default: return BF_ERR_UNSUPPORTED;
    }
}

}  // namespace bf
