// K2, bf16 operands: exact sliding-window + sink attention over a prefill chunk with per-row log-sum-exp and the
// fused gamma mix (reference: HybridAttention._window_fp32, Heimdall/heimdall/hibrit.py:341-361, mix :409-411).
//
// Semantics are those of window.hip (which serves fp32 operands): query i of the chunk sits at position
// p = start + i and sees the sinks j < n_sinks with j <= p and the keys kp with S <= kp <= p, p - kp < W (the ring
// for kp < start, slot kp mod W valid iff ring_pos[slot] == kp; the chunk for kp >= start).
//
// Work split. One workgroup = 128 consecutive queries of one query head. D <= 128: 4 waves x 32 queries, held as two
// 16-query MFMA tiles, so every K / V fragment a wave reads from LDS feeds two v_mfma_f32_16x16x32_bf16. D = 256:
// 8 waves x 16 queries, so that two waves fit each SIMD's registers.
//   S^T = K Q^T      A = K rows (LDS),             B = Q (registers, loaded once)
//   O^T += V^T P^T   A = V^T via ds_read_b64_tr_b16 of the row-major V tile,  B = P straight from the S registers
// Scores are transposed so that a query's softmax statistics live in its own lane column (max: two lane swaps per
// block; sum: per-lane partials reduced once at the end). The scale D^-1/2 log2(e) is applied inside the exponent
// (one FMA per score). The running max is raised only when a block's max exceeds it by more than 8 (log2 units), so
// O is rescaled rarely and P stays <= 2^8.
//
// Keys come in blocks of 64 rows from one contiguous source (sinks, ring before / after its wrap point, chunk). A
// block's K and V tiles are copied global -> LDS with buffer_load ... lds (no registers; one buffer descriptor per
// source, lanes of other sources masked off), double-buffered: block i+1 is in flight while block i is computed.
// When block i+1 is all chunk rows, a wave issues its copies one per step of its S product (a base offset and a
// scalar step per copy), so no wave stalls on a burst of copies before its first MFMA.
// Buffer rather than global loads: the compiler counts a global load into LDS as a flat access that may touch LDS
// and then drains every LDS wait to zero while one is in flight, which serialised the fragment reads. Per wave, blocks no query of the wave can see are skipped and blocks every
// query sees skip the mask. Workgroups are mapped XCD-aware (WinMap): consecutive workgroups of one XCD take the R
// query heads of one query block, then an earlier query block of the same KV head, so one L2 serves their K / V
// re-reads; when query blocks differ in length (causal attention, a prefill's first W positions) pairs of XCDs
// share the blocks of a KV head alternately, so both get long and short ones.
#include "bf_common.h"
#include "bf_internal.h"

namespace bf {

namespace {

constexpr int FA_BQ = 128;                  // queries per workgroup
constexpr int FA_KB = 64;                   // keys per block
constexpr int FA_NXCD = 8;
constexpr float FA_LOG2E = 1.4426950408889634f;
constexpr float FA_LN2 = 0.6931471805599453f;
constexpr float FA_SLACK = 8.f;             // lazy max: rescale only when a block max exceeds the running max by this

// Waves per workgroup and 16-query MFMA tiles per wave: D <= 128 holds 32 queries per wave (two tiles share each
// K / V fragment read), D = 256 holds 16 queries in each of 8 waves so that two waves fit one SIMD's registers.
template <int D>
struct FaShape {
    static constexpr int QT = D <= 128 ? 2 : 1;
    static constexpr int NW = FA_BQ / (16 * QT);
    static constexpr int NT = 64 * NW;
};

template <int D>
struct __align__(16) FaTile {
    uint16_t k[FA_KB * D];     // key rows, 16-byte blocks permuted by fa_swk(row)
    uint16_t v[FA_KB * D];     // value rows, 16-byte blocks permuted by fa_swv(row)
};

// LDS block permutations (NBLK = 16-byte blocks per row). K: the 16 rows of an A fragment read (one block each) hit
// 16 distinct 16-byte bank groups. V: the 8 consecutive rows x 32 bytes of a 32-lane transposing read do too.
template <int NBLK>
__device__ __forceinline__ int fa_swk(int row) { return NBLK >= 16 ? (row & 15) : ((row >> 1) & 7); }
template <int NBLK>
__device__ __forceinline__ int fa_swv(int row) { return NBLK >= 16 ? 2 * (row & 7) : 2 * ((row >> 1) & 3); }

typedef short fa_v4s __attribute__((ext_vector_type(4)));
// ds_read_b64_tr_b16: in each 16-lane group, lane 4q + r receives element r of the 8-byte chunks that lanes 4e + q
// (e = 0..3) address, in order of e.
__device__ __forceinline__ uint2 fa_tr16(const char* p) {
    const fa_v4s v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) fa_v4s*)(p));
    return make_uint2((uint16_t)v[0] | ((uint32_t)(uint16_t)v[1] << 16), (uint16_t)v[2] | ((uint32_t)(uint16_t)v[3] << 16));
}


// max / sum of a value over lanes l, l ^ 16, l ^ 32, l ^ 48 by lane swaps (v_permlane16_swap, v_permlane32_swap)
__device__ __forceinline__ float fa_max4(float v) {
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ __forceinline__ float fa_sum4(float v) {
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = __uint_as_float(a[0]) + __uint_as_float(a[1]);
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// Streaming (non-temporal) accesses of the epilogue: the memory rows are read once and the output rows written once,
// so they should not displace the K / V tiles other workgroups re-read from L2 (the sliding window over 32768
// queries ran 1909-1927 us against 1938-1963 us with ordinary accesses).
typedef unsigned int fa_u2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint2 fa_ld8_nt(const void* p) {
    const fa_u2 v = __builtin_nontemporal_load(reinterpret_cast<const fa_u2*>(p));
    return make_uint2(v[0], v[1]);
}
template <bool BO>
__device__ __forceinline__ void fa_st4_nt(void* o, long i, const float (&r)[4]) {
    if constexpr (BO) {
        const fa_u2 v = {(uint32_t)f2bf(r[0]) | ((uint32_t)f2bf(r[1]) << 16),
                         (uint32_t)f2bf(r[2]) | ((uint32_t)f2bf(r[3]) << 16)};
        __builtin_nontemporal_store(v, reinterpret_cast<fa_u2*>(reinterpret_cast<uint16_t*>(o) + i));
    } else {
        nt_stf4(reinterpret_cast<float*>(o) + i, make_float4(r[0], r[1], r[2], r[3]));
    }
}

}  // namespace

template <int D, bool BO, bool SPLIT>
__global__ __launch_bounds__(FaShape<D>::NT, 1) void window_fa_kernel(WinArgs a) {
    constexpr int QT = FaShape<D>::QT, NW = FaShape<D>::NW, QW = 16 * QT;
    constexpr int ROWB = D * 2, NBLK = ROWB / 16;
    constexpr int NKD = D / 32;                 // K fragments along D (S product)
    constexpr int NDT = D / 16;                 // output d tiles (PV product)
    constexpr int NKB = NKD < 4 ? NKD : 4;      // distinct per-lane K fragment bases
    constexpr int NVB = NDT < 8 ? NDT : 8;      // distinct per-lane V fragment bases
    constexpr int NLD = FA_KB * ROWB / 1024 / NW;   // global -> LDS copies per wave per tile (64 x 16 bytes each)
    static_assert(NLD * NW * 1024 == FA_KB * ROWB, "tile copy split");
    __shared__ FaTile<D> t0;
    __shared__ FaTile<D> t1;

    // ---- work item (the map of WinMap: workgroup x is dispatch slot x / 8 of XCD x mod 8). SPLIT: the last split_x
    // slots of each XCD run as split_p workgroups each, one per part of the item's key blocks (two halves, or more
    // parts for a grid of a few items), and write partial rows that window_merge_kernel combines.
    const int R = a.R, G = a.G, H = G * R;
    const int nqb = (a.T + FA_BQ - 1) / FA_BQ;
    const long per = a.map.per;
    const int xcd = (int)(blockIdx.x % FA_NXCD), sx = SPLIT ? a.split_x : 0;
    long idx = blockIdx.x / FA_NXCD;
    const int P = SPLIT ? a.split_p : 1;
    int half = -1;                                      // -1: the whole item, else its key part 0 .. P - 1
    if (SPLIT && idx >= per - sx) {
        const long k = idx - (per - sx);
        idx = per - sx + k / P;
        half = (int)(k % P);
    }
    const long wi = window_item(a.map, xcd, idx);
    if (wi < 0) return;
    const int r = (int)(wi % R);
    long rest = wi / R;
    const int qb = nqb - 1 - (int)(rest % nqb);        // later query blocks (the most keys) are dispatched first
    rest /= nqb;
    const int g = (int)(rest % G), b = (int)(rest / G);
    const int h = g * R + r;

    const int lane = lane_id(), wv = wave_id(), l16 = lane & 15, lg = lane >> 4;
    const long qi0 = (long)qb * FA_BQ;
    const int nq = (int)min((long)FA_BQ, (long)a.T - qi0);
    const long p_first = a.start + qi0, p_last = p_first + nq - 1;
    const int nqw = max(0, min(QW, nq - QW * wv));                // queries of this wave
    const long qw0 = p_first + QW * wv, qw1 = qw0 + nqw - 1;

    // ---- Q fragments (B operand of S^T = K Q^T): query tile qt, column l16, d range 32 kf + 8 lg. Each query row is
    // read by this workgroup only: streaming loads leave L2 to the K / V tiles (1.5 % on the sliding window).
    const uint16_t* Qb = reinterpret_cast<const uint16_t*>(a.q) + b * a.q_sb + h * a.q_sh;
    uint4 fq[QT][NKD];
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
        const int qi = QW * wv + 16 * qt + l16;
        const uint16_t* qrow = Qb + (qi0 + qi) * a.q_st;
#pragma unroll
        for (int kf = 0; kf < NKD; ++kf) fq[qt][kf] = qi < nq ? nt_ld16(qrow + 32 * kf + 8 * lg) : zero16();
    }

    // ---- key blocks: [the sink block] then 64 consecutive positions each from kp_lo (window start of the first
    // query) to p_last. A window key at kp < start is ring slot kp mod W (valid iff ring_pos[slot] == kp), at
    // kp >= start chunk row kp - start. Rows outside [kp_lo, p_last] (or past the sinks) are masked.
    const uint16_t* ck = reinterpret_cast<const uint16_t*>(a.k) + b * a.k_sb + g * a.k_sh;
    const uint16_t* cv = reinterpret_cast<const uint16_t*>(a.v) + b * a.v_sb + g * a.v_sh;
    const long gbase = ((long)b * G + g);
    const uint16_t* rk = a.ring_k ? reinterpret_cast<const uint16_t*>(a.ring_k) + gbase * a.W * D : nullptr;
    const uint16_t* rv = a.ring_v ? reinterpret_cast<const uint16_t*>(a.ring_v) + gbase * a.W * D : nullptr;
    const int ns = a.n_sinks;
    const uint16_t* sk = ns ? reinterpret_cast<const uint16_t*>(a.sink_k) + gbase * ns * D : nullptr;
    const uint16_t* sv = ns ? reinterpret_cast<const uint16_t*>(a.sink_v) + gbase * ns * D : nullptr;
    const long kp_lo = max((long)a.sinks, p_first - a.W + 1);
    const int has_sink = ns > 0 ? 1 : 0;
    const int nwin = kp_lo <= p_last ? (int)((p_last - kp_lo) / FA_KB) + 1 : 0;
    const int nblk = has_sink + nwin;
    // key part p of a split item: blocks ceil(nblk p / P) .. ceil(nblk (p + 1) / P) - 1 (P = 2: the two halves)
    const int i_beg = SPLIT && half >= 0 ? (nblk * half + P - 1) / P : 0;
    const int i_end = SPLIT && half >= 0 ? (nblk * (half + 1) + P - 1) / P : nblk;
    const int slot_lo = rk ? (int)(kp_lo % a.W) : 0;               // ring slot of kp_lo (one division)
    const long start = a.start;

    // Copy block i's K and V rows into tile t with buffer_load ... lds (row r's 16-byte block pb holds the row's block
    // pb ^ sw(r)). Instruction j of wave wv fills 1 KB of the tile: rows row0 + RPI j .. + RPL - 1, lane -> (row,
    // block) fixed; the swizzle depends only on row0 (RPI is a multiple of the swizzle period), so each lane's byte
    // offset is one clamp and one multiply-add per instruction. The source of a block is wave-uniform: the sinks, the
    // chunk (rows past the last query are clamped to it: valid data, masked), the ring (slot kp mod W), or, for the
    // one block that straddles the chunk start, each lane's row from its own source. Every descriptor stays uniform,
    // so no load is serialised over distinct lane values.
    constexpr int RPL = 64 / NBLK;                 // tile rows per 1 KB copy
    constexpr int RPI = NW * RPL;                  // rows between a wave's consecutive copies
    static_assert(NBLK >= 16 ? RPI % 16 == 0 : RPI % 32 == 0, "swizzle must be invariant across a wave's copies");
    const int row0 = wv * RPL + lane / NBLK, pb0 = lane % NBLK;
    const uint32_t kb0 = 16u * (pb0 ^ fa_swk<NBLK>(row0)), vb0 = 16u * (pb0 ^ fa_swv<NBLK>(row0));
    const rsrc_t rsk = make_rsrc(sk, (uint32_t)(ns * ROWB)), rsv = make_rsrc(sv, (uint32_t)(ns * ROWB));
    const rsrc_t rrk = make_rsrc(rk, rk ? (uint32_t)(a.W * ROWB) : 0u), rrv = make_rsrc(rv, rv ? (uint32_t)(a.W * ROWB) : 0u);
    const rsrc_t rck = make_rsrc(ck, (uint32_t)(((long)(a.T - 1) * a.k_st + D) * 2));
    const rsrc_t rcv = make_rsrc(cv, (uint32_t)(((long)(a.T - 1) * a.v_st + D) * 2));
    const uint32_t kst_b = (uint32_t)(a.k_st * 2), vst_b = (uint32_t)(a.v_st * 2);
    const uint32_t crow_max = (uint32_t)(p_last - start);          // chunk row of the last query
    // 16 bytes at byte offset off + soff (per lane; soff wave-uniform) -> dst + 16 lane
    auto dma = [](rsrc_t r, void* dst, uint32_t off, uint32_t soff = 0u) {
        __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)dst, 16, off, soff, 0, 0);
    };
    auto stage = [&](FaTile<D>& t, int i) {
        char* tk = reinterpret_cast<char*>(t.k) + wv * 1024;
        char* tv = reinterpret_cast<char*>(t.v) + wv * 1024;
        if (has_sink && i == 0) {
#pragma unroll
            for (int j = 0; j < NLD; ++j) {
                const uint32_t r = (uint32_t)min(row0 + RPI * j, ns - 1);
                dma(rsk, tk + NW * j * 1024, r * ROWB + kb0);
                dma(rsv, tv + NW * j * 1024, r * ROWB + vb0);
            }
            return;
        }
        const long kpb = kp_lo + (long)(i - has_sink) * FA_KB;        // position of the block's row 0
        if (kpb >= start || !rk) {                                     // chunk rows only
            const uint32_t rb = (uint32_t)(kpb - start);               // wraps (huge) before the chunk: clamped
#pragma unroll
            for (int j = 0; j < NLD; ++j) {
                const uint32_t cr = min(rb + (uint32_t)(row0 + RPI * j), crow_max);
                dma(rck, tk + NW * j * 1024, __umul24(cr, kst_b) + kb0);
                dma(rcv, tv + NW * j * 1024, __umul24(cr, vst_b) + vb0);
            }
            return;
        }
        // ring rows (position < start): slot (slot_lo + kp - kp_lo) mod W, below 2W since kp - kp_lo <= W - 2
        int sb = slot_lo + (int)(kpb - kp_lo);
        sb = sb >= a.W ? sb - a.W : sb;
        const int nring = (int)min((long)FA_KB, start - kpb);          // rows before the chunk start
        const uint32_t rb = (uint32_t)(kpb - start);
#pragma unroll
        for (int j = 0; j < NLD; ++j) {
            const int r = row0 + RPI * j;
            if (r < nring) {
                const uint32_t u = (uint32_t)(sb + r), sl = min(u, u - (uint32_t)a.W);
                dma(rrk, tk + NW * j * 1024, sl * ROWB + kb0);
                dma(rrv, tv + NW * j * 1024, sl * ROWB + vb0);
            }
            if (r >= nring) {                                          // the block straddles the chunk start
                const uint32_t cr = min(rb + (uint32_t)r, crow_max);
                dma(rck, tk + NW * j * 1024, __umul24(cr, kst_b) + kb0);
                dma(rcv, tv + NW * j * 1024, __umul24(cr, vst_b) + vb0);
            }
        }
    };
    // ring_pos of row `lane` of block i (0 when the row is not a ring row)
    const rsrc_t rpos = make_rsrc(a.ring_pos, a.ring_pos ? (uint32_t)a.W * 8u : 0u);
    auto load_rp = [&](int i) {
        const long kp = kp_lo + (long)(i - has_sink) * FA_KB + lane;
        int slot = slot_lo + (int)(kp - kp_lo);
        slot = slot >= a.W ? slot - a.W : slot;
        const bool ring = rk && !(has_sink && i == 0) && kp < start && kp <= p_last;
        return buf_ld8(rpos, ring ? (uint32_t)slot * 8u : 0xFFFFFFF0u);
    };
    auto valid_row = [&](int i, uint2 rp) {
        if (has_sink && i == 0) return lane < ns;
        const long kp = kp_lo + (long)(i - has_sink) * FA_KB + lane;
        if (kp > p_last) return false;
        return kp >= start || (rk && (long)(((uint64_t)rp.y << 32) | rp.x) == kp);
    };

    // ---- per-lane LDS fragment offsets
    int kbase[NKB];
    {
        const int skz = fa_swk<NBLK>(l16);
#pragma unroll
        for (int c = 0; c < NKB; ++c) kbase[c] = l16 * ROWB + 64 * (c ^ (skz >> 2)) + 16 * (lg ^ (skz & 3));
    }
    int vbase[NVB];
    {
        const int e = l16 >> 2, rowl = 4 * lg + e;            // row inside a 16-row group of the tile
        const int rho = fa_swv<NBLK>(rowl) >> 1;
#pragma unroll
        for (int c = 0; c < NVB; ++c)
            vbase[c] = rowl * ROWB + 32 * (c ^ rho) + 16 * ((l16 & 3) >> 1) + 8 * (l16 & 1);
    }

    f32x4 o[NDT][QT];
    float m[QT], l[QT];
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
        m[qt] = -INFINITY;
        l[qt] = 0.f;
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt) o[dt][qt] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
    const float cs = FA_LOG2E * rsqrtf((float)D);             // score scale in log2 units
    // the next block's copy plan when it is spread over the S product (set per block by step)
    bool spread = false;
    uint32_t off_k = 0, off_v = 0;
    char* tk_next = nullptr;
    char* tv_next = nullptr;
    const uint32_t step_k = (uint32_t)RPI * kst_b, step_v = (uint32_t)RPI * vst_b;

    auto compute = [&](const FaTile<D>& t, int i, uint64_t vmask) {
        const bool sink = has_sink && i == 0;
        const long kp0 = sink ? 0 : kp_lo + (long)(i - has_sink) * FA_KB;
        const int cnt = 64 - __builtin_clzll(vmask | 1ull);   // rows up to the last valid one
        const long kp1 = kp0 + cnt - 1;
        // this wave's queries see nothing of the block: skip; every row visible to every query: no mask
        const bool none = nqw == 0 || vmask == 0 || kp0 > qw1 || (!sink && qw0 - kp1 >= a.W);
        if (none) return;
        const bool full = vmask == ~0ull && kp1 <= qw0 && (sink || qw1 - kp0 < a.W);
        const char* Kb = reinterpret_cast<const char*>(t.k);
        const char* Vb = reinterpret_cast<const char*>(t.v);

        // S^T = K Q^T. K fragments of step kf + 1 are read while step kf multiplies; the scheduling barrier keeps the
        // compiler from hoisting every step's reads (and their registers) to the front.
        f32x4 s[4][QT];
#pragma unroll
        for (int kt = 0; kt < 4; ++kt)
#pragma unroll
            for (int qt = 0; qt < QT; ++qt) s[kt][qt] = f32x4{0.f, 0.f, 0.f, 0.f};
        auto read_k = [&](int kf, uint4 (&ak)[4]) {
#pragma unroll
            for (int kt = 0; kt < 4; ++kt) ak[kt] = lds16(Kb, kbase[kf % NKB] + 16 * kt * ROWB + 256 * (kf / NKB));
        };
        uint4 ak[4];
        read_k(0, ak);
#pragma unroll
        for (int kf = 0; kf < NKD; ++kf) {
            uint4 an[4];
            if (kf + 1 < NKD) read_k(kf + 1, an);
#pragma unroll
            for (int kt = 0; kt < 4; ++kt)
#pragma unroll
                for (int qt = 0; qt < QT; ++qt) mma<BF16>(s[kt][qt], ak[kt], fq[qt][kf]);
            if (spread) {                                    // copies j: K rows row0 + RPI j, then V rows
                constexpr int CPS = (2 * NLD + NKD - 1) / NKD;
#pragma unroll
                for (int c = 0; c < CPS; ++c) {
                    const int j = kf * CPS + c;
                    if (j < NLD) dma(rck, tk_next + NW * j * 1024, off_k, j * step_k);
                    else if (j < 2 * NLD) dma(rcv, tv_next + NW * (j - NLD) * 1024, off_v, (j - NLD) * step_v);
                }
            }
            if (kf + 1 < NKD) {
#pragma unroll
                for (int kt = 0; kt < 4; ++kt) ak[kt] = an[kt];
            }
            __builtin_amdgcn_sched_barrier(0);
        }

        // mask: element (kt, qt, e) is key row 16 kt + 4 lg + e, query 16 qt + l16 of the wave
        if (!full) {
            const long dq = qw0 - kp0;
            const int base = (int)max(min(dq, (long)(1 << 30)), -(long)(1 << 30)) + l16 - 4 * lg;
            const uint64_t vm = vmask >> (4 * lg);
#pragma unroll
            for (int kt = 0; kt < 4; ++kt)
#pragma unroll
                for (int qt = 0; qt < QT; ++qt)
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const int rel = base + 16 * (qt - kt) - e;
                        const bool vis = ((vm >> (16 * kt + e)) & 1ull) && rel >= 0 && (sink || rel < a.W);
                        s[kt][qt][e] = vis ? s[kt][qt][e] : -INFINITY;
                    }
        }

        // online softmax (lazy max)
#pragma unroll
        for (int qt = 0; qt < QT; ++qt) {
            float bm = s[0][qt][0];
#pragma unroll
            for (int kt = 0; kt < 4; ++kt)
#pragma unroll
                for (int e = 0; e < 4; ++e) bm = fmaxf(bm, s[kt][qt][e]);
            bm = fa_max4(bm) * cs;
            const bool up = bm > m[qt] + FA_SLACK;
            if (__builtin_amdgcn_ballot_w64(up)) {
                const float mn = up ? bm : m[qt];
                // 0 when m was -inf, 1 without update (also for a row that has seen no key yet while others update)
                const float corr = up ? __builtin_amdgcn_exp2f(m[qt] - mn) : 1.f;
                m[qt] = mn;
                l[qt] *= corr;
#pragma unroll
                for (int dt = 0; dt < NDT; ++dt) {
                    o[dt][qt][0] *= corr; o[dt][qt][1] *= corr; o[dt][qt][2] *= corr; o[dt][qt][3] *= corr;
                }
            }
            const float msub = m[qt] == -INFINITY ? 0.f : m[qt];
            float ls = 0.f;
#pragma unroll
            for (int kt = 0; kt < 4; ++kt)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float p = __builtin_amdgcn_exp2f(fmaf(s[kt][qt][e], cs, -msub));
                    s[kt][qt][e] = p;
                    ls += p;
                }
            l[qt] += ls;
        }

        // O^T += V^T P^T; P fragment f holds keys {32 f + 4 lg + e} (tile 2f) and {32 f + 16 + 4 lg + e} (tile 2f+1)
#pragma unroll
        for (int f = 0; f < 2; ++f) {
            uint4 pb[QT];
#pragma unroll
            for (int qt = 0; qt < QT; ++qt) {
                const f32x4 x0 = s[2 * f][qt], x1 = s[2 * f + 1][qt];
                pb[qt] = make_uint4(pack_bf16x2(x0[0], x0[1]), pack_bf16x2(x0[2], x0[3]), pack_bf16x2(x1[0], x1[1]),
                                    pack_bf16x2(x1[2], x1[3]));
            }
            // V^T fragments are read VPF tiles ahead of their MFMAs
            constexpr int VPF = 4;
            auto read_v = [&](int dt) {
                const char* p = Vb + vbase[dt % NVB] + 32 * f * ROWB + 256 * (dt / NVB);
                const uint2 lo = fa_tr16(p), hi = fa_tr16(p + 16 * ROWB);
                return make_uint4(lo.x, lo.y, hi.x, hi.y);
            };
            uint4 vr[VPF];
#pragma unroll
            for (int q = 0; q < VPF - 1; ++q) vr[q] = read_v(q);
#pragma unroll
            for (int dt = 0; dt < NDT; ++dt) {
                if (dt + VPF - 1 < NDT) vr[(dt + VPF - 1) % VPF] = read_v(dt + VPF - 1);
#pragma unroll
                for (int qt = 0; qt < QT; ++qt) mma<BF16>(o[dt][qt], vr[dt % VPF], pb[qt]);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
    };

    // ---- main loop over key blocks, two tiles in turn. The next block is staged unconditionally (the last block
    // re-stages itself into the idle tile), so the compiler's wait counts never drain it before the current compute.
    // Its copies are spread over the S product when they need no clamping (all rows chunk rows up to the last query)
    // and the wave computes block i; a wave that sees nothing of block i skips its S product and copies at once.
    // (an unsplit item always runs its first block, masked out when the item has none)
    const bool run = !SPLIT || i_beg < i_end;
    uint2 rp = make_uint2(0u, 0u);
    if (run) {
        rp = load_rp(i_beg);
        stage(t0, i_beg);
    }
    auto step = [&](FaTile<D>& tc, FaTile<D>& tn, int i) {
        wait_vmem_all();
        __syncthreads();                                   // block i is in tc; every wave is done with tn
        const uint64_t vmask = __builtin_amdgcn_ballot_w64(valid_row(i, rp));
        const int inext = i + 1 < i_end ? i + 1 : i;
        rp = load_rp(inext);
        {
            const bool sink = has_sink && i == 0;
            const long kp0 = sink ? 0 : kp_lo + (long)(i - has_sink) * FA_KB;
            const long kp1 = kp0 + (64 - __builtin_clzll(vmask | 1ull)) - 1;
            const bool none = nqw == 0 || vmask == 0 || kp0 > qw1 || (!sink && qw0 - kp1 >= a.W);   // as in compute
            const long kpb = kp_lo + (long)(inext - has_sink) * FA_KB;
            spread = !none && !(has_sink && inext == 0) && (kpb >= start || !rk) &&
                     kpb + FA_KB - 1 - start <= (long)crow_max;
            if (spread) {
                const uint32_t rb = (uint32_t)(kpb - start) + (uint32_t)row0;
                off_k = __umul24(rb, kst_b) + kb0;
                off_v = __umul24(rb, vst_b) + vb0;
                tk_next = reinterpret_cast<char*>(tn.k) + wv * 1024;
                tv_next = reinterpret_cast<char*>(tn.v) + wv * 1024;
            } else {
                stage(tn, inext);
            }
        }
        compute(tc, i, vmask);
    };
    if (run) {                                             // uniform over the workgroup
        for (int i = i_beg;;) {
            step(t0, t1, i);
            if (++i >= i_end) break;
            step(t1, t0, i);
            if (++i >= i_end) break;
        }
        wait_vmem_all();                                   // the last (redundant) stage has landed: the epilogue
                                                           // reuses the tiles
    }

    if (SPLIT && half >= 0) {
        // partial rows of the key half, query qi at row qi: m (running max, log2 units), l, 2 unused, o unnormalised
        float* pp = a.part + (((long)xcd * sx + (idx - (per - sx))) * P + half) * FA_BQ * (D + 4);
#pragma unroll
        for (int qt = 0; qt < QT; ++qt) {
            const float lt = fa_sum4(l[qt]);
            const int qi = QW * wv + 16 * qt + l16;
            if (qi >= nq) continue;
            float* row = pp + (long)qi * (D + 4);
            if (lg == 0) *reinterpret_cast<float2*>(row) = make_float2(m[qt], lt);
#pragma unroll
            for (int dt = 0; dt < NDT; ++dt)
                nt_stf4(row + 4 + 16 * dt + 4 * lg, make_float4(o[dt][qt][0], o[dt][qt][1], o[dt][qt][2], o[dt][qt][3]));
        }
        return;
    }

    // ---- epilogue: row sums, normalise, lse (natural log), gamma mix, store o [B][T][H][D]. The normalised rows go
    // through LDS (the tiles are free now): a wave's MFMA layout gives each store instruction 64 bytes of 16 rows,
    // the row layout D / 4 lanes x 16 bytes of whole rows, so the memory reads and the stores move whole rows. The
    // memory reads and gate logits are issued first, so the transpose overlaps their latency. (The rows staged
    // this way measured the same as the direct MFMA-layout stores; the streaming accesses below gained 1.5 %.)
    constexpr int NC = D / 4;                      // 16-byte chunks per row
    constexpr int RPE = 64 / NC;                   // rows per row-phase instruction
    constexpr int NIE = QW / RPE;                  // row-phase instructions per wave
    constexpr int EB = QW * D * 4;                 // LDS bytes per wave
    static_assert(sizeof(FaTile<D>) % EB == 0 && RPE <= 16 && NC >= 16, "epilogue staging");
    __syncthreads();                               // every wave is done with both tiles
    char* eb = wv * EB < (int)sizeof(FaTile<D>) ? reinterpret_cast<char*>(&t0) + wv * EB
                                                : reinterpret_cast<char*>(&t1) + (wv * EB - (int)sizeof(FaTile<D>));
    const long orow0 = ((long)b * a.T + qi0) * H + h;   // (b, qi0, h) of [B][T][H]: query qi at orow0 + qi H
    const int rsub = lane / NC, cc = lane % NC;
    const bool om16 = a.mix_on && a.o_mem_dtype == DT_BF16;
    uint2 omr[NIE];
    if (om16) {
#pragma unroll
        for (int i = 0; i < NIE; ++i) {
            const int q = min(QW * wv + RPE * i + rsub, nq - 1);
            omr[i] = fa_ld8_nt(reinterpret_cast<const uint16_t*>(a.o_mem) + (orow0 + (long)q * H) * D + 4 * cc);
        }
    }
    float zr[QT];
#pragma unroll
    for (int qt = 0; qt < QT; ++qt)
        zr[qt] = a.mix_on ? a.z[orow0 + (long)min(QW * wv + 16 * qt + l16, nq - 1) * H] : 0.f;   // z [B][T][H]
    const float lnW = logf((float)a.W);
    const float ms = a.mix_on ? a.mem_scale[h] : 0.f;
    float gam[QT];
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
        const float lt = fa_sum4(l[qt]);
        const int qi = QW * wv + 16 * qt + l16;
        const float inv = 1.f / lt;
        const float lse = (m[qt] + __log2f(lt)) * FA_LN2;
        if (a.lse && lg == 0 && qi < nq) a.lse[((long)b * H + h) * a.T + qi0 + qi] = lse;
        gam[qt] = 0.f;
        if (a.mix_on && p_first + qi >= a.W) gam[qt] = 1.f / (1.f + __expf(-(zr[qt] + a.mix_lse[h] * (lse - lnW))));
        // row r = 16 qt + l16 of the wave, chunk c = 4 dt + lg at chunk position c ^ (r mod 16)
        const int r = 16 * qt + l16;
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt)
            *reinterpret_cast<float4*>(eb + r * (D * 4) + 16 * ((4 * dt + lg) ^ l16)) =
                make_float4(o[dt][qt][0] * inv, o[dt][qt][1] * inv, o[dt][qt][2] * inv, o[dt][qt][3] * inv);
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
    for (int i = 0; i < NIE; ++i) {
        const int r = RPE * i + rsub, qi = QW * wv + r;
        const float4 x = *reinterpret_cast<const float4*>(eb + r * (D * 4) + 16 * (cc ^ (r & 15)));
        float r4[4] = {x.x, x.y, x.z, x.w};
        const long orow = (orow0 + (long)min(qi, nq - 1) * H) * D + 4 * cc;
        if (a.mix_on) {
            // lanes before the first memory query (gamma 0) keep the window output by selection, so rows the delta
            // rule never wrote cannot leak in
            const float g = __shfl(gam[(RPE * i) / 16], r & 15);
            float mv[4];
            if (om16) {
                mv[0] = __uint_as_float(omr[i].x << 16); mv[1] = __uint_as_float(omr[i].x & 0xffff0000u);
                mv[2] = __uint_as_float(omr[i].y << 16); mv[3] = __uint_as_float(omr[i].y & 0xffff0000u);
            } else {
                const float4 f4 = nt_ldf4(reinterpret_cast<const float*>(a.o_mem) + orow);
                mv[0] = f4.x; mv[1] = f4.y; mv[2] = f4.z; mv[3] = f4.w;
            }
#pragma unroll
            for (int e = 0; e < 4; ++e) r4[e] = g != 0.f ? r4[e] + g * (ms * mv[e] - r4[e]) : r4[e];
        }
        if (qi < nq) fa_st4_nt<BO>(a.o, orow, r4);
    }
}

// The P key parts of each split item: rows m_p, l_p, o_p (each relative to its own running max) combine as
// L = sum c_p l_p, O = sum c_p o_p with c_p = exp2(m_p - max m); then the window epilogue of window_fa_kernel:
// o = O / L, lse, gamma mix, store. D / 4 threads per query row, 4 consecutive d each.
template <int D, bool BO>
__global__ __launch_bounds__(256) void window_merge_kernel(WinArgs a) {
    constexpr int LPR = D / 4;
    const long t = (long)blockIdx.x * 256 + threadIdx.x;
    const long row = t / LPR;
    const int c = (int)(t % LPR), sx = a.split_x;
    if (row >= (long)FA_NXCD * sx * FA_BQ) return;
    const int s = (int)(row / FA_BQ), qi = (int)(row % FA_BQ);
    const int R = a.R, G = a.G, H = G * R;
    const int nqb = (a.T + FA_BQ - 1) / FA_BQ;
    const long wi = window_item(a.map, s / sx, a.map.per - sx + s % sx);
    if (wi < 0) return;
    const int r = (int)(wi % R);
    long rest = wi / R;
    const int qb = nqb - 1 - (int)(rest % nqb);
    rest /= nqb;
    const int g = (int)(rest % G), b = (int)(rest / G), h = g * R + r;
    const long tq = (long)qb * FA_BQ + qi;
    if (tq >= a.T) return;
    // parts p = 0 .. P - 1 of the slot, added in order (P = 2: c0 x0 + c1 x1)
    const int P = a.split_p;
    const float* p0 = a.part + ((long)s * P * FA_BQ + qi) * (D + 4);
    constexpr long PS = (long)FA_BQ * (D + 4);           // floats between consecutive parts of a row
    float mx = -INFINITY;
    for (int p = 0; p < P; ++p) mx = fmaxf(mx, p0[p * PS]);
    float lt = 0.f, ox = 0.f, oy = 0.f, oz = 0.f, ow = 0.f;
    for (int p = 0; p < P; ++p) {
        const float* pp = p0 + p * PS;
        const float2 ml = *reinterpret_cast<const float2*>(pp);
        const float4 op = *reinterpret_cast<const float4*>(pp + 4 + 4 * c);
        const float cp = ml.x == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(ml.x - mx);
        if (p == 0) {
            lt = cp * ml.y; ox = cp * op.x; oy = cp * op.y; oz = cp * op.z; ow = cp * op.w;
        } else {
            lt += cp * ml.y; ox += cp * op.x; oy += cp * op.y; oz += cp * op.z; ow += cp * op.w;
        }
    }
    const float inv = 1.f / lt;
    const float lse = (mx + __log2f(lt)) * FA_LN2;
    if (a.lse && c == 0) a.lse[((long)b * H + h) * a.T + tq] = lse;
    float r4[4] = {ox * inv, oy * inv, oz * inv, ow * inv};
    const long orow = (((long)b * a.T + tq) * H + h) * D;
    if (a.mix_on && a.start + tq >= a.W) {
        const float gam =
            1.f / (1.f + __expf(-(a.z[((long)b * a.T + tq) * H + h] + a.mix_lse[h] * (lse - logf((float)a.W)))));
        if (gam != 0.f) {                                  // rows the delta rule never wrote stay out, as in the kernel
            const float ms = a.mem_scale[h];
            float4 om[1];
            load_om<1>(a, orow + 4 * c, om);
            const float mv[4] = {om[0].x, om[0].y, om[0].z, om[0].w};
#pragma unroll
            for (int e = 0; e < 4; ++e) r4[e] = r4[e] + gam * (ms * mv[e] - r4[e]);
        }
    }
    if constexpr (BO) store4<BF16>(reinterpret_cast<uint16_t*>(a.o) + orow + 4 * c, r4[0], r4[1], r4[2], r4[3]);
    else store4<F32>(reinterpret_cast<float*>(a.o) + orow + 4 * c, r4[0], r4[1], r4[2], r4[3]);
}

namespace {

template <int D>
int launch_window_fa(const WinArgs& args, hipStream_t stream) {
    static_assert(FA_BQ == 128 && FA_NXCD == 8, "WinMap assumes 128-query items over 8 XCDs");
    WinArgs a = args;
    a.map = window_map(a.B, a.G, a.R, a.T, a.W, a.start);
    const long per = a.map.per;
    const int sx = a.split_x, P = sx ? a.split_p : 1;
    if (sx < 0 || sx > per || (sx && (!a.part || P < 2 || P > 8))) return BF_STATUS_INVALID;
    if (FA_NXCD * (per + (long)sx * (P - 1)) > 0x7fffffffL) return BF_STATUS_INVALID;
    // chunk K / V rows are addressed by 32-bit buffer offsets
    if (((long)(a.T - 1) * a.k_st + D) * 2 > 0xffffffffL || ((long)(a.T - 1) * a.v_st + D) * 2 > 0xffffffffL)
        return BF_ERR_UNSUPPORTED;
    // the tile copy forms row offsets with 24-bit multiplies: chunk rows and row strides in bytes below 2^24
    if (a.T >= (1L << 24) || a.k_st * 2 >= (1L << 24) || a.v_st * 2 >= (1L << 24)) return BF_ERR_UNSUPPORTED;
    const dim3 grid((unsigned)(FA_NXCD * (per + (long)sx * (P - 1)))), block(FaShape<D>::NT);
    const bool bo = a.o_dtype == DT_BF16;
    if (sx) {
        if (bo) hipLaunchKernelGGL((window_fa_kernel<D, true, true>), grid, block, 0, stream, a);
        else hipLaunchKernelGGL((window_fa_kernel<D, false, true>), grid, block, 0, stream, a);
    } else {
        if (bo) hipLaunchKernelGGL((window_fa_kernel<D, true, false>), grid, block, 0, stream, a);
        else hipLaunchKernelGGL((window_fa_kernel<D, false, false>), grid, block, 0, stream, a);
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || !sx) return e == hipSuccess ? 0 : (int)e;
    const dim3 mgrid((unsigned)(((long)FA_NXCD * sx * FA_BQ * (D / 4) + 255) / 256));
    if (bo) hipLaunchKernelGGL((window_merge_kernel<D, true>), mgrid, dim3(256), 0, stream, a);
    else hipLaunchKernelGGL((window_merge_kernel<D, false>), mgrid, dim3(256), 0, stream, a);
    e = hipGetLastError();
    return e == hipSuccess ? 0 : (int)e;
}

}  // namespace

int window_fa_dispatch(const WinArgs& a, hipStream_t stream) {
    switch (a.D) {
        case 64: return launch_window_fa<64>(a, stream);
        case 128: return launch_window_fa<128>(a, stream);
        case 256: return launch_window_fa<256>(a, stream);
        default: return BF_ERR_UNSUPPORTED;
    }
}

}  // namespace bf
