// K1: chunked gated delta rule, GQA form (one fp32 state per KV head, read by R query heads), packed varlen.
//
// Algorithm (UT/WY representation; reference: Heimdall/heimdall/kernels.py:94-129, motor.py:70-102). For chunk
// of C = 64 tokens of KV head g with in-chunk cumulative log-decay gc:
//   A  = strict_lower(beta_i e^{gc_i - gc_j} k_i.k_j),  Tm = (I + A)^-1
//   w  = Tm diag(beta e^{gc}) K,   u = Tm diag(beta) V,   kt = (K e^{gc_last - gc})^T
//   attn_r = scale (q_r K^T * e^{gc_i - gc_j})[i >= j]
//   scan:  v_new = u - w S;  o_r = scale (q_r e^{gc}) S + attn_r v_new;  S = e^{gc_last} S + kt v_new
//
// Two kernels:
//   gdn_prep  grid (chunks, G): everything that does not depend on S, fully parallel.
//   gdn_scan  one workgroup per (sequence, KV head, Dv / BV slab), XCD-grouped: the sequential pass. Columns of S are independent, so each workgroup
//             owns a BV-column slab of one KV head's state, keeps it in registers (fp32) for the whole sequence and
//             a bf16/fp32 copy in LDS as the MFMA B operand.
//
// Workspace (per chunk id cid, KV head g; C = 64):
//   gcum [cid][g][C] f32 | w [cid][g][C][D] E | uT [cid][g][D][C] f32 | kt [cid][g][D][C] E | attn [cid][h][C][C] E
#include "bf_common.h"
#include "bf_internal.h"

namespace bf {

constexpr int CH = 64;     // chunk length
constexpr int kXcds = 8;   // XCDs of an MI355X (gfx950); workgroups are dispatched round-robin across them
constexpr int NT = 256;    // threads per workgroup (4 waves)

template <class E, int D>
struct PrepShared {
    typename E::T xT[D][CH + E::VEC];      // K^T, later V^T (t contiguous)
    float A[CH][CH + 4];                   // strictly lower A (fp32)
    typename E::T Tw[CH][CH + E::VEC];     // Tm diag(beta e^gc)
    typename E::T Tu[CH][CH + E::VEC];     // Tm diag(beta)
    float gc[CH];
    float beta[CH];
};

// Load rows [0, len) of a C x D token-major tile (row stride ld elements) transposed into dst[D][C + VEC].
template <class E, int D>
__device__ __forceinline__ void load_transposed(typename E::T (*dst)[CH + E::VEC], const typename E::T* src, long ld,
                                                int len) {
    constexpr int VEC = E::VEC, NBT = CH / VEC, NBD = D / VEC;
    for (int blk = threadIdx.x; blk < NBT * NBD; blk += NT) {
        const int bt = blk % NBT, bd = blk / NBT;
        uint4 r[VEC];
#pragma unroll
        for (int i = 0; i < VEC; ++i) {
            const int t = bt * VEC + i;
            r[i] = t < len ? ld16(src + (long)t * ld + bd * VEC) : zero16();
        }
        transpose_block<E>(r);
#pragma unroll
        for (int j = 0; j < VEC; ++j) st16(&dst[bd * VEC + j][bt * VEC], r[j]);
    }
}

template <class E, int D>
__global__ __launch_bounds__(NT) void gdn_prep_kernel(GdnArgs a) {
    using T = typename E::T;
    constexpr int VEC = E::VEC, KF = E::KF;
    __shared__ PrepShared<E, D> sm;
    SeqInfo si;
    if (!locate_chunk(blockIdx.x, a.cu_seqlens, a.num_seqs, a.seq_len, CH, si)) return;
    const int g = blockIdx.y, G = a.G, R = a.R, H = G * R;
    const long cid = blockIdx.x;
    const int lane = lane_id(), wv = wave_id(), l16 = lane & 15, lg = lane >> 4;
    const T* K = reinterpret_cast<const T*>(a.k) + si.tok0 * G * D + (long)g * D;
    const T* V = reinterpret_cast<const T*>(a.v) + si.tok0 * G * D + (long)g * D;
    const long ldk = (long)G * D;

    if (wv == 0) {
        float gv = 0.f, bv = 0.f;
        if (lane < si.len) {
            gv = a.g[(si.tok0 + lane) * G + g];
            bv = a.beta[(si.tok0 + lane) * G + g];
        }
#pragma unroll
        for (int off = 1; off < WAVE; off <<= 1) {
            const float y = __shfl_up(gv, off);
            if (lane >= off) gv += y;
        }
        sm.gc[lane] = gv;
        sm.beta[lane] = bv;
        a.ws_gcum[(cid * G + g) * CH + lane] = gv;
    }
    load_transposed<E, D>(sm.xT, K, ldk, si.len);
    __syncthreads();

    // A = strict_lower(beta_r e^{gc_r - gc_c} (K K^T)_{rc}). K K^T is symmetric: tile (rt, ct) with rt <= ct read
    // in transposed form fills rows 16ct.., columns 16rt.. of A.
    for (int tix = wv; tix < 10; tix += 4) {
        const int rt = tix < 4 ? 0 : tix < 7 ? 1 : tix < 9 ? 2 : 3;
        const int ct = rt + (tix - (rt == 0 ? 0 : rt == 1 ? 4 : rt == 2 ? 7 : 9));
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
        const int ra = 16 * rt + l16, rb = 16 * ct + l16;
#pragma unroll
        for (int kk = 0; kk < D; kk += KF) {
            const uint4 fa = ra < si.len ? ld16(K + (long)ra * ldk + kk + VEC * lg) : zero16();
            const uint4 fb = rb < si.len ? ld16(K + (long)rb * ldk + kk + VEC * lg) : zero16();
            mma<E>(acc, fa, fb);
        }
        const int r = 16 * ct + l16;
        const float br = sm.beta[r], gr = sm.gc[r];
        float o[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int c = 16 * rt + 4 * lg + i;
            o[i] = r > c ? br * __expf(gr - sm.gc[c]) * acc[i] : 0.f;
        }
        *reinterpret_cast<float4*>(&sm.A[r][16 * rt + 4 * lg]) = make_float4(o[0], o[1], o[2], o[3]);
    }
    __syncthreads();

    if (wv == 0) {
        // (I + A)^-1 by forward substitution, one column per lane: x_i = [i == j] - sum_{m < i} A[i][m] x_m
        const int j = lane;
        float x[CH];
#pragma unroll
        for (int i = 0; i < CH; ++i) {
            float acc = i == j ? 1.f : 0.f;
#pragma unroll
            for (int m = 0; m < i; ++m) acc -= sm.A[i][m] * x[m];
            x[i] = acc;
        }
        const float bj = sm.beta[j], ej = bj * __expf(sm.gc[j]);
#pragma unroll
        for (int i = 0; i < CH; ++i) {
            sm.Tw[i][j] = E::from_f(x[i] * ej);
            sm.Tu[i][j] = E::from_f(x[i] * bj);
        }
    } else {
        // attn_r^T = K q_r^T (rows t' = key, cols t = query), masked to t' <= t, decayed and scaled.
        const T* Q = reinterpret_cast<const T*>(a.q) + si.tok0 * H * D + (long)g * R * D;
        const long ldq = (long)H * D;
        for (int item = wv - 1; item < R * 16; item += 3) {
            const int r = item >> 4, tile = item & 15;
            const int at = tile >> 2, bt = tile & 3;     // at: key tile (rows), bt: query tile (cols)
            const int t = 16 * bt + l16;
            T* dst = reinterpret_cast<T*>(a.ws_attn) + ((cid * H + (long)g * R + r) * CH + t) * CH + 16 * at + 4 * lg;
            if (at > bt) {
                store4<E>(dst, 0.f, 0.f, 0.f, 0.f);
                continue;
            }
            f32x4 acc = {0.f, 0.f, 0.f, 0.f};
            const int ka = 16 * at + l16;
#pragma unroll
            for (int kk = 0; kk < D; kk += KF) {
                const uint4 fa = ka < si.len ? ld16(K + (long)ka * ldk + kk + VEC * lg) : zero16();
                const uint4 fb = t < si.len ? ld16(Q + (long)t * ldq + (long)r * D + kk + VEC * lg) : zero16();
                mma<E>(acc, fa, fb);
            }
            float o[4];
            const float gt = sm.gc[t];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int tk = 16 * at + 4 * lg + i;
                o[i] = tk <= t ? a.scale * __expf(gt - sm.gc[tk]) * acc[i] : 0.f;
            }
            store4<E>(dst, o[0], o[1], o[2], o[3]);
        }
    }
    __syncthreads();

    // w^T = K^T Tw^T (rows d, cols t) -> w [t][d] row-major; kt = K^T e^{gc_last - gc}.
    {
        T* W = reinterpret_cast<T*>(a.ws_w) + (cid * G + g) * CH * D;
        for (int tile = wv; tile < (D / 16) * 4; tile += 4) {
            const int rd = tile >> 2, ct = tile & 3;
            f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int kk = 0; kk < CH; kk += KF) {
                const uint4 fa = ld16(&sm.xT[16 * rd + l16][kk + VEC * lg]);
                const uint4 fb = ld16(&sm.Tw[16 * ct + l16][kk + VEC * lg]);
                mma<E>(acc, fa, fb);
            }
            store4<E>(W + (long)(16 * ct + l16) * D + 16 * rd + 4 * lg, acc[0], acc[1], acc[2], acc[3]);
        }
        T* KT = reinterpret_cast<T*>(a.ws_kt) + (cid * G + g) * D * CH;
        const float glast = sm.gc[CH - 1];
        for (int idx = threadIdx.x; idx < D * (CH / VEC); idx += NT) {
            const int d = idx / (CH / VEC), t0 = (idx % (CH / VEC)) * VEC;
            typename E::T vals[VEC];
            *reinterpret_cast<uint4*>(vals) = ld16(&sm.xT[d][t0]);
#pragma unroll
            for (int e = 0; e < VEC; ++e) vals[e] = E::from_f(E::to_f(vals[e]) * __expf(glast - sm.gc[t0 + e]));
            st16(KT + (long)d * CH + t0, *reinterpret_cast<uint4*>(vals));
        }
    }
    __syncthreads();
    load_transposed<E, D>(sm.xT, V, ldk, si.len);
    __syncthreads();

    // u = Tu V (rows t, cols d) -> uT [d][t] fp32.
    {
        float* UT = a.ws_uT + (cid * G + g) * D * CH;
        for (int tile = wv; tile < (D / 16) * 4; tile += 4) {
            const int rd = tile >> 2, ct = tile & 3;
            f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int kk = 0; kk < CH; kk += KF) {
                const uint4 fa = ld16(&sm.Tu[16 * ct + l16][kk + VEC * lg]);
                const uint4 fb = ld16(&sm.xT[16 * rd + l16][kk + VEC * lg]);
                mma<E>(acc, fa, fb);
            }
            *reinterpret_cast<float4*>(UT + (long)(16 * rd + l16) * CH + 16 * ct + 4 * lg) =
                make_float4(acc[0], acc[1], acc[2], acc[3]);
        }
    }
}

// ------------------------------------------------------------------------------------------------ sequential scan
// 8 waves per workgroup, specialised:
//   row waves   (0-3): wave w owns chunk rows 16w..16w+15: v_new = u - w S (step 1); the outputs
//                      o = scale e^{gc} q S_old + attn v_new (step 3).
//   state waves (4-7): wave w owns state row tiles (w-4) + 4i: S = e^{gc_last} S + kt v_new (step 2), reading
//                      each v_new fragment once for all of its row tiles.
// Per chunk: step 1 | barrier | step 2 || step 3 | barrier.
// Prefetch: each wave issues the loads of its next-chunk operand fragments at the start of the current chunk and
// copies them into its current set after the chunk's work, so the only memory wait sits at the end of the chunk.
// Chunk operands are read through buffer descriptors (uniform base in SGPRs, 32-bit lane offsets); rows past the end
// of a sequence read as zero and their output stores are dropped by the descriptor's range.
constexpr int NT_SCAN = 512;

template <class E, int D, int BV>
struct ScanShared {
    typename E::T sT[2][BV][D + E::VEC];   // S^T slab (double buffered): [column j][row d]
    typename E::T vnT[BV][CH + E::VEC];    // v_new^T slab: [column j][token t]
};

template <class E, int D, int BV>
struct RowFrags {                         // row-wave operands of one chunk
    static constexpr int NKD = D / E::KF, NKC = CH / E::KF, NCT = BV / 16;
    uint4 w[NKD];          // w rows (A operand of w S)
    uint4 at[NKC];         // attn rows of query head r = 0
    float4 u[NCT];         // u^T[j][t..t+3]
    float4 gq;             // gc of accumulator rows 16w + 4lg .. +3
};

template <class E, int D, int BV>
struct StateFrags {                       // state-wave operands of one chunk
    static constexpr int NKC = CH / E::KF, RPW = (D / 16 + 3) / 4;
    uint4 kt[RPW][NKC];    // kt rows of this wave's state row tiles
    float gc;              // gc of row `lane` (vector load; a scalar load would be waited on at every barrier)
};

struct ChunkPos {
    long cid, t0;
    int len;
};

__device__ __forceinline__ ChunkPos chunk_pos(int c, int first, long tok0, long tok1) {
    ChunkPos p;
    p.cid = first + c;
    p.t0 = tok0 + (long)c * CH;
    p.len = (int)((tok1 - p.t0) < CH ? (tok1 - p.t0) : CH);
    return p;
}

template <class E, int D>
__device__ __forceinline__ rsrc_t q_rsrc(const GdnArgs& a, const ChunkPos& p, int h) {
    const long H = (long)a.G * a.R, es = sizeof(typename E::T);
    return make_rsrc(reinterpret_cast<const char*>(a.q) + (p.t0 * H + h) * D * es, (uint32_t)(p.len * H * D * es));
}

template <class E>
__device__ __forceinline__ rsrc_t attn_rsrc(const GdnArgs& a, const ChunkPos& p, int h) {
    constexpr int ES = sizeof(typename E::T);
    const long H = (long)a.G * a.R;
    return make_rsrc(reinterpret_cast<const char*>(a.ws_attn) + (p.cid * H + h) * CH * CH * ES, CH * CH * ES);
}

template <class E, int D, int BV>
__device__ __forceinline__ void load_rows(RowFrags<E, D, BV>& f, const GdnArgs& a, const ChunkPos& p, int g, int j0,
                                          int wv, int l16, int lg) {
    using F = RowFrags<E, D, BV>;
    constexpr int VEC = E::VEC, KF = E::KF, ES = sizeof(typename E::T);
    const int G = a.G, H = G * a.R, h = g * a.R;
    const int t = 16 * wv + l16;
    const rsrc_t rw = make_rsrc(reinterpret_cast<const char*>(a.ws_w) + (p.cid * G + g) * CH * D * ES, CH * D * ES);
#pragma unroll
    for (int kf = 0; kf < F::NKD; ++kf) f.w[kf] = buf_ld16(rw, (t * D + VEC * lg + kf * KF) * ES);
    const rsrc_t ra = attn_rsrc<E>(a, p, h);
#pragma unroll
    for (int kf = 0; kf < F::NKC; ++kf) f.at[kf] = buf_ld16(ra, (t * CH + VEC * lg + kf * KF) * ES);
    const rsrc_t ru = make_rsrc(a.ws_uT + (p.cid * G + g) * D * CH, D * CH * 4);
#pragma unroll
    for (int ct = 0; ct < F::NCT; ++ct) f.u[ct] = buf_ldf4(ru, ((j0 + 16 * ct + l16) * CH + 16 * wv + 4 * lg) * 4);
    const rsrc_t rg = make_rsrc(a.ws_gcum + (p.cid * G + g) * CH, CH * 4);
    f.gq = buf_ldf4(rg, (16 * wv + 4 * lg) * 4);
}

template <class E, int D, int BV>
__device__ __forceinline__ void load_state(StateFrags<E, D, BV>& f, const GdnArgs& a, const ChunkPos& p, int g,
                                           int ws, int l16, int lg) {
    using F = StateFrags<E, D, BV>;
    constexpr int VEC = E::VEC, KF = E::KF, ES = sizeof(typename E::T);
    const rsrc_t rk = make_rsrc(reinterpret_cast<const char*>(a.ws_kt) + (p.cid * a.G + g) * D * CH * ES,
                                D * CH * ES);
#pragma unroll
    for (int ri = 0; ri < F::RPW; ++ri) {
        const int rt = ws + 4 * ri < D / 16 ? ws + 4 * ri : 0;
#pragma unroll
        for (int kf = 0; kf < F::NKC; ++kf) f.kt[ri][kf] = buf_ld16(rk, ((16 * rt + l16) * CH + VEC * lg + kf * KF) * ES);
    }
    const rsrc_t rg = make_rsrc(a.ws_gcum + (p.cid * a.G + g) * CH, CH * 4);
    f.gc = buf_ldf(rg, lane_id() * 4);
}

// acc(rows 16*wv.., BV columns) += A(rows, D) S_old.
template <class E, int D, int BV>
__device__ __forceinline__ void times_state(const ScanShared<E, D, BV>& sm, int buf, const uint4 (&a0)[D / E::KF],
                                            f32x4 (&c0)[BV / 16], int l16, int lg) {
    constexpr int VEC = E::VEC, KF = E::KF, NCT = BV / 16, NKD = D / E::KF;
#pragma unroll
    for (int kf = 0; kf < NKD; ++kf)
#pragma unroll
        for (int ct = 0; ct < NCT; ++ct) mma<E>(c0[ct], a0[kf], ld16(&sm.sT[buf][16 * ct + l16][kf * KF + VEC * lg]));
}

// acc += attn_rows(16 x C) v_new(C x BV), then store the rows (row i of acc scaled by rs[i] before the add).
template <class E, int D, int BV, bool BO>
__device__ __forceinline__ void finish_output(const ScanShared<E, D, BV>& sm, const uint4 (&fa)[CH / E::KF],
                                              f32x4 (&acc)[BV / 16], const float4& rs, const GdnArgs& a,
                                              const ChunkPos& p, int h, int j0, int wv, int l16, int lg) {
    constexpr int VEC = E::VEC, KF = E::KF, NCT = BV / 16, NKC = CH / E::KF;
    constexpr int OS = BO ? 2 : 4;
    const int H = a.G * a.R;
#pragma unroll
    for (int ct = 0; ct < NCT; ++ct) {
        acc[ct][0] *= rs.x;
        acc[ct][1] *= rs.y;
        acc[ct][2] *= rs.z;
        acc[ct][3] *= rs.w;
    }
#pragma unroll
    for (int kf = 0; kf < NKC; ++kf)
#pragma unroll
        for (int ct = 0; ct < NCT; ++ct) mma<E>(acc[ct], fa[kf], ld16(&sm.vnT[16 * ct + l16][kf * KF + VEC * lg]));
    const rsrc_t ro = make_rsrc(reinterpret_cast<char*>(a.o) + (p.t0 * H + h) * (long)D * OS,
                                (uint32_t)((long)p.len * H * D * OS));
#pragma unroll
    for (int ct = 0; ct < NCT; ++ct)
#pragma unroll
        for (int i = 0; i < 4; ++i) buf_st_out<BO>(ro, (16 * wv + 4 * lg + i) * H * D + j0 + 16 * ct + l16, acc[ct][i]);
}

template <class E, int D, int BV, bool BO>
__device__ __forceinline__ void rows_loop(ScanShared<E, D, BV>& sm, const GdnArgs& a, int count, int first, long tok0,
                                          long tok1, int g, int j0, int wv, int lane) {
    using F = RowFrags<E, D, BV>;
    constexpr int VEC = E::VEC, KF = E::KF, NCT = F::NCT, NKD = F::NKD, NKC = F::NKC, ES = sizeof(typename E::T);
    const int l16 = lane & 15, lg = lane >> 4;
    const int t = 16 * wv + l16;
    const int G = a.G, R = a.R, H = G * R;
    F cur;
    if (count > 0) load_rows<E, D, BV>(cur, a, chunk_pos(0, first, tok0, tok1), g, j0, wv, l16, lg);
    wait_vmem_all();
    __syncthreads();                                      // initial S^T written by the state waves
    for (int c = 0; c < count; ++c) {
        const int buf = c & 1;
        const ChunkPos p = chunk_pos(c, first, tok0, tok1);
        // the next-chunk prefetch is unconditional (the last chunk re-reads itself): a conditional prefetch makes the
        // compiler's wait counts cover both paths and drain the prefetch early
        const int cn = c + 1 < count ? c + 1 : c;
        // q rows of query head 0 for this chunk (used in step 3), issued ahead of the next-chunk prefetch
        uint4 fq0[NKD];
        {
            const rsrc_t rq = q_rsrc<E, D>(a, p, g * R);
#pragma unroll
            for (int kf = 0; kf < NKD; ++kf) fq0[kf] = buf_ld16(rq, (t * H * D + VEC * lg + kf * KF) * ES);
        }
        __builtin_amdgcn_sched_barrier(0);
        F nxt;
        load_rows<E, D, BV>(nxt, a, chunk_pos(cn, first, tok0, tok1), g, j0, wv, l16, lg);

        // step 1: v_new = u - w S
        f32x4 av[NCT], ao[NCT];
#pragma unroll
        for (int ct = 0; ct < NCT; ++ct) av[ct] = ao[ct] = f32x4{0.f, 0.f, 0.f, 0.f};
        times_state<E, D, BV>(sm, buf, cur.w, av, l16, lg);
#pragma unroll
        for (int ct = 0; ct < NCT; ++ct) {
            const float4 u = cur.u[ct];
            store4<E>(&sm.vnT[16 * ct + l16][16 * wv + 4 * lg], u.x - av[ct][0], u.y - av[ct][1], u.z - av[ct][2],
                      u.w - av[ct][3]);
        }
        // row factors scale * e^{gc} of the accumulator rows
        const float4 rs = make_float4(a.scale * __expf(cur.gq.x), a.scale * __expf(cur.gq.y),
                                      a.scale * __expf(cur.gq.z), a.scale * __expf(cur.gq.w));
        __syncthreads();

        // step 3: o_0 = q_0 S_old (row-scaled) + attn_0 v_new; further query heads of the group (R > 1) likewise
        times_state<E, D, BV>(sm, buf, fq0, ao, l16, lg);
        finish_output<E, D, BV, BO>(sm, cur.at, ao, rs, a, p, g * R, j0, wv, l16, lg);
        for (int r = 1; r < R; ++r) {
            const int h = g * R + r;
            uint4 fq[NKD], fa[NKC];
            const rsrc_t rq = q_rsrc<E, D>(a, p, h);
#pragma unroll
            for (int kf = 0; kf < NKD; ++kf) fq[kf] = buf_ld16(rq, (t * H * D + VEC * lg + kf * KF) * ES);
            const rsrc_t ra = attn_rsrc<E>(a, p, h);
#pragma unroll
            for (int kf = 0; kf < NKC; ++kf) fa[kf] = buf_ld16(ra, (t * CH + VEC * lg + kf * KF) * ES);
            f32x4 o2[NCT];
#pragma unroll
            for (int ct = 0; ct < NCT; ++ct) o2[ct] = f32x4{0.f, 0.f, 0.f, 0.f};
            times_state<E, D, BV>(sm, buf, fq, o2, l16, lg);
            finish_output<E, D, BV, BO>(sm, fa, o2, rs, a, p, h, j0, wv, l16, lg);
        }
        __syncthreads();
        cur = nxt;
    }
}

template <class E, int D, int BV>
__device__ __forceinline__ void state_loop(ScanShared<E, D, BV>& sm, f32x4 (&S)[StateFrags<E, D, BV>::RPW][BV / 16],
                                           const GdnArgs& a, int count, int first, long tok0, long tok1, int g, int ws,
                                           int lane) {
    using F = StateFrags<E, D, BV>;
    constexpr int VEC = E::VEC, KF = E::KF, NCT = BV / 16, NKC = F::NKC, RPW = F::RPW;
    const int l16 = lane & 15, lg = lane >> 4;
    F cur;
    if (count > 0) load_state<E, D, BV>(cur, a, chunk_pos(0, first, tok0, tok1), g, ws, l16, lg);
    wait_vmem_all();
    __syncthreads();
    for (int c = 0; c < count; ++c) {
        const int buf = c & 1;
        const int cn = c + 1 < count ? c + 1 : c;
        F nxt;
        load_state<E, D, BV>(nxt, a, chunk_pos(cn, first, tok0, tok1), g, ws, l16, lg);
        const float decay = __expf(__int_as_float(__builtin_amdgcn_readlane(__float_as_int(cur.gc), CH - 1)));
        __syncthreads();
        // step 2: S = e^{gc_last} S + kt v_new, each v_new fragment read once for all row tiles
        f32x4 acc[RPW][NCT];
#pragma unroll
        for (int ri = 0; ri < RPW; ++ri)
#pragma unroll
            for (int ct = 0; ct < NCT; ++ct) acc[ri][ct] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kf = 0; kf < NKC; ++kf)
#pragma unroll
            for (int ct = 0; ct < NCT; ++ct) {
                const uint4 b = ld16(&sm.vnT[16 * ct + l16][kf * KF + VEC * lg]);
#pragma unroll
                for (int ri = 0; ri < RPW; ++ri)
                    if (ws + 4 * ri < D / 16) mma<E>(acc[ri][ct], cur.kt[ri][kf], b);
            }
#pragma unroll
        for (int ri = 0; ri < RPW; ++ri) {
            const int rt = ws + 4 * ri;
            if (rt < D / 16) {
#pragma unroll
                for (int ct = 0; ct < NCT; ++ct) {
                    f32x4 s = S[ri][ct];
#pragma unroll
                    for (int i = 0; i < 4; ++i) s[i] = decay * s[i] + acc[ri][ct][i];
                    S[ri][ct] = s;
                    store4<E>(&sm.sT[buf ^ 1][16 * ct + l16][16 * rt + 4 * lg], s[0], s[1], s[2], s[3]);
                }
            }
        }
        __syncthreads();
        cur = nxt;
    }
}

template <class E, int D, int BV, bool BO>
__global__ __launch_bounds__(NT_SCAN) void gdn_scan_kernel(GdnArgs a) {
    using SF = StateFrags<E, D, BV>;
    constexpr int NCT = BV / 16, NRT = D / 16, RPW = SF::RPW;
    __shared__ ScanShared<E, D, BV> sm;

    // XCD-aware mapping: workgroups are dispatched round-robin over the XCDs by linear id, and every column slab of
    // one (sequence, KV head) reads the same chunk operands, so all slabs of a group go to one XCD (one L2).
    const int xcd = blockIdx.x % kXcds, local = blockIdx.x / kXcds;
    const int nslab = D / BV;
    const int grp = xcd + kXcds * (local / nslab), jb = local % nslab;
    const int G = a.G;
    if (grp >= a.num_seqs * G) return;
    const int g = grp % G, n = grp / G;
    const int lane = lane_id(), wv = wave_id(), lg = lane >> 4, l16 = lane & 15;
    const int j0 = jb * BV;
    int first, count;
    long tok0, tok1;
    seq_chunks(n, a.cu_seqlens, a.seq_len, CH, first, count, tok0, tok1);

    if (wv < 4) {
        rows_loop<E, D, BV, BO>(sm, a, count, first, tok0, tok1, g, j0, wv, lane);
        return;
    }

    // state waves: the slab of S in registers, tile (rt = ws + 4*ri, ct) holds S[16rt + 4lg + i][j0 + 16ct + l16]
    const int ws = wv - 4;
    f32x4 S[RPW][NCT];
#pragma unroll
    for (int ri = 0; ri < RPW; ++ri)
#pragma unroll
        for (int ct = 0; ct < NCT; ++ct) {
            const int rt = ws + 4 * ri;
            f32x4 v = {0.f, 0.f, 0.f, 0.f};
            if (a.s0 && rt < NRT) {
                const float* p = a.s0 + (((long)n * G + g) * D + 16 * rt + 4 * lg) * D + j0 + 16 * ct + l16;
#pragma unroll
                for (int i = 0; i < 4; ++i) v[i] = p[(long)i * D];
            }
            S[ri][ct] = v;
            if (rt < NRT) store4<E>(&sm.sT[0][16 * ct + l16][16 * rt + 4 * lg], v[0], v[1], v[2], v[3]);
        }
    state_loop<E, D, BV>(sm, S, a, count, first, tok0, tok1, g, ws, lane);
    if (a.s_out) {
#pragma unroll
        for (int ri = 0; ri < RPW; ++ri)
#pragma unroll
            for (int ct = 0; ct < NCT; ++ct) {
                const int rt = ws + 4 * ri;
                if (rt >= NRT) continue;
                float* p = a.s_out + (((long)n * G + g) * D + 16 * rt + 4 * lg) * D + j0 + 16 * ct + l16;
#pragma unroll
                for (int i = 0; i < 4; ++i) p[(long)i * D] = S[ri][ct][i];
            }
    }
}

// ------------------------------------------------------------------------------------------------ host launchers
template <class E, int D, int BV>
static int launch_gdn(const GdnArgs& a, int phases, hipStream_t stream) {
    if (phases & GDN_PHASE_PREP) {
        hipLaunchKernelGGL((gdn_prep_kernel<E, D>), dim3(a.max_chunks, a.G), dim3(NT), 0, stream, a);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return (int)e;
    }
    if (phases & GDN_PHASE_SCAN) {
        const int groups = a.num_seqs * a.G;
        const dim3 grid(kXcds * ((groups + kXcds - 1) / kXcds) * (D / BV));
        if (a.o_dtype == DT_BF16) hipLaunchKernelGGL((gdn_scan_kernel<E, D, BV, true>), grid, dim3(NT_SCAN), 0, stream, a);
        else hipLaunchKernelGGL((gdn_scan_kernel<E, D, BV, false>), grid, dim3(NT_SCAN), 0, stream, a);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return (int)e;
    }
    return 0;
}

int gdn_dispatch(const GdnArgs& a, int phases, hipStream_t stream) {
    const bool bf = a.in_dtype == DT_BF16;
    switch (a.D) {
        case 64: return bf ? launch_gdn<BF16, 64, 16>(a, phases, stream) : launch_gdn<F32, 64, 16>(a, phases, stream);
        case 128: return bf ? launch_gdn<BF16, 128, 32>(a, phases, stream) : launch_gdn<F32, 128, 32>(a, phases, stream);
        case 256: return bf ? launch_gdn<BF16, 256, 32>(a, phases, stream) : launch_gdn<F32, 256, 32>(a, phases, stream);
        default: return BF_ERR_UNSUPPORTED;
    }
}

}  // namespace bf
