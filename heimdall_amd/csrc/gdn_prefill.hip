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
//   gdn_scan  grid (Dv / BV, G, sequences): the sequential pass. Columns of S are independent, so each workgroup
//             owns a BV-column slab of one KV head's state, keeps it in registers (fp32) for the whole sequence and
//             a bf16/fp32 copy in LDS as the MFMA B operand.
//
// Workspace (per chunk id cid, KV head g; C = 64):
//   gcum [cid][g][C] f32 | w [cid][g][C][D] E | uT [cid][g][D][C] f32 | kt [cid][g][D][C] E | attn [cid][h][C][C] E
#include "bf_common.h"
#include "bf_internal.h"

namespace bf {

constexpr int CH = 64;     // chunk length
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
template <class E, int D, int BV>
struct ScanShared {
    typename E::T sT[2][BV][D + E::VEC];   // S^T slab (double buffered): [column j][row d]
    typename E::T vnT[BV][CH + E::VEC];    // v_new^T slab: [column j][token t]
};

template <class E, int D, int BV>
__global__ __launch_bounds__(NT) void gdn_scan_kernel(GdnArgs a) {
    using T = typename E::T;
    constexpr int VEC = E::VEC, KF = E::KF;
    constexpr int NCT = BV / 16;          // column tiles of the slab
    constexpr int NRT = D / 16;           // row tiles of S
    constexpr int RPW = (NRT + 3) / 4;    // S row tiles per wave
    constexpr int NKD = D / KF;           // fragments along D
    constexpr int NKC = CH / KF;          // fragments along the chunk
    __shared__ ScanShared<E, D, BV> sm;

    const int jb = blockIdx.x, g = blockIdx.y, n = blockIdx.z;
    const int G = a.G, R = a.R, H = G * R;
    const int lane = lane_id(), wv = wave_id(), l16 = lane & 15, lg = lane >> 4;
    const int j0 = jb * BV;
    int first, count;
    long tok0, tok1;
    seq_chunks(n, a.cu_seqlens, a.seq_len, CH, first, count, tok0, tok1);

    // state slab in registers: tile (rt = wv + 4*ri, ct) holds S[16rt + 4lg + i][j0 + 16ct + l16]
    f32x4 S[RPW][NCT];
#pragma unroll
    for (int ri = 0; ri < RPW; ++ri)
#pragma unroll
        for (int ct = 0; ct < NCT; ++ct) {
            const int rt = wv + 4 * ri;
            f32x4 v = {0.f, 0.f, 0.f, 0.f};
            if (a.s0 && rt < NRT) {
                const float* p = a.s0 + (((long)n * G + g) * D + 16 * rt + 4 * lg) * D + j0 + 16 * ct + l16;
#pragma unroll
                for (int i = 0; i < 4; ++i) v[i] = p[(long)i * D];
            }
            S[ri][ct] = v;
            if (rt < NRT) store4<E>(&sm.sT[0][16 * ct + l16][16 * rt + 4 * lg], v[0], v[1], v[2], v[3]);
        }
    __syncthreads();

    const T* Wb = reinterpret_cast<const T*>(a.ws_w);
    const T* KTb = reinterpret_cast<const T*>(a.ws_kt);
    const T* ATb = reinterpret_cast<const T*>(a.ws_attn);
    const T* Qb = reinterpret_cast<const T*>(a.q);

    for (int c = 0; c < count; ++c) {
        const int cur = c & 1;
        const long cid = first + c;
        const long t0 = tok0 + (long)c * CH;
        const int len = (int)((tok1 - t0) < CH ? (tok1 - t0) : CH);
        const float* gcum = a.ws_gcum + (cid * G + g) * CH;

        // ---- step 1: v_new rows 16*wv.. = u - w S   (A = w rows, B = S^T)
        {
            const T* W = Wb + (cid * G + g) * CH * D + (long)(16 * wv + l16) * D;
            uint4 fw[NKD];
#pragma unroll
            for (int kf = 0; kf < NKD; ++kf) fw[kf] = ld16(W + kf * KF + VEC * lg);
            const float* UT = a.ws_uT + (cid * G + g) * D * CH;
#pragma unroll
            for (int ct = 0; ct < NCT; ++ct) {
                f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int kf = 0; kf < NKD; ++kf) mma<E>(acc, fw[kf], ld16(&sm.sT[cur][16 * ct + l16][kf * KF + VEC * lg]));
                const float4 u = *reinterpret_cast<const float4*>(UT + (long)(j0 + 16 * ct + l16) * CH + 16 * wv + 4 * lg);
                store4<E>(&sm.vnT[16 * ct + l16][16 * wv + 4 * lg], u.x - acc[0], u.y - acc[1], u.z - acc[2],
                          u.w - acc[3]);
            }
        }
        __syncthreads();

        // ---- step 2: S = e^{gc_last} S + kt v_new   (A = kt rows d, B = v_new^T) -> next S^T buffer
        {
            const float decay = __expf(gcum[CH - 1]);
            const T* KT = KTb + (cid * G + g) * D * CH;
#pragma unroll
            for (int ri = 0; ri < RPW; ++ri) {
                const int rt = wv + 4 * ri;
                if (rt >= NRT) break;
                uint4 fk[NKC];
#pragma unroll
                for (int kf = 0; kf < NKC; ++kf) fk[kf] = ld16(KT + (long)(16 * rt + l16) * CH + kf * KF + VEC * lg);
#pragma unroll
                for (int ct = 0; ct < NCT; ++ct) {
                    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                    for (int kf = 0; kf < NKC; ++kf) mma<E>(acc, fk[kf], ld16(&sm.vnT[16 * ct + l16][kf * KF + VEC * lg]));
                    f32x4 s = S[ri][ct];
#pragma unroll
                    for (int i = 0; i < 4; ++i) s[i] = decay * s[i] + acc[i];
                    S[ri][ct] = s;
                    store4<E>(&sm.sT[cur ^ 1][16 * ct + l16][16 * rt + 4 * lg], s[0], s[1], s[2], s[3]);
                }
            }
        }

        // ---- step 3: outputs rows 16*wv..: o_r = scale e^{gc} q_r S_old + attn_r v_new
        {
            const int t = 16 * wv + l16;                 // A-fragment row of this lane
            const float qs = a.scale * __expf(gcum[t]);
            for (int r = 0; r < R; ++r) {
                const int h = g * R + r;
                const T* Q = Qb + (t0 + t) * (long)H * D + (long)h * D;
                uint4 fq[NKD];
#pragma unroll
                for (int kf = 0; kf < NKD; ++kf) fq[kf] = t < len ? scale16<E>(ld16(Q + kf * KF + VEC * lg), qs) : zero16();
                const T* AT = ATb + ((cid * H + h) * CH + t) * CH;
                uint4 fa[NKC];
#pragma unroll
                for (int kf = 0; kf < NKC; ++kf) fa[kf] = ld16(AT + kf * KF + VEC * lg);
#pragma unroll
                for (int ct = 0; ct < NCT; ++ct) {
                    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                    for (int kf = 0; kf < NKD; ++kf) mma<E>(acc, fq[kf], ld16(&sm.sT[cur][16 * ct + l16][kf * KF + VEC * lg]));
#pragma unroll
                    for (int kf = 0; kf < NKC; ++kf) mma<E>(acc, fa[kf], ld16(&sm.vnT[16 * ct + l16][kf * KF + VEC * lg]));
                    const int j = j0 + 16 * ct + l16;
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const int tr = 16 * wv + 4 * lg + i;
                        if (tr < len) {
                            const long off = (t0 + tr) * (long)H * D + (long)h * D + j;
                            if (a.o_dtype == DT_F32) reinterpret_cast<float*>(a.o)[off] = acc[i];
                            else reinterpret_cast<uint16_t*>(a.o)[off] = f2bf(acc[i]);
                        }
                    }
                }
            }
        }
        __syncthreads();
    }

    if (a.s_out) {
#pragma unroll
        for (int ri = 0; ri < RPW; ++ri)
#pragma unroll
            for (int ct = 0; ct < NCT; ++ct) {
                const int rt = wv + 4 * ri;
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
        hipLaunchKernelGGL((gdn_scan_kernel<E, D, BV>), dim3(D / BV, a.G, a.num_seqs), dim3(NT), 0, stream, a);
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
