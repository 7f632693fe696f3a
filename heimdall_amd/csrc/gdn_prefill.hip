// K1 part 1: per-chunk preparation of the chunked gated delta rule (GQA form, packed varlen).
//
// Algorithm (UT/WY representation; reference: Heimdall/heimdall/kernels.py:94-129, motor.py:70-102). For a chunk of
// C = 64 tokens of KV head g with in-chunk cumulative log-decay gc:
//   A  = strict_lower(beta_i e^{gc_i - gc_j} k_i.k_j),   T' = (I + A)^-1 diag(beta)
//   attn_r = scale (q_r K^T * e^{gc_i - gc_j})[i >= j]           for the R query heads of the group
// so that the reference's u - w S equals T' (V - e^{gc} K S): the scan (gdn_scan.hip) needs only T', attn and gc
// next to the inputs q, k, v, and nothing of size C x D is written back here.
//
// gdn_prep_kernel, grid (chunks, G), 4 waves: wave 0 forms gc, then everybody computes A by MFMA; wave 0 inverts
// (I + A) by forward substitution (one column per lane, fp32) while waves 1-3 compute the R attn tiles.
//
// Workspace written (chunk id cid, KV head g, query head h):
//   gcum [cid][g][C] f32 | T [cid][g][C][C] in_dtype | attn [cid][h][C][C] in_dtype
#include "bf_common.h"
#include "bf_internal.h"

namespace bf {

constexpr int CH = 64;     // chunk length
constexpr int NT = 256;    // threads per workgroup (4 waves)

struct PrepShared {
    float A[CH][CH + 4];   // strictly lower A (fp32)
    float gc[CH];
    float beta[CH];
};

template <class E, int D>
__global__ __launch_bounds__(NT) void gdn_prep_kernel(GdnArgs a) {
    using T = typename E::T;
    constexpr int VEC = E::VEC, KF = E::KF;
    __shared__ PrepShared sm;
    SeqInfo si;
    if (!locate_chunk(blockIdx.x, a.cu_seqlens, a.num_seqs, a.seq_len, CH, si)) return;
    const int g = blockIdx.y, G = a.G, R = a.R, H = G * R;
    const long cid = blockIdx.x;
    const int lane = lane_id(), wv = wave_id(), l16 = lane & 15, lg = lane >> 4;
    const T* K = reinterpret_cast<const T*>(a.k) + si.tok0 * G * D + (long)g * D;
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
        // (I + A)^-1 by forward substitution, one column per lane: x_i = [i == j] - sum_{m < i} A[i][m] x_m;
        // T'[i][j] = x_i beta_j (rows of tokens past the end are zero because their A rows and beta are).
        const int j = lane;
        float x[CH];
#pragma unroll
        for (int i = 0; i < CH; ++i) {
            float acc = i == j ? 1.f : 0.f;
#pragma unroll
            for (int m = 0; m < i; ++m) acc -= sm.A[i][m] * x[m];
            x[i] = acc;
        }
        const float bj = sm.beta[j];
        T* Tp = reinterpret_cast<T*>(a.ws_T) + (cid * G + g) * CH * CH + j;
#pragma unroll
        for (int i = 0; i < CH; ++i) Tp[i * CH] = E::from_f(x[i] * bj);
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
}

template <class E, int D>
static int launch_prep(const GdnArgs& a, hipStream_t stream) {
    hipLaunchKernelGGL((gdn_prep_kernel<E, D>), dim3(a.max_chunks, a.G), dim3(NT), 0, stream, a);
    return (int)hipGetLastError();
}

int gdn_prep(const GdnArgs& a, hipStream_t stream) {
    const bool bf = a.in_dtype == DT_BF16;
    switch (a.D) {
        case 64: return bf ? launch_prep<BF16, 64>(a, stream) : launch_prep<F32, 64>(a, stream);
        case 128: return bf ? launch_prep<BF16, 128>(a, stream) : launch_prep<F32, 128>(a, stream);
        case 256: return bf ? launch_prep<BF16, 256>(a, stream) : launch_prep<F32, 256>(a, stream);
        default: return BF_ERR_UNSUPPORTED;
    }
}

}  // namespace bf
