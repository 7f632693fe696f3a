// K1 part 1: per-chunk preparation of the chunked gated delta rule (GQA form, packed varlen).
//
// Algorithm (UT/WY representation; reference: Heimdall/heimdall/kernels.py:94-129, motor.py:70-102). For a chunk of
// C = 64 tokens of KV head g with in-chunk cumulative log-decay gc:
//   A  = strict_lower(beta_i e^{gc_i - gc_j} k_i.k_j),   T' = (I + A)^-1 diag(beta)
// so that the reference's u - w S equals T' (V - e^{gc} K S): the scan (gdn_scan.hip) needs only T' and gc next to
// the inputs q, k, v (it forms the causal q K^T block of each query head itself), and nothing of size C x D is
// written back here.
//
// gdn_prep_kernel, grid G x chunks (head fastest), 4 waves: the K tile is staged in LDS (buffer_load ... lds); the waves compute A
// by MFMA; (I + A) is inverted in fp32 by 16 x 16 blocks (diagonal blocks by forward substitution, the rest by fp32
// MFMA block products, one block column per wave).
//
// Workspace written (chunk id cid, KV head g):
//   gcum [cid][g][C] f32 | T [cid][g][C*C] in_dtype in MFMA A-fragment order (tfrag_index), the layout the scan reads
#include "bf_common.h"
#include "bf_internal.h"

namespace bf {

constexpr int CH = 64;     // chunk length
constexpr int NT = 256;    // threads per workgroup (4 waves)

// LDS: the chunk's K tile (swizzled rows, staged by buffer_load ... lds) and A. The inverse's diagonal blocks X_bb are
// written over A's diagonal blocks once forward substitution has read them (the block products read A only below the
// diagonal), so no LDS is set aside for X: 34 KB at D = 128 (four workgroups per CU, three with a separate X; the
// prep phase of 4 packed sequences {8192, 16384, 24576, 16384}, H = 32, went from 279-307 to 236-269 us).
template <class E, int D>
struct __align__(16) PrepLds {
    typename E::T K[CH * D];
    float A[CH][CH + 4];
    float gc[CH];
    float beta[CH];
};

template <class E, int D>
__global__ __launch_bounds__(NT) void gdn_prep_kernel(GdnArgs a) {
    using T = typename E::T;
    constexpr int KF = E::KF, ES = (int)sizeof(T), ROWB = D * ES, NKD = D / KF;
    __shared__ PrepLds<E, D> sm;
    // 1D grid, KV head fastest: the G workgroups of one chunk are dispatched together, so the cache lines of g and
    // beta ([token][G], one line holds the values of all heads) are fetched from HBM once per XCD, not once per head
    const int G = a.G, g = (int)(blockIdx.x % G);
    const long cid = blockIdx.x / G;
    SeqInfo si;
    if (!locate_chunk(cid, a.cu_seqlens, a.num_seqs, a.seq_len, CH, si)) return;
    const int lane = lane_id(), wv = wave_id(), l16 = lane & 15, lg = lane >> 4;
    // LDS block permutation of the K tile: a fragment read covers 16 consecutive rows at one 16-byte block, so
    // the block is XORed with row & 15 (rows of >= 16 blocks) or (row >> 1) & 7 (8 blocks: two rows share a 256-byte
    // bank window), putting the 16 rows on 16 distinct bank groups.
    const auto sw_row = [](int row) { return ROWB / 16 >= 16 ? (row & 15) : ((row >> 1) & 7); };
    const int nw = NT / WAVE;

    const rsrc_t rk = make_rsrc(reinterpret_cast<const char*>(a.k) + (si.tok0 * G + g) * D * ES,
                                (uint32_t)((long)si.len * G * D * ES));
    stage_tile(rk, (uint32_t)(G * D * ES), ROWB, sm.K, CH * ROWB, wv, nw, lane, sw_row, 1 << 30);
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
    wait_vmem_all();
    __syncthreads();

    // fragment of rows 16*tile + l16 of a swizzled tile, K index KF*ks + VEC*lg .. (16 bytes)
    auto frag = [&](const T* base, int tile, int ks) {
        const int row = 16 * tile + l16;
        return lds16(base, row * ROWB + (((4 * ks + lg) ^ sw_row(row)) << 4));
    };

    // A = strict_lower(beta_r e^{gc_r - gc_c} (K K^T)_{rc}). K K^T is symmetric: tile (rt, ct) with rt <= ct read
    // in transposed form fills rows 16ct.., columns 16rt.. of A.
    for (int tix = wv; tix < 10; tix += nw) {
        const int rt = tix < 4 ? 0 : tix < 7 ? 1 : tix < 9 ? 2 : 3;
        const int ct = rt + (tix - (rt == 0 ? 0 : rt == 1 ? 4 : rt == 2 ? 7 : 9));
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < NKD; ++ks) mma<E>(acc, frag(sm.K, rt, ks), frag(sm.K, ct, ks));
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

    // (I + A)^-1, blocked over 16 x 16 blocks (L = I + A unit lower triangular, X = L^-1):
    //   X_bb = L_bb^-1 for the 4 diagonal blocks: forward substitution, one column per lane (wave 0, lane 16 b + c),
    //   written over A's diagonal block b after all of its reads (one wave: its LDS accesses run in order);
    //   X_ij = -X_ii sum_{k=j}^{i-1} A_ik X_kj for i > j: wave j walks i = j+1 .. 3 with fp32 MFMAs; every 16 x 16
    //   accumulator (lane: column l16, rows 4 lg ..) is already laid out as the B operand of the next product.
    // T'[i][j] = X[i][j] beta_j (rows of tokens past the end are zero because their A rows and beta are).
    float (*X)[CH + 4] = sm.A;
    if (wv == 0) {
        const int bb = lane >> 4, c = lane & 15, o = 16 * bb;
        float x[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            float acc = i == c ? 1.f : 0.f;
#pragma unroll
            for (int m = 0; m < i; ++m) acc -= sm.A[o + i][o + m] * x[m];
            x[i] = acc;
        }
#pragma unroll
        for (int i = 0; i < 16; ++i) X[o + i][o + c] = x[i];
    }
    __syncthreads();
    {
        const int j = wv;                                  // block column of this wave
        T* Tg = reinterpret_cast<T*>(a.ws_T) + (cid * G + g) * CH * CH;
        const float bj = sm.beta[16 * j + l16];
        auto put = [&](int i, const f32x4& v) {            // block (i, j) of T' from an accumulator tile
#pragma unroll
            for (int e = 0; e < 4; ++e) Tg[tfrag_index<E>(16 * i + 4 * lg + e, 16 * j + l16)] = E::from_f(v[e] * bj);
        };
        // A fragment of a 16 x 16 fp32 block of an LDS matrix M (rows r0.., columns c0..): lane row l16, k = 4 lg ..
        auto afrag = [&](const float (*M)[CH + 4], int r0, int c0) {
            const float4 v = *reinterpret_cast<const float4*>(&M[r0 + l16][c0 + 4 * lg]);
            return make_uint4(__float_as_uint(v.x), __float_as_uint(v.y), __float_as_uint(v.z), __float_as_uint(v.w));
        };
        auto bfrag = [](const f32x4& v) {
            return make_uint4(__float_as_uint(v[0]), __float_as_uint(v[1]), __float_as_uint(v[2]), __float_as_uint(v[3]));
        };
        f32x4 xc[4];                                       // X_kj, k = j .. 3, as accumulator tiles
#pragma unroll
        for (int e = 0; e < 4; ++e) xc[j][e] = X[16 * j + 4 * lg + e][16 * j + l16];
        put(j, xc[j]);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            if (i <= j) {
                if (i < j) put(i, f32x4{0.f, 0.f, 0.f, 0.f});   // above the diagonal
                continue;
            }
            f32x4 msum = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int k = 0; k < 4; ++k)
                if (k >= j && k < i) mma<F32>(msum, afrag(sm.A, 16 * i, 16 * k), bfrag(xc[k]));
            f32x4 xi = {0.f, 0.f, 0.f, 0.f};
            mma<F32>(xi, afrag(X, 16 * i, 16 * i), bfrag(msum));
#pragma unroll
            for (int e = 0; e < 4; ++e) xi[e] = -xi[e];
            xc[i] = xi;
            put(i, xi);
        }
    }
}

template <class E, int D>
static int launch_prep(const GdnArgs& a, hipStream_t stream) {
    hipLaunchKernelGGL((gdn_prep_kernel<E, D>), dim3((unsigned)((long)a.G * a.max_chunks)), dim3(NT), 0, stream, a);
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
