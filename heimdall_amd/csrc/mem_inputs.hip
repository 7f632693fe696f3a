// Memory-branch read/write keys of the converted layer (reference: HybridAttention._mem_inputs,
// Heimdall/heimdall/hibrit.py:327-334):
//   y_{t,h} = scale * normalize(x_{t,h} F_h),   normalize(u) = u / max(||u||_2, 1e-12)
// used for qm (x = q, F = fq, scale = D^-1/2) and km (x = k, F = fk, scale = 1), for bf16 activations.
//
// One workgroup owns one head h and a strided set of 64-token tiles (one round of workgroups over the CUs). F_h^T
// (D x D bf16, 128 KB at D = 256) is staged in LDS once; each of the 4 waves computes 16 tokens x D outputs per tile
// as Y^T = F_h^T X^T with v_mfma_f32_16x16x32_bf16 (A = rows of F_h^T from LDS, read 8 MFMAs ahead; B = the token
// rows of x from global memory, loaded two tiles ahead), so every lane holds 4 consecutive outputs of one token: the
// row norm is a sum over the lane's values and two cross-lane steps, and the bf16 result is stored 8 bytes at a
// time. The pass reads x and writes y once (806 MB at T = 32768, 24 heads, D = 256).
#include "bf_common.h"
#include "bf_internal.h"

namespace bf {

namespace {

constexpr int MP_WAVES = 4;
constexpr int MP_TILE = 16 * MP_WAVES;       // tokens per tile
constexpr int MP_AHEAD = 8;                  // A fragment reads in flight ahead of their MFMAs

template <int NBLK>
__device__ __forceinline__ int mp_sw(int row) { return NBLK >= 16 ? (row & 15) : ((row >> 1) & 7); }

}  // namespace

template <int D>
__global__ __launch_bounds__(64 * MP_WAVES, 1) void mem_project_kernel(MemProjArgs a) {
    constexpr int ROWB = D * 2, NBLK = ROWB / 16;
    constexpr int NKD = D / 32, NDT = D / 16;
    constexpr int NKB = NKD < 4 ? NKD : 4;
    __shared__ __align__(16) uint16_t ft[D * D];

    const int h = blockIdx.x % a.nh, tg = blockIdx.x / a.nh, ntg = gridDim.x / a.nh;
    const int lane = lane_id(), wv = wave_id(), l16 = lane & 15, lg = lane >> 4;

    // stage F_h^T: LDS row j holds row j of F_h^T with its 16-byte blocks permuted by mp_sw(j)
    const rsrc_t rf = make_rsrc(reinterpret_cast<const uint16_t*>(a.ft) + (long)h * D * D, (uint32_t)(D * ROWB));
    stage_tile(rf, (uint32_t)ROWB, ROWB, ft, D * ROWB, wv, MP_WAVES, lane, [](int row) { return mp_sw<NBLK>(row); },
               NBLK);

    int abase[NKB];
    {
        const int s = mp_sw<NBLK>(l16);
#pragma unroll
        for (int c = 0; c < NKB; ++c) abase[c] = l16 * ROWB + 64 * (c ^ (s >> 2)) + 16 * (lg ^ (s & 3));
    }
    const char* Fb = reinterpret_cast<const char*>(ft);
    const uint16_t* X = reinterpret_cast<const uint16_t*>(a.x) + (long)h * a.x_sh;
    uint16_t* Out = reinterpret_cast<uint16_t*>(a.out);

    const long ntiles = (a.n_tok + MP_TILE - 1) / MP_TILE;
    // B fragments of token 16 wv + l16 of tile t: x[token][32 ks + 8 lg .. +7]
    auto load_x = [&](long t, uint4 (&xf)[NKD]) {
        const rsrc_t rx = make_rsrc(X + (t * MP_TILE + 16 * wv) * a.x_st,
                                    t < ntiles ? (uint32_t)(max(0L, min((long)16, a.n_tok - (t * MP_TILE + 16 * wv))) *
                                                            a.x_st * 2) : 0u);
#pragma unroll
        for (int ks = 0; ks < NKD; ++ks)
            xf[ks] = buf_ld16(rx, (uint32_t)((l16 * a.x_st + 32 * ks + 8 * lg) * 2));
    };
    // x is read two tiles ahead of its use (the pass streams x in and out once; more bytes in flight per CU)
    uint4 xf[NKD], x1[NKD];
    load_x(tg, xf);
    load_x(tg + ntg, x1);
    wait_vmem_all();
    __syncthreads();

    for (long t = tg; t < ntiles; t += ntg) {
        uint4 x2[NKD];
        load_x(t + 2 * ntg, x2);                    // out of range: reads zero
        f32x4 acc[NDT];
#pragma unroll
        for (int jt = 0; jt < NDT; ++jt) acc[jt] = f32x4{0.f, 0.f, 0.f, 0.f};
        // the NKD x NDT products in one sequence (k step outer, so consecutive MFMAs use distinct accumulators),
        // each A fragment read MP_AHEAD products ahead of its MFMA so LDS latency overlaps the MFMAs
        constexpr int NP = NKD * NDT;
        auto read_a = [&](int i) {
            const int ks = i / NDT, jt = i % NDT;
            return lds16(Fb, abase[ks % NKB] + 16 * jt * ROWB + 256 * (ks / NKB));
        };
        uint4 af[MP_AHEAD];
#pragma unroll
        for (int i = 0; i < MP_AHEAD; ++i) af[i] = read_a(i);
#pragma unroll
        for (int i = 0; i < NP; ++i) {
            const uint4 a_i = af[i % MP_AHEAD];
            if (i + MP_AHEAD < NP) af[i % MP_AHEAD] = read_a(i + MP_AHEAD);
            mma<BF16>(acc[i % NDT], a_i, xf[i / NDT]);
            __builtin_amdgcn_sched_barrier(0);       // keeps the reads in their slots (no hoisting of all 128)
        }
        float ss = 0.f;
#pragma unroll
        for (int jt = 0; jt < NDT; ++jt)
#pragma unroll
            for (int i = 0; i < 4; ++i) ss += acc[jt][i] * acc[jt][i];
        ss += __shfl_xor(ss, 16);
        ss += __shfl_xor(ss, 32);
        const float inv = a.scale / fmaxf(sqrtf(ss), 1e-12f);
        const long tok = t * MP_TILE + 16 * wv + l16;
        if (tok < a.n_tok) {
            uint16_t* orow = Out + (tok * a.nh + h) * D;
#pragma unroll
            for (int jt = 0; jt < NDT; ++jt) {
                uint2 v;
                v.x = pack_bf16x2(acc[jt][0] * inv, acc[jt][1] * inv);
                v.y = pack_bf16x2(acc[jt][2] * inv, acc[jt][3] * inv);
                *reinterpret_cast<uint2*>(orow + 16 * jt + 4 * lg) = v;
            }
        }
#pragma unroll
        for (int ks = 0; ks < NKD; ++ks) {
            xf[ks] = x1[ks];
            x1[ks] = x2[ks];
        }
    }
}

int mem_project_dispatch(const MemProjArgs& a, hipStream_t stream) {
    const long ntiles = (a.n_tok + MP_TILE - 1) / MP_TILE;
    // one round of workgroups over the 256 CUs (F_h^T takes D * D * 2 bytes of LDS per workgroup)
    const long per_cu = (long)(160 * 1024) / ((long)a.D * a.D * 2);
    const long want = (256 * (per_cu > 0 ? per_cu : 1)) / a.nh;
    const int ntg = (int)(ntiles < want ? ntiles : (want > 0 ? want : 1));
    const dim3 grid((unsigned)(a.nh * (ntg > 0 ? ntg : 1))), block(64 * MP_WAVES);
    switch (a.D) {
        case 64: hipLaunchKernelGGL(mem_project_kernel<64>, grid, block, 0, stream, a); break;
        case 128: hipLaunchKernelGGL(mem_project_kernel<128>, grid, block, 0, stream, a); break;
        case 256: hipLaunchKernelGGL(mem_project_kernel<256>, grid, block, 0, stream, a); break;
        default: return BF_ERR_UNSUPPORTED;
    }
    return (int)hipGetLastError();
}

// Gates of the memory branch (reference: HybridAttention._mem_inputs, Heimdall/heimdall/hibrit.py:331-333), one
// thread per (token, KV head): g = -exp(A_log) softplus(a + dt_bias) decay_mask, beta = sigmoid(b) [pos >= sinks].
__global__ __launch_bounds__(256) void mem_gates_kernel(MemGatesArgs a) {
    const long e = (long)blockIdx.x * 256 + threadIdx.x;
    if (e >= a.n_tok * a.G) return;
    const long t = e / a.G;
    const int j = (int)(e % a.G);
    const float* row = a.ab + t * a.ab_st;
    const float x = row[j] + a.dt_bias[j];
    const float sp = x > 20.f ? x : log1pf(expf(x));            // softplus, torch's default threshold
    a.g[e] = -expf(a.A_log[j]) * sp * a.decay_mask[j];
    const long pos = a.start + t % a.T;
    a.beta[e] = pos >= a.sinks ? 1.f / (1.f + expf(-row[a.G + j])) : 0.f;
}

int mem_gates_dispatch(const MemGatesArgs& a, hipStream_t stream) {
    const long n = a.n_tok * a.G;
    hipLaunchKernelGGL(mem_gates_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, a);
    return (int)hipGetLastError();
}

}  // namespace bf
