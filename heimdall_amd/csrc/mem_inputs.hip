// Memory-branch read/write keys of the converted layer (reference: HybridAttention._mem_inputs,
// Heimdall/heimdall/hibrit.py:327-334):
//   y_{t,h} = scale * normalize(x_{t,h} F_h),   normalize(u) = u / max(||u||_2, 1e-12)
// used for qm (x = q, F = fq, scale = D^-1/2) and km (x = k, F = fk, scale = 1), for bf16 activations.
//
// One workgroup owns one head h and a strided set of 64-token tiles (one round of workgroups over the CUs). F_h^T
// (D x D bf16, 128 KB at D = 256) is built in LDS once from the module's fp32 F_h (each thread assembles one 16-byte
// row block of F_h^T from 8 loads down a column of F_h, coalesced across lanes, rounded to bf16 to nearest even);
// each of the 4 waves computes 16 tokens x D outputs per tile
// as Y^T = F_h^T X^T with v_mfma_f32_16x16x32_bf16 (A = rows of F_h^T from LDS, read 8 MFMAs ahead; B = the token
// rows of x from global memory, loaded two tiles ahead), so every lane holds 4 consecutive outputs of one token: the
// row norm is a sum over the lane's values and two cross-lane steps. bf16 results go through a per-wave LDS
// buffer so that every store writes whole output rows (512 bytes at D = 256; stored straight from the fragments,
// 32-byte pieces of 16 rows per instruction, the qm pass took 240 us instead of 180); fp32 results are stored
// 16 bytes per lane from the fragments. The pass reads x and writes y once (806 MB at T = 32768, 24 heads,
// D = 256, bf16 out).
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
    // each wave's 16 output rows (bf16), 16-byte blocks permuted by the row (r & 15), for whole-row stores
    __shared__ __align__(16) uint16_t ot[MP_WAVES][16 * D];

    const int h = blockIdx.x % a.nh, tg = blockIdx.x / a.nh, ntg = gridDim.x / a.nh;
    const int lane = lane_id(), wv = wave_id(), l16 = lane & 15, lg = lane >> 4;

    // F_h^T into LDS: row j holds column j of F_h in bf16, its 16-byte blocks permuted by mp_sw(j). Block c of row j
    // (elements F_h[8 c .. 8 c + 7][j]) is one thread's: consecutive threads take consecutive j, so each of the 8 loads
    // reads 4 bytes per lane from one row of F_h, contiguous across the lanes.
    {
        const float* F = a.f + (long)h * D * D;
        constexpr int NB = D * D / 8, UN = NB / (64 * MP_WAVES) < 4 ? NB / (64 * MP_WAVES) : 4;
        static_assert(NB % (64 * MP_WAVES * UN) == 0, "F staging split");
        for (int i0 = threadIdx.x; i0 < NB; i0 += 64 * MP_WAVES * UN) {
            float v[UN][8];
#pragma unroll
            for (int u = 0; u < UN; ++u) {
                const int idx = i0 + u * 64 * MP_WAVES, j = idx % D, c = idx / D;
#pragma unroll
                for (int e = 0; e < 8; ++e) v[u][e] = F[(long)(8 * c + e) * D + j];
            }
#pragma unroll
            for (int u = 0; u < UN; ++u) {
                const int idx = i0 + u * 64 * MP_WAVES, j = idx % D, c = idx / D;
                st16(reinterpret_cast<char*>(ft) + j * ROWB + 16 * (c ^ mp_sw<NBLK>(j)),
                     make_uint4(pack_bf16x2(v[u][0], v[u][1]), pack_bf16x2(v[u][2], v[u][3]),
                                pack_bf16x2(v[u][4], v[u][5]), pack_bf16x2(v[u][6], v[u][7])));
            }
        }
    }

    int abase[NKB];
    {
        const int s = mp_sw<NBLK>(l16);
#pragma unroll
        for (int c = 0; c < NKB; ++c) abase[c] = l16 * ROWB + 64 * (c ^ (s >> 2)) + 16 * (lg ^ (s & 3));
    }
    const char* Fb = reinterpret_cast<const char*>(ft);
    const uint16_t* X = reinterpret_cast<const uint16_t*>(a.x) + (long)h * a.x_sh;

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
            if (a.out_dtype == DT_BF16) {
            } else {
                float* orow = reinterpret_cast<float*>(a.out) + (tok * a.nh + h) * D;
#pragma unroll
                for (int jt = 0; jt < NDT; ++jt)
                    *reinterpret_cast<float4*>(orow + 16 * jt + 4 * lg) =
                        make_float4(acc[jt][0] * inv, acc[jt][1] * inv, acc[jt][2] * inv, acc[jt][3] * inv);
            }
        }
        if (a.out_dtype == DT_BF16) {
            char* ow = reinterpret_cast<char*>(ot[wv]);
            constexpr int RB = D * 2, NB = RB / 16;
#pragma unroll
            for (int jt = 0; jt < NDT; ++jt) {
                uint2 v;
                v.x = pack_bf16x2(acc[jt][0] * inv, acc[jt][1] * inv);
                v.y = pack_bf16x2(acc[jt][2] * inv, acc[jt][3] * inv);
                const int blk = (2 * jt + (lg >> 1)) ^ (l16 & 15 & (NB - 1));
                *reinterpret_cast<uint2*>(ow + l16 * RB + 16 * blk + 8 * (lg & 1)) = v;
            }
            constexpr int RPI = 64 / NB;                     // rows per 64-lane pass
#pragma unroll
            for (int p = 0; p < 16 / RPI; ++p) {
                const int r = p * RPI + lane / NB, bk = lane % NB;
                const long tk = t * MP_TILE + 16 * wv + r;
                const uint4 v = *reinterpret_cast<const uint4*>(ow + r * RB + 16 * (bk ^ (r & 15 & (NB - 1))));
                if (tk < a.n_tok)
                    *reinterpret_cast<uint4*>(reinterpret_cast<uint16_t*>(a.out) + (tk * a.nh + h) * D + 8 * bk) = v;
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
    const long per_cu = (long)(160 * 1024) / ((long)a.D * a.D * 2 + (long)MP_WAVES * 16 * a.D * 2);
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
    const long pos = (a.pos_arr ? a.pos_arr[t / a.T] : a.start) + t % a.T;
    a.beta[e] = pos >= a.sinks ? 1.f / (1.f + expf(-row[a.G + j])) : 0.f;
}

int mem_gates_dispatch(const MemGatesArgs& a, hipStream_t stream) {
    const long n = a.n_tok * a.G;
    hipLaunchKernelGGL(mem_gates_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, a);
    return (int)hipGetLastError();
}

// Gate projections of the converted layer for bf16 activations (reference: HybridAttention._mem_inputs' ab(x),
// Heimdall/heimdall/hibrit.py:330, and the gamma logit mix(x), :409): y = x W^T + b for the two small Linear layers
// at once, out0 = x W0^T + b0 ([n_tok][n0], the ab columns [a | b]) and out1 = x W1^T + b1 ([n_tok][n1], mix), fp32.
//
// d is walked in 128-wide sub-steps with v_mfma_f32_16x16x32_bf16: A = the tokens' x rows (bf16, exact), B = W^T split
// into bf16 high and low parts (W = hi + lo + r, |r| <= 2^-18 |W|), so the sum over d is the fp32 product to ~4e-6
// relative, without a cast of x to fp32 in HBM. Within a sub-step lane group lg takes the 32 consecutive elements
// 32 lg .. + 31 (four 16-byte loads: each row read as whole 256-byte pieces) and MFMA j sums elements 8 j .. + 7 of
// each group, the same permutation of d on both operands.
//
// Above GP_SPLIT_MAX_TOK tokens: gate_split_w_kernel first writes W^T, split, into the workspace in B-fragment order
// (1 KB per fragment). gate_project_kernel then runs 4 waves x 16 tokens per workgroup, two workgroups per CU. Each
// step (SUB sub-steps) copies its fragments from L2 into LDS by DMA (buffer_load ... lds, no registers, no VALU work),
// double-buffered with one barrier per step, while the x rows of the next step load. Two independent workgroups per
// CU and 256-wide steps keep the x stream going across the barriers: 89 us at 32768 tokens, d = 5120, 32 outputs,
// against 113 us for 8-wave workgroups that split their 128-wide W tile on the VALU each step (100 us with the
// split W, 8 waves and 256-wide steps; 92 us with 4 waves and 128-wide steps; streaming x loads 135 us). The bits are
// the same: the products are added in the same order. Bound by reading x once: 2 d bytes per token.
constexpr int GP_WAVES = 4;
constexpr int GP_FRAG = 64 * 16;                               // bytes of one B fragment

// W^T of both projections split into bf16 high and low parts, in the B-fragment order of gate_project_kernel's LDS
// tile: sub-step s (elements 128 s .. 128 s + 127 of d), then fragment (nt * 4 + j) * 2 + hl (output tile nt, MFMA j,
// high / low part) of 64 lanes x 16 bytes. Thread (s, r, c) splits elements 8 c .. 8 c + 7 of sub-step s of output
// row r (zero past d and past n0 + n1 rows); lane 16 (c / 4) + r % 16 of fragment (r / 16 * 4 + c % 4) holds them.
__global__ __launch_bounds__(256) void gate_split_w_kernel(GateProjArgs a, char* ws, int nsub) {
    const int nout = a.n0 + a.n1, ntu = (nout + 15) / 16, rows = 16 * ntu;
    const long e = (long)blockIdx.x * 256 + threadIdx.x;
    if (e >= (long)nsub * rows * 16) return;
    const int c = (int)(e & 15), r = (int)((e >> 4) % rows), s = (int)((e >> 4) / rows);
    const int k = 128 * s + 8 * c;
    const float* src = r < a.n0 ? a.w0 + (long)r * a.d : (r < nout ? a.w1 + (long)(r - a.n0) * a.d : nullptr);
    float w[8];
    if (src && k < a.d) {                                      // d is a multiple of 8: the 8 floats are in the row
        const float4 u = *reinterpret_cast<const float4*>(src + k), v = *reinterpret_cast<const float4*>(src + k + 4);
        w[0] = u.x; w[1] = u.y; w[2] = u.z; w[3] = u.w; w[4] = v.x; w[5] = v.y; w[6] = v.z; w[7] = v.w;
    } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) w[i] = 0.f;
    }
    uint32_t hi[4], lo[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        hi[i] = pack_bf16x2(w[2 * i], w[2 * i + 1]);
        lo[i] = pack_bf16x2(w[2 * i] - __uint_as_float(hi[i] << 16),
                            w[2 * i + 1] - __uint_as_float(hi[i] & 0xffff0000u));
    }
    const int ln = 16 * (c >> 2) + (r & 15);
    char* f = ws + ((long)s * ntu * 8 + ((r >> 4) * 4 + (c & 3)) * 2) * GP_FRAG + 16 * ln;
    st16(f, make_uint4(hi[0], hi[1], hi[2], hi[3]));
    st16(f + GP_FRAG, make_uint4(lo[0], lo[1], lo[2], lo[3]));
}

// MAXT: output tiles of 16 columns the LDS tile holds (n0 + n1 <= 16 MAXT); SUB: 128-wide sub-steps per step. ws:
// the split W^T of gate_split_w_kernel, at least SUB * ceil(d / (128 SUB)) sub-steps.
template <int MAXT, int SUB>
__global__ __launch_bounds__(64 * GP_WAVES) void gate_project_kernel(GateProjArgs a, const char* ws) {
    constexpr int TILE = SUB * MAXT * 4 * 2 * GP_FRAG;        // (sub-step, nt, j, hi / lo) fragments of one step
    constexpr int KSTEP = 128 * SUB;
    __shared__ __align__(16) char wt[2][TILE];
    const int lane = lane_id(), wv = wave_id(), l16 = lane & 15, lg = lane >> 4;
    const long tok0 = ((long)blockIdx.x * GP_WAVES + wv) * 16;
    const int nout = a.n0 + a.n1, nt_used = (nout + 15) / 16, nfr = nt_used * 8;
    const int nstep = (a.d + KSTEP - 1) / KSTEP;
    const long tok = tok0 + l16;
    const bool tok_ok = tok < a.n_tok;
    const uint16_t* xrow = a.x + (tok_ok ? tok : 0) * a.x_st + 32 * lg;
    const rsrc_t wsrc = make_rsrc(ws, (uint32_t)(nstep * SUB * nfr * GP_FRAG));
    f32x4 acc[MAXT];
#pragma unroll
    for (int nt = 0; nt < MAXT; ++nt) acc[nt] = f32x4{0.f, 0.f, 0.f, 0.f};

    // the step's SUB * nfr fragments (contiguous in ws) into LDS: fragment f of sub-step h at (h * MAXT * 8 + f) KB
    auto dma_w = [&](int st, char* t) {
        for (int i = wv; i < SUB * nfr; i += GP_WAVES) {
            const int h = i / nfr, f = i % nfr;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                wsrc, (__attribute__((address_space(3))) void*)(t + (h * MAXT * 8 + f) * GP_FRAG), 16,
                (uint32_t)(((st * SUB + h) * nfr + f) * GP_FRAG + 16 * lane), 0, 0, 0);
        }
    };
    auto load_x = [&](int k0, uint4 (&xa)[4 * SUB]) {
#pragma unroll
        for (int h = 0; h < SUB; ++h)
#pragma unroll
            for (int j = 0; j < 4; ++j)
                xa[4 * h + j] = tok_ok && k0 + 128 * h + 32 * lg + 8 * j < a.d ? ld16(xrow + k0 + 128 * h + 8 * j)
                                                                              : zero16();
    };

    uint4 xc[4 * SUB], xn[4 * SUB];
    dma_w(0, wt[0]);
    load_x(0, xc);
    wait_vmem_all();                                            // this wave's copies have landed
    __syncthreads();
    int buf = 0;
    for (int st = 0; st < nstep; ++st) {
        const bool more = st + 1 < nstep;
        if (more) {
            dma_w(st + 1, wt[buf ^ 1]);
            load_x((st + 1) * KSTEP, xn);
        }
        const char* t = wt[buf];
#pragma unroll
        for (int h = 0; h < SUB; ++h)
#pragma unroll
            for (int nt = 0; nt < MAXT; ++nt) {
                if (nt >= nt_used) break;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const char* f = t + ((h * MAXT + nt) * 4 + j) * 2 * GP_FRAG + 16 * lane;
                    mma<BF16>(acc[nt], xc[4 * h + j], lds16(f, 0));
                    mma<BF16>(acc[nt], xc[4 * h + j], lds16(f, GP_FRAG));
                }
            }
        if (more) {
#pragma unroll
            for (int j = 0; j < 4 * SUB; ++j) xc[j] = xn[j];
        }
        // every wave has read tile buf, and (the barrier's wait for all memory operations) every wave's copies into
        // tile buf ^ 1 have landed
        __syncthreads();
        buf ^= 1;
    }
    // accumulator: lane holds output column 16 nt + l16, tokens tok0 + 4 lg .. + 3
    if (tok0 >= a.n_tok) return;
#pragma unroll
    for (int nt = 0; nt < MAXT; ++nt) {
        if (nt >= nt_used) break;
        const int c = 16 * nt + l16;
        if (c >= nout) continue;
        float* out = c < a.n0 ? a.out0 : a.out1;
        const int n = c < a.n0 ? a.n0 : a.n1, cc = c < a.n0 ? c : c - a.n0;
        const float bias = c < a.n0 ? (a.b0 ? a.b0[cc] : 0.f) : (a.b1 ? a.b1[cc] : 0.f);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const long t = tok0 + 4 * lg + e;
            if (t < a.n_tok) out[t * n + cc] = acc[nt][e] + bias;
        }
    }
}

// The same projections for up to GP_SPLIT_MAX_TOK tokens (decode steps, a prompt's 2048-token chunks), where one
// workgroup per token tile would read all of W (n0 + n1 rows of d fp32) on one CU: workgroup (s, tile) = one wave, 16
// tokens, the d range of split s (whole 128-wide steps). It reads its W rows straight from memory (L2-resident: every
// tile reads the same rows), splits them into bf16 high and low parts in registers, loads the next step's x and W
// while the current one multiplies (the lane / MFMA mapping of gate_project_kernel), and writes its partial sums to
// part[s][token][n0 + n1]; gate_project_reduce_kernel adds the splits in a fixed order (s = 0, 1, ..) and the bias.
template <int NT>
__global__ __launch_bounds__(64) void gate_project_split_kernel(GateProjArgs a, int steps_per) {
    const int lane = lane_id(), l16 = lane & 15, lg = lane >> 4;
    const int sp = blockIdx.x;
    const long tok0 = (long)blockIdx.y * 16;
    const int nout = a.n0 + a.n1;
    const long tok = tok0 + l16;
    const bool tok_ok = tok < a.n_tok;
    const uint16_t* xrow = a.x + (tok_ok ? tok : 0) * a.x_st + 32 * lg;
    const float* wrow[NT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
        const int c = 16 * nt + l16;
        wrow[nt] = c < a.n0 ? a.w0 + (long)c * a.d : (c < nout ? a.w1 + (long)(c - a.n0) * a.d : nullptr);
        if (wrow[nt]) wrow[nt] += 32 * lg;
    }
    const int kb = sp * steps_per * 128, ke = min(a.d, kb + steps_per * 128);
    auto ldx = [&](int k0, uint4 (&xa)[4]) {
#pragma unroll
        for (int j = 0; j < 4; ++j)
            xa[j] = tok_ok && k0 + 32 * lg + 8 * j < ke ? ld16(xrow + k0 + 8 * j) : zero16();
    };
    auto ldw = [&](int k0, float4 (&w4)[NT][4][2]) {
#pragma unroll
        for (int nt = 0; nt < NT; ++nt)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const bool ok = wrow[nt] && k0 + 32 * lg + 8 * j < ke;
                w4[nt][j][0] = ok ? *reinterpret_cast<const float4*>(wrow[nt] + k0 + 8 * j) : make_float4(0.f, 0.f, 0.f, 0.f);
                w4[nt][j][1] = ok ? *reinterpret_cast<const float4*>(wrow[nt] + k0 + 8 * j + 4)
                                  : make_float4(0.f, 0.f, 0.f, 0.f);
            }
    };
    f32x4 acc[NT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) acc[nt] = f32x4{0.f, 0.f, 0.f, 0.f};
    uint4 xc[4];
    float4 wc[NT][4][2];
    ldx(kb, xc);
    ldw(kb, wc);
    for (int k0 = kb; k0 < ke; k0 += 128) {
        uint4 xn[4];
        float4 wn[NT][4][2];
        ldx(k0 + 128, xn);                                     // past the split: zeros
        ldw(k0 + 128, wn);
#pragma unroll
        for (int nt = 0; nt < NT; ++nt)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float w[8] = {wc[nt][j][0].x, wc[nt][j][0].y, wc[nt][j][0].z, wc[nt][j][0].w,
                                    wc[nt][j][1].x, wc[nt][j][1].y, wc[nt][j][1].z, wc[nt][j][1].w};
                uint32_t hi[4], lo[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    hi[e] = pack_bf16x2(w[2 * e], w[2 * e + 1]);
                    lo[e] = pack_bf16x2(w[2 * e] - __uint_as_float(hi[e] << 16),
                                        w[2 * e + 1] - __uint_as_float(hi[e] & 0xffff0000u));
                }
                mma<BF16>(acc[nt], xc[j], make_uint4(hi[0], hi[1], hi[2], hi[3]));
                mma<BF16>(acc[nt], xc[j], make_uint4(lo[0], lo[1], lo[2], lo[3]));
            }
#pragma unroll
        for (int j = 0; j < 4; ++j) xc[j] = xn[j];
#pragma unroll
        for (int nt = 0; nt < NT; ++nt)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                wc[nt][j][0] = wn[nt][j][0];
                wc[nt][j][1] = wn[nt][j][1];
            }
    }
    // accumulator: lane holds output column 16 nt + l16, tokens tok0 + 4 lg .. + 3
    float* part = a.part + (long)sp * a.n_tok * nout;
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
        const int c = 16 * nt + l16;
        if (c >= nout) continue;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const long t = tok0 + 4 * lg + e;
            if (t < a.n_tok) part[t * nout + c] = acc[nt][e];
        }
    }
}

__global__ __launch_bounds__(256) void gate_project_reduce_kernel(GateProjArgs a, int nsplit) {
    const int nout = a.n0 + a.n1;
    const long e = (long)blockIdx.x * 256 + threadIdx.x;
    if (e >= a.n_tok * nout) return;
    const long t = e / nout;
    const int c = (int)(e % nout);
    float s = 0.f;
    for (int sp = 0; sp < nsplit; ++sp) s += a.part[(long)sp * a.n_tok * nout + e];
    if (c < a.n0) a.out0[t * a.n0 + c] = s + (a.b0 ? a.b0[c] : 0.f);
    else a.out1[t * a.n1 + (c - a.n0)] = s + (a.b1 ? a.b1[c - a.n0] : 0.f);
}

int gate_project_dispatch(const GateProjArgs& a, hipStream_t stream) {
    const int nsplit = gate_project_nsplit(a.n_tok, a.d);
    if (nsplit > 0) {
        if (!a.part) return BF_STATUS_WORKSPACE;
        const int steps = (a.d + 127) / 128, per = (steps + nsplit - 1) / nsplit;
        const int ns = (steps + per - 1) / per;               // splits that hold at least one step
        const dim3 grid((unsigned)ns, (unsigned)((a.n_tok + 15) / 16));
        if (a.n0 + a.n1 <= 32) hipLaunchKernelGGL(gate_project_split_kernel<2>, grid, dim3(64), 0, stream, a, per);
        else hipLaunchKernelGGL(gate_project_split_kernel<GP_MAX_OUT / 16>, grid, dim3(64), 0, stream, a, per);
        const long n = a.n_tok * (a.n0 + a.n1);
        hipLaunchKernelGGL(gate_project_reduce_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, a, ns);
        return (int)hipGetLastError();
    }
    // split W^T, then the projection: 256-wide steps (64 KB of LDS) up to 32 outputs, else 128-wide (64 KB)
    if (!a.part) return BF_STATUS_WORKSPACE;
    const int nsub = gate_project_wsplit_substeps(a.d);
    const long nthr = (long)nsub * 16 * ((a.n0 + a.n1 + 15) / 16) * 16;
    hipLaunchKernelGGL(gate_split_w_kernel, dim3((unsigned)((nthr + 255) / 256)), dim3(256), 0, stream, a,
                       reinterpret_cast<char*>(a.part), nsub);
    const long tiles = (a.n_tok + 15) / 16;
    const dim3 grid((unsigned)((tiles + GP_WAVES - 1) / GP_WAVES)), block(64 * GP_WAVES);
    const char* ws = reinterpret_cast<const char*>(a.part);
    if (a.n0 + a.n1 <= 32) hipLaunchKernelGGL((gate_project_kernel<2, 2>), grid, block, 0, stream, a, ws);
    else hipLaunchKernelGGL((gate_project_kernel<GP_MAX_OUT / 16, 1>), grid, block, 0, stream, a, ws);
    return (int)hipGetLastError();
}

}  // namespace bf
