// The native Gated DeltaNet layer around K1 (reference: GatedDeltaNet.forward, Heimdall/heimdall/hibrit.py:159-184,
// causal_conv Heimdall/heimdall/kernels.py:29-37, l2norm hibrit.py:132-133, GatedNorm hibrit.py:118-129): the two
// memory-bound passes on either side of the delta rule, each one read and one write of its tensors.
//
// gdn_conv_inputs_kernel: from z = in_proj_qkv(x) (channels [q | k | v], C = 2 HK D + HV D) and the a / b gate
// projections, per token
//   y_c = SiLU(sum_j w[c][K-1-j] z[t-j][c])        causal depthwise conv, rows before the sequence start from the
//                                                   carried prefix (or zero)
//   q_h = D^-1/2 l2norm(y_q(h / r)), k_h = l2norm(y_k(h / r)), v_h = y_v(h)     for the HV value heads, r = HV / HK
//   beta = sigmoid(b), g = -exp(A_log) softplus(a + dt_bias)
// One unit = one q / k / v head of D channels, handled by D / 8 consecutive lanes of 8 channels each; the l2norm sum
// is a butterfly over those lanes. q and k are written once per value head that reads them (the
// reference's repeat_interleave), so the delta rule sees one key per state.
//
// gated_norm_kernel: out = w * RMSNorm(o) * SiLU(zg) per row of D; a bf16 layer keeps the reference's bf16 rounding
// points (o rounded to bf16, the normalised row rounded, the weight product rounded, then the SiLU product).
#include "bf_common.h"
#include "bf_internal.h"

namespace bf {

namespace {

__device__ __forceinline__ float bf_round(float x) { return bf2f(f2bf(x)); }

__device__ __forceinline__ void unpack8(const uint4& u, float (&x)[8]) {
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        x[2 * i] = __uint_as_float(w[i] << 16);
        x[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
    }
}

__device__ __forceinline__ uint4 pack8(const float (&x)[8]) {
    return make_uint4(pack_bf16x2(x[0], x[1]), pack_bf16x2(x[2], x[3]), pack_bf16x2(x[4], x[5]),
                      pack_bf16x2(x[6], x[7]));
}

__device__ __forceinline__ void store8(void* base, long elem, int dtype, const float (&x)[8]) {
    if (dtype == DT_BF16) {
        *reinterpret_cast<uint4*>(reinterpret_cast<uint16_t*>(base) + elem) = pack8(x);
    } else {
        float4* p = reinterpret_cast<float4*>(reinterpret_cast<float*>(base) + elem);
        p[0] = make_float4(x[0], x[1], x[2], x[3]);
        p[1] = make_float4(x[4], x[5], x[6], x[7]);
    }
}

// sum over the LPU consecutive lanes of a unit (LPU a power of two <= 64)
template <int LPU>
__device__ __forceinline__ float unit_sum(float v) {
#pragma unroll
    for (int m = LPU / 2; m >= 1; m >>= 1) v += __shfl_xor(v, m);
    return v;
}

__device__ __forceinline__ float silu(float y) { return y / (1.f + __expf(-y)); }

// eight consecutive elements of a bf16 or fp32 row as fp32 (zero when !ok)
template <bool BF>
__device__ __forceinline__ void load8(const void* base, long elem, bool ok, float (&x)[8]) {
    if constexpr (BF) {
        unpack8(ok ? ld16(reinterpret_cast<const uint16_t*>(base) + elem) : zero16(), x);
    } else {
        const float4* p = reinterpret_cast<const float4*>(reinterpret_cast<const float*>(base) + elem);
        const float4 v0 = ok ? p[0] : make_float4(0.f, 0.f, 0.f, 0.f);
        const float4 v1 = ok ? p[1] : make_float4(0.f, 0.f, 0.f, 0.f);
        x[0] = v0.x; x[1] = v0.y; x[2] = v0.z; x[3] = v0.w; x[4] = v1.x; x[5] = v1.y; x[6] = v1.z; x[7] = v1.w;
    }
}

// channels c0 .. c0 + 7 of token n - j (rows before the sequence start come from the carried prefix, or are zero)
template <bool BF>
__device__ __forceinline__ void load_tap(const GdnInArgs& a, bool valid, long n, int j, long seq0, int seq, long C,
                                         int c0, float (&x)[8]) {
    const long p = n - j;
    if (p >= seq0) load8<BF>(a.z, p * a.z_st + c0, valid, x);
    else load8<BF>(a.prefix, ((long)seq * (a.K - 1) + (p - seq0 + a.K - 1)) * C + c0, valid && a.prefix, x);
}

}  // namespace

template <int D, bool BF>
__global__ __launch_bounds__(256) void gdn_conv_inputs_kernel(GdnInArgs a) {
    constexpr int LPU = D / 8;
    const int U = 2 * a.HK + a.HV;
    const long tid = (long)blockIdx.x * blockDim.x + threadIdx.x;
    const long unit = tid / LPU;
    const int s = (int)(tid % LPU);
    const bool valid = unit < a.n_tok * U;
    const long n = valid ? unit / U : 0;
    const int u = valid ? (int)(unit % U) : 0;

    // sequence of token n and its first token
    int lo = 0, hi = a.num_seqs;                          // cu[lo] <= n < cu[hi]
    while (hi - lo > 1) {
        const int mid = (lo + hi) >> 1;
        if (a.cu_seqlens[mid] <= n) lo = mid;
        else hi = mid;
    }
    const long seq0 = a.cu_seqlens[lo];

    const int kind = u < a.HK ? 0 : (u < 2 * a.HK ? 1 : 2);          // q, k, v
    const int head = kind == 0 ? u : (kind == 1 ? u - a.HK : u - 2 * a.HK);
    const long C = (long)(2 * a.HK + a.HV) * D;
    const int c0 = (kind == 0 ? head * D : (kind == 1 ? (a.HK + head) * D : 2 * a.HK * D + head * D)) + 8 * s;

    // tap j reads token n - j with weight column K - 1 - j; K = 4 (the models' conv width) takes each channel's
    // weights as one float4
    float y[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) y[e] = 0.f;
    if (a.K == 4) {
        float4 wc[8];
#pragma unroll
        for (int e = 0; e < 8; ++e)
            wc[e] = valid ? *reinterpret_cast<const float4*>(a.w + (long)(c0 + e) * 4) : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            float x[8];
            load_tap<BF>(a, valid, n, j, seq0, lo, C, c0, x);
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float wj = j == 0 ? wc[e].w : (j == 1 ? wc[e].z : (j == 2 ? wc[e].y : wc[e].x));
                y[e] = fmaf(x[e], wj, y[e]);
            }
        }
    } else {
        for (int j = 0; j < a.K; ++j) {
            float x[8];
            load_tap<BF>(a, valid, n, j, seq0, lo, C, c0, x);
#pragma unroll
            for (int e = 0; e < 8; ++e) y[e] = fmaf(x[e], valid ? a.w[(long)(c0 + e) * a.K + (a.K - 1 - j)] : 0.f, y[e]);
        }
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) y[e] = silu(y[e]);

    if (kind < 2) {
        float ss = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) ss += y[e] * y[e];
        ss = unit_sum<LPU>(ss);                           // every lane of the wave takes part
        const float f = rsqrtf(ss + a.eps) * (kind == 0 ? a.q_scale : 1.f);
#pragma unroll
        for (int e = 0; e < 8; ++e) y[e] *= f;
        if (!valid) return;
        const int r = a.HV / a.HK;
        void* dst = kind == 0 ? a.q : a.k;
        for (int rr = 0; rr < r; ++rr) store8(dst, (n * a.HV + head * r + rr) * D + 8 * s, a.out_dtype, y);
    } else {
        if (!valid) return;
        store8(a.v, (n * a.HV + head) * D + 8 * s, a.out_dtype, y);
        if (s == 0) {
            const long i = n * a.HV + head;
            const float x = a.a[i] + a.dt_bias[head];
            const float sp = x > 20.f ? x : log1pf(__expf(x));   // softplus with torch's default threshold
            a.g[i] = -__expf(a.A_log[head]) * sp;
            a.beta[i] = 1.f / (1.f + __expf(-a.b[i]));
        }
    }
}

// Conv width K = 4 (the models'): a thread keeps one unit's 8 channels over a block of CT consecutive tokens, with
// the channels' weights and the previous three rows in registers, so z is read once and the weights once per block
// (the per-token kernel above re-reads 4 rows and 128 bytes of weights for every 16 bytes of output).
// The outputs may alias z as far as the compiler knows, so a load of z is never moved above an earlier store: the
// rows of CP tokens are therefore loaded together before the group's stores, and the gates of the block's tokens are
// computed first, spread over the unit's lanes (computed per token by one lane, their loads put a second memory
// round trip into every token's chain). Measured on 4 packed sequences {8192, 16384, 24576, 16384}, H = 32, D = 128,
// bf16: 915-999 us before, 770-880 us with the gates first, 740-820 us with 4-row groups and 64-token blocks (2-row
// groups 870 us; 8-row groups 820-850 us at 155 VGPRs; streaming z loads or output stores within noise).
constexpr int CT = 64;
constexpr int CP = 4;

template <int D, bool BF>
__global__ __launch_bounds__(256) void gdn_conv_inputs_k4_kernel(GdnInArgs a) {
    constexpr int LPU = D / 8, UPB = 256 / LPU;
    const int U = 2 * a.HK + a.HV;
    const int ugroups = (U + UPB - 1) / UPB;
    const long n0 = (long)(blockIdx.x / ugroups) * CT;
    const int u = (blockIdx.x % ugroups) * UPB + (int)threadIdx.x / LPU;
    const int s = (int)threadIdx.x % LPU;
    const bool uv = u < U;                                // the unit exists (all lanes of a unit agree)
    const int uu = uv ? u : 0;
    const int kind = uu < a.HK ? 0 : (uu < 2 * a.HK ? 1 : 2);
    const int head = kind == 0 ? uu : (kind == 1 ? uu - a.HK : uu - 2 * a.HK);
    const long C = (long)U * D;
    const int c0 = (kind == 0 ? head * D : (kind == 1 ? (a.HK + head) * D : 2 * a.HK * D + head * D)) + 8 * s;
    const long n1 = n0 + CT < a.n_tok ? n0 + CT : a.n_tok;

    float w[4][8];                                        // w[j][e]: tap j (token n - j) of channel c0 + e
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const float4 wc = uv ? *reinterpret_cast<const float4*>(a.w + (long)(c0 + e) * 4) : make_float4(0.f, 0.f, 0.f, 0.f);
        w[0][e] = wc.w; w[1][e] = wc.z; w[2][e] = wc.y; w[3][e] = wc.x;
    }
    // sequence of n0
    int seq = 0, hi = a.num_seqs;
    while (hi - seq > 1) {
        const int mid = (seq + hi) >> 1;
        if (a.cu_seqlens[mid] <= n0) seq = mid;
        else hi = mid;
    }
    long seq0 = a.cu_seqlens[seq], seq_end = a.cu_seqlens[seq + 1];
    // rows n - 1, n - 2, n - 3 of the current token n
    float r1[8], r2[8], r3[8];
    auto fill = [&](long n) {
        load_tap<BF>(a, uv, n, 1, seq0, seq, C, c0, r1);
        load_tap<BF>(a, uv, n, 2, seq0, seq, C, c0, r2);
        load_tap<BF>(a, uv, n, 3, seq0, seq, C, c0, r3);
    };
    fill(n0);
    const int r = a.HV / a.HK;
    // gates of the block's tokens: lane s of a v unit takes tokens n0 + s, n0 + s + LPU, ..
    if (kind == 2 && uv) {
        const float dtb = a.dt_bias[head], ea = -__expf(a.A_log[head]);
        for (int i = s; i < CT; i += LPU) {
            const long n = n0 + i;
            if (n >= n1) break;
            const long gi = n * a.HV + head;
            const float xg = a.a[gi] + dtb;
            const float sp = xg > 20.f ? xg : log1pf(__expf(xg));
            a.g[gi] = ea * sp;
            a.beta[gi] = 1.f / (1.f + __expf(-a.b[gi]));
        }
    }
    for (long nb = n0; nb < n1; nb += CP) {
        float zr[CP][8];                                  // rows nb .. nb + CP - 1, loaded before the group's stores
#pragma unroll
        for (int i = 0; i < CP; ++i) load8<BF>(a.z, (nb + i) * a.z_st + c0, uv && nb + i < n1, zr[i]);
#pragma unroll
        for (int i = 0; i < CP; ++i) {
            const long n = nb + i;
            if (n >= n1) break;
            while (n == seq_end) {                        // a new sequence starts at n: rows before it from its prefix
                ++seq;
                seq0 = n;
                seq_end = a.cu_seqlens[seq + 1];
                fill(n);
            }
            float y[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float x = zr[i][e];
                y[e] = silu(w[0][e] * x + w[1][e] * r1[e] + w[2][e] * r2[e] + w[3][e] * r3[e]);
                r3[e] = r2[e];
                r2[e] = r1[e];
                r1[e] = x;
            }
            if (kind < 2) {
                float ss = 0.f;
#pragma unroll
                for (int e = 0; e < 8; ++e) ss += y[e] * y[e];
                ss = unit_sum<LPU>(ss);
                const float f = rsqrtf(ss + a.eps) * (kind == 0 ? a.q_scale : 1.f);
#pragma unroll
                for (int e = 0; e < 8; ++e) y[e] *= f;
                if (uv) {
                    void* dst = kind == 0 ? a.q : a.k;
                    for (int rr = 0; rr < r; ++rr) store8(dst, (n * a.HV + head * r + rr) * D + 8 * s, a.out_dtype, y);
                }
            } else if (uv) {
                store8(a.v, (n * a.HV + head) * D + 8 * s, a.out_dtype, y);
            }
        }
    }
}

template <int D, bool BF>
__global__ __launch_bounds__(256) void gated_norm_kernel(GatedNormArgs a) {
    constexpr int LPR = D / 8;
    const long tid = (long)blockIdx.x * blockDim.x + threadIdx.x;
    const long row = tid / LPR;
    const int s = (int)(tid % LPR);
    const bool valid = row < a.rows;
    const long e0 = (valid ? row : 0) * D + 8 * s;

    // BF: the layer runs in bf16 (gate and output bf16, the reference's bf16 rounding points); else all fp32
    float o[8], zg[8];
    if (a.o_dtype == DT_BF16) load8<true>(a.o, e0, valid, o);
    else load8<false>(a.o, e0, valid, o);
    if constexpr (BF) {
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] = bf_round(o[e]);     // o.to(x.dtype)
    }
    load8<BF>(a.z, e0, valid, zg);
    float ss = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) ss += o[e] * o[e];
    ss = unit_sum<LPR>(ss);
    const float inv = rsqrtf(ss / (float)D + a.eps);
    if (!valid) return;
    float r[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        if constexpr (BF) {
            const float h = bf_round(o[e] * inv);
            const float wh = bf_round(a.w[8 * s + e] * h);
            r[e] = wh * silu(zg[e]);
        } else {
            r[e] = a.w[8 * s + e] * (o[e] * inv) * silu(zg[e]);
        }
    }
    store8(a.out, e0, BF ? DT_BF16 : DT_F32, r);
}

int gdn_conv_inputs_dispatch(const GdnInArgs& a, hipStream_t stream) {
    const long threads = a.n_tok * (2 * a.HK + a.HV) * (a.D / 8);
    if (threads == 0) return 0;
    if (a.K == 4) {
        const int upb = 256 / (a.D / 8), U = 2 * a.HK + a.HV;
        const long blocks = ((a.n_tok + CT - 1) / CT) * ((U + upb - 1) / upb);
        if (blocks > 0x7fffffffL) return BF_STATUS_INVALID;
        const dim3 grid((unsigned)blocks), block(256);
        const bool bf = a.in_dtype == DT_BF16;
        switch (a.D) {
            case 64: if (bf) hipLaunchKernelGGL((gdn_conv_inputs_k4_kernel<64, true>), grid, block, 0, stream, a);
                     else hipLaunchKernelGGL((gdn_conv_inputs_k4_kernel<64, false>), grid, block, 0, stream, a); break;
            case 128: if (bf) hipLaunchKernelGGL((gdn_conv_inputs_k4_kernel<128, true>), grid, block, 0, stream, a);
                      else hipLaunchKernelGGL((gdn_conv_inputs_k4_kernel<128, false>), grid, block, 0, stream, a); break;
            case 256: if (bf) hipLaunchKernelGGL((gdn_conv_inputs_k4_kernel<256, true>), grid, block, 0, stream, a);
                      else hipLaunchKernelGGL((gdn_conv_inputs_k4_kernel<256, false>), grid, block, 0, stream, a); break;
            default: return BF_ERR_UNSUPPORTED;
        }
        return (int)hipGetLastError();
    }
    const long blocks = (threads + 255) / 256;
    if (blocks > 0x7fffffffL) return BF_STATUS_INVALID;
    const dim3 grid((unsigned)blocks), block(256);
    auto launch = [&](bool b16, auto kb, auto kf) {
        if (b16) hipLaunchKernelGGL(kb, grid, block, 0, stream, a);
        else hipLaunchKernelGGL(kf, grid, block, 0, stream, a);
    };
    const bool bf = a.in_dtype == DT_BF16;
    switch (a.D) {
        case 64: launch(bf, gdn_conv_inputs_kernel<64, true>, gdn_conv_inputs_kernel<64, false>); break;
        case 128: launch(bf, gdn_conv_inputs_kernel<128, true>, gdn_conv_inputs_kernel<128, false>); break;
        case 256: launch(bf, gdn_conv_inputs_kernel<256, true>, gdn_conv_inputs_kernel<256, false>); break;
        default: return BF_ERR_UNSUPPORTED;
    }
    return (int)hipGetLastError();
}

int gated_norm_dispatch(const GatedNormArgs& a, hipStream_t stream) {
    const long threads = a.rows * (a.D / 8);
    if (threads == 0) return 0;
    const long blocks = (threads + 255) / 256;
    if (blocks > 0x7fffffffL) return BF_STATUS_INVALID;
    const dim3 grid((unsigned)blocks), block(256);
    auto launch = [&](bool b16, auto kb, auto kf) {
        if (b16) hipLaunchKernelGGL(kb, grid, block, 0, stream, a);
        else hipLaunchKernelGGL(kf, grid, block, 0, stream, a);
    };
    const bool bf = a.io_dtype == DT_BF16;
    switch (a.D) {
        case 64: launch(bf, gated_norm_kernel<64, true>, gated_norm_kernel<64, false>); break;
        case 128: launch(bf, gated_norm_kernel<128, true>, gated_norm_kernel<128, false>); break;
        case 256: launch(bf, gated_norm_kernel<256, true>, gated_norm_kernel<256, false>); break;
        default: return BF_ERR_UNSUPPORTED;
    }
    return (int)hipGetLastError();
}

}  // namespace bf
