// The converted layer's prefill of one chunk as one library call (reference: HybridAttention._student with t > 1,
// Heimdall/heimdall/hibrit.py:363-424): the delta-rule write stream (the ring rows leaving the window, then the
// chunk's own rows), the memory on the GDN kernels, the window + sinks + LSE with the gamma mix, then the ring /
// position / state write-back. The helper kernels here move rows; the arithmetic is in gdn_*.hip and window_fa.hip.
//
// layer_query_kernel      the memory queries qm of the chunk (from token qoff on) in the compute dtype
// layer_stream_kernel     write row i' of sequence b: position p = start + qoff + i' - W, from the ring (p < start,
//                         valid iff ring_pos says so, else g = beta = 0) or the chunk (token p - start)
// layer_place_kernel      o_mem [B][T][H][D] rows qoff.. from the GDN output rows (the rows before qoff are never
//                         read: their queries sit in the first W positions, where gamma is 0)
// layer_writeback_kernel  the last min(T, W) tokens into their ring slots (position mod W), and ring_pos
// layer_copy_kernel       the new state over the old one (after every kernel that reads the old one)
#include "bf_common.h"
#include "bf_internal.h"

namespace bf {

namespace {

constexpr int LT = 256;

__device__ __forceinline__ float ldx(const void* p, long i, int dt) {
    return dt == DT_BF16 ? bf2f(reinterpret_cast<const uint16_t*>(p)[i]) : reinterpret_cast<const float*>(p)[i];
}
__device__ __forceinline__ void stx(void* p, long i, float v, int dt) {
    if (dt == DT_BF16) reinterpret_cast<uint16_t*>(p)[i] = f2bf(v);
    else reinterpret_cast<float*>(p)[i] = v;
}

}  // namespace

__global__ __launch_bounds__(LT) void layer_query_kernel(LayerArgs a) {
    const int H = a.G * a.R, D = a.D;
    const long total = (long)a.B * a.Tq * H * D, e = (long)blockIdx.x * LT + threadIdx.x;
    if (e >= total) return;
    const int hd = (int)(e % ((long)H * D));
    const long bi = e / ((long)H * D);
    const int b = (int)(bi / a.Tq), i = (int)(bi % a.Tq);
    stx(a.wq, e, ldx(a.qm, (((long)b * a.T + i + a.qoff) * H) * D + hd, a.qm_dtype), a.in_dtype);
}

__global__ __launch_bounds__(LT) void layer_stream_kernel(LayerArgs a) {
    const int G = a.G, D = a.D, W = a.W;
    const long total = (long)a.B * a.Tq * G * D, e = (long)blockIdx.x * LT + threadIdx.x;
    if (e >= total) return;
    const int d = (int)(e % D), g = (int)((e / D) % G);
    const long bi = e / ((long)G * D);
    const int b = (int)(bi / a.Tq), i = (int)(bi % a.Tq);
    const long p = a.start + a.qoff + i - W;                    // the position written before query qoff + i reads
    float kx = 0.f, vx = 0.f, gx = 0.f, bx = 0.f;
    if (p >= a.start) {                                         // a token of this chunk
        const long t = p - a.start;
        kx = ldx(a.km, (((long)b * a.T + t) * G + g) * D + d, a.km_dtype);
        vx = ldx(a.v, b * a.v_sb + g * a.v_sh + t * a.v_st + d, a.in_dtype);
        gx = a.g[((long)b * a.T + t) * G + g];
        bx = a.beta[((long)b * a.T + t) * G + g];
    } else if (p >= 0) {                                        // a ring row, if it holds that position
        const int s = (int)(p % W);
        if (a.ring_pos[s] == p) {
            kx = a.ring_km[(((long)b * W + s) * G + g) * D + d];
            vx = ldx(a.ring_v, (((long)b * G + g) * W + s) * D + d, a.in_dtype);
            gx = a.ring_g[((long)b * W + s) * G + g];
            bx = a.ring_beta[((long)b * W + s) * G + g];
        }
    }
    stx(a.wk, e, kx, a.in_dtype);
    stx(a.wv, e, vx, a.in_dtype);
    if (d == 0) {
        a.wg[bi * G + g] = gx;
        a.wb[bi * G + g] = bx;
    }
}

__global__ __launch_bounds__(LT) void layer_place_kernel(LayerArgs a) {
    const int H = a.G * a.R, D = a.D;
    const long total = (long)a.B * a.Tq * H * D, e = (long)blockIdx.x * LT + threadIdx.x;
    if (e >= total) return;
    const int hd = (int)(e % ((long)H * D));
    const long bi = e / ((long)H * D);
    const int b = (int)(bi / a.Tq), i = (int)(bi % a.Tq);
    stx(a.o_mem, (((long)b * a.T + a.qoff + i) * H) * D + hd, ldx(a.om, e, a.in_dtype), a.in_dtype);
}

__global__ __launch_bounds__(LT) void layer_writeback_kernel(LayerArgs a) {
    const int G = a.G, D = a.D, W = a.W;
    const int n = a.T < W ? a.T : W;
    const long total = (long)a.B * n * G * D, e = (long)blockIdx.x * LT + threadIdx.x;
    if (e >= total) return;
    const int d = (int)(e % D), g = (int)((e / D) % G);
    const long bi = e / ((long)G * D);
    const int b = (int)(bi / n), j = (int)(bi % n);
    const long t = a.T - n + j, p = a.start + t;
    const int s = (int)(p % W);
    stx(a.ring_k_w, (((long)b * G + g) * W + s) * D + d, ldx(a.kr, b * a.k_sb + g * a.k_sh + t * a.k_st + d, a.in_dtype),
        a.in_dtype);
    stx(a.ring_v_w, (((long)b * G + g) * W + s) * D + d, ldx(a.v, b * a.v_sb + g * a.v_sh + t * a.v_st + d, a.in_dtype),
        a.in_dtype);
    a.ring_km_w[(((long)b * W + s) * G + g) * D + d] = ldx(a.km, (((long)b * a.T + t) * G + g) * D + d, a.km_dtype);
    if (d == 0) {
        a.ring_g_w[((long)b * W + s) * G + g] = a.g[((long)b * a.T + t) * G + g];
        a.ring_beta_w[((long)b * W + s) * G + g] = a.beta[((long)b * a.T + t) * G + g];
        if (b == 0 && g == 0) a.ring_pos_w[s] = p;
    }
}

// The write-back with 4 consecutive dims per thread (8-byte bf16 or 16-byte fp32 accesses); strides multiples of 4.
__device__ __forceinline__ float4 ldx4(const void* p, long i, int dt) {
    if (dt == DT_BF16) {
        const uint2 u = *reinterpret_cast<const uint2*>(reinterpret_cast<const uint16_t*>(p) + i);
        return make_float4(__uint_as_float(u.x << 16), __uint_as_float(u.x & 0xffff0000u), __uint_as_float(u.y << 16),
                           __uint_as_float(u.y & 0xffff0000u));
    }
    return *reinterpret_cast<const float4*>(reinterpret_cast<const float*>(p) + i);
}
__device__ __forceinline__ void stx4(void* p, long i, float4 v, int dt) {
    if (dt == DT_BF16)
        *reinterpret_cast<uint2*>(reinterpret_cast<uint16_t*>(p) + i) =
            make_uint2(pack_bf16x2(v.x, v.y), pack_bf16x2(v.z, v.w));
    else *reinterpret_cast<float4*>(reinterpret_cast<float*>(p) + i) = v;
}

__global__ __launch_bounds__(LT) void layer_writeback4_kernel(LayerArgs a) {
    const int G = a.G, D4 = a.D / 4, W = a.W;
    const int n = a.T < W ? a.T : W;
    const long total = (long)a.B * n * G * D4, e = (long)blockIdx.x * LT + threadIdx.x;
    if (e >= total) return;
    const int d = 4 * (int)(e % D4), g = (int)((e / D4) % G);
    const long bi = e / ((long)G * D4);
    const int b = (int)(bi / n), j = (int)(bi % n);
    const long t = a.T - n + j, p = a.start + t;
    const int s = (int)(p % W);
    const float4 kx = ldx4(a.kr, b * a.k_sb + g * a.k_sh + t * a.k_st + d, a.in_dtype);
    const float4 vx = ldx4(a.v, b * a.v_sb + g * a.v_sh + t * a.v_st + d, a.in_dtype);
    const float4 mx = ldx4(a.km, (((long)b * a.T + t) * G + g) * a.D + d, a.km_dtype);
    stx4(a.ring_k_w, (((long)b * G + g) * W + s) * a.D + d, kx, a.in_dtype);
    stx4(a.ring_v_w, (((long)b * G + g) * W + s) * a.D + d, vx, a.in_dtype);
    *reinterpret_cast<float4*>(a.ring_km_w + (((long)b * W + s) * G + g) * a.D + d) = mx;
    if (d == 0) {
        a.ring_g_w[((long)b * W + s) * G + g] = a.g[((long)b * a.T + t) * G + g];
        a.ring_beta_w[((long)b * W + s) * G + g] = a.beta[((long)b * a.T + t) * G + g];
        if (b == 0 && g == 0) a.ring_pos_w[s] = p;
    }
}

__global__ __launch_bounds__(LT) void layer_copy_kernel(const float* src, float* dst, long n) {
    const long e = ((long)blockIdx.x * LT + threadIdx.x) * 4;
    if (e + 3 < n) {
        *reinterpret_cast<float4*>(dst + e) = *reinterpret_cast<const float4*>(src + e);
    } else {
        for (long x = e; x < n; ++x) dst[x] = src[x];
    }
}

namespace {
unsigned blocks_for(long n) { return (unsigned)((n + LT - 1) / LT); }
}  // namespace

int layer_launch(const LayerArgs& a, int what, hipStream_t s) {
    const int H = a.G * a.R;
    switch (what) {
        case 0:
            hipLaunchKernelGGL(layer_stream_kernel, dim3(blocks_for((long)a.B * a.Tq * a.G * a.D)), dim3(LT), 0, s, a);
            break;
        case 1:
            hipLaunchKernelGGL(layer_place_kernel, dim3(blocks_for((long)a.B * a.Tq * H * a.D)), dim3(LT), 0, s, a);
            break;
        case 4:
            hipLaunchKernelGGL(layer_query_kernel, dim3(blocks_for((long)a.B * a.Tq * H * a.D)), dim3(LT), 0, s, a);
            break;
        case 2: {
            const long n = a.T < a.W ? a.T : a.W;
            // 4 dims per thread when every row start is 4-element aligned
            const uintptr_t ain = a.in_dtype == DT_BF16 ? 7 : 15, akm = a.km_dtype == DT_BF16 ? 7 : 15;
            const bool al = !(((uintptr_t)a.kr | (uintptr_t)a.v | (uintptr_t)a.ring_k_w | (uintptr_t)a.ring_v_w) & ain) &&
                            !((uintptr_t)a.km & akm) && !((uintptr_t)a.ring_km_w & 15);
            if (al && ((a.k_sb | a.k_sh | a.k_st | a.v_sb | a.v_sh | a.v_st) & 3) == 0)
                hipLaunchKernelGGL(layer_writeback4_kernel, dim3(blocks_for((long)a.B * n * a.G * a.D / 4)), dim3(LT), 0,
                                   s, a);
            else
                hipLaunchKernelGGL(layer_writeback_kernel, dim3(blocks_for((long)a.B * n * a.G * a.D)), dim3(LT), 0, s,
                                   a);
            break;
        }
        default: {
            const long n = (long)a.B * a.G * a.D * a.D;
            hipLaunchKernelGGL(layer_copy_kernel, dim3(blocks_for((n + 3) / 4)), dim3(LT), 0, s, a.s_new, a.state, n);
            break;
        }
    }
    return (int)hipGetLastError();
}

}  // namespace bf
