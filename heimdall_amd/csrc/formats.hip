// The llama.cpp per-sequence Bifrost state row (reference: llama_hparams::bifrost_state / bifrost_region /
// bifrost_ring_ch, Heimdall/llamacpp/bifrost.patch:221-239, and the views of build_layer_bifrost, :1000-1013) <->
// the student cache of heimdall_amd.hibrit (ring / sinks / state, the reference's HybridAttention cache).
//
// Row of one sequence, f32, LR = ceil((S + W + 2) / 32) * 32 slots, C = 3 G D + 2 G channels:
//   region [LR][C]      slot l: sinks l < S, ring slot S + p mod (W + 1) for position p, scratch after;
//                       channels [k_rope (g, d) | v (g, d) | k_mem (g, d) | g (g) | beta (g)], (g, d) at g D + d
//   K plane [G][LR][D]  k_rope of every slot (ggml [D, LR, G])
//   V plane [G][D][LR]  v of every slot, transposed (ggml [LR, D, G])
//   delta   [G][dv][dk] the memory state (ggml [D, D, G] read as o = S^T q: dk innermost)
// The cache (position n = tokens seen): ring_k / ring_v [B][G][W][D] (kv dtype), ring_km [B][W][G][D],
// ring_g / ring_beta [B][W][G], ring_pos [W] (slot p mod W holds position p when ring_pos says so), sink_k / sink_v
// [B][G][ns][D] (ns = min(S, n)), state [B][G][dk][dv]. The ring holds positions max(0, n - W) .. n - 1.
// A sink slot's k_mem, g and beta are taken from the ring while the sink position is still in it, else written 0 (the
// layer never reads them: a sink's beta is 0 and its row is attended through k_rope / v only).
// Kernels: the row is written section by section (region rows and the K plane with four channels per thread, the V
// plane and the delta block through 64 x 64 LDS tile transposes) and read back the same way (one cache ring slot or
// sink per block, the state through tile transposes).
#include "bf_common.h"
#include "bf_internal.h"

namespace bf {

namespace {

constexpr int FT = 256;

__device__ __forceinline__ float ld_kv(const void* p, long i, int dt) {
    return dt == DT_BF16 ? bf2f(reinterpret_cast<const uint16_t*>(p)[i]) : reinterpret_cast<const float*>(p)[i];
}
__device__ __forceinline__ void st_kv(void* p, long i, float v, int dt) {
    if (dt == DT_BF16) reinterpret_cast<uint16_t*>(p)[i] = f2bf(v);
    else reinterpret_cast<float*>(p)[i] = v;
}

// position held by llama.cpp ring slot r (0 .. W) at length n, or -1
__device__ __forceinline__ long llama_ring_pos(long r, long n, int W) {
    const long lo = n > W ? n - W : 0;
    long p = lo + ((r - lo % (W + 1)) % (W + 1) + (W + 1)) % (W + 1);
    return p < n ? p : -1;
}

// what slot l of the region holds: the sink index (or -1) and the cache ring slot of its position (or -1)
struct SlotSrc {
    int sink, rs;
};
__device__ __forceinline__ SlotSrc slot_src(const LlamaStateArgs& a, long l) {
    SlotSrc s{-1, -1};
    long p = -1;
    if (l < a.S) {
        if (l < a.n_sinks) { s.sink = (int)l; p = l; }
    } else if (l < a.S + a.W + 1) {
        p = llama_ring_pos(l - a.S, a.n, a.W);
    }
    const long lo = a.n > a.W ? a.n - a.W : 0;
    if (p >= lo && p < a.n && a.ring_pos[p % a.W] == p) s.rs = (int)(p % a.W);
    return s;
}

// k_rope (kind 0) or v (kind 1) of a slot, head g, dim d
__device__ __forceinline__ float slot_kv(const LlamaStateArgs& a, const SlotSrc& s, int b, int kind, int g, int d) {
    if (s.sink >= 0)
        return ld_kv(kind ? a.sink_v : a.sink_k, (((long)b * a.G + g) * a.n_sinks + s.sink) * a.D + d, a.kv_dtype);
    if (s.rs >= 0)
        return ld_kv(kind ? a.ring_v : a.ring_k, (((long)b * a.G + g) * a.W + s.rs) * a.D + d, a.kv_dtype);
    return 0.f;
}

}  // namespace

// four consecutive k_rope / v values of a slot (d a multiple of 4)
__device__ __forceinline__ float4 slot_kv4(const LlamaStateArgs& a, const SlotSrc& s, int b, int kind, int g, int d) {
    long at;
    const void* src;
    if (s.sink >= 0) {
        src = kind ? a.sink_v : a.sink_k;
        at = (((long)b * a.G + g) * a.n_sinks + s.sink) * a.D + d;
    } else if (s.rs >= 0) {
        src = kind ? a.ring_v : a.ring_k;
        at = (((long)b * a.G + g) * a.W + s.rs) * a.D + d;
    } else {
        return make_float4(0.f, 0.f, 0.f, 0.f);
    }
    if (a.kv_dtype == DT_BF16) {
        const uint2 u = *reinterpret_cast<const uint2*>(reinterpret_cast<const uint16_t*>(src) + at);
        return make_float4(__uint_as_float(u.x << 16), __uint_as_float(u.x & 0xffff0000u), __uint_as_float(u.y << 16),
                           __uint_as_float(u.y & 0xffff0000u));
    }
    return *reinterpret_cast<const float4*>(reinterpret_cast<const float*>(src) + at);
}

// ---- pack, region rows and the K plane: grid (LR, B), four channels per thread; the k_rope channels also go to
// K plane [G][LR][D]
__global__ __launch_bounds__(FT) void llama_pack_region_kernel(LlamaStateArgs a) {
    const long l = blockIdx.x;
    const int b = blockIdx.y, G = a.G, D = a.D, GD = G * D, C = 3 * GD + 2 * G;
    const SlotSrc s = slot_src(a, l);
    float* row = a.rows + (long)b * a.row;
    float* out = row + l * C;
    float* kp = row + a.LR * C;
    for (int c = 4 * threadIdx.x; c < 3 * GD; c += 4 * FT) {     // k_rope, v, k_mem: whole float4s
        float4 v;
        if (c < 2 * GD) {
            const int g = (c % GD) / D, d = c % D;
            v = slot_kv4(a, s, b, c / GD, g, d);
            if (c < GD) *reinterpret_cast<float4*>(kp + ((long)g * a.LR + l) * D + d) = v;
        } else {
            v = s.rs >= 0 ? *reinterpret_cast<const float4*>(a.ring_km + ((long)b * a.W + s.rs) * GD + (c - 2 * GD))
                          : make_float4(0.f, 0.f, 0.f, 0.f);
        }
        *reinterpret_cast<float4*>(out + c) = v;
    }
    for (int c = 3 * GD + threadIdx.x; c < C; c += FT) {          // g, beta
        float v = 0.f;
        if (s.rs >= 0) {
            const long base = (long)b * a.W + s.rs;
            v = c < 3 * GD + G ? a.ring_g[base * G + (c - 3 * GD)] : a.ring_beta[base * G + (c - 3 * GD - G)];
        }
        out[c] = v;
    }
}

// ---- pack, V plane [G][D][LR] (transposed through a 64 x 64 LDS tile, four dims per thread on the read, four
// slots per thread on the write): grid (ceil(LR / 64), D / 64, G B)
__global__ __launch_bounds__(FT) void llama_pack_vplane_kernel(LlamaStateArgs a) {
    __shared__ float tile[64][65];
    const int l0 = blockIdx.x * 64, d0 = blockIdx.y * 64, g = blockIdx.z % a.G, b = blockIdx.z / a.G;
    const int t = threadIdx.x;
    {
        const int r0 = t / 16, dq = (t % 16) * 4;            // 16 threads per slot row, 16 rows per pass
        for (int r = r0; r < 64; r += FT / 16) {
            const long l = l0 + r;
            const float4 v = l < a.LR ? slot_kv4(a, slot_src(a, l), b, 1, g, d0 + dq) : make_float4(0.f, 0.f, 0.f, 0.f);
            tile[r][dq] = v.x; tile[r][dq + 1] = v.y; tile[r][dq + 2] = v.z; tile[r][dq + 3] = v.w;
        }
    }
    __syncthreads();
    const long C = 3L * a.G * a.D + 2 * a.G;
    float* out = a.rows + (long)b * a.row + a.LR * C + (long)a.G * a.LR * a.D;
    const int d_r = t / 16, lq = (t % 16) * 4;               // 16 threads per dim row, four slots each
    for (int r = d_r; r < 64; r += FT / 16) {
        const long l = l0 + lq;
        float* o = out + ((long)g * a.D + d0 + r) * a.LR + l;
        if (l + 3 < a.LR && ((a.LR & 3) == 0)) {
            *reinterpret_cast<float4*>(o) = make_float4(tile[lq][r], tile[lq + 1][r], tile[lq + 2][r], tile[lq + 3][r]);
        } else {
            for (int j = 0; j < 4; ++j)
                if (l + j < a.LR) o[j] = tile[lq + j][r];
        }
    }
}

// ---- pack, delta [G][dv][dk] <- state [G][dk][dv] (64 x 64 tiles): grid (D / 64, D / 64, G B)
__global__ __launch_bounds__(FT) void llama_pack_delta_kernel(LlamaStateArgs a) {
    __shared__ float tile[64][65];
    const int k0 = blockIdx.x * 64, v0 = blockIdx.y * 64, g = blockIdx.z % a.G, b = blockIdx.z / a.G, D = a.D;
    const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
    const float* st = a.state + ((long)b * a.G + g) * D * D;
    for (int r = ty; r < 64; r += FT / 64) tile[r][tx] = st[(long)(k0 + r) * D + v0 + tx];   // [dk][dv]
    __syncthreads();
    const long C = 3L * a.G * D + 2 * a.G;
    float* out = a.rows + (long)b * a.row + a.LR * C + 2L * a.G * a.LR * D + (long)g * D * D;
    for (int r = ty; r < 64; r += FT / 64) out[(long)(v0 + r) * D + k0 + tx] = tile[tx][r];      // [dv][dk]
}

// ---- unpack, the ring: grid (W, B), one cache ring slot per block, the region row of its position, four channels
// per thread
__global__ __launch_bounds__(FT) void llama_unpack_ring_kernel(LlamaStateArgs a) {
    const int s = blockIdx.x, b = blockIdx.y, G = a.G, D = a.D, W = a.W, GD = G * D;
    const long C = 3L * GD + 2 * G;
    const long lo = a.n > W ? a.n - W : 0;
    long p = lo + ((s - lo % W) % W + W) % W;
    if (p >= a.n) p = -1;
    const float* row = p < 0 ? nullptr : a.rows + (long)b * a.row + (a.S + p % (W + 1)) * C;
    for (int c = 4 * threadIdx.x; c < 3 * GD; c += 4 * FT) {
        const float4 v = row ? *reinterpret_cast<const float4*>(row + c) : make_float4(0.f, 0.f, 0.f, 0.f);
        if (c < 2 * GD) {
            const int g = (c % GD) / D, d = c % D;
            const long at = (((long)b * G + g) * W + s) * D + d;
            void* dst = c < GD ? a.ring_k_out : a.ring_v_out;
            if (a.kv_dtype == DT_BF16) {
                *reinterpret_cast<uint2*>(reinterpret_cast<uint16_t*>(dst) + at) =
                    make_uint2(pack_bf16x2(v.x, v.y), pack_bf16x2(v.z, v.w));
            } else {
                *reinterpret_cast<float4*>(reinterpret_cast<float*>(dst) + at) = v;
            }
        } else {
            *reinterpret_cast<float4*>(a.ring_km_out + ((long)b * W + s) * GD + (c - 2 * GD)) = v;
        }
    }
    for (int c = 3 * GD + threadIdx.x; c < C; c += FT) {
        const float v = row ? row[c] : 0.f;
        if (c < 3 * GD + G) a.ring_g_out[((long)b * W + s) * G + (c - 3 * GD)] = v;
        else a.ring_beta_out[((long)b * W + s) * G + (c - 3 * GD - G)] = v;
    }
    if (b == 0 && threadIdx.x == 0) a.ring_pos_out[s] = p;
}

// ---- unpack, the sinks: grid (n_sinks, B)
__global__ __launch_bounds__(FT) void llama_unpack_sinks_kernel(LlamaStateArgs a) {
    const int j = blockIdx.x, b = blockIdx.y, G = a.G, D = a.D, GD = G * D;
    const long C = 3L * GD + 2 * G;
    const float* row = a.rows + (long)b * a.row + (long)j * C;
    for (int c = threadIdx.x; c < 2 * GD; c += FT) {
        const int g = (c % GD) / D, d = c % D;
        st_kv(c < GD ? a.sink_k_out : a.sink_v_out, (((long)b * G + g) * a.n_sinks + j) * D + d, row[c], a.kv_dtype);
    }
}

// ---- unpack, the state [G][dk][dv] <- delta [G][dv][dk]: grid (D / 64, D / 64, G B)
__global__ __launch_bounds__(FT) void llama_unpack_state_kernel(LlamaStateArgs a) {
    __shared__ float tile[64][65];
    const int v0 = blockIdx.x * 64, k0 = blockIdx.y * 64, g = blockIdx.z % a.G, b = blockIdx.z / a.G, D = a.D;
    const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
    const long C = 3L * a.G * D + 2 * a.G;
    const float* dl = a.rows + (long)b * a.row + a.LR * C + 2L * a.G * a.LR * D + (long)g * D * D;
    for (int r = ty; r < 64; r += FT / 64) tile[r][tx] = dl[(long)(v0 + r) * D + k0 + tx];      // [dv][dk]
    __syncthreads();
    float* st = a.state_out + ((long)b * a.G + g) * D * D;
    for (int r = ty; r < 64; r += FT / 64) st[(long)(k0 + r) * D + v0 + tx] = tile[tx][r];       // [dk][dv]
}

long llama_state_floats(int G, int D, int W, int S) {
    const long LR = (S + W + 2 + 31) / 32 * 32;
    return LR * (3L * G * D + 2 * G + 2L * G * D) + (long)D * D * G;
}

int llama_state(const LlamaStateArgs& a, bool pack, hipStream_t stream) {
    const dim3 blk(FT), tiles(a.D / 64, a.D / 64, a.G * a.B);
    if (pack) {
        hipLaunchKernelGGL(llama_pack_region_kernel, dim3((unsigned)a.LR, a.B), blk, 0, stream, a);
        hipLaunchKernelGGL(llama_pack_vplane_kernel, dim3((unsigned)((a.LR + 63) / 64), a.D / 64, a.G * a.B), blk, 0,
                           stream, a);
        hipLaunchKernelGGL(llama_pack_delta_kernel, tiles, blk, 0, stream, a);
    } else {
        hipLaunchKernelGGL(llama_unpack_ring_kernel, dim3(a.W, a.B), blk, 0, stream, a);
        if (a.n_sinks) hipLaunchKernelGGL(llama_unpack_sinks_kernel, dim3(a.n_sinks, a.B), blk, 0, stream, a);
        hipLaunchKernelGGL(llama_unpack_state_kernel, tiles, blk, 0, stream, a);
    }
    return (int)hipGetLastError();
}

}  // namespace bf
