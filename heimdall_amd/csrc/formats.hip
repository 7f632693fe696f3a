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

// value of cache quantity `kind` (0 k_rope, 1 v, 2 k_mem, 3 g, 4 beta) of llama.cpp slot l, head g, dim d
__device__ float slot_value(const LlamaStateArgs& a, int b, long l, int kind, int g, int d) {
    const int G = a.G, D = a.D, W = a.W, S = a.S;
    long p = -1;                                          // position of the slot
    bool sink = false;
    if (l < S) {
        p = l;
        sink = p < a.n_sinks;
        if (!sink) return 0.f;
    } else if (l < S + W + 1) {
        p = llama_ring_pos(l - S, a.n, W);
        if (p < 0) return 0.f;
    } else {
        return 0.f;                                       // scratch / padding
    }
    if (sink && kind <= 1) {
        const long at = (((long)b * G + g) * a.n_sinks + p) * D + d;
        return ld_kv(kind == 0 ? a.sink_k : a.sink_v, at, a.kv_dtype);
    }
    const int rs = (int)(p % W);                          // the cache's ring slot
    if (p < (a.n > W ? a.n - W : 0) || a.ring_pos[rs] != p) return 0.f;
    switch (kind) {
        case 0: return ld_kv(a.ring_k, (((long)b * G + g) * W + rs) * D + d, a.kv_dtype);
        case 1: return ld_kv(a.ring_v, (((long)b * G + g) * W + rs) * D + d, a.kv_dtype);
        case 2: return a.ring_km[(((long)b * W + rs) * G + g) * D + d];
        case 3: return a.ring_g[((long)b * W + rs) * G + g];
        default: return a.ring_beta[((long)b * W + rs) * G + g];
    }
}

}  // namespace

// ---- pack: one thread per f32 of the output rows [B][Nb]
__global__ __launch_bounds__(FT) void llama_state_pack_kernel(LlamaStateArgs a) {
    const long nb = a.row, e = (long)blockIdx.x * FT + threadIdx.x;
    if (e >= (long)a.B * nb) return;
    const int b = (int)(e / nb);
    const long x = e % nb;
    const int G = a.G, D = a.D;
    const long LR = a.LR, C = 3L * G * D + 2 * G, GD = (long)G * D;
    const long o_kp = LR * C, o_vp = o_kp + LR * GD, o_dl = o_vp + LR * GD;
    float v;
    if (x < o_kp) {
        const long l = x / C, c = x % C;
        if (c < 3 * GD) v = slot_value(a, b, l, (int)(c / GD), (int)((c % GD) / D), (int)(c % D));
        else v = slot_value(a, b, l, c < 3 * GD + G ? 3 : 4, (int)((c - 3 * GD) % G), 0);
    } else if (x < o_vp) {                                // K plane [G][LR][D]
        const long y = x - o_kp;
        v = slot_value(a, b, (y / D) % LR, 0, (int)(y / (LR * D)), (int)(y % D));
    } else if (x < o_dl) {                                // V plane [G][D][LR]
        const long y = x - o_vp;
        v = slot_value(a, b, y % LR, 1, (int)(y / (LR * D)), (int)((y / LR) % D));
    } else {                                              // delta [G][dv][dk] <- state [G][dk][dv]
        const long y = x - o_dl;
        const int g = (int)(y / ((long)D * D)), dv = (int)((y / D) % D), dk = (int)(y % D);
        v = a.state[(((long)b * G + g) * D + dk) * D + dv];
    }
    a.rows[e] = v;
}

// ---- unpack: one thread per element of the cache (ring k / v, k_mem, g / beta, positions, sinks, state)
__global__ __launch_bounds__(FT) void llama_state_unpack_kernel(LlamaStateArgs a) {
    const long e = (long)blockIdx.x * FT + threadIdx.x;
    const int B = a.B, G = a.G, D = a.D, W = a.W, S = a.S;
    const long LR = a.LR, C = 3L * G * D + 2 * G, GD = (long)G * D, nb = a.row;
    const long o_dl = LR * C + 2 * LR * GD;
    const long n_ring = (long)B * G * W * D;              // ring_k, then ring_v
    const long n_km = (long)B * W * G * D, n_gb = (long)B * W * G, n_sk = (long)B * G * a.n_sinks * D;
    const long n_st = (long)B * G * D * D;
    const long lo = a.n > W ? a.n - W : 0;
    // cache ring slot s holds position p = lo + ((s - lo) mod W) when p < n
    auto ring_p = [&](long s) {
        const long p = lo + ((s - lo % W) % W + W) % W;
        return p < a.n ? p : -1L;
    };
    auto region = [&](int b, long l, long c) { return a.rows[(long)b * nb + l * C + c]; };
    long x = e;
    if (x < 2 * n_ring) {
        const bool is_v = x >= n_ring;
        const long y = is_v ? x - n_ring : x;
        const int d = (int)(y % D);
        const long s = (y / D) % W;
        const int g = (int)((y / ((long)D * W)) % G), b = (int)(y / ((long)D * W * G));
        const long p = ring_p(s);
        const float v = p < 0 ? 0.f : region(b, S + p % (W + 1), (is_v ? GD : 0) + (long)g * D + d);
        st_kv(is_v ? a.ring_v_out : a.ring_k_out, y, v, a.kv_dtype);
        return;
    }
    x -= 2 * n_ring;
    if (x < n_km) {
        const int d = (int)(x % D), g = (int)((x / D) % G);
        const long s = (x / GD) % W;
        const int b = (int)(x / (GD * W));
        const long p = ring_p(s);
        a.ring_km_out[x] = p < 0 ? 0.f : region(b, S + p % (W + 1), 2 * GD + (long)g * D + d);
        return;
    }
    x -= n_km;
    if (x < 2 * n_gb) {
        const bool is_b = x >= n_gb;
        const long y = is_b ? x - n_gb : x;
        const int g = (int)(y % G);
        const long s = (y / G) % W;
        const int b = (int)(y / ((long)G * W));
        const long p = ring_p(s);
        const float v = p < 0 ? 0.f : region(b, S + p % (W + 1), 3 * GD + (is_b ? G : 0) + g);
        (is_b ? a.ring_beta_out : a.ring_g_out)[y] = v;
        return;
    }
    x -= 2 * n_gb;
    if (x < W) {
        a.ring_pos_out[x] = ring_p(x);
        return;
    }
    x -= W;
    if (x < 2 * n_sk) {
        const bool is_v = x >= n_sk;
        const long y = is_v ? x - n_sk : x;
        const int d = (int)(y % D);
        const long j = (y / D) % a.n_sinks;
        const int g = (int)((y / ((long)D * a.n_sinks)) % G), b = (int)(y / ((long)D * a.n_sinks * G));
        st_kv(is_v ? a.sink_v_out : a.sink_k_out, y, region(b, j, (is_v ? GD : 0) + (long)g * D + d), a.kv_dtype);
        return;
    }
    x -= 2 * n_sk;
    if (x < n_st) {                                       // state [B][G][dk][dv] <- delta [G][dv][dk]
        const int dv = (int)(x % D), dk = (int)((x / D) % D), g = (int)((x / ((long)D * D)) % G);
        const int b = (int)(x / ((long)D * D * G));
        a.state_out[x] = a.rows[(long)b * nb + o_dl + ((long)g * D + dv) * D + dk];
    }
}

long llama_state_floats(int G, int D, int W, int S) {
    const long LR = (S + W + 2 + 31) / 32 * 32;
    return LR * (3L * G * D + 2 * G + 2L * G * D) + (long)D * D * G;
}

int llama_state(const LlamaStateArgs& a, bool pack, hipStream_t stream) {
    long total;
    if (pack) {
        total = (long)a.B * a.row;
    } else {
        const long B = a.B, G = a.G, D = a.D, W = a.W;
        total = 2 * B * G * W * D + B * W * G * D + 2 * B * W * G + W + 2 * B * G * a.n_sinks * D + B * G * D * D;
    }
    const unsigned blocks = (unsigned)((total + FT - 1) / FT);
    if (pack) hipLaunchKernelGGL(llama_state_pack_kernel, dim3(blocks), dim3(FT), 0, stream, a);
    else hipLaunchKernelGGL(llama_state_unpack_kernel, dim3(blocks), dim3(FT), 0, stream, a);
    return (int)hipGetLastError();
}

}  // namespace bf
