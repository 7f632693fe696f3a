// Backward of the chunked GQA gated delta rule (reference: autograd through motor.delta_rule_gqa,
// Heimdall/heimdall/motor.py:70-102, as motor.seq_loss uses it, :149-193), fp32 like the reference's training path.
//
// Per chunk of C = 64 tokens and KV head (gc = in-chunk cumulative log decay, e = exp, C' = last row):
//   A = strict_lower((k b) k^T * e^(gc_i - gc_j)),  M = (I + A)^-1,  u = M (v b),  w = M (k b e^gc)
//   attn_r = tril((s q_r) k^T * e^(gc_i - gc_j)),  qd_r = s q_r e^gc,  kt = k e^(gc_C' - gc)
//   v_new = u - w S,  o_r = qd_r S + attn_r v_new,  S' = e^(gc_C') S + kt^T v_new
// The gradient of a chunk's entry state is affine in the gradient of its exit state (columns independent):
//   dvn = kt dS' + sum_r attn_r^T dO_r,   dS = e^(gc_C') dS' + sum_r qd_r^T dO_r - w^T dvn
// so with every chunk's entry state S (a forward walk) and exit-state gradient dS' (a reverse walk), the gradients of
// q, k, v, b and g are dense per-chunk products, all chunks at once:
//   dattn_r = tril(dO_r v_new^T), dqd_r = dO_r S^T, dkt = v_new dS'^T, dw = -dvn S^T,
//   d(v b) = M^T dvn, d(k b e^gc) = M^T dw, dM = dvn (v b)^T + dw (k b e^gc)^T, dA = -strict_lower(M^T dM M^T)
// followed by the decay, gate and cumulative-sum chains (chunk_final_kernel).
//
// Kernels: bgemm_kernel (batched strided fp32 GEMM on v_mfma_f32_16x16x4f32, optional triangular mask, addend and
// accumulate, in-chunk decay, row scale and row / column dots in the epilogue), chunk_prep_kernel,
// unit_lower_inverse_kernel, walk_fwd_kernel / walk_bwd_kernel (the two state walks), state_dot_kernel,
// chunk_final_kernel, dg_scan_kernel. The host side runs the forward walk, the products that need only its states and
// the state dot on a second stream, beside the reverse walk and its products.
#include <array>
#include <mutex>

#include "bf_common.h"
#include "bf_internal.h"

namespace bf {

namespace {

constexpr int BC = 64;                  // chunk length
constexpr int BW_NT = 256;

// Column scale of a GEMM's A operand when it has none (loaded like a real scale, so no branch drains the prefetch).
__device__ const float kOnes[4] = {1.f, 1.f, 1.f, 1.f};

// Fragment order of an R x C fp32 matrix (C a multiple of 16): its 16 x 16 tiles one after another, row-major over
// tiles, each as 64 lanes x 4 floats with lane 16 q + i holding row i, columns 4 q .. 4 q + 3 of the tile, so a wave
// reads a tile (the operand fragment of v_mfma_f32_16x16x4f32 over 4 k steps) as one contiguous 1 KB.
__device__ __forceinline__ long frag16(int r, int c, int C) {
    return ((long)((r >> 4) * (C >> 4) + (c >> 4)) * 64 + ((c & 15) >> 2) * 16 + (r & 15)) * 4 + (c & 3);
}

// ------------------------------------------------------------------------------------ batched strided fp32 GEMM
// C[z] (M x N) = add[z] + alpha * A[z] diag(ksc) (M x K) B[z] (K x N)   (or C += ... when acc), z = (z0, z1, z2);
// element (m, k) of A at A + z0 sa0 + z1 sa1 + z2 sa2 + m am + (k >> kshift) sak + (k & (2^kshift - 1)) ak (B, C,
// add likewise): the reduction index may run over two strides, e.g. (query head, token) pairs of a token-major
// [token][head][D] tensor. M, N multiples of 64, K of 16 (and 2^kshift a multiple of 16 when it splits K), each
// operand contiguous along one dimension, 16-byte aligned. ksc (or null) scales A's column k by
// ksc[z0 ks0 + z1 ks1 + (k & (2^kshift - 1))], msc (or null) the product's row m by msc[z0 ms0 + z1 ms1 + m]; with
// P = alpha msc A B so scaled, dgc (or null) multiplies kept element (m, n) by e^(gc[m] - gc[n]), gc = dgc + z0 dg0 +
// z1 dg1 (the in-chunk decay). mask 1 keeps m >= n, mask 2 keeps m > n (the rest is written 0, or left unchanged when
// accumulating). C contiguous along n only: with rdo, the row dots of P with rdx (addressed like C) go to
// rdo[(z N/64 + n/64) M + m], one partial per 64 columns, and with cdo the column dots to cdo[(z M/64 + m/64) N + n]
// (z = blockIdx.x). With cfrag, C is written in fragment order (frag16) at its batch offset.
struct BgArgs {
    int M, N, K, n1, n2, nz, kshift;
    const float* A; long sa0, sa1, sa2, am, ak, sak;
    const float* B; long sb0, sb1, sb2, bk, bn, sbk;
    float* C; long sc0, sc1, sc2, cm, cn;
    const float* add;                   // same strides as C, or null
    const float* ksc; long ks0, ks1;
    const float* msc; long ms0, ms1;
    const float* dgc; long dg0, dg1;
    const float* rdx; float* rdo; float* cdo;
    float alpha;
    int acc, mask, cfrag;               // cfrag: C (per z at its batch offset) in fragment order, cm / cn unused
};

// Tiles of 64 x BN (BN = 64 or 128; 4 waves of 32 x BN/2) over K steps of 32. Each step's 64 x 32 tile of A and
// 32 x BN tile of B are read with 16-byte loads along whichever dimension is contiguous (AK: A's k, else its m; BK:
// B's k, else its n) and stored in LDS in the same orientation with 16-byte writes: a k-contiguous operand as
// [row][k] (pitch 36 floats: the 16 rows of a fragment hit distinct banks; a fragment is one 16-byte read), the other
// as [k][row] (pitch 4 mod 16 floats: the four k rows a fragment read spans fall 16 banks apart; a fragment is four
// 4-byte reads). Fragment value j of lane (i, q) is k = 16 kh + 4 q + j for both operands. The LDS tiles are double
// buffered: step s computes from one buffer, then writes step s + 1's operands (loaded from global during step s - 1)
// into the other and issues step s + 2's loads, with one barrier per step.
// EX: the epilogue extras compiled in: 0 none, 1 msc and rdo, 2 also dgc and cdo. The plain products measurably need
// the small epilogue, and the row-scaled ones one without the per-element decay.
template <bool AK, bool BK, int BN, int EX>
__global__ __launch_bounds__(BW_NT) void bgemm_kernel(BgArgs a) {
    constexpr int KS = 32, LDK = KS + 4;        // k per step, LDS row pitch (floats)
    constexpr int WN = BN / 2, TU = WN / 16;    // wave tile 32 x WN: 2 x TU MFMA tiles
    constexpr int KQ = KS / 4, KG = KS / 16;    // 16-byte slots along k per row; 16-k groups per step
    constexpr int NA = 64 * KS / 1024, NB = BN * KS / 1024;   // 16-byte global loads per thread per step
    const int lane = lane_id(), wv = wave_id(), tid = threadIdx.x;
    const long z = blockIdx.x;
    const long z2 = z % a.n2, z1 = (z / a.n2) % a.n1, z0 = z / ((long)a.n1 * a.n2);
    const float* A = a.A + z0 * a.sa0 + z1 * a.sa1 + z2 * a.sa2;
    const float* B = a.B + z0 * a.sb0 + z1 * a.sb1 + z2 * a.sb2;
    // A's column scale (ones without one): loaded with the tile and applied when the tile is stored to LDS a step
    // later, since a multiply right after the loads would wait for them
    const float* ksc = a.ksc ? a.ksc + z0 * a.ks0 + z1 * a.ks1 : kOnes;
    const int kscm = a.ksc ? -1 : 0;                      // index mask: every k, or element 0 of kOnes
    const int ksh = a.kshift, klo = (1 << ksh) - 1;
    const long coff = z0 * a.sc0 + z1 * a.sc1 + z2 * a.sc2;
    const int tm = blockIdx.y * 64, tn = blockIdx.z * BN;
    const int m0 = (wv >> 1) * 32, n0 = (wv & 1) * WN;      // the wave's 32 x WN block inside the tile
    const int i = lane & 15, q = lane >> 4;
    constexpr int AR = AK ? 64 : KS, AP = AK ? LDK : 64 + 4;     // LDS rows and pitch of A
    constexpr int BR = BK ? BN : KS, BP = BK ? LDK : BN + 4;     // and of B
    constexpr int ASZ = 2 * AR * AP, BSZ = 2 * BR * BP, CSZ = 64 * (BN + 4);
    __shared__ __align__(16) float lds[ASZ + BSZ > CSZ ? ASZ + BSZ : CSZ];   // operand tiles, then the output tile
    float (*As)[AR][AP] = reinterpret_cast<float (*)[AR][AP]>(lds);
    float (*Bs)[BR][BP] = reinterpret_cast<float (*)[BR][BP]>(lds + ASZ);
    f32x4 acc[2][TU];
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int u = 0; u < TU; ++u) acc[t][u] = f32x4{0.f, 0.f, 0.f, 0.f};
    // the block-level skip of a masked tile wholly outside the kept triangle
    const bool skip = (a.mask == 1 && tm + 63 < tn) || (a.mask == 2 && tm + 63 <= tn);
    // Load slot h of a thread. k-contiguous operand: row tid / KQ + (256 / KQ) h, k (tid % KQ) * 4 .. + 3; otherwise
    // k tid / 16 + 16 (h % KG), rows (tid % 16) * 4 + 64 (h / KG) .. + 3. A step starts at a multiple of 16 and
    // 2^kshift is a multiple of 16, so the 4 k of a k-contiguous slot share their high part.
    auto koff = [&](int k, long shi, long slo) { return (long)(k >> ksh) * shi + (long)(k & klo) * slo; };
    auto load_a = [&](int k0, int h, float4& sv) {
        if (AK) {
            const int k = k0 + (tid % KQ) * 4;
            sv = *reinterpret_cast<const float4*>(ksc + (k & klo & kscm));
            return *reinterpret_cast<const float4*>(A + (long)(tm + tid / KQ + (256 / KQ) * h) * a.am + koff(k, a.sak, a.ak));
        }
        const int k = k0 + tid / 16 + 16 * (h % KG);
        const float c = ksc[k & klo & kscm];
        sv = make_float4(c, c, c, c);
        return *reinterpret_cast<const float4*>(A + koff(k, a.sak, a.ak) + tm + (tid % 16) * 4 + 64 * (h / KG));
    };
    auto load_b = [&](int k0, int h) {
        if (BK) {
            const int k = k0 + (tid % KQ) * 4;
            return *reinterpret_cast<const float4*>(B + (long)(tn + tid / KQ + (256 / KQ) * h) * a.bn + koff(k, a.sbk, a.bk));
        }
        const int k = k0 + tid / 16 + 16 * (h % KG);
        return *reinterpret_cast<const float4*>(B + koff(k, a.sbk, a.bk) + tn + (tid % 16) * 4 + 64 * (h / KG));
    };
    auto store = [&](int buf, const float4 (&xa)[NA], const float4 (&sa)[NA], const float4 (&xb)[NB]) {
#pragma unroll
        for (int h = 0; h < NA; ++h) {
            const float4 x = make_float4(xa[h].x * sa[h].x, xa[h].y * sa[h].y, xa[h].z * sa[h].z, xa[h].w * sa[h].w);
            if (AK) *reinterpret_cast<float4*>(&As[buf][tid / KQ + (256 / KQ) * h][(tid % KQ) * 4]) = x;
            else *reinterpret_cast<float4*>(&As[buf][tid / 16 + 16 * (h % KG)][(tid % 16) * 4 + 64 * (h / KG)]) = x;
        }
#pragma unroll
        for (int h = 0; h < NB; ++h) {
            if (BK) *reinterpret_cast<float4*>(&Bs[buf][tid / KQ + (256 / KQ) * h][(tid % KQ) * 4]) = xb[h];
            else *reinterpret_cast<float4*>(&Bs[buf][tid / 16 + 16 * (h % KG)][(tid % 16) * 4 + 64 * (h / KG)]) = xb[h];
        }
    };
    auto compute = [&](int buf) {
#pragma unroll
        for (int kh = 0; kh < KG; ++kh) {
            uint4 af[2], bf[TU];
            const int kr = 16 * kh + 4 * q;
#pragma unroll
            for (int t = 0; t < 2; ++t) {
                const int r = m0 + 16 * t + i;
                af[t] = AK ? *reinterpret_cast<const uint4*>(&As[buf][r][kr])
                           : make_uint4(__float_as_uint(As[buf][kr][r]), __float_as_uint(As[buf][kr + 1][r]),
                                        __float_as_uint(As[buf][kr + 2][r]), __float_as_uint(As[buf][kr + 3][r]));
            }
#pragma unroll
            for (int u = 0; u < TU; ++u) {
                const int r = n0 + 16 * u + i;
                bf[u] = BK ? *reinterpret_cast<const uint4*>(&Bs[buf][r][kr])
                           : make_uint4(__float_as_uint(Bs[buf][kr][r]), __float_as_uint(Bs[buf][kr + 1][r]),
                                        __float_as_uint(Bs[buf][kr + 2][r]), __float_as_uint(Bs[buf][kr + 3][r]));
            }
#pragma unroll
            for (int t = 0; t < 2; ++t)
#pragma unroll
                for (int u = 0; u < TU; ++u) mma<F32>(acc[t][u], af[t], bf[u]);
        }
    };
    if (!skip) {
        const int ns = a.K / KS;
        float4 xa[NA], sa[NA], xb[NB];
        auto fetch = [&](int s) {
#pragma unroll
            for (int h = 0; h < NA; ++h) xa[h] = load_a(s * KS, h, sa[h]);
#pragma unroll
            for (int h = 0; h < NB; ++h) xb[h] = load_b(s * KS, h);
        };
        fetch(0);
        store(0, xa, sa, xb);
        if (ns > 1) fetch(1);
        __syncthreads();
        for (int s = 0; s < ns; ++s) {
            compute(s & 1);
            if (s + 1 < ns) {
                store((s + 1) & 1, xa, sa, xb);
                if (s + 2 < ns) fetch(s + 2);
            }
            __syncthreads();
        }
    }
    const float* msc = EX >= 1 && a.msc ? a.msc + z0 * a.ms0 + z1 * a.ms1 : nullptr;
    if (a.cn == 1) {
        // Row-contiguous output: the tile goes through LDS (free after the last step's barrier) and each thread then
        // handles 16-byte row pieces, so C, the addend and rdx move as whole rows. All reads of a thread are issued
        // before the first use. Out = prev + (kept ? alpha msc[m] x : 0), prev = C when accumulating, else the
        // addend or 0 (a masked element keeps its C).
        float (*Cs)[BN + 4] = reinterpret_cast<float (*)[BN + 4]>(lds);
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int u = 0; u < TU; ++u)
#pragma unroll
                for (int v = 0; v < 4; ++v) Cs[m0 + 16 * t + 4 * q + v][n0 + 16 * u + i] = acc[t][u][v];
        __syncthreads();
        constexpr int RW = BN / 4, NP = 64 * RW / BW_NT;    // pieces per row, per thread
        const int c4 = tid % RW;
        const int n = tn + 4 * c4;
        auto row = [&](int j) { return tid / RW + (BW_NT / RW) * j; };
        const bool cf = EX >= 1 && a.cfrag;
        auto at = [&](int j) { return cf ? coff + frag16(tm + row(j), n, a.N) : coff + (long)(tm + row(j)) * a.cm + n; };
        const bool dots = (EX >= 1 && a.rdo) || (EX == 2 && a.cdo);
        const float* gc = EX == 2 && a.dgc ? a.dgc + z0 * a.dg0 + z1 * a.dg1 : nullptr;
        float4 prev[NP], rx[NP], gn = make_float4(0.f, 0.f, 0.f, 0.f);
        if (a.acc || a.add) {
            const float* src = a.acc ? a.C : a.add;
#pragma unroll
            for (int j = 0; j < NP; ++j) prev[j] = *reinterpret_cast<const float4*>(src + at(j));
        } else {
#pragma unroll
            for (int j = 0; j < NP; ++j) prev[j] = make_float4(0.f, 0.f, 0.f, 0.f);
        }
        if (dots) {
#pragma unroll
            for (int j = 0; j < NP; ++j) rx[j] = *reinterpret_cast<const float4*>(a.rdx + at(j));
        }
        if (gc) gn = *reinterpret_cast<const float4*>(gc + n);
#pragma unroll
        for (int j = 0; j < NP; ++j) {
            const int m = tm + row(j);
            const float4 x = *reinterpret_cast<const float4*>(&Cs[row(j)][4 * c4]);
            const float al = msc ? a.alpha * msc[m] : a.alpha;
            const float pv[4] = {al * x.x, al * x.y, al * x.z, al * x.w};
            if (dots) {
                const float zv[4] = {pv[0] * rx[j].x, pv[1] * rx[j].y, pv[2] * rx[j].z, pv[3] * rx[j].w};
                if (a.rdo) {                              // one partial per 64 columns: 16 pieces of the row
                    float d = (zv[0] + zv[1]) + (zv[2] + zv[3]);
#pragma unroll
                    for (int off = 1; off < 16; off <<= 1) d += __shfl_xor(d, off);
                    if (c4 % 16 == 0) a.rdo[((long)z * (a.N / 64) + (tn + 4 * c4) / 64) * a.M + m] = d;
                }
                if (EX == 2 && a.cdo)                      // the piece's own slot: only this thread reads it
                    *reinterpret_cast<float4*>(&Cs[row(j)][4 * c4]) = make_float4(zv[0], zv[1], zv[2], zv[3]);
            }
            const float gm = gc ? gc[m] : 0.f;
            const float gv[4] = {gn.x, gn.y, gn.z, gn.w};
            float ov[4] = {prev[j].x, prev[j].y, prev[j].z, prev[j].w};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const bool keep = a.mask == 0 || (a.mask == 1 && m >= n + e) || (a.mask == 2 && m > n + e);
                if (keep) ov[e] += gc ? pv[e] * expf(gm - gv[e]) : pv[e];
            }
            *reinterpret_cast<float4*>(a.C + at(j)) = make_float4(ov[0], ov[1], ov[2], ov[3]);
        }
        if (EX == 2 && a.cdo) {                            // column sums of the tile's row dots
            __syncthreads();
            if (tid < BN) {
                float cs = 0.f;
#pragma unroll 8
                for (int r = 0; r < 64; ++r) cs += Cs[r][tid];
                a.cdo[((long)z * (a.M / 64) + tm / 64) * a.N + tn + tid] = cs;
            }
        }
        return;
    }
    // Column-strided output: per lane. The prior values are read first, all under one branch: tested per element, each
    // read sat in its own basic block and was waited for before the next one was issued. The tiles cover M x N
    // exactly (multiples of 64 and BN), so every address is in range.
    auto at_of = [&](int t, int u, int v) {
        const int m = tm + m0 + 16 * t + 4 * q + v, n = tn + n0 + 16 * u + i;
        return coff + (long)m * a.cm + (long)n * a.cn;
    };
    float prev[2][TU][4];
    if (a.acc || a.add) {
        const float* src = a.acc ? a.C : a.add;
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int u = 0; u < TU; ++u)
#pragma unroll
                for (int v = 0; v < 4; ++v) prev[t][u][v] = src[at_of(t, u, v)];
    } else {
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int u = 0; u < TU; ++u)
#pragma unroll
                for (int v = 0; v < 4; ++v) prev[t][u][v] = 0.f;
    }
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int u = 0; u < TU; ++u)
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int m = tm + m0 + 16 * t + 4 * q + v, n = tn + n0 + 16 * u + i;
                const bool keep = a.mask == 0 || (a.mask == 1 && m >= n) || (a.mask == 2 && m > n);
                const long at = at_of(t, u, v);
                const float al = msc ? a.alpha * msc[m] : a.alpha;
                const float val = keep ? al * acc[t][u][v] : 0.f;
                if (a.acc) {
                    if (keep) a.C[at] = prev[t][u][v] + val;
                } else {
                    a.C[at] = val + prev[t][u][v];
                }
            }
}

// ------------------------------------------------------------------------------------ per-chunk elementwise prep
// one workgroup per (chunk, KV head, row quarter): gc, e^gc, k b, v b, k b e^gc, kt (and transposed)
__global__ __launch_bounds__(BW_NT) void chunk_prep_kernel(GdnBwdArgs a) {
    const long bc = blockIdx.x;
    const int g = blockIdx.y, r0 = blockIdx.z * 16, tid = threadIdx.x;   // rows r0 .. r0 + 15 of the chunk
    const int D = a.D, G = a.G;
    __shared__ float gc[BC], eg[BC];
    const long cg = bc * G + g;
    if (tid < 64) {
        // inclusive prefix sum of g over the chunk (one wave, shuffle scan)
        float x = a.g[(bc * BC + tid) * G + g];
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
            const float y = __shfl_up(x, off);
            if (tid >= off) x += y;
        }
        gc[tid] = x;
        eg[tid] = expf(x);
        if (blockIdx.z == 0) {
            a.gam[cg * BC + tid] = x;
            a.eg[cg * BC + tid] = eg[tid];
        }
    }
    __syncthreads();
    const float gl = gc[BC - 1];
    // 16-byte pieces: rows r0 .. r0 + 15, four dims each (every output row-contiguous or a fragment-order float4)
    const int D4 = D / 4;
    for (int e = tid; e < 16 * D4; e += BW_NT) {
        const int i = r0 + e / D4, d = 4 * (e % D4);
        const long tok = bc * BC + i;
        const float be = a.beta[tok * G + g], ei = eg[i], et = expf(gl - gc[i]);
        const float4 kx = *reinterpret_cast<const float4*>(a.k + (tok * G + g) * D + d);
        const float4 vx = *reinterpret_cast<const float4*>(a.v + (tok * G + g) * D + d);
        const long o = (cg * BC + i) * D + d;
        const float4 kb = make_float4(kx.x * be, kx.y * be, kx.z * be, kx.w * be);
        const float4 kt = make_float4(kx.x * et, kx.y * et, kx.z * et, kx.w * et);
        *reinterpret_cast<float4*>(a.kb + o) = kb;
        *reinterpret_cast<float4*>(a.vb + o) = make_float4(vx.x * be, vx.y * be, vx.z * be, vx.w * be);
        *reinterpret_cast<float4*>(a.kbe + o) = make_float4(kb.x * ei, kb.y * ei, kb.z * ei, kb.w * ei);
        *reinterpret_cast<float4*>(a.ktl + o) = kt;
        *reinterpret_cast<float4*>(a.ktlF + cg * BC * D + frag16(i, d, D)) = kt;   // fragment order, reverse walk
    }
    // kt transposed [D][C] in fragment order (forward walk): dim d, tokens i .. i + 3 of the quarter per piece
    for (int e = tid; e < 4 * D; e += BW_NT) {
        const int d = e % D, i = r0 + 4 * (e / D);
        float x[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) x[u] = a.k[((bc * BC + i + u) * G + g) * D + d] * expf(gl - gc[i + u]);
        *reinterpret_cast<float4*>(a.ktlTF + cg * D * BC + frag16(d, i, BC)) = make_float4(x[0], x[1], x[2], x[3]);
    }
}


// M = (I + A)^-1 for a strictly lower A (C x C): forward substitution, lane j owns column j
__global__ __launch_bounds__(64) void unit_lower_inverse_kernel(const float* Am, float* Mi) {
    const long cg = blockIdx.x;
    __shared__ float As[BC][BC + 1];
    __shared__ float Ms[BC][BC + 1];
    const int j = threadIdx.x;
    for (int i = 0; i < BC; ++i) As[i][j] = Am[(cg * BC + i) * BC + j];
    __syncthreads();
    for (int i = 0; i < BC; ++i) {
        float s = i == j ? 1.f : 0.f;
        for (int k = 0; k < i; ++k) s -= As[i][k] * Ms[k][j];
        Ms[i][j] = s;
    }
    for (int i = 0; i < BC; ++i) Mi[(cg * BC + i) * BC + j] = Ms[i][j];
}

// ------------------------------------------------------------------------------------ state walks
// Grid (sequences, G, D / 16) per walk: a workgroup owns 16 state columns of one KV head and walks the chunks in order
// (forward, or backward in the reverse walk), the strip held in fp32 MFMA accumulators; per chunk two products on
// v_mfma_f32_16x16x4f32 with the strip (and v_new / dvn) passed through LDS transposed, so every operand fragment is
// one 16-byte read. WALK_NW<D> waves: 8 at D >= 128 (two per SIMD, so one wave's loads and LDS exchange overlap the
// other's MFMAs), 4 at D = 64. Wave w owns row tiles [w RT, (w + 1) RT) of the strip; for the 64-token product the
// waves split into KH = NW / 4 parts of the D-long reduction, each part's partial sums go to LDS and the reader adds
// them. The next chunk's operands go into a second register set, their loads (and the chunk's own stores) issued one
// per MFMA step; the barriers order LDS only (lds_barrier), so the loads stay in flight across them.
template <int D>
constexpr int walk_nw() { return D >= 128 ? 8 : 4; }
// 16-column strips per workgroup. Every workgroup streams all of w and kt each chunk whatever its width; two strips
// per workgroup halve that traffic but measured slower (978 against 756 us per launch at T = 8192, G = 4, D = 256).
template <int D>
constexpr int walk_sw() { return 1; }

template <int D>
__device__ __forceinline__ void walk_fwd(const GdnBwdArgs& a, int strip) {
    constexpr int NW = walk_nw<D>(), NTD = D / 16, RT = NTD / NW;   // row tiles per wave
    constexpr int KH = NW / 4;                                       // parts of the D-long reduction of v_new
    constexpr int KD = D / 16 / KH, KC = BC / 16;                    // 16-wide k steps per part / over the chunk
    constexpr int SW = walk_sw<D>(), NE = SW * RT * 4;              // strips; state elements per lane
    const int b = blockIdx.x, g = blockIdx.y, col0 = strip * 16 * SW;
    const int lane = lane_id(), wv = wave_id(), i16 = lane & 15, q = lane >> 4;
    const int tq = wv & 3, kh = wv >> 2;                             // v_new token tile and reduction part
    const int G = a.G, n = a.n_chunks;
    __shared__ float ST[16 * SW][D + 4];                  // strips transposed: ST[col][row]
    __shared__ float VT[KH][16 * SW][BC + 4];             // v_new partial sums transposed: VT[part][col][token]
    // element e of a lane: strip e / (4 RT), row tile (e / 4) % RT, accumulator row e % 4
    auto erow = [&](int e) { return (wv * RT + (e / 4) % RT) * 16 + 4 * q + e % 4; };
    auto ecol = [&](int e) { return col0 + 16 * (e / (4 * RT)) + i16; };
    f32x4 S[SW][RT];
#pragma unroll
    for (int e = 0; e < NE; ++e) S[e / (4 * RT)][(e / 4) % RT][e % 4] = a.s0 ? a.s0[(((long)b * G + g) * D + erow(e)) * D + ecol(e)] : 0.f;
    // One chunk's operands: w row fragments of this wave's reduction part, kt^T fragments of its row tiles, the u strip
    // (part 0), the chunk decay. Each workgroup streams all of w and kt (128 KB at D = 256) per chunk, more than the
    // CU's vector memory path takes in the chunk's MFMA time, so a wave issuing them back to back stalls on the full
    // queue (3.6-6.4 K cycles a chunk, measured) with its MFMAs behind it. Two register sets: chunk c + 1's loads
    // (and chunk c's state stores) are issued one per MFMA step of chunk c, after chunk c's operands have been waited
    // for, so they queue while the MFMAs run and have the rest of the chunk to land.
    struct Ops {
        float4 wf[KD], kf[RT][KC];
        float uf[SW][4], gl;
    };
    // (w and kt^T in fragment order: each load is one contiguous 1 KB tile)
    auto ld_w = [&](Ops& o, long cg, int k) {
        o.wf[k] = *reinterpret_cast<const float4*>(a.wF + cg * BC * D + (long)(tq * (D / 16) + kh * (D / KH / 16) + k) * 256 + 4 * lane);
    };
    auto ld_k = [&](Ops& o, long cg, int t, int k) {
        o.kf[t][k] = *reinterpret_cast<const float4*>(a.ktlTF + cg * D * BC + (long)((wv * RT + t) * (BC / 16) + k) * 256 + 4 * lane);
    };
    auto ld_rest = [&](Ops& o, long cg) {
#pragma unroll
        for (int c2 = 0; c2 < SW; ++c2)
#pragma unroll
            for (int v = 0; v < 4; ++v)
                o.uf[c2][v] = kh == 0 ? a.u[(cg * BC + 16 * tq + 4 * q + v) * D + col0 + 16 * c2 + i16] : 0.f;
        o.gl = a.gam[cg * BC + BC - 1];
    };
    Ops o0, o1;
    {
        const long cg = (long)b * n * G + g;
#pragma unroll
        for (int k = 0; k < KD; ++k) ld_w(o0, cg, k);
#pragma unroll
        for (int t = 0; t < RT; ++t)
#pragma unroll
            for (int k = 0; k < KC; ++k) ld_k(o0, cg, t, k);
        ld_rest(o0, cg);
    }
    auto chunk = [&](int c, const Ops& cur, Ops& nxt) {
        const long cg = ((long)b * n + c) * G + g;
        const long cn = ((long)b * n + (c + 1 < n ? c + 1 : c)) * G + g;   // the next chunk (the last one refetches)
#pragma unroll
        for (int e = 0; e < NE; ++e) ST[16 * (e / (4 * RT)) + i16][erow(e)] = S[e / (4 * RT)][(e / 4) % RT][e % 4];
        lds_barrier();
        wait_vmem_all();                                   // this chunk's operands (and the last chunk's stores)
        // v_new rows [16 tq, 16 tq + 16) = u - w S, this wave's part of the reduction (four partial accumulators:
        // shorter MFMA dependency chains); the next chunk's w and this chunk's entry-state stores ride along
        f32x4 part[SW][4];
#pragma unroll
        for (int c2 = 0; c2 < SW; ++c2) {
            part[c2][0] = f32x4{cur.uf[c2][0], cur.uf[c2][1], cur.uf[c2][2], cur.uf[c2][3]};
#pragma unroll
            for (int p = 1; p < 4; ++p) part[c2][p] = f32x4{0.f, 0.f, 0.f, 0.f};
        }
#pragma unroll
        for (int k = 0; k < KD; ++k) {
            const uint4 af = make_uint4(__float_as_uint(-cur.wf[k].x), __float_as_uint(-cur.wf[k].y),
                                        __float_as_uint(-cur.wf[k].z), __float_as_uint(-cur.wf[k].w));
#pragma unroll
            for (int c2 = 0; c2 < SW; ++c2) {
                const uint4 bf = *reinterpret_cast<const uint4*>(&ST[16 * c2 + i16][kh * (D / KH) + 16 * k + 4 * q]);
                mma<F32>(part[c2][k & 3], af, bf);
            }
            ld_w(nxt, cn, k);
#pragma unroll
            for (int e = k * NE / KD; e < (k + 1) * NE / KD; ++e)              // entry state of chunk c
                a.Sc[(cg * D + erow(e)) * D + ecol(e)] = S[e / (4 * RT)][(e / 4) % RT][e % 4];
            __builtin_amdgcn_sched_barrier(0);
        }
#pragma unroll
        for (int c2 = 0; c2 < SW; ++c2) {
            const f32x4 acc = (part[c2][0] + part[c2][1]) + (part[c2][2] + part[c2][3]);
#pragma unroll
            for (int v = 0; v < 4; ++v) VT[kh][16 * c2 + i16][16 * tq + 4 * q + v] = acc[v];
        }
        lds_barrier();
        // S = e^(gc_C') S + kt^T v_new (v_new = the sum of the parts); the next chunk's kt^T rides along
        const float ec = expf(cur.gl);
#pragma unroll
        for (int t = 0; t < RT; ++t) {
#pragma unroll
            for (int c2 = 0; c2 < SW; ++c2)
#pragma unroll
                for (int v = 0; v < 4; ++v) S[c2][t][v] *= ec;
#pragma unroll
            for (int k = 0; k < KC; ++k) {
#pragma unroll
                for (int c2 = 0; c2 < SW; ++c2) {
                    float4 vs = *reinterpret_cast<const float4*>(&VT[0][16 * c2 + i16][16 * k + 4 * q]);
#pragma unroll
                    for (int p = 1; p < KH; ++p) {
                        const float4 x = *reinterpret_cast<const float4*>(&VT[p][16 * c2 + i16][16 * k + 4 * q]);
                        vs.x += x.x; vs.y += x.y; vs.z += x.z; vs.w += x.w;
                    }
                    mma<F32>(S[c2][t], __builtin_bit_cast(uint4, cur.kf[t][k]), __builtin_bit_cast(uint4, vs));
                }
                ld_k(nxt, cn, t, k);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
        ld_rest(nxt, cn);
        lds_barrier();
    };
    for (int c = 0;;) {
        chunk(c, o0, o1);
        if (++c >= n) break;
        chunk(c, o1, o0);
        if (++c >= n) break;
    }
}

// reverse: every chunk's exit-state gradient dS' and dvn, and ds0; same grid and layout
template <int D>
__device__ __forceinline__ void walk_bwd(const GdnBwdArgs& a, int strip) {
    constexpr int NW = walk_nw<D>(), NTD = D / 16, RT = NTD / NW;
    constexpr int KH = NW / 4;
    constexpr int KD = D / 16 / KH, KC = BC / 16;
    constexpr int SW = walk_sw<D>(), NE = SW * RT * 4;
    const int b = blockIdx.x, g = blockIdx.y, col0 = strip * 16 * SW;
    const int lane = lane_id(), wv = wave_id(), i16 = lane & 15, q = lane >> 4;
    const int tq = wv & 3, kh = wv >> 2;
    const int G = a.G, n = a.n_chunks;
    __shared__ float LT[16 * SW][D + 4];
    __shared__ float VT[KH][16 * SW][BC + 4];
    auto erow = [&](int e) { return (wv * RT + (e / 4) % RT) * 16 + 4 * q + e % 4; };
    auto ecol = [&](int e) { return col0 + 16 * (e / (4 * RT)) + i16; };
    f32x4 L[SW][RT];
#pragma unroll
    for (int e = 0; e < NE; ++e) L[e / (4 * RT)][(e / 4) % RT][e % 4] = a.dsf ? a.dsf[(((long)b * G + g) * D + erow(e)) * D + ecol(e)] : 0.f;
    // one chunk's operands: kt row fragments of this wave's reduction part, w^T fragments of its row tiles, the E1
    // strip (part 0) and E2 rows, the chunk decay; two register sets, the next chunk's loads and this chunk's stores
    // issued one per MFMA step as in the forward walk
    struct Ops {
        float4 kf[KD], wf[RT][KC];
        float e1[SW][4], e2[SW][RT][4], gl;
    };
    auto ld_k = [&](Ops& o, long cg, int k) {
        o.kf[k] = *reinterpret_cast<const float4*>(a.ktlF + cg * BC * D + (long)(tq * (D / 16) + kh * (D / KH / 16) + k) * 256 + 4 * lane);
    };
    auto ld_w = [&](Ops& o, long cg, int t, int k) {
        o.wf[t][k] = *reinterpret_cast<const float4*>(a.wTF + cg * D * BC + (long)((wv * RT + t) * (BC / 16) + k) * 256 + 4 * lane);
    };
    auto ld_rest = [&](Ops& o, long cg) {
#pragma unroll
        for (int e = 0; e < NE; ++e) o.e2[e / (4 * RT)][(e / 4) % RT][e % 4] = a.E2[(cg * D + erow(e)) * D + ecol(e)];
#pragma unroll
        for (int c2 = 0; c2 < SW; ++c2)
#pragma unroll
            for (int v = 0; v < 4; ++v)
                o.e1[c2][v] = kh == 0 ? a.E1[(cg * BC + 16 * tq + 4 * q + v) * D + col0 + 16 * c2 + i16] : 0.f;
        o.gl = a.gam[cg * BC + BC - 1];
    };
    Ops o0, o1;
    {
        const long cg = ((long)b * n + n - 1) * G + g;
#pragma unroll
        for (int k = 0; k < KD; ++k) ld_k(o0, cg, k);
#pragma unroll
        for (int t = 0; t < RT; ++t)
#pragma unroll
            for (int k = 0; k < KC; ++k) ld_w(o0, cg, t, k);
        ld_rest(o0, cg);
    }
    auto chunk = [&](int c, const Ops& cur, Ops& nxt) {
        const long cg = ((long)b * n + c) * G + g;
        const long cn = ((long)b * n + (c > 0 ? c - 1 : c)) * G + g;       // the next chunk down (0 refetches)
#pragma unroll
        for (int e = 0; e < NE; ++e) LT[16 * (e / (4 * RT)) + i16][erow(e)] = L[e / (4 * RT)][(e / 4) % RT][e % 4];
        lds_barrier();
        wait_vmem_all();                                   // this chunk's operands (and the last chunk's stores)
        // dvn rows [16 tq, 16 tq + 16) = E1 + kt dS', this wave's part of the reduction; the next chunk's kt rows and
        // this chunk's exit-state gradient stores ride along
        f32x4 part[SW][4];
#pragma unroll
        for (int c2 = 0; c2 < SW; ++c2) {
            part[c2][0] = f32x4{cur.e1[c2][0], cur.e1[c2][1], cur.e1[c2][2], cur.e1[c2][3]};
#pragma unroll
            for (int p = 1; p < 4; ++p) part[c2][p] = f32x4{0.f, 0.f, 0.f, 0.f};
        }
#pragma unroll
        for (int k = 0; k < KD; ++k) {
#pragma unroll
            for (int c2 = 0; c2 < SW; ++c2) {
                const uint4 bf = *reinterpret_cast<const uint4*>(&LT[16 * c2 + i16][kh * (D / KH) + 16 * k + 4 * q]);
                mma<F32>(part[c2][k & 3], __builtin_bit_cast(uint4, cur.kf[k]), bf);
            }
            ld_k(nxt, cn, k);
#pragma unroll
            for (int e = k * NE / KD; e < (k + 1) * NE / KD; ++e)              // exit-state gradient of chunk c
                a.dSx[(cg * D + erow(e)) * D + ecol(e)] = L[e / (4 * RT)][(e / 4) % RT][e % 4];
            __builtin_amdgcn_sched_barrier(0);
        }
#pragma unroll
        for (int c2 = 0; c2 < SW; ++c2) {
            const f32x4 acc = (part[c2][0] + part[c2][1]) + (part[c2][2] + part[c2][3]);
#pragma unroll
            for (int v = 0; v < 4; ++v) VT[kh][16 * c2 + i16][16 * tq + 4 * q + v] = acc[v];
        }
        lds_barrier();
        // dvn (the sum of the parts) out; dS = e^(gc_C') dS' + E2 - w^T dvn; the next chunk's w^T rides along
        if (kh == 0) {
#pragma unroll
            for (int c2 = 0; c2 < SW; ++c2)
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    float x = VT[0][16 * c2 + i16][16 * tq + 4 * q + v];
#pragma unroll
                    for (int p = 1; p < KH; ++p) x += VT[p][16 * c2 + i16][16 * tq + 4 * q + v];
                    a.dvn[(cg * BC + 16 * tq + 4 * q + v) * D + col0 + 16 * c2 + i16] = x;
                }
        }
        const float ec = expf(cur.gl);
#pragma unroll
        for (int t = 0; t < RT; ++t) {
#pragma unroll
            for (int c2 = 0; c2 < SW; ++c2)
#pragma unroll
                for (int v = 0; v < 4; ++v) L[c2][t][v] = ec * L[c2][t][v] + cur.e2[c2][t][v];
#pragma unroll
            for (int k = 0; k < KC; ++k) {
                const uint4 af = make_uint4(__float_as_uint(-cur.wf[t][k].x), __float_as_uint(-cur.wf[t][k].y),
                                            __float_as_uint(-cur.wf[t][k].z), __float_as_uint(-cur.wf[t][k].w));
#pragma unroll
                for (int c2 = 0; c2 < SW; ++c2) {
                    float4 vs = *reinterpret_cast<const float4*>(&VT[0][16 * c2 + i16][16 * k + 4 * q]);
#pragma unroll
                    for (int p = 1; p < KH; ++p) {
                        const float4 x = *reinterpret_cast<const float4*>(&VT[p][16 * c2 + i16][16 * k + 4 * q]);
                        vs.x += x.x; vs.y += x.y; vs.z += x.z; vs.w += x.w;
                    }
                    mma<F32>(L[c2][t], af, __builtin_bit_cast(uint4, vs));
                }
                ld_w(nxt, cn, t, k);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
        ld_rest(nxt, cn);
        lds_barrier();
    };
    for (int c = n - 1;;) {
        chunk(c, o0, o1);
        if (--c < 0) break;
        chunk(c, o1, o0);
        if (--c < 0) break;
    }
    if (a.ds0)
#pragma unroll
        for (int e = 0; e < NE; ++e)
            a.ds0[(((long)b * G + g) * D + erow(e)) * D + ecol(e)] = L[e / (4 * RT)][(e / 4) % RT][e % 4];
}

// the two walks are independent (the reverse one needs E1, E2, kt, w, not the entry states): separate launches, so
// each starts as soon as its own operands exist and the products around it fill the CUs the walks leave idle
template <int D>
__global__ __launch_bounds__(64 * walk_nw<D>()) void walk_fwd_kernel(GdnBwdArgs a) { walk_fwd<D>(a, blockIdx.z); }
template <int D>
__global__ __launch_bounds__(64 * walk_nw<D>()) void walk_bwd_kernel(GdnBwdArgs a) { walk_bwd<D>(a, blockIdx.z); }


// ------------------------------------------------------------------------------------ final assembly
// grid (chunks, G, 4): rows r0 .. r0 + 15 of (chunk, KV head): dk, dv, d beta, and each row's share
// of d gc (into dgz, which holds the decay's share); the last row's extra terms (sum dkt kt and e^(gc_C') <S, dS'>,
// the latter over a quarter of the D x D entries) into part[cg][z]
__global__ __launch_bounds__(BW_NT) void chunk_final_kernel(GdnBwdArgs a) {
    const long bc = blockIdx.x;
    const int g = blockIdx.y, z = blockIdx.z, r0 = z * 16, tid = threadIdx.x, lane = lane_id(), wv = wave_id();
    const int D = a.D, G = a.G, R = a.R;
    const long cg = bc * G + g;
    __shared__ float gc[BC], red[BW_NT / 64];
    if (tid < BC) gc[tid] = a.gam[cg * BC + tid];
    __syncthreads();
    const float gl = gc[BC - 1];
    float ktsum = 0.f;
    for (int i = r0 + wv; i < r0 + 16; i += BW_NT / 64) {
        const long tok = bc * BC + i;
        const float egi = expf(gc[i]), eti = expf(gl - gc[i]);
        const float be = a.beta[tok * G + g];
        // the query path's share: s e^gc sum_r dqd_r . q_r, from the row-dot partials of the dqd products
        float dgi = 0.f, dbi = 0.f;
        for (int e = lane; e < R * (D / 64); e += 64) dgi += a.qdot[(cg * R * (D / 64) + e) * BC + i];
        // the decay's share: row minus column sums of dP . P and of dQK_r . QK_r (dP = the gradient of the
        // decayed strict-lower A, dQK_r of attn_r), from the epilogues of the dA and dattn products
        if (lane == 0) dgi += a.zrA[cg * BC + i] - a.zcA[cg * BC + i];
        for (int r = lane; r < R; r += 64) dgi += a.zr[(cg * R + r) * BC + i] - a.zc[(cg * R + r) * BC + i];
        for (int d = 4 * lane; d < D; d += 256) {          // four dims per lane, 16-byte accesses
            const long o = (cg * BC + i) * D + d, ot = (tok * G + g) * D + d;
            auto ld = [&](const float* p) {
                const float4 x = *reinterpret_cast<const float4*>(p);
                return std::array<float, 4>{x.x, x.y, x.z, x.w};
            };
            const auto dkt = ld(a.dkt + o), kt = ld(a.ktl + o), dkbe = ld(a.dkbe + o), dkb = ld(a.dkb + o);
            const auto kx = ld(a.k + ot), vx = ld(a.v + ot), dvb = ld(a.dvb + o), kbe = ld(a.kbe + o);
            const auto dka = ld(a.dkacc + o);
            float dk[4], dv[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const float dkbt = dkb[u] + dkbe[u] * egi;
                dgi += dkbe[u] * kbe[u] - dkt[u] * kt[u];
                ktsum += dkt[u] * kt[u];
                dbi += dkbt * kx[u] + dvb[u] * vx[u];
                dk[u] = dka[u] + dkt[u] * eti + dkbt * be;
                dv[u] = dvb[u] * be;
            }
            *reinterpret_cast<float4*>(a.dk + ot) = make_float4(dk[0], dk[1], dk[2], dk[3]);
            *reinterpret_cast<float4*>(a.dv + ot) = make_float4(dv[0], dv[1], dv[2], dv[3]);
        }
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) {
            dgi += __shfl_xor(dgi, off);
            dbi += __shfl_xor(dbi, off);
        }
        if (lane == 0) {
            a.dgz[cg * BC + i] = dgi;
            a.dbeta[tok * G + g] = dbi;
        }
    }
    float t = ktsum;
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) t += __shfl_xor(t, off);
    if (lane == 0) red[wv] = t;
    __syncthreads();
    if (tid == 0) {
        float s = 0.f;
        for (int w = 0; w < BW_NT / 64; ++w) s += red[w];
        a.part[cg * 4 + z] = s;
    }
}

// grid (chunks, G, 4): the state path's share of the last row's d gc, e^(gc_C') <S, dS'>, over a quarter of the D x D
// entries into psd[cg][z] (it needs only the two walks, so it runs beside the products that follow them)
__global__ __launch_bounds__(BW_NT) void state_dot_kernel(GdnBwdArgs a) {
    const long bc = blockIdx.x;
    const int g = blockIdx.y, z = blockIdx.z, tid = threadIdx.x, lane = lane_id(), wv = wave_id();
    const int D = a.D, G = a.G;
    const long cg = bc * G + g;
    __shared__ float red[BW_NT / 64];
    float sdot = 0.f;
    const long q4 = (long)D * D / 16;                     // this quarter's 16-byte pieces of S and dS'
    const float4* S4 = reinterpret_cast<const float4*>(a.Sc + cg * D * D) + z * q4;
    const float4* X4 = reinterpret_cast<const float4*>(a.dSx + cg * D * D) + z * q4;
    // four iterations' loads issued together over the whole multiples of 4 BW_NT, then the rest one at a time
    const long q4u = q4 - q4 % (4 * BW_NT);
    for (long e = tid; e < q4u; e += 4 * BW_NT) {
        float4 x[4], y[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            x[u] = S4[e + u * BW_NT];
            y[u] = X4[e + u * BW_NT];
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) sdot += (x[u].x * y[u].x + x[u].y * y[u].y) + (x[u].z * y[u].z + x[u].w * y[u].w);
    }
    for (long e = q4u + tid; e < q4; e += BW_NT) {
        const float4 x = S4[e], y = X4[e];
        sdot += (x.x * y.x + x.y * y.y) + (x.z * y.z + x.w * y.w);
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) sdot += __shfl_xor(sdot, off);
    if (lane == 0) red[wv] = sdot;
    __syncthreads();
    if (tid == 0) {
        float s_ = 0.f;
        for (int w = 0; w < BW_NT / 64; ++w) s_ += red[w];
        a.psd[cg * 4 + z] = s_ * expf(a.gam[cg * BC + BC - 1]);
    }
}

// per (chunk, KV head), one wave: dg_j = sum_{i >= j} d gc_i (the last row with its extra terms)
__global__ __launch_bounds__(64) void dg_scan_kernel(GdnBwdArgs a) {
    const long cg = blockIdx.x;
    const int tid = threadIdx.x, G = a.G;
    const long bc = cg / G;
    const int g = (int)(cg % G);
    float x = a.dgz[cg * BC + BC - 1 - tid];
    if (tid == 0)
        x += (a.part[cg * 4] + a.part[cg * 4 + 1]) + (a.part[cg * 4 + 2] + a.part[cg * 4 + 3]) +
             (a.psd[cg * 4] + a.psd[cg * 4 + 1]) + (a.psd[cg * 4 + 2] + a.psd[cg * 4 + 3]);
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const float y = __shfl_up(x, off);
        if (tid >= off) x += y;
    }
    a.dg[(bc * BC + (BC - 1 - tid)) * G + g] = x;
}

// ------------------------------------------------------------------------------------ host side
int bgemm(const BgArgs& a, hipStream_t s) {
    // each operand must be contiguous along k or along its other dimension (16-byte tile loads)
    if ((a.ak != 1 && a.am != 1) || (a.bk != 1 && a.bn != 1)) return BF_ERR_UNSUPPORTED;
    if (a.M % 64 || a.N % 64 || a.K % 32 || a.K <= 0) return BF_ERR_UNSUPPORTED;
    if ((a.rdo || a.cdo || a.dgc || a.cfrag) && a.cn != 1) return BF_ERR_UNSUPPORTED;
    if (a.cfrag && (a.acc || a.add || a.rdo || a.cdo)) return BF_ERR_UNSUPPORTED;
    // 16-byte row pieces of C, the addend and rdx when C is contiguous along n
    if (a.cn == 1 && ((a.cm | a.sc0 | a.sc1 | a.sc2) % 4)) return BF_ERR_UNSUPPORTED;
    const bool ak = a.ak == 1, bk = a.bk == 1;
    const int ex = a.dgc || a.cdo ? 2 : a.msc || a.rdo || a.cfrag ? 1 : 0;
    auto go = [&](auto kern, int bn) {
        hipLaunchKernelGGL(kern, dim3((unsigned)a.nz, a.M / 64, a.N / bn), dim3(BW_NT), 0, s, a);
    };
#define BG_GO(BN, EX)                                                                         \
    do {                                                                                      \
        if (ak && bk) go(bgemm_kernel<true, true, BN, EX>, BN);                               \
        else if (ak) go(bgemm_kernel<true, false, BN, EX>, BN);                               \
        else if (bk) go(bgemm_kernel<false, true, BN, EX>, BN);                               \
        else go(bgemm_kernel<false, false, BN, EX>, BN);                                      \
    } while (0)
    if (a.N % 128 == 0) {
        if (ex == 2) BG_GO(128, 2);
        else if (ex == 1) BG_GO(128, 1);
        else BG_GO(128, 0);
    } else {
        if (ex == 2) BG_GO(64, 2);
        else if (ex == 1) BG_GO(64, 1);
        else BG_GO(64, 0);
    }
#undef BG_GO
    return (int)hipGetLastError();
}

// a matrix operand: base pointer, batch strides over (chunk, KV head, query head), row and column strides
struct Op {
    const float* p;
    long s0, s1, s2, rs, cs;
};

// a split reduction index k = (kh, kl), kl < 2^shift: the operands' strides of kh, and the optional column scale
// of A (ksc[z0 s0 + z1 s1 + kl])
struct KSplit {
    int shift = 30;
    long a = 0, b = 0;
    const float* ksc = nullptr;
    long s0 = 0, s1 = 0;
};

// epilogue extras: a row scale msc[z0 s0 + z1 s1 + m], the in-chunk decay from dgc[z0 g0 + z1 g1 + .], and the row /
// column dots with rdx into rdo / cdo
struct Epi {
    const float* msc = nullptr;
    long s0 = 0, s1 = 0;
    const float* dgc = nullptr;
    long g0 = 0, g1 = 0;
    const float* rdx = nullptr;
    float* rdo = nullptr;
    float* cdo = nullptr;
    int frag = 0;
};

// C (M x N) per (chunk, g[, r]) = add + alpha * A B, with A, B given as Op (transposes by swapping strides)
int gemm(int M, int N, int K, int nz, int n1, int n2, Op A, Op B, float* C, long c0, long c1, long c2, long cm,
         long cn, float alpha, int acc, int mask, const float* add, hipStream_t s, const KSplit& ks = KSplit{},
         const Epi& ep = Epi{}) {
    BgArgs g{};
    g.M = M; g.N = N; g.K = K; g.n1 = n1; g.n2 = n2; g.nz = nz; g.kshift = ks.shift;
    g.A = A.p; g.sa0 = A.s0; g.sa1 = A.s1; g.sa2 = A.s2; g.am = A.rs; g.ak = A.cs; g.sak = ks.a;
    g.B = B.p; g.sb0 = B.s0; g.sb1 = B.s1; g.sb2 = B.s2; g.bk = B.rs; g.bn = B.cs; g.sbk = ks.b;
    g.C = C; g.sc0 = c0; g.sc1 = c1; g.sc2 = c2; g.cm = cm; g.cn = cn;
    g.ksc = ks.ksc; g.ks0 = ks.s0; g.ks1 = ks.s1;
    g.msc = ep.msc; g.ms0 = ep.s0; g.ms1 = ep.s1; g.dgc = ep.dgc; g.dg0 = ep.g0; g.dg1 = ep.g1;
    g.rdx = ep.rdx; g.rdo = ep.rdo; g.cdo = ep.cdo; g.cfrag = ep.frag;
    g.alpha = alpha; g.acc = acc; g.mask = mask; g.add = add;
    if (ks.shift < 30 && ((1 << ks.shift) % 16 != 0 || K % (1 << ks.shift) != 0)) return BF_ERR_UNSUPPORTED;
    return bgemm(g, s);
}

Op tr(Op o) { std::swap(o.rs, o.cs); return o; }

// The backward's second stream on each device (default priority, created on a device's first call) and the events
// that order it against the caller's stream. The caller holds g_bwd_mu over a call's whole enqueue, so the records and
// waits of concurrent calls from several host threads do not interleave.
constexpr int kBwdMaxDevices = 64;
struct BwdSide {
    hipStream_t s = nullptr;
    hipEvent_t ev[7] = {};
};
std::mutex g_bwd_mu;
BwdSide g_bwd_side[kBwdMaxDevices];

int side_stream(hipStream_t& s2, hipEvent_t (&ev)[7]) {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return (int)e;
    if (dev < 0 || dev >= kBwdMaxDevices) return BF_ERR_UNSUPPORTED;
    BwdSide& sd = g_bwd_side[dev];
    for (hipEvent_t& x : sd.ev)
        if (!x && (e = hipEventCreateWithFlags(&x, hipEventDisableTiming)) != hipSuccess) return (int)e;
    if (!sd.s && (e = hipStreamCreateWithFlags(&sd.s, hipStreamNonBlocking)) != hipSuccess) return (int)e;
    s2 = sd.s;
    for (int i = 0; i < 7; ++i) ev[i] = sd.ev[i];
    return 0;
}

}  // namespace

size_t gdn_bwd_workspace(int num_seqs, long T, int G, int R, int D) {
    const long n = T / BC, NC = (long)num_seqs * n * G;             // chunk-heads
    const long cc = BC * BC, cd = (long)BC * D, dd = (long)D * D;
    const long floats = NC * (BC * 5 + 8                             // gam, eg, dgz, zrA, zcA, part, psd
                              + cc * 3                               // Am, M, dA
                              + cd * 10                              // kb, vb, kbe, ktl, u, w; ktl, kt^T, w, w^T in fragment order
                              + (long)R * (cc * 2 + (D / 64 + 2) * BC)   // attn, dattn; qdot, zr, zc
                              + dd * 3                               // Sc, E2, dSx
                              + cd * 9                               // E1, dvn, vn, dkt, dw, dvb, dkbe, dkb, dkacc
                              + cc * 2);                             // dM, T1
    return (size_t)floats * sizeof(float) + 256 * 49;                // each buffer rounded up to 256 bytes
}

int gdn_bwd(GdnBwdArgs a, void* ws, hipStream_t s) {
    std::lock_guard<std::mutex> lock(g_bwd_mu);
    const int D = a.D, G = a.G, R = a.R, H = G * R;
    const long n = a.n_chunks, NB = (long)a.num_seqs * n, NC = NB * G;
    const long cc = BC * BC, cd = (long)BC * D, dd = (long)D * D;
    char* p = static_cast<char*>(ws);
    auto take = [&](long count) {
        float* r = reinterpret_cast<float*>(p);
        p += ((count * (long)sizeof(float) + 255) / 256) * 256;
        return r;
    };
    a.gam = take(NC * BC); a.eg = take(NC * BC); a.dgz = take(NC * BC); a.part = take(NC * 4); a.psd = take(NC * 4);
    a.Am = take(NC * cc); a.Mi = take(NC * cc); a.dA = take(NC * cc);
    a.zrA = take(NC * BC); a.zcA = take(NC * BC); a.zr = take(NC * R * BC); a.zc = take(NC * R * BC);
    a.kb = take(NC * cd); a.vb = take(NC * cd); a.kbe = take(NC * cd); a.ktl = take(NC * cd);
    a.u = take(NC * cd); a.w = take(NC * cd);
    a.ktlF = take(NC * cd); a.ktlTF = take(NC * cd); a.wF = take(NC * cd); a.wTF = take(NC * cd);
    a.attn = take(NC * R * cc); a.dattn = take(NC * R * cc);
    a.qdot = take(NC * R * (D / 64) * BC);
    a.Sc = take(NC * dd); a.E2 = take(NC * dd); a.dSx = take(NC * dd);
    a.E1 = take(NC * cd); a.dvn = take(NC * cd); a.vn = take(NC * cd); a.dkt = take(NC * cd); a.dw = take(NC * cd);
    a.dvb = take(NC * cd); a.dkbe = take(NC * cd); a.dkb = take(NC * cd); a.dkacc = take(NC * cd);
    float* dM = take(NC * cc);
    float* T1 = take(NC * cc);

    int e = 0;
    auto ok = [&](int r) { if (r != 0 && e == 0) e = r; };
    // every product batches over z = (chunk, g, r) with n1 = G, n2 = R (or 1)
    // token-major inputs, chunk views: k [C x D] of (chunk, g); q_r, dO_r [C x D] of (chunk, g, r)
    auto kT = [&]() { return Op{a.k, (long)BC * G * D, D, 0, (long)G * D, 1}; };
    auto qR = [&]() { return Op{a.q, (long)BC * H * D, (long)R * D, D, (long)H * D, 1}; };   // q_r chunk
    auto dOR = [&]() { return Op{a.dO, (long)BC * H * D, (long)R * D, D, (long)H * D, 1}; }; // dO_r chunk
    // per (chunk, g) workspace arrays addressed with z = (chunk, g): s0 = G * size, s1 = size
    auto W = [&](const float* q, long rows, long cols) { return Op{q, (long)G * rows * cols, rows * cols, 0, cols, 1}; };
    auto WR = [&](const float* q, long rows, long cols) {
        return Op{q, (long)G * R * rows * cols, (long)R * rows * cols, rows * cols, cols, 1};
    };
    const int nzg = (int)NC, nzr = (int)(NC * R);

    hipStream_t s2 = nullptr;
    hipEvent_t ev[7] = {};
    ok(side_stream(s2, ev));
    if (e) return e;
    // prep
    hipLaunchKernelGGL(chunk_prep_kernel, dim3((unsigned)NB, G, 4), dim3(BW_NT), 0, s, a);
    ok((int)hipGetLastError());
    // Am = strict_lower((k b) k^T * decay)
    Epi dec;
    dec.dgc = a.gam; dec.g0 = (long)G * BC; dec.g1 = BC;
    ok(gemm(BC, BC, D, nzg, G, 1, W(a.kb, BC, D), tr(kT()), a.Am, (long)G * cc, cc, 0, BC, 1, 1.f, 0, 2, nullptr, s,
            KSplit{}, dec));
    hipLaunchKernelGGL(unit_lower_inverse_kernel, dim3((unsigned)NC), dim3(64), 0, s, a.Am, a.Mi);
    ok((int)hipGetLastError());
    // u = M (v b), w = M (k b e^gc)
    ok(gemm(BC, D, BC, nzg, G, 1, W(a.Mi, BC, BC), W(a.vb, BC, D), a.u, (long)G * cd, cd, 0, D, 1, 1.f, 0, 0, nullptr, s));
    ok(gemm(BC, D, BC, nzg, G, 1, W(a.Mi, BC, BC), W(a.kbe, BC, D), a.w, (long)G * cd, cd, 0, D, 1, 1.f, 0, 0, nullptr, s));
    Epi fr;
    fr.frag = 1;                                          // w and w^T in fragment order for the state walks
    ok(gemm(BC, D, BC, nzg, G, 1, W(a.Mi, BC, BC), W(a.kbe, BC, D), a.wF, (long)G * cd, cd, 0, D, 1, 1.f, 0, 0, nullptr,
            s, KSplit{}, fr));
    ok(gemm(D, BC, BC, nzg, G, 1, tr(W(a.kbe, BC, D)), tr(W(a.Mi, BC, BC)), a.wTF, (long)G * cd, cd, 0, BC, 1, 1.f, 0, 0,
            nullptr, s, KSplit{}, fr));                   // w^T = (k b e^gc)^T M^T
    // Side stream: the forward walk, then what needs only the entry states (v_new, dattn, dq). Main stream: attn, E1,
    // E2, the reverse walk, then what needs dS' and dvn, joining the side stream where its results are read.
    ok((int)hipEventRecord(ev[0], s));
    ok((int)hipStreamWaitEvent(s2, ev[0], 0));
    const dim3 wgrid(a.num_seqs, G, D / 16);               // walk_sw<D>() == 1: one workgroup per 16-column strip
    // The walks are the call's critical path on few workgroups: each asks for LDS up to 128 KB of the CU's 160 KB,
    // so no product workgroup (34-55 KB) shares its CU and slows it (2.11 -> 2.06 ms with the attn product after the
    // fork, T = 8192, G = 4, R = 6, D = 256)
    auto walk = [&](bool fwd, hipStream_t st) {
        const dim3 blk(64 * (D >= 128 ? 8 : 4));
        const int kh = D >= 128 ? 2 : 1;
        const size_t res = 128 * 1024 - (size_t)(16 * (D + 4) + kh * 16 * (BC + 4)) * sizeof(float);
        if (D == 64) hipLaunchKernelGGL(fwd ? walk_fwd_kernel<64> : walk_bwd_kernel<64>, wgrid, blk, res, st, a);
        else if (D == 128) hipLaunchKernelGGL(fwd ? walk_fwd_kernel<128> : walk_bwd_kernel<128>, wgrid, blk, res, st, a);
        else hipLaunchKernelGGL(fwd ? walk_fwd_kernel<256> : walk_bwd_kernel<256>, wgrid, blk, res, st, a);
        ok((int)hipGetLastError());
    };
    // attn_r = tril(s q_r k^T * decay)
    ok(gemm(BC, BC, D, nzr, G, R, qR(), tr(Op{a.k, (long)BC * G * D, D, 0, (long)G * D, 1}), a.attn, (long)G * R * cc,
            (long)R * cc, cc, BC, 1, a.scale, 0, 1, nullptr, s, KSplit{}, dec));
    ok((int)hipEventRecord(ev[4], s));                     // attn
    walk(true, s2);
    ok((int)hipEventRecord(ev[1], s2));                    // entry states Sc
    // v_new = u - w S
    ok(gemm(BC, D, D, nzg, G, 1, W(a.w, BC, D), W(a.Sc, D, D), a.vn, (long)G * cd, cd, 0, D, 1, -1.f, 0, 0, a.u, s2));
    ok((int)hipEventRecord(ev[2], s2));                    // v_new
    // dattn_r = tril(dO_r v_new^T); dqd_r = dO_r S^T goes straight into dq_r = s e^gc dqd_r (token-major; the attn
    // share is added below), with each row's dot with q_r (the query path's d gc share) as partials in qdot
    // (the decayed dattn_r; the decay's d gc share from dQK_r . QK_r = dattn_r(undecayed) . attn_r as row and column
    // sums)
    ok((int)hipStreamWaitEvent(s2, ev[4], 0));
    Epi da = dec;
    da.rdx = a.attn; da.rdo = a.zr; da.cdo = a.zc;
    ok(gemm(BC, BC, D, nzr, G, R, dOR(), tr(Op{a.vn, (long)G * cd, cd, 0, D, 1}), a.dattn, (long)G * R * cc,
            (long)R * cc, cc, BC, 1, 1.f, 0, 1, nullptr, s2, KSplit{}, da));
    // dk from attn: sum_r dattn_r^T (s q_r), K = R C (the share from A is added on the main stream)
    KSplit rk;
    rk.shift = 6; rk.a = cc; rk.b = D;                    // attn^T / dattn^T (chunk-major [r][i][j]) against dO or q
    const Op qk{a.q, (long)BC * H * D, (long)R * D, 0, (long)H * D, 1};
    ok(gemm(BC, D, R * BC, nzg, G, 1, tr(Op{a.dattn, (long)G * R * cc, (long)R * cc, 0, BC, 1}), qk, a.dkacc,
            (long)G * cd, cd, 0, D, 1, a.scale, 0, 0, nullptr, s2, rk));
    ok((int)hipEventRecord(ev[5], s2));                    // dkacc (attn share)
    Epi eq;
    eq.msc = a.eg; eq.s0 = (long)G * BC; eq.s1 = BC; eq.rdx = a.q; eq.rdo = a.qdot;
    ok(gemm(BC, D, D, nzr, G, R, dOR(), tr(Op{a.Sc, (long)G * dd, dd, 0, D, 1}), a.dq, (long)BC * H * D, (long)R * D, D,
            (long)H * D, 1, a.scale, 0, 0, nullptr, s2, KSplit{}, eq));
    // dq_r += s dattn_r k
    ok(gemm(BC, D, BC, nzr, G, R, WR(a.dattn, BC, BC), Op{a.k, (long)BC * G * D, D, 0, (long)G * D, 1}, a.dq,
            (long)BC * H * D, (long)R * D, D, (long)H * D, 1, a.scale, 1, 0, nullptr, s2));

    // E1 = sum_r attn_r^T dO_r [C x D], E2 = sum_r qd_r^T dO_r = s sum_r q_r^T diag(e^gc) dO_r [D x D]: one product
    // each over K = R C, the (r, token) pairs, read from the token-major q and dO (k = 64 r + i: token stride H D,
    // head stride D)
    const Op dOk{a.dO, (long)BC * H * D, (long)R * D, 0, (long)H * D, 1};
    ok(gemm(BC, D, R * BC, nzg, G, 1, tr(Op{a.attn, (long)G * R * cc, (long)R * cc, 0, BC, 1}), dOk, a.E1, (long)G * cd,
            cd, 0, D, 1, 1.f, 0, 0, nullptr, s, rk));
    KSplit rq;
    rq.shift = 6; rq.a = D; rq.b = D; rq.ksc = a.eg; rq.s0 = (long)G * BC; rq.s1 = BC;   // A = q^T, columns e^gc
    ok(gemm(D, D, R * BC, nzg, G, 1, tr(qk), dOk, a.E2, (long)G * dd, dd, 0, D, 1, a.scale, 0, 0, nullptr, s, rq));
    walk(false, s);
    // Side stream, after its products: the state path's d gc share, e^(gc_C') <S, dS'>, once the reverse walk has
    // written dS' (enqueued here, after that walk's record, so the wait binds to this call's walk)
    ok((int)hipEventRecord(ev[6], s));                     // dS'
    ok((int)hipStreamWaitEvent(s2, ev[6], 0));
    hipLaunchKernelGGL(state_dot_kernel, dim3((unsigned)NB, G, 4), dim3(BW_NT), 0, s2, a);
    ok((int)hipGetLastError());
    ok((int)hipEventRecord(ev[3], s2));                    // dattn, dq, qdot, zr, zc, psd
    // d(v b) = M^T dvn
    ok(gemm(BC, D, BC, nzg, G, 1, tr(W(a.Mi, BC, BC)), W(a.dvn, BC, D), a.dvb, (long)G * cd, cd, 0, D, 1, 1.f, 0, 0,
            nullptr, s));
    // dw = -dvn S^T, d(k b e^gc) = M^T dw
    ok((int)hipStreamWaitEvent(s, ev[1], 0));
    ok(gemm(BC, D, D, nzg, G, 1, W(a.dvn, BC, D), tr(W(a.Sc, D, D)), a.dw, (long)G * cd, cd, 0, D, 1, -1.f, 0, 0,
            nullptr, s));
    ok(gemm(BC, D, BC, nzg, G, 1, tr(W(a.Mi, BC, BC)), W(a.dw, BC, D), a.dkbe, (long)G * cd, cd, 0, D, 1, 1.f, 0, 0,
            nullptr, s));
    // dM = dvn (v b)^T + dw (k b e^gc)^T ; T1 = M^T dM ; dA = -strict_lower(T1 M^T)
    ok(gemm(BC, BC, D, nzg, G, 1, W(a.dvn, BC, D), tr(W(a.vb, BC, D)), dM, (long)G * cc, cc, 0, BC, 1, 1.f, 0, 0,
            nullptr, s));
    ok(gemm(BC, BC, D, nzg, G, 1, W(a.dw, BC, D), tr(W(a.kbe, BC, D)), dM, (long)G * cc, cc, 0, BC, 1, 1.f, 1, 0,
            nullptr, s));
    ok(gemm(BC, BC, BC, nzg, G, 1, tr(W(a.Mi, BC, BC)), W(dM, BC, BC), T1, (long)G * cc, cc, 0, BC, 1, 1.f, 0, 0,
            nullptr, s));
    // (written decayed, the decay's d gc share from dP . P = dA(undecayed) . Am as row and column sums)
    Epi dd_ = dec;
    dd_.rdx = a.Am; dd_.rdo = a.zrA; dd_.cdo = a.zcA;
    ok(gemm(BC, BC, BC, nzg, G, 1, W(T1, BC, BC), tr(W(a.Mi, BC, BC)), a.dA, (long)G * cc, cc, 0, BC, 1, -1.f, 0, 2,
            nullptr, s, KSplit{}, dd_));
    // d(k b) from A: dAd k ; dk from A: dAd^T (k b), added to the attn share
    ok(gemm(BC, D, BC, nzg, G, 1, W(a.dA, BC, BC), kT(), a.dkb, (long)G * cd, cd, 0, D, 1, 1.f, 0, 0, nullptr, s));
    ok((int)hipStreamWaitEvent(s, ev[5], 0));
    ok(gemm(BC, D, BC, nzg, G, 1, tr(W(a.dA, BC, BC)), W(a.kb, BC, D), a.dkacc, (long)G * cd, cd, 0, D, 1, 1.f, 1, 0,
            nullptr, s));
    // dkt = v_new dS'^T
    ok((int)hipStreamWaitEvent(s, ev[2], 0));
    ok(gemm(BC, D, D, nzg, G, 1, W(a.vn, BC, D), tr(W(a.dSx, D, D)), a.dkt, (long)G * cd, cd, 0, D, 1, 1.f, 0, 0,
            nullptr, s));
    ok((int)hipStreamWaitEvent(s, ev[3], 0));             // the side stream's dq, qdot, zr, zc
    hipLaunchKernelGGL(chunk_final_kernel, dim3((unsigned)NB, G, 4), dim3(BW_NT), 0, s, a);
    hipLaunchKernelGGL(dg_scan_kernel, dim3((unsigned)NC), dim3(64), 0, s, a);
    ok((int)hipGetLastError());
    return e;
}

}  // namespace bf
