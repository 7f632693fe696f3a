// K1 part 2: the sequential part of the chunked gated delta rule, cut into segments that are scanned in parallel.
//
// With T' = (I + A)^-1 diag(beta), gc and attn from gdn_prefill.hip, one chunk of KV head g maps the state S
// (D x D, fp32) as (reference: Heimdall/heimdall/kernels.py:112-127, motor.py:86-100)
//   Y = K S,   v_new = T' (V - e^{gc} Y),   o_r = scale e^{gc} q_r S + attn_r v_new,
//   S' = e^{gc_last} S + K^T (e^{gc_last - gc} v_new).
// S' is affine in S, so each sequence is cut into segments of L chunks and three kernels run in turn:
//   gdn_seg_kernel<.., OUT=false>  (summary) per (segment, KV head, column group): the chunk map applied to the 2D
//                       columns [N | Phi] from [0 | I], with V for the N columns and zero for the Phi columns, gives the
//                       segment's map S_end = Phi S_start + N (the last segment of a sequence is skipped).
//   gdn_combine_kernel  per (sequence, KV head, 16-column strip): X_0 = S0, X_{p+1} = Phi_p X_p + N_p in fp32
//                       (bf16 runs: Psi = Phi - cI in bf16 times X split into bf16 high and low parts, plus the exact
//                       c X term), the entry state of every segment.
//   gdn_seg_kernel<.., OUT=true>   (output) per (segment, KV head, column group): the chunk map with outputs of all R
//                       query heads of the KV head from the segment's entry state; the last segment of a sequence
//                       writes the final state.
// Inside a workgroup each wave owns 16 state columns (one 16-column MFMA tile) for all D rows, held in registers as
// MFMA accumulators, so the per-chunk chain runs inside the wave with no exchange between waves:
//   K S, q S      A = K / q rows (LDS),     B = S packed from the accumulators
//   T' y          A = T' fragments (LDS),   B = the Y accumulators after y = V - e^{gc} Y
//   attn_r        A = K rows, B = q_r rows (LDS): attn_r^T tiles, masked and decayed into attn_r's A fragments
//   attn_r v_new  A = attn_r fragments (LDS, written by the waves),  B = the v_new accumulators
//   K^T v'        A = K^T through transposing reads of the K tile in LDS,  B = the v_new accumulators scaled by
//                 e^{gc_last - gc}
// An accumulator tile holds rows 4g..4g+3 of its 16 rows in lane group g, while an MFMA operand fragment holds VEC
// consecutive K indices per lane group. Tiles over the token and state-row dimensions therefore use the row
// permutation prow(tile, m): rows 4g..4g+3 of the HP = VEC/4 tiles of one K fragment are that fragment's VEC values
// of group g, so accumulators feed the next product directly. A rows are read through the same permutation.
//
// The chunk operands all waves share (K, q, T', gc, V) are staged in LDS with buffer_load ... lds (no registers,
// out-of-range rows read as zero); bf16 runs double-buffer the stage so chunk c+1 is in flight while chunk c is
// computed. K, q and V rows are swizzled by 16-byte blocks (swz) so that the fragment reads of 16 rows hit distinct
// banks; T' and attn are kept in fragment order (tfrag_index), one contiguous 1 KB per fragment.
//
// The output scan runs the R query heads of a KV head inside one workgroup: the chunk's K S, T' y and K^T v' products
// are shared, and per query head the waves form the causal block attn_r = scale (q_r K^T e^{gc_i - gc_j})[i >= j]
// (its nonzero A fragments, one per wave) into LDS, then o_r = scale e^{gc} q_r S + attn_r v_new. bf16 runs double
// buffer q so that head r + 1 loads while head r is computed, and write o_r while head r + 1 is computed.
#include <type_traits>

#include "bf_common.h"
#include "bf_internal.h"

namespace bf {

namespace {

constexpr int SC = 64;       // chunk length
constexpr int NXCD = 8;      // XCDs of an MI355X: workgroups are dispatched round-robin over them by linear id
// State columns per wave (one or two 16-column MFMA tiles) and columns per workgroup. 16 columns per wave keep a
// wave under 256 registers, so two waves share a SIMD and one's MFMA work overlaps the other's VALU and LDS work.
constexpr int WCOLS = 16;
constexpr int NJ = WCOLS / 16;
constexpr int WG_COLS = 128;
constexpr int SEG_THREADS = WG_COLS / WCOLS * 64;
constexpr int SEG_WAVES_PER_EU = SEG_THREADS / 256;

// Nonzero A fragments (token tile b, K step ks) of the causal 64 x 64 attn block: K step ks covers tokens KF*ks ..
// KF*ks + KF - 1, which reach the tile's last token 16b + 15 for ks <= (16b + 15) / KF. Fragments are numbered tile by
// tile (attn_fidx); the others are all zero and skipped.
template <class E>
__device__ __forceinline__ constexpr int attn_nks(int b) { return (16 * b + 15) / E::KF + 1; }
template <class E>
__device__ __forceinline__ constexpr int attn_fidx(int b, int ks) {
    int n = 0;
    for (int bb = 0; bb < b; ++bb) n += attn_nks<E>(bb);
    return n + ks;
}
template <class E>
constexpr int attn_frags() {
    int n = 0;
    for (int b = 0; b < SC / 16; ++b) n += (16 * b + 15) / E::KF + 1;
    return n;
}

template <class E>
__device__ __forceinline__ int prow(int tile, int m) {
    constexpr int VEC = E::VEC, KF = E::KF, HP = VEC / 4;
    return KF * (tile / HP) + VEC * (m >> 2) + 4 * (tile % HP) + (m & 3);
}

// Per-chunk stage: K, gc and (TP) T'.
template <class E, int D, bool TP>
struct __align__(16) ChunkLds {
    typename E::T K[SC * D];
    typename E::T Tp[TP ? SC * SC : 8];
    float gc[SC];
};
// Operands outside the chunk stage: NQ q buffers (bf16 output scan), the V columns of the workgroup, the attn
// fragments of one query head (NAT elements, output scan) and (TP) a single T' buffer (bf16 output scan). V and T' are
// reloaded for the next chunk as soon as the current chunk has consumed them.
template <class E, int D, int NQ, int VW, int NAT, bool TP>
struct __align__(16) OnceLds {
    typename E::T Q[NQ > 0 ? NQ : 1][NQ > 0 ? SC * D : 8];
    typename E::T V[SC * VW];
    typename E::T At[NAT > 0 ? NAT : 8];
    typename E::T Tp[TP ? SC * SC : 8];
};
struct __align__(16) NoLds {
    float pad[4];
};

// B operand (K index = accumulator rows) from the HP accumulator tiles of one fragment.
template <class E>
__device__ __forceinline__ uint4 pack_b(const f32x4& a, const f32x4& b);
template <>
__device__ __forceinline__ uint4 pack_b<F32>(const f32x4& a, const f32x4&) {
    return make_uint4(__float_as_uint(a[0]), __float_as_uint(a[1]), __float_as_uint(a[2]), __float_as_uint(a[3]));
}
template <>
__device__ __forceinline__ uint4 pack_b<BF16>(const f32x4& a, const f32x4& b) {
    return make_uint4(pack_bf16x2(a[0], a[1]), pack_bf16x2(a[2], a[3]), pack_bf16x2(b[0], b[1]), pack_bf16x2(b[2], b[3]));
}

// Psi = Phi - cI of a segment map is stored in MFMA fragment order, so that the combine kernel's A-fragment loads are
// contiguous 1 KB pieces (an A fragment read straight from a row-major matrix touches 16 rows x 64 bytes per
// instruction, about 4x slower from L2). Element (d, j) sits in fragment (tile d / 16, k step j / KF) at lane
// 16 * ((j % KF) / VEC) + d % 16, element j % VEC.
template <class E, int D>
__device__ __forceinline__ long psi_frag_index(int d, int j) {
    constexpr int VEC = E::VEC, KF = E::KF, NKD = D / KF;
    const int lane = 16 * ((j % KF) / VEC) + (d & 15);
    return ((long)((d >> 4) * NKD + j / KF) * 64 + lane) * VEC + j % VEC;
}

// N and the segment entry states (fp32 D x D) are stored in accumulator-fragment order: element (d, j) sits in the
// 16 x 16 tile (d / 16, j / 16) at lane 16 * ((d % 16) / 4) + j % 16, element d % 4, so the combine kernel reads and
// writes each tile of a 16-column strip as one contiguous float4 per lane.
template <int D>
__device__ __forceinline__ long acc_frag_index(int d, int j) {
    const int lane = 16 * ((d & 15) >> 2) + (j & 15);
    return ((long)((d >> 4) * (D / 16) + (j >> 4)) * 64 + lane) * 4 + (d & 3);
}

struct SegInfo {
    int n;        // sequence
    int p;        // segment index inside the sequence
    int nseg;     // segments of the sequence
    int cid0;     // chunk id of the segment's first chunk
    int count;    // chunks in the segment (0 only for an empty sequence)
    long tok0;    // first token of the segment
    long tok1;    // end of the sequence (exclusive)
};

__device__ __forceinline__ void seq_bounds(const GdnArgs& a, int n, long& s0, long& s1) {
    s0 = a.cu_seqlens ? (long)a.cu_seqlens[n] : (long)n * a.seq_len;
    s1 = a.cu_seqlens ? (long)a.cu_seqlens[n + 1] : (long)(n + 1) * a.seq_len;
}

// Segments enumerate sequence 0's segments, then sequence 1's, ...; an empty sequence has one empty segment.
__device__ __forceinline__ bool locate_segment(const GdnArgs& a, int sid, SegInfo& s) {
    const int L = a.seg_chunks;
    int base_seg = 0, base_cid = 0;
    for (int n = 0; n < a.num_seqs; ++n) {
        long s0, s1;
        seq_bounds(a, n, s0, s1);
        const int nc = (int)((s1 - s0 + SC - 1) / SC);
        const int ns = nc > 0 ? (nc + L - 1) / L : 1;
        if (sid < base_seg + ns) {
            const int p = sid - base_seg;
            s.n = n;
            s.p = p;
            s.nseg = ns;
            s.cid0 = base_cid + p * L;
            s.count = nc - p * L < L ? nc - p * L : L;
            s.tok0 = s0 + (long)p * L * SC;
            s.tok1 = s1;
            return true;
        }
        base_seg += ns;
        base_cid += nc;
    }
    return false;
}

__device__ __forceinline__ void seq_segments(const GdnArgs& a, int n, int& first_sid, int& nseg) {
    const int L = a.seg_chunks;
    int base = 0;
    for (int m = 0; m <= n; ++m) {
        long s0, s1;
        seq_bounds(a, m, s0, s1);
        const int nc = (int)((s1 - s0 + SC - 1) / SC);
        const int ns = nc > 0 ? (nc + L - 1) / L : 1;
        if (m == n) {
            first_sid = base;
            nseg = ns;
        }
        base += ns;
    }
}

template <class E, int D, bool OUT>
struct SegCfg {
    static constexpr int COLS = OUT ? D : 2 * D;                    // state columns per (segment, KV head)
    static constexpr int NW = (COLS < WG_COLS ? COLS : WG_COLS) / WCOLS;  // waves per workgroup
    static constexpr int NCG = COLS / (NW * WCOLS);                 // column groups (workgroups per head)
    static constexpr bool DBUF = E::VEC == 8;                       // bf16: double-buffered stage
    static constexpr bool TPS = !(OUT && DBUF);                      // T' in the chunk stage (else single-buffered)
};

}  // namespace

// ------------------------------------------------------------------------------------------------ segment scan
// Addressing. With tp(tile) = KF*(tile/HP) + 4*(tile%HP) and lt = VEC*(l16/4) + l16%4, a fragment row is
// prow(tile, l16) = tp(tile) + lt and an accumulator row is prow(tile, 4lg + i) = tp(tile) + VEC*lg + i. Every LDS and
// global offset below is split into a per-lane part (computed once) and a part that depends only on unrolled loop
// indices (an instruction immediate or a scalar offset), so the chunk loop keeps a handful of address registers.
// GatedNorm of one bf16 row held by LPR consecutive lanes, 8 channels each (the arithmetic of gated_norm_kernel with
// bf16 rows, Heimdall/heimdall/hibrit.py:118-129): out = bf16(bf16(w bf16(o rsqrt(mean(o^2) + eps))) SiLU(z)).
template <int LPR>
__device__ __forceinline__ uint4 gated_norm_row(const uint4& ov, const uint4& zv, const float (&w)[8], float eps,
                                                int D) {
    auto unpack = [](const uint4& u, float (&x)[8]) {
        const uint32_t q[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            x[2 * i] = __uint_as_float(q[i] << 16);
            x[2 * i + 1] = __uint_as_float(q[i] & 0xffff0000u);
        }
    };
    float o[8], z[8];
    unpack(ov, o);
    unpack(zv, z);
    float ss = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) ss += o[e] * o[e];
#pragma unroll
    for (int m = LPR / 2; m >= 1; m >>= 1) ss += __shfl_xor(ss, m);
    const float inv = rsqrtf(ss / (float)D + eps);
    float r[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const float h = bf2f(f2bf(o[e] * inv));
        const float wh = bf2f(f2bf(w[e] * h));
        r[e] = wh * (z[e] / (1.f + __expf(-z[e])));
    }
    return make_uint4(pack_bf16x2(r[0], r[1]), pack_bf16x2(r[2], r[3]), pack_bf16x2(r[4], r[5]),
                      pack_bf16x2(r[6], r[7]));
}

template <class E>
__device__ __forceinline__ constexpr int tpart(int tile) {
    return E::KF * (tile / (E::VEC / 4)) + 4 * (tile % (E::VEC / 4));
}

typedef short v4s __attribute__((ext_vector_type(4)));
// ds_read_b64_tr_b16: in each 16-lane group, output lane 4q + r receives element r of the 8-byte chunks that lanes
// 4e + q (e = 0..3) address.
__device__ __forceinline__ uint2 lds_tr16(const char* p) {
    const v4s v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) v4s*)(p));
    return make_uint2((uint16_t)v[0] | ((uint32_t)(uint16_t)v[1] << 16),
                      (uint16_t)v[2] | ((uint32_t)(uint16_t)v[3] << 16));
}

// GN (output scan, bf16, whole rows per workgroup): each o row goes through the GatedNorm of the native layer before
// it is stored, with the arithmetic of gated_norm_kernel (gdn_layer.hip), so the bits equal the two separate passes.
template <class E, int D, bool OUT, bool BO, bool GN = false>
__global__ __launch_bounds__(SEG_THREADS, SEG_WAVES_PER_EU) void gdn_seg_kernel(GdnArgs a) {
    using T = typename E::T;
    using Cfg = SegCfg<E, D, OUT>;
    constexpr int VEC = E::VEC, KF = E::KF, ES = (int)sizeof(T), HP = VEC / 4;
    constexpr int NTD = D / 16, NTC = SC / 16, NKD = D / KF, NKC = SC / KF;
    constexpr int ROWB = D * ES, TROWB = SC * ES;
    constexpr int NW = Cfg::NW, NCG = Cfg::NCG;
    constexpr bool DBUF = Cfg::DBUF, TPS = Cfg::TPS;
    constexpr bool QL = OUT && DBUF;                     // q staged in LDS, two buffers (bf16); fp32 reads it from global
    constexpr int VW = NW * WCOLS, VROWB = VW * ES;      // V tile: the workgroup's columns
    constexpr int NFR = OUT ? attn_frags<E>() : 0;       // nonzero attn fragments of one query head
    using CL = ChunkLds<E, D, TPS>;
    using OL = OnceLds<E, D, QL ? 2 : 0, VW, NFR * 64 * VEC, !TPS>;
    __shared__ CL cl0;
    __shared__ typename std::conditional<DBUF, CL, NoLds>::type cl1;
    __shared__ OL ol;

    const int G = a.G, R = a.R, H = G * R;
    const int xcd = blockIdx.x % NXCD, local = blockIdx.x / NXCD;
    const int grp = xcd + NXCD * (local / NCG), cg = local % NCG;
    if (grp >= a.max_segs * G) return;
    const int g = grp % G, sid = grp / G;
    SegInfo sg;
    if (!locate_segment(a, sid, sg)) return;
    if (!OUT && sg.p == sg.nseg - 1) return;

    const int lane = lane_id(), wv = wave_id(), l16 = lane & 15, lg = lane >> 4;
    const int cb = cg * VW;                              // first column of the workgroup in [0, COLS)
    const int j0 = cb + wv * WCOLS;                      // first of this wave's columns
    const bool phi_part = !OUT && j0 >= D;
    const int jc = phi_part ? j0 - D : j0;               // column inside the D x D block
    const int n = sg.n;
    const int v_blk = OUT ? VROWB / 16 : (cb < D ? ((D - cb < VW ? D - cb : VW) * ES) / 16 : 0);  // loaded V blocks

    // per-lane address parts
    constexpr int NBLK = ROWB / 16;
    constexpr bool FAST = ES == 2 && NBLK >= 16;           // 4-bit swizzle of the K / q tiles
    constexpr int NX = FAST ? 4 : 2;
    const int lt = VEC * (l16 >> 2) + (l16 & 3);         // fragment row offset inside a tile
    // K / q fragment of K index group (ks, lg) at row tp(tile) + lt: block (4ks + lg) ^ swz(row), and the swizzle of
    // those rows depends on the lane only, so the block is 4*NX*(ks / NX) + xb[ks % NX]
    const int sl = swz<E>(lt, NBLK);
    int kq_base[NX];
#pragma unroll
    for (int c = 0; c < NX; ++c) kq_base[c] = lt * ROWB + 16 * (4 * (c ^ (sl >> 2)) + (lg ^ (sl & 3)));
    const int fo = lane * 16;                            // lane offset inside a 1 KB fragment-order piece
    // K^T A fragments (rows tp(td) + lt, K index = tokens KF*ks + VEC*lg + e).
    // bf16: two transposing reads per fragment; lane (e, q) = (l16/4, l16%4) of group lg reads the 4 state rows
    // tp(td) + 8q .. +3 of token 32ks + 8lg + 4h + e, so lane 4q + r collects tokens 8lg + 4h + 0..3 of row
    // prow(td, 4q + r). That chunk's block is (4A + q) ^ swz(token) with A = td/2, i.e. 4(A ^ s) + (q ^ e) for the lane
    // constant s, so it lies at trb[A % NTR] + (32ks + 4h)*ROWB + 64*A + 8*(td&1).
    // fp32: one 4-byte read per element, at ktb[td & 1][e] + (16ks + e)*ROWB + 64*td.
    constexpr int NTR = FAST ? 4 : 2;
    int trb[NTR], ktb[2][4];
    if constexpr (ES == 2) {
        const int e_ = l16 >> 2, q_ = l16 & 3;
        const int s_ = FAST ? (lg ^ (e_ & 2)) : ((lg ^ e_) & 1);
#pragma unroll
        for (int c = 0; c < NTR; ++c) trb[c] = (8 * lg + e_) * ROWB + 64 * ((c ^ s_) - c) + 16 * (q_ ^ e_);
    } else {
#pragma unroll
        for (int par = 0; par < 2; ++par)
#pragma unroll
            for (int c = 0; c < 4; ++c)
                ktb[par][c] = VEC * lg * ROWB + (par ? -64 : 64) * (lg & 1) + 16 * ((l16 >> 2) ^ c) + (l16 & 3) * ES;
    }
    // V B fragments (K index = tokens KF*ks + VEC*lg + e, column wv*32 + 16jt + l16 of the V tile).
    // bf16: lane (e, q) of group lg reads columns 16jt + 4q .. +3 of token 32ks + 8lg + 4h + e: at
    // vtb[jt] + (32ks + 4h)*VROWB. fp32: element (token, column) read directly.
    int vtb[NJ];
    if constexpr (ES == 2) {
        const int e_ = l16 >> 2, q_ = l16 & 3;
        const int sv = swz_v(8 * lg + e_, VROWB / 16);
#pragma unroll
        for (int jt = 0; jt < NJ; ++jt)
            vtb[jt] = (8 * lg + e_) * VROWB + 16 * ((wv * WCOLS / 8 + 2 * jt + (q_ >> 1)) ^ sv) + 8 * (q_ & 1);
    } else {
#pragma unroll
        for (int jt = 0; jt < NJ; ++jt) vtb[jt] = 0;
    }

    // state strip: S[tile over rows][column tile], rows prow(tile, 4lg + i), column jc + 16 jt + l16
    f32x4 S[NTD][NJ];
#pragma unroll
    for (int td = 0; td < NTD; ++td)
#pragma unroll
        for (int jt = 0; jt < NJ; ++jt) {
            const int j = jc + 16 * jt + l16;
            f32x4 v = {0.f, 0.f, 0.f, 0.f};
            if constexpr (OUT) {
                if (sg.p > 0) {                          // entry state from the combine (fragment order)
                    const float* src = a.ws_sin + ((long)sid * G + g) * D * D;
#pragma unroll
                    for (int i = 0; i < 4; ++i) v[i] = src[acc_frag_index<D>(prow<E>(td, 4 * lg + i), j)];
                } else if (a.s0) {                       // the caller's initial state (row-major)
                    const float* src = a.s0 + ((long)n * G + g) * D * D;
#pragma unroll
                    for (int i = 0; i < 4; ++i) v[i] = src[(long)prow<E>(td, 4 * lg + i) * D + j];
                }
            } else if (phi_part) {
#pragma unroll
                for (int i = 0; i < 4; ++i) v[i] = prow<E>(td, 4 * lg + i) == j ? 1.f : 0.f;
            }
            S[td][jt] = v;
        }

    const int count = sg.count;
    // The state is kept as S_stored with S = sc * S_stored for a wave-uniform scale sc, so the per-chunk decay
    // multiplies one scalar instead of the whole strip; sc is folded into the row factors of Y, o and the update, and
    // the strip is rescaled only when sc leaves [2^-32, 2^32]. cum_g is the segment's summed log-decay.
    float sc = 1.f, cum_g = 0.f;

    auto chunk_tok0 = [&](int c) { return sg.tok0 + (long)c * SC; };
    auto chunk_len = [&](int c) {
        const long rem = sg.tok1 - chunk_tok0(c);
        return (int)(rem < SC ? rem : SC);
    };
    const auto sw_row = [](int row) { return swz<E>(row, ROWB / 16); };
    const auto sw_v = [](int row) { return swz_v(row, VROWB / 16); };
    const auto sw_lin = [](int) { return 0; };
    auto load_tp = [&](T* dst, int c) {                  // T' of chunk c: a linear copy of its fragment-order block
        const long cid = sg.cid0 + c;
        const rsrc_t rt = make_rsrc(reinterpret_cast<const char*>(a.ws_T) + (cid * G + g) * SC * SC * ES,
                                    (uint32_t)(SC * SC * ES));
        stage_tile(rt, (uint32_t)TROWB, TROWB, dst, SC * TROWB, wv, NW, lane, sw_lin, 1 << 30);
    };
    auto load_chunk = [&](CL& cl, int c) {
        const long t0 = chunk_tok0(c);
        const int len = chunk_len(c);
        const long cid = sg.cid0 + c;
        const rsrc_t rk = make_rsrc(reinterpret_cast<const char*>(a.k) + (t0 * G + g) * D * ES,
                                    (uint32_t)((long)len * G * D * ES));
        stage_tile(rk, (uint32_t)(G * D * ES), ROWB, cl.K, SC * ROWB, wv, NW, lane, sw_row, 1 << 30);
        if constexpr (TPS) load_tp(cl.Tp, c);
        if (wv == 0 && lane < SC / 4) {
            const rsrc_t rg = make_rsrc(a.ws_gcum + (cid * G + g) * SC, SC * 4);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rg, (__attribute__((address_space(3))) void*)cl.gc, 16,
                                                     lane * 16, 0, 0, 0);
        }
    };
    auto load_q = [&](int buf, int c, int r) {           // q of query head r of chunk c into buffer buf (bf16)
        if constexpr (QL) {
            const long t0 = chunk_tok0(c);
            const rsrc_t rq = make_rsrc(reinterpret_cast<const char*>(a.q) + (t0 * H + (long)g * R + r) * D * ES,
                                        (uint32_t)((long)chunk_len(c) * H * D * ES));
            stage_tile<kCpolStream>(rq, (uint32_t)(H * D * ES), ROWB, ol.Q[buf], SC * ROWB, wv, NW, lane, sw_row,
                                    1 << 30);
        }
    };
    auto load_v = [&](int c) {
        if (v_blk > 0) {
            const long t0 = chunk_tok0(c);
            const rsrc_t rv = make_rsrc(reinterpret_cast<const char*>(a.v) + ((t0 * G + g) * D + cb) * ES,
                                        (uint32_t)((long)chunk_len(c) * G * D * ES - (long)cb * ES));
            stage_tile(rv, (uint32_t)(G * D * ES), VROWB, ol.V, SC * VROWB, wv, NW, lane, sw_v, v_blk);
        }
    };

    // acc = X S_stored over the D state rows for the 64 x D operand X whose A fragment (K step ks, token tile tt)
    // frag(ks, tt) returns; the fragments of step ks + 1 are read while step ks multiplies, and the scheduling
    // barrier keeps the compiler from hoisting every step's reads (and their registers) to the front.
    auto times_s = [&](auto&& frag, f32x4 (&acc)[NTC][NJ]) {
#pragma unroll
        for (int tt = 0; tt < NTC; ++tt)
#pragma unroll
            for (int jt = 0; jt < NJ; ++jt) acc[tt][jt] = f32x4{0.f, 0.f, 0.f, 0.f};
        uint4 af[NTC];
#pragma unroll
        for (int tt = 0; tt < NTC; ++tt) af[tt] = frag(0, tt);
#pragma unroll
        for (int ks = 0; ks < NKD; ++ks) {
            uint4 nf[NTC];
            if (ks + 1 < NKD) {
#pragma unroll
                for (int tt = 0; tt < NTC; ++tt) nf[tt] = frag(ks + 1, tt);
            }
            uint4 sb[NJ];
#pragma unroll
            for (int jt = 0; jt < NJ; ++jt) sb[jt] = pack_b<E>(S[ks * HP][jt], S[ks * HP + HP - 1][jt]);
#pragma unroll
            for (int tt = 0; tt < NTC; ++tt)
#pragma unroll
                for (int jt = 0; jt < NJ; ++jt) mma<E>(acc[tt][jt], af[tt], sb[jt]);
            if (ks + 1 < NKD) {
#pragma unroll
                for (int tt = 0; tt < NTC; ++tt) af[tt] = nf[tt];
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    };
    auto kq_off = [&](int ks, int row0) { return kq_base[ks % NX] + row0 * ROWB + 64 * NX * (ks / NX); };

    // o tiles of query head h for chunk rows t0 .. t0 + len - 1. With bf16 inputs each 16 x 16 tile is transposed
    // inside every quad of lanes (l16 = 4qa + qb holds rows VEC*lg + 0..3 of column 4qa + qb and gets row VEC*lg + qb
    // of columns 4qa .. 4qa + 3): a lane-dependent rotation, a rotation across the quad (DPP quad_perm: register k read
    // from lane (qb - k) mod 4) and the inverse lane-dependent rotation. A lane then writes 4 consecutive columns with
    // one store (8 bytes bf16, 16 bytes fp32) instead of four 2- or 4-byte stores. fp32-input scans (register-bound at
    // D = 256) store the accumulator layout directly.
    constexpr int OS = BO ? 2 : 4;
    using OPk = typename std::conditional<BO, uint2, uint4>::type;   // one lane's 4 columns of one row
    // bf16 output scans whose o block (64 rows x the workgroup's columns) fits a q buffer stage o through it
    constexpr bool STG = OUT && DBUF && SC * VW * OS <= SC * D * ES;
    static_assert(!GN || (STG && BO && VW == D), "the fused GatedNorm needs staged whole bf16 rows");
    // GN: the norm weights of the lane's 8 channels (lane % (D / 8) of a row's D / 8 lanes, as in gated_norm_kernel)
    float gnw[8];
    if constexpr (GN) {
#pragma unroll
        for (int e = 0; e < 8; ++e) gnw[e] = a.gn_w[8 * (lane % (D / 8)) + e];
    }
    auto pack_o = [&](const f32x4 (&O)[NTC][NJ], OPk (&P)[NTC][NJ]) {
        const int qb4 = l16 & 3;
        auto pick = [&](const float (&x)[4], int idx) {
            const float lo = (idx & 1) ? x[1] : x[0], hi = (idx & 1) ? x[3] : x[2];
            return (idx & 2) ? hi : lo;
        };
        auto dpp = [](float x, auto ctrl) {
            return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), decltype(ctrl)::value, 0xF, 0xF, true));
        };
#pragma unroll
        for (int tt = 0; tt < NTC; ++tt)
#pragma unroll
            for (int jt = 0; jt < NJ; ++jt) {
                const float x[4] = {O[tt][jt][0], O[tt][jt][1], O[tt][jt][2], O[tt][jt][3]};
                float u[4], z[4], w[4];
#pragma unroll
                for (int k = 0; k < 4; ++k) u[k] = pick(x, (k + qb4) & 3);
                z[0] = u[0];
                z[1] = dpp(u[1], std::integral_constant<int, 0x93>());   // quad_perm [3, 0, 1, 2]
                z[2] = dpp(u[2], std::integral_constant<int, 0x4E>());   // quad_perm [2, 3, 0, 1]
                z[3] = dpp(u[3], std::integral_constant<int, 0x39>());   // quad_perm [1, 2, 3, 0]
#pragma unroll
                for (int jj = 0; jj < 4; ++jj) w[jj] = pick(z, (qb4 - jj) & 3);
                if constexpr (BO) P[tt][jt] = make_uint2(pack_bf16x2(w[0], w[1]), pack_bf16x2(w[2], w[3]));
                else P[tt][jt] = make_uint4(__float_as_uint(w[0]), __float_as_uint(w[1]), __float_as_uint(w[2]),
                                            __float_as_uint(w[3]));
            }
    };
    // o is written once and q read once per kernel: streaming accesses keep them from displacing the K / V / T tiles
    // other workgroups re-read from L2 (output phase 0.1135-0.119 -> 0.1066-0.1127 ms at T = 32768, H = 4, D = 256)
    auto write_o = [&](const OPk (&P)[NTC][NJ], long t0, int len, int h) {
        const rsrc_t ro = make_rsrc(reinterpret_cast<char*>(a.o) + (t0 * H + h) * (long)D * OS,
                                    (uint32_t)((long)len * H * D * OS));
        const int row_l = VEC * lg + (l16 & 3);          // the lane's row inside a tile after the transpose
#pragma unroll
        for (int tt = 0; tt < NTC; ++tt)
#pragma unroll
            for (int jt = 0; jt < NJ; ++jt) {
                const int row = tpart<E>(tt) + row_l;
                // rows past the end of a partial chunk get an offset past the descriptor's range and are dropped
                const uint32_t off = row < len ? (uint32_t)((row * H * D + jc + 16 * jt + 4 * (l16 >> 2)) * OS)
                                               : 0xFFFFFFF0u;
                if constexpr (BO) {
                    typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
                    const u32x2 v2 = {P[tt][jt].x, P[tt][jt].y};
                    __builtin_amdgcn_raw_buffer_store_b64(v2, ro, off, 0, kCpolStream);
                } else {
                    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
                    const u32x4 v4 = {P[tt][jt].x, P[tt][jt].y, P[tt][jt].z, P[tt][jt].w};
                    __builtin_amdgcn_raw_buffer_store_b128(v4, ro, off, 0, kCpolStream);
                }
            }
    };
    auto store_o = [&](const f32x4 (&O)[NTC][NJ], long t0, int len, int h) {
        if constexpr (ES == 4) {
            const uint32_t o_lane = (uint32_t)((VEC * lg * H * D + l16) * OS);
#pragma unroll
            for (int tt = 0; tt < NTC; ++tt)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int row = tpart<E>(tt) + i;
                    const int nrow = len > row ? len - row : 0;
                    const rsrc_t ro = make_rsrc(reinterpret_cast<char*>(a.o) + ((t0 + row) * H + h) * (long)D * OS,
                                                (uint32_t)(nrow * H * D * OS));
#pragma unroll
                    for (int jt = 0; jt < NJ; ++jt) {
                        const uint32_t voff = o_lane + (uint32_t)((jc + 16 * jt) * OS);
                        if constexpr (BO) __builtin_amdgcn_raw_buffer_store_b16(f2bf(O[tt][jt][i]), ro, voff, 0u, 0);
                        else __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(O[tt][jt][i]), ro, voff, 0u, 0);
                    }
                }
        } else {
            OPk P[NTC][NJ];
            pack_o(O, P);
            write_o(P, t0, len, h);
        }
    };

    // attn fragment f of one query head: the accumulators of K tiles ks*HP + h (rows = keys t') times q tile b
    // (columns = queries t) are attn^T, and lane l16 of group lg holds query t = tp(b) + lt with keys
    // t' = KF*ks + VEC*lg + 4h + i, i.e. the A fragment (b, ks) of o = attn v_new once masked to t' <= t and scaled by
    // scale e^{gc_t - gc_t'}. q: LDS (bf16) or global (fp32).
    auto attn_frag = [&](int f, const char* Kb, const char* Qb, const rsrc_t& rq, const float* gcl, char* Atb) {
        int b = 0, ks = f;
#pragma unroll
        for (int i = 0; i < NTC - 1; ++i)
            if (ks >= attn_nks<E>(b)) {
                ks -= attn_nks<E>(b);
                ++b;
            }
        const int qrow = tpart<E>(b), krow = KF * ks;
        f32x4 acc[HP];
#pragma unroll
        for (int hh = 0; hh < HP; ++hh) acc[hh] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kk = 0; kk < NKD; ++kk) {
            uint4 qf;
            if constexpr (QL) qf = lds16(Qb, kq_off(kk, qrow));
            else qf = buf_ld16(rq, (uint32_t)(((qrow + lt) * H * D + KF * kk + VEC * lg) * ES));
#pragma unroll
            for (int hh = 0; hh < HP; ++hh) mma<E>(acc[hh], lds16(Kb, kq_off(kk, krow + 4 * hh)), qf);
        }
        const int t = qrow + lt;
        const float gt = gcl[t];
        f32x4 m[HP];
#pragma unroll
        for (int hh = 0; hh < HP; ++hh) {
            const float4 gk = *reinterpret_cast<const float4*>(&gcl[krow + VEC * lg + 4 * hh]);
            const float gkv[4] = {gk.x, gk.y, gk.z, gk.w};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int tk = krow + VEC * lg + 4 * hh + i;
                m[hh][i] = tk <= t ? a.scale * __expf(gt - gkv[i]) * acc[hh][i] : 0.f;
            }
        }
        *reinterpret_cast<uint4*>(Atb + f * 1024 + fo) = pack_b<E>(m[0], m[HP - 1]);
    };

    int qb = 0;                                          // q buffer of the current query head (bf16)
    // bf16: the o tiles of the last DEP query heads (pk), written DEP heads later so that the stores
    // complete under the MFMAs of the heads in between (pq_h < 0: empty entry). One head of delay measured best at
    // T = 32768, G = 4, R = 6 (364 us per output launch; two heads: 390 us).
    constexpr int DEP = 1;
    f32x4 pk[DEP][NTC][NJ];
    long pq_t0[DEP];
    int pq_len[DEP], pq_h[DEP];
#pragma unroll
    for (int d = 0; d < DEP; ++d) {
        pq_t0[d] = 0;
        pq_len[d] = 0;
        pq_h[d] = -1;
    }
    auto flush_oldest = [&]() {                          // write entry 0 and move the others down
        if (pq_h[0] >= 0) store_o(pk[0], pq_t0[0], pq_len[0], pq_h[0]);
#pragma unroll
        for (int d = 0; d + 1 < DEP; ++d) {
#pragma unroll
            for (int tt = 0; tt < NTC; ++tt)
#pragma unroll
                for (int jt = 0; jt < NJ; ++jt) pk[d][tt][jt] = pk[d + 1][tt][jt];
            pq_t0[d] = pq_t0[d + 1];
            pq_len[d] = pq_len[d + 1];
            pq_h[d] = pq_h[d + 1];
        }
        pq_h[DEP - 1] = -1;
    };
    // next: the idle stage buffer, loaded with chunk cn by DMA once this chunk's V fragments are in registers. The
    // compiler waits for every outstanding DMA before a transposing LDS read (ds_read_b64_tr_b16), so the V reads
    // come first and the copy then overlaps phases 1 to 3 instead of phase 1 only.
    auto compute = [&](const CL& cl, int c, bool prefetch, CL* next) {
        const int cn = c + 1 < count ? c + 1 : c;
        // GN: the z rows of query head r of this chunk for the fused GatedNorm (rows past the chunk's end read as
        // zero through the descriptor's range). Head 0's go out after the V fragment reads (the compiler drains every
        // outstanding load before a transposing LDS read) and the next stage's copy, so they arrive under phases 1-3
        constexpr int GRB = VW * 2, GLPR = GRB / 16, GRPI = 64 / GLPR, GNK = GN ? SC / NW / GRPI : 1;
        uint4 zgv[GNK];
        auto load_zg = [&](int r) {
            if constexpr (GN) {
                const rsrc_t rz = make_rsrc(reinterpret_cast<const char*>(a.gn_z) +
                                                (chunk_tok0(c) * H + (long)g * R + r) * (long)D * 2,
                                            (uint32_t)((long)chunk_len(c) * H * D * 2));
#pragma unroll
                for (int kk = 0; kk < GNK; ++kk) {
                    const int row = (SC / NW) * wv + GRPI * kk + lane / GLPR;
                    zgv[kk] = buf_ld16(rz, (uint32_t)(row * H * D * 2 + 16 * (lane % GLPR)));
                }
            }
        };
        const char* Kb = reinterpret_cast<const char*>(cl.K);
        const char* Tb = reinterpret_cast<const char*>(TPS ? cl.Tp : ol.Tp);
        const char* Vb = reinterpret_cast<const char*>(ol.V);
        uint4 vf[NKC][NJ];
        auto read_vf = [&]() {
#pragma unroll
        for (int ks = 0; ks < NKC; ++ks)
#pragma unroll
            for (int jt = 0; jt < NJ; ++jt) {
                if constexpr (ES == 2) {
                    const uint2 lo = lds_tr16(Vb + vtb[jt] + 32 * ks * VROWB);
                    const uint2 hi = lds_tr16(Vb + vtb[jt] + (32 * ks + 4) * VROWB);
                    vf[ks][jt] = make_uint4(lo.x, lo.y, hi.x, hi.y);
                } else {
                    // element (token t, tile column cv) of the swizzled V tile
                    const int cv = wv * WCOLS + 16 * jt + l16;
                    uint32_t w[4];
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const int t = KF * ks + VEC * lg + e;
                        w[e] = *reinterpret_cast<const uint32_t*>(
                            Vb + t * VROWB + (((cv >> 2) ^ swz_v(t, VROWB / 16)) << 4) + (cv & 3) * 4);
                    }
                    vf[ks][jt] = make_uint4(w[0], w[1], w[2], w[3]);
                }
            }
        };
        if constexpr (DBUF) read_vf();                  // single-buffered runs read V in phase 2 (fewer live registers)
        if (next) load_chunk(*next, cn);
        load_zg(0);
        const float glast = cl.gc[SC - 1];
        const float decay = __expf(glast);
        float egc[NTC][4];                        // sc e^{gc} of the accumulator rows
#pragma unroll
        for (int tt = 0; tt < NTC; ++tt) {
            const float4 gq = *reinterpret_cast<const float4*>(&cl.gc[tpart<E>(tt) + VEC * lg]);
            egc[tt][0] = sc * __expf(gq.x);
            egc[tt][1] = sc * __expf(gq.y);
            egc[tt][2] = sc * __expf(gq.z);
            egc[tt][3] = sc * __expf(gq.w);
        }

        // phase 1: Y = K S_stored; output scan: then the attn fragments of the chunk's first query head (their LDS
        // writes are ordered by the barrier that starts head 0, which saves that head its own barrier)
        f32x4 Y[NTC][NJ];
        times_s([&](int ks, int tt) { return lds16(Kb, kq_off(ks, tpart<E>(tt))); }, Y);
        if constexpr (OUT) {
            const char* Q0b = reinterpret_cast<const char*>(ol.Q[QL ? qb : 0]);
            const rsrc_t rq0 = make_rsrc(reinterpret_cast<const char*>(a.q) + (chunk_tok0(c) * H + (long)g * R) * D * ES,
                                         (uint32_t)(QL ? 0 : (long)chunk_len(c) * H * D * ES));
            for (int f = wv; f < NFR; f += NW) attn_frag(f, Kb, Q0b, rq0, cl.gc, reinterpret_cast<char*>(ol.At));
        }

        // phase 2: v_new = T' (V - e^{gc} K S) = T' V + T' (-sc e^{gc} Y). The T' fragments (and, single-buffered,
        // the V fragments) are read first, so their LDS latency is covered by the scaling of Y.
        uint4 tf[NKC][NTC];
#pragma unroll
        for (int ks = 0; ks < NKC; ++ks)
#pragma unroll
            for (int tt = 0; tt < NTC; ++tt) tf[ks][tt] = lds16(Tb, (ks * NTC + tt) * 1024 + fo);
        if constexpr (!DBUF) read_vf();
        f32x4 Vn[NTC][NJ];
#pragma unroll
        for (int tt = 0; tt < NTC; ++tt)
#pragma unroll
            for (int jt = 0; jt < NJ; ++jt)
#pragma unroll
                for (int i = 0; i < 4; ++i) Y[tt][jt][i] *= -egc[tt][i];
#pragma unroll
        for (int ks = 0; ks < NKC; ++ks) {
            uint4 yb[NJ];
#pragma unroll
            for (int jt = 0; jt < NJ; ++jt) yb[jt] = pack_b<E>(Y[ks * HP][jt], Y[ks * HP + HP - 1][jt]);
#pragma unroll
            for (int tt = 0; tt < NTC; ++tt) {
#pragma unroll
                for (int jt = 0; jt < NJ; ++jt) {
                    if (ks == 0) Vn[tt][jt] = f32x4{0.f, 0.f, 0.f, 0.f};
                    mma<E>(Vn[tt][jt], tf[ks][tt], yb[jt]);
                    if (!phi_part) mma<E>(Vn[tt][jt], tf[ks][tt], vf[ks][jt]);
                }
            }
        }
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (!OUT) {
            if (prefetch) {
                lds_barrier();                     // every wave is done with V of this chunk (its LDS reads)
                load_v(cn);
            }
        }

        // phase 3, per query head r: o_r = scale e^{gc} (q_r S) + attn_r v_new
        if constexpr (OUT) {
            const long t0 = chunk_tok0(c);
            const int len = chunk_len(c);
            char* Atb = reinterpret_cast<char*>(ol.At);
            uint4 vb[NKC][NJ];
#pragma unroll
            for (int ks = 0; ks < NKC; ++ks)
#pragma unroll
                for (int jt = 0; jt < NJ; ++jt) vb[ks][jt] = pack_b<E>(Vn[ks * HP][jt], Vn[ks * HP + HP - 1][jt]);
            for (int r = 0; r < R; ++r) {
                const int h = g * R + r;
                if (r > 0) load_zg(r);                   // head 0's rows were loaded at the chunk's start
                const char* Qb = reinterpret_cast<const char*>(ol.Q[QL ? qb : 0]);
                const rsrc_t rq = make_rsrc(reinterpret_cast<const char*>(a.q) + (t0 * H + h) * D * ES,
                                            (uint32_t)(QL ? 0 : (long)len * H * D * ES));
                if constexpr (DBUF) {
                    if (r == 0) {
                        lds_barrier();             // q_0 landed before the chunk; every wave is done with T' and V
                    } else {
                        wait_vmem_all();
                        __syncthreads();           // q_r has landed; every wave is done with head r - 1
                    }
                    if (prefetch) {
                        if (r == 0) {              // T' and V of this chunk were consumed in phase 2
                            load_tp(ol.Tp, cn);
                            load_v(cn);
                        }
                        if (r + 1 < R) load_q(qb ^ 1, c, r + 1);
                        else load_q(qb ^ 1, cn, 0);
                    }
                    flush_oldest();
                } else {
                    lds_barrier();                 // head 0: its attn fragments are complete; later heads: every
                }                                  // wave is done with the attn fragments of head r - 1
                if (r > 0) for (int f = wv; f < NFR; f += NW) attn_frag(f, Kb, Qb, rq, cl.gc, Atb);
                f32x4 O[NTC][NJ];
                if constexpr (QL) times_s([&](int ks, int tt) { return lds16(Qb, kq_off(ks, tpart<E>(tt))); }, O);
                else
                    times_s([&](int ks, int tt) {
                        return buf_ld16(rq, (uint32_t)(((tpart<E>(tt) + lt) * H * D + KF * ks + VEC * lg) * ES));
                    }, O);
                if (r > 0) lds_barrier();          // the attn fragments of head r are complete (head 0: above)
                uint4 af[NFR];
#pragma unroll
                for (int f = 0; f < NFR; ++f) af[f] = lds16(Atb, f * 1024 + fo);
#pragma unroll
                for (int tt = 0; tt < NTC; ++tt)
#pragma unroll
                    for (int jt = 0; jt < NJ; ++jt)
#pragma unroll
                        for (int i = 0; i < 4; ++i) O[tt][jt][i] *= a.scale * egc[tt][i];   // egc carries sc
#pragma unroll
                for (int ks = 0; ks < NKC; ++ks)
#pragma unroll
                    for (int tt = 0; tt < NTC; ++tt)
                        if (ks < attn_nks<E>(tt)) {
#pragma unroll
                            for (int jt = 0; jt < NJ; ++jt) mma<E>(O[tt][jt], af[attn_fidx<E>(tt, ks)], vb[ks][jt]);
                        }
                if constexpr (DBUF && STG) {
                    // o through the q buffer this head has consumed (its q reads are ordered before this barrier; the
                    // next head's copy into it waits for the top barrier of head r + 1), then whole-row stores
                    if (r == 0) lds_barrier();
                    char* stg = reinterpret_cast<char*>(ol.Q[qb]);
                    OPk P[NTC][NJ];
                    pack_o(O, P);
#pragma unroll
                    for (int tt = 0; tt < NTC; ++tt)
#pragma unroll
                        for (int jt = 0; jt < NJ; ++jt) {
                            const int row = tpart<E>(tt) + VEC * lg + (l16 & 3);
                            *reinterpret_cast<OPk*>(stg + (row * VW + wv * WCOLS + 16 * jt + 4 * (l16 >> 2)) * OS) =
                                P[tt][jt];
                        }
                    lds_barrier();
                    constexpr int RB = VW * OS, LPR = RB / 16, RPI = 64 / LPR;   // row bytes, lanes per row, rows
                    const rsrc_t ro = make_rsrc(reinterpret_cast<char*>(a.o) + (t0 * H + h) * (long)D * OS,
                                                (uint32_t)((long)len * H * D * OS));
#pragma unroll
                    for (int k = 0; k < SC / NW / RPI; ++k) {
                        const int row = (SC / NW) * wv + RPI * k + lane / LPR, ch = lane % LPR;
                        uint4 v4 = lds16(stg, row * RB + 16 * ch);
                        if constexpr (GN) {
                            static_assert(!GN || (BO && VW == D && LPR == GLPR), "GatedNorm needs whole bf16 rows");
                            v4 = gated_norm_row<LPR>(v4, zgv[k], gnw, a.gn_eps, D);
                        }
                        typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
                        const u32x4 w4 = {v4.x, v4.y, v4.z, v4.w};
                        __builtin_amdgcn_raw_buffer_store_b128(
                            w4, ro, (uint32_t)((row * H * D + cb) * OS + 16 * ch), 0, kCpolStream);
                    }
                    qb ^= 1;
                } else if constexpr (DBUF) {
#pragma unroll
                    for (int tt = 0; tt < NTC; ++tt)
#pragma unroll
                        for (int jt = 0; jt < NJ; ++jt) pk[DEP - 1][tt][jt] = O[tt][jt];
                    pq_t0[DEP - 1] = t0;
                    pq_len[DEP - 1] = len;
                    pq_h[DEP - 1] = h;
                    qb ^= 1;
                } else {
                    store_o(O, t0, len, h);
                }
                __builtin_amdgcn_sched_barrier(0);
            }
        }

        // phase 4: S = e^{gc_last} S + K^T (e^{gc_last - gc} v_new), as S_stored += K^T (e^{gc_last - gc} v_new / sc')
        // row factor e^{gc_last - gc} / sc' = (sc e^{gc_last} / sc') / (sc e^{gc}) = ratio / egc
        const float scn = sc * decay;
        cum_g += glast;
        float ratio = 1.f;
        if (scn >= 0x1p-32f && scn <= 0x1p32f) {
            sc = scn;
        } else {
#pragma unroll
            for (int td = 0; td < NTD; ++td)
#pragma unroll
                for (int jt = 0; jt < NJ; ++jt)
#pragma unroll
                    for (int i = 0; i < 4; ++i) S[td][jt][i] *= scn;
            ratio = scn;
            sc = 1.f;
        }
#pragma unroll
        for (int tt = 0; tt < NTC; ++tt) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float f = ratio * __builtin_amdgcn_rcpf(egc[tt][i]);
#pragma unroll
                for (int jt = 0; jt < NJ; ++jt) Vn[tt][jt][i] *= f;
            }
        }
        auto frag_kt = [&](int td, int ks) {
            if constexpr (ES == 2) {
                const int at = td >> 1;
                const char* p = Kb + trb[at % NTR] + 32 * ks * ROWB + 64 * at + 8 * (td & 1);
                const uint2 lo = lds_tr16(p), hi = lds_tr16(p + 4 * ROWB);
                return make_uint4(lo.x, lo.y, hi.x, hi.y);
            } else {
                uint32_t w[4];
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    w[e] = *reinterpret_cast<const uint32_t*>(Kb + ktb[td & 1][e] + (KF * ks + e) * ROWB + 64 * td);
                return make_uint4(w[0], w[1], w[2], w[3]);
            }
        };
        // K^T fragments are read PF4 tiles ahead of their MFMAs (a ring of PF4 + 1 fragments over the
        // NKC * NTD (ks, td) steps), so the LDS latency of the transposing reads stays covered
        constexpr int NST = NKC * NTD, PF4 = 3;
        uint4 ring[PF4 + 1];
#pragma unroll
        for (int q = 0; q < PF4; ++q) ring[q] = frag_kt(q % NTD, q / NTD);
        uint4 vb[NKC][NJ];
#pragma unroll
        for (int ks = 0; ks < NKC; ++ks)
#pragma unroll
            for (int jt = 0; jt < NJ; ++jt) vb[ks][jt] = pack_b<E>(Vn[ks * HP][jt], Vn[ks * HP + HP - 1][jt]);
#pragma unroll
        for (int st = 0; st < NST; ++st) {
            const int ks = st / NTD, td = st % NTD;
            if (st + PF4 < NST) ring[(st + PF4) % (PF4 + 1)] = frag_kt((st + PF4) % NTD, (st + PF4) / NTD);
#pragma unroll
            for (int jt = 0; jt < NJ; ++jt) mma<E>(S[td][jt], ring[st % (PF4 + 1)], vb[ks][jt]);
            __builtin_amdgcn_sched_barrier(0);
        }
    };

    if (count > 0) {
        if constexpr (DBUF) {
            load_chunk(cl0, 0);
            if constexpr (!TPS) load_tp(ol.Tp, 0);
            load_q(0, 0, 0);
            load_v(0);
            wait_vmem_all();
            __syncthreads();
            for (int c = 0;;) {
                // the next chunk's stage is loaded unconditionally inside compute (the last chunk re-loads itself
                // into the idle buffer): a conditional load would make the wait counts drain it before the current
                // chunk
                compute(cl0, c, true, &cl1);
                wait_vmem_all();
                __syncthreads();
                if (++c >= count) break;
                compute(cl1, c, true, &cl0);
                wait_vmem_all();
                __syncthreads();
                if (++c >= count) break;
            }
        } else {
            for (int c = 0; c < count; ++c) {
                load_chunk(cl0, c);
                load_v(c);
                wait_vmem_all();
                __syncthreads();
                compute(cl0, c, false, nullptr);
                __syncthreads();
            }
        }
    }

    if constexpr (OUT) {
#pragma unroll
        for (int d = 0; d < DEP; ++d) flush_oldest();
        if (sg.p == sg.nseg - 1 && a.s_out) {
            float* dst = a.s_out + ((long)n * G + g) * D * D;
#pragma unroll
            for (int td = 0; td < NTD; ++td)
#pragma unroll
                for (int jt = 0; jt < NJ; ++jt)
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        dst[(long)prow<E>(td, 4 * lg + i) * D + jc + 16 * jt + l16] = sc * S[td][jt][i];
        }
    } else {
        // segment map S_end = Phi S_start + N, stored as N (fp32), Psi = Phi - c I (in_dtype) and c = e^{sum of g}
        const float c = __expf(cum_g);
        const long off = ((long)sid * G + g) * D * D;
#pragma unroll
        for (int td = 0; td < NTD; ++td)
#pragma unroll
            for (int jt = 0; jt < NJ; ++jt) {
                const int d0 = prow<E>(td, 4 * lg), j = jc + 16 * jt + l16;   // the lane's rows d0 .. d0 + 3
                if (phi_part) {
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        reinterpret_cast<T*>(a.ws_phi)[off + psi_frag_index<E, D>(d0 + i, j)] =
                            E::from_f(sc * S[td][jt][i] - (d0 + i == j ? c : 0.f));
                } else {                                  // one float4 of the accumulator-fragment layout
                    *reinterpret_cast<float4*>(a.ws_n + off + acc_frag_index<D>(d0, j)) =
                        make_float4(sc * S[td][jt][0], sc * S[td][jt][1], sc * S[td][jt][2], sc * S[td][jt][3]);
                }
            }
        if (cg == 0 && wv == 0 && lane == 0) a.ws_c[(long)sid * G + g] = c;
    }
}

// ------------------------------------------------------------------------------------------------ segment combine
// One workgroup per (sequence, KV head, 16-column strip), NW waves; wave w produces row tiles w*NTD/NW ..
// (w+1)*NTD/NW - 1 of X_{p+1} = c_p X_p + Psi_p X_p + N_p (Psi_p = Phi_p - c_p I). The pure-decay part c_p X_p is exact
// fp32; Psi_p X_p is an MFMA with Psi_p in in_dtype and, for bf16, X split into bf16 high and low parts. X^T is shared
// through LDS between steps. bf16 prefetches the next step's Psi fragments, N and c while a step computes.
// Waves per combine workgroup: 4 (one per SIMD, up to 512 registers); at D = 256, 8 (two per SIMD, 2 row tiles
// each, 176 registers), so one wave's loads and LDS exchange overlap the other's MFMAs: 64 -> 60 us per launch at
// T = 32768, H = 4.
constexpr int kCombineWaves256 = 8;
template <int D>
constexpr int combine_waves() { return D == 256 ? kCombineWaves256 : 4; }

template <class E, int D>
__global__ __launch_bounds__(64 * combine_waves<D>())
__attribute__((amdgpu_waves_per_eu(combine_waves<D>() / 4, combine_waves<D>() / 4))) void gdn_combine_kernel(GdnArgs a) {
    using T = typename E::T;
    constexpr int VEC = E::VEC, KF = E::KF, NTD = D / 16, NKD = D / KF, TPW = NTD / combine_waves<D>();
    constexpr bool DBUF = E::VEC == 8;
    __shared__ __align__(16) float XT[16][D + 4];
    // XCD-aware mapping: all strips of one (sequence, KV head) read the same Psi, so they go to one XCD (one L2)
    const int strips = D / 16, G = a.G;
    const int xcd = blockIdx.x % NXCD, local = blockIdx.x / NXCD;
    const int grp = xcd + NXCD * (local / strips), jb = local % strips;
    const int n = grp / G, g = grp % G;
    if (n >= a.num_seqs) return;
    int first, nseg;
    seq_segments(a, n, first, nseg);
    if (nseg <= 1) return;
    const int lane = lane_id(), wv = wave_id(), l16 = lane & 15, lg = lane >> 4;
    const int j0 = 16 * jb;
    const float* s0 = a.s0 ? a.s0 + ((long)n * G + g) * D * D : nullptr;
    for (int idx = threadIdx.x; idx < 16 * D; idx += blockDim.x) {
        const int j = idx & 15, d = idx >> 4;
        XT[j][d] = s0 ? s0[(long)d * D + j0 + j] : 0.f;
    }

    struct Pre {
        uint4 A[TPW][NKD];     // Psi rows 16*(wv*TPW + u) + l16, K index KF*ks + VEC*lg
        float N[TPW][4];       // N at the accumulator rows
        float c;
    };
    // Each strip walks the row tiles starting at its own index (tile (wv * TPW + u + jb) mod NTD).
    auto load_nc = [&](Pre& P, int p) {
        const long sid = first + p;
        const float* Nm = a.ws_n + (sid * G + g) * D * D;
#pragma unroll
        for (int u = 0; u < TPW; ++u) {
            const int tr = (wv * TPW + u + jb) & (NTD - 1);
            const float4 nv = *reinterpret_cast<const float4*>(Nm + ((long)(tr * (D / 16) + jb) * 64 + lane) * 4);
            P.N[u][0] = nv.x; P.N[u][1] = nv.y; P.N[u][2] = nv.z; P.N[u][3] = nv.w;
        }
        P.c = a.ws_c[sid * G + g];
    };
    auto load_frag = [&](Pre& P, int p, int ks) {      // the Psi fragments of K step ks
        const T* Psi = reinterpret_cast<const T*>(a.ws_phi) + ((long)(first + p) * G + g) * D * D;
#pragma unroll
        for (int u = 0; u < TPW; ++u) {
            const int tr = (wv * TPW + u + jb) & (NTD - 1);
            P.A[u][ks] = ld16(Psi + ((long)(tr * NKD + ks) * 64 + lane) * VEC);
        }
    };
    auto load = [&](Pre& P, int p) {
#pragma unroll
        for (int ks = 0; ks < NKD; ++ks) load_frag(P, p, ks);
        load_nc(P, p);
    };
    // One step; bf16 runs also load the next step's operands into Pn (map pn): N and c first, the Psi fragments of
    // K step ks next to the MFMAs of K step ks, so the loads stream while the MFMAs run instead of stalling the wave
    // in one burst.
    auto step = [&](const Pre& P, Pre& Pn, int p, int pn) {
        const long sid = first + p;
        if constexpr (DBUF) load_nc(Pn, pn);
        // acc collects Psi X_hi (bf16) or Psi X (fp32); accl collects Psi X_lo, in separate accumulators so that no
        // MFMA waits for the one before it
        f32x4 acc[TPW], accl[TPW];
#pragma unroll
        for (int u = 0; u < TPW; ++u) {
            const int tr = (wv * TPW + u + jb) & (NTD - 1);   // rotated by the strip: see load()
            const float4 x = *reinterpret_cast<const float4*>(&XT[l16][16 * tr + 4 * lg]);
            acc[u][0] = P.N[u][0] + P.c * x.x;
            acc[u][1] = P.N[u][1] + P.c * x.y;
            acc[u][2] = P.N[u][2] + P.c * x.z;
            acc[u][3] = P.N[u][3] + P.c * x.w;
            accl[u] = f32x4{0.f, 0.f, 0.f, 0.f};
        }
        // the whole B operand (X, split into bf16 high and low parts) is read from LDS and converted before the
        // first MFMA, so the MFMA stream does not wait on LDS
        uint4 BH[NKD], BL[VEC == 8 ? NKD : 1];
#pragma unroll
        for (int ks = 0; ks < NKD; ++ks) {
            float bv[VEC];
#pragma unroll
            for (int e = 0; e < VEC; e += 4) {
                const float4 x = *reinterpret_cast<const float4*>(&XT[l16][KF * ks + VEC * lg + e]);
                bv[e] = x.x; bv[e + 1] = x.y; bv[e + 2] = x.z; bv[e + 3] = x.w;
            }
            if constexpr (VEC == 8) {
                uint32_t hw[4], lw[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    hw[e] = pack_bf16x2(bv[2 * e], bv[2 * e + 1]);
                    lw[e] = pack_bf16x2(bv[2 * e] - __uint_as_float(hw[e] << 16),
                                        bv[2 * e + 1] - __uint_as_float(hw[e] & 0xffff0000u));
                }
                BH[ks] = make_uint4(hw[0], hw[1], hw[2], hw[3]);
                BL[ks] = make_uint4(lw[0], lw[1], lw[2], lw[3]);
            } else {
                BH[ks] = make_uint4(__float_as_uint(bv[0]), __float_as_uint(bv[1]), __float_as_uint(bv[2]),
                                    __float_as_uint(bv[3]));
            }
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int ks = 0; ks < NKD; ++ks) {
            if constexpr (DBUF) load_frag(Pn, pn, ks);
            if constexpr (VEC == 8) {
#pragma unroll
                for (int u = 0; u < TPW; ++u) mma<E>(accl[u], P.A[u][ks], BL[ks]);
#pragma unroll
                for (int u = 0; u < TPW; ++u) mma<E>(acc[u], P.A[u][ks], BH[ks]);
                __builtin_amdgcn_sched_barrier(0);
            } else {
#pragma unroll
                for (int u = 0; u < TPW; ++u) mma<E>((ks & 1) ? accl[u] : acc[u], P.A[u][ks], BH[ks]);
            }
        }
#pragma unroll
        for (int u = 0; u < TPW; ++u)
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[u][i] += accl[u][i];
        // no drain of the vector-memory counter here: it would also wait for the next step's prefetch and for this
        // workgroup's state stores, putting their latency on the sequential path; the compiler waits only for the
        // prefetched registers the next step reads, and the barriers order the XT exchange in LDS only
        lds_barrier();
        float* dst = a.ws_sin + ((sid + 1) * G + g) * D * D;
#pragma unroll
        for (int u = 0; u < TPW; ++u) {
            const int tr = (wv * TPW + u + jb) & (NTD - 1);   // rotated by the strip: see load()
#pragma unroll
            for (int i = 0; i < 4; ++i) XT[l16][16 * tr + 4 * lg + i] = acc[u][i];
            *reinterpret_cast<float4*>(dst + ((long)(tr * (D / 16) + jb) * 64 + lane) * 4) =
                make_float4(acc[u][0], acc[u][1], acc[u][2], acc[u][3]);
        }
        lds_barrier();
    };

    const int steps = nseg - 1;
    // L2 warm-up: while step p runs, workgroup jb touches rows 16 jb .. 16 jb + 15 of Psi_{p+2}, so the 16 strips of a
    // head together bring the whole matrix into their XCD's L2 before any of them prefetches it. The touch is a plain
    // load into registers whose values are folded into a sink one step later (when they have long arrived) and never
    // used. It is not a load into LDS: the LDS fence of the step's barriers would then wait for it, and with it for
    // the prefetch issued just before. Past the last step it touches the last map again, so the loads are
    // unconditional and the compiler's wait counts stay exact.
    constexpr int TBYTES = 16 * D * (int)sizeof(T), NTCH = TBYTES >= 4096 ? TBYTES / 4096 : 1;
    uint4 tv[NTCH];
#pragma unroll
    for (int i = 0; i < NTCH; ++i) tv[i] = make_uint4(0u, 0u, 0u, 0u);
    uint32_t tsink = 0;
    auto touch = [&](int p) {
#pragma unroll
        for (int i = 0; i < NTCH; ++i) tsink ^= tv[i].x ^ tv[i].w;
        const int pp = p < steps ? p : steps - 1;
        const char* rows = reinterpret_cast<const char*>(reinterpret_cast<const T*>(a.ws_phi) +
                                                         ((long)(first + pp) * G + g) * D * D + (long)16 * jb * D);
#pragma unroll
        for (int i = 0; i < NTCH; ++i) tv[i] = ld16(rows + (wv * 1024 + i * 4096) % TBYTES + 16 * lane);
    };
    if constexpr (DBUF) {
        Pre P0, P1;
        load(P0, 0);
        touch(1);
        __syncthreads();
        // the next step's operands are loaded unconditionally (past the last step the last map is loaded again): a
        // conditional load makes the compiler drain every outstanding load where the branches join, which would put
        // the whole prefetch on the sequential path
        for (int p = 0;;) {
            touch(p + 2);
            step(P0, P1, p, p + 1 < steps ? p + 1 : p);
            if (++p >= steps) break;
            touch(p + 2);
            step(P1, P0, p, p + 1 < steps ? p + 1 : p);
            if (++p >= steps) break;
        }
    } else {
        __syncthreads();
        for (int p = 0; p < steps; ++p) {
            Pre P;
            load(P, p);
            step(P, P, p, p);
        }
    }
#pragma unroll
    for (int i = 0; i < NTCH; ++i) tsink ^= tv[i].x ^ tv[i].w;
    if (a.num_seqs < 0) a.ws_c[0] = __uint_as_float(tsink);      // keeps the touches; never taken
}

// ------------------------------------------------------------------------------------------------ host launchers
namespace {

template <class E, int D, bool OUT>
dim3 seg_grid(const GdnArgs& a) {
    using Cfg = SegCfg<E, D, OUT>;
    const int per = Cfg::NCG;
    const int groups = a.max_segs * a.G;
    return dim3(NXCD * ((groups + NXCD - 1) / NXCD) * per);
}

template <class E, int D>
int launch_states(const GdnArgs& a, hipStream_t stream, bool summary, bool combine) {
    if (summary) {
        const dim3 grid = seg_grid<E, D, false>(a), block(SegCfg<E, D, false>::NW * 64);
        hipLaunchKernelGGL((gdn_seg_kernel<E, D, false, false>), grid, block, 0, stream, a);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return (int)e;
    }
    if (!combine) return 0;
    const int groups = a.num_seqs * a.G;
    hipLaunchKernelGGL((gdn_combine_kernel<E, D>), dim3(NXCD * ((groups + NXCD - 1) / NXCD) * (D / 16)),
                       dim3(64 * combine_waves<D>()), 0,
                       stream, a);
    return (int)hipGetLastError();
}

template <class E, int D>
int launch_output(const GdnArgs& a, hipStream_t stream) {
    const dim3 grid = seg_grid<E, D, true>(a), block(SegCfg<E, D, true>::NW * 64);
    if (a.gn_z) {                                        // the fused GatedNorm: bf16 rows of D <= 128
        if constexpr (std::is_same<E, BF16>::value && D <= 128) {
            if (a.o_dtype != DT_BF16) return BF_ERR_UNSUPPORTED;
            hipLaunchKernelGGL((gdn_seg_kernel<E, D, true, true, true>), grid, block, 0, stream, a);
            return (int)hipGetLastError();
        } else {
            return BF_ERR_UNSUPPORTED;
        }
    }
    if (a.o_dtype == DT_BF16)
        hipLaunchKernelGGL((gdn_seg_kernel<E, D, true, true>), grid, block, 0, stream, a);
    else
        hipLaunchKernelGGL((gdn_seg_kernel<E, D, true, false>), grid, block, 0, stream, a);
    return (int)hipGetLastError();
}

}  // namespace

int gdn_states(const GdnArgs& a, hipStream_t stream, bool summary, bool combine) {
    if (!a.multi_seg) return 0;
    const bool bf = a.in_dtype == DT_BF16;
    const bool su = summary, co = combine;
    switch (a.D) {
        case 64: return bf ? launch_states<BF16, 64>(a, stream, su, co) : launch_states<F32, 64>(a, stream, su, co);
        case 128: return bf ? launch_states<BF16, 128>(a, stream, su, co) : launch_states<F32, 128>(a, stream, su, co);
        case 256: return bf ? launch_states<BF16, 256>(a, stream, su, co) : launch_states<F32, 256>(a, stream, su, co);
        default: return BF_ERR_UNSUPPORTED;
    }
}

int gdn_output(const GdnArgs& a, hipStream_t stream) {
    const bool bf = a.in_dtype == DT_BF16;
    switch (a.D) {
        case 64: return bf ? launch_output<BF16, 64>(a, stream) : launch_output<F32, 64>(a, stream);
        case 128: return bf ? launch_output<BF16, 128>(a, stream) : launch_output<F32, 128>(a, stream);
        case 256: return bf ? launch_output<BF16, 256>(a, stream) : launch_output<F32, 256>(a, stream);
        default: return BF_ERR_UNSUPPORTED;
    }
}

}  // namespace bf
