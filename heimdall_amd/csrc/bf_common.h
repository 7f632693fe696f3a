// Shared device helpers for the Bifrost core kernels (gfx950 / CDNA4 only).
//
// Operand element types: bf16 (storage uint16_t, MFMA v_mfma_f32_16x16x32_bf16) and fp32 (MFMA
// v_mfma_f32_16x16x4_f32). Every MFMA operand fragment is one 16-byte load per lane:
//   - A fragment (M x K tile, 16 rows): lane l holds row (l % 16), elements k0 + VEC*(l/16) .. + VEC-1
//   - B fragment (K x N tile, 16 cols): lane l holds col (l % 16), the same k range
// so both operands are read from memory laid out with K contiguous. A bf16 fragment feeds one 16x16x32
// MFMA; an fp32 fragment feeds four 16x16x4 MFMAs (step s uses k = k0 + 4*(l/16) + s on both operands,
// a consistent permutation of the K index, which leaves the sum unchanged).
// Accumulator (16x16 fp32): lane l holds column (l % 16), rows 4*(l/16) .. +3.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace bf {

typedef __attribute__((ext_vector_type(4))) float f32x4;
typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;

constexpr int WAVE = 64;

__device__ __forceinline__ float bf2f(uint16_t x) { return __uint_as_float(((uint32_t)x) << 16); }
__device__ __forceinline__ uint16_t f2bf(float f) {
    __bf16 b = (__bf16)f;  // v_cvt_pk_bf16_f32: round to nearest even
    return __builtin_bit_cast(uint16_t, b);
}
// Two floats to packed bf16 (x in the low half) with one v_cvt_pk_bf16_f32, round to nearest even.
typedef __attribute__((ext_vector_type(2))) float f32x2;
typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2;
__device__ __forceinline__ uint32_t pack_bf16x2(float x, float y) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{x, y}, bf16x2));
}

// Element-type traits. VEC = elements per 16-byte vector; KF = K covered by one fragment per MFMA group.
struct BF16 {
    using T = uint16_t;
    static constexpr int VEC = 8;
    static constexpr int KF = 32;
    __device__ static __forceinline__ float to_f(T x) { return bf2f(x); }
    __device__ static __forceinline__ T from_f(float f) { return f2bf(f); }
};
struct F32 {
    using T = float;
    static constexpr int VEC = 4;
    static constexpr int KF = 16;
    __device__ static __forceinline__ float to_f(T x) { return x; }
    __device__ static __forceinline__ T from_f(float f) { return f; }
};

// acc += A(16 x KF) * B(KF x 16) for one fragment pair.
template <class E>
__device__ __forceinline__ void mma(f32x4& acc, const uint4& a, const uint4& b);

template <>
__device__ __forceinline__ void mma<BF16>(f32x4& acc, const uint4& a, const uint4& b) {
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), acc,
                                                   0, 0, 0);
}
template <>
__device__ __forceinline__ void mma<F32>(f32x4& acc, const uint4& a, const uint4& b) {
    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(a.x), __uint_as_float(b.x), acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(a.y), __uint_as_float(b.y), acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(a.z), __uint_as_float(b.z), acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(a.w), __uint_as_float(b.w), acc, 0, 0, 0);
}

__device__ __forceinline__ uint4 ld16(const void* p) { return *reinterpret_cast<const uint4*>(p); }
__device__ __forceinline__ void st16(void* p, const uint4& v) { *reinterpret_cast<uint4*>(p) = v; }
__device__ __forceinline__ uint4 zero16() { return make_uint4(0u, 0u, 0u, 0u); }
// Streaming (non-temporal) 16-byte accesses, for data touched once per kernel (the decode step's state slabs, the
// window kernel's queries): the loads and stores skip cache retention, which measured 4 % faster on the state read +
// write of a decode step.
typedef unsigned int nt_u32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ float4 nt_ldf4(const float* p) {
    const nt_u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const nt_u32x4*>(p));
    return make_float4(__uint_as_float(v.x), __uint_as_float(v.y), __uint_as_float(v.z), __uint_as_float(v.w));
}
__device__ __forceinline__ uint4 nt_ld16(const void* p) {
    const nt_u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const nt_u32x4*>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ void nt_stf4(float* p, const float4& s) {
    __builtin_nontemporal_store(nt_u32x4{__float_as_uint(s.x), __float_as_uint(s.y), __float_as_uint(s.z),
                                         __float_as_uint(s.w)}, reinterpret_cast<nt_u32x4*>(p));
}

// Multiply the VEC elements of a 16-byte vector by s (through fp32), returning the same element type.
template <class E>
__device__ __forceinline__ uint4 scale16(const uint4& v, float s);
template <>
__device__ __forceinline__ uint4 scale16<F32>(const uint4& v, float s) {
    return make_uint4(__float_as_uint(__uint_as_float(v.x) * s), __float_as_uint(__uint_as_float(v.y) * s),
                      __float_as_uint(__uint_as_float(v.z) * s), __float_as_uint(__uint_as_float(v.w) * s));
}
__device__ __forceinline__ uint32_t scale_pair(uint32_t p, float s) {
    float lo = __uint_as_float(p << 16) * s, hi = __uint_as_float(p & 0xffff0000u) * s;
    return (uint32_t)f2bf(lo) | ((uint32_t)f2bf(hi) << 16);
}
template <>
__device__ __forceinline__ uint4 scale16<BF16>(const uint4& v, float s) {
    return make_uint4(scale_pair(v.x, s), scale_pair(v.y, s), scale_pair(v.z, s), scale_pair(v.w, s));
}

// Store 4 consecutive fp32 values (an accumulator column segment) as element type E.
template <class E>
__device__ __forceinline__ void store4(typename E::T* p, float a, float b, float c, float d);
template <>
__device__ __forceinline__ void store4<F32>(float* p, float a, float b, float c, float d) {
    *reinterpret_cast<float4*>(p) = make_float4(a, b, c, d);
}
template <>
__device__ __forceinline__ void store4<BF16>(uint16_t* p, float a, float b, float c, float d) {
    uint2 v;
    v.x = (uint32_t)f2bf(a) | ((uint32_t)f2bf(b) << 16);
    v.y = (uint32_t)f2bf(c) | ((uint32_t)f2bf(d) << 16);
    *reinterpret_cast<uint2*>(p) = v;
}

// Transpose a VEC x VEC block held as VEC 16-byte row vectors (rows[i] = row i) into column vectors.
template <class E>
__device__ __forceinline__ void transpose_block(uint4 (&r)[E::VEC]);
template <>
__device__ __forceinline__ void transpose_block<F32>(uint4 (&r)[4]) {
    uint32_t m[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i) { m[i][0] = r[i].x; m[i][1] = r[i].y; m[i][2] = r[i].z; m[i][3] = r[i].w; }
#pragma unroll
    for (int j = 0; j < 4; ++j) r[j] = make_uint4(m[0][j], m[1][j], m[2][j], m[3][j]);
}
template <>
__device__ __forceinline__ void transpose_block<BF16>(uint4 (&r)[8]) {
    uint16_t m[8][8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const uint32_t w[4] = {r[i].x, r[i].y, r[i].z, r[i].w};
#pragma unroll
        for (int j = 0; j < 4; ++j) { m[i][2 * j] = (uint16_t)(w[j] & 0xffffu); m[i][2 * j + 1] = (uint16_t)(w[j] >> 16); }
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        uint32_t w[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) w[i] = (uint32_t)m[2 * i][j] | ((uint32_t)m[2 * i + 1][j] << 16);
        r[j] = make_uint4(w[0], w[1], w[2], w[3]);
    }
}

// s_waitcnt vmcnt(0): all outstanding vector-memory operations of the wave have completed. Used before a loop whose
// first iteration consumes loads issued ahead of it, so the compiler's wait analysis at the loop header starts clean.
__device__ __forceinline__ void wait_vmem_all() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// Workgroup barrier that orders LDS accesses only. __syncthreads() is a workgroup fence over every address space, and
// the fence waits for all of the wave's outstanding global loads and stores (vmcnt(0)), and an LDS-only fence still
// waits for loads into LDS by DMA (buffer_load ... lds), which puts the latency of a prefetch issued earlier on the
// path of every barrier. This barrier waits for the wave's LDS operations only (the memory clobber keeps the compiler
// from moving memory accesses across it). A DMA load whose LDS data is read after it still needs wait_vmem_all().
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// Element offset of (row, col) of a 64 x 64 chunk matrix stored in MFMA A-fragment order: fragment (tt, ks) = 64
// lanes x VEC elements, lane (lg, l16) holding row tpart(tt) + VEC*(l16/4) + l16%4 at K indices KF*ks + VEC*lg + e,
// with tpart(tt) = KF*(tt/HP) + 4*(tt%HP) and HP = VEC/4 (the row permutation under which MFMA accumulator tiles of
// successive products chain without data exchange). Each fragment is one contiguous 1 KB piece.
template <class E>
__device__ __forceinline__ int tfrag_index(int row, int col) {
    constexpr int VEC = E::VEC, KF = E::KF, HP = VEC / 4;
    const int tt = HP * (row / KF) + (row % VEC) / 4;
    const int l16 = 4 * ((row % KF) / VEC) + row % 4;
    const int ks = col / KF, lg = (col % KF) / VEC, e = col % VEC;
    return ((ks * 4 + tt) * 64 + 16 * lg + l16) * VEC + e;
}

__device__ __forceinline__ int lane_id() { return threadIdx.x & (WAVE - 1); }
// Wave index inside the workgroup, marked wave-uniform (readfirstlane) so that values derived from it (buffer
// descriptors, LDS bases, loop bounds) live in SGPRs; plain threadIdx.x / 64 is treated as divergent and descriptors
// built from it are executed in a waterfall loop.
__device__ __forceinline__ int wave_id() { return __builtin_amdgcn_readfirstlane(threadIdx.x / WAVE); }

// Sequence/chunk bookkeeping for packed variable-length input. cu (device, num_seqs + 1 entries) may be null, in
// which case every sequence has length seq_len. Chunk ids enumerate the chunks of sequence 0, then 1, ...
struct SeqInfo {
    int seq;      // sequence index
    int chunk;    // chunk index inside the sequence
    long tok0;    // first token of the chunk (packed index)
    int len;      // valid tokens in the chunk (1..C)
};

__device__ __forceinline__ bool locate_chunk(int cid, const int32_t* cu, int num_seqs, int seq_len, int C,
                                             SeqInfo& out) {
    int base = 0;
    for (int n = 0; n < num_seqs; ++n) {
        const long s0 = cu ? (long)cu[n] : (long)n * seq_len;
        const long s1 = cu ? (long)cu[n + 1] : (long)(n + 1) * seq_len;
        const int nc = (int)((s1 - s0 + C - 1) / C);
        if (cid < base + nc) {
            out.seq = n;
            out.chunk = cid - base;
            out.tok0 = s0 + (long)out.chunk * C;
            const long rem = s1 - out.tok0;
            out.len = rem < C ? (int)rem : C;
            return true;
        }
        base += nc;
    }
    return false;
}

// First chunk id of sequence n and its chunk count.
__device__ __forceinline__ void seq_chunks(int n, const int32_t* cu, int seq_len, int C, int& first, int& count,
                                           long& tok0, long& tok1) {
    int base = 0;
    for (int m = 0; m < n; ++m) {
        const long s0 = cu ? (long)cu[m] : (long)m * seq_len;
        const long s1 = cu ? (long)cu[m + 1] : (long)(m + 1) * seq_len;
        base += (int)((s1 - s0 + C - 1) / C);
    }
    tok0 = cu ? (long)cu[n] : (long)n * seq_len;
    tok1 = cu ? (long)cu[n + 1] : (long)(n + 1) * seq_len;
    first = base;
    count = (int)((tok1 - tok0 + C - 1) / C);
}

}  // namespace bf

namespace bf {

// Buffer-resource memory access: the (uniform) base address and byte range live in an SGPR descriptor, each lane
// supplies a 32-bit byte offset. Loads outside [0, nbytes) return 0 and stores outside are dropped, which the
// kernels use for rows past the end of a sequence.
typedef __amdgpu_buffer_rsrc_t rsrc_t;
constexpr int kRsrcWord3 = 0x00020000;   // raw (untyped) 32-bit buffer, gfx9-family layout

// The base and range must be wave-uniform: they are moved to SGPRs with readfirstlane (a descriptor the compiler
// cannot prove uniform is otherwise used through a waterfall loop, one iteration per distinct lane value).
__device__ __forceinline__ rsrc_t make_rsrc(const void* base, uint32_t nbytes) {
    const uint64_t b = reinterpret_cast<uint64_t>(base);
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)b);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(b >> 32));
    void* ub = reinterpret_cast<void*>(((uint64_t)hi << 32) | lo);
    return __builtin_amdgcn_make_buffer_rsrc(ub, (short)0, (int)__builtin_amdgcn_readfirstlane(nbytes), kRsrcWord3);
}
__device__ __forceinline__ uint4 buf_ld16(rsrc_t r, uint32_t off) {
    return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}
__device__ __forceinline__ float4 buf_ldf4(rsrc_t r, uint32_t off) {
    return __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}
__device__ __forceinline__ uint2 buf_ld8(rsrc_t r, uint32_t off) {
    return __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0));
}
__device__ __forceinline__ float buf_ldf(rsrc_t r, uint32_t off) {
    return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0));
}
__device__ __forceinline__ void buf_stf(rsrc_t r, uint32_t off, float v) {
    __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, v), r, off, 0, 0);
}
__device__ __forceinline__ void buf_sth(rsrc_t r, uint32_t off, uint16_t v) {
    __builtin_amdgcn_raw_buffer_store_b16(v, r, off, 0, 0);
}
__device__ __forceinline__ void buf_st16(rsrc_t r, uint32_t off, const uint4& v) {
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(__attribute__((ext_vector_type(4))) uint32_t, v), r,
                                           off, 0, 0);
}

// Store one fp32 value as the output element type (fp32 or bf16) through a buffer descriptor.
template <bool BF16OUT>
__device__ __forceinline__ void buf_st_out(rsrc_t r, uint32_t elem, float v) {
    if constexpr (BF16OUT) buf_sth(r, elem * 2u, f2bf(v));
    else buf_stf(r, elem * 4u, v);
}

// ------------------------------------------------------------------------------------------------ LDS staging
// 16-byte block permutation of LDS row `row` of a tile with nblk >= 8 blocks per row, chosen by measurement on gfx950
// with 4 and 8 waves reading the same tile concurrently (the case in the scan kernels):
//  - bf16 rows of >= 16 blocks: every 16-lane phase of an MFMA fragment read (the 16 rows prow(tile, 0..15) at one
//    block) and of a transposing K^T read (rows 4 consecutive tokens from a multiple of 4, 4 lanes each) spreads over
//    16 distinct blocks, at the same speed as a linear read;
//  - bf16 rows of 8 blocks and fp32: 3-bit form (8 distinct blocks per fragment phase).
// The value depends on the row only through row & 3, (row >> 3) & 3 and bit 1 or bit 2, so fragment addresses are a
// per-lane base plus an instruction immediate.
template <class E>
__device__ __forceinline__ int swz(int row, int nblk) {
    if constexpr (E::VEC == 8) {
        if (nblk >= 16) return (row & 3) | ((((row >> 3) & 3) ^ (row & 2)) << 2);
        return (row & 3) | ((((row >> 3) ^ row) & 1) << 2);
    } else {
        return (row & 3) | (((row >> 2) & 1) << 2);
    }
}

// 16-byte block permutation of the V tile rows (rows of VROWB >= 128 bytes): the 4 consecutive rows (from a multiple
// of 4) that a 16-lane group of a transposing V read touches land 32 bytes apart, and bit 3 separates the two 16-lane
// groups of a 32-lane half, so those 8-byte reads do not share banks.
__device__ __forceinline__ int swz_v(int row, int nblk) { return ((2 * (row & 3)) | (((row >> 3) & 1) << 3)) & (nblk - 1); }

// Per-chunk operands, double-buffered for bf16: K (C x D), T' and attn (C x C), gc.
__device__ __forceinline__ uint4 lds16(const void* base, int byte_off) {
    return *reinterpret_cast<const uint4*>(reinterpret_cast<const char*>(base) + byte_off);
}

// Cache policy of a buffer access: streaming (non-temporal), for data read or written once per kernel.
constexpr int kCpolStream = 2;

// Copy a tile of SC rows into LDS with buffer_load ... lds: LDS row r (rowb bytes) holds global row r (pitch bytes)
// with its 16-byte blocks permuted by sw(r). One instruction moves 64 x 16 bytes; `nbytes` = SC * rowb is a multiple
// of 1 KB. Blocks at or beyond `valid_blk` of a row read as zero, as do rows past the descriptor's range. `cpol`:
// the loads' cache policy (0, or kCpolStream for rows no other workgroup reads).
template <int cpol = 0, class Swz>
__device__ __forceinline__ void stage_tile(rsrc_t src, uint32_t pitch, int rowb, void* lds, int nbytes, int wv,
                                           int nw, int lane, Swz sw, int valid_blk) {
    const int nblk = rowb / 16;
    for (int i = wv; i < nbytes / 1024; i += nw) {
        const int s = i * 64 + lane;
        const int r = s / nblk, pb = s % nblk;
        const int lb = pb ^ sw(r);
        const uint32_t off = lb < valid_blk ? (uint32_t)r * pitch + (uint32_t)(lb * 16) : 0xFFFFFFF0u;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            src, (__attribute__((address_space(3))) void*)(reinterpret_cast<char*>(lds) + i * 1024), 16, off, 0, 0,
            cpol);
    }
}

}  // namespace bf
