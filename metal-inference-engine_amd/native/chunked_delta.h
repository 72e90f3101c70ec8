// Definitions shared by the two translation units of P3 (the chunked gated delta rule): chunked_delta.hip (the
// prep kernel, the fp32-input scan, the C ABI) and chunked_delta_cols.hip (the bf16-input scan, built with MFMA
// results in VGPRs). See chunked_delta.hip for the semantics.
#pragma once

#include "rk_device.h"

namespace rk {
namespace delta {


constexpr int kC = 64;                       // tokens per chunk
constexpr int kDk = 128, kDv = 128;
constexpr int kCT = 2;                       // 16-column tiles of the state per scan wave
constexpr int kCols = 16 * kCT;              // state columns per scan workgroup
constexpr int kSlices = kDv / kCols;         // 4
constexpr int kNS = 3;                       // bf16 pieces of an fp32 operand that changes with the state
// bf16 pieces of the stored T and P entries: 3 = exact (truncation); 2 = round to nearest (2^-17), which saves a
// third of the workspace traffic (6% of the call at config 4) but raises the output error ~10x, to ~5e-6
constexpr int kTP = 3;
constexpr int kCoefRows = 4;                 // beta, G, exp(G), exp(G_last - G)
// per (chunk, head): T and P as kTP bf16 pieces of 3072 elements each, then the coefficient rows
constexpr int kChunkFloats = 2 * kTP * 3072 / 2 + kCoefRows * kC;
constexpr int kPieceRow = kC + 8;            // bf16 row stride of the [piece][column][token] exchange arrays
constexpr int kStateRow = kDk + 8;           // bf16 row stride of the [piece][column][dk] state pieces

struct DeltaArgs {
    float* out;                 // [N, H, dv] fp32
    float* S;                   // state of sequence i at S + idx(i) * s_stride, [H, dk, dv] fp32, in place
    const void* q;              // [N, H, dk] bf16 or fp32 (q already scaled)
    const void* k;              // [N, H, dk]
    const void* v;              // [N, H, dv]
    const float* beta;          // [N, H]
    const float* g;             // [N, H] log-decay (<= 0)
    const int32_t* cu;          // [n_seqs + 1] token offsets
    const int32_t* cu_chunks;   // [n_seqs + 1] chunk offsets (ceil(len / 64) per sequence)
    const int32_t* seq_index;   // [n_seqs] state index of each sequence, or null for 0 .. n_seqs-1
    float* ws;                  // [total_chunks, H] records of kChunkFloats floats
    long long s_stride;
    int n_seqs, H, n_pairs;
};

// ---- operands: 8 consecutive elements of one row per lane, as bf16 pieces
__device__ __forceinline__ uint32_t mask_if(bool keep) { return keep ? 0xffffffffu : 0u; }
__device__ __forceinline__ float to_f32(uint16_t x) { return __uint_as_float((uint32_t)x << 16); }
__device__ __forceinline__ float to_f32(uint32_t x) { return __uint_as_float(x << 16); }   // bf16 bits, zero-extended
__device__ __forceinline__ float to_f32(float x) { return x; }

template <typename In> struct Row8;
template <> struct Row8<uint16_t> {            // bf16 input: one exact piece
    static constexpr int KP = 1;
    u32x4 v;
    __device__ __forceinline__ void load(const uint16_t* p) { v = *reinterpret_cast<const u32x4*>(p); }
    __device__ __forceinline__ void keep(uint32_t m) { v &= (u32x4){m, m, m, m}; }
    __device__ __forceinline__ void pieces(u32x4 (&o)[1]) const { o[0] = v; }
    __device__ __forceinline__ uint16_t raw(int e) const { return (uint16_t)(v[e >> 1] >> (16 * (e & 1))); }
};
template <> struct Row8<float> {               // fp32 input: three pieces
    static constexpr int KP = kNS;
    f32x4 a, b;
    __device__ __forceinline__ void load(const float* p) {
        a = *reinterpret_cast<const f32x4*>(p);
        b = *reinterpret_cast<const f32x4*>(p + 4);
    }
    __device__ __forceinline__ void keep(uint32_t m) {
        for (int e = 0; e < 4; ++e) {
            a[e] = __uint_as_float(__float_as_uint(a[e]) & m);
            b[e] = __uint_as_float(__float_as_uint(b[e]) & m);
        }
    }
    __device__ __forceinline__ float raw(int e) const { return e < 4 ? a[e] : b[e - 4]; }
    __device__ __forceinline__ void pieces(u32x4 (&o)[kNS]) const;
};

// Exact split of 8 fp32 values into kNS bf16 pieces, packed as MFMA operands (element e in slot e).
__device__ __forceinline__ void split8(const float (&x)[8], u32x4 (&o)[kNS]) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const Split3 s0 = split3(x[2 * j]), s1 = split3(x[2 * j + 1]);
        o[0][j] = pack_hi2(s0.hi, s1.hi);
        o[1][j] = pack_hi2(s0.mid, s1.mid);
        o[2][j] = pack_hi2(s0.lo, s1.lo);
    }
}
// Two-piece split of 4 fp32 values, rounding to nearest at both steps: x = hi + lo + e with |e| <= 2^-17 |x|.
__device__ __forceinline__ void split4_rn(const float (&x)[4], u32x2 (&o)[kTP]) {
    uint32_t hi[4], lo[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        hi[e] = f32_to_bf16_rne(x[e]);
        lo[e] = f32_to_bf16_rne(x[e] - __uint_as_float(hi[e] << 16));
    }
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        o[0][j] = hi[2 * j] | (hi[2 * j + 1] << 16);
        o[1][j] = lo[2 * j] | (lo[2 * j + 1] << 16);
    }
}
// Split of 4 fp32 values: kNS pieces of 4 bf16 each (2 dwords).
__device__ __forceinline__ void split4(const float (&x)[4], u32x2 (&o)[kNS]) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const Split3 s0 = split3(x[2 * j]), s1 = split3(x[2 * j + 1]);
        o[0][j] = pack_hi2(s0.hi, s1.hi);
        o[1][j] = pack_hi2(s0.mid, s1.mid);
        o[2][j] = pack_hi2(s0.lo, s1.lo);
    }
}

__device__ __forceinline__ void Row8<float>::pieces(u32x4 (&o)[kNS]) const {
    const float x[8] = {a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
    split8(x, o);
}

// Sum of the piece products a_i * b_j with i + j < kNS (smallest terms first).
template <int PA, int PB>
__device__ __forceinline__ f32x4 mma(const u32x4 (&a)[PA], const u32x4 (&b)[PB], f32x4 c) {
#pragma unroll
    for (int d = kNS - 1; d >= 0; --d)
#pragma unroll
        for (int i = 0; i < PA; ++i) {
            const int j = d - i;
            if (j >= 0 && j < PB) c = mfma16x16x32(a[i], b[j], c);
        }
    return c;
}

__device__ __forceinline__ f32x4 mfma_f32(float a, float b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// Sequence owning global chunk gc: the last s with cu_chunks[s] <= gc (empty sequences own no chunk).
__device__ __forceinline__ int seq_of_chunk(const DeltaArgs& p, int gc) {
    int lo = 0, hi = p.n_seqs;
    while (hi - lo > 1) {
        const int mid = (lo + hi) >> 1;
        if (p.cu_chunks[mid] <= gc) lo = mid; else hi = mid;
    }
    return lo;
}

// Per-chunk workspace record (floats): T and P as kNS bf16 pieces each, in the operand order the scan reads, then the
// coefficient rows. Row tile a (rows 16a .. 16a+15) keeps columns 0 .. rt_width(a)-1, the 32-token k-steps that reach
// its diagonal: 32, 32, 64, 64 columns (3072 elements per piece).
__host__ __device__ constexpr int rt_width(int a) { return a < 2 ? 32 : 64; }
__host__ __device__ constexpr int rt_base(int a) { return a == 0 ? 0 : (a == 1 ? 512 : (a == 2 ? 1024 : 2048)); }
constexpr int kPieceElems = 3072;                                  // bf16 elements of one piece of T or P
constexpr int kTOff = 0;                                           // T pieces   (uint16 offset)
constexpr int kPOff = kTP * kPieceElems;                           // P pieces   (uint16 offset)
constexpr int kCoefOff = kTP * kPieceElems;                        // coefficients (float offset: after 2 x kTP pieces)

// Per-chunk workspace record of the bf16-input path (delta_chunk_scan_cols): T as an fp32 lower triangle, row i
// holding columns 0 .. i zero-padded to a multiple of 4 floats from tri_base(i), then the coefficient rows (9.5 KB,
// a quarter of the pieces' size: the scan's loading waves split T into pieces in LDS themselves, and compute P from
// the chunk's K and Q rows).
__host__ __device__ constexpr int tri_base(int i) { return 4 * (i / 4 + 1) * (2 * (i / 4) + i % 4); }
constexpr int kTriFloats = tri_base(kC);                            // 2176
constexpr int kLaneCoefOff = kTriFloats;                            // float offsets: T at 0, then the coefficients
constexpr int kLaneChunkFloats = kLaneCoefOff + kCoefRows * kC;     // record stride (floats)
static_assert(kLaneChunkFloats <= kChunkFloats, "the workspace size covers both record layouts");
static_assert(kLaneChunkFloats % 64 == 0, "records stay 256-byte aligned");

// Lane order (bf16 inputs, the LDS stage of delta_chunk_scan_cols): the A operand of row tile a and 32-token k-step
// k (the pairs (a, k) with k <= a / 2, numbered pair_of(a, k) = 0 .. 5) is one 1 KB block per piece, block 6 pi +
// pair, lane (q, r) holding 8 bf16 at 16 lane bytes: entries (16a + r, 32k + perm(8q + e)), where perm(8q + e) =
// 4q + e for e < 4 and 16 + 4q + (e - 4) for e >= 4. That k order is the one in which an MFMA accumulator pair (row
// tiles 2k, 2k+1, lane (q, r) holding rows 4q + i) is already a B operand, so no operand of the scan is transposed.
__host__ __device__ constexpr int pair_of(int a, int k) { return a < 2 ? a : 2 + 2 * (a - 2) + k; }
__device__ __forceinline__ int perm_k(int j) { return (j & 4 ? 16 : 0) + 4 * (j >> 3) + (j & 3); }

// The bf16-input scan (chunked_delta_cols.hip): `grid` workgroups of 256 threads, ids mapped as delta_chunk_scan's.
int launch_scan_cols(const DeltaArgs& a, int grid, hipStream_t stream);

}  // namespace delta
}  // namespace rk
