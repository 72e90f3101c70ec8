// P1: paged GQA decode attention over a block-table KV pool, gfx950.
//
// Semantics (reference): TorchBackend.paged_attention gathers each sequence's positions through its block table and
// runs ops.attention with one query (src/backend/torch_ref.py:75-88, src/ops.py:65-104); the Metal kernel it
// replaces is paged_attention_decode<T> (src/kernels/attention.metal:87-159). Pool row of position s of sequence i:
// ((tables[i][s / bs] * bs + s % bs) * Hkv + kvh) * D (attention.metal:115).
//
// Design (split over positions, then a merge):
//   * Work unit = one 16-position tile of one sequence. The tiles of the whole batch, in (sequence, tile) order,
//     are cut into NW contiguous ranges of equal cost (stream-K): a tile costs one unit and each sequence kSegCost
//     more (its segment's combine and restart); workgroup w takes cost units [Uc w / NW, Uc (w + 1) / NW) of the Uc
//     in all, so every workgroup does the same work however unequal the lengths are (with under kSegMinTiles tiles
//     per workgroup, tiles [U w / NW, U (w + 1) / NW) of the U in all). A range
//     may cross sequence boundaries; the workgroup writes one partial (m, l, acc) per kv-head for each sequence it
//     touches, into slot w + b (unique: a later workgroup never touches an earlier sequence). NW is sized so that
//     the whole grid is resident at once (no second wave of workgroups).
//   * A split workgroup has one wave per kv-head; the waves walk the same tiles, so the interleaved halves of every
//     pool row ([bs][Hkv][D]) are fetched together. Each wave serves all G = Hq/Hkv query heads of its kv-head, so
//     every K/V byte is read from HBM once.
//   * QK^T on MFMA (v_mfma_f32_16x16x32_bf16): A = the G query rows split exactly into three bf16 parts
//     (q = hi + mid + lo, built in LDS by the whole wave when a sequence starts), B = 16 keys x 32 dims. bf16 keys
//     are exact MFMA operands; fp32 keys are split the same way (three MFMA passes), so both pool types get
//     fp32-accurate scores, and a bf16 pool gives bit for bit the result of the fp32 pool holding the widened values
//     (the extra passes only add exact zeros).
//   * Loads are software-pipelined: each register set of keys (values) is refilled with the next tile's as soon as
//     this tile's MFMA operands (widened values) are taken from it, so a wave has the next tile in flight for
//     nearly the whole of this tile's compute, also across a sequence boundary. One
//     vector load per 64 tiles fetches each tile's sequence, position and (block_size % 16 == 0) block number.
//   * Online softmax in base 2 (scores pre-scaled by log2(e)/sqrt(D)); row max by DPP inside 16-lane rows.
//   * PV on the VALU in fp32: each lane owns 8 consecutive dims of one position row (coalesced 16/32-byte loads);
//     probabilities are broadcast through LDS.
//   * Merge kernel: one workgroup per (sequence, kv-head) finds the sequence's workgroups in closed form from the
//     same tile prefix sums, combines their partials in workgroup order, divides, applies the optional sigmoid gate
//     and writes [B, Hq, D].
// Bounds: lens are clamped to max_nb * bs and table entries to [0, num_blocks), so a malformed table cannot make a
// load leave the pool. Positions outside [s0, len) are never used: their scores are replaced (not added) by -inf and
// their V values by 0 before the FMA, so a NaN-poisoned block outside the window cannot leak in.
#include "rk_device.h"
#include "rk_internal.h"

#include <mutex>

namespace rk {

// Split-K partials of the allocation-free entry point (rk_paged_decode_noalloc): a file-scope device array, one
// copy per GPU, held until the process ends. Host code never passes the array's name to a kernel (on the host it
// is only a stand-in for the symbol); each device's address comes from hipGetSymbolAddress with that device current.
constexpr size_t kScratchBytes = size_t(16) << 20;
static __device__ __align__(256) char scratch[kScratchBytes];

namespace {

constexpr int kMaxBatch = 1024;
constexpr int kMaxKvHeads = 4;     // one wave per kv head in a split workgroup of at most 256 threads
constexpr int kTile = 16;
constexpr int kStash = 2;   // segments per split workgroup whose records wait in LDS until the range is done
// Waves of a split workgroup: 4, one per SIMD, with up to 512 registers each, so that every instance holds the
// whole next tile in flight, the values included, while it computes this one. With the non-temporal K/V loads this
// beats 8-wave workgroups (two waves per SIMD, 256 registers, at most half of the next tile's values early) at
// every batch size measured: config 3's split kernel 88.5 -> 86.5 us, batch 128 169.6 -> 165.7 us, batch 256
// 351.5 -> 344.9 us, batch 16 unchanged (with temporal loads the 8-wave form had been faster, 101 vs 104 us at
// config 3). Two 4-wave workgroups per CU measured slower again (87.6-88.1 us at config 3). The count is the same
// for both pool dtypes, so a bf16 pool and an fp32 pool holding the same (widened) values are cut and combined
// identically and give bit-equal outputs.
constexpr int kSplitWaves = 4;
// the tile count's upper bound: every sequence at its table's full width
inline long long tile_upper(int B, int block_size, int max_nb) {
    return (long long)B * (((long long)max_nb * block_size + kTile - 1) / kTile);
}

struct DecodeArgs {
    const int32_t* plan;  // the batch layout plan of rk_paged_decode_plan, or null (computed in the kernels)
    float* part;
    float* out;
    const float* q;
    const void* kp;
    const void* vp;
    const int32_t* tables;
    const int32_t* lens;
    const float* gate;
    long long gate_ld;  // elements between the gate rows of consecutive sequences
    int B, Hq, Hkv, G, bs, max_nb, num_blocks, window, NW;
    int NG;         // groups of Hkv waves in a split workgroup
    float qscale;   // log2(e) / sqrt(D)
};

struct SeqRange {
    int L, s0, t0, units;   // clamped length, first visible position, first tile, tile count
};

__device__ __forceinline__ SeqRange seq_range(const DecodeArgs& a, int b) {
    SeqRange r;
    int L = a.lens[b];
    int cap = a.max_nb * a.bs;
    L = L < cap ? L : cap;
    if (L <= 0) {
        r.L = 0; r.s0 = 0; r.t0 = 0; r.units = 0;
        return r;
    }
    r.L = L;
    r.s0 = (a.window > 0 && L > a.window) ? L - a.window : 0;
    r.t0 = r.s0 / kTile;
    r.units = (L + kTile - 1) / kTile - r.t0;
    return r;
}

// Element offset of position s (already clamped to a visible position) of one sequence / kv-head.
__device__ __forceinline__ long long kv_row(const int32_t* table, int s, int bs, int Hkv, int kvh, int D,
                                            int num_blocks) {
    int blk = table[s / bs];
    blk = blk < 0 ? 0 : (blk >= num_blocks ? num_blocks - 1 : blk);
    return ((long long)(blk * (long long)bs + s % bs) * Hkv + kvh) * D;
}

// Cost units a sequence adds to a split workgroup's range besides its tiles: a segment ends with a combine of the
// groups' states, a partial record and a query restage, and its first tiles wait on a new block-table row. Per
// workgroup that costs about as much as streaming a few more tiles (at batch 64 the split kernel measured 100.8 /
// 98.4 / 98.0 / 98.9 / 99.7 µs at 0 / 2 / 4 / 5 / 6 units). The ranges are cut by cost only when the workgroups
// average at least kSegMinTiles tiles; with a tile or two per group (batch 1, small batches) a whole cost unit is
// too coarse, and the ranges are cut by tiles.
constexpr int kSegCost = 4;
constexpr int kSegMinTiles = 16;

// Tile prefix sums, computed by one wave: P[0] = 0, P[b + 1] = P[b] + units(b); with Ls, also Ls[b] = the clamped
// length of sequence b; with V, the same sums in cost units, V[b + 1] = V[b] + units(b) + (units(b) > 0 ? kSegCost
// : 0). Returns U = P[B] (all tiles).
__device__ int plan_prefix(const DecodeArgs& a, int* P, int* Ls = nullptr, int* V = nullptr) {
    const int lane = threadIdx.x & 63;
    int carry = 0, vcarry = 0;
    for (int b0 = 0; b0 < a.B; b0 += 64) {
        const int b = b0 + lane;
        const SeqRange sr = b < a.B ? seq_range(a, b) : SeqRange{0, 0, 0, 0};
        if (Ls && b < a.B) Ls[b] = sr.L;
        int x = sr.units, y = sr.units + (sr.units > 0 ? kSegCost : 0);
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
            const int xu = __shfl_up(x, off), yu = __shfl_up(y, off);
            if (lane >= off) { x += xu; y += yu; }
        }
        if (b < a.B) P[b + 1] = carry + x;
        if (V && b < a.B) V[b + 1] = vcarry + y;
        carry += __shfl(x, 63);
        vcarry += __shfl(y, 63);
    }
    if (lane == 0) {
        P[0] = 0;
        if (V) V[0] = 0;
    }
    return carry;
}

// First cost unit of workgroup w's range (Uc cost units over NW workgroups).
__device__ __forceinline__ int range_lo(int Uc, int NW, int w) { return (int)((long long)Uc * w / NW); }

// Sequence of global tile g (0 <= g <= P[B], g the same in every lane): the largest b in [0, B) with P[b] <= g,
// which for g < P[B] has P[b + 1] > g; g = P[B] (the end of the last range) gives B - 1. P is non-decreasing from
// P[0] = 0, so b = #{b' in [1, B) : P[b'] <= g}: one ballot per 64 sequences, with independent LDS reads (a binary
// search would chain log2(B) dependent ones). tile_at calls it on the cost sums V with v up to V[B] inclusive.
__device__ __forceinline__ int seq_of_tile(const int* P, int B, int g) {
    const int lane = threadIdx.x & 63;
    int b = 0;
    for (int c = 1; c < B; c += 64) {
        const int bb = c + lane;
        b += __popcll(__ballot(bb < B && P[bb] <= g));
    }
    return b;
}

// Global tile at cost unit v (0 <= v <= V[B]): sequence b's cost units [V[b], V[b + 1]) are its kSegCost segment
// units, which all map to its first tile, then one unit per tile. Non-decreasing in v, P[B] at v = V[B], and a
// sequence's first tile maps back from cost unit V[b] + kSegCost.
__device__ __forceinline__ int tile_at(const int* P, const int* V, int B, int v) {
    const int b = seq_of_tile(V, B, v);
    const int n = P[b + 1] - P[b], c = n > 0 ? kSegCost : 0;
    const int t = v - V[b] - c;
    return P[b] + (t < 0 ? 0 : (t > n ? n : t));
}

template <typename T>
struct KVLoad;

// bf16 pool: 8 elements = one 16-byte load.
template <>
struct KVLoad<uint16_t> {
    static constexpr int KS = 1;   // key splits
    struct Vec { u32x4 w; };
    // Non-temporal: every K / V byte of a decode is read exactly once, and streaming it past the caches (instead of
    // allocating it there) raised the split kernel's HBM rate at config 3 from 5.57 to 5.90 TB/s (same bits)
    __device__ static Vec load(const void* base, long long off) {
        Vec v;
        v.w = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(reinterpret_cast<const uint16_t*>(base) + off));
        return v;
    }
    __device__ static void key_operands(const Vec& v, u32x4* ops) { ops[0] = v.w; }
    __device__ static void keep_if(Vec& v, bool keep) {
        const uint32_t m = keep ? 0xffffffffu : 0u;
        v.w &= u32x4{m, m, m, m};
    }
    __device__ static void widen(const Vec& v, float* f) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            f[2 * j] = bf16_lo(v.w[j]);
            f[2 * j + 1] = bf16_hi(v.w[j]);
        }
    }
};

// fp32 pool: 8 elements = two 16-byte loads; keys are split into three exact bf16 parts.
template <>
struct KVLoad<float> {
    static constexpr int KS = 3;
    struct Vec { u32x4 w0, w1; };
    __device__ static Vec load(const void* base, long long off) {
        const u32x4* p = reinterpret_cast<const u32x4*>(reinterpret_cast<const float*>(base) + off);
        Vec v;
        v.w0 = p[0];
        v.w1 = p[1];
        return v;
    }
    __device__ static void keep_if(Vec& v, bool keep) {
        const uint32_t m = keep ? 0xffffffffu : 0u;
        v.w0 &= u32x4{m, m, m, m};
        v.w1 &= u32x4{m, m, m, m};
    }
    __device__ static void key_operands(const Vec& v, u32x4* ops) {
        Split3 s[8];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            s[j] = split3(__uint_as_float(v.w0[j]));
            s[4 + j] = split3(__uint_as_float(v.w1[j]));
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            ops[0][j] = pack_hi2(s[2 * j].hi, s[2 * j + 1].hi);
            ops[1][j] = pack_hi2(s[2 * j].mid, s[2 * j + 1].mid);
            ops[2][j] = pack_hi2(s[2 * j].lo, s[2 * j + 1].lo);
        }
    }
    __device__ static void widen(const Vec& v, float* f) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            f[j] = __uint_as_float(v.w0[j]);
            f[4 + j] = __uint_as_float(v.w1[j]);
        }
    }
};

// LDS bytes of the per-sequence plan of a split workgroup: tile prefix sums [B + 1], clamped lengths [B] and cost
// prefix sums [B + 1].
constexpr int seq_lds_bytes(int B) { return ((3 * B + 2) * 4 + 15) & ~15; }

// The batch layout plan (rk_paged_decode_plan), int32: a header of kPlanHdr ints (U, Uc, NW, NG, B, by_cost,
// max_nb, block_size), then the per-sequence arrays in the split kernel's LDS layout (P [B + 1], Ls [B], V [B + 1],
// padded to seq_lds_bytes), then per split workgroup w {lo, hi, bA, bZ} (its tile range and first / last
// sequence), then per (w, group g) the group's first 64 tile list entries, one int4 {b, tpos, L, blk} per lane
// (b = -1: no tile): what the split kernel otherwise derives from the lengths and the block table before its first
// K / V load. The entries start 16-byte aligned.
constexpr int kPlanHdr = 8;
constexpr int plan_seq_ints(int B) { return seq_lds_bytes(B) / 4; }
inline size_t plan_ints(int B, int NW, int NG) {
    return kPlanHdr + plan_seq_ints(B) + 4 * (size_t)NW + (size_t)4 * 64 * NW * NG;
}

// LDS bytes one wave of the split kernel uses: the query A operands (NT x NIT x 64 lanes x 16 B), the 16 x GP
// probabilities of the current tile and the GP rescale factors.
template <int D, int GP>
constexpr int wave_lds_bytes() {
    return ((3 * GP + 15) / 16) * (D / 32) * 64 * 16 + kTile * GP * 4 + GP * 4;
}

// Element offsets of the pool rows this lane reads for one tile, and which of them are visible positions. With
// block-aligned tiles (ALIGNED: block_size % 16 == 0) the 16 positions lie in one block, so the V rows are one base
// plus a uniform stride; otherwise every row is looked up through the table (positions clamped to visible ones).
template <int NVI, int TPI, int LPT, bool ALIGNED>
struct TileRows;

template <int NVI, int TPI, int LPT>
struct TileRows<NVI, TPI, LPT, true> {
    long long krow, vbase, vstride;
    uint32_t vmask;            // bit vi: V position of step vi is visible
    bool kvalid, partial;
    __device__ long long vrow(int vi) const { return vbase + vi * vstride; }
    __device__ bool vvalid(int vi) const { return (vmask >> vi) & 1u; }
};

template <int NVI, int TPI, int LPT>
struct TileRows<NVI, TPI, LPT, false> {
    long long krow, vr[NVI];
    uint32_t vmask;
    bool kvalid, partial;
    __device__ long long vrow(int vi) const { return vr[vi]; }
    __device__ bool vvalid(int vi) const { return (vmask >> vi) & 1u; }
};

template <int NVI, int TPI, int LPT, bool ALIGNED>
__device__ __forceinline__ TileRows<NVI, TPI, LPT, ALIGNED> tile_rows(const DecodeArgs& a, const int32_t* table,
                                                                        int s0, int L, int tbase, int blk, int kvh,
                                                                        int D, int lane) {
    TileRows<NVI, TPI, LPT, ALIGNED> r;
    r.partial = tbase < s0 || tbase + kTile > L;
    const int tk = tbase + (lane & 15);
    r.kvalid = tk >= s0 && tk < L;
    r.vmask = 0;
#pragma unroll
    for (int vi = 0; vi < NVI; ++vi) {
        const int tv = tbase + vi * TPI + lane / LPT;
        r.vmask |= (uint32_t)(tv >= s0 && tv < L) << vi;
    }
    if constexpr (ALIGNED) {
        // rows past the length are still rows of the allocated block: no clamping needed for addressing
        const long long row0 = (long long)blk * a.bs + tbase % a.bs;
        r.krow = ((row0 + (lane & 15)) * a.Hkv + kvh) * D;
        r.vbase = ((row0 + lane / LPT) * a.Hkv + kvh) * D + (lane % LPT) * 8;
        r.vstride = (long long)TPI * a.Hkv * D;
    } else {
        const int tkc = tk < s0 ? s0 : (tk >= L ? L - 1 : tk);
        r.krow = kv_row(table, tkc, a.bs, a.Hkv, kvh, D, a.num_blocks);
#pragma unroll
        for (int vi = 0; vi < NVI; ++vi) {
            const int tv = tbase + vi * TPI + lane / LPT;
            const int tvc = tv < s0 ? s0 : (tv >= L ? L - 1 : tv);
            r.vr[vi] = kv_row(table, tvc, a.bs, a.Hkv, kvh, D, a.num_blocks) + (lane % LPT) * 8;
        }
    }
    return r;
}

// Group g's share of split workgroup w's tile range [lo, hi) (first / last sequences bA, bZ), and the entries of the
// group's tile list: within each sequence segment of the range the group takes the segment's tiles g, g + NG, ...;
// entry e of the list is (sequence, first position, clamped length, first visible position, physical block). The
// split kernel and the plan kernel both derive their entries here, so a plan holds exactly what the split kernel
// would compute itself.
struct GroupRange {
    const int* P;           // tile prefix sums [B + 1]
    const int* Ls;          // clamped lengths [B]
    int lo, hi, bA, bZ, g, NG;
    __device__ int seg_lo(int b) const { const int x = P[b]; return (x > lo ? x : lo) - lo; }
    __device__ int seg_hi(int b) const { const int x = P[b + 1]; return (x < hi ? x : hi) - lo; }
    __device__ int count(int b) const {
        const int len = seg_hi(b) - seg_lo(b);
        return len > g ? (len - g + NG - 1) / NG : 0;
    }
    __device__ int total() const {
        int t = 0;
        for (int b = bA; b <= bZ; ++b) t += count(b);
        return t;
    }
};

struct TileEntry {
    int b, tpos, L, s0, blk;
};

// Entry e (clamped to [0, total)) of the group's tile list; bA .. bZ is the same in every lane, so the loop is
// uniform and each lane keeps the segment holding its entry.
template <bool ALIGNED>
__device__ __forceinline__ TileEntry tile_entry(const DecodeArgs& a, const GroupRange& r, int e, int total) {
    e = e < total ? e : total - 1;
    int b = r.bA, k = 0;
    for (int bb = r.bA; bb <= r.bZ; ++bb) {
        const int c = r.count(bb);
        if (e >= 0 && e < c) { b = bb; k = e; }
        e -= c;
    }
    const int gt = r.lo + r.seg_lo(b) + r.g + k * r.NG;   // global tile
    TileEntry x;
    x.b = b;
    x.L = r.Ls[b];
    x.s0 = (a.window > 0 && x.L > a.window) ? x.L - a.window : 0;
    x.tpos = (x.s0 / kTile + gt - r.P[b]) * kTile;
    x.blk = 0;
    if (ALIGNED) {
        int ti = x.tpos / a.bs;                          // < ceil(L / bs) <= max_nb for a consistent plan
        ti = ti < 0 ? 0 : (ti >= a.max_nb ? a.max_nb - 1 : ti);
        const int blk = a.tables[(long long)b * a.max_nb + ti];
        x.blk = blk < 0 ? 0 : (blk >= a.num_blocks ? a.num_blocks - 1 : blk);
    }
    return x;
}

// One workgroup = NG groups of Hkv waves (NG = WPG / Hkv, WPG = kSplitWaves); wave g * Hkv + k serves
// kv-head k for group g. The Hkv waves of a group walk the same tiles, so both halves of every interleaved pool row ([bs][Hkv][D]) are
// fetched together. Within each sequence segment of the workgroup's range, group g takes the segment's tiles
// g, g + NG, g + 2 NG, ...; at the segment's end the groups' (m, l, acc) states are combined through LDS and one
// partial per kv-head is written.
template <typename T, int D, int GP, bool ALIGNED, int WPG>
__global__ __launch_bounds__(64 * WPG) void paged_decode_split(DecodeArgs a) {
    using LD = KVLoad<T>;
    constexpr int NIT = D / 32;              // MFMA k-steps per tile
    constexpr int NT = (3 * GP + 15) / 16;   // A tiles: 3 query splits x GP heads, 16 rows each
    constexpr int LPT = D / 8;               // lanes per position row in the V layout
    constexpr int TPI = 64 / LPT;            // positions per V step
    constexpr int NVI = kTile / TPI;         // V steps per tile
    constexpr int KS = LD::KS;
    constexpr int HB = GP / 4;               // head blocks of 4 in the score layout
    constexpr int QV = (GP * D / 4 + 63) / 64;   // float4 query pieces per lane when a sequence starts
    // register sets for keys (KB = NIT k-steps) and values (VB = NVI steps): a whole tile, the next one in flight
    constexpr int KB = NIT, VB = NVI;
    constexpr int REC = GP * D + 2 * GP;     // floats of one (acc, m, l) record
    static_assert(REC * 4 <= NT * NIT * 64 * 16, "a combine record must fit in the wave's query operand area");

    extern __shared__ __attribute__((aligned(16))) char smem[];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int kvh = wave % a.Hkv;
    const int g = wave / a.Hkv;
    const int NG = a.NG;
    const int w = blockIdx.x;
    const int row = lane & 15;     // MFMA row / column owned by this lane
    const int grp = lane >> 4;     // k-slot group (operands) / row block (accumulator)

    int* P = reinterpret_cast<int*>(smem);          // tile prefix sums [B + 1]
    int* Ls = P + a.B + 1;                           // clamped lengths [B]
    int* V = Ls + a.B;                               // cost prefix sums [B + 1]
    char* wl = smem + seq_lds_bytes(a.B) + wave * wave_lds_bytes<D, GP>();
    u32x4* qop = reinterpret_cast<u32x4*>(wl);
    float* p_lds = reinterpret_cast<float*>(wl + NT * NIT * 64 * 16);
    float* alpha_lds = p_lds + kTile * GP;
    // record of wave ww for the segment combine: the start of its query operand area (re-staged after a combine)
    auto crec = [&](int ww) {
        return reinterpret_cast<float*>(smem + seq_lds_bytes(a.B) + ww * wave_lds_bytes<D, GP>());
    };

    // query operand rows that no (split, head) pair fills are zero (again after every combine)
    auto zero_q = [&]() {
#pragma unroll
        for (int i = 0; i < NT * NIT; ++i) qop[i * 64 + lane] = u32x4{0u, 0u, 0u, 0u};
    };
    typename LD::Vec kv[KB], vv[VB];
    // The next tile's values (bf16 pools; half of them for fp32 pools) are requested into vn right after its keys,
    // before this tile's softmax, instead of one step at a time as this tile's values are used: more bytes in
    // flight per wave through the scores and the softmax (config 3: 86.8 -> 86.5 us; all of an fp32 tile's values
    // that early made config 1 slower, 11.1 -> 11.4 us; with the unaligned tables' per-step row offsets the
    // instance keeps the later requests)
    constexpr int VE = !ALIGNED ? 0 : (sizeof(T) == 2 ? VB : VB / 2);
    typename LD::Vec vn[VE > 0 ? VE : 1];
    TileRows<NVI, TPI, LPT, ALIGNED> cur;
    // issue order K then V, here and in the loop, so that waiting for a tile's keys never waits for its values
    // (the scheduling barriers keep the compiler from reordering the two groups of loads); `mid` issues loads
    // between the two (the first sequence's queries: staging them then waits for the keys, not the values)
    auto issue_first = [&](auto mid) {
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int it = 0; it < KB; ++it) kv[it] = LD::load(a.kp, cur.krow + 32 * it + 8 * grp);
        __builtin_amdgcn_sched_barrier(0);
        mid();
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int vi = 0; vi < VB; ++vi) vv[vi] = LD::load(a.vp, cur.vrow(vi));
        __builtin_amdgcn_sched_barrier(0);
    };
    // per-lane description of this group's tile list entry j0 + lane: sequence, first position, clamped length,
    // first visible position and (ALIGNED) physical block
    int b_l = 0, tpos_l = 0, L_l = 0, s0_l = 0, blk_l = 0;
    auto rows_of = [&](int jj) {
        const int b = __builtin_amdgcn_readlane(b_l, jj);
        const int blk = ALIGNED ? __builtin_amdgcn_readlane(blk_l, jj) : 0;
        return tile_rows<NVI, TPI, LPT, ALIGNED>(a, a.tables + (long long)b * a.max_nb,
                                                  __builtin_amdgcn_readlane(s0_l, jj),
                                                  __builtin_amdgcn_readlane(L_l, jj),
                                                  __builtin_amdgcn_readlane(tpos_l, jj), blk, kvh, D, lane);
    };
    // Query operands. Row m = s * GP + h of the A tiles holds split s of head h, scaled by log2(e)/sqrt(D); element
    // (it, grp, e) of a row is dim 32 it + 8 grp + e. The queries of the next sequence this wave has tiles in are
    // fetched into registers (coalesced: 4 consecutive dims per lane and step) a whole segment ahead, so a sequence
    // switch waits on no load (the first sequence's before the first tile's K / V, so that staging them waits for
    // no K / V load); there the pieces are split and scattered into the operand layout.
    float4 qn[QV];
    // (branch-free: every lane loads, from a clamped index, and stage_q skips the pieces past the group's heads; a
    // conditional load would put branches between the loads and make the compiler's load counts inexact)
    auto fetch_q = [&](int b) {
        const float* qb = a.q + ((long long)b * a.Hq + (long long)kvh * a.G) * D;
        const int n4 = a.G * (D / 4);
#pragma unroll
        for (int k = 0; k < QV; ++k) {
            const int e4 = lane + 64 * k;
            qn[k] = *reinterpret_cast<const float4*>(qb + 4 * (e4 < n4 ? e4 : n4 - 1));
        }
    };
    bool planned = false;
    int lo, hi, bA, bZ;
    if (a.plan) {
        // With a plan, the group's first 64 tile list entries (one 16-byte load per lane) and the workgroup's range
        // are all the first tile needs: its K / V loads are issued before the per-sequence arrays are staged and
        // before the workgroup's barrier, with no block-table load in between. The per-sequence arrays are requested
        // first, so that staging them waits for them alone (loads complete in issue order). The first loads are
        // issued unconditionally (a group without tiles reads position 0 of its first table row, unused): a branch
        // around them would make every later wait a wait for all loads in flight. Entries are clamped into the
        // batch and the pool, so a plan for other lengths gives wrong numbers but never an access outside them.
        constexpr int kSeqPer = (plan_seq_ints(kMaxBatch) + 64 * WPG - 1) / (64 * WPG);
        const int n_seq = plan_seq_ints(a.B);
        const int32_t* pseq = a.plan + kPlanHdr;
        const int4 ev = reinterpret_cast<const int4*>(pseq + n_seq + 4 * a.NW)[(w * NG + g) * 64 + lane];
        const int wv = pseq[n_seq + 4 * w + (lane & 3)];
        int seqv[kSeqPer];
#pragma unroll
        for (int k = 0; k < kSeqPer; ++k) {
            const int i = threadIdx.x + 64 * WPG * k;
            seqv[k] = pseq[i < n_seq ? i : n_seq - 1];
        }
        const bool has = __builtin_amdgcn_readfirstlane(ev.x) >= 0;
        const int cap = a.max_nb * a.bs;
        b_l = has ? (ev.x >= a.B ? a.B - 1 : ev.x) : 0;
        L_l = has ? (ev.z < 1 ? 1 : (ev.z > cap ? cap : ev.z)) : 1;
        s0_l = (a.window > 0 && L_l > a.window) ? L_l - a.window : 0;
        tpos_l = has ? (ev.y < 0 ? 0 : (ev.y >= cap ? (cap - 1) / kTile * kTile : ev.y)) : 0;
        blk_l = has ? (ev.w < 0 ? 0 : (ev.w >= a.num_blocks ? a.num_blocks - 1 : ev.w)) : 0;
        cur = rows_of(0);
        // the group's first tile's sequence's queries (unused without tiles), between its keys and values
        issue_first([&]() { fetch_q(__builtin_amdgcn_readlane(b_l, 0)); });
        planned = has;
#pragma unroll
        for (int k = 0; k < kSeqPer; ++k) {
            const int i = threadIdx.x + 64 * WPG * k;
            if (i < n_seq) P[i] = seqv[k];           // P, Ls, V
        }
        lo = __builtin_amdgcn_readlane(wv, 0);
        hi = __builtin_amdgcn_readlane(wv, 1);
        bA = __builtin_amdgcn_readlane(wv, 2);
        bZ = __builtin_amdgcn_readlane(wv, 3);
        zero_q();
        __syncthreads();
        if (lo >= hi) return;                        // uniform over the workgroup: no barrier is left waiting
        bA = bA < 0 ? 0 : (bA >= a.B ? a.B - 1 : bA);
        bZ = bZ < bA ? bA : (bZ >= a.B ? a.B - 1 : bZ);
    } else {
        if (wave == 0) plan_prefix(a, P, Ls, V);
        zero_q();
        __syncthreads();
        const int U = P[a.B], Uc = V[a.B];
        const bool by_cost = U >= kSegMinTiles * a.NW;   // uniform: U and NW are the same in every workgroup
        lo = by_cost ? tile_at(P, V, a.B, range_lo(Uc, a.NW, w)) : range_lo(U, a.NW, w);
        hi = by_cost ? tile_at(P, V, a.B, range_lo(Uc, a.NW, w + 1)) : range_lo(U, a.NW, w + 1);
        if (lo >= hi) return;                        // uniform over the workgroup: no barrier is left waiting
        bA = seq_of_tile(P, a.B, lo);
        bZ = seq_of_tile(P, a.B, hi - 1);
    }
    const GroupRange rg{P, Ls, lo, hi, bA, bZ, g, NG};
    auto seg_lo = [&](int b) { return rg.seg_lo(b); };
    auto seg_hi = [&](int b) { return rg.seg_hi(b); };
    auto my_count = [&](int b) { return rg.count(b); };
    const int my_total = rg.total();

    auto set_entry = [&](const TileEntry& x) {
        b_l = x.b;
        tpos_l = x.tpos;
        L_l = x.L;
        s0_l = x.s0;
        blk_l = x.blk;
    };
    auto refill = [&](int j0) { set_entry(tile_entry<ALIGNED>(a, rg, j0 + lane, my_total)); };

    float m_run[4], l_run[4];
    float acc[GP][8];
    auto reset = [&]() {
#pragma unroll
        for (int i = 0; i < 4; ++i) { m_run[i] = -INFINITY; l_run[i] = 0.0f; }
#pragma unroll
        for (int h = 0; h < GP; ++h)
#pragma unroll
            for (int e = 0; e < 8; ++e) acc[h][e] = 0.0f;
    };

    auto stage_q = [&]() {
#pragma unroll
        for (int k = 0; k < QV; ++k) {
            const int e4 = lane + 64 * k;
            if (e4 < a.G * (D / 4)) {
                const int h = (4 * e4) / D, d = (4 * e4) % D;
                const Split3 s0 = split3(qn[k].x * a.qscale), s1 = split3(qn[k].y * a.qscale);
                const Split3 s2 = split3(qn[k].z * a.qscale), s3 = split3(qn[k].w * a.qscale);
                const uint32_t pc[3][2] = {{pack_hi2(s0.hi, s1.hi), pack_hi2(s2.hi, s3.hi)},
                                           {pack_hi2(s0.mid, s1.mid), pack_hi2(s2.mid, s3.mid)},
                                           {pack_hi2(s0.lo, s1.lo), pack_hi2(s2.lo, s3.lo)}};
#pragma unroll
                for (int s = 0; s < 3; ++s) {
                    const int m = s * GP + h;
                    const int idx = ((m / 16) * NIT + d / 32) * 64 + (m % 16) + 16 * ((d % 32) / 8);
                    u32x2* dst = reinterpret_cast<u32x2*>(reinterpret_cast<char*>(qop + idx) + 8 * ((d % 8) / 4));
                    *dst = u32x2{pc[s][0], pc[s][1]};
                }
            }
        }
        wave_lds_sync();
    };
    // the next sequence after b (exclusive) in which this wave has tiles, or -1
    auto next_mine = [&](int b) {
        for (int bb = b + 1; bb <= bZ; ++bb)
            if (my_count(bb) > 0) return bb;
        return -1;
    };

    // A segment's result per wave is a record (acc [GP][D], m [GP], l [GP]) in LDS. write_record reduces this
    // wave's state across its lanes into `rec`; combine_slice merges slice g of kv-head kvh's GP x D outputs over
    // the NG groups' records of one segment (a group with no tile in the segment holds m = -inf, l = 0, acc = 0)
    // into the partial `dst` = slot w + b of the workspace, same layout; group 0 also writes m and l.
    auto write_record = [&](float* rec) {
#pragma unroll
        for (int h = 0; h < GP; ++h)
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                float x = acc[h][e];
                if (TPI >= 8) x += dpp_f32<0x128>(x);   // lanes l and l ^ 8 share dims when a row is 8 lanes
                if (TPI >= 4) x += __shfl_xor(x, 16);
                x += __shfl_xor(x, 32);
                acc[h][e] = x;
            }
        if (lane < LPT) {
#pragma unroll
            for (int h = 0; h < GP; ++h) {
                float4* d4 = reinterpret_cast<float4*>(rec + h * D + lane * 8);
                d4[0] = make_float4(acc[h][0], acc[h][1], acc[h][2], acc[h][3]);
                d4[1] = make_float4(acc[h][4], acc[h][5], acc[h][6], acc[h][7]);
            }
        }
        float lsum[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) lsum[i] = row16_sum(l_run[i]);
        if (grp < HB && row == 0) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                rec[GP * D + 4 * grp + i] = m_run[i];
                rec[GP * D + GP + 4 * grp + i] = lsum[i];
            }
        }
    };
    auto combine_slice = [&](auto rec_of, float* dst) {
        const int SL = GP * D / NG;                  // outputs of this wave's slice (a multiple of 4)
        for (int e = g * SL + 4 * lane; e < (g + 1) * SL; e += 256) {
            const int h = e / D;
            float mx = -INFINITY;
            for (int gg = 0; gg < NG; ++gg) mx = fmaxf(mx, rec_of(gg * a.Hkv + kvh)[GP * D + h]);
            float4 num = make_float4(0.f, 0.f, 0.f, 0.f);
            for (int gg = 0; gg < NG; ++gg) {
                const float* r = rec_of(gg * a.Hkv + kvh);
                const float sc = fast_exp2(r[GP * D + h] - mx);
                const float4 x = *reinterpret_cast<const float4*>(r + e);
                num.x = fmaf(sc, x.x, num.x);
                num.y = fmaf(sc, x.y, num.y);
                num.z = fmaf(sc, x.z, num.z);
                num.w = fmaf(sc, x.w, num.w);
            }
            *reinterpret_cast<float4*>(dst + e) = num;
        }
        if (g == 0 && lane < GP) {
            float mx = -INFINITY, den = 0.0f;
            for (int gg = 0; gg < NG; ++gg) mx = fmaxf(mx, rec_of(gg * a.Hkv + kvh)[GP * D + lane]);
            for (int gg = 0; gg < NG; ++gg) {
                const float* r = rec_of(gg * a.Hkv + kvh);
                den = fmaf(fast_exp2(r[GP * D + lane] - mx), r[GP * D + GP + lane], den);
            }
            dst[GP * D + lane] = mx;
            dst[GP * D + GP + lane] = den;
        }
    };

    // Segments that end inside the range: each wave stashes its record in LDS and goes straight on to its next
    // tile, with no barrier (the groups' tile counts in a segment differ by one, so a combine barrier there would
    // idle some groups for a tile); the stashed segments are combined with the last one when the range is done.
    // Up to kStash segments are stashed; any further one is combined at its end.
    auto stash_rec = [&](int s, int ww) {
        return reinterpret_cast<float*>(smem + seq_lds_bytes(a.B) + NG * a.Hkv * wave_lds_bytes<D, GP>()) +
               (s * NG * a.Hkv + ww) * REC;
    };
    int stashed_b[kStash];
    int n_stashed = 0;
    auto part_of = [&](int b) { return a.part + ((long long)(w + b) * a.Hkv + kvh) * REC; };

    reset();
    int j0 = 0;                                      // first entry held by the lane arrays
    if (my_total > 0 && !planned) {                  // with a plan, entries 0 .. 63 and the first loads are in place
        fetch_q(next_mine(bA - 1));
        refill(0);
        cur = rows_of(0);
        issue_first([]() {});
    }
    int j = 0;                                       // this group's next tile list entry
    for (int b = bA; b <= bZ; ++b) {
        if (seg_hi(b) == seg_lo(b)) continue;        // an empty sequence inside the range: no partial
        const int cnt = my_count(b);
        if (cnt > 0) {
            stage_q();
            const int bn = next_mine(b);
            if (bn >= 0) fetch_q(bn);
        }
        for (int k = 0; k < cnt; ++k, ++j) {
            // the next entry's rows: from the lane arrays, refilled when the next entry starts a new 64-entry chunk
            // (the refill's table load makes that one prefetch wait). The last entry's prefetch is never used: it
            // is aimed at position 0 of the pool's first block (one 512-byte row per kv-head that the last
            // prefetch of every wave shares, so it stays cached), not at this tile again, whose bf16 rows were
            // streamed past the caches and would be fetched a second time (32 MB per call at config 3)
            const TileRows<NVI, TPI, LPT, ALIGNED> cur_now = cur;
            TileRows<NVI, TPI, LPT, ALIGNED> nxt;
            if (j + 1 >= my_total) {
                nxt = cur_now;
                nxt.krow = (long long)kvh * D;
                if constexpr (ALIGNED) {
                    nxt.vbase = (long long)kvh * D + (lane % LPT) * 8;
                    nxt.vstride = 0;
                } else {
#pragma unroll
                    for (int vi = 0; vi < NVI; ++vi) nxt.vr[vi] = (long long)kvh * D + (lane % LPT) * 8;
                }
            } else {
                if (j + 1 - j0 == 64) {
                    j0 += 64;
                    refill(j0);
                }
                nxt = rows_of(j + 1 - j0);
            }

            // ---- scores: S[m][n] = sum_d A[m][d] * K[n][d]. Each key register set is refilled with the next
            // tile's keys as soon as its MFMA operands are built, so the next tile is in flight while this one
            // computes. Issued unconditionally: a conditional issue would make every later wait for this tile's
            // values a wait for all outstanding loads.
            f32x4 sacc[NT];
#pragma unroll
            for (int tt = 0; tt < NT; ++tt) sacc[tt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int it = 0; it < NIT; ++it) {
                u32x4 kb[KS];
                LD::key_operands(kv[it % KB], kb);
                __builtin_amdgcn_sched_barrier(0);
                kv[it % KB] = LD::load(a.kp, it + KB < NIT ? cur_now.krow + 32 * (it + KB) + 8 * grp
                                                          : nxt.krow + 32 * (it + KB - NIT) + 8 * grp);
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int ks = 0; ks < KS; ++ks)
#pragma unroll
                    for (int tt = 0; tt < NT; ++tt)
                        sacc[tt] = mfma16x16x32(qop[(tt * NIT + it) * 64 + lane], kb[ks], sacc[tt]);
            }

            if constexpr (VE > 0) {
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int vi = 0; vi < VE; ++vi) vn[vi] = LD::load(a.vp, nxt.vrow(vi));
                __builtin_amdgcn_sched_barrier(0);
            }
            // sum the three query splits: lane (grp, row) then holds heads 4 * (grp % HB) + i of position row
            float sc[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                float x = sacc[0][i];
#pragma unroll
                for (int tt = 1; tt < NT; ++tt) x += sacc[tt][i];
                if (GP == 4) x += __shfl_xor(x, 16);
                x += __shfl_xor(x, 32);
                sc[i] = cur_now.kvalid ? x : -INFINITY;
            }

            // ---- online softmax (base 2) per head over the 16 positions of this row
            float pr[4], al[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float mt = row16_max(sc[i]);
                const float mn = fmaxf(m_run[i], mt);
                al[i] = fast_exp2(m_run[i] - mn);
                pr[i] = fast_exp2(sc[i] - mn);
                l_run[i] = l_run[i] * al[i] + pr[i];
                m_run[i] = mn;
            }
            if (grp < HB) {
                *reinterpret_cast<float4*>(&p_lds[row * GP + 4 * grp]) = make_float4(pr[0], pr[1], pr[2], pr[3]);
                if (row == 0)
                    *reinterpret_cast<float4*>(&alpha_lds[4 * grp]) = make_float4(al[0], al[1], al[2], al[3]);
            }
            wave_lds_sync();

            // ---- acc = acc * alpha + P V
            float alh[GP];
#pragma unroll
            for (int h4 = 0; h4 < GP / 4; ++h4) {
                const float4 t = *reinterpret_cast<const float4*>(&alpha_lds[4 * h4]);
                alh[4 * h4] = t.x; alh[4 * h4 + 1] = t.y; alh[4 * h4 + 2] = t.z; alh[4 * h4 + 3] = t.w;
            }
#pragma unroll
            for (int h = 0; h < GP; ++h)
#pragma unroll
                for (int e = 0; e < 8; ++e) acc[h][e] *= alh[h];
            // values of hidden positions become 0 (branch-free: a branch here would make the compiler wait for
            // every outstanding load, including the next tile's keys); each value register set is refilled with
            // the next tile's values as soon as it is widened
#pragma unroll
            for (int vi = 0; vi < NVI; ++vi) {
                float vf[8];
                LD::keep_if(vv[vi % VB], cur_now.vvalid(vi));
                LD::widen(vv[vi % VB], vf);
                if (vi >= VE) {
                    __builtin_amdgcn_sched_barrier(0);
                    vv[vi % VB] = LD::load(a.vp, vi + VB < NVI ? cur_now.vrow(vi + VB) : nxt.vrow(vi + VB - NVI));
                    __builtin_amdgcn_sched_barrier(0);
                }
                const int pos = vi * TPI + lane / LPT;
                float ph[GP];
#pragma unroll
                for (int h4 = 0; h4 < GP / 4; ++h4) {
                    const float4 t = *reinterpret_cast<const float4*>(&p_lds[pos * GP + 4 * h4]);
                    ph[4 * h4] = t.x; ph[4 * h4 + 1] = t.y; ph[4 * h4 + 2] = t.z; ph[4 * h4 + 3] = t.w;
                }
#pragma unroll
                for (int h = 0; h < GP; ++h)
#pragma unroll
                    for (int e = 0; e < 8; ++e) acc[h][e] = fmaf(ph[h], vf[e], acc[h][e]);
            }
            if constexpr (VE > 0) {
#pragma unroll
                for (int vi = 0; vi < VE; ++vi) vv[vi] = vn[vi];
            }
            cur = nxt;
            wave_lds_sync();   // p_lds / alpha_lds are rewritten by the next tile
        }
        if (b < bZ && n_stashed < kStash) {           // uniform over the workgroup
            write_record(stash_rec(n_stashed, wave));
            stashed_b[n_stashed++] = b;
        } else {
            // the records of this segment go in the query operand areas (re-staged at the next segment start)
            write_record(reinterpret_cast<float*>(wl));
            lds_barrier();
            for (int s = 0; s < n_stashed; ++s)
                combine_slice([&](int ww) { return stash_rec(s, ww); }, part_of(stashed_b[s]));
            n_stashed = 0;
            combine_slice([&](int ww) { return crec(ww); }, part_of(b));
            if (b < bZ) {                             // more segments follow: the areas hold query operands again
                lds_barrier();
                zero_q();
            }
        }
        reset();
    }
}

// One workgroup per (sequence, kv-head). Sequence b owns global tiles [P[b], P[b + 1]), cost units V[b] + kSegCost ..
// V[b + 1] - 1; the split workgroups whose ranges meet it are w_first = the one holding the unit (cost unit or tile,
// as the split kernel cut the ranges) of tile P[b] .. w_last = the one holding its last unit (empty ranges in between,
// possible only when NW exceeds the units, are skipped), with partials in slots w + b. The workgroup's threads form SL
// slices of TS threads (TS = GP * D / 4, one float4 output of the GP x D block each); with n partials, the first
// min(SL, ceil(n / kMergeCh)) slices take consecutive runs of them, so a sequence over many partials (few
// sequences, many split workgroups) needs up to SL times fewer memory round trips. Within a slice the partials are combined in workgroup order, up to kMergeCh per
// round trip (every load of a chunk is issued before any is used, with no branch between them), with a running
// maximum: M' = max(M, m_w), num = num 2^(M - M') + sum_w 2^(m_w - M') acc_w, den likewise with l_w; the slices'
// (M, num, den) are then combined in slice order the same way, and out = num / den, times the gate.
constexpr int kMergeThreads = 1024;

template <int D, int GP>
__global__ __launch_bounds__(kMergeThreads) void paged_decode_merge(DecodeArgs a) {
    constexpr int TS = GP * D / 4;                    // threads per slice: one float4 output each
    constexpr int SL = kMergeThreads / TS;            // slices
    static_assert(TS <= kMergeThreads && kMergeThreads % TS == 0, "slices tile the workgroup");
    constexpr int REC = GP * D + 2 * GP;
    constexpr int kMergeCh = 8;                       // partials combined per memory round trip
    __shared__ int P[kMaxBatch + 1], V[kMaxBatch + 1];
    __shared__ float4 num_s[SL > 1 ? SL - 1 : 1][TS];
    __shared__ float2 md_s[SL > 1 ? SL - 1 : 1][TS];  // (M, den)
    const int tid = threadIdx.x, sl = tid / TS, ti = tid % TS;
    const int b = blockIdx.x / a.Hkv, kvh = blockIdx.x % a.Hkv;
    const int n4 = a.G * (D / 4);
    const long long obase = ((long long)b * a.Hq + (long long)kvh * a.G) * D;
    const float* grow = a.gate ? a.gate + (long long)b * a.gate_ld + (long long)kvh * a.G * D : nullptr;
    const float4 gv = sl == 0 && grow && ti < n4 ? *reinterpret_cast<const float4*>(grow + 4 * ti)
                                                 : make_float4(0.f, 0.f, 0.f, 0.f);
    if (a.plan) {
        const int32_t* pseq = a.plan + kPlanHdr;
        for (int i = tid; i <= a.B; i += kMergeThreads) {
            P[i] = pseq[i];
            V[i] = pseq[2 * a.B + 1 + i];
        }
    } else if (tid < 64) {
        plan_prefix(a, P, nullptr, V);
    }
    __syncthreads();
    const int U = P[a.B], pb = P[b], pe = P[b + 1];
    float4* out = reinterpret_cast<float4*>(a.out + obase);
    if (pe == pb) {                                  // empty sequence (length 0)
        if (sl == 0 && ti < n4) out[ti] = make_float4(0.f, 0.f, 0.f, 0.f);
        return;
    }
    // the split workgroups' units (cost units or tiles, as the split kernel cut them), the first and last units of b
    const bool by_cost = U >= kSegMinTiles * a.NW;
    const int Uu = by_cost ? V[a.B] : U, u0 = by_cost ? V[b] + kSegCost : pb, u1 = by_cost ? V[b + 1] : pe;
    if (Uu <= 0) {                                   // only from a plan for other lengths: nothing to merge
        if (sl == 0 && ti < n4) out[ti] = make_float4(0.f, 0.f, 0.f, 0.f);
        return;
    }
    // (clamped to the split grid: a plan for other lengths must not send the loads below past the workspace)
    const int wf = max(0, min(a.NW - 1, (int)(((long long)(u0 + 1) * a.NW - 1) / Uu)));
    const int wlast = max(wf, min(a.NW - 1, (int)(((long long)u1 * a.NW - 1) / Uu)));
    // slices in use: one per chunk of partials, up to SL (the rest hold none); partials per slice
    const int npart = wlast - wf + 1;
    const int slr = min(SL, (npart + kMergeCh - 1) / kMergeCh);
    const int per = (npart + slr - 1) / slr;
    const int s_first = sl < slr ? wf + sl * per : wlast + 1, s_last = min(wlast, s_first + per - 1);

    const int ic = ti < n4 ? ti : 0;
    const int off = 4 * ic, hk = (4 * ic) / D;        // this thread's float4 output: element offset, head
    float M = -INFINITY, den = 0.0f;
    float4 num = make_float4(0.f, 0.f, 0.f, 0.f);
    // a workgroup's range in [wf, wlast] can be empty only when there are more split workgroups than units;
    // otherwise every one of them holds a partial, and no range has to be recomputed per partial
    const bool sparse = a.NW > Uu;
    for (int w0 = s_first; w0 <= s_last; w0 += kMergeCh) {
        float4 v[kMergeCh];
        float mj[kMergeCh], lj[kMergeCh];
        bool use[kMergeCh];
        // every load of the chunk first, without branches: slots past the slice's last re-read it (unused)
#pragma unroll
        for (int j = 0; j < kMergeCh; ++j) {
            const int wj = min(w0 + j, s_last);
            const float* base = a.part + ((long long)(wj + b) * a.Hkv + kvh) * REC;
            v[j] = *reinterpret_cast<const float4*>(base + off);
            mj[j] = base[GP * D + hk];
            lj[j] = base[GP * D + GP + hk];
        }
#pragma unroll
        for (int j = 0; j < kMergeCh; ++j) {
            const int wj = w0 + j;
            use[j] = wj <= s_last && (!sparse || range_lo(Uu, a.NW, wj + 1) > range_lo(Uu, a.NW, wj));
        }
        float mx = M;
#pragma unroll
        for (int j = 0; j < kMergeCh; ++j) mx = use[j] ? fmaxf(mx, mj[j]) : mx;
        // 0 before the first partial (M = -inf): num and den are 0 then, also in a chunk with none to use
        const float rs = M == -INFINITY ? 0.0f : fast_exp2(M - mx);
        float4 nk = make_float4(num.x * rs, num.y * rs, num.z * rs, num.w * rs);
        float dk = den * rs;
        // a slot not in use is selected away, not multiplied by 0: an empty range never wrote its slot, so the
        // bytes there are whatever the workspace held before (possibly Inf / NaN)
#pragma unroll
        for (int j = 0; j < kMergeCh; ++j) {
            const float sc = fast_exp2(mj[j] - mx);
            nk.x = use[j] ? fmaf(sc, v[j].x, nk.x) : nk.x;
            nk.y = use[j] ? fmaf(sc, v[j].y, nk.y) : nk.y;
            nk.z = use[j] ? fmaf(sc, v[j].z, nk.z) : nk.z;
            nk.w = use[j] ? fmaf(sc, v[j].w, nk.w) : nk.w;
            dk = use[j] ? fmaf(sc, lj[j], dk) : dk;
        }
        num = nk;
        den = dk;
        M = mx;
    }
    if constexpr (SL > 1) {
        if (sl > 0) {
            num_s[sl - 1][ti] = num;
            md_s[sl - 1][ti] = make_float2(M, den);
        }
        __syncthreads();
        if (sl > 0) return;
        // slice 0 holds the first partials, so M is finite; a slice without partials has M = -inf and adds 0
        float mx = M;
#pragma unroll
        for (int q = 0; q < SL - 1; ++q) mx = fmaxf(mx, md_s[q][ti].x);
        const float rs = fast_exp2(M - mx);
        num = make_float4(num.x * rs, num.y * rs, num.z * rs, num.w * rs);
        den *= rs;
#pragma unroll
        for (int q = 0; q < SL - 1; ++q) {
            const float2 md = md_s[q][ti];
            const float4 nq = num_s[q][ti];
            const float sc = fast_exp2(md.x - mx);
            num.x = fmaf(sc, nq.x, num.x);
            num.y = fmaf(sc, nq.y, num.y);
            num.z = fmaf(sc, nq.z, num.z);
            num.w = fmaf(sc, nq.w, num.w);
            den = fmaf(sc, md.y, den);
        }
    }
    if (ti >= n4) return;
    float4 o = make_float4(num.x / den, num.y / den, num.z / den, num.w / den);
    if (a.gate) {
        o.x *= 1.0f / (1.0f + expf(-gv.x));
        o.y *= 1.0f / (1.0f + expf(-gv.y));
        o.z *= 1.0f / (1.0f + expf(-gv.z));
        o.w *= 1.0f / (1.0f + expf(-gv.w));
    }
    out[ti] = o;
}

// The batch layout plan: split workgroup w's range and each group's first 64 tile list entries, computed by the same
// functions as the split kernel (one workgroup of NG waves per split workgroup; workgroup 0 also writes the
// per-sequence arrays and the header). Written once per decode step and read by every attention layer's split and
// merge launches of that step.
template <bool ALIGNED>
__global__ __launch_bounds__(512) void paged_decode_plan(DecodeArgs a, int32_t* plan) {
    extern __shared__ __attribute__((aligned(16))) char smem[];
    int* P = reinterpret_cast<int*>(smem);
    int* Ls = P + a.B + 1;
    int* V = Ls + a.B;
    const int lane = threadIdx.x & 63, g = threadIdx.x >> 6, w = blockIdx.x;
    if (g == 0) plan_prefix(a, P, Ls, V);
    __syncthreads();
    const int U = P[a.B], Uc = V[a.B];
    const bool by_cost = U >= kSegMinTiles * a.NW;
    const int lo = by_cost ? tile_at(P, V, a.B, range_lo(Uc, a.NW, w)) : range_lo(U, a.NW, w);
    const int hi = by_cost ? tile_at(P, V, a.B, range_lo(Uc, a.NW, w + 1)) : range_lo(U, a.NW, w + 1);
    const int bA = lo < hi ? seq_of_tile(P, a.B, lo) : 0, bZ = lo < hi ? seq_of_tile(P, a.B, hi - 1) : 0;
    int32_t* pseq = plan + kPlanHdr;
    if (w == 0) {
        for (int i = threadIdx.x; i < plan_seq_ints(a.B); i += blockDim.x) pseq[i] = i < 3 * a.B + 2 ? P[i] : 0;
        if (threadIdx.x < kPlanHdr) {
            const int hdr[kPlanHdr] = {U, Uc, a.NW, a.NG, a.B, by_cost ? 1 : 0, a.max_nb, a.bs};
            int v = 0;
#pragma unroll
            for (int i = 0; i < kPlanHdr; ++i) v = (int)threadIdx.x == i ? hdr[i] : v;
            plan[threadIdx.x] = v;
        }
    }
    if (threadIdx.x < 4) {
        const int wr[4] = {lo, hi, bA, bZ};
        int v = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) v = (int)threadIdx.x == i ? wr[i] : v;
        pseq[plan_seq_ints(a.B) + 4 * w + threadIdx.x] = v;
    }
    int4 e = make_int4(-1, 0, 0, 0);                 // b = -1: the group has no tile in the range
    if (lo < hi) {
        const GroupRange rg{P, Ls, lo, hi, bA, bZ, g, a.NG};
        const int total = rg.total();
        if (total > 0) {
            const TileEntry x = tile_entry<ALIGNED>(a, rg, lane, total);
            e = make_int4(x.b, x.tpos, x.L, x.blk);
        }
    }
    reinterpret_cast<int4*>(pseq + plan_seq_ints(a.B) + 4 * a.NW)[(w * a.NG + g) * 64 + lane] = e;
}

typedef void (*SplitFn)(DecodeArgs);
typedef void (*MergeFn)(DecodeArgs);

template <typename T, bool ALIGNED>
SplitFn pick_split(int D, int GP) {
    constexpr int W = kSplitWaves;
    if (GP == 4) {
        if (D == 64) return paged_decode_split<T, 64, 4, ALIGNED, W>;
        if (D == 128) return paged_decode_split<T, 128, 4, ALIGNED, W>;
        if (D == 256) return paged_decode_split<T, 256, 4, ALIGNED, W>;
    } else {
        if (D == 64) return paged_decode_split<T, 64, 8, ALIGNED, W>;
        if (D == 128) return paged_decode_split<T, 128, 8, ALIGNED, W>;
        if (D == 256) return paged_decode_split<T, 256, 8, ALIGNED, W>;
    }
    return nullptr;
}

SplitFn pick_split(int kv_dtype, bool aligned, int D, int GP) {
    if (kv_dtype == RK_BF16) return aligned ? pick_split<uint16_t, true>(D, GP) : pick_split<uint16_t, false>(D, GP);
    return aligned ? pick_split<float, true>(D, GP) : pick_split<float, false>(D, GP);
}

int groups_of(int Hkv) { return kSplitWaves / Hkv > 0 ? kSplitWaves / Hkv : 1; }

int split_lds_bytes(int B, int Hkv, int D, int GP, int NG) {
    int per_wave = 0;
    if (GP == 4) per_wave = D == 64 ? wave_lds_bytes<64, 4>() : D == 128 ? wave_lds_bytes<128, 4>() : wave_lds_bytes<256, 4>();
    else per_wave = D == 64 ? wave_lds_bytes<64, 8>() : D == 128 ? wave_lds_bytes<128, 8>() : wave_lds_bytes<256, 8>();
    return seq_lds_bytes(B) + NG * Hkv * per_wave + kStash * NG * Hkv * (GP * D + 2 * GP) * 4;
}

MergeFn pick_merge(int D, int GP) {
    if (GP == 4) {
        if (D == 64) return paged_decode_merge<64, 4>;
        if (D == 128) return paged_decode_merge<128, 4>;
        if (D == 256) return paged_decode_merge<256, 4>;
    } else {
        if (D == 64) return paged_decode_merge<64, 8>;
        if (D == 128) return paged_decode_merge<128, 8>;
        if (D == 256) return paged_decode_merge<256, 8>;
    }
    return nullptr;
}

// Workgroups of the split phase (NG groups of Hkv waves): enough for about one tile per group at the tile count's
// upper bound, capped at one workgroup per compute unit (one wave per SIMD), all resident at once.
int split_groups(int B, int Hkv, int block_size, int max_nb) {
    const long long upper = tile_upper(B, block_size, max_nb);
    int cus = device_cus();
    if (cus <= 0) cus = 256;
    const int ng = groups_of(Hkv);
    const long long cap = (long long)cus * kSplitWaves / (ng * Hkv);
    const long long want = (upper + ng - 1) / ng;
    long long nw = want < cap ? want : cap;
    return (int)(nw < 1 ? 1 : nw);
}

// Partial slots w + b: w < NW and b < B, so NW + B - 1 slots are ever written.
size_t workspace_bytes(int B, int Hkv, int D, int GP, int NW) {
    return (size_t)(NW + (size_t)B) * Hkv * GP * (D + 2) * sizeof(float);
}

int validate(const float* out, const float* q, const void* kp, const void* vp, int kv_dtype, const int32_t* tables,
             const int32_t* lens, int B, int Hq, int Hkv, int D, int bs, int max_nb, int num_blocks, int window) {
    if (!out || !q || !kp || !vp || !tables || !lens) return fail(RK_ERR_ARG, "rk_paged_decode: null pointer");
    if (B < 1 || B > kMaxBatch) return fail(RK_ERR_ARG, "rk_paged_decode: batch %d outside [1, %d]", B, kMaxBatch);
    if (Hkv < 1 || Hq < Hkv || Hq % Hkv) return fail(RK_ERR_ARG, "rk_paged_decode: %d query heads over %d kv heads", Hq, Hkv);
    if (Hq / Hkv > 8) return fail(RK_ERR_UNSUPPORTED, "rk_paged_decode: group size %d > 8", Hq / Hkv);
    if (Hkv > kMaxKvHeads) return fail(RK_ERR_UNSUPPORTED, "rk_paged_decode: %d kv heads > %d", Hkv, kMaxKvHeads);
    if (D != 64 && D != 128 && D != 256) return fail(RK_ERR_UNSUPPORTED, "rk_paged_decode: head_dim %d not in {64,128,256}", D);
    if (bs < 1 || max_nb < 1 || num_blocks < 1) return fail(RK_ERR_ARG, "rk_paged_decode: block_size %d, max_nb %d, num_blocks %d", bs, max_nb, num_blocks);
    if (window < 0) return fail(RK_ERR_ARG, "rk_paged_decode: window %d < 0", window);
    if ((long long)B * (((long long)max_nb * bs + kTile - 1) / kTile) >= (1ll << 31))
        return fail(RK_ERR_ARG, "rk_paged_decode: %d sequences x %d blocks of %d positions exceed 2^31 tiles", B, max_nb, bs);
    if (kv_dtype != RK_F32 && kv_dtype != RK_BF16) return fail(RK_ERR_UNSUPPORTED, "rk_paged_decode: kv dtype %d", kv_dtype);
    return RK_OK;
}

}  // namespace
}  // namespace rk

using namespace rk;

extern "C" {

size_t rk_paged_decode_workspace_bytes(int B, int Hq, int Hkv, int D, int block_size, int max_nb) {
    if (B < 1 || Hkv < 1 || Hq < Hkv || block_size < 1 || max_nb < 1) return 0;
    const int GP = (Hq / Hkv) <= 4 ? 4 : 8;
    return workspace_bytes(B, Hkv, D, GP, split_groups(B, Hkv, block_size, max_nb));
}

size_t rk_paged_decode_plan_ints(int B, int Hq, int Hkv, int D, int block_size, int max_nb) {
    if (B < 1 || Hkv < 1 || Hq < Hkv || block_size < 1 || max_nb < 1) return 0;
    const int GP = (Hq / Hkv) <= 4 ? 4 : 8;
    return plan_ints(B, split_groups(B, Hkv, block_size, max_nb), groups_of(Hkv));
}

int rk_paged_decode_plan(int32_t* plan, size_t plan_ints_, const int32_t* tables, const int32_t* lens, int B, int Hq,
                         int Hkv, int D, int block_size, int max_nb, int num_blocks, int window, void* stream) {
    float dummy = 0.0f;   // validate() checks the pointers the decode itself needs; the plan reads none of these
    int rc = validate(&dummy, &dummy, &dummy, &dummy, RK_BF16, tables, lens, B, Hq, Hkv, D, block_size, max_nb,
                      num_blocks, window);
    if (rc) return rc;
    const size_t need = rk_paged_decode_plan_ints(B, Hq, Hkv, D, block_size, max_nb);
    if (!plan || plan_ints_ < need || reinterpret_cast<uintptr_t>(plan) % 16)
        return fail(RK_ERR_WORKSPACE, "rk_paged_decode_plan: plan of %zu ints (need %zu, 16-byte aligned)", plan_ints_,
                    need);
    const int GP = (Hq / Hkv) <= 4 ? 4 : 8;
    DecodeArgs a{};
    a.tables = tables;
    a.lens = lens;
    a.B = B; a.Hq = Hq; a.Hkv = Hkv; a.G = Hq / Hkv; a.bs = block_size; a.max_nb = max_nb;
    a.num_blocks = num_blocks; a.window = window;
    a.NW = split_groups(B, Hkv, block_size, max_nb);
    a.NG = groups_of(Hkv);
    auto fn = block_size % kTile == 0 ? paged_decode_plan<true> : paged_decode_plan<false>;
    hipLaunchKernelGGL(fn, dim3(a.NW), dim3(64 * a.NG), seq_lds_bytes(B), static_cast<hipStream_t>(stream), a, plan);
    return check_launch("paged_decode_plan");
}

namespace rk {
namespace {

int decode_launch(int phase, float* out, const float* q, const void* k_pool, const void* v_pool, int kv_dtype,
                  const int32_t* tables, const int32_t* lens, int B, int Hq, int Hkv, int D, int block_size,
                  int max_nb, int num_blocks, int window, const float* gate, long long gate_ld, const int32_t* plan,
                  size_t plan_ints_, void* workspace, size_t workspace_bytes_, void* stream) {
    int rc = validate(out, q, k_pool, v_pool, kv_dtype, tables, lens, B, Hq, Hkv, D, block_size, max_nb,
                      num_blocks, window);
    if (rc) return rc;
    if (gate && (gate_ld < (long long)Hq * D || gate_ld % 4 || reinterpret_cast<uintptr_t>(gate) % 16))
        return fail(RK_ERR_ARG, "rk_paged_decode: gate rows of %lld elements (>= %d, a multiple of 4, 16-byte "
                    "aligned)", gate_ld, Hq * D);
    if (phase != 0 && phase != 1) return fail(RK_ERR_ARG, "rk_paged_decode_phase: phase %d", phase);
    if (plan && (plan_ints_ < rk_paged_decode_plan_ints(B, Hq, Hkv, D, block_size, max_nb) ||
                 reinterpret_cast<uintptr_t>(plan) % 16))
        return fail(RK_ERR_WORKSPACE, "rk_paged_decode: plan of %zu ints (need %zu, 16-byte aligned)", plan_ints_,
                    rk_paged_decode_plan_ints(B, Hq, Hkv, D, block_size, max_nb));
    const int G = Hq / Hkv;
    const int GP = G <= 4 ? 4 : 8;
    const int NW = split_groups(B, Hkv, block_size, max_nb);
    const size_t need = workspace_bytes(B, Hkv, D, GP, NW);
    if (!workspace || workspace_bytes_ < need)
        return fail(RK_ERR_WORKSPACE, "rk_paged_decode: workspace %zu bytes < %zu needed", workspace_bytes_, need);

    DecodeArgs a;
    a.plan = plan;
    a.part = static_cast<float*>(workspace);
    a.out = out;
    a.q = q;
    a.kp = k_pool;
    a.vp = v_pool;
    a.tables = tables;
    a.lens = lens;
    a.gate = gate;
    a.gate_ld = gate_ld;
    a.B = B; a.Hq = Hq; a.Hkv = Hkv; a.G = G; a.bs = block_size; a.max_nb = max_nb;
    a.num_blocks = num_blocks; a.window = window; a.NW = NW; a.NG = groups_of(Hkv);
    a.qscale = kLog2e / sqrtf((float)D);
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (phase == 0) {
        SplitFn fn = pick_split(kv_dtype, block_size % kTile == 0, D, GP);
        const int lds = split_lds_bytes(B, Hkv, D, GP, a.NG);
        rc = allow_dynamic_lds(reinterpret_cast<const void*>(fn), lds);
        if (rc) return rc;
        hipLaunchKernelGGL(fn, dim3(NW), dim3(64 * a.NG * Hkv), lds, s, a);
        return check_launch("paged_decode_split");
    }
    hipLaunchKernelGGL(pick_merge(D, GP), dim3(B * Hkv), dim3(kMergeThreads), 0, s, a);
    return check_launch("paged_decode_merge");
}

}  // namespace
}  // namespace rk

int rk_paged_decode_phase(int phase, float* out, const float* q, const void* k_pool, const void* v_pool,
                          int kv_dtype, const int32_t* tables, const int32_t* lens, int B, int Hq, int Hkv, int D,
                          int block_size, int max_nb, int num_blocks, int window, const float* gate,
                          long long gate_ld, const int32_t* plan, size_t plan_ints_, void* workspace,
                          size_t workspace_bytes_, void* stream) {
    return decode_launch(phase, out, q, k_pool, v_pool, kv_dtype, tables, lens, B, Hq, Hkv, D, block_size, max_nb,
                         num_blocks, window, gate, gate_ld, plan, plan_ints_, workspace, workspace_bytes_, stream);
}

int rk_paged_decode_planned(float* out, const float* q, const void* k_pool, const void* v_pool, int kv_dtype,
                            const int32_t* tables, const int32_t* lens, int B, int Hq, int Hkv, int D, int block_size,
                            int max_nb, int num_blocks, int window, const float* gate, long long gate_ld,
                            const int32_t* plan, size_t plan_ints_, void* workspace, size_t workspace_bytes_,
                            void* stream) {
    if (!plan) return fail(RK_ERR_ARG, "rk_paged_decode_planned: null plan");
    int rc = decode_launch(0, out, q, k_pool, v_pool, kv_dtype, tables, lens, B, Hq, Hkv, D, block_size, max_nb,
                           num_blocks, window, gate, gate_ld, plan, plan_ints_, workspace, workspace_bytes_, stream);
    if (rc) return rc;
    return decode_launch(1, out, q, k_pool, v_pool, kv_dtype, tables, lens, B, Hq, Hkv, D, block_size, max_nb,
                         num_blocks, window, gate, gate_ld, plan, plan_ints_, workspace, workspace_bytes_, stream);
}

size_t rk_paged_decode_noalloc_max_bytes(void) { return kScratchBytes; }

int rk_paged_decode_noalloc(float* out, const float* q, const void* k_pool, const void* v_pool, int kv_dtype,
                            const int32_t* tables, const int32_t* lens, int B, int Hq, int Hkv, int D, int block_size,
                            int max_nb, int num_blocks, int window, const float* gate, long long gate_ld,
                            void* stream) {
    static std::mutex mu;
    static void* addr[64] = {};                // per device: the address of `scratch` in that device's memory
    int rc = validate(out, q, k_pool, v_pool, kv_dtype, tables, lens, B, Hq, Hkv, D, block_size, max_nb,
                      num_blocks, window);
    if (rc) return rc;
    const int GP = (Hq / Hkv) <= 4 ? 4 : 8;
    const size_t need = workspace_bytes(B, Hkv, D, GP, split_groups(B, Hkv, block_size, max_nb));
    if (need > kScratchBytes)
        return fail(RK_ERR_WORKSPACE, "rk_paged_decode_noalloc: %zu bytes of partials for batch %d x %d kv-heads x "
                    "head_dim %d exceed its fixed %zu-byte scratch (use rk_paged_decode with a workspace)", need, B,
                    Hkv, D, kScratchBytes);
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return fail(RK_ERR_HIP, "rk_paged_decode_noalloc: hipGetDevice: %s", hipGetErrorString(e));
    if (dev < 0 || dev >= 64) return fail(RK_ERR_UNSUPPORTED, "rk_paged_decode_noalloc: device %d >= 64", dev);
    void* ptr = nullptr;
    {
        std::lock_guard<std::mutex> lock(mu);
        if (!addr[dev]) {
            e = hipGetSymbolAddress(&addr[dev], HIP_SYMBOL(scratch));
            if (e != hipSuccess) {
                addr[dev] = nullptr;
                return fail(RK_ERR_HIP, "rk_paged_decode_noalloc: hipGetSymbolAddress: %s", hipGetErrorString(e));
            }
        }
        ptr = addr[dev];
    }
    return rk_paged_decode(out, q, k_pool, v_pool, kv_dtype, tables, lens, B, Hq, Hkv, D, block_size, max_nb,
                           num_blocks, window, gate, gate_ld, ptr, kScratchBytes, stream);
}

int rk_paged_decode(float* out, const float* q, const void* k_pool, const void* v_pool, int kv_dtype,
                    const int32_t* tables, const int32_t* lens, int B, int Hq, int Hkv, int D, int block_size,
                    int max_nb, int num_blocks, int window, const float* gate, long long gate_ld, void* workspace,
                    size_t workspace_bytes_, void* stream) {
    int rc = decode_launch(0, out, q, k_pool, v_pool, kv_dtype, tables, lens, B, Hq, Hkv, D, block_size, max_nb,
                           num_blocks, window, gate, gate_ld, nullptr, 0, workspace, workspace_bytes_, stream);
    if (rc) return rc;
    return decode_launch(1, out, q, k_pool, v_pool, kv_dtype, tables, lens, B, Hq, Hkv, D, block_size, max_nb,
                         num_blocks, window, gate, gate_ld, nullptr, 0, workspace, workspace_bytes_, stream);
}

}  // extern "C"
