// P1: paged GQA decode attention over a block-table KV pool, gfx950.
//
// Semantics (reference): TorchBackend.paged_attention gathers each sequence's positions through its block table and
// runs ops.attention with one query (src/backend/torch_ref.py:75-88, src/ops.py:65-104); the Metal kernel it
// replaces is paged_attention_decode<T> (src/kernels/attention.metal:87-159). Pool row of position s of sequence i:
// ((tables[i][s / bs] * bs + s % bs) * Hkv + kvh) * D (attention.metal:115).
//
// Design (split over positions, then a merge):
//   * Work unit = one 16-position tile of one sequence. Sequence b gets n(b) = max(1, round(units(b) NW / U))
//     split workgroups (U = all tiles, NW = the target workgroup count) that take equal contiguous parts of its
//     tiles, so every workgroup streams about U / NW tiles however unequal the lengths are, never crosses a
//     sequence, and writes exactly one partial (m, l, acc) per kv-head.
//   * A split workgroup has one wave per kv-head; the waves walk the same tiles, so the interleaved halves of every
//     pool row ([bs][Hkv][D]) are fetched together. Each wave serves all G = Hq/Hkv query heads of its kv-head, so
//     every K/V byte is read from HBM once.
//   * QK^T on MFMA (v_mfma_f32_16x16x32_bf16): A = the G query rows split exactly into three bf16 parts
//     (q = hi + mid + lo, kept in LDS), B = 16 keys x 32 dims. bf16 keys are exact MFMA operands; fp32 keys are split
//     the same way (three MFMA passes), so both pool types get fp32-accurate scores, and a bf16 pool gives bit for
//     bit the result of the fp32 pool holding the widened values (the extra passes only add exact zeros).
//   * Loads are software-pipelined: the next tile's keys are issued after this tile's MFMAs and its values after
//     this tile's PV, so every wave always has a tile's K or V in flight. When tiles align with blocks
//     (block_size % 16 == 0) one vector load fetches the block numbers of 64 tiles.
//   * Online softmax in base 2 (scores pre-scaled by log2(e)/sqrt(D)); row max by DPP inside 16-lane rows.
//   * PV on the VALU in fp32: each lane owns 8 consecutive dims of one position row (coalesced 16/32-byte loads);
//     probabilities are broadcast through LDS.
//   * Merge kernel: one workgroup per (sequence, kv-head) combines its partials (m, l, acc) in workgroup order,
//     divides, applies the optional sigmoid gate and writes [B, Hq, D].
// Bounds: lens are clamped to max_nb * bs and table entries to [0, num_blocks), so a malformed table cannot make a
// load leave the pool. Positions outside [s0, len) are never used: their scores are replaced (not added) by -inf and
// their V values by 0 before the FMA, so a NaN-poisoned block outside the window cannot leak in.
#include "rk_device.h"
#include "rk_internal.h"

#include <stdlib.h>

namespace rk {
namespace {

constexpr int kMaxBatch = 1024;
constexpr int kMaxKvHeads = 4;     // one wave per kv head in a split workgroup of at most 256 threads
constexpr int kTile = 16;

struct DecodeArgs {
    float* part;
    float* out;
    const float* q;
    const void* kp;
    const void* vp;
    const int32_t* tables;
    const int32_t* lens;
    const float* gate;
    int B, Hq, Hkv, G, bs, max_nb, num_blocks, window, NW;
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

// Workgroup plan, computed by one wave: wg0[b] = first split workgroup of sequence b (exclusive prefix of
// n(b) = units ? max(1, round(units * NW / U)) : 0), wg0[B] = workgroups in use. Returns U (all tiles).
__device__ long long plan_workgroups(const DecodeArgs& a, int* wg0) {
    const int lane = threadIdx.x & 63;
    long long U = 0;
    for (int b0 = 0; b0 < a.B; b0 += 64) {
        const int b = b0 + lane;
        int x = b < a.B ? seq_range(a, b).units : 0;
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) x += __shfl_xor(x, off);
        U += x;
    }
    int carry = 0;
    for (int b0 = 0; b0 < a.B; b0 += 64) {
        const int b = b0 + lane;
        const int units = b < a.B ? seq_range(a, b).units : 0;
        int x = 0;
        if (units > 0) {
            const long long r = ((long long)units * a.NW + U / 2) / U;
            x = r < 1 ? 1 : (int)r;
        }
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
            const int y = __shfl_up(x, off);
            if (lane >= off) x += y;
        }
        if (b < a.B) wg0[b + 1] = carry + x;
        carry += __shfl(x, 63);
    }
    if (lane == 0) wg0[0] = 0;
    return U;
}

// largest b with wg0[b] <= w (wg0 non-decreasing, wg0[0] = 0)
__device__ __forceinline__ int seq_of_workgroup(const int* wg0, int B, int w) {
    int lo = 0, hi = B - 1;
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (wg0[mid] <= w) lo = mid; else hi = mid - 1;
    }
    return lo;
}

template <typename T>
struct KVLoad;

// bf16 pool: 8 elements = one 16-byte load.
template <>
struct KVLoad<uint16_t> {
    static constexpr int KS = 1;   // key splits
    struct Vec { u32x4 w; };
    __device__ static Vec load(const void* base, long long off) {
        Vec v;
        v.w = *reinterpret_cast<const u32x4*>(reinterpret_cast<const uint16_t*>(base) + off);
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
                                                                        const SeqRange& sr, int tbase, int blk,
                                                                        int kvh, int D, int lane) {
    TileRows<NVI, TPI, LPT, ALIGNED> r;
    r.partial = tbase < sr.s0 || tbase + kTile > sr.L;
    const int tk = tbase + (lane & 15);
    r.kvalid = tk >= sr.s0 && tk < sr.L;
    r.vmask = 0;
#pragma unroll
    for (int vi = 0; vi < NVI; ++vi) {
        const int tv = tbase + vi * TPI + lane / LPT;
        r.vmask |= (uint32_t)(tv >= sr.s0 && tv < sr.L) << vi;
    }
    if constexpr (ALIGNED) {
        // rows past the length are still rows of the allocated block: no clamping needed for addressing
        const long long row0 = (long long)blk * a.bs + tbase % a.bs;
        r.krow = ((row0 + (lane & 15)) * a.Hkv + kvh) * D;
        r.vbase = ((row0 + lane / LPT) * a.Hkv + kvh) * D + (lane % LPT) * 8;
        r.vstride = (long long)TPI * a.Hkv * D;
    } else {
        const int tkc = tk < sr.s0 ? sr.s0 : (tk >= sr.L ? sr.L - 1 : tk);
        r.krow = kv_row(table, tkc, a.bs, a.Hkv, kvh, D, a.num_blocks);
#pragma unroll
        for (int vi = 0; vi < NVI; ++vi) {
            const int tv = tbase + vi * TPI + lane / LPT;
            const int tvc = tv < sr.s0 ? sr.s0 : (tv >= sr.L ? sr.L - 1 : tv);
            r.vr[vi] = kv_row(table, tvc, a.bs, a.Hkv, kvh, D, a.num_blocks) + (lane % LPT) * 8;
        }
    }
    return r;
}

// One workgroup = Hkv waves, wave k serving kv-head k: the waves of a workgroup walk the same tiles, so both halves
// of every interleaved pool row ([bs][Hkv][D]) are fetched together.
template <typename T, int D, int GP, bool ALIGNED>
__global__ __launch_bounds__(256) void paged_decode_split(DecodeArgs a) {
    using LD = KVLoad<T>;
    constexpr int NIT = D / 32;              // MFMA k-steps per tile
    constexpr int NT = (3 * GP + 15) / 16;   // A tiles: 3 query splits x GP heads, 16 rows each
    constexpr int LPT = D / 8;               // lanes per position row in the V layout
    constexpr int TPI = 64 / LPT;            // positions per V step
    constexpr int NVI = kTile / TPI;         // V steps per tile
    constexpr int KS = LD::KS;
    constexpr int HB = GP / 4;               // head blocks of 4 in the score layout

    extern __shared__ __attribute__((aligned(16))) char smem[];
    const int lane = threadIdx.x & 63;
    const int kvh = threadIdx.x >> 6;
    const int w = blockIdx.x;
    const int row = lane & 15;     // MFMA row / column owned by this lane
    const int grp = lane >> 4;     // k-slot group (operands) / row block (accumulator)

    int* wg0 = reinterpret_cast<int*>(smem);
    char* wl = smem + (((a.B + 1) * 4 + 15) & ~15) + kvh * wave_lds_bytes<D, GP>();
    u32x4* qop = reinterpret_cast<u32x4*>(wl);
    float* p_lds = reinterpret_cast<float*>(wl + NT * NIT * 64 * 16);
    float* alpha_lds = p_lds + kTile * GP;

    if (kvh == 0) plan_workgroups(a, wg0);
    __syncthreads();
    if (w >= wg0[a.B]) return;
    const int b = seq_of_workgroup(wg0, a.B, w);
    const int r = w - wg0[b], nwg = wg0[b + 1] - wg0[b];
    const SeqRange sr = seq_range(a, b);
    const int ta = (int)((long long)sr.units * r / nwg), tb = (int)((long long)sr.units * (r + 1) / nwg);
    const int n_here = tb - ta;
    const int32_t* table = a.tables + (long long)b * a.max_nb;
    const int tile0 = sr.t0 + ta;

    // ---- query rows of (b, kvh) requested first; split into MFMA operands once the first tile's loads are out
    float4 qx[NT][NIT][2];
#pragma unroll
    for (int tt = 0; tt < NT; ++tt) {
        const int m = 16 * tt + row;
        const int h = m % GP;
        const bool valid = m / GP < 3 && h < a.G;
        const float* qh = a.q + ((long long)b * a.Hq + kvh * a.G + (valid ? h : 0)) * D;
#pragma unroll
        for (int it = 0; it < NIT; ++it) {
            const int d = 32 * it + 8 * grp;
            qx[tt][it][0] = *reinterpret_cast<const float4*>(qh + d);
            qx[tt][it][1] = *reinterpret_cast<const float4*>(qh + d + 4);
        }
    }

    float m_run[4], l_run[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) { m_run[i] = -INFINITY; l_run[i] = 0.0f; }
    float acc[GP][8];
#pragma unroll
    for (int h = 0; h < GP; ++h)
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[h][e] = 0.0f;

    // block of each tile (ALIGNED): lane j holds the table entry of tile seg + j; tiles are walked in segments of 64
    // so the inner loop never reloads it
    int blk_lane = 0;
    auto refill = [&](int seg) {
        if (!ALIGNED) return;
        const int t = (tile0 + seg + lane) * kTile;
        const int j = seg + lane < n_here ? t / a.bs : 0;
        const int blk = table[j < a.max_nb ? j : 0];
        blk_lane = blk < 0 ? 0 : (blk >= a.num_blocks ? a.num_blocks - 1 : blk);
    };
    auto rows_of = [&](int seg, int ti) {
        const int blk = ALIGNED ? __builtin_amdgcn_readlane(blk_lane, ti) : 0;
        return tile_rows<NVI, TPI, LPT, ALIGNED>(a, table, sr, (tile0 + seg + ti) * kTile, blk, kvh, D, lane);
    };

    for (int seg = 0; seg < n_here; seg += 64) {
        const int nseg = n_here - seg < 64 ? n_here - seg : 64;
        refill(seg);
        TileRows<NVI, TPI, LPT, ALIGNED> cur = rows_of(seg, 0);
        typename LD::Vec kv[NIT], vv[NVI];
        // issue order K then V, here and in the loop, so that waiting for a tile's keys never waits for its values
        // (the scheduling barriers keep the compiler from reordering the two groups of loads)
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int it = 0; it < NIT; ++it) kv[it] = LD::load(a.kp, cur.krow + 32 * it + 8 * grp);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int vi = 0; vi < NVI; ++vi) vv[vi] = LD::load(a.vp, cur.vrow(vi));
        __builtin_amdgcn_sched_barrier(0);

        if (seg == 0) {
            // operands: row r of A tile tt holds split (m / GP) of head (m % GP), m = 16 tt + r, scaled by
            // log2(e)/sqrt(D); each lane reads back only its own operands, so no barrier is needed
#pragma unroll
            for (int tt = 0; tt < NT; ++tt) {
                const int s = (16 * tt + row) / GP;
                const bool valid = s < 3 && (16 * tt + row) % GP < a.G;
#pragma unroll
                for (int it = 0; it < NIT; ++it) {
                    const float xs[8] = {qx[tt][it][0].x, qx[tt][it][0].y, qx[tt][it][0].z, qx[tt][it][0].w,
                                         qx[tt][it][1].x, qx[tt][it][1].y, qx[tt][it][1].z, qx[tt][it][1].w};
                    uint32_t bits[8];
#pragma unroll
                    for (int e = 0; e < 8; ++e) {
                        const Split3 sp = split3(valid ? xs[e] * a.qscale : 0.0f);
                        bits[e] = s == 0 ? sp.hi : (s == 1 ? sp.mid : sp.lo);
                    }
                    u32x4 op;
#pragma unroll
                    for (int j = 0; j < 4; ++j) op[j] = pack_hi2(bits[2 * j], bits[2 * j + 1]);
                    qop[(tt * NIT + it) * 64 + lane] = op;
                }
            }
        }

        for (int ti = 0; ti < nseg; ++ti) {
            // ---- scores: S[m][n] = sum_d A[m][d] * K[n][d]
            f32x4 sacc[NT];
#pragma unroll
            for (int tt = 0; tt < NT; ++tt) sacc[tt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int it = 0; it < NIT; ++it) {
                u32x4 kb[KS];
                LD::key_operands(kv[it], kb);
#pragma unroll
                for (int ks = 0; ks < KS; ++ks)
#pragma unroll
                    for (int tt = 0; tt < NT; ++tt)
                        sacc[tt] = mfma16x16x32(qop[(tt * NIT + it) * 64 + lane], kb[ks], sacc[tt]);
            }

            // ---- keys of the next tile go in flight now. Issued unconditionally (the last tile of a segment
            // re-requests its own rows, which hit in L2): a conditional issue would make every later wait for this
            // tile's values a wait for all outstanding loads.
            const TileRows<NVI, TPI, LPT, ALIGNED> nxt = rows_of(seg, ti + 1 < nseg ? ti + 1 : ti);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int it = 0; it < NIT; ++it) kv[it] = LD::load(a.kp, nxt.krow + 32 * it + 8 * grp);
            __builtin_amdgcn_sched_barrier(0);

            // sum the three query splits: lane (grp, row) then holds heads 4 * (grp % HB) + i of position row
            float sc[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                float x = sacc[0][i];
#pragma unroll
                for (int tt = 1; tt < NT; ++tt) x += sacc[tt][i];
                if (GP == 4) x += __shfl_xor(x, 16);
                x += __shfl_xor(x, 32);
                sc[i] = cur.kvalid ? x : -INFINITY;
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
            // every outstanding load, including the next tile's keys)
#pragma unroll
            for (int vi = 0; vi < NVI; ++vi) LD::keep_if(vv[vi], cur.vvalid(vi));
#pragma unroll
            for (int vi = 0; vi < NVI; ++vi) {
                float vf[8];
                LD::widen(vv[vi], vf);
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

            // ---- values of the next tile go in flight now
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int vi = 0; vi < NVI; ++vi) vv[vi] = LD::load(a.vp, nxt.vrow(vi));
            __builtin_amdgcn_sched_barrier(0);
            cur = nxt;
            wave_lds_sync();   // p_lds / alpha_lds are rewritten by the next tile
        }
    }

    // ---- the partial of (workgroup w, kv-head): acc [GP][D], then m [GP], l [GP]
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
    float* slot = a.part + ((long long)w * a.Hkv + kvh) * (GP * (D + 2));
    if (lane < LPT) {
#pragma unroll
        for (int h = 0; h < GP; ++h) {
            float4* dst = reinterpret_cast<float4*>(slot + h * D + lane * 8);
            dst[0] = make_float4(acc[h][0], acc[h][1], acc[h][2], acc[h][3]);
            dst[1] = make_float4(acc[h][4], acc[h][5], acc[h][6], acc[h][7]);
        }
    }
    float lsum[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) lsum[i] = row16_sum(l_run[i]);
    if (grp < HB && row == 0) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            slot[GP * D + 4 * grp + i] = m_run[i];
            slot[GP * D + GP + 4 * grp + i] = lsum[i];
        }
    }
}

// One workgroup per (sequence, kv-head) pair: combines the partials of the sequence's split workgroups
// [wg0[b], wg0[b + 1]) in workgroup order with a running maximum. For each chunk of up to 32 partials the
// accumulators, maxima and sums are all requested before any is used (one memory round trip per chunk), then
// M' = max(M, m_w), num = num * 2^(M - M') + sum_w 2^(m_w - M') acc_w, den likewise with l_w; out = num / den.
constexpr int kMergeThreads = 512;

template <int D, int GP>
__global__ __launch_bounds__(kMergeThreads) void paged_decode_merge(DecodeArgs a) {
    constexpr int kT = kMergeThreads;
    constexpr int NO = (GP * D + kT - 1) / kT;      // outputs per thread (upper bound)
    constexpr int kCh = NO <= 2 ? 32 : 16;           // partials per memory round trip
    __shared__ int wg0[kMaxBatch + 1];
    __shared__ float ml[kCh][2][GP];
    const int tid = threadIdx.x;
    const int pair = blockIdx.x;
    const int b = pair / a.Hkv, kvh = pair % a.Hkv;
    if (tid < 64) plan_workgroups(a, wg0);
    __syncthreads();
    const int w0 = wg0[b], nwg = wg0[b + 1] - wg0[b];
    float* out = a.out + ((long long)b * a.Hq + kvh * a.G) * D;
    if (nwg == 0) {                                  // empty sequence (length 0)
        for (int i = tid; i < a.G * D; i += kT) out[i] = 0.0f;
        return;
    }
    const long long stride = GP * (D + 2);
    auto slot_of = [&](int w) { return ((long long)w * a.Hkv + kvh) * stride; };

    int off[NO], hk[NO];                 // this thread's outputs i = tid + k * kT: offset h * D + d, head h
    float M[NO], num[NO], den[NO];
#pragma unroll
    for (int k = 0; k < NO; ++k) {
        const int i = tid + k * kT;
        const int ic = i < a.G * D ? i : 0;
        hk[k] = ic / D;
        off[k] = ic;
        M[k] = -INFINITY;
        num[k] = 0.0f;
        den[k] = 0.0f;
    }
    for (int c0 = 0; c0 < nwg; c0 += kCh) {
        const int n_in = min(kCh, nwg - c0);
        // all loads of the chunk first (indices clamped to the chunk's last partial)
        float v[kCh][NO];
#pragma unroll
        for (int j = 0; j < kCh; ++j) {
            const long long base = slot_of(w0 + c0 + min(j, n_in - 1));
#pragma unroll
            for (int k = 0; k < NO; ++k) v[j][k] = a.part[base + off[k]];
        }
        for (int t = tid; t < kCh * 2 * GP; t += kT) {
            const int j = t / (2 * GP), rr = t % (2 * GP);
            ml[j][rr / GP][rr % GP] = a.part[slot_of(w0 + c0 + min(j, n_in - 1)) + GP * D + rr];
        }
        __syncthreads();
#pragma unroll
        for (int k = 0; k < NO; ++k) {
            float mx = M[k];
#pragma unroll
            for (int j = 0; j < kCh; ++j) mx = j < n_in ? fmaxf(mx, ml[j][0][hk[k]]) : mx;
            const float rs = fast_exp2(M[k] - mx);      // 0 on the first chunk (M = -inf, mx finite)
            float nk = num[k] * rs, dk = den[k] * rs;
#pragma unroll
            for (int j = 0; j < kCh; ++j) {
                const float sc = fast_exp2(ml[j][0][hk[k]] - mx);
                const float tn = fmaf(sc, v[j][k], nk), td = fmaf(sc, ml[j][1][hk[k]], dk);
                nk = j < n_in ? tn : nk;                 // a select: clamped duplicates never enter
                dk = j < n_in ? td : dk;
            }
            num[k] = nk;
            den[k] = dk;
            M[k] = mx;
        }
        __syncthreads();
    }
#pragma unroll
    for (int k = 0; k < NO; ++k) {
        const int i = tid + k * kT;
        if (i >= a.G * D) break;
        float o = num[k] / den[k];
        if (a.gate) {
            const float gv = a.gate[(long long)b * a.Hq * D + (long long)kvh * a.G * D + i];
            o = o * (1.0f / (1.0f + expf(-gv)));
        }
        out[i] = o;
    }
}

typedef void (*SplitFn)(DecodeArgs);
typedef void (*MergeFn)(DecodeArgs);

template <typename T, bool ALIGNED>
SplitFn pick_split(int D, int GP) {
    if (GP == 4) {
        if (D == 64) return paged_decode_split<T, 64, 4, ALIGNED>;
        if (D == 128) return paged_decode_split<T, 128, 4, ALIGNED>;
        if (D == 256) return paged_decode_split<T, 256, 4, ALIGNED>;
    } else {
        if (D == 64) return paged_decode_split<T, 64, 8, ALIGNED>;
        if (D == 128) return paged_decode_split<T, 128, 8, ALIGNED>;
        if (D == 256) return paged_decode_split<T, 256, 8, ALIGNED>;
    }
    return nullptr;
}

SplitFn pick_split(int kv_dtype, bool aligned, int D, int GP) {
    if (kv_dtype == RK_BF16) return aligned ? pick_split<uint16_t, true>(D, GP) : pick_split<uint16_t, false>(D, GP);
    return aligned ? pick_split<float, true>(D, GP) : pick_split<float, false>(D, GP);
}

int split_lds_bytes(int B, int Hkv, int D, int GP) {
    int per_wave = 0;
    if (GP == 4) per_wave = D == 64 ? wave_lds_bytes<64, 4>() : D == 128 ? wave_lds_bytes<128, 4>() : wave_lds_bytes<256, 4>();
    else per_wave = D == 64 ? wave_lds_bytes<64, 8>() : D == 128 ? wave_lds_bytes<128, 8>() : wave_lds_bytes<256, 8>();
    return (((B + 1) * 4 + 15) & ~15) + Hkv * per_wave;
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

// Workgroups of the split phase (Hkv waves each): the tile count's upper bound, capped so that about
// kWavesPerCU waves per compute unit are resident. RK_PAGED_DECODE_WAVES_PER_CU overrides the cap (tuning).
constexpr int kWavesPerCU = 6;

int split_groups(int B, int Hkv, int block_size, int max_nb) {
    static int per_cu = [] {
        const char* e = getenv("RK_PAGED_DECODE_WAVES_PER_CU");
        const int v = e ? atoi(e) : 0;
        return v > 0 ? v : kWavesPerCU;
    }();
    const long long upper = (long long)B * (((long long)max_nb * block_size + kTile - 1) / kTile);
    int cus = device_cus();
    if (cus <= 0) cus = 256;
    const long long cap = (long long)cus * per_cu / Hkv;
    long long nw = upper < cap ? upper : cap;
    return (int)(nw < 1 ? 1 : nw);
}

// n(b) <= units(b) NW / U + 1, so at most NW + B split workgroups are ever used: the grid and the partials.
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

int rk_paged_decode_phase(int phase, float* out, const float* q, const void* k_pool, const void* v_pool,
                          int kv_dtype, const int32_t* tables, const int32_t* lens, int B, int Hq, int Hkv, int D,
                          int block_size, int max_nb, int num_blocks, int window, const float* gate,
                          void* workspace, size_t workspace_bytes_, void* stream) {
    int rc = validate(out, q, k_pool, v_pool, kv_dtype, tables, lens, B, Hq, Hkv, D, block_size, max_nb,
                      num_blocks, window);
    if (rc) return rc;
    if (phase != 0 && phase != 1) return fail(RK_ERR_ARG, "rk_paged_decode_phase: phase %d", phase);
    const int G = Hq / Hkv;
    const int GP = G <= 4 ? 4 : 8;
    const int NW = split_groups(B, Hkv, block_size, max_nb);
    const size_t need = workspace_bytes(B, Hkv, D, GP, NW);
    if (!workspace || workspace_bytes_ < need)
        return fail(RK_ERR_WORKSPACE, "rk_paged_decode: workspace %zu bytes < %zu needed", workspace_bytes_, need);

    DecodeArgs a;
    a.part = static_cast<float*>(workspace);
    a.out = out;
    a.q = q;
    a.kp = k_pool;
    a.vp = v_pool;
    a.tables = tables;
    a.lens = lens;
    a.gate = gate;
    a.B = B; a.Hq = Hq; a.Hkv = Hkv; a.G = G; a.bs = block_size; a.max_nb = max_nb;
    a.num_blocks = num_blocks; a.window = window; a.NW = NW;
    a.qscale = kLog2e / sqrtf((float)D);
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (phase == 0) {
        SplitFn fn = pick_split(kv_dtype, block_size % kTile == 0, D, GP);
        hipLaunchKernelGGL(fn, dim3(NW + B), dim3(64 * Hkv), split_lds_bytes(B, Hkv, D, GP), s, a);
        return check_launch("paged_decode_split");
    }
    hipLaunchKernelGGL(pick_merge(D, GP), dim3(B * Hkv), dim3(kMergeThreads), 0, s, a);
    return check_launch("paged_decode_merge");
}

int rk_paged_decode(float* out, const float* q, const void* k_pool, const void* v_pool, int kv_dtype,
                    const int32_t* tables, const int32_t* lens, int B, int Hq, int Hkv, int D, int block_size,
                    int max_nb, int num_blocks, int window, const float* gate, void* workspace,
                    size_t workspace_bytes_, void* stream) {
    int rc = rk_paged_decode_phase(0, out, q, k_pool, v_pool, kv_dtype, tables, lens, B, Hq, Hkv, D, block_size,
                                   max_nb, num_blocks, window, gate, workspace, workspace_bytes_, stream);
    if (rc) return rc;
    return rk_paged_decode_phase(1, out, q, k_pool, v_pool, kv_dtype, tables, lens, B, Hq, Hkv, D, block_size,
                                 max_nb, num_blocks, window, gate, workspace, workspace_bytes_, stream);
}

}  // extern "C"
