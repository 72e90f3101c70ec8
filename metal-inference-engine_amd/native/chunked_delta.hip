// P3: chunked gated delta rule (WY / UT form, 64-token chunks) for packed prefill, gfx950.
//
// Semantics: ops.gated_delta_chunked (src/ops.py:160-193), reached through Backend.gated_delta with T > 1
// (src/backend/torch_ref.py:52-56) from the packed prefill of the linear-attention layers
// (src/models/qwen3_5.py:136-162). Per sequence and head, chunk by chunk, with the chunk-local cumulative log-decay
// G = cumsum(g) and the state S [dk, dv] carried between chunks:
//   D[i][j] = exp(G_i - G_j) for j <= i, else 0                              (:177-178, masked before exp)
//   T  = (I + tril(diag(beta) K K^T * D, -1))^-1                              (:179-182, the forward substitution)
//   vn = T diag(beta) (V - diag(e^G) K S)                                     (= U - W S, :183-184, :188)
//   o  = diag(e^G) Q S + (Q K^T * D) vn                                       (:187, :189)
//   S <- e^{G_last} S + K^T diag(e^{G_last - G}) vn                           (:190)
// Rows past a sequence's end are zero (k = v = beta = g = 0), which leaves S untouched, as the reference's padding.
//
// Kernels:
//   delta_chunk_prep  one workgroup per (chunk, head), all chunks in parallel: beta, G (summed in fp64 and rounded
//                     once, as torch's CPU cumsum of fp32 accumulates in double), exp(G), exp(G_last - G); K K^T (and
//                     for fp32 inputs Q K^T) on MFMA from K rows staged in LDS; T by blocked inversion of the unit lower
//                     triangular matrix (16 x 16 diagonal blocks by substitution, off-diagonal blocks by fp32 MFMA
//                     products in three levels). For fp32 inputs T and P = Q K^T * D go to the workspace already split
//                     into bf16 pieces, in the operand order the scan loads, so the scan workgroups of a head share
//                     them instead of each recomputing them; for bf16 inputs T goes there as an fp32 triangle.
//   delta_chunk_scan_cols (bf16 inputs, chunked_delta_cols.hip)  one workgroup per (sequence, head, 32-column slice
//                     of S), one wave per 16 columns over all 64 tokens of a chunk: no exchange between waves at all.
//                     Its two loading waves, on SIMDs of their own, split T into pieces and compute P from the
//                     chunk's K and Q rows while the previous chunk is computed.
//   delta_chunk_scan  (fp32 inputs) one workgroup per (sequence, head, 32-column slice of S): the columns of S evolve
//                     independently, so the serial pass over a sequence's chunks runs 4 workgroups wide per head.
//                     Wave w owns token rows 16w..16w+15 of the chunk and state rows 32w..32w+31 (two 16-column
//                     tiles sharing every A operand: the K / Q / T / P bytes a CU pulls from L2 per chunk are spread
//                     over 32 columns); the three
//                     exchanges per chunk (state pieces, Y, vn) go through LDS behind LDS-only barriers. Everything
//                     chunk c+1 reads from global memory (K, Q, V rows, coefficients, T and P pieces) is requested at
//                     the start of chunk c, so memory latency hides behind a whole chunk of work.
// Precision: every product with an fp32 operand (S, Y, vn, T, P, fp32 inputs) runs on bf16 MFMA with that operand
// split exactly into three bf16 pieces (truncation) and the piece products of order >= 2^-16 kept; bf16 inputs are
// exact operands. Products are therefore exact to ~2^-20 relative and accumulate in fp32: fp32-level results.
#include <type_traits>

#include "chunked_delta.h"
#include "rk_internal.h"

namespace rk {
namespace {

using namespace delta;

// =====================================================================================================================
// Phase 1: per-chunk coefficients, T and P
// =====================================================================================================================
template <typename In>
struct PrepStage {
    static constexpr int kRow = kDk + (sizeof(In) == 2 ? 8 : 4);
};

// split 4 fp32 values and store them as kTP pieces of 4 bf16 at dst + piece * kPieceElems
__device__ __forceinline__ void store_pieces4(uint16_t* dst, const float (&x)[4]) {
    u32x2 pc[kTP];
    if constexpr (kTP == kNS) split4(x, pc); else split4_rn(x, pc);
#pragma unroll
    for (int pi = 0; pi < kTP; ++pi) *reinterpret_cast<u32x2*>(dst + pi * kPieceElems) = pc[pi];
}

// The prep's LDS holds only the 10 lower-triangular 16 x 16 blocks of A0 and of T, each padded to 16 x 17 floats,
// block (w, b) (b <= w) at index w (w + 1) / 2 + b; the chunk's K rows share the same bytes until the Gram products
// are in registers. 21.8 KB per workgroup for bf16 inputs (38.4 KB with full 64 x 65 arrays and separate K rows), so
// 7 workgroups fit a CU instead of 4: the prep's time is the latency of its dependent steps, hidden by occupancy.
constexpr int kBlkF = 16 * 17;                             // floats of one padded block
constexpr int kTriBlocks = 10;
__device__ __forceinline__ int tri_blk(int w, int b) { return w * (w + 1) / 2 + b; }

template <typename In>
__global__ __launch_bounds__(256) void delta_chunk_prep(DeltaArgs p) {
    using St = PrepStage<In>;
    constexpr int kKBytes = kC * St::kRow * sizeof(In), kTriBytes = 2 * kTriBlocks * kBlkF * 4;
    __shared__ __align__(16) char smem[kKBytes > kTriBytes ? kKBytes : kTriBytes];
    In* sK = reinterpret_cast<In*>(smem);                  // K rows of the chunk, until the Gram products are done
    float* const sAb = reinterpret_cast<float*>(smem);     // then A0 = -beta_i (K K^T)_ij D_ij below the diagonal
    float* const sTb = sAb + kTriBlocks * kBlkF;           // and T
    // element (i, m) of block (w, b): A0 / T rows 16 w + i, columns 16 b + m
    auto sA = [&](int w, int b, int i, int m) -> float& { return sAb[tri_blk(w, b) * kBlkF + 17 * i + m]; };
    auto sT = [&](int w, int b, int i, int m) -> float& { return sTb[tri_blk(w, b) * kBlkF + 17 * i + m]; };
    // per-wave 16 x 16 scratch of the off-diagonal products: A0's diagonal block w, dead once T's is formed
    auto sTmp = [&](int w, int i, int m) -> float& { return sAb[tri_blk(w, w) * kBlkF + 17 * i + m]; };

    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, q = lane >> 4, r = lane & 15;
    const int gc = blockIdx.x, h = blockIdx.y, H = p.H;
    const int s = seq_of_chunk(p, gc);
    const int t0 = p.cu[s] + (gc - p.cu_chunks[s]) * kC;
    const int nt = min(kC, p.cu[s + 1] - t0);
    if (nt <= 0) return;                  // offsets inconsistent with cu_chunks: nothing of this chunk is read
    const In* K = static_cast<const In*>(p.k);
    const In* Q = static_cast<const In*>(p.q);

    // bf16 inputs (lane order): the scan computes P itself, so only K K^T is formed here
    constexpr bool kLane = sizeof(In) == 2;
    // K (and Q) rows of row tile w, zero past the sequence's end; all loads issued up front
    Row8<In> ka[4], qa[4];
    {
        const int t = 16 * w + r;
        const long long off = ((long long)(t0 + min(t, nt - 1)) * H + h) * kDk + 8 * q;
        const uint32_t m = mask_if(t < nt);
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            ka[k].load(K + off + 32 * k);
            ka[k].keep(m);
            if constexpr (!kLane) {
                qa[k].load(Q + off + 32 * k);
                qa[k].keep(m);
            }
        }
    }
    const bool live = lane < nt;
    const long long ti = (long long)(t0 + min(lane, nt - 1)) * H + h;
    const float bl = live ? p.beta[ti] : 0.f;
    const float gl = live ? p.g[ti] : 0.f;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        In* dst = sK + (16 * w + r) * St::kRow + 32 * k + 8 * q;
        if constexpr (sizeof(In) == 2) {
            *reinterpret_cast<u32x4*>(dst) = ka[k].v;
        } else {
            *reinterpret_cast<f32x4*>(dst) = ka[k].a;
            *reinterpret_cast<f32x4*>(dst + 4) = ka[k].b;
        }
    }
    // cumulative log-decay of the chunk, one token per lane (every wave keeps its own copy)
    double acc = gl;
#pragma unroll
    for (int off = 1; off < kC; off <<= 1) {
        const double y = __shfl_up(acc, off);
        if (lane >= off) acc += y;
    }
    const float G = (float)acc;
    lds_barrier();

    // Tiles (b, w) of K K^T and of P^T = K Q^T (A = K rows of tile b from LDS, B = this wave's K / Q rows): lane (q, r)
    // holds entries (t', t) = (16b + 4q + i, 16w + r), i.e. row t of A0 and P at columns t'.
    float* rec = p.ws + ((size_t)gc * H + h) * (kLane ? kLaneChunkFloats : kChunkFloats);
    uint16_t* ws16 = reinterpret_cast<uint16_t*>(rec);
    const float Gt = __shfl(G, 16 * w + r), bt = __shfl(bl, 16 * w + r);
    const int t = 16 * w + r;
    float av[4][4];                        // A0 entries of tiles b <= w, kept until every wave is done with sK
#pragma unroll
    for (int b = 0; b < 4; ++b) {
        if (b >= (kLane ? w + 1 : 2 * ((w >> 1) + 1))) break;      // uniform per wave
        float pv[4] = {0.f, 0.f, 0.f, 0.f};
        if (b <= w) {
            f32x4 kk = {0.f, 0.f, 0.f, 0.f}, pq = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                Row8<In> kb;
                const In* src = sK + (16 * b + r) * St::kRow + 32 * k + 8 * q;
                if constexpr (sizeof(In) == 2) {
                    kb.v = *reinterpret_cast<const u32x4*>(src);
                } else {
                    kb.a = *reinterpret_cast<const f32x4*>(src);
                    kb.b = *reinterpret_cast<const f32x4*>(src + 4);
                }
                u32x4 pa[Row8<In>::KP], pb[Row8<In>::KP];
                kb.pieces(pa);
                ka[k].pieces(pb);
                kk = mma(pa, pb, kk);
                if constexpr (!kLane) {
                    qa[k].pieces(pb);
                    pq = mma(pa, pb, pq);
                }
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int tp = 16 * b + 4 * q + i;
                const float Gp = __shfl(G, tp);
                // masked before exp; exp(x) as 2^(x log2 e) on v_exp_f32: within ~1e-6 relative for the
                // |x| < 20 that carry weight (the rounding of x log2 e is |x| 2^-24)
                const float d = tp <= t ? fast_exp2((Gt - Gp) * kLog2e) : 0.f;
                av[b][i] = tp < t ? -(bt * kk[i]) * d : 0.f;
                pv[i] = pq[i] * d;
            }
        }
        if constexpr (!kLane) store_pieces4(ws16 + kPOff + rt_base(w) + r * rt_width(w) + 16 * b + 4 * q, pv);
    }
    lds_barrier();                         // sK is dead from here: its bytes hold A0 and T
#pragma unroll
    for (int b = 0; b < 4; ++b)
        if (b <= w)
#pragma unroll
            for (int i = 0; i < 4; ++i) sA(w, b, r, 4 * q + i) = av[b][i];
    lds_barrier();

    // diagonal block w of T = (I - A0)^-1: lane r keeps column r, rows by forward substitution
    {
        float x[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            float a = i == r ? 1.f : 0.f;
#pragma unroll
            for (int m = 0; m < i; ++m) a = fmaf(sA(w, w, i, m), x[m], a);
            x[i] = a;
        }
        if (q == 0)
#pragma unroll
            for (int i = 0; i < 16; ++i) sT(w, w, i, r) = x[i];
    }
    lds_barrier();

    // off-diagonal blocks, one distance d = w - j at a time: T_wj = T_ww * sum_{k=j}^{w-1} A0_wk T_kj
    for (int d = 1; d < 4; ++d) {
        if (w >= d) {
            const int j = w - d;
            f32x4 tt = {0.f, 0.f, 0.f, 0.f};
            for (int kb = j; kb < w; ++kb)
#pragma unroll
                for (int ks = 0; ks < 4; ++ks)
                    tt = mfma_f32(sA(w, kb, r, 4 * ks + q), sT(kb, j, 4 * ks + q, r), tt);
#pragma unroll
            for (int i = 0; i < 4; ++i) sTmp(w, 4 * q + i, r) = tt[i];
            wave_lds_sync();
            f32x4 u = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int ks = 0; ks < 4; ++ks)
                u = mfma_f32(sT(w, w, r, 4 * ks + q), sTmp(w, 4 * ks + q, r), u);
#pragma unroll
            for (int i = 0; i < 4; ++i) sT(w, j, 4 * q + i, r) = u[i];
        }
        lds_barrier();
    }

    // T: the padded fp32 triangle for bf16 inputs, else row-tile blocks of pieces; entries above the diagonal are 0
    if constexpr (kLane) {
#pragma unroll
        for (int it = 0; it < kC * 16 / 256; ++it) {
            const int idx = threadIdx.x + 256 * it, row = idx >> 4, col = 4 * (idx & 15);
            if (col <= row) {
                f32x4 x;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int c = min(col + e, row);            // entries above the diagonal are not held
                    const float v = sT(row >> 4, c >> 4, row & 15, c & 15);
                    x[e] = col + e <= row ? v : 0.f;
                }
                *reinterpret_cast<f32x4*>(rec + tri_base(row) + col) = x;
            }
        }
    } else
#pragma unroll
    for (int it = 0; it < kPieceElems / 4 / 256; ++it) {
        const int off = 4 * (threadIdx.x + 256 * it);
        const int a = off < 512 ? 0 : (off < 1024 ? 1 : (off < 2048 ? 2 : 3));
        const int rel = off - rt_base(a);
        const int row = 16 * a + rel / rt_width(a), col = rel % rt_width(a);
        float x[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int c = min(col + e, row);
            const float v = sT(row >> 4, c >> 4, row & 15, c & 15);
            x[e] = col + e <= row ? v : 0.f;
        }
        store_pieces4(ws16 + kTOff + off, x);
    }
    if (w == 0) {
        const float Glast = __shfl(G, kC - 1);
        float* cf = rec + (kLane ? kLaneCoefOff : kCoefOff);
        cf[lane] = bl;
        cf[kC + lane] = G;
        cf[2 * kC + lane] = expf(G);
        cf[3 * kC + lane] = expf(Glast - G);
    }
}

// =====================================================================================================================
// Phase 2: the serial pass over chunks, one 16-column slice of S per workgroup
// =====================================================================================================================
template <typename In>
struct ScanLayout {
    static constexpr int kKt = kC + (sizeof(In) == 2 ? 8 : 4);    // row stride of staged K^T [dk][token]
    static constexpr size_t sp = 0;                                               // state pieces
    static constexpr size_t yp = sp + (size_t)kNS * kCols * kStateRow * 2;        // Y pieces
    static constexpr size_t vp = yp + (size_t)kNS * kCols * kPieceRow * 2;        // vn pieces
    static constexpr size_t vq = vp + (size_t)kNS * kCols * kPieceRow * 2;        // exp(G_last - G) vn pieces
    static constexpr size_t kt = vq + (size_t)kNS * kCols * kPieceRow * 2;        // K^T
    static constexpr size_t bytes = kt + (size_t)kDk * kKt * sizeof(In);
};

template <typename In, int W>
__device__ __forceinline__ void scan_wave(const DeltaArgs& p, char* lds, int s, int h, int slice) {
    using L = ScanLayout<In>;
    constexpr int KP = Row8<In>::KP;
    constexpr int KS = (W >> 1) + 1;      // 32-token k-steps of T and P that reach row tile W's diagonal
    const int lane = threadIdx.x & 63, q = lane >> 4, r = lane & 15;
    const int H = p.H;
    const int T0 = p.cu[s], Tn = p.cu[s + 1] - T0;
    const int gc0 = p.cu_chunks[s];
    // chunks of this sequence; never more than its workspace records (both offsets arrays come from the caller)
    const int nch = min((Tn + kC - 1) / kC, p.cu_chunks[s + 1] - gc0);
    const int col0 = slice * kCols;
    if (nch <= 0) return;                 // empty sequence: state unchanged, no barrier is reached by any wave
    float* Sg = p.S + (long long)(p.seq_index ? p.seq_index[s] : s) * p.s_stride + (long long)h * kDk * kDv + col0;
    const In* Kg = static_cast<const In*>(p.k);
    const In* Qg = static_cast<const In*>(p.q);
    const In* Vg = static_cast<const In*>(p.v);

    uint16_t* sp = reinterpret_cast<uint16_t*>(lds + L::sp);
    uint16_t* yp = reinterpret_cast<uint16_t*>(lds + L::yp);
    uint16_t* vp = reinterpret_cast<uint16_t*>(lds + L::vp);
    uint16_t* vq = reinterpret_cast<uint16_t*>(lds + L::vq);
    In* kt = reinterpret_cast<In*>(lds + L::kt);
    // [piece][column][row] exchange arrays: element (row, column 16 ct + r) of piece pi
    auto xrow = [&](uint16_t* base, int stride, int pi, int ct) { return base + (pi * kCols + 16 * ct + r) * stride; };

    // state rows 32W + 16u + 4q + i, columns col0 + 16ct + r (MFMA accumulator layout of the update)
    f32x4 st[2][kCT];
#pragma unroll
    for (int u = 0; u < 2; ++u)
#pragma unroll
        for (int ct = 0; ct < kCT; ++ct)
#pragma unroll
            for (int i = 0; i < 4; ++i) st[u][ct][i] = Sg[(32 * W + 16 * u + 4 * q + i) * kDv + 16 * ct + r];

    using VRaw = typename std::conditional<sizeof(In) == 2, uint32_t, float>::type;
    // What row tile W of chunk c needs first, loaded one chunk ahead: K and Q rows 16W + r (columns 32k + 8q .. +7,
    // zero past the sequence's end), the values at rows 16W + 4q + i and the coefficients of those rows.
    struct Ahead {
        Row8<In> k[4], q[4];                // raw rows; zeroed past the sequence's end by finish()
        uint32_t keep;
        VRaw v[kCT][4];                     // values as loaded (bf16 bits zero-extended, or fp32)
        float beta, eg, egr;                // row 16W + (lane & 15); rows 16W + 4q + i come by shuffle
        float glast;
        u32x4 ta[KS][kTP], pa[KS][kTP];     // T and P pieces of row tile W (A operands, k-steps 0 .. KS-1)
    };
    auto load_ahead = [&](int c, Ahead& a) {
        const int nt = min(kC, Tn - c * kC);
        const int tc = T0 + c * kC;
        const int t = 16 * W + r;
        const long long off = ((long long)(tc + min(t, nt - 1)) * H + h) * kDk + 8 * q;
        a.keep = mask_if(t < nt);
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            a.k[k].load(Kg + off + 32 * k);
            a.q[k].load(Qg + off + 32 * k);
        }
    };
    // the values and coefficients of row tile W
    auto load_ahead_v = [&](int c, Ahead& a) {
        const int nt = min(kC, Tn - c * kC);
        const int tc = T0 + c * kC;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int tv = min(16 * W + 4 * q + i, nt - 1);
            const In* vrow = Vg + ((long long)(tc + tv) * H + h) * kDv + col0 + r;
#pragma unroll
            for (int ct = 0; ct < kCT; ++ct) a.v[ct][i] = (VRaw)vrow[16 * ct];
        }
        const float* cf = p.ws + ((size_t)(gc0 + c) * H + h) * kChunkFloats + kCoefOff;
        a.beta = cf[16 * W + r];
        a.eg = cf[2 * kC + 16 * W + r];
        a.egr = cf[3 * kC + 16 * W + r];
        a.glast = cf[2 * kC + kC - 1];
    };
    // the T and P pieces of row tile W (the larger part of the look-ahead bytes), requested separately so that
    // their issue overlaps the X / QS products instead of preceding them
    auto load_ahead_tp = [&](int c, Ahead& a, int which) {   // which: 0 = T pieces, 1 = P pieces
        const uint16_t* ws16 = reinterpret_cast<const uint16_t*>(p.ws + ((size_t)(gc0 + c) * H + h) * kChunkFloats);
#pragma unroll
        for (int k = 0; k < KS; ++k)
#pragma unroll
            for (int pi = 0; pi < kTP; ++pi) {
                const int e = rt_base(W) + r * rt_width(W) + 32 * k + 8 * q + pi * kPieceElems;
                if (which == 0) a.ta[k][pi] = *reinterpret_cast<const u32x4*>(ws16 + kTOff + e);
                else a.pa[k][pi] = *reinterpret_cast<const u32x4*>(ws16 + kPOff + e);
            }
    };
    // An empty asm that takes every register of `a` as input and output: the loads behind them complete at this
    // point, and everything computed from them comes after it. Placed before a chunk's output stores, it keeps the
    // compiler from deferring (or hoisting) that wait: gfx950 counts loads and stores in one in-order counter, so a
    // wait placed after the stores would also wait for the stores.
    auto resident = [](Ahead& a) {
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            if constexpr (sizeof(In) == 2) {
                asm volatile("" : "+v"(a.k[k].v), "+v"(a.q[k].v));
            } else {
                asm volatile("" : "+v"(a.k[k].a), "+v"(a.k[k].b), "+v"(a.q[k].a), "+v"(a.q[k].b));
            }
            a.k[k].keep(a.keep);
            a.q[k].keep(a.keep);
        }
#pragma unroll
        for (int ct = 0; ct < kCT; ++ct)
#pragma unroll
            for (int i = 0; i < 4; ++i) asm volatile("" : "+v"(a.v[ct][i]));
        asm volatile("" : "+v"(a.beta), "+v"(a.eg), "+v"(a.egr), "+v"(a.glast));
#pragma unroll
        for (int k = 0; k < KS; ++k)
#pragma unroll
            for (int pi = 0; pi < kTP; ++pi) asm volatile("" : "+v"(a.ta[k][pi]), "+v"(a.pa[k][pi]));
    };
    Ahead cur;
    load_ahead(0, cur);
    load_ahead_v(0, cur);
    load_ahead_tp(0, cur, 0);
    load_ahead_tp(0, cur, 1);
    // the first chunk's data and the initial state complete before the loop, so no wait for them lands inside it
    resident(cur);
#pragma unroll
    for (int u = 0; u < 2; ++u)
#pragma unroll
        for (int ct = 0; ct < kCT; ++ct) asm volatile("" : "+v"(st[u][ct]));

    // One chunk: uses `cur` (chunk c), fills `nxt` with chunk c+1. The loop below alternates two buffers, so no
    // register copy of freshly loaded data (which would wait for the load) is ever needed.
    auto step = [&](int c, Ahead& cur, Ahead& nxt) __attribute__((always_inline)) {
        const int nt = min(kC, Tn - c * kC);
        const int tc = T0 + c * kC;
        // everything chunk c+1 reads from global memory is requested now and first used at the end of this chunk
        // (before this chunk's output stores are issued, so that wait never includes store completions)
        load_ahead(c + 1 < nch ? c + 1 : c, nxt);
        load_ahead_v(c + 1 < nch ? c + 1 : c, nxt);

        // ---- A1: state pieces -> LDS [piece][column][dk]
#pragma unroll
        for (int u = 0; u < 2; ++u)
#pragma unroll
            for (int ct = 0; ct < kCT; ++ct) {
                const float x[4] = {st[u][ct][0], st[u][ct][1], st[u][ct][2], st[u][ct][3]};
                u32x2 pc[kNS];
                split4(x, pc);
#pragma unroll
                for (int pi = 0; pi < kNS; ++pi)
                    *reinterpret_cast<u32x2*>(xrow(sp, kStateRow, pi, ct) + 32 * W + 16 * u + 4 * q) = pc[pi];
            }
        lds_barrier();

        // ---- A2: X = K S and Q S for row tile W; Y = beta (V - e^G X) -> LDS; K^T -> LDS
        f32x4 x[kCT], qs[kCT];
#pragma unroll
        for (int ct = 0; ct < kCT; ++ct) x[ct] = qs[ct] = (f32x4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            if (k == 1 || k == 3) {
                __builtin_amdgcn_sched_barrier(0);
                load_ahead_tp(c + 1 < nch ? c + 1 : c, nxt, k == 1 ? 0 : 1);
                __builtin_amdgcn_sched_barrier(0);
            }

            u32x4 ok[KP], oq[KP];
            cur.k[k].pieces(ok);
            cur.q[k].pieces(oq);
#pragma unroll
            for (int ct = 0; ct < kCT; ++ct) {
                u32x4 sb[kNS];
#pragma unroll
                for (int pi = 0; pi < kNS; ++pi)
                    sb[pi] = *reinterpret_cast<const u32x4*>(xrow(sp, kStateRow, pi, ct) + 32 * k + 8 * q);
                x[ct] = mma(ok, sb, x[ct]);
                qs[ct] = mma(oq, sb, qs[ct]);
            }
        }
        float beta4[4], eg4[4], egr4[4];  // coefficients of rows 16W + 4q + i
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            beta4[i] = __shfl(cur.beta, 4 * q + i);
            eg4[i] = __shfl(cur.eg, 4 * q + i);
            egr4[i] = __shfl(cur.egr, 4 * q + i);
        }
#pragma unroll
        for (int ct = 0; ct < kCT; ++ct) {
            float y[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) y[i] = beta4[i] * (to_f32(cur.v[ct][i]) - eg4[i] * x[ct][i]);
            u32x2 pc[kNS];
            split4(y, pc);
#pragma unroll
            for (int pi = 0; pi < kNS; ++pi)
                *reinterpret_cast<u32x2*>(xrow(yp, kPieceRow, pi, ct) + 16 * W + 4 * q) = pc[pi];
        }
#pragma unroll
        for (int k = 0; k < 4; ++k)
#pragma unroll
            for (int e = 0; e < 8; ++e) kt[(32 * k + 8 * q + e) * L::kKt + 16 * W + r] = cur.k[k].raw(e);
        lds_barrier();

        // ---- C: vn = T Y (row tile W); vn and e^{G_last-G} vn -> LDS
#pragma unroll
        for (int ct = 0; ct < kCT; ++ct) {
            f32x4 vn = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int k = 0; k < KS; ++k) {
                u32x4 yb[kNS];
#pragma unroll
                for (int pi = 0; pi < kNS; ++pi)
                    yb[pi] = *reinterpret_cast<const u32x4*>(xrow(yp, kPieceRow, pi, ct) + 32 * k + 8 * q);
                vn = mma(cur.ta[k], yb, vn);
            }
            float a4[4], b4[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                a4[i] = vn[i];
                b4[i] = egr4[i] * vn[i];
            }
            u32x2 pva[kNS], pvb[kNS];
            split4(a4, pva);
            split4(b4, pvb);
#pragma unroll
            for (int pi = 0; pi < kNS; ++pi) {
                *reinterpret_cast<u32x2*>(xrow(vp, kPieceRow, pi, ct) + 16 * W + 4 * q) = pva[pi];
                *reinterpret_cast<u32x2*>(xrow(vq, kPieceRow, pi, ct) + 16 * W + 4 * q) = pvb[pi];
            }
        }
        const float glast = cur.glast;
        resident(nxt);                    // complete the look-ahead loads here, ahead of this chunk's stores
        lds_barrier();

        // ---- D: o = e^G Q S + P vn; state update S = e^{G_last} S + K^T (e^{G_last-G} vn)
#pragma unroll
        for (int ct = 0; ct < kCT; ++ct) {
            f32x4 o;
#pragma unroll
            for (int i = 0; i < 4; ++i) o[i] = eg4[i] * qs[ct][i];
#pragma unroll
            for (int k = 0; k < KS; ++k) {
                u32x4 vb[kNS];
#pragma unroll
                for (int pi = 0; pi < kNS; ++pi)
                    vb[pi] = *reinterpret_cast<const u32x4*>(xrow(vp, kPieceRow, pi, ct) + 32 * k + 8 * q);
                o = mma(cur.pa[k], vb, o);
            }
            float* orow = p.out + ((long long)(tc + 16 * W + 4 * q) * H + h) * kDv + col0 + 16 * ct + r;
            if (nt == kC) {
#pragma unroll
                for (int i = 0; i < 4; ++i) orow[(long long)i * H * kDv] = o[i];
            } else {
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    if (16 * W + 4 * q + i < nt) orow[(long long)i * H * kDv] = o[i];
            }
        }
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            Row8<In> kb[2];
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                const In* src = kt + (32 * W + 16 * u + r) * L::kKt + 32 * k + 8 * q;
                if constexpr (sizeof(In) == 2) {
                    kb[u].v = *reinterpret_cast<const u32x4*>(src);
                } else {
                    kb[u].a = *reinterpret_cast<const f32x4*>(src);
                    kb[u].b = *reinterpret_cast<const f32x4*>(src + 4);
                }
            }
#pragma unroll
            for (int ct = 0; ct < kCT; ++ct) {
                u32x4 qb[kNS];
#pragma unroll
                for (int pi = 0; pi < kNS; ++pi)
                    qb[pi] = *reinterpret_cast<const u32x4*>(xrow(vq, kPieceRow, pi, ct) + 32 * k + 8 * q);
#pragma unroll
                for (int u = 0; u < 2; ++u) {
                    if (k == 0)
#pragma unroll
                        for (int i = 0; i < 4; ++i) st[u][ct][i] *= glast;
                    u32x4 op[KP];
                    kb[u].pieces(op);
                    st[u][ct] = mma(op, qb, st[u][ct]);
                }
            }
        }
    };
    Ahead other;
    for (int c = 0; c < nch; c += 2) {
        step(c, cur, other);
        if (c + 1 < nch) step(c + 1, other, cur);
    }
#pragma unroll
    for (int u = 0; u < 2; ++u)
#pragma unroll
        for (int ct = 0; ct < kCT; ++ct)
#pragma unroll
            for (int i = 0; i < 4; ++i) Sg[(32 * W + 16 * u + 4 * q + i) * kDv + 16 * ct + r] = st[u][ct][i];
}

// 86 KiB of LDS (bf16 inputs; 103 KiB for fp32): one workgroup per CU, one wave per SIMD with 512 registers.
template <typename In>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1))) void delta_chunk_scan(DeltaArgs p) {
    extern __shared__ __align__(16) char lds[];
    // All slices of one (sequence, head) get ids congruent mod 8: with round-robin dispatch over the XCDs they
    // share one L2, where their common K / Q / T / P reads hit.
    const int id = blockIdx.x;
    const int slice = (id >> 3) % kSlices;
    const int pair = (id / (8 * kSlices)) * 8 + (id & 7);
    if (pair >= p.n_pairs) return;
    const int s = pair / p.H, h = pair % p.H;
    switch (threadIdx.x >> 6) {
        case 0: scan_wave<In, 0>(p, lds, s, h, slice); break;
        case 1: scan_wave<In, 1>(p, lds, s, h, slice); break;
        case 2: scan_wave<In, 2>(p, lds, s, h, slice); break;
        default: scan_wave<In, 3>(p, lds, s, h, slice); break;
    }
}

template <typename In>
int launch(const DeltaArgs& a, int total_chunks, hipStream_t stream) {
    if (total_chunks > 0) {
        hipLaunchKernelGGL(delta_chunk_prep<In>, dim3(total_chunks, a.H), dim3(256), 0, stream, a);
        if (int rc = check_launch("delta_chunk_prep")) return rc;
    }
    const int groups = (a.n_pairs + 7) / 8;
    if constexpr (sizeof(In) == 2) {
        return launch_scan_cols(a, groups * 8 * kSlices, stream);
    } else {
        const size_t lds = ScanLayout<In>::bytes;
        if (int rc = allow_dynamic_lds((const void*)delta_chunk_scan<In>, lds)) return rc;
        hipLaunchKernelGGL(delta_chunk_scan<In>, dim3(groups * 8 * kSlices), dim3(256), lds, stream, a);
        return check_launch("delta_chunk_scan");
    }
}

}  // namespace
}  // namespace rk

using namespace rk;

extern "C" {

size_t rk_gated_delta_workspace_bytes(int total_chunks, int H) {
    if (total_chunks < 0 || H < 1) return 0;
    return (size_t)total_chunks * H * kChunkFloats * sizeof(float);
}

int rk_gated_delta_chunked(float* out, float* S, long long s_stride, const void* q, const void* k, const void* v,
                           int in_dtype, const float* beta, const float* g, const int32_t* cu_seqlens,
                           const int32_t* cu_chunks, const int32_t* seq_index, int n_seqs, int total_chunks, int H,
                           int dk, int dv, void* workspace, size_t workspace_bytes, void* stream) {
    if (!out || !S || !q || !k || !v || !beta || !g || !cu_seqlens || !cu_chunks)
        return fail(RK_ERR_ARG, "rk_gated_delta_chunked: null pointer");
    if (n_seqs < 1 || H < 1 || total_chunks < 0 || (long long)n_seqs * H > (1LL << 24))
        return fail(RK_ERR_ARG, "rk_gated_delta_chunked: n_seqs %d H %d total_chunks %d", n_seqs, H, total_chunks);
    if (dk != kDk || dv != kDv)
        return fail(RK_ERR_UNSUPPORTED, "rk_gated_delta_chunked: dk %d dv %d (built for 128 x 128)", dk, dv);
    if (in_dtype != RK_F32 && in_dtype != RK_BF16)
        return fail(RK_ERR_UNSUPPORTED, "rk_gated_delta_chunked: input dtype %d", in_dtype);
    if (s_stride < (long long)H * dk * dv)
        return fail(RK_ERR_ARG, "rk_gated_delta_chunked: state stride %lld < H * dk * dv", s_stride);
    const size_t need = rk_gated_delta_workspace_bytes(total_chunks, H);
    if (need && (!workspace || workspace_bytes < need))
        return fail(RK_ERR_WORKSPACE, "rk_gated_delta_chunked: workspace %zu bytes, need %zu", workspace_bytes, need);
    DeltaArgs a;
    a.out = out; a.S = S; a.q = q; a.k = k; a.v = v; a.beta = beta; a.g = g;
    a.cu = cu_seqlens; a.cu_chunks = cu_chunks; a.seq_index = seq_index;
    a.ws = static_cast<float*>(workspace); a.s_stride = s_stride;
    a.n_seqs = n_seqs; a.H = H; a.n_pairs = n_seqs * H;
    hipStream_t st = static_cast<hipStream_t>(stream);
    return in_dtype == RK_BF16 ? launch<uint16_t>(a, total_chunks, st) : launch<float>(a, total_chunks, st);
}

}  // extern "C"
