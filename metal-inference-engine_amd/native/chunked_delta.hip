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
// Two kernels:
//   delta_chunk_prep  one workgroup per (chunk, head), all chunks in parallel: beta, G (summed in fp64 and rounded
//                     once, as torch's CPU cumsum of fp32 accumulates in double), exp(G), exp(G_last - G); the Gram
//                     matrix K K^T on MFMA; T by blocked inversion of the unit lower triangular matrix (16 x 16
//                     diagonal blocks by substitution, off-diagonal blocks by fp32 MFMA products in three levels).
//                     Writes T's ten lower 16 x 16 tiles and the coefficient rows to the workspace.
//   delta_chunk_scan  one workgroup per (sequence, head, 16-column slice of S): the columns of S evolve
//                     independently, so the serial pass over a sequence's chunks runs 8 workgroups wide per head.
//                     Wave w owns token rows 16w..16w+15 of the chunk and state rows 32w..32w+31; the three
//                     exchanges per chunk (state pieces, Y, vn) go through LDS behind LDS-only barriers, so the next
//                     chunk's global loads stay in flight across them.
// Precision: every product with an fp32 operand (S, Y, vn, T, P, fp32 inputs) runs on bf16 MFMA with that operand
// split exactly into three bf16 pieces (truncation) and the piece products of order >= 2^-16 kept; bf16 inputs are
// exact operands. Products are therefore exact to ~2^-20 relative and accumulate in fp32: fp32-level results.
#include "rk_device.h"
#include "rk_internal.h"

namespace rk {
namespace {

constexpr int kC = 64;                       // tokens per chunk
constexpr int kDk = 128, kDv = 128;
constexpr int kCols = 16;                    // state columns per scan workgroup
constexpr int kSlices = kDv / kCols;         // 8
constexpr int kNS = 3;                       // bf16 pieces of an fp32 operand
constexpr int kTiles = 10;                   // lower 16 x 16 tiles of a 64 x 64 matrix
constexpr int kCoefRows = 4;                 // beta, G, exp(G), exp(G_last - G)
constexpr int kChunkFloats = kTiles * 256 + kCoefRows * kC;
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
    float* ws;                  // [total_chunks, H, kChunkFloats]
    long long s_stride;
    int n_seqs, H, n_pairs;
};

// ---- operands: 8 consecutive elements of one row per lane, as bf16 pieces
__device__ __forceinline__ uint32_t mask_if(bool keep) { return keep ? 0xffffffffu : 0u; }
__device__ __forceinline__ float to_f32(uint16_t x) { return __uint_as_float((uint32_t)x << 16); }
__device__ __forceinline__ float to_f32(float x) { return x; }
// Index of lower tile (a, b), b <= a, of a 64 x 64 matrix stored as its ten 16 x 16 lower tiles.
__host__ __device__ constexpr int tile_of(int a, int b) { return a * (a + 1) / 2 + b; }

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

// Workgroup barrier ordering LDS only: outstanding global loads are not waited for.
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
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

// =====================================================================================================================
// Phase 1: per-chunk coefficients and T
// =====================================================================================================================
template <typename In>
__global__ __launch_bounds__(256) void delta_chunk_prep(DeltaArgs p) {
    __shared__ float sA[kC][kC + 1];       // -beta_i (K K^T)_ij D_ij, strictly lower (read only below the diagonal)
    __shared__ float sT[kC][kC + 1];       // T, lower triangle
    __shared__ float sTmp[4][16][17];      // per-wave 16 x 16 scratch

    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, q = lane >> 4, r = lane & 15;
    const int gc = blockIdx.x, h = blockIdx.y, H = p.H;
    const int s = seq_of_chunk(p, gc);
    const int t0 = p.cu[s] + (gc - p.cu_chunks[s]) * kC;
    const int nt = min(kC, p.cu[s + 1] - t0);
    if (nt <= 0) return;                  // offsets inconsistent with cu_chunks: nothing of this chunk is read
    const In* K = static_cast<const In*>(p.k);

    // K rows of row tile w (A operand); issued first
    Row8<In> ka[4];
    {
        const int t = 16 * w + r;
        const long long off = ((long long)(t0 + min(t, nt - 1)) * H + h) * kDk + 8 * q;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            ka[k].load(K + off + 32 * k);
            ka[k].keep(mask_if(t < nt));
        }
    }

    // beta and the cumulative log-decay of the chunk, one token per lane (every wave keeps its own copy)
    const bool live = lane < nt;
    const long long ti = (long long)(t0 + min(lane, nt - 1)) * H + h;
    const float bl = live ? p.beta[ti] : 0.f;
    double acc = live ? (double)p.g[ti] : 0.0;
#pragma unroll
    for (int off = 1; off < kC; off <<= 1) {
        const double y = __shfl_up(acc, off);
        if (lane >= off) acc += y;
    }
    const float G = (float)acc;

    // A0 tiles (w, b), b <= w: -beta_i * (K K^T)_ij * exp(G_i - G_j) for j < i
    float Gi[4], bi[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        Gi[i] = __shfl(G, 16 * w + 4 * q + i);
        bi[i] = __shfl(bl, 16 * w + 4 * q + i);
    }
    for (int b = 0; b <= w; ++b) {
        const int t = 16 * b + r;
        const long long off = ((long long)(t0 + min(t, nt - 1)) * H + h) * kDk + 8 * q;
        f32x4 kk = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            Row8<In> kb;
            kb.load(K + off + 32 * k);
            kb.keep(mask_if(t < nt));
            u32x4 pa[Row8<In>::KP], pb[Row8<In>::KP];
            ka[k].pieces(pa);
            kb.pieces(pb);
            kk = mma(pa, pb, kk);
        }
        const float Gj = __shfl(G, t);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int row = 16 * w + 4 * q + i;
            sA[row][t] = t < row ? -(bi[i] * kk[i]) * expf(Gi[i] - Gj) : 0.f;
        }
    }
    lds_barrier();

    // diagonal block w of T = (I - A0)^-1: lane r keeps column r, rows by forward substitution
    {
        float x[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            float a = i == r ? 1.f : 0.f;
#pragma unroll
            for (int m = 0; m < i; ++m) a = fmaf(sA[16 * w + i][16 * w + m], x[m], a);
            x[i] = a;
        }
        if (q == 0)
#pragma unroll
            for (int i = 0; i < 16; ++i) sT[16 * w + i][16 * w + r] = x[i];
    }
    lds_barrier();

    // off-diagonal blocks, one level of distance d = w - j at a time: T_wj = T_ww * sum_{k=j}^{w-1} A0_wk T_kj
    for (int d = 1; d < 4; ++d) {
        if (w >= d) {
            const int j = w - d;
            f32x4 t = {0.f, 0.f, 0.f, 0.f};
            for (int kb = j; kb < w; ++kb)
#pragma unroll
                for (int ks = 0; ks < 4; ++ks)
                    t = mfma_f32(sA[16 * w + r][16 * kb + 4 * ks + q], sT[16 * kb + 4 * ks + q][16 * j + r], t);
#pragma unroll
            for (int i = 0; i < 4; ++i) sTmp[w][4 * q + i][r] = t[i];
            wave_lds_sync();
            f32x4 u = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int ks = 0; ks < 4; ++ks)
                u = mfma_f32(sT[16 * w + r][16 * w + 4 * ks + q], sTmp[w][4 * ks + q][r], u);
#pragma unroll
            for (int i = 0; i < 4; ++i) sT[16 * w + 4 * q + i][16 * j + r] = u[i];
        }
        lds_barrier();
    }

    float* wsc = p.ws + ((size_t)gc * H + h) * kChunkFloats;
#pragma unroll
    for (int tile = 0; tile < kTiles; ++tile) {
        const int a = tile < 1 ? 0 : (tile < 3 ? 1 : (tile < 6 ? 2 : 3));
        const int b = tile - tile_of(a, 0);
        const int e = threadIdx.x;
        wsc[tile * 256 + e] = sT[16 * a + (e >> 4)][16 * b + (e & 15)];
    }
    if (w == 0) {
        const float Glast = __shfl(G, kC - 1);
        float* cf = wsc + kTiles * 256;
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
    static constexpr int kKr = kDk + (sizeof(In) == 2 ? 8 : 4);   // row stride of staged K rows [token][dk]
    static constexpr int kKt = kC + (sizeof(In) == 2 ? 8 : 4);    // row stride of staged K^T [dk][token]
    static constexpr size_t sp = 0;                                               // state pieces
    static constexpr size_t yp = sp + (size_t)kNS * kCols * kStateRow * 2;        // Y pieces
    static constexpr size_t vp = yp + (size_t)kNS * kCols * kPieceRow * 2;        // vn pieces
    static constexpr size_t vq = vp + (size_t)kNS * kCols * kPieceRow * 2;        // exp(G_last - G) vn pieces
    static constexpr size_t kr = vq + (size_t)kNS * kCols * kPieceRow * 2;        // K rows
    static constexpr size_t kt = kr + (size_t)kC * kKr * sizeof(In);              // K^T
    static constexpr size_t bytes = kt + (size_t)kDk * kKt * sizeof(In);
};

template <typename In, int W>
__device__ __forceinline__ void scan_wave(const DeltaArgs& p, char* lds, int s, int h, int slice) {
    using L = ScanLayout<In>;
    constexpr int KP = Row8<In>::KP;
    constexpr int KS = (W >> 1) + 1;      // 32-token k-steps of T and P below the diagonal for row tile W
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
    In* kr = reinterpret_cast<In*>(lds + L::kr);
    In* kt = reinterpret_cast<In*>(lds + L::kt);

    // state rows 32W + 16u + 4q + i, column col0 + r (MFMA accumulator layout of the update)
    f32x4 st[2];
#pragma unroll
    for (int u = 0; u < 2; ++u)
#pragma unroll
        for (int i = 0; i < 4; ++i) st[u][i] = Sg[(32 * W + 16 * u + 4 * q + i) * kDv + r];

    // K and Q rows 16W + r of chunk c (columns 32k + 8q .. +7), zero past the sequence's end
    auto load_rows = [&](int c, Row8<In> (&kk)[4], Row8<In> (&qq)[4]) {
        const int nt = min(kC, Tn - c * kC);
        const int t = 16 * W + r;
        const long long off = ((long long)(T0 + c * kC + min(t, nt - 1)) * H + h) * kDk + 8 * q;
        const uint32_t m = mask_if(t < nt);
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            kk[k].load(Kg + off + 32 * k);
            qq[k].load(Qg + off + 32 * k);
            kk[k].keep(m);
            qq[k].keep(m);
        }
    };
    Row8<In> ka[4], qa[4];
    load_rows(0, ka, qa);

    for (int c = 0; c < nch; ++c) {
        const int nt = min(kC, Tn - c * kC);
        const int tc = T0 + c * kC;
        const float* wsc = p.ws + ((size_t)(gc0 + c) * H + h) * kChunkFloats;
        const float* cf = wsc + kTiles * 256;

        // ---- loads of this chunk's T tiles, values and coefficients; next chunk's K / Q rows
        float tv[KS][8];
#pragma unroll
        for (int k = 0; k < KS; ++k) {
            const int b = 2 * k + (q >> 1);
            const int bc = b <= W ? b : W;
            const float* tp = wsc + tile_of(W, bc) * 256 + r * 16 + 8 * (q & 1);
            const f32x4 lo = *reinterpret_cast<const f32x4*>(tp);
            const f32x4 hi = *reinterpret_cast<const f32x4*>(tp + 4);
            const uint32_t m = mask_if(b <= W);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                tv[k][e] = __uint_as_float(__float_as_uint(lo[e]) & m);
                tv[k][4 + e] = __uint_as_float(__float_as_uint(hi[e]) & m);
            }
        }
        float vv[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int t = min(16 * W + 4 * q + i, nt - 1);
            vv[i] = to_f32(Vg[((long long)(tc + t) * H + h) * kDv + col0 + r]);
        }
        const f32x4 beta4 = *reinterpret_cast<const f32x4*>(cf + 16 * W + 4 * q);
        const f32x4 eg4 = *reinterpret_cast<const f32x4*>(cf + 2 * kC + 16 * W + 4 * q);
        const f32x4 egr4 = *reinterpret_cast<const f32x4*>(cf + 3 * kC + 16 * W + 4 * q);
        const float Gt = cf[kC + 16 * W + r];
        f32x4 Gq[W + 1];
#pragma unroll
        for (int b = 0; b <= W; ++b) Gq[b] = *reinterpret_cast<const f32x4*>(cf + kC + 16 * b + 4 * q);
        const float glast = cf[2 * kC + kC - 1];
        Row8<In> kn[4], qn[4];
        load_rows(c + 1 < nch ? c + 1 : c, kn, qn);

        // ---- A1: state pieces -> LDS [piece][column][dk]
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const float x[4] = {st[u][0], st[u][1], st[u][2], st[u][3]};
            u32x2 pc[kNS];
            split4(x, pc);
#pragma unroll
            for (int pi = 0; pi < kNS; ++pi)
                *reinterpret_cast<u32x2*>(sp + (pi * kCols + r) * kStateRow + 32 * W + 16 * u + 4 * q) = pc[pi];
        }
        lds_barrier();

        // ---- A2: X = K S and Q S for row tile W; Y = beta (V - e^G X) -> LDS; K rows and K^T -> LDS
        f32x4 x = {0.f, 0.f, 0.f, 0.f}, qs = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            u32x4 sb[kNS];
#pragma unroll
            for (int pi = 0; pi < kNS; ++pi)
                sb[pi] = *reinterpret_cast<const u32x4*>(sp + (pi * kCols + r) * kStateRow + 32 * k + 8 * q);
            u32x4 pa[KP];
            ka[k].pieces(pa);
            x = mma(pa, sb, x);
            qa[k].pieces(pa);
            qs = mma(pa, sb, qs);
        }
        {
            float y[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) y[i] = beta4[i] * (vv[i] - eg4[i] * x[i]);
            u32x2 pc[kNS];
            split4(y, pc);
#pragma unroll
            for (int pi = 0; pi < kNS; ++pi)
                *reinterpret_cast<u32x2*>(yp + (pi * kCols + r) * kPieceRow + 16 * W + 4 * q) = pc[pi];
        }
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            In* dst = kr + (16 * W + r) * L::kKr + 32 * k + 8 * q;
            if constexpr (sizeof(In) == 2) {
                *reinterpret_cast<u32x4*>(dst) = ka[k].v;
            } else {
                *reinterpret_cast<f32x4*>(dst) = ka[k].a;
                *reinterpret_cast<f32x4*>(dst + 4) = ka[k].b;
            }
#pragma unroll
            for (int e = 0; e < 8; ++e) kt[(32 * k + 8 * q + e) * L::kKt + 16 * W + r] = ka[k].raw(e);
        }
        lds_barrier();

        // ---- C: vn = T Y (row tile W); P^T tiles; vn and e^{G_last-G} vn -> LDS
        f32x4 vn = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int k = 0; k < KS; ++k) {
            u32x4 ta[kNS], yb[kNS];
            split8(tv[k], ta);
#pragma unroll
            for (int pi = 0; pi < kNS; ++pi)
                yb[pi] = *reinterpret_cast<const u32x4*>(yp + (pi * kCols + r) * kPieceRow + 32 * k + 8 * q);
            vn = mma(ta, yb, vn);
        }
        // P^T tile b: rows t' = 16b + 4q + i, column t = 16W + r; kept where t' <= t
        float pt[2 * KS][4];
#pragma unroll
        for (int b = 0; b < 2 * KS; ++b) {
            if (b <= W) {
                f32x4 a = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    Row8<In> kb;
                    const In* src = kr + (16 * b + r) * L::kKr + 32 * k + 8 * q;
                    if constexpr (sizeof(In) == 2) {
                        kb.v = *reinterpret_cast<const u32x4*>(src);
                    } else {
                        kb.a = *reinterpret_cast<const f32x4*>(src);
                        kb.b = *reinterpret_cast<const f32x4*>(src + 4);
                    }
                    u32x4 pa[KP], pb[KP];
                    kb.pieces(pa);
                    qa[k].pieces(pb);
                    a = mma(pa, pb, a);
                }
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int tp = 16 * b + 4 * q + i;
                    pt[b][i] = tp <= 16 * W + r ? a[i] * expf(Gt - Gq[b][i]) : 0.f;
                }
            } else {
#pragma unroll
                for (int i = 0; i < 4; ++i) pt[b][i] = 0.f;
            }
        }
        {
            float a4[4], b4[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                a4[i] = vn[i];
                b4[i] = egr4[i] * vn[i];
            }
            u32x2 pa[kNS], pb[kNS];
            split4(a4, pa);
            split4(b4, pb);
#pragma unroll
            for (int pi = 0; pi < kNS; ++pi) {
                *reinterpret_cast<u32x2*>(vp + (pi * kCols + r) * kPieceRow + 16 * W + 4 * q) = pa[pi];
                *reinterpret_cast<u32x2*>(vq + (pi * kCols + r) * kPieceRow + 16 * W + 4 * q) = pb[pi];
            }
        }
        lds_barrier();

        // ---- D: o = e^G Q S + P vn (P as A operand in the accumulator's k order); state update
        f32x4 o;
#pragma unroll
        for (int i = 0; i < 4; ++i) o[i] = eg4[i] * qs[i];
#pragma unroll
        for (int k = 0; k < KS; ++k) {
            const float pv[8] = {pt[2 * k][0], pt[2 * k][1], pt[2 * k][2], pt[2 * k][3],
                                 pt[2 * k + 1][0], pt[2 * k + 1][1], pt[2 * k + 1][2], pt[2 * k + 1][3]};
            u32x4 pa[kNS], vb[kNS];
            split8(pv, pa);
#pragma unroll
            for (int pi = 0; pi < kNS; ++pi) {
                const uint16_t* base = vp + (pi * kCols + r) * kPieceRow + 32 * k + 4 * q;
                const u32x2 lo = *reinterpret_cast<const u32x2*>(base);
                const u32x2 hi = *reinterpret_cast<const u32x2*>(base + 16);
                vb[pi] = (u32x4){lo[0], lo[1], hi[0], hi[1]};
            }
            o = mma(pa, vb, o);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int t = 16 * W + 4 * q + i;
            if (t < nt) p.out[((long long)(tc + t) * H + h) * kDv + col0 + r] = o[i];
        }
        u32x4 qb[2][kNS];
#pragma unroll
        for (int k = 0; k < 2; ++k)
#pragma unroll
            for (int pi = 0; pi < kNS; ++pi)
                qb[k][pi] = *reinterpret_cast<const u32x4*>(vq + (pi * kCols + r) * kPieceRow + 32 * k + 8 * q);
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            f32x4 a;
#pragma unroll
            for (int i = 0; i < 4; ++i) a[i] = glast * st[u][i];
#pragma unroll
            for (int k = 0; k < 2; ++k) {
                Row8<In> kb;
                const In* src = kt + (32 * W + 16 * u + r) * L::kKt + 32 * k + 8 * q;
                if constexpr (sizeof(In) == 2) {
                    kb.v = *reinterpret_cast<const u32x4*>(src);
                } else {
                    kb.a = *reinterpret_cast<const f32x4*>(src);
                    kb.b = *reinterpret_cast<const f32x4*>(src + 4);
                }
                u32x4 pa[KP];
                kb.pieces(pa);
                a = mma(pa, qb[k], a);
            }
            st[u] = a;
        }
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            ka[k] = kn[k];
            qa[k] = qn[k];
        }
    }
#pragma unroll
    for (int u = 0; u < 2; ++u)
#pragma unroll
        for (int i = 0; i < 4; ++i) Sg[(32 * W + 16 * u + 4 * q + i) * kDv + r] = st[u][i];
}

// bf16 inputs: 68 KiB of LDS, two workgroups per CU (256 registers per lane); fp32 inputs stage K in fp32: one.
template <typename In, int WPE = sizeof(In) == 2 ? 2 : 1>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(WPE, WPE))) void delta_chunk_scan(DeltaArgs p) {
    extern __shared__ __align__(16) char lds[];
    // All 8 slices of one (sequence, head) get ids congruent mod 8: with round-robin dispatch over the XCDs they
    // share one L2, where their common K / Q / T reads hit.
    const int id = blockIdx.x;
    const int slice = (id >> 3) & (kSlices - 1);
    const int pair = ((id >> 6) << 3) | (id & 7);
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
    const size_t lds = ScanLayout<In>::bytes;
    if (int rc = allow_dynamic_lds((const void*)delta_chunk_scan<In>, lds)) return rc;
    const int groups = (a.n_pairs + 7) / 8;
    hipLaunchKernelGGL(delta_chunk_scan<In>, dim3(groups * 8 * kSlices), dim3(256), lds, stream, a);
    return check_launch("delta_chunk_scan");
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
