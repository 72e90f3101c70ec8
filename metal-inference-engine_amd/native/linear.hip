// Decode-time linears (a few rows of activations times a bf16 / INT8 / INT4 weight matrix), gfx950.
//
// Semantics (reference): MetalBackend.linear / _qlinear for M <= 32 rows (src/backend/metal.py:59-133; kernels
// matvec.metal / qmatvec.metal): y [M, N] = x [M, K] (fp32) @ W^T, W [N, K] either bf16 or block-quantized
// (src/quant.py:1-10, 45-56: blocks of 32 weights along a row share fp16 parameters; INT8 w = q * scale, q int8;
// INT4 w = q * scale + min, q in 0..15, element 2j in the low nibble of byte j, 2j+1 in the high nibble), then
// y += bias, y += residual, fp32 throughout.
//
// Design: y^T [N, M] = W [N, K] x^T [K, M] on MFMA (v_mfma_f32_16x16x32_bf16), a 16-row tile of W against the (up
// to 16) activation rows as the 16 columns. Weights are exact bf16 operands (bf16 as stored; INT8 and INT4 codes are
// small integers), activations enter as their exact three-piece bf16 split (x = hi + mid + lo), so every product is
// exact and accumulates in fp32: fp32-level results (the VALU alternative tops out near 2.5 TB/s of INT4 at 8 rows).
// One MFMA k-extent is one quantization block, so a block's dot products come out of three MFMAs and its scale (and
// min, times the block's activation sum) is applied to them on the VALU.
// Work: workgroups of 4 waves take 64 rows x one K-split of NB blocks (16 or 32), so every matrix gives hundreds of
// workgroups (a decode step's 2048-row projections too) and each wave requests all its weights at once: no loop
// over K, no per-tile barrier, whole K-splits in flight. Splits of one row block are added by the last workgroup to
// finish (see linear_rows_kernel).
#include "rk_device.h"
#include "rk_internal.h"

namespace rk {
namespace {

constexpr int kQB = 32;            // weights per quantization block = the MFMA k-extent
constexpr int kCols = 16;          // activation rows per launch (MFMA columns)

struct LinArgs {
    float* y;                      // [M, N] fp32
    const float* x;                // [M, K] fp32
    const void* w;                 // bf16 [N, K] | int8 [N, K] | uint8 [N, K / 2]
    const uint16_t* scales;        // fp16 [N, K / 32] (quantized types)
    const uint16_t* mins;          // fp16 [N, K / 32] (INT4)
    const float* bias;             // [N] or null
    const float* res;              // [M, N] or null
    float* part;                   // [S, M, N] partial sums (S > 1)
    uint32_t* cnt;                 // [row blocks] arrival counters, zero between calls (S > 1)
    int M, N, K, S;
};

template <int WT> struct WTraits;
// DPB: dwords of one lane's MFMA slots of one block (8 weights); BPB: bytes of one block of one row
template <> struct WTraits<RK_W_BF16> { static constexpr int DPB = 4; static constexpr int BPB = 64; };
template <> struct WTraits<RK_W_INT8> { static constexpr int DPB = 2; static constexpr int BPB = 32; };
template <> struct WTraits<RK_W_INT4> { static constexpr int DPB = 1; static constexpr int BPB = 16; };

__device__ __forceinline__ float half_to_f32(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }

// 8 weights (one lane's MFMA slots of one block) as bf16 bits, from the raw bytes
template <int WT> struct Slot;
template <> struct Slot<RK_W_BF16> {
    u32x4 v;
    __device__ __forceinline__ void load(const uint8_t* p) { v = *reinterpret_cast<const u32x4*>(p); }
    __device__ __forceinline__ u32x4 bf16() const { return v; }
};
template <> struct Slot<RK_W_INT8> {
    u32x2 v;
    __device__ __forceinline__ void load(const uint8_t* p) { v = *reinterpret_cast<const u32x2*>(p); }
    __device__ __forceinline__ u32x4 bf16() const {
        // q in [-127, 127]: exact in bf16; the top half of the fp32 value is its bf16 pattern
        u32x4 o;
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int e = 0; e < 2; ++e) {
                const uint32_t w = v[h];
                const float f0 = (float)(int)__builtin_amdgcn_sbfe(w, 16 * e, 8);
                const float f1 = (float)(int)__builtin_amdgcn_sbfe(w, 16 * e + 8, 8);
                o[2 * h + e] = pack_hi2(__float_as_uint(f0), __float_as_uint(f1));
            }
        return o;
    }
};
template <> struct Slot<RK_W_INT4> {
    uint32_t v;
    __device__ __forceinline__ void load(const uint8_t* p) { v = *reinterpret_cast<const uint32_t*>(p); }
    __device__ __forceinline__ u32x4 bf16() const {
        // byte j holds elements 2j (low nibble) and 2j+1 (high nibble); q in 0..15 is exact in bf16
        u32x4 o;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const float f0 = (float)__builtin_amdgcn_ubfe(v, 8 * j, 4);
            const float f1 = (float)__builtin_amdgcn_ubfe(v, 8 * j + 4, 4);
            o[j] = pack_hi2(__float_as_uint(f0), __float_as_uint(f1));
        }
        return o;
    }
};

constexpr int kRows = 64;                  // weight rows per workgroup: 4 waves x one 16-row MFMA tile

// Workgroup (row block rb, K-split sp): rows rb*64 .. +63, blocks sp*NB .. +NB-1. Everything it reads is requested
// first (activations, then the rows' scales / mins, then all NB blocks of this lane's weights, so the staging wait
// never includes the weights); the activations' pieces, block sums and the parameters go to LDS behind one barrier;
// then the NB blocks of MFMAs. With S > 1 splits the workgroup stores its partial sums (device-coherent stores),
// counts itself in for its row block, and the last to arrive adds the S partials in split order (deterministic,
// whatever the arrival order), the bias and the residual, and writes y.
template <int WT, int COLS, int NB>
__global__ __launch_bounds__(256) void linear_rows_kernel(LinArgs a) {
    using TR = WTraits<WT>;
    constexpr int KG = 4 * NB;                     // 8-element k-groups of the workgroup's K-range
    constexpr bool QUANT = WT != RK_W_BF16;
    constexpr int XI = COLS * KG / 256;            // staging items (8 activations each) per thread
    constexpr int PB = NB / 4;                     // parameter blocks per thread (4 threads per row)
    __shared__ __align__(16) u32x4 xs[3 * KG * COLS];
    __shared__ float xsum[WT == RK_W_INT4 ? COLS * KG : 1];
    __shared__ __align__(16) float ss[QUANT ? NB * kRows : 4];
    __shared__ __align__(16) float ms[WT == RK_W_INT4 ? NB * kRows : 4];
    __shared__ int is_last;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int r = lane & 15, grp = lane >> 4;
    const int rb = blockIdx.x / a.S, sp = blockIdx.x % a.S;
    const int row0 = rb * kRows;
    const int nblk = a.K / kQB;
    const int b0 = sp * NB;
    const int nb = min(NB, nblk - b0);             // blocks of this workgroup (>= 1)

    // ---- requests: activations, parameters, weights
    f32x4 xa[XI], xb[XI];
#pragma unroll
    for (int u = 0; u < XI; ++u) {
        const int i = tid + 256 * u;
        const int col = i % COLS, kg = i / COLS;
        const bool ok = col < a.M && kg < 4 * nb;
        const float* p = a.x + (size_t)min(col, a.M - 1) * a.K + (size_t)kQB * b0 + 8 * min(kg, 4 * nb - 1);
        const f32x4 v0 = *reinterpret_cast<const f32x4*>(p);
        const f32x4 v1 = *reinterpret_cast<const f32x4*>(p + 4);
        const f32x4 z = {0.f, 0.f, 0.f, 0.f};
        xa[u] = ok ? v0 : z;
        xb[u] = ok ? v1 : z;
    }
    const int prow = tid % kRows, pq = tid / kRows;            // parameters: row prow, blocks pq*PB .. +PB-1
    uint16_t sc16[QUANT ? PB : 1], mn16[WT == RK_W_INT4 ? PB : 1];
    if constexpr (QUANT) {
        const size_t base = (size_t)min(row0 + prow, a.N - 1) * nblk + b0;
#pragma unroll
        for (int e = 0; e < PB; ++e) {
            const int j = min(pq * PB + e, nb - 1);
            sc16[e] = a.scales[base + j];
            if constexpr (WT == RK_W_INT4) mn16[e] = a.mins[base + j];
        }
    }
    const uint8_t* wrow = static_cast<const uint8_t*>(a.w) +
                          (size_t)min(row0 + 16 * wave + r, a.N - 1) * ((size_t)a.K * TR::BPB / kQB) +
                          (size_t)b0 * TR::BPB + grp * (TR::BPB / 4);
    Slot<WT> wv[NB];
#pragma unroll
    for (int j = 0; j < NB; ++j) wv[j].load(wrow + (size_t)min(j, nb - 1) * TR::BPB);

    // ---- staging: activation pieces [3][KG][COLS], block sums [COLS][KG], parameters [NB][64 rows]
#pragma unroll
    for (int u = 0; u < XI; ++u) {
        const int i = tid + 256 * u;
        const int col = i % COLS, kg = i / COLS;
        const float v[8] = {xa[u][0], xa[u][1], xa[u][2], xa[u][3], xb[u][0], xb[u][1], xb[u][2], xb[u][3]};
        u32x4 pc[3];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const Split3 s0 = split3(v[2 * j]), s1 = split3(v[2 * j + 1]);
            pc[0][j] = pack_hi2(s0.hi, s1.hi);
            pc[1][j] = pack_hi2(s0.mid, s1.mid);
            pc[2][j] = pack_hi2(s0.lo, s1.lo);
        }
#pragma unroll
        for (int p = 0; p < 3; ++p) xs[(p * KG + kg) * COLS + col] = pc[p];
        if constexpr (WT == RK_W_INT4) {
            float sum = 0.0f;
#pragma unroll
            for (int e = 0; e < 8; ++e) sum += v[e];
            xsum[col * KG + kg] = sum;
        }
    }
    if constexpr (QUANT) {
#pragma unroll
        for (int e = 0; e < PB; ++e) {
            ss[(pq * PB + e) * kRows + prow] = half_to_f32(sc16[e]);
            if constexpr (WT == RK_W_INT4) ms[(pq * PB + e) * kRows + prow] = half_to_f32(mn16[e]);
        }
    }
    __syncthreads();

    // ---- MFMAs: block j of this workgroup = MFMA k-extent j; accumulator rows 16 wave + 4 grp + i, column r
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    const u32x4 zero4 = {0u, 0u, 0u, 0u};
    const int lr = 16 * wave + 4 * grp;
#pragma unroll
    for (int j = 0; j < NB; ++j) {
        if (j < nb) {                               // uniform: the last split may hold fewer blocks
        const int kg = 4 * j + grp;                 // this lane's k-group: k = 32 (b0 + j) + 8 grp .. + 7
        const bool col_ok = COLS == 16 || r < COLS;
        const int cr = COLS == 16 ? r : (r & (COLS - 1));
        const u32x4 p0 = col_ok ? xs[(0 * KG + kg) * COLS + cr] : zero4;
        const u32x4 p1 = col_ok ? xs[(1 * KG + kg) * COLS + cr] : zero4;
        const u32x4 p2 = col_ok ? xs[(2 * KG + kg) * COLS + cr] : zero4;
        const u32x4 av = wv[j].bf16();
        if constexpr (QUANT) {
            f32x4 d = mfma16x16x32(av, p0, (f32x4){0.f, 0.f, 0.f, 0.f});
            d = mfma16x16x32(av, p1, d);
            d = mfma16x16x32(av, p2, d);
            const f32x4 sc = *reinterpret_cast<const f32x4*>(&ss[j * kRows + lr]);
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[i] = fmaf(sc[i], d[i], acc[i]);
            if constexpr (WT == RK_W_INT4) {
                // block sum of activation column r: four k-group partials, in order
                const float bsum = col_ok ? ((xsum[cr * KG + 4 * j] + xsum[cr * KG + 4 * j + 1]) +
                                             xsum[cr * KG + 4 * j + 2]) + xsum[cr * KG + 4 * j + 3]
                                          : 0.0f;
                const f32x4 mn = *reinterpret_cast<const f32x4*>(&ms[j * kRows + lr]);
#pragma unroll
                for (int i = 0; i < 4; ++i) acc[i] = fmaf(mn[i], bsum, acc[i]);
            }
        } else {
            acc = mfma16x16x32(av, p0, acc);
            acc = mfma16x16x32(av, p1, acc);
            acc = mfma16x16x32(av, p2, acc);
        }
        }
    }

    // ---- epilogue: y[m][n] (+ bias, + residual, separately rounded), m = r, n = row0 + lr + i
    const int n0 = row0 + lr;
    if (a.S == 1) {
        if (r < a.M) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int n = n0 + i;
                if (n < a.N) {
                    float v = acc[i];
                    if (a.bias) v = __fadd_rn(v, a.bias[n]);
                    if (a.res) v = __fadd_rn(v, a.res[(size_t)r * a.N + n]);
                    a.y[(size_t)r * a.N + n] = v;
                }
            }
        }
        return;
    }
    if (r < a.M) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
            if (n0 + i < a.N)
                __hip_atomic_store(&a.part[((size_t)sp * a.M + r) * a.N + n0 + i], acc[i], __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();                                // every partial store of the workgroup has completed
    if (tid == 0) {
        const uint32_t before = __hip_atomic_fetch_add(&a.cnt[rb], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        is_last = before == (uint32_t)(a.S - 1);
    }
    __syncthreads();
    if (!is_last) return;
    for (int i = tid; i < a.M * kRows; i += 256) {
        const int m = i / kRows, n = row0 + i % kRows;
        if (n >= a.N) continue;
        float v = 0.0f;
        for (int q = 0; q < a.S; ++q)
            v += __hip_atomic_load(&a.part[((size_t)q * a.M + m) * a.N + n], __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
        if (a.bias) v = __fadd_rn(v, a.bias[n]);
        if (a.res) v = __fadd_rn(v, a.res[(size_t)m * a.N + n]);
        a.y[(size_t)m * a.N + n] = v;
    }
    if (tid == 0) __hip_atomic_store(&a.cnt[rb], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Blocks per workgroup (32 INT8 / INT4 blocks, 16 bf16 blocks: a fixed K-split, so the summation order of an output
// does not depend on M) and staged activation columns (8 for M <= 8, else 16).
struct LinPlan {
    int cols, nb, S, row_blocks;
};
LinPlan lin_plan(int M, int N, int K, int w_type) {
    LinPlan p;
    p.cols = M <= 8 ? 8 : 16;
    p.nb = w_type == RK_W_BF16 ? 16 : 32;          // never depends on M: a row's sums do not depend on the batch
    const int nblk = K / kQB;
    p.S = (nblk + p.nb - 1) / p.nb;
    p.row_blocks = (N + kRows - 1) / kRows;
    return p;
}

// rows of W as fp32 (the reference's dequantize, src/quant.py:45-56: q * scale, + min for INT4, each rounded):
// out[i, k] for i < n_rows, source row rows ? rows[i] : row0 + i. One thread per 8 weights.
template <int WT>
__global__ __launch_bounds__(256) void dequant_rows_kernel(float* out, const void* w, const uint16_t* scales,
                                                           const uint16_t* mins, const int32_t* rows, int row0,
                                                           int n_rows, int K, int N) {
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    const int per_row = K / 8;
    if (i >= (long long)n_rows * per_row) return;
    const int ri = (int)(i / per_row), k0 = (int)(i % per_row) * 8;
    int src = rows ? rows[ri] : row0 + ri;
    src = src < 0 ? 0 : (src >= N ? N - 1 : src);
    float v[8];
    if constexpr (WT == RK_W_BF16) {
        const u32x4 q = *reinterpret_cast<const u32x4*>(static_cast<const uint16_t*>(w) + (size_t)src * K + k0);
#pragma unroll
        for (int j = 0; j < 4; ++j) { v[2 * j] = bf16_lo(q[j]); v[2 * j + 1] = bf16_hi(q[j]); }
    } else {
        const size_t pb = (size_t)src * (K / kQB) + k0 / kQB;
        const float s = half_to_f32(scales[pb]);
        if constexpr (WT == RK_W_INT8) {
            const u32x2 q = *reinterpret_cast<const u32x2*>(static_cast<const int8_t*>(w) + (size_t)src * K + k0);
#pragma unroll
            for (int e = 0; e < 8; ++e) v[e] = __fmul_rn((float)(int)__builtin_amdgcn_sbfe(q[e >> 2], 8 * (e & 3), 8), s);
        } else {
            const float mn = half_to_f32(mins[pb]);
            const uint8_t* wb = static_cast<const uint8_t*>(w) + (size_t)src * (K / 2) + k0 / 2;
            const uint32_t q = *reinterpret_cast<const uint32_t*>(wb);
#pragma unroll
            for (int e = 0; e < 8; ++e)
                v[e] = __fadd_rn(__fmul_rn((float)__builtin_amdgcn_ubfe(q, 4 * e, 4), s), mn);
        }
    }
    float4* o = reinterpret_cast<float4*>(out + (size_t)ri * K + k0);
    o[0] = make_float4(v[0], v[1], v[2], v[3]);
    o[1] = make_float4(v[4], v[5], v[6], v[7]);
}

}  // namespace
}  // namespace rk

using namespace rk;

extern "C" {

size_t rk_linear_workspace_bytes(int M, int N, int K, int w_type) {
    if (M < 1 || M > kCols || N < 1 || K < kQB || K % kQB) return 0;
    const LinPlan p = lin_plan(M, N, K, w_type);
    return p.S == 1 ? 0 : (size_t)p.S * M * N * sizeof(float);
}

int rk_linear_rows(float* y, const float* x, int M, int N, int K, const void* w, int w_type, const void* scales,
                   const void* mins, const float* bias, const float* residual, float* partials,
                   size_t partial_bytes, uint32_t* counters, int n_counters, void* stream) {
    if (M == 0 || N == 0) return RK_OK;
    const bool quant = w_type == RK_W_INT8 || w_type == RK_W_INT4;
    if (!y || !x || !w || (quant && !scales) || (w_type == RK_W_INT4 && !mins))
        return fail(RK_ERR_ARG, "rk_linear_rows: null pointer");
    if (w_type != RK_W_BF16 && !quant) return fail(RK_ERR_UNSUPPORTED, "rk_linear_rows: weight type %d", w_type);
    if (M < 0 || M > kCols || N < 0 || K < kQB || K % kQB)
        return fail(RK_ERR_ARG, "rk_linear_rows: M %d (1..%d), N %d, K %d (a multiple of %d)", M, kCols, N, K, kQB);
    if (reinterpret_cast<uintptr_t>(x) % 16 || reinterpret_cast<uintptr_t>(w) % 16)
        return fail(RK_ERR_ARG, "rk_linear_rows: x and w must be 16-byte aligned");
    const LinPlan p = lin_plan(M, N, K, w_type);
    const size_t need = rk_linear_workspace_bytes(M, N, K, w_type);
    if (need && (!partials || partial_bytes < need || !counters || n_counters < p.row_blocks))
        return fail(RK_ERR_WORKSPACE, "rk_linear_rows: partials %zu bytes (need %zu), %d counters (need %d)",
                    partial_bytes, need, n_counters, p.row_blocks);
    if ((long long)p.row_blocks * p.S >= (1ll << 31)) return fail(RK_ERR_ARG, "rk_linear_rows: N %d too large", N);
    LinArgs a;
    a.y = y; a.x = x; a.w = w; a.scales = static_cast<const uint16_t*>(scales);
    a.mins = static_cast<const uint16_t*>(mins); a.bias = bias; a.res = residual;
    a.cnt = counters;
    a.part = partials;
    a.M = M; a.N = N; a.K = K; a.S = p.S;
    using Fn = void (*)(LinArgs);
    Fn fn;
    if (p.cols == 8) {
        fn = w_type == RK_W_BF16 ? linear_rows_kernel<RK_W_BF16, 8, 16>
             : w_type == RK_W_INT8 ? linear_rows_kernel<RK_W_INT8, 8, 32> : linear_rows_kernel<RK_W_INT4, 8, 32>;
    } else {
        fn = w_type == RK_W_BF16 ? linear_rows_kernel<RK_W_BF16, 16, 16>
             : w_type == RK_W_INT8 ? linear_rows_kernel<RK_W_INT8, 16, 32> : linear_rows_kernel<RK_W_INT4, 16, 32>;
    }
    hipLaunchKernelGGL(fn, dim3((unsigned)(p.row_blocks * p.S)), dim3(256), 0, static_cast<hipStream_t>(stream), a);
    return check_launch("linear_rows");
}

int rk_dequant_rows(float* out, const void* w, int w_type, const void* scales, const void* mins,
                    const int32_t* rows, int row0, int n_rows, int N, int K, void* stream) {
    if (n_rows == 0) return RK_OK;
    const bool quant = w_type == RK_W_INT8 || w_type == RK_W_INT4;
    if (!out || !w || (quant && !scales) || (w_type == RK_W_INT4 && !mins))
        return fail(RK_ERR_ARG, "rk_dequant_rows: null pointer");
    if (w_type != RK_W_BF16 && w_type != RK_W_INT8 && w_type != RK_W_INT4)
        return fail(RK_ERR_UNSUPPORTED, "rk_dequant_rows: weight type %d", w_type);
    if (n_rows < 0 || N < 1 || K < kQB || K % kQB || (!rows && (row0 < 0 || row0 + n_rows > N)))
        return fail(RK_ERR_ARG, "rk_dequant_rows: rows %d + %d of %d, K %d (a multiple of %d)", row0, n_rows, N, K,
                    kQB);
    const long long n = (long long)n_rows * (K / 8);
    const dim3 grid((unsigned)ceil_div((size_t)n, 256));
    hipStream_t s = static_cast<hipStream_t>(stream);
    const uint16_t* sc = static_cast<const uint16_t*>(scales);
    const uint16_t* mn = static_cast<const uint16_t*>(mins);
    using Fn = void (*)(float*, const void*, const uint16_t*, const uint16_t*, const int32_t*, int, int, int, int);
    const Fn fn = w_type == RK_W_BF16 ? dequant_rows_kernel<RK_W_BF16>
                  : w_type == RK_W_INT8 ? dequant_rows_kernel<RK_W_INT8> : dequant_rows_kernel<RK_W_INT4>;
    hipLaunchKernelGGL(fn, grid, dim3(256), 0, s, out, w, sc, mn, rows, row0, n_rows, K, N);
    return check_launch("dequant_rows");
}

}  // extern "C"
