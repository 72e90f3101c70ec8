// The row-wise and elementwise operations of a decode step around the linears, gfx950: RMSNorm, LayerNorm (no
// bias), RoPE and silu(gate) * up. With the linears (linear.hip), the token mixers (P1-P4) and the embedding
// (rk_dequant_rows) they make every operation of the backend protocol a HIP kernel.
//
// Semantics (reference), fp32 throughout, each operation rounded as the reference's tensor ops round it:
//   rms_norm(x, w, eps)   = (x / sqrt(mean(x * x) + eps)) * w                        (src/ops.py:7-15)
//   layer_norm(x, w, eps) = w * ((x - mean(x)) * (1 / sqrt(var + eps))),
//                           var = mean((x - mean(x))^2)                                (src/ops.py:18-24)
//   rope(x, pos, theta)   : pairs (i, i + d/2) rotated by pos * inv_freq[i] (host-computed fp32 inv_freq,
//                           rope_inv_freq): a cos - b sin, a sin + b cos               (src/ops.py:27-54)
//   silu_mul(g, u)        = (g / (1 + exp(-g))) * u                                   (src/ops.py:107-110)
// Means are sums of rounded terms in a different order than torch's (a wave tree), within the 1e-5 bar; the square
// root and divisions are correctly rounded, cos / sin / exp are the device library's.
// Norms: one wave per row, lane l holding 4-float chunks l, l + 64, ... of it (rows of up to 64 * 4 * MAXV
// values stay in registers: one read of x, one write of out); any other row (longer than 4096, a length not a
// multiple of 4, or unaligned) takes a workgroup of its own and reads its row two or three times. RoPE and silu_mul: one thread per element pair /
// four elements.
#include "rk_device.h"
#include "rk_internal.h"

namespace rk {
namespace {

__device__ __forceinline__ f32x4 ld4(const void* p, long long off, int dt) {
    if (dt == RK_BF16) {
        const u32x2 w = *reinterpret_cast<const u32x2*>(static_cast<const uint16_t*>(p) + off);
        return (f32x4){bf16_lo(w.x), bf16_hi(w.x), bf16_lo(w.y), bf16_hi(w.y)};
    }
    return *reinterpret_cast<const f32x4*>(static_cast<const float*>(p) + off);
}

// The row norms. KIND 0: RMSNorm; 1: LayerNorm. MAXV: 4-float chunks per lane (D <= 256 MAXV).
template <int KIND, int MAXV>
__global__ __launch_bounds__(256) void row_norm_kernel(float* __restrict__ out, const void* __restrict__ x,
                                                       int x_dtype, long long ld, const void* __restrict__ w,
                                                       int w_dtype, int rows, int D, float eps) {
    const int lane = threadIdx.x & 63;
    const long long row = (long long)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= rows) return;                        // whole waves leave: no barrier below
    const int nv = D >> 2;                          // 4-float chunks in the row
    f32x4 v[MAXV], wv[MAXV];
#pragma unroll
    for (int i = 0; i < MAXV; ++i) {                // the row and the weights requested together: one round trip
        const int c = lane + 64 * i;
        v[i] = c < nv ? ld4(x, row * ld + 4 * c, x_dtype) : (f32x4){0.f, 0.f, 0.f, 0.f};
        wv[i] = c < nv ? ld4(w, 4 * c, w_dtype) : (f32x4){0.f, 0.f, 0.f, 0.f};
    }
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < MAXV; ++i) {
        if constexpr (KIND == 0) {
#pragma unroll
            for (int e = 0; e < 4; ++e) s = __fadd_rn(s, __fmul_rn(v[i][e], v[i][e]));
        } else {
#pragma unroll
            for (int e = 0; e < 4; ++e) s = __fadd_rn(s, v[i][e]);
        }
    }
    float scale;
    float mean = 0.0f;
    if constexpr (KIND == 0) {
        scale = sqrtf(__fadd_rn(__fdiv_rn(wave_sum(s), (float)D), eps));          // the rms (divided by)
    } else {
        mean = __fdiv_rn(wave_sum(s), (float)D);
        float q = 0.0f;
#pragma unroll
        for (int i = 0; i < MAXV; ++i) {
            const int c = lane + 64 * i;
            if (c < nv) {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float ce = __fsub_rn(v[i][e], mean);
                    q = __fadd_rn(q, __fmul_rn(ce, ce));
                }
            }
        }
        scale = __fdiv_rn(1.0f, sqrtf(__fadd_rn(__fdiv_rn(wave_sum(q), (float)D), eps)));   // rsqrt(var + eps)
    }
#pragma unroll
    for (int i = 0; i < MAXV; ++i) {
        const int c = lane + 64 * i;
        if (c < nv) {
            f32x4 o;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                if constexpr (KIND == 0) o[e] = __fmul_rn(__fdiv_rn(v[i][e], scale), wv[i][e]);
                else o[e] = __fmul_rn(wv[i][e], __fmul_rn(__fsub_rn(v[i][e], mean), scale));
            }
            *reinterpret_cast<f32x4*>(out + row * D + 4 * c) = o;
        }
    }
}

// Rows the register kernel does not take (D above 4096, D not a multiple of 4, or unaligned rows): one workgroup of
// 256 threads per row, thread t holding elements t, t + 256, ... of it; the sums go through a wave tree and LDS.
// RMSNorm reads the row twice (sum of squares, then the output), LayerNorm three times (mean, centred squares,
// output); a row of a few thousand values stays in L2 between the passes.
__device__ __forceinline__ float ld1(const void* p, long long off, int dt) {
    return dt == RK_BF16 ? bf16_bits_to_f32(static_cast<const uint16_t*>(p)[off]) : static_cast<const float*>(p)[off];
}

__device__ __forceinline__ float block256_sum(float x, float* red) {
    x = wave_sum(x);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) red[wave] = x;
    __syncthreads();
    const float t = __fadd_rn(__fadd_rn(red[0], red[1]), __fadd_rn(red[2], red[3]));
    __syncthreads();                                // red is reused by the next reduction
    return t;
}

template <int KIND>
__global__ __launch_bounds__(256) void row_norm_wide_kernel(float* __restrict__ out, const void* __restrict__ x,
                                                            int x_dtype, long long ld, const void* __restrict__ w,
                                                            int w_dtype, int D, float eps) {
    __shared__ float red[4];
    const long long row = blockIdx.x;
    const long long xo = row * ld;
    float s = 0.0f;
    for (int i = threadIdx.x; i < D; i += 256) {
        const float v = ld1(x, xo + i, x_dtype);
        s = KIND == 0 ? __fadd_rn(s, __fmul_rn(v, v)) : __fadd_rn(s, v);
    }
    s = block256_sum(s, red);
    float scale, mean = 0.0f;
    if constexpr (KIND == 0) {
        scale = sqrtf(__fadd_rn(__fdiv_rn(s, (float)D), eps));
    } else {
        mean = __fdiv_rn(s, (float)D);
        float q = 0.0f;
        for (int i = threadIdx.x; i < D; i += 256) {
            const float c = __fsub_rn(ld1(x, xo + i, x_dtype), mean);
            q = __fadd_rn(q, __fmul_rn(c, c));
        }
        q = block256_sum(q, red);
        scale = __fdiv_rn(1.0f, sqrtf(__fadd_rn(__fdiv_rn(q, (float)D), eps)));
    }
    for (int i = threadIdx.x; i < D; i += 256) {
        const float v = ld1(x, xo + i, x_dtype), wv = ld1(w, i, w_dtype);
        out[row * D + i] = KIND == 0 ? __fmul_rn(__fdiv_rn(v, scale), wv) : __fmul_rn(wv, __fmul_rn(__fsub_rn(v, mean), scale));
    }
}

// RoPE over whole heads: thread (t, h, i < d/2) rotates the pair (i, i + d/2) of x[t, h].
__global__ __launch_bounds__(256) void rope_kernel(float* __restrict__ out, const float* __restrict__ x,
                                                   const int32_t* __restrict__ pos,
                                                   const float* __restrict__ inv_freq, long long n, int H, int half) {
    const long long idx = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= n) return;
    const int i = (int)(idx % half);
    const long long th = idx / half;                // t * H + h
    const long long t = th / H;
    const long long base = th * 2 * half;
    const float ang = __fmul_rn((float)pos[t], inv_freq[i]);
    const float c = cosf(ang), s = sinf(ang);
    const float a = x[base + i], b = x[base + i + half];
    out[base + i] = __fsub_rn(__fmul_rn(a, c), __fmul_rn(b, s));
    out[base + i + half] = __fadd_rn(__fmul_rn(a, s), __fmul_rn(b, c));
}

// out [rows, F] = silu(gate) * up, gate / up rows at gate + r * g_ld, up + r * u_ld (fp32). V = 4: F, the strides
// and the pointers allow 16-byte accesses; V = 1 otherwise.
template <int V>
__global__ __launch_bounds__(256) void silu_mul_kernel(float* __restrict__ out, const float* __restrict__ gate,
                                                       long long g_ld, const float* __restrict__ up, long long u_ld,
                                                       int rows, int F) {
    const long long idx = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    const int per_row = F / V;
    if (idx >= (long long)rows * per_row) return;
    const long long r = idx / per_row;
    const int f = (int)(idx % per_row) * V;
    float g[V], u[V], o[V];
    if constexpr (V == 4) {
        const f32x4 gv = *reinterpret_cast<const f32x4*>(gate + r * g_ld + f);
        const f32x4 uv = *reinterpret_cast<const f32x4*>(up + r * u_ld + f);
#pragma unroll
        for (int e = 0; e < 4; ++e) { g[e] = gv[e]; u[e] = uv[e]; }
    } else {
        g[0] = gate[r * g_ld + f];
        u[0] = up[r * u_ld + f];
    }
#pragma unroll
    for (int e = 0; e < V; ++e) o[e] = __fmul_rn(__fdiv_rn(g[e], __fadd_rn(1.0f, expf(-g[e]))), u[e]);
    if constexpr (V == 4) *reinterpret_cast<f32x4*>(out + r * F + f) = (f32x4){o[0], o[1], o[2], o[3]};
    else out[r * F + f] = o[0];
}

constexpr int kMaxNormD = 64 * 4 * 16;             // 4096: rows kept in registers (16 chunks of 4 per lane)

template <int KIND>
int launch_norm(float* out, const void* x, int x_dtype, long long ld, const void* w, int w_dtype, int rows, int D,
                float eps, void* stream, const char* name) {
    if (rows == 0) return RK_OK;
    if (!out || !x || !w) return fail(RK_ERR_ARG, "%s: null pointer", name);
    if ((x_dtype != RK_F32 && x_dtype != RK_BF16) || (w_dtype != RK_F32 && w_dtype != RK_BF16))
        return fail(RK_ERR_UNSUPPORTED, "%s: dtypes x %d, w %d", name, x_dtype, w_dtype);
    if (rows < 0 || D < 1 || ld < D)
        return fail(RK_ERR_ARG, "%s: rows %d, D %d, row stride %lld", name, rows, D, ld);
    const size_t xa = x_dtype == RK_BF16 ? 8 : 16, wa = w_dtype == RK_BF16 ? 8 : 16;
    const bool in_registers = D % 4 == 0 && D <= kMaxNormD && ld % 4 == 0 &&
                              reinterpret_cast<uintptr_t>(x) % xa == 0 && reinterpret_cast<uintptr_t>(w) % wa == 0 &&
                              reinterpret_cast<uintptr_t>(out) % 16 == 0;
    if (!in_registers) {
        if ((unsigned long long)rows > 0x7fffffffull) return fail(RK_ERR_ARG, "%s: %d rows", name, rows);
        hipLaunchKernelGGL(row_norm_wide_kernel<KIND>, dim3((unsigned)rows), dim3(256), 0,
                           static_cast<hipStream_t>(stream), out, x, x_dtype, ld, w, w_dtype, D, eps);
        return check_launch(name);
    }
    using Fn = void (*)(float*, const void*, int, long long, const void*, int, int, int, float);
    const int nv = (D / 4 + 63) / 64;
    const Fn fn = nv <= 1 ? row_norm_kernel<KIND, 1> : nv <= 2 ? row_norm_kernel<KIND, 2>
                  : nv <= 4 ? row_norm_kernel<KIND, 4> : nv <= 8 ? row_norm_kernel<KIND, 8> : row_norm_kernel<KIND, 16>;
    hipLaunchKernelGGL(fn, dim3((unsigned)ceil_div((size_t)rows, 4)), dim3(256), 0, static_cast<hipStream_t>(stream),
                       out, x, x_dtype, ld, w, w_dtype, rows, D, eps);
    return check_launch(name);
}

}  // namespace
}  // namespace rk

using namespace rk;

extern "C" {

int rk_rms_norm(float* out, const void* x, int x_dtype, long long x_ld, const void* w, int w_dtype, int rows, int D,
                float eps, void* stream) {
    return launch_norm<0>(out, x, x_dtype, x_ld, w, w_dtype, rows, D, eps, stream, "rk_rms_norm");
}

int rk_layer_norm(float* out, const void* x, int x_dtype, long long x_ld, const void* w, int w_dtype, int rows, int D,
                  float eps, void* stream) {
    return launch_norm<1>(out, x, x_dtype, x_ld, w, w_dtype, rows, D, eps, stream, "rk_layer_norm");
}

int rk_rope(float* out, const float* x, const int32_t* positions, const float* inv_freq, int T, int H, int d,
            void* stream) {
    if (T == 0 || H == 0) return RK_OK;
    if (!out || !x || !positions || !inv_freq) return fail(RK_ERR_ARG, "rk_rope: null pointer");
    if (T < 0 || H < 0 || d < 2 || d % 2) return fail(RK_ERR_ARG, "rk_rope: T %d, H %d, d %d (even)", T, H, d);
    const long long n = (long long)T * H * (d / 2);
    hipLaunchKernelGGL(rope_kernel, dim3((unsigned)ceil_div((size_t)n, 256)), dim3(256), 0,
                       static_cast<hipStream_t>(stream), out, x, positions, inv_freq, n, H, d / 2);
    return check_launch("rope");
}

int rk_silu_mul(float* out, const float* gate, long long gate_ld, const float* up, long long up_ld, int rows, int F,
                void* stream) {
    if (rows == 0 || F == 0) return RK_OK;
    if (!out || !gate || !up) return fail(RK_ERR_ARG, "rk_silu_mul: null pointer");
    if (rows < 0 || F < 0 || gate_ld < F || up_ld < F)
        return fail(RK_ERR_ARG, "rk_silu_mul: rows %d, F %d, strides %lld / %lld", rows, F, gate_ld, up_ld);
    const bool vec = F % 4 == 0 && gate_ld % 4 == 0 && up_ld % 4 == 0 && reinterpret_cast<uintptr_t>(out) % 16 == 0 &&
                     reinterpret_cast<uintptr_t>(gate) % 16 == 0 && reinterpret_cast<uintptr_t>(up) % 16 == 0;
    const long long n = (long long)rows * (vec ? F / 4 : F);
    hipStream_t s = static_cast<hipStream_t>(stream);
    const dim3 grid((unsigned)ceil_div((size_t)n, 256));
    if (vec) hipLaunchKernelGGL(silu_mul_kernel<4>, grid, dim3(256), 0, s, out, gate, gate_ld, up, up_ld, rows, F);
    else hipLaunchKernelGGL(silu_mul_kernel<1>, grid, dim3(256), 0, s, out, gate, gate_ld, up, up_ld, rows, F);
    return check_launch("silu_mul");
}

}  // extern "C"
