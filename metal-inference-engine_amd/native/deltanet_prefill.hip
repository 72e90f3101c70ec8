// Gated DeltaNet prefill companions around the chunked delta rule, gfx950: everything a linear-attention layer's
// packed prefill does besides the projections and the delta rule itself.
//
// Semantics (reference): per segment, src/models/qwen3_5.py:144-162 runs
//   u, new_tail = b.causal_conv1d(qkv, tail, conv_w)         (TorchBackend, src/backend/torch_ref.py:49-50: x widened
//                                                              to fp32 first, then src/ops.py:127-139: hist =
//                                                              [tail; x] all fp32 (the fp32 tail as stored),
//                                                              y_t = sum_j hist[t + j] * w[:, j], SiLU, new tail =
//                                                              the last K-1 rows of hist, fp32)
//   q, k, v = split(u);  beta = sigmoid(b);  g = -exp(A_log) * softplus(a + dt_bias)   (threshold 20)
//   q = l2norm(q) * (1 / sqrt(dk));  k = l2norm(k)          (src/ops.py:115-117: x * rsqrt(sum x^2 + 1e-6))
//   o, S = gated_delta(q, k, v, beta, g, S)                  (native/chunked_delta.hip)
//   out = rms_norm_gated(o, z, norm_w, eps)                  (src/ops.py:120-124: x * rsqrt(mean x^2 + eps) * w *
//                                                              silu(z), plain w)
// Kernels:
//   causal_conv_kernel      one segment, out-of-place (Backend.causal_conv1d): thread per (row, channel) of
//                           [silu(conv) rows; new tail rows].
//   prefill_front_kernel    packed segments, fused: one wave per (run of 32 tokens, 128-channel group); lanes own two
//                           channels and slide the conv window through the run in registers (each qkv row read once;
//                           the window starts from the segment's conv-state tail), the l2 norm of a q / k head is one
//                           wave reduction per token, the lanes of a q group write beta and g for the run.
//   tail_handoff_kernel     packed segments: each segment's new tail into its conv-state slot, after the front kernel
//                           has read the old one (stream order; a thread reads all K-1 old rows before writing).
//   rms_norm_gated_kernel   one wave per 8 rows of dv values, vector loads, all loads issued before the reductions.
// Arithmetic order follows the reference wherever it rounds separately (conv products rounded, then summed tap by
// tap; l2norm multiplies by the reciprocal square root; q scaled after the norm); length-128 sums are tree-reduced,
// and the streaming kernels take exp / reciprocal / reciprocal square root from the hardware instructions.
// All of it is HBM-bound elementwise work: every byte is read or written once (the conv's neighbouring taps hit in
// L1 / L2).
#include "rk_device.h"
#include "rk_internal.h"

namespace rk {
namespace {

constexpr int kMaxTaps = 8;         // rk_causal_conv1d
constexpr int kFrontMaxTaps = 4;    // rk_deltanet_prefill_front (instances K = 2, 3, 4)

// element `off` of a buffer of dtype dt, as fp32
__device__ __forceinline__ float ld_elem(const void* p, long long off, int dt) {
    return dt == RK_BF16 ? bf16_bits_to_f32(reinterpret_cast<const uint16_t*>(p)[off])
                         : reinterpret_cast<const float*>(p)[off];
}
// elements off, off + 1 (off even; the host checks the alignment this needs)
__device__ __forceinline__ float2 ld_pair(const void* p, long long off, int dt) {
    if (dt == RK_BF16) {
        const uint32_t w = reinterpret_cast<const uint32_t*>(p)[off >> 1];
        return make_float2(bf16_lo(w), bf16_hi(w));
    }
    return reinterpret_cast<const float2*>(p)[off >> 1];
}
__device__ __forceinline__ float silu(float y) { return y / (1.0f + expf(-y)); }
// The streaming front and norm kernels would be VALU-bound with the correctly rounded division, square root and
// the library exp (about 3x the instructions of the loads they hide behind): there SiLU and the reciprocal norms use
// the hardware's v_exp_f32 / v_rcp_f32 / v_rsq_f32 (each within 1-2 ulp; a few 1e-7 relative on the result).
__device__ __forceinline__ float silu_hw(float y) {
    return y * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-y * kLog2e));
}
__device__ __forceinline__ float rsqrt_hw(float x) { return __builtin_amdgcn_rsqf(x); }
// Outputs that the next kernel reads once are written with non-temporal (streaming) stores: they do not displace
// the rows still being read from the caches (measured 1.05-1.13x on the front, 1.3x on the norm).
__device__ __forceinline__ void stream_store2(float* p, float x0, float x1) {
    __builtin_nontemporal_store((f32x2_t{x0, x1}), reinterpret_cast<f32x2_t*>(p));
}

// ---- single segment, out-of-place (Backend.causal_conv1d): thread i < T*C computes u[t][c] = silu(conv); the
// next (K-1)*C threads copy hist rows T .. T+K-2 into new_tail (fp32: bf16 x rows widened exactly).
__global__ __launch_bounds__(256) void causal_conv_kernel(float* u, float* new_tail, const void* x, int x_dtype,
                                                          long long x_ld, const float* tail, const float* w, int T,
                                                          int C, int K) {
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (long long)(T + K - 1) * C) return;
    const int r = (int)(i / C), c = (int)(i % C);
    // hist row h: old tail row h (fp32 as stored) for h < K-1, else x row h - (K-1) widened
    auto hist = [&](int h) {
        return h < K - 1 ? tail[(long long)h * C + c] : ld_elem(x, (long long)(h - (K - 1)) * x_ld + c, x_dtype);
    };
    if (r < T) {
        // ((h0 w0 + h1 w1) + h2 w2) + ...: products rounded, summed tap by tap, as the reference's sum()
        float y = __fmul_rn(hist(r), w[(long long)c * K]);
        for (int j = 1; j < K; ++j) y = __fadd_rn(y, __fmul_rn(hist(r + j), w[(long long)c * K + j]));
        u[(long long)r * C + c] = silu(y);
    } else {
        new_tail[(long long)(r - T) * C + c] = hist(r);           // the last K-1 rows of hist
    }
}

struct FrontArgs {
    float* q;                   // [N, H, dk] fp32: l2-normalised, * 1/sqrt(dk)
    float* k;                   // [N, H, dk] fp32: l2-normalised
    float* v;                   // [N, H, dv] fp32
    float* beta;                // [N, H]
    float* g;                   // [N, H]
    const void* qkv;            // row n at qkv + n * ld: C = 2 H dk + H dv channels, x_dtype
    const void* b;              // row n at b + n * ld: H beta logits, x_dtype
    const void* a;              // row n at a + n * ld: H decay inputs, x_dtype
    const float* conv;          // segment s's tail [K-1, C] fp32 at conv + seq[s] * conv_stride
    const float* w;             // [C, K]
    const float* A_log;         // [H]
    const float* dt_bias;       // [H]
    const int32_t* cu;          // [S + 1] row offsets
    const int32_t* seq;         // [S] state index of each segment, or null (zero tails, no write-back)
    long long ld, conv_stride;
    int S, N, H, C, K, x_dtype;
    float qscale;               // 1 / sqrt(dk), rounded to fp32
};

// largest s with cu[s] <= row (cu non-decreasing; empty segments own no row)
__device__ __forceinline__ int segment_of_row(const int32_t* cu, int S, int row) {
    int lo = 0, hi = S - 1;
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (cu[mid] <= row) lo = mid; else hi = mid - 1;
    }
    return lo;
}

// One wave per (run of kRun consecutive packed tokens, 128-channel group); group index 0 .. H-1: q heads,
// H .. 2H-1: k heads, 2H .. 3H-1: v heads (the split of the conv output, qwen3_5.py:148-150). The 4 waves of a
// workgroup take 4 neighbouring groups of one run and consecutive workgroups walk the groups first, so the waves in
// flight read whole qkv rows and write whole q / k / v rows (walking the runs first instead has them write 512-byte
// slices at a fixed 8 KiB stride: measured 1.2x slower). Lanes own two channels; the K-1 hist rows before the
// current token stay in registers (win) and slide by one row per token, so a run reads its qkv rows once plus K-1
// rows to start; a run that crosses into another segment reloads the window from that segment's tail. Rows are
// fetched kBatch at a time so that many loads are in flight per wave.
constexpr int kRun = 32;
constexpr int kBatch = 8;

template <int K>
__global__ __launch_bounds__(256) void prefill_front_kernel(FrontArgs p) {
    const int lane = threadIdx.x & 63;
    // workgroups are dealt to the 8 XCDs round-robin; renumber them so that each XCD walks one contiguous range of
    // runs (the K-1 rows a run re-reads before its first token were fetched by the previous run into the same L2;
    // measured 1.1x)
    const unsigned per_xcd = gridDim.x / 8;
    unsigned wg = blockIdx.x;
    if (wg < per_xcd * 8) wg = (wg % 8) * per_xcd + wg / 8;
    const int quads = (3 * p.H + 3) >> 2;
    const int grp = (int)(wg % quads) * 4 + (threadIdx.x >> 6);
    if (grp >= 3 * p.H) return;                      // whole waves
    const int n0 = (int)(wg / quads) * kRun;
    const int n_end = min(n0 + kRun, p.N);
    const int c0 = grp * 128 + 2 * lane;
    const int xdt = p.x_dtype;
    const char kind = grp < p.H ? 0 : grp < 2 * p.H ? 1 : 2;      // q, k, v
    const int h = grp - kind * p.H;

    float2 wt[K];                                    // taps of channels c0, c0 + 1
#pragma unroll
    for (int j = 0; j < K; ++j) wt[j] = make_float2(p.w[(long long)c0 * K + j], p.w[(long long)(c0 + 1) * K + j]);

    int s = segment_of_row(p.cu, p.S, n0);
    int seg_lo = p.cu[s], seg_hi = p.cu[s + 1];
    // hist row r of segment s (r < K-1 + its length): old tail row r, fp32 as stored (zeros without a state), or
    // row seg_lo + r - (K-1) of qkv widened
    auto hist = [&](int r) {
        if (r < K - 1) {
            if (!p.seq) return make_float2(0.0f, 0.0f);
            const float* tail = p.conv + (long long)p.seq[s] * p.conv_stride;
            return *reinterpret_cast<const float2*>(tail + (long long)r * p.C + c0);
        }
        return ld_pair(p.qkv, (long long)(seg_lo + r - (K - 1)) * p.ld + c0, xdt);
    };
    float2 win[K - 1];                               // hist rows t .. t+K-2 of the next token (position t)
#pragma unroll
    for (int j = 0; j < K - 1; ++j) win[j] = hist(n0 - seg_lo + j);

    for (int nb = n0; nb < n_end; nb += kBatch) {
        float2 xr[kBatch];
#pragma unroll
        for (int i = 0; i < kBatch; ++i)
            xr[i] = nb + i < n_end ? ld_pair(p.qkv, (long long)(nb + i) * p.ld + c0, xdt) : make_float2(0.0f, 0.0f);
#pragma unroll
        for (int i = 0; i < kBatch; ++i) {
            const int n = nb + i;
            if (n >= n_end) break;
            if (n == seg_hi) {                       // the run enters the next non-empty segment: its old tail
                while (p.cu[s + 1] <= n) ++s;
                seg_lo = n;
                seg_hi = p.cu[s + 1];
#pragma unroll
                for (int j = 0; j < K - 1; ++j) win[j] = hist(j);
            }
            // ((h0 w0 + h1 w1) + h2 w2) + ...: products rounded, summed tap by tap, as the reference's sum()
            float y0 = __fmul_rn(win[0].x, wt[0].x), y1 = __fmul_rn(win[0].y, wt[0].y);
#pragma unroll
            for (int j = 1; j < K - 1; ++j) {
                y0 = __fadd_rn(y0, __fmul_rn(win[j].x, wt[j].x));
                y1 = __fadd_rn(y1, __fmul_rn(win[j].y, wt[j].y));
            }
            y0 = __fadd_rn(y0, __fmul_rn(xr[i].x, wt[K - 1].x));
            y1 = __fadd_rn(y1, __fmul_rn(xr[i].y, wt[K - 1].y));
#pragma unroll
            for (int j = 0; j < K - 2; ++j) win[j] = win[j + 1];
            win[K - 2] = xr[i];
            const float u0 = silu_hw(y0), u1 = silu_hw(y1);
            const long long o = ((long long)n * p.H + h) * 128 + 2 * lane;
            if (kind == 2) {
                stream_store2(p.v + o, u0, u1);
            } else {
                // l2norm (ops.py:115-117): x * (1 / sqrt(sum x^2 + 1e-6)); q is then scaled by fp32(1 / sqrt(dk))
                const float ss = wave_sum(__fadd_rn(__fmul_rn(u0, u0), __fmul_rn(u1, u1)));
                const float inv = rsqrt_hw(ss + 1e-6f);
                float2 r = make_float2(__fmul_rn(u0, inv), __fmul_rn(u1, inv));
                if (kind == 0) r = make_float2(__fmul_rn(r.x, p.qscale), __fmul_rn(r.y, p.qscale));
                stream_store2((kind == 0 ? p.q : p.k) + o, r.x, r.y);
            }
        }
    }
    if (kind == 0 && n0 + lane < n_end) {
        // beta = sigmoid(b); g = -exp(A_log) * softplus(a + dt_bias), softplus(x) = x above 20: lane i, token n0 + i
        const int n = n0 + lane;
        const long long bo = (long long)n * p.ld + h;
        const float bl = ld_elem(p.b, bo, xdt);
        const float ab = __fadd_rn(ld_elem(p.a, bo, xdt), p.dt_bias[h]);
        const float sp = ab > 20.0f ? ab : log1pf(expf(ab));
        p.beta[(long long)n * p.H + h] = 1.0f / (1.0f + expf(-bl));
        p.g[(long long)n * p.H + h] = __fmul_rn(-expf(p.A_log[h]), sp);
    }
}

// one thread per (segment, channel): hist rows T .. T+K-2 of [old tail; x] become the segment's tail (fp32: carried
// old rows keep their bits, x rows are widened). Launched after the front kernel has read every old tail; the
// thread reads all K-1 old rows before it writes.
__global__ __launch_bounds__(256) void tail_handoff_kernel(FrontArgs p, float* conv) {
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (long long)p.S * p.C) return;
    const int s = (int)(i / p.C), c = (int)(i % p.C);
    const int T = p.cu[s + 1] - p.cu[s];
    if (T == 0) return;                              // an empty segment leaves its state as it is
    float* tail = conv + (long long)p.seq[s] * p.conv_stride;
    float old[kMaxTaps];
    for (int r = 0; r < p.K - 1; ++r) old[r] = tail[(long long)r * p.C + c];
    for (int r = 0; r < p.K - 1; ++r) {
        const int h = T + r;
        tail[(long long)r * p.C + c] =
            h < p.K - 1 ? old[h] : ld_elem(p.qkv, (long long)(p.cu[s] + h - (p.K - 1)) * p.ld + c, p.x_dtype);
    }
}

// rms_norm_gated, ops.py:120-124: y = x * (1 / sqrt(mean x^2 + eps)), out = (y * w) * silu(z). One wave per kRows
// consecutive rows of dv = 64 * PER values (lane l owns elements PER*l .. PER*l + PER-1 of a row); all of a wave's
// loads are issued before the first reduction. Row r of z starts at z + (r / z_group) * z_ld + (r % z_group) * dv
// (z_group = 1 and z_ld = dv for a contiguous [rows, dv] z; z_group = H, z_ld = the projection row length for the
// z columns of a fused projection output).
constexpr int kRows = 8;

template <int PER>
__device__ __forceinline__ void ld_vec(float (&d)[PER], const float* p) {
    if constexpr (PER == 1) d[0] = *p;
    else if constexpr (PER == 2) { const float2 v = *reinterpret_cast<const float2*>(p); d[0] = v.x; d[1] = v.y; }
    else {
#pragma unroll
        for (int i = 0; i < PER; i += 4) {
            const float4 v = *reinterpret_cast<const float4*>(p + i);
            d[i] = v.x; d[i + 1] = v.y; d[i + 2] = v.z; d[i + 3] = v.w;
        }
    }
}
template <int PER>
__device__ __forceinline__ void ld_vec_bf16(float (&d)[PER], const uint16_t* p) {
    if constexpr (PER == 1) d[0] = bf16_bits_to_f32(*p);
    else if constexpr (PER == 2) {
        const uint32_t v = *reinterpret_cast<const uint32_t*>(p);
        d[0] = bf16_lo(v); d[1] = bf16_hi(v);
    }
    else {
#pragma unroll
        for (int i = 0; i < PER; i += 4) {
            const u32x2 v = *reinterpret_cast<const u32x2*>(p + i);
            d[i] = bf16_lo(v.x); d[i + 1] = bf16_hi(v.x); d[i + 2] = bf16_lo(v.y); d[i + 3] = bf16_hi(v.y);
        }
    }
}
template <int PER>
__device__ __forceinline__ void st_vec(float* p, const float (&d)[PER]) {
    if constexpr (PER == 1) __builtin_nontemporal_store(d[0], p);
    else if constexpr (PER == 2) stream_store2(p, d[0], d[1]);
    else {
#pragma unroll
        for (int i = 0; i < PER; i += 4)
            __builtin_nontemporal_store((f32x4{d[i], d[i + 1], d[i + 2], d[i + 3]}), reinterpret_cast<f32x4*>(p + i));
    }
}

template <int PER>
__global__ __launch_bounds__(256) void rms_norm_gated_kernel(float* out, const float* x, const void* z, int z_dtype,
                                                             long long z_ld, int z_group, const float* w, int rows,
                                                             float eps) {
    constexpr int dv = 64 * PER;
    const int lane = threadIdx.x & 63;
    const long long r0 = ((long long)blockIdx.x * 4 + (threadIdx.x >> 6)) * kRows;
    if (r0 >= rows) return;
    const int nr = (int)min((long long)kRows, rows - r0);
    float xv[kRows][PER], zv[kRows][PER], wv[PER];
#pragma unroll
    for (int i = 0; i < kRows; ++i) {
        if (i < nr) {
            const long long row = r0 + i;
            const long long zrow = (row / z_group) * z_ld + (row % z_group) * dv + PER * lane;
            ld_vec<PER>(xv[i], x + row * dv + PER * lane);
            if (z_dtype == RK_BF16) ld_vec_bf16<PER>(zv[i], reinterpret_cast<const uint16_t*>(z) + zrow);
            else ld_vec<PER>(zv[i], reinterpret_cast<const float*>(z) + zrow);
        }
    }
    ld_vec<PER>(wv, w + PER * lane);
#pragma unroll
    for (int i = 0; i < kRows; ++i) {
        if (i < nr) {
            float ss = 0.0f;
#pragma unroll
            for (int e = 0; e < PER; ++e) ss = __fadd_rn(ss, __fmul_rn(xv[i][e], xv[i][e]));
            ss = wave_sum(ss);
            const float rstd = rsqrt_hw(__fadd_rn(ss * (1.0f / dv), eps));          // dv a power of 2: exact
            float o[PER];
#pragma unroll
            for (int e = 0; e < PER; ++e)
                o[e] = __fmul_rn(__fmul_rn(__fmul_rn(xv[i][e], rstd), wv[e]), silu_hw(zv[i][e]));
            st_vec<PER>(out + (r0 + i) * dv + PER * lane, o);
        }
    }
}

}  // namespace
}  // namespace rk

using namespace rk;

extern "C" {

int rk_causal_conv1d(float* u, float* new_tail, const void* x, int x_dtype, long long x_ld, const float* tail,
                     const float* w, int T, int C, int K, void* stream) {
    if (!u || !new_tail || !tail || !w || (T > 0 && !x)) return fail(RK_ERR_ARG, "rk_causal_conv1d: null pointer");
    if (T < 0 || C < 1 || K < 2 || K > kMaxTaps || (T > 0 && x_ld < C))
        return fail(RK_ERR_ARG, "rk_causal_conv1d: T %d, C %d, K %d (2..%d), row stride %lld", T, C, K, kMaxTaps,
                    x_ld);
    if (x_dtype != RK_F32 && x_dtype != RK_BF16) return fail(RK_ERR_UNSUPPORTED, "rk_causal_conv1d: dtype %d", x_dtype);
    const long long n = (long long)(T + K - 1) * C;
    hipLaunchKernelGGL(causal_conv_kernel, dim3((unsigned)ceil_div((size_t)n, 256)), dim3(256), 0,
                       static_cast<hipStream_t>(stream), u, new_tail, x, x_dtype, x_ld, tail, w, T, C, K);
    return check_launch("causal_conv1d");
}

int rk_deltanet_prefill_front(float* q, float* k, float* v, float* beta, float* g, const void* qkv, const void* b,
                              const void* a, int x_dtype, long long ld, float* conv_state, long long conv_stride,
                              const float* conv_w, const float* A_log, const float* dt_bias,
                              const int32_t* cu_seqlens, const int32_t* seq_index, int n_seqs, int N, int H, int dk,
                              int dv, int conv_k, void* stream) {
    if (!q || !k || !v || !beta || !g || !conv_w || !A_log || !dt_bias || !cu_seqlens ||
        (N > 0 && (!qkv || !b || !a)) || (seq_index && !conv_state))
        return fail(RK_ERR_ARG, "rk_deltanet_prefill_front: null pointer");
    if (dk != 128 || dv != 128)
        return fail(RK_ERR_UNSUPPORTED, "rk_deltanet_prefill_front: dk %d dv %d (built for 128)", dk, dv);
    if (x_dtype != RK_F32 && x_dtype != RK_BF16)
        return fail(RK_ERR_UNSUPPORTED, "rk_deltanet_prefill_front: dtype %d", x_dtype);
    const int C = 2 * H * dk + H * dv;
    if (n_seqs < 1 || N < 0 || H < 1 || conv_k < 2 || conv_k > kFrontMaxTaps || (N > 0 && ld < C) ||
        (seq_index && conv_stride < (long long)(conv_k - 1) * C))
        return fail(RK_ERR_ARG, "rk_deltanet_prefill_front: %d segments, N %d, H %d, conv kernel %d (2..%d), row "
                    "stride %lld, state stride %lld", n_seqs, N, H, conv_k, kFrontMaxTaps, ld, conv_stride);
    // channel pairs are read as one 8-byte (fp32) / 4-byte (bf16) load
    const size_t al = x_dtype == RK_BF16 ? 4 : 8;
    if ((N > 0 && (reinterpret_cast<uintptr_t>(qkv) % al || ld % 2)) ||
        (seq_index && (reinterpret_cast<uintptr_t>(conv_state) % 8 || conv_stride % 2)))
        return fail(RK_ERR_ARG, "rk_deltanet_prefill_front: qkv and conv state rows must start %zu / 8-byte aligned "
                    "(even strides)", al);
    if (N == 0) return RK_OK;
    FrontArgs p;
    p.q = q; p.k = k; p.v = v; p.beta = beta; p.g = g; p.qkv = qkv; p.b = b; p.a = a; p.conv = conv_state;
    p.w = conv_w; p.A_log = A_log; p.dt_bias = dt_bias; p.cu = cu_seqlens; p.seq = seq_index;
    p.ld = ld; p.conv_stride = conv_stride;
    p.S = n_seqs; p.N = N; p.H = H; p.C = C; p.K = conv_k; p.x_dtype = x_dtype;
    p.qscale = (float)(1.0 / sqrt((double)dk));
    hipStream_t s = static_cast<hipStream_t>(stream);
    const dim3 grid((unsigned)(ceil_div((size_t)N, kRun) * ceil_div((size_t)(3 * H), 4)));
    if (conv_k == 2) hipLaunchKernelGGL(prefill_front_kernel<2>, grid, dim3(256), 0, s, p);
    else if (conv_k == 3) hipLaunchKernelGGL(prefill_front_kernel<3>, grid, dim3(256), 0, s, p);
    else hipLaunchKernelGGL(prefill_front_kernel<4>, grid, dim3(256), 0, s, p);
    int rc = check_launch("deltanet_prefill_front");
    if (rc || !seq_index) return rc;
    const long long n = (long long)n_seqs * C;
    hipLaunchKernelGGL(tail_handoff_kernel, dim3((unsigned)ceil_div((size_t)n, 256)), dim3(256), 0, s, p, conv_state);
    return check_launch("deltanet_tail_handoff");
}

int rk_rms_norm_gated(float* out, const float* x, const void* z, int z_dtype, long long z_ld, int z_group,
                      const float* w, int rows, int dv, float eps, void* stream) {
    if (rows < 0 || (dv != 64 && dv != 128 && dv != 256 && dv != 512) || z_group < 1 ||
        (rows > 0 && z_ld < (long long)z_group * dv))
        return fail(RK_ERR_ARG, "rk_rms_norm_gated: rows %d, dv %d (64, 128, 256 or 512), z rows of %d heads "
                    "at stride %lld", rows, dv, z_group, z_ld);
    if (rows == 0) return RK_OK;
    if (!out || !x || !z || !w) return fail(RK_ERR_ARG, "rk_rms_norm_gated: null pointer");
    if (z_dtype != RK_F32 && z_dtype != RK_BF16)
        return fail(RK_ERR_UNSUPPORTED, "rk_rms_norm_gated: z dtype %d", z_dtype);
    // vector loads of PER elements: z rows must start PER-element aligned
    const int per = dv / 64;
    const size_t zes = z_dtype == RK_BF16 ? 2 : 4;
    if (reinterpret_cast<uintptr_t>(x) % (per * 4) || reinterpret_cast<uintptr_t>(out) % (per * 4) ||
        reinterpret_cast<uintptr_t>(w) % (per * 4) || reinterpret_cast<uintptr_t>(z) % (per * zes) || z_ld % per)
        return fail(RK_ERR_ARG, "rk_rms_norm_gated: x, out, w, z and z's row stride must be aligned to %d elements "
                    "(dv %d)", per, dv);
    const dim3 grid((unsigned)ceil_div(ceil_div((size_t)rows, kRows), 4));
    auto launch = [&](auto kernel) {
        hipLaunchKernelGGL(kernel, grid, dim3(256), 0, static_cast<hipStream_t>(stream), out, x, z, z_dtype, z_ld,
                           z_group, w, rows, eps);
    };
    if (per == 1) launch(rms_norm_gated_kernel<1>);
    else if (per == 2) launch(rms_norm_gated_kernel<2>);
    else if (per == 4) launch(rms_norm_gated_kernel<4>);
    else launch(rms_norm_gated_kernel<8>);
    return check_launch("rms_norm_gated");
}

}  // extern "C"
