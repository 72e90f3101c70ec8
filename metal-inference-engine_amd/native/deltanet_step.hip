// P2: fused Gated DeltaNet decode step (one new token per sequence), gfx950.
//
// Semantics: TorchBackend.deltanet_decode (src/backend/torch_ref.py:61-73) = ops.causal_conv1d (src/ops.py:127-139)
// -> split q|k|v -> ops.l2norm (q also * 1/sqrt(dk)) -> beta = sigmoid(b), g = -exp(A_log) * softplus(a + dt_bias)
// (threshold 20) -> ops.gated_delta_recurrent with T = 1 (src/ops.py:142-157) -> ops.rms_norm_gated
// (src/ops.py:120-124). The conv tail and S are updated in place at [seq_index[i], slot] (src/state.py:428-429;
// the Metal pair conv_step + gdn_decode, src/kernels/deltanet.metal:9-92, indexes them the same way).
//
// One workgroup of 256 threads per (sequence, head) (6.62 -> 6.33 us per config-2 step against 512 threads, A/B in
// one process). The head's 128 x 128 fp32 state is loaded once into registers (thread = 16 rows x 4 columns, a row
// of 32 threads reads 512 contiguous bytes), decayed, rank-1 updated and written back once: 2 x 64 KiB of HBM traffic per head, the algorithmic minimum. The S loads are issued first, so the
// convolution of the head's 384 channels, the l2 norms and the gate parameters are computed while they are in
// flight. Elementwise steps keep the reference's operation order (products rounded before sums, no contraction into
// FMA) wherever the reference rounds them separately; only the lengths-128 sums are reordered (tree instead of
// sequential), which moves results by a few ulp.
#include "rk_device.h"
#include "rk_internal.h"

namespace rk {
namespace {

constexpr int kDK = 128, kDV = 128, kTaps = 4, kThreads = 256;
constexpr int kRowGroups = kThreads / 32, kRowsPer = kDK / kRowGroups;   // 8 row groups of 16 state rows

struct StepArgs {
    float* out;
    const float* qkv;
    const float* z;
    const float* b;
    const float* a;
    long long qkv_ld, z_ld, ba_ld;   // row strides (elements) of qkv, z, and b / a: column slices of one projection
    float* conv;
    float* S;
    const float* conv_w;
    const float* A_log;
    const float* dt_bias;
    const float* norm_w;
    const int32_t* seq;
    int B, H, C, n_linear, slot;
    float eps;
};

__global__ __launch_bounds__(kThreads) void deltanet_step_kernel(StepArgs p) {
    __shared__ float us[3 * kDK];        // conv + SiLU output of this head: q | k | v
    __shared__ float qn[kDK], kn[kDK], dl[kDV];
    __shared__ float red[kRowGroups][kDV];   // partial sums over row groups
    __shared__ float wsum[8];

    const int t = threadIdx.x;
    const int bi = blockIdx.x / p.H, h = blockIdx.x % p.H;
    const int H = p.H, C = p.C;

    // ---- 0. every small input first, the state after them: one in-order counter serves loads and stores, so a
    // load issued after the state stores could only be waited for together with them. Thread t owns channel t of
    // q | k (t < 128: q, else k) and, for t < 128, v channel t as well.
    const int ca = t < kDK ? h * kDK + t : H * kDK + h * kDK + (t - kDK);
    const int cb = 2 * H * kDK + h * kDV + (t & (kDV - 1));
    const bool has_v = t < kDV;
    const float xa = p.qkv[(long long)bi * p.qkv_ld + ca];
    const float xb = has_v ? p.qkv[(long long)bi * p.qkv_ld + cb] : 0.0f;
    const float4 wa = *reinterpret_cast<const float4*>(p.conv_w + (long long)ca * kTaps);
    const float4 wb = has_v ? *reinterpret_cast<const float4*>(p.conv_w + (long long)cb * kTaps)
                            : make_float4(0.f, 0.f, 0.f, 0.f);
    const float b_in = p.b[(long long)bi * p.ba_ld + h], a_in = p.a[(long long)bi * p.ba_ld + h];
    const float dtb = p.dt_bias[h], alog = p.A_log[h];
    const float zj = t < kDV ? p.z[(long long)bi * p.z_ld + h * kDV + t] : 0.0f;
    const float nw = t < kDV ? p.norm_w[t] : 0.0f;
    const long long seq = p.seq[bi];
    float* Sh = p.S + (((seq * p.n_linear + p.slot) * H + h) * kDK) * kDV;
    float* tail = p.conv + (seq * p.n_linear + p.slot) * (long long)(kTaps - 1) * C;
    const float a0 = tail[ca], a1 = tail[C + ca], a2 = tail[2 * C + ca];
    float b0 = 0.0f, b1 = 0.0f, b2 = 0.0f;
    if (has_v) {
        b0 = tail[cb];
        b1 = tail[C + cb];
        b2 = tail[2 * C + cb];
    }

    // ---- 1. state tile of this thread: columns 4 cg .. +3, rows kRowsPer rg .. +kRowsPer-1 (a row group of 32
    // threads reads 512 contiguous bytes per row). Non-temporal: the head's state is read once and written once per
    // step (streamed past the caches, same bits)
    const int cg = t & 31, rg = t >> 5;
    float4 s[kRowsPer];
#pragma unroll
    for (int r = 0; r < kRowsPer; ++r) {
        const f32x4 v = __builtin_nontemporal_load(
            reinterpret_cast<const f32x4*>(Sh + (kRowsPer * rg + r) * kDV + 4 * cg));
        s[r] = make_float4(v[0], v[1], v[2], v[3]);
    }

    // ---- 2. causal conv (taps 0..2 = tail, tap 3 = current token) + SiLU for the head's 384 channels
    auto conv = [](float h0, float h1, float h2, float x, float4 w) {
        float y = __fmul_rn(h0, w.x);
        y = __fadd_rn(y, __fmul_rn(h1, w.y));
        y = __fadd_rn(y, __fmul_rn(h2, w.z));
        y = __fadd_rn(y, __fmul_rn(x, w.w));
        return y / (1.0f + expf(-y));
    };
    us[t] = conv(a0, a1, a2, xa, wa);
    tail[ca] = a1;
    tail[C + ca] = a2;
    tail[2 * C + ca] = xa;
    if (has_v) {
        us[2 * kDK + t] = conv(b0, b1, b2, xb, wb);
        tail[cb] = b1;
        tail[C + cb] = b2;
        tail[2 * C + cb] = xb;
    }
    __syncthreads();

    // ---- 3. l2 norms of q and k (sum of squares + 1e-6), q scale 1/sqrt(dk); gate parameters
    {
        const float x = us[t];
        const float sq = wave_sum(__fmul_rn(x, x));
        if ((t & 63) == 0) wsum[t >> 6] = sq;
    }
    __syncthreads();
    if (t < kDK) {
        const float inv_q = 1.0f / sqrtf(wsum[0] + wsum[1] + 1e-6f);
        const float inv_k = 1.0f / sqrtf(wsum[2] + wsum[3] + 1e-6f);
        qn[t] = __fmul_rn(__fmul_rn(us[t], inv_q), 1.0f / sqrtf((float)kDK));
        kn[t] = __fmul_rn(us[kDK + t], inv_k);
    }
    const float beta = 1.0f / (1.0f + expf(-b_in));
    const float ab = a_in + dtb;
    const float sp = ab > 20.0f ? ab : log1pf(expf(ab));
    const float g = -expf(alog) * sp;
    const float decay = expf(g);
    __syncthreads();

    // ---- 4. decay, kv = k^T S (decayed), delta = beta * (v - kv)
    float kvp[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int r = 0; r < kRowsPer; ++r) {
        const float kr = kn[kRowsPer * rg + r];
        s[r].x = __fmul_rn(s[r].x, decay);
        s[r].y = __fmul_rn(s[r].y, decay);
        s[r].z = __fmul_rn(s[r].z, decay);
        s[r].w = __fmul_rn(s[r].w, decay);
        kvp[0] = fmaf(s[r].x, kr, kvp[0]);
        kvp[1] = fmaf(s[r].y, kr, kvp[1]);
        kvp[2] = fmaf(s[r].z, kr, kvp[2]);
        kvp[3] = fmaf(s[r].w, kr, kvp[3]);
    }
    *reinterpret_cast<float4*>(&red[rg][4 * cg]) = make_float4(kvp[0], kvp[1], kvp[2], kvp[3]);
    __syncthreads();
    if (t < kDV) {
        float kv = 0.0f;
#pragma unroll
        for (int r = 0; r < kRowGroups; ++r) kv += red[r][t];
        dl[t] = __fmul_rn(us[2 * kDK + t] - kv, beta);
    }
    __syncthreads();

    // ---- 5. S += k delta^T (written back), o = q^T S (updated state)
    const float4 d4 = *reinterpret_cast<const float4*>(&dl[4 * cg]);
    float op[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int r = 0; r < kRowsPer; ++r) {
        const float kr = kn[kRowsPer * rg + r], qr = qn[kRowsPer * rg + r];
        s[r].x = __fadd_rn(s[r].x, __fmul_rn(kr, d4.x));
        s[r].y = __fadd_rn(s[r].y, __fmul_rn(kr, d4.y));
        s[r].z = __fadd_rn(s[r].z, __fmul_rn(kr, d4.z));
        s[r].w = __fadd_rn(s[r].w, __fmul_rn(kr, d4.w));
        __builtin_nontemporal_store((f32x4{s[r].x, s[r].y, s[r].z, s[r].w}),
                                    reinterpret_cast<f32x4*>(Sh + (kRowsPer * rg + r) * kDV + 4 * cg));
        op[0] = fmaf(s[r].x, qr, op[0]);
        op[1] = fmaf(s[r].y, qr, op[1]);
        op[2] = fmaf(s[r].z, qr, op[2]);
        op[3] = fmaf(s[r].w, qr, op[3]);
    }
    *reinterpret_cast<float4*>(&red[rg][4 * cg]) = make_float4(op[0], op[1], op[2], op[3]);
    __syncthreads();

    // ---- 6. gated RMSNorm over dv: o * rsqrt(mean(o^2) + eps) * w * silu(z)
    float o = 0.0f;
    if (t < kDV) {
#pragma unroll
        for (int r = 0; r < kRowGroups; ++r) o += red[r][t];
        const float sq = wave_sum(__fmul_rn(o, o));
        if ((t & 63) == 0) wsum[4 + (t >> 6)] = sq;
    }
    __syncthreads();
    if (t < kDV) {
        const float rstd = 1.0f / sqrtf((wsum[4] + wsum[5]) / (float)kDV + p.eps);
        const float silu = zj / (1.0f + expf(-zj));
        p.out[(long long)bi * H * kDV + h * kDV + t] = __fmul_rn(__fmul_rn(__fmul_rn(o, rstd), nw), silu);
    }
}

}  // namespace
}  // namespace rk

using namespace rk;

extern "C" {

int rk_deltanet_decode(float* out, const float* qkv, const float* z, const float* b, const float* a, long long qkv_ld,
                       long long z_ld, long long ba_ld, float* conv_state, float* S, const float* conv_w,
                       const float* A_log, const float* dt_bias, const float* norm_w, const int32_t* seq_index, int B,
                       int H, int dk, int dv, int conv_k, int n_linear, int slot, float eps, void* stream) {
    if (!out || !qkv || !z || !b || !a || !conv_state || !S || !conv_w || !A_log || !dt_bias || !norm_w || !seq_index)
        return fail(RK_ERR_ARG, "rk_deltanet_decode: null pointer");
    if (B < 1 || H < 1 || n_linear < 1 || slot < 0 || slot >= n_linear)
        return fail(RK_ERR_ARG, "rk_deltanet_decode: B %d H %d n_linear %d slot %d", B, H, n_linear, slot);
    if (dk != kDK || dv != kDV || conv_k != kTaps)
        return fail(RK_ERR_UNSUPPORTED, "rk_deltanet_decode: dk %d dv %d conv kernel %d (built for 128/128/4)", dk, dv,
                    conv_k);
    if (qkv_ld < 2LL * H * dk + (long long)H * dv || z_ld < (long long)H * dv || ba_ld < H)
        return fail(RK_ERR_ARG, "rk_deltanet_decode: row strides qkv %lld, z %lld, b / a %lld below the rows", qkv_ld,
                    z_ld, ba_ld);
    StepArgs p;
    p.out = out; p.qkv = qkv; p.z = z; p.b = b; p.a = a; p.qkv_ld = qkv_ld; p.z_ld = z_ld; p.ba_ld = ba_ld;
    p.conv = conv_state; p.S = S; p.conv_w = conv_w;
    p.A_log = A_log; p.dt_bias = dt_bias; p.norm_w = norm_w; p.seq = seq_index;
    p.B = B; p.H = H; p.C = 2 * H * dk + H * dv; p.n_linear = n_linear; p.slot = slot; p.eps = eps;
    hipLaunchKernelGGL(deltanet_step_kernel, dim3(B * H), dim3(kThreads), 0, static_cast<hipStream_t>(stream), p);
    return check_launch("deltanet_step");
}

}  // extern "C"
