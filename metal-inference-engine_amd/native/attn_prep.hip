// What a gated-attention layer does to its projection output before attention, in one launch, gfx950:
// the per-head q / k RMSNorm with (1 + w) weights, the partial RoPE over the first `rot` dims, and (decode) the write
// of the new K / V rows into the paged pool.
//
// Semantics (reference): src/models/qwen3_5.py:251-262 (decode; :100-110 for a packed prefill):
//   q = rms_norm(y[:, :Hq d], 1 + q_w), k = rms_norm(y[:, Hq d:(Hq+Hkv) d], 1 + k_w)     (src/ops.py:7-15:
//       x / sqrt(mean x^2 + eps) * w, per head of d values)
//   qk = rope(cat(q[..., :rot], k[..., :rot]), positions, theta); q, k = cat(qk part, rest)   (src/ops.py:27-54: the
//       HF rotate_half pairing (i, i + rot/2) with inv_freq = 1 / theta^(i / (rot/2)), host-computed in fp32)
//   kv_pool.write_batch(layer, blocks, offsets, k, v)      (src/state.py:131-134: k.to(pool dtype), v.to(pool dtype))
// One wave per (token, 1 or 4 of the Hq q heads, Hkv k heads and Hkv v heads); lane l holds elements EPL*l ..
// EPL*l + EPL-1 (d = 64 EPL) of each. The RoPE partner of element e < rot is e +- rot/2, which lives rot/(2 EPL)
// lanes away: one xor-shuffle. The norm's square root and division and the angle's cos / sin are the correctly
// rounded / library routines (this kernel is latency- or bandwidth-bound, never VALU-bound), and the rotation keeps
// the reference's separate roundings: a cos - b sin, a sin + b cos.
#include "rk_device.h"
#include "rk_internal.h"

namespace rk {
namespace {

struct PrepArgs {
    float* q_out;               // [N, Hq, d] fp32
    float* k_out;               // [N, Hkv, d] fp32, or null
    float* v_out;               // [N, Hkv, d] fp32, or null
    void* k_pool;               // [pool_rows, Hkv, d] pool_dtype (one layer, rows = num_blocks * block_size), or null
    void* v_pool;
    const int64_t* slots;       // [N]: pool row block * block_size + offset of each token
    long long pool_rows;
    const void* y;              // row n at y + n * ld: [Hq d | Hkv d | Hkv d | ...] in y_dtype
    long long ld;
    const float* q_w;           // [d] (1 + q_norm.weight)
    const float* k_w;           // [d] (1 + k_norm.weight)
    const int32_t* pos;         // [N]
    const float* inv_freq;      // [rot / 2]
    float eps;
    int rot, N, Hq, Hkv, y_dtype, pool_dtype;
};

template <int EPL>
__device__ __forceinline__ void load_row(float (&x)[EPL], const void* p, long long off, int dt) {
    if (dt == RK_BF16) {
        const uint16_t* s = reinterpret_cast<const uint16_t*>(p) + off;
        if constexpr (EPL == 1) {
            x[0] = bf16_bits_to_f32(*s);
        } else if constexpr (EPL == 2) {
            const uint32_t w = *reinterpret_cast<const uint32_t*>(s);
            x[0] = bf16_lo(w); x[1] = bf16_hi(w);
        } else {
            const u32x2 w = *reinterpret_cast<const u32x2*>(s);
            x[0] = bf16_lo(w.x); x[1] = bf16_hi(w.x); x[2] = bf16_lo(w.y); x[3] = bf16_hi(w.y);
        }
    } else {
        const float* s = reinterpret_cast<const float*>(p) + off;
        if constexpr (EPL == 1) {
            x[0] = *s;
        } else if constexpr (EPL == 2) {
            const float2 v = *reinterpret_cast<const float2*>(s);
            x[0] = v.x; x[1] = v.y;
        } else {
            const float4 v = *reinterpret_cast<const float4*>(s);
            x[0] = v.x; x[1] = v.y; x[2] = v.z; x[3] = v.w;
        }
    }
}

template <int EPL>
__device__ __forceinline__ void store_f32(float* p, const float (&x)[EPL]) {
    if constexpr (EPL == 1) *p = x[0];
    else if constexpr (EPL == 2) *reinterpret_cast<float2*>(p) = make_float2(x[0], x[1]);
    else *reinterpret_cast<float4*>(p) = make_float4(x[0], x[1], x[2], x[3]);
}
// outputs the next kernel reads once: non-temporal (streaming) stores
template <int EPL>
__device__ __forceinline__ void stream_f32(float* p, const float (&x)[EPL]) {
    if constexpr (EPL == 1) __builtin_nontemporal_store(x[0], p);
    else if constexpr (EPL == 2) __builtin_nontemporal_store((f32x2_t{x[0], x[1]}), reinterpret_cast<f32x2_t*>(p));
    else __builtin_nontemporal_store((f32x4{x[0], x[1], x[2], x[3]}), reinterpret_cast<f32x4*>(p));
}

// a pool row in its dtype: fp32 as is, bf16 rounded to nearest even (torch's .to(torch.bfloat16))
template <int EPL>
__device__ __forceinline__ void store_pool(void* pool, long long off, int dt, const float (&x)[EPL]) {
    if (dt == RK_BF16) {
        uint16_t* d = reinterpret_cast<uint16_t*>(pool) + off;
        if constexpr (EPL == 1) {
            *d = f32_to_bf16_rne(x[0]);
        } else if constexpr (EPL == 2) {
            *reinterpret_cast<uint32_t*>(d) =
                (uint32_t)f32_to_bf16_rne(x[0]) | ((uint32_t)f32_to_bf16_rne(x[1]) << 16);
        } else {
            u32x2 w;
            w.x = (uint32_t)f32_to_bf16_rne(x[0]) | ((uint32_t)f32_to_bf16_rne(x[1]) << 16);
            w.y = (uint32_t)f32_to_bf16_rne(x[2]) | ((uint32_t)f32_to_bf16_rne(x[3]) << 16);
            *reinterpret_cast<u32x2*>(d) = w;
        }
    } else {
        store_f32<EPL>(reinterpret_cast<float*>(pool) + off, x);
    }
}

// One wave per (token, group of KH consecutive heads of the Hq + 2 Hkv): the group's rows are loaded before any
// arithmetic, and the rotation's cos / sin (which depend only on the token's position and the element) are computed
// once per wave for all of its q / k heads. KH = 4 for prefill-sized batches (bandwidth-bound: 1.6x faster than one
// head per wave at 10k tokens); KH = 1 for decode batches, where the shorter chain per wave wins (3.9 vs 6.0 us at
// 64 tokens).
template <int EPL, int kHeads>
__global__ __launch_bounds__(256) void attn_prep_kernel(PrepArgs p) {
    constexpr int d = 64 * EPL;
    const int lane = threadIdx.x & 63;
    const int HT = p.Hq + 2 * p.Hkv;
    const int groups = (HT + kHeads - 1) / kHeads;
    const long long w = (long long)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (w >= (long long)p.N * groups) return;        // whole waves
    const int n = (int)(w / groups), h0 = (int)(w % groups) * kHeads;
    const int nh = min(kHeads, HT - h0);
    const int e0 = EPL * lane;                       // first element of this lane
    float x[kHeads][EPL];
#pragma unroll
    for (int i = 0; i < kHeads; ++i)
        if (i < nh) load_row<EPL>(x[i], p.y, (long long)n * p.ld + (long long)(h0 + i) * d + e0, p.y_dtype);
    const long long slot = p.slots ? p.slots[n] : -1;

    // cos / sin of this lane's rotary elements (ops.py:27-54): angle = fp32(position * inv_freq[i]), i = e mod rot/2
    const int half = p.rot >> 1;
    float cs[EPL], sn[EPL];
    if (h0 < p.Hq + p.Hkv && p.rot > 0) {
        const float pf = (float)p.pos[n];
#pragma unroll
        for (int j = 0; j < EPL; ++j) {
            const int e = e0 + j;
            if (e < p.rot) {
                const float ang = __fmul_rn(pf, p.inv_freq[e < half ? e : e - half]);
                cs[j] = cosf(ang);
                sn[j] = sinf(ang);
            }
        }
    }

#pragma unroll
    for (int i = 0; i < kHeads; ++i) {
        if (i >= nh) break;
        const int h = h0 + i;
        const bool is_q = h < p.Hq, is_k = !is_q && h < p.Hq + p.Hkv;
        if (is_q || is_k) {
            // rms_norm (ops.py:7-15): x / sqrt(mean(x^2) + eps) * w
            float ss = 0.0f;
#pragma unroll
            for (int j = 0; j < EPL; ++j) ss = __fadd_rn(ss, __fmul_rn(x[i][j], x[i][j]));
            ss = wave_sum(ss);
            const float rms = sqrtf(__fadd_rn(ss * (1.0f / d), p.eps));     // d a power of 2: the mean is exact
            const float* wt = is_q ? p.q_w : p.k_w;
#pragma unroll
            for (int j = 0; j < EPL; ++j) x[i][j] = __fmul_rn(x[i][j] / rms, wt[e0 + j]);
            // partial RoPE on elements e < rot: (a, b) = (x[e], x[e + rot/2]) for e < rot/2; the partner is
            // rot / (2 EPL) lanes away (a power of 2)
            if (p.rot > 0) {
                const int mask = half / EPL;
#pragma unroll
                for (int j = 0; j < EPL; ++j) {
                    const float other = __shfl_xor(x[i][j], mask);
                    const int e = e0 + j;
                    if (e < p.rot)
                        x[i][j] = e < half ? __fsub_rn(__fmul_rn(x[i][j], cs[j]), __fmul_rn(other, sn[j]))
                                           : __fadd_rn(__fmul_rn(other, sn[j]), __fmul_rn(x[i][j], cs[j]));
                }
            }
        }
        if (is_q) {
            stream_f32<EPL>(p.q_out + ((long long)n * p.Hq + h) * d + e0, x[i]);
            continue;
        }
        const int kh = is_k ? h - p.Hq : h - p.Hq - p.Hkv;
        float* out = is_k ? p.k_out : p.v_out;
        if (out) stream_f32<EPL>(out + ((long long)n * p.Hkv + kh) * d + e0, x[i]);
        if (slot >= 0 && slot < p.pool_rows)         // out-of-range slots are skipped, as rk_kv_write does
            store_pool<EPL>(is_k ? p.k_pool : p.v_pool, (slot * p.Hkv + kh) * d + e0, p.pool_dtype, x[i]);
    }
}

}  // namespace
}  // namespace rk

using namespace rk;

extern "C" int rk_attn_prep(float* q_out, float* k_out, float* v_out, void* k_pool, void* v_pool, int pool_dtype,
                            const int64_t* slots, int num_blocks, int block_size, const void* y, int y_dtype,
                            long long ld, const float* q_w, const float* k_w, float eps, const int32_t* positions,
                            const float* inv_freq, int rot, int N, int Hq, int Hkv, int d, void* stream) {
    if (N == 0) return RK_OK;
    if (!q_out || !y || !q_w || !k_w || (rot > 0 && (!positions || !inv_freq)) ||
        (slots && (!k_pool || !v_pool)))
        return fail(RK_ERR_ARG, "rk_attn_prep: null pointer");
    if (d != 64 && d != 128 && d != 256) return fail(RK_ERR_UNSUPPORTED, "rk_attn_prep: head_dim %d", d);
    const int EPL = d / 64;
    // the pair partner must sit a power-of-2 number of lanes away: rot = 2 EPL 2^k, rot <= d
    const int half_lanes = rot / 2 / EPL;
    if (rot < 0 || rot > d || (rot > 0 && (rot % (2 * EPL) || (half_lanes & (half_lanes - 1)))))
        return fail(RK_ERR_UNSUPPORTED, "rk_attn_prep: rotary dims %d of %d (0 or 2 * %d * a power of 2)", rot, d,
                    EPL);
    if (N < 0 || Hq < 1 || Hkv < 1 || ld < (long long)(Hq + 2 * Hkv) * d ||
        (slots && (num_blocks < 1 || block_size < 1)))
        return fail(RK_ERR_ARG, "rk_attn_prep: N %d, heads %d / %d, row stride %lld, pool %d x %d", N, Hq, Hkv, ld,
                    num_blocks, block_size);
    if ((y_dtype != RK_F32 && y_dtype != RK_BF16) || (slots && pool_dtype != RK_F32 && pool_dtype != RK_BF16))
        return fail(RK_ERR_UNSUPPORTED, "rk_attn_prep: dtypes %d / %d", y_dtype, pool_dtype);
    const size_t ye = y_dtype == RK_BF16 ? 2 : 4;
    if (reinterpret_cast<uintptr_t>(y) % (EPL * ye) || ld % EPL)
        return fail(RK_ERR_ARG, "rk_attn_prep: projection rows must start %zu-byte aligned", EPL * ye);
    PrepArgs p;
    p.q_out = q_out; p.k_out = k_out; p.v_out = v_out; p.k_pool = k_pool; p.v_pool = v_pool; p.slots = slots;
    p.pool_rows = (long long)num_blocks * block_size; p.y = y; p.ld = ld; p.q_w = q_w; p.k_w = k_w;
    p.pos = positions; p.inv_freq = inv_freq; p.eps = eps; p.rot = rot; p.N = N; p.Hq = Hq; p.Hkv = Hkv;
    p.y_dtype = y_dtype; p.pool_dtype = pool_dtype;
    const bool wide = N >= 1024;
    const int KH = wide ? 4 : 1;
    const dim3 grid((unsigned)ceil_div((size_t)N * ceil_div((size_t)(Hq + 2 * Hkv), KH), 4));
    hipStream_t s = static_cast<hipStream_t>(stream);
    using PrepFn = void (*)(PrepArgs);
    PrepFn fn;
    if (EPL == 1) fn = wide ? attn_prep_kernel<1, 4> : attn_prep_kernel<1, 1>;
    else if (EPL == 2) fn = wide ? attn_prep_kernel<2, 4> : attn_prep_kernel<2, 1>;
    else fn = wide ? attn_prep_kernel<4, 4> : attn_prep_kernel<4, 1>;
    hipLaunchKernelGGL(fn, grid, dim3(256), 0, s, p);
    return check_launch("attn_prep");
}
