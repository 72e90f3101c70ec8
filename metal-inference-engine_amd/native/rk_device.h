// Device-side helpers shared by the token-mixing kernels (gfx950 / CDNA4 only).
//
// Conventions used by every kernel in this directory:
//   * A wavefront is 64 lanes. Workgroup sizes are multiples of 64.
//   * bf16 values are carried as raw 16-bit patterns (uint16_t) in memory and widened to fp32 by a shift, which is
//     exact. fp32 -> bf16 narrowing is round-to-nearest-even with NaN kept quiet (the same rule as torch's
//     Tensor.to(torch.bfloat16)).
//   * MFMA operands are 8 x bf16 per lane (v_mfma_f32_16x16x32_bf16): lane l supplies row / column (l % 16) and the
//     k-slot group (l / 16); the accumulator lane l, element i holds D[4 * (l / 16) + i][l % 16].
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace rk {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kWave = 64;
constexpr float kLog2e = 1.4426950408889634f;

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t h16) { return __uint_as_float(h16 << 16); }
__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// fp32 -> bf16 bits, round to nearest even; NaN -> canonical quiet NaN.
__device__ __forceinline__ uint16_t f32_to_bf16_rne(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)0x7fc0u;
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

// Two fp32 values -> packed bf16 pair (element 0 in the low 16 bits), round to nearest even: one
// v_cvt_pk_bf16_f32 on gfx950. For finite inputs this is the rule of f32_to_bf16_rne.
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pack_bf16x2_rne(float x0, float x1) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t{x0, x1}), bf16x2_t));
}

// Pack the top halves (truncated bf16 patterns) of two fp32 bit patterns: element 0 in the low 16 bits. One
// v_perm_b32: result bytes = bytes 2, 3 of e0 then bytes 2, 3 of e1 (selectors 4..7 address the first operand).
__device__ __forceinline__ uint32_t pack_hi2(uint32_t e0, uint32_t e1) {
    return __builtin_amdgcn_perm(e1, e0, 0x07060302u);
}

// Exact three-way split of an fp32 value into bf16-representable parts x = hi + mid + lo (truncation at every
// step: hi keeps sign, exponent and the top 7 mantissa bits; the remainder has at most 16 significant bits, so its
// truncated top part and the final rest are exact in bf16). Returned as fp32 bit patterns: hi and mid with low halves
// 0; lo is the final rest as is, whose low half is 0 as well (it is exact in bf16), and which is only ever packed
// by its top half (pack_hi2), so no mask is spent on it.
struct Split3 {
    uint32_t hi, mid, lo;
};
__device__ __forceinline__ Split3 split3(float x) {
    uint32_t hb = __float_as_uint(x) & 0xffff0000u;
    float r1 = x - __uint_as_float(hb);
    uint32_t mb = __float_as_uint(r1) & 0xffff0000u;
    float r2 = r1 - __uint_as_float(mb);
    return {hb, mb, __float_as_uint(r2)};
}

__device__ __forceinline__ bf16x8 as_bf16x8(u32x4 v) { return __builtin_bit_cast(bf16x8, v); }

__device__ __forceinline__ f32x4 mfma16x16x32(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(a), as_bf16x8(b), c, 0, 0, 0);
}

// Butterfly reductions inside one row of 16 lanes (DPP row rotations; every lane of the row gets the result).
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float x) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xf, 0xf, false));
}
__device__ __forceinline__ float row16_max(float x) {
    x = fmaxf(x, dpp_f32<0x128>(x));   // row_ror:8
    x = fmaxf(x, dpp_f32<0x124>(x));   // row_ror:4
    x = fmaxf(x, dpp_f32<0x122>(x));   // row_ror:2
    x = fmaxf(x, dpp_f32<0x121>(x));   // row_ror:1
    return x;
}
__device__ __forceinline__ float row16_sum(float x) {
    x += dpp_f32<0x128>(x);
    x += dpp_f32<0x124>(x);
    x += dpp_f32<0x122>(x);
    x += dpp_f32<0x121>(x);
    return x;
}

__device__ __forceinline__ float wave_sum(float x) {
    x = row16_sum(x);
    x += __shfl_xor(x, 16);
    x += __shfl_xor(x, 32);
    return x;
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Ordering point for LDS data exchanged between the lanes of ONE wave (a wave-private LDS region). The LDS unit
// executes a wave's instructions in order, so only the compiler has to be kept from moving accesses across it;
// unlike __syncthreads() it does not wait for the wave's outstanding global loads.
__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Workgroup barrier ordering LDS only: outstanding global loads are not waited for.
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

}  // namespace rk
