// Paged KV cache scatter (write) and gather (read), gfx950.
//
// rk_kv_write: pool[slot / bs, slot % bs] = src (K and V), converting to the pool's element type. This is
//   PagedKVPool.write_batch / PagedSequence.write (src/state.py:131-134, 163-170): an index_put over (block, offset).
// rk_kv_gather: the rows of positions lo..end-1 of one sequence, gathered through its block table into a contiguous
//   [end - lo, Hkv, D] buffer; PagedSequence.read (src/state.py:172-180). A pure copy, bit-exact by construction.
// One thread moves 8 elements; a row of Hkv * D elements is contiguous in the pool, so a wave covers 512 contiguous
// bytes (bf16) and loads / stores are fully coalesced. Slots and table entries are bounds-checked: an out-of-range
// slot is skipped (write) and an out-of-range table entry yields a zero row (gather); neither touches memory
// outside the pool.
#include "rk_device.h"
#include "rk_internal.h"

namespace rk {
namespace {

template <typename S>
__device__ __forceinline__ void load8(const S* p, float* f);
template <>
__device__ __forceinline__ void load8<float>(const float* p, float* f) {
    const float4 a = reinterpret_cast<const float4*>(p)[0];
    const float4 b = reinterpret_cast<const float4*>(p)[1];
    f[0] = a.x; f[1] = a.y; f[2] = a.z; f[3] = a.w; f[4] = b.x; f[5] = b.y; f[6] = b.z; f[7] = b.w;
}
template <>
__device__ __forceinline__ void load8<uint16_t>(const uint16_t* p, float* f) {
    const u32x4 w = *reinterpret_cast<const u32x4*>(p);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        f[2 * j] = bf16_lo(w[j]);
        f[2 * j + 1] = bf16_hi(w[j]);
    }
}

template <typename P>
__device__ __forceinline__ void store8(P* p, const float* f);
template <>
__device__ __forceinline__ void store8<float>(float* p, const float* f) {
    reinterpret_cast<float4*>(p)[0] = make_float4(f[0], f[1], f[2], f[3]);
    reinterpret_cast<float4*>(p)[1] = make_float4(f[4], f[5], f[6], f[7]);
}
template <>
__device__ __forceinline__ void store8<uint16_t>(uint16_t* p, const float* f) {
    u32x4 w;
#pragma unroll
    for (int j = 0; j < 4; ++j)
        w[j] = (uint32_t)f32_to_bf16_rne(f[2 * j]) | ((uint32_t)f32_to_bf16_rne(f[2 * j + 1]) << 16);
    *reinterpret_cast<u32x4*>(p) = w;
}

// grid: (ceil(n * row / 8 / 256)), row = Hkv * D elements
template <typename P, typename S>
__global__ __launch_bounds__(256) void kv_write_kernel(P* kp, P* vp, const int64_t* slots, const S* ks, const S* vs,
                                                       int n, int row, int bs, int num_blocks) {
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    const int per_row = row / 8;
    if (i >= (long long)n * per_row) return;
    const int r = (int)(i / per_row), c = (int)(i % per_row) * 8;
    const long long slot = slots[r];
    if (slot < 0 || slot >= (long long)num_blocks * bs) return;
    float f[8];
    load8<S>(ks + (long long)r * row + c, f);
    store8<P>(kp + slot * row + c, f);
    load8<S>(vs + (long long)r * row + c, f);
    store8<P>(vp + slot * row + c, f);
}

template <typename P>
__global__ __launch_bounds__(256) void kv_gather_kernel(P* ko, P* vo, const P* kp, const P* vp, const int32_t* table,
                                                        int table_len, int lo, int end, int row, int bs,
                                                        int num_blocks) {
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    const int per_row = row / 8;
    if (i >= (long long)(end - lo) * per_row) return;
    const int t = lo + (int)(i / per_row), c = (int)(i % per_row) * 8;
    const int j = t / bs;
    const int blk = j < table_len ? table[j] : -1;
    u32x4 kw = {0u, 0u, 0u, 0u}, vw = {0u, 0u, 0u, 0u};
    u32x4 kw2 = kw, vw2 = kw;
    const bool ok = blk >= 0 && blk < num_blocks;
    const long long src = ((long long)blk * bs + t % bs) * row + c;
    const long long dst = (long long)(t - lo) * row + c;
    if (sizeof(P) == 2) {
        if (ok) {
            kw = *reinterpret_cast<const u32x4*>(kp + src);
            vw = *reinterpret_cast<const u32x4*>(vp + src);
        }
        *reinterpret_cast<u32x4*>(ko + dst) = kw;
        *reinterpret_cast<u32x4*>(vo + dst) = vw;
    } else {
        if (ok) {
            kw = reinterpret_cast<const u32x4*>(kp + src)[0];
            kw2 = reinterpret_cast<const u32x4*>(kp + src)[1];
            vw = reinterpret_cast<const u32x4*>(vp + src)[0];
            vw2 = reinterpret_cast<const u32x4*>(vp + src)[1];
        }
        reinterpret_cast<u32x4*>(ko + dst)[0] = kw;
        reinterpret_cast<u32x4*>(ko + dst)[1] = kw2;
        reinterpret_cast<u32x4*>(vo + dst)[0] = vw;
        reinterpret_cast<u32x4*>(vo + dst)[1] = vw2;
    }
}

}  // namespace
}  // namespace rk

using namespace rk;

extern "C" {

int rk_kv_write(void* k_pool, void* v_pool, int pool_dtype, const int64_t* slots, const void* k_src,
                const void* v_src, int src_dtype, int n, int Hkv, int D, int block_size, int num_blocks,
                void* stream) {
    if (n == 0) return RK_OK;
    if (!k_pool || !v_pool || !slots || !k_src || !v_src) return fail(RK_ERR_ARG, "rk_kv_write: null pointer");
    if (n < 0 || Hkv < 1 || D < 8 || D % 8 || block_size < 1 || num_blocks < 1)
        return fail(RK_ERR_ARG, "rk_kv_write: n %d, Hkv %d, D %d, block_size %d, num_blocks %d", n, Hkv, D,
                    block_size, num_blocks);
    if ((pool_dtype != RK_F32 && pool_dtype != RK_BF16) || (src_dtype != RK_F32 && src_dtype != RK_BF16))
        return fail(RK_ERR_UNSUPPORTED, "rk_kv_write: dtypes pool %d src %d", pool_dtype, src_dtype);
    const int row = Hkv * D;
    const long long threads = (long long)n * (row / 8);
    const dim3 grid((unsigned)ceil_div((size_t)threads, 256)), block(256);
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (pool_dtype == RK_BF16 && src_dtype == RK_F32)
        hipLaunchKernelGGL((kv_write_kernel<uint16_t, float>), grid, block, 0, s, (uint16_t*)k_pool,
                           (uint16_t*)v_pool, slots, (const float*)k_src, (const float*)v_src, n, row, block_size,
                           num_blocks);
    else if (pool_dtype == RK_BF16)
        hipLaunchKernelGGL((kv_write_kernel<uint16_t, uint16_t>), grid, block, 0, s, (uint16_t*)k_pool,
                           (uint16_t*)v_pool, slots, (const uint16_t*)k_src, (const uint16_t*)v_src, n, row,
                           block_size, num_blocks);
    else if (src_dtype == RK_F32)
        hipLaunchKernelGGL((kv_write_kernel<float, float>), grid, block, 0, s, (float*)k_pool, (float*)v_pool, slots,
                           (const float*)k_src, (const float*)v_src, n, row, block_size, num_blocks);
    else
        hipLaunchKernelGGL((kv_write_kernel<float, uint16_t>), grid, block, 0, s, (float*)k_pool, (float*)v_pool,
                           slots, (const uint16_t*)k_src, (const uint16_t*)v_src, n, row, block_size, num_blocks);
    return check_launch("kv_write");
}

int rk_kv_gather(void* k_out, void* v_out, const void* k_pool, const void* v_pool, int dtype, const int32_t* table,
                 int table_len, int lo, int end, int Hkv, int D, int block_size, int num_blocks, void* stream) {
    if (end == lo) return RK_OK;
    if (!k_out || !v_out || !k_pool || !v_pool || !table) return fail(RK_ERR_ARG, "rk_kv_gather: null pointer");
    if (lo < 0 || end < lo || Hkv < 1 || D < 8 || D % 8 || block_size < 1 || num_blocks < 1 || table_len < 0)
        return fail(RK_ERR_ARG, "rk_kv_gather: lo %d end %d Hkv %d D %d block_size %d", lo, end, Hkv, D, block_size);
    if ((long long)(end - 1) / block_size >= table_len)
        return fail(RK_ERR_ARG, "rk_kv_gather: position %d needs table entry %d, table has %d", end - 1,
                    (end - 1) / block_size, table_len);
    const int row = Hkv * D;
    const long long threads = (long long)(end - lo) * (row / 8);
    const dim3 grid((unsigned)ceil_div((size_t)threads, 256)), block(256);
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (dtype == RK_BF16)
        hipLaunchKernelGGL(kv_gather_kernel<uint16_t>, grid, block, 0, s, (uint16_t*)k_out, (uint16_t*)v_out,
                           (const uint16_t*)k_pool, (const uint16_t*)v_pool, table, table_len, lo, end, row,
                           block_size, num_blocks);
    else if (dtype == RK_F32)
        hipLaunchKernelGGL(kv_gather_kernel<float>, grid, block, 0, s, (float*)k_out, (float*)v_out,
                           (const float*)k_pool, (const float*)v_pool, table, table_len, lo, end, row, block_size,
                           num_blocks);
    else
        return fail(RK_ERR_UNSUPPORTED, "rk_kv_gather: dtype %d", dtype);
    return check_launch("kv_gather");
}

}  // extern "C"
