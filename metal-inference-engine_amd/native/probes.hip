// Measurement probes: what the memory system gives for the access patterns of the two decode kernels, with no
// arithmetic. They bound what the kernels can reach and are not on the path (no counterpart in the reference).
//
//   probe_block_stream: reads whole 16-position KV tiles (both pools) given as a list of pool tile offsets, in the
//     list's order, with 16-byte non-temporal loads (as the decode kernel reads them), and keeps an xor of everything
//     read. With the decode's own tiles in table order this is the paged decode's K/V traffic (scattered 16 KiB
//     blocks) without the softmax or the merge; with the same tiles sorted by address it is a near-sequential stream
//     of the same bytes. Either as persistent waves striding over the list, or as one-shot workgroups over
//     consecutive runs of it.
//   probe_state_rmw: reads each selected (sequence, head) state block of the DeltaNet pool, scales it, and writes it
//     back with non-temporal loads and stores (as the step kernel does): the recurrent step's state traffic (one
//     read and one write of 64 KiB per head) without the conv, norms or delta rule, with `split` workgroups per head.
#include "rk_device.h"
#include "rk_internal.h"

namespace rk {
namespace {

constexpr int kProbeWaves = 8;

// Each wave takes tiles w, w + waves, ... of the list; a tile is 64 * kVec * 16 contiguous bytes at the listed
// offset in each pool (kVec 16-byte loads per lane and pool, all issued before any is used).
template <int kVec>
__global__ __launch_bounds__(64 * kProbeWaves) void probe_block_stream(const char* kp, const char* vp,
                                                                        const long long* tiles, int n_tiles,
                                                                        uint32_t* sink) {
    const int lane = threadIdx.x & 63;
    const int wave = blockIdx.x * kProbeWaves + (threadIdx.x >> 6);
    const int waves = gridDim.x * kProbeWaves;
    uint32_t acc = 0;
    for (int t = wave; t < n_tiles; t += waves) {
        const long long off = tiles[t] + 16ll * lane;
        u32x4 x[2 * kVec];
#pragma unroll
        for (int j = 0; j < kVec; ++j) {
            x[j] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(kp + off + 1024ll * j));
            x[kVec + j] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(vp + off + 1024ll * j));
        }
#pragma unroll
        for (int j = 0; j < 2 * kVec; ++j) acc ^= x[j][0] ^ x[j][1] ^ x[j][2] ^ x[j][3];
    }
    sink[blockIdx.x * blockDim.x + threadIdx.x] = acc;
}

// One-shot workgroups: workgroup w reads list entries [w * per_group, (w + 1) * per_group), its waves taking
// consecutive entries in turn (one tile per wave in flight), and exits; the hardware dispatcher hands the next
// workgroup to whichever compute unit frees a slot first.
template <int kVec>
__global__ __launch_bounds__(64 * kProbeWaves) void probe_block_oneshot(const char* kp, const char* vp,
                                                                         const long long* tiles, int n_tiles,
                                                                         int per_group, uint32_t* sink) {
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int t0 = blockIdx.x * per_group, t1 = min(n_tiles, t0 + per_group);
    uint32_t acc = 0;
    for (int t = t0 + wave; t < t1; t += kProbeWaves) {
        const long long off = tiles[t] + 16ll * lane;
        u32x4 x[2 * kVec];
#pragma unroll
        for (int j = 0; j < kVec; ++j) {
            x[j] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(kp + off + 1024ll * j));
            x[kVec + j] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(vp + off + 1024ll * j));
        }
#pragma unroll
        for (int j = 0; j < 2 * kVec; ++j) acc ^= x[j][0] ^ x[j][1] ^ x[j][2] ^ x[j][3];
    }
    if (acc == 0x9e3779b9u) sink[threadIdx.x] = acc;     // keeps the loads; practically never stores
}

// One workgroup of 256 threads per (batch row, head, part): part p of `split` covers state rows
// [p * dk / split, (p + 1) * dk / split) of the head's dk x dv block.
__global__ __launch_bounds__(256) void probe_state_rmw(float* S, const int32_t* seq_index, int n_linear, int slot,
                                                       int H, int dk, int dv, int split, float scale) {
    const int part = blockIdx.x % split;
    const int h = (blockIdx.x / split) % H;
    const int b = blockIdx.x / (split * H);
    const long long head = (((long long)seq_index[b] * n_linear + slot) * H + h) * dk * dv;
    const int n4 = dk * dv / 4 / split;
    f32x4* p = reinterpret_cast<f32x4*>(S + head) + (long long)part * n4;
    constexpr int kMax = 16;                    // f32x4 per thread held at once (64 KiB / 256 threads)
    f32x4 x[kMax];
#pragma unroll
    for (int i = 0; i < kMax; ++i)
        if (threadIdx.x + 256 * i < n4) x[i] = __builtin_nontemporal_load(p + threadIdx.x + 256 * i);
#pragma unroll
    for (int i = 0; i < kMax; ++i)
        if (threadIdx.x + 256 * i < n4) __builtin_nontemporal_store(x[i] * scale, p + threadIdx.x + 256 * i);
}

}  // namespace
}  // namespace rk

using namespace rk;

extern "C" {

int rk_probe_block_stream(const void* k_pool, const void* v_pool, const long long* tile_offsets, int n_tiles,
                          int tile_bytes, int workgroups, int tiles_per_group, uint32_t* sink, void* stream) {
    if (!k_pool || !v_pool || !tile_offsets || !sink || n_tiles < 1 || (tiles_per_group <= 0 && workgroups < 1))
        return fail(RK_ERR_ARG, "rk_probe_block_stream: null pointer or empty list");
    if (tile_bytes != 16384 && tile_bytes != 8192 && tile_bytes != 4096)
        return fail(RK_ERR_ARG, "rk_probe_block_stream: tile_bytes %d (4096, 8192 or 16384)", tile_bytes);
    const hipStream_t s = static_cast<hipStream_t>(stream);
    const char* kp = static_cast<const char*>(k_pool);
    const char* vp = static_cast<const char*>(v_pool);
    if (tiles_per_group > 0) {
        typedef void (*Fn)(const char*, const char*, const long long*, int, int, uint32_t*);
        Fn fn = tile_bytes == 16384 ? probe_block_oneshot<16> : tile_bytes == 8192 ? probe_block_oneshot<8>
                                                                                   : probe_block_oneshot<4>;
        const int grid = (n_tiles + tiles_per_group - 1) / tiles_per_group;
        hipLaunchKernelGGL(fn, dim3(grid), dim3(64 * kProbeWaves), 0, s, kp, vp, tile_offsets, n_tiles,
                           tiles_per_group, sink);
        return check_launch("probe_block_oneshot");
    }
    typedef void (*Fn)(const char*, const char*, const long long*, int, uint32_t*);
    Fn fn = tile_bytes == 16384 ? probe_block_stream<16> : tile_bytes == 8192 ? probe_block_stream<8>
                                                                              : probe_block_stream<4>;
    hipLaunchKernelGGL(fn, dim3(workgroups), dim3(64 * kProbeWaves), 0, s, kp, vp, tile_offsets, n_tiles, sink);
    return check_launch("probe_block_stream");
}

int rk_probe_state_rmw(float* S, const int32_t* seq_index, int B, int n_linear, int slot, int H, int dk, int dv,
                       int split, float scale, void* stream) {
    if (!S || !seq_index || B < 1 || H < 1 || n_linear < 1 || slot < 0 || slot >= n_linear)
        return fail(RK_ERR_ARG, "rk_probe_state_rmw: bad arguments");
    if (split < 1 || (dk * dv / 4) % split || dk * dv / 4 / split > 16 * 256)
        return fail(RK_ERR_ARG, "rk_probe_state_rmw: split %d of a %d x %d block", split, dk, dv);
    hipLaunchKernelGGL(probe_state_rmw, dim3(B * H * split), dim3(256), 0, static_cast<hipStream_t>(stream), S,
                       seq_index, n_linear, slot, H, dk, dv, split, scale);
    return check_launch("probe_state_rmw");
}

}  // extern "C"
