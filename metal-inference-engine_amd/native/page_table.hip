// Device-resident paged-KV bookkeeping: block tables, lengths and the free-block stack live in device memory, and
// a decode (or prefill-chunk) step's layout -- the pool rows the new tokens go to, the batch's block tables and
// lengths -- is produced by one small kernel with no host work and no host-to-device copy per step, so the whole
// step, layout included, can be captured in a HIP graph.
//
// Semantics kept from the reference (src/state.py:78-103, 148-157, 182-186):
//   * blocks come off a free stack whose initial order hands out block 0 first;
//   * a step's growth is all or nothing: if the free blocks cannot cover every sequence's missing blocks, nothing is
//     taken or written and the step reports out-of-blocks (the reference raises OutOfBlocks before any layer runs;
//     here a status word is set, read by the host when it checks);
//   * within a step, sequences take their blocks in batch order (sequence 0 first), as the reference's per-state
//     reserve loop does;
//   * a released sequence's blocks go back on the stack in reverse table order, so they are handed out again in
//     table order.
// Layout (int32, all device memory): tables [max_seqs, max_blocks] (row = sequence slot), lens [max_seqs],
// stack [num_blocks], meta[0] = free blocks on the stack, meta[1] = status (0 ok, 1 out of blocks, 2 a sequence
// would outgrow its table row, 3 a release would overfill the stack, 4 a row index outside [0, max_seqs), 5 a row named
// twice in one step: a double allocation or a double free, which the reference's allocator refuses). Row indices come
// from device memory, so every kernel checks them before it addresses anything with them.
#include "rk_device.h"
#include "rk_internal.h"

#include <algorithm>

namespace rk {
namespace {

constexpr int kPageThreads = 1024;

// Whether row rows[i] (i < n, this thread's entry, valid) also appears at an earlier entry: the n rows staged in LDS,
// each thread compares with the entries before its own. One LDS barrier; every thread must call it.
__device__ bool named_before(const int32_t* rows, int n, int i, bool valid, int row) {
    __shared__ int rs[kPageThreads];
    if (i < n) rs[i] = rows[i];
    __syncthreads();
    bool dup = false;
    if (valid)
        for (int j = 0; j < i; ++j) dup |= rs[j] == row;
    return dup;
}

// Exclusive prefix sum over the workgroup (kPageThreads threads); *total gets the sum. Two LDS barriers.
__device__ int block_exclusive_scan(int x, int* total) {
    __shared__ int wsum[kPageThreads / 64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    int inc = x;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const int y = __shfl_up(inc, off);
        if (lane >= off) inc += y;
    }
    if (lane == 63) wsum[wave] = inc;
    __syncthreads();
    int before = 0, all = 0;
    for (int w = 0; w < kPageThreads / 64; ++w) {
        const int s = wsum[w];
        before += w < wave ? s : 0;
        all += s;
    }
    __syncthreads();                      // wsum may be reused by a later scan
    *total = all;
    return before + inc - x;
}

struct PageArgs {
    int32_t* tables;
    int32_t* lens;
    int32_t* stack;
    int32_t* meta;
    const int32_t* rows;
    int64_t* slots;        // [B * n_new] or null
    int32_t* out_lens;     // [B] or null
    int max_seqs, max_blocks, block_size, B, n_new, num_blocks;
};

__global__ __launch_bounds__(kPageThreads) void pages_init(PageArgs a) {
    const int max_seqs = a.max_seqs;
    const long long n_tab = (long long)max_seqs * a.max_blocks;
    for (long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x; i < n_tab; i += (long long)gridDim.x * blockDim.x)
        a.tables[i] = 0;
    for (long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x; i < a.num_blocks;
         i += (long long)gridDim.x * blockDim.x)
        a.stack[i] = a.num_blocks - 1 - (int)i;
    for (long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x; i < max_seqs; i += (long long)gridDim.x * blockDim.x)
        a.lens[i] = 0;
    if (blockIdx.x == 0 && threadIdx.x == 0) {
        a.meta[0] = a.num_blocks;
        a.meta[1] = 0;
    }
}

// One workgroup: batch entry b (thread b) grows sequence rows[b] by n_new positions.
__global__ __launch_bounds__(kPageThreads) void pages_advance(PageArgs a) {
    __shared__ int s_fail;
    const int b = threadIdx.x;
    const int row_in = b < a.B ? a.rows[b] : 0;
    const bool bad_row = b < a.B && (row_in < 0 || row_in >= a.max_seqs);
    const bool live = b < a.B && !bad_row;
    const int row = live ? row_in : 0;
    const int pos_in = live ? a.lens[row] : 0;
    const bool bad_len = pos_in < 0;      // lengths are written by these kernels only; a negative one is refused
    const int pos = bad_len ? 0 : pos_in;
    const int end = pos + a.n_new;
    const int held = (pos + a.block_size - 1) / a.block_size;
    const int want = live ? (end + a.block_size - 1) / a.block_size : 0;
    const int need = live ? want - held : 0;
    const int top = a.meta[0];            // read by every thread before thread 0 rewrites it (after the barriers)
    if (threadIdx.x == 0) s_fail = 0;
    const bool dup = named_before(a.rows, a.B, b, live, row);     // its barrier also publishes s_fail = 0
    if ((live && want > a.max_blocks) || bad_len) atomicOr(&s_fail, 2);   // LDS atomics
    if (bad_row) atomicOr(&s_fail, 4);
    if (dup) atomicOr(&s_fail, 8);
    int total = 0;
    const int before = block_exclusive_scan(need, &total);        // barriers also publish s_fail
    int fail = s_fail;
    if (!fail && total > top) fail = 1;
    if (fail) {                                                   // nothing taken, nothing written but the status
        if (threadIdx.x == 0) a.meta[1] = fail & 4 ? 4 : (fail & 8 ? 5 : (fail & 2 ? 2 : 1));
        if (b < a.B && a.out_lens) a.out_lens[b] = pos;
        if (b < a.B && a.slots)
            for (int t = 0; t < a.n_new; ++t) a.slots[(long long)b * a.n_new + t] = -1;
        return;
    }
    int32_t* trow = a.tables + (long long)row * a.max_blocks;
    for (int j = 0; j < need; ++j) trow[held + j] = a.stack[top - 1 - (before + j)];
    if (live) {
        a.lens[row] = end;
        if (a.out_lens) a.out_lens[b] = end;
        if (a.slots)
            for (int t = 0; t < a.n_new; ++t) {
                const int p = pos + t;
                a.slots[(long long)b * a.n_new + t] = (long long)trow[p / a.block_size] * a.block_size + p % a.block_size;
            }
    }
    if (threadIdx.x == 0) a.meta[0] = top - total;
}

// One workgroup: rows[r] (thread r) returns its blocks to the stack (reverse table order) and is emptied.
__global__ __launch_bounds__(kPageThreads) void pages_release(PageArgs a) {
    __shared__ int s_bad;
    const int r = threadIdx.x;
    const int row_in = r < a.B ? a.rows[r] : 0;
    const bool bad_row = r < a.B && (row_in < 0 || row_in >= a.max_seqs);
    const bool live = r < a.B && !bad_row;
    const int row = live ? row_in : 0;
    // the blocks a row holds, never more than its table row (lengths are written by these kernels only)
    const int n = live ? min(max((a.lens[row] + a.block_size - 1) / a.block_size, 0), a.max_blocks) : 0;
    const int top = a.meta[0];            // read by every thread before thread 0 rewrites it (after the barriers)
    if (threadIdx.x == 0) s_bad = 0;
    const bool dup = named_before(a.rows, a.B, r, live, row);     // its barrier also publishes s_bad = 0
    if (bad_row) atomicOr(&s_bad, 1);
    if (dup) atomicOr(&s_bad, 2);
    int total = 0;
    const int before = block_exclusive_scan(n, &total);
    if (s_bad || top + total > a.num_blocks) {                   // nothing returned
        if (threadIdx.x == 0) a.meta[1] = s_bad & 1 ? 4 : (s_bad ? 5 : 3);
        return;
    }
    const int32_t* trow = a.tables + (long long)row * a.max_blocks;
    for (int j = 0; j < n; ++j) a.stack[top + before + j] = trow[n - 1 - j];
    if (live) a.lens[row] = 0;
    if (threadIdx.x == 0) a.meta[0] = top + total;
}

// out [B, width]: the tables of rows[b], entries past the blocks a sequence holds set to 0 (the reference pads with
// 0, src/state.py:124-128); the blocks held are ceil(lens / block_size).
__global__ __launch_bounds__(256) void pages_gather(const int32_t* tables, const int32_t* lens, const int32_t* rows,
                                                    int max_seqs, int max_blocks, int block_size, int B, int width,
                                                    int32_t* out) {
    const long long n = (long long)B * width;
    for (long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (long long)gridDim.x * blockDim.x) {
        const int b = (int)(i / width), j = (int)(i % width);
        const int row = rows[b];
        if (row < 0 || row >= max_seqs) {                        // a row outside the table: zeros
            out[i] = 0;
            continue;
        }
        const int held = (lens[row] + block_size - 1) / block_size;
        out[i] = j < held && j < max_blocks ? tables[(long long)row * max_blocks + j] : 0;
    }
}

int check_common(const char* who, const int32_t* tables, const int32_t* lens, const int32_t* stack,
                 const int32_t* meta, int max_blocks, int num_blocks, int block_size) {
    if (!tables || !lens || !stack || !meta) return fail(RK_ERR_ARG, "%s: null pointer", who);
    if (max_blocks < 1 || num_blocks < 1 || block_size < 1)
        return fail(RK_ERR_ARG, "%s: max_blocks %d num_blocks %d block_size %d", who, max_blocks, num_blocks, block_size);
    return RK_OK;
}

}  // namespace
}  // namespace rk

using namespace rk;

extern "C" {

int rk_pages_init(int32_t* tables, int32_t* lens, int32_t* stack, int32_t* meta, int max_seqs, int max_blocks,
                  int num_blocks, void* stream) {
    if (int rc = check_common("rk_pages_init", tables, lens, stack, meta, max_blocks, num_blocks, 1)) return rc;
    if (max_seqs < 1) return fail(RK_ERR_ARG, "rk_pages_init: max_seqs %d", max_seqs);
    PageArgs a{};
    a.tables = tables; a.lens = lens; a.stack = stack; a.meta = meta; a.max_blocks = max_blocks;
    a.num_blocks = num_blocks; a.max_seqs = max_seqs;
    const long long work = std::max<long long>((long long)max_seqs * max_blocks, num_blocks);
    const int grid = (int)std::min<long long>(1024, (work + kPageThreads - 1) / kPageThreads);
    hipLaunchKernelGGL(pages_init, dim3(grid), dim3(kPageThreads), 0, static_cast<hipStream_t>(stream), a);
    return check_launch("pages_init");
}

int rk_pages_advance(int32_t* tables, int32_t* lens, int32_t* stack, int32_t* meta, int max_seqs, int max_blocks,
                     int num_blocks, int block_size, const int32_t* rows, int B, int n_new, int64_t* slots,
                     int32_t* out_lens, void* stream) {
    if (int rc = check_common("rk_pages_advance", tables, lens, stack, meta, max_blocks, num_blocks, block_size))
        return rc;
    if (max_seqs < 1) return fail(RK_ERR_ARG, "rk_pages_advance: max_seqs %d", max_seqs);
    if (!rows || B < 1 || B > kPageThreads || n_new < 0)
        return fail(RK_ERR_ARG, "rk_pages_advance: rows %p, batch %d (1 .. %d), n_new %d", (const void*)rows, B,
                    kPageThreads, n_new);
    PageArgs a{};
    a.tables = tables; a.lens = lens; a.stack = stack; a.meta = meta; a.rows = rows; a.slots = slots;
    a.out_lens = out_lens; a.max_blocks = max_blocks; a.block_size = block_size; a.B = B; a.n_new = n_new;
    a.num_blocks = num_blocks; a.max_seqs = max_seqs;
    hipLaunchKernelGGL(pages_advance, dim3(1), dim3(kPageThreads), 0, static_cast<hipStream_t>(stream), a);
    return check_launch("pages_advance");
}

int rk_pages_release(int32_t* tables, int32_t* lens, int32_t* stack, int32_t* meta, int max_seqs, int max_blocks,
                     int num_blocks, int block_size, const int32_t* rows, int R, void* stream) {
    if (int rc = check_common("rk_pages_release", tables, lens, stack, meta, max_blocks, num_blocks, block_size))
        return rc;
    if (max_seqs < 1) return fail(RK_ERR_ARG, "rk_pages_release: max_seqs %d", max_seqs);
    if (!rows || R < 1 || R > kPageThreads)
        return fail(RK_ERR_ARG, "rk_pages_release: %d rows (1 .. %d)", R, kPageThreads);
    PageArgs a{};
    a.tables = tables; a.lens = lens; a.stack = stack; a.meta = meta; a.rows = rows; a.max_blocks = max_blocks;
    a.block_size = block_size; a.B = R; a.num_blocks = num_blocks; a.max_seqs = max_seqs;
    hipLaunchKernelGGL(pages_release, dim3(1), dim3(kPageThreads), 0, static_cast<hipStream_t>(stream), a);
    return check_launch("pages_release");
}

int rk_pages_gather(const int32_t* tables, const int32_t* lens, int max_seqs, int max_blocks, int block_size,
                    const int32_t* rows, int B, int width, int32_t* out, void* stream) {
    if (!tables || !lens || !rows || !out || max_seqs < 1 || max_blocks < 1 || block_size < 1 || B < 1 || width < 1)
        return fail(RK_ERR_ARG, "rk_pages_gather: bad arguments");
    const long long n = (long long)B * width;
    const int grid = (int)std::min<long long>(2048, (n + 255) / 256);
    hipLaunchKernelGGL(pages_gather, dim3(grid), dim3(256), 0, static_cast<hipStream_t>(stream), tables, lens, rows,
                       max_seqs, max_blocks, block_size, B, width, out);
    return check_launch("pages_gather");
}

}  // extern "C"
