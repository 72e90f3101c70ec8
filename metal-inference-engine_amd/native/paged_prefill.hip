// P4: packed (varlen) prefill attention over a paged KV pool, gfx950.
//
// Semantics: for every packed segment s (new rows cu[s] .. cu[s+1]-1 of one sequence whose first new token sits at
// absolute position p[s]) the reference writes the new keys / values into the sequence's blocks, gathers positions
// 0 .. p[s]+n[s]-1 back through the block table and runs causal GQA attention, query i at position p[s]+i; the
// output is then multiplied by sigmoid(gate) (src/models/qwen3_5.py:112-120, src/state.py:163-180,
// src/ops.py:65-104, src/models/packing.py:21-31). Here:
//   1. prefill_kv_write: the new K/V rows go into the pool first (rounded to the pool's type), so attention reads
//      exactly what the reference's gather reads back.
//   2. attention, one of three kernels by the inputs (the host's rule at rk_paged_prefill): for bf16 q and pool,
//      prefill_attention (one workgroup per (segment, block of 32 queries, kv-head): one consumer wave per query
//      head of a group of 4, MFMA products and online softmax, and as many producer waves, which stream the key
//      range through a 2-stage LDS ring with 4 tiles of 32 keys in flight in their registers) or, at every other
//      bf16 shape, prefill_attention_b16 (16 queries per consumer wave); both on bf16 operands (q, k, v as stored;
//      p rounded; fp32 accumulation), so results carry bf16-level error. For an fp32 q or pool, or an exact
//      request, prefill_attention_f32 (fp32 products and probabilities). Details at each kernel.
//   3. The output is divided by the softmax sum, gated and written as fp32 [N, Hq, D].
// With a window W (causal only), query i also sees only keys above position p[s]+i-W (src/ops.py:77-81, 97-98): a
// work item starts at the tile holding its first query's first visible key, so whole tiles below every query's
// window are never read, and the keys below it in that first tile are read as that key (never from blocks outside
// the window) and masked. Without causal masking every query of a segment sees all its keys (ops.attention with
// causal=False). Without new rows (k_new null) nothing is written: the keys are already in the pool, which is how
// Backend.attention's contiguous K / V run here (one block holding all S positions).
// Bounds: key positions past a segment's length are clamped for addressing (and masked), table entries clamped to
// the pool, query rows past the segment clamped for loading (and not stored).
#include "rk_device.h"
#include "rk_internal.h"

#include <climits>

namespace rk {
namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kBQ = 32;    // queries per wave
constexpr int kMaxGroup = 4;  // query heads per kv-head of the bf16-operand kernel
constexpr int kWorkInts = 5;  // int32 per work entry
constexpr int kKPad = 8;   // bf16 padding of a K row in LDS (16 bytes)
constexpr int kVPad = 4;   // bf16 padding of a V^T row in LDS: rows of 18 dwords (= 2 mod 4) put 16
                           // consecutive rows' 8-byte pieces on distinct bank pairs

struct PrefillArgs {
    float* out;                 // [N, Hq, D]
    const void* q;              // [N, Hq, D] q_dtype
    const void* k_new;          // [N, Hkv, D] new_dtype
    const void* v_new;
    void* kp;                   // pool layer [NB, bs, Hkv, D] pool_dtype
    void* vp;
    const int32_t* tables;      // [S, max_nb]
    const int32_t* cu;          // [S + 1] new-row offsets
    const int32_t* start;       // [S] absolute position of each segment's first new token
    const int32_t* work;        // [n_work][kWorkInts]: (segment << 16) | query block, first and end key tile, first
                                // partial slot (-1: the whole item), (piece << 16) | pieces; longest first
    float* part;                // split items: per (slot, kv-head, head) the piece's (o, m, l) record
    uint32_t* cnt;              // split items: per (first slot, kv-head, head) arrival counter, zero between calls
    const void* gate;           // [N, Hq * D] gate_dtype, or null
    int gate_dtype;
    int window;                 // 0: none; W: keys above position - W (causal only)
    int causal;                 // 0: every query sees all of its segment's keys
    int q_dtype, new_dtype, pool_dtype;
    int S, n_work, N, Hq, Hkv, G, bs, max_nb, num_blocks, n_slots;
    float qscale;               // log2(e) / sqrt(D)
    uint32_t bs_recip_up;       // ceil(2^32 / bs) (bs >= 2): mulhi(pos, bs_recip_up) = pos / bs while pos * bs < 2^32
    uint32_t bs_recip;          // floor((2^32 - 1) / bs): mulhi(pos, bs_recip) is pos / bs or one less
};

// Workgroup -> (work entry, head chunk, kv-head). The grid is one-dimensional with the kv-head fastest, then the head
// chunk, then the entry: the hardware dispatcher starts workgroups in index order, so every kv-head and chunk of an
// entry starts before the next entry and the list's longest-first order holds across kv-heads. (With the kv-head
// as a second grid dimension, the second kv-head's longest entries were dispatched only after every entry of the
// first kv-head.)
struct WorkSlot {
    int entry, kvh, chunk;
};
__device__ __forceinline__ WorkSlot work_slot(int Hkv, int chunks) {
    const int i = blockIdx.x;
    return WorkSlot{i / (Hkv * chunks), i % Hkv, (i / Hkv) % chunks};
}

__device__ __forceinline__ f32x16 mfma32(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(a), as_bf16x8(b), c, 0, 0, 0);
}

__device__ __forceinline__ long long pool_row(const PrefillArgs& a, const int32_t* table, int pos, int kvh, int D) {
    int blk = table[pos / a.bs];
    blk = blk < 0 ? 0 : (blk >= a.num_blocks ? a.num_blocks - 1 : blk);
    return (((long long)blk * a.bs + pos % a.bs) * a.Hkv + kvh) * D;
}

// 8 consecutive elements at element offset off as bf16 bits (fp32 sources rounded to nearest even)
__device__ __forceinline__ u32x4 load8_bf16(const void* base, long long off, int dtype) {
    if (dtype == RK_BF16) return *reinterpret_cast<const u32x4*>(reinterpret_cast<const uint16_t*>(base) + off);
    const float4* p = reinterpret_cast<const float4*>(reinterpret_cast<const float*>(base) + off);
    const float4 x = p[0], y = p[1];
    u32x4 r;
    r[0] = (uint32_t)f32_to_bf16_rne(x.x) | ((uint32_t)f32_to_bf16_rne(x.y) << 16);
    r[1] = (uint32_t)f32_to_bf16_rne(x.z) | ((uint32_t)f32_to_bf16_rne(x.w) << 16);
    r[2] = (uint32_t)f32_to_bf16_rne(y.x) | ((uint32_t)f32_to_bf16_rne(y.y) << 16);
    r[3] = (uint32_t)f32_to_bf16_rne(y.z) | ((uint32_t)f32_to_bf16_rne(y.w) << 16);
    return r;
}

__device__ __forceinline__ int segment_of(const int32_t* cu, int S, int row) {
    int lo = 0, hi = S - 1;                 // largest s with cu[s] <= row
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (cu[mid] <= row) lo = mid; else hi = mid - 1;
    }
    return lo;
}

// ---- 1. new K/V rows into the pool: one thread moves 8 elements of one row (K and V)
__global__ __launch_bounds__(256) void prefill_kv_write(PrefillArgs a, int D) {
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    const int row = a.Hkv * D, per = row / 8;
    if (i >= (long long)a.N * per) return;
    const int n = (int)(i / per), c = (int)(i % per) * 8;
    const int s = segment_of(a.cu, a.S, n);
    const int pos = a.start[s] + (n - a.cu[s]);
    const int32_t* table = a.tables + (long long)s * a.max_nb;
    const int j = pos / a.bs;
    if (j >= a.max_nb) return;
    const int blk = table[j];
    if (blk < 0 || blk >= a.num_blocks) return;
    const long long dst = ((long long)blk * a.bs + pos % a.bs) * row + c;
    const long long src = (long long)n * row + c;
    if (a.pool_dtype == RK_BF16) {
        *reinterpret_cast<u32x4*>(reinterpret_cast<uint16_t*>(a.kp) + dst) = load8_bf16(a.k_new, src, a.new_dtype);
        *reinterpret_cast<u32x4*>(reinterpret_cast<uint16_t*>(a.vp) + dst) = load8_bf16(a.v_new, src, a.new_dtype);
    } else {
        const void* srcs[2] = {a.k_new, a.v_new};
        void* dsts[2] = {a.kp, a.vp};
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            float f[8];
            if (a.new_dtype == RK_BF16) {
                const u32x4 w = *reinterpret_cast<const u32x4*>(reinterpret_cast<const uint16_t*>(srcs[t]) + src);
#pragma unroll
                for (int e = 0; e < 4; ++e) { f[2 * e] = bf16_lo(w[e]); f[2 * e + 1] = bf16_hi(w[e]); }
            } else {
                const float4* p = reinterpret_cast<const float4*>(reinterpret_cast<const float*>(srcs[t]) + src);
                const float4 x = p[0], y = p[1];
                f[0] = x.x; f[1] = x.y; f[2] = x.z; f[3] = x.w; f[4] = y.x; f[5] = y.y; f[6] = y.z; f[7] = y.w;
            }
            float4* d4 = reinterpret_cast<float4*>(reinterpret_cast<float*>(dsts[t]) + dst);
            d4[0] = make_float4(f[0], f[1], f[2], f[3]);
            d4[1] = make_float4(f[4], f[5], f[6], f[7]);
        }
    }
}

// ---- 2. attention: a warp-specialised pipeline. blockDim = 2 G * 64 (G = 4): waves 0 .. G-1 are consumers (query
// head kvh * G + wave, the work item's 32 queries), waves G .. 2G-1 are producers. Keys go in tiles of kBKP = 32.
// Producers keep DEPTH tiles of K / V rows in flight in their registers (per lane and tile 4 keys x 8 dims of K and
// of V; the block ids of the whole key range are cached in LDS first, so no table load ever sits between two
// tiles), and per tile move the oldest one into a 2-stage LDS ring (K as rows, V transposed to [dim][key], both
// rounded to bf16; the lane orders and row paddings keep every LDS write and read free of bank conflicts), then
// request the tile DEPTH ahead. Consumers compute S^T = K Q^T on v_mfma_f32_32x32x16_bf16 (A = 32 keys x 16 dims
// from LDS, B = 16 dims x 32 queries from registers), so each lane owns one query column: the online softmax needs
// one cross-lane exchange, and the probabilities, rounded to bf16, are already the B operand of O^T += V^T P^T
// (A = 32 dims x 16 keys from LDS). Operand reads from LDS run two k-steps (one 32-dim block) ahead of the MFMAs
// that use them. One LDS-only barrier per tile hands the stages over; it never waits for the producers'
// outstanding loads. fp32 accumulation; bf16 operands (q, k, v as stored, p rounded).
constexpr int kBKP = 32;        // keys per tile
constexpr int kStages = 2;      // LDS ring stages
constexpr int kTabCache = 4096; // block ids cached in LDS (max_nb above it takes the table from global memory)
constexpr float kLazy = 8.0f;   // log2 headroom before the running maximum is raised

// 8 consecutive bf16 elements of one pool row, as a producer loads them
struct PoolRow {
    static constexpr int kDepth = 4;     // tiles in flight per producer lane
    u32x4 w;
    __device__ void load(const void* base, long long off) {
        w = *reinterpret_cast<const u32x4*>(reinterpret_cast<const uint16_t*>(base) + off);
    }
    __device__ u32x4 bf16() const { return w; }
};

template <int D, bool TAB_LDS>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2))) void prefill_attention(PrefillArgs a) {
    constexpr int NKS = D / 16;          // k-steps of S^T (dims)
    constexpr int NDT = D / 32;          // 32-row tiles of O^T (dims)
    constexpr int KROW = D + kKPad;      // LDS K row stride (bf16)
    constexpr int VROW = kBKP + kVPad;   // LDS V^T row stride (bf16)
    constexpr int KBUF = kBKP * KROW, VBUF = D * VROW;
    constexpr int DEPTH = PoolRow::kDepth;
    constexpr int NJ = (kBKP / 4) * (D / 8);   // jobs of 4 keys x 8 dims per tile
    extern __shared__ __attribute__((aligned(16))) char smem[];
    int* tab = reinterpret_cast<int*>(smem);                                  // [kTabCache] when TAB_LDS
    uint16_t* kst = reinterpret_cast<uint16_t*>(smem + (TAB_LDS ? kTabCache * 4 : 0));   // [kStages][K tile]
    uint16_t* vst = kst + kStages * KBUF;                                     // [kStages][V^T tile]

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int G = a.G;
    const bool producer = wave >= G;
    const WorkSlot ws = work_slot(a.Hkv, 1);
    const int kvh = ws.kvh;
    const int32_t* we = a.work + (long long)kWorkInts * ws.entry;
    const int item = we[0];
    const int seg = item >> 16, qblk = item & 0xffff;
    const int row0 = a.cu[seg] + qblk * kBQ;
    const int nq = min(kBQ, a.cu[seg + 1] - row0);
    const int p0 = a.start[seg] + qblk * kBQ;       // position of the block's first query
    // keys kmin .. n_keys - 1: causal, up to the last query (and from the first query's window); otherwise the
    // whole segment
    const int n_keys = a.causal ? p0 + nq : a.start[seg] + (a.cu[seg + 1] - a.cu[seg]);
    const int kmin = a.window > 0 ? max(0, p0 - a.window + 1) : 0;
    // this work entry's key tiles: the item's (kmin / 32 .. the tile holding key n_keys - 1) within the entry's range
    const int t_first = max(kmin / kBKP, we[1]);     // tiles t_first .. t_first + n_tiles - 1
    const int n_tiles = min((n_keys + kBKP - 1) / kBKP, we[2]) - t_first;
    const int b_first = kmin / a.bs;                 // first block read
    const int32_t* table = a.tables + (long long)seg * a.max_nb;

    if (TAB_LDS) {
        const int nb = (n_keys + a.bs - 1) / a.bs;  // <= max_nb <= kTabCache
        for (int i = b_first + tid; i < nb; i += blockDim.x) {
            const int blk = table[i];
            tab[i - b_first] = blk < 0 ? 0 : (blk >= a.num_blocks ? a.num_blocks - 1 : blk);
        }
    }

    // ---- producer state: per tile a producer lane moves job = 4 keys x 8 dims of both K and V (4 + 4 row pieces
    // of 16 bytes), the same code for every lane: a branch between K and V work would make the compiler wait for
    // all loads in flight where the branches join
    const int pl = tid - G * 64;
    const int job = pl;                              // 0 .. NJ-1 in use
    const bool has_job = producer && __builtin_amdgcn_readfirstlane(job) < NJ;   // whole waves: uniform
    // K and V pieces use different lane orders, each chosen for conflict-free LDS writes: for K consecutive lanes
    // take consecutive dim chunks of one key group (16-byte pieces of the same rows, contiguous); for V consecutive
    // lanes take consecutive key groups of one dim chunk (their 8-byte V^T writes at key 4 kq of rows 8 dc + e
    // spread over all banks; dim-chunk-major lanes would put 16 lanes on 2 bank groups)
    const int kqk = job / (D / 8), dck = job % (D / 8);
    const int kqv = job % (kBKP / 4), dcv = job / (kBKP / 4);
    PoolRow buf[DEPTH][8];                       // [0..3] K rows of keys 4 kqk + j, [4..7] V rows of 4 kqv + j
    // the 4 keys of a job: one block lookup and one base address when they lie in one block (block_size % 4 == 0:
    // rows then differ by a constant stride), one per key otherwise
    const bool rows4 = a.bs % 4 == 0;
    const long long rstride = (long long)a.Hkv * D;
    auto issue = [&](int t_rel, PoolRow (&slot)[8]) {
        const int tile = t_first + t_rel;
        // pos = b * bs + r with b = mulhi(pos, ceil(2^32 / bs)): exact because pos * bs < 2^32 (checked on the host)
        auto row_of = [&](int pos) {
            const int b = (int)__umulhi((uint32_t)pos, a.bs_recip_up);
            int blk;
            if (TAB_LDS) {
                blk = tab[b - b_first];
            } else {
                blk = table[b];
                blk = blk < 0 ? 0 : (blk >= a.num_blocks ? a.num_blocks - 1 : blk);
            }
            return (long long)blk * a.bs + (pos - b * a.bs);
        };
        auto group = [&](int kq, int dc, const void* base, PoolRow* rows) {
            const int p4 = tile * kBKP + 4 * kq;
            if (rows4) {
                // tiles past the end re-read the last key (never used); a clamped group of 4 stays in its block;
                // groups below the window read the group holding its first key (same block: bs % 4 == 0)
                int pos = p4 + 3 < n_keys ? p4 : (n_keys - 1) / 4 * 4;
                pos = pos < kmin ? kmin / 4 * 4 : pos;
                const long long off = (row_of(pos) * a.Hkv + kvh) * D + 8 * dc;
#pragma unroll
                for (int j = 0; j < 4; ++j) rows[j].load(base, off + j * rstride);
            } else {
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    int pos = p4 + j;
                    pos = pos < n_keys ? pos : n_keys - 1;
                    pos = pos < kmin ? kmin : pos;
                    rows[j].load(base, (row_of(pos) * a.Hkv + kvh) * D + 8 * dc);
                }
            }
        };
        group(kqk, dck, a.kp, slot);
        group(kqv, dcv, a.vp, slot + 4);
    };
    auto stash = [&](const PoolRow (&slot)[8], int stage) {
        uint16_t* ks = kst + stage * KBUF;
        uint16_t* vt = vst + stage * VBUF;
        u32x4 v[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            *reinterpret_cast<u32x4*>(&ks[(4 * kqk + j) * KROW + 8 * dck]) = slot[j].bf16();
            v[j] = slot[4 + j].bf16();
        }
        // transpose: V^T row 8 dc + e gets element e of the 4 key rows (8 bytes); one byte permute per word picks
        // the same 16-bit half (low for even e, high for odd e) of two rows
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const uint32_t sel = e & 1 ? 0x07060302u : 0x05040100u;
            const uint32_t w0 = __builtin_amdgcn_perm(v[1][e / 2], v[0][e / 2], sel);
            const uint32_t w1 = __builtin_amdgcn_perm(v[3][e / 2], v[2][e / 2], sel);
            *reinterpret_cast<u32x2*>(&vt[(8 * dcv + e) * VROW + 4 * kqv]) = u32x2{w0, w1};
        }
    };

    // ---- consumer state
    const int head = kvh * G + (producer ? 0 : wave);
    const int col = lane & 31, kg = lane >> 5;      // query column, k-slot group
    const int qpos = a.causal ? p0 + (col < nq ? col : nq - 1) : n_keys - 1;
    const int qlo = a.window > 0 ? qpos - a.window : -1;    // keys at or below qlo are outside the window
    const int qfirst = a.causal ? p0 : n_keys - 1;           // the smallest qpos of the work item
    const int qlast = a.causal ? p0 + nq - 1 : n_keys - 1;    // the largest
    // tiles starting at or below lo_edge hold keys outside some query's window; tiles reaching past qfirst hold keys
    // after some query: only those are masked
    const int lo_edge = a.window > 0 ? qlast - a.window : INT_MIN;
    u32x4 qop[NKS];                                  // Q^T operands: q[query col][d = 16 t + 8 kg .. + 8]
    f32x16 o[NDT];
    float m_run = -INFINITY, l_run = 0.0f;

    if (TAB_LDS) __syncthreads();                    // the block ids are in LDS

    auto consume = [&](int t_rel, int stage) {
        const int k0 = (t_first + t_rel) * kBKP;
        const uint16_t* ks = kst + stage * KBUF;
        const uint16_t* vt = vst + stage * VBUF;
        // ---- S^T = K Q^T for the 32 keys; the K operands of the next two k-steps are requested before this
        // pair's MFMAs, so four LDS reads are in flight and the MFMA chain does not wait on each one
        f32x16 s = f32x16{};
        const uint16_t* krow = &ks[col * KROW + 8 * kg];
        u32x4 ka0 = *reinterpret_cast<const u32x4*>(krow), ka1 = *reinterpret_cast<const u32x4*>(krow + 16);
#pragma unroll
        for (int t = 0; t < NKS; t += 2) {
            u32x4 nb0 = ka0, nb1 = ka1;
            if (t + 2 < NKS) {
                nb0 = *reinterpret_cast<const u32x4*>(krow + 16 * (t + 2));
                nb1 = *reinterpret_cast<const u32x4*>(krow + 16 * (t + 3));
            }
            __builtin_amdgcn_sched_barrier(0);       // keep the reads ahead of the MFMAs that do not need them
            s = mfma32(ka0, qop[t], s);
            s = mfma32(ka1, qop[t + 1], s);
            __builtin_amdgcn_sched_barrier(0);
            ka0 = nb0;
            ka1 = nb1;
        }
        // ---- mask (only tiles reaching past the block's first query hold keys above any query), online softmax
        // over this lane's query column in base 2 with the scale folded into the exponent's FMA. The running
        // maximum m is raised only when a tile's maximum exceeds it by more than kLazy: p = 2^(s - m) then stays
        // <= 2^kLazy (exact in fp32, representable in bf16), and the accumulators are rescaled only when some
        // column's m moves, which after the first tiles is rare.
        if (k0 + kBKP - 1 > qfirst || k0 <= lo_edge) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int key = k0 + 8 * (r / 4) + 4 * kg + (r % 4);
                s[r] = key <= qpos && key > qlo ? s[r] : -INFINITY;
            }
        }
        // the lane compares its own 16 scores first; only when some lane exceeds m + kLazy is the maximum over the
        // column's two lanes formed (the same m as max-then-compare over all 32 keys: scaling by qscale > 0 is
        // monotonic, so it commutes with max)
        float tmax = s[0];
#pragma unroll
        for (int r = 1; r < 16; ++r) tmax = fmaxf(tmax, s[r]);
        tmax *= a.qscale;
        const float m_prev = m_run;
        if (__any(tmax > m_run + kLazy)) {
            tmax = fmaxf(tmax, __shfl_xor(tmax, 32));
            m_run = tmax > m_run + kLazy ? tmax : m_run;
        }
        // -inf only while every key this column has seen was masked (a window starting past the first tile); then
        // the exponents are taken against 0, so the masked keys give 0 (not NaN) and nothing is rescaled
        const float mb = m_run == -INFINITY ? 0.0f : m_run;
        if (__any(m_run != m_prev)) {
            const float alpha = fast_exp2(m_prev - mb);     // 0 on the first tile (m_prev = -inf)
            l_run *= alpha;
#pragma unroll
            for (int t = 0; t < NDT; ++t) o[t] *= alpha;
        }
        u32x4 pop[2];                                // B operands of the 2 key k-steps
#pragma unroll
        for (int half = 0; half < 2; ++half) {
            float pv[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                pv[e] = fast_exp2(fmaf(s[8 * half + e], a.qscale, -mb));
                l_run += pv[e];                      // this lane's 16 keys; the column's two lanes are summed at the end
            }
            u32x4 w;
#pragma unroll
            for (int j = 0; j < 4; ++j) w[j] = pack_bf16x2_rne(pv[2 * j], pv[2 * j + 1]);
            pop[half] = w;
        }
        // ---- O^T += V^T P^T: k-step u covers keys 16 u + 8 (e / 4) + 4 kg + e % 4
        // (the V^T operands of the next 32-dim block are requested before this block's MFMAs)
        auto vread = [&](int dt, u32x4 (&va)[2]) {
            const uint16_t* vrow = &vt[(32 * dt + col) * VROW];
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                const int kb = 16 * u + 4 * kg;
                const u32x2 lo = *reinterpret_cast<const u32x2*>(vrow + kb);
                const u32x2 hi = *reinterpret_cast<const u32x2*>(vrow + kb + 8);
                va[u] = u32x4{lo[0], lo[1], hi[0], hi[1]};
            }
        };
        u32x4 vcur[2], vnext[2];
        vread(0, vcur);
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt) {
            if (dt + 1 < NDT) vread(dt + 1, vnext);
            __builtin_amdgcn_sched_barrier(0);
            o[dt] = mfma32(vcur[0], pop[0], o[dt]);
            o[dt] = mfma32(vcur[1], pop[1], o[dt]);
            __builtin_amdgcn_sched_barrier(0);
            vcur[0] = vnext[0];
            vcur[1] = vnext[1];
        }
    };

    // The two roles run separate loops with the same number of LDS-only barriers: one after the prologue and one per
    // iteration, n_iter = n_tiles rounded up to a multiple of DEPTH. Neither role's registers are live in the other's
    // loop, and the producers' loop body has no branch at all, so the compiler can count their loads in flight
    // exactly (a branch there makes it wait for all of them).
    const int n_iter = (n_tiles + DEPTH - 1) / DEPTH * DEPTH;
    if (producer) {
        if (!has_job) {                              // whole waves without a share of the tile (D = 128)
            for (int k = 0; k <= n_iter; ++k) lds_barrier();
            return;
        }
        // tile t lives in slot t % DEPTH, then in stage t % 2 (DEPTH is even: both compile-time in the unrolled
        // inner loop); at iteration t the slot of tile t + 1 goes to LDS and is refilled with tile t + 1 + DEPTH.
        // Tiles from n_tiles on read the last key again and fill stages nobody reads.
        static_assert(DEPTH % kStages == 0, "slot and stage of a tile must be compile-time in the unrolled loop");
#pragma unroll
        for (int d = 0; d < DEPTH; ++d) issue(d, buf[d]);
        stash(buf[0], 0);
        issue(DEPTH, buf[0]);
        lds_barrier();
        for (int i = 0; i < n_iter; i += DEPTH) {
#pragma unroll
            for (int d = 0; d < DEPTH; ++d) {
                stash(buf[(d + 1) % DEPTH], (d + 1) % kStages);
                issue(i + d + 1 + DEPTH, buf[(d + 1) % DEPTH]);
                lds_barrier();
            }
        }
        return;
    }
    {
        // q is bf16 here (the host's rule for this kernel): its rows are the operands as they are
        const uint16_t* qb = reinterpret_cast<const uint16_t*>(a.q) +
                             ((long long)(row0 + (col < nq ? col : nq - 1)) * a.Hq + head) * D + 8 * kg;
#pragma unroll
        for (int t = 0; t < NKS; ++t) qop[t] = *reinterpret_cast<const u32x4*>(qb + 16 * t);
#pragma unroll
        for (int t = 0; t < NDT; ++t) o[t] = f32x16{};
    }
    lds_barrier();
    for (int t = 0; t < n_iter; ++t) {
        if (t < n_tiles) consume(t, t & (kStages - 1));
        lds_barrier();
    }
    l_run += __shfl_xor(l_run, 32);

    // A piece of a split item stores its (o, m, l) for its head, then counts itself in; the last of the item's
    // pieces to finish reads all of them back in piece order and combines them: m = max m_p,
    // l = sum 2^(m_p - m) l_p, o = sum 2^(m_p - m) o_p, so the result depends only on the pieces, not on which
    // finishes last. It then leaves the counter at zero and goes on to the normal output below.
    // Memory ordering. The records go through a buffer resource of exactly one record with the sc1 cache policy:
    // the bit the compiler puts on agent-scope atomic stores and loads for gfx950, which makes each 16-byte store
    // and load an access at the device's coherence point rather than in one XCD's L2 alone. The protocol is
    // therefore: agent-scope stores of the records, a wait for their completion (s_waitcnt vmcnt(0): a store
    // counts as complete once the coherence point has it), an agent-scope atomic increment of the counter issued
    // only after that wait, and, in the wave whose increment returns pieces - 1, agent-scope loads issued only
    // after the increment returned. Every piece's records are thus complete at the coherence point before the
    // counter can reach its final value, and the reader's loads fetch them from there. A release / acquire pair on
    // the counter would give the same order through the memory model, but at agent scope on gfx950 it emits a
    // write-back of the writer's whole L2 (buffer_wbl2) and an invalidate of the reader's (buffer_inv) at every
    // arrival; these records are never held dirty in an L2, so the completion wait is the part of the release
    // that they need. tests/test_gpu_prefill.py (split blocks, several pieces per block, repeated calls) checks
    // the combined output against the oracle and across calls.
    const int piece = we[4] >> 16, pieces = we[4] & 0xffff;
    const int first = we[3] >= 0 && piece < pieces && we[3] + pieces <= a.n_slots ? we[3] : -1;   // slots in range
    if (first >= 0) {
        constexpr int REC = kBQ * D + 2 * kBQ;
        constexpr int kSc1 = 16;                     // cache-policy operand: sc1
        auto rsrc_of = [&](int pc) {
            const unsigned long long u = reinterpret_cast<unsigned long long>(
                a.part + (((long long)(first + pc) * a.Hkv + kvh) * kMaxGroup + wave) * REC);
            const unsigned lo = __builtin_amdgcn_readfirstlane((unsigned)u);
            const unsigned hi = __builtin_amdgcn_readfirstlane((unsigned)(u >> 32));
            return __builtin_amdgcn_make_buffer_rsrc(reinterpret_cast<void*>(((unsigned long long)hi << 32) | lo),
                                                     (short)0, REC * 4, 0x00020000);
        };
        auto o_off = [&](int dt, int q) { return 4 * (col * D + 32 * dt + 8 * q + 4 * kg); };
        const int m_off = 4 * (kBQ * D + col), l_off = 4 * (kBQ * D + kBQ + col);
        {
            const auto rs = rsrc_of(piece);
#pragma unroll
            for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
                for (int q = 0; q < 4; ++q)
                    __builtin_amdgcn_raw_buffer_store_b128(
                        __builtin_bit_cast(u32x4, f32x4{o[dt][4 * q], o[dt][4 * q + 1], o[dt][4 * q + 2],
                                                        o[dt][4 * q + 3]}),
                        rs, o_off(dt, q), 0, kSc1);
            if (kg == 0) {
                __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(m_run), rs, m_off, 0, kSc1);
                __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(l_run), rs, l_off, 0, kSc1);
            }
        }
        __builtin_amdgcn_s_waitcnt(0x0F70);          // vmcnt(0): this wave's stores have completed
        uint32_t* counter = a.cnt + ((long long)first * a.Hkv + kvh) * kMaxGroup + wave;
        uint32_t before = 0;
        if (lane == 0) before = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        before = __shfl(before, 0);
        if (before != (uint32_t)(pieces - 1)) return;
        float mx = -INFINITY;
#pragma unroll 4
        for (int pc = 0; pc < pieces; ++pc)
            mx = fmaxf(mx, __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rsrc_of(pc), m_off, 0, kSc1)));
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt) o[dt] = f32x16{};
        l_run = 0.0f;
        for (int pc = 0; pc < pieces; ++pc) {
            const auto rs = rsrc_of(pc);
            u32x4 v[NDT][4];
#pragma unroll
            for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
                for (int q = 0; q < 4; ++q) v[dt][q] = __builtin_amdgcn_raw_buffer_load_b128(rs, o_off(dt, q), 0, kSc1);
            const float mp = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rs, m_off, 0, kSc1));
            const float lp = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rs, l_off, 0, kSc1));
            const float sc = mp == -INFINITY ? 0.0f : fast_exp2(mp - mx);     // a piece with no key for this row
            l_run = fmaf(sc, lp, l_run);
#pragma unroll
            for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
                for (int r = 0; r < 16; ++r) o[dt][r] = fmaf(sc, __uint_as_float(v[dt][r / 4][r % 4]), o[dt][r]);
        }
        if (lane == 0) __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }

    // The gate values of a 32-dim block are requested together (one branch per block, not per element: a
    // branch per element would make every gate load a round trip of its own).
    if (col < nq) {
        const float inv = 1.0f / l_run;
        const long long orow = (long long)(row0 + col) * a.Hq + head;
        const bool has_gate = a.gate != nullptr;
        const bool gate16 = a.gate_dtype == RK_BF16;
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt) {
            float4 gv[4];
            if (has_gate && gate16) {
                const uint16_t* gp = reinterpret_cast<const uint16_t*>(a.gate) + orow * D;
                u32x2 w[4];
#pragma unroll
                for (int r4 = 0; r4 < 4; ++r4) w[r4] = *reinterpret_cast<const u32x2*>(gp + 32 * dt + 8 * r4 + 4 * kg);
#pragma unroll
                for (int r4 = 0; r4 < 4; ++r4)
                    gv[r4] = make_float4(bf16_lo(w[r4][0]), bf16_hi(w[r4][0]), bf16_lo(w[r4][1]), bf16_hi(w[r4][1]));
            } else if (has_gate) {
                const float* gp = reinterpret_cast<const float*>(a.gate) + orow * D;
#pragma unroll
                for (int r4 = 0; r4 < 4; ++r4) gv[r4] = *reinterpret_cast<const float4*>(gp + 32 * dt + 8 * r4 + 4 * kg);
            }
#pragma unroll
            for (int r4 = 0; r4 < 4; ++r4) {
                const int d = 32 * dt + 8 * r4 + 4 * kg;
                float v[4] = {o[dt][4 * r4] * inv, o[dt][4 * r4 + 1] * inv, o[dt][4 * r4 + 2] * inv,
                              o[dt][4 * r4 + 3] * inv};
                if (has_gate) {
                    const float g[4] = {gv[r4].x, gv[r4].y, gv[r4].z, gv[r4].w};
#pragma unroll
                    for (int i = 0; i < 4; ++i) v[i] = v[i] * (1.0f / (1.0f + expf(-g[i])));
                }
                *reinterpret_cast<float4*>(a.out + orow * D + d) = make_float4(v[0], v[1], v[2], v[3]);
            }
        }
    }
}

// ---- 3. attention with fp32 operands: the same work list, masks, splits and gate as prefill_attention, for an
// fp32 q or pool and for exact requests (any group size, D = 64 / 128 / 256). The reference computes
// attention in fp32 on widened inputs (src/ops.py:84-87, 91-103), so the products here are fp32 products:
// v_mfma_f32_16x16x4_f32, bf16 pool rows widened exactly when staged, the probabilities kept in fp32.
// blockDim = 512: wave w takes query head (chunk * 4 + w % 4) of the group (none past the group's end: that
// wave only helps stage) and queries 16 (w / 4) .. + 15 of the work item's 32. All 8 waves stage each tile of 32
// keys into a 2-stage LDS ring, requested a whole tile ahead: K row-major ([32 keys][D + 4 floats]) and V transposed
// ([D dims][32 + 4 floats]), both fp32. A staging unit is one 16-byte piece of 4 consecutive key rows (4 loads);
// the V unit's 4 x 4 (fp32) or 4 x 8 (bf16) values are transposed in registers into 16-byte V^T writes. Per wave and
// tile, on 16 x 16 accumulators (lane l: query l % 16, rows 4 (l / 16) .. + 3):
//   S^T = K Q^T:  A = 16 keys x 4 dims from LDS (one 16-byte read feeds four MFMAs: quarter l / 16 takes dims
//                 16 c + 4 (l / 16) + j of MFMA j), B = Q^T from registers (the same dims of the lane's query);
//   O^T += V^T P^T: A = 16 dims x 4 keys from V^T (one 16-byte read of V^T[16 dt + l % 16][16 kt + 4 (l / 16) ..
//                 + 3] feeds MFMAs r = 0 .. 3: keys 4 (l / 16) + r), B = P^T, the score accumulator's register r.
// So every lane keeps its own query's softmax state (one reduction over the 4 quarters per tile), and O^T is
// rescaled per lane. LDS reads are conflict-free: keys and dims are stored in permuted row orders (at the kernel)
// under which the 16 rows a wave's lanes read lie an effective 2 (mod 4) 16-byte units apart, in lane order (the
// rule measured for 16-byte reads on gfx950, at the 16-query bf16 kernel). Staging writes are conflict-free
// for V^T (consecutive lanes take consecutive key groups of one piece) and at most 2-way for K (consecutive lanes
// take consecutive pieces of one row group).
constexpr int kF32QW = 16;      // queries per wave
constexpr int kF32Heads = 4;    // query heads per workgroup
constexpr int kF32Pad = 4;      // fp32 padding of an LDS row

__device__ __forceinline__ f32x4 mfma_f32(float a, float b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// The lazy running maximum of a 16-query wave (scores s[kt][r] of lane l: query l % 16, keys 16 kt + 4 (l / 16) + r):
// m is raised to the tile's maximum (scaled by qscale) only where that exceeds m by more than kLazy, so
// p = 2^(s qscale - m) stays <= 2^kLazy (exact in fp32, representable in bf16). Each lane first compares its own 8
// scores; only when some lane of the wave exceeds the bound is the maximum over the query's 4 lanes formed, so the
// result equals max-then-compare over all 32 keys while the common case needs no cross-lane exchange (scaling by
// qscale > 0 is monotonic, so it commutes with max).
__device__ __forceinline__ void lazy_max(const f32x4 (&s)[2], float& m, float qscale) {
    float t = fmaxf(fmaxf(fmaxf(s[0][0], s[0][1]), fmaxf(s[0][2], s[0][3])),
                    fmaxf(fmaxf(s[1][0], s[1][1]), fmaxf(s[1][2], s[1][3]))) * qscale;
    if (__any(t > m + kLazy)) {
        t = fmaxf(t, __shfl_xor(t, 16));
        t = fmaxf(t, __shfl_xor(t, 32));
        m = t > m + kLazy ? t : m;
    }
}

// The end of a 16-query wave of the fp32- and bf16-operand kernels: o[dt] holds O^T[16 dt + 4 (lane / 16) + r][query
// lane % 16] for D / 16 dim tiles, with the running (m, l) of the lane's query. Split items: the piece's (o, m, l) per
// (slot, head, half) of 16 queries, then the arrival count; the last piece combines all of them in piece order (the
// protocol and memory ordering of prefill_attention above). Then the rows are divided by l, gated and stored.
template <int D>
__device__ __forceinline__ void finish_queries(const PrefillArgs& a, const int32_t* we, f32x4 (&o)[D / 16],
                                               float m_run, float l_run, int head, int half, int row0, int nq) {
    constexpr int NC = D / 16;
    const int lane = threadIdx.x & 63, qc = lane & 15, qq = lane >> 4;
    const int qi = half * kF32QW + qc;
    const int piece = we[4] >> 16, pieces = we[4] & 0xffff;
    const int first = we[3] >= 0 && piece < pieces && we[3] + pieces <= a.n_slots ? we[3] : -1;
    if (first >= 0) {
        constexpr int REC = kF32QW * D + 2 * kF32QW;
        constexpr int kSc1 = 16;
        auto rsrc_of = [&](int pc) {
            const unsigned long long u = reinterpret_cast<unsigned long long>(
                a.part + (((long long)(first + pc) * a.Hq + head) * 2 + half) * REC);
            const unsigned lo = __builtin_amdgcn_readfirstlane((unsigned)u);
            const unsigned hi = __builtin_amdgcn_readfirstlane((unsigned)(u >> 32));
            return __builtin_amdgcn_make_buffer_rsrc(reinterpret_cast<void*>(((unsigned long long)hi << 32) | lo),
                                                     (short)0, REC * 4, 0x00020000);
        };
        auto o_off = [&](int dt) { return 4 * (qc * D + 16 * dt + 4 * qq); };
        const int m_off = 4 * (kF32QW * D + qc), l_off = 4 * (kF32QW * D + kF32QW + qc);
        {
            const auto rs = rsrc_of(piece);
#pragma unroll
            for (int dt = 0; dt < NC; ++dt)
                __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, o[dt]), rs, o_off(dt), 0, kSc1);
            if (qq == 0) {
                __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(m_run), rs, m_off, 0, kSc1);
                __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(l_run), rs, l_off, 0, kSc1);
            }
        }
        __builtin_amdgcn_s_waitcnt(0x0F70);          // vmcnt(0): this wave's stores have completed
        uint32_t* counter = a.cnt + ((long long)first * a.Hq + head) * 2 + half;
        uint32_t before = 0;
        if (lane == 0) before = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        before = __shfl(before, 0);
        if (before != (uint32_t)(pieces - 1)) return;
        float mx = -INFINITY;
        for (int pc = 0; pc < pieces; ++pc)
            mx = fmaxf(mx, __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rsrc_of(pc), m_off, 0, kSc1)));
#pragma unroll
        for (int dt = 0; dt < NC; ++dt) o[dt] = f32x4{};
        l_run = 0.0f;
        for (int pc = 0; pc < pieces; ++pc) {
            const auto rs = rsrc_of(pc);
            u32x4 v[NC];
#pragma unroll
            for (int dt = 0; dt < NC; ++dt) v[dt] = __builtin_amdgcn_raw_buffer_load_b128(rs, o_off(dt), 0, kSc1);
            const float mp = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rs, m_off, 0, kSc1));
            const float lp = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rs, l_off, 0, kSc1));
            const float sc = mp == -INFINITY ? 0.0f : fast_exp2(mp - mx);
            l_run = fmaf(sc, lp, l_run);
#pragma unroll
            for (int dt = 0; dt < NC; ++dt)
#pragma unroll
                for (int r = 0; r < 4; ++r) o[dt][r] = fmaf(sc, __uint_as_float(v[dt][r]), o[dt][r]);
        }
        if (lane == 0) __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }

    if (qi < nq) {
        const float inv = 1.0f / l_run;
        const long long orow = (long long)(row0 + qi) * a.Hq + head;
        float4 gv[NC];
        if (a.gate) {
            if (a.gate_dtype == RK_BF16) {
                const uint16_t* gp = reinterpret_cast<const uint16_t*>(a.gate) + orow * D + 4 * qq;
#pragma unroll
                for (int dt = 0; dt < NC; ++dt) {
                    const u32x2 w = *reinterpret_cast<const u32x2*>(gp + 16 * dt);
                    gv[dt] = make_float4(bf16_lo(w[0]), bf16_hi(w[0]), bf16_lo(w[1]), bf16_hi(w[1]));
                }
            } else {
                const float* gp = reinterpret_cast<const float*>(a.gate) + orow * D + 4 * qq;
#pragma unroll
                for (int dt = 0; dt < NC; ++dt) gv[dt] = *reinterpret_cast<const float4*>(gp + 16 * dt);
            }
        }
#pragma unroll
        for (int dt = 0; dt < NC; ++dt) {
            float v[4] = {o[dt][0] * inv, o[dt][1] * inv, o[dt][2] * inv, o[dt][3] * inv};
            if (a.gate) {
                const float g[4] = {gv[dt].x, gv[dt].y, gv[dt].z, gv[dt].w};
#pragma unroll
                for (int i = 0; i < 4; ++i) v[i] = v[i] * (1.0f / (1.0f + expf(-g[i])));
            }
            *reinterpret_cast<float4*>(a.out + orow * D + 16 * dt + 4 * qq) = make_float4(v[0], v[1], v[2], v[3]);
        }
    }
}

template <int D, typename TP, bool TAB_LDS>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2))) void prefill_attention_f32(PrefillArgs a) {
    constexpr int ROW = D + kF32Pad;                 // K row stride (floats)
    constexpr int ROWT = kBKP + kF32Pad;             // V^T row stride (floats)
    constexpr int KST = kBKP * ROW;                  // K floats per stage
    constexpr int STAGE = KST + D * ROWT;            // K rows, then V^T rows
    constexpr int EL = 16 / (int)sizeof(TP);         // elements per 16-byte load
    constexpr int PER_ROW = D / EL;                  // 16-byte pieces per row
    constexpr int GROUPS = kBKP / 4;                 // groups of 4 key rows per tile
    constexpr int UNITS_T = GROUPS * PER_ROW;        // staging units per tensor per tile
    constexpr int NU = (2 * UNITS_T + 511) / 512;    // units per thread per tile
    static_assert(UNITS_T % 64 == 0 && (UNITS_T % 512 == 0 || 512 % UNITS_T == 0),
                  "each unit slot of a wave must take one tensor");
    constexpr int NC = D / 16;                       // 16-dim groups
    extern __shared__ __attribute__((aligned(16))) char smem[];
    float* lds = reinterpret_cast<float*>(smem);                               // [2 stages][K rows; V^T rows]
    int* tab = reinterpret_cast<int*>(smem + 2 * STAGE * sizeof(float));       // [kTabCache] block ids

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const WorkSlot ws = work_slot(a.Hkv, (a.G + kF32Heads - 1) / kF32Heads);
    const int kvh = ws.kvh;
    const int gh = ws.chunk * kF32Heads + (wave & 3);        // head within the group
    const int half = wave >> 2;
    const int32_t* we = a.work + (long long)kWorkInts * ws.entry;
    const int item = we[0];
    const int seg = item >> 16, qblk = item & 0xffff;
    const int row0 = a.cu[seg] + qblk * kBQ;
    const int nq = min(kBQ, a.cu[seg + 1] - row0);
    const int p0 = a.start[seg] + qblk * kBQ;
    const int n_keys = a.causal ? p0 + nq : a.start[seg] + (a.cu[seg + 1] - a.cu[seg]);
    const int kmin = a.window > 0 ? max(0, p0 - a.window + 1) : 0;
    const int t_first = max(kmin / kBKP, we[1]);
    const int n_tiles = min((n_keys + kBKP - 1) / kBKP, we[2]) - t_first;
    const int32_t* table = a.tables + (long long)seg * a.max_nb;
    const bool active = gh < a.G && half * kF32QW < nq;     // whole waves
    const int head = kvh * a.G + (gh < a.G ? gh : 0);
    // pos / bs: the estimate from floor((2^32 - 1) / bs) is exact or one short for every pos < 2^32
    auto block_of = [&](int pos, int& r) {
        uint32_t b = __umulhi((uint32_t)pos, a.bs_recip);
        r = pos - (int)b * a.bs;
        if (r >= a.bs) { ++b; r -= a.bs; }
        return (int)b;
    };
    // TAB_LDS (at most kTabCache blocks per table row): the block ids of every position this entry reads (kmin ..
    // n_keys - 1 within its tiles), clamped to the pool, cached in LDS first
    int r0;
    const int b_lo = n_tiles > 0 ? block_of(max(kmin, t_first * kBKP), r0) : 0;
    if (TAB_LDS) {
        const int b_hi = n_tiles > 0 ? block_of(min(n_keys, (t_first + n_tiles) * kBKP) - 1, r0) : -1;
        for (int i = b_lo + tid; i <= b_hi; i += 512) {
            const int blk = table[i];
            tab[i - b_lo] = blk < 0 ? 0 : (blk >= a.num_blocks ? a.num_blocks - 1 : blk);
        }
        __syncthreads();
    }

    // ---- staging: unit u = tid + 512 j (u < 2 UNITS_T) of tensor u / UNITS_T (K, V), e = u % UNITS_T; K: piece
    // e % PER_ROW of rows 4 (e / PER_ROW) .. + 3, V: piece e / GROUPS of rows 4 (e % GROUPS) .. + 3. Load r of a unit
    // is row 4 g + r; every load of a wave reads whole 128-byte row segments.
    u32x4 st[NU][4];
    // LDS rows are permuted so that the 16 rows a wave's lanes read for one 16-byte operand (lane l: row l % 16,
    // column piece l / 16) lie 2 (mod 4) 16-byte units apart, in lane order, which gfx950 serves without bank
    // conflicts: key 16 kt + i of a tile sits in K row 2 i + kt, dim 32 a + 16 b + i in V^T row 32 a + 2 i + b, so
    // with the odd 16-byte strides (D + 4 and 36 floats) lane i's row is 2 i rows (2 x odd units) from lane 0's.
    auto k_row = [](int key) { return 2 * (key & 15) + (key >> 4); };
    auto v_row = [](int dim) { return (dim & ~31) + 2 * (dim & 15) + ((dim >> 4) & 1); };
    auto unit_of = [&](int j, int& g, int& pc) {
        const int u = tid + 512 * j, e = u % UNITS_T;
        const bool is_v = u >= UNITS_T;
        g = is_v ? e % GROUPS : e / PER_ROW;
        pc = is_v ? e / GROUPS : e % PER_ROW;
        return is_v;
    };
    auto issue = [&](int t_rel) {
        const int tile = t_first + t_rel;
        // all block ids of the tile first (one wait for them), then the row loads
        int blk[NU][4], rr[NU][4];
#pragma unroll
        for (int j = 0; j < NU; ++j) {
            int g, pc;
            unit_of(j, g, pc);
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                int pos = tile * kBKP + 4 * g + r;
                pos = pos < n_keys ? pos : n_keys - 1;   // keys past the range read its last key (masked, never used)
                pos = pos < kmin ? kmin : pos;           // keys below the window read its first one
                const int b = block_of(pos, rr[j][r]);
                if (TAB_LDS) {
                    blk[j][r] = tab[b - b_lo];
                } else {
                    const int t = table[b];
                    blk[j][r] = t < 0 ? 0 : (t >= a.num_blocks ? a.num_blocks - 1 : t);
                }
            }
        }
#pragma unroll
        for (int j = 0; j < NU; ++j) {
            if (tid + 512 * j < 2 * UNITS_T) {           // whole waves (UNITS_T is a multiple of 64)
                int g, pc;
                const bool is_v = unit_of(j, g, pc);
                const TP* base = reinterpret_cast<const TP*>(is_v ? a.vp : a.kp);
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const long long off = (((long long)blk[j][r] * a.bs + rr[j][r]) * a.Hkv + kvh) * D + pc * EL;
                    st[j][r] = *reinterpret_cast<const u32x4*>(base + off);
                }
            }
        }
    };
    auto stash = [&](int stage) {
        float* s = lds + stage * STAGE;
#pragma unroll
        for (int j = 0; j < NU; ++j) {
            if (tid + 512 * j >= 2 * UNITS_T) continue;
            int g, pc;
            if (unit_of(j, g, pc)) {                 // V^T[v_row(pc EL + d)][4 g .. + 3]
                float* dst = s + KST + 4 * g;
                if constexpr (sizeof(TP) == 4) {
#pragma unroll
                    for (int d = 0; d < 4; ++d)
                        *reinterpret_cast<f32x4*>(dst + v_row(pc * EL + d) * ROWT) = f32x4{
                            __uint_as_float(st[j][0][d]), __uint_as_float(st[j][1][d]),
                            __uint_as_float(st[j][2][d]), __uint_as_float(st[j][3][d])};
                } else {                             // bf16 -> fp32, exact
#pragma unroll
                    for (int d = 0; d < 4; ++d) {
                        *reinterpret_cast<f32x4*>(dst + v_row(pc * EL + 2 * d) * ROWT) = f32x4{
                            bf16_lo(st[j][0][d]), bf16_lo(st[j][1][d]), bf16_lo(st[j][2][d]), bf16_lo(st[j][3][d])};
                        *reinterpret_cast<f32x4*>(dst + v_row(pc * EL + 2 * d + 1) * ROWT) = f32x4{
                            bf16_hi(st[j][0][d]), bf16_hi(st[j][1][d]), bf16_hi(st[j][2][d]), bf16_hi(st[j][3][d])};
                    }
                }
            } else {                                 // K[k_row(4 g + r)][pc EL ..]
                float* dst = s + pc * EL;
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    if constexpr (sizeof(TP) == 4) {
                        *reinterpret_cast<u32x4*>(dst + k_row(4 * g + r) * ROW) = st[j][r];
                    } else {
                        const u32x4 w = st[j][r];
                        *reinterpret_cast<f32x4*>(dst + k_row(4 * g + r) * ROW) =
                            f32x4{bf16_lo(w[0]), bf16_hi(w[0]), bf16_lo(w[1]), bf16_hi(w[1])};
                        *reinterpret_cast<f32x4*>(dst + k_row(4 * g + r) * ROW + 4) =
                            f32x4{bf16_lo(w[2]), bf16_hi(w[2]), bf16_lo(w[3]), bf16_hi(w[3])};
                    }
                }
            }
        }
    };

    // ---- per-wave query state
    const int qc = lane & 15, qq = lane >> 4;
    const int qi = half * kF32QW + qc;               // query within the work item
    const int qpos = a.causal ? p0 + (qi < nq ? qi : nq - 1) : n_keys - 1;
    const int qlo = a.window > 0 ? qpos - a.window : -1;
    const int qfirst = a.causal ? p0 + half * kF32QW : n_keys - 1;
    const int qlast = a.causal ? p0 + min(half * kF32QW + kF32QW, nq) - 1 : n_keys - 1;
    const int lo_edge = a.window > 0 ? qlast - a.window : INT_MIN;
    f32x4 qv[NC];                                    // Q[query][16 c + 4 qq .. + 3]
    f32x4 o[NC];                                     // O^T[16 dt + 4 qq + r][query]
    float m_run = -INFINITY, l_run = 0.0f;
    if (active) {
        const long long qb = ((long long)(row0 + (qi < nq ? qi : nq - 1)) * a.Hq + head) * D + 4 * qq;
        if (a.q_dtype == RK_BF16) {
            const uint16_t* qp = reinterpret_cast<const uint16_t*>(a.q) + qb;
#pragma unroll
            for (int c = 0; c < NC; ++c) {
                const u32x2 w = *reinterpret_cast<const u32x2*>(qp + 16 * c);
                qv[c] = f32x4{bf16_lo(w[0]), bf16_hi(w[0]), bf16_lo(w[1]), bf16_hi(w[1])};
            }
        } else {
            const float* qp = reinterpret_cast<const float*>(a.q) + qb;
#pragma unroll
            for (int c = 0; c < NC; ++c) qv[c] = *reinterpret_cast<const f32x4*>(qp + 16 * c);
        }
#pragma unroll
        for (int c = 0; c < NC; ++c) o[c] = f32x4{};
    }

    auto consume = [&](int t_rel, int stage) {
        const float* ks = lds + stage * STAGE;
        const float* vs = ks + KST;
        const int k0 = (t_first + t_rel) * kBKP;
        f32x4 s[2] = {f32x4{}, f32x4{}};
#pragma unroll
        for (int c = 0; c < NC; ++c) {
#pragma unroll
            for (int kt = 0; kt < 2; ++kt) {
                const f32x4 kv = *reinterpret_cast<const f32x4*>(ks + (2 * qc + kt) * ROW + 16 * c + 4 * qq);
#pragma unroll
                for (int j = 0; j < 4; ++j) s[kt] = mfma_f32(kv[j], qv[c][j], s[kt]);
            }
        }
        // lane (qc, qq), register r of sub-tile kt: key k0 + 16 kt + 4 qq + r
        if (k0 + kBKP - 1 > qfirst || k0 <= lo_edge) {
#pragma unroll
            for (int kt = 0; kt < 2; ++kt)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int key = k0 + 16 * kt + 4 * qq + r;
                    s[kt][r] = key <= qpos && key > qlo ? s[kt][r] : -INFINITY;
                }
        }
        const float m_prev = m_run;
        lazy_max(s, m_run, a.qscale);
        const float mb = m_run == -INFINITY ? 0.0f : m_run;
        if (__any(m_run != m_prev)) {
            const float alpha = fast_exp2(m_prev - mb);     // 0 on the first tile (m_prev = -inf)
            l_run *= alpha;
#pragma unroll
            for (int dt = 0; dt < NC; ++dt) o[dt] *= alpha;
        }
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                s[kt][r] = fast_exp2(fmaf(s[kt][r], a.qscale, -mb));
                l_run += s[kt][r];                   // this lane's keys; the 4 lanes of a query are summed at the end
            }
        // V^T reads one dim group ahead of their MFMAs (group i: dims 16 (i % NC) + qc, keys 16 (i / NC) + 4 qq ..)
        const float* vt = vs + 2 * qc * ROWT + 4 * qq;
        auto vread = [&](int i) {
            const int dt = i % NC, kt = i / NC;
            return *reinterpret_cast<const f32x4*>(vt + (32 * (dt >> 1) + (dt & 1)) * ROWT + 16 * kt);
        };
        f32x4 vv = vread(0);
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);       // the first read,
#pragma unroll
        for (int i = 0; i < 2 * NC; ++i) {
            const int kt = i / NC, dt = i % NC;
            const f32x4 cur = vv;
            if (i + 1 < 2 * NC) vv = vread(i + 1);
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);   // the next read,
            __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);   // then this group's four MFMAs
#pragma unroll
            for (int r = 0; r < 4; ++r) o[dt] = mfma_f32(cur[r], s[kt][r], o[dt]);
        }
    };

    // Stage t's rows are written after tile t - 1 is computed (stage (t - 1) & 1 is free once every wave passed the
    // barrier that ended tile t - 2), then tile t + 1 is requested; one LDS-only barrier per tile.
    if (n_tiles > 0) {
        issue(0);
        stash(0);
        if (n_tiles > 1) issue(1);
        lds_barrier();
        for (int t = 0; t < n_tiles; ++t) {
            if (active) consume(t, t & 1);
            if (t + 1 < n_tiles) {
                stash((t + 1) & 1);
                if (t + 2 < n_tiles) issue(t + 2);
            }
            lds_barrier();
        }
    }
    if (!active) return;
    l_run += __shfl_xor(l_run, 16);
    l_run += __shfl_xor(l_run, 32);
    finish_queries<D>(a, we, o, m_run, l_run, head, half, row0, nq);
}

// ---- 4. attention on bf16 operands, 16 queries per consumer wave, for bf16 q and pool (v_mfma_f32_16x16x32_bf16).
// blockDim = 768, warp-specialised: waves 0 .. 7 are consumers (wave w: query head chunk * 4 + w % 4 of the
// group, queries 16 (w / 4) .. + 15 of the work item: the fp32-operand kernel's split of the work, its work list,
// masks, split records and epilogue), waves 8 .. 11 are producers. Three waves per SIMD: two consumers, so one's
// softmax and LDS waits hide behind the other's MFMAs, and a producer, whose loads and LDS writes overlap both.
// Producers keep kB16Depth tiles of 32 keys in flight in their registers (per lane and tile one staging unit of K and
// one of V: a 16-byte piece, 8 dims, of 4 consecutive key rows) and per tile move the oldest into a 2-stage LDS
// ring, K as rows, V transposed to [dim][key] (bf16 as stored), then request the next; one LDS-only barrier per tile.
// Per consumer wave and tile, on 16 x 16 accumulators (lane l: query l % 16, rows 4 (l / 16) .. + 3):
//   S^T = K Q^T:  A = 16 keys x 32 dims (one 16-byte LDS read: row 16 kt + l % 16, dims 32 c + 8 (l / 16) .. + 7),
//                 B = Q^T from registers (the same dims of the lane's query);
//   O^T += V^T P^T: one MFMA per 16 dims over all 32 keys. k-slot 8 (l / 16) + j stands for key 4 (l / 16) + j
//                 (j < 4) or 16 + 4 (l / 16) + j - 4, which are exactly the keys of the lane's own scores
//                 s[0][0..3], s[1][0..3]: the B operand is those 8 probabilities rounded to bf16, and V^T rows hold
//                 their keys in that order, so A is one 16-byte read at slot 8 (l / 16) of the dim's row.
// LDS banks (measured on gfx950 with SQ_LDS_BANK_CONFLICT, one probe dispatch per row stride S in 16-byte units):
// 16-byte reads (ds_read_b128) where lane l takes row l % 16 at column piece l / 16 are conflict-free exactly when
// S = 2 (mod 4) and the rows are taken in lane order; any other stride, or the same rows permuted among the lanes,
// conflicts (and with lane l taking row l % 32 at piece l / 32, odd S). So K rows are D + 16 bf16 (S = D / 8 + 2)
// and V^T rows 48 bf16 (S = 6), read in lane order. The producers' 8-byte V^T writes, whose half wave covers 4
// dims 8 apart, share banks under that stride; they are 8x fewer than the reads (a rotation of the V^T rows that
// spread them made every read conflict: 2,545 against 2,343 us at config 5's batch on 16/2 heads x 256).
constexpr int kB16Depth = 4;    // tiles in flight in producer registers
constexpr int kB16KPad = 16;    // bf16 padding of a K row in LDS
constexpr int kB16VRow = 48;    // bf16 per V^T row in LDS: 32 keys + 16 padding
constexpr int kB16Ahead = 4;    // K and V^T operand reads in flight ahead of their MFMAs
constexpr int kB16Threads = 768;

template <int D, bool TAB_LDS>
__global__ __launch_bounds__(kB16Threads) void prefill_attention_b16(PrefillArgs a) {
    constexpr int KROW = D + kB16KPad;               // K row stride (bf16)
    constexpr int KBUF = kBKP * KROW;                // K bf16 per stage
    constexpr int STAGE = KBUF + D * kB16VRow;       // bf16 per stage: K rows, then V^T rows
    constexpr int PER_ROW = D / 8;                   // 16-byte pieces per row
    constexpr int GROUPS = kBKP / 4;                 // groups of 4 key rows per tile
    constexpr int UNITS_T = GROUPS * PER_ROW;        // staging units per tensor per tile
    static_assert(UNITS_T <= 256 && UNITS_T % 64 == 0, "one K and one V unit per producer lane, whole waves");
    constexpr int DEPTH = kB16Depth;
    static_assert(DEPTH % 2 == 0, "the stage of tile i + d is d % 2 in the loop unrolled by DEPTH");
    constexpr int NC = D / 16;                       // dim tiles of O^T
    constexpr int NQ = D / 32;                       // k-steps of S^T
    extern __shared__ __attribute__((aligned(16))) char smem[];
    uint16_t* lds = reinterpret_cast<uint16_t*>(smem);                                 // [2 stages][K; V^T]
    int* tab = reinterpret_cast<int*>(smem + 2 * STAGE * sizeof(uint16_t));             // [kTabCache] block ids

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const bool producer = wave >= 8;
    const WorkSlot ws = work_slot(a.Hkv, (a.G + kF32Heads - 1) / kF32Heads);
    const int kvh = ws.kvh;
    const int gh = ws.chunk * kF32Heads + (wave & 3);        // head within the group (consumers)
    const int half = (wave >> 2) & 1;
    const int32_t* we = a.work + (long long)kWorkInts * ws.entry;
    const int item = we[0];
    const int seg = item >> 16, qblk = item & 0xffff;
    const int row0 = a.cu[seg] + qblk * kBQ;
    const int nq = min(kBQ, a.cu[seg + 1] - row0);
    const int p0 = a.start[seg] + qblk * kBQ;
    const int n_keys = a.causal ? p0 + nq : a.start[seg] + (a.cu[seg + 1] - a.cu[seg]);
    const int kmin = a.window > 0 ? max(0, p0 - a.window + 1) : 0;
    const int t_first = max(kmin / kBKP, we[1]);
    const int n_tiles = min((n_keys + kBKP - 1) / kBKP, we[2]) - t_first;
    const int32_t* table = a.tables + (long long)seg * a.max_nb;
    const bool active = !producer && gh < a.G && half * kF32QW < nq;     // whole waves
    const int head = kvh * a.G + (gh < a.G ? gh : 0);
    // pos / bs: the estimate from floor((2^32 - 1) / bs) is exact or one short for every pos < 2^32
    auto block_of = [&](int pos, int& r) {
        uint32_t b = __umulhi((uint32_t)pos, a.bs_recip);
        r = pos - (int)b * a.bs;
        if (r >= a.bs) { ++b; r -= a.bs; }
        return (int)b;
    };
    // every position a producer reads lies in [b_lo's first row, the entry's last key]: groups are clamped into
    // the entry's key range (rounded down to 4 for groups below the window)
    int r0;
    const int b_lo = n_tiles > 0 ? block_of(max(kmin, t_first * kBKP) / 4 * 4, r0) : 0;
    if (TAB_LDS) {
        const int b_hi = n_tiles > 0 ? block_of(min(n_keys, (t_first + n_tiles) * kBKP) - 1, r0) : -1;
        for (int i = b_lo + tid; i <= b_hi; i += kB16Threads) {
            const int blk = table[i];
            tab[i - b_lo] = blk < 0 ? 0 : (blk >= a.num_blocks ? a.num_blocks - 1 : blk);
        }
        __syncthreads();
    }
    // an entry without tiles (not produced by the host's work lists) stages nothing; its consumers still write
    // their (empty) split record, so a split item is always combined
    const int n_iter = n_tiles > 0 ? (n_tiles + DEPTH - 1) / DEPTH * DEPTH : 0;

    if (producer) {
        // ---- producer lane pl: K unit pl (piece pl % PER_ROW of rows 4 (pl / PER_ROW) .. + 3: consecutive lanes,
        // consecutive pieces of one row group) and V unit pl (piece pl / GROUPS of rows 4 (pl % GROUPS) .. + 3:
        // consecutive lanes, consecutive key groups). The same code for every lane: a branch between K and V work
        // would make the compiler wait for all loads in flight where the branches join.
        const int pl = tid - 8 * 64;
        if (__builtin_amdgcn_readfirstlane(pl) >= UNITS_T || n_tiles <= 0) {   // whole waves without a unit
            for (int k = 0; k <= n_iter; ++k) lds_barrier();                     // (D < 256), or nothing to stage
            return;
        }
        const int gk = pl / PER_ROW, pk = pl % PER_ROW;
        const int gv = pl % GROUPS, pv = pl / GROUPS;
        const uint16_t* ksrc = reinterpret_cast<const uint16_t*>(a.kp) + (long long)kvh * D + pk * 8;
        const uint16_t* vsrc = reinterpret_cast<const uint16_t*>(a.vp) + (long long)kvh * D + pv * 8;
        const long long rstride = (long long)a.Hkv * D;  // elements between consecutive pool rows
        const bool rows4 = a.bs % 4 == 0;                // a group of 4 aligned keys lies in one block
        auto pool_block = [&](int b) {
            if (TAB_LDS) return tab[b - b_lo];
            const int t = table[b];
            return t < 0 ? 0 : (t >= a.num_blocks ? a.num_blocks - 1 : t);
        };
        // pool row offsets (elements) of keys 4 g .. + 3 of tile t_rel; prefetches past the entry's last tile re-read
        // it, so every position read lies in the entry's own key range, whose block ids are the ones cached
        auto rows_of = [&](int t_rel, int g, long long (&off)[4]) {
            const int p4 = (t_first + min(t_rel, n_tiles - 1)) * kBKP + 4 * g;
            if (rows4) {
                // groups past the end re-read the group holding the last key, groups below the window the one
                // holding its first key: the same block either way (masked, never used)
                int pos = p4 + 3 < n_keys ? p4 : (n_keys - 1) / 4 * 4;
                pos = pos < kmin ? kmin / 4 * 4 : pos;
                int r;
                const int b = block_of(pos, r);
                const long long row = ((long long)pool_block(b) * a.bs + r) * rstride;
#pragma unroll
                for (int j = 0; j < 4; ++j) off[j] = row + j * rstride;
            } else {
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    int pos = p4 + j;
                    pos = pos < n_keys ? pos : n_keys - 1;
                    pos = pos < kmin ? kmin : pos;
                    int r;
                    const int b = block_of(pos, r);
                    off[j] = ((long long)pool_block(b) * a.bs + r) * rstride;
                }
            }
        };
        auto issue = [&](int t_rel, u32x4 (&slot)[8]) {
            long long ok[4], ov[4];
            rows_of(t_rel, gk, ok);
            rows_of(t_rel, gv, ov);
#pragma unroll
            for (int j = 0; j < 4; ++j) slot[j] = *reinterpret_cast<const u32x4*>(ksrc + ok[j]);
#pragma unroll
            for (int j = 0; j < 4; ++j) slot[4 + j] = *reinterpret_cast<const u32x4*>(vsrc + ov[j]);
        };
        auto stash = [&](const u32x4 (&slot)[8], int stage) {
            uint16_t* s = lds + stage * STAGE;
#pragma unroll
            for (int j = 0; j < 4; ++j) *reinterpret_cast<u32x4*>(s + (4 * gk + j) * KROW + pk * 8) = slot[j];
            // V^T row 8 pv + d, keys 4 gv .. + 3 at slots 8 gv (gv < 4) or 8 (gv - 4) + 4; one byte permute per word
            // takes the same 16-bit half (low: even d, high: odd d) of two key rows
            uint16_t* vt = s + KBUF + pv * 8 * kB16VRow + (gv < 4 ? 8 * gv : 8 * (gv - 4) + 4);
#pragma unroll
            for (int d = 0; d < 8; ++d) {
                const uint32_t sel = d & 1 ? 0x07060302u : 0x05040100u;
                const uint32_t w0 = __builtin_amdgcn_perm(slot[5][d / 2], slot[4][d / 2], sel);
                const uint32_t w1 = __builtin_amdgcn_perm(slot[7][d / 2], slot[6][d / 2], sel);
                *reinterpret_cast<u32x2*>(vt + d * kB16VRow) = u32x2{w0, w1};
            }
        };
        // tile t sits in slot t % DEPTH, then in stage t % 2; at iteration t the slot of tile t + 1 goes to LDS (into
        // tile t - 1's stage, released by the barrier that ended iteration t - 1) and is refilled with tile
        // t + 1 + DEPTH. The loop body has no branch, so the compiler counts the loads in flight exactly.
        u32x4 st[DEPTH][8];
#pragma unroll
        for (int d = 0; d < DEPTH; ++d) issue(d, st[d]);
        stash(st[0], 0);
        issue(DEPTH, st[0]);
        lds_barrier();
        for (int i = 0; i < n_iter; i += DEPTH) {
#pragma unroll
            for (int d = 0; d < DEPTH; ++d) {
                stash(st[(d + 1) % DEPTH], (d + 1) & 1);
                issue(i + d + 1 + DEPTH, st[(d + 1) % DEPTH]);
                lds_barrier();
            }
        }
        return;
    }

    // ---- consumer wave
    const int qc = lane & 15, qq = lane >> 4;
    const int qi = half * kF32QW + qc;
    const int qpos = a.causal ? p0 + (qi < nq ? qi : nq - 1) : n_keys - 1;
    const int qlo = a.window > 0 ? qpos - a.window : -1;
    const int qfirst = a.causal ? p0 + half * kF32QW : n_keys - 1;
    const int qlast = a.causal ? p0 + min(half * kF32QW + kF32QW, nq) - 1 : n_keys - 1;
    const int lo_edge = a.window > 0 ? qlast - a.window : INT_MIN;
    u32x4 qop[NQ];                                   // Q[query][32 c + 8 qq .. + 7]
    f32x4 o[NC];                                     // O^T[16 dt + 4 qq + r][query]
    float m_run = -INFINITY, l_run = 0.0f;
    {
        const uint16_t* qp = reinterpret_cast<const uint16_t*>(a.q) +
                             ((long long)(row0 + (qi < nq ? qi : nq - 1)) * a.Hq + head) * D + 8 * qq;
#pragma unroll
        for (int c = 0; c < NQ; ++c) qop[c] = *reinterpret_cast<const u32x4*>(qp + 32 * c);
#pragma unroll
        for (int c = 0; c < NC; ++c) o[c] = f32x4{};
    }

    auto consume = [&](int t_rel, int stage) {
        const uint16_t* ks = lds + stage * STAGE;
        const uint16_t* kr = ks + qc * KROW + 8 * qq;
        const uint16_t* vr = ks + KBUF + qc * kB16VRow + 8 * qq;      // V^T row 16 dt + qc
        auto vread = [&](int dt) { return *reinterpret_cast<const u32x4*>(vr + 16 * dt * kB16VRow); };
        const int k0 = (t_first + t_rel) * kBKP;
        f32x4 s[2] = {f32x4{}, f32x4{}};
        // K operands kB16Ahead reads ahead of their MFMAs (read i: dims 32 (i / 2), keys 16 (i % 2) ..); the
        // scheduling fences keep the compiler from moving the reads back next to their uses
        auto kread = [&](int i) {
            return *reinterpret_cast<const u32x4*>(kr + 16 * (i % 2) * KROW + 32 * (i / 2));
        };
        u32x4 ka[kB16Ahead];
#pragma unroll
        for (int i = 0; i < kB16Ahead; ++i) ka[i] = kread(i);
#pragma unroll
        for (int i = 0; i < 2 * NQ; ++i) {
            const u32x4 cur = ka[i % kB16Ahead];
            if (i + kB16Ahead < 2 * NQ) ka[i % kB16Ahead] = kread(i + kB16Ahead);
            __builtin_amdgcn_sched_barrier(0);
            s[i % 2] = mfma16x16x32(cur, qop[i / 2], s[i % 2]);
            __builtin_amdgcn_sched_barrier(0);
        }
        // lane (qc, qq), register r of sub-tile kt: key k0 + 16 kt + 4 qq + r
        if (k0 + kBKP - 1 > qfirst || k0 <= lo_edge) {
#pragma unroll
            for (int kt = 0; kt < 2; ++kt)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int key = k0 + 16 * kt + 4 * qq + r;
                    s[kt][r] = key <= qpos && key > qlo ? s[kt][r] : -INFINITY;
                }
        }
        // the first V^T operands are requested before the softmax, so their latency passes during it
        u32x4 va[kB16Ahead];
#pragma unroll
        for (int i = 0; i < kB16Ahead; ++i) va[i] = vread(i);
        __builtin_amdgcn_sched_barrier(0);
        const float m_prev = m_run;
        lazy_max(s, m_run, a.qscale);
        const float mb = m_run == -INFINITY ? 0.0f : m_run;
        if (__any(m_run != m_prev)) {
            const float alpha = fast_exp2(m_prev - mb);     // 0 on the first tile (m_prev = -inf)
            l_run *= alpha;
#pragma unroll
            for (int dt = 0; dt < NC; ++dt) o[dt] *= alpha;
        }
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                s[kt][r] = fast_exp2(fmaf(s[kt][r], a.qscale, -mb));
                l_run += s[kt][r];
            }
        const u32x4 pop = u32x4{pack_bf16x2_rne(s[0][0], s[0][1]), pack_bf16x2_rne(s[0][2], s[0][3]),
                                pack_bf16x2_rne(s[1][0], s[1][1]), pack_bf16x2_rne(s[1][2], s[1][3])};
#pragma unroll
        for (int dt = 0; dt < NC; ++dt) {
            const u32x4 cur = va[dt % kB16Ahead];
            if (dt + kB16Ahead < NC) va[dt % kB16Ahead] = vread(dt + kB16Ahead);
            __builtin_amdgcn_sched_barrier(0);
            o[dt] = mfma16x16x32(cur, pop, o[dt]);
            __builtin_amdgcn_sched_barrier(0);
        }
    };

    lds_barrier();                                   // the producers' first tile is in stage 0
    for (int t = 0; t < n_iter; ++t) {
        if (active && t < n_tiles) consume(t, t & 1);
        lds_barrier();
    }
    if (!active) return;
    l_run += __shfl_xor(l_run, 16);                  // each lane summed the probabilities of its own keys
    l_run += __shfl_xor(l_run, 32);
    finish_queries<D>(a, we, o, m_run, l_run, head, half, row0, nq);
}

}  // namespace
}  // namespace rk

using namespace rk;

extern "C" {

size_t rk_paged_prefill_workspace_bytes(int n_slots, int Hq, int D) {
    if (n_slots <= 0 || Hq <= 0 || D <= 0) return 0;
    return (size_t)n_slots * Hq * (kBQ * (size_t)D + 2 * kBQ) * sizeof(float);
}

size_t rk_paged_prefill_counters(int n_slots, int Hq) {
    if (n_slots <= 0 || Hq <= 0) return 0;
    return (size_t)n_slots * Hq * 2;
}

int rk_paged_prefill(float* out, const void* q, int q_dtype, const void* k_new, const void* v_new, int new_dtype,
                     void* k_pool, void* v_pool, int pool_dtype, const int32_t* tables, int max_nb,
                     const int32_t* cu_seqlens, const int32_t* start_pos, const int32_t* work, int n_work, int S,
                     int N, int Hq, int Hkv, int D, int block_size, int num_blocks, const void* gate, int gate_dtype,
                     int window, int causal, int exact, int n_slots, float* partials, size_t partial_bytes,
                     uint32_t* counters, size_t n_counters, void* stream) {
    if (N == 0) return RK_OK;
    if (n_slots < 0 || (n_slots > 0 && (!partials || !counters)))
        return fail(RK_ERR_ARG, "rk_paged_prefill: %d partial slots need partials and counters", n_slots);
    if (n_slots > 0 && (partial_bytes < rk_paged_prefill_workspace_bytes(n_slots, Hq, D) ||
                        n_counters < rk_paged_prefill_counters(n_slots, Hq)))
        return fail(RK_ERR_WORKSPACE, "rk_paged_prefill: %zu partial bytes and %zu counters for %d slots (need %zu "
                    "and %zu)", partial_bytes, n_counters, n_slots, rk_paged_prefill_workspace_bytes(n_slots, Hq, D),
                    rk_paged_prefill_counters(n_slots, Hq));
    if (!out || !q || !k_pool || !v_pool || !tables || !cu_seqlens || !start_pos || !work)
        return fail(RK_ERR_ARG, "rk_paged_prefill: null pointer");
    if (!k_new != !v_new) return fail(RK_ERR_ARG, "rk_paged_prefill: k_new and v_new must both be given or both null");
    if (window < 0 || (window > 0 && !causal))
        return fail(RK_ERR_ARG, "rk_paged_prefill: window %d (>= 0, and only with causal masking)", window);
    if (S < 1 || N < 1 || n_work < 1 || n_work > 65535 * 8 || max_nb < 1 || block_size < 1 || num_blocks < 1)
        return fail(RK_ERR_ARG, "rk_paged_prefill: S %d N %d n_work %d max_nb %d block_size %d", S, N, n_work, max_nb,
                    block_size);
    if (Hkv < 1 || Hq < Hkv || Hq % Hkv)
        return fail(RK_ERR_ARG, "rk_paged_prefill: %d query heads over %d kv heads", Hq, Hkv);
    if ((unsigned long long)n_work * Hq * 768 >= (1ull << 32))   // workgroups (entry, chunk, kv-head) x threads
        return fail(RK_ERR_UNSUPPORTED, "rk_paged_prefill: %d work entries x %d query heads exceed one launch", n_work,
                    Hq);
    if (D != 64 && D != 128 && D != 256)
        return fail(RK_ERR_UNSUPPORTED, "rk_paged_prefill: head_dim %d not in {64, 128, 256}", D);
    if ((unsigned long long)max_nb * block_size >= (1ull << 31))
        return fail(RK_ERR_UNSUPPORTED, "rk_paged_prefill: %d blocks of %d positions (positions must stay below 2^31)",
                    max_nb, block_size);
    // Which kernel. fp32 operands (prefill_attention_f32) for an fp32 q or pool and for exact requests; bf16
    // operands where q and the pool both are bf16: the 32-query kernel (prefill_attention) at 4 query heads per
    // kv-head and head_dim 128 / 256 where its producers' one-multiply block index is exact (positions x block size
    // below 2^32, block_size >= 2: the reciprocal ceil(2^32 / bs) must fit 32 bits), the 16-query kernel
    // (prefill_attention_b16) for every other shape.
    const bool bf16_ops = !exact && q_dtype == RK_BF16 && pool_dtype == RK_BF16;
    const bool wide_q = bf16_ops && Hq == kMaxGroup * Hkv && (D == 128 || D == 256) && block_size >= 2 &&
                        (unsigned long long)max_nb * block_size * block_size < (1ull << 32);
    for (int dt : {q_dtype, k_new ? new_dtype : RK_F32, pool_dtype, gate ? gate_dtype : RK_F32})
        if (dt != RK_F32 && dt != RK_BF16) return fail(RK_ERR_UNSUPPORTED, "rk_paged_prefill: dtype %d", dt);
    PrefillArgs a;
    a.out = out; a.q = q; a.k_new = k_new; a.v_new = v_new; a.kp = k_pool; a.vp = v_pool; a.tables = tables;
    a.cu = cu_seqlens; a.start = start_pos; a.work = work; a.gate = gate; a.gate_dtype = gate_dtype;
    a.window = window; a.causal = causal ? 1 : 0;
    a.q_dtype = q_dtype; a.new_dtype = new_dtype; a.pool_dtype = pool_dtype;
    a.S = S; a.n_work = n_work; a.N = N; a.Hq = Hq; a.Hkv = Hkv; a.G = Hq / Hkv; a.bs = block_size;
    a.max_nb = max_nb; a.num_blocks = num_blocks;
    a.part = partials; a.cnt = counters; a.n_slots = n_slots;
    a.qscale = kLog2e / sqrtf((float)D);
    a.bs_recip_up = block_size >= 2 ? 0xffffffffu / (uint32_t)block_size + 1u : 0u;   // used only when bs >= 2
    a.bs_recip = 0xffffffffu / (uint32_t)block_size;
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (k_new) {
        const long long threads = (long long)N * (Hkv * D / 8);
        hipLaunchKernelGGL(prefill_kv_write, dim3((unsigned)ceil_div((size_t)threads, 256)), dim3(256), 0, s, a, D);
        if (int rc = check_launch("prefill_kv_write")) return rc;
    }
    typedef void (*AttnFn)(PrefillArgs);
    AttnFn fn;
    const bool tab_lds = max_nb <= kTabCache;
    const int chunks = (a.G + kF32Heads - 1) / kF32Heads;   // head chunks of the 16-query kernels
    if (wide_q) {
        const size_t lds = (tab_lds ? kTabCache * 4 : 0) +
                           (size_t)kStages * (kBKP * (D + kKPad) + D * (kBKP + kVPad)) * sizeof(uint16_t);
        if (D == 256) fn = tab_lds ? prefill_attention<256, true> : prefill_attention<256, false>;
        else fn = tab_lds ? prefill_attention<128, true> : prefill_attention<128, false>;
        if (int rc2 = allow_dynamic_lds((const void*)fn, lds)) return rc2;
        hipLaunchKernelGGL(fn, dim3(n_work * Hkv), dim3(2 * 64 * a.G), lds, s, a);
        return check_launch("prefill_attention");
    }
    if (bf16_ops) {
        const size_t lds = (size_t)2 * (kBKP * (D + kB16KPad) + D * kB16VRow) * sizeof(uint16_t) +
                           (tab_lds ? kTabCache * sizeof(int) : 0);
        if (D == 256) fn = tab_lds ? prefill_attention_b16<256, true> : prefill_attention_b16<256, false>;
        else if (D == 128) fn = tab_lds ? prefill_attention_b16<128, true> : prefill_attention_b16<128, false>;
        else fn = tab_lds ? prefill_attention_b16<64, true> : prefill_attention_b16<64, false>;
        if (int rc2 = allow_dynamic_lds((const void*)fn, lds)) return rc2;
        hipLaunchKernelGGL(fn, dim3(n_work * Hkv * chunks), dim3(kB16Threads), lds, s, a);
        return check_launch("prefill_attention_b16");
    }
    const size_t lds = (size_t)2 * (kBKP * (D + kF32Pad) + D * (kBKP + kF32Pad)) * sizeof(float) +
                       (tab_lds ? kTabCache * sizeof(int) : 0);
    const bool f32_pool = pool_dtype == RK_F32;
#define RK_F32_PICK(DD)                                                                                      \
    fn = f32_pool ? (tab_lds ? prefill_attention_f32<DD, float, true> : prefill_attention_f32<DD, float, false>)  \
                  : (tab_lds ? prefill_attention_f32<DD, uint16_t, true> : prefill_attention_f32<DD, uint16_t, false>)
    if (D == 256) RK_F32_PICK(256);
    else if (D == 128) RK_F32_PICK(128);
    else RK_F32_PICK(64);
#undef RK_F32_PICK
    if (int rc2 = allow_dynamic_lds((const void*)fn, lds)) return rc2;
    hipLaunchKernelGGL(fn, dim3(n_work * Hkv * chunks), dim3(512), lds, s, a);
    return check_launch("prefill_attention_f32");
}

}  // extern "C"
