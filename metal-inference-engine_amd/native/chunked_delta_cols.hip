// P3, bf16 inputs: the serial pass over a sequence's chunks with one wave per 16 state columns over all 64 tokens
// of a chunk (delta_chunk_scan_cols). Same maths and precision as chunked_delta.hip, which builds its operands
// (delta_chunk_prep, lane order) and holds the C ABI. Built on its own so that the compiler keeps MFMA results in
// VGPRs here (the piece splits and scalings read them every chunk) without changing the other kernels' allocation.
#include <type_traits>

#include "chunked_delta.h"
#include "rk_internal.h"

namespace rk {
namespace delta {
namespace {

// =====================================================================================================================
// Phase 2 for bf16 inputs: one wave per 16 state columns over all 64 tokens of a chunk
// =====================================================================================================================
// The columns of S evolve independently, so a wave that owns 16 columns for all 64 tokens needs nothing from any
// other wave: X = K S, (Q S)^T, vn = T Y, o^T = (Q S)^T diag(e^G) + vn^T P^T and the update K^T vn' keep the wave's 16
// columns in one MFMA dimension and 64 tokens (or 128 state rows) in the other. Every operand that is a product of
// the chunk (the state, Y, vn) is an accumulator pair of the product before, read in the k order perm_k (see
// pair_of), so no value moves between lanes. K rows, Q rows, T, P (and K^T, by transposed reads of the K rows) come
// from an LDS stage shared by the workgroup: waves 0 and 1 compute (32 columns); waves 2 and 3 fill the stage of
// chunk c+1 (K, Q, V rows by global_load_lds_dwordx4, 1 KB per instruction, no registers; T split into pieces) and
// form chunk c's P while chunk c is computed; one barrier per chunk hands the two stages over. The output of chunk c
// (o^T: 16-byte rows of 4 columns per lane) is formed and stored at the start of chunk c+1, when its P is ready.
// K and Q rows: 16 groups of 4 rows (one 1 KB direct load each); the K and Q groups g share a 2 KB pair at
// pair_base(g), each at an offset kq_group_off(g) (see kq_unit).
__host__ __device__ constexpr int pair_base(int g) { return 2048 * g + 256 * (g >> 1); }
__host__ __device__ constexpr int kq_group_off(int g) { return (g & 1 ? 32 : 0) + (g & 2 ? 16 : 0); }
struct ColStage {
    static constexpr int kK = 0;                        // K rows, group g at kK + pair_base(g) + kq_group_off(g)
    static constexpr int kQ = kK + 1024;                // Q rows, the same
    static constexpr int kT = 34816;                    // T pieces, 18 blocks of 1 KB in lane order
    static constexpr int kP = kT + 18 * 1024;           // P pieces, the same
    static constexpr int kV = kP + 18 * 1024;           // V [64 tokens][32 columns] bf16 of the workgroup's columns
    static constexpr int kCf = kV + kC * 64;            // beta, G, exp(G), exp(G_last - G): 4 x 64 floats
    static constexpr int bytes = kCf + kCoefRows * kC * 4;
};
static_assert(2 * ColStage::bytes <= 160 * 1024, "two stages fit the LDS");
static_assert(pair_base(15) + 2048 + kq_group_off(15) <= ColStage::kT, "the K / Q pairs end before T");

// Byte offset, from kK or kQ, of the 16-byte unit u (dims 8u .. 8u+7) of K / Q row `row`: row t = row & 3 of group
// row >> 2 stores unit u at slot u ^ 4t. So:
//  - a row operand's two 8-byte halves (units 4kd + j and 4kd + 2 + j, j < 2; 4t never has bit 1) are always 32
//    bytes apart, one ds_read2_b64 into the operand's four registers;
//  - the 8 rows x 32 bytes of a transposed read sit on distinct 16-byte slots of the 256-byte bank line (slot 4t^u
//    within a group, the groups 0 / 2 / 1 / 3 slots apart). Row-operand reads see 2-way bank conflicts (counters),
//    which measured no time: the computing waves' issue bounds the kernel.
__device__ __forceinline__ int kq_unit(int row, int u) {
    const int g = row >> 2, t = row & 3;
    return pair_base(g) + kq_group_off(g) + 256 * t + 16 * (u ^ (4 * t));
}

__device__ __forceinline__ void load_to_lds(const void* src, char* dst) {
    __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void*)dst, 16, 0, 0);
}
// the same with the non-temporal cache policy (aux bit 1, `nt`), for rows read by one workgroup only
__device__ __forceinline__ void load_to_lds_nt(const void* src, char* dst) {
    __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void*)dst, 16, 0, 2);
}
typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
// Transposed 8-byte LDS read: within each 16 lanes, lane a + 4 j supplies 4 consecutive bf16 and lane 4 a + b
// receives element b of the 4 lanes a, a + 4, a + 8, a + 12.
__device__ __forceinline__ u32x2 read_tr16(const char* p) {
    const bf16x4_t v = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((__attribute__((address_space(3))) bf16x4_t*)p);
    return __builtin_bit_cast(u32x2, v);
}

// Row operand of row `row` (token) of a K / Q stage, 32-dim step kd, in the k order perm_k: dims 32 kd + 4q .. +3 and
// 32 kd + 16 + 4q .. +3.
__device__ __forceinline__ u32x4 row_operand(const char* base, int row, int kd, int q) {
    const char* rp = base + kq_unit(row, 4 * kd + (q >> 1)) + 8 * (q & 1);
    const u32x2 lo = *reinterpret_cast<const u32x2*>(rp);
    const u32x2 hi = *reinterpret_cast<const u32x2*>(rp + 32);
    return (u32x4){lo[0], lo[1], hi[0], hi[1]};
}

// K^T operand: rows 16 a2 + r (dims) of K^T, tokens 32k + perm_k(8q + e), by two transposed reads of the K rows.
__device__ __forceinline__ u32x4 kt_operand(const char* base, int a2, int k, int lane) {
    const int q = lane >> 4, m = lane & 15;
    const int row0 = 32 * k + 4 * q + (m >> 2);
    const int u = 2 * a2 + ((m & 3) >> 1);
    const char* p0 = base + kq_unit(row0, u) + 8 * (m & 1);
    const u32x2 lo = read_tr16(p0);
    const u32x2 hi = read_tr16(p0 + pair_base(4) - pair_base(0));       // row0 + 16: group + 4, same slot
    return (u32x4){lo[0], lo[1], hi[0], hi[1]};
}

// the 8 fp32 values of an accumulator pair as kNS bf16 pieces in the k order perm_k
__device__ __forceinline__ void pair_pieces(f32x4 lo, f32x4 hi, u32x4 (&o)[kNS]) {
    const float x[8] = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    split8(x, o);
}

__global__ __launch_bounds__(256) void delta_chunk_scan_cols(DeltaArgs p) {
    __shared__ __align__(16) char stage0[ColStage::bytes];
    __shared__ __align__(16) char stage1[ColStage::bytes];
    // all slices of one (sequence, head) get ids congruent mod 8: one XCD, one L2 for their common operand reads
    const int id = blockIdx.x;
    const int slice = (id >> 3) % kSlices;
    const int pair = (id / (8 * kSlices)) * 8 + (id & 7);
    if (pair >= p.n_pairs) return;
    const int s = pair / p.H, h = pair % p.H, H = p.H;
    const int lane = threadIdx.x & 63, ct = threadIdx.x >> 6, q = lane >> 4, r = lane & 15;
    const int T0 = p.cu[s], Tn = p.cu[s + 1] - T0;
    const int gc0 = p.cu_chunks[s];
    // chunks of this sequence; never more than its workspace records (both offsets arrays come from the caller)
    const int nch = min((Tn + kC - 1) / kC, p.cu_chunks[s + 1] - gc0);
    if (nch <= 0) return;                 // empty sequence: state unchanged, no barrier is reached by either wave
    const int col0 = slice * kCols;
    const int col = col0 + 16 * (ct & 1) + r;
    float* Sg = p.S + (long long)(p.seq_index ? p.seq_index[s] : s) * p.s_stride + (long long)h * kDk * kDv + col;
    const uint16_t* Kg = static_cast<const uint16_t*>(p.k);
    const uint16_t* Qg = static_cast<const uint16_t*>(p.q);
    const uint16_t* Vg = static_cast<const uint16_t*>(p.v);

    // Waves 2 and 3 only load and prepare, on SIMDs of their own (a direct load holds its issuing wave for ~90 cycles,
    // which on the computing waves would add up to a third of a chunk). While chunk c is computed, wave WV = ct & 1
    //  - fills its share of chunk c+1's stage: direct loads of the K, Q and V groups j with j % 2 == WV (and of the
    //    coefficient rows: WV 0), and T blocks pair_of = WV, WV + 2, WV + 4, loaded as fp32 from the padded triangle
    //    a chunk ahead and split into pieces;
    //  - computes chunk c's P blocks of the same pairs into chunk c's stage, from the K and Q rows there (complete
    //    since the last barrier): block (a, k) is tiles b = 2k, 2k+1 of P^T = K Q^T (those with b <= a; the others
    //    are zero) times D. The computing waves read them during chunk c+1, when they form chunk c's o.
    // All four waves meet at the one barrier per chunk: after it, stage c+1 and chunk c's P are complete and stage
    // c-1 (whose P chunk c read) is free. A chunk that ends early repeats its last K / Q / V row (rows past the
    // sequence's end have beta 0, so they leave S and the rows before them untouched, and their P entries meet
    // vn = 0).
    if (ct >= 2) {
        auto loader = [&](auto wv_c) __attribute__((always_inline)) {
            constexpr int WV = decltype(wv_c)::value;
            constexpr int kA[3] = {WV, 2, 3};        // block jj = pair WV + 2 jj = (kA[jj], kKs[jj])
            constexpr int kKs[3] = {0, WV, WV};
            uint32_t kq_off[8], v_off[2];
#pragma unroll
            for (int jj = 0; jj < 8; ++jj) {
                const int row = 4 * (2 * jj + WV) + (lane >> 4), u = lane & 15;
                kq_off[jj] = 2u * (uint32_t)(row * H * kDk + 8 * (u ^ (4 * (row & 3))));
            }
#pragma unroll
            for (int jj = 0; jj < 2; ++jj) {
                const int tok = 16 * (2 * jj + WV) + (lane >> 2);
                v_off[jj] = 2u * (uint32_t)(tok * H * kDv + col0 + 8 * (lane & 3));
            }
            // T entries of this lane in block jj: row 16a + r, columns 32k + 4q .. +3 (half 0) and 32k + 16 + 4q ..
            // +3 (half 1). A group past the row's diagonal is not stored: its load reads the row's first group and
            // the value is replaced by zeros; a half past the diagonal for every lane (2k + hf > a) is not loaded.
            uint32_t t_off[3][2], t_keep[3][2];
#pragma unroll
            for (int jj = 0; jj < 3; ++jj) {
                const int row = 16 * kA[jj] + r;
#pragma unroll
                for (int hf = 0; hf < 2; ++hf) {
                    const int colg = 32 * kKs[jj] + 16 * hf + 4 * q;
                    t_keep[jj][hf] = mask_if(colg <= row);
                    t_off[jj][hf] = (uint32_t)(tri_base(row) + (colg <= row ? colg : 0));
                }
            }
            f32x4 tr[3][2];                          // T entries of the next stage, requested a chunk ahead
            auto issue = [&](int c) __attribute__((always_inline)) {
                const float* rec = p.ws + ((size_t)(gc0 + c) * H + h) * kLaneChunkFloats;
#pragma unroll
                for (int jj = 0; jj < 3; ++jj)
#pragma unroll
                    for (int hf = 0; hf < 2; ++hf)
                        tr[jj][hf] = 2 * kKs[jj] + hf <= kA[jj] ? *reinterpret_cast<const f32x4*>(rec + t_off[jj][hf])
                                                                : (f32x4){0.f, 0.f, 0.f, 0.f};
            };
            constexpr int kIssued = 5;               // loads in issue(): the T halves with 2k + hf <= a
            // chunk c's direct loads (K, Q, V, coefficients), rows past the sequence's end repeating its last row
            auto direct = [&](int c, char* stage) __attribute__((always_inline)) {
                const int nt = min(kC, Tn - c * kC);
                const long long row0 = (long long)(T0 + c * kC) * H + h;
                const char* rec = reinterpret_cast<const char*>(p.ws + ((size_t)(gc0 + c) * H + h) * kLaneChunkFloats);
#pragma unroll
                for (int part = 0; part < 2; ++part) {
                    const char* base = reinterpret_cast<const char*>((part == 0 ? Kg : Qg) + row0 * kDk);
                    char* dst = stage + (part == 0 ? ColStage::kK : ColStage::kQ);
#pragma unroll
                    for (int jj = 0; jj < 8; ++jj) {
                        const int g = 2 * jj + WV, row = 4 * g + (lane >> 4), u = lane & 15;
                        const uint32_t off = nt == kC ? kq_off[jj]
                                                      : 2u * (uint32_t)(min(row, nt - 1) * H * kDk + 8 * (u ^ (4 * (row & 3))));
                        load_to_lds(base + off, dst + pair_base(g) + kq_group_off(g));
                    }
                }
                const char* vbase = reinterpret_cast<const char*>(Vg + row0 * kDv);
#pragma unroll
                for (int jj = 0; jj < 2; ++jj) {
                    const int tok = 16 * (2 * jj + WV) + (lane >> 2);
                    const uint32_t off = nt == kC ? v_off[jj]
                                                  : 2u * (uint32_t)(min(tok, nt - 1) * H * kDv + col0 + 8 * (lane & 3));
                    // V columns col0 .. +31 are this workgroup's alone (all four column slices of the head read
                    // the K and Q rows): streamed past the caches, and o likewise below (233.4 against 238.0 µs per
                    // C4 call)
                    load_to_lds_nt(vbase + off, stage + ColStage::kV + 1024 * WV + 2048 * jj);
                }
                if (WV == 0) load_to_lds(rec + 4 * kLaneCoefOff + 16 * lane, stage + ColStage::kCf);
            };
            // T split into pieces, written to the stage's lane-order blocks
            auto put_t = [&](char* stage) __attribute__((always_inline)) {
#pragma unroll
                for (int jj = 0; jj < 3; ++jj) {
                    float x[8];
#pragma unroll
                    for (int e = 0; e < 8; ++e)
                        x[e] = __uint_as_float(__float_as_uint(tr[jj][e >> 2][e & 3]) & t_keep[jj][e >> 2]);
                    u32x4 pc[kNS];
                    split8(x, pc);
                    char* dst = stage + ColStage::kT + 1024 * (WV + 2 * jj) + 16 * lane;
#pragma unroll
                    for (int pi = 0; pi < kNS; ++pi) *reinterpret_cast<u32x4*>(dst + 6 * 1024 * pi) = pc[pi];
                }
            };
            // P of the chunk in `stage` (its K, Q rows and G there), split into pieces and written to its P blocks
            auto put_p = [&](char* stage) __attribute__((always_inline)) {
                const float* gr = reinterpret_cast<const float*>(stage + ColStage::kCf) + kC;
#pragma unroll
                for (int jj = 0; jj < 3; ++jj) {
                    const int a = kA[jj], t = 16 * a + r;
                    const float gq = gr[t];
                    float x[8];
#pragma unroll
                    for (int hb = 0; hb < 2; ++hb) {
                        const int b = 2 * kKs[jj] + hb;
                        f32x4 pq = {0.f, 0.f, 0.f, 0.f};
                        // operands as one 16-byte read of dims 32 kd + 8q .. +7 per lane (the same k order on both
                        // sides; fewer bank conflicts than the computing waves' paired reads)
                        if (b <= a)
#pragma unroll
                            for (int kd = 0; kd < 4; ++kd)
                                pq = mfma16x16x32(
                                    *reinterpret_cast<const u32x4*>(stage + ColStage::kK + kq_unit(16 * b + r, 4 * kd + q)),
                                    *reinterpret_cast<const u32x4*>(stage + ColStage::kQ + kq_unit(t, 4 * kd + q)), pq);
                        const f32x4 gk = *reinterpret_cast<const f32x4*>(gr + 16 * b + 4 * q);
#pragma unroll
                        for (int i = 0; i < 4; ++i) {
                            // P[t][t'] = (q_t . k_t') exp(G_t - G_t') for t' <= t (masked before exp)
                            const int tp = 16 * b + 4 * q + i;
                            const float d = tp <= t ? fast_exp2((gq - gk[i]) * kLog2e) : 0.f;
                            x[4 * hb + i] = pq[i] * d;
                        }
                    }
                    u32x4 pc[kNS];
                    split8(x, pc);
                    char* dst = stage + ColStage::kP + 1024 * (WV + 2 * jj) + 16 * lane;
#pragma unroll
                    for (int pi = 0; pi < kNS; ++pi) *reinterpret_cast<u32x4*>(dst + 6 * 1024 * pi) = pc[pi];
                }
            };
            // Before each barrier the wave waits for its direct loads only (the in-order counter allows the kIssued
            // newer T requests to stay in flight), then for its LDS writes; written out, as a fence would make the
            // compiler wait for every load (it cannot tell the direct loads' LDS writes from the requests).
            // tests/test_build.py checks kIssued against the compiled code.
            auto sync = [&]() __attribute__((always_inline)) {
                asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(kIssued) : "memory");
            };
            // stage 1's P blocks start at zero: chunk 0 forms the o of "chunk -1" from them, with zero factors
#pragma unroll
            for (int jj = 0; jj < 3; ++jj)
#pragma unroll
                for (int pi = 0; pi < kNS; ++pi)
                    *reinterpret_cast<u32x4*>(stage1 + ColStage::kP + 1024 * (6 * pi + WV + 2 * jj) + 16 * lane) =
                        (u32x4){0u, 0u, 0u, 0u};
            issue(0);
            direct(0, stage0);
            put_t(stage0);
            __builtin_amdgcn_sched_barrier(0);
            issue(min(1, nch - 1));
            sync();
            for (int c = 0; c < nch; ++c) {
                char* cur = (c & 1) ? stage1 : stage0;
                char* nxt = (c & 1) ? stage0 : stage1;
                if (c + 1 < nch) {
                    direct(c + 1, nxt);
                    put_t(nxt);
                    __builtin_amdgcn_sched_barrier(0);      // the T requests stay after the direct loads
                    issue(min(c + 2, nch - 1));
                }
                put_p(cur);
                sync();
            }
        };
        if (ct == 2) loader(std::integral_constant<int, 0>{});
        else loader(std::integral_constant<int, 1>{});
        return;
    }

    // state rows 16 a2 + 4q + i, column `col` (accumulator layout of the update)
    f32x4 st[8];
#pragma unroll
    for (int a2 = 0; a2 < 8; ++a2)
#pragma unroll
        for (int i = 0; i < 4; ++i) st[a2][i] = Sg[(long long)(16 * a2 + 4 * q + i) * kDv];
    __syncthreads();                                      // waits for this wave's loads; then both waves' are in LDS

    // o^T of chunk c is formed during chunk c+1 (its P is computed by the loading waves during chunk c, from chunk c's
    // stage) and stored at once: lane (q, r) of tile a holds token 16a + r, columns 16 (wave & 1) + 4q .. +3. What
    // it needs from chunk c is kept in registers: (Q S)^T, vn's pieces and exp(G) of the lane's tokens.
    f32x4 qs_prev[4];
    u32x4 vb_prev[2][kNS];
    float egt_prev[4];
#pragma unroll
    for (int a = 0; a < 4; ++a) {
        qs_prev[a] = (f32x4){0.f, 0.f, 0.f, 0.f};
        egt_prev[a] = 0.f;
    }
#pragma unroll
    for (int k = 0; k < 2; ++k)
#pragma unroll
        for (int pi = 0; pi < kNS; ++pi) vb_prev[k][pi] = (u32x4){0u, 0u, 0u, 0u};
    // o of chunk c (its P in stage `pst`), stored to chunk c's rows
    auto out_chunk = [&](int c, const char* pst) __attribute__((always_inline)) {
        f32x4 o[4];
#pragma unroll
        for (int a = 0; a < 4; ++a) {
#pragma unroll
            for (int i = 0; i < 4; ++i) o[a][i] = egt_prev[a] * qs_prev[a][i];
#pragma unroll
            for (int k = 0; k <= (a >> 1); ++k) {
                u32x4 pb[kTP];
#pragma unroll
                for (int pi = 0; pi < kTP; ++pi)
                    pb[pi] = *reinterpret_cast<const u32x4*>(pst + ColStage::kP + 1024 * (6 * pi + pair_of(a, k)) +
                                                             16 * lane);
                o[a] = mma(vb_prev[k], pb, o[a]);
            }
        }
        const int nt = min(kC, Tn - c * kC);
        float* orow = p.out + ((long long)(T0 + c * kC + r) * H + h) * kDv + col0 + 16 * (ct & 1) + 4 * q;
        auto orow_a = [&](int a) { return reinterpret_cast<f32x4*>(orow + (long long)16 * a * H * kDv); };
        if (nt == kC) {
#pragma unroll
            for (int a = 0; a < 4; ++a) __builtin_nontemporal_store(o[a], orow_a(a));
        } else {
#pragma unroll
            for (int a = 0; a < 4; ++a)
                if (16 * a + r < nt) __builtin_nontemporal_store(o[a], orow_a(a));
        }
    };

    // one chunk on stage `cur` (chunk c); the o of chunk c-1 from stage `prv` (for c = 0: zeros into chunk 0's rows,
    // which chunk 0's own o overwrites later)
    auto step = [&](int c, const char* cur, const char* prv) __attribute__((always_inline)) {
        out_chunk(max(c - 1, 0), prv);
        // this chunk's coefficients and values, read before they are needed
        const float* cf = reinterpret_cast<const float*>(cur + ColStage::kCf);
        const uint16_t* vs = reinterpret_cast<const uint16_t*>(cur + ColStage::kV);
        f32x4 be[4], eg[4], er[4];
        float vv[4][4];
#pragma unroll
        for (int a = 0; a < 4; ++a) {
            be[a] = *reinterpret_cast<const f32x4*>(cf + 16 * a + 4 * q);
            eg[a] = *reinterpret_cast<const f32x4*>(cf + 2 * kC + 16 * a + 4 * q);
            egt_prev[a] = cf[2 * kC + 16 * a + r];          // exp(G) of token 16a + r, for this chunk's o
            er[a] = *reinterpret_cast<const f32x4*>(cf + 3 * kC + 16 * a + 4 * q);
#pragma unroll
            for (int i = 0; i < 4; ++i) vv[a][i] = to_f32(vs[(16 * a + 4 * q + i) * kCols + 16 * ct + r]);
        }
        const float glast = cf[2 * kC + kC - 1];

        // ---- X = K S (B: the state, in perm_k order of its rows) and (Q S)^T (A: the same state pieces)
        f32x4 x[4];
#pragma unroll
        for (int a = 0; a < 4; ++a) x[a] = qs_prev[a] = (f32x4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kd = 0; kd < 4; ++kd) {
            u32x4 sb[kNS];
            pair_pieces(st[2 * kd], st[2 * kd + 1], sb);
#pragma unroll
            for (int a = 0; a < 4; ++a) {
                const u32x4 ka[1] = {row_operand(cur + ColStage::kK, 16 * a + r, kd, q)};
                x[a] = mma(ka, sb, x[a]);
                const u32x4 qb[1] = {row_operand(cur + ColStage::kQ, 16 * a + r, kd, q)};
                qs_prev[a] = mma(sb, qb, qs_prev[a]);
            }
        }

        // ---- Y = beta (V - e^G X), then vn = T Y
        u32x4 yb[2][kNS];
        {
            f32x4 y[4];
#pragma unroll
            for (int a = 0; a < 4; ++a)
#pragma unroll
                for (int i = 0; i < 4; ++i) y[a][i] = be[a][i] * (vv[a][i] - eg[a][i] * x[a][i]);
            pair_pieces(y[0], y[1], yb[0]);
            pair_pieces(y[2], y[3], yb[1]);
        }
        f32x4 vn[4];
#pragma unroll
        for (int a = 0; a < 4; ++a) {
            vn[a] = (f32x4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int k = 0; k <= (a >> 1); ++k) {
                u32x4 ta[kTP];
#pragma unroll
                for (int pi = 0; pi < kTP; ++pi)
                    ta[pi] = *reinterpret_cast<const u32x4*>(cur + ColStage::kT + 1024 * (6 * pi + pair_of(a, k)) +
                                                             16 * lane);
                vn[a] = mma(ta, yb[k], vn[a]);
            }
        }

        // ---- S = e^{G_last} S + K^T (e^{G_last - G} vn); vn's pieces kept for this chunk's o
        u32x4 vq[2][kNS];
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            pair_pieces(vn[2 * k], vn[2 * k + 1], vb_prev[k]);
            f32x4 w0, w1;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                w0[i] = er[2 * k][i] * vn[2 * k][i];
                w1[i] = er[2 * k + 1][i] * vn[2 * k + 1][i];
            }
            pair_pieces(w0, w1, vq[k]);
        }
#pragma unroll
        for (int a2 = 0; a2 < 8; ++a2)
#pragma unroll
            for (int k = 0; k < 2; ++k) {
                if (k == 0)
#pragma unroll
                    for (int i = 0; i < 4; ++i) st[a2][i] *= glast;
                const u32x4 kt[1] = {kt_operand(cur + ColStage::kK, a2, k, lane)};
                st[a2] = mma(kt, vq[k], st[a2]);
            }
        // the loading waves have completed stage c+1 and chunk c's P, and this wave is done with stage `prv`, which
        // they refill next
        __syncthreads();
    };
    for (int c = 0; c < nch; c += 2) {
        step(c, stage0, stage1);
        if (c + 1 < nch) step(c + 1, stage1, stage0);
    }
    out_chunk(nch - 1, (nch - 1) & 1 ? stage1 : stage0);
#pragma unroll
    for (int a2 = 0; a2 < 8; ++a2)
#pragma unroll
        for (int i = 0; i < 4; ++i) Sg[(long long)(16 * a2 + 4 * q + i) * kDv] = st[a2][i];
}

}  // namespace

int launch_scan_cols(const DeltaArgs& a, int grid, hipStream_t stream) {
    hipLaunchKernelGGL(delta_chunk_scan_cols, dim3(grid), dim3(256), 0, stream, a);
    return check_launch("delta_chunk_scan_cols");
}

}  // namespace delta
}  // namespace rk
