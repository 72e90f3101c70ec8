// Decode-time linears (a few rows of activations times a bf16 / INT8 / INT4 weight matrix), gfx950.
//
// Semantics (reference): MetalBackend.linear / _qlinear for M <= 32 rows (src/backend/metal.py:59-133; kernels
// matvec.metal / qmatvec.metal): y [M, N] = x [M, K] (fp32) @ W^T, W [N, K] either bf16 or block-quantized
// (src/quant.py:1-10, 45-56: blocks of 32 weights along a row share fp16 parameters; INT8 w = q * scale, q int8;
// INT4 w = q * scale + min, q in 0..15, element 2j in the low nibble of byte j, 2j+1 in the high nibble), then
// y += bias, y += residual, fp32 throughout.
//
// Design: y [M, N] = X [M, K] W^T on MFMA (v_mfma_f32_16x16x32_bf16): the (up to 16) activation rows are the A
// operand's 16 rows, a 16-row tile of W the B operand's 16 columns. Weights are exact bf16 operands (bf16 as stored;
// INT8 and INT4 codes are small integers), activations enter as their exact three-piece bf16 split
// (x = hi + mid + lo), so every product is exact and accumulates in fp32: fp32-level results (the VALU alternative
// tops out near 2.5 TB/s of INT4 at 8 rows). One MFMA k-extent is one quantization block, so a block's dot products
// come out of three MFMAs and its scale (and min, times the block's activation sum) is applied to them on the VALU.
// Work: a workgroup of 4 waves takes 16, 32 or 64 rows (1, 2 or 4 row tiles, the most that leave 512 workgroups)
// and a 1024-weight K-split, one quarter of the split per wave, so each wave requests all its weights at once (no
// loop over K) and reuses every activation piece it reads from LDS across its row tiles. Splits of one row group
// are added by the last workgroup to finish (see linear_rows_kernel).
#include "rk_device.h"
#include "rk_internal.h"

namespace rk {
namespace {

constexpr int kQB = 32;            // weights per quantization block = the MFMA k-extent
constexpr int kCols = 16;          // activation rows per launch (MFMA columns)

struct LinArgs {
    float* y;                      // [M, N] fp32
    const float* x;                // [M, K] fp32
    const void* w;                 // bf16 [N, K] | int8 [N, K] | uint8 [N, K / 2]
    const uint16_t* scales;        // fp16 [N, K / 32] (quantized types)
    const uint16_t* mins;          // fp16 [N, K / 32] (INT4)
    const float* bias;             // [N] or null
    const float* res;              // [M, N] or null
    float* part;                   // [S, M, N] partial sums (S > 1)
    uint32_t* cnt;                 // [row groups] arrival counters, zero between calls (S > 1)
    const float* aux;              // XF 1: the up rows (row m at aux + m * aux_ld); XF 2: the sums of squares
    long long x_ld, aux_ld;        // row strides (elements) of x and of aux
    const float* nw;               // XF 2: the norm weight [K] (fp32)
    float* ss;                     // [M, ceil(N / 16)] sums of squares of y's 16-column tiles, or null
    float eps;                     // XF 2
    int M, N, K, S;
    int glu;                       // 1: W = [gate; up] (N = 2F rows), y [M, F] = silu(x gate^T) * (x up^T)
};

constexpr int kMaxSsTiles = 128;   // XF 2: at most 128 sums of squares per row (K <= 2048)

template <int WT> struct WTraits;
// BPB: bytes of one block of one row
template <> struct WTraits<RK_W_BF16> { static constexpr int BPB = 64; };
template <> struct WTraits<RK_W_INT8> { static constexpr int BPB = 32; };
template <> struct WTraits<RK_W_INT4> { static constexpr int BPB = 16; };

__device__ __forceinline__ float half_to_f32(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }

// silu(g) * u = g / (1 + exp(-g)) * u with the hardware exp2 and reciprocal: SwiGLU's product, in the one form that
// both the silu * up input transform (XF 1) and the paired [gate; up] output (glu) compute, so they give equal bits.
// The result is the rounded fp32 product, as the reference hands silu * up to the next op as an fp32 tensor: the
// empty asm makes it opaque, since an inlined product would otherwise be contracted into the activation split that
// consumes it (x - hi as fma(a, u, -hi)), whose pieces would then carry the unrounded product.
__device__ __forceinline__ float silu_times(float g, float u) {
    const float d = 1.0f + __builtin_amdgcn_exp2f(-g * 1.4426950408889634f);
    float h = g * __builtin_amdgcn_rcpf(d) * u;
    asm("" : "+v"(h));
    return h;
}

// the weight row behind output row lr of the kernel: lr itself, or with glu (W = [gate; up], N = 2F rows, F % 8 == 0)
// gate rows 8T .. 8T+7 then up rows F + 8T .. F + 8T+7 for 16-row tile T, so that in the MFMA result each gate
// output's up partner is 8 lanes away and the tile's 8 outputs silu(gate) * up are columns 8T .. 8T+7 of y
__device__ __forceinline__ size_t weight_row(const LinArgs& a, int lr) {
    const int c = lr & 15, base = 8 * (lr >> 4) + (c & 7);
    return (size_t)(a.glu ? (c < 8 ? base : (a.N >> 1) + base) : lr);
}

// 8 INT8 codes (one lane's MFMA slots of one block: bytes of lo then hi) as bf16 bits; q in [-127, 127] is exact in
// bf16, and the top half of the fp32 value is its bf16 pattern
__device__ __forceinline__ u32x4 int8_bf16(uint32_t lo, uint32_t hi) {
    u32x4 o;
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int e = 0; e < 2; ++e) {
            const uint32_t w = h ? hi : lo;
            const float f0 = (float)(int)__builtin_amdgcn_sbfe(w, 16 * e, 8);
            const float f1 = (float)(int)__builtin_amdgcn_sbfe(w, 16 * e + 8, 8);
            o[2 * h + e] = pack_hi2(__float_as_uint(f0), __float_as_uint(f1));
        }
    return o;
}

// 8 INT4 codes (4 bytes; byte j holds elements 2j in the low nibble, 2j+1 in the high one) as bf16 bits, in the
// element order 0 2 4 6 1 3 5 7 (kInt4Order; the activations are staged in the same order, so the MFMA's k-sum
// is unchanged). A code q alone in a byte, read as an fp8 e4m3 pattern 0000qqqq, is exactly q * 2^-9 (codes 0-7
// are subnormals m * 2^-9, 8-15 the first normal binade (8 + m) * 2^-9), so v_cvt_scalef32_pk_bf16_fp8 with the
// scale 2^9 turns two such bytes into two exact bf16 integers: 7 instructions for 8 codes.
__device__ __forceinline__ u32x4 int4_bf16(uint32_t v) {
    const uint32_t lo = v & 0x0F0F0F0Fu, hi = (v >> 4) & 0x0F0F0F0Fu;   // codes 0 2 4 6 | 1 3 5 7, one per byte
    u32x4 o;
    o[0] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(lo, 512.0f, false));
    o[1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(lo, 512.0f, true));
    o[2] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(hi, 512.0f, false));
    o[3] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(hi, 512.0f, true));
    return o;
}
// element pairs of the four bf16-pair registers of an INT4 operand (int4_bf16), and of the activation pieces staged
// against it
constexpr int kInt4Order[4][2] = {{0, 2}, {4, 6}, {1, 3}, {5, 7}};

// 4 x 4 transpose over the wave's four 16-lane groups: afterwards register d of lane group g holds what register g
// of lane group d held. v_permlane32_swap exchanges the upper 32 lanes of its first operand with the lower 32 of its
// second, v_permlane16_swap the odd 16-lane groups of the first with the even ones of the second; all 64 lanes must
// be active.
__device__ __forceinline__ u32x4 xpose4(uint32_t a0, uint32_t a1, uint32_t a2, uint32_t a3) {
    const auto s02 = __builtin_amdgcn_permlane32_swap(a0, a2, false, false);
    const auto s13 = __builtin_amdgcn_permlane32_swap(a1, a3, false, false);
    const auto s01 = __builtin_amdgcn_permlane16_swap(s02[0], s13[0], false, false);
    const auto s23 = __builtin_amdgcn_permlane16_swap(s02[1], s13[1], false, false);
    return (u32x4){s01[0], s01[1], s23[0], s23[1]};
}

constexpr int kWaveBlocks = 8;                     // quantization blocks per wave
constexpr int kSplitBlocks = 4 * kWaveBlocks;      // blocks per workgroup (its K-split: 1024 weights)

// Workgroup (row group rg, K-split sp): rows rg*16*RT .. +16*RT-1 against blocks sp*32 .. +31; wave w takes blocks
// 8w .. 8w+7 of the split for all the group's rows (RT 16-row tiles), so the activations a wave reads from LDS feed RT
// tiles of MFMAs. The MFMA computes D[m][n] = sum_k X[m][k] W[n][k]: activation pieces are the A operand, the
// weights the B operand, so a lane's four outputs share weight row n = r and one scale (and min) per block, which the
// lane holds in registers. Each thread requests everything first (its activations for staging, then its rows'
// scales / mins, then its RT tiles' weight chunks; the staging wait covers the activations only), stages activation
// pieces and block sums in LDS behind one barrier, runs the MFMAs, and the four waves' sums meet in LDS (added in
// wave order). With S > 1 splits the workgroup stores its partial sums (device-coherent stores), counts itself in
// for its row group, and the last to arrive adds the S partials in split order (deterministic, whatever the arrival
// order), the bias and the residual, and writes y. Every output's summation order depends on K alone.
template <int WT, int COLS, int RT, bool PV, int XF, int NW>
__global__ __launch_bounds__(64 * NW) void linear_rows_kernel(LinArgs a) {
    using TR = WTraits<WT>;
    constexpr bool QUANT = WT != RK_W_BF16;
    constexpr int SB = NW * kWaveBlocks;           // blocks of the workgroup's K-split (1024 or 2048 weights)
    constexpr int KG = 4 * SB;                     // 8-element k-groups of the split
    constexpr int NT = 64 * NW;                    // threads
    constexpr int XI = COLS * KG / NT;             // staged k-groups (8 activations of one row) per thread
    extern __shared__ __attribute__((aligned(16))) char smem[];
    u32x4* xs = reinterpret_cast<u32x4*>(smem);    // [piece][k-group][activation row]: 3 KG COLS (linear_xs_bytes)
    __shared__ __align__(16) float bsum_s[WT == RK_W_INT4 ? SB * COLS : 4];   // [block][activation row]
    __shared__ int is_last;
    static_assert(NW * RT * 64 * sizeof(f32x4) <= 3 * KG * COLS * sizeof(u32x4), "wave sums reuse the staging buffer");

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int r = lane & 15, grp = lane >> 4;
    const int rg = blockIdx.x / a.S, sp = blockIdx.x % a.S;
    const int row0 = rg * 16 * RT;
    const int nblk = a.K / kQB;
    const int b0 = sp * SB;
    const int nb = min(SB, nblk - b0);             // blocks of this split (>= 1)
    const int wb0 = b0 + wave * kWaveBlocks;       // this wave's first block
    const int nbw = max(0, min(kWaveBlocks, nblk - wb0));

    // ---- requests: activations, parameters, weights (in this order, all before any use)
    // activations: thread k-groups id = tid + NT u, activation row id % COLS, k-group id / COLS (the row varies
    // fastest, so consecutive lanes write consecutive 16 bytes of the staging buffer: no LDS bank conflicts)
    // XF 1: also the up rows
    f32x4 xv[XI][2], xa[XF != 0 ? XI : 1][2];
#pragma unroll
    for (int u = 0; u < XI; ++u) {
        const int id = tid + NT * u;
        const int col = id % COLS, kg = id / COLS;
        const size_t row = (size_t)min(col, a.M - 1);
        const int kk = 8 * min(kg, 4 * nb - 1);
        const f32x4* p = reinterpret_cast<const f32x4*>(a.x + row * a.x_ld + (size_t)kQB * b0 + kk);
        xv[u][0] = p[0];
        xv[u][1] = p[1];
        if constexpr (XF == 1) {
            const f32x4* pu = reinterpret_cast<const f32x4*>(a.aux + row * a.aux_ld + (size_t)kQB * b0 + kk);
            xa[u][0] = pu[0];
            xa[u][1] = pu[1];
        } else if constexpr (XF == 2) {
            const f32x4* pw = reinterpret_cast<const f32x4*>(a.nw + (size_t)kQB * b0 + kk);
            xa[u][0] = pw[0];
            xa[u][1] = pw[1];
        }
    }
    // XF 2: the sums of squares of the rows this wave normalises (rows wave + NW j), up to 8 per lane, branch-free
    constexpr int SSR = XF == 2 ? (COLS / NW > 0 ? COLS / NW : 1) : 1;
    float ssv[SSR][kMaxSsTiles / 64];
    const int n_ss = a.K / 16;
    if constexpr (XF == 2) {
#pragma unroll
        for (int j = 0; j < SSR; ++j) {
            const size_t row = (size_t)min(wave + NW * j, a.M - 1);
#pragma unroll
            for (int q = 0; q < kMaxSsTiles / 64; ++q)
                ssv[j][q] = a.aux[row * a.aux_ld + min(lane + 64 * q, n_ss - 1)];
        }
    }
    __builtin_amdgcn_sched_barrier(0);
    // scales / mins of blocks wb0 .. +7 of row 16t + r: PV (K % 256 == 0) one 16-byte load per tile and kind
    // (wb0 + 8 <= nblk whenever the wave has blocks), else 8 two-byte loads kept unpacked until use
    u32x4 sc[QUANT && PV ? RT : 1], mn[WT == RK_W_INT4 && PV ? RT : 1];
    uint32_t sch[QUANT && !PV ? RT : 1][8], mnh[WT == RK_W_INT4 && !PV ? RT : 1][8];
    if constexpr (QUANT) {
#pragma unroll
        for (int t = 0; t < RT; ++t) {
            const size_t rowp = weight_row(a, min(row0 + 16 * t + r, a.N - 1)) * nblk;
            if constexpr (PV) {
                const size_t i0 = rowp + min(wb0, nblk - kWaveBlocks);
                sc[t] = *reinterpret_cast<const u32x4*>(a.scales + i0);
                if constexpr (WT == RK_W_INT4) mn[t] = *reinterpret_cast<const u32x4*>(a.mins + i0);
            } else {
#pragma unroll
                for (int j = 0; j < kWaveBlocks; ++j) {
                    const size_t i0 = rowp + min(wb0 + j, nblk - 1);
                    sch[t][j] = a.scales[i0];
                    if constexpr (WT == RK_W_INT4) mnh[t][j] = a.mins[i0];
                }
            }
        }
    }
    __builtin_amdgcn_sched_barrier(0);
    // weights, 16 bytes per lane and load: 64 contiguous bytes of each of 16 rows per instruction. bf16: lane group g
    // loads its own k-group of each block. INT8 / INT4: lane group g loads all of block 4q + g (two / one chunks),
    // and a 4 x 4 transpose over the lane groups (xpose4) then hands each lane its k-group of blocks 4q .. 4q+3.
    constexpr int CH = WT == RK_W_INT4 ? 2 : (WT == RK_W_INT8 ? 4 : kWaveBlocks);   // chunks per tile
    u32x4 raw[RT][CH];
#pragma unroll
    for (int t = 0; t < RT; ++t) {
        const uint8_t* wrow = static_cast<const uint8_t*>(a.w) +
                              weight_row(a, min(row0 + 16 * t + r, a.N - 1)) * ((size_t)nblk * TR::BPB);
#pragma unroll
        for (int c = 0; c < CH; ++c) {
            size_t off;
            if constexpr (WT == RK_W_BF16) off = (size_t)min(wb0 + c, nblk - 1) * TR::BPB + 16 * grp;
            else if constexpr (WT == RK_W_INT8) off = (size_t)min(wb0 + 4 * (c >> 1) + grp, nblk - 1) * TR::BPB + 16 * (c & 1);
            else off = (size_t)min(wb0 + 4 * c + grp, nblk - 1) * TR::BPB;
            raw[t][c] = *reinterpret_cast<const u32x4*>(wrow + off);
        }
    }
    __builtin_amdgcn_sched_barrier(0);

    // XF 2: 1 / rms of each row, rms = sqrt(sum / K + eps), from its tiles' sums of squares (a wave tree, lane 0's
    // result)
    __shared__ float rms_s[XF == 2 ? COLS : 1];
    if constexpr (XF == 2) {
#pragma unroll
        for (int j = 0; j < SSR; ++j) {
            float t = 0.0f;
#pragma unroll
            for (int q = 0; q < kMaxSsTiles / 64; ++q) t += lane + 64 * q < n_ss ? ssv[j][q] : 0.0f;
#pragma unroll
            for (int o = 32; o >= 1; o >>= 1) t += __shfl_xor(t, o);
            if (lane == 0 && wave + NW * j < COLS)
                rms_s[wave + NW * j] = __fdiv_rn(1.0f, sqrtf(__fadd_rn(__fdiv_rn(t, (float)a.K), a.eps)));
        }
        __syncthreads();
    }

    // ---- staging: activation pieces [3][KG][COLS]; block sums [32][COLS] (INT4: the four k-groups of a block sit in
    // lanes i, i + COLS, i + 2 COLS, i + 3 COLS and are added pairwise, (s0 + s1) + (s2 + s3), identically in all four)
#pragma unroll
    for (int u = 0; u < XI; ++u) {
        const int id = tid + NT * u;
        const int col = id % COLS, kg = id / COLS;
        const bool ok = col < a.M && kg < 4 * nb;
        float v[8];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            v[e] = ok ? xv[u][0][e] : 0.0f;
            v[4 + e] = ok ? xv[u][1][e] : 0.0f;
        }
        if constexpr (XF == 1) {                    // silu(gate) * up
#pragma unroll
            for (int e = 0; e < 8; ++e) v[e] = silu_times(v[e], ok ? xa[u][e >> 2][e & 3] : 0.0f);
        } else if constexpr (XF == 2) {             // rms_norm: (x * (1 / rms)) * w, each rounded
            const float ir = rms_s[col];
#pragma unroll
            for (int e = 0; e < 8; ++e) v[e] = __fmul_rn(__fmul_rn(v[e], ir), xa[u][e >> 2][e & 3]);
        }
        u32x4 pc[3];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int e0 = WT == RK_W_INT4 ? kInt4Order[q][0] : 2 * q, e1 = WT == RK_W_INT4 ? kInt4Order[q][1] : 2 * q + 1;
            const Split3 s0 = split3(v[e0]), s1 = split3(v[e1]);
            pc[0][q] = pack_hi2(s0.hi, s1.hi);
            pc[1][q] = pack_hi2(s0.mid, s1.mid);
            pc[2][q] = pack_hi2(s0.lo, s1.lo);
        }
#pragma unroll
        for (int p = 0; p < 3; ++p) xs[(p * KG + kg) * COLS + col] = pc[p];
        if constexpr (WT == RK_W_INT4) {
            float sum = 0.0f;
#pragma unroll
            for (int e = 0; e < 8; ++e) sum += v[e];
            sum += __shfl_xor(sum, COLS);           // the block's k-groups sit COLS lanes apart
            sum += __shfl_xor(sum, 2 * COLS);
            if ((kg & 3) == 0) bsum_s[(kg >> 2) * COLS + col] = sum;
        }
    }
    __syncthreads();

    // ---- MFMAs: block wb0 + j; lane (r, grp) supplies activation row r's k-group grp and weight row 16t + r's
    f32x4 acc[RT];
#pragma unroll
    for (int t = 0; t < RT; ++t) acc[t] = (f32x4){0.f, 0.f, 0.f, 0.f};
    // with 8 staged rows, lanes r >= 8 supply A rows 8 .. 15 as copies of rows 0 .. 7: row m of D depends on A's row
    // m alone, and D's rows 8 .. 15 are never stored (M <= 8), so they need no zeroing
    const int cr = COLS == 16 ? r : (r & (COLS - 1));
#pragma unroll
    for (int j = 0; j < kWaveBlocks; ++j) {
        if (j < nbw) {                              // uniform per wave: the last split may hold fewer blocks
            const int kg = 4 * (wave * kWaveBlocks + j) + grp;
            const u32x4 p0 = xs[(0 * KG + kg) * COLS + cr];
            const u32x4 p1 = xs[(1 * KG + kg) * COLS + cr];
            const u32x4 p2 = xs[(2 * KG + kg) * COLS + cr];
            f32x4 bs = {0.f, 0.f, 0.f, 0.f};
            if constexpr (WT == RK_W_INT4) {
                if (4 * grp < COLS) bs = *reinterpret_cast<const f32x4*>(&bsum_s[(wave * kWaveBlocks + j) * COLS + 4 * grp]);
            }
            if constexpr (WT != RK_W_BF16) {
                if ((j & 3) == 0) {                 // blocks j .. j+3 arrive in this wave's lane groups
                    const int q = j >> 2;
#pragma unroll
                    for (int t = 0; t < RT; ++t) {
                        if constexpr (WT == RK_W_INT4) {
                            const u32x4 c = raw[t][q];
                            raw[t][q] = xpose4(c[0], c[1], c[2], c[3]);
                        } else {
                            // qword k (k-group k of the lane group's block) = dwords (2k, 2k+1) of chunks 2q, 2q+1
                            const u32x4 c0 = raw[t][2 * q], c1 = raw[t][2 * q + 1];
                            const u32x4 lo = xpose4(c0[0], c0[2], c1[0], c1[2]);
                            const u32x4 hi = xpose4(c0[1], c0[3], c1[1], c1[3]);
                            raw[t][2 * q] = (u32x4){lo[0], hi[0], lo[1], hi[1]};
                            raw[t][2 * q + 1] = (u32x4){lo[2], hi[2], lo[3], hi[3]};
                        }
                    }
                }
            }
#pragma unroll
            for (int t = 0; t < RT; ++t) {
                const int d = j & 3;
                u32x4 bw;
                if constexpr (WT == RK_W_BF16) bw = raw[t][j];
                else if constexpr (WT == RK_W_INT8)
                    bw = int8_bf16(raw[t][2 * (j >> 2) + (d >> 1)][2 * (d & 1)], raw[t][2 * (j >> 2) + (d >> 1)][2 * (d & 1) + 1]);
                else bw = int4_bf16(raw[t][j >> 2][d]);
                if constexpr (QUANT) {
                    f32x4 d = mfma16x16x32(p0, bw, (f32x4){0.f, 0.f, 0.f, 0.f});
                    d = mfma16x16x32(p1, bw, d);
                    d = mfma16x16x32(p2, bw, d);
                    const float s = half_to_f32((uint16_t)(PV ? sc[t][j >> 1] >> (16 * (j & 1)) : sch[t][j]));
#pragma unroll
                    for (int i = 0; i < 4; ++i) acc[t][i] = fmaf(s, d[i], acc[t][i]);
                    if constexpr (WT == RK_W_INT4) {
                        const float m = half_to_f32((uint16_t)(PV ? mn[t][j >> 1] >> (16 * (j & 1)) : mnh[t][j]));
#pragma unroll
                        for (int i = 0; i < 4; ++i) acc[t][i] = fmaf(m, bs[i], acc[t][i]);
                    }
                } else {
                    acc[t] = mfma16x16x32(p0, bw, acc[t]);
                    acc[t] = mfma16x16x32(p1, bw, acc[t]);
                    acc[t] = mfma16x16x32(p2, bw, acc[t]);
                }
            }
        }
    }

    // ---- the NW waves' sums, in wave order; thread (t, l) then owns outputs m = 4(l/16) + i, n = row0 + 16t + l%16
    __syncthreads();                                // every wave has finished reading the staging buffer
    f32x4* red = reinterpret_cast<f32x4*>(xs);
#pragma unroll
    for (int t = 0; t < RT; ++t) red[(wave * RT + t) * 64 + lane] = acc[t];
    __syncthreads();
    if (tid < RT * 64) {
        const int t = tid >> 6, l = tid & 63;
        // waves in order within groups of 4, the groups in order: with 8 waves over the whole K, the association of
        // two 4-wave K-splits added by the last arriver, so a row's result does not depend on which form ran
        f32x4 s;
#pragma unroll
        for (int g4 = 0; g4 < NW / 4; ++g4) {
            f32x4 sg = red[(4 * g4 * RT + t) * 64 + l];
#pragma unroll
            for (int w = 4 * g4 + 1; w < 4 * g4 + 4; ++w) {
                const f32x4 o = red[(w * RT + t) * 64 + l];
#pragma unroll
                for (int i = 0; i < 4; ++i) sg[i] += o[i];
            }
            if (g4 == 0) s = sg;
            else {
#pragma unroll
                for (int i = 0; i < 4; ++i) s[i] += sg[i];
            }
        }
        const int n = row0 + 16 * t + (l & 15), m0 = 4 * (l >> 4);
        float sq[4] = {0.f, 0.f, 0.f, 0.f};
        if (a.glu && a.S == 1) {                    // uniform: lanes l % 16 < 8 hold gates, l % 16 >= 8 their ups
            float u[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) u[i] = __shfl_xor(s[i], 8);
            if ((l & 8) == 0 && n < a.N) {
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    if (m0 + i < a.M) a.y[(size_t)(m0 + i) * (a.N >> 1) + 8 * (n >> 4) + (l & 7)] = silu_times(s[i], u[i]);
            }
        } else if (n < a.N) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int m = m0 + i;
                if (m < a.M) {
                    if (a.S == 1) {
                        float v = s[i];
                        if (a.bias) v = __fadd_rn(v, a.bias[n]);
                        if (a.res) v = __fadd_rn(v, a.res[(size_t)m * a.N + n]);
                        a.y[(size_t)m * a.N + n] = v;
                        sq[i] = v * v;
                    } else {
                        __hip_atomic_store(&a.part[((size_t)sp * a.M + m) * a.N + n], s[i], __ATOMIC_RELAXED,
                                           __HIP_MEMORY_SCOPE_AGENT);
                    }
                }
            }
        }
        if (a.S == 1 && a.ss) {                     // uniform: the tile's 16 lanes add their squares (lane 0's sum)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
#pragma unroll
                for (int o = 1; o < 16; o <<= 1) sq[i] += __shfl_xor(sq[i], o);
                if ((l & 15) == 0 && m0 + i < a.M && row0 + 16 * t < a.N) a.ss[(size_t)(m0 + i) * ((a.N + 15) / 16) + (row0 + 16 * t) / 16] = sq[i];
            }
        }
    }
    if (a.S == 1) return;
    // every partial store of the workgroup is complete (acknowledged at the device-coherent level: they are
    // agent-scope atomic stores) before the workgroup counts itself in
    __builtin_amdgcn_s_waitcnt(0x0F70);             // vmcnt(0): loads and stores issued so far have completed
    __syncthreads();
    if (tid == 0) {
        const uint32_t before = __hip_atomic_fetch_add(&a.cnt[rg], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        is_last = before == (uint32_t)(a.S - 1);
    }
    __syncthreads();
    if (!is_last) return;
    // the 16 outputs of one 16-column tile are 16 consecutive lanes (16 RT divides the row's count), so the tile's
    // sum of squares is a 16-lane tree (lane 0's sum)
    for (int i = tid; i < a.M * 16 * RT; i += NT) {
        const int m = i / (16 * RT), n = row0 + i % (16 * RT);
        float v = 0.0f;
        if (n < a.N) {
            for (int q = 0; q < a.S; ++q)
                v += __hip_atomic_load(&a.part[((size_t)q * a.M + m) * a.N + n], __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
            if (a.bias) v = __fadd_rn(v, a.bias[n]);
            if (a.res) v = __fadd_rn(v, a.res[(size_t)m * a.N + n]);
            if (!a.glu) a.y[(size_t)m * a.N + n] = v;
        }
        if (a.glu) {                                // uniform: the up partner of output n is output n + 8, 8 lanes on
            const float u = __shfl_xor(v, 8);
            if ((n & 8) == 0 && n < a.N) a.y[(size_t)m * (a.N >> 1) + 8 * (n >> 4) + (n & 7)] = silu_times(v, u);
        }
        if (a.ss) {                                 // uniform
            float q2 = v * v;
#pragma unroll
            for (int o = 1; o < 16; o <<= 1) q2 += __shfl_xor(q2, o);
            if ((i & 15) == 0 && n < a.N) a.ss[(size_t)m * ((a.N + 15) / 16) + (n >> 4)] = q2;
        }
    }
    if (tid == 0) __hip_atomic_store(&a.cnt[rg], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Long INT8 matrices (the tied LM head: N ~ 2.5e5 rows, half a GB): a persistent grid of one 8-wave workgroup per
// CU. linear_rows_kernel gives such a matrix thousands of short workgroups, each staging the activations again and
// adding its K-split through memory, with no weight loads in flight between one workgroup's requests and the next's.
// Here each workgroup stages the (up to 8) activation rows once for the whole K (three bf16 pieces, 48 K bytes of
// LDS; the RMSNorm of XF 2 applied as in linear_rows_kernel), then every wave streams whole 16-row tiles of its
// share of the rows over the full K, in chunks of 512 weights per row, one chunk ahead in a two-slot register ring:
// no cross-wave or cross-workgroup reduction, and every output's blocks are added in order (a different order from
// linear_rows_kernel's, within 1e-6 of it). The grid's waves take the tiles in turn (wave g of W: tiles g, g + W,
// ...), so that at any time all of them read one contiguous stretch of the matrix (4 % faster than contiguous
// shares per workgroup), in rounds of up to kLongRound tiles. Inside a round the stream holds loads only: the loads
// of chunk s + 1 are issued (from a clamped index, so unconditionally) before chunk s is used, and a finished tile's outputs
// go to the wave's LDS area, so that the compiler's count of loads in flight stays exact (a store or a conditional
// load in the stream makes it wait for every load); the round's outputs are written (with bias, residual and sums
// of squares) after its stream.
constexpr int kLongWaves = 8;                      // waves per workgroup (two per SIMD)
constexpr int kLongChunk = 512;                    // weights per row and chunk: 16 blocks
constexpr int kLongRound = 12;                     // tiles per wave and round (their outputs wait in LDS); even
constexpr int kLongSlots = 2;                      // chunks held per wave: one in flight while one is used
constexpr int kLongMinRows = 65536;                // the long path from this many output rows

template <int XF>
__global__ __launch_bounds__(64 * kLongWaves) void linear_long_int8_kernel(LinArgs a) {
    constexpr int COLS = 8;
    constexpr int CB = kLongChunk / kQB;           // blocks per chunk (16)
    extern __shared__ __attribute__((aligned(16))) char smem[];
    u32x4* xs = reinterpret_cast<u32x4*>(smem);    // [piece][k-group][activation row]
    __shared__ float rms_s[COLS];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);   // uniform: the tile arithmetic stays scalar
    const int r = lane & 15, grp = lane >> 4;
    const int K = a.K, KG = K / 8, nblk = K / kQB, nch = K / kLongChunk;   // nch even (K % 1024 == 0)
    float* outs = reinterpret_cast<float*>(smem + (size_t)3 * KG * COLS * sizeof(u32x4)) + wave * kLongRound * COLS * 16;

    // ---- staging, once: XF 2 first needs each row's 1 / rms (wave v < 8: row v, from its K / 16 tile sums)
    if constexpr (XF == 2) {
        if (wave < COLS) {                         // uniform per wave
            const int n_ss = K / 16;
            const size_t row = (size_t)min(wave, a.M - 1);
            float t = 0.0f;
#pragma unroll
            for (int q = 0; q < kMaxSsTiles / 64; ++q) {
                const int i = lane + 64 * q;
                const float v = a.aux[row * a.aux_ld + min(i, n_ss - 1)];
                t += i < n_ss ? v : 0.0f;
            }
#pragma unroll
            for (int o = 32; o >= 1; o >>= 1) t += __shfl_xor(t, o);
            if (lane == 0) rms_s[wave] = __fdiv_rn(1.0f, sqrtf(__fadd_rn(__fdiv_rn(t, (float)K), a.eps)));
        }
        __syncthreads();
    }
    for (int id = tid; id < KG * COLS; id += 64 * kLongWaves) {
        const int col = id % COLS, kg = id / COLS;
        const bool ok = col < a.M;
        const f32x4* p = reinterpret_cast<const f32x4*>(a.x + (size_t)min(col, a.M - 1) * a.x_ld + 8 * kg);
        const f32x4 x0 = p[0], x1 = p[1];
        float v[8];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            v[e] = ok ? x0[e] : 0.0f;
            v[4 + e] = ok ? x1[e] : 0.0f;
        }
        if constexpr (XF == 2) {
            const f32x4* pw = reinterpret_cast<const f32x4*>(a.nw + 8 * kg);
            const f32x4 w0 = pw[0], w1 = pw[1];
            const float ir = rms_s[col];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                v[e] = __fmul_rn(__fmul_rn(v[e], ir), w0[e]);
                v[4 + e] = __fmul_rn(__fmul_rn(v[4 + e], ir), w1[e]);
            }
        }
        u32x4 pc[3];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const Split3 s0 = split3(v[2 * q]), s1 = split3(v[2 * q + 1]);
            pc[0][q] = pack_hi2(s0.hi, s1.hi);
            pc[1][q] = pack_hi2(s0.mid, s1.mid);
            pc[2][q] = pack_hi2(s0.lo, s1.lo);
        }
#pragma unroll
        for (int pp = 0; pp < 3; ++pp) xs[(pp * KG + kg) * COLS + col] = pc[pp];
    }
    __syncthreads();

    // ---- the wave's tiles
    const int T = (a.N + 15) / 16;
    const int NWV = gridDim.x * kLongWaves, gv = blockIdx.x * kLongWaves + wave;   // the grid's waves; this one
    const int my_tiles = T > gv ? (T - gv + NWV - 1) / NWV : 0;
    const int cr = r & (COLS - 1);                 // lanes r >= 8: copies of rows 0 .. 7 (D's rows 8 .. 15 unused)
    auto tile_of = [&](int i) { return gv + NWV * i; };   // the wave's i-th tile

    u32x4 raw[kLongSlots][8], sc[kLongSlots][2];
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    for (int t0 = 0; t0 < my_tiles; t0 += kLongRound) {
        // S_real chunks; the stream runs S, a multiple of the ring's 4 slots: with 2 chunks per tile an odd tile
        // count gets one more tile, computed from the round's last chunk again and never written out (its LDS
        // outputs lie past the round's tiles, within the area: kLongRound is even)
        const int nt = min(kLongRound, my_tiles - t0), S_real = nt * nch;
        const int S = (kLongSlots > 2 && nch == 2 ? (nt + 1) & ~1 : nt) * nch;
        // chunk s of the round: the wave's tile t0 + s / nch, blocks 16 (s % nch) .. +15; lane group g loads blocks
        // 4q + g (32 bytes: two 16-byte loads) of row 16 tile + r, and every lane its row's 16 scales of the chunk
        auto load = [&](int s, int slot) {
            s = min(s, S_real - 1);
            const int b0 = CB * (s % nch);
            const size_t n = (size_t)min(16 * tile_of(t0 + s / nch) + r, a.N - 1);
            const uint8_t* wrow = static_cast<const uint8_t*>(a.w) + n * (size_t)K;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const u32x4* p = reinterpret_cast<const u32x4*>(wrow + (size_t)kQB * (b0 + 4 * q + grp));
                raw[slot][2 * q] = p[0];
                raw[slot][2 * q + 1] = p[1];
            }
            const u32x4* ps = reinterpret_cast<const u32x4*>(a.scales + n * nblk + b0);
            sc[slot][0] = ps[0];
            sc[slot][1] = ps[1];
        };
        auto compute = [&](int s, int slot) {
            const int c = s % nch, b0 = CB * c;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                // qword k (k-group k of the lane group's block) = dwords (2k, 2k+1) of the block's two 16-byte pieces
                const u32x4 c0 = raw[slot][2 * q], c1 = raw[slot][2 * q + 1];
                const u32x4 xl = xpose4(c0[0], c0[2], c1[0], c1[2]);
                const u32x4 xh = xpose4(c0[1], c0[3], c1[1], c1[3]);
                const u32x4 w2[2] = {{xl[0], xh[0], xl[1], xh[1]}, {xl[2], xh[2], xl[3], xh[3]}};
#pragma unroll
                for (int d = 0; d < 4; ++d) {
                    const int blk = 4 * q + d;     // block of the chunk
                    const int kg = 4 * (b0 + blk) + grp;
                    const u32x4 p0 = xs[(0 * KG + kg) * COLS + cr];
                    const u32x4 p1 = xs[(1 * KG + kg) * COLS + cr];
                    const u32x4 p2 = xs[(2 * KG + kg) * COLS + cr];
                    const u32x4 bw = int8_bf16(w2[d >> 1][2 * (d & 1)], w2[d >> 1][2 * (d & 1) + 1]);
                    f32x4 dd = mfma16x16x32(p0, bw, (f32x4){0.f, 0.f, 0.f, 0.f});
                    dd = mfma16x16x32(p1, bw, dd);
                    dd = mfma16x16x32(p2, bw, dd);
                    const float sv = half_to_f32((uint16_t)(sc[slot][blk >> 3][(blk & 7) >> 1] >> (16 * (blk & 1))));
#pragma unroll
                    for (int i = 0; i < 4; ++i) acc[i] = fmaf(sv, dd[i], acc[i]);
                }
            }
            if (c == nch - 1) {                    // tile done: lane (r, g < 2) holds rows 4g + i, column r
                if (grp < 2)
                    *reinterpret_cast<f32x4*>(&outs[((s / nch) * COLS + 4 * grp) * 16 + 4 * r]) = acc;
                acc = (f32x4){0.f, 0.f, 0.f, 0.f};
            }
        };
        // (the scheduling barriers keep each chunk's loads ahead of the previous chunk's arithmetic)
#pragma unroll
        for (int u = 0; u < kLongSlots - 1; ++u) load(u, u);
        for (int s = 0; s < S; s += kLongSlots) {  // S is a multiple of the slot count
#pragma unroll
            for (int u = 0; u < kLongSlots; ++u) {
                load(s + u + kLongSlots - 1, (u + kLongSlots - 1) % kLongSlots);
                __builtin_amdgcn_sched_barrier(0);
                compute(s + u, u);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
        wave_lds_sync();
        // the round's outputs: element e = (tile i, row m, column j) of the wave's area, 16 columns per 16 lanes
        for (int e = lane; e < nt * COLS * 16; e += 64) {
            const int i = e / (COLS * 16), m = (e / 16) % COLS, j = e % 16;
            const int tile = tile_of(t0 + i), n = 16 * tile + j;
            const f32x4 q4 = *reinterpret_cast<const f32x4*>(&outs[(i * COLS + (m & ~3)) * 16 + 4 * j]);
            float v = q4[m & 3];
            const bool ok = m < a.M && n < a.N;
            if (ok && a.bias) v = __fadd_rn(v, a.bias[n]);
            if (ok && a.res) v = __fadd_rn(v, a.res[(size_t)m * a.N + n]);
            if (ok) a.y[(size_t)m * a.N + n] = v;
            if (a.ss) {                            // uniform
                float q2 = ok ? v * v : 0.0f;
#pragma unroll
                for (int o = 1; o < 16; o <<= 1) q2 += __shfl_xor(q2, o);
                if (j == 0 && m < a.M) a.ss[(size_t)m * T + tile] = q2;
            }
        }
        wave_lds_sync();                           // the area is rewritten by the next round
    }
}

// Row tiles per workgroup: the most (4; 2 for bf16, whose weight slots are 4x wider than INT4's) that still leave
// min_groups workgroups, down to 1: 512, and 256 for the fused silu * up input, whose workgroups stage twice the
// activation bytes (gate and up rows), so more weight rows per workgroup pay for them. Staged activation rows: 8 for
// M <= 8, else 16. Quantized weights with K = 2048 at up to 8 rows (`wide`: 16-byte parameter loads, no silu * up
// input) instead take one 8-wave workgroup over the whole K, with no K-split and so no reduction through memory,
// and the row tiles per workgroup (1 to 4) that fit the tiles into the fewest rounds of one workgroup per CU, then
// the fewest rounds. None of this changes any output's summation order (blocks in order within a wave, waves in
// order, splits in order).
struct LinPlan {
    int cols, rt, S, groups, nw;
};

constexpr bool kWideLinears = true;

LinPlan lin_plan(int M, int N, int K, int w_type, int min_groups = 512, bool wide = false) {
    LinPlan p;
    p.cols = M <= 8 ? 8 : 16;
    p.nw = 4;
    const int nblk = K / kQB;
    if (kWideLinears && wide && p.cols == 8 && w_type != RK_W_BF16 && nblk == 8 * kWaveBlocks) {
        int cus = device_cus();
        if (cus <= 0) cus = 256;
        const long long T = (N + 15) / 16;
        long long best_cost = -1, best_rounds = 0;
        for (int rt = 1; rt <= 4; ++rt) {
            const long long g = (T + rt - 1) / rt, rounds = (g + cus - 1) / cus, cost = rounds * rt;
            if (best_cost < 0 || cost < best_cost || (cost == best_cost && rounds < best_rounds)) {
                best_cost = cost;
                best_rounds = rounds;
                p.rt = rt;
            }
        }
        p.nw = 8;
        p.S = 1;
        p.groups = (int)((T + p.rt - 1) / p.rt);
        return p;
    }
    p.S = (nblk + kSplitBlocks - 1) / kSplitBlocks;
    p.rt = w_type == RK_W_BF16 ? 2 : 4;
    while (p.rt > 1 && (long long)((N + 16 * p.rt - 1) / (16 * p.rt)) * p.S < min_groups) p.rt /= 2;
    p.groups = (N + 16 * p.rt - 1) / (16 * p.rt);
    return p;
}

// the staging buffer of linear_rows_kernel: three bf16 pieces of COLS rows over the workgroup's K-split
constexpr size_t linear_xs_bytes(int cols, int nw) { return (size_t)3 * 4 * nw * kWaveBlocks * cols * 16; }

// rows of W as fp32 (the reference's dequantize, src/quant.py:45-56: q * scale, + min for INT4, each rounded):
// out[i, k] for i < n_rows, source row rows ? rows[i] : row0 + i. One thread per 8 weights.
template <int WT>
__global__ __launch_bounds__(256) void dequant_rows_kernel(float* out, const void* w, const uint16_t* scales,
                                                           const uint16_t* mins, const int32_t* rows, int row0,
                                                           int n_rows, int K, int N) {
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    const int per_row = K / 8;
    if (i >= (long long)n_rows * per_row) return;
    const int ri = (int)(i / per_row), k0 = (int)(i % per_row) * 8;
    int src = rows ? rows[ri] : row0 + ri;
    src = src < 0 ? 0 : (src >= N ? N - 1 : src);
    float v[8];
    if constexpr (WT == RK_W_BF16) {
        const u32x4 q = *reinterpret_cast<const u32x4*>(static_cast<const uint16_t*>(w) + (size_t)src * K + k0);
#pragma unroll
        for (int j = 0; j < 4; ++j) { v[2 * j] = bf16_lo(q[j]); v[2 * j + 1] = bf16_hi(q[j]); }
    } else {
        const size_t pb = (size_t)src * (K / kQB) + k0 / kQB;
        const float s = half_to_f32(scales[pb]);
        if constexpr (WT == RK_W_INT8) {
            const u32x2 q = *reinterpret_cast<const u32x2*>(static_cast<const int8_t*>(w) + (size_t)src * K + k0);
#pragma unroll
            for (int e = 0; e < 8; ++e) v[e] = __fmul_rn((float)(int)__builtin_amdgcn_sbfe(q[e >> 2], 8 * (e & 3), 8), s);
        } else {
            const float mn = half_to_f32(mins[pb]);
            const uint8_t* wb = static_cast<const uint8_t*>(w) + (size_t)src * (K / 2) + k0 / 2;
            const uint32_t q = *reinterpret_cast<const uint32_t*>(wb);
#pragma unroll
            for (int e = 0; e < 8; ++e)
                v[e] = __fadd_rn(__fmul_rn((float)__builtin_amdgcn_ubfe(q, 4 * e, 4), s), mn);
        }
    }
    float4* o = reinterpret_cast<float4*>(out + (size_t)ri * K + k0);
    o[0] = make_float4(v[0], v[1], v[2], v[3]);
    o[1] = make_float4(v[4], v[5], v[6], v[7]);
}

}  // namespace
}  // namespace rk

using namespace rk;

extern "C" {

size_t rk_linear_workspace_bytes(int M, int N, int K, int w_type) {
    if (M < 1 || M > kCols || N < 1 || K < kQB || K % kQB) return 0;
    const LinPlan p = lin_plan(M, N, K, w_type);
    return p.S == 1 ? 0 : (size_t)p.S * M * N * sizeof(float);
}

}  // extern "C"

namespace {

// rk_linear_rows_ex2, and with glu rk_swiglu_rows (N = 2F weight rows, y [M, F]; no bias, residual or sums of squares)
int linear_rows_impl(float* y, float* ss_out, const float* x, long long x_ld, int x_op, const float* aux,
                     long long aux_ld, const float* norm_w, float eps, int M, int N, int K, const void* w, int w_type,
                     const void* scales, const void* mins, const float* bias, const float* residual, float* partials,
                     size_t partial_bytes, uint32_t* counters, int n_counters, bool glu, void* stream) {
    if (M == 0 || N == 0) return RK_OK;
    const bool quant = w_type == RK_W_INT8 || w_type == RK_W_INT4;
    if (!y || !x || !w || (quant && !scales) || (w_type == RK_W_INT4 && !mins) || (x_op != RK_X_PLAIN && !aux))
        return fail(RK_ERR_ARG, "rk_linear_rows: null pointer");
    if (w_type != RK_W_BF16 && !quant) return fail(RK_ERR_UNSUPPORTED, "rk_linear_rows: weight type %d", w_type);
    if (M < 0 || M > kCols || N < 0 || K < kQB || K % kQB)
        return fail(RK_ERR_ARG, "rk_linear_rows: M %d (1..%d), N %d, K %d (a multiple of %d)", M, kCols, N, K, kQB);
    if (reinterpret_cast<uintptr_t>(x) % 16 || reinterpret_cast<uintptr_t>(w) % 16 || x_ld < K || x_ld % 4)
        return fail(RK_ERR_ARG, "rk_linear_rows: x and w must be 16-byte aligned, x rows at a stride >= K of 4n");
    // 16-byte parameter loads: K % 256 == 0 and 16-byte aligned scale / min arrays
    const bool pv = (K / kQB) % kWaveBlocks == 0 && reinterpret_cast<uintptr_t>(scales) % 16 == 0 &&
                    reinterpret_cast<uintptr_t>(mins) % 16 == 0;
    if (x_op != RK_X_PLAIN) {
        if (x_op != RK_X_SILU_MUL && x_op != RK_X_RMS_NORM)
            return fail(RK_ERR_ARG, "rk_linear_rows: input transform %d", x_op);
        if (M > 8 || !pv)
            return fail(RK_ERR_UNSUPPORTED, "rk_linear_rows: the fused input transform needs M <= 8 and K %% 256 == 0: "
                        "M %d, K %d", M, K);
        if (x_op == RK_X_SILU_MUL && (reinterpret_cast<uintptr_t>(aux) % 16 || aux_ld < K || aux_ld % 4))
            return fail(RK_ERR_ARG, "rk_linear_rows: up rows must be 16-byte aligned, at a stride >= K of 4n");
        if (x_op == RK_X_RMS_NORM) {
            if (!norm_w || reinterpret_cast<uintptr_t>(norm_w) % 16)
                return fail(RK_ERR_ARG, "rk_linear_rows: the norm weight must be a 16-byte aligned fp32 vector");
            if (aux_ld < K / 16 || K / 16 > kMaxSsTiles)
                return fail(RK_ERR_ARG, "rk_linear_rows: %d sums of squares per row (at most %d) at a stride of %lld",
                            K / 16, kMaxSsTiles, aux_ld);
        }
    }
    // long INT8 matrices: the persistent kernel (no partials or counters used)
    if (!glu && w_type == RK_W_INT8 && M <= 8 && N >= kLongMinRows && K % (2 * kLongChunk) == 0 && K / 16 <= kMaxSsTiles && pv &&
        (x_op == RK_X_PLAIN || x_op == RK_X_RMS_NORM)) {
        LinArgs a{};
        a.y = y; a.x = x; a.w = w; a.scales = static_cast<const uint16_t*>(scales);
        a.bias = bias; a.res = residual; a.aux = aux; a.x_ld = x_ld; a.aux_ld = aux_ld;
        a.nw = norm_w; a.ss = ss_out; a.eps = eps; a.M = M; a.N = N; a.K = K; a.S = 1;
        int cus = device_cus();
        if (cus <= 0) cus = 256;
        const int T = (N + 15) / 16;
        const size_t lds = (size_t)3 * (K / 8) * 8 * sizeof(u32x4) + (size_t)kLongWaves * kLongRound * 8 * 16 * 4;
        const auto fn = x_op == RK_X_RMS_NORM ? linear_long_int8_kernel<2> : linear_long_int8_kernel<0>;
        if (int rc = allow_dynamic_lds((const void*)fn, lds)) return rc;
        hipLaunchKernelGGL(fn, dim3((unsigned)(cus < T ? cus : T)), dim3(64 * kLongWaves), lds,
                           static_cast<hipStream_t>(stream), a);
        return check_launch("linear_long_int8");
    }
    const LinPlan p = lin_plan(M, N, K, w_type, x_op == RK_X_SILU_MUL ? 256 : 512,
                               pv && (x_op == RK_X_PLAIN || x_op == RK_X_RMS_NORM));
    const size_t need = p.S == 1 ? 0 : rk_linear_workspace_bytes(M, N, K, w_type);
    if (need && (!partials || partial_bytes < need || !counters || n_counters < p.groups))
        return fail(RK_ERR_WORKSPACE, "rk_linear_rows: partials %zu bytes (need %zu), %d counters (need %d)",
                    partial_bytes, need, n_counters, p.groups);
    if ((long long)p.groups * p.S >= (1ll << 31)) return fail(RK_ERR_ARG, "rk_linear_rows: N %d too large", N);
    LinArgs a;
    a.y = y; a.x = x; a.w = w; a.scales = static_cast<const uint16_t*>(scales);
    a.mins = static_cast<const uint16_t*>(mins); a.bias = bias; a.res = residual;
    a.cnt = counters;
    a.part = partials;
    a.aux = aux; a.x_ld = x_ld; a.aux_ld = aux_ld;
    a.nw = norm_w; a.ss = ss_out; a.eps = eps;
    a.M = M; a.N = N; a.K = K; a.S = p.S; a.glu = glu ? 1 : 0;
    using Fn = void (*)(LinArgs);
    Fn fn = nullptr;
#define RK_LIN_PICK(C, R, V, X)                                                                                \
    if (p.nw == 4 && p.cols == C && p.rt == R && pv == V && x_op == X)                                         \
        fn = w_type == RK_W_BF16 ? linear_rows_kernel<RK_W_BF16, C, (R > 2 ? 2 : R), V, X, 4>                  \
             : w_type == RK_W_INT8 ? linear_rows_kernel<RK_W_INT8, C, R, V, X, 4>                              \
                                   : linear_rows_kernel<RK_W_INT4, C, R, V, X, 4>;
#define RK_LIN_WIDE(R, X)                                                                                      \
    if (p.nw == 8 && p.rt == R && x_op == X)                                                                   \
        fn = w_type == RK_W_INT8 ? linear_rows_kernel<RK_W_INT8, 8, R, true, X, 8>                             \
                                 : linear_rows_kernel<RK_W_INT4, 8, R, true, X, 8>;
    RK_LIN_PICK(8, 1, true, 0) RK_LIN_PICK(8, 2, true, 0) RK_LIN_PICK(8, 4, true, 0)
    RK_LIN_PICK(16, 1, true, 0) RK_LIN_PICK(16, 2, true, 0) RK_LIN_PICK(16, 4, true, 0)
    RK_LIN_PICK(8, 1, false, 0) RK_LIN_PICK(8, 2, false, 0) RK_LIN_PICK(8, 4, false, 0)
    RK_LIN_PICK(16, 1, false, 0) RK_LIN_PICK(16, 2, false, 0) RK_LIN_PICK(16, 4, false, 0)
    RK_LIN_PICK(8, 1, true, 1) RK_LIN_PICK(8, 2, true, 1) RK_LIN_PICK(8, 4, true, 1)
    RK_LIN_PICK(8, 1, true, 2) RK_LIN_PICK(8, 2, true, 2) RK_LIN_PICK(8, 4, true, 2)
    RK_LIN_WIDE(1, 0) RK_LIN_WIDE(2, 0) RK_LIN_WIDE(3, 0) RK_LIN_WIDE(4, 0)
    RK_LIN_WIDE(1, 2) RK_LIN_WIDE(2, 2) RK_LIN_WIDE(3, 2) RK_LIN_WIDE(4, 2)
#undef RK_LIN_PICK
#undef RK_LIN_WIDE
    if (!fn) return fail(RK_ERR_ARG, "rk_linear_rows: no kernel for %d columns, %d row tiles", p.cols, p.rt);
    const size_t lds = linear_xs_bytes(p.cols, p.nw);
    if (int rc = allow_dynamic_lds((const void*)fn, lds)) return rc;
    hipLaunchKernelGGL(fn, dim3((unsigned)(p.groups * p.S)), dim3(64 * p.nw), lds, static_cast<hipStream_t>(stream), a);
    return check_launch("linear_rows");
}

}  // namespace

extern "C" {

int rk_linear_rows_ex2(float* y, float* ss_out, const float* x, long long x_ld, int x_op, const float* aux,
                       long long aux_ld, const float* norm_w, float eps, int M, int N, int K, const void* w,
                       int w_type, const void* scales, const void* mins, const float* bias, const float* residual,
                       float* partials, size_t partial_bytes, uint32_t* counters, int n_counters, void* stream) {
    return linear_rows_impl(y, ss_out, x, x_ld, x_op, aux, aux_ld, norm_w, eps, M, N, K, w, w_type, scales, mins, bias,
                            residual, partials, partial_bytes, counters, n_counters, false, stream);
}

int rk_swiglu_rows(float* y, const float* x, long long x_ld, int x_op, const float* aux, long long aux_ld,
                   const float* norm_w, float eps, int M, int F, int K, const void* w, int w_type, const void* scales,
                   const void* mins, float* partials, size_t partial_bytes, uint32_t* counters, int n_counters,
                   void* stream) {
    if (x_op != RK_X_PLAIN && x_op != RK_X_RMS_NORM) return fail(RK_ERR_ARG, "rk_swiglu_rows: input transform %d", x_op);
    if (F < 0 || F > (1 << 29)) return fail(RK_ERR_ARG, "rk_swiglu_rows: F %d", F);
    if (F % 8) return fail(RK_ERR_UNSUPPORTED, "rk_swiglu_rows: F %d (a multiple of 8)", F);
    return linear_rows_impl(y, nullptr, x, x_ld, x_op, aux, aux_ld, norm_w, eps, M, 2 * F, K, w, w_type, scales, mins,
                            nullptr, nullptr, partials, partial_bytes, counters, n_counters, true, stream);
}

int rk_linear_rows_ex(float* y, const float* x, long long x_ld, int x_op, const float* aux, long long aux_ld, int M,
                      int N, int K, const void* w, int w_type, const void* scales, const void* mins,
                      const float* bias, const float* residual, float* partials, size_t partial_bytes,
                      uint32_t* counters, int n_counters, void* stream) {
    if (x_op == RK_X_RMS_NORM) return fail(RK_ERR_ARG, "rk_linear_rows_ex: input transform %d", x_op);
    return rk_linear_rows_ex2(y, nullptr, x, x_ld, x_op, aux, aux_ld, nullptr, 0.0f, M, N, K, w, w_type, scales, mins,
                              bias, residual, partials, partial_bytes, counters, n_counters, stream);
}

int rk_linear_rows(float* y, const float* x, int M, int N, int K, const void* w, int w_type, const void* scales,
                   const void* mins, const float* bias, const float* residual, float* partials,
                   size_t partial_bytes, uint32_t* counters, int n_counters, void* stream) {
    return rk_linear_rows_ex(y, x, K, RK_X_PLAIN, nullptr, 0, M, N, K, w, w_type, scales, mins, bias, residual, partials,
                             partial_bytes, counters, n_counters, stream);
}

int rk_dequant_rows(float* out, const void* w, int w_type, const void* scales, const void* mins,
                    const int32_t* rows, int row0, int n_rows, int N, int K, void* stream) {
    if (n_rows == 0) return RK_OK;
    const bool quant = w_type == RK_W_INT8 || w_type == RK_W_INT4;
    if (!out || !w || (quant && !scales) || (w_type == RK_W_INT4 && !mins))
        return fail(RK_ERR_ARG, "rk_dequant_rows: null pointer");
    if (w_type != RK_W_BF16 && w_type != RK_W_INT8 && w_type != RK_W_INT4)
        return fail(RK_ERR_UNSUPPORTED, "rk_dequant_rows: weight type %d", w_type);
    if (n_rows < 0 || N < 1 || K < kQB || K % kQB || (!rows && (row0 < 0 || row0 + n_rows > N)))
        return fail(RK_ERR_ARG, "rk_dequant_rows: rows %d + %d of %d, K %d (a multiple of %d)", row0, n_rows, N, K,
                    kQB);
    const long long n = (long long)n_rows * (K / 8);
    const dim3 grid((unsigned)ceil_div((size_t)n, 256));
    hipStream_t s = static_cast<hipStream_t>(stream);
    const uint16_t* sc = static_cast<const uint16_t*>(scales);
    const uint16_t* mn = static_cast<const uint16_t*>(mins);
    using Fn = void (*)(float*, const void*, const uint16_t*, const uint16_t*, const int32_t*, int, int, int, int);
    const Fn fn = w_type == RK_W_BF16 ? dequant_rows_kernel<RK_W_BF16>
                  : w_type == RK_W_INT8 ? dequant_rows_kernel<RK_W_INT8> : dequant_rows_kernel<RK_W_INT4>;
    hipLaunchKernelGGL(fn, grid, dim3(256), 0, s, out, w, sc, mn, rows, row0, n_rows, K, N);
    return check_launch("dequant_rows");
}

}  // extern "C"
