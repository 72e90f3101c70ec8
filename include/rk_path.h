/* rk_path.h — C ABI of the MI355X (gfx950) token-mixing kernels.
 *
 * Every entry point takes raw device pointers, plain integer shapes and the caller's stream (a hipStream_t passed
 * as void*; NULL means the null stream). Nothing here allocates device memory, copies a pool or synchronises:
 * outputs, workspaces and state buffers belong to the caller (PyTorch tensors in the Python host code), and every
 * launch is enqueued on the given stream. Return value: RK_OK (0) or an RK_ERR_* code, with a message available from
 * rk_last_error() (thread-local). No entry point aborts the process.
 *
 * Reference interfaces each entry point replaces are cited as path:line in MeKaustubh07/metal-inference-engine.
 */
#ifndef RK_PATH_H
#define RK_PATH_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define RK_ABI_VERSION 17

/* status codes */
#define RK_OK 0
#define RK_ERR_ARG 1         /* null pointer, bad shape or size */
#define RK_ERR_UNSUPPORTED 2 /* dtype or shape with no kernel instance */
#define RK_ERR_WORKSPACE 3   /* caller workspace smaller than the *_workspace_bytes() figure */
#define RK_ERR_HIP 4         /* HIP runtime error (launch, device query) */

/* element types of caller buffers */
#define RK_F32 0
#define RK_BF16 1

/* weight matrix types of rk_linear_rows / rk_dequant_rows (src/quant.py:1-10: blocks of 32 weights along a row share
 * fp16 parameters) */
#define RK_W_BF16 1 /* bf16 [N, K] */
#define RK_W_INT8 2 /* int8 q [N, K], fp16 scales [N, K/32]: w = q * scale */
#define RK_W_INT4 3 /* uint8 [N, K/2] (element 2j low nibble, 2j+1 high), fp16 scales and mins [N, K/32]: w = q * s + m */

/* ---- library / errors (replaces the mr_* status + error-buffer convention of src/native/metal_runtime.mm:20-43) */
const char* rk_last_error(void);
void rk_clear_error(void);
int rk_abi_version(void);
/* compute units and gcnArchName ("gfx950:...") of the current device */
int rk_device_info(int* compute_units, char* arch, int arch_len);

/* ---- P1: paged GQA decode attention (+ optional fused sigmoid output gate)
 * Replaces MetalBackend.paged_attention + paged_attention_decode<T> (src/backend/metal.py:212-223,
 * src/kernels/attention.metal:87-159); semantics of TorchBackend.paged_attention (src/backend/torch_ref.py:75-88)
 * and the gate of src/models/qwen3_5.py:271.
 *   out    [B, Hq, D] fp32              q [B, Hq, D] fp32
 *   k_pool, v_pool: one layer of the pool, [num_blocks, block_size, Hkv, D], kv_dtype RK_F32 or RK_BF16
 *   tables [B, max_nb] int32 (rows 0-padded), lens [B] int32 (positions 0..lens[i]-1 are read)
 *   window 0 = none, else each sequence reads only positions lens[i]-window .. lens[i]-1
 *   gate   NULL or B rows of Hq*D fp32, row i at gate + i * gate_ld (gate_ld >= Hq*D, a multiple of 4; the gate
 *          columns of a projection output are read in place): out *= sigmoid(gate)
 *   workspace: rk_paged_decode_workspace_bytes(...) bytes of device memory (split-K partials); no zeroing needed.
 * D in {64, 128, 256}; Hq / Hkv <= 8; B <= 1024. */
size_t rk_paged_decode_workspace_bytes(int B, int Hq, int Hkv, int D, int block_size, int max_nb);
int rk_paged_decode(float* out, const float* q, const void* k_pool, const void* v_pool, int kv_dtype,
                    const int32_t* tables, const int32_t* lens, int B, int Hq, int Hkv, int D, int block_size,
                    int max_nb, int num_blocks, int window, const float* gate, long long gate_ld, void* workspace,
                    size_t workspace_bytes, void* stream);
/* rk_paged_decode without a workspace argument and without any device allocation: the split-K partials go to a
 * fixed scratch array of rk_paged_decode_noalloc_max_bytes() (16 MiB) that the library holds on every GPU it runs on
 * until the process ends. No counterpart in the reference: for callers that cannot allocate (code under HIP graph
 * capture, serving loops that forbid hipMalloc). Shapes whose partials exceed the scratch are refused with
 * RK_ERR_WORKSPACE before any launch (batch 64 at 2 kv-heads x 256 needs 2.6 MB; the limit binds only beyond
 * several hundred sequences). All calls on one GPU share its scratch: calls that overlap on that GPU (different
 * streams, no ordering between them) race and must not be issued; stream-ordered calls are safe. */
size_t rk_paged_decode_noalloc_max_bytes(void);
int rk_paged_decode_noalloc(float* out, const float* q, const void* k_pool, const void* v_pool, int kv_dtype,
                            const int32_t* tables, const int32_t* lens, int B, int Hq, int Hkv, int D, int block_size,
                            int max_nb, int num_blocks, int window, const float* gate, long long gate_ld,
                            void* stream);
/* The batch layout plan of a decode step. Every attention layer of a step decodes the same batch: the same block
 * tables and lengths (src/state.py:119-129 builds them once per step; src/models/qwen3_5.py:263 and
 * src/models/cohere2.py:263-271 pass them to each layer). rk_paged_decode_plan turns them, once, into what the split
 * kernel otherwise derives at the start of every call: the tiles' prefix sums, each split workgroup's range and
 * each wave group's first 64 tiles with their physical blocks. rk_paged_decode_planned then issues its first K / V
 * loads after a single 16-byte load. No counterpart in the reference (its Metal kernel has no split partition).
 *   plan: device int32, rk_paged_decode_plan_ints(...) ints, 16-byte aligned, written by rk_paged_decode_plan for
 *   the same tables, lens, window and shape arguments as the decode calls that read it (a plan for other lengths
 *   gives wrong outputs, but every index it supplies is clamped into the batch, the tables and the pool). */
size_t rk_paged_decode_plan_ints(int B, int Hq, int Hkv, int D, int block_size, int max_nb);
int rk_paged_decode_plan(int32_t* plan, size_t plan_ints, const int32_t* tables, const int32_t* lens, int B, int Hq,
                         int Hkv, int D, int block_size, int max_nb, int num_blocks, int window, void* stream);
/* rk_paged_decode reading a plan of rk_paged_decode_plan instead of deriving the layout itself: the same partition,
 * the same arithmetic and order, bit-identical outputs. */
int rk_paged_decode_planned(float* out, const float* q, const void* k_pool, const void* v_pool, int kv_dtype,
                            const int32_t* tables, const int32_t* lens, int B, int Hq, int Hkv, int D, int block_size,
                            int max_nb, int num_blocks, int window, const float* gate, long long gate_ld,
                            const int32_t* plan, size_t plan_ints, void* workspace, size_t workspace_bytes,
                            void* stream);
/* The two launches of rk_paged_decode, separately (phase 0: split-K partials into the workspace; phase 1: merge,
 * gate, write out), with an optional plan (NULL: derived in the kernels). Used to time the dominant phase on its
 * own; rk_paged_decode == phase 0 then phase 1 without a plan. */
int rk_paged_decode_phase(int phase, float* out, const float* q, const void* k_pool, const void* v_pool,
                          int kv_dtype, const int32_t* tables, const int32_t* lens, int B, int Hq, int Hkv, int D,
                          int block_size, int max_nb, int num_blocks, int window, const float* gate,
                          long long gate_ld, const int32_t* plan, size_t plan_ints, void* workspace,
                          size_t workspace_bytes, void* stream);

/* ---- paged KV cache write (scatter) and read (gather)
 * rk_kv_write replaces PagedKVPool.write_batch / PagedSequence.write (src/state.py:131-134, 163-170):
 *   pool[slot[i] / block_size, slot[i] % block_size, :, :] = src[i]  for i < n, both K and V,
 *   slot = block * block_size + offset (int64), src [n, Hkv, D] in src_dtype, converted to pool_dtype
 *   (fp32 -> bf16 rounds to nearest even, as torch's .to(torch.bfloat16)).
 * rk_kv_gather replaces PagedSequence.read and the gather of TorchBackend.paged_attention
 * (src/state.py:172-180; src/backend/torch_ref.py:82-86): out[t - lo] = pool row of position t for lo <= t < end,
 * through one sequence's block table `table` (int32, entry j = physical block of logical block j). Bit-exact copy. */
int rk_kv_write(void* k_pool, void* v_pool, int pool_dtype, const int64_t* slots, const void* k_src,
                const void* v_src, int src_dtype, int n, int Hkv, int D, int block_size, int num_blocks,
                void* stream);
int rk_kv_gather(void* k_out, void* v_out, const void* k_pool, const void* v_pool, int dtype, const int32_t* table,
                 int table_len, int lo, int end, int Hkv, int D, int block_size, int num_blocks, void* stream);

/* ---- paged KV bookkeeping on the device: the block allocator and block tables (BlockAllocator, PagedSequence,
 * PagedKVPool.batch_layout, src/state.py:78-103, 119-157, 182-186) kept in device memory, so a step's layout needs no
 * host work and no host-to-device copy. tables [max_seqs, max_blocks] int32 (row = sequence slot), lens [max_seqs]
 * int32 (positions written), stack [num_blocks] int32 (free blocks), meta [2] int32: meta[0] = free blocks,
 * meta[1] = status (0 ok; 1 out of blocks; 2 a sequence would outgrow max_blocks; 3 a release would overfill the
 * stack; 4 a row outside [0, max_seqs); 5 a row named twice in one call: a double allocation or a double free,
 * which BlockAllocator.free refuses, src/state.py:94-99). A step that fails changes nothing but the status (all or nothing, as
 * PagedSequence._ensure), writes slots of -1 (skipped by rk_kv_write) and the old lengths.
 *   rk_pages_init: empty tables, stack handing out block 0 first (BlockAllocator.__init__).
 *   rk_pages_advance: batch entry b grows sequence rows[b] (distinct rows, B <= 1024) by n_new positions, taking
 *     blocks in batch order; slots [B * n_new] int64 = block * block_size + offset of each new position (the rows
 *     rk_kv_write / rk_attn_prep write; NULL to skip), out_lens [B] = lengths after the step (NULL to skip).
 *   rk_pages_release: rows[r] (distinct rows, R <= 1024) return their blocks (reverse table order, as
 *     BlockAllocator.free) and become empty.
 *   rk_pages_gather: out [B, width] int32 = the tables of rows[b], entries past the blocks held set to 0 (the
 *     0-padded tables of batch_layout, src/state.py:124-128). */
int rk_pages_init(int32_t* tables, int32_t* lens, int32_t* stack, int32_t* meta, int max_seqs, int max_blocks,
                  int num_blocks, void* stream);
int rk_pages_advance(int32_t* tables, int32_t* lens, int32_t* stack, int32_t* meta, int max_seqs, int max_blocks,
                     int num_blocks, int block_size, const int32_t* rows, int B, int n_new, int64_t* slots,
                     int32_t* out_lens, void* stream);
int rk_pages_release(int32_t* tables, int32_t* lens, int32_t* stack, int32_t* meta, int max_seqs, int max_blocks,
                     int num_blocks, int block_size, const int32_t* rows, int R, void* stream);
int rk_pages_gather(const int32_t* tables, const int32_t* lens, int max_seqs, int max_blocks, int block_size,
                    const int32_t* rows, int B, int width, int32_t* out, void* stream);

/* ---- P2: fused Gated DeltaNet decode step for B sequences (conv + SiLU, l2norm, beta/decay, delta rule, gated
 * RMSNorm). Replaces MetalBackend.deltanet_decode_batch + conv_step + gdn_decode (src/backend/metal.py:232-256;
 * src/kernels/deltanet.metal:9-92) with the semantics of TorchBackend.deltanet_decode(_batch)
 * (src/backend/torch_ref.py:61-73, 90-93).
 *   out [B, H*dv] fp32; qkv [B, C] fp32 (C = 2*H*dk + H*dv, pre-conv), z [B, H*dv], b, a [B, H], row i of each at
 *   qkv + i*qkv_ld, z + i*z_ld, b / a + i*ba_ld (the column slices of one in_proj output row, read in place)
 *   conv_state [seqs, n_linear, K-1, C] fp32 and S [seqs, n_linear, H, dk, dv] fp32, both updated in place at
 *   [seq_index[i], slot]; conv_w [C, K]; A_log, dt_bias [H]; norm_w [dv]; seq_index [B] int32.
 * dk = dv = 128, K = 4. */
int rk_deltanet_decode(float* out, const float* qkv, const float* z, const float* b, const float* a, long long qkv_ld,
                       long long z_ld, long long ba_ld, float* conv_state, float* S, const float* conv_w,
                       const float* A_log, const float* dt_bias, const float* norm_w, const int32_t* seq_index, int B,
                       int H, int dk, int dv, int conv_k, int n_linear, int slot, float eps, void* stream);

/* ---- P4: packed (varlen) prefill attention over the paged pool, with the KV write-back of the new tokens.
 * Replaces, per packed segment, the model's kv.write -> kv.read -> attention(causal) -> * sigmoid(gate) sequence
 * (src/models/qwen3_5.py:112-120; PagedSequence.write / read, src/state.py:163-180; ops.attention, src/ops.py:65-104;
 * the packing of src/models/packing.py:21-31, cu_seqlens = segment row offsets).
 *   out [N, Hq, D] fp32; q [N, Hq, D] (q_dtype); k_new, v_new [N, Hkv, D] (new_dtype): rows cu[s] .. cu[s+1]-1 are
 *   segment s, whose first new token is at absolute position start[s] of the sequence with block-table row s of
 *   tables [S, max_nb] (blocks for positions < start[s] + n[s] must be allocated).
 *   The new rows are written into k_pool / v_pool (pool_dtype; fp32 -> bf16 rounds to nearest even) before any
 *   attention reads, then query i of segment s attends causally to positions 0 .. start[s] + i.
 *   work [n_work][5] int32, in the order to schedule them (longest first balances the grid): {(segment << 16) |
 *   query block (blocks of 32 queries), first key tile, end key tile (tiles of 32 positions; the entry covers the
 *   block's keys within [first * 32, end * 32)), first partial slot or -1, (piece << 16) | pieces}. An entry with
 *   slot -1 is a whole block (every block of every segment appears once, as one whole entry or as all the pieces
 *   of one split). A block split into `pieces` entries over disjoint consecutive tile ranges uses the partial slots
 *   first .. first + pieces - 1 (unique, < n_slots): each piece writes its (o, m, l) there and the last to finish
 *   combines them in piece order, so the output does not depend on the finishing order.
 *   n_slots 0: no splits (partials, counters may be NULL); else partials of rk_paged_prefill_workspace_bytes(n_slots,
 *   Hq, D) bytes (no zeroing needed) and n_counters >= rk_paged_prefill_counters(n_slots, Hq) uint32 counters, zero
 *   before the call; every call leaves them at zero.
 *   gate NULL or [N, Hq*D] in gate_dtype (RK_F32 or RK_BF16, read as stored). Any group size Hq / Hkv, D in
 *   {64, 128, 256}, max_nb * block_size < 2^31.
 *   Operands: the reference computes in fp32 on widened inputs (src/ops.py:84-87, 91-103). exact = 0 with q and the
 *   pool both bf16 takes bf16 MFMA operands (q, K, V as stored, the probabilities rounded to bf16; fp32
 *   accumulation): bf16-level results, on 32 queries per wave at group size 4, D in {128, 256}, block_size >= 2 and
 *   max_nb * block_size^2 < 2^32 (config 5), on 16 queries per wave otherwise. exact = 1 or an fp32 q or pool takes
 *   fp32 operands (fp32 MFMA, bf16 pool rows widened exactly, fp32 probabilities): fp32-level results.
 *   window 0 or W >= 1 (causal only): query i also sees only positions above start[s] + i - W (the sliding-window
 *   prefill of src/models/cohere2.py:155-163; ops.attention's window, src/ops.py:77-81, 97-98); blocks wholly below
 *   every query's window are never read. causal 0: every query of segment s sees positions 0 .. start[s]+n[s]-1
 *   (ops.attention with causal=False). k_new = v_new = NULL: nothing is written (the keys are already in the pool);
 *   this is how Backend.attention with T > 1 (src/backend/base.py:32-35) runs on a contiguous [S, Hkv, D] cache
 *   viewed as one block of S positions, start = S - T. */
int rk_paged_prefill(float* out, const void* q, int q_dtype, const void* k_new, const void* v_new, int new_dtype,
                     void* k_pool, void* v_pool, int pool_dtype, const int32_t* tables, int max_nb,
                     const int32_t* cu_seqlens, const int32_t* start_pos, const int32_t* work, int n_work, int S,
                     int N, int Hq, int Hkv, int D, int block_size, int num_blocks, const void* gate, int gate_dtype,
                     int window, int causal, int exact, int n_slots, float* partials, size_t partial_bytes,
                     uint32_t* counters, size_t n_counters, void* stream);

/* Bytes of rk_paged_prefill's partial records, and the count of its arrival counters, for n_slots split pieces
 * (query heads Hq, head_dim D). */
size_t rk_paged_prefill_workspace_bytes(int n_slots, int Hq, int D);
size_t rk_paged_prefill_counters(int n_slots, int Hq);

/* ---- P3: chunked gated delta rule (64-token chunks, WY / UT form) for packed prefill of the linear-attention
 * layers. Replaces Backend.gated_delta with T > 1 (TorchBackend.gated_delta -> ops.gated_delta_chunked,
 * src/backend/torch_ref.py:52-56, src/ops.py:160-193; called per segment from src/models/qwen3_5.py:157), for any
 * number of packed sequences in one call.
 *   out [N, H, dv] fp32; q, k [N, H, dk], v [N, H, dv] in in_dtype (RK_F32 or RK_BF16; q already scaled);
 *   beta, g [N, H] fp32; rows cu_seqlens[i] .. cu_seqlens[i+1]-1 are sequence i (device int32 [n_seqs + 1]);
 *   cu_chunks (device int32 [n_seqs + 1]) = prefix sums of ceil(len_i / 64), total_chunks = cu_chunks[n_seqs].
 *   State of sequence i: S + idx * s_stride (elements), [H, dk, dv] fp32, read as the initial state and
 *   overwritten with the final state; idx = seq_index[i] (device int32 [n_seqs]) or i when seq_index is NULL.
 *   workspace: rk_gated_delta_workspace_bytes(total_chunks, H) bytes (per-chunk coefficients and T, and for fp32
 *   inputs P); no zeroing.
 * dk = dv = 128. fp32-level results: fp32 operands enter the bf16 MFMA as exact three-piece splits. */
size_t rk_gated_delta_workspace_bytes(int total_chunks, int H);
int rk_gated_delta_chunked(float* out, float* S, long long s_stride, const void* q, const void* k, const void* v,
                           int in_dtype, const float* beta, const float* g, const int32_t* cu_seqlens,
                           const int32_t* cu_chunks, const int32_t* seq_index, int n_seqs, int total_chunks, int H,
                           int dk, int dv, void* workspace, size_t workspace_bytes, void* stream);

/* ---- DeltaNet prefill companions: the rest of a linear-attention segment's prefill around P3
 * (src/models/qwen3_5.py:144-162). fp32 outputs; x_dtype / z_dtype RK_F32 or RK_BF16 (read as stored).
 *
 * rk_causal_conv1d replaces Backend.causal_conv1d (ops.causal_conv1d, src/ops.py:127-139) for one segment:
 *   x: row t (t < T) at x + t * x_ld, C channels; tail [K-1, C] fp32; w [C, K] fp32 (tap K-1 multiplies the
 *   current token). x is widened to fp32 first, as TorchBackend.causal_conv1d does (src/backend/torch_ref.py:49-50):
 *   hist = [tail as stored; x widened]; u [T, C] fp32 = silu(sum_j hist[t + j] * w[:, j]);
 *   new_tail [K-1, C] fp32 = the last K-1 rows of hist. 2 <= K <= 8.
 *
 * rk_deltanet_prefill_front fuses, for n_seqs packed segments (rows cu_seqlens[s] .. cu_seqlens[s+1]-1, device
 * int32 [n_seqs + 1]), the conv, the q/k/v split, l2norm (src/ops.py:115-117), q * 1/sqrt(dk), beta = sigmoid(b)
 * and g = -exp(A_log) * softplus(a + dt_bias) of src/models/qwen3_5.py:145-155, and the conv-state update of :159:
 *   qkv / b / a: row n at ptr + n * ld (x_dtype; C = 2*H*dk + H*dv, H and H channels) -- the columns of the fused
 *   in_proj output; q, k [N, H, dk], v [N, H, dv], beta, g [N, H] fp32 (the inputs of rk_gated_delta_chunked).
 *   Segment s's conv tail is [K-1, C] fp32 at conv_state + seq_index[s] * conv_stride: read as the old tail and
 *   overwritten with the new one (fp32: carried rows keep their bits, x rows widened; x widened before the conv as
 *   TorchBackend.causal_conv1d does). seq_index NULL: zero tails, conv_state untouched.
 *   Indices of non-empty segments must be distinct. dk = dv = 128, 2 <= K <= 4; qkv and conv_state 8-byte (fp32) /
 *   4-byte (bf16) aligned with even strides.
 *
 * rk_rms_norm_gated replaces Backend.rms_norm_gated (ops.rms_norm_gated, src/ops.py:120-124):
 *   out [rows, dv] fp32 = x * (1 / sqrt(mean(x^2) + eps)) * w * silu(z); x [rows, dv] fp32, w [dv] fp32; row r of
 *   z at z + (r / z_group) * z_ld + (r % z_group) * dv (contiguous: z_group 1, z_ld dv). dv in {64, 128, 256, 512};
 *   x, out, w, z and z_ld aligned to dv / 64 elements. */
int rk_causal_conv1d(float* u, float* new_tail, const void* x, int x_dtype, long long x_ld, const float* tail,
                     const float* w, int T, int C, int K, void* stream);
int rk_deltanet_prefill_front(float* q, float* k, float* v, float* beta, float* g, const void* qkv, const void* b,
                              const void* a, int x_dtype, long long ld, float* conv_state, long long conv_stride,
                              const float* conv_w, const float* A_log, const float* dt_bias,
                              const int32_t* cu_seqlens, const int32_t* seq_index, int n_seqs, int N, int H, int dk,
                              int dv, int conv_k, void* stream);
int rk_rms_norm_gated(float* out, const float* x, const void* z, int z_dtype, long long z_ld, int z_group,
                      const float* w, int rows, int dv, float eps, void* stream);

/* ---- The steps of a gated-attention layer between its projection and attention, one launch: per-head RMSNorm of
 * q and k with (1 + w) weights (ops.rms_norm, src/ops.py:7-15), RoPE over the first `rot` dims of q and k
 * (ops.rope, src/ops.py:27-54), and, for decode, the write of the new K / V rows into the paged pool
 * (PagedKVPool.write_batch, src/state.py:131-134) -- src/models/qwen3_5.py:251-262 (decode) and :100-110 (prefill).
 *   y: row n at y + n * ld (y_dtype RK_F32 / RK_BF16): [Hq*d q | Hkv*d k | Hkv*d v | ...] (the gate columns that
 *   follow are not read); q_w, k_w [d] fp32 = 1 + q_norm.weight / k_norm.weight; positions [N] int32;
 *   inv_freq [rot / 2] fp32 = ops.rope_inv_freq(theta, rot), computed on the host.
 *   q_out [N, Hq, d] fp32. k_out, v_out: NULL or [N, Hkv, d] fp32 (normed + rotated k; v as is).
 *   slots: NULL, or [N] int64 pool rows (block * block_size + offset): k and v are written into one layer's
 *   k_pool / v_pool [num_blocks, block_size, Hkv, d] (pool_dtype; fp32 -> bf16 rounds to nearest even); a slot
 *   outside the pool is skipped.
 * d in {64, 128, 256}; rot = 0 or 2 * (d / 64) * a power of 2, at most d; y 4 * (d / 64)-byte aligned (fp32). */
int rk_attn_prep(float* q_out, float* k_out, float* v_out, void* k_pool, void* v_pool, int pool_dtype,
                 const int64_t* slots, int num_blocks, int block_size, const void* y, int y_dtype, long long ld,
                 const float* q_w, const float* k_w, float eps, const int32_t* positions, const float* inv_freq,
                 int rot, int N, int Hq, int Hkv, int d, void* stream);

/* ---- Decode-time linears (the other half of a decode step): y [M, N] = x [M, K] @ W^T (+ bias) (+ residual), fp32,
 * for M <= 16 activation rows. Replaces MetalBackend.linear / _qlinear for batched decode (src/backend/metal.py:59-133;
 * matvec / qmatvec kernels) with the reference's math: W dequantized as src/quant.py:45-56 (QuantTensor.dequantize),
 * y = x @ W^T, then + bias, then + residual, each rounded.
 *   x [M, K] fp32 contiguous, 16-byte aligned; w per w_type (16-byte aligned); scales / mins fp16 [N, K/32] or NULL
 *   (bf16); bias [N] or NULL; residual [M, N] or NULL; y [M, N]. K a multiple of 32.
 *   K is cut into splits of 1024; when there is more than one, partials (rk_linear_workspace_bytes(M, N, K, w_type)
 *   bytes, no zeroing needed) receive the splits' sums and counters[ceil(N / 16)] (uint32) count the splits of each
 *   row group as they finish: counters must be zero before the first call, and every call leaves them zero. Calls
 *   that share them must be stream-ordered. Results depend on neither timing nor M nor N (every output's terms are
 *   added in an order fixed by K).
 * rk_dequant_rows: rows of W as fp32 (the reference's dequantize; bit-exact: q * scale then + min, each rounded):
 *   out [n_rows, K], source row rows[i] (int32, clamped into [0, N)) or row0 + i when rows is NULL. */
size_t rk_linear_workspace_bytes(int M, int N, int K, int w_type);
int rk_linear_rows(float* y, const float* x, int M, int N, int K, const void* w, int w_type, const void* scales,
                   const void* mins, const float* bias, const float* residual, float* partials,
                   size_t partial_bytes, uint32_t* counters, int n_counters, void* stream);
int rk_dequant_rows(float* out, const void* w, int w_type, const void* scales, const void* mins,
                    const int32_t* rows, int row0, int n_rows, int N, int K, void* stream);

/* rk_linear_rows_ex: rk_linear_rows with the row stride x_ld of x and an optional input transform applied while x
 * is staged. RK_X_SILU_MUL: x -> (x / (1 + exp(-x))) * up, up rows at aux + m * aux_ld (ops.silu_mul,
 * src/ops.py:107-110, with the hardware exp2 and reciprocal): SwiGLU's down projection reading the gate / up halves
 * of the gate_up output in place, one launch instead of silu_mul then linear (src/models/qwen3_5.py:166-170;
 * MetalBackend.swiglu / silu_mul / linear, src/backend/metal.py:55-157, 225-230); results equal that composition
 * within 1e-5. The transform needs M <= 8 and K % 256 == 0 (else RK_ERR_UNSUPPORTED: apply it first).
 * rk_linear_rows(...) == rk_linear_rows_ex(y, x, K, RK_X_PLAIN, NULL, 0, ...). */
#define RK_X_PLAIN 0
#define RK_X_SILU_MUL 1
int rk_linear_rows_ex(float* y, const float* x, long long x_ld, int x_op, const float* aux, long long aux_ld, int M,
                      int N, int K, const void* w, int w_type, const void* scales, const void* mins,
                      const float* bias, const float* residual, float* partials, size_t partial_bytes,
                      uint32_t* counters, int n_counters, void* stream);

/* rk_linear_rows_ex2: rk_linear_rows_ex with two more options, so that a decode layer's RMSNorm needs no launch of
 * its own (src/models/qwen3_5.py:228-290: every input_layernorm / post_attention_layernorm / final norm reads the
 * residual stream that the linear before it wrote).
 *   ss_out (or NULL): also writes, for each output row m and 16-column tile t, the sum of squares of y[m, 16t ..
 *     16t+15] at ss_out[m * ceil(N / 16) + t] (the tile's 16 squares added as a tree).
 *   RK_X_RMS_NORM: x -> (x * (1 / sqrt(sum / K + eps))) * norm_w, each step rounded (ops.rms_norm,
 *     src/ops.py:7-15, with the division by the rms as a product with its reciprocal; Backend.rms_norm,
 *     src/backend/base.py:26-27), where sum adds row m's K / 16 tile sums of squares at aux + m * aux_ld
 *     (written by the linear that produced x, with ss_out) in a fixed order; norm_w fp32 [K], 16-byte aligned;
 *     K <= 2048. Needs M <= 8 and K % 256 == 0 like RK_X_SILU_MUL (else
 *     RK_ERR_UNSUPPORTED: run rk_rms_norm first). Results equal rk_rms_norm then rk_linear_rows within 1e-5.
 * No counterpart in the reference as one call: it replaces the pair Backend.rms_norm + Backend.linear. */
#define RK_X_RMS_NORM 2
int rk_linear_rows_ex2(float* y, float* ss_out, const float* x, long long x_ld, int x_op, const float* aux,
                       long long aux_ld, const float* norm_w, float eps, int M, int N, int K, const void* w,
                       int w_type, const void* scales, const void* mins, const float* bias, const float* residual,
                       float* partials, size_t partial_bytes, uint32_t* counters, int n_counters, void* stream);

/* rk_swiglu_rows: y [M, F] = silu(x @ gate^T) * (x @ up^T) for w = [gate; up] stacked [2F, K] in one launch: replaces
 * Backend.swiglu (src/backend/base.py:40-41; MetalBackend.swiglu, src/backend/metal.py:145-157, whose fused
 * matvec_swiglu_bf16 kernel, src/kernels/matvec.metal:80, covers one bf16 row; TorchBackend.swiglu,
 * src/backend/torch_ref.py:43-46). The linear is rk_linear_rows_ex2's over the 2F rows (the same sums, bit for
 * bit, with x_op RK_X_PLAIN or RK_X_RMS_NORM and its aux / aux_ld / norm_w / eps); each gate output g and its up
 * output u then give (g / (1 + exp(-g))) * u with the hardware exp2 and reciprocal, the form of RK_X_SILU_MUL, so
 * rk_swiglu_rows then rk_linear_rows equals rk_linear_rows_ex2 then rk_linear_rows_ex(RK_X_SILU_MUL) bit for bit.
 * F % 8 == 0 (else RK_ERR_UNSUPPORTED); workspace rk_linear_workspace_bytes(M, 2F, K, w_type) and ceil(2F / 16)
 * counters as rk_linear_rows. No bias, residual or sums of squares (SwiGLU has none). */
int rk_swiglu_rows(float* y, const float* x, long long x_ld, int x_op, const float* aux, long long aux_ld,
                   const float* norm_w, float eps, int M, int F, int K, const void* w, int w_type, const void* scales,
                   const void* mins, float* partials, size_t partial_bytes, uint32_t* counters, int n_counters,
                   void* stream);

/* ---- the rest of a decode step (native/decode_ops.hip): the row norms, RoPE and SwiGLU's silu * up
 * Replace Backend.rms_norm / layer_norm / rope / silu_mul (src/backend/base.py:26-40, the protocol's v1 and v3
 * methods; MetalBackend.rms_norm / layer_norm / rope / silu_mul, src/backend/metal.py:159-187, 225-230; semantics
 * ops.rms_norm, ops.layer_norm, ops.rope, ops.silu_mul, src/ops.py:7-54, 107-110). fp32 outputs, contiguous.
 *
 * rk_rms_norm: out [rows, D] = (x / sqrt(mean(x^2) + eps)) * w; x rows at x + r * x_ld (RK_F32 / RK_BF16),
 *   w [D] (RK_F32 / RK_BF16); any D >= 1 and x_ld >= D (rows of up to 4096 values, a multiple of 4, with x, w,
 *   out aligned to 4 elements stay in registers, one wave per row; other rows take a workgroup each).
 * rk_layer_norm: out = w * ((x - mean) * (1 / sqrt(var + eps))), no bias; arguments as rk_rms_norm.
 * rk_rope: out [T, H, d] = x rotated by positions[t] * inv_freq[i] over the pairs (i, i + d/2) (HF rotate_half);
 *   inv_freq [d/2] fp32 as the reference computes it on the host (ops.rope_inv_freq).
 * rk_silu_mul: out [rows, F] = (g / (1 + exp(-g))) * u, g rows at gate + r * gate_ld, u at up + r * up_ld (fp32:
 *   SwiGLU reads the two halves of one [rows, 2F] projection in place). */
int rk_rms_norm(float* out, const void* x, int x_dtype, long long x_ld, const void* w, int w_dtype, int rows, int D,
                float eps, void* stream);
int rk_layer_norm(float* out, const void* x, int x_dtype, long long x_ld, const void* w, int w_dtype, int rows, int D,
                  float eps, void* stream);
int rk_rope(float* out, const float* x, const int32_t* positions, const float* inv_freq, int T, int H, int d,
            void* stream);
int rk_silu_mul(float* out, const float* gate, long long gate_ld, const float* up, long long up_ld, int rows, int F,
                void* stream);

#ifdef __cplusplus
}
#endif

#endif /* RK_PATH_H */
