/* rk_probe.h — measurement probes of librk_probe.so (gfx950). No counterpart in the reference: bench.py uses them to
 * measure what the memory system gives for the two decode kernels' access patterns, with no arithmetic, so each
 * kernel's fraction of the HBM peak can be read against the ceiling of its own access pattern. Same conventions as
 * rk_path.h: device pointers, the caller's stream, RK_OK or an RK_ERR_* code; the library also exports
 * rk_abi_version and rk_last_error (declared in rk_path.h) for its own calls. */
#ifndef RK_PROBE_H
#define RK_PROBE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Reads tile_bytes (4096, 8192 or 16384) contiguous bytes at each byte offset tile_offsets[i] (16-byte aligned) of
 * both k_pool and v_pool. tiles_per_group 0: `workgroups` persistent workgroups of 8 waves, wave i taking entries
 * i, i + waves, ...; xors of the data go to sink [workgroups * 512] uint32. tiles_per_group n > 0: ceil(n_tiles / n)
 * one-shot workgroups of 8 waves over consecutive runs of n entries (sink [512], written only on an improbable
 * value). With the paged decode's tiles (16 positions x Hkv x D of one block) in table order it is that kernel's
 * K / V traffic alone. */
int rk_probe_block_stream(const void* k_pool, const void* v_pool, const long long* tile_offsets, int n_tiles,
                          int tile_bytes, int workgroups, int tiles_per_group, uint32_t* sink, void* stream);

/* For each of the B rows seq_index[b] of the DeltaNet state pool S [seqs, n_linear, H, dk, dv] fp32 and each head,
 * reads the [dk, dv] block at layer `slot`, multiplies it by `scale` and writes it back, with `split` workgroups of
 * 256 threads per head (each a contiguous 1/split of the block): the recurrent step's state traffic alone. */
int rk_probe_state_rmw(float* S, const int32_t* seq_index, int B, int n_linear, int slot, int H, int dk, int dv,
                       int split, float scale, void* stream);

#ifdef __cplusplus
}
#endif

#endif
