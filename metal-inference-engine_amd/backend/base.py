"""The token-mixing slice of the engine's Backend protocol (src/backend/base.py:11-67).

The model calls only these methods for attention and DeltaNet mixing; a backend that implements them with the same
signatures and fp32 return tensors drops in without a change to model code (callers: src/models/qwen3_5.py:118, 157,
263, 281-283). The weight-side methods of the full protocol (prepare, linear, embedding, rms_norm, rope, silu_mul,
swiglu, layer_norm) are outside this path and are not restated here.
"""
from typing import Protocol

import torch


class TokenMixingBackend(Protocol):
    name: str
    device: torch.device

    def attention(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, causal: bool = True,
                  window: int | None = None) -> torch.Tensor:
        """q [T, Hq, d], k/v [S, Hkv, d] -> [T, Hq, d]; query i sits at position S - T + i (base.py:32-35)."""

    def causal_conv1d(self, x: torch.Tensor, tail: torch.Tensor, w: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        """Depthwise causal conv + SiLU: x [T, C], tail [K-1, C], w [C, K] -> (out [T, C], new tail) (base.py:44-45)."""

    def gated_delta(self, q, k, v, beta, g, S) -> tuple[torch.Tensor, torch.Tensor]:
        """q, k [T, H, dk], v [T, H, dv], beta, g [T, H], S [H, dk, dv] -> (o [T, H, dv], S) (base.py:47-48)."""

    def rms_norm_gated(self, x, z, w, eps) -> torch.Tensor:
        """RMSNorm(x) * w * silu(z) over the last dim (base.py:50-51)."""

    def deltanet_decode(self, qkv, z, b, a, state, slot, conv_w, A_log, dt_bias, norm_w, eps, dims) -> torch.Tensor:
        """One token of one Gated DeltaNet layer; updates the state's slot in place -> [1, H * dv] (base.py:53-54)."""

    def deltanet_decode_batch(self, qkv, z, b, a, states, slot, conv_w, A_log, dt_bias, norm_w, eps,
                              dims) -> torch.Tensor:
        """The same for B sequences (row i belongs to states[i]) -> [B, H * dv] (base.py:56-58)."""

    def paged_attention(self, q, k_pool, v_pool, tables, lens, block_size, window=None) -> torch.Tensor:
        """Batched decode attention over a paged pool read in place: q [B, Hq, d] -> [B, Hq, d] (base.py:60-63)."""
