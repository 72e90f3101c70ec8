"""Shared test helpers."""
import torch


def rel_err(got, want) -> float:
    """max |got - want| / max |want| (the reference's relative-error convention, tests/test_kernels.py:60, 73)."""
    got = torch.as_tensor(got).detach().double().cpu()
    want = torch.as_tensor(want).detach().double().cpu()
    return float((got - want).abs().max() / want.abs().max().clamp_min(1e-300))


class SlotState:
    """A duck-typed DeltaNet state for the oracle: S [n_linear, H, dk, dv] and conv_tail [n_linear, K-1, C]."""

    def __init__(self, S, conv_tail):
        self.S, self.conv_tail = S, conv_tail
