"""Block-quantized weights in the reference's format (src/quant.py), for the decode-time linears.

Every BLOCK = 32 consecutive weights along a row share fp16 parameters (src/quant.py:1-10):
    INT8 (symmetric):  scale = absmax / 127, q = round(w / scale) in [-127, 127]; w ~ q * scale
    INT4 (asymmetric): min = fp16(block min), scale = (max - min) / 15, q = round((w - min) / scale) in [0, 15],
                       two per byte (element 2j in the low nibble, 2j+1 in the high); w ~ q * scale + min
Blocks never cross rows, so stacking quantized matrices row-wise (fused QKV, gate+up) is exact. Quantizing is a
one-time host step (loading a checkpoint); the matvec and dequantize run as HIP kernels (native/linear.hip).
"""
import json
from dataclasses import dataclass

import torch

BLOCK = 32
CHUNK = 1 << 24                  # weights quantized at a time (whole rows), bounding the fp32 temporaries


@dataclass
class QuantTensor:
    """src/quant.py:27-56: data int8 [N, K] or uint8 [N, K/2]; scales (and INT4 mins) fp16 [N, K/BLOCK]."""
    scheme: str                  # "int8" | "int4"
    data: torch.Tensor
    scales: torch.Tensor
    shape: tuple
    block: int = BLOCK
    mins: torch.Tensor | None = None

    def to(self, device) -> "QuantTensor":
        mins = self.mins.to(device) if self.mins is not None else None
        return QuantTensor(self.scheme, self.data.to(device), self.scales.to(device), self.shape, self.block, mins)

    @property
    def nbytes(self) -> int:
        extra = self.mins.numel() * 2 if self.mins is not None else 0
        return self.data.numel() * self.data.element_size() + self.scales.numel() * 2 + extra

    def dequantize(self, rows: torch.Tensor | None = None) -> torch.Tensor:
        """fp32 weights (optionally only the given rows), through rk_dequant_rows (a HIP kernel: the tensor must
        be on the GPU)."""
        from native import kernels
        return kernels.dequantize(self, rows)


def quantize(w: torch.Tensor, scheme: str, block: int = BLOCK) -> QuantTensor:
    """Quantize a [N, K] weight (src/quant.py:59-89), CHUNK weights (whole rows) at a time; the result is bit-identical
    to quantizing the whole matrix at once (blocks never cross rows)."""
    N, K = w.shape
    if K % block:
        raise ValueError(f"K={K} is not a multiple of the block size {block}")
    if scheme not in ("int8", "int4"):
        raise ValueError(f"unknown scheme {scheme}")
    rows = max(1, CHUNK // K)
    if N <= rows:
        return _quantize_rows(w, scheme, block)
    return concat_rows([_quantize_rows(w[r:r + rows], scheme, block) for r in range(0, N, rows)])


def _quantize_rows(w: torch.Tensor, scheme: str, block: int) -> QuantTensor:
    N, K = w.shape
    x = w.float().view(N, K // block, block)
    if scheme == "int8":
        scales16 = (x.abs().amax(-1) / 127).clamp(min=1e-12).to(torch.float16)
        q = torch.round(x / scales16.float()[..., None])                  # divided by the stored (fp16) scale
        return QuantTensor(scheme, q.clamp(-127, 127).to(torch.int8).view(N, K), scales16, (N, K), block)
    lo, hi = x.amin(-1), x.amax(-1)
    mins16 = lo.to(torch.float16)
    scales16 = ((hi - mins16.float()) / 15).clamp(min=1e-12).to(torch.float16)
    q = torch.round((x - mins16.float()[..., None]) / scales16.float()[..., None]).clamp(0, 15)
    q = q.to(torch.uint8).view(N, K)
    return QuantTensor(scheme, (q[:, 0::2] | (q[:, 1::2] << 4)).contiguous(), scales16, (N, K), block, mins16)


def select_rows(w, idx: torch.Tensor):
    """Rows idx of a plain or quantized weight (src/quant.py:131-136)."""
    if isinstance(w, QuantTensor):
        mins = w.mins[idx] if w.mins is not None else None
        return QuantTensor(w.scheme, w.data[idx], w.scales[idx], (len(idx), w.shape[1]), w.block, mins)
    return w[idx]


def concat_rows(parts: list):
    """Row-wise stack of plain tensors or of QuantTensors of one scheme (src/quant.py:139-147)."""
    if not isinstance(parts[0], QuantTensor):
        return torch.cat(parts, dim=0)
    if len({p.scheme for p in parts}) != 1:
        raise ValueError(f"cannot stack mixed quantization schemes {[p.scheme for p in parts]}")
    mins = torch.cat([p.mins for p in parts]) if parts[0].mins is not None else None
    return QuantTensor(parts[0].scheme, torch.cat([p.data for p in parts]), torch.cat([p.scales for p in parts]),
                       (sum(p.shape[0] for p in parts), parts[0].shape[1]), parts[0].block, mins)


# The fused-weight groups of the INT4 precision policy (src/quant.py:92-98): checkpoint components and the fused
# matrices they are stacked into share one group, so a stacked matrix gets a single scheme.
POLICY_GROUPS = [
    (("self_attn.q_proj.weight", "self_attn.k_proj.weight", "self_attn.v_proj.weight",
      "self_attn.qkvg.weight", "self_attn.qkv.weight"), "attn_in"),
    (("mlp.gate_proj.weight", "mlp.up_proj.weight", "mlp.gate_up.weight"), "mlp_in"),
    (("linear_attn.in_proj_qkv.weight", "linear_attn.in_proj_z.weight", "linear_attn.in_proj_b.weight",
      "linear_attn.in_proj_a.weight", "linear_attn.in_proj.weight"), "linear_in"),
]


def policy_group(name: str) -> str:
    """The policy id of a weight name (src/quant.py:101-112): the part from 'layers.' on, with a fused-group
    member's suffix replaced by its group, so checkpoint and fused names of one matrix agree."""
    i = name.find("layers.")
    base = name[i:] if i >= 0 else name
    for suffixes, group in POLICY_GROUPS:
        for suf in suffixes:
            if base.endswith(suf):
                return base[: -len(suf)] + group
    return base


def scheme_for(name, scheme: str, keep_int8: frozenset = frozenset()) -> str:
    """INT4 mode keeps the tied embedding / output head and the policy's groups at INT8 (src/quant.py:115-121)."""
    if scheme == "int4" and name is not None and (
            "embed_tokens" in name or policy_group(name) in {policy_group(k) for k in keep_int8}):
        return "int8"
    return scheme


def load_policy(path) -> frozenset:
    """The groups a configs/quant/<model>.json keeps at INT8 (src/quant.py:124-128); empty without a file."""
    if not path:
        return frozenset()
    return frozenset(policy_group(n) for n in json.load(open(path))["keep_int8"])
