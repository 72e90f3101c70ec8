"""CPU restatement of the reference's block dequantization and linear (src/quant.py:45-56; the fp32 linear of the
decode backends, src/backend/metal.py:59-133 / torch_ref.py:19-23). TEST INFRASTRUCTURE ONLY."""
import torch


def dequantize(scheme: str, data: torch.Tensor, scales: torch.Tensor, mins: torch.Tensor | None, block: int = 32,
               rows: torch.Tensor | None = None) -> torch.Tensor:
    """fp32 weights: INT8 q * scale; INT4 q * scale + min (element 2j = low nibble of byte j), src/quant.py:45-56."""
    if rows is not None:
        data, scales = data[rows], scales[rows]
        mins = mins[rows] if mins is not None else None
    if scheme == "int8":
        q = data.float()
        return (q.view(*q.shape[:-1], -1, block) * scales.float()[..., None]).flatten(-2)
    lo, hi = (data & 0x0F).float(), (data >> 4).float()
    q = torch.stack([lo, hi], dim=-1).flatten(-2)
    q = q.view(*q.shape[:-1], -1, block)
    return (q * scales.float()[..., None] + mins.float()[..., None]).flatten(-2)


def linear(x: torch.Tensor, w: torch.Tensor, bias=None, residual=None) -> torch.Tensor:
    """y = x @ w.T in fp32, then + bias, then + residual (each rounded), as the backends compute it."""
    y = x.float() @ w.float().T
    if bias is not None:
        y = y + bias.float()
    return y + residual.float() if residual is not None else y
