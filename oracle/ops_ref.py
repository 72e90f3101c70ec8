"""fp32 CPU restatement of the reference math for this path (src/ops.py). TEST INFRASTRUCTURE ONLY.

Each function follows the operation order of the cited reference lines, so it rounds where the reference rounds.
"""
import math

import torch


def attention(q, k, v, causal: bool = True, window: int | None = None) -> torch.Tensor:
    """GQA attention, src/ops.py:65-104. q [T, Hq, d]; k, v [S, Hkv, d]; query i sits at position S - T + i.
    window W: each query sees itself and the W - 1 keys before it. Returns [T, Hq, d] fp32."""
    T, Hq, d = q.shape
    if window is not None:
        if window < 1:
            raise ValueError(f"window must be at least 1, not {window}")
        keep = T + window - 1                                   # ops.py:80-81: drop keys no query can see
        if k.shape[0] > keep:
            k, v = k[k.shape[0] - keep:], v[v.shape[0] - keep:]
    S, Hkv, _ = k.shape
    rep = Hq // Hkv
    kh = k.float().repeat_interleave(rep, dim=1).transpose(0, 1)   # [Hq, S, d] (ops.py:84-87)
    vh = v.float().repeat_interleave(rep, dim=1).transpose(0, 1)
    qh = q.float().transpose(0, 1)
    scores = qh @ kh.transpose(1, 2)                              # ops.py:91-92
    scores.div_(math.sqrt(d))
    if causal:                                                    # ops.py:94-99
        hidden = torch.ones(T, S, dtype=torch.bool).triu(diagonal=S - T + 1)
        if window is not None:
            hidden |= torch.ones(T, S, dtype=torch.bool).tril(diagonal=S - T - window)
        scores.masked_fill_(hidden, float("-inf"))
    scores.sub_(scores.max(dim=-1, keepdim=True).values).exp_()   # ops.py:101-102
    scores.div_(scores.sum(dim=-1, keepdim=True))
    return (scores @ vh).transpose(0, 1)                          # ops.py:103-104


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """x / sqrt(mean(x^2) + eps) * weight over the last dim, src/ops.py:7-15 (weight already 1 + w for Qwen3.5)."""
    x32 = x.float()
    rms = torch.sqrt(torch.mean(x32 * x32, dim=-1, keepdim=True) + eps)
    return (x32 / rms) * weight.float()


def layer_norm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """LayerNorm without bias, src/ops.py:18-24: mean removed first, then weight * (centered * rsqrt(var + eps))."""
    x32 = x.float()
    centered = x32 - x32.mean(dim=-1, keepdim=True)
    variance = centered.pow(2).mean(dim=-1, keepdim=True)
    return weight.float() * (centered * torch.rsqrt(variance + eps))


def silu_mul(gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor:
    """silu(gate) * up with silu(g) = g / (1 + e^-g), src/ops.py:107-110."""
    g = gate.float()
    return (g / (1.0 + torch.exp(-g))) * up.float()


def rope_inv_freq(theta: float, d: int) -> torch.Tensor:
    """1 / theta^(i / (d/2)) for i < d/2, fp32 on the CPU, src/ops.py:27-33."""
    half = d // 2
    return 1.0 / (theta ** (torch.arange(0, half, dtype=torch.float32) / half))


def rope(x: torch.Tensor, positions: torch.Tensor, theta: float) -> torch.Tensor:
    """Rotary embedding with the rotate_half pairing (i, i + d/2), src/ops.py:35-54. x [T, H, d], positions [T]."""
    d = x.shape[-1]
    half = d // 2
    angles = positions.float()[:, None] * rope_inv_freq(theta, d)[None, :]
    cos, sin = torch.cos(angles)[:, None, :], torch.sin(angles)[:, None, :]
    x32 = x.float()
    a, b = x32[..., :half], x32[..., half:]
    return torch.cat((a * cos - b * sin, a * sin + b * cos), dim=-1)


def l2norm(x: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """x * rsqrt(sum(x^2) + eps) over the last dim, src/ops.py:115-117."""
    return x * torch.rsqrt((x * x).sum(-1, keepdim=True) + eps)


def rms_norm_gated(x, z, w, eps) -> torch.Tensor:
    """rmsnorm(x) * w * silu(z) with plain w, src/ops.py:120-124."""
    xf, zf = x.float(), z.float()
    y = xf * torch.rsqrt((xf * xf).mean(-1, keepdim=True) + eps)
    return y * w.float() * (zf / (1.0 + torch.exp(-zf)))


def causal_conv1d(x, tail, w) -> tuple[torch.Tensor, torch.Tensor]:
    """Depthwise causal conv + SiLU, src/ops.py:127-139. x [T, C], tail [K-1, C], w [C, K] (tap K-1 = current
    token, no flip) -> (silu(conv) [T, C], new tail = last K-1 raw inputs)."""
    K, T = w.shape[1], x.shape[0]
    hist = torch.cat([tail.to(x.dtype), x], dim=0)
    y = 0
    for j in range(K):                          # the reference's sum() starts at 0 and adds tap by tap
        y = y + hist[j:j + T] * w[:, j].float()
    return y / (1.0 + torch.exp(-y)), hist[-(K - 1):].clone()


def gated_delta_recurrent(q, k, v, beta, g, S):
    """Gated delta rule token by token, src/ops.py:142-157. q, k [T, H, dk] (q pre-scaled), v [T, H, dv],
    beta, g [T, H], S [H, dk, dv]. Per token: S = e^g S; kv = k^T S; S += k (x) beta (v - kv); o = q^T S."""
    T = q.shape[0]
    out = torch.empty(T, v.shape[1], v.shape[2], dtype=torch.float32)
    for t in range(T):
        S = S * torch.exp(g[t])[:, None, None]
        kv = (S * k[t][:, :, None]).sum(-2)
        delta = (v[t] - kv) * beta[t][:, None]
        S = S + k[t][:, :, None] * delta[:, None, :]
        out[t] = (S * q[t][:, :, None]).sum(-2)
    return out, S


def gated_delta_chunked(q, k, v, beta, g, S, chunk: int = 64):
    """The same rule 64 tokens at a time (WY / UT transform), src/ops.py:160-193."""
    T, H, dk = q.shape
    dv = v.shape[-1]
    pad = (-T) % chunk
    if pad:                                                   # zero rows leave S untouched (ops.py:167-170)
        zpad = lambda t, *tail: torch.cat([t, t.new_zeros(pad, *tail)], 0)
        q, k, v, beta, g = zpad(q, H, dk), zpad(k, H, dk), zpad(v, H, dv), zpad(beta, H), zpad(g, H)
    n = q.shape[0] // chunk
    hc = lambda t: t.transpose(0, 1).reshape(H, n, chunk, *t.shape[2:])   # [H, n, C, ...] (ops.py:173-174)
    q, k, v, beta, g = hc(q), hc(k), hc(v), hc(beta), hc(g)
    vb, kb = v * beta[..., None], k * beta[..., None]
    G = g.cumsum(-1)                                          # ops.py:176
    lower = torch.ones(chunk, chunk, dtype=torch.bool).tril()
    D = (G[..., :, None] - G[..., None, :]).masked_fill(~lower, float("-inf")).exp()      # ops.py:178
    strict = torch.ones(chunk, chunk, dtype=torch.bool).tril(-1)
    A = -((kb @ k.transpose(-1, -2)) * D).masked_fill(~strict, 0.0)                     # ops.py:179
    for i in range(1, chunk):                                 # forward substitution, row by row (ops.py:180-181)
        A[..., i, :i] = A[..., i, :i] + (A[..., i, :, None] * A[..., :, :i]).sum(-2)[..., :i]
    A = A + torch.eye(chunk)
    U = A @ vb                                                # ops.py:183-184
    W = A @ (kb * G.exp()[..., None])
    out = torch.empty(H, n, chunk, dv, dtype=torch.float32)
    for c in range(n):                                        # ops.py:186-191
        qc, kc, Gc = q[:, c], k[:, c], G[:, c]
        P = (qc @ kc.transpose(-1, -2)) * D[:, c]
        vn = U[:, c] - W[:, c] @ S
        out[:, c] = (qc * Gc.exp()[..., None]) @ S + P @ vn
        S = S * Gc[:, -1].exp()[:, None, None] + (kc * (Gc[:, -1:] - Gc).exp()[..., None]).transpose(-1, -2) @ vn
    return out.reshape(H, n * chunk, dv).transpose(0, 1)[:T], S
