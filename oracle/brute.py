"""float64 brute-force definitions used to pin the fp32 oracle. TEST INFRASTRUCTURE ONLY.

Written from the definitions (absolute positions, explicit loops, numpy float64), not from the reference's vectorised
formulation, so that a slip in the restatement (a wrong mask offset, a transposed operand, a dropped decay factor)
shows up as a disagreement rather than being copied.
"""
import numpy as np


def attention(q, k, v, causal=True, window=None):
    """q [T, Hq, d], k/v [S, Hkv, d]; query i at absolute position S - T + i sees keys j with j <= pos and, with a
    window W, pos - W < j. Returns [T, Hq, d] float64."""
    q, k, v = (np.asarray(x, dtype=np.float64) for x in (q, k, v))
    T, Hq, d = q.shape
    S, Hkv, _ = k.shape
    G = Hq // Hkv
    out = np.zeros((T, Hq, d))
    for i in range(T):
        pos = S - T + i
        lo = 0
        hi = pos + 1 if causal else S
        if window is not None:
            lo = max(0, pos - window + 1)
        for h in range(Hq):
            kk, vv = k[lo:hi, h // G], v[lo:hi, h // G]
            s = kk @ q[i, h] / np.sqrt(d)
            p = np.exp(s - s.max())
            out[i, h] = (p / p.sum()) @ vv
    return out


def gather_positions(pool, table, lo, end, block_size):
    """Rows lo..end-1 of one sequence by the closed-form address map: position s lives at
    pool[table[s // bs], s % bs] (src/kernels/attention.metal:115)."""
    pool = np.asarray(pool)
    return np.stack([pool[int(table[s // block_size]), s % block_size] for s in range(lo, end)]) \
        if end > lo else pool[:0, 0]


def conv_silu(x, tail, w):
    """Depthwise causal conv: y[t, c] = sum_j w[c, j] * hist[t + j, c] over hist = [tail; x]; then y * sigmoid(y).
    Returns (out [T, C], new tail = last K-1 rows of hist)."""
    x, tail, w = (np.asarray(a, dtype=np.float64) for a in (x, tail, w))
    K = w.shape[1]
    hist = np.concatenate([tail, x], 0)
    T = x.shape[0]
    y = np.zeros_like(x)
    for t in range(T):
        for j in range(K):
            y[t] += w[:, j] * hist[t + j]
    return y / (1.0 + np.exp(-y)), hist[-(K - 1):]


def delta_rule(q, k, v, beta, g, S):
    """Gated delta rule, one token at a time in float64, written per head with explicit outer products:
    S <- e^{g} S;  S <- S + beta * k (v - S^T k)^T;  o = S^T q (after the update)."""
    q, k, v, beta, g, S = (np.array(a, dtype=np.float64) for a in (q, k, v, beta, g, S))
    T, H, dk = q.shape
    out = np.zeros((T, H, v.shape[2]))
    for t in range(T):
        for h in range(H):
            Sh = S[h] * np.exp(g[t, h])
            err = v[t, h] - Sh.T @ k[t, h]
            Sh = Sh + beta[t, h] * np.outer(k[t, h], err)
            out[t, h] = Sh.T @ q[t, h]
            S[h] = Sh
    return out, S


def deltanet_step(qkv, z, b, a, tail, S, conv_w, A_log, dt_bias, norm_w, eps, dims):
    """One decode token of a Gated DeltaNet layer for one sequence, float64: conv + SiLU, split, l2-normalise q and
    k (q also / sqrt(dk)), beta = sigmoid(b), g = -e^{A_log} softplus(a + dt_bias), delta rule, then
    rmsnorm(o) * w * silu(z) per head. qkv [1, C]; tail [K-1, C]; S [H, dk, dv]. Returns (out [1, H*dv], tail, S)."""
    H, dk, dv, key_dim = dims
    u, tail = conv_silu(qkv, tail, conv_w)
    u = u[0]
    q = u[:key_dim].reshape(H, dk)
    k = u[key_dim:2 * key_dim].reshape(H, dk)
    v = u[2 * key_dim:].reshape(H, dv)
    q = q / np.sqrt((q * q).sum(-1, keepdims=True) + 1e-6) / np.sqrt(dk)
    k = k / np.sqrt((k * k).sum(-1, keepdims=True) + 1e-6)
    b, a = np.asarray(b, np.float64).reshape(H), np.asarray(a, np.float64).reshape(H)
    beta = 1.0 / (1.0 + np.exp(-b))
    ab = a + np.asarray(dt_bias, np.float64)
    sp = np.where(ab > 20, ab, np.log1p(np.exp(np.minimum(ab, 20))))
    g = -np.exp(np.asarray(A_log, np.float64)) * sp
    o, S = delta_rule(q[None], k[None], v[None], beta[None], g[None], S)
    o = o[0]
    zz = np.asarray(z, np.float64).reshape(H, dv)
    y = o / np.sqrt((o * o).mean(-1, keepdims=True) + eps) * np.asarray(norm_w, np.float64) * (zz / (1 + np.exp(-zz)))
    return y.reshape(1, H * dv), tail, S
