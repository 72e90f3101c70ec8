"""fp32 CPU restatement of TorchBackend's token-mixing methods (src/backend/torch_ref.py). TEST INFRASTRUCTURE ONLY.

States are duck-typed: anything with `S` [n_linear, H, dk, dv] and `conv_tail` [n_linear, K-1, C] tensors (a
HybridState view of a pool slot, or a plain holder), updated in place at [slot] as the reference does.
"""
import torch

from oracle import ops_ref


def gated_delta(q, k, v, beta, g, S):
    """Recurrent form for one token, chunked form otherwise (torch_ref.py:52-56)."""
    if q.shape[0] == 1:
        return ops_ref.gated_delta_recurrent(q, k, v, beta, g, S)
    return ops_ref.gated_delta_chunked(q, k, v, beta, g, S)


def causal_conv1d(x, tail, w):
    """TorchBackend.causal_conv1d (torch_ref.py:49-50): x is widened to fp32 BEFORE ops.causal_conv1d, so the old
    tail is used as stored (tail.to(x.dtype) is then a no-op on an fp32 tail) and the new tail comes back fp32."""
    return ops_ref.causal_conv1d(x.float(), tail, w)


def deltanet_decode(qkv, z, b, a, state, slot, conv_w, A_log, dt_bias, norm_w, eps, dims):
    """One token of one DeltaNet layer, torch_ref.py:61-73. Returns [1, H * dv]; updates state.conv_tail[slot] and
    state.S[slot] in place."""
    H, dk, dv, key_dim = dims
    u, state.conv_tail[slot] = causal_conv1d(qkv, state.conv_tail[slot], conv_w)   # self.causal_conv1d (:65)
    q = ops_ref.l2norm(u[:, :key_dim].reshape(1, H, dk).float()) * (1.0 / dk ** 0.5)
    k = ops_ref.l2norm(u[:, key_dim:2 * key_dim].reshape(1, H, dk).float())
    v = u[:, 2 * key_dim:].reshape(1, H, dv).float()
    beta = torch.sigmoid(b.float())
    ab = a.float() + dt_bias
    g = -torch.exp(A_log) * torch.where(ab > 20, ab, torch.log1p(torch.exp(ab)))
    o, state.S[slot] = gated_delta(q, k, v, beta, g, state.S[slot])
    return ops_ref.rms_norm_gated(o.reshape(H, dv), z.reshape(H, dv), norm_w, eps).reshape(1, H * dv)


def deltanet_decode_batch(qkv, z, b, a, states, slot, conv_w, A_log, dt_bias, norm_w, eps, dims):
    """One sequence at a time (torch_ref.py:90-93) -> [B, H * dv]."""
    return torch.cat([deltanet_decode(qkv[i:i + 1], z[i:i + 1], b[i:i + 1], a[i:i + 1], st, slot, conv_w, A_log,
                                      dt_bias, norm_w, eps, dims) for i, st in enumerate(states)])


def linear_attention_front(qkv, b, a, tail, conv_w, A_log, dt_bias, dims):
    """One prefill segment's conv, split, beta / g and l2norm, src/models/qwen3_5.py:145-155
    -> (q, k [T, H, dk], v [T, H, dv], beta, g [T, H], new conv tail [K-1, C] fp32). The conv is the backend's
    (b.causal_conv1d at :145), which widens qkv first (torch_ref.py:49-50)."""
    H, dk, dv, key_dim = dims
    T = qkv.shape[0]
    u, new_tail = causal_conv1d(qkv, tail, conv_w)                         # conv BEFORE the split (:145)
    q = u[:, :key_dim].reshape(T, H, dk)
    k = u[:, key_dim:2 * key_dim].reshape(T, H, dk)
    v = u[:, 2 * key_dim:].reshape(T, H, dv)
    beta = torch.sigmoid(b.float())
    ab = a.float() + dt_bias
    g = -torch.exp(A_log) * torch.where(ab > 20, ab, torch.log1p(torch.exp(ab)))
    q = ops_ref.l2norm(q.float()) * (1.0 / dk ** 0.5)
    k = ops_ref.l2norm(k.float())
    return q, k, v.float(), beta, g, new_tail


def linear_attention_segments(qkv, z, b, a, states, slot, cu, conv_w, A_log, dt_bias, norm_w, eps, dims):
    """The per-segment loop of src/models/qwen3_5.py:136-162 (projections excluded): rows cu[i] .. cu[i+1]-1 belong
    to states[i] (updated in place at [slot]), or to a fresh zero state when states is None (nothing stored).
    A one-token segment with a state takes the decode step (:139-143). Returns [N, H * dv]."""
    H, dk, dv, key_dim = dims
    K, C = conv_w.shape[1], conv_w.shape[0]
    outs = []
    for i, (lo, hi) in enumerate(zip(cu, cu[1:])):
        T = hi - lo
        if T == 0:
            continue
        st = states[i] if states is not None else None
        if T == 1 and st is not None:
            outs.append(deltanet_decode(qkv[lo:hi], z[lo:hi], b[lo:hi], a[lo:hi], st, slot, conv_w, A_log, dt_bias,
                                        norm_w, eps, dims))
            continue
        tail = st.conv_tail[slot] if st is not None else torch.zeros(K - 1, C)
        q, k, v, beta, g, new_tail = linear_attention_front(qkv[lo:hi], b[lo:hi], a[lo:hi], tail, conv_w, A_log,
                                                            dt_bias, dims)
        S = st.S[slot] if st is not None else torch.zeros(H, dk, dv)
        o, S = gated_delta(q, k, v, beta, g, S)
        if st is not None:
            st.S[slot] = S
            st.conv_tail[slot] = new_tail
        o = ops_ref.rms_norm_gated(o.reshape(T * H, dv), z[lo:hi].reshape(T * H, dv), norm_w, eps)
        outs.append(o.reshape(T, H * dv))
    return torch.cat(outs)


def attention_prep(y, q_w, k_w, eps, positions, theta, rot, dims):
    """The gated-attention layer's steps between its projection and attention, src/models/qwen3_5.py:251-259
    (decode; then write_batch, :262) and :100-110 (prefill): per-head RMSNorm of q and k with the (1 + w) weights, RoPE over the first `rot`
    dims of q and k together, v and the gate split off. y [N, (2 Hq + 2 Hkv) d] -> (q [N, Hq, d], k, v [N, Hkv, d],
    gate [N, Hq d]) fp32 (k and v are what write_batch then stores)."""
    Hq, Hkv, d = dims
    N = y.shape[0]
    q = ops_ref.rms_norm(y[:, :Hq * d].reshape(N, Hq, d), q_w, eps)
    k = ops_ref.rms_norm(y[:, Hq * d:(Hq + Hkv) * d].reshape(N, Hkv, d), k_w, eps)
    v = y[:, (Hq + Hkv) * d:(Hq + 2 * Hkv) * d].reshape(N, Hkv, d).float()
    gate = y[:, (Hq + 2 * Hkv) * d:]
    qk = ops_ref.rope(torch.cat([q[..., :rot], k[..., :rot]], dim=1).contiguous(), positions, theta)
    q = torch.cat([qk[:, :Hq], q[..., rot:]], dim=-1)
    k = torch.cat([qk[:, Hq:], k[..., rot:]], dim=-1)
    return q, k, v, gate


def paged_gather(k_pool, v_pool, table_row, n: int, block_size: int, window: int | None = None):
    """The positions a decode query reads, gathered through one block-table row (torch_ref.py:81-86)."""
    nb = -(-n // block_size)
    s0 = max(0, n - window) if window else 0
    b0 = s0 // block_size
    rows = slice(s0 - b0 * block_size, n - b0 * block_size)
    idx = table_row[b0:nb].long()
    return k_pool[idx].flatten(0, 1)[rows], v_pool[idx].flatten(0, 1)[rows]


def paged_attention(q, k_pool, v_pool, tables, lens, block_size, window=None):
    """Gather each sequence, then ordinary attention with its one query (torch_ref.py:75-88) -> [B, Hq, d]."""
    outs = []
    for i in range(q.shape[0]):
        K, V = paged_gather(k_pool, v_pool, tables[i], int(lens[i]), block_size, window)
        outs.append(ops_ref.attention(q[i:i + 1], K, V, causal=True, window=window))
    return torch.cat(outs)


def gate(o: torch.Tensor, gate_logits: torch.Tensor) -> torch.Tensor:
    """The attention output gate before o_proj: o.reshape(N, Hq*d) * sigmoid(gate) (src/models/qwen3_5.py:271)."""
    N = o.shape[0]
    return (o.reshape(N, -1) * torch.sigmoid(gate_logits.float())).reshape(o.shape)
