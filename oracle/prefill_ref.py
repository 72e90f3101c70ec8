"""fp32 CPU restatement of the packed prefill attention path. TEST INFRASTRUCTURE ONLY.

Follows Qwen35Model.full_attention (src/models/qwen3_5.py:112-120) for the attention part of each packed segment:
kv.write(slot, start, k, v) (PagedSequence.write, src/state.py:163-170) -> kv.read(slot, start + T)
(PagedSequence.read, src/state.py:172-180) -> ops.attention(q, K, V, causal=True) (src/ops.py:65-104), segments in
pack order (src/models/packing.py:21-31), then o * sigmoid(gate) over all rows (qwen3_5.py:120).
Queries are processed in chunks of at most 512 rows against the same keys (as the reference's generate.py bounds
prefill chunks): each row's softmax is independent of the others, so this only bounds the score buffer.
"""
import torch

from oracle import ops_ref


def packed_prefill(q, k_new, v_new, k_pool, v_pool, tables, cu_seqlens, starts, block_size, gate=None,
                   chunk: int = 512):
    """q [N, Hq, d]; k_new, v_new [N, Hkv, d]; k_pool / v_pool one layer [NB, bs, Hkv, d] (updated in place);
    tables [S, max_nb]; cu_seqlens S + 1 offsets; starts S positions. Returns [N, Hq, d] fp32."""
    cu = [int(x) for x in cu_seqlens]
    outs = []
    for s in range(len(cu) - 1):
        lo, hi, p = cu[s], cu[s + 1], int(starts[s])
        n = hi - lo
        table = tables[s].long()
        pos = torch.arange(p, p + n)
        k_pool[table[pos // block_size], pos % block_size] = k_new[lo:hi].to(k_pool.dtype)     # write
        v_pool[table[pos // block_size], pos % block_size] = v_new[lo:hi].to(v_pool.dtype)
        nb = -(-(p + n) // block_size)
        K = k_pool[table[:nb]].flatten(0, 1)[:p + n]                                             # read back
        V = v_pool[table[:nb]].flatten(0, 1)[:p + n]
        rows = []
        for c0 in range(0, n, chunk):
            c1 = min(n, c0 + chunk)
            # queries c0 .. c1-1 sit at positions p + c0 .. p + c1 - 1: keys up to p + c1 - 1, causal inside
            rows.append(ops_ref.attention(q[lo + c0:lo + c1], K[:p + c1], V[:p + c1], causal=True))
        outs.append(torch.cat(rows) if rows else q.new_zeros(0, q.shape[1], q.shape[2]).float())
    o = torch.cat(outs)
    if gate is not None:
        o = (o.reshape(o.shape[0], -1) * torch.sigmoid(gate.float())).reshape(o.shape)
    return o
