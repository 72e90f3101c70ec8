"""fp32 CPU restatement of one hybrid decode step, the sequence of backend calls of Qwen3_5Model.decode_batch
(src/models/qwen3_5.py:228-290), on the oracle's functions. TEST INFRASTRUCTURE ONLY.

Each backend call is replaced by its oracle counterpart: embedding rows, rms_norm (ops.rms_norm), the projections
(x @ w.T (+ residual) in fp32 on the dequantized weights), the attention layer's q / k norms + partial RoPE
(backend_ref.attention_prep), its KV write (write_batch: rows rounded to the pool dtype) and paged attention with the
sigmoid gate, the DeltaNet step per sequence (backend_ref.deltanet_decode_batch), and the SwiGLU MLP (silu_mul of the
stacked projection's halves)."""
import torch

from oracle import backend_ref, ops_ref, quant_ref


class _Slot:
    """A sequence's DeltaNet state as the oracle's deltanet_decode takes it: S [n_linear, H, dk, dv] and
    conv_tail [n_linear, K-1, C], views of the pool rows (updated in place)."""

    def __init__(self, S, conv_tail):
        self.S, self.conv_tail = S, conv_tail


def hybrid_decode_step(cfg, w: dict, k_pool, v_pool, S, conv, seq_index, slot, slots, tables, lens, positions,
                       tokens) -> torch.Tensor:
    """w: fp32 weights by name (2-D ones dequantized as the backend holds them); k_pool / v_pool [n_full, NB, bs,
    Hkv, d] and S [seqs, n_linear, ...] / conv [seqs, n_linear, K-1, C] are updated in place as the step writes them.
    slot[i]: layer i's index into the KV pool (attention) or the state pool (DeltaNet). -> logits [B, vocab]."""
    B = tokens.shape[0]
    h = w["embed_tokens.weight"][tokens.long()]                                  # embedding rows (fp32)
    states = [_Slot(S[s], conv[s]) for s in seq_index.tolist()]
    for i in range(cfg.layers):
        p = f"layers.{i}."
        x = ops_ref.rms_norm(h, w[p + "input_layernorm.weight"], cfg.eps)
        L = slot[i]
        if cfg.is_full(i):
            a = p + "self_attn."
            y = quant_ref.linear(x, w[a + "qkvg.weight"])
            q, k, v, gate = backend_ref.attention_prep(y, w[a + "q_norm.weight"], w[a + "k_norm.weight"], cfg.eps,
                                                       positions, cfg.theta, cfg.rot, (cfg.Hq, cfg.Hkv, cfg.d))
            kl = k_pool[L].view(-1, cfg.Hkv, cfg.d)                              # write_batch (state.py:131-134)
            vl = v_pool[L].view(-1, cfg.Hkv, cfg.d)
            kl[slots.long()] = k.to(kl.dtype)
            vl[slots.long()] = v.to(vl.dtype)
            o = backend_ref.paged_attention(q, k_pool[L], v_pool[L], tables, lens, cfg.block_size)
            o = backend_ref.gate(o.reshape(B, cfg.Hq * cfg.d), gate)            # o * sigmoid(gate) (:271)
            h = quant_ref.linear(o, w[a + "o_proj.weight"], None, h)
        else:
            a = p + "linear_attn."
            y = quant_ref.linear(x, w[a + "in_proj.weight"])
            C, Z, H = cfg.conv_dim, cfg.H * cfg.dv, cfg.H
            o = backend_ref.deltanet_decode_batch(y[:, :C], y[:, C:C + Z], y[:, C + Z:C + Z + H], y[:, C + Z + H:],
                                                  states, L, w[a + "conv1d.weight"], w[a + "A_log"],
                                                  w[a + "dt_bias"], w[a + "norm.weight"], cfg.eps,
                                                  (H, cfg.dk, cfg.dv, H * cfg.dk))
            h = quant_ref.linear(o, w[a + "out_proj.weight"], None, h)
        x = ops_ref.rms_norm(h, w[p + "post_attention_layernorm.weight"], cfg.eps)
        gu = quant_ref.linear(x, w[p + "mlp.gate_up.weight"])
        F = gu.shape[1] // 2
        h = quant_ref.linear(ops_ref.silu_mul(gu[:, :F], gu[:, F:]), w[p + "mlp.down_proj.weight"], None, h)
    h = ops_ref.rms_norm(h, w["norm.weight"], cfg.eps)
    return quant_ref.linear(h, w["embed_tokens.weight"])
