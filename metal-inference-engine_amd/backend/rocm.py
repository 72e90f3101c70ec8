"""RocmBackend: the engine's token-mixing operations on hand-written HIP kernels for MI355X (gfx950).

The `rocm` counterpart of MetalBackend (src/backend/metal.py:28): the same method names, signatures and fp32 return
tensors as the Backend protocol (src/backend/base.py:11-67) for the decode/prefill token-mixing path. Every method
runs through librk_path.so; there is no CPU path and no second implementation to fall back to: without a ROCm GPU or
without the built library, construction raises.

Method -> kernel:
  paged_attention        rk_paged_decode   (P1; + optional fused sigmoid gate)
  attention, T == 1      rk_paged_decode on the contiguous cache viewed as one block (the reference's
                         attention_decode, src/backend/metal.py:197-210)
  attention, T > 1       rk_paged_prefill on the same one-block view, no KV write (causal, optional window); fp32
                         operands (fp32-level results) unless q, k and v are all bf16 (then bf16 operands)
  deltanet_decode[_batch] rk_deltanet_decode (P2; states of one HybridPool in one launch, a standalone state as a
                         pool of one, src/backend/metal.py:232-256)
  paged_prefill_attention rk_paged_prefill (P4; the packed prefill of full_attention, src/models/qwen3_5.py:112-120:
                         KV write-back, causal attention over prefix + new tokens, fused gate; optional window)
  gated_delta[_packed]   rk_gated_delta_chunked (P3; the chunked delta rule of the linear-attention prefill,
                         src/models/qwen3_5.py:157, for one sequence or many packed sequences per launch pair)
  causal_conv1d          rk_causal_conv1d (src/ops.py:127-139)
  rms_norm_gated         rk_rms_norm_gated (src/ops.py:120-124)
  deltanet_prefill       rk_deltanet_prefill_front + rk_gated_delta_chunked + rk_rms_norm_gated: a whole packed
                         linear-attention prefill (src/models/qwen3_5.py:144-162) in four launches
  attention_prep         rk_attn_prep: q / k RMSNorm + partial RoPE (+ the decode KV write) of a gated-attention
                         layer (src/models/qwen3_5.py:251-262, 100-110) in one launch
  linear, embedding      rk_linear_rows (bf16 / INT8 / INT4 weights, up to 32 rows), rk_dequant_rows (+ a BLAS GEMM
                         beyond 32 rows; embedding rows), src/backend/metal.py:50-133
  swiglu                 rk_swiglu_rows: the linear on the stacked [gate; up] weight with silu * up of each gate / up
                         output pair in its epilogue (one launch; beyond 32 rows the linear then rk_silu_mul)
  rms_norm_swiglu        rk_swiglu_rows with the RMSNorm applied while x is staged (the MLP of a decode step)
  silu_mul               rk_silu_mul on the two halves of a gate_up output, in place
  silu_mul_linear        rk_linear_rows_ex: SwiGLU's silu * up applied while the down projection stages its
                         activations (one launch instead of two)
  rms_norm, layer_norm   rk_rms_norm, rk_layer_norm (src/ops.py:7-24)
  rope                   rk_rope (src/ops.py:27-54)
  prepare                the reference's weight policy (src/backend/metal.py:43-48): bf16 on the device, or with a
                         scheme every 2-D weight block-quantized (the tied embedding / head and policy groups INT8)
"""
import torch

from native import kernels
from native.rocm_native import load

KV_DTYPES = kernels.KV_DTYPES


class RocmBackend:
    """Token-mixing backend on one ROCm device. Not thread-safe (one engine thread owns the device, as in the
    reference's scheduler); every launch goes on torch's current stream of that device, without host syncs."""

    def __init__(self, device: str | torch.device = "cuda", scheme: str | None = None, policy: str | None = None):
        """scheme None keeps bf16 weights; "int8" / "int4" quantizes every 2-D weight in prepare (or accepts
        QuantTensors), with the INT4 policy of src/quant.py:115-121 (policy: a configs/quant JSON of groups kept
        INT8), as MetalBackend(scheme, policy)."""
        if scheme not in (None, "int8", "int4"):
            raise ValueError(f"unknown scheme {scheme}")
        if not torch.cuda.is_available():
            raise RuntimeError("RocmBackend needs a ROCm GPU (torch.cuda.is_available() is False)")
        dev = torch.device(device)
        self.device = torch.device("cuda", dev.index if dev.index is not None else torch.cuda.current_device())
        self.lib = load()
        arch = torch.cuda.get_device_properties(self.device).gcnArchName
        if not arch.startswith("gfx950"):
            raise RuntimeError(f"librk_path.so is built for gfx950 only; device {self.device} is {arch}")
        from quant import load_policy
        self.scheme = scheme
        self.keep_int8 = load_policy(policy)
        self.weight_dtype = torch.bfloat16
        self.name = f"rocm-{scheme or 'bf16'}"
        self._seq0 = torch.zeros(1, dtype=torch.int32, device=self.device)

    # ---- weights
    def prepare(self, w, name=None):
        """One weight into its resident format (src/backend/metal.py:43-48): a QuantTensor moves to the device;
        with a scheme, a 2-D weight whose rows are whole blocks is quantized (INT8 for the tied embedding / head and
        the policy's groups in INT4 mode); anything else is bf16 on the device (src/backend/torch_ref.py:16-17)."""
        from quant import QuantTensor, quantize, scheme_for
        if isinstance(w, QuantTensor):
            return w.to(self.device)
        if self.scheme and w.ndim == 2 and w.shape[1] % 32 == 0:
            return quantize(w, scheme_for(name, self.scheme, self.keep_int8)).to(self.device)
        return w.to(device=self.device, dtype=self.weight_dtype)

    # ---- P1: decode attention
    def paged_attention(self, q, k_pool, v_pool, tables, lens, block_size, window=None, gate=None, plan=None):
        """q [B, Hq, d]; k_pool / v_pool one layer [blocks, bs, Hkv, d] (fp32 or bf16, read in place); tables
        [B, max_nb] int32; lens [B] int32 -> [B, Hq, d] fp32. gate [B, Hq * d] (optional): the sigmoid output gate of
        src/models/qwen3_5.py:271 applied in the same launch sequence. plan (optional): decode_plan of this step's
        tables and lens, shared by the step's attention layers (same bits, a shorter start per call)."""
        if k_pool.dtype != v_pool.dtype or k_pool.dtype not in KV_DTYPES:
            raise TypeError(f"paged_attention: keys and values must both be float32 or bfloat16, not "
                            f"{k_pool.dtype} / {v_pool.dtype}")
        return kernels.paged_decode(q, k_pool, v_pool, tables, lens, block_size, window, gate, plan=plan)

    def decode_plan(self, tables, lens, block_size, n_heads, n_kv_heads, head_dim, num_blocks, window=None):
        """The batch layout plan of a decode step (rk_paged_decode_plan), made once from the step's tables and lens
        and passed to every paged_attention of the step (its attention layers all decode the same batch)."""
        return kernels.decode_plan(tables, lens, block_size, n_heads, n_kv_heads, head_dim, num_blocks, window)

    def attention(self, q, k, v, causal=True, window=None):
        """Backend.attention (src/backend/base.py:32-35): q [T, Hq, d], k/v [S, Hkv, d] -> [T, Hq, d] fp32; query i
        sits at position S - T + i; with a window W it sees its last W keys (ops.attention, src/ops.py:65-104).
        T == 1 (decode on a contiguous cache) runs the paged decode kernel on the cache viewed as a single block;
        T > 1 (the per-segment prefill of src/models/qwen3_5.py:118 and src/models/cohere2.py:163) runs the prefill
        attention kernel on the same one-block view, with no KV write."""
        T, Hq, d = q.shape
        if T != 1:
            return kernels.attention(q, k, v, causal, window)
        if window is not None and window < 1:
            raise ValueError(f"window must be at least 1, not {window}")
        if window and k.shape[0] > window:
            k, v = k[-window:], v[-window:]
        if k.dtype != v.dtype or k.dtype not in KV_DTYPES:
            k, v = k.float(), v.float()
        S, Hkv, _ = k.shape
        kp = k.contiguous().view(1, S, Hkv, d)
        vp = v.contiguous().view(1, S, Hkv, d)
        tables = self._seq0.view(1, 1)
        lens = torch.full((1,), S, dtype=torch.int32, device=self.device)
        return kernels.paged_decode(q, kp, vp, tables, lens, S)

    # ---- P4: packed prefill attention
    def paged_prefill_attention(self, q, k_new, v_new, k_pool, v_pool, tables, cu_seqlens, start_pos, block_size,
                                gate=None, window=None, exact=False):
        """Packed prefill of one attention layer for S segments: writes k_new / v_new [N, Hkv, d] into the pool
        layer at positions start_pos[s] + i of segment s (rows cu_seqlens[s] .. cu_seqlens[s+1]-1, block-table row
        s of tables [S, max_nb]), then causal attention of q [N, Hq, d] over each segment's prefix and new keys
        -> [N, Hq, d] fp32, times sigmoid(gate [N, Hq*d]) when given. The reference runs this per segment as
        kv.write -> kv.read -> attention(causal) -> gate (src/models/qwen3_5.py:112-120). With a window W each query
        sees its last W positions (the sliding layers' prefill, src/models/cohere2.py:155-163), and blocks below
        every query's window are never read. The reference computes in fp32 (src/ops.py:84-87): an fp32 q or pool
        runs on fp32 operands (fp32-level results); bf16 q and pool run on bf16 operands (probabilities rounded to
        bf16) unless exact=True."""
        return kernels.paged_prefill(q, k_new, v_new, k_pool, v_pool, tables, cu_seqlens, start_pos, block_size,
                                     gate, window=window, exact=exact)

    # ---- P3: chunked gated delta rule
    def gated_delta(self, q, k, v, beta, g, S):
        """Backend.gated_delta (src/backend/base.py:47-48): q, k [T, H, dk] (q already scaled), v [T, H, dv],
        beta, g [T, H], S [H, dk, dv] -> (o [T, H, dv] fp32, new S fp32); the input state is left as it was. The
        reference runs the chunked form for T > 1 and the recurrent form for T == 1 (src/backend/torch_ref.py:52-56);
        both compute the same rule, and here both run the chunked kernel (one token is one partial chunk)."""
        S_new = S.to(torch.float32).contiguous().clone().unsqueeze(0)
        o = kernels.gated_delta_chunked(q, k, v, beta, g, S_new, [0, q.shape[0]])
        return o, S_new[0]

    def gated_delta_packed(self, q, k, v, beta, g, cu_seqlens, S, seq_index=None):
        """gated_delta for several packed sequences in one launch pair (the model's packed prefill calls it once
        per segment, src/models/qwen3_5.py:136-162): rows cu_seqlens[i] .. cu_seqlens[i+1]-1 are sequence i, whose
        state S[seq_index[i]] (or S[i]) of the fp32 [n, H, dk, dv] states is updated in place -> o [N, H, dv]."""
        return kernels.gated_delta_chunked(q, k, v, beta, g, S, cu_seqlens, seq_index)

    # ---- P2: DeltaNet decode step
    def deltanet_decode(self, qkv, z, b, a, state, slot, conv_w, A_log, dt_bias, norm_w, eps, dims):
        return self.deltanet_decode_batch(qkv, z, b, a, [state], slot, conv_w, A_log, dt_bias, norm_w, eps, dims)

    def deltanet_decode_batch(self, qkv, z, b, a, states, slot, conv_w, A_log, dt_bias, norm_w, eps, dims):
        """B sequences, one token each; row i belongs to states[i]. One launch when the states share a HybridPool
        (or for a lone standalone state); otherwise one launch per state, each a pool of one."""
        pool = getattr(states[0], "pool", None)
        if pool is not None and all(getattr(st, "pool", None) is pool for st in states):
            S, conv, seqs = pool.S, pool.conv, pool.seq_index(states)
        elif len(states) == 1:
            S, conv, seqs = states[0].S.unsqueeze(0), states[0].conv_tail.unsqueeze(0), self._seq0
        else:
            return torch.cat([self.deltanet_decode_batch(qkv[i:i + 1], z[i:i + 1], b[i:i + 1], a[i:i + 1], [st], slot,
                                                         conv_w, A_log, dt_bias, norm_w, eps, dims)
                              for i, st in enumerate(states)])
        return kernels.deltanet_decode(qkv, z, b, a, conv, S, seqs, slot, conv_w, A_log, dt_bias, norm_w, eps, dims)

    # ---- DeltaNet prefill companions
    def causal_conv1d(self, x, tail, w):
        """Backend.causal_conv1d (src/backend/base.py:44-45): x [T, C], tail [K-1, C], w [C, K] -> (silu(conv)
        [T, C] fp32, new tail [K-1, C] fp32): ops.causal_conv1d (src/ops.py:127-139) on x widened to fp32, as
        TorchBackend.causal_conv1d does (src/backend/torch_ref.py:49-50)."""
        return kernels.causal_conv1d(x, tail, w)

    def rms_norm_gated(self, x, z, w, eps):
        """Backend.rms_norm_gated (src/backend/base.py:50-51): x, z [rows, dv] -> fp32 [rows, dv],
        ops.rms_norm_gated (src/ops.py:120-124)."""
        return kernels.rms_norm_gated(x, z, w, eps)

    def deltanet_prefill(self, qkv, z, b, a, states, slot, cu_seqlens, conv_w, A_log, dt_bias, norm_w, eps, dims):
        """Packed prefill of one linear-attention layer, every segment at once (the per-segment loop of
        src/models/qwen3_5.py:144-162): conv + split + l2norm + beta / g (one fused launch, conv tails handed over
        in the state), the chunked delta rule (P3) and the gated RMSNorm -> [N, H * dv] fp32.
        qkv [N, C], z [N, H * dv], b, a [N, H] may be column slices of the fused in_proj output (strided rows).
        Rows cu_seqlens[i] .. cu_seqlens[i+1]-1 belong to states[i] (HybridStates of one HybridPool, or a single
        standalone state), whose slot `slot` is updated; states None: zero initial states, nothing stored (the
        reference's `state is None` branch)."""
        H, dk, dv, _ = dims
        cu = [int(x) for x in cu_seqlens]
        n = len(cu) - 1
        N = qkv.shape[0]
        if states is None:
            conv = seqs = None
            S = torch.zeros(n, H, dk, dv, dtype=torch.float32, device=self.device)
        else:
            if len(states) != n:
                raise ValueError(f"deltanet_prefill: {n} segments but {len(states)} states")
            pool = getattr(states[0], "pool", None)
            if pool is not None and all(getattr(st, "pool", None) is pool for st in states):
                conv, S, seqs = pool.conv[:, slot], pool.S[:, slot], pool.seq_index(states)
            elif n == 1:
                conv, S, seqs = states[0].conv_tail[slot].unsqueeze(0), states[0].S[slot].unsqueeze(0), self._seq0
            else:
                return torch.cat([self.deltanet_prefill(qkv[lo:hi], z[lo:hi], b[lo:hi], a[lo:hi], [st], slot,
                                                        [0, hi - lo], conv_w, A_log, dt_bias, norm_w, eps, dims)
                                  for st, lo, hi in zip(states, cu, cu[1:])])
        q, k, v, beta, g = kernels.deltanet_prefill_front(qkv, b, a, conv, seqs, conv_w, A_log, dt_bias, cu, dims)
        o = kernels.gated_delta_chunked(q, k, v, beta, g, S, cu, seqs)
        return kernels.rms_norm_gated(o.view(N * H, dv), z, norm_w, eps).view(N, H * dv)

    # ---- decode-time linears
    def linear(self, x, w, b=None, residual=None):
        """Backend.linear (src/backend/base.py:19-21) on a bf16 weight or a block-quantized QuantTensor
        (src/backend/metal.py:59-133): up to 32 rows through rk_linear_rows (16 per launch), beyond that an fp32
        GEMM on row chunks of the weight dequantized by rk_dequant_rows -> [M, N] fp32."""
        return kernels.linear(x, w, b, residual)

    def embedding(self, table, ids):
        """Rows of a bf16 or quantized embedding table as fp32 (src/backend/metal.py:50-53)."""
        from quant import QuantTensor
        if isinstance(table, QuantTensor) or table.dtype == torch.bfloat16:
            return kernels.dequantize(table, rows=ids.to(self.device))
        return table[ids.to(table.device)].float()

    def swiglu(self, x, w_gate_up):
        """silu(x @ gate.T) * (x @ up.T) for w_gate_up = [gate; up] stacked [2F, K] (src/backend/base.py:40-41): up
        to 32 rows one rk_swiglu_rows launch per 16 (the linear over the stacked weight with silu * up of each gate /
        up output pair in its epilogue, as MetalBackend.swiglu's fused matvec_swiglu_bf16, src/backend/metal.py:
        145-157); beyond, the linear then silu * up over the two column halves of its output, read in place."""
        return kernels.swiglu(x, w_gate_up)

    def rms_norm_swiglu(self, x, ss, norm_w, eps, w_gate_up):
        """swiglu(rms_norm(x, norm_w, eps), w_gate_up) in one launch from the sums of squares ss that the linear
        producing x returned (the MLP input of src/models/qwen3_5.py:166-170 follows a residual add)."""
        return kernels.rms_norm_swiglu(x, ss, norm_w, eps, w_gate_up)

    def silu_mul_linear(self, gate, up, w, b=None, residual=None):
        """linear(silu_mul(gate, up), w, b, residual): SwiGLU's down projection (src/models/qwen3_5.py:166-170)
        reading the gate / up halves of the gate_up output in place, in one launch (rk_linear_rows_ex)."""
        return kernels.silu_mul_linear(gate, up, w, b, residual)

    def linear_ss(self, x, w, b=None, residual=None):
        """linear, also returning the sums of squares of the output's 16-column tiles (or None) for the RMSNorm
        of the next layer input (rms_norm_linear): the residual-stream producers of a decode step."""
        return kernels.linear_ss(x, w, b, residual)

    def silu_mul_linear_ss(self, gate, up, w, b=None, residual=None):
        """silu_mul_linear, also returning the sums of squares of the output's 16-column tiles (or None)."""
        return kernels.silu_mul_linear_ss(gate, up, w, b, residual)

    def rms_norm_linear(self, x, ss, norm_w, eps, w, b=None, residual=None):
        """linear(rms_norm(x, norm_w, eps), w, b, residual) in one launch from the sums of squares ss that the
        linear producing x returned (src/models/qwen3_5.py: every norm of a layer input follows a residual add)."""
        return kernels.rms_norm_linear(x, ss, norm_w, eps, w, b, residual)

    def silu_mul(self, gate, up):
        """silu(gate) * up, fp32 (src/ops.py:107-110)."""
        return kernels.silu_mul(gate, up)

    # ---- row norms and rotary embedding
    def rms_norm(self, x, w, eps):
        """[..., D] -> (x / sqrt(mean(x^2) + eps)) * w, fp32 (src/ops.py:7-15)."""
        return kernels.rms_norm(x, w, eps)

    def layer_norm(self, x, w, eps):
        """LayerNorm without bias over the last dim, fp32 (src/ops.py:18-24; Cohere2)."""
        return kernels.layer_norm(x, w, eps)

    def rope(self, x, positions, theta):
        """x [T, H, d] rotated by absolute positions [T] (HF rotate_half pairs), fp32 (src/ops.py:27-54)."""
        return kernels.rope(x, positions, theta)

    # ---- gated-attention pre-processing
    def attention_prep(self, y, q_w, k_w, eps, positions, theta, rot, dims, k_pool=None, v_pool=None, slots=None):
        """The steps between a gated-attention layer's fused projection and its attention, one launch
        (src/models/qwen3_5.py:251-262 for decode, :100-110 for prefill): per-head q / k RMSNorm with the (1 + w)
        weights q_w / k_w, RoPE over the first `rot` dims at `positions` (int32 [N]), and, given one pool layer and
        int64 slots (block * block_size + offset, as write_batch addresses rows), the new K / V rows written there.
        y [N, (2 Hq + 2 Hkv) d]; dims (Hq, Hkv, d). Returns (q [N, Hq, d] fp32, gate) with a pool, else
        (q, k, v, gate); gate is the column slice of y (no copy)."""
        Hq, Hkv, d = dims
        gate = y[:, (Hq + 2 * Hkv) * d:]
        if k_pool is None:
            return (*kernels.attn_prep(y, q_w, k_w, eps, positions, theta, rot, dims), gate)
        return kernels.attn_prep(y, q_w, k_w, eps, positions, theta, rot, dims, k_pool, v_pool, slots), gate

    def sync(self) -> None:
        torch.cuda.synchronize(self.device)
