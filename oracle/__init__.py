"""CPU oracle of the token-mixing path — TEST INFRASTRUCTURE ONLY.

A restatement, in torch fp32 on the CPU, of the reference engine's algorithm for this path (src/ops.py,
src/backend/torch_ref.py, src/state.py, src/models/qwen3_5.py:94-164), each function citing the file:line it follows,
plus float64 brute-force versions (brute.py) written from the definitions, used to pin the restatement.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this package, and only as the checker
or the timed CPU baseline. The product (metal-inference-engine_amd/) never imports it: the ROCm backend has no CPU
path.

Pinning status (what checks each function; see tests/test_oracle.py):
  ops_ref.attention            float64 brute force from absolute positions; reference invariants (S = 1 -> v,
                               q-scale 30 finite, window edges); committed fixtures tests/golden/paged_decode.npz,
                               prefill_attention.npz
  backend_ref.paged_attention  closed-form address map (brute gather) bit-exact; paged == contiguous exactly
  ops_ref.causal_conv1d        float64 brute force; torch.nn.functional.conv1d depthwise (transformers'
                               causal_conv1d_update formulation)
  backend_ref.causal_conv1d    float64 brute force on the widened inputs (bf16 x, fp32 tail not representable in
                               bf16); the fp32 new tail equal to the widened rows
  ops_ref.l2norm, rms_norm_gated  float64 closed forms; transformers l2norm
  ops_ref.gated_delta_recurrent  float64 brute force; transformers torch_recurrent_gated_delta_rule (fixtures)
  ops_ref.gated_delta_chunked  == recurrent (float64); transformers torch_chunk_gated_delta_rule (fixtures);
                               float64 brute force at dk = dv = 128 (tests/golden/delta_rule_128.npz);
                               special cases S0 = 0, T < 64 padding, beta = g = 0 leaves S unchanged
  backend_ref.deltanet_decode  float64 brute-force step (conv, norms, gates, delta rule, gated norm)
  prefill_ref.packed_prefill   float64 brute force per segment: closed-form writes and gather, query i at p + i, the
                               gate's closed form; n > 512 across the query chunking; the pool bit-exact after the
                               writes (tests/test_oracle_compositions.py)
  decode_ref.hybrid_decode_step  a float64 composition of the model's definitions on a 4-layer stack: logits, states,
                               conv tails and written KV rows (tests/test_oracle_compositions.py)
"""
