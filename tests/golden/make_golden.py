"""Write the small golden fixtures under tests/golden/ (run from the repo root: python tests/golden/make_golden.py).

Expected values come from sources independent of the fp32 oracle:
  * oracle/brute.py — float64 definitions written from absolute positions and explicit per-head loops;
  * transformers 5.15's Qwen3.5 library routines (modeling_qwen3_5.torch_recurrent_gated_delta_rule,
    torch_chunk_gated_delta_rule) — a separate implementation of the same gated delta rule, given float64 inputs
    (the routines compute in float32 internally; HF_HUB_OFFLINE=1: no hub kernels are fetched).
Inputs are seeded; every file holds its inputs and expected outputs as float64 / int arrays (np.savez, no pickles).
"""
import os
import sys
from pathlib import Path

os.environ.setdefault("HF_HUB_OFFLINE", "1")
import numpy as np
import torch

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))
from oracle import brute  # noqa: E402

OUT = Path(__file__).resolve().parent


def paged_decode():
    """B = 3 sequences (lengths 1, 17, 40), block size 8, scrambled tables over a 12-block fp32 pool, 8/2 heads x 32,
    window None and 12."""
    rng = np.random.default_rng(101)
    lens = [1, 17, 40]
    bs, nb_pool, Hq, Hkv, d = 8, 12, 8, 2, 32
    perm = rng.permutation(nb_pool)
    nbs = [-(-n // bs) for n in lens]
    tables = np.zeros((3, max(nbs)), np.int32)
    at = 0
    for i, n in enumerate(nbs):
        tables[i, :n] = perm[at:at + n]
        at += n
    q = rng.standard_normal((3, Hq, d)).astype(np.float32)
    kp = rng.standard_normal((nb_pool, bs, Hkv, d)).astype(np.float32)
    vp = rng.standard_normal((nb_pool, bs, Hkv, d)).astype(np.float32)
    gate = rng.standard_normal((3, Hq * d)).astype(np.float32)
    out = {}
    for name, W in (("full", None), ("w12", 12)):
        rows = []
        for i, n in enumerate(lens):
            K = brute.gather_positions(kp, tables[i], 0, n, bs)
            V = brute.gather_positions(vp, tables[i], 0, n, bs)
            rows.append(brute.attention(q[i:i + 1], K, V, causal=True, window=W)[0])
        out[f"out_{name}"] = np.stack(rows)
    gated = out["out_full"].reshape(3, -1) / (1 + np.exp(-gate.astype(np.float64)))
    np.savez(OUT / "paged_decode.npz", q=q, k_pool=kp, v_pool=vp, tables=tables, lens=np.array(lens, np.int32),
             block_size=bs, gate=gate, out_gated=gated.reshape(3, Hq, d), **out)


def prefill_attention():
    """T = 6 new queries over S = 15 keys (a 9-position prefix), 4/2 heads x 16, causal, window None and 4."""
    rng = np.random.default_rng(102)
    q = rng.standard_normal((6, 4, 16)).astype(np.float32)
    k = rng.standard_normal((15, 2, 16)).astype(np.float32)
    v = rng.standard_normal((15, 2, 16)).astype(np.float32)
    np.savez(OUT / "prefill_attention.npz", q=q, k=k, v=v, out_full=brute.attention(q, k, v, True),
             out_w4=brute.attention(q, k, v, True, window=4))


def delta_rule():
    """Gated delta rule, T = 70 (crosses the 64-token chunk boundary), 2 heads x (dk 16, dv 8), nonzero S0: the
    float64 brute force, transformers' recurrent routine and its chunked routine (fp32 inside). transformers scales
    q by 1/sqrt(dk) itself, so it gets the unscaled q."""
    from transformers.models.qwen3_5 import modeling_qwen3_5 as hf
    rng = np.random.default_rng(103)
    T, H, dk, dv = 70, 2, 16, 8
    q_raw = rng.standard_normal((T, H, dk))
    k_raw = rng.standard_normal((T, H, dk))
    q_raw /= np.sqrt((q_raw ** 2).sum(-1, keepdims=True) + 1e-6)
    k = k_raw / np.sqrt((k_raw ** 2).sum(-1, keepdims=True) + 1e-6)
    v = rng.standard_normal((T, H, dv))
    beta = 1 / (1 + np.exp(-rng.standard_normal((T, H))))
    g = -np.log1p(np.exp(rng.standard_normal((T, H))))
    S0 = rng.standard_normal((H, dk, dv)) * 0.1
    q = q_raw / np.sqrt(dk)
    o_b, S_b = brute.delta_rule(q, k, v, beta, g, S0)
    t = lambda a: torch.tensor(a, dtype=torch.float64)[None]
    o_r, S_r = hf.torch_recurrent_gated_delta_rule(t(q_raw), t(k), t(v), t(g), t(beta), initial_state=t(S0),
                                                   output_final_state=True)
    o_c, S_c = hf.torch_chunk_gated_delta_rule(t(q_raw), t(k), t(v), t(g), t(beta), chunk_size=64,
                                               initial_state=t(S0), output_final_state=True)
    np.savez(OUT / "delta_rule.npz", q=q, k=k, v=v, beta=beta, g=g, S0=S0, out_brute=o_b, S_brute=S_b,
             out_hf_recurrent=o_r[0].numpy(), S_hf_recurrent=S_r[0].numpy(), out_hf_chunked=o_c[0].numpy(),
             S_hf_chunked=S_c[0].numpy())


def delta_rule_128():
    """The kernel's shape: T = 70 (one full chunk + 6 tokens), 1 head, dk = dv = 128, nonzero S0. Inputs are
    bf16-representable (stored as bf16 bit patterns, uint16), so the same values feed the bf16 and fp32 kernel paths;
    expected values from the float64 brute force, rounded to fp32."""
    rng = np.random.default_rng(106)
    T, H, dk, dv = 70, 1, 128, 128
    to_bf16 = lambda a: (torch.tensor(a, dtype=torch.float32).to(torch.bfloat16).view(torch.int16).numpy()
                         .view(np.uint16))
    from_bf16 = lambda b: (b.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    l2 = lambda x: x / np.sqrt((x ** 2).sum(-1, keepdims=True) + 1e-6)
    q = to_bf16(l2(rng.standard_normal((T, H, dk))) / np.sqrt(dk))
    k = to_bf16(l2(rng.standard_normal((T, H, dk))))
    v = to_bf16(rng.standard_normal((T, H, dv)))
    S0 = to_bf16(rng.standard_normal((H, dk, dv)) * 0.1)
    beta = (1 / (1 + np.exp(-rng.standard_normal((T, H))))).astype(np.float32)
    g = (-np.log1p(np.exp(rng.standard_normal((T, H))))).astype(np.float32)
    o, S = brute.delta_rule(from_bf16(q), from_bf16(k), from_bf16(v), beta.astype(np.float64), g.astype(np.float64),
                            from_bf16(S0))
    np.savez(OUT / "delta_rule_128.npz", q_bf16=q, k_bf16=k, v_bf16=v, S0_bf16=S0, beta=beta, g=g,
             out=o.astype(np.float32), S=S.astype(np.float32))


def deltanet_step():
    """One decode step of a small DeltaNet layer (H 2, dk = dv = 8, conv 4 over 2*16 + 16 = 48 channels)."""
    rng = np.random.default_rng(104)
    H, dk, dv = 2, 8, 8
    key_dim = H * dk
    C = 2 * key_dim + H * dv
    inp = dict(qkv=rng.standard_normal((1, C)), z=rng.standard_normal((1, H * dv)), b=rng.standard_normal((1, H)),
               a=3 * rng.standard_normal((1, H)), tail=rng.standard_normal((3, C)),
               S=0.05 * rng.standard_normal((H, dk, dv)), conv_w=0.5 * rng.standard_normal((C, 4)),
               A_log=rng.standard_normal(H), dt_bias=rng.standard_normal(H),
               norm_w=1 + 0.1 * rng.standard_normal(dv))
    inp = {k: v.astype(np.float32) for k, v in inp.items()}
    out, tail, S = brute.deltanet_step(inp["qkv"], inp["z"], inp["b"], inp["a"], inp["tail"], inp["S"],
                                       inp["conv_w"], inp["A_log"], inp["dt_bias"], inp["norm_w"], 1e-6,
                                       (H, dk, dv, key_dim))
    np.savez(OUT / "deltanet_step.npz", **inp, out=out, tail_new=tail, S_new=S, dims=np.array([H, dk, dv, key_dim]))


def conv():
    """Depthwise causal conv + SiLU over T = 5 tokens, C = 6, K = 4: torch.nn.functional.conv1d on [tail; x] with
    groups = C (the formulation of transformers' causal_conv1d_update), in float64."""
    rng = np.random.default_rng(105)
    x, tail, w = rng.standard_normal((5, 6)), rng.standard_normal((3, 6)), rng.standard_normal((6, 4))
    hist = torch.tensor(np.concatenate([tail, x]).T[None])                     # [1, C, T + K - 1]
    y = torch.nn.functional.conv1d(hist, torch.tensor(w)[:, None, :], groups=6)[0].T.numpy()
    np.savez(OUT / "conv.npz", x=x.astype(np.float32), tail=tail.astype(np.float32), w=w.astype(np.float32),
             out=y / (1 + np.exp(-y)), tail_new=np.concatenate([tail, x])[-3:])


if __name__ == "__main__":
    for f in (paged_decode, prefill_attention, delta_rule, delta_rule_128, deltanet_step, conv):
        f()
        print("wrote", f.__name__)
