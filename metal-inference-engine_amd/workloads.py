"""Seeded synthetic inputs for the five benchmark configurations of the token-mixing path.

Every tensor is drawn on the CPU from a torch.Generator seeded per configuration, so the HIP kernels (after a copy
to the GPU) and the CPU reference see identical bits. Model shapes are Qwen3.5-0.8B/2B's: attention 8 query / 2 kv
heads x 256, DeltaNet 16 heads x 128 x 128, conv kernel 4 over 6144 channels, KV blocks of 16 positions.
"""
import math
from dataclasses import dataclass, field

import torch

HQ, HKV, HEAD_DIM, BLOCK = 8, 2, 256, 16
DN_HEADS, DN_DK, DN_DV, CONV_K = 16, 128, 128, 4
KEY_DIM = DN_HEADS * DN_DK
CONV_DIM = 2 * KEY_DIM + DN_HEADS * DN_DV


@dataclass
class PagedDecodeCase:
    """One layer of a paged pool plus a decode batch: q [B, Hq, d] fp32, gate [B, Hq*d] fp32,
    k_pool / v_pool [NB, bs, Hkv, d], tables [B, max_nb] int32 (0-padded), lens [B] int32."""
    q: torch.Tensor
    gate: torch.Tensor
    k_pool: torch.Tensor
    v_pool: torch.Tensor
    tables: torch.Tensor
    lens: torch.Tensor
    block_size: int
    window: int | None = None
    meta: dict = field(default_factory=dict)

    def to(self, device) -> "PagedDecodeCase":
        f = lambda t: t.to(device)
        return PagedDecodeCase(f(self.q), f(self.gate), f(self.k_pool), f(self.v_pool), f(self.tables),
                               f(self.lens), self.block_size, self.window, dict(self.meta))

    def kv_bytes(self) -> int:
        """Bytes of K and V one decode call must read: every visible position of every sequence, both pools."""
        Hkv, d = self.k_pool.shape[2], self.k_pool.shape[3]
        L = self.lens.long()
        if self.window:
            L = L.clamp(max=self.window)
        return int(L.sum()) * Hkv * d * self.k_pool.element_size() * 2

    def table_entries(self) -> int:
        """Block-table entries one decode call reads: the blocks holding each sequence's visible positions."""
        L = self.lens.long()
        nb = (L + self.block_size - 1) // self.block_size
        if self.window:
            nb = nb - (L - self.window).clamp(min=0) // self.block_size
        return int(nb.sum())

    def algorithmic_bytes(self) -> int:
        """KV read once + q, gate, out (fp32) + the table entries and lens actually read."""
        B, Hq, d = self.q.shape
        return self.kv_bytes() + B * Hq * d * 4 * 3 + 4 * self.table_entries() + 4 * B


def _tables_from_perm(perm: list[int], nbs: list[int]) -> torch.Tensor:
    width = max(nbs)
    rows, at = [], 0
    for n in nbs:
        rows.append(perm[at:at + n] + [0] * (width - n))
        at += n
    return torch.tensor(rows, dtype=torch.int32)


def paged_decode_case(lens: list[int], num_blocks: int, Hq: int = HQ, Hkv: int = HKV, d: int = HEAD_DIM,
                      block_size: int = BLOCK, kv_dtype=torch.float32, seed: int = 0, q_scale: float = 1.0,
                      window: int | None = None) -> PagedDecodeCase:
    """Sequences of the given lengths whose blocks are a seeded random, non-contiguous choice of the pool's."""
    gen = torch.Generator().manual_seed(seed)
    nbs = [math.ceil(n / block_size) for n in lens]
    if sum(nbs) > num_blocks:
        raise ValueError(f"{sum(nbs)} blocks needed, pool has {num_blocks}")
    perm = torch.randperm(num_blocks, generator=gen).tolist()
    tables = _tables_from_perm(perm, nbs)
    B = len(lens)
    q = torch.randn(B, Hq, d, generator=gen) * q_scale
    gate = torch.randn(B, Hq * d, generator=gen)
    k_pool = torch.randn(num_blocks, block_size, Hkv, d, generator=gen).to(kv_dtype)
    v_pool = torch.randn(num_blocks, block_size, Hkv, d, generator=gen).to(kv_dtype)
    return PagedDecodeCase(q, gate, k_pool, v_pool, tables, torch.tensor(lens, dtype=torch.int32), block_size,
                           window, {"lens": list(lens), "num_blocks": num_blocks})


def c1_paged_decode(seed: int = 1) -> PagedDecodeCase:
    """Config 1: batch 1, fp32 pool of 256 blocks, context 512 (32 blocks, a seeded permutation), gate ~ N(0,1)."""
    gen = torch.Generator().manual_seed(seed)
    table = torch.randperm(256, generator=gen)[:32].to(torch.int32).view(1, 32)
    q = torch.randn(1, HQ, HEAD_DIM, generator=gen)
    gate = torch.randn(1, HQ * HEAD_DIM, generator=gen)
    k_pool = torch.randn(256, BLOCK, HKV, HEAD_DIM, generator=gen)
    v_pool = torch.randn(256, BLOCK, HKV, HEAD_DIM, generator=gen)
    return PagedDecodeCase(q, gate, k_pool, v_pool, table, torch.tensor([512], dtype=torch.int32), BLOCK, None,
                           {"config": "c1"})


def c3_lens(seed: int = 3, batch: int = 64) -> list[int]:
    gen = torch.Generator().manual_seed(seed)
    return torch.randint(128, 8193, (batch,), generator=gen).tolist()


def c3_paged_decode(seed: int = 3, batch: int = 64) -> PagedDecodeCase:
    """Config 3: batch 64, lengths U[128, 8192], bf16 pool sized to 1.25 x total positions (in blocks), each
    sequence's blocks a slice of a seeded permutation of the pool; q, gate fp32 ~ N(0,1)."""
    lens = c3_lens(seed, batch)
    num_blocks = math.ceil(1.25 * sum(lens) / BLOCK)
    case = paged_decode_case(lens, num_blocks, kv_dtype=torch.bfloat16, seed=seed + 1000)
    case.meta["config"] = "c3"
    return case


# ---------------------------------------------------------------- layouts the kernels read
# The engine keeps its KV and recurrent state in fixed layouts (src/state.py:11-17, 106-129, 196-262, 420-460), and
# the kernels read those buffers in place. The builders below produce the same layouts directly from a list of
# lengths, for the benchmark workloads and the tests; the engine's own bookkeeping (which block a sequence gets
# next, when a slot is freed) is not part of the token-mixing path and is not restated here.

def kv_pool(shape: tuple, device="cpu", dtype=torch.float32) -> tuple[torch.Tensor, torch.Tensor]:
    """K and V pools of `shape` ([layers, blocks, block_size, Hkv, d]) as the two halves of one zero-filled
    [2, *shape] buffer, the engine's pool layout."""
    both = torch.zeros(2, *shape, device=device, dtype=dtype)
    return both[0], both[1]


def scattered_tables(lens: list[int], num_blocks: int, block_size: int, gen: torch.Generator) -> torch.Tensor:
    """Block tables [B, max_nb] int32 (0-padded) for sequences of `lens` positions whose blocks are consecutive
    slices of a seeded permutation of the pool: every sequence's blocks are scattered over the pool."""
    nbs = [math.ceil(n / block_size) for n in lens]
    if sum(nbs) > num_blocks:
        raise ValueError(f"{sum(nbs)} blocks needed, pool has {num_blocks}")
    return _tables_from_perm(torch.randperm(num_blocks, generator=gen).tolist(), nbs)


def ring_size(window: int, block_size: int, max_chunk: int) -> int:
    """Units in a sliding layer's ring: every block one forward of at most max_chunk tokens reads or writes
    (the first query's window through the last new token) fits, so logical block b can live in slot b % ring."""
    return math.ceil((window + max_chunk + block_size - 2) / block_size)


def ring_tables(lens: list[int], window: int, block_size: int, ring: int, gen: torch.Generator):
    """Decode tables of a sliding-window layer whose sequences keep their blocks in rings: sequence i owns
    min(ring, blocks) units (a seeded scattered choice), logical block b sits in ring slot b % ring, and the table
    (by absolute block, up to the block of position len - 1) names that unit for the blocks of the window
    [len - W, len) and unit 0 for every block below it, which the kernels never read; unit 0 belongs to no ring.
    -> (tables [B, width] int32, number of units, [the units of each ring])."""
    held = [min(ring, math.ceil(n / block_size)) for n in lens]
    perm = (torch.randperm(sum(held), generator=gen) + 1).tolist()
    rings, at = [], 0
    for h in held:
        rings.append(perm[at:at + h])
        at += h
    width = max(math.ceil(n / block_size) for n in lens)
    rows = []
    for n, units in zip(lens, rings):
        nb = math.ceil(n / block_size)
        first = max(0, n - window) // block_size
        rows.append([units[b % ring] if b >= first else 0 for b in range(nb)] + [0] * (width - nb))
    return torch.tensor(rows, dtype=torch.int32), sum(held) + 1, rings


WD_WINDOW, WD_HQ, WD_HKV, WD_DIM = 4096, 16, 4, 128


def wd_windowed_decode(seed: int = 7, batch: int = 64) -> PagedDecodeCase:
    """Sliding-window decode through ring tables (Tiny Aya's sliding layers: 16 query / 4 kv heads x 128, a
    4096-token window, bf16 KV): config 3's batch shape (lengths U[128, 8192]), each sequence's blocks in a ring
    of ceil((W + 512 + 14) / 16) units (so longer sequences have wrapped), the decode step's tables by absolute
    block. The pool holds the rings only (one sliding layer)."""
    lens = c3_lens(seed, batch)
    gen = torch.Generator().manual_seed(seed)
    ring = ring_size(WD_WINDOW, BLOCK, 512)
    tables, units, _ = ring_tables(lens, WD_WINDOW, BLOCK, ring, gen)
    k, v = kv_pool((units, BLOCK, WD_HKV, WD_DIM), dtype=torch.bfloat16)
    k.copy_(torch.randn(k.shape, generator=gen))
    v.copy_(torch.randn(v.shape, generator=gen))
    q = torch.randn(batch, WD_HQ, WD_DIM, generator=gen)
    gate = torch.randn(batch, WD_HQ * WD_DIM, generator=gen)
    lens_t = torch.tensor(lens, dtype=torch.int32)
    return PagedDecodeCase(q, gate, k, v, tables, lens_t, BLOCK, WD_WINDOW,
                           {"config": "wd", "lens": lens, "units": units, "ring": ring})


@dataclass
class DeltaNetStepCase:
    """Inputs of one batched DeltaNet decode step. S / conv are full pool tensors
    [max_seqs, n_linear, ...]; seq_index picks the batch's slots; slot is the layer."""
    qkv: torch.Tensor
    z: torch.Tensor
    b: torch.Tensor
    a: torch.Tensor
    conv: torch.Tensor
    S: torch.Tensor
    seq_index: torch.Tensor
    slot: int
    conv_w: torch.Tensor
    A_log: torch.Tensor
    dt_bias: torch.Tensor
    norm_w: torch.Tensor
    eps: float
    dims: tuple

    def to(self, device) -> "DeltaNetStepCase":
        f = lambda t: t.to(device)
        return DeltaNetStepCase(f(self.qkv), f(self.z), f(self.b), f(self.a), f(self.conv), f(self.S),
                                f(self.seq_index), self.slot, f(self.conv_w), f(self.A_log), f(self.dt_bias),
                                f(self.norm_w), self.eps, self.dims)

    def algorithmic_bytes(self) -> int:
        B = self.qkv.shape[0]
        H, dk, dv, _ = self.dims
        C = self.qkv.shape[1]
        K = self.conv_w.shape[1]
        state = 2 * B * H * dk * dv * 4
        tail = 2 * B * (K - 1) * C * 4
        io = B * C * 4 + self.conv_w.numel() * 4 + 2 * B * H * dv * 4
        small = (2 * B * H + 2 * H + dv + B) * 4
        return state + tail + io + small


def c2_deltanet_step(seed: int = 2, batch: int = 8, max_seqs: int | None = None, n_linear: int = 1,
                     slot: int = 0, A_log_zero: bool = True) -> DeltaNetStepCase:
    """Config 2: batch 8, 16 heads, 128 x 128 fp32 state S ~ N(0, 0.02^2), conv tail ~ N(0,1), conv_w = 0.5 N,
    z, b, a ~ N(0,1), A_log = dt_bias = 0 (so beta = sigmoid(N), log-decay = -softplus(N)), norm_w = 1 + 0.1 N,
    eps 1e-6. max_seqs > batch gives a larger pool whose slots the batch occupies at seeded positions."""
    gen = torch.Generator().manual_seed(seed)
    max_seqs = max_seqs or batch
    r = lambda *s, scale=1.0: torch.randn(*s, generator=gen) * scale
    S = r(max_seqs, n_linear, DN_HEADS, DN_DK, DN_DV, scale=0.02)
    conv = r(max_seqs, n_linear, CONV_K - 1, CONV_DIM)
    seq_index = torch.randperm(max_seqs, generator=gen)[:batch].to(torch.int32)
    qkv, z = r(batch, CONV_DIM), r(batch, DN_HEADS * DN_DV)
    b, a = r(batch, DN_HEADS), r(batch, DN_HEADS)
    conv_w = r(CONV_DIM, CONV_K, scale=0.5)
    A_log = torch.zeros(DN_HEADS) if A_log_zero else r(DN_HEADS)
    dt_bias = torch.zeros(DN_HEADS) if A_log_zero else r(DN_HEADS)
    norm_w = 1.0 + r(DN_DV, scale=0.1)
    return DeltaNetStepCase(qkv, z, b, a, conv, S, seq_index, slot, conv_w, A_log, dt_bias, norm_w, 1e-6,
                            (DN_HEADS, DN_DK, DN_DV, KEY_DIM))


@dataclass
class PrefillCase:
    """Packed prefill of one attention layer: segment s adds lengths[s] tokens after a prefix of starts[s] positions
    already in the pool. q [N, Hq, d], k_new / v_new [N, Hkv, d], gate [N, Hq*d]; pool [NB, bs, Hkv, d];
    tables [S, max_nb] int32 (each segment's blocks, non-contiguous, covering prefix + new tokens)."""
    q: torch.Tensor
    k_new: torch.Tensor
    v_new: torch.Tensor
    gate: torch.Tensor
    k_pool: torch.Tensor
    v_pool: torch.Tensor
    tables: torch.Tensor
    cu_seqlens: list
    starts: list
    block_size: int

    def to(self, device) -> "PrefillCase":
        f = lambda t: t.to(device)
        return PrefillCase(f(self.q), f(self.k_new), f(self.v_new), f(self.gate), f(self.k_pool), f(self.v_pool),
                           f(self.tables), list(self.cu_seqlens), list(self.starts), self.block_size)

    def clone(self) -> "PrefillCase":
        return PrefillCase(self.q, self.k_new, self.v_new, self.gate, self.k_pool.clone(), self.v_pool.clone(),
                           self.tables, list(self.cu_seqlens), list(self.starts), self.block_size)

    def lengths(self) -> list[int]:
        return [b - a for a, b in zip(self.cu_seqlens, self.cu_seqlens[1:])]

    def flops(self) -> int:
        """QK^T and PV over the causal key range: sum over segments of 4 Hq d (n p + n (n + 1) / 2)."""
        Hq, d = self.q.shape[1], self.q.shape[2]
        return sum(4 * Hq * d * (n * p + n * (n + 1) // 2) for n, p in zip(self.lengths(), self.starts))

    def hbm_bytes(self) -> int:
        """Each segment's prefix + new K/V read once, the new rows written once, q / gate read and out written."""
        Hkv, d = self.k_pool.shape[2], self.k_pool.shape[3]
        e = self.k_pool.element_size()
        row = 2 * Hkv * d * e
        N, Hq = self.q.shape[0], self.q.shape[1]
        return sum((n + p) * row + n * row for n, p in zip(self.lengths(), self.starts)) + \
            N * Hq * d * (self.q.element_size() + self.gate.element_size() + 4)


def prefill_case(lengths: list[int], starts: list[int], Hq: int = HQ, Hkv: int = HKV, d: int = HEAD_DIM,
                 block_size: int = BLOCK, dtype=torch.bfloat16, seed: int = 0, slack: float = 1.25) -> PrefillCase:
    gen = torch.Generator().manual_seed(seed)
    nbs = [math.ceil((n + p) / block_size) for n, p in zip(lengths, starts)]
    num_blocks = max(1, math.ceil(slack * sum(nbs)))
    perm = torch.randperm(num_blocks, generator=gen).tolist()
    tables = _tables_from_perm(perm, nbs)
    N = sum(lengths)
    r = lambda *s: torch.randn(*s, generator=gen).to(dtype)
    q, k_new, v_new, gate = r(N, Hq, d), r(N, Hkv, d), r(N, Hkv, d), r(N, Hq * d)
    k_pool, v_pool = r(num_blocks, block_size, Hkv, d), r(num_blocks, block_size, Hkv, d)
    cu = [0]
    for n in lengths:
        cu.append(cu[-1] + n)
    return PrefillCase(q, k_new, v_new, gate, k_pool, v_pool, tables, cu, list(starts), block_size)


def c5_prefill(seed: int = 5, dtype=torch.bfloat16, Hq: int = HQ, Hkv: int = HKV, d: int = HEAD_DIM) -> PrefillCase:
    """Config 5: 8 segments, new lengths U[64, 2048], prefixes U[0, 16384], bf16 everything, 8/2 heads x 256,
    block 16, sigmoid gate; the prefix K/V are the random pool contents under each segment's table. dtype fp32 gives
    the same batch in the Qwen3.5 engine's own fp32 pool and activations (src/models/qwen3_5.py:70-71); Hq / Hkv / d
    the same batch at other heads."""
    gen = torch.Generator().manual_seed(seed)
    lengths = torch.randint(64, 2049, (8,), generator=gen).tolist()
    starts = torch.randint(0, 16385, (8,), generator=gen).tolist()
    return prefill_case(lengths, starts, Hq, Hkv, d, dtype=dtype, seed=seed + 1000)


def chunk_prefill(seed: int = 6) -> PrefillCase:
    """One chunk of a chunked prefill over a long history: 512 new tokens after 32,768 cached positions, config 5's
    heads (8/2 x 256), block 16, bf16 everything, sigmoid gate. 16 query blocks x 2 KV heads: the case the split
    key ranges of the prefill work list are for."""
    return prefill_case([512], [32768], seed=seed)


@dataclass
class ChunkedDeltaCase:
    """Packed prefill of one linear-attention layer's delta rule: sequence i is rows cu_seqlens[i] ..
    cu_seqlens[i+1]-1 of q, k [N, H, dk] (l2-normalised, q also * 1/sqrt(dk)), v [N, H, dv], beta, g [N, H] (fp32),
    starting from state S [n_seqs, H, dk, dv] fp32."""
    q: torch.Tensor
    k: torch.Tensor
    v: torch.Tensor
    beta: torch.Tensor
    g: torch.Tensor
    S: torch.Tensor
    cu_seqlens: list

    def to(self, device) -> "ChunkedDeltaCase":
        f = lambda t: t.to(device)
        return ChunkedDeltaCase(f(self.q), f(self.k), f(self.v), f(self.beta), f(self.g), f(self.S),
                                list(self.cu_seqlens))

    def lengths(self) -> list[int]:
        return [b - a for a, b in zip(self.cu_seqlens, self.cu_seqlens[1:])]

    def chunks(self) -> int:
        return sum(-(-n // 64) for n in self.lengths())

    def flops(self) -> int:
        """Algorithmic flops of the reference's chunked form per (chunk, head): five 64 x 64 x dk products (K K^T,
        Q K^T, A V, A K, P vn), three 64 x dk x dv products (W S, Q S, K^T vn) and the 64^3 / 3 substitution."""
        H, dk, dv = self.q.shape[1], self.q.shape[2], self.v.shape[2]
        per = 5 * 2 * 64 * 64 * dk + 3 * 2 * 64 * dk * dv + 64 ** 3 // 3
        return self.chunks() * H * per

    def hbm_bytes(self) -> int:
        """q, k, v and beta, g read once, o written once (fp32), the states read and written once."""
        N, H, dk = self.q.shape
        dv = self.v.shape[2]
        return N * H * (2 * dk * self.q.element_size() + dv * self.v.element_size() + 2 * 4 + dv * 4) + \
            2 * self.S.numel() * 4


def chunked_delta_case(lengths: list[int], H: int = DN_HEADS, dtype=torch.bfloat16, seed: int = 0,
                       state_scale: float = 0.0) -> ChunkedDeltaCase:
    """q, k ~ N(0,1) l2-normalised (q then * 1/sqrt(dk)), v ~ N(0,1), all stored in dtype; beta = sigmoid(N);
    g = -softplus(N); S0 = state_scale * N (0: zero state)."""
    gen = torch.Generator().manual_seed(seed)
    N = sum(lengths)
    r = lambda *s: torch.randn(*s, generator=gen)
    l2 = lambda x: x * torch.rsqrt((x * x).sum(-1, keepdim=True) + 1e-6)
    q = (l2(r(N, H, DN_DK)) * (1.0 / math.sqrt(DN_DK))).to(dtype)
    k = l2(r(N, H, DN_DK)).to(dtype)
    v = r(N, H, DN_DV).to(dtype)
    beta = torch.sigmoid(r(N, H))
    g = -torch.nn.functional.softplus(r(N, H))
    S = r(len(lengths), H, DN_DK, DN_DV) * state_scale
    cu = [0]
    for n in lengths:
        cu.append(cu[-1] + n)
    return ChunkedDeltaCase(q, k, v, beta, g, S, cu)


def c4_chunked_delta(seed: int = 4) -> ChunkedDeltaCase:
    """Config 4: batch 4 x 4096 tokens, 16 heads, dk = dv = 128, bf16 inputs, fp32 state starting at zero."""
    return chunked_delta_case([4096] * 4, seed=seed)


@dataclass
class LinearPrefillCase:
    """Packed prefill of one linear-attention layer around the delta rule (src/models/qwen3_5.py:128-162): the fused
    in_proj output y [N, C | H*dv | H | H] (qkv, z, beta logits, a; fp32, as the reference's linear returns), the
    layer's conv_w [C, K], A_log, dt_bias [H], norm_w [dv], segment offsets cu_seqlens, and per-segment states
    S [n, H, dk, dv], conv [n, K-1, C] fp32."""
    y: torch.Tensor
    conv_w: torch.Tensor
    A_log: torch.Tensor
    dt_bias: torch.Tensor
    norm_w: torch.Tensor
    S: torch.Tensor
    conv: torch.Tensor
    cu_seqlens: list
    eps: float = 1e-6
    dims: tuple = (DN_HEADS, DN_DK, DN_DV, KEY_DIM)

    def to(self, device) -> "LinearPrefillCase":
        f = lambda t: t.to(device)
        return LinearPrefillCase(f(self.y), f(self.conv_w), f(self.A_log), f(self.dt_bias), f(self.norm_w),
                                 f(self.S), f(self.conv), list(self.cu_seqlens), self.eps, self.dims)

    def cols(self):
        """(qkv, z, b, a): the column slices of y (strided rows), as the model takes them."""
        H, _, dv, _ = self.dims
        C = self.conv_w.shape[0]
        return self.y[:, :C], self.y[:, C:C + H * dv], self.y[:, -2 * H:-H], self.y[:, -H:]

    def front_bytes(self) -> int:
        """Algorithmic HBM bytes of the fused front (conv + split + norms + beta / g + tail handoff): the qkv, b, a
        columns read once, q, k, v, beta, g written once (fp32), conv_w read, each segment's tail read and written."""
        N = self.y.shape[0]
        H, dk, dv, _ = self.dims
        C, K = self.conv_w.shape
        xb = self.y.element_size()
        per_token = (C + 2 * H) * xb + (2 * H * dk + H * dv + 2 * H) * 4
        return N * per_token + C * K * 4 + 2 * (len(self.cu_seqlens) - 1) * (K - 1) * C * 4

    def norm_bytes(self) -> int:
        """rms_norm_gated: x [N*H, dv] fp32 and z read, out written, norm_w read."""
        N = self.y.shape[0]
        H, _, dv, _ = self.dims
        return N * H * dv * (4 + self.y.element_size() + 4) + dv * 4


def linear_prefill_case(lengths: list[int], dtype=torch.float32, seed: int = 0) -> LinearPrefillCase:
    """y ~ N(0, 1) (a column block * 3 to reach softplus's linear range), conv_w = 0.5 N, A_log, dt_bias = 0.5 N,
    norm_w = 1 + 0.1 N, states S = 0.05 N and conv tails N(0, 1)."""
    gen = torch.Generator().manual_seed(seed)
    r = lambda *s, scale=1.0: scale * torch.randn(*s, generator=gen)
    N, H, C = sum(lengths), DN_HEADS, CONV_DIM
    y = r(N, C + H * DN_DV + 2 * H)
    y[:, -H:] *= 3.0
    cu = [0]
    for n in lengths:
        cu.append(cu[-1] + n)
    return LinearPrefillCase(y.to(dtype), r(C, CONV_K, scale=0.5), r(H, scale=0.5), r(H, scale=0.5),
                             1.0 + r(DN_DV, scale=0.1), r(len(lengths), H, DN_DK, DN_DV, scale=0.05),
                             r(len(lengths), CONV_K - 1, C), cu)


def lp_linear_prefill(seed: int = 6) -> LinearPrefillCase:
    """The config-4 batch (4 x 4096 tokens, 16 heads x 128 x 128, conv 4 over 6144 channels) one step earlier: the
    fp32 in_proj output of a linear-attention layer, before conv, norms and the delta rule."""
    return linear_prefill_case([4096] * 4, seed=seed)


# ---------------------------------------------------------------- a whole hybrid decode step (decode_batch)

@dataclass
class HybridConfig:
    """Shapes of a Qwen3.5 hybrid stack (src/models/qwen3_5.py): every 4th layer (i % 4 == 3) full attention with
    a sigmoid output gate and partial RoPE, the rest Gated DeltaNet; SwiGLU MLPs; tied embedding / head."""
    layers: int
    hidden: int
    intermediate: int
    vocab: int
    Hq: int = HQ
    Hkv: int = HKV
    d: int = HEAD_DIM
    rot: int = 64
    theta: float = 1e7
    H: int = DN_HEADS
    dk: int = DN_DK
    dv: int = DN_DV
    conv_k: int = CONV_K
    eps: float = 1e-6
    block_size: int = BLOCK

    def is_full(self, i: int) -> bool:
        return i % 4 == 3

    @property
    def conv_dim(self) -> int:
        return 2 * self.H * self.dk + self.H * self.dv

    @property
    def in_proj_rows(self) -> int:
        return self.conv_dim + self.H * self.dv + 2 * self.H

    @property
    def qkvg_rows(self) -> int:
        return (2 * self.Hq + 2 * self.Hkv) * self.d


QWEN35_2B = HybridConfig(layers=24, hidden=2048, intermediate=6144, vocab=248320)


def hybrid_weight_shapes(cfg: HybridConfig) -> dict:
    """name -> shape of every weight, named as the reference's fused model tensors (so prepare() applies the same
    per-tensor precision policy); norm weights are stored as (1 + w), as the model's _vec(one_plus=True) hands them
    to the backend."""
    s = {"embed_tokens.weight": (cfg.vocab, cfg.hidden), "norm.weight": (cfg.hidden,)}
    for i in range(cfg.layers):
        p = f"layers.{i}."
        s[p + "input_layernorm.weight"] = (cfg.hidden,)
        s[p + "post_attention_layernorm.weight"] = (cfg.hidden,)
        s[p + "mlp.gate_up.weight"] = (2 * cfg.intermediate, cfg.hidden)
        s[p + "mlp.down_proj.weight"] = (cfg.hidden, cfg.intermediate)
        if cfg.is_full(i):
            s[p + "self_attn.qkvg.weight"] = (cfg.qkvg_rows, cfg.hidden)
            s[p + "self_attn.q_norm.weight"] = (cfg.d,)
            s[p + "self_attn.k_norm.weight"] = (cfg.d,)
            s[p + "self_attn.o_proj.weight"] = (cfg.hidden, cfg.Hq * cfg.d)
        else:
            s[p + "linear_attn.in_proj.weight"] = (cfg.in_proj_rows, cfg.hidden)
            s[p + "linear_attn.conv1d.weight"] = (cfg.conv_dim, cfg.conv_k)
            s[p + "linear_attn.A_log"] = (cfg.H,)
            s[p + "linear_attn.dt_bias"] = (cfg.H,)
            s[p + "linear_attn.norm.weight"] = (cfg.dv,)
            s[p + "linear_attn.out_proj.weight"] = (cfg.hidden, cfg.H * cfg.dv)
    return s


def hybrid_weights(cfg: HybridConfig, seed: int = 0) -> dict:
    """Seeded fp32 host weights of the stack (random init at the scale of a trained model's)."""
    gen = torch.Generator().manual_seed(seed)
    out = {}
    for name, shape in hybrid_weight_shapes(cfg).items():
        if name.endswith(("layernorm.weight", "norm.weight", "q_norm.weight", "k_norm.weight")):
            w = 1.0 + 0.1 * torch.randn(shape, generator=gen)
        elif name.endswith("conv1d.weight"):
            w = 0.5 * torch.randn(shape, generator=gen)
        elif name.endswith(("A_log", "dt_bias")):
            w = 0.5 * torch.randn(shape, generator=gen)
        else:
            w = torch.randn(shape, generator=gen) / math.sqrt(shape[1])
        out[name] = w
    return out


def random_device_weights(cfg: HybridConfig, scheme: str, dev, seed: int = 0) -> dict:
    """The same names and shapes drawn directly in the device format (random codes and fp16 scales for the 2-D
    weights, INT8 for the tied embedding in INT4 mode, per the reference's policy), for models too large to draw in
    fp32 on the host: a bandwidth workload, where the values do not change the work."""
    from quant import BLOCK as QB, QuantTensor, scheme_for
    gen = torch.Generator(device=dev).manual_seed(seed)
    out = {}
    for name, shape in hybrid_weight_shapes(cfg).items():
        if len(shape) == 2 and shape[1] % QB == 0 and not name.endswith("conv1d.weight"):
            N, K = shape
            sch = scheme_for(name, scheme)
            if sch == "int8":
                data = torch.randint(-127, 128, (N, K), generator=gen, device=dev, dtype=torch.int8)
            else:
                data = torch.randint(0, 256, (N, K // 2), generator=gen, device=dev, dtype=torch.uint8)
            scale = 2.0 / (127 if sch == "int8" else 15) / math.sqrt(K)
            scales = (torch.rand(N, K // QB, generator=gen, device=dev) * scale + 0.5 * scale).to(torch.float16)
            mins = (-7.5 * scales.float()).to(torch.float16) if sch == "int4" else None
            out[name] = QuantTensor(sch, data, scales, (N, K), QB, mins)
        else:
            t = torch.randn(shape, generator=gen, device=dev)
            out[name] = 1.0 + 0.1 * t if name.endswith("norm.weight") else 0.5 * t
    return out


class StateSlots:
    """Gated DeltaNet state of max_seqs sequences in the engine's pool layout (src/state.py:428-429):
    S [max_seqs, n_linear, H, dk, dv] and conv [max_seqs, n_linear, K-1, C], fp32. views(rows) hands out one object
    per sequence with the attributes the backend reads from the engine's states (pool, seq, S, conv_tail), and
    seq_index(states) the rows of a batch as a device int32 tensor, cached per batch composition."""

    def __init__(self, max_seqs: int, n_linear: int, H: int, dk: int, dv: int, conv_dim: int, conv_k: int,
                 device="cpu"):
        self.S = torch.zeros(max_seqs, n_linear, H, dk, dv, device=device, dtype=torch.float32)
        self.conv = torch.zeros(max_seqs, n_linear, conv_k - 1, conv_dim, device=device, dtype=torch.float32)
        self._index: dict[tuple, torch.Tensor] = {}

    def views(self, rows) -> list:
        return [SlotView(self, int(r)) for r in rows]

    def seq_index(self, states) -> torch.Tensor:
        key = tuple(st.seq for st in states)
        if key not in self._index:
            from native.kernels import to_device
            self._index[key] = to_device(torch.tensor(key, dtype=torch.int32), self.S.device)
        return self._index[key]


class SlotView:
    """One sequence's row of a StateSlots."""

    def __init__(self, pool: StateSlots, seq: int):
        self.pool, self.seq = pool, seq
        self.S, self.conv_tail = pool.S[seq], pool.conv[seq]


class HybridDecodeState:
    """The sequences of one decode batch in the engine's layouts: a KV pool layer per attention layer (bf16, blocks
    scattered over the pool) and a DeltaNet state row per sequence (S and conv tails of every DeltaNet layer), with
    histories of `lens` positions already written (seeded random K / V, S ~ N(0, 0.02^2), tails ~ N(0, 1)). The
    blocks for one more position are in the tables."""

    def __init__(self, cfg: HybridConfig, lens: list[int], device, seed: int = 0, kv_dtype=torch.bfloat16):
        self.cfg = cfg
        self.lens = list(lens)
        n_full = sum(cfg.is_full(i) for i in range(cfg.layers))
        n_linear = cfg.layers - n_full
        bs = cfg.block_size
        gen = torch.Generator().manual_seed(seed)
        num_blocks = sum(math.ceil((L + 1) / bs) for L in lens) + 1
        self.tables = scattered_tables([L + 1 for L in lens], num_blocks, bs, gen)
        self.k, self.v = kv_pool((n_full, num_blocks, bs, cfg.Hkv, cfg.d), device, kv_dtype)
        self.k.copy_(torch.randn(self.k.shape, generator=gen).to(kv_dtype))
        self.v.copy_(torch.randn(self.v.shape, generator=gen).to(kv_dtype))
        self.pool = StateSlots(len(lens), n_linear, cfg.H, cfg.dk, cfg.dv, cfg.conv_dim, cfg.conv_k, device)
        self.pool.S.copy_(0.02 * torch.randn(self.pool.S.shape, generator=gen))
        self.pool.conv.copy_(torch.randn(self.pool.conv.shape, generator=gen))
        self.seqs = self.pool.views(range(len(lens)))
        # layer slots: attention layers index the KV pool, DeltaNet layers the state pool (the model's self.slot)
        self.slot, nf, nl = [], 0, 0
        for i in range(cfg.layers):
            self.slot.append(nf if cfg.is_full(i) else nl)
            nf, nl = nf + cfg.is_full(i), nl + (not cfg.is_full(i))

    def layout(self):
        """One step's KV layout (src/models/qwen3_5.py:237-245): the pool row each new token is written to
        (block * block_size + offset, int64), the tables, the lengths after the step and the new tokens'
        positions, as device tensors."""
        from native.kernels import to_device
        bs, dev = self.cfg.block_size, self.k.device
        slots = torch.tensor([int(self.tables[i, L // bs]) * bs + L % bs for i, L in enumerate(self.lens)])
        lens = torch.tensor([L + 1 for L in self.lens], dtype=torch.int32)
        positions = torch.tensor(self.lens, dtype=torch.int32)
        return tuple(to_device(t, dev) for t in (slots, self.tables, lens, positions))


def hybrid_decode_step(backend, w: dict, st: HybridDecodeState, tokens: torch.Tensor, layout) -> torch.Tensor:
    """One decode step for the batch through the backend protocol, in the order of Qwen3_5Model.decode_batch
    (src/models/qwen3_5.py:228-290) -> logits [B, vocab] fp32. The attention layer's q / k norms, partial RoPE and
    KV write are the one fused attention_prep call, the output gate is fused into paged_attention, and (with a
    backend that has rms_norm_swiglu) the MLP is the reference's swiglu then linear, with silu * up in the gate_up
    projection's epilogue (else, with one that has silu_mul_linear, inside the down projection), and (with one that
    has rms_norm_linear) every RMSNorm after the first runs inside the linear that follows it, from the sums of squares
    the linear before it returned; with one that has decode_plan, the attention layers share one batch layout plan;
    the sequences' lengths are not advanced (a benchmark replays the same step)."""
    cfg = st.cfg
    B = tokens.shape[0]
    slots, tables, lens, positions = layout
    fused = hasattr(backend, "silu_mul_linear")
    fused_norm = hasattr(backend, "rms_norm_linear")
    fused_swiglu = fused_norm and hasattr(backend, "rms_norm_swiglu")
    ss = None                       # sums of squares of h's 16-column tiles, from the linear that wrote h

    def norm_linear(h, norm_w, wt):
        if fused_norm and ss is not None:
            return backend.rms_norm_linear(h, ss, norm_w, cfg.eps, wt)
        return backend.linear(backend.rms_norm(h, norm_w, cfg.eps), wt)

    def residual_linear(x, wt, h):
        if fused_norm:
            return backend.linear_ss(x, wt, residual=h)
        return backend.linear(x, wt, residual=h), None

    h = backend.embedding(w["embed_tokens.weight"], tokens)
    # every attention layer of the step decodes the same batch layout: its plan is made once (with a backend that
    # has decode_plan) and read by each layer's paged attention
    plan = None
    if hasattr(backend, "decode_plan") and any(cfg.is_full(i) for i in range(cfg.layers)):
        k0 = st.k[st.slot[next(i for i in range(cfg.layers) if cfg.is_full(i))]]
        plan = backend.decode_plan(tables, lens, cfg.block_size, cfg.Hq, cfg.Hkv, cfg.d, k0.shape[0])
    for i in range(cfg.layers):
        p = f"layers.{i}."
        L = st.slot[i]
        if cfg.is_full(i):
            a = p + "self_attn."
            y = norm_linear(h, w[p + "input_layernorm.weight"], w[a + "qkvg.weight"])
            q, gate = backend.attention_prep(y, w[a + "q_norm.weight"], w[a + "k_norm.weight"], cfg.eps, positions,
                                             cfg.theta, cfg.rot, (cfg.Hq, cfg.Hkv, cfg.d), st.k[L], st.v[L], slots)
            o = backend.paged_attention(q, st.k[L], st.v[L], tables, lens, cfg.block_size, gate=gate,
                                        **({"plan": plan} if plan is not None else {}))
            h, ss = residual_linear(o.reshape(B, cfg.Hq * cfg.d), w[a + "o_proj.weight"], h)
        else:
            a = p + "linear_attn."
            y = norm_linear(h, w[p + "input_layernorm.weight"], w[a + "in_proj.weight"])
            C, Z, H = cfg.conv_dim, cfg.H * cfg.dv, cfg.H
            o = backend.deltanet_decode_batch(y[:, :C], y[:, C:C + Z], y[:, C + Z:C + Z + H], y[:, C + Z + H:],
                                              st.seqs, L, w[a + "conv1d.weight"], w[a + "A_log"], w[a + "dt_bias"],
                                              w[a + "norm.weight"], cfg.eps, (H, cfg.dk, cfg.dv, H * cfg.dk))
            h, ss = residual_linear(o, w[a + "out_proj.weight"], h)
        if fused_swiglu:
            act = backend.rms_norm_swiglu(h, ss, w[p + "post_attention_layernorm.weight"], cfg.eps,
                                          w[p + "mlp.gate_up.weight"])
            h, ss = residual_linear(act, w[p + "mlp.down_proj.weight"], h)
            continue
        gu = norm_linear(h, w[p + "post_attention_layernorm.weight"], w[p + "mlp.gate_up.weight"])
        F = gu.shape[1] // 2
        if fused_norm:
            h, ss = backend.silu_mul_linear_ss(gu[:, :F], gu[:, F:], w[p + "mlp.down_proj.weight"], residual=h)
        elif fused:
            h = backend.silu_mul_linear(gu[:, :F], gu[:, F:], w[p + "mlp.down_proj.weight"], residual=h)
        else:
            h = backend.linear(backend.silu_mul(gu[:, :F], gu[:, F:]), w[p + "mlp.down_proj.weight"], residual=h)
    return norm_linear(h, w["norm.weight"], w["embed_tokens.weight"])
