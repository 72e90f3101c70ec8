"""Tensor-level wrappers of the C ABI: argument checks, dtype codes, output / workspace allocation, current stream.

PyTorch is used here only for device memory and the stream: every computation is a HIP kernel of librk_path.so.
Checks mirror the reference's host-side refusals (MetalBackend._kv_kernel raises TypeError for a KV dtype it has no
kernel for, src/backend/metal.py:189-195) and turn shape mistakes into ValueError before anything is launched.
"""
import math

import torch

from native.rocm_native import RK_BF16, RK_F32, RK_W_BF16, RK_W_INT4, RK_W_INT8, load

DTYPE_CODES = {torch.float32: RK_F32, torch.bfloat16: RK_BF16}
KV_DTYPES = (torch.float32, torch.bfloat16)

_workspaces: dict[int, torch.Tensor] = {}
# Buffers replaced by a larger one are kept until the process ends, never freed: a HIP graph captured before the
# growth still holds their addresses and writes there on every replay, so the allocator must not hand them out again.
_retired: list[torch.Tensor] = []


def to_device(t: torch.Tensor, device) -> torch.Tensor:
    """A small host tensor (offsets, positions, work lists) on `device`, copied without waiting for queued kernels:
    from a private pinned clone, which keeps the host bytes unchanged until the copy has read them whatever the
    caller does with its own tensor afterwards."""
    dev = torch.device(device)
    if dev.type != "cuda":
        return t.to(dev)
    return t.clone().pin_memory().to(dev, non_blocking=True)


def _stream(dev: torch.device) -> int:
    return torch.cuda.current_stream(dev).cuda_stream


def _need_cuda(name: str, *ts: torch.Tensor) -> torch.device:
    dev = ts[0].device
    for t in ts:
        if t.device.type != "cuda":
            raise ValueError(f"{name}: tensors must be on a ROCm device, got {t.device}")
        if t.device != dev:
            raise ValueError(f"{name}: tensors on different devices ({dev}, {t.device})")
    return dev


def _contig(name: str, t: torch.Tensor, arg: str) -> torch.Tensor:
    if not t.is_contiguous():
        raise ValueError(f"{name}: {arg} must be contiguous")
    return t


def workspace(dev: torch.device, nbytes: int) -> torch.Tensor:
    """A device scratch buffer of at least nbytes, reused across calls on the device (calls are stream-ordered)."""
    idx = dev.index if dev.index is not None else torch.cuda.current_device()
    buf = _workspaces.get(idx)
    if buf is None or buf.numel() < nbytes:
        if buf is not None:
            _retired.append(buf)
        grow = 2 * buf.numel() if buf is not None else 0      # geometric growth bounds the retired total
        buf = torch.empty(max(nbytes, 1 << 20, grow), dtype=torch.uint8, device=dev)
        _workspaces[idx] = buf
    return buf


_cus: dict[int, int] = {}


def device_cus(dev: torch.device) -> int:
    """The device's compute units (256 on an MI355X), read once per device."""
    idx = dev.index if dev.index is not None else torch.cuda.current_device()
    if idx not in _cus:
        _cus[idx] = torch.cuda.get_device_properties(idx).multi_processor_count
    return _cus[idx]


class DecodePlan:
    """A decode step's batch layout plan (rk_paged_decode_plan): made once from the step's block tables and lengths,
    read by every attention layer's paged_decode of that step. It records the layout it was made for; paged_decode
    refuses it for another one. It does not follow later writes into the same tables / lens tensors: make a new
    plan whenever they change (every decode step)."""

    def __init__(self, buf: torch.Tensor, key: tuple):
        self.buf, self.key = buf, key


def _plan_key(tables, lens, block_size, Hq, Hkv, d, num_blocks, window):
    return (tables.data_ptr(), lens.data_ptr(), tuple(tables.shape), int(block_size), int(Hq), int(Hkv), int(d),
            int(num_blocks), int(window or 0))


def decode_plan(tables, lens, block_size: int, Hq: int, Hkv: int, d: int, num_blocks: int,
                window: int | None = None) -> DecodePlan:
    """rk_paged_decode_plan: the split partition and each wave group's first tiles of one decode step's batch
    (tables [B, max_nb] int32, lens [B] int32 on the device) for pools of num_blocks blocks of block_size positions,
    Hq / Hkv heads of head_dim d; one launch, no host sync."""
    name = "decode_plan"
    B, max_nb = tables.shape
    if lens.shape != (B,) or tables.dtype != torch.int32 or lens.dtype != torch.int32:
        raise ValueError(f"{name}: tables {tuple(tables.shape)} {tables.dtype}, lens {tuple(lens.shape)} {lens.dtype}")
    dev = _need_cuda(name, tables, lens)
    _contig(name, tables, "tables"); _contig(name, lens, "lens")
    lib = load()
    n = lib.lib.rk_paged_decode_plan_ints(B, Hq, Hkv, d, block_size, max_nb)
    buf = torch.empty(n, dtype=torch.int32, device=dev)
    lib.call("rk_paged_decode_plan", buf.data_ptr(), n, tables.data_ptr(), lens.data_ptr(), B, Hq, Hkv, d,
             int(block_size), max_nb, int(num_blocks), int(window or 0), _stream(dev))
    return DecodePlan(buf, _plan_key(tables, lens, block_size, Hq, Hkv, d, num_blocks, window))


def paged_decode(q, k_pool, v_pool, tables, lens, block_size: int, window: int | None = None, gate=None,
                 out=None, phase: int | None = None, plan: DecodePlan | None = None) -> torch.Tensor:
    """Batched decode attention over one layer of a paged pool (rk_paged_decode). q [B, Hq, d] -> [B, Hq, d] fp32.
    k_pool / v_pool [num_blocks, block_size, Hkv, d] fp32 or bf16; tables [B, max_nb] int32; lens [B] int32;
    gate None or [B, Hq * d] (out *= sigmoid(gate); rows may be strided). plan: the step's decode_plan for these
    tables and lens (rk_paged_decode_planned; the same bits, a shorter start). phase 0 / 1 runs one of the two
    launches (for timing)."""
    name = "paged_attention"
    if k_pool.dtype != v_pool.dtype or k_pool.dtype not in KV_DTYPES:
        raise TypeError(f"{name}: keys and values must both be float32 or bfloat16, not "
                        f"{k_pool.dtype} / {v_pool.dtype}")
    if q.dim() != 3 or k_pool.dim() != 4 or k_pool.shape != v_pool.shape:
        raise ValueError(f"{name}: q {tuple(q.shape)}, pools {tuple(k_pool.shape)} / {tuple(v_pool.shape)}")
    B, Hq, d = q.shape
    NB, bs, Hkv, dp = k_pool.shape
    if dp != d or bs != block_size:
        raise ValueError(f"{name}: pool [{NB}, {bs}, {Hkv}, {dp}] vs head_dim {d}, block_size {block_size}")
    if tables.dim() != 2 or tables.shape[0] != B or lens.shape != (B,):
        raise ValueError(f"{name}: tables {tuple(tables.shape)} / lens {tuple(lens.shape)} for batch {B}")
    if tables.dtype != torch.int32 or lens.dtype != torch.int32:
        raise TypeError(f"{name}: tables and lens must be int32, not {tables.dtype} / {lens.dtype}")
    dev = _need_cuda(name, q, k_pool, v_pool, tables, lens)
    _contig(name, k_pool, "k_pool"); _contig(name, v_pool, "v_pool")
    _contig(name, tables, "tables"); _contig(name, lens, "lens")
    q = q.to(torch.float32).contiguous()
    if gate is not None:
        # rows of Hq * d fp32 at any 16-byte-aligned stride (the gate columns of a projection output: no copy)
        gate = gate.to(torch.float32)
        if gate.dim() != 2:
            gate = gate.reshape(B, -1)
        if gate.shape != (B, Hq * d):
            raise ValueError(f"{name}: gate {tuple(gate.shape)}, expected [{B}, {Hq * d}]")
        if gate.stride(1) != 1 or gate.stride(0) % 4 or gate.data_ptr() % 16:
            gate = gate.contiguous() if not gate.is_contiguous() else gate.clone()
        _need_cuda(name, q, gate)
    if out is None:
        out = torch.empty(B, Hq, d, dtype=torch.float32, device=dev)
    lib = load()
    max_nb = tables.shape[1]
    need = lib.lib.rk_paged_decode_workspace_bytes(B, Hq, Hkv, d, bs, max_nb)
    ws = workspace(dev, need)
    if plan is not None and plan.key != _plan_key(tables, lens, bs, Hq, Hkv, d, NB, window):
        raise ValueError(f"{name}: the plan was made for another batch layout or shape")
    head = (out.data_ptr(), q.data_ptr(), k_pool.data_ptr(), v_pool.data_ptr(), DTYPE_CODES[k_pool.dtype],
            tables.data_ptr(), lens.data_ptr(), B, Hq, Hkv, d, bs, max_nb, NB, int(window or 0),
            gate.data_ptr() if gate is not None else None, gate.stride(0) if gate is not None else 0)
    tail = (ws.data_ptr(), ws.numel(), _stream(dev))
    pl = (plan.buf.data_ptr(), plan.buf.numel()) if plan is not None else (None, 0)
    if phase is not None:
        lib.call("rk_paged_decode_phase", int(phase), *head, *pl, *tail)
    elif plan is not None:
        lib.call("rk_paged_decode_planned", *head, *pl, *tail)
    else:
        lib.call("rk_paged_decode", *head, *tail)
    return out


def kv_write(k_pool, v_pool, slots, k, v) -> None:
    """pool[slots // bs, slots % bs] = k / v for a [num_blocks, bs, Hkv, d] pool layer (rk_kv_write). slots int64."""
    name = "kv_write"
    n = slots.numel()
    if n == 0:
        return
    if k_pool.dtype not in KV_DTYPES or v_pool.dtype != k_pool.dtype:
        raise TypeError(f"{name}: pool dtype {k_pool.dtype} / {v_pool.dtype}")
    NB, bs, Hkv, d = k_pool.shape
    k = k.reshape(n, Hkv, d)
    v = v.reshape(n, Hkv, d)
    if k.dtype not in KV_DTYPES:
        k = k.float()
    if v.dtype != k.dtype:
        v = v.to(k.dtype)
    k, v = k.contiguous(), v.contiguous()
    slots = slots.to(device=k_pool.device, dtype=torch.int64).contiguous()
    dev = _need_cuda(name, k_pool, v_pool, slots, k, v)
    _contig(name, k_pool, "k_pool"); _contig(name, v_pool, "v_pool")
    load().call("rk_kv_write", k_pool.data_ptr(), v_pool.data_ptr(), DTYPE_CODES[k_pool.dtype], slots.data_ptr(),
                k.data_ptr(), v.data_ptr(), DTYPE_CODES[k.dtype], n, Hkv, d, bs, NB, _stream(dev))


def kv_gather(k_pool, v_pool, table, lo: int, end: int) -> tuple[torch.Tensor, torch.Tensor]:
    """Positions lo .. end-1 of one sequence, gathered through its block table (int32 device tensor)."""
    name = "kv_gather"
    NB, bs, Hkv, d = k_pool.shape
    dev = _need_cuda(name, k_pool, v_pool, table)
    table = table.to(torch.int32).contiguous()
    ko = torch.empty(end - lo, Hkv, d, dtype=k_pool.dtype, device=dev)
    vo = torch.empty(end - lo, Hkv, d, dtype=v_pool.dtype, device=dev)
    if end > lo:
        load().call("rk_kv_gather", ko.data_ptr(), vo.data_ptr(), k_pool.data_ptr(), v_pool.data_ptr(),
                    DTYPE_CODES[k_pool.dtype], table.data_ptr(), table.numel(), lo, end, Hkv, d, bs, NB,
                    _stream(dev))
    return ko, vo


def deltanet_decode(qkv, z, b, a, conv_state, S, seq_index, slot: int, conv_w, A_log, dt_bias, norm_w,
                    eps: float, dims) -> torch.Tensor:
    """One fused Gated DeltaNet decode step for B sequences (rk_deltanet_decode) -> [B, H * dv] fp32.
    conv_state [seqs, n_linear, K-1, C] and S [seqs, n_linear, H, dk, dv] (fp32, contiguous) are updated in place at
    [seq_index[i], slot]."""
    name = "deltanet_decode"
    H, dk, dv, key_dim = dims
    if key_dim != H * dk:
        raise ValueError(f"{name}: key_dim {key_dim} != H * dk = {H * dk}")
    B, C = qkv.shape
    if C != 2 * key_dim + H * dv:
        raise ValueError(f"{name}: qkv has {C} channels, expected {2 * key_dim + H * dv}")
    if S.dtype != torch.float32 or conv_state.dtype != torch.float32:
        raise TypeError(f"{name}: state must be float32, not {S.dtype} / {conv_state.dtype}")
    if S.dim() != 5 or S.shape[2:] != (H, dk, dv) or conv_state.dim() != 4 or conv_state.shape[3] != C:
        raise ValueError(f"{name}: S {tuple(S.shape)}, conv {tuple(conv_state.shape)}")
    n_linear = S.shape[1]
    K = conv_w.shape[1]
    if conv_state.shape[1] != n_linear or conv_state.shape[2] != K - 1:
        raise ValueError(f"{name}: conv state {tuple(conv_state.shape)} vs {n_linear} layers, kernel {K}")
    if not 0 <= slot < n_linear:
        raise ValueError(f"{name}: slot {slot} outside [0, {n_linear})")
    dev = _need_cuda(name, qkv, S, conv_state)
    _contig(name, S, "S"); _contig(name, conv_state, "conv_state")
    f = lambda t: t.to(device=dev, dtype=torch.float32).contiguous()
    # qkv / z / b / a are read in place with their row strides (column slices of one in_proj output row: no copies)
    rowwise = lambda t: t if t.dtype == torch.float32 and t.device == dev and t.stride(-1) == 1 else f(t)
    qkv, z, b, a = rowwise(qkv), rowwise(z), rowwise(b), rowwise(a)
    if z.shape != (B, H * dv) or b.shape != (B, H) or a.shape != (B, H):
        raise ValueError(f"{name}: z {tuple(z.shape)}, b {tuple(b.shape)}, a {tuple(a.shape)} for batch {B}, {H} heads")
    ld = lambda t: t.stride(0) if t.shape[0] > 1 else t.shape[1]     # a 1-row view's stride is arbitrary
    if ld(b) != ld(a):
        b, a = b.contiguous(), a.contiguous()
    conv_w, A_log, dt_bias, norm_w = f(conv_w), f(A_log), f(dt_bias), f(norm_w)
    seq_index = seq_index.to(device=dev, dtype=torch.int32).contiguous()
    out = torch.empty(B, H * dv, dtype=torch.float32, device=dev)
    load().call("rk_deltanet_decode", out.data_ptr(), qkv.data_ptr(), z.data_ptr(), b.data_ptr(), a.data_ptr(),
                ld(qkv), ld(z), ld(b), conv_state.data_ptr(), S.data_ptr(), conv_w.data_ptr(), A_log.data_ptr(), dt_bias.data_ptr(),
                norm_w.data_ptr(), seq_index.data_ptr(), B, H, dk, dv, K, n_linear, int(slot), float(eps),
                _stream(dev))
    return out


PREFILL_BLOCK = 32          # queries per work item of rk_paged_prefill
PREFILL_TILE = 32           # key positions per tile of rk_paged_prefill
PREFILL_SPLIT_TILES = None  # None: split only when the blocks x KV heads leave CUs idle; an int forces a split size
PREFILL_MIN_SPLIT = 32      # the smallest automatic piece, in tiles (1024 keys: the merge stays a small fraction)
PREFILL_BALANCE_PIECES = 4  # balance split: no piece above 1/4 of a CU's share of the tiles


def prefill_split_tiles(spans: list[int], heads: int, n_cu: int, balance: bool = False) -> int:
    """The automatic split size of rk_paged_prefill's work list, from the key span (in tiles) of each 32-query
    block. When the blocks times the KV heads (workgroups per block) leave CUs without a workgroup: the size that
    cuts the total into about one workgroup per CU, at least PREFILL_MIN_SPLIT tiles (one long chunk over a long
    prefix: a 512-query chunk is 16 blocks, 32 workgroups with 2 KV heads, on 256 CUs). Otherwise 0 (no split),
    unless balance: then blocks longer than 1/PREFILL_BALANCE_PIECES of a CU's share are cut to that size (at least
    2 PREFILL_MIN_SPLIT tiles), so that the last workgroups to start end close together. balance is for the
    fp32-operand kernel (one workgroup per CU, where a packed batch like config 5's 632 uneven workgroups on 256
    CUs leaves ~14% of the CU time idle at the end); a piece costs a partial record and its share of the merge,
    and on the bf16-operand kernel the longer start-up of its producer pipeline outweighs the gain."""
    if not spans:
        return 0
    total = sum(spans) * heads
    if len(spans) * heads < n_cu:
        return max(PREFILL_MIN_SPLIT, -(-total // n_cu))
    if balance:
        size = max(2 * PREFILL_MIN_SPLIT, -(-total // (n_cu * PREFILL_BALANCE_PIECES)))
        return size if max(spans) > size else 0
    return 0


def prefill_work(lengths: list[int], starts: list[int], window: int | None = None, causal: bool = True,
                 split_tiles: int | None = PREFILL_SPLIT_TILES, heads: int = 1,
                 n_cu: int = 256, balance: bool = False) -> tuple[list[int], int]:
    """The work list of rk_paged_prefill -> (entries, partial slots used). One entry of 5 int32 per block of 32 new
    queries, {(segment << 16) | block, first tile, end tile, first slot or -1, (piece << 16) | pieces}; a block whose
    key range spans more than split_tiles tiles of 32 positions is split at absolute multiples of split_tiles into
    pieces (consecutive partial slots), which the kernel combines in piece order. split_tiles None takes
    prefill_split_tiles over the blocks (heads = workgroups per block, n_cu = the device's CUs, balance as there);
    0 never splits. For a given
    split size, where a block is cut depends only on the block, so a segment packed with others gives the same
    bits as the segment alone under the same split size. Entries go longest first, so the longest start first (a
    window bounds a block's range to about W + 32 keys; without causal masking every block of a segment reads all
    of its keys)."""
    blocks = []
    for s, (n, p) in enumerate(zip(lengths, starts)):
        for qb in range(-(-n // PREFILL_BLOCK)):
            hi = p + min(n, (qb + 1) * PREFILL_BLOCK) if causal else p + n
            lo = max(0, p + qb * PREFILL_BLOCK - window + 1) if window else 0
            blocks.append(((s << 16) | qb, lo // PREFILL_TILE, -(-hi // PREFILL_TILE)))
    if split_tiles is None:
        split_tiles = prefill_split_tiles([t1 - t0 for _, t0, t1 in blocks], heads, n_cu, balance)
    entries, n_slots = [], 0
    for word, t0, t1 in blocks:
        if split_tiles <= 0 or t1 - t0 <= split_tiles:
            entries.append((t1 - t0, [word, t0, t1, -1, 1]))
            continue
        cuts = [t0] + list(range((t0 // split_tiles + 1) * split_tiles, t1, split_tiles)) + [t1]
        pieces = len(cuts) - 1
        for i in range(pieces):
            entries.append((cuts[i + 1] - cuts[i], [word, cuts[i], cuts[i + 1], n_slots, (i << 16) | pieces]))
        n_slots += pieces
    entries.sort(key=lambda x: -x[0])
    return [v for _, e in entries for v in e], n_slots


PREFILL_F32_HEADS = 4       # query heads per workgroup of rk_paged_prefill's 16-query kernels (fp32 and bf16 operands)


def prefill_kernel(q_dtype, pool_dtype, Hq: int, Hkv: int, d: int, exact: bool, max_nb: int = 1,
                   block_size: int = 16) -> str:
    """Which kernel rk_paged_prefill runs (its rule, include/rk_path.h): "bf16_32" (bf16 operands, 32 queries per
    wave) for bf16 q and pool at 4 query heads per kv-head, head_dim 128 / 256, block size >= 2 and positions x
    block size below 2^32; "bf16_16" (bf16 operands, 16 queries per wave) for every other bf16 q and pool; "fp32"
    (fp32 operands) for an fp32 q or pool and for exact requests."""
    if exact or q_dtype != torch.bfloat16 or pool_dtype != torch.bfloat16:
        return "fp32"
    if Hq == 4 * Hkv and d in (128, 256) and block_size >= 2 and max_nb * block_size * block_size < 2 ** 32:
        return "bf16_32"
    return "bf16_16"


def prefill_bf16_operands(q_dtype, pool_dtype, Hq: int, Hkv: int, d: int, exact: bool, max_nb: int = 1,
                          block_size: int = 16) -> bool:
    """Whether rk_paged_prefill runs on bf16 MFMA operands: q and the pool both bf16 and no exact request."""
    return prefill_kernel(q_dtype, pool_dtype, Hq, Hkv, d, exact, max_nb, block_size) != "fp32"


def _prefill_launch(out, q, k_new, v_new, k_pool, v_pool, tables, cu: list[int], st: list[int], gate,
                    window: int, causal: bool, exact: bool = False) -> None:
    """rk_paged_prefill with the host-side segment offsets, start positions and work list in one int32 array, and
    the partial records / arrival counters of split blocks from the device's shared workspace."""
    S = len(st)
    N, Hq, d = q.shape
    NB, bs, Hkv, _ = k_pool.shape
    dev = q.device
    # workgroups per 32-query block: one per kv-head, times the head chunks of the 16-query kernels
    which = prefill_kernel(q.dtype, k_pool.dtype, Hq, Hkv, d, exact, tables.shape[1], bs)
    wg_heads = Hkv if which == "bf16_32" else Hkv * -(-(Hq // Hkv) // PREFILL_F32_HEADS)
    work, n_slots = prefill_work([b - a for a, b in zip(cu, cu[1:])], st, window, causal, PREFILL_SPLIT_TILES,
                                 wg_heads, device_cus(dev), balance=which == "fp32")
    meta = to_device(torch.tensor(cu + st + work, dtype=torch.int32), dev)
    n_work = len(work) // 5
    lib = load()
    part_ptr, part_bytes, cnt_ptr, n_cnt = None, 0, None, 0
    if n_slots:
        part_bytes = lib.lib.rk_paged_prefill_workspace_bytes(n_slots, Hq, d)
        part_ptr = workspace(dev, part_bytes).data_ptr()
        n_cnt = lib.lib.rk_paged_prefill_counters(n_slots, Hq)
        cnt_ptr = linear_counters(dev, n_cnt).data_ptr()
    lib.call("rk_paged_prefill", out.data_ptr(), q.data_ptr(), DTYPE_CODES[q.dtype],
             k_new.data_ptr() if k_new is not None else None, v_new.data_ptr() if v_new is not None else None,
             DTYPE_CODES[k_new.dtype] if k_new is not None else DTYPE_CODES[torch.float32],
             k_pool.data_ptr(), v_pool.data_ptr(), DTYPE_CODES[k_pool.dtype], tables.data_ptr(), tables.shape[1],
             meta.data_ptr(), meta.data_ptr() + 4 * (S + 1), meta.data_ptr() + 4 * (2 * S + 1), n_work, S, N, Hq,
             Hkv, d, bs, NB, gate.data_ptr() if gate is not None else None,
             DTYPE_CODES[gate.dtype] if gate is not None else DTYPE_CODES[torch.float32], int(window or 0),
             1 if causal else 0, 1 if exact else 0, n_slots, part_ptr, part_bytes, cnt_ptr, n_cnt, _stream(dev))


def _prefill_shape_check(name: str, Hq: int, Hkv: int, d: int) -> None:
    if Hkv < 1 or Hq < Hkv or Hq % Hkv:
        raise ValueError(f"{name}: {Hq} query heads do not split into groups over {Hkv} kv-heads")
    if d not in (64, 128, 256):
        raise NotImplementedError(f"{name}: the prefill attention kernels are built for head_dim 64, 128 or 256, "
                                  f"not {d}")


def paged_prefill(q, k_new, v_new, k_pool, v_pool, tables, cu_seqlens, start_pos, block_size: int, gate=None,
                  out=None, window: int | None = None, exact: bool = False) -> torch.Tensor:
    """Packed prefill attention (rk_paged_prefill): writes the new K/V rows into one pool layer, then causal GQA
    attention of every segment's new queries over its prefix + new keys -> [N, Hq, d] fp32 (* sigmoid(gate)); with a
    window W each query sees only its last W positions. cu_seqlens (S + 1 row offsets) and start_pos (S absolute
    positions) are host-side lists / CPU tensors, as the packing step produces them; tables [S, max_nb] int32 on
    the device. fp32 operands (fp32-level results) unless q and the pool are both bf16 (then bf16 MFMA operands,
    probabilities rounded to bf16); exact=True asks for fp32 operands there too."""
    name = "paged_prefill"
    cu = [int(x) for x in cu_seqlens]
    st = [int(x) for x in start_pos]
    S = len(st)
    if len(cu) != S + 1 or cu[0] != 0 or any(b < a for a, b in zip(cu, cu[1:])):
        raise ValueError(f"{name}: cu_seqlens {cu[:8]}... must be S + 1 non-decreasing offsets from 0")
    if window is not None and window < 1:
        raise ValueError(f"window must be at least 1, not {window}")
    N, Hq, d = q.shape
    if cu[-1] != N or k_new.shape[0] != N or v_new.shape != k_new.shape:
        raise ValueError(f"{name}: q {tuple(q.shape)}, k_new {tuple(k_new.shape)}, cu_seqlens end {cu[-1]}")
    if k_pool.dtype != v_pool.dtype or k_pool.dtype not in KV_DTYPES:
        raise TypeError(f"{name}: pools must both be float32 or bfloat16, not {k_pool.dtype} / {v_pool.dtype}")
    NB, bs, Hkv, dp = k_pool.shape
    if dp != d or bs != block_size or k_new.shape[1:] != (Hkv, d):
        raise ValueError(f"{name}: pool {tuple(k_pool.shape)} vs q {tuple(q.shape)}, k_new {tuple(k_new.shape)}")
    _prefill_shape_check(name, Hq, Hkv, d)
    if tables.dim() != 2 or tables.shape[0] != S or tables.dtype != torch.int32:
        raise ValueError(f"{name}: tables {tuple(tables.shape)} {tables.dtype} for {S} segments")
    for s in range(S):
        if st[s] < 0 or -(-(st[s] + cu[s + 1] - cu[s]) // bs) > tables.shape[1]:
            raise ValueError(f"{name}: segment {s} reaches position {st[s] + cu[s + 1] - cu[s]}, table covers "
                             f"{tables.shape[1] * bs}")
    dev = _need_cuda(name, q, k_new, v_new, k_pool, v_pool, tables)
    _contig(name, k_pool, "k_pool"); _contig(name, v_pool, "v_pool"); _contig(name, tables, "tables")
    as_kv = lambda t: t if t.dtype in KV_DTYPES else t.float()
    q, k_new, v_new = as_kv(q).contiguous(), as_kv(k_new).contiguous(), as_kv(v_new).to(as_kv(k_new).dtype).contiguous()
    if gate is not None:
        gate = (gate if gate.dtype in KV_DTYPES else gate.float()).contiguous()   # bf16 / fp32 read as stored
        if gate.numel() != N * Hq * d:
            raise ValueError(f"{name}: gate has {gate.numel()} elements, expected {N * Hq * d}")
    if out is None:
        out = torch.empty(N, Hq, d, dtype=torch.float32, device=dev)
    if N == 0:
        return out
    _prefill_launch(out, q, k_new, v_new, k_pool, v_pool, tables, cu, st, gate, window or 0, True, exact)
    return out


def attention(q, k, v, causal: bool = True, window: int | None = None, exact: bool = False) -> torch.Tensor:
    """Backend.attention for T >= 1 queries (src/backend/base.py:32-35, ops.attention, src/ops.py:65-104):
    q [T, Hq, d], k / v [S, Hkv, d] (fp32 or bf16 read as stored, anything else widened) -> [T, Hq, d] fp32; query i
    sits at position S - T + i. The cache is viewed in place as a pool of one block holding all S positions and run
    through rk_paged_prefill with no KV write; with a window the keys no query sees are dropped first, as the
    reference does. Operands as paged_prefill (fp32 unless q, k and v are all bf16 and exact is False)."""
    name = "attention"
    if q.dim() != 3 or k.dim() != 3 or v.shape != k.shape:
        raise ValueError(f"{name}: q {tuple(q.shape)}, k {tuple(k.shape)}, v {tuple(v.shape)}")
    if window is not None and window < 1:
        raise ValueError(f"window must be at least 1, not {window}")
    T, Hq, d = q.shape
    S, Hkv, dk = k.shape
    if dk != d:
        raise ValueError(f"{name}: q head_dim {d}, k head_dim {dk}")
    if S < T:
        raise ValueError(f"{name}: {T} queries need at least as many keys, got {S}")
    _prefill_shape_check(name, Hq, Hkv, d)
    dev = _need_cuda(name, q, k, v)
    if window is not None and S > T + window - 1:       # older than the first query's window: no query sees them
        k, v = k[S - T - window + 1:], v[S - T - window + 1:]
        S = k.shape[0]
    if k.dtype != v.dtype or k.dtype not in KV_DTYPES:
        k, v = k.float(), v.float()
    q = (q if q.dtype in KV_DTYPES else q.float()).contiguous()
    out = torch.empty(T, Hq, d, dtype=torch.float32, device=dev)
    if T == 0:
        return out
    if S >= 2 ** 31:
        raise NotImplementedError(f"{name}: {S} positions (the kernels address positions below 2^31)")
    # viewed in place as one block of S positions; past 65,535 positions (where the 32-query bf16 kernel's block
    # index needs positions x block size < 2^32) as S / bs blocks of the largest power of two bs <= 16 dividing S, in
    # order (an odd S gives blocks of one position, which the 16-query kernels take)
    bs = S if S < 65536 else math.gcd(S, 16)
    nb = S // bs
    kp, vp = k.contiguous().view(nb, bs, Hkv, d), v.contiguous().view(nb, bs, Hkv, d)
    tables = torch.arange(nb, dtype=torch.int32, device=dev).view(1, nb)
    _prefill_launch(out, q, None, None, kp, vp, tables, [0, T], [S - T], None,
                    (window or 0) if causal else 0, causal, exact)
    return out


DELTA_CHUNK = 64            # tokens per chunk of rk_gated_delta_chunked


def gated_delta_chunked(q, k, v, beta, g, S, cu_seqlens, seq_index=None, out=None) -> torch.Tensor:
    """Chunked gated delta rule over packed sequences (rk_gated_delta_chunked) -> o [N, H, dv] fp32.
    q, k [N, H, dk], v [N, H, dv] (bf16 all three, or anything else, taken as fp32; q already scaled);
    beta, g [N, H]; cu_seqlens: host list / CPU tensor of n_seqs + 1 row offsets (as the packing step produces).
    S: fp32 states, updated in place, indexed along dim 0 (each S[i] a contiguous [H, dk, dv]); sequence i uses
    S[seq_index[i]] (seq_index: device int32 [n_seqs]) or S[i]."""
    name = "gated_delta"
    cu = [int(x) for x in cu_seqlens]
    n_seqs = len(cu) - 1
    if n_seqs < 1 or cu[0] != 0 or any(b < a for a, b in zip(cu, cu[1:])):
        raise ValueError(f"{name}: cu_seqlens {cu[:8]}... must be n_seqs + 1 non-decreasing offsets from 0")
    if q.dim() != 3 or k.shape != q.shape or v.dim() != 3 or v.shape[:2] != q.shape[:2]:
        raise ValueError(f"{name}: q {tuple(q.shape)}, k {tuple(k.shape)}, v {tuple(v.shape)}")
    N, H, dk = q.shape
    dv = v.shape[2]
    if cu[-1] != N or beta.shape != (N, H) or g.shape != (N, H):
        raise ValueError(f"{name}: {N} rows, cu_seqlens end {cu[-1]}, beta {tuple(beta.shape)}, g {tuple(g.shape)}")
    if S.dtype != torch.float32 or S.dim() != 4 or S.shape[1:] != (H, dk, dv) or \
            S.stride()[1:] != (dk * dv, dv, 1):
        raise ValueError(f"{name}: states {tuple(S.shape)} {S.dtype} must be fp32 [n, {H}, {dk}, {dv}] with "
                         "contiguous inner dims")
    if seq_index is None and S.shape[0] < n_seqs:
        raise ValueError(f"{name}: {n_seqs} sequences but {S.shape[0]} states")
    dev = _need_cuda(name, q, k, v, beta, g, S)
    if seq_index is not None:
        _need_cuda(name, seq_index)
        if seq_index.dtype != torch.int32 or seq_index.numel() != n_seqs:
            raise ValueError(f"{name}: seq_index must be int32 [{n_seqs}]")
    if not (q.dtype == k.dtype == v.dtype == torch.bfloat16):
        q, k, v = q.float(), k.float(), v.float()
    # rows are read as 16-byte vectors: a contiguous view at an odd offset is copied to a fresh (aligned) buffer
    q, k, v = (x.contiguous() if x.is_contiguous() and x.data_ptr() % 16 == 0 else x.clone(
        memory_format=torch.contiguous_format) for x in (q, k, v))
    beta, g = beta.to(torch.float32).contiguous(), g.to(torch.float32).contiguous()
    if out is None:
        out = torch.empty(N, H, dv, dtype=torch.float32, device=dev)
    if N == 0:
        return out
    cuc = [0]
    for a, b in zip(cu, cu[1:]):
        cuc.append(cuc[-1] + -(-(b - a) // DELTA_CHUNK))
    meta = to_device(torch.tensor(cu + cuc, dtype=torch.int32), dev)
    lib = load()
    nbytes = lib.lib.rk_gated_delta_workspace_bytes(cuc[-1], H)
    ws = workspace(dev, nbytes)
    lib.call("rk_gated_delta_chunked", out.data_ptr(), S.data_ptr(), S.stride(0), q.data_ptr(), k.data_ptr(),
             v.data_ptr(), DTYPE_CODES[q.dtype], beta.data_ptr(), g.data_ptr(), meta.data_ptr(),
             meta.data_ptr() + 4 * (n_seqs + 1), seq_index.data_ptr() if seq_index is not None else None, n_seqs,
             cuc[-1], H, dk, dv, ws.data_ptr(), ws.numel(), _stream(dev))
    return out


def _rows(t: torch.Tensor) -> torch.Tensor:
    """A 2-D view whose rows are unit-stride (any row stride): kept as is, or copied when the columns are strided."""
    return t if t.stride(1) == 1 else t.contiguous()


def causal_conv1d(x, tail, w) -> tuple[torch.Tensor, torch.Tensor]:
    """Backend.causal_conv1d for one segment (rk_causal_conv1d): x [T, C] (fp32 or bf16 read as stored; rows may be
    strided, as the qkv columns of a fused projection output), tail [K-1, C], w [C, K]
    -> (silu(conv) [T, C] fp32, new tail [K-1, C] fp32). As TorchBackend.causal_conv1d (torch_ref.py:49-50), x is
    taken widened: the fp32 tail is used as stored and the new tail holds x's rows widened."""
    name = "causal_conv1d"
    if x.dim() != 2 or tail.dim() != 2 or w.dim() != 2:
        raise ValueError(f"{name}: x {tuple(x.shape)}, tail {tuple(tail.shape)}, w {tuple(w.shape)}")
    T, C = x.shape
    K = w.shape[1]
    if w.shape[0] != C or tail.shape != (K - 1, C):
        raise ValueError(f"{name}: x [{T}, {C}], tail {tuple(tail.shape)}, w {tuple(w.shape)}")
    dev = _need_cuda(name, x, tail, w)
    if x.dtype not in KV_DTYPES:
        x = x.float()
    x = _rows(x)
    tail = tail.to(device=dev, dtype=torch.float32).contiguous()
    w = w.to(device=dev, dtype=torch.float32).contiguous()
    u = torch.empty(T, C, dtype=torch.float32, device=dev)
    new_tail = torch.empty(K - 1, C, dtype=torch.float32, device=dev)
    load().call("rk_causal_conv1d", u.data_ptr(), new_tail.data_ptr(), x.data_ptr(), DTYPE_CODES[x.dtype],
                x.stride(0), tail.data_ptr(), w.data_ptr(), T, C, K, _stream(dev))
    return u, new_tail


def deltanet_prefill_front(qkv, b, a, conv_state, seq_index, conv_w, A_log, dt_bias, cu_seqlens, dims):
    """Conv + split + l2norm + beta / g for packed segments, with the conv-state update (rk_deltanet_prefill_front)
    -> (q, k [N, H, dk], v [N, H, dv], beta, g [N, H]), all fp32: the inputs of gated_delta_chunked.
    qkv [N, C], b, a [N, H]: fp32 or bf16 (one dtype), rows may be strided (the column slices of the fused in_proj
    output). cu_seqlens: host list of n_seqs + 1 row offsets, or a device int32 tensor of them.
    conv_state: fp32 tails indexed along dim 0 (each [K-1, C] contiguous), segment i uses conv_state[seq_index[i]]
    (seq_index device int32 [n_seqs]) and leaves the new tail there; conv_state None: zero tails, nothing written."""
    name = "deltanet_prefill_front"
    H, dk, dv, key_dim = dims
    if key_dim != H * dk:
        raise ValueError(f"{name}: key_dim {key_dim} != H * dk = {H * dk}")
    N, C = qkv.shape
    if C != 2 * key_dim + H * dv or b.shape != (N, H) or a.shape != (N, H):
        raise ValueError(f"{name}: qkv {tuple(qkv.shape)} (expected {2 * key_dim + H * dv} channels), "
                         f"b {tuple(b.shape)}, a {tuple(a.shape)}")
    K = conv_w.shape[1]
    if conv_w.shape != (C, K):
        raise ValueError(f"{name}: conv_w {tuple(conv_w.shape)}, expected [{C}, K]")
    dev = _need_cuda(name, qkv, b, a)
    if isinstance(cu_seqlens, torch.Tensor) and cu_seqlens.device.type == "cuda":
        cu_dev = cu_seqlens
        if cu_dev.dtype != torch.int32 or cu_dev.dim() != 1:
            raise ValueError(f"{name}: device cu_seqlens must be int32 [n_seqs + 1]")
        n_seqs = cu_dev.numel() - 1
    else:
        cu = [int(x) for x in cu_seqlens]
        if len(cu) < 2 or cu[0] != 0 or cu[-1] != N or any(hi < lo for lo, hi in zip(cu, cu[1:])):
            raise ValueError(f"{name}: cu_seqlens {cu[:8]}... must be non-decreasing offsets from 0 to {N}")
        n_seqs = len(cu) - 1
        cu_dev = to_device(torch.tensor(cu, dtype=torch.int32), dev)
    if conv_state is not None:
        if conv_state.dtype != torch.float32 or conv_state.dim() != 3 or conv_state.shape[1:] != (K - 1, C) or \
                conv_state.stride()[1:] != (C, 1):
            raise ValueError(f"{name}: conv state {tuple(conv_state.shape)} {conv_state.dtype} must be fp32 "
                             f"[n, {K - 1}, {C}] with contiguous inner dims")
        _need_cuda(name, conv_state, seq_index)
        if seq_index.dtype != torch.int32 or seq_index.numel() != n_seqs:
            raise ValueError(f"{name}: seq_index must be int32 [{n_seqs}]")
    if not (qkv.dtype == b.dtype == a.dtype and qkv.dtype in KV_DTYPES):
        qkv, b, a = qkv.float(), b.float(), a.float()
    qkv, b, a = _rows(qkv), _rows(b), _rows(a)
    if not (qkv.stride(0) == b.stride(0) == a.stride(0)) or qkv.stride(0) % 2 or \
            qkv.data_ptr() % (2 * qkv.element_size()):
        packed = torch.cat([qkv, b, a], dim=1)            # one row stride for the three inputs, aligned rows
        if packed.shape[1] % 2:
            packed = torch.nn.functional.pad(packed, (0, 1))
        qkv, b, a = packed[:, :C], packed[:, C:C + H], packed[:, C + H:C + 2 * H]
    f = lambda t: t.to(device=dev, dtype=torch.float32).contiguous()
    conv_w, A_log, dt_bias = f(conv_w), f(A_log), f(dt_bias)
    q = torch.empty(N, H, dk, dtype=torch.float32, device=dev)
    k = torch.empty_like(q)
    v = torch.empty(N, H, dv, dtype=torch.float32, device=dev)
    beta = torch.empty(N, H, dtype=torch.float32, device=dev)
    g = torch.empty_like(beta)
    load().call("rk_deltanet_prefill_front", q.data_ptr(), k.data_ptr(), v.data_ptr(), beta.data_ptr(), g.data_ptr(),
                qkv.data_ptr(), b.data_ptr(), a.data_ptr(), DTYPE_CODES[qkv.dtype], qkv.stride(0),
                conv_state.data_ptr() if conv_state is not None else None,
                conv_state.stride(0) if conv_state is not None else 0, conv_w.data_ptr(), A_log.data_ptr(),
                dt_bias.data_ptr(), cu_dev.data_ptr(), seq_index.data_ptr() if conv_state is not None else None,
                n_seqs, N, H, dk, dv, K, _stream(dev))
    return q, k, v, beta, g


def rms_norm_gated(x, z, w, eps: float, out=None) -> torch.Tensor:
    """Backend.rms_norm_gated (rk_rms_norm_gated): x [rows, dv] -> x * rsqrt(mean(x^2) + eps) * w * silu(z), fp32.
    z [rows, dv], or [rows / G, G * dv] (G heads per row with any row stride: the z columns of a fused projection
    output, without the copy a reshape to [rows, dv] would make); fp32 or bf16 read as stored."""
    name = "rms_norm_gated"
    if x.dim() != 2 or z.dim() != 2:
        raise ValueError(f"{name}: x {tuple(x.shape)}, z {tuple(z.shape)}")
    rows, dv = x.shape
    if z.shape[1] % dv or z.shape[0] * (z.shape[1] // dv) != rows or w.numel() != dv:
        raise ValueError(f"{name}: x {tuple(x.shape)}, z {tuple(z.shape)}, w {tuple(w.shape)}")
    group = z.shape[1] // dv
    dev = _need_cuda(name, x, z)
    per = dv // 64                                        # the kernel's vector width (elements)
    al = lambda t: t.data_ptr() % (per * t.element_size()) == 0
    x = x.to(torch.float32).contiguous()
    if not al(x):
        x = x.clone()
    if z.dtype not in KV_DTYPES:
        z = z.float()
    z = _rows(z)
    if not al(z) or z.stride(0) % per:
        z = z.contiguous() if not z.is_contiguous() else z.clone()
    w = w.to(device=dev, dtype=torch.float32).contiguous()
    if not al(w):
        w = w.clone()
    if out is None:
        out = torch.empty(rows, dv, dtype=torch.float32, device=dev)
    load().call("rk_rms_norm_gated", out.data_ptr(), x.data_ptr(), z.data_ptr(), DTYPE_CODES[z.dtype],
                z.stride(0), group, w.data_ptr(), rows, dv, float(eps), _stream(dev))
    return out


_inv_freq: dict[tuple, torch.Tensor] = {}


def rope_inv_freq(theta: float, rot: int, dev: torch.device) -> torch.Tensor:
    """1 / theta^(i / (rot/2)), computed once in fp32 on the host (as the reference computes it, src/ops.py:27-33:
    the same bits whatever device runs the rotation) and cached on the device."""
    key = (float(theta), int(rot), str(dev))
    t = _inv_freq.get(key)
    if t is None:
        half = rot // 2
        t = (1.0 / (theta ** (torch.arange(0, half, dtype=torch.float32) / half))).to(dev)
        _inv_freq[key] = t
    return t


def attn_prep(y, q_w, k_w, eps: float, positions, theta: float, rot: int, dims, k_pool=None, v_pool=None,
              slots=None):
    """q / k RMSNorm (1 + w weights given), partial RoPE and the KV write of a gated-attention layer (rk_attn_prep).
    y [N, >= (Hq + 2 Hkv) d] (fp32 or bf16; rows may be strided: the fused projection output); positions [N] int32
    (device); dims (Hq, Hkv, d). With k_pool / v_pool (one layer [num_blocks, bs, Hkv, d]) and slots ([N] int64
    device, block * bs + offset) the new K / V rows go into the pool and q [N, Hq, d] fp32 is returned; without,
    (q, k, v) fp32 are returned."""
    name = "attn_prep"
    Hq, Hkv, d = dims
    if y.dim() != 2 or y.shape[1] < (Hq + 2 * Hkv) * d or q_w.numel() != d or k_w.numel() != d:
        raise ValueError(f"{name}: y {tuple(y.shape)}, norm weights {q_w.numel()} / {k_w.numel()} for {dims}")
    if not 0 <= rot <= d:
        raise ValueError(f"{name}: rotary dims {rot} of {d}")
    N = y.shape[0]
    dev = _need_cuda(name, y, positions)
    if positions.dtype != torch.int32 or positions.numel() != N:
        raise ValueError(f"{name}: positions must be int32 [{N}]")
    if y.dtype not in KV_DTYPES:
        y = y.float()
    y = _rows(y)
    if y.data_ptr() % (d // 64 * y.element_size()) or y.stride(0) % (d // 64):
        y = y.contiguous() if not y.is_contiguous() else y.clone()
    f = lambda t: t.to(device=dev, dtype=torch.float32).contiguous()
    q_w, k_w = f(q_w), f(k_w)
    inv = rope_inv_freq(theta, rot, dev) if rot else None
    q = torch.empty(N, Hq, d, dtype=torch.float32, device=dev)
    lib = load()
    common = (y.data_ptr(), DTYPE_CODES[y.dtype], y.stride(0), q_w.data_ptr(), k_w.data_ptr(), float(eps),
              positions.data_ptr(), inv.data_ptr() if inv is not None else None, int(rot), N, Hq, Hkv, d, _stream(dev))
    if k_pool is None:
        k = torch.empty(N, Hkv, d, dtype=torch.float32, device=dev)
        v = torch.empty_like(k)
        lib.call("rk_attn_prep", q.data_ptr(), k.data_ptr(), v.data_ptr(), None, None, RK_F32, None, 0, 0, *common)
        return q, k, v
    if k_pool.dtype != v_pool.dtype or k_pool.dtype not in KV_DTYPES:
        raise TypeError(f"{name}: keys and values must both be float32 or bfloat16, not "
                        f"{k_pool.dtype} / {v_pool.dtype}")
    if k_pool.dim() != 4 or k_pool.shape != v_pool.shape or k_pool.shape[2:] != (Hkv, d):
        raise ValueError(f"{name}: pools {tuple(k_pool.shape)} / {tuple(v_pool.shape)} for {dims}")
    _need_cuda(name, k_pool, v_pool, slots)
    _contig(name, k_pool, "k_pool"); _contig(name, v_pool, "v_pool")
    if slots.dtype != torch.int64 or slots.numel() != N:
        raise ValueError(f"{name}: slots must be int64 [{N}]")
    lib.call("rk_attn_prep", q.data_ptr(), None, None, k_pool.data_ptr(), v_pool.data_ptr(),
             DTYPE_CODES[k_pool.dtype], slots.contiguous().data_ptr(), k_pool.shape[0], k_pool.shape[1], *common)
    return q


W_TYPES = {"int8": RK_W_INT8, "int4": RK_W_INT4}
LINEAR_ROWS = 16            # activation rows per rk_linear_rows launch (the MFMA's 16 columns)
KERNEL_ROWS = 32            # up to here: the matvec kernel in groups of 16; beyond: dequantize + GEMM
LINEAR_LONG_ROWS = 65536    # rk_linear_rows' persistent kernel for INT8 weights from this many rows (M <= 8)


def _weight_args(w):
    """(w_type, data, scales, mins, N, K) of a bf16 tensor or a QuantTensor, checked."""
    from quant import QuantTensor
    if isinstance(w, QuantTensor):
        if w.scheme not in W_TYPES or w.block != 32:
            raise TypeError(f"linear: quantized scheme {w.scheme} / block {w.block} has no kernel")
        N, K = w.shape
        if w.data.dtype != (torch.int8 if w.scheme == "int8" else torch.uint8) or \
                w.data.shape != (N, K if w.scheme == "int8" else K // 2) or w.scales.shape != (N, K // 32) or \
                w.scales.dtype != torch.float16 or \
                (w.scheme == "int4" and (w.mins is None or w.mins.shape != (N, K // 32))):
            raise ValueError(f"linear: malformed {w.scheme} weight {tuple(w.data.shape)} / {tuple(w.scales.shape)}")
        for t in (w.data, w.scales) + ((w.mins,) if w.mins is not None else ()):
            _contig("linear", t, "quantized weight parts")
        return W_TYPES[w.scheme], w.data, w.scales, w.mins, N, K
    if w.dtype != torch.bfloat16 or w.dim() != 2:
        raise TypeError(f"linear: weight dtype {w.dtype} has no matvec kernel (bf16 or quantized)")
    _contig("linear", w, "w")
    return RK_W_BF16, w, None, None, w.shape[0], w.shape[1]


def linear_rows(x, w, bias=None, residual=None, out=None) -> torch.Tensor:
    """y [M, N] = x [M, K] @ dequant(w)^T (+ bias) (+ residual), fp32, for M <= KERNEL_ROWS (rk_linear_rows, 16 rows
    per launch): the decode-time linear of src/backend/metal.py:59-133. w: bf16 [N, K] or a QuantTensor."""
    wt, data, scales, mins, N, K = _weight_args(w)
    M = x.shape[0]
    if x.dim() != 2 or x.shape[1] != K or M > KERNEL_ROWS or K % 32:
        raise ValueError(f"linear: x {tuple(x.shape)} for a [{N}, {K}] weight (M <= {KERNEL_ROWS}, K % 32 == 0)")
    dev = _need_cuda("linear", x, data)
    x = x.to(torch.float32).contiguous()
    if x.data_ptr() % 16:
        x = x.clone()
    if bias is not None:
        bias = bias.to(device=dev, dtype=torch.float32).contiguous()
    if residual is not None:
        residual = residual.to(device=dev, dtype=torch.float32).contiguous()
        if residual.shape != (M, N):
            raise ValueError(f"linear: residual {tuple(residual.shape)}, expected [{M}, {N}]")
    if out is None:
        out = torch.empty(M, N, dtype=torch.float32, device=dev)
    lib = load()
    cnt = linear_counters(dev, -(-N // 16))
    for m0 in range(0, M, LINEAR_ROWS):
        m = min(LINEAR_ROWS, M - m0)
        need = lib.lib.rk_linear_workspace_bytes(m, N, K, wt)
        part = workspace(dev, need) if need else None
        lib.call("rk_linear_rows", out[m0:].data_ptr(), x[m0:].data_ptr(), m, N, K, data.data_ptr(), wt,
                 scales.data_ptr() if scales is not None else None, mins.data_ptr() if mins is not None else None,
                 bias.data_ptr() if bias is not None else None,
                 residual[m0:].data_ptr() if residual is not None else None,
                 part.data_ptr() if part is not None else None, part.numel() if part is not None else 0,
                 cnt.data_ptr(), cnt.numel(), _stream(dev))
    return out



def _ex2(x, x_ld: int, w, x_op: int, aux=None, aux_ld: int = 0, norm_w=None, eps: float = 0.0, bias=None,
         residual=None, want_ss: bool = False):
    """One rk_linear_rows_ex2 launch over M <= 16 rows: y [M, N] fp32 and, with want_ss, the sums of squares of
    y's 16-column tiles [M, ceil(N / 16)] (else None)."""
    wt, data, scales, mins, N, K = _weight_args(w)
    M = x.shape[0]
    dev = x.device
    if bias is not None:
        bias = bias.to(device=dev, dtype=torch.float32).contiguous()
    if residual is not None:
        residual = residual.to(device=dev, dtype=torch.float32).contiguous()
        if residual.shape != (M, N):
            raise ValueError(f"linear: residual {tuple(residual.shape)}, expected [{M}, {N}]")
    out = torch.empty(M, N, dtype=torch.float32, device=dev)
    ss = torch.empty(M, -(-N // 16), dtype=torch.float32, device=dev) if want_ss else None
    lib = load()
    cnt = linear_counters(dev, -(-N // 16))
    need = lib.lib.rk_linear_workspace_bytes(M, N, K, wt)
    part = workspace(dev, need) if need else None
    lib.call("rk_linear_rows_ex2", out.data_ptr(), ss.data_ptr() if ss is not None else None, x.data_ptr(), x_ld,
             x_op, aux.data_ptr() if aux is not None else None, aux_ld,
             norm_w.data_ptr() if norm_w is not None else None, float(eps), M, N, K, data.data_ptr(), wt,
             scales.data_ptr() if scales is not None else None, mins.data_ptr() if mins is not None else None,
             bias.data_ptr() if bias is not None else None, residual.data_ptr() if residual is not None else None,
             part.data_ptr() if part is not None else None, part.numel() if part is not None else 0, cnt.data_ptr(),
             cnt.numel(), _stream(dev))
    return out, ss


def _rows_k(t, K: int):
    """fp32 rows with unit column stride, 16-byte aligned, at a row stride >= K of 4n (a copy when not)."""
    t = t.to(torch.float32)
    if t.stride(1) != 1 or t.stride(0) % 4 or t.data_ptr() % 16 or (t.shape[0] > 1 and t.stride(0) < K):
        t = t.contiguous() if not t.is_contiguous() else t.clone()
    return t, (t.stride(0) if t.shape[0] > 1 else K)


def linear_ss(x, w, bias=None, residual=None):
    """linear(x, w, bias, residual) -> (y, ss): with up to 16 rows (rk_linear_rows_ex2) also the sums of squares of
    y's 16-column tiles [M, ceil(N / 16)], which let the RMSNorm before the next linear run inside it
    (rms_norm_linear); beyond 16 rows (or K % 32 != 0) the plain linear and ss = None."""
    wt, data, scales, mins, N, K = _weight_args(w)
    M = x.shape[0]
    if x.dim() != 2 or x.shape[1] != K or M > LINEAR_ROWS or K % 32:
        return linear(x, w, bias, residual), None
    _need_cuda("linear", x, data)
    xr, ld = _rows_k(x, K)
    from native.rocm_native import RK_X_PLAIN
    return _ex2(xr, ld, w, RK_X_PLAIN, bias=bias, residual=residual, want_ss=True)


def silu_mul_linear_ss(gate, up, w, bias=None, residual=None):
    """silu_mul_linear -> (y, ss) like linear_ss: one launch with the sums of squares of y's 16-column tiles where
    the fused kernel covers the shapes, else (silu_mul_linear(...), None)."""
    wt, data, scales, mins, N, K = _weight_args(w)
    M = gate.shape[0]
    if gate.dim() != 2 or gate.shape[1] != K or up.shape != gate.shape or M > 8 or K % 256:
        return silu_mul_linear(gate, up, w, bias, residual), None
    _need_cuda("linear", gate, up, data)
    g, g_ld = _rows_k(gate, K)
    u, u_ld = _rows_k(up, K)
    from native.rocm_native import RK_X_SILU_MUL
    return _ex2(g, g_ld, w, RK_X_SILU_MUL, aux=u, aux_ld=u_ld, bias=bias, residual=residual, want_ss=True)


def rms_norm_linear(x, ss, norm_w, eps: float, w, bias=None, residual=None) -> torch.Tensor:
    """linear(rms_norm(x, norm_w, eps), w, bias, residual) with the norm applied while rk_linear_rows_ex2 stages x
    (one launch), from ss = the sums of squares of x's 16-column tiles that the linear producing x wrote
    (linear_ss / silu_mul_linear_ss). Without ss, beyond 8 rows, K % 256 != 0 or K > 2048, and for long matrices
    (N > 16384 outside the persistent INT8 kernel's shapes: every workgroup recomputes the rows' rms, which costs
    more than the separate launch there):
    rms_norm, then linear (the same results within 1e-5)."""
    wt, data, scales, mins, N, K = _weight_args(w)
    M = x.shape[0]
    long_int8 = wt == RK_W_INT8 and N >= LINEAR_LONG_ROWS and K % 1024 == 0      # the persistent kernel's shapes
    if (ss is None or x.dim() != 2 or x.shape[1] != K or M > 8 or K % 256 or K > 2048 or (N > 16384 and not long_int8)
            or ss.shape != (M, K // 16) or norm_w.numel() != K):
        return linear(rms_norm(x, norm_w, eps), w, bias, residual)
    _need_cuda("linear", x, ss, norm_w, data)
    xr, ld = _rows_k(x, K)
    nw = norm_w.to(torch.float32).contiguous()
    if nw.data_ptr() % 16:
        nw = nw.clone()
    ssr = ss.to(torch.float32).contiguous()
    from native.rocm_native import RK_X_RMS_NORM
    y, _ = _ex2(xr, ld, w, RK_X_RMS_NORM, aux=ssr, aux_ld=ssr.stride(0), norm_w=nw, eps=eps, bias=bias,
                residual=residual)
    return y

def _swiglu_launch(x, x_ld: int, w, x_op: int, aux=None, aux_ld: int = 0, norm_w=None, eps: float = 0.0):
    """One rk_swiglu_rows launch over M <= 16 rows of x (fp32, row stride x_ld) and w = [gate; up] -> [M, F]."""
    wt, data, scales, mins, N, K = _weight_args(w)
    M, F = x.shape[0], N // 2
    dev = x.device
    out = torch.empty(M, F, dtype=torch.float32, device=dev)
    lib = load()
    cnt = linear_counters(dev, -(-N // 16))
    need = lib.lib.rk_linear_workspace_bytes(M, N, K, wt)
    part = workspace(dev, need) if need else None
    lib.call("rk_swiglu_rows", out.data_ptr(), x.data_ptr(), x_ld, x_op, aux.data_ptr() if aux is not None else None,
             aux_ld, norm_w.data_ptr() if norm_w is not None else None, float(eps), M, F, K, data.data_ptr(), wt,
             scales.data_ptr() if scales is not None else None, mins.data_ptr() if mins is not None else None,
             part.data_ptr() if part is not None else None, part.numel() if part is not None else 0, cnt.data_ptr(),
             cnt.numel(), _stream(dev))
    return out


def _swiglu_fused(w, K: int) -> bool:
    """Whether rk_swiglu_rows covers a [2F, K] weight: F a multiple of 8, K of 32."""
    wt, data, scales, mins, N, Kw = _weight_args(w)
    return N % 16 == 0 and K == Kw and K % 32 == 0


def swiglu(x, w) -> torch.Tensor:
    """Backend.swiglu (src/backend/base.py:40-41): silu(x @ gate^T) * (x @ up^T) for w = [gate; up] stacked [2F, K]
    (bf16 or a QuantTensor) -> [M, F] fp32. Up to KERNEL_ROWS rows: rk_swiglu_rows, one launch per 16 rows (the
    linear's sums, then silu * up on each gate / up pair in the same launch); beyond that, or for F % 8 != 0, the
    linear and then silu_mul on its two halves (the same results within 1e-5)."""
    N, K = w.shape
    M = x.shape[0]
    if x.dim() != 2 or x.shape[1] != K or N % 2:
        raise ValueError(f"swiglu: x {tuple(x.shape)} for a [{N}, {K}] stacked [gate; up] weight")
    from quant import QuantTensor
    if M > KERNEL_ROWS or not (isinstance(w, QuantTensor) or w.dtype == torch.bfloat16) or not _swiglu_fused(w, K):
        y = linear(x, w)
        return silu_mul(y[:, :N // 2], y[:, N // 2:])
    _need_cuda("swiglu", x, w.data if isinstance(w, QuantTensor) else w)
    xr, ld = _rows_k(x, K)
    from native.rocm_native import RK_X_PLAIN
    if M <= LINEAR_ROWS:
        return _swiglu_launch(xr, ld, w, RK_X_PLAIN)
    return torch.cat([_swiglu_launch(xr[m0:m0 + LINEAR_ROWS], ld, w, RK_X_PLAIN) for m0 in range(0, M, LINEAR_ROWS)])


def rms_norm_swiglu(x, ss, norm_w, eps: float, w) -> torch.Tensor:
    """swiglu(rms_norm(x, norm_w, eps), w) in one launch (rk_swiglu_rows with the RMSNorm input transform), from
    ss = the sums of squares of x's 16-column tiles that the linear producing x wrote; the cases rms_norm_linear
    sends to the separate norm (no ss, more than 8 rows, K % 256 != 0 or K > 2048, more than 16384 weight rows)
    and the weights swiglu does not fuse: rms_norm, then swiglu (the same results within 1e-5)."""
    N, K = w.shape
    M = x.shape[0]
    from quant import QuantTensor
    if (ss is None or x.dim() != 2 or x.shape[1] != K or M > 8 or K % 256 or K > 2048 or N > 16384
            or ss.shape != (M, K // 16) or norm_w.numel() != K
            or not (isinstance(w, QuantTensor) or w.dtype == torch.bfloat16) or not _swiglu_fused(w, K)):
        return swiglu(rms_norm(x, norm_w, eps), w)
    _need_cuda("swiglu", x, ss, norm_w, w.data if isinstance(w, QuantTensor) else w)
    xr, ld = _rows_k(x, K)
    nw = norm_w.to(torch.float32).contiguous()
    if nw.data_ptr() % 16:
        nw = nw.clone()
    ssr = ss.to(torch.float32).contiguous()
    from native.rocm_native import RK_X_RMS_NORM
    return _swiglu_launch(xr, ld, w, RK_X_RMS_NORM, aux=ssr, aux_ld=ssr.stride(0), norm_w=nw, eps=eps)


_linear_cnt: dict[int, torch.Tensor] = {}


def linear_counters(dev: torch.device, n: int) -> torch.Tensor:
    """The arrival counters of rk_linear_rows (per row block) and rk_paged_prefill (per split block, kv-head and
    head) on dev: zero-filled when (re)allocated, and every call of either leaves them at zero, so one buffer serves
    all stream-ordered calls."""
    idx = dev.index if dev.index is not None else torch.cuda.current_device()
    buf = _linear_cnt.get(idx)
    if buf is None or buf.numel() < n:
        if buf is not None:
            _retired.append(buf)                               # see _retired: a captured graph may still use it
        grow = 2 * buf.numel() if buf is not None else 0
        buf = torch.zeros(max(n, 1 << 14, grow), dtype=torch.int32, device=dev)
        _linear_cnt[idx] = buf
    return buf


def dequantize(w, rows=None, row0: int = 0, n_rows: int | None = None) -> torch.Tensor:
    """Rows of a bf16 / quantized weight as fp32 [n, K] (rk_dequant_rows; bit-exact with the reference's
    dequantize, src/quant.py:45-56): the given row indices (device int64 / int32 tensor) or rows row0 .. row0+n-1."""
    wt, data, scales, mins, N, K = _weight_args(w)
    dev = _need_cuda("dequantize", data)
    if rows is not None:
        rows = rows.to(device=dev, dtype=torch.int32).contiguous()
        n = rows.numel()
    else:
        n = N - row0 if n_rows is None else n_rows
    out = torch.empty(n, K, dtype=torch.float32, device=dev)
    load().call("rk_dequant_rows", out.data_ptr(), data.data_ptr(), wt,
                scales.data_ptr() if scales is not None else None, mins.data_ptr() if mins is not None else None,
                rows.data_ptr() if rows is not None else None, row0, n, N, K, _stream(dev))
    return out


DEQUANT_CHUNK = 1 << 23     # weights expanded per prefill GEMM piece (32 MB fp32), as the reference


def linear(x, w, bias=None, residual=None) -> torch.Tensor:
    """The reference's decode / prefill linear on a bf16 or quantized weight (src/backend/metal.py:59-133): up to 32
    rows through the matvec kernel, beyond that an fp32 GEMM (the ROCm BLAS through torch) on row chunks of the
    dequantized weight, so the full-size fp32 weight never exists. fp32 / other-dtype weights: x @ w.T in fp32."""
    from quant import QuantTensor
    M = x.shape[0]
    if not isinstance(w, QuantTensor) and w.dtype != torch.bfloat16:
        y = x.float() @ w.float().T
    elif M <= KERNEL_ROWS and w.shape[1] % 32 == 0:
        return linear_rows(x, w, bias, residual)
    else:
        N, K = w.shape
        x = x.float()
        y = torch.empty(M, N, dtype=torch.float32, device=x.device)
        step = max(1, DEQUANT_CHUNK // K)
        for r in range(0, N, step):
            n = min(step, N - r)
            if isinstance(w, QuantTensor) or K % 32 == 0:
                wr = dequantize(w, row0=r, n_rows=n)
            else:
                wr = w[r:r + n].float()
            y[:, r:r + n] = x @ wr.T
    if bias is not None:
        y = y + bias.float()
    return y + residual.float() if residual is not None else y


def _norm(entry: str, x, w, eps: float) -> torch.Tensor:
    """Rows of any length D: up to 4096 values (a multiple of 4, aligned) stay in registers, one wave per row; any
    other row takes a workgroup of its own (rk_rms_norm / rk_layer_norm choose)."""
    name = entry[3:]
    D = x.shape[-1]
    if w.numel() != D or D < 1:
        raise ValueError(f"{name}: x {tuple(x.shape)}, w {tuple(w.shape)}")
    dev = _need_cuda(name, x)
    shape = x.shape
    if x.dtype not in KV_DTYPES:
        x = x.float()
    x = x.reshape(-1, D)
    if x.stride(1) != 1:
        x = x.contiguous()
    if w.dtype not in KV_DTYPES:
        w = w.float()
    w = w.to(dev).contiguous()
    rows = x.shape[0]
    out = torch.empty(rows, D, dtype=torch.float32, device=dev)
    load().call(entry, out.data_ptr(), x.data_ptr(), DTYPE_CODES[x.dtype], x.stride(0), w.data_ptr(),
                DTYPE_CODES[w.dtype], rows, D, float(eps), _stream(dev))
    return out.view(shape)


def rms_norm(x, w, eps: float) -> torch.Tensor:
    """Backend.rms_norm (rk_rms_norm): [..., D] -> (x / sqrt(mean(x^2) + eps)) * w in fp32 (src/ops.py:7-15); x fp32
    or bf16 read as stored, rows may be strided; w fp32 or bf16."""
    return _norm("rk_rms_norm", x, w, eps)


def layer_norm(x, w, eps: float) -> torch.Tensor:
    """Backend.layer_norm (rk_layer_norm): LayerNorm without bias, w * ((x - mean) * rsqrt(var + eps)) in fp32
    (src/ops.py:18-24)."""
    return _norm("rk_layer_norm", x, w, eps)


def rope(x, positions, theta: float) -> torch.Tensor:
    """Backend.rope (rk_rope): x [T, H, d] rotated by positions [T] over the pairs (i, i + d/2), fp32 out
    (src/ops.py:36-54), with the host-computed fp32 inv_freq of the reference (rope_inv_freq)."""
    if x.dim() != 3 or x.shape[-1] % 2 or positions.numel() != x.shape[0]:
        raise ValueError(f"rope: x {tuple(x.shape)}, positions {tuple(positions.shape)}")
    T, H, d = x.shape
    dev = _need_cuda("rope", x)
    x = x.to(torch.float32).contiguous()
    pos = positions.to(device=dev, dtype=torch.int32).contiguous()
    out = torch.empty_like(x)
    load().call("rk_rope", out.data_ptr(), x.data_ptr(), pos.data_ptr(), rope_inv_freq(theta, d, dev).data_ptr(),
                T, H, d, _stream(dev))
    return out


def silu_mul(gate, up) -> torch.Tensor:
    """Backend.silu_mul (rk_silu_mul): (g / (1 + exp(-g))) * u in fp32 (src/ops.py:107-110). 2-D gate / up may be
    strided row views (the two halves of one projection output are read in place)."""
    if gate.shape != up.shape:
        raise ValueError(f"silu_mul: gate {tuple(gate.shape)}, up {tuple(up.shape)}")
    dev = _need_cuda("silu_mul", gate, up)
    shape = gate.shape
    F = shape[-1] if gate.dim() else 1

    def rows2(t):
        t = t.to(torch.float32)
        t = t.reshape(-1, F) if t.dim() != 2 else t
        return t if t.stride(1) == 1 else t.contiguous()

    g, u = rows2(gate), rows2(up)
    out = torch.empty(g.shape[0], F, dtype=torch.float32, device=dev)
    load().call("rk_silu_mul", out.data_ptr(), g.data_ptr(), g.stride(0), u.data_ptr(), u.stride(0), g.shape[0], F,
                _stream(dev))
    return out.view(shape)


def silu_mul_linear(gate, up, w, bias=None, residual=None) -> torch.Tensor:
    """linear(silu_mul(gate, up), w, bias, residual) with silu * up applied while rk_linear_rows_ex stages the
    activations (one launch). gate / up may be strided row views (the halves of one gate_up output). Outside what
    the fused kernel covers (more than 8 rows, K not a multiple of 256) silu_mul runs as its own kernel first: the
    same results within 1e-5."""
    from native.rocm_native import RK_X_SILU_MUL
    wt, data, scales, mins, N, K = _weight_args(w)
    M = gate.shape[0]
    if gate.dim() != 2 or gate.shape[1] != K or up.shape != gate.shape:
        raise ValueError(f"linear: gate {tuple(gate.shape)}, up {tuple(up.shape)} for a [{N}, {K}] weight")
    if M > 8 or K % 256:
        return linear(silu_mul(gate, up), w, bias, residual)
    dev = _need_cuda("linear", gate, up, data)

    def rows(t):
        t = t.to(torch.float32)
        if t.stride(1) != 1 or t.stride(0) % 4 or t.data_ptr() % 16 or (t.shape[0] > 1 and t.stride(0) < K):
            t = t.contiguous() if not t.is_contiguous() else t.clone()
        return t
    g, u = rows(gate), rows(up)
    g_ld = g.stride(0) if M > 1 else K
    u_ld = u.stride(0) if M > 1 else K
    if bias is not None:
        bias = bias.to(device=dev, dtype=torch.float32).contiguous()
    if residual is not None:
        residual = residual.to(device=dev, dtype=torch.float32).contiguous()
        if residual.shape != (M, N):
            raise ValueError(f"linear: residual {tuple(residual.shape)}, expected [{M}, {N}]")
    out = torch.empty(M, N, dtype=torch.float32, device=dev)
    lib = load()
    cnt = linear_counters(dev, -(-N // 16))
    need = lib.lib.rk_linear_workspace_bytes(M, N, K, wt)
    part = workspace(dev, need) if need else None
    lib.call("rk_linear_rows_ex", out.data_ptr(), g.data_ptr(), g_ld, RK_X_SILU_MUL, u.data_ptr(), u_ld, M, N, K,
             data.data_ptr(), wt, scales.data_ptr() if scales is not None else None,
             mins.data_ptr() if mins is not None else None, bias.data_ptr() if bias is not None else None,
             residual.data_ptr() if residual is not None else None, part.data_ptr() if part is not None else None,
             part.numel() if part is not None else 0, cnt.data_ptr(), cnt.numel(), _stream(dev))
    return out
