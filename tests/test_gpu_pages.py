"""The device page table (rk_pages_*, pages.DevicePages) against its CPU model (oracle/pages_ref.py, the reference's
BlockAllocator / PagedSequence / batch_layout semantics): random schedules of batched growth (decode steps and
prefill chunks) and releases, compared entry for entry after every operation -- tables, lengths, free stack, write
slots, status; a decode loop whose layouts come from the device (KV written through the slots, attention over the
gathered tables) against the oracle's attention over the written history; and the same step captured once in a HIP
graph and replayed, each replay advancing the batch, bit-identical to the eager steps."""
import random

import pytest
import torch

from helpers import rel_err
from oracle.pages_ref import PagesModel

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def assert_same(pages, model):
    torch.cuda.synchronize()
    lens = pages.lens.cpu().tolist()
    assert lens == model.lens
    tab = pages.tables.cpu().tolist()
    for r in range(model.max_seqs):
        held = -(-lens[r] // model.bs)
        assert tab[r][:held] == model.tables[r], f"row {r}"
    free = pages.free_blocks()
    assert free == len(model.free)
    assert pages.stack[:free].cpu().tolist() == model.free
    assert pages.status() == model.status


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_random_schedule_matches_the_model(seed):
    from pages import DevicePages
    rnd = random.Random(seed)
    NB, S, MB, bs = 70, 12, 24, 4
    pages, model = DevicePages(NB, S, MB, bs, DEV), PagesModel(NB, S, MB, bs)
    assert_same(pages, model)
    for it in range(150):
        op = rnd.random()
        rows = rnd.sample(range(S), rnd.randint(1, S))
        if op < 0.8:
            n_new = rnd.choice([1, 1, 1, 2, 5, 13])
            want = model.advance(rows, n_new)
            slots, lens = pages.advance(torch.tensor(rows, dtype=torch.int32), n_new)
            if want is None:
                assert slots.cpu().tolist() == [-1] * len(slots)
            else:
                assert slots.cpu().tolist() == want[0] and lens.cpu().tolist() == want[1]
            width = rnd.choice([MB, 7])
            got_t = pages.tables_for(torch.tensor(rows, dtype=torch.int32), width).cpu().tolist()
            assert got_t == model.table_rows(rows, width)
        else:
            model.release(rows)
            pages.release(torch.tensor(rows, dtype=torch.int32))
        assert_same(pages, model)
        if model.status:
            model.status = 0
            with pytest.raises(Exception):
                pages.check()
            assert pages.status() == 0


def test_out_of_blocks_and_bad_rows_change_nothing():
    from pages import DevicePages, OutOfBlocks
    pages, model = DevicePages(5, 4, 10, 2, DEV), PagesModel(5, 4, 10, 2)
    pages.advance([0, 1], 4)
    model.advance([0, 1], 4)
    assert_same(pages, model)
    slots, lens = pages.advance([2, 3], 3)                   # needs 4 blocks, 1 free
    assert model.advance([2, 3], 3) is None
    assert slots.cpu().tolist() == [-1] * 6 and lens.cpu().tolist() == [0, 0]
    assert_same(pages, model)
    with pytest.raises(OutOfBlocks):
        pages.check()
    model.status = 0
    pages.advance(torch.tensor([1, 7], dtype=torch.int32), 1)    # row 7 is outside the table
    assert model.advance([1, 7], 1) is None and model.status == 4
    assert_same(pages, model)
    with pytest.raises(RuntimeError):
        pages.check()
    pages.release(torch.tensor([-1], dtype=torch.int32))
    torch.cuda.synchronize()
    assert pages.status() == 4
    pages.meta[1].zero_()
    # a row named twice in one call: a double allocation or a double free (BlockAllocator.free refuses the latter,
    # src/state.py:94-99): refused with status 5, nothing taken or returned
    model.status = 0
    slots, lens = pages.advance(torch.tensor([1, 2, 1], dtype=torch.int32), 2)
    assert model.advance([1, 2, 1], 2) is None and model.status == 5
    assert slots.cpu().tolist() == [-1] * 6
    assert_same(pages, model)
    with pytest.raises(RuntimeError, match="twice"):
        pages.check()
    model.status = 0
    pages.release(torch.tensor([0, 0], dtype=torch.int32))
    model.release([0, 0])
    assert model.status == 5
    assert_same(pages, model)
    with pytest.raises(RuntimeError, match="twice"):
        pages.check()


def _decode_setup(B=6, Hq=8, Hkv=2, d=128, bs=16, NB=400, S=10, seed=3):
    from pages import DevicePages
    g = torch.Generator().manual_seed(seed)
    pages = DevicePages(NB, S, 64, bs, DEV)
    rows = torch.tensor([7, 0, 3, 9, 1, 5][:B], dtype=torch.int32, device=DEV)
    hist = [random.Random(seed + i).randint(1, 300) for i in range(B)]
    k_pool = torch.zeros(NB, bs, Hkv, d, dtype=torch.bfloat16, device=DEV)
    v_pool = torch.zeros_like(k_pool)
    return pages, rows, hist, k_pool, v_pool, g


def test_decode_loop_on_device_layouts(backend):
    """Prefill each sequence's history through advance + kv_write (one chunk per sequence), then decode steps:
    advance(rows, 1) -> kv_write(slots) -> paged_attention(tables_for(rows), lens); every step's output against the
    oracle's attention over the history as stored (bf16)."""
    from native import kernels
    from oracle import ops_ref
    pages, rows, hist, k_pool, v_pool, g = _decode_setup()
    B, Hkv, d = rows.numel(), 2, 128
    K = [torch.randn(n + 40, Hkv, d, generator=g).to(torch.bfloat16) for n in hist]
    V = [torch.randn(n + 40, Hkv, d, generator=g).to(torch.bfloat16) for n in hist]
    for b in range(B):
        slots, _ = pages.advance(rows[b:b + 1], hist[b])
        kernels.kv_write(k_pool, v_pool, slots, K[b][:hist[b]].to(DEV), V[b][:hist[b]].to(DEV))
    for step in range(40):
        slots, lens = pages.advance(rows, 1)
        kn = torch.stack([K[b][hist[b] + step] for b in range(B)]).to(DEV)
        vn = torch.stack([V[b][hist[b] + step] for b in range(B)]).to(DEV)
        kernels.kv_write(k_pool, v_pool, slots, kn, vn)
        tables = pages.tables_for(rows)
        q = torch.randn(B, 8, d, generator=g)
        out = backend.paged_attention(q.to(DEV), k_pool, v_pool, tables, lens, 16)
        if step % 13 == 0 or step == 39:
            n = [hist[b] + step + 1 for b in range(B)]
            want = torch.cat([ops_ref.attention(q[b:b + 1], K[b][:n[b]].float(), V[b][:n[b]].float())
                              for b in range(B)])
            assert rel_err(out, want) < 1e-5, f"step {step}"
    pages.check()


def test_graph_replays_advance_the_batch(backend):
    """advance -> kv_write -> paged_attention captured once; ten replays equal ten eager steps on a twin state."""
    from native import kernels
    pages, rows, hist, k_pool, v_pool, g = _decode_setup(seed=5)
    twin, _, _, k2, v2, _ = _decode_setup(seed=5)
    B = rows.numel()
    for p in (pages, twin):
        for b in range(B):
            p.advance(rows[b:b + 1], hist[b])
    kn = torch.randn(B, 2, 128, generator=g).to(DEV)
    q = torch.randn(B, 8, 128, generator=g).to(DEV)
    slots = torch.empty(B, dtype=torch.int64, device=DEV)
    lens = torch.empty(B, dtype=torch.int32, device=DEV)
    tables = torch.empty(B, 64, dtype=torch.int32, device=DEV)

    def step(p, kp, vp):
        p.advance(rows, 1, slots, lens)
        kernels.kv_write(kp, vp, slots, kn, kn)
        p.tables_for(rows, out=tables)
        return backend.paged_attention(q, kp, vp, tables, lens, 16)

    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        out = step(pages, k_pool, v_pool)
    torch.cuda.synchronize()
    for rep in range(10):
        graph.replay()
        torch.cuda.synchronize()
        got = out.clone()
        want = step(twin, k2, v2).clone()
        torch.cuda.synchronize()
        assert torch.equal(got, want), f"replay {rep}"
    assert torch.equal(pages.tables, twin.tables) and torch.equal(pages.lens, twin.lens)
    assert torch.equal(k_pool, k2)
