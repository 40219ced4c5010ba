"""GPU checks of the device-resident block allocator and decode-step
metadata against the oracle's pure-Python restatement of the reference's
block manager and slot rule (oracle.BlockManager, oracle.slot_for_position:
paged_cache_runtime.rs:217-371, paged_kv_cache.rs:74-103; pinned by the
reference's KATs in tests/test_oracle.py, and equal to the library's host
block manager there).

A batch is admitted (prompt blocks, row by row), then decoded step by step
while rows finish (trim to their tokens, or free) and the pool runs dry (rows
stall, as try_allocate_slots fails); after every call the device block
tables, block counts, slots, context lengths and free count must equal the
host's, and replaying the step from a captured HIP graph must do the same."""

import numpy as np
import pytest
import torch

import vpa
from oracle import oracle as orc

pytestmark = pytest.mark.gpu


def u32(a, device):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.uint32)).to(device)


def host_step(mgr, rids, pos, finished, bs, num_blocks):
    """The reference's decode step for rows in order (paged_batch_engine.rs:
    629-639, paged_kv_cache.rs:924-1059): grow by the block the next token
    needs (try_allocate_slots), then slot / context of that token."""
    slots, ctx = [], []
    for r, rid in enumerate(rids):
        if finished[r] or not mgr.try_allocate_slots(rid, pos[r] + 1):
            slots.append(-1)
            ctx.append(1)
            continue
        table = mgr.block_ids(rid)
        slots.append(orc.slot_for_position(table, bs, num_blocks, pos[r]))
        ctx.append(pos[r] + 1)
        pos[r] += 1
    return np.array(slots, np.int64), np.array(ctx, np.uint32)


def check_same(alloc, mgr, rids, device_note):
    bt = alloc.block_tables.cpu().numpy()
    nb = alloc.row_blocks.cpu().numpy()
    for r, rid in enumerate(rids):
        ids = mgr.block_ids(rid) if mgr.blocks_for_request(rid) > 0 else []
        assert nb[r] == len(ids), f"{device_note}: row {r} holds {nb[r]} blocks, host {len(ids)}"
        assert bt[r, :nb[r]].tolist() == ids, f"{device_note}: row {r} table"
    assert int(alloc.free_ring_state[1].item()) == mgr.free_blocks(), f"{device_note}: free count"


@pytest.mark.parametrize("graph", [False, True])
def test_device_allocator_follows_host_block_manager(device, graph):
    rng = np.random.default_rng(6 + graph)
    num_blocks, bs, batch, cols = 72, 16, 24, 24
    prompts = rng.integers(1, 60, size=batch)
    rids = list(range(100, 100 + batch))
    mgr = orc.BlockManager(num_blocks, bs)
    alloc = vpa.DeviceBlockAllocator(num_blocks, bs, batch, cols, device)

    # admission: rows in order, as many as the pool holds
    ok_host = [mgr.try_allocate_slots(rid, int(p)) for rid, p in zip(rids, prompts)]
    ok_dev = alloc.allocate(u32(prompts, device)).cpu().numpy().astype(bool)
    assert ok_dev.tolist() == ok_host
    check_same(alloc, mgr, rids, "admission")
    pos = [int(p) if ok else 0 for p, ok in zip(prompts, ok_host)]
    finished = np.array([not ok for ok in ok_host], dtype=np.uint8)
    alloc.positions.copy_(u32(pos, device))
    fin_dev = torch.from_numpy(finished).to(device)

    g = None
    if graph:
        g = torch.cuda.CUDAGraph()
        # capture on a copy of the state, then restore it: the capture runs once
        saved = [t.clone() for t in (alloc.block_tables, alloc.row_blocks, alloc.positions,
                                     alloc.free_ring, alloc.free_ring_state)]
        with torch.cuda.graph(g):
            alloc.step(fin_dev)
        torch.cuda.synchronize()
        for t, s in zip((alloc.block_tables, alloc.row_blocks, alloc.positions, alloc.free_ring,
                         alloc.free_ring_state), saved):
            t.copy_(s)
        torch.cuda.synchronize()

    stalls_seen = 0
    for step in range(40):
        if g is not None:
            g.replay()
        else:
            alloc.step(fin_dev)
        torch.cuda.synchronize()
        want_slots, want_ctx = host_step(mgr, rids, pos, finished, bs, num_blocks)
        np.testing.assert_array_equal(alloc.slot_mapping.cpu().numpy(), want_slots)
        np.testing.assert_array_equal(alloc.context_lens.cpu().numpy(), want_ctx)
        np.testing.assert_array_equal(alloc.positions.cpu().numpy(), np.array(pos, np.uint32))
        st = alloc.status.cpu().numpy()
        stalls_seen += int(st[0])
        assert st[1] == 0
        check_same(alloc, mgr, rids, f"step {step}")
        # some rows finish: trim to their tokens (EOS) or free (request done)
        keep = np.full(batch, 0xFFFFFFFF, dtype=np.uint32)
        for r in rng.choice(batch, size=step % 2, replace=False):
            if finished[r]:
                continue
            finished[r] = 1
            if rng.random() < 0.5:
                mgr.trim_request_to_num_tokens(rids[r], pos[r])
                keep[r] = (pos[r] + bs - 1) // bs
            else:
                mgr.free_request(rids[r])
                keep[r] = 0
        fin_dev.copy_(torch.from_numpy(finished))
        alloc.release(u32(keep, device))
        torch.cuda.synchronize()
        check_same(alloc, mgr, rids, f"release {step}")
    assert stalls_seen > 0, "the pool never ran dry: the stall path was not exercised"


def test_admission_fits_then_overflows(device):
    """A first admission whose missing blocks all fit the ring (every row
    takes its blocks at once) and a second, growing the same rows, that does
    not (rows are served in order until the ring runs dry, later rows that
    still fit succeed): tables, counts and ok flags equal the oracle block
    manager's after each. (The manager has no table width, so rows are kept
    within the device tables' columns.)"""
    rng = np.random.default_rng(21)
    num_blocks, bs, batch, cols = 130, 16, 40, 12
    mgr = orc.BlockManager(num_blocks, bs)
    alloc = vpa.DeviceBlockAllocator(num_blocks, bs, batch, cols, device)
    rids = list(range(batch))
    first = rng.integers(1, 50, size=batch)
    second = np.minimum(first + rng.integers(0, 120, size=batch), cols * bs)
    for round_, target in enumerate((first, second)):
        ok_host = [mgr.try_allocate_slots(rid, int(t)) for rid, t in zip(rids, target)]
        ok_dev = alloc.allocate(u32(target, device)).cpu().numpy().astype(bool)
        torch.cuda.synchronize()
        assert ok_dev.tolist() == ok_host, f"round {round_}"
        check_same(alloc, mgr, rids, f"round {round_}")
        if round_ == 0:
            assert all(ok_host), "the first admission should fit"
        else:
            assert not all(ok_host) and any(ok_host[6:]), "want failures and later successes"
