"""The host bookkeeping of vpa.host driving the HIP ops end to end, the way
vASR's runtime drives them: a block manager hands out blocks, the metadata
builders produce slots / tables / lengths, reshape_and_cache appends,
the prefill and decode kernels attend; every output is checked against the
fp64 oracle. Also the hipMemGetInfo pool sizing."""

import numpy as np
import pytest
import torch

import vpa
from vpa import host
from oracle import oracle as orc
from tests._util import assert_attention_close, i64, random_words, to_dev, to_host, u32

pytestmark = pytest.mark.gpu


def test_pool_blocks_for_memory_fraction(device):
    bpb = host.bytes_per_paged_block(28, 8, 128, 16, "bf16")
    n = host.resolve_num_blocks("fraction", 0.5, 28, 8, 128, 16, "bf16")
    free_b, total_b = torch.cuda.mem_get_info(device)
    used_mib = (total_b - free_b) >> 20
    budget_mib = int((total_b >> 20) * 0.5) - used_mib
    # the process's own allocations may move `used` by a few MiB between the calls
    assert abs(n - (budget_mib * (1 << 20) // bpb + 1)) <= 8
    assert n > 1


def test_runtime_prefill_then_decode_steps(device):
    code, h, kvh, d, bs = orc.BF16, 16, 8, 128, 16
    rng = np.random.default_rng(31)
    num_blocks = 96
    mgr = host.BlockManager(num_blocks, bs)
    kc, vc = (np.zeros((num_blocks, kvh, d // 8, bs, 8), np.uint16),
              np.zeros((num_blocks, kvh, d, bs), np.uint16))
    kc_d, vc_d = to_dev(kc, code, device), to_dev(vc, code, device)
    prompts = [37, 5, 120, 64, 1]
    rids = [100 + i for i in range(len(prompts))]
    for r, p in zip(rids, prompts):
        mgr.allocate_slots(r, p)
    tables = mgr.block_tables_for(rids)
    meta = host.input_metadata_from_query_lens(tables, prompts, bs, num_blocks)
    tq = sum(prompts)
    k = random_words(rng, (tq, kvh, d), code)
    v = random_words(rng, (tq, kvh, d), code)
    q = random_words(rng, (tq, h, d), code)
    vpa.reshape_and_cache(to_dev(k, code, device), to_dev(v, code, device), None, None, kc_d,
                          vc_d, i64(meta["slot_mapping"], device))
    out = vpa.paged_attention_varlen_prefill(
        to_dev(q, code, device), kc_d, vc_d, u32(meta["block_tables"], device),
        u32(meta["context_lens"], device), u32(meta["cu_seqlens_q"], device), None, None,
        d ** -0.5, 1.0, causal=True, max_query_len=meta["max_query_len"],
        max_context_len=meta["max_context_len"])
    torch.cuda.synchronize()
    orc.reshape_and_cache(k, v, kc, vc, meta["slot_mapping"], dtype=code)
    assert np.array_equal(to_host(kc_d), kc) and np.array_equal(to_host(vc_d), vc)
    want = orc.prefill_attention(q, kc, vc, meta["block_tables"], meta["context_lens"],
                                 meta["cu_seqlens_q"], d ** -0.5, causal=True, dtype=code)
    assert_attention_close(orc.to_f32(to_host(out), code), want, code, "runtime prefill")

    # decode: grow every request by one token per step, rebuild the tables,
    # pad the batch to its graph bucket and run append + attention
    ws = None
    for step in range(3):
        for r, p in zip(rids, prompts):
            assert mgr.try_allocate_slots(r, p + step + 1)
        tables = mgr.block_tables_for(rids)
        dm = host.decode_metadata_for_batch_steps(tables, [p + step for p in prompts], 1, bs,
                                                  num_blocks, num_blocks * bs,
                                                  graph_buckets=True)[0]
        b = len(rids)
        bucket = host.cuda_graph_batch_bucket(b, 256)
        ids, slots, ctx, bt = host.pad_decode_batch_to_max(
            bucket, np.arange(b), dm["slot_mapping"], dm["context_lens"], dm["block_tables"],
            dm["block_tables"].shape[1])
        kn = random_words(rng, (bucket, kvh, d), code)
        vn = random_words(rng, (bucket, kvh, d), code)
        qd = random_words(rng, (bucket, h, d), code)
        if ws is None:
            ws = vpa.paged_attention_workspace(bucket, h, d, int(bt.shape[1]) * bs, device)
        vpa.reshape_and_cache(to_dev(kn[:b], code, device), to_dev(vn[:b], code, device), None,
                              None, kc_d, vc_d, i64(slots[:b], device))
        o = vpa.paged_attention(to_dev(qd, code, device), None, None, kc_d, vc_d, u32(bt, device),
                                u32(ctx, device), None, int(bt.shape[1]) * bs, d ** -0.5, 1.0,
                                None, workspace=ws)
        torch.cuda.synchronize()
        orc.reshape_and_cache(kn[:b], vn[:b], kc, vc, slots[:b], dtype=code)
        assert np.array_equal(to_host(kc_d), kc) and np.array_equal(to_host(vc_d), vc)
        want = orc.paged_attention(qd, kc, vc, bt, ctx, int(bt.shape[1]) * bs, d ** -0.5,
                                   dtype=code)
        got = orc.to_f32(to_host(o), code)
        assert np.all(np.isfinite(got))  # pad rows (ctx 1, block 0) stay harmless
        assert_attention_close(got[:b], want[:b], code, f"runtime decode step {step}")
    for r in rids:
        mgr.free_request(r)
    assert mgr.free_blocks() == num_blocks - 1
