"""c5 at full size on the GPU: batch 1024, contexts U[256, 8192], every
layer's cache one pool of about 60 % of the 288 GB of HBM (2.6 M blocks of
16 tokens, 173 GB), block tables drawn at random from all of it, so block
offsets run far past 2^32 bytes.

Two layers over the shared pool, each: reshape_and_cache of the batch's new
rows, then paged_attention over all 1024 sequences (layer 0 through the
unplanned call, layer 1 through plan + planned call). Checks:
* appends bit-exact: every slot written by exactly one sequence holds that
  sequence's new K and V rows (sequences may share blocks in c5, so a slot
  two sequences write is left out);
* attention: every sequence against the fp64 oracle over its blocks
  copied to host memory
  (workloads.compact_tables), bf16 tolerance 2e-2;
* every output row finite."""

import sys

import numpy as np
import pytest
import torch

import vpa
from oracle import oracle as orc
from tests._util import assert_attention_close, to_host
from vpa import workloads

pytestmark = pytest.mark.gpu


def test_c5_full_pool_append_and_decode(device):
    w = workloads.c5(num_layers=2)
    kvh, d, bs, h = w.num_kv_heads, w.head_dim, w.block_size, w.num_heads
    nb = w.layers[0].num_blocks
    pool_bytes = 2 * nb * kvh * d * bs * 2
    free, _ = torch.cuda.mem_get_info(device)
    if free < pool_bytes + (8 << 30):
        pytest.skip(f"c5 needs a {pool_bytes / 1e9:.0f} GB pool; {free / 1e9:.0f} GB free")
    print(f"c5: {w.num_seqs} seqs, max context {w.max_context_len}, {nb} blocks "
          f"({pool_bytes / 1e9:.1f} GB)", flush=True)
    g = torch.Generator(device=device)
    g.manual_seed(w.seed)
    bf = torch.bfloat16
    kc = vc = None
    try:
        kc = torch.randn((nb, kvh, d // 8, bs, 8), generator=g, device=device, dtype=bf)
        vc = torch.randn((nb, kvh, d, bs), generator=g, device=device, dtype=bf)
        ctx = torch.from_numpy(w.context_lens).to(device)
        ws = vpa.paged_attention_workspace(w.num_seqs, h, d, w.max_context_len, device)
        scale = d ** -0.5
        for li, layer in enumerate(w.layers):
            print(f"c5 layer {li}: append + {'planned' if li else 'unplanned'} decode",
                  flush=True)
            q = torch.randn((w.num_seqs, h, d), generator=g, device=device, dtype=bf)
            k = torch.randn((w.num_seqs, kvh, d), generator=g, device=device, dtype=bf)
            v = torch.randn((w.num_seqs, kvh, d), generator=g, device=device, dtype=bf)
            slots = torch.from_numpy(layer.slot_mapping.astype(np.int64)).to(device)
            bt = torch.from_numpy(layer.block_tables).to(device)
            vpa.reshape_and_cache(k, v, None, None, kc, vc, slots)
            if li == 0:
                out = vpa.paged_attention(q, None, None, kc, vc, bt, ctx, None,
                                          w.max_context_len, scale, 1.0, None)
            else:
                vpa.paged_attention_plan(ctx, w.max_context_len, bt.shape[1], h, kc, vc, bf, ws)
                out = vpa.paged_attention(q, None, None, kc, vc, bt, ctx, None,
                                          w.max_context_len, scale, 1.0, None, workspace=ws,
                                          planned=True)
            torch.cuda.synchronize()

            # appends: the rows at the slots written once
            sm = layer.slot_mapping.astype(np.int64)
            _, inv, cnt = np.unique(sm, return_inverse=True, return_counts=True)
            once = torch.from_numpy(np.flatnonzero(cnt[inv] == 1)).to(device)
            blk = slots[once] // bs
            off = slots[once] % bs
            got_k = kc[blk, :, :, off, :].reshape(len(once), kvh, d)
            got_v = vc[blk, :, :, off]
            assert torch.equal(got_k.view(torch.int16), k[once].view(torch.int16)), "K append"
            assert torch.equal(got_v.view(torch.int16), v[once].view(torch.int16)), "V append"
            assert bool(torch.isfinite(out).all()), "non-finite attention output"

            # attention on every sequence against the oracle (their blocks,
            # about 17 GB, copied out to host memory)
            lens = w.context_lens
            pick = np.arange(w.num_seqs)
            blocks, tables, _ = workloads.compact_tables(layer.block_tables[pick], lens[pick], bs)
            idx = torch.from_numpy(blocks).to(device)
            kh, vh = to_host(kc.index_select(0, idx)), to_host(vc.index_select(0, idx))
            qh = to_host(q[torch.from_numpy(pick).to(device)])
            want = orc.paged_attention(qh, kh, vh, tables, lens[pick], int(lens[pick].max()),
                                       scale, dtype=orc.BF16)
            got = orc.to_f32(to_host(out[torch.from_numpy(pick).to(device)]), orc.BF16)
            assert_attention_close(got, want, orc.BF16, f"c5 layer {li}")
            del q, k, v, out, got_k, got_v
    finally:
        del kc, vc
        torch.cuda.synchronize()
        torch.cuda.empty_cache()
        sys.stdout.flush()
