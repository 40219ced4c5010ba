"""vpa.graph.DecodeGraphCache: decode graphs per (batch bucket, column
bucket), replayed with the step's inputs padded into their buffers (pad
rows: slot 0, context 1, table row 0; columns repeating each row's last).

A sequence of steps of different batch sizes and table widths (misses,
hits, and an eviction with a small cache) runs append + paged_attention of
two layers through the cache; after every step the real rows' outputs
must equal the eager ops on the unpadded inputs bit for bit and the fp64
oracle over the caches after the step, and at the end both sets of caches
must be equal outside block 0 (the null block the pad rows write to)."""

import numpy as np
import pytest
import torch

import vpa
from oracle import oracle as orc
from tests._util import assert_attention_close, to_host
from vpa.graph import DecodeGraphCache

pytestmark = pytest.mark.gpu

H, KVH, D, BS, NL, MAXB = 16, 8, 128, 16, 2, 24
ROW_INPUTS = {}
for _i in range(NL):
    ROW_INPUTS[f"q{_i}"] = ((H, D), torch.bfloat16)
    ROW_INPUTS[f"k{_i}"] = ((KVH, D), torch.bfloat16)
    ROW_INPUTS[f"v{_i}"] = ((KVH, D), torch.bfloat16)


def make_caches(device, nb, seed):
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    return [(torch.randn((nb, KVH, D // 8, BS, 8), generator=g, device=device,
                         dtype=torch.bfloat16),
             torch.randn((nb, KVH, D, BS), generator=g, device=device, dtype=torch.bfloat16))
            for _ in range(NL)]


def make_forward(caches, device):
    workspaces = {}

    def forward(bufs, max_ctx):
        b = bufs["input_ids"].shape[0]
        if (b, max_ctx) not in workspaces:  # first built by the warm-up run, outside capture
            workspaces[(b, max_ctx)] = vpa.paged_attention_workspace(b, H, D, max_ctx, device)
        ws = workspaces[(b, max_ctx)]
        bt, ctx = bufs["block_tables"], bufs["context_lens"]
        vpa.paged_attention_plan(ctx, max_ctx, bt.shape[1], H, caches[0][0], caches[0][1],
                                 torch.bfloat16, ws)
        outs = []
        for i, (kc, vc) in enumerate(caches):
            vpa.reshape_and_cache(bufs[f"k{i}"], bufs[f"v{i}"], None, None, kc, vc,
                                  bufs["slot_mapping"])
            outs.append(vpa.paged_attention(bufs[f"q{i}"], None, None, kc, vc, bt, ctx, None,
                                            max_ctx, D ** -0.5, 1.0, None, workspace=ws,
                                            planned=True))
        return torch.stack(outs, dim=1)

    return forward


def eager_step(caches, rows, slots, ctx, bt, max_ctx):
    outs = []
    for i, (kc, vc) in enumerate(caches):
        vpa.reshape_and_cache(rows[f"k{i}"], rows[f"v{i}"], None, None, kc, vc, slots)
        outs.append(vpa.paged_attention(rows[f"q{i}"], None, None, kc, vc, bt, ctx, None,
                                        max_ctx, D ** -0.5, 1.0, None))
    return torch.stack(outs, dim=1)


@pytest.mark.parametrize("max_graphs", [256, 2])
def test_graph_cache_padded_replays_equal_eager(device, max_graphs):
    rng = np.random.default_rng(12 + max_graphs)
    nb = 1200
    cg, ce = make_caches(device, nb, 3), make_caches(device, nb, 3)
    cache = DecodeGraphCache(make_forward(cg, device), MAXB, BS, ROW_INPUTS, device,
                             max_graphs=max_graphs)
    g = torch.Generator(device=device)
    g.manual_seed(5)
    # (batch, longest context): misses, then repeats of earlier keys
    steps = [(3, 200), (7, 150), (16, 1000), (20, 900), (3, 180), (5, 60), (16, 950), (1, 5)]
    keys_seen = []
    for s, (a, lmax) in enumerate(steps):
        lens = rng.integers(1, lmax + 1, size=a)
        lens[0] = lmax
        need = (lens + BS - 1) // BS
        cols = int(need.max())
        ids = rng.permutation(np.arange(1, nb))[:int(need.sum())]
        bt = np.zeros((a, cols), dtype=np.uint32)
        off = 0
        for r, n in enumerate(need):
            bt[r, :n] = ids[off:off + n]
            off += n
        pos = lens - 1
        slots = bt[np.arange(a), pos // BS].astype(np.int64) * BS + pos % BS
        rows = {name: torch.randn((a,) + shape, generator=g, device=device, dtype=dt)
                for name, (shape, dt) in ROW_INPUTS.items()}
        ids_t = torch.arange(a, dtype=torch.int32, device=device).to(torch.uint32)
        slots_t = torch.from_numpy(slots).to(device)
        ctx_t = torch.from_numpy(lens.astype(np.uint32)).to(device)
        bt_t = torch.from_numpy(bt).to(device)
        key = cache.key(a, cols)
        hit = key in cache.graphs
        captures = cache.captures
        got = cache.run(ids_t, slots_t, ctx_t, bt_t, rows).clone()
        want = eager_step(ce, rows, slots_t, ctx_t, bt_t, int(lens.max()))
        torch.cuda.synchronize()
        assert cache.captures == captures + (0 if hit else 1), f"step {s}: hit={hit}"
        assert got.shape == want.shape
        assert torch.equal(got.view(torch.int16), want.view(torch.int16)), f"step {s} key {key}"
        for i, (kc, vc) in enumerate(cg):
            ref = orc.paged_attention(to_host(rows[f"q{i}"]), to_host(kc), to_host(vc), bt,
                                      lens.astype(np.uint32), int(lens.max()), D ** -0.5,
                                      dtype=orc.BF16)
            assert_attention_close(orc.to_f32(to_host(got[:, i]), orc.BF16), ref, orc.BF16,
                                   f"step {s} layer {i} vs oracle")
        keys_seen.append(key)
        assert len(cache.graphs) <= max_graphs
    assert any(k == keys_seen[0] for k in keys_seen[1:]), "want a repeated key"
    if max_graphs == 2:
        assert cache.captures > len(set(keys_seen)), "the small cache should have evicted"
    for (kg, vg), (ke, ve) in zip(cg, ce):
        assert torch.equal(kg[1:].view(torch.int16), ke[1:].view(torch.int16))
        assert torch.equal(vg[1:].view(torch.int16), ve[1:].view(torch.int16))

