"""The decode step captured in a HIP graph (the way vASR replays decode,
vasr-paged-attn/src/cuda_graph.rs:204-225): append + paged_attention of
several layers recorded once, replayed with new per-step metadata copied
into the captured buffers (cuda_graph.rs:342-371). Every replay is checked
against the eager ops on the same inputs (bit for bit), with eager work and
host synchronisation between replays, and every replayed layer's output
against the fp64 oracle over the caches the replay left."""

import numpy as np
import pytest
import torch

import vpa
from oracle import oracle as orc
from tests._util import assert_attention_close, block_tables_for, to_host

pytestmark = pytest.mark.gpu


def test_graph_replay_of_decode_steps_matches_eager(device):
    rng = np.random.default_rng(41)
    B, H, KVH, D, BS, LAYERS = 12, 16, 8, 128, 16, 3
    max_ctx = 1024
    nb = B * (max_ctx // BS) + 8
    lens0 = rng.integers(20, 700, size=B)
    g = torch.Generator(device=device)
    g.manual_seed(41)
    bf = torch.bfloat16
    caches = [(torch.randn((nb, KVH, D // 8, BS, 8), generator=g, device=device, dtype=bf),
               torch.randn((nb, KVH, D, BS), generator=g, device=device, dtype=bf))
              for _ in range(LAYERS)]
    # captured inputs: metadata and per-layer q/k/v buffers, refreshed before replays
    bt_np = block_tables_for(rng, [max_ctx] * B, nb, BS)
    bt = torch.from_numpy(bt_np).to(device)
    ctx = torch.zeros(B, dtype=torch.uint32, device=device)
    slots = torch.zeros(B, dtype=torch.int64, device=device)
    q = [torch.empty((B, H, D), device=device, dtype=bf) for _ in range(LAYERS)]
    k = [torch.empty((B, KVH, D), device=device, dtype=bf) for _ in range(LAYERS)]
    v = [torch.empty((B, KVH, D), device=device, dtype=bf) for _ in range(LAYERS)]
    out = [torch.empty((B, H, D), device=device, dtype=bf) for _ in range(LAYERS)]
    ws = vpa.paged_attention_workspace(B, H, D, max_ctx, device)

    def step(outs):
        for i in range(LAYERS):
            vpa.reshape_and_cache(k[i], v[i], None, None, caches[i][0], caches[i][1], slots)
            vpa.paged_attention(q[i], None, None, caches[i][0], caches[i][1], bt, ctx, None,
                                max_ctx, D ** -0.5, 1.0, None, out=outs[i], workspace=ws)

    def refresh(step_idx):
        lens = lens0 + step_idx
        pos = lens - 1
        s = bt_np[np.arange(B), pos // BS].astype(np.int64) * BS + pos % BS
        ctx.copy_(torch.from_numpy(lens.astype(np.uint32)))
        slots.copy_(torch.from_numpy(s))
        for i in range(LAYERS):
            q[i].normal_(generator=g)
            k[i].normal_(generator=g)
            v[i].normal_(generator=g)

    refresh(0)
    step(out)  # warm up (and the first real step) before capture
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step(out)
    torch.cuda.synchronize()
    for t in range(1, 5):
        refresh(t)
        # eager reference on copies of the caches (the graph appends to the originals)
        saved = [(kc.clone(), vc.clone()) for kc, vc in caches]
        want = [torch.empty_like(o) for o in out]
        orig = [c for c in caches]
        caches[:] = saved
        step(want)
        caches[:] = orig
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        lens = (lens0 + t).astype(np.uint32)
        for i in range(LAYERS):
            assert torch.equal(out[i], want[i]), f"replay {t} layer {i}"
            assert torch.equal(caches[i][0], saved[i][0]) and torch.equal(caches[i][1],
                                                                           saved[i][1])
            ref = orc.paged_attention(to_host(q[i]), to_host(caches[i][0]), to_host(caches[i][1]),
                                      bt_np, lens, max_ctx, D ** -0.5, dtype=orc.BF16)
            assert_attention_close(orc.to_f32(to_host(out[i]), orc.BF16), ref, orc.BF16,
                                   f"replay {t} layer {i} vs oracle")
