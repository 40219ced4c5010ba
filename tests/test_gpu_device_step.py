"""The device-resident decode step (vpa.DeviceDecodeStep) captured once as a
HIP graph and replayed, against the same calls made eagerly on a copy of
every buffer: after each step the attention outputs, the caches, the
allocator's tables / slots / lengths / free ring and the token state
(next ids, finished flags, generated lists, input ids, active count) must be
equal bit for bit. New inputs (q, k, v, logits) are written into the
graph's buffers between replays, with an eager step and synchronisations in
between. The last step's attention is also checked against the fp64 oracle
over the caches and the allocator's tables, and every row's appended K/V
against its input, so the composition (block growth -> slot -> append ->
attention over the grown table) is what the reference computes."""

import numpy as np
import pytest
import torch

import vpa
from oracle import oracle as orc
from tests._util import assert_attention_close, to_host

pytestmark = pytest.mark.gpu

B, NL, H, KVH, D, BS, V = 24, 2, 16, 8, 128, 16, 300
EOS = [7, 11]


def make_state(device, prompts, nb, seed):
    st = vpa.DeviceDecodeStep(B, nb, BS, max_context_len=int(prompts.max()) + 40, num_heads=H,
                              head_dim=D, eos_token_ids=EOS, max_new_tokens=16, device=device)
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    caches = [(torch.randn((nb, KVH, D // 8, BS, 8), generator=g, device=device,
                           dtype=torch.bfloat16),
               torch.randn((nb, KVH, D, BS), generator=g, device=device, dtype=torch.bfloat16))
              for _ in range(NL)]
    st.admit(torch.from_numpy(prompts.astype(np.uint32)).to(device))
    return st, caches


def buffers(device):
    bf = torch.bfloat16
    return dict(q=torch.zeros((NL, B, H, D), dtype=bf, device=device),
                k=torch.zeros((NL, B, KVH, D), dtype=bf, device=device),
                v=torch.zeros((NL, B, KVH, D), dtype=bf, device=device),
                out=torch.zeros((NL, B, H, D), dtype=bf, device=device),
                logits=torch.zeros((B, V), dtype=bf, device=device))


def run_step(st, caches, buf):
    st.begin(caches[0][0], caches[0][1], torch.bfloat16)
    for i, (kc, vc) in enumerate(caches):
        st.layer(buf["q"][i], buf["k"][i], buf["v"][i], kc, vc, buf["out"][i])
    st.end(buf["logits"])


def state_tensors(st, caches, buf):
    a, t = st.allocator, st.tokens
    return ([buf["out"], a.block_tables, a.row_blocks, a.positions, a.slot_mapping,
             a.context_lens, a.free_ring, a.free_ring_state, t.next_ids, t.finished,
             t.generated, t.gen_len, t.input_ids, t.active_count]
            + [c for kv in caches for c in kv])


def test_device_step_graph_replays_equal_eager(device):
    rng = np.random.default_rng(5)
    prompts = rng.integers(1, 200, size=B)
    prompts[3] = 16   # the first step starts a new block
    prompts[4] = 15
    nb = int(((prompts + 40 + BS - 1) // BS).sum()) + 4
    ga, ca = make_state(device, prompts, nb, seed=9)   # replayed from the graph
    gb, cb = make_state(device, prompts, nb, seed=9)   # eager
    ba, bb = buffers(device), buffers(device)
    torch.cuda.synchronize()

    # capture on a copy of A's state, then restore it
    saved = [x.clone() for x in state_tensors(ga, ca, ba)]
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        run_step(ga, ca, ba)
    torch.cuda.synchronize()
    for x, y in zip(state_tensors(ga, ca, ba), saved):
        x.copy_(y)
    torch.cuda.synchronize()

    g = torch.Generator(device=device)
    g.manual_seed(77)
    steps = 10
    for s in range(steps):
        for name in ("q", "k", "v"):
            x = torch.randn(ba[name].shape, generator=g, device=device, dtype=torch.bfloat16)
            ba[name].copy_(x)
            bb[name].copy_(x)
        lg = torch.randn((B, V), generator=g, device=device, dtype=torch.float32)
        lg[:, EOS[0]] += 1.2  # some rows finish along the way
        ba["logits"].copy_(lg)
        bb["logits"].copy_(lg)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        run_step(gb, cb, bb)
        torch.cuda.synchronize()
        for i, (x, y) in enumerate(zip(state_tensors(ga, ca, ba), state_tensors(gb, cb, bb))):
            assert torch.equal(x.view(torch.uint8), y.view(torch.uint8)), f"step {s} tensor {i}"

    # the last step against the oracle: every unfinished row's appended K/V
    # sits at its slot, and its attention is the oracle's over the caches
    a = gb.allocator
    fin = gb.tokens.finished.cpu().numpy().astype(bool)
    live = np.flatnonzero(~fin)
    assert 0 < len(live) < B, "want both finished and running rows"
    slots = a.slot_mapping.cpu().numpy()
    assert np.all(slots[live] >= 0) and np.all(slots[fin] == -1)
    kc, vc = cb[0]
    idx = torch.from_numpy(live).to(device)
    blk, off = a.slot_mapping[idx] // BS, a.slot_mapping[idx] % BS
    assert torch.equal(kc[blk, :, :, off, :].reshape(len(live), KVH, D).view(torch.int16),
                       bb["k"][0][idx].view(torch.int16))
    assert torch.equal(vc[blk, :, :, off].view(torch.int16), bb["v"][0][idx].view(torch.int16))
    bt = a.block_tables.cpu().numpy()[live]
    lens = a.context_lens.cpu().numpy()[live]
    np.testing.assert_array_equal(lens, a.positions.cpu().numpy()[live])
    want = orc.paged_attention(to_host(bb["q"][0][idx]), to_host(kc), to_host(vc), bt, lens,
                               int(lens.max()), D ** -0.5, dtype=orc.BF16)
    got = orc.to_f32(to_host(bb["out"][0][idx]), orc.BF16)
    assert_attention_close(got, want, orc.BF16, "device step layer 0")
