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


def test_device_step_over_a_pool_that_runs_dry(device):
    """DeviceDecodeStep over a pool with a few spare blocks, so rows stall
    when their next token needs a block, and resume when finished rows free
    theirs; in lockstep with a host model of the same loop: the oracle's
    step-start bookkeeping (with the stall rule), the oracle's block manager
    and slot rule, the oracle's appends, the oracle's argmax. After every
    step the token state (generated lists, finished flags, input and
    pending ids), slots, context lengths, positions and tables must equal the
    host's; at the end both layers' caches bit for bit, and the last step's
    attention of every row that ran against the fp64 oracle."""
    from tests.test_gpu_device_metadata import check_same, host_step

    rng = np.random.default_rng(23)
    b, nl, steps, cap = 20, 2, 22, 32
    prompts = rng.integers(1, 60, size=b)
    nb = int(((prompts + BS - 1) // BS).sum()) + 1 + 1  # one spare block
    st = vpa.DeviceDecodeStep(b, nb, BS, max_context_len=int(prompts.max()) + steps + 1,
                              num_heads=H, head_dim=D, eos_token_ids=EOS, max_new_tokens=cap,
                              device=device)
    g = torch.Generator(device=device)
    g.manual_seed(31)
    caches = [(torch.randn((nb, KVH, D // 8, BS, 8), generator=g, device=device,
                           dtype=torch.bfloat16),
               torch.randn((nb, KVH, D, BS), generator=g, device=device, dtype=torch.bfloat16))
              for _ in range(nl)]
    host_caches = [(to_host(kc), to_host(vc)) for kc, vc in caches]
    pend = rng.integers(20, V, size=b).astype(np.uint32)
    st.tokens.next_ids.copy_(torch.from_numpy(pend).to(device))
    ok = st.admit(torch.from_numpy(prompts.astype(np.uint32)).to(device)).cpu().numpy()

    rids = list(range(b))
    mgr = orc.BlockManager(nb, BS)
    assert [mgr.try_allocate_slots(r, int(p)) for r, p in zip(rids, prompts)] == \
        ok.astype(bool).tolist() == [True] * b
    pos = [int(p) for p in prompts]
    nid, fin = pend.copy(), np.zeros(b, np.uint8)
    gen, glen = np.zeros((b, cap), np.uint32), np.zeros(b, np.uint32)
    inp, prev = np.zeros(b, np.uint32), np.zeros(b, np.int64)
    bf = torch.bfloat16
    stalls = resumed = 0
    stalled_before = np.zeros(b, bool)
    for s in range(steps):
        q = torch.randn((nl, b, H, D), generator=g, device=device, dtype=bf)
        k = torch.randn((nl, b, KVH, D), generator=g, device=device, dtype=bf)
        v = torch.randn((nl, b, KVH, D), generator=g, device=device, dtype=bf)
        out = torch.empty((nl, b, H, D), device=device, dtype=bf)
        lg = torch.randn((b, V), generator=g, device=device, dtype=torch.float32)
        lg[:, EOS[0]] += 1.0  # rows finish along the way and free their blocks
        logits = lg.to(bf)
        st.begin(caches[0][0], caches[0][1], bf)
        for i, (kc, vc) in enumerate(caches):
            st.layer(q[i], k[i], v[i], kc, vc, out[i])
        st.end(logits)
        torch.cuda.synchronize()

        # host model of the same step
        inp, active = orc.decode_consume_tokens(nid, fin, gen, glen, EOS, EOS[0], prev, inp)
        slots, ctx = host_step(mgr, rids, pos, fin, BS, nb)
        for i, (kc_h, vc_h) in enumerate(host_caches):
            orc.reshape_and_cache(to_host(k[i]), to_host(v[i]), kc_h, vc_h, slots,
                                  dtype=orc.BF16)
        nid = orc.argmax_rows(to_host(logits), dtype=orc.BF16)
        ran = slots >= 0
        stalled = (fin == 0) & ~ran
        stalls += int(stalled.sum())
        resumed += int((stalled_before & ran).sum())
        stalled_before = stalled
        prev = slots

        t, a = st.tokens, st.allocator
        note = f"step {s}"
        assert int(t.active_count.item()) == active, note
        np.testing.assert_array_equal(t.finished.cpu().numpy(), fin, note)
        np.testing.assert_array_equal(t.gen_len.cpu().numpy(), glen, note)
        np.testing.assert_array_equal(t.generated.cpu().numpy(), gen, note)
        np.testing.assert_array_equal(t.input_ids.cpu().numpy(), inp, note)
        np.testing.assert_array_equal(t.next_ids.cpu().numpy(), nid, note)
        np.testing.assert_array_equal(a.slot_mapping.cpu().numpy(), slots, note)
        np.testing.assert_array_equal(a.context_lens.cpu().numpy(), ctx, note)
        np.testing.assert_array_equal(a.positions.cpu().numpy(), np.array(pos, np.uint32), note)
        check_same(a, mgr, rids, note)
        if s == steps - 1:
            break
        # rows that finished this step give their blocks back (request done)
        keep = np.full(b, 0xFFFFFFFF, dtype=np.uint32)
        for r in range(b):
            if fin[r] and mgr.blocks_for_request(rids[r]) > 0:
                mgr.free_request(rids[r])
                keep[r] = 0
        a.release(torch.from_numpy(keep).to(device))
        torch.cuda.synchronize()
        check_same(a, mgr, rids, f"release {s}")
    assert stalls > 0 and resumed > 0, f"stalls {stalls}, resumed {resumed}: want both"
    assert 0 < int(fin.sum()) < b
    for i, (kc, vc) in enumerate(caches):
        assert np.array_equal(to_host(kc), host_caches[i][0]), f"layer {i} key cache"
        assert np.array_equal(to_host(vc), host_caches[i][1]), f"layer {i} value cache"
    live = np.flatnonzero(slots >= 0)
    bt = st.allocator.block_tables.cpu().numpy()[live]
    want = orc.paged_attention(to_host(q[0][live]), host_caches[0][0], host_caches[0][1], bt,
                               ctx[live], int(ctx[live].max()), D ** -0.5, dtype=orc.BF16)
    got = orc.to_f32(to_host(out[0][torch.from_numpy(live).to(device)]), orc.BF16)
    assert_attention_close(got, want, orc.BF16, "dry pool, last step, layer 0")
