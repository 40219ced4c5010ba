"""Run-to-run determinism and independent calls on concurrent streams.

The decode hands out its work items through a per-workspace queue, the
prefill orders its workgroups on the device, and the library keeps no
global device state outside the allocation-free entry point's scratch; so
repeated calls on the same inputs give the same bits, and calls with their
own workspaces and outputs on two streams at once give the same bits as the
same calls one after another on one stream. Streams keep the default
priority."""

import numpy as np
import pytest
import torch

import vpa
from oracle import oracle as orc
from tests._util import block_tables_for, i64, make_cache, random_words, to_dev, u32

pytestmark = pytest.mark.gpu

H, KVH, D, BS = 16, 8, 128, 16


def decode_problem(device, seed, lens):
    rng = np.random.default_rng(seed)
    code = orc.BF16
    nb = sum((L + BS - 1) // BS for L in lens) + 9
    kc, vc = make_cache(rng, nb, KVH, D, BS, code)
    bt = block_tables_for(rng, lens, nb, BS)
    q = random_words(rng, (len(lens), H, D), code)
    kn = random_words(rng, (len(lens), KVH, D), code)
    vn = random_words(rng, (len(lens), KVH, D), code)
    # the appended token goes to the last slot of each context
    slots = np.array([int(bt[s, (L - 1) // BS]) * BS + (L - 1) % BS for s, L in enumerate(lens)],
                     dtype=np.int64)
    t = dict(q=to_dev(q, code, device), kc=to_dev(kc, code, device),
             vc=to_dev(vc, code, device), bt=u32(bt, device),
             cl=u32(np.asarray(lens, dtype=np.uint32), device), kn=to_dev(kn, code, device),
             vn=to_dev(vn, code, device), slots=i64(slots, device), max_ctx=max(lens))
    t["ws"] = vpa.paged_attention_workspace(len(lens), H, D, t["max_ctx"], device)
    t["out"] = torch.empty((len(lens), H, D), dtype=torch.bfloat16, device=device)
    return t


def prefill_problem(device, seed, prior, qlens):
    rng = np.random.default_rng(seed)
    code = orc.BF16
    lens = [p + n for p, n in zip(prior, qlens)]
    nb = sum((L + BS - 1) // BS for L in lens) + 9
    kc, vc = make_cache(rng, nb, KVH, D, BS, code)
    bt = block_tables_for(rng, lens, nb, BS)
    q = random_words(rng, (sum(qlens), H, D), code)
    cu = np.concatenate([[0], np.cumsum(qlens)]).astype(np.uint32)
    t = dict(q=to_dev(q, code, device), kc=to_dev(kc, code, device),
             vc=to_dev(vc, code, device), bt=u32(bt, device),
             cl=u32(np.asarray(lens, dtype=np.uint32), device), cu=u32(cu, device))
    t["out"] = torch.empty((sum(qlens), H, D), dtype=torch.bfloat16, device=device)
    return t


def run_decode(t, planned):
    vpa.reshape_and_cache(t["kn"], t["vn"], None, None, t["kc"], t["vc"], t["slots"])
    if planned:
        vpa.paged_attention_plan(t["cl"], t["max_ctx"], t["bt"].shape[1], H, t["kc"], t["vc"],
                                 torch.bfloat16, t["ws"])
    vpa.paged_attention(t["q"], None, None, t["kc"], t["vc"], t["bt"], t["cl"], None,
                        t["max_ctx"], D ** -0.5, 1.0, None, out=t["out"], workspace=t["ws"],
                        planned=planned)


def run_prefill(t):
    vpa.paged_attention_varlen_prefill(t["q"], t["kc"], t["vc"], t["bt"], t["cl"], t["cu"], None,
                                       None, D ** -0.5, 1.0, causal=True, out=t["out"])


def test_repeated_calls_are_bit_identical(device):
    dec = decode_problem(device, 1, [1, 17, 300, 2048, 2049, 3999, 777])
    pre = prefill_problem(device, 2, [0, 40, 333], [64, 129, 7])
    outs = {"plain": [], "planned": [], "prefill": []}
    for _ in range(3):
        run_decode(dec, planned=False)
        outs["plain"].append(dec["out"].clone())
        run_decode(dec, planned=True)
        outs["planned"].append(dec["out"].clone())
        run_prefill(pre)
        outs["prefill"].append(pre["out"].clone())
    torch.cuda.synchronize()
    for k, v in outs.items():
        for o in v[1:]:
            assert torch.equal(o.view(torch.int16), v[0].view(torch.int16)), k
    # the planned and the plain call compute the same rows
    assert torch.equal(outs["plain"][0].view(torch.int16), outs["planned"][0].view(torch.int16))


def test_concurrent_streams_with_own_workspaces_match_serial(device):
    problems = [decode_problem(device, 10 + i, lens) for i, lens in
                enumerate(([5, 2100, 64, 4000], [1, 33, 1500, 2048, 2500], [900] * 6))]
    pre = prefill_problem(device, 20, [10, 0, 500], [200, 33, 64])
    caches0 = [(p["kc"].clone(), p["vc"].clone()) for p in problems]
    pre_kc0 = pre["kc"].clone()

    def reset():
        for p, (k, v) in zip(problems, caches0):
            p["kc"].copy_(k)
            p["vc"].copy_(v)
        pre["kc"].copy_(pre_kc0)

    # serial reference on the current stream: two rounds of every call
    for _ in range(2):
        for i, p in enumerate(problems):
            run_decode(p, planned=i % 2 == 1)
        run_prefill(pre)
    torch.cuda.synchronize()
    want = [p["out"].clone() for p in problems] + [pre["out"].clone()]
    want_caches = [(p["kc"].clone(), p["vc"].clone()) for p in problems]
    for p in problems:
        p["out"].zero_()
    pre["out"].zero_()
    reset()
    torch.cuda.synchronize()

    streams = [torch.cuda.Stream(device) for _ in range(2)]
    for _ in range(2):
        for i, p in enumerate(problems):
            with torch.cuda.stream(streams[i % 2]):
                run_decode(p, planned=i % 2 == 1)
        with torch.cuda.stream(streams[1]):
            run_prefill(pre)
    torch.cuda.synchronize()
    got = [p["out"] for p in problems] + [pre["out"]]
    for i, (g, w) in enumerate(zip(got, want)):
        assert torch.equal(g.view(torch.int16), w.view(torch.int16)), f"output {i}"
    for i, (p, (k, v)) in enumerate(zip(problems, want_caches)):
        assert torch.equal(p["kc"].view(torch.int16), k.view(torch.int16)), f"key cache {i}"
        assert torch.equal(p["vc"].view(torch.int16), v.view(torch.int16)), f"value cache {i}"
