"""vpa_reshape_and_cache_paged_attention (one decode layer's append and
attention behind one call, in one launch for small batches over 16-bit
caches) against the two calls it stands for:
reshape_and_cache of row s at position context_lens[s] - 1 of sequence s's
table (thinker_text.rs:1101-1109), then paged_attention
(thinker_text.rs:1126-1139). Both run on the GPU through the C ABI from the
same inputs; the whole caches (every byte, other blocks and stale slots
included) and the outputs must be equal bit for bit, and the fused output is
also checked against the fp64 oracle over the oracle's own append."""

import numpy as np
import pytest
import torch

import vpa
from oracle import oracle as orc
from tests._util import (assert_attention_close, block_tables_for, i64, make_cache,
                         random_words, to_dev, to_host, u32)

pytestmark = pytest.mark.gpu


def case(rng, code, h, kvh, d, bs, lens, extra_blocks=8, fp8=False):
    need = sum((int(L) + bs - 1) // bs for L in lens)
    nb = need + extra_blocks
    if fp8:
        kc = rng.integers(0, 256, size=(nb, kvh, d // 16, bs, 16), dtype=np.uint8)
        vc = rng.integers(0, 256, size=(nb, kvh, d, bs), dtype=np.uint8)
        for a in (kc, vc):
            a[(a & 0x7F) == 0x7F] = 0x38  # no NaN codes
    else:
        kc, vc = make_cache(rng, nb, kvh, d, bs, code)
    bt = block_tables_for(rng, [max(int(L), 1) for L in lens], nb, bs)
    lens = np.asarray(lens, dtype=np.uint32)
    q = random_words(rng, (len(lens), h, d), code)
    k = random_words(rng, (len(lens), kvh, d), code)
    v = random_words(rng, (len(lens), kvh, d), code)
    return dict(kc=kc, vc=vc, bt=bt, lens=lens, q=q, k=k, v=v, nb=nb)


def last_slots(bt, lens, bs):
    """Slot of position L - 1 of each sequence; -1 (nothing appended) for L = 0."""
    pos = lens.astype(np.int64) - 1
    safe = np.maximum(pos, 0)
    slots = bt[np.arange(len(lens)), safe // bs].astype(np.int64) * bs + safe % bs
    return np.where(pos >= 0, slots, -1)


def dev_caches(c, code, device):
    if c["kc"].dtype == np.uint8:  # fp8 E4M3FN bytes
        return (torch.from_numpy(c["kc"]).to(device).view(torch.float8_e4m3fn),
                torch.from_numpy(c["vc"]).to(device).view(torch.float8_e4m3fn))
    return to_dev(c["kc"], code, device), to_dev(c["vc"], code, device)


def host_cache(t):
    if t.dtype == torch.float8_e4m3fn:
        return t.view(torch.uint8).cpu().numpy()
    return to_host(t)


def scales(c, device):
    if c["kc"].dtype != np.uint8:
        return None, None
    return (torch.tensor([c["k_scale"]], dtype=torch.float32, device=device),
            torch.tensor([c["v_scale"]], dtype=torch.float32, device=device))


def two_calls(device, c, code, bs, max_ctx, scale):
    kc, vc = dev_caches(c, code, device)
    q, k, v = (to_dev(c[x], code, device) for x in ("q", "k", "v"))
    bt, lens = u32(c["bt"], device), u32(c["lens"], device)
    ks, vs = scales(c, device)
    vpa.reshape_and_cache(k, v, ks, vs, kc, vc, i64(last_slots(c["bt"], c["lens"], bs), device))
    out = vpa.paged_attention(q, ks, vs, kc, vc, bt, lens, None, max_ctx, scale, 1.0, None)
    torch.cuda.synchronize()
    return to_host(out), host_cache(kc), host_cache(vc)


def fused(device, c, code, max_ctx, scale, planned=False):
    kc, vc = dev_caches(c, code, device)
    q, k, v = (to_dev(c[x], code, device) for x in ("q", "k", "v"))
    bt, lens = u32(c["bt"], device), u32(c["lens"], device)
    ks, vs = scales(c, device)
    ws = None
    if planned:
        b, h, d = c["q"].shape
        ws = vpa.paged_attention_workspace(b, h, d, max_ctx, device)
        vpa.paged_attention_plan(lens, max_ctx, bt.shape[1], h, kc, vc, q.dtype, ws)
    out = vpa.reshape_and_cache_paged_attention(q, k, v, ks, vs, kc, vc, bt, lens, max_ctx,
                                                scale, workspace=ws, planned=planned)
    torch.cuda.synchronize()
    return to_host(out), host_cache(kc), host_cache(vc)


def oracle_fused(c, code, bs, max_ctx, scale):
    kc, vc = c["kc"].copy(), c["vc"].copy()
    orc.reshape_and_cache(c["k"], c["v"], kc, vc, last_slots(c["bt"], c["lens"], bs), dtype=code)
    want = orc.paged_attention(c["q"], kc, vc, c["bt"], c["lens"], max_ctx, scale, dtype=code)
    return want, kc, vc


EDGES = [1, 2, 15, 16, 17, 31, 32, 33, 511, 512, 513, 2047, 2048, 2049, 4097, 6000]


@pytest.mark.parametrize("code", [orc.BF16, orc.F16])
@pytest.mark.parametrize("d,bs", [(128, 16), (128, 8), (128, 32), (64, 16), (64, 8), (64, 32),
                                  (96, 32), (192, 16), (256, 8), (256, 16)])
@pytest.mark.parametrize("h,kvh", [(16, 8), (16, 4), (8, 8)])
@pytest.mark.parametrize("planned", [False, True])
def test_fused_equals_two_calls(device, code, d, bs, h, kvh, planned):
    rng = np.random.default_rng(1000 + d + bs + h + kvh + 7 * code + planned)
    c = case(rng, code, h, kvh, d, bs, EDGES)
    max_ctx, scale = int(c["lens"].max()), d ** -0.5
    got, gk, gv = fused(device, c, code, max_ctx, scale, planned=planned)
    want, wk, wv = two_calls(device, c, code, bs, max_ctx, scale)
    np.testing.assert_array_equal(gk, wk)
    np.testing.assert_array_equal(gv, wv)
    np.testing.assert_array_equal(got, want)
    ref, rk, rv = oracle_fused(c, code, bs, max_ctx, scale)
    np.testing.assert_array_equal(gk, rk)
    np.testing.assert_array_equal(gv, rv)
    assert_attention_close(orc.to_f32(got, code), ref, code, f"fused d={d} bs={bs} h={h}")


@pytest.mark.parametrize("what", ["bf16 batch 64", "f32", "fp8 cache", "head dim 96",
                                  "head dim 192"])
def test_two_launch_form_equals_two_calls(device, what):
    """The configurations the one-launch form does not take (more than 48
    sequences, f32 and fp8 caches, 16-bit (block, head) tiles under 2 KiB,
    as head dim 96 at 16-token blocks, and the shapes the rows kernel does
    not take, as head dim 192 at 32) run the append kernel on the slots
    derived from the tables, then the decode: still the two calls' bytes and
    outputs."""
    rng = np.random.default_rng(sum(map(ord, what)))
    code, d, fp8, lens = orc.BF16, 128, False, EDGES
    if what == "bf16 batch 64":
        lens = [int(x) for x in rng.integers(1, 3000, size=64)]
    elif what == "f32":
        code = orc.F32
    elif what == "fp8 cache":
        fp8 = True
    else:
        d = int(what.split()[-1])
    bs = 32 if d == 192 else 16
    c = case(rng, code, 16, 8, d, bs, lens, fp8=fp8)
    if fp8:
        c["k_scale"], c["v_scale"] = 0.7, 1.9
    max_ctx = int(c["lens"].max())
    for planned in (False, True):
        got, gk, gv = fused(device, c, code, max_ctx, d ** -0.5, planned=planned)
        want, wk, wv = two_calls(device, c, code, bs, max_ctx, d ** -0.5)
        np.testing.assert_array_equal(gk, wk)
        np.testing.assert_array_equal(gv, wv)
        np.testing.assert_array_equal(got, want)


def test_fused_config_c3_shape(device):
    """c3's shape and length rule (bf16, 256 sequences of
    clip(Geom(mean 800), 16, 4096) tokens, 16 q / 8 kv heads, block 16), one
    layer, planned as the bench runs it."""
    rng = np.random.default_rng(3)
    lens = np.clip(rng.geometric(1.0 / 800.0, size=256), 16, 4096)
    c = case(rng, orc.BF16, 16, 8, 128, 16, lens, extra_blocks=64)
    max_ctx = int(c["lens"].max())
    got, gk, gv = fused(device, c, orc.BF16, max_ctx, 128 ** -0.5, planned=True)
    want, wk, wv = two_calls(device, c, orc.BF16, 16, max_ctx, 128 ** -0.5)
    np.testing.assert_array_equal(gk, wk)
    np.testing.assert_array_equal(gv, wv)
    np.testing.assert_array_equal(got, want)


def test_fused_graph_pad_rows_and_empty_contexts(device):
    """Graph pad rows (context 1 over table row 0, the slot-0 rule of
    cuda_graph.rs:395-408) and a context of 0: the real rows' caches and
    outputs equal the two calls; block 0, shared by the pad rows, is
    compared outside token 0 (which holds one pad row's token in either
    form); a context of 0 appends nothing and gives zeros."""
    rng = np.random.default_rng(77)
    code, h, kvh, d, bs = orc.BF16, 16, 8, 128, 16
    real = [700, 33, 1, 2049]
    c = case(rng, code, h, kvh, d, bs, real + [1, 1, 1, 5])
    c["bt"][4:7, :] = 0  # three pad rows: context 1, table row 0
    c["lens"][7] = 0  # an empty context
    max_ctx = int(c["lens"].max())
    got, gk, gv = fused(device, c, code, max_ctx, d ** -0.5)
    want, wk, wv = two_calls(device, c, code, bs, max_ctx, d ** -0.5)
    np.testing.assert_array_equal(gk[1:], wk[1:])
    np.testing.assert_array_equal(gv[1:], wv[1:])
    np.testing.assert_array_equal(gk[0, :, :, 1:], wk[0, :, :, 1:])
    np.testing.assert_array_equal(gv[0, :, :, 1:], wv[0, :, :, 1:])
    np.testing.assert_array_equal(got[:4], want[:4])
    assert not np.any(orc.to_f32(got[7], code))
    # each pad row attends over its own new token alone: out = V_new (context 1)
    for s in range(4, 7):
        for hh in range(h):
            v_row = orc.to_f32(c["v"][s, hh // (h // kvh)], code)
            np.testing.assert_allclose(orc.to_f32(got[s, hh], code), v_row / (1.0 + 1e-6),
                                       rtol=1e-2, atol=1e-3)


def test_fused_layers_under_graph_replay(device):
    """Three layers of plan + fused planned calls captured in one HIP graph
    and replayed with refreshed new rows and queries: every replay equals the
    eager two-call step bit for bit (caches and outputs)."""
    rng = np.random.default_rng(91)
    code, h, kvh, d, bs = orc.BF16, 16, 8, 128, 16
    lens = [1, 300, 2048, 2049, 5000, 17]
    cases = [case(rng, code, h, kvh, d, bs, lens) for _ in range(3)]
    max_ctx = 5000
    scale = d ** -0.5
    dev_c = []
    for c in cases:
        dev_c.append(dict(kc=to_dev(c["kc"], code, device), vc=to_dev(c["vc"], code, device),
                          bt=u32(c["bt"], device)))
    lens_d = u32(np.asarray(lens, dtype=np.uint32), device)
    q = torch.empty((len(lens), h, d), dtype=torch.bfloat16, device=device)
    k = torch.empty((len(lens), kvh, d), dtype=torch.bfloat16, device=device)
    v = torch.empty_like(k)
    outs = [torch.empty_like(q) for _ in cases]
    ws = vpa.paged_attention_workspace(len(lens), h, d, max_ctx, device)

    def step():
        vpa.paged_attention_plan(lens_d, max_ctx, dev_c[0]["bt"].shape[1], h, dev_c[0]["kc"],
                                 dev_c[0]["vc"], q.dtype, ws)
        for dc, o in zip(dev_c, outs):
            vpa.reshape_and_cache_paged_attention(q, k, v, None, None, dc["kc"], dc["vc"],
                                                  dc["bt"], lens_d, max_ctx, scale, out=o,
                                                  workspace=ws, planned=True)

    torch.cuda.synchronize()
    s = torch.cuda.Stream(device)
    with torch.cuda.stream(s):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            step()
    torch.cuda.synchronize()
    for rep in range(3):
        qn = random_words(rng, (len(lens), h, d), code)
        kn = random_words(rng, (len(lens), kvh, d), code)
        vn = random_words(rng, (len(lens), kvh, d), code)
        q.copy_(to_dev(qn, code, device))
        k.copy_(to_dev(kn, code, device))
        v.copy_(to_dev(vn, code, device))
        before = [(to_host(dc["kc"]), to_host(dc["vc"])) for dc in dev_c]
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for li, (dc, o) in enumerate(zip(dev_c, outs)):
            ref = dict(kc=before[li][0], vc=before[li][1], bt=cases[li]["bt"],
                       lens=np.asarray(lens, dtype=np.uint32), q=qn, k=kn, v=vn)
            want, wk, wv = two_calls(device, ref, code, bs, max_ctx, scale)
            np.testing.assert_array_equal(to_host(dc["kc"]), wk, err_msg=f"replay {rep} layer {li}")
            np.testing.assert_array_equal(to_host(dc["vc"]), wv, err_msg=f"replay {rep} layer {li}")
            np.testing.assert_array_equal(to_host(o), want, err_msg=f"replay {rep} layer {li}")
