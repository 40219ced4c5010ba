"""vpa_paged_attention_noalloc (the allocation-free decode entry point, whose
split-K scratch is a static device array of the library) against
vpa_paged_attention with a caller workspace, both called through the C ABI
on the same inputs: outputs equal bit for bit (the same kernels run; only
the scratch layout differs), on two calls in a row, the second with a
smaller batch and shorter contexts so that it runs over what the first left
in the array. The second call is also checked against the fp64 oracle.
Covered: the rows kernel with multi-chunk sequences (bf16, merge launch),
the fp8-cache rows kernel, the generic kernel (f32, 256-token partitions;
fp8 tiles under bf16 queries at head dim 256 with 32-token blocks), a pair
on the chunked-prefill vector kernel (head dim 96, 8-token blocks); calls
on two streams; the call captured in a HIP graph and replayed. The rejection of a call larger than the scratch happens on the
host before any device access and is tested in the CPU suite
(tests/test_abi.py), where no GPU exists for a wrong launch to reach."""

import numpy as np
import pytest
import torch

from oracle import oracle as orc
from tests._util import (assert_attention_close, block_tables_for, make_cache, random_words,
                         to_dev, to_host, u32)
from vpa import _lib

pytestmark = pytest.mark.gpu

H, KVH, D, BS = 16, 8, 128, 16


def case(rng, code, lens, cache_code=None, D=D, BS=BS):
    cache_code = code if cache_code is None else cache_code
    nb = sum((int(L) + BS - 1) // BS for L in lens) + 8
    if cache_code == orc.FP8 and code == orc.F32:
        # f32 queries are checked at rel 1e-5: codes of normal values (any
        # byte would reach +-448 and logits in the thousands, where f32 dot
        # products alone differ from the fp64 oracle by more)
        kc = orc.fp8_from_f32((rng.standard_normal((nb, KVH, D // 16, BS, 16)) * 2)
                              .astype(np.float32))
        vc = orc.fp8_from_f32((rng.standard_normal((nb, KVH, D, BS)) * 2).astype(np.float32))
    elif cache_code == orc.FP8:
        kc = rng.integers(0, 256, size=(nb, KVH, D // 16, BS, 16), dtype=np.uint8)
        vc = rng.integers(0, 256, size=(nb, KVH, D, BS), dtype=np.uint8)
        for c in (kc, vc):
            c[(c & 0x7F) == 0x7F] = 0x38  # no NaN codes
    else:
        kc, vc = make_cache(rng, nb, KVH, D, BS, cache_code)
    bt = block_tables_for(rng, lens, nb, BS)
    q = random_words(rng, (len(lens), H, D), code)
    return dict(q=q, kc=kc, vc=vc, bt=bt, lens=np.asarray(lens, dtype=np.uint32), nb=nb, D=D, BS=BS)


def dev_cache(a, cache_code, device):
    if cache_code == orc.FP8:
        return torch.from_numpy(a).to(device)
    return to_dev(a, cache_code, device)


def call(device, c, code, cache_code, noalloc, max_ctx):
    """One decode through the C ABI; returns the output words on the host."""
    lib = _lib.load()
    dt = {orc.F32: _lib.DTYPE_F32, orc.BF16: _lib.DTYPE_BF16, orc.F16: _lib.DTYPE_F16}[code]
    cdt = _lib.DTYPE_FP8_E4M3 if cache_code == orc.FP8 else dt
    q = to_dev(c["q"], code, device)
    kc, vc = dev_cache(c["kc"], cache_code, device), dev_cache(c["vc"], cache_code, device)
    bt, lens = u32(c["bt"], device), u32(c["lens"], device)
    out = torch.full_like(q, float("nan"))
    one = torch.ones(1, dtype=torch.float32, device=device)
    ks = one.data_ptr() if cache_code == orc.FP8 else None
    b = len(c["lens"])
    D, BS = c["D"], c["BS"]
    stride_b, stride_h = kc.stride(0), kc.stride(1)
    stream = torch.cuda.current_stream(device).cuda_stream
    common = (out.data_ptr(), q.data_ptr(), ks, ks, kc.data_ptr(), vc.data_ptr(), bt.data_ptr(),
              bt.shape[1], lens.data_ptr(), None, max_ctx, D ** -0.5, 1.0, None, b, H, KVH, D, BS,
              c["nb"], stride_b, stride_h, dt, cdt)
    torch.cuda.synchronize()
    if noalloc:
        rc = lib.vpa_paged_attention_noalloc(*common, stream)
    else:
        n = lib.vpa_paged_attention_workspace_size(b, H, D, max_ctx)
        ws = torch.empty(n, dtype=torch.uint8, device=device)
        rc = lib.vpa_paged_attention(*common, ws.data_ptr(), n, stream)
    assert rc == 0, lib.vpa_last_error().decode()
    torch.cuda.synchronize()
    return to_host(out)


@pytest.mark.parametrize("code,cache_code,d,bs", [
    (orc.BF16, orc.BF16, D, BS), (orc.BF16, orc.FP8, D, BS), (orc.F32, orc.F32, D, BS),
    (orc.F32, orc.FP8, D, BS),
    # the generic split-K kernel over fp8 tiles under 16-bit queries, and a
    # pair on the chunked-prefill vector kernel (no scratch used)
    (orc.BF16, orc.FP8, 256, 32), (orc.BF16, orc.BF16, 96, 8)])
def test_noalloc_equals_workspace_entry_point_twice(device, code, cache_code, d, bs):
    rng = np.random.default_rng(31 + code + 7 * cache_code + d + bs)
    first = [int(x) for x in rng.integers(1, 4500, size=40)]
    first[:4] = [4096, 2049, 2048, 1]  # multi-chunk and single-chunk rows
    second = [int(x) for x in rng.integers(1, 1500, size=17)]
    for lens in (first, second):
        c = case(rng, code, lens, cache_code, d, bs)
        max_ctx = int(max(lens))
        got = call(device, c, code, cache_code, True, max_ctx)
        want = call(device, c, code, cache_code, False, max_ctx)
        assert np.array_equal(got, want), f"batch {len(lens)}: noalloc differs from workspace call"
        assert np.all(np.isfinite(orc.to_f32(got, code)))
    # the second (smaller) call against the oracle
    ref = orc.paged_attention(c["q"], c["kc"], c["vc"], c["bt"], c["lens"], max_ctx, d ** -0.5,
                              dtype=code, kv_dtype=orc.FP8 if cache_code == orc.FP8 else None)
    assert_attention_close(orc.to_f32(got, code), ref, code, "noalloc second call")



def test_noalloc_calls_on_two_streams_are_ordered(device):
    """A large call on one stream and a small one on another, issued back to
    back with no synchronisation between them, both on the one scratch array:
    each equals the workspace entry point's result (the library makes the
    second call's stream wait for the first call)."""
    lib = _lib.load()
    rng = np.random.default_rng(77)
    big = [int(x) for x in rng.integers(2000, 4500, size=256)]
    small = [int(x) for x in rng.integers(1000, 3000, size=16)]
    cases = [case(rng, orc.BF16, big), case(rng, orc.BF16, small)]
    want = [call(device, c, orc.BF16, orc.BF16, False, int(max(c["lens"]))) for c in cases]
    args = []
    for c in cases:
        q = to_dev(c["q"], orc.BF16, device)
        kc, vc = dev_cache(c["kc"], orc.BF16, device), dev_cache(c["vc"], orc.BF16, device)
        bt, lens = u32(c["bt"], device), u32(c["lens"], device)
        out = torch.full_like(q, float("nan"))
        args.append((out, q, kc, vc, bt, lens, c))
    streams = [torch.cuda.Stream(device), torch.cuda.Stream(device)]
    torch.cuda.synchronize()
    for (out, q, kc, vc, bt, lens, c), st in zip(args, streams):
        b = len(c["lens"])
        rc = lib.vpa_paged_attention_noalloc(
            out.data_ptr(), q.data_ptr(), None, None, kc.data_ptr(), vc.data_ptr(), bt.data_ptr(),
            bt.shape[1], lens.data_ptr(), None, int(max(c["lens"])), D ** -0.5, 1.0, None, b, H,
            KVH, D, BS, c["nb"], kc.stride(0), kc.stride(1), _lib.DTYPE_BF16, _lib.DTYPE_BF16,
            st.cuda_stream)
        assert rc == 0, lib.vpa_last_error().decode()
    torch.cuda.synchronize()
    for (out, *_), w in zip(args, want):
        assert np.array_equal(to_host(out), w), "a call on the other stream changed the result"


def test_noalloc_captured_in_a_graph_matches_eager(device):
    """The allocation-free decode recorded in a HIP graph (what the entry
    point is for: it makes no allocation under capture), replayed four
    times with new queries and longer contexts copied into the captured
    buffers, eager work and synchronisation between replays: every replay
    equals the workspace entry point run eagerly on the same inputs, bit for
    bit, and the last one the fp64 oracle."""
    lib = _lib.load()
    rng = np.random.default_rng(53)
    lens0 = np.array([int(x) for x in rng.integers(1, 3000, size=24)])
    lens0[:3] = [2047, 2048, 4000]  # multi-chunk rows at the later steps: the merge launch
    max_ctx = 4096
    c = case(rng, orc.BF16, [max_ctx] * len(lens0))
    b = len(lens0)
    q = to_dev(c["q"], orc.BF16, device)
    kc, vc = dev_cache(c["kc"], orc.BF16, device), dev_cache(c["vc"], orc.BF16, device)
    bt = u32(c["bt"], device)
    lens = u32(lens0.astype(np.uint32), device)
    out = torch.full_like(q, float("nan"))

    def decode(stream):
        rc = lib.vpa_paged_attention_noalloc(
            out.data_ptr(), q.data_ptr(), None, None, kc.data_ptr(), vc.data_ptr(), bt.data_ptr(),
            bt.shape[1], lens.data_ptr(), None, max_ctx, D ** -0.5, 1.0, None, b, H, KVH, D, BS,
            c["nb"], kc.stride(0), kc.stride(1), _lib.DTYPE_BF16, _lib.DTYPE_BF16, stream)
        assert rc == 0, lib.vpa_last_error().decode()

    decode(torch.cuda.current_stream(device).cuda_stream)  # set-up and warm-up, before capture
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        decode(torch.cuda.current_stream(device).cuda_stream)
    torch.cuda.synchronize()
    for t in range(1, 5):
        c["q"] = random_words(rng, (b, H, D), orc.BF16)
        c["lens"] = np.minimum(lens0 + 37 * t, max_ctx).astype(np.uint32)
        q.copy_(to_dev(c["q"], orc.BF16, device))
        lens.copy_(u32(c["lens"], device))
        want = call(device, c, orc.BF16, orc.BF16, False, max_ctx)  # eager, with a workspace
        out.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        got = to_host(out)
        assert np.array_equal(got, want), f"replay {t} differs from the eager call"
    ref = orc.paged_attention(c["q"], c["kc"], c["vc"], c["bt"], c["lens"], max_ctx, D ** -0.5,
                              dtype=orc.BF16)
    assert_attention_close(orc.to_f32(got, orc.BF16), ref, orc.BF16, "noalloc graph replay")
