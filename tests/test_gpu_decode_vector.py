"""paged_attention at the head-dim / block-size pairs of the reference's set
that no decode kernel takes (their (block, head) tiles are not whole 1 KiB
wave loads): 16-bit head dim 96 at 8-token blocks; fp8 caches at head dim 64
with 8-token blocks, 96 with 8 and 16, 192 with 8 under 16-bit queries; f32
queries over fp8 caches at 8-token blocks and at head dim 256 with 32. The
library runs them on the chunked-prefill vector kernel with one causal
query per sequence over its whole context and the decode's 1e-6 in the
denominator. Checked against the fp64 oracle of the decode
(attention.rs:243-286 semantics; fp8 elements f32(E4M3FN(byte) * scale)
rounded to the query type, as the reference dequantises) over the edges of
the 32-key tiles and of the blocks, empty contexts, stale NaN past every
context, scales, 1 to 8 query heads per kv head, the planned form, padded
table columns, graph replays against eager calls, and the fused append
entry point against its two calls."""

import numpy as np
import pytest
import torch

import vpa
from oracle import oracle as orc
from tests._util import (assert_attention_close, assert_attention_close_normwise,
                         block_tables_for, make_cache, random_words, to_dev, to_host, u32)
from tests.test_gpu_decode import decode_case
from tests.test_gpu_fp8 import fp8_decode_case
from tests.test_gpu_fused_append import case as fused_case
from tests.test_gpu_fused_append import fused, two_calls

pytestmark = pytest.mark.gpu

EDGES = [1, 7, 8, 9, 31, 32, 33, 255, 256, 257, 1000, 2049, 4100]


@pytest.mark.parametrize("code", [orc.BF16, orc.F16])
@pytest.mark.parametrize("h,kvh", [(16, 8), (8, 8), (24, 8), (64, 8)])
def test_decode_16bit_head_dim_96_block_8(device, code, h, kvh):
    got, want = decode_case(device, code, h, kvh, 96, 8, EDGES, seed=h + kvh + code)
    assert_attention_close(got, want, code, f"d=96 bs=8 code={code} h={h} kvh={kvh}")


def test_decode_16bit_head_dim_96_block_8_empty_and_stale_nan(device):
    """An empty context gives zeros; NaN past a context in its last block
    does not leak in."""
    rng = np.random.default_rng(5)
    code, d, bs = orc.BF16, 96, 8
    kc, vc = make_cache(rng, 16, 8, d, bs, code)
    bt = np.array([[3, 5, 0], [7, 0, 0], [9, 11, 13]], dtype=np.uint32)
    nan = 0x7FC0  # bf16 quiet NaN
    kc[5, :, :, 3:, :] = nan
    vc[5, :, :, 3:] = nan
    kc[13, :, :, 1:, :] = nan
    vc[13, :, :, 1:] = nan
    q = random_words(rng, (3, 16, d), code)
    lens = np.array([11, 0, 17], dtype=np.uint32)
    out = vpa.paged_attention(to_dev(q, code, device), None, None, to_dev(kc, code, device),
                              to_dev(vc, code, device), u32(bt, device), u32(lens, device), None,
                              24, d ** -0.5, 1.0, None)
    torch.cuda.synchronize()
    got = orc.to_f32(to_host(out), code)
    want = orc.paged_attention(q, kc, vc, bt, lens, 24, d ** -0.5, dtype=code)
    assert not got[1].any()
    assert_attention_close(got, want, code, "d=96 bs=8 empty / stale nan")


FP8_SHAPES_16 = [(64, 8), (96, 8), (96, 16), (192, 8)]
FP8_EDGES = [1, 7, 31, 32, 33, 511, 512, 513, 2047, 2049, 4097]


@pytest.mark.parametrize("d,bs", FP8_SHAPES_16)
@pytest.mark.parametrize("code,scales,planned", [(orc.BF16, (1.0, 1.0), False),
                                                 (orc.F16, (0.37, 3.1), True),
                                                 (orc.BF16, (0.6, 1.7), False)])
def test_decode_fp8_vector_shapes(device, d, bs, code, scales, planned):
    got, want = fp8_decode_case(device, code, 16, 8, d, bs, FP8_EDGES, seed=d + bs + 5 * code,
                                scales=scales, planned=planned)
    assert_attention_close(got, want, code, f"fp8 d={d} bs={bs} code={code} scales={scales}")


@pytest.mark.parametrize("d,bs", [(96, 16), (192, 8)])
@pytest.mark.parametrize("h,kvh", [(8, 8), (16, 4), (24, 8), (64, 8)])
def test_decode_fp8_vector_shapes_groups(device, d, bs, h, kvh):
    got, want = fp8_decode_case(device, orc.BF16, h, kvh, d, bs, [3, 64, 300, 2500],
                                seed=d + bs + h + kvh, scales=(0.5, 2.0))
    assert_attention_close(got, want, orc.BF16, f"fp8 d={d} bs={bs} h={h} kvh={kvh}")


@pytest.mark.parametrize("d,bs", [(64, 8), (128, 8), (256, 8), (256, 32)])
@pytest.mark.parametrize("scales,planned", [((1.0, 1.0), False), ((0.37, 3.1), True)])
def test_decode_fp8_f32_queries_vector_shapes(device, d, bs, scales, planned):
    """f32 queries over fp8 caches at the pairs the generic split-K kernel
    does not take, at rel 1e-5 against the oracle's same dequantisation."""
    got, want = fp8_decode_case(device, orc.F32, 16, 8, d, bs, FP8_EDGES, seed=d + bs + 17,
                                scales=scales, planned=planned)
    assert_attention_close(got, want, orc.F32, f"f32/fp8 d={d} bs={bs} scales={scales}")


@pytest.mark.parametrize("code,d,bs,fp8", [(orc.BF16, 96, 8, False), (orc.F16, 96, 16, True),
                                           (orc.BF16, 192, 8, True)])
def test_fused_append_on_vector_shapes_equals_two_calls(device, code, d, bs, fp8):
    """vpa_reshape_and_cache_paged_attention at these pairs (the append
    kernel, then the vector kernel) equals reshape_and_cache followed by
    paged_attention, caches and outputs bit for bit."""
    rng = np.random.default_rng(d + bs + code)
    lens = [1, 9, 33, 257, 1000]
    c = fused_case(rng, code, 16, 8, d, bs, lens, fp8=fp8)
    if fp8:
        c["k_scale"], c["v_scale"] = 0.8, 1.3
    max_ctx = int(max(lens))
    want = two_calls(device, c, code, bs, max_ctx, d ** -0.5)
    got = fused(device, c, code, max_ctx, d ** -0.5)
    for g, w, name in zip(got, want, ("out", "key_cache", "value_cache")):
        assert np.array_equal(g, w), f"{name} differs from the two calls"


# (query type, head dim, block size) of every decode pair served outside the
# rows kernel's fp8 / 16-bit instances: the vector kernel's pairs and the
# generic kernel's fp8 tiles under 16-bit queries
_FALLBACK = ([(c, 96, 8, False) for c in (orc.BF16, orc.F16)] +
             [(c, d, bs, True) for c in (orc.BF16, orc.F16)
              for d, bs in FP8_SHAPES_16 + [(192, 32), (256, 32)]] +
             [(orc.F32, d, bs, True) for d, bs in [(64, 8), (96, 8), (128, 8), (192, 8),
                                                   (256, 8), (256, 32)]])


@pytest.mark.parametrize("case", range(24))
def test_decode_fallback_random(device, case):
    """Seeded random draws over those pairs: query heads per kv head 1-8 (3
    and 6 included), 1-8 sequences with lengths up to 3000 and block edges,
    logit scales 0.5-1.5 of 1/sqrt(d), fp8 scales 0.3-1.5 and 0.2-3.0, against
    the fp64 oracle: element-wise for 16-bit queries (these paths round each
    dequantised fp8 element to the query type as the reference and the
    oracle do); normwise for f32 queries over fp8 caches, where outputs near
    zero are the residue of f32 sums over thousands of cancelling terms
    (seed 31005: head dim 256, k_scale 1.5, 1.8x the element-wise bound at
    about 1e-6 of the largest output)."""
    rng = np.random.default_rng(31000 + case)
    code, d, bs, fp8 = _FALLBACK[int(rng.integers(0, len(_FALLBACK)))]
    g = int(rng.choice([1, 2, 3, 4, 6, 8]))
    kvh = int(rng.choice([1, 2, 4, 8]))
    n = int(rng.integers(1, 9))
    lens = [int(v) for v in rng.integers(1, 3000, size=n)]
    k = int(rng.integers(0, n + 1))
    lens[:k] = [int(v) for v in rng.choice([1, bs - 1, bs, bs + 1, 31, 32, 33, 512, 2049], size=k)]
    lens = [max(1, v) for v in lens]
    scale = float(rng.uniform(0.5, 1.5)) * d ** -0.5
    what = f"case {case}: code={code} d={d} bs={bs} fp8={fp8} h={g * kvh} kvh={kvh} lens={lens}"
    if fp8:
        scales = (float(rng.uniform(0.3, 1.5)), float(rng.uniform(0.2, 3.0)))
        got, want = fp8_decode_case(device, code, g * kvh, kvh, d, bs, lens, seed=32000 + case,
                                    scales=scales, softmax_scale=scale)
        what += f" scales={scales}"
    else:
        got, want = decode_case(device, code, g * kvh, kvh, d, bs, lens, seed=32000 + case,
                                scale=scale)
    if fp8 and code == orc.F32:
        assert_attention_close_normwise(got, want, code, what)
    else:
        assert_attention_close(got, want, code, what)


def test_decode_vector_pair_padded_columns_and_larger_max_context(device):
    """max_context_len above every context and padded block-table columns
    (the graph-padding case) leave the result unchanged."""
    lens = [1, 9, 100, 1000]
    a, want = decode_case(device, orc.BF16, 16, 8, 96, 8, lens, seed=61)
    b, _ = decode_case(device, orc.BF16, 16, 8, 96, 8, lens, seed=61, pad_cols=40,
                       max_ctx=1000 + 40 * 8)
    assert np.array_equal(a, b)
    assert_attention_close(a, want, orc.BF16, "d=96 bs=8 padded")


@pytest.mark.parametrize("d,bs,fp8", [(96, 8, False), (256, 32, True)])
def test_decode_graph_replays_match_eager(device, d, bs, fp8):
    """paged_attention at a vector-kernel pair (head dim 96, 8-token blocks)
    and on the generic kernel's fp8 tiles (head dim 256, 32-token blocks,
    bf16 queries) captured in a HIP graph and replayed with new queries and
    longer contexts copied into the captured buffers (lengths crossing the
    generic kernel's partitions): every replay equals the eager call bit for
    bit."""
    rng = np.random.default_rng(71 + d)
    code, h, kvh = orc.BF16, 16, 8
    lens0 = np.array([5, 40, 333, 900], dtype=np.uint32)
    max_ctx = 1024
    nb = len(lens0) * (max_ctx // bs) + 8
    if fp8:
        kc = orc.fp8_from_f32((rng.standard_normal((nb, kvh, d // 16, bs, 16)) * 2)
                              .astype(np.float32))
        vc = orc.fp8_from_f32((rng.standard_normal((nb, kvh, d, bs)) * 2).astype(np.float32))
        kc_d = torch.from_numpy(kc).to(device).view(torch.float8_e4m3fn)
        vc_d = torch.from_numpy(vc).to(device).view(torch.float8_e4m3fn)
        ks = torch.tensor([0.8], dtype=torch.float32, device=device)
        vs = torch.tensor([1.3], dtype=torch.float32, device=device)
    else:
        kc, vc = make_cache(rng, nb, kvh, d, bs, code)
        kc_d, vc_d = to_dev(kc, code, device), to_dev(vc, code, device)
        ks = vs = None
    bt_d = u32(block_tables_for(rng, [max_ctx] * len(lens0), nb, bs), device)
    q_d = to_dev(random_words(rng, (len(lens0), h, d), code), code, device)
    ctx = u32(lens0, device)
    ws = vpa.paged_attention_workspace(len(lens0), h, d, max_ctx, device)
    out = torch.empty_like(q_d)

    def call(o):
        vpa.paged_attention(q_d, ks, vs, kc_d, vc_d, bt_d, ctx, None, max_ctx, d ** -0.5,
                            1.0, None, out=o, workspace=ws)

    call(out)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        call(out)
    torch.cuda.synchronize()
    for t in range(1, 5):
        q_d.copy_(to_dev(random_words(rng, (len(lens0), h, d), code), code, device))
        ctx.copy_(u32(np.minimum(lens0 + 50 * t, max_ctx), device))
        want = torch.empty_like(out)
        call(want)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), want.view(torch.int16)), f"replay {t}"
