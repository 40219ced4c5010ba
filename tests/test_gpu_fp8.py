"""GPU parity of the FP8 (E4M3FN) KV cache against the CPU oracle.

* reshape_and_cache into an fp8 cache: bit-exact bytes against the oracle's
  encode (round to nearest even of x / scale, saturation at 448, NaN kept),
  for f32 / f16 / bf16 rows, scale 1 and others, decode and prefill slot
  patterns;
* gather_kv_cache out of an fp8 cache holding every one of the 256 codes:
  bit-exact against the oracle's dequantisation byte * scale for f32, f16
  and bf16 outputs (this pins the device conversion instructions the decode
  kernel shares);
* paged_attention over an fp8 cache: the fp64 oracle over the dequantised
  cache (the reference's fp8 semantics, prefill_paged_attn.metal:698-769),
  bf16/f16 tolerance 2e-2, with stale NaN bytes past each context;
* chunked prefill over an fp8 cache: the fp64 oracle (causal and not,
  scales, absent blocks, NaN bytes in every unused slot), and with scales 1
  bit-equal to the bf16 kernel over a bf16 copy of the cache (also at c4's
  full size).
"""

import numpy as np
import pytest
import torch

import vpa
from oracle import oracle as orc
from tests._util import (TORCH, assert_attention_close, block_tables_for, i64, random_words,
                         to_dev, to_host, u32)

pytestmark = pytest.mark.gpu


def f8(a: np.ndarray, device) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.uint8)).to(device).view(
        torch.float8_e4m3fn)


def f8_host(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().view(torch.uint8).numpy()


def scalar(v: float, device) -> torch.Tensor:
    return torch.tensor([v], dtype=torch.float32, device=device)


def spread_values(rng, shape):
    """Normal values with a tail of large (saturating), tiny (subnormal in
    E4M3) and special values."""
    x = (rng.standard_normal(shape) * 20).astype(np.float32)
    flat = x.reshape(-1)
    n = flat.size
    idx = rng.choice(n, size=max(n // 50, 8), replace=False)
    flat[idx[0::4]] = (rng.standard_normal(len(idx[0::4])) * 1000).astype(np.float32)
    flat[idx[1::4]] = (rng.standard_normal(len(idx[1::4])) * 1e-3).astype(np.float32)
    flat[idx[2]] = np.inf
    flat[idx[3]] = -np.inf
    flat[idx[5]] = np.nan
    return x


@pytest.mark.parametrize("code", [orc.BF16, orc.F16, orc.F32])
@pytest.mark.parametrize("scales", [(1.0, 1.0), (0.37, 3.1)])
@pytest.mark.parametrize("pattern", ["decode", "prefill"])
def test_fp8_append_bit_exact(device, code, scales, pattern):
    rng = np.random.default_rng(100 * code + int(10 * scales[0]) + (pattern == "decode"))
    kvh, d, bs, nb = 8, 128, 16, 64
    ks, vs = scales
    kc = rng.integers(0, 256, size=(nb, kvh, d // 16, bs, 16), dtype=np.uint8)
    vc = rng.integers(0, 256, size=(nb, kvh, d, bs), dtype=np.uint8)
    if pattern == "decode":  # one token per sequence, each alone in its block
        t = 40
        slots = rng.choice(nb, size=t, replace=False).astype(np.int64) * bs + rng.integers(
            0, bs, size=t)
        slots[::7] = -1  # padding rows
    else:  # runs through blocks, not block-aligned
        t = 5 * bs + 3
        blocks = rng.choice(nb, size=7, replace=False)
        pos = np.arange(t) + 5
        slots = blocks[pos // bs].astype(np.int64) * bs + pos % bs
    kf = spread_values(rng, (t, kvh, d))
    vf = spread_values(rng, (t, kvh, d))
    k = kf if code == orc.F32 else orc.from_f32(kf, code)
    v = vf if code == orc.F32 else orc.from_f32(vf, code)
    kcd, vcd = f8(kc, device), f8(vc, device)
    vpa.reshape_and_cache(to_dev(k, code, device), to_dev(v, code, device), scalar(ks, device),
                          scalar(vs, device), kcd, vcd, i64(slots, device))
    torch.cuda.synchronize()
    orc.reshape_and_cache_fp8(k, v, kc, vc, slots, code, ks, vs)
    np.testing.assert_array_equal(f8_host(kcd), kc)
    np.testing.assert_array_equal(f8_host(vcd), vc)


@pytest.mark.parametrize("out", [orc.F32, orc.F16, orc.BF16])
@pytest.mark.parametrize("scales", [(1.0, 1.0), (0.5, 3.0)])
def test_fp8_gather_every_code_bit_exact(device, out, scales):
    ks, vs = scales
    rng = np.random.default_rng(11 + out)
    kvh, d, bs, nb = 2, 128, 16, 24
    # every byte value appears in both caches
    kc = rng.permutation(np.resize(np.arange(256, dtype=np.uint8), nb * kvh * d * bs)).reshape(
        nb, kvh, d // 16, bs, 16)
    vc = rng.permutation(np.resize(np.arange(256, dtype=np.uint8), nb * kvh * d * bs)).reshape(
        nb, kvh, d, bs)
    lens = np.array([37, 1, 16, 130], dtype=np.uint32)
    bt = block_tables_for(rng, lens, nb, bs)
    bt[1, 0] = nb + 5  # an absent block gives zero rows
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.uint32)
    gk, gv = vpa.gather_kv_cache(f8(kc, device), f8(vc, device), scalar(ks, device),
                                 scalar(vs, device), u32(bt, device), u32(cu, device), TORCH[out])
    torch.cuda.synchronize()
    wk, wv = orc.gather_kv_cache_fp8(kc, vc, bt, cu, out, ks, vs)
    for got, want in ((to_host(gk), wk), (to_host(gv), wv)):
        gf = got if out == orc.F32 else orc.to_f32(got, out)
        wf = want if out == orc.F32 else orc.to_f32(want, out)
        assert np.array_equal(np.isnan(gf), np.isnan(wf))
        fin = ~np.isnan(wf)
        np.testing.assert_array_equal(got[fin], want[fin])


def fp8_decode_case(device, code, h, kvh, d, bs, lens, seed, scales=(1.0, 1.0), planned=False,
                    softmax_scale=None):
    rng = np.random.default_rng(seed)
    ks, vs = scales
    need = sum((int(L) + bs - 1) // bs for L in lens)
    nb = need + 8
    kc = orc.fp8_from_f32((rng.standard_normal((nb, kvh, d // 16, bs, 16)) * 2).astype(np.float32))
    vc = orc.fp8_from_f32((rng.standard_normal((nb, kvh, d, bs)) * 2).astype(np.float32))
    bt = block_tables_for(rng, [max(int(L), 1) for L in lens], nb, bs)
    # stale NaN bytes past every context in its last block
    for s, L in enumerate(lens):
        if L % bs:
            blk = bt[s, (L - 1) // bs]
            kc[blk, :, :, L % bs:, :] = 0x7F
            vc[blk, :, :, L % bs:] = 0x7F
    q = random_words(rng, (len(lens), h, d), code)
    lens = np.asarray(lens, dtype=np.uint32)
    max_ctx = int(lens.max())
    scale = d ** -0.5 if softmax_scale is None else softmax_scale
    args = (to_dev(q, code, device), scalar(ks, device), scalar(vs, device), f8(kc, device),
            f8(vc, device), u32(bt, device), u32(lens, device), None, max_ctx, scale, 1.0, None)
    if planned:
        ws = vpa.paged_attention_workspace(len(lens), h, d, max_ctx, device)
        vpa.paged_attention_plan(args[6], max_ctx, bt.shape[1], h, args[3], args[4], TORCH[code],
                                 ws)
        out = vpa.paged_attention(*args, workspace=ws, planned=True)
    else:
        out = vpa.paged_attention(*args)
    torch.cuda.synchronize()
    want = orc.paged_attention(q, kc, vc, bt, lens, max_ctx, scale, dtype=code,
                               kv_dtype=orc.FP8, k_scale=ks, v_scale=vs)
    return orc.to_f32(to_host(out), code), want


@pytest.mark.parametrize("code", [orc.BF16, orc.F16])
@pytest.mark.parametrize("bs", [16, 32])
def test_fp8_decode_qwen3_asr_shape(device, code, bs):
    lens = [1, 2, 15, 16, 17, 100, 255, 256, 257, 1023, 1024, 1025, 2600]
    got, want = fp8_decode_case(device, code, 16, 8, 128, bs, lens, seed=bs + code)
    assert_attention_close(got, want, code, f"fp8 code={code} bs={bs}")


@pytest.mark.parametrize("bs", [16, 32])
def test_fp8_decode_chunk_and_wave_boundaries(device, bs):
    """Lengths at the per-wave (512-token) and per-chunk (2048-token)
    boundaries of the rows kernel, merges of up to 4 chunks."""
    lens = [1, 511, 512, 513, 2047, 2048, 2049, 4095, 4096, 4097, 6145, 8191]
    got, want = fp8_decode_case(device, orc.BF16, 16, 8, 128, bs, lens, seed=200 + bs)
    assert_attention_close(got, want, orc.BF16, f"fp8 edges bs={bs}")


@pytest.mark.parametrize("factor", [2.0, 3.0, 10.0])
@pytest.mark.parametrize("code", [orc.F16, orc.BF16])
def test_fp8_decode_large_logit_scales(device, factor, code):
    """Logit scales of 2, 3 and 10 times 1/sqrt(head_dim) over the chunk and
    wave edges, f16 and bf16 queries: element-wise bound (worst 0.21 of it)."""
    lens = [1, 511, 512, 513, 2047, 2048, 2049, 4097, 6145]
    got, want = fp8_decode_case(device, code, 16, 8, 128, 16, lens, seed=400 + int(factor) + code,
                                softmax_scale=factor * 128 ** -0.5)
    assert_attention_close(got, want, code, f"fp8 scale x{factor} code={code}")


@pytest.mark.parametrize("h,kvh", [(64, 8), (24, 8)])
@pytest.mark.parametrize("code", [orc.BF16, orc.F16])
def test_fp8_decode_query_heads_per_kv_head(device, h, kvh, code):
    """8 and 3 query heads per kv head over an fp8 cache with scales."""
    got, want = fp8_decode_case(device, code, h, kvh, 128, 16, [1, 300, 2049, 4097],
                                seed=h + kvh + code, scales=(0.6, 1.7))
    assert_attention_close(got, want, code, f"fp8 h={h} kvh={kvh} code={code}")


def test_fp8_decode_longest_supported_context(device):
    """A 262 144-token context over an fp8 cache (the longest the decode
    takes: 128 chunks merged) beside a one-token sequence, with scales."""
    lens = [262144, 1]
    got, want = fp8_decode_case(device, orc.BF16, 2, 1, 128, 16, lens, seed=93,
                                scales=(0.6, 1.7))
    assert_attention_close(got, want, orc.BF16, "fp8 longest context")


@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("h,kvh", [(8, 8), (16, 8), (16, 4)])
def test_fp8_decode_head_dims_and_groups(device, d, h, kvh):
    got, want = fp8_decode_case(device, orc.BF16, h, kvh, d, 16, [3, 64, 300, 1500],
                                seed=d + h + kvh)
    assert_attention_close(got, want, orc.BF16, f"fp8 d={d} h={h} kvh={kvh}")


# wave and chunk edges of the rows kernel (merges of 2 to 4 chunks)
FP8_EDGES = [1, 7, 511, 512, 513, 2047, 2048, 2049, 4097, 6145]


@pytest.mark.parametrize("d,bs", [(96, 32), (192, 16), (256, 8), (256, 16), (192, 32),
                                  (256, 32)])
@pytest.mark.parametrize("code,scales,planned", [(orc.BF16, (1.0, 1.0), False),
                                                 (orc.F16, (0.37, 3.1), True)])
def test_fp8_decode_head_dims_96_192_256(device, d, bs, code, scales, planned):
    """fp8 caches at head dims 96 (32-token blocks), 192 (16) and 256 (8 and
    16; at 8 a value unit holds two dims of the block's 8 tokens) on the rows
    kernel, 192 and 256 at 32-token blocks on the generic split-K kernel,
    with and without scales, planned and not, over the wave, chunk and
    partition edges."""
    got, want = fp8_decode_case(device, code, 16, 8, d, bs, FP8_EDGES, seed=d + bs + code,
                                scales=scales, planned=planned)
    assert_attention_close(got, want, code, f"fp8 d={d} bs={bs} code={code}")


@pytest.mark.parametrize("d", [192, 256])
@pytest.mark.parametrize("code,scales", [(orc.BF16, (0.6, 1.7)), (orc.BF16, (0.37, 3.1)),
                                         (orc.F16, (1.9, 0.45))])
def test_fp8_decode_generic_kernel_rounds_like_the_reference(device, d, code, scales):
    """16-bit queries over fp8 caches at 32-token blocks (head dims 192 and
    256, the generic split-K kernel): each element is dequantised as the
    reference does, f32(E4M3FN(byte) * scale) rounded to the query type, so
    non-unit scales stay within the element-wise bound against the fp64
    oracle's same dequantisation (bf16 included)."""
    got, want = fp8_decode_case(device, code, 16, 8, d, 32, FP8_EDGES, seed=d + 7 * code + 3,
                                scales=scales, planned=False)
    assert_attention_close(got, want, code, f"fp8 generic d={d} code={code} scales={scales}")


@pytest.mark.parametrize("d,bs", [(96, 32), (256, 16), (256, 32)])
@pytest.mark.parametrize("h,kvh", [(8, 8), (16, 4), (64, 8)])
def test_fp8_decode_head_dims_groups(device, d, bs, h, kvh):
    got, want = fp8_decode_case(device, orc.BF16, h, kvh, d, bs, [3, 64, 300, 2500],
                                seed=d + h + kvh + bs)
    assert_attention_close(got, want, orc.BF16, f"fp8 d={d} bs={bs} h={h} kvh={kvh}")


@pytest.mark.parametrize("d,bs", [(64, 16), (96, 32), (128, 16), (128, 32), (192, 16),
                                  (192, 32), (256, 16)])
@pytest.mark.parametrize("scales,planned", [((1.0, 1.0), False), ((0.37, 3.1), True)])
def test_fp8_decode_f32_queries(device, d, bs, scales, planned):
    """f32 queries over fp8 caches (the generic split-K kernel: each element
    read as f32(E4M3FN(byte) * scale), rel 1e-5 against the fp64 oracle's same
    dequantisation) over the 128-token partitions and the merge of many."""
    got, want = fp8_decode_case(device, orc.F32, 16, 8, d, bs, FP8_EDGES, seed=d + bs + 11,
                                scales=scales, planned=planned)
    assert_attention_close(got, want, orc.F32, f"f32/fp8 d={d} bs={bs} scales={scales}")


@pytest.mark.parametrize("h,kvh", [(8, 8), (16, 4), (24, 8), (64, 8)])
def test_fp8_decode_f32_queries_groups(device, h, kvh):
    got, want = fp8_decode_case(device, orc.F32, h, kvh, 128, 16, [1, 5, 128, 129, 700, 3000],
                                seed=h + kvh + 13, scales=(0.5, 2.0))
    assert_attention_close(got, want, orc.F32, f"f32/fp8 h={h} kvh={kvh}")


@pytest.mark.parametrize("planned", [False, True])
@pytest.mark.parametrize("h,kvh", [(16, 8), (16, 4)])
def test_fp8_decode_block_size_8(device, h, kvh, planned):
    """8-token blocks (paged_cache_runtime.rs:406-411 allows 8, 16, 32 for
    any cache type): a 16-byte value vector then holds two dims of the
    block's 8 tokens. Lengths across wave and chunk boundaries, stale NaN
    bytes past each context."""
    lens = [1, 7, 8, 9, 511, 512, 513, 2047, 2049, 3000]
    got, want = fp8_decode_case(device, orc.BF16, h, kvh, 128, 8, lens, seed=h + kvh + planned,
                                scales=(0.37, 3.1), planned=planned)
    assert_attention_close(got, want, orc.BF16, f"fp8 bs=8 h={h} kvh={kvh}")


@pytest.mark.parametrize("scales", [(0.37, 3.1), (4.0, 0.25)])
def test_fp8_decode_scales_and_planned(device, scales):
    lens = [5, 700, 1100, 2049]
    got, want = fp8_decode_case(device, orc.BF16, 16, 8, 128, 16, lens, seed=77, scales=scales,
                                planned=True)
    assert_attention_close(got, want, orc.BF16, f"fp8 scales={scales}")


def test_fp8_append_then_decode_end_to_end(device):
    """bf16 rows appended into an fp8 cache and attended: the same as the
    oracle's append followed by its fp8 attention."""
    rng = np.random.default_rng(3)
    h, kvh, d, bs = 16, 8, 128, 16
    lens = [1, 33, 500, 1030]
    nb = sum((L + bs - 1) // bs for L in lens) + 4
    kc = np.zeros((nb, kvh, d // 16, bs, 16), np.uint8)
    vc = np.zeros((nb, kvh, d, bs), np.uint8)
    bt = block_tables_for(rng, lens, nb, bs)
    slots = np.concatenate([bt[s, np.arange(L) // bs].astype(np.int64) * bs + np.arange(L) % bs
                            for s, L in enumerate(lens)])
    tot = int(sum(lens))
    k = random_words(rng, (tot, kvh, d), orc.BF16)
    v = random_words(rng, (tot, kvh, d), orc.BF16)
    kcd, vcd = f8(kc, device), f8(vc, device)
    one = scalar(1.0, device)
    vpa.reshape_and_cache(to_dev(k, orc.BF16, device), to_dev(v, orc.BF16, device), one, one,
                          kcd, vcd, i64(slots, device))
    q = random_words(rng, (len(lens), h, d), orc.BF16)
    out = vpa.paged_attention(to_dev(q, orc.BF16, device), one, one, kcd, vcd, u32(bt, device),
                              u32(lens, device), None, max(lens), d ** -0.5, 1.0, None)
    torch.cuda.synchronize()
    orc.reshape_and_cache_fp8(k, v, kc, vc, slots, orc.BF16, 1.0, 1.0)
    np.testing.assert_array_equal(f8_host(kcd), kc)
    want = orc.paged_attention(q, kc, vc, bt, np.array(lens), max(lens), d ** -0.5,
                               dtype=orc.BF16, kv_dtype=orc.FP8)
    assert_attention_close(orc.to_f32(to_host(out), orc.BF16), want, orc.BF16, "fp8 e2e")


# ---- chunked prefill over an fp8 cache ----------------------------------------

def fp8_prefill_case(device, code, h, kvh, bs, prior, qlens, seed, causal=True,
                     scales=(1.0, 1.0), mutate_bt=None, d=128):
    """Random fp8 caches with NaN bytes (0x7F) in every slot no sequence
    holds; returns (kernel output as f32, fp64 oracle, inputs)."""
    rng = np.random.default_rng(seed)
    ks, vs = scales
    prior = np.asarray(prior, dtype=np.int64)
    qlens = np.asarray(qlens, dtype=np.int64)
    lens = prior + qlens
    nb = int(sum((int(L) + bs - 1) // bs for L in lens)) + 6
    kc = orc.fp8_from_f32((rng.standard_normal((nb, kvh, d // 16, bs, 16)) * 2).astype(np.float32))
    vc = orc.fp8_from_f32((rng.standard_normal((nb, kvh, d, bs)) * 2).astype(np.float32))
    bt = block_tables_for(rng, [max(int(L), 1) for L in lens], nb, bs)
    used = np.zeros((nb, bs), dtype=bool)
    for s, L in enumerate(lens):
        t = np.arange(int(L))
        used[bt[s, t // bs], t % bs] = True
    kc[~used[:, None, None, :, None].repeat(kvh, 1).repeat(d // 16, 2).repeat(16, 4)] = 0x7F
    vc[~used[:, None, None, :].repeat(kvh, 1).repeat(d, 2)] = 0x7F
    if mutate_bt is not None:
        mutate_bt(bt)
    q = random_words(rng, (int(qlens.sum()), h, d), code)
    cu = np.concatenate([[0], np.cumsum(qlens)]).astype(np.uint32)
    lens32 = lens.astype(np.uint32)
    scale = d ** -0.5
    out = vpa.paged_attention_varlen_prefill(
        to_dev(q, code, device), f8(kc, device), f8(vc, device), u32(bt, device),
        u32(lens32, device), u32(cu, device), scalar(ks, device), scalar(vs, device), scale, 1.0,
        causal=causal)
    torch.cuda.synchronize()
    want = orc.prefill_attention(q, kc, vc, bt, lens32, cu, scale, causal=causal, dtype=code,
                                 kv_dtype=orc.FP8, k_scale=ks, v_scale=vs)
    return orc.to_f32(to_host(out), code), want, (q, kc, vc, bt, lens32, cu, scale)


@pytest.mark.parametrize("bs", [8, 16])
def test_fp8_prefill_long_context(device, bs):
    """16 000 prior tokens over an fp8 cache: four-tile steps walked ~125
    times at 16-token blocks, per-step block-id loads at 8-token blocks."""
    got, want, _ = fp8_prefill_case(device, orc.BF16, 16, 8, bs, [16000, 40], [160, 24],
                                    seed=33)
    assert_attention_close(got, want, orc.BF16, f"fp8 prefill long context bs={bs}")


PF_PRIOR = [0, 5, 31, 100, 0, 333]
PF_NEW = [1, 31, 32, 33, 129, 70]


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("bs", [16, 32])
@pytest.mark.parametrize("code", [orc.BF16, orc.F16])
def test_fp8_prefill_qwen3_asr_shape(device, code, bs, causal):
    got, want, _ = fp8_prefill_case(device, code, 16, 8, bs, PF_PRIOR, PF_NEW,
                                    seed=3 * bs + code + causal, causal=causal)
    assert_attention_close(got, want, code, f"fp8 prefill code={code} bs={bs} causal={causal}")


@pytest.mark.parametrize("h,kvh", [(8, 8), (16, 4)])
def test_fp8_prefill_groups(device, h, kvh):
    got, want, _ = fp8_prefill_case(device, orc.BF16, h, kvh, 16, [7, 0, 260], [40, 65, 17],
                                    seed=h + kvh)
    assert_attention_close(got, want, orc.BF16, f"fp8 prefill h={h} kvh={kvh}")


@pytest.mark.parametrize("scales", [(0.37, 3.1), (4.0, 0.25), (-0.5, 1.5)])
def test_fp8_prefill_scales(device, scales):
    """k_scale folds into the softmax scale (a negative one flips which key
    dominates), v_scale into the output."""
    got, want, _ = fp8_prefill_case(device, orc.BF16, 16, 8, 16, [300, 0, 45], [90, 200, 1],
                                    seed=int(10 * scales[0]) + 60, scales=scales)
    assert_attention_close(got, want, orc.BF16, f"fp8 prefill scales={scales}")


def test_fp8_prefill_absent_blocks(device):
    def mutate(bt):
        bt[0, 1] = 1 << 30     # out of the pool: its tokens are absent
        bt[1, 0] = 0xFFFFFFFF
    got, want, _ = fp8_prefill_case(device, orc.BF16, 16, 8, 16, [40, 20], [30, 50], seed=15,
                                    mutate_bt=mutate)
    assert_attention_close(got, want, orc.BF16, "fp8 prefill absent blocks")


@pytest.mark.parametrize("col", [2, 4, 7])
def test_fp8_prefill_absent_block_in_either_tile_of_a_step(device, col):
    """An absent block in the second tile of step 0 (column 2), the first of
    step 1 (column 4) or the second of step 1 (column 7) of the two-tile
    steps; block 0, read in its place, holds NaN bytes in every slot no
    sequence uses: its values must be zeroed bytewise in either tile."""
    def mutate(bt):
        bt[0, col] = 1 << 30
    got, want, _ = fp8_prefill_case(device, orc.BF16, 16, 8, 16, [100, 60], [40, 50],
                                    seed=40 + col, mutate_bt=mutate)
    assert np.isfinite(got).all()
    assert_attention_close(got, want, orc.BF16, f"fp8 prefill absent column {col}")


@pytest.mark.parametrize("col", [17, 29])
def test_fp8_prefill_absent_block_in_a_later_step(device, col):
    """Four-tile steps of 8 blocks: an absent block in step 2 (column 17) or
    step 3 (column 29), whose ids come from the window loaded two steps
    ahead; the step works its mask out from its ids loaded again."""
    def mutate(bt):
        bt[0, col] = 1 << 30
    got, want, _ = fp8_prefill_case(device, orc.BF16, 16, 8, 16, [500, 60], [40, 50],
                                    seed=50 + col, mutate_bt=mutate)
    assert np.isfinite(got).all()
    assert_attention_close(got, want, orc.BF16, f"fp8 prefill absent column {col}")


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("bs", [16, 32])
def test_fp8_prefill_head_dim_64(device, bs, causal):
    got, want, _ = fp8_prefill_case(device, orc.BF16, 16, 8, bs, PF_PRIOR, PF_NEW,
                                    seed=70 + bs + causal, causal=causal, d=64)
    assert np.isfinite(got).all()
    assert_attention_close(got, want, orc.BF16, f"fp8 prefill d=64 bs={bs} causal={causal}")


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("d,bs", [(96, 32), (192, 16), (192, 32), (256, 16), (256, 32)])
def test_fp8_prefill_head_dims(device, d, bs, causal):
    """The Metal prefill's other head dims (varlen_prefill.rs:15) over fp8
    caches (head_dim 96 needs 32-token blocks at fp8)."""
    got, want, _ = fp8_prefill_case(device, orc.BF16, 16, 8, bs, PF_PRIOR, PF_NEW,
                                    seed=d + bs + causal, causal=causal, d=d,
                                    scales=(0.37, 3.1))
    assert np.isfinite(got).all()
    assert_attention_close(got, want, orc.BF16, f"fp8 prefill d={d} bs={bs} causal={causal}")


@pytest.mark.parametrize("code", [orc.BF16, orc.F16])
@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("d", [128, 256])
def test_fp8_prefill_block_size_8(device, d, causal, code):
    """fp8 caches at 8-token blocks: each value unit holds two dims of a
    block's keys, copied to LDS as is; absent blocks and NaN bytes in every
    unused slot."""
    def mutate(bt):
        bt[3, 2] = 1 << 30  # an absent block inside sequence 3's context
    got, want, _ = fp8_prefill_case(device, code, 16, 8, 8, PF_PRIOR, PF_NEW,
                                    seed=d + causal + code, causal=causal, d=d,
                                    scales=(0.37, 3.1), mutate_bt=mutate)
    assert np.isfinite(got).all()
    assert_attention_close(got, want, code, f"fp8 prefill bs=8 d={d} causal={causal}")


def test_fp8_prefill_block_size_8_equals_bf16_over_dequantised_cache(device):
    """Scales 1 at 8-token blocks: bit-equal to the bf16 kernel over a bf16
    copy of the cache (the two-dims-per-unit value layout feeds the MFMAs
    the same operands)."""
    code, h, kvh, bs = orc.BF16, 16, 8, 8
    got, _, (q, kc, vc, bt, lens, cu, scale) = fp8_prefill_case(
        device, code, h, kvh, bs, [0, 17, 500], [64, 33, 90], seed=23, d=128)
    nb, _, c16, _, _ = kc.shape
    d = c16 * 16
    kf = orc.fp8_to_f32(kc).transpose(0, 1, 3, 2, 4).reshape(nb, kvh, bs, d)
    kb = orc.from_f32(np.ascontiguousarray(
        kf.reshape(nb, kvh, bs, d // 8, 8).transpose(0, 1, 3, 2, 4)), code)
    vb = orc.from_f32(orc.fp8_to_f32(vc), code)
    ref = vpa.paged_attention_varlen_prefill(
        to_dev(q, code, device), to_dev(kb, code, device), to_dev(vb, code, device),
        u32(bt, device), u32(lens, device), u32(cu, device), None, None, scale, 1.0,
        causal=True)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(got.view(np.uint32), orc.to_f32(to_host(ref), code).view(np.uint32))


@pytest.mark.parametrize("d", [96, 192])
def test_fp8_append_and_gather_head_dims(device, d):
    """Append into and gather out of fp8 caches at head_dim 96 and 192:
    bit-exact bytes and dequantised rows."""
    rng = np.random.default_rng(d)
    kvh, bs, nb = 4, 32, 16
    lens = np.array([5, 40, 70], dtype=np.uint32)
    bt = block_tables_for(rng, lens, nb, bs)
    pos = [np.arange(int(L)) for L in lens]
    slots = np.concatenate([bt[s, p // bs].astype(np.int64) * bs + p % bs
                            for s, p in enumerate(pos)])
    t = len(slots)
    k = orc.from_f32(spread_values(rng, (t, kvh, d)), orc.BF16)
    v = orc.from_f32(spread_values(rng, (t, kvh, d)), orc.BF16)
    kc = np.zeros((nb, kvh, d // 16, bs, 16), np.uint8)
    vc = np.zeros((nb, kvh, d, bs), np.uint8)
    kcd, vcd = f8(kc, device), f8(vc, device)
    vpa.reshape_and_cache(to_dev(k, orc.BF16, device), to_dev(v, orc.BF16, device),
                          scalar(0.5, device), scalar(2.0, device), kcd, vcd, i64(slots, device))
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.uint32)
    gk, gv = vpa.gather_kv_cache(kcd, vcd, scalar(0.5, device), scalar(2.0, device),
                                 u32(bt, device), u32(cu, device), TORCH[orc.F32])
    torch.cuda.synchronize()
    orc.reshape_and_cache_fp8(k, v, kc, vc, slots, orc.BF16, 0.5, 2.0)
    np.testing.assert_array_equal(f8_host(kcd), kc)
    np.testing.assert_array_equal(f8_host(vcd), vc)
    wk, wv = orc.gather_kv_cache_fp8(kc, vc, bt, cu, orc.F32, 0.5, 2.0)
    for got, want in ((to_host(gk), wk), (to_host(gv), wv)):
        assert np.array_equal(np.isnan(got), np.isnan(want))
        fin = ~np.isnan(want)
        np.testing.assert_array_equal(got[fin], want[fin])


@pytest.mark.parametrize("d", [64, 128])
def test_fp8_prefill_equals_bf16_prefill_over_dequantised_cache(device, d):
    """Scales 1: E4M3 values are exact in bf16, so the fp8 kernel feeds the
    MFMAs the same operands as the bf16 kernel over a bf16 copy of the cache
    (re-packed from 16 to 8 elements per key vector): the outputs are equal
    bit for bit."""
    code, h, kvh, bs = orc.BF16, 16, 8, 16
    got, _, (q, kc, vc, bt, lens, cu, scale) = fp8_prefill_case(
        device, code, h, kvh, bs, [0, 17, 500], [64, 33, 90], seed=21, d=d)
    nb, _, c16, _, _ = kc.shape
    d = c16 * 16
    kf = orc.fp8_to_f32(kc).transpose(0, 1, 3, 2, 4).reshape(nb, kvh, bs, d)
    kb = orc.from_f32(np.ascontiguousarray(
        kf.reshape(nb, kvh, bs, d // 8, 8).transpose(0, 1, 3, 2, 4)), code)
    vb = orc.from_f32(orc.fp8_to_f32(vc), code)
    ref = vpa.paged_attention_varlen_prefill(
        to_dev(q, code, device), to_dev(kb, code, device), to_dev(vb, code, device),
        u32(bt, device), u32(lens, device), u32(cu, device), None, None, scale, 1.0,
        causal=True)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(got.view(np.uint32), orc.to_f32(to_host(ref), code).view(np.uint32))


def test_fp8_append_then_prefill_end_to_end(device):
    """The new tokens appended into the fp8 cache, then prefill over it:
    the cache bytes equal the oracle's encode and the attention its fp64
    attention over the dequantised cache."""
    rng = np.random.default_rng(31)
    code, h, kvh, d, bs = orc.BF16, 16, 8, 128, 16
    prior, new = np.array([20, 0, 130]), np.array([45, 70, 16])
    lens = prior + new
    nb = int(sum((int(L) + bs - 1) // bs for L in lens)) + 3
    kc = orc.fp8_from_f32((rng.standard_normal((nb, kvh, d // 16, bs, 16))).astype(np.float32))
    vc = orc.fp8_from_f32((rng.standard_normal((nb, kvh, d, bs))).astype(np.float32))
    bt = block_tables_for(rng, lens, nb, bs)
    slots = np.concatenate([bt[s, np.arange(P, L) // bs].astype(np.int64) * bs
                            + np.arange(P, L) % bs for s, (P, L) in enumerate(zip(prior, lens))])
    tq = int(new.sum())
    k = random_words(rng, (tq, kvh, d), code)
    v = random_words(rng, (tq, kvh, d), code)
    q = random_words(rng, (tq, h, d), code)
    ks, vs = 0.5, 0.75
    kcd, vcd = f8(kc, device), f8(vc, device)
    ksd, vsd = scalar(ks, device), scalar(vs, device)
    vpa.reshape_and_cache(to_dev(k, code, device), to_dev(v, code, device), ksd, vsd, kcd, vcd,
                          i64(slots, device))
    cu = np.concatenate([[0], np.cumsum(new)]).astype(np.uint32)
    out = vpa.paged_attention_varlen_prefill(
        to_dev(q, code, device), kcd, vcd, u32(bt, device), u32(lens.astype(np.uint32), device),
        u32(cu, device), ksd, vsd, d ** -0.5, 1.0, causal=True)
    torch.cuda.synchronize()
    orc.reshape_and_cache_fp8(k, v, kc, vc, slots, code, ks, vs)
    np.testing.assert_array_equal(f8_host(kcd), kc)
    np.testing.assert_array_equal(f8_host(vcd), vc)
    want = orc.prefill_attention(q, kc, vc, bt, lens.astype(np.uint32), cu, d ** -0.5,
                                 causal=True, dtype=code, kv_dtype=orc.FP8, k_scale=ks,
                                 v_scale=vs)
    assert_attention_close(orc.to_f32(to_host(out), code), want, code, "fp8 append + prefill")


@pytest.mark.parametrize("t", [2048, 2049])
@pytest.mark.parametrize("pattern", ["decode", "prefill"])
def test_fp8_append_slot_patterns(device, t, pattern):
    """The quantising append over large calls of scattered single tokens and
    of runs through shuffled blocks, bit-exact with the oracle."""
    from tests.test_gpu_cache import _pattern_slots

    rng = np.random.default_rng(t + len(pattern))
    kvh, d, bs = 2, 128, 16
    nb = t + 8 if pattern == "decode" else t // bs + 24
    slots = _pattern_slots(rng, pattern, t, nb, bs)
    kc = rng.integers(0, 256, size=(nb, kvh, d // 16, bs, 16), dtype=np.uint8)
    vc = rng.integers(0, 256, size=(nb, kvh, d, bs), dtype=np.uint8)
    k = orc.from_f32(spread_values(rng, (t, kvh, d)), orc.BF16)
    v = orc.from_f32(spread_values(rng, (t, kvh, d)), orc.BF16)
    kcd, vcd = f8(kc, device), f8(vc, device)
    vpa.reshape_and_cache(to_dev(k, orc.BF16, device), to_dev(v, orc.BF16, device),
                          scalar(0.5, device), scalar(2.0, device), kcd, vcd, i64(slots, device))
    torch.cuda.synchronize()
    orc.reshape_and_cache_fp8(k, v, kc, vc, slots, orc.BF16, 0.5, 2.0)
    np.testing.assert_array_equal(f8_host(kcd), kc)
    np.testing.assert_array_equal(f8_host(vcd), vc)


def test_fp8_prefill_c4_equals_bf16_prefill_over_dequantised_cache(device):
    """c4 at full size (64 sequences x 512 new tokens over 62..1008 prior
    ones, 5502-block pool): with scales 1 the fp8 kernel's output equals, bit
    for bit, the bf16 kernel's over a bf16 copy of the cache (E4M3 values
    are exact in bf16, and both kernels share their softmax groups)."""
    from vpa import workloads
    w = workloads.c4()
    code, h, kvh, d, bs = orc.BF16, w.num_heads, w.num_kv_heads, w.head_dim, w.block_size
    nb = w.num_blocks
    rng = np.random.default_rng(w.seed + 1)
    kc = orc.fp8_from_f32((rng.standard_normal((nb, kvh, d // 16, bs, 16)) * 2)
                          .astype(np.float32))
    vc = orc.fp8_from_f32((rng.standard_normal((nb, kvh, d, bs)) * 2).astype(np.float32))
    tq = int(w.query_lens.sum())
    q = to_dev(random_words(rng, (tq, h, d), code), code, device)
    bt, lens, cu = u32(w.block_tables, device), u32(w.context_lens, device), u32(w.cu_seqlens_q, device)
    one = scalar(1.0, device)
    mq, mk = int(w.query_lens.max()), int(w.context_lens.max())
    got = vpa.paged_attention_varlen_prefill(q, f8(kc, device), f8(vc, device), bt, lens, cu,
                                             one, one, d ** -0.5, 1.0, causal=True,
                                             max_query_len=mq, max_context_len=mk)
    kf = orc.fp8_to_f32(kc).transpose(0, 1, 3, 2, 4).reshape(nb, kvh, bs, d)
    kb = orc.from_f32(np.ascontiguousarray(
        kf.reshape(nb, kvh, bs, d // 8, 8).transpose(0, 1, 3, 2, 4)), code)
    vb = orc.from_f32(orc.fp8_to_f32(vc), code)
    ref = vpa.paged_attention_varlen_prefill(q, to_dev(kb, code, device), to_dev(vb, code, device),
                                             bt, lens, cu, None, None, d ** -0.5, 1.0,
                                             causal=True, max_query_len=mq, max_context_len=mk)
    torch.cuda.synchronize()
    assert torch.equal(got.view(torch.int16), ref.view(torch.int16))
    assert torch.isfinite(got.float()).all()
