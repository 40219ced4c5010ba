"""GPU parity of reshape_and_cache and gather_kv_cache against the oracle:
bit-exact cache contents (including bytes outside the target slots)."""

import numpy as np
import pytest
import torch

import vpa
from oracle import oracle as orc
from tests._util import (TORCH, block_tables_for, i64, make_cache, random_words, to_dev, to_host,
                         u32)

pytestmark = pytest.mark.gpu


def run_append(device, code, kvh, d, bs, nb, slots, seed, zero_cache=False):
    rng = np.random.default_rng(seed)
    kc, vc = make_cache(rng, nb, kvh, d, bs, code, zero=zero_cache)
    t = len(slots)
    k = random_words(rng, (t, kvh, d), code)
    v = random_words(rng, (t, kvh, d), code)
    kc_d, vc_d = to_dev(kc, code, device), to_dev(vc, code, device)
    vpa.reshape_and_cache(to_dev(k, code, device), to_dev(v, code, device), None, None, kc_d, vc_d,
                          i64(slots, device))
    torch.cuda.synchronize()
    orc.reshape_and_cache(k, v, kc, vc, np.asarray(slots, dtype=np.int64), dtype=code)
    np.testing.assert_array_equal(to_host(kc_d), kc)
    np.testing.assert_array_equal(to_host(vc_d), vc)


@pytest.mark.parametrize("code", [orc.F32, orc.BF16, orc.F16])
@pytest.mark.parametrize("bs", [8, 16, 32])
@pytest.mark.parametrize("d", [64, 96, 128, 192, 256])
def test_append_decode_pattern(device, code, bs, d):
    """One token per sequence into scattered blocks (the decode append)."""
    rng = np.random.default_rng(bs * d + code)
    nb = 64
    slots = rng.choice(nb * bs, size=37, replace=False)
    run_append(device, code, 4, d, bs, nb, slots, seed=bs + d)


@pytest.mark.parametrize("code", [orc.BF16, orc.F32])
@pytest.mark.parametrize("bs", [8, 16, 32])
def test_append_prefill_pattern(device, code, bs):
    """Consecutive positions of several sequences: whole blocks plus ragged
    heads/tails (prior tokens not aligned to a block)."""
    rng = np.random.default_rng(50 + bs)
    nb, kvh, d = 200, 8, 128
    prior = [0, 5, bs, 3 * bs - 1]
    new = [3 * bs, 2 * bs + 7, 1, bs + 1]
    lens = [p + n for p, n in zip(prior, new)]
    bt = block_tables_for(rng, lens, nb, bs)
    slots = []
    for s, (p, n) in enumerate(zip(prior, new)):
        pos = np.arange(p, p + n)
        slots.append(bt[s, pos // bs].astype(np.int64) * bs + pos % bs)
    run_append(device, code, kvh, d, bs, nb, np.concatenate(slots), seed=bs)


def test_append_padding_and_out_of_range_slots(device):
    rng = np.random.default_rng(3)
    nb, bs = 16, 16
    slots = rng.choice(nb * bs, size=40, replace=False).astype(np.int64)
    slots[::3] = -1                 # PAD_SLOT_ID
    slots[1] = nb * bs              # past the pool: skipped
    slots[4] = nb * bs + 12345
    run_append(device, orc.BF16, 8, 128, bs, nb, slots, seed=4)
    # a whole aligned group of padding
    run_append(device, orc.BF16, 8, 128, bs, nb, np.full(16, -1, dtype=np.int64), seed=5)


def test_append_small_call_mixes_lone_and_shared_blocks(device):
    """Tokens alone in their block next to tokens sharing a block with
    another token of the same call (and of the same 16-token group)."""
    nb, bs = 32, 16
    slots = np.array([3 * bs + 0, 3 * bs + 5, 7 * bs + 2, 9 * bs + 15, 9 * bs + 14, 11 * bs + 8,
                      -1, 12 * bs + 1, 31 * bs + 15], dtype=np.int64)
    for code in (orc.BF16, orc.F32):
        run_append(device, code, 8, 128, bs, nb, slots, seed=21 + code)
    # scattered single tokens at two sizes
    rng = np.random.default_rng(22)
    for t in (1024, 1025):
        nb2 = 2048
        run_append(device, orc.BF16, 2, 64, bs, nb2, rng.choice(nb2 * bs, size=t, replace=False),
                   seed=23)


def test_append_large_mixed_call(device):
    """A large call: aligned whole blocks, ragged heads and tails, padding
    and out-of-pool slots."""
    rng = np.random.default_rng(24)
    nb, kvh, d, bs = 400, 4, 128, 16
    prior = [0, 7, 16, 40, 3]
    new = [512, 300, 257, 200, 33]
    lens = [p + n for p, n in zip(prior, new)]
    bt = block_tables_for(rng, lens, nb, bs)
    slots = []
    for s, (p, n) in enumerate(zip(prior, new)):
        pos = np.arange(p, p + n)
        slots.append(bt[s, pos // bs].astype(np.int64) * bs + pos % bs)
    slots = np.concatenate(slots)
    slots[100:116] = -1
    slots[700] = nb * bs + 3
    assert len(slots) > 1024
    for code in (orc.BF16, orc.F32):
        run_append(device, code, kvh, d, bs, nb, slots, seed=25 + code)


def test_append_config_c1_prefill_then_append(device):
    """c1: 511 prefilled positions then one append at 511 into 32 blocks of a
    64-block pool, f32, 8 kv heads x 128."""
    from vpa import workloads
    w = workloads.c1()
    bt = w.layers[0].block_tables[0]
    pos = np.arange(511)
    pre = bt[pos // 16].astype(np.int64) * 16 + pos % 16
    run_append(device, orc.F32, 8, 128, 16, 64, pre, seed=11, zero_cache=True)
    run_append(device, orc.F32, 8, 128, 16, 64, w.layers[0].slot_mapping, seed=12)


def test_append_strided_rows_and_cache_views(device):
    """Token-strided key/value rows and caches that are views into a larger
    pool (block stride > kv_heads * tile)."""
    rng = np.random.default_rng(8)
    code, kvh, d, bs, nb = orc.BF16, 2, 128, 16, 12
    big_k, big_v = make_cache(rng, nb, kvh + 1, d, bs, code)   # 3 heads, use the first 2
    kc_full = to_dev(big_k, code, device)
    vc_full = to_dev(big_v, code, device)
    kc_view, vc_view = kc_full[:, :kvh], vc_full[:, :kvh]
    t = 20
    rows = random_words(rng, (t, kvh + 1, d), code)  # token stride (kvh+1)*d
    slots = rng.choice(nb * bs, size=t, replace=False)
    kr = to_dev(rows, code, device)[:, :kvh]
    vpa.reshape_and_cache(kr, kr, None, None, kc_view, vc_view, i64(slots, device))
    torch.cuda.synchronize()
    k = np.ascontiguousarray(rows[:, :kvh])
    exp_k, exp_v = big_k.copy(), big_v.copy()
    sub_k = np.ascontiguousarray(exp_k[:, :kvh])
    sub_v = np.ascontiguousarray(exp_v[:, :kvh])
    orc.reshape_and_cache(k, k, sub_k, sub_v, slots.astype(np.int64), dtype=code)
    exp_k[:, :kvh], exp_v[:, :kvh] = sub_k, sub_v
    np.testing.assert_array_equal(to_host(kc_full), exp_k)
    np.testing.assert_array_equal(to_host(vc_full), exp_v)


@pytest.mark.parametrize("code", [orc.F32, orc.BF16, orc.F16])
@pytest.mark.parametrize("bs", [8, 16, 32])
def test_gather_kv_cache(device, code, bs):
    rng = np.random.default_rng(70 + bs + code)
    nb, kvh, d = 96, 8, 128
    lens = [1, bs, 5 * bs + 3, 2 * bs - 1, 77]
    kc, vc = make_cache(rng, nb, kvh, d, bs, code)
    bt = block_tables_for(rng, lens, nb, bs, pad_cols=2)
    bt[1, 1] = nb + 3       # beyond the sequence: never read
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.uint32)
    gk, gv = vpa.gather_kv_cache(to_dev(kc, code, device), to_dev(vc, code, device), None, None,
                                 u32(bt, device), u32(cu, device), TORCH[code])
    torch.cuda.synchronize()
    ek, ev = orc.gather_kv_cache(kc, vc, bt, cu, dtype=code)
    np.testing.assert_array_equal(to_host(gk), ek)
    np.testing.assert_array_equal(to_host(gv), ev)


@pytest.mark.parametrize("code", [orc.F32, orc.BF16])
@pytest.mark.parametrize("bs", [8, 32])
@pytest.mark.parametrize("d", [96, 192])
def test_gather_kv_cache_head_dims(device, code, bs, d):
    """The head dims of the Metal prefill's set (varlen_prefill.rs:15) that
    are not powers of two."""
    rng = np.random.default_rng(90 + bs + d + code)
    nb, kvh = 48, 4
    lens = [1, bs + 3, 4 * bs - 1, 50]
    kc, vc = make_cache(rng, nb, kvh, d, bs, code)
    bt = block_tables_for(rng, lens, nb, bs, pad_cols=1)
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.uint32)
    gk, gv = vpa.gather_kv_cache(to_dev(kc, code, device), to_dev(vc, code, device), None, None,
                                 u32(bt, device), u32(cu, device), TORCH[code])
    torch.cuda.synchronize()
    ek, ev = orc.gather_kv_cache(kc, vc, bt, cu, dtype=code)
    np.testing.assert_array_equal(to_host(gk), ek)
    np.testing.assert_array_equal(to_host(gv), ev)


def test_gather_invalid_block_gives_zero_rows(device):
    rng = np.random.default_rng(5)
    code, nb, kvh, d, bs = orc.BF16, 10, 8, 128, 16
    kc, vc = make_cache(rng, nb, kvh, d, bs, code)
    bt = np.array([[3, nb + 1, 4]], dtype=np.uint32)
    cu = np.array([0, 40], dtype=np.uint32)
    gk, gv = vpa.gather_kv_cache(to_dev(kc, code, device), to_dev(vc, code, device), None, None,
                                 u32(bt, device), u32(cu, device), torch.bfloat16, total_tokens=40)
    torch.cuda.synchronize()
    ek, ev = orc.gather_kv_cache(kc, vc, bt, cu, dtype=code)
    np.testing.assert_array_equal(to_host(gk), ek)
    assert not to_host(gv)[16:32].any()


def _pattern_slots(rng, pattern, t, nb, bs):
    """Slots of t tokens: 'decode' one token per block, scattered; 'prefill'
    runs of consecutive positions through shuffled blocks, not aligned;
    'mixed' runs and lone tokens with padding, out-of-pool slots and tokens
    that share a block without being neighbours."""
    if pattern == "decode":
        return (rng.choice(nb, size=t, replace=False).astype(np.int64) * bs
                + rng.integers(0, bs, size=t))
    blocks = rng.permutation(nb).astype(np.int64)
    pos = np.arange(t) + 5
    slots = blocks[pos // bs] * bs + pos % bs
    if pattern == "mixed":
        lone = rng.choice(t, size=t // 3, replace=False)
        slots[lone] = rng.permutation(slots[lone])  # neighbours in other blocks
        slots[::11] = -1
        slots[7::97] = nb * bs + 3
    return slots


@pytest.mark.parametrize("t", [2048, 2049])
@pytest.mark.parametrize("pattern", ["decode", "prefill", "mixed"])
@pytest.mark.parametrize("code,bs", [(orc.BF16, 16), (orc.F32, 8), (orc.F16, 32)])
def test_append_slot_patterns(device, t, pattern, code, bs):
    """Large calls of each slot pattern (scattered single tokens, runs
    through shuffled blocks, runs mixed with lone tokens, padding,
    out-of-pool slots and tokens sharing a block without being neighbours),
    at a whole and a ragged number of token groups: bit-exact."""
    rng = np.random.default_rng(t + 3 * bs + code + len(pattern))
    nb = t + 8 if pattern == "decode" else t // bs + 24
    slots = _pattern_slots(rng, pattern, t, nb, bs)
    run_append(device, code, 2, 128, bs, nb, slots, seed=t + bs)
