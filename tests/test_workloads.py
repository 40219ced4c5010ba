"""The synthetic workloads against the generation rules of the five configs
(lengths, pool sizes, distinct blocks, the decode slot rule of
paged_kv_cache.rs:74-103), and compact_tables: attention and the decode step
of the oracle over a compacted copy of the blocks equal the same over the
whole pool."""

import numpy as np

from oracle import oracle as orc
from tests._util import block_tables_for, make_cache, random_words
from vpa import workloads


def check_slots(bt, lens, slots, bs):
    pos = lens.astype(np.int64) - 1
    np.testing.assert_array_equal(
        slots, bt[np.arange(len(lens)), pos // bs].astype(np.int64) * bs + pos % bs)


def check_tables(bt, lens, nb, bs):
    need = (lens.astype(np.int64) + bs - 1) // bs
    for i, n in enumerate(need):
        ids = bt[i, :n]
        assert len(np.unique(ids)) == n, f"row {i}: repeated blocks"
        assert ids.min() >= 1 and ids.max() < nb, f"row {i}: id outside 1..nb-1"


def test_decode_configs_follow_their_rules():
    w = workloads.c1()
    assert w.dtype == "f32" and w.num_seqs == 1 and int(w.context_lens[0]) == 512
    assert w.layers[0].num_blocks == 64 and len(np.unique(w.layers[0].block_tables[0])) == 32
    w = workloads.c2()
    assert w.num_seqs == 32 and w.context_lens.min() >= 100 and w.context_lens.max() <= 1500
    need = int(((w.context_lens.astype(np.int64) + 15) // 16).sum())
    assert w.layers[0].num_blocks >= 1.25 * need
    w = workloads.c3(num_layers=3)
    assert w.num_seqs == 256 and w.context_lens.min() >= 16 and w.context_lens.max() <= 4096
    assert 600 < w.context_lens.mean() < 1000  # geometric, mean 800, clipped
    w5 = workloads.c5(num_layers=2)
    assert w5.num_seqs == 1024 and w5.shared_pool
    assert w5.context_lens.min() >= 256 and w5.context_lens.max() <= 8192
    pool = w5.layers[0].num_blocks * 2 * 8 * 128 * 16 * 2
    assert 0.59 * 288e9 < pool <= 0.6 * 288e9
    for wl in (workloads.c2(), w, w5):
        for layer in wl.layers:
            check_tables(layer.block_tables, wl.context_lens, layer.num_blocks, wl.block_size)
            check_slots(layer.block_tables, wl.context_lens, layer.slot_mapping, wl.block_size)


def test_compact_tables_keeps_attention_and_decode_step():
    rng = np.random.default_rng(8)
    h, kvh, d, bs, nb = 8, 4, 64, 16, 90
    lens = np.array([1, 17, 200, 33, 64], dtype=np.uint32)
    bt = block_tables_for(rng, lens, nb, bs, pad_cols=2)
    bt[2, 3] = bt[3, 0]  # a block shared by two sequences
    kc, vc = make_cache(rng, nb, kvh, d, bs, orc.BF16)
    q = random_words(rng, (len(lens), h, d), orc.BF16)
    pick = np.array([0, 2, 3])
    pos = lens[pick].astype(np.int64) - 1
    slots = bt[pick, pos // bs].astype(np.int64) * bs + pos % bs
    slots[0] = -1
    blocks, tables, new_slots = workloads.compact_tables(bt[pick], lens[pick], bs, slots)
    assert blocks[0] == 0 and np.all(np.diff(blocks) > 0)
    need = (lens[pick].astype(np.int64) + bs - 1) // bs
    assert len(blocks) == 1 + len(np.unique(np.concatenate([bt[i, :n] for i, n in
                                                            zip(pick, need)])))
    for r, n in enumerate(need):
        np.testing.assert_array_equal(blocks[tables[r, :n]], bt[pick[r], :n])
    assert new_slots[0] == -1
    np.testing.assert_array_equal(blocks[new_slots[1:] // bs] * bs + new_slots[1:] % bs,
                                  slots[1:])
    kh, vh = np.ascontiguousarray(kc[blocks]), np.ascontiguousarray(vc[blocks])
    scale = d ** -0.5
    want = orc.paged_attention(q[pick], kc, vc, bt[pick], lens[pick], 200, scale, dtype=orc.BF16)
    got = orc.paged_attention(q[pick], kh, vh, tables, lens[pick], 200, scale, dtype=orc.BF16)
    np.testing.assert_array_equal(got, want)
    k = random_words(rng, (len(pick), kvh, d), orc.BF16)
    v = random_words(rng, (len(pick), kvh, d), orc.BF16)
    full, _ = orc.cpu_baseline_decode_step(q[pick], k, v, slots, kc.copy(), vc.copy(), bt[pick],
                                           lens[pick], scale, dtype=orc.BF16)
    part, _ = orc.cpu_baseline_decode_step(q[pick], k, v, new_slots, kh, vh, tables, lens[pick],
                                           scale, dtype=orc.BF16)
    np.testing.assert_array_equal(part, full)
