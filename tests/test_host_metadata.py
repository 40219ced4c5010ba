"""Host-side paged-cache bookkeeping (include/vpa_host.h, vpa/host.py) against
the reference's own known-answer tests:

* vasr-paged-attn/src/paged_kv_cache.rs:1076-1376 (slots, tables, contexts,
  cu_seqlens, decode steps);
* vasr-paged-attn/src/paged_cache_runtime.rs:720-778 (block sizing, block
  manager);
* vasr-paged-attn/src/cuda_graph.rs:642-763 (graph buckets, padding);
* vasr-models/src/model/generation.rs:1789-1793 (decode slot/context).

All CPU: these functions never touch a device (except the memory-fraction
sizing, which is exercised on the GPU box only)."""

import numpy as np
import pytest

from vpa import host
from vpa.graph import DecodeGraphCache
from vpa._lib import VPA_ERR_CAPACITY, VPA_ERR_INVALID_ARGUMENT, VPA_ERR_NOT_FOUND, VpaError

PAD = host.PAD_SLOT_ID


# ---------------------------------------------------------------- paged_kv_cache.rs

def test_single_sequence_layout_kat():
    # PagedKvCache::new(2, 4, 8, 16, 40, F32)  (paged_kv_cache.rs:1077-1087)
    c = host.ContiguousCache(block_size=16, batch_size=1, max_tokens_per_sequence=40)
    assert c.num_blocks == 3
    assert c.block_table_host() == [0, 1, 2]
    assert c.slot_for_position(0) == 0
    assert c.slot_for_position(16) == 16
    assert c.slot_for_position(39) == 39


def test_metadata_tensors_kat():
    # PagedKvCache::new(1, 2, 8, 4, 10, F32)  (:1090-1109)
    c = host.ContiguousCache(block_size=4, batch_size=1, max_tokens_per_sequence=10)
    assert c.slot_mapping_for_range(3, 4).tolist() == [3, 4, 5, 6]
    assert [c.block_table_host()] == [[0, 1, 2]]


def test_multi_sequence_layout_kat():
    # PagedKvCache::new_batched(1, 2, 8, 4, 2, 10, F32)  (:1112-1138)
    c = host.ContiguousCache(block_size=4, batch_size=2, max_tokens_per_sequence=10)
    assert c.num_blocks_per_sequence == 3 and c.num_blocks == 6
    assert c.slot_for_sequence_position(0, 0) == 0
    assert c.slot_for_sequence_position(0, 9) == 9
    assert c.slot_for_sequence_position(1, 0) == 12
    assert c.slot_for_sequence_position(1, 9) == 21
    # input_metadata_for_batch_ranges(&[0, 0], 3, &[3, 3]) over the cache's own tables
    m = host.input_metadata_from_block_tables(c.block_tables_for_batch(2), [0, 0], 3, [3, 3],
                                              block_size=4, num_blocks=c.num_blocks)
    assert m["slot_mapping"].tolist() == [0, 1, 2, 12, 13, 14]
    assert m["block_tables"].tolist() == [[0, 1, 2], [3, 4, 5]]
    assert m["context_lens"].tolist() == [3, 3]
    assert m["max_context_len"] == 3


def test_contiguous_slot_bounds():
    c = host.ContiguousCache(block_size=4, batch_size=2, max_tokens_per_sequence=10)
    with pytest.raises(VpaError, match="sequence exceeds"):
        c.slot_for_sequence_position(2, 0)
    with pytest.raises(VpaError, match="position exceeds"):
        c.slot_for_sequence_position(0, 10)


def test_metadata_from_physical_block_tables_kat():
    # new_pool(1, 2, 8, 4, 8); tables [[3,4],[6,7]], starts [2,4], len 2, ctx [4,6]  (:1141-1161)
    m = host.input_metadata_from_block_tables([[3, 4], [6, 7]], [2, 4], 2, [4, 6], 4, 8)
    assert m["slot_mapping"].tolist() == [14, 15, 28, 29]
    assert m["block_tables"].tolist() == [[3, 4], [6, 7]]
    assert m["context_lens"].tolist() == [4, 6]
    assert m["max_context_len"] == 6
    assert m["cu_seqlens_q"].tolist() == [0, 2, 4]
    assert m["cu_seqlens_kv"].tolist() == [0, 4, 10]


def test_metadata_from_attention_masks_kat():
    # (:1164-1257)
    masks = [[1, 1, 1, 1, 0, 0], [1, 1, 1, 1, 1, 0]]
    m = host.input_metadata_from_attention_masks([[3, 4], [6, 7]], masks, 4, 8)
    assert m["slot_mapping"].tolist() == [12, 13, 14, 15, PAD, PAD, 24, 25, 26, 27, 28, PAD]
    assert m["token_attention_mask"].tolist() == masks
    assert m["context_lens"].tolist() == [4, 5]
    assert m["query_lens"] == [4, 5] and m["kv_lens"] == [4, 5]
    assert m["cu_seqlens_q"].tolist() == [0, 4, 9]
    assert m["cu_seqlens_kv"].tolist() == [0, 4, 9]
    assert m["max_query_len"] == 5 and m["max_kv_len"] == 5 and m["max_context_len"] == 5
    assert not m["prefill_causal_only"]
    full = host.input_metadata_from_attention_masks([[3, 4]], [[1] * 6], 4, 8)
    assert full["prefill_causal_only"]


def test_decode_metadata_for_steps_matches_per_step_builder():
    # new_pool(1, 2, 8, 4, 64): prompt 10, 4 steps  (:1260-1288)
    c = host.ContiguousCache(block_size=4, batch_size=1, max_tokens_per_sequence=256)
    steps = c.decode_metadata_for_steps(10, 4)
    for t, m in enumerate(steps):
        want = host.input_metadata_from_block_tables([c.block_table_host()], [10 + t], 1,
                                                     [10 + t + 1], 4, c.num_blocks)
        assert m["slot_mapping"].tolist() == want["slot_mapping"].tolist()
        assert m["context_lens"].tolist() == want["context_lens"].tolist()
        assert m["max_context_len"] == want["max_context_len"]


def test_metadata_from_query_lens_is_packed_kat():
    # (:1291-1314)
    m = host.input_metadata_from_query_lens([[3, 4], [6, 7]], [4, 5], 4, 8)
    assert m["slot_mapping"].tolist() == [12, 13, 14, 15, 24, 25, 26, 27, 28]
    assert m["block_tables"].tolist() == [[3, 4], [6, 7]]
    assert m["context_lens"].tolist() == [4, 5]
    assert m["max_context_len"] == 5
    assert m["query_lens"] == [4, 5] and m["kv_lens"] == [4, 5]
    assert m["token_attention_mask"] is None
    assert m["prefill_causal_only"]


@pytest.mark.parametrize("graph_buckets", [False, True])
def test_decode_metadata_for_batch_steps_matches_per_step_builder(graph_buckets):
    # new_pool(1, 2, 8, 4, 16): tables [[3,4],[6,7]], prompts [4,5], 3 steps  (:1317-1375)
    tables, prompts, steps = [[3, 4], [6, 7]], [4, 5], 3
    pre = host.decode_metadata_for_batch_steps(tables, prompts, steps, 4, 16, 16 * 4,
                                               graph_buckets=graph_buckets)
    cols = host.bucket_block_table_cols(2, 4) if graph_buckets else 2
    padded = [t + [0] * (cols - len(t)) for t in tables]
    for t in range(steps):
        want = host.input_metadata_from_block_tables(padded, [p + t for p in prompts], 1,
                                                     [p + t + 1 for p in prompts], 4, 16)
        got = pre[t]
        assert got["slot_mapping"].tolist() == want["slot_mapping"].tolist()
        assert got["block_tables"].tolist() == want["block_tables"].tolist()
        assert got["context_lens"].tolist() == want["context_lens"].tolist()
        assert got["max_context_len"] == want["max_context_len"]
        assert got["cu_seqlens_q"] is None and got["cu_seqlens_kv"] is None
    if graph_buckets:
        assert pre[0]["block_tables"].shape == (2, 64)  # ceil(256 / 4) columns


def test_decode_slot_and_context_kat():
    # generation.rs:1789-1793: (prompt 42, step 0) -> (42, 43); step 7 -> (49, 50)
    c = host.ContiguousCache(block_size=16, batch_size=1, max_tokens_per_sequence=128)
    steps = c.decode_metadata_for_steps(42, 8)
    assert (int(steps[0]["slot_mapping"][0]), int(steps[0]["context_lens"][0])) == (42, 43)
    assert (int(steps[7]["slot_mapping"][0]), int(steps[7]["context_lens"][0])) == (49, 50)


def test_slot_lookup_errors():
    assert host.slot_for_block_table_position([3, 4], 4, 8, 5) == 17
    with pytest.raises(VpaError, match="missing block table entry"):
        host.slot_for_block_table_position([3, 4], 4, 8, 8)
    with pytest.raises(VpaError, match="exceeds paged cache capacity"):
        host.slot_for_block_table_position([3, 9], 4, 8, 5)
    with pytest.raises(VpaError, match="non-zero"):
        host.input_metadata_from_query_lens([[3, 4]], [0], 4, 8)
    with pytest.raises(VpaError, match="at least one block"):
        host.input_metadata_from_block_tables([[]], [0], 1, [1], 4, 8)
    with pytest.raises(VpaError, match="sequence capacity"):
        host.decode_metadata_for_batch_steps([[3, 4]], [7], 2, 4, 8, 8)


def test_cumulative_seqlens():
    assert host.cumulative_seqlens([4, 5, 0, 7]).tolist() == [0, 4, 9, 9, 16]
    assert host.cumulative_seqlens([]).tolist() == [0]
    with pytest.raises(VpaError, match="overflow"):
        host.cumulative_seqlens([2 ** 31, 2 ** 31])


# ---------------------------------------------------------- paged_cache_runtime.rs

def test_bytes_per_paged_block_matches_qwen3_asr_defaults():
    # (:721-726)
    assert host.bytes_per_paged_block(28, 8, 128, 32, "bf16") == 3_670_016


def test_blocks_for_byte_budget_reserves_null_block():
    # (:729-734)
    bpb = host.bytes_per_paged_block(28, 8, 128, 32, "bf16")
    assert host.blocks_for_byte_budget(bpb * 10, bpb) == 11
    with pytest.raises(VpaError) as e:
        host.blocks_for_byte_budget(bpb - 1, bpb)
    assert e.value.code == VPA_ERR_CAPACITY


def test_resolve_num_blocks_context_size():
    # ContextSize(tokens) -> ceil(tokens / block_size) + 1  (:161)
    assert host.resolve_num_blocks("context", 1000, 28, 8, 128, 16) == 64
    assert host.resolve_num_blocks("context", 1024, 28, 8, 128, 16) == 65
    assert host.resolve_num_blocks("blocks", 77, 28, 8, 128, 16) == 77


def test_block_manager_allocates_extends_and_frees_requests():
    # (:737-752)
    m = host.BlockManager(8, 4)
    assert m.free_blocks() == 7
    m.allocate_slots(10, 5)
    assert len(m.block_ids(10)) == 2 and m.free_blocks() == 5
    m.allocate_slots(10, 9)
    assert len(m.block_ids(10)) == 3 and m.free_blocks() == 4
    m.free_request(10)
    assert m.free_blocks() == 7


def test_block_manager_trim_releases_tail_blocks():
    # (:755-769)
    m = host.BlockManager(8, 4)
    m.allocate_slots(10, 12)
    assert len(m.block_ids(10)) == 3 and m.free_blocks() == 4
    m.trim_request_to_num_tokens(10, 5)
    assert len(m.block_ids(10)) == 2 and m.free_blocks() == 5
    m.trim_request_to_num_tokens(10, 1)
    assert len(m.block_ids(10)) == 1 and m.free_blocks() == 6


def test_block_manager_try_allocate_reports_exhaustion():
    # (:772-778)
    m = host.BlockManager(4, 4)
    assert m.try_allocate_slots(1, 4)
    assert not m.try_allocate_slots(2, 16)
    assert m.free_blocks() == 2
    with pytest.raises(VpaError) as e:
        m.allocate_slots(2, 16)
    assert e.value.code == VPA_ERR_CAPACITY and "exhausted" in e.value.message


def test_block_manager_fifo_order_and_reverse_release():
    """Free list semantics of PagedBlockManager (paged_cache_runtime.rs:224-363):
    ids 1.. handed out from the front; a freed or trimmed tail goes to the
    back, last block first; block 0 is never handed out."""
    m = host.BlockManager(8, 4)
    m.allocate_slots(1, 8)        # blocks 1, 2
    m.allocate_slots(2, 4)        # block 3
    assert m.block_ids(1) == [1, 2] and m.block_ids(2) == [3]
    m.free_request(1)             # free list: 4 5 6 7 2 1
    m.allocate_slots(3, 24)       # six blocks
    assert m.block_ids(3) == [4, 5, 6, 7, 2, 1]
    m.trim_request_to_num_tokens(3, 9)  # keep 3 blocks; 1, 2, 7 return (last first)
    assert m.block_ids(3) == [4, 5, 6]
    m.allocate_slots(4, 12)
    assert m.block_ids(4) == [1, 2, 7]
    assert 0 not in m.block_ids(3) + m.block_ids(4)
    assert m.total_allocated_blocks() == 7 and m.free_blocks() == 0
    assert m.slots_available_for(3, 12) and not m.slots_available_for(3, 13)
    assert m.block_tables_for([2, 4]) == [[3], [1, 2, 7]]
    with pytest.raises(VpaError) as e:
        m.block_ids(99)
    assert e.value.code == VPA_ERR_NOT_FOUND
    m.free_request(99)            # unknown ids are ignored
    m.free_many([2, 3, 4])
    assert m.free_blocks() == 7 and m.total_allocated_blocks() == 0
    assert host.BlockManager.allocatable_block_capacity(8) == 7


def test_block_manager_zero_tokens_allocates_nothing():
    m = host.BlockManager(8, 4)
    assert m.try_allocate_slots(5, 0)
    assert m.blocks_for_request(5) == 0
    with pytest.raises(VpaError):
        m.block_ids(5)


# ------------------------------------------------------------------- cuda_graph.rs

def test_cuda_graph_batch_bucket_kat():
    # (:642-663)
    cases = [(0, 64, None), (1, 64, 1), (2, 64, 2), (3, 64, 4), (4, 64, 4), (5, 64, 8),
             (8, 64, 8), (9, 64, 16), (16, 64, 16), (17, 64, 32), (20, 64, 32), (33, 64, 48),
             (64, 64, 64), (65, 64, None), (20, 20, 20)]
    for actual, mx, want in cases:
        assert host.cuda_graph_batch_bucket(actual, mx) == want, (actual, mx)


def test_cuda_graph_batch_buckets_kat():
    # (:666-673)
    assert host.cuda_graph_batch_buckets(0) == []
    assert host.cuda_graph_batch_buckets(8) == [1, 2, 4, 8]
    assert host.cuda_graph_batch_buckets(20) == [1, 2, 4, 8, 16, 20]
    assert host.cuda_graph_batch_buckets(64) == [1, 2, 4, 8, 16, 32, 48, 64]
    # clamped to the capture limit of 256 (cuda_graph.rs:19, 78-80)
    assert host.cuda_graph_batch_buckets(1000)[-1] == 256


def test_block_table_bucket_kat():
    # (:676-686)
    for blocks, want in [(0, 8), (1, 8), (8, 8), (9, 16), (16, 16), (17, 32), (24, 32), (33, 64)]:
        assert host.bucket_block_table_cols(blocks, 32) == want, blocks


def test_pad_decode_batch_kat():
    # (:689-763)
    bt = np.array([[1, 2, 3, 4], [5, 6, 7, 8], [9, 10, 11, 12]], dtype=np.uint32)
    ids, slots, ctx, tables = host.pad_decode_batch_to_max(
        8, [11, 22, 33], [64, 96, 128], [65, 97, 129], bt, 8)
    assert ids.tolist() == [11, 22, 33, 0, 0, 0, 0, 0]
    assert slots.tolist() == [64, 96, 128, 0, 0, 0, 0, 0]
    assert ctx.tolist() == [65, 97, 129, 1, 1, 1, 1, 1]
    assert tables.tolist() == [
        [1, 2, 3, 4, 4, 4, 4, 4],
        [5, 6, 7, 8, 8, 8, 8, 8],
        [9, 10, 11, 12, 12, 12, 12, 12],
    ] + [[0] * 8] * 5
    with pytest.raises(VpaError) as e:
        host.pad_decode_batch_to_max(2, [1, 2, 3], [0, 0, 0], [1, 1, 1], bt, 8)
    assert e.value.code == VPA_ERR_INVALID_ARGUMENT
    with pytest.raises(VpaError, match="down to"):
        host.pad_decode_batch_to_max(8, [1, 2, 3], [0, 0, 0], [1, 1, 1], bt, 2)


def test_graph_cache_keys_follow_the_reference_buckets():
    """Batch buckets 1, 2, 4, 8, then multiples of 16; columns a power of two
    of at least 256 / block_size (cuda_graph.rs:28-81)."""
    cache = DecodeGraphCache(lambda bufs, m: bufs["input_ids"], 256, 16, {}, "cpu")
    assert cache.key(1, 1) == (1, 16)
    assert cache.key(3, 16) == (4, 16)
    assert cache.key(9, 17) == (16, 32)
    assert cache.key(17, 100) == (32, 128)
    assert cache.key(256, 300) == (256, 512)
    assert host.cuda_graph_batch_buckets(40) == [1, 2, 4, 8, 16, 32, 40]
    assert DecodeGraphCache(lambda b, m: b, 40, 16, {}, "cpu").key(33, 1) == (40, 16)
    with pytest.raises(ValueError):
        cache.key(257, 1)
    with pytest.raises(ValueError):
        cache.key(0, 1)
