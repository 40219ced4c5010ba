"""A decode step whose per-step state never leaves the device.

The reference drives each decode step from the host
(vasr-models/src/model/paged_batch_engine.rs:629-722): it reads the
previous step's argmax ids back (generation.rs:443-460), runs the EOS /
generated-list bookkeeping on the host (:640-667), grows every running
request by a block when its next token starts one (try_allocate_slots,
paged_cache_runtime.rs:260-300), builds slot_mapping, context_lens and the
padded block tables on the host and uploads them
(decode_metadata_for_batch_step, paged_kv_cache.rs:924-1059), then runs the
forward, whose layers call reshape_and_cache and paged_attention
(thinker_text.rs:1101-1139).

``DeviceDecodeStep`` puts the same sequence on one stream with no host
read or allocation, so a whole step (bookkeeping, block growth, metadata,
the work list, every layer's append and attention, argmax) can be captured
once as a HIP graph and replayed:

    begin()                    consume the pending ids, grow blocks, build
                               slot_mapping / context_lens, plan the work list
    layer(q, k, v, kc, vc, out) append the step's K/V rows, attend (per layer)
    end(logits)                next ids = argmax of the step's logits

Every layer shares the allocator's block tables (one block manager for the
model, each layer its own cache tensors), as the reference does. Rows that
finished feed the EOS fill id and get the PAD slot; a row the pool cannot
grow stalls for the step (its slot is PAD and its position does not move;
``allocator.status[0]`` counts them): the next step's bookkeeping sees the
PAD slot left in ``allocator.slot_mapping``, feeds the row's input id again
and appends nothing (the argmax of a forward the row took no part in is
dropped), as the reference keeps a slot that could not allocate out of the
forward with its pending id (paged_batch_engine.rs:209-227)."""

from __future__ import annotations

from typing import Sequence

import torch

from . import ops


class DeviceDecodeStep:
    def __init__(self, batch: int, num_blocks: int, block_size: int, max_context_len: int,
                 num_heads: int, head_dim: int, eos_token_ids: Sequence[int],
                 max_new_tokens: int, device):
        self.batch, self.block_size = batch, block_size
        self.max_context_len = int(max_context_len)
        self.num_heads, self.head_dim = num_heads, head_dim
        self.cols = max(1, (self.max_context_len + block_size - 1) // block_size)
        self.allocator = ops.DeviceBlockAllocator(num_blocks, block_size, batch, self.cols, device)
        self.tokens = ops.DecodeTokenState(batch, max_new_tokens, eos_token_ids, device)
        self.workspace = ops.paged_attention_workspace(batch, num_heads, head_dim,
                                                       self.max_context_len, device)
        self.scale = head_dim ** -0.5

    def admit(self, prompt_lens: torch.Tensor) -> torch.Tensor:
        """Rows hold prompt_lens[r] tokens already written to the caches (u32
        [batch]); the first step appends at that position. Returns the
        allocator's ok flags; rows the pool could not hold start finished."""
        ok = self.allocator.allocate(prompt_lens)
        self.allocator.positions.copy_(prompt_lens.to(torch.uint32))
        self.tokens.finished.copy_((ok == 0).to(torch.uint8))
        # no step has run yet: every admitted row consumes its pending id at
        # the first step (a non-negative previous slot; block 0 is the null
        # block, nothing is written there before the first step's metadata)
        self.allocator.slot_mapping.zero_()
        return ok

    def begin(self, key_cache: torch.Tensor, value_cache: torch.Tensor,
              query_dtype: torch.dtype) -> None:
        """Step start: pending ids consumed (EOS rows finish), blocks grown,
        this step's slot_mapping / context_lens and the decode work list
        built (the caches of any layer give the geometry and cache type)."""
        self.tokens.consume(self.allocator.slot_mapping)
        self.allocator.step(self.tokens.finished)
        ops.paged_attention_plan(self.allocator.context_lens, self.max_context_len, self.cols,
                                 self.num_heads, key_cache, value_cache, query_dtype,
                                 self.workspace)

    def layer(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, key_cache: torch.Tensor,
              value_cache: torch.Tensor, out: torch.Tensor, k_scale=None, v_scale=None) -> None:
        """One layer's attention of the step: append the new K/V rows at the
        step's slots, then attend over the shared block tables."""
        ops.reshape_and_cache(k, v, k_scale, v_scale, key_cache, value_cache,
                              self.allocator.slot_mapping)
        ops.paged_attention(q, k_scale, v_scale, key_cache, value_cache,
                            self.allocator.block_tables, self.allocator.context_lens, None,
                            self.max_context_len, self.scale, 1.0, None, out=out,
                            workspace=self.workspace, planned=True)

    def end(self, logits: torch.Tensor) -> None:
        """After the forward: next ids = argmax of the step's logits rows."""
        self.tokens.select(logits)
