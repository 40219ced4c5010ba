"""Decode graphs per (batch bucket, block-table column bucket), replayed with
padded metadata: the runtime side of vASR's CUDA decode graphs.

The reference keeps one captured decode graph per key (batch bucket 1, 2,
4, 8, then multiples of 16; table columns rounded up to a power of two of
at least 256 / block_size), captures on a miss, evicts the smallest key
once 256 graphs are held, and before every replay pads the step's inputs
to the key's shape and copies them into the graph's buffers: padded rows
get id 0, slot 0 (block 0, the null block), context 1 and table row 0;
table columns past the step's width repeat each row's last column; the
graph's max_context_len is frozen at columns x block_size. The outputs of
the real rows are then narrowed out (paged_cache_runtime.rs:498-704,
cuda_graph.rs:28-81, 131-243, 342-486).

Here the padding and copies run on the device (no host round trip), before
the replay and outside the graph. The captured forward is the caller's
(this package has no model): ``forward(bufs, max_context_len)`` reads the
padded buffers ``bufs`` (``input_ids`` u32 [batch], ``slot_mapping`` i64,
``context_lens`` u32, ``block_tables`` u32 [batch, cols], and every per-row
input named in ``row_inputs``) and returns a tensor (or tuple of tensors)
whose first dimension is the batch; it must allocate nothing it returns
outside the graph pool and read nothing on the host, like every op of this
package."""

from __future__ import annotations

from typing import Callable, Dict, Optional, Tuple

import torch

from . import host

MAX_GRAPHS = 256  # CUDA_DECODE_GRAPH_MAX_GRAPHS, cuda_graph.rs:21


class _Entry:
    def __init__(self, graph, bufs, out, max_context_len):
        self.graph, self.bufs, self.out, self.max_context_len = graph, bufs, out, max_context_len


class DecodeGraphCache:
    def __init__(self, forward: Callable, max_batch: int, block_size: int,
                 row_inputs: Dict[str, Tuple[Tuple[int, ...], torch.dtype]], device,
                 max_graphs: int = MAX_GRAPHS):
        """row_inputs: name -> (shape after the batch dimension, dtype) of the
        per-row inputs the forward reads (e.g. q / k / v of every layer)."""
        if max_batch <= 0 or block_size <= 0 or max_graphs <= 0:
            raise ValueError("max_batch, block_size and max_graphs must be positive")
        self.forward, self.max_batch, self.block_size = forward, max_batch, block_size
        self.row_inputs = dict(row_inputs)
        self.device = torch.device(device)
        self.max_graphs = max_graphs
        self.graphs: Dict[Tuple[int, int], _Entry] = {}
        self.captures = 0

    def key(self, actual_batch: int, cols: int) -> Tuple[int, int]:
        """(batch bucket, column bucket) of a step (cuda_decode_graph_key,
        paged_cache_runtime.rs:499-528)."""
        if actual_batch <= 0 or actual_batch > self.max_batch:
            raise ValueError(f"decode batch must be in 1..={self.max_batch}; got {actual_batch}")
        b = host.cuda_graph_batch_bucket(actual_batch, self.max_batch)
        if b is None:
            raise ValueError(f"no batch bucket for {actual_batch} (max {self.max_batch})")
        return b, host.bucket_block_table_cols(cols, self.block_size)

    def _buffers(self, batch: int, cols: int) -> Dict[str, torch.Tensor]:
        d = self.device
        bufs = {"input_ids": torch.zeros(batch, dtype=torch.uint32, device=d),
                "slot_mapping": torch.zeros(batch, dtype=torch.int64, device=d),
                "context_lens": torch.ones(batch, dtype=torch.uint32, device=d),
                "block_tables": torch.zeros((batch, cols), dtype=torch.uint32, device=d)}
        for name, (shape, dtype) in self.row_inputs.items():
            bufs[name] = torch.zeros((batch,) + tuple(shape), dtype=dtype, device=d)
        return bufs

    def _insert(self, key, entry) -> None:
        if len(self.graphs) >= self.max_graphs and key not in self.graphs:
            del self.graphs[min(self.graphs)]  # the smallest key, as the reference's ordered map
        self.graphs[key] = entry

    def _capture(self, key) -> _Entry:
        batch, cols = key
        bufs = self._buffers(batch, cols)
        max_ctx = cols * self.block_size
        stream = torch.cuda.Stream(device=self.device)
        stream.wait_stream(torch.cuda.current_stream(self.device))
        with torch.cuda.stream(stream):
            self.forward(bufs, max_ctx)  # warm-up on the padded (pad rows only) buffers
        torch.cuda.current_stream(self.device).wait_stream(stream)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            out = self.forward(bufs, max_ctx)
        self.captures += 1
        return _Entry(graph, bufs, out, max_ctx)

    def prewarm(self, col_buckets: Optional[Tuple[int, ...]] = None) -> int:
        """Capture every batch bucket for the base column bucket and twice it
        (prewarm_cuda_decode_graphs, paged_cache_runtime.rs:651-704)."""
        base = host.bucket_block_table_cols(1, self.block_size)
        n = 0
        for cols in (col_buckets or (base, 2 * base)):
            for b in host.cuda_graph_batch_buckets(self.max_batch):
                if (b, cols) not in self.graphs:
                    self._insert((b, cols), self._capture((b, cols)))
                    n += 1
        return n

    def run(self, input_ids: torch.Tensor, slot_mapping: torch.Tensor,
            context_lens: torch.Tensor, block_tables: torch.Tensor,
            rows: Optional[Dict[str, torch.Tensor]] = None):
        """Pad this step's inputs into the key's graph buffers, replay, and
        return the forward's outputs narrowed to the real rows."""
        a = int(input_ids.shape[0])
        cols = int(block_tables.shape[1])
        key = self.key(a, cols)
        entry = self.graphs.get(key)
        if entry is None:
            entry = self._capture(key)
            self._insert(key, entry)
        b, gc = key
        bufs = entry.bufs
        bufs["input_ids"][:a].copy_(input_ids)
        bufs["input_ids"][a:].zero_()
        bufs["slot_mapping"][:a].copy_(slot_mapping)
        bufs["slot_mapping"][a:].zero_()
        bufs["context_lens"][:a].copy_(context_lens)
        bufs["context_lens"][a:].fill_(1)
        bt = bufs["block_tables"]
        bt[:a, :cols].copy_(block_tables)
        if gc > cols:
            bt[:a, cols:].copy_(block_tables[:, cols - 1:cols].expand(a, gc - cols))
        bt[a:].zero_()
        for name, x in (rows or {}).items():
            bufs[name][:a].copy_(x)
            bufs[name][a:].zero_()
        entry.graph.replay()
        if isinstance(entry.out, (tuple, list)):
            return type(entry.out)(o[:a] for o in entry.out)
        return entry.out[:a]
