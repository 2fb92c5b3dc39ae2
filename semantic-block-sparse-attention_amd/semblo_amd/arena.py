"""Fixed-address decode state of one layer (the reference's DecodeArena,
semblo/vllm_plugin/arena.py:66-253, reduced to what the HIP decode step reads).

It holds the prompt index (descriptors, sizes, run starts, the packed K/V),
a suffix store for the generated tokens, [2, NBLK, 256, Hkv, D], whose
blocks are addressed by absolute position through ``suffix_table``, and the
step's workspace.  Every buffer is allocated once, so a captured step replays
at fixed addresses.
"""
from __future__ import annotations

import torch


class DecodeArena:
    def __init__(self, index, *, reserve: int = 1024, suffix_block: int = 256,
                 suffix_splits: int = 8, shuffle_blocks: torch.Generator | None = None) -> None:
        self.index = index
        if index.packed_kv is None:
            raise ValueError("the arena needs the index's packed K/V (pack_prompt_kv)")
        dev = index.packed_kv.device
        hkv, d = index.packed_kv.shape[2], index.packed_kv.shape[3]
        self.num_clusters = index.num_buckets
        self.codebooks = index.codebooks
        self.sizes = index.bucket_sizes
        self.indptr = index.bucket_indptr
        self.packed_kv = index.packed_kv
        self.posting = index.posting_positions
        self.prompt_length = int(index.prompt_length)
        self.reserve = int(reserve)
        self.suffix_block = int(suffix_block)
        self.suffix_splits = int(suffix_splits)
        tile = 16
        self.max_tiles = -(-self.reserve // tile)
        # blocks from the one holding the prompt's end to the reservation's end
        base = self.prompt_length // self.suffix_block
        last = (self.prompt_length + self.max_tiles * tile) // self.suffix_block
        self.suffix_blocks = last - base + 1
        self.suffix_kv = torch.zeros(2, self.suffix_blocks, self.suffix_block, hkv, d,
                                     dtype=index.packed_kv.dtype, device=dev)
        table = torch.zeros(last + 1, dtype=torch.int32)
        phys = torch.arange(self.suffix_blocks, dtype=torch.int32)
        if shuffle_blocks is not None:
            phys = phys[torch.randperm(self.suffix_blocks, generator=shuffle_blocks)]
        table[base:last + 1] = phys
        self.suffix_table = table.to(dev)
        self.prompt_length_t = torch.tensor([self.prompt_length], dtype=torch.int32, device=dev)
        self.steps = 0          # decode steps taken through the layer (host count, no device read)

    def suffix_rows(self, positions: torch.Tensor, kv_head: int):
        """K and V of the generated tokens at ``positions`` (host helper for tests)."""
        pos = positions.to(self.suffix_table.device).long()
        blk = pos // self.suffix_block
        phys = self.suffix_table[blk].long()
        off = pos - blk * self.suffix_block
        return (self.suffix_kv[0, phys, off, kv_head], self.suffix_kv[1, phys, off, kv_head])
