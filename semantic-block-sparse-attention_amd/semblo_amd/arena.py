"""Fixed-address decode state of one layer (the reference's DecodeArena,
semblo/vllm_plugin/arena.py:66-253, reduced to what the HIP decode step reads).

It holds the prompt index (descriptors, sizes, run starts, the packed K/V),
a suffix store for the generated tokens, [2, NBLK, 256, Hkv, D], whose
blocks are addressed by absolute position through ``suffix_table``, and the
step's workspace.  Every buffer is allocated once, so a captured step replays
at fixed addresses.

With the suffix flush on (``flush_room`` > 0, suffix_flush.py) the arena also
keeps each generated token's pre-RoPE key beside its K/V, its packed store,
posting lists and inverse map have room for ``flush_room`` more positions, and
the block table maps every block a generation can reach onto the suffix store
as a ring (arena.py:186-202): a flush frees the oldest blocks and the blocks
that follow take them.  The decode step then reads the prompt length from
``prompt_length_t`` on the device, which a flush advances.
"""
from __future__ import annotations

import torch

PACK_ALIGN = 256        # rows: the packed store's width is a multiple of this


class DecodeArena:
    def __init__(self, index, *, reserve: int = 1024, suffix_block: int = 256,
                 suffix_splits: int = 8, shuffle_blocks: torch.Generator | None = None,
                 flush_room: int = 0) -> None:
        self.index = index
        if index.packed_kv is None:
            raise ValueError("the arena needs the index's packed K/V (pack_prompt_kv)")
        dev = index.packed_kv.device
        hkv, d = index.packed_kv.shape[2], index.packed_kv.shape[3]
        self.num_clusters = index.num_buckets
        self.codebooks = index.codebooks
        self.sizes = index.bucket_sizes
        self.indptr = index.bucket_indptr
        self.prompt_length = int(index.prompt_length)
        self.first_prompt_length = self.prompt_length      # before any flush
        self.page_align = max(int(getattr(index, "page_align", 16) or 1), 1)
        self.reserve = int(reserve)
        self.suffix_block = int(suffix_block)
        self.suffix_splits = int(suffix_splits)
        self.flush_room = max(0, int(flush_room))
        tile = 16
        self.max_tiles = -(-self.reserve // tile)
        bs = self.suffix_block
        if self.flush_room:
            # room for flush_room more positions in the clusters (arena.py:88-96)
            width = self.prompt_length + self.flush_room + self.num_clusters * self.page_align
            width += (-width) % PACK_ALIGN
            self.packed_kv = torch.zeros(2, width, hkv, d, dtype=index.packed_kv.dtype, device=dev)
            self.packed_kv[:, :index.packed_kv.shape[1]].copy_(index.packed_kv)
            self.posting = torch.zeros(hkv, width, dtype=torch.int32, device=dev)
            self.posting[:, :index.posting_positions.shape[1]].copy_(index.posting_positions)
            inv = index.inverse_positions()
            self.inverse = torch.zeros(hkv, self.prompt_length + self.flush_room, dtype=torch.int32,
                                       device=dev)
            self.inverse[:, :inv.shape[1]].copy_(inv)
            index.packed_kv = self.packed_kv
            index.posting_positions = self.posting
            index._inverse_positions = self.inverse
            self.suffix_kpre_needed = True
        else:
            self.packed_kv = index.packed_kv
            self.posting = index.posting_positions
            self.inverse = None
            self.suffix_kpre_needed = False
        self.spare = None                 # the other store of a flush's repack, made at the first
        self.flushes = 0
        # blocks from the one holding the prompt's end to the reservation's end
        base = self.prompt_length // bs
        last = (self.prompt_length + self.max_tiles * tile) // bs
        self.suffix_blocks = last - base + 1
        self.suffix_kv = torch.zeros(2, self.suffix_blocks, bs, hkv, d,
                                     dtype=index.packed_kv.dtype, device=dev)
        self.suffix_kpre = (torch.zeros(self.suffix_blocks, bs, hkv, d, dtype=index.packed_kv.dtype,
                                        device=dev) if self.suffix_kpre_needed else None)
        # logical block b >= base -> physical block perm[(b - base) mod NBLK]: the
        # identity over the reservation without a flush, a ring with one
        span = self.prompt_length + self.flush_room + self.max_tiles * tile
        table = torch.zeros(span // bs + 1, dtype=torch.int32)
        phys = torch.arange(self.suffix_blocks, dtype=torch.int32)
        if shuffle_blocks is not None:
            phys = phys[torch.randperm(self.suffix_blocks, generator=shuffle_blocks)]
        blocks = torch.arange(base, table.numel())
        table[base:] = phys[(blocks - base) % self.suffix_blocks]
        self.suffix_table = table.to(dev)
        self.prompt_length_t = torch.tensor([self.prompt_length], dtype=torch.int32, device=dev)
        self.steps = 0          # decode steps taken through the layer (host count, no device read)

    @property
    def reads_prompt_length_on_device(self) -> bool:
        """The decode step takes the prompt length from ``prompt_length_t`` (a flush
        moves it); without the flush it is the host value, known at capture."""
        return self.flush_room > 0

    def suffix_rows(self, positions: torch.Tensor, kv_head: int):
        """K and V of the generated tokens at ``positions`` (host helper for tests)."""
        pos = positions.to(self.suffix_table.device).long()
        blk = pos // self.suffix_block
        phys = self.suffix_table[blk].long()
        off = pos - blk * self.suffix_block
        return (self.suffix_kv[0, phys, off, kv_head], self.suffix_kv[1, phys, off, kv_head])
