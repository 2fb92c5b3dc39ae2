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

``DecodeArena.with_capacity`` makes an arena before any request, shaped for a
prompt capacity and a fixed cluster count (arena.py:66-160, vLLM's FULL graph
mode): a decode step captured on it at warm-up replays for every later request,
because ``adopt`` copies each request's index into the same buffers.  Clusters
past the request's own have size 0, an empty run and a zero descriptor, so no
selection reaches them (their zero scores still count in each component's
log-sum-exp, as in the reference's arena); the suffix table is rewritten for the
request's prompt length, and the step reads that length on the device.
"""
from __future__ import annotations

import torch

PACK_ALIGN = 256        # rows: the packed store's width is a multiple of this


def _upload(holder, table: torch.Tensor, dev) -> torch.Tensor:
    """``table`` on the device by an asynchronous copy from pinned memory, so that
    making or adopting an arena at the end of a prefill does not wait for the GPU to
    finish it (a copy from pageable memory would).  The pinned copy stays on
    ``holder`` until the next upload, which waits for this one first."""
    if torch.device(dev).type != "cuda":
        return table.to(dev, copy=True)
    prev = getattr(holder, "_upload_done", None)
    if prev is not None:
        prev.synchronize()
    pinned = table.pin_memory()
    out = pinned.to(dev, non_blocking=True)
    holder._upload_host = pinned
    holder._upload_done = torch.cuda.Event()
    holder._upload_done.record()
    return out


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
        self.suffix_table = _upload(self, table, dev)
        self.prompt_length_t = torch.full((1,), self.prompt_length, dtype=torch.int32, device=dev)
        self.steps = 0          # decode steps taken through the layer (host count, no device read)

    @property
    def reads_prompt_length_on_device(self) -> bool:
        """The decode step takes the prompt length from ``prompt_length_t`` (a flush
        moves it, an adoption sets it); otherwise it is the host value, known at capture."""
        return self.flush_room > 0 or self.capacity is not None

    capacity: int | None = None     # set by with_capacity: the arena outlives its requests

    @classmethod
    def with_capacity(cls, *, capacity: int, num_kv_heads: int, head_dim: int, num_clusters: int,
                      page_align: int = 16, reserve: int = 1024, suffix_block: int = 256,
                      suffix_splits: int = 8, dtype=torch.bfloat16, device="cuda") -> "DecodeArena":
        """An arena for prompts of up to ``capacity`` positions and ``num_clusters``
        clusters, made before any request (arena.py:66-130).  Until the first ``adopt``
        it holds a one-token index (cluster 0 of every head holds position 0, the other
        clusters are empty), so a step captured on it reads finite, zero K/V.  The suffix
        flush does not run on such an arena."""
        self = cls.__new__(cls)
        dev = torch.device(device)
        hkv, d, c = int(num_kv_heads), int(head_dim), int(num_clusters)
        self.capacity = int(capacity)
        self.num_clusters = c
        self.page_align = max(int(page_align), 1)
        self.reserve = int(reserve)
        self.suffix_block = int(suffix_block)
        self.suffix_splits = int(suffix_splits)
        self.flush_room = 0
        tile = 16
        self.max_tiles = -(-self.reserve // tile)
        bs = self.suffix_block
        width = self.capacity + c * self.page_align
        width += (-width) % PACK_ALIGN
        self.codebooks = torch.zeros(hkv, 2, c, d // 2, dtype=dtype, device=dev)
        self.sizes = torch.zeros(hkv, c, dtype=torch.int32, device=dev)
        self.indptr = torch.zeros(hkv, c + 1, dtype=torch.int32, device=dev)
        self.packed_kv = torch.zeros(2, width, hkv, d, dtype=dtype, device=dev)
        self.posting = torch.zeros(hkv, width, dtype=torch.int32, device=dev)
        self.inverse = None
        self.suffix_kpre_needed = False
        # positions L .. L + reserve - 1 of any prompt length L <= capacity span at most
        # reserve / bs + 2 blocks
        self.suffix_blocks = -(-self.reserve // bs) + 2
        self.suffix_kv = torch.zeros(2, self.suffix_blocks, bs, hkv, d, dtype=dtype, device=dev)
        self.suffix_kpre = None
        span = self.capacity + self.max_tiles * tile
        self.suffix_table = torch.zeros(span // bs + 2, dtype=torch.int32, device=dev)
        self.prompt_length_t = torch.zeros(1, dtype=torch.int32, device=dev)
        self.spare = None
        self.flushes = 0
        self.steps = 0
        self.index = None
        # the one-token index, with the prompt length at the capacity (arena.py:116-121)
        self.sizes[:, 0] = 1
        self.indptr[:, 1:] = 1
        self._map_suffix(self.capacity)
        return self

    def _map_suffix(self, prompt_length: int) -> None:
        """Blocks from the one holding the prompt's end onward map onto the suffix store
        in order, and the step reads the new prompt length."""
        bs = self.suffix_block
        base = int(prompt_length) // bs
        n = self.suffix_table.numel()
        table = torch.zeros(n, dtype=torch.int32)
        blocks = torch.arange(base, n)
        table[base:] = ((blocks - base) % self.suffix_blocks).to(torch.int32)
        self.suffix_table.copy_(_upload(self, table, self.suffix_table.device))
        self.prompt_length = int(prompt_length)
        self.first_prompt_length = int(prompt_length)
        self.prompt_length_t.fill_(int(prompt_length))

    def adopt(self, index) -> None:
        """Copy a request's finished index into this capacity arena (arena.py:160-253):
        every buffer keeps its address, so a step captured before the request replays
        over it.  Refuses an index larger than the arena."""
        if self.capacity is None:
            raise RuntimeError("adopt is for an arena made with_capacity")
        hkv, c = index.bucket_sizes.shape
        length = int(index.prompt_length)
        packed = index.packed_kv
        if packed is None:
            raise ValueError("the arena needs the index's packed K/V (pack_prompt_kv)")
        if hkv != self.sizes.shape[0] or packed.shape[3] != self.packed_kv.shape[3]:
            raise ValueError(f"index of {hkv} KV heads x D={packed.shape[3]} for an arena of "
                             f"{self.sizes.shape[0]} x D={self.packed_kv.shape[3]}")
        if c > self.num_clusters:
            raise ValueError(f"the index has {c} clusters; the arena holds {self.num_clusters}")
        if length > self.capacity:
            raise ValueError(f"a prompt of {length} positions; the arena holds {self.capacity}")
        rows = packed.shape[1]
        if rows > self.packed_kv.shape[1]:
            raise ValueError(f"{rows} packed rows; the arena holds {self.packed_kv.shape[1]}")
        self.codebooks.zero_()
        self.codebooks[:, :, :c].copy_(index.codebooks)
        self.sizes.zero_()
        self.sizes[:, :c].copy_(index.bucket_sizes)
        self.indptr[:, :c + 1].copy_(index.bucket_indptr)
        self.indptr[:, c + 1:] = index.bucket_indptr[:, c:c + 1]
        self.packed_kv[:, :rows].copy_(packed)
        npost = index.posting_positions.shape[1]
        self.posting[:, :npost].copy_(index.posting_positions)
        self._map_suffix(length)
        self.spare = None
        self.steps = 0
        self.index = index

    def suffix_rows(self, positions: torch.Tensor, kv_head: int):
        """K and V of the generated tokens at ``positions`` (host helper for tests)."""
        pos = positions.to(self.suffix_table.device).long()
        blk = pos // self.suffix_block
        phys = self.suffix_table[blk].long()
        off = pos - blk * self.suffix_block
        return (self.suffix_kv[0, phys, off, kv_head], self.suffix_kv[1, phys, off, kv_head])
