"""Sequence-level paged KV cache over the ``memopt_C`` pool.

The reference leaves block tables, slot mappings and context lengths to its
caller: ``DynamicAttention.forward`` takes them as arguments
(src/memopt/attention.py:204-274) and no reference code builds them. This
module is that caller-side bookkeeping for the one pool ``memopt_C`` keeps
(src/csrc/kv_cache.cu:83-201): pages are taken from the FIFO free list with
``allocate_block`` as sequences grow, a sequence's block table lists its
pages in token order, and ``context_lens`` are the tokens written so far.

Every device operation goes through ``memopt_C`` (HIP kernels); the host
side only does list bookkeeping and builds the small index tensors.
"""
from __future__ import annotations

from typing import Dict, Iterable, List, Optional, Sequence

import numpy as np
import torch

import memopt_C


def slots_for(pages: Sequence[int], start: int, count: int, block_size: int) -> List[int]:
    """Flat pool slots (``page * block_size + offset``) of token positions
    ``start .. start + count - 1`` of a sequence whose logical blocks map to
    ``pages`` (the slot_mapping convention of src/csrc/kv_cache.cu:244-259)."""
    out = []
    for pos in range(start, start + count):
        page = pages[pos // block_size]
        if page < 0:
            raise RuntimeError(f"slot of position {pos}: logical block {pos // block_size} is unlinked")
        out.append(page * block_size + pos % block_size)
    return out


def pages_needed(length: int, block_size: int) -> int:
    """Logical blocks covering ``length`` tokens."""
    return (length + block_size - 1) // block_size


class PagedKVCache:
    """Block tables and lengths of a set of sequences stored in the ``memopt_C`` pool.

    Args:
        num_blocks: pool pages (``init_pool``).
        num_heads, head_dim: pool geometry.
        block_size: tokens per page (16 for INT4 page pools).
        kv_format: ``"fp16"`` (reference layout) or ``"int4"`` (INT4 pages).

    The pool is the process-wide ``memopt_C`` pool and this cache owns its
    free list: construction starts a fresh pool (any previous one, and the
    block tables built on it, are dropped).
    """

    def __init__(self, num_blocks: int, num_heads: int, head_dim: int, block_size: int = 16,
                 kv_format: str = "fp16") -> None:
        memopt_C.reset_pool()
        memopt_C.init_pool(num_blocks, block_size, num_heads, head_dim, kv_format=kv_format)
        self.num_blocks = num_blocks
        self.num_heads = num_heads
        self.head_dim = head_dim
        self.block_size = block_size
        self._pages: Dict[int, List[int]] = {}
        self._len: Dict[int, int] = {}

    # -- pool ---------------------------------------------------------------
    @property
    def kv_format(self) -> str:
        return memopt_C.pool_kv_format()

    @property
    def device(self) -> torch.device:
        return memopt_C.get_key_pool().device

    def key_value_pools(self):
        """The pool views ``dynamic_sparse_attention`` takes (``get_key_pool`` / ``get_value_pool``)."""
        return memopt_C.get_key_pool(), memopt_C.get_value_pool()

    def convert(self, kv_format: str) -> None:
        """Switch the pool between fp16 and INT4 storage; block tables stay valid."""
        memopt_C.convert_pool(kv_format)

    # -- sequences ----------------------------------------------------------
    def add_sequence(self, seq_id: int) -> None:
        if seq_id in self._pages:
            raise RuntimeError(f"sequence {seq_id} already exists")
        self._pages[seq_id] = []
        self._len[seq_id] = 0

    def free_sequence(self, seq_id: int) -> None:
        """Return the sequence's linked pages to the pool's free list."""
        for page in self._pages.pop(seq_id):
            if page >= 0:
                memopt_C.free_block(page)
        del self._len[seq_id]

    def length(self, seq_id: int) -> int:
        return self._len[seq_id]

    def pages(self, seq_id: int) -> List[int]:
        return list(self._pages[seq_id])

    def reserve(self, seq_id: int, new_tokens: int) -> None:
        """Allocate the pages ``new_tokens`` more tokens need. On exhaustion
        the pages taken by this call go back and ``RuntimeError`` is raised
        (``allocate_block`` returns -1, src/csrc/kv_cache.cu:163-172)."""
        pages = self._pages[seq_id]
        need = pages_needed(self._len[seq_id] + new_tokens, self.block_size) - len(pages)
        taken = []
        for _ in range(max(0, need)):
            b = memopt_C.allocate_block()
            if b < 0:
                for t in taken:
                    memopt_C.free_block(t)
                raise RuntimeError(f"PagedKVCache: pool exhausted (sequence {seq_id} needs {need} more pages)")
            taken.append(b)
        pages.extend(taken)

    # -- index tensors ------------------------------------------------------
    def block_tables(self, seq_ids: Sequence[int], max_blocks: Optional[int] = None) -> torch.Tensor:
        """int32 ``[B, M]`` block table, -1 past a sequence's pages (and for unlinked blocks)."""
        M = max_blocks if max_blocks is not None else max(1, max(len(self._pages[s]) for s in seq_ids))
        rows = []
        for s in seq_ids:
            p = self._pages[s]
            if len(p) > M:
                raise RuntimeError(f"sequence {s} has {len(p)} pages, more than max_blocks={M}")
            rows.append(p + [-1] * (M - len(p)))
        # (through numpy: half the host time of torch.tensor on nested lists)
        return torch.from_numpy(np.array(rows, dtype=np.int32)).to(self.device)

    def context_lens(self, seq_ids: Sequence[int]) -> torch.Tensor:
        return torch.tensor([self._len[s] for s in seq_ids], dtype=torch.int32).to(self.device)

    def slot_mapping(self, seq_ids: Sequence[int], new_tokens: int) -> torch.Tensor:
        """int32 slots of the next ``new_tokens`` positions of each sequence (sequence-major)."""
        slots: List[int] = []
        for s in seq_ids:
            slots += slots_for(self._pages[s], self._len[s], new_tokens, self.block_size)
        return torch.from_numpy(np.array(slots, dtype=np.int32)).to(self.device)

    # -- writes -------------------------------------------------------------
    def append(self, seq_ids: Sequence[int], keys: torch.Tensor, values: torch.Tensor) -> None:
        """Decode append step: write the next tokens of every sequence.

        ``keys`` / ``values``: fp16 ``[B, T, H, D]`` (T new tokens each) or
        ``[B, H, D]`` (one token each). Pages are reserved first, then one
        ``write_cache`` call scatters (fp16 pool) or quantizes (INT4 pages)
        all ``B*T`` rows; the context lengths advance by T.
        """
        if keys.dim() == 3:
            keys, values = keys.unsqueeze(1), values.unsqueeze(1)
        B, T, H, D = keys.shape
        if B != len(seq_ids):
            raise RuntimeError("append: keys batch != number of sequences")
        for s in seq_ids:
            self.reserve(s, T)
        slots = self.slot_mapping(seq_ids, T)
        bt = self.block_tables(seq_ids)
        # Slots come from pages this cache allocated: in range by construction.
        memopt_C.write_cache(keys.reshape(B * T, H, D), values.reshape(B * T, H, D), bt, slots,
                             validate_slots=False)
        for s in seq_ids:
            self._len[s] += T

    # -- eviction -------------------------------------------------------------
    def evict(self, seq_ids: Sequence[int], scores: torch.Tensor, retain_ratio: float,
              num_sink_tokens: int = 4) -> List[int]:
        """Ada-KV eviction of the sequences' tokens, then the free-list sweep.

        ``scores``: f32 ``[B, H, L]`` per-token scores over the first L
        positions. ``evict_tokens`` zeroes evicted rows and unlinks blocks
        evicted in every head; ``free_evicted_blocks`` returns those pages to
        the pool (src/csrc/kv_cache.cu:1033-1036). Unlinked blocks stay as
        holes (-1) in the sequence's block table, which attention skips.
        Returns the freed page ids.
        """
        L = scores.shape[2]
        M = max(pages_needed(L, self.block_size), max(len(self._pages[s]) for s in seq_ids))
        bt = self.block_tables(seq_ids, M)
        ibf = torch.zeros(self.num_blocks, dtype=torch.int32, device=bt.device)
        memopt_C.evict_tokens(scores, bt, ibf, retain_ratio, num_sink_tokens)
        freed = memopt_C.free_evicted_blocks(ibf)
        new_bt = bt.cpu().tolist()
        for s, row in zip(seq_ids, new_bt):
            n = len(self._pages[s])
            self._pages[s] = row[:n]
        return freed

    def linked_pages(self, seq_ids: Iterable[int]) -> int:
        return sum(1 for s in seq_ids for p in self._pages[s] if p >= 0)
