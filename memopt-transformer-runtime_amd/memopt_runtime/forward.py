"""Policy forward wrapper: applies MemoryScheduler's policy to the paged KV path.

The reference's ``MemoryScheduler`` maintains ``retain_ratio`` and
``use_int4`` and documents that "the forward wrapper" applies them
(src/memopt/scheduler.py:9-18, :215-242), but no reference code reads
them. ``PolicyForward`` is that wrapper for one attention layer's step:

* ``use_int4`` selects the pool format: when it changes, the live pool is
  converted (fp16 pages quantized into INT4 pages, or INT4 pages
  dequantized), keeping every block table valid;
* the new tokens' K/V are appended (fused group-64 quantize for INT4 pages);
* attention runs over the paged cache (decode: one query per sequence;
  prefill/chunk: causal StreamingLLM mask), with the layer's window and
  attention sinks;
* ``retain_ratio < 1`` with per-token scores runs Ada-KV eviction
  (``evict_tokens``) and returns fully evicted pages to the pool.

The policy source is any object with ``retain_ratio`` and ``use_int4``
attributes, e.g. the reference's ``MemoryScheduler``; when it has a
``_lock`` (as ``MemoryScheduler`` does, src/memopt/scheduler.py:151-158) both
values are read under it, as one snapshot.
"""
from __future__ import annotations

from contextlib import nullcontext
from dataclasses import dataclass
from typing import Optional, Sequence, Tuple

import torch

import memopt_C

from .kv_cache import PagedKVCache


@dataclass(frozen=True)
class Policy:
    """One snapshot of the scheduler's policy variables."""
    retain_ratio: float = 1.0
    use_int4: bool = False


def read_policy(source) -> Policy:
    """Atomic snapshot of ``source.retain_ratio`` / ``source.use_int4``."""
    if source is None:
        return Policy()
    lock = getattr(source, "_lock", None)
    with (lock if lock is not None else nullcontext()):
        # MemoryScheduler's properties take the (non-reentrant) lock themselves,
        # so read the backing fields when they exist.
        rr = getattr(source, "_retain_ratio", None)
        q = getattr(source, "_use_int4", None)
        if rr is None or q is None:
            rr, q = source.retain_ratio, source.use_int4
    return Policy(float(rr), bool(q))


class PolicyForward:
    """One attention layer's paged-KV step under a memory policy.

    Args:
        cache: the sequences' paged cache.
        policy_source: object exposing ``retain_ratio`` / ``use_int4``
            (e.g. ``memopt.MemoryScheduler``); ``None`` = full retention, fp16.
        window_size: keys visible behind each query (``<= 0``: all).
        num_sink_tokens: leading tokens always visible and never evicted.
    """

    def __init__(self, cache: PagedKVCache, policy_source=None, window_size: int = -1,
                 num_sink_tokens: int = 4) -> None:
        self.cache = cache
        self.policy_source = policy_source
        self.window_size = window_size
        self.num_sink_tokens = num_sink_tokens
        self.last_policy = Policy()
        self.conversions = 0
        self.evicted_pages = 0

    def apply_format(self, policy: Policy) -> None:
        want = "int4" if policy.use_int4 else "fp16"
        if self.cache.kv_format != want:
            self.cache.convert(want)
            self.conversions += 1

    def step(self, seq_ids: Sequence[int], query: torch.Tensor, keys: torch.Tensor, values: torch.Tensor,
             scores: Optional[torch.Tensor] = None) -> torch.Tensor:
        """Append the new tokens, attend, then evict under the current policy.

        ``query``/``keys``/``values``: fp16 ``[B, T, H, D]`` (T new tokens
        per sequence; T = 1 for decode). ``scores``: optional f32
        ``[B, H, L]`` per-token scores used for eviction when
        ``retain_ratio < 1``. Returns fp16 ``[B, T, H, D]``.
        """
        policy = read_policy(self.policy_source)
        self.last_policy = policy
        self.apply_format(policy)
        self.cache.append(seq_ids, keys, values)
        out = self.attend(seq_ids, query)
        if policy.retain_ratio < 1.0 and scores is not None:
            self.evicted_pages += len(self.cache.evict(seq_ids, scores, policy.retain_ratio, self.num_sink_tokens))
        return out

    def attend(self, seq_ids: Sequence[int], query: torch.Tensor) -> torch.Tensor:
        """Attention of ``query`` ``[B, T, H, D]`` (the last T positions of each
        sequence) over the paged cache."""
        T = query.shape[1]
        bt = self.cache.block_tables(seq_ids)
        ctx = self.cache.context_lens(seq_ids)
        max_len = max(self.cache.length(s) for s in seq_ids)
        k, v = self.cache.key_value_pools()
        return memopt_C.dynamic_sparse_attention(query, k, v, bt, ctx, max_len, self.window_size,
                                                 num_sink_tokens=self.num_sink_tokens, causal=T > 1)


def attention_inputs(cache: PagedKVCache, seq_ids: Sequence[int]) -> Tuple[torch.Tensor, torch.Tensor, int]:
    """``(block_tables, context_lens, max_seq_len)`` of ``seq_ids``, the paged
    arguments ``DynamicAttention.forward`` expects (src/memopt/attention.py:204-240)."""
    return cache.block_tables(seq_ids), cache.context_lens(seq_ids), max(cache.length(s) for s in seq_ids)
