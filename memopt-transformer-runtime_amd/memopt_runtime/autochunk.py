"""AutoChunk: chunked prefill with a bounded activation footprint.

The reference advertises "AutoChunk Activation Chunking ... activation
dependencies are chunked temporally so the peak VRAM spike never exceeds
the physical GPU memory limit" (README.md:60, :430) and ships no code for
it. Here it is the prefill driver of the paged KV path: a long prompt is
written and attended in chunks of C tokens. Chunk i writes its K/V into the
cache, then its C queries attend causally (StreamingLLM window + sinks)
over everything written so far, so each query sees exactly the keys it
would see in one whole-prompt causal prefill; only the per-call buffers
(queries, outputs, the attention kernel's staged K/V workspace) scale with
C instead of the prompt length.
"""
from __future__ import annotations

from typing import Optional

import torch

import memopt_C

from .kv_cache import PagedKVCache

STAGED_BYTES_PER_TOKEN_HEAD_DIM = 4  # fp16 K + fp16 V of one (token, head, dim) in the staging workspace


def chunk_call_bytes(chunk: int, context_tokens: int, num_heads: int, head_dim: int, window: int = -1) -> int:
    """Device bytes of one chunk call over ``chunk`` queries at the end of
    ``context_tokens``: fp16 queries and outputs (2 * C * H * D * 2) and the
    staged fp16 K/V of the keys the call can see (min(context, C + window)
    tokens; the whole context without a window), 4 * H * D bytes each."""
    hd = num_heads * head_dim
    seen = min(context_tokens, chunk + window) if window > 0 else context_tokens
    return 2 * chunk * hd * 2 + STAGED_BYTES_PER_TOKEN_HEAD_DIM * hd * seen


def chunk_tokens_for_budget(budget_bytes: int, context_tokens: int, num_heads: int, head_dim: int,
                            window: int = -1, multiple: int = 128, minimum: int = 16) -> int:
    """Largest chunk (a multiple of ``multiple``, at most the context) whose
    :func:`chunk_call_bytes` fit ``budget_bytes``; ``minimum`` if none does."""
    lo, hi = 0, max(0, context_tokens // multiple)
    while lo < hi:  # chunk_call_bytes grows with the chunk: largest feasible count of `multiple`s
        mid = (lo + hi + 1) // 2
        if chunk_call_bytes(mid * multiple, context_tokens, num_heads, head_dim, window) <= budget_bytes:
            lo = mid
        else:
            hi = mid - 1
    return max(minimum, lo * multiple)


def autochunk_prefill(cache: PagedKVCache, seq_id: int, query: torch.Tensor, keys: torch.Tensor,
                      values: torch.Tensor, window_size: int = -1, num_sink_tokens: int = 0,
                      chunk_tokens: Optional[int] = None, budget_bytes: Optional[int] = None) -> torch.Tensor:
    """Prefill ``S`` new tokens of one sequence in chunks; returns fp16 ``[S, H, D]``.

    ``query``/``keys``/``values``: fp16 ``[S, H, D]``, the positions that
    follow the sequence's current length. The chunk size is ``chunk_tokens``
    or, with ``budget_bytes``, :func:`chunk_tokens_for_budget`; with neither
    the whole prompt is one chunk.
    """
    S, H, D = query.shape
    start = cache.length(seq_id)
    if chunk_tokens is None:
        chunk_tokens = (chunk_tokens_for_budget(budget_bytes, start + S, H, D, window_size)
                        if budget_bytes is not None else S)
    if chunk_tokens <= 0:
        raise RuntimeError("autochunk_prefill: chunk_tokens must be positive")
    out = torch.empty_like(query)
    k_pool, v_pool = cache.key_value_pools()
    for s0 in range(0, S, chunk_tokens):
        s1 = min(S, s0 + chunk_tokens)
        cache.append([seq_id], keys[s0:s1].unsqueeze(0), values[s0:s1].unsqueeze(0))
        bt = cache.block_tables([seq_id])
        ctx = cache.context_lens([seq_id])
        n = start + s1
        out[s0:s1] = memopt_C.dynamic_sparse_attention(query[s0:s1].unsqueeze(0), k_pool, v_pool, bt, ctx, n,
                                                      window_size, num_sink_tokens=num_sink_tokens,
                                                      causal=True)[0]
    return out
