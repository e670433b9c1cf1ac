"""Host-side runtime of the paged INT4 KV path on top of ``memopt_C``.

* :class:`PagedKVCache` — sequence block tables, slot mappings and context
  lengths over the ``memopt_C`` pool; the decode append step.
* :class:`PolicyForward` — applies ``MemoryScheduler``'s ``use_int4`` /
  ``retain_ratio`` to one attention layer's step.
* :func:`autochunk_prefill` — chunked prefill with a bounded footprint.
* :class:`ThresholdPolicy` — ``MemoryScheduler``'s threshold rule as a
  policy source, for runs without the reference package.

All device work runs in the HIP library behind ``memopt_C``; importing this
package fails when that library is missing.
"""
from .autochunk import autochunk_prefill, chunk_call_bytes, chunk_tokens_for_budget
from .forward import Policy, PolicyForward, attention_inputs, read_policy
from .kv_cache import PagedKVCache, pages_needed, slots_for
from .policy import ThresholdPolicy, vram_utilization

__all__ = ["PagedKVCache", "PolicyForward", "Policy", "read_policy", "attention_inputs", "autochunk_prefill",
           "chunk_tokens_for_budget", "chunk_call_bytes", "pages_needed", "slots_for", "ThresholdPolicy",
           "vram_utilization"]
