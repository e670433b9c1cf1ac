"""A policy source with ``MemoryScheduler``'s threshold rule.

The reference's ``MemoryScheduler`` (src/memopt/scheduler.py:114-436) polls
VRAM in a background thread and, in ``adjust_policy`` (:338-384), moves
``retain_ratio`` / ``use_int4`` with hysteresis: utilization at or above
``vram_high_threshold`` sets ``drop_retain_ratio`` and INT4, at or below
``vram_low_threshold`` restores full retention and fp16, anything between
leaves the state alone. Utilization is ``torch.cuda.memory_allocated()``
over the device's total memory (:444-461).

``ThresholdPolicy`` applies that rule on demand, without the thread, and
keeps the scheduler's field names (``_lock``, ``_retain_ratio``,
``_use_int4``; ``retain_ratio`` / ``use_int4`` properties), so
``PolicyForward`` reads it exactly as it reads a ``MemoryScheduler``. It
serves runs where the reference package is not installed (a GPU box running
only this library); with the package, pass the real scheduler instead.
"""
from __future__ import annotations

import threading
from typing import Optional

import torch


def vram_utilization(device: Optional[int] = None) -> Optional[float]:
    """Bytes allocated by torch tensors over the device's total memory
    (src/memopt/scheduler.py:444-461); ``None`` when it cannot be sampled."""
    try:
        dev = torch.cuda.current_device() if device is None else device
        total = torch.cuda.get_device_properties(dev).total_memory
        if total == 0:
            return None
        return torch.cuda.memory_allocated(dev) / total
    except Exception:  # noqa: BLE001 - no device, or a failed query
        return None


class ThresholdPolicy:
    """``retain_ratio`` / ``use_int4`` under ``MemoryScheduler``'s threshold rule.

    Arguments and their checks follow ``SchedulerConfig``
    (src/memopt/scheduler.py:63-106): ``0 < vram_high_threshold <= 1``,
    ``0 <= vram_low_threshold < vram_high_threshold``,
    ``0 <= drop_retain_ratio < 1``; violations raise ``ValueError``. The
    state starts at full retention, fp16 (:177-178).
    """

    def __init__(self, vram_high_threshold: float = 0.85, vram_low_threshold: float = 0.50,
                 drop_retain_ratio: float = 0.75) -> None:
        if not (0.0 < vram_high_threshold <= 1.0):
            raise ValueError(f"vram_high_threshold must be in (0.0, 1.0], got {vram_high_threshold}")
        if not (0.0 <= vram_low_threshold < vram_high_threshold):
            raise ValueError("vram_low_threshold must be in [0.0, vram_high_threshold), "
                             f"got low={vram_low_threshold}, high={vram_high_threshold}")
        if not (0.0 <= drop_retain_ratio < 1.0):
            raise ValueError(f"drop_retain_ratio must be in [0.0, 1.0), got {drop_retain_ratio}")
        self.vram_high_threshold = vram_high_threshold
        self.vram_low_threshold = vram_low_threshold
        self.drop_retain_ratio = drop_retain_ratio
        self._lock = threading.Lock()
        self._retain_ratio = 1.0
        self._use_int4 = False

    @property
    def retain_ratio(self) -> float:
        with self._lock:
            return self._retain_ratio

    @property
    def use_int4(self) -> bool:
        with self._lock:
            return self._use_int4

    def adjust_policy(self, utilization: Optional[float] = None) -> bool:
        """Apply the threshold rule to ``utilization`` (sampled from the
        current device when ``None``); returns whether the policy changed.
        A failed sample leaves the state unchanged (:353-355)."""
        if utilization is None:
            utilization = vram_utilization()
        if utilization is None:
            return False
        with self._lock:
            old = (self._retain_ratio, self._use_int4)
            if utilization >= self.vram_high_threshold:
                self._retain_ratio, self._use_int4 = self.drop_retain_ratio, True
            elif utilization <= self.vram_low_threshold:
                self._retain_ratio, self._use_int4 = 1.0, False
            return (self._retain_ratio, self._use_int4) != old
