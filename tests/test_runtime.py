"""CPU tests of the host runtime's pure logic: slot mappings, page counts,
AutoChunk's budget-derived chunk size and the policy snapshot (no GPU)."""
import threading

import pytest

import memopt_runtime as R


def test_slots_follow_the_block_table():
    # positions 14..18 of a sequence on pages [5, 2, 9] with 16-token pages
    assert R.slots_for([5, 2, 9], 14, 5, 16) == [5 * 16 + 14, 5 * 16 + 15, 2 * 16, 2 * 16 + 1, 2 * 16 + 2]
    assert R.slots_for([3], 0, 0, 16) == []
    with pytest.raises(RuntimeError, match="unlinked"):
        R.slots_for([4, -1], 16, 1, 16)
    assert [R.pages_needed(n, 16) for n in (0, 1, 16, 17, 4096)] == [0, 1, 1, 2, 256]


def test_chunk_size_fits_budget():
    H, D = 32, 128
    hd = H * D
    # the cost model: fp16 queries and outputs plus staged K/V of the visible keys
    assert R.chunk_call_bytes(1024, 16384, H, D, 4096) == 2 * 1024 * hd * 2 + 4 * hd * 5120
    assert R.chunk_call_bytes(1024, 16384, H, D, -1) == 2 * 1024 * hd * 2 + 4 * hd * 16384
    assert R.chunk_call_bytes(15000, 16384, H, D, 4096) == 2 * 15000 * hd * 2 + 4 * hd * 16384
    for budget in (8 << 20, 64 << 20, 300 << 20, 512 << 20, 4 << 30):
        for window in (-1, 4096):
            c = R.chunk_tokens_for_budget(budget, 16384, H, D, window)
            if c == 16:
                continue
            assert c % 128 == 0 and c <= 16384
            assert R.chunk_call_bytes(c, 16384, H, D, window) <= budget
            if c < 16384:  # the next multiple does not fit
                assert R.chunk_call_bytes(c + 128, 16384, H, D, window) > budget
    assert R.chunk_tokens_for_budget(1, 16384, H, D) == 16  # floor
    assert R.chunk_tokens_for_budget(1 << 40, 16384, H, D) == 16384  # whole prompt


class _Scheduler:
    """MemoryScheduler's policy fields behind its non-reentrant lock
    (src/memopt/scheduler.py:151-172, :212-233)."""

    def __init__(self, rr, q):
        self._lock = threading.Lock()
        self._retain_ratio, self._use_int4 = rr, q

    @property
    def retain_ratio(self):
        with self._lock:
            return self._retain_ratio

    @property
    def use_int4(self):
        with self._lock:
            return self._use_int4


class _Plain:
    retain_ratio = 0.75
    use_int4 = True


def test_policy_snapshot():
    assert R.read_policy(None) == R.Policy(1.0, False)
    assert R.read_policy(_Scheduler(0.75, True)) == R.Policy(0.75, True)
    assert R.read_policy(_Plain()) == R.Policy(0.75, True)
    # the snapshot holds the scheduler's lock: a writer waits for it
    s = _Scheduler(1.0, False)
    s._lock.acquire()
    got = []
    t = threading.Thread(target=lambda: got.append(R.read_policy(s)))
    t.start()
    t.join(0.2)
    assert t.is_alive() and not got
    s._retain_ratio, s._use_int4 = 0.5, True
    s._lock.release()
    t.join(5)
    assert got == [R.Policy(0.5, True)]


def test_threshold_policy_rule():
    """MemoryScheduler.adjust_policy's rule (src/memopt/scheduler.py:357-369):
    high -> drop ratio + INT4, low -> full + fp16, dead band -> unchanged."""
    p = R.ThresholdPolicy(vram_high_threshold=0.85, vram_low_threshold=0.5, drop_retain_ratio=0.75)
    assert R.read_policy(p) == R.Policy(1.0, False)
    assert p.adjust_policy(0.7) is False and R.read_policy(p) == R.Policy(1.0, False)   # dead band
    assert p.adjust_policy(0.85) is True and R.read_policy(p) == R.Policy(0.75, True)   # at the high mark
    assert p.adjust_policy(0.6) is False and R.read_policy(p) == R.Policy(0.75, True)   # hysteresis
    assert p.adjust_policy(0.5) is True and R.read_policy(p) == R.Policy(1.0, False)    # at the low mark
    # config 5's forcing: any allocation crosses a tiny high mark
    f = R.ThresholdPolicy(vram_high_threshold=1e-9, vram_low_threshold=0.0, drop_retain_ratio=0.75)
    assert f.adjust_policy(1e-6) and (f.retain_ratio, f.use_int4) == (0.75, True)


@pytest.mark.parametrize("kw", [dict(vram_high_threshold=0.0), dict(vram_high_threshold=1.5),
                                dict(vram_low_threshold=0.9, vram_high_threshold=0.9),
                                dict(drop_retain_ratio=1.0), dict(drop_retain_ratio=-0.1)])
def test_threshold_policy_validation(kw):
    """SchedulerConfig's range checks (src/memopt/scheduler.py:90-106)."""
    with pytest.raises(ValueError):
        R.ThresholdPolicy(**kw)
