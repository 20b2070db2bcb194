"""bench.py's clock sampler (host logic, no GPU): AMD SMI's clock is the
power-management firmware's snapshot, refreshed about once a second, so the
sampler keeps one value per snapshot (keyed by its firmware timestamp) and
counts the reads apart; a source without timestamps keeps every read."""

import sys
import time
from pathlib import Path

sys.path.insert(0, str(Path(__file__).resolve().parents[1]))

import bench  # noqa: E402


class FakeClock:
    """Replays (MHz, stamp) reads, then repeats the last one."""

    def __init__(self, reads):
        self.reads, self.i = list(reads), 0

    def gpu_clock_sample(self):
        r = self.reads[min(self.i, len(self.reads) - 1)]
        self.i += 1
        return r


def sample(reads, seconds=0.05):
    s = bench.ClockSampler(FakeClock(reads), period_s=0.001)
    with s:
        time.sleep(seconds)
    return s


def test_one_value_per_firmware_snapshot():
    s = sample([(205.6, 10**9)] * 5 + [(2279.1, 2 * 10**9)] * 5 + [(2396.1, 3 * 10**9)])
    summary = s.summary()
    assert s.samples == [205.6, 2279.1, 2396.1]
    assert summary["samples"] == 3 and summary["reads"] > 3
    assert summary["min_mhz"] == 205.6 and summary["max_mhz"] == 2396.1 and summary["median_mhz"] == 2279.1
    assert summary["snapshot_refresh_s"] == 1.0


def test_reads_without_a_timestamp_each_count():
    s = sample([(1900.0, 0), (2000.0, 0), (2100.0, 0)], seconds=0.02)
    assert s.samples[:3] == [1900.0, 2000.0, 2100.0]
    assert s.summary()["snapshot_refresh_s"] is None


def test_an_unreadable_clock_gives_no_samples():
    summary = sample([(0.0, 0)], seconds=0.01).summary()
    assert summary["samples"] == 0 and summary["reads"] == 0
