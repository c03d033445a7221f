"""Benchmark statistics: raw samples plus p10/p50/p90/p99 latency and throughput
(src/nanoquant/runtime/benchmark.py:12-112) and aligned profile accounting
(src/nanoquant/runtime/profiling.py:8-49)."""

from __future__ import annotations

import math
import time
from collections.abc import Callable, Mapping, Sequence
from dataclasses import dataclass
from typing import Any


def _quantile(ordered: Sequence[float], q: float) -> float:
    """Linear interpolation between closest ranks."""

    if not ordered:
        raise ValueError("runtime benchmark samples must be non-empty")
    if not 0.0 <= q <= 1.0:
        raise ValueError("runtime benchmark quantile must be in [0, 1]")
    position = q * (len(ordered) - 1)
    low = math.floor(position)
    high = math.ceil(position)
    if low == high:
        return float(ordered[low])
    frac = position - low
    return float(ordered[low] + (ordered[high] - ordered[low]) * frac)


def _summary(ordered: Sequence[float]) -> dict[str, float]:
    return {
        "min": float(ordered[0]),
        "p10": _quantile(ordered, 0.10),
        "p50": _quantile(ordered, 0.50),
        "p90": _quantile(ordered, 0.90),
        "p99": _quantile(ordered, 0.99),
        "max": float(ordered[-1]),
        "mean": float(math.fsum(ordered) / len(ordered)),
    }


@dataclass(frozen=True, slots=True)
class BenchmarkDistribution:
    samples_seconds: tuple[float, ...]
    unit_name: str
    units_per_sample: int
    latency_seconds: dict[str, float]
    throughput_per_second: dict[str, float]

    def as_dict(self) -> dict[str, Any]:
        return {
            "samples_seconds": list(self.samples_seconds),
            "unit_name": self.unit_name,
            "units_per_sample": self.units_per_sample,
            "latency_seconds": dict(self.latency_seconds),
            "throughput_per_second": dict(self.throughput_per_second),
        }


def summarize_benchmark(
    samples_seconds: Sequence[float],
    *,
    unit_name: str,
    units_per_sample: int,
) -> BenchmarkDistribution:
    samples = tuple(float(s) for s in samples_seconds)
    if not samples or not all(math.isfinite(s) and s > 0 for s in samples):
        raise ValueError("runtime benchmark samples must be finite and positive")
    if not unit_name:
        raise ValueError("runtime benchmark unit name must be non-empty")
    if units_per_sample <= 0:
        raise ValueError("runtime benchmark units per sample must be positive")
    latency = _summary(sorted(samples))
    throughput = _summary(sorted(units_per_sample / s for s in samples))
    return BenchmarkDistribution(samples, unit_name, units_per_sample, latency, throughput)


def benchmark_wall(
    operation: Callable[[], object],
    *,
    warmups: int,
    repetitions: int,
    synchronize: Callable[[], object] | None = None,
    unit_name: str,
    units_per_sample: int,
) -> BenchmarkDistribution:
    """Wall-clock samples with synchronisation outside each timed region."""

    if warmups < 0 or repetitions <= 0:
        raise ValueError("runtime benchmark warmups must be non-negative and repetitions positive")
    sync = synchronize if synchronize is not None else (lambda: None)
    for _ in range(warmups):
        operation()
    sync()
    samples: list[float] = []
    for _ in range(repetitions):
        sync()
        begin = time.perf_counter()
        operation()
        sync()
        samples.append(time.perf_counter() - begin)
    return summarize_benchmark(samples, unit_name=unit_name, units_per_sample=units_per_sample)


def _region(values: Sequence[float], name: str) -> tuple[float, ...]:
    samples = tuple(float(v) for v in values)
    if not samples:
        raise ValueError(f"runtime profile region {name!r} has no samples")
    if not all(math.isfinite(v) and v >= 0 for v in samples):
        raise ValueError(f"runtime profile region {name!r} has invalid samples")
    return samples


def sum_aligned_profile_samples(
    regions: Mapping[str, Sequence[float]],
    names: Sequence[str],
) -> tuple[float, ...]:
    """Per-sample sum of non-overlapping regions with equal sample counts."""

    chosen = tuple(names)
    if not chosen or len(set(chosen)) != len(chosen):
        raise ValueError("runtime profile region names must be non-empty and unique")
    missing = [n for n in chosen if n not in regions]
    if missing:
        raise ValueError(f"runtime profile regions are missing: {missing}")
    columns = [_region(regions[n], n) for n in chosen]
    if len({len(c) for c in columns}) != 1:
        raise ValueError("runtime profile region sample counts differ")
    return tuple(math.fsum(row) for row in zip(*columns, strict=True))


def profile_ratio_samples(
    numerator: Sequence[float],
    denominator: Sequence[float],
) -> tuple[float, ...]:
    top = _region(numerator, "numerator")
    bottom = _region(denominator, "denominator")
    if len(top) != len(bottom):
        raise ValueError("runtime profile ratio sample counts differ")
    if any(v <= 0 for v in bottom):
        raise ValueError("runtime profile ratio denominators must be positive")
    return tuple(a / b for a, b in zip(top, bottom, strict=True))
