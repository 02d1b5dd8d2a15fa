"""Timing summaries, restating reference ``src/paged_decode/metrics.py:6-27``."""
import math
import statistics


def percentile(values, quantile):
    """Percentile by linear interpolation between closest ranks.

    For ``n`` sorted samples the rank is ``quantile * (n - 1)``; a fractional
    rank blends its two neighbours (numpy's default 'linear' method).
    """
    samples = sorted(values)
    if len(samples) == 0:
        raise ValueError("percentile of an empty sample set")
    if quantile < 0 or quantile > 1:
        raise ValueError(f"quantile {quantile} lies outside [0, 1]")
    rank = quantile * (len(samples) - 1)
    below = int(math.floor(rank))
    frac = rank - below
    if frac == 0:
        return samples[below]
    return samples[below] * (1 - frac) + samples[below + 1] * frac


def summarize(device_ms, wall_ms, batch):
    """p50/p95/min of paired device and wall samples, plus decode rates.

    The keys are the reference report's schema. One decode call advances every
    sequence of the batch by one token, so the sequence-token rate is ``batch``
    times the call rate.
    """
    device, wall = list(device_ms), list(wall_ms)
    if not device or len(device) != len(wall):
        raise ValueError(f"need equally many device and wall samples, got {len(device)} and {len(wall)}")
    if any(x <= 0 for x in device + wall):
        raise ValueError("timing samples must be positive")
    p50 = statistics.median(device)
    calls_per_second = 1000.0 / p50
    return {
        "sample_count": len(device),
        "device_ms_p50": p50,
        "device_ms_p95": percentile(device, 0.95),
        "device_ms_min": min(device),
        "wall_ms_p50": statistics.median(wall),
        "decode_steps_per_second": calls_per_second,
        "sequence_tokens_per_second": batch * calls_per_second,
    }


def kv_bytes(lengths, kv_heads, head_dim, element_size):
    """Logical KV bytes one decode call must read.

    ``sum(lengths) * kv_heads * head_dim * 2 (K and V) * element_size``; pages
    shared between sequences are counted once per sequence that reads them.
    """
    return int(sum(int(x) for x in lengths)) * kv_heads * head_dim * 2 * element_size


def unique_token_bytes(table, lengths, page_size, kv_heads, head_dim, element_size):
    """KV bytes of the distinct physical token slots a call reads.

    A slot is ``(physical page, offset)``; a prefix page shared by several
    sequences is counted once, which is the HBM floor when caches dedupe reads.
    """
    import numpy as np

    slots = []
    for row, length in zip(np.asarray(table), np.asarray(lengths)):
        positions = np.arange(int(length), dtype=np.int64)
        if positions.size:
            slots.append(row[positions // page_size].astype(np.int64) * page_size + positions % page_size)
    count = int(np.unique(np.concatenate(slots)).size) if slots else 0
    return count * kv_heads * head_dim * 2 * element_size
