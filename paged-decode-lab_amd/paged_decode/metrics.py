"""Timing summaries, restating reference ``src/paged_decode/metrics.py:6-27``."""
import math
import statistics


def percentile(values, quantile):
    """Linearly interpolated percentile (the 'linear' method of numpy)."""
    if not values or not 0 <= quantile <= 1:
        raise ValueError("nonempty values and quantile in [0,1] required")
    ordered = sorted(values)
    position = (len(ordered) - 1) * quantile
    lower = math.floor(position)
    upper = math.ceil(position)
    return ordered[lower] + (ordered[upper] - ordered[lower]) * (position - lower)


def summarize(device_ms, wall_ms, batch):
    """p50/p95/min of paired device and wall samples, plus decode rates.

    One decode call advances every sequence of the batch by one token, so the
    sequence-token rate is ``batch`` times the call rate.
    """
    if len(device_ms) != len(wall_ms) or not device_ms or min(list(device_ms) + list(wall_ms)) <= 0:
        raise ValueError("paired positive timing samples required")
    median = statistics.median(device_ms)
    return {
        "sample_count": len(device_ms),
        "device_ms_p50": median,
        "device_ms_p95": percentile(list(device_ms), 0.95),
        "device_ms_min": min(device_ms),
        "wall_ms_p50": statistics.median(wall_ms),
        "decode_steps_per_second": 1000.0 / median,
        "sequence_tokens_per_second": batch * 1000.0 / median,
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
