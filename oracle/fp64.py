"""FP64 NumPy oracle for split-K paged GQA decode (test infrastructure only).

Every function restates the semantics of reference ``src/paged_decode/oracle.py``
(cited per function) in float64 so FP32/FP16 accumulation errors of the device
path are visible.

Pinned by (``tests/test_oracle.py``):
* ``dense_attention`` -- brute force against an independent formulation
  (explicit per-token loop with ``math.exp`` and ``math.fsum``) on tiny inputs;
  closed forms: empty row -> zeros, ``q = 0`` -> mean of V over live tokens,
  one live token -> that token's V, page relabelling invariance, GQA equal to
  MHA over repeated KV heads, shared-prefix pages; the reference's own
  known-answer merge vector.
* ``partial_softmax`` / ``merge_partials`` -- the reference known-answer test
  (scores ``[-1e4, 1e4, 9999]``, values ``arange(12).reshape(3, 4)``), empty
  partition is the identity, all-empty gives zeros, and split invariance
  against ``dense_attention`` at 1e-11 (``tests/test_oracle.py`` mirrors
  reference ``tests/test_oracle.py:8-63``).
* ``gather_tokens`` -- addressing pinned by the relabelling and shared-page
  checks above and by a direct index check on a hand-built cache.
* ``scatter_tokens`` / ``append_advance`` -- the inverse of ``gather_tokens``:
  pinned by round trips (scatter then gather returns the written rows, rows
  not written are untouched) and by the skip rules on hand-built tables.
"""
import math

import numpy as np


def gather_tokens(cache, pages, length, kv_head):
    """Live tokens ``[length, D]`` of one sequence and KV head, as float64.

    Token ``t`` lives in physical page ``pages[t // T]`` at offset ``t % T``;
    entries of ``pages`` past the live prefix are never read (they may be -1).
    Reference ``oracle.py:50-56``.
    """
    page_size = cache.shape[1]
    if length == 0:
        return np.zeros((0, cache.shape[-1]), dtype=np.float64)
    positions = np.arange(length)
    physical = np.asarray(pages)[positions // page_size]
    return cache[physical, positions % page_size, kv_head].astype(np.float64)


def dense_attention(q, k, v, table, lengths):
    """One-token decode attention, computed densely in float64.

    ``out[b, h] = softmax(K_b q_bh / sqrt(D)) V_b`` over the live tokens of
    sequence ``b`` through KV head ``h // (Hq / Hkv)``; empty sequences give
    zeros. Reference ``oracle.py:59-71`` and ``docs/DESIGN.md:5-13``.
    """
    q = np.asarray(q)
    batch, heads, dim = q.shape
    kv_heads = k.shape[2]
    group = heads // kv_heads
    out = np.zeros((batch, heads, dim), dtype=np.float64)
    inv_sqrt_d = 1.0 / math.sqrt(dim)
    for b in range(batch):
        length = int(lengths[b])
        if length == 0:
            continue
        for kv_head in range(kv_heads):
            keys = gather_tokens(k, table[b], length, kv_head)
            values = gather_tokens(v, table[b], length, kv_head)
            heads_here = q[b, kv_head * group:(kv_head + 1) * group].astype(np.float64)
            scores = heads_here @ keys.T * inv_sqrt_d            # [group, length]
            weights = np.exp(scores - scores.max(axis=1, keepdims=True))
            out[b, kv_head * group:(kv_head + 1) * group] = (
                weights @ values) / weights.sum(axis=1, keepdims=True)
    return out


def partial_softmax(scores, values):
    """Online-softmax state ``(m, l, n)`` of one partition, token by token.

    ``m' = max(m, x); alpha = e^(m - m'); beta = e^(x - m'); l' = alpha l + beta;
    n' = alpha n + beta v``, starting from ``(-inf, 0, 0)``. Reference
    ``oracle.py:74-85`` and ``docs/DESIGN.md:31-42``.
    """
    values = np.asarray(values, dtype=np.float64)
    maximum, denominator = -np.inf, 0.0
    numerator = np.zeros(values.shape[-1], dtype=np.float64)
    for score, value in zip(np.asarray(scores, dtype=np.float64), values):
        new_maximum = max(maximum, score)
        alpha = math.exp(maximum - new_maximum) if maximum != -np.inf else 0.0
        beta = math.exp(score - new_maximum)
        numerator = numerator * alpha + beta * value
        denominator = denominator * alpha + beta
        maximum = new_maximum
    return maximum, denominator, numerator


def merge_partials(partials):
    """Max-corrected merge of ``(m, l, n)`` partition states.

    Partitions with ``l == 0`` are skipped (the empty partition is the
    identity); if all are empty the result is zeros. Otherwise
    ``M = max m_j, L = sum e^(m_j - M) l_j, N = sum e^(m_j - M) n_j`` and the
    result is ``N / L``. Reference ``oracle.py:88-96``, ``docs/DESIGN.md:48-61``.
    """
    active = [part for part in partials if part[1] > 0]
    if not active:
        return np.zeros_like(np.asarray(partials[0][2], dtype=np.float64))
    maximum = max(part[0] for part in active)
    denominator = 0.0
    numerator = np.zeros_like(np.asarray(active[0][2], dtype=np.float64))
    for m, l, n in active:
        weight = math.exp(m - maximum)
        denominator += weight * l
        numerator = numerator + weight * np.asarray(n, dtype=np.float64)
    return numerator / denominator


def streaming_attention(q, k, v, table, lengths, split_tokens=256, lanes=4):
    """Split-K decode through the partition algebra, in float64.

    Each sequence's context is cut into ``split_tokens`` partitions; each
    partition is further divided into ``lanes`` strided sub-partitions (the
    reference's four warps per CTA); every sub-partition goes through
    ``partial_softmax`` and all states meet in one ``merge_partials``.
    Reference ``oracle.py:99-117``.
    """
    if split_tokens <= 0:
        raise ValueError("split_tokens must be positive")
    q = np.asarray(q)
    batch, heads, dim = q.shape
    group = heads // k.shape[2]
    out = np.zeros((batch, heads, dim), dtype=np.float64)
    for b in range(batch):
        length = int(lengths[b])
        for h in range(heads):
            keys = gather_tokens(k, table[b], length, h // group)
            values = gather_tokens(v, table[b], length, h // group)
            scores = keys @ q[b, h].astype(np.float64) / math.sqrt(dim)
            states = []
            for start in range(0, max(length, 1), split_tokens):
                stop = min(start + split_tokens, length)
                for lane in range(lanes):
                    states.append(partial_softmax(scores[start + lane:stop:lanes],
                                                  values[start + lane:stop:lanes]))
            out[b, h] = merge_partials(states)
    return out


def scatter_tokens(cache, table, positions, new):
    """Cache after writing ``new[b, j]`` at logical position ``positions[b] + j``.

    Restates the decode's addressing (reference ``docs/DESIGN.md:10-13``) in the
    write direction: page ``table[b, pos // T]``, slot ``pos % T``. Positions
    outside ``[0, W * T)`` and page ids outside ``[0, P)`` are skipped. Works on
    a copy; exact (no arithmetic on values).
    """
    out = cache.copy()
    pages, page_size = cache.shape[0], cache.shape[1]
    table = np.asarray(table)
    capacity = table.shape[1] * page_size
    for b in range(new.shape[0]):
        for j in range(new.shape[1]):
            pos = int(positions[b]) + j
            if not 0 <= pos < capacity:
                continue
            page = int(table[b, pos // page_size])
            if not 0 <= page < pages:
                continue
            out[page, pos % page_size] = new[b, j]
    return out


def append_advance(cache, table, lengths, new, max_context=None):
    """All-or-nothing append at the current lengths; returns (cache, lengths).

    Sequence b is written only if every new position is below the context
    capacity -- the table's, or ``max_context`` when that is smaller (the
    context a plan's partitions cover) -- and lands on a valid page.
    """
    pages, page_size = cache.shape[0], cache.shape[1]
    table = np.asarray(table)
    capacity = table.shape[1] * page_size
    if max_context is not None:
        capacity = min(capacity, int(max_context))
    out, grown = cache.copy(), np.array(lengths, dtype=np.int64).copy()
    for b in range(new.shape[0]):
        base = int(lengths[b])
        rows = []
        for j in range(new.shape[1]):
            pos = base + j
            page = int(table[b, pos // page_size]) if 0 <= pos < capacity else -1
            rows.append(None if not 0 <= page < pages else (page, pos % page_size))
        if any(r is None for r in rows):
            continue
        for j, (page, slot) in enumerate(rows):
            out[page, slot] = new[b, j]
        grown[b] = base + new.shape[1]
    return out, grown.astype(np.int32)
