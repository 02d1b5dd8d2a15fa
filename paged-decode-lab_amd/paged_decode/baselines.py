"""Dense PyTorch baselines for comparison rows (not the product path).

Restates the reference's PyTorch baselines (``src/paged_decode/reference.py:7-46``)
so they can be timed beside the operator on the same GPU: gather the paged cache
into dense ``[B, Hkv, Lmax, D]`` tensors with a padding mask, repeat KV heads for
GQA, then either an explicit FP32 softmax ("eager") or
``torch.nn.functional.scaled_dot_product_attention``. Neither is a paged
operator; they are what a caller without one would run.
"""
import math

import torch
import torch.nn.functional as F


def gather_dense(k, v, table, lengths):
    """Dense K/V ``[B, Hkv, Lmax, D]`` (zero padded) and mask ``[B, 1, 1, Lmax]``.

    ``table`` and ``lengths`` are int tensors on the cache device. Slots past a
    sequence's length read physical page 0 slot 0 (a valid address) and are
    zeroed, so invalid page ids are never dereferenced.
    """
    page_size = k.shape[1]
    batch = lengths.shape[0]
    longest = max(1, int(lengths.max().item()))
    pos = torch.arange(longest, device=k.device)
    live = pos[None, :] < lengths[:, None].long()                           # [B, L]
    logical_page = torch.clamp(pos // page_size, max=table.shape[1] - 1)
    pages = torch.where(live, table[:, logical_page].long(), 0)             # [B, L]
    slots = torch.where(live, (pos % page_size)[None, :].expand(batch, -1), 0)
    dense_k = k[pages, slots] * live[..., None, None]                       # [B, L, Hkv, D]
    dense_v = v[pages, slots] * live[..., None, None]
    mask = live[:, None, None, :]
    return dense_k.permute(0, 2, 1, 3).contiguous(), dense_v.permute(0, 2, 1, 3).contiguous(), mask


def expand_gqa(q, dense_k, dense_v):
    repeats = q.shape[1] // dense_k.shape[1]
    return (dense_k.repeat_interleave(repeats, dim=1), dense_v.repeat_interleave(repeats, dim=1))


def eager_attention(q, dense_k, dense_v, mask):
    """FP32 softmax attention; an all-masked row gives zeros."""
    keys_t = dense_k.float().transpose(-1, -2).contiguous()
    logits = (q.float().unsqueeze(2) @ keys_t) / math.sqrt(q.shape[-1])
    logits = logits.masked_fill(~mask, -torch.inf)
    weights = torch.nan_to_num(torch.softmax(logits, dim=-1), nan=0.0)
    return (weights @ dense_v.float()).squeeze(2)


def sdpa_attention(q, dense_k, dense_v, mask):
    """``scaled_dot_product_attention`` over the dense tensors (output in q's dtype)."""
    return F.scaled_dot_product_attention(q.unsqueeze(2).contiguous(), dense_k, dense_v, attn_mask=mask,
                                          dropout_p=0.0).squeeze(2)


def dense_decode(q, k, v, table, lengths, kind="sdpa", k_scale=1.0, v_scale=1.0):
    """Gather + expand + attention in one call (what a timed baseline step does).

    FP8 caches are dequantized to q's dtype first (``k.to(q.dtype) * k_scale``),
    as a caller without a quantized-KV operator would.
    """
    if k.dtype in (torch.float8_e4m3fn, torch.float8_e5m2):
        k = k.to(q.dtype) * k_scale
        v = v.to(q.dtype) * v_scale
    dense_k, dense_v, mask = gather_dense(k, v, table, lengths)
    dense_k, dense_v = expand_gqa(q, dense_k, dense_v)
    return (sdpa_attention if kind == "sdpa" else eager_attention)(q, dense_k, dense_v, mask)
