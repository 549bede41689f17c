"""Restatement of the reference's SDPA paged-attention path (CPU, torch).

Follows miniserve/attention.py step by step:
  write_kv      :111-133  position -> (table[b, pos // bs], pos % bs) scatter
  build_mask    :135-153  keep = key < len [& key <= q_pos] [& key > q_pos - window]
  gather        :155-171  padded gather to max_ctx, positions >= len read page 0
  forward       :205-250  gather -> cast to query dtype -> transpose ->
                          repeat_interleave(group) -> mask -> SDPA (scale 1/sqrt(D))
This is the algorithm the bench's cpu_baseline leg times (kind "port").
"""
from __future__ import annotations

from typing import Sequence

import torch
import torch.nn.functional as F


def build_mask(context_lens, q_len: int, window: int | None = None, causal: bool = True
               ) -> torch.Tensor:
    """Keep-mask [batch, q_len, max_ctx] (attention.py:135-153)."""
    lens = torch.as_tensor(context_lens).reshape(-1)
    max_ctx = int(lens.max()) if lens.numel() else 0
    key_pos = torch.arange(max_ctx)[None, None, :]
    q_pos = lens[:, None] - q_len + torch.arange(q_len)[None, :]
    mask = torch.ones(lens.numel(), q_len, max_ctx, dtype=torch.bool)
    if causal:
        mask &= key_pos <= q_pos[:, :, None]
    mask &= key_pos < lens[:, None, None]
    if window is not None:
        mask &= key_pos > (q_pos - window)[:, :, None]
    return mask


def gather(cache: torch.Tensor, block_table: torch.Tensor, lens: torch.Tensor, max_ctx: int
           ) -> torch.Tensor:
    """[batch, max_ctx, kv_heads, head_dim] rows (attention.py:155-171)."""
    bs = cache.shape[1]
    pos = torch.arange(max_ctx)
    blk = block_table[:, pos // bs]
    off = pos % bs
    valid = pos[None, :] < lens[:, None]
    blk = torch.where(valid, blk, torch.zeros_like(blk))
    if cache.dtype == torch.float8_e4m3fn:
        return cache.view(torch.uint8)[blk, off].view(cache.dtype)
    return cache[blk, off]


def write_kv(k_cache: torch.Tensor, v_cache: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
             block_table: torch.Tensor, start: int | Sequence[int] = 0) -> None:
    """cache[table[b, pos // bs], pos % bs] = k[b, t], pos = start_b + t (attention.py:111-133).

    Vectorised per row; negative page ids wrap like torch indexing does.
    """
    bs = k_cache.shape[1]
    B, T = k.shape[0], k.shape[1]
    starts = list(start) if isinstance(start, Sequence) else [start] * B
    for b in range(B):
        pos = torch.arange(T) + int(starts[b])
        phys = block_table[b, pos // bs].to(torch.long)
        k_cache[phys, pos % bs] = k[b].to(k_cache.dtype)
        v_cache[phys, pos % bs] = v[b].to(v_cache.dtype)


def paged_attention_sdpa(query: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                         block_table, context_lens, causal: bool = True,
                         window: int | None = None) -> torch.Tensor:
    """PagedAttention.forward with backend="sdpa" (attention.py:205-250), CPU tensors."""
    group = query.shape[2] // k_cache.shape[2]
    lens = torch.as_tensor(context_lens).reshape(-1)
    q_len = query.shape[1]
    max_ctx = int(lens.max())
    table = torch.as_tensor(block_table, dtype=torch.long)
    if table.ndim == 1:
        table = table[None, :]
    k = gather(k_cache, table, lens, max_ctx).to(query.dtype)
    v = gather(v_cache, table, lens, max_ctx).to(query.dtype)
    q = query.transpose(1, 2)
    k = k.transpose(1, 2)
    v = v.transpose(1, 2)
    if group > 1:
        k = k.repeat_interleave(group, dim=1)
        v = v.repeat_interleave(group, dim=1)
    mask = build_mask(lens, q_len, window, causal)[:, None]
    out = F.scaled_dot_product_attention(q, k, v, attn_mask=mask, is_causal=False)
    return out.transpose(1, 2)
