"""Split-K decode with log-sum-exp merge (CPU, fp32).

Restates kernels/paged_attn_triton.py:
  num_splits_for          :80-84   1 split up to 2048 tokens, then ceil(ctx/2048), at most 8
  gather_paged            :92-99   flat index table[p // bs] * bs + p % bs
  flash_decode_reference  :102-171 per-split (m_s, l_s, acc_s) with the running merge
                                   alpha = e^(m - m'), beta = e^(m_s - m'); out = acc / l;
                                   rows with L <= 0 give zeros; optional RoPE on q.
"""
from __future__ import annotations

import torch

MAX_SPLITS = 8
MIN_SPLIT_CTX = 2048


def num_splits_for(context_len: int) -> int:
    if context_len <= MIN_SPLIT_CTX:
        return 1
    return max(1, min(MAX_SPLITS, (context_len + MIN_SPLIT_CTX - 1) // MIN_SPLIT_CTX))


def _rotate_half(x: torch.Tensor) -> torch.Tensor:
    half = x.shape[-1] // 2
    return torch.cat((-x[..., half:], x[..., :half]), dim=-1)


def gather_paged(cache: torch.Tensor, table_row: torch.Tensor, length: int) -> torch.Tensor:
    bs = cache.shape[1]
    pos = torch.arange(length)
    idx = table_row[pos // bs].to(torch.long) * bs + pos % bs
    return cache.reshape(-1, cache.shape[2], cache.shape[3]).index_select(0, idx)


def split_partials(qf: torch.Tensor, k: torch.Tensor, v: torch.Tensor, scale: float, splits: int):
    """Per-split (m_s, l_s, acc_s) for one row: qf [H, D], k/v [L, H, D] (GQA-expanded)."""
    L = k.shape[0]
    per = (L + splits - 1) // splits
    parts = []
    for s in range(splits):
        lo, hi = s * per, min(L, (s + 1) * per)
        if hi <= lo:
            continue
        scores = torch.einsum("hd,nhd->hn", qf, k[lo:hi]) * scale
        m_s = scores.max(dim=-1).values
        p = torch.exp(scores - m_s[:, None])
        parts.append((m_s, p.sum(dim=-1), torch.einsum("hn,nhd->hd", p, v[lo:hi])))
    return parts


def lse_merge(parts):
    """Running merge of flash_decode_reference (:152-170): returns acc / l."""
    H, D = parts[0][2].shape
    best_m = torch.full((H,), float("-inf"))
    best_acc = torch.zeros(H, D)
    best_l = torch.zeros(H)
    for m_s, l_s, acc_s in parts:
        m = torch.maximum(best_m, m_s)
        alpha = torch.exp(best_m - m)
        beta = torch.exp(m_s - m)
        best_acc = best_acc * alpha[:, None] + acc_s * beta[:, None]
        best_l = best_l * alpha + l_s * beta
        best_m = m
    return best_acc / best_l[:, None]


def split_k_decode(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor, block_table,
                   context_lens, *, num_splits: int | None = None, scale: float | None = None,
                   cos: torch.Tensor | None = None, sin: torch.Tensor | None = None,
                   position: torch.Tensor | None = None) -> torch.Tensor:
    """[B, 1, H, D] -> [B, 1, H, D] in q.dtype, computed in fp32."""
    if q.shape[1] != 1:
        raise ValueError("flash decode expects q_len == 1")
    B, _, H, D = q.shape
    KVH = k_cache.shape[2]
    group = H // KVH
    lens = torch.as_tensor(context_lens).reshape(-1).to(torch.long)
    table = torch.as_tensor(block_table, dtype=torch.long)
    if table.ndim == 1:
        table = table[None, :]
    scale = scale if scale is not None else 1.0 / (D ** 0.5)
    qf = q.reshape(B, H, D).to(torch.float32)
    if cos is not None and sin is not None and position is not None:
        pos = torch.as_tensor(position).reshape(-1).to(torch.long)[:B]
        cs = cos.index_select(0, pos).to(torch.float32)
        sn = sin.index_select(0, pos).to(torch.float32)
        qf = qf * cs[:, None, :] + _rotate_half(qf) * sn[:, None, :]
    out = torch.zeros(B, 1, H, D, dtype=torch.float32)
    for b in range(B):
        L = int(lens[b])
        if L <= 0:
            continue
        k = gather_paged(k_cache, table[b], L).to(torch.float32).repeat_interleave(group, dim=1)
        v = gather_paged(v_cache, table[b], L).to(torch.float32).repeat_interleave(group, dim=1)
        splits = max(1, min(num_splits or num_splits_for(L), L))
        out[b, 0] = lse_merge(split_partials(qf[b], k, v, scale, splits))
    return out.to(q.dtype)
