"""Float64 closed-form paged attention (CPU) -- the numerical truth for tolerances.

out[b, i, h] = sum_k softmax_k(scale * q[b,i,h] . K[b,k,h//group]) V[b,k,h//group]
over the keys the reference's mask keeps (miniserve/attention.py:143-153):
k < len_b, k <= q_pos when causal, k > q_pos - window when windowed, with
q_pos = len_b - q_len + i. K/V rows come from the block table with the
closed-form page map phys = table[b, k // bs], slot = k % bs
(miniserve/attention.py:163-171; kernels/paged_attn_triton.py:92-99).
Rows that keep no key are defined as zeros. This is the einsum + masked
softmax pattern of tests/test_parity.py:99-117, evaluated per row without
padding and in float64.
"""
from __future__ import annotations

import math

import numpy as np
import torch


def gather_rows(cache: torch.Tensor, table_row, length: int,
                cast_to: torch.dtype | None = None) -> np.ndarray:
    """Float64 [length, kv_heads, head_dim] rows of one sequence (integer page map).

    ``cast_to``: the rows are first converted to that dtype, as the reference casts the
    gathered K/V to the query dtype before attending (miniserve/attention.py:240-241).
    """
    bs = cache.shape[1]
    pos = torch.arange(length)
    phys = torch.as_tensor(np.asarray(table_row, dtype=np.int64))[pos // bs]
    if cache.dtype == torch.float8_e4m3fn:  # index the bytes, then decode
        rows = cache.view(torch.uint8)[phys, pos % bs].view(torch.float8_e4m3fn)
    else:
        rows = cache[phys, pos % bs]
    if cast_to is not None:
        rows = rows.to(cast_to)
    return rows.double().numpy()


def keep_mask(length: int, q_len: int, causal: bool, window: int | None) -> np.ndarray:
    """Boolean [q_len, length]."""
    key = np.arange(length)[None, :]
    q_pos = length - q_len + np.arange(q_len)[:, None]
    keep = np.ones((q_len, length), dtype=bool)
    if causal:
        keep &= key <= q_pos
    if window is not None:
        keep &= key > q_pos - window
    return keep


def attend_f64(q: np.ndarray, k: np.ndarray, v: np.ndarray, keep: np.ndarray, scale: float
               ) -> np.ndarray:
    """q [q_len, H, D], k/v [L, KVH, D], keep [q_len, L] -> [q_len, H, D] float64."""
    q_len, H, D = q.shape
    KVH = k.shape[1]
    group = H // KVH
    out = np.zeros((q_len, H, D), dtype=np.float64)
    for kvh in range(KVH):
        qh = q[:, kvh * group:(kvh + 1) * group, :]               # [q_len, g, D]
        s = np.einsum("igd,kd->igk", qh, k[:, kvh, :]) * scale    # [q_len, g, L]
        s = np.where(keep[:, None, :], s, -np.inf)
        m = s.max(axis=-1, keepdims=True)
        m = np.where(np.isfinite(m), m, 0.0)
        p = np.exp(s - m)
        p = np.where(keep[:, None, :], p, 0.0)
        denom = p.sum(axis=-1, keepdims=True)
        o = np.einsum("igk,kd->igd", p, v[:, kvh, :])
        out[:, kvh * group:(kvh + 1) * group, :] = np.where(denom > 0, o / np.where(denom > 0, denom, 1.0), 0.0)
    return out


def paged_attention_f64(query: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                        block_table, context_lens, causal: bool = True,
                        window: int | None = None, scale: float | None = None,
                        rows: list[int] | None = None, kv_cast: bool = False) -> np.ndarray:
    """Float64 [batch, q_len, H, D] (only `rows` filled when given, others zero).

    ``kv_cast``: K/V rows are converted to the query dtype before the float64 math, the
    reference's ``.to(query.dtype)`` of the gathered rows (attention.py:240-241); it
    matters when the cache type is wider than the query's or differs from it.
    """
    B, q_len, H, D = query.shape
    scale = 1.0 / math.sqrt(D) if scale is None else scale
    table = torch.as_tensor(block_table)
    if table.ndim == 1:
        table = table[None, :]
    table = table.numpy()
    lens = [int(x) for x in torch.as_tensor(context_lens).reshape(-1)]
    qf = query.float().numpy().astype(np.float64)
    out = np.zeros((B, q_len, H, D), dtype=np.float64)
    for b in (range(B) if rows is None else rows):
        L = lens[b]
        if L <= 0:
            continue
        cast = query.dtype if kv_cast else None
        k = gather_rows(k_cache, table[b], L, cast)
        v = gather_rows(v_cache, table[b], L, cast)
        out[b] = attend_f64(qf[b], k, v, keep_mask(L, q_len, causal, window), scale)
    return out
