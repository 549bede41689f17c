"""miniserve_amd.attention -- PagedAttention over hand-written HIP kernels.

Drop-in for ``miniserve.attention`` (miniserve/attention.py:65-250): the same
constructor, ``allocate_kv_cache``, ``write_kv``, ``build_mask`` and
``forward`` signature, the same cache layout ``[num_blocks, block_size,
num_kv_heads, head_dim]``, the same GQA head map (query head h reads KV head
h // group) and the same mask rules. ``forward`` and ``write_kv`` run on the
GPU through libmsattn.so (include/msattn.h); there is no CPU or PyTorch
fallback -- CPU tensors raise.

Differences from the reference, all deliberate:
  * ``forward`` takes an optional keyword ``scale`` (default 1/sqrt(head_dim),
    the value the reference's SDPA call uses, attention.py:249).
  * Rows with no visible key (context length 0) return zeros instead of the
    NaN an all-False SDPA mask row produces.
  * Block-table entries outside [0, num_blocks) are holes: never read or
    written (the reference wraps -1 to the last page, attention.py:131, 171).
  * The result is a contiguous [batch, q_len, heads, head_dim] tensor (the
    reference returns a transposed view; its caller reshapes it either way).
"""
from __future__ import annotations

import math
import threading
import weakref
from typing import Sequence

import torch

from . import _native as nat

_BACKENDS = ("sdpa", "triton_flash")

# Per-call host work of the eager path (the reference runner calls forward once per layer
# with an int64 device table and a Python-list context_lens, model_runner.py:72-83) is kept
# off the common case: the int32 table of a source tensor is converted once while the
# tensor is unchanged, list lengths go through pinned memory, and a call without a
# workspace reuses one zeroed workspace per (device, stream).
_cache_lock = threading.Lock()
_table_cache: dict[tuple, tuple] = {}   # (id, device) -> (weakref, version, meta, int32 table)
_TABLE_CACHE_MAX = 16
_workspaces: dict[tuple, torch.Tensor] = {}  # (device index, stream handle) -> uint8 tensor


def _rotate_half(x: torch.Tensor) -> torch.Tensor:
    half = x.shape[-1] // 2
    return torch.cat((-x[..., half:], x[..., :half]), dim=-1)


def apply_rope(q: torch.Tensor, k: torch.Tensor | None, cos: torch.Tensor, sin: torch.Tensor,
               position_ids: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor | None]:
    """Rotate-half RoPE, signature of miniserve/attention.py:41-62.

    ``q`` [batch, heads, seq, dim], ``k`` [batch, kv_heads, seq, dim] or None,
    ``cos``/``sin`` [max_pos, dim], ``position_ids`` [seq] or [batch, seq].
    """
    cos = cos[position_ids].to(q.dtype)
    sin = sin[position_ids].to(q.dtype)
    if cos.ndim == 2:
        cos, sin = cos.unsqueeze(0), sin.unsqueeze(0)
    cos, sin = cos.unsqueeze(1), sin.unsqueeze(1)
    q_rot = q * cos + _rotate_half(q) * sin
    k_rot = None if k is None else k * cos + _rotate_half(k) * sin
    return q_rot, k_rot


def _require_gpu(t: torch.Tensor, what: str) -> None:
    if t.device.type != "cuda":
        raise RuntimeError(
            f"msattn needs ROCm GPU tensors: {what} is on {t.device} (there is no CPU path)")


def _convert_table(table: torch.Tensor) -> torch.Tensor:
    if table.ndim == 1:
        table = table[None, :]
    if table.ndim != 2:
        raise ValueError("block_table must be 1-D or 2-D")
    if table.dtype != torch.int32:
        table = table.to(torch.int32)
    return table.contiguous()


def block_table_i32(block_table, device: torch.device) -> torch.Tensor:
    """Block table as a contiguous int32 [batch, width] tensor on `device`.

    A device tensor that needs converting (the reference keeps int64 tables,
    attention.py:237) is converted once and reused while it is unchanged: same object,
    same torch version counter (every in-place write through torch bumps it), same shape
    and strides. Not during graph capture, whose conversions must be captured."""
    if not isinstance(block_table, torch.Tensor) or block_table.device != device or \
            (block_table.dtype == torch.int32 and block_table.is_contiguous() and
             block_table.ndim == 2) or torch.cuda.is_current_stream_capturing():
        return _convert_table(torch.as_tensor(block_table, device=device))
    try:
        version = block_table._version
    except RuntimeError:  # inference-mode tensors keep no version counter: no reuse
        return _convert_table(block_table)
    key = (id(block_table), str(device))
    meta = (block_table.data_ptr(), tuple(block_table.shape), block_table.stride(),
            block_table.dtype)
    with _cache_lock:
        hit = _table_cache.get(key)
        if hit is not None and hit[0]() is block_table and hit[1] == version and hit[2] == meta:
            return hit[3]
    table = _convert_table(block_table)
    with _cache_lock:
        if len(_table_cache) >= _TABLE_CACHE_MAX:
            _table_cache.clear()
        _table_cache[key] = (weakref.ref(block_table), version, meta, table)
    return table


def _host_ints_to_device(values: list[int], device: torch.device) -> torch.Tensor:
    """int32 device copy of host integers through pinned memory (an asynchronous copy;
    torch's pinned-memory allocator keeps the staging block until the copy has run)."""
    if device.type != "cuda":
        return torch.tensor(values, dtype=torch.int32, device=device)
    staged = torch.tensor(values, dtype=torch.int32, pin_memory=True)
    return staged.to(device, non_blocking=True)


def context_lens_i32(context_lens, device: torch.device, batch: int) -> tuple[torch.Tensor, int | None]:
    """(int32 [batch] device tensor, host-known max or None) for context_lens."""
    if isinstance(context_lens, torch.Tensor):
        lens = context_lens.reshape(-1)
        host_max = int(lens.max()) if (lens.device.type == "cpu" and lens.numel()) else None
        lens = lens.to(device=device, dtype=torch.int32).contiguous()
    else:
        values = [int(x) for x in context_lens]
        host_max = max(values) if values else 0
        lens = _host_ints_to_device(values, device)
    if lens.numel() != batch:
        raise ValueError(f"context_lens has {lens.numel()} entries for a batch of {batch}")
    return lens, host_max


def _workspace(device: torch.device, nbytes: int) -> torch.Tensor:
    """A zeroed workspace of at least `nbytes` for calls on the current stream of `device`.

    One per (device, stream): calls on one stream run one after another, and every call
    leaves the in-kernel merge's counters at zero, so the next call may reuse it. Under
    graph capture a fresh one is allocated (from the graph's pool)."""
    if torch.cuda.is_current_stream_capturing():
        return torch.zeros(nbytes, dtype=torch.uint8, device=device)
    key = (device.index if device.index is not None else torch.cuda.current_device(),
           nat.stream_handle(device))
    with _cache_lock:
        ws = _workspaces.get(key)
        if ws is None or ws.numel() < nbytes:
            if ws is None and len(_workspaces) >= 16:  # streams come and go: keep a few
                _workspaces.clear()
            ws = torch.zeros(max(nbytes, 1 << 20), dtype=torch.uint8, device=device)
            _workspaces[key] = ws
    return ws


class PagedAttention:
    """Paged attention over a block-table-mapped KV cache (HIP kernels)."""

    def __init__(
        self,
        num_heads: int,
        num_kv_heads: int | None = None,
        head_dim: int | None = None,
        *,
        num_blocks: int,
        block_size: int,
        dtype: torch.dtype = torch.float16,
        device: torch.device | str = "cpu",
        window: int | None = None,
        kv_dtype: torch.dtype = torch.float16,
    ) -> None:
        # Argument contract of miniserve/attention.py:81-92.
        if num_heads <= 0:
            raise ValueError("num_heads must be positive")
        if num_kv_heads is None:
            num_kv_heads = num_heads
        if num_kv_heads <= 0 or num_heads % num_kv_heads:
            raise ValueError("num_heads must be a multiple of num_kv_heads")
        if head_dim is None or head_dim <= 0 or head_dim % 2:
            raise ValueError("head_dim must be a positive even integer")
        if num_blocks <= 0 or block_size <= 0:
            raise ValueError("num_blocks and block_size must be positive")
        if window is not None and window <= 0:
            raise ValueError("window must be positive")
        self.num_heads = num_heads
        self.num_kv_heads = num_kv_heads
        self.head_dim = head_dim
        self.num_blocks = num_blocks
        self.block_size = block_size
        self.dtype = dtype
        self.device = torch.device(device)
        self.window = window
        self.kv_dtype = kv_dtype
        self.group = num_heads // num_kv_heads

    def allocate_kv_cache(self) -> tuple[torch.Tensor, torch.Tensor]:
        """(k_cache, v_cache), each zeros [num_blocks, block_size, kv_heads, head_dim]."""
        shape = (self.num_blocks, self.block_size, self.num_kv_heads, self.head_dim)
        k = torch.zeros(shape, dtype=self.kv_dtype, device=self.device)
        v = torch.zeros(shape, dtype=self.kv_dtype, device=self.device)
        return k, v

    def write_kv(
        self,
        k_cache: torch.Tensor,
        v_cache: torch.Tensor,
        k: torch.Tensor,
        v: torch.Tensor,
        block_table: torch.Tensor,
        start: int | Sequence[int] | torch.Tensor = 0,
    ) -> None:
        """Scatter k/v [batch, tokens, kv_heads, head_dim] into the cache.

        Row b's token t lands at position start[b] + t (``start`` is an int,
        one entry per row, or an int tensor already on the device).
        """
        for t, name in ((k_cache, "k_cache"), (v_cache, "v_cache"), (k, "k"), (v, "v")):
            _require_gpu(t, name)
        if k.shape != v.shape or k.ndim != 4:
            raise ValueError("k and v must both be [batch, tokens, kv_heads, head_dim]")
        if k.dtype != v.dtype:
            raise ValueError("k and v must share a dtype")
        if k_cache.shape != v_cache.shape or k_cache.dtype != v_cache.dtype or \
                k_cache.stride() != v_cache.stride():
            raise ValueError("k_cache and v_cache must share shape, dtype and strides")
        B, T, KVH, D = k.shape
        if k_cache.shape[2] != KVH or k_cache.shape[3] != D:
            raise ValueError("k/v heads or head_dim do not match the cache")
        if k_cache.stride(3) != 1:
            raise ValueError("cache head_dim must be contiguous")
        dev = k_cache.device
        table = block_table_i32(block_table, dev)
        if table.shape[0] < B:
            raise ValueError("block_table has fewer rows than k")
        if isinstance(start, torch.Tensor):
            starts = start.reshape(-1).to(device=dev, dtype=torch.int32)
        elif isinstance(start, Sequence):
            starts = _host_ints_to_device([int(s) for s in start], dev)
        else:
            starts = torch.full((B,), int(start), dtype=torch.int32, device=dev)
        if starts.numel() < B:
            raise ValueError("start needs one entry per batch row")
        starts = starts.contiguous()
        kc = k.contiguous()
        vc = v.contiguous()
        status = nat.lib().msattn_write_kv(
            k_cache.data_ptr(), v_cache.data_ptr(), k_cache.stride(0), k_cache.stride(1),
            k_cache.stride(2), kc.data_ptr(), vc.data_ptr(), table.data_ptr(), starts.data_ptr(),
            B, T, KVH, D, k_cache.shape[1], k_cache.shape[0], table.shape[1],
            nat.dtype_code(k.dtype), nat.dtype_code(k_cache.dtype), nat.stream_handle(dev))
        nat.check("msattn_write_kv", status)

    def build_mask(
        self,
        context_lens: torch.Tensor | Sequence[int],
        q_len: int,
        window: int | None = None,
        causal: bool = True,
    ) -> torch.Tensor:
        """Boolean keep-mask [batch, q_len, max_ctx] (True = attend).

        The rules of miniserve/attention.py:135-153, which the kernels apply as
        per-key predicates: q_pos = len - q_len + i; keep key if key < len,
        key <= q_pos when causal, key > q_pos - window when windowed.
        """
        lens = torch.as_tensor(context_lens, device=self.device).reshape(-1)
        max_ctx = int(lens.max()) if lens.numel() else 0
        key = torch.arange(max_ctx, device=self.device).view(1, 1, -1)
        q_pos = (lens.view(-1, 1) - q_len + torch.arange(q_len, device=self.device).view(1, -1))
        keep = key < lens.view(-1, 1, 1)
        if causal:
            keep = keep & (key <= q_pos.unsqueeze(-1))
        if window is not None:
            keep = keep & (key > (q_pos - window).unsqueeze(-1))
        return keep.expand(lens.numel(), q_len, max_ctx).contiguous()

    def forward(
        self,
        query: torch.Tensor,
        k_cache: torch.Tensor,
        v_cache: torch.Tensor,
        block_table: torch.Tensor,
        context_lens: torch.Tensor | Sequence[int],
        causal: bool = True,
        window: int | None = None,
        *,
        backend: str = "sdpa",
        cos: torch.Tensor | None = None,
        sin: torch.Tensor | None = None,
        position: torch.Tensor | None = None,
        scale: float | None = None,
        shared_prefix_pages: int | None = None,
    ) -> torch.Tensor:
        """Paged attention; ``window`` overrides the constructor value.

        ``backend`` is kept for signature compatibility. Both accepted names run
        the same HIP kernels; "triton_flash" keeps the reference's decode-only
        contract (attention.py:187-194) and its optional RoPE on the query
        (cos/sin/position, kernels/paged_attn_triton.py:135-139).
        ``shared_prefix_pages``: the leading block-table entries every row shares (a
        radix-cache hit, prefix_cache.py:66-96); a decode reads them once per KV head.
        """
        if backend not in _BACKENDS:
            raise ValueError(f"unknown attention backend: {backend!r}")
        if backend == "triton_flash":
            if not causal:
                raise ValueError("triton_flash supports causal decode only")
            if (self.window if window is None else window) is not None:
                raise ValueError("triton_flash does not support a sliding window")
            if query.shape[1] != 1:
                raise ValueError("triton_flash is decode-only (q_len == 1)")
            if k_cache.dtype == torch.float8_e4m3fn or v_cache.dtype == torch.float8_e4m3fn:
                raise ValueError("triton_flash does not support an FP8 KV cache")
            if query.device.type != "cuda":
                raise RuntimeError("triton_flash requires CUDA tensors (a ROCm GPU device)")
            rope = (cos, sin, position) if cos is not None and sin is not None and \
                position is not None else None
            return paged_attention(query, k_cache, v_cache, block_table, context_lens,
                                   causal=True, window=None, scale=scale, rope=rope,
                                   prefix_pages=shared_prefix_pages if rope is None else None)
        window = self.window if window is None else window
        cascade = shared_prefix_pages if (query.shape[1] == 1 and causal and window is None) \
            else None
        return paged_attention(query, k_cache, v_cache, block_table, context_lens,
                               causal=causal, window=window, scale=scale, prefix_pages=cascade)

    __call__ = forward


def paged_attention(query: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                    block_table, context_lens, *, causal: bool = True, window: int | None = None,
                    scale: float | None = None, max_context: int | None = None,
                    workspace: torch.Tensor | None = None, out: torch.Tensor | None = None,
                    rope: tuple | None = None, prefix_pages: int | None = None) -> torch.Tensor:
    """Functional form of PagedAttention.forward on the HIP kernels.

    ``max_context`` bounds context_lens; when context_lens is a device tensor
    and it is None, the table capacity (width * block_size) is used so that no
    device->host read happens (the call is then safe to capture in a graph).
    ``workspace``/``out`` let a caller pass preallocated buffers; a workspace must be
    zero when first used (``torch.zeros``), and every call leaves it reusable.
    ``rope`` = (cos, sin, position) applies rotate-half RoPE to a decode query inside
    the attention kernels (cos/sin [max_pos, head_dim], position [batch] or a scalar;
    kernels/paged_attn_triton.py:211-220).
    ``prefix_pages`` > 0 declares that the first prefix_pages entries of every block-table
    row are the same physical pages (a shared prefix): a causal decode then reads them
    once per KV head for the whole batch (cascade decode).
    """
    _require_gpu(query, "query")
    _require_gpu(k_cache, "k_cache")
    _require_gpu(v_cache, "v_cache")
    if query.ndim != 4 or k_cache.ndim != 4:
        raise ValueError("query must be [batch, q_len, heads, head_dim] and the caches "
                         "[num_blocks, block_size, kv_heads, head_dim]")
    if k_cache.shape != v_cache.shape or k_cache.dtype != v_cache.dtype or \
            k_cache.stride() != v_cache.stride():
        raise ValueError("k_cache and v_cache must share shape, dtype and strides")
    B, q_len, H, D = query.shape
    nb, bs, KVH, Dk = k_cache.shape
    if Dk != D:
        raise ValueError(f"head_dim mismatch: query {D}, cache {Dk}")
    if D > nat.MAX_HEAD_DIM or D % 2:
        raise ValueError(f"head_dim {D}: the kernels take even head sizes up to "
                         f"{nat.MAX_HEAD_DIM}")
    if H % KVH:
        raise ValueError("num_heads must be a multiple of num_kv_heads")
    if k_cache.stride(3) != 1:
        raise ValueError("cache head_dim must be contiguous")
    if window is not None and window <= 0:
        raise ValueError("window must be positive")
    dev = query.device
    q = query.contiguous()
    table = block_table_i32(block_table, dev)
    if table.shape[0] != B:
        raise ValueError(f"block_table has {table.shape[0]} rows for a batch of {B}")
    lens, host_max = context_lens_i32(context_lens, dev, B)
    W = table.shape[1]
    cap = W * bs
    if max_context is None:
        max_context = cap if host_max is None else host_max
    if host_max is not None and host_max > cap:
        raise ValueError(f"context length {host_max} exceeds the block table capacity {cap}")
    max_context = max(0, min(int(max_context), cap))
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    qcode = nat.dtype_code(query.dtype)
    kvcode = nat.dtype_code(k_cache.dtype)
    L = nat.lib()
    if prefix_pages:
        if q_len != 1 or not causal or window is not None or rope is not None:
            raise ValueError("prefix_pages applies to causal decode (q_len == 1) without "
                             "a window or RoPE")
        if not 0 <= int(prefix_pages) <= W:
            raise ValueError(f"prefix_pages {prefix_pages} outside [0, {W}]")
        ws_bytes = L.msattn_prefix_workspace_bytes(B, H, KVH, D, bs, max_context,
                                                   int(prefix_pages))
    else:
        ws_bytes = L.msattn_workspace_bytes(B, q_len, H, KVH, D, max_context)
    if ws_bytes == 0:
        raise ValueError("unsupported attention geometry")
    if workspace is None or workspace.numel() * workspace.element_size() < ws_bytes:
        # zeroed: the in-kernel merge's tickets must start at zero (calls leave them so)
        workspace = _workspace(dev, ws_bytes)
    if out is None:
        out = torch.empty((B, q_len, H, D), dtype=query.dtype, device=dev)
    args = (q.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), k_cache.stride(0),
            k_cache.stride(1), k_cache.stride(2), table.data_ptr(), lens.data_ptr(),
            out.data_ptr(), workspace.data_ptr(), ws_bytes, B, q_len, H, KVH, D, bs, nb, W,
            max_context, 1 if causal else 0, int(window or 0), float(scale), qcode, kvcode)
    if prefix_pages:
        status = L.msattn_paged_attention_prefix(
            q.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), k_cache.stride(0),
            k_cache.stride(1), k_cache.stride(2), table.data_ptr(), lens.data_ptr(),
            out.data_ptr(), workspace.data_ptr(), ws_bytes, B, H, KVH, D, bs, nb, W,
            max_context, int(prefix_pages), float(scale), qcode, kvcode, nat.stream_handle(dev))
        nat.check("msattn_paged_attention_prefix", status)
        return out
    if rope is None:
        status = L.msattn_paged_attention(*args, nat.stream_handle(dev))
        nat.check("msattn_paged_attention", status)
        return out
    if q_len != 1:
        raise ValueError("RoPE inside the kernel is decode-only (q_len == 1)")
    cos, sin, position = rope
    cos = torch.as_tensor(cos, device=dev).to(torch.float32).contiguous()
    sin = torch.as_tensor(sin, device=dev).to(torch.float32).contiguous()
    if cos.ndim != 2 or cos.shape != sin.shape or cos.shape[1] != D:
        raise ValueError(f"cos/sin must be [max_pos, {D}] and of one shape")
    pos = torch.as_tensor(position, device=dev).reshape(-1).to(torch.int32)
    if pos.numel() == 1 and B > 1:
        pos = pos.expand(B)
    pos = pos[:B].contiguous()
    if pos.numel() != B:
        raise ValueError(f"position has {pos.numel()} entries for a batch of {B}")
    status = L.msattn_paged_attention_rope(*args, cos.data_ptr(), sin.data_ptr(), pos.data_ptr(),
                                           cos.shape[0], nat.stream_handle(dev))
    nat.check("msattn_paged_attention_rope", status)
    return out


def paged_attention_append(query: torch.Tensor, k_new: torch.Tensor, v_new: torch.Tensor,
                           k_cache: torch.Tensor, v_cache: torch.Tensor, block_table,
                           context_lens, *, window: int | None = None,
                           scale: float | None = None, max_context: int | None = None,
                           workspace: torch.Tensor | None = None,
                           out: torch.Tensor | None = None) -> torch.Tensor:
    """One decode step with the new token appended: ``write_kv`` of k_new / v_new
    ([batch, 1, kv_heads, head_dim], the query's dtype) at position context_lens[b] - 1
    of each row, then the causal decode over ``context_lens`` (which count the new
    token), as msattn_paged_attention_append. Rows with context_lens[b] <= 0 write
    nothing. On the partition kernel (small decodes, bf16/fp16 query, at most 8 query rows
    per KV head) both happen in one launch; the caches and the output equal those of
    ``write_kv`` followed by ``paged_attention`` bit for bit.
    """
    _require_gpu(query, "query")
    _require_gpu(k_cache, "k_cache")
    _require_gpu(v_cache, "v_cache")
    if query.ndim != 4 or query.shape[1] != 1:
        raise ValueError("query must be [batch, 1, heads, head_dim] (decode)")
    if k_cache.ndim != 4 or k_cache.shape != v_cache.shape or k_cache.dtype != v_cache.dtype \
            or k_cache.stride() != v_cache.stride():
        raise ValueError("k_cache and v_cache must share a [num_blocks, block_size, kv_heads, "
                         "head_dim] shape, dtype and strides")
    B, _, H, D = query.shape
    nb, bs, KVH, Dk = k_cache.shape
    if Dk != D or H % KVH:
        raise ValueError("head_dim and kv_heads must match the query")
    if D > nat.MAX_HEAD_DIM or D % 2:
        raise ValueError(f"head_dim {D}: the kernels take even head sizes up to "
                         f"{nat.MAX_HEAD_DIM}")
    if k_cache.stride(3) != 1:
        raise ValueError("cache head_dim must be contiguous")
    for name, t in (("k_new", k_new), ("v_new", v_new)):
        if tuple(t.shape) != (B, 1, KVH, D) or t.dtype != query.dtype:
            raise ValueError(f"{name} must be [{B}, 1, {KVH}, {D}] in the query dtype")
    if window is not None and window <= 0:
        raise ValueError("window must be positive")
    dev = query.device
    q = query.contiguous()
    kn = k_new.contiguous()
    vn = v_new.contiguous()
    table = block_table_i32(block_table, dev)
    if table.shape[0] != B:
        raise ValueError(f"block_table has {table.shape[0]} rows for a batch of {B}")
    lens, host_max = context_lens_i32(context_lens, dev, B)
    W = table.shape[1]
    cap = W * bs
    if max_context is None:
        max_context = cap if host_max is None else host_max
    if host_max is not None and host_max > cap:
        raise ValueError(f"context length {host_max} exceeds the block table capacity {cap}")
    max_context = max(0, min(int(max_context), cap))
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    L = nat.lib()
    ws_bytes = L.msattn_workspace_bytes(B, 1, H, KVH, D, max_context)
    if ws_bytes == 0:
        raise ValueError("unsupported attention geometry")
    if workspace is None or workspace.numel() * workspace.element_size() < ws_bytes:
        workspace = _workspace(dev, ws_bytes)
    if out is None:
        out = torch.empty((B, 1, H, D), dtype=query.dtype, device=dev)
    status = L.msattn_paged_attention_append(
        q.data_ptr(), kn.data_ptr(), vn.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(),
        k_cache.stride(0), k_cache.stride(1), k_cache.stride(2), table.data_ptr(),
        lens.data_ptr(), out.data_ptr(), workspace.data_ptr(), ws_bytes, B, H, KVH, D, bs, nb,
        W, max_context, int(window or 0), float(scale), nat.dtype_code(query.dtype),
        nat.dtype_code(k_cache.dtype), nat.stream_handle(dev))
    nat.check("msattn_paged_attention_append", status)
    return out


def kernel_route(query: torch.Tensor, k_cache: torch.Tensor, block_table,
                 max_context: int | None = None, out: torch.Tensor | None = None,
                 workspace_bytes: int | None = None) -> str:
    """Name of the kernel ``paged_attention`` runs for this call: "prefill", "prefill
    stream-K" (the prefill kernel's stream-K schedule), "partition-fused", "partition",
    "stream-K" (the stream-K decode kernel) or "generic" (msattn_paged_attention_route).

    The choice depends on shapes, types and alignment, not on context-length values;
    ``max_context`` defaults to the table capacity, ``workspace_bytes`` to the call's own
    workspace size (pass ``_native.NOALLOC_SCRATCH_BYTES`` for the no-allocation entry)."""
    import ctypes

    B, q_len, H, D = query.shape
    nb, bs, KVH, _ = k_cache.shape
    width = block_table.shape[-1]
    cap = width * bs
    max_context = cap if max_context is None else max(0, min(int(max_context), cap))
    lib = nat.lib()
    if workspace_bytes is None:
        workspace_bytes = lib.msattn_workspace_bytes(B, q_len, H, KVH, D, max_context)
    q = query if query.is_contiguous() else query.contiguous()
    out_ptr = out.data_ptr() if out is not None else q.data_ptr()
    r = ctypes.c_int(0)
    nat.check("msattn_paged_attention_route", lib.msattn_paged_attention_route(
        q.data_ptr(), out_ptr, k_cache.data_ptr(), k_cache.data_ptr(), k_cache.stride(0),
        k_cache.stride(1), k_cache.stride(2), B, q_len, H, KVH, D, bs, max_context,
        nat.dtype_code(query.dtype), nat.dtype_code(k_cache.dtype), workspace_bytes,
        ctypes.byref(r)))
    return nat.ROUTE_NAMES[r.value]


def gather_kv(cache: torch.Tensor, block_table, context_lens, max_context: int | None = None
              ) -> torch.Tensor:
    """[batch, max_ctx, kv_heads, head_dim] rows gathered through the block table.

    The addressing of PagedAttention._gather (miniserve/attention.py:155-171),
    done by the library's gather kernel: positions at or past a row's context
    length read page 0; holes give zero rows.
    """
    _require_gpu(cache, "cache")
    dev = cache.device
    table = block_table_i32(block_table, dev)
    B = table.shape[0]
    lens, host_max = context_lens_i32(context_lens, dev, B)
    if max_context is None:
        max_context = host_max if host_max is not None else table.shape[1] * cache.shape[1]
    nb, bs, KVH, D = cache.shape
    out = torch.empty((B, max_context, KVH, D), dtype=cache.dtype, device=dev)
    status = nat.lib().msattn_gather_kv(
        cache.data_ptr(), cache.stride(0), cache.stride(1), cache.stride(2), table.data_ptr(),
        lens.data_ptr(), out.data_ptr(), B, max_context, KVH, D, bs, nb, table.shape[1],
        nat.dtype_code(cache.dtype), nat.stream_handle(dev))
    nat.check("msattn_gather_kv", status)
    return out
