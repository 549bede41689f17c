"""miniserve_amd -- MI355X-native paged attention for miniserve.

``PagedAttention`` keeps the interface of miniserve.attention.PagedAttention
and runs on hand-written gfx950 HIP kernels (libmsattn.so, C ABI in
include/msattn.h).
"""
from .attention import (PagedAttention, apply_rope, gather_kv, kernel_route, paged_attention,
                        paged_attention_append)

__all__ = ["PagedAttention", "apply_rope", "gather_kv", "kernel_route", "paged_attention",
           "paged_attention_append"]
