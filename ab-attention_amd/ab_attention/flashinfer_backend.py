"""Import path of the reference's ``ab_attention.flashinfer_backend.paged_attention``.

The prefill itself is the gfx950 kernel behind ``ab_attention.paged``; this
module only keeps the reference's import path working for callers.
"""
from .paged import paged_attention

__all__ = ["paged_attention"]
