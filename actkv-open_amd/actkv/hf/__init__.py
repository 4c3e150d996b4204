"""Serving on the paged cache through Hugging Face transformers (see paged_session)."""
from .paged_session import PagedHFCache, PagedSession, paged_attention_forward, register

__all__ = ["PagedHFCache", "PagedSession", "paged_attention_forward", "register"]
