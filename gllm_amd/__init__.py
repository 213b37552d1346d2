"""gllm_amd — MI355X (gfx950) attention hot path for gLLM.

Drop-ins for the reference's attention op (``attention_op.reference_attention``),
call site (``attention.Attention`` / ``AttentionMetadata``) and paged pool
(``kv_cache.PagedKVCache``), backed by hand-written HIP kernels in
``libgllm_attn.so`` (``csrc/``, C ABI in ``include/gllm_attn.h``).
"""
from .attention import Attention, AttentionMetadata, plan_for
from .attention_op import flash_attention, reference_attention
from .kv_cache import PagedKVCache
from .paged import AttentionPlan, paged_attention, rope_kv_write, rope_rotate

__all__ = [
    "Attention", "AttentionMetadata", "AttentionPlan", "PagedKVCache", "flash_attention",
    "paged_attention", "plan_for", "reference_attention", "rope_kv_write", "rope_rotate",
]
