"""metalllm_amd: MI355X (gfx950) attention hot path of metalLLM.

The product is libmetalllm_attn.so (C ABI in include/metalllm_attn.h); this package builds it
(`metalllm_amd.build`) and binds it (`metalllm_amd.attention`).
"""
from .attention import (AttentionError, AttentionParams, attention_backward, attention_forward, backward_part,
                        computeD, flashAttentionBackward, flashAttentionBackwardNoAlloc, flashAttentionBackwardWorkspace,
                        flashAttentionForward, forward_items, library, work_map, workspace_bytes)

from . import glue  # noqa: E402  (layernorm, residual add, dX cast around the sublayer)
from . import sublayer  # noqa: E402  (the GEMMs around the attention core)

__all__ = ["glue", "sublayer", "AttentionError", "AttentionParams", "attention_backward", "attention_forward", "backward_part",
           "computeD", "flashAttentionBackward", "flashAttentionBackwardNoAlloc", "flashAttentionBackwardWorkspace",
           "flashAttentionForward", "forward_items", "library",
           "work_map", "workspace_bytes"]
