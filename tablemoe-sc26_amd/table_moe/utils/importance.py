"""Importance for the expert-level keep rule on a HIP kernel.

The two reference functions keep their inputs and their effect (the head
average of the last query's attention probabilities, stored with
ModalityContext.set_attn_weights for build_prefill_keep_mask):

* compute_and_cache_importance -- HybridQwen3Attention._compute_and_cache_importance
  (models/qwen3_vl_moe/hybrid_attention.py:111-146): query_states [B, H, S, D],
  key_states [B, Hkv, S, D] after RoPE; scores = (last_q K^T) in the model
  dtype times `scaling` in the model dtype; softmax in fp32; mean over heads.
* cache_last_token_attention -- DeepSeek _cache_last_token_attention
  (models/deepseek_vl2/deepseek_attention.py:206-249): query_states
  [B, q_len, H, D], key_states [B, kv_len, H, D]; fp32 scores times
  softmax_scale; padded keys get probability 0; the last query_length keys.

Both are one tm_last_query_importance call (no repeat_interleave copy of the
keys, no host sync).  Like the reference, a failure stores None; a missing
native library raises instead (there is no silent fallback).
"""

from __future__ import annotations

import torch

from .. import _native as N
from .modality import ModalityContext


def last_query_importance(last_q: torch.Tensor, keys: torch.Tensor, n_kv_heads: int, scale: float,
                          fp32_scores: bool, key_mask: torch.Tensor | None = None, out_len: int | None = None,
                          workspace: torch.Tensor | None = None) -> torch.Tensor:
    """last_q [B, H, D] and keys as a [B, S, Hkv, D] view (any strides with
    unit stride along D) -> importance [B, out_len] fp32."""
    dev = N.require_hip(last_q, keys)
    b, h, d = last_q.shape
    s = keys.shape[1]
    if keys.shape != (b, s, n_kv_heads, d) or last_q.stride(-1) != 1 or keys.stride(-1) != 1:
        raise ValueError("last_query_importance: keys must be a [B, S, Hkv, D] view with unit stride along D")
    out_len = s if out_len is None else int(out_len)
    dt = last_q.dtype
    if keys.dtype != dt:
        raise ValueError("query and key dtypes differ")
    mode = N.TM_SCORE_F32 if (fp32_scores or dt == torch.float32) else N.TM_SCORE_MODEL
    out = torch.empty((b, out_len), dtype=torch.float32, device=dev)
    nbytes = N.lib().tm_importance_workspace_size(b, h, s)
    if workspace is None or workspace.numel() < nbytes:
        workspace = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=dev)
    km = None
    if key_mask is not None:
        km = N.as_u8(key_mask.to(device=dev, dtype=torch.bool).contiguous())
    N.call("tm_last_query_importance", N.dtype_tag(dt), N.ptr(last_q), last_q.stride(0), last_q.stride(1),
           N.ptr(keys), keys.stride(0), keys.stride(1), keys.stride(2), b, h, n_kv_heads, d, s, float(scale), mode,
           N.ptr(km), 0 if km is None else km.stride(0), out_len, N.ptr(out), out.stride(0), N.ptr(workspace),
           workspace.numel(), N.stream(dev))
    return out


def compute_and_cache_importance(query_states: torch.Tensor, key_states: torch.Tensor, scaling: float):
    try:
        with torch.no_grad():
            last_q = query_states[:, :, -1, :]               # [B, H, D]
            keys = key_states.transpose(1, 2)                # [B, S, Hkv, D] view
            mean_score = last_query_importance(last_q, keys, key_states.shape[1], scaling, fp32_scores=False)
            ModalityContext.set_attn_weights(mean_score.view(-1))
            return mean_score
    except N.NativeLibraryMissing:
        raise
    except (ValueError, RuntimeError):
        ModalityContext.set_attn_weights(None)
        return None


def cache_last_token_attention(query_states: torch.Tensor, key_states: torch.Tensor, softmax_scale: float,
                               key_padding_mask: torch.Tensor | None, query_length: int):
    try:
        with torch.no_grad():
            last_q = query_states[:, -1]                     # [B, H, D]
            if last_q.dtype != key_states.dtype:
                last_q = last_q.to(key_states.dtype)
            mean_score = last_query_importance(last_q.contiguous() if last_q.stride(-1) != 1 else last_q,
                                               key_states, key_states.shape[2], softmax_scale, fp32_scores=True,
                                               key_mask=key_padding_mask, out_len=query_length)
            ModalityContext.set_attn_weights(mean_score.reshape(-1))
            return mean_score
    except N.NativeLibraryMissing:
        raise
    except (ValueError, RuntimeError):
        ModalityContext.set_attn_weights(None)
        return None
