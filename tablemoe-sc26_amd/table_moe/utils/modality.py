"""Per-thread prompt context for the MoE layers: which tokens are vision
tokens, and the importance scores the attention layer leaves for the keep
rule.

Interface of table_moe/utils/modality.py:6-69 (the layer hooks call these
classmethods: cached_layers.py:74,289, deepseek_layers.py:359,578,
hybrid_attention.py:81,141,146, deepseek_attention.py:194,246,249):
set_input_ids / get_input_ids, set_attn_weights / get_attn_weights, clear,
and get_modality_mask(current_device, seq_len=None) -> bool [1, seq_len]
(a token is a vision token when its id is one of the Qwen3-VL image/video
pad ids 151655, 151656; no prompt set: all text; a seq_len shorter than the
prompt selects its last seq_len tokens).

Each thread holds one _PromptState.  The masks of a prompt are memoised per
(device, seq_len) -- a prefill call and every decode step of the same
prompt reuse them -- and the memo is dropped whenever a new prompt is set.
"""

from __future__ import annotations

import threading

import torch

VISION_TOKEN_IDS = (151655, 151656)


class _PromptState(threading.local):
    """Per-thread fields, initialised on first use in each thread."""

    def __init__(self):
        self.input_ids: torch.Tensor | None = None
        self.attn_weights: torch.Tensor | None = None
        self.masks: dict = {}


def _vision_tokens(input_ids: torch.Tensor) -> torch.Tensor:
    ids = torch.tensor(VISION_TOKEN_IDS, dtype=input_ids.dtype, device=input_ids.device)
    return torch.isin(input_ids, ids)


class ModalityContext:
    _state = _PromptState()

    @classmethod
    def set_input_ids(cls, input_ids: torch.Tensor):
        cls._state.input_ids = input_ids
        cls._state.masks = {}

    @classmethod
    def get_input_ids(cls):
        return cls._state.input_ids

    @classmethod
    def set_attn_weights(cls, weights: torch.Tensor):
        cls._state.attn_weights = weights

    @classmethod
    def get_attn_weights(cls):
        return cls._state.attn_weights

    @classmethod
    def clear(cls):
        cls._state.input_ids = None
        cls._state.attn_weights = None
        cls._state.masks = {}

    @classmethod
    def get_modality_mask(cls, current_device, seq_len=None):
        key = (torch.device(current_device), seq_len)
        mask = cls._state.masks.get(key)
        if mask is not None:
            return mask
        ids = cls._state.input_ids
        if ids is None:
            mask = torch.zeros((1, 1 if seq_len is None else seq_len), dtype=torch.bool, device=current_device)
        else:
            vision = _vision_tokens(ids)
            if seq_len is not None and seq_len != vision.shape[1]:
                vision = vision[:, -seq_len:]  # the last seq_len tokens (a decode step: the newest)
            mask = vision.to(current_device)
        cls._state.masks[key] = mask
        return mask
