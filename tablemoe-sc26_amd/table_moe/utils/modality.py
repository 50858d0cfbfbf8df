"""Per-thread modality / importance context (table_moe/utils/modality.py:6-69).

Host-side bookkeeping: the vision mask of the current prompt is derived once
per (device, seq_len) from the Qwen vision token ids and cached.
"""

from __future__ import annotations

import threading

import torch

VISION_TOKEN_IDS = (151655, 151656)


class ModalityContext:
    _local = threading.local()

    @classmethod
    def set_input_ids(cls, input_ids: torch.Tensor):
        cls._local.input_ids = input_ids
        cls._clear_cache()

    @classmethod
    def get_input_ids(cls):
        return getattr(cls._local, "input_ids", None)

    @classmethod
    def set_attn_weights(cls, weights: torch.Tensor):
        cls._local.attn_weights = weights

    @classmethod
    def get_attn_weights(cls):
        return getattr(cls._local, "attn_weights", None)

    @classmethod
    def clear(cls):
        for name in ("input_ids", "attn_weights"):
            if hasattr(cls._local, name):
                delattr(cls._local, name)
        cls._clear_cache()

    @classmethod
    def _clear_cache(cls):
        if hasattr(cls._local, "cached_result"):
            del cls._local.cached_result

    @classmethod
    def get_modality_mask(cls, current_device, seq_len=None):
        cached = getattr(cls._local, "cached_result", None)
        if cached is not None and cached[0] == current_device and cached[1] == seq_len:
            return cached[2]
        ids = cls.get_input_ids()
        if ids is None:
            mask = torch.zeros((1, seq_len if seq_len is not None else 1), dtype=torch.bool, device=current_device)
        else:
            vis = (ids == VISION_TOKEN_IDS[0]) | (ids == VISION_TOKEN_IDS[1])
            if seq_len is not None and vis.shape[1] != seq_len:
                vis = vis[:, -1:] if seq_len == 1 else vis[:, -seq_len:]
            mask = vis.to(current_device)
        cls._local.cached_result = (current_device, seq_len, mask)
        return mask
