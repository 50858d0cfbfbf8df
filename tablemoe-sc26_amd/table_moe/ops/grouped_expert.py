"""Grouped recompute of the slots that are not reused: every (token, slot)
pair selected by ``mask`` runs its routed expert's SwiGLU MLP and writes
``slot_out[token, slot]`` — the collected[token, slot] rows the reference
fills one expert at a time (models/qwen3_vl_moe/cached_layers.py:431-437)
and the combine consumes.  Two C-ABI calls: tm_group_slots_ws (bucket the pairs
by expert on the device, no host sync) and tm_grouped_swiglu (two grouped
GEMMs on the matrix cores).  Weights are stacked per expert as nn.Linear
keeps them: w1, w3 [E, I, H], w2 [E, H, I]; by default a packed copy of
them (tm_expert_pack_weights: each GEMM tile's 32-column stages stored
contiguously, in the order the GEMM stages them) is made once and
tm_grouped_swiglu_packed runs on it, with the same results bit for bit.
"""

from __future__ import annotations

import torch

from .. import _native as N


class GroupedExperts:
    """Stacked expert weights plus the reusable grouping buffers."""

    def __init__(self, w1: torch.Tensor, w3: torch.Tensor, w2: torch.Tensor, packed: bool = True):
        dev = N.require_hip(w1, w3, w2)
        e, inter, h = w1.shape
        if w3.shape != (e, inter, h) or w2.shape != (e, h, inter):
            raise ValueError("w1/w3 must be [E, I, H] and w2 [E, H, I]")
        if not (w1.dtype == w3.dtype == w2.dtype) or w1.dtype not in (torch.float16, torch.bfloat16):
            raise ValueError("expert weights must share dtype float16 or bfloat16")
        self.w1, self.w3, self.w2 = w1.contiguous(), w3.contiguous(), w2.contiguous()
        self.n_experts, self.inter, self.hidden = e, inter, h
        self.dtype, self.device = w1.dtype, dev
        self._bufs: dict = {}
        self.packed = None
        if packed and h % 128 == 0 and inter % 128 == 0:
            tag = N.dtype_tag(self.dtype)
            ws = []
            for w, role in ((self.w1, N.TM_PACK_GATE_UP), (self.w3, N.TM_PACK_GATE_UP), (self.w2, N.TM_PACK_DOWN)):
                out = torch.empty_like(w)
                N.call("tm_expert_pack_weights", tag, N.ptr(w), e, h, inter, role, N.ptr(out), N.stream(dev))
                ws.append(out)
            self.packed = tuple(ws)

    def _buf(self, name, numel, dtype):
        t = self._bufs.get(name)
        if t is None or t.numel() < numel or t.dtype != dtype:
            t = torch.empty(max(numel, 1), dtype=dtype, device=self.device)
            self._bufs[name] = t
        return t

    def group(self, ids: torch.Tensor, mask: torch.Tensor, slot_out: torch.Tensor):
        """Bucket the masked (token, slot) pairs by expert; ``mask`` is [N, k]
        or a per-token [N] flag."""
        n, k = ids.shape
        m = N.as_u8(mask)
        ms_b, ms_s = (m.stride(0), 0) if m.dim() == 1 else (m.stride(0), m.stride(1))
        t_max = N.lib().tm_group_slots_tiles(n * k, self.n_experts)
        offs = self._buf("offsets", self.n_experts + 1, torch.int32)
        row_token = self._buf("row_token", n * k, torch.int32)
        row_out = self._buf("row_out", n * k, torch.int64)
        tiles = self._buf("tiles", 2 + 2 * t_max, torch.int32)
        nbytes = N.lib().tm_group_slots_workspace_size(n, k, self.n_experts)
        ws = self._buf("group_ws", max(nbytes, 1), torch.uint8)
        N.call("tm_group_slots_ws", N.ptr(ids), n, k, ids.stride(0), N.ptr(m), ms_b, ms_s, self.n_experts,
               slot_out.stride(0), slot_out.stride(1), N.ptr(offs), N.ptr(row_token), N.ptr(row_out), N.ptr(tiles),
               N.ptr(ws), ws.numel(), N.stream(self.device))
        return offs, row_token, row_out, tiles

    def forward(self, hidden: torch.Tensor, ids: torch.Tensor, mask: torch.Tensor, slot_out: torch.Tensor):
        """slot_out[b, s] = expert(ids[b, s]) MLP of hidden[b] for masked pairs
        (others untouched); returns slot_out."""
        N.require_hip(hidden, ids, mask, slot_out)
        if hidden.dtype != self.dtype or slot_out.dtype != self.dtype:
            raise ValueError(f"hidden/slot_out must be {self.dtype}")
        if ids.dtype != torch.long:
            ids = ids.long()
        n, k = ids.shape
        if slot_out.shape != (n, k, self.hidden) or slot_out.stride(-1) != 1:
            raise ValueError(f"slot_out must be [N, {k}, {self.hidden}] with unit stride along hidden")
        if slot_out.stride(0) % 8 or slot_out.stride(1) % 8 or slot_out.data_ptr() % 16:
            raise ValueError("slot_out rows must start on 16-byte boundaries (strides multiples of 8 elements)")
        x = hidden if hidden.stride(-1) == 1 else hidden.contiguous()
        offs, row_token, row_out, tiles = self.group(ids, mask, slot_out)
        tag = N.dtype_tag(self.dtype)
        nbytes = (N.lib().tm_grouped_swiglu_packed_workspace_size(n * k, self.inter, self.n_experts, tag)
                  if self.packed is not None else N.lib().tm_swiglu_workspace_size(n * k, self.inter, tag))
        ws = self._buf("fused", nbytes, torch.uint8)
        fn, (w1, w3, w2) = (("tm_grouped_swiglu_packed", self.packed) if self.packed is not None
                            else ("tm_grouped_swiglu", (self.w1, self.w3, self.w2)))
        N.call(fn, N.dtype_tag(self.dtype), N.ptr(x), x.stride(0), self.hidden, self.inter, self.n_experts, N.ptr(w1),
               N.ptr(w3), N.ptr(w2), n * k, N.ptr(offs), N.ptr(row_token), N.ptr(row_out), N.ptr(tiles),
               N.ptr(slot_out), N.ptr(ws), ws.numel(), N.stream(self.device))
        return slot_out


class SharedExperts:
    """One dense SwiGLU MLP run over every row — a DeepSeek layer's shared
    experts (models/deepseek_vl2/deepseek_layers.py:743) — on a packed copy of
    its nn.Linear weights w1, w3 [I, H] and w2 [H, I] (tm_expert_pack_weights
    with one expert; tm_expert_swiglu_packed), with the same results bit for
    bit as ``expert_swiglu`` on the plain weights."""

    def __init__(self, w1: torch.Tensor, w3: torch.Tensor, w2: torch.Tensor):
        dev = N.require_hip(w1, w3, w2)
        inter, h = w1.shape
        if w3.shape != (inter, h) or w2.shape != (h, inter):
            raise ValueError("w1/w3 must be [I, H] and w2 [H, I]")
        if not (w1.dtype == w3.dtype == w2.dtype) or w1.dtype not in (torch.float16, torch.bfloat16):
            raise ValueError("shared expert weights must share dtype float16 or bfloat16")
        if h % 128 or inter % 128:
            raise ValueError("hidden and intermediate sizes must be multiples of 128")
        self.inter, self.hidden, self.dtype, self.device = inter, h, w1.dtype, dev
        tag = N.dtype_tag(self.dtype)
        packed = []
        for w, role in ((w1, N.TM_PACK_GATE_UP), (w3, N.TM_PACK_GATE_UP), (w2, N.TM_PACK_DOWN)):
            w = w.contiguous()
            out = torch.empty_like(w)
            N.call("tm_expert_pack_weights", tag, N.ptr(w), 1, h, inter, role, N.ptr(out), N.stream(dev))
            packed.append(out)
        self.packed = tuple(packed)
        self._ws = None

    def forward(self, hidden: torch.Tensor, out: torch.Tensor | None = None,
                addend: torch.Tensor | None = None) -> torch.Tensor:
        """y = MLP(hidden) [M, H], or dtype(addend + MLP) with ``addend`` [M, H]
        (not overlapping ``out``) in one rounding."""
        N.require_hip(hidden)
        m, h = hidden.shape
        if h != self.hidden or hidden.dtype != self.dtype or hidden.stride(-1) != 1:
            raise ValueError(f"hidden must be [M, {self.hidden}] {self.dtype} with unit stride")
        if out is None:
            out = torch.empty((m, h), dtype=self.dtype, device=self.device)
        if addend is not None:
            N.require_hip(addend)
            if addend.shape != (m, h) or addend.dtype != self.dtype or addend.stride(-1) != 1:
                raise ValueError(f"addend must be [{m}, {h}] {self.dtype} with unit stride along hidden")
        tag = N.dtype_tag(self.dtype)
        nbytes = N.lib().tm_grouped_swiglu_packed_workspace_size(m, self.inter, 1, tag)
        if self._ws is None or self._ws.numel() < nbytes:
            self._ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=self.device)
        w1, w3, w2 = self.packed
        N.call("tm_expert_swiglu_packed", tag, N.ptr(hidden), m, h, hidden.stride(0), N.ptr(w1), N.ptr(w3), N.ptr(w2),
               self.inter, N.ptr(addend), 0 if addend is None else addend.stride(0), N.ptr(out), out.stride(0),
               N.ptr(self._ws), self._ws.numel(), N.stream(self.device))
        return out
