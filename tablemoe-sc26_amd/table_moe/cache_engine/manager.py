"""HybridStorageManager: per-layer offline table + online window, resident in HBM.

Same constructor, attributes and methods as the reference
(table_moe/cache_engine/manager.py:34-228).  One deliberate difference: the
cached expert outputs ``values_buffer`` live in device memory (HBM) instead of
pinned host memory, so ``gather_values`` is a device gather (``tm_gather_rows``)
and returns a device tensor; the reference's caller then calls ``.to(device)``,
which is a no-op.  Reading the on-disk table (PCA + per-(expert, modality)
``*_cache.pt`` files) is load-time work done with torch as in the reference;
a layer converted to the packed format (``table_file.py``: one file, the
buffers' own layout) is loaded from it instead when present, with the same
resulting buffers bit for bit.
"""

from __future__ import annotations

import glob
import os

import torch

from .. import _native as N
from . import table_file
from .config import CacheConfig


def _resolve_cache_dtype():
    dtype = getattr(CacheConfig, "MODEL_DTYPE", torch.bfloat16)
    if isinstance(dtype, torch.dtype):
        return dtype
    if isinstance(dtype, str):
        name = dtype.removeprefix("torch.").lower()
        table = {"float16": torch.float16, "bfloat16": torch.bfloat16, "float32": torch.float32}
        if name in table:
            return table[name]
    raise ValueError(f"Unsupported cache dtype: {dtype!r}")


# key normalisation at load (manager.py:24-31) and the cache file name rule,
# shared with the packed-format converter
_normalize_last_dim = table_file.normalize_last_dim
_parse_cache_name = table_file.parse_cache_name


class HybridStorageManager:
    def __init__(self, layer_idx, num_experts, hidden_dim, device="cuda:0", use_packed: bool = True):
        self.layer_idx = layer_idx
        self.num_experts = num_experts
        self.hidden_dim = hidden_dim
        self.device = torch.device(device) if not isinstance(device, torch.device) else device
        self.dtype = _resolve_cache_dtype()

        packed = table_file.packed_path(layer_idx)
        if use_packed and os.path.exists(packed):
            self._load_packed(packed)
        else:
            self.pca = self._load_pca()
            shape = (num_experts, 2, CacheConfig.FIXED_K, CacheConfig.COMPRESSED_DIM)
            self.keys_buffer = torch.zeros(shape, dtype=self.dtype, device=self.device)
            self.raw_keys_buffer = torch.zeros(shape, dtype=self.dtype, device=self.device)
            self.values_buffer = torch.zeros(
                (num_experts, 2, CacheConfig.FIXED_K, hidden_dim), dtype=self.dtype, device=self.device
            )
            self._load_cache_data()

        self.enable_online = CacheConfig.ONLINE_MIN_LAYER_IDX <= layer_idx <= CacheConfig.ONLINE_MAX_LAYER_IDX
        self.online_ptr = 0
        self.online_size = 0
        self.online_full = False
        self.online_topk = 0
        if self.enable_online:
            self.online_size = CacheConfig.ONLINE_CACHE_SIZE
            self.online_topk = CacheConfig.ONLINE_TOP_K
            self.online_keys = torch.zeros((self.online_size, hidden_dim), dtype=self.dtype, device=self.device)
            self.online_values = torch.zeros(
                (self.online_size, self.online_topk, hidden_dim), dtype=self.dtype, device=self.device
            )
            self.online_expert_ids = torch.full(
                (self.online_size, self.online_topk), -1, dtype=torch.long, device=self.device
            )
        else:
            self.online_keys = None
            self.online_values = None
            self.online_expert_ids = None

    # --------------------------------------------------------------- loading
    def _pca_entry(self, data):
        """{"mean", "proj"} -> projection and bias -mean @ proj in the model dtype
        on the table's device (manager.py:157-181)."""
        if data is None:
            return {
                "proj": torch.zeros((self.hidden_dim, CacheConfig.COMPRESSED_DIM), device=self.device,
                                    dtype=self.dtype),
                "bias": torch.zeros(CacheConfig.COMPRESSED_DIM, device=self.device, dtype=self.dtype),
            }
        mean = data["mean"].to(device=self.device, dtype=self.dtype)
        proj = data["proj"].to(device=self.device, dtype=self.dtype)
        return {"proj": proj, "bias": -torch.matmul(mean, proj)}

    def _load_pca(self):
        pca_dir = os.path.join(CacheConfig.PCA_DIR, f"layer_{self.layer_idx}")
        out = {}
        for mod in ("vision", "text"):
            path = os.path.join(pca_dir, f"L{self.layer_idx}_{mod}_pca.pt")
            data = torch.load(path, map_location=self.device, weights_only=True) if os.path.exists(path) else None
            out[mod] = self._pca_entry(data)
        return out

    def _load_packed(self, path):
        """One packed file (table_file.py): bulk copies of the buffers."""
        expect = {"num_experts": self.num_experts, "hidden": self.hidden_dim, "fixed_k": int(CacheConfig.FIXED_K),
                  "dim": int(CacheConfig.COMPRESSED_DIM), "dtype": table_file._TORCH_TO_NAME[self.dtype],
                  "layer": self.layer_idx}
        data = table_file.load_layer(path, self.device, expect=expect)
        self.raw_keys_buffer = data["keys"]
        self.keys_buffer = data["keys_norm"]
        self.values_buffer = data["values"]
        self.pca = {}
        for mod in ("vision", "text"):
            entry = None
            if f"pca_mean_{mod}" in data:
                entry = {"mean": data[f"pca_mean_{mod}"], "proj": data[f"pca_proj_{mod}"]}
            self.pca[mod] = self._pca_entry(entry)

    def _load_cache_data(self):
        layer_dir = os.path.join(CacheConfig.CACHE_DIR, f"layer_{self.layer_idx}")
        for path in sorted(glob.glob(os.path.join(layer_dir, "*_cache.pt"))):
            try:
                eid, mod = _parse_cache_name(os.path.basename(path))
                mid = CacheConfig.MODALITY_MAP.get(mod, -1)
                if mid == -1 or eid >= self.num_experts:
                    continue
                data = torch.load(path, map_location="cpu", weights_only=True)
                self.load_table_entry(eid, mid, data["key"], data["value"])
            except Exception as exc:  # a bad file is reported and skipped, as the reference does
                print(f"Error loading {path}: {exc}")

    def load_table_entry(self, expert_id: int, modality_id: int, keys: torch.Tensor, values: torch.Tensor):
        """Install one (expert, modality) table: raw keys, normalised keys, values."""
        keys = keys.to(dtype=self.dtype)
        k = keys.shape[0]
        norm_keys = _normalize_last_dim(keys, float(CacheConfig.OFFLINE_COSINE_EPS))
        self.raw_keys_buffer[expert_id, modality_id, :k] = keys.to(self.device)
        self.keys_buffer[expert_id, modality_id, :k] = norm_keys.to(self.device)
        self.values_buffer[expert_id, modality_id, :k] = values.to(device=self.device, dtype=self.dtype)

    # --------------------------------------------------------- online window
    @torch.no_grad()
    def update_online_cache_bs1(self, hidden_state, expert_ids, expert_outputs, valid_slot_mask=None):
        if not self.enable_online:
            return
        self._ring_write(hidden_state.reshape(1, -1), expert_ids.reshape(1, -1),
                         expert_outputs.reshape(1, *expert_outputs.shape[-2:]),
                         None if valid_slot_mask is None else valid_slot_mask.reshape(1, -1), self.online_ptr)
        self.online_ptr = (self.online_ptr + 1) % self.online_size
        if self.online_ptr == 0:
            self.online_full = True

    @torch.no_grad()
    def update_online_cache(self, hidden_states, expert_ids, expert_outputs, valid_slot_mask=None):
        if not self.enable_online:
            return
        n = hidden_states.shape[0]
        if n == 0:
            return
        if n > self.online_size:
            hidden_states = hidden_states[-self.online_size:]
            expert_ids = expert_ids[-self.online_size:]
            expert_outputs = expert_outputs[-self.online_size:]
            if valid_slot_mask is not None:
                valid_slot_mask = valid_slot_mask[-self.online_size:]
            n = self.online_size
        start = self.online_ptr
        self._ring_write(hidden_states, expert_ids, expert_outputs, valid_slot_mask, start)
        end = start + n
        if end > self.online_size:
            self.online_full = True
        self.online_ptr = end % self.online_size
        if self.online_ptr == 0:
            self.online_full = True

    def _ring_write(self, hidden, ids, outputs, valid, start):
        dev = N.require_hip(hidden, ids, outputs, self.online_keys)
        if hidden.dtype != self.dtype or outputs.dtype != self.dtype:
            hidden, outputs = hidden.to(self.dtype), outputs.to(self.dtype)
        if hidden.stride(-1) != 1:
            hidden = hidden.contiguous()
        if outputs.stride(-1) != 1:
            outputs = outputs.contiguous()
        ids = ids if (ids.dtype == torch.long and ids.stride(-1) == 1) else ids.long().contiguous()
        v = None if valid is None else N.as_u8(valid.to(device=dev, dtype=torch.bool).contiguous())
        n, top_k = ids.shape
        N.call(
            "tm_online_update", N.dtype_tag(self.dtype), N.ptr(hidden), hidden.stride(0), N.ptr(ids), ids.stride(0),
            N.ptr(outputs), outputs.stride(0), outputs.stride(1), N.ptr(v), 0 if v is None else v.stride(0), n,
            top_k, self.hidden_dim, int(start), self.online_size, N.ptr(self.online_keys),
            N.ptr(self.online_expert_ids), N.ptr(self.online_values), N.stream(dev),
        )

    @torch.no_grad()
    def combine_and_update_bs1(self, hidden_state, routing_weights_row, selected_experts_row, is_vision,
                               compute_mask_row, computed, on_hit, on_idx, on_slot, off_hit, off_idx, out,
                               target: str = "one"):
        """The decode step's tail for one token in one launch
        (tm_decode_combine_update): out = sum of the surviving slots' sources
        (computed / online window / offline table) with renormalised weights,
        then the token enters the online window (ring row online_ptr, as
        update_online_cache_bs1 with the survivor mask).  Without an online
        window only the combine runs (tm_slot_combine)."""
        dev = N.require_hip(hidden_state, routing_weights_row, selected_experts_row, out)
        k = int(selected_experts_row.numel())
        mode = N.TM_TARGET_ORIG_SUM if target == "orig_sum" else N.TM_TARGET_ONE
        w = routing_weights_row.reshape(-1).to(torch.float32).contiguous()
        sel = selected_experts_row.reshape(-1).to(torch.long).contiguous()
        u8 = lambda t: None if t is None else N.as_u8(t.reshape(-1).to(device=dev, dtype=torch.bool).contiguous())  # noqa: E731
        cm, oh, fh = u8(compute_mask_row), u8(on_hit), u8(off_hit)
        isv = None if is_vision is None else u8(is_vision)
        ix = lambda t: None if t is None else t.reshape(-1).to(device=dev, dtype=torch.long).contiguous()  # noqa: E731
        oi, osl, fi = ix(on_idx), ix(on_slot), ix(off_idx)
        x = hidden_state.reshape(-1)
        comp = None if computed is None else computed.reshape(k, -1)
        v = self.values_buffer
        if self.enable_online:
            ov = self.online_values
            N.call("tm_decode_combine_update", N.dtype_tag(self.dtype), k, self.hidden_dim, N.ptr(w), N.ptr(cm),
                   N.ptr(comp), 0 if comp is None else comp.stride(0), N.ptr(fh), N.ptr(fi), N.ptr(sel), N.ptr(isv),
                   N.ptr(v), v.shape[0], v.shape[2], v.stride(0), v.stride(1), v.stride(2), N.ptr(oh), N.ptr(oi),
                   N.ptr(osl), N.ptr(ov), self.online_size, ov.shape[1], ov.stride(0), ov.stride(1), mode, None,
                   N.ptr(out), N.ptr(x), N.ptr(self.online_keys), N.ptr(self.online_expert_ids),
                   int(self.online_ptr), N.stream(dev))
            self.online_ptr = (self.online_ptr + 1) % self.online_size
            if self.online_ptr == 0:
                self.online_full = True
        else:
            N.call("tm_slot_combine", N.dtype_tag(self.dtype), 1, k, self.hidden_dim, N.ptr(w), k, N.ptr(cm),
                   N.ptr(comp), 0, 0 if comp is None else comp.stride(0), N.ptr(fh), N.ptr(fi), N.ptr(sel), k,
                   N.ptr(isv), N.ptr(v), v.shape[0], v.shape[2], v.stride(0), v.stride(1), v.stride(2), None, None,
                   None, None, 0, 1, 0, 0, mode, None, 0, N.ptr(out), out.stride(0) if out.dim() > 1 else
                   self.hidden_dim, N.stream(dev))
        return out

    @torch.no_grad()
    def combine_slots(self, routing_weights, selected_experts, is_vision, compute_mask, computed, off_hit, off_idx,
                      on_hit=None, on_idx=None, on_slot=None, out=None, residual=None, target: str = "one"):
        """The slot combine of a prefill/decode batch in one launch
        (tm_slot_combine), for a hook that calls it instead of filling the
        [N, k, H] collected buffer (cached_layers.py:302 zero-fill, :441-461
        scatters, :462-465 renormalise + bmm): out[b] = sum over the surviving
        slots s of w~[b, s] * source(b, s), source = computed[b, s] where
        compute_mask, else the online window row (on_idx[b], on_slot[b, s])
        where on_hit, else the table row values[sel[b, s], m(b), off_idx[b, s]]
        where off_hit; w~ = the routing weights renormalised over the
        survivors (target "one": rounded to the model dtype, as the hook's
        .to(dtype); "orig_sum").  No host sync: the hit indices stay on the
        device.  residual (optional) is added before the one rounding."""
        dev = N.require_hip(routing_weights, selected_experts, compute_mask)
        n, k = selected_experts.shape
        mode = N.TM_TARGET_ORIG_SUM if target == "orig_sum" else N.TM_TARGET_ONE
        w = routing_weights.to(torch.float32).contiguous()
        sel = selected_experts.to(torch.long).contiguous()
        u8 = lambda t: None if t is None else N.as_u8(t.to(device=dev, dtype=torch.bool).contiguous())  # noqa: E731
        ix = lambda t: None if t is None else t.to(device=dev, dtype=torch.long).contiguous()  # noqa: E731
        cm, fh, oh = u8(compute_mask), u8(off_hit), u8(on_hit)
        isv = None if is_vision is None else u8(is_vision.reshape(-1))
        fi, oi, osl = ix(off_idx), ix(None if on_idx is None else on_idx.reshape(-1)), ix(on_slot)
        if computed is not None and (computed.stride(-1) != 1 or computed.dtype != self.dtype):
            raise ValueError(f"computed must be [N, k, H] {self.dtype} with unit stride along hidden")
        if out is None:
            out = torch.empty((n, self.hidden_dim), dtype=self.dtype, device=dev)
        v = self.values_buffer
        ov = self.online_values if (oh is not None and self.enable_online) else None
        N.call("tm_slot_combine", N.dtype_tag(self.dtype), n, k, self.hidden_dim, N.ptr(w), w.stride(0), N.ptr(cm),
               N.ptr(computed), 0 if computed is None else computed.stride(0),
               0 if computed is None else computed.stride(1), N.ptr(fh), N.ptr(fi), N.ptr(sel), k, N.ptr(isv),
               N.ptr(v), v.shape[0], v.shape[2], v.stride(0), v.stride(1), v.stride(2), N.ptr(oh), N.ptr(oi),
               N.ptr(osl), N.ptr(ov), 0 if ov is None else self.online_size, 1 if ov is None else ov.shape[1],
               0 if ov is None else ov.stride(0), 0 if ov is None else ov.stride(1), mode, N.ptr(residual),
               0 if residual is None else residual.stride(0), N.ptr(out), out.stride(0), N.stream(dev))
        return out

    # ---------------------------------------------------------------- gather
    def _gather_into(self, expert_ids, modality_ids, modality, cluster_ids, dst_rows, out):
        dev = out.device
        v = self.values_buffer
        eids = expert_ids.to(device=dev, dtype=torch.long).contiguous()
        cids = cluster_ids.to(device=dev, dtype=torch.long).contiguous()
        mids = None if modality_ids is None else modality_ids.to(device=dev, dtype=torch.long).contiguous()
        dst = None if dst_rows is None else dst_rows.to(device=dev, dtype=torch.long).contiguous()
        N.call(
            "tm_gather_rows", N.dtype_tag(v.dtype), N.ptr(v), v.shape[0], v.shape[2], v.shape[3], v.stride(0),
            v.stride(1), v.stride(2), N.ptr(eids), N.ptr(mids), int(modality), N.ptr(cids), eids.numel(), N.ptr(dst),
            N.ptr(out), out.shape[0], out.stride(0), N.stream(dev),
        )

    def gather_values(self, expert_ids, modality_ids, cluster_ids):
        """values[e, m, c] rows -> [n, hidden] device tensor (reference manager.py:212-213)."""
        n = int(expert_ids.numel())
        out = torch.empty((n, self.hidden_dim), dtype=self.dtype, device=self.values_buffer.device)
        if n:
            N.require_hip(out)
            self._gather_into(expert_ids.reshape(-1), modality_ids.reshape(-1), 0, cluster_ids.reshape(-1), None, out)
        return out

    @torch.no_grad()
    def gather_values_decode_bs1(self, expert_ids, modality_id, cluster_ids, slot_ids, out_buffer):
        """out_buffer[slot_ids[i]] = values[expert_ids[i], modality_id, cluster_ids[i]]
        (reference manager.py:216-228), one launch instead of a per-slot loop."""
        if int(expert_ids.numel()) == 0:
            return
        N.require_hip(out_buffer)
        self._gather_into(expert_ids.reshape(-1), None, int(modality_id), cluster_ids.reshape(-1),
                          slot_ids.reshape(-1), out_buffer)
