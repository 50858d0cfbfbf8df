"""VectorSearchEngine: the reference search surface over HIP kernels.

Same class, method names, argument meaning, return conventions (fresh tensors,
workspace views for ``search_decode_hybrid``, caller buffers for ``*_into``)
and error types as the reference (table_moe/cache_engine/search.py:388-1105).
The work runs in ``tm_project`` + ``tm_search_gated`` (offline searches) and
``tm_search_hybrid`` (decode window + offline), enqueued on torch's current
stream with no host synchronisation.

Semantics follow the reference's torch path (the one its unit tests pin):
cosine searches hit on ``max >= threshold``, raw-dot searches on
``max > OFFLINE_DOT_THRESHOLD``, decode searches against normalised keys on
``max >= 0``; scores are fp32 sums of the model-dtype products.
"""

from __future__ import annotations

import torch

from .. import _native as N
from .config import CacheConfig

# The reference exports whether its Triton kernels are active; this
# implementation has none.
HAS_TRITON = False


def _round_cap(batch_size: int) -> int:
    cap = max(batch_size, 128)
    return ((cap + 127) // 128) * 128


_BYTE_MASKS = (torch.bool, torch.uint8)

class VectorSearchEngine:
    def __init__(self, manager):
        self.manager = manager
        self.device = manager.device
        self.workspace_capacity = 0
        self.workspace = {}
        self.prefill_query_workspace_capacity = 0
        self.prefill_query_workspace = None
        self.decode_query_workspace_capacity = 0
        self.decode_query_workspace = None
        self.search_dims_cache = None
        self._workspace_top_k = None

    # ------------------------------------------------------------------ setup
    def _get_pca_pair(self):
        pca_map = getattr(self.manager, "pca", None)
        if not isinstance(pca_map, dict) or not pca_map:
            raise ValueError("manager.pca must be a non-empty dict")
        if "vision" in pca_map and "text" in pca_map:
            return pca_map["vision"], pca_map["text"]
        shared = pca_map[next(iter(pca_map))]
        return shared, shared

    def _get_search_dims(self):
        if self.search_dims_cache is not None:
            return self.search_dims_cache
        pca_vis, pca_txt = self._get_pca_pair()
        compressed_dim = int(pca_vis["proj"].shape[1])
        if int(pca_txt["proj"].shape[1]) != compressed_dim:
            raise ValueError("vision/text PCA projection dims must match")
        online_topk = None
        if getattr(self.manager, "online_expert_ids", None) is not None:
            online_topk = int(self.manager.online_expert_ids.shape[1])
        self.search_dims_cache = {
            "pca_vis": pca_vis,
            "pca_txt": pca_txt,
            "compressed_dim": compressed_dim,
            "fixed_k": int(self.manager.keys_buffer.shape[2]),
            "online_topk": online_topk,
            # k-contiguous copies of the projections (fused decode projection)
            "proj_t": (self._transposed(pca_vis["proj"]), self._transposed(pca_txt["proj"])),
            # packed layouts for tm_project (None: the strided copies are used)
            "proj_pk": self._packed(pca_vis, pca_txt),
        }
        return self.search_dims_cache

    @staticmethod
    def _transposed(proj: torch.Tensor) -> torch.Tensor:
        return proj.t().contiguous()  # [dim, hidden]

    @staticmethod
    def _packed(pca_vis, pca_txt):
        pk = (N.pack_projection(pca_vis["proj"], pca_vis["bias"]), N.pack_projection(pca_txt["proj"], pca_txt["bias"]))
        return None if any(p is None for p in pk) else pk

    def _ensure_workspace(self, batch_size, top_k):
        if batch_size > self.workspace_capacity or top_k != self._workspace_top_k:
            cap = _round_cap(max(batch_size, self.workspace_capacity))
            dev = self.device
            self.workspace["on_hit"] = torch.zeros((cap, top_k), dtype=torch.bool, device=dev)
            self.workspace["off_hit"] = torch.zeros((cap, top_k), dtype=torch.bool, device=dev)
            self.workspace["off_idx"] = torch.zeros((cap, top_k), dtype=torch.long, device=dev)
            self.workspace["on_idx"] = torch.full((cap,), -1, dtype=torch.long, device=dev)
            self.workspace["on_slot"] = torch.zeros((cap, top_k), dtype=torch.long, device=dev)
            self.workspace["reuse"] = torch.zeros((cap, top_k), dtype=torch.bool, device=dev)
            self.workspace_capacity = cap
            self._workspace_top_k = top_k

    def _query_workspace(self, attr_ws, attr_cap, batch_size, compressed_dim):
        dtype = self.manager.keys_buffer.dtype
        ws = getattr(self, attr_ws)
        if (
            ws is None
            or batch_size > getattr(self, attr_cap)
            or ws.shape[1] != compressed_dim
            or ws.dtype != dtype
        ):
            cap = _round_cap(batch_size)
            ws = torch.zeros((cap, compressed_dim), dtype=dtype, device=self.device)
            setattr(self, attr_ws, ws)
            setattr(self, attr_cap, cap)
        return ws[:batch_size]

    def _ensure_prefill_query_workspace(self, batch_size, compressed_dim):
        return self._query_workspace(
            "prefill_query_workspace", "prefill_query_workspace_capacity", batch_size, compressed_dim
        )

    def _ensure_decode_query_workspace(self, batch_size, compressed_dim):
        return self._query_workspace(
            "decode_query_workspace", "decode_query_workspace_capacity", batch_size, compressed_dim
        )

    # ------------------------------------------------------------ projection
    def _project_queries_into(self, hidden_states, is_vision_mask, search_dims, query_low, normalize):
        """q = dtype(x @ P_m + bias_m) (+ L2 normalisation) into ``query_low``
        (reference search.py:476-498)."""
        dev = N.require_hip(hidden_states, query_low)
        x = hidden_states if hidden_states.stride(-1) == 1 else hidden_states.contiguous()
        n, hidden = x.shape
        self._project_call(dev, x, n, hidden, x.stride(0), is_vision_mask, search_dims, query_low,
                           query_low.stride(0), normalize)
        return query_low

    def _project_call(self, dev, x, n, hidden, ld_x, is_vision_mask, search_dims, query_low, ld_q, normalize):
        """tm_project on plain pointers and row strides (the bs1 path passes its
        1-D row without a 2-D view)."""
        dtype = self.manager.keys_buffer.dtype
        if x.dtype != dtype:
            raise RuntimeError(f"hidden_states dtype {x.dtype} != table dtype {dtype}")
        pv, pt = search_dims["pca_vis"], search_dims["pca_txt"]
        tv, tt = search_dims["proj_t"]
        isv = N.mask_bytes(is_vision_mask, dev)
        d = search_dims["compressed_dim"]
        pk = search_dims["proj_pk"]
        x_ptr, q_ptr = x.data_ptr(), query_low.data_ptr()
        if pk is not None and x_ptr % 16 == 0 and ld_x % 8 == 0 and q_ptr % 16 == 0 and ld_q % 8 == 0:
            (tv, tt), ps_h, ps_d, ws = pk, 0, 0, None  # packed layout, no workspace
        else:
            ps_h, ps_d = 1, hidden
            ws = self._scratch("project", N.lib().tm_project_workspace_size(n, hidden, d))
        N.call(
            "tm_project", N.dtype_tag(dtype), x_ptr, n, hidden, ld_x, isv.data_ptr(),
            N.ptr(tv), N.ptr(pv["bias"]), N.ptr(tt), N.ptr(pt["bias"]), ps_h, ps_d, d,
            1 if normalize else 0, float(CacheConfig.OFFLINE_COSINE_EPS), q_ptr, ld_q,
            None, N.ptr(ws), 0 if ws is None else ws.numel(), N.stream(dev),
        )

    def _scratch(self, name, nbytes):
        """Reusable device workspace of at least ``nbytes`` (None for 0)."""
        if nbytes <= 0:
            return None
        cache = self.__dict__.setdefault("_scratch_bufs", {})
        buf = cache.get(name)
        if buf is None or buf.numel() < nbytes:
            buf = torch.empty(nbytes, dtype=torch.uint8, device=self.device)
            cache[name] = buf
        return buf

    def _build_prefill_queries(self, hidden_states, is_vision_mask, search_dims):
        q = self._ensure_prefill_query_workspace(hidden_states.shape[0], search_dims["compressed_dim"])
        return self._project_queries_into(hidden_states, is_vision_mask, search_dims, q, normalize=True)

    def _build_prefill_queries_offline_dot(self, hidden_states, is_vision_mask, search_dims):
        q = self._ensure_prefill_query_workspace(hidden_states.shape[0], search_dims["compressed_dim"])
        return self._project_queries_into(hidden_states, is_vision_mask, search_dims, q, normalize=False)

    def _build_decode_queries(self, hidden_states, is_vision_mask, search_dims):
        q = self._ensure_decode_query_workspace(hidden_states.shape[0], search_dims["compressed_dim"])
        return self._project_queries_into(hidden_states, is_vision_mask, search_dims, q, normalize=False)

    # ----------------------------------------------------------- gated search
    def _gated_into(self, query_low, keys, selected_experts, is_vision_mask, reuse_mask, out_hit, out_idx,
                    thr_vision, thr_text, cmp, col_offset=0):
        dev = N.require_hip(query_low, keys, selected_experts, out_hit, out_idx)
        n, top_k = selected_experts.shape
        sel = selected_experts if selected_experts.dtype == torch.long else selected_experts.long()
        rs = None if reuse_mask is None else N.as_u8(reuse_mask.to(device=dev, dtype=torch.bool))
        self._gated_call(dev, query_low, n, query_low.stride(0), keys, sel, top_k, sel.stride(0), sel.stride(1),
                         is_vision_mask, rs, 0 if rs is None else rs.stride(0), 0 if rs is None else rs.stride(1),
                         out_hit, out_idx, out_hit.stride(0), out_hit.stride(1), thr_vision, thr_text, cmp,
                         col_offset)

    def _gated_call(self, dev, query_low, n, ld_q, keys, sel, top_k, sel_s0, sel_s1, is_vision_mask, rs, rs_s0,
                    rs_s1, out_hit, out_idx, out_s0, out_s1, thr_vision, thr_text, cmp, col_offset):
        """tm_search_gated on plain pointers and strides (out_hit and out_idx
        share the element strides out_s0/out_s1)."""
        isv = N.mask_bytes(is_vision_mask, dev)
        if keys.stride(-1) != 1:
            raise ValueError("keys must have a unit stride along the PCA dimension")
        if out_hit.dtype not in _BYTE_MASKS:
            raise ValueError("out_hit must be a bool (or uint8) tensor")
        N.call(
            "tm_search_gated", N.dtype_tag(keys.dtype), query_low.data_ptr(), n, ld_q, keys.data_ptr(),
            keys.shape[0], keys.shape[2], keys.shape[3], keys.stride(0), keys.stride(1), keys.stride(2),
            sel.data_ptr(), top_k, sel_s0, sel_s1, isv.data_ptr(), N.ptr(rs), rs_s0, rs_s1, col_offset,
            float(thr_vision), float(thr_text), cmp, out_hit.data_ptr(), out_idx.data_ptr(), out_s0, out_s1,
            N.stream(dev),
        )

    def _search_prefill_offline_into(self, query_low, selected_experts, is_vision_mask, reuse_mask,
                                     out_hit_mask, out_cluster_indices):
        self._gated_into(
            query_low, self.manager.keys_buffer, selected_experts, is_vision_mask, reuse_mask,
            out_hit_mask, out_cluster_indices, CacheConfig.OFFLINE_COSINE_THRESHOLD_VISION,
            CacheConfig.OFFLINE_COSINE_THRESHOLD_TEXT, N.TM_CMP_GE,
        )

    def _search_decode_offline_from_low_into(self, query_low, selected_experts, is_vision_mask, reuse_mask,
                                             out_hit_mask, out_cluster_indices, threshold_vision=0.0,
                                             threshold_text=0.0):
        self._gated_into(
            query_low, self.manager.keys_buffer, selected_experts, is_vision_mask, reuse_mask,
            out_hit_mask, out_cluster_indices, threshold_vision, threshold_text, N.TM_CMP_GE,
        )

    def _search_offline_dot_from_low_into(self, query_low, selected_experts, is_vision_mask, reuse_mask,
                                          out_hit_mask, out_cluster_indices):
        thr = float(CacheConfig.OFFLINE_DOT_THRESHOLD)
        self._gated_into(
            query_low, self.manager.raw_keys_buffer, selected_experts, is_vision_mask, reuse_mask,
            out_hit_mask, out_cluster_indices, thr, thr, N.TM_CMP_GT,
        )

    def _search_decode_offline_into(self, hidden_states, selected_experts, is_vision_mask, reuse_mask,
                                    out_hit_mask, out_cluster_indices):
        q = self._build_decode_queries(hidden_states, is_vision_mask, self._get_search_dims())
        self._search_decode_offline_from_low_into(
            q, selected_experts, is_vision_mask, reuse_mask, out_hit_mask, out_cluster_indices
        )

    def _fresh_outputs(self, selected_experts):
        bs, top_k = selected_experts.shape
        return (
            torch.empty((bs, top_k), dtype=torch.bool, device=self.device),
            torch.empty((bs, top_k), dtype=torch.long, device=self.device),
        )

    # ------------------------------------------------------- public searches
    def search_prefill_offline(self, layer_idx, hidden_states, selected_experts, is_vision_mask, reuse_mask):
        hit, idx = self._fresh_outputs(selected_experts)
        q = self._build_prefill_queries(hidden_states, is_vision_mask, self._get_search_dims())
        self._search_prefill_offline_into(q, selected_experts, is_vision_mask, reuse_mask, hit, idx)
        return hit, idx

    def search_prefill_offline_dot(self, layer_idx, hidden_states, selected_experts, is_vision_mask, reuse_mask):
        hit, idx = self._fresh_outputs(selected_experts)
        q = self._build_prefill_queries_offline_dot(hidden_states, is_vision_mask, self._get_search_dims())
        self._search_offline_dot_from_low_into(q, selected_experts, is_vision_mask, reuse_mask, hit, idx)
        return hit, idx

    def search_decode_offline(self, layer_idx, hidden_states, selected_experts, is_vision_mask, reuse_mask):
        hit, idx = self._fresh_outputs(selected_experts)
        self._search_decode_offline_into(hidden_states, selected_experts, is_vision_mask, reuse_mask, hit, idx)
        return hit, idx

    def search_decode_offline_dot(self, layer_idx, hidden_states, selected_experts, is_vision_mask, reuse_mask):
        hit, idx = self._fresh_outputs(selected_experts)
        q = self._build_decode_queries(hidden_states, is_vision_mask, self._get_search_dims())
        self._search_offline_dot_from_low_into(q, selected_experts, is_vision_mask, reuse_mask, hit, idx)
        return hit, idx

    # ---------------------------------------------------------- hybrid search
    def _online_state(self):
        m = self.manager
        valid = m.online_size if getattr(m, "online_full", False) else getattr(m, "online_ptr", 0)
        keys = getattr(m, "online_keys", None)
        ids = getattr(m, "online_expert_ids", None)
        if keys is None or ids is None or valid <= 0:
            return None, None, 0
        return keys, ids, int(valid)

    def _hybrid_into(self, hidden_states, selected_experts, is_vision_mask, keep_k, on_hit, on_idx, off_hit,
                     off_idx, on_slot):
        dev = N.require_hip(hidden_states, selected_experts, on_hit, off_idx)
        x = hidden_states if hidden_states.stride(-1) == 1 else hidden_states.contiguous()
        n, hidden = x.shape
        sel = selected_experts if selected_experts.dtype == torch.long else selected_experts.long()
        self._hybrid_call(dev, x, n, hidden, x.stride(0), is_vision_mask, sel, sel.shape[1], sel.stride(0),
                          sel.stride(1), keep_k, on_hit, on_idx, off_hit, off_idx, on_slot, on_hit.stride(0),
                          on_hit.stride(1))

    def _hybrid_call(self, dev, x, n, hidden, ld_x, is_vision_mask, sel, top_k, sel_s0, sel_s1, keep_k, on_hit,
                     on_idx, off_hit, off_idx, on_slot, out_s0, out_s1):
        """tm_search_hybrid on plain pointers and strides (the four [n, top_k]
        outputs share the element strides out_s0/out_s1); the bs1 path calls
        it on its 1-D tensors without building 2-D views."""
        dims = self._get_search_dims()
        dtype = self.manager.keys_buffer.dtype
        if x.dtype != dtype:
            raise RuntimeError(f"hidden_states dtype {x.dtype} != table dtype {dtype}")
        if on_hit.dtype not in _BYTE_MASKS or off_hit.dtype not in _BYTE_MASKS:
            raise ValueError("on_hit/off_hit must be bool (or uint8) tensors")
        num_search = max(top_k - keep_k, 0)
        on_keys, on_ids, n_valid = self._online_state()
        if num_search <= 0:
            n_valid = 0  # nothing is searched: outputs are only cleared
        if on_ids is not None and on_ids.stride(-1) != 1:
            raise ValueError("online_expert_ids must have a unit stride along slots")
        keys = self.manager.keys_buffer
        isv = N.mask_bytes(is_vision_mask, dev)
        d = dims["compressed_dim"]
        q_ws = self.decode_query_workspace
        if q_ws is None or n > self.decode_query_workspace_capacity or q_ws.shape[1] != d or q_ws.dtype != dtype:
            q_ws = self._ensure_decode_query_workspace(n, d)
        sizes = self.__dict__.setdefault("_hybrid_ws_sizes", {})
        nbytes = sizes.get((n, hidden, d))
        if nbytes is None:
            nbytes = sizes[(n, hidden, d)] = N.lib().tm_search_hybrid_workspace_size(n, hidden, d)
        ws = self._scratch("hybrid", nbytes)
        pv, pt = dims["pca_vis"], dims["pca_txt"]
        tv, tt = dims["proj_t"]
        N.call(
            "tm_search_hybrid", N.dtype_tag(dtype), x.data_ptr(), n, hidden, ld_x, isv.data_ptr(),
            N.ptr(tv), N.ptr(pv["bias"]), N.ptr(tt), N.ptr(pt["bias"]), 1, hidden, d,
            N.ptr(on_keys), 0 if on_keys is None else on_keys.stride(0), n_valid, N.ptr(on_ids),
            0 if on_ids is None else on_ids.shape[1], 0 if on_ids is None else on_ids.stride(0),
            keys.data_ptr(), keys.shape[0], keys.shape[2], keys.stride(0), keys.stride(1), keys.stride(2),
            sel.data_ptr(), top_k, sel_s0, sel_s1, int(keep_k), on_hit.data_ptr(), on_idx.data_ptr(),
            off_hit.data_ptr(), off_idx.data_ptr(), on_slot.data_ptr(), out_s0, out_s1,
            q_ws.data_ptr(), q_ws.stride(0), N.ptr(ws), 0 if ws is None else ws.numel(), N.stream(dev),
        )

    def search_decode_hybrid(self, layer_idx, hidden_states, selected_experts, is_vision_mask, keep_k=None):
        batch_size, top_k = selected_experts.shape
        if keep_k is None:
            keep_k = CacheConfig.KEEP_K
        keep_k = max(0, min(int(keep_k), top_k))
        self._ensure_workspace(batch_size, top_k)
        ws = self.workspace
        on_hit = ws["on_hit"][:batch_size, :top_k]
        off_hit = ws["off_hit"][:batch_size, :top_k]
        off_idx = ws["off_idx"][:batch_size, :top_k]
        on_idx = ws["on_idx"][:batch_size]
        on_slot = ws["on_slot"][:batch_size, :top_k]
        self._hybrid_into(hidden_states, selected_experts, is_vision_mask, keep_k, on_hit, on_idx, off_hit,
                          off_idx, on_slot)
        return on_hit, on_idx, off_hit, off_idx, on_slot

    def search_decode_offline_bs1_into(self, hidden_state, selected_experts_row, is_vision, keep_k,
                                       out_off_hit, out_off_idx):
        top_k = int(selected_experts_row.shape[0])
        if top_k == 0:
            return
        keep_k = max(0, min(int(keep_k), top_k))
        # one token: the 1-D tensors go straight to the two calls (no 2-D views)
        dev = N.require_hip(hidden_state, selected_experts_row, out_off_hit, out_off_idx)
        x = hidden_state if hidden_state.stride(-1) == 1 else hidden_state.contiguous()
        hidden = x.shape[-1]
        if x.numel() != hidden:
            raise ValueError(f"hidden_state must hold one token; got shape {tuple(hidden_state.shape)}")
        dims = self._get_search_dims()
        d = dims["compressed_dim"]
        q = self.decode_query_workspace
        if q is None or q.shape[1] != d or q.dtype != self.manager.keys_buffer.dtype:
            q = self._ensure_decode_query_workspace(1, d)
        self._project_call(dev, x, 1, hidden, hidden, is_vision, dims, q, q.stride(0), False)
        sel = selected_experts_row if selected_experts_row.dtype == torch.long else selected_experts_row.long()
        s1, o1 = sel.stride(0), out_off_hit.stride(0)
        thr = float(CacheConfig.OFFLINE_DOT_THRESHOLD)
        self._gated_call(dev, q, 1, q.stride(0), self.manager.raw_keys_buffer, sel, top_k, top_k * s1, s1,
                         is_vision, None, 0, 0, out_off_hit, out_off_idx, top_k * o1, o1, thr, thr, N.TM_CMP_GT,
                         keep_k)

    def search_decode_hybrid_bs1_into(self, hidden_state, selected_experts_row, is_vision, keep_k, out_on_hit,
                                      out_on_idx, out_off_hit, out_off_idx, out_on_slot):
        top_k = int(selected_experts_row.shape[0])
        if top_k == 0:
            out_on_idx.fill_(-1)
            return
        keep_k = max(0, min(int(keep_k), top_k))
        # one token: the 1-D tensors go straight to the call (no 2-D views),
        # which keeps the eager per-call host time near the kernels' own
        dev = N.require_hip(hidden_state, selected_experts_row, out_on_hit, out_off_idx)
        x = hidden_state if hidden_state.stride(-1) == 1 else hidden_state.contiguous()
        hidden = x.shape[-1]
        if x.numel() != hidden:
            raise ValueError(f"hidden_state must hold one token; got shape {tuple(hidden_state.shape)}")
        sel = selected_experts_row if selected_experts_row.dtype == torch.long else selected_experts_row.long()
        s1 = sel.stride(0)
        o1 = out_on_hit.stride(0)
        self._hybrid_call(dev, x, 1, hidden, hidden, is_vision, sel, top_k, top_k * s1, s1, keep_k, out_on_hit,
                          out_on_idx, out_off_hit, out_off_idx, out_on_slot, top_k * o1, o1)
