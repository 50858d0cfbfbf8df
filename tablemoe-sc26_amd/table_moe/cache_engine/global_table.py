"""GlobalTable: one global centroid table with cached per-cluster outputs.

The single-table generalisation of the offline search that the north-star
configurations measure: PCA projection, L2 (or dot) top-k search over C
centroids, keep-by-largest-distance selection of the tokens to recompute, and
the gather of cached outputs fused with the router-weighted combine of the
recomputed slots and the residual add.  Each stage is one C-ABI call:

    tm_topk_softmax -> tm_project -> tm_search_global -> tm_keep_select
    -> tm_gather_combine

The reference counterparts it generalises: the projection
(table_moe/cache_engine/search.py:476-498), the offline search fallback
(search.py:566-602), the keep count (table_moe/skip/pruning.py:45), the gather
(table_moe/cache_engine/manager.py:212-213) and the combine
(table_moe/models/qwen3_vl_moe/cached_layers.py:455-465).
"""

from __future__ import annotations

import torch

from .. import _native as N

_METRICS = {"l2": N.TM_METRIC_L2, "dot": N.TM_METRIC_DOT}


class GlobalTable:
    def __init__(self, centroids: torch.Tensor, values: torch.Tensor, pca_vis, pca_txt=None, metric: str = "l2"):
        """centroids [C, d] and values [C, H] in bf16/fp16 on a HIP device;
        pca_vis / pca_txt = (proj [H, d], bias [d]) in the same dtype."""
        dev = N.require_hip(centroids, values)
        if centroids.dtype not in (torch.bfloat16, torch.float16) or values.dtype != centroids.dtype:
            raise ValueError("centroids/values must share dtype bfloat16 or float16")
        if metric not in _METRICS:
            raise ValueError(f"metric must be one of {sorted(_METRICS)}")
        self.device = dev
        self.dtype = centroids.dtype
        self.metric = metric
        self.centroids = centroids.contiguous()
        self.values = values if values.stride(-1) == 1 else values.contiguous()
        self.n_cent, self.dim = self.centroids.shape
        self.hidden = self.values.shape[1]
        if self.values.shape[0] != self.n_cent:
            raise ValueError("values must have one row per centroid")
        pca_txt = pca_vis if pca_txt is None else pca_txt
        self.proj = (pca_vis[0], pca_txt[0])
        self.proj_t = tuple(p.t().contiguous() for p in self.proj)  # [d, H], k-contiguous
        self.bias = tuple(b.contiguous() for b in (pca_vis[1], pca_txt[1]))
        for p in self.proj:
            if p.shape != (self.hidden, self.dim) or p.dtype != self.dtype:
                raise ValueError(f"projection must be [{self.hidden}, {self.dim}] {self.dtype}")
        self.c_sqnorm = torch.empty(self.n_cent, dtype=torch.float32, device=dev)
        N.call("tm_centroid_sqnorms", N.dtype_tag(self.dtype), N.ptr(self.centroids), self.n_cent, self.dim,
               self.centroids.stride(0), N.ptr(self.c_sqnorm), N.stream(dev))
        self._bufs: dict = {}

    # --------------------------------------------------------------- buffers
    def _buf(self, name, shape, dtype):
        t = self._bufs.get(name)
        numel = 1
        for s in shape:
            numel *= s
        if t is None or t.dtype != dtype or t.numel() < numel:
            t = torch.empty(max(numel, 1), dtype=dtype, device=self.device)
            self._bufs[name] = t
        return t[:numel].view(shape)

    # ---------------------------------------------------------------- stages
    def project(self, hidden: torch.Tensor, is_vision: torch.Tensor | None = None):
        """q = dtype(x @ P_m + bias_m) and ||q||^2 (fp32)."""
        N.require_hip(hidden)
        if hidden.dtype != self.dtype:
            raise RuntimeError(f"hidden dtype {hidden.dtype} != table dtype {self.dtype}")
        x = hidden if hidden.stride(-1) == 1 else hidden.contiguous()
        n = x.shape[0]
        q = self._buf("q", (n, self.dim), self.dtype)
        qn = self._buf("qn", (n,), torch.float32)
        isv = None if is_vision is None else N.as_u8(is_vision.reshape(-1).to(dtype=torch.bool))
        N.call("tm_project", N.dtype_tag(self.dtype), N.ptr(x), n, self.hidden, x.stride(0), N.ptr(isv),
               N.ptr(self.proj_t[0]), N.ptr(self.bias[0]), N.ptr(self.proj_t[1]), N.ptr(self.bias[1]), 1,
               self.hidden, self.dim, 0, 1e-6, N.ptr(q), q.stride(0), N.ptr(qn), N.stream(self.device))
        return q, qn

    def search(self, q: torch.Tensor, top_k: int = 1, q_sqnorm: torch.Tensor | None = None):
        """Nearest centroids: (dist [n, k] fp32, idx [n, k] int64)."""
        N.require_hip(q)
        n = q.shape[0]
        dist = self._buf("dist", (n, top_k), torch.float32)
        idx = self._buf("idx", (n, top_k), torch.long)
        nbytes = N.lib().tm_search_global_workspace_size(n, self.n_cent, self.dim, top_k)
        ws = self._buf("search_ws", (max(nbytes, 1),), torch.uint8)
        N.call("tm_search_global", N.dtype_tag(self.dtype), N.ptr(q), n, q.stride(0), N.ptr(q_sqnorm),
               N.ptr(self.centroids), self.n_cent, self.centroids.stride(0), N.ptr(self.c_sqnorm), self.dim,
               int(top_k), _METRICS[self.metric], N.ptr(dist), N.ptr(idx), N.ptr(ws), ws.numel(),
               N.stream(self.device))
        return dist, idx

    @staticmethod
    def keep_count(n: int, keep_rate: float) -> int:
        return int(N.lib().tm_keep_count(int(n), float(keep_rate)))

    def keep_select(self, score: torch.Tensor, n_keep: int):
        """bool [n]: the n_keep largest scores (ties to the lower index)."""
        N.require_hip(score)
        n = score.shape[0]
        keep = self._buf("keep", (n,), torch.bool)
        N.call("tm_keep_select", N.ptr(score), n, score.stride(0), int(n_keep), N.ptr(N.as_u8(keep)), None, 0,
               N.stream(self.device))
        return keep

    def gather_combine(self, keep, slot_out, weights, idx, dist, residual=None, out=None):
        """out = residual + (keep ? sum_s w~ slot_out : blend of values[idx])."""
        N.require_hip(keep, slot_out, weights, idx)
        n, top_k = weights.shape
        if out is None:
            out = self._buf("out", (n, self.hidden), self.dtype)
        so = slot_out
        N.call("tm_gather_combine", N.dtype_tag(self.dtype), n, self.hidden, N.ptr(N.as_u8(keep)), N.ptr(so),
               so.stride(0), so.stride(1), N.ptr(weights), weights.stride(0), top_k, N.ptr(self.values),
               self.n_cent, self.values.stride(0), N.ptr(idx), N.ptr(dist), idx.stride(0), idx.shape[1],
               N.ptr(residual), 0 if residual is None else residual.stride(0), N.ptr(out), out.stride(0),
               N.stream(self.device))
        return out

    def route(self, router_logits: torch.Tensor, top_k: int):
        n, e = router_logits.shape
        w = self._buf("route_w", (n, top_k), torch.float32)
        ids = self._buf("route_ids", (n, top_k), torch.long)
        N.call("tm_topk_softmax", N.ptr(router_logits), n, e, router_logits.stride(0), int(top_k), 0, N.ptr(w),
               N.ptr(ids), N.stream(self.device))
        return w, ids

    def layer_forward(self, hidden, is_vision, router_logits, slot_out, residual, router_top_k: int = 8,
                      n_nearest: int = 1, keep_rate: float = 0.6, out=None):
        """One MoE layer of the table path; returns a dict of every stage's output."""
        w, ids = self.route(router_logits, router_top_k)
        q, qn = self.project(hidden, is_vision)
        dist, idx = self.search(q, n_nearest, qn)
        keep = self.keep_select(dist[:, 0], self.keep_count(hidden.shape[0], keep_rate))
        y = self.gather_combine(keep, slot_out, w, idx, dist, residual, out)
        return {"weights": w, "ids": ids, "q": q, "qn": qn, "dist": dist, "idx": idx, "keep": keep, "out": y}
