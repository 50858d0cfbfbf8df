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

import ctypes as C
import os

import torch

from .. import _native as N

_METRICS = {"l2": N.TM_METRIC_L2, "dot": N.TM_METRIC_DOT}


class GlobalTable:
    #: After every tm_table_forward call, synchronise and raise when one of the
    #: launch's bounded cross-workgroup waits ran out (the workspace's error
    #: word grew): a debugging aid for devices shared with other work, on by
    #: TABLEMOE_CHECK_WAITS=1 or per table.
    check_waits = os.environ.get("TABLEMOE_CHECK_WAITS", "0") not in ("", "0")

    def __init__(self, centroids: torch.Tensor, values: torch.Tensor, pca_vis, pca_txt=None, metric: str = "l2"):
        """centroids [C, d] and values [C, H] in bf16/fp16 (matrix-core
        search) or fp32 on a HIP device; pca_vis / pca_txt = (proj [H, d],
        bias [d]) in the same dtype."""
        dev = N.require_hip(centroids, values)
        if centroids.dtype not in (torch.bfloat16, torch.float16, torch.float32) or values.dtype != centroids.dtype:
            raise ValueError("centroids/values must share dtype bfloat16, float16 or float32")
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
        self.bias = tuple(b.contiguous() for b in (pca_vis[1], pca_txt[1]))
        for p in self.proj:
            if p.shape != (self.hidden, self.dim) or p.dtype != self.dtype:
                raise ValueError(f"projection must be [{self.hidden}, {self.dim}] {self.dtype}")
        # packed layout for the matrix cores when it applies, else a k-contiguous copy
        packed = tuple(N.pack_projection(p, b) for p, b in zip(self.proj, self.bias))
        if all(p is not None for p in packed):
            self.proj_dev, self.ps = packed, (0, 0)
        else:
            self.proj_dev, self.ps = tuple(p.t().contiguous() for p in self.proj), (1, self.hidden)
        self.c_sqnorm = torch.empty(self.n_cent, dtype=torch.float32, device=dev)
        N.call("tm_centroid_sqnorms", N.dtype_tag(self.dtype), N.ptr(self.centroids), self.n_cent, self.dim,
               self.centroids.stride(0), N.ptr(self.c_sqnorm), N.stream(dev))
        self._bufs: dict = {}
        self._desc = N.TableLayer(
            dtype=N.dtype_tag(self.dtype), metric=_METRICS[metric], dim=self.dim, hidden=self.hidden,
            n_cent=self.n_cent, cents=N.ptr(self.centroids), ld_c=self.centroids.stride(0),
            c_sqnorm=N.ptr(self.c_sqnorm), values=N.ptr(self.values), ld_v=self.values.stride(0),
            proj_vis=N.ptr(self.proj_dev[0]), bias_vis=N.ptr(self.bias[0]), proj_txt=N.ptr(self.proj_dev[1]),
            bias_txt=N.ptr(self.bias[1]), ps_h=self.ps[0], ps_d=self.ps[1])

    # --------------------------------------------------------------- buffers
    def _out_buf(self, n, residual):
        """The pooled output buffer, or its twin when ``residual`` is the
        pooled buffer itself (chained calls: y = layer_forward(..., y))."""
        out = self._buf("out", (n, self.hidden), self.dtype)
        if residual is not None and residual.data_ptr() == out.data_ptr():
            out = self._buf("out_alt", (n, self.hidden), self.dtype)
        return out

    def _buf(self, name, shape, dtype):
        t = self._bufs.get(name)
        numel = 1
        for s in shape:
            numel *= s
        if t is None or t.dtype != dtype or t.numel() < numel:
            # zero-filled: the search workspace starts with counters that must be zero
            t = torch.zeros(max(numel, 1), dtype=dtype, device=self.device)
            self._bufs[name] = t
            # layer-call descriptions cached on the old buffers are stale now
            self.__dict__.pop("_io_cache", None)
        return t[:numel].view(shape)

    def _side_stream(self) -> torch.cuda.Stream:
        """The table's second stream on its device (default priority), made
        on first use."""
        s = getattr(self, "_side", None)
        if s is None:
            s = self._side = torch.cuda.Stream(self.device)
        return s

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
        nbytes = N.lib().tm_project_workspace_size(n, self.hidden, self.dim)
        ws = self._buf("project_ws", (max(nbytes, 1),), torch.uint8)
        N.call("tm_project", N.dtype_tag(self.dtype), N.ptr(x), n, self.hidden, x.stride(0), N.ptr(isv),
               N.ptr(self.proj_dev[0]), N.ptr(self.bias[0]), N.ptr(self.proj_dev[1]), N.ptr(self.bias[1]),
               self.ps[0], self.ps[1], self.dim, 0, 1e-6, N.ptr(q), q.stride(0), N.ptr(qn), N.ptr(ws), ws.numel(),
               N.stream(self.device))
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
            out = self._out_buf(n, residual)
        so = slot_out
        N.call("tm_gather_combine", N.dtype_tag(self.dtype), n, self.hidden, N.ptr(N.as_u8(keep)), N.ptr(so),
               so.stride(0), so.stride(1), N.ptr(weights), weights.stride(0), top_k, N.ptr(self.values),
               self.n_cent, self.values.stride(0), N.ptr(idx), N.ptr(dist), idx.stride(0), idx.shape[1],
               N.ptr(residual), 0 if residual is None else residual.stride(0), N.ptr(out), out.stride(0),
               N.stream(self.device))
        return out

    def gather_combine_ranked(self, slot_out, weights, idx, dist, n_keep: int, residual=None, out=None, keep=None):
        """gather_combine for a top-1 table whose keep set is decided in the
        same launch: token i is kept when fewer than n_keep tokens have a
        larger distance (ties -> lower index), as keep_select would choose.
        Returns (out, keep)."""
        N.require_hip(slot_out, weights, idx, dist)
        n, top_k = weights.shape
        if out is None:
            out = self._out_buf(n, residual)
        if keep is None:
            keep = self._buf("keep", (n,), torch.bool)
        d = dist.reshape(-1) if dist.dim() > 1 else dist
        if d.numel() != n or not d.is_contiguous():
            raise ValueError("gather_combine_ranked: dist must hold one contiguous distance per token")
        so = slot_out
        N.call("tm_gather_combine_ranked", N.dtype_tag(self.dtype), n, self.hidden, N.ptr(so), so.stride(0),
               so.stride(1), N.ptr(weights), weights.stride(0), top_k, N.ptr(self.values), self.n_cent,
               self.values.stride(0), N.ptr(idx), N.ptr(d), N.ptr(residual),
               0 if residual is None else residual.stride(0), N.ptr(out), out.stride(0), int(n_keep),
               N.ptr(N.as_u8(keep)), N.stream(self.device))
        return out, keep

    def route(self, router_logits: torch.Tensor, top_k: int):
        n, e = router_logits.shape
        w = self._buf("route_w", (n, top_k), torch.float32)
        ids = self._buf("route_ids", (n, top_k), torch.long)
        N.call("tm_topk_softmax", N.ptr(router_logits), n, e, router_logits.stride(0), int(top_k), 0, N.ptr(w),
               N.ptr(ids), N.stream(self.device))
        return w, ids

    def layer_forward_staged(self, hidden, is_vision, router_logits, slot_out, residual, router_top_k: int = 8,
                             n_nearest: int = 1, keep_rate: float = 0.6, out=None):
        """The layer as five separate C-ABI calls (one per stage)."""
        w, ids = self.route(router_logits, router_top_k)
        q, qn = self.project(hidden, is_vision)
        dist, idx = self.search(q, n_nearest, qn)
        keep = self.keep_select(dist[:, 0], self.keep_count(hidden.shape[0], keep_rate))
        y = self.gather_combine(keep, slot_out, w, idx, dist, residual, out)
        return {"weights": w, "ids": ids, "q": q, "qn": qn, "dist": dist, "idx": idx, "keep": keep, "out": y}

    def _layer_io(self, hidden, is_vision, router_logits, slot_out, residual, router_top_k, n_nearest, keep_rate,
                  out, flags=0):
        """The tm_layer_io of one layer call (buffers from this table's pool)
        and the dict of every stage's output it fills.  With
        TM_LAYER_NO_COMBINE, slot_out/residual/out are not used."""
        combine = not (flags & N.TM_LAYER_NO_COMBINE)
        N.require_hip(hidden, router_logits, *( (slot_out,) if combine else ()))
        if hidden.dtype != self.dtype or (combine and slot_out.dtype != self.dtype):
            raise RuntimeError(f"hidden/slot_out dtype must be the table dtype {self.dtype}")
        x = hidden if hidden.stride(-1) == 1 else hidden.contiguous()
        logits = router_logits.float()
        if logits.stride(-1) != 1:
            logits = logits.contiguous()
        if combine and slot_out.stride(-1) != 1:
            slot_out = slot_out.contiguous()
        n = x.shape[0]
        if combine and out is None:
            out = self._out_buf(n, residual)
        if not combine:
            slot_out = residual = out = None
        isv = None if is_vision is None else N.mask_bytes(is_vision, x.device)
        # the stage buffers and their pointers depend on (n, top_k, n_nearest)
        # only: built once per shape (a decode loop calls this per token) and
        # dropped whenever _buf reallocates a buffer
        cache = self.__dict__.setdefault("_io_cache", {})
        key = (n, router_top_k, n_nearest)
        entry = cache.get(key)
        if entry is None:
            stages = {
                "weights": self._buf("route_w", (n, router_top_k), torch.float32),
                "ids": self._buf("route_ids", (n, router_top_k), torch.long),
                "q": self._buf("q", (n, self.dim), self.dtype),
                "qn": self._buf("qn", (n,), torch.float32),
                "dist": self._buf("dist", (n, n_nearest), torch.float32),
                "idx": self._buf("idx", (n, n_nearest), torch.long),
                "keep": self._buf("keep", (n,), torch.bool),
            }
            io = N.LayerIO(
                n_tokens=n, router_top_k=router_top_k, n_nearest=n_nearest, weights=N.ptr(stages["weights"]),
                expert_ids=N.ptr(stages["ids"]), q=N.ptr(stages["q"]), q_sqnorm=N.ptr(stages["qn"]),
                dist=N.ptr(stages["dist"]), idx=N.ptr(stages["idx"]), keep=N.ptr(stages["keep"]))
            entry = (io, stages)
            cache = self.__dict__.setdefault("_io_cache", {})  # a _buf above may have dropped it
            cache[key] = entry
        io, stages = entry
        io.x, io.ld_x, io.is_vision = x.data_ptr(), x.stride(0), N.ptr(isv)
        io.router_logits, io.ld_logits, io.n_experts = logits.data_ptr(), logits.stride(0), logits.shape[1]
        io.keep_rate, io.flags = float(keep_rate), int(flags)
        io.slot_out = N.ptr(slot_out)
        io.so_b, io.so_s = (0, 0) if slot_out is None else (slot_out.stride(0), slot_out.stride(1))
        io.residual, io.ld_r = N.ptr(residual), 0 if residual is None else residual.stride(0)
        io.out, io.ld_o = N.ptr(out), 0 if out is None else out.stride(0)
        # the tensors the io points at stay referenced by the returned dict
        res = dict(stages)
        res["out"] = out
        res["_inputs"] = (x, logits, slot_out, isv)
        return io, res

    def _layer_ws(self, n, n_nearest):
        """The layer call's workspace (at least tm_table_forward_workspace_size
        bytes; the size is queried once per shape)."""
        sizes = self.__dict__.setdefault("_ws_sizes", {})
        nbytes = sizes.get((n, n_nearest))
        if nbytes is None:
            nbytes = sizes[(n, n_nearest)] = max(
                N.lib().tm_table_forward_workspace_size(C.byref(self._desc), n, n_nearest), 1)
        ws = self._bufs.get("layer_ws")
        if ws is None or ws.numel() < nbytes:
            ws = self._buf("layer_ws", (nbytes,), torch.uint8)
        return ws

    def layer_forward(self, hidden, is_vision, router_logits, slot_out, residual, router_top_k: int = 8,
                      n_nearest: int = 1, keep_rate: float = 0.6, out=None, stage_events=None):
        """One MoE layer of the table path in one C-ABI call (tm_table_forward);
        returns a dict of every stage's output.  ``stage_events``: optional six
        torch.cuda.Event recorded around the stages.  The returned tensors are
        this table's reusable buffers: the next call overwrites them (pass
        ``out`` to keep an output)."""
        io, res = self._layer_io(hidden, is_vision, router_logits, slot_out, residual, router_top_k, n_nearest,
                                 keep_rate, out)
        ws = self._layer_ws(io.n_tokens, n_nearest)
        evs = None
        if stage_events is not None:
            evs = (C.c_void_p * 6)(*[e.cuda_event for e in stage_events])
        N.check(N.lib().tm_table_forward(C.byref(self._desc), C.byref(io), N.ptr(ws), ws.numel(), evs,
                                         N.stream(self.device)), "tm_table_forward")
        if self.check_waits:
            self._raise_on_wait_errors()
        res.pop("_inputs")
        return res

    def _raise_on_wait_errors(self):
        if torch.cuda.is_current_stream_capturing():
            return  # nothing ran yet: read wait_errors() after the replays
        seen = getattr(self, "_wait_errors_seen", 0)
        now = self.wait_errors()
        self._wait_errors_seen = now
        if now != seen:
            # a late workgroup of the failed call may have left flags the next
            # call would take for its own: clear the sync region (the error
            # word with it) before the workspace is used again
            self._bufs["layer_ws"][:N.TM_LAYER_SYNC_BYTES].zero_()
            self._wait_errors_seen = 0
            raise RuntimeError(f"tm_table_forward: {now - seen} cross-workgroup wait(s) ran out; the call's outputs "
                               "are undefined (the launch's workgroups could not all be resident together); the "
                               "workspace's sync region was cleared")

    def wait_errors(self) -> int:
        """Bounded cross-workgroup waits of the one-launch decode plan that ran
        out on this table's workspace (zero unless the device was so busy that
        the launch's workgroups could not all be resident); synchronises."""
        ws = self._bufs.get("layer_ws")
        if ws is None or ws.numel() < N.TM_LAYER_SYNC_BYTES:
            return 0
        e = N.TM_LAYER_SYNC_ERR_BYTE
        return int(ws[e:e + 4].view(torch.int32).item())

    def layer_search(self, hidden, is_vision, router_logits, router_top_k: int = 8, n_nearest: int = 1,
                     keep_rate: float = 0.6):
        """The layer call up to the keep set (tm_table_forward with
        TM_LAYER_NO_COMBINE): router, projection, nearest centroids and the
        tokens to recompute, for callers that recompute the kept tokens before
        combining (layer_forward_recompute)."""
        io, res = self._layer_io(hidden, is_vision, router_logits, None, None, router_top_k, n_nearest, keep_rate,
                                 None, flags=N.TM_LAYER_NO_COMBINE)
        ws = self._layer_ws(io.n_tokens, n_nearest)
        N.check(N.lib().tm_table_forward(C.byref(self._desc), C.byref(io), N.ptr(ws), ws.numel(), None,
                                         N.stream(self.device)), "tm_table_forward")
        if self.check_waits:
            self._raise_on_wait_errors()
        res.pop("_inputs")
        del res["out"]
        return res

    def layer_forward_recompute(self, hidden, is_vision, router_logits, experts, residual, router_top_k: int = 6,
                                keep_rate: float = 0.6, shared=None, out=None):
        """A DeepSeek-style MoE layer on the table (models/deepseek_vl2/
        deepseek_layers.py:569-745 shape): the layer call up to the keep set,
        the kept tokens' routed slots recomputed by ``experts``
        (GroupedExperts, on the device, no host sync), the shared experts
        ``shared`` = (w1, w3, w2) or a ``SharedExperts`` (packed weights, same
        bits) run over every token with the residual folded into their down
        projection (dtype(residual + shared)), then the
        gather + combine on top: out = dtype(dtype(residual + shared) + y),
        y = the renormalised routed slots (kept tokens) or the cached output
        of the nearest centroid (the others).  Top-1 table.  Returns the
        stage outputs and ``slot_out``; buffers are reused by the next call.

        The shared experts depend on neither the search nor the routed
        recompute, so they run on a second stream of the device (default
        priority), forked from the caller's stream before the search and
        joined before the combine: their workgroups fill the CUs that the
        single-workgroup launches (keep select, slot grouping) and the last
        partial rounds of the routed GEMMs leave idle.  The fork and join are
        stream waits, so the call stays capturable in a HIP graph."""
        from ..ops import SharedExperts, expert_swiglu

        n = hidden.shape[0]
        main = torch.cuda.current_stream(self.device)
        side = None
        base = residual
        if shared is not None:
            # allocated on the caller's stream, which waits for the side
            # stream at the join, before any later call can free them
            base = self._buf("shared_plus_residual", (n, self.hidden), self.dtype)
            if isinstance(shared, SharedExperts):
                nbytes = N.lib().tm_grouped_swiglu_packed_workspace_size(n, shared.inter, 1, N.dtype_tag(self.dtype))
                if shared._ws is None or shared._ws.numel() < nbytes:
                    shared._ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=self.device)
                run = lambda: shared.forward(hidden, out=base, addend=residual)  # noqa: E731
            else:
                w1, w3, w2 = shared
                nbytes = N.lib().tm_swiglu_workspace_size(n, w1.shape[0], N.dtype_tag(self.dtype))
                ws = self._buf("shared_ws", (max(nbytes, 1),), torch.uint8)
                run = lambda: expert_swiglu(hidden, w1, w3, w2, out=base, workspace=ws, addend=residual)  # noqa: E731
            side = self._side_stream()
            side.wait_stream(main)
            with torch.cuda.stream(side):
                run()
        res = self.layer_search(hidden, is_vision, router_logits, router_top_k, 1, keep_rate)
        slot_out = self._buf("recompute_slots", (n, router_top_k, self.hidden), self.dtype)
        experts.forward(hidden, res["ids"], res["keep"], slot_out)
        if side is not None:
            main.wait_stream(side)
        out = self.gather_combine(res["keep"], slot_out, res["weights"], res["idx"], res["dist"], base, out)
        res["slot_out"] = slot_out
        res["out"] = out
        return res

    def layer_forward_noalloc(self, hidden, is_vision, router_logits, slot_out, residual, router_top_k: int = 8,
                              n_nearest: int = 1, keep_rate: float = 0.6, out=None):
        """layer_forward through tm_table_forward_noalloc: the library's static
        scratch instead of a workspace (at most TM_NOALLOC_SCRATCH_BYTES; calls
        overlapping on one GPU race for it).  It takes no plan whose
        workgroups wait for each other, so there is no error word to check."""
        io, res = self._layer_io(hidden, is_vision, router_logits, slot_out, residual, router_top_k, n_nearest,
                                 keep_rate, out)
        N.check(N.lib().tm_table_forward_noalloc(C.byref(self._desc), C.byref(io), N.stream(self.device)),
                "tm_table_forward_noalloc")
        res.pop("_inputs")
        return res
