"""Seeded synthetic workloads of the north-star configurations.

There are no real tables or checkpoints offline, so the global-table
workloads are drawn as follows (CPU torch.Generator, fp32 draws rounded to the
table dtype, then moved to the requested device):

* PCA matrix P_m [H, d]: Q factor of the QR decomposition of a Gaussian
  matrix, one per modality; bias 0 (``bias_scale`` > 0 draws a nonzero bias).
* centroids mu_c ~ N(0, I_d); cached outputs V, router logits, recomputed slot
  outputs E and residual R ~ N(0, 1).
* "near" tokens: x = P_m (mu_c + sigma_w eps) + 0.05 (I - P_m P_m^T) g;
  outliers: x ~ U(-sqrt(3), sqrt(3))^H.

``gen_device`` (e.g. "cuda") draws the large tensors (hidden states, cached
outputs, router logits, slot outputs, residual) with a generator on that
device instead: the same distributions, other random streams, and seconds
instead of minutes for the 48-layer stack.

Configs:
  1  CPU reference: N=256, H=2048, d=64, C=1024, fp32, top-1, 100 % near
  2  Qwen3-VL-30B-A3B prefill: N=4096 (3584 vision + 512 text), H=2048, d=128,
     C=8192, 128 experts top-8, 70 % near / 30 % outliers, bf16
  3  decode: N in {1, 8, 32} text tokens, C=16384, d=128, H=2048, top-4 blend
  4  one layer of the 48-layer stack: N=2048, C=8192, d=128, H=2048
  5  DeepSeek-VL2-style: H=2560, 64 experts top-6, N=4096, C=8192, d=128
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch

CONFIGS = {
    1: dict(n=256, hidden=2048, dim=64, n_cent=1024, n_experts=128, router_top_k=8, n_nearest=1,
            keep_rate=0.6, near_frac=1.0, n_vision=256, dtype=torch.float32, seed=1),
    2: dict(n=4096, hidden=2048, dim=128, n_cent=8192, n_experts=128, router_top_k=8, n_nearest=1,
            keep_rate=0.6, near_frac=0.7, n_vision=3584, dtype=torch.bfloat16, seed=2),
    3: dict(n=32, hidden=2048, dim=128, n_cent=16384, n_experts=128, router_top_k=8, n_nearest=4,
            keep_rate=0.6, near_frac=0.7, n_vision=0, dtype=torch.bfloat16, seed=3),
    4: dict(n=2048, hidden=2048, dim=128, n_cent=8192, n_experts=128, router_top_k=8, n_nearest=1,
            keep_rate=0.6, near_frac=0.7, n_vision=1792, dtype=torch.bfloat16, seed=40),
    5: dict(n=4096, hidden=2560, dim=128, n_cent=8192, n_experts=64, router_top_k=6, n_nearest=1,
            keep_rate=0.6, near_frac=0.7, n_vision=3584, dtype=torch.bfloat16, seed=5),
}


@dataclass
class Workload:
    cfg: dict
    x: torch.Tensor            # [N, H]
    is_vision: torch.Tensor    # [N] bool
    proj_vis: torch.Tensor     # [H, d]
    bias_vis: torch.Tensor     # [d]
    proj_txt: torch.Tensor
    bias_txt: torch.Tensor
    centroids: torch.Tensor    # [C, d]
    values: torch.Tensor       # [C, H]
    logits: torch.Tensor       # [N, E] fp32
    slot_out: torch.Tensor     # [N, k, H]
    residual: torch.Tensor     # [N, H]
    cluster_of: torch.Tensor   # [N] int64, -1 for outliers

    def to(self, device) -> "Workload":
        kw = {k: (v.to(device) if isinstance(v, torch.Tensor) else v) for k, v in self.__dict__.items()}
        return Workload(**kw)


def _orthonormal(gen, hidden, dim):
    a = torch.randn(hidden, dim, generator=gen, dtype=torch.float64)
    q, r = torch.linalg.qr(a)
    q = q * torch.sign(torch.diagonal(r)).unsqueeze(0)
    return q.float()


def make_workload(config: int = 2, *, n: int | None = None, seed: int | None = None,
                  dtype: torch.dtype | None = None, device="cpu", bias_scale: float = 0.0,
                  sigma_w: float = 0.2, with_slot_out: bool = True, gen_device=None, **overrides) -> Workload:
    cfg = dict(CONFIGS[config])
    cfg.update(overrides)
    if n is not None:
        if "n_vision" not in overrides:  # keep the vision share of the config
            cfg["n_vision"] = int(round(n * CONFIGS[config]["n_vision"] / CONFIGS[config]["n"]))
        cfg["n"] = n
    if dtype is not None:
        cfg["dtype"] = dtype
    if seed is not None:
        cfg["seed"] = seed
    N, H, d, C = cfg["n"], cfg["hidden"], cfg["dim"], cfg["n_cent"]
    E, k, dt = cfg["n_experts"], cfg["router_top_k"], cfg["dtype"]
    gen = torch.Generator().manual_seed(int(cfg["seed"]))

    pv = _orthonormal(gen, H, d)
    pt = _orthonormal(gen, H, d)
    bv = torch.randn(d, generator=gen) * bias_scale
    bt = torch.randn(d, generator=gen) * bias_scale
    mu = torch.randn(C, d, generator=gen)
    is_vision = torch.zeros(N, dtype=torch.bool)
    is_vision[: cfg["n_vision"]] = True

    n_near = int(round(cfg["near_frac"] * N))
    perm = torch.randperm(N, generator=gen)
    near_rows = perm[:n_near]
    cluster_of = torch.full((N,), -1, dtype=torch.long)
    cluster_of[near_rows] = torch.randint(0, C, (n_near,), generator=gen)

    if gen_device is None:
        gd, g2 = torch.device("cpu"), gen
    else:
        gd = torch.device(gen_device)
        g2 = torch.Generator(device=gd).manual_seed(int(cfg["seed"]))
    rnd = lambda *shape: torch.randn(*shape, generator=g2, device=gd)  # noqa: E731
    x = (torch.rand(N, H, generator=g2, device=gd) * 2.0 - 1.0) * math.sqrt(3.0)
    if n_near:
        c = cluster_of[near_rows].to(gd)
        z = mu.to(gd)[c] + sigma_w * rnd(n_near, d)
        g = rnd(n_near, H)
        vis = is_vision[near_rows].to(gd)
        xn = torch.empty(n_near, H, device=gd)
        for sel, P, b in ((vis, pv.to(gd), bv.to(gd)), (~vis, pt.to(gd), bt.to(gd))):
            if sel.any():
                # x = P (z - b) + 0.05 (I - P P^T) g, so that x @ P + b = z
                gs = g[sel]
                xn[sel] = (z[sel] - b) @ P.T + 0.05 * (gs - (gs @ P) @ P.T)
        x[near_rows.to(gd)] = xn

    values = rnd(C, H)
    logits = rnd(N, E)
    slot_out = rnd(N, k, H) if with_slot_out else torch.empty(0, device=gd)
    residual = rnd(N, H)

    def cvt(t):
        return t.to(dt).to(device)

    return Workload(
        cfg=cfg, x=cvt(x), is_vision=is_vision.to(device), proj_vis=cvt(pv), bias_vis=cvt(bv),
        proj_txt=cvt(pt), bias_txt=cvt(bt), centroids=cvt(mu), values=cvt(values),
        logits=logits.to(device), slot_out=cvt(slot_out), residual=cvt(residual), cluster_of=cluster_of.to(device),
    )


def make_stack(n_layers: int = 48, *, n: int | None = None, device="cuda", gen_device="cuda",
               **overrides) -> list[Workload]:
    """Config 4: ``n_layers`` independent layers (seed 40 + l), each with its
    own table (C=8192, d=128, cached outputs 8192x2048 bf16), hidden states,
    router logits, slot outputs and residual, drawn on ``gen_device``."""
    return [make_workload(4, n=n, seed=CONFIGS[4]["seed"] + l, device=device, gen_device=gen_device, **overrides)
            for l in range(n_layers)]


def make_mode_r_manager(dev, E=128, H=2048, d=64, K=256, seed=7):
    """A HybridStorageManager of the reference's default shape (128 experts x
    2 modalities x 256 centroids in 64-d, hidden 2048) filled on the device:
    random keys (normalised copy as the loader makes it), cached outputs, PCA
    pairs, a full 64-entry online window."""
    from table_moe.cache_engine import CacheConfig, HybridStorageManager
    from table_moe.cache_engine.table_file import normalize_last_dim

    saved = {k: getattr(CacheConfig, k) for k in ("FIXED_K", "COMPRESSED_DIM", "MODEL_DTYPE", "ONLINE_CACHE_SIZE",
                                                  "ONLINE_TOP_K")}
    CacheConfig.FIXED_K, CacheConfig.COMPRESSED_DIM, CacheConfig.MODEL_DTYPE = K, d, torch.bfloat16
    CacheConfig.ONLINE_CACHE_SIZE, CacheConfig.ONLINE_TOP_K = 64, 8
    try:
        mgr = HybridStorageManager(2, E, H, dev)
    finally:
        for k_, v in saved.items():
            setattr(CacheConfig, k_, v)
    g = torch.Generator(device=dev).manual_seed(seed)
    raw = torch.randn(E, 2, K, d, generator=g, device=dev)
    mgr.raw_keys_buffer.copy_(raw.to(torch.bfloat16))
    mgr.keys_buffer.copy_(normalize_last_dim(raw, 1e-6).to(torch.bfloat16))
    mgr.values_buffer.copy_(torch.randn(E, 2, K, H, generator=g, device=dev).to(torch.bfloat16))
    for mod in ("vision", "text"):
        p = torch.linalg.qr(torch.randn(H, d, generator=g, device=dev, dtype=torch.float32))[0]
        mgr.pca[mod] = {"proj": p.to(torch.bfloat16), "bias": (torch.randn(d, generator=g, device=dev) * 0.05)
                        .to(torch.bfloat16)}
    hist = torch.randn(64, H, generator=g, device=dev).to(torch.bfloat16)
    ids = torch.stack([torch.randperm(E, device=dev)[:8] for _ in range(64)])
    mgr.update_online_cache(hist, ids, torch.randn(64, 8, H, generator=g, device=dev).to(torch.bfloat16))
    return mgr
