"""Packed on-disk table format: one file per layer instead of 2 + 2E ``.pt`` files.

The reference keeps a layer's offline table as separate torch pickles:
``L{l}_{modality}_pca.pt`` ({"mean", "proj"}, offline_table/step2_pca_cluster.py:234-237)
and ``L{l}_E{e}_{modality}_cache.pt`` ({"id", "key", "value"},
offline_table/step3_offline_cache_builder.py:145-151), which
``HybridStorageManager`` loads one by one (table_moe/cache_engine/manager.py:157-210):
unpickle, normalise the keys, copy each slice to its place.

A packed file holds the same layer already in the layout the device buffers
use, so loading is a handful of bulk copies from a memory map:

    bytes 0..7    magic b"TMTABLE1"
    bytes 8..15   little-endian uint64: length L of the JSON header
    bytes 16..    UTF-8 JSON header (format version, layer, shapes, model dtype,
                  which (expert, modality) tables and PCA models are present,
                  and for every section its offset, shape and element type)
    sections      at 4096-byte aligned offsets, C order, little-endian:
      count       int32  [E, 2]        rows installed per (expert, modality) table
      keys        model dtype [E, 2, K, d]  raw keys (rows past `count` are zero)
      keys_norm   model dtype [E, 2, K, d]  keys normalised as the loader does
                  (manager.py:24-31: fp32 norm and quotient, rows with norm <= eps -> 0)
      values      model dtype [E, 2, K, H]  cached expert outputs
      pca_mean_{vision,text}, pca_proj_{vision,text}
                  the step-2 PCA tensors as saved (their own dtype); the bias
                  -mean @ proj is computed at load on the load device exactly as
                  the .pt path does, so both paths give the same bits.

bf16 sections are stored as their raw 16-bit patterns.  The header is plain
JSON and the sections plain arrays: nothing in the file is executed when it
is read.  ``pack_layer`` converts a reference layer directory (the same file
names, parse rules and skip rules as the .pt loader, so both give the same
buffers, tested bit for bit); ``load_layer`` maps a file and copies its
sections to a device.
"""

from __future__ import annotations

import glob
import json
import os
import struct
import time

import numpy as np
import torch

from .config import CacheConfig

MAGIC = b"TMTABLE1"
VERSION = 1
ALIGN = 4096

_TORCH_TO_NAME = {torch.float32: "float32", torch.float16: "float16", torch.bfloat16: "bfloat16",
                  torch.int32: "int32", torch.uint8: "uint8"}
_NAME_TO_TORCH = {v: k for k, v in _TORCH_TO_NAME.items()}
# element type on disk: bf16 travels as its 16-bit pattern
_NAME_TO_NP = {"float32": np.float32, "float16": np.float16, "bfloat16": np.uint16, "int32": np.int32,
               "uint8": np.uint8}


def _to_numpy(t: torch.Tensor) -> np.ndarray:
    t = t.detach().contiguous().cpu()
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).numpy().view(np.uint16)
    return t.numpy()


def packed_path(layer_idx: int, cache_dir: str | None = None) -> str:
    """Where the loader looks for a layer's packed file."""
    return os.path.join(cache_dir or CacheConfig.CACHE_DIR, f"layer_{layer_idx}.tmtable")


def parse_cache_name(fname: str):
    """``L{layer}_E{expert}_{modality}_cache.pt`` -> (expert, modality name)."""
    parts = fname.replace(".pt", "").split("_")
    return int(parts[1][1:]), parts[2]


def normalize_last_dim(x: torch.Tensor, eps: float) -> torch.Tensor:
    """Key normalisation at load: fp32 norm and division, rounded back to the
    keys' dtype; rows with norm <= eps become 0 (manager.py:24-31)."""
    x32 = x.float()
    norm = torch.linalg.vector_norm(x32, dim=-1, keepdim=True)
    out = x32 / norm.clamp_min(eps)
    out = torch.where(norm <= eps, torch.zeros_like(out), out)
    return out.to(dtype=x.dtype)


def collect_layer(layer_idx: int, num_experts: int, hidden_dim: int, cache_dir: str | None = None,
                  pca_dir: str | None = None, dtype: torch.dtype | None = None) -> dict:
    """Read a reference layer directory into host tensors in the device layout
    (the .pt loader's rules: unknown modalities, expert ids past num_experts and
    unreadable files are skipped, the latter with a message)."""
    cache_dir = cache_dir or CacheConfig.CACHE_DIR
    pca_dir = pca_dir or CacheConfig.PCA_DIR
    dtype = dtype or CacheConfig.MODEL_DTYPE
    K, d = int(CacheConfig.FIXED_K), int(CacheConfig.COMPRESSED_DIM)
    eps = float(CacheConfig.OFFLINE_COSINE_EPS)
    count = torch.zeros((num_experts, 2), dtype=torch.int32)
    keys = torch.zeros((num_experts, 2, K, d), dtype=dtype)
    keys_norm = torch.zeros_like(keys)
    values = torch.zeros((num_experts, 2, K, hidden_dim), dtype=dtype)
    layer_dir = os.path.join(cache_dir, f"layer_{layer_idx}")
    for path in sorted(glob.glob(os.path.join(layer_dir, "*_cache.pt"))):
        try:
            eid, mod = parse_cache_name(os.path.basename(path))
            mid = CacheConfig.MODALITY_MAP.get(mod, -1)
            if mid == -1 or eid >= num_experts:
                continue
            data = torch.load(path, map_location="cpu", weights_only=True)
            key, value = data["key"], data["value"]  # both present before anything is written
            k_t = key.to(dtype=dtype)
            k = k_t.shape[0]
            keys[eid, mid, :k] = k_t
            keys_norm[eid, mid, :k] = normalize_last_dim(k_t, eps)
            values[eid, mid, :k] = value.to(dtype=dtype)
            count[eid, mid] = max(int(count[eid, mid]), k)
        except Exception as exc:  # a bad file is reported and skipped, as the reference does
            print(f"Error loading {path}: {exc}")
    pca = {}
    for mod in ("vision", "text"):
        path = os.path.join(pca_dir, f"layer_{layer_idx}", f"L{layer_idx}_{mod}_pca.pt")
        if os.path.exists(path):
            data = torch.load(path, map_location="cpu", weights_only=True)
            pca[mod] = {"mean": data["mean"], "proj": data["proj"]}
    return {"layer": layer_idx, "count": count, "keys": keys, "keys_norm": keys_norm, "values": values, "pca": pca,
            "dtype": dtype}


def write_layer(path: str, tables: dict) -> int:
    """Write collected tables (``collect_layer``'s result) as a packed file;
    returns the file size in bytes."""
    arrays = {"count": tables["count"], "keys": tables["keys"], "keys_norm": tables["keys_norm"],
              "values": tables["values"]}
    for mod, p in tables["pca"].items():
        arrays[f"pca_mean_{mod}"] = p["mean"]
        arrays[f"pca_proj_{mod}"] = p["proj"]
    E, _, K, d = tables["keys"].shape
    H = tables["values"].shape[-1]
    sections = {}
    off = 0
    for name, t in arrays.items():
        nbytes = t.numel() * t.element_size()
        sections[name] = {"offset": off, "shape": list(t.shape), "dtype": _TORCH_TO_NAME[t.dtype], "nbytes": nbytes}
        off += (nbytes + ALIGN - 1) // ALIGN * ALIGN
    header = {"format": "tablemoe-table", "version": VERSION, "layer": int(tables["layer"]), "num_experts": int(E),
              "fixed_k": int(K), "dim": int(d), "hidden": int(H), "dtype": _TORCH_TO_NAME[tables["dtype"]],
              "modalities": ["vision", "text"], "pca": sorted(tables["pca"].keys()), "sections": sections}
    hb = json.dumps(header, sort_keys=True).encode("utf-8")
    base = (16 + len(hb) + ALIGN - 1) // ALIGN * ALIGN
    tmp = path + ".tmp"
    with open(tmp, "wb") as f:
        f.write(MAGIC)
        f.write(struct.pack("<Q", len(hb)))
        f.write(hb)
        for name, t in arrays.items():
            f.seek(base + sections[name]["offset"])
            f.write(_to_numpy(t).tobytes(order="C"))
        f.truncate(base + off)
    os.replace(tmp, path)
    return base + off


def pack_layer(layer_idx: int, num_experts: int, hidden_dim: int, out_path: str | None = None,
               cache_dir: str | None = None, pca_dir: str | None = None, dtype: torch.dtype | None = None) -> str:
    """Convert one reference layer (PCA + per-table .pt files) into a packed file."""
    out_path = out_path or packed_path(layer_idx, cache_dir)
    write_layer(out_path, collect_layer(layer_idx, num_experts, hidden_dim, cache_dir, pca_dir, dtype))
    return out_path


def read_header(path: str) -> tuple[dict, int]:
    """The JSON header and the byte offset of the first section."""
    with open(path, "rb") as f:
        magic = f.read(8)
        if magic != MAGIC:
            raise ValueError(f"{path}: not a packed table file (magic {magic!r})")
        (hl,) = struct.unpack("<Q", f.read(8))
        if hl > (1 << 24):
            raise ValueError(f"{path}: header length {hl} out of range")
        header = json.loads(f.read(hl).decode("utf-8"))
    if header.get("format") != "tablemoe-table" or header.get("version") != VERSION:
        raise ValueError(f"{path}: unsupported packed table version {header.get('version')!r}")
    base = (16 + hl + ALIGN - 1) // ALIGN * ALIGN
    size = os.path.getsize(path)
    for name, s in header["sections"].items():
        if s["dtype"] not in _NAME_TO_NP:
            raise ValueError(f"{path}: section {name} has unknown type {s['dtype']!r}")
        n = int(np.prod(s["shape"], dtype=np.int64)) * np.dtype(_NAME_TO_NP[s["dtype"]]).itemsize
        if n != s["nbytes"] or base + s["offset"] + n > size:
            raise ValueError(f"{path}: section {name} does not fit the file")
    return header, base


def load_layer(path: str, device="cpu", expect: dict | None = None) -> dict:
    """Map a packed file and copy its sections to `device`.  `expect` (optional):
    header fields that must match (e.g. num_experts, hidden, fixed_k, dim, dtype)."""
    header, base = read_header(path)
    for k, v in (expect or {}).items():
        if header.get(k) != v:
            raise ValueError(f"{path}: {k} is {header.get(k)!r}, expected {v!r}")
    out = {"header": header}
    device = torch.device(device)
    for name, s in header["sections"].items():
        arr = np.memmap(path, dtype=_NAME_TO_NP[s["dtype"]], mode="c", offset=base + s["offset"],
                        shape=tuple(s["shape"]))
        t = torch.from_numpy(arr)
        if s["dtype"] == "bfloat16":
            t = t.view(torch.bfloat16)
        out[name] = t.to(device) if device.type != "cpu" else t.clone()
        del arr
    return out


def _bench(args):  # load-time comparison on a synthetic layer of the reference's default size
    import tempfile

    from .config import update_active_cache_config
    from .manager import HybridStorageManager

    E, K, d, H = args.experts, 256, 64, args.hidden
    root = tempfile.mkdtemp(prefix="tmtable_", dir=args.dir)
    cache_dir, pca_dir = os.path.join(root, "cache"), os.path.join(root, "pca")
    os.makedirs(os.path.join(cache_dir, "layer_0"))
    os.makedirs(os.path.join(pca_dir, "layer_0"))
    g = torch.Generator().manual_seed(0)
    for mod in ("vision", "text"):
        torch.save({"mean": torch.randn(H, generator=g).half(), "proj": torch.randn(H, d, generator=g).half()},
                   os.path.join(pca_dir, "layer_0", f"L0_{mod}_pca.pt"))
        for e in range(E):
            torch.save({"id": torch.arange(K, dtype=torch.int32), "key": torch.randn(K, d, generator=g).bfloat16(),
                        "value": torch.randn(K, H, generator=g).bfloat16()},
                       os.path.join(cache_dir, "layer_0", f"L0_E{e}_{mod}_cache.pt"))
    update_active_cache_config(CACHE_DIR=cache_dir, PCA_DIR=pca_dir, FIXED_K=K, COMPRESSED_DIM=d,
                               MODEL_DTYPE=torch.bfloat16)
    dev = args.device
    nbytes = 0
    t_pt = []
    for _ in range(args.reps):
        torch.cuda.synchronize() if dev.startswith("cuda") else None
        t0 = time.perf_counter()
        m = HybridStorageManager(0, E, H, device=dev, use_packed=False)
        torch.cuda.synchronize() if dev.startswith("cuda") else None
        t_pt.append(time.perf_counter() - t0)
        nbytes = m.values_buffer.numel() * 2 + m.keys_buffer.numel() * 4
        del m
    path = pack_layer(0, E, H)
    t_pk = []
    for _ in range(args.reps):
        torch.cuda.synchronize() if dev.startswith("cuda") else None
        t0 = time.perf_counter()
        m = HybridStorageManager(0, E, H, device=dev)
        torch.cuda.synchronize() if dev.startswith("cuda") else None
        t_pk.append(time.perf_counter() - t0)
        del m
    import shutil

    file_bytes = os.path.getsize(path)
    shutil.rmtree(root, ignore_errors=True)
    a, b = min(t_pt), min(t_pk)
    print(json.dumps({"experts": E, "fixed_k": K, "dim": d, "hidden": H, "device": dev,
                      "table_bytes": nbytes, "file_bytes": file_bytes, "reps": args.reps,
                      "pt_files_s": round(a, 4), "packed_s": round(b, 4), "speedup": round(a / b, 2),
                      "packed_GBps": round(nbytes / b / 1e9, 2), "page_cache": "warm (files just written)"}))


if __name__ == "__main__":
    import argparse

    ap = argparse.ArgumentParser(description="packed table files: convert a reference layer, or time loading")
    sub = ap.add_subparsers(dest="cmd", required=True)
    pk = sub.add_parser("pack", help="convert one reference layer directory")
    pk.add_argument("--layer", type=int, required=True)
    pk.add_argument("--num-experts", type=int, required=True)
    pk.add_argument("--hidden", type=int, required=True)
    pk.add_argument("--cache-dir")
    pk.add_argument("--pca-dir")
    pk.add_argument("--out")
    bn = sub.add_parser("bench", help="time .pt-directory vs packed loading of a synthetic layer")
    bn.add_argument("--experts", type=int, default=128)
    bn.add_argument("--hidden", type=int, default=2048)
    bn.add_argument("--device", default="cuda:0")
    bn.add_argument("--reps", type=int, default=3)
    bn.add_argument("--dir", default=None)
    a = ap.parse_args()
    if a.cmd == "pack":
        print(pack_layer(a.layer, a.num_experts, a.hidden, a.out, a.cache_dir, a.pca_dir))
    else:
        _bench(a)
