"""Packed table files (table_moe/cache_engine/table_file.py): a layer converted
from the reference's on-disk layout (PCA + per-(expert, modality) .pt files,
offline_table/step2_pca_cluster.py:234-237, step3_offline_cache_builder.py:145-151)
loads into the same HybridStorageManager buffers, bit for bit, as the .pt
loader (manager.py:157-210) produces from the same directory."""

import json
import os
import struct

import numpy as np
import pytest
import torch

from table_moe.cache_engine import HybridStorageManager, update_active_cache_config
from table_moe.cache_engine import table_file as TF
from table_moe.cache_engine.config import get_active_cache_config, set_active_cache_config

E, K, D, H, LAYER = 6, 16, 8, 40, 3


@pytest.fixture
def ref_dirs(tmp_path):
    """A reference-format layer directory with the cases the loader must handle:
    tables shorter than FIXED_K, a missing (expert, modality), an expert id
    past num_experts, an unknown modality, an unreadable file, keys in another
    dtype than the model's, an all-zero key row (normalises to zero)."""
    saved = get_active_cache_config()
    cache_dir, pca_dir = tmp_path / "cache", tmp_path / "pca"
    (cache_dir / f"layer_{LAYER}").mkdir(parents=True)
    (pca_dir / f"layer_{LAYER}").mkdir(parents=True)
    g = torch.Generator().manual_seed(7)
    torch.save({"mean": torch.randn(H, generator=g).half(), "proj": torch.randn(H, D, generator=g).half()},
               pca_dir / f"layer_{LAYER}" / f"L{LAYER}_vision_pca.pt")  # no text PCA: zero projection
    ld = cache_dir / f"layer_{LAYER}"
    for e in range(E):
        for mod in ("vision", "text"):
            if (e, mod) == (2, "text"):
                continue
            k = K if e % 2 == 0 else K - 5
            key = torch.randn(k, D, generator=g)
            if e == 3:
                key[1] = 0.0
            key = key.half() if e == 4 else key.bfloat16()
            torch.save({"id": torch.arange(k, dtype=torch.int32), "key": key,
                        "value": torch.randn(k, H, generator=g).bfloat16()}, ld / f"L{LAYER}_E{e}_{mod}_cache.pt")
    torch.save({"key": torch.randn(K, D), "value": torch.randn(K, H)}, ld / f"L{LAYER}_E{E + 1}_vision_cache.pt")
    torch.save({"key": torch.randn(K, D), "value": torch.randn(K, H)}, ld / f"L{LAYER}_E0_audio_cache.pt")
    (ld / f"L{LAYER}_E5_vision_cache.pt").write_bytes(b"not a torch file")  # replaces a good one
    update_active_cache_config(CACHE_DIR=str(cache_dir), PCA_DIR=str(pca_dir), FIXED_K=K, COMPRESSED_DIM=D,
                               MODEL_DTYPE=torch.bfloat16)
    yield cache_dir, pca_dir
    set_active_cache_config(saved)


def _same(a: torch.Tensor, b: torch.Tensor) -> bool:
    return a.dtype == b.dtype and a.shape == b.shape and torch.equal(a.view(torch.int16) if a.dtype == torch.bfloat16
                                                                     else a, b.view(torch.int16)
                                                                     if b.dtype == torch.bfloat16 else b)


def test_packed_layer_loads_same_buffers_as_pt_files(ref_dirs, capsys):
    ref = HybridStorageManager(LAYER, E, H, device="cpu", use_packed=False)
    path = TF.pack_layer(LAYER, E, H)
    assert path == TF.packed_path(LAYER) and os.path.exists(path)
    out = capsys.readouterr().out
    assert "Error loading" in out and "E5_vision" in out  # the unreadable file is reported, not fatal
    got = HybridStorageManager(LAYER, E, H, device="cpu")  # picks the packed file
    for name in ("raw_keys_buffer", "keys_buffer", "values_buffer"):
        assert _same(getattr(ref, name), getattr(got, name)), name
    for mod in ("vision", "text"):
        for part in ("proj", "bias"):
            assert _same(ref.pca[mod][part], got.pca[mod][part]), (mod, part)
    # what the directory held, independently of both loaders
    assert torch.count_nonzero(got.values_buffer[2, 1]) == 0  # missing (expert, modality)
    assert torch.count_nonzero(got.values_buffer[5, 0]) == 0  # unreadable file
    assert torch.count_nonzero(got.raw_keys_buffer[1, 0, K - 5:]) == 0  # short table: rows past k stay zero
    assert torch.count_nonzero(got.keys_buffer[3, 0, 1]) == 0  # zero key row normalises to zero
    n = got.keys_buffer[0, 0].float().norm(dim=-1)
    assert torch.allclose(n, torch.ones_like(n), atol=1e-2)
    assert torch.count_nonzero(got.pca["text"]["proj"]) == 0


def test_packed_header_and_sections(ref_dirs):
    path = TF.pack_layer(LAYER, E, H)
    header, base = TF.read_header(path)
    assert base % TF.ALIGN == 0
    assert (header["num_experts"], header["fixed_k"], header["dim"], header["hidden"], header["layer"]) == (E, K, D, H,
                                                                                                            LAYER)
    assert header["dtype"] == "bfloat16" and header["pca"] == ["vision"]
    secs = header["sections"]
    assert secs["values"]["shape"] == [E, 2, K, H] and secs["keys"]["shape"] == [E, 2, K, D]
    for s in secs.values():
        assert s["offset"] % TF.ALIGN == 0
    data = TF.load_layer(path)
    count = data["count"].numpy()
    assert count[2, 1] == 0 and count[5, 0] == 0 and count[1, 0] == K - 5 and count[0, 0] == K
    # a section read straight from the file bytes equals the loaded tensor
    with open(path, "rb") as f:
        f.seek(base + secs["values"]["offset"])
        raw = np.frombuffer(f.read(secs["values"]["nbytes"]), dtype=np.uint16).reshape(E, 2, K, H)
    assert np.array_equal(raw, data["values"].view(torch.int16).numpy().view(np.uint16))


def test_packed_file_rejects_mismatch_and_corruption(ref_dirs, tmp_path):
    path = TF.pack_layer(LAYER, E, H)
    with pytest.raises(ValueError, match="num_experts"):
        HybridStorageManager(LAYER, E + 1, H, device="cpu")
    with pytest.raises(ValueError, match="hidden"):
        HybridStorageManager(LAYER, E, H + 8, device="cpu")
    bad = tmp_path / "bad.tmtable"
    bad.write_bytes(b"NOTTABLE" + bytes(64))
    with pytest.raises(ValueError, match="magic"):
        TF.read_header(str(bad))
    # a truncated file: the sections no longer fit
    blob = open(path, "rb").read()
    short = tmp_path / "short.tmtable"
    short.write_bytes(blob[: len(blob) - 4096])
    with pytest.raises(ValueError, match="does not fit"):
        TF.read_header(str(short))
    # a header naming an element type that is not a plain array
    (hl,) = struct.unpack("<Q", blob[8:16])
    hdr = json.loads(blob[16:16 + hl])
    hdr["sections"]["keys"]["dtype"] = "object"
    hb = json.dumps(hdr).encode()
    odd = tmp_path / "odd.tmtable"
    odd.write_bytes(b"TMTABLE1" + struct.pack("<Q", len(hb)) + hb)
    with pytest.raises(ValueError):
        TF.read_header(str(odd))


def test_without_packed_file_the_pt_path_is_used(ref_dirs):
    assert not os.path.exists(TF.packed_path(LAYER))
    m = HybridStorageManager(LAYER, E, H, device="cpu")
    assert torch.count_nonzero(m.values_buffer[0, 0]) > 0


@pytest.mark.gpu
def test_packed_layer_device_load_matches_host(ref_dirs, hip_device):
    ref = HybridStorageManager(LAYER, E, H, device="cpu", use_packed=False)
    TF.pack_layer(LAYER, E, H)
    got = HybridStorageManager(LAYER, E, H, device=hip_device)
    for name in ("raw_keys_buffer", "keys_buffer", "values_buffer"):
        t = getattr(got, name)
        assert t.device.type == "cuda"
        assert _same(getattr(ref, name), t.cpu()), name
    # the bias is computed on the load device: compare with the .pt path on the same device
    ref_dev = HybridStorageManager(LAYER, E, H, device=hip_device, use_packed=False)
    for mod in ("vision", "text"):
        for part in ("proj", "bias"):
            assert _same(ref_dev.pca[mod][part].cpu(), got.pca[mod][part].cpu()), (mod, part)
