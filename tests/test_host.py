"""Host-side logic that needs no device: configuration, modality context,
table-file parsing/loading, workload generator, and the no-fallback rule."""

import numpy as np
import pytest
import torch

from oracle import tm_oracle as O


def test_cache_config_semantics():
    from table_moe.cache_engine import CacheConfig, get_active_cache_config, set_active_cache_config
    from table_moe.cache_engine import update_active_cache_config

    saved = get_active_cache_config()
    try:
        assert CacheConfig.FIXED_K == 256 and CacheConfig.COMPRESSED_DIM == 64
        assert CacheConfig.OFFLINE_COSINE_THRESHOLD_VISION == 0.6 and CacheConfig.OFFLINE_COSINE_THRESHOLD_TEXT == 0.7
        set_active_cache_config({"KEEP_RATE": 0.25})
        assert CacheConfig.KEEP_RATE == 0.25 and CacheConfig.FIXED_K == 256  # merged with defaults
        update_active_cache_config(FIXED_K=128)
        assert CacheConfig.FIXED_K == 128
        CacheConfig.FIXED_K = 64
        assert get_active_cache_config()["FIXED_K"] == 64
        with pytest.raises(AttributeError):
            _ = CacheConfig.NOT_A_KEY
    finally:
        set_active_cache_config(saved)


def test_modality_context_mask():
    from table_moe.utils import ModalityContext

    ModalityContext.clear()
    m = ModalityContext.get_modality_mask(torch.device("cpu"), 3)
    assert m.shape == (1, 3) and not m.any()
    ids = torch.tensor([[5, 151655, 151656, 7, 151655]])
    ModalityContext.set_input_ids(ids)
    got = ModalityContext.get_modality_mask(torch.device("cpu"), 5)
    np.testing.assert_array_equal(got.numpy(), O.modality_mask(ids.numpy()))
    assert ModalityContext.get_modality_mask(torch.device("cpu"), 5) is got  # cached per (device, seq_len)
    np.testing.assert_array_equal(ModalityContext.get_modality_mask(torch.device("cpu"), 1).numpy(), [[True]])
    ModalityContext.clear()


def test_modality_context_per_thread_and_reset():
    """State is per thread (the reference's thread-local contract), a new
    prompt drops the memoised masks, attention weights round-trip, and a
    seq_len shorter than the prompt selects its last tokens."""
    import threading

    from table_moe.utils.modality import ModalityContext

    ModalityContext.clear()
    ids = torch.tensor([[151656, 3, 151655, 151655]])
    ModalityContext.set_input_ids(ids)
    w = torch.rand(4)
    ModalityContext.set_attn_weights(w)
    seen = {}

    def other():
        seen["ids"] = ModalityContext.get_input_ids()
        seen["w"] = ModalityContext.get_attn_weights()
        seen["mask"] = ModalityContext.get_modality_mask(torch.device("cpu"), 4)

    t = threading.Thread(target=other)
    t.start()
    t.join()
    assert seen["ids"] is None and seen["w"] is None and not seen["mask"].any()
    assert ModalityContext.get_attn_weights() is w
    m4 = ModalityContext.get_modality_mask(torch.device("cpu"), 4)
    np.testing.assert_array_equal(m4.numpy(), [[True, False, True, True]])
    np.testing.assert_array_equal(ModalityContext.get_modality_mask(torch.device("cpu"), 2).numpy(), [[True, True]])
    np.testing.assert_array_equal(ModalityContext.get_modality_mask(torch.device("cpu")).numpy(), m4.numpy())
    ModalityContext.set_input_ids(torch.tensor([[1, 2, 3, 4]]))  # a new prompt: memo dropped
    assert not ModalityContext.get_modality_mask(torch.device("cpu"), 4).any()
    ModalityContext.clear()
    assert ModalityContext.get_input_ids() is None and ModalityContext.get_attn_weights() is None


def test_table_files_load_on_host(tmp_path):
    """The on-disk table format (step2/step3 .pt files) is parsed and installed;
    bad files are reported and skipped (reference manager.py:157-210)."""
    from table_moe.cache_engine import CacheConfig, HybridStorageManager
    from table_moe.cache_engine.manager import _parse_cache_name

    assert _parse_cache_name("L3_E17_vision_cache.pt") == (17, "vision")
    g = torch.Generator().manual_seed(0)
    layer = 3
    (tmp_path / "pca" / f"layer_{layer}").mkdir(parents=True)
    (tmp_path / "tab" / f"layer_{layer}").mkdir(parents=True)
    H, d, K = 32, 8, 16
    mean = torch.randn(H, generator=g)
    proj = torch.randn(H, d, generator=g)
    torch.save({"mean": mean, "proj": proj}, tmp_path / "pca" / f"layer_{layer}" / f"L{layer}_vision_pca.pt")
    key = torch.randn(K, d, generator=g)
    val = torch.randn(K, H, generator=g)
    torch.save({"id": torch.arange(K, dtype=torch.int32), "key": key, "value": val},
               tmp_path / "tab" / f"layer_{layer}" / f"L{layer}_E2_text_cache.pt")
    (tmp_path / "tab" / f"layer_{layer}" / f"L{layer}_E1_vision_cache.pt").write_bytes(b"not a torch file")
    saved = {k: getattr(CacheConfig, k) for k in ("PCA_DIR", "CACHE_DIR", "FIXED_K", "COMPRESSED_DIM", "MODEL_DTYPE")}
    try:
        CacheConfig.PCA_DIR, CacheConfig.CACHE_DIR = str(tmp_path / "pca"), str(tmp_path / "tab")
        CacheConfig.FIXED_K, CacheConfig.COMPRESSED_DIM, CacheConfig.MODEL_DTYPE = K, d, torch.float32
        mgr = HybridStorageManager(layer, 4, H, "cpu")
    finally:
        for k, v in saved.items():
            setattr(CacheConfig, k, v)
    torch.testing.assert_close(mgr.raw_keys_buffer[2, 1], key)
    torch.testing.assert_close(mgr.values_buffer[2, 1], val)
    np.testing.assert_allclose(mgr.keys_buffer[2, 1].numpy(), O.normalize_keys(key.numpy(), O.F32), rtol=1e-6)
    torch.testing.assert_close(mgr.pca["vision"]["bias"], -(mean @ proj))
    assert mgr.pca["text"]["proj"].abs().sum() == 0  # missing PCA file -> zeros
    assert mgr.keys_buffer[1].abs().sum() == 0       # unreadable file skipped
    assert mgr.enable_online and mgr.online_keys.shape == (64, H)


def test_no_cpu_fallback_for_host_tensors():
    from table_moe.ops import qwen_topk_softmax
    from table_moe.skip import build_fixed_keep_mask, renormalize_surviving_weights

    with pytest.raises(RuntimeError, match="HIP device"):
        renormalize_surviving_weights(torch.rand(2, 4), torch.ones(2, 4, dtype=torch.bool))
    with pytest.raises(RuntimeError, match="HIP device"):
        qwen_topk_softmax(torch.rand(3, 8), 2)
    with pytest.raises(RuntimeError, match="HIP device"):
        build_fixed_keep_mask(torch.zeros(2, 4, dtype=torch.long), 2)
    with pytest.raises(ValueError, match="2D"):
        qwen_topk_softmax(torch.rand(3), 2)


def test_synthetic_workload_properties():
    from synth import make_workload

    wl = make_workload(2, n=512)
    assert wl.x.shape == (512, 2048) and wl.x.dtype == torch.bfloat16
    assert int(wl.is_vision.sum()) == 448  # vision share of config 2 (3584/4096)
    near = wl.cluster_of >= 0
    assert abs(float(near.float().mean()) - 0.7) < 0.01
    # near tokens project onto their centroid (+ within-cluster noise sigma 0.2)
    x = wl.x.float()
    q = torch.where(wl.is_vision[:, None], x @ wl.proj_vis.float(), x @ wl.proj_txt.float())
    err = (q[near] - wl.centroids.float()[wl.cluster_of[near]]).pow(2).sum(1).sqrt()
    assert float(err.median()) < 0.2 * np.sqrt(128) * 1.3
    w3 = make_workload(3, n=8)
    assert w3.centroids.shape == (16384, 128) and not w3.is_vision.any()


def test_wait_error_clears_the_sync_region(monkeypatch):
    """A grown error word makes the layer call raise, and the workspace's sync
    region (flags, counters, the word) is cleared before the next call, so no
    flag a late workgroup of the failed call left can pass for the next
    call's; a later check with the word at zero passes.  Host logic only: the
    workspace is a host tensor standing in for the device one (and no stream
    is being captured)."""
    from table_moe import _native as N
    from table_moe.cache_engine import GlobalTable

    monkeypatch.setattr(torch.cuda, "is_current_stream_capturing", lambda: False)

    t = object.__new__(GlobalTable)
    ws = torch.zeros(N.TM_LAYER_SYNC_BYTES + 256, dtype=torch.uint8)
    ws[:N.TM_LAYER_SYNC_BYTES] = 7  # stale flags and counters
    e = N.TM_LAYER_SYNC_ERR_BYTE
    ws[e:e + 4].view(torch.int32)[0] = 1
    ws[N.TM_LAYER_SYNC_BYTES:] = 5  # past the sync region: untouched
    t._bufs = {"layer_ws": ws}
    with pytest.raises(RuntimeError, match="ran out"):
        t._raise_on_wait_errors()
    assert int(ws[:N.TM_LAYER_SYNC_BYTES].count_nonzero()) == 0
    assert bool((ws[N.TM_LAYER_SYNC_BYTES:] == 5).all())
    assert t.wait_errors() == 0
    t._raise_on_wait_errors()  # nothing new: no error
