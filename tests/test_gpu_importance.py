"""GPU parity of the importance kernel (tm_last_query_importance) and its
Python mirrors against the oracle's last_query_importance, and its use as the
attention input of the expert keep mask."""

import numpy as np
import pytest
import torch

from oracle import tm_oracle as O
from parity_util import ODT, np64

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("b,h,hkv,d,s,dtype", [(1, 32, 4, 128, 4096, torch.bfloat16),   # Qwen3-VL-30B-A3B heads
                                               (2, 16, 16, 64, 777, torch.float16),
                                               (1, 8, 2, 256, 513, torch.bfloat16),
                                               (3, 4, 1, 192, 100, torch.bfloat16)])
def test_qwen_importance_vs_oracle(hip_device, b, h, hkv, d, s, dtype):
    """Model-dtype scores (the Qwen hook): query_states [B, H, S, D] and
    key_states [B, Hkv, S, D]; the stored weights are the head mean of the
    last query's probabilities."""
    from table_moe.utils import ModalityContext, compute_and_cache_importance

    g = torch.Generator().manual_seed(s + h)
    qs = torch.randn(b, h, 5, d, generator=g).to(dtype)
    ks = torch.randn(b, hkv, s, d, generator=g).to(dtype)
    scale = d ** -0.5
    dev = hip_device
    got = compute_and_cache_importance(qs.to(dev), ks.to(dev), scale)
    torch.cuda.synchronize()
    assert ModalityContext.get_attn_weights() is not None
    assert torch.equal(ModalityContext.get_attn_weights(), got.view(-1))
    want = O.last_query_importance(np64(qs[:, :, -1]), np64(ks.transpose(1, 2)), hkv, scale, ODT[dtype])
    # fp32 accumulation order of the dot products may move a score by one
    # model-dtype ulp; the probabilities then differ by about that ratio
    np.testing.assert_allclose(np64(got), want, rtol=0.02, atol=1e-7)
    assert np.mean(np.abs(np64(got) - want) <= 1e-6 * np.abs(want) + 1e-9) > 0.9
    np.testing.assert_allclose(np64(got).sum(axis=1), 1.0, rtol=1e-5)


def test_deepseek_importance_masked_tail(hip_device):
    """fp32 scores with a key padding mask and only the last query_length keys
    (the DeepSeek hook): query_states [B, q, H, D], key_states [B, kv, H, D]."""
    from table_moe.utils import cache_last_token_attention

    g = torch.Generator().manual_seed(3)
    b, h, d, kv, qlen = 2, 16, 128, 1500, 600
    qs = torch.randn(b, qlen, h, d, generator=g).to(torch.bfloat16)
    ks = torch.randn(b, kv, h, d, generator=g).to(torch.bfloat16)
    mask = torch.rand(b, kv, generator=g) < 0.9
    dev = hip_device
    got = cache_last_token_attention(qs.to(dev), ks.to(dev), 0.088, mask.to(dev), qlen)
    torch.cuda.synchronize()
    want = O.last_query_importance(np64(qs[:, -1]), np64(ks), h, 0.088, O.F32, key_mask=mask.numpy(), out_len=qlen)
    np.testing.assert_allclose(np64(got), want, rtol=1e-4, atol=1e-9)
    assert np.all(np64(got)[~mask.numpy()[:, -qlen:]] == 0.0)


def test_importance_feeds_expert_keep_mask(hip_device):
    """End to end: importance -> tm_expert_keep_mask equals the oracle's
    build_prefill_keep_mask on the device's importance (random scores leave
    no near-tie at the keep boundary here)."""
    from table_moe.skip.pruning import build_prefill_keep_mask
    from table_moe.utils import compute_and_cache_importance

    g = torch.Generator().manual_seed(9)
    n, h, hkv, d, e, k = 1024, 32, 4, 128, 128, 8
    qs = torch.randn(1, h, n, d, generator=g).to(torch.bfloat16)
    ks = torch.randn(1, hkv, n, d, generator=g).to(torch.bfloat16)
    dev = hip_device
    attn = compute_and_cache_importance(qs.to(dev), ks.to(dev), d ** -0.5).view(-1)
    sel = torch.stack([torch.randperm(e, generator=g)[:k] for _ in range(n)])
    w = torch.softmax(torch.randn(n, e, generator=g), dim=1).gather(1, sel)
    mask = build_prefill_keep_mask(sel.to(dev), w.to(dev), attn, e, 0.6)
    torch.cuda.synchronize()
    want, _ = O.build_prefill_keep_mask(sel.numpy(), np64(w), np64(attn), e, 0.6)
    np.testing.assert_array_equal(mask.cpu().numpy(), want)
