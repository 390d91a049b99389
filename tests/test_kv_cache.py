"""KVStore.to_cache: the DynamicCache handed to HF's decode loop after a prefill is in the state HF's
own first `update` of each owning layer would leave (transformers cache_utils DynamicLayer.update,
DynamicSlidingWindowLayer.update), built without that update's copy.  Host logic only: CPU tensors
on the small Gemma 4 of hf_tiny.py (sliding and full layers, KV-shared layers), prompts shorter
and longer than the sliding window of 16, then one decode update on both caches."""
import pytest
import torch

from hf_tiny import build


@pytest.mark.parametrize("T", [5, 15, 16, 37])
@pytest.mark.parametrize("copy", [False, True])
def test_to_cache_equals_hf_first_update(T, copy):
    from transformers import DynamicCache
    from w8a8.pipeline import KVStore
    cfg = build(seed=1).config.get_text_config()
    g = torch.Generator().manual_seed(T)
    store = KVStore(T)
    owning = range(cfg.num_hidden_layers - cfg.num_kv_shared_layers)
    for layer in owning:
        store.kv[layer] = (torch.randn(2, T, 8, generator=g), torch.randn(2, T, 8, generator=g))
    ours = store.to_cache(cfg, copy=copy)
    want = DynamicCache(config=cfg)
    for layer in owning:
        k, v = store.kv[layer]
        want.update(k[None].clone(), v[None].clone(), layer)
    assert any(lw.is_sliding for lw in want.layers) and not all(lw.is_sliding for lw in want.layers)
    for i, (a, b) in enumerate(zip(ours.layers, want.layers)):
        assert type(a) is type(b) and a.is_initialized == b.is_initialized, f"layer {i}"
        if not b.is_initialized:
            continue
        assert torch.equal(a.keys, b.keys) and torch.equal(a.values, b.values), f"layer {i}"
        assert a.get_seq_length() == b.get_seq_length() == T, f"layer {i}"
        assert a.get_mask_sizes(1) == b.get_mask_sizes(1), f"layer {i}"
        if copy:
            k, _ = store.kv[i]
            assert a.keys.untyped_storage().data_ptr() != k.untyped_storage().data_ptr(), f"layer {i} aliases the store"
    for layer in owning:  # the next decode step's update
        k, v = torch.full((1, 2, 1, 8), float(layer)), torch.ones(1, 2, 1, 8)
        ka, va = ours.update(k, v, layer)
        kb, vb = want.update(k, v, layer)
        assert torch.equal(ka, kb) and torch.equal(va, vb), f"layer {layer}"
        assert torch.equal(ours.layers[layer].keys, want.layers[layer].keys), f"layer {layer}"
    assert ours.get_seq_length() == T + 1
