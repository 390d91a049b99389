"""prompt_inputs' RoPE rows kept per prompt length (CPU, with a stand-in language model): a second
prompt of the same length reuses the rows without calling the model's rotary module, another length
computes its own, at most four lengths are kept, the rows equal a fresh computation, and a dynamic
RoPE (frequencies that follow the longest sequence seen) is never kept."""
import types

import torch

from w8a8.pipeline import prompt_inputs


class StandIn:
    """The four members of the HF language model prompt_inputs reads."""

    def __init__(self):
        self.config = types.SimpleNamespace(layer_types=["sliding_attention", "full_attention", "sliding_attention"])
        self.rotary_calls = 0

    def embed_tokens(self, ids):
        return ids[..., None].to(torch.bfloat16).expand(*ids.shape, 8) * 0.5

    def get_per_layer_inputs(self, ids, emb):
        return emb[..., :4]

    def project_per_layer_inputs(self, emb, pl):
        return pl[..., None, :] + 1

    def rotary_emb(self, emb, positions, kind):
        self.rotary_calls += 1
        D = 4 if kind == "sliding_attention" else 6
        ang = positions[..., None].float() * torch.arange(1, D + 1).float() * (0.1 if kind == "full_attention" else 1.0)
        return ang.cos().to(emb.dtype), ang.sin().to(emb.dtype)


def test_rope_rows_are_kept_per_prompt_length():
    lm, cache = StandIn(), {}
    ids = torch.arange(5)[None]
    _, _, rope = prompt_inputs(lm, ids, cache)
    assert lm.rotary_calls == 2  # one call per attention kind
    _, _, again = prompt_inputs(lm, ids + 3, cache)
    assert lm.rotary_calls == 2 and again is rope
    _, _, fresh = prompt_inputs(StandIn(), ids)
    for kind in fresh:
        assert torch.equal(rope[kind][0], fresh[kind][0]) and torch.equal(rope[kind][1], fresh[kind][1])
    prompt_inputs(lm, torch.arange(7)[None], cache)
    assert lm.rotary_calls == 4 and len(cache) == 2


def test_at_most_four_lengths_are_kept():
    lm, cache = StandIn(), {}
    for T in (2, 3, 4, 5, 6):
        prompt_inputs(lm, torch.arange(T)[None], cache)
    assert len(cache) == 4 and all(key[0] != 2 for key in cache)
    prompt_inputs(lm, torch.arange(2)[None], cache)  # evicted: computed again
    assert lm.rotary_calls == 12


def test_without_a_cache_nothing_is_kept():
    lm = StandIn()
    prompt_inputs(lm, torch.arange(4)[None])
    prompt_inputs(lm, torch.arange(4)[None])
    assert lm.rotary_calls == 4


def test_a_dynamic_rope_is_never_kept():
    cache, dyn = {}, StandIn()
    rotary = dyn.rotary_emb

    class Rotary:
        rope_type = {"sliding_attention": "default", "full_attention": "dynamic"}

        def __call__(self, emb, positions, kind):
            return rotary(emb, positions, kind)

    dyn.rotary_emb = Rotary()
    prompt_inputs(dyn, torch.arange(4)[None], cache)
    prompt_inputs(dyn, torch.arange(4)[None], cache)
    assert dyn.rotary_calls == 4 and not cache
