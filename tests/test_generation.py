"""Host checks of the generation-input slicing (ccq_amd.generation), following the cases the
reference's CCQGenerationMixin distinguishes (ccq/generation.py:17-50): nothing seen -> the whole
prompt (or the prompt embeddings); `seen` tokens -> the tokens after position `seen`; a cache that
claims every token -> the last one; a cache whose length cannot be read counts as empty."""

import torch

from ccq_amd.generation import CCQGenerationMixin, cache_seen_tokens
from ccq_amd.layers import LayerCache


class _Model(CCQGenerationMixin):
    pass


class _Broken:
    def get_seq_length(self):
        raise RuntimeError("no length")


def _cache(seen):
    c = LayerCache()
    if seen:
        c.update(0, recurrent_state=None, conv_state=None, offset=seen)
    return c


def test_seen_tokens():
    assert cache_seen_tokens(None) == 0
    assert cache_seen_tokens(_Broken()) == 0
    assert cache_seen_tokens(_cache(0)) == 0
    assert cache_seen_tokens(_cache(7)) == 7


def test_first_call_feeds_the_whole_prompt():
    ids = torch.arange(12).view(2, 6)
    out = _Model().prepare_inputs_for_generation(ids, past_key_values=_cache(0), attention_mask=None)
    assert torch.equal(out["input_ids"], ids)
    # a pre-allocated (empty) cache object is not mistaken for a filled one
    out = _Model().prepare_inputs_for_generation(ids, past_key_values=LayerCache())
    assert torch.equal(out["input_ids"], ids)


def test_later_calls_feed_only_unseen_tokens():
    ids = torch.arange(12).view(2, 6)
    out = _Model().prepare_inputs_for_generation(ids, past_key_values=_cache(5), use_cache=True)
    assert torch.equal(out["input_ids"], ids[:, 5:])
    assert out["input_ids"].is_contiguous()
    out = _Model().prepare_inputs_for_generation(ids, past_key_values=_cache(3))
    assert torch.equal(out["input_ids"], ids[:, 3:])
    # a cache that claims the whole sequence (or more) gets the newest token
    for seen in (6, 9):
        out = _Model().prepare_inputs_for_generation(ids, past_key_values=_cache(seen))
        assert torch.equal(out["input_ids"], ids[:, -1:])
    # a single new token passes through as it is
    out = _Model().prepare_inputs_for_generation(ids[:, -1:], past_key_values=_cache(5))
    assert torch.equal(out["input_ids"], ids[:, -1:])


def test_embeddings_only_while_the_cache_is_empty():
    ids = torch.arange(8).view(2, 4)
    emb = torch.randn(2, 4, 16)
    out = _Model().prepare_inputs_for_generation(ids, past_key_values=_cache(0), inputs_embeds=emb)
    assert "input_ids" not in out and out["inputs_embeds"] is emb
    out = _Model().prepare_inputs_for_generation(ids, past_key_values=_cache(3), inputs_embeds=emb)
    assert "inputs_embeds" not in out and torch.equal(out["input_ids"], ids[:, 3:])


def test_passes_the_other_arguments_through():
    ids = torch.arange(4).view(1, 4)
    cache, mask = _cache(2), torch.ones(1, 4)
    out = _Model().prepare_inputs_for_generation(ids, past_key_values=cache, attention_mask=mask, use_cache=False,
                                                 logits_to_keep=1)
    assert out["past_key_values"] is cache and out["attention_mask"] is mask
    assert out["use_cache"] is False and out["logits_to_keep"] == 1
    assert "logits_to_keep" not in _Model().prepare_inputs_for_generation(ids, past_key_values=cache)
