"""Host side of the transformers adapter (no GPU): registration and refusals."""

import pytest
import torch

pytest.importorskip("transformers")

from wavelet_amd import hf


def test_register_names_the_attention_and_mask_functions():
    from transformers.masking_utils import ALL_MASK_ATTENTION_FUNCTIONS
    from transformers.modeling_utils import ALL_ATTENTION_FUNCTIONS

    name = hf.register()
    assert name == "wavelet_paged"
    assert ALL_ATTENTION_FUNCTIONS[name] is hf.paged_attention_forward
    assert ALL_MASK_ATTENTION_FUNCTIONS[name](batch_size=1, q_length=4, kv_length=4) is None


def test_attention_refuses_states_not_from_the_paged_cache():
    q = torch.zeros(1, 8, 1, 128)
    k = torch.zeros(1, 2, 1, 128)
    with pytest.raises(ValueError, match="PagedCache.update"):
        hf.paged_attention_forward(None, q, k, k, None, scaling=0.1)


def test_cache_refuses_a_non_gqa_pool():
    class FakePool:
        layers = []

    with pytest.raises(ValueError, match="GQA KVPool"):
        hf.PagedCache(FakePool(), [0])
