"""Decoding host logic without a GPU (alodlm/inference.py; tests/test_inference.py):
settings validation, the prefix cache's keys, completion and append."""

import pytest
import torch


def model_config(max_depth=4):
    from alodlm_amd.config import ModelConfig
    return ModelConfig(loop_start=1, loop_end=2, max_depth=max_depth, mask_token_id=3,
                       block_size=4, gate_init_pi=tuple([1.0 / max_depth] * max_depth))


def test_decode_config_validation():
    from alodlm_amd.inference import DecodeConfig
    DecodeConfig().validate()
    DecodeConfig(q=0, tau=0, mode="left1", position_penalty=0.0).validate()
    for bad in (DecodeConfig(q=1.1), DecodeConfig(q=-0.1), DecodeConfig(tau=float("nan")),
                DecodeConfig(tau=float("inf")), DecodeConfig(window_size=0),
                DecodeConfig(max_new_tokens=0), DecodeConfig(mode="greedy"),
                DecodeConfig(position_penalty=-1.0), DecodeConfig(position_penalty=float("inf"))):
        with pytest.raises(ValueError):
            bad.validate()


def test_cache_keys():
    from alodlm_amd.inference import PrefixCache
    cache = PrefixCache(model_config())
    assert cache.key(0, 3) == (0, 0)
    assert cache.key(1, 3) == (1, 3)
    assert cache.key(2, 2) == (2, 0)


def fill(cache, key, start, values_k, values_v):
    k, v = cache.rows(key, start, values_k.shape[0])
    k.copy_(values_k)
    v.copy_(values_v)
    return k, v


@pytest.mark.parametrize("completed", [1, 2, 3, 4])
def test_cache_completion_preserves_computed_depths(completed):
    """tests/test_inference.py:16-29: depths a window did not execute take the
    last executed depth's K/V; append keeps the chosen rows in order."""
    from alodlm_amd.inference import PrefixCache
    cache = PrefixCache(model_config())
    cache._bind(2, 8, torch.float32, torch.device("cpu"))
    cache.reserve(3)
    window = {}
    for d in range(completed):
        window[1, d] = fill(cache, (1, d), 0, torch.full((3, 2, 8), float(d)),
                            torch.full((3, 2, 8), float(d + 10)))
    window[0, 0] = fill(cache, (0, 0), 0, torch.ones(3, 2, 8), torch.ones(3, 2, 8))
    cache.complete(window, completed)
    for d in range(4):
        assert float(window[1, d][0][0, 0, 0]) == min(d, completed - 1)
        assert float(window[1, d][1][0, 0, 0]) == min(d, completed - 1) + 10
    expect = {key: (k[[2, 0]].clone(), v[[2, 0]].clone()) for key, (k, v) in window.items()}
    cache.append(window, torch.tensor([2, 0]))
    assert cache.length == 2
    for key in window:
        torch.testing.assert_close(cache.values[key][0], expect[key][0])
        torch.testing.assert_close(cache.values[key][1], expect[key][1])


def test_cache_growth_keeps_prefix():
    """Growing the buffers keeps the cached rows; a window writes after them."""
    from alodlm_amd.inference import PrefixCache
    cache = PrefixCache(model_config())
    cache._bind(1, 4, torch.float32, torch.device("cpu"))
    cache.reserve(2)
    rows = torch.arange(8.0).view(2, 1, 4)
    window = {(0, 0): fill(cache, (0, 0), 0, rows, -rows)}
    cache.append(window, torch.tensor([1, 0]))
    cache.reserve(500)
    k, v = cache.values[(0, 0)]
    torch.testing.assert_close(k, rows[[1, 0]])
    torch.testing.assert_close(v, -rows[[1, 0]])
    more = torch.full((3, 1, 4), 7.0)
    window = {(0, 0): fill(cache, (0, 0), cache.length, more, more)}
    cache.append(window, torch.tensor([0, 2]))
    assert cache.length == 4
    torch.testing.assert_close(cache.values[(0, 0)][0][2:], more[[0, 2]])
    with pytest.raises(ValueError):
        cache._bind(2, 4, torch.float32, torch.device("cpu"))
