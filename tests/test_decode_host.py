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


def test_decode_state_struct_matches_header(tmp_path):
    """The ctypes mirror of alodlm_decode_state has the C struct's field
    order, offsets and size (a gcc-compiled probe prints them)."""
    import ctypes
    import shutil
    import subprocess
    from pathlib import Path
    from alodlm_amd.inference import DecodeState
    gcc = shutil.which("gcc")
    if gcc is None:
        pytest.skip("gcc not available")
    include = Path(__file__).resolve().parents[1] / "include"
    fields = [name for name, _ in DecodeState._fields_]
    src = tmp_path / "probe.c"
    src.write_text("#include <stddef.h>\n#include <stdio.h>\n#include \"alodlm_hip.h\"\n"
                   "int main(void) {\n" + "".join(
                       f'  printf("%zu\\n", offsetof(alodlm_decode_state, {f}));\n'
                       for f in fields) +
                   '  printf("%zu\\n", sizeof(alodlm_decode_state));\n  return 0;\n}\n')
    exe = tmp_path / "probe"
    subprocess.run([gcc, "-I", str(include), str(src), "-o", str(exe)], check=True)
    out = [int(v) for v in subprocess.run([str(exe)], check=True, capture_output=True,
                                          text=True).stdout.split()]
    assert out[:-1] == [getattr(DecodeState, f).offset for f in fields]
    assert out[-1] == ctypes.sizeof(DecodeState)


def test_stop_tokens_and_penalty():
    """EOS id(s) plus the chat end markers the vocabulary holds
    (alodlm/inference.py:158-163); the default position penalty is tau / 20."""
    from alodlm_amd.inference import DecodeConfig, stop_token_ids

    class Tok:
        def __init__(self, eos, vocab):
            self.eos_token_id, self.vocab = eos, vocab

        def get_vocab(self):
            return self.vocab

        def convert_tokens_to_ids(self, t):
            return self.vocab[t]

    assert stop_token_ids(Tok(7, {"<|im_end|>": 9, "x": 1})) == [7, 9]
    assert stop_token_ids(Tok([5, 2], {"</s>": 2})) == [2, 5]
    assert stop_token_ids(Tok(None, {})) == []
    assert DecodeConfig(tau=0.4).penalty == pytest.approx(0.02)
    assert DecodeConfig(tau=0.4, position_penalty=0.0).penalty == 0.0
