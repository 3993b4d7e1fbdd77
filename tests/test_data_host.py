"""Packed-data path (alodlm/data.py) on the host: the cache format and packing
against caches written by the reference, and the behaviours of the
reference's own tests (tests/test_workflow.py:86-135)."""

import json
import shutil
from pathlib import Path

import numpy as np
import pytest
import torch

from tests.golden import HERE as GOLDEN

FIXTURE = GOLDEN / "workflow" / "fixture"


def golden_cache(name):
    with np.load(GOLDEN / "workflow" / f"{name}.npz", allow_pickle=False) as data:
        return {k: data[k] for k in data.files}


@pytest.fixture(scope="module")
def tokenizer():
    from alodlm_amd.data import load_tokenizer
    return load_tokenizer(FIXTURE / "base")


@pytest.mark.parametrize("name,source,max_length,seed", [
    ("cache_fixture", "training.jsonl", 24, 17),
    ("cache_varied", "varied.jsonl", 48, 5),
])
def test_cache_matches_reference(tmp_path, tokenizer, name, source, max_length, seed):
    """Every tensor, the identity digest and the filtered count equal the
    reference's cache for the same file, tokenizer, length and seed."""
    from alodlm_amd.data import prepare_cache
    train_file = tmp_path / source
    shutil.copy(FIXTURE / source, train_file)
    path = prepare_cache(train_file, tokenizer, tmp_path / "cache.pt", max_length, seed)
    got = torch.load(path, weights_only=True)
    want = golden_cache(name)
    assert got["identity"] == str(want["identity"])
    assert got["filtered_records"] == int(want["filtered_records"])
    for key in ("input_ids", "labels", "batch_offsets", "cum_flat", "cum_offsets"):
        assert got[key].dtype == torch.from_numpy(want[key]).dtype, key
        assert np.array_equal(got[key].numpy(), want[key]), key


def test_varied_cache_invariants(tmp_path, tokenizer):
    """Packs hold at most max_length tokens (all but the last exactly), every
    pack's boundaries run from 0 to its length, strictly increasing."""
    from alodlm_amd.data import PackedDataset, prepare_cache
    train_file = tmp_path / "varied.jsonl"
    shutil.copy(FIXTURE / "varied.jsonl", train_file)
    dataset = PackedDataset(prepare_cache(train_file, tokenizer, tmp_path / "c.pt", 48, 5))
    assert len(dataset) > 10
    total = 0
    for i in range(len(dataset)):
        pack = dataset[i]
        b = pack["boundaries"]
        assert int(b[0]) == 0 and int(b[-1]) == len(pack["ids"]) == len(pack["labels"])
        assert bool((b[1:] > b[:-1]).all())
        assert len(pack["ids"]) == 48 or i == len(dataset) - 1
        assert pack["ids"].dtype == torch.int64 and pack["labels"].dtype == torch.int64
        total += len(pack["ids"])
    assert total == len(dataset.cache["input_ids"])
    with pytest.raises(IndexError):
        dataset[len(dataset)]
    with pytest.raises(IndexError):
        dataset[-1]


def test_pack_stream_cases():
    """Conversation ends and pack ends both cut segments; a conversation that
    ends exactly at a pack end gives one boundary, not two."""
    from alodlm_amd.data import pack_stream
    offsets, flat, starts = pack_stream([10, 20], 24)
    assert offsets.tolist() == [0, 24, 30]
    assert flat.tolist() == [0, 10, 24, 0, 6]
    assert starts.tolist() == [0, 3, 5]
    offsets, flat, starts = pack_stream([24, 3], 24)
    assert offsets.tolist() == [0, 24, 27]
    assert flat.tolist() == [0, 24, 0, 3]
    assert starts.tolist() == [0, 2, 4]
    # one conversation spanning three packs
    offsets, flat, starts = pack_stream([50], 20)
    assert offsets.tolist() == [0, 20, 40, 50]
    assert flat.tolist() == [0, 20, 0, 20, 0, 10]
    assert starts.tolist() == [0, 2, 4, 6]


def test_cache_binds_data(tmp_path, tokenizer):
    """A cache is reused for the same inputs and refused once the data file
    changes (tests/test_workflow.py:86-99)."""
    from alodlm_amd.data import PackedDataset, prepare_cache
    train_file = tmp_path / "training.jsonl"
    shutil.copy(FIXTURE / "training.jsonl", train_file)
    cache = tmp_path / "packed.pt"
    path = prepare_cache(train_file, tokenizer, cache, 24, 17)
    assert prepare_cache(train_file, tokenizer, cache, 24, 17) == path
    dataset = PackedDataset(path)
    assert len(dataset) > 0
    for pack in dataset:
        assert int(pack["boundaries"][-1]) == len(pack["ids"])
        assert len(pack["ids"]) <= 24
    with train_file.open("a") as handle:
        handle.write("\n")
    with pytest.raises(ValueError):
        prepare_cache(train_file, tokenizer, cache, 24, 17)
    with pytest.raises(ValueError):
        prepare_cache(train_file, tokenizer, tmp_path / "other.pt", 1, 17)


def test_multiturn_labels_and_overlength(tokenizer):
    """Only the last assistant turn is supervised; too-long conversations are
    dropped; a single message is fully unsupervised
    (tests/test_workflow.py:101-115)."""
    from alodlm_amd.data import tokenize_messages
    messages = [
        {"role": "user", "content": "Return value one"},
        {"role": "assistant", "content": "one"},
        {"role": "user", "content": "Return value three"},
        {"role": "assistant", "content": "three"},
    ]
    ids, labels = tokenize_messages(messages, tokenizer, 64)
    assert ids.dtype == torch.int32 and labels.dtype == torch.int32
    assert bool((labels[ids == tokenizer.convert_tokens_to_ids("one")] == -100).all())
    assert tokenizer.convert_tokens_to_ids("three") in labels.tolist()
    supervised = labels != -100
    # the supervised part is a suffix and equals the ids there
    first = int(supervised.nonzero()[0])
    assert bool(supervised[first:].all()) and torch.equal(labels[first:], ids[first:])
    assert tokenize_messages(messages, tokenizer, 4) is None
    _, labels = tokenize_messages(messages[:1], tokenizer, 64)
    assert bool((labels == -100).all())
    assert tokenize_messages([], tokenizer, 64) is None


def test_invalid_conversations_are_filtered(tmp_path, tokenizer):
    """A conversation ending on a user turn is rejected by tokenize_messages
    and counted as filtered by prepare_cache (tests/test_workflow.py:117-135)."""
    from alodlm_amd.data import PackedDataset, prepare_cache, tokenize_messages
    valid = [{"role": "user", "content": "Return value one"},
             {"role": "assistant", "content": "one"}]
    invalid = valid + [{"role": "user", "content": "Return value three"}]
    with pytest.raises(ValueError, match="assistant"):
        tokenize_messages(invalid, tokenizer, 64)
    with pytest.raises(ValueError, match="message list"):
        tokenize_messages({"role": "user", "content": "x"}, tokenizer, 64)
    with pytest.raises(ValueError, match="text"):
        tokenize_messages([{"role": "user", "content": 3}], tokenizer, 64)
    train_file = tmp_path / "training.jsonl"
    train_file.write_text(json.dumps(valid) + "\n" + json.dumps(invalid) + "\n")
    dataset = PackedDataset(prepare_cache(train_file, tokenizer, tmp_path / "c.pt", 64, 17))
    assert dataset.cache["filtered_records"] == 1
    ids, labels = tokenize_messages(valid, tokenizer, 64)
    assert torch.equal(dataset[0]["ids"], ids.long())
    assert torch.equal(dataset[0]["labels"], labels.long())
    empty = tmp_path / "empty.jsonl"
    empty.write_text(json.dumps(invalid) + "\n")
    with pytest.raises(ValueError, match="No usable"):
        prepare_cache(empty, tokenizer, tmp_path / "e.pt", 64, 17)


def test_one_pack():
    from alodlm_amd.data import one_pack
    assert one_pack([{"ids": 1}]) == {"ids": 1}
    with pytest.raises(ValueError):
        one_pack([{}, {}])


def test_tokenizer_requires_chat_template(tmp_path):
    from alodlm_amd.data import load_tokenizer
    base = tmp_path / "base"
    shutil.copytree(FIXTURE / "base", base)
    (base / "chat_template.jinja").unlink()
    config = json.loads((base / "tokenizer_config.json").read_text())
    config.pop("chat_template", None)
    (base / "tokenizer_config.json").write_text(json.dumps(config))
    with pytest.raises(ValueError, match="chat template"):
        load_tokenizer(base)
    with pytest.raises(ValueError):
        load_tokenizer(tmp_path / "missing")
