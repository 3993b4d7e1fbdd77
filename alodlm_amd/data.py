"""Packed training data (drop-in for alodlm/data.py).

The cache file format is the reference's (alodlm/data.py:70-130), so a cache
written by either implementation loads in the other: a ``torch.save`` mapping
with ``identity`` (sha256 of the data file, tokenizer, chat template, special
tokens, ``max_length`` and seed; format version 3), ``input_ids`` and
``labels`` (int32, every pack's tokens back to back), ``batch_offsets`` (token
offset of every pack), ``cum_flat`` (every pack's segment boundaries, each list
starting at 0) with ``cum_offsets`` (where each pack's list starts in
``cum_flat``), and ``filtered_records``.

Packing: the shuffled conversations form one token stream that is cut into
packs of ``max_length`` tokens; a conversation that crosses a pack end
continues as the first segment of the next pack.  Segment boundaries are the
conversation ends and the pack ends.  Here the cut is computed with array
arithmetic over the whole stream instead of a per-conversation loop.
"""

import argparse
import hashlib
import json
import random
from pathlib import Path

import numpy as np
import torch
from torch.utils.data import Dataset

from .config import local_dir

FORMAT_VERSION = 3
IGNORE = -100


def load_tokenizer(directory):
    """Local tokenizer with a chat template (alodlm/data.py:16-25); the pad
    token is ``<|im_end|>`` when the vocabulary has it, else the eos token."""
    from transformers import AutoTokenizer
    tokenizer = AutoTokenizer.from_pretrained(
        str(local_dir(directory)), local_files_only=True, trust_remote_code=False)
    if not tokenizer.chat_template:
        raise ValueError("A local tokenizer with a chat template is required")
    vocab = tokenizer.get_vocab()
    if "<|im_end|>" in vocab:
        tokenizer.pad_token_id = vocab["<|im_end|>"]
    elif tokenizer.eos_token_id is not None:
        tokenizer.pad_token_id = tokenizer.eos_token_id
    return tokenizer


def digest_file(path):
    """sha256 hex digest of a file, read in 1 MiB blocks."""
    digest = hashlib.sha256()
    with Path(path).open("rb") as handle:
        while True:
            block = handle.read(1 << 20)
            if not block:
                break
            digest.update(block)
    return digest.hexdigest()


def cache_identity(train_file, tokenizer, max_length, seed):
    """Digest binding a cache to its data, tokenizer and packing settings
    (alodlm/data.py:36-45; the same fields, so identities agree)."""
    spec = {
        "format_version": FORMAT_VERSION,
        "data_sha256": digest_file(train_file),
        "vocabulary": sorted(tokenizer.get_vocab().items()),
        "tokenizer": tokenizer.backend_tokenizer.to_str(),
        "chat_template": tokenizer.chat_template,
        "special_tokens": tokenizer.special_tokens_map,
        "max_length": max_length,
        "seed": seed,
    }
    return hashlib.sha256(json.dumps(spec, sort_keys=True).encode()).hexdigest()


def tokenize_messages(messages, tokenizer, max_length):
    """(ids, labels) int32 of one conversation, or None when it is empty or
    longer than ``max_length`` (alodlm/data.py:48-67).

    Only the last assistant message is supervised: every position before the
    tokens of the conversation without it (with the generation prompt) is
    ``-100``.  A single message is kept but entirely unsupervised.
    """
    if not messages:
        return None
    if not isinstance(messages, list):
        raise ValueError("Each record must contain a message list")
    for message in messages:
        if not isinstance(message, dict) or not isinstance(message.get("content"), str):
            raise ValueError("Message content must be text")
    if len(messages) > 1 and messages[-1].get("role") != "assistant":
        raise ValueError("Multi-message conversations must end with an assistant response")
    text = tokenizer.apply_chat_template(messages, tokenize=False, add_generation_prompt=False)
    ids = tokenizer.encode(text, add_special_tokens=False)
    if not ids or len(ids) > max_length:
        return None
    unsupervised = len(ids)
    if len(messages) > 1:
        prompt = tokenizer.apply_chat_template(messages[:-1], tokenize=False,
                                               add_generation_prompt=True)
        unsupervised = min(len(tokenizer.encode(prompt, add_special_tokens=False)), len(ids))
    ids = torch.tensor(ids, dtype=torch.int32)
    labels = ids.clone()
    labels[:unsupervised] = IGNORE
    return ids, labels


def pack_stream(lengths, max_length):
    """Pack conversations of the given lengths, in order, into packs of at most
    ``max_length`` tokens.

    Returns ``(batch_offsets, cum_flat, cum_offsets)`` as int64 arrays in the
    cache's layout.  Every pack but the last holds exactly ``max_length``
    tokens; a pack's boundaries are 0, each conversation end inside it, and
    its length.
    """
    lengths = np.asarray(lengths, dtype=np.int64)
    total = int(lengths.sum())
    batch_offsets = np.append(np.arange(0, total, max_length, dtype=np.int64), total)
    ends = np.cumsum(lengths)
    # cut points: conversation ends and pack ends (a conversation end that is
    # also a pack end appears once)
    cuts = np.union1d(ends, batch_offsets[1:])
    pack_of_cut = (cuts - 1) // max_length
    n_packs = len(batch_offsets) - 1
    per_pack = np.bincount(pack_of_cut, minlength=n_packs)
    # each pack's list is [0, cuts inside it relative to its start]
    starts = np.concatenate(([0], np.cumsum(per_pack + 1)[:-1]))
    cum_flat = np.zeros(len(cuts) + n_packs, dtype=np.int64)
    slots = np.arange(len(cuts)) + pack_of_cut + 1
    cum_flat[slots] = cuts - batch_offsets[pack_of_cut]
    cum_offsets = np.append(starts, len(cum_flat)).astype(np.int64)
    return batch_offsets, cum_flat, cum_offsets


def prepare_cache(train_file, tokenizer, cache_file, max_length=4096, seed=42):
    """Tokenize, shuffle and pack a JSONL file of conversations into
    ``cache_file`` (alodlm/data.py:70-130); an existing cache is reused when
    its identity matches and rejected otherwise.  Returns the cache path."""
    if max_length < 2:
        raise ValueError("max_length must be at least two")
    identity = cache_identity(train_file, tokenizer, max_length, seed)
    target = Path(cache_file)
    if target.exists():
        cached = torch.load(target, mmap=True, weights_only=True)
        if cached.get("identity") != identity:
            raise ValueError("Packed cache does not match the local input and tokenizer")
        return target
    samples, filtered = [], 0
    with Path(train_file).open() as handle:
        for line in handle:
            if not line.strip():
                continue
            try:
                sample = tokenize_messages(json.loads(line), tokenizer, max_length)
            except (TypeError, ValueError, KeyError, AttributeError):
                sample = None
            if sample is None:
                filtered += 1
            else:
                samples.append(sample)
    if not samples:
        raise ValueError("No usable training conversations")
    # Python's seeded shuffle, so that the order is the reference's
    random.Random(seed).shuffle(samples)
    batch_offsets, cum_flat, cum_offsets = pack_stream([len(s[0]) for s in samples], max_length)
    packed = {
        "identity": identity,
        "input_ids": torch.cat([s[0] for s in samples]),
        "labels": torch.cat([s[1] for s in samples]),
        "batch_offsets": torch.from_numpy(batch_offsets),
        "cum_flat": torch.from_numpy(cum_flat),
        "cum_offsets": torch.from_numpy(cum_offsets),
        "filtered_records": filtered,
    }
    target.parent.mkdir(parents=True, exist_ok=True)
    partial = target.with_suffix(target.suffix + ".tmp")
    torch.save(packed, partial)
    partial.replace(target)
    return target


class PackedDataset(Dataset):
    """One item per pack: ``{"ids", "labels", "boundaries"}`` int64 tensors
    (alodlm/data.py:133-148).  The cache is memory-mapped."""

    def __init__(self, filename):
        self.cache = torch.load(filename, mmap=True, weights_only=True)

    def __len__(self):
        return len(self.cache["batch_offsets"]) - 1

    def __getitem__(self, index):
        if not 0 <= index < len(self):
            raise IndexError("Pack index out of range")
        c = self.cache
        left, right = (int(v) for v in c["batch_offsets"][index:index + 2])
        a, b = (int(v) for v in c["cum_offsets"][index:index + 2])
        return {"ids": c["input_ids"][left:right].long(),
                "labels": c["labels"][left:right].long(),
                "boundaries": c["cum_flat"][a:b].clone()}


def one_pack(items):
    """Collate for batch size 1: a microbatch is exactly one pack."""
    if len(items) != 1:
        raise ValueError("Each microbatch contains one packed sequence")
    return items[0]


def main():
    parser = argparse.ArgumentParser(description="Pack locally supplied conversations.")
    parser.add_argument("--model", required=True)
    parser.add_argument("--input", required=True)
    parser.add_argument("--output", required=True)
    parser.add_argument("--max-length", type=int, default=4096)
    parser.add_argument("--seed", type=int, default=42)
    args = parser.parse_args()
    path = prepare_cache(args.input, load_tokenizer(args.model), args.output,
                         args.max_length, args.seed)
    print(json.dumps({"packs": len(PackedDataset(path))}))


if __name__ == "__main__":
    main()
