"""WikiText loading for the decode driver (reference hybrid_quant/data.py:14-32).

`datasets` is imported on first use, so importing this module needs no network or dataset.
"""
from __future__ import annotations

from pathlib import Path
from typing import Iterable, List

from .env import configure_cache_env

configure_cache_env()


def load_wikitext_texts(dataset_path: str, split: str = "test") -> List[str]:
    """Non-blank lines of wikitext-103-raw-v1 from a local dataset directory or hub name."""
    from datasets import load_dataset

    source = str(Path(dataset_path)) if Path(dataset_path).exists() else dataset_path
    ds = load_dataset(source, "wikitext-103-raw-v1", split=split)
    return [text for text in ds["text"] if text and not text.isspace()]


def token_segments(tokenizer, texts: Iterable[str], context_length: int, max_eval_tokens: int):
    """Overlapping windows of context_length + 1 token ids over the joined texts."""
    ids = tokenizer("\n\n".join(texts), add_special_tokens=False, return_tensors="pt").input_ids[0]
    usable = min(ids.numel() - 1, max_eval_tokens)
    start = 0
    while start < usable:
        stop = min(start + context_length + 1, usable + 1)
        if stop - start >= 2:
            yield ids[start:stop]
        start = stop - 1
