"""WikiText text source of the decode driver and its token windows.

Interface of reference hybrid_quant/data.py:14-32 (the driver imports only
`load_wikitext_texts`; `token_segments` completes the module's interface). `datasets` is
imported on first use, so importing this module needs neither the package nor a network.
"""
from __future__ import annotations

from pathlib import Path
from typing import Iterable, Iterator

from .env import configure_cache_env

configure_cache_env()

WIKITEXT_CONFIG = "wikitext-103-raw-v1"


def load_wikitext_texts(dataset_path: str, split: str = "test") -> list[str]:
    """Lines of the WikiText-103 (raw) split that hold any non-whitespace character.

    `dataset_path` names a local dataset directory when one exists there, otherwise a dataset
    known to `datasets.load_dataset`.
    """
    import datasets

    where = Path(dataset_path)
    rows = datasets.load_dataset(str(where) if where.exists() else dataset_path, WIKITEXT_CONFIG,
                                 split=split)
    return [line for line in rows["text"] if line.strip()]


def token_segments(tokenizer, texts: Iterable[str], context_length: int,
                   max_eval_tokens: int) -> Iterator:
    """Overlapping evaluation windows over the tokens of `texts` joined by blank lines
    (reference hybrid_quant/data.py:23-32).

    The texts are tokenized as one string without special tokens; only the first
    min(n_tokens - 1, max_eval_tokens) tokens are predicted. Window k starts at token
    k * context_length and holds up to context_length + 1 tokens (inputs plus the next-token
    targets), so consecutive windows share one token and every predicted token is a target
    exactly once. A context_length below 1 raises ValueError (the reference loops forever).
    """
    if context_length < 1:
        raise ValueError(f"context_length must be >= 1, got {context_length}")
    ids = tokenizer("\n\n".join(texts), add_special_tokens=False, return_tensors="pt").input_ids[0]
    predicted = min(ids.numel() - 1, max_eval_tokens)
    for start in range(0, max(predicted, 0), context_length):
        yield ids[start:min(start + context_length, predicted) + 1]
