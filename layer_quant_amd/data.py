"""WikiText text source of the decode driver.

Interface of reference hybrid_quant/data.py:14-20 (the driver imports only
`load_wikitext_texts`). `datasets` is imported on first use, so importing this module needs
neither the package nor a network.
"""
from __future__ import annotations

from pathlib import Path

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
