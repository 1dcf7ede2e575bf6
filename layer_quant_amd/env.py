"""Hugging Face cache locations (reference hybrid_quant/env.py:7-14)."""
from __future__ import annotations

import os
from pathlib import Path


def configure_cache_env() -> Path:
    """Point the HF caches below $HYBRID_QUANT_CACHE_DIR (default ./.cache) unless already set."""
    root = Path(os.environ.get("HYBRID_QUANT_CACHE_DIR", Path.cwd() / ".cache")).resolve()
    defaults = {
        "HF_HOME": root / "hf",
        "HF_XET_CACHE": root / "hf-xet",
        "HF_MODULES_CACHE": root / "hf-modules",
        "HF_DATASETS_CACHE": root / "hf" / "datasets",
        "XDG_CACHE_HOME": root / "xdg",
    }
    for key, value in defaults.items():
        os.environ.setdefault(key, str(value))
    return root
