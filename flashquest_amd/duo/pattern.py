"""DuoAttention head classifications (src/flashquest/duo/pattern.py:16-60).

The file format is DuoAttention's full_attention_heads.tsv: one line per
layer, one tab-separated number in [0, 1] per KV head, the probability that
the head needs full (retrieval) attention.
"""
from __future__ import annotations

from pathlib import Path

import torch


def load_duo_pattern(path: str | Path, threshold: float = 0.5) -> torch.Tensor:
    """(num_layers, num_kv_heads) bool on the CPU: True where the value is at
    least ``threshold`` (retrieval head), False otherwise (streaming head).
    Raises FileNotFoundError for a missing file and ValueError for an empty
    file or lines of different lengths."""
    path = Path(path)
    if not path.is_file():
        raise FileNotFoundError(f"no DuoAttention pattern file at {path}")
    table = []
    for n, text in enumerate(path.read_text().splitlines(), start=1):
        fields = [f for f in text.strip().split("\t") if f]
        if not fields:
            continue
        if table and len(fields) != len(table[0]):
            raise ValueError(f"{path}:{n}: {len(fields)} heads on this line, {len(table[0])} on the first")
        table.append([float(f) for f in fields])
    if not table:
        raise ValueError(f"{path}: no pattern rows")
    return torch.tensor(table) >= threshold
