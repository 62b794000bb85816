"""DuoAttention pattern files and head-pattern arguments on the host
(src/flashquest/duo/pattern.py; the reference's tests/test_duo_pattern.py:28-45)."""
import pytest
import torch

from flashquest_amd import _ops
from flashquest_amd.duo import load_duo_pattern


def test_threshold_and_default(tmp_path):
    p = tmp_path / "tiny.tsv"
    p.write_text("0.4\t0.6\n0.5\t0.51\n")
    assert load_duo_pattern(p).tolist() == [[False, True], [True, True]]
    assert load_duo_pattern(p, threshold=0.51).tolist() == [[False, True], [False, True]]
    assert load_duo_pattern(p).dtype == torch.bool


def test_bad_files(tmp_path):
    with pytest.raises(FileNotFoundError):
        load_duo_pattern(tmp_path / "missing.tsv")
    empty = tmp_path / "empty.tsv"
    empty.write_text("\n\n")
    with pytest.raises(ValueError):
        load_duo_pattern(empty)
    ragged = tmp_path / "ragged.tsv"
    ragged.write_text("0.1\t0.9\n0.3\n")
    with pytest.raises(ValueError):
        load_duo_pattern(ragged)


def test_retention_rows_from_patterns():
    r, ls = _ops.retention_rows(0.25, None, 6, 2, 3, "cpu")
    assert ls == 0 and r.tolist() == [0.25] * 6
    r, ls = _ops.retention_rows(0.25, torch.tensor([True, False]), 6, 2, 3, "cpu")
    assert ls == 0 and r.tolist() == [0.25] * 3 + [0.0] * 3
    pat = torch.tensor([[True, False], [False, False], [True, True]])
    r, ls = _ops.retention_rows(0.5, pat, 4, 2, 3, "cpu")
    assert ls == 4 and r.shape == (3, 4)
    assert r.tolist() == [[0.5, 0.5, 0.0, 0.0], [0.0] * 4, [0.5] * 4]
    # a per-query-head retention vector is masked by the pattern
    r, _ = _ops.retention_rows(torch.tensor([0.1, 0.2, 0.3, 0.4]), torch.tensor([False, True]), 4, 2, 1, "cpu")
    assert r.tolist() == pytest.approx([0.0, 0.0, 0.3, 0.4])
    with pytest.raises(ValueError, match="head_pattern"):
        _ops.retention_rows(0.25, torch.tensor([True, False, True]), 6, 2, 1, "cpu")
    with pytest.raises(ValueError, match="bool"):
        _ops.retention_rows(0.25, torch.tensor([1, 0]), 6, 2, 1, "cpu")
