"""KVCache host logic (no kernels): per-sequence lengths and the RoPE tables a
ragged cache decodes with.  The reference keeps one scalar fill level
(kempnerforge/model/attention.py:29-70); equal lengths must behave exactly as
that."""

from __future__ import annotations

import pytest
import torch

from kempnerforge_amd import KVCache


def _cache(B=3, T=16):
    return KVCache(B, T, 2, 8, torch.float32, torch.device("cpu"))


def test_update_matches_reference_contract():
    c = _cache()
    k = torch.randn(3, 2, 5, 8)
    kk, vv = c.update(k, k + 1)
    assert c.seq_len == 5 and c.lens.tolist() == [5, 5, 5]
    assert torch.equal(kk, k) and torch.equal(vv, k + 1)
    assert not c.ragged


def test_set_lengths_and_tables():
    c = _cache()
    c.set_lengths([3, 9, 4])
    assert c.seq_len == 9 and c.lens.tolist() == [3, 9, 4] and c.ragged
    cos, sin = torch.zeros(16, 4), torch.ones(16, 4)
    with pytest.raises(ValueError):
        c._decode_tables(cos[9:10], sin[9:10])  # ragged needs the full tables
    c.use_rope_tables(cos, sin)
    t = c._decode_tables(cos[9:10], sin[9:10])
    assert t[0] is cos and t[1] is sin and t[2] == 0
    c.set_lengths(torch.tensor([4, 4, 4]))
    assert not c.ragged and c.seq_len == 4


def test_equal_lengths_use_the_callers_slice():
    c = _cache()
    c.set_lengths([6, 6, 6])
    cos, sin = torch.zeros(1, 4), torch.ones(1, 4)
    assert c._decode_tables(cos, sin) == (cos, sin, 6)


def test_set_lengths_validation():
    c = _cache()
    with pytest.raises(ValueError):
        c.set_lengths([1, 2])
    with pytest.raises(ValueError):
        c.set_lengths([1, 2, 17])


def test_seq_len_is_writable_and_moves_lens():
    """The reference's seq_len is a plain attribute a caller may rewind to reuse
    a cache; lens (what the decode kernel reads) must follow it."""
    c = _cache()
    c.update(torch.randn(3, 2, 7, 8), torch.randn(3, 2, 7, 8))
    c.seq_len = 2
    assert c.seq_len == 2 and c.lens.tolist() == [2, 2, 2] and not c.ragged
    c.set_lengths([1, 5, 3])
    c.seq_len = 0  # rewinding a ragged cache makes it uniform again
    assert c.lens.tolist() == [0, 0, 0] and not c.ragged
    c.update(torch.randn(3, 2, 4, 8), torch.randn(3, 2, 4, 8))
    assert c.seq_len == 4 and c.lens.tolist() == [4, 4, 4]
    with pytest.raises(ValueError):
        c.seq_len = 17
    with pytest.raises(ValueError):
        c.seq_len = -1
