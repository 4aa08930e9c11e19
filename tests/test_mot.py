"""MoTAttention structure on the CPU (reference tests/unit/test_mot.py:83-135):
construction, state-dict layout and argument validation, none of which reach
the kernels."""

from __future__ import annotations

import pytest
import torch

from kempnerforge_amd import MoTAttention


def test_zero_init_o_proj_and_keys():
    attn = MoTAttention(dim=64, n_heads=4, n_kv_heads=2, modalities=("image", "text"))
    for m in ("image", "text"):
        assert torch.count_nonzero(attn.o_proj[m].weight) == 0
    keys = set(attn.state_dict())
    assert keys == {f"{p}.{m}.weight" for p in ("q_proj", "k_proj", "v_proj", "o_proj")
                    for m in ("image", "text")}
    assert attn.k_proj["text"].weight.shape == (2 * 16, 64)
    assert attn.q_norm is None and attn.k_norm is None


def test_qk_norm_per_modality():
    attn = MoTAttention(dim=64, n_heads=4, n_kv_heads=4, modalities=("image", "text"),
                        qk_norm=True)
    assert {"q_norm.image.weight", "k_norm.text.weight"} <= set(attn.state_dict())
    assert attn.q_norm["image"] is not attn.q_norm["text"]


def test_invalid_arguments():
    with pytest.raises(ValueError):
        MoTAttention(dim=64, n_heads=4, n_kv_heads=4, modalities=())
    with pytest.raises(ValueError):
        MoTAttention(dim=64, n_heads=4, n_kv_heads=3, modalities=("text",))
    attn = MoTAttention(dim=64, n_heads=4, n_kv_heads=4, modalities=("image", "text"))
    with pytest.raises(ValueError):
        attn({"image": torch.zeros(1, 2, 64)}, {})
