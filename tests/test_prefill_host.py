"""Host-side checks of the blocked prefill (ai_amd.prefill): the bf16 split of
fp32 activations and the reference's mode switch (prefill.py:14-20)."""
import numpy as np
import pytest
import torch

from ai_amd import prefill


def test_split3_is_exact_for_normal_fp32():
    """hi + mid + lo reproduces every normal fp32 value exactly (24
    significand bits in three 8-bit parts), including values near 1, powers of
    two, huge and tiny normals."""
    g = torch.Generator().manual_seed(0)
    x = torch.cat([torch.randn(4000, generator=g) * s for s in (1e-30, 1e-3, 1.0, 7.0, 1e20)]
                  + [torch.tensor([1.0, -1.0, 1.0 + 2 ** -23, 3.0, 2.0 ** -100, 65504.0, 0.0, -0.0])])
    x = x.reshape(-1, 8)
    parts = prefill.split3(x).float()
    T = x.shape[0]
    back = (parts[:T].double() + parts[T:2 * T].double() + parts[2 * T:].double())
    assert torch.equal(back, x.double())


def test_split3_planted_mistake_is_caught():
    """A split that drops the lowest part loses bits: the exactness check
    above is not vacuous."""
    x = torch.tensor([[1.0 + 2 ** -23, 1.2345678]])
    hi = x.bfloat16()
    mid = (x - hi.float()).bfloat16()
    assert not torch.equal(hi.double() + mid.double(), x.double())


def test_enabled_follows_the_reference_variables(monkeypatch):
    monkeypatch.delenv("RAMVI_PREFILL", raising=False)
    monkeypatch.delenv("RAMVI_PREFILL_MIN_TOKENS", raising=False)
    assert not prefill.enabled(10_000)             # legacy by default
    monkeypatch.setenv("RAMVI_PREFILL", "blocked")
    assert prefill.enabled(256) and not prefill.enabled(255) and prefill.enabled()
    monkeypatch.setenv("RAMVI_PREFILL_MIN_TOKENS", "1")
    assert prefill.enabled(1)
    monkeypatch.setenv("RAMVI_PREFILL_MIN_TOKENS", "-1")
    with pytest.raises(ValueError):
        prefill.enabled(5)
    monkeypatch.setenv("RAMVI_PREFILL", "fast")
    with pytest.raises(ValueError):
        prefill.enabled(5)
