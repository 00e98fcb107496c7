"""Host-side checks of the blocked prefill (ai_amd.prefill): the reference's
mode switch (prefill.py:14-20) and the prefill linear's workspace."""
import pytest

from ai_amd import prefill


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


def test_prefill_workspace_bytes():
    """Six bytes per column and token (three bf16 parts), tokens padded to
    128, plus a scale exponent and an RMS factor per padded token; 0 for bad
    arguments."""
    from ai_amd import _lib
    L = _lib.lib()
    assert L.rv12_prefill_workspace_bytes(4096, 2048) == 2048 * 4096 * 10 + 2048 * 8
    assert L.rv12_prefill_workspace_bytes(1024, 300) == 384 * 1024 * 10 + 384 * 8
    assert L.rv12_prefill_workspace_bytes(1000, 5) == 0 and L.rv12_prefill_workspace_bytes(1024, 0) == 0
    assert L.rv12_prefill_workspace_bytes(1024, (1 << 16) + 1) == 0
