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
    """Ten bytes per column and token (three bf16 parts and the transposed
    fp32 x'), tokens padded to 128, plus a scale exponent and an RMS factor per
    padded token; with a K split, a float per split, padded token and row for
    the partial sums: none for the Qwen3-8B gu and o over 2048 tokens (six
    rounds of workgroups, one full round), between 2 and 16 splits for the o
    matrix over 256 tokens (32 workgroups); 0 for bad arguments."""
    from ai_amd import _lib
    L = _lib.lib()
    base = lambda k, tp: tp * k * 10 + tp * 8
    assert L.rv12_prefill_workspace_bytes(24576, 4096, 2048) == base(4096, 2048)
    assert L.rv12_prefill_workspace_bytes(4096, 4096, 2048) == base(4096, 2048)
    extra = L.rv12_prefill_workspace_bytes(4096, 4096, 256) - base(4096, 256)
    assert extra % (256 * 4096 * 4) == 0 and 2 <= extra // (256 * 4096 * 4) <= 16
    assert L.rv12_prefill_workspace_bytes(300, 1024, 300) >= base(1024, 384)
    assert L.rv12_prefill_workspace_bytes(300, 1000, 5) == 0 and L.rv12_prefill_workspace_bytes(300, 1024, 0) == 0
    assert L.rv12_prefill_workspace_bytes(0, 1024, 5) == 0
    assert L.rv12_prefill_workspace_bytes(300, 1024, (1 << 16) + 1) == 0