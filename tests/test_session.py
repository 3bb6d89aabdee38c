"""Host logic of DeviceSession (Session::prefill / step, src/engine.rs:120-145) on a
recording stand-in for the model: which positions are recomputed, in which chunks."""
import pytest

from wick_amd.session import CHUNK, DeviceSession


class _Cache:
    def __init__(self, capacity):
        self.capacity, self.len = capacity, 0

    def close(self):
        pass


class _Model:
    """Records every forward as (start position, tokens)."""

    def __init__(self):
        self.calls = []

    def new_cache(self, capacity):
        return _Cache(capacity)

    def forward(self, cache, tokens):
        self.calls.append((cache.len, list(tokens)))
        cache.len += len(tokens)
        return [[float(len(self.calls))]]


def test_prefix_reuse_keeps_common_prefix_and_chunks():
    m = _Model()
    s = DeviceSession(m, 1024)
    a = list(range(600))
    _, keep = s.prefill(a)
    assert keep == 0
    assert [(st, len(t)) for st, t in m.calls] == [(0, CHUNK), (CHUNK, CHUNK), (2 * CHUNK, 600 - 2 * CHUNK)]
    m.calls.clear()
    b = a[:450] + [7, 7, 7]
    _, keep = s.prefill(b)
    assert keep == 450 and m.calls == [(450, [7, 7, 7])]
    assert s.tokens == b and s.cache.len == 453


def test_same_prompt_recomputes_only_the_last_token():
    m = _Model()
    s = DeviceSession(m, 64)
    s.prefill([1, 2, 3, 4])
    m.calls.clear()
    _, keep = s.prefill([1, 2, 3, 4])
    assert keep == 3 and m.calls == [(3, [4])]


def test_step_appends_and_errors():
    m = _Model()
    s = DeviceSession(m, 8)
    s.prefill([5, 6])
    s.step(9)
    assert s.tokens == [5, 6, 9] and m.calls[-1] == (2, [9]) and len(s) == 3
    with pytest.raises(ValueError, match="empty"):
        s.prefill([])
    with pytest.raises(ValueError, match="context"):
        s.prefill(list(range(9)))
