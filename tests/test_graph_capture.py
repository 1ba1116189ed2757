"""Host logic of the graph runners' capture helper (CPU, no graph is made):
Python's cyclic garbage collector is off while a capture is open -- a
collection there could destroy the graphs and graph memory pools of dead
runners inside the capture -- and is restored afterwards, also when the
captured call raises; a caller that had it off keeps it off."""

from __future__ import annotations

import contextlib
import gc

import pytest
import torch

from umic import graph


class _FakeGraph:
    def pool(self):
        return None


@pytest.fixture
def fake_capture(monkeypatch):
    monkeypatch.setattr(torch.cuda, "CUDAGraph", _FakeGraph)
    monkeypatch.setattr(torch.cuda, "graph", lambda g, pool=None: contextlib.nullcontext())


def test_capture_holds_the_collector_off(fake_capture):
    assert gc.isenabled()
    seen = []
    _, out = graph._capture(lambda: seen.append(gc.isenabled()) or 7, warm=False)
    assert out == 7 and seen == [False]
    assert gc.isenabled()


def test_capture_restores_the_collector_when_the_call_raises(fake_capture):
    def boom():
        raise RuntimeError("capture failed")

    with pytest.raises(RuntimeError):
        graph._capture(boom, warm=False)
    assert gc.isenabled()


def test_capture_keeps_a_disabled_collector_disabled(fake_capture):
    gc.disable()
    try:
        graph._capture(lambda: None, warm=False)
        assert not gc.isenabled()
    finally:
        gc.enable()
