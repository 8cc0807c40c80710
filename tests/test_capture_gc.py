"""Graph capture runs with Python's automatic garbage collection off.

A collection inside a HIP graph capture can release a pinned host block or an
event with calls that a capturing stream forbids, and the error raised in that
destructor aborts the process.  GraphedDecoder.capture collects once, turns
automatic collection off for the captured segments and restores it after.
torch's graph and stream calls are replaced by stand-ins (no GPU needed)."""

import contextlib
import gc
from types import SimpleNamespace

import torch

from beam_engine_amd import llama


class _Stream:
    def wait_stream(self, other):
        pass


def _decoder(layers, seen, fail_at=None):
    gd = llama.GraphedDecoder.__new__(llama.GraphedDecoder)
    gd.model = SimpleNamespace(cfg=SimpleNamespace(num_hidden_layers=layers))
    gd.tok = torch.full((4,), 7, dtype=torch.long)
    gd.pos = torch.full((4,), 9, dtype=torch.long)
    gd.wpg = torch.zeros(4, dtype=torch.int32)
    gd.wps = torch.zeros(4, dtype=torch.int32)
    gd._scratch_page = 3
    gd.graphs, gd.q = [], []

    def segment(l, x):
        seen.append(gc.isenabled())
        if fail_at is not None and len(seen) == fail_at:
            raise RuntimeError("segment failed")
        return x, None, (torch.zeros(1) if l == layers else None)

    gd._segment = segment
    return gd


def _stub_cuda(monkeypatch):
    monkeypatch.setattr(torch.cuda, "Stream", lambda *a, **k: _Stream())
    monkeypatch.setattr(torch.cuda, "stream", lambda s: contextlib.nullcontext())
    monkeypatch.setattr(torch.cuda, "current_stream", lambda *a, **k: _Stream())
    monkeypatch.setattr(torch.cuda, "synchronize", lambda *a, **k: None)
    monkeypatch.setattr(torch.cuda, "graph_pool_handle", lambda: None)
    monkeypatch.setattr(torch.cuda, "CUDAGraph", lambda: object())
    monkeypatch.setattr(torch.cuda, "graph", lambda g, pool=None: contextlib.nullcontext())


def test_capture_disables_automatic_gc(monkeypatch):
    _stub_cuda(monkeypatch)
    seen = []
    gd = _decoder(2, seen)
    assert gc.isenabled()
    gd.capture()
    # three warm-up segments with collection on, three captured with it off
    assert seen == [True] * 3 + [False] * 3
    assert gc.isenabled() and len(gd.graphs) == 3 and gd.wpg.tolist() == [3] * 4
    # the warm-up pass reads valid inputs: token 0 at position 0
    assert gd.tok.tolist() == [0] * 4 and gd.pos.tolist() == [0] * 4


def test_capture_restores_gc_after_an_error(monkeypatch):
    _stub_cuda(monkeypatch)
    seen = []
    gd = _decoder(2, seen, fail_at=5)
    try:
        gd.capture()
    except RuntimeError:
        pass
    else:
        raise AssertionError("the segment error must propagate")
    assert seen == [True] * 3 + [False] * 2 and gc.isenabled()
