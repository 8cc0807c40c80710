"""Beam token selection on the GPU (be_beam_topk).

Replaces the reference's per-step ``log_softmax`` + ``topk`` (beam.py:269-276),
the 2*N*2B ``.item()`` transfers (beam.py:282-302) and the Python sort of
``VanillaBeamSearchStrategy.select_candidates`` (beam_strategy.py:433-488)
with one HIP call and one small device-to-host copy.  Floating-point contract
and tie order: see ``include/beam_engine_amd.h`` (be_beam_topk).
"""

from __future__ import annotations

from typing import Optional, Sequence, Tuple

import numpy as np

import torch

from . import _lib


class TopkWorkspace:
    """Device scratch for be_beam_topk, grown on demand and reused (the call
    clears the arrival counters at its start, so the contents need no
    initialisation)."""

    def __init__(self, device=None):
        self.device = torch.device(device) if device is not None else torch.device("cuda")
        self.buf = torch.zeros(0, dtype=torch.uint8, device=self.device)

    def get(self, nbytes: int) -> torch.Tensor:
        if self.buf.numel() < nbytes:
            self.buf = torch.zeros(max(nbytes, 2 * self.buf.numel()), dtype=torch.uint8, device=self.device)
        return self.buf


_default_ws = {}


def decode_k(beam_size: int, vocab: int) -> int:
    """Row k of a decode step (beam.py:275)."""
    return min(beam_size * 2, vocab) if beam_size != 1 else 1


_row_ptrs = {}      # (device, request rows) -> device int32 row pointers
_pinned = {}        # (device, name) -> pinned host staging tensor


def _staging(dev, name, n, dtype):
    key = (dev.type, dev.index, name)
    t = _pinned.get(key)
    if t is None or t.numel() < n or t.dtype != dtype:
        t = _pinned[key] = torch.empty(max(n, 256), dtype=dtype, pin_memory=True)
    return t[:n]


_dev_outs = {}


def _selection_block(dev, m: int):
    """Device block (cached per device) holding a selection's parent (i32),
    token (i32) and score (f64) arrays back to back, and its pinned twin: one
    copy brings all three to the host.  Only for calls that synchronise before
    returning copies of the host views."""
    key = (dev.type, dev.index)
    a = (4 * m + 7) // 8 * 8
    nbytes = 2 * a + 8 * m
    blk = _dev_outs.get(key)
    if blk is None or blk[0].numel() < nbytes:
        blk = _dev_outs[key] = (torch.empty(max(nbytes, 4096), dtype=torch.uint8, device=dev),
                                torch.empty(max(nbytes, 4096), dtype=torch.uint8, pin_memory=True))
    d, h = blk

    def views(t):
        return (t[:4 * m].view(torch.int32), t[a:a + 4 * m].view(torch.int32), t[2 * a:2 * a + 8 * m].view(torch.float64))
    return d[:nbytes], h[:nbytes], views(d), views(h)


TEMPERATURE_MODES = {"reciprocal": _lib.BE_TEMP_RECIPROCAL, "divide": _lib.BE_TEMP_DIVIDE}


def beam_topk(logits: torch.Tensor, k: int, parent_scores: Optional[torch.Tensor] = None, beam: int = 0,
              temperature: float = 1.0, workspace: Optional[TopkWorkspace] = None,
              request_rows: Optional[Sequence[int]] = None, to_host: bool = False,
              temperature_mode: str = "reciprocal"):
    """Row top-k of log_softmax(logits / T) and, when ``beam > 0``, the top-``beam``
    of ``parent_scores[r] + logp`` (float64) within every request.

    ``logits / T`` (beam.py:107, :270) has the arithmetic of ``temperature_mode``:
    "reciprocal" multiplies by ``fl32(1.0 / T)`` (the reciprocal of the Python
    float taken in double, rounded to float) -- what torch computes for a GPU
    tensor divided by a Python float, i.e. the reference's own arithmetic --
    and "divide" divides by ``fl32(T)`` with correct rounding, as torch does
    for a CPU tensor.

    ``request_rows`` partitions the rows into consecutive requests (default:
    one request).  Returns ``(row_vals [N, k] f32, row_idx [N, k] i32)`` and, if
    beam > 0, ``(parent [R * beam] i32 global row, token [R * beam] i32,
    score [R * beam] f64)``; request q's entries are ``[q * beam, (q + 1) * beam)``
    in emission order (rows ascending, children in selection order), unused
    entries have parent -1.  ``to_host``: the selection outputs come back as
    CPU tensors through pinned staging with one synchronisation (host
    ``parent_scores`` go up the same way)."""
    lib = _lib.load()
    _lib.require_device(logits, "logits")
    if logits.dim() != 2:
        raise ValueError("logits must be [N, V]")
    if logits.stride(1) != 1:
        logits = logits.contiguous()
    n, v = logits.shape
    if not temperature > 0 or not np.isfinite(temperature):
        raise ValueError("temperature must be positive and finite")
    try:
        tmode = TEMPERATURE_MODES[temperature_mode]
    except KeyError:
        raise ValueError(f"temperature_mode must be one of {sorted(TEMPERATURE_MODES)}") from None
    dev = logits.device
    ws = workspace or _default_ws.setdefault((dev.type, dev.index), TopkWorkspace(dev))
    need = lib.be_beam_topk_workspace_bytes(n, v, k)
    buf = ws.get(need)
    row_vals = torch.empty((n, k), dtype=torch.float32, device=dev)
    row_idx = torch.empty((n, k), dtype=torch.int32, device=dev)
    outs = (None, None, None)
    ps = ptr_dev = None
    n_req, max_rows = 1, n
    if beam > 0:
        if parent_scores is None:
            raise ValueError("parent_scores are required when beam > 0")
        if parent_scores.device.type == "cpu" and to_host:
            # the staging buffer is free again once this call synchronises
            host = _staging(dev, "parents", parent_scores.numel(), torch.float64)
            host.copy_(parent_scores.reshape(-1))
            ps = host.to(dev, non_blocking=True)
        else:
            ps = parent_scores.to(device=dev, dtype=torch.float64).contiguous()
        if ps.numel() != n:
            raise ValueError("parent_scores must have one entry per row")
        if request_rows is not None:
            rows = tuple(int(x) for x in request_rows)
            if sum(rows) != n or min(rows, default=0) < 0:
                raise ValueError("request_rows must partition the rows")
            n_req, max_rows = len(rows), max(rows)
            key = (dev.type, dev.index, rows)
            ptr_dev = _row_ptrs.get(key)
            if ptr_dev is None:
                if len(_row_ptrs) > 64:
                    _row_ptrs.clear()
                ptr_dev = _row_ptrs[key] = torch.tensor(
                    np.concatenate([[0], np.cumsum(rows)]).astype(np.int32)).to(dev)
        if to_host:
            blk_dev, blk_host, outs, outs_host = _selection_block(dev, n_req * beam)
        else:
            outs = (torch.empty(n_req * beam, dtype=torch.int32, device=dev),
                    torch.empty(n_req * beam, dtype=torch.int32, device=dev),
                    torch.empty(n_req * beam, dtype=torch.float64, device=dev))
    rc = lib.be_beam_topk(logits.data_ptr(), _lib.dtype_code(logits.dtype), n, v, logits.stride(0),
                          float(temperature), tmode, k,
                          _lib.ptr(ps), beam, n_req, _lib.ptr(ptr_dev), max_rows, row_vals.data_ptr(),
                          row_idx.data_ptr(), _lib.ptr(outs[0]), _lib.ptr(outs[1]), _lib.ptr(outs[2]),
                          buf.data_ptr(), buf.numel(), _lib.stream_ptr(dev))
    _lib.check(rc, "beam top-k")
    if beam > 0:
        if to_host:
            blk_host.copy_(blk_dev, non_blocking=True)
            torch.cuda.current_stream(dev).synchronize()
            outs = tuple(t.clone() for t in outs_host)
        return row_vals, row_idx, outs
    return row_vals, row_idx


def diverse_select(row_vals: torch.Tensor, row_idx: torch.Tensor, parent_scores: torch.Tensor, beam: int,
                   num_groups: int, diversity_penalty: float, request_rows: Optional[Sequence[int]] = None,
                   to_host: bool = True):
    """Diverse beam search with the Hamming penalty over a row top-k already on
    the device (``row_vals [N, k]`` f32, ``row_idx [N, k]`` i32, as returned by
    ``beam_topk``): ``be_diverse_select`` per request.  Returns ``(parent,
    token, score)`` of ``R * beam`` entries (request q's at ``[q * beam, (q +
    1) * beam)``, grouped by row, unused entries parent -1); on the host with
    ``to_host`` (one synchronisation)."""
    lib = _lib.load()
    for t, nm in ((row_vals, "row_vals"), (row_idx, "row_idx")):
        _lib.require_device(t, nm)
    if row_vals.dim() != 2 or row_vals.shape != row_idx.shape:
        raise ValueError("row_vals and row_idx must be [N, k] of the same shape")
    if row_vals.dtype != torch.float32 or row_idx.dtype != torch.int32:
        raise ValueError("row_vals must be float32 and row_idx int32")
    n, k = row_vals.shape
    dev = row_vals.device
    row_vals, row_idx = row_vals.contiguous(), row_idx.contiguous()
    if parent_scores.numel() != n:
        raise ValueError("parent_scores must have one entry per row")
    if parent_scores.device.type == "cpu" and to_host:
        # the shared staging buffer is free again once this call synchronises
        host = _staging(dev, "dbs_parents", n, torch.float64)
        host.copy_(parent_scores.reshape(-1))
        ps = host.to(dev, non_blocking=True)
    elif parent_scores.device.type == "cpu":
        # no synchronisation at the end: a copy that completes before returning
        ps = parent_scores.reshape(-1).to(dtype=torch.float64).to(dev)
    else:
        ps = parent_scores.to(dtype=torch.float64).contiguous()
    n_req, max_rows, ptr_dev = 1, n, None
    if request_rows is not None:
        rows = tuple(int(x) for x in request_rows)
        if sum(rows) != n or min(rows, default=0) < 0:
            raise ValueError("request_rows must partition the rows")
        n_req, max_rows = len(rows), max(rows)
        key = (dev.type, dev.index, rows)
        ptr_dev = _row_ptrs.get(key)
        if ptr_dev is None:
            if len(_row_ptrs) > 64:
                _row_ptrs.clear()
            ptr_dev = _row_ptrs[key] = torch.tensor(np.concatenate([[0], np.cumsum(rows)]).astype(np.int32)).to(dev)
    outs = (torch.empty(n_req * beam, dtype=torch.int32, device=dev),
            torch.empty(n_req * beam, dtype=torch.int32, device=dev),
            torch.empty(n_req * beam, dtype=torch.float64, device=dev))
    rc = lib.be_diverse_select(row_vals.data_ptr(), row_idx.data_ptr(), n, k, ps.data_ptr(), n_req,
                               _lib.ptr(ptr_dev), max_rows, beam, num_groups, float(diversity_penalty),
                               outs[0].data_ptr(), outs[1].data_ptr(), outs[2].data_ptr(), _lib.stream_ptr(dev))
    _lib.check(rc, "diverse selection")
    if not to_host:
        return outs
    m = outs[0].numel()
    hp = _staging(dev, "dbs_parent", m, torch.int32)
    ht = _staging(dev, "dbs_token", m, torch.int32)
    hs = _staging(dev, "dbs_score", m, torch.float64)
    hp.copy_(outs[0], non_blocking=True)
    ht.copy_(outs[1], non_blocking=True)
    hs.copy_(outs[2], non_blocking=True)
    torch.cuda.current_stream(dev).synchronize()
    return hp.clone(), ht.clone(), hs.clone()
