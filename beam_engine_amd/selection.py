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
    """Device scratch for be_beam_topk, grown on demand and reused."""

    def __init__(self, device=None):
        self.device = torch.device(device) if device is not None else torch.device("cuda")
        self.buf = torch.empty(0, dtype=torch.uint8, device=self.device)

    def get(self, nbytes: int) -> torch.Tensor:
        if self.buf.numel() < nbytes:
            self.buf = torch.empty(max(nbytes, 2 * self.buf.numel()), dtype=torch.uint8, device=self.device)
        return self.buf


_default_ws = {}


def decode_k(beam_size: int, vocab: int) -> int:
    """Row k of a decode step (beam.py:275)."""
    return min(beam_size * 2, vocab) if beam_size != 1 else 1


def beam_topk(logits: torch.Tensor, k: int, parent_scores: Optional[torch.Tensor] = None, beam: int = 0,
              temperature: float = 1.0, workspace: Optional[TopkWorkspace] = None,
              request_rows: Optional[Sequence[int]] = None):
    """Row top-k of log_softmax(logits / T) and, when ``beam > 0``, the top-``beam``
    of ``parent_scores[r] + logp`` (float64) within every request.

    ``request_rows`` partitions the rows into consecutive requests (default:
    one request).  Returns ``(row_vals [N, k] f32, row_idx [N, k] i32)`` and, if
    beam > 0, ``(parent [R * beam] i32 global row, token [R * beam] i32,
    score [R * beam] f64)``; request q's entries are ``[q * beam, (q + 1) * beam)``
    in emission order (rows ascending, children in selection order), unused
    entries have parent -1."""
    lib = _lib.load()
    _lib.require_device(logits, "logits")
    if logits.dim() != 2:
        raise ValueError("logits must be [N, V]")
    if logits.stride(1) != 1:
        logits = logits.contiguous()
    n, v = logits.shape
    if temperature <= 0:
        raise ValueError("temperature must be positive")
    dev = logits.device
    inv_t = 1.0 if temperature == 1.0 else float(torch.tensor(1.0 / temperature, dtype=torch.float32))
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
        ps = parent_scores.to(device=dev, dtype=torch.float64).contiguous()
        if ps.numel() != n:
            raise ValueError("parent_scores must have one entry per row")
        if request_rows is not None:
            rows = [int(x) for x in request_rows]
            if sum(rows) != n or min(rows, default=0) < 0:
                raise ValueError("request_rows must partition the rows")
            n_req, max_rows = len(rows), max(rows)
            ptr_dev = torch.tensor(np.concatenate([[0], np.cumsum(rows)]).astype(np.int32)).to(dev)
        outs = (torch.empty(n_req * beam, dtype=torch.int32, device=dev),
                torch.empty(n_req * beam, dtype=torch.int32, device=dev),
                torch.empty(n_req * beam, dtype=torch.float64, device=dev))
    rc = lib.be_beam_topk(logits.data_ptr(), _lib.dtype_code(logits.dtype), n, v, logits.stride(0), inv_t, k,
                          _lib.ptr(ps), beam, n_req, _lib.ptr(ptr_dev), max_rows, row_vals.data_ptr(),
                          row_idx.data_ptr(), _lib.ptr(outs[0]), _lib.ptr(outs[1]), _lib.ptr(outs[2]),
                          buf.data_ptr(), buf.numel(), _lib.stream_ptr(dev))
    _lib.check(rc, "beam top-k")
    if beam > 0:
        return row_vals, row_idx, outs
    return row_vals, row_idx
