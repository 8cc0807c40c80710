"""CPU restatement of the reference's beam token selection (test infrastructure).

Reference path (src/beam_engine/):

* decode: ``logits / temperature`` (when temperature != 1), ``log_softmax``,
  ``topk(k)`` per row with ``k = min(2B, V)`` or 1 when B == 1
  (beam.py:269-276); ``.item()`` turns every value into a Python float
  (beam.py:296-300);
* ``VanillaBeamSearchStrategy.select_candidates`` (beam_strategy.py:433-488):
  ``total = parent_score + log_prob`` in Python float64, a stable
  ``sort(reverse=True)`` over the flattened (row, rank) pool, the first B
  kept, then regrouped per parent row in row order with each row's children
  in selection order;
* prefill: one row, ``topk(min(2B, V))`` and the first B kept (beam.py:105-141).

Floating-point contract restated here and implemented bit-for-bit by the GPU
kernel (torch's own reduction order is unspecified, so this is the pinned
form): for a row x (already in the logits dtype),

    x'   = round_dtype(x * fl32(1/T))          only when T != 1
    m    = max(x')
    S    = sum_i exp(fl64(x'_i - m))            float64 accumulation
    L    = fl32(ln S)
    logp = fl32(fl32(x'_i - m) - L)             then round_dtype for fp16/bf16 logits

This is the structure of torch's log_softmax epilogue (input - max - logsum in
the accumulate type, output in the input dtype).  Ties are broken by lower
vocabulary index within a row and by lower (row, rank) position in the pool.
"""

from __future__ import annotations

from typing import List, Tuple

import numpy as np


def round_bf16(x: np.ndarray) -> np.ndarray:
    """Round float32 values to bfloat16 (round-to-nearest-even), returned as float32."""
    x = np.asarray(x, dtype=np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    nan = np.isnan(x)
    lsb = (u >> 16) & 1
    r = ((u + 0x7FFF + lsb) >> 16) << 16
    out = (r & 0xFFFFFFFF).astype(np.uint32).view(np.float32)
    return np.where(nan, x, out).astype(np.float32)


def round_dtype(x: np.ndarray, dtype: str) -> np.ndarray:
    if dtype == "float32":
        return np.asarray(x, dtype=np.float32)
    if dtype == "bfloat16":
        return round_bf16(x)
    if dtype == "float16":
        return np.asarray(x, dtype=np.float32).astype(np.float16).astype(np.float32)
    raise ValueError(f"unsupported logits dtype {dtype}")


def log_softmax_rows(logits: np.ndarray, dtype: str = "float32", temperature: float = 1.0) -> np.ndarray:
    """Row log_softmax under the pinned contract above; returns float32 values."""
    x = np.asarray(logits, dtype=np.float32)
    if temperature != 1.0:
        inv_t = np.float32(1.0 / temperature)
        x = round_dtype(x * inv_t, dtype)
    m = x.max(axis=1, keepdims=True)
    s = np.exp(x.astype(np.float64) - m.astype(np.float64)).sum(axis=1, keepdims=True)
    lse_off = np.log(s).astype(np.float32)
    logp = (x - m).astype(np.float32) - lse_off
    return round_dtype(logp.astype(np.float32), dtype)


def row_topk(logp: np.ndarray, k: int) -> Tuple[np.ndarray, np.ndarray]:
    """Per-row top-k by (value desc, index asc).  Returns (values f32, indices i64)."""
    n, v = logp.shape
    idx = np.empty((n, k), dtype=np.int64)
    val = np.empty((n, k), dtype=np.float32)
    cols = np.arange(v)
    for r in range(n):
        order = np.lexsort((cols, -logp[r].astype(np.float64)))[:k]
        idx[r] = order
        val[r] = logp[r, order]
    return val, idx


def decode_k(beam_size: int, vocab: int) -> int:
    """Per-row k of the decode step (beam.py:275)."""
    return min(beam_size * 2, vocab) if beam_size != 1 else 1


def select_global(parent_scores, top_vals: np.ndarray, top_idx: np.ndarray, beam_size: int):
    """Vanilla global selection (beam_strategy.py:433-488).

    Returns ``(per_row_children, flat)`` where ``per_row_children[r]`` is a list
    of ``(token, total_score)`` and ``flat`` the emission-ordered list of
    ``(row, token, total_score)`` (rows ascending, children in selection order).
    """
    pool = []
    n, k = top_idx.shape
    for r in range(n):
        ps = float(parent_scores[r])
        for j in range(k):
            pool.append((r, int(top_idx[r, j]), ps + float(top_vals[r, j])))
    pool.sort(key=lambda t: t[2], reverse=True)        # Python's sort is stable
    chosen = pool[:beam_size]
    per_row: List[List[Tuple[int, float]]] = [[] for _ in range(n)]
    for r, tok, sc in chosen:
        per_row[r].append((tok, sc))
    flat = [(r, tok, sc) for r in range(n) for tok, sc in per_row[r]]
    return per_row, flat


def beam_step(logits: np.ndarray, parent_scores, beam_size: int, dtype: str = "float32",
              temperature: float = 1.0):
    """One full decode-step selection: log_softmax -> row top-k -> global top-B."""
    logp = log_softmax_rows(logits, dtype, temperature)
    k = decode_k(beam_size, logp.shape[1])
    vals, idx = row_topk(logp, k)
    per_row, flat = select_global(parent_scores, vals, idx, beam_size)
    return logp, vals, idx, per_row, flat


def prefill_select(logits_row: np.ndarray, beam_size: int, dtype: str = "float32",
                   temperature: float = 1.0):
    """Prefill expansion (beam.py:105-141): first B of topk(min(2B, V)) of one row."""
    logp = log_softmax_rows(np.asarray(logits_row)[None, :], dtype, temperature)
    k = min(beam_size * 2, logp.shape[1])
    vals, idx = row_topk(logp, k)
    b = min(beam_size, k)
    return [(int(idx[0, j]), float(vals[0, j])) for j in range(b)]
