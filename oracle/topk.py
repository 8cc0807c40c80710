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

    x'   = round_dtype(x * fl32(fl64(1 / T)))      only when T != 1, mode "reciprocal"
    x'   = round_dtype(fl32(x / fl32(T)))          only when T != 1, mode "divide"

``logits / temperature`` (beam.py:107, :270) runs on a GPU tensor in the
reference; torch evaluates a tensor divided by a Python float on the GPU as a
multiply by the scalar's reciprocal, taken in double and rounded to float
(mode "reciprocal", the default), and on a CPU tensor as a correctly rounded
division by the float temperature (mode "divide").  Both forms are pinned
against torch itself: "divide" against torch's CPU division in the CPU
tests, "reciprocal" against torch's GPU division in the GPU tests (at T = 1.1
the two reciprocal roundings fl32(fl64(1 / T)) = 0x3F68BA2F and
fl32(1 / fl32(T)) = 0x3F68BA2E differ; the GPU gives the former).  The rest
of the row:

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


def scale_temperature(x: np.ndarray, dtype: str, temperature: float, mode: str = "reciprocal") -> np.ndarray:
    """``logits / temperature`` of beam.py:107, :270 (x already in the logits
    dtype, held as float32) in the arithmetic of ``mode``; T == 1 is skipped as
    the reference skips it."""
    x = np.asarray(x, dtype=np.float32)
    if temperature == 1.0:
        return x
    t = np.float32(temperature)
    if mode == "reciprocal":
        return round_dtype(x * np.float32(1.0 / float(temperature)), dtype)
    if mode == "divide":
        return round_dtype(x / t, dtype)
    raise ValueError(f"unknown temperature mode {mode}")


def log_softmax_rows(logits: np.ndarray, dtype: str = "float32", temperature: float = 1.0,
                     temperature_mode: str = "reciprocal") -> np.ndarray:
    """Row log_softmax under the pinned contract above; returns float32 values."""
    x = scale_temperature(logits, dtype, temperature, temperature_mode)
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
              temperature: float = 1.0, temperature_mode: str = "reciprocal"):
    """One full decode-step selection: log_softmax -> row top-k -> global top-B."""
    logp = log_softmax_rows(logits, dtype, temperature, temperature_mode)
    k = decode_k(beam_size, logp.shape[1])
    vals, idx = row_topk(logp, k)
    per_row, flat = select_global(parent_scores, vals, idx, beam_size)
    return logp, vals, idx, per_row, flat


def prefill_select(logits_row: np.ndarray, beam_size: int, dtype: str = "float32",
                   temperature: float = 1.0, temperature_mode: str = "reciprocal"):
    """Prefill expansion (beam.py:105-141): first B of topk(min(2B, V)) of one row."""
    logp = log_softmax_rows(np.asarray(logits_row)[None, :], dtype, temperature, temperature_mode)
    k = min(beam_size * 2, logp.shape[1])
    vals, idx = row_topk(logp, k)
    b = min(beam_size, k)
    return [(int(idx[0, j]), float(vals[0, j])) for j in range(b)]


def diverse_select(parent_scores, top_vals: np.ndarray, top_idx: np.ndarray, beam_size: int, num_groups: int,
                   diversity_penalty: float, diversity_type: str = "hamming", length_penalty: float = 1.0,
                   parent_sequences=None):
    """Diverse beam search selection (beam_strategy.py:173-312), restated step
    by step: the pool of (row, token, log_prob) choices in (row, rank) order is
    stably sorted by log_prob; group g (of ``num_groups``, ``max(1, B // G)``
    slots each) scores every not yet selected choice as
    ``(log_prob - penalty) / len ** length_penalty`` (``len`` = parent
    sequence length + 1; no division when the penalty exponent is 0), where
    the Hamming penalty applies to a token already chosen by an earlier group
    this step and the cumulative one is the mean positional overlap with the
    sequences chosen so far times the penalty; a stable sort picks the group's
    slots.  Children are regrouped per row (selection order) with
    ``parent_score + log_prob``; a total above B is cut from the last rows'
    last children.  ``parent_sequences[r]`` (token lists) are needed for the
    cumulative type and for ``len``; without them every parent has length 0.
    Returns ``(per_row_children, flat)`` as ``select_global``."""
    n, k = top_idx.shape
    bpg = max(1, beam_size // num_groups)
    seqs = parent_sequences if parent_sequences is not None else [[] for _ in range(n)]
    choices = [(r, int(top_idx[r, j]), float(top_vals[r, j])) for r in range(n) for j in range(k)]
    choices.sort(key=lambda c: c[2], reverse=True)                 # stable
    selected = []                                                  # (row, token) in selection order
    sel_keys = set()
    sel_tokens = set()
    sel_seqs = []
    for _ in range(num_groups):
        adjusted = []
        for r, tok, lp in choices:
            if (r, tok) in sel_keys:
                continue
            cand = list(seqs[r]) + [tok]
            if diversity_type == "hamming":
                pen = diversity_penalty if tok in sel_tokens else 0.0
            else:
                if sel_seqs:
                    tot = 0.0
                    for s in sel_seqs:
                        tot += sum(1 for a, b in zip(cand, s) if a == b) * diversity_penalty
                    pen = tot / len(sel_seqs)
                else:
                    pen = 0.0
            adj = lp - pen
            if length_penalty != 0:
                adj = adj / (len(cand) ** length_penalty)
            adjusted.append((r, tok, lp, adj))
        adjusted.sort(key=lambda c: c[3], reverse=True)            # stable
        for r, tok, lp, _ in adjusted[:bpg]:
            selected.append((r, tok, lp))
            sel_keys.add((r, tok))
            sel_tokens.add(tok)
            sel_seqs.append(list(seqs[r]) + [tok])
    per_row: List[List[Tuple[int, float]]] = [[] for _ in range(n)]
    for r, tok, lp in selected:
        per_row[r].append((tok, float(parent_scores[r]) + lp))
    extra = sum(len(c) for c in per_row) - beam_size
    for r in range(n - 1, -1, -1):
        while extra > 0 and per_row[r]:
            per_row[r].pop()
            extra -= 1
        if extra <= 0:
            break
    flat = [(r, tok, sc) for r in range(n) for tok, sc in per_row[r]]
    return per_row, flat
