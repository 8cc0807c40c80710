"""Beam strategies (src/beam_engine/beam_strategy.py).

``BeamStrategy`` keeps the reference's abstract interface (:8-58).
``VanillaBeamSearchStrategy`` keeps ``select_candidates`` / ``should_stop`` /
``get_final_sequences`` with the reference's semantics (:404-552) and adds
``select_from_logits``: the same selection computed on the GPU straight from
the logits (one HIP call, one transfer of B entries), which is what the decode
loop uses.  ``DiverseBeamSearchStrategy`` keeps the reference's diverse beam
search (:60-400) with the same selection, and selects on the GPU from the
logits for the Hamming penalty (``be_diverse_select``).
"""

from __future__ import annotations

from abc import ABC, abstractmethod
from typing import Dict, List, Optional, Tuple

import torch

from .beam_state import (BeamCandidate, BeamGenerateInput, BeamGenerateResult, BeamState, BeamToken,
                         BeamTokenCandidate)
from .selection import beam_topk, decode_k, diverse_select


class BeamStrategy(ABC):
    @abstractmethod
    def select_candidates(self, beam_state: BeamState, new_candidates: List[BeamGenerateInput],
                          step: int) -> List[BeamGenerateResult]:
        ...

    @abstractmethod
    def should_stop(self, beam_state: BeamState, max_length: int, step: int) -> bool:
        ...

    @abstractmethod
    def get_final_sequences(self, beam_state: BeamState,
                            num_return: Optional[int] = None) -> List[Tuple[List[int], float]]:
        ...


class VanillaBeamSearchStrategy(BeamStrategy):
    def __init__(self, length_penalty: float = 1.0, early_stopping: bool = True):
        self.length_penalty = length_penalty
        self.early_stopping = early_stopping

    def _apply_length_penalty(self, log_prob: float, length: int) -> float:
        if self.length_penalty == 0 or length <= 1:
            return log_prob
        return log_prob / (length ** self.length_penalty)

    def select_candidates(self, beam_state: BeamState, new_candidates: List[BeamGenerateInput],
                          step: int) -> List[BeamGenerateResult]:
        """Global top-B over (parent score + log_prob) in float64, stable order
        (beam_strategy.py:433-488), regrouped per parent in input order."""
        if not new_candidates:
            return []
        pool = []
        for idx, inp in enumerate(new_candidates):
            base = inp.candidate.score
            for tok in inp.children:
                pool.append((idx, tok.token_id, base + tok.log_prob))
        pool.sort(key=lambda t: t[2], reverse=True)
        per: Dict[int, List[BeamToken]] = {i: [] for i in range(len(new_candidates))}
        for idx, tok, total in pool[:beam_state.beam_size]:
            per[idx].append(BeamToken(token_id=tok, accumulated_score=total))
        return [BeamGenerateResult(candidate=inp.candidate, children=per[i])
                for i, inp in enumerate(new_candidates)]

    def select_from_logits(self, beam_state: BeamState, logits: torch.Tensor, temperature: float = 1.0,
                           rows: Optional[Tuple[int, int]] = None,
                           temperature_mode: str = "reciprocal") -> List[BeamGenerateResult]:
        """GPU selection for the candidates ``rows = (begin, end)`` (default:
        all) of ``beam_state`` from their logits ``[end - begin, V]``."""
        cands = beam_state.candidates
        b, e = rows if rows is not None else (0, len(cands))
        sub = cands[b:e]
        if not sub:
            return []
        k = decode_k(beam_state.beam_size, logits.shape[-1])
        parents = torch.tensor([c.score for c in sub], dtype=torch.float64)
        _, _, (par, tok, sc) = beam_topk(logits, k, parents, beam_state.beam_size, temperature,
                                         temperature_mode=temperature_mode)
        par, tok, sc = par.tolist(), tok.tolist(), sc.tolist()
        per: List[List[BeamToken]] = [[] for _ in sub]
        for p, t, s in zip(par, tok, sc):
            if p >= 0:
                per[p].append(BeamToken(token_id=t, accumulated_score=s))
        return [BeamGenerateResult(candidate=c, children=per[i]) for i, c in enumerate(sub)]

    def select_batched(self, beam_state: BeamState, logits: torch.Tensor, temperature: float = 1.0,
                       temperature_mode: str = "reciprocal") -> List[BeamGenerateResult]:
        """GPU selection for every request of a multi-request state in one
        call: candidates of one request are consecutive; ``logits [N, V]``."""
        cands = beam_state.candidates
        if not cands:
            return []
        rows = []
        for i, c in enumerate(cands):
            if i == 0 or c.request_id != cands[i - 1].request_id:
                rows.append(0)
            rows[-1] += 1
        k = decode_k(beam_state.beam_size, logits.shape[-1])
        parents = torch.tensor([c.score for c in cands], dtype=torch.float64)
        b = beam_state.beam_size
        _, _, (par, tok, sc) = beam_topk(logits, k, parents, b, temperature, request_rows=rows, to_host=True,
                                         temperature_mode=temperature_mode)
        per: List[List[BeamToken]] = [[] for _ in cands]
        for p, t, s_ in zip(par.tolist(), tok.tolist(), sc.tolist()):
            if p >= 0:
                per[p].append(BeamToken(token_id=t, accumulated_score=s_))
        return [BeamGenerateResult(candidate=c, children=per[i]) for i, c in enumerate(cands)]

    def should_stop(self, beam_state: BeamState, max_length: int, step: int) -> bool:
        """beam_strategy.py:490-517."""
        if step >= max_length:
            return True
        if not beam_state.candidates:
            return True
        if self.early_stopping and len(beam_state.finished_candidates) >= beam_state.beam_size:
            return True
        if all(c.finished for c in beam_state.candidates):
            return True
        return False

    def get_final_sequences(self, beam_state: BeamState, num_return: Optional[int] = None,
                            request_id: Optional[int] = None) -> List[Tuple[List[int], float]]:
        if num_return is None:
            num_return = beam_state.beam_size
        return beam_state.get_final_sequences(num_return, self.length_penalty, request_id)

    def finalize_scores(self, candidates: List[BeamCandidate], step: int) -> List[Tuple[BeamCandidate, float]]:
        """(candidate, score / step^length_penalty) pairs, highest first, the
        length being the ``step`` the caller passes (beam_strategy.py:539-552;
        unchanged when the penalty is 0 or step <= 1; ties keep input order)."""
        scored = [(c, self._apply_length_penalty(c.score, step)) for c in candidates]
        return sorted(scored, key=lambda x: x[1], reverse=True)


class DiverseBeamSearchStrategy(BeamStrategy):
    """Diverse beam search (beam_strategy.py:60-400; Vijayakumar et al. 2018).

    ``select_candidates`` restates the reference's selection exactly: the pool
    of every candidate's children in input order, stably sorted by log_prob;
    each of ``num_groups`` groups takes ``max(1, B // num_groups)`` choices not
    taken yet, by ``(log_prob - penalty) / len ** length_penalty`` (stable),
    where the Hamming penalty applies to a token an earlier group took this
    step and the cumulative one is the mean positional overlap with the
    sequences taken so far times ``diversity_penalty``; the picks return per
    candidate in pick order with ``parent score + log_prob``, and a total above
    B is cut from the last candidates' last children (:173-312).
    ``select_from_logits`` / ``select_batched`` compute it from the logits on
    the GPU (row top-k, then ``be_diverse_select``) for the Hamming type; the
    cumulative type, which needs whole sequences, takes the row top-k to the
    host and runs ``select_candidates``."""

    def __init__(self, num_groups: int = 4, diversity_penalty: float = 0.5, diversity_type: str = "hamming",
                 length_penalty: float = 1.0, early_stopping: bool = True):
        if diversity_type not in ("hamming", "cumulative"):
            raise ValueError(f"diversity_type must be 'hamming' or 'cumulative', got {diversity_type!r}")
        if num_groups < 1:
            raise ValueError("num_groups must be positive")
        self.num_groups = num_groups
        self.diversity_penalty = diversity_penalty
        self.diversity_type = diversity_type
        self.length_penalty = length_penalty
        self.early_stopping = early_stopping

    @staticmethod
    def _sequence(node) -> List[int]:
        """Tokens from the root to ``node`` (beam_strategy.py:97-104)."""
        parts = []
        while node is not None and node.tokens:
            parts.append(node.tokens)
            node = node.parent
        return [t for part in reversed(parts) for t in part]

    def _apply_length_penalty(self, score: float, length: int) -> float:
        if self.length_penalty == 0:
            return score
        return score / (length ** self.length_penalty)

    def select_candidates(self, beam_state: BeamState, new_candidates: List[BeamGenerateInput],
                          step: int) -> List[BeamGenerateResult]:
        if not new_candidates:
            return []
        per = max(1, beam_state.beam_size // self.num_groups)
        seqs = [self._sequence(inp.candidate.trie_node) for inp in new_candidates]
        choices = [(i, tc.token_id, tc.log_prob) for i, inp in enumerate(new_candidates) for tc in inp.children]
        choices.sort(key=lambda c: c[2], reverse=True)
        taken = set()
        taken_tokens = set()
        taken_seqs: List[List[int]] = []
        picks: List[Tuple[int, int, float]] = []
        for _ in range(self.num_groups):
            adjusted = []
            for i, tok, lp in choices:
                if (i, tok) in taken:
                    continue
                length = len(seqs[i]) + 1
                if self.diversity_type == "hamming":
                    pen = self.diversity_penalty if tok in taken_tokens else 0.0
                elif taken_seqs:
                    cand = seqs[i] + [tok]
                    pen = sum(sum(1 for a, b in zip(cand, s) if a == b) * self.diversity_penalty
                              for s in taken_seqs) / len(taken_seqs)
                else:
                    pen = 0.0
                adjusted.append((i, tok, lp, self._apply_length_penalty(lp - pen, length)))
            adjusted.sort(key=lambda c: c[3], reverse=True)
            for i, tok, lp, _ in adjusted[:per]:
                picks.append((i, tok, lp))
                taken.add((i, tok))
                taken_tokens.add(tok)
                taken_seqs.append(seqs[i] + [tok])
        children: List[List[BeamToken]] = [[] for _ in new_candidates]
        for i, tok, lp in picks:
            children[i].append(BeamToken(token_id=tok, accumulated_score=new_candidates[i].candidate.score + lp))
        extra = sum(len(c) for c in children) - beam_state.beam_size
        for c in reversed(children):
            while extra > 0 and c:
                c.pop()
                extra -= 1
            if extra <= 0:
                break
        return [BeamGenerateResult(candidate=inp.candidate, children=children[i])
                for i, inp in enumerate(new_candidates)]

    def _rows_to_results(self, cands, par, tok, sc, offset: int = 0) -> List[BeamGenerateResult]:
        per: List[List[BeamToken]] = [[] for _ in cands]
        for p, t, s_ in zip(par.tolist(), tok.tolist(), sc.tolist()):
            if p >= 0:
                per[p - offset].append(BeamToken(token_id=t, accumulated_score=s_))
        return [BeamGenerateResult(candidate=c, children=per[i]) for i, c in enumerate(cands)]

    def select_from_logits(self, beam_state: BeamState, logits: torch.Tensor, temperature: float = 1.0,
                           rows: Optional[Tuple[int, int]] = None,
                           temperature_mode: str = "reciprocal") -> List[BeamGenerateResult]:
        """Selection for the candidates ``rows = (begin, end)`` (default: all)
        of ``beam_state`` from their logits ``[end - begin, V]``."""
        cands = beam_state.candidates
        b, e = rows if rows is not None else (0, len(cands))
        sub = cands[b:e]
        if not sub:
            return []
        k = decode_k(beam_state.beam_size, logits.shape[-1])
        vals, idx = beam_topk(logits, k, temperature=temperature, temperature_mode=temperature_mode)
        if self.diversity_type != "hamming":
            v, ix = vals.cpu().tolist(), idx.cpu().tolist()
            inputs = [BeamGenerateInput(c, [BeamTokenCandidate(int(t), float(x)) for t, x in zip(ix[r], v[r])])
                      for r, c in enumerate(sub)]
            return self.select_candidates(beam_state, inputs, 0)
        parents = torch.tensor([c.score for c in sub], dtype=torch.float64)
        par, tok, sc = diverse_select(vals, idx, parents, beam_state.beam_size, self.num_groups,
                                      self.diversity_penalty)
        return self._rows_to_results(sub, par, tok, sc)

    def select_batched(self, beam_state: BeamState, logits: torch.Tensor, temperature: float = 1.0,
                       temperature_mode: str = "reciprocal") -> List[BeamGenerateResult]:
        """Selection for every request of a multi-request state (its candidates
        consecutive per request; ``logits [N, V]``), each request on its own."""
        cands = beam_state.candidates
        if not cands:
            return []
        if self.diversity_type != "hamming":
            out, b = [], 0
            while b < len(cands):
                e = b
                while e < len(cands) and cands[e].request_id == cands[b].request_id:
                    e += 1
                out += self.select_from_logits(beam_state, logits[b:e], temperature, rows=(b, e),
                                               temperature_mode=temperature_mode)
                b = e
            return out
        rows = []
        for i, c in enumerate(cands):
            if i == 0 or c.request_id != cands[i - 1].request_id:
                rows.append(0)
            rows[-1] += 1
        k = decode_k(beam_state.beam_size, logits.shape[-1])
        vals, idx = beam_topk(logits, k, temperature=temperature, temperature_mode=temperature_mode)
        parents = torch.tensor([c.score for c in cands], dtype=torch.float64)
        par, tok, sc = diverse_select(vals, idx, parents, beam_state.beam_size, self.num_groups,
                                      self.diversity_penalty, request_rows=rows)
        return self._rows_to_results(cands, par, tok, sc)

    def should_stop(self, beam_state: BeamState, max_length: int, step: int) -> bool:
        """beam_strategy.py:346-379."""
        if step >= max_length:
            return True
        if self.early_stopping:
            if not beam_state.candidates:
                return True
            if all(c.finished for c in beam_state.candidates):
                return True
        if len(beam_state.finished_candidates) >= beam_state.beam_size:
            return True
        return False

    def get_final_sequences(self, beam_state: BeamState, num_return: Optional[int] = None,
                            request_id: Optional[int] = None) -> List[Tuple[List[int], float]]:
        if num_return is None:
            num_return = beam_state.beam_size
        return beam_state.get_final_sequences(num_return, self.length_penalty, request_id)

    def get_diverse_groups(self, beam_state: BeamState) -> List[List[BeamCandidate]]:
        """Candidates (finished first, then live) by score, cut into the groups
        (beam_strategy.py:381-400)."""
        per = max(1, beam_state.beam_size // self.num_groups)
        allc = beam_state.finished_candidates + beam_state.candidates
        allc.sort(key=lambda x: x.score, reverse=True)
        return [allc[i * per: min(i * per + per, len(allc))] for i in range(self.num_groups) if i * per < len(allc)]
