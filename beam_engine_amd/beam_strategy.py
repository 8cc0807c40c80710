"""Beam strategies (src/beam_engine/beam_strategy.py).

``BeamStrategy`` keeps the reference's abstract interface (:8-58).
``VanillaBeamSearchStrategy`` keeps ``select_candidates`` / ``should_stop`` /
``get_final_sequences`` with the reference's semantics (:404-552) and adds
``select_from_logits``: the same selection computed on the GPU straight from
the logits (one HIP call, one transfer of B entries), which is what the decode
loop uses.  DiverseBeamSearchStrategy is not part of the decode hot path and
is not provided.
"""

from __future__ import annotations

from abc import ABC, abstractmethod
from typing import Dict, List, Optional, Tuple

import torch

from .beam_state import BeamGenerateInput, BeamGenerateResult, BeamState, BeamToken
from .selection import beam_topk, decode_k


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
                           rows: Optional[Tuple[int, int]] = None) -> List[BeamGenerateResult]:
        """GPU selection for the candidates ``rows = (begin, end)`` (default:
        all) of ``beam_state`` from their logits ``[end - begin, V]``."""
        cands = beam_state.candidates
        b, e = rows if rows is not None else (0, len(cands))
        sub = cands[b:e]
        if not sub:
            return []
        k = decode_k(beam_state.beam_size, logits.shape[-1])
        parents = torch.tensor([c.score for c in sub], dtype=torch.float64)
        _, _, (par, tok, sc) = beam_topk(logits, k, parents, beam_state.beam_size, temperature)
        par, tok, sc = par.tolist(), tok.tolist(), sc.tolist()
        per: List[List[BeamToken]] = [[] for _ in sub]
        for p, t, s in zip(par, tok, sc):
            if p >= 0:
                per[p].append(BeamToken(token_id=t, accumulated_score=s))
        return [BeamGenerateResult(candidate=c, children=per[i]) for i, c in enumerate(sub)]

    def select_batched(self, beam_state: BeamState, logits: torch.Tensor,
                       temperature: float = 1.0) -> List[BeamGenerateResult]:
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
        _, _, (par, tok, sc) = beam_topk(logits, k, parents, b, temperature, request_rows=rows, to_host=True)
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
