"""Batched beam-search decode loop over the HIP path.

Restates the reference's driver (src/beam_engine/beam.py:48-352) for several
requests decoded together in one forward per step:

* prefill: prompt pages allocated per request (``add_root_sequence``), one
  batched prefill, then each request's first B tokens of top-2B of the last
  position (beam.py:105-141) expand its root;
* per step (beam.py:145-317): cascade (or flat) metadata from the trie, the
  write location and position of every candidate, one decode forward with the
  attention plan built once and reused by every layer (the reference builds a
  FlashInfer wrapper per step, models/modeling_llama.py:732-755), GPU beam
  selection per request (log_softmax + top-2B + global top-B), trie update
  with the step's fork copies in one launch.

``kernel_type``: "cascade" (per-level groups of the reference's
get_cascade_input), "flat" (each candidate's whole path, the baseline),
"tree" (the path attention as shared passes over trie segments, each edge
absorbed or split by the MI355X cost model, as FastTree's preparation decides
them, attention/fasttree/preparation.py:60-105) or "auto" (per step, the
cheaper of flat, fully split and tree under that model).  "flat", "tree" and
"auto" give every candidate its path tokens exactly once; "cascade" keeps the
reference's repetition of a shallow candidate's leaf group on deeper levels.
``include_self`` False follows the reference's cascade convention (a query
does not attend to the K/V it appends in the same step, beam_state.py:347-354).
``eos_token_id`` (off by default, as in the reference, which never finishes a
beam): a pick of that token finishes its beam (``state.finished_candidates``)
and the request continues with its other beams; steps whose candidate count
differs from the captured one run eagerly.
"""

from __future__ import annotations

import time
from typing import List, Optional, Sequence

import numpy as np
import torch

from .attention import BatchDecodeWithPagedKVCacheWrapper, MultiLevelCascadeAttentionWrapper
from .beam_state import BeamGenerateResult, BeamState, BeamToken
from .beam_strategy import VanillaBeamSearchStrategy
from .page_table import PageTable
from .selection import beam_topk


class BatchedBeamSearch:
    def __init__(self, model, page_table: PageTable, beam_size: int,
                 strategy: Optional[VanillaBeamSearchStrategy] = None, kernel_type: str = "cascade",
                 temperature: float = 1.0, workspace_bytes: int = 256 << 20, include_self: bool = False,
                 graphs: bool = False, eos_token_id: Optional[int] = None, temperature_mode: str = "reciprocal",
                 picker_costs: str = "mi355x"):
        if kernel_type not in ("cascade", "flat", "tree", "auto"):
            raise ValueError(f"Unknown kernel_type: {kernel_type}. Must be 'cascade', 'flat', 'tree' or 'auto'.")
        self.model = model
        self.pt = page_table
        self.beam_size = beam_size
        self.strategy = strategy or VanillaBeamSearchStrategy()
        self.kernel_type = kernel_type
        self.temperature = temperature
        self.temperature_mode = temperature_mode   # arithmetic of logits / T: see selection.beam_topk
        self.include_self = include_self
        self.eos_token_id = eos_token_id    # a pick of this token finishes its beam (off: None)
        self.device = page_table.device
        self.state = BeamState(beam_size, page_table, fast_metadata=True)
        self.ws = torch.empty(workspace_bytes, dtype=torch.uint8, device=self.device)
        self.cascade = MultiLevelCascadeAttentionWrapper(1, self.ws)
        self.flat = BatchDecodeWithPagedKVCacheWrapper(self.ws)
        self.last_attn = None
        self.picker = None
        self.picker_costs = picker_costs    # "mi355x" fitted costs or "fasttree" (the reference's edge model)
        self.step_log: List[dict] = []
        self._staging = torch.empty(4 * 4096, dtype=torch.int64, pin_memory=True)
        self.attn_timer = None          # optional callable(layer, fn) used by benchmarks
        self.graphs = graphs            # capture the non-attention work of a step in HIP graphs
        self._gd = None

    # ---------------------------------------------------------------- prefill
    @torch.no_grad()
    def prefill(self, prompts: Sequence[Sequence[int]]) -> torch.Tensor:
        if len({len(p) for p in prompts}) != 1:
            raise ValueError("batched prefill needs prompts of equal length")
        page_ids = []
        for r, p in enumerate(prompts):
            nodes = self.state.add_root_sequence(list(p), request_id=r)
            page_ids.append([n.page_id for n in nodes])
        ids = torch.tensor([list(p) for p in prompts], dtype=torch.long, device=self.device)
        logits = self.model.prefill(ids, self.pt, page_ids)
        results = []
        k = min(2 * self.beam_size, logits.shape[-1])
        vals, idx = beam_topk(logits, k, temperature=self.temperature, temperature_mode=self.temperature_mode)
        self.pt.stage_errors()
        vals, idx = vals[:, : self.beam_size].tolist(), idx[:, : self.beam_size].tolist()
        self.pt.raise_staged_errors()          # the prompt's KV writes (ValueError on a bad page)
        for r, cand in enumerate(self.state.candidates):
            results.append(BeamGenerateResult(cand, [BeamToken(int(t), float(s)) for t, s in zip(idx[r], vals[r])]))
        self.state.add_filtered_results(results)
        return logits

    # ---------------------------------------------------------------- decode
    def _get_picker(self):
        if self.picker is None:
            from .picker import MI355X, StrategyPicker
            cfg = self.model.cfg
            costs = "fasttree" if self.picker_costs == "fasttree" else MI355X
            self.picker = StrategyPicker(cfg.num_attention_heads, cfg.num_key_value_heads, self.pt.page_size, costs)
        return self.picker

    def _plan(self, kind: str, levels=None):
        m = self.model
        cfg = m.cfg
        st = self.state
        if kind != "flat" or levels is not None:
            if levels is None:
                levels = st._cascade_lists()
            if self.include_self:
                raise NotImplementedError("include_self with cascade or tree levels")
            w = MultiLevelCascadeAttentionWrapper(len(levels), self.ws)
            w.plan([l[0] for l in levels], [l[1] for l in levels], [l[2] for l in levels], [l[3] for l in levels],
                   cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim, self.pt.page_size,
                   causal=kind == "cascade", q_data_type=m.dtype)
        else:
            kvp, kvi, lpl = st.flat_lists(self.include_self)
            w = self.flat
            w.plan(kvp, kvi, lpl, cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim,
                   self.pt.page_size, q_data_type=m.dtype)
        self.last_attn = w
        return w

    @torch.no_grad()
    def step(self) -> None:
        st = self.state
        n = len(st.candidates)
        if n == 0:                  # every beam finished
            return
        kind = self.kernel_type
        levels = None
        if kind == "cascade":
            # the cascade arrays and the candidates' inputs from the native builder
            levels, qids, wp, wpos, pos = st.step_metadata()
        else:
            if kind == "tree":
                p = self._get_picker()
                levels = st.tree_lists((p.edges or p.model).absorb)
            elif kind == "auto":
                plan = self._get_picker().choose(st)
                kind, levels = plan.kind, plan.levels
        w = self._plan(kind, levels)
        if self.kernel_type != "cascade":
            qids = st.query_token_ids()
            wp, wpos = st.write_locations()
            pos = st.position_ids(reuse_annotation=True)     # _plan's metadata pass just ran
        if self._staging.numel() < 4 * n:
            self._staging = torch.empty(8 * n, dtype=torch.int64, pin_memory=True)
        stg = self._staging[: 4 * n].view(4, n)
        for i, v in enumerate((qids, wp, wpos, pos)):
            stg[i] = torch.from_numpy(v) if isinstance(v, np.ndarray) else torch.tensor(v)
        dev = stg.to(self.device, non_blocking=True)
        tok, wpg, wps, psn = dev[0], dev[1].to(torch.int32), dev[2].to(torch.int32), dev[3]

        timer = self.attn_timer

        def attn(li, q, kv, out=None):
            if timer is None:
                return w.run(q, kv, out=out)
            return timer(li, lambda between: w.run(q, kv, out=out, between=between), w)

        if self.graphs and hasattr(self.model, "decode") and self._graph_ready(n):
            self._gd.load_inputs(tok, psn, wpg, wps)
            logits = self._gd.run(attn)
        else:
            logits = self.model.decode(tok, psn, wpg, wps, self.pt, attn)
        self._select(logits)
        self.step_log.append({"n": n, "kind": kind})

    def prepare_graphs(self) -> None:
        """Capture the segment graphs now for the current candidate count (the
        first decode step would otherwise capture them)."""
        if self.graphs and hasattr(self.model, "decode") and self.state.candidates:
            self._graph_ready(len(self.state.candidates))

    def _graph_ready(self, n: int) -> bool:
        """Capture the segment graphs once the candidate count is known (it
        stays B per request); a different count runs eagerly."""
        from .llama import GraphedDecoder
        if self._gd is None:
            self._gd = GraphedDecoder(self.model, self.pt, n)
            self._gd.capture()
        return self._gd.n == n

    def _select(self, logits: torch.Tensor) -> None:
        st = self.state
        # the step's KV appends (and the previous step's fork copies) report
        # out-of-pool entries at the selection's synchronisation
        self.pt.stage_errors()
        results = self.strategy.select_batched(st, logits, self.temperature, self.temperature_mode)
        self.pt.raise_staged_errors()
        st.add_filtered_results(results, self.eos_token_id)

    # ---------------------------------------------------------------- results
    def final_sequences(self, num_return: Optional[int] = None):
        reqs = sorted({c.request_id for c in self.state.candidates})
        return {r: self.strategy.get_final_sequences(self.state, num_return, r) for r in reqs}

    @torch.no_grad()
    def generate(self, prompts: Sequence[Sequence[int]], steps: int):
        self.prefill(prompts)
        for _ in range(steps):
            if not self.state.candidates or self.strategy.should_stop(self.state, 1 << 30, 0):
                break
            self.step()
        return self.final_sequences()
