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

``kernel_type``: the reference's two (beam.py:20, 191-206) and three more --
"cascade" (per-level groups of the reference's get_cascade_input),
"fasttree" (the reference's FastTree strategy: each candidate attends its
whole root-to-leaf path, its newest token included as FastTree's
req_to_token includes it, beam_state.py:512-564, decomposed into shared passes
over trie segments with each edge absorbed or split by FastTree's own cost
model, attention/fasttree/preparation.py:34-88), "flat" (each candidate's whole
path, the baseline), "split" (one pass per trie segment, merged), "tree" (the fasttree decomposition with each edge decided
by this build's fitted MI355X costs, or FastTree's with
``picker_costs="fasttree"``) or "auto" (per step, the cheapest of flat, fully
split and tree under the fitted costs: the per-step picker).  Every kind's
metadata and attention plan come from the native trie in one call
(``be_trie_plan_kind``) and every kind runs as the whole-step graph.  "flat",
"tree", "auto" and "fasttree" give every candidate its path tokens exactly
once; "cascade" keeps the reference's repetition of a shallow candidate's leaf
group on deeper levels.  ``include_self`` False follows the reference's
cascade convention (a query does not attend to the K/V it appends in the same
step, beam_state.py:347-354); "fasttree" always includes it.
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
from .beam_state import BeamGenerateResult, BeamState, BeamToken, NativeBeamState
from .beam_strategy import VanillaBeamSearchStrategy
from .page_table import PageTable
from .selection import beam_topk, decode_k


# Bytes reserved in front of the attention workspace for a graphed step's
# upload header (inputs and staged copy list: 48 bytes per candidate and some
# alignment), and of the pinned twin's plan area (a fixed-layout plan).
_STEP_HEADER_BYTES = 1 << 20
_STEP_PLAN_BYTES = 8 << 20


class BatchedBeamSearch:
    def __init__(self, model, page_table: PageTable, beam_size: int,
                 strategy: Optional[VanillaBeamSearchStrategy] = None, kernel_type: str = "cascade",
                 temperature: float = 1.0, workspace_bytes: int = 256 << 20, include_self: bool = False,
                 graphs: bool = False, eos_token_id: Optional[int] = None, temperature_mode: str = "reciprocal",
                 picker_costs: str = "mi355x", step_graph: bool = True):
        if kernel_type not in ("cascade", "fasttree", "flat", "split", "tree", "auto"):
            raise ValueError(f"Unknown kernel_type: {kernel_type}. Must be 'cascade', 'fasttree', 'flat', 'split', "
                             "'tree' or 'auto'.")
        if kernel_type == "cascade" and include_self:
            raise NotImplementedError("include_self with the cascade levels (their last level excludes the newest "
                                      "token, beam_state.py:343-356)")
        self.model = model
        self.pt = page_table
        self.beam_size = beam_size
        self.strategy = strategy or VanillaBeamSearchStrategy()
        self.kernel_type = kernel_type
        self.temperature = temperature
        self.temperature_mode = temperature_mode   # arithmetic of logits / T: see selection.beam_topk
        # the reference's FastTree attends the whole path, the query's own new token included
        self.include_self = include_self or kernel_type == "fasttree"
        self.eos_token_id = eos_token_id    # a pick of this token finishes its beam (off: None)
        self.device = page_table.device
        # the trie and its pages live in native code: one call per selection,
        # one for the step's metadata and attention plan (any strategy kind)
        self.state = NativeBeamState(beam_size, page_table)
        # The wrappers' workspace (an attention plan at its start) follows a
        # reserved region whose last bytes hold the graphed step's inputs and
        # staged fork-copy list: header and plan are contiguous, so a graphed
        # step uploads all of its host data with one copy from a pinned twin
        self._hdr = _STEP_HEADER_BYTES
        self.ws_all = torch.empty(self._hdr + workspace_bytes, dtype=torch.uint8, device=self.device)
        self.ws = self.ws_all[self._hdr:]
        self._hblock: Optional[torch.Tensor] = None   # pinned twin of ws_all[hdr - header : hdr + plan]
        self._hb = 0                                  # the graphed step's header bytes
        self._up_key, self._up = None, None           # (bytes, (device, host) views) of the step upload
        self._host_plan: Optional[torch.Tensor] = None   # the pinned twin's plan area (int32)
        self.cascade = MultiLevelCascadeAttentionWrapper(1, self.ws)
        self.flat = BatchDecodeWithPagedKVCacheWrapper(self.ws)
        self.last_attn = None
        self.picker = None
        # "mi355x" fitted costs or "fasttree" (the reference's edge model) for
        # the tree's edges; the "fasttree" kind always takes FastTree's model
        self.picker_costs = "fasttree" if kernel_type == "fasttree" else picker_costs
        self._model = None                  # the picker's costs as the native planner's be_tree_model
        self.step_log: List[dict] = []
        self._staging = torch.empty(4 * 4096, dtype=torch.int64, pin_memory=True)
        self.attn_timer = None          # optional callable(layer, fn) used by benchmarks
        self.graphs = graphs            # capture the non-attention work of a step in HIP graphs
        # cascade with graphs: the whole step, attention included, as one graph
        # over a fixed-layout plan (a step whose plan does not fit that layout
        # runs the per-layer graphs with eager attention)
        self.step_graph = step_graph
        self.step_graphed = False       # the last step ran as one graph
        self.graphed_steps = 0          # decode steps that ran as one graph
        self._gd = None
        self._fixed = None              # the fixed-layout cascade wrapper of the step graph
        self._fixed_key = None          # its launch shape (plan fields the captured launches read)
        self._fixed_caps = None

    # ---------------------------------------------------------------- prefill
    @torch.no_grad()
    def prefill(self, prompts: Sequence[Sequence[int]]) -> torch.Tensor:
        if len({len(p) for p in prompts}) != 1:
            raise ValueError("batched prefill needs prompts of equal length")
        for p in prompts:
            self._check_tokens(p)
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

    def _check_tokens(self, ids) -> None:
        """Token ids outside the vocabulary raise here: the embedding lookup
        on the device would read out of bounds."""
        a = np.asarray(ids)
        vocab = self.model.cfg.vocab_size
        if a.size and (int(a.min()) < 0 or int(a.max()) >= vocab):
            bad = a[(a < 0) | (a >= vocab)]
            raise ValueError(f"token id {int(bad[0])} is outside the vocabulary [0, {vocab})")

    # ---------------------------------------------------------------- decode
    def _get_picker(self):
        if self.picker is None:
            from .picker import MI355X, StrategyPicker
            cfg = self.model.cfg
            costs = "fasttree" if self.picker_costs == "fasttree" else MI355X
            self.picker = StrategyPicker(cfg.num_attention_heads, cfg.num_key_value_heads, self.pt.page_size, costs)
        return self.picker

    def _native_kind(self):
        """(kind code name for be_trie_plan_kind, its be_tree_model or None)."""
        kind = self.kernel_type
        if kind == "cascade":
            return "cascade", None
        if kind in ("flat", "split"):
            return kind, None
        if self._model is None:
            self._model = self._get_picker().tree_model()
        return ("tree" if kind == "fasttree" else kind), self._model

    def _plan(self, levels, causal: bool):
        """An eager plan of ``levels`` on a workspace wrapper."""
        m = self.model
        cfg = m.cfg
        w = MultiLevelCascadeAttentionWrapper(len(levels), self.ws)
        w.plan([l[0] for l in levels], [l[1] for l in levels], [l[2] for l in levels], [l[3] for l in levels],
               cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim, self.pt.page_size,
               causal=causal, q_data_type=m.dtype)
        self.last_attn = w
        return w

    # ---------------------------------------------------------------- whole-step graph
    _LAUNCH_FIELDS = ("kernel", "num_wg", "stream_loop", "tail_waves", "grid_merge", "static_layout", "off_wg",
                      "off_items", "off_seg_causal", "off_tail_items", "off_tails", "off_pages", "off_records",
                      "off_record_slots", "part_rows_cap", "dtype", "num_qo_heads", "num_kv_heads", "head_dim",
                      "page_size", "plan_ints", "partial_bytes")

    @classmethod
    def _launch_key(cls, info):
        return tuple(getattr(info, f) for f in cls._LAUNCH_FIELDS)

    def _fixed_plan(self, levels, n: int, causal: bool = True):
        """This step's cascade plan in the step graph's fixed layout, or None
        when the step graph cannot run it (the per-layer path runs instead).
        The first call sizes the layout from this step's plan with room to
        grow and captures the graph; a plan beyond the layout re-sizes and
        re-captures it."""
        m = self.model
        cfg = m.cfg
        args = ([l[0] for l in levels], [l[1] for l in levels], [l[2] for l in levels], [l[3] for l in levels],
                cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim, self.pt.page_size)
        w = self._fixed
        if w is not None:
            w.num_levels = len(levels)
            try:
                w.plan(*args, causal=causal, q_data_type=m.dtype)
            except MemoryError:
                w = None                            # outgrew the layout: re-size below
            else:
                if self._launch_key(w._info) == self._fixed_key:
                    return w
                return None
        # size the layout: this step's compact plan, doubled, with margins
        probe = MultiLevelCascadeAttentionWrapper(len(levels), self.ws)
        probe.plan(*args, causal=causal, q_data_type=m.dtype)
        pi = probe._info
        if pi.kernel != 2 or cfg.head_dim != 128:
            self.step_graph = False                 # the fixed layout serves the streaming kernel only
            return None
        pages = sum(len(l[2]) for l in levels)
        old = self._fixed_caps
        grow = 2 if old is None else 4
        caps = dict(max_items=grow * pi.num_items + 1024, max_queries=n,
                    max_pages=grow * pages + 4096, max_merge=n * cfg.num_key_value_heads,
                    max_merge_rows=grow * pi.num_part_rows + 1024, max_zero=n, tile_rows=64,
                    max_tails=grow * pi.num_tails + 4096)
        if old is not None:
            caps = {k: max(v, old[k]) for k, v in caps.items()}
        w = MultiLevelCascadeAttentionWrapper(len(levels), self.ws)
        w.use_fixed_layout(**caps)
        if not self.pt.stage_copies_enabled:
            # from now on each selection's fork copies go to the staged list that
            # the step graph's first part performs (in the upload header when
            # there is one)
            if self._gd.copy_list is not None:
                self.pt.enable_staged_copies(2 * n, *self._gd.copy_list)
            else:
                self.pt.enable_staged_copies(2 * n)
        try:
            w.plan(*args, causal=causal, q_data_type=m.dtype)
        except (MemoryError, ValueError):
            self.step_graph = False
            return None
        if w._info.kernel != 2:
            self.step_graph = False
            return None
        self._fixed, self._fixed_caps, self._fixed_key = w, caps, self._launch_key(w._info)
        self._gd.capture_step(lambda l, q, kv, out: w.run(q, kv, out=out))
        return w

    @torch.no_grad()
    def step(self) -> None:
        st = self.state
        n = st.num_candidates()
        if n == 0:                  # every beam finished
            return
        nkind, model = self._native_kind()
        causal = nkind == "cascade"
        inc = self.include_self
        cfg = self.model.cfg
        w = None
        built, costs = nkind, None
        graphed = self.graphs and self.step_graph and hasattr(self.model, "decode") and self._graph_ready(n)
        upload = False                  # one copy uploads the header and the plan
        if graphed and self._fixed is not None:
            # metadata and the fixed-layout plan in one native call, the plan
            # written straight into the upload block's pinned twin
            host_plan = self._host_plan
            try:
                qids, wp, wpos, pos, built, costs = st.plan_kind(
                    self._fixed, nkind, cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim,
                    self.model.dtype, include_self=inc, model=model, host_plan=host_plan)
            except MemoryError:
                pass                                # beyond the layout: _fixed_plan re-sizes it
            else:
                if self._launch_key(self._fixed._info) == self._fixed_key:
                    w = self.last_attn = self._fixed
                    upload = host_plan is not None
        if w is None:
            levels, qids, wp, wpos, pos, built, costs = st.step_levels(nkind, inc, model)
            if graphed:
                w = self.last_attn = self._fixed_plan(levels, n, causal)
        self.step_graphed = w is not None
        self.graphed_steps += int(self.step_graphed)
        if not self.step_graphed:
            self.pt.run_staged_copies()     # an eager step performs the staged fork copies first
            w = self._plan(levels, causal)
        self._check_tokens(qids)
        graph_run = self.step_graphed or (self.graphs and hasattr(self.model, "decode") and self._graph_ready(n))
        if graph_run:
            self._gd.stage_inputs(qids, pos, wp, wpos, upload=not upload)
        if upload:
            nb = self._hb + 4 * int(w._info.plan_ints)
            if self._up_key != nb:
                self._up_key = nb
                self._up = (self.ws_all[self._hdr - self._hb: self._hdr - self._hb + nb], self._hblock[:nb])
            self._up[0].copy_(self._up[1], non_blocking=True)
            self.pt.staged_uploaded()
        elif self.step_graphed:
            self.pt.upload_staged()          # the step graph's first node reads the device list
        else:
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

        if self.step_graphed:
            logits = self._gd.run_step()     # the staged fork copies first, inside the graph
        elif graph_run:
            logits = self._gd.run(attn)
        else:
            logits = self.model.decode(tok, psn, wpg, wps, self.pt, attn)
        self._select(logits)
        entry = {"n": n, "kind": built if self.kernel_type == "auto" else self.kernel_type}
        if costs is not None:
            entry["costs"] = {"flat": float(costs[0]), "split": float(costs[1]), "tree": float(costs[2])}
        self.step_log.append(entry)

    def prepare_graphs(self) -> None:
        """Capture the segment graphs and the whole-step graph now for the
        current candidate count (the first decode step would otherwise
        capture them)."""
        n = self.state.num_candidates()
        if self.graphs and hasattr(self.model, "decode") and n:
            self._graph_ready(n)
            if self.step_graph and self._fixed is None:
                nkind, model = self._native_kind()
                levels = self.state.step_levels(nkind, self.include_self, model)[0]
                self._fixed_plan(levels, n, nkind == "cascade")    # capture the whole-step graph too

    def _graph_ready(self, n: int) -> bool:
        """Capture the segment graphs once the candidate count is known (it
        stays B per request); a different count runs eagerly."""
        from .llama import GraphedDecoder
        if self._gd is None:
            header = None
            hb = GraphedDecoder.header_bytes(n)
            if self.device.type == "cuda" and self.step_graph and hb <= self._hdr:
                self._hb = hb
                self._hblock = torch.zeros(hb + _STEP_PLAN_BYTES, dtype=torch.uint8, pin_memory=True)
                self._host_plan = self._hblock[hb:].view(torch.int32)
                header = (self.ws_all[self._hdr - hb: self._hdr], self._hblock[:hb])
            self._gd = GraphedDecoder(self.model, self.pt, n, header=header)
            self._gd.capture()
        return self._gd.n == n

    def _select(self, logits: torch.Tensor) -> None:
        st = self.state
        # the step's KV appends (and the previous step's fork copies) report
        # out-of-pool entries at the selection's synchronisation
        self.pt.stage_errors()
        if type(self.strategy) is VanillaBeamSearchStrategy and "select_batched" not in vars(self.strategy):
            # the selection arrays go straight to the native trie (no per-child objects)
            req, score = st.candidate_arrays()
            cut = np.flatnonzero(np.diff(req)) + 1
            rows = np.diff(np.concatenate([[0], cut, [len(req)]])).tolist()
            b = st.beam_size
            _, _, (par, tok, sc) = beam_topk(logits, decode_k(b, logits.shape[-1]), torch.from_numpy(score), b,
                                             self.temperature, request_rows=rows, to_host=True,
                                             temperature_mode=self.temperature_mode)
            self.pt.raise_staged_errors()
            st.apply_selection(par, tok, sc, self.eos_token_id)
            return
        results = self.strategy.select_batched(st, logits, self.temperature, self.temperature_mode)
        self.pt.raise_staged_errors()
        st.add_filtered_results(results, self.eos_token_id)

    # ---------------------------------------------------------------- results
    def flush(self) -> None:
        """Perform fork copies the last selection staged for a next step."""
        self.pt.run_staged_copies()

    def final_sequences(self, num_return: Optional[int] = None):
        self.flush()
        reqs = sorted({c.request_id for c in self.state.candidates})
        return {r: self.strategy.get_final_sequences(self.state, num_return, r) for r in reqs}

    @torch.no_grad()
    def generate(self, prompts: Sequence[Sequence[int]], steps: int):
        self.prefill(prompts)
        for _ in range(steps):
            st = self.state
            if type(self.strategy) is VanillaBeamSearchStrategy:
                # VanillaBeamSearchStrategy.should_stop without building the
                # Python view: no live beam, or early stopping with beam_size
                # finished ones (live beams are never finished)
                if st.num_candidates() == 0 or (self.strategy.early_stopping and st.num_finished() >= st.beam_size):
                    break
            elif not st.candidates or self.strategy.should_stop(st, 1 << 30, 0):
                break
            self.step()
        self.flush()
        return self.final_sequences()
