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
        # cascade decoding keeps the trie and its pages in native code (one call
        # per selection, one for the metadata); the other kinds read the
        # Python trie's passes every step and keep the Python state
        self.state = NativeBeamState(beam_size, page_table) if kernel_type == "cascade" else \
            BeamState(beam_size, page_table, fast_metadata=True)
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
        self.picker_costs = picker_costs    # "mi355x" fitted costs or "fasttree" (the reference's edge model)
        self.step_log: List[dict] = []
        self._staging = torch.empty(4 * 4096, dtype=torch.int64, pin_memory=True)
        self.attn_timer = None          # optional callable(layer, fn) used by benchmarks
        self.graphs = graphs            # capture the non-attention work of a step in HIP graphs
        # cascade with graphs: the whole step, attention included, as one graph
        # over a fixed-layout plan (a step whose plan does not fit that layout
        # runs the per-layer graphs with eager attention)
        self.step_graph = step_graph
        self.step_graphed = False       # the last step ran as one graph
        self._gd = None
        self._fixed = None              # the fixed-layout cascade wrapper of the step graph
        self._fixed_key = None          # its launch shape (plan fields the captured launches read)
        self._fixed_caps = None

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

    # ---------------------------------------------------------------- whole-step graph
    _LAUNCH_FIELDS = ("kernel", "num_wg", "stream_loop", "tail_waves", "grid_merge", "static_layout", "off_wg",
                      "off_items", "off_seg_causal", "off_tail_items", "off_tails", "off_pages", "off_records",
                      "off_record_slots", "part_rows_cap", "dtype", "num_qo_heads", "num_kv_heads", "head_dim",
                      "page_size", "plan_ints", "partial_bytes")

    @classmethod
    def _launch_key(cls, info):
        return tuple(getattr(info, f) for f in cls._LAUNCH_FIELDS)

    def _fixed_plan(self, levels, n: int):
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
                w.plan(*args, causal=True, q_data_type=m.dtype)
            except MemoryError:
                w = None                            # outgrew the layout: re-size below
            else:
                if self._launch_key(w._info) == self._fixed_key:
                    return w
                return None
        # size the layout: this step's compact plan, doubled, with margins
        probe = MultiLevelCascadeAttentionWrapper(len(levels), self.ws)
        probe.plan(*args, causal=True, q_data_type=m.dtype)
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
        if isinstance(self.state, NativeBeamState) and not self.pt.stage_copies_enabled:
            # from now on each selection's fork copies go to the staged list that
            # the step graph's first part performs (in the upload header when
            # there is one)
            if self._gd.copy_list is not None:
                self.pt.enable_staged_copies(2 * n, *self._gd.copy_list)
            else:
                self.pt.enable_staged_copies(2 * n)
        try:
            w.plan(*args, causal=True, q_data_type=m.dtype)
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
        kind = self.kernel_type
        levels = None
        w = None
        graphed = kind == "cascade" and self.graphs and self.step_graph and hasattr(self.model, "decode") and \
            self._graph_ready(n)
        upload = False                  # one copy uploads the header and the plan
        if graphed and self._fixed is not None and isinstance(st, NativeBeamState):
            # metadata and the fixed-layout plan in one native call, the plan
            # written straight into the upload block's pinned twin
            cfg = self.model.cfg
            host_plan = self._host_plan
            try:
                qids, wp, wpos, pos = st.plan_cascade(self._fixed, cfg.num_attention_heads,
                                                      cfg.num_key_value_heads, cfg.head_dim, self.model.dtype,
                                                      host_plan=host_plan)
            except MemoryError:
                pass                                # beyond the layout: _fixed_plan re-sizes it
            else:
                if self._launch_key(self._fixed._info) == self._fixed_key:
                    w = self.last_attn = self._fixed
                    upload = host_plan is not None
        if w is None:
            if kind == "cascade":
                # the cascade arrays and the candidates' inputs from the native builder
                levels, qids, wp, wpos, pos = st.step_metadata()
            elif kind == "tree":
                p = self._get_picker()
                levels = st.tree_lists((p.edges or p.model).absorb)
            elif kind == "auto":
                plan = self._get_picker().choose(st)
                kind, levels = plan.kind, plan.levels
            if graphed:
                w = self.last_attn = self._fixed_plan(levels, n)
        self.step_graphed = w is not None
        if not self.step_graphed:
            self.pt.run_staged_copies()     # an eager step performs the staged fork copies first
        if w is None:
            w = self._plan(kind, levels)
        if self.kernel_type != "cascade":
            qids = st.query_token_ids()
            wp, wpos = st.write_locations()
            pos = st.position_ids(reuse_annotation=True)     # _plan's metadata pass just ran
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
        self.step_log.append({"n": n, "kind": kind})

    def prepare_graphs(self) -> None:
        """Capture the segment graphs (and, for cascade, the whole-step graph)
        now for the current candidate count (the first decode step would
        otherwise capture them)."""
        n = self.state.num_candidates()
        if self.graphs and hasattr(self.model, "decode") and n:
            self._graph_ready(n)
            if self.kernel_type == "cascade" and self.step_graph and self._fixed is None:
                self._fixed_plan(self.state.step_metadata()[0], n)    # capture the whole-step graph too

    def _graph_ready(self, n: int) -> bool:
        """Capture the segment graphs once the candidate count is known (it
        stays B per request); a different count runs eagerly."""
        from .llama import GraphedDecoder
        if self._gd is None:
            header = None
            hb = GraphedDecoder.header_bytes(n)
            if self.device.type == "cuda" and self.kernel_type == "cascade" and self.step_graph and hb <= self._hdr:
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
        if isinstance(st, NativeBeamState) and type(self.strategy) is VanillaBeamSearchStrategy and \
                "select_batched" not in vars(self.strategy):
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
            if isinstance(st, NativeBeamState) and type(self.strategy) is VanillaBeamSearchStrategy:
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
