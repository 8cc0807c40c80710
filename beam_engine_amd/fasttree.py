"""The reference's FastTree entry points on this build's planner and kernels.

The reference's ``kernel_type="fasttree"`` decode builds, per step,
``BeamState.get_fasttree_input()`` -> (tree_nodes, req_to_token, ...)
(src/beam_engine/beam_state.py:414-633), then
``prepare_fasttree_metadata_for_paged_cache(tree_nodes, req_to_token,
batch_size, num_qo_heads, num_kv_heads, head_dim, device)``
(src/beam_engine/attention/fasttree/preparation.py:11-225) once per step
(models/modeling_llama.py:757-773), and per layer ``fasttree_decode(q,
k_buffer, v_buffer, o, <metadata arrays>, sm_scale)``
(attention/fasttree/kernel.py:288-348) over copies of the layer's K and V
(models/modeling_llama.py:369-425).

Here:

* ``prepare_fasttree_metadata_for_paged_cache`` keeps the reference's
  arguments.  It reads the tree (``KVTreeNode``: parent, cumulative
  ``seqlen``, requests) and ``req_to_token`` (slot = page * page_size + i) on
  the host, merges each chain of only-children into one segment (the trie's
  unbranched page chains), decides every edge top down with FastTree's own
  SplitQ / SplitK model (preparation.py:34-88; or this build's fitted costs)
  and lays the decomposition out as levels of shared passes, planned once for
  every layer of the step (``be_attn_plan``).  Each candidate attends every
  token of its root-to-leaf path once -- the tokens its ``req_to_token`` row
  lists, its newest one included -- which is FastTree's intent (every
  token of the path once); the reference's own metadata reads ``seqlen`` as a node's own
  length and starts only from node 0, which breaks deeper trees and forests.
* ``fasttree_decode(q, paged_kv_cache, o, metadata)`` runs the plan on the
  layer's paged cache (``kv_cache_at_layer[layer]``) in place: no K / V
  buffer copies, no ``mid_o`` of the reference's size (partials live in the
  plan's workspace).

The engine's own loop (``BatchedBeamSearch(kernel_type="fasttree")``) takes
the same decomposition from the native trie in one call per step and runs it
inside the whole-step graph; this module is the boundary for a caller that
keeps the reference's per-step FastTree calls.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import List, Optional, Sequence

import numpy as np
import torch

from .attention import MultiLevelCascadeAttentionWrapper
from .beam_state import decomposition_levels

_WORKSPACE = {}


def _workspace(device) -> torch.Tensor:
    dev = torch.device(device)
    ws = _WORKSPACE.get(dev)
    if ws is None:
        ws = _WORKSPACE[dev] = torch.empty(128 << 20, dtype=torch.uint8, device=dev)
    return ws


def fasttree_segments(tree_info: Sequence, req_to_token, batch_size: int, page_size: int):
    """The segment tree of a FastTree input: ``(segs, paths)`` as
    ``BeamState.segment_tree`` gives them (``segs[i] = [pages, tokens,
    parent, candidates, children]``, numbered as the candidates' paths first
    reach them; ``paths[c]`` candidate c's segments top down), every token of
    each candidate's ``req_to_token`` path counted (its newest included)."""
    n = len(tree_info)
    rtt = req_to_token.cpu().numpy() if isinstance(req_to_token, torch.Tensor) else np.asarray(req_to_token)
    parent = [int(t.parent) for t in tree_info]
    seqlen = [int(t.seqlen) for t in tree_info]
    for i, t in enumerate(tree_info):
        if int(t.id) != i:
            raise ValueError(f"tree node {i} has id {t.id}: nodes must be listed by id")
        if parent[i] >= i:
            raise ValueError(f"tree node {i}: parent {parent[i]} is not listed before it")
    kids: List[List[int]] = [[] for _ in range(n)]
    for i in range(n):
        if parent[i] >= 0:
            kids[parent[i]].append(i)
    own = [seqlen[i] - (seqlen[parent[i]] if parent[i] >= 0 else 0) for i in range(n)]
    # each candidate's nodes, top down
    cand_nodes: List[List[int]] = [[] for _ in range(batch_size)]
    for i, t in enumerate(tree_info):
        for r in t.requests:
            if not 0 <= int(r) < batch_size:
                raise ValueError(f"tree node {i} names request {r} of {batch_size}")
            cand_nodes[int(r)].append(i)
    # segment key of a node: the last node of its chain of only-children
    head = list(range(n))
    for i in range(n):
        p = parent[i]
        if p >= 0 and len(kids[p]) == 1:
            head[i] = head[p]
    index = {}
    segs: List[list] = []
    paths: List[List[int]] = []
    for c in range(batch_size):
        nodes = sorted(cand_nodes[c])
        if not nodes:
            raise ValueError(f"request {c} has no tree node")
        # split the path at segment heads: each run of one head is one segment
        runs: List[List[int]] = []
        for x in nodes:
            if runs and head[x] == head[runs[-1][-1]]:
                runs[-1].append(x)
            else:
                runs.append([x])
        path, prev = [], -1
        for run in runs:
            key = run[-1]
            i = index.get(key)
            if i is None:
                start = seqlen[parent[run[0]]] if parent[run[0]] >= 0 else 0
                slots = rtt[c, start: seqlen[key]].astype(np.int64)
                pages = list(dict.fromkeys((slots // page_size).tolist()))
                i = index[key] = len(segs)
                segs.append([pages, sum(own[x] for x in run), prev, [], []])
                if prev >= 0:
                    segs[prev][4].append(i)
            segs[i][3].append(c)
            path.append(i)
            prev = i
        paths.append(path)
    return segs, paths


def fasttree_levels(tree_info: Sequence, req_to_token, batch_size: int, num_qo_heads: int, num_kv_heads: int,
                    page_size: int, costs: str = "fasttree"):
    """The level arrays of the FastTree decomposition of a tree: each edge
    absorbed or split by FastTree's model (``costs="fasttree"``) or this
    build's fitted costs (``"mi355x"``).  [(qo, kv_indptr, kv_indices,
    last_page_len)] per level."""
    from .picker import MI355X, CostModel, FastTreeCostModel
    from .beam_state import BeamState
    segs, paths = fasttree_segments(tree_info, req_to_token, batch_size, page_size)
    model = FastTreeCostModel(num_qo_heads, num_kv_heads) if costs == "fasttree" else \
        CostModel(num_qo_heads, num_kv_heads, page_size, MI355X)
    absorbed, _ = BeamState.absorb_edges(segs, model.absorb)
    return decomposition_levels(segs, paths, absorbed, page_size)


@dataclass
class FastTreeMetadata:
    """One step's FastTree plan (the reference's FastTreeMetadata,
    attention/fasttree/metadata.py:5-66): the planned wrapper every layer's
    ``fasttree_decode`` runs, and its levels."""
    wrapper: MultiLevelCascadeAttentionWrapper
    levels: list
    num_qo_heads: int
    num_kv_heads: int
    head_dim: int


def prepare_fasttree_metadata_for_paged_cache(tree_info: Sequence, req_to_token, batch_size: int,
                                              num_qo_heads: int, num_kv_heads: int, head_dim: int,
                                              device: str = "cuda", *, page_size: int = 16,
                                              q_data_type=torch.bfloat16,
                                              workspace: Optional[torch.Tensor] = None,
                                              costs: str = "fasttree") -> FastTreeMetadata:
    """Drop-in for preparation.py:11-225 (same leading arguments): plans the
    step's tree attention once for every layer.  ``page_size`` is the page
    table's (the reference's kernel reads slots, the plan reads pages);
    ``workspace`` a device byte buffer for the plan and its partials (a
    shared 128 MB one per device by default)."""
    levels = fasttree_levels(tree_info, req_to_token, batch_size, num_qo_heads, num_kv_heads, page_size, costs)
    ws = workspace if workspace is not None else _workspace(device)
    w = MultiLevelCascadeAttentionWrapper(max(1, len(levels)), ws)
    w.plan([l[0] for l in levels], [l[1] for l in levels], [l[2] for l in levels], [l[3] for l in levels],
           num_qo_heads, num_kv_heads, head_dim, page_size, causal=False, q_data_type=q_data_type)
    return FastTreeMetadata(w, levels, num_qo_heads, num_kv_heads, head_dim)


def fasttree_decode(q: torch.Tensor, paged_kv_cache: torch.Tensor, o: Optional[torch.Tensor],
                    metadata: FastTreeMetadata, sm_scale: Optional[float] = None) -> torch.Tensor:
    """Drop-in for kernel.py:288-348: o[i] = attention of q[i] ([N, Hq, D])
    over candidate i's whole path in the layer's paged cache ``[P, 2,
    page_size, Hkv, D]`` (the reference passes K / V buffer copies instead).
    ``sm_scale`` must be D^-1/2 (the plan's scale) when given."""
    if sm_scale is not None and abs(sm_scale - metadata.head_dim ** -0.5) > 1e-12 * sm_scale:
        raise NotImplementedError("fasttree_decode runs at sm_scale = head_dim ** -0.5")
    return metadata.wrapper.run(q, paged_kv_cache, out=o)
