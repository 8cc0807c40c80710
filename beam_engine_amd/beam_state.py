"""Beam trie over KV pages: drop-in for the reference's ``BeamState``
(src/beam_engine/beam_state.py).

Same data classes and methods with the same results (page ids, candidate
order, cascade index arrays are identical).  Differences in how they are
computed:

* ``get_cascade_input`` makes one top-down pass over the live trie: every
  node gets its cascade level, the page list of its level segment (a chain of
  only-children shares one list) and the representative node of each lower
  level.  Each candidate's groups then come from its leaf in O(levels) instead
  of walking every root-to-leaf path (beam_state.py:267-306).
* Several requests can share one state: ``add_root_sequence`` may be called
  once per request; each root is a separate cascade group at level 0 and
  every candidate carries its ``request_id``.
* ``add_filtered_results`` defers the page fork copies of one step to a
  single batched launch (page ids are allocated in the reference's order).
* ``NativeBeamState`` is the same state kept in native code (the trie and its
  page allocator, ``be_beam_trie``): the decode loop applies each selection
  and builds the next step's metadata without Python work per candidate;
  the Python objects (``candidates``, nodes, ``sequence`` ...) are built
  from it when read.
"""

from __future__ import annotations

from dataclasses import dataclass
import ctypes
import logging
from typing import Dict, List, Optional, Tuple

import numpy as np
import torch

from .kv_tree_node import KVTreeNode
from .page_table import PageTable

logger = logging.getLogger(__name__)


class TrieNode:
    """One page of tokens in the beam trie (beam_state.py:12-30)."""

    __slots__ = ("tokens", "parent", "children", "page_id", "_lvl", "_seg", "_seglen", "_reps", "_pre",
                 "_stamp", "nid")

    def __init__(self, tokens: List[int], page_id: int, parent: Optional["TrieNode"] = None):
        self.tokens = tokens
        self.parent = parent
        self.children: List["TrieNode"] = []
        self.page_id = page_id
        self._stamp = -1
        self.nid = -1            # row in the owning state's node table (-1: not tracked)
        if parent:
            parent.children.append(self)

    def __repr__(self):
        return f"TrieNode(tokens={self.tokens}, page_id={self.page_id}, children={len(self.children)})"


@dataclass
class BeamCandidate:
    """A live beam: its leaf node and accumulated log-probability (beam_state.py:33-38).
    A beam finished by an end-of-sequence pick keeps its whole token sequence
    (``sequence``, ending with the EOS token); its ``trie_node`` is the node it
    was picked from."""
    trie_node: TrieNode
    score: float
    finished: bool = False
    request_id: int = 0
    sequence: Optional[List[int]] = None


@dataclass
class BeamTokenCandidate:
    token_id: int
    log_prob: float


@dataclass
class BeamToken:
    token_id: int
    accumulated_score: float


@dataclass
class BeamGenerateInput:
    candidate: BeamCandidate
    children: List[BeamTokenCandidate]


@dataclass
class BeamGenerateResult:
    candidate: BeamCandidate
    children: List[BeamToken]


class _NodeTable:
    """Flat mirror of a trie for the native metadata builder: per node its
    parent row (-1 for a root), page, token count, last token and liveness.
    Rows follow creation order, so a parent's row is below its children's."""

    def __init__(self, cap: int = 1024):
        self.n = 0
        self._alloc(cap)

    def _alloc(self, cap):
        old = getattr(self, "parent", None)
        arrs = [np.full(cap, -1, np.int32), np.zeros(cap, np.int32), np.zeros(cap, np.int32),
                np.zeros(cap, np.int32), np.zeros(cap, np.uint8)]
        if old is not None:
            for a, b in zip(arrs, (self.parent, self.page, self.ntok, self.last, self.alive)):
                a[:self.n] = b[:self.n]
        self.parent, self.page, self.ntok, self.last, self.alive = arrs

    def add(self, node: "TrieNode") -> None:
        if self.n == len(self.parent):
            self._alloc(2 * len(self.parent))
        i = self.n
        self.n += 1
        node.nid = i
        self.parent[i] = node.parent.nid if node.parent is not None else -1
        self.page[i] = node.page_id
        self.ntok[i] = len(node.tokens)
        self.last[i] = node.tokens[-1] if node.tokens else 0
        self.alive[i] = 1

    def append(self, node: "TrieNode", token: int) -> None:
        i = node.nid
        self.ntok[i] += 1
        self.last[i] = token


class BeamState:
    """Live candidates and their page trie (beam_state.py:62-683).

    ``fast_metadata``: keep a node table of the trie as it changes and build
    each step's cascade arrays, write locations and positions natively
    (``step_metadata``).  The table follows changes made through this class's
    methods only, so it is for the engine's own states; a trie edited by hand
    keeps the Python pass."""

    def __init__(self, beam_size: int, page_table: PageTable, fast_metadata: bool = False):
        self.beam_size = beam_size
        self.page_table = page_table
        self.root: Optional[TrieNode] = None
        self.roots: List[TrieNode] = []
        self.candidates: List[BeamCandidate] = []
        self.finished_candidates: List[BeamCandidate] = []
        self._cached_write_batch_indices = None
        self._cached_write_kv_indptr = None
        self._stamp = 0
        self._tab: Optional[_NodeTable] = _NodeTable() if fast_metadata else None
        self._meta_buf = np.zeros(1 << 16, np.int32)
        self._meta_used = ctypes.c_int64(0)

    def num_candidates(self) -> int:
        return len(self.candidates)

    def num_finished(self) -> int:
        return len(self.finished_candidates)

    # ------------------------------------------------------------ building
    def add_root_sequence(self, sequence: List[int], request_id: int = 0) -> List[TrieNode]:
        """Allocate pages for a prompt and add its candidate (beam_state.py:76-98).
        Returns the created nodes in creation order."""
        ps = self.page_table.page_size
        cur = None
        created = []
        for start in range(0, len(sequence), ps):
            page = self.page_table.allocate_block()
            node = TrieNode(list(sequence[start:start + ps]), page, cur)
            if self._tab is not None:
                self._tab.add(node)
            created.append(node)
            if cur is None:
                self.roots.append(node)
                if self.root is None:
                    self.root = node
            cur = node
        self.candidates.append(BeamCandidate(cur, 0, False, request_id))
        return created

    def add_filtered_results(self, results: List[BeamGenerateResult], eos_token_id: Optional[int] = None) -> None:
        """Prune dead branches, then expand survivors with the reference's fork
        rules (beam_state.py:101-209): a single child appends to a non-full
        page or opens a new page; several children of a full page open one
        page each; several children of a partial page copy it for every child
        after the first (siblings under the same parent), then the first child
        appends to the original page.

        ``eos_token_id`` (the reference resolves one but never finishes a beam,
        beam.py:68-69): a child with that token finishes its beam instead --
        it joins ``finished_candidates`` with its sequence and score and takes
        no page; the remaining children expand as above, and a candidate left
        without children is pruned."""
        if eos_token_id is not None:
            kept = []
            for r in results:
                live = []
                for ch in r.children:
                    if ch.token_id == eos_token_id:
                        c = r.candidate
                        self.finished_candidates.append(BeamCandidate(
                            c.trie_node, ch.accumulated_score, True, c.request_id,
                            self.sequence(c) + [ch.token_id]))
                    else:
                        live.append(ch)
                kept.append(r if len(live) == len(r.children) else BeamGenerateResult(r.candidate, live))
            results = kept
        pt = self.page_table
        ps = pt.page_size
        tab = self._tab

        for r in results:
            if not r.children:
                node = r.candidate.trie_node
                while node is not None and not node.children:
                    pt.free_block(node.page_id)
                    if tab is not None:
                        tab.alive[node.nid] = 0
                    parent = node.parent
                    if parent is not None:
                        parent.children.remove(node)
                    elif node in self.roots:
                        self.roots.remove(node)
                        if self.root is node:
                            self.root = self.roots[0] if self.roots else None
                    node = parent

        new: List[BeamCandidate] = []
        with pt.defer_copies():
            for r in results:
                children = r.children
                if not children:
                    continue
                node = r.candidate.trie_node
                rid = r.candidate.request_id
                tokens = node.tokens
                if len(children) == 1:
                    child = children[0]
                    if len(tokens) < ps:
                        tokens.append(child.token_id)
                        if tab is not None:
                            tab.append(node, child.token_id)
                        new.append(BeamCandidate(node, child.accumulated_score, False, rid))
                    else:
                        page = pt.allocate_block()
                        leaf = TrieNode([child.token_id], page, node)
                        if tab is not None:
                            tab.add(leaf)
                        new.append(BeamCandidate(leaf, child.accumulated_score, False, rid))
                    continue
                if len(tokens) == ps:
                    for child in children:
                        page = pt.allocate_block()
                        leaf = TrieNode([child.token_id], page, node)
                        if tab is not None:
                            tab.add(leaf)
                        new.append(BeamCandidate(leaf, child.accumulated_score, False, rid))
                else:
                    first, rest = children[0], children[1:]
                    for child in rest:
                        page = pt.copy_block(node.page_id, len(node.tokens))
                        sib = TrieNode([*tokens, child.token_id], page, node.parent)
                        if tab is not None:
                            tab.add(sib)
                        if node.parent is None:          # forking a partial root page makes a new root
                            self.roots.append(sib)
                        new.append(BeamCandidate(sib, child.accumulated_score, False, rid))
                    tokens.append(first.token_id)
                    if tab is not None:
                        tab.append(node, first.token_id)
                    new.append(BeamCandidate(node, first.accumulated_score, False, rid))
        self.candidates = new

    # ------------------------------------------------------------ trie pass
    def _annotate(self) -> None:
        """Top-down pass over every tree holding a candidate: level, segment
        page list, lower-level representatives and prefix token count."""
        self._stamp += 1
        stamp = self._stamp
        roots = list(self.roots)
        if self.root is not None and self.root not in roots:
            roots.append(self.root)
        self._dfs(roots, stamp)
        for c in self.candidates:           # trees whose root was never registered (hand-built)
            n = c.trie_node
            if n._stamp == stamp:
                continue
            while n.parent is not None:
                n = n.parent
            self._dfs([n], stamp)

    @staticmethod
    def _dfs(roots: List[TrieNode], stamp: int) -> None:
        stack = []
        for r in roots:
            r._lvl = 0
            r._seg = [r.page_id]
            r._seglen = 1
            r._reps = ()
            r._pre = 0
            r._stamp = stamp
            stack.append(r)
        while stack:
            p = stack.pop()
            ch = p.children
            if not ch:
                continue
            pre = p._pre + len(p.tokens)
            if len(ch) > 1:
                reps = p._reps + (p,)
                lvl = p._lvl + 1
                for n in ch:
                    n._lvl = lvl
                    n._seg = [n.page_id]
                    n._seglen = 1
                    n._reps = reps
                    n._pre = pre
                    n._stamp = stamp
                    stack.append(n)
            else:
                n = ch[0]
                seg = p._seg
                if len(seg) > p._seglen:         # the list was extended past p before: fork a copy
                    seg = seg[:p._seglen]
                seg.append(n.page_id)
                n._lvl = p._lvl
                n._seg = seg
                n._seglen = p._seglen + 1
                n._reps = p._reps
                n._pre = pre
                n._stamp = stamp
                stack.append(n)

    @staticmethod
    def _seg_pages(node: TrieNode) -> List[int]:
        pages = node._seg[:node._seglen]
        if len(pages) > 1 and len(set(pages)) != len(pages):
            pages = list(dict.fromkeys(pages))
        return pages

    def get_cascade_input(self):
        """Per-level FlashInfer cascade arrays (beam_state.py:211-412).

        Returns ``(qo_indptr_arr, kv_indptr_arr, kv_indices_arr,
        last_page_len_arr, query_token_ids, write_batch_indices,
        write_kv_indptr)``; the index arrays are CPU int32 tensors, the rest
        live on the page table's device.  An empty state returns the
        reference's 5-tuple."""
        if not self.candidates:
            return ([], [], [], [], torch.empty(0, 0, 0))
        levels = self._cascade_lists()
        qo_arr = [torch.tensor(l[0], dtype=torch.int32) for l in levels]
        kvp_arr = [torch.tensor(l[1], dtype=torch.int32) for l in levels]
        kvi_arr = [torch.tensor(l[2], dtype=torch.int32) for l in levels]
        lpl_arr = [torch.tensor(l[3], dtype=torch.int32) for l in levels]
        dev = self.page_table.device
        qids = torch.tensor(self.query_token_ids(), dtype=torch.long, device=dev)
        n = len(self.candidates)
        if self._cached_write_batch_indices is None or self._cached_write_batch_indices.shape[0] != n:
            self._cached_write_batch_indices = torch.arange(n, dtype=torch.int32, device=dev)
            self._cached_write_kv_indptr = torch.arange(n + 1, dtype=torch.int32, device=dev)
        return (qo_arr, kvp_arr, kvi_arr, lpl_arr, qids, self._cached_write_batch_indices,
                self._cached_write_kv_indptr)

    def _cascade_lists(self):
        """The cascade arrays as Python lists: [(qo, kv_indptr, kv_indices, last_page_len)] per level."""
        self._annotate()
        cands = self.candidates
        max_level = max(c.trie_node._lvl for c in cands)
        levels = []
        for lv in range(max_level + 1):
            groups: Dict[int, list] = {}
            for c in cands:
                leaf = c.trie_node
                rep = leaf._reps[lv] if lv < leaf._lvl else leaf
                key = id(rep)
                g = groups.get(key)
                if g is None:
                    cnt = len(rep.tokens)
                    groups[key] = [1, rep, (max(0, cnt - 1) if rep is leaf else cnt)]
                else:
                    g[0] += 1
            qo, kvp, kvi, lpl = [0], [0], [], []
            for cnt, rep, last in groups.values():
                kvi.extend(self._seg_pages(rep))
                kvp.append(len(kvi))
                lpl.append(last)
                qo.append(qo[-1] + cnt)
            levels.append((qo, kvp, kvi, lpl))
        return levels

    def step_metadata(self):
        """This step's cascade arrays and per-candidate inputs, built natively
        from the node table (``fast_metadata`` states; else the Python pass).

        Returns ``(levels, query_tokens, write_pages, write_slots, positions)``:
        ``levels`` as ``_cascade_lists`` gives them (int32 arrays here), the
        rest one int per candidate as ``query_token_ids``, ``write_locations``
        and ``position_ids`` give them."""
        tab = self._tab
        cands = self.candidates
        if tab is None or any(c.trie_node.nid < 0 for c in cands):
            levels = self._cascade_lists()
            wp, ws = self.write_locations()
            return levels, self.query_token_ids(), wp, ws, self.position_ids(reuse_annotation=True)
        from . import _lib
        lib = _lib.load()
        leaves = np.fromiter((c.trie_node.nid for c in cands), np.int32, len(cands))
        while True:
            buf = self._meta_buf
            rc = lib.be_trie_cascade(tab.parent.ctypes.data, tab.page.ctypes.data, tab.ntok.ctypes.data,
                                     tab.last.ctypes.data, tab.alive.ctypes.data, tab.n, leaves.ctypes.data,
                                     len(cands), buf.ctypes.data, buf.size, ctypes.byref(self._meta_used))
            if rc == _lib.BE_ERR_CAPACITY:
                self._meta_buf = np.zeros(2 * int(self._meta_used.value), np.int32)
                continue
            _lib.check(rc, "trie cascade metadata")
            break
        buf = self._meta_buf[: int(self._meta_used.value)].copy()
        nl, oc = int(buf[0]), int(buf[1])
        levels = []
        for lv in range(nl):
            ng, oq, op, oi, ol = (int(x) for x in buf[2 + 5 * lv: 7 + 5 * lv])
            levels.append((buf[oq: oq + ng + 1], buf[op: op + ng + 1], buf[oi: oi + int(buf[op + ng])],
                           buf[ol: ol + ng]))
        n = len(cands)
        return levels, buf[oc: oc + n], buf[oc + n: oc + 2 * n], buf[oc + 2 * n: oc + 3 * n], \
            buf[oc + 3 * n: oc + 4 * n]

    def segment_tree(self, include_self: bool = False):
        """The live trie's segments (the cascade's groups: unbranched page
        chains between branch points), parents before children.

        Returns ``(segs, paths)``: ``segs[i] = [pages, tokens, parent index or
        -1, candidate indices below it, child indices]`` (a candidate's own
        leaf segment excludes its newest token, the cascade convention, unless
        ``include_self``: FastTree's req_to_token covers the whole path,
        beam_state.py:512-564) and ``paths[q]`` = the segment indices of
        candidate q's path, top down."""
        self._annotate()
        ps = self.page_table.page_size
        index: Dict[int, int] = {}
        segs: List[list] = []
        paths: List[List[int]] = []
        for qi, c in enumerate(self.candidates):
            leaf = c.trie_node
            path = []
            parent = -1
            for rep in leaf._reps + (leaf,):
                i = index.get(id(rep))
                if i is None:
                    pages = self._seg_pages(rep)
                    last = max(0, len(rep.tokens) - 1) if rep is leaf and not include_self else len(rep.tokens)
                    i = index[id(rep)] = len(segs)
                    segs.append([pages, (len(pages) - 1) * ps + last, parent, [], []])
                    if parent >= 0:
                        segs[parent][4].append(i)
                segs[i][3].append(qi)
                path.append(i)
                parent = i
            paths.append(path)
        return segs, paths

    @staticmethod
    def absorb_edges(segs, absorb):
        """Top-down edge decisions (preparation.py:69-88 over segments):
        ``absorb(nq_cur, nq_child, len_parent, len_child)`` True makes the
        child's pass also read its parent's (effective) tokens, and the
        parent's pass serve nq_child fewer queries.  Returns the set of
        absorbing segments and the effective token count of every segment."""
        nq = [len(s[3]) for s in segs]
        teff = [s[1] for s in segs]
        absorbed = set()
        for k, s in enumerate(segs):
            for ch in s[4]:
                nch = len(segs[ch][3])
                if absorb(nq[k], nch, teff[k], segs[ch][1]):
                    absorbed.add(ch)
                    nq[k] -= nch
                    teff[ch] = segs[ch][1] + teff[k]
        return absorbed, teff

    def tree_levels(self, segs, paths, absorbed):
        """Level arrays of a decomposition (``decomposition_levels`` at this
        state's page size)."""
        return decomposition_levels(segs, paths, absorbed, self.page_table.page_size)

    def tree_lists(self, absorb, include_self: bool = False):
        """Exact path attention as levels of shared passes (the decomposition of
        FastTree's preparation, attention/fasttree/preparation.py:60-105, over
        the cascade's segments instead of single pages): every candidate
        attends each token of its path once (the flat strategy's result, own
        newest token excluded); ``absorb`` decides each edge (see
        ``absorb_edges``).  Returns [(qo, kv_indptr, kv_indices,
        last_page_len)] per level."""
        if not self.candidates:
            return []
        segs, paths = self.segment_tree(include_self)
        absorbed, _ = self.absorb_edges(segs, absorb)
        return self.tree_levels(segs, paths, absorbed)

    def query_token_ids(self) -> List[int]:
        return [c.trie_node.tokens[-1] if c.trie_node.tokens else 0 for c in self.candidates]

    def write_locations(self) -> Tuple[List[int], List[int]]:
        """(page, slot) each candidate's new K/V goes to (beam.py:180-189)."""
        return ([c.trie_node.page_id for c in self.candidates],
                [len(c.trie_node.tokens) - 1 for c in self.candidates])

    def position_ids(self, reuse_annotation: bool = False) -> List[int]:
        """Total path tokens minus one per candidate (beam.py:208-221).
        ``reuse_annotation``: the caller has built this step's metadata since
        the last change of the trie, so its top-down pass still holds."""
        if not reuse_annotation:
            self._annotate()
        return [c.trie_node._pre + len(c.trie_node.tokens) - 1 for c in self.candidates]

    def path_pages(self, idx: int) -> List[int]:
        out = []
        n = self.candidates[idx].trie_node
        while n is not None:
            out.append(n.page_id)
            n = n.parent
        return out[::-1]

    def flat_lists(self, include_self: bool = False):
        """Flat strategy arrays: one group per candidate over its whole path.

        ``include_self=False`` follows the cascade convention of the reference
        (the query's own new token is not attended, beam_state.py:347-354);
        True attends to it (FastTree / HF convention)."""
        self._annotate()
        kvp, kvi, lpl = [0], [], []
        for c in self.candidates:
            leaf = c.trie_node
            pages: List[int] = []
            for rep in leaf._reps:
                pages.extend(rep._seg[:rep._seglen])
            pages.extend(leaf._seg[:leaf._seglen])
            kvi.extend(pages)
            kvp.append(len(kvi))
            n = len(leaf.tokens)
            lpl.append(n if include_self else max(0, n - 1))
        return kvp, kvi, lpl

    # ------------------------------------------------------------ FastTree inputs
    def _build_kv_tree_structure(self) -> Tuple[List[KVTreeNode], Dict[int, int]]:
        """BFS numbering of the live trie for FastTree (beam_state.py:414-510).
        ``seqlen`` is cumulative from the root, as in the reference."""
        self._annotate()
        roots = []
        seen = set()
        for c in self.candidates:
            n = c.trie_node
            while n.parent is not None:
                n = n.parent
            if id(n) not in seen:
                seen.add(id(n))
                roots.append(n)
        users: Dict[int, List[int]] = {}
        for ci, c in enumerate(self.candidates):
            n = c.trie_node
            while n is not None:
                users.setdefault(id(n), []).append(ci)
                n = n.parent
        out: List[KVTreeNode] = []
        ids: Dict[int, int] = {}
        queue = list(roots)
        head = 0
        while head < len(queue):
            t = queue[head]
            head += 1
            k = KVTreeNode()
            k.id = len(out)
            ids[id(t)] = k.id
            k.parent = ids[id(t.parent)] if t.parent is not None else -1
            k.seqlen = t._pre + len(t.tokens)
            k.num_children = len(t.children)
            k.requests = sorted(users.get(id(t), []))
            out.append(k)
            queue.extend(t.children)
        return out, ids

    def _build_req_to_token(self, tree_nodes=None) -> torch.Tensor:
        """``[N, max_len]`` slot ids page * page_size + i (beam_state.py:512-564),
        built on the host and copied once."""
        self._annotate()
        ps = self.page_table.page_size
        rows = []
        for c in self.candidates:
            path = []
            n = c.trie_node
            while n is not None:
                path.append(n)
                n = n.parent
            row = []
            for node in reversed(path):
                base = node.page_id * ps
                row.extend(range(base, base + len(node.tokens)))
            rows.append(row)
        width = max((len(r) for r in rows), default=0)
        out = torch.zeros((len(rows), width), dtype=torch.int32)
        for i, r in enumerate(rows):
            out[i, :len(r)] = torch.tensor(r, dtype=torch.int32)
        return out.to(self.page_table.device)

    def get_fasttree_input(self):
        """(tree_nodes, req_to_token, query_ids, write_pages, write_positions) (beam_state.py:566-633)."""
        tree_nodes, _ = self._build_kv_tree_structure()
        req_to_token = self._build_req_to_token(tree_nodes)
        dev = self.page_table.device
        wp, wpos = self.write_locations()
        return (tree_nodes, req_to_token,
                torch.tensor(self.query_token_ids(), dtype=torch.long, device=dev),
                torch.tensor(wp, dtype=torch.int32, device=dev),
                torch.tensor(wpos, dtype=torch.int32, device=dev))

    # ------------------------------------------------------------ results
    def sequence(self, cand: BeamCandidate) -> List[int]:
        if cand.sequence is not None:
            return list(cand.sequence)
        seq: List[int] = []
        n = cand.trie_node
        parts = []
        while n is not None:
            parts.append(n.tokens)
            n = n.parent
        for p in reversed(parts):
            seq.extend(p)
        return seq

    def get_best_finished(self, num_return: int) -> List[BeamCandidate]:
        """Best candidates by score / sequence length.  (The reference reads a
        missing ``length`` attribute here, beam_state.py:635-644; the length
        used is the full sequence length.)"""
        pool = self.finished_candidates or self.candidates
        return sorted(pool, key=lambda c: c.score / max(1, len(self.sequence(c))), reverse=True)[:num_return]

    def get_final_sequences(self, num_return: int, length_penalty: float = 1.0,
                            request_id: Optional[int] = None) -> List[Tuple[List[int], float]]:
        """(sequence, score / len^penalty) sorted by score (beam_state.py:646-682)."""
        pool = self.finished_candidates + self.candidates
        if request_id is not None:
            pool = [c for c in pool if c.request_id == request_id]
        out = []
        for c in pool:
            seq = self.sequence(c)
            sc = c.score
            if length_penalty != 0 and len(seq) > 1:
                sc = sc / (len(seq) ** length_penalty)
            out.append((seq, sc))
        out.sort(key=lambda x: x[1], reverse=True)
        return out[:num_return]


def decomposition_levels(segs, paths, absorbed, page_size: int):
    """Level arrays of a decomposition: a segment's pass reads its own
    pages after those of the ancestors it absorbed and serves the
    candidates below it that no absorbing child covers; a candidate's
    passes along its path are its levels 0, 1, ...  Candidates served at
    a level by one segment but not contiguous in candidate order get one
    group per run; candidates without a pass at a level get empty
    groups."""
    ps = page_size
    pages_eff: Dict[int, List[int]] = {}

    def eff(k):
        p = pages_eff.get(k)
        if p is None:
            p = segs[k][0]
            if k in absorbed:
                p = eff(segs[k][2]) + p
            pages_eff[k] = p
        return p
    per_level: List[Dict[int, List[int]]] = []
    for qi, keys in enumerate(paths):
        lv = 0
        for j, k in enumerate(keys):
            if j + 1 < len(keys) and keys[j + 1] in absorbed:
                continue
            if lv == len(per_level):
                per_level.append({})
            per_level[lv].setdefault(k, []).append(qi)
            lv += 1
    n = len(paths)
    levels = []
    for groups in per_level:
        runs = []
        for k, qs in groups.items():
            start = prev = qs[0]
            for q in qs[1:]:
                if q != prev + 1:
                    runs.append((start, prev + 1, k))
                    start = q
                prev = q
            runs.append((start, prev + 1, k))
        runs.sort()
        qo, kvp, kvi, lpl = [0], [0], [], []
        for q0, q1, k in runs:
            if q0 > qo[-1]:                      # candidates without a pass here
                qo.append(q0); kvp.append(len(kvi)); lpl.append(0)
            pages = eff(k)
            tok = len(pages) * ps - (ps * len(segs[k][0]) - segs[k][1])
            kvi.extend(pages)
            kvp.append(len(kvi))
            lpl.append(tok - (len(pages) - 1) * ps if pages else 0)
            qo.append(q1)
        if qo[-1] < n:
            qo.append(n); kvp.append(len(kvi)); lpl.append(0)
        levels.append((qo, kvp, kvi, lpl))
    return levels


class _PageRef:
    """A created page of ``NativeBeamState.add_root_sequence`` (its id)."""
    __slots__ = ("page_id",)

    def __init__(self, page_id: int):
        self.page_id = page_id


def _parse_metadata(buf: np.ndarray, n: int):
    """Split be_trie_cascade's output words into (levels, query tokens, write
    pages, write slots, positions)."""
    nl, oc = int(buf[0]), int(buf[1])
    levels = []
    for lv in range(nl):
        ng, oq, op, oi, ol = (int(x) for x in buf[2 + 5 * lv: 7 + 5 * lv])
        levels.append((buf[oq: oq + ng + 1], buf[op: op + ng + 1], buf[oi: oi + int(buf[op + ng])],
                       buf[ol: ol + ng]))
    return levels, buf[oc: oc + n], buf[oc + n: oc + 2 * n], buf[oc + 2 * n: oc + 3 * n], \
        buf[oc + 3 * n: oc + 4 * n]


class NativeBeamState:
    """``BeamState`` kept in native code: the trie, its candidates and the
    page allocator of ``page_table`` live in ``be_beam_trie`` /
    ``be_page_pool`` (the reference's BeamState.add_root_sequence and
    add_filtered_results rules, beam_state.py:76-209, with pages from its
    PageTable, page_table.py:77-124).  A decode step needs two native calls:
    ``apply_selection`` with the selection arrays (prune, expand, fork copies
    in one device launch) and ``step_metadata`` (the cascade arrays and the
    candidates' inputs).

    Everything else -- ``candidates``, ``finished_candidates``, ``root(s)``,
    ``sequence``, ``get_final_sequences``, the Python metadata passes -- is
    read from a ``BeamState`` built from the native state when first asked
    for after a change (its nodes carry the same pages, tokens and order).
    ``add_filtered_results`` takes results for the candidates of that view,
    in its order, as ``BeamState.add_filtered_results`` does."""

    def __init__(self, beam_size: int, page_table: PageTable):
        from . import _lib
        self._lib = lib = _lib.load()
        self.beam_size = beam_size
        self.page_table = page_table
        self._h = lib.be_trie_create(int(page_table.page_size), page_table._pool)
        if not self._h:
            _lib.check(_lib.BE_ERR_INVALID, "beam trie")
        self._sizes = np.zeros(5, np.int32)
        self._ver = ctypes.c_int64(0)
        self._mirror: Optional[BeamState] = None
        self._mirror_ver = -1
        self._meta_buf = np.zeros(1 << 16, np.int32)
        self._meta_ptr = (None, 0)          # (buffer, its address) for the planner call
        self._meta_used = ctypes.c_int64(0)
        self._copies = np.zeros(3 * 1024, np.int32)
        self._copies_ptr = (None, 0)        # (buffer, its address) for the trie update call
        self._ncopies = ctypes.c_int32(0)
        self._warn = ctypes.c_int32(0)

    def __del__(self):
        h, self._h = getattr(self, "_h", None), None
        if h:
            self._lib.be_trie_destroy(h)

    # ------------------------------------------------------------ native state
    def _read_sizes(self) -> np.ndarray:
        self._lib.be_trie_sizes(self._h, self._sizes.ctypes.data, ctypes.byref(self._ver))
        return self._sizes

    def num_candidates(self) -> int:
        return int(self._read_sizes()[1])

    def num_finished(self) -> int:
        return int(self._read_sizes()[2])

    def candidate_arrays(self) -> Tuple[np.ndarray, np.ndarray]:
        """Each live candidate's request id (int32) and score (float64)."""
        n = self.num_candidates()
        req = np.zeros(n, np.int32)
        score = np.zeros(n, np.float64)
        self._lib.be_trie_candidates(self._h, None, req.ctypes.data, score.ctypes.data)
        return req, score

    def add_root_sequence(self, sequence: List[int], request_id: int = 0) -> List[_PageRef]:
        """A prompt's pages and its candidate (beam_state.py:76-98); returns
        the created pages in creation order."""
        from . import _lib
        toks = np.ascontiguousarray(sequence, dtype=np.int32)
        ps = self.page_table.page_size
        pages = np.zeros(max(1, -(-len(toks) // ps)), np.int32)
        _lib.check(self._lib.be_trie_add_root(self._h, toks.ctypes.data, len(toks), int(request_id),
                                              pages.ctypes.data), "add_root_sequence")
        return [_PageRef(int(p)) for p in pages[: -(-len(toks) // ps)]]

    def apply_selection(self, parent, token, score, eos_token_id: Optional[int] = None) -> int:
        """One step's selection in emission order (entry e: parent candidate
        index, -1 for an unused entry; token; accumulated score): the
        reference's prune and expand rules, with this step's fork copies issued
        in one launch.  Returns the number of fork copies."""
        from . import _lib
        arrs = []
        for x, dt, tdt in ((parent, np.int32, torch.int32), (token, np.int32, torch.int32),
                           (score, np.float64, torch.float64)):
            if isinstance(x, torch.Tensor) and x.device.type == "cpu" and x.dtype == tdt and x.is_contiguous():
                arrs.append((x.numel(), x.data_ptr(), x))       # the selection's host tensors as they are
            else:
                a = np.ascontiguousarray(x, dtype=dt)
                arrs.append((len(a), a.ctypes.data, a))
        n = arrs[0][0]
        if arrs[1][0] != n or arrs[2][0] != n:
            raise ValueError("parent, token and score must have one entry each")
        if self._copies.size < 3 * n:
            self._copies = np.zeros(6 * n, np.int32)
        if self._copies_ptr[0] is not self._copies:
            self._copies_ptr = (self._copies, self._copies.ctypes.data)
        rc = self._lib.be_trie_apply(self._h, arrs[0][1], arrs[1][1], arrs[2][1], n,
                                     -1 if eos_token_id is None else int(eos_token_id), self._copies_ptr[1],
                                     self._copies.size // 3, ctypes.byref(self._ncopies), ctypes.byref(self._warn))
        _lib.check(rc, "trie update")
        if self._warn.value:
            logger.warning("%d freed pages were not allocated", self._warn.value)
        nc = int(self._ncopies.value)
        pt = self.page_table
        if pt.stage_copies_enabled:
            # to the staged list: the next step (its graph, or its eager path
            # first) performs them
            pt.stage_copies(self._copies[: 3 * nc].reshape(nc, 3))
        elif nc:
            if pt._defer:
                pt._pending.extend(map(tuple, self._copies[: 3 * nc].reshape(nc, 3).tolist()))
            else:
                pt.copy_pages(self._copies[: 3 * nc].reshape(nc, 3))
        return nc

    def add_filtered_results(self, results: List[BeamGenerateResult], eos_token_id: Optional[int] = None) -> None:
        """``BeamState.add_filtered_results`` for results on this state's
        ``candidates`` (beam_state.py:101-209)."""
        index = {id(c): i for i, c in enumerate(self.candidates)}
        par, tok, sc = [], [], []
        for r in results:
            i = index.get(id(r.candidate))
            if i is None:
                raise ValueError("a result's candidate is not a live candidate of this state")
            for ch in r.children:
                par.append(i)
                tok.append(ch.token_id)
                sc.append(ch.accumulated_score)
        self.apply_selection(par, tok, sc, eos_token_id)

    def step_metadata(self):
        """``BeamState.step_metadata`` from the native trie: (levels, query
        tokens, write pages, write slots, positions)."""
        from . import _lib
        n = self.num_candidates()
        while True:
            buf = self._meta_buf
            rc = self._lib.be_trie_metadata(self._h, buf.ctypes.data, buf.size, ctypes.byref(self._meta_used))
            if rc == _lib.BE_ERR_CAPACITY:
                self._meta_buf = np.zeros(2 * int(self._meta_used.value), np.int32)
                continue
            _lib.check(rc, "trie cascade metadata")
            break
        return _parse_metadata(self._meta_buf[: int(self._meta_used.value)].copy(), n)

    def step_levels(self, kind: str = "cascade", include_self: bool = False, model=None):
        """One strategy's levels and the candidates' inputs from the native
        trie (``be_trie_levels``): ``kind`` "cascade" (``step_metadata``),
        "flat", "split", "tree" or "auto" (``model``: a ``be_tree_model``,
        ``StrategyPicker.tree_model()``).  Returns ``(levels, query tokens,
        write pages, write slots, positions, kind built, option costs)``; the
        costs (flat, split, tree) are given for "auto" only."""
        from . import _lib
        n = self.num_candidates()
        chosen = ctypes.c_int32(-1)
        costs = np.full(3, np.nan)
        pm = ctypes.byref(model) if model is not None else None
        while True:
            buf = self._meta_buf
            rc = self._lib.be_trie_metadata_kind(self._h, _lib.KIND_CODES[kind], int(include_self), pm,
                                                 buf.ctypes.data, buf.size, ctypes.byref(self._meta_used),
                                                 ctypes.byref(chosen), costs.ctypes.data)
            if rc == _lib.BE_ERR_CAPACITY and int(self._meta_used.value) > buf.size:
                self._meta_buf = np.zeros(2 * int(self._meta_used.value), np.int32)
                continue
            _lib.check(rc, f"{kind} levels")
            break
        out = _parse_metadata(self._meta_buf[: int(self._meta_used.value)].copy(), n)
        return out + (_lib.KIND_NAMES[int(chosen.value)], costs if kind == "auto" else None)

    def plan_cascade(self, wrapper, num_qo_heads: int, num_kv_heads: int, head_dim: int, q_data_type,
                     host_plan: Optional[torch.Tensor] = None):
        """This step's cascade metadata and ``wrapper``'s plan of it in one
        native call (``be_trie_plan``: the same plan as ``wrapper.plan`` of
        ``step_metadata``'s levels with ``causal=True``), the plan uploaded
        to the wrapper's workspace.  Returns the candidates' query tokens,
        write pages, write slots and positions.  ``host_plan`` (pinned int32):
        the plan is written there and not uploaded -- the caller copies its
        first ``wrapper._info.plan_ints`` words to the workspace's start before
        the next run (a plan beyond it raises MemoryError)."""
        return self.plan_kind(wrapper, "cascade", num_qo_heads, num_kv_heads, head_dim, q_data_type,
                              host_plan=host_plan)[:4]

    def plan_kind(self, wrapper, kind: str, num_qo_heads: int, num_kv_heads: int, head_dim: int, q_data_type,
                  include_self: bool = False, model=None, host_plan: Optional[torch.Tensor] = None):
        """``plan_cascade`` for any strategy kind (``be_trie_plan_kind``: the
        levels of ``step_levels(kind, include_self, model)`` and ``wrapper``'s
        plan of them, causal only for "cascade").  Returns the candidates'
        query tokens, write pages, write slots and positions, the kind built
        and, for "auto", the modelled flat / split / tree costs."""
        from . import _lib
        from .attention import _Staging, _num_cus
        if isinstance(q_data_type, str):
            q_data_type = getattr(torch, q_data_type)
        staging = None if host_plan is not None else _Staging.get(wrapper._ws.device)
        info = _lib.BeAttnPlanInfo()
        max_page = ctypes.c_int32(-1)
        chosen = ctypes.c_int32(-1)
        costs = self._costs_buf = getattr(self, "_costs_buf", None)
        if costs is None:
            costs = self._costs_buf = np.full(3, np.nan)
        caps = ctypes.byref(wrapper._caps) if wrapper._caps is not None else None
        pm = ctypes.byref(model) if model is not None else None
        code = _lib.KIND_CODES[kind]
        cap = host_plan.numel() if host_plan is not None else staging.buf.numel()
        while True:
            buf = host_plan if host_plan is not None else staging.acquire(cap)
            meta = self._meta_buf
            if self._meta_ptr[0] is not meta:
                self._meta_ptr = (meta, meta.ctypes.data)
            rc = self._lib.be_trie_plan_kind(self._h, code, int(include_self), pm, num_qo_heads, num_kv_heads,
                                             head_dim, _lib.dtype_code(q_data_type), wrapper._plan_flags(),
                                             wrapper._num_cus or _num_cus(wrapper._ws.device), caps,
                                             self._meta_ptr[1], meta.size, ctypes.byref(self._meta_used),
                                             buf.data_ptr(), buf.numel(), ctypes.byref(info), ctypes.byref(max_page),
                                             ctypes.byref(chosen), costs.ctypes.data)
            if rc == _lib.BE_ERR_CAPACITY:
                if int(self._meta_used.value) > meta.size:
                    self._meta_buf = np.zeros(2 * int(self._meta_used.value), np.int32)
                elif host_plan is None and info.plan_ints > buf.numel():
                    cap = max(int(info.plan_ints), 2 * buf.numel())
                else:
                    # a full caller buffer, or a plan beyond the fixed layout's
                    # capacities (plan_ints 0: no buffer size cures it): MemoryError
                    _lib.check(rc, f"{kind} plan")
                continue
            _lib.check(rc, f"{kind} plan")
            break
        wrapper.num_levels = int(self._meta_buf[0])
        wrapper._install_plan(info, buf, staging, int(max_page.value), head_dim, None, q_data_type,
                              upload=host_plan is None)
        n = int(info.num_queries)                      # one query per candidate
        oc = int(self._meta_buf[1])
        m = self._meta_buf[oc: oc + 4 * n].copy()
        return (m[:n], m[n: 2 * n], m[2 * n: 3 * n], m[3 * n:], _lib.KIND_NAMES[int(chosen.value)],
                costs.copy() if kind == "auto" else None)

    # ------------------------------------------------------------ Python view
    def python_state(self) -> BeamState:
        """The state as ``BeamState`` objects (rebuilt after every change)."""
        sz = self._read_sizes()
        if self._mirror is not None and self._mirror_ver == self._ver.value:
            return self._mirror
        nn, nc, nf, nft, ps = (int(x) for x in sz)
        parent = np.zeros(nn, np.int32)
        page = np.zeros(nn, np.int32)
        ntok = np.zeros(nn, np.int32)
        alive = np.zeros(nn, np.uint8)
        tokens = np.zeros(nn * ps, np.int32)
        fin_req = np.zeros(nf, np.int32)
        fin_score = np.zeros(nf, np.float64)
        fin_off = np.zeros(nf + 1, np.int32)
        fin_tok = np.zeros(nft, np.int32)
        self._lib.be_trie_export(self._h, parent.ctypes.data, page.ctypes.data, ntok.ctypes.data, alive.ctypes.data,
                                 tokens.ctypes.data, fin_req.ctypes.data, fin_score.ctypes.data, fin_off.ctypes.data,
                                 fin_tok.ctypes.data)
        cnode = np.zeros(nc, np.int32)
        creq = np.zeros(nc, np.int32)
        cscore = np.zeros(nc, np.float64)
        self._lib.be_trie_candidates(self._h, cnode.ctypes.data, creq.ctypes.data, cscore.ctypes.data)
        st = BeamState(self.beam_size, self.page_table)
        tok2 = tokens.reshape(nn, ps) if nn else tokens.reshape(0, max(ps, 1))
        nodes: List[Optional[TrieNode]] = [None] * nn
        for i in range(nn):
            if not alive[i]:
                continue
            p = int(parent[i])
            node = TrieNode(tok2[i, : ntok[i]].tolist(), int(page[i]), nodes[p] if p >= 0 else None)
            node.nid = i
            nodes[i] = node
            if p < 0:
                st.roots.append(node)
        st.root = st.roots[0] if st.roots else None
        st.candidates = [BeamCandidate(nodes[int(nd)], float(s_), False, int(r))
                         for nd, r, s_ in zip(cnode, creq, cscore)]
        st.finished_candidates = [BeamCandidate(None, float(fin_score[f]), True, int(fin_req[f]),
                                                fin_tok[fin_off[f]: fin_off[f + 1]].tolist()) for f in range(nf)]
        self._mirror, self._mirror_ver = st, self._ver.value
        return st

    @property
    def candidates(self) -> List[BeamCandidate]:
        return self.python_state().candidates

    @property
    def finished_candidates(self) -> List[BeamCandidate]:
        return self.python_state().finished_candidates

    def __getattr__(self, name):
        # the rest of BeamState's interface reads the Python view
        if name.startswith("__") or name in ("_h", "_lib", "_mirror", "_sizes", "_ver"):
            raise AttributeError(name)
        return getattr(self.python_state(), name)
