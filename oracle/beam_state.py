"""CPU restatement of the reference's page allocator, beam trie and cascade
metadata (test infrastructure).

Pure-Python, integer-only.  Page contents are not modelled; page copies are
recorded as ``(src, dst, length)`` triples in issue order so that a test can
replay them against a KV pool.

Reference semantics restated (all line numbers are in
``src/beam_engine/``):

* FIFO allocator: ``free = list(range(P))``; allocate pops index 0, free
  appends; freeing an unallocated page is ignored (page_table.py:59-60,
  77-94, 110-124).
* ``copy_block(page, n)`` allocates then copies the first n slots of K and V
  of every layer (page_table.py:96-106).
* ``add_root_sequence`` (beam_state.py:76-98) and the fork / copy-on-write
  policy of ``add_filtered_results`` (beam_state.py:101-209).
* ``get_cascade_input`` level and group rules (beam_state.py:211-412).
* ``get_final_sequences`` length penalty and ranking (beam_state.py:646-682).
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import Dict, List, Optional, Tuple


class OracleAllocator:
    """FIFO free list, page_table.py:59-60, 77-94, 110-124."""

    def __init__(self, max_num_pages: int, page_size: int):
        self.page_size = page_size
        self.max_num_pages = max_num_pages
        self.free_pages = list(range(max_num_pages))
        self.allocated_pages = set()
        self.copies: List[Tuple[int, int, int]] = []   # (src, dst, length) in issue order

    def allocate_block(self) -> int:
        if not self.free_pages:
            raise MemoryError("No free pages available")
        p = self.free_pages.pop(0)
        self.allocated_pages.add(p)
        return p

    def free_block(self, p: int) -> None:
        if p not in self.allocated_pages:
            return  # the reference only logs a warning (page_table.py:117-119)
        self.allocated_pages.remove(p)
        self.free_pages.append(p)

    def copy_block(self, p: int, length: int) -> int:
        if length > self.page_size:
            raise ValueError("length cannot be larger than page size")
        new = self.allocate_block()
        self.copies.append((p, new, length))
        return new


class ONode:
    """One trie node = one page (beam_state.py:12-30)."""

    def __init__(self, tokens: List[int], page_id: int, parent: Optional["ONode"] = None):
        self.tokens = tokens
        self.page_id = page_id
        self.parent = parent
        self.children: List["ONode"] = []
        if parent is not None:
            parent.children.append(self)


@dataclass
class OCand:
    node: ONode
    score: float
    sequence: Optional[List[int]] = None    # a finished beam's own tokens (else read from the trie)


@dataclass
class OResult:
    cand: OCand
    children: List[Tuple[int, float]] = field(default_factory=list)   # (token, accumulated score)


class OracleBeamState:
    """Single-root beam trie with the reference's fork rules."""

    def __init__(self, beam_size: int, alloc: OracleAllocator):
        self.beam_size = beam_size
        self.alloc = alloc
        self.root: Optional[ONode] = None
        self.candidates: List[OCand] = []
        self.finished_candidates: List[OCand] = []

    # beam_state.py:76-98
    def add_root_sequence(self, seq: List[int]) -> List[ONode]:
        ps = self.alloc.page_size
        cur = None
        made = []
        for start in range(0, len(seq), ps):
            pid = self.alloc.allocate_block()
            node = ONode(list(seq[start:start + ps]), pid, cur)
            made.append(node)
            if cur is None:
                self.root = node
            cur = node
        self.candidates.append(OCand(cur, 0.0))
        return made

    # beam_state.py:101-209
    def add_filtered_results(self, results: List[OResult]) -> None:
        ps = self.alloc.page_size

        def free_dead(node: Optional[ONode]) -> None:
            while node is not None and not node.children:
                self.alloc.free_block(node.page_id)
                parent = node.parent
                if parent is not None:
                    parent.children.remove(node)
                node = parent

        for r in results:                       # dead branches first (:122-129)
            if not r.children:
                free_dead(r.cand.node)

        new: List[OCand] = []
        for r in results:                       # expansion (:131-206)
            if not r.children:
                continue
            node = r.cand.node
            if len(r.children) == 1:
                tok, sc = r.children[0]
                if len(node.tokens) < ps:
                    node.tokens.append(tok)
                    new.append(OCand(node, sc))
                else:
                    pid = self.alloc.allocate_block()
                    new.append(OCand(ONode([tok], pid, node), sc))
                continue
            if len(node.tokens) == ps:          # full page: one fresh page per child
                for tok, sc in r.children:
                    pid = self.alloc.allocate_block()
                    new.append(OCand(ONode([tok], pid, node), sc))
            else:                               # partial page: copies first, original last
                first, rest = r.children[0], r.children[1:]
                base = list(node.tokens)
                for tok, sc in rest:
                    pid = self.alloc.copy_block(node.page_id, len(node.tokens))
                    new.append(OCand(ONode(base + [tok], pid, node.parent), sc))
                node.tokens.append(first[0])
                new.append(OCand(node, first[1]))
        self.candidates = new

    # beam_state.py:211-412
    def get_cascade_input(self):
        """Returns (qo_indptr, kv_indptr, kv_indices, last_page_len, query_ids) as int lists."""
        if not self.candidates:
            return [], [], [], [], []
        memo: Dict[int, int] = {}

        def level(node: ONode) -> int:
            key = id(node)
            if key not in memo:
                if node.parent is None:
                    memo[key] = 0
                else:
                    memo[key] = level(node.parent) + (1 if len(node.parent.children) > 1 else 0)
            return memo[key]

        infos = []
        max_level = 0
        for ci, cand in enumerate(self.candidates):
            path = []
            n = cand.node
            while n is not None:
                path.append(n)
                n = n.parent
            path.reverse()
            by_level: Dict[int, List[ONode]] = {}
            for n in path:
                lv = level(n)
                by_level.setdefault(lv, []).append(n)
                max_level = max(max_level, lv)
            infos.append((ci, cand, by_level))

        groups: List[Dict[int, list]] = [dict() for _ in range(max_level + 1)]
        for ci, cand, by_level in infos:
            deepest = max(by_level)
            for lv in range(max_level + 1):
                nodes = by_level[lv] if lv in by_level else by_level[deepest]
                groups[lv].setdefault(id(nodes[-1]), []).append((ci, cand, nodes))

        qo_arr, kvp_arr, kvi_arr, lpl_arr = [], [], [], []
        for lv in range(max_level + 1):
            ordered = sorted(groups[lv].values(), key=lambda members: members[0][0])
            qo, kvp, kvi, lpl = [0], [0], [], []
            for members in ordered:
                _, cand, nodes = members[0]
                seen = set()
                for n in nodes:
                    if n.page_id not in seen:
                        kvi.append(n.page_id)
                        seen.add(n.page_id)
                last = nodes[-1]
                cnt = len(last.tokens)
                lpl.append(max(0, cnt - 1) if last is cand.node else cnt)
                kvp.append(len(kvi))
                qo.append(qo[-1] + len(members))
            qo_arr.append(qo)
            kvp_arr.append(kvp)
            kvi_arr.append(kvi)
            lpl_arr.append(lpl)
        qids = [c.node.tokens[-1] if c.node.tokens else 0 for c in self.candidates]
        return qo_arr, kvp_arr, kvi_arr, lpl_arr, qids

    def write_locations(self) -> Tuple[List[int], List[int]]:
        """Per-candidate (page, slot) the decode step appends K/V to (beam.py:180-189)."""
        return ([c.node.page_id for c in self.candidates],
                [len(c.node.tokens) - 1 for c in self.candidates])

    def position_ids(self) -> List[int]:
        """Total path tokens minus one, per candidate (beam.py:208-221)."""
        out = []
        for c in self.candidates:
            t = 0
            n = c.node
            while n is not None:
                t += len(n.tokens)
                n = n.parent
            out.append(t - 1)
        return out

    def path_pages(self, ci: int) -> List[int]:
        out = []
        n = self.candidates[ci].node
        while n is not None:
            out.append(n.page_id)
            n = n.parent
        return out[::-1]

    def sequence(self, ci: int) -> List[int]:
        return self.sequence_of(self.candidates[ci])

    @staticmethod
    def sequence_of(c: OCand) -> List[int]:
        """Tokens root to leaf (beam_state.py:667-671); a finished beam that
        keeps its own sequence returns that."""
        if c.sequence is not None:
            return list(c.sequence)
        seq: List[int] = []
        n = c.node
        while n is not None:
            seq = n.tokens + seq
            n = n.parent
        return seq

    # beam_state.py:646-682
    def get_final_sequences(self, num_return: int, length_penalty: float = 1.0):
        """Finished candidates first, then the live ones (:658); score divided
        by len ** penalty unless the penalty is 0 or len <= 1 (:674-676); a
        stable sort by that score, descending (:681), the first num_return."""
        out = []
        for c in self.finished_candidates + self.candidates:
            seq = self.sequence_of(c)
            sc = c.score
            if length_penalty != 0 and len(seq) > 1:
                sc = sc / (len(seq) ** length_penalty)
            out.append((seq, sc))
        out.sort(key=lambda x: x[1], reverse=True)
        return out[:num_return]


def build_tree(spec, page_size: int = 4):
    """Build an OracleBeamState from a hand-written tree spec.

    ``spec`` = {"nodes": [{"id", "tokens", "page", "parent"}...], "candidates": [node ids]}
    as stored in tests/golden/cascade_fixtures.json (the reference's
    test_cascade.py trees).
    """
    alloc = OracleAllocator(max(n["page"] for n in spec["nodes"]) + 1, page_size)
    st = OracleBeamState(len(spec["candidates"]), alloc)
    nodes: Dict[str, ONode] = {}
    for n in spec["nodes"]:
        parent = nodes[n["parent"]] if n["parent"] is not None else None
        nodes[n["id"]] = ONode(list(n["tokens"]), n["page"], parent)
        if parent is None:
            st.root = nodes[n["id"]]
    st.candidates = [OCand(nodes[c], 0.0) for c in spec["candidates"]]
    return st
