"""The product BeamState (beam_engine_amd.beam_state) against the oracle:
identical cascade arrays on the reference's test trees, identical page ids,
candidate order and copies over the fork trace and over long random runs.
Host logic only: a recording page allocator stands in for the device pool."""

import random
from collections import deque
from contextlib import contextmanager

import pytest

from beam_engine_amd.beam_state import (BeamCandidate, BeamGenerateResult, BeamState, BeamToken, TrieNode)
from oracle.beam_state import OCand, OracleAllocator, OracleBeamState, OResult, build_tree
from tests.conftest import load_fixtures

FX = load_fixtures()


class RecordingPages:
    """FIFO allocator with the PageTable interface BeamState uses; records copies."""

    def __init__(self, max_num_pages, page_size):
        self.page_size = page_size
        self.max_num_pages = max_num_pages
        self.free_pages = deque(range(max_num_pages))
        self.allocated_pages = set()
        self.copies = []
        self.device = "cpu"

    def allocate_block(self):
        if not self.free_pages:
            raise MemoryError("No free pages available")
        p = self.free_pages.popleft()
        self.allocated_pages.add(p)
        return p

    def free_block(self, p):
        if p in self.allocated_pages:
            self.allocated_pages.remove(p)
            self.free_pages.append(p)

    def copy_block(self, p, n):
        new = self.allocate_block()
        self.copies.append((p, new, n))
        return new

    @contextmanager
    def defer_copies(self):
        yield self


def build_product(tree):
    pages = RecordingPages(64, tree["page_size"])
    st = BeamState(len(tree["candidates"]), pages)
    nodes = {}
    for n in tree["nodes"]:
        parent = nodes[n["parent"]] if n["parent"] is not None else None
        nodes[n["id"]] = TrieNode(list(n["tokens"]), n["page"], parent)
        if parent is None:
            st.root = nodes[n["id"]]
    st.candidates = [BeamCandidate(nodes[c], 0.0) for c in tree["candidates"]]
    return st


@pytest.mark.parametrize("name", ["cascade_md", "swapped", "uneven"])
def test_product_matches_fixture(name):
    tree = FX["trees"][name]
    st = build_product(tree)
    levels = st._cascade_lists()
    exp = tree["expected"]
    assert [l[0] for l in levels] == exp["qo_indptr"]
    assert [l[1] for l in levels] == exp["kv_indptr"]
    assert [l[2] for l in levels] == exp["kv_indices"]
    assert [l[3] for l in levels] == exp["last_page_len"]
    assert st.query_token_ids() == exp["query_ids"]


def test_product_fork_trace():
    tr = FX["fork_trace"]
    pages = RecordingPages(tr["max_num_pages"], tr["page_size"])
    st = BeamState(tr["beam_size"], pages)
    made = st.add_root_sequence(tr["prompt"])
    assert [n.page_id for n in made] == tr["after_root"]["pages"]
    for step in tr["steps"]:
        nc = len(pages.copies)
        res = [BeamGenerateResult(c, [BeamToken(t, s) for t, s in ch]) for c, ch in zip(st.candidates, step["select"])]
        st.add_filtered_results(res)
        got = [{"page": c.trie_node.page_id, "tokens": c.trie_node.tokens, "score": c.score} for c in st.candidates]
        assert got == step["expect_candidates"]
        assert [list(x) for x in pages.copies[nc:]] == step["expect_copies"]
        if "expect_free_list" in step:
            assert list(pages.free_pages) == step["expect_free_list"]
        e = step["expect_cascade"]
        lv = st._cascade_lists()
        assert ([l[0] for l in lv], [l[1] for l in lv], [l[2] for l in lv], [l[3] for l in lv]) == \
            (e["qo_indptr"], e["kv_indptr"], e["kv_indices"], e["last_page_len"])
        assert st.query_token_ids() == e["query_ids"]
        assert st.write_locations() == (step["expect_write_pages"], step["expect_write_pos"])
        assert st.position_ids() == step["expect_position_ids"]


@pytest.mark.parametrize("seed", range(8))
def test_product_random_runs_match_oracle(seed):
    rng = random.Random(seed)
    page = rng.choice([2, 3, 4, 16])
    beam = rng.choice([2, 3, 4, 8])
    prompt = list(range(rng.randint(1, 40)))
    o_alloc = OracleAllocator(20000, page)
    o = OracleBeamState(beam, o_alloc)
    pages = RecordingPages(20000, page)
    p = BeamState(beam, pages, fast_metadata=True)
    o.add_root_sequence(prompt)
    p.add_root_sequence(prompt)
    first = [(1000 + j, -0.25 * j) for j in range(beam)]
    o.add_filtered_results([OResult(o.candidates[0], first)])
    p.add_filtered_results([BeamGenerateResult(p.candidates[0], [BeamToken(t, s) for t, s in first])])
    for step in range(40):
        pool = []
        for ci, c in enumerate(o.candidates):
            for j in range(2 * beam):
                pool.append((ci, rng.randrange(30), c.score - rng.random()))
        pool.sort(key=lambda t: t[2], reverse=True)
        chosen = pool[:beam]
        o_res = [OResult(c, [(t, s) for ci2, t, s in chosen if ci2 == ci]) for ci, c in enumerate(o.candidates)]
        p_res = [BeamGenerateResult(c, [BeamToken(t, s) for ci2, t, s in chosen if ci2 == ci])
                 for ci, c in enumerate(p.candidates)]
        o.add_filtered_results(o_res)
        p.add_filtered_results(p_res)
        assert o_alloc.copies == pages.copies
        assert list(o_alloc.free_pages) == list(pages.free_pages)
        assert [(c.node.page_id, c.node.tokens, c.score) for c in o.candidates] == \
            [(c.trie_node.page_id, c.trie_node.tokens, c.score) for c in p.candidates]
        qo, kvp, kvi, lpl, qids = o.get_cascade_input()
        lv = p._cascade_lists()
        assert [l[0] for l in lv] == qo and [l[1] for l in lv] == kvp
        assert [l[2] for l in lv] == kvi and [l[3] for l in lv] == lpl
        assert p.query_token_ids() == qids
        assert p.position_ids() == o.position_ids()
        assert p.write_locations() == o.write_locations()
        # the native builder over the state's node table gives the same arrays
        nlv, nq, nwp, nws, npos = p.step_metadata()
        assert [l[0].tolist() for l in nlv] == qo and [l[1].tolist() for l in nlv] == kvp
        assert [l[2].tolist() for l in nlv] == kvi and [l[3].tolist() for l in nlv] == lpl
        assert nq.tolist() == qids and npos.tolist() == o.position_ids()
        assert (nwp.tolist(), nws.tolist()) == tuple(o.write_locations())
    assert p.get_final_sequences(beam) == o.get_final_sequences(beam)


@pytest.mark.parametrize("seed", range(6))
def test_native_metadata_on_random_forests(seed):
    """Several requests in one state (forest), including partial root pages
    forked into new roots and whole requests dying: the native builder equals
    the Python pass at every step."""
    rng = random.Random(100 + seed)
    page = rng.choice([2, 4, 16])
    beam = rng.choice([2, 4, 8])
    pages = RecordingPages(50000, page)
    st = BeamState(beam, pages, fast_metadata=True)
    for r in range(rng.randint(1, 4)):
        st.add_root_sequence(list(range(rng.randint(1, 3 * page))), request_id=r)
    for step in range(30):
        res = []
        by_req = {}
        for i, c in enumerate(st.candidates):
            by_req.setdefault(c.request_id, []).append(i)
        chosen = {}
        for r, idx in by_req.items():
            if step == 10 and r == 0 and len(by_req) > 1:
                continue                              # request 0 dies: its whole tree is pruned
            pool = [(i, rng.randrange(50), st.candidates[i].score - rng.random()) for i in idx
                    for _ in range(2 * beam)]
            pool.sort(key=lambda t: t[2], reverse=True)
            for i, t, sc in pool[:beam]:
                chosen.setdefault(i, []).append(BeamToken(t, sc))
        res = [BeamGenerateResult(c, chosen.get(i, [])) for i, c in enumerate(st.candidates)]
        st.add_filtered_results(res)
        lv = st._cascade_lists()
        nlv, nq, nwp, nws, npos = st.step_metadata()
        assert [tuple(x.tolist() for x in l) for l in nlv] == [tuple(l) for l in lv]
        assert nq.tolist() == st.query_token_ids()
        assert (nwp.tolist(), nws.tolist()) == tuple(st.write_locations())
        assert npos.tolist() == st.position_ids()


def test_native_metadata_needs_tracked_nodes():
    """A hand-built trie (nodes not made by the state) takes the Python pass."""
    tree = FX["trees"]["uneven"]
    st = build_product(tree)
    st._tab = __import__("beam_engine_amd.beam_state", fromlist=["_NodeTable"])._NodeTable()
    lv, q, wp, ws, pos = st.step_metadata()
    assert lv == st._cascade_lists() and q == st.query_token_ids()


def test_forest_of_requests_groups_by_root():
    pages = RecordingPages(100, 4)
    st = BeamState(2, pages)
    st.add_root_sequence([1, 2, 3, 4, 5], request_id=0)
    st.add_root_sequence([6, 7, 8], request_id=1)
    r0, r1 = st.candidates
    st.add_filtered_results([BeamGenerateResult(r0, [BeamToken(10, -1.0), BeamToken(11, -2.0)]),
                             BeamGenerateResult(r1, [BeamToken(12, -1.0), BeamToken(13, -1.5)])])
    assert [c.request_id for c in st.candidates] == [0, 0, 1, 1]
    # request 1's prompt fits one partial page: its fork copies the root page,
    # giving a second root (parent None), as in the reference (beam_state.py:193-197)
    lv = st._cascade_lists()
    assert lv[0][0] == [0, 2, 3, 4]
    assert lv[0][2] == [0, 4, 2]
    assert lv[0][3] == [4, 3, 3]
    assert lv[1][2] == [3, 1, 4, 2] and lv[1][3] == [1, 1, 3, 3]
    kvp, kvi, lpl = st.flat_lists()
    assert kvi == [0, 3, 0, 1, 4, 2]        # full path pages per candidate
    assert lpl == [1, 1, 3, 3]              # cascade convention: own new token excluded
    assert len(st.roots) == 3


def test_fasttree_structure_is_bfs_with_cumulative_seqlen():
    tree = FX["trees"]["uneven"]
    st = build_product(tree)
    nodes, _ = st._build_kv_tree_structure()
    assert [n.seqlen for n in nodes] == [2, 4, 6, 5, 5, 7]
    assert [n.parent for n in nodes] == [-1, 0, 0, 1, 1, 2]
    assert nodes[0].requests == [0, 1, 2]


@pytest.mark.parametrize("seed", range(4))
def test_eos_finishes_beams_without_pages(seed):
    """With an end-of-sequence token, a pick of it finishes its beam (score,
    whole sequence ending with the token, no page); the trie evolves exactly as
    the oracle's with those picks removed, so page ids, copies and candidates
    stay the reference's."""
    rng = random.Random(200 + seed)
    page, beam, eos = rng.choice([2, 4]), 4, 7
    o_alloc = OracleAllocator(20000, page)
    o = OracleBeamState(beam, o_alloc)
    pages = RecordingPages(20000, page)
    p = BeamState(beam, pages, fast_metadata=True)
    prompt = list(range(20, 20 + rng.randint(1, 9)))
    o.add_root_sequence(prompt)
    p.add_root_sequence(prompt)
    first = [(100 + j, -0.25 * j) for j in range(beam)]
    o.add_filtered_results([OResult(o.candidates[0], first)])
    p.add_filtered_results([BeamGenerateResult(p.candidates[0], [BeamToken(t, s) for t, s in first])], eos)
    n_fin = 0
    for step in range(25):
        if not p.candidates:
            break
        pool = []
        for ci, c in enumerate(p.candidates):
            for j in range(2 * beam):
                pool.append((ci, eos if rng.random() < 0.08 else rng.randrange(30), c.score - rng.random()))
        pool.sort(key=lambda t: t[2], reverse=True)
        chosen, seen = [], set()
        for ci, t, s in pool:
            if (ci, t) not in seen and len(chosen) < beam:
                seen.add((ci, t))
                chosen.append((ci, t, s))
        p_res = [BeamGenerateResult(c, [BeamToken(t, s) for ci2, t, s in chosen if ci2 == ci])
                 for ci, c in enumerate(p.candidates)]
        # finished in result order (candidates in order, children in order)
        expect_fin = [(p.sequence(r.candidate) + [eos], ch.accumulated_score) for r in p_res for ch in r.children
                      if ch.token_id == eos]
        o_res = [OResult(c, [(t, s) for ci2, t, s in chosen if ci2 == ci and t != eos])
                 for ci, c in enumerate(o.candidates)]
        p.add_filtered_results(p_res, eos)
        o.add_filtered_results(o_res)
        o.finished_candidates += [OCand(None, sc, sequence=seq) for seq, sc in expect_fin]
        got_fin = [(c.sequence, c.score) for c in p.finished_candidates[n_fin:]]
        assert got_fin == expect_fin and all(c.finished for c in p.finished_candidates)
        n_fin = len(p.finished_candidates)
        assert o_alloc.copies == pages.copies and list(o_alloc.free_pages) == list(pages.free_pages)
        assert [(c.node.page_id, c.node.tokens, c.score) for c in o.candidates] == \
            [(c.trie_node.page_id, c.trie_node.tokens, c.score) for c in p.candidates]
        if p.candidates:
            nlv, *_ = p.step_metadata()
            assert [tuple(x.tolist() for x in l) for l in nlv] == [tuple(l) for l in p._cascade_lists()]
    final = p.get_final_sequences(100)
    assert len(final) == len(p.finished_candidates) + len(p.candidates)
    for pen in (1.0, 0.0, 0.5):
        assert p.get_final_sequences(100, pen) == o.get_final_sequences(100, pen)
    # finished beams end with the token; live ones never carry it (an EOS pick never continues)
    assert n_fin > 0 and sum(seq[-1] == eos for seq, _ in final) == n_fin
    assert all(eos not in p.sequence(c) for c in p.candidates)


def test_final_sequences_with_finished_hand_case():
    """The product's get_final_sequences (beam_state.py:646-682) on the oracle's
    hand case: finished candidates first in the pool, one read from the trie
    and one with its own sequence; same order and scores as the oracle."""
    from tests.test_oracle_beam_state import _final_ranking_case
    o = _final_ranking_case()
    pages = RecordingPages(8, 4)
    st = BeamState(2, pages)
    root = TrieNode([1, 2, 3, 4], 0)
    a, b, c = TrieNode([5, 6], 1, root), TrieNode([7], 2, root), TrieNode([8], 3, root)
    st.root = root
    st.candidates = [BeamCandidate(a, -1.0), BeamCandidate(b, -0.6)]
    st.finished_candidates = [BeamCandidate(c, -0.9, finished=True),
                              BeamCandidate(b, -1.2, finished=True, sequence=[1, 2, 3, 4, 9, 0])]
    for pen in (1.0, 0.0, 2.0):
        assert st.get_final_sequences(4, pen) == o.get_final_sequences(4, pen)
    assert [s for s, _ in st.get_final_sequences(4, 1.0)] == [[1, 2, 3, 4, 7], [1, 2, 3, 4, 5, 6], [1, 2, 3, 4, 8],
                                                             [1, 2, 3, 4, 9, 0]]


def test_finalize_scores_hand_case():
    """VanillaBeamSearchStrategy.finalize_scores (beam_strategy.py:539-552):
    score / step^penalty, highest first, input order kept on ties; penalty 0
    or step <= 1 leaves the scores alone."""
    from beam_engine_amd.beam_state import BeamCandidate
    from beam_engine_amd.beam_strategy import VanillaBeamSearchStrategy
    a, b, c = BeamCandidate(None, -4.0), BeamCandidate(None, -2.0), BeamCandidate(None, -4.0)
    got = VanillaBeamSearchStrategy(length_penalty=1.0).finalize_scores([a, b, c], 4)
    assert [(x is y, s) for (x, s), y in zip(got, [b, a, c])] == [(True, -0.5), (True, -1.0), (True, -1.0)]
    got = VanillaBeamSearchStrategy(length_penalty=2.0).finalize_scores([a, b], 2)
    assert [s for _, s in got] == [-0.5, -1.0]
    assert [s for _, s in VanillaBeamSearchStrategy(length_penalty=0.0).finalize_scores([a, b], 9)] == [-2.0, -4.0]
    assert [s for _, s in VanillaBeamSearchStrategy().finalize_scores([a, b], 1)] == [-2.0, -4.0]
