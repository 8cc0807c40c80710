"""Pins the beam-state oracle (oracle/beam_state.py) against the hand-derived
golden fixtures of the reference's own test trees and allocator trace, the
reconstruction invariant of the reference's verify_cascade_output
(test_cascade.py:218-298, deduplicated per level) and random-run invariants."""

import random

import pytest

from oracle.beam_state import OCand, ONode, OracleAllocator, OracleBeamState, OResult, build_tree
from tests.conftest import load_fixtures

FX = load_fixtures()


@pytest.mark.parametrize("name", ["cascade_md", "swapped", "uneven"])
def test_reference_trees(name):
    tree = FX["trees"][name]
    st = build_tree(tree, tree["page_size"])
    qo, kvp, kvi, lpl, qids = st.get_cascade_input()
    exp = tree["expected"]
    assert qo == exp["qo_indptr"]
    assert kvp == exp["kv_indptr"]
    assert kvi == exp["kv_indices"]
    assert lpl == exp["last_page_len"]
    assert qids == exp["query_ids"]


def reconstruct(st, qo, kvp, kvi):
    """Concatenate each candidate's group pages over levels, dropping pages
    already seen on earlier levels (a candidate whose path ends early repeats
    its deepest level)."""
    out = []
    for ci in range(len(st.candidates)):
        pages = []
        for lv in range(len(qo)):
            g = next(i for i in range(len(qo[lv]) - 1) if qo[lv][i] <= ci < qo[lv][i + 1])
            for p in kvi[lv][kvp[lv][g]:kvp[lv][g + 1]]:
                if p not in pages:
                    pages.append(p)
        out.append(pages)
    return out


@pytest.mark.parametrize("name", ["cascade_md", "swapped", "uneven"])
def test_reconstruction_invariant(name):
    tree = FX["trees"][name]
    st = build_tree(tree, tree["page_size"])
    qo, kvp, kvi, _, _ = st.get_cascade_input()
    rec = reconstruct(st, qo, kvp, kvi)
    for ci in range(len(st.candidates)):
        assert rec[ci] == st.path_pages(ci)


def run_trace(trace):
    alloc = OracleAllocator(trace["max_num_pages"], trace["page_size"])
    st = OracleBeamState(trace["beam_size"], alloc)
    made = st.add_root_sequence(trace["prompt"])
    assert [n.page_id for n in made] == trace["after_root"]["pages"]
    assert len(made[-1].tokens) == trace["after_root"]["last_page_len"]
    for step in trace["steps"]:
        ncopies = len(alloc.copies)
        results = [OResult(c, [tuple(x) for x in ch]) for c, ch in zip(st.candidates, step["select"])]
        st.add_filtered_results(results)
        got = [{"page": c.node.page_id, "tokens": c.node.tokens, "score": c.score} for c in st.candidates]
        assert got == step["expect_candidates"]
        assert [list(x) for x in alloc.copies[ncopies:]] == step["expect_copies"]
        if "expect_free_list" in step:
            assert alloc.free_pages == step["expect_free_list"]
        qo, kvp, kvi, lpl, qids = st.get_cascade_input()
        e = step["expect_cascade"]
        assert (qo, kvp, kvi, lpl, qids) == (e["qo_indptr"], e["kv_indptr"], e["kv_indices"],
                                             e["last_page_len"], e["query_ids"])
        wp, wpos = st.write_locations()
        assert wp == step["expect_write_pages"] and wpos == step["expect_write_pos"]
        assert st.position_ids() == step["expect_position_ids"]
    return st


def test_fork_trace():
    run_trace(FX["fork_trace"])


def test_planted_fork_order_mistake_is_caught():
    """If the oracle appended the first child before copying (instead of
    copies first), the copy would carry one extra token: the trace must fail."""
    class Wrong(OracleBeamState):
        def add_filtered_results(self, results):
            for r in results:
                if len(r.children) > 1 and len(r.cand.node.tokens) < self.alloc.page_size:
                    r.cand.node.tokens.append(-7)   # corrupt: extra token before the copy
            return super().add_filtered_results(results)
    trace = FX["fork_trace"]
    alloc = OracleAllocator(trace["max_num_pages"], trace["page_size"])
    st = Wrong(trace["beam_size"], alloc)
    st.add_root_sequence(trace["prompt"])
    step = trace["steps"][0]
    st.add_filtered_results([OResult(st.candidates[0], [tuple(x) for x in step["select"][0]])])
    got = [{"page": c.node.page_id, "tokens": c.node.tokens, "score": c.score} for c in st.candidates]
    assert got != step["expect_candidates"]


def random_run(seed, page_size=4, beam=4, steps=30, prompt_len=9):
    rng = random.Random(seed)
    alloc = OracleAllocator(4096, page_size)
    st = OracleBeamState(beam, alloc)
    st.add_root_sequence(list(range(prompt_len)))
    first = [(1000 + j, -0.1 * j) for j in range(beam)]
    st.add_filtered_results([OResult(st.candidates[0], first)])
    for s in range(steps):
        pool = []
        for ci, c in enumerate(st.candidates):
            for j in range(2 * beam):
                pool.append((ci, rng.randrange(50000), c.score - rng.random()))
        pool.sort(key=lambda t: t[2], reverse=True)
        chosen = pool[:beam]
        results = [OResult(c, [(t, sc) for (ci2, t, sc) in chosen if ci2 == ci]) for ci, c in enumerate(st.candidates)]
        st.add_filtered_results(results)
        yield st, s


@pytest.mark.parametrize("seed", range(6))
def test_random_run_invariants(seed):
    prompt_len = 9
    for st, s in random_run(seed, prompt_len=prompt_len):
        ps = st.alloc.page_size
        # every candidate path: ancestors full, total tokens = prompt + steps + 1
        for ci, c in enumerate(st.candidates):
            n = c.node.parent
            while n is not None:
                assert len(n.tokens) == ps
                n = n.parent
            assert len(st.sequence(ci)) == prompt_len + s + 2
        # live pages are exactly the allocated set, no page used twice
        live = set()
        stack = [st.root]
        while stack:
            n = stack.pop()
            assert n.page_id not in live
            live.add(n.page_id)
            stack.extend(n.children)
        assert live == st.alloc.allocated_pages
        assert not (live & set(st.alloc.free_pages))
        # reconstruction
        qo, kvp, kvi, lpl, _ = st.get_cascade_input()
        rec = reconstruct(st, qo, kvp, kvi)
        for ci in range(len(st.candidates)):
            assert rec[ci] == st.path_pages(ci)
        # groups are contiguous candidate ranges covering all candidates
        for lv in range(len(qo)):
            assert qo[lv][0] == 0 and qo[lv][-1] == len(st.candidates)


def _final_ranking_case():
    """Page size 4: root [1, 2, 3, 4] with children A [5, 6], B [7], C [8];
    live candidates A (score -1.0) and B (-0.6), finished F at C (-0.9) read
    from the trie, and finished E with its own sequence [1, 2, 3, 4, 9, 0]
    (score -1.2)."""
    alloc = OracleAllocator(8, 4)
    st = OracleBeamState(2, alloc)
    root = ONode([1, 2, 3, 4], 0)
    a, b, c = ONode([5, 6], 1, root), ONode([7], 2, root), ONode([8], 3, root)
    st.root = root
    st.candidates = [OCand(a, -1.0), OCand(b, -0.6)]
    st.finished_candidates = [OCand(c, -0.9), OCand(b, -1.2, sequence=[1, 2, 3, 4, 9, 0])]
    return st


def test_final_sequences_hand_case_with_finished():
    """beam_state.py:646-682 by hand.  Lengths: A 6, B 5, F 5, E 6.
    Penalty 1: A -1/6 = -0.1667, B -0.6/5 = -0.12, F -0.9/5 = -0.18, E -1.2/6 = -0.2
    -> B, A, F, E.  Penalty 0: B -0.6, F -0.9, A -1.0, E -1.2."""
    st = _final_ranking_case()
    got = st.get_final_sequences(4, 1.0)
    assert [s for s, _ in got] == [[1, 2, 3, 4, 7], [1, 2, 3, 4, 5, 6], [1, 2, 3, 4, 8], [1, 2, 3, 4, 9, 0]]
    assert [round(x, 6) for _, x in got] == [-0.12, round(-1 / 6, 6), -0.18, -0.2]
    got0 = st.get_final_sequences(3, 0.0)
    assert got0 == [([1, 2, 3, 4, 7], -0.6), ([1, 2, 3, 4, 8], -0.9), ([1, 2, 3, 4, 5, 6], -1.0)]


def test_final_sequences_ties_keep_finished_first():
    """Equal normalised scores keep pool order, finished candidates first
    (:658, stable sort): F at -0.6 ties B at penalty 0; a one-token sequence
    is not divided (len <= 1)."""
    alloc = OracleAllocator(4, 4)
    st = OracleBeamState(2, alloc)
    root = ONode([1, 2, 3, 4], 0)
    b = ONode([7], 1, root)
    st.candidates = [OCand(b, -0.6)]
    st.finished_candidates = [OCand(root, -0.6, sequence=[1, 2, 3, 4, 0])]
    assert st.get_final_sequences(2, 0.0) == [([1, 2, 3, 4, 0], -0.6), ([1, 2, 3, 4, 7], -0.6)]
    one = OracleBeamState(1, OracleAllocator(2, 4))
    one.candidates = [OCand(ONode([5], 0), -0.7)]
    assert one.get_final_sequences(1, 1.0) == [([5], -0.7)]
