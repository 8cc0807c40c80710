"""The native beam trie (be_beam_trie) and page pool (be_page_pool) against
the Python BeamState and the reference allocator rules, step by step, on the
host: the same random selections (deaths, single children, forks of full and
partial pages, end-of-sequence picks, several requests) give the same
candidates (page, tokens, score, request), the same page free list, the same
fork copies in the same order and the same cascade metadata."""

import random

import numpy as np
import pytest
import torch

from beam_engine_amd.beam_state import BeamGenerateResult, BeamState, BeamToken, NativeBeamState
from beam_engine_amd.page_table import PageTable


def make_pt(pages, page_size):
    pt = PageTable(1, page_size=page_size, max_num_pages=pages, head_num=1, head_dim=8, device="cpu",
                   store_dtype=torch.float32)
    pt._defer = 1          # keep every fork copy pending: the test compares the lists (no device here)
    return pt


def random_results(st, rng, beam, eos=None, p_eos=0.0):
    """Per request: some beams die, some fork two or three ways, the rest go
    on with one child; children of a beam in a random score order."""
    res = []
    cands = st.candidates
    for rid in sorted({c.request_id for c in cands}):
        idx = [i for i, c in enumerate(cands) if c.request_id == rid]
        kids = {i: 1 for i in idx}
        budget = beam
        for i in idx:
            r = rng.random()
            kids[i] = 0 if r < 0.25 else (1 if r < 0.6 else rng.choice([2, 3]))
        total = sum(kids.values())
        while total > budget:                     # at most `beam` children per request
            i = rng.choice([j for j in idx if kids[j] > 0])
            kids[i] -= 1
            total -= 1
        if total == 0:
            kids[idx[0]] = 1
        for i in idx:
            c = cands[i]
            ch = []
            for _ in range(kids[i]):
                t = eos if (eos is not None and rng.random() < p_eos) else rng.randrange(1000)
                ch.append(BeamToken(t, c.score - rng.random()))
            res.append(BeamGenerateResult(c, ch))
    return res


def snapshot(st):
    return [(c.trie_node.page_id, list(c.trie_node.tokens), c.score, c.request_id) for c in st.candidates]


@pytest.mark.parametrize("page_size,steps,seed,eos", [(4, 60, 1, None), (16, 80, 2, None), (4, 50, 3, 7),
                                                       (8, 70, 4, 11), (2, 400, 6, None)])
def test_native_trie_matches_python_state(page_size, steps, seed, eos):
    rng_a, rng_b = random.Random(seed), random.Random(seed)
    beam = 6
    pa, pb = make_pt(4096, page_size), make_pt(4096, page_size)
    a = BeamState(beam, pa, fast_metadata=True)
    b = NativeBeamState(beam, pb)
    rp = random.Random(seed + 100)
    prompts = [[rp.randrange(1000) for _ in range(rp.choice([1, 5, 9, 17]))] for _ in range(3)]
    for r, p in enumerate(prompts):
        na = a.add_root_sequence(list(p), request_id=r)
        nb = b.add_root_sequence(list(p), request_id=r)
        assert [n.page_id for n in na] == [n.page_id for n in nb]
    # the prefill's first children: beam tokens per request
    first = [[BeamToken(100 + j, -0.1 * j) for j in range(beam)] for _ in prompts]
    a.add_filtered_results([BeamGenerateResult(c, first[i]) for i, c in enumerate(a.candidates)])
    b.add_filtered_results([BeamGenerateResult(c, first[i]) for i, c in enumerate(b.candidates)])
    for step in range(steps):
        ra = random_results(a, rng_a, beam, eos, 0.1)
        rb = random_results(b, rng_b, beam, eos, 0.1)
        a.add_filtered_results(ra, eos)
        b.add_filtered_results(rb, eos)
        assert snapshot(a) == snapshot(b), f"candidates differ after step {step}"
        assert list(pa.free_pages) == list(pb.free_pages), f"free list differs after step {step}"
        assert pa._pending == pb._pending, f"fork copies differ after step {step}"
        assert [(c.score, c.request_id, list(c.sequence)) for c in a.finished_candidates] == \
            [(c.score, c.request_id, list(c.sequence)) for c in b.finished_candidates]
        if not a.candidates:
            break
        ma, mb = a.step_metadata(), b.step_metadata()
        assert len(ma[0]) == len(mb[0])
        for la, lb in zip(ma[0], mb[0]):
            for xa, xb in zip(la, lb):
                assert np.array_equal(np.asarray(xa), np.asarray(xb)), f"cascade arrays differ after step {step}"
        for xa, xb in zip(ma[1:], mb[1:]):
            assert np.array_equal(np.asarray(xa), np.asarray(xb)), f"candidate inputs differ after step {step}"
    assert pa._pending, "the run should fork partial pages"
    if steps >= 400:
        # long runs compact the native node table (dead nodes dropped, order kept)
        sz = b._read_sizes()
        assert sz[0] < a._tab.n, "the native table should have been compacted"
    # the Python view of the native state reads like the Python state
    assert [len(r.tokens) for r in a.roots] == [len(r.tokens) for r in b.roots]
    for rid in range(3):
        assert a.get_final_sequences(4, 1.0, rid) == b.get_final_sequences(4, 1.0, rid)


def test_native_apply_arrays_equal_results_path():
    """apply_selection with the selection arrays (the decode loop's path)
    equals add_filtered_results with the same children."""
    rng = random.Random(9)
    pa, pb = make_pt(1024, 4), make_pt(1024, 4)
    a, b = NativeBeamState(4, pa), NativeBeamState(4, pb)
    for st in (a, b):
        st.add_root_sequence([1, 2, 3, 4, 5, 6], request_id=0)
        st.add_root_sequence([9, 8], request_id=1)
    for step in range(30):
        res = random_results(a, rng, 4)
        par, tok, sc = [], [], []
        for i, r in enumerate(res):
            for ch in r.children:
                par.append(i)
                tok.append(ch.token_id)
                sc.append(ch.accumulated_score)
        # unused entries (parent -1) are skipped
        par.insert(0, -1), tok.insert(0, 0), sc.insert(0, 0.0)
        a.add_filtered_results(res)
        b.apply_selection(np.array(par), np.array(tok), np.array(sc))
        assert snapshot(a) == snapshot(b)
        assert list(pa.free_pages) == list(pb.free_pages) and pa._pending == pb._pending


def test_page_pool_fifo_and_refcounts():
    """The native allocator keeps the reference's FIFO order: oldest free
    page first, freed pages to the back; shared pages free at the last
    holder; an unallocated free only warns; exhaustion is MemoryError."""
    pt = make_pt(5, 4)
    got = [pt.allocate_block() for _ in range(3)]
    assert got == [0, 1, 2] and list(pt.free_pages) == [3, 4]
    pt.free_block(1)
    assert list(pt.free_pages) == [3, 4, 1]
    assert pt.share_block(0) == 2
    pt.free_block(0)
    assert pt.ref_count(0) == 1 and 0 not in pt.free_pages
    pt.free_block(0)
    assert list(pt.free_pages) == [3, 4, 1, 0]
    pt.free_block(0)                       # not allocated: a warning, no change
    assert list(pt.free_pages) == [3, 4, 1, 0]
    assert pt.reserve_block(1) == 1 and list(pt.free_pages) == [3, 4, 0]
    with pytest.raises(ValueError):
        pt.reserve_block(2)
    assert [pt.allocate_block() for _ in range(3)] == [3, 4, 0]
    with pytest.raises(MemoryError):
        pt.allocate_block()
    assert pt.allocated_pages == {0, 1, 2, 3, 4} and pt.num_free_pages() == 0


@pytest.mark.parametrize("caps", [False, True])
def test_trie_plan_equals_attn_plan_of_its_metadata(caps):
    """be_trie_plan (metadata and plan in one native call) writes the same
    plan words and plan info as be_attn_plan over be_trie_metadata's levels,
    compact and fixed-layout."""
    import ctypes
    from beam_engine_amd import _lib
    from beam_engine_amd.beam_state import _parse_metadata
    lib = _lib.load()
    rng = random.Random(5)
    pt = make_pt(8192, 16)
    st = NativeBeamState(8, pt)
    for r in range(3):
        st.add_root_sequence([rng.randrange(1000) for _ in range(150 + 40 * r)], request_id=r)
    st.add_filtered_results([BeamGenerateResult(c, [BeamToken(100 + j, -0.1 * j) for j in range(8)])
                             for c in st.candidates])
    for _ in range(25):
        st.add_filtered_results(random_results(st, rng, 8))
    n = st.num_candidates()
    cp = _lib.BePlanCaps(4096, n, 16384, n * 8, 4096, n, 64, 8192) if caps else None
    cpp = ctypes.byref(cp) if caps else None
    hq, hkv, d = 32, 8, 128
    meta = np.zeros(1 << 18, np.int32)
    used = ctypes.c_int64(0)
    plan_a = np.zeros(1 << 21, np.int32)
    info_a = _lib.BeAttnPlanInfo()
    mp = ctypes.c_int32(0)
    _lib.check(lib.be_trie_plan(st._h, hq, hkv, d, _lib.BE_BF16, 0, 256, cpp, meta.ctypes.data, meta.size,
                                ctypes.byref(used), plan_a.ctypes.data, plan_a.size, ctypes.byref(info_a),
                                ctypes.byref(mp)), "trie plan")
    levels, *_ = _parse_metadata(meta[: used.value].copy(), n)
    arr = (_lib.BeLevel * len(levels))()
    keep = []
    for i, (qo, kvp, kvi, lpl) in enumerate(levels):
        qo, kvp, kvi, lpl = (np.ascontiguousarray(x, np.int32) for x in (qo, kvp, kvi, lpl))
        keep += [qo, kvp, kvi, lpl]
        arr[i] = _lib.BeLevel(qo.ctypes.data, kvp.ctypes.data, kvi.ctypes.data if len(kvi) else 0, lpl.ctypes.data,
                              len(qo) - 1)
    max_page = max(int(np.max(l[2])) for l in levels if len(l[2]))
    assert mp.value == max_page
    plan_b = np.zeros_like(plan_a)
    info_b = _lib.BeAttnPlanInfo()
    _lib.check(lib.be_attn_plan(arr, len(levels), n, hq, hkv, d, 16, max_page + 1, _lib.BE_BF16, 0, 256, cpp,
                                plan_b.ctypes.data, plan_b.size, ctypes.byref(info_b)), "attention plan")
    assert bytes(info_a) == bytes(info_b)
    assert info_a.kernel == 2 and info_a.static_layout == int(caps)
    assert np.array_equal(plan_a[: info_a.plan_ints], plan_b[: info_b.plan_ints])


def _py_levels(st, kind, include_self, picker):
    """The Python restatement's levels of one strategy (BeamState.segment_tree /
    absorb_edges / tree_levels, StrategyPicker.choose)."""
    if kind == "auto":
        plan = picker.choose(st, include_self)
        return plan.levels, plan.kind, [plan.costs["flat"], plan.costs["split"], plan.costs["tree"]]
    segs, paths = st.segment_tree(include_self)
    if kind == "flat":
        absorbed = set(k for k, sg in enumerate(segs) if sg[2] >= 0)
    elif kind == "split":
        absorbed = set()
    else:
        absorbed, _ = st.absorb_edges(segs, (picker.edges or picker.model).absorb)
    return st.tree_levels(segs, paths, absorbed), kind, None


@pytest.mark.parametrize("page_size,hq,hkv,edges,seed", [(4, 32, 8, "mi355x", 11), (16, 32, 8, "fasttree", 12),
                                                         (16, 64, 8, "mi355x", 13), (8, 8, 8, "fasttree", 14),
                                                         (16, 32, 8, "mi355x", 15)])
def test_native_levels_match_python_decompositions(page_size, hq, hkv, edges, seed):
    """be_trie_levels (flat, split, tree, auto; with and without each
    candidate's newest token) gives the Python restatement's level arrays,
    kind and modelled option costs exactly, on random multi-request tries."""
    from beam_engine_amd.picker import MI355X, StrategyPicker
    rng_a, rng_b = random.Random(seed), random.Random(seed)
    beam = 8
    pa, pb = make_pt(8192, page_size), make_pt(8192, page_size)
    a = BeamState(beam, pa, fast_metadata=True)
    b = NativeBeamState(beam, pb)
    rp = random.Random(seed + 7)
    for r in range(3):
        p = [rp.randrange(1000) for _ in range(rp.choice([3, 17, 70, 200]))]
        a.add_root_sequence(list(p), request_id=r)
        b.add_root_sequence(list(p), request_id=r)
    first = [BeamToken(100 + j, -0.1 * j) for j in range(beam)]
    a.add_filtered_results([BeamGenerateResult(c, first) for c in a.candidates])
    b.add_filtered_results([BeamGenerateResult(c, first) for c in b.candidates])
    picker = StrategyPicker(hq, hkv, page_size, "fasttree" if edges == "fasttree" else MI355X)
    model = picker.tree_model()
    checked = 0
    for step in range(40):
        a.add_filtered_results(random_results(a, rng_a, beam))
        b.add_filtered_results(random_results(b, rng_b, beam))
        if step % 3:
            continue
        for kind in ("flat", "split", "tree", "auto"):
            for inc in (False, True):
                want, want_kind, want_costs = _py_levels(a, kind, inc, picker)
                levels, qids, wp, ws, pos, got_kind, got_costs = b.step_levels(kind, inc, model)
                assert got_kind == want_kind, (step, kind, inc)
                assert len(levels) == len(want), (step, kind, inc)
                for lg, lw in zip(levels, want):
                    for xg, xw in zip(lg, lw):
                        assert np.array_equal(np.asarray(xg), np.asarray(xw, dtype=np.int32)), (step, kind, inc)
                if want_costs is not None:
                    assert list(got_costs) == want_costs, (step, kind, inc)
                assert list(qids) == a.query_token_ids()
                assert (list(wp), list(ws)) == tuple(map(list, a.write_locations()))
                assert list(pos) == a.position_ids()
                if kind == "flat":
                    kvp, kvi, lpl = a.flat_lists(inc)
                    assert list(levels[0][0]) == list(range(len(lpl) + 1))
                    assert (list(levels[0][1]), list(levels[0][2]), list(levels[0][3])) == (kvp, kvi, lpl)
                checked += 1
    assert checked >= 8 * 10


def test_trie_plan_kind_equals_attn_plan_of_its_levels():
    """be_trie_plan_kind writes the plan be_attn_plan gives for the levels of
    be_trie_metadata_kind (no causal mask outside the cascade kind)."""
    import ctypes
    from beam_engine_amd import _lib
    from beam_engine_amd.beam_state import _parse_metadata
    from beam_engine_amd.picker import StrategyPicker
    lib = _lib.load()
    rng = random.Random(21)
    pt = make_pt(8192, 16)
    st = NativeBeamState(8, pt)
    for r in range(3):
        st.add_root_sequence([rng.randrange(1000) for _ in range(150 + 40 * r)], request_id=r)
    st.add_filtered_results([BeamGenerateResult(c, [BeamToken(100 + j, -0.1 * j) for j in range(8)])
                             for c in st.candidates])
    for _ in range(25):
        st.add_filtered_results(random_results(st, rng, 8))
    n = st.num_candidates()
    hq, hkv, d = 32, 8, 128
    model = StrategyPicker(hq, hkv, 16, "fasttree").tree_model()
    for kind in ("flat", "split", "tree", "auto"):
        meta = np.zeros(1 << 18, np.int32)
        used = ctypes.c_int64(0)
        plan_a = np.zeros(1 << 21, np.int32)
        info_a = _lib.BeAttnPlanInfo()
        mp, chosen = ctypes.c_int32(0), ctypes.c_int32(-1)
        _lib.check(lib.be_trie_plan_kind(st._h, _lib.KIND_CODES[kind], 1, ctypes.byref(model), hq, hkv, d,
                                         _lib.BE_BF16, 0, 256, None, meta.ctypes.data, meta.size, ctypes.byref(used),
                                         plan_a.ctypes.data, plan_a.size, ctypes.byref(info_a), ctypes.byref(mp),
                                         ctypes.byref(chosen), None), "trie plan")
        levels, *_ = _parse_metadata(meta[: used.value].copy(), n)
        ref = st.step_levels(kind, True, model)
        assert ref[5] == _lib.KIND_NAMES[chosen.value]
        for lg, lw in zip(levels, ref[0]):
            for xg, xw in zip(lg, lw):
                assert np.array_equal(xg, xw)
        arr = (_lib.BeLevel * len(levels))()
        keep = []
        for i, (qo, kvp, kvi, lpl) in enumerate(levels):
            qo, kvp, kvi, lpl = (np.ascontiguousarray(x, np.int32) for x in (qo, kvp, kvi, lpl))
            keep += [qo, kvp, kvi, lpl]
            arr[i] = _lib.BeLevel(qo.ctypes.data, kvp.ctypes.data, kvi.ctypes.data if len(kvi) else 0,
                                  lpl.ctypes.data, len(qo) - 1)
        max_page = max(int(np.max(l[2])) for l in levels if len(l[2]))
        plan_b = np.zeros_like(plan_a)
        info_b = _lib.BeAttnPlanInfo()
        _lib.check(lib.be_attn_plan(arr, len(levels), n, hq, hkv, d, 16, max_page + 1, _lib.BE_BF16, 0, 256, None,
                                    plan_b.ctypes.data, plan_b.size, ctypes.byref(info_b)), "attention plan")
        assert bytes(info_a) == bytes(info_b)
        assert np.array_equal(plan_a[: info_a.plan_ints], plan_b[: info_b.plan_ints])


def test_trie_apply_fails_before_changing_state_when_pages_run_out():
    """A selection whose expansion needs more pages than the pool holds after
    the prune raises MemoryError and leaves the trie, its candidates, the
    free list and the version as they were; the same selection succeeds once
    the pool has room (pages the prune frees count as room)."""
    pt = make_pt(10, 4)
    st = NativeBeamState(4, pt)
    st.add_root_sequence([1, 2, 3, 4], request_id=0)         # one full page
    st.add_root_sequence([5, 6], request_id=1)               # one partial page
    before = (snapshot(st), list(pt.free_pages), int(st._read_sizes()[0]))
    ver = st._ver.value
    # candidate 0 forks 4 ways on a full page (4 pages), candidate 1 forks 4
    # ways on a partial page (3 copies): 7 pages, 8 free -> fine; take 2 first
    held = [pt.allocate_block(), pt.allocate_block()]
    par = [0, 0, 0, 0, 1, 1, 1, 1]
    tok = [10, 11, 12, 13, 20, 21, 22, 23]
    sc = [-0.1 * i for i in range(8)]
    with pytest.raises(MemoryError):
        st.apply_selection(par, tok, sc)
    assert (snapshot(st), list(pt.free_pages), int(st._read_sizes()[0])) == \
        (before[0], list(pt.free_pages), before[2])
    assert st._ver.value == ver and pt._pending == []
    pt.free_block(held[0])
    st.apply_selection(par, tok, sc)                         # 7 pages needed, 7 free
    assert len(st.candidates) == 8 and pt.num_free_pages() == 0
    # the prune's pages count: no page is free, the first candidate (one
    # token on its page) forks 4 ways (3 copies) and the other 7 die, freeing
    # 7 pages first
    st.apply_selection([0, 0, 0, 0], [30, 31, 32, 33], [-1.0, -1.1, -1.2, -1.3])
    assert len(st.candidates) == 4 and pt.num_free_pages() == 4


@pytest.mark.parametrize("page_size,hq,hkv,seed", [(4, 32, 8, 31), (16, 32, 8, 32), (16, 64, 8, 33)])
def test_fasttree_boundary_levels_equal_native_fasttree_kind(page_size, hq, hkv, seed):
    """The reference's FastTree call path -- BeamState.get_fasttree_input ->
    prepare_fasttree_metadata_for_paged_cache -- plans the same levels as the
    engine's native "fasttree" kind (be_trie_levels with FastTree's edges and
    each candidate's newest token) on the same trie, and those attend each
    candidate to exactly its req_to_token row: per level, every query's pages
    and token counts, concatenated, give its whole path."""
    from beam_engine_amd.fasttree import fasttree_levels
    from beam_engine_amd.picker import StrategyPicker
    rng_a, rng_b = random.Random(seed), random.Random(seed)
    beam = 8
    pa, pb = make_pt(8192, page_size), make_pt(8192, page_size)
    a = BeamState(beam, pa, fast_metadata=True)
    b = NativeBeamState(beam, pb)
    rp = random.Random(seed + 3)
    for r in range(3):
        p = [rp.randrange(1000) for _ in range(rp.choice([5, 40, 130]))]
        a.add_root_sequence(list(p), request_id=r)
        b.add_root_sequence(list(p), request_id=r)
    first = [BeamToken(100 + j, -0.1 * j) for j in range(beam)]
    a.add_filtered_results([BeamGenerateResult(c, first) for c in a.candidates])
    b.add_filtered_results([BeamGenerateResult(c, first) for c in b.candidates])
    model = StrategyPicker(hq, hkv, page_size, "fasttree").tree_model()
    for step in range(30):
        a.add_filtered_results(random_results(a, rng_a, beam))
        b.add_filtered_results(random_results(b, rng_b, beam))
        tree_nodes, req_to_token, qids, wp, wpos = a.get_fasttree_input()
        n = len(a.candidates)
        got = fasttree_levels(tree_nodes, req_to_token, n, hq, hkv, page_size)
        want = b.step_levels("tree", True, model)[0]
        assert len(got) == len(want), step
        for lg, lw in zip(got, want):
            for xg, xw in zip(lg, lw):
                assert np.array_equal(np.asarray(xg, np.int32), np.asarray(xw)), step
        # every query's slots over the levels = its req_to_token row
        rtt = req_to_token.cpu().numpy()
        for ci in range(n):
            slots = []
            for qo, kvp, kvi, lpl in got:
                j = int(np.searchsorted(qo, ci, side="right")) - 1
                pages = kvi[kvp[j]: kvp[j + 1]]
                for t, pg in enumerate(pages):
                    cnt = page_size if t + 1 < len(pages) else lpl[j]
                    slots.extend(pg * page_size + i for i in range(cnt))
            length = sum(len(x.tokens) for x in _path(a.candidates[ci].trie_node))
            assert sorted(slots) == sorted(rtt[ci, :length].tolist()), (step, ci)


def _path(node):
    out = []
    while node is not None:
        out.append(node)
        node = node.parent
    return out[::-1]


def test_native_costs_price_wide_segments_like_python():
    """On a trie whose shared prompts are long enough for the planner's wide
    segments (2 requests x 64 beams, GQA 8, 16384-token prompts), the native
    option costs equal the Python picker's (wide pricing included)."""
    from beam_engine_amd.picker import MI355X, StrategyPicker
    rng_a, rng_b = random.Random(71), random.Random(71)
    pa, pb = make_pt(8192, 16), make_pt(8192, 16)
    a = BeamState(64, pa, fast_metadata=True)
    b = NativeBeamState(64, pb)
    for r in range(2):
        a.add_root_sequence(list(range(16384)), request_id=r)
        b.add_root_sequence(list(range(16384)), request_id=r)
    first = [BeamToken(100 + j, -0.01 * j) for j in range(64)]
    a.add_filtered_results([BeamGenerateResult(c, first) for c in a.candidates])
    b.add_filtered_results([BeamGenerateResult(c, first) for c in b.candidates])
    for _ in range(20):
        a.add_filtered_results(random_results(a, rng_a, 64))
        b.add_filtered_results(random_results(b, rng_b, 64))
    picker = StrategyPicker(64, 8, 16, MI355X)
    plan = picker.choose(a)
    got = b.step_levels("auto", False, picker.tree_model())
    assert got[5] == plan.kind and list(got[6]) == [plan.costs["flat"], plan.costs["split"], plan.costs["tree"]]
    segs, _ = a.segment_tree()
    root = max(segs, key=lambda sg: sg[1])
    assert picker.model.group(len(root[3]), root[1]) < 0.9 * CostModelNoWide(picker).group(len(root[3]), root[1])


def CostModelNoWide(picker):
    """The same costs with the wide segments priced as 64-row ones."""
    from dataclasses import replace
    from beam_engine_amd.picker import CostModel
    c = picker.model.c
    return CostModel(64, 8, 16, replace(c, tile_w128=c.tile_nt[3] * 2, tile_w256=c.tile_nt[3] * 4))
