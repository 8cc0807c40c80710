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
