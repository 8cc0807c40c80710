"""Tree decompositions and the per-step strategy picker (host logic).

Every decomposition the picker may run must give each candidate exactly the
tokens of its path once (the flat strategy's keys), whatever the edge
decisions; the float64 oracle then gives identical attention for the flat
lists and the tree levels.  The fully split decomposition of a trie whose
candidates all sit on the deepest level is the reference's cascade."""

import random
from collections import Counter

import numpy as np
import pytest

from beam_engine_amd.beam_state import BeamGenerateResult, BeamState, BeamToken
from beam_engine_amd.picker import CostModel, KernelCosts, StrategyPicker, plan_cost
from oracle import attention as oa
from tests.test_beam_state_product import RecordingPages, build_product
from tests.conftest import load_fixtures

FX = load_fixtures()


def keys_per_query(levels, page, n):
    out = [Counter() for _ in range(n)]
    for qo, kvp, kvi, lpl in levels:
        assert qo[0] == 0 and qo[-1] == n and all(a <= b for a, b in zip(qo, qo[1:]))
        assert len(kvp) == len(qo) and len(lpl) == len(qo) - 1
        for j in range(len(qo) - 1):
            npg = kvp[j + 1] - kvp[j]
            m = 0 if npg == 0 else (npg - 1) * page + lpl[j]
            assert 0 <= lpl[j] <= page and m >= 0
            keys = [(kvi[kvp[j] + t // page], t % page) for t in range(m)]
            for q in range(qo[j], qo[j + 1]):
                out[q].update(keys)
    return out


def flat_keys(st, page):
    kvp, kvi, lpl = st.flat_lists()
    return keys_per_query([(list(range(len(kvp))), kvp, kvi, lpl)], page, len(kvp) - 1)


def random_state(seed, steps=30):
    rng = random.Random(seed)
    page = rng.choice([2, 4, 16])
    beam = rng.choice([2, 3, 4, 8])
    pages = RecordingPages(20000, page)
    st = BeamState(beam, pages)
    for r in range(rng.choice([1, 2, 3])):
        st.add_root_sequence(list(range(rng.randint(1, 40))), request_id=r)
    st.add_filtered_results([BeamGenerateResult(c, [BeamToken(1000 + j, -0.25 * j) for j in range(beam)])
                             for c in st.candidates])
    states = []
    for _ in range(steps):
        res = []
        for rid in sorted({c.request_id for c in st.candidates}):
            idx = [i for i, c in enumerate(st.candidates) if c.request_id == rid]
            pool = [(i, rng.randrange(30), st.candidates[i].score - rng.random()) for i in idx for _ in range(2 * beam)]
            pool.sort(key=lambda t: t[2], reverse=True)
            chosen = pool[:beam]
            for i in idx:
                res.append(BeamGenerateResult(st.candidates[i], [BeamToken(t, s) for i2, t, s in chosen if i2 == i]))
        res.sort(key=lambda r: st.candidates.index(r.candidate))
        st.add_filtered_results(res)
        states.append(st)
    return st, page


@pytest.mark.parametrize("seed", range(10))
def test_every_decomposition_reads_each_path_token_once(seed):
    st, page = random_state(seed)
    rng = random.Random(seed + 100)
    want = flat_keys(st, page)
    model = CostModel(32, 8, page)
    deciders = {"split": lambda *a: False, "flat-like": lambda *a: True,
                "random": lambda *a: rng.random() < 0.5, "model": model.absorb}
    for name, fn in deciders.items():
        levels = st.tree_lists(fn)
        got = keys_per_query(levels, page, len(st.candidates))
        assert got == want, name


def test_split_decomposition_is_the_cascade_when_candidates_share_the_deepest_level():
    checked = 0
    for name in ("cascade_md", "swapped", "uneven"):
        st = build_product(FX["trees"][name])
        st._annotate()
        if len({c.trie_node._lvl for c in st.candidates}) != 1:
            continue
        assert st.tree_lists(lambda *a: False) == st._cascade_lists(), name
        checked += 1
    assert checked >= 1


def test_uneven_tree_differs_from_the_cascade_only_by_repeated_leaf_groups():
    # the reference cascade repeats a shallow candidate's leaf group on deeper levels
    # (each repetition counts its tokens again); the tree decomposition does not.  (This
    # hand-built fixture has partial internal pages, which the engine's own tries never
    # have, so it is compared with the cascade rather than with the flat lists.)
    st = build_product(FX["trees"]["uneven"])
    page = FX["trees"]["uneven"]["page_size"]
    n = len(st.candidates)
    tree = keys_per_query(st.tree_lists(lambda *a: False), page, n)
    casc = keys_per_query(st._cascade_lists(), page, n)
    assert all(max(t.values()) == 1 for t in tree)
    st._annotate()
    depth = [c.trie_node._lvl for c in st.candidates]
    top = max(depth)
    for q in range(n):
        extra = casc[q] - tree[q]
        assert (sum(extra.values()) > 0) == (depth[q] < top)
        assert not (tree[q] - casc[q])


@pytest.mark.parametrize("seed", [1, 4])
def test_oracle_attention_of_tree_levels_equals_flat(seed):
    st, page = random_state(seed, steps=12)
    n = len(st.candidates)
    npages = 1 + max(max(l[2]) for l in st.tree_lists(lambda *a: False) if l[2])
    rng = np.random.default_rng(seed)
    hkv, hq, d = 2, 4, 16
    kv = rng.standard_normal((npages, 2, page, hkv, d))
    q = rng.standard_normal((n, hq, d))
    kvp, kvi, lpl = st.flat_lists()
    ref, ref_lse = oa.paged_attention(q, kv, kvp, kvi, lpl, page, d ** -0.5)
    for fn in (lambda *a: False, lambda *a: True, CostModel(hq, hkv, page).absorb):
        lv = st.tree_lists(fn)
        o, lse = oa.cascade_attention(q, kv, [l[0] for l in lv], [l[1] for l in lv], [l[2] for l in lv],
                                      [l[3] for l in lv], page, d ** -0.5)
        np.testing.assert_allclose(o, ref, rtol=1e-10, atol=1e-12)
        np.testing.assert_allclose(lse, ref_lse, rtol=1e-10, atol=1e-12)


def test_cost_model_prices_tail_stream_and_rows():
    c = KernelCosts(tile_nt=(1.0, 2.0, 3.0, 4.0), seg=10.0, slot=0.5, tail=0.25, fixed=0.0, tile_sib=0.75)
    m = CostModel(32, 8, 16, c)
    assert m.group(0, 100) == 0 and m.group(3, 0) == 0
    assert m.group(2, 40) == 2 * 8 * 3 * 0.25                 # tail: 3 chunks x 2 queries x 8 heads
    assert m.group(1, 65) == 8 * 5 * 0.25                     # 65 tokens, one query: 5 tail chunks
    assert m.group(5, 65) == 8 * (2 * 2.0 + 10.0)             # 20 rows: two 16-row tiles, 2 tiles
    assert m.group(1, 129) == 8 * (3 * 1.0 + 10.0)            # 4 rows: one 16-row tile, 3 tiles
    assert m.group(16, 64) == 8 * (4.0 + 10.0)                # 64 rows: a full segment
    assert m.group(20, 64) == 8 * (4.0 + 10.0 + 0.75 + 10.0)  # 80 rows: 64 + a 16-row sibling tile
    assert m.group(64, 128) == 8 * (2 * 4.0 + 10.0 + 3 * (2 * 0.75 + 10.0))   # 256 rows: 1 + 3 siblings
    assert CostModel(32, 8, 8, c).group(2, 40) == 8 * (1.0 + 10.0)   # page 8: no tail pass
    # wide segments: more than 64 rows, at least 8 tiles, and 64 x 256 tiles of
    # 64 rows over the KV heads (the planner's 128- / 256-row tasks)
    cw = KernelCosts(tile_nt=(1.0, 2.0, 3.0, 4.0), seg=10.0, slot=0.5, tail=0.25, fixed=0.0, tile_w128=6.0,
                     tile_w256=9.0, tile_sib=4.0)
    m8 = CostModel(64, 8, 16, cw)
    assert m8.group(64, 16384) == 8 * (256 * 9.0 + 10.0) * 2        # 512 rows: two 256-row segments
    assert m8.group(40, 16384 * 2) == 8 * (512 * 9.0 + 10.0 + 512 * 9.0 + 10.0)   # 320 rows: 256 + 64
    assert m8.group(24, 16384 * 3) == 8 * (768 * 6.0 + 10.0) * 2    # 192 rows: two 128-row segments
    assert m8.group(64, 8192) == 8 * (128 * 4.0 + 10.0) * 8         # 8 x 128 x 8 tiles64: below the bar
                                                                    # (tile_sib = tile_nt[3] here)
    assert CostModel(32, 8, 16, cw).group(16, 1 << 20) == 8 * ((1 << 14) * 4.0 + 10.0)   # 64 rows: never wide
    # absorbing a short parent into a single child saves a pass and a slot
    assert m.absorb(1, 1, 16, 16)
    # a long parent shared by many queries stays a separate pass
    assert not m.absorb(64, 1, 4096, 16)


def test_picker_prefers_shared_passes_for_a_shared_prefix_and_flat_without_sharing():
    page = 16
    pages = RecordingPages(20000, page)
    st = BeamState(8, pages)
    st.add_root_sequence(list(range(2048)))
    st.add_filtered_results([BeamGenerateResult(st.candidates[0], [BeamToken(j, -j) for j in range(8)])])
    pk = StrategyPicker(32, 8, page)
    plan = pk.choose(st)
    assert plan.kind in ("split", "tree")
    costs = pk.costs(st)
    fixed = pk.model.c.fixed                  # both launches: paid by every option
    assert costs["flat"] - fixed > 2 * (min(costs["split"], costs["tree"]) - fixed)
    assert plan.cost == min(costs.values()) and plan.costs == costs
    # one candidate per request: nothing is shared, every decomposition is one pass per query
    st2 = BeamState(1, RecordingPages(20000, page))
    for r in range(4):
        st2.add_root_sequence(list(range(100 + r)), request_id=r)
    costs2 = pk.costs(st2)
    assert costs2["flat"] == pytest.approx(costs2["tree"]) and costs2["flat"] <= costs2["split"] + 1e-9
    assert plan_cost(pk.model, st2.tree_lists(lambda *a: True), page)[1] == 4


@pytest.mark.parametrize("seed", range(6))
def test_segment_tree_costs_match_the_level_arrays(seed):
    """The picker costs decompositions on the segment tree; laid out as level
    arrays they cost the same (up to candidates split into several runs)."""
    st, page = random_state(seed)
    pk = StrategyPicker(32, 8, page)
    segs, paths = st.segment_tree()
    opts = pk.options(segs, paths)
    for kind, (cost, absorbed) in opts.items():
        levels = st.tree_levels(segs, paths, absorbed)
        lv_cost, _ = plan_cost(pk.model, levels, page)
        # a segment's candidates may form several runs, each priced as its own group
        assert cost - 1e-9 <= lv_cost <= 1.5 * cost, kind
