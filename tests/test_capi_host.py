"""Host-side checks of the C ABI (no GPU needed): the library loads and
exports every function include/beam_engine_amd.h declares, and the attention
planner (host code) validates its inputs and produces a consistent work list."""

import ctypes
import os
import re

import numpy as np
import pytest

from tests.conftest import ROOT

HEADER = os.path.join(ROOT, "include", "beam_engine_amd.h")
TILE = 4      # BE_PLAN_TILE_KERNEL
_NO_TAIL_ROLE = 2048   # BE_PLAN_NO_TAIL_ROLE


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(be_[a-z0-9_]+)\s*\(", text)))


def lib():
    from beam_engine_amd import _lib
    if not os.path.exists(_lib.LIB_PATH):
        pytest.skip("HIP library not built (run __graft_entry__.build())")
    return _lib, _lib.load()


def test_library_exports_every_declared_symbol():
    _lib, L = lib()
    names = declared_functions()
    assert len(names) >= 9
    for n in names:
        assert hasattr(L, n), n
    assert set(names) == set(_lib.EXPORTS)
    assert L.be_version() >= 100


def plan(levels, nq=None, hq=8, hkv=2, d=128, page=4, num_pages=64, dtype=2, flags=0, cus=256, caps=None):
    _lib, L = lib()
    keep = []
    arr = (_lib.BeLevel * len(levels))()
    for i, (qo, kvp, kvi, lpl) in enumerate(levels):
        a = [np.asarray(x, dtype=np.int32) for x in (qo, kvp, kvi, lpl)]
        keep.append(a)
        arr[i] = _lib.BeLevel(a[0].ctypes.data, a[1].ctypes.data, a[2].ctypes.data if len(a[2]) else 0,
                              a[3].ctypes.data, len(a[0]) - 1)
    if nq is None:
        nq = max(int(l[0][-1]) for l in levels)
    buf = np.zeros(1 << 20, dtype=np.int32)
    info = _lib.BeAttnPlanInfo()
    rc = L.be_attn_plan(arr, len(levels), nq, hq, hkv, d, page, num_pages, dtype, flags, cus,
                        ctypes.byref(caps) if caps is not None else None, buf.ctypes.data, buf.size,
                        ctypes.byref(info))
    return rc, info, buf, _lib, L


def decode_items(info, buf):
    it = buf[info.off_items: info.off_items + 8 * info.num_items].reshape(-1, 8)
    return it


def test_plan_covers_every_token_once_per_query():
    # A.1-shaped cascade (page 4), bf16
    levels = [([0, 8], [0, 4], [0, 1, 2, 3], [1]),
              ([0, 3, 5, 8], [0, 2, 4, 6], [4, 5, 6, 7, 8, 9], [1, 1, 1]),
              ([0, 1, 2, 3, 4, 5, 6, 7, 8], [0, 1, 3, 4, 5, 6, 7, 8, 9],
               [10, 11, 12, 13, 14, 15, 16, 17, 18], [1, 1, 1, 0, 0, 3, 3, 3])]
    rc, info, buf, _lib, L = plan(levels, hq=8, hkv=2, num_pages=19, flags=TILE)
    assert rc == 0, L.be_last_error()
    items = decode_items(info, buf)
    # every query sees exactly the tokens of its groups
    cover = {q: 0 for q in range(8)}
    for q0, qn, pb, t0, tc, orow, _, _ in items:
        assert tc > 0 and qn > 0
        for q in range(q0, q0 + qn):
            cover[q] += tc
    expect = {}
    for qo, kvp, kvi, lpl in levels:
        for g in range(len(qo) - 1):
            npg = kvp[g + 1] - kvp[g]
            n = 0 if npg == 0 else (npg - 1) * 4 + lpl[g]
            for q in range(qo[g], qo[g + 1]):
                expect[q] = expect.get(q, 0) + n
    assert cover == expect
    # merge CSR lists one partial row per (item, query) of merged queries
    mq = buf[info.off_merge_q: info.off_merge_q + info.num_merge]
    mp = buf[info.off_merge_ptr: info.off_merge_ptr + info.num_merge + 1]
    mr = buf[info.off_merge_rows: info.off_merge_rows + mp[-1]]
    assert sorted(mr.tolist()) == list(range(info.num_part_rows))
    assert set(mq.tolist()) == set(range(8))
    # algorithmic bytes: distinct valid tokens x Hkv x D x 2 bytes x (K, V)
    valid = 3 * 4 + 1 + 3 * (4 + 1) + (1 + 4 + 1 + 1 + 0 + 0 + 3 + 3 + 3)
    assert info.kv_bytes == valid * 2 * 128 * 2 * 2
    assert info.kernel == 1


def test_plan_direct_output_for_single_partial_queries():
    # flat: each query one group of 3 pages -> a single item, written directly
    levels = [([0, 1, 2], [0, 3, 6], [0, 1, 2, 3, 4, 5], [4, 2])]
    rc, info, buf, *_ = plan(levels, num_pages=6, flags=TILE)
    assert rc == 0
    assert info.num_part_rows == 0 and info.num_merge == 0
    assert (decode_items(info, buf)[:, 5] == -1).all()


def test_plan_split_k_when_few_groups():
    # one group, long sequence -> chunked into several items sharing partial rows
    n_pages = 512
    levels = [([0, 4], [0, n_pages], list(range(n_pages)), [16])]
    rc, info, buf, *_ = plan(levels, hq=32, hkv=8, page=16, num_pages=n_pages, cus=256, flags=TILE)
    assert rc == 0
    items = decode_items(info, buf)
    assert len(items) > 1
    assert items[:, 4].sum() == n_pages * 16 * 1   # tokens x query tiles (4 queries x g 4 = 16 rows -> one tile)
    assert (items[:, 3] % 32 == 0).all()
    assert info.chunk_tokens % 128 == 0


@pytest.mark.parametrize("bad,exc_code", [
    (([0, 1], [0, 1], [7], [2]), 1),          # page 7 >= num_pages 4
    (([0, 1], [0, 1], [1], [5]), 1),          # last_page_len > page_size
    (([0, 2], [0, 1], [1], [2]), 1),          # qo beyond num_queries (1)
    (([0, 1], [1, 1], [1], [2]), 1),          # indptr not starting at 0
    (([0, 1], [0, 1], [-1], [2]), 1),         # negative page
])
def test_plan_rejects_bad_indices(bad, exc_code):
    rc, info, buf, _lib, L = plan([bad], nq=1, num_pages=4)
    assert rc == exc_code
    assert L.be_last_error()


def test_plan_unsupported_head_dim():
    rc, info, buf, _lib, L = plan([([0, 1], [0, 1], [0], [2])], nq=1, d=96, num_pages=4)
    assert rc == 4


def test_status_codes_map_to_reference_exceptions():
    _lib, L = lib()
    rc, *_ = plan([([0, 1], [0, 1], [9], [2])], nq=1, num_pages=4)     # invalid page -> ValueError
    with pytest.raises(ValueError, match="out of range"):
        _lib.check(rc, "plan")
    with pytest.raises(MemoryError):
        _lib.check(_lib.BE_ERR_CAPACITY, "x")
    with pytest.raises(NotImplementedError):
        _lib.check(_lib.BE_ERR_UNSUPPORTED, "x")
    with pytest.raises(RuntimeError):
        _lib.check(_lib.BE_ERR_HIP, "x")
    _lib.check(_lib.BE_OK, "x")


def test_plan_lists_keyless_queries_for_zero_fill():
    # query 1's group is empty (one page, 0 valid tokens); query 2 belongs to no group
    levels = [([0, 1, 2], [0, 1, 2], [0, 1], [3, 0])]
    rc, info, buf, *_ = plan(levels, nq=3, num_pages=2, flags=TILE)
    assert rc == 0
    assert info.num_zero == 2
    assert buf[info.off_zero_q: info.off_zero_q + 2].tolist() == [1, 2]
    assert buf[info.off_zero_ptr: info.off_zero_ptr + 3].tolist() == [0, 0, 0]
    assert info.num_items == 1 and info.num_merge == 0


def test_fixed_layout_offsets_do_not_depend_on_the_plan():
    _lib, L = lib()
    caps = _lib.BePlanCaps(64, 16, 256, 16, 128, 16, 32)
    a = [([0, 8], [0, 4], [0, 1, 2, 3], [1]), ([0, 3, 5, 8], [0, 2, 4, 6], [4, 5, 6, 7, 8, 9], [1, 1, 1])]
    b = [([0, 1, 2], [0, 3, 6], [0, 1, 2, 3, 4, 5], [4, 2])]
    rc1, i1, buf1, *_ = plan(a, nq=8, num_pages=19, caps=caps)
    rc2, i2, buf2, *_ = plan(b, nq=2, num_pages=19, caps=caps)
    assert i1.kernel == 1 and i2.kernel == 1       # tile_rows 32: the tile kernel's layout
    assert rc1 == 0 and rc2 == 0
    fields = ["plan_ints", "off_items", "off_qindex", "off_pages", "off_merge_q", "off_merge_ptr", "off_merge_rows",
              "off_zero_q", "off_zero_ptr", "grid_items", "grid_merge", "grid_zero", "part_rows_cap",
              "partial_bytes", "tile_rows"]
    assert [getattr(i1, f) for f in fields] == [getattr(i2, f) for f in fields]
    assert i1.static_layout == 1 and i1.grid_items == 64 and i1.tile_rows == 32
    assert buf1[0] == i1.num_items and buf2[0] == i2.num_items and buf2[1] == i2.num_merge
    # exceeding a capacity is a capacity error
    tiny = _lib.BePlanCaps(1, 16, 256, 16, 128, 16, 32)
    rc3, *_ = plan(a, nq=8, num_pages=19, caps=tiny)
    assert rc3 == _lib.BE_ERR_CAPACITY


# ---------------------------------------------------------------- streaming plan
def decode_stream(info, buf):
    wg = buf[info.off_wg: info.off_wg + 4 * info.num_wg].reshape(-1, 4)
    segs = buf[info.off_items: info.off_items + 8 * info.num_items].reshape(-1, 8)
    recs = buf[info.off_records: info.off_records + 8 * info.num_merge].reshape(-1, 8)
    rslots = buf[info.off_record_slots: info.off_record_slots + info.num_part_rows]
    tails = buf[info.off_tails: info.off_tails + 2 * info.num_tails].reshape(-1, 2)
    return wg, segs, recs, rslots, tails


def decode_tail_items(info, buf):
    """Tail items of tail-role workgroups: [n][8] (query, KV head, first tail entry, entries, slot, 0, 0, 0)."""
    return buf[info.off_tail_items: info.off_tail_items + 8 * info.num_tail_items].reshape(-1, 8)


def expected_keys(levels, page, nq):
    """Per query: the multiset of (page id, in-page slot) of every token of every group it is in."""
    from collections import Counter
    exp = [Counter() for _ in range(nq)]
    for qo, kvp, kvi, lpl in levels:
        for g in range(len(qo) - 1):
            npg = kvp[g + 1] - kvp[g]
            n = 0 if npg == 0 else (npg - 1) * page + lpl[g]
            keys = [(kvi[kvp[g] + t // page], t % page) for t in range(n)]
            for q in range(qo[g], qo[g + 1]):
                exp[q].update(keys)
    return exp


def expected_tokens(levels, page, nq, hkv):
    exp = np.zeros((nq, hkv), dtype=np.int64)
    for qo, kvp, kvi, lpl in levels:
        for g in range(len(qo) - 1):
            npg = kvp[g + 1] - kvp[g]
            n = 0 if npg == 0 else (npg - 1) * page + lpl[g]
            exp[qo[g]:qo[g + 1], :] += n
    return exp


def check_stream_plan(levels, nq, hq, hkv, page, info, buf):
    from collections import Counter
    assert info.kernel == 2
    wg, segs, recs, rslots, tails = decode_stream(info, buf)
    pages = buf[info.off_pages:]
    g = hq // hkv
    items = decode_tail_items(info, buf)
    TAIL_ROLE = 8
    # workgroup table: segment runs with their tile totals that together partition the
    # segment list (workgroups of sibling query tiles are placed 8 apart, so the runs need
    # not follow the workgroup order), then the tail-role workgroups' contiguous item runs
    role = wg[:, 3] == TAIL_ROLE
    assert wg[~role, 1].sum() == info.num_items and wg[role, 1].sum() == info.num_tail_items
    if role.any():
        first = int(np.argmax(role))
        assert role[first:].all()                          # tail roles are the last workgroups
    istart = 0
    covered = np.zeros(len(segs), dtype=bool)
    seg_cls = np.full(len(segs), -1)
    for b, (s0, ns, tiles, cls) in enumerate(wg):
        if cls == TAIL_ROLE:
            assert s0 == istart and tiles == 0
            istart += ns
            continue
        # wave-role mode 0 / 2, per segment (1), wide roles over up to 128 (5) or 256 rows (6;
        # 7: the same through the direct-load loop)
        assert cls in (0, 1, 2, 5, 6, 7)
        if ns:
            assert not covered[s0:s0 + ns].any()
            covered[s0:s0 + ns] = True
            assert tiles == segs[s0:s0 + ns, 7].sum()
            seg_cls[s0:s0 + ns] = cls
            rows = segs[s0:s0 + ns, 1] * g
            if cls == 5:
                assert (rows > 64).any() and (rows <= 128).all()
            elif cls in (6, 7):
                assert (rows > 64).any() and (rows <= 256).all()
            else:
                assert (rows <= 64).all()
    assert covered.all()
    # coverage: every (query, KV head) sees exactly its tokens (segments: whole tiles from a
    # 64-aligned start; tail chunks: up to 16 tokens of one page), page by page
    seen = [[Counter() for _ in range(hkv)] for _ in range(nq)]
    for q0, qn, pb, t0, tc, head, slot, nt in segs:
        assert tc > 0 and qn > 0 and qn * g <= 256 and t0 % 64 == 0 and nt == -(-tc // 64)
        keys = [(int(pages[pb + t // page]), t % page) for t in range(t0, t0 + tc)]
        for q in range(q0, q0 + qn):
            seen[q][head].update(keys)
    tails_of = {}
    chunks = [(q, h, tb, tn) for q, h, ptr, n, tb, tn, z0, z1 in recs if tn > 0]
    chunks += [(q, h, tb, tn) for q, h, tb, tn, slot, *_ in items]
    assert not (info.num_tail_items and (recs[:, 5] > 0).any())   # chunks go to items or to records
    assert (recs[:, 6:] == 0).all() and (items[:, 5:] == 0).all()
    assert (items[:, 3] <= 4).all()                                 # an item holds at most 4 chunks
    per_qh = {}
    for q, h, tb, tn in chunks:
        assert tn > 0
        per_qh.setdefault((int(q), int(h)), []).extend(tuple(int(v) for v in e) for e in tails[tb:tb + tn])
    for (q, h), chunk in per_qh.items():
        assert tails_of.setdefault(q, sorted(chunk)) == sorted(chunk)   # every head of a query has its chunks
        for pg, ov in chunk:
            off, valid = ov & 0xFFFF, ov >> 16
            assert 1 <= valid <= 16 and off + valid <= page
            seen[q][h].update((pg, off + t) for t in range(valid))
    exp = expected_keys(levels, page, nq)
    for q in range(nq):
        for h in range(hkv):
            assert seen[q][h] == exp[q], (q, h)
    # slots: each non-direct segment owns qn consecutive slots; every slot is in exactly one record
    owned = []
    cover = {}
    for q0, qn, pb, t0, tc, head, slot, nt in segs:
        for j in range(qn):
            cover.setdefault((q0 + j, head), []).append(-1 if slot < 0 else slot + j)
        if slot >= 0:
            owned.extend(range(slot, slot + qn))
    for q, h, tb, tn, slot, *_ in items:
        cover.setdefault((q, h), []).append(slot)
        owned.append(slot)
    assert sorted(owned) == list(range(info.num_part_rows))
    assert sorted(rslots.tolist()) == list(range(info.num_part_rows))
    rec_keys = set()
    for q, h, ptr, n, tb, tn, *_ in recs:
        rec_keys.add((q, h))
        assert sorted(rslots[ptr:ptr + n].tolist()) == sorted(x for x in cover.get((q, h), []) if x >= 0)
    for q in range(nq):
        for h in range(hkv):
            c = cover.get((q, h), [])
            direct = len(c) == 1 and c[0] == -1 and not tails_of.get(q)
            assert ((q, h) in rec_keys) != direct
    # the loop: register-staged when the longest run reaches 8 tiles (never for fixed layouts
    # nor with wide-role workgroups, which run in the direct-load loop)
    assert info.stream_loop == (1 if int(wg[wg[:, 3] != TAIL_ROLE, 2].max(initial=0)) >= 8
                                and not info.static_layout and not ((wg[:, 3] == 5) | (wg[:, 3] == 6)).any()
                                else 0)
    return wg, segs, recs, rslots


def test_stream_plan_cascade_coverage_and_records():
    levels = [([0, 8], [0, 4], [0, 1, 2, 3], [1]),
              ([0, 3, 5, 8], [0, 2, 4, 6], [4, 5, 6, 7, 8, 9], [1, 1, 1]),
              ([0, 1, 2, 3, 4, 5, 6, 7, 8], [0, 1, 3, 4, 5, 6, 7, 8, 9],
               [10, 11, 12, 13, 14, 15, 16, 17, 18], [1, 1, 1, 0, 0, 3, 3, 3])]
    # (the streaming kernel takes page sizes that are multiples of 16)
    # tail chunks in the merge kernel (no tail role), no tail pass, the tail role
    for flags in (_NO_TAIL_ROLE, 8, 16, 0):
        rc, info, buf, _lib, L = plan(levels, hq=8, hkv=2, page=16, num_pages=19, flags=flags)
        assert rc == 0, L.be_last_error()
        check_stream_plan(levels, 8, 8, 2, 16, info, buf)
        valid = 3 * 16 + 1 + 3 * (16 + 1) + (1 + 16 + 1 + 1 + 0 + 0 + 3 + 3 + 3)
        assert info.kv_bytes == valid * 2 * 128 * 2 * 2
        assert (info.num_tails > 0) == (flags != 8)
        # by default the tail role too: here the tail chunks outweigh the streamed tiles
        assert (info.num_tail_items > 0) == (flags in (16, 0))
        assert buf[4] == info.num_tail_items                     # header: tail item count
    rc, info, *_ = plan(levels, hq=8, hkv=2, page=4, num_pages=19)
    assert rc == 0 and info.kernel == 1                 # page 4: the tile kernel


@pytest.mark.parametrize("cus", [2, 7, 256])
def test_stream_plan_balances_tiles_across_workgroups(cus):
    # north-star-like shape: 2 requests x 16 beams, prefix 1024 tokens, suffix 128 per beam
    hq, hkv, page = 32, 8, 16
    pre, suf = 64, 8
    qo0, kvp0, kvi0 = [0, 16, 32], [0, pre, 2 * pre], list(range(2 * pre))
    qo1 = list(range(33))
    kvp1 = [2 * pre + 0] + [0] * 32
    kvp1 = list(range(0, 33 * suf, suf))
    kvi1 = list(range(2 * pre, 2 * pre + 32 * suf))
    levels = [(qo0, kvp0, kvi0, [16, 16]), (qo1, kvp1, kvi1, [16] * 32)]
    # (tail pass off: the 128-token suffixes would otherwise leave the persistent kernel)
    rc, info, buf, _lib, L = plan(levels, nq=32, hq=hq, hkv=hkv, page=page, num_pages=2 * pre + 32 * suf, cus=cus,
                                  flags=8)
    assert rc == 0, L.be_last_error()
    wg, segs, recs, rslots = check_stream_plan(levels, 32, hq, hkv, page, info, buf)
    assert info.num_wg == cus
    tiles = wg[:, 2]
    total = (2 * 16 + 32 * 2) * hkv            # prefix 2 x 16 tiles, suffix 32 x 2 tiles, per KV head
    assert tiles.sum() == total
    if cus > 1:
        # balanced in the planner's cost (one unit per tile and per segment start) up to
        # the granularity of the cuts: within two tiles and two segment starts
        cost = tiles + wg[:, 1]
        assert cost.max() - cost.min() <= 4
    assert info.num_merge == 32 * hkv           # every (query, head) merges prefix and suffix


@pytest.mark.parametrize("beams,cus", [(32, 256), (32, 5), (18, 4), (64, 13), (64, 5), (10, 5), (80, 5)])
def test_stream_plan_wide_roles(beams, cus):
    """Long groups of more than 64 rows go to wide-role workgroups when the
    launch gives every workgroup a long run (at least 64 tiles of 64 rows
    each): 256-row segments (class 6) when every such group has at least 256
    rows, else 128-row segments (class 5); BE_PLAN_NO_WIDE256 keeps the
    128-row ones, BE_PLAN_NO_WIDE 64-row segments; every (query, KV head)
    still sees exactly its tokens."""
    hq, hkv, page = 32, 8, 16
    pre, suf = 96, 3                            # 1536-token prefix, 48-token suffixes
    qo0, kvp0, kvi0 = [0, beams], [0, pre], list(range(pre))
    qo1 = list(range(beams + 1))
    kvp1 = list(range(0, (beams + 1) * suf, suf))
    kvi1 = list(range(pre, pre + beams * suf))
    levels = [(qo0, kvp0, kvi0, [16]), (qo1, kvp1, kvi1, [16] * beams)]
    g = hq // hkv
    tiles64 = (pre * page // 64) * -(-beams * g // 64) * hkv
    expect = beams * g > 64 and tiles64 >= 64 * cus
    for flags in (0, 64, 1024):
        rc, info, buf, _lib, L = plan(levels, nq=beams, hq=hq, hkv=hkv, page=page, num_pages=pre + beams * suf,
                                      cus=cus, flags=flags)
        assert rc == 0, L.be_last_error()
        wg, segs, recs, rslots = check_stream_plan(levels, beams, hq, hkv, page, info, buf)
        rows = segs[:, 1] * g
        if flags == 64 or not expect:
            assert (rows <= 64).all() and not ((wg[:, 3] == 5) | (wg[:, 3] == 6)).any()
        elif beams * g >= 256 and flags == 0:
            assert rows.max() > 128 and rows.max() <= 256 and (wg[:, 3] == 6).any() and not (wg[:, 3] == 5).any()
            assert info.stream_loop == 0
        else:
            assert rows.max() > 64 and rows.max() <= 128 and (wg[:, 3] == 5).any() and not (wg[:, 3] == 6).any()
            assert info.stream_loop == 0


@pytest.mark.parametrize("beams,cus", [(64, 256), (64, 64), (96, 256), (64, 20)])
def test_stream_plan_pairs_sibling_query_tiles(beams, cus):
    """A wide group split into several 256-row query tiles reads the same K/V
    tiles once per query tile: the planner balances each (group, KV head) set
    of sibling tiles as one unit and puts sibling s of virtual run v in
    workgroup (v // 8) 8 k + 8 s + v % 8, so that the k workgroups of a piece
    share an XCD and the same tile range.  Config-5-like shape: 2 requests,
    GQA 8, a long prefix, 1..4-token suffixes (tail pass)."""
    hq, hkv, page = 64, 8, 16
    pre = 512                                   # 8192-token prefix per request
    qo0, kvp0, kvi0, lpl0 = [0, beams, 2 * beams], [0, pre, 2 * pre], list(range(2 * pre)), [16, 16]
    rng = np.random.default_rng(beams + cus)
    suf = rng.integers(1, 5, size=2 * beams)
    qo1 = list(range(2 * beams + 1))
    kvp1 = list(range(2 * beams + 1))
    kvi1 = list(range(2 * pre, 2 * pre + 2 * beams))
    levels = [(qo0, kvp0, kvi0, lpl0), (qo1, kvp1, kvi1, [int(x) for x in suf])]
    rc, info, buf, _lib, L = plan(levels, nq=2 * beams, hq=hq, hkv=hkv, page=page,
                                  num_pages=2 * pre + 2 * beams, cus=cus)
    assert rc == 0, L.be_last_error()
    wg, segs, recs, rslots = check_stream_plan(levels, 2 * beams, hq, hkv, page, info, buf)
    g = hq // hkv
    k = -(-beams * g // 256)                    # 256-row query tiles per (request, KV head)
    wide = np.flatnonzero(wg[:, 3] == 6)
    if 8 * (cus // (8 * k)) == 0:               # fewer than 8 k workgroups: no pairing
        return
    assert len(wide) > 0 and len(wide) % k == 0
    for b in wide:
        sib = int(b) % (8 * k) // 8             # sibling index of workgroup b
        group = [int(b) + 8 * (s - sib) for s in range(k)]
        assert all(wg[x, 3] == 6 for x in group), (b, group)
        runs = [segs[wg[x, 0]: wg[x, 0] + wg[x, 1]] for x in group]
        for r in runs[1:]:
            # same KV head, pages and tile ranges; different query tiles
            assert len(r) == len(runs[0])
            assert (r[:, [2, 3, 4, 5, 7]] == runs[0][:, [2, 3, 4, 5, 7]]).all()
            assert (r[:, 0] != runs[0][:, 0]).all()


@pytest.mark.parametrize("cus", [256, 24, 40])
def test_stream_plan_pairs_narrow_sibling_tiles(cus):
    """The same placement for a group cut into 64-row query tiles (config 3's
    root: 32 beams x GQA 4 = 128 rows, two tiles) beside single-tile groups:
    each root segment of query tile 1 lies in the workgroup 8 after its tile-0
    twin (same KV head, tokens and tiles), and the single-tile groups fill the
    other workgroups (on at least 17 workgroups: fewer give every workgroup
    64 root tiles, and the root takes the 128-row wide roles instead)."""
    hq, hkv, page, beams = 32, 8, 16, 32
    root = 256                                  # 4096-token root
    qo0, kvp0, kvi0 = [0, beams], [0, root], list(range(root))
    # level 1: two branches of 16 beams, 8 pages each; level 2: 2-token leaves
    qo1, kvp1 = [0, 16, 32], [0, 8, 16]
    kvi1 = list(range(root, root + 16))
    qo2 = list(range(beams + 1))
    kvp2 = list(range(beams + 1))
    kvi2 = list(range(root + 16, root + 16 + beams))
    levels = [(qo0, kvp0, kvi0, [16]), (qo1, kvp1, kvi1, [16, 16]), (qo2, kvp2, kvi2, [2] * beams)]
    rc, info, buf, _lib, L = plan(levels, nq=beams, hq=hq, hkv=hkv, page=page, num_pages=root + 16 + beams,
                                  cus=cus, flags=8)
    assert rc == 0, L.be_last_error()
    wg, segs, recs, rslots = check_stream_plan(levels, beams, hq, hkv, page, info, buf)
    seg_wg = np.empty(len(segs), dtype=np.int64)
    for b, (s0, ns, tiles, cls) in enumerate(wg):
        seg_wg[s0:s0 + ns] = b
    rootseg = segs[:, 2] == 0                   # segments of the root group (page list from 0)
    a = {(int(x[5]), int(x[3]), int(x[7])): int(seg_wg[i]) for i, x in enumerate(segs) if rootseg[i] and x[0] == 0}
    b16 = {(int(x[5]), int(x[3]), int(x[7])): int(seg_wg[i]) for i, x in enumerate(segs) if rootseg[i] and x[0] == 16}
    assert len(a) > 0 and a.keys() == b16.keys()
    for key, b0 in a.items():
        assert b16[key] == b0 + 8 and b0 % 16 < 8, (key, b0, b16[key])


def test_stream_plan_zero_records_for_keyless_queries():
    levels = [([0, 1, 2], [0, 1, 2], [0, 1], [3, 0])]
    rc, info, buf, *_ = plan(levels, nq=3, page=16, num_pages=2)
    assert rc == 0
    wg, segs, recs, rslots = check_stream_plan(levels, 3, 8, 2, 16, info, buf)
    zero = sorted((int(q), int(h)) for q, h, p, n, tb, tn, *_ in recs if n == 0 and tn == 0)
    assert zero == [(1, 0), (1, 1), (2, 0), (2, 1)]


def test_stream_plan_fixed_layout_offsets():
    _lib, L = lib()
    caps = _lib.BePlanCaps(4096, 16, 256, 64, 4096, 0, 64, 64)
    a = [([0, 8], [0, 4], [0, 1, 2, 3], [1]), ([0, 3, 5, 8], [0, 2, 4, 6], [4, 5, 6, 7, 8, 9], [1, 1, 1])]
    b = [([0, 1, 2], [0, 3, 6], [0, 1, 2, 3, 4, 5], [4, 2])]
    rc1, i1, buf1, *_ = plan(a, nq=8, page=16, num_pages=19, caps=caps)
    rc2, i2, buf2, *_ = plan(b, nq=2, page=16, num_pages=19, caps=caps)
    assert rc1 == 0 and rc2 == 0 and i1.kernel == 2 and i2.kernel == 2
    fields = ["plan_ints", "off_items", "off_pages", "off_wg", "off_records", "off_record_slots", "off_tails",
              "num_wg", "grid_merge", "part_rows_cap", "partial_bytes"]
    assert [getattr(i1, f) for f in fields] == [getattr(i2, f) for f in fields]
    assert buf1[0] == i1.num_items and buf1[1] == i1.num_merge and buf2[1] == i2.num_merge
    tiny = _lib.BePlanCaps(1, 16, 256, 64, 4096, 0, 64, 64)
    rc3, *_ = plan(a, nq=8, page=16, num_pages=19, caps=tiny)
    assert rc3 == _lib.BE_ERR_CAPACITY


def test_stream_plan_falls_back_to_tile_kernel_when_a_workgroup_overflows():
    # one workgroup, 300 groups x 2 heads = 600 segments > the per-workgroup table
    n = 300
    levels = [(list(range(n + 1)), list(range(n + 1)), list(range(n)), [4] * n)]
    rc, info, buf, *_ = plan(levels, nq=n, page=16, num_pages=n, cus=1, flags=8)
    assert rc == 0 and info.kernel == 1


def e2e_like_levels(nreq=2, beams=4, pre_pages=16, page=16, seed=0):
    """Request prefixes shared by their beams, then single-query levels of a few tokens (the
    shape of a beam trie that re-converges every step)."""
    rng = np.random.default_rng(seed)
    nq = nreq * beams
    nxt = 0
    kvi0 = list(range(nxt, nxt + nreq * pre_pages)); nxt += nreq * pre_pages
    l0 = (list(range(0, nq + 1, beams)), list(range(0, nreq * pre_pages + 1, pre_pages)), kvi0, [page] * nreq)
    levels = [l0]
    for _ in range(2):
        lens = rng.integers(1, 49, size=nq)                  # 1..48 tokens
        kvp, kvi, lpl = [0], [], []
        for n in lens:
            npg = -(-int(n) // page)
            kvi += list(range(nxt, nxt + npg)); nxt += npg
            kvp.append(kvp[-1] + npg)
            lpl.append(int(n) - (npg - 1) * page)
        levels.append((list(range(nq + 1)), kvp, kvi, lpl))
    return levels, nq, nxt


@pytest.mark.parametrize("page", [16, 32])
def test_stream_plan_routes_short_groups_to_tail_chunks(page):
    levels, nq, npages = e2e_like_levels(page=page)
    rc, info, buf, _lib, L = plan(levels, nq=nq, hq=32, hkv=8, page=page, num_pages=npages)
    assert rc == 0, L.be_last_error()
    check_stream_plan(levels, nq, 32, 8, page, info, buf)
    lens = [(np.diff(kvp) - 1) * page + np.asarray(lpl) for _, kvp, _, lpl in levels[1:]]
    assert info.num_tails == sum(int(-(-n // 16)) for l in lens for n in l)
    # the prefix level stays in the streaming kernel; every (query, head) merges
    assert info.num_items > 0 and info.num_merge == nq * 8
    rc, info2, buf2, *_ = plan(levels, nq=nq, hq=32, hkv=8, page=page, num_pages=npages, flags=_lib.BE_PLAN_NO_TAIL)
    assert rc == 0 and info2.num_tails == 0
    check_stream_plan(levels, nq, 32, 8, page, info2, buf2)


def test_stream_plan_tail_limits():
    page = 16
    # a 5-query group (more than the tail pass takes) and 70 single-token levels for query 0
    # (more chunks than one query holds)
    levels = [([0, 5], [0, 1], [0], [3])]
    nxt = 1
    for _ in range(70):
        levels.append(([0, 1], [0, 1], [nxt], [1]))
        nxt += 1
    rc, info, buf, _lib, L = plan(levels, nq=5, hq=8, hkv=2, page=page, num_pages=nxt)
    assert rc == 0, L.be_last_error()
    check_stream_plan(levels, 5, 8, 2, page, info, buf)
    wg, segs, recs, rslots, tails = decode_stream(info, buf)
    assert info.num_tails == 64
    assert any(q0 == 0 and qn == 5 for q0, qn, *_ in segs)    # the 5-query group is a segment
    # page sizes that are not a multiple of 16 never use tail chunks
    rc, info, buf, *_ = plan(levels, nq=5, hq=8, hkv=2, page=8, num_pages=nxt)
    assert rc == 0 and info.num_tails == 0


@pytest.mark.parametrize("nq,nk,cus", [(200, 200, 256), (200, 700, 7), (9, 5, 3), (40, 40, 1)])
def test_stream_plan_causal_groups(nq, nk, cus):
    """BE_PLAN_CAUSAL on the streaming kernel: each 16-query tile (64 rows at
    GQA 4) of a causal group is streamed over [0, its last query's visible
    tokens) only, every segment carries its tile's first-query count (unclamped:
    query j of the tile sees that + j), causal groups never become tail
    chunks, and tiles whose queries see nothing get no segment."""
    hq, hkv, page = 32, 8, 16
    npg = -(-nk // page)
    levels = [([0, nq], [0, npg], list(range(npg)), [nk - (npg - 1) * page])]
    rc, info, buf, _lib, L = plan(levels, nq=nq, hq=hq, hkv=hkv, page=page, num_pages=npg, cus=cus, flags=128)
    assert rc == 0, L.be_last_error()
    assert info.kernel == 2 and info.off_seg_causal > 0 and info.num_tails == 0
    wg, segs, recs, rslots, tails = decode_stream(info, buf)
    vis = buf[info.off_seg_causal: info.off_seg_causal + info.num_items]
    g, qt = hq // hkv, 64 // (hq // hkv)
    covered = {}
    for (q0, qn, pb, t0, tc, head, slot, nt), v in zip(segs, vis):
        assert v == nk - nq + q0 + 1                     # first query's count, unclamped
        assert qn == min(qt, nq - q0) and t0 % 64 == 0
        covered.setdefault((int(q0), int(head)), []).append((int(t0), int(tc)))
    for qa in range(0, nq, qt):
        qn = min(qt, nq - qa)
        last = max(0, min(nk, nk - nq + qa + qn))        # the tile's last query sees this many
        for h in range(hkv):
            got = sorted(covered.get((qa, h), []))
            if last == 0:
                assert not got
                continue
            assert got[0][0] == 0 and sum(tc for _, tc in got) == last
            assert all(a + b == c for (a, b), (c, _) in zip(got, got[1:]))


def test_causal_flag_without_multi_query_groups_changes_nothing():
    levels = [([0, 1, 2], [0, 4, 8], list(range(8)), [16, 16])]
    a = plan(levels, hq=32, hkv=8, page=16, num_pages=8)
    b = plan(levels, hq=32, hkv=8, page=16, num_pages=8, flags=128)
    assert a[0] == b[0] == 0 and b[1].off_seg_causal == 0
    assert np.array_equal(a[2][: a[1].plan_ints], b[2][: b[1].plan_ints])


# ---------------------------------------------------------------- row-block plans
ROWS = 256     # BE_PLAN_ROWS


def rows_coverage(levels, info, buf, nq, hq, hkv, page):
    """Decode a row-block plan: for every (query, query head), the multiset of
    (page, slot) keys its task's passes cover for it; and the workgroup order's
    placement of tasks sharing a level-0 group on one XCD lane (id mod 8)."""
    g = hq // hkv
    tasks = buf[info.off_items: info.off_items + 8 * info.num_items].reshape(-1, 8)
    pages = buf[info.off_pages:]
    got = {}
    for wg, (q0, n, p0, np_, head, nsub, _, _) in enumerate(tasks):
        assert 1 <= n and n * g <= 16 and 0 <= head < hkv
        subs = 0
        for pi in range(p0, p0 + np_):
            base, tokens, mask, sub = buf[info.off_merge_rows + 4 * pi: info.off_merge_rows + 4 * pi + 4]
            assert tokens > 0 and sub == (tokens + 15) // 16
            subs += sub
            keys = [(int(pages[base + t // page]), t % page) for t in range(tokens)]
            for r in range(n * g):
                if (int(mask) >> r) & 1:
                    qi, qh = q0 + r // g, head * g + r % g
                    got.setdefault((qi, qh), []).extend(keys)
        assert subs == nsub
    return got


@pytest.mark.parametrize("seed", range(4))
@pytest.mark.parametrize("hq,hkv", [(32, 8), (64, 8), (8, 8), (16, 2)])
def test_rows_plan_covers_each_query_groups_once(seed, hq, hkv):
    """BE_PLAN_ROWS plans of random multi-request beam tries (page 16): every
    (query, head) gets exactly the (page, slot) keys of its groups on every
    level (once per level it appears in)."""
    import random
    from beam_engine_amd.beam_state import BeamGenerateResult, BeamState, BeamToken
    from tests.test_beam_state_product import RecordingPages
    rng = random.Random(seed)
    page = 16
    pages = RecordingPages(4000, page)
    st = BeamState(4, pages)
    for r in range(rng.randint(1, 3)):
        st.add_root_sequence(list(range(rng.randint(1, 90))), request_id=r)
    for step in range(rng.randint(5, 60)):
        res = []
        for rid in sorted({c.request_id for c in st.candidates}):
            idx = [i for i, c in enumerate(st.candidates) if c.request_id == rid]
            pool = sorted(((i, rng.randrange(50), st.candidates[i].score - rng.random()) for i in idx for _ in range(3)),
                          key=lambda t: -t[2])
            chosen, seen = [], set()
            for i, t, s_ in pool:
                if (i, t) not in seen and len(chosen) < 4:
                    seen.add((i, t))
                    chosen.append((i, t, s_))
            res += [BeamGenerateResult(st.candidates[i], [BeamToken(t, s_) for ii, t, s_ in chosen if ii == i])
                    for i in idx]
        st.add_filtered_results(res)
    levels = st._cascade_lists()
    nq = len(st.candidates)
    rc, info, buf, _lib, L = plan(levels, nq=nq, hq=hq, hkv=hkv, page=page, num_pages=4000, flags=ROWS)
    if hq // hkv > 16:
        assert info.kernel != 3
        return
    assert rc == 0 and info.kernel == 3
    got = rows_coverage(levels, info, buf, nq, hq, hkv, page)
    for qi in range(nq):
        want = []
        for qo, kvp, kvi, lpl in levels:
            for j in range(len(qo) - 1):
                if qo[j] <= qi < qo[j + 1]:
                    npg = kvp[j + 1] - kvp[j]
                    t = 0 if npg == 0 else (npg - 1) * page + lpl[j]
                    want += [(kvi[kvp[j] + k // page], k % page) for k in range(t)]
        for qh in range(hq):
            assert sorted(got.get((qi, qh), [])) == sorted(want), (qi, qh)


def test_rows_plan_places_shared_blocks_on_one_xcd_lane():
    """8 requests x 16 beams over a shared prefix, g = 4: four blocks of four
    queries per (request, KV head); the four tasks of each get workgroup ids
    equal modulo 8 (one XCD)."""
    qo0 = list(range(0, 129, 16))
    kvp0 = [0] + [64 * (r + 1) for r in range(8)]
    kvi0 = list(range(512))
    lv0 = (qo0, kvp0, kvi0, [16] * 8)
    lv1 = (list(range(129)), list(range(129)), list(range(512, 640)), [7] * 128)
    rc, info, buf, _lib, L = plan([lv0, lv1], nq=128, hq=32, hkv=8, page=16, num_pages=640, flags=ROWS)
    assert rc == 0 and info.kernel == 3 and info.num_items == 256
    tasks = buf[info.off_items: info.off_items + 8 * 256].reshape(-1, 8)
    lanes = {}
    for wg, t in enumerate(tasks):
        key = (int(t[0]) // 16, int(t[4]))          # (request, KV head)
        lanes.setdefault(key, set()).add(wg % 8)
        assert int(t[1]) == 4 and int(t[3]) == 5     # four queries: the prefix pass and four suffix passes
    assert len(lanes) == 64 and all(len(v) == 1 for v in lanes.values())


def test_generator_rejects_out_of_vocabulary_token_ids():
    """Token ids outside the vocabulary raise ValueError on the host before
    anything reaches the device embedding: prompts before the trie or the
    pool change, and every step's staged ids (``_check_tokens``)."""
    import types

    import numpy as np
    import torch
    from beam_engine_amd import PageTable
    from beam_engine_amd.beam_state import NativeBeamState
    from beam_engine_amd.generator import BatchedBeamSearch
    from beam_engine_amd.llama import LlamaConfig

    cfg = LlamaConfig(num_hidden_layers=1, hidden_size=64, num_attention_heads=2, num_key_value_heads=1,
                      head_dim=32, intermediate_size=64, vocab_size=100, max_position_embeddings=64)
    pt = PageTable(1, page_size=4, max_num_pages=16, head_num=1, head_dim=32, device="cpu",
                   store_dtype=torch.float32)
    gen = types.SimpleNamespace(model=types.SimpleNamespace(cfg=cfg), state=NativeBeamState(2, pt))
    gen._check_tokens = lambda ids: BatchedBeamSearch._check_tokens(gen, ids)
    for bad in ([[1, 2, 100]], [[-1, 2, 3]], [[1, 2, 3], [4, 5, 1000]]):
        with pytest.raises(ValueError, match="outside the vocabulary"):
            BatchedBeamSearch.prefill(gen, bad)
    assert gen.state.num_candidates() == 0 and pt.num_free_pages() == 16
    gen._check_tokens(np.array([0, 99]))
    with pytest.raises(ValueError, match="token id 100"):
        gen._check_tokens(np.array([5, 100, 7]))


@pytest.mark.parametrize("name, tail_role", [("e2e_step", True), ("config2", False), ("config3", True),
                                             ("north_star", False), ("config5", True)])
def test_stream_plan_tail_role_default_on_benchmark_shapes(name, tail_role):
    """The planner's default for who attends the tail chunks, at the benchmark
    shapes: tail-role workgroups of the streaming launch when the chunks
    average at most 2 per query (e2e step 1.5, config 5 1.2) or are at least
    two thirds of the streamed tiles' work (config 3: 14 chunks per query, 0.82
    of it); the tail-and-merge kernel otherwise (config 2 and the north-star:
    8 per query, half of it)."""
    from beam_engine_amd import workloads
    wl = getattr(workloads, name)()
    levels = [tuple(wl.levels[j][i] for j in range(4)) for i in range(len(wl.levels[0]))]
    rc, info, buf, _lib, L = plan(levels, nq=wl.num_queries, hq=wl.hq, hkv=wl.hkv, page=wl.page,
                                  num_pages=wl.num_pages, cus=256)
    assert rc == 0, L.be_last_error()
    wg, segs, recs, rslots, tails = decode_stream(info, buf)
    assert (info.num_tail_items > 0) == tail_role
    assert ((wg[:, 3] == 8).any()) == tail_role              # class 8: tail-role workgroups
    if tail_role:
        assert (recs[:, 5] == 0).all()                 # the merge kernel only merges
