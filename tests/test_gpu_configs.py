"""GPU parity at the benchmark configurations' full sizes (bf16, page 16):

* the north-star shape (8 requests x beam 16, 32/8 heads, 4096-token prefix,
  128-token suffixes) and config 5 (2 x 64 beams, 64/8 heads, 32768-token
  prefix, suffixes U[1, 512] from seed 5), cascade and flat, against the
  float64 oracle on a seeded subset of queries and KV heads (the oracle
  gathers each chosen query's path tokens from the device pool);
* a config-5-shaped beam trie (two 32768-token prompts, 64 beams each, grown by
  random selections) decoded with every strategy the picker can choose --
  ``auto``, tree (MI355X and FastTree edge models), fully split, flat;
* config 4 end to end: the Llama-3-8B-shaped decoder, 8 requests x beam 16,
  1024-token prompts, decoding with HIP graphs while the trie is replayed on
  the oracle with the engine's own selections at every step; selections are
  checked bit for bit against the oracle on some steps, and one layer's
  attention at the live state against the oracle on the real pages.

Tolerance (bf16 storage against the float64 oracle): 2e-2 relative, 1e-2
absolute on outputs; 2e-3 on lse."""

import math
import random
import sys

import numpy as np
import pytest
import torch

from oracle import attention as oa

pytestmark = pytest.mark.gpu

TOL = dict(rtol=2e-2, atol=1e-2)


def say(msg):
    print(f"[case] {msg}", flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def ws():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    return torch.empty(256 << 20, dtype=torch.uint8, device="cuda")


def oracle_path(kv_dev, pages, last_len, page, q_row, kv_heads, g, scale):
    """Float64 oracle attention of one query over one path (pages, last page
    length) for the chosen KV heads and their query heads.  Returns
    (o [len(kv_heads) * g, D], lse [len(kv_heads) * g])."""
    pages = torch.as_tensor(pages, dtype=torch.long, device=kv_dev.device)
    t = (len(pages) - 1) * page + int(last_len)
    kh = torch.as_tensor(kv_heads, dtype=torch.long, device=kv_dev.device)
    k = kv_dev[pages, 0].reshape(-1, kv_dev.shape[3], kv_dev.shape[4])[:t][:, kh].float().cpu().numpy()
    v = kv_dev[pages, 1].reshape(-1, kv_dev.shape[3], kv_dev.shape[4])[:t][:, kh].float().cpu().numpy()
    qh = np.concatenate([q_row[h * g:(h + 1) * g] for h in kv_heads])[None]
    o, lse = oa.partial_attention(qh, k, v, scale)
    return o[0], lse[0]


def check_subset(out, lse, kv_dev, flat, q, queries, kv_heads, page, scale):
    """Compare rows ``queries`` x heads of ``kv_heads`` of a GPU result with the
    oracle over each query's flat path (``flat`` = kv_indptr, kv_indices,
    last_page_len)."""
    kvp, kvi, lpl = flat
    hq, hkv = q.shape[1], kv_dev.shape[3]
    g = hq // hkv
    heads = [h * g + j for h in kv_heads for j in range(g)]
    o_all = out.float().cpu().numpy()
    l_all = lse.cpu().numpy() if lse is not None else None
    qn = q.float().cpu().numpy()
    for i in queries:
        ref_o, ref_l = oracle_path(kv_dev, kvi[kvp[i]:kvp[i + 1]], lpl[i], page, qn[i], kv_heads, g, scale)
        np.testing.assert_allclose(o_all[i, heads], ref_o, **TOL, err_msg=f"query {i}")
        if l_all is not None:
            np.testing.assert_allclose(l_all[i, heads], ref_l, rtol=2e-3, atol=2e-3, err_msg=f"query {i} lse")


def workload_case(ws, name, queries, kv_heads):
    from beam_engine_amd import BatchDecodeWithPagedKVCacheWrapper, MultiLevelCascadeAttentionWrapper
    from beam_engine_amd.workloads import BUILDERS
    wl = BUILDERS[name]()
    scale = 1.0 / math.sqrt(wl.d)
    gen = torch.Generator(device="cuda").manual_seed(17)
    kv = (torch.randn((wl.num_pages, 2, wl.page, wl.hkv, wl.d), generator=gen, device="cuda") * scale
          ).to(torch.bfloat16)
    q = (torch.randn((wl.num_queries, wl.hq, wl.d), generator=gen, device="cuda") * scale).to(torch.bfloat16)
    w = MultiLevelCascadeAttentionWrapper(2, ws)
    w.plan(*wl.levels, wl.hq, wl.hkv, wl.d, wl.page, q_data_type=torch.bfloat16)
    o, lse = w.run(q, kv, return_lse=True)
    f = BatchDecodeWithPagedKVCacheWrapper(ws)
    f.plan(*wl.flat, wl.hq, wl.hkv, wl.d, wl.page, q_data_type=torch.bfloat16)
    fo, fl = f.run(q, kv, return_lse=True)
    torch.cuda.synchronize()
    say(f"{name}: cascade kernel {w.stats.kernel}, {w.stats.kv_bytes} algorithmic KV bytes")
    check_subset(o, lse, kv, wl.flat, q, queries, kv_heads, wl.page, wl.d ** -0.5)
    check_subset(fo, fl, kv, wl.flat, q, queries, kv_heads, wl.page, wl.d ** -0.5)
    return w, wl


def test_north_star_shape(ws):
    say("north-star shape: 8 x 16 beams, prefix 4096, suffix 128, 32/8 heads")
    w, wl = workload_case(ws, "ns", [0, 17, 63, 64, 127], [0, 5])
    # distinct (page, head) valid tokens: 8 x 4096 prefix + 128 x 128 suffix, 4 KiB per token
    assert w.stats.kv_bytes == (8 * 4096 + 128 * 128) * 4096


def test_config5_full_shape(ws):
    say("config 5: 2 x 64 beams, prefix 32768, suffix U[1,512] seed 5, 64/8 heads")
    rng = np.random.default_rng(5)
    suf = rng.integers(1, 513, size=128)
    # the longest and the shortest suffixes of each request, and two others
    picks = sorted({int(np.argmax(suf[:64])), int(np.argmin(suf[:64])), 64 + int(np.argmax(suf[64:])),
                    64 + int(np.argmin(suf[64:])), 5, 100})
    w, wl = workload_case(ws, "c5", picks, [0, 7])
    assert w.stats.kv_bytes == (2 * 32768 + int(suf.sum())) * 4096


def grow_trie(pt, prompts, beam, steps, seed):
    """A multi-request beam trie grown by random selections: each step, per
    request, a few random beams die and as many others fork in two, the rest
    continue with one token -- branch points at every depth, so the beams'
    private suffixes take many lengths."""
    from beam_engine_amd.beam_state import BeamGenerateResult, BeamState, BeamToken
    rng = random.Random(seed)
    st = BeamState(beam, pt, fast_metadata=True)
    for r, p in enumerate(prompts):
        st.add_root_sequence(p, request_id=r)
    st.add_filtered_results([BeamGenerateResult(c, [BeamToken(1000 + j, -0.1 * j) for j in range(beam)])
                             for c in st.candidates])
    for _ in range(steps):
        res = []
        for rid in sorted({c.request_id for c in st.candidates}):
            idx = [i for i, c in enumerate(st.candidates) if c.request_id == rid]
            kids = {i: 1 for i in idx}
            swap = rng.choice([0, 0, 1, 1, 2, 3])
            for i in rng.sample(idx, 2 * swap):
                kids[i] = 0 if kids[i] == 1 and sum(v == 0 for v in kids.values()) < swap else 2
            for i in idx:
                c = st.candidates[i]
                res.append(BeamGenerateResult(c, [BeamToken(rng.randrange(50000), c.score - rng.random())
                                                  for _ in range(kids[i])]))
        st.add_filtered_results(res)
    return st


def test_config5_trie_every_strategy(ws):
    """A config-5-shaped trie (2 requests x 64 beams over 32768-token
    prompts, 300 random decode steps: forks, dead branches and private
    suffixes of many lengths) attended by every decomposition the picker
    chooses among; each equals the oracle's path attention."""
    from beam_engine_amd import BatchDecodeWithPagedKVCacheWrapper, MultiLevelCascadeAttentionWrapper, PageTable
    from beam_engine_amd.picker import StrategyPicker
    say("config 5 trie: growing 2 x 64 beams over 32768-token prompts")
    hq, hkv, d, page = 64, 8, 128, 16
    pt = PageTable(1, page_size=page, max_num_pages=16384, head_num=hkv, head_dim=d, device="cuda",
                   store_dtype=torch.bfloat16)
    gen = torch.Generator(device="cuda").manual_seed(23)
    pt.kv_pool.copy_((torch.randn(pt.kv_pool.shape, generator=gen, device="cuda") / math.sqrt(d)).to(torch.bfloat16))
    st = grow_trie(pt, [list(range(32768)), list(range(7, 32775))], 64, 300, seed=5)
    torch.cuda.synchronize()
    n = len(st.candidates)
    segs, paths = st.segment_tree()
    lens = sorted(segs[p[-1]][1] for p in paths)
    say(f"config 5 trie: {n} candidates, {len(segs)} segments, private suffixes {lens[0]}..{lens[-1]} tokens")
    q = (torch.randn((n, hq, d), generator=gen, device="cuda") / math.sqrt(d)).to(torch.bfloat16)
    flat = st.flat_lists()
    picks = [0, 31, 63, 64, 100, 127][: n]
    picker = StrategyPicker(hq, hkv, page)
    plans = {"auto": picker.choose(st)}
    say(f"config 5 trie: picker costs {plans['auto'].costs}, chose {plans['auto'].kind}")
    for kind in ("flat", "split", "tree"):
        picker.candidates = (kind,)
        plans[kind] = picker.choose(st)
    ft = StrategyPicker(hq, hkv, page, "fasttree", candidates=("tree",))
    plans["tree-fasttree"] = ft.choose(st)
    for name, plan in plans.items():
        say(f"config 5 trie: {name} ({len(plan.levels)} levels)")
        w = MultiLevelCascadeAttentionWrapper(len(plan.levels), ws)
        lv = plan.levels
        w.plan([l[0] for l in lv], [l[1] for l in lv], [l[2] for l in lv], [l[3] for l in lv], hq, hkv, d, page,
               causal=False, q_data_type=torch.bfloat16)
        o, lse = w.run(q, pt.kv_cache_at_layer[0], return_lse=True)
        torch.cuda.synchronize()
        check_subset(o, lse, pt.kv_cache_at_layer[0], flat, q, picks, [0, 6], page, d ** -0.5)
    f = BatchDecodeWithPagedKVCacheWrapper(ws)
    f.plan(*flat, hq, hkv, d, page, q_data_type=torch.bfloat16)
    fo, fl = f.run(q, pt.kv_cache_at_layer[0], return_lse=True)
    torch.cuda.synchronize()
    check_subset(fo, fl, pt.kv_cache_at_layer[0], flat, q, picks, [3], page, d ** -0.5)


def test_config4_e2e_live_state():
    """Config 4 end to end, all 256 decode steps with HIP graphs: the trie is
    replayed on the oracle with the engine's own selections (page ids,
    candidates, fork copies, free list identical at every step); the
    selections of steps 0, 13, 39, 97, 163 and 255 are checked bit for bit
    against the oracle on the same logits; the final ranking of every request
    (beam_state.py:646-682) equals the oracle's; then layer 5's cascade
    attention at the live state after step 256 (beam suffixes past 128 tokens,
    leaf groups on the streaming kernel) is checked against the oracle on the
    real pages."""
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    from beam_engine_amd import MultiLevelCascadeAttentionWrapper, PageTable
    from beam_engine_amd.generator import BatchedBeamSearch
    from beam_engine_amd.llama import LlamaConfig, LlamaDecoder
    from oracle import topk as ot
    from oracle.beam_state import OracleAllocator, OracleBeamState, OResult
    say("config 4 e2e: Llama-3-8B shape, 8 x beam 16, 1024-token prompts")
    cfg = LlamaConfig.llama3_8b()
    model = LlamaDecoder(cfg, "cuda", torch.bfloat16, seed=0)
    pages = 4096
    pt = PageTable(cfg.num_hidden_layers, page_size=16, max_num_pages=pages, head_num=8, head_dim=128,
                   device="cuda", store_dtype=torch.bfloat16)
    beam, n_req = 16, 8
    gen = BatchedBeamSearch(model, pt, beam, kernel_type="cascade", graphs=True)
    prompts = np.random.default_rng(0).integers(0, cfg.vocab_size, size=(n_req, 1024)).tolist()
    o_alloc = OracleAllocator(pages, 16)
    o = OracleBeamState(beam, o_alloc)
    for p in prompts:
        o.add_root_sequence(p)

    def root_of(node):
        while node.parent is not None:
            node = node.parent
        return node
    # request r's root page node (each request's candidates stay below it)
    request_of_root = {id(root_of(o.candidates[r].node)): r for r in range(n_req)}
    # the graph capture reserves the pool's last page as its scratch slot
    o_alloc.free_pages.remove(pages - 1)
    step = {"i": 0}
    check_steps = {0, 13, 39, 97, 163, 255}
    steps = 256
    real_select = gen.strategy.select_batched

    def select(state, logits, temperature, mode):
        res = real_select(state, logits, temperature, mode)
        if step["i"] in check_steps:
            say(f"config 4 e2e: selection of step {step['i']} against the oracle")
            lg = logits.float().cpu().numpy()
            cands = state.candidates
            for r in range(n_req):
                rows = [i for i, c in enumerate(cands) if c.request_id == r]
                _, _, _, per_row, _ = ot.beam_step(lg[rows], [cands[i].score for i in rows], beam, "bfloat16")
                for j, i in enumerate(rows):
                    assert [(t.token_id, t.accumulated_score) for t in res[i].children] == per_row[j], \
                        f"step {step['i']} request {r} row {j}"
        o.add_filtered_results([OResult(o.candidates[i], [(t.token_id, t.accumulated_score) for t in r.children])
                                for i, r in enumerate(res)])
        step["i"] += 1
        return res
    gen.strategy.select_batched = select

    logits = gen.prefill(prompts)
    lg = logits.float().cpu().numpy()
    o.add_filtered_results([OResult(o.candidates[r], ot.prefill_select(lg[r], beam, "bfloat16"))
                            for r in range(n_req)])
    say(f"config 4 e2e: prefill done; decoding {steps} steps")
    for i in range(steps):
        gen.step()
        got = [(c.trie_node.page_id, list(c.trie_node.tokens), c.score) for c in gen.state.candidates]
        want = [(c.node.page_id, c.node.tokens, c.score) for c in o.candidates]
        assert got == want, f"trie differs after step {i}"
        assert list(pt.free_pages) == list(o_alloc.free_pages), f"free list differs after step {i}"
        if (i + 1) % 32 == 0:
            say(f"config 4 e2e: step {i + 1}/{steps} trie replay equal")
    assert step["i"] == steps and o_alloc.copies, "the run should fork partial pages"
    # the final ranking of every request against the oracle's
    finals = gen.final_sequences()
    for r in range(n_req):
        sub = OracleBeamState.__new__(OracleBeamState)
        sub.finished_candidates = []
        sub.candidates = [c for c in o.candidates if request_of_root[id(root_of(c.node))] == r]
        want = sub.get_final_sequences(beam, 1.0)
        assert [(list(sq), sc) for sq, sc in finals[r]] == [(list(sq), sc) for sq, sc in want], f"request {r}"
        assert len(want[0][0]) == 1024 + steps + 1
    say("config 4 e2e: final sequences of the 8 requests equal the oracle's")
    # the last selection's fork copies (staged for a next step) into the pages
    gen.flush()
    # one layer's attention at the live state, on the real pages
    st = gen.state
    lv = st._cascade_lists()
    levels = ([l[0] for l in lv], [l[1] for l in lv], [l[2] for l in lv], [l[3] for l in lv])
    n = len(st.candidates)
    g = torch.Generator(device="cuda").manual_seed(3)
    q = (torch.randn((n, 32, 128), generator=g, device="cuda") / math.sqrt(128)).to(torch.bfloat16)
    ws = torch.empty(256 << 20, dtype=torch.uint8, device="cuda")
    w = MultiLevelCascadeAttentionWrapper(len(lv), ws)
    w.plan(*levels, 32, 8, 128, 16, causal=True, q_data_type=torch.bfloat16)
    out, lse = w.run(q, pt.kv_cache_at_layer[5], return_lse=True)
    torch.cuda.synchronize()
    used = sorted({p for l in levels[2] for p in l})
    remap = {p: i for i, p in enumerate(used)}
    kv = pt.kv_cache_at_layer[5][torch.tensor(used, device="cuda")].float().cpu()
    ref_o, ref_lse = oa.cascade_attention(q.float().cpu(), kv, levels[0], levels[1],
                                          [[remap[p] for p in l] for l in levels[2]], levels[3], 16, 128 ** -0.5)
    np.testing.assert_allclose(out.float().cpu().numpy(), ref_o, **TOL)
    fin = np.isfinite(ref_lse)
    np.testing.assert_allclose(lse.cpu().numpy()[fin], ref_lse[fin], rtol=2e-3, atol=2e-3)
    say(f"config 4 e2e: layer 5 attention after step {steps} equal ({len(lv)} levels, {n} candidates)")
