"""The decode step as one HIP graph: fixed-layout attention plans replayed in
a captured graph equal the compact plans run eagerly, and the whole-step
graph gives the per-layer path's logits."""

import math
import random
import sys

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def say(msg):
    print(f"[case] {msg}", flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module", autouse=True)
def need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")


def step_trie(st, rng):
    """One random decode step that keeps each request's beam count: a few
    beams die and as many others fork in two, the rest go on."""
    from beam_engine_amd.beam_state import BeamGenerateResult, BeamToken
    res = []
    cands = st.candidates
    for rid in sorted({c.request_id for c in cands}):
        idx = [i for i, c in enumerate(cands) if c.request_id == rid]
        kids = {i: 1 for i in idx}
        for i, j in zip(rng.sample(idx, 3), rng.sample(idx, 3)):
            if i != j and kids[i] == 1 and kids[j] == 1:
                kids[i], kids[j] = 0, 2
        for i in idx:
            c = cands[i]
            res.append(BeamGenerateResult(c, [BeamToken(rng.randrange(50000), c.score - rng.random())
                                              for _ in range(kids[i])]))
    st.add_filtered_results(res)


def test_fixed_layout_graph_replay_matches_compact_plan():
    """A fixed-layout cascade launch captured once and replayed after each
    re-plan of a growing multi-request trie (forks, deaths, suffixes of many
    lengths) writes what the compact plan of the same step writes eagerly;
    every replay is checked, with eager work between replays."""
    from beam_engine_amd import MultiLevelCascadeAttentionWrapper, PageTable
    from beam_engine_amd.generator import BatchedBeamSearch
    from test_gpu_configs import grow_trie
    say("fixed-layout graph replay: 4 requests x beam 16 over 300-token prompts, 12 re-plans")
    hq, hkv, d, page = 32, 8, 128, 16
    pt = PageTable(1, page_size=page, max_num_pages=4096, head_num=hkv, head_dim=d, device="cuda",
                   store_dtype=torch.bfloat16)
    g = torch.Generator(device="cuda").manual_seed(7)
    pt.kv_pool.copy_((torch.randn(pt.kv_pool.shape, generator=g, device="cuda") / math.sqrt(d)).to(torch.bfloat16))
    st = grow_trie(pt, [list(range(300 + 17 * r)) for r in range(4)], 16, 3, seed=11)
    ws_a = torch.empty(64 << 20, dtype=torch.uint8, device="cuda")
    ws_b = torch.empty(64 << 20, dtype=torch.uint8, device="cuda")
    n = len(st.candidates)
    q = (torch.randn((n, hq, d), generator=g, device="cuda") / math.sqrt(d)).to(torch.bfloat16)
    out_b = torch.zeros_like(q)
    kv = pt.kv_cache_at_layer[0]
    fixed = graph = key = None
    rng = random.Random(3)
    replays = 0
    for it in range(12):
        lv = st._cascade_lists()
        levels = ([l[0] for l in lv], [l[1] for l in lv], [l[2] for l in lv], [l[3] for l in lv])
        a = MultiLevelCascadeAttentionWrapper(len(lv), ws_a)
        a.plan(*levels, hq, hkv, d, page, causal=True, q_data_type=torch.bfloat16)
        want = a.run(q, kv)
        if fixed is None:
            fixed = MultiLevelCascadeAttentionWrapper(len(lv), ws_b)
            fixed.use_fixed_layout(max_items=4 * a.stats.num_items + 1024, max_queries=n, max_pages=16384,
                                   max_merge=n * hkv, max_merge_rows=4 * a.stats.num_part_rows + 1024, max_zero=n,
                                   tile_rows=64, max_tails=8192)
        fixed.num_levels = len(lv)
        fixed.plan(*levels, hq, hkv, d, page, causal=True, q_data_type=torch.bfloat16)
        assert fixed._info.kernel == 2 and fixed._info.static_layout == 1
        if graph is None:
            key = BatchedBeamSearch._launch_key(fixed._info)
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                fixed.run(q, kv, out=out_b)
        assert BatchedBeamSearch._launch_key(fixed._info) == key, "the fixed layout changed its launch shape"
        out_b.zero_()
        graph.replay()
        replays += 1
        torch.cuda.synchronize()
        assert torch.allclose(out_b.float(), want.float(), atol=1e-2, rtol=2e-2), \
            f"replay {it}: max diff {(out_b.float() - want.float()).abs().max().item()}"
        # grow the trie two steps (new plan, new counts) before the next replay
        for _ in range(2):
            step_trie(st, rng)
    assert replays >= 2


def test_step_graph_logits_match_per_layer_path():
    """One decode step of a 2-layer Llama-3-8B-shaped model: the whole-step
    graph (fixed-layout attention inside) and the per-layer graphs with eager
    attention give the same logits from the same state and inputs."""
    from beam_engine_amd.generator import BatchedBeamSearch
    from beam_engine_amd.llama import LlamaConfig, LlamaDecoder
    from beam_engine_amd.page_table import PageTable
    say("step graph vs per-layer path: 2 layers, 4 requests x beam 8, 200-token prompts")
    cfg = LlamaConfig.llama3_8b()
    cfg.num_hidden_layers = 2
    model = LlamaDecoder(cfg, "cuda", torch.bfloat16, seed=1)
    pt = PageTable(cfg.num_hidden_layers, page_size=16, max_num_pages=2048, head_num=8, head_dim=128,
                   device="cuda", store_dtype=torch.bfloat16)
    gen = BatchedBeamSearch(model, pt, 8, kernel_type="cascade", graphs=True)
    prompts = np.random.default_rng(2).integers(0, cfg.vocab_size, size=(4, 200)).tolist()
    gen.prefill(prompts)
    gen.prepare_graphs()
    for step in range(3):
        st = gen.state
        n = st.num_candidates()
        # the previous selection's fork copies (staged for the step graph's first
        # part) into the pages before either path reads them
        gen.flush()
        levels, qids, wp, wpos, pos = st.step_metadata()
        dev = torch.device("cuda")
        tok = torch.from_numpy(np.asarray(qids, np.int64)).to(dev)
        psn = torch.from_numpy(np.asarray(pos, np.int64)).to(dev)
        wpg = torch.from_numpy(np.asarray(wp, np.int32)).to(dev)
        wps = torch.from_numpy(np.asarray(wpos, np.int32)).to(dev)
        w = gen._plan(levels, True)
        gen._gd.load_inputs(tok, psn, wpg, wps)
        want = gen._gd.run(lambda l, q, kv, out=None: w.run(q, kv, out=out)).float().clone()
        wf = gen._fixed_plan(levels, n)
        assert wf is not None, "the step graph should take this plan"
        gen._gd.load_inputs(tok, psn, wpg, wps)
        got = gen._gd.run_step().float().clone()
        torch.cuda.synchronize()
        assert torch.allclose(got, want, atol=5e-2, rtol=5e-2), \
            f"step {step}: max logit diff {(got - want).abs().max().item()}"
        # the decode loop's path: metadata and plan from one native call
        ins = st.plan_cascade(gen._fixed, cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim,
                              torch.bfloat16)
        for x, y in zip(ins, (qids, wp, wpos, pos)):
            assert np.array_equal(np.asarray(x), np.asarray(y))
        assert gen._launch_key(gen._fixed._info) == gen._fixed_key
        gen._gd.load_inputs(tok, psn, wpg, wps)
        got2 = gen._gd.run_step().float().clone()
        torch.cuda.synchronize()
        assert torch.equal(got2, got), f"step {step}: the native plan's replay differs"
        gen.step()                              # advance (the step graph path)
        assert gen.step_graphed
