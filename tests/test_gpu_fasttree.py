"""The reference's FastTree call path on the GPU, through this build's
entry points: ``BeamState.get_fasttree_input()`` (beam_state.py:566-633) ->
``prepare_fasttree_metadata_for_paged_cache`` (preparation.py:11-225) ->
``fasttree_decode`` (kernel.py:288-348) per layer.  Every candidate's output
must equal the float64 oracle's attention over the slots its ``req_to_token``
row lists (its whole root-to-leaf path once, the newest token included),
for multi-request forests grown by random selections (branch points at
every depth, dead branches, private suffixes of many lengths).

Tolerance (bf16 storage against the float64 oracle): 2e-2 relative, 1e-2
absolute."""

import math
import random
import sys

import numpy as np
import pytest
import torch

from oracle import attention as oa

pytestmark = pytest.mark.gpu


def say(msg):
    print(f"[case] {msg}", flush=True)
    sys.stdout.flush()


def grow(pt, prompts, beam, steps, seed):
    from beam_engine_amd.beam_state import BeamGenerateResult, BeamState, BeamToken
    rng = random.Random(seed)
    st = BeamState(beam, pt)
    for r, p in enumerate(prompts):
        st.add_root_sequence(p, request_id=r)
    st.add_filtered_results([BeamGenerateResult(c, [BeamToken(1000 + j, -0.1 * j) for j in range(beam)])
                             for c in st.candidates])
    for _ in range(steps):
        res = []
        for rid in sorted({c.request_id for c in st.candidates}):
            idx = [i for i, c in enumerate(st.candidates) if c.request_id == rid]
            kids = {i: 1 for i in idx}
            swap = min(rng.choice([0, 1, 2]), len(idx) // 2)
            pick = rng.sample(idx, 2 * swap)
            for i in pick[:swap]:
                kids[i] = 0                 # a beam dies ...
            for i in pick[swap:]:
                kids[i] = 2                 # ... and another forks
            for i in idx:
                c = st.candidates[i]
                res.append(BeamGenerateResult(c, [BeamToken(rng.randrange(50000), c.score - rng.random())
                                                  for _ in range(kids[i])]))
        st.add_filtered_results(res)
    return st


@pytest.mark.parametrize("hq,hkv,page,beam,prompt,steps,costs", [
    (32, 8, 16, 8, [300, 170, 45], 60, "fasttree"),
    (64, 8, 16, 16, [700, 33], 40, "fasttree"),
    (32, 8, 16, 8, [200, 90, 520], 50, "mi355x"),
    (8, 8, 4, 4, [23, 9], 30, "fasttree"),
])
def test_fasttree_entry_points_match_oracle(hq, hkv, page, beam, prompt, steps, costs):
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    from beam_engine_amd import PageTable
    from beam_engine_amd.fasttree import fasttree_decode, prepare_fasttree_metadata_for_paged_cache
    d = 128
    say(f"fasttree entry points: {hq}/{hkv} heads, page {page}, beam {beam}, prompts {prompt}, {steps} steps, "
        f"{costs} edges")
    pt = PageTable(1, page_size=page, max_num_pages=4096, head_num=hkv, head_dim=d, device="cuda",
                   store_dtype=torch.bfloat16)
    gen = torch.Generator(device="cuda").manual_seed(hq + page + steps)
    pt.kv_pool.copy_((torch.randn(pt.kv_pool.shape, generator=gen, device="cuda") / math.sqrt(d)).to(torch.bfloat16))
    rp = random.Random(steps)
    st = grow(pt, [[rp.randrange(50000) for _ in range(n)] for n in prompt], beam, steps, seed=steps + hq)
    tree_nodes, req_to_token, qids, wp, wpos = st.get_fasttree_input()
    n = len(st.candidates)
    q = (torch.randn((n, hq, d), generator=gen, device="cuda") / math.sqrt(d)).to(torch.bfloat16)
    md = prepare_fasttree_metadata_for_paged_cache(tree_nodes, req_to_token, n, hq, hkv, d, "cuda", page_size=page,
                                                   q_data_type=torch.bfloat16, costs=costs)
    say(f"  {n} candidates, {len(tree_nodes)} tree nodes, {len(md.levels)} levels")
    o = fasttree_decode(q, pt.kv_cache_at_layer[0], None, md, sm_scale=d ** -0.5)
    torch.cuda.synchronize()
    # the oracle: each candidate over its req_to_token row (every path token)
    rtt = req_to_token.cpu().numpy()
    kvp, kvi, lpl = [0], [], []
    for ci, c in enumerate(st.candidates):
        length = len(st.sequence(c))
        slots = rtt[ci, :length]
        pages = list(dict.fromkeys((slots // page).tolist()))
        assert all(int(s) == pages[j // page] * page + j % page for j, s in enumerate(slots))
        kvi.extend(pages)
        kvp.append(len(kvi))
        lpl.append(length - (len(pages) - 1) * page)
    ref, _ = oa.paged_attention(q.float().cpu(), pt.kv_cache_at_layer[0].float().cpu(), kvp, kvi, lpl, page,
                                d ** -0.5)
    np.testing.assert_allclose(o.float().cpu().numpy(), ref, rtol=2e-2, atol=1e-2)
