"""End-to-end decode loop on a tiny Llama through the HIP path, checked step by
step against the oracle: every layer's attention output (same q, same paged
KV state), the beam selection (bit-exact on the same logits) and the trie /
page allocation (an oracle replay of the same selections)."""

import sys

import numpy as np
import pytest
import torch

from oracle import attention as oa
from oracle import topk as ot
from oracle.beam_state import OracleAllocator, OracleBeamState, OResult

pytestmark = pytest.mark.gpu


def say(msg):
    print(f"[case] {msg}", flush=True)
    sys.stdout.flush()


@pytest.mark.parametrize("kind", ["cascade", "fasttree", "flat", "split", "tree", "auto"])
def test_tiny_llama_beam_search_matches_oracle(kind):
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    say(f"tiny llama beam search {kind}")
    from beam_engine_amd import PageTable
    from beam_engine_amd.generator import BatchedBeamSearch
    from beam_engine_amd.llama import LlamaConfig, LlamaDecoder

    cfg = LlamaConfig(num_hidden_layers=2, hidden_size=256, num_attention_heads=8, num_key_value_heads=2,
                      head_dim=128, intermediate_size=512, vocab_size=512, max_position_embeddings=512)
    model = LlamaDecoder(cfg, "cuda", torch.bfloat16, seed=3)
    pt = PageTable(2, page_size=4, max_num_pages=512, head_num=2, head_dim=128, device="cuda",
                   store_dtype=torch.bfloat16)
    beam, n_req = 4, 2
    gen = BatchedBeamSearch(model, pt, beam, kernel_type=kind)
    prompts = [list(range(5, 23)), list(range(100, 118))]

    # oracle replay of the trie, fed with the engine's own selections
    o_alloc = OracleAllocator(512, 4)
    o = OracleBeamState(beam, o_alloc)
    for p in prompts:
        o.add_root_sequence(p)

    checks = {"attn": 0}

    def timer(li, run_fn, w):
        out = run_fn(lambda: None)
        # oracle attention on the same q and the same KV pool (read after the append)
        torch.cuda.synchronize()
        q = timer.q[li]
        kv = pt.kv_cache_at_layer[li].float().cpu()
        if kind == "cascade":
            lv = gen.state._cascade_lists()
            ref, _ = oa.cascade_attention(q, kv, [l[0] for l in lv], [l[1] for l in lv], [l[2] for l in lv],
                                          [l[3] for l in lv], 4, 128 ** -0.5)
        else:
            # every other kind attends each candidate's whole path once (the
            # oracle replay's pages; "fasttree" with the newest token, as the
            # reference's req_to_token covers it)
            inc = kind == "fasttree"
            kvp, kvi, lpl = [0], [], []
            for ci, c in enumerate(o.candidates):
                kvi.extend(o.path_pages(ci))
                kvp.append(len(kvi))
                lpl.append(len(c.node.tokens) - (0 if inc else 1))
            ref, _ = oa.paged_attention(q, kv, kvp, kvi, lpl, 4, 128 ** -0.5)
        np.testing.assert_allclose(out.float().cpu().numpy(), ref, rtol=2e-2, atol=1e-2)
        checks["attn"] += 1
        return out
    timer.q = {}

    def capture_attn(li, run_fn, w):
        return timer(li, run_fn, w)

    # capture q per layer by wrapping the model's decode attention callback
    real_decode = model.decode

    def decode(tok, pos, wpg, wps, page_table, attn):
        def attn2(li, q, kvl):
            timer.q[li] = q.float().cpu()
            return attn(li, q, kvl)
        return real_decode(tok, pos, wpg, wps, page_table, attn2)
    model.decode = decode
    gen.attn_timer = capture_attn

    # selection check: wrap _select to compare with the oracle on the same logits
    real_select = gen._select

    def select(logits):
        cands = list(gen.state.candidates)
        lg = logits.float().cpu().numpy()
        res_by_idx = {}
        for r in range(n_req):
            rows = [i for i, c in enumerate(cands) if c.request_id == r]
            _, _, _, per_row, _ = ot.beam_step(lg[rows], [cands[i].score for i in rows], beam, "bfloat16")
            for j, i in enumerate(rows):
                res_by_idx[i] = per_row[j]
        real_select(logits)
        o.add_filtered_results([OResult(o.candidates[i], res_by_idx[i]) for i in range(len(cands))])
        got = [(c.trie_node.page_id, list(c.trie_node.tokens), c.score) for c in gen.state.candidates]
        want = [(c.node.page_id, c.node.tokens, c.score) for c in o.candidates]
        assert got == want
    gen._select = select

    # prefill expansion: replay on the oracle with the engine's choice (checked against prefill_select)
    logits = gen.prefill(prompts)
    lg = logits.float().cpu().numpy()
    o_res = []
    for r in range(n_req):
        sel = ot.prefill_select(lg[r], beam, "bfloat16")
        o_res.append(OResult(o.candidates[r], sel))
    o.add_filtered_results(o_res)
    assert [(c.trie_node.page_id, list(c.trie_node.tokens), c.score) for c in gen.state.candidates] == \
        [(c.node.page_id, c.node.tokens, c.score) for c in o.candidates]
    for _ in range(10):
        gen.step()
    assert checks["attn"] == 10 * cfg.num_hidden_layers
    assert o_alloc.copies, "the run should have forked partial pages"
    if kind == "auto":
        say(f"auto picks: {[e['kind'] for e in gen.step_log]}")


def test_graph_replays_match_eager_steps():
    """The segment-graph decode (HIP graphs replayed every step, eager attention,
    eager selection and trie updates in between) gives the same logits and the
    same beams as the fully eager decode, step after step."""
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    say("graph replays vs eager")
    from beam_engine_amd import PageTable
    from beam_engine_amd.generator import BatchedBeamSearch
    from beam_engine_amd.llama import LlamaConfig, LlamaDecoder

    cfg = LlamaConfig(num_hidden_layers=3, hidden_size=256, num_attention_heads=8, num_key_value_heads=2,
                      head_dim=128, intermediate_size=512, vocab_size=700, max_position_embeddings=512)
    runs = []
    for graphs in (False, True):
        model = LlamaDecoder(cfg, "cuda", torch.bfloat16, seed=11)
        pt = PageTable(3, page_size=8, max_num_pages=256, head_num=2, head_dim=128, device="cuda",
                       store_dtype=torch.bfloat16)
        gen = BatchedBeamSearch(model, pt, 4, kernel_type="cascade", graphs=graphs)
        logs = []
        real = gen._select

        def sel(logits, real=real, logs=logs):
            logs.append(logits.clone())
            real(logits)
        gen._select = sel
        gen.prefill([list(range(3, 23)), list(range(40, 60))])
        runs.append((gen, logs))
    (ge, le), (gg, lg) = runs
    for step in range(8):
        ge.step()
        gg.step()
        torch.cuda.synchronize()
        assert torch.equal(le[step], lg[step]), f"step {step} logits differ"
        assert [(c.trie_node.page_id, c.trie_node.tokens, c.score) for c in ge.state.candidates] == \
            [(c.trie_node.page_id, c.trie_node.tokens, c.score) for c in gg.state.candidates]
    assert gg._gd is not None and len(gg._gd.graphs) == cfg.num_hidden_layers + 1


def test_eos_finishes_beams_and_decoding_continues():
    """With eos_token_id set to a token the model picks, beams finish, requests
    continue with fewer live beams (eager steps: the candidate count changes),
    and every step's selection equals the oracle's on the same logits."""
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    say("tiny llama with an end-of-sequence token")
    from beam_engine_amd import PageTable
    from beam_engine_amd.generator import BatchedBeamSearch
    from beam_engine_amd.llama import LlamaConfig, LlamaDecoder
    from beam_engine_amd.selection import beam_topk

    cfg = LlamaConfig(num_hidden_layers=2, hidden_size=256, num_attention_heads=8, num_key_value_heads=2,
                      head_dim=128, intermediate_size=512, vocab_size=512, max_position_embeddings=512)
    prompts = [list(range(5, 23)), list(range(100, 118))]

    def run(eos, steps, check=False):
        model = LlamaDecoder(cfg, "cuda", torch.bfloat16, seed=3)
        pt = PageTable(2, page_size=4, max_num_pages=512, head_num=2, head_dim=128, device="cuda",
                       store_dtype=torch.bfloat16)
        gen = BatchedBeamSearch(model, pt, 4, kernel_type="cascade", graphs=True, eos_token_id=eos)
        gen.prefill(prompts)
        counts = []
        if check:
            orig = gen._select

            def sel(logits):
                st = gen.state
                cands = list(st.candidates)
                vals, idx = beam_topk(logits, 8)
                v, ix = vals.cpu().numpy(), idx.cpu().numpy().astype(np.int64)
                exp, r0 = [], 0
                while r0 < len(cands):
                    r1 = r0
                    while r1 < len(cands) and cands[r1].request_id == cands[r0].request_id:
                        r1 += 1
                    per_row, _ = ot.select_global([c.score for c in cands[r0:r1]], v[r0:r1], ix[r0:r1], 4)
                    exp += per_row
                    r0 = r1
                res = gen.strategy.select_batched(st, logits)
                assert [[(b.token_id, b.accumulated_score) for b in r.children] for r in res] == exp
                counts.append(len(cands))
                st.add_filtered_results(res, eos)
            gen._select = sel
        for _ in range(steps):
            if not gen.state.candidates:
                break
            gen.step()
        torch.cuda.synchronize()
        return gen, counts

    base, _ = run(None, 3)
    eos = base.state.candidates[0].trie_node.tokens[-1]        # a token picked in step 3 of the plain run
    gen, counts = run(eos, 8, check=True)
    assert gen.state.finished_candidates and all(c.sequence[-1] == eos for c in gen.state.finished_candidates)
    assert min(counts) < 8 and counts[0] == 8
    assert all(eos not in gen.state.sequence(c)[18:] for c in gen.state.candidates)


@pytest.mark.parametrize("kind", ["cascade", "fasttree", "flat", "auto"])
def test_graphed_decoder_inputs_start_valid_on_reused_memory(kind):
    """The graphed decoder's input buffers are carved from the generator's
    workspace (torch.empty).  Memory the caching allocator hands back holds
    earlier contents: the buffers must still read token 0 at position 0 for
    the capture's warm-up pass, and the graphed steps must match the eager
    ones.  The workspace's block is first filled with 0x7f bytes and freed,
    so that the generator reuses it.  Every strategy kind runs its steps as
    the whole-step graph (native plan into the fixed layout)."""
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    say(f"graphed decoder on reused workspace memory ({kind})")
    from beam_engine_amd import PageTable
    from beam_engine_amd.generator import BatchedBeamSearch, _STEP_HEADER_BYTES
    from beam_engine_amd.llama import LlamaConfig, LlamaDecoder

    cfg = LlamaConfig(num_hidden_layers=2, hidden_size=256, num_attention_heads=8, num_key_value_heads=2,
                      head_dim=128, intermediate_size=512, vocab_size=700, max_position_embeddings=512)
    ws_bytes = 8 << 20
    runs = []
    for graphs in (False, True):
        junk = torch.full((_STEP_HEADER_BYTES + ws_bytes,), 0x7F, dtype=torch.uint8, device="cuda")
        torch.cuda.synchronize()
        del junk
        model = LlamaDecoder(cfg, "cuda", torch.bfloat16, seed=12)
        pt = PageTable(2, page_size=16, max_num_pages=256, head_num=2, head_dim=128, device="cuda",
                       store_dtype=torch.bfloat16)
        gen = BatchedBeamSearch(model, pt, 4, kernel_type=kind, graphs=graphs, workspace_bytes=ws_bytes)
        gen.prefill([list(range(3, 40)), list(range(50, 87))])
        runs.append(gen)
    ge, gg = runs
    for step in range(6):
        ge.step()
        gg.step()
        torch.cuda.synchronize()
        assert [(c.trie_node.page_id, c.trie_node.tokens, c.score) for c in ge.state.candidates] == \
            [(c.trie_node.page_id, c.trie_node.tokens, c.score) for c in gg.state.candidates], f"step {step}"
    assert gg._gd is not None
    say(f"{kind}: {gg.graphed_steps} of 6 steps as one graph; kinds {[e['kind'] for e in gg.step_log]}")
    assert gg.graphed_steps >= 5 and ge.graphed_steps == 0
