"""Diverse beam search (reference: src/beam_engine/beam_strategy.py:60-400).

The oracle restatement (oracle.topk.diverse_select) is pinned by hand-derived
cases that each exercise one rule of the reference's selection: the pool
sorted by log_prob (not by the accumulated score), group-by-group picks with
the Hamming or cumulative penalty, ties kept in the stable pool order, the
length normalisation, and the cut from the last candidates when the groups
pick more than the beam.  The product's host selection and the GPU kernel
(be_diverse_select, Hamming) are checked against the oracle."""

import random

import numpy as np
import pytest
import torch

from beam_engine_amd.beam_state import (BeamCandidate, BeamGenerateInput, BeamState, BeamTokenCandidate,
                                        TrieNode)
from beam_engine_amd.beam_strategy import DiverseBeamSearchStrategy
from oracle import topk as ot


def _pool(rows):
    vals = np.array([[lp for _, lp in r] for r in rows], dtype=np.float32)
    idx = np.array([[t for t, _ in r] for r in rows], dtype=np.int64)
    return vals, idx


def test_oracle_hamming_hand_case():
    # B = 4, 2 groups of 2, penalty 0.6, parents of 3 tokens (length 4: every
    # adjusted score divided by 4, which keeps the order)
    vals, idx = _pool([[(10, -0.5), (11, -1.0), (12, -2.0), (13, -3.0)],
                       [(11, -0.5), (10, -1.5), (14, -1.75), (15, -4.0)]])
    _, flat = ot.diverse_select([-1.0, -0.2], vals, idx, 4, 2, 0.6, "hamming", 1.0, [[1, 2, 3], [1, 2, 3]])
    # group 0 takes the two -0.5 choices (10 of row 0, 11 of row 1); group 1 sees
    # 11 -> (-1.0 - 0.6) / 4 = -0.4, 14 -> -0.4375, 12 -> -0.5, 10 -> -0.525
    assert flat == [(0, 10, -1.0 + -0.5), (0, 11, -1.0 + -1.0), (1, 11, -0.2 + -0.5), (1, 14, -0.2 + -1.75)]


def test_oracle_ties_follow_the_stable_pool_order():
    vals, idx = _pool([[(1, -1.0), (2, -1.5)], [(1, -1.0), (3, -1.5)]])
    _, flat = ot.diverse_select([0.0, 0.0], vals, idx, 2, 2, 0.5, "hamming", 1.0)
    # group 0: (row 0, token 1) before the equal (row 1, token 1); group 1: three
    # choices at -1.5 -- the penalised (row 1, token 1) came first in the pool
    assert flat == [(0, 1, -1.0), (1, 1, -1.0)]


def test_oracle_cut_from_the_last_candidates():
    # B = 2 with 4 groups of max(1, 0) = 1: four picks, the last two dropped from
    # the end of the last rows, so row 0 keeps its worse second child
    vals, idx = _pool([[(5, -1.0), (6, -2.0)], [(7, -1.5), (8, -3.0)]])
    per_row, flat = ot.diverse_select([0.0, 0.0], vals, idx, 2, 4, 0.0, "hamming", 1.0)
    assert flat == [(0, 5, -1.0), (0, 6, -2.0)] and per_row[1] == []


def test_oracle_cumulative_hand_case():
    vals, idx = _pool([[(4, -1.0), (5, -1.25)], [(4, -1.125), (6, -1.375)]])
    _, flat = ot.diverse_select([0.0, 0.0], vals, idx, 2, 2, 1.0, "cumulative", 0.0, [[1, 2], [1, 3]])
    # group 1 against [1, 2, 4]: [1, 3, 4] overlaps 2 (-3.125), [1, 2, 5] 2 (-3.25), [1, 3, 6] 1 (-2.375)
    assert flat == [(0, 4, -1.0), (1, 6, -1.375)]


def test_oracle_single_group_without_penalty_is_log_prob_order():
    rng = np.random.default_rng(3)
    vals = rng.standard_normal((5, 6)).astype(np.float32)
    idx = rng.permutation(1000)[:30].reshape(5, 6)
    parents = rng.standard_normal(5)
    _, flat = ot.diverse_select(parents, vals, idx, 7, 1, 0.0)
    order = sorted(range(30), key=lambda i: (-float(vals.flat[i]), i))[:7]      # log_prob, not the total
    exp = sorted(order, key=lambda i: (i // 6, order.index(i)))                  # by row, in pick order
    assert [(r, t) for r, t, _ in flat] == [(i // 6, int(idx.flat[i])) for i in exp]


def test_planted_mistake_ranking_by_total_score_is_caught():
    """A restatement that ranks the pool by parent score + log_prob (the vanilla
    rule) instead of log_prob disagrees with the hand case."""
    vals, idx = _pool([[(10, -0.5), (11, -1.0), (12, -2.0), (13, -3.0)],
                       [(11, -0.5), (10, -1.5), (14, -1.75), (15, -4.0)]])
    parents = [-1.0, -0.2]
    wrong = vals + np.array(parents, dtype=np.float32)[:, None]
    _, flat = ot.diverse_select([0.0, 0.0], wrong, idx, 4, 2, 0.6, "hamming", 1.0, [[1, 2, 3], [1, 2, 3]])
    assert [(r, t) for r, t, _ in flat] != [(0, 10), (0, 11), (1, 11), (1, 14)]


class _Pages:
    page_size = 4


def _state(n, beam, rng, seq_len=5):
    st = BeamState(beam, _Pages())
    cands = []
    for i in range(n):
        root = TrieNode([rng.randrange(6) for _ in range(seq_len)], i)
        cands.append(BeamCandidate(root, -rng.random()))
    st.candidates = cands
    return st


@pytest.mark.parametrize("kind", ["hamming", "cumulative"])
@pytest.mark.parametrize("seed", range(6))
def test_product_host_selection_matches_oracle(kind, seed):
    rng = random.Random(seed)
    beam, groups = rng.choice([(4, 2), (8, 4), (6, 4), (2, 4), (16, 3)])
    n = rng.randint(1, beam)
    k = 2 * beam
    st = _state(n, beam, rng)
    # log-probs on a coarse grid: many ties
    vals = np.array([[-0.25 * rng.randrange(12) for _ in range(k)] for _ in range(n)], dtype=np.float32)
    vals = -np.sort(-vals, axis=1)
    idx = np.array([rng.sample(range(40), k) for _ in range(n)])
    penalty = rng.choice([0.0, 0.25, 0.5, 2.0])
    lpen = rng.choice([0.0, 1.0, 0.5])
    inputs = [BeamGenerateInput(c, [BeamTokenCandidate(int(t), float(v)) for t, v in zip(idx[r], vals[r])])
              for r, c in enumerate(st.candidates)]
    strat = DiverseBeamSearchStrategy(groups, penalty, kind, lpen)
    got = strat.select_candidates(st, inputs, 0)
    seqs = [strat._sequence(c.trie_node) for c in st.candidates]
    per_row, _ = ot.diverse_select([c.score for c in st.candidates], vals, idx, beam, groups, penalty, kind, lpen,
                                   seqs)
    assert [[(b.token_id, b.accumulated_score) for b in r.children] for r in got] == per_row


@pytest.mark.gpu
@pytest.mark.parametrize("case", ["b4g2", "b8g4", "b16g4", "b16g16", "b2g4", "b16g3_multi", "b64g8_multi"])
def test_gpu_diverse_select_matches_oracle(case):
    """be_diverse_select on the GPU row top-k of bf16 logits (frequent ties)
    against the oracle, request by request."""
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    from beam_engine_amd.selection import beam_topk, diverse_select
    print(f"[case] diverse select {case}", flush=True)
    beam = int(case[1:].split("g")[0])
    groups = int(case.split("g")[1].split("_")[0])
    rng = np.random.default_rng(sum(map(ord, case)))
    reqs = [beam, beam - 1, beam] if case.endswith("multi") else [beam]
    n = sum(reqs)
    vocab = 3000
    logits = torch.from_numpy(rng.standard_normal((n, vocab)).astype(np.float32) * 2).to(torch.bfloat16).cuda()
    parents = torch.from_numpy(-rng.random(n))
    k = 2 * beam
    penalty = 0.75
    vals, idx = beam_topk(logits, k)
    par, tok, sc = diverse_select(vals, idx, parents, beam, groups, penalty,
                                  request_rows=reqs if len(reqs) > 1 else None)
    v, ix = vals.cpu().numpy(), idx.cpu().numpy().astype(np.int64)
    r0 = 0
    for q, nr in enumerate(reqs):
        _, flat = ot.diverse_select(parents[r0:r0 + nr].tolist(), v[r0:r0 + nr], ix[r0:r0 + nr], beam, groups,
                                    penalty)
        got = [(int(p) - r0, int(t), float(s)) for p, t, s in
               zip(par[q * beam:(q + 1) * beam], tok[q * beam:(q + 1) * beam], sc[q * beam:(q + 1) * beam]) if p >= 0]
        assert got == [(r, t, s) for r, t, s in flat], f"request {q}"
        r0 += nr


@pytest.mark.gpu
def test_gpu_engine_decodes_with_diverse_strategy():
    """The batched engine with DiverseBeamSearchStrategy on a tiny model: each
    step's GPU selection equals the oracle's on the same logits, per request."""
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    print("[case] engine with diverse strategy", flush=True)
    from beam_engine_amd import PageTable
    from beam_engine_amd.generator import BatchedBeamSearch
    from beam_engine_amd.llama import LlamaConfig, LlamaDecoder
    from beam_engine_amd.selection import beam_topk
    cfg = LlamaConfig(num_hidden_layers=2, hidden_size=256, num_attention_heads=8, num_key_value_heads=2,
                      head_dim=128, intermediate_size=512, vocab_size=512, max_position_embeddings=512)
    model = LlamaDecoder(cfg, "cuda", torch.bfloat16, seed=5)
    pt = PageTable(2, page_size=4, max_num_pages=512, head_num=2, head_dim=128, device="cuda",
                   store_dtype=torch.bfloat16)
    beam = 4
    strat = DiverseBeamSearchStrategy(num_groups=2, diversity_penalty=0.5)
    gen = BatchedBeamSearch(model, pt, beam, strategy=strat, kernel_type="cascade")
    gen.prefill([list(range(5, 23)), list(range(100, 118))])
    seen = []
    orig = gen._select

    def check(logits):
        st = gen.state
        cands = list(st.candidates)
        vals, idx = beam_topk(logits, 2 * beam)
        v, ix = vals.cpu().numpy(), idx.cpu().numpy().astype(np.int64)
        exp = []
        r0 = 0
        while r0 < len(cands):
            r1 = r0
            while r1 < len(cands) and cands[r1].request_id == cands[r0].request_id:
                r1 += 1
            per_row, _ = ot.diverse_select([c.score for c in cands[r0:r1]], v[r0:r1], ix[r0:r1], beam, 2, 0.5)
            exp += per_row
            r0 = r1
        res = strat.select_batched(st, logits)
        assert [[(b.token_id, b.accumulated_score) for b in r.children] for r in res] == exp
        seen.append(len(cands))
        st.add_filtered_results(res)

    gen._select = check
    for _ in range(6):
        gen.step()
    torch.cuda.synchronize()
    assert seen == [8] * 6 and len(gen.state.candidates) == 8
