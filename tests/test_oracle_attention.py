"""Pins the CPU attention oracle (oracle/attention.py) to mathematics that is
independent of its own formulas: explicit-loop brute force, closed forms,
torch's scaled_dot_product_attention in float64, and the merge identities."""

import math

import numpy as np
import pytest
import torch

from oracle import attention as oa


def rnd(shape, seed):
    return np.random.default_rng(seed).standard_normal(shape)


def test_partial_matches_loop_brute_force():
    q, k, v = rnd((3, 4, 5), 1), rnd((7, 2, 5), 2), rnd((7, 2, 5), 3)
    o, lse = oa.partial_attention(q, k, v, 0.37)
    o2, lse2 = oa.reference_attention_dense(q, k, v, 0.37)
    np.testing.assert_allclose(o, o2, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(lse, lse2, rtol=1e-12, atol=1e-12)


def test_partial_matches_torch_sdpa_fp64():
    n, hq, hkv, d, t = 5, 8, 2, 16, 33
    q, k, v = rnd((n, hq, d), 4), rnd((t, hkv, d), 5), rnd((t, hkv, d), 6)
    scale = d ** -0.5
    o, _ = oa.partial_attention(q, k, v, scale)
    g = hq // hkv
    tq = torch.from_numpy(q).permute(1, 0, 2)                              # [Hq, n, D]
    tk = torch.from_numpy(np.repeat(k, g, axis=1)).permute(1, 0, 2)       # [Hq, T, D]
    tv = torch.from_numpy(np.repeat(v, g, axis=1)).permute(1, 0, 2)
    ref = torch.nn.functional.scaled_dot_product_attention(tq, tk, tv, scale=scale)
    np.testing.assert_allclose(o, ref.permute(1, 0, 2).numpy(), rtol=1e-12, atol=1e-12)


def test_single_token_gives_v_and_score():
    q, k, v = rnd((2, 4, 8), 7), rnd((1, 1, 8), 8), rnd((1, 1, 8), 9)
    o, lse = oa.partial_attention(q, k, v, 0.5)
    np.testing.assert_allclose(o, np.broadcast_to(v[0, 0], o.shape), atol=1e-14)
    np.testing.assert_allclose(lse, (q @ k[0, 0]) * 0.5, atol=1e-14)


def test_constant_scores_give_mean_and_log_t():
    t = 11
    q, v = rnd((2, 2, 4), 10), rnd((t, 2, 4), 11)
    k = np.zeros((t, 2, 4))
    o, lse = oa.partial_attention(q, k, v, 1.0)
    np.testing.assert_allclose(o, np.broadcast_to(v.mean(axis=0), o.shape), atol=1e-14)
    np.testing.assert_allclose(lse, math.log(t), atol=1e-14)


def test_empty_set_is_zero_and_minus_inf():
    o, lse = oa.partial_attention(rnd((2, 4, 8), 1), np.zeros((0, 2, 8)), np.zeros((0, 2, 8)), 1.0)
    assert np.all(o == 0) and np.all(np.isneginf(lse))


def test_merge_identities_and_union():
    q = rnd((3, 4, 8), 12)
    k, v = rnd((20, 2, 8), 13), rnd((20, 2, 8), 14)
    oA, lA = oa.partial_attention(q, k[:7], v[:7], 0.3)
    oB, lB = oa.partial_attention(q, k[7:15], v[7:15], 0.3)
    oC, lC = oa.partial_attention(q, k[15:], v[15:], 0.3)
    oU, lU = oa.partial_attention(q, k, v, 0.3)
    o, l = oa.merge_states([oA, oB, oC], [lA, lB, lC])
    np.testing.assert_allclose(o, oU, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(l, lU, rtol=1e-12, atol=1e-12)
    # associativity
    oAB, lAB = oa.merge_states([oA, oB], [lA, lB])
    o2, l2 = oa.merge_states([oAB, oC], [lAB, lC])
    np.testing.assert_allclose(o2, o, rtol=1e-12, atol=1e-12)
    # merge(x, x) = (o, lse + ln 2)
    o3, l3 = oa.merge_states([oA, oA], [lA, lA])
    np.testing.assert_allclose(o3, oA, atol=1e-13)
    np.testing.assert_allclose(l3, lA + math.log(2), atol=1e-13)
    # (0, -inf) is the identity; all -inf gives (0, -inf)
    z, zl = np.zeros_like(oA), np.full_like(lA, -np.inf)
    o4, l4 = oa.merge_states([z, oA, z], [zl, lA, zl])
    np.testing.assert_allclose(o4, oA, atol=1e-14)
    np.testing.assert_allclose(l4, lA, atol=1e-14)
    o5, l5 = oa.merge_states([z, z], [zl, zl])
    assert np.all(o5 == 0) and np.all(np.isneginf(l5))


def test_cascade_equals_flat_attention_over_paths():
    """A two-level cascade (shared prefix + per-query suffix) equals one-pass
    attention over each query's concatenated path (Appendix B.4/B.5)."""
    page, hkv, hq, d = 4, 2, 4, 8
    rng = np.random.default_rng(3)
    kv = rng.standard_normal((12, 2, page, hkv, d))
    q = rng.standard_normal((3, hq, d))
    qo = [[0, 3], [0, 1, 2, 3]]
    kvp = [[0, 2], [0, 1, 3, 4]]
    kvi = [[0, 1], [2, 3, 4, 5]]
    lpl = [[4], [2, 3, 0]]
    o, lse = oa.cascade_attention(q, kv, qo, kvp, kvi, lpl, page, 0.4)
    paths = [([0, 1, 2], 2), ([0, 1, 3, 4], 3), ([0, 1, 5], 0)]
    for i, (pages, last) in enumerate(paths):
        k, v = oa.gather_kv(kv, pages, last, page)
        oi, li = oa.partial_attention(q[i:i + 1], k, v, 0.4)
        np.testing.assert_allclose(o[i], oi[0], rtol=1e-12, atol=1e-12)
        np.testing.assert_allclose(lse[i], li[0], rtol=1e-12, atol=1e-12)


def test_gather_rule():
    assert oa.group_slots([7, 3, 9], 2, 4) == [(7, 0), (7, 1), (7, 2), (7, 3), (3, 0), (3, 1), (3, 2), (3, 3), (9, 0), (9, 1)]
    assert oa.group_slots([5], 0, 4) == []


def test_planted_head_mapping_mistake_is_caught():
    """A plausible oracle bug (query head h reading kv head h % Hkv instead of
    h // g) must fail the torch fp64 comparison above."""
    n, hq, hkv, d, t = 2, 8, 2, 8, 9
    q, k, v = rnd((n, hq, d), 40), rnd((t, hkv, d), 41), rnd((t, hkv, d), 42)
    g = hq // hkv
    wrong_k = np.tile(k, (1, g, 1))      # head h -> kv head h % Hkv
    wrong_v = np.tile(v, (1, g, 1))
    o_wrong, _ = oa.partial_attention(q, wrong_k, wrong_v, 0.3)   # g == 1 path
    o_right, _ = oa.partial_attention(q, k, v, 0.3)
    assert not np.allclose(o_wrong, o_right, atol=1e-6)


def _one_request_levels(n_q, n_kv, page):
    npg = -(-n_kv // page)
    return ([[0, n_q]], [[0, npg]], [list(range(npg))], [[n_kv - (npg - 1) * page]]), npg


def test_causal_prefill_equals_torch_sdpa_lower_triangle():
    """qo_len == kv_len (a fresh prompt): the causal restatement is the plain
    lower-triangular mask of torch's fp64 scaled_dot_product_attention."""
    import torch
    rng = np.random.default_rng(11)
    page, hq, hkv, d, n = 4, 4, 2, 8, 13
    levels, npg = _one_request_levels(n, n, page)
    kv = rng.standard_normal((npg, 2, page, hkv, d))
    q = rng.standard_normal((n, hq, d))
    o, lse = oa.cascade_attention(q, kv, *levels, page, causal=True)
    k, v = oa.gather_kv(kv, levels[2][0], levels[3][0][0], page)
    qt = torch.from_numpy(q).permute(1, 0, 2)[None]                             # [1, Hq, n, D]
    kt = torch.from_numpy(np.repeat(k, hq // hkv, axis=1)).permute(1, 0, 2)[None]
    vt = torch.from_numpy(np.repeat(v, hq // hkv, axis=1)).permute(1, 0, 2)[None]
    ref = torch.nn.functional.scaled_dot_product_attention(qt, kt, vt, is_causal=True)[0].permute(1, 0, 2)
    np.testing.assert_allclose(o, ref.numpy(), rtol=0, atol=1e-12)
    assert np.isfinite(lse).all()


def test_causal_block_aligned_to_the_end_of_the_keys():
    """qo_len < kv_len (a prompt continuing cached tokens): query i of n sees
    the first kv_len - n + i + 1 tokens -- the dense loop on each query's
    visible prefix agrees, and the top-left alignment (i + 1 tokens) does not."""
    rng = np.random.default_rng(12)
    page, hq, hkv, d, n, t = 4, 2, 1, 4, 3, 9
    levels, npg = _one_request_levels(n, t, page)
    kv = rng.standard_normal((npg, 2, page, hkv, d))
    q = rng.standard_normal((n, hq, d))
    o, lse = oa.cascade_attention(q, kv, *levels, page, causal=True)
    k, v = oa.gather_kv(kv, levels[2][0], levels[3][0][0], page)
    for i in range(n):
        oi, li = oa.reference_attention_dense(q[i:i + 1], k[:t - n + i + 1], v[:t - n + i + 1], d ** -0.5)
        np.testing.assert_allclose(o[i:i + 1], oi, rtol=0, atol=1e-12)
        np.testing.assert_allclose(lse[i:i + 1], li, rtol=0, atol=1e-12)
    wrong, _ = oa.reference_attention_dense(q[:1], k[:1], v[:1], d ** -0.5)       # top-left: query 0 sees 1 token
    assert np.abs(wrong - o[:1]).max() > 1e-3


def test_causal_masks_only_the_last_level():
    rng = np.random.default_rng(13)
    page, hq, hkv, d = 4, 2, 1, 4
    kv = rng.standard_normal((4, 2, page, hkv, d))
    q = rng.standard_normal((2, hq, d))
    levels = ([[0, 2], [0, 2]], [[0, 2], [0, 2]], [[0, 1], [2, 3]], [[4, 3]])
    levels = (levels[0], levels[1], levels[2], [[4], [3]])
    a = oa.cascade_attention(q, kv, *levels, page, causal=True)
    # level 0 unmasked, level 1 causal: merge of the two computed separately
    o0, l0 = oa.cascade_attention(q, kv, [levels[0][0]], [levels[1][0]], [levels[2][0]], [levels[3][0]], page)
    o1, l1 = oa.cascade_attention(q, kv, [levels[0][1]], [levels[1][1]], [levels[2][1]], [levels[3][1]], page,
                                  causal=True)
    b = oa.merge_states([o0, o1], [l0, l1])
    np.testing.assert_allclose(a[0], b[0], atol=1e-12)
    np.testing.assert_allclose(a[1], b[1], atol=1e-12)


@pytest.mark.parametrize("name", ["cascade_md", "swapped", "uneven"])
def test_torch_fp32_cascade_matches_fp64(name):
    """The torch float32 CPU form (the CPU baseline's attention) equals the
    float64 restatement within float32 rounding on the reference's trees,
    with GQA and an empty group."""
    import torch
    from tests.conftest import load_fixtures
    tree = load_fixtures()["trees"][name]
    e = tree["expected"]
    levels = [e["qo_indptr"], e["kv_indptr"], e["kv_indices"], e["last_page_len"]]
    page = tree["page_size"]
    n = e["qo_indptr"][0][-1]
    npages = max(max(l) for l in e["kv_indices"] if l) + 2
    g = torch.Generator().manual_seed(3)
    kv = torch.randn((npages, 2, page, 2, 64), generator=g)
    q = torch.randn((n, 8, 64), generator=g)
    o64, lse64 = oa.cascade_attention(q, kv, *levels, page, 0.125)
    o32, lse32 = oa.cascade_attention_torch(q, kv, *levels, page, 0.125)
    np.testing.assert_allclose(o32.numpy(), o64, rtol=0, atol=1e-5)
    fin = np.isfinite(lse64)
    assert np.array_equal(fin, np.isfinite(lse32.numpy()))
    np.testing.assert_allclose(lse32.numpy()[fin], lse64[fin], rtol=0, atol=1e-5)
