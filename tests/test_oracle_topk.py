"""Pins the selection oracle (oracle/topk.py): torch.log_softmax / torch.topk on
the CPU for tie-free rows, a brute-force stable sort of the whole pool, the
bfloat16 rounding against torch's conversion, and explicit tie cases."""

import numpy as np
import pytest
import torch

from oracle import topk as ot


def test_bf16_rounding_matches_torch():
    x = np.random.default_rng(0).standard_normal(100000).astype(np.float32) * 37.0
    x[:4] = [0.0, -0.0, 1e-40, 3.3895314e38]
    ours = ot.round_bf16(x)
    ref = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    assert np.array_equal(ours.view(np.uint32), ref.view(np.uint32))


def test_log_softmax_close_to_torch():
    x = np.random.default_rng(1).standard_normal((4, 32000)).astype(np.float32)
    ours = ot.log_softmax_rows(x)
    ref = torch.log_softmax(torch.from_numpy(x), dim=-1).numpy()
    # same formula up to reduction order: at most a couple of float32 ulps
    np.testing.assert_allclose(ours, ref, rtol=0, atol=4e-6)
    # the normaliser: logsumexp of the logp row is zero
    np.testing.assert_allclose(np.log(np.exp(ours.astype(np.float64)).sum(axis=1)), 0.0, atol=1e-5)


def test_row_topk_matches_torch_without_ties():
    rng = np.random.default_rng(2)
    x = rng.permutation(50000).reshape(5, 10000).astype(np.float32)  # distinct values
    v, i = ot.row_topk(x, 8)
    tv, ti = torch.topk(torch.from_numpy(x), 8, dim=-1)
    assert np.array_equal(i, ti.numpy()) and np.array_equal(v, tv.numpy())


def test_row_topk_ties_lower_index_first():
    x = np.array([[1.0, 3.0, 3.0, 2.0, 3.0, 0.5]], dtype=np.float32)
    v, i = ot.row_topk(x, 4)
    assert i.tolist() == [[1, 2, 4, 3]]


def test_select_global_brute_force():
    rng = np.random.default_rng(3)
    for trial in range(20):
        n, k, b = 6, 8, 4
        vals = np.round(rng.standard_normal((n, k)), 1).astype(np.float32)   # many ties
        vals = -np.sort(-vals, axis=1)
        idx = rng.integers(0, 1000, (n, k))
        parents = np.round(rng.standard_normal(n), 1)
        per_row, flat = ot.select_global(parents, vals, idx, b)
        pool = [(float(parents[r]) + float(vals[r, j]), r * k + j, r, int(idx[r, j]))
                for r in range(n) for j in range(k)]
        brute = sorted(pool, key=lambda t: (-t[0], t[1]))[:b]
        exp_rows = [[(tok, sc) for sc, _, rr, tok in brute if rr == r] for r in range(n)]
        assert per_row == exp_rows
        assert flat == [(r, t, s) for r in range(n) for t, s in exp_rows[r]]


def test_decode_k_rule():
    assert ot.decode_k(16, 128256) == 32
    assert ot.decode_k(1, 128256) == 1
    assert ot.decode_k(8, 10) == 10


def test_prefill_select():
    x = np.array([0.1, 2.0, -1.0, 2.0, 0.5, 1.5], dtype=np.float32)
    sel = ot.prefill_select(x, 2)
    assert [t for t, _ in sel] == [1, 3]
    lp = torch.log_softmax(torch.from_numpy(x), -1).numpy()
    assert abs(sel[0][1] - lp[1]) < 1e-6


def test_bf16_logp_rounded_and_ties_by_index():
    x = np.random.default_rng(5).standard_normal((3, 4096)).astype(np.float32)
    xb = ot.round_bf16(x)
    lp = ot.log_softmax_rows(xb, "bfloat16")
    assert np.array_equal(lp, ot.round_bf16(lp))
    v, i = ot.row_topk(lp, 32)
    for r in range(3):
        for j in range(31):
            assert v[r, j] > v[r, j + 1] or (v[r, j] == v[r, j + 1] and i[r, j] < i[r, j + 1])


def _nearest_f32(q):
    """The float32 nearest to the rational q (ties to even), from exact arithmetic."""
    from fractions import Fraction
    f = np.float32(float(q))
    best = None
    for c in (np.nextafter(f, np.float32(-np.inf)), f, np.nextafter(f, np.float32(np.inf))):
        d = abs(Fraction(float(c)) - q)
        if best is None or d < best[0] or (d == best[0] and (int(c.view(np.uint32)) & 1) == 0):
            best = (d, c)
    return best[1]


@pytest.mark.parametrize("temperature", [0.7, 0.9, 1.1, 1.3])
def test_temperature_reciprocal_constant(temperature):
    """Mode "reciprocal" multiplies by fl32(fl64(1 / T)): the exact reciprocal
    of the Python float rounded to double, then to float32 (two roundings, as
    torch forms the constant for a GPU tensor divided by a Python float; the
    GPU tests check torch's device division against it).  At T = 1.1 that is
    0x3F68BA2F, whereas the float division 1.0f / fl32(1.1) gives 0x3F68BA2E --
    a plausible restatement this test rejects."""
    from fractions import Fraction
    want = _nearest_f32(Fraction(float(1 / Fraction(temperature))))
    got = ot.scale_temperature(np.array([1.0], dtype=np.float32), "float32", temperature, "reciprocal")[0]
    assert got.view(np.uint32) == want.view(np.uint32)
    if temperature == 1.1:
        assert int(got.view(np.uint32)) == 0x3F68BA2F
        assert int((np.float32(1) / np.float32(1.1)).view(np.uint32)) == 0x3F68BA2E


@pytest.mark.parametrize("dtype", ["float32", "bfloat16"])
@pytest.mark.parametrize("temperature", [0.7, 0.9, 1.1, 1.3])
def test_temperature_divide_matches_torch_cpu(dtype, temperature):
    """Mode "divide" equals torch's ``logits / T`` on a CPU tensor bit for
    bit (float32 and bfloat16 logits); for float32 logits it differs from mode
    "reciprocal" on a sizeable share of the values, so the two modes are
    distinct arithmetic (after bfloat16 rounding they almost always agree)."""
    tdt = {"float32": torch.float32, "bfloat16": torch.bfloat16}[dtype]
    x = (torch.randn(200000, generator=torch.Generator().manual_seed(7)) * 3).to(tdt)
    ref = (x / temperature).float().numpy()
    ours = ot.scale_temperature(x.float().numpy(), dtype, temperature, "divide")
    assert np.array_equal(ours.view(np.uint32), ref.view(np.uint32))
    if dtype == "float32":
        rec = ot.scale_temperature(x.float().numpy(), dtype, temperature, "reciprocal")
        assert np.mean(rec != ours) > 0.01


def test_temperature_one_is_skipped():
    x = (np.random.default_rng(8).standard_normal(1000) * 3).astype(np.float32)
    for mode in ("reciprocal", "divide"):
        assert np.array_equal(ot.scale_temperature(x, "float32", 1.0, mode), x)
    with pytest.raises(ValueError):
        ot.scale_temperature(x, "float32", 0.5, "bogus")
