"""GPU beam selection (be_beam_topk) bit-exact against the oracle: row top-k
values and indices, and the global top-B parents, tokens and float64 scores."""

import sys

import numpy as np
import pytest
import torch

from oracle import topk as ot

pytestmark = pytest.mark.gpu


def say(msg):
    print(f"[case] {msg}", flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module", autouse=True)
def need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")


DT = {torch.float32: "float32", torch.bfloat16: "bfloat16", torch.float16: "float16"}


def compare(logits, parents, beam, temperature=1.0, mode="reciprocal"):
    from beam_engine_amd import beam_topk, decode_k
    n, v = logits.shape
    k = decode_k(beam, v)
    x = logits.float().numpy()
    logp = ot.log_softmax_rows(x, DT[logits.dtype], temperature, mode)
    vals, idx = ot.row_topk(logp, k)
    _, flat = ot.select_global(parents, vals, idx, beam)
    rv, ri, (par, tok, sc) = beam_topk(logits.cuda(), k, torch.tensor(parents, dtype=torch.float64), beam,
                                       temperature, temperature_mode=mode)
    torch.cuda.synchronize()
    assert np.array_equal(ri.cpu().numpy(), idx), "row indices differ"
    assert np.array_equal(rv.cpu().numpy().view(np.uint32), vals.view(np.uint32)), "row values differ"
    got = list(zip(par.tolist(), tok.tolist(), sc.tolist()))
    assert got == flat


def test_config1_fp32():
    say("topk config 1 [4, 32000] fp32 beam 4")
    g = torch.Generator().manual_seed(1)
    logits = torch.randn((4, 32000), generator=g)
    compare(logits, [0.0, -0.5, -0.7, -1.25], 4)


def test_config4_bf16():
    say("topk config 4 [128, 128256] bf16 beam 16")
    g = torch.Generator().manual_seed(2)
    logits = (torch.randn((128, 128256), generator=g) * 3).to(torch.bfloat16)
    parents = (-torch.rand(128, generator=g, dtype=torch.float64) * 5).tolist()
    # the engine selects per request: 8 requests x 16 rows
    for r in range(8):
        compare(logits[16 * r:16 * (r + 1)], parents[16 * r:16 * (r + 1)], 16)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_ties_and_temperature(dtype):
    say(f"topk ties/temperature {dtype}")
    g = torch.Generator().manual_seed(3)
    logits = torch.randint(-3, 4, (6, 5000), generator=g).to(torch.float32).to(dtype)   # massive ties
    parents = [0.0, 0.0, -1.0, -1.0, -2.0, 0.0]                                        # tied parents too
    compare(logits, parents, 4)
    for t in (0.7, 0.9, 1.1, 1.3):
        compare(logits, parents, 4, temperature=t)
        compare(logits, parents, 4, temperature=t, mode="divide")
    compare(logits, parents, 1)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("temperature", [0.7, 0.9, 1.1, 1.3])
def test_temperature_matches_torch_division(dtype, temperature):
    """The reference scales with ``logits / temperature`` on a GPU tensor
    (beam.py:107, :270).  torch's device division equals the oracle's
    "reciprocal" form bit for bit, and be_beam_topk with that mode selects
    exactly what it selects from torch's divided logits at T = 1; the "divide"
    mode does the same against torch's CPU division."""
    from beam_engine_amd import beam_topk
    say(f"topk temperature {temperature} vs torch division, {dtype}")
    g = torch.Generator().manual_seed(21)
    logits = (torch.randn((16, 50000), generator=g) * 3).to(dtype)
    parents = torch.from_numpy(-np.random.default_rng(21).random(16))
    dev = logits.cuda()
    dev_div = dev / temperature                               # the reference's own expression
    one = (torch.ones(1, device="cuda") / temperature).cpu().numpy()
    torch.cuda.synchronize()
    # torch's device division multiplies by the double reciprocal rounded to float
    assert one.view(np.uint32)[0] == np.float32(1.0 / temperature).view(np.uint32)
    ours = ot.scale_temperature(logits.float().numpy(), DT[dtype], temperature, "reciprocal")
    assert np.array_equal(dev_div.float().cpu().numpy().view(np.uint32), ours.view(np.uint32)), \
        "torch's device division differs from the reciprocal form"
    for mode, pre in (("reciprocal", dev_div), ("divide", (logits / temperature).cuda())):
        a = beam_topk(dev, 32, parents, 16, temperature, temperature_mode=mode)
        b = beam_topk(pre, 32, parents, 16, 1.0)
        torch.cuda.synchronize()
        assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1]), mode
        assert all(torch.equal(x, y) for x, y in zip(a[2], b[2])), mode
        compare(logits, parents.tolist(), 16, temperature, mode)


def test_prefill_single_row_and_small_vocab():
    say("topk prefill row / small vocab")
    from beam_engine_amd import beam_topk
    g = torch.Generator().manual_seed(4)
    row = torch.randn((1, 128256), generator=g).to(torch.bfloat16)
    rv, ri = beam_topk(row.cuda(), 32)
    sel = ot.prefill_select(row[0].float().numpy(), 16, "bfloat16")
    assert [int(t) for t in ri[0, :16].tolist()] == [t for t, _ in sel]
    assert rv[0, :16].tolist() == [s for _, s in sel]
    small = torch.randn((3, 7), generator=g)
    compare(small, [0.0, -1.0, -2.0], 3)


def test_batched_requests_in_one_call():
    say("topk batched requests")
    from beam_engine_amd import beam_topk
    g = torch.Generator().manual_seed(6)
    rows = [16, 16, 5, 16]
    logits = (torch.randn((sum(rows), 50000), generator=g) * 2).to(torch.bfloat16)
    parents = (-torch.rand(sum(rows), generator=g, dtype=torch.float64) * 3)
    _, _, (par, tok, sc) = beam_topk(logits.cuda(), 32, parents, 16, request_rows=rows)
    torch.cuda.synchronize()
    par, tok, sc = par.tolist(), tok.tolist(), sc.tolist()
    b = 0
    for q, r in enumerate(rows):
        x = logits[b:b + r].float().numpy()
        _, _, _, _, flat = ot.beam_step(x, parents[b:b + r].tolist(), 16, "bfloat16")
        got = [(p - b, t, s) for p, t, s in zip(par[q * 16:(q + 1) * 16], tok[q * 16:(q + 1) * 16],
                                                 sc[q * 16:(q + 1) * 16]) if p >= 0]
        assert got == flat, f"request {q}"
        b += r


@pytest.mark.parametrize("case", ["strided_best", "chunk_best", "constant", "two_levels", "near_ties_bf16",
                                  "few_finite", "large_magnitude", "mixed_offsets_f16", "tiny_values_bf16",
                                  "zero_runs_bf16"])
def test_segment_select_paths(case):
    """Logits that stress the per-segment selection: the best values all in
    one thread's stride (a single thread maximum among them), constant rows
    (every key tied: more candidates than threads), two value levels, bf16
    logp values tied after rounding (runs of equal logp from different
    logits, reordered by index), rows with fewer finite logits than k (the
    rest of the k are -inf, lowest indices first), and 16-bit logits of
    large magnitude (maxima far from 0, rows whose halves sit hundreds
    apart: float64 rescaling between threads, waves and segments)."""
    say(f"topk segment paths {case}")
    g = torch.Generator().manual_seed(11)
    v = 128256
    if case == "strided_best":
        x = torch.randn((4, v), generator=g)
        x[:, ::256] += 8.0                       # every 256th token (one thread's stride per segment) is best
        logits = x.to(torch.bfloat16)
    elif case == "chunk_best":
        x = torch.randn((4, v), generator=g)
        pos = torch.arange(v)
        x[:, (pos % 2048) < 8] += 8.0            # one thread's 16-byte chunks of every segment are best
        logits = x.to(torch.bfloat16)
    elif case == "constant":
        logits = torch.full((3, v), 0.5).to(torch.bfloat16)
    elif case == "two_levels":
        x = torch.zeros((3, v))
        x[:, torch.randperm(v, generator=g)[:40]] = 1.0
        logits = x.to(torch.float16)
    elif case == "few_finite":
        x = torch.full((2, v), float("-inf"))
        x[0, torch.randperm(v, generator=g)[:10]] = torch.randn(10, generator=g)
        x[1, 70000:70005] = 1.0
        logits = x.to(torch.bfloat16)
    elif case == "large_magnitude":
        x = torch.randn((3, v), generator=g)
        x[0] *= 400.0                            # maxima far above 300
        x[1] -= 900.0                            # every value far below -300
        x[2] = x[2] * 3.0 + 310.0
        logits = x.to(torch.bfloat16)
    elif case == "tiny_values_bf16":
        # zeros and values below 2^-22 in magnitude scattered among N(0, 1): the
        # waves holding them sum against their own max, beside waves with a larger one
        x = torch.randn((4, v), generator=g)
        pos = torch.randperm(v, generator=g)[:300]
        x[:, pos[:100]] = 0.0
        x[:, pos[100:200]] = 3.0e-8
        x[:, pos[200:]] = -1.0e-9
        x[1, :2048] = 0.0                        # whole waves of zeros
        logits = x.to(torch.bfloat16)
    elif case == "zero_runs_bf16":
        x = torch.zeros((3, v))
        x[:, torch.randperm(v, generator=g)[:40]] = 1.0
        x[1] = torch.randn(v, generator=g) * 0.25
        x[1, 50000:90000] = 0.0
        x[2, :8016] = -2.0
        logits = x.to(torch.bfloat16)
    elif case == "mixed_offsets_f16":
        x = torch.randn((3, v), generator=g) * 2.0
        x[:, : v // 2] += 305.0                  # half the segments hundreds above the rest
        x[1, v // 2:] += 296.0
        logits = x.to(torch.float16)
    else:
        logits = (torch.randn((4, v), generator=g) * 0.05).to(torch.bfloat16)
    parents = [0.0, -0.25, -0.5, -0.75][: logits.shape[0]]
    compare(logits, parents, 16)
    compare(logits, parents, 1)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_unaligned_row_stride(dtype):
    """Rows of a wider device tensor (row stride vocab + 3): segment starts
    are not 16-byte aligned, so the kernels take their one-load-per-logit
    path; the result is the same selection."""
    from beam_engine_amd import beam_topk, decode_k
    say(f"topk unaligned row stride {dtype}")
    g = torch.Generator().manual_seed(5)
    n, v, beam = 5, 32003, 4
    wide = torch.randn((n, v + 3), generator=g).to(dtype)
    logits = wide[:, :v]
    k = decode_k(beam, v)
    logp = ot.log_softmax_rows(logits.float().numpy(), DT[dtype], 1.0)
    vals, idx = ot.row_topk(logp, k)
    parents = [0.0, -0.5, -1.0, -0.25, -2.0]
    _, flat = ot.select_global(parents, vals, idx, beam)
    dev = wide.cuda()[:, :v]
    assert dev.stride(0) == v + 3
    rv, ri, (par, tok, sc) = beam_topk(dev, k, torch.tensor(parents, dtype=torch.float64), beam)
    torch.cuda.synchronize()
    assert np.array_equal(ri.cpu().numpy(), idx)
    assert np.array_equal(rv.cpu().numpy().view(np.uint32), vals.view(np.uint32))
    assert list(zip(par.tolist(), tok.tolist(), sc.tolist())) == flat


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_masked_vocabulary_range(dtype):
    """-inf over a range covering whole segments (a masked part of the
    vocabulary): those segments add nothing to the row's exp-sum and the
    selection equals the oracle's over the unmasked logits."""
    say(f"topk masked vocabulary range {dtype}")
    g = torch.Generator().manual_seed(13)
    x = torch.randn((3, 128256), generator=g)
    x[:, 20000:60000] = float("-inf")
    x[1, :100] = float("-inf")
    compare(x.to(dtype), [0.0, -0.5, -1.0], 4)


def test_workspace_shared_across_paths_and_empty_requests():
    """One workspace across calls that take the two-kernel 16-bit path (its
    per-request arrival counters must be back at zero after every call) and
    the three-kernel path (fp32 logits, or a pool above 512 entries), with
    requests that have no rows (their selections are empty: parent -1)."""
    from beam_engine_amd import beam_topk
    from beam_engine_amd.selection import TopkWorkspace
    say("topk shared workspace, empty requests, both paths")
    g = torch.Generator().manual_seed(12)
    ws = TopkWorkspace(torch.device("cuda"))
    cases = [([16, 0, 5, 16], torch.bfloat16, 16), ([3, 3], torch.float32, 4), ([0, 7, 0], torch.float16, 8),
             ([32, 32], torch.bfloat16, 32), ([16, 0, 5, 16], torch.bfloat16, 16), ([1] * 40, torch.bfloat16, 1)]
    for rows, dtype, beam in cases:
        k = 2 * beam if beam > 1 else 1
        logits = (torch.randn((sum(rows), 20000), generator=g) * 2).to(dtype)
        parents = -torch.rand(sum(rows), generator=g, dtype=torch.float64) * 3
        for _ in range(2):
            _, _, (par, tok, sc) = beam_topk(logits.cuda(), k, parents, beam, request_rows=rows, workspace=ws)
            torch.cuda.synchronize()
            par, tok, sc = par.tolist(), tok.tolist(), sc.tolist()
            b = 0
            for q, r in enumerate(rows):
                got = [(p - b, t, s) for p, t, s in zip(par[q * beam:(q + 1) * beam], tok[q * beam:(q + 1) * beam],
                                                         sc[q * beam:(q + 1) * beam]) if p >= 0]
                if r == 0:
                    assert got == [] and par[q * beam:(q + 1) * beam] == [-1] * beam, f"{rows} request {q}"
                else:
                    x = logits[b:b + r].float().numpy()
                    _, _, _, _, flat = ot.beam_step(x, parents[b:b + r].tolist(), beam, DT[dtype])
                    assert got == flat, f"{rows} {dtype} request {q}"
                b += r


def test_pool_bound_and_full_ranking():
    """The pool's sample bound (the beam-th best of each row's first entries):
    a request whose best entries all sit in one row (more than 32 entries reach
    the bound, so every entry is ranked), a request of 48 rows (too many to
    sample: every entry is ranked), rows with one far outlier (their keys span
    more than 256 values: two radix passes), and identical rows under equal
    parents (totals tied across rows, ordered by pool position)."""
    from beam_engine_amd import beam_topk
    say("topk pool bound, full ranking, wide key range, tied totals")
    g = torch.Generator().manual_seed(31)
    rows = [16, 48, 8]
    v = 50000
    x = torch.randn((sum(rows), v), generator=g)
    x[16:64, 997::4999] = 50.0                     # one outlier every 4999 logits
    x[64:72] = x[64]                               # identical rows
    logits = x.to(torch.bfloat16)
    parents = -torch.rand(sum(rows), generator=g, dtype=torch.float64) * 3
    parents[:16] = -100.0
    parents[3] = 0.0                               # one dominant row
    parents[64:72] = -1.0
    for beam in (16, 4):
        k = 2 * beam
        _, _, (par, tok, sc) = beam_topk(logits.cuda(), k, parents, beam, request_rows=rows)
        torch.cuda.synchronize()
        par, tok, sc = par.tolist(), tok.tolist(), sc.tolist()
        b = 0
        for q, r in enumerate(rows):
            got = [(p - b, t, s) for p, t, s in zip(par[q * beam:(q + 1) * beam], tok[q * beam:(q + 1) * beam],
                                                     sc[q * beam:(q + 1) * beam]) if p >= 0]
            _, _, _, _, flat = ot.beam_step(logits[b:b + r].float().numpy(), parents[b:b + r].tolist(), beam,
                                            "bfloat16")
            assert got == flat, f"beam {beam} request {q}"
            b += r
