"""GPU parity of the HIP attention path against the CPU oracle.

Tolerances: fp32 storage within 1e-5 max-abs of
the float64 oracle; bf16/fp16 storage within 2e-2 relative / 1e-2 absolute of
the oracle evaluated on the same (rounded) inputs.  Each case prints its name
before touching the GPU."""

import math
import sys

import numpy as np
import pytest
import torch

from oracle import attention as oa
from tests.conftest import load_fixtures

pytestmark = pytest.mark.gpu
FX = load_fixtures()

TOL = {torch.float32: dict(rtol=0.0, atol=1e-5), torch.bfloat16: dict(rtol=2e-2, atol=1e-2),
       torch.float16: dict(rtol=2e-2, atol=1e-2)}


def say(msg):
    print(f"[case] {msg}", flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def ws():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    return torch.empty(128 << 20, dtype=torch.uint8, device="cuda")


def make_pool(num_pages, page, hkv, d, dtype, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    kv = torch.randn((num_pages, 2, page, hkv, d), generator=g, dtype=torch.float32) * scale
    return kv.to(dtype)


def make_q(n, hq, d, dtype, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn((n, hq, d), generator=g, dtype=torch.float32) * scale).to(dtype)


def run_cascade(ws, q, kv, levels, page, force_valu=False, return_lse=True, fused_merge=False, tile_kernel=False,
                num_cus=None, no_regs=False, no_wide=False, no_wide256=False):
    from beam_engine_amd import MultiLevelCascadeAttentionWrapper
    w = MultiLevelCascadeAttentionWrapper(len(levels[0]), ws)
    w._no_regs = no_regs
    w._no_wide = no_wide
    w._no_wide256 = no_wide256
    w._force_valu = force_valu
    w._fused_merge = fused_merge
    w._tile_kernel = tile_kernel
    w._num_cus = num_cus
    hq, d = q.shape[1], q.shape[2]
    w.plan(levels[0], levels[1], levels[2], levels[3], hq, kv.shape[3], d, page, causal=True,
           pos_encoding_mode="NONE", q_data_type=q.dtype)
    out = w.run(q.cuda(), kv.cuda(), return_lse=return_lse)
    torch.cuda.synchronize()
    return out, w


def check(out, lse, ref_o, ref_lse, dtype):
    o = out.float().cpu().numpy()
    np.testing.assert_allclose(o, ref_o, **TOL[dtype])
    if lse is not None:
        l = lse.cpu().numpy()
        fin = np.isfinite(ref_lse)
        assert np.array_equal(np.isfinite(l), fin)
        np.testing.assert_allclose(l[fin], ref_lse[fin], rtol=1e-5 if dtype == torch.float32 else 2e-3,
                                   atol=1e-5 if dtype == torch.float32 else 2e-3)


def tree_levels(name):
    e = FX["trees"][name]["expected"]
    return e["qo_indptr"], e["kv_indptr"], e["kv_indices"], e["last_page_len"]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("name", ["cascade_md", "swapped", "uneven"])
@pytest.mark.parametrize("d", [64, 128])
def test_reference_trees(ws, dtype, name, d):
    say(f"reference tree {name} d={d} {dtype}")
    page, hq, hkv = 4, 8, 2
    levels = tree_levels(name)
    n = levels[0][0][-1]
    kv = make_pool(20, page, hkv, d, dtype, 1)
    q = make_q(n, hq, d, dtype, 2)
    (out, lse), _ = run_cascade(ws, q, kv, levels, page)
    ref_o, ref_lse = oa.cascade_attention(q, kv, *levels, page, d ** -0.5)
    check(out, lse, ref_o, ref_lse, dtype)


@pytest.mark.parametrize("fused_merge", [False, True])
@pytest.mark.parametrize("force_valu", [False, True])
def test_mfma_and_valu_agree_on_bf16(ws, force_valu, fused_merge):
    say(f"mfma/valu bf16 force_valu={force_valu} fused_merge={fused_merge}")
    levels = tree_levels("cascade_md")
    kv = make_pool(20, 4, 2, 128, torch.bfloat16, 3)
    q = make_q(8, 8, 128, torch.bfloat16, 4)
    (out, lse), w = run_cascade(ws, q, kv, levels, 4, force_valu=force_valu, fused_merge=fused_merge)
    # page 4: the streaming kernel takes page sizes that are multiples of 16
    assert w.stats.kernel == ("valu" if force_valu else "tile")
    ref_o, ref_lse = oa.cascade_attention(q, kv, *levels, 4, 128 ** -0.5)
    check(out, lse, ref_o, ref_lse, torch.bfloat16)


def shared_prefix_levels(n_req, beams, prefix, suffixes, page):
    """Two levels: per-request prefix pages, per-beam suffix pages."""
    pp = -(-prefix // page)
    pages = 0
    qo0, kvp0, kvi0, lpl0 = [0], [0], [], []
    qo1, kvp1, kvi1, lpl1 = [0], [0], [], []
    for r in range(n_req):
        kvi0.extend(range(pages, pages + pp))
        pages += pp
        kvp0.append(len(kvi0))
        lpl0.append(prefix - (pp - 1) * page)
        qo0.append(qo0[-1] + beams)
        for b in range(beams):
            s = suffixes[r * beams + b]
            sp = max(1, -(-s // page))
            kvi1.extend(range(pages, pages + sp))
            pages += sp
            kvp1.append(len(kvi1))
            lpl1.append(s - (sp - 1) * page)
            qo1.append(qo1[-1] + 1)
    return ([qo0, qo1], [kvp0, kvp1], [kvi0, kvi1], [lpl0, lpl1]), pages


def test_config1_fp32(ws):
    """Config 1: B=4, prefix 512, suffix 32, 8/8 heads, D=64, fp32, page 16."""
    say("config 1 fp32 cascade")
    levels, pages = shared_prefix_levels(1, 4, 512, [32] * 4, 16)
    kv = make_pool(pages, 16, 8, 64, torch.float32, 5)
    q = make_q(4, 8, 64, torch.float32, 6)
    (out, lse), w = run_cascade(ws, q, kv, levels, 16)
    ref_o, ref_lse = oa.cascade_attention(q, kv, *levels, 16, 64 ** -0.5)
    check(out, lse, ref_o, ref_lse, torch.float32)
    assert np.abs(out.cpu().numpy() - ref_o).max() <= 1e-5


def test_config2_bf16_and_flat(ws):
    """Config 2: 4 req x 8 beams, 32/8 heads, D=128, bf16, prefix 2048, suffix 128."""
    say("config 2 bf16 cascade + flat")
    from beam_engine_amd import BatchDecodeWithPagedKVCacheWrapper
    levels, pages = shared_prefix_levels(4, 8, 2048, [128] * 32, 16)
    s = 1 / math.sqrt(128)
    kv = make_pool(pages, 16, 8, 128, torch.bfloat16, 7, s)
    q = make_q(32, 32, 128, torch.bfloat16, 8, s)
    (out, lse), w = run_cascade(ws, q, kv, levels, 16)
    assert w.stats.kv_bytes == 50331648
    ref_o, ref_lse = oa.cascade_attention(q, kv, *levels, 16, 128 ** -0.5)
    check(out, lse, ref_o, ref_lse, torch.bfloat16)
    # flat over the same pages: one group per query with prefix + suffix pages
    kvp, kvi, lpl = [0], [], []
    for i in range(32):
        r = i // 8
        kvi.extend(levels[2][0][levels[1][0][r]:levels[1][0][r + 1]])
        kvi.extend(levels[2][1][levels[1][1][i]:levels[1][1][i + 1]])
        kvp.append(len(kvi))
        lpl.append(levels[3][1][i])
    f = BatchDecodeWithPagedKVCacheWrapper(ws)
    f.plan(kvp, kvi, lpl, 32, 8, 128, 16, q_data_type=torch.bfloat16)
    fo, fl = f.run(q.cuda(), kv.cuda(), return_lse=True)
    torch.cuda.synchronize()
    check(fo, fl, ref_o, ref_lse, torch.bfloat16)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_run_py_shape_fixture(ws, dtype):
    """run.py:18-41 shapes: 7 queries, 512 shared pages + ragged unique pages, 64/8 heads."""
    say(f"run.py shape {dtype}")
    fx = FX["run_py_shape"]
    page, hq, hkv, d = fx["page_size"], fx["num_qo_heads"], fx["num_kv_heads"], fx["head_dim"]
    shared = fx["shared_kv_num_pages"]
    uptr = fx["unique_kv_page_indptr"]
    levels = ([[0, 7], list(range(8))], [[0, shared], uptr],
              [list(range(shared)), list(range(shared, shared + uptr[-1]))],
              [[page], fx["unique_kv_last_page_len"]])
    kv = make_pool(shared + uptr[-1], page, hkv, d, dtype, 9, 0.3)
    q = make_q(7, hq, d, dtype, 10, 0.3)
    (out, lse), _ = run_cascade(ws, q, kv, levels, page)
    ref_o, ref_lse = oa.cascade_attention(q, kv, *levels, page, d ** -0.5)
    check(out, lse, ref_o, ref_lse, dtype)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_ragged_edges(ws, dtype):
    """Token counts around block edges, empty groups, a query without groups."""
    say(f"ragged edges {dtype}")
    page, hq, hkv, d = 16, 16, 4, 128
    lens = [1, 15, 16, 17, 31, 32, 33, 127, 128, 129, 0, 300, 5]
    kvp, kvi, lpl = [0], [], []
    pages = 0
    for L in lens:
        npg = max(1, -(-L // page))
        kvi.extend(range(pages, pages + npg))
        pages += npg
        kvp.append(len(kvi))
        lpl.append(L - (npg - 1) * page)
    n = len(lens) + 1      # the last query belongs to no group
    levels = ([list(range(len(lens) + 1))], [kvp], [kvi], [lpl])
    kv = make_pool(pages, page, hkv, d, dtype, 11)
    q = make_q(n, hq, d, dtype, 12)
    from beam_engine_amd import MultiLevelCascadeAttentionWrapper
    w = MultiLevelCascadeAttentionWrapper(1, ws)
    w._plan_levels(*levels, hq, hkv, d, page, None, dtype, num_queries=n)
    out, lse = w.run(q.cuda(), kv.cuda(), return_lse=True)
    torch.cuda.synchronize()
    ref_o, ref_lse = oa.cascade_attention(q[:len(lens)], kv, *levels, page, d ** -0.5)
    ref_o = np.concatenate([ref_o, np.zeros((1, hq, d))])
    ref_lse = np.concatenate([ref_lse, np.full((1, hq), -np.inf)])
    check(out, lse, ref_o, ref_lse, dtype)
    assert np.all(out[10].float().cpu().numpy() == 0)     # empty group


def test_long_prefix_split_k_and_strided_q(ws):
    """One 8192-token prefix shared by 16 queries (many split-K chunks), q a strided view."""
    say("long prefix split-K strided q")
    page, hq, hkv, d = 16, 32, 8, 128
    levels, pages = shared_prefix_levels(1, 16, 8192, [40] * 16, page)
    kv = make_pool(pages, page, hkv, d, torch.bfloat16, 13, 0.1)
    big = make_q(16, hq * 2, d, torch.bfloat16, 14, 0.1)
    q = big.cuda()[:, ::2]                                   # stride(1) = 2*D
    (out, lse), w = run_cascade(ws, q, kv, levels, page)
    assert w.stats.num_items > 8
    ref_o, ref_lse = oa.cascade_attention(q.cpu(), kv, *levels, page, d ** -0.5)
    check(out, lse, ref_o, ref_lse, torch.bfloat16)


def test_deep_tree_config3_shape(ws):
    """Config 3 tree (root 4096, fanout 2/4/4 with 256/128/64, leaf suffix 32), 32/8 heads, bf16:
    every leaf attends its root-to-leaf path; cascade levels equal flat attention."""
    say("config 3 tree as cascade")
    page, hq, hkv, d = 16, 32, 8, 128
    from beam_engine_amd import BatchDecodeWithPagedKVCacheWrapper
    next_page = [0]

    def alloc(tokens):
        n = tokens // page
        out = list(range(next_page[0], next_page[0] + n))
        next_page[0] += n
        return out
    root = alloc(4096)
    l1 = [alloc(256) for _ in range(2)]
    l2 = [alloc(128) for _ in range(8)]
    l3 = [alloc(64) + alloc(32) for _ in range(32)]
    levels = ([[0, 32], [0, 16, 32], list(range(0, 33, 4)), list(range(33))],
              [[0, len(root)], [0, 16, 32], list(range(0, 8 * 8 + 1, 8)), list(range(0, 32 * 6 + 1, 6))],
              [root, sum(l1, []), sum(l2, []), sum(l3, [])],
              [[16], [16, 16], [16] * 8, [16] * 32])
    kv = make_pool(next_page[0], page, hkv, d, torch.bfloat16, 15, 1 / math.sqrt(128))
    q = make_q(32, hq, d, torch.bfloat16, 16, 1 / math.sqrt(128))
    (out, lse), w = run_cascade(ws, q, kv, levels, page)
    assert w.stats.kv_bytes == 35651584
    ref_o, ref_lse = oa.cascade_attention(q, kv, *levels, page, d ** -0.5)
    check(out, lse, ref_o, ref_lse, torch.bfloat16)


def test_merge_state(ws):
    say("merge_state")
    from beam_engine_amd import merge_state
    g = torch.Generator().manual_seed(17)
    va, vb = torch.randn(5, 8, 128, generator=g), torch.randn(5, 8, 128, generator=g)
    sa, sb = torch.randn(5, 8, generator=g), torch.randn(5, 8, generator=g)
    sa[0, :] = -math.inf
    sb[0, :2] = -math.inf
    v, s = merge_state(va.cuda(), sa.cuda(), vb.cuda(), sb.cuda())
    ro, rl = oa.merge_states([va.numpy(), vb.numpy()], [sa.numpy(), sb.numpy()])
    np.testing.assert_allclose(v.cpu().numpy(), ro, rtol=1e-5, atol=1e-6)
    got = s.cpu().numpy()
    assert np.array_equal(np.isfinite(got), np.isfinite(rl))
    np.testing.assert_allclose(got[np.isfinite(rl)], rl[np.isfinite(rl)], rtol=1e-6, atol=1e-6)


@pytest.mark.parametrize("fused_merge", [False, True])
def test_repeated_runs_of_one_plan(ws, fused_merge):
    """One plan, many runs (as over the layers of a step): every run matches
    the oracle, so the fused-merge arrival counters return to zero each run."""
    say(f"repeated runs fused_merge={fused_merge}")
    from beam_engine_amd import MultiLevelCascadeAttentionWrapper
    levels, pages = shared_prefix_levels(2, 8, 1024, [64] * 16, 16)
    kv = make_pool(pages, 16, 8, 128, torch.bfloat16, 21, 0.2).cuda()
    w = MultiLevelCascadeAttentionWrapper(2, ws)
    w._fused_merge = fused_merge
    w.plan(*levels, 32, 8, 128, 16, q_data_type=torch.bfloat16)
    # merge entries: per query (tile kernel) or per (query, KV head) (streaming kernel)
    assert w.stats.num_merge == (16 if fused_merge else 16 * 8)
    for rep in range(6):
        q = make_q(16, 32, 128, torch.bfloat16, 100 + rep, 0.2)
        out, lse = w.run(q.cuda(), kv, return_lse=True)
        torch.cuda.synchronize()
        ref_o, ref_lse = oa.cascade_attention(q, kv.cpu(), *levels, 16, 128 ** -0.5)
        check(out, lse, ref_o, ref_lse, torch.bfloat16)


def config3_levels(page):
    next_page = [0]

    def alloc(tokens):
        n = tokens // page
        out = list(range(next_page[0], next_page[0] + n))
        next_page[0] += n
        return out
    root = alloc(4096)
    l1 = [alloc(256) for _ in range(2)]
    l2 = [alloc(128) for _ in range(8)]
    l3 = [alloc(64) + alloc(32) for _ in range(32)]
    levels = ([[0, 32], [0, 16, 32], list(range(0, 33, 4)), list(range(33))],
              [[0, len(root)], [0, 16, 32], list(range(0, 8 * 8 + 1, 8)), list(range(0, 32 * 6 + 1, 6))],
              [root, sum(l1, []), sum(l2, []), sum(l3, [])],
              [[16], [16, 16], [16] * 8, [16] * 32])
    return levels, next_page[0]


@pytest.mark.parametrize("shape", ["config2", "config3", "ragged_suffix"])
@pytest.mark.parametrize("kernel,num_cus", [("tile", None), ("stream", None), ("stream", 4), ("stream", 7),
                                            ("stream", 61), ("stream-dma", 4), ("stream-dma", 7)])
def test_stream_and_tile_kernels(ws, shape, kernel, num_cus):
    """Both MFMA kernels against the oracle; small CU counts make every
    streaming workgroup walk many segments and cut work items mid-way.
    Launches with long workgroup runs take the register-staged loop, others
    the direct-load loop; "stream-dma" keeps the latter."""
    say(f"{kernel} kernel {shape} cus={num_cus}")
    page, hq, hkv, d = 16, 32, 8, 128
    s = 1 / math.sqrt(128)
    if shape == "config2":
        levels, pages = shared_prefix_levels(4, 8, 2048, [128] * 32, page)
    elif shape == "config3":
        levels, pages = config3_levels(page)
    else:
        g = torch.Generator().manual_seed(31)
        suf = torch.randint(1, 300, (24,), generator=g).tolist()
        levels, pages = shared_prefix_levels(3, 8, 1000, suf, page)
    n = levels[0][0][-1] if shape != "config3" else 32
    kv = make_pool(pages, page, hkv, d, torch.bfloat16, 41, s)
    q = make_q(n, hq, d, torch.bfloat16, 42, s)
    (out, lse), w = run_cascade(ws, q, kv, levels, page, tile_kernel=(kernel == "tile"), num_cus=num_cus,
                                no_regs=(kernel == "stream-dma"))
    assert w.stats.kernel == kernel.split("-")[0]
    if kernel != "tile":
        info = w._info
        wg = w._plan_dev[info.off_wg: info.off_wg + 4 * info.num_wg].view(-1, 4).cpu()
        wide = bool(((wg[:, 3] == 4) | (wg[:, 3] == 5) | (wg[:, 3] == 6)).any())
        assert info.stream_loop == (1 if kernel == "stream" and int(wg[:, 2].max()) >= 8 and not wide else 0)
    ref_o, ref_lse = oa.cascade_attention(q, kv, *levels, page, d ** -0.5)
    check(out, lse, ref_o, ref_lse, torch.bfloat16)


@pytest.mark.parametrize("case", ["rows72", "rows100", "rows128", "rows256_g8", "rows512_g8", "rows296_g8", "mixed"])
@pytest.mark.parametrize("cus", [None, 4, 7, 13])
def test_stream_wide_roles(ws, case, cus):
    """Wide wave roles (32 rows per wave: 128-row segments of long groups of
    more than 64 rows, or 256-row segments, every wave over all tokens, when
    every such group has at least 256 rows) against the oracle and against the
    plans without them, with ragged token counts (partial last tiles, split
    segments), row counts that leave row groups empty (296 rows: a 40-row
    remainder segment), and shorter groups in the same launch.  They apply
    when every workgroup's run is long (few CUs here); with all 256 CUs the
    same shapes take 64-row segments."""
    say(f"wide roles {case} cus={cus}")
    page, hkv, d = 16, 8, 128
    hq = 64 if case.endswith("g8") else 32
    g = hq // hkv
    s = 1 / math.sqrt(d)
    gen = torch.Generator().manual_seed(sum(map(ord, case)))
    if case == "mixed":
        # requests of 10 / 32 / 18 beams (40 / 128 / 72 rows) over ragged prefixes
        beams, prefixes = [10, 32, 18], [2000, 3100, 1613]
    else:
        beams = [int(case[4:].split("_")[0]) // g] * 2
        prefixes = [3000, 1777]
    # shared prefix per request, private ragged suffix per beam, all in one pool
    pages = 0
    lv0 = [[0], [0], [], []]
    lv1 = [[0], [0], [], []]
    for r, (b, pre) in enumerate(zip(beams, prefixes)):
        pp = -(-pre // page)
        lv0[2].extend(range(pages, pages + pp)); pages += pp
        lv0[1].append(len(lv0[2])); lv0[3].append(pre - (pp - 1) * page); lv0[0].append(lv0[0][-1] + b)
        for _ in range(b):
            sfx = int(torch.randint(1, 200, (1,), generator=gen))
            sp = -(-sfx // page)
            lv1[2].extend(range(pages, pages + sp)); pages += sp
            lv1[1].append(len(lv1[2])); lv1[3].append(sfx - (sp - 1) * page); lv1[0].append(lv1[0][-1] + 1)
    levels = tuple([lv0[i], lv1[i]] for i in range(4))
    n = lv0[0][-1]
    kv = make_pool(pages, page, hkv, d, torch.bfloat16, 51, s)
    q = make_q(n, hq, d, torch.bfloat16, 52, s)
    (out, lse), w = run_cascade(ws, q, kv, levels, page, num_cus=cus)
    info = w._info
    wg = w._plan_dev[info.off_wg: info.off_wg + 4 * info.num_wg].view(-1, 4).cpu()
    tiles64 = sum(-(-p // 64) * -(-b * g // 64) * hkv for b, p in zip(beams, prefixes))
    expect = any(b * g > 64 for b in beams) and tiles64 >= 64 * info.num_wg
    w256 = expect and all(b * g >= 256 for b in beams if b * g > 64)
    if w.stats.kernel != "stream":
        # more segments than a workgroup's table holds (512 rows of 1-query suffix
        # groups over 4 CUs): the planner falls back to the tile kernel
        assert cus is not None and cus <= 4
        expect = w256 = False
    assert bool((wg[:, 3] == 5).any()) == (expect and not w256)
    assert bool((wg[:, 3] == 6).any()) == w256
    ref_o, ref_lse = oa.cascade_attention(q, kv, *levels, page, d ** -0.5)
    check(out, lse, ref_o, ref_lse, torch.bfloat16)
    (out2, lse2), _ = run_cascade(ws, q, kv, levels, page, num_cus=cus, no_wide=True)
    torch.testing.assert_close(out.float(), out2.float(), rtol=2e-2, atol=1e-2)
    if w256:
        (out3, lse3), w3 = run_cascade(ws, q, kv, levels, page, num_cus=cus, no_wide256=True)
        if w3.stats.kernel == "stream":
            i3 = w3._info
            wg3 = w3._plan_dev[i3.off_wg: i3.off_wg + 4 * i3.num_wg].view(-1, 4).cpu()
            assert (wg3[:, 3] == 5).any() and not (wg3[:, 3] == 6).any()
        else:
            # 128-row segments need more of them per workgroup than 256-row ones:
            # on 4 CUs that plan can exceed the table where the 256-row plan fits
            assert cus is not None and cus <= 4
        torch.testing.assert_close(out.float(), out3.float(), rtol=2e-2, atol=1e-2)
        # the 256-row roles through the direct-load loop (class 7) instead of registers
        (out4, lse4), w4 = run_cascade(ws, q, kv, levels, page, num_cus=cus, no_regs=True)
        i4 = w4._info
        wg4 = w4._plan_dev[i4.off_wg: i4.off_wg + 4 * i4.num_wg].view(-1, 4).cpu()
        assert (wg4[:, 3] == 7).any() and not (wg4[:, 3] == 6).any()
        check(out4, lse4, ref_o, ref_lse, torch.bfloat16)
        torch.testing.assert_close(out.float(), out4.float(), rtol=2e-2, atol=1e-2)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_stream_kernel_flat_long_paths(ws, dtype):
    """Flat decode (one group per query) with paths longer than a workgroup's
    share: queries split across workgroups are merged from slots."""
    say(f"stream flat long paths {dtype}")
    from beam_engine_amd import BatchDecodeWithPagedKVCacheWrapper
    page, hq, hkv, d = 16, 64, 8, 128
    lens = [3000, 17, 1, 64, 65, 2048, 129, 700]
    kvp, kvi, lpl, pages = [0], [], [], 0
    for L in lens:
        npg = -(-L // page)
        kvi.extend(range(pages, pages + npg))
        pages += npg
        kvp.append(len(kvi))
        lpl.append(L - (npg - 1) * page)
    kv = make_pool(pages, page, hkv, d, dtype, 43, 0.2)
    q = make_q(len(lens), hq, d, dtype, 44, 0.2)
    f = BatchDecodeWithPagedKVCacheWrapper(ws)
    f._num_cus = 13
    f.plan(kvp, kvi, lpl, hq, hkv, d, page, q_data_type=dtype)
    assert f.stats.kernel == "stream"
    out, lse = f.run(q.cuda(), kv.cuda(), return_lse=True)
    torch.cuda.synchronize()
    levels = ([list(range(len(lens) + 1))], [kvp], [kvi], [lpl])
    ref_o, ref_lse = oa.cascade_attention(q, kv, *levels, page, d ** -0.5)
    check(out, lse, ref_o, ref_lse, dtype)


def trie_levels(n_req, beams, prefix, page, seed, depth=2, max_tail=48, shared=True):
    """A request prefix shared by its beams, then `depth` levels of short groups: mostly
    single queries of 1..max_tail tokens, and (shared=True) a few groups of 2-4 beams — the
    shape of a beam trie that re-converges every step."""
    rng = np.random.default_rng(seed)
    nq = n_req * beams
    nxt = [0]

    def alloc(n):
        npg = -(-n // page)
        out = list(range(nxt[0], nxt[0] + npg))
        nxt[0] += npg
        return out, n - (npg - 1) * page
    qo, kvp, kvi, lpl = [[0]], [[0]], [[]], [[]]
    for r in range(n_req):
        pg, last = alloc(prefix)
        qo[0].append(qo[0][-1] + beams); kvi[0] += pg; kvp[0].append(len(kvi[0])); lpl[0].append(last)
    for lv in range(depth):
        q, p, i, l = [0], [0], [], []
        while q[-1] < nq:
            size = int(rng.integers(2, 5)) if shared and rng.random() < 0.15 else 1
            size = min(size, nq - q[-1])
            pg, last = alloc(int(rng.integers(1, max_tail + 1)))
            q.append(q[-1] + size); i += pg; p.append(len(i)); l.append(last)
        qo.append(q); kvp.append(p); kvi.append(i); lpl.append(l)
    return (qo, kvp, kvi, lpl), nxt[0], nq


@pytest.mark.parametrize("case", ["bf16_p16", "f16_p16", "bf16_p32", "bf16_g8", "bf16_g16", "bf16_deep",
                                  "bf16_mixed"])
@pytest.mark.parametrize("tails,cus", [("role", 7), ("role", 61), ("role", None), ("merge", 7), ("merge", 61),
                                       ("merge", None), ("off", 7)])
def test_stream_tail_pass_on_trie_shapes(ws, case, tails, cus):
    """Short groups attended as 16-token tail chunks — by tail-role workgroups
    of the persistent kernel ("role"), or by the tail-and-merge kernel
    ("merge") — or, with tails off, in the persistent kernel's tiles, against
    the oracle on beam-trie shapes (each plan run twice).  In the merge kernel the device's CU count
    gives few records per CU (several waves per record); "mixed" has groups on
    both sides of the tail threshold, so records with and without tail chunks
    share workgroups (61 CUs: two waves per record)."""
    say(f"tail pass {case} tails={tails} cus={cus}")
    dtype = torch.float16 if case.startswith("f16") else torch.bfloat16
    page = 32 if case.endswith("p32") else 16
    hq, hkv = {"bf16_g8": (64, 8), "bf16_g16": (64, 4)}.get(case, (32, 8))
    depth = 5 if case == "bf16_deep" else 2
    d = 128
    levels, pages, nq = trie_levels(3, 8, 300, page, seed=len(case) + 7 * depth, depth=depth,
                                    max_tail=200 if case == "bf16_mixed" else 48)
    s = 1 / math.sqrt(d)
    kv = make_pool(pages, page, hkv, d, dtype, 51, s)
    q = make_q(nq, hq, d, dtype, 52, s)
    from beam_engine_amd import MultiLevelCascadeAttentionWrapper
    w = MultiLevelCascadeAttentionWrapper(len(levels[0]), ws)
    w._no_tail = tails == "off"
    w._tail_role = tails == "role"
    w._num_cus = cus
    w.plan(*levels, hq, hkv, d, page, q_data_type=dtype)
    st = w.stats
    assert st.kernel == "stream"
    assert (st.num_tails > 0) == (tails != "off")
    assert (w._info.num_tail_items > 0) == (tails == "role")
    ref_o, ref_lse = oa.cascade_attention(q, kv, *levels, page, d ** -0.5)
    qd, kvd = q.cuda(), kv.cuda()
    for _ in range(2):
        out, lse = w.run(qd, kvd, return_lse=True)
        torch.cuda.synchronize()
        check(out, lse, ref_o, ref_lse, dtype)


@pytest.mark.parametrize("cus", [1, 5, None])
def test_stream_tail_role_without_streamed_groups(ws, cus):
    """Every group short enough for tail chunks, tail role on: every workgroup
    takes the tail role (no segments), down to a single one."""
    say(f"tail role only, cus={cus}")
    page, hq, hkv, d = 16, 32, 8, 128
    rng = np.random.default_rng(11)
    nq = 24
    levels = ([], [], [], [])
    pg = 0
    for _ in range(3):
        qo, kvp, kvi, lpl = [0], [0], [], []
        for _q in range(nq):
            n = int(rng.integers(1, 49))
            npg = -(-n // page)
            kvi += list(range(pg, pg + npg)); pg += npg
            kvp.append(len(kvi)); lpl.append(n - (npg - 1) * page); qo.append(qo[-1] + 1)
        for i, x in enumerate((qo, kvp, kvi, lpl)):
            levels[i].append(x)
    s = 1 / math.sqrt(d)
    kv = make_pool(pg, page, hkv, d, torch.bfloat16, 53, s)
    q = make_q(nq, hq, d, torch.bfloat16, 54, s)
    from beam_engine_amd import MultiLevelCascadeAttentionWrapper
    w = MultiLevelCascadeAttentionWrapper(3, ws)
    w._num_cus = cus
    w._tail_role = True
    w.plan(*levels, hq, hkv, d, page, q_data_type=torch.bfloat16)
    assert w.stats.kernel == "stream" and w.stats.num_items == 0
    assert w._info.num_tail_items >= nq * hkv
    out, lse = w.run(q.cuda(), kv.cuda(), return_lse=True)
    torch.cuda.synchronize()
    ref_o, ref_lse = oa.cascade_attention(q, kv, *levels, page, d ** -0.5)
    check(out, lse, ref_o, ref_lse, torch.bfloat16)


@pytest.mark.parametrize("case", ["trees", "ns", "g8_ragged", "tree_c3", "keyless"])
def test_row_block_kernel(ws, case):
    """The merge-free row-block kernel (BE_PLAN_ROWS) against the float64
    oracle: the reference's trees at page 16 (scaled), the north-star shape
    (queries subset), GQA 8 with ragged suffixes, the config-3 tree, and a
    query without any keys (o = 0, lse = -inf)."""
    say(f"row-block kernel {case}")
    from beam_engine_amd.workloads import BUILDERS, shared_prefix
    if case == "trees":
        for name in ("cascade_md", "swapped", "uneven"):
            e = FX["trees"][name]["expected"]
            levels = (e["qo_indptr"], e["kv_indptr"], e["kv_indices"], e["last_page_len"])
            npages = max(max(l) for l in e["kv_indices"] if l) + 1
            # page 16 with each fixture page's tokens kept (last_page_len scaled by 4)
            lv = (levels[0], levels[1], levels[2], [[min(16, 4 * x) for x in l] for l in levels[3]])
            kv = make_pool(npages, 16, 2, 128, torch.bfloat16, 31, 128 ** -0.5)
            q = make_q(levels[0][0][-1], 8, 128, torch.bfloat16, 32, 128 ** -0.5)
            from beam_engine_amd import MultiLevelCascadeAttentionWrapper
            w = MultiLevelCascadeAttentionWrapper(len(lv[0]), ws)
            w._rows = True
            w.plan(*lv, 8, 2, 128, 16, q_data_type=torch.bfloat16)
            assert w.stats.kernel == "rows"
            out, lse = w.run(q.cuda(), kv.cuda(), return_lse=True)
            torch.cuda.synchronize()
            ref_o, ref_lse = oa.cascade_attention(q, kv, *lv, 16, 128 ** -0.5)
            check(out, lse, ref_o, ref_lse, torch.bfloat16)
        return
    if case == "keyless":
        levels = ([[0, 2, 3]], [[0, 2, 2]], [[0, 1]], [[16, 0]])
        kv = make_pool(4, 16, 8, 128, torch.bfloat16, 33, 128 ** -0.5)
        q = make_q(3, 32, 128, torch.bfloat16, 34, 128 ** -0.5)
        from beam_engine_amd import MultiLevelCascadeAttentionWrapper
        w = MultiLevelCascadeAttentionWrapper(1, ws)
        w._rows = True
        w.plan(*levels, 32, 8, 128, 16, q_data_type=torch.bfloat16)
        out, lse = w.run(q.cuda(), kv.cuda(), return_lse=True)
        torch.cuda.synchronize()
        ref_o, ref_lse = oa.cascade_attention(q, kv, *levels, 16, 128 ** -0.5)
        check(out, lse, ref_o, ref_lse, torch.bfloat16)
        assert torch.all(out[2] == 0) and torch.all(torch.isinf(lse[2]))
        return
    wl = {"ns": lambda: BUILDERS["ns"](), "tree_c3": lambda: BUILDERS["c3"](),
          "g8_ragged": lambda: shared_prefix("g8", 2, 8, 320, list(range(1, 17)), 64, 8, 128)}[case]()
    kv = make_pool(wl.num_pages, wl.page, wl.hkv, wl.d, torch.bfloat16, 35, wl.d ** -0.5)
    q = make_q(wl.num_queries, wl.hq, wl.d, torch.bfloat16, 36, wl.d ** -0.5)
    from beam_engine_amd import MultiLevelCascadeAttentionWrapper
    w = MultiLevelCascadeAttentionWrapper(len(wl.levels[0]), ws)
    w._rows = True
    w.plan(*wl.levels, wl.hq, wl.hkv, wl.d, wl.page, q_data_type=torch.bfloat16)
    assert w.stats.kernel == "rows"
    out, lse = w.run(q.cuda(), kv.cuda(), return_lse=True)
    torch.cuda.synchronize()
    sub = sorted({0, 1, wl.num_queries // 3, wl.num_queries // 2, wl.num_queries - 1})
    kvp, kvi, lpl = wl.flat
    ref_o, ref_lse = oa.paged_attention(q[sub], kv, [0] + list(np.cumsum([kvp[i + 1] - kvp[i] for i in sub])),
                                        [p for i in sub for p in kvi[kvp[i]:kvp[i + 1]]], [lpl[i] for i in sub],
                                        wl.page, wl.d ** -0.5)
    check(out[sub], lse[sub], ref_o, ref_lse, torch.bfloat16)
