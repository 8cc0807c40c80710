"""GPU checks of the KV-cache kernels (bit-exact against torch indexing) and of
PageTable + BeamState driving them through the reference's fork trace."""

import sys

import numpy as np
import pytest
import torch

from tests.conftest import load_fixtures

pytestmark = pytest.mark.gpu
FX = load_fixtures()


def say(msg):
    print(f"[case] {msg}", flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module", autouse=True)
def need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_append_matches_indexing(dtype):
    say(f"kv append {dtype}")
    from beam_engine_amd import PageTable
    pt = PageTable(3, page_size=16, max_num_pages=64, head_num=8, head_dim=128, device="cuda", store_dtype=dtype)
    g = torch.Generator().manual_seed(1)
    n = 37
    pages = torch.randperm(64, generator=g)[:n].to(torch.int32)
    pos = torch.randint(0, 16, (n,), generator=g, dtype=torch.int32)
    # keys as a strided view of a projection output [N, Hkv, 2*D]
    proj = torch.randn((n, 8, 256), generator=g).to(dtype).cuda()
    k, v = proj[:, :, :128], proj[:, :, 128:]
    ref = pt.kv_cache_at_layer[1].clone()
    ref[pages.long(), 0, pos.long()] = k
    ref[pages.long(), 1, pos.long()] = v
    pt.write_blocks_vectorized(1, pages.cuda(), k, v, pos.cuda())
    torch.cuda.synchronize()
    assert torch.equal(pt.kv_cache_at_layer[1], ref)
    assert torch.count_nonzero(pt.kv_cache_at_layer[0]) == 0 and torch.count_nonzero(pt.kv_cache_at_layer[2]) == 0


def test_append_skips_out_of_range_entries():
    say("kv append out-of-range entries")
    from beam_engine_amd import _lib
    kv = torch.zeros((4, 2, 8, 2, 64), dtype=torch.bfloat16, device="cuda")
    k = torch.ones((3, 2, 64), dtype=torch.bfloat16, device="cuda")
    pages = torch.tensor([1, 9, 2], dtype=torch.int32, device="cuda")
    pos = torch.tensor([0, 0, 8], dtype=torch.int32, device="cuda")      # 9 >= 4 pages, slot 8 >= page 8
    err = torch.zeros(1, dtype=torch.int32, device="cuda")
    L = _lib.load()
    _lib.check(L.be_kv_append(kv.data_ptr(), _lib.BE_BF16, 4, 8, 2, 64, pages.data_ptr(), pos.data_ptr(),
                              k.data_ptr(), 128, 64, k.data_ptr(), 128, 64, 3, err.data_ptr(),
                              _lib.stream_ptr()), "append")
    torch.cuda.synchronize()
    assert int(err) == 2
    assert torch.all(kv[1, :, 0] == 1) and torch.count_nonzero(kv) == 2 * 2 * 64


@pytest.mark.parametrize("dtype,page,heads,dim", [(torch.float32, 8, 2, 64), (torch.bfloat16, 8, 2, 64),
                                                   (torch.bfloat16, 16, 8, 256), (torch.float32, 16, 8, 128)])
def test_batched_page_copy_all_layers(dtype, page, heads, dim):
    """Batched fork copies over every layer; the larger shapes give page planes
    of 64 KB, more than one batch of loads per workgroup."""
    say(f"page copy {dtype} page={page} heads={heads} dim={dim}")
    from beam_engine_amd import PageTable
    pt = PageTable(4, page_size=page, max_num_pages=32, head_num=heads, head_dim=dim, device="cuda",
                   store_dtype=dtype)
    g = torch.Generator().manual_seed(2)
    pt.kv_pool.copy_(torch.randn(pt.kv_pool.shape, generator=g).to(dtype))
    for _ in range(10):
        pt.allocate_block()
    before = pt.kv_pool.clone()
    n1, n2 = 5, page - 1
    with pt.defer_copies():
        a = pt.copy_block(3, n1)
        b = pt.copy_block(7, page)
        c = pt.copy_block(3, 0)
        e = pt.copy_block(9, n2)
    assert (a, b, c, e) == (10, 11, 12, 13)
    torch.cuda.synchronize()
    ref = before.clone()
    ref[:, a, :, :n1] = before[:, 3, :, :n1]
    ref[:, b, :, :page] = before[:, 7, :, :page]
    ref[:, e, :, :n2] = before[:, 9, :, :n2]
    assert torch.equal(pt.kv_pool, ref)


def test_staged_copies_counted_launch_and_graph_replay():
    """The staged fork-copy list: the counted launch copies exactly the
    entries below the device count (the rest of the fixed arrays are stale
    and untouched), eagerly and from one captured launch replayed with two
    different lists; a bad page id is counted, not written."""
    say("staged page copies: counted launch, graph replays")
    from beam_engine_amd import PageTable
    dt = torch.bfloat16
    pt = PageTable(3, page_size=16, max_num_pages=40, head_num=2, head_dim=128, device="cuda", store_dtype=dt)
    g = torch.Generator().manual_seed(9)
    pt.kv_pool.copy_(torch.randn(pt.kv_pool.shape, generator=g).to(dt))
    pt.enable_staged_copies(6)

    def expect(base, copies):
        ref = base.clone()
        for s_, d_, n_ in copies:
            ref[:, d_, :, :n_] = base[:, s_, :, :n_]
        return ref

    # eager: five entries staged, then three -- the arrays keep the stale fourth and fifth
    pt.stage_copies(np.array([[1, 20, 5], [2, 21, 16], [3, 22, 1], [4, 23, 7], [5, 24, 3]]))
    pt.run_staged_copies()
    before = pt.kv_pool.clone()
    cp = [[6, 25, 9], [7, 26, 16], [8, 27, 2]]
    pt.stage_copies(np.array(cp))
    pt.run_staged_copies()
    torch.cuda.synchronize()
    assert torch.equal(pt.kv_pool, expect(before, cp))
    # one captured launch replayed with two lists
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph):
            pt.record_staged_copies()
    torch.cuda.current_stream().wait_stream(side)
    for cp in ([[9, 28, 4], [10, 29, 11]], [[11, 30, 16], [12, 31, 6], [13, 32, 1], [14, 33, 15], [15, 34, 8]]):
        torch.cuda.synchronize()
        before = pt.kv_pool.clone()
        pt.stage_copies(np.array(cp))
        graph.replay()
        pt.consume_staged_copies()
        torch.cuda.synchronize()
        assert torch.equal(pt.kv_pool, expect(before, cp)), cp
    # a source page outside the pool is skipped and counted
    before = pt.kv_pool.clone()
    pt.stage_copies(np.array([[99, 35, 4], [16, 36, 4]]))
    pt.run_staged_copies()
    with pytest.raises(ValueError):
        pt.check_errors()
    assert torch.equal(pt.kv_pool, expect(before, [[16, 36, 4]]))


def test_copy_block_errors():
    from beam_engine_amd import PageTable
    from beam_engine_amd.page_table import PageCopyError
    pt = PageTable(1, page_size=4, max_num_pages=4, head_num=1, head_dim=64, device="cuda")
    with pytest.raises(TypeError):
        pt.copy_block(0, 5)
    with pytest.raises(ValueError):
        pt.copy_block(4, 1)
    for _ in range(4):
        pt.allocate_block()
    with pytest.raises(MemoryError):
        pt.allocate_block()


def test_fork_trace_moves_page_contents():
    """Run the reference's fork trace on a real PageTable: after each fork the
    copied page holds the source's first len slots on every layer."""
    say("fork trace on device")
    from beam_engine_amd import BeamGenerateResult, BeamState, BeamToken, PageTable
    tr = FX["fork_trace"]
    pt = PageTable(2, page_size=tr["page_size"], max_num_pages=tr["max_num_pages"], head_num=2, head_dim=64,
                   device="cuda", store_dtype=torch.bfloat16)
    g = torch.Generator().manual_seed(3)
    pt.kv_pool.copy_(torch.randn(pt.kv_pool.shape, generator=g).to(torch.bfloat16))
    st = BeamState(tr["beam_size"], pt)
    st.add_root_sequence(tr["prompt"])
    for step in tr["steps"]:
        before = pt.kv_pool.clone()
        res = [BeamGenerateResult(c, [BeamToken(t, s) for t, s in ch]) for c, ch in zip(st.candidates, step["select"])]
        st.add_filtered_results(res)
        torch.cuda.synchronize()
        assert [c.trie_node.page_id for c in st.candidates] == [c["page"] for c in step["expect_candidates"]]
        for src, dst, n in step["expect_copies"]:
            assert torch.equal(pt.kv_pool[:, dst, :, :n], before[:, src, :, :n])
        assert list(pt.free_pages) == step.get("expect_free_list", list(pt.free_pages))


@pytest.mark.parametrize("pad", [0, 4])
def test_rope_append_matches_eager_tensor_code(pad):
    """be_rope_qkv_append is bit-identical to the eager HF-style RoPE + append,
    on a contiguous projection (pad 0) and on a row view 8 bytes past a 16-byte
    boundary with a row stride of 4 mod 8 elements (pad 4)."""
    say(f"rope append vs eager pad={pad}")
    from beam_engine_amd import PageTable
    from beam_engine_amd.llama import LlamaConfig, LlamaDecoder
    cfg = LlamaConfig(num_hidden_layers=1, hidden_size=256, num_attention_heads=8, num_key_value_heads=2,
                      head_dim=128, intermediate_size=256, vocab_size=64, max_position_embeddings=2048)
    m = LlamaDecoder(cfg, "cuda", torch.bfloat16, seed=1)
    g = torch.Generator().manual_seed(5)
    n = 37
    full = (torch.randn((n, (8 + 4) * 128 + pad), generator=g) * 2).to(torch.bfloat16).cuda()
    qkv = full[:, pad:]
    pos = torch.randint(0, 2048, (n,), generator=g).cuda()
    pages = torch.randperm(64, generator=g)[:n].to(torch.int32).cuda()
    slots = torch.randint(0, 16, (n,), generator=g, dtype=torch.int32).cuda()
    a = PageTable(1, page_size=16, max_num_pages=64, head_num=2, head_dim=128, device="cuda",
                  store_dtype=torch.bfloat16)
    b = PageTable(1, page_size=16, max_num_pages=64, head_num=2, head_dim=128, device="cuda",
                  store_dtype=torch.bfloat16)
    q_fused = a.write_rope_qkv(0, qkv, 8, pos, m.cos, m.sin, pages, slots)
    q = qkv[:, :1024].unflatten(-1, (8, 128))
    k = qkv[:, 1024:1280].unflatten(-1, (2, 128))
    v = qkv[:, 1280:].unflatten(-1, (2, 128))
    q_ref = m._rope(q, pos)
    b.write_blocks_vectorized(0, pages, m._rope(k, pos), v, slots)
    torch.cuda.synchronize()
    assert torch.equal(q_fused, q_ref)
    assert torch.equal(a.kv_pool, b.kv_pool)


def test_page_table_raises_on_bad_page_ids():
    """A bad page id or slot in write_blocks_vectorized / write_rope_qkv is
    skipped on the device and counted; check_errors then raises ValueError (the
    reference raises ValueError for a page it does not hold,
    page_table.py:150-151).  Good entries are written; the count is cleared."""
    say("page table: bad page ids raise ValueError")
    from beam_engine_amd import PageTable
    pt = PageTable(2, page_size=16, max_num_pages=8, head_num=2, head_dim=64, device="cuda",
                   store_dtype=torch.bfloat16)
    k = torch.ones((3, 2, 64), dtype=torch.bfloat16, device="cuda")
    pages = torch.tensor([1, 8, 2], dtype=torch.int32, device="cuda")          # 8 >= 8 pages
    slots = torch.tensor([0, 0, 3], dtype=torch.int32, device="cuda")
    pt.write_blocks_vectorized(0, pages, k, k, slots)
    with pytest.raises(ValueError, match="outside the pool"):
        pt.check_errors()
    assert torch.all(pt.kv_cache_at_layer[0][1, :, 0] == 1) and torch.all(pt.kv_cache_at_layer[0][2, :, 3] == 1)
    pt.check_errors()                                                            # cleared: no raise
    # a slot past the page and a bad page in the fused RoPE append
    hq, d = 4, 64
    qkv = torch.randn((2, (hq + 4) * d), device="cuda").to(torch.bfloat16)
    cos = torch.ones((32, d), dtype=torch.bfloat16, device="cuda")
    sin = torch.zeros((32, d), dtype=torch.bfloat16, device="cuda")
    pos = torch.tensor([3, 4], dtype=torch.int64, device="cuda")
    pt.write_rope_qkv(1, qkv, hq, pos, cos, sin, torch.tensor([0, -1], dtype=torch.int32, device="cuda"),
                      torch.tensor([16, 1], dtype=torch.int32, device="cuda"))
    with pytest.raises(ValueError):
        pt.check_errors()
    pt.check_errors()
