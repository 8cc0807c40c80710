"""Paged prefill attention (causal) on the GPU against the float64 oracle.

The reference prefills with FlashInfer's BatchPrefillWithPagedKVCacheWrapper
and causal=True (models/modeling_llama.py:213-283, 775-798).  Cases: fresh
prompts (queries == keys), prompts continuing cached tokens (fewer queries
than keys), more queries than keys (the first see nothing: o = 0, lse =
-inf), ragged batches, GQA groups 1/4/8, head_dim 64/128, page sizes 4/16,
fp32 (1e-5) and bf16 / fp16 (2e-2 rel, 1e-2 abs), few CUs (many chunks and
partial rows), and causal multi-query groups on a cascade's last level."""

import math

import numpy as np
import pytest
import torch

from oracle import attention as oa

pytestmark = pytest.mark.gpu

TOL = {torch.float32: dict(rtol=0.0, atol=1e-5), torch.bfloat16: dict(rtol=2e-2, atol=1e-2),
       torch.float16: dict(rtol=2e-2, atol=1e-2)}


@pytest.fixture(scope="module")
def ws():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    return torch.empty(256 << 20, dtype=torch.uint8, device="cuda")


def _levels(q_lens, kv_lens, page):
    qo, kvp, kvi, lpl = [0], [0], [], []
    nxt = 0
    for nq, nk in zip(q_lens, kv_lens):
        npg = max(1, -(-nk // page))
        kvi.extend(range(nxt, nxt + npg))
        nxt += npg
        kvp.append(len(kvi))
        lpl.append(nk - (npg - 1) * page)
        qo.append(qo[-1] + nq)
    return (qo, kvp, kvi, lpl), nxt


def _check(out, lse, ref_o, ref_lse, dtype):
    np.testing.assert_allclose(out.float().cpu().numpy(), ref_o, **TOL[dtype])
    l = lse.cpu().numpy()
    fin = np.isfinite(ref_lse)
    assert np.array_equal(np.isfinite(l), fin)
    tol = 1e-5 if dtype == torch.float32 else 2e-3
    np.testing.assert_allclose(l[fin], ref_lse[fin], rtol=tol, atol=tol)


CASES = {
    # name: (q_lens, kv_lens, hq, hkv, d, page)
    "fresh_1000": ([1000], [1000], 32, 8, 128, 16),
    "ragged_batch": ([17, 300, 1025], [17, 300, 1025], 32, 8, 128, 16),
    "continue_cached": ([200, 64], [700, 64 + 33], 32, 8, 128, 16),
    "more_queries_than_keys": ([8], [5], 8, 8, 128, 4),
    "g8_page4": ([129, 77], [129, 200], 64, 8, 128, 4),
    "mha_d64": ([96, 31], [96, 31], 8, 8, 64, 16),
    # a long prompt at every storage type, fp32 included (the VALU kernel's long causal path)
    "long_mha_d64": ([1000], [1000], 8, 8, 64, 16),
}


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("case", list(CASES))
@pytest.mark.parametrize("cus", [None, 3])
def test_prefill_wrapper_causal(ws, dtype, case, cus):
    from beam_engine_amd import BatchPrefillWithPagedKVCacheWrapper
    q_lens, kv_lens, hq, hkv, d, page = CASES[case]
    print(f"[case] prefill {case} {dtype} cus={cus}", flush=True)
    (qo, kvp, kvi, lpl), pages = _levels(q_lens, kv_lens, page)
    g = torch.Generator().manual_seed(7)
    s = 1 / math.sqrt(d)
    kv = (torch.randn((pages, 2, page, hkv, d), generator=g) * s).to(dtype)
    q = (torch.randn((qo[-1], hq, d), generator=g) * s).to(dtype)
    w = BatchPrefillWithPagedKVCacheWrapper(ws)
    w._num_cus = cus
    w.plan(torch.tensor(qo, dtype=torch.int32), torch.tensor(kvp, dtype=torch.int32),
           torch.tensor(kvi, dtype=torch.int32), torch.tensor(lpl, dtype=torch.int32), hq, hkv, d, page,
           causal=True, q_data_type=dtype)
    # 16-bit storage at head_dim 128 with 16-token pages streams (on 3 CUs a workgroup may need more
    # segments than its table holds: the tile kernel then); other shapes take the tile / VALU kernels
    if dtype == torch.float32:
        assert w.stats.kernel == "valu"
    elif d == 128 and page % 16 == 0:
        assert w.stats.kernel == "stream" or (cus is not None and w.stats.kernel == "tile")
    else:
        assert w.stats.kernel == "tile"
    out, lse = w.run(q.cuda(), kv.cuda(), return_lse=True)
    torch.cuda.synchronize()
    ref_o, ref_lse = oa.cascade_attention(q, kv, [qo], [kvp], [kvi], [lpl], page, causal=True)
    _check(out, lse, ref_o, ref_lse, dtype)


def test_cascade_causal_last_level(ws):
    """Cascade wrapper with causal=True and multi-query groups on its last
    level: a shared prefix (unmasked) plus per-request causal blocks."""
    from beam_engine_amd import MultiLevelCascadeAttentionWrapper
    print("[case] cascade causal last level", flush=True)
    page, hq, hkv, d = 16, 32, 8, 128
    dtype = torch.bfloat16
    (qo1, kvp1, kvi1, lpl1), p1 = _levels([40, 70], [40, 90], page)
    pre = 300
    npre = -(-pre // page)
    kvi0 = list(range(p1, p1 + npre))
    levels = ([[0, 110], qo1], [[0, npre], kvp1], [kvi0, kvi1], [[pre - (npre - 1) * page], lpl1])
    g = torch.Generator().manual_seed(9)
    s = 1 / math.sqrt(d)
    kv = (torch.randn((p1 + npre, 2, page, hkv, d), generator=g) * s).to(dtype)
    q = (torch.randn((110, hq, d), generator=g) * s).to(dtype)
    w = MultiLevelCascadeAttentionWrapper(2, ws)
    w.plan(*levels, hq, hkv, d, page, causal=True, q_data_type=dtype)
    assert w.stats.kernel == "stream"
    out, lse = w.run(q.cuda(), kv.cuda(), return_lse=True)
    torch.cuda.synchronize()
    ref_o, ref_lse = oa.cascade_attention(q, kv, *levels, page, causal=True)
    _check(out, lse, ref_o, ref_lse, dtype)
