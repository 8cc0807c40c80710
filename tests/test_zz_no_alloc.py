"""be_beam_topk_noalloc (static device scratch, no workspace argument, no
allocation) through the C ABI against be_beam_topk with a caller workspace:
identical row top-k and selection outputs on two calls in a row, the second on
a smaller input, and a clear capacity error beyond the static scratch."""

import ctypes
import sys

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def say(msg):
    print(f"[case] {msg}", flush=True)
    sys.stdout.flush()


def _outs(n, k, n_req, beam, dev):
    return (torch.empty((n, k), dtype=torch.float32, device=dev), torch.empty((n, k), dtype=torch.int32, device=dev),
            torch.empty(n_req * beam, dtype=torch.int32, device=dev),
            torch.empty(n_req * beam, dtype=torch.int32, device=dev),
            torch.empty(n_req * beam, dtype=torch.float64, device=dev))


def _call(lib, noalloc, logits, temperature, k, parents, beam, rows):
    from beam_engine_amd import _lib
    n, v = logits.shape
    dev = logits.device
    n_req = len(rows)
    ptr = torch.tensor(np.concatenate([[0], np.cumsum(rows)]).astype(np.int32), device=dev)
    rv, ri, op, ot, os_ = _outs(n, k, n_req, beam, dev)
    common = (logits.data_ptr(), _lib.dtype_code(logits.dtype), n, v, logits.stride(0), ctypes.c_double(temperature),
              _lib.BE_TEMP_RECIPROCAL, k, parents.data_ptr(), beam, n_req, ptr.data_ptr(), max(rows), rv.data_ptr(),
              ri.data_ptr(), op.data_ptr(), ot.data_ptr(), os_.data_ptr())
    if noalloc:
        rc = lib.be_beam_topk_noalloc(*common, _lib.stream_ptr(dev))
    else:
        need = lib.be_beam_topk_workspace_bytes(n, v, k)
        ws = torch.zeros(need, dtype=torch.uint8, device=dev)
        rc = lib.be_beam_topk(*common, ws.data_ptr(), ws.numel(), _lib.stream_ptr(dev))
    _lib.check(rc, "top-k")
    torch.cuda.synchronize()
    return rv, ri, op, ot, os_


def test_noalloc_topk_matches_workspace_entry_point():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    from beam_engine_amd import _lib
    lib = _lib.load()
    g = torch.Generator().manual_seed(31)
    cases = [
        ("bf16 [32, 128256], k 32, beam 16, 2 requests, T 1", (torch.randn((32, 128256), generator=g) * 3)
         .to(torch.bfloat16), 1.0, 32, 16, [16, 16]),
        ("fp32 [5, 32000], k 8, beam 4, 1 request, T 0.7", torch.randn((5, 32000), generator=g), 0.7, 8, 4, [5]),
    ]
    for name, logits, temp, k, beam, rows in cases:
        say(f"no-alloc top-k: {name}")
        x = logits.cuda()
        parents = torch.from_numpy(-np.random.default_rng(len(rows)).random(x.shape[0])).cuda()
        a = _call(lib, True, x, temp, k, parents, beam, rows)
        b = _call(lib, False, x, temp, k, parents, beam, rows)
        for u, w_ in zip(a, b):
            assert torch.equal(u, w_), name
        assert int((a[2] >= 0).sum()) == beam * len(rows)
    say("no-alloc top-k: capacity error beyond the static scratch")
    big = torch.zeros((2048, 128256), dtype=torch.bfloat16, device="cuda")
    parents = torch.zeros(2048, dtype=torch.float64, device="cuda")
    rv, ri, op, ot, os_ = _outs(2048, 32, 1, 16, "cuda")
    rc = lib.be_beam_topk_noalloc(big.data_ptr(), _lib.BE_BF16, 2048, 128256, 128256, ctypes.c_double(1.0),
                                  _lib.BE_TEMP_RECIPROCAL, 32, parents.data_ptr(), 0, 1, None, 2048, rv.data_ptr(),
                                  ri.data_ptr(), op.data_ptr(), ot.data_ptr(), os_.data_ptr(), _lib.stream_ptr())
    assert rc == _lib.BE_ERR_CAPACITY
    assert b"static" in lib.be_last_error()
