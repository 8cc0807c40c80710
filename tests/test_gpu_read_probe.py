"""``be_read_probe``, the measurement kernel behind ``bench.py --workload
read-ns``: every chunk of the rows it is given must be read exactly once.  The
XOR of its per-workgroup folds equals the XOR of the bytes those rows cover
(as uint32 words): a chunk skipped, or read twice, changes it.  Bit-exact."""

import sys

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def say(msg):
    print(f"[case] {msg}", flush=True)
    sys.stdout.flush()


def probe(buf, rows, inner, istr, ostr, row_bytes, grid):
    from beam_engine_amd import _lib
    lib = _lib.load()
    sink = torch.zeros(grid, dtype=torch.int32, device=buf.device)
    stream = torch.cuda.current_stream()
    _lib.check(lib.be_read_probe(buf.data_ptr(), rows, inner, istr, ostr, row_bytes, sink.data_ptr(), grid,
                                 stream.cuda_stream), "read probe")
    torch.cuda.synchronize()
    return np.bitwise_xor.reduce(sink.cpu().numpy().view(np.uint32))


def expected(host, rows, inner, istr, ostr, row_bytes):
    words = []
    for r in range(rows):
        off = (r % inner) * istr + (r // inner) * ostr
        words.append(host[off: off + row_bytes].view(np.uint32))
    return np.bitwise_xor.reduce(np.concatenate(words)) if words else np.uint32(0)


@pytest.mark.parametrize("grid", [1, 7, 256, 4096])
def test_read_probe_per_kv_head_layer(grid):
    P, page, hkv, d = 24, 16, 8, 128
    say(f"read probe per KV head P={P} grid={grid}")
    rng = np.random.default_rng(grid)
    host = rng.integers(0, 256, size=P * 2 * page * hkv * d * 2, dtype=np.uint8)
    buf = torch.from_numpy(host.copy()).cuda()
    rows, inner, istr, ostr, rb = P * 2 * page * hkv, P * 2 * page, hkv * d * 2, d * 2, d * 2
    got = probe(buf, rows, inner, istr, ostr, rb, grid)
    assert got == np.bitwise_xor.reduce(host.view(np.uint32))
    assert got == expected(host, rows, inner, istr, ostr, rb)


@pytest.mark.parametrize("rows,row_bytes,grid", [(1, 16, 3), (333, 256, 5), (4099, 64, 64), (5, 32768, 2)])
def test_read_probe_partial_and_ragged(rows, row_bytes, grid):
    say(f"read probe contiguous rows={rows} row_bytes={row_bytes} grid={grid}")
    rng = np.random.default_rng(rows)
    host = rng.integers(0, 256, size=rows * row_bytes + 4096, dtype=np.uint8)
    buf = torch.from_numpy(host.copy()).cuda()
    got = probe(buf, rows, rows, row_bytes, 0, row_bytes, grid)
    assert got == expected(host, rows, rows, row_bytes, 0, row_bytes)
    # a strided subset: 3 outer blocks of rows // 3 rows at twice the row pitch
    if rows >= 3:
        inner = rows // 3
        got = probe(buf, 3 * inner, inner, row_bytes, inner * row_bytes // 2 // 16 * 16, row_bytes, grid)
        assert got == expected(host, 3 * inner, inner, row_bytes, inner * row_bytes // 2 // 16 * 16, row_bytes)


def test_read_probe_rejects_bad_rows():
    from beam_engine_amd import _lib
    lib = _lib.load()
    buf = torch.zeros(4096, dtype=torch.uint8, device="cuda")
    sink = torch.zeros(4, dtype=torch.int32, device="cuda")
    for rb in (0, 24, 48, 65536):
        rc = lib.be_read_probe(buf.data_ptr(), 1, 1, 16, 0, rb, sink.data_ptr(), 4, None)
        assert rc != 0, rb
