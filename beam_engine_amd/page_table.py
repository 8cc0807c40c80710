"""Paged KV cache: drop-in for the reference's ``PageTable`` (src/beam_engine/page_table.py).

Same constructor, attributes and methods.  MI355X-first differences:

* All layers live in one HBM allocation ``kv_pool`` of shape
  ``[L, P, 2, page_size, Hkv, D]``; ``kv_cache_at_layer[l]`` is the
  contiguous per-layer view with the reference's layout (page_table.py:62-72).
  A fork copy of every layer is then one kernel launch (``be_page_copy``).
* The allocator is native (``be_page_pool``): the same FIFO free list order,
  O(1) allocate and free, shared with the native beam trie so that a decode
  step's page bookkeeping needs no Python.  ``free_pages`` and
  ``allocated_pages`` are read-only snapshots of it.
* Pages carry a reference count: ``allocate_block`` sets it to 1,
  ``share_block`` adds a holder, ``free_block`` drops one and returns the page
  to the free list at zero.  With one holder per page (the reference's trie)
  this is exactly the reference's allocate / free behaviour.
* ``write_blocks_vectorized`` calls the HIP append kernel instead of
  FlashInfer's ``append_paged_kv_cache``.
* ``copy_block`` can defer the data copy (``defer_copies()`` context) so that
  all forks of a decode step are copied in a single launch; page ids are
  allocated immediately, in the reference's order.
"""

from __future__ import annotations

import contextlib
import ctypes
import logging
from collections import deque
from typing import List, Optional, Tuple

import numpy as np
import torch

from . import _lib

logger = logging.getLogger(__name__)


class PageCopyError(ValueError, TypeError):
    """Bad ``copy_block`` arguments.  The reference raises a bare string there
    (page_table.py:97-100), which Python 3 turns into a TypeError; this error
    is both a ValueError and a TypeError so either handler catches it."""


class PageTable:
    def __init__(self, layer_num: int, page_size: int = 8, max_num_pages: int = 1024, head_num: int = 32,
                 head_dim: int = 128, v_head_dim: Optional[int] = None, device: torch.device = None,
                 store_dtype: torch.dtype = torch.float16):
        if v_head_dim is not None and v_head_dim != head_dim:
            raise ValueError("the paged layout stores K and V with one head_dim")
        self.layer_num = layer_num
        self.page_size = page_size
        self.max_num_pages = max_num_pages
        self.head_num = head_num
        self.head_dim = head_dim
        self.v_head_dim = v_head_dim or head_dim
        self.device = torch.device(device) if device is not None else torch.device("cuda")
        self.store_dtype = store_dtype

        lib = _lib.load()
        self._lib = lib
        self._pool = lib.be_pages_create(int(max_num_pages))
        if not self._pool:
            _lib.check(_lib.BE_ERR_INVALID, "page pool")
        self._page_out = ctypes.c_int32(0)
        self._pending: List[Tuple[int, int, int]] = []
        self._copy_host = self._copy_dev = self._copy_ev = None     # fork-copy lists' staging
        self._defer = 0
        # staged fork copies (stage_copies): a device list [count, src[m], dst[m], len[m]]
        # and its pinned host twin, run by one counted launch (run_staged_copies),
        # which a decode-step graph can hold
        self._staged_dev = self._staged_host = None
        self._staged_max = 0
        self._staged_pending = False
        self._staged_external = False   # the list's buffers are a caller's, who uploads them
        self._staged_dirty = False      # the pinned list is newer than the device list
        self.stage_copies_enabled = False

        self.kv_pool = torch.zeros((layer_num, max_num_pages, 2, page_size, head_num, head_dim),
                                   dtype=store_dtype, device=self.device)
        self.kv_cache_at_layer: List[torch.Tensor] = [self.kv_pool[l] for l in range(layer_num)]
        self.layer_stride_bytes = self.kv_pool.stride(0) * self.kv_pool.element_size()
        # device count of append / copy entries the kernels skipped for naming a
        # page, slot or position outside the pool (read by check_errors)
        self._err = torch.zeros(1, dtype=torch.int32, device=self.device)
        self._err_host = torch.zeros(1, dtype=torch.int32, pin_memory=self.device.type == "cuda")
        self._err_np = self._err_host.numpy()     # its numpy view (a cheap read after each synchronisation)
        logger.info("Initialized PageTable: %d layers, %d pages of size %d", layer_num, max_num_pages, page_size)

    # ------------------------------------------------------------ allocator
    def __del__(self):
        pool, self._pool = getattr(self, "_pool", None), None
        if pool:
            self._lib.be_pages_destroy(pool)

    @property
    def free_pages(self) -> deque:
        """The free list, oldest page first (a snapshot)."""
        n = self._lib.be_pages_num_free(self._pool)
        out = np.zeros(max(n, 1), np.int32)
        self._lib.be_pages_free_list(self._pool, out.ctypes.data, n)
        return deque(out[:n].tolist())

    @property
    def allocated_pages(self) -> set:
        """Pages with at least one holder (a snapshot)."""
        free = set(self.free_pages)
        return {p for p in range(self.max_num_pages) if p not in free}

    def allocate_block(self) -> int:
        """Pop the oldest free page (page_table.py:77-94)."""
        rc = self._lib.be_pages_allocate(self._pool, ctypes.byref(self._page_out))
        if rc == _lib.BE_ERR_CAPACITY:
            raise MemoryError("No free pages available")
        _lib.check(rc, "allocate_block")
        return int(self._page_out.value)

    def share_block(self, page_idx: int) -> int:
        """Add a holder to an allocated page; returns the new count."""
        cnt = ctypes.c_int32(0)
        _lib.check(self._lib.be_pages_share(self._pool, int(page_idx), ctypes.byref(cnt)), "share_block")
        return int(cnt.value)

    def ref_count(self, page_idx: int) -> int:
        return int(self._lib.be_pages_ref_count(self._pool, int(page_idx)))

    def free_block(self, page_idx: int) -> None:
        """Drop one holder; at zero the page goes to the back of the free list
        (page_table.py:110-124).  Freeing an unallocated page only warns."""
        state = ctypes.c_int32(0)
        _lib.check(self._lib.be_pages_release(self._pool, int(page_idx), ctypes.byref(state)), "free_block")
        if state.value < 0:
            logger.warning("Page %s is not allocated", page_idx)

    def reserve_block(self, page_idx: int) -> int:
        """Take one specific free page out of the free list (e.g. the last one,
        as a scratch slot) without changing the FIFO order of the others."""
        _lib.check(self._lib.be_pages_reserve(self._pool, int(page_idx)), "reserve_block")
        return page_idx

    def num_free_pages(self) -> int:
        return int(self._lib.be_pages_num_free(self._pool))

    # ------------------------------------------------------------ device errors
    def stage_errors(self) -> None:
        """Queue a copy of the device error count to the host on the current
        stream; ``raise_staged_errors`` reads it after the caller's next
        synchronisation (the decode step's selection), costing no extra wait."""
        self._err_host.copy_(self._err, non_blocking=True)

    def raise_staged_errors(self) -> None:
        """Raise ValueError if the staged count is non-zero (the reference
        raises ValueError for a write to a page it does not hold,
        page_table.py:150-151); the device count is cleared first."""
        bad = int(self._err_np[0])
        if bad:
            self._err.zero_()
            self._err_host.zero_()
            raise ValueError(f"{bad} KV append / copy entries named a page, slot or position outside the pool "
                             f"({self.max_num_pages} pages of {self.page_size} slots) and were not written")

    def check_errors(self) -> None:
        """Synchronise the stream and raise ValueError if any append or copy
        since the last check skipped an entry (see ``raise_staged_errors``)."""
        self.stage_errors()
        torch.cuda.current_stream(self.device).synchronize()
        self.raise_staged_errors()

    # ------------------------------------------------------------ copies
    def copy_block(self, page_idx: int, length: int) -> int:
        """Allocate a page and copy the first ``length`` slots of K and V of
        ``page_idx`` into it on every layer (page_table.py:96-106)."""
        if length > self.page_size or length < 0:
            raise PageCopyError("length cannot be larger than page size")
        if page_idx < 0 or page_idx >= self.max_num_pages:
            raise PageCopyError("page idx out of bound")
        new_page = self.allocate_block()
        self._pending.append((page_idx, new_page, length))
        if not self._defer:
            self.flush_copies()
        return new_page

    @contextlib.contextmanager
    def defer_copies(self):
        """Collect copy_block data copies and issue them in one launch on exit."""
        self._defer += 1
        try:
            yield self
        finally:
            self._defer -= 1
            if not self._defer:
                self.flush_copies()

    def flush_copies(self) -> int:
        """Issue every pending fork copy in one be_page_copy launch."""
        if not self._pending:
            return 0
        todo, self._pending = self._pending, []
        return self.copy_pages(np.asarray(todo, dtype=np.int32))

    def copy_pages(self, copies: np.ndarray) -> int:
        """Fork copies ``[n, 3]`` (source page, new page, tokens) in one
        be_page_copy launch, now."""
        todo = copies
        n = len(todo)
        if n == 0:
            return 0
        if self.device.type == "cuda":
            # pinned staging, reused once the previous flush's copy has run
            if self._copy_host is None or self._copy_host.shape[1] < n:
                cap = max(256, 2 * n)
                self._copy_host = torch.empty((3, cap), dtype=torch.int32, pin_memory=True)
                self._copy_dev = torch.empty((3, cap), dtype=torch.int32, device=self.device)
                self._copy_ev = None
            if self._copy_ev is not None:
                self._copy_ev.synchronize()
            self._copy_host.numpy()[:, :n] = np.asarray(todo, dtype=np.int32).T
            dev = self._copy_dev[:, :n]
            dev.copy_(self._copy_host[:, :n], non_blocking=True)
            self._copy_ev = torch.cuda.Event()
            self._copy_ev.record()
        else:
            dev = torch.from_numpy(np.ascontiguousarray(np.asarray(todo, dtype=np.int32).T))
        lib = _lib.load()
        rc = lib.be_page_copy(self.kv_pool.data_ptr(), self.layer_stride_bytes, self.layer_num,
                              _lib.dtype_code(self.store_dtype), self.max_num_pages, self.page_size,
                              self.head_num, self.head_dim, dev[0].data_ptr(), dev[1].data_ptr(),
                              dev[2].data_ptr(), len(todo), self._err.data_ptr(), _lib.stream_ptr(self.device))
        _lib.check(rc, "page copy")
        return len(todo)

    # ------------------------------------------------------------ staged copies
    def enable_staged_copies(self, max_copies: int, dev: Optional[torch.Tensor] = None,
                             host: Optional[torch.Tensor] = None) -> None:
        """From now on ``stage_copies`` takes the fork copies of a trie update:
        their list goes to a fixed device buffer, and ``run_staged_copies``
        (eager) or a captured ``record_staged_copies`` launch (a graph replay)
        performs them before anything reads the pages.  ``dev`` / ``host``
        (int32, ``1 + 3 * max_copies`` words, the host one pinned): buffers of
        the caller, who uploads the host list with the rest of a step's data
        and then calls ``staged_uploaded``; ``upload_staged`` uploads it alone."""
        if self.device.type != "cuda":
            raise ValueError("staged copies need a HIP device")
        if (dev is None) != (host is None):
            raise ValueError("give both the device and the pinned host list, or neither")
        if dev is not None:
            words = 1 + 3 * int(max_copies)
            if dev.dtype != torch.int32 or host.dtype != torch.int32 or dev.numel() < words or host.numel() < words:
                raise ValueError(f"staged-copy buffers must be int32 with {words} words")
            self.run_staged_copies()
            self._staged_max = int(max_copies)
            self._staged_dev, self._staged_host = dev, host
            self._staged_host.zero_()
            self._staged_dev.zero_()
            self._staged_external = True
            self._staged_dirty = False
        elif self._staged_dev is None or self._staged_max < max_copies:
            self._staged_max = int(max_copies)
            self._staged_dev = torch.zeros(1 + 3 * self._staged_max, dtype=torch.int32, device=self.device)
            self._staged_host = torch.zeros(1 + 3 * self._staged_max, dtype=torch.int32, pin_memory=True)
            self._staged_external = False
        self.stage_copies_enabled = True

    def stage_copies(self, copies: np.ndarray) -> None:
        """Write a step's fork copies ``[n, 3]`` (source page, new page, tokens)
        into the staged list (one host-to-device copy, stream-ordered).  The
        pinned twin is rewritten only after the stream has passed the previous
        upload: callers stage once per decode step, after the step's
        synchronising selection.  More copies than the list holds run now."""
        n = len(copies)
        if self._staged_pending:
            self.run_staged_copies()           # an earlier list that no launch consumed yet
        if n > self._staged_max:
            self.copy_pages(copies)
            n = 0
        h = self._staged_host.numpy()
        if n == 0 and h[0] == 0:
            return                             # the device list already holds no copies
        m = self._staged_max
        h[0] = n
        if n:
            c = np.asarray(copies, dtype=np.int32)
            h[1:1 + n] = c[:, 0]
            h[1 + m:1 + m + n] = c[:, 1]
            h[1 + 2 * m:1 + 2 * m + n] = c[:, 2]
        if self._staged_external:
            self._staged_dirty = True          # the caller's step upload carries it
        else:
            self._staged_dev[: 1 + 3 * m].copy_(self._staged_host[: 1 + 3 * m], non_blocking=True)
        self._staged_pending = n > 0

    def staged_uploaded(self) -> None:
        """The caller's step upload copied the pinned list to the device list."""
        self._staged_dirty = False

    def upload_staged(self) -> None:
        """Upload the pinned list alone if it is newer than the device list."""
        if self._staged_dirty:
            m = self._staged_max
            self._staged_dev[: 1 + 3 * m].copy_(self._staged_host[: 1 + 3 * m], non_blocking=True)
            self._staged_dirty = False

    def record_staged_copies(self) -> None:
        """Launch the counted copy of the staged list (inside a graph capture,
        or eagerly): entries below the device count are copied."""
        lib = _lib.load()
        if not torch.cuda.is_current_stream_capturing():
            self.upload_staged()
        d = self._staged_dev
        m = self._staged_max
        base = d.data_ptr()
        rc = lib.be_page_copy_counted(self.kv_pool.data_ptr(), self.layer_stride_bytes, self.layer_num,
                                      _lib.dtype_code(self.store_dtype), self.max_num_pages, self.page_size,
                                      self.head_num, self.head_dim, base + 4, base + 4 * (1 + m),
                                      base + 4 * (1 + 2 * m), base, m, self._err.data_ptr(),
                                      _lib.stream_ptr(self.device))
        _lib.check(rc, "staged page copy")

    def consume_staged_copies(self) -> None:
        """A graph replay holding the counted launch ran the staged list."""
        self._staged_pending = False

    def run_staged_copies(self) -> None:
        """Perform a staged list that no graph replay consumed (eager path)."""
        if self._staged_pending:
            self.record_staged_copies()
            self._staged_pending = False

    # ------------------------------------------------------------ writes
    def write_block(self, layer: int, page_idx: int, key: torch.Tensor, value: torch.Tensor, index: int) -> None:
        """Prefill write of ``key``/``value`` ``[n, Hkv, D]`` at slots
        index..index+n of one page (page_table.py:126-165)."""
        assert key.shape == value.shape
        assert key.shape[0] + index <= self.page_size, \
            f"Cannot fit {key.shape[0]} tokens at index {index} in page size {self.page_size}"
        if layer >= self.layer_num:
            raise ValueError(f"Layer {layer} out of range (max: {self.layer_num - 1})")
        if self.ref_count(page_idx) == 0:
            raise ValueError(f"Page {page_idx} is not allocated")
        if index > self.page_size:
            raise ValueError(f"Index {index} exceeds page size {self.page_size}")
        n = key.shape[0]
        if n > 0:
            self.kv_cache_at_layer[layer][page_idx, 0, index:index + n] = key
            self.kv_cache_at_layer[layer][page_idx, 1, index:index + n] = value

    def write_blocks_vectorized(self, layer: int, page_indices: torch.Tensor, keys: torch.Tensor,
                                values: torch.Tensor, indices: torch.Tensor,
                                batch_indices: Optional[torch.Tensor] = None,
                                kv_indptr: Optional[torch.Tensor] = None) -> None:
        """Append one token per candidate: ``kv[page_indices[i], :, indices[i]] = (keys[i], values[i])``
        (page_table.py:167-209).  ``batch_indices``/``kv_indptr`` are accepted
        for signature compatibility (the reference passes the identity layout).
        Entries outside the pool are skipped on the device and counted; the
        next ``check_errors`` (the engine's per-step check) raises ValueError."""
        if layer < 0 or layer >= self.layer_num:
            raise ValueError(f"Layer {layer} out of range (max: {self.layer_num - 1})")
        n = keys.shape[0]
        if keys.shape != values.shape or keys.dim() != 3 or keys.shape[1:] != (self.head_num, self.head_dim):
            raise ValueError(f"keys/values must be [N, {self.head_num}, {self.head_dim}]")
        if keys.dtype != self.store_dtype or values.dtype != self.store_dtype:
            raise ValueError(f"keys/values must be {self.store_dtype}")
        if keys.stride(2) != 1 or values.stride(2) != 1:
            keys, values = keys.contiguous(), values.contiguous()
        for t, nm in ((page_indices, "page_indices"), (indices, "indices"), (keys, "keys")):
            _lib.require_device(t, nm)
        page_indices = page_indices.to(torch.int32)
        indices = indices.to(torch.int32)
        if page_indices.numel() < n or indices.numel() < n:
            raise ValueError("page_indices / indices shorter than keys")
        lib = _lib.load()
        rc = lib.be_kv_append(self.kv_cache_at_layer[layer].data_ptr(), _lib.dtype_code(self.store_dtype),
                              self.max_num_pages, self.page_size, self.head_num, self.head_dim,
                              page_indices.data_ptr(), indices.data_ptr(), keys.data_ptr(), keys.stride(0),
                              keys.stride(1), values.data_ptr(), values.stride(0), values.stride(1), n,
                              self._err.data_ptr(), _lib.stream_ptr(self.device))
        _lib.check(rc, "kv append")

    def write_rope_qkv(self, layer: int, qkv: torch.Tensor, num_qo_heads: int, positions: torch.Tensor,
                       cos: torch.Tensor, sin: torch.Tensor, page_indices: torch.Tensor, indices: torch.Tensor,
                       q_out: Optional[torch.Tensor] = None) -> torch.Tensor:
        """Decode-step RoPE fused with the append: ``qkv [N, (Hq + 2 Hkv) * D]``
        (q | k | v heads), ``positions [N]`` int64, HF cos/sin tables ``[max_pos, D]``.
        Writes RoPE(k) and v to ``(page_indices[i], indices[i])`` and returns
        RoPE(q) as ``[N, Hq, D]``."""
        if layer < 0 or layer >= self.layer_num:
            raise ValueError(f"Layer {layer} out of range (max: {self.layer_num - 1})")
        n = qkv.shape[0]
        width = (num_qo_heads + 2 * self.head_num) * self.head_dim
        if qkv.dim() != 2 or qkv.shape[1] != width or qkv.stride(1) != 1:
            raise ValueError(f"qkv must be [N, {width}] with a contiguous last dim")
        if qkv.dtype != self.store_dtype or cos.dtype != self.store_dtype or sin.dtype != self.store_dtype:
            raise ValueError(f"qkv and cos/sin tables must be {self.store_dtype}")
        if cos.shape != sin.shape or cos.dim() != 2 or cos.shape[1] != self.head_dim or not cos.is_contiguous() \
                or not sin.is_contiguous():
            raise ValueError("cos/sin must be contiguous [max_pos, head_dim]")
        for t, nm in ((qkv, "qkv"), (positions, "positions"), (page_indices, "page_indices"), (indices, "indices")):
            _lib.require_device(t, nm)
        if positions.dtype != torch.int64 or page_indices.dtype != torch.int32 or indices.dtype != torch.int32:
            raise ValueError("positions must be int64, page_indices / indices int32")
        if positions.numel() < n or page_indices.numel() < n or indices.numel() < n:
            raise ValueError("positions / page_indices / indices shorter than qkv")
        if q_out is None:
            q_out = torch.empty((n, num_qo_heads, self.head_dim), dtype=qkv.dtype, device=qkv.device)
        elif q_out.shape != (n, num_qo_heads, self.head_dim) or not q_out.is_contiguous() or q_out.dtype != qkv.dtype:
            raise ValueError("q_out must be a contiguous [N, Hq, D] tensor of the storage dtype")
        lib = _lib.load()
        rc = lib.be_rope_qkv_append(qkv.data_ptr(), qkv.stride(0), _lib.dtype_code(self.store_dtype), n, num_qo_heads,
                                    self.head_num, self.head_dim, positions.data_ptr(), cos.data_ptr(),
                                    sin.data_ptr(), cos.shape[0], q_out.data_ptr(),
                                    self.kv_cache_at_layer[layer].data_ptr(), self.max_num_pages, self.page_size,
                                    page_indices.data_ptr(), indices.data_ptr(), self._err.data_ptr(),
                                    _lib.stream_ptr(self.device))
        _lib.check(rc, "rope append")
        return q_out

    # ------------------------------------------------------------ flat views
    def get_k_buffer(self, layer: int) -> torch.Tensor:
        """K of every slot as ``[P * page, Hkv, D]`` (a copy, as in the reference,
        page_table.py:211-226; the HIP attention path never needs it)."""
        return self.kv_cache_at_layer[layer][:, 0].reshape(self.max_num_pages * self.page_size,
                                                           self.head_num, self.head_dim)

    def get_v_buffer(self, layer: int) -> torch.Tensor:
        return self.kv_cache_at_layer[layer][:, 1].reshape(self.max_num_pages * self.page_size,
                                                           self.head_num, self.head_dim)
