"""Decode attention wrappers over the HIP work-list kernels.

``MultiLevelCascadeAttentionWrapper`` keeps the interface the reference uses
(flashinfer.cascade.MultiLevelCascadeAttentionWrapper: constructed per step
with a workspace, ``plan(...)`` once per step, ``run(q, kv_layer)`` once per
layer -- src/beam_engine/models/modeling_llama.py:732-755, 321-367).
``BatchDecodeWithPagedKVCacheWrapper`` is the flat strategy: one level, one
group per query.  Both share one plan format and the same kernels.

Semantics (every level, every group): o = softmax(sm_scale * q K^T) V over the
group's valid tokens, query head h reading KV head h // (Hq / Hkv); levels are
merged by log-sum-exp.  ``run(..., return_lse=True)`` returns the natural-log
lse (FlashInfer returns base 2; the reference never reads it).
"""

from __future__ import annotations

import ctypes
import threading
from typing import List, Optional, Sequence

import numpy as np
import torch

from . import _lib

_WS_ALIGN = 256


def _as_i32(x) -> np.ndarray:
    if isinstance(x, torch.Tensor):
        x = x.detach()
        if x.is_cuda:
            x = x.cpu()
        x = x.numpy()
    return np.ascontiguousarray(np.asarray(x, dtype=np.int32))


class _Staging:
    """Pinned host staging for plans (one per device), reused across wrappers.

    The buffer is only rewritten after the previous upload from it finished."""

    _lock = threading.Lock()
    _by_dev = {}

    def __init__(self, device: torch.device):
        self.device = device
        self.buf = torch.empty(1 << 16, dtype=torch.int32, pin_memory=True)
        self.event: Optional[torch.cuda.Event] = None

    @classmethod
    def get(cls, device: torch.device) -> "_Staging":
        key = (device.type, device.index)
        with cls._lock:
            st = cls._by_dev.get(key)
            if st is None:
                st = cls._by_dev[key] = _Staging(device)
            return st

    def acquire(self, ints: int) -> torch.Tensor:
        if self.event is not None:
            self.event.synchronize()
            self.event = None
        if self.buf.numel() < ints:
            self.buf = torch.empty(max(ints, 2 * self.buf.numel()), dtype=torch.int32, pin_memory=True)
        return self.buf


_cus_by_dev = {}


def _num_cus(device: torch.device) -> int:
    key = (device.type, device.index)
    n = _cus_by_dev.get(key)
    if n is None:
        try:
            n = int(torch.cuda.get_device_properties(device).multi_processor_count)
        except Exception:   # noqa: BLE001 - properties are a sizing hint only
            n = 256
        _cus_by_dev[key] = n
    return n


class PlanStats:
    """Algorithmic work of a plan (for roofline reporting)."""

    def __init__(self, info: _lib.BeAttnPlanInfo):
        self.kv_bytes = int(info.kv_bytes)
        self.qo_bytes = int(info.qo_bytes)
        self.flops = float(info.flops)
        self.num_items = int(info.num_items)
        self.num_part_rows = int(info.num_part_rows)
        self.num_merge = int(info.num_merge)
        self.kernel = {0: "valu", 1: "tile", 2: "stream", 3: "rows"}[int(info.kernel)]
        self.num_tails = int(info.num_tails) if self.kernel == "stream" else 0
        self.chunk_tokens = int(info.chunk_tokens)

    @property
    def bytes(self) -> int:
        return self.kv_bytes + self.qo_bytes


class _PagedPlanner:
    """Shared plan/run machinery for the cascade and flat wrappers."""

    def __init__(self, workspace: torch.Tensor, kv_layout: str):
        if kv_layout != "NHD":
            raise ValueError(f"kv_layout {kv_layout!r}: only 'NHD' ([P, 2, page, Hkv, D]) is supported")
        if not isinstance(workspace, torch.Tensor) or workspace.dtype != torch.uint8:
            raise ValueError("workspace buffer must be a uint8 tensor")
        _lib.require_device(workspace, "workspace buffer")
        self._ws = workspace
        self._info: Optional[_lib.BeAttnPlanInfo] = None
        self._plan_dev: Optional[torch.Tensor] = None
        self._partials: Optional[torch.Tensor] = None
        self._max_page = -1
        self._sm_scale = 1.0
        self._dtype: Optional[torch.dtype] = None
        self._force_valu = False
        self._fused_merge = False
        self._tile_kernel = False     # force the per-(item, head) tile kernel over the streaming kernel
        self._no_tail = False         # streaming kernel: keep short groups in whole tiles, no tail chunks
        self._tail_role = None        # streaming kernel: tail chunks in tail-role workgroups (True), in the merge
                                      # kernel (False), or as the planner decides (None)
        self._no_regs = False         # streaming kernel: direct-load loop in every workgroup
        self._no_wide = False         # streaming kernel: no wide (32-row) wave roles, no 128-row segments
        self._no_wide256 = False      # streaming kernel: wide roles on 128-row segments only
        self._rows = None             # row-block kernel: True forces it, False forbids it, None lets the planner pick
        self._num_cus: Optional[int] = None   # planner's CU count (default: the device's)
        self._caps: Optional[_lib.BePlanCaps] = None
        self._views_key = None          # (plan bytes, workspace bytes) of the cached workspace views
        self._views = (None, None)

    # ---------------------------------------------------------------- plan
    def _plan_levels(self, qo: Sequence, kvp: Sequence, kvi: Sequence, lpl: Sequence, num_qo_heads: int,
                     num_kv_heads: int, head_dim: int, page_size: int, sm_scale: Optional[float],
                     q_data_type, num_queries: Optional[int] = None, causal: bool = False) -> None:
        lib = _lib.load()
        if not (len(qo) == len(kvp) == len(kvi) == len(lpl)):
            raise ValueError("per-level index lists must have the same length")
        qo = [_as_i32(x) for x in qo]
        kvp = [_as_i32(x) for x in kvp]
        kvi = [_as_i32(x) for x in kvi]
        lpl = [_as_i32(x) for x in lpl]
        levels = (_lib.BeLevel * max(1, len(qo)))()
        max_page = -1
        nq = 0
        for i, (a, b, c, d) in enumerate(zip(qo, kvp, kvi, lpl)):
            ng = len(a) - 1
            if ng < 0 or len(b) != ng + 1 or len(d) != ng:
                raise ValueError(f"level {i}: qo_indptr / kv_indptr / last_page_len lengths disagree")
            if ng > 0 and len(c) < int(b[-1]):
                raise ValueError(f"level {i}: kv_indices shorter than kv_indptr[-1]")
            levels[i] = _lib.BeLevel(a.ctypes.data, b.ctypes.data, c.ctypes.data if len(c) else 0,
                                     d.ctypes.data, ng)
            if len(c):
                if int(c.min()) < 0:
                    raise ValueError(f"level {i}: negative page index")
                max_page = max(max_page, int(c.max()))
            if ng > 0:
                nq = max(nq, int(a[-1]))
        if num_queries is not None:
            nq = max(nq, int(num_queries))
        if isinstance(q_data_type, str):
            q_data_type = getattr(torch, q_data_type)
        dt = _lib.dtype_code(q_data_type)
        flags = self._plan_flags() | (_lib.BE_PLAN_CAUSAL if causal else 0)
        staging = _Staging.get(self._ws.device)
        info = _lib.BeAttnPlanInfo()
        cap = staging.buf.numel()
        while True:
            buf = staging.acquire(cap)
            rc = lib.be_attn_plan(levels, len(qo), nq, num_qo_heads, num_kv_heads, head_dim, page_size,
                                  max(max_page + 1, 1), dt, flags, self._num_cus or _num_cus(self._ws.device),
                                  ctypes.byref(self._caps) if self._caps is not None else None,
                                  buf.data_ptr(), buf.numel(), ctypes.byref(info))
            if rc == _lib.BE_ERR_CAPACITY and info.plan_ints > buf.numel():
                cap = max(int(info.plan_ints), 2 * buf.numel())
                continue
            # (a capacity error with plan_ints 0 is a fixed layout's, which no
            # buffer size cures: MemoryError)
            _lib.check(rc, "attention plan")
            break
        self._install_plan(info, buf, staging, max_page, head_dim, sm_scale, q_data_type)

    def _plan_flags(self) -> int:
        return (_lib.BE_PLAN_FORCE_VALU if self._force_valu else 0) | \
            (_lib.BE_PLAN_FUSED_MERGE if self._fused_merge else 0) | \
            (_lib.BE_PLAN_TILE_KERNEL if self._tile_kernel else 0) | \
            (_lib.BE_PLAN_NO_TAIL if self._no_tail else 0) | \
            (_lib.BE_PLAN_TAIL_ROLE if self._tail_role is True else 0) | \
            (_lib.BE_PLAN_NO_TAIL_ROLE if self._tail_role is False else 0) | \
            (_lib.BE_PLAN_NO_REGS if self._no_regs else 0) | \
            (_lib.BE_PLAN_NO_WIDE if self._no_wide else 0) | \
            (_lib.BE_PLAN_NO_WIDE256 if self._no_wide256 else 0) | \
            (_lib.BE_PLAN_ROWS if self._rows is True else 0) | \
            (_lib.BE_PLAN_NO_ROWS if self._rows is False else 0)

    def _install_plan(self, info, buf: torch.Tensor, staging: Optional["_Staging"], max_page: int, head_dim: int,
                      sm_scale: Optional[float], q_data_type, upload: bool = True) -> None:
        """Upload a plan written into the pinned staging ``buf`` to the
        workspace (stream-ordered before the next run) and adopt it.
        ``upload=False``: the caller copies ``buf`` to the workspace's first
        ``plan_ints`` words itself, before the next run."""
        plan_bytes = int(info.plan_ints) * 4
        part_off = (plan_bytes + _WS_ALIGN - 1) // _WS_ALIGN * _WS_ALIGN
        need = part_off + int(info.partial_bytes)
        if need > self._ws.numel():
            raise MemoryError(f"attention plan needs {need} workspace bytes, buffer has {self._ws.numel()}")
        key = (plan_bytes, need)
        if self._views_key != key:
            # the workspace views of this plan size (a fixed layout keeps them)
            self._views_key = key
            self._views = (self._ws[:plan_bytes].view(torch.int32),
                           self._ws[part_off:need] if info.partial_bytes else None)
        ws_i32 = self._views[0]
        if upload:
            ws_i32.copy_(buf[: info.plan_ints], non_blocking=True)
            ev = torch.cuda.Event()
            ev.record()
            staging.event = ev
        self._plan_dev = ws_i32
        self._partials = self._views[1]
        if info.counter_bytes:
            c0 = part_off + int(info.counter_offset)
            self._ws[c0:c0 + int(info.counter_bytes)].zero_()
        self._info = info
        self._max_page = max_page
        self._sm_scale = float(head_dim ** -0.5 if sm_scale is None else sm_scale)
        self._dtype = q_data_type

    # ---------------------------------------------------------------- run
    def _run(self, q: torch.Tensor, kv: torch.Tensor, out: Optional[torch.Tensor], return_lse: bool,
             between=None):
        info = self._info
        if info is None:
            raise RuntimeError("plan() must be called before run()")
        lib = _lib.load()
        _lib.require_device(q, "q")
        _lib.require_device(kv, "paged_kv_cache")
        hq, hkv, d, ps = info.num_qo_heads, info.num_kv_heads, info.head_dim, info.page_size
        if q.dim() != 3 or q.shape[1] != hq or q.shape[2] != d:
            raise ValueError(f"q must be [N, {hq}, {d}], got {tuple(q.shape)}")
        if q.shape[0] < info.num_queries:
            raise ValueError(f"q has {q.shape[0]} rows, plan covers {info.num_queries} queries")
        if kv.dim() != 5 or kv.shape[1] != 2 or kv.shape[2] != ps or kv.shape[3] != hkv or kv.shape[4] != d:
            raise ValueError(f"paged_kv_cache must be [P, 2, {ps}, {hkv}, {d}], got {tuple(kv.shape)}")
        if not kv.is_contiguous():
            raise ValueError("paged_kv_cache must be contiguous")
        if kv.shape[0] <= self._max_page:
            raise ValueError(f"plan references page {self._max_page}, cache has {kv.shape[0]} pages")
        if q.dtype != self._dtype or kv.dtype != self._dtype:
            raise ValueError(f"q ({q.dtype}) and cache ({kv.dtype}) must match the planned dtype {self._dtype}")
        if q.stride(2) != 1 or (q.data_ptr() % 16) or (q.stride(0) * q.element_size()) % 16 or \
                (q.stride(1) * q.element_size()) % 16:
            q = q.contiguous()
        if out is None:
            out = torch.empty(q.shape, dtype=q.dtype, device=q.device)
        elif out.shape != q.shape or out.dtype != q.dtype or out.stride(2) != 1:
            raise ValueError("out must match q's shape and dtype with a contiguous head_dim")
        elif (out.data_ptr() % 16) or (out.stride(0) * out.element_size()) % 16 or \
                (out.stride(1) * out.element_size()) % 16:
            raise ValueError("out must be 16-byte aligned in every row (vector stores)")
        lse = torch.empty((q.shape[0], hq), dtype=torch.float32, device=q.device) if return_lse else None
        args = (ctypes.byref(info), self._plan_dev.data_ptr(), _lib.ptr(self._partials), q.data_ptr(),
                q.stride(0), q.stride(1), kv.data_ptr(), out.data_ptr(), out.stride(0), out.stride(1),
                _lib.ptr(lse), self._sm_scale)
        stream = _lib.stream_ptr(q.device)
        if between is None:
            _lib.check(lib.be_attn_run(*args, _lib.BE_RUN_ATTENTION | _lib.BE_RUN_MERGE, stream), "attention run")
        else:   # e.g. an event recorded between the attention and the merge kernels
            _lib.check(lib.be_attn_run(*args, _lib.BE_RUN_ATTENTION, stream), "attention run")
            between()
            _lib.check(lib.be_attn_run(*args, _lib.BE_RUN_MERGE, stream), "attention merge")
        return (out, lse) if return_lse else out

    def use_fixed_layout(self, max_items: int, max_queries: int, max_pages: int, max_merge: int,
                         max_merge_rows: int, max_zero: int, tile_rows: int, max_tails: int = 0) -> None:
        """Plan into a fixed-capacity layout from now on: every plan has the
        same device addresses and launch sizes (the live counts are read on
        the device), so runs can be captured in a HIP graph and replayed with
        later plans.  A plan beyond a capacity raises MemoryError."""
        self._caps = _lib.BePlanCaps(max_items, max_queries, max_pages, max_merge, max_merge_rows, max_zero,
                                     tile_rows, max_tails)

    @property
    def stats(self) -> PlanStats:
        if self._info is None:
            raise RuntimeError("no plan")
        return PlanStats(self._info)


class MultiLevelCascadeAttentionWrapper(_PagedPlanner):
    """Cascade decode attention (drop-in for the FlashInfer wrapper the
    reference builds per step, models/modeling_llama.py:732-755)."""

    def __init__(self, num_levels: int, float_workspace_buffer: torch.Tensor, kv_layout: str = "NHD"):
        super().__init__(float_workspace_buffer, kv_layout)
        if num_levels < 1:
            raise ValueError("num_levels must be >= 1")
        self.num_levels = num_levels

    def plan(self, qo_indptr_arr: List, paged_kv_indptr_arr: List, paged_kv_indices_arr: List,
             paged_kv_last_page_len: List, num_qo_heads: int, num_kv_heads: int, head_dim: int,
             page_size: int, causal: bool = False, pos_encoding_mode: str = "NONE",
             use_fp16_qk_reduction: bool = False, sm_scale: Optional[float] = None,
             window_left: int = -1, logits_soft_cap: Optional[float] = None,
             rope_scale: Optional[float] = None, rope_theta: Optional[float] = None,
             q_data_type="float16", kv_data_type=None) -> None:
        if len(qo_indptr_arr) != self.num_levels:
            raise ValueError(f"wrapper has {self.num_levels} levels, plan got {len(qo_indptr_arr)}")
        if pos_encoding_mode != "NONE":
            raise NotImplementedError("RoPE is applied before attention (pos_encoding_mode='NONE' only)")
        if window_left not in (-1, None) or logits_soft_cap not in (None, 0.0):
            raise NotImplementedError("sliding window / soft cap are not part of the decode path")
        if kv_data_type is not None and kv_data_type != q_data_type:
            raise NotImplementedError("q and KV must share one dtype")
        # causal applies to the last level: query i of a group of n sees the
        # group's first kv_len - n + i + 1 tokens; one query per group (the
        # decode case) masks nothing and keeps the streaming kernel
        mask = False
        if causal:
            last = _as_i32(qo_indptr_arr[-1])
            mask = len(last) > 1 and int(np.max(np.diff(last))) > 1
        self._plan_levels(qo_indptr_arr, paged_kv_indptr_arr, paged_kv_indices_arr, paged_kv_last_page_len,
                          num_qo_heads, num_kv_heads, head_dim, page_size, sm_scale, q_data_type, causal=mask)

    def run(self, q: torch.Tensor, paged_kv_cache: torch.Tensor, out: Optional[torch.Tensor] = None,
            return_lse: bool = False, between=None):
        return self._run(q, paged_kv_cache, out, return_lse, between)

    forward = run


class BatchDecodeWithPagedKVCacheWrapper(_PagedPlanner):
    """Flat paged decode: query i attends to its own page list (the baseline
    strategy the cascade and tree strategies are measured against)."""

    def __init__(self, float_workspace_buffer: torch.Tensor, kv_layout: str = "NHD"):
        super().__init__(float_workspace_buffer, kv_layout)

    def plan(self, indptr, indices, last_page_len, num_qo_heads: int, num_kv_heads: int, head_dim: int,
             page_size: int, pos_encoding_mode: str = "NONE", window_left: int = -1,
             logits_soft_cap: Optional[float] = None, q_data_type="float16", kv_data_type=None,
             sm_scale: Optional[float] = None, **_unused) -> None:
        if pos_encoding_mode != "NONE":
            raise NotImplementedError("RoPE is applied before attention (pos_encoding_mode='NONE' only)")
        if kv_data_type is not None and kv_data_type != q_data_type:
            raise NotImplementedError("q and KV must share one dtype")
        n = len(_as_i32(last_page_len))
        self._plan_levels([np.arange(n + 1, dtype=np.int32)], [indptr], [indices], [last_page_len],
                          num_qo_heads, num_kv_heads, head_dim, page_size, sm_scale, q_data_type)

    def run(self, q: torch.Tensor, paged_kv_cache: torch.Tensor, out: Optional[torch.Tensor] = None,
            return_lse: bool = False, between=None):
        return self._run(q, paged_kv_cache, out, return_lse, between)

    forward = run


class BatchPrefillWithPagedKVCacheWrapper(_PagedPlanner):
    """Paged prefill attention (drop-in for the FlashInfer wrapper of the
    reference's prefill, models/modeling_llama.py:213-283, 775-798): request
    r's queries ``q[qo_indptr[r]:qo_indptr[r+1]]`` attend to its pages, whose
    K/V the caller wrote first; ``causal=True`` gives query i of n the first
    kv_len - n + i + 1 tokens.  Runs on the MFMA tile kernel (bf16 / fp16) or
    the VALU kernel (fp32) with a per-row causal limit; query tiles stop at
    the chunk holding their last visible token."""

    def __init__(self, float_workspace_buffer: torch.Tensor, kv_layout: str = "NHD"):
        super().__init__(float_workspace_buffer, kv_layout)

    def plan(self, qo_indptr, paged_kv_indptr, paged_kv_indices, paged_kv_last_page_len, num_qo_heads: int,
             num_kv_heads: int, head_dim_qk: int, page_size: int, head_dim_vo: Optional[int] = None,
             causal: bool = False, pos_encoding_mode: str = "NONE", use_fp16_qk_reduction: bool = False,
             sm_scale: Optional[float] = None, window_left: int = -1, logits_soft_cap: Optional[float] = None,
             q_data_type="float16", kv_data_type=None, **_unused) -> None:
        if pos_encoding_mode != "NONE":
            raise NotImplementedError("RoPE is applied before attention (pos_encoding_mode='NONE' only)")
        if window_left not in (-1, None) or logits_soft_cap not in (None, 0.0):
            raise NotImplementedError("sliding window / soft cap are not supported")
        if head_dim_vo is not None and head_dim_vo != head_dim_qk:
            raise NotImplementedError("head_dim_vo must equal head_dim_qk")
        if kv_data_type is not None and kv_data_type != q_data_type:
            raise NotImplementedError("q and KV must share one dtype")
        qo = _as_i32(qo_indptr)
        self._plan_levels([qo], [paged_kv_indptr], [paged_kv_indices], [paged_kv_last_page_len], num_qo_heads,
                          num_kv_heads, head_dim_qk, page_size, sm_scale, q_data_type,
                          causal=bool(causal) and len(qo) > 1 and int(np.max(np.diff(qo))) > 1)

    def run(self, q: torch.Tensor, paged_kv_cache: torch.Tensor, out: Optional[torch.Tensor] = None,
            return_lse: bool = False):
        return self._run(q, paged_kv_cache, out, return_lse)

    forward = run


def merge_state(v_a: torch.Tensor, s_a: torch.Tensor, v_b: torch.Tensor, s_b: torch.Tensor):
    """Merge two attention states (v [n, H, D] float32, s [n, H] natural-log lse)."""
    lib = _lib.load()
    for t, nm in ((v_a, "v_a"), (s_a, "s_a"), (v_b, "v_b"), (s_b, "s_b")):
        _lib.require_device(t, nm)
        if t.dtype != torch.float32:
            raise ValueError(f"{nm} must be float32")
    if v_a.shape != v_b.shape or s_a.shape != s_b.shape or v_a.shape[:2] != s_a.shape:
        raise ValueError("state shapes disagree")
    v_a, s_a, v_b, s_b = (t.contiguous() for t in (v_a, s_a, v_b, s_b))
    v = torch.empty_like(v_a)
    s = torch.empty_like(s_a)
    n, h, d = v_a.shape
    _lib.check(lib.be_merge_states(v_a.data_ptr(), s_a.data_ptr(), v_b.data_ptr(), s_b.data_ptr(),
                                   v.data_ptr(), s.data_ptr(), n, h, d, _lib.stream_ptr(v_a.device)),
               "merge_state")
    return v, s
