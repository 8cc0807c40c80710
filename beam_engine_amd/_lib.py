"""ctypes binding of libbeam_engine_amd.so (the C ABI in include/beam_engine_amd.h).

torch is imported first so that the library binds to the HIP runtime torch
already loaded (same SONAME), i.e. one runtime per process.  There is no CPU
fallback: if the library is missing every entry point raises.
"""

from __future__ import annotations

import ctypes
import os

import torch  # noqa: F401  (loads the process's HIP runtime before the library)

_PKG = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_PKG, "libbeam_engine_amd.so")

BE_F32, BE_F16, BE_BF16 = 0, 1, 2
BE_OK, BE_ERR_INVALID, BE_ERR_HIP, BE_ERR_CAPACITY, BE_ERR_UNSUPPORTED = 0, 1, 2, 3, 4
BE_PLAN_FORCE_VALU = 1
BE_PLAN_FUSED_MERGE = 2
BE_PLAN_TILE_KERNEL = 4
BE_PLAN_NO_TAIL = 8
BE_PLAN_TAIL_ROLE = 16
BE_PLAN_NO_REGS = 32
BE_PLAN_NO_WIDE = 64
BE_PLAN_CAUSAL = 128
BE_PLAN_ROWS = 256
BE_PLAN_NO_ROWS = 512
BE_PLAN_NO_WIDE256 = 1024
BE_PLAN_NO_TAIL_ROLE = 2048
BE_RUN_ATTENTION, BE_RUN_MERGE = 1, 2
BE_TEMP_RECIPROCAL, BE_TEMP_DIVIDE = 0, 1

_DTYPES = {torch.float32: BE_F32, torch.float16: BE_F16, torch.bfloat16: BE_BF16}


def dtype_code(dt: torch.dtype) -> int:
    try:
        return _DTYPES[dt]
    except KeyError:
        raise ValueError(f"unsupported dtype {dt}; expected float32, float16 or bfloat16") from None


class BeLevel(ctypes.Structure):
    _fields_ = [
        ("qo_indptr", ctypes.c_void_p),
        ("kv_indptr", ctypes.c_void_p),
        ("kv_indices", ctypes.c_void_p),
        ("last_page_len", ctypes.c_void_p),
        ("num_groups", ctypes.c_int32),
    ]


class BePlanCaps(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int32) for n in (
        "max_items", "max_queries", "max_pages", "max_merge", "max_merge_rows", "max_zero", "tile_rows",
        "max_tails")]


class BeAttnPlanInfo(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int32) for n in (
        "num_items", "num_part_rows", "num_merge", "num_queries", "num_qo_heads", "num_kv_heads",
        "head_dim", "page_size", "num_pages", "dtype", "kernel", "tile_rows", "chunk_tokens",
        "plan_ints", "off_items", "off_qindex", "off_pages", "off_merge_q", "off_merge_ptr",
        "off_merge_rows", "off_q_merge", "fused_merge", "num_zero", "off_zero_q", "off_zero_ptr",
        "static_layout", "grid_items", "grid_merge", "grid_zero", "part_rows_cap")] + [
        ("partial_bytes", ctypes.c_int64),
        ("counter_offset", ctypes.c_int64),
        ("counter_bytes", ctypes.c_int64),
        ("kv_bytes", ctypes.c_int64),
        ("qo_bytes", ctypes.c_int64),
        ("flops", ctypes.c_double),
    ] + [(n, ctypes.c_int32) for n in ("num_wg", "off_wg", "off_records", "off_record_slots",
                                              "num_tails", "off_tails", "tail_waves",
                                              "num_tail_items", "off_tail_items", "stream_loop",
                                              "off_seg_causal")]


BE_KIND_CASCADE, BE_KIND_FLAT, BE_KIND_SPLIT, BE_KIND_TREE, BE_KIND_AUTO = 0, 1, 2, 3, 4
BE_EDGES_FITTED, BE_EDGES_FASTTREE = 0, 1
KIND_CODES = {"cascade": BE_KIND_CASCADE, "flat": BE_KIND_FLAT, "split": BE_KIND_SPLIT, "tree": BE_KIND_TREE,
              "auto": BE_KIND_AUTO}
KIND_NAMES = {v: k for k, v in KIND_CODES.items()}


class BeTreeModel(ctypes.Structure):
    _fields_ = [("tile_nt", ctypes.c_double * 4)] + [
        (n, ctypes.c_double) for n in ("seg", "slot", "tail", "fixed", "alpha", "beta", "gamma", "tile_w128",
                                       "tile_w256", "tile_sib")] + [
        (n, ctypes.c_int32) for n in ("num_qo_heads", "num_kv_heads", "edge_model", "reserved")]


EXPORTS = (
    "be_version", "be_last_error", "be_kv_append", "be_rope_qkv_append", "be_page_copy", "be_page_copy_counted",
    "be_attn_plan",
    "be_attn_run",
    "be_merge_states", "be_beam_topk_workspace_bytes", "be_beam_topk", "be_beam_topk_noalloc", "be_trie_cascade",
    "be_diverse_select", "be_pages_create", "be_pages_destroy", "be_pages_allocate", "be_pages_share",
    "be_pages_release", "be_pages_reserve", "be_pages_num_free", "be_pages_ref_count", "be_pages_free_list",
    "be_trie_create", "be_trie_destroy", "be_trie_add_root", "be_trie_apply", "be_trie_sizes",
    "be_trie_candidates", "be_trie_export", "be_trie_metadata", "be_trie_plan", "be_trie_levels",
    "be_trie_plan_kind", "be_trie_metadata_kind", "be_read_probe",
)

_lib = None


class HipLibraryMissing(RuntimeError):
    pass


def load() -> ctypes.CDLL:
    """Load the HIP library once; raise HipLibraryMissing if it was not built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise HipLibraryMissing(
            f"{LIB_PATH} is missing: build it with `python -m beam_engine_amd.build` "
            "(beam_engine_amd has no CPU fallback)")
    lib = ctypes.CDLL(LIB_PATH)
    vp, i32, i64 = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64
    lib.be_version.restype = i32
    lib.be_last_error.restype = ctypes.c_char_p
    lib.be_kv_append.argtypes = [vp, i32, i32, i32, i32, i32, vp, vp, vp, i64, i64, vp, i64, i64, i32, vp, vp]
    lib.be_rope_qkv_append.argtypes = [vp, i64, i32, i32, i32, i32, i32, vp, vp, vp, i32, vp, vp, i32, i32, vp, vp,
                                       vp, vp]
    lib.be_page_copy.argtypes = [vp, i64, i32, i32, i32, i32, i32, i32, vp, vp, vp, i32, vp, vp]
    lib.be_page_copy_counted.argtypes = [vp, i64, i32, i32, i32, i32, i32, i32, vp, vp, vp, vp, i32, vp, vp]
    lib.be_attn_plan.argtypes = [ctypes.POINTER(BeLevel), i32, i32, i32, i32, i32, i32, i32, i32, i32, i32,
                                 ctypes.POINTER(BePlanCaps), vp, i64, ctypes.POINTER(BeAttnPlanInfo)]
    lib.be_attn_run.argtypes = [ctypes.POINTER(BeAttnPlanInfo), vp, vp, vp, i64, i64, vp, vp, i64, i64, vp,
                                ctypes.c_float, i32, vp]
    lib.be_merge_states.argtypes = [vp, vp, vp, vp, vp, vp, i32, i32, i32, vp]
    lib.be_beam_topk_workspace_bytes.argtypes = [i32, i32, i32]
    lib.be_beam_topk_workspace_bytes.restype = i64
    lib.be_beam_topk.argtypes = [vp, i32, i32, i32, i64, ctypes.c_double, i32, i32, vp, i32, i32, vp, i32, vp, vp,
                                 vp, vp, vp, vp, i64, vp]
    lib.be_beam_topk_noalloc.argtypes = [vp, i32, i32, i32, i64, ctypes.c_double, i32, i32, vp, i32, i32, vp, i32,
                                         vp, vp, vp, vp, vp, vp]
    lib.be_diverse_select.argtypes = [vp, vp, i32, i32, vp, i32, vp, i32, i32, i32, ctypes.c_double, vp, vp, vp,
                                      vp]
    lib.be_trie_cascade.argtypes = [vp, vp, vp, vp, vp, i32, vp, i32, vp, i64, ctypes.POINTER(ctypes.c_int64)]
    i32p, i64p = ctypes.POINTER(ctypes.c_int32), ctypes.POINTER(ctypes.c_int64)
    lib.be_pages_create.argtypes = [i32]
    lib.be_pages_create.restype = vp
    lib.be_pages_destroy.argtypes = [vp]
    lib.be_pages_destroy.restype = None
    lib.be_pages_allocate.argtypes = [vp, i32p]
    lib.be_pages_share.argtypes = [vp, i32, i32p]
    lib.be_pages_release.argtypes = [vp, i32, i32p]
    lib.be_pages_reserve.argtypes = [vp, i32]
    lib.be_pages_num_free.argtypes = [vp]
    lib.be_pages_ref_count.argtypes = [vp, i32]
    lib.be_pages_free_list.argtypes = [vp, vp, i32]
    lib.be_trie_create.argtypes = [i32, vp]
    lib.be_trie_create.restype = vp
    lib.be_trie_destroy.argtypes = [vp]
    lib.be_trie_destroy.restype = None
    lib.be_trie_add_root.argtypes = [vp, vp, i32, i32, vp]
    lib.be_trie_apply.argtypes = [vp, vp, vp, vp, i32, i32, vp, i32, i32p, i32p]
    lib.be_trie_sizes.argtypes = [vp, vp, i64p]
    lib.be_trie_candidates.argtypes = [vp, vp, vp, vp]
    lib.be_trie_export.argtypes = [vp, vp, vp, vp, vp, vp, vp, vp, vp, vp]
    lib.be_trie_metadata.argtypes = [vp, vp, i64, i64p]
    lib.be_trie_plan.argtypes = [vp, i32, i32, i32, i32, i32, i32, ctypes.POINTER(BePlanCaps), vp, i64, i64p, vp,
                                 i64, ctypes.POINTER(BeAttnPlanInfo), i32p]
    lib.be_trie_levels.argtypes = [vp, vp, vp, vp, vp, i32, vp, i32, i32, i32, i32, ctypes.POINTER(BeTreeModel), vp,
                                   i64, i64p, i32p, vp]
    lib.be_read_probe.argtypes = [vp, i64, i64, i64, i64, i32, vp, i32, vp]
    lib.be_trie_metadata_kind.argtypes = [vp, i32, i32, ctypes.POINTER(BeTreeModel), vp, i64, i64p, i32p, vp]
    lib.be_trie_plan_kind.argtypes = [vp, i32, i32, ctypes.POINTER(BeTreeModel), i32, i32, i32, i32, i32, i32,
                                      ctypes.POINTER(BePlanCaps), vp, i64, i64p, vp, i64,
                                      ctypes.POINTER(BeAttnPlanInfo), i32p, i32p, vp]
    for name in EXPORTS:
        if name not in ("be_version", "be_last_error", "be_beam_topk_workspace_bytes", "be_pages_create",
                        "be_pages_destroy", "be_trie_create", "be_trie_destroy"):
            getattr(lib, name).restype = i32
    _lib = lib
    return lib


def check(rc: int, what: str) -> None:
    """Map a be_status to the reference's exception types."""
    if rc == BE_OK:
        return
    msg = load().be_last_error().decode(errors="replace")
    text = f"{what}: {msg}"
    if rc == BE_ERR_INVALID:
        raise ValueError(text)
    if rc == BE_ERR_CAPACITY:
        raise MemoryError(text)
    if rc == BE_ERR_UNSUPPORTED:
        raise NotImplementedError(text)
    raise RuntimeError(text)


def ptr(t) -> int:
    """Device (or host) address of a tensor, or 0 for None."""
    return 0 if t is None else t.data_ptr()


def stream_ptr(device=None) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def require_device(t: torch.Tensor, name: str) -> None:
    if not t.is_cuda:
        raise ValueError(f"{name} must be a HIP device tensor (got {t.device}); there is no CPU path")
