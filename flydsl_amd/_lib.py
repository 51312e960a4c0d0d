"""ctypes binding of ``libpa_fp8.so`` (the C ABI in ``include/pa_fp8.h``).

The library is built in-tree by :func:`flydsl_amd.build.build_library`.  A
missing library is an error: there is no fallback implementation.
"""

from __future__ import annotations

import ctypes
import os
from typing import Optional

LIB_NAME = "libpa_fp8.so"
LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), LIB_NAME)
# The checked build (same kernels; every index they clamp is also recorded).
CHECKED_LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libpa_fp8_checked.so")

ABI_VERSION = 1

DTYPE_BF16 = 0
DTYPE_F16 = 1
DTYPE_F32 = 2

CACHE_FLASH = 0
CACHE_ATOM = 1
CACHE_ATOM_TRANS_V = 2

ERRORS = {
    -1: "PA_ERR_NULL_ARG",
    -2: "PA_ERR_HEAD_SIZE",
    -3: "PA_ERR_BLOCK_SIZE",
    -4: "PA_ERR_GROUP",
    -5: "PA_ERR_DTYPE",
    -6: "PA_ERR_SHAPE",
    -7: "PA_ERR_ALIGN",
    -8: "PA_ERR_ABI",
    -9: "PA_ERR_SCRATCH",
}

EXPORTED_SYMBOLS = (
    "pa_fp8_decode_partition",
    "pa_fp8_decode_reduce",
    "pa_fp8_recommended_splits",
    "pa_fp8_plan_slot",
    "pa_fp8_plan_visible",
    "pa_fp8_version",
    "pa_fp8_error_string",
    "pa_fp8_decode_worklist",
    "pa_fp8_decode_balanced",
    "pa_fp8_merge_balanced",
    "pa_fp8_decode_balanced_static",
    "pa_fp8_static_scratch_bytes",
    "pa_fp8_balanced_workspace_bytes",
    "pa_fp8_stream_workers",
    "pa_fp8_reduce_worklist",
    "pa_fp8_worklist_sizes",
    "pa_fp8_plan_worklist",
    "pa_fp8_rope_cache",
    "pa_fp8_qk_norm_rope_quant",
    "pa_fp8_mla_decode",
    "pa_fp8_mla_reduce",
    "pa_fp8_mla_plan_sizes",
    "pa_fp8_mla_plan",
    "pa_fp8_fnuz_to_fn",
    "pa_fp8_debug_violations",
    "pa_fp8_checked_build",
)

# Bits of pa_fp8_debug_violations (a checked build's record of clamped indices).
VIOLATION_PAGE = 1
VIOLATION_WORK = 2
VIOLATION_POSITION = 4
VIOLATION_SLOT = 8

_i32 = ctypes.c_int32
_i64 = ctypes.c_int64
_vp = ctypes.c_void_p


class PartitionArgs(ctypes.Structure):
    """Mirror of ``pa_fp8_partition_args`` (field order matters)."""

    _fields_ = [
        ("abi_version", _i32),
        ("exp_sums", _vp),
        ("max_logits", _vp),
        ("tmp_out", _vp),
        ("output", _vp),
        ("query", _vp),
        ("key_cache", _vp),
        ("value_cache", _vp),
        ("block_tables", _vp),
        ("kv_indptr", _vp),
        ("context_lengths", _vp),
        ("key_scale", _vp),
        ("value_scale", _vp),
        ("stride_q_tok", _i64),
        ("stride_q_head", _i64),
        ("stride_k_block", _i64),
        ("stride_k_head", _i64),
        ("stride_v_block", _i64),
        ("stride_v_head", _i64),
        ("stride_es_seq", _i64),
        ("stride_es_head", _i64),
        ("stride_es_part", _i64),
        ("stride_to_seq", _i64),
        ("stride_to_head", _i64),
        ("stride_to_part", _i64),
        ("stride_to_group", _i64),
        ("stride_bt_seq", _i64),
        ("stride_ks_block", _i64),
        ("stride_ks_head", _i64),
        ("stride_out_tok", _i64),
        ("stride_out_head", _i64),
        ("num_seqs", _i32),
        ("num_kv_heads", _i32),
        ("num_partitions", _i32),
        ("slots_per_workgroup", _i32),
        ("query_length", _i32),
        ("query_group_size", _i32),
        ("head_size", _i32),
        ("block_size", _i32),
        ("num_blocks", _i32),
        ("max_blocks_per_seq", _i32),
        ("sliding_window", _i32),
        ("per_token_kv", _i32),
        ("trans_v", _i32),
        ("query_dtype", _i32),
        ("tmp_dtype", _i32),
        ("output_dtype", _i32),
        ("softmax_scale", ctypes.c_float),
    ]


class ReduceArgs(ctypes.Structure):
    """Mirror of ``pa_fp8_reduce_args``."""

    _fields_ = [
        ("abi_version", _i32),
        ("output", _vp),
        ("exp_sums", _vp),
        ("max_logits", _vp),
        ("tmp_out", _vp),
        ("stride_out_seq", _i64),
        ("stride_out_ql", _i64),
        ("stride_out_kv_head", _i64),
        ("stride_out_group", _i64),
        ("stride_es_seq", _i64),
        ("stride_es_head", _i64),
        ("stride_es_part", _i64),
        ("stride_to_seq", _i64),
        ("stride_to_head", _i64),
        ("stride_to_part", _i64),
        ("stride_to_group", _i64),
        ("num_seqs", _i32),
        ("num_kv_heads", _i32),
        ("num_partitions", _i32),
        ("query_length", _i32),
        ("query_group_size", _i32),
        ("head_size", _i32),
        ("output_dtype", _i32),
        ("tmp_dtype", _i32),
    ]


class StreamArgs(ctypes.Structure):
    """Mirror of ``pa_fp8_stream_args``."""

    _fields_ = [
        ("abi_version", _i32),
        ("output", _vp),
        ("query", _vp),
        ("key_cache", _vp),
        ("value_cache", _vp),
        ("block_tables", _vp),
        ("kv_indptr", _vp),
        ("context_lengths", _vp),
        ("key_scale", _vp),
        ("value_scale", _vp),
        ("work_indptr", _vp),
        ("work_info", _vp),
        ("partition_indptr", _vp),
        ("partial_output", _vp),
        ("partial_lse", _vp),
        ("stride_q_tok", _i64),
        ("stride_q_head", _i64),
        ("stride_k_block", _i64),
        ("stride_k_head", _i64),
        ("stride_v_block", _i64),
        ("stride_v_head", _i64),
        ("stride_bt_seq", _i64),
        ("stride_ks_block", _i64),
        ("stride_ks_head", _i64),
        ("stride_out_tok", _i64),
        ("stride_out_head", _i64),
        ("stride_po_row", _i64),
        ("stride_pl_row", _i64),
        ("num_seqs", _i32),
        ("num_kv_heads", _i32),
        ("query_length", _i32),
        ("query_group_size", _i32),
        ("head_size", _i32),
        ("block_size", _i32),
        ("num_blocks", _i32),
        ("max_blocks_per_seq", _i32),
        ("sliding_window", _i32),
        ("per_token_kv", _i32),
        ("trans_v", _i32),
        ("query_dtype", _i32),
        ("output_dtype", _i32),
        ("num_workers", _i32),
        ("softmax_scale", ctypes.c_float),
    ]


class WorklistReduceArgs(ctypes.Structure):
    """Mirror of ``pa_fp8_worklist_reduce_args``."""

    _fields_ = [
        ("abi_version", _i32),
        ("output", _vp),
        ("partial_output", _vp),
        ("partial_lse", _vp),
        ("reduce_indptr", _vp),
        ("reduce_final_map", _vp),
        ("reduce_partial_map", _vp),
        ("stride_out_tok", _i64),
        ("stride_out_head", _i64),
        ("stride_po_row", _i64),
        ("stride_pl_row", _i64),
        ("num_groups", _i32),
        ("num_query_heads", _i32),
        ("head_size", _i32),
        ("max_query_length", _i32),
        ("output_dtype", _i32),
    ]


class RopeCacheArgs(ctypes.Structure):
    """Mirror of ``pa_fp8_rope_cache_args``."""

    _fields_ = [
        ("abi_version", _i32),
        ("q", _vp),
        ("k", _vp),
        ("v", _vp),
        ("positions", _vp),
        ("cos_cache", _vp),
        ("sin_cache", _vp),
        ("slot_mapping", _vp),
        ("key_cache", _vp),
        ("value_cache", _vp),
        ("q_out", _vp),
        ("k_out", _vp),
        ("k_scale", _vp),
        ("v_scale", _vp),
        ("stride_q_tok", _i64),
        ("stride_q_head", _i64),
        ("stride_k_tok", _i64),
        ("stride_k_head", _i64),
        ("stride_v_tok", _i64),
        ("stride_v_head", _i64),
        ("stride_qo_tok", _i64),
        ("stride_qo_head", _i64),
        ("stride_ko_tok", _i64),
        ("stride_ko_head", _i64),
        ("stride_cos_pos", _i64),
        ("stride_sin_pos", _i64),
        ("num_tokens", _i32),
        ("num_q_heads", _i32),
        ("num_kv_heads", _i32),
        ("head_dim", _i32),
        ("block_size", _i32),
        ("num_blocks", _i32),
        ("max_pos", _i32),
        ("dtype", _i32),
        ("cache_layout", _i32),
        ("apply_scale", _i32),
        ("reuse_freqs_front_part", _i32),
        ("index_i64", _i32),
    ]


_LIB: Optional[ctypes.CDLL] = None


class QkNormRopeArgs(ctypes.Structure):
    """Mirror of ``pa_qk_norm_rope_args`` (field order matters)."""

    _fields_ = [
        ("abi_version", ctypes.c_int32),
        ("q", _vp),
        ("kv", _vp),
        ("q_weight", _vp),
        ("kv_weight", _vp),
        ("cos_cache", _vp),
        ("sin_cache", _vp),
        ("positions", _vp),
        ("q_out", _vp),
        ("kv_out", _vp),
        ("q_scale", _vp),
        ("kv_scale", _vp),
        ("stride_q_tok", _i64),
        ("stride_kv_tok", _i64),
        ("num_tokens", ctypes.c_int32),
        ("num_q_heads", ctypes.c_int32),
        ("head_dim", ctypes.c_int32),
        ("rope_head_dim", ctypes.c_int32),
        ("max_pos", ctypes.c_int32),
        ("quant", ctypes.c_int32),
        ("group_size", ctypes.c_int32),
        ("scale_e8m0", ctypes.c_int32),
    ]


class MlaDecodeArgs(ctypes.Structure):
    """Mirror of ``pa_mla_decode_args`` (field order matters)."""

    _fields_ = [
        ("abi_version", ctypes.c_int32),
        ("query", _vp),
        ("kv_buffer", _vp),
        ("kv_page_indices", _vp),
        ("work_indptr", _vp),
        ("work_info", _vp),
        ("final_output", _vp),
        ("split_output", _vp),
        ("split_lse", _vp),
        ("num_pages", _i64),
        ("num_page_indices", ctypes.c_int32),
        ("num_rows", ctypes.c_int32),
        ("num_workers", ctypes.c_int32),
        ("num_works", ctypes.c_int32),
        ("num_partial", ctypes.c_int32),
        ("softmax_scale", ctypes.c_float),
        ("precise_p", ctypes.c_int32),
    ]


class MlaReduceArgs(ctypes.Structure):
    """Mirror of ``pa_mla_reduce_args`` (field order matters)."""

    _fields_ = [
        ("abi_version", ctypes.c_int32),
        ("split_output", _vp),
        ("split_lse", _vp),
        ("reduce_indptr", _vp),
        ("reduce_final_map", _vp),
        ("reduce_partial_map", _vp),
        ("final_output", _vp),
        ("final_lse", _vp),
        ("num_groups", ctypes.c_int32),
        ("num_partial", ctypes.c_int32),
        ("num_partial_map", ctypes.c_int32),
        ("num_rows", ctypes.c_int32),
    ]


class LibraryNotBuilt(RuntimeError):
    pass


def load(path: Optional[str] = None) -> ctypes.CDLL:
    """Load (once) and type the shared library; raise if it is not built."""
    global _LIB
    if _LIB is not None and path is None:
        return _LIB
    p = path or os.environ.get("PA_FP8_LIB") or LIB_PATH
    if not os.path.exists(p):
        raise LibraryNotBuilt(
            f"{p} is missing: build the HIP library first (python -c 'import __graft_entry__ as g; g.build()')"
        )
    lib = ctypes.CDLL(p)
    lib.pa_fp8_decode_partition.argtypes = [ctypes.POINTER(PartitionArgs), _vp]
    lib.pa_fp8_decode_partition.restype = ctypes.c_int
    lib.pa_fp8_decode_reduce.argtypes = [ctypes.POINTER(ReduceArgs), _vp]
    lib.pa_fp8_decode_reduce.restype = ctypes.c_int
    lib.pa_fp8_recommended_splits.argtypes = [ctypes.c_int] * 7
    lib.pa_fp8_recommended_splits.restype = ctypes.c_int
    lib.pa_fp8_plan_slot.argtypes = [ctypes.c_int] * 5 + [ctypes.POINTER(ctypes.c_int)] * 2
    lib.pa_fp8_plan_slot.restype = ctypes.c_int
    lib.pa_fp8_plan_visible.argtypes = [ctypes.c_int] * 4 + [ctypes.POINTER(ctypes.c_int)] * 2
    lib.pa_fp8_plan_visible.restype = ctypes.c_int
    lib.pa_fp8_version.argtypes = []
    lib.pa_fp8_version.restype = ctypes.c_char_p
    lib.pa_fp8_error_string.argtypes = [ctypes.c_int]
    lib.pa_fp8_error_string.restype = ctypes.c_char_p
    lib.pa_fp8_decode_worklist.argtypes = [ctypes.POINTER(StreamArgs), _vp]
    lib.pa_fp8_decode_worklist.restype = ctypes.c_int
    lib.pa_fp8_decode_balanced.argtypes = [ctypes.POINTER(StreamArgs), _vp, _i64, _vp]
    lib.pa_fp8_decode_balanced.restype = ctypes.c_int
    lib.pa_fp8_merge_balanced.argtypes = [ctypes.POINTER(StreamArgs), _vp, _i64, _vp]
    lib.pa_fp8_merge_balanced.restype = ctypes.c_int
    lib.pa_fp8_decode_balanced_static.argtypes = [ctypes.POINTER(StreamArgs), _vp]
    lib.pa_fp8_decode_balanced_static.restype = ctypes.c_int
    lib.pa_fp8_static_scratch_bytes.argtypes = []
    lib.pa_fp8_static_scratch_bytes.restype = _i64
    lib.pa_fp8_balanced_workspace_bytes.argtypes = [ctypes.c_int] * 5
    lib.pa_fp8_balanced_workspace_bytes.restype = _i64
    lib.pa_fp8_stream_workers.argtypes = [ctypes.c_int] * 4
    lib.pa_fp8_stream_workers.restype = ctypes.c_int
    lib.pa_fp8_reduce_worklist.argtypes = [ctypes.POINTER(WorklistReduceArgs), _vp]
    lib.pa_fp8_reduce_worklist.restype = ctypes.c_int
    lib.pa_fp8_worklist_sizes.argtypes = [ctypes.c_int] * 3 + [ctypes.POINTER(ctypes.c_int)] * 2
    lib.pa_fp8_worklist_sizes.restype = ctypes.c_int
    lib.pa_fp8_plan_worklist.argtypes = [_vp] + [ctypes.c_int] * 6 + [_vp] * 5
    lib.pa_fp8_plan_worklist.restype = ctypes.c_int
    lib.pa_fp8_rope_cache.argtypes = [ctypes.POINTER(RopeCacheArgs), _vp]
    lib.pa_fp8_rope_cache.restype = ctypes.c_int
    lib.pa_fp8_qk_norm_rope_quant.argtypes = [ctypes.POINTER(QkNormRopeArgs), _vp]
    lib.pa_fp8_qk_norm_rope_quant.restype = ctypes.c_int
    lib.pa_fp8_mla_decode.argtypes = [ctypes.POINTER(MlaDecodeArgs), _vp]
    lib.pa_fp8_mla_decode.restype = ctypes.c_int
    lib.pa_fp8_mla_reduce.argtypes = [ctypes.POINTER(MlaReduceArgs), _vp]
    lib.pa_fp8_mla_reduce.restype = ctypes.c_int
    lib.pa_fp8_mla_plan_sizes.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.POINTER(ctypes.c_int),
                                          ctypes.POINTER(ctypes.c_int)]
    lib.pa_fp8_mla_plan_sizes.restype = ctypes.c_int
    lib.pa_fp8_mla_plan.argtypes = [_vp, _vp] + [ctypes.c_int] * 4 + [_vp] * 5 + [ctypes.POINTER(ctypes.c_int)] * 2
    lib.pa_fp8_mla_plan.restype = ctypes.c_int
    lib.pa_fp8_fnuz_to_fn.argtypes = [_vp, _vp, _i64, _i64, _i64, _vp, _vp]
    lib.pa_fp8_fnuz_to_fn.restype = ctypes.c_int
    lib.pa_fp8_debug_violations.argtypes = [ctypes.POINTER(ctypes.c_uint)]
    lib.pa_fp8_debug_violations.restype = ctypes.c_int
    lib.pa_fp8_checked_build.argtypes = []
    lib.pa_fp8_checked_build.restype = ctypes.c_int
    if path is None:
        _LIB = lib
    return lib


def check(rc: int, what: str) -> None:
    if rc != 0:
        msg = load().pa_fp8_error_string(rc).decode()
        raise RuntimeError(f"{what} failed: {ERRORS.get(rc, 'hipError')} ({rc}): {msg}")


def debug_violations(lib: Optional[ctypes.CDLL] = None) -> int:
    """VIOLATION_* bits a checked build recorded since the last call (then
    cleared; 0 from a release build).  Synchronises the current device."""
    lib = lib or load()
    bits = ctypes.c_uint(0)
    rc = lib.pa_fp8_debug_violations(ctypes.byref(bits))
    if rc != 0:
        raise RuntimeError(f"pa_fp8_debug_violations failed: {rc}")
    return int(bits.value)


def plan_slot(context_length: int, num_partitions: int, slot: int, sliding_window: int, query_length: int):
    t0, t1 = ctypes.c_int(), ctypes.c_int()
    check(
        load().pa_fp8_plan_slot(context_length, num_partitions, slot, sliding_window, query_length, t0, t1),
        "pa_fp8_plan_slot",
    )
    return t0.value, t1.value


def plan_visible(context_length: int, qi: int, query_length: int, sliding_window: int):
    lo, hi = ctypes.c_int(), ctypes.c_int()
    check(load().pa_fp8_plan_visible(context_length, qi, query_length, sliding_window, lo, hi), "pa_fp8_plan_visible")
    return lo.value, hi.value


def recommended_splits(num_seqs, num_kv_heads, split_kv_blocks, sliding_window, partition_tokens, query_length, num_cu):
    return int(
        load().pa_fp8_recommended_splits(
            num_seqs, num_kv_heads, split_kv_blocks, sliding_window, partition_tokens, query_length, num_cu
        )
    )


def stream_workers(num_cu: int, query_length: int, query_group_size: int, per_token_kv: bool) -> int:
    n = int(load().pa_fp8_stream_workers(num_cu, query_length, query_group_size, int(per_token_kv)))
    if n < 0:
        check(n, "pa_fp8_stream_workers")
    return n


def balanced_workspace_bytes(num_seqs: int, num_kv_heads: int, query_length: int, query_group_size: int,
                             num_workers: int) -> int:
    n = int(load().pa_fp8_balanced_workspace_bytes(num_seqs, num_kv_heads, query_length, query_group_size,
                                                   num_workers))
    if n < 0:
        check(n, "pa_fp8_balanced_workspace_bytes")
    return n


def worklist_sizes(num_seqs: int, num_kv_heads: int, num_cu: int):
    mw, ms = ctypes.c_int(), ctypes.c_int()
    check(load().pa_fp8_worklist_sizes(num_seqs, num_kv_heads, num_cu, mw, ms), "pa_fp8_worklist_sizes")
    return mw.value, ms.value


def plan_worklist(context_lengths, num_kv_heads: int, query_group_size: int, query_length: int, num_cu: int,
                  kv_granularity: int = 256):
    """Host work list (numpy int32 arrays); returns (num_works, dict)."""
    import numpy as np

    ctx = np.ascontiguousarray(np.asarray(context_lengths, dtype=np.int32))
    B = int(ctx.shape[0])
    max_works, max_split = worklist_sizes(B, num_kv_heads, num_cu)
    out = {
        "work_indptr": np.zeros(num_cu + 1, np.int32),
        "work_info": np.zeros((max(max_works, 0), 8), np.int32),
        "reduce_indptr": np.zeros(B + 1, np.int32),
        "reduce_final_map": np.zeros((B, 2), np.int32),
        "reduce_partial_map": np.zeros(max(max_split, 1), np.int32),
    }
    ptr = lambda a: a.ctypes.data_as(ctypes.c_void_p)
    n = int(load().pa_fp8_plan_worklist(ptr(ctx), B, num_kv_heads, query_group_size, query_length, num_cu,
                                        kv_granularity, ptr(out["work_indptr"]), ptr(out["work_info"]),
                                        ptr(out["reduce_indptr"]), ptr(out["reduce_final_map"]),
                                        ptr(out["reduce_partial_map"])))
    if n < 0:
        check(n, "pa_fp8_plan_worklist")
    return n, out


def mla_plan_sizes(num_rows: int, num_workers: int):
    mw, mp = ctypes.c_int(), ctypes.c_int()
    check(load().pa_fp8_mla_plan_sizes(num_rows, num_workers, mw, mp), "pa_fp8_mla_plan_sizes")
    return mw.value, mp.value


def mla_plan(qo_indptr, kv_indptr, num_workers: int):
    """Host MLA work list (numpy int32 arrays); returns (num_works, num_groups,
    num_partials, dict)."""
    import numpy as np

    qo = np.ascontiguousarray(np.asarray(qo_indptr, dtype=np.int32))
    kv = np.ascontiguousarray(np.asarray(kv_indptr, dtype=np.int32))
    B = int(qo.shape[0]) - 1
    rows = int(qo[-1] - qo[0]) if B >= 0 else 0
    max_works, max_partials = mla_plan_sizes(rows, num_workers)
    out = {
        "work_indptr": np.zeros(num_workers + 1, np.int32),
        "work_info": np.zeros((max(max_works, 1), 8), np.int32),
        "reduce_indptr": np.zeros(rows + 1, np.int32),
        "reduce_final_map": np.zeros((max(rows, 1), 2), np.int32),
        "reduce_partial_map": np.zeros(max(max_partials, 1), np.int32),
    }
    ng, npart = ctypes.c_int(), ctypes.c_int()
    ptr = lambda a: a.ctypes.data_as(ctypes.c_void_p)
    n = int(load().pa_fp8_mla_plan(ptr(qo), ptr(kv), B, num_workers, max(max_works, 1), max(max_partials, 1),
                                   ptr(out["work_indptr"]), ptr(out["work_info"]), ptr(out["reduce_indptr"]),
                                   ptr(out["reduce_final_map"]), ptr(out["reduce_partial_map"]), ng, npart))
    if n < 0:
        check(n, "pa_fp8_mla_plan")
    return n, ng.value, npart.value, out
