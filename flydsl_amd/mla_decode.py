"""MLA (multi-head latent attention) fp8 decode: drop-in for FlyDSL's
``flydsl_mla_fwd_decode`` plus the work-list and reduce calls its test takes
from aiter.

Reference interface:
  * kernels/mla_fwd_decode.py:57-167 -- :func:`flydsl_mla_fwd_decode`
    (same arguments, assertions and NotImplementedError for other shapes);
  * tests/kernels/test_mla_decode.py:252-295, :356-365 -- the aiter calls
    ``get_mla_metadata_info_v1``, ``get_mla_metadata_v1`` and
    ``mla_reduce_v1``.  aiter is not part of the reference; these are our
    own with the same call signatures and buffer formats: the work list is
    planned on the host (128-token blocks dealt to one worker per CU) and
    the reduce is a log-sum-exp merge kernel of this library.

Device work runs in ``libpa_fp8.so`` (C ABI: ``include/pa_fp8.h``,
``pa_fp8_mla_decode`` / ``pa_fp8_mla_reduce`` / ``pa_fp8_mla_plan``).
"""

from __future__ import annotations

import ctypes
from typing import Optional

import torch

from . import _lib

NUM_QO_HEADS = 128
KV_LORA_RANK = 512
QK_ROPE_HEAD_DIM = 64
QK_HEAD_DIM = KV_LORA_RANK + QK_ROPE_HEAD_DIM  # 576
V_HEAD_DIM = KV_LORA_RANK  # 512
BLOCK_TOKENS = 128  # tokens per work-list block (one LDS stage of the kernel)


_FNUZ = torch.float8_e4m3fnuz


def _is_fp8(dtype: torch.dtype) -> bool:
    """The fp8 dtypes the reference's launcher accepts (kernels/mla_fwd_decode.py:52-53)."""
    return dtype in (torch.float8_e4m3fn, _FNUZ)


def _stream_handle(device: torch.device):
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def _num_cu(device=None) -> int:
    if torch.cuda.is_available():
        dev = torch.device("cuda") if device is None else torch.device(device)
        return int(torch.cuda.get_device_properties(dev).multi_processor_count)
    return 256  # MI355X


def flydsl_mla_fwd_decode(
    query: torch.Tensor,  # [num_seqs, num_heads, head_size]
    kv_buffer: torch.Tensor,  # [num_page, page_size, num_kv_heads, head_size]
    kv_page_indices: torch.Tensor,
    work_indptr: torch.Tensor,
    work_info_set: torch.Tensor,
    final_output: torch.Tensor,  # [num_seqs, num_heads, v_head_dim]
    split_output: torch.Tensor,  # [num_partial_slots, 1, num_heads, v_head_dim]
    split_lse: torch.Tensor,  # [num_partial_slots, 1, num_heads, 1]
    softmax_scale: float,
    *,
    precise_p: bool = False,
) -> None:
    """Launch the MLA decode (kernels/mla_fwd_decode.py:57-167).

    Works with partial row -1 write ``final_output`` (bf16); the others
    write the normalised partial output and its log-sum-exp into
    ``split_output`` / ``split_lse`` for :func:`mla_reduce_v1`.
    ``precise_p`` (our extension) carries the probabilities as two fp8 terms
    in the value product instead of one (the reference's arithmetic)."""
    num_heads = query.size(1)
    q_dtype = query.dtype
    kv_dtype = kv_buffer.dtype
    if not (num_heads == NUM_QO_HEADS and _is_fp8(q_dtype) and _is_fp8(kv_dtype)):
        raise NotImplementedError(
            f"flydsl_mla_fwd_decode: unsupported num_heads={num_heads}, q_dtype={q_dtype}, kv_dtype={kv_dtype}"
        )
    # shape validation (kernels/mla_fwd_decode.py:83-134)
    assert query.ndim == 3, f"query: expected 3D [num_seqs, num_heads, qk_head_dim], got shape {list(query.shape)}"
    assert query.size(2) == QK_HEAD_DIM, f"query: head_dim={query.size(2)}, expected {QK_HEAD_DIM}"
    assert kv_buffer.ndim == 4, (
        f"kv_buffer: expected 4D [num_page, page_size, num_kv_heads, qk_head_dim], got shape {list(kv_buffer.shape)}"
    )
    assert kv_buffer.size(1) * kv_buffer.size(2) == 1, (
        f"kv_buffer: page_size*num_kv_heads must be 1, "
        f"got page_size={kv_buffer.size(1)}, num_kv_heads={kv_buffer.size(2)}"
    )
    assert kv_buffer.size(3) == QK_HEAD_DIM, f"kv_buffer: head_dim={kv_buffer.size(3)}, expected {QK_HEAD_DIM}"
    num_seqs = query.size(0)
    assert final_output.shape == (num_seqs, num_heads, V_HEAD_DIM), (
        f"final_output: expected shape [{num_seqs}, {num_heads}, {V_HEAD_DIM}], got {list(final_output.shape)}"
    )
    num_partial = split_output.size(0)
    assert split_output.ndim == 4 and split_output.shape[1:] == (1, num_heads, V_HEAD_DIM), (
        f"split_output: expected [N, 1, {num_heads}, {V_HEAD_DIM}], got {list(split_output.shape)}"
    )
    assert split_lse.ndim == 4 and split_lse.shape[1:] == (1, num_heads, 1), (
        f"split_lse: expected [N, 1, {num_heads}, 1], got {list(split_lse.shape)}"
    )
    assert split_lse.size(0) == num_partial, (
        f"split_lse batch dim ({split_lse.size(0)}) != split_output batch dim ({num_partial})"
    )
    dev = query.device
    for name, t in [("kv_buffer", kv_buffer), ("kv_page_indices", kv_page_indices), ("work_indptr", work_indptr),
                    ("work_info_set", work_info_set), ("final_output", final_output),
                    ("split_output", split_output), ("split_lse", split_lse)]:
        assert t.device == dev, f"{name}: expected device {dev}, got {t.device}"
    for name, t in [("final_output", final_output), ("split_output", split_output), ("split_lse", split_lse)]:
        assert t.is_contiguous(), (
            f"{name}: must be contiguous (stride={list(t.stride())}, shape={list(t.shape)}); reshape() would "
            f"silently copy and the kernel's writes would not be visible to the caller"
        )
    # dtypes the kernel reads and writes (the reference's test allocates these)
    assert final_output.dtype == torch.bfloat16, f"final_output: expected bfloat16, got {final_output.dtype}"
    assert split_output.dtype == torch.float32 and split_lse.dtype == torch.float32, "split buffers must be float32"
    for name, t in [("kv_page_indices", kv_page_indices), ("work_indptr", work_indptr),
                    ("work_info_set", work_info_set)]:
        assert t.dtype == torch.int32, f"{name}: expected int32, got {t.dtype}"
    assert query.is_contiguous() and kv_buffer.is_contiguous(), "query and kv_buffer must be contiguous"
    if num_seqs == 0:
        return  # no query rows: nothing to decode or write
    if dev.type != "cuda":
        raise RuntimeError("flydsl_mla_fwd_decode: tensors must be on a GPU (the decode runs only in libpa_fp8.so)")

    kv_idx = kv_page_indices.contiguous()
    # gfx950's matrix cores read OCP e4m3fn only.  float8_e4m3fnuz inputs
    # (gfx942's format, which the reference's launcher also accepts) are
    # converted by value in one byte-wise pass of the library: exact for
    # |x| >= 2^-6, smaller magnitudes rounded to a multiple of 2^-9 (e4m3fn's
    # subnormal step; e4m3fnuz goes to 2^-10).  Only the kv rows the page
    # list names are converted, into a buffer of that many rows that the
    # decode then reads through the identity page list.
    if query.dtype == _FNUZ:
        query = _fnuz_rows_to_fn(query, None, query.shape)
    if kv_buffer.dtype == _FNUZ:
        n_idx = kv_idx.numel()
        kv_buffer = _fnuz_rows_to_fn(kv_buffer, kv_idx, (max(n_idx, 1),) + tuple(kv_buffer.shape[1:]))
        kv_idx = torch.arange(n_idx, dtype=torch.int32, device=dev)

    wi = work_info_set.contiguous().view(-1)
    wp = work_indptr.contiguous()
    a = _lib.MlaDecodeArgs()
    a.abi_version = _lib.ABI_VERSION
    a.query = query.data_ptr()
    a.kv_buffer = kv_buffer.data_ptr()
    a.kv_page_indices = kv_idx.data_ptr()
    a.work_indptr = wp.data_ptr()
    a.work_info = wi.data_ptr()
    a.final_output = final_output.data_ptr()
    a.split_output = split_output.data_ptr() if num_partial > 0 else None
    a.split_lse = split_lse.data_ptr() if num_partial > 0 else None
    a.num_pages = kv_buffer.size(0)
    a.num_page_indices = kv_idx.numel()
    a.num_rows = num_seqs
    a.num_workers = wp.numel() - 1
    a.num_works = wi.numel() // 8
    a.num_partial = num_partial
    a.softmax_scale = float(softmax_scale)
    a.precise_p = 1 if precise_p else 0
    rc = _lib.load().pa_fp8_mla_decode(ctypes.byref(a), _stream_handle(dev))
    _lib.check(rc, "pa_fp8_mla_decode")


def _fnuz_rows_to_fn(src: torch.Tensor, rows: Optional[torch.Tensor], shape) -> torch.Tensor:
    """e4m3fn tensor of ``shape`` (dense 576-byte rows): row i = the 576-byte
    row ``rows[i]`` of ``src`` (row i when ``rows`` is None), converted from
    e4m3fnuz by the library's byte-wise kernel."""
    dst = torch.empty(shape, dtype=torch.float8_e4m3fn, device=src.device)
    n = dst.numel() // QK_HEAD_DIM
    if rows is not None:
        n = min(n, rows.numel())
    rc = _lib.load().pa_fp8_fnuz_to_fn(src.data_ptr(), rows.data_ptr() if rows is not None else None, n,
                                      src.numel() // QK_HEAD_DIM, QK_HEAD_DIM, dst.data_ptr(),
                                      _stream_handle(src.device))
    _lib.check(rc, "pa_fp8_fnuz_to_fn")
    return dst


def get_mla_metadata_info_v1(
    batch_size: int,
    max_seqlen_qo: int,
    num_head_qo: int,
    q_dtype=None,
    kv_dtype=None,
    is_sparse: bool = False,
    fast_mode: bool = True,
    num_kv_splits: int = 32,
    intra_batch_mode: bool = False,
    *,
    num_cu: Optional[int] = None,
):
    """(size, dtype) of the six metadata buffers, in the order the
    reference's test unpacks them (tests/kernels/test_mla_decode.py:252-272):
    work_meta_data, work_indptr, work_info_set, reduce_indptr,
    reduce_final_map, reduce_partial_map.  One worker per CU."""
    if is_sparse or intra_batch_mode:
        raise NotImplementedError("get_mla_metadata_info_v1: sparse and intra-batch modes are not supported")
    if num_head_qo != NUM_QO_HEADS:
        raise NotImplementedError(f"get_mla_metadata_info_v1: num_head_qo={num_head_qo}, expected {NUM_QO_HEADS}")
    workers = int(num_cu if num_cu is not None else _num_cu())
    rows = int(batch_size) * int(max_seqlen_qo)
    max_works, max_partials = _lib.mla_plan_sizes(rows, workers)
    i32 = torch.int32
    return (
        ((4,), i32),
        ((workers + 1,), i32),
        ((max(max_works, 1), 8), i32),
        ((rows + 1,), i32),
        ((max(rows, 1), 2), i32),
        ((max(max_partials, 1),), i32),
    )


def get_mla_metadata_v1(
    qo_indptr: torch.Tensor,
    kv_indptr: torch.Tensor,
    kv_last_page_lens: torch.Tensor,
    num_heads_per_head_k: int,
    num_heads_k: int,
    is_causal: bool,
    work_metadata: torch.Tensor,
    work_info_set: torch.Tensor,
    work_indptr: torch.Tensor,
    reduce_indptr: torch.Tensor,
    reduce_final_map: torch.Tensor,
    reduce_partial_map: torch.Tensor,
    kv_granularity: int = 16,
    max_seqlen_qo: int = 1,
    uni_seqlen_qo: int = 1,
    fast_mode: bool = True,
    max_split_per_batch: int = 32,
    intra_batch_mode: bool = False,
    dtype_q=None,
    dtype_kv=None,
) -> None:
    """Fill the work list for ``flydsl_mla_fwd_decode`` (call site:
    tests/kernels/test_mla_decode.py:274-295).  Planned on the host (the
    indptr tensors are copied down, one synchronisation): every query row
    attends pages kv_indptr[b] .. kv_indptr[b+1] (page size 1, so
    ``kv_last_page_lens`` must be 1 for every non-empty sequence); its
    128-token blocks are dealt to ``work_indptr.numel() - 1`` workers in
    balanced contiguous runs; rows cut across workers get partial rows and
    a reduce group.  ``work_metadata`` receives (works, groups, partial rows,
    workers).  ``kv_granularity``, ``fast_mode`` and ``max_split_per_batch``
    are accepted for signature compatibility; the block size is fixed."""
    if num_heads_k != 1 or num_heads_per_head_k != NUM_QO_HEADS:
        raise NotImplementedError(
            f"get_mla_metadata_v1: expected 1 kv head x {NUM_QO_HEADS} query heads, "
            f"got {num_heads_k} x {num_heads_per_head_k}"
        )
    if intra_batch_mode:
        raise NotImplementedError("get_mla_metadata_v1: intra-batch mode is not supported")
    qo = qo_indptr.detach().to("cpu", torch.int32).numpy()
    kv = kv_indptr.detach().to("cpu", torch.int32).numpy()
    lp = kv_last_page_lens.detach().to("cpu", torch.int32).numpy()
    pages = kv[1:] - kv[:-1]
    if ((pages > 0) & (lp != 1)).any():
        raise ValueError("get_mla_metadata_v1: page size 1 expects kv_last_page_lens == 1")
    workers = work_indptr.numel() - 1
    n, ng, npart, out = _lib.mla_plan(qo, kv, workers)
    if work_info_set.numel() < 8 * max(n, 1) or reduce_partial_map.numel() < max(npart, 1):
        raise ValueError("get_mla_metadata_v1: buffers smaller than get_mla_metadata_info_v1 sizes")
    rows = reduce_indptr.numel() - 1
    if rows < int(qo[-1] - qo[0]):
        raise ValueError("get_mla_metadata_v1: reduce_indptr smaller than the number of query rows + 1")

    def put(dst: torch.Tensor, src):
        t = torch.from_numpy(src.reshape(-1)[: dst.numel()].copy())
        flat = dst.view(-1)
        flat.zero_()
        flat[: t.numel()].copy_(t.to(dst.device))

    put(work_indptr, out["work_indptr"])
    put(work_info_set, out["work_info"])
    ri = out["reduce_indptr"]
    put(reduce_indptr, ri)
    put(reduce_final_map, out["reduce_final_map"])
    put(reduce_partial_map, out["reduce_partial_map"])
    if work_metadata.numel() > 0:
        import numpy as np

        put(work_metadata, np.array([n, ng, npart, workers], np.int32))


def mla_reduce_v1(
    partial_output: torch.Tensor,  # [num_partial, 1, num_heads, 512] float32
    partial_lse: torch.Tensor,  # [num_partial, 1, num_heads, 1] float32
    reduce_indptr: torch.Tensor,
    reduce_final_map: torch.Tensor,
    reduce_partial_map: torch.Tensor,
    max_seqlen_qo: int,
    final_output: torch.Tensor,  # [num_rows, num_heads, 512] bf16
    final_lse: Optional[torch.Tensor] = None,  # [num_rows, num_heads] float32
) -> None:
    """Log-sum-exp merge of the split rows into ``final_output`` (call site:
    tests/kernels/test_mla_decode.py:356-365).  Every reduce group slot is
    launched; empty ones exit, so no host synchronisation is needed."""
    assert partial_output.dtype == torch.float32 and partial_lse.dtype == torch.float32
    assert final_output.dtype == torch.bfloat16 and final_output.is_contiguous()
    assert partial_output.is_contiguous() and partial_lse.is_contiguous()
    assert final_output.size(-1) == V_HEAD_DIM and final_output.size(-2) == NUM_QO_HEADS
    for name, t in [("reduce_indptr", reduce_indptr), ("reduce_final_map", reduce_final_map),
                    ("reduce_partial_map", reduce_partial_map)]:
        assert t.dtype == torch.int32 and t.is_contiguous(), f"{name}: expected contiguous int32"
    assert reduce_final_map.numel() >= 2 * (reduce_indptr.numel() - 1), "reduce_final_map: one (row0, row1) per group"
    dev = final_output.device
    if dev.type != "cuda":
        raise RuntimeError("mla_reduce_v1: tensors must be on a GPU")
    if final_lse is not None:
        assert final_lse.dtype == torch.float32 and final_lse.is_contiguous()
    r = _lib.MlaReduceArgs()
    r.abi_version = _lib.ABI_VERSION
    r.split_output = partial_output.data_ptr()
    r.split_lse = partial_lse.data_ptr()
    r.reduce_indptr = reduce_indptr.data_ptr()
    r.reduce_final_map = reduce_final_map.data_ptr()
    r.reduce_partial_map = reduce_partial_map.data_ptr()
    r.final_output = final_output.data_ptr()
    r.final_lse = final_lse.data_ptr() if final_lse is not None else None
    r.num_groups = reduce_indptr.numel() - 1
    r.num_partial = partial_output.numel() // (NUM_QO_HEADS * V_HEAD_DIM)
    r.num_partial_map = reduce_partial_map.numel()
    r.num_rows = final_output.numel() // (NUM_QO_HEADS * V_HEAD_DIM)
    rc = _lib.load().pa_fp8_mla_reduce(ctypes.byref(r), _stream_handle(dev))
    _lib.check(rc, "pa_fp8_mla_reduce")
