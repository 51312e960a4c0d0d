"""Host launcher of the MI355X FP8 paged-attention decode.

Drop-in for the reference's Python API in kernels/pa_decode_fp8.py:
``pa_decode_ps_launch`` (:2812-3202), ``get_recommended_splits``
(:1922-1949) and ``get_pa_metadata`` (:1729-1859).  Same argument names,
defaults, tensor layouts, validation errors and route strings; the device
work is done by the HIP kernels of ``libpa_fp8.so`` through its C ABI.

Scheduling (see ``_schedule`` and ``_balanced_ok``): when the batch has
enough (sequence, kv head) pairs and bounded contexts, one workgroup per
pair walks all of its slots and merges them itself (one launch).  When the
caller does not ask for the slot partials and the contexts may be long or
ragged, every wave of the GPU takes an equal run of the batch's chunks
(balanced stream split, a decode launch plus a merge launch).  Otherwise
workgroups take one or a few slots each and the reduce kernel merges them.

``exp_sums`` / ``max_logits`` / ``temporary_output`` are workspace, as in
the reference (preallocated so that graph capture allocates nothing,
:2898-2902, :3030-3034): the slot routes write the reference's slot
partials into them and the reduce reads them back; an owner launch, which
merges in LDS, leaves them untouched.  (The C ABI still writes them from an
owner launch when its arguments carry them.)

Routes (same dispatch order as the reference, :2883 / :3010 / :3123):
  * ``sliding_window > 0``    -> window partition pass + LSE reduce
                                 ("ps_sw_partitioned"), or the fused
                                 single-slot pass ("ps_sw_fused_partitioned")
                                 when only one slot is asked for.  Works for
                                 every supported page size (the reference
                                 kernel is correct for 1024-token pages only,
                                 kernels/pa_decode_swa.py:1228).
  * page size 16 or 64        -> split-context partition pass + LSE reduce
                                 ("ps_small_block").
  * other page sizes (1024)   -> flat ``kv_page_indices``/``kv_indptr``
                                 page list ("ps_split_reduce"): with the
                                 ``metadata`` of :func:`get_pa_metadata`, the
                                 work-list decode + its reduce, as the
                                 reference's persistent route; without it,
                                 the balanced split or the partition pass.
"""

from __future__ import annotations

import ctypes
import functools
import math
from typing import Optional

import torch

from . import _lib
from ._lib import DTYPE_BF16, DTYPE_F16, DTYPE_F32

KV_COMPUTE_BLOCK = 256  # tokens per context sub-partition
_PA_DECODE_PS_SMALL_BLOCK_SIZES = (16, 64)

_PACKED_FP8_QUERY_DTYPES = tuple(
    d
    for d in (
        torch.uint8,
        getattr(torch, "float8_e4m3fn", None),
        getattr(torch, "float8_e4m3fnuz", None),
    )
    if d is not None
)


def _cdiv(a: int, b: int) -> int:
    return -(-a // b)


@functools.lru_cache(maxsize=None)
def _device_cu_count(index: int) -> int:
    return int(torch.cuda.get_device_properties(index).multi_processor_count)


def _cu_count(device: Optional[torch.device] = None) -> int:
    dev = torch.device("cuda") if device is None else torch.device(device)
    idx = dev.index if dev.index is not None else torch.cuda.current_device()
    return _device_cu_count(idx)


def get_recommended_splits(
    num_sequences: int,
    num_kv_heads: int,
    split_kv_blocks: int = 1,
    *,
    sliding_window: int = 0,
    context_partition_size: int = KV_COMPUTE_BLOCK,
    query_length: int = 1,
    num_cu: Optional[int] = None,
) -> int:
    """Slots (``max_context_partition_num``) for the partitioned routes.

    Same result as the reference (kernels/pa_decode_fp8.py:1922-1949): for a
    window, ``cdiv(W + ql - 1, cps) + 1``; otherwise two workgroups per CU
    spread over ``B * Hkv * split_kv_blocks`` units, clamped to [4, 8].
    ``num_cu`` defaults to the current device's CU count (256 on MI355X);
    pass it to plan without a GPU.
    """
    if sliding_window > 0:
        cu = 1
    else:
        cu = num_cu if num_cu is not None else _cu_count()
    return _lib.recommended_splits(
        int(num_sequences),
        int(num_kv_heads),
        int(split_kv_blocks),
        int(sliding_window),
        int(context_partition_size),
        int(query_length),
        int(cu),
    )


def _is_current_stream_capturing() -> bool:
    if not torch.cuda.is_available():
        return False
    try:
        return torch.cuda.is_current_stream_capturing()
    except RuntimeError:
        return False


def _prepare_scale_tensor(name: str, scale, *, device: torch.device, is_graph_capturing: bool) -> torch.Tensor:
    """float / tensor -> float32 tensor on ``device`` (kernels/pa_decode_fp8.py:1871-1895)."""
    if isinstance(scale, torch.Tensor):
        if is_graph_capturing:
            if scale.device != device:
                raise ValueError(f"CUDA graph capture requires `{name}` to already be on {device}, got {scale.device}.")
            if scale.dtype != torch.float32:
                raise ValueError(f"CUDA graph capture requires `{name}` to already be float32, got {scale.dtype}.")
            return scale
        return scale.to(device=device, dtype=torch.float32)
    if is_graph_capturing:
        raise ValueError(
            f"CUDA graph capture requires `{name}` to be passed as a pre-created float32 tensor on the target device."
        )
    return torch.tensor([float(scale or 1.0)], device=device, dtype=torch.float32)


def _get_query_input_dtype(query: torch.Tensor) -> str:
    if query.dtype in _PACKED_FP8_QUERY_DTYPES:
        return "packed_fp8"
    if query.dtype == torch.bfloat16:
        return "bf16"
    if query.dtype == torch.float16:
        return "f16"
    raise ValueError(
        f"Unsupported query dtype for pa_decode_ps_launch: {query.dtype}. Expected packed FP8/uint8, bf16, or f16."
    )


def _get_output_dtype_code(output: torch.Tensor) -> int:
    if output.dtype == torch.bfloat16:
        return DTYPE_BF16
    if output.dtype == torch.float16:
        return DTYPE_F16
    if output.dtype == torch.float32:
        return DTYPE_F32
    raise ValueError(
        f"Unsupported output dtype for pa_decode_ps_launch reduce: {output.dtype}. Expected bf16, f16, or f32."
    )


def _tmp_dtype_code(t: torch.Tensor) -> int:
    if t.dtype == torch.bfloat16:
        return DTYPE_BF16
    if t.dtype == torch.float32:
        return DTYPE_F32
    raise ValueError(f"temporary_output must be bfloat16 or float32, got {t.dtype}")


def _check_int32(name: str, t: torch.Tensor, device: torch.device) -> None:
    if t.dtype != torch.int32:
        raise ValueError(f"`{name}` must be int32, got {t.dtype}")
    if t.device != device:
        raise ValueError(f"`{name}` must be on {device}, got {t.device}")


def _check_partials(exp_sums, max_logits, tmp, shape, head_size):
    if tuple(exp_sums.shape) != shape or tuple(max_logits.shape) != shape:
        raise ValueError(f"exp_sums/max_logits must have shape {shape}, got {tuple(exp_sums.shape)}")
    if tuple(tmp.shape) != shape + (head_size,):
        raise ValueError(f"temporary_output must have shape {shape + (head_size,)}, got {tuple(tmp.shape)}")
    if exp_sums.dtype != torch.float32 or max_logits.dtype != torch.float32:
        raise ValueError("exp_sums and max_logits must be float32")
    if exp_sums.stride() != max_logits.stride() or exp_sums.stride(-1) != 1:
        raise ValueError("exp_sums and max_logits must share strides with a contiguous last dimension")
    if tmp.stride(-1) != 1:
        raise ValueError("temporary_output must be contiguous in its last dimension")


# A workgroup that owns a whole (sequence, kv head) streams at most this many
# tokens; beyond it the slots are spread over workgroups (slot mode).
OWNER_MAX_CONTEXT = 8192
WAVES_PER_WORKGROUP = 4


def _schedule(route: str, batch: int, kv_heads: int, P: int, eqgs: int, capacity: Optional[int], num_cu: int):
    """Slots per workgroup for one call.

    Owner mode (slots_per_workgroup = P): one workgroup per (sequence, kv
    head) streams every slot and merges them in LDS, so one launch finishes
    the decode; used when there are enough (sequence, kv head) pairs to fill
    the GPU and no sequence can be long (its workgroup would set the
    kernel's duration).  Slot mode otherwise: one slot per wave when slots
    are short, else the four waves share a slot; a reduce launch merges.
    """
    ncg = -(-eqgs // 16)
    if P == 1:
        return 1
    multi_ok = ncg == 1 or P <= WAVES_PER_WORKGROUP
    if route == "sw" and batch * kv_heads >= num_cu and multi_ok:
        return P  # a window bounds every (sequence, kv head)'s work
    if (route != "flat" and capacity is not None and capacity <= OWNER_MAX_CONTEXT
            and batch * kv_heads >= 2 * num_cu and multi_ok):
        return P
    if route == "sw":
        slot_tokens = KV_COMPUTE_BLOCK
    elif capacity is None:
        return 1
    else:
        slot_tokens = -(-(-(-capacity // KV_COMPUTE_BLOCK)) // P) * KV_COMPUTE_BLOCK
    if slot_tokens <= 16 * 32 and P >= WAVES_PER_WORKGROUP:
        return WAVES_PER_WORKGROUP
    return 1


# Balanced stream split: per-wave runs for at most BALANCED_MAX_COLUMNS query
# columns per kv head (the per-wave query images then leave room for two
# workgroups per CU), cooperative workgroup runs above STREAM_MAX_COLUMNS
# (one wave per 16-column block), up to this many sequences (the in-kernel
# split scans them in one pass).
BALANCED_MAX_COLUMNS = 4
# Head sizes the library decodes (128 on the tuned kernels, the others and
# more than COOP_MAX_COLUMNS columns per kv head on the generic ones).
GENERIC_HEAD_SIZES = tuple(range(64, 513, 64))  # 64, 128, ..., 512
BALANCED_MAX_SEQS = 1024
# Per-wave streaming decode: one 16-column query block; cooperative beyond.
STREAM_MAX_COLUMNS = 16
COOP_MAX_COLUMNS = 64


# A generic-kernel owner launch runs one wave per (sequence, kv head,
# 16-column block), each walking every slot in turn; with fewer waves than
# this per CU it leaves SIMDs idle and the slot launch (a workgroup per slot)
# plus the LSE reduce is faster (C2's batch at head size 64: 119 -> 57 us).
GENERIC_OWNER_MIN_WAVES_PER_CU = 8


def _generic_owner_ok(batch: int, kv_heads: int, eqgs: int, num_cu: int) -> bool:
    """Whether a generic-kernel owner launch fills the GPU."""
    return batch * kv_heads * -(-eqgs // 16) >= GENERIC_OWNER_MIN_WAVES_PER_CU * num_cu


def _balanced_ok(route: str, batch: int, eqgs: int, user_partials: bool, owner: bool) -> bool:
    """Balanced stream split for a call whose slot partials nobody reads:
    every wave (or, for more than 16 query columns, every cooperative
    workgroup) gets an equal run of the batch's chunks, so one long sequence
    no longer sets the duration.  Up to 16 columns the owner schedule keeps
    the calls it takes (one launch, nothing to merge)."""
    if route not in ("small", "flat") or user_partials or not 0 < batch <= BALANCED_MAX_SEQS:
        return False
    if eqgs <= BALANCED_MAX_COLUMNS:
        return not owner
    return STREAM_MAX_COLUMNS < eqgs <= COOP_MAX_COLUMNS


class PreparedDecode:
    """A validated decode call whose C-ABI arguments are already marshalled.

    ``launch()`` issues exactly the device work ``pa_decode_ps_launch`` would
    (partition pass [+ reduce], balanced decode + merge, or work-list decode
    + reduce) without re-validating or rebuilding arguments; the tensors
    captured at preparation must stay alive and unchanged in shape.
    """

    def __init__(self, route: str, stream, keepalive, *, partition_args=None, reduce_args=None, stream_args=None,
                 worklist_reduce_args=None, workspace=None):
        self.route = route
        self._pa = partition_args
        self._ra = reduce_args
        self._sa = stream_args
        self._wra = worklist_reduce_args
        self._ws = workspace
        self._keep = keepalive
        if stream is None:  # an empty batch: nothing to launch, no library needed
            self._stream = self._lib = None
            self._kernels = []
            return
        self._stream = ctypes.c_void_p(stream.cuda_stream)
        self._lib = _lib.load()
        self._kernels = self.kernels()

    @classmethod
    def empty(cls, route: str) -> "PreparedDecode":
        """The call for a batch of zero sequences: ``launch()`` issues no
        device work and returns the route the call would have taken."""
        return cls(route, None, ())

    def kernels(self):
        """The call's kernel launches in order, as (C entry point, thunk);
        the first is the decode kernel, a second one its merge.  The thunks
        hold the marshalled structs, not this object (no reference cycle:
        a call's buffers are released as soon as the call is dropped)."""
        lib, s = self._lib, self._stream
        pa, ra, sa, wra = self._pa, self._ra, self._sa, self._wra
        if pa is not None:
            out = [("pa_fp8_decode_partition", lambda: lib.pa_fp8_decode_partition(ctypes.byref(pa), s))]
            if ra is not None:
                out.append(("pa_fp8_decode_reduce", lambda: lib.pa_fp8_decode_reduce(ctypes.byref(ra), s)))
            return out
        if wra is not None:
            return [("pa_fp8_decode_worklist", lambda: lib.pa_fp8_decode_worklist(ctypes.byref(sa), s)),
                    ("pa_fp8_reduce_worklist", lambda: lib.pa_fp8_reduce_worklist(ctypes.byref(wra), s))]
        ws, n = self._ws.data_ptr(), self._ws.numel()
        return [("pa_fp8_decode_balanced", lambda: lib.pa_fp8_decode_balanced(ctypes.byref(sa), ws, n, s)),
                ("pa_fp8_merge_balanced", lambda: lib.pa_fp8_merge_balanced(ctypes.byref(sa), ws, n, s))]

    def launch(self) -> str:
        for name, fn in self._kernels:
            _lib.check(fn(), name)
        return self.route


def pa_decode_ps_launch(
    output: torch.Tensor,
    query: torch.Tensor,
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
    context_lengths: torch.Tensor,
    kv_page_indices: torch.Tensor,
    kv_indptr: torch.Tensor,
    softmax_scale: float,
    key_scale: torch.Tensor = None,
    value_scale: torch.Tensor = None,
    *,
    sliding_window: int = 0,
    metadata: dict = None,
    block_tables: torch.Tensor = None,
    max_context_partition_num: int = 0,
    exp_sums: torch.Tensor = None,
    max_logits: torch.Tensor = None,
    temporary_output: torch.Tensor = None,
    stream=None,
) -> str:
    """FP8 paged-attention decode (drop-in for kernels/pa_decode_fp8.py:2812).

    output [B*ql, Hq, D] (bf16/f16/f32) is written in place.  query
    [B*ql, Hq, D] bf16/f16; key_cache [NB, Hkv, D/16, bs, 16] fp8; value_cache
    trans [NB, Hkv, bs/16, D, 16] (or [NB, Hkv, D, bs]); context_lengths [B]
    int32; block_tables [B, max_blocks] int32 (page sizes 16/64 and windows);
    kv_page_indices / kv_indptr: flat page list (other page sizes).
    key/value_scale: float, [1] tensor (per tensor) or [NB, Hkv, bs, 1]
    (per token per head).  Returns the route name.
    """
    call = prepare_pa_decode(
        output, query, key_cache, value_cache, context_lengths, kv_page_indices, kv_indptr, softmax_scale,
        key_scale, value_scale, sliding_window=sliding_window, metadata=metadata, block_tables=block_tables,
        max_context_partition_num=max_context_partition_num, exp_sums=exp_sums, max_logits=max_logits,
        temporary_output=temporary_output, stream=stream,
    )
    return call.launch()


def prepare_pa_decode(
    output: torch.Tensor,
    query: torch.Tensor,
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
    context_lengths: torch.Tensor,
    kv_page_indices: torch.Tensor,
    kv_indptr: torch.Tensor,
    softmax_scale: float,
    key_scale: torch.Tensor = None,
    value_scale: torch.Tensor = None,
    *,
    sliding_window: int = 0,
    metadata: dict = None,
    block_tables: torch.Tensor = None,
    max_context_partition_num: int = 0,
    exp_sums: torch.Tensor = None,
    max_logits: torch.Tensor = None,
    temporary_output: torch.Tensor = None,
    stream=None,
) -> PreparedDecode:
    """Validate and marshal one decode call (same arguments and errors as
    :func:`pa_decode_ps_launch`); returns a :class:`PreparedDecode`."""
    num_query_heads = query.shape[1]
    num_kv_heads = key_cache.shape[1]
    trans_v = value_cache.dim() == 5
    query_input_dtype = _get_query_input_dtype(query)
    dev = query.device
    is_graph_capturing = _is_current_stream_capturing()

    key_scale = _prepare_scale_tensor("key_scale", key_scale, device=dev, is_graph_capturing=is_graph_capturing)
    value_scale = _prepare_scale_tensor("value_scale", value_scale, device=dev, is_graph_capturing=is_graph_capturing)
    if query_input_dtype == "packed_fp8":
        raise ValueError(
            "`pa_decode_ps_launch` no longer accepts host query_scale and only supports "
            "bf16/f16 query inputs with kernel-internal query scale computation."
        )
    per_token_kv = key_scale.dim() > 1

    batch_size = int(context_lengths.shape[0])
    # A batch of zero sequences decodes nothing (the reference divides by the
    # batch size here); it is validated like any other call, then launches
    # no kernel.
    query_length = query.shape[0] // batch_size if batch_size else 0
    if query_length * batch_size != query.shape[0]:
        raise ValueError(f"query rows ({query.shape[0]}) must be a multiple of the batch size ({batch_size})")
    if num_query_heads % num_kv_heads != 0:
        raise ValueError("Query heads must be divisible by KV heads")
    query_group_size = num_query_heads // num_kv_heads
    head_size = int(query.shape[-1])
    if head_size % 64 != 0:
        raise ValueError(f"Unsupported head_dim={head_size}; must be a multiple of 64.")
    if head_size not in GENERIC_HEAD_SIZES:
        raise NotImplementedError(
            f"head_dim={head_size} is not built; this library supports head_dim in {GENERIC_HEAD_SIZES} "
            "(larger heads would not fit one wave's register file).")
    eqgs = query_length * query_group_size
    # head sizes other than 128 and more than 64 query columns per kv head
    # run on the library's generic kernels: no balanced split for them
    generic = head_size != 128 or eqgs > COOP_MAX_COLUMNS
    block_size = int(key_cache.shape[-2])
    if tuple(key_cache.shape[2:]) != (head_size // 16, block_size, 16):
        raise ValueError(f"key_cache must be [NB, Hkv, {head_size // 16}, bs, 16], got {tuple(key_cache.shape)}")
    if key_cache.element_size() != 1 or value_cache.element_size() != 1:
        raise ValueError("key_cache and value_cache must be 1-byte fp8 (e4m3fn) tensors")
    if trans_v:
        if tuple(value_cache.shape[2:]) != (block_size // 16, head_size, 16):
            raise ValueError(f"trans value_cache must be [NB, Hkv, bs/16, D, 16], got {tuple(value_cache.shape)}")
    elif tuple(value_cache.shape[2:]) != (head_size, block_size):
        raise ValueError(f"value_cache must be [NB, Hkv, D, bs], got {tuple(value_cache.shape)}")
    for t, name in ((key_cache, "key_cache"), (value_cache, "value_cache"), (query, "query"), (output, "output")):
        if t.stride(-1) != 1:
            raise ValueError(f"`{name}` must be contiguous in its last dimension")
    if tuple(output.shape) != tuple(query.shape):
        raise ValueError(f"output shape {tuple(output.shape)} must match query shape {tuple(query.shape)}")
    if per_token_kv:
        if key_scale.dim() != 4 or tuple(key_scale.shape[:3]) != (key_cache.shape[0], num_kv_heads, block_size):
            raise ValueError(f"per-token key_scale must be [NB, Hkv, bs, 1], got {tuple(key_scale.shape)}")
        if key_scale.stride() != value_scale.stride() or key_scale.stride(2) != 1:
            raise ValueError("key_scale and value_scale must share strides with a contiguous token dimension")
    output_dtype = _get_output_dtype_code(output)
    _check_int32("context_lengths", context_lengths, dev)
    if batch_size == 0:
        if sliding_window > 0:
            return PreparedDecode.empty(
                "ps_sw_fused_partitioned" if max_context_partition_num == 1 else "ps_sw_partitioned")
        return PreparedDecode.empty(
            "ps_small_block" if block_size in _PA_DECODE_PS_SMALL_BLOCK_SIZES else "ps_split_reduce")

    s = stream or torch.cuda.current_stream(dev)

    kv_ind = None
    if sliding_window > 0:
        route = "sw"
        if block_tables is None:
            raise ValueError("pa_decode_ps_launch: sliding_window > 0 requires `block_tables`.")
        needed = get_recommended_splits(
            batch_size,
            num_kv_heads,
            sliding_window=sliding_window,
            context_partition_size=KV_COMPUTE_BLOCK,
            query_length=query_length,
        )
        if max_context_partition_num == 0:
            max_context_partition_num = needed
        elif 1 < max_context_partition_num < needed:
            raise ValueError(
                f"max_context_partition_num={max_context_partition_num} cannot cover a window of {sliding_window} "
                f"tokens (needs {needed} slots)."
            )
    elif block_size in _PA_DECODE_PS_SMALL_BLOCK_SIZES:
        route = "small"
        if block_tables is None:
            raise ValueError(
                f"pa_decode_ps_launch: block_size={block_size} requires `block_tables` "
                "(per-sequence physical block index table)."
            )
        if max_context_partition_num == 0:
            max_context_partition_num = get_recommended_splits(
                batch_size, num_kv_heads, split_kv_blocks=KV_COMPUTE_BLOCK // block_size
            )
    else:
        route = "flat"
        if kv_page_indices is None or kv_indptr is None:
            raise ValueError(f"pa_decode_ps_launch: block_size={block_size} requires `kv_page_indices` and `kv_indptr`.")
        _check_int32("kv_page_indices", kv_page_indices, dev)
        _check_int32("kv_indptr", kv_indptr, dev)
        if is_graph_capturing and metadata is None and (exp_sums is None or max_logits is None or temporary_output is None):
            raise ValueError(
                "CUDA graph capture requires precomputed `metadata`; "
                "call `get_pa_metadata()` before capture and pass it via `metadata=`."
            )
        if max_context_partition_num == 0:
            max_context_partition_num = get_recommended_splits(batch_size, num_kv_heads, split_kv_blocks=1)
        kv_ind = kv_indptr
        if metadata is not None:
            return _prepare_worklist(
                metadata, output, query, key_cache, value_cache, context_lengths, kv_page_indices, kv_indptr,
                softmax_scale, key_scale, value_scale, per_token_kv, trans_v, query_input_dtype, output_dtype, s)
    if route != "flat":
        _check_int32("block_tables", block_tables, dev)
        if block_tables.dim() != 2 or block_tables.stride(-1) != 1:
            raise ValueError("block_tables must be a 2-D int32 tensor with a contiguous last dimension")
    P = int(max_context_partition_num)

    capacity = None if route == "flat" else int(block_tables.shape[1]) * block_size
    spw = _schedule(route, batch_size, num_kv_heads, P, eqgs, capacity, _cu_count(dev) if P > 1 else 1)
    owner = spw >= P
    user_partials = exp_sums is not None or max_logits is not None or temporary_output is not None
    have_partials = exp_sums is not None and max_logits is not None and temporary_output is not None
    if (generic and owner and P > 1 and not (is_graph_capturing and not have_partials)
            and not _generic_owner_ok(batch_size, num_kv_heads, eqgs, _cu_count(dev))):
        spw, owner = 1, False
    if not generic and _balanced_ok(route, batch_size, eqgs, user_partials, owner):
        route_name = "ps_small_block" if route == "small" else "ps_split_reduce"
        sa = _stream_args(output, query, key_cache, value_cache, context_lengths,
                          kv_page_indices if route == "flat" else block_tables, kv_ind, softmax_scale, key_scale,
                          value_scale, per_token_kv, trans_v, query_input_dtype, output_dtype, sliding_window)
        sa.num_workers = _lib.stream_workers(_cu_count(dev), query_length, query_group_size, per_token_kv)
        nbytes = _lib.balanced_workspace_bytes(batch_size, num_kv_heads, query_length, query_group_size,
                                               sa.num_workers)
        ws = torch.empty(nbytes, dtype=torch.uint8, device=dev)
        keep = (output, query, key_cache, value_cache, context_lengths, block_tables, kv_page_indices, kv_indptr,
                key_scale, value_scale, ws)
        return PreparedDecode(route_name, s, keep, stream_args=sa, workspace=ws)
    # An owner launch needs no slot partials; caller buffers stay unused
    # (validated all the same, as the slot routes validate them).
    if exp_sums is not None and max_logits is not None and temporary_output is not None:
        _check_partials(exp_sums, max_logits, temporary_output, (batch_size, num_kv_heads, P, eqgs), head_size)
    fused = owner
    if fused and route != "sw":
        # Nobody observes the slot partials: let each of the workgroup's
        # waves stream one contiguous quarter of the context.  (The window
        # route keeps its 256-token tiles, whose layout its slots define.)
        P = spw = min(P, WAVES_PER_WORKGROUP)
    shape = (batch_size, num_kv_heads, P, eqgs)
    if not fused:
        if not owner and is_graph_capturing and (exp_sums is None or max_logits is None or temporary_output is None):
            which = "sliding-window" if route == "sw" else "small-block PS"
            raise ValueError(
                "CUDA graph capture requires preallocated `exp_sums`, `max_logits`, "
                f"and `temporary_output` for the {which} path."
            )
        # Every slot writes all of its cells (empty slots write 0 / -inf /
        # zeros), so uninitialised buffers are fine: no fill kernels.
        if exp_sums is None:
            exp_sums = torch.empty(shape, device=dev, dtype=torch.float32)
        if max_logits is None:
            max_logits = torch.empty(shape, device=dev, dtype=torch.float32)
        if temporary_output is None:
            temporary_output = torch.empty(shape + (head_size,), device=dev, dtype=torch.bfloat16)
        _check_partials(exp_sums, max_logits, temporary_output, shape, head_size)

    pa = _lib.PartitionArgs()
    pa.abi_version = _lib.ABI_VERSION
    pa.query = query.data_ptr()
    pa.key_cache = key_cache.data_ptr()
    pa.value_cache = value_cache.data_ptr()
    if route == "flat":
        pa.block_tables = kv_page_indices.data_ptr()
        pa.kv_indptr = kv_ind.data_ptr()
        pa.stride_bt_seq = 0
        pa.max_blocks_per_seq = max(1, int(kv_page_indices.numel()))
    else:
        pa.block_tables = block_tables.data_ptr()
        pa.kv_indptr = None
        pa.stride_bt_seq = block_tables.stride(0)
        pa.max_blocks_per_seq = int(block_tables.shape[1])
    pa.context_lengths = context_lengths.data_ptr()
    pa.key_scale = key_scale.data_ptr()
    pa.value_scale = value_scale.data_ptr()
    pa.stride_q_tok, pa.stride_q_head = query.stride(0), query.stride(1)
    pa.stride_k_block, pa.stride_k_head = key_cache.stride(0), key_cache.stride(1)
    pa.stride_v_block, pa.stride_v_head = value_cache.stride(0), value_cache.stride(1)
    if per_token_kv:
        pa.stride_ks_block, pa.stride_ks_head = key_scale.stride(0), key_scale.stride(1)
    pa.num_seqs = batch_size
    pa.num_kv_heads = num_kv_heads
    pa.num_partitions = P
    pa.query_length = query_length
    pa.query_group_size = query_group_size
    pa.head_size = head_size
    pa.block_size = block_size
    pa.num_blocks = int(key_cache.shape[0])
    pa.sliding_window = int(sliding_window)
    pa.per_token_kv = int(per_token_kv)
    pa.trans_v = int(trans_v)
    pa.query_dtype = DTYPE_BF16 if query_input_dtype == "bf16" else DTYPE_F16
    pa.softmax_scale = float(softmax_scale)
    pa.slots_per_workgroup = spw
    if owner:
        pa.output = output.data_ptr()
        pa.output_dtype = output_dtype
        pa.stride_out_tok, pa.stride_out_head = output.stride(0), output.stride(1)
    if fused:
        pa.tmp_dtype = DTYPE_BF16
    else:
        pa.exp_sums = exp_sums.data_ptr()
        pa.max_logits = max_logits.data_ptr()
        pa.tmp_out = temporary_output.data_ptr()
        pa.stride_es_seq, pa.stride_es_head, pa.stride_es_part = exp_sums.stride()[:3]
        (pa.stride_to_seq, pa.stride_to_head, pa.stride_to_part, pa.stride_to_group) = temporary_output.stride()[:4]
        pa.tmp_dtype = _tmp_dtype_code(temporary_output)
    keep = (output, query, key_cache, value_cache, context_lengths, block_tables, kv_page_indices, kv_indptr,
            key_scale, value_scale, exp_sums, max_logits, temporary_output)
    route_name = {"sw": "ps_sw_partitioned", "small": "ps_small_block", "flat": "ps_split_reduce"}[route]
    if route == "sw" and P <= 1:
        route_name = "ps_sw_fused_partitioned"
    if owner:
        return PreparedDecode(route_name, s, keep, partition_args=pa)

    ra = _lib.ReduceArgs()
    ra.abi_version = _lib.ABI_VERSION
    ra.output = output.data_ptr()
    ra.exp_sums = exp_sums.data_ptr()
    ra.max_logits = max_logits.data_ptr()
    ra.tmp_out = temporary_output.data_ptr()
    # output [B*ql, Hq, D] addressed as [B, ql, Hkv, gqa, D]
    so0, so1 = output.stride(0), output.stride(1)
    ra.stride_out_seq, ra.stride_out_ql = query_length * so0, so0
    ra.stride_out_kv_head, ra.stride_out_group = query_group_size * so1, so1
    ra.stride_es_seq, ra.stride_es_head, ra.stride_es_part = exp_sums.stride()[:3]
    (ra.stride_to_seq, ra.stride_to_head, ra.stride_to_part, ra.stride_to_group) = temporary_output.stride()[:4]
    ra.num_seqs = batch_size
    ra.num_kv_heads = num_kv_heads
    ra.num_partitions = P
    ra.query_length = query_length
    ra.query_group_size = query_group_size
    ra.head_size = head_size
    ra.output_dtype = output_dtype
    ra.tmp_dtype = _tmp_dtype_code(temporary_output)
    return PreparedDecode(route_name, s, keep, partition_args=pa, reduce_args=ra)


def _stream_args(output, query, key_cache, value_cache, context_lengths, pages, kv_indptr, softmax_scale, key_scale,
                 value_scale, per_token_kv, trans_v, query_input_dtype, output_dtype, sliding_window=0):
    """C-ABI arguments shared by the balanced and work-list decodes.
    ``pages`` is the [B, max_blocks] block table, or the flat page list
    when ``kv_indptr`` is given."""
    sa = _lib.StreamArgs()
    sa.abi_version = _lib.ABI_VERSION
    sa.output = output.data_ptr()
    sa.query = query.data_ptr()
    sa.key_cache = key_cache.data_ptr()
    sa.value_cache = value_cache.data_ptr()
    sa.block_tables = pages.data_ptr()
    sa.context_lengths = context_lengths.data_ptr()
    sa.key_scale = key_scale.data_ptr()
    sa.value_scale = value_scale.data_ptr()
    if kv_indptr is not None:
        sa.kv_indptr = kv_indptr.data_ptr()
        sa.max_blocks_per_seq = max(1, int(pages.numel()))
    else:
        sa.stride_bt_seq = pages.stride(0)
        sa.max_blocks_per_seq = int(pages.shape[1])
    sa.stride_q_tok, sa.stride_q_head = query.stride(0), query.stride(1)
    sa.stride_k_block, sa.stride_k_head = key_cache.stride(0), key_cache.stride(1)
    sa.stride_v_block, sa.stride_v_head = value_cache.stride(0), value_cache.stride(1)
    if per_token_kv:
        sa.stride_ks_block, sa.stride_ks_head = key_scale.stride(0), key_scale.stride(1)
    sa.stride_out_tok, sa.stride_out_head = output.stride(0), output.stride(1)
    b = int(context_lengths.shape[0])
    sa.num_seqs = b
    sa.num_kv_heads = int(key_cache.shape[1])
    sa.query_length = query.shape[0] // b
    sa.query_group_size = query.shape[1] // int(key_cache.shape[1])
    sa.head_size = int(query.shape[-1])
    sa.block_size = int(key_cache.shape[-2])
    sa.num_blocks = int(key_cache.shape[0])
    sa.sliding_window = int(sliding_window)
    sa.per_token_kv = int(per_token_kv)
    sa.trans_v = int(trans_v)
    sa.query_dtype = DTYPE_BF16 if query_input_dtype == "bf16" else DTYPE_F16
    sa.output_dtype = output_dtype
    sa.softmax_scale = float(softmax_scale)
    return sa


_METADATA_KEYS = ("work_indptr", "work_info_flat", "partition_indptr", "reduce_indptr", "reduce_final_map",
                  "reduce_partial_map", "num_sm", "partial_output", "partial_lse")


def _prepare_worklist(md, output, query, key_cache, value_cache, context_lengths, kv_page_indices, kv_indptr,
                      softmax_scale, key_scale, value_scale, per_token_kv, trans_v, query_input_dtype, output_dtype,
                      s):
    """Persistent route with precomputed metadata (kernels/pa_decode_fp8.py:
    3123-3202): work-list decode, then the reduce of split works."""
    missing = [k for k in _METADATA_KEYS if k not in md]
    if missing:
        raise ValueError(f"metadata is missing {missing}; build it with get_pa_metadata()")
    if int(md.get("partition_size", KV_COMPUTE_BLOCK)) != KV_COMPUTE_BLOCK:
        raise ValueError(f"metadata must use partition_size={KV_COMPUTE_BLOCK}")
    b = int(context_lengths.shape[0])
    ql = query.shape[0] // b
    if int(md.get("query_length", ql)) != ql or int(md["partition_indptr"].shape[0]) != b + 1:
        raise ValueError("metadata was built for a different batch or query length")
    sa = _stream_args(output, query, key_cache, value_cache, context_lengths, kv_page_indices, kv_indptr,
                      softmax_scale, key_scale, value_scale, per_token_kv, trans_v, query_input_dtype, output_dtype)
    po, pl = md["partial_output"], md["partial_lse"]
    sa.work_indptr = md["work_indptr"].data_ptr()
    sa.work_info = md["work_info_flat"].data_ptr()
    sa.partition_indptr = md["partition_indptr"].data_ptr()
    sa.partial_output = po.data_ptr()
    sa.partial_lse = pl.data_ptr()
    sa.stride_po_row = int(md.get("stride_po_ql", po.stride(0)))
    sa.stride_pl_row = int(md.get("stride_pl_ql", pl.stride(0)))
    sa.num_workers = int(md["num_sm"])
    wr = _lib.WorklistReduceArgs()
    wr.abi_version = _lib.ABI_VERSION
    wr.output = output.data_ptr()
    # the reduce reads partial rows from row query_length on (:3189-3200)
    wr.partial_output = po.data_ptr() + ql * sa.stride_po_row * po.element_size()
    wr.partial_lse = pl.data_ptr() + ql * sa.stride_pl_row * pl.element_size()
    wr.reduce_indptr = md["reduce_indptr"].data_ptr()
    wr.reduce_final_map = md["reduce_final_map"].data_ptr()
    wr.reduce_partial_map = md["reduce_partial_map"].data_ptr()
    wr.stride_out_tok, wr.stride_out_head = output.stride(0), output.stride(1)
    wr.stride_po_row, wr.stride_pl_row = sa.stride_po_row, sa.stride_pl_row
    wr.num_groups = b
    wr.num_query_heads = int(query.shape[1])
    wr.head_size = int(query.shape[-1])
    wr.max_query_length = ql
    wr.output_dtype = output_dtype
    keep = (output, query, key_cache, value_cache, context_lengths, kv_page_indices, kv_indptr, key_scale,
            value_scale, md)
    return PreparedDecode("ps_split_reduce", s, keep, stream_args=sa, worklist_reduce_args=wr)


# Bins of the persistent route per CU (kernels/pa_decode_fp8.py:40, the
# reference's _PA_METADATA_GRID_OVERSUB): the work-list decode runs one
# workgroup per bin, and three of its workgroups fit in a CU.
PA_METADATA_GRID_OVERSUB = 3


def metadata_bins(num_cu: int, num_kv_heads: int) -> int:
    """Bins of :func:`get_pa_metadata`: ``num_cu * 3`` rounded down to a
    multiple of ``num_kv_heads`` (kernels/pa_decode_fp8.py:1766-1771); at
    least ``num_kv_heads``."""
    n = num_cu * PA_METADATA_GRID_OVERSUB
    return max(num_kv_heads, (n // num_kv_heads) * num_kv_heads)


def get_pa_metadata(
    query: torch.Tensor,
    key_cache: torch.Tensor,
    context_lengths: torch.Tensor,
    kv_indptr: torch.Tensor,
    num_query_heads: int,
    num_kv_heads: int,
    partition_size: int = KV_COMPUTE_BLOCK,
    *,
    num_cu: Optional[int] = None,
):
    """Work list of the persistent route (kernels/pa_decode_fp8.py:1729-1859).

    The scheduler of kernels/pa_metadata.py:145-420 runs on the host
    (``pa_fp8_plan_worklist``; the context lengths are copied to the host,
    the synchronisation the reference makes with ``.item()``) over the
    reference's bins, ``(num_cu * 3 // num_kv_heads) * num_kv_heads``
    (:func:`metadata_bins`; 768 on MI355X for 4 or 8 kv heads), so the work
    list, reduce maps and partition base are the reference's on the same
    inputs.  ``num_cu`` defaults to the query device's CU count; pass it to
    plan on the host.  Returns the reference's keys: work list, reduce maps,
    ``partition_indptr`` and the float32 partial buffers ``partial_output``
    [(n + 1) * ql, 1, Hq, D] / ``partial_lse`` [(n + 1) * ql, 1, Hq, 1] with
    their strides; plus ``partition_size``.  All tensors live on the query's
    device.
    """
    dev = query.device
    batch_size = int(context_lengths.shape[0])
    query_length = query.shape[0] // max(batch_size, 1)
    head_size = int(query.shape[-1])
    gqa = num_query_heads // num_kv_heads
    if num_cu is None:
        num_cu = _cu_count(dev)
    num_sm = metadata_bins(int(num_cu), num_kv_heads)
    ctx_host = context_lengths.detach().to("cpu", torch.int32)
    n_works, plan = _lib.plan_worklist(ctx_host.numpy(), num_kv_heads, gqa, query_length, num_sm, partition_size)
    parts = (ctx_host + (partition_size - 1)) // partition_size
    partition_indptr = torch.zeros(batch_size + 1, dtype=torch.int32)
    partition_indptr[1:] = torch.cumsum(parts, dim=0).to(torch.int32)
    up = lambda a: torch.from_numpy(a).to(dev)
    # partial rows: every split work's partial_qo_loc + query rows (the
    # reduce count of the last kv head, as the reference sizes it, unless a
    # work of another head reaches further)
    works = plan["work_info"][: max(n_works, 0)]
    max_loc = int(works[:, 1].max()) if n_works > 0 else -1
    num_partials = max(int(plan["reduce_indptr"][-1]), max_loc // query_length + 1 if max_loc >= 0 else 0)
    partial_output = torch.empty(((num_partials + 1) * query_length, 1, num_query_heads, head_size),
                                 dtype=torch.float32, device=dev)
    partial_lse = torch.empty(((num_partials + 1) * query_length, 1, num_query_heads, 1), dtype=torch.float32,
                              device=dev)
    return {
        "work_indptr": up(plan["work_indptr"]),
        "work_info_flat": up(plan["work_info"].reshape(-1)),
        "partition_indptr": partition_indptr.to(dev),
        "reduce_indptr": up(plan["reduce_indptr"]),
        "reduce_final_map": up(plan["reduce_final_map"]),
        "reduce_partial_map": up(plan["reduce_partial_map"]),
        "num_sm": num_sm,
        "partial_output": partial_output,
        "partial_lse": partial_lse,
        "stride_po_partial": query_length * num_query_heads * head_size,
        "stride_pl_partial": query_length * num_query_heads,
        "stride_po_ql": num_query_heads * head_size,
        "stride_pl_ql": num_query_heads,
        "query_length": query_length,
        "partition_size": partition_size,
    }
