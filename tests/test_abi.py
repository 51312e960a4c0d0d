"""The C-ABI library loads, exports every declared symbol and its structs
match the header layout (checked by compiling the header with gcc)."""

from __future__ import annotations

import ctypes
import os
import re
import subprocess

import pytest

from flydsl_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "pa_fp8.h")


def declared_functions():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\s*\*?\s*(pa_fp8_\w+)\s*\(", text, re.M)))


def test_header_declares_the_bound_symbols():
    assert declared_functions() == sorted(_lib.EXPORTED_SYMBOLS)


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    for name in declared_functions():
        assert hasattr(lib, name), name
    out = subprocess.run(["nm", "-D", "--defined-only", _lib.LIB_PATH], capture_output=True, text=True).stdout
    for name in declared_functions():
        assert re.search(rf"\bT {name}$", out, re.M), name


def test_checked_build_exports_every_declared_symbol():
    """The checked build (the same sources with -DPA_FP8_CHECKED) exports the
    same entry points and says it is checked; the release library's
    violation reader returns 0 without touching a device."""
    lib = _lib.load(_lib.CHECKED_LIB_PATH)
    out = subprocess.run(["nm", "-D", "--defined-only", _lib.CHECKED_LIB_PATH], capture_output=True, text=True).stdout
    for name in declared_functions():
        assert hasattr(lib, name), name
        assert re.search(rf"\bT {name}$", out, re.M), name
    assert lib.pa_fp8_checked_build() == 1
    rel = _lib.load()
    assert rel.pa_fp8_checked_build() == 0
    assert _lib.debug_violations(rel) == 0
    assert rel.pa_fp8_debug_violations(None) == -1
    assert lib.pa_fp8_debug_violations(None) == -1


def test_version_and_error_strings():
    lib = _lib.load()
    assert b"gfx950" in lib.pa_fp8_version()
    assert lib.pa_fp8_error_string(-7) == b"pointer or stride not 16-byte aligned"


def test_null_args_rejected_without_gpu():
    lib = _lib.load()
    assert lib.pa_fp8_decode_partition(None, None) == -1
    assert lib.pa_fp8_decode_reduce(None, None) == -1
    a = _lib.PartitionArgs()
    a.abi_version = 99
    assert lib.pa_fp8_decode_partition(ctypes.byref(a), None) == -8
    assert lib.pa_fp8_decode_worklist(None, None) == -1
    assert lib.pa_fp8_decode_balanced(None, None, 0, None) == -1
    assert lib.pa_fp8_reduce_worklist(None, None) == -1
    sa = _lib.StreamArgs()
    sa.abi_version = 99
    assert lib.pa_fp8_decode_balanced(ctypes.byref(sa), None, 0, None) == -8
    assert lib.pa_fp8_rope_cache(None, None) == -1
    ra = _lib.RopeCacheArgs()
    ra.abi_version = 99
    assert lib.pa_fp8_rope_cache(ctypes.byref(ra), None) == -8
    ra.abi_version = _lib.ABI_VERSION
    ra.head_dim, ra.block_size, ra.max_pos, ra.num_tokens, ra.num_q_heads = 72, 16, 8, 1, 1
    assert lib.pa_fp8_rope_cache(ctypes.byref(ra), None) == -2  # half a row is not a whole number of lanes
    ra.head_dim = 1024
    assert lib.pa_fp8_rope_cache(ctypes.byref(ra), None) == -2  # a row beyond one wave
    ra.head_dim = 96
    assert lib.pa_fp8_rope_cache(ctypes.byref(ra), None) == -1  # 5 rows of 12 lanes per wave: accepted; no tensors
    ra.head_dim = 128
    assert lib.pa_fp8_rope_cache(ctypes.byref(ra), None) == -1  # no tensors
    ra.num_tokens = 0
    assert lib.pa_fp8_rope_cache(ctypes.byref(ra), None) == 0  # nothing to do
    assert lib.pa_fp8_qk_norm_rope_quant(None, None) == -1
    qa = _lib.QkNormRopeArgs()
    qa.abi_version = 99
    assert lib.pa_fp8_qk_norm_rope_quant(ctypes.byref(qa), None) == -8
    qa.abi_version = _lib.ABI_VERSION
    qa.head_dim, qa.rope_head_dim, qa.max_pos, qa.num_tokens, qa.num_q_heads = 64, 0, 8, 1, 1
    assert lib.pa_fp8_qk_norm_rope_quant(ctypes.byref(qa), None) == -2  # one wave per row needs D in {128, 256, 512}
    qa.head_dim, qa.rope_head_dim = 512, 63
    assert lib.pa_fp8_qk_norm_rope_quant(ctypes.byref(qa), None) == -6  # odd rotary width
    qa.rope_head_dim, qa.quant, qa.group_size = 64, 1, 48
    assert lib.pa_fp8_qk_norm_rope_quant(ctypes.byref(qa), None) == -6  # group does not divide the row
    qa.group_size = 128
    assert lib.pa_fp8_qk_norm_rope_quant(ctypes.byref(qa), None) == -1  # no tensors
    qa.num_tokens = 0
    assert lib.pa_fp8_qk_norm_rope_quant(ctypes.byref(qa), None) == 0  # nothing to do
    assert lib.pa_fp8_mla_decode(None, None) == -1
    assert lib.pa_fp8_mla_reduce(None, None) == -1
    ma = _lib.MlaDecodeArgs()
    ma.abi_version = 99
    assert lib.pa_fp8_mla_decode(ctypes.byref(ma), None) == -8
    ma.abi_version = _lib.ABI_VERSION
    assert lib.pa_fp8_mla_decode(ctypes.byref(ma), None) == 0  # no workers: nothing to do
    ma.num_workers, ma.num_works, ma.num_rows, ma.num_pages = 4, 4, 1, 0
    assert lib.pa_fp8_mla_decode(ctypes.byref(ma), None) == -6  # no pages to read
    ma.num_pages = 8
    assert lib.pa_fp8_mla_decode(ctypes.byref(ma), None) == -1  # no tensors
    mr = _lib.MlaReduceArgs()
    mr.abi_version = _lib.ABI_VERSION
    assert lib.pa_fp8_mla_reduce(ctypes.byref(mr), None) == 0
    mr.num_groups = 3
    assert lib.pa_fp8_mla_reduce(ctypes.byref(mr), None) == -1


def test_stream_worker_counts():
    # one query image per wave fits two workgroups per CU; larger ones one
    assert _lib.stream_workers(256, 1, 4, True) == 2048
    assert _lib.stream_workers(256, 1, 8, False) == 1024
    assert _lib.stream_workers(256, 4, 4, True) == 1024
    # 17..64 columns: cooperative workgroups, by the LDS of their ring: two
    # waves (17..32 columns) 3 per CU, four waves (nine chunk slots) 2 per CU
    assert _lib.stream_workers(256, 4, 8, True) == 768
    assert _lib.stream_workers(256, 4, 16, True) == 512
    with pytest.raises(RuntimeError):
        _lib.stream_workers(256, 4, 32, True)  # 128 columns: not supported
    ws = _lib.balanced_workspace_bytes(128, 8, 1, 4, 2048)
    # pair descriptors, float32 lse and bf16 partial rows, two of each per run
    assert ws >= 128 * 8 * 8 + 2 * 2048 * 4 * 4 + 2 * 2048 * 4 * 128 * 2


@pytest.mark.parametrize("struct,cname", [(_lib.PartitionArgs, "pa_fp8_partition_args"),
                                          (_lib.ReduceArgs, "pa_fp8_reduce_args"),
                                          (_lib.StreamArgs, "pa_fp8_stream_args"),
                                          (_lib.WorklistReduceArgs, "pa_fp8_worklist_reduce_args"),
                                          (_lib.RopeCacheArgs, "pa_fp8_rope_cache_args"),
                                          (_lib.QkNormRopeArgs, "pa_qk_norm_rope_args"),
                                          (_lib.MlaDecodeArgs, "pa_mla_decode_args"),
                                          (_lib.MlaReduceArgs, "pa_mla_reduce_args")])
def test_struct_layout_matches_header(tmp_path, struct, cname):
    fields = [f for f, _ in struct._fields_]
    src = ["#include <stdio.h>", "#include <stddef.h>", f'#include "{HEADER}"', "int main(void){",
           f'printf("%zu\\n", sizeof({cname}));']
    src += [f'printf("%zu\\n", offsetof({cname}, {f}));' for f in fields]
    src += ["return 0;}"]
    c = tmp_path / "layout.c"
    c.write_text("\n".join(src))
    exe = tmp_path / "layout"
    subprocess.run(["gcc", str(c), "-o", str(exe)], check=True)
    vals = [int(x) for x in subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.split()]
    assert vals[0] == ctypes.sizeof(struct)
    assert vals[1:] == [getattr(struct, f).offset for f in fields]


def test_static_scratch_entry_checks_before_any_gpu_call():
    """pa_fp8_decode_balanced_static validates like pa_fp8_decode_balanced
    and refuses a workspace beyond its 64 MiB static scratch (PA_ERR_SCRATCH)
    before touching the device."""
    lib = _lib.load()
    assert lib.pa_fp8_static_scratch_bytes() == 64 << 20
    assert lib.pa_fp8_decode_balanced_static(None, None) == -1
    sa = _lib.StreamArgs()
    sa.abi_version = 99
    assert lib.pa_fp8_decode_balanced_static(ctypes.byref(sa), None) == -8
    sa.abi_version = _lib.ABI_VERSION
    for f in ("output", "query", "key_cache", "value_cache", "block_tables", "context_lengths", "key_scale",
              "value_scale"):
        setattr(sa, f, 4096)  # aligned stand-ins; nothing is dereferenced on these paths
    sa.head_size, sa.block_size, sa.num_blocks, sa.max_blocks_per_seq = 128, 16, 64, 4
    sa.num_seqs, sa.num_kv_heads, sa.query_length, sa.query_group_size = 8, 4, 4, 16
    sa.query_dtype = sa.output_dtype = _lib.DTYPE_BF16
    sa.stride_q_tok, sa.stride_q_head, sa.stride_out_tok, sa.stride_out_head = 64 * 128, 128, 64 * 128, 128
    sa.stride_k_block, sa.stride_k_head, sa.stride_v_block, sa.stride_v_head = 4 * 2048, 2048, 4 * 2048, 2048
    sa.num_workers = 2048  # 64 columns x 2048 runs: 64 MiB of bf16 partial rows, plus their lse
    need = _lib.balanced_workspace_bytes(8, 4, 4, 16, 2048)
    assert need > 64 << 20
    assert lib.pa_fp8_decode_balanced_static(ctypes.byref(sa), None) == -9
    assert lib.pa_fp8_error_string(-9).startswith(b"the call needs more workspace")
    sa.num_seqs = 1025  # the balanced split's batch limit
    assert lib.pa_fp8_decode_balanced_static(ctypes.byref(sa), None) == -6


def _stream_stub(head_size, ql, gqa):
    sa = _lib.StreamArgs()
    sa.abi_version = _lib.ABI_VERSION
    for f in ("output", "query", "key_cache", "value_cache", "block_tables", "context_lengths", "key_scale",
              "value_scale"):
        setattr(sa, f, 4096)  # aligned stand-ins; nothing is dereferenced on these paths
    sa.head_size, sa.block_size, sa.num_blocks, sa.max_blocks_per_seq = head_size, 16, 64, 4
    sa.num_seqs, sa.num_kv_heads, sa.query_length, sa.query_group_size = 2, 2, ql, gqa
    sa.query_dtype = sa.output_dtype = _lib.DTYPE_BF16
    sa.stride_q_tok, sa.stride_q_head = 2 * gqa * head_size, head_size
    sa.stride_out_tok, sa.stride_out_head = sa.stride_q_tok, sa.stride_q_head
    sa.stride_k_block, sa.stride_k_head = 2 * 16 * head_size, 16 * head_size
    sa.stride_v_block, sa.stride_v_head = sa.stride_k_block, sa.stride_k_head
    sa.num_workers = 8
    return sa


def test_head_sizes_and_column_counts_without_gpu():
    """Head sizes 64 / 128 / 192 / 256 and any ql * gqa pass the partition,
    reduce and work-list checks (the generic kernels take them); other head
    sizes are PA_ERR_HEAD_SIZE; the balanced decode keeps D = 128 and <= 64
    columns.  Every call here stops before a launch."""
    lib = _lib.load()
    # balanced: D = 128 and at most 64 columns only
    assert lib.pa_fp8_decode_balanced(ctypes.byref(_stream_stub(256, 1, 4)), None, 0, None) == -2
    assert lib.pa_fp8_decode_balanced(ctypes.byref(_stream_stub(128, 8, 16)), None, 0, None) == -4
    # work list: any of the four head sizes and any column count reach the
    # work-list pointer check (NULL here)
    for d, ql, gqa in ((64, 1, 4), (192, 2, 8), (256, 1, 16), (128, 8, 16), (256, 4, 32)):
        assert lib.pa_fp8_decode_worklist(ctypes.byref(_stream_stub(d, ql, gqa)), None) == -1, (d, ql, gqa)
    for d in (96, 576, 1024):
        assert lib.pa_fp8_decode_worklist(ctypes.byref(_stream_stub(d, 1, 4)), None) == -2, d
    for d in (320, 384, 448, 512):
        assert lib.pa_fp8_decode_worklist(ctypes.byref(_stream_stub(d, 1, 4)), None) == -1, d
    # partition: nothing to do for an empty batch once the shape is accepted
    pa = _lib.PartitionArgs()
    pa.abi_version = _lib.ABI_VERSION
    for f in ("query", "key_cache", "value_cache", "block_tables", "context_lengths", "key_scale", "value_scale",
              "exp_sums", "max_logits", "tmp_out"):
        setattr(pa, f, 4096)
    pa.slots_per_workgroup, pa.num_partitions = 1, 3
    pa.block_size, pa.num_blocks, pa.max_blocks_per_seq = 16, 64, 4
    pa.num_seqs, pa.num_kv_heads, pa.query_length, pa.query_group_size = 0, 2, 8, 16
    pa.query_dtype = pa.tmp_dtype = _lib.DTYPE_BF16
    for d in (64, 128, 192, 256, 320, 384, 448, 512):
        pa.head_size = d
        pa.stride_q_tok, pa.stride_q_head = 32 * d, d
        pa.stride_to_group, pa.stride_to_part = d, 128 * d
        pa.stride_to_head, pa.stride_to_seq = 3 * 128 * d, 2 * 3 * 128 * d
        assert lib.pa_fp8_decode_partition(ctypes.byref(pa), None) == 0, d
    pa.head_size = 96
    assert lib.pa_fp8_decode_partition(ctypes.byref(pa), None) == -2
    ra = _lib.ReduceArgs()
    ra.abi_version = _lib.ABI_VERSION
    for f in ("output", "exp_sums", "max_logits", "tmp_out"):
        setattr(ra, f, 4096)
    ra.num_seqs, ra.num_kv_heads, ra.num_partitions, ra.query_length, ra.query_group_size = 0, 2, 3, 8, 16
    ra.output_dtype = ra.tmp_dtype = _lib.DTYPE_BF16
    for d, rc in ((64, 0), (192, 0), (256, 0), (320, 0), (512, 0), (96, -2), (576, -2)):
        ra.head_size = d
        assert lib.pa_fp8_decode_reduce(ctypes.byref(ra), None) == rc, d
    wr = _lib.WorklistReduceArgs()
    wr.abi_version = _lib.ABI_VERSION
    for f in ("output", "partial_output", "partial_lse", "reduce_indptr", "reduce_final_map", "reduce_partial_map"):
        setattr(wr, f, 4096)
    wr.num_groups, wr.num_query_heads, wr.max_query_length = 0, 32, 8
    wr.output_dtype = _lib.DTYPE_BF16
    for d, rc in ((64, 0), (256, 0), (320, 0), (448, 0), (96, -2), (640, -2)):
        wr.head_size = d
        assert lib.pa_fp8_reduce_worklist(ctypes.byref(wr), None) == rc, d


@pytest.mark.skipif(__import__("torch").cuda.is_available(), reason="the stand-in pointers would be launched on a GPU")
def test_static_entry_device_lookup_without_gpu():
    """pa_fp8_decode_balanced_static finds its scratch on the device of the
    stream it is given (the current device for the null stream).  Without a
    GPU that lookup is where a valid call stops: the runtime's error comes
    back as a positive hipError_t, not a crash and not success."""
    lib = _lib.load()
    sa = _stream_stub(128, 1, 4)
    rc = lib.pa_fp8_decode_balanced_static(ctypes.byref(sa), None)
    assert rc > 0, rc
    assert lib.pa_fp8_error_string(rc) not in (b"ok", b"")
