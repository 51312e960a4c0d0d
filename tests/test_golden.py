"""The committed golden fixtures (tests/golden/) against the oracle and the
library's host planner, on the CPU.

The fixtures were written by tests/golden/make_golden.py from the oracle;
these tests fail when the oracle, the case builders or the host planner drift
from them.  The decode outputs are also checked against the independent
float64 NumPy brute force (oracle/np_ref.py), so the frozen values are
attention and not just whatever the torch restatement gave.
"""

from __future__ import annotations

import json
import os

import numpy as np
import pytest
import torch

from flydsl_amd import _lib
from oracle import plan, worklist
from tests._cases import make_case, numpy_oracle, torch_oracle
from tests.golden import make_golden as mg

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load(name: str) -> dict:
    with np.load(os.path.join(HERE, name), allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def decode_case(fx: dict, name: str, device="cpu") -> dict:
    """A decode case (the tensors of make_case) rebuilt from the fixture."""
    meta = json.loads(bytes(fx["meta"]).decode())[name]

    def t(key):
        return torch.from_numpy(np.ascontiguousarray(fx[f"{name}/{key}"])).to(device)

    return {
        "query": torch.from_numpy(fx[f"{name}/query_bf16"].view(np.int16)).view(torch.bfloat16).to(device),
        "key_cache": t("key_cache").view(torch.float8_e4m3fn),
        "value_cache": t("value_cache").view(torch.float8_e4m3fn),
        "block_tables": t("block_tables"),
        "context_lengths": t("context_lengths"),
        "key_scale": t("key_scale"),
        "value_scale": t("value_scale"),
        "softmax_scale": meta["softmax_scale"],
        "query_length": meta["query_length"],
        "sliding_window": meta["sliding_window"],
    }


@pytest.mark.parametrize("name", list(mg.DECODE_CASES))
def test_decode_inputs_are_the_seeded_case(name):
    fx = load("decode.npz")
    case = make_case(**mg.DECODE_CASES[name])
    got = decode_case(fx, name)
    for key in ("query", "key_cache", "value_cache"):
        assert torch.equal(got[key].view(torch.uint8), case[key].view(torch.uint8)), key
    for key in ("block_tables", "context_lengths", "key_scale", "value_scale"):
        assert torch.equal(got[key], case[key]), key


@pytest.mark.parametrize("name", list(mg.DECODE_CASES))
def test_decode_outputs_reproduce(name):
    fx = load("decode.npz")
    case = decode_case(fx, name)
    want = fx[f"{name}/out"]
    got = torch_oracle(case).float().numpy()
    assert np.allclose(got, want, atol=1e-5, rtol=1e-5)
    brute = numpy_oracle(case)
    assert np.allclose(brute.reshape(want.shape), want, atol=1e-4, rtol=1e-4)


def test_recommended_splits_reproduce():
    fx = load("planner.npz")
    for row, want in zip(fx["split_grid"].tolist(), fx["splits"].tolist()):
        b, h, s, w, ql, cu = row
        assert plan.get_recommended_splits(b, h, s, sliding_window=w, query_length=ql, num_cu=cu) == want, row
        assert _lib.recommended_splits(b, h, s, w, 256, ql, cu) == want, row


def test_slot_ranges_reproduce():
    fx = load("planner.npz")
    for ctx, P, z, W, ql, t0, t1 in fx["slot_ranges"].tolist():
        assert plan.slot_token_range(ctx, P, z, sliding_window=W, query_length=ql) == (t0, t1)
        assert _lib.plan_slot(ctx, P, z, W, ql) == (t0, t1)


@pytest.mark.parametrize("name", list(mg.WORKLISTS))
def test_worklists_reproduce(name):
    fx = load("planner.npz")
    kw = json.loads(bytes(fx["worklist_args"]).decode())[name]
    ref = worklist.pa_metadata_v1(**kw)
    n, got = _lib.plan_worklist(kw["context_lens"], kw["num_heads_k"], kw["gqa"], kw["query_length"], kw["num_cu"],
                                kw["kv_granularity"])
    assert n == ref["num_works"] == fx[f"{name}/work_info"].shape[0]
    g = fx[f"{name}/reduce_final_map"].shape[0]
    used = fx[f"{name}/reduce_partial_map"].shape[0]
    for key, cut in (("work_indptr", None), ("work_info", n), ("reduce_indptr", None), ("reduce_final_map", g),
                     ("reduce_partial_map", used)):
        want = fx[f"{name}/{key}"]
        for src in (ref[key], got[key]):
            have = src if cut is None else src[:cut]
            assert np.array_equal(have, want), key


@pytest.mark.parametrize("name", list(mg.ROPE_CASES))
def test_rope_cache_outputs_reproduce(name):
    fx = load("rope_cache.npz")
    inp = mg.rope_inputs(name)
    for key, t in inp.items():
        want = fx[f"{name}/{key}"]
        have = mg._bits(t) if t.is_floating_point() else t.numpy()
        assert np.array_equal(have, want), key
    for key, t in zip(("q_out", "k_out", "key_cache_out", "value_cache_out"), mg.rope_reference(name, inp)):
        assert np.array_equal(mg._bits(t), fx[f"{name}/{key}"]), key


@pytest.mark.parametrize("name", list(mg.QKNR_CASES))
def test_qk_norm_rope_outputs_reproduce(name):
    fx = load("qk_norm_rope.npz")
    inp = mg.qknr_inputs(name)
    for key, t in inp.items():
        if t is not None:
            want = fx[f"{name}/{key}"]
            have = mg._bits(t) if t.is_floating_point() else t.numpy()
            assert (have == want.reshape(have.shape)).all(), f"{name}: input {key}"
    for key, a in zip(("q_out", "kv_out", "q_scale", "kv_scale"), mg.qknr_reference(name, inp)):
        if a is None:
            assert f"{name}/{key}" not in fx
        else:
            assert np.array_equal(a, fx[f"{name}/{key}"]), f"{name}: {key}"
