"""The HIP library against the committed golden fixtures (tests/golden/).

No oracle runs here: the expected values are the frozen fixture outputs.
Decode: every case under the launcher's own schedule and under one slot per
workgroup (partition pass + LSE reduce), bf16 output within atol = rtol =
2e-2 of the fixture, every element.  KV-cache writer: Q_out, K_out and every
cache byte equal to the fixture.
"""

from __future__ import annotations

import pytest
import torch

import flydsl_amd.pa_decode as pd
from flydsl_amd import build_fused_rope_cache_module, pa_decode_ps_launch
from oracle import rope_cache as rc
from tests.golden import make_golden as mg
from tests.test_golden import decode_case, load

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
ATOL = RTOL = 2e-2


def _decode(case: dict, slot_schedule: bool) -> torch.Tensor:
    q = case["query"]
    out = torch.empty(q.shape, dtype=torch.bfloat16, device=q.device)
    saved = pd._schedule, pd._balanced_ok
    if slot_schedule:
        pd._schedule = lambda *args: 1
        pd._balanced_ok = lambda *args: False
    try:
        pa_decode_ps_launch(out, q, case["key_cache"], case["value_cache"], case["context_lengths"], None, None,
                            case["softmax_scale"], case["key_scale"], case["value_scale"],
                            block_tables=case["block_tables"], sliding_window=case["sliding_window"])
    finally:
        pd._schedule, pd._balanced_ok = saved
    torch.cuda.synchronize()
    return out.float().cpu()


@pytest.mark.parametrize("slot_schedule", [False, True], ids=["auto", "slot"])
@pytest.mark.parametrize("name", list(mg.DECODE_CASES))
def test_decode_matches_fixture(name, slot_schedule):
    fx = load("decode.npz")
    case = decode_case(fx, name, device=DEV)
    want = torch.from_numpy(fx[f"{name}/out"])
    got = _decode(case, slot_schedule)
    bad = ~torch.isclose(got, want, atol=ATOL, rtol=RTOL)
    assert not bad.any(), f"{name}: {int(bad.sum())} elements off, max |err| {(got - want).abs().max():.3e}"


def _from_bits(a, like: torch.Tensor) -> torch.Tensor:
    """A fixture array (raw bits of a float tensor, or integers) as ``like``'s dtype."""
    if like.is_floating_point():
        return torch.from_numpy(a.view({2: "i2", 4: "i4"}[a.itemsize])).view(like.dtype)
    return torch.from_numpy(a).to(like.dtype)


@pytest.mark.parametrize("name", list(mg.ROPE_CASES))
def test_rope_cache_matches_fixture(name):
    fx = load("rope_cache.npz")
    T, QH, KH, D, bs, NB, max_pos, dt, layout, apply_scale, reuse, idt, _ = mg.ROPE_CASES[name]
    shapes = mg.rope_inputs(name)  # dtypes and shapes; the values come from the fixture
    d = {k: _from_bits(fx[f"{name}/{k}"], t).reshape(t.shape).to(DEV) for k, t in shapes.items()}
    if apply_scale:
        d["key_cache"] = d["key_cache"].view(torch.float8_e4m3fn)
        d["value_cache"] = d["value_cache"].view(torch.float8_e4m3fn)
    ks = torch.tensor([mg.ROPE_SCALES[0]], dtype=torch.float32, device=DEV)
    vs = torch.tensor([mg.ROPE_SCALES[1]], dtype=torch.float32, device=DEV)
    launch = build_fused_rope_cache_module(head_dim=D, num_q_heads=QH, num_kv_heads=KH, block_size=bs,
                                           flash_layout=layout == rc.FLASH, dtype_str=dt, apply_scale=apply_scale,
                                           reuse_freqs_front_part=reuse,
                                           pos_dtype="i32" if idt == torch.int32 else "i64")
    q_out, k_out = torch.empty_like(d["q"]), torch.empty_like(d["k"])
    launch(d["q"], d["k"], d["v"], d["positions"], d["cos"], d["sin"], d["slots"], d["key_cache"], d["value_cache"],
           q_out, k_out, T, ks, vs)
    torch.cuda.synchronize()
    for key, got in (("q_out", q_out), ("k_out", k_out), ("key_cache_out", d["key_cache"]),
                     ("value_cache_out", d["value_cache"])):
        want = fx[f"{name}/{key}"]
        have = mg._bits(got.cpu().view(torch.uint8) if got.element_size() == 1 else got.cpu())
        assert (have == want.reshape(have.shape)).all(), f"{name}: {key}"
