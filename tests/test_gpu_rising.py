"""GPU parity when the softmax references keep moving along a sequence.

The decode kernels keep a running maximum per query column and, with
per-token scales, a running value-scale reference, both moved lazily (only
when a block of keys passes them by a margin), and rescale their
accumulators when they move.  Here the per-token key scales grow along each
sequence (the logits' spread grows ~8x from the first key to the last, so
the maximum keeps rising, in small steps and, with jumps, by more than the
lazy margin at once) and the value scales grow ~4x (the value reference
moves along the way), on the cooperative kernel's shapes (17..64 query
columns per kv head), the per-wave streaming decode and the partition
schedules.  Bar as everywhere: bf16 outputs within atol/rtol 2e-2 of the
CPU oracle, every element.

The value-scale spread stays realistic: the probabilities enter the value
product as fp8 hi + lo terms (2^-8 relative per key), so an output that is
a small difference of much larger weighted values -- value magnitudes
spread 32x along one sequence -- can exceed the absolute tolerance on every
kernel here.
"""

from __future__ import annotations

import pytest
import torch

import tests.test_gpu_parity as tp
from tests._cases import make_case, torch_oracle
from tests.test_gpu_stream import assert_parity, balanced, run, to_dev

pytestmark = pytest.mark.gpu


def rising(case, kgrow=3.0, vgrow=2.0, jump_every=0):
    """Scale key scales by 2^(kgrow * t / ctx) and value scales by
    2^(vgrow * t / ctx) at logical token t of each sequence; with
    jump_every > 0 the key scale also doubles at every jump_every-th token
    (logits that grow by more than the lazy margin at once)."""
    bt = case["block_tables"]
    bs = case["key_cache"].shape[-2]
    ks, vs = case["key_scale"].clone(), case["value_scale"].clone()
    for b, ctx in enumerate(case["context_lengths"].tolist()):
        t = torch.arange(ctx)
        kf = torch.pow(2.0, kgrow * t / max(ctx, 1))
        if jump_every:
            kf = kf * torch.pow(2.0, (t // jump_every).float())
        vf = torch.pow(2.0, vgrow * t / max(ctx, 1))
        pages = bt[b, t // bs].long()
        slots = t % bs
        ks[pages, :, slots, 0] *= kf[:, None]
        vs[pages, :, slots, 0] *= vf[:, None]
    case = dict(case)
    case["key_scale"], case["value_scale"] = ks, vs
    return case


CASES = {
    # cooperative workgroups: 64 columns (MTP ql 4 x GQA 16) on 64-token pages, like C5
    "coop_ql4_gqa16_page64": dict(batch=5, query_length=4, num_query_heads=64, num_kv_heads=4, block_size=64,
                                  ctx=[4, 200, 1300, 3000, 5000]),
    "coop_ql2_gqa16": dict(batch=4, query_length=2, num_query_heads=32, num_kv_heads=2, ctx=[40, 900, 2500, 4100]),
    # per-wave streaming (4 columns) and the partition schedules
    "gqa4": dict(batch=6, num_query_heads=8, num_kv_heads=2, ctx=[1, 33, 700, 2000, 4096, 6000]),
}


@pytest.mark.parametrize("jump", [0, 600])
@pytest.mark.parametrize("name", sorted(CASES))
def test_rising_references(name, jump):
    case = rising(make_case(seed=400 + len(name) + jump, per_token=True, **CASES[name]), jump_every=jump)
    ref = torch_oracle(case, float_out=False)
    d = to_dev(case)
    with balanced():
        out, route = run(d)
    assert_parity(out, ref, f"{name} jump={jump} balanced")
    with balanced(num_cu=3):
        out, _ = run(d)
    assert_parity(out, ref, f"{name} jump={jump} balanced, 3 CUs")
    for sched in ("owner", "slot"):
        out, _, _ = tp.launch(d, sched=sched)
        assert_parity(out, ref, f"{name} jump={jump} {sched}")
