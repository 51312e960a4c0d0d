"""The KV-cache writer's CPU restatement (oracle/rope_cache.py), pinned.

The reference holds no fixtures for this kernel (its test recomputes a
torch reference each run, tests/kernels/test_fused_rope_cache.py:162-237).
What pins the restatement here:
  * an independent bit-level NumPy computation of the same rounding
    sequence (bf16 round-to-nearest-even done on the integer bits);
  * closed forms: cos = 1, sin = 0 is the identity; a rotation by theta
    then by -theta returns the input up to rounding; pair norms are kept;
  * the cache written through each layout reads back, token by token,
    through the decode oracle's page gather (oracle/torch_ref.py), which
    pins the writer's layouts to the reader's;
  * slots < 0 and slots past the cache write nothing;
  * fp8: every finite e4m3fn code survives a round trip, values beyond
    the range saturate, NaN stays NaN.
Planted mistakes (a flipped sign, swapped halves, mirrored page positions)
fail these checks.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import rope_cache as rc
from oracle import torch_ref


def bf16_round_bits(x: np.ndarray) -> np.ndarray:
    """float32 -> bf16 -> float32 by integer round-to-nearest-even."""
    u = x.astype(np.float32).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    return r.astype(np.uint32).view(np.float32)


def np_round(x: np.ndarray, dtype: str) -> np.ndarray:
    return bf16_round_bits(x) if dtype == "bf16" else x.astype(np.float16).astype(np.float32)


def np_rope(x: np.ndarray, c: np.ndarray, s: np.ndarray, dtype: str, reuse: bool) -> np.ndarray:
    """Loop restatement: out[d] = r(r(x[d] c[d]) -+ r(x[d +- D/2] s[d]))."""
    T, H, D = x.shape
    h = D // 2
    out = np.empty_like(x)
    for t in range(T):
        for d in range(D):
            ci = d % h if reuse else d
            first = d < h
            pd = d + h if first else d - h
            xc = np_round(x[t, :, d] * c[t, ci], dtype)
            ps = np_round(x[t, :, pd] * s[t, ci], dtype)
            out[t, :, d] = np_round(xc - ps if first else xc + ps, dtype)
    return out


def _inputs(T, H, D, dtype, reuse, seed=0, max_pos=64):
    g = torch.Generator().manual_seed(seed)
    tdt = torch.bfloat16 if dtype == "bf16" else torch.float16
    x = torch.randn(T, H, D, generator=g).to(tdt)
    cols = D // 2 if reuse else D
    cos = torch.randn(max_pos, cols, generator=g).to(tdt)
    sin = torch.randn(max_pos, cols, generator=g).to(tdt)
    pos = torch.randint(0, max_pos, (T,), generator=g, dtype=torch.int32)
    return x, cos, sin, pos


@pytest.mark.parametrize("dtype", ["bf16", "f16"])
@pytest.mark.parametrize("reuse", [True, False])
@pytest.mark.parametrize("D", [16, 64, 96, 128, 192])
def test_rotation_matches_bitwise_restatement(dtype, reuse, D):
    x, cos, sin, pos = _inputs(5, 3, D, dtype, reuse, seed=D + reuse)
    got = rc.rope_neox(x, cos[pos.long()], sin[pos.long()], reuse).float().numpy()
    want = np_rope(x.float().numpy(), cos[pos.long()].float().numpy(), sin[pos.long()].float().numpy(), dtype, reuse)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_planted_mistakes_fail_the_restatement():
    x, cos, sin, pos = _inputs(4, 2, 64, "bf16", True, seed=5)
    c, s = cos[pos.long()], sin[pos.long()]
    want = np_rope(x.float().numpy(), c.float().numpy(), s.float().numpy(), "bf16", True)
    flipped = rc.rope_neox(x, c, -s, True).float().numpy()  # sign of the sine term
    swapped = rc.rope_neox(x.flip(-1), c, s, True).flip(-1).float().numpy()  # halves exchanged
    assert not np.array_equal(flipped, want)
    assert not np.array_equal(swapped, want)


@pytest.mark.parametrize("dtype", ["bf16", "f16"])
def test_identity_and_inverse_rotation(dtype):
    tdt = torch.bfloat16 if dtype == "bf16" else torch.float16
    x = torch.randn(6, 4, 128, generator=torch.Generator().manual_seed(1)).to(tdt)
    ones, zeros = torch.ones(6, 64, dtype=tdt), torch.zeros(6, 64, dtype=tdt)
    assert torch.equal(rc.rope_neox(x, ones, zeros, True), x)
    theta = torch.linspace(0.1, 3.0, 6 * 64).reshape(6, 64)
    c, s = torch.cos(theta).to(tdt), torch.sin(theta).to(tdt)
    back = rc.rope_neox(rc.rope_neox(x, c, s, True), c, -s, True)
    eps = 2.0 ** -7 if dtype == "bf16" else 2.0 ** -10
    assert torch.allclose(back.float(), x.float(), atol=8 * eps, rtol=8 * eps)
    y = rc.rope_neox(x, c, s, True).float()
    xf = x.float()
    n_in = xf[..., :64] ** 2 + xf[..., 64:] ** 2
    n_out = y[..., :64] ** 2 + y[..., 64:] ** 2
    assert torch.allclose(n_out, n_in, rtol=16 * eps, atol=16 * eps)


def _caches(layout, NB, KH, D, bs, dtype=torch.bfloat16):
    if layout == rc.FLASH:
        return torch.zeros(NB, bs, KH, D, dtype=dtype), torch.zeros(NB, bs, KH, D, dtype=dtype)
    kc = torch.zeros(NB, KH, D // 16, bs, 16, dtype=dtype)
    vc = torch.zeros(NB, KH, D, bs, dtype=dtype) if layout == rc.ATOM else torch.zeros(NB, KH, bs // 16, D, 16,
                                                                                        dtype=dtype)
    return kc, vc


@pytest.mark.parametrize("layout", [rc.ATOM, rc.ATOM_TRANS_V])
@pytest.mark.parametrize("bs", [16, 64])
def test_cache_reads_back_through_the_decode_gather(layout, bs):
    """Tokens 0..T-1 of a sequence written to the slots its block table
    names come back, in order, through the decode oracle's gather."""
    T, QH, KH, D, NB = 100, 4, 2, 128, 12
    g = torch.Generator().manual_seed(bs)
    q = torch.randn(T, QH, D, generator=g).to(torch.bfloat16)
    k = torch.randn(T, KH, D, generator=g).to(torch.bfloat16)
    v = torch.randn(T, KH, D, generator=g).to(torch.bfloat16)
    cos = torch.randn(32, D // 2, generator=g).to(torch.bfloat16)
    sin = torch.randn(32, D // 2, generator=g).to(torch.bfloat16)
    pos = torch.randint(0, 32, (T,), generator=g, dtype=torch.int32)
    table = torch.randperm(NB, generator=g)[: math.ceil(T / bs)]
    slots = (table.repeat_interleave(bs)[:T] * bs + torch.arange(T) % bs).to(torch.int32)
    kc, vc = _caches(layout, NB, KH, D, bs)
    _, k_out, kc2, vc2 = rc.rope_cache_ref(q, k, v, pos, cos, sin, slots, kc, vc, block_size=bs, layout=layout)
    kg, vg = torch_ref.gather_tokens(kc2, vc2, table.tolist(), T)
    assert torch.equal(kg, k_out.float()) and torch.equal(vg, v.float())
    # tokens placed at mirrored page positions would not read back
    kg_bad, _ = torch_ref.gather_tokens(kc2.flip(3), vc2, table.tolist(), T)
    assert not torch.equal(kg_bad, k_out.float())


def test_flash_layout_and_skipped_slots():
    T, QH, KH, D, bs, NB = 9, 2, 2, 64, 16, 2
    g = torch.Generator().manual_seed(3)
    q = torch.randn(T, QH, D, generator=g).to(torch.bfloat16)
    k = torch.randn(T, KH, D, generator=g).to(torch.bfloat16)
    v = torch.randn(T, KH, D, generator=g).to(torch.bfloat16)
    cos = torch.randn(16, D // 2, generator=g).to(torch.bfloat16)
    sin = torch.randn(16, D // 2, generator=g).to(torch.bfloat16)
    pos = torch.arange(T, dtype=torch.int32)
    slots = torch.tensor([0, -1, 5, 17, -7, 31, 32, 40, 2], dtype=torch.int32)  # 32, 40: past the 2-block cache
    kc, vc = _caches(rc.FLASH, NB, KH, D, bs)
    _, k_out, kc2, vc2 = rc.rope_cache_ref(q, k, v, pos, cos, sin, slots, kc, vc, block_size=bs, layout=rc.FLASH)
    written = {0: 0, 5: 2, 17: 3, 31: 5, 2: 8}
    flat_k, flat_v = kc2.reshape(NB * bs, KH, D), vc2.reshape(NB * bs, KH, D)
    for sl in range(NB * bs):
        if sl in written:
            assert torch.equal(flat_k[sl], k_out[written[sl]]) and torch.equal(flat_v[sl], v[written[sl]])
        else:
            assert not flat_k[sl].any() and not flat_v[sl].any()


def test_fp8_codes_round_trip_and_saturate():
    codes = torch.arange(256, dtype=torch.uint8)
    vals = codes.view(torch.float8_e4m3fn).float()
    finite = ~torch.isnan(vals)
    for scale in (1.0, 0.1, 0.037):
        # value * scale -> quantised with 1/scale: the code comes back
        # (float32 rounding of value * scale * (1/scale) stays within half
        # an fp8 step for every finite code)
        back = rc.fp8_bytes(vals[finite] * torch.tensor(scale), scale)
        assert torch.equal(back, codes[finite]), scale
    sat = rc.fp8_bytes(torch.tensor([1e6, -1e6, 465.0, 449.0]), 1.0)
    assert sat.tolist() == [0x7E, 0xFE, 0x7E, 0x7E]
    nan = rc.fp8_bytes(torch.tensor([float("nan")]), 1.0).view(torch.float8_e4m3fn).float()
    assert torch.isnan(nan).all()


def test_int64_indices_read_as_low_words():
    x = torch.tensor([5, -1, 2**32 + 7, -(2**32) - 3, 2**31 - 1], dtype=torch.int64)
    assert rc.low_words(x).tolist() == [5, -1, 7, -3, 2**31 - 1]
    assert rc.low_words(torch.tensor([3, -2], dtype=torch.int32)).tolist() == [3, -2]


def test_positions_are_clamped_into_the_tables():
    x, cos, sin, _ = _inputs(3, 1, 32, "bf16", True, seed=9, max_pos=8)
    k = x
    v = torch.zeros_like(k)
    kc, vc = _caches(rc.FLASH, 1, 1, 32, 16)
    slots = torch.full((3,), -1, dtype=torch.int32)
    q1, _, _, _ = rc.rope_cache_ref(x, k, v, torch.tensor([-4, 100, 7], dtype=torch.int32), cos, sin, slots, kc, vc,
                                    block_size=16, layout=rc.FLASH)
    q2, _, _, _ = rc.rope_cache_ref(x, k, v, torch.tensor([0, 7, 7], dtype=torch.int32), cos, sin, slots, kc, vc,
                                    block_size=16, layout=rc.FLASH)
    assert torch.equal(q1, q2)
