"""Independent float64 NumPy brute force (test infrastructure).

Pins ``torch_ref`` with a second restatement that shares none of its code:
fp8 bytes are decoded through ``fp8.decode`` (the format's bit fields, not
torch's cast), each key/value is located by walking the block table byte
layout by hand, masks are evaluated per (query, key) pair from positions,
and softmax is an explicit max-subtract / sum loop.  Only for small inputs.

Semantics followed: tests/kernels/test_pa.py:214-331 (masked attention over
the paged gather) with K layout [NB, H, D/16, bs, 16] and V layout either
[NB, H, D, bs] or trans [NB, H, bs/16, D, 16] (test_pa.py:193-200, 419-429).
"""

from __future__ import annotations

import numpy as np

from . import fp8


def _key_vector(kc: np.ndarray, page: int, head: int, slot: int) -> np.ndarray:
    # kc: uint8 [NB, H, D/16, bs, 16]; the head vector is the 16-byte groups
    # of every chunk for this token slot.
    return fp8.decode(kc[page, head, :, slot, :].reshape(-1))


def _value_vector(vc: np.ndarray, page: int, head: int, slot: int) -> np.ndarray:
    if vc.ndim == 4:  # [NB, H, D, bs]
        return fp8.decode(vc[page, head, :, slot])
    # trans: [NB, H, bs/16, D, 16]
    return fp8.decode(vc[page, head, slot // 16, :, slot % 16])


def paged_decode_f64(
    query: np.ndarray,
    key_cache_u8: np.ndarray,
    value_cache_u8: np.ndarray,
    block_tables: np.ndarray,
    context_lengths: np.ndarray,
    query_length: int,
    softmax_scale: float,
    k_scale,
    v_scale,
    sliding_window: int = 0,
) -> np.ndarray:
    """float64 output [B * ql, Hq, D].

    ``k_scale``/``v_scale``: a Python float (per tensor) or an array
    [NB, H, bs] / [NB, H, bs, 1] (per token per head).
    """
    q = np.asarray(query, dtype=np.float64)
    nb, hkv, dchunks, bs, _ = key_cache_u8.shape
    d = dchunks * 16
    hq = q.shape[1]
    gqa = hq // hkv
    batch = len(context_lengths)
    per_token = not np.isscalar(k_scale)
    ks = np.asarray(k_scale, dtype=np.float64).reshape(nb, hkv, bs) if per_token else float(k_scale)
    vs = np.asarray(v_scale, dtype=np.float64).reshape(nb, hkv, bs) if per_token else float(v_scale)
    out = np.zeros((batch * query_length, hq, d), dtype=np.float64)
    for b in range(batch):
        ctx = int(context_lengths[b])
        if ctx == 0:
            continue
        keys = np.zeros((ctx, hkv, d))
        vals = np.zeros((ctx, hkv, d))
        for t in range(ctx):
            page = int(block_tables[b][t // bs])
            slot = t % bs
            for h in range(hkv):
                ksc = ks[page, h, slot] if per_token else ks
                vsc = vs[page, h, slot] if per_token else vs
                keys[t, h] = _key_vector(key_cache_u8, page, h, slot) * ksc
                vals[t, h] = _value_vector(value_cache_u8, page, h, slot) * vsc
        for qi in range(query_length):
            qpos = ctx - query_length + qi
            row = b * query_length + qi
            for hh in range(hq):
                h = hh // gqa
                logits = np.full(ctx, -np.inf)
                for t in range(ctx):
                    if t > qpos:
                        continue
                    if sliding_window > 0 and qpos - t >= sliding_window + 1:
                        continue
                    logits[t] = float(np.dot(q[row, hh], keys[t, h])) * softmax_scale
                m = logits.max()
                if not np.isfinite(m):
                    continue
                w = np.exp(logits - m)
                w /= w.sum()
                out[row, hh] = w @ vals[:, h]
    return out
