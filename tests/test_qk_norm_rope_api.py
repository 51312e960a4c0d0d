"""flydsl_qk_norm_rope_quant's argument checks, on the CPU (they run before
any launch), against the reference's messages and exception types
(kernels/qk_norm_rope_quant.py:800-899, :201-242)."""

from __future__ import annotations

import pytest
import torch

from flydsl_amd import compile_flydsl_qk_norm_rope_quant, flydsl_qk_norm_rope_quant
from tests.test_qk_norm_rope_oracle import make_inputs

H, D, RD = 2, 512, 64


def call(**over):
    inp = make_inputs(T=3, H=H, D=D, RD=RD)
    args = dict(q=inp["q"], kv=inp["kv"], kv_weight=inp["kv_weight"], cos_cache=inp["cos_cache"],
                sin_cache=inp["sin_cache"], positions=inp["positions"])
    kw = dict(num_q_heads=H, head_dim=D, rope_head_dim=RD)
    for k, v in over.items():
        (args if k in args else kw)[k] = v
    return flydsl_qk_norm_rope_quant(*args.values(), **kw)


@pytest.mark.parametrize("over,exc,msg", [
    (dict(q=torch.zeros(3, H * D, dtype=torch.float16)), TypeError, "q must be bf16"),
    (dict(kv=torch.zeros(3, D)), TypeError, "kv must be bf16"),
    (dict(kv_weight=torch.zeros(D)), TypeError, "kv_weight must be bf16"),
    (dict(positions=torch.zeros(3, dtype=torch.int32)), TypeError, "positions must be int64"),
    (dict(scale_dtype="fp16"), ValueError, "scale_dtype"),
    (dict(q_weight=torch.zeros(D)), TypeError, "q_weight must be bf16"),
    (dict(kv=torch.zeros(3, 2 * D + 1, dtype=torch.bfloat16)[:, :D]), ValueError, "must be even"),
    (dict(kv=torch.zeros(D, 3, dtype=torch.bfloat16).t()), ValueError, "dense in the last dim"),
    (dict(q=torch.zeros(3, H * D + 2, dtype=torch.bfloat16)), ValueError, "!= [T, H*D"),
    (dict(q=torch.zeros(3, H, D + 2, dtype=torch.bfloat16)[..., :D]), ValueError, "contiguous in the (H, D)"),
    (dict(cos_cache=torch.zeros(8, RD, dtype=torch.bfloat16)), ValueError, "cos_cache last dim"),
    (dict(quant=True, quant_group_size=96), ValueError, "divisible by quant_group_size"),
])
def test_argument_errors(over, exc, msg):
    with pytest.raises(exc, match=msg.replace("(", r"\(").replace(")", r"\)").replace("[", r"\[").replace("*", r"\*")):
        call(**over)


def test_sin_shape_mismatch():
    inp = make_inputs(T=3, H=H, D=D, RD=RD)
    with pytest.raises(ValueError, match="cos/sin shape mismatch"):
        call(sin_cache=inp["sin_cache"][:4])


@pytest.mark.parametrize("kw", [
    dict(head_dim=64, rope_head_dim=64, group_size=64),
    dict(head_dim=512, rope_head_dim=63, group_size=512),
    dict(head_dim=512, rope_head_dim=64, group_size=48),
    dict(head_dim=512, rope_head_dim=64, group_size=4),
    dict(head_dim=512, rope_head_dim=64, group_size=512, scale_dtype="int8"),
])
def test_unsupported_configurations_assert(kw):
    base = dict(num_q_heads=4, quant=True, scale_dtype="fp32", q_weighted=False)
    base.update(kw)
    with pytest.raises(AssertionError):
        compile_flydsl_qk_norm_rope_quant(**base)
