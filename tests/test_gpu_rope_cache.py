"""GPU parity of the KV-cache writer against its CPU restatement.

Mirrors the reference test's categories (tests/kernels/test_fused_rope_cache.py:
decode and prefill token counts, model head shapes, flash / ATOM layouts,
bf16 / f16, int32 / int64 indices, half / full cos-sin tables, negative slots,
fp8 cache) with the reference's own inputs (seed 42, N(0,1) data, slots
0..T-1) and, beyond it, scattered slots over a permuted cache and the decode
kernels' value layout.  The bar is bit-exact: Q_out, K_out and every cache
byte equal the oracle's (the reference's own check is atol 1e-2 for bf16 and
max/8 for the fp8 cache, :380-414, which these results also meet).  A last
test feeds the written fp8 cache to the decode kernel.
"""

from __future__ import annotations

import pytest
import torch

from flydsl_amd import build_fused_rope_cache_module, pa_decode_ps_launch
from oracle import rope_cache as rc
from tests._cases import torch_oracle

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
MAX_POS = 8192


def run(T, QH, KH, D, *, flash=True, dtype="bf16", apply_scale=False, reuse=True, pos_dtype="i32",
        negative_slots=False, scattered=False, trans_v=False, block_size=16, seed=42):
    tdt = torch.bfloat16 if dtype == "bf16" else torch.float16
    nb = max(32, (T + block_size - 1) // block_size + 4)
    cols = D // 2 if reuse else D
    torch.manual_seed(seed)
    q = torch.randn(T, QH, D, dtype=tdt)
    k = torch.randn(T, KH, D, dtype=tdt)
    v = torch.randn(T, KH, D, dtype=tdt)
    cos = torch.randn(MAX_POS, cols, dtype=tdt)
    sin = torch.randn(MAX_POS, cols, dtype=tdt)
    pos = torch.randint(0, MAX_POS, (T,), dtype=torch.int32)
    if scattered:
        slots = torch.randperm(nb * block_size)[:T].to(torch.int32)
    else:
        slots = torch.arange(T, dtype=torch.int32)
    if negative_slots:
        slots[1::2] = -1
    idt = torch.int32 if pos_dtype == "i32" else torch.int64
    cdt = torch.uint8 if apply_scale else tdt
    if flash:
        layout = rc.FLASH
        kc = torch.zeros(nb, block_size, KH, D, dtype=cdt)
        vc = torch.zeros(nb, block_size, KH, D, dtype=cdt)
    else:
        layout = rc.ATOM_TRANS_V if trans_v else rc.ATOM
        kc = torch.zeros(nb, KH, D // 16, block_size, 16, dtype=cdt)
        vc = (torch.zeros(nb, KH, block_size // 16, D, 16, dtype=cdt) if trans_v
              else torch.zeros(nb, KH, D, block_size, dtype=cdt))
    ks = torch.tensor([0.1], dtype=torch.float32)
    vs = torch.tensor([0.1], dtype=torch.float32)

    launch = build_fused_rope_cache_module(head_dim=D, num_q_heads=QH, num_kv_heads=KH, block_size=block_size,
                                           flash_layout=flash, dtype_str=dtype, apply_scale=apply_scale,
                                           reuse_freqs_front_part=reuse, pos_dtype=pos_dtype)
    d = {n: t.to(DEV) for n, t in dict(q=q, k=k, v=v, cos=cos, sin=sin, ks=ks, vs=vs).items()}
    pos_d, slots_d = pos.to(idt).to(DEV), slots.to(idt).to(DEV)
    kc_d = kc.to(DEV).view(torch.float8_e4m3fn) if apply_scale else kc.to(DEV)
    vc_d = vc.to(DEV).view(torch.float8_e4m3fn) if apply_scale else vc.to(DEV)
    q_out, k_out = torch.empty_like(d["q"]), torch.empty_like(d["k"])
    launch(d["q"], d["k"], d["v"], pos_d, d["cos"], d["sin"], slots_d, kc_d, vc_d, q_out, k_out, T, d["ks"], d["vs"])
    torch.cuda.synchronize()

    rq, rk, rkc, rvc = rc.rope_cache_ref(q, k, v, pos.to(idt), cos, sin, slots.to(idt), kc, vc,
                                         block_size=block_size, layout=layout, reuse_freqs_front_part=reuse,
                                         apply_scale=apply_scale, k_scale=0.1, v_scale=0.1)
    got_kc = kc_d.view(torch.uint8).cpu() if apply_scale else kc_d.cpu()
    got_vc = vc_d.view(torch.uint8).cpu() if apply_scale else vc_d.cpu()
    what = f"T={T} QH={QH} KH={KH} D={D} flash={flash} {dtype} scale={apply_scale} reuse={reuse} {pos_dtype}"
    assert torch.equal(q_out.cpu(), rq), f"q_out {what}"
    assert torch.equal(k_out.cpu(), rk), f"k_out {what}"
    assert torch.equal(got_kc, rkc), f"key cache {what}"
    assert torch.equal(got_vc, rvc), f"value cache {what}"
    # the reference test's own bounds (:380-414)
    atol = 1e-2 if dtype == "bf16" else 5e-3
    assert (q_out.cpu().float() - rq.float()).abs().max() < atol
    if apply_scale:
        deq = got_kc.view(torch.float8_e4m3fn).float() * 0.1
        kref = rc.rope_cache_ref(q, k, v, pos.to(idt), cos, sin, slots.to(idt), kc.to(tdt), vc.to(tdt),
                                 block_size=block_size, layout=layout, reuse_freqs_front_part=reuse)[2].float()
        assert (deq - kref).abs().max() <= max(1e-3, kref.abs().max() / 8)
    return q_out, k_out, kc_d, vc_d


MODELS = {
    "Llama8B-TP1": (32, 8, 128),
    "Llama8B-TP8": (4, 1, 128),
    "Llama70B-TP1": (64, 8, 128),
    "Llama405B-TP1": (128, 8, 128),
    "Qwen72B-TP1": (64, 4, 128),
    "GPTOSS-TP1": (64, 8, 64),
    "GPTOSS-TP8": (8, 1, 64),
}


@pytest.mark.parametrize("T", [1, 32, 128])
@pytest.mark.parametrize("model", sorted(MODELS))
def test_flash_bf16(model, T):
    run(T, *MODELS[model], flash=True)


@pytest.mark.parametrize("T", [1, 32, 128])
@pytest.mark.parametrize("model", ["Llama8B-TP1", "Llama8B-TP8", "GPTOSS-TP8"])
def test_nonflash_bf16(model, T):
    run(T, *MODELS[model], flash=False)


@pytest.mark.parametrize("flash", [True, False])
@pytest.mark.parametrize("T", [1, 32])
def test_f16(T, flash):
    run(T, 4, 1, 128, flash=flash, dtype="f16")


@pytest.mark.parametrize("pos_dtype", ["i32", "i64"])
@pytest.mark.parametrize("T", [1, 32, 128])
def test_pos_dtype(pos_dtype, T):
    run(T, 8, 1, 128, pos_dtype=pos_dtype)


@pytest.mark.parametrize("flash", [True, False])
@pytest.mark.parametrize("reuse", [True, False])
def test_reuse_freqs(reuse, flash):
    run(32, 8, 1, 128, flash=flash, reuse=reuse)


@pytest.mark.parametrize("flash", [True, False])
@pytest.mark.parametrize("T", [4, 32])
def test_negative_slots(T, flash):
    run(T, 8, 1, 128, flash=flash, negative_slots=True)


@pytest.mark.parametrize("flash", [True, False])
@pytest.mark.parametrize("T", [1, 32])
@pytest.mark.parametrize("D", [64, 128])
def test_fp8_cache(D, T, flash):
    run(T, 8, 1, D, flash=flash, apply_scale=True)


@pytest.mark.parametrize("flash", [True, False])
@pytest.mark.parametrize("apply_scale", [False, True])
@pytest.mark.parametrize("D", [48, 96, 192, 512])
def test_head_sizes_whose_rows_do_not_tile_a_wave(D, apply_scale, flash):
    """D / 8 lanes per row not dividing 64 (48: 6 lanes, 96: 12, 192: 24)
    leaves lanes past the last whole row idle; 512 is one row per wave.
    Decode, prefill and scattered slots, with a ragged tail."""
    for T in (1, 37, 16 * 5 + 3):
        run(T, 12, 3, D, flash=flash, apply_scale=apply_scale, scattered=T == 37, block_size=16 if flash else 32)


@pytest.mark.parametrize("apply_scale", [False, True])
@pytest.mark.parametrize("block_size", [16, 64])
def test_scattered_slots_and_decode_value_layout(block_size, apply_scale):
    run(200, 16, 4, 128, flash=False, trans_v=True, scattered=True, negative_slots=True, block_size=block_size,
        apply_scale=apply_scale)
    run(200, 16, 4, 128, flash=False, scattered=True, block_size=block_size, apply_scale=apply_scale, seed=7)


@pytest.mark.parametrize("apply_scale", [False, True])
@pytest.mark.parametrize("trans_v", [False, True])
@pytest.mark.parametrize("block_size,D", [(16, 128), (64, 128), (16, 64), (64, 64)])
def test_prefill_page_runs(block_size, D, trans_v, apply_scale):
    """Slots 0..T-1 fill whole pages in order (the prefill pattern the value
    transpose writes 16 tokens at a time), with a ragged tail."""
    run(16 * 13 + 5, 8, 2, D, flash=False, trans_v=trans_v, block_size=block_size, apply_scale=apply_scale)


def test_prefill_page_runs_misaligned():
    """A sequence starting mid-page: page runs that begin off a 16-token
    boundary take the per-token path, aligned ones the transpose."""
    T, QH, KH, D, bs = 150, 8, 2, 128, 64
    torch.manual_seed(11)
    tdt = torch.bfloat16
    q, k, v = (torch.randn(T, h, D, dtype=tdt) for h in (QH, KH, KH))
    cos = torch.randn(MAX_POS, D // 2, dtype=tdt)
    sin = torch.randn(MAX_POS, D // 2, dtype=tdt)
    pos = torch.arange(T, dtype=torch.int32) + 7
    slots = (torch.arange(T, dtype=torch.int32) + 7 + 64 * 3)  # starts at page 3, position 7
    nb = 12
    kc = torch.zeros(nb, KH, D // 16, bs, 16, dtype=torch.uint8)
    vc = torch.zeros(nb, KH, bs // 16, D, 16, dtype=torch.uint8)
    launch = build_fused_rope_cache_module(head_dim=D, num_q_heads=QH, num_kv_heads=KH, block_size=bs,
                                           flash_layout=False, apply_scale=True)
    dev = [t.to(DEV) for t in (q, k, v, pos, cos, sin, slots)]
    kc_d, vc_d = kc.to(DEV).view(torch.float8_e4m3fn), vc.to(DEV).view(torch.float8_e4m3fn)
    ks, vs = torch.tensor([0.05], device=DEV), torch.tensor([0.05], device=DEV)
    q_out, k_out = torch.empty_like(dev[0]), torch.empty_like(dev[1])
    launch(dev[0], dev[1], dev[2], dev[3], dev[4], dev[5], dev[6], kc_d, vc_d, q_out, k_out, T, ks, vs)
    torch.cuda.synchronize()
    _, _, rkc, rvc = rc.rope_cache_ref(q, k, v, pos, cos, sin, slots, kc, vc, block_size=bs, layout=rc.ATOM_TRANS_V,
                                       apply_scale=True, k_scale=0.05, v_scale=0.05)
    assert torch.equal(kc_d.view(torch.uint8).cpu(), rkc) and torch.equal(vc_d.view(torch.uint8).cpu(), rvc)


@pytest.mark.parametrize("D", [16, 32, 256])
def test_other_head_sizes(D):
    run(33, 6, 2, D, flash=True, scattered=True)
    run(33, 6, 2, D, flash=False, scattered=True, seed=3)


def test_written_cache_feeds_the_decode():
    """Write a batch's context through the writer (fp8, decode layout), then
    decode from that cache: matches attention over the written K/V."""
    B, ctx, QH, KH, D, bs = 3, 300, 8, 2, 128, 16
    T = B * ctx
    torch.manual_seed(5)
    q_new = torch.randn(T, QH, D, dtype=torch.bfloat16)
    k = torch.randn(T, KH, D, dtype=torch.bfloat16)
    v = torch.randn(T, KH, D, dtype=torch.bfloat16)
    cos = torch.randn(MAX_POS, D // 2, dtype=torch.bfloat16)
    sin = torch.randn(MAX_POS, D // 2, dtype=torch.bfloat16)
    pos = torch.arange(T, dtype=torch.int32) % ctx
    pages = -(-ctx // bs)
    nb = B * pages + 4
    table = torch.randperm(nb)[: B * pages].reshape(B, pages).to(torch.int32)
    slots = torch.cat([table[b].repeat_interleave(bs)[:ctx] * bs + torch.arange(ctx) % bs for b in range(B)])
    launch = build_fused_rope_cache_module(head_dim=D, num_q_heads=QH, num_kv_heads=KH, block_size=bs,
                                           flash_layout=False, apply_scale=True)
    kc = torch.zeros(nb, KH, D // 16, bs, 16, dtype=torch.float8_e4m3fn, device=DEV)
    vc = torch.zeros(nb, KH, bs // 16, D, 16, dtype=torch.float8_e4m3fn, device=DEV)
    ks = torch.tensor([0.02], device=DEV)
    vs = torch.tensor([0.02], device=DEV)
    q_out = torch.empty(T, QH, D, dtype=torch.bfloat16, device=DEV)
    k_out = torch.empty(T, KH, D, dtype=torch.bfloat16, device=DEV)
    launch(q_new.to(DEV), k.to(DEV), v.to(DEV), pos.to(DEV), cos.to(DEV), sin.to(DEV), slots.to(torch.int32).to(DEV),
           kc, vc, q_out, k_out, T, ks, vs)
    # decode the last token of every sequence from the written cache
    query = q_out.view(B, ctx, QH, D)[:, -1].contiguous()
    out = torch.empty_like(query)
    lens = torch.full((B,), ctx, dtype=torch.int32, device=DEV)
    pa_decode_ps_launch(out, query, kc, vc, lens, None, None, D ** -0.5, ks, vs, block_tables=table.to(DEV))
    torch.cuda.synchronize()
    case = dict(query=query.cpu(), key_cache=kc.cpu(), value_cache=vc.cpu(), block_tables=table,
                context_lengths=lens.cpu(), key_scale=ks.cpu(), value_scale=vs.cpu(), softmax_scale=D ** -0.5,
                query_length=1, sliding_window=0)
    ref = torch_oracle(case, float_out=False)
    assert torch.isclose(out.cpu().float(), ref.float(), atol=2e-2, rtol=2e-2).all()
