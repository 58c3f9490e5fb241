"""Pins the CPU oracle (oracle/reference.py) before anything is checked against it.

Three independent pins, chosen so a plausible slip fails at least one:
  1. float64 NumPy brute force (oracle/closed_form.py), written from the
     definition rather than through torch's gather + SDPA;
  2. textbook special cases: ctx == 1 returns v_0; a zero query averages V;
     a one-hot score selects one row of V; the last query of a fresh prompt
     equals decode over the same context; query 0 of a fresh prompt is v_0;
  3. planted mistakes (wrong GQA head map, off-by-one masks, dropped scale,
     reversed pages, V/K swapped, prefix ignored) must each be caught.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import closed_form, reference
from tests.helpers import assert_within, max_violation, query_starts, random_tables, scattered_cache

BS = 16


def _decode_inputs(heads, kv, d, ctx_lens, dtype=torch.float32, seed=0, pool=400):
    k, v = scattered_cache(pool, BS, kv, d, seed=seed, dtype=dtype)
    bt = random_tables(ctx_lens, BS, pool, seed=seed)
    g = torch.Generator().manual_seed(seed + 7)
    q = torch.randn(len(ctx_lens), heads, d, generator=g).to(dtype)
    ctx = torch.tensor(ctx_lens, dtype=torch.int32)
    return q, k, v, ctx, bt, d ** -0.5


def _prefill_inputs(heads, kv, d, seqs, dtype=torch.float32, seed=1, pool=400):
    k, v = scattered_cache(pool, BS, kv, d, seed=seed, dtype=dtype)
    ctx_lens = [c for _, c in seqs]
    bt = random_tables(ctx_lens, BS, pool, seed=seed)
    qs = query_starts([ql for ql, _ in seqs])
    g = torch.Generator().manual_seed(seed + 11)
    q = torch.randn(qs[-1], heads, d, generator=g).to(dtype)
    return (q, k, v, torch.tensor(qs, dtype=torch.int32), torch.tensor(ctx_lens, dtype=torch.int32), bt, d ** -0.5,
            qs, ctx_lens)


DECODE_CASES = [
    (32, 4, 64, [1, 17, 64, 100, 255, 300]),
    (8, 8, 64, [700, 33]),
    (32, 8, 128, [1, 129, 511, 1000]),
    (12, 4, 64, list(range(1, 200, 37))),
]
PREFILL_CASES = [
    (32, 4, 64, [(5, 5), (64, 64), (130, 130)]),
    (8, 8, 64, [(3, 40), (17, 17), (1, 9), (70, 200)]),
    (32, 8, 128, [(1, 1), (33, 100)]),
]


# ---------------------------------------------------------------- pin 1: float64 brute force

@pytest.mark.parametrize("heads,kv,d,ctx_lens", DECODE_CASES)
def test_decode_oracle_matches_float64_brute_force(heads, kv, d, ctx_lens):
    q, k, v, ctx, bt, scale = _decode_inputs(heads, kv, d, ctx_lens)
    got = reference.paged_decode_attention(q, k, v, ctx, bt, max(ctx_lens), scale)
    want = closed_form.decode(q, k, v, ctx, bt, scale)
    np.testing.assert_allclose(got.double().numpy(), want, atol=2e-5, rtol=1e-4)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_decode_oracle_low_precision_within_bar(dtype):
    q, k, v, ctx, bt, scale = _decode_inputs(32, 8, 128, [1, 77, 300, 1024], dtype=dtype)
    got = reference.paged_decode_attention(q, k, v, ctx, bt, 1024, scale)
    assert_within(got, closed_form.decode(q, k, v, ctx, bt, scale), what=f"oracle {dtype}")


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_fp32_accumulated_oracle_on_half_inputs_matches_float64(dtype):
    """The GPU parity checker: the reference ops on fp16/bf16 inputs upcast
    exactly to fp32 (fp32 accumulation) agree with the float64 brute force to
    ~1e-6, far inside the output tolerance, for decode and long prefill."""
    q, k, v, ctx, bt, scale = _decode_inputs(32, 8, 128, [1, 77, 300, 1024, 1500], dtype=dtype)
    got = reference.paged_decode_attention(q.float(), k.float(), v.float(), ctx, bt, 1500, scale)
    np.testing.assert_allclose(got.double().numpy(), closed_form.decode(q, k, v, ctx, bt, scale), atol=2e-5,
                               rtol=1e-4)
    args = _prefill_inputs(32, 4, 64, [(200, 201), (512, 700), (1, 1)], dtype=dtype)
    q, k, v, qst, ctxt, bt, scale, qs, ctx_lens = args
    got = reference.paged_prefill_attention(q.float(), k.float(), v.float(), qst, ctxt, bt, scale, qs, ctx_lens)
    np.testing.assert_allclose(got.double().numpy(), closed_form.prefill(q, k, v, qs, ctx_lens, bt, scale),
                               atol=2e-5, rtol=1e-4)


@pytest.mark.parametrize("heads,kv,d,seqs", PREFILL_CASES)
def test_prefill_oracle_matches_float64_brute_force(heads, kv, d, seqs):
    args = _prefill_inputs(heads, kv, d, seqs)
    q, k, v, _, _, bt, scale, qs, ctx_lens = args
    got = reference.paged_prefill_attention(*args)
    want = closed_form.prefill(q, k, v, qs, ctx_lens, bt, scale)
    np.testing.assert_allclose(got.double().numpy(), want, atol=2e-5, rtol=1e-4)


def test_decode_rows_form_equals_batched_form():
    q, k, v, ctx, bt, scale = _decode_inputs(32, 4, 64, [5, 300, 17, 1024])
    a = reference.paged_decode_attention(q, k, v, ctx, bt, 1024, scale)
    b = reference.decode_attention_rows(q, k, v, ctx.tolist(), bt, scale)
    torch.testing.assert_close(a, b, atol=1e-6, rtol=1e-5)


def test_gather_matches_slot_rule():
    k, _ = scattered_cache(50, BS, 2, 8, seed=3)
    bt = random_tables([37], BS, 50, seed=3)
    got = reference.gather_kv(k, bt[0], 37).numpy()
    want = closed_form.token_rows(k, bt[0], 37)
    np.testing.assert_array_equal(got, want)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_write_kv_oracle_is_a_bitwise_scatter(dtype):
    kc, vc = scattered_cache(30, BS, 4, 64, seed=5, dtype=dtype)
    g = torch.Generator().manual_seed(5)
    slots = torch.randperm(30 * BS, generator=g)[:77].to(torch.int64)
    k = torch.randn(77, 4, 64, generator=g).to(dtype)
    v = torch.randn(77, 4, 64, generator=g).to(dtype)
    want_k, want_v = closed_form.write_kv(k.view(torch.int16), v.view(torch.int16), kc.view(torch.int16),
                                          vc.view(torch.int16), slots)
    reference.write_kv(k, v, kc, vc, slots)
    np.testing.assert_array_equal(kc.view(torch.int16).numpy(), want_k)
    np.testing.assert_array_equal(vc.view(torch.int16).numpy(), want_v)


def test_write_then_gather_roundtrip():
    """Tokens written at slot table[p // 16] * 16 + p % 16 (nimbus/runner.py:61)
    come back from gather_kv at position p."""
    kc, vc = scattered_cache(40, BS, 2, 16, seed=9, dtype=torch.float32)
    bt = random_tables([70], BS, 40, seed=9)
    table = bt[0].tolist()
    pos = torch.arange(20, 70)
    slots = torch.tensor([table[p // BS] * BS + p % BS for p in pos.tolist()], dtype=torch.int64)
    k = torch.randn(50, 2, 16)
    reference.write_kv(k, k.clone(), kc, vc, slots)
    torch.testing.assert_close(reference.gather_kv(kc, bt[0], 70)[20:70], k, atol=0, rtol=0)


# ---------------------------------------------------------------- pin 2: textbook special cases

@pytest.mark.parametrize("impl", ["reference", "closed_form"])
def test_context_of_one_returns_first_value_row(impl):
    q, k, v, ctx, bt, scale = _decode_inputs(8, 2, 64, [1, 1, 1])
    out = _decode(impl, q, k, v, ctx, bt, scale)
    for b in range(3):
        page = int(bt[b, 0])
        want = v[page, 0].double().repeat_interleave(4, 0).numpy()  # head h uses kv head h // 4
        np.testing.assert_allclose(out[b], want, atol=1e-6)


@pytest.mark.parametrize("impl", ["reference", "closed_form"])
def test_zero_query_averages_values(impl):
    q, k, v, ctx, bt, scale = _decode_inputs(8, 2, 32, [40, 7])
    q.zero_()
    out = _decode(impl, q, k, v, ctx, bt, scale)
    for b, c in enumerate([40, 7]):
        rows = closed_form.token_rows(v, bt[b], c)  # [c, KV, D]
        want = rows.mean(axis=0).repeat(4, axis=0)
        np.testing.assert_allclose(out[b], want, atol=1e-5)


@pytest.mark.parametrize("impl", ["reference", "closed_form"])
def test_one_hot_score_selects_one_value_row(impl):
    heads, kv, d, c = 4, 2, 16, 45
    q, k, v, ctx, bt, _ = _decode_inputs(heads, kv, d, [c])
    k.zero_()
    j = 29  # the selected token
    page, row = int(bt[0, j // BS]), j % BS
    k[page, row, :, 0] = 1.0
    q.zero_()
    q[0, :, 0] = 1000.0
    out = _decode(impl, q, k, v, ctx, bt, 1.0)
    want = v[page, row].double().repeat_interleave(2, 0).numpy()
    np.testing.assert_allclose(out[0], want, atol=1e-6)


@pytest.mark.parametrize("impl", ["reference", "closed_form"])
def test_fresh_prompt_first_query_sees_only_first_key(impl):
    args = _prefill_inputs(8, 2, 64, [(50, 50)])
    out = _prefill(impl, args)
    page = int(args[5][0, 0])
    want = args[2][page, 0].double().repeat_interleave(4, 0).numpy()
    np.testing.assert_allclose(out[0], want, atol=1e-6)


@pytest.mark.parametrize("impl", ["reference", "closed_form"])
def test_last_prefill_query_equals_decode_over_same_context(impl):
    args = _prefill_inputs(8, 2, 64, [(30, 95)])
    q, k, v, _, ctx, bt, scale, _, _ = args
    pre = _prefill(impl, args)
    dec = _decode(impl, q[-1:], k, v, ctx, bt, scale)
    np.testing.assert_allclose(pre[-1], dec[0], atol=1e-6)


def _decode(impl, q, k, v, ctx, bt, scale):
    if impl == "reference":
        return reference.paged_decode_attention(q, k, v, ctx, bt, int(ctx.max()), scale).double().numpy()
    return closed_form.decode(q, k, v, ctx, bt, scale)


def _prefill(impl, args):
    if impl == "reference":
        return reference.paged_prefill_attention(*args).double().numpy()
    q, k, v, _, _, bt, scale, qs, ctx_lens = args
    return closed_form.prefill(q, k, v, qs, ctx_lens, bt, scale)


# ---------------------------------------------------------------- pin 3: planted mistakes are caught

def _mutant_decode(kind, q, k_cache, v_cache, context_lens, block_tables, max_context, scale):
    """oracle.reference.paged_decode_attention with one planted mistake."""
    b, h, d = q.shape
    kv = k_cache.shape[2]
    nb = -(-max_context // BS)
    bt = block_tables[:, :nb].long()
    if kind == "reversed_pages":
        bt = bt.flip(1)
    k = k_cache[bt].flatten(1, 2).transpose(1, 2)
    v = v_cache[bt].flatten(1, 2).transpose(1, 2)
    if kind == "swap_kv":
        v = k
    if kind == "gqa_modulo":
        k = k.repeat(1, h // kv, 1, 1)
        v = v.repeat(1, h // kv, 1, 1)
    else:
        k = k.repeat_interleave(h // kv, 1)
        v = v.repeat_interleave(h // kv, 1)
    lim = context_lens[:, None] - (1 if kind == "mask_off_by_one" else 0)
    mask = torch.arange(k.shape[2])[None, :] < lim
    s = 1.0 if kind == "no_scale" else scale
    o = F.scaled_dot_product_attention(q.unsqueeze(2), k, v, attn_mask=mask[:, None, None, :], scale=s)
    return o.view(b, h, d)


@pytest.mark.parametrize("kind", ["reversed_pages", "swap_kv", "gqa_modulo", "mask_off_by_one", "no_scale"])
def test_planted_decode_mistakes_are_caught(kind):
    q, k, v, ctx, bt, scale = _decode_inputs(32, 4, 64, [2, 17, 100, 300])
    want = closed_form.decode(q, k, v, ctx, bt, scale)
    good = reference.paged_decode_attention(q, k, v, ctx, bt, 300, scale)
    assert max_violation(good, want) <= 0
    bad = _mutant_decode(kind, q, k, v, ctx, bt, 300, scale)
    assert not (max_violation(torch.nan_to_num(bad, nan=1e9), want) <= 0), kind


def _mutant_prefill(kind, q, k_cache, v_cache, qs, ctx_lens, bt, scale):
    out = torch.empty_like(q)
    for i, ctx in enumerate(ctx_lens):
        s, e = qs[i], qs[i + 1]
        ql = e - s
        qi = q[s:e].transpose(0, 1).unsqueeze(0)
        ki = reference.gather_kv(k_cache, bt[i], ctx).transpose(0, 1).unsqueeze(0)
        vi = reference.gather_kv(v_cache, bt[i], ctx).transpose(0, 1).unsqueeze(0)
        base = 0 if kind == "ignores_prefix" else ctx - ql
        qpos = torch.arange(base, base + ql)[:, None]
        kpos = torch.arange(ctx)[None, :]
        allowed = kpos < qpos if kind == "strict_causal" else kpos <= qpos
        o = F.scaled_dot_product_attention(qi, ki, vi, attn_mask=allowed, scale=scale, enable_gqa=True)
        out[s:e] = o[0].transpose(0, 1)
    return out


@pytest.mark.parametrize("kind", ["strict_causal", "ignores_prefix"])
def test_planted_prefill_mistakes_are_caught(kind):
    args = _prefill_inputs(8, 2, 64, [(3, 40), (17, 17), (70, 200)])
    q, k, v, _, _, bt, scale, qs, ctx_lens = args
    want = closed_form.prefill(q, k, v, qs, ctx_lens, bt, scale)
    assert max_violation(reference.paged_prefill_attention(*args), want) <= 0
    bad = _mutant_prefill(kind, q, k, v, qs, ctx_lens, bt, scale)
    assert not (max_violation(torch.nan_to_num(bad, nan=1e9), want) <= 0), kind


# ---------------------------------------------------------------- fused residual add + RMSNorm

@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_add_rms_norm_residual_is_the_element_type_add(dtype):
    """The new residual is x + r rounded once to the element type (NumPy's
    float16 addition is IEEE; bf16 is checked through float32, where the
    exact sum of two bf16 values fits)."""
    g = torch.Generator().manual_seed(5)
    x = (torch.randn(7, 256, generator=g) * 3).to(dtype)
    r = (torch.randn(7, 256, generator=g) * 3).to(dtype)
    w = torch.randn(256, generator=g).to(dtype)
    _, res = reference.add_rms_norm(x, r, w, 1e-5)
    if dtype == torch.float16:
        want = (x.numpy() + r.numpy()).astype(np.float16)
        assert np.array_equal(res.numpy().view(np.uint16), want.view(np.uint16))
    else:
        want = (x.float() + r.float()).to(torch.bfloat16)
        assert torch.equal(res.view(torch.int16), want.view(torch.int16))


@pytest.mark.parametrize("rows,cols", [(1, 2048), (37, 2048), (5, 768), (3, 4096)])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_rms_norm_oracle_matches_float64(rows, cols, dtype):
    """The restated norm (float32 normalise, two roundings to the element
    type) is within a few element-type ulps of the float64 definition."""
    g = torch.Generator().manual_seed(rows * 31 + cols)
    x = torch.randn(rows, cols, generator=g).to(dtype)
    w = torch.randn(cols, generator=g).to(dtype)
    got = reference.rms_norm(x, w, 1e-5).float().numpy()
    want = closed_form.rms_norm(x, w, 1e-5)
    ulp = 2.0 ** -10 if dtype == torch.float16 else 2.0 ** -7
    assert np.all(np.abs(got - want) <= 2 * ulp * np.abs(want) + 1e-6)


def test_rms_norm_of_a_constant_row_is_its_sign():
    """mean(x^2) = c^2, so x / sqrt(c^2 + eps) = sign(c) (for eps << c^2)."""
    x = torch.tensor([[2.5] * 64, [-0.75] * 64], dtype=torch.float16)
    w = torch.ones(64, dtype=torch.float16)
    got = reference.rms_norm(x, w, 1e-6)
    assert torch.equal(got[0], torch.ones(64, dtype=torch.float16))
    assert torch.equal(got[1], -torch.ones(64, dtype=torch.float16))
    assert np.allclose(closed_form.rms_norm(x, w, 1e-6), np.sign(x.float().numpy()), atol=1e-6)


@pytest.mark.parametrize("kind", ["no_eps", "wrong_axis", "weight_before_cast_missing", "sum_not_mean"])
def test_planted_rms_norm_mistakes_are_caught(kind):
    """The float64 check rejects plausible slips in the norm."""
    g = torch.Generator().manual_seed(11)
    x = torch.randn(6, 64, generator=g, dtype=torch.float32)
    w = torch.randn(64, generator=g, dtype=torch.float32)
    eps = 0.5  # large enough that dropping it shows
    if kind == "no_eps":
        bad = w * x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True))
    elif kind == "wrong_axis":
        bad = w * x * torch.rsqrt(x.pow(2).mean(0, keepdim=True) + eps)
    elif kind == "weight_before_cast_missing":
        bad = x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps)
    else:
        bad = w * x * torch.rsqrt(x.pow(2).sum(-1, keepdim=True) + eps)
    want = closed_form.rms_norm(x, w, eps)
    assert np.allclose(reference.rms_norm(x, w, eps).numpy(), want, atol=1e-5)
    assert not np.allclose(bad.numpy(), want, atol=1e-3)


# ---------------------------------------------------------------- INT8 weight-only matmul

def test_quantize_roundtrip_error_is_within_half_a_step():
    """nimbus's own check (tests/test_quant.py:7-13): |dequant(q) - w| <= s / 2."""
    g = torch.Generator().manual_seed(0)
    w = torch.randn(64, 300, generator=g) * torch.rand(64, 1, generator=g) * 3
    q, s = reference.quantize_weight(w)
    assert q.dtype == torch.int8 and int(q.abs().max()) <= 127
    err = (reference.dequantize_weight(q, s) - w).abs()
    assert bool((err <= s[:, None] / 2 + 1e-6).all())


def test_quantize_maps_each_row_maximum_to_127_and_zero_rows_to_zero():
    w = torch.tensor([[0.5, -2.0, 1.0, 0.0], [3.0, 1.5, -0.25, 0.1], [0.0, 0.0, 0.0, 0.0]])
    q, s = reference.quantize_weight(w)
    assert q.tolist()[0] == [32, -127, 64, 0]  # 0.5 / (2 / 127) = 31.75 -> 32
    assert q.tolist()[1][0] == 127 and q.tolist()[2] == [0, 0, 0, 0]
    assert np.allclose(s.numpy(), [2 / 127, 3 / 127, 1e-8 / 127])


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_int8_matmul_oracle_is_exact_on_small_integers(dtype):
    """Integer x and q with a power-of-two scale: the fp32 sum is exact, so
    the oracle equals the float64 product rounded once to the element type."""
    g = torch.Generator().manual_seed(3)
    x = torch.randint(-3, 4, (9, 48), generator=g).to(dtype)
    q = torch.randint(-127, 128, (20, 48), generator=g).to(torch.int8)
    s = torch.full((20,), 2.0 ** -7).to(dtype) * torch.randint(1, 4, (20,), generator=g).to(dtype)
    got = reference.int8_matmul(x, q, s)
    want = torch.from_numpy(closed_form.int8_matmul(x, q, s)).to(dtype)
    assert torch.equal(got, want)


@pytest.mark.parametrize("m,n,k", [(1, 64, 2048), (7, 40, 96), (64, 128, 5632)])
def test_int8_matmul_oracle_matches_float64(m, n, k):
    """fp16 inputs, real-valued scales: within one fp16 rounding of float64,
    and equal to the dequantized-weight product (tests/test_quant.py:16-21)."""
    g = torch.Generator().manual_seed(m + n + k)
    w = torch.randn(n, k, generator=g) * 0.02
    q, s = reference.quantize_weight(w.half())
    x = torch.randn(m, k, generator=g).half()
    got = reference.int8_matmul(x, q, s).double().numpy()
    want = closed_form.int8_matmul(x, q, s)
    assert np.all(np.abs(got - want) <= 2.0 ** -10 * np.abs(want) + 1e-4)
    deq = x.float() @ reference.dequantize_weight(q, s.float()).T
    assert np.allclose(reference.int8_matmul(x.float(), q, s.float()).numpy(), deq.numpy(), atol=1e-5, rtol=1e-5)


@pytest.mark.parametrize("kind", ["no_scale", "scale_per_token", "transposed_weight", "x_rounded"])
def test_planted_int8_matmul_mistakes_are_caught(kind):
    """The float64 check and the reference's bar (atol 2e-2, rtol 1e-2) reject
    plausible slips in the int8 product."""
    g = torch.Generator().manual_seed(8)
    n = k = 64
    w = torch.randn(n, k, generator=g) * 0.05
    q, s = reference.quantize_weight(w)
    x = torch.randn(n, k, generator=g) * 2
    want = closed_form.int8_matmul(x, q, s)
    if kind == "no_scale":
        bad = x @ q.float().T
    elif kind == "scale_per_token":
        bad = (x @ q.float().T) * s[:, None]
    elif kind == "transposed_weight":
        bad = (x @ q.float()) * s
    else:
        bad = (torch.round(x) @ q.float().T) * s
    assert max_violation(reference.int8_matmul(x, q, s), want, 2e-2, 1e-2) <= 0
    assert max_violation(bad, want, 2e-2, 1e-2) > 0
