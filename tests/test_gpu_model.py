"""GPU: the Llama decoder on this build's kernels, its whole-step decode
graphs and the on-device greedy chain.

- The model (fp16 and bf16, random weights) against oracle/model.py (the
  CPU fp32 restatement of nimbus/model/llama.py, itself pinned to HF's
  Llama): a mixed prefill step of three prompts, then greedy decode steps,
  logits within a bar set by the element type.
- Decode steps replayed from DecodeGraphs against the eager model
  (nimbus's test_cuda_graph_decode_matches_eager, test_kernels.py:118-142):
  the same greedy tokens, logits within rounding, batches padded to captured
  sizes; replays are repeatable bit for bit.
- greedy_chain against step-by-step graph runs with host argmax: identical
  tokens (the same kernels), and every graph replay equals the eager call.
- The INT8-quantized model stays close to the unquantized one
  (nimbus's test_quantized_tiny_model_stays_close: cosine > 0.99); its
  MLP (gate_up with the SiLU gate in the epilogue) equals the separate
  launches within rounding, and its decode graphs match its eager steps.
- The rotary, SiLU and greedy-step kernels against torch.
"""

from __future__ import annotations

import random

import pytest
import torch
import torch.nn.functional as F

from nimbus_amd.graphs import DecodeGraphs, VerifyGraphs
from nimbus_amd.kernels import cache_ops
from nimbus_amd.kernels.elementwise import greedy_step, rope_, silu_mul
from nimbus_amd.model.attention import AttnMetadata
from nimbus_amd.model.config import ModelConfig
from nimbus_amd.model.llama import build_model
from nimbus_amd.quant import quantize_model
from nimbus_amd.workloads import SeqState, flat_step, is_decode
from oracle import model as omodel
from tests.gpu_helpers import announce

pytestmark = pytest.mark.gpu

CFG = ModelConfig(vocab_size=1000, hidden_size=256, intermediate_size=512, num_layers=2, num_heads=4,
                  num_kv_heads=2, head_dim=64, rms_norm_eps=1e-5, rope_theta=10000.0, max_position=1024)
BS = 16


def _setup(dtype, prompt_lens, num_blocks=96, seed=0, cfg=CFG):
    model = build_model(cfg, dtype, "cuda", seed, max_position=cfg.max_position)
    shape = (num_blocks + 1, BS, cfg.num_kv_heads, cfg.head_dim)  # + the scratch block (num_blocks)
    caches = [(torch.zeros(shape, dtype=dtype, device="cuda"), torch.zeros(shape, dtype=dtype, device="cuda"))
              for _ in range(cfg.num_layers)]
    rng = random.Random(seed)
    pool = rng.sample(range(num_blocks), num_blocks)
    seqs = []
    for i, n in enumerate(prompt_lens):
        ids = [rng.randrange(1, cfg.vocab_size) for _ in range(n)]
        seqs.append(SeqState(ids, [pool.pop() for _ in range(-(-(n + 24) // BS))]))  # room for 24 more tokens
    return model, caches, seqs


def _cpu_meta(meta: AttnMetadata) -> AttnMetadata:
    c = lambda t: t.cpu()  # noqa: E731
    return AttnMetadata(c(meta.slot_mapping), meta.num_prefill_tokens, c(meta.prefill_query_start),
                        c(meta.prefill_context_lens), c(meta.prefill_block_tables), c(meta.decode_context_lens),
                        c(meta.decode_block_tables), meta.max_decode_context, meta.prefill_query_start_host,
                        meta.prefill_context_lens_host)


def _eager_step(model, caches, batch):
    step = flat_step(batch, "cuda", BS)
    logits = model.logits(model(step.input_ids, step.positions, caches, step.meta))
    return step, logits[step.sample_rows]


@pytest.mark.parametrize("dtype,atol", [(torch.float16, 2e-2), (torch.bfloat16, 6e-2)])
def test_model_matches_oracle_prefill_then_decode(dtype, atol):
    announce(f"model vs oracle {dtype}")
    model, caches, seqs = _setup(dtype, [5, 17, 40])
    w = {k: v.float().cpu() for k, v in model.state_dict().items()}
    ocaches = [(torch.zeros(kc.shape), torch.zeros(vc.shape)) for kc, vc in caches]
    batch = [(s, len(s)) for s in seqs]
    for step_i in range(4):
        step, got = _eager_step(model, caches, batch)
        meta = _cpu_meta(step.meta)
        hid = omodel.forward(w, CFG, step.input_ids.cpu(), step.positions.cpu(), ocaches, meta, CFG.max_position)
        want = omodel.logits(w, hid)[step.sample_rows.cpu()]
        got = got.cpu()
        err = (got - want).abs().max().item()
        announce(f"  step {step_i}: max |logit error| {err:.2e} (logit scale {want.abs().max().item():.2f})")
        assert err <= atol * max(1.0, want.abs().max().item()), err
        for s, tok in zip(seqs, got.argmax(-1).tolist()):  # same inputs for both next step
            s.feed(tok)
        batch = [(s, 1) for s in seqs]


def _prefill(model, caches, seqs):
    _, logits = _eager_step(model, caches, [(s, len(s)) for s in seqs])
    for s, tok in zip(seqs, logits.argmax(-1).tolist()):
        s.feed(tok)


def _clone_seqs(seqs):
    return [s.copy() for s in seqs]


def _clone_caches(caches):
    return [(kc.clone(), vc.clone()) for kc, vc in caches]


def test_interleaved_batches_match_solo_runs():
    """The property of nimbus tests/test_paged.py:63-95 on the GPU path:
    sequences whose prompts go through in random chunks while others
    decode, on scattered blocks, produce their solo runs' results. Both runs
    feed the solo run's tokens (the interleaved run is teacher-forced), and
    every sampled logits row matches the solo row within rounding, with the
    same argmax wherever the solo row's top two differ by more than 0.05 (the
    batch moves decode's split points, so rows can differ in the last bits,
    which the reference's fp32 CPU run does not)."""
    announce("interleaved chunked batches vs solo runs")
    model, caches, _ = _setup(torch.float16, [], num_blocks=200, seed=31)
    rng = random.Random(1)
    prompts = [[rng.randrange(1, CFG.vocab_size) for _ in range(rng.randrange(1, 40))] for _ in range(6)]
    n_new = 12
    solo = []
    for p in prompts:
        s = SeqState(list(p), list(range(-(-(len(p) + n_new) // BS))))
        rows = []
        _, lg = _eager_step(model, caches, [(s, len(s))])
        for i in range(n_new):
            rows.append(lg[0].clone())
            s.feed(int(lg[0].argmax()))
            if i + 1 < n_new:
                _, lg = _eager_step(model, caches, [(s, 1)])
        solo.append((list(s.token_ids), rows))

    pool = rng.sample(range(200), 200)
    seqs = [SeqState(list(p), [pool.pop() for _ in range(-(-(len(p) + n_new) // BS))]) for p in prompts]
    got = [0] * len(seqs)
    waiting, running = list(range(len(seqs))), []
    checked = 0
    while any(g < n_new for g in got):
        for _ in range(2):
            if waiting:
                running.append(waiting.pop(0))
        active = [i for i in running if got[i] < n_new]
        pre = [i for i in active if not is_decode(seqs[i], len(seqs[i]) - seqs[i].num_computed)]
        dec = [i for i in active if i not in pre]
        batch = [(seqs[i], min(len(seqs[i]) - seqs[i].num_computed, rng.randrange(1, 12))) for i in pre]
        batch += [(seqs[i], 1) for i in dec]
        order = pre + dec
        _, lg = _eager_step(model, caches, batch)
        row = 0
        for i, (s, n) in zip(order, batch):
            s.num_computed += n
            if s.num_computed < len(s):
                continue
            want = solo[i][1][got[i]]
            torch.testing.assert_close(lg[row], want, atol=1e-2, rtol=1e-2)
            top2 = want.topk(2).values
            if float(top2[0] - top2[1]) > 0.05:
                assert int(lg[row].argmax()) == int(want.argmax()), (i, got[i])
            row += 1
            checked += 1
            s.token_ids.append(solo[i][0][len(s)])  # the solo run's next token
            got[i] += 1
        assert row == lg.shape[0]
    assert checked == len(prompts) * n_new


@pytest.mark.parametrize("n,dtype", [(5, torch.float16), (3, torch.bfloat16), (16, torch.float16)])
def test_decode_graphs_match_eager(n, dtype):
    announce(f"decode graphs n={n} {dtype}")
    model, caches, seqs = _setup(dtype, [3 + 7 * i for i in range(n)], num_blocks=160, seed=n)
    _prefill(model, caches, seqs)
    g_seqs, e_seqs = _clone_seqs(seqs), _clone_seqs(seqs)
    g_caches, e_caches = _clone_caches(caches), _clone_caches(caches)
    graphs = DecodeGraphs(model, g_caches, BS, max_model_len=512, max_batch=16, scratch_block=160,
                          num_kv_heads=CFG.num_kv_heads, device="cuda")
    graphs.capture()
    for step_i in range(5):
        assert graphs.can_run([(s, 1) for s in g_seqs])
        got = graphs.run(g_seqs).clone()
        _, want = _eager_step(model, e_caches, [(s, 1) for s in e_seqs])
        torch.testing.assert_close(got, want, atol=1e-2, rtol=1e-2)
        g_tok, e_tok = got.argmax(-1).tolist(), want.argmax(-1).tolist()
        assert g_tok == e_tok, (step_i, g_tok, e_tok)
        for s, t in zip(g_seqs, g_tok):
            s.feed(t)
        for s, t in zip(e_seqs, e_tok):
            s.feed(t)


@pytest.mark.parametrize("n,dtype,kernel", [(3, torch.float16, "auto"), (5, torch.bfloat16, "auto"),
                                             (8, torch.float16, "tile")])
def test_verify_graphs_match_eager(n, dtype, kernel):
    """The whole-model verification graph (nimbus/spec/engine.py:60-150):
    every sequence feeds its pending token and k drafts; the replayed logits
    of all k + 1 rows equal an eager forward pass over the same tokens within
    rounding, with the same argmax, over three rounds in which a prefix of
    the drafts is kept and the rest overwritten."""
    announce(f"verify graphs n={n} {dtype} {kernel}")
    k = 4
    q = k + 1
    model, caches, seqs = _setup(dtype, [3 + 9 * i for i in range(n)], num_blocks=160, seed=20 + n)
    _prefill(model, caches, seqs)
    g_seqs, e_seqs = _clone_seqs(seqs), _clone_seqs(seqs)
    g_caches, e_caches = _clone_caches(caches), _clone_caches(caches)
    graphs = VerifyGraphs(model, g_caches, BS, max_model_len=512, max_batch=8, k=k, scratch_block=160,
                          device="cuda", kernel=kernel)
    graphs.capture()
    rng = random.Random(n)
    for round_i in range(3):
        drafts = [[rng.randrange(1, CFG.vocab_size) for _ in range(k)] for _ in range(n)]
        for ss in (g_seqs, e_seqs):
            for s, d in zip(ss, drafts):
                s.token_ids.extend(d)
        got = graphs.run(g_seqs).clone()
        step = flat_step([(s, q) for s in e_seqs], "cuda", BS)
        want = model.logits(model(step.input_ids, step.positions, e_caches, step.meta))
        assert got.shape == want.shape == (n * q, CFG.vocab_size)
        torch.testing.assert_close(got, want, atol=1e-2, rtol=1e-2)
        g_tok, e_tok = got.argmax(-1).view(n, q).tolist(), want.argmax(-1).view(n, q).tolist()
        assert g_tok == e_tok, round_i
        # keep a prefix of each sequence's drafts, then the target's token after it
        for i in range(n):
            keep = rng.randrange(0, k + 1)
            for ss in (g_seqs, e_seqs):
                s = ss[i]
                del s.token_ids[len(s) - k + keep:]
                s.num_computed = len(s)
                s.token_ids.append(g_tok[i][keep])
    for (ka, va), (kb, vb) in zip(g_caches, e_caches):
        torch.testing.assert_close(ka[:160], kb[:160], atol=1e-2, rtol=1e-2)
        torch.testing.assert_close(va[:160], vb[:160], atol=1e-2, rtol=1e-2)


def test_greedy_chain_matches_stepwise_runs():
    """The chain's on-device argmax and state advance equal host-side
    argmax + _load between single-step replays, token for token."""
    announce("greedy chain")
    model, caches, seqs = _setup(torch.float16, [9, 30, 4, 51, 17], num_blocks=160, seed=11)
    _prefill(model, caches, seqs)
    a_seqs, b_seqs = _clone_seqs(seqs), _clone_seqs(seqs)
    a_caches, b_caches = _clone_caches(caches), _clone_caches(caches)
    steps = 12
    ga = DecodeGraphs(model, a_caches, BS, 512, 8, 160, CFG.num_kv_heads, "cuda", max_chain=32)
    ga.capture()
    chain = ga.greedy_chain(a_seqs, steps).cpu()
    gb = DecodeGraphs(model, b_caches, BS, 512, 8, 160, CFG.num_kv_heads, "cuda")
    gb.capture()
    for k in range(steps):
        toks = gb.run(b_seqs).argmax(-1).tolist()
        assert toks == chain[:, k].tolist(), k
        for s, t in zip(b_seqs, toks):
            s.feed(t)
    # both graph paths wrote the same K/V into their caches
    for (ka, va), (kb, vb) in zip(a_caches, b_caches):
        assert torch.equal(ka[:160], kb[:160]) and torch.equal(va[:160], vb[:160])


def test_int8_model_stays_close():
    announce("int8 model vs fp16")
    model, caches, seqs = _setup(torch.float16, [12, 33, 7], seed=5)
    q_model, _, _ = _setup(torch.float16, [12, 33, 7], seed=5)
    quantize_model(q_model)
    assert q_model.layers[0].mlp.down_proj.weight_q.dtype == torch.int8
    q_caches = _clone_caches(caches)
    batch = [(s, len(s)) for s in seqs]
    q_seqs = _clone_seqs(seqs)
    q_batch = [(s, len(s)) for s in q_seqs]
    for _ in range(4):
        _, ref = _eager_step(model, caches, batch)
        _, got = _eager_step(q_model, q_caches, q_batch)
        cos = F.cosine_similarity(ref, got, dim=-1)
        assert cos.min().item() > 0.99, cos
        toks = ref.argmax(-1).tolist()  # feed both the unquantized model's tokens
        for s, t in zip(seqs, toks):
            s.feed(t)
        for s, t in zip(q_seqs, toks):
            s.feed(t)
        batch = [(s, 1) for s in seqs]
        q_batch = [(s, 1) for s in q_seqs]


@pytest.mark.parametrize("n,dtype", [(5, torch.bfloat16), (16, torch.float16)])
def test_int8_decode_graphs_match_eager(n, dtype):
    """The INT8-quantized model, whose MLP runs the gate_up projection with
    the SiLU gate in its epilogue: its MLP equals the projection, then
    silu_mul, then down_proj, within rounding (each wrapper tunes its own
    launch plan, so the sums over K may be added in another order; under
    one plan the two are equal bit for bit, tests/test_gpu_int8.py); its
    decode steps replayed from DecodeGraphs give the eager steps' greedy
    tokens and logits within rounding."""
    announce(f"int8 decode graphs n={n} {dtype}")
    model, caches, seqs = _setup(dtype, [3 + 7 * i for i in range(n)], num_blocks=160, seed=40 + n)
    quantize_model(model)
    mlp = model.layers[0].mlp
    x = torch.randn(n, CFG.hidden_size, device="cuda").to(dtype)
    assert mlp.gate_up_proj.forward_silu(x) is not None  # the fused path is the one MLP.forward takes
    torch.testing.assert_close(mlp(x), mlp.down_proj(silu_mul(mlp.gate_up_proj(x))), atol=1e-2, rtol=1e-2)
    _prefill(model, caches, seqs)
    g_seqs, e_seqs = _clone_seqs(seqs), _clone_seqs(seqs)
    g_caches, e_caches = _clone_caches(caches), _clone_caches(caches)
    graphs = DecodeGraphs(model, g_caches, BS, max_model_len=512, max_batch=16, scratch_block=160,
                          num_kv_heads=CFG.num_kv_heads, device="cuda")
    graphs.capture()
    for step_i in range(4):
        got = graphs.run(g_seqs).clone()
        _, want = _eager_step(model, e_caches, [(s, 1) for s in e_seqs])
        torch.testing.assert_close(got, want, atol=1e-2, rtol=1e-2)
        g_tok, e_tok = got.argmax(-1).tolist(), want.argmax(-1).tolist()
        assert g_tok == e_tok, (step_i, g_tok, e_tok)
        for ss in (g_seqs, e_seqs):
            for s, t in zip(ss, e_tok):
                s.feed(t)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_int8_split_partials_folded_into_the_norms_give_the_same_logits(dtype):
    """With split plans for o_proj and down_proj (forced here; the tuner
    picks them where they are faster), the decoder layer's norms fold the
    projections' split-K partials in themselves: the logits are bit for bit
    those of the same model with the partials reduced by their own launch,
    over a prefill step and decode steps, eager and graph-replayed."""
    from nimbus_amd.kernels import int8_matmul as im

    announce(f"int8 split partials into the norms {dtype}")
    model, caches, seqs = _setup(dtype, [9, 30, 4, 51, 17], num_blocks=160, seed=13)
    quantize_model(model)
    saved = dict(im._TUNED)
    try:
        for m in (1, 2, 4, 8, 16, 32, 64, 111):  # every bucket the steps below use
            for n, k in ((CFG.hidden_size, CFG.num_heads * CFG.head_dim), (CFG.hidden_size, CFG.intermediate_size)):
                im._TUNED[(im.m_bucket(m), n, k, dtype, 0)] = (16, 1, 2, 1)
        runs = []
        for defer in (True, False):
            im.DEFER_SPLITS = defer
            c, ss = _clone_caches(caches), _clone_seqs(seqs)
            _, lg = _eager_step(model, c, [(s, len(s)) for s in ss])
            out = [lg]
            for s, t in zip(ss, lg.argmax(-1).tolist()):
                s.feed(t)
            graphs = DecodeGraphs(model, c, BS, max_model_len=512, max_batch=8, scratch_block=160,
                                  num_kv_heads=CFG.num_kv_heads, device="cuda")
            graphs.capture()
            for _ in range(3):
                lg = graphs.run(ss).clone()
                out.append(lg)
                for s, t in zip(ss, lg.argmax(-1).tolist()):
                    s.feed(t)
            torch.cuda.synchronize()
            runs.append(out)
        for a, b in zip(*runs):
            assert torch.equal(a, b)
    finally:
        im.DEFER_SPLITS = True
        im._TUNED.clear()
        im._TUNED.update(saved)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("heads,d", [(40, 128), (6, 64)])
def test_rope_kernel_is_the_reference_arithmetic(dtype, heads, d):
    """x * cos + rotate_half(x) * sin in the element type, tables cast from
    fp32 (nimbus/model/llama.py:49-58), bit for bit; a position outside the
    table leaves its row alone."""
    announce(f"rope {dtype} heads={heads} d={d}")
    g = torch.Generator(device="cuda").manual_seed(d)
    t = 37
    x = torch.randn(t, heads * d + 3 * 8, generator=g, device="cuda").to(dtype)  # row wider than the heads
    pos = torch.randint(0, 500, (t,), generator=g, device="cuda")
    pos[5] = 600  # past the table
    ang = torch.arange(512, device="cuda", dtype=torch.float32)[:, None] * torch.rand(d // 2, generator=g,
                                                                                      device="cuda")[None]
    ang = torch.cat([ang, ang], -1)
    cos, sin = ang.cos(), ang.sin()
    got = rope_(x.clone(), heads, d, pos, cos, sin)
    xh = x[:, :heads * d].view(t, heads, d)
    pc = pos.clamp(max=511)
    c, s = cos[pc].to(dtype)[:, None, :], sin[pc].to(dtype)[:, None, :]
    rot = torch.cat([-xh[..., d // 2:], xh[..., :d // 2]], -1)
    want = (xh * c + rot * s).view(t, heads * d)
    keep = torch.ones(t, dtype=torch.bool, device="cuda")
    keep[5] = False
    assert torch.equal(got[keep, :heads * d], want[keep])
    assert torch.equal(got[5], x[5]) and torch.equal(got[:, heads * d:], x[:, heads * d:])


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("heads,kv,d,t", [(32, 8, 128, 301), (32, 4, 64, 37), (8, 8, 64, 1), (32, 8, 128, 2108)])
def test_rope_write_kv_is_rope_then_write_kv(dtype, heads, kv, d, t):
    """The fused launch leaves qkv and both caches exactly as rope_ on the q
    and k heads followed by write_kv of the k and v heads do, including a
    position past the table (its k goes to the cache unrotated) and slots
    outside the cache (skipped)."""
    announce(f"rope_write_kv {dtype} heads={heads} kv={kv} d={d} t={t}")
    g = torch.Generator(device="cuda").manual_seed(d + t)
    width = (heads + 2 * kv) * d
    qkv = torch.randn(t, width + 8, generator=g, device="cuda").to(dtype)  # rows wider than the heads
    pos = torch.randint(0, 500, (t,), generator=g, device="cuda")
    blocks = (t + 40) // 16 + 1
    slots = torch.randperm(blocks * 16, generator=g, device="cuda")[:t].contiguous()
    if t > 5:
        pos[3] = 700  # past the table
        slots[4] = -1  # outside the cache
        slots[5] = blocks * 16
    ang = torch.arange(512, device="cuda", dtype=torch.float32)[:, None] * torch.rand(d // 2, generator=g,
                                                                                      device="cuda")[None]
    ang = torch.cat([ang, ang], -1)
    cos, sin = ang.cos().contiguous(), ang.sin().contiguous()
    kc0 = torch.randn(blocks, 16, kv, d, generator=g, device="cuda").to(dtype)
    vc0 = torch.randn(blocks, 16, kv, d, generator=g, device="cuda").to(dtype)

    want_qkv = rope_(qkv.clone(), heads + kv, d, pos, cos, sin)
    want_k, want_v = kc0.clone(), vc0.clone()
    hd, kvd = heads * d, kv * d
    cache_ops.write_kv(want_qkv[:, hd:hd + kvd].view(t, kv, d), want_qkv[:, hd + kvd:width].view(t, kv, d),
                       want_k, want_v, slots)

    got_qkv, got_k, got_v = qkv.clone(), kc0.clone(), vc0.clone()
    cache_ops.rope_write_kv(got_qkv, heads, kv, d, pos, cos, sin, got_k, got_v, slots)
    torch.cuda.synchronize()
    assert torch.equal(got_qkv, want_qkv)
    assert torch.equal(got_k, want_k) and torch.equal(got_v, want_v)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_silu_mul_kernel(dtype):
    announce(f"silu_mul {dtype}")
    g = torch.Generator(device="cuda").manual_seed(1)
    x = (torch.randn(19, 2 * 1376, generator=g, device="cuda") * 3).to(dtype)
    got = silu_mul(x)
    gate, up = x.split(1376, -1)
    want = F.silu(gate) * up
    ulp = 2.0 ** -10 if dtype == torch.float16 else 2.0 ** -7
    assert torch.all((got.float() - want.float()).abs() <= 2 * ulp * want.float().abs() + 1e-6)


@pytest.mark.parametrize("vocab,stride", [(50000, 50000), (50001, 50004), (32003, 32003), (128256, 128256)])
def test_greedy_step_kernel(vocab, stride):
    """argmax with ties (first index), recording, and the state advance of
    real rows; padding rows only take the token. Rows with 16-byte aligned
    starts take the vector path (with a scalar tail when vocab % 4 != 0),
    others the scalar path."""
    announce(f"greedy step vocab={vocab} stride={stride}")
    g = torch.Generator(device="cuda").manual_seed(2)
    b = 6
    logits = torch.randn(b, stride, generator=g, device="cuda")[:, :vocab]
    logits[2, 100] = logits[2, 40000 % vocab] = 50.0  # a tie: first index wins
    logits[3, vocab - 1] = 60.0  # the maximum in the last (tail) element
    ids = torch.zeros(b, dtype=torch.int64, device="cuda")
    pos = torch.tensor([15, 0, 31, 7, 200, 0], dtype=torch.int64, device="cuda")
    ctx = (pos + 1).int()
    slots = torch.zeros(b, dtype=torch.int64, device="cuda")
    tables = torch.arange(b * 8, dtype=torch.int32, device="cuda").view(b, 8) + 1000
    active = torch.tensor([1, 1, 1, 1, 1, 0], dtype=torch.int32, device="cuda")
    ctx_start = ctx.clone()
    tokens = torch.full((b, 4), -1, dtype=torch.int64, device="cuda")
    greedy_step(logits, ids, pos, ctx, slots, tables, 16, active, ctx_start, tokens, 9999)
    want = logits.argmax(-1)
    assert want[2].item() == 100 and want[3].item() == vocab - 1 and torch.equal(ids, want)
    assert torch.equal(tokens[:5, 0], want[:5]) and tokens[5, 0].item() == -1
    assert pos.tolist() == [16, 1, 32, 8, 201, 0] and ctx.tolist() == [17, 2, 33, 9, 202, 1]
    t = tables.cpu()
    want_slots = [int(t[r, p // 16]) * 16 + p % 16 for r, p in enumerate([16, 1, 32, 8])] + [9999, 0]
    assert slots.tolist() == want_slots  # row 4: position 201 is past the 8-block table (128 tokens)
