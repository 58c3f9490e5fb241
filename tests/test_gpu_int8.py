"""GPU: INT8 weight-only matmul against the oracle.

The bar is nimbus's own (tests/test_quant.py:57-67): within atol 2e-2,
rtol 1e-2 of fp32(x @ w_q^T) * scale rounded to the element type, on its
matrix of M in {1, 7, 64, 300} and TinyLlama's projection shapes, in fp16.
Added: bf16 and Llama-3-8B shapes, an exact check on small integers (pins
the int8 -> fp16/bf16 widening bit for bit), shapes whose N and K leave
partial tiles and steps, shapes and layouts only the general kernel takes
(any N and K, as the Triton kernel's masked tiles), strided activations,
and repeatability. Every
product check runs on both weight layouts: row-major w_q (int8_matmul) and
the tile order Int8Linear packs (int8_matmul_packed).
"""

from __future__ import annotations

import pytest
import torch

from nimbus_amd import _lib
from nimbus_amd.kernels.int8_matmul import (int8_matmul, int8_matmul_packed, int8_matmul_workspace_bytes,
                                            pack_int8_weight, unpack_int8_weight)
from nimbus_amd.quant import Int8Linear, quantize_weight
from oracle import closed_form, reference
from tests.gpu_helpers import announce

pytestmark = pytest.mark.gpu


def _mm(x, q, s, packed):
    if packed:
        return int8_matmul_packed(x, pack_int8_weight(q), s, q.shape[0], q.shape[1])
    return int8_matmul(x, q, s)


def _case(m, n, k, dtype, seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    w = (torch.randn(n, k, generator=g, device="cuda") * 0.02).to(dtype)
    q, s = quantize_weight(w)
    x = torch.randn(m, k, generator=g, device="cuda").to(dtype)
    return x, q, s


@pytest.mark.parametrize("packed", [False, True])
@pytest.mark.parametrize("m", [1, 7, 64, 300])
@pytest.mark.parametrize("n,k", [(3072, 2048), (2048, 5632), (11264, 2048)])
def test_reference_matrix_fp16(m, n, k, packed):
    announce(f"int8_matmul fp16 m={m} n={n} k={k} packed={packed} ws={int8_matmul_workspace_bytes(m, n, k)}")
    x, q, s = _case(m, n, k, torch.float16, m * 7 + n + k)
    got = _mm(x, q, s, packed)
    want = reference.int8_matmul(x.cpu(), q.cpu(), s.cpu())
    torch.cuda.synchronize()
    torch.testing.assert_close(got.cpu(), want, atol=2e-2, rtol=1e-2)


@pytest.mark.parametrize("packed", [False, True])
@pytest.mark.parametrize("m", [1, 16, 64, 130])
@pytest.mark.parametrize("n,k", [(6144, 4096), (4096, 14336), (28672, 4096)])
def test_llama3_shapes_bf16(m, n, k, packed):
    announce(f"int8_matmul bf16 m={m} n={n} k={k} packed={packed}")
    x, q, s = _case(m, n, k, torch.bfloat16, m + n + k)
    got = _mm(x, q, s, packed)
    want = reference.int8_matmul(x.cpu(), q.cpu(), s.cpu())
    torch.cuda.synchronize()
    torch.testing.assert_close(got.cpu(), want, atol=2e-2, rtol=1e-2)


@pytest.mark.parametrize("packed", [False, True])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("m,n,k", [(5, 260, 96), (33, 4100, 1040), (64, 128, 8192), (1, 4, 16), (130, 36, 4104)])
def test_small_integers_are_exact(dtype, m, n, k, packed):
    """Integer x and w_q with power-of-two scales: every product and partial
    sum is exact in fp32, so the kernel must equal the float64 product
    rounded once, whatever the tiling or K split."""
    announce(f"int8_matmul exact {dtype} m={m} n={n} k={k} packed={packed}")
    g = torch.Generator(device="cuda").manual_seed(m * n + k)
    x = torch.randint(-3, 4, (m, k), generator=g, device="cuda").to(dtype)
    q = torch.randint(-127, 128, (n, k), generator=g, device="cuda").to(torch.int8)
    s = (2.0 ** -torch.randint(6, 10, (n,), generator=g, device="cuda").float()).to(dtype)
    got = _mm(x, q, s, packed)
    want = torch.from_numpy(closed_form.int8_matmul(x.cpu(), q.cpu(), s.cpu())).to(dtype)
    torch.cuda.synchronize()
    assert torch.equal(got.cpu(), want)


def test_strided_rows_leading_dims_and_repeatability():
    """x as a column slice of a wider [B, T, 3K] buffer; the same call twice
    gives the same bits (fixed summation order)."""
    announce("int8_matmul strided x, repeat")
    g = torch.Generator(device="cuda").manual_seed(4)
    wide = torch.randn(3, 5, 3 * 2048, generator=g, device="cuda").half()
    x = wide[..., 2048:4096]
    w = (torch.randn(3072, 2048, generator=g, device="cuda") * 0.02).half()
    q, s = quantize_weight(w)
    a = int8_matmul(x, q, s)
    b = int8_matmul(x, q, s)
    want = reference.int8_matmul(x.reshape(-1, 2048).cpu(), q.cpu(), s.cpu()).view(3, 5, 3072)
    torch.cuda.synchronize()
    assert a.shape == (3, 5, 3072)
    assert torch.equal(a, b)
    torch.testing.assert_close(a.cpu(), want, atol=2e-2, rtol=1e-2)


@pytest.mark.parametrize("packed", [False, True])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("m,n,k", [(7, 4098, 2040), (3, 37, 4099), (1, 6, 13), (5, 130, 2056)])
def test_any_shape_runs_like_the_masked_triton_tiles(dtype, m, n, k, packed):
    """The reference's Triton kernel masks its tiles, so it takes any N and
    K; shapes the tiled kernels do not take (N not a multiple of 4, K not of
    16 row-major / 8 packed) run the general kernel, to the same bar, with
    the same bits on a repeat."""
    announce(f"int8_matmul any shape {dtype} m={m} n={n} k={k} packed={packed}")
    x, q, s = _case(m, n, k, dtype, m + 3 * n + k)
    got = _mm(x, q, s, packed)
    again = _mm(x, q, s, packed)
    want = reference.int8_matmul(x.cpu(), q.cpu(), s.cpu())
    torch.cuda.synchronize()
    assert torch.equal(got, again)
    torch.testing.assert_close(got.cpu(), want, atol=2e-2, rtol=1e-2)


@pytest.mark.parametrize("packed", [False, True])
def test_unaligned_activations_take_the_general_kernel(packed):
    """Through the C ABI (the Python wrappers copy such an x first): x one
    element into its buffer (2-byte aligned, not 16) with an odd row stride
    and y likewise, so the tiled kernels' alignment does not hold and the
    general kernel runs; against the oracle and the aligned call."""
    announce(f"int8_matmul unaligned x, y through the C ABI packed={packed}")
    g = torch.Generator(device="cuda").manual_seed(9)
    m, n, k = 9, 512, 1024
    wide = torch.randn(m, k + 3, generator=g, device="cuda").half()
    x = wide[:, 1:1 + k]
    ybuf = torch.zeros(m, n + 3, dtype=torch.float16, device="cuda")
    y = ybuf[:, 1:1 + n]
    assert x.data_ptr() % 16 != 0 and x.stride(0) % 8 != 0 and y.data_ptr() % 16 != 0
    w = (torch.randn(n, k, generator=g, device="cuda") * 0.02).half()
    q, s = quantize_weight(w)
    lib = _lib.load()
    stream = torch.cuda.current_stream().cuda_stream
    if packed:
        wp = pack_int8_weight(q)
        rc = lib.nimbus_int8_matmul_packed(x.data_ptr(), x.stride(0), wp.data_ptr(), s.data_ptr(), y.data_ptr(),
                                           y.stride(0), m, n, k, None, 0, _lib.dtype_code(x.dtype), stream)
    else:
        rc = lib.nimbus_int8_matmul(x.data_ptr(), x.stride(0), q.data_ptr(), q.stride(0), s.data_ptr(), y.data_ptr(),
                                    y.stride(0), m, n, k, None, 0, _lib.dtype_code(x.dtype), stream)
    assert rc == 0
    want = reference.int8_matmul(x.cpu(), q.cpu(), s.cpu())
    aligned = _mm(x.contiguous(), q, s, packed)
    torch.cuda.synchronize()
    torch.testing.assert_close(y.cpu(), want, atol=2e-2, rtol=1e-2)
    torch.testing.assert_close(y, aligned, atol=2e-3, rtol=2e-3)
    assert torch.all(ybuf[:, 0] == 0) and torch.all(ybuf[:, n + 1:] == 0)  # nothing outside y written


def test_int8_linear_matches_dequantized_linear():
    """Int8Linear (nimbus/quant/int8.py:32-47) against F.linear with the
    dequantized weight, the reference module's own definition."""
    announce("Int8Linear")
    torch.manual_seed(1)
    lin = torch.nn.Linear(2048, 512, bias=False).cuda().half()
    mod = Int8Linear(lin)
    x = torch.randn(4, 7, 2048, device="cuda").half()
    got = mod(x)
    want = reference.int8_matmul(x.reshape(-1, 2048).cpu(), mod.weight_q.cpu(), mod.scale.cpu()).view(4, 7, 512)
    torch.cuda.synchronize()
    torch.testing.assert_close(got.cpu(), want, atol=2e-2, rtol=1e-2)
    assert mod.weight_q.dtype == torch.int8 and mod.weight_q.shape == (512, 2048)
    # features that leave partial tiles and an odd K (the general kernel)
    lin = torch.nn.Linear(1027, 301, bias=False).cuda().half()
    mod = Int8Linear(lin)
    x = torch.randn(3, 1027, device="cuda").half()
    got = mod(x)
    want = reference.int8_matmul(x.cpu(), mod.weight_q.cpu(), mod.scale.cpu())
    torch.cuda.synchronize()
    torch.testing.assert_close(got.cpu(), want, atol=2e-2, rtol=1e-2)


def test_zero_rows_and_explicit_workspace():
    announce("int8_matmul m=0, caller workspace")
    x, q, s = _case(16, 3072, 2048, torch.float16, 2)
    assert int8_matmul(x[:0], q, s).shape == (0, 3072)
    need = int8_matmul_workspace_bytes(16, 3072, 2048)
    assert need > 0  # 24 channel tiles: K is split
    ws = torch.empty(need, dtype=torch.uint8, device="cuda")
    out = torch.empty(16, 3072, dtype=torch.float16, device="cuda")
    int8_matmul(x, q, s, out=out, workspace=ws)
    torch.cuda.synchronize()
    assert torch.equal(out, int8_matmul(x, q, s))
    with pytest.raises(ValueError):
        int8_matmul(x, q, s, workspace=ws[:need - 16])


@pytest.mark.parametrize("n,k", [(16, 64), (260, 1040), (3072, 2048), (5, 24)])
def test_pack_unpack_roundtrip_and_layout(n, k):
    """The tile order of nimbus_int8_matmul_packed: block (nb, kc), lane l's
    16 bytes = row 16 nb + l % 16, columns 64 kc + 16 (l / 16) .. +16, zero
    padded; unpacking gives w_q back."""
    announce(f"pack n={n} k={k}")
    g = torch.Generator(device="cuda").manual_seed(n + k)
    q = torch.randint(-127, 128, (n, k), generator=g, device="cuda").to(torch.int8)
    p = pack_int8_weight(q)
    assert p.shape == (-(-n // 16), -(-k // 64), 1024)
    assert torch.equal(unpack_int8_weight(p, n, k), q)
    qc, pc = q.cpu(), p.cpu()
    nb, kc, lane, e = p.shape[0] - 1, p.shape[1] - 1, 37, 5
    row, colk = 16 * nb + lane % 16, 64 * kc + 16 * (lane // 16) + e
    want = int(qc[row, colk]) if row < n and colk < k else 0
    assert int(pc[nb, kc, 16 * lane + e]) == want


@pytest.mark.parametrize("m,n,k", [(33, 4100, 1040), (64, 4096, 4096), (7, 6144, 4096), (1, 260, 8192),
                                   (200, 2080, 1040)])
def test_every_launch_plan_is_exact(m, n, k):
    """Each plan the tuner may pick (token tile, k slices, K splits, row
    blocks per wave) gives
    the float64 product rounded once on integer inputs, so tuning can only
    change speed."""
    from nimbus_amd import _lib
    from nimbus_amd.kernels import int8_matmul as mod

    announce(f"int8 plans m={m} n={n} k={k}")
    g = torch.Generator(device="cuda").manual_seed(m + n)
    x = torch.randint(-3, 4, (m, k), generator=g, device="cuda").to(torch.bfloat16)
    q = torch.randint(-127, 128, (n, k), generator=g, device="cuda").to(torch.int8)
    s = (2.0 ** -torch.randint(6, 10, (n,), generator=g, device="cuda").float()).to(torch.bfloat16)
    want = torch.from_numpy(closed_form.int8_matmul(x.cpu(), q.cpu(), s.cpu())).to(torch.bfloat16)
    p = pack_int8_weight(q)
    lib = _lib.load()
    plans = mod._candidate_plans(m, n, k)
    assert plans
    # one workspace for every plan, each run twice into an output poisoned with NaN
    need = max(lib.nimbus_int8_matmul_packed_plan_workspace_bytes(m, n, k, *plan) for plan in plans)
    ws = torch.empty(max(need, 256), dtype=torch.uint8, device="cuda")
    for plan in plans:
        for rep in range(2):
            y = torch.full((m, n), float("nan"), dtype=torch.bfloat16, device="cuda")
            rc = lib.nimbus_int8_matmul_packed_plan(x.data_ptr(), k, p.data_ptr(), s.data_ptr(), y.data_ptr(), n, m, n,
                                                    k, *plan, ws.data_ptr(), ws.numel(), 1, None)
            assert rc == 0, plan
            torch.cuda.synchronize()
            assert torch.equal(y.cpu(), want), (plan, rep)


def test_split_plan_replays_in_a_graph():
    """A plan that splits K (its kernel and the reducing launch), captured in
    a hipGraph and replayed several times with eager calls on the same
    workspace in between: every replay and every eager call gives the exact
    product."""
    from nimbus_amd import _lib

    announce("int8 split plan in a graph")
    m, n, k = 64, 4096, 4096
    plan = (64, 2, 4, 1)
    g = torch.Generator(device="cuda").manual_seed(9)
    x = torch.randint(-3, 4, (m, k), generator=g, device="cuda").to(torch.bfloat16)
    q = torch.randint(-127, 128, (n, k), generator=g, device="cuda").to(torch.int8)
    s = (2.0 ** -torch.randint(6, 10, (n,), generator=g, device="cuda").float()).to(torch.bfloat16)
    want = torch.from_numpy(closed_form.int8_matmul(x.cpu(), q.cpu(), s.cpu())).to(torch.bfloat16).cuda()
    p = pack_int8_weight(q)
    lib = _lib.load()
    need = lib.nimbus_int8_matmul_packed_plan_workspace_bytes(m, n, k, *plan)
    assert need > 0
    ws = torch.empty(need, dtype=torch.uint8, device="cuda")
    y = torch.full((m, n), float("nan"), dtype=torch.bfloat16, device="cuda")

    def call():
        rc = lib.nimbus_int8_matmul_packed_plan(x.data_ptr(), k, p.data_ptr(), s.data_ptr(), y.data_ptr(), n, m, n, k,
                                                *plan, ws.data_ptr(), ws.numel(), 1,
                                                torch.cuda.current_stream().cuda_stream)
        assert rc == 0

    call()
    torch.cuda.synchronize()
    assert torch.equal(y, want)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        call()
    for rep in range(4):
        y.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, want), rep
        y.fill_(float("nan"))
        call()
        torch.cuda.synchronize()
        assert torch.equal(y, want), rep


@pytest.mark.parametrize("dtype,n,k", [(torch.float16, 11264, 2048), (torch.bfloat16, 28672, 4096),
                                       (torch.bfloat16, 96, 200), (torch.float16, 160, 64)])
@pytest.mark.parametrize("m", [1, 7, 64, 300])
def test_packed_silu_equals_projection_then_gate(dtype, n, k, m):
    """The gate_up projection fused with the SiLU gate gives, bit for bit,
    silu_mul of the projection's output under the same launch plan, for
    every plan it takes (and its default): TinyLlama's and Llama-3-8B's
    gate_up shapes, and small ones whose gate half leaves a workgroup's last
    row-block groups empty (n = 96: 3 gate blocks; n = 160: 5)."""
    from nimbus_amd.kernels.elementwise import silu_mul
    from nimbus_amd.kernels.int8_matmul import _silu_plans, int8_matmul_packed_silu

    announce(f"int8 packed silu m={m} n={n} k={k} {dtype}")
    x, q, s = _case(m, n, k, dtype, seed=m + n)
    p = pack_int8_weight(q)
    lib = _lib.load()
    stream = torch.cuda.current_stream().cuda_stream
    dt = _lib.dtype_code(dtype)
    for plan in _silu_plans(m, n, k) + [(0, 1, 1)]:
        fused = torch.full((m, n // 2), 7.0, dtype=dtype, device="cuda")
        rc = lib.nimbus_int8_matmul_packed_silu(x.data_ptr(), k, p.data_ptr(), s.data_ptr(), fused.data_ptr(),
                                                n // 2, m, n, k, *plan, dt, stream)
        assert rc == 0, plan
        bm, ks, rw = plan if plan[0] else ((16 if m <= 16 else 32 if m <= 32 else 64), 1, 1)
        y = torch.empty(m, n, dtype=dtype, device="cuda")
        rc = lib.nimbus_int8_matmul_packed_plan(x.data_ptr(), k, p.data_ptr(), s.data_ptr(), y.data_ptr(), n, m, n,
                                                k, bm, ks, 1, rw, None, 0, dt, stream)
        assert rc == 0, plan
        want = silu_mul(y)
        assert torch.equal(fused, want), (plan, (fused.float() - want.float()).abs().max().item())
    # the wrapper (tuned plan) and the INT8 layer's fused path agree with the two steps within rounding
    got = int8_matmul_packed_silu(x, p, s, n, k)
    two = silu_mul(int8_matmul_packed(x, p, s, n, k))
    assert torch.allclose(got.float(), two.float(), atol=2e-2, rtol=1e-2)


@pytest.mark.parametrize("seed", range(6))
def test_random_shapes_are_exact_on_small_integers(seed):
    """Seeded random shapes (1-700 tokens; any N and K, and multiples of 32
    and 64) on small-integer activations, where every fp32 sum is exact: the
    row-major kernel, the packed kernel under its tuned plan and, for N a
    multiple of 32, the fused gate_up + SiLU all give the reference formula's
    bits (the fused one silu_mul's of the exact projection)."""
    import numpy as np

    from nimbus_amd.kernels.elementwise import silu_mul
    from nimbus_amd.kernels.int8_matmul import int8_matmul_packed_silu

    rng = np.random.default_rng(4000 + seed)
    dtype = [torch.float16, torch.bfloat16][seed % 2]
    m = int(np.exp(rng.uniform(0, np.log(700))))
    n = int(rng.choice([int(rng.integers(1, 9000)), 32 * int(rng.integers(1, 300))]))
    k = int(rng.choice([int(rng.integers(1, 6000)), 64 * int(rng.integers(1, 90))]))
    announce(f"int8 random shape seed={seed} m={m} n={n} k={k} {dtype}")
    g = torch.Generator().manual_seed(seed)
    x = torch.randint(-4, 5, (m, k), generator=g).to(dtype)
    wq = torch.randint(-127, 128, (n, k), generator=g).to(torch.int8)
    sc = (torch.rand(n, generator=g) * 0.01 + 1e-4).to(dtype)
    want = reference.int8_matmul(x, wq, sc)
    xd, wd, sd = x.cuda(), wq.cuda(), sc.cuda()
    assert torch.equal(int8_matmul(xd, wd, sd).cpu(), want)
    if k % 8 == 0:
        packed = pack_int8_weight(wd)
        assert torch.equal(int8_matmul_packed(xd, packed, sd, n, k).cpu(), want)
        if n % 32 == 0:
            fused = int8_matmul_packed_silu(xd, packed, sd, n, k)
            assert torch.equal(fused.cpu(), silu_mul(want.cuda()).cpu())
