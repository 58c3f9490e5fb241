"""GPU: the HIP slot write is bit-exact against the oracle's index_copy_."""

from __future__ import annotations

import pytest
import torch

from nimbus_amd.kernels.cache_ops import write_kv
from oracle import reference
from tests import golden_io
from tests.gpu_helpers import announce

pytestmark = pytest.mark.gpu


def _bits(t):
    return t.view(torch.int16)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("kv,d", [(4, 64), (8, 128)])
@pytest.mark.parametrize("tokens", [1, 301, 2108])
def test_write_kv_bit_exact_from_fused_qkv_views(dtype, kv, d, tokens):
    announce(f"write_kv dtype={dtype} kv={kv} d={d} T={tokens}")
    heads, nb = 32, 256
    g = torch.Generator(device="cuda").manual_seed(tokens)
    qkv = torch.randn(tokens, (heads + 2 * kv) * d, generator=g, device="cuda").to(dtype)
    k = qkv[:, heads * d:(heads + kv) * d].view(tokens, kv, d)  # strided, as Attention.forward produces it
    v = qkv[:, (heads + kv) * d:].view(tokens, kv, d)
    slots = torch.randperm(nb * 16, generator=g, device="cuda")[:tokens].to(torch.int64)
    kc = torch.randn(nb, 16, kv, d, generator=g, device="cuda").to(dtype)
    vc = torch.randn(nb, 16, kv, d, generator=g, device="cuda").to(dtype)
    want_k, want_v = kc.cpu(), vc.cpu()
    reference.write_kv(k.cpu(), v.cpu(), want_k, want_v, slots.cpu())
    write_kv(k, v, kc, vc, slots)
    torch.cuda.synchronize()
    assert torch.equal(_bits(kc.cpu()), _bits(want_k))
    assert torch.equal(_bits(vc.cpu()), _bits(want_v))


def test_write_kv_unaligned_rows_use_scalar_path():
    announce("write_kv unaligned")
    t, kv, d = 33, 2, 64
    buf = torch.randn(t, kv * d + 3, device="cuda").half()  # row stride not a multiple of 8
    k = buf[:, :kv * d].view(t, kv, d)
    v = buf[:, 3:3 + kv * d].view(t, kv, d)
    kc = torch.zeros(8, 16, kv, d, device="cuda").half()
    vc = torch.zeros_like(kc)
    slots = torch.arange(5, 5 + t, device="cuda")
    want_k, want_v = kc.cpu(), vc.cpu()
    reference.write_kv(k.cpu(), v.cpu(), want_k, want_v, slots.cpu())
    write_kv(k, v, kc, vc, slots)
    assert torch.equal(_bits(kc.cpu()), _bits(want_k)) and torch.equal(_bits(vc.cpu()), _bits(want_v))


def test_write_kv_skips_slots_outside_the_cache():
    announce("write_kv out-of-range slots")
    kv, d, nb = 2, 64, 4
    kc = torch.zeros(nb, 16, kv, d, device="cuda", dtype=torch.bfloat16)
    vc = torch.zeros_like(kc)
    k = torch.ones(3, kv, d, device="cuda", dtype=torch.bfloat16)
    slots = torch.tensor([-1, 7, nb * 16], device="cuda", dtype=torch.int64)
    write_kv(k, k, kc, vc, slots)
    flat = kc.view(-1, kv, d).cpu()
    assert flat[7].eq(1).all()
    assert flat.sum().item() == kv * d


@pytest.mark.parametrize("name", golden_io.names("write_kv"))
def test_write_kv_golden(name):
    announce(f"write_kv golden {name}")
    f = golden_io.load(name, device="cuda")
    kc, vc = f["k_cache"].clone(), f["v_cache"].clone()
    write_kv(f["k"], f["v"], kc, vc, f["slot_mapping"])
    assert torch.equal(_bits(kc.cpu()), _bits(f["k_cache_out"].cpu()))
    assert torch.equal(_bits(vc.cpu()), _bits(f["v_cache_out"].cpu()))


def test_write_kv_empty_batch():
    kc = torch.zeros(2, 16, 2, 64, device="cuda").half()
    e = torch.zeros(0, 2, 64, device="cuda").half()
    write_kv(e, e, kc, kc.clone(), torch.zeros(0, dtype=torch.int64, device="cuda"))
    assert kc.eq(0).all()
