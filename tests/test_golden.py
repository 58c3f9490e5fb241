"""CPU: the oracle and the closed form reproduce the committed fixtures."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import closed_form, reference
from tests import golden_io
from tests.helpers import assert_within


def test_fixtures_present():
    assert len(golden_io.names("decode")) >= 3
    assert len(golden_io.names("prefill")) >= 2
    assert len(golden_io.names("write_kv")) >= 2


@pytest.mark.parametrize("name", golden_io.names("decode"))
def test_decode_fixture(name):
    f = golden_io.load(name)
    ctx = f["context_lens"]
    args = (f["q"], f["k_cache"], f["v_cache"], ctx, f["block_tables"])
    cf = closed_form.decode(*args, f["scale"])
    np.testing.assert_allclose(cf, f["out"].numpy(), rtol=1e-6, atol=1e-6)
    got = reference.paged_decode_attention(*args, int(ctx.max()), f["scale"])
    assert_within(got, f["out"], what=name)


@pytest.mark.parametrize("name", golden_io.names("prefill"))
def test_prefill_fixture(name):
    f = golden_io.load(name)
    qs = f["query_start"].tolist()
    ctx = f["context_lens"].tolist()
    cf = closed_form.prefill(f["q"], f["k_cache"], f["v_cache"], qs, ctx, f["block_tables"], f["scale"])
    np.testing.assert_allclose(cf, f["out"].numpy(), rtol=1e-6, atol=1e-6)
    got = reference.paged_prefill_attention(f["q"], f["k_cache"], f["v_cache"], f["query_start"],
                                            f["context_lens"], f["block_tables"], f["scale"], qs, ctx)
    assert_within(got, f["out"], what=name)


@pytest.mark.parametrize("name", golden_io.names("write_kv"))
def test_write_kv_fixture(name):
    f = golden_io.load(name)
    kc, vc = f["k_cache"].clone(), f["v_cache"].clone()
    reference.write_kv(f["k"], f["v"], kc, vc, f["slot_mapping"])
    np.testing.assert_array_equal(kc.view(torch.int16).numpy(), f["k_cache_out"].view(torch.int16).numpy())
    np.testing.assert_array_equal(vc.view(torch.int16).numpy(), f["v_cache_out"].view(torch.int16).numpy())
