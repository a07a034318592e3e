"""The streamed reference forward (`model.streamed_reference_forward`, the product's
counterpart of `scripts/shape14.py:124-166, 363-419`) equals the reference layer's own
forward, and the oracle, where both can run (CPU).

Mirrors the reference's `tests/test_streamed_reference.py:39-76` (chunked == naive)."""
from __future__ import annotations

import pytest
import torch

from oracle import reference as R
from techjam2026_amd import harness
from techjam2026_amd.model import TransformerConfig, reference_forward, streamed_reference_forward
from techjam2026_amd.numerics import check

from conftest import make_model, params_of


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("chunk", [7, 16, 64])
def test_streamed_equals_naive_on_ragged_chunks(causal, chunk):
    cfg = TransformerConfig(3, 45, 32, 4, 48, 2, causal)
    model = make_model(cfg)
    x, m = harness.generate_random_case(cfg, "cpu", torch.float32, 5, 0.5)
    m[1, 3] = False                     # a hole: not a prefix mask
    x = x.masked_fill(~m[..., None], 0.0)
    with torch.inference_mode():
        naive = reference_forward(model, x, m)
        streamed = streamed_reference_forward(model, x, m, chunk=chunk)
        oracle = R.stack_forward(params_of(model), x, m, cfg.num_heads, cfg.causal)
    assert torch.allclose(streamed, naive, atol=1e-5, rtol=1e-5)
    assert check(oracle, streamed).envelope_utilization < 0.01
    assert torch.count_nonzero(streamed[~m]) == 0


def test_streamed_without_mask():
    cfg = TransformerConfig(2, 33, 32, 2, 32, 1, True)
    model = make_model(cfg)
    x = torch.randn(2, 33, 32)
    with torch.inference_mode():
        assert torch.allclose(streamed_reference_forward(model, x, None, chunk=8),
                              reference_forward(model, x, None), atol=1e-5, rtol=1e-5)
