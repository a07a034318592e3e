"""Pinning the oracle before it is trusted (CPU only).

The reference ships no golden tensors (its tests compute references on the fly from
PyTorch composites), so `oracle.reference` is pinned by checks that a plausible mistake
fails:

* brute force: `oracle.brute` (pure-Python loops, math.erf/exp/sqrt, float64) agrees with
  `stack_forward` in fp64 to 1e-10 on tiny shapes, causal and not, padded and not;
* textbook routines: `layer_norm` == `F.layer_norm`, `gelu_erf` == `F.gelu(approximate=
  "none")`, `attention_core` == `F.scaled_dot_product_attention` with the combined mask;
* closed forms: LN of an all-zero row is beta; S = 1 makes attention the identity on V;
  padded rows of the stack output are exactly zero; LN is invariant to scaling its input;
* structure: query-chunked attention equals naive attention on ragged chunk sizes
  (333, 4097-style tails), per-element and in the full stack;
* planted mistakes: a stack variant with the final mask moved before the final norm, or
  the GELU swapped for the tanh approximation, or the causal diagonal excluded, is
  detected by these checks (so they are not tautologies).
"""
from __future__ import annotations

import math

import pytest
import torch
import torch.nn.functional as F

from oracle import brute
from oracle import reference as R
from techjam2026_amd import harness
from techjam2026_amd.model import BaselineTransformer, TransformerConfig

from conftest import make_model, params_of


def _tiny(cfg, seed=3, random_norms=True):
    model = make_model(cfg, seed=seed, random_norms=random_norms)
    return params_of(model)


def _to_lists(p):
    return {k: v.double().tolist() for k, v in p.items()}


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("pad", [0.0, 0.5])
def test_reference_matches_brute_force(causal, pad):
    cfg = TransformerConfig(2, 6, 8, 2, 12, 2, causal)
    p = _tiny(cfg)
    x, m = harness.generate_random_case(cfg, "cpu", torch.float32, 11, pad)
    want = torch.tensor(brute.forward(_to_lists(p), x.double().tolist(), m.tolist(), 2, causal),
                        dtype=torch.float64)
    got = R.stack_forward(p, x, m, 2, causal, dtype=torch.float64)
    assert (got - want).abs().max().item() < 1e-10


def test_layer_norm_and_gelu_are_the_library_routines():
    torch.manual_seed(0)
    x = torch.randn(37, 96, dtype=torch.float64)
    w, b = torch.randn(96, dtype=torch.float64), torch.randn(96, dtype=torch.float64)
    assert torch.allclose(R.layer_norm(x, w, b), F.layer_norm(x, (96,), w, b, 1e-5),
                          atol=1e-13, rtol=0)
    assert torch.allclose(R.gelu_erf(x), F.gelu(x, approximate="none"), atol=1e-14, rtol=0)
    # and not the tanh approximation (a plausible mistake)
    assert (R.gelu_erf(x) - F.gelu(x, approximate="tanh")).abs().max() > 1e-5
    for v in (-3.0, -0.5, 0.0, 0.7, 2.5):
        assert abs(R.gelu_erf(torch.tensor(v, dtype=torch.float64)).item()
                   - 0.5 * v * (1 + math.erf(v / math.sqrt(2)))) < 1e-15


def test_layer_norm_of_zero_row_is_beta_and_scale_invariant():
    w, b = torch.randn(64, dtype=torch.float64), torch.randn(64, dtype=torch.float64)
    z = torch.zeros(3, 64, dtype=torch.float64)
    assert torch.equal(R.layer_norm(z, w, b), b.expand(3, 64))
    x = torch.randn(5, 64, dtype=torch.float64)
    assert torch.allclose(R.layer_norm(64 * x, w, b, eps=0.0), R.layer_norm(x, w, b, eps=0.0),
                          atol=1e-12)


@pytest.mark.parametrize("causal", [False, True])
def test_attention_core_matches_sdpa_with_combined_mask(causal):
    torch.manual_seed(1)
    B, H, S, Dh = 2, 3, 19, 8
    q, k, v = (torch.randn(B, H, S, Dh, dtype=torch.float64) for _ in range(3))
    keep = torch.rand(B, S) > 0.3
    keep[:, 0] = True
    allowed = keep[:, None, None, :].expand(B, 1, S, S)
    if causal:
        allowed = allowed & torch.ones(S, S, dtype=torch.bool).tril()
    want = F.scaled_dot_product_attention(q, k, v, attn_mask=allowed)
    got = R.attention_core(q, k, v, keep, causal)
    assert (got - want).abs().max().item() < 1e-12


def test_single_token_attention_is_identity_on_v():
    torch.manual_seed(2)
    q, k, v = (torch.randn(4, 2, 1, 16, dtype=torch.float64) for _ in range(3))
    assert torch.equal(R.attention_core(q, k, v, None, True), v)


@pytest.mark.parametrize("S,chunk", [(333, 128), (97, 32), (65, 64), (64, 64), (130, 1000)])
@pytest.mark.parametrize("causal", [False, True])
def test_chunked_attention_equals_naive(S, chunk, causal):
    torch.manual_seed(S)
    q, k, v = (torch.randn(2, 2, S, 16, dtype=torch.float64) for _ in range(3))
    keep = torch.arange(S)[None, :] < torch.tensor([S, S // 2 + 1])[:, None]
    naive = R.attention_core(q, k, v, keep, causal)
    chunked = R.attention_core(q, k, v, keep, causal, chunk=chunk)
    assert (naive - chunked).abs().max().item() < 1e-12


def test_stack_rows_and_chunking_match_whole_forward():
    cfg = TransformerConfig(3, 70, 32, 4, 48, 2, True)
    p = _tiny(cfg)
    x, m = harness.generate_random_case(cfg, "cpu", torch.float32, 5, 0.5)
    whole = R.stack_forward(p, x, m, 4, True, dtype=torch.float64)
    rows = R.stack_forward_rows(p, x, m, 4, True, chunk=16, dtype=torch.float64)
    assert (whole - rows).abs().max().item() < 1e-12
    assert torch.count_nonzero(whole[~m]) == 0


def test_package_baseline_forward_equals_oracle():
    """The drop-in's fallback forward (the reference layer) agrees with the oracle."""
    cfg = TransformerConfig(2, 40, 64, 4, 96, 3, True)
    model = make_model(cfg, random_norms=True)
    x, m = harness.generate_random_case(cfg, "cpu", torch.float32, 9, 0.4)
    with torch.inference_mode():
        got = model(x, m).double()
    want = R.stack_forward(params_of(model), x, m, 4, True, dtype=torch.float64)
    assert (got - want).abs().max().item() < 1e-4


# ------------------------------------------------------------- planted mistakes
def _final_mask_first(p, x, m, H, causal):
    for i in range(R.num_layers_of(p)):
        x = R.block_forward(p, i, x, m, causal, H)
    x = x.masked_fill(~m[..., None], 0)
    return R.layer_norm(x, p["final_norm.weight"], p["final_norm.bias"])


def test_planted_mistakes_are_caught():
    cfg = TransformerConfig(2, 6, 8, 2, 12, 2, True)
    p = _tiny(cfg)
    x, m = harness.generate_random_case(cfg, "cpu", torch.float32, 11, 0.5)
    p64 = {k: v.double() for k, v in p.items()}
    want = torch.tensor(brute.forward(_to_lists(p), x.double().tolist(), m.tolist(), 2, True),
                        dtype=torch.float64)
    # mask before the final norm -> padded rows hold beta, not zero
    bad = _final_mask_first(p64, x.double(), m, 2, True)
    assert (bad - want).abs().max().item() > 1e-3
    # non-causal attention where causal was asked
    bad2 = R.stack_forward(p, x, m, 2, False, dtype=torch.float64)
    assert (bad2 - want).abs().max().item() > 1e-3
    # ignoring the key-padding mask (visible without causality: under a causal prefix
    # mask a valid query never sees a padded key, so the key mask cannot change it)
    want_nc = torch.tensor(brute.forward(_to_lists(p), x.double().tolist(), m.tolist(), 2, False),
                           dtype=torch.float64)
    bad3 = R.stack_forward(p, x, None, 2, False, dtype=torch.float64) * m[..., None]
    assert (bad3 - want_nc).abs().max().item() > 1e-3
    assert (R.stack_forward(p, x, m, 2, False, dtype=torch.float64) - want_nc).abs().max() < 1e-10


def test_generator_semantics():
    """`torch_transformer_benchmark.py:234-272`: lengths in [round(S(1-p)), S], mask a
    prefix, padded rows of x zero, deterministic per seed, x ~ N(0, 1) * scale."""
    cfg = TransformerConfig(64, 128, 16, 2, 16, 1, True)
    x, m = harness.generate_random_case(cfg, "cpu", torch.float32, 1234, 0.75, 2.0)
    lens = m.sum(1)
    assert lens.min().item() >= round(128 * 0.25) and lens.max().item() <= 128
    assert torch.equal(m, torch.arange(128)[None, :] < lens[:, None])
    assert torch.count_nonzero(x[~m]) == 0
    x2, m2 = harness.generate_random_case(cfg, "cpu", torch.float32, 1234, 0.75, 2.0)
    assert torch.equal(x, x2) and torch.equal(m, m2)
    g = torch.Generator().manual_seed(1234)
    assert torch.equal(x[m], (torch.randn(64, 128, 16, generator=g) * 2.0)[m])
    x0, m0 = harness.generate_random_case(cfg, "cpu", torch.float32, 1, 0.0)
    assert bool(m0.all())


def test_xavier_init_bounds_and_determinism():
    cfg = TransformerConfig(1, 4, 64, 4, 256, 2, False)
    a, b = make_model(cfg, seed=3), make_model(cfg, seed=3)
    for (n1, t1), (n2, t2) in zip(a.state_dict().items(), b.state_dict().items()):
        assert torch.equal(t1, t2)
    w = a.layers[0].ffn_in.weight
    bound = math.sqrt(6.0 / (w.shape[0] + w.shape[1]))
    assert w.abs().max().item() <= bound and w.abs().max().item() > 0.9 * bound
    assert torch.equal(a.layers[0].norm1.weight, torch.ones(64))
