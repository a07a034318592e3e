"""The gfx950 kernels against plain PyTorch references of the same op.

Mirrors the reference's `tests/test_kernels.py`: LayerNorm against `F.layer_norm` over
widths and masks (:23-74), the LN(0) = beta trap, flash attention against an exact
softmax attention over the reference's shape list crossed with causal and padding
(:79-116), the fully masked row (:119-128), strided fused-QKV views (:131-144), and the
causal split loop at ragged lengths (:261-298). Adds the GEMM (which the reference left
to cuBLAS) in every MFMA precision. Tolerances: the organizer's gate (atol 2e-3,
rtol 2e-2, `numerics.check`) unless a tighter, precision-specific bound is stated.
"""
from __future__ import annotations

import math

import pytest
import torch
import torch.nn.functional as F

from techjam2026_amd import _lib as L
from techjam2026_amd import kernels as K
from techjam2026_amd.numerics import check

pytestmark = pytest.mark.gpu
DEV = "cuda"


# --------------------------------------------------------------- layernorm
@pytest.mark.parametrize("d", [64, 256, 512, 768, 1024, 4096, 100])
@pytest.mark.parametrize("out_dtype", [torch.float32, torch.float16])
@pytest.mark.parametrize("mask_out", [False, True])
def test_fused_add_mask_layernorm(d, out_dtype, mask_out):
    torch.manual_seed(0)
    M = 517
    x = torch.randn(M, d, device=DEV)
    y = torch.randn(M, d, device=DEV)
    keep = torch.rand(M, device=DEV) > 0.3
    w = torch.randn(d, device=DEV)
    b = torch.randn(d, device=DEV)
    s, h = K.add_mask_layernorm(x, y, keep, w, b, 1e-5, mask_out=mask_out,
                                out_dtype=out_dtype, residual_dtype=torch.float32)
    ref_s = (x.double() + y.double()) * keep[:, None].double()
    ref_h = F.layer_norm(ref_s, (d,), w.double(), b.double(), 1e-5)
    if mask_out:
        ref_h = ref_h * keep[:, None].double()
    assert torch.equal(s, ((x + y) * keep[:, None].float())), "residual must be exact fp32"
    tol = 2e-5 if out_dtype == torch.float32 else 2e-3
    assert (h.double() - ref_h).abs().max().item() < tol * max(1.0, ref_h.abs().max().item())


@pytest.mark.parametrize("keep_kind", ["bool", "float"])
def test_layernorm_keep_dtypes(keep_kind):
    d, M = 256, 64
    x = torch.randn(M, d, device=DEV)
    keep = torch.rand(M, device=DEV) > 0.5
    k = keep if keep_kind == "bool" else keep.float()
    w, b = torch.randn(d, device=DEV), torch.randn(d, device=DEV)
    s, h = K.add_mask_layernorm(x, None, k, w, b, 1e-5, mask_out=True)
    assert torch.equal(s, x * keep[:, None].float())
    assert torch.count_nonzero(h[~keep]) == 0


def test_layernorm_of_an_all_zero_row_returns_bias():
    """LN(0) == bias, so the final mask must come after the norm (`mask_out`)."""
    d = 256
    x = torch.zeros(8, d, device=DEV)
    w, b = torch.randn(d, device=DEV), torch.randn(d, device=DEV)
    _, h = K.add_mask_layernorm(x, None, None, w, b, 1e-5, mask_out=False)
    assert torch.allclose(h, b.expand_as(h), atol=1e-6)
    keep = torch.zeros(8, device=DEV)
    _, hm = K.add_mask_layernorm(x, None, keep, w, b, 1e-5, mask_out=True)
    assert torch.count_nonzero(hm) == 0


def test_layernorm_without_residual_or_mask():
    d = 512
    x = torch.randn(64, d, device=DEV)
    w, b = torch.randn(d, device=DEV), torch.randn(d, device=DEV)
    s, h = K.add_mask_layernorm(x, None, None, w, b, 1e-5, want_residual=False)
    assert s is None
    assert check(F.layer_norm(x, (d,), w, b, 1e-5), h).passed


def test_layernorm_generic_path_strided_rows():
    d, M = 300, 33                       # d % 4 != 0 -> generic kernel
    base = torch.randn(M, d + 20, device=DEV)
    x = base[:, :d]                      # row stride d + 20
    w, b = torch.randn(d, device=DEV), torch.randn(d, device=DEV)
    _, h = K.add_mask_layernorm(x, None, None, w, b, 1e-5)
    ref = F.layer_norm(x.double(), (d,), w.double(), b.double(), 1e-5)
    assert (h.double() - ref).abs().max().item() < 1e-4


# --------------------------------------------------------------- GEMM
GEMM_TOL = {  # max |err| / (sqrt(K) * max|a| * max|w|): precision-specific bounds
    "float32": 1e-6, "f16x3": 4e-6, "bf16x3": 3e-5, "float16": 1e-3, "bfloat16": 8e-3}


@pytest.mark.parametrize("precision", list(GEMM_TOL))
@pytest.mark.parametrize("M,N,K_", [(256, 768, 256), (517, 192, 64), (1000, 1024, 520),
                                    (64, 4096, 1024), (130, 36, 2048)])
def test_gemm_matches_fp64(precision, M, N, K_):
    torch.manual_seed(1)
    a = torch.randn(M, K_, device=DEV)
    w = torch.randn(N, K_, device=DEV) * 0.05
    bias = torch.randn(N, device=DEV)
    pw = K.PreparedLinear(w, bias, K.MODES[precision])
    c = K.linear(a, pw)
    ref = a.double() @ w.double().t() + bias.double()
    err = (c.double() - ref).abs().max().item()
    scale = K_ ** 0.5 * a.abs().max().item() * w.abs().max().item()
    assert err / scale < GEMM_TOL[precision], f"{precision}: err {err:.3e} scale {scale:.3e}"


@pytest.mark.parametrize("out_dtype", [torch.float32, torch.float16, torch.bfloat16])
def test_gemm_gelu_epilogue_and_cast(out_dtype):
    torch.manual_seed(2)
    M, N, K_ = 300, 512, 256
    a = torch.randn(M, K_, device=DEV)
    w = torch.randn(N, K_, device=DEV) * 0.1
    bias = torch.randn(N, device=DEV)
    pw = K.PreparedLinear(w, bias, L.MMA_F16X3)
    c = K.linear(a, pw, act=L.ACT_GELU_ERF, out_dtype=out_dtype)
    ref = F.gelu(a.double() @ w.double().t() + bias.double(), approximate="none")
    assert c.dtype == out_dtype
    tol = {torch.float32: 1e-5, torch.float16: 2e-3, torch.bfloat16: 1.6e-2}[out_dtype]
    assert ((c.double() - ref).abs() / ref.abs().clamp_min(1.0)).max().item() < tol


def test_gemm_strided_and_narrow_inputs():
    torch.manual_seed(3)
    big = torch.randn(200, 640, device=DEV)
    a = big[:, 64:576]                   # lda 640, K 512
    w = torch.randn(256, 512, device=DEV) * 0.05
    pw = K.PreparedLinear(w, None, L.MMA_F16X3)
    c = K.linear(a, pw)
    ref = a.double() @ w.double().t()
    assert (c.double() - ref).abs().max().item() < 1e-4
    c16 = K.linear(a.half(), K.PreparedLinear(w, None, L.MMA_F16))
    assert (c16.double() - a.half().double() @ w.half().double().t()).abs().max().item() < 5e-3


def test_gemm_rejects_unsupported_shapes():
    a = torch.randn(16, 30, device=DEV)
    w = torch.randn(8, 30, device=DEV)
    with pytest.raises(L.UnsupportedError):
        K.linear(a, K.PreparedLinear(w, None, L.MMA_F16X3))


@pytest.mark.parametrize("M,N,K_", [(256, 768, 256), (517, 192, 64), (1000, 1024, 512),
                                    (64, 4096, 1024), (130, 36, 2048), (77, 260, 96)])
def test_gemm_f16x2_matches_fp64(M, N, K_):
    """f16x2: A is one fp16 plane (exact input), W keeps 22 bits as hi/lo planes, so the
    product of the fp16 A with the fp32 W is fp32-accurate (the f16x3 bound)."""
    torch.manual_seed(11)
    a = torch.randn(M, K_, device=DEV).half()
    w = torch.randn(N, K_, device=DEV) * 0.05
    bias = torch.randn(N, device=DEV)
    pw = K.PreparedLinear(w, bias, L.MMA_F16X2)
    assert pw.lo is not None and pw.hi.dtype == torch.float16
    c = K.linear(a, pw)
    ref = a.double() @ w.double().t() + bias.double()
    err = (c.double() - ref).abs().max().item()
    scale = K_ ** 0.5 * a.abs().max().item() * w.abs().max().item()
    assert err / scale < GEMM_TOL["f16x3"], f"err {err:.3e} scale {scale:.3e}"
    # the weight's lo plane is used: dropping it (single-pass fp16) is measurably worse
    c1 = K.linear(a, K.PreparedLinear(w, bias, L.MMA_F16))
    assert (c1.double() - ref).abs().max().item() > 4 * err


def test_gemm_f16x2_rejects_what_it_cannot_read():
    w = torch.randn(64, 96, device=DEV)
    pw = K.PreparedLinear(w, None, L.MMA_F16X2)
    for a in (torch.randn(32, 96, device=DEV),                       # fp32 A
              K.Planes.from_float(torch.randn(32, 96, device=DEV))):   # X2 planes
        with pytest.raises(L.UnsupportedError):
            K.linear(a, pw)
    w40 = K.PreparedLinear(torch.randn(64, 40, device=DEV), None, L.MMA_F16X2)
    with pytest.raises(L.UnsupportedError):                          # K % 32 != 0
        K.linear(torch.randn(32, 40, device=DEV).half(), w40)


# --------------------------------------------------------------- attention
def reference_attention(q, k, v, keep, causal, scale=None):
    """Exact softmax attention in fp64 (`BaselineSelfAttention.forward` order)."""
    scale = q.shape[-1] ** -0.5 if scale is None else scale
    s = torch.matmul(q.double(), k.double().transpose(-2, -1)) * scale
    S = q.shape[2]
    if causal:
        s = s.masked_fill(torch.ones(S, S, device=q.device, dtype=torch.bool).triu(1), float("-inf"))
    if keep is not None:
        s = s.masked_fill(~keep.bool()[:, None, None, :], float("-inf"))
    p = torch.softmax(s, dim=-1)
    p = torch.nan_to_num(p, nan=0.0)      # rows with no valid key -> 0 (kernel guard)
    return torch.matmul(p, v.double())


# (2, 2, 2048, 64) and (2, 1, 1024, 128): fewer than 8 heads with query blocks to spare,
# so the grid deals each head's query blocks out in parts (and, for the first, the second
# half of each XCD's range takes its light/heavy pairs heavy block first)
SHAPES = [(2, 8, 128, 64), (1, 4, 1, 64), (2, 8, 333, 64), (1, 8, 2048, 64),
          (1, 4, 100, 128), (2, 4, 64, 32), (2, 2, 300, 256), (2, 8, 200, 8), (1, 4, 77, 16),
          (2, 2, 2048, 64), (2, 1, 1024, 128)]


@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("pad", [0.0, 0.4])
@pytest.mark.parametrize("dtype,mode", [(torch.float32, L.MMA_F16X3), (torch.float16, L.MMA_F16),
                                        (torch.float32, L.MMA_BF16X3)])
def test_flash_attention_matches_reference(shape, causal, pad, dtype, mode):
    torch.manual_seed(0)
    B, H, S, Dh = shape
    q, k, v = (torch.randn(B, H, S, Dh, device=DEV).to(dtype) for _ in range(3))
    keep = None
    if pad > 0:
        lens = torch.randint(1, S + 1, (B,), device=DEV)
        keep = (torch.arange(S, device=DEV)[None, :] < lens[:, None]).to(torch.uint8)
    out = K.flash_attention(q, k, v, keep=keep, causal=causal, mode=mode)
    ref = reference_attention(q, k, v, keep, causal)
    err = (out.double() - ref).abs().max().item()
    tol = {L.MMA_F16X3: 2e-5, L.MMA_BF16X3: 2e-4, L.MMA_F16: 4e-3}[mode]
    assert err < tol, f"max err {err:.3e}"


@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("pad", [0.0, 0.4])
def test_flash_single_plane_probabilities(shape, causal, pad):
    """KF_FLASH_P16: q.k in f16x3, P.V with P rounded once to fp16 (nearest). Each weight
    moves by at most 2^-11 of itself (normal range) or 2^-25 (subnormal), and l comes from
    the unrounded p >= 0.5 at the row maximum, so |out - ref| <= 2^-11 max|v| + S 2^-24 max|v|
    beyond the f16x3 error."""
    torch.manual_seed(0)
    B, H, S, Dh = shape
    q, k, v = (torch.randn(B, H, S, Dh, device=DEV) for _ in range(3))
    keep = None
    if pad > 0:
        lens = torch.randint(1, S + 1, (B,), device=DEV)
        keep = (torch.arange(S, device=DEV)[None, :] < lens[:, None]).to(torch.uint8)
    out = K.flash_attention(q, k, v, keep=keep, causal=causal, mode=L.MMA_F16X3, p16=True)
    ref = reference_attention(q, k, v, keep, causal)
    vmax = v.abs().max().item()
    err = (out.double() - ref).abs().max().item()
    assert err < 2e-5 + (2.0 ** -11 + S * 2.0 ** -24) * vmax, f"max err {err:.3e}"
    full = K.flash_attention(q, k, v, keep=keep, causal=causal, mode=L.MMA_F16X3)
    assert not torch.equal(out, full) or S == 1, "the P16 flag must change the P.V path"


def _rounded_scores_attention(q, k, v, keep, causal, dtype):
    """The reference's narrow score path (`torch_transformer_benchmark.py` attention in a
    16-bit dtype, as `ops/flash.py:145-157` reproduces it): s = E(E(q.k) * scale) with the
    product taken in fp32; masks, softmax and P.V then exact (fp64)."""
    scale = q.shape[-1] ** -0.5
    qk = torch.matmul(q.double(), k.double().transpose(-2, -1)).to(dtype)
    s = (qk.float() * scale).to(dtype).double()
    S = q.shape[2]
    if causal:
        s = s.masked_fill(torch.ones(S, S, device=q.device, dtype=torch.bool).triu(1), float("-inf"))
    if keep is not None:
        s = s.masked_fill(~keep.bool()[:, None, None, :], float("-inf"))
    p = torch.nan_to_num(torch.softmax(s, dim=-1), nan=0.0)
    return torch.matmul(p, v.double())


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("S", [256, 77])
def test_flash_round_scores_follows_the_narrow_reference(dtype, causal, S):
    """KF_FLASH_ROUND_SCORES: against the narrow score rounding done exactly, the kernel
    stays within its own P.V rounding, and is several times closer than the same kernel
    without the rounding (whose fp32 scores differ from the narrow ones by up to an ulp
    of the 16-bit type -- the gap the reference's flag exists to close)."""
    torch.manual_seed(3)
    B, H, Dh = 2, 4, 64
    q, k, v = ((2.0 * torch.randn(B, H, S, Dh, device=DEV)).to(dtype) for _ in range(3))
    lens = torch.randint(S // 2, S + 1, (B,), device=DEV)
    keep = (torch.arange(S, device=DEV)[None, :] < lens[:, None]).to(torch.uint8)
    emul = _rounded_scores_attention(q, k, v, keep, causal, dtype)
    out = K.flash_attention(q, k, v, keep=keep, causal=causal, round_scores_to=dtype)
    plain = K.flash_attention(q, k, v, keep=keep, causal=causal)
    assert out.dtype == dtype and torch.isfinite(out).all()
    e_rs = (out.double() - emul).abs()
    e_plain = (plain.double() - emul).abs()
    vmax = v.abs().max().item()
    eps = 2.0 ** -11 if dtype == torch.float16 else 2.0 ** -8
    assert e_rs.max().item() < 8 * eps * vmax, f"max err {e_rs.max().item():.3e}"
    assert e_rs.mean().item() < 0.5 * e_plain.mean().item(), \
        f"rounded {e_rs.mean().item():.3e} vs plain {e_plain.mean().item():.3e}"


def test_flash_round_scores_needs_a_single_pass_mode():
    q = torch.randn(1, 2, 64, 64, device=DEV)
    with pytest.raises(ValueError):
        K.flash_attention(q, q, q, round_scores_to=torch.float16, mode=L.MMA_F16X3)
    with pytest.raises(ValueError):
        K.flash_attention(q, q, q, round_scores_to=torch.float64)


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("Dh", [8, 16, 32, 64, 128, 256])
@pytest.mark.parametrize("variant", ["f16x3", "f16x3+p16", "float16", "bf16x3",
                                     "round_scores_f16", "round_scores_bf16"])
def test_flash_random_keep_mask_not_prefix(causal, Dh, variant):
    """Arbitrary (non-prefix) key masks run the general-mask instantiation, which reads
    keep per key: every head_dim and precision variant against the exact reference (or,
    for score rounding, the narrow reference). One batch row keeps a prefix mask, so both
    instantiations run in the same call and each must serve only its own rows."""
    torch.manual_seed(4 + Dh)
    B, H, S = 3, 2, 257
    dtype = {"float16": torch.float16, "round_scores_f16": torch.float16,
             "round_scores_bf16": torch.bfloat16}.get(variant, torch.float32)
    q, k, v = (torch.randn(B, H, S, Dh, device=DEV).to(dtype) for _ in range(3))
    keep = (torch.rand(B, S, device=DEV) > 0.3).to(torch.int32)
    keep[:, 0] = 1
    keep[2] = (torch.arange(S, device=DEV) < 150).to(torch.int32)      # a prefix row
    kw = {}
    if variant == "f16x3+p16":
        kw = dict(mode=L.MMA_F16X3, p16=True)
    elif variant == "bf16x3":
        kw = dict(mode=L.MMA_BF16X3)
    elif variant.startswith("round_scores"):
        kw = dict(round_scores_to=dtype)
    out = K.flash_attention(q, k, v, keep=keep, causal=causal, **kw)
    if variant.startswith("round_scores"):
        ref = _rounded_scores_attention(q, k, v, keep, causal, dtype)
    else:
        ref = reference_attention(q, k, v, keep, causal)
    vmax = v.abs().max().item()
    tol = {"f16x3": 2e-5, "f16x3+p16": 2e-5 + (2.0 ** -11 + S * 2.0 ** -24) * vmax,
           "float16": 4e-3, "bf16x3": 2e-4, "round_scores_f16": 8 * 2.0 ** -11 * vmax,
           "round_scores_bf16": 8 * 2.0 ** -8 * vmax}[variant]
    err = (out.double() - ref).abs().max().item()
    assert err < tol, f"max err {err:.3e} (tol {tol:.3e})"


def test_fully_masked_row_yields_zero_not_nan():
    q, k, v = (torch.randn(1, 2, 32, 64, device=DEV) for _ in range(3))
    keep = torch.zeros(1, 32, device=DEV, dtype=torch.uint8)
    out = K.flash_attention(q, k, v, keep=keep, causal=False)
    assert torch.isfinite(out).all()
    assert torch.count_nonzero(out) == 0


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
def test_flash_accepts_strided_views_without_copying(dtype):
    B, S, H, Dh = 2, 64, 4, 64
    qkv = torch.randn(B, S, 3, H, Dh, device=DEV).to(dtype)
    q, k, v = (qkv[:, :, i].permute(0, 2, 1, 3) for i in range(3))
    assert not q.is_contiguous() and q.stride(-1) == 1
    out_bshd = torch.empty((B, S, H, Dh), device=DEV, dtype=dtype)
    K.flash_attention(q, k, v, out=out_bshd.permute(0, 2, 1, 3))
    ref = reference_attention(q, k, v, None, False)
    tol = 2e-5 if dtype == torch.float32 else 4e-3
    assert (out_bshd.permute(0, 2, 1, 3).double() - ref).abs().max().item() < tol


@pytest.mark.parametrize("seq_len", [128, 512, 1024, 777])
@pytest.mark.parametrize("padded", [False, True])
def test_causal_masked_blocks_match_exact(seq_len, padded):
    """Diagonal-only masking and padded-block skipping change speed, nothing else."""
    torch.manual_seed(seq_len)
    B, H, Dh = 2, 4, 64
    q, k, v = (torch.randn(B, H, seq_len, Dh, device=DEV) for _ in range(3))
    keep = None
    if padded:
        lens = torch.tensor([seq_len // 3, seq_len], device=DEV)
        keep = (torch.arange(seq_len, device=DEV)[None, :] < lens[:, None]).to(torch.uint8)
    got = K.flash_attention(q, k, v, keep=keep, causal=True)
    want = reference_attention(q, k, v, keep, True)
    assert (got.double() - want).abs().max().item() < 2e-5


def test_skip_pad_rows_zeroes_only_padding_rows():
    torch.manual_seed(5)
    B, H, S, Dh = 2, 4, 300, 64
    q, k, v = (torch.randn(B, H, S, Dh, device=DEV) for _ in range(3))
    lens = torch.tensor([100, 300], device=DEV)
    keep = (torch.arange(S, device=DEV)[None, :] < lens[:, None]).to(torch.uint8)
    full = K.flash_attention(q, k, v, keep=keep, causal=True)
    skip = K.flash_attention(q, k, v, keep=keep, causal=True, skip_pad_rows=True)
    valid = keep.bool()[:, None, :, None].expand_as(full)
    assert torch.equal(full[valid], skip[valid])
    assert torch.count_nonzero(skip[~valid]) == 0


def test_mask_prep_extent_and_prefix():
    keep = torch.zeros(4, 100, dtype=torch.uint8, device=DEV)
    keep[0, :37] = 1
    keep[1, :] = 1
    keep[2, 5] = 1
    keep[2, 50] = 1
    kv, pre = K.mask_prep(keep)
    assert kv.tolist() == [37, 100, 51, 0]
    assert pre.tolist() == [1, 1, 0, 1]


@pytest.mark.parametrize("S", [16, 1000, 4096, 65541])
def test_mask_prep_byte_rows_against_a_cpu_count(S):
    """Byte masks with a 16-byte aligned row stride take 16 positions per load (the tail
    past the last whole 16 one at a time): extents and prefix flags against a CPU count,
    for prefix rows, holed rows, a lone key in each byte of the 16, non-1 truthy bytes
    and empty rows; the row stride padded to a multiple of 16 when S is not one."""
    g = torch.Generator().manual_seed(S)
    ld = (S + 15) // 16 * 16
    rows = []
    for length in (S, S // 2, 1, 0):
        r = torch.zeros(S, dtype=torch.uint8)
        r[:length] = 1
        rows.append(r)
    rows.append((torch.rand(S, generator=g) > 0.5).to(torch.uint8) * 7)
    for j in range(min(16, S)):
        r = torch.zeros(S, dtype=torch.uint8)
        r[S - 1 - j] = 255
        rows.append(r)
    buf = torch.zeros(len(rows), ld, dtype=torch.uint8)
    for i, r in enumerate(rows):
        buf[i, :S] = r
    keep = buf.to(DEV)[:, :S]
    assert keep.stride(0) % 16 == 0 and keep.data_ptr() % 16 == 0
    kv, pre = K.mask_prep(keep)
    want_kv, want_pre = [], []
    for r in rows:
        nz = torch.nonzero(r).flatten()
        n = int(nz[-1]) + 1 if len(nz) else 0
        want_kv.append(n)
        want_pre.append(int(len(nz) == n))
    assert kv.tolist() == want_kv
    assert pre.tolist() == want_pre


def test_flash_is_run_to_run_deterministic():
    torch.manual_seed(6)
    q, k, v = (torch.randn(2, 8, 1000, 64, device=DEV) for _ in range(3))
    a = K.flash_attention(q, k, v, causal=True)
    b = K.flash_attention(q, k, v, causal=True)
    assert torch.equal(a, b)


# --------------------------------------------------------------- split planes / tiles
def test_planes_input_is_bit_identical_to_on_the_fly_split():
    """A producer-written hi/lo pair is the same split the GEMM makes of fp32 input."""
    torch.manual_seed(7)
    a = torch.randn(300, 512, device=DEV)
    w = torch.randn(768, 512, device=DEV) * 0.05
    pw = K.PreparedLinear(w, torch.randn(768, device=DEV), L.MMA_F16X3)
    assert torch.equal(K.linear(K.Planes.from_float(a), pw), K.linear(a, pw))
    pb = K.PreparedLinear(w, None, L.MMA_BF16X3)
    assert torch.equal(K.linear(K.Planes.from_float(a, K.BF16X2), pb), K.linear(a, pb))


@pytest.mark.parametrize("fmt", ["f16x2", "bf16x2"])
def test_planes_outputs_reconstruct_fp32(fmt):
    pf = K.F16X2 if fmt == "f16x2" else K.BF16X2
    # representation error of hi + lo: 2^-21 relative (fp16 lo) / 2^-15 (bf16 lo), plus
    # the fp16 subnormal step 2^-24 for the lo of tiny values
    rel = 2.0 ** -21 if fmt == "f16x2" else 2.0 ** -15
    floor = 2.0 ** -24 if fmt == "f16x2" else 0.0
    torch.manual_seed(8)
    # GEMM epilogue
    a = torch.randn(200, 256, device=DEV)
    pw = K.PreparedLinear(torch.randn(512, 256, device=DEV) * 0.05, torch.randn(512, device=DEV),
                          L.MMA_F16X3)
    ref = K.linear(a, pw, act=L.ACT_GELU_ERF)
    got = K.linear(a, pw, act=L.ACT_GELU_ERF, out_dtype=pf)
    assert ((got.float() - ref).abs() <= rel * ref.abs() + floor + 1e-30).all()
    # LayerNorm output
    x = torch.randn(100, 512, device=DEV)
    wln, bln = torch.randn(512, device=DEV), torch.randn(512, device=DEV)
    _, h32 = K.add_mask_layernorm(x, None, None, wln, bln)
    _, hp = K.add_mask_layernorm(x, None, None, wln, bln, out_dtype=pf)
    assert ((hp.float() - h32).abs() <= rel * h32.abs() + floor + 1e-30).all()
    # attention output, written straight into a [B, S, H, Dh] planes buffer
    q, k, v = (torch.randn(2, 4, 100, 64, device=DEV) for _ in range(3))
    o32 = K.flash_attention(q, k, v, causal=True)
    op = K.Planes.empty((2, 100, 4, 64), pf, DEV)
    K.flash_attention(q, k, v, causal=True, out=op.permute(0, 2, 1, 3))
    got = op.permute(0, 2, 1, 3).float()
    assert ((got - o32).abs() <= rel * o32.abs() + floor + 1e-30).all()


@pytest.mark.parametrize("M,N,K_", [(1000, 768, 512), (4096, 512, 2048), (130, 36, 64),
                                    (77, 260, 96)])
def test_every_gemm_tile_is_bit_identical(M, N, K_):
    """The K accumulation order does not depend on the tile, so every configuration
    must produce the same bits; a tiling bug cannot hide behind a tolerance."""
    torch.manual_seed(9)
    a = K.Planes.from_float(torch.randn(M, K_, device=DEV))
    pw = K.PreparedLinear(torch.randn(N, K_, device=DEV) * 0.05, torch.randn(N, device=DEV),
                          L.MMA_F16X3)
    outs, outs_p, outs_g = [], [], []
    tiles = K.gemm_tiles()
    for tile, _ in tiles:                       # every register-staged and LDS-DMA tile
        outs.append(K.linear(a, pw, tile=tile))
        # 16-bit planes out, with and without the GELU epilogue (8-column stores)
        if (M * N) % 8 == 0:    # the lo plane of [2, M, N] starts 16-byte aligned
            outs_p.append(K.linear(a, pw, out_dtype=K.F16X2, tile=tile).float())
        outs_g.append(K.linear(a, pw, act=L.ACT_GELU_ERF, out_dtype=torch.float16, tile=tile))
    assert len(outs) >= 15
    for o in outs_p[1:]:
        assert torch.equal(o, outs_p[0])
    for o in outs_g[1:]:
        assert torch.equal(o, outs_g[0])
    if outs_p:
        assert ((outs_p[0] - outs[0]).abs() <= 2.0 ** -21 * outs[0].abs() + 2.0 ** -24).all()
    ref = a.float().double() @ pw.hi.double().t()
    for o in outs[1:]:
        assert torch.equal(o, outs[0])
    assert (outs[0].double() - (a.float().double() @ (pw.hi.double() + pw.lo.double()).t()
                                + pw.bias.double())).abs().max().item() < 1e-3


@pytest.mark.parametrize("M,N,K_", [(1000, 768, 512), (4096, 512, 2048), (130, 36, 64),
                                    (77, 260, 96)])
def test_every_f16x2_tile_is_bit_identical(M, N, K_):
    """f16x2 over every LDS-DMA tile (register-staged overrides yield to the automatic
    DMA tile): fp32, fp16 and GELU outputs identical to the bit."""
    torch.manual_seed(12)
    a = torch.randn(M, K_, device=DEV).half()
    pw = K.PreparedLinear(torch.randn(N, K_, device=DEV) * 0.05, torch.randn(N, device=DEV),
                          L.MMA_F16X2)
    outs, outs_g = [], []
    for tile, _ in K.gemm_tiles():
        outs.append(K.linear(a, pw, tile=tile))
        outs_g.append(K.linear(a, pw, act=L.ACT_GELU_ERF, out_dtype=torch.float16, tile=tile))
    assert len(outs) >= 15
    for o in outs[1:]:
        assert torch.equal(o, outs[0])
    for o in outs_g[1:]:
        assert torch.equal(o, outs_g[0])
    ref = a.double() @ (pw.hi.double() + pw.lo.double()).t() + pw.bias.double()
    assert (outs[0].double() - ref).abs().max().item() < 1e-4


@pytest.mark.parametrize("M,N,K_", [(1000, 768, 512), (4096, 512, 4096), (130, 36, 64),
                                    (300, 260, 128), (2000, 1028, 4096)])
def test_every_fp16_tile_is_bit_identical(M, N, K_):
    """fp16 over every tile (the 256 x 256 LDS-DMA tile runs only in the single-pass modes,
    whose stages fit it): fp32 with and without bias, fp16 GELU and GELU into fp16 planes
    identical to the bit, ragged N edges included (the bias of columns past N is read as
    zero and never stored). The planes must also hold the fp32 GELU to their precision:
    hi and lo split from one value (a hi re-rounded from the exact product had put hi + lo
    an fp16 ulp off at ties)."""
    torch.manual_seed(14)
    a = torch.randn(M, K_, device=DEV).half()
    w = torch.randn(N, K_, device=DEV) * K_ ** -0.5
    pw = K.PreparedLinear(w, torch.randn(N, device=DEV), L.MMA_F16)
    pn = K.PreparedLinear(w, None, L.MMA_F16)
    outs, outs_n, outs_g, outs_p = [], [], [], []
    for tile, _ in K.gemm_tiles():
        outs.append(K.linear(a, pw, tile=tile))
        outs_n.append(K.linear(a, pn, tile=tile))
        outs_g.append(K.linear(a, pw, act=L.ACT_GELU_ERF, out_dtype=torch.float16, tile=tile))
        if (M * N) % 8 == 0:
            outs_p.append(K.linear(a, pw, act=L.ACT_GELU_ERF, out_dtype=K.F16X2, tile=tile).float())
    assert len(outs) >= 16
    for group in (outs, outs_n, outs_g, outs_p):
        for o in group[1:]:
            assert torch.equal(o, group[0])
    if outs_p:
        x = outs[0].double()
        gelu = 0.5 * x * (1.0 + torch.erf(x / math.sqrt(2.0)))
        assert ((outs_p[0].double() - gelu).abs() <= 2.0 ** -20 * gelu.abs() + 2.0 ** -23).all()
    ref = a.double() @ pw.hi.double().t()
    assert (outs_n[0].double() - ref).abs().max().item() < 1e-3
    assert (outs[0].double() - ref - pw.bias.double()).abs().max().item() < 1e-3


@pytest.mark.parametrize("mode", [L.MMA_BF16X3, L.MMA_BF16])
@pytest.mark.parametrize("M,N,K_", [(1000, 768, 512), (2000, 1028, 4096), (130, 36, 64),
                                    (300, 260, 128)])
def test_every_bf16_tile_is_bit_identical(mode, M, N, K_):
    """The bf16 modes over every tile (bf16x3 from bf16 planes of A, single-pass bf16 from
    one bf16 plane; the 256 x 256 tiles where their stages fit): fp32 with and without bias,
    bf16 GELU and GELU into bf16 planes identical to the bit, ragged N edges included, and
    the fp32 result against float64 at the mode's precision."""
    torch.manual_seed(16)
    a32 = torch.randn(M, K_, device=DEV)
    a = K.Planes.from_float(a32, K.BF16X2) if mode == L.MMA_BF16X3 else a32.bfloat16()
    w = torch.randn(N, K_, device=DEV) * K_ ** -0.5
    pw = K.PreparedLinear(w, torch.randn(N, device=DEV), mode)
    pn = K.PreparedLinear(w, None, mode)
    outs, outs_n, outs_g, outs_p = [], [], [], []
    for tile, _ in K.gemm_tiles():
        outs.append(K.linear(a, pw, tile=tile))
        outs_n.append(K.linear(a, pn, tile=tile))
        outs_g.append(K.linear(a, pw, act=L.ACT_GELU_ERF, out_dtype=torch.bfloat16, tile=tile))
        if (M * N) % 8 == 0:
            outs_p.append(K.linear(a, pw, act=L.ACT_GELU_ERF, out_dtype=K.BF16X2, tile=tile).float())
    assert len(outs) >= 16
    for group in (outs, outs_n, outs_g, outs_p):
        for o in group[1:]:
            assert torch.equal(o, group[0])
    a64 = a.float().double() if isinstance(a, K.Planes) else a.double()
    w64 = pw.hi.double() + (pw.lo.double() if pw.lo is not None else 0.0)
    ref = a64 @ w64.t()
    bound = (2e-4 if mode == L.MMA_BF16X3 else 2e-2) * K_ ** 0.5 * a64.abs().max().item() \
        * w64.abs().max().item()
    assert (outs_n[0].double() - ref).abs().max().item() < bound
    assert (outs[0].double() - ref - pw.bias.double()).abs().max().item() < bound


@pytest.mark.parametrize("mode", [L.MMA_F16X3, L.MMA_F16, L.MMA_F16X2])
@pytest.mark.parametrize("M,N", [(65536, 1024), (262144, 1024), (98304, 3072)])
def test_grouped_tile_walk_is_bit_identical_to_row_major(mode, M, N):
    """Grids that take many rounds of tiles walk them in groups of row blocks (4 or 8 at
    these sizes); slices of the same rows small enough for one round walk them row-major.
    Each output tile is the same computation either way: the bits must agree."""
    torch.manual_seed(13)
    K_ = 256
    a = torch.randn(M, K_, device=DEV)
    a = a.half() if mode in (L.MMA_F16, L.MMA_F16X2) else K.Planes.from_float(a)
    pw = K.PreparedLinear(torch.randn(N, K_, device=DEV) * 0.05, torch.randn(N, device=DEV),
                          mode)
    whole = K.linear(a, pw)
    rows = 2048                      # <= 16 x 8 tiles: one round on 256 CUs
    for lo in range(0, M, M // 8):   # eight slices spread over the rows
        part = a[lo:lo + rows] if not isinstance(a, K.Planes) else \
            K.Planes(a.hi[lo:lo + rows], a.lo[lo:lo + rows])
        assert torch.equal(K.linear(part, pw), whole[lo:lo + rows]), lo


def _a16(h, mode):
    """h in the 16-bit operand format of `mode` (what the layer's producers write)."""
    if mode == L.MMA_F16X3:
        return K.Planes.from_float(h, K.F16X2)
    if mode == L.MMA_BF16X3:
        return K.Planes.from_float(h, K.BF16X2)
    return h.half() if mode in (L.MMA_F16, L.MMA_F16X2) else h.bfloat16()


@pytest.mark.parametrize("mode,a16", [(L.MMA_F16X3, False), (L.MMA_F16X3, True),
                                      (L.MMA_BF16X3, False), (L.MMA_BF16X3, True),
                                      (L.MMA_F16, False), (L.MMA_F16, True),
                                      (L.MMA_F16X2, True)])
@pytest.mark.parametrize("B,S,H,Dh", [(2, 77, 4, 64), (1, 128, 8, 8), (2, 33, 2, 256)])
def test_qkv_epilogue_writes_the_attention_layout(mode, B, S, H, Dh, a16):
    """q token-major fp32 (bit-identical to the plain GEMM), k split planes, v^T planes;
    fp32 A (register-staged kernel) and 16-bit A (LDS-DMA kernel). f16x2 (fp16 A only)
    writes split k / v^T planes like f16x3."""
    torch.manual_seed(10)
    d = H * Dh
    h = torch.randn(B * S, d, device=DEV)
    pw = K.PreparedLinear(torch.randn(3 * d, d, device=DEV) * 0.05,
                          torch.randn(3 * d, device=DEV), mode)
    if a16:
        h = _a16(h, mode)
    ref = K.linear(h, pw)
    ops = K.linear_qkv(h, pw, B, S, H, Dh)
    view = lambda t: t.reshape(B, S, H, Dh).permute(0, 2, 1, 3)  # noqa: E731
    assert torch.equal(ops.q, view(ref[:, :d]))
    k = ops.k_hi.float() + (ops.k_lo.float() if ops.k_lo is not None else 0)
    v = ops.vt_hi.float() + (ops.vt_lo.float() if ops.vt_lo is not None else 0)
    rel = {L.MMA_F16X3: 2.0 ** -21, L.MMA_BF16X3: 2.0 ** -15, L.MMA_F16: 2.0 ** -11,
           L.MMA_F16X2: 2.0 ** -21}[mode]
    assert ops.mode == (L.MMA_F16X3 if mode == L.MMA_F16X2 else mode)
    kr, vr = view(ref[:, d:2 * d]), view(ref[:, 2 * d:]).transpose(-1, -2)
    assert ((k - kr).abs() <= rel * kr.abs() + 2.0 ** -24).all()
    assert ((v[..., :S] - vr).abs() <= rel * vr.abs() + 2.0 ** -24).all()
    if mode == L.MMA_F16X3:
        # "f16x3s": the same GEMM writing one plane of k and v^T (epilogue 5) -- the fp32
        # projection rounded to nearest fp16, bit-identical to the split planes' hi part
        one = K.linear_qkv(h, pw, B, S, H, Dh, single=True)
        assert one.mode == L.MMA_F16 and one.k_lo is None and one.vt_lo is None
        assert torch.equal(one.q, ops.q)
        assert torch.equal(one.k_hi, ops.k_hi) and torch.equal(one.vt_hi[..., :S], ops.vt_hi[..., :S])
        assert torch.equal(one.k_hi, kr.half()) and torch.equal(one.vt_hi[..., :S], vr.half())


@pytest.mark.parametrize("mode", [L.MMA_F16X3, L.MMA_F16, L.MMA_F16X2, L.MMA_BF16X3, L.MMA_BF16])
@pytest.mark.parametrize("B,S,H,Dh", [(2, 300, 4, 64), (1, 1000, 3, 128)])
def test_qkv_epilogue_is_bit_identical_over_every_tile(mode, B, S, H, Dh):
    """The QKV epilogue (q fp32, k and v^T in the attention layout; for f16x3 also the
    single-plane form) on every tile, the 256 x 256 tiles that C4's and C5's projections
    take included: the same bits as the automatic tile, rows ending mid-tile (S not a
    multiple of the tile rows) and v^T rows mid-chunk."""
    torch.manual_seed(15)
    d = H * Dh
    h = _a16(torch.randn(B * S, d, device=DEV), mode)
    pw = K.PreparedLinear(torch.randn(3 * d, d, device=DEV) * d ** -0.5,
                          torch.randn(3 * d, device=DEV), mode)
    view = lambda t: t.reshape(B, S, H, Dh).permute(0, 2, 1, 3)  # noqa: E731
    ref_q = view(K.linear(h, pw)[:, :d])
    for single in ([False, True] if mode == L.MMA_F16X3 else [False]):
        base = K.linear_qkv(h, pw, B, S, H, Dh, single=single)
        assert torch.equal(base.q, ref_q)
        assert (base.k_lo is None) == (base.vt_lo is None) == (single or mode in (L.MMA_F16, L.MMA_BF16))
        n = 0
        for tile, _ in K.gemm_tiles():
            o = K.linear_qkv(h, pw, B, S, H, Dh, tile=tile, single=single)
            why = (tile, single)
            assert torch.equal(o.q, base.q), why
            assert torch.equal(o.k_hi, base.k_hi), why
            assert torch.equal(o.vt_hi[..., :S], base.vt_hi[..., :S]), why
            if base.k_lo is not None:
                assert torch.equal(o.k_lo, base.k_lo), why
                assert torch.equal(o.vt_lo[..., :S], base.vt_lo[..., :S]), why
            n += 1
        assert n >= 16


@pytest.mark.parametrize("Dh", [64, 128])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("S,pad", [(77, 0.0), (300, 0.4), (1000, 0.3), (2048, 0.0)])
def test_pipelined_and_unpipelined_single_pass_kernels_both_match(Dh, dtype, causal, S, pad):
    """Single-pass fp16 / bf16 at head_dim 64 / 128 runs the kernel pipelined over 32-key
    chunks on the 32x32x16 MFMA; KF_FLASH_NO_PIPE selects the unpipelined one. Both
    against exact attention, over sequence lengths that end mid-chunk, mid-tile and on a
    tile edge, with padded rows (the fast/slow chunk split and the four- / three-stage
    copy pipeline)."""
    torch.manual_seed(S + Dh)
    B, H = 3, 2
    q, k, v = (torch.randn(B, H, S, Dh, device=DEV).to(dtype) for _ in range(3))
    keep = None
    if pad > 0:
        lens = torch.tensor([S, max(1, int(S * (1 - pad))), max(1, S // 3)], device=DEV)
        keep = (torch.arange(S, device=DEV)[None, :] < lens[:, None]).to(torch.uint8)
    mode = L.MMA_F16 if dtype == torch.float16 else L.MMA_BF16
    k_hi, _, vt_hi, _ = K.attn_prep(k, v, mode)
    ref = reference_attention(q, k, v, keep, causal)
    outs = []
    for extra in (0, L.FLASH_NO_PIPE):
        o = torch.empty_like(q)
        kv_len = prefix = None
        if keep is not None:
            kv_len, prefix = K.mask_prep(keep)
        flags = (L.FLASH_CAUSAL if causal else 0) | extra
        st = L.lib().kf_flash_fwd(
            q.data_ptr(), L.strides4(q), K._code(q), k_hi.data_ptr(), None, L.strides4(k_hi),
            vt_hi.data_ptr(), None, L.strides4(vt_hi), o.data_ptr(), None, L.strides4(o),
            K._code(o), None if keep is None else keep.data_ptr(), L.U8, S,
            None if kv_len is None else kv_len.data_ptr(),
            None if prefix is None else prefix.data_ptr(), B, H, S, Dh, Dh ** -0.5, mode, flags,
            torch.cuda.current_stream().cuda_stream)
        L.check("kf_flash_fwd", st)
        outs.append(o)
    tol = 4e-3 if dtype == torch.float16 else 3e-2
    for o in outs:
        err = (o.double() - ref).abs().max().item()
        assert err < tol, f"max err {err:.3e}"
    assert not torch.equal(outs[0], outs[1]) or S < 64, "the flag must select the other kernel"


@pytest.mark.parametrize("kernel", ["pipe hd64 fp16", "small hd8 f16x3"])
@pytest.mark.parametrize("causal", [False, True])
def test_stage_unrolled_fast_loop_every_length(kernel, causal):
    """The hd-64 pipelined kernel (two query tiles per wavefront: passes of six steady
    chunks, the rest checked) and the hd-8 packed kernel (entered at tile 1 when tiles 1-3
    are all fast, three tiles per pass, the rest in the generic loop) unroll their loops
    over the three LDS stages: key loops of 1 to 12 fast tiles (S = 64 t + 32 keys, every
    count mod 3, below and above the entry) against exact attention, bidirectional (every
    wavefront the same length) and causal (a length per wavefront)."""
    hd8 = kernel.startswith("small")
    Dh = 8 if hd8 else 64
    mode = L.MMA_F16X3 if hd8 else L.MMA_F16
    for t in range(1, 13):
        S = 64 * t + 32
        torch.manual_seed(S + Dh)
        q, k, v = (torch.randn(1, 2, S, Dh, device=DEV) for _ in range(3))
        if not hd8:
            q, k, v = (x.half() for x in (q, k, v))
        ref = reference_attention(q, k, v, None, causal)
        o = _flash_both_kernels(q, k, v, None, causal, mode)[0]
        tol = 2e-5 if hd8 else 4e-3
        err = (o.double() - ref).abs().max().item()
        assert err < tol, f"S={S}: max err {err:.3e}"


def _moving_reference_case(profile, B, H, S, Dh, dtype, seed):
    """q, k, v whose score rows make the lazy softmax reference move at chosen places:
    "rising" adds a key ramp along a shared direction (the row maximum climbs ~43 (hd 64) /
    ~30 (hd 128) log2 units over the row, so the reference passes its 2^8 bound several
    times inside the steady part of the key loop), "falling" the same ramp reversed (the
    first chunk holds the maximum: no move after it), "wide" large random scores (moves at
    random chunks, and chunks whose probabilities sum past 2^8 without any one passing it)."""
    g = torch.Generator(device="cpu").manual_seed(seed)
    q, k, v = (torch.randn(B, H, S, Dh, generator=g) for _ in range(3))
    if profile == "wide":
        q, k = 3.0 * q, 3.0 * k
    else:
        u = torch.full((Dh,), Dh ** -0.5)
        ramp = torch.linspace(0.0, 1.0, S) if profile == "rising" else torch.linspace(1.0, 0.0, S)
        q = 0.3 * q + 4.0 * u
        k = 0.3 * k + (60.0 * ramp)[:, None] * u
    return tuple(t.to(DEV).to(dtype) for t in (q, k, v))


@pytest.mark.parametrize("Dh", [64, 128])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("profile", ["rising", "falling", "wide"])
@pytest.mark.parametrize("causal", [False, True])
def test_pipelined_reference_moves_inside_the_key_loop(Dh, dtype, profile, causal):
    """The pipelined kernel checks a chunk's row maximum only where a row sum of
    probabilities reaches 2^8; where some score then passed the lazy bound it forms the
    chunk's scores again and moves the reference. Score rows built to move it (or not)
    at chosen places, against exact attention and against the unpipelined kernel, which
    checks every tile's maximum.

    Tolerance: both kernels form scores from q pre-scaled and rounded to the 16-bit type
    (unit roundoff u), so a score x (log2 units) moves by up to u|x| and its weight by a
    factor 2^(±u|x|); over the keys a row mixes these errors largely cancel, and u (1 +
    max|x| / 16) of max|v| holds with >= 1.4x margin on every row here (the largest rows
    reach |x| ~ 80). A reference that failed to move would overflow p (these rows climb
    past 2^16); one that moved without re-forming the scores would be off by 2^8."""
    B, H, S = 2, 2, 2048
    q, k, v = _moving_reference_case(profile, B, H, S, Dh, dtype, seed=Dh + S)
    mode = L.MMA_F16 if dtype == torch.float16 else L.MMA_BF16
    ref = reference_attention(q, k, v, None, causal)
    got = K.flash_attention(q, k, v, causal=causal, mode=mode)
    k_hi, _, vt_hi, _ = K.attn_prep(k, v, mode)
    o = torch.empty_like(q)
    st = L.lib().kf_flash_fwd(
        q.data_ptr(), L.strides4(q), K._code(q), k_hi.data_ptr(), None, L.strides4(k_hi),
        vt_hi.data_ptr(), None, L.strides4(vt_hi), o.data_ptr(), None, L.strides4(o),
        K._code(o), None, L.U8, S, None, None, B, H, S, Dh, Dh ** -0.5, mode,
        (L.FLASH_CAUSAL if causal else 0) | L.FLASH_NO_PIPE,
        torch.cuda.current_stream().cuda_stream)
    L.check("kf_flash_fwd", st)
    vmax = v.abs().max().item()
    smax = ((q.double() @ k.double().transpose(-1, -2)).abs().max().item()
            * Dh ** -0.5 / math.log(2.0))
    u = 2.0 ** -11 if dtype == torch.float16 else 2.0 ** -8
    tol = u * (1.0 + smax / 16.0) * vmax
    for out in (got, o):
        assert torch.isfinite(out).all()
        err = (out.double() - ref).abs().max().item()
        assert err < tol, f"max err {err:.3e} (tol {tol:.1e})"
    if Dh == 64:
        # the two-tile kernel takes the one-tile kernel's moves (and re-forms) bit for bit
        two, one = _flash_both_kernels(q, k, v, None, causal, mode, other=L.FLASH_ONE_TILE)
        assert torch.equal(two, one) and torch.equal(two, got)


def _flash_both_kernels(q, k, v, keep, causal, mode, extra_flags=0, other=L.FLASH_NO_PIPE):
    """kf_flash_fwd on the default kernel and on the one `other` selects (KF_FLASH_NO_PIPE:
    the 16x16x32 kernel)."""
    B, H, S, Dh = q.shape
    k_hi, k_lo, vt_hi, vt_lo = K.attn_prep(k, v, mode)
    kv_len = prefix = None
    if keep is not None:
        kv_len, prefix = K.mask_prep(keep)
    outs = []
    for extra in (0, other):
        o = torch.empty_like(q)
        st = L.lib().kf_flash_fwd(
            q.data_ptr(), L.strides4(q), K._code(q), k_hi.data_ptr(),
            None if k_lo is None else k_lo.data_ptr(), L.strides4(k_hi),
            vt_hi.data_ptr(), None if vt_lo is None else vt_lo.data_ptr(), L.strides4(vt_hi),
            o.data_ptr(), None, L.strides4(o), K._code(o),
            None if keep is None else keep.data_ptr(), L.U8, S,
            None if kv_len is None else kv_len.data_ptr(),
            None if prefix is None else prefix.data_ptr(), B, H, S, Dh, Dh ** -0.5, mode,
            (L.FLASH_CAUSAL if causal else 0) | extra_flags | extra,
            torch.cuda.current_stream().cuda_stream)
        L.check("kf_flash_fwd", st)
        outs.append(o)
    return outs


@pytest.mark.parametrize("dtype,qdtype", [(torch.float16, torch.float16),
                                          (torch.bfloat16, torch.bfloat16),
                                          (torch.float16, torch.float32)])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("S,pad", [(77, 0.0), (449, 0.4), (1000, 0.3), (64 * 13 + 32, 0.0),
                                   (4128, 0.2)])
def test_two_tile_kernel_equals_one_tile_kernel_bit_for_bit(dtype, qdtype, causal, S, pad):
    """Single-pass attention at head_dim 64 runs two 32-row query tiles per wavefront,
    sharing each K / V^T fragment between them; each tile takes the MFMAs and softmax steps
    of the one-tile pipelined kernel (KF_FLASH_ONE_TILE) in the same order, so the outputs
    agree bit for bit: lengths that end mid-chunk and around the unrolled passes of six
    chunks, padded rows, 16-bit and fp32 queries; and both against exact attention."""
    torch.manual_seed(S + 64)
    B, H, Dh = 3, 2, 64
    q = torch.randn(B, H, S, Dh, device=DEV).to(qdtype)
    k, v = (torch.randn(B, H, S, Dh, device=DEV).to(dtype) for _ in range(2))
    keep = None
    if pad > 0:
        lens = torch.tensor([S, max(1, int(S * (1 - pad))), max(1, S // 3)], device=DEV)
        keep = (torch.arange(S, device=DEV)[None, :] < lens[:, None]).to(torch.uint8)
    mode = L.MMA_F16 if dtype == torch.float16 else L.MMA_BF16
    two, one = _flash_both_kernels(q, k, v, keep, causal, mode, other=L.FLASH_ONE_TILE)
    assert torch.equal(two, one)
    ref = reference_attention(q.to(dtype).float(), k, v, keep, causal)
    tol = 4e-3 if dtype == torch.float16 else 3e-2
    assert (two.double() - ref).abs().max().item() < tol


@pytest.mark.parametrize("variant", ["f16x3", "f16x3+p16", "bf16x3"])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("S,pad", [(77, 0.0), (300, 0.4), (1000, 0.3), (2048, 0.0)])
def test_head_dim_8_packed_contraction_kernel(variant, causal, S, pad):
    """Head dim 8 in the split modes runs the kernel that packs the split products and
    the reference into the 16-slot contraction of the 32x32x16 MFMA and takes the row
    sum from a ones row of V^T; KF_FLASH_NO_PIPE selects the zero-padded 16x16x32
    kernel. Both against exact attention (the split-mode bounds of
    test_flash_attention_matches_reference; with P as one fp16 plane, the P16 bound of
    test_flash_single_plane_probabilities) over lengths that end mid-chunk, mid-tile and
    on a tile edge, with padded rows."""
    torch.manual_seed(S + 8)
    B, H, Dh = 3, 2, 8
    q, k, v = (torch.randn(B, H, S, Dh, device=DEV) for _ in range(3))
    keep = None
    if pad > 0:
        lens = torch.tensor([S, max(1, int(S * (1 - pad))), max(1, S // 3)], device=DEV)
        keep = (torch.arange(S, device=DEV)[None, :] < lens[:, None]).to(torch.uint8)
    mode = L.MMA_BF16X3 if variant == "bf16x3" else L.MMA_F16X3
    p16 = variant.endswith("p16")
    outs = _flash_both_kernels(q, k, v, keep, causal, mode, L.FLASH_P16 if p16 else 0)
    ref = reference_attention(q, k, v, keep, causal)
    vmax = v.abs().max().item()
    tol = {L.MMA_F16X3: 2e-5, L.MMA_BF16X3: 2e-4}[mode]
    if p16:
        tol += (2.0 ** -11 + S * 2.0 ** -24) * vmax
    for o in outs:
        err = (o.double() - ref).abs().max().item()
        assert err < tol, f"max err {err:.3e}"
    assert not torch.equal(outs[0], outs[1]), "the flag must select the other kernel"


@pytest.mark.parametrize("profile", ["rising", "falling", "wide"])
@pytest.mark.parametrize("causal", [False, True])
def test_head_dim_8_reference_moves_inside_the_key_loop(profile, causal):
    """The packed-contraction kernel's steady chunks on score rows built to move the lazy
    reference (or not) at chosen places (`_moving_reference_case`), f16x3 on fp32 inputs:
    q and k are carried to 22 bits, so scores of |x| ~ 80 stay exact to ~2^-15 and the
    split-mode bound holds, scaled by the largest |v|."""
    B, H, S = 2, 2, 2048
    q, k, v = _moving_reference_case(profile, B, H, S, 8, torch.float32, seed=8 + S)
    outs = _flash_both_kernels(q, k, v, None, causal, L.MMA_F16X3)
    ref = reference_attention(q, k, v, None, causal)
    tol = 2e-5 * v.abs().max().item()
    for o in outs:
        assert torch.isfinite(o).all()
        err = (o.double() - ref).abs().max().item()
        assert err < tol, f"max err {err:.3e} (tol {tol:.1e})"


@pytest.mark.parametrize("dtype,mode", [(torch.float16, L.MMA_F16), (torch.bfloat16, L.MMA_BF16)])
@pytest.mark.parametrize("Dh", [64, 128])
def test_flash_reads_matching_k_in_place(dtype, mode, Dh):
    """Single-pass attention on k already in the mode's type reads it in place (only V is
    transposed, kf_attn_prep with k NULL): bit-identical to the path that copies K into
    its own planes first. Split modes (fp32 k) always copy it into hi / lo planes."""
    torch.manual_seed(21)
    B, H, S = 2, 4, 300
    q, k, v = (torch.randn(B, H, S, Dh, device=DEV).to(dtype) for _ in range(3))
    assert K.k_in_place(k, mode)
    got = K.flash_attention(q, k, v, causal=True, mode=mode)
    k_hi, k_lo, vt_hi, vt_lo = K.attn_prep(k, v, mode)
    ref = K.flash_attention_ops(K.AttnOperands(q, k_hi, k_lo, vt_hi, vt_lo, mode), causal=True)
    assert torch.equal(got, ref)
    # V-only prep writes the same V^T planes as the full prep
    _, _, vt2, _ = K.attn_prep(None, v, mode)
    assert torch.equal(vt2, vt_hi)
    assert not K.k_in_place(k.float(), L.MMA_F16X3)
    assert not K.k_in_place(k, L.MMA_BF16 if mode == L.MMA_F16 else L.MMA_F16)


@pytest.mark.parametrize("dtype,mode", [(torch.float16, L.MMA_F16), (torch.bfloat16, L.MMA_BF16)])
@pytest.mark.parametrize("Dh", [64, 128])
@pytest.mark.parametrize("masked", [False, True])
def test_flash_reads_a_strided_k_view_in_place(dtype, mode, Dh, masked):
    """k as the [B, H, S, Dh] view of a token-major [B, S, H, Dh] tensor (the layout of a
    fused projection's output: strides H*Dh*S, Dh, H*Dh, 1) is read in place by the
    pipelined kernel, with its 32-bit slice offsets; with and without a padded keep mask
    (prefix rows and a row with holes, so both mask launches run). Bit-identical to the
    path that copies K into contiguous planes first."""
    torch.manual_seed(22)
    B, H, S = 3, 4, 333
    q, v = (torch.randn(B, H, S, Dh, device=DEV).to(dtype) for _ in range(2))
    k = torch.randn(B, S, H, Dh, device=DEV).to(dtype).permute(0, 2, 1, 3)
    assert not k.is_contiguous() and K.k_in_place(k, mode)
    keep = None
    if masked:
        keep = torch.arange(S, device=DEV)[None, :] < torch.tensor([S, 200, 77], device=DEV)[:, None]
        keep[2, 10:20] = False                      # a row that is not a prefix
    got = K.flash_attention(q, k, v, keep=keep, causal=True, mode=mode)
    k_hi, k_lo, vt_hi, vt_lo = K.attn_prep(k.contiguous(), v, mode)
    assert k_hi.is_contiguous()
    ref = K.flash_attention_ops(K.AttnOperands(q, k_hi, k_lo, vt_hi, vt_lo, mode), keep=keep,
                                causal=True)
    assert torch.equal(got, ref)
