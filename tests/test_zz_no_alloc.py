"""kf_flash_attention_static (the allocation-free variant of the op-level attention) against
the existing path -- kf_attn_prep + kf_mask_prep + kf_flash_fwd with caller buffers, through
`kernels.flash_attention` -- bit for bit, on two calls in a row, the second smaller; and its
refusal of a problem larger than its static buffer (checked on the host, nothing launched)."""
from __future__ import annotations

import pytest
import torch

from techjam2026_amd import _lib as L
from techjam2026_amd import kernels as K

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda")


def _static(q, k, v, keep, causal, mode, p16=False):
    B, H, S, Dh = q.shape
    o = torch.empty_like(q, memory_format=torch.contiguous_format)
    keep_u8 = None if keep is None else keep.to(torch.uint8).contiguous()
    flags = (L.FLASH_CAUSAL if causal else 0) | (L.FLASH_P16 if p16 else 0)
    code = {torch.float32: L.F32, torch.float16: L.F16, torch.bfloat16: L.BF16}[q.dtype]
    st = L.lib().kf_flash_attention_static(
        q.data_ptr(), L.strides4(q), k.data_ptr(), L.strides4(k), v.data_ptr(), L.strides4(v),
        code, o.data_ptr(), None, L.strides4(o), code,
        None if keep_u8 is None else keep_u8.data_ptr(), L.U8, S,
        B, H, S, Dh, float(Dh ** -0.5), mode, flags, torch.cuda.current_stream().cuda_stream)
    L.check("kf_flash_attention_static", st)
    return o


def _case(B, H, S, Dh, dtype, seed):
    g = torch.Generator(device=DEV).manual_seed(seed)
    q, k, v = (torch.randn(B, H, S, Dh, device=DEV, generator=g).to(dtype) for _ in range(3))
    keep = (torch.rand(B, S, device=DEV, generator=g) > 0.25).to(torch.uint8)
    keep[:, 0] = 1
    keep[0] = (torch.arange(S, device=DEV) < (S * 2) // 3).to(torch.uint8)   # a prefix row
    return q, k, v, keep


@pytest.mark.parametrize("dtype,mode,p16", [(torch.float32, L.MMA_F16X3, False),
                                            (torch.float32, L.MMA_F16X3, True),
                                            (torch.float16, L.MMA_F16, False),
                                            (torch.float32, L.MMA_BF16X3, False)])
@pytest.mark.parametrize("causal", [True, False])
def test_static_matches_the_allocating_path_twice_second_smaller(dtype, mode, p16, causal):
    for (B, H, S, Dh), seed in (((2, 8, 700, 64), 1), ((1, 2, 77, 32), 2)):
        q, k, v, keep = _case(B, H, S, Dh, dtype, seed)
        for kp in (keep, None):
            got = _static(q, k, v, kp, causal, mode, p16)
            want = K.flash_attention(q, k, v, keep=kp, causal=causal, mode=mode, p16=p16)
            torch.cuda.synchronize()
            assert torch.equal(got, want), f"B{B} H{H} S{S} d{Dh} keep={kp is not None}"


def test_static_refuses_a_problem_beyond_its_buffer():
    q = torch.empty(1, 1, 8, 64, device=DEV)
    S = 1 << 20           # 16 heads x 1M keys x hd 64 of split planes: far beyond 64 MiB
    with pytest.raises(L.KernelError, match="static scratch holds"):
        L.check("kf_flash_attention_static", L.lib().kf_flash_attention_static(
            q.data_ptr(), L.strides4(q), q.data_ptr(), L.strides4(q), q.data_ptr(),
            L.strides4(q), L.F32, q.data_ptr(), None, L.strides4(q), L.F32, None, L.U8, S,
            1, 16, S, 64, 0.125, L.MMA_F16X3, 0, torch.cuda.current_stream().cuda_stream))
