"""kf_flash_attention_static (the allocation-free variant of the op-level attention) against
the existing path -- kf_attn_prep + kf_mask_prep + kf_flash_fwd with caller buffers, through
`kernels.flash_attention` -- bit for bit, on two calls in a row, the second smaller; the
property it exists for (no device memory taken after the first call on a device, and a
first call made under hipGraph capture, replayed); and its refusal of a problem larger
than its static buffer (checked on the host, nothing launched)."""
from __future__ import annotations

import os
import subprocess
import sys

import pytest
import torch

from techjam2026_amd import _lib as L
from techjam2026_amd import kernels as K

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda")


def _static(q, k, v, keep, causal, mode, p16=False, out=None):
    B, H, S, Dh = q.shape
    o = out if out is not None else torch.empty_like(q, memory_format=torch.contiguous_format)
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


def test_static_takes_no_device_memory_after_its_first_call():
    """After one warm call (which looks the static array's address up), further calls --
    with and without a keep mask, split and single-pass -- leave the device's free memory
    and torch's allocation unchanged: inputs and outputs are the caller's, the staging is
    the static array."""
    q, k, v, keep = _case(2, 8, 700, 64, torch.float32, 3)
    keep_u8 = keep.contiguous()
    o = torch.empty_like(q)
    q16, k16, v16 = q.half(), k.half(), v.half()
    o16 = torch.empty_like(q16)
    _static(q, k, v, keep_u8, True, L.MMA_F16X3, out=o)
    torch.cuda.synchronize()
    free0, _ = torch.cuda.mem_get_info()
    alloc0 = torch.cuda.memory_allocated()
    for _ in range(3):
        _static(q, k, v, keep_u8, True, L.MMA_F16X3, out=o)
        _static(q, k, v, None, False, L.MMA_F16X3, p16=True, out=o)
        _static(q16, k16, v16, keep_u8, True, L.MMA_F16, out=o16)
    torch.cuda.synchronize()
    assert torch.cuda.mem_get_info()[0] == free0
    assert torch.cuda.memory_allocated() == alloc0


# Run in a fresh process, so that the library's first call on the device -- its
# hipGetSymbolAddress lookup of the static array -- happens inside the capture.
_CAPTURE_SCRIPT = r"""
import sys, torch
sys.path.insert(0, sys.argv[1])
sys.path.insert(0, sys.argv[1] + "/tests")
import test_zz_no_alloc as T
from techjam2026_amd import _lib as L, kernels as K
q, k, v, keep = T._case(2, 4, 500, 64, torch.float32, 4)
keep = keep.contiguous()
o = torch.empty_like(q)
s = torch.cuda.Stream()
s.wait_stream(torch.cuda.current_stream())
g = torch.cuda.CUDAGraph()
with torch.cuda.graph(g, stream=s):
    T._static(q, k, v, keep, True, L.MMA_F16X3, out=o)
want = K.flash_attention(q, k, v, keep=keep, causal=True, mode=L.MMA_F16X3)
for i in range(3):
    o.zero_()
    g.replay()
    torch.cuda.synchronize()
    assert torch.equal(o, want), f"replay {i}"
    q.mul_(1.0001)                          # eager work between replays; inputs change
    want = K.flash_attention(q, k, v, keep=keep, causal=True, mode=L.MMA_F16X3)
    torch.cuda.synchronize()
print("CAPTURE_OK", flush=True)
"""


def test_static_first_call_under_graph_capture_replays():
    """A fresh process whose first kf_flash_attention_static call is made under hipGraph
    capture (torch.cuda.graph): each replay, with eager work and a changed input between
    replays, equals the allocating path on the current inputs, bit for bit."""
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    env = dict(os.environ, KF950_STRICT="1")
    r = subprocess.run([sys.executable, "-c", _CAPTURE_SCRIPT, root], capture_output=True,
                       text=True, timeout=240, env=env)
    print(r.stdout[-2000:], r.stderr[-2000:], flush=True)
    assert r.returncode == 0 and "CAPTURE_OK" in r.stdout
