"""Python surface of the gfx950 kernels, with the reference's op signatures.

The reference's `kernelforge/ops` exports `add_mask_layernorm`, `flash_attention` and
`flash_supported` (`kernelforge/ops/__init__.py:7-11`); the same names and argument
meanings are kept here, so the layer code and the tests read the same. Each call checks
shapes on the host and then goes straight to libkf950 through ctypes on the current
stream; device memory for outputs is allocated with torch (no allocation happens inside
the library). The GEMM wrapper (`linear`, `PreparedLinear`) replaces `F.linear` with the
per-stage MFMA precision.

Activations that feed a split-precision MFMA are carried as `Planes`: an fp32 value x as
hi = round16(x) and lo = round16(x - hi) in two 16-bit tensors of one shape and stride
(dtype codes KF_F16X2 / KF_BF16X2). The producer writes them once, and every GEMM
block that reads them copies 16-bit data straight into LDS.
"""
from __future__ import annotations

import ctypes
from typing import List, Optional, Tuple, Union

import torch

from . import _lib as L

_DT = {torch.float32: L.F32, torch.float16: L.F16, torch.bfloat16: L.BF16,
       torch.uint8: L.U8, torch.bool: L.U8}

# Stage precision names (Plan.compute_dtype / overrides) -> MFMA mode.
# "f16x3p": f16x3 everywhere except the attention probabilities, which enter P.V as one
# fp16 plane (KF_FLASH_P16); for a GEMM stage it is f16x3.
# "f16x2": GEMMs read the activation as one fp16 plane and the weight as hi/lo planes
# (KF_MMA_F16X2); an attention stage's QKV GEMM runs f16x2 and writes split k / v^T, so
# the attention itself is f16x3 ("f16x2p": with the probabilities as one plane).
# "f16x3s": an attention stage whose QKV GEMM runs f16x3 and whose attention runs the
# single-pass fp16 kernel on the rounded-to-nearest hi planes the GEMM writes (q stays
# fp32 and is rounded in the kernel): the projections carry no h or W rounding, only the
# attention operands are 16-bit.
MODES = {"float32": L.MMA_F32, "float16": L.MMA_F16, "bfloat16": L.MMA_BF16,
         "f16x3p": L.MMA_F16X3, "f16x2": L.MMA_F16X2, "f16x2p": L.MMA_F16X2,
         "f16x3": L.MMA_F16X3, "bf16x3": L.MMA_BF16X3, "f16x3s": L.MMA_F16X3}
P16_PRECISIONS = ("f16x3p", "f16x2p")
SINGLE_ATTN_PRECISIONS = ("f16x3s",)        # split QKV GEMM, single-pass fp16 attention
SPLIT_MODES = (L.MMA_F16X3, L.MMA_BF16X3)               # activations as hi/lo planes
W_SPLIT_MODES = SPLIT_MODES + (L.MMA_F16X2,)             # weights as hi/lo planes
MODE_STORAGE = {L.MMA_F16: torch.float16, L.MMA_BF16: torch.bfloat16,
                L.MMA_F16X3: torch.float16, L.MMA_BF16X3: torch.bfloat16,
                L.MMA_F16X2: torch.float16, L.MMA_F32: torch.float32}

FLASH_HEAD_DIMS = (8, 16, 32, 64, 128, 256)
LDS_KB = 160.0   # per CU on gfx950; one block may use all of it


# ------------------------------------------------------------------ split planes
class PlanesFormat:
    """Marker passed as an `out_dtype`: produce Planes of this 16-bit type."""

    def __init__(self, dtype: torch.dtype):
        self.dtype = dtype
        self.code = L.F16X2 if dtype == torch.float16 else L.BF16X2

    def __repr__(self) -> str:
        return f"PlanesFormat({self.dtype})"


F16X2 = PlanesFormat(torch.float16)
BF16X2 = PlanesFormat(torch.bfloat16)


class Planes:
    """An fp32 tensor carried as hi + lo 16-bit planes of one shape and stride."""

    def __init__(self, hi: torch.Tensor, lo: torch.Tensor):
        assert hi.shape == lo.shape and hi.stride() == lo.stride() and hi.dtype == lo.dtype
        assert hi.dtype in (torch.float16, torch.bfloat16)
        self.hi, self.lo = hi, lo

    @staticmethod
    def empty(shape, fmt: PlanesFormat, device) -> "Planes":
        buf = torch.empty((2, *shape), dtype=fmt.dtype, device=device)
        return Planes(buf[0], buf[1])

    @staticmethod
    def from_float(x: torch.Tensor, fmt: PlanesFormat = F16X2) -> "Planes":
        buf = torch.empty((2, *x.shape), dtype=fmt.dtype, device=x.device)
        buf[0].copy_(x)
        buf[1].copy_(x - buf[0].float())
        return Planes(buf[0], buf[1])

    @property
    def code(self) -> int:
        return L.F16X2 if self.hi.dtype == torch.float16 else L.BF16X2

    @property
    def shape(self):
        return self.hi.shape

    @property
    def is_cuda(self) -> bool:
        return self.hi.is_cuda

    def stride(self, *a):
        return self.hi.stride(*a)

    def element_size(self) -> int:
        return 2 * self.hi.element_size()

    def view(self, *shape) -> "Planes":
        return Planes(self.hi.view(*shape), self.lo.view(*shape))

    def permute(self, *dims) -> "Planes":
        return Planes(self.hi.permute(*dims), self.lo.permute(*dims))

    def float(self) -> torch.Tensor:
        return self.hi.float() + self.lo.float()


Act = Union[torch.Tensor, Planes]


def _code(t) -> int:
    if isinstance(t, Planes):
        return t.code
    try:
        return _DT[t.dtype]
    except KeyError:
        raise TypeError(f"unsupported dtype {t.dtype}") from None


def _lo(t) -> Optional[int]:
    return t.lo.data_ptr() if isinstance(t, Planes) else None


def _hi(t) -> Optional[int]:
    if t is None:
        return None
    return t.hi.data_ptr() if isinstance(t, Planes) else t.data_ptr()


def _alloc(shape, fmt, device) -> Act:
    if isinstance(fmt, PlanesFormat):
        return Planes.empty(shape, fmt, device)
    return torch.empty(shape, dtype=fmt, device=device)


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def _need_cuda(*ts) -> None:
    for t in ts:
        if t is not None and not t.is_cuda:
            raise RuntimeError("libkf950 kernels need device tensors")


# ------------------------------------------------------------------ timing hook
class KernelTimer:
    """Per-launch HIP-event timing of the wrappers below, for roofline reporting.

    While `kernels.TIMER` is a KernelTimer, every wrapper records an event pair around
    its launch on the stream it launches on, tagged with a label and the launch's
    algorithmic FLOPs and bytes. `summary()` synchronises and returns, per label, the
    launch count, mean duration and achieved rates. Off (None) by default; it is not
    usable under graph capture.
    """

    def __init__(self, pad_us: float = 0.0):
        """`pad_us` > 0 queues a GPU spin of about that long before each start event, so
        the GPU is still busy while the host prepares the launch and the event pair spans
        the kernel alone (without it, a host slower than the kernels makes short kernels'
        pairs include the host's launch time). It also measures `bracket_ms`, what an
        event pair adds to the kernels it brackets (the queue's event-to-dispatch and
        completion-to-event latency): with b1 and b2 the median pair times around one and
        two empty kernels (zero-cycle spins) under the same protocol, an empty kernel costs
        b2 - b1 and the pair itself 2 b1 - b2. `summary` reports both the raw pair time and
        the pair time net of it."""
        self.records = []
        self.pad_cycles = 0
        self.bracket_ms = 0.0
        if pad_us > 0:
            probe_cycles = 200000
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            torch.cuda._sleep(probe_cycles)          # warm the spin kernel
            a.record()
            torch.cuda._sleep(probe_cycles)
            b.record()
            b.synchronize()
            per_us = probe_cycles / max(a.elapsed_time(b) * 1e3, 1e-3)
            self.pad_cycles = int(pad_us * per_us)
            def bracket(kernels: int) -> float:
                pairs = []
                for _ in range(21):
                    torch.cuda._sleep(self.pad_cycles)
                    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                    s.record()
                    for _k in range(kernels):
                        torch.cuda._sleep(0)
                    e.record()
                    pairs.append((s, e))
                torch.cuda.synchronize()
                times = sorted(s.elapsed_time(e) for s, e in pairs)
                return times[len(times) // 2]
            # one empty kernel costs b2 - b1 inside a pair; what the pair adds is the rest
            b1, b2 = bracket(1), bracket(2)
            self.bracket_ms = max(0.0, 2.0 * b1 - b2)

    def begin(self, label: str, flops: float, nbytes: float, dispatches: int = 1):
        if self.pad_cycles:
            torch.cuda._sleep(self.pad_cycles)
        s = torch.cuda.Event(enable_timing=True)
        s.record()
        return (label, flops, nbytes, dispatches, s)

    def end(self, tok) -> None:
        e = torch.cuda.Event(enable_timing=True)
        e.record()
        self.records.append((*tok, e))

    def dispatch_labels(self) -> list:
        """[label, kernel dispatches, algorithmic bytes] per wrapper call, in launch order
        (lets a profiler's per-dispatch records be attributed to labels)."""
        return [[r[0], r[3], r[2]] for r in self.records]

    def summary(self) -> dict:
        """Per label: launches, mean duration, mean algorithmic FLOPs and bytes per launch,
        and the rates of the label's total work over its total time (launches under one
        label may differ in work, e.g. the entry and final LayerNorms read one operand
        fewer or write one output fewer than the others).

        `mean_ms` and the rates use the raw event-pair time, which bounds the kernel's
        duration from above: subtracting the measured pair overhead (`bracket_ms`, the
        median over empty kernels) undercut the profiler's per-dispatch duration of short
        kernels (a 10-20 us LayerNorm by up to 2 us), so the net figure is only reported
        beside (`net_ms`), never used for a rate."""
        torch.cuda.synchronize()
        out = {}
        for label, flops, nbytes, _n, s, e in self.records:
            r = out.setdefault(label, {"launches": 0, "total_ms": 0.0, "net_total_ms": 0.0,
                                       "total_flops": 0.0, "total_bytes": 0.0})
            t = s.elapsed_time(e)
            r["launches"] += 1
            r["total_ms"] += t
            r["net_total_ms"] += max(t - self.bracket_ms, 1e-6)
            r["total_flops"] += flops or 0.0
            r["total_bytes"] += nbytes or 0.0
        for r in out.values():
            r["mean_ms"] = r["total_ms"] / r["launches"]
            r["event_ms"] = r["mean_ms"]
            r["net_ms"] = r["net_total_ms"] / r["launches"]
            r["bracket_ms"] = self.bracket_ms
            r["flops"] = r["total_flops"] / r["launches"]
            r["bytes"] = r["total_bytes"] / r["launches"]
            sec = r["total_ms"] / 1e3
            r["tflops"] = (r["total_flops"] / sec / 1e12) if r["total_flops"] else None
            r["gbs"] = (r["total_bytes"] / sec / 1e9) if r["total_bytes"] else None
        return out


TIMER: Optional[KernelTimer] = None


def _begin(label: str, flops: float, nbytes: float, dispatches: int = 1):
    return TIMER.begin(label, flops, nbytes, dispatches) if TIMER is not None else None


def _end(tok) -> None:
    if tok is not None and TIMER is not None:
        TIMER.end(tok)


# ------------------------------------------------------------------ LayerNorm
def supported(d_model: int) -> bool:
    """Every width is handled (a register fast path up to 4096, a generic path beyond)."""
    return d_model > 0


def add_mask_layernorm(x: torch.Tensor, y: Optional[torch.Tensor],
                       keep: Optional[torch.Tensor], weight: torch.Tensor,
                       bias: torch.Tensor, eps: float = 1e-5, mask_out: bool = False,
                       out_dtype=None,
                       residual_dtype: Optional[torch.dtype] = None,
                       want_residual: bool = True,
                       ) -> Tuple[Optional[torch.Tensor], Act]:
    """(s, h) with s = (x + y) * keep and h = LayerNorm(s) [* keep when mask_out].

    Signature and semantics of `kernelforge/ops/layernorm.py:101-156`. x, y: [M, d]
    (unit column stride); keep: [M] 0/1 (bool, uint8 or float) or None. `out_dtype` may
    be a torch dtype or a PlanesFormat (F16X2 / BF16X2), which returns h as Planes.
    """
    assert x.dim() == 2, "pass [M, d]"
    _need_cuda(x, y, keep, weight, bias)
    M, d = x.shape
    out_dtype = out_dtype or x.dtype
    residual_dtype = residual_dtype or x.dtype
    if x.stride(1) != 1:
        x = x.contiguous()
    if y is not None and (y.stride(1) != 1 or y.shape != x.shape):
        y = y.reshape(M, d).contiguous()
    weight = weight.contiguous()
    bias = bias.contiguous()
    if bias.dtype != weight.dtype:
        bias = bias.to(weight.dtype)
    if keep is not None:
        keep = keep.reshape(M)
        if keep.dtype == torch.bool:
            keep = keep.view(torch.uint8)
        keep = keep.contiguous()
    s = torch.empty((M, d), dtype=residual_dtype, device=x.device) if want_residual else None
    h = _alloc((M, d), out_dtype, x.device)
    flags = ((L.LN_HAS_Y if y is not None else 0) | (L.LN_HAS_MASK if keep is not None else 0)
             | (L.LN_MASK_OUT if mask_out else 0) | (L.LN_WRITE_S if want_residual else 0))
    nbytes = M * d * (x.element_size() + (y.element_size() if y is not None else 0)
                      + (s.element_size() if s is not None else 0) + h.element_size()) \
        + (M * keep.element_size() if keep is not None else 0) + 2 * d * weight.element_size()
    tok = _begin(f"add_mask_ln[{M}x{d}]", 0.0, nbytes)
    st = L.lib().kf_add_mask_ln(
        x.data_ptr(), _code(x), x.stride(0),
        _hi(y), _code(y) if y is not None else L.F32, y.stride(0) if y is not None else d,
        _hi(keep), _code(keep) if keep is not None else L.U8,
        weight.data_ptr(), bias.data_ptr(), _code(weight),
        _hi(s), _code(s) if s is not None else L.F32, s.stride(0) if s is not None else d,
        _hi(h), _lo(h), _code(h), h.stride(0),
        M, d, float(eps), flags, _stream())
    _end(tok)
    L.check("kf_add_mask_ln", st)
    return s, h


# ------------------------------------------------------------------ GEMM
def planes_format(mode: int):
    """The activation format a GEMM of `mode` reads best: its X2 planes for split modes,
    its 16-bit type for single-pass modes and f16x2, fp32 for the fp32 mode."""
    if mode == L.MMA_F16X3:
        return F16X2
    if mode == L.MMA_BF16X3:
        return BF16X2
    return MODE_STORAGE[mode]


class PreparedLinear:
    """A weight [N, K] (+ bias [N]) laid out for one MFMA mode.

    Split modes (and f16x2) keep hi and lo 16-bit planes; single-pass modes one 16-bit
    plane; the fp32 mode the fp32 weight itself. Built once per (weights, mode) -- the analog of the
    reference's fused-QKV concatenation and cast cache (`optimized.py:186-214`).
    """

    def __init__(self, weight: torch.Tensor, bias: Optional[torch.Tensor], mode: int):
        _need_cuda(weight)
        w = weight.detach().float().contiguous()
        self.N, self.K = w.shape
        self.mode = mode
        self.bias = None if bias is None else bias.detach().float().contiguous()
        if mode == L.MMA_F32:
            self.hi, self.lo = w, None
        else:
            storage = MODE_STORAGE[mode]
            self.hi = torch.empty_like(w, dtype=storage)
            self.lo = torch.empty_like(w, dtype=storage) if mode in W_SPLIT_MODES else None
            tok = _begin(f"split[{w.numel()}]", 0.0, float(w.numel() * 8))
            st = L.lib().kf_split(w.data_ptr(), w.numel(), mode, self.hi.data_ptr(),
                                  None if self.lo is None else self.lo.data_ptr(), _stream())
            _end(tok)
            L.check("kf_split", st)


def gemm_tiles() -> List[Tuple[int, dict]]:
    """Every GEMM tile id of the library (0 = automatic) with its shape
    (kf_gemm_tile_info): BM, BN, BK, LDS stages, wavefronts, LDS-DMA kernel."""
    out = []
    info = (ctypes.c_int * 6)()
    tile = 0
    while L.lib().kf_gemm_tile_info(tile, info) == L.OK:
        out.append((tile, dict(zip(("bm", "bn", "bk", "stages", "waves", "dma"), list(info)))))
        tile += 1
    return out


def linear(a: Act, w: PreparedLinear, act: int = L.ACT_NONE,
           out_dtype=torch.float32, out: Optional[Act] = None, tile: int = 0) -> Act:
    """act(a . W^T + bias) for a [M, K] (tensor or Planes, unit column stride) -> [M, N].

    `out_dtype` may be a torch dtype or a PlanesFormat; `tile` forces a GEMM tile id for
    this call (0: the library's automatic choice)."""
    assert len(a.shape) == 2 and a.shape[1] == w.K, f"shape {tuple(a.shape)} vs K={w.K}"
    _need_cuda(a)
    if isinstance(a, torch.Tensor) and a.stride(1) != 1:
        a = a.contiguous()
    M = a.shape[0]
    c = out if out is not None else _alloc((M, w.N), out_dtype, a.hi.device
                                           if isinstance(a, Planes) else a.device)
    planes = 2 if w.lo is not None else 1
    tok = _begin(f"gemm[{M}x{w.N}x{w.K}]", 2.0 * M * w.N * w.K,
                 M * w.K * a.element_size() + planes * w.N * w.K * w.hi.element_size()
                 + M * w.N * c.element_size())
    st = L.lib().kf_gemm_tiled(_hi(a), _lo(a), _code(a), a.stride(0),
                               w.hi.data_ptr(), None if w.lo is None else w.lo.data_ptr(),
                               w.hi.stride(0), None if w.bias is None else w.bias.data_ptr(),
                               _hi(c), _lo(c), _code(c), c.stride(0),
                               M, w.N, w.K, w.mode, act, tile, _stream())
    _end(tok)
    L.check("kf_gemm", st)
    return c


# ------------------------------------------------------------------ attention
def flash_supported(head_dim: int) -> bool:
    return head_dim in FLASH_HEAD_DIMS and L.available()


def mask_prep(keep: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
    """(kv_len, prefix) int32 [B] for a [B, S] validity mask (see kf_mask_prep)."""
    _need_cuda(keep)
    if keep.dtype == torch.bool:
        keep = keep.view(torch.uint8)
    if keep.stride(1) != 1:
        keep = keep.contiguous()
    B, S = keep.shape
    kv_len = torch.empty(B, dtype=torch.int32, device=keep.device)
    prefix = torch.empty(B, dtype=torch.int32, device=keep.device)
    tok = _begin(f"mask_prep[{B}x{S}]", 0.0, float(B * S))
    st = L.lib().kf_mask_prep(keep.data_ptr(), _code(keep), keep.stride(0), B, S,
                              kv_len.data_ptr(), prefix.data_ptr(), _stream())
    _end(tok)
    L.check("kf_mask_prep", st)
    return kv_len, prefix


def default_flash_mode(dtype: torch.dtype) -> int:
    if dtype == torch.float16:
        return L.MMA_F16
    if dtype == torch.bfloat16:
        return L.MMA_BF16
    return L.MMA_F16X3


def _strides4(t: Act):
    return L.strides4(t.hi if isinstance(t, Planes) else t)


class AttnOperands:
    """q, k, v in the attention layout kf_flash_fwd reads.

    q: [B, H, S, Dh] view (fp32 / fp16 / bf16); k: [B, H, S, Dh] views of 16-bit planes
    (hi, and lo for split modes); vt: [B, H, Dh, sp] views of 16-bit planes, keys
    contiguous (V transposed), sp = S rounded up to 8.
    """

    def __init__(self, q, k_hi, k_lo, vt_hi, vt_lo, mode: int):
        self.q, self.k_hi, self.k_lo, self.vt_hi, self.vt_lo, self.mode = \
            q, k_hi, k_lo, vt_hi, vt_lo, mode


    @staticmethod
    def empty_stack(B: int, S: int, H: int, Dh: int, mode: int, device) -> "AttnOperands":
        """Buffers in the layout kf_gemm_qkv writes: q and k token-major [B, S, H, Dh]."""
        planes = 2 if mode in SPLIT_MODES else 1
        dt = MODE_STORAGE[mode]
        sp = (S + 7) // 8 * 8
        q = torch.empty((B, S, H, Dh), dtype=torch.float32, device=device)
        k = torch.empty((planes, B, S, H, Dh), dtype=dt, device=device)
        vt = torch.empty((planes, B, H, Dh, sp), dtype=dt, device=device)
        if sp > S:      # kf_flash_fwd reads V^T up to sp: the pad must be finite
            vt[..., S:].zero_()
        p = lambda t: t.permute(0, 2, 1, 3)  # noqa: E731
        return AttnOperands(p(q), p(k[0]), p(k[planes - 1]) if planes == 2 else None,
                            vt[0], vt[planes - 1] if planes == 2 else None, mode)


def linear_qkv(h: Act, w: PreparedLinear, B: int, S: int, H: int, Dh: int,
               tile: int = 0, single: bool = False) -> AttnOperands:
    """Fused QKV projection straight into the attention layout (kf_gemm_qkv). An f16x2
    GEMM writes split k / v^T planes: its attention runs f16x3. `single` (an f16x3 GEMM):
    k / v^T as one fp16 plane each, the values rounded to nearest, for the single-pass fp16
    attention (the lo planes are not written)."""
    assert len(h.shape) == 2 and h.shape[1] == w.K == H * Dh and w.N == 3 * w.K
    assert not single or w.mode == L.MMA_F16X3, "single-plane k / v^T from an f16x3 GEMM"
    _need_cuda(h)
    dev = h.hi.device if isinstance(h, Planes) else h.device
    attn_mode = (L.MMA_F16 if single else
                 L.MMA_F16X3 if w.mode == L.MMA_F16X2 else w.mode)
    ops = AttnOperands.empty_stack(B, S, H, Dh, attn_mode, dev)
    sp = ops.vt_hi.shape[-1]
    M, d = B * S, H * Dh
    kv_planes = 2 if ops.k_lo is not None else 1
    tok = _begin(f"gemm_qkv[{M}x{3 * d}x{d}]", 2.0 * M * 3 * d * d,
                 M * d * h.element_size() + (2 if w.lo is not None else 1) * 3 * d * d * 2
                 + M * d * 4 + 2 * M * d * 2 * kv_planes)
    st = L.lib().kf_gemm_qkv_tiled(_hi(h), _lo(h), _code(h), h.stride(0),
                                   w.hi.data_ptr(), None if w.lo is None else w.lo.data_ptr(),
                                   w.hi.stride(0), w.bias.data_ptr(),
                                   ops.q.data_ptr(), ops.k_hi.data_ptr(), _hi(ops.k_lo),
                                   ops.vt_hi.data_ptr(), _hi(ops.vt_lo), sp, B, S, H, Dh, w.mode,
                                   tile, _stream())
    _end(tok)
    L.check("kf_gemm_qkv", st)
    return ops


def k_in_place(k: torch.Tensor, mode: int) -> bool:
    """True when k can be read by kf_flash_fwd as it is: a single-pass mode whose 16-bit
    type k already has, unit stride along Dh, other strides multiples of 8 elements and a
    16-byte aligned base (then only V needs the transposed layout)."""
    return (mode not in SPLIT_MODES and k.dtype == MODE_STORAGE.get(mode) and k.stride(-1) == 1
            and all(s % 8 == 0 for s in k.stride()[:3]) and k.data_ptr() % 16 == 0)


def attn_prep(k: Optional[torch.Tensor], v: torch.Tensor, mode: int) -> Tuple:
    """Arbitrary [B, H, S, Dh] k, v -> K planes and V^T planes (kf_attn_prep). k None:
    only V^T (the K planes come back as None)."""
    B, H, S, Dh = v.shape
    planes = 2 if mode in SPLIT_MODES else 1
    dt = MODE_STORAGE[mode]
    sp = (S + 7) // 8 * 8
    kb = None if k is None else torch.empty((planes, B, H, S, Dh), dtype=dt, device=v.device)
    vb = torch.empty((planes, B, H, Dh, sp), dtype=dt, device=v.device)
    st = L.lib().kf_attn_prep(None if k is None else k.data_ptr(),
                              None if k is None else L.strides4(k),
                              v.data_ptr(), L.strides4(v), _code(v),
                              None if kb is None else kb[0].data_ptr(),
                              kb[planes - 1].data_ptr() if kb is not None and planes == 2 else None,
                              None if kb is None else L.strides4(kb[0]), vb[0].data_ptr(),
                              vb[planes - 1].data_ptr() if planes == 2 else None,
                              L.strides4(vb[0]), B, H, S, Dh, mode, _stream())
    L.check("kf_attn_prep", st)
    if kb is None:
        return (None, None, vb[0], vb[1] if planes == 2 else None)
    return (kb[0], kb[1] if planes == 2 else None, vb[0], vb[1] if planes == 2 else None)


def flash_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                    keep: Optional[torch.Tensor] = None, causal: bool = False,
                    sm_scale: Optional[float] = None, smem_kb: float = LDS_KB,
                    block: Optional[Tuple[int, int, int, int]] = None,
                    out: Optional[Act] = None,
                    round_scores_to: Optional[torch.dtype] = None,
                    mode: Optional[int] = None,
                    kv_len: Optional[torch.Tensor] = None,
                    prefix: Optional[torch.Tensor] = None,
                    skip_pad_rows: bool = False, p16: bool = False) -> Act:
    """softmax(q k^T * sm_scale + masks) v for [B, H, S, Dh] views (unit Dh stride).

    Signature of `kernelforge/ops/flash.py:363-422`. The scale defaults to the ORIGINAL
    head_dim^-0.5 (hd 8/16 are zero-padded inside the kernel, which changes no result).
    `keep` is a [B, S] key-validity mask. `block` (BLOCK_M, BLOCK_N, wavefronts, stages)
    must be a tiling the kernel is built with for this head_dim (`legal_blocks`; None: its
    own), within `smem_kb` of LDS. `round_scores_to`
    (float16 / bfloat16, `ops/flash.py:145-157`) rounds q.k to that type, scales it and
    rounds again before the softmax, as the reference's narrow forward does; it runs the
    single-pass MFMA of that type (KF_FLASH_ROUND_SCORES).
    `mode` is the MFMA precision (default: the input's 16-bit type, f16x3 for fp32;
    there is no fp32-MFMA attention, so the fp32 mode runs f16x3). `out` may be Planes.
    `kv_len`/`prefix` (from `mask_prep`) let the kernel skip fully padded key blocks;
    they are computed here when `keep` is given and they are not. v is first put in the
    transposed attention layout (kf_attn_prep), and k too unless it already is the mode's
    16-bit type with aligned rows (`k_in_place`); the layer stack writes that layout
    directly from its QKV GEMM and calls `flash_attention_ops`.
    """
    rs_mode = {None: None, torch.float32: None, torch.float16: L.MMA_F16,
               torch.bfloat16: L.MMA_BF16}
    if round_scores_to not in rs_mode:
        raise ValueError(f"round_scores_to must be float16 or bfloat16, not {round_scores_to}")
    rs = rs_mode[round_scores_to]
    if rs is not None and mode is not None and mode != rs:
        raise ValueError("round_scores_to runs the single-pass MFMA of its own type")
    mode = rs if rs is not None else mode
    B, H, S, Dh = q.shape
    if Dh not in FLASH_HEAD_DIMS:
        raise L.UnsupportedError("flash_attention", L.EUNSUPPORTED, f"unsupported head_dim {Dh}")
    _need_cuda(q, k, v, keep, out)
    assert k.shape == q.shape and v.shape == q.shape, "q, k, v must have one shape"
    assert q.stride(-1) == 1 and k.stride(-1) == 1 and v.stride(-1) == 1, \
        "flash_attention needs unit stride along head_dim"
    assert q.dtype == k.dtype == v.dtype
    mode = default_flash_mode(q.dtype) if mode is None else mode
    if mode in (L.MMA_F32, L.MMA_F16X2):
        mode = L.MMA_F16X3
    check_block(block, S, Dh, smem_kb, mode)
    if k_in_place(k, mode):          # K read as it is; only V is transposed
        _, _, vt_hi, vt_lo = attn_prep(None, v, mode)
        k_hi, k_lo = k, None
    else:
        k_hi, k_lo, vt_hi, vt_lo = attn_prep(k, v, mode)
    ops = AttnOperands(q, k_hi, k_lo, vt_hi, vt_lo, mode)
    o = out if out is not None else torch.empty_like(q, memory_format=torch.contiguous_format)
    return flash_attention_ops(ops, keep=keep, causal=causal, sm_scale=sm_scale, out=o,
                               kv_len=kv_len, prefix=prefix, skip_pad_rows=skip_pad_rows,
                               p16=p16, round_scores=rs is not None)


def flash_attention_ops(ops: AttnOperands, keep: Optional[torch.Tensor] = None,
                        causal: bool = False, sm_scale: Optional[float] = None,
                        out: Optional[Act] = None, kv_len: Optional[torch.Tensor] = None,
                        prefix: Optional[torch.Tensor] = None,
                        skip_pad_rows: bool = False, p16: bool = False,
                        round_scores: bool = False) -> Act:
    """Attention on operands already in the attention layout (see AttnOperands).

    `p16` (f16x3 operands only, KF_FLASH_P16): the probabilities enter P.V as one fp16
    plane rounded to nearest, so P.V costs two MFMAs per tile instead of three.
    `round_scores` (fp16 / bf16 operands, KF_FLASH_ROUND_SCORES): q.k rounded to the
    operands' type, scaled, and rounded again, as the reference's narrow forward."""
    q = ops.q
    B, H, S, Dh = q.shape
    sm_scale = Dh ** -0.5 if sm_scale is None else sm_scale
    o = out if out is not None else torch.empty_like(q, memory_format=torch.contiguous_format)
    assert tuple(o.shape) == tuple(q.shape) and o.stride(-1) == 1, \
        "output needs unit stride along head_dim"
    keep_u8 = None
    if keep is not None:
        keep_u8 = keep.view(torch.uint8) if keep.dtype == torch.bool else keep
        if keep_u8.dtype not in (torch.uint8, torch.float32, torch.float16, torch.bfloat16):
            keep_u8 = (keep_u8 != 0).to(torch.uint8)
        if keep_u8.stride(1) != 1:
            keep_u8 = keep_u8.contiguous()
        if kv_len is None:
            kv_len, prefix = mask_prep(keep_u8)
    flags = ((L.FLASH_CAUSAL if causal else 0) | (L.FLASH_SKIP_PAD_ROWS if skip_pad_rows else 0)
             | (L.FLASH_P16 if p16 and ops.mode == L.MMA_F16X3 else 0)
             | (L.FLASH_ROUND_SCORES if round_scores else 0))
    # kf_flash_fwd launches the prefix-mask kernel and, when a keep mask is given, the
    # general-mask one
    n_disp = int(keep_u8 is None or (kv_len is not None and prefix is not None)) \
        + int(keep_u8 is not None)
    # algorithmic bytes: q, K and V^T read once, o written once (each plane it carries)
    nbytes = float(B * H * S * Dh) * (
        q.element_size() + ops.k_hi.element_size() * (2 if ops.k_lo is not None else 1)
        + ops.vt_hi.element_size() * (2 if ops.vt_lo is not None else 1) + o.element_size())
    tok = _begin(f"flash[B{B}H{H}S{S}d{Dh}]", 0.0, nbytes, n_disp)
    st = L.lib().kf_flash_fwd(
        q.data_ptr(), L.strides4(q), _code(q),
        ops.k_hi.data_ptr(), _hi(ops.k_lo), L.strides4(ops.k_hi),
        ops.vt_hi.data_ptr(), _hi(ops.vt_lo), L.strides4(ops.vt_hi),
        _hi(o), _lo(o), _strides4(o), _code(o),
        _hi(keep_u8), _code(keep_u8) if keep_u8 is not None else L.U8,
        keep_u8.stride(0) if keep_u8 is not None else S,
        _hi(kv_len), _hi(prefix), B, H, S, Dh, float(sm_scale), ops.mode, flags, _stream())
    _end(tok)
    L.check("kf_flash_fwd", st)
    return o


# ---------------------------------------------------------- tile legality (LDS budget)
# The reference sizes Triton tilings against NVIDIA shared memory (`kernelforge/ops/
# flash.py:277-360`: CANDIDATE_BLOCKS, smem_bytes, legal_blocks, pick_block). The gfx950
# kernel has one tiling per (head_dim, precision), set at compile time; the library
# reports it (kf_flash_tile_info), and these functions describe exactly that tiling:
# (BLOCK_M, BLOCK_N, wavefronts, LDS stages), with BLOCK_M = 16 rows x query groups per
# wavefront x wavefronts, and LDS rows of BLOCK_N keys (K) / head_dim (V^T) 16-bit values
# with no padding (XOR-swizzled chunks), hi and lo planes in the split modes.
def flash_tile(head_dim: int, mode: int = L.MMA_F16X3) -> dict:
    """The kernel's tile at this head_dim and MFMA mode (kf_flash_tile_info)."""
    info = (ctypes.c_int * 6)()
    if L.lib().kf_flash_tile_info(int(head_dim), int(mode), info) != L.OK:
        raise L.UnsupportedError("kf_flash_tile_info", L.EUNSUPPORTED,
                                 f"no flash tile for head_dim {head_dim}, mode {mode}")
    return dict(zip(("block_m", "block_n", "waves", "stages", "query_groups", "lds_bytes"),
                    list(info)))


def lds_bytes(bn: int, head_dim: int, stages: int, split: bool = True) -> int:
    """LDS of a K / V^T staging pipeline: per stage a K tile [BN][hd'] and a V^T tile
    [hd'][BN] of 16-bit values (hd' = head_dim, at least the 32-wide MFMA contraction),
    doubled for hi/lo planes. The query tile stays in registers. Head dim 8 in the split
    modes packs its products into the contraction instead (no padding to 32): hi/lo
    planes of [BN][8] and [8][BN], a 128-byte offset of the V^T lo plane and three 8-wide
    constant rows, rounded up to 128 bytes per stage."""
    if split and head_dim == 8:
        stage = 2 * 2 * (2 * bn * 8) + 128 + 3 * 8 * 2
        return stages * ((stage + 127) // 128 * 128)
    hdp = max(32, head_dim)
    return stages * (2 if split else 1) * 2 * (2 * bn * hdp)


def candidate_blocks(head_dim: int, mode: int = L.MMA_F16X3) -> Tuple[Tuple[int, int, int, int], ...]:
    """Every tiling the kernel is built with at this head_dim and mode."""
    t = flash_tile(head_dim, mode)
    return ((t["block_m"], t["block_n"], t["waves"], t["stages"]),)


def legal_blocks(seq_len: int, head_dim: int, smem_kb: float = LDS_KB,
                 mode: int = L.MMA_F16X3) -> List[Tuple[int, int, int, int]]:
    """The built tilings whose LDS fits `smem_kb` (the kernel needs its full tile; any
    sequence length is served by the same tile, with masked tails)."""
    split = mode in SPLIT_MODES
    return [b for b in candidate_blocks(head_dim, mode)
            if lds_bytes(b[1], head_dim, b[3], split) <= smem_kb * 1024]


def pick_block(seq_len: int, head_dim: int, smem_kb: float = LDS_KB, causal: bool = False,
               mode: int = L.MMA_F16X3) -> Tuple[int, int, int, int]:
    """The tiling a launch uses; raises when it does not fit the LDS budget."""
    legal = legal_blocks(seq_len, head_dim, smem_kb, mode)
    if not legal:
        raise L.UnsupportedError("pick_block", L.EUNSUPPORTED,
                                 f"head_dim {head_dim}: the kernel's tile needs more than "
                                 f"{smem_kb} KB of LDS")
    return legal[0]


def check_block(block: Optional[Tuple[int, int, int, int]], seq_len: int, head_dim: int,
                smem_kb: float = LDS_KB, mode: int = L.MMA_F16X3) -> None:
    """A plan's `flash_block` must name a tiling the kernel is built with (None: the
    kernel's own)."""
    if block is None:
        return
    legal = legal_blocks(seq_len, head_dim, smem_kb, mode)
    if tuple(block) not in legal:
        raise L.UnsupportedError("flash_block", L.EUNSUPPORTED,
                                 f"tile {tuple(block)} is not built for head_dim {head_dim} "
                                 f"(built: {legal})")
