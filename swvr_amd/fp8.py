"""Opt-in e4m3 (fp8) forward of the readout: h and W stream as OCP e4m3.

The reference has no fp8 path (its precision policy is swvr/chunked.py:7-9:
scores in fp32 from compute-dtype operands).  This module adds one for
inference and evaluation, outside that policy and with its own tolerance:

* W is quantised per vocabulary row, ``W[v] ~ w_scale[v] * W_e4m3[v]``, and h
  per tensor, ``h ~ h_scale * h_e4m3``, each scale = amax / 448 (the largest
  finite e4m3 value), rounding to nearest even (bit-identical to torch's
  ``float8_e4m3fn`` cast of ``x / scale``; ``swvr_quantize_e4m3``);
* the scores ``S = logit_scale * h_scale * w_scale[v] * (h_e4m3 . W_e4m3[v]) + b``
  accumulate in fp32 on gfx950's k64 e4m3 matrix instruction, at twice the bf16
  rate; P is rounded to bf16 for ``P @ E`` as in the bf16 forward; O and LSE
  are fp32.

Given the quantised operands, the result matches the fp64 readout of the
dequantised h and W to the bf16 forward's tolerance; against the unquantised
inputs the e4m3 rounding of h and W adds its own error (a few per cent of the
scores' spread).  There is no fp8 backward: train with ``softmax_readout``.
"""
import torch

from . import _lib
from ._ops import _require_device

E4M3 = torch.float8_e4m3fn
E4M3_MAX = 448.0


def _quantize(x, per_row):
    """``swvr_quantize_e4m3`` of a [R, K] matrix: (e4m3 [R, Kp], fp32 scales), Kp = K padded to 16."""
    _require_device(x)
    lib = _lib.load()
    x = x.detach()
    if x.dtype not in _lib.DTYPE_TAG:
        x = x.to(torch.float32)
    if x.stride(-1) != 1:
        x = x.contiguous()
    R, K = x.shape
    Kp = (K + 15) // 16 * 16
    out = torch.empty(R, Kp, dtype=E4M3, device=x.device)
    scale = torch.empty(R if per_row else 1, dtype=torch.float32, device=x.device)
    ws_bytes = lib.swvr_quantize_e4m3_workspace_size(R, int(per_row))
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=x.device)
    ld = x.stride(0) if R > 1 else K
    with torch.cuda.device(x.device):
        rc = lib.swvr_quantize_e4m3(R, K, Kp, _lib.ptr(x), ld, _lib.DTYPE_TAG[x.dtype], int(per_row), _lib.ptr(out),
                                    Kp, _lib.ptr(scale), _lib.ptr(ws), ws_bytes, _lib.stream_of(x.device))
    _lib.check(rc)
    return out, scale


def quantize_rows(W):
    """``(W_e4m3 [V, Kp], w_scale [V] fp32)`` with one scale per row, ``max(amax, 1e-30) / 448``
    (Kp: K padded to 16 with zero bytes)."""
    return _quantize(W, True)


def quantize_tensor(h):
    """``(h_e4m3 [N, Kp], h_scale [1] fp32)`` with one scale for the whole matrix."""
    return _quantize(h, False)


def dequantize(q, scale):
    """fp32 values the e4m3 forward computes with."""
    return q.to(torch.float32) * (scale[:, None] if scale.numel() > 1 else scale)


def softmax_readout_fp8(h, W, E, bias=None, *, logit_scale=1.0, w_q=None):
    """``(O, LSE)`` of ``softmax(logit_scale * h @ W.T + bias) @ E`` with h and W in e4m3.

    Shapes as ``softmax_readout``: h ``[..., K]``, W ``[V, K]``, E ``[V, D]`` (D <= 128),
    bias ``[V]``.  ``w_q`` = ``quantize_rows(W)`` reuses a quantised W across calls (W is
    then only used for its shape).  Forward only: raises if autograd would need gradients.
    """
    from .api import _check
    _check(h, W, E, bias)
    _require_device(h)
    if torch.is_grad_enabled() and any(
            t is not None and t.requires_grad for t in (h, W, E, bias)):
        raise RuntimeError("softmax_readout_fp8 is forward only; use softmax_readout to train")
    lib = _lib.load()
    lead = h.shape[:-1]
    h2 = h.reshape(-1, h.shape[-1])
    N = h2.shape[0]
    V, D = E.shape
    hq, hs = quantize_tensor(h2)
    Wq, ws = w_q if w_q is not None else quantize_rows(W)
    if Wq.shape != (V, hq.shape[1]) or Wq.dtype != E4M3 or ws.shape != (V,):
        raise ValueError(f"w_q must be quantize_rows(W) of a [{V}, {W.shape[1]}] W")
    Kp = hq.shape[1]
    Eb = E.to(torch.bfloat16)
    Eb = Eb if Eb.stride(-1) == 1 else Eb.contiguous()
    b = bias.to(torch.float32).contiguous() if bias is not None else None
    O = torch.empty(N, D, dtype=torch.float32, device=h.device)
    lse = torch.empty(N, dtype=torch.float32, device=h.device)
    ws_bytes = lib.swvr_fwd_fp8_workspace_size(N, Kp, V, D)
    if ws_bytes == 0 and N > 0:
        raise NotImplementedError(f"swvr_amd: no e4m3 forward for D={D} (at most 128)")
    work = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=h.device)
    lde = Eb.stride(0) if V > 1 else D
    with torch.cuda.device(h.device):
        rc = lib.swvr_fwd_fp8(N, Kp, V, D, _lib.ptr(hq), Kp, _lib.ptr(hs), _lib.ptr(Wq), Kp, _lib.ptr(ws),
                              _lib.ptr(Eb), lde, _lib.ptr(b), float(logit_scale), _lib.ptr(O), _lib.ptr(lse),
                              _lib.ptr(work), ws_bytes, _lib.stream_of(h.device))
    _lib.check(rc)
    return O.view(*lead, D), lse.view(lead)
