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
scores' spread).  The backward (``swvr_bwd_fp8``) recomputes the same e4m3 scores,
so P is the forward's, and forms gh = s dS W and gW = s dS^T h from the bf16
h and W (the quantisation passes gradients through as the identity).
"""
import torch

from . import _lib
from ._ops import _grad_buffer, _kpad, _lead_stride, _matrix, _require_device

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


def _fwd(hq, hs, Wq, ws, E, bias, logit_scale):
    lib = _lib.load()
    N, Kq = hq.shape
    V, D = E.shape
    Eb = E.detach().to(torch.bfloat16)
    Eb = Eb if Eb.stride(-1) == 1 else Eb.contiguous()
    b = bias.detach().to(torch.float32).contiguous() if bias is not None else None
    O = torch.empty(N, D, dtype=torch.float32, device=hq.device)
    lse = torch.empty(N, dtype=torch.float32, device=hq.device)
    ws_bytes = lib.swvr_fwd_fp8_workspace_size(N, Kq, V, D)
    if ws_bytes == 0 and N > 0:
        raise NotImplementedError(f"swvr_amd: no e4m3 forward for D={D} (at most 128)")
    work = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=hq.device)
    lde = Eb.stride(0) if V > 1 else D
    with torch.cuda.device(hq.device):
        rc = lib.swvr_fwd_fp8(N, Kq, V, D, _lib.ptr(hq), Kq, _lib.ptr(hs), _lib.ptr(Wq), Kq, _lib.ptr(ws),
                              _lib.ptr(Eb), lde, _lib.ptr(b), float(logit_scale), _lib.ptr(O), _lib.ptr(lse),
                              _lib.ptr(work), ws_bytes, _lib.stream_of(hq.device))
    _lib.check(rc)
    return O, lse


def _bwd(gO, glse, h, W, E, bias, O, lse, hq, hs, Wq, ws, logit_scale, chunk, needs):
    """``swvr_bwd_fp8``: the scores recomputed from the forward's e4m3 operands, the gradient
    products on bf16 h and W (swvr/chunked.py:108-151 otherwise)."""
    lib = _lib.load()
    N, K = h.shape
    V, D = E.shape
    Kp = _kpad(K)
    hb = _matrix(h.detach(), torch.bfloat16, Kp)
    Wb = _matrix(W.detach(), torch.bfloat16, Kp)
    Eb = E.detach().to(torch.bfloat16)
    Eb = Eb if Eb.stride(-1) == 1 else Eb.contiguous()
    b = bias.detach().to(torch.float32).contiguous() if bias is not None else None
    need_h, need_W, need_E, need_b = needs
    dev = h.device
    gh = _grad_buffer((N, Kp), h.dtype, dev) if need_h else None
    gW = _grad_buffer((V, Kp), W.dtype, dev) if need_W else None
    gE = _grad_buffer((V, D), E.dtype, dev) if need_E else None
    gb = torch.empty(V, dtype=torch.float32, device=dev) if need_b else None
    gO32 = gO.to(torch.float32).contiguous()
    glse32 = glse.to(torch.float32).contiguous()
    Kq = hq.shape[1]
    ws_bytes = lib.swvr_bwd_fp8_workspace_size(N, Kp, Kq, V, D, int(chunk), int(need_h))
    work = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)

    def tag_of(t):
        return _lib.DTYPE_TAG[t.dtype] if t is not None else 0

    lde = Eb.stride(0) if V > 1 else D
    with torch.cuda.device(dev):
        rc = lib.swvr_bwd_fp8(N, Kp, V, D, _lib.ptr(hb), _lead_stride(hb), _lib.ptr(Wb), _lead_stride(Wb),
                              _lib.ptr(Eb), lde, _lib.ptr(b), float(logit_scale), _lib.ptr(hq), Kq, Kq,
                              _lib.ptr(hs), _lib.ptr(Wq), Kq, _lib.ptr(ws), _lib.ptr(O), _lib.ptr(lse),
                              _lib.ptr(gO32), _lib.ptr(glse32), int(chunk), _lib.ptr(gh), tag_of(gh), _lib.ptr(gW),
                              tag_of(gW), _lib.ptr(gE), tag_of(gE), _lib.ptr(gb), _lib.ptr(work), ws_bytes,
                              _lib.stream_of(dev))
    _lib.check(rc)
    if gh is not None:
        gh = gh[:, :K] if Kp != K else gh
        gh = gh.to(h.dtype) if gh.dtype != h.dtype else gh
    if gW is not None:
        gW = gW[:, :K].contiguous() if Kp != K else gW
        gW = gW.to(W.dtype) if gW.dtype != W.dtype else gW
    if gE is not None and gE.dtype != E.dtype:
        gE = gE.to(E.dtype)
    if gb is not None and gb.dtype != bias.dtype:
        gb = gb.to(bias.dtype)
    return gh, gW, gE, gb


class _Fp8Readout(torch.autograd.Function):
    """e4m3 forward; the backward recomputes the same e4m3 scores (so P is the forward's) and
    takes the gradient products on bf16 h and W, treating the quantisation as the identity."""

    @staticmethod
    def forward(ctx, h2, W, E, bias, logit_scale, chunk, hq, hs, Wq, ws):
        O, lse = _fwd(hq, hs, Wq, ws, E, bias, logit_scale)
        ctx.save_for_backward(h2, W, E, bias, O, lse, hq, hs, Wq, ws)
        ctx.args = (logit_scale, chunk)
        return O, lse

    @staticmethod
    def backward(ctx, gO, glse):
        h2, W, E, bias, O, lse, hq, hs, Wq, ws = ctx.saved_tensors
        needs = [bool(n) for n in ctx.needs_input_grad[:4]]
        needs[3] = needs[3] and bias is not None
        gO = gO if gO is not None else torch.zeros_like(O)
        glse = glse if glse is not None else torch.zeros_like(lse)
        grads = _bwd(gO, glse, h2, W, E, bias, O, lse, hq, hs, Wq, ws, *ctx.args, needs)
        return (*[g if n else None for g, n in zip(grads, needs)], None, None, None, None, None, None)


def softmax_readout_fp8(h, W, E, bias=None, *, logit_scale=1.0, w_q=None, chunk_size=None):
    """``(O, LSE)`` of ``softmax(logit_scale * h @ W.T + bias) @ E`` with h and W in e4m3.

    Shapes as ``softmax_readout``: h ``[..., K]``, W ``[V, K]``, E ``[V, D]`` (D <= 128),
    bias ``[V]``.  ``w_q`` = ``quantize_rows(W)`` reuses a quantised W across calls (W is
    then only used for its shape, and for the gradient products).  Differentiable: the
    backward recomputes the same e4m3 scores and stages ``chunk_size`` (default 8192)
    vocabulary rows of dS at a time; gh, gW, gE and gb come out in the parameters' dtypes.
    """
    from .api import _check, default_chunk_size
    _check(h, W, E, bias)
    _require_device(h)
    lead = h.shape[:-1]
    h2 = h.reshape(-1, h.shape[-1])
    V, D = E.shape
    hq, hs = quantize_tensor(h2)
    Wq, ws = w_q if w_q is not None else quantize_rows(W)
    if Wq.shape != (V, hq.shape[1]) or Wq.dtype != E4M3 or ws.shape != (V,) or Wq.device != h.device:
        raise ValueError(f"w_q must be quantize_rows(W) of a [{V}, {W.shape[1]}] W on {h.device}")
    # the kernels read dense rows of Kp bytes and fp32 scales
    Wq = Wq.contiguous()
    ws = ws.to(device=h.device, dtype=torch.float32).contiguous()
    chunk = int(chunk_size) if chunk_size else default_chunk_size()
    if chunk <= 0:
        raise ValueError(f"chunk_size must be positive, got {chunk}")
    if torch.is_grad_enabled() and any(t is not None and t.requires_grad for t in (h, W, E, bias)):
        O, lse = _Fp8Readout.apply(h2, W, E, bias, float(logit_scale), chunk, hq, hs, Wq, ws)
    else:
        O, lse = _fwd(hq, hs, Wq, ws, E, bias, logit_scale)
    return O.view(*lead, D), lse.view(lead)


def softmax_readout_mse_fp8(h, W, E, target, bias=None, *, weight=None, reduction="mean", z_loss_weight=0.0,
                            logit_scale=1.0, chunk_size=None, w_q=None):
    """``softmax_readout_mse`` over the e4m3 readout: the same loss (swvr/api.py:53-66) on the
    O and LSE of ``softmax_readout_fp8``."""
    from .api import _mse_loss
    O, lse = softmax_readout_fp8(h, W, E, bias, logit_scale=logit_scale, w_q=w_q, chunk_size=chunk_size)
    return _mse_loss(O, lse, target, weight, reduction, z_loss_weight)
