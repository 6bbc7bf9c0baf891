"""Op boundary: the ``swvr::chunked_fwd`` / ``swvr::chunked_bwd`` custom ops.

Mirrors swvr/chunked.py:154-212 of the reference: the forward and backward
are opaque torch.library custom ops (so torch.compile keeps them whole), with
fake implementations for tracing and autograd wired through
``register_autograd``.  Their bodies call the HIP kernels through the C ABI
(include/swvr.h) on the current stream; there is no other implementation.

The schemas are the reference's (chunked.py:157-161, 170-174), ``use_triton``
flag included, so graphs and callers written against them keep working.  The
flag chose between the reference's Triton and torch elementwise paths; here
both are the same HIP kernels, so it is accepted and has no effect.
"""
from typing import List, Optional, Tuple

import torch
import torch.nn.functional as F

from . import _lib

DEFAULT_CHUNK = 8192


def acc_dtype(cdt):
    """Accumulation / output dtype (swvr/chunked.py:26-27): fp64 for an fp64 compute dtype, else fp32."""
    return torch.float64 if cdt == torch.float64 else torch.float32


def _require_device(t):
    if t.device.type != "cuda":
        raise RuntimeError(
            f"swvr_amd runs on AMD GPUs through HIP; got a tensor on {t.device}. "
            "Move h, W, E and bias to the GPU.")


def _kpad(K):
    return (K + 7) // 8 * 8


def _matrix(x, cdt, Kp):
    """``x`` [R, K] in the compute dtype with K padded to Kp, unit inner stride,
    16-byte aligned rows (the C ABI's alignment contract)."""
    if x.dtype != cdt:
        x = x.to(cdt)
    if x.shape[1] != Kp:
        x = F.pad(x, (0, Kp - x.shape[1]))
    if x.stride(1) != 1 or (x.shape[0] > 1 and x.stride(0) % 8 != 0) or x.data_ptr() % 16 != 0:
        x = x.contiguous()
        if x.data_ptr() % 16 != 0:
            x = x.clone()
    return x


def _operand(x, cdt, Kp):
    """``(tensor, dtype tag)`` of h or W for the C ABI: an fp32 matrix under a 2-byte compute
    dtype (autocast with fp32 weights) goes as it is, and the kernels round it while packing;
    anything else goes through ``_matrix``."""
    if (x.dtype == torch.float32 and cdt in (torch.bfloat16, torch.float16) and x.shape[1] == Kp
            and x.stride(1) == 1 and (x.shape[0] <= 1 or x.stride(0) % 8 == 0) and x.data_ptr() % 16 == 0):
        return x, _lib.F32
    return _matrix(x, cdt, Kp), _lib.DTYPE_TAG[cdt]


def _embed(E, cdt):
    if E.dtype != cdt:
        E = E.to(cdt)
    return E if E.stride(1) == 1 else E.contiguous()


def _lead_stride(x):
    if x.shape[1] == 0:  # empty rows (K = 0 or D = 0): any stride, 0 satisfies the ABI
        return 0
    return x.stride(0) if x.shape[0] > 1 else x.shape[1]


def _f64(x):
    """``x`` in fp64 with unit stride in its last dimension (or None)."""
    if x is None:
        return None
    x = x.to(torch.float64)
    return x if x.dim() < 2 or x.stride(-1) == 1 else x.contiguous()


def _forward_f64(h, W, E, bias, logit_scale, chunk):
    """fp64 readout (swvr_fwd_f64): fp64 O and lse, as the reference returns for fp64 inputs."""
    lib = _lib.load()
    hd, Wd, Ed, bd = _f64(h), _f64(W), _f64(E), _f64(bias)
    N, K = hd.shape
    V, D = Ed.shape
    O = torch.empty(N, D, dtype=torch.float64, device=h.device)
    lse = torch.empty(N, dtype=torch.float64, device=h.device)
    ws_bytes = lib.swvr_fwd_f64_workspace_size(N, V, D, int(chunk))
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=h.device)
    with torch.cuda.device(h.device):
        rc = lib.swvr_fwd_f64(N, K, V, D, _lib.ptr(hd), _lead_stride(hd), _lib.ptr(Wd), _lead_stride(Wd),
                              _lib.ptr(Ed), _lead_stride(Ed), _lib.ptr(bd), float(logit_scale), int(chunk),
                              _lib.ptr(O), _lib.ptr(lse), _lib.ptr(ws), ws_bytes, _lib.stream_of(h.device))
    _lib.check(rc)
    return O, lse


def _backward_f64(gO, glse, h, W, E, bias, O, lse, logit_scale, chunk, need_h, need_W, need_E, need_b):
    lib = _lib.load()
    hd, Wd, Ed, bd = _f64(h), _f64(W), _f64(E), _f64(bias)
    N, K = hd.shape
    V, D = Ed.shape
    dev = h.device
    f64 = torch.float64
    gh = torch.empty(N, K, dtype=f64, device=dev) if need_h else None
    gW = torch.empty(V, K, dtype=f64, device=dev) if need_W else None
    gE = torch.empty(V, D, dtype=f64, device=dev) if need_E else None
    gb = torch.empty(V, dtype=f64, device=dev) if need_b else None
    gOd, glsed = gO.to(f64).contiguous(), glse.to(f64).contiguous()
    Od, lsed = O.to(f64).contiguous(), lse.to(f64).contiguous()
    ws_bytes = lib.swvr_bwd_f64_workspace_size(N, V, D, int(chunk))
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)
    with torch.cuda.device(dev):
        rc = lib.swvr_bwd_f64(N, K, V, D, _lib.ptr(hd), _lead_stride(hd), _lib.ptr(Wd), _lead_stride(Wd),
                              _lib.ptr(Ed), _lead_stride(Ed), _lib.ptr(bd), float(logit_scale), _lib.ptr(Od),
                              _lib.ptr(lsed), _lib.ptr(gOd), _lib.ptr(glsed), int(chunk), _lib.ptr(gh), _lib.ptr(gW),
                              _lib.ptr(gE), _lib.ptr(gb), _lib.ptr(ws), ws_bytes, _lib.stream_of(dev))
    _lib.check(rc)
    # gradients in the parameters' own dtypes (the reference's gH.to(h.dtype), empty_like(W), ...)
    cast = lambda g, x: g.to(x.dtype) if g is not None and g.dtype != x.dtype else g
    return cast(gh, h), cast(gW, W), cast(gE, E), cast(gb, bias)


def _forward(h, W, E, bias, logit_scale, chunk, cdt):
    _require_device(h)
    if cdt == torch.float64:
        return _forward_f64(h, W, E, bias, logit_scale, chunk)
    lib = _lib.load()
    if cdt not in _lib.DTYPE_TAG:
        raise NotImplementedError(f"swvr_amd: compute dtype {cdt} is not supported (bf16, fp16, fp32, fp64)")
    N, K = h.shape
    V, D = E.shape
    Kp = _kpad(K)
    (hc, h_tag), (Wc, w_tag), Ec = _operand(h, cdt, Kp), _operand(W, cdt, Kp), _embed(E, cdt)
    b = bias.to(torch.float32).contiguous() if bias is not None else None
    O = torch.empty(N, D, dtype=torch.float32, device=h.device)
    lse = torch.empty(N, dtype=torch.float32, device=h.device)
    tag = _lib.DTYPE_TAG[cdt]
    ws_bytes = lib.swvr_fwd_workspace_size(tag, N, Kp, V, D)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=h.device)
    with torch.cuda.device(h.device):
        rc = lib.swvr_fwd_mixed(tag, h_tag, w_tag, N, Kp, V, D, _lib.ptr(hc), _lead_stride(hc), _lib.ptr(Wc),
                                _lead_stride(Wc), _lib.ptr(Ec), _lead_stride(Ec), _lib.ptr(b), float(logit_scale),
                                _lib.ptr(O), _lib.ptr(lse), _lib.ptr(ws), ws_bytes, _lib.stream_of(h.device))
    _lib.check(rc)
    return O, lse


def _forward_active(h, W, E, bias, weight, logit_scale, chunk, cdt):
    """Readout of the tokens with a non-zero weight (swvr_fwd_active): O rows and lse of the
    other tokens are 0, which leaves a weighted loss unchanged (their terms are weight x finite)."""
    _require_device(h)
    lib = _lib.load()
    if cdt not in _lib.DTYPE_TAG:
        raise NotImplementedError(f"swvr_amd: compute dtype {cdt} has no active-token forward")
    N, K = h.shape
    V, D = E.shape
    Kp = _kpad(K)
    (hc, h_tag), (Wc, w_tag), Ec = _operand(h, cdt, Kp), _operand(W, cdt, Kp), _embed(E, cdt)
    b = bias.to(torch.float32).contiguous() if bias is not None else None
    w = weight.reshape(-1).to(torch.float32).contiguous()
    O = torch.empty(N, D, dtype=torch.float32, device=h.device)
    lse = torch.empty(N, dtype=torch.float32, device=h.device)
    tag = _lib.DTYPE_TAG[cdt]
    ws_bytes = lib.swvr_fwd_active_workspace_size(tag, N, Kp, V, D)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=h.device)
    with torch.cuda.device(h.device):
        rc = lib.swvr_fwd_active(tag, h_tag, w_tag, N, Kp, V, D, _lib.ptr(hc), _lead_stride(hc), _lib.ptr(Wc),
                                 _lead_stride(Wc), _lib.ptr(Ec), _lead_stride(Ec), _lib.ptr(b), float(logit_scale),
                                 _lib.ptr(w), _lib.ptr(O), _lib.ptr(lse), _lib.ptr(ws), ws_bytes,
                                 _lib.stream_of(h.device))
    _lib.check(rc)
    return O, lse


def _grad_buffer(shape, want, device):
    """Buffer the kernels write a gradient into: the parameter's own dtype when
    the ABI has a tag for it, else fp32 (cast afterwards)."""
    dt = want if want in _lib.DTYPE_TAG else torch.float32
    return torch.empty(shape, dtype=dt, device=device)


def _backward(gO, glse, h, W, E, bias, O, lse, logit_scale, chunk, cdt, need_h, need_W, need_E, need_b):
    _require_device(h)
    if cdt == torch.float64:
        return _backward_f64(gO, glse, h, W, E, bias, O, lse, logit_scale, chunk, need_h, need_W, need_E, need_b)
    lib = _lib.load()
    N, K = h.shape
    V, D = E.shape
    Kp = _kpad(K)
    (hc, h_tag), (Wc, w_tag), Ec = _operand(h, cdt, Kp), _operand(W, cdt, Kp), _embed(E, cdt)
    b = bias.to(torch.float32).contiguous() if bias is not None else None
    dev = h.device
    gh = _grad_buffer((N, Kp), h.dtype, dev) if need_h else None
    gW = _grad_buffer((V, Kp), W.dtype, dev) if need_W else None
    gE = _grad_buffer((V, D), E.dtype, dev) if need_E else None
    gb = torch.empty(V, dtype=torch.float32, device=dev) if need_b else None
    gO32 = gO.to(torch.float32).contiguous()
    glse32 = glse.to(torch.float32).contiguous()
    O32 = O.to(torch.float32).contiguous()
    lse32 = lse.to(torch.float32).contiguous()
    tag = _lib.DTYPE_TAG[cdt]
    ws_bytes = lib.swvr_bwd_workspace_size_mixed(tag, w_tag, N, Kp, V, D, int(chunk), int(need_h))
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)

    def tag_of(t):
        return _lib.DTYPE_TAG[t.dtype] if t is not None else 0

    with torch.cuda.device(dev):
        rc = lib.swvr_bwd_mixed(tag, h_tag, w_tag, N, Kp, V, D, _lib.ptr(hc), _lead_stride(hc), _lib.ptr(Wc),
                                _lead_stride(Wc), _lib.ptr(Ec), _lead_stride(Ec), _lib.ptr(b), float(logit_scale),
                                _lib.ptr(O32), _lib.ptr(lse32), _lib.ptr(gO32), _lib.ptr(glse32), int(chunk),
                                _lib.ptr(gh), tag_of(gh), _lib.ptr(gW), tag_of(gW), _lib.ptr(gE), tag_of(gE),
                                _lib.ptr(gb), _lib.ptr(ws), ws_bytes, _lib.stream_of(dev))
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


@torch.library.custom_op("swvr::chunked_fwd", mutates_args=())
def _fwd_op(h: torch.Tensor, W: torch.Tensor, E: torch.Tensor, bias: Optional[torch.Tensor],
            logit_scale: float, chunk: int, cdt: torch.dtype,
            use_triton: bool) -> Tuple[torch.Tensor, torch.Tensor]:
    return _forward(h, W, E, bias, logit_scale, chunk, cdt)


@_fwd_op.register_fake
def _(h, W, E, bias, logit_scale, chunk, cdt, use_triton):
    adt = acc_dtype(cdt)
    return h.new_empty(h.shape[0], E.shape[1], dtype=adt), h.new_empty(h.shape[0], dtype=adt)


@torch.library.custom_op("swvr::chunked_bwd", mutates_args=())
def _bwd_op(gO: torch.Tensor, glse: torch.Tensor, h: torch.Tensor, W: torch.Tensor, E: torch.Tensor,
            bias: Optional[torch.Tensor], O: torch.Tensor, lse: torch.Tensor, logit_scale: float,
            chunk: int, cdt: torch.dtype, use_triton: bool, need_h: bool, need_W: bool, need_E: bool,
            need_b: bool) -> List[torch.Tensor]:
    grads = _backward(gO, glse, h, W, E, bias, O, lse, logit_scale, chunk, cdt,
                      need_h, need_W, need_E, need_b)
    # a custom op cannot return None: an empty tensor stands for "no gradient"
    return [g if g is not None else h.new_empty(0) for g in grads]


@_bwd_op.register_fake
def _(gO, glse, h, W, E, bias, O, lse, logit_scale, chunk, cdt, use_triton, need_h, need_W, need_E, need_b):
    like = [(need_h, h), (need_W, W), (need_E, E), (need_b, bias)]
    return [torch.empty_like(x) if need else h.new_empty(0) for need, x in like]


def _setup_context(ctx, inputs, output):
    h, W, E, bias, logit_scale, chunk, cdt, use_triton = inputs
    O, lse = output
    ctx.save_for_backward(h, W, E, bias, O, lse)
    ctx.args = (logit_scale, chunk, cdt, use_triton)


def _autograd_backward(ctx, gO, glse):
    h, W, E, bias, O, lse = ctx.saved_tensors
    needs = [bool(n) for n in ctx.needs_input_grad[:4]]
    needs[3] = needs[3] and bias is not None
    gO = gO if gO is not None else torch.zeros_like(O)
    glse = glse if glse is not None else torch.zeros_like(lse)
    grads = _bwd_op(gO, glse, h, W, E, bias, O, lse, *ctx.args, *needs)
    return (*[g if need else None for g, need in zip(grads, needs)], None, None, None, None)


_fwd_op.register_autograd(_autograd_backward, setup_context=_setup_context)


@torch.library.custom_op("swvr::chunked_fwd_active", mutates_args=())
def _fwd_active_op(h: torch.Tensor, W: torch.Tensor, E: torch.Tensor, bias: Optional[torch.Tensor],
                   weight: torch.Tensor, logit_scale: float, chunk: int,
                   cdt: torch.dtype) -> Tuple[torch.Tensor, torch.Tensor]:
    return _forward_active(h, W, E, bias, weight, logit_scale, chunk, cdt)


@_fwd_active_op.register_fake
def _(h, W, E, bias, weight, logit_scale, chunk, cdt):
    return h.new_empty(h.shape[0], E.shape[1], dtype=torch.float32), h.new_empty(h.shape[0], dtype=torch.float32)


def _setup_context_active(ctx, inputs, output):
    h, W, E, bias, weight, logit_scale, chunk, cdt = inputs
    _setup_context(ctx, (h, W, E, bias, logit_scale, chunk, cdt, True), output)


def _autograd_backward_active(ctx, gO, glse):
    gh, gW, gE, gb, *_ = _autograd_backward(ctx, gO, glse)
    return gh, gW, gE, gb, None, None, None, None


_fwd_active_op.register_autograd(_autograd_backward_active, setup_context=_setup_context_active)


def softmax_readout_op(h2, W, E, bias, logit_scale, chunk, cdt):
    """``h2`` is ``[N, K]``; returns ``(O [N, D], LSE [N])`` in fp32 (swvr/chunked.py:208-212)."""
    if h2.device.type not in ("cuda", "cpu"):  # meta / fake tracing: no autocast state
        return _fwd_op(h2, W, E, bias, float(logit_scale), int(chunk), cdt, True)
    with torch.autocast(h2.device.type, enabled=False):
        return _fwd_op(h2, W, E, bias, float(logit_scale), int(chunk), cdt, True)


def softmax_readout_active_op(h2, W, E, bias, weight, logit_scale, chunk, cdt):
    """``softmax_readout_op`` for a weighted loss: tokens with ``weight == 0`` get O rows and lse
    of 0 instead of their readout (``swvr_fwd_active``); ``weight`` is [N], no gradient."""
    if h2.device.type not in ("cuda", "cpu"):
        return _fwd_active_op(h2, W, E, bias, weight, float(logit_scale), int(chunk), cdt)
    with torch.autocast(h2.device.type, enabled=False):
        return _fwd_active_op(h2, W, E, bias, weight, float(logit_scale), int(chunk), cdt)


# ---------------------------------------------------------------- fused MSE loss
REDUCTIONS = {"none": 0, "sum": 1, "mean": 2}


def _mse_loss(O, lse, target, weight, z, reduction, need_grad):
    """Loss of swvr/api.py:53-66 over ``O`` [N, D] and ``lse`` [N] in one library call
    (``swvr_mse_loss``): the output, the factor c of the reduction, and the loss's
    derivatives divided by c (empty tensors when ``need_grad`` is false)."""
    _require_device(O)
    lib = _lib.load()
    N, D = O.shape
    O = O.contiguous()
    lse = lse.contiguous()
    t = target if target.dtype in _lib.DTYPE_TAG else target.to(torch.float32)
    if t.stride(1) != 1 or (N > 1 and t.stride(0) < D):
        t = t.contiguous()
    w = weight.to(torch.float32).contiguous() if weight is not None else None
    dev = O.device
    out = torch.empty((N,) if reduction == 0 else (), dtype=torch.float32, device=dev)
    scale = torch.empty((), dtype=torch.float32, device=dev)
    gO = torch.empty_like(O) if need_grad else O.new_empty(0)
    glse = torch.empty_like(lse) if need_grad else lse.new_empty(0)
    ws_bytes = lib.swvr_mse_loss_workspace_size(N) if reduction else 0
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)
    with torch.cuda.device(dev):
        rc = lib.swvr_mse_loss(N, D, _lib.ptr(O), _lib.ptr(lse), _lib.ptr(t), _lib.DTYPE_TAG[t.dtype],
                               t.stride(0) if N > 1 else D, _lib.ptr(w), float(z), int(reduction),
                               _lib.ptr(out), _lib.ptr(scale) if reduction else None,
                               _lib.ptr(gO) if need_grad else None, _lib.ptr(glse) if need_grad else None,
                               _lib.ptr(ws), ws_bytes, _lib.stream_of(dev))
    _lib.check(rc)
    if not reduction:
        scale.fill_(1.0)
    return out, scale, gO, glse


@torch.library.custom_op("swvr::mse_loss", mutates_args=())
def _mse_op(O: torch.Tensor, lse: torch.Tensor, target: torch.Tensor, weight: Optional[torch.Tensor],
            z: float, reduction: int, need_grad: bool) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor,
                                                                torch.Tensor]:
    return _mse_loss(O, lse, target, weight, z, reduction, need_grad)


@_mse_op.register_fake
def _(O, lse, target, weight, z, reduction, need_grad):
    N = O.shape[0]
    out = O.new_empty((N,) if reduction == 0 else ())
    gO = O.new_empty(O.shape) if need_grad else O.new_empty(0)
    glse = lse.new_empty(lse.shape) if need_grad else lse.new_empty(0)
    return out, O.new_empty(()), gO, glse


def _mse_setup_context(ctx, inputs, output):
    reduction = inputs[5]
    _, scale, gO, glse = output
    ctx.mark_non_differentiable(scale, gO, glse)
    ctx.save_for_backward(scale, gO, glse)
    ctx.reduction = reduction


def _mse_autograd_backward(ctx, g, _g_scale, _g_gO, _g_glse):
    scale, gO, glse = ctx.saved_tensors
    if ctx.reduction == 0:
        return gO * g[:, None], glse * g, None, None, None, None, None
    s = g * scale
    return gO * s, glse * s, None, None, None, None, None


_mse_op.register_autograd(_mse_autograd_backward, setup_context=_mse_setup_context)


def mse_loss_op(O2, lse, target2, weight, z_loss_weight, reduction):
    """Fused loss over ``O2`` [N, D] and ``lse`` [N] (swvr/api.py:53-66); ``reduction`` is
    "none", "sum" or "mean".  Returns the loss ([N] for "none", else a scalar)."""
    need_grad = torch.is_grad_enabled() and (O2.requires_grad or lse.requires_grad)
    out, _, _, _ = _mse_op(O2, lse, target2, weight, float(z_loss_weight), REDUCTIONS[reduction], need_grad)
    return out
