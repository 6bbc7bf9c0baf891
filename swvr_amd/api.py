"""The package's public functions, with the reference's signatures and errors (swvr/api.py:1-93).

Callers see the same argument shapes, output dtypes, ValueError messages, loss
reductions and module wrapper as the reference; underneath, every call goes to
the gfx950 HIP library through the ``swvr::chunked_fwd`` / ``swvr::chunked_bwd``
custom ops (and ``swvr::mse_loss`` for the loss when it applies).
"""
import os

import torch
from torch import nn

from ._ops import DEFAULT_CHUNK, REDUCTIONS, mse_loss_op, softmax_readout_active_op, softmax_readout_op


def default_chunk_size():
    """Vocabulary rows staged per step of the backward: ``SWVR_CHUNK`` if set, else 8192
    (swvr/chunked.py:57-59)."""
    raw = os.environ.get("SWVR_CHUNK")
    return int(raw) if raw else DEFAULT_CHUNK


def _compute_dtype(h, W):
    """dtype the products run in: autocast's if it is active on h's device, otherwise the type
    promotion of h and W (swvr/api.py:8-11)."""
    if h.device.type in ("cuda", "cpu") and torch.is_autocast_enabled(h.device.type):
        return torch.get_autocast_dtype(h.device.type)
    return torch.promote_types(h.dtype, W.dtype)


def _check(h, W, E, bias):
    """Raise ValueError for inconsistent shapes; the messages are the reference's, word for word,
    since callers may match on them (swvr/api.py:14-22)."""
    if W.dim() != 2 or E.dim() != 2:
        raise ValueError(f"W and E must be 2-D, got {tuple(W.shape)} and {tuple(E.shape)}")
    if h.shape[-1] != W.shape[1]:
        raise ValueError(f"h has hidden size {h.shape[-1]} but W is {tuple(W.shape)}")
    if E.shape[0] != W.shape[0]:
        raise ValueError(f"W has {W.shape[0]} vocabulary rows but E has {E.shape[0]}")
    if bias is not None and bias.shape != (W.shape[0],):
        raise ValueError(f"bias must have shape ({W.shape[0]},), got {tuple(bias.shape)}")


def softmax_readout(h, W, E, bias=None, *, logit_scale=1.0, chunk_size=None):
    """Softmax-weighted readout of the embedding table (swvr/api.py:25-41).

    With scores ``S = logit_scale * h W^T + bias`` over the V vocabulary rows, returns the
    probability-weighted mix of E's rows, ``O = softmax(S) E`` (shape ``h.shape[:-1] + (D,)``),
    and the log-normaliser ``LSE = logsumexp(S)`` (shape ``h.shape[:-1]``).  Inputs:
    h ``[..., K]``, W ``[V, K]``, E ``[V, D]``, optional bias ``[V]``.  O and LSE are fp32,
    or fp64 when the products run in fp64.  The [tokens, V] scores never exist in memory;
    the backward recomputes them ``chunk_size`` rows of the vocabulary at a time (default
    8192, or ``SWVR_CHUNK``), which bounds its extra memory by O(tokens * chunk_size).
    Autograd reaches every input that requires a gradient.
    """
    _check(h, W, E, bias)
    lead = h.shape[:-1]
    h2 = h.reshape(-1, h.shape[-1])
    chunk = int(chunk_size) if chunk_size else default_chunk_size()
    if chunk <= 0:
        raise ValueError(f"chunk_size must be positive, got {chunk}")
    O, lse = softmax_readout_op(h2, W, E, bias, logit_scale, chunk, _compute_dtype(h, W))
    return O.view(*lead, E.shape[1]), lse.view(lead)


def softmax_readout_mse(h, W, E, target, bias=None, *, weight=None, reduction="mean",
                        z_loss_weight=0.0, logit_scale=1.0, chunk_size=None):
    """Squared-error loss of the readout against ``target`` (``[..., D]``) (swvr/api.py:44-66).

    Each token contributes the mean over D of ``(O - target)^2``, plus ``z_loss_weight``
    times ``LSE^2`` to keep the log-normaliser small.  An optional per-token ``weight``
    multiplies each contribution (a zero drops the token).  ``reduction``: "mean" (the
    weighted sum over the sum of the weights, or over the token count without weights),
    "sum", or "none" (the per-token values).
    """
    if _skips_zero_weight(h, W, weight, reduction):
        # The loss is weight x (a finite term) per token, so zero-weight tokens need no readout:
        # the library computes the others only and gives these O rows and lse of 0, for which
        # the term is finite again (swvr_fwd_active lists the rows it still computes to keep
        # the reference's NaNs).
        _check(h, W, E, bias)
        lead = h.shape[:-1]
        chunk = int(chunk_size) if chunk_size else default_chunk_size()
        if chunk <= 0:
            raise ValueError(f"chunk_size must be positive, got {chunk}")
        O, lse = softmax_readout_active_op(h.reshape(-1, h.shape[-1]), W, E, bias, weight.reshape(-1),
                                           logit_scale, chunk, _compute_dtype(h, W))
        O, lse = O.view(*lead, E.shape[1]), lse.view(lead)
    else:
        O, lse = softmax_readout(h, W, E, bias, logit_scale=logit_scale, chunk_size=chunk_size)
    return _mse_loss(O, lse, target, weight, reduction, z_loss_weight)


def _skips_zero_weight(h, W, weight, reduction):
    """Whether the loss's readout may leave out zero-weight tokens: a per-token weight of exactly
    the token shape on h's GPU, with no gradient of its own (its gradient would be each token's
    loss), a known reduction, and a compute dtype the library's forward runs in."""
    if not isinstance(weight, torch.Tensor) or not isinstance(h, torch.Tensor) or reduction not in REDUCTIONS:
        return False
    if h.device.type != "cuda" or weight.device != h.device or weight.shape != h.shape[:-1]:
        return False
    if weight.requires_grad or weight.is_complex() or h.shape[-1] != W.shape[-1] or W.dim() != 2:
        return False
    return _compute_dtype(h, W) in (torch.bfloat16, torch.float16, torch.float32)


def _mse_loss(O, lse, target, weight, reduction, z_loss_weight):
    """The loss of swvr/api.py:53-66 over the readout's O and lse: the library's loss kernels
    where they apply, else the composite formula."""
    if _fusable_loss(O, lse, target, weight, reduction):
        D = O.shape[-1]
        out = mse_loss_op(O.reshape(-1, D), lse.reshape(-1), target.reshape(-1, D),
                          weight.reshape(-1) if weight is not None else None, z_loss_weight, reduction)
        return out.view(lse.shape) if reduction == "none" else out
    per_tok = (O - target.to(O.dtype)).pow(2).mean(dim=-1)
    if z_loss_weight:
        per_tok = per_tok + z_loss_weight * lse.pow(2)
    if weight is not None:
        per_tok = per_tok * weight.to(per_tok.dtype)
    if reduction == "none":
        return per_tok
    if reduction == "sum":
        return per_tok.sum()
    if reduction == "mean":
        denom = weight.to(per_tok.dtype).sum() if weight is not None else per_tok.numel()
        return per_tok.sum() / denom
    raise ValueError(f"unknown reduction {reduction!r}")


def _fusable_loss(O, lse, target, weight, reduction):
    """The library's loss kernels (``swvr::mse_loss``) compute the loss when the target and the
    weight have exactly the token shapes, live on O's device and need no gradient of their own;
    anything else (broadcasting, a differentiable target, an unknown reduction) takes the
    composite formula, which keeps the reference's semantics and errors."""
    if reduction not in REDUCTIONS or O.device.type != "cuda" or O.shape[-1] < 1 or lse.numel() == 0:
        return False
    if O.dtype != torch.float32 or lse.dtype != torch.float32:  # the loss kernels read fp32 (fp64 readouts: composite)
        return False
    if not isinstance(target, torch.Tensor) or target.shape != O.shape or target.device != O.device:
        return False
    if target.requires_grad or target.is_complex():
        return False
    if weight is not None:
        if not isinstance(weight, torch.Tensor) or weight.shape != lse.shape or weight.device != O.device:
            return False
        if weight.requires_grad or weight.is_complex():
            return False
    return True


def _weight_of(x):
    return x.weight if isinstance(x, nn.Module) else x


class SoftmaxReadoutMSE(nn.Module):
    """``softmax_readout_mse`` as a module that refers to a model's own head and embedding
    (swvr/api.py:73-93).

    ``head``: an ``nn.Linear(K, V)``, whose bias joins the scores when it has one, or a plain
    ``[V, K]`` tensor.  ``embedding``: an ``nn.Embedding(V, D)`` or a ``[V, D]`` tensor.  The
    parameters are read at each call, never copied, so tied weights stay tied and optimizers
    see the gradients on the model's tensors.
    """

    def __init__(self, head, embedding, *, z_loss_weight=0.0, logit_scale=1.0,
                 reduction="mean", chunk_size=None):
        super().__init__()
        self.head, self.embedding = head, embedding
        self.z_loss_weight, self.logit_scale = z_loss_weight, logit_scale
        self.reduction, self.chunk_size = reduction, chunk_size

    def forward(self, h, target, weight=None):
        bias = getattr(self.head, "bias", None) if isinstance(self.head, nn.Module) else None
        return softmax_readout_mse(
            h, _weight_of(self.head), _weight_of(self.embedding), target, bias,
            weight=weight, reduction=self.reduction, z_loss_weight=self.z_loss_weight,
            logit_scale=self.logit_scale, chunk_size=self.chunk_size)
