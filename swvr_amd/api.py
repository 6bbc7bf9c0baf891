"""Public entry points: ``softmax_readout``, ``softmax_readout_mse`` and ``SoftmaxReadoutMSE``.

Same contract as the reference's swvr/api.py:1-93 (argument shapes, dtypes of
the outputs, ValueError on bad shapes, loss reductions, module wrapper); the
work runs in the gfx950 HIP kernels behind ``swvr::chunked_fwd`` /
``swvr::chunked_bwd``.
"""
import os

import torch
from torch import nn

from ._ops import DEFAULT_CHUNK, REDUCTIONS, mse_loss_op, softmax_readout_op


def default_chunk_size():
    """Vocabulary staging chunk of the backward: env ``SWVR_CHUNK`` or 8192 (swvr/chunked.py:57-59)."""
    raw = os.environ.get("SWVR_CHUNK")
    return int(raw) if raw else DEFAULT_CHUNK


def _compute_dtype(h, W):
    """Autocast dtype when autocast is on, else the promoted input dtype (swvr/api.py:8-11)."""
    if h.device.type in ("cuda", "cpu") and torch.is_autocast_enabled(h.device.type):
        return torch.get_autocast_dtype(h.device.type)
    return torch.promote_types(h.dtype, W.dtype)


def _check(h, W, E, bias):
    """Shape validation with the reference's messages (swvr/api.py:14-22)."""
    if W.dim() != 2 or E.dim() != 2:
        raise ValueError(f"W and E must be 2-D, got {tuple(W.shape)} and {tuple(E.shape)}")
    if h.shape[-1] != W.shape[1]:
        raise ValueError(f"h has hidden size {h.shape[-1]} but W is {tuple(W.shape)}")
    if E.shape[0] != W.shape[0]:
        raise ValueError(f"W has {W.shape[0]} vocabulary rows but E has {E.shape[0]}")
    if bias is not None and bias.shape != (W.shape[0],):
        raise ValueError(f"bias must have shape ({W.shape[0]},), got {tuple(bias.shape)}")


def softmax_readout(h, W, E, bias=None, *, logit_scale=1.0, chunk_size=None):
    """Return ``(O, LSE)`` for ``S = logit_scale * h @ W.T + bias`` (swvr/api.py:25-41).

    ``O = softmax(S) @ E`` has shape ``[..., D]`` and ``LSE = logsumexp(S)`` has shape
    ``[...]``, both fp32.  ``h`` is ``[..., K]``, ``W`` is ``[V, K]``, ``E`` is ``[V, D]`` and
    ``bias`` is ``[V]``.  Gradients flow to every input that requires them.  The scores are
    never materialised; the backward stages ``chunk_size`` (default 8192, or env
    ``SWVR_CHUNK``) vocabulary rows of dS at a time, so its extra memory is O(N * chunk_size).
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
    """MSE between ``softmax(S) @ E`` and ``target`` plus an optional z-loss (swvr/api.py:44-66).

    The per-token loss is ``mean_d (O - target)^2 + z_loss_weight * LSE^2``.  ``weight``
    (shape ``[...]``) scales each token's loss and 0 masks it out.  ``reduction="mean"``
    divides by ``weight.sum()`` when a weight is given, else by the token count; ``"sum"`` and
    ``"none"`` are also accepted.
    """
    O, lse = softmax_readout(h, W, E, bias, logit_scale=logit_scale, chunk_size=chunk_size)
    return _mse_loss(O, lse, target, weight, reduction, z_loss_weight)


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
    """Loss module over an existing LM head and embedding table, without copying them
    (swvr/api.py:73-93).

    ``head`` is an ``nn.Linear(K, V)`` (its bias is used if present) or a ``[V, K]`` tensor;
    ``embedding`` is an ``nn.Embedding(V, D)`` or a ``[V, D]`` tensor.  Passing the model's own
    modules keeps weight tying and optimizer state intact.
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
