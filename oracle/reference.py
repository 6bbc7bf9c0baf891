"""Eager closed-form oracle (CPU, fp32/fp64) — test infrastructure only.

Restates swvr/reference.py:5-14 (the reference's parity target) and the loss of
swvr/api.py:53-66 / tests/test_cpu.py:150-159.  It materialises the [N, V]
scores, so it is for sizes the CPU finishes in seconds.
"""
import torch


def softmax_readout_reference(h, W, E, bias=None, logit_scale=1.0, dtype=None):
    """``(softmax(S) E, logsumexp(S))`` with ``S = logit_scale * h W^T + bias``.

    Evaluated in ``dtype`` (default: the promotion of fp32 and the inputs, as
    swvr/reference.py:7-10 does).  Differentiable through torch autograd.
    """
    if dtype is None:
        dtype = torch.float32
        for t in (h, W, E, bias):
            if t is not None:
                dtype = torch.promote_types(dtype, t.dtype)
    S = logit_scale * (h.to(dtype) @ W.to(dtype).T)
    if bias is not None:
        S = S + bias.to(dtype)
    return torch.softmax(S, dim=-1) @ E.to(dtype), torch.logsumexp(S, dim=-1)


def mse_reference(h, W, E, target, bias=None, weight=None, reduction="mean", z_loss_weight=0.0,
                  logit_scale=1.0, dtype=None):
    """Per-token ``mean_d (O - t)^2 + z * lse^2``, times weight, reduced (swvr/api.py:53-66)."""
    O, lse = softmax_readout_reference(h, W, E, bias, logit_scale, dtype=dtype)
    per_tok = (O - target.to(O.dtype)).pow(2).mean(-1) + z_loss_weight * lse.pow(2)
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


def reference_grads(h, W, E, bias, gO, glse, logit_scale=1.0, dtype=torch.float64, rows=None):
    """``(O, lse, gh, gW, gE, gb)`` of the closed form for output cotangents (gO, glse).

    ``rows`` (a LongTensor of token indices) restricts the computation to those
    tokens: O, lse and gh are then for those rows, and gW, gE, gb are the
    gradients of the loss with gO / glse zero outside ``rows`` — each token's
    contribution is independent, so this is exact.
    """
    if rows is not None:
        h, gO, glse = h[rows], gO[rows], glse[rows]
    xs = [x.detach().to(dtype).requires_grad_(True) if x is not None else None for x in (h, W, E, bias)]
    O, lse = softmax_readout_reference(*xs, logit_scale=logit_scale, dtype=dtype)
    loss = (O * gO.to(dtype)).sum() + (lse * glse.to(dtype)).sum()
    want = [x for x in xs if x is not None]
    gs = torch.autograd.grad(loss, want, allow_unused=True)
    it = iter(gs)
    g = [next(it) if x is not None else None for x in xs]
    return (O.detach(), lse.detach(), *g)
