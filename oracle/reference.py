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


def reference_grads_blocked(h, W, E, bias, gO, glse, logit_scale=1.0, dtype=torch.float64, block=1024):
    """``reference_grads`` over every row, evaluated ``block`` rows at a time.

    Rows of the readout are independent, so O, lse and gh are the per-block
    results concatenated, and gW, gE, gb the per-block gradients summed (the
    loss is a sum over rows).  Memory is O(block * V) instead of O(N * V),
    which lets the closed form check every row at the full benchmark sizes.
    Runs on the device of its inputs.
    """
    N, K = h.shape
    V, D = E.shape
    dev = h.device
    Wd, Ed = W.detach().to(dtype), E.detach().to(dtype)
    bd = bias.detach().to(dtype) if bias is not None else None
    O = torch.empty(N, D, dtype=dtype, device=dev)
    lse = torch.empty(N, dtype=dtype, device=dev)
    gh = torch.empty(N, K, dtype=dtype, device=dev)
    gW = torch.zeros(V, K, dtype=dtype, device=dev)
    gE = torch.zeros(V, D, dtype=dtype, device=dev)
    gb = torch.zeros(V, dtype=dtype, device=dev) if bias is not None else None
    for r0 in range(0, N, block):
        r1 = min(N, r0 + block)
        o, l, g_h, g_W, g_E, g_b = reference_grads(h[r0:r1], Wd, Ed, bd, gO[r0:r1], glse[r0:r1],
                                                   logit_scale=logit_scale, dtype=dtype)
        O[r0:r1], lse[r0:r1], gh[r0:r1] = o, l, g_h
        gW += g_W
        gE += g_E
        if gb is not None:
            gb += g_b
        del o, l, g_h, g_W, g_E, g_b
    return O, lse, gh, gW, gE, gb


def mse_grads_blocked(h, W, E, target, bias=None, weight=None, reduction="mean", z_loss_weight=0.0,
                      logit_scale=1.0, dtype=torch.float64, block=1024):
    """``(loss, gh, gW, gE, gb)`` of ``mse_reference`` ("sum" or "mean"), ``block`` rows at a time.

    The loss is a sum over rows divided by a constant (sum of the weights, or N,
    for "mean"), so it and its gradients are the per-block ones summed (gh
    concatenated), each block evaluated as ``mse_reference(..., "sum")`` over
    its rows and divided by that constant.
    """
    if reduction not in ("sum", "mean"):
        raise ValueError(f"blocked evaluation needs a sum over rows, not {reduction!r}")
    N, K = h.shape
    V, D = E.shape
    dev = h.device
    den = 1.0
    if reduction == "mean":
        den = weight.to(dtype).sum() if weight is not None else float(N)
    Wd = W.detach().to(dtype).requires_grad_(True)
    Ed = E.detach().to(dtype).requires_grad_(True)
    bd = bias.detach().to(dtype).requires_grad_(True) if bias is not None else None
    loss = torch.zeros((), dtype=dtype, device=dev)
    gh = torch.empty(N, K, dtype=dtype, device=dev)
    gW = torch.zeros(V, K, dtype=dtype, device=dev)
    gE = torch.zeros(V, D, dtype=dtype, device=dev)
    gb = torch.zeros(V, dtype=dtype, device=dev) if bias is not None else None
    for r0 in range(0, N, block):
        r1 = min(N, r0 + block)
        hb = h[r0:r1].detach().to(dtype).requires_grad_(True)
        wb = weight[r0:r1] if weight is not None else None
        part = mse_reference(hb, Wd, Ed, target[r0:r1], bd, weight=wb, reduction="sum",
                             z_loss_weight=z_loss_weight, logit_scale=logit_scale, dtype=dtype) / den
        xs = [hb, Wd, Ed] + ([bd] if bd is not None else [])
        gs = torch.autograd.grad(part, xs)
        loss += part.detach()
        gh[r0:r1] = gs[0]
        gW += gs[1]
        gE += gs[2]
        if gb is not None:
            gb += gs[3]
        del part, gs
    return loss, gh, gW, gE, gb
