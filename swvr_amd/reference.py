"""Eager reference, part of the public API (swvr/reference.py:1-14 of the reference).

It materialises the ``[N, V]`` scores, so it is meant for small shapes: a user's
own oracle.  It is not on the path of ``softmax_readout``, which always runs the
HIP kernels.
"""
import torch


def softmax_readout_reference(h, W, E, bias=None, logit_scale=1.0):
    """``(softmax(S) @ E, logsumexp(S))`` for ``S = logit_scale * h @ W.T + bias``, evaluated
    eagerly in the promotion of fp32 and the input dtypes."""
    dtype = torch.float32
    for t in (h, W, E, bias):
        if t is not None:
            dtype = torch.promote_types(dtype, t.dtype)
    scores = logit_scale * (h.to(dtype) @ W.to(dtype).T)
    if bias is not None:
        scores = scores + bias.to(dtype)
    return torch.softmax(scores, dim=-1) @ E.to(dtype), torch.logsumexp(scores, dim=-1)
