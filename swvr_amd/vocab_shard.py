"""Vocabulary-parallel building blocks: the shard-local forward and the combine.

With W, E and bias split by vocabulary rows over S shards (one per rank of a
vocabulary-parallel job), the readout needs one exchange:

    m_s, l_s, acc_s = softmax_readout_partial(h, W_s, E_s, b_s)    # on each shard
    (all-gather of m, l, acc: N (D + 2) floats per shard)
    O, lse = combine_partials(m, l, acc)                           # same on every rank

and the backward none but a sum of gh over the shards:

    gh_s, gW_s, gE_s, gb_s = shard_backward(gO, glse, h, W_s, E_s, b_s, O, lse)
    gh = sum_s gh_s

The exchange itself is the caller's (this build runs on one GPU); the shard
kernels are the same HIP kernels as softmax_readout's (C ABI:
swvr_fwd_partial, swvr_combine, swvr_bwd), so the shards' results merge to the
whole vocabulary's up to summation order.  These are plain functions without
autograd: a vocabulary-parallel training step calls them from its own
autograd.Function around the collectives.
"""
from typing import Optional, Tuple

import torch

from . import _lib
from ._ops import _backward, _embed, _kpad, _lead_stride, _matrix, _require_device
from .api import _check, _compute_dtype, default_chunk_size


def softmax_readout_partial(h: torch.Tensor, W: torch.Tensor, E: torch.Tensor, bias: Optional[torch.Tensor] = None,
                            *, logit_scale: float = 1.0) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Softmax partials of a vocabulary shard: ``m [...]``, ``l [...]``, ``acc [..., D]`` (fp32).

    ``m = max_v S``, ``l = sum_v exp(S - m)``, ``acc = sum_v exp(S - m) E[v]`` over the shard's rows
    ``v`` of ``S = logit_scale * h @ W.T + bias``."""
    _check(h, W, E, bias)
    _require_device(h)
    cdt = _compute_dtype(h, W)
    if cdt not in _lib.DTYPE_TAG:
        raise NotImplementedError(f"swvr_amd: compute dtype {cdt} is not supported (bf16, fp16, fp32)")
    lead = h.shape[:-1]
    h2 = h.reshape(-1, h.shape[-1])
    N, K = h2.shape
    V, D = E.shape
    Kp = _kpad(K)
    hc, Wc, Ec = _matrix(h2, cdt, Kp), _matrix(W, cdt, Kp), _embed(E, cdt)
    b = bias.to(torch.float32).contiguous() if bias is not None else None
    m = torch.empty(N, dtype=torch.float32, device=h.device)
    l = torch.empty(N, dtype=torch.float32, device=h.device)
    acc = torch.empty(N, D, dtype=torch.float32, device=h.device)
    lib = _lib.load()
    tag = _lib.DTYPE_TAG[cdt]
    ws_bytes = lib.swvr_fwd_workspace_size(tag, N, Kp, V, D)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=h.device)
    with torch.cuda.device(h.device):
        rc = lib.swvr_fwd_partial(tag, N, Kp, V, D, _lib.ptr(hc), _lead_stride(hc), _lib.ptr(Wc), _lead_stride(Wc),
                                  _lib.ptr(Ec), _lead_stride(Ec), _lib.ptr(b), float(logit_scale),
                                  _lib.ptr(m), _lib.ptr(l), _lib.ptr(acc), _lib.ptr(ws), ws_bytes,
                                  _lib.stream_of(h.device))
    _lib.check(rc)
    return m.view(lead), l.view(lead), acc.view(*lead, D)


def combine_partials(m: torch.Tensor, l: torch.Tensor, acc: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
    """Merge the shards' partials, stacked on dim 0 (``m, l [S, ...]``, ``acc [S, ..., D]``), in shard
    order into ``O [..., D]`` and ``lse [...]`` (fp32), as softmax_readout gives for the union."""
    if m.dim() < 1 or l.shape != m.shape or acc.shape[:-1] != m.shape:
        raise ValueError(f"partials must be m, l [S, ...] and acc [S, ..., D]; got {tuple(m.shape)}, "
                         f"{tuple(l.shape)}, {tuple(acc.shape)}")
    _require_device(m)
    S, lead, D = m.shape[0], m.shape[1:], acc.shape[-1]
    N = m[0].numel()
    m32, l32 = m.to(torch.float32).contiguous(), l.to(torch.float32).contiguous()
    a32 = acc.to(torch.float32).contiguous()
    O = torch.empty(N, D, dtype=torch.float32, device=m.device)
    lse = torch.empty(N, dtype=torch.float32, device=m.device)
    lib = _lib.load()
    with torch.cuda.device(m.device):
        rc = lib.swvr_combine(S, N, D, _lib.ptr(m32), _lib.ptr(l32), _lib.ptr(a32), _lib.ptr(O), _lib.ptr(lse),
                              _lib.stream_of(m.device))
    _lib.check(rc)
    return O.view(*lead, D), lse.view(lead)


def shard_backward(gO: torch.Tensor, glse: torch.Tensor, h: torch.Tensor, W: torch.Tensor, E: torch.Tensor,
                   bias: Optional[torch.Tensor], O: torch.Tensor, lse: torch.Tensor, *, logit_scale: float = 1.0,
                   chunk_size: Optional[int] = None, need=(True, True, True, True)):
    """Gradients of one shard given the merged ``O`` and ``lse``: ``(gh_s, gW_s, gE_s, gb_s)``.

    ``gW_s``, ``gE_s``, ``gb_s`` are the shard's rows of the full gradients; the full ``gh`` is the
    sum of ``gh_s`` over the shards.  ``need`` selects (gh, gW, gE, gb); a gradient not needed is None."""
    _check(h, W, E, bias)
    _require_device(h)
    cdt = _compute_dtype(h, W)
    lead = h.shape[:-1]
    h2 = h.reshape(-1, h.shape[-1])
    N, D = h2.shape[0], E.shape[1]
    chunk = int(chunk_size) if chunk_size else default_chunk_size()
    if chunk <= 0:
        raise ValueError(f"chunk_size must be positive, got {chunk}")
    need_h, need_W, need_E, need_b = need
    gh, gW, gE, gb = _backward(gO.reshape(N, D), glse.reshape(N), h2, W, E, bias, O.reshape(N, D), lse.reshape(N),
                               logit_scale, chunk, cdt, need_h, need_W, need_E, need_b and bias is not None)
    if gh is not None:
        gh = gh.view(*lead, h.shape[-1])
    return gh, gW, gE, gb
