"""Restatement of the reference's chunked CPU algorithm — test infrastructure only.

Follows the torch branch of swvr/chunked.py:82-151 (docs/DESIGN.md:12-37):
vocabulary chunks, online softmax forward, recomputing backward, with the
reference's precision policy:
  * products take operands in the compute dtype ``cdt`` and accumulate and
    output in fp32 (fp64 for fp64); on the CPU bf16/fp16 operands are upcast
    to fp32 before the product (mm_acc, chunked.py:30-55);
  * P is rounded to ``cdt`` before ``P @ E`` (chunked.py:103) and before
    ``P^T @ gO`` (chunked.py:139); gO is rounded to ``cdt`` (chunked.py:115);
    the scaled dS is rounded to ``cdt`` before the dh / dW products
    (chunked.py:143-145);
  * a row whose scores so far are all -inf is shifted by 0 (chunked.py:98-99).
This is the CPU baseline the bench times ("port"), and a second CPU
implementation the tests hold against the eager oracle.
"""
import torch


def _acc_dtype(cdt):
    return torch.float64 if cdt == torch.float64 else torch.float32


def _mm(a, b):
    """``a @ b`` never rounded below fp32 (chunked.py:30-55, CPU branch :55)."""
    if a.dtype in (torch.bfloat16, torch.float16):
        return torch.mm(a.float(), b.float())
    return torch.mm(a, b)


def _scores(hc, W, bias, v0, v1, s, cdt, adt):
    """``s * hc @ W[v0:v1]^T + bias[v0:v1]`` in ``adt`` (chunked.py:72-79)."""
    S = _mm(hc, W[v0:v1].to(cdt).T)
    if s != 1.0:
        S.mul_(s)
    if bias is not None:
        S.add_(bias[v0:v1].to(adt))
    return S


@torch.no_grad()
def forward(h, W, E, bias=None, logit_scale=1.0, chunk=8192, cdt=None):
    """``(O [N, D], lse [N])`` in the accumulation dtype (chunked.py:82-105)."""
    cdt = cdt or torch.promote_types(h.dtype, W.dtype)
    adt = _acc_dtype(cdt)
    N, V, D = h.shape[0], W.shape[0], E.shape[1]
    hc = h.to(cdt)
    m = torch.full((N,), float("-inf"), dtype=adt)
    l = torch.zeros(N, dtype=adt)
    acc = torch.zeros(N, D, dtype=adt)
    for v0 in range(0, V, chunk):
        v1 = min(v0 + chunk, V)
        S = _scores(hc, W, bias, v0, v1, logit_scale, cdt, adt)
        m_new = torch.maximum(m, S.amax(dim=1))
        shift = torch.where(torch.isinf(m_new), torch.zeros_like(m_new), m_new)
        alpha = torch.exp(m - shift)
        P = S.sub_(shift[:, None]).exp_()
        l.mul_(alpha).add_(P.sum(dim=1))
        acc.mul_(alpha[:, None]).add_(_mm(P.to(cdt), E[v0:v1].to(cdt)))
        m = m_new
    return acc.div_(l[:, None]), m + torch.log(l)


@torch.no_grad()
def backward(gO, glse, h, W, E, bias, O, lse, logit_scale=1.0, chunk=8192, cdt=None,
             need_h=True, need_W=True, need_E=True, need_b=True):
    """``(gh, gW, gE, gb)`` for output cotangents (gO, glse) (chunked.py:108-151).

    Gradients that are not needed (or have no input, for the bias) are None.
    """
    cdt = cdt or torch.promote_types(h.dtype, W.dtype)
    adt = O.dtype
    N, V = h.shape[0], W.shape[0]
    need_b = need_b and bias is not None
    hc = h.to(cdt)
    delta = (O * gO.to(adt)).sum(dim=1) - glse.to(adt)
    gOc = gO.to(cdt).contiguous()
    gH = torch.zeros(N, h.shape[1], dtype=adt) if need_h else None
    gW = torch.empty_like(W) if need_W else None
    gE = torch.empty_like(E) if need_E else None
    gb = torch.empty_like(bias) if need_b else None
    s = logit_scale
    for v0 in range(0, V, chunk):
        v1 = min(v0 + chunk, V)
        P = _scores(hc, W, bias, v0, v1, s, cdt, adt).sub_(lse[:, None]).exp_()
        gS = _mm(gOc, E[v0:v1].to(cdt).T).sub_(delta[:, None]).mul_(P)
        if need_b:
            gb[v0:v1] = gS.sum(dim=0)
        if need_E:
            gE[v0:v1] = _mm(P.to(cdt).T, gOc)
        del P
        if not (need_h or need_W):
            continue
        if s != 1.0:
            gS.mul_(s)
        gS = gS.to(cdt)
        Wc = W[v0:v1].to(cdt)
        if need_h:
            gH.add_(_mm(gS, Wc))
        if need_W:
            gW[v0:v1] = _mm(gS.T, hc)
    return (gH.to(h.dtype) if need_h else None), gW, gE, gb
