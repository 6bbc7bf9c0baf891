"""Sizes past 32-bit element offsets: h with more than 2^31 elements.

N = 2^20 + 37 tokens of K = 2048 put h (and the backward's h over positions,
its packed copy, the fp32 dh accumulator and gh) past 2^31 elements, so every
offset into them must be 64-bit; the token count also leaves a partial last
token block.  The readout is checked against the fp64 oracle on every row, a
block of rows at a time (rows are independent: O, lse and gh per block, gW,
gE and gb summed over the blocks), to the north-star bar: O and lse rel err
<= 1e-2, every gradient rel err <= 2e-2 and cosine >= 0.999.  The weighted
loss at the same size runs the forward over the non-zero-weight tokens
(compaction, gathered h) and the backward over them.
"""
import pytest
import torch

import swvr_amd as swvr
from oracle import reference as ref

pytestmark = pytest.mark.gpu

N, K, V, D = (1 << 20) + 37, 2048, 2048, 16
BLOCK = 1 << 16


def rel_err(a, r):
    a, r = a.detach().double(), r.detach().double()
    return ((a - r).norm() / r.norm().clamp_min(1e-30)).item()


def cosine(a, r):
    a, r = a.detach().double().flatten(), r.detach().double().flatten()
    return (a @ r / (a.norm() * r.norm()).clamp_min(1e-300)).item()


def inputs(seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    h = torch.randn(N, K, device="cuda", generator=g, dtype=torch.bfloat16)
    W = (torch.randn(V, K, device="cuda", generator=g) * (3.0 / K ** 0.5)).bfloat16()
    E = torch.randn(V, D, device="cuda", generator=g).bfloat16()
    b = (0.5 * torch.randn(V, device="cuda", generator=g)).bfloat16()
    return g, h, W, E, b


def test_more_than_2_31_hidden_elements_match_fp64_on_every_row():
    assert N * K > 2 ** 31
    g, h, W, E, b = inputs(0)
    gO = torch.randn(N, D, device="cuda", generator=g)
    glse = 0.1 * torch.randn(N, device="cuda", generator=g)
    xs = [x.requires_grad_(True) for x in (h, W, E, b)]
    O, lse = swvr.softmax_readout(*xs)
    gh, gW, gE, gb = torch.autograd.grad((O * gO).sum() + (lse * glse).sum(), xs)
    O, lse = O.detach(), lse.detach()
    assert gh.shape == (N, K) and torch.isfinite(gh).all()
    rW = torch.zeros(V, K, dtype=torch.float64, device="cuda")
    rE = torch.zeros(V, D, dtype=torch.float64, device="cuda")
    rb = torch.zeros(V, dtype=torch.float64, device="cuda")
    worst = {"O": 0.0, "lse": 0.0, "gh": 0.0}
    min_cos_gh = 1.0
    for r0 in range(0, N, BLOCK):
        r1 = min(N, r0 + BLOCK)
        o, l, g_h, g_W, g_E, g_b = ref.reference_grads(h[r0:r1], W, E, b, gO[r0:r1], glse[r0:r1])
        worst["O"] = max(worst["O"], rel_err(O[r0:r1], o))
        worst["lse"] = max(worst["lse"], rel_err(lse[r0:r1], l))
        worst["gh"] = max(worst["gh"], rel_err(gh[r0:r1], g_h))
        min_cos_gh = min(min_cos_gh, cosine(gh[r0:r1], g_h))
        rW += g_W
        rE += g_E
        rb += g_b
        del o, l, g_h, g_W, g_E, g_b
    errs = {**worst, "gW": rel_err(gW, rW), "gE": rel_err(gE, rE), "gb": rel_err(gb, rb)}
    print({k: f"{v:.1e}" for k, v in errs.items()}, flush=True)
    assert errs["O"] <= 1e-2 and errs["lse"] <= 1e-2, errs
    for n in ("gh", "gW", "gE", "gb"):
        assert errs[n] <= 2e-2, errs
    assert min_cos_gh >= 0.999
    for a, r in ((gW, rW), (gE, rE), (gb, rb)):
        assert cosine(a, r) >= 0.999


def test_weighted_loss_at_more_than_2_31_hidden_elements():
    """softmax_readout_mse with a Bernoulli(0.75) weight: the forward and backward over the
    non-zero-weight tokens only, at the same size, against the fp64 oracle's loss and gradients."""
    g, h, W, E, b = inputs(1)
    target = torch.randn(N, D, device="cuda", generator=g)
    weight = (torch.rand(N, device="cuda", generator=g) < 0.75).float()
    xs = [x.requires_grad_(True) for x in (h, W, E, b)]
    loss = swvr.softmax_readout_mse(*xs[:3], target, xs[3], weight=weight, z_loss_weight=1e-3)
    gh, gW, gE, gb = torch.autograd.grad(loss, xs)
    assert torch.count_nonzero(gh[weight == 0]) == 0
    den = weight.double().sum()
    r_loss = torch.zeros((), dtype=torch.float64, device="cuda")
    rW = torch.zeros(V, K, dtype=torch.float64, device="cuda")
    rE = torch.zeros(V, D, dtype=torch.float64, device="cuda")
    rb = torch.zeros(V, dtype=torch.float64, device="cuda")
    worst_gh = 0.0
    for r0 in range(0, N, BLOCK):
        r1 = min(N, r0 + BLOCK)
        ys = [h[r0:r1].detach().double().requires_grad_(True)] + [
            x.detach().double().requires_grad_(True) for x in (W, E, b)]
        l_blk = ref.mse_reference(ys[0], ys[1], ys[2], target[r0:r1].double(), ys[3],
                                  weight=weight[r0:r1].double(), reduction="sum", z_loss_weight=1e-3) / den
        g_blk = torch.autograd.grad(l_blk, ys)
        r_loss += l_blk.detach()
        worst_gh = max(worst_gh, rel_err(gh[r0:r1], g_blk[0]) if g_blk[0].norm() > 0 else 0.0)
        rW += g_blk[1]
        rE += g_blk[2]
        rb += g_blk[3]
        del ys, l_blk, g_blk
    errs = {"loss": rel_err(loss, r_loss), "gh": worst_gh, "gW": rel_err(gW, rW), "gE": rel_err(gE, rE),
            "gb": rel_err(gb, rb)}
    print({k: f"{v:.1e}" for k, v in errs.items()}, flush=True)
    assert errs["loss"] <= 1e-2, errs
    for n in ("gh", "gW", "gE", "gb"):
        assert errs[n] <= 2e-2, errs
    for a, r in ((gW, rW), (gE, rE), (gb, rb)):
        assert cosine(a, r) >= 0.999
