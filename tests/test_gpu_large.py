"""Sizes past 32-bit element offsets: h, and W, with more than 2^31 elements.

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
    """Cosine similarity, accumulated over pieces (a BLAS dot takes at most 2^31 - 1 elements)."""
    a, r = a.detach().flatten(), r.detach().flatten()
    dot = aa = rr = 0.0
    for i in range(0, a.numel(), 1 << 28):
        x, y = a[i:i + (1 << 28)].double(), r[i:i + (1 << 28)].double()
        dot, aa, rr = dot + (x @ y).item(), aa + (x @ x).item(), rr + (y @ y).item()
    return dot / max((aa * rr) ** 0.5, 1e-300)


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


def test_more_than_2_31_weight_elements_match_fp64():
    """V = 2^19 + 5 rows of K = 4096: W, its packed copies and gW past 2^31 elements (64 chunks and
    a partial one), 1000 tokens against the fp64 oracle."""
    n, k, v, d = 1000, 4096, (1 << 19) + 5, 16
    assert v * k > 2 ** 31
    g = torch.Generator(device="cuda").manual_seed(2)
    h = torch.randn(n, k, device="cuda", generator=g, dtype=torch.bfloat16)
    W = (torch.randn(v, k, device="cuda", generator=g) * (3.0 / k ** 0.5)).bfloat16()
    E = torch.randn(v, d, device="cuda", generator=g).bfloat16()
    b = (0.5 * torch.randn(v, device="cuda", generator=g)).bfloat16()
    gO = torch.randn(n, d, device="cuda", generator=g)
    glse = 0.1 * torch.randn(n, device="cuda", generator=g)
    xs = [x.requires_grad_(True) for x in (h, W, E, b)]
    O, lse = swvr.softmax_readout(*xs)
    grads = torch.autograd.grad((O * gO).sum() + (lse * glse).sum(), xs)
    got = (O.detach(), lse.detach(), *grads)
    del xs, O, lse, grads
    want = ref.reference_grads(h, W, E, b, gO, glse)
    errs = {name: rel_err(a, r) for name, a, r in zip(("O", "lse", "gh", "gW", "gE", "gb"), got, want)}
    print({key: f"{val:.1e}" for key, val in errs.items()}, flush=True)
    assert errs["O"] <= 1e-2 and errs["lse"] <= 1e-2, errs
    for name, a, r in zip(("gh", "gW", "gE", "gb"), got[2:], want[2:]):
        assert errs[name] <= 2e-2, errs
        assert cosine(a, r) >= 0.999, name
