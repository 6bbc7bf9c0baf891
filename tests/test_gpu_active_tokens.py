"""The backward over the active tokens only.

A token whose cotangents are all zero (gO row = 0 and gLSE = 0, e.g. a token of
weight 0 in the MSE loss) contributes nothing to gW, gE and gb, and its gh row
is zero: the HIP backward compacts the other tokens and runs over them alone
(csrc/bwd.hip, bwd_compact_kernel).  These tests pin that against the fp64
closed form with cotangents that vanish on seeded subsets of tokens, spanning
several 256-token blocks and 32-position stage blocks, and the edge cases of
no active token and a single one.
"""
import pytest
import torch

import swvr_amd as swvr
from oracle import reference as ref

pytestmark = pytest.mark.gpu
f32, f64 = torch.float32, torch.float64
TOL = dict(rtol=2e-5, atol=2e-5)


def inputs(N, K, V, D, seed=0):
    """Logits of order one (W ~ N(0, 1/K)), so fp32 rounding stays inside the fp32 bar."""
    g = torch.Generator().manual_seed(seed)
    t = lambda *s, sc=1.0: (sc * torch.randn(*s, generator=g, dtype=f64)).to(device="cuda", dtype=f32).requires_grad_(True)
    return t(N, K), t(V, K, sc=K ** -0.5), t(V, D), t(V)


def run(h, W, E, b, gO, glse, chunk):
    O, lse = swvr.softmax_readout(h, W, E, b, chunk_size=chunk)
    return torch.autograd.grad((O * gO).sum() + (lse * glse).sum(), (h, W, E, b))


def oracle(h, W, E, b, gO, glse):
    xs = [x.detach().cpu().double().requires_grad_(True) for x in (h, W, E, b)]
    O, lse = ref.softmax_readout_reference(*xs)
    return torch.autograd.grad((O * gO.cpu().double()).sum() + (lse * glse.cpu().double()).sum(), xs)


def cotangents(N, D, active, seed=1):
    g = torch.Generator().manual_seed(seed)
    gO = torch.randn(N, D, generator=g, dtype=f64).to("cuda", f32)
    glse = (0.5 * torch.randn(N, generator=g, dtype=f64)).to("cuda", f32)
    gO[~active] = 0
    glse[~active] = 0
    return gO, glse


@pytest.mark.parametrize("frac,chunk", [(0.7, 256), (0.1, 600), (0.97, 128)])
def test_zero_cotangent_tokens_match_the_oracle(frac, chunk):
    N, K, V, D = 700, 64, 600, 16
    h, W, E, b = inputs(N, K, V, D)
    g = torch.Generator().manual_seed(2)
    active = (torch.rand(N, generator=g) < frac).cuda()
    active[0] = active[-1] = True
    gO, glse = cotangents(N, D, active)
    got = run(h, W, E, b, gO, glse, chunk)
    want = oracle(h, W, E, b, gO, glse)
    for a, r in zip(got, want):
        torch.testing.assert_close(a.double().cpu(), r, **TOL)
    assert (got[0][~active] == 0).all()  # gh of an inactive token is exactly zero


def test_only_gO_or_only_glse_keeps_a_token_active():
    N, K, V, D = 300, 32, 200, 8
    h, W, E, b = inputs(N, K, V, D)
    active = torch.zeros(N, dtype=torch.bool, device="cuda")
    active[[3, 100, 299]] = True
    gO, glse = cotangents(N, D, active)
    gO[100] = 0      # token 100: gLSE only
    glse[3] = 0      # token 3: gO only
    got = run(h, W, E, b, gO, glse, 64)
    want = oracle(h, W, E, b, gO, glse)
    for a, r in zip(got, want):
        torch.testing.assert_close(a.double().cpu(), r, **TOL)


def test_no_active_token_gives_zero_gradients():
    N, K, V, D = 520, 32, 300, 8
    h, W, E, b = inputs(N, K, V, D)
    gO = torch.zeros(N, D, device="cuda")
    glse = torch.zeros(N, device="cuda")
    for x in run(h, W, E, b, gO, glse, 128):
        assert (x == 0).all()


def test_weighted_mse_skips_zero_weight_tokens_bf16():
    """The north-star case: zero-weight tokens of the MSE loss in bf16."""
    N, K, V, D = 1000, 256, 3001, 64
    g = torch.Generator(device="cuda").manual_seed(0)
    r = lambda *s, sc=1.0: (sc * torch.randn(*s, device="cuda", generator=g)).to(torch.bfloat16).requires_grad_(True)
    h, W, b, E = r(N, K), r(V, K, sc=K ** -0.5), r(V, sc=0.02), r(V, D)
    target = torch.randn(N, D, device="cuda", generator=g)
    weight = (torch.rand(N, device="cuda", generator=g) >= 0.3).float()
    loss = swvr.softmax_readout_mse(h, W, E, target, b, weight=weight, z_loss_weight=1e-4)
    got = torch.autograd.grad(loss, (h, W, E, b))
    xs = [x.detach().double().requires_grad_(True) for x in (h, W, E, b)]
    want = torch.autograd.grad(ref.mse_reference(xs[0], xs[1], xs[2], target.double(), xs[3], weight=weight.double(),
                                                 z_loss_weight=1e-4, dtype=f64), xs)
    for a, w in zip(got, want):
        a = a.double()
        cos = (a.flatten() @ w.flatten() / (a.norm() * w.norm())).item()
        rel = ((a - w).norm() / w.norm()).item()
        assert cos >= 0.999 and rel <= 2e-2, (cos, rel)
    assert (got[0][weight == 0] == 0).all()
