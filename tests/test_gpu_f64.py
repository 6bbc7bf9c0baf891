"""fp64 readouts: fp64 inputs compute and return fp64, as the reference's do
(swvr/chunked.py:26-27, 62-63; swvr/api.py:35 "fp64 for fp64 inputs").

The HIP fp64 path (csrc/f64.hip, swvr_fwd_f64 / swvr_bwd_f64) is compared with
the fp64 closed form (oracle.reference) to fp64 rounding, and its gradients
with finite differences through torch.autograd.gradcheck.
"""
import pytest
import torch

import swvr_amd as swvr
from oracle import reference as ref

pytestmark = pytest.mark.gpu
f64 = torch.float64
TOL = dict(rtol=1e-9, atol=1e-11)


def make(N, K, V, D, bias=True, seed=0, lead=None, dtype=f64):
    g = torch.Generator().manual_seed(seed)
    t = lambda *s, sc=1.0: (sc * torch.randn(*s, generator=g, dtype=f64)).to("cuda", dtype).requires_grad_(True)
    h = t(*(lead or (N,)), K)
    return h, t(V, K, sc=3 * K ** -0.5), t(V, D), (t(V, sc=0.5) if bias else None)


def grads_of(fn, xs, gO, glse):
    O, lse = fn(*xs)
    want = [x for x in xs if x is not None and x.requires_grad]
    return [O, lse, *torch.autograd.grad((O * gO).sum() + (lse * glse).sum(), want)]


@pytest.mark.parametrize("N,K,V,D,chunk,bias,scale", [
    (37, 24, 101, 5, 16, True, 1.0),
    (300, 96, 1000, 40, 256, True, 0.7),
    (64, 130, 513, 300, 5000, False, 1.3),
    (1, 8, 1, 3, 7, True, 1.0),
])
def test_f64_matches_the_closed_form(N, K, V, D, chunk, bias, scale):
    xs = make(N, K, V, D, bias)
    g = torch.Generator().manual_seed(1)
    gO = torch.randn(N, D, generator=g, dtype=f64).cuda()
    glse = torch.randn(N, generator=g, dtype=f64).cuda()
    got = grads_of(lambda *a: swvr.softmax_readout(*a, logit_scale=scale, chunk_size=chunk), xs, gO, glse)
    want = grads_of(lambda *a: ref.softmax_readout_reference(*a, logit_scale=scale, dtype=f64), xs, gO, glse)
    assert got[0].dtype == f64 and got[1].dtype == f64
    for a, r in zip(got, want):
        torch.testing.assert_close(a, r, **TOL)


def test_f64_gradcheck():
    """Every gradient against central finite differences (the reference's fp64 gradcheck,
    tests/test_cpu.py:46-51), through the HIP path."""
    h, W, E, b = make(5, 7, 11, 3)
    fn = lambda h, W, E, b: swvr.softmax_readout(h, W, E, b, logit_scale=0.9, chunk_size=4)
    assert torch.autograd.gradcheck(fn, (h, W, E, b), eps=1e-6, atol=1e-6, rtol=1e-5)


def test_f64_leading_dims_masks_and_fully_masked_rows():
    h, W, E, b = make(0, 16, 50, 4, lead=(3, 7))
    with torch.no_grad():
        b[10:20] = -float("inf")
    O, lse = swvr.softmax_readout(h, W, E, b, chunk_size=8)
    Or, lser = ref.softmax_readout_reference(h, W, E, b, dtype=f64)
    assert O.shape == (3, 7, 4) and lse.shape == (3, 7)
    torch.testing.assert_close(O.detach(), Or.detach(), **TOL)
    torch.testing.assert_close(lse.detach(), lser.detach(), **TOL)
    gb = torch.autograd.grad(O.sum() + lse.sum(), b)[0]
    assert (gb[10:20] == 0).all()
    # every score -inf: O = NaN and lse = -inf, as the reference gives
    with torch.no_grad():
        b.fill_(-float("inf"))
    O, lse = swvr.softmax_readout(h.detach(), W.detach(), E.detach(), b.detach(), chunk_size=8)
    assert torch.isnan(O).all() and (lse == -float("inf")).all()


def test_f64_no_tokens_gives_zero_vocabulary_gradients():
    h, W, E, b = make(0, 16, 40, 4)
    O, lse = swvr.softmax_readout(h, W, E, b)
    assert O.shape == (0, 4) and O.dtype == f64
    gW, gE, gb = torch.autograd.grad(O.sum() + lse.sum(), (W, E, b), allow_unused=True)
    for g, x in ((gW, W), (gE, E), (gb, b)):
        assert g is None or (g.shape == x.shape and (g == 0).all())


def test_f64_promotion_from_mixed_inputs_and_grad_dtypes():
    """fp32 h with fp64 W promotes to fp64 (swvr/api.py:8-11); gh comes back in h's dtype."""
    h, W, E, b = make(20, 16, 70, 6)
    h32 = h.detach().float().requires_grad_(True)
    O, lse = swvr.softmax_readout(h32, W, E, b, chunk_size=32)
    assert O.dtype == f64 and lse.dtype == f64
    gh, gW = torch.autograd.grad(O.sum() + lse.sum(), (h32, W))
    assert gh.dtype == torch.float32 and gW.dtype == f64
    Or, lser = ref.softmax_readout_reference(h32.double(), W, E, b, dtype=f64)
    ghr, gWr = torch.autograd.grad(Or.sum() + lser.sum(), (h32, W))
    torch.testing.assert_close(gh, ghr.float(), rtol=1e-6, atol=1e-7)
    torch.testing.assert_close(gW, gWr, **TOL)


def test_f64_mse_loss_matches_the_reference_formula():
    h, W, E, b = make(50, 32, 300, 8)
    g = torch.Generator().manual_seed(3)
    target = torch.randn(50, 8, generator=g, dtype=f64).cuda()
    weight = (torch.rand(50, generator=g) > 0.3).to(f64).cuda()
    for red in ("mean", "sum", "none"):
        loss = swvr.softmax_readout_mse(h, W, E, target, b, weight=weight, reduction=red, z_loss_weight=1e-3,
                                        chunk_size=64)
        want = ref.mse_reference(h, W, E, target, b, weight=weight, reduction=red, z_loss_weight=1e-3, dtype=f64)
        assert loss.dtype == f64
        torch.testing.assert_close(loss, want, **TOL)
        gs = torch.autograd.grad(loss.sum(), (h, W, E, b))
        ws = torch.autograd.grad(want.sum(), (h, W, E, b))
        for a, r in zip(gs, ws):
            torch.testing.assert_close(a, r, **TOL)


def test_f64_is_deterministic():
    xs = make(200, 64, 900, 16)
    gO = torch.randn(200, 16, dtype=f64).cuda()
    glse = torch.randn(200, dtype=f64).cuda()
    a = grads_of(lambda *x: swvr.softmax_readout(*x, chunk_size=128), xs, gO, glse)
    b = grads_of(lambda *x: swvr.softmax_readout(*x, chunk_size=128), xs, gO, glse)
    for x, y in zip(a, b):
        assert torch.equal(x, y)
