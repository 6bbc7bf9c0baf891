"""The library's MSE loss kernels (``swvr_mse_loss`` behind ``swvr::mse_loss``).

The loss is swvr/api.py:53-66: per token mean_d (O - target)^2 + z * lse^2, times
the token weight, reduced by "none", "sum" or "mean" (mean over sum w when
weighted).  These tests hold the kernels to the fp64 formula on the same O and
lse, check the end-to-end loss against the composite torch formula over the same
forward, and pin the cases the composite path keeps (broadcast or
differentiable targets)."""
import pytest
import torch

import swvr_amd as swvr
from swvr_amd._ops import mse_loss_op
from tests.gpu_util import rel_err

pytestmark = pytest.mark.gpu


def formula(O, lse, target, weight, z, reduction):
    per_tok = (O - target.to(O.dtype)).pow(2).mean(-1)
    if z:
        per_tok = per_tok + z * lse.pow(2)
    if weight is not None:
        per_tok = per_tok * weight.to(per_tok.dtype)
    if reduction == "none":
        return per_tok
    if reduction == "sum":
        return per_tok.sum()
    denom = weight.to(per_tok.dtype).sum() if weight is not None else per_tok.numel()
    return per_tok.sum() / denom


def make_loss_inputs(N, D, tdt, wkind, seed=0):
    g = torch.Generator(device="cuda").manual_seed(seed)
    O = torch.randn(N, D, device="cuda", generator=g)
    lse = 3 + torch.randn(N, device="cuda", generator=g)
    target = torch.randn(N, D, device="cuda", generator=g).to(tdt)
    if wkind is None:
        weight = None
    elif wkind == "bernoulli":
        weight = (torch.rand(N, device="cuda", generator=g) >= 0.3).float()
    else:
        weight = torch.rand(N, device="cuda", generator=g)
    return O, lse, target, weight


@pytest.mark.parametrize("reduction", ["none", "sum", "mean"])
@pytest.mark.parametrize("wkind", [None, "bernoulli", "uniform"])
@pytest.mark.parametrize("z", [0.0, 1e-2])
@pytest.mark.parametrize("tdt,D", [(torch.float32, 5), (torch.bfloat16, 64), (torch.float16, 200)])
def test_loss_kernel_matches_the_fp64_formula(reduction, wkind, z, tdt, D):
    N = 1000
    O, lse, target, weight = make_loss_inputs(N, D, tdt, wkind)
    Og, lseg = O.clone().requires_grad_(True), lse.clone().requires_grad_(True)
    out = mse_loss_op(Og, lseg, target, weight, z, reduction)
    gout = torch.rand_like(out) + 0.5
    gO, glse = torch.autograd.grad(out, (Og, lseg), gout)
    O64, lse64 = O.double().requires_grad_(True), lse.double().requires_grad_(True)
    want = formula(O64, lse64, target.double(), weight.double() if weight is not None else None, z, reduction)
    wO, wlse = torch.autograd.grad(want, (O64, lse64), gout.double(), allow_unused=True)
    assert out.shape == want.shape and out.dtype == torch.float32
    assert rel_err(out, want) < 1e-5
    assert rel_err(gO, wO) < 1e-5
    if z:
        assert rel_err(glse, wlse) < 1e-5
    else:
        assert torch.count_nonzero(glse) == 0


def test_loss_is_deterministic_and_needs_no_grad_buffers_under_no_grad():
    O, lse, target, weight = make_loss_inputs(4099, 64, torch.bfloat16, "uniform", seed=3)
    a = mse_loss_op(O, lse, target, weight, 1e-3, "mean")
    b = mse_loss_op(O, lse, target, weight, 1e-3, "mean")
    assert torch.equal(a, b)
    Og = O.clone().requires_grad_(True)
    c = mse_loss_op(Og, lse, target, weight, 1e-3, "mean")
    with torch.no_grad():
        d = mse_loss_op(Og, lse, target, weight, 1e-3, "mean")
    assert torch.equal(a, c) and torch.equal(c, d) and not d.requires_grad


def test_all_zero_weights_give_nan_like_the_reference():
    O, lse, target, _ = make_loss_inputs(64, 8, torch.float32, None)
    weight = torch.zeros(64, device="cuda")
    out = mse_loss_op(O, lse, target, weight, 0.0, "mean")
    assert torch.isnan(out)
    assert torch.isnan(formula(O, lse, target, weight, 0.0, "mean"))
    assert mse_loss_op(O, lse, target, weight, 0.0, "sum").item() == 0.0


def readout_inputs(N=300, K=96, V=1500, D=24, seed=1):
    g = torch.Generator(device="cuda").manual_seed(seed)
    h = torch.randn(N, K, device="cuda", generator=g)
    W = torch.randn(V, K, device="cuda", generator=g) / K ** 0.5
    E = torch.randn(V, D, device="cuda", generator=g)
    b = 0.1 * torch.randn(V, device="cuda", generator=g)
    target = torch.randn(N, D, device="cuda", generator=g)
    weight = (torch.rand(N, device="cuda", generator=g) >= 0.2).float()
    return [h, W, E, b], target, weight


@pytest.mark.parametrize("reduction", ["none", "sum", "mean"])
def test_fused_loss_equals_the_composite_formula_over_the_same_forward(reduction):
    xs, target, weight = readout_inputs()
    xs = [x.to(torch.bfloat16).requires_grad_(True) for x in xs]
    kw = dict(weight=weight, z_loss_weight=1e-3, reduction=reduction, chunk_size=512)
    fused = swvr.softmax_readout_mse(xs[0], xs[1], xs[2], target, xs[3], **kw)
    gout = torch.rand_like(fused) + 0.5
    gf = torch.autograd.grad(fused, xs, gout)
    O, lse = swvr.softmax_readout(xs[0], xs[1], xs[2], xs[3], chunk_size=512)
    comp = formula(O, lse, target, weight, 1e-3, reduction)
    gc = torch.autograd.grad(comp, xs, gout)
    assert rel_err(fused, comp) < 1e-5
    for a, r in zip(gf, gc):
        assert rel_err(a, r) < 1e-2   # bf16 gradients: the same kernels, gO differs by fp32 rounding


def test_leading_dims_and_the_composite_cases():
    xs, target, weight = readout_inputs(N=240)
    h3, t3, w3 = xs[0].reshape(4, 60, -1), target.reshape(4, 60, -1), weight.reshape(4, 60)
    per_tok = swvr.softmax_readout_mse(h3, xs[1], xs[2], t3, xs[3], weight=w3, reduction="none")
    assert per_tok.shape == (4, 60)
    O, lse = swvr.softmax_readout(h3, xs[1], xs[2], xs[3])
    assert rel_err(per_tok, formula(O, lse, t3, w3, 0.0, "none")) < 1e-6
    # a differentiable target takes the composite formula and gets its gradient
    tg = t3.clone().requires_grad_(True)
    loss = swvr.softmax_readout_mse(h3, xs[1], xs[2], tg, xs[3], weight=w3)
    (gt,) = torch.autograd.grad(loss, tg)
    want = -2 * (O - t3) * w3[..., None] / (O.shape[-1] * w3.sum())
    assert rel_err(gt, want) < 1e-5
    # a weight that broadcasts over the leading dims: the reference divides by weight.sum() as given
    wb = weight[:60]
    loss = swvr.softmax_readout_mse(h3, xs[1], xs[2], t3, xs[3], weight=wb)
    assert rel_err(loss, formula(O, lse, t3, wb, 0.0, "mean")) < 1e-6


def test_loss_over_no_tokens_follows_the_reference():
    O = torch.empty(0, 8, device="cuda")
    lse = torch.empty(0, device="cuda")
    t = torch.empty(0, 8, device="cuda")
    assert mse_loss_op(O, lse, t, None, 0.0, "none").shape == (0,)
    assert mse_loss_op(O, lse, t, None, 0.0, "sum").item() == 0.0
    assert torch.isnan(mse_loss_op(O, lse, t, None, 0.0, "mean"))       # 0 / 0, as sum() / numel()
    assert torch.isnan(formula(O, lse, t, None, 0.0, "mean"))
