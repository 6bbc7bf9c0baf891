"""The forward over the non-zero-weight tokens of a weighted loss (``swvr_fwd_active``).

``softmax_readout_mse`` with a per-token weight multiplies each token's loss by
its weight (swvr/api.py:53-66), so a zero-weight token's readout only enters the
loss as 0 x (a finite term).  The library computes the other tokens alone:
compaction of the active tokens on the device, h rows gathered into the packed
tile image, the vocabulary re-split from the device count so the grid stays
full, and O rows / lse of 0 for the skipped tokens.  These tests hold the
computed rows to the fp64 oracle and the skipped ones to exact zeros, over
every forward tile (D = 16 ... 300, bf16 / fp16 / fp32, fp32 storage under a
2-byte compute dtype, K = 0), over masks that halve the token blocks (so the
vocabulary splits change), and pin the rows kept to reproduce the reference's
NaNs (a non-finite h row, W, E or bias, every bias -inf, a non-finite logit
scale, a NaN weight or target).
"""
import math

import pytest
import torch

import swvr_amd as swvr
from swvr_amd import _ops
from oracle import reference as ref
from tests.gpu_util import rel_err

pytestmark = pytest.mark.gpu
f64 = torch.float64


def inputs(N, K, V, D, dtype, bias=True, seed=0):
    g = torch.Generator(device="cuda").manual_seed(seed)
    t = lambda *s, sc=1.0: (sc * torch.randn(*s, generator=g, device="cuda")).to(dtype)
    h, W, E = t(N, K), t(V, K, sc=2.0 / max(K, 1) ** 0.5), t(V, D)
    b = t(V, sc=0.5) if bias else None
    return h, W, E, b


def mask(N, frac, seed=1, device="cuda"):
    g = torch.Generator(device=device).manual_seed(seed)
    return (torch.rand(N, generator=g, device=device) >= frac).float()


def oracle(h, W, E, b, scale=1.0):
    """fp64 readout on the GPU (the oracle's formula), in blocks of rows."""
    xs = [x.to(f64) if x is not None else None for x in (h, W, E, b)]
    O, lse = [], []
    for i in range(0, h.shape[0], 2048):
        o, l = ref.softmax_readout_reference(xs[0][i:i + 2048], xs[1], xs[2], xs[3], logit_scale=scale, dtype=f64)
        O.append(o)
        lse.append(l)
    return torch.cat(O), torch.cat(lse)


def tol(cdt):
    return 1e-5 if cdt == torch.float32 else 1e-2


def check_active(h, W, E, b, weight, cdt, scale=1.0, chunk=8192):
    O, lse = _ops._forward_active(h, W, E, b, weight, scale, chunk, cdt)
    on = weight != 0
    assert torch.count_nonzero(O[~on]) == 0 and torch.count_nonzero(lse[~on]) == 0
    if int(on.sum()) == 0:
        return O, lse
    hs = h.to(cdt) if h.dtype != cdt else h
    Ws = W.to(cdt) if W.dtype != cdt else W
    Or, lr = oracle(hs[on], Ws, E.to(cdt), b, scale)
    assert rel_err(O[on], Or) < tol(cdt), rel_err(O[on], Or)
    assert rel_err(lse[on], lr) < tol(cdt) / 10, rel_err(lse[on], lr)
    return O, lse


CASES = [
    # (dtype, N, K, V, D): each forward tile family
    (torch.bfloat16, 3000, 256, 5000, 64),    # narrow tile, BM 256
    (torch.bfloat16, 2000, 128, 3000, 16),    # DP 32
    (torch.bfloat16, 1500, 128, 3000, 128),   # wide tile, BM 128
    (torch.bfloat16, 1500, 128, 3000, 256),   # E^T streamed through the ring
    (torch.float16, 1200, 64, 2500, 200),     # the same at D 200
    (torch.bfloat16, 700, 64, 2000, 300),     # two slices of E's columns
    (torch.float32, 900, 64, 1500, 64),
    (torch.float32, 700, 64, 1500, 200),      # fp32 slices of 128
]


@pytest.mark.parametrize("cdt,N,K,V,D", CASES, ids=lambda v: str(v).replace("torch.", ""))
@pytest.mark.parametrize("frac", [0.3, 0.9])
def test_active_forward_matches_the_oracle(cdt, N, K, V, D, frac):
    h, W, E, b = inputs(N, K, V, D, cdt, seed=N + D)
    check_active(h, W, E, b, mask(N, frac, seed=D), cdt)


def test_halving_the_active_blocks_resplits_the_vocabulary():
    """20000 tokens in 79 blocks, half of them masked: about 40 active blocks, so
    active_grid doubles the vocabulary splits; the partials then span the same buffer."""
    N, K, V, D = 20000, 128, 4096, 64
    h, W, E, b = inputs(N, K, V, D, torch.bfloat16, seed=5)
    for frac in (0.5, 0.75, 0.02):
        check_active(h, W, E, b, mask(N, frac, seed=int(frac * 100)), torch.bfloat16)


def test_fp32_storage_under_a_bf16_compute_dtype():
    h, W, E, b = inputs(1000, 96, 2000, 64, torch.float32, seed=2)
    w = mask(1000, 0.4)
    O, lse = _ops._forward_active(h, W, E, b, w, 1.0, 8192, torch.bfloat16)
    O2, lse2 = _ops._forward_active(h.bfloat16(), W.bfloat16(), E, b, w, 1.0, 8192, torch.bfloat16)
    assert torch.equal(O, O2) and torch.equal(lse, lse2)   # rounded while packing, as a pre-cast run
    check_active(h, W, E, b, w, torch.bfloat16)


def test_all_none_one_and_zero_hidden():
    h, W, E, b = inputs(600, 64, 1000, 32, torch.bfloat16, seed=3)
    O, lse = check_active(h, W, E, b, torch.zeros(600, device="cuda"), torch.bfloat16)
    assert torch.count_nonzero(O) == 0 and torch.count_nonzero(lse) == 0
    check_active(h, W, E, b, torch.ones(600, device="cuda"), torch.bfloat16)
    one = torch.zeros(600, device="cuda")
    one[417] = 0.25
    check_active(h, W, E, b, one, torch.bfloat16)
    h0, W0, E0, b0 = inputs(300, 0, 800, 16, torch.bfloat16, seed=4)
    check_active(h0, W0, E0, b0, mask(300, 0.5), torch.bfloat16)     # K = 0: bias-only scores


def test_masked_rows_and_padding_tail_of_a_batched_input():
    """Config 5's weight shape at a small size: leading dims (8, T) with a ragged padded tail."""
    T, K, V, D = 512, 128, 4000, 256
    h, W, E, b = inputs(8 * T, K, V, D, torch.bfloat16, seed=9)
    g = torch.Generator(device="cuda").manual_seed(3)
    tails = torch.randint(0, 129, (8,), device="cuda", generator=g)
    w = (torch.arange(T, device="cuda")[None, :] < (T - tails)[:, None]).float()
    target = torch.randn(8, T, D, device="cuda", generator=g)
    xs = [x.requires_grad_(True) for x in (h.view(8, T, K), W, E, b)]
    loss = swvr.softmax_readout_mse(xs[0], xs[1], xs[2], target, xs[3], weight=w, z_loss_weight=1e-4)
    grads = torch.autograd.grad(loss, xs)
    c = [x.detach().to(f64).requires_grad_(True) for x in (h, W, E, b)]
    O, lse = ref.softmax_readout_reference(*c, dtype=f64)
    per = ((O - target.reshape(-1, D).to(f64)) ** 2).mean(-1) + 1e-4 * lse ** 2
    want = (per * w.reshape(-1).to(f64)).sum() / w.sum().to(f64)
    wg = torch.autograd.grad(want, c)
    assert rel_err(loss, want) < 1e-2
    for a, r in zip(grads, wg):
        assert rel_err(a.reshape(r.shape), r) < 2e-2


def composite(h, W, E, b, target, weight, z, reduction, scale=1.0):
    """The reference's loss in fp64 (swvr/api.py:53-66) over the oracle's readout."""
    O, lse = ref.softmax_readout_reference(*(x.cpu().to(f64) if x is not None else None for x in (h, W, E, b)),
                                           logit_scale=scale, dtype=f64)
    per = (O - target.cpu().to(f64)).pow(2).mean(-1) + z * lse.pow(2)
    per = per * weight.cpu().to(f64)
    if reduction == "none":
        return per
    return per.sum() if reduction == "sum" else per.sum() / weight.cpu().to(f64).sum()


def same_nan_pattern_and_values(got, want):
    got, want = got.detach().cpu().to(f64), want.detach().to(f64)
    assert torch.equal(torch.isnan(got), torch.isnan(want)), (got, want)
    fin = ~torch.isnan(want)
    if fin.any():
        assert rel_err(got[fin], want[fin]) < 1e-2 or torch.allclose(got[fin], want[fin], atol=1e-6)


def poison(kind, h, W, E, b, target, w):
    h, W, E, b, target, w = (x.clone() if x is not None else None for x in (h, W, E, b, target, w))
    scale = 1.0
    if kind == "h_nan_masked":
        w[5] = 0
        h[5, 3] = float("nan")
    elif kind == "h_inf_masked":
        w[7] = 0
        h[7, 0] = float("inf")
    elif kind == "W_nan":
        W[11, 2] = float("nan")
    elif kind == "E_inf":
        E[3, 1] = float("inf")
    elif kind == "bias_nan":
        b[2] = float("nan")
    elif kind == "bias_all_neg_inf":
        b.fill_(float("-inf"))
    elif kind == "bias_some_neg_inf":
        b[::3] = float("-inf")
    elif kind == "target_inf_masked":
        w[9] = 0
        target[9, 0] = float("inf")
    elif kind == "weight_nan":
        w[4] = float("nan")
    elif kind == "scale_inf":
        scale = math.inf
    return h, W, E, b, target, w, scale


KINDS = ["h_nan_masked", "h_inf_masked", "W_nan", "E_inf", "bias_nan", "bias_all_neg_inf", "bias_some_neg_inf",
         "target_inf_masked", "weight_nan", "scale_inf"]


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("reduction", ["none", "sum"])
def test_non_finite_inputs_give_the_reference_nans(kind, reduction):
    N, K, V, D = 64, 32, 300, 8
    h, W, E, b = inputs(N, K, V, D, torch.float32, seed=11)
    g = torch.Generator(device="cuda").manual_seed(12)
    target = torch.randn(N, D, device="cuda", generator=g)
    w = mask(N, 0.3, seed=13)
    h, W, E, b, target, w, scale = poison(kind, h, W, E, b, target, w)
    got = swvr.softmax_readout_mse(h, W, E, target, b, weight=w, z_loss_weight=1e-3, reduction=reduction,
                                   logit_scale=scale)
    want = composite(h, W, E, b, target, w, 1e-3, reduction, scale)
    same_nan_pattern_and_values(got, want)


def test_the_loss_takes_the_active_forward_only_where_it_is_exact():
    from swvr_amd.api import _skips_zero_weight
    h, W, E, b = inputs(64, 32, 300, 8, torch.bfloat16)
    w = mask(64, 0.3)
    assert _skips_zero_weight(h, W, w, "mean")
    assert not _skips_zero_weight(h, W, w.requires_grad_(True), "mean")    # d loss / d w needs every row
    assert not _skips_zero_weight(h, W, w.detach()[:32], "mean")           # broadcasting weight
    assert not _skips_zero_weight(h, W, None, "mean")
    assert not _skips_zero_weight(h.double(), W.double(), w.detach(), "mean")  # fp64: the fp64 path
    assert not _skips_zero_weight(h, W, w.detach(), "max")                 # unknown reduction: its error
