"""Pins the CPU oracle (oracle/) before anything is checked against it.

  * golden fixtures (tests/golden/readout_cases.json, pure-Python fp64 with
    finite-difference-checked gradients) — forward, gradients, MSE loss;
  * closed forms: V = 1, constant scores, a dominant bias, the naive formula;
  * gradcheck of the closed form in fp64;
  * the chunked restatement against the eager closed form, over the
    behaviours of the reference's tests/test_cpu.py (chunk sizes, scales,
    masked vocabulary, large logits, frozen inputs, tied W = E, fp32, bf16);
  * planted mistakes in a copy of the oracle's math must fail the fixtures.
"""
import json
import math
import os

import pytest
import torch

from oracle import chunked
from oracle import reference as ref

f64 = torch.float64
GOLD = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "readout_cases.json")))["cases"]
CASES = {c["name"]: c for c in GOLD}


def T(x):
    return None if x is None else torch.tensor(x, dtype=f64)


def inputs_of(c):
    return T(c["h"]), T(c["W"]), T(c["E"]), T(c["bias"])


def close(a, b, rtol=1e-10, atol=1e-10):
    torch.testing.assert_close(a, b, rtol=rtol, atol=atol)


@pytest.mark.parametrize("name", list(CASES))
def test_reference_forward_matches_golden(name):
    c = CASES[name]
    O, lse = ref.softmax_readout_reference(*inputs_of(c), logit_scale=c["logit_scale"])
    close(O, T(c["O"]))
    close(lse, T(c["lse"]))


@pytest.mark.parametrize("name", list(CASES))
def test_reference_gradients_match_golden(name):
    c = CASES[name]
    h, W, E, b = inputs_of(c)
    out = ref.reference_grads(h, W, E, b, T(c["gO"]), T(c["glse"]), c["logit_scale"])
    for got, key in zip(out, ["O", "lse", "gh", "gW", "gE", "gb"]):
        if c[key] is None:
            assert got is None
        else:
            close(got, T(c[key]), rtol=1e-9, atol=1e-9)


@pytest.mark.parametrize("name", list(CASES))
@pytest.mark.parametrize("chunk", [1, 2, 3, 1000])
def test_chunked_matches_golden(name, chunk):
    c = CASES[name]
    h, W, E, b = inputs_of(c)
    s = c["logit_scale"]
    O, lse = chunked.forward(h, W, E, b, s, chunk)
    close(O, T(c["O"]))
    close(lse, T(c["lse"]))
    gh, gW, gE, gb = chunked.backward(T(c["gO"]), T(c["glse"]), h, W, E, b, O, lse, s, chunk)
    for got, key in zip((gh, gW, gE, gb), ["gh", "gW", "gE", "gb"]):
        if c[key] is None:
            assert got is None
        else:
            close(got, T(c[key]), rtol=1e-9, atol=1e-9)


def test_mse_matches_golden():
    c = CASES["mse"]
    h, W, E, b = inputs_of(c)
    kw = dict(weight=T(c["weight"]), z_loss_weight=c["z_loss_weight"], logit_scale=c["logit_scale"])
    for red, want in c["mse"].items():
        got = ref.mse_reference(h, W, E, T(c["target"]), b, reduction=red, **kw)
        close(got, T(want))
    got = ref.mse_reference(h, W, E, T(c["target"]), b, z_loss_weight=c["z_loss_weight"],
                            logit_scale=c["logit_scale"])
    close(got, T(c["mse_unweighted_mean"]))


@pytest.mark.parametrize("name", list(CASES))
@pytest.mark.parametrize("block", [1, 2, 1024])
def test_blocked_reference_matches_golden(name, block):
    """The row-blocked evaluation the full-size GPU tests use gives the golden values."""
    c = CASES[name]
    h, W, E, b = inputs_of(c)
    out = ref.reference_grads_blocked(h, W, E, b, T(c["gO"]), T(c["glse"]), c["logit_scale"], block=block)
    for got, key in zip(out, ["O", "lse", "gh", "gW", "gE", "gb"]):
        if c[key] is None:
            assert got is None
        else:
            close(got, T(c[key]), rtol=1e-9, atol=1e-9)


@pytest.mark.parametrize("reduction", ["sum", "mean"])
@pytest.mark.parametrize("block", [1, 4, 1024])
def test_blocked_mse_matches_golden_and_autograd(reduction, block):
    c = CASES["mse"]
    h, W, E, b = inputs_of(c)
    t, w, z, s = T(c["target"]), T(c["weight"]), c["z_loss_weight"], c["logit_scale"]
    loss, *grads = ref.mse_grads_blocked(h, W, E, t, b, weight=w, reduction=reduction, z_loss_weight=z,
                                         logit_scale=s, block=block)
    close(loss, T(c["mse"][reduction]))
    xs = [x.clone().requires_grad_(True) for x in (h, W, E, b)]
    want = torch.autograd.grad(ref.mse_reference(*xs[:3], t, xs[3], weight=w, reduction=reduction,
                                                 z_loss_weight=z, logit_scale=s), xs)
    for got, r in zip(grads, want):
        close(got, r)
    with pytest.raises(ValueError):
        ref.mse_grads_blocked(h, W, E, t, b, reduction="none")


def test_blocked_reference_has_no_cross_block_terms():
    """A planted mistake: a block size that drops the last partial block must not pass."""
    h, W, E, b = make(N=7)
    gO, glse = torch.randn(7, 5, dtype=f64), torch.randn(7, dtype=f64)
    full = ref.reference_grads(h, W, E, b, gO, glse)
    blocked = ref.reference_grads_blocked(h, W, E, b, gO, glse, block=3)
    for a, r in zip(blocked, full):
        close(a, r)
    dropped = ref.reference_grads_blocked(h[:6], W, E, b, gO[:6], glse[:6], block=3)
    assert not torch.allclose(dropped[3], full[3])


def make(N=6, K=12, V=41, D=5, dtype=f64, bias=True, seed=0):
    g = torch.Generator().manual_seed(seed)
    t = lambda *s: torch.randn(*s, generator=g, dtype=f64).to(dtype)
    return t(N, K), t(V, K), t(V, D), (t(V) if bias else None)


def test_single_vocab_closed_form():
    h, W, E, b = make(V=1)
    O, lse = ref.softmax_readout_reference(h, W, E, b, logit_scale=0.3)
    close(O, E[0].expand_as(O))
    close(lse, 0.3 * (h @ W[0]) + b[0])


def test_constant_scores_closed_form():
    h, _, E, _ = make(V=9)
    W = torch.zeros(9, h.shape[1], dtype=f64)
    O, lse = ref.softmax_readout_reference(h, W, E)
    close(O, E.mean(0).expand_as(O))
    close(lse, torch.full((h.shape[0],), math.log(9), dtype=f64))


def test_dominant_bias_closed_form():
    h, W, E, b = make()
    b[3], b[7] = 1e4, -1e4
    O, lse = ref.softmax_readout_reference(h, W, E, b)
    close(O, E[3].expand_as(O))
    close(lse, h @ W[3] + b[3])


def test_naive_formula():
    h, W, E, b = make(N=10)
    O, lse = ref.softmax_readout_reference(h, W, E, b, logit_scale=0.5)
    S = 0.5 * torch.einsum("nk,vk->nv", h, W) + b
    close(O, (S.exp() / S.exp().sum(-1, keepdim=True)) @ E)
    close(lse, S.exp().sum(-1).log())


@pytest.mark.parametrize("bias", [True, False])
@pytest.mark.parametrize("scale", [1.0, 0.3, 2.5])
def test_reference_gradcheck(bias, scale):
    xs = [x.requires_grad_(True) if x is not None else None for x in make(N=4, K=6, V=13, D=3, bias=bias)]
    fn = lambda *a: ref.softmax_readout_reference(*a, logit_scale=scale)
    assert torch.autograd.gradcheck(fn, tuple(xs))


# ---- the chunked restatement against the eager closed form


def ref_and_chunked(h, W, E, b, scale=1.0, chunk=8, seed=1, needs=(True, True, True, True)):
    g = torch.Generator().manual_seed(seed)
    N, D = h.shape[0], E.shape[1]
    gO = torch.randn(N, D, generator=g, dtype=f64)
    glse = torch.randn(N, generator=g, dtype=f64)
    want = ref.reference_grads(h, W, E, b, gO, glse, scale, dtype=f64)
    O, lse = chunked.forward(h, W, E, b, scale, chunk)
    got = (O, lse, *chunked.backward(gO.to(O.dtype), glse.to(O.dtype), h, W, E, b, O, lse, scale, chunk,
                                     need_h=needs[0], need_W=needs[1], need_E=needs[2], need_b=needs[3]))
    return got, want


@pytest.mark.parametrize("chunk", [1, 3, 8, 40, 41, 42, 1000])
def test_chunked_chunk_sizes(chunk):
    got, want = ref_and_chunked(*make(), chunk=chunk)
    for a, r in zip(got, want):
        close(a, r)


@pytest.mark.parametrize("scale", [0.3, 2.5])
def test_chunked_scales(scale):
    got, want = ref_and_chunked(*make(), scale=scale, chunk=7)
    for a, r in zip(got, want):
        close(a, r)


def test_chunked_masked_vocab():
    h, W, E, b = make(V=40)
    b[:16] = float("-inf")  # two fully masked chunks come first
    b[30:] = float("-inf")
    got, want = ref_and_chunked(h, W, E, b, chunk=8)
    for a, r in zip(got, want):
        close(a, r)
    assert (got[5][:16] == 0).all() and (got[5][30:] == 0).all()


def test_chunked_large_logits():
    h, W, E, b = make()
    b[3], b[7] = 1e4, -1e4
    got, want = ref_and_chunked(h, W, E, b)
    for a, r in zip(got, want):
        close(a, r)
    close(got[0], E[3].expand_as(got[0]))


@pytest.mark.parametrize("frozen", ["h", "W", "E", "b", "WE"])
def test_chunked_frozen_inputs(frozen):
    needs = tuple(k not in frozen for k in "hWEb")
    got, want = ref_and_chunked(*make(), needs=needs)
    for a, r, need in zip(got[2:], want[2:], needs):
        if need:
            close(a, r)
        else:
            assert a is None


def test_chunked_tied_W_and_E():
    h, W, _, b = make(K=7, D=7)
    g = torch.Generator().manual_seed(3)
    gO, glse = torch.randn(6, 7, generator=g, dtype=f64), torch.randn(6, generator=g, dtype=f64)
    Wt = W.clone().requires_grad_(True)
    O, lse = ref.softmax_readout_reference(h, Wt, Wt, b)
    (gtied,) = torch.autograd.grad((O * gO).sum() + (lse * glse).sum(), Wt)
    O2, lse2 = chunked.forward(h, W, W, b, 1.0, 8)
    _, gW, gE, _ = chunked.backward(gO, glse, h, W, W, b, O2, lse2, 1.0, 8)
    close(gW + gE, gtied)


def test_chunked_fp32_inputs():
    h, W, E, b = make(dtype=torch.float32)
    O, lse = chunked.forward(h, W, E, b, 1.0, 8)
    Or, lr = ref.softmax_readout_reference(h.double(), W.double(), E.double(), b.double())
    torch.testing.assert_close(O.double(), Or, rtol=1e-4, atol=1e-5)
    torch.testing.assert_close(lse.double(), lr, rtol=1e-4, atol=1e-5)


def test_chunked_bf16_inputs_return_fp32():
    h, W, E, b = make(dtype=torch.bfloat16, K=32, V=300)
    O, lse = chunked.forward(h, W, E, b, 1.0, 64)
    assert O.dtype == torch.float32 and lse.dtype == torch.float32
    Or, lr = ref.softmax_readout_reference(*(x.double() for x in (h, W, E, b)))
    torch.testing.assert_close(lse.double(), lr, rtol=1e-3, atol=1e-2)
    torch.testing.assert_close(O.double(), Or, rtol=2e-2, atol=2e-2)


# ---- planted mistakes: a plausible slip in the backward math must fail the fixtures


def _grads_with(c, mutate):
    h, W, E, b = inputs_of(c)
    s = c["logit_scale"]
    gO, glse = T(c["gO"]), T(c["glse"])
    S = s * h @ W.T + (b if b is not None else 0)
    lse = torch.logsumexp(S, -1)
    P = torch.exp(S - lse[:, None])
    O = P @ E
    delta = (O * gO).sum(1) - glse
    dS = P * (gO @ E.T - delta[:, None])
    grads = dict(gh=s * dS @ W, gW=s * dS.T @ h, gE=P.T @ gO, gb=dS.sum(0))
    mutate(grads, locals())
    return grads


@pytest.mark.parametrize("mistake", ["drop_glse", "no_scale_on_gW", "transposed_gE", "sign_of_delta"])
def test_planted_mistakes_fail_the_fixtures(mistake):
    c = CASES["basic"]

    def mutate(g, v):
        if mistake == "drop_glse":
            d = (v["O"] * v["gO"]).sum(1)
            dS = v["P"] * (v["gO"] @ v["E"].T - d[:, None])
            g["gh"] = v["s"] * dS @ v["W"]
        elif mistake == "no_scale_on_gW":
            g["gW"] = v["dS"].T @ v["h"]
        elif mistake == "transposed_gE":
            g["gE"] = (v["gO"].T @ v["P"]).T.flip(0)
        elif mistake == "sign_of_delta":
            dS = v["P"] * (v["gO"] @ v["E"].T + v["delta"][:, None])
            g["gb"] = dS.sum(0)

    clean = _grads_with(c, lambda g, v: None)
    for k in clean:
        close(clean[k], T(c[k]), rtol=1e-9, atol=1e-9)
    bad = _grads_with(c, mutate)
    assert any(not torch.allclose(bad[k], T(c[k]), rtol=1e-6, atol=1e-6) for k in bad)
