"""Vocabulary-parallel building blocks on one GPU: shard partials, combine, shard backward.

The vocabulary is split into uneven shards; each shard's partials
(swvr_fwd_partial) merged by swvr_combine must give softmax_readout's O and
lse for the whole vocabulary, and each shard's backward (swvr_bwd with the
merged O and lse) its rows of gW, gE, gb and a term of gh whose sum is the
whole gh.  Pinned against the fp64 closed form (oracle.reference) and against
the single-call path.
"""
import math

import pytest
import torch

import swvr_amd as swvr
from swvr_amd import _lib
from swvr_amd import vocab_shard as vs
from oracle import reference as ref

pytestmark = pytest.mark.gpu


def inputs(N, K, V, D, dtype, seed=0):
    g = torch.Generator().manual_seed(seed)
    t = lambda *s, sc=1.0: (sc * torch.randn(*s, generator=g, dtype=torch.float64)).to("cuda", dtype)
    return t(N, K), t(V, K, sc=K ** -0.5), t(V, D), t(V, sc=0.5)


def shard_forward(h, W, E, b, bounds):
    parts = [vs.softmax_readout_partial(h, W[a:z], E[a:z], b[a:z]) for a, z in zip(bounds[:-1], bounds[1:])]
    m, l, acc = (torch.stack(x) for x in zip(*parts))
    return vs.combine_partials(m, l, acc)


BOUNDS = [0, 1200, 2501, 3700, 5003]


@pytest.mark.parametrize("D", [64, 128, 200])
@pytest.mark.parametrize("dtype,tol", [(torch.float32, 2e-5), (torch.bfloat16, 1e-2)])
def test_shards_combine_to_the_whole_vocabulary(dtype, tol, D):
    # D = 128 and 200 (bf16) run the streamed-E^T forward for each shard
    N, K, V = 700, 256, 5003
    h, W, E, b = inputs(N, K, V, D, dtype)
    O, lse = shard_forward(h, W, E, b, BOUNDS)
    O1, lse1 = swvr.softmax_readout(h, W, E, b)
    O_r, lse_r = ref.softmax_readout_reference(*(x.double() for x in (h, W, E, b)))
    rel = lambda a, r: ((a.double() - r.double()).norm() / r.double().norm()).item()
    for a, r in ((O, O_r), (lse, lse_r), (O1, O_r)):
        assert rel(a, r) <= tol
    if dtype == torch.float32:
        torch.testing.assert_close(O, O1, rtol=1e-5, atol=1e-5)
        torch.testing.assert_close(lse, lse1, rtol=1e-6, atol=1e-5)
    else:
        # P is rounded to bf16 relative to the running maximum, which differs between
        # a shard and the whole vocabulary: agreement at bf16 rounding level
        assert rel(O, O1) <= 5e-3 and rel(lse, lse1) <= 1e-5


def test_one_shard_is_the_forward_and_a_masked_shard_drops_out():
    N, K, V, D = 300, 64, 900, 16
    h, W, E, b = inputs(N, K, V, D, torch.float32)
    O1, lse1 = swvr.softmax_readout(h, W, E, b)
    O, lse = shard_forward(h, W, E, b, [0, V])
    torch.testing.assert_close(O, O1, rtol=1e-6, atol=1e-6)
    torch.testing.assert_close(lse, lse1, rtol=1e-6, atol=1e-6)
    bm = b.clone()
    bm[300:600] = float("-inf")             # the middle shard is fully masked
    m, l, acc = vs.softmax_readout_partial(h, W[300:600], E[300:600], bm[300:600])
    assert torch.isneginf(m).all() and (l == 0).all() and (acc == 0).all()
    O, lse = shard_forward(h, W, E, bm, [0, 300, 600, V])
    O1, lse1 = swvr.softmax_readout(h, W, E, bm)
    torch.testing.assert_close(O, O1, rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(lse, lse1, rtol=1e-6, atol=1e-5)


def test_shard_backward_sums_to_the_whole_gradient():
    N, K, V, D = 700, 256, 5003, 64
    h, W, E, b = inputs(N, K, V, D, torch.float32)
    g = torch.Generator().manual_seed(3)
    gO = torch.randn(N, D, generator=g, dtype=torch.float64).to("cuda", torch.float32)
    glse = (0.3 * torch.randn(N, generator=g, dtype=torch.float64)).to("cuda", torch.float32)
    O, lse = shard_forward(h, W, E, b, BOUNDS)
    gh = torch.zeros_like(h)
    gW, gE, gb = [], [], []
    for a, z in zip(BOUNDS[:-1], BOUNDS[1:]):
        s = vs.shard_backward(gO, glse, h, W[a:z], E[a:z], b[a:z], O, lse, chunk_size=1024)
        gh += s[0]
        gW.append(s[1])
        gE.append(s[2])
        gb.append(s[3])
    xs = [x.detach().clone().requires_grad_(True) for x in (h, W, E, b)]
    O1, lse1 = swvr.softmax_readout(*xs, chunk_size=1024)
    want = torch.autograd.grad((O1 * gO).sum() + (lse1 * glse).sum(), xs)
    got = (gh, torch.cat(gW), torch.cat(gE), torch.cat(gb))
    for a, r in zip(got, want):
        torch.testing.assert_close(a, r, rtol=1e-4, atol=1e-5)


def _rel(a, r):
    a, r = a.detach().double(), r.detach().double().to(a.device)
    return ((a - r).norm() / r.norm().clamp_min(1e-30)).item()


def _cos(a, r):
    a, r = a.detach().double().flatten(), r.detach().double().to(a.device).flatten()
    return (a @ r / (a.norm() * r.norm()).clamp_min(1e-300)).item()


# (tag, dtype, N, K, V, D, shard bounds, chunk): uneven shards with a partial last chunk, and shards
# of whole 8192-row chunks over 17 token blocks of 256, so that every scores workgroup of a full chunk
# walks two or more blocks (the backward's steady-state loop, swvr_bwd_tiling)
SHARD_CASES = [
    ("small-f32", torch.float32, 700, 256, 5003, 64, BOUNDS, 1024),
    ("small-bf16", torch.bfloat16, 700, 256, 5003, 64, BOUNDS, 1024),
    ("wide-bf16", torch.bfloat16, 700, 256, 5003, 128, BOUNDS, 1024),  # wide scores kernel, dE^T pieces
    ("multiblock-bf16", torch.bfloat16, 4096 + 77, 256, 16384 + 300, 64, [0, 8192, 16384 + 300], 8192),
    ("multiblock-f32", torch.float32, 2048 + 9, 128, 16384, 64, [0, 8192, 16384], 8192),
]


@pytest.mark.parametrize("tag,dtype,N,K,V,D,bounds,chunk", SHARD_CASES, ids=[c[0] for c in SHARD_CASES])
def test_shard_backward_matches_the_oracle(tag, dtype, N, K, V, D, bounds, chunk):
    """Each shard's gW, gE, gb rows and the sum of the shards' gh against the fp64 closed form of the
    whole vocabulary (swvr/reference.py:5-14 differentiated; the reference computes these with
    swvr/chunked.py:108-151 over the whole vocabulary), at the north-star bars."""
    h, W, E, b = inputs(N, K, V, D, dtype, seed=5)
    g = torch.Generator().manual_seed(7)
    gO = torch.randn(N, D, generator=g, dtype=torch.float64).to("cuda", torch.float32)
    glse = (0.3 * torch.randn(N, generator=g, dtype=torch.float64)).to("cuda", torch.float32)
    if tag.startswith("multiblock"):
        for a, z in zip(bounds[:-1], bounds[1:]):
            t = _lib.bwd_tiling(dtype, N, K, z - a, D, chunk)
            assert math.ceil(N / t["BM"]) >= 2 * t["G"], (t, N)
    O, lse = shard_forward(h, W, E, b, bounds)
    gh = torch.zeros(N, K, dtype=torch.float64, device="cuda")
    parts = []
    for a, z in zip(bounds[:-1], bounds[1:]):
        s = vs.shard_backward(gO, glse, h, W[a:z], E[a:z], b[a:z], O, lse, chunk_size=chunk)
        gh += s[0].double()
        parts.append((a, z, s[1], s[2], s[3]))
    torch.cuda.synchronize()
    O_r, lse_r, gh_r, gW_r, gE_r, gb_r = ref.reference_grads_blocked(h, W, E, b, gO, glse, block=1024)
    lo = dtype != torch.float32
    tol_out, tol_grad, min_cos = (1e-2, 2e-2, 0.999) if lo else (1e-5, 1e-4, 0.999999)
    errs = {"O": _rel(O, O_r), "lse": _rel(lse, lse_r), "gh": _rel(gh, gh_r)}
    cos = {"gh": _cos(gh, gh_r)}
    for i, (a, z, gW, gE, gb) in enumerate(parts):
        for n, x, r in (("gW", gW, gW_r[a:z]), ("gE", gE, gE_r[a:z]), ("gb", gb, gb_r[a:z])):
            assert x.dtype == dtype and torch.isfinite(x).all(), (tag, i, n)
            errs[f"{n}{i}"], cos[f"{n}{i}"] = _rel(x, r), _cos(x, r)
    print(tag, {k: f"{v:.1e}" for k, v in errs.items()}, flush=True)
    assert errs["O"] <= tol_out and errs["lse"] <= tol_out, errs
    for n in errs:
        if n not in ("O", "lse"):
            assert errs[n] <= tol_grad and cos[n] >= min_cos, (tag, n, errs[n], cos[n])
