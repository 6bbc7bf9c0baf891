"""The reference's CPU test behaviours (tests/test_cpu.py) run through the HIP path.

The reference checks these in fp64 on the CPU; this build has no CPU path and
its fp64 is not supported, so they run in fp32 on the GPU against the fp64
oracle with fp32-sized tolerances, plus the golden fixtures.
"""
import json
import os

import pytest
import torch
from torch import nn

import swvr_amd as swvr
from oracle import reference as ref
from tests.gpu_util import rel_err

pytestmark = pytest.mark.gpu
f32, f64 = torch.float32, torch.float64
TOL = dict(rtol=2e-5, atol=2e-5)


def make(N=6, K=12, V=41, D=5, dtype=f32, bias=True, lead=None, seed=0):
    g = torch.Generator().manual_seed(seed)
    shape = (*(lead or (N,)), K)
    t = lambda *s: torch.randn(*s, generator=g, dtype=f64).to(device="cuda", dtype=dtype)
    h, W, E = t(*shape), t(V, K), t(V, D)
    b = t(V) if bias else None
    for x in (h, W, E, b):
        if x is not None:
            x.requires_grad_(True)
    return h, W, E, b


def grads(fn, inputs, seed=1):
    outs = fn(*inputs)
    g = torch.Generator().manual_seed(seed)
    loss = sum((o * torch.randn(o.shape, generator=g, dtype=f64).to(o)).sum() for o in outs)
    xs = [x for x in inputs if x is not None and x.requires_grad]
    return outs, torch.autograd.grad(loss, xs, allow_unused=True)


def oracle_grads(inputs, scale=1.0, seed=1):
    """fp64 CPU copies that keep tied inputs tied (the same tensor passed twice)."""
    copies = {}
    for x in inputs:
        if x is not None and id(x) not in copies:
            copies[id(x)] = x.detach().cpu().double().requires_grad_(x.requires_grad)
    cpu = [copies[id(x)] if x is not None else None for x in inputs]
    return grads(lambda *a: ref.softmax_readout_reference(*a, logit_scale=scale), cpu, seed)


def assert_matches_oracle(h, W, E, b, scale=1.0, chunk=8, tol=TOL):
    (o1, g1) = grads(lambda *a: swvr.softmax_readout(*a, logit_scale=scale, chunk_size=chunk), (h, W, E, b))
    (o2, g2) = oracle_grads((h, W, E, b), scale)
    for a, r in zip(o1, o2):
        torch.testing.assert_close(a.double().cpu(), r, **tol)
    for a, r in zip(g1, g2):
        torch.testing.assert_close(a.double().cpu(), r, **tol)


@pytest.mark.parametrize("chunk", [1, 3, 8, 40, 41, 42, 1000])
def test_chunk_sizes_match_oracle(chunk):
    assert_matches_oracle(*make(), chunk=chunk)


@pytest.mark.parametrize("bias", [True, False])
@pytest.mark.parametrize("scale", [1.0, 0.3, 2.5])
def test_scales_and_bias(bias, scale):
    assert_matches_oracle(*make(N=4, K=6, V=13, D=3, bias=bias), scale=scale, chunk=5)


def test_leading_dims():
    h, W, E, b = make(lead=(2, 3, 4))
    O, lse = swvr.softmax_readout(h, W, E, b, chunk_size=7)
    assert O.shape == (2, 3, 4, 5) and lse.shape == (2, 3, 4)
    assert_matches_oracle(h, W, E, b)


def test_non_contiguous_h():
    h, W, E, b = make(N=8)
    h_t = h.detach().t().contiguous().t()[::2].requires_grad_(True)
    assert not h_t.is_contiguous()
    assert_matches_oracle(h_t, W, E, b)


def test_empty_batch():
    h, W, E, b = make(N=0)
    O, lse = swvr.softmax_readout(h, W, E, b, chunk_size=8)
    assert O.shape == (0, 5) and lse.shape == (0,)
    (O.sum() + lse.sum()).backward()
    assert W.grad.abs().sum() == 0 and E.grad.abs().sum() == 0 and b.grad.abs().sum() == 0


def test_single_token_and_tiny_vocab():
    assert_matches_oracle(*make(N=1, V=1), chunk=8)
    assert_matches_oracle(*make(N=1, V=2), chunk=1)


def test_large_logits_no_overflow():
    h, W, E, b = make()
    with torch.no_grad():
        b[3] = 1e4
        b[7] = -1e4
    assert_matches_oracle(h, W, E, b)
    O, _ = swvr.softmax_readout(h, W, E, b, chunk_size=8)
    torch.testing.assert_close(O, E[3].expand_as(O).detach())


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "f16"])
@pytest.mark.parametrize("D", [16, 64, 128])
def test_large_logits_low_precision(dtype, D):
    """Logits near 1e4 in the 2-byte dtypes: an fp32 bias of 1e4 + N(0, 0.5) on every row leaves the
    softmax as well conditioned as N(0, 0.5) logits, while the exponent arithmetic runs at 1e4
    (the ring scores kernel, D <= 64, forms P in base 2; the wide one, D = 128, in natural units).
    Outputs and gradients at the low-precision bar against the fp64 closed form."""
    N, K, V = 700, 128, 1000
    g = torch.Generator(device="cuda").manual_seed(D)
    h = torch.randn(N, K, device="cuda", generator=g).to(dtype)
    W = (torch.randn(V, K, device="cuda", generator=g) * K ** -0.5).to(dtype)
    E = torch.randn(V, D, device="cuda", generator=g).to(dtype)
    b = 1e4 + 0.5 * torch.randn(V, device="cuda", generator=g)
    gO = torch.randn(N, D, device="cuda", generator=g)
    glse = torch.randn(N, device="cuda", generator=g)
    xs = [x.requires_grad_(True) for x in (h, W, E, b)]
    O, lse = swvr.softmax_readout(*xs, chunk_size=512)
    got = [O, lse, *torch.autograd.grad((O * gO).sum() + (lse * glse).sum(), xs)]
    cpu = [x.detach().double().cpu().requires_grad_(True) for x in xs]
    Or, lr = ref.softmax_readout_reference(*cpu, dtype=f64)
    want = [Or, lr, *torch.autograd.grad((Or * gO.double().cpu()).sum() + (lr * glse.double().cpu()).sum(), cpu)]
    for n, a, r in zip(("O", "lse", "gh", "gW", "gE", "gb"), got, want):
        a = a.detach().double().cpu()
        e = rel_err(a, r)
        cos = (a.flatten() @ r.flatten() / (a.norm() * r.norm())).item()
        assert e <= (1e-2 if n in ("O", "lse") else 2e-2) and cos >= 0.999, (n, e, cos)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "f16"])
@pytest.mark.parametrize("D", [64, 129, 300])
def test_one_vocabulary_row_with_all_of_p_in_low_precision(dtype, D):
    """V = 1 (P = 1 for every token), and a vocabulary whose first row takes nearly all of P: dP and
    delta then nearly cancel and dS is about glse alone.  The gradients still meet the low-precision
    bar against the fp64 formula (rel err <= 2e-2, cosine >= 0.999), because delta sums gO rounded to
    the compute dtype, as dP uses it; the reference's unrounded delta (swvr/chunked.py:113) misses
    it by 2-7% in gh and gb at D = 300 in bf16."""
    N, K = 1500, 216
    for V, lead in ((1, None), (64, 30.0)):
        g = torch.Generator(device="cuda").manual_seed(D + V)
        h = torch.randn(N, K, device="cuda", generator=g).to(dtype)
        W = (torch.randn(V, K, device="cuda", generator=g) * K ** -0.5).to(dtype)
        E = torch.randn(V, D, device="cuda", generator=g).to(dtype)
        b = 0.3 * torch.randn(V, device="cuda", generator=g)
        if lead is not None:
            b[0] = lead
        b = b.to(dtype)
        gO = torch.randn(N, D, device="cuda", generator=g)
        glse = torch.randn(N, device="cuda", generator=g)
        xs = [x.requires_grad_(True) for x in (h, W, E, b)]
        O, lse = swvr.softmax_readout(*xs, chunk_size=1000)
        got = torch.autograd.grad((O * gO).sum() + (lse * glse).sum(), xs)
        c = [x.detach().double().requires_grad_(True) for x in xs]
        Or, lr = ref.softmax_readout_reference(*c, dtype=f64)
        want = torch.autograd.grad((Or * gO.double()).sum() + (lr * glse.double()).sum(), c)
        for name, a, r in zip(("gh", "gW", "gE", "gb"), got, want):
            e = rel_err(a, r)
            cos = torch.nn.functional.cosine_similarity(a.double().flatten(), r.flatten(), dim=0).item()
            assert e <= 2e-2 and cos >= 0.999, (V, name, e, cos)


def test_masked_vocab_with_neg_inf_bias():
    h, W, E, b = make(V=40)
    with torch.no_grad():
        b[:16] = float("-inf")
        b[30:] = float("-inf")
    O, lse = swvr.softmax_readout(h, W, E, b, chunk_size=8)
    cpu = [x.detach().cpu().double() for x in (h, W, E, b)]
    O_r, lse_r = ref.softmax_readout_reference(*cpu)
    torch.testing.assert_close(O.double().cpu(), O_r, **TOL)
    torch.testing.assert_close(lse.double().cpu(), lse_r, **TOL)
    (_, gs) = grads(lambda *a: swvr.softmax_readout(*a, chunk_size=8), (h, W, E, b))
    (_, gs_r) = oracle_grads((h, W, E, b))
    for a, r in zip(gs, gs_r):
        torch.testing.assert_close(a.double().cpu(), r, **TOL)
    assert (gs[3][:16] == 0).all() and (gs[3][30:] == 0).all()


def test_fully_masked_row_matches_reference_nan():
    h, W, E, b = make(V=10)
    with torch.no_grad():
        b[:] = float("-inf")
    O, lse = swvr.softmax_readout(h, W, E, b)
    assert torch.isnan(O).all() and torch.isneginf(lse).all()


@pytest.mark.parametrize("frozen", ["h", "W", "E", "b", "WE"])
def test_frozen_inputs(frozen):
    h, W, E, b = make()
    names = dict(h=h, W=W, E=E, b=b)
    for k in frozen:
        names[k].requires_grad_(False)
    assert_matches_oracle(h, W, E, b)


def test_tied_W_and_E():
    h, W, _, b = make(K=7, D=7)
    assert_matches_oracle(h, W, W, b)


def test_only_lse_or_only_O_used():
    h, W, E, b = make()
    cpu = [x.detach().cpu().double().requires_grad_(True) for x in (h, W, E, b)]
    for pick in (0, 1):
        out = swvr.softmax_readout(h, W, E, b, chunk_size=8)[pick].sum()
        want = ref.softmax_readout_reference(*cpu)[pick].sum()
        g = torch.autograd.grad(out, (h, W, E, b), allow_unused=True)
        gr = torch.autograd.grad(want, cpu, allow_unused=True)
        for a, r in zip(g, gr):
            if r is None:
                assert a is None or a.abs().max() == 0
            else:
                torch.testing.assert_close(a.double().cpu(), r, **TOL)


def test_bf16_inputs_return_fp32():
    h, W, E, b = make(dtype=torch.bfloat16, K=32, V=300)
    O, lse = swvr.softmax_readout(h, W, E, b, chunk_size=64)
    assert O.dtype == f32 and lse.dtype == f32
    O_r, lse_r = ref.softmax_readout_reference(*(x.detach().cpu().double() for x in (h, W, E, b)))
    torch.testing.assert_close(lse.double().cpu(), lse_r, rtol=1e-3, atol=1e-2)
    torch.testing.assert_close(O.double().cpu(), O_r, rtol=2e-2, atol=2e-2)


@pytest.mark.parametrize("reduction", ["mean", "sum", "none"])
def test_mse_matches_oracle(reduction):
    h, W, E, b = make(lead=(2, 3))
    target = torch.randn(2, 3, 5, dtype=f64).cuda().float()
    weight = torch.tensor([[1., 0., 2.], [1., 1., 0.]], device="cuda")
    kw = dict(weight=weight, reduction=reduction, z_loss_weight=0.1, logit_scale=0.5)
    loss = swvr.softmax_readout_mse(h, W, E, target, b, chunk_size=8, **kw)
    cpu = [x.detach().cpu().double().requires_grad_(True) for x in (h, W, E, b)]
    kwc = dict(kw, weight=weight.cpu().double())
    want = ref.mse_reference(cpu[0], cpu[1], cpu[2], target.cpu().double(), cpu[3], **kwc)
    torch.testing.assert_close(loss.double().cpu(), want, **TOL)
    g = torch.autograd.grad(loss.sum(), (h, W, E, b))
    gr = torch.autograd.grad(want.sum(), cpu)
    for a, r in zip(g, gr):
        torch.testing.assert_close(a.double().cpu(), r, **TOL)


def test_module_wraps_linear_and_embedding():
    torch.manual_seed(0)
    head, emb = nn.Linear(12, 41).cuda(), nn.Embedding(41, 5).cuda()
    h, target = torch.randn(7, 12, device="cuda"), torch.randn(7, 5, device="cuda")
    loss_fn = swvr.SoftmaxReadoutMSE(head, emb, z_loss_weight=1e-2, chunk_size=8)
    loss = loss_fn(h, target)
    cpu = [p.detach().cpu().double() for p in (head.weight, emb.weight, head.bias)]
    want = ref.mse_reference(h.cpu().double(), cpu[0], cpu[1], target.cpu().double(), cpu[2], z_loss_weight=1e-2)
    torch.testing.assert_close(loss.double().cpu(), want, **TOL)
    loss.backward()
    assert head.weight.grad is not None and head.bias.grad is not None and emb.weight.grad is not None


def test_activation_checkpointing():
    from torch.utils.checkpoint import checkpoint
    h, W, E, b = make()
    fn = lambda h: swvr.softmax_readout(h, W, E, b, chunk_size=8)[0].pow(2).sum()
    g1 = torch.autograd.grad(checkpoint(fn, h, use_reentrant=False), h)[0]
    g2 = torch.autograd.grad(fn(h), h)[0]
    torch.testing.assert_close(g1, g2)


GOLD = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "readout_cases.json")))["cases"]


@pytest.mark.parametrize("case", GOLD, ids=[c["name"] for c in GOLD])
def test_golden_fixtures_through_hip_fp32(case):
    c = case
    t = lambda x: None if x is None else torch.tensor(x, dtype=f32, device="cuda")
    xs = [t(c[k]) for k in ("h", "W", "E", "bias")]
    xs = [x.requires_grad_(True) if x is not None else None for x in xs]
    O, lse = swvr.softmax_readout(*xs, logit_scale=c["logit_scale"], chunk_size=3)
    gO, glse = t(c["gO"]), t(c["glse"])
    want_in = [x for x in xs if x is not None]
    gs = torch.autograd.grad((O * gO).sum() + (lse * glse).sum(), want_in)
    got = dict(O=O, lse=lse, gh=gs[0], gW=gs[1], gE=gs[2], gb=gs[3] if len(gs) > 3 else None)
    for k, v in got.items():
        if c[k] is None:
            continue
        want = torch.tensor(c[k], dtype=f64)
        assert rel_err(v, want) < 1e-5, (k, rel_err(v, want))
    if "mse" in c:
        kw = dict(weight=t(c["weight"]), z_loss_weight=c["z_loss_weight"], logit_scale=c["logit_scale"])
        for red, want in c["mse"].items():
            got = swvr.softmax_readout_mse(*xs[:3], t(c["target"]), xs[3], reduction=red, **kw)
            assert rel_err(got, torch.tensor(want, dtype=f64)) < 1e-5



def test_zero_hidden_size():
    # the public API flattens h with reshape(-1, K), which raises for K = 0
    # exactly as swvr/api.py:36 does
    h, W, E, b = make(K=0)
    with pytest.raises(RuntimeError):
        swvr.softmax_readout(h, W, E, b, chunk_size=8)
    # the C ABI takes K = 0: every score is the bias, so O = softmax(b) E
    from swvr_amd import _lib
    lib = _lib.load()
    N, V, D = 6, 41, 5
    Ed, bd = E.detach().contiguous(), b.detach().contiguous()
    O = torch.empty(N, D, device="cuda")
    lse = torch.empty(N, device="cuda")
    ws = torch.empty(lib.swvr_fwd_workspace_size(2, N, 0, V, D), dtype=torch.uint8, device="cuda")
    _lib.check(lib.swvr_fwd(2, N, 0, V, D, None, 0, None, 0, _lib.ptr(Ed), D, _lib.ptr(bd), 1.0,
                            _lib.ptr(O), _lib.ptr(lse), _lib.ptr(ws), ws.numel(), _lib.stream_of(O.device)))
    torch.cuda.synchronize()
    want = torch.softmax(bd.double(), 0) @ Ed.double()
    torch.testing.assert_close(O.double(), want.expand_as(O), **TOL)
    torch.testing.assert_close(lse.double(), torch.logsumexp(bd.double(), 0).expand(N), **TOL)


@pytest.mark.parametrize("D", [5, 128, 256])
def test_zero_hidden_size_bf16_forwards(D):
    """K = 0 through the C ABI in bf16: the one all-zero reduction slice of the 256 x 256 forward
    (D = 5) and of the streamed-E^T forward's two-slice stages (D = 128, 256: a zero slice beside
    it).  Every score is the bias, so O = softmax(b) E."""
    from swvr_amd import _lib
    lib = _lib.load()
    N, V = 70, 700
    g = torch.Generator().manual_seed(5)
    E = torch.randn(V, D, generator=g).to(device="cuda", dtype=torch.bfloat16)
    b = (2.0 * torch.randn(V, generator=g)).to("cuda")
    O = torch.empty(N, D, device="cuda")
    lse = torch.empty(N, device="cuda")
    ws = torch.empty(lib.swvr_fwd_workspace_size(_lib.BF16, N, 0, V, D), dtype=torch.uint8, device="cuda")
    _lib.check(lib.swvr_fwd(_lib.BF16, N, 0, V, D, None, 0, None, 0, _lib.ptr(E), D, _lib.ptr(b), 1.0,
                            _lib.ptr(O), _lib.ptr(lse), _lib.ptr(ws), ws.numel(), _lib.stream_of(O.device)))
    torch.cuda.synchronize()
    want = torch.softmax(b.double(), 0) @ E.double()
    assert rel_err(O, want.expand_as(O)) < 1e-2
    torch.testing.assert_close(lse.double(), torch.logsumexp(b.double(), 0).expand(N), rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("dtype,N,K,V,D", [
    (torch.bfloat16, 40, 32, 1000, 64), (torch.bfloat16, 300, 32, 3000, 16), (torch.float16, 40, 32, 1000, 200),
    (torch.float32, 40, 16, 1000, 64), (torch.float32, 40, 16, 1000, 128), (torch.bfloat16, 6, 32, 300, 5),
])
def test_one_slice_stages_over_several_vocabulary_tiles(dtype, N, K, V, D):
    """K of one reduction slice: every ring stage is a whole vocabulary tile, so the forward's
    first stages are issued back to back (a stale condition code once reloaded tile 0 there)."""
    h, W, E, b = make(N=N, K=K, V=V, D=D, dtype=dtype)
    O, lse = swvr.softmax_readout(h, W, E, b)
    O_r, lse_r = ref.softmax_readout_reference(*(x.detach().cpu().double() for x in (h, W, E, b)))
    tol = 1e-5 if dtype == f32 else 1e-2
    assert rel_err(lse, lse_r) < tol / 10
    assert rel_err(O, O_r) < tol


@pytest.mark.parametrize("dtype,D", [(torch.bfloat16, 4096), (torch.float32, 4000), (torch.bfloat16, 65536)])
def test_embedding_widths_up_to_the_maximum(dtype, D):
    """D far above one pass (the forward runs 256-column slices of E, fp32 128; the backward's wide
    kernel streams D in 32-column slices, fp32 16), up to swvr_max_d = 65536, against the fp64
    oracle: the north-star bar for bf16, fp32-sized for fp32."""
    N, K, V = 300, 96, 700
    h, W, E, b = make(N=N, K=K, V=V, D=D, dtype=dtype)
    g = torch.Generator(device="cuda").manual_seed(3)
    gO = torch.randn(N, D, device="cuda", generator=g)
    glse = torch.randn(N, device="cuda", generator=g)
    O, lse = swvr.softmax_readout(h, W, E, b)
    got = (O, lse, *torch.autograd.grad((O * gO).sum() + (lse * glse).sum(), (h, W, E, b)))
    want = ref.reference_grads(h, W, E, b, gO, glse)
    lo = dtype != f32
    for name, a, r in zip(("O", "lse", "gh", "gW", "gE", "gb"), got, want):
        bar = (1e-2 if name in ("O", "lse") else 2e-2) if lo else 1e-5
        assert rel_err(a, r) <= bar, (name, rel_err(a, r))


@pytest.mark.parametrize("dtype,K", [(torch.bfloat16, 20007), (torch.float32, 9001)])
def test_long_hidden_rows(dtype, K):
    """K in the tens of thousands, not a multiple of the 32-element slice: the packed operands'
    625 slices (fp32 16-element slices: 563) and the tail slice, against the fp64 oracle."""
    N, V, D = 300, 700, 16
    h, W, E, b = make(N=N, K=K, V=V, D=D, dtype=dtype)
    with torch.no_grad():
        W.mul_(K ** -0.5)
    g = torch.Generator(device="cuda").manual_seed(4)
    gO = torch.randn(N, D, device="cuda", generator=g)
    glse = torch.randn(N, device="cuda", generator=g)
    O, lse = swvr.softmax_readout(h, W, E, b)
    got = (O, lse, *torch.autograd.grad((O * gO).sum() + (lse * glse).sum(), (h, W, E, b)))
    want = ref.reference_grads(h, W, E, b, gO, glse)
    lo = dtype != f32
    for name, a, r in zip(("O", "lse", "gh", "gW", "gE", "gb"), got, want):
        bar = (1e-2 if name in ("O", "lse") else 2e-2) if lo else 1e-5
        assert rel_err(a, r) <= bar, (name, rel_err(a, r))
