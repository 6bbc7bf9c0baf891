"""Helpers shared by the GPU parity tests."""
import torch

from oracle import reference as ref


def make(N, K, V, D, dtype, bias=True, seed=0, lead=None, w_scale=3.0, b_scale=0.5, requires_grad=True):
    """Seeded inputs on the GPU at the reference test's realistic scales
    (tests/test_cuda.py:17-23 of the reference: W ~ 3/sqrt(K), bias ~ 0.5)."""
    g = torch.Generator(device="cuda").manual_seed(seed)
    t = lambda *s, scale=1.0: (scale * torch.randn(*s, generator=g, device="cuda")).to(dtype)
    shape = (*(lead or (N,)), K)
    h, W, E = t(*shape), t(V, K, scale=w_scale / K ** 0.5), t(V, D)
    b = t(V, scale=b_scale) if bias else None
    xs = [h, W, E, b]
    if requires_grad:
        xs = [x.requires_grad_(True) if x is not None else None for x in xs]
    return xs


def run(fn, inputs, gO, glse):
    """Outputs and the gradients of sum(gO*O) + sum(glse*lse) w.r.t. the inputs that require them."""
    O, lse = fn(*inputs)
    xs = [x for x in inputs if x is not None and x.requires_grad]
    gs = torch.autograd.grad((O * gO).sum() + (lse * glse).sum(), xs)
    return [O, lse, *gs]


def oracle_run(inputs, gO, glse, logit_scale=1.0, dtype=torch.float64):
    """Same quantities from the CPU oracle in ``dtype`` (fp64 by default)."""
    cpu = [x.detach().cpu().to(dtype).requires_grad_(x.requires_grad) if x is not None else None
           for x in inputs]
    O, lse = ref.softmax_readout_reference(*cpu, logit_scale=logit_scale, dtype=dtype)
    xs = [x for x in cpu if x is not None and x.requires_grad]
    gs = torch.autograd.grad((O * gO.cpu().to(dtype)).sum() + (lse * glse.cpu().to(dtype)).sum(), xs)
    return [O, lse, *gs]


def rel_err(a, r):
    """Norm-wise relative error (tests/test_cuda.py:33-34 of the reference)."""
    a, r = a.detach().double().cpu(), r.detach().double().cpu()
    return ((a - r).norm() / r.norm().clamp_min(1e-30)).item()


def cosine(a, r):
    a, r = a.detach().double().cpu().flatten(), r.detach().double().cpu().flatten()
    return (a @ r / (a.norm() * r.norm()).clamp_min(1e-300)).item()
