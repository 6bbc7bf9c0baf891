"""Seeded parity sweeps over shapes, dtypes, chunk sizes, biases, scales, frozen inputs and the loss path.

Each sweep draws a fixed list of cases from its own seed (the list is the same on every run), runs
the HIP path and compares every output and gradient with the fp64 closed form (swvr/reference.py:5-14
and the loss of swvr/api.py:44-66, differentiated by torch autograd), at the north-star bars:
O, lse and the loss rel err <= 1e-2 (bf16 / fp16) or 1e-5 (fp32); every gradient rel err <= 2e-2
and cosine >= 0.999 (bf16 / fp16), or rel err <= 1e-4 (fp32).  A sweep stops at its first failing
case and names it.

Inputs that are ill-conditioned for the reference's algorithm itself are held to that algorithm, not
to the bar.  The rule: when a quantity misses the bar, the reference's chunked algorithm
(swvr/chunked.py:82-151, restated in oracle/chunked.py) is run on the CPU on the same inputs in the
same compute dtype.  The case passes only if that algorithm misses the same bar too and the HIP
result is within 2x of its error.  Examples are nearly one-hot P over two vocabulary rows, where
dS = P (dP - delta) cancels to rounding error, and fp16 cotangents below fp16's normal range.  The
rule is applied per quantity and reported in the output.
"""
import math
import random

import pytest
import torch

import swvr_amd as swvr
from oracle import chunked, reference as ref

pytestmark = pytest.mark.gpu

bf16, f16, f32 = torch.bfloat16, torch.float16, torch.float32


def rel(a, r):
    a, r = a.detach().double().cpu(), r.detach().double().cpu()
    return ((a - r).norm() / r.norm().clamp_min(1e-30)).item()


def cos(a, r):
    a, r = a.detach().double().cpu().flatten(), r.detach().double().cpu().flatten()
    n = (a.norm() * r.norm()).item()
    return 1.0 if n == 0 else (a @ r).item() / n


def bars(dt):
    lo = dt != f32
    return (1e-2, 2e-2, 0.999) if lo else (1e-5, 1e-4, 0.999999)


def misses(name, e, c, dt):
    tol_out, tol_grad, min_cos = bars(dt)
    if name in ("O", "lse", "loss"):
        return e > tol_out
    return e > tol_grad or c < min_cos


def judge(case, dt, names, got, want, ref_algo):
    """Assert the bar for every quantity; ``ref_algo()`` gives the reference algorithm's results
    (same order as ``got``) for the rule above, computed only when something misses."""
    errs = {n: (rel(a, r), cos(a, r)) for n, a, r in zip(names, got, want)}
    bad = [n for n, (e, c) in errs.items() if misses(n, e, c, dt)]
    if bad:
        alg = ref_algo()
        for n in bad:
            i = names.index(n)
            e_ref, c_ref = rel(alg[i], want[i]), cos(alg[i], want[i])
            assert misses(n, e_ref, c_ref, dt), (case, n, errs[n], "reference algorithm meets the bar", e_ref)
            assert errs[n][0] <= 2 * e_ref, (case, n, errs[n], "more than 2x the reference algorithm", e_ref)
            print(case, f"{n}: ill-conditioned for the algorithm (here {errs[n][0]:.1e}, "
                        f"reference algorithm {e_ref:.1e})", flush=True)
    return {n: e for n, (e, _) in errs.items()}


# ---------------------------------------------------------------- the readout and its gradients
def readout_cases(seed=2026, n=40):
    rng = random.Random(seed)
    out = []
    for i in range(n):
        dt = rng.choice([bf16, f16, f32])
        N = rng.choice([1, 2, 33, 255, 257, 700, 1500, 3000])
        K = 8 * rng.randint(1, 64)
        V = rng.choice([1, 7, 255, 256, 257, 1000, 4097, 9000])
        D = rng.choice([1, 5, 16, 31, 32, 33, 63, 64, 65, 100, 128, 129, 200, 256, 300])
        chunk = rng.choice([1, 64, 256, 1000, 4096, 8192] if V <= 257 else [64, 256, 1000, 4096, 8192])
        bias = rng.random() < 0.7
        scale = rng.choice([1.0, 0.5, 2.0, 1.0 / math.sqrt(K), -1.0])
        need = [rng.random() < 0.8 for _ in range(4)]
        if not any(need[:3]):
            need[rng.randrange(3)] = True
        strided = rng.random() < 0.2
        out.append(dict(i=i, dt=dt, N=N, K=K, V=V, D=D, chunk=chunk, bias=bias, scale=scale, need=need,
                        strided=strided))
    return out


def test_readout_sweep():
    for c in readout_cases():
        dt, N, K, V, D = c["dt"], c["N"], c["K"], c["V"], c["D"]
        tag = (f"readout case {c['i']}: {dt} N={N} K={K} V={V} D={D} chunk={c['chunk']} bias={c['bias']} "
               f"scale={c['scale']:.3g} need={c['need']} strided={c['strided']}")
        print(tag, flush=True)
        g = torch.Generator(device="cuda").manual_seed(1000 + c["i"])
        hfull = torch.randn(N, 2 * K if c["strided"] else K, device="cuda", generator=g).to(dt)
        h = hfull[:, ::2] if c["strided"] else hfull
        W = (torch.randn(V, K, device="cuda", generator=g) * K ** -0.5).to(dt)
        E = torch.randn(V, D, device="cuda", generator=g).to(dt)
        b = (0.3 * torch.randn(V, device="cuda", generator=g)).to(dt) if c["bias"] else None
        gO = torch.randn(N, D, device="cuda", generator=g)
        glse = torch.randn(N, device="cuda", generator=g)
        leaves = [hfull, W, E, b]
        trains = [x is not None and nd for x, nd in zip(leaves, c["need"])]
        for x, t in zip(leaves, trains):
            if t:
                x.requires_grad_(True)
        h = hfull[:, ::2] if c["strided"] else hfull
        xs = [x for x, t in zip(leaves, trains) if t]
        O, lse = swvr.softmax_readout(h, W, E, b, logit_scale=c["scale"], chunk_size=c["chunk"])
        grads = torch.autograd.grad((O * gO).sum() + (lse * glse).sum(), xs)
        torch.cuda.synchronize()
        # fp64 closed form on the same (compute-dtype) values
        d = [x.detach().double().requires_grad_(t) if x is not None else None for x, t in zip(leaves, trains)]
        hd = d[0][:, ::2] if c["strided"] else d[0]
        Or, lr = ref.softmax_readout_reference(hd, d[1], d[2], d[3], logit_scale=c["scale"], dtype=torch.float64)
        gr = torch.autograd.grad((Or * gO.double()).sum() + (lr * glse.double()).sum(), [x for x in d if x is not None and x.requires_grad])
        names = ["O", "lse"] + [n for n, t in zip(("gh", "gW", "gE", "gb"), trains) if t]
        got = [O, lse] + [gx[:, ::2] if (n == "gh" and c["strided"]) else gx for n, gx in zip(names[2:], grads)]
        want = [Or, lr] + [gx[:, ::2] if (n == "gh" and c["strided"]) else gx for n, gx in zip(names[2:], gr)]

        def ref_algo():
            cpu = [x.detach().cpu() if x is not None else None for x in (h, W, E, b)]
            Oc, lc = chunked.forward(cpu[0], cpu[1], cpu[2], cpu[3], c["scale"], c["chunk"], dt)
            gs = chunked.backward(gO.cpu(), glse.cpu(), cpu[0], cpu[1], cpu[2], cpu[3], Oc, lc, c["scale"],
                                  c["chunk"], dt, *trains)
            return [Oc, lc] + [x for x, t in zip(gs, trains) if t]

        errs = judge(tag, dt, names, got, want, ref_algo)
        print("   ", {k: f"{v:.1e}" for k, v in errs.items()}, flush=True)


# ---------------------------------------------------------------- the MSE loss path
def loss_cases(seed=2027, n=24):
    rng = random.Random(seed)
    out = []
    for i in range(n):
        dt = rng.choice([bf16, f16, f32])
        mode = rng.choice(["plain", "plain", "autocast", "strided", "lead"])
        if mode == "autocast" and dt == f32:
            dt = bf16
        out.append(dict(i=i, dt=dt, mode=mode, N=rng.choice([1, 3, 64, 255, 257, 1000, 2500]),
                        K=8 * rng.randint(1, 64), V=rng.choice([2, 100, 256, 1000, 5000]),
                        D=rng.choice([1, 8, 16, 33, 64, 100, 128, 200, 256]), chunk=rng.choice([128, 1000, 8192]),
                        bias=rng.random() < 0.7, scale=rng.choice([1.0, 0.3, 3.0]),
                        weight=rng.choice([None, "bernoulli", "fraction", "every_third_zero"]),
                        reduction=rng.choice(["mean", "sum", "none"]), z=rng.choice([0.0, 1e-4, 1e-2])))
    return out


def test_loss_sweep():
    for c in loss_cases():
        dt, N, K, V, D, mode = c["dt"], c["N"], c["K"], c["V"], c["D"], c["mode"]
        tag = (f"loss case {c['i']}: {dt} {mode} N={N} K={K} V={V} D={D} chunk={c['chunk']} bias={c['bias']} "
               f"scale={c['scale']} weight={c['weight']} reduction={c['reduction']} z={c['z']}")
        print(tag, flush=True)
        g = torch.Generator(device="cuda").manual_seed(5000 + c["i"])
        pdt = f32 if mode == "autocast" else dt
        hfull = torch.randn(N, 2 * K if mode == "strided" else K, device="cuda", generator=g).to(pdt)
        W = (torch.randn(V, K, device="cuda", generator=g) * 2 * K ** -0.5).to(pdt)
        E = torch.randn(V, D, device="cuda", generator=g).to(pdt)
        b = (0.3 * torch.randn(V, device="cuda", generator=g)).to(pdt) if c["bias"] else None
        target = torch.randn(N, D, device="cuda", generator=g)
        w = None
        if c["weight"] == "bernoulli":
            w = (torch.rand(N, device="cuda", generator=g) < 0.8).float()
        elif c["weight"] == "fraction":
            w = torch.rand(N, device="cuda", generator=g)
        elif c["weight"] == "every_third_zero":
            w = torch.ones(N, device="cuda")
            w[::3] = 0
        if w is not None and float(w.sum()) == 0:
            w[0] = 1.0
        leaves = [x for x in (hfull, W, E, b) if x is not None]
        for x in leaves:
            x.requires_grad_(True)
        h = hfull[:, ::2] if mode == "strided" else hfull
        hin, tin = (h.reshape(1, N, K), target.reshape(1, N, D)) if mode == "lead" else (h, target)
        win = w.reshape(1, N) if (mode == "lead" and w is not None) else w
        kw = dict(weight=win, reduction=c["reduction"], z_loss_weight=c["z"], logit_scale=c["scale"],
                  chunk_size=c["chunk"])
        if mode == "autocast":
            with torch.autocast("cuda", dtype=dt):
                loss = swvr.softmax_readout_mse(hin, W, E, tin, b, **kw)
        else:
            loss = swvr.softmax_readout_mse(hin, W, E, tin, b, **kw)
        loss = loss.reshape(-1)
        cot = torch.randn(loss.shape, device="cuda", generator=g) if c["reduction"] == "none" else torch.ones_like(loss)
        grads = torch.autograd.grad((loss * cot).sum(), leaves)
        torch.cuda.synchronize()
        # fp64 closed form of the loss on the compute-dtype values (autocast rounds to dt first)
        cd = [x.detach().to(dt).double().requires_grad_(True) for x in leaves]
        hd = cd[0][:, ::2] if mode == "strided" else cd[0]
        loss_r = ref.mse_reference(hd, cd[1], cd[2], target.double(), cd[3] if c["bias"] else None,
                                   weight=w.double() if w is not None else None, reduction=c["reduction"],
                                   z_loss_weight=c["z"], logit_scale=c["scale"], dtype=torch.float64).reshape(-1)
        gr = torch.autograd.grad((loss_r * cot.double()).sum(), cd)
        names = ["loss", "gh", "gW", "gE"] + (["gb"] if c["bias"] else [])
        sl = (lambda x: x[:, ::2]) if mode == "strided" else (lambda x: x)
        got = [loss, sl(grads[0]), *grads[1:]]
        want = [loss_r, sl(gr[0]), *gr[1:]]

        def ref_algo():
            # the reference's composite: chunked forward, the loss in fp32 torch ops and its autograd,
            # then the chunked backward, all in the compute dtype dt (swvr/api.py:25-66)
            cpu = [x.detach().cpu().to(dt) for x in (h, W, E)] + ([b.detach().cpu().to(dt)] if c["bias"] else [None])
            Oc, lc = chunked.forward(cpu[0], cpu[1], cpu[2], cpu[3], c["scale"], c["chunk"], dt)
            Ol, ll = Oc.clone().requires_grad_(True), lc.clone().requires_grad_(True)
            per_tok = (Ol - target.cpu()).pow(2).mean(-1) + c["z"] * ll.pow(2)
            wc = w.cpu() if w is not None else None
            if wc is not None:
                per_tok = per_tok * wc
            if c["reduction"] == "none":
                lo = per_tok
            elif c["reduction"] == "sum":
                lo = per_tok.sum()
            else:
                lo = per_tok.sum() / (wc.sum() if wc is not None else per_tok.numel())
            lo = lo.reshape(-1)
            gO, glse = torch.autograd.grad((lo * cot.cpu()).sum(), (Ol, ll))
            gs = chunked.backward(gO, glse, cpu[0], cpu[1], cpu[2], cpu[3], Oc, lc, c["scale"], c["chunk"], dt,
                                  True, True, True, c["bias"])
            out = [lo.detach(), gs[0], gs[1], gs[2]]  # gs[0]: the gradient of the [N, K] view itself
            return out + ([gs[3]] if c["bias"] else [])

        errs = judge(tag, dt, names, got, want, ref_algo)
        print("   ", {k: f"{v:.1e}" for k, v in errs.items()}, flush=True)
