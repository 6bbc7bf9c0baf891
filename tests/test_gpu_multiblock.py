"""The backward's steady-state loop: scores workgroups that walk several token blocks.

The scores kernels split a vocabulary tile's active token blocks over G
workgroups (``swvr_bwd_tiling``), so a workgroup walks ceil(blocks / G) of them.
Every case here makes most tokens active and asserts that the active token
blocks are at least 2 G, so every workgroup takes the path that only a second
block takes: the catch-up issue of the next block's slices behind the previous
epilogue, the alternating LSE / delta strips and the ring waits that count
stages across blocks (narrow embeddings), and the reloads of the gO / gO^T /
LSE tiles per block (the general kernel).  The reference's kernel walks every
row block in one program too (swvr/triton_kernels.py:92-113).

Every row of every output is compared with the fp64 closed form, evaluated
block by block of rows on the GPU (oracle.reference.reference_grads_blocked,
pinned against the golden fixtures on the CPU).  Bars, as the north star's:
bf16 / fp16 O and lse rel err <= 1e-2 (whole tensor and every row), gradients
rel err <= 2e-2 and cosine >= 0.999; fp32 O / lse <= 1e-5 (every row <= 1e-4),
gradients <= 1e-4.
"""
import math

import pytest
import torch

import swvr_amd as swvr
from swvr_amd import _lib
from oracle import reference as ref

pytestmark = pytest.mark.gpu
bf16, f16, f32, f64 = torch.bfloat16, torch.float16, torch.float32, torch.float64


def rel_err(a, r):
    a, r = a.detach().double(), r.detach().double()
    return ((a - r).norm() / r.norm().clamp_min(1e-30)).item()


def cosine(a, r):
    a, r = a.detach().double().flatten(), r.detach().double().flatten()
    return (a @ r / (a.norm() * r.norm()).clamp_min(1e-300)).item()


def row_rel_max(a, r):
    """Largest per-row norm-wise relative error."""
    a, r = a.detach().double().reshape(r.shape[0], -1), r.detach().double().reshape(r.shape[0], -1)
    return ((a - r).norm(dim=1) / r.norm(dim=1).clamp_min(1e-30)).max().item()


def draw(N, K, V, D, dtype, seed, lead=None, w_scale=1.0, bias=True):
    """h ~ N(0,1), W ~ N(0, w_scale^2/K), bias ~ N(0, 0.02^2), E ~ N(0,1) (the benchmark's draws)."""
    g = torch.Generator(device="cuda").manual_seed(seed)
    r = lambda *s, sc=1.0: (sc * torch.randn(*s, device="cuda", generator=g)).to(dtype)
    h = r(*(lead or (N,)), K)
    W = r(V, K, sc=w_scale * K ** -0.5)
    b = r(V, sc=0.02) if bias else None
    E = r(V, D)
    return h, W, E, b


def assert_multiblock(dtype, N_active, K, V, D, chunk):
    """The tiling gives every scores workgroup at least two token blocks."""
    t = _lib.bwd_tiling(dtype, N_active, K, V, D, chunk)
    n_tb_act = math.ceil(N_active / t["BM"])
    assert n_tb_act >= 2 * t["G"], (t, n_tb_act)
    return t


def check(got, want, dtype, tag):
    """got/want = (O, lse, gh, gW, gE, gb); every row of O and lse, all gradients."""
    names = ("O", "lse", "gh", "gW", "gE", "gb")
    lo = dtype in (bf16, f16)
    tol_out, tol_row, tol_grad = (1e-2, 1e-2, 2e-2) if lo else (1e-5, 1e-4, 1e-4)
    errs = {}
    for n, a, r in zip(names, got, want):
        if r is None:
            assert a is None, n
            continue
        a = a.reshape(r.shape)
        assert torch.isfinite(a).all(), (tag, n)
        errs[n] = rel_err(a, r)
        if n in ("O", "lse"):
            errs[n + "_row"] = row_rel_max(a, r)
        else:
            c = cosine(a, r)
            assert c >= (0.999 if lo else 0.999999), (tag, n, c)
    print(tag, {k: f"{v:.1e}" for k, v in errs.items()}, flush=True)
    for n, e in errs.items():
        bar = tol_row if n.endswith("_row") else tol_out if n in ("O", "lse") else tol_grad
        assert e <= bar, (tag, n, errs)


def run_case(h, W, E, b, gO, glse, chunk):
    xs = [x.requires_grad_(True) for x in (h, W, E, b) if x is not None]
    O, lse = swvr.softmax_readout(h, W, E, b, chunk_size=chunk)
    N, D = gO.shape
    grads = list(torch.autograd.grad((O.reshape(N, D) * gO).sum() + (lse.reshape(N) * glse).sum(), xs))
    torch.cuda.synchronize()
    if b is None:
        grads.append(None)
    return (O.reshape(N, D), lse.reshape(N), *grads)


# (dtype, N, K, V, D, chunk): narrow ring kernel (2-byte dtypes, D <= 64), wide kernel
# (2-byte dtypes above 64 in 256-token blocks, fp32 above 128 in 128-token blocks, including
# widths beyond one forward pass: the forward runs slices of E's columns) and general kernel
# (fp32 up to 128), token counts that leave a partial last block, vocabularies with a partial
# last chunk, and a small chunk (G = 32) whose groups get 2 or 3 blocks.
CASES = [
    ("ring-bf16-D64", bf16, 8192 + 77, 256, 8192 + 300, 64, 8192),
    ("ring-bf16-D16", bf16, 8192 + 256, 128, 8192, 16, 8192),
    ("ring-f16-D48", f16, 9000, 192, 4096 + 64, 48, 4096),
    ("ring-bf16-chunk2048", bf16, 16384 + 5, 128, 4096 + 17, 64, 2048),
    ("wide-bf16-D128", bf16, 4096 + 33, 256, 8192 + 128, 128, 8192),
    ("wide-f16-D200", f16, 4096 + 100, 128, 8192, 200, 8192),
    ("wide-bf16-D256", bf16, 4096 + 64, 256, 8192 + 40, 256, 8192),
    ("wide-bf16-D300", bf16, 4096 + 64, 256, 8192 + 100, 300, 8192),
    ("wide-f16-D520", f16, 4096 + 5, 128, 8192, 520, 8192),
    ("wide-bf16-D80", bf16, 4096 + 31, 192, 8192, 80, 8192),
    ("wide-f32-D200", f32, 2048 + 1, 64, 8192, 200, 8192),
    ("general-f32-D64", f32, 2048 + 9, 128, 8192, 64, 8192),
    ("general-f32-D128", f32, 2048 + 3, 64, 4096, 128, 4096),
    # one reduction slice per stage (K = one slice): the stage cursor advances a whole
    # token block per issue, the case a stale condition code once broke
    ("ring-bf16-D64-K32", bf16, 8192 + 77, 32, 8192 + 300, 64, 8192),
    ("wide-bf16-D128-K32", bf16, 4096 + 33, 32, 8192 + 128, 128, 8192),
    ("general-f32-D64-K16", f32, 2048 + 9, 16, 8192, 64, 8192),
    ("general-f32-D128-K16", f32, 2048 + 3, 16, 4096, 128, 4096),
]


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_multiblock_backward_matches_fp64_on_every_row(case):
    tag, dtype, N, K, V, D, chunk = case
    print("case", tag, flush=True)
    t = assert_multiblock(dtype, N, K, V, D, chunk)
    assert t["kernel"] == {"ring": 1, "wide": 2, "general": 0}[tag.split("-")[0]], t
    h, W, E, b = draw(N, K, V, D, dtype, seed=sum(map(ord, tag)), w_scale=3.0)
    g = torch.Generator(device="cuda").manual_seed(7)
    gO = torch.randn(N, D, device="cuda", generator=g)
    glse = 0.5 * torch.randn(N, device="cuda", generator=g)
    got = run_case(h, W, E, b, gO, glse, chunk)
    want = ref.reference_grads_blocked(h.detach(), W.detach(), E.detach(), b.detach(), gO, glse, block=2048)
    check(got, want, dtype, tag)


def test_multiblock_backward_with_inactive_tokens_interleaved():
    """Zero-cotangent tokens scattered between active ones: the compacted positions still
    fill at least 2 G blocks per vocabulary tile, and the inactive tokens' gh rows are zero."""
    N, K, V, D, chunk = 12000, 256, 8192 + 50, 64, 8192
    h, W, E, b = draw(N, K, V, D, bf16, seed=3, w_scale=3.0)
    g = torch.Generator(device="cuda").manual_seed(8)
    active = torch.rand(N, device="cuda", generator=g) < 0.8
    gO = torch.randn(N, D, device="cuda", generator=g) * active[:, None]
    glse = 0.5 * torch.randn(N, device="cuda", generator=g) * active
    assert_multiblock(bf16, int(active.sum()), K, V, D, chunk)
    got = run_case(h, W, E, b, gO, glse, chunk)
    want = ref.reference_grads_blocked(h.detach(), W.detach(), E.detach(), b.detach(), gO, glse, block=2048)
    check(got, want, bf16, "interleaved")
    assert got[2][~active].abs().max().item() == 0.0


# BASELINE.json configs 2-5 at full size: (lead dims, K, V, D, bias)
FULL = {
    2: dict(lead=(16384,), K=1024, V=151936, D=16, bias=False),
    3: dict(lead=(16384,), K=2560, V=151936, D=64, bias=True),
    4: dict(lead=(8192,), K=4096, V=128256, D=128, bias=True),
    5: dict(lead=(8, 4096), K=4096, V=256000, D=256, bias=True),
}


@pytest.mark.parametrize("config", sorted(FULL))
def test_full_size_every_token_active_matches_fp64(config):
    """Every token carries a cotangent, so the backward runs the benchmark's tiling with all
    token blocks active; O, lse and the four gradients are checked on every row."""
    cfg = FULL[config]
    print("config", config, flush=True)
    K, V, D = cfg["K"], cfg["V"], cfg["D"]
    N = math.prod(cfg["lead"])
    assert_multiblock(bf16, N, K, V, D, 8192)
    h, W, E, b = draw(N, K, V, D, bf16, seed=0, lead=cfg["lead"], bias=cfg["bias"])
    g = torch.Generator(device="cuda").manual_seed(1)
    gO = torch.randn(N, D, device="cuda", generator=g)
    glse = 0.1 * torch.randn(N, device="cuda", generator=g)
    got = run_case(h, W, E, b, gO, glse, 8192)
    want = ref.reference_grads_blocked(h.detach().reshape(N, K), W.detach(), E.detach(),
                                       b.detach() if b is not None else None, gO, glse, block=1024)
    check(got, want, bf16, f"config {config}")


def bench_weight(config, lead, g):
    """The benchmark's per-token weights: Bernoulli(0.9) at config 3, a seeded ragged tail of
    zeros (U{0..1024} per row of the batch) at config 5."""
    if config == 3:
        return (torch.rand(*lead, device="cuda", generator=g) >= 0.1).float()
    rows, T = lead
    tails = torch.randint(0, 1025, (rows,), device="cuda", generator=g)
    pos = torch.arange(T, device="cuda")[None, :]
    return (pos < (T - tails)[:, None]).float()


@pytest.mark.parametrize("config", [3, 5])
def test_full_size_benchmark_loss_matches_fp64(config):
    """The benchmark's step: the weighted MSE with z-loss, reduction "mean", at full size.
    Zero-weight tokens drop out of the backward, the rest fill many token blocks per
    workgroup; the loss and every gradient are compared with the row-blocked fp64 MSE."""
    cfg = FULL[config]
    print("config", config, flush=True)
    K, V, D = cfg["K"], cfg["V"], cfg["D"]
    N = math.prod(cfg["lead"])
    h, W, E, b = draw(N, K, V, D, bf16, seed=0, lead=cfg["lead"])
    g = torch.Generator(device="cuda").manual_seed(2)
    target = torch.randn(*cfg["lead"], D, device="cuda", generator=g)
    weight = bench_weight(config, cfg["lead"], g)
    n_act = int((weight != 0).sum())
    assert n_act < N
    assert_multiblock(bf16, n_act, K, V, D, 8192)
    z = 1e-4
    xs = [x.requires_grad_(True) for x in (h, W, E, b)]
    loss = swvr.softmax_readout_mse(h, W, E, target, b, weight=weight, z_loss_weight=z)
    grads = torch.autograd.grad(loss, xs)
    torch.cuda.synchronize()
    want_loss, *want = ref.mse_grads_blocked(h.detach().reshape(N, K), W.detach(), E.detach(),
                                             target.reshape(N, D), b.detach(), weight=weight.reshape(N),
                                             reduction="mean", z_loss_weight=z, block=1024)
    errs = {"loss": abs(loss.item() - want_loss.item()) / abs(want_loss.item())}
    for n, a, r in zip(("gh", "gW", "gE", "gb"), grads, want):
        a = a.reshape(r.shape)
        errs[n] = rel_err(a, r)
        c = cosine(a, r)
        assert c >= 0.999, (config, n, c)
    print(config, {k: f"{v:.1e}" for k, v in errs.items()}, flush=True)
    assert errs["loss"] <= 1e-2, errs
    for n in ("gh", "gW", "gE", "gb"):
        assert errs[n] <= 2e-2, (config, n, errs)
    # zero-weight tokens have zero cotangents: their gh rows are exactly zero
    assert grads[0].reshape(N, K)[weight.reshape(N) == 0].abs().max().item() == 0.0
