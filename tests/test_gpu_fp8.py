"""The opt-in e4m3 forward (``swvr_fwd_fp8`` behind ``swvr_amd.fp8``).

The reference has no fp8 path, so there is nothing of its to match: the
kernel is held to the fp64 oracle evaluated on the dequantised operands (the
values it computes with) at the bf16 forward's tolerance, and to the
unquantised readout at a tolerance for e4m3 rounding of h and W.
"""
import pytest
import torch

from oracle import reference as ref
from swvr_amd import fp8
from tests.gpu_util import cosine, rel_err

pytestmark = pytest.mark.gpu


def make(N, K, V, D, seed=0, bias=True):
    g = torch.Generator(device="cuda").manual_seed(seed)
    h = torch.randn(N, K, device="cuda", generator=g)
    W = torch.randn(V, K, device="cuda", generator=g) / K ** 0.5
    E = torch.randn(V, D, device="cuda", generator=g).to(torch.bfloat16)
    b = 0.5 * torch.randn(V, device="cuda", generator=g) if bias else None
    return h, W, E, b


def oracle(h, W, E, b, logit_scale):
    O, lse = ref.softmax_readout_reference(h.double().cpu(), W.double().cpu(), E.double().cpu(),
                                           b.double().cpu() if b is not None else None, logit_scale)
    return O, lse


@pytest.mark.parametrize("N,K,V,D", [(300, 512, 4099, 64), (1, 64, 1000, 5), (1000, 80, 2500, 128),
                                     (517, 2560, 8192, 32), (256, 16, 300, 64)])
@pytest.mark.parametrize("bias", [True, False])
def test_fp8_forward_matches_fp64_on_the_dequantised_operands(N, K, V, D, bias):
    h, W, E, b = make(N, K, V, D, bias=bias)
    O, lse = fp8.softmax_readout_fp8(h, W, E, b, logit_scale=0.7)
    hq, hs = fp8.quantize_tensor(h)
    Wq, ws = fp8.quantize_rows(W)
    Or, lr = oracle(fp8.dequantize(hq, hs), fp8.dequantize(Wq, ws), E, b, 0.7)
    eo, el = rel_err(O, Or), rel_err(lse, lr)
    print(N, K, V, D, bias, f"vs dequantised: O {eo:.1e} lse {el:.1e}")
    assert O.shape == (N, D) and lse.shape == (N,)
    assert eo <= 1e-2 and el <= 1e-5


@pytest.mark.parametrize("K", [512, 2560])
def test_fp8_forward_stays_within_e4m3_rounding_of_the_unquantised_readout(K):
    N, V, D = 512, 8192, 64
    h, W, E, b = make(N, K, V, D, seed=1)
    O, lse = fp8.softmax_readout_fp8(h, W, E, b)
    Or, lr = oracle(h, W, E, b, 1.0)
    eo, el = rel_err(O, Or), (lse.double().cpu() - lr).abs().max().item()
    print(K, f"vs unquantised: O {eo:.2e}, lse max abs {el:.2e}")
    assert eo <= 0.1 and el <= 0.1


def test_fp8_masks_leading_dims_and_reuse_of_a_quantised_W():
    N, K, V, D = 240, 128, 3000, 16
    h, W, E, b = make(N, K, V, D, seed=2)
    b[::3] = float("-inf")  # masked vocabulary rows
    h3 = h.reshape(4, 60, K)
    O, lse = fp8.softmax_readout_fp8(h3, W, E, b)
    assert O.shape == (4, 60, D) and lse.shape == (4, 60)
    O2, lse2 = fp8.softmax_readout_fp8(h3, W, E, b, w_q=fp8.quantize_rows(W))
    assert torch.equal(O, O2) and torch.equal(lse, lse2)   # deterministic, same quantisation
    hq, hs = fp8.quantize_tensor(h)
    Wq, ws = fp8.quantize_rows(W)
    Or, lr = oracle(fp8.dequantize(hq, hs), fp8.dequantize(Wq, ws), E, b, 1.0)
    assert rel_err(O.reshape(N, D), Or) <= 1e-2 and rel_err(lse.reshape(N), lr) <= 1e-5


def torch_quantize(x, per_row):
    """The quantisation rule in torch ops: scale = max(amax, 1e-30) / 448, q = e4m3(x / scale)."""
    x32 = x.to(torch.float32)
    Kp = (x.shape[1] + 15) // 16 * 16
    x32 = torch.nn.functional.pad(x32, (0, Kp - x.shape[1]))
    if per_row:
        scale = x32.abs().amax(dim=1).clamp_min(1e-30) / 448.0
        return (x32 / scale[:, None]).to(fp8.E4M3), scale
    scale = (x32.abs().amax().clamp_min(1e-30) / 448.0).reshape(1)
    return (x32 / scale).to(fp8.E4M3), scale


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("R,K", [(1000, 2560), (37, 100), (5, 7), (1, 16)])
def test_quantisation_is_bit_identical_to_the_torch_cast(dtype, R, K):
    g = torch.Generator(device="cuda").manual_seed(R + K)
    x = (torch.randn(R, K, device="cuda", generator=g) * torch.logspace(-3, 2, R, device="cuda")[:, None]).to(dtype)
    x[0, :3] = 0.0
    if R > 2:
        x[2] = 0.0                                    # an all-zero row: tiny scale, zero bytes
    for per_row in (True, False):
        q, s = fp8._quantize(x, per_row)
        qr, sr = torch_quantize(x, per_row)
        assert torch.equal(s, sr), per_row
        assert torch.equal(q.view(torch.uint8), qr.view(torch.uint8)), per_row
    xs = x[:, : K // 2] if K >= 4 else x               # a strided view (leading dim > K)
    q, s = fp8._quantize(xs, True)
    qr, sr = torch_quantize(xs, True)
    assert torch.equal(q.view(torch.uint8), qr.view(torch.uint8)) and torch.equal(s, sr)


def mixed_grads(h, W, E, b, gO, glse, logit_scale, quantised=True):
    """fp64 gradients of the e4m3 readout: scores from the dequantised h and W, the gradient
    products on h and W as given (the quantisation passes gradients as the identity).
    quantised=False: the scores from h and W themselves (the bf16 readout's gradients)."""
    hq, hs = fp8.quantize_tensor(h)
    Wq, ws = fp8.quantize_rows(W)
    d = lambda t: t.detach().double().cpu()
    hd, Wd = d(fp8.dequantize(hq, hs))[:, : h.shape[1]], d(fp8.dequantize(Wq, ws))[:, : W.shape[1]]
    if not quantised:
        hd, Wd = d(h), d(W)
    S = logit_scale * hd @ Wd.T + (d(b) if b is not None else 0.0)
    P = torch.softmax(S, dim=-1)
    O = P @ d(E)
    gO64, glse64 = d(gO), d(glse)
    delta = (O * gO64).sum(-1) - glse64
    dS = P * (gO64 @ d(E).T - delta[:, None])
    return (logit_scale * dS @ d(W), logit_scale * dS.T @ d(h), P.T @ gO64, dS.sum(0))


@pytest.mark.parametrize("N,K,V,D,chunk,bias", [(300, 512, 3000, 64, 1024, True), (517, 256, 4099, 5, 700, True),
                                               (256, 80, 2000, 128, 1024, False), (64, 16, 1000, 32, 512, True)])
def test_fp8_backward_matches_fp64_with_the_forwards_scores(N, K, V, D, chunk, bias):
    g = torch.Generator(device="cuda").manual_seed(5)
    h = torch.randn(N, K, device="cuda", generator=g).to(torch.bfloat16).requires_grad_(True)
    W = (torch.randn(V, K, device="cuda", generator=g) / K ** 0.5).to(torch.bfloat16).requires_grad_(True)
    E = torch.randn(V, D, device="cuda", generator=g).to(torch.bfloat16).requires_grad_(True)
    b = (0.5 * torch.randn(V, device="cuda", generator=g)).requires_grad_(True) if bias else None
    gO = torch.randn(N, D, device="cuda", generator=g)
    glse = 0.1 * torch.randn(N, device="cuda", generator=g)
    gO[::7] = 0.0
    glse[::7] = 0.0  # zero cotangents: tokens the backward skips
    xs = [x for x in (h, W, E, b) if x is not None]
    O, lse = fp8.softmax_readout_fp8(h, W, E, b, logit_scale=0.8, chunk_size=chunk)
    got = torch.autograd.grad((O * gO).sum() + (lse * glse).sum(), xs)
    want = mixed_grads(h, W, E, b, gO, glse, 0.8)
    for name, a, r in zip(["gh", "gW", "gE", "gb"], got, want):
        err, cos = rel_err(a, r), cosine(a, r)
        print(N, K, V, D, name, f"rel {err:.1e} cos {cos:.6f}")
        assert a.dtype == xs[["gh", "gW", "gE", "gb"].index(name)].dtype
        assert err <= 2e-2 and cos >= 0.999, (name, err, cos)
    assert torch.count_nonzero(got[0][::7]) == 0  # inactive tokens get zero rows
    # the backward used the e4m3 scores: the gradients of bf16 scores are much farther away
    other = mixed_grads(h, W, E, b, gO, glse, 0.8, quantised=False)
    assert rel_err(got[1], other[1]) > 3 * rel_err(got[1], want[1])


def test_fp8_caps_D():
    h, W, E, b = make(64, 64, 500, 200)
    with pytest.raises(NotImplementedError):
        fp8.softmax_readout_fp8(h, W, E, b)


def test_fp8_edge_sizes_no_tokens_and_one_vocabulary_row():
    # no tokens: empty outputs; the backward gives zero vocabulary gradients (as swvr_bwd)
    h, W, E, b = make(0, 64, 300, 16)
    xs = [x.requires_grad_(True) for x in (h, W, E, b)]
    O, lse = fp8.softmax_readout_fp8(*xs)
    assert O.shape == (0, 16) and lse.shape == (0,)
    gW, gE, gb = torch.autograd.grad(O.sum() + lse.sum(), xs[1:], allow_unused=True)
    for g in (gW, gE, gb):
        assert g is None or torch.count_nonzero(g) == 0
    # one vocabulary row: softmax is 1, O = E[0], lse = the score itself
    h, W, E, b = make(40, 32, 1, 8)
    O, lse = fp8.softmax_readout_fp8(h, W, E, b)
    assert torch.allclose(O, E.float().expand(40, 8), rtol=0, atol=0)
    hq, hs = fp8.quantize_tensor(h)
    Wq, ws = fp8.quantize_rows(W)
    S = (fp8.dequantize(hq, hs) @ fp8.dequantize(Wq, ws).T).squeeze(1) + b
    assert rel_err(lse, S) < 1e-5


def test_fp8_accepts_a_strided_quantised_W():
    h, W, E, b = make(100, 64, 700, 16, seed=4)
    Wq, ws = fp8.quantize_rows(W)
    big = torch.zeros(700, 128, dtype=torch.uint8, device="cuda")
    big[:, :64] = Wq.view(torch.uint8)
    big = big.view(fp8.E4M3)                          # rows of 128 bytes, the first 64 used
    O1, l1 = fp8.softmax_readout_fp8(h, W, E, b, w_q=(Wq, ws))
    O2, l2 = fp8.softmax_readout_fp8(h, W, E, b, w_q=(big[:, :64], ws))
    assert torch.equal(O1, O2) and torch.equal(l1, l2)
    with pytest.raises(ValueError):
        fp8.softmax_readout_fp8(h, W, E, b, w_q=(Wq[:, :48], ws))
