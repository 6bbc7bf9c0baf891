"""swvr_mse_loss_noalloc: the loss entry point that allocates nothing.

Its partial sums live in a fixed per-device array instead of the caller's
workspace; otherwise it runs the same kernels as swvr_mse_loss, so every output
must equal swvr_mse_loss's bit for bit.  Two calls in a row, the second with
fewer tokens, check that the array's leftover contents from the first call do
not reach the second's result.  Called through the C ABI.
"""
import ctypes

import pytest
import torch

from swvr_amd import _lib

pytestmark = pytest.mark.gpu
REDUCE = {"none": 0, "sum": 1, "mean": 2}
MAX_N = 1 << 22


def inputs(N, D, seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    O = torch.randn(N, D, device="cuda", generator=g)
    lse = 10 + torch.randn(N, device="cuda", generator=g)
    target = torch.randn(N, D, device="cuda", generator=g).to(torch.bfloat16)
    weight = (torch.rand(N, device="cuda", generator=g) > 0.2).float()
    return O, lse, target, weight


def call(noalloc, O, lse, target, weight, z, reduction):
    """One loss call; returns (status, out, scale, gO, glse)."""
    lib = _lib.load()
    N, D = O.shape
    red = REDUCE[reduction]
    out = torch.full((N,) if red == 0 else (1,), -7.0, device="cuda")
    scale = torch.full((1,), -7.0, device="cuda")
    gO = torch.full_like(O, -7.0)
    glse = torch.full_like(lse, -7.0)
    p = _lib.ptr
    stream = _lib.stream_of(O.device)
    args = (N, D, p(O), p(lse), p(target), _lib.DTYPE_TAG[target.dtype], D, p(weight), float(z), red,
            p(out), p(scale) if red else None, p(gO), p(glse))
    if noalloc:
        rc = lib.swvr_mse_loss_noalloc(*args, stream)
    else:
        ws_bytes = lib.swvr_mse_loss_workspace_size(N) if red else 0
        ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device="cuda")
        rc = lib.swvr_mse_loss(*args, p(ws), ws_bytes, stream)
    torch.cuda.synchronize()
    return rc, out, scale, gO, glse


def same(a, b):
    torch.testing.assert_close(a, b, rtol=0, atol=0, equal_nan=True)


@pytest.mark.parametrize("reduction", ["sum", "mean", "none"])
@pytest.mark.parametrize("weighted", [True, False])
def test_noalloc_loss_equals_the_workspace_entry_point(reduction, weighted):
    for N, D, seed in ((200003, 64, 0), (3001, 16, 1)):  # the second call is smaller
        O, lse, target, weight = inputs(N, D, seed)
        w = weight if weighted else None
        want = call(False, O, lse, target, w, 1e-4, reduction)
        got = call(True, O, lse, target, w, 1e-4, reduction)
        assert want[0] == _lib.OK and got[0] == _lib.OK, _lib.load().swvr_last_error()
        for a, b in zip(got[1:], want[1:]):
            same(a, b)
        # and the value is the loss: sum (or mean) of the weighted per-token terms
        if reduction != "none":
            per = ((O - target.float()) ** 2).mean(-1) + 1e-4 * lse ** 2
            if w is not None:
                per = per * w
            ref = per.double().sum() / (1 if reduction == "sum" else (w.sum() if w is not None else N))
            assert abs(got[1].item() - ref.item()) <= 1e-5 * abs(ref.item())


def test_noalloc_loss_with_no_tokens_matches():
    O, lse, target, weight = inputs(0, 8, 2)
    want = call(False, O, lse, target, weight, 0.0, "mean")
    got = call(True, O, lse, target, weight, 0.0, "mean")
    assert want[0] == got[0] == _lib.OK
    same(got[1], want[1])


def test_noalloc_loss_rejects_more_tokens_than_its_scratch_holds():
    """Checked on the host before anything is launched (no device pointer is read)."""
    lib = _lib.load()
    dummy = ctypes.c_void_p(16)
    rc = lib.swvr_mse_loss_noalloc(MAX_N + 1, 4, dummy, dummy, dummy, _lib.F32, 4, None, 0.0, 1, dummy, None,
                                   None, None, None)
    assert rc == _lib.EINVAL
    assert b"maximum" in lib.swvr_last_error()
