"""Host-side checks that need no GPU: the C-ABI library loads and exports every
symbol include/swvr.h declares, its argument checks report errors without
touching the device, and the Python API validates, traces and refuses CPU
tensors the way the reference's does (swvr/api.py:14-22, 37-39)."""
import ctypes
import os
import re

import pytest
import torch

import swvr_amd
from swvr_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "swvr.h")


def declared_symbols():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(swvr_\w+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    names = declared_symbols()
    assert len(names) >= 10, names
    for name in names:
        assert hasattr(lib, name), name
    assert set(names) == set(_lib.SIGNATURES), "binding and header disagree"


def test_abi_constants():
    lib = _lib.load()
    assert lib.swvr_abi_version() == _lib.ABI_VERSION
    for tag in (_lib.BF16, _lib.F16, _lib.F32):
        assert lib.swvr_max_d(tag) == 65536   # no practical cap: wide D runs in slices
    assert lib.swvr_max_d(9) == 0
    assert lib.swvr_kernel_name(0).decode() == "fwd_tile_kernel"
    assert lib.swvr_kernel_name(99) == b""


def test_workspace_sizes():
    lib = _lib.load()
    N, K, V, D = 16384, 2560, 151936, 64
    fwd = lib.swvr_fwd_workspace_size(_lib.BF16, N, K, V, D)
    assert 0 < fwd < 2**30
    bwd = lib.swvr_bwd_workspace_size(_lib.BF16, N, K, V, D, 8192, 1)
    # dS stage (N x 8192 bf16) + fp32 dh accumulator + packed h, the position-ordered h (bf16) and
    # one chunk's packed W rows + small partials: O(N * chunk + (N + chunk) * K)
    need = N * 8192 * 2 + N * K * 4 + (2 * N + 8192) * K * 2
    assert need <= bwd < need + 2**27
    # per vocabulary row only the packed E row (DP = 64) and the bias remain
    grow = lib.swvr_bwd_workspace_size(_lib.BF16, N, K, 2 * V, D, 8192, 1) - bwd
    assert 0 < grow <= V * (64 * 2 + 4) + 2 * 256
    assert lib.swvr_bwd_workspace_size(_lib.BF16, N, K, V, D, 0, 1) == 0
    # a forward wider than one pass (256; fp32 128) reuses one pass's workspace for every slice
    assert lib.swvr_fwd_workspace_size(_lib.F32, N, K, V, 300) == lib.swvr_fwd_workspace_size(_lib.F32, N, K, V, 128)
    assert lib.swvr_fwd_workspace_size(_lib.BF16, N, K, V, 600) == lib.swvr_fwd_workspace_size(_lib.BF16, N, K, V, 256)
    assert lib.swvr_bwd_workspace_size(_lib.BF16, N, K, V, 300, 8192, 1) > bwd


def call_fwd(dtype=_lib.BF16, N=4, K=16, V=8, D=4, h=16, ldh=16, W=16, ldw=16, E=16, lde=4):
    lib = _lib.load()
    p = lambda x: ctypes.c_void_p(x) if x else None
    return lib.swvr_fwd(dtype, N, K, V, D, p(h), ldh, p(W), ldw, p(E), lde, None, 1.0,
                        p(16), p(16), p(16), 1 << 20, None)


@pytest.mark.parametrize("kw,code", [
    (dict(dtype=7), _lib.EDTYPE),
    (dict(K=12, ldh=12, ldw=12), _lib.EINVAL),      # K must be a multiple of 8
    (dict(ldh=8), _lib.EINVAL),                     # ldh < K
    (dict(h=8), _lib.EINVAL),                       # misaligned h
    (dict(W=0), _lib.EINVAL),                       # null W
    (dict(D=65537, lde=65537), _lib.EDTYPE),        # D above SWVR_MAX_D
    (dict(dtype=_lib.F32, D=65537, lde=65537), _lib.EDTYPE),
    (dict(N=-1), _lib.EINVAL),
    (dict(K=(1 << 21) + 8, ldh=(1 << 21) + 8, ldw=(1 << 21) + 8), _lib.EINVAL),  # K above the 32-bit offset cap
])
def test_abi_rejects_bad_arguments_without_touching_the_device(kw, code):
    assert call_fwd(**kw) == code
    assert _lib.load().swvr_last_error()


def test_abi_combine_rejects_bad_arguments_without_touching_the_device():
    lib = _lib.load()
    assert lib.swvr_combine(0, 4, 4, None, None, None, None, None, None) == _lib.EINVAL
    assert b"S=0" in lib.swvr_last_error()
    assert lib.swvr_combine(2, 4, 4, None, None, None, None, None, None) == _lib.EINVAL
    assert lib.swvr_combine(2, 0, 4, None, None, None, None, None, None) == _lib.OK  # no rows: nothing to do
    p = ctypes.c_void_p(16)
    assert lib.swvr_fwd_partial(_lib.BF16, 4, 16, 8, 4, p, 16, p, 16, p, 4, None, 1.0,
                                None, None, None, p, 1 << 20, None) == _lib.EINVAL


def test_abi_mixed_storage_dtypes_are_checked():
    lib = _lib.load()
    p = ctypes.c_void_p(16)
    args = (4, 16, 8, 4, p, 16, p, 16, p, 4, None, 1.0, p, p, p, 1 << 20, None)
    assert lib.swvr_fwd_mixed(_lib.BF16, _lib.F16, _lib.BF16, *args) == _lib.EDTYPE   # h in another 2-byte dtype
    assert b"h dtype" in lib.swvr_last_error()
    assert lib.swvr_fwd_mixed(_lib.F16, _lib.F16, _lib.BF16, *args) == _lib.EDTYPE
    assert b"W dtype" in lib.swvr_last_error()
    # an fp32 W adds the compute-dtype copy of two chunks' rows to the backward workspace
    N, K, V, D = 1024, 512, 4096, 64
    same = lib.swvr_bwd_workspace_size_mixed(_lib.BF16, _lib.BF16, N, K, V, D, 1024, 1)
    f32w = lib.swvr_bwd_workspace_size_mixed(_lib.BF16, _lib.F32, N, K, V, D, 1024, 1)
    assert same == lib.swvr_bwd_workspace_size(_lib.BF16, N, K, V, D, 1024, 1)
    assert f32w - same == 2 * 1024 * K * 2
    one = lib.swvr_bwd_workspace_size_mixed(_lib.BF16, _lib.F32, N, K, V, D, V, 1)  # one chunk
    assert one - lib.swvr_bwd_workspace_size(_lib.BF16, N, K, V, D, V, 1) == V * K * 2


def test_abi_bwd_rejects_bad_chunk_and_gradient_dtype():
    lib = _lib.load()
    p = ctypes.c_void_p(16)
    args = [_lib.BF16, 4, 16, 8, 4, p, 16, p, 16, p, 4, None, 1.0, p, p, p, p]
    rc = lib.swvr_bwd(*args, 0, p, _lib.BF16, None, 0, None, 0, None, p, 1 << 20, None)
    assert rc == _lib.EINVAL and b"chunk" in lib.swvr_last_error()
    rc = lib.swvr_bwd(*args, 64, p, 5, None, 0, None, 0, None, p, 1 << 20, None)
    assert rc == _lib.EDTYPE
    rc = lib.swvr_bwd(*args, 64, None, 0, None, 0, None, 0, p, p, 1 << 20, None)
    assert rc == _lib.EINVAL and b"bias" in lib.swvr_last_error()


def test_check_maps_codes_to_exceptions():
    lib = _lib.load()
    call_fwd(K=12, ldh=12, ldw=12)
    with pytest.raises(ValueError):
        _lib.check(_lib.EINVAL)
    with pytest.raises(NotImplementedError):
        _lib.check(_lib.EDTYPE)
    with pytest.raises(RuntimeError):
        _lib.check(_lib.EHIP)
    _lib.check(_lib.OK)
    assert lib is _lib.load()


def make(N=6, K=12, V=41, D=5, device="cpu", dtype=torch.float32):
    g = torch.Generator().manual_seed(0)
    t = lambda *s: torch.randn(*s, generator=g).to(device=device, dtype=dtype)
    return t(N, K), t(V, K), t(V, D), t(V)


def test_input_validation_matches_reference():
    h, W, E, b = make()
    with pytest.raises(ValueError):
        swvr_amd.softmax_readout(h, W[:, :-1], E)
    with pytest.raises(ValueError):
        swvr_amd.softmax_readout(h, W, E[:-1])
    with pytest.raises(ValueError):
        swvr_amd.softmax_readout(h, W, E, b[:-1])
    with pytest.raises(ValueError):
        swvr_amd.softmax_readout(h, W, E, chunk_size=-1)
    with pytest.raises(ValueError):
        swvr_amd.softmax_readout(h, W[None], E)
    hm, Wm, Em, bm = make(device="meta")
    with pytest.raises(ValueError):
        swvr_amd.softmax_readout_mse(hm, Wm, Em, torch.zeros(6, 5, device="meta"), bm, reduction="max")


def test_cpu_tensors_fail_loudly():
    h, W, E, b = make()
    with pytest.raises(RuntimeError, match="GPU"):
        swvr_amd.softmax_readout(h, W, E, b)


def test_meta_tensors_trace_through_the_fake_kernels():
    h, W, E, b = make(device="meta")
    h = h.reshape(2, 3, 12)
    O, lse = swvr_amd.softmax_readout(h, W, E, b)
    assert O.shape == (2, 3, 5) and lse.shape == (2, 3)
    assert O.dtype == torch.float32 and lse.dtype == torch.float32
    hb, Wb, Eb, bb = (x.to(torch.bfloat16) for x in make(device="meta"))
    O, lse = swvr_amd.softmax_readout(hb, Wb, Eb, bb)
    assert O.dtype == torch.float32   # scores, O and LSE stay fp32 for bf16 inputs
    grads = torch.ops.swvr.chunked_bwd(torch.empty(6, 5, device="meta"), torch.empty(6, device="meta"),
                                       hb, Wb, Eb, bb, O, lse, 1.0, 8, torch.bfloat16, True,
                                       True, False, True, True)
    assert [tuple(g.shape) for g in grads] == [(6, 12), (0,), (41, 5), (41,)]
    assert grads[0].dtype == torch.bfloat16


def test_fp64_inputs_trace_to_fp64_outputs():
    """fp64 compute returns fp64 O and lse (swvr/chunked.py:26-27), in the fakes too."""
    h, W, E, b = (x.double() for x in make(device="meta"))
    O, lse = swvr_amd.softmax_readout(h, W, E, b)
    assert O.dtype == torch.float64 and lse.dtype == torch.float64


@pytest.mark.parametrize("use_triton", [True, False])
def test_op_schemas_take_the_reference_argument_lists(use_triton):
    """swvr::chunked_fwd / chunked_bwd with the reference's positional and keyword arguments
    (swvr/chunked.py:157-161, 170-174), use_triton included; the flag has no effect here."""
    hb, Wb, Eb, bb = (x.to(torch.bfloat16) for x in make(device="meta"))
    O, lse = torch.ops.swvr.chunked_fwd(hb, Wb, Eb, bb, 1.0, 8, torch.bfloat16, use_triton)
    assert O.shape == (6, 5) and lse.shape == (6,) and O.dtype == torch.float32
    O2, _ = torch.ops.swvr.chunked_fwd(h=hb, W=Wb, E=Eb, bias=None, logit_scale=0.5, chunk=4,
                                       cdt=torch.bfloat16, use_triton=use_triton)
    assert O2.shape == (6, 5)
    grads = torch.ops.swvr.chunked_bwd(gO=torch.empty(6, 5, device="meta"), glse=torch.empty(6, device="meta"),
                                       h=hb, W=Wb, E=Eb, bias=bb, O=O, lse=lse, logit_scale=1.0, chunk=8,
                                       cdt=torch.bfloat16, use_triton=use_triton, need_h=False, need_W=True,
                                       need_E=False, need_b=True)
    assert [tuple(g.shape) for g in grads] == [(0,), (41, 12), (0,), (41,)]
    schema = str(torch.ops.swvr.chunked_fwd.default._schema)
    assert "bool use_triton" in schema


def test_drop_in_alias():
    import swvr
    assert swvr.softmax_readout is swvr_amd.softmax_readout
    assert swvr.softmax_readout_mse is swvr_amd.softmax_readout_mse
    assert swvr.SoftmaxReadoutMSE is swvr_amd.SoftmaxReadoutMSE
    assert swvr.softmax_readout_reference is swvr_amd.softmax_readout_reference
    assert set(swvr.__all__) == {"softmax_readout", "softmax_readout_mse", "SoftmaxReadoutMSE",
                                 "softmax_readout_reference"}


def test_public_reference_matches_oracle():
    from oracle import reference as ref
    h, W, E, b = (x.double() for x in make())
    a = swvr_amd.softmax_readout_reference(h, W, E, b, logit_scale=0.5)
    r = ref.softmax_readout_reference(h, W, E, b, logit_scale=0.5)
    for x, y in zip(a, r):
        torch.testing.assert_close(x, y)


def test_default_chunk_size_env(monkeypatch):
    monkeypatch.delenv("SWVR_CHUNK", raising=False)
    assert swvr_amd.default_chunk_size() == 8192
    monkeypatch.setenv("SWVR_CHUNK", "4096")
    assert swvr_amd.default_chunk_size() == 4096


def test_abi_loss_rejects_bad_arguments_without_touching_the_device():
    lib = _lib.load()
    p = ctypes.c_void_p(16)
    ws = lib.swvr_mse_loss_workspace_size(100)
    assert ws == 2 * 7 * 4  # two fp32 partial sums per 16-token workgroup

    def call(N=100, D=8, tdt=_lib.F32, ldt=8, red=2, out=p, gO=None, glse=None, wsb=ws, wsp=p):
        return lib.swvr_mse_loss(N, D, p, p, p, tdt, ldt, None, 0.0, red, out, None, gO, glse, wsp, wsb, None)

    assert call(D=0) == _lib.EINVAL
    assert call(tdt=7) == _lib.EDTYPE
    assert call(red=3) == _lib.EINVAL and b"reduction" in lib.swvr_last_error()
    assert call(ldt=4) == _lib.EINVAL and b"ldt" in lib.swvr_last_error()
    assert call(out=None) == _lib.EINVAL
    assert call(gO=p) == _lib.EINVAL and b"both" in lib.swvr_last_error()
    assert call(wsb=ws - 4) == _lib.EWORKSPACE
    assert call(N=0, red=0, wsb=0, wsp=None) == _lib.OK  # no tokens, no reduction: nothing to do


def test_abi_fp8_forward_checks_arguments_without_touching_the_device():
    lib = _lib.load()
    p = ctypes.c_void_p(16)
    assert lib.swvr_fwd_fp8_workspace_size(100, 64, 1000, 64) > 0
    assert lib.swvr_fwd_fp8_workspace_size(100, 40, 1000, 64) == 0     # K not a multiple of 16
    assert lib.swvr_fwd_fp8_workspace_size(100, 64, 1000, 200) == 0    # D above 128

    def call(K=64, ldh=64, ldw=64, D=16, hs=p, ws=p):
        return lib.swvr_fwd_fp8(8, K, 40, D, p, ldh, hs, p, ldw, ws, p, D, None, 1.0, p, p, p, 1 << 20, None)

    assert call(K=40, ldh=40, ldw=40) == _lib.EINVAL
    assert call(ldh=72) == _lib.EINVAL          # leading dim not a multiple of 16
    assert call(D=200) == _lib.EDTYPE
    assert call(hs=None) == _lib.EINVAL and b"scale" in lib.swvr_last_error()


def test_abi_fp8_backward_checks_arguments_without_touching_the_device():
    lib = _lib.load()
    p = ctypes.c_void_p(16)
    N, K, V, D = 64, 64, 500, 16
    base = lib.swvr_bwd_workspace_size(_lib.BF16, N, K, V, D, 256, 1)
    f8 = lib.swvr_bwd_fp8_workspace_size(N, K, K, V, D, 256, 1)
    assert f8 > base                                   # + e4m3 h over positions and the row factors
    assert lib.swvr_bwd_fp8_workspace_size(N, K, K, V, 200, 256, 1) == 0   # D above 128
    assert lib.swvr_bwd_fp8_workspace_size(N, K, 40, V, D, 256, 1) == 0    # K8 not a multiple of 16

    def call(K8=64, ldhq=64, ldwq=64, hs=p, D=16):
        return lib.swvr_bwd_fp8(N, K, V, D, p, K, p, K, p, D, None, 1.0, p, K8, ldhq, hs, p, ldwq, p,
                                p, p, p, p, 256, p, _lib.BF16, None, 0, None, 0, None, p, 1 << 30, None)

    assert call(K8=48, ldhq=48, ldwq=48) == _lib.EINVAL   # K8 below K
    assert call(ldhq=72) == _lib.EINVAL
    assert call(hs=None) == _lib.EINVAL and b"scale" in lib.swvr_last_error()
    assert call(D=200) == _lib.EDTYPE


def test_embedding_widths_beyond_the_maximum_are_refused():
    lib = _lib.load()
    p = ctypes.c_void_p(16)
    rc = lib.swvr_fwd(_lib.BF16, 4, 16, 8, 65537, p, 16, p, 16, p, 65537, None, 1.0, p, p, p, 1 << 20, None)
    assert rc == _lib.EDTYPE and b"D=65537" in lib.swvr_last_error()


def test_bwd_tiling_reports_the_scores_kernel_plan():
    """swvr_bwd_tiling needs no GPU: the headline's ring-kernel tiling and the general kernel's."""
    t = _lib.bwd_tiling(torch.bfloat16, 16384, 2560, 151936, 64, 8192)
    assert t == dict(BM=256, BV=256, G=8, C=8192, n_chunks=19, DP=64, kernel=1)
    t = _lib.bwd_tiling(torch.bfloat16, 32768, 4096, 256000, 256, 8192)
    assert (t["BM"], t["BV"], t["G"], t["DP"], t["kernel"]) == (256, 256, 8, 256, 2)
    t = _lib.bwd_tiling(torch.float32, 2051, 64, 4096, 128, 4096)
    assert (t["BM"], t["G"], t["C"], t["kernel"]) == (64, 16, 4096, 0)
    # beyond the old caps: the wide kernel streams any multiple of 32 (fp32: 16) columns
    assert (_lib.bwd_tiling(torch.bfloat16, 64, 64, 512, 300, 512)["DP"], _lib.bwd_tiling(torch.bfloat16, 64, 64, 512, 300, 512)["kernel"]) == (320, 2)
    assert _lib.bwd_tiling(torch.bfloat16, 64, 64, 512, 100, 512)["DP"] == 128
    t = _lib.bwd_tiling(torch.float32, 64, 64, 512, 200, 512)
    assert (t["BM"], t["DP"], t["kernel"]) == (128, 208, 2)   # fp32: 128-token blocks
    lib = _lib.load()
    out = (ctypes.c_int64 * 7)()
    assert lib.swvr_bwd_tiling(_lib.BF16, 16, 16, 16, 16, 0, out, 7) == _lib.EINVAL
    assert b"chunk" in lib.swvr_last_error()
    assert lib.swvr_bwd_tiling(9, 16, 16, 16, 16, 64, out, 7) == _lib.EDTYPE
    assert lib.swvr_bwd_tiling(_lib.BF16, 16, 16, 16, 16, 64, None, 7) == _lib.EINVAL


def test_abi_active_forward_checks_arguments_without_touching_the_device():
    """swvr_fwd_active (the weighted loss's forward over its non-zero-weight tokens)."""
    lib = _lib.load()
    N, K, V, D = 3000, 256, 5000, 64
    full = lib.swvr_fwd_workspace_size(_lib.BF16, N, K, V, D)
    act = lib.swvr_fwd_active_workspace_size(_lib.BF16, N, K, V, D)
    # twice the partial rows (the count's re-split) plus flags, positions and the count block
    assert act > full and act - full < full
    assert lib.swvr_fwd_active_workspace_size(3, N, K, V, D) == 0          # no e4m3 active forward
    assert lib.swvr_fwd_active_workspace_size(_lib.F32, N, K, V, 300) > 0  # fp32, D in slices
    p = ctypes.c_void_p(16)

    def call(n=N, weight=p, ws=act, wsp=p, dtype=_lib.BF16):
        return lib.swvr_fwd_active(dtype, dtype, dtype, n, K, V, D, p, K, p, K, p, D, None, 1.0, weight,
                                   p, p, wsp, ws, None)

    assert call(weight=None) == _lib.EINVAL and b"weight" in lib.swvr_last_error()
    assert call(ws=act - 256) == _lib.EWORKSPACE
    assert call(dtype=9) == _lib.EDTYPE
    assert call(n=0, weight=None, ws=0, wsp=None) == _lib.OK  # no tokens: nothing to do


def test_the_loss_skips_zero_weight_readouts_only_on_the_gpu_path():
    from swvr_amd.api import _skips_zero_weight
    h, W = torch.randn(8, 16), torch.randn(40, 16)
    w = torch.ones(8)
    assert not _skips_zero_weight(h, W, w, "mean")  # CPU tensors: the op raises, as every other path
    hm, Wm, wm = h.to("meta"), W.to("meta"), w.to("meta")
    assert not _skips_zero_weight(hm, Wm, wm, "mean")
