"""Benchmark: fwd+bwd of swvr_amd.softmax_readout_mse on one MI355X.

    python bench.py                      # headline (config 3), 150 timed steps (about 6 s of GPU work)
    python bench.py --config 2 --steps 20 --warmup 3
    python bench.py --no-cpu             # skip the CPU baseline leg
    python bench.py --copy-probe-mib 1024  # only a plain device copy (HBM counter calibration)
    python bench.py --mfma-probe         # only the matrix-core probe (the power / clock ceiling)
    python bench.py --library-gemm       # only hipBLASLt (torch.mm) on the gradient GEMMs' shapes
    python bench.py --reference-table    # only the reference bench's eager vs swvr table (ms, peak GiB)

A step is one forward + backward of the MSE loss (the reference's bench,
bench/bench.py:30-45) on seeded synthetic inputs already resident in HBM.
Prints ONE JSON line.  ``value`` is the algorithmic fwd+bwd TFLOP/s,
2 N V (4K + 3D) / step time — the FLOPs of the reference's algorithm with one
score recompute (docs/DESIGN.md:39); ``ms_per_step`` is the step time.  Both
passes skip tokens of weight 0 in the loss (their loss terms are 0 x finite, so
the forward leaves their readout out and their cotangents are zero):
``active_tokens`` says how many they ran over, ``work_tflops`` counts only the
FLOPs done, and the per-kernel rates and the roofline are priced on them.

The dominant kernel's roofline is measured live: every launch in the timed
region is bracketed by HIP events on its own stream (the C ABI's timing
record), and its average duration is priced against its algorithmic FLOPs.
The CPU baseline times this repository's restatement of the reference's
chunked CPU path (oracle/chunked.py) on the host cores, on a token sample of
the same workload.

``fp8`` reports the opt-in e4m3 path (swvr_amd.fp8) on the same inputs after
the timed bf16 steps: the forward with W quantised once, and the same fwd+bwd
step with h and W quantised every step.  It is outside the reference's
precision policy and is not part of ``value``.
"""
import argparse
import json
import os
import sys
import time

import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

METRIC = "fwd+bwd ms, TFLOP/s & % bf16 MFMA peak at N16k K2560 V152k D64; peak GiB"
PEAK_BF16_TFLOPS = 2516.6   # MI355X dense bf16 MFMA: 256 CU x 2.4 GHz x 4096 flop/clk
PEAK_HBM_GBS = 8000.0

# BASELINE.json configs (2-5 run on the GPU; config 1 is the CPU plumbing case)
CONFIGS = {
    2: dict(N=16384, K=1024, V=151936, D=16, bias=False, weight=None, z=0.0),
    3: dict(N=16384, K=2560, V=151936, D=64, bias=True, weight="bernoulli", z=1e-4),
    4: dict(N=8192, K=4096, V=128256, D=128, bias=True, weight=None, z=0.0),
    5: dict(N=32768, K=4096, V=256000, D=256, bias=True, weight="ragged", z=1e-4, lead=(8, 4096)),
}


def make_inputs(cfg, device, seed=0):
    """Draw order h, W, bias, E, target, weight; fp32 draws cast to bf16."""
    g = torch.Generator(device=device).manual_seed(seed)
    N, K, V, D = cfg["N"], cfg["K"], cfg["V"], cfg["D"]
    shape = (*cfg.get("lead", (N,)), K)
    r = lambda *s, sc=1.0: sc * torch.randn(*s, device=device, generator=g)
    h = r(*shape).to(torch.bfloat16)
    W = r(V, K, sc=K ** -0.5).to(torch.bfloat16)
    b = r(V, sc=0.02).to(torch.bfloat16) if cfg["bias"] else None
    E = r(V, D).to(torch.bfloat16)
    target = r(*shape[:-1], D)
    weight = None
    if cfg["weight"] == "bernoulli":
        weight = (torch.rand(*shape[:-1], device=device, generator=g) >= 0.1).float()
    elif cfg["weight"] == "ragged":
        rows, T = shape[0], shape[1]
        tails = torch.randint(0, 1025, (rows,), device=device, generator=g)
        pos = torch.arange(T, device=device)[None, :]
        weight = (pos < (T - tails)[:, None]).float()
    params = [x.requires_grad_(True) for x in (h, W, E, b) if x is not None]
    return h, W, E, b, target, weight, params


def step_fn(swvr, h, W, E, b, target, weight, z, chunk):
    return swvr.softmax_readout_mse(h, W, E, target, b, weight=weight, z_loss_weight=z, chunk_size=chunk)


def algorithmic_flops(N, K, V, D):
    fwd = 2.0 * N * V * (K + D)
    return fwd, 2.0 * N * V * (4 * K + 3 * D)


def kernel_flops(name, N, K, V, D, n_act=None, de_in_gemm=False):
    """Algorithmic FLOPs of all launches of one kernel kind over one step.

    Both passes run over the ``n_act`` tokens of non-zero weight (a zero-weight
    token's loss term is 0 x finite: no readout, zero cotangents), so the kernels
    are priced on the work they do: n_act tokens.  ``de_in_gemm``: the
    wide-embedding scores kernel stages P and the gradient GEMM launch forms
    dE = P^T gO."""
    nb = N if n_act is None else n_act
    if name == "fwd_tile_kernel":
        return 2.0 * nb * V * (K + D)            # S = h W^T, P E
    if name == "bwd_scores_kernel":
        # S recompute, dP = gO E^T (and dE = P^T gO unless the GEMM launch forms it)
        return 2.0 * nb * V * (K + (1 if de_in_gemm else 2) * D)
    if name == "bwd_gemm_kernel":
        return 4.0 * nb * V * K + (2.0 * nb * V * D if de_in_gemm else 0.0)  # dh = dS W, dW = dS^T h (, dE)
    return 0.0


TRAFFIC_PATH = os.path.join(ROOT, "profiles", "readout_traffic.json")
STREAMING_KERNELS = ("fwd_tile_kernel", "bwd_scores_kernel", "bwd_gemm_kernel")


def source_sha():
    """SHA-256 (16 hex digits) of the HIP sources the library is built from: counter figures
    measured on another build of them are stale."""
    import hashlib
    d = os.path.join(ROOT, "swvr_amd", "csrc")
    h = hashlib.sha256()
    for name in sorted(os.listdir(d)):
        if name.endswith((".hip", ".hpp")):
            h.update(name.encode())
            with open(os.path.join(d, name), "rb") as f:
                h.update(f.read())
    return h.hexdigest()[:16]


def load_traffic():
    """The committed counter summary (profiles/readout_traffic.json) and whether it was measured
    on these sources."""
    try:
        with open(TRAFFIC_PATH) as f:
            t = json.load(f)
    except (OSError, ValueError):
        return None, False
    return t, t.get("source_sha") == source_sha()


def measured_traffic(t, config, kernel):
    """Calibrated L2-miss (fetch, write) bytes per launch of ``kernel`` at ``config``, or None
    (fabric bytes: Infinity Cache hits included)."""
    try:
        e = t["configs"][str(config)][kernel]
    except (TypeError, KeyError):
        return None
    return e["fetch_kib"] * 1024 * t["fetch_scale"], e["write_kib"] * 1024 * t["write_scale"]


def algorithmic_bytes(name, N, K, V, D, chunk, n_act, wide):
    """Bytes one launch must move at least: each operand read once, each result written once.
    fwd: h of the active tokens, W, E in, O and lse (every token) out.  scores (a chunk of C rows): h of the active tokens, W_c, E_c,
    gO in; the dS stage (and the P stage of the wide kernel) out.  gradient GEMM (a chunk): the dS
    stage, h, W_c in; gW_c out; the fp32 dh accumulator read and written."""
    C = min(chunk, V)
    if name == "fwd_tile_kernel":
        return 2 * (n_act * K + V * K + V * D) + 4 * N * (D + 1)
    if name == "bwd_scores_kernel":
        return 2 * (n_act * K + C * K + C * D + n_act * D) + 2 * C * n_act * (2 if wide else 1)
    if name == "bwd_gemm_kernel":
        return 2 * (C * n_act + n_act * K + 2 * C * K) + 8 * n_act * K + (2 * C * n_act if wide else 0)
    return None


def traffic_summary(root):
    """The traffic file from rocprofv3 counter runs under ``root``: fetch_c<N>/ and write_c<N>/
    (FETCH_SIZE and WRITE_SIZE passes of ``bench.py --config N --no-cpu --no-fp8``) and copy_fetch/,
    copy_write/ (the same counters over ``bench.py --copy-probe-mib 1024``, which moves 1 GiB each
    way per launch and calibrates them).  Per-dispatch averages of this package's streaming kernels."""
    import csv
    import glob
    import re

    def per_kernel(d, counter):
        acc = {}
        for f in glob.glob(os.path.join(root, d, "**", "*counter_collection.csv"), recursive=True):
            for r in csv.DictReader(open(f)):
                if r["Counter_Name"] != counter:
                    continue
                m = re.search(r"(fwd_tile_kernel|fwd_stream_kernel|bwd_scores_ring_kernel|bwd_scores_wide_kernel|"
                              r"bwd_scores_kernel|bwd_gemm_kernel|elementwise_kernel|copy)", r["Kernel_Name"])
                if not m:
                    continue
                # the launch-timing kinds: both forward kernels are "fwd_tile_kernel", every scores
                # kernel "bwd_scores_kernel"
                k = ("bwd_scores_kernel" if m.group(1).startswith("bwd_scores") else
                     "fwd_tile_kernel" if m.group(1).startswith("fwd_") else m.group(1))
                acc.setdefault(k, []).append(float(r["Counter_Value"]))
        return {k: sum(v) / len(v) for k, v in acc.items()}, {k: len(v) for k, v in acc.items()}

    mib = 1024 * 1024
    cf, _ = per_kernel("copy_fetch", "FETCH_SIZE")
    cw, _ = per_kernel("copy_write", "WRITE_SIZE")
    copy_f = max(cf.values()) if cf else None
    copy_w = max(cw.values()) if cw else None
    out = {"about": "L2-miss (fabric) bytes per dispatch of the streaming kernels: rocprofv3 FETCH_SIZE and "
                    "WRITE_SIZE (KiB per dispatch, averaged; they count the L2's requests to the fabric, Infinity "
                    "Cache hits included, so they bound DRAM traffic from above) scaled by what the same counters "
                    "read for a plain 1 GiB copy, which misses the 256 MB Infinity Cache; "
                    "bytes = fetch_kib * 1024 * fetch_scale + write_kib * 1024 * write_scale. "
                    "source_sha: the HIP sources measured (bench.py source_sha).",
           "source_sha": source_sha(),
           "fetch_scale": round(mib / copy_f, 4) if copy_f else None,
           "write_scale": round(mib / copy_w, 4) if copy_w else None,
           "copy_probe_kib": {"fetch": copy_f, "write": copy_w},
           "configs": {}}
    for c in sorted(CONFIGS):
        f, nf = per_kernel(f"fetch_c{c}", "FETCH_SIZE")
        w, _ = per_kernel(f"write_c{c}", "WRITE_SIZE")
        if f:
            out["configs"][str(c)] = {k: {"fetch_kib": round(f[k], 1), "write_kib": round(w.get(k, 0.0), 1),
                                          "dispatches": nf[k]} for k in STREAMING_KERNELS if k in f}
    return out


def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return None


def cpu_baseline(cfg, tokens, chunk, device):
    """Time oracle/chunked.py (the reference's CPU algorithm) fwd+bwd on `tokens` tokens, on every
    host CPU this process may use (the affinity mask, capped by OMP_NUM_THREADS when it is set)."""
    from oracle import chunked
    usable = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    cap = int(os.environ.get("OMP_NUM_THREADS", "0") or 0)
    torch.set_num_threads(min(usable, cap) if cap > 0 else usable)
    N, K, V, D = cfg["N"], cfg["K"], cfg["V"], cfg["D"]
    g = torch.Generator(device=device).manual_seed(1)
    r = lambda *s, sc=1.0: (sc * torch.randn(*s, device=device, generator=g)).to(torch.bfloat16).cpu()
    h, W, E = r(tokens, K), r(V, K, sc=K ** -0.5), r(V, D)
    b = r(V, sc=0.02) if cfg["bias"] else None
    gO = torch.randn(tokens, D) * 1e-3
    glse = torch.randn(tokens) * 1e-4
    threads = torch.get_num_threads()
    t0 = time.perf_counter()
    O, lse = chunked.forward(h, W, E, b, 1.0, chunk, torch.bfloat16)
    chunked.backward(gO, glse, h, W, E, b, O, lse, 1.0, chunk, torch.bfloat16)
    dt = time.perf_counter() - t0
    _, flops = algorithmic_flops(tokens, K, V, D)
    return {"value": round(flops / dt / 1e12, 4), "unit": "TFLOP/s", "cores": threads, "kind": "port",
            "os_cpu_count": os.cpu_count(), "usable_cpus": usable, "torch_threads": threads,
            "cpu_model": cpu_model(), "seconds": round(dt, 2),
            "sample": f"fwd+bwd of {tokens} tokens x the full V={V}, K={K}, D={D} (bf16 operands upcast "
                      f"to fp32 BLAS, vocabulary chunk {chunk}) in {dt:.1f} s on {threads} threads; the "
                      f"rate is the workload's 2 N V (4K + 3D) flops over that time (one timed iteration)"}


def copy_probe(mib):
    """A plain copy of a known size: reads and writes exactly ``mib`` MiB per launch."""
    src = torch.ones(mib * 2**20 // 4, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(5):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_probe_mib": mib, "launches": 5}), flush=True)


def mfma_probe(iters=1 << 20, launches=3):
    """Matrix-core rate of the bare k16 step (swvr_probe_mfma): 256 workgroups of 8 waves (one per
    CU, two waves per SIMD, as the hot kernels), each wave-step 8 x 32x32x16 bf16 MFMAs = 2^18 flops.
    Modes: random operands in registers, zeros in registers, random operands read from LDS each
    step (6, 4 or 3 reads per 8 MFMAs), the 6 reads in the hot loops' software-pipelined order,
    4 LDS reads with the B operands loaded from an L2-resident array into registers, and the hot
    loops' whole step (pipelined reads, a barrier and 32 KB of direct-to-LDS stage loads every 2
    steps), and that step with the barrier and 64 KB of stage loads every 4 steps (two slices per
    stage).  The launches of a mode run back to back; the rate is the mean over them."""
    from swvr_amd import _lib
    lib = _lib.load()
    wgs = 256
    out = torch.empty(wgs * 512, dtype=torch.float32, device="cuda")
    flops = float(wgs) * 8 * iters * 2.0 ** 18
    res = {}
    for mode, name in ((0, "random_registers"), (1, "zero_registers"), (2, "random_lds"),
                       (3, "random_lds_4_reads"), (4, "random_lds_3_reads"), (5, "random_lds_pipelined"),
                       (6, "random_lds_4_reads_b_from_l2"), (7, "random_lds_pipelined_stage_loads_barriers"),
                       (8, "random_lds_pipelined_stage_loads_barrier_per_4_steps")):
        _lib.check(lib.swvr_probe_mfma(wgs, 1 << 14, mode, _lib.ptr(out), _lib.stream_of(out.device)))
        torch.cuda.synchronize()
        t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0.record()
        for _ in range(launches):
            _lib.check(lib.swvr_probe_mfma(wgs, iters, mode, _lib.ptr(out), _lib.stream_of(out.device)))
        t1.record()
        torch.cuda.synchronize()
        ms = t0.elapsed_time(t1) / launches
        tf = flops / (ms * 1e-3) / 1e12
        res[name] = {"ms_per_launch": round(ms, 2), "tflops": round(tf, 1), "pct_bf16_peak": round(100 * tf / PEAK_BF16_TFLOPS, 1)}
        print(json.dumps({"mfma_probe": name, **res[name]}), flush=True)
    return res


def library_gemm(cfg, chunk, reps=10):
    """Calibration of the gradient GEMMs against the vendor library (hipBLASLt through torch.mm) on
    one vocabulary chunk of this configuration: W, E and bias cut to their first ``chunk`` rows, so
    that the whole backward is one chunk.

    * ``real_ds``: the library on the dS our kernel consumes.  The same one-chunk problem runs
      through swvr_amd (the MSE loss with the config's weight and z-loss, forward and backward, its
      launches timed); torch recomputes that chunk's dS over the active tokens from swvr_amd's O
      and lse (S in fp32, P = exp(S + b - lse), dP from gO rounded to bf16, dS rounded to bf16) and
      times dW_c = dS^T h (C x Q)(Q x K, bf16 out) and dh = dS W_c (Q x C)(C x K, fp32 out).  Operand
      values set the chip's power and clock, so only identical operands compare kernels.
      ``bwd_gemm_kernel`` forms both products in one launch (dh read-modify-written in fp32) and
      the chunk's dE / db reduction after its tiles.
    * ``normal_operands``: the library on N(0,1) bf16 operands of the same shapes (the earlier
      calibration).
    Measurement only: the product's gradient GEMMs are this repository's own kernel."""
    import swvr_amd as swvr
    from swvr_amd import _lib
    dev = torch.device("cuda")
    h, W, E, b, target, weight, _ = make_inputs(cfg, dev)
    N, K, D = cfg["N"], cfg["K"], cfg["D"]
    h = h.detach().reshape(-1, K)
    target = target.reshape(-1, D)
    weight = weight.reshape(-1) if weight is not None else None
    C = min(chunk, cfg["V"])
    Wc = W.detach()[:C].clone().requires_grad_(True)
    Ec = E.detach()[:C].clone().requires_grad_(True)
    bc = b.detach()[:C].clone().requires_grad_(True) if b is not None else None
    hl = h.clone().requires_grad_(True)
    z = cfg["z"]

    def ours():
        for x in (hl, Wc, Ec, bc):
            if x is not None:
                x.grad = None
        swvr.softmax_readout_mse(hl, Wc, Ec, target, bc, weight=weight, z_loss_weight=z, chunk_size=C).backward()

    ours()
    torch.cuda.synchronize()
    _lib.kernel_timing(True)
    _lib.kernel_timing(None)
    for _ in range(reps):
        ours()
    torch.cuda.synchronize()
    k = _lib.kernel_timing(None)
    _lib.kernel_timing(False)
    gemm_ms = k["bwd_gemm_kernel"][0] / k["bwd_gemm_kernel"][1]

    with torch.no_grad():
        O, lse = swvr.softmax_readout(h, Wc.detach(), Ec.detach(), bc.detach() if bc is not None else None,
                                      chunk_size=C)
        w = weight if weight is not None else torch.ones(N, device=dev)
        den = w.sum()
        gO = 2.0 * (O - target) * (w / (D * den))[:, None]
        glse = 2.0 * z * lse * w / den
        rows = torch.nonzero(w != 0).flatten()
        n_act = rows.numel()
        Q = (n_act + 31) // 32 * 32
        hA = torch.zeros(Q, K, dtype=torch.bfloat16, device=dev)
        hA[:n_act] = h[rows]
        gOA = gO[rows].to(torch.bfloat16).float()
        S = hA[:n_act].float() @ Wc.detach().float().t()
        if bc is not None:
            S += bc.detach().float()[None, :]
        P = torch.exp(S - lse[rows][:, None])
        del S
        dP = gOA @ Ec.detach().float().t()
        delta = (O[rows] * gOA).sum(1) - glse[rows]
        dS = torch.zeros(Q, C, dtype=torch.bfloat16, device=dev)
        dS[:n_act] = (P * (dP - delta[:, None])).to(torch.bfloat16)
        del P, dP
        dSt = dS.t().contiguous()
        Wcb = Wc.detach().contiguous()
    flops = 2.0 * C * Q * K

    def timed(fn):
        fn()
        torch.cuda.synchronize()
        t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0.record()
        for _ in range(reps):
            fn()
        t1.record()
        torch.cuda.synchronize()
        ms = t0.elapsed_time(t1) / reps
        return {"ms": round(ms, 3), "tflops": round(flops / (ms * 1e-3) / 1e12, 1)}

    real = {"dW_bf16_out": timed(lambda: torch.mm(dSt, hA)),
            "dh_fp32_out": timed(lambda: torch.mm(dS, Wcb, out_dtype=torch.float32))}
    lib_ms = real["dW_bf16_out"]["ms"] + real["dh_fp32_out"]["ms"]
    real["library_pair_ms"] = round(lib_ms, 3)
    real["library_pair_tflops"] = round(2 * flops / (lib_ms * 1e-3) / 1e12, 1)
    real["bwd_gemm_kernel_ms"] = round(gemm_ms, 3)
    real["bwd_gemm_kernel_tflops"] = round(2 * flops / (gemm_ms * 1e-3) / 1e12, 1)
    real["ds_abs_mean"] = float(dS.float().abs().mean())
    g = torch.Generator(device="cuda").manual_seed(0)
    r = lambda *s: torch.randn(*s, device="cuda", generator=g).to(torch.bfloat16)
    Sn, hn, Wn = r(C, Q), r(Q, K), r(C, K)
    Snt = Sn.t().contiguous()
    normal = {"dW_bf16_out": timed(lambda: torch.mm(Sn, hn)), "dh_bf16_out": timed(lambda: torch.mm(Snt, Wn)),
              "dh_fp32_out": timed(lambda: torch.mm(Snt, Wn, out_dtype=torch.float32))}
    return {"shape": {"C": C, "Q": Q, "K": K, "active_tokens": n_act}, "real_ds": real, "normal_operands": normal}


# The reference bench's shapes (bench/bench.py:14-18): N (tokens per step), K, V, D
REFERENCE_SHAPES = {"0.6B": (16384, 1024, 151936, 16), "4B": (16384, 2560, 151936, 64),
                    "8B": (8192, 4096, 128256, 128)}


def reference_table(chunks=(8192,), iters=5):
    """The reference's own benchmark table (bench/bench.py:30-71, README.md:47-53) on this GPU: fwd+bwd
    time and peak memory of the unweighted MSE loss, the eager formula that materialises the [N, V]
    logits (bench/bench.py:21-23, run by torch on this GPU) beside swvr_amd, at the reference's three
    shapes and input draws (h ~ N(0,1), W ~ N(0, 9/K), E ~ N(0,1), bias ~ N(0, 0.25), bf16; target
    fp32).  Peak memory is measured above the inputs and includes the gradient buffers; 2 untimed
    steps, then ``iters`` timed ones.  Measurement only: the eager leg is torch's, not the product."""
    import swvr_amd as swvr

    def eager(h, W, E, b, target, chunk=None):
        O = torch.softmax(torch.addmm(b, h, W.T).float(), dim=-1) @ E.float()
        return (O - target).pow(2).mean()

    def ours(h, W, E, b, target, chunk=None):
        return swvr.softmax_readout_mse(h, W, E, target, b, chunk_size=chunk)

    def measure(fn, inputs, chunk):
        torch.cuda.synchronize()
        base = torch.cuda.memory_allocated()
        torch.cuda.reset_peak_memory_stats()
        try:
            for _ in range(2):
                fn(*inputs, chunk=chunk).backward()
            torch.cuda.synchronize()
            peak = (torch.cuda.max_memory_allocated() - base) / 2**30
            t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            t0.record()
            for _ in range(iters):
                fn(*inputs, chunk=chunk).backward()
            t1.record()
            torch.cuda.synchronize()
            return t0.elapsed_time(t1) / iters, peak
        except torch.OutOfMemoryError:
            return None, None
        finally:
            for x in inputs[:4]:
                x.grad = None
            torch.cuda.empty_cache()

    rows = []
    for name, (N, K, V, D) in REFERENCE_SHAPES.items():
        g = torch.Generator(device="cuda").manual_seed(0)
        r = lambda *s, sc=1.0: (sc * torch.randn(*s, device="cuda", generator=g)).to(torch.bfloat16)
        inputs = [r(N, K), r(V, K, sc=3 / K ** 0.5), r(V, D), r(V, sc=0.5)]
        inputs = [x.requires_grad_(True) for x in inputs] + [torch.randn(N, D, device="cuda")]
        runs = [("eager", eager, None)] + [(f"swvr_amd C={c}", ours, c) for c in chunks]
        for label, fn, chunk in runs:
            ms, gib = measure(fn, inputs, chunk)
            row = {"shape": name, "N": N, "K": K, "V": V, "D": D, "run": label,
                   "ms": None if ms is None else round(ms, 2), "peak_gib": None if gib is None else round(gib, 2)}
            print(json.dumps({"reference_table": row}), flush=True)
            rows.append(row)
        del inputs
    return rows


def fp8_path(h, W, E, b, target, weight, z, chunk, params, fwd_flops, flops, iters):
    """The opt-in e4m3 path (swvr_amd.fp8) on the same inputs, reported beside the bf16 line
    (not part of it).  Forward: W quantised once, as a server would keep it; each call quantises
    h.  Training step: fwd+bwd of the same MSE loss, h and W quantised every step, the backward
    recomputing the e4m3 scores.  TF/s count the same 2NV(K+D) and 2NV(4K+3D) as the bf16 line."""
    from swvr_amd import _lib, fp8

    def step():
        for p in params:
            p.grad = None
        fp8.softmax_readout_mse_fp8(h, W, E, target, b, weight=weight, z_loss_weight=z, chunk_size=chunk).backward()

    step()
    torch.cuda.synchronize()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0.record()
    for _ in range(iters):
        step()
    t1.record()
    torch.cuda.synchronize()
    step_ms = t0.elapsed_time(t1) / iters
    for p in params:
        p.grad = None
    with torch.no_grad():
        fp8.quantize_rows(W)  # first call: kernel load
        q0, q1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        q0.record()
        wq = fp8.quantize_rows(W)
        q1.record()
        fp8.softmax_readout_fp8(h, W, E, b, w_q=wq)
        torch.cuda.synchronize()
        _lib.kernel_timing(True)
        _lib.kernel_timing(None)
        s0, s1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s0.record()
        for _ in range(iters):
            fp8.softmax_readout_fp8(h, W, E, b, w_q=wq)
        s1.record()
        torch.cuda.synchronize()
        k = _lib.kernel_timing(None)
        _lib.kernel_timing(False)
    del wq
    ms = s0.elapsed_time(s1) / iters
    tile = k["fwd_tile_kernel"][0] / iters
    return {"fwd_ms": round(ms, 3), "fwd_tflops": round(fwd_flops / (ms * 1e-3) / 1e12, 1),
            "fwd_tile_kernel_ms": round(tile, 3),
            "fwd_tile_kernel_tflops": round(fwd_flops / (tile * 1e-3) / 1e12, 1),
            "w_quantise_ms": round(q0.elapsed_time(q1), 3),
            "step_ms": round(step_ms, 3), "step_tflops": round(flops / (step_ms * 1e-3) / 1e12, 1),
            "dtype": "e4m3 h and W in the scores; bf16 E, P, dS and the gradient products"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=150)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--config", type=int, default=3, choices=sorted(CONFIGS))
    ap.add_argument("--chunk", type=int, default=8192)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-tokens", type=int, default=4096)
    ap.add_argument("--copy-probe-mib", type=int, default=0,
                    help="run only a plain device-to-device copy of this many MiB, 5 times, and exit: "
                         "its FETCH_SIZE / WRITE_SIZE under rocprofv3 --pmc calibrate the L2-miss (fabric) traffic counters")
    ap.add_argument("--no-fp8", action="store_true", help="skip the opt-in e4m3 leg")
    ap.add_argument("--traffic-from", default=None,
                    help="print the traffic summary (profiles/readout_traffic.json) built from rocprofv3 "
                         "counter runs under this directory, and exit")
    ap.add_argument("--library-gemm", action="store_true",
                    help="only time torch.mm (hipBLASLt) on the config's gradient GEMM shapes (calibration)")
    ap.add_argument("--reference-table", action="store_true",
                    help="run only the reference's own benchmark table (bench/bench.py): eager vs swvr_amd "
                         "fwd+bwd time and peak memory at its three shapes")
    ap.add_argument("--mfma-probe", action="store_true",
                    help="run only the matrix-core probe (swvr_probe_mfma: the bare MFMA step with random, zero "
                         "and LDS-fed operands) and print its rates")
    args = ap.parse_args()
    if args.copy_probe_mib:
        copy_probe(args.copy_probe_mib)
        return
    if args.library_gemm:
        print(json.dumps({"library_gemm": library_gemm(CONFIGS[args.config], args.chunk)}), flush=True)
        return
    if args.mfma_probe:
        print(json.dumps({"mfma_probe_summary": mfma_probe()}), flush=True)
        return
    if args.reference_table:
        reference_table()
        return
    if args.traffic_from:
        print(json.dumps(traffic_summary(args.traffic_from), indent=1))
        return
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print(json.dumps({"error": "this build measures one GPU only (N=1); multi-GPU runs are not part of it"}))
        sys.exit(2)

    import swvr_amd as swvr
    from swvr_amd import _lib
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    cfg = CONFIGS[args.config]
    N, K, V, D = cfg["N"], cfg["K"], cfg["V"], cfg["D"]
    h, W, E, b, target, weight, params = make_inputs(cfg, dev)
    run = lambda: step_fn(swvr, h, W, E, b, target, weight, cfg["z"], args.chunk)

    def zero():
        for p in params:
            p.grad = None

    # warm-up and peak memory above the inputs, grad buffers included (bench/bench.py:32-38)
    torch.cuda.synchronize()
    base = torch.cuda.memory_allocated()
    torch.cuda.reset_peak_memory_stats()
    for _ in range(max(args.warmup, 1)):
        zero()
        run().backward()
    torch.cuda.synchronize()
    peak_gib = (torch.cuda.max_memory_allocated() - base) / 2**30

    # forward only
    fwd_iters = 5
    with torch.no_grad():
        run()
        s0, s1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        s0.record()
        for _ in range(fwd_iters):
            run()
        s1.record()
        torch.cuda.synchronize()
    fwd_ms = s0.elapsed_time(s1) / fwd_iters

    # timed fwd+bwd steps, every kernel launch bracketed by HIP events
    _lib.kernel_timing(True)
    _lib.kernel_timing(None)  # clear
    zero()
    torch.cuda.synchronize()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0.record()
    for _ in range(args.steps):
        zero()
        run().backward()
    t1.record()
    torch.cuda.synchronize()
    ms = t0.elapsed_time(t1) / args.steps
    kernels = _lib.kernel_timing(None)
    _lib.kernel_timing(False)

    fwd_flops, flops = algorithmic_flops(N, K, V, D)
    tflops = flops / (ms * 1e-3) / 1e12
    fp8 = (fp8_path(h, W, E, b, target, weight, cfg["z"], args.chunk, params, fwd_flops, flops, fwd_iters)
           if D <= 128 and not args.no_fp8 else None)
    # tokens with a non-zero weight: the forward leaves the others out and the
    # backward skips them (a weighted token's gO is 2 (O - t) w / (D den) != 0)
    n_act = int((weight != 0).sum().item()) if weight is not None else N
    work_tflops = tflops * n_act / N
    de_in_gemm = _lib.bwd_tiling(torch.bfloat16, N, K, V, D, args.chunk)["kernel"] == 2
    traffic, fresh = load_traffic()
    per_kernel = {}
    stream_bytes = stream_ms = 0.0
    for name, (kms, cnt) in kernels.items():
        kf = kernel_flops(name, N, K, V, D, n_act, de_in_gemm) * args.steps
        per_kernel[name] = {"ms_per_step": round(kms / args.steps, 3), "launches_per_step": cnt // args.steps,
                            "avg_launch_ms": round(kms / cnt, 4),
                            "tflops": round(kf / (kms * 1e-3) / 1e12, 1) if kf else None}
        alg = algorithmic_bytes(name, N, K, V, D, args.chunk, n_act, de_in_gemm)
        tr = measured_traffic(traffic, args.config, name) if fresh else None
        if alg is not None:
            per_kernel[name]["algorithmic_bytes_per_launch"] = int(alg)
        if tr is not None:
            # FETCH_SIZE / WRITE_SIZE count the L2's requests to the fabric: Infinity Cache (MALL)
            # hits are included, so these are L2-miss bytes, an upper bound on DRAM traffic
            per_kernel[name]["l2_miss_fetch_bytes_per_launch"] = int(tr[0])
            per_kernel[name]["l2_miss_write_bytes_per_launch"] = int(tr[1])
            per_kernel[name]["fetch_over_algorithmic"] = round(tr[0] / alg, 2) if alg else None
            stream_bytes += (tr[0] + tr[1]) * cnt
            stream_ms += kms
    dom = max(per_kernel, key=lambda k: per_kernel[k]["ms_per_step"])
    dk = per_kernel[dom]
    launch_flops = kernel_flops(dom, N, K, V, D, n_act, de_in_gemm) / dk["launches_per_step"]
    achieved = launch_flops / (dk["avg_launch_ms"] * 1e-3) / 1e12
    # W and E bytes the algorithm streams per step: fwd (W, E), bwd scores (W, E), dh GEMM (W)
    we_bytes = (3 * V * K + 2 * V * D) * 2
    dom_tr = measured_traffic(traffic, args.config, dom) if fresh else None

    out = {
        "metric": METRIC, "value": round(tflops, 1), "unit": "TFLOP/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 3),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": f"config {args.config}: fwd+bwd of softmax_readout_mse, N={N} K={K} V={V} D={D} bf16"
                               + (", bias" if cfg["bias"] else "") + (f", weight {cfg['weight']}" if cfg["weight"] else "")
                               + (f", z_loss {cfg['z']}" if cfg["z"] else ""),
                   "N": N, "K": K, "V": V, "D": D, "chunk": args.chunk},
        "active_tokens": n_act,
        # the FLOPs executed (both passes run over the active tokens only) and their share of the peak;
        # value / effective_pct_bf16_peak count the workload's 2 N V (4K + 3D) over all N tokens
        "work_tflops": round(work_tflops, 1),
        "pct_bf16_peak": round(100 * work_tflops / PEAK_BF16_TFLOPS, 1),
        "effective_pct_bf16_peak": round(100 * tflops / PEAK_BF16_TFLOPS, 1),
        "fwd_ms": round(fwd_ms, 3), "fwd_tflops": round(fwd_flops * n_act / N / (fwd_ms * 1e-3) / 1e12, 1),
        "fwd_effective_tflops": round(fwd_flops / (fwd_ms * 1e-3) / 1e12, 1),
        "peak_gib": round(peak_gib, 3),
        # fabric rate of the kernels that stream W and E: their counter-measured L2-miss bytes
        # (FETCH_SIZE + WRITE_SIZE, calibrated, profiles/readout_traffic.json; Infinity Cache hits
        # included, so an upper bound on DRAM traffic) over their own time; null when the counters
        # were taken on other sources
        "we_stream_fabric_gbps": round(stream_bytes / (stream_ms * 1e-3) / 1e9, 1) if stream_ms else None,
        "we_algorithmic_gbps": round(we_bytes / (ms * 1e-3) / 1e9, 1),
        "traffic_source": {"file": "profiles/readout_traffic.json", "source_sha": source_sha(),
                           "measured_sha": traffic.get("source_sha") if traffic else None, "fresh": fresh},
        "kernels": per_kernel,
        "roofline": {"kernel": dom, "bound": "mfma", "achieved": round(achieved, 1), "peak": PEAK_BF16_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(achieved / PEAK_BF16_TFLOPS, 4),
                     "traffic": int(dom_tr[0] + dom_tr[1]) if dom_tr else None,
                     "traffic_counts": "L2-miss bytes per launch (FETCH_SIZE + WRITE_SIZE, copy-calibrated); "
                                       "Infinity Cache hits included"},
        "fp8": fp8,
        "published_reference_ms": {"A100": {3: 240, 2: 115, 4: 160}.get(args.config),
                                   "H200": {3: 98, 2: 48, 4: 62}.get(args.config)},
    }
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline(cfg, args.cpu_tokens, args.chunk, dev)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
