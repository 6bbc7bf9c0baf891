"""Compile the gfx950 HIP sources of swvr_amd into ``swvr_amd/libswvr_hip.so``.

    python -m swvr_amd.build          # build (always recompiles)
    python -m swvr_amd.build --remarks  # also print register / LDS usage per kernel

hipcc cross-compiles for gfx950 without a GPU, so this runs anywhere ROCm is
installed.  The library is a plain C-ABI shared object (include/swvr.h): it
links against the HIP runtime only, not against torch.
"""
import argparse
import os
import re
import shutil
import subprocess
import sys
import tempfile
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIB_NAME = "libswvr_hip.so"
LIB_PATH = os.path.join(HERE, LIB_NAME)
SOURCES = ["fwd.hip", "bwd.hip", "loss.hip", "quant.hip", "f64.hip", "probe.hip", "abi.hip"]
ARCH = "gfx950"

# Packed-fp32 VALU forms are kept out of the code objects; the host pass warns
# that it does not know the feature, which is harmless.
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-result",
]


def hipcc():
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found: install ROCm or set HIPCC")


def _compile(src, obj, remarks):
    cmd = [hipcc(), *HIPCC_FLAGS, "-c", os.path.join(CSRC, src), "-o", obj]
    if remarks:
        cmd.append("-Rpass-analysis=kernel-resource-usage")
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n{r.stderr[-8000:]}")
    return r.stderr


_FIELDS = {"VGPRs": "vgprs", "AGPRs": "agprs", "ScratchSize [bytes/lane]": "scratch",
           "Occupancy [waves/SIMD]": "occupancy", "VGPRs Spill": "vgpr_spill", "SGPRs Spill": "sgpr_spill",
           "LDS Size [bytes/block]": "lds"}


def resource_usage(remarks):
    """Per-kernel register, scratch and LDS figures from hipcc's
    -Rpass-analysis=kernel-resource-usage remarks: {mangled name: {field: int}}."""
    out, cur = {}, None
    for line in remarks.splitlines():
        m = re.search(r"remark: Function Name: (\S+)", line)
        if m:
            cur = out.setdefault(m.group(1), {})
            continue
        m = re.search(r"remark:\s+([A-Za-z][^:]*?(?: \[[^\]]*\])?): (\d+)", line)
        if m and cur is not None and m.group(1) in _FIELDS:
            cur[_FIELDS[m.group(1)]] = int(m.group(2))
    return out


_TYPES = {"DF16b": "bf16", "DF16_": "f16", "f": "float"}


def kernel_label(mangled):
    """Short readable name of a kernel instantiation, e.g. ``fwd_tile_kernel<bf16,64,0>``
    (template arguments of the Itanium-mangled name: types and integer literals)."""
    m = re.match(r"_ZN4swvr(?:12_GLOBAL__N_1)?(\d+)", mangled)
    if not m:
        return mangled
    n = int(m.group(1))
    start = m.end()
    name = mangled[start:start + n]
    rest = mangled[start + n:]
    if not rest.startswith("I"):
        return name
    args = []
    for tok in re.finditer(r"DF16b|DF16_|L[a-z](\d+)E|(?<![A-Za-z])f", rest[1:rest.find("EE") + 1]):
        t = tok.group(0)
        args.append(tok.group(1) if t.startswith("L") else _TYPES[t])
    return f"{name}<{','.join(args)}>"


def resource_report():
    """Compile every source with resource remarks into a scratch directory (the built library is
    left as it is) and return {kernel label: resource usage}."""
    with tempfile.TemporaryDirectory(prefix="swvr_remarks_") as tmp:
        objs = [os.path.join(tmp, s + ".o") for s in SOURCES]
        with ThreadPoolExecutor(max_workers=min(len(SOURCES), os.cpu_count() or 1)) as ex:
            logs = list(ex.map(lambda a: _compile(a[0], a[1], True), zip(SOURCES, objs)))
    usage = {}
    for log in logs:
        usage.update({kernel_label(k): v for k, v in resource_usage(log).items()})
    return usage


def build(remarks=False, verbose=False):
    """Compile every source and link the shared library (atomically replaced).
    With remarks=True returns (path, {kernel: resource usage}) instead of the path."""
    with tempfile.TemporaryDirectory(prefix="swvr_build_") as tmp:
        objs = [os.path.join(tmp, s + ".o") for s in SOURCES]
        with ThreadPoolExecutor(max_workers=min(len(SOURCES), os.cpu_count() or 1)) as ex:
            logs = list(ex.map(lambda a: _compile(a[0], a[1], remarks), zip(SOURCES, objs)))
        if verbose:
            for s, log in zip(SOURCES, logs):
                sys.stderr.write(f"---- {s}\n{log}")
        tmp_lib = os.path.join(tmp, LIB_NAME)
        r = subprocess.run([hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp_lib],
                           capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError(f"link failed:\n{r.stderr[-8000:]}")
        shutil.copyfile(tmp_lib, LIB_PATH + ".tmp")
        os.replace(LIB_PATH + ".tmp", LIB_PATH)
    if remarks:
        usage = {}
        for log in logs:
            usage.update(resource_usage(log))
        return LIB_PATH, usage
    return LIB_PATH


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--remarks", action="store_true", help="print registers, scratch and LDS per kernel")
    args = ap.parse_args()
    if args.remarks:
        path, usage = build(remarks=True)
        print(f"{'kernel':72s} {'vgpr':>5s} {'agpr':>5s} {'spill':>5s} {'scratch':>7s} {'occ':>3s} {'lds':>7s}")
        for k in sorted(usage, key=kernel_label):
            u = usage[k]
            print(f"{kernel_label(k)[:72]:72s} {u.get('vgprs', 0):5d} {u.get('agprs', 0):5d} "
                  f"{u.get('vgpr_spill', 0):5d} {u.get('scratch', 0):7d} {u.get('occupancy', 0):3d} {u.get('lds', 0):7d}")
        print(path)
    else:
        print(build())
