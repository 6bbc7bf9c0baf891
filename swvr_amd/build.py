"""Compile the gfx950 HIP sources of swvr_amd into ``swvr_amd/libswvr_hip.so``.

    python -m swvr_amd.build          # build (always recompiles)
    python -m swvr_amd.build --remarks  # also print register / LDS usage per kernel

hipcc cross-compiles for gfx950 without a GPU, so this runs anywhere ROCm is
installed.  The library is a plain C-ABI shared object (include/swvr.h): it
links against the HIP runtime only, not against torch.
"""
import argparse
import os
import shutil
import subprocess
import sys
import tempfile
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIB_NAME = "libswvr_hip.so"
LIB_PATH = os.path.join(HERE, LIB_NAME)
SOURCES = ["fwd.hip", "bwd.hip", "loss.hip", "quant.hip", "abi.hip"]
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


def build(remarks=False, verbose=False):
    """Compile every source and link the shared library (atomically replaced)."""
    with tempfile.TemporaryDirectory(prefix="swvr_build_") as tmp:
        objs = [os.path.join(tmp, s + ".o") for s in SOURCES]
        with ThreadPoolExecutor(max_workers=min(len(SOURCES), os.cpu_count() or 1)) as ex:
            logs = list(ex.map(lambda a: _compile(a[0], a[1], remarks), zip(SOURCES, objs)))
        if remarks or verbose:
            for s, log in zip(SOURCES, logs):
                sys.stderr.write(f"---- {s}\n{log}")
        tmp_lib = os.path.join(tmp, LIB_NAME)
        r = subprocess.run([hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp_lib],
                           capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError(f"link failed:\n{r.stderr[-8000:]}")
        shutil.copyfile(tmp_lib, LIB_PATH + ".tmp")
        os.replace(LIB_PATH + ".tmp", LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--remarks", action="store_true")
    args = ap.parse_args()
    print(build(remarks=args.remarks))
