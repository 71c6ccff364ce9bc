"""Build libwam_block.so from the HIP sources with hipcc, for gfx950 only.

Each source compiles to an object in parallel; one hipcc link makes the shared
library, which is renamed into place atomically.  No torch headers are used.
"""
import os
import shutil
import subprocess
import sys
import tempfile
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG.parent / "csrc"
SOURCES = ["block.hip", "gemm.hip", "norm.hip", "attention.hip", "kv_cache.hip", "dit_io.hip", "probe.hip"]
ARCH = "gfx950"
FLAGS = ["-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
         # Packed-FP32 VALU ops are disabled for all device code on this target.
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
         "-Wall", "-Wno-unused-function"]


def hipcc():
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    path = Path(rocm) / "bin" / "hipcc"
    if path.exists():
        return str(path)
    found = shutil.which("hipcc")
    if not found:
        raise RuntimeError("hipcc not found")
    return found


def _run(cmd):
    res = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in res.stderr.splitlines() if noise not in l)
    if res.returncode != 0:
        raise RuntimeError(f"command failed: {' '.join(cmd)}\n{err}")
    return err


def build(verbose=False, jobs=None):
    out = PKG / "libwam_block.so"
    cc = hipcc()
    with tempfile.TemporaryDirectory(prefix="wam_build_") as tmp:
        objs = [str(Path(tmp) / (s + ".o")) for s in SOURCES]
        cmds = [[cc, *FLAGS, "-c", str(CSRC / s), "-o", o] for s, o in zip(SOURCES, objs)]
        with ThreadPoolExecutor(jobs or min(len(cmds), os.cpu_count() or 1)) as ex:
            for msg in ex.map(_run, cmds):
                if verbose and msg.strip():
                    print(msg, file=sys.stderr)
        tmp_so = str(out) + ".tmp"
        _run([cc, "-shared", f"--offload-arch={ARCH}", "-o", tmp_so, *objs])
        os.replace(tmp_so, out)
    return out


if __name__ == "__main__":
    print(build(verbose=True))
