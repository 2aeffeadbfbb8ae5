"""Build libmacai_gdr.so in-tree for gfx950 (hipcc; no cmake, no JIT cache): `python build.py`."""
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
SRCS = [os.path.join(HERE, "csrc", f) for f in ("gdr_kernels.hip", "gdr_forward.hip", "gdr_producers.hip", "gdr_probe.hip")]
OUT = os.path.join(HERE, "macai", "gated_delta", "libmacai_gdr.so")
ARCH = os.environ.get("MACAI_GPU_ARCH", "gfx950")


def command(out=OUT):
    return ["hipcc", f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-shared",
            "-I", os.path.join(ROOT, "include"), "-I", os.path.join(HERE, "csrc"),
            # no packed fp32 VALU instructions: some of their forms have given wrong results on this hardware pool
            "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
            *SRCS, "-o", out]


def build(verbose=True):
    tmp = OUT + ".tmp"
    cmd = command(tmp)
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    err = "\n".join(x for x in r.stderr.splitlines() if "packed-fp32-ops' is not a recognized feature" not in x)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed ({r.returncode}):\n{err}")
    if verbose and err.strip():
        print(err)
    os.replace(tmp, OUT)
    return OUT


if __name__ == "__main__":
    print(build())
    sys.exit(0)
