"""Build libmacai_gdr.so in-tree for gfx950 (hipcc; no cmake, no JIT cache): `python build.py`."""
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
SRCS = [os.path.join(HERE, "csrc", f) for f in ("gdr_kernels.hip", "gdr_forward.hip", "gdr_producers.hip", "gdr_probe.hip")]
# chunk_bwd8's translation unit, compiled on its own with LLVM's max-memory-clause scheduling strategy (faster for that
# kernel; for the whole library it slowed the reverse state pass and grew the float32 state kernels' spills)
CB8_SRC = os.path.join(HERE, "csrc", "gdr_chunk_bwd8.hip")
CB8_FLAGS = ["-mllvm", "-amdgpu-sched-strategy=max-memory-clause"]
OUT = os.path.join(HERE, "macai", "gated_delta", "libmacai_gdr.so")
ARCH = os.environ.get("MACAI_GPU_ARCH", "gfx950")


def _common():
    return ["hipcc", f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
            "-I", os.path.join(ROOT, "include"), "-I", os.path.join(HERE, "csrc"),
            # no packed fp32 VALU instructions: some of their forms have given wrong results on this hardware pool
            "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]


def cb8_command(obj):
    return _common() + CB8_FLAGS + ["-c", CB8_SRC, "-o", obj]


def command(out=OUT, cb8_obj=None):
    """The link of the library: with cb8_obj, chunk_bwd8's separately compiled object (placed first: hipcc marks every
    file after a .hip source as HIP source); without it, its source compiled like the others (no scheduler flag)."""
    return _common() + ["-shared", *([cb8_obj] if cb8_obj else []), *SRCS, *([] if cb8_obj else [CB8_SRC]), "-o", out]


def _run(cmd, verbose):
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    err = "\n".join(x for x in r.stderr.splitlines() if "packed-fp32-ops' is not a recognized feature" not in x)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed ({r.returncode}):\n{err}")
    if verbose and err.strip():
        print(err)


def build(verbose=True):
    tmp, obj = OUT + ".tmp", OUT + ".cb8.o"
    try:
        _run(cb8_command(obj), verbose)
        _run(command(tmp, obj), verbose)
    finally:
        if os.path.exists(obj):
            os.remove(obj)
    os.replace(tmp, OUT)
    return OUT


if __name__ == "__main__":
    print(build())
    sys.exit(0)
