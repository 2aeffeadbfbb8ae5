"""Build libmacai_gdr.so in-tree for gfx950 (hipcc; no cmake, no JIT cache): `python build.py`.

Each source compiles to an object of its own, side by side (gdr_kernels.hip once per part of its C ABI, -DGDR_PART=n:
the parts instantiate disjoint sets of kernels), then one link makes the library."""
import os
import subprocess
import sys
import tempfile
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
KERNELS = os.path.join(CSRC, "gdr_kernels.hip")
KERNEL_PARTS = 5                  # GDR_PART values of gdr_kernels.hip's C ABI section
OTHERS = [os.path.join(CSRC, f) for f in ("gdr_forward.hip", "gdr_producers.hip", "gdr_probe.hip")]
SRCS = [KERNELS] + OTHERS         # the sources the library is built from (besides chunk_bwd8's unit below)
# chunk_bwd8's translation unit, compiled on its own with LLVM's max-memory-clause machine-scheduling strategy (faster
# for that kernel; for the whole library it slowed the reverse state pass and grew the float32 state kernels' spills)
CB8_SRC = os.path.join(CSRC, "gdr_chunk_bwd8.hip")
CB8_FLAGS = ["-mllvm", "-amdgpu-sched-strategy=max-memory-clause"]
OUT = os.path.join(HERE, "macai", "gated_delta", "libmacai_gdr.so")
ARCH = os.environ.get("MACAI_GPU_ARCH", "gfx950")


def _common():
    return ["hipcc", f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
            "-I", os.path.join(ROOT, "include"), "-I", CSRC,
            # no packed fp32 VALU instructions: some of their forms have given wrong results on this hardware pool
            "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]


def compile_commands(objdir):
    """[(object, hipcc command)] of every object the library links."""
    out = [(os.path.join(objdir, "cb8.o"), _common() + CB8_FLAGS + ["-c", CB8_SRC])]
    for n in range(1, KERNEL_PARTS + 1):
        out.append((os.path.join(objdir, f"kernels{n}.o"), _common() + [f"-DGDR_PART={n}", "-c", KERNELS]))
    for src in OTHERS:
        out.append((os.path.join(objdir, os.path.basename(src) + ".o"), _common() + ["-c", src]))
    return [(o, cmd + ["-o", o]) for o, cmd in out]


def link_command(objs, out=OUT):
    return _common() + ["-shared", *objs, "-o", out]


def _run(cmd, verbose):
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    err = "\n".join(x for x in r.stderr.splitlines() if "packed-fp32-ops' is not a recognized feature" not in x)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed ({r.returncode}):\n{err}")
    if verbose and err.strip():
        print(err)


def build(verbose=True, jobs=None):
    tmp = OUT + ".tmp"
    with tempfile.TemporaryDirectory(prefix="macai_build_") as objdir:
        cmds = compile_commands(objdir)
        with ThreadPoolExecutor(max_workers=jobs or min(len(cmds), os.cpu_count() or 1, 16)) as pool:
            for f in [pool.submit(_run, cmd, verbose) for _, cmd in cmds]:
                f.result()
        _run(link_command([o for o, _ in cmds], tmp), verbose)
    os.replace(tmp, OUT)
    return OUT


if __name__ == "__main__":
    print(build())
    sys.exit(0)
