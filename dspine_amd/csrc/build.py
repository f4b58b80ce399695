"""Build libdspine_verify.so (all HIP sources of this directory) for gfx950 with hipcc."""

import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
OUT = os.path.join(os.path.dirname(HERE), "libdspine_verify.so")
SOURCES = ["dsv_misc.hip", "dsv_verify.hip", "dsv_chain.hip", "dsv_plan.hip", "dsv_commit.hip",
           "dsv_table.hip", "dsv_factor.hip"]
FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-shared",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-munsafe-fp-atomics", "-Wall", "-Wno-unused-function",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found: the HIP library cannot be built")


def build(verbose: bool = False, jobs: int | None = None) -> str:
    """Compile every source to an object, ``jobs`` at a time (default: the CPUs this process may
    use, at most 8), then link the shared library in-tree."""
    from concurrent.futures import ThreadPoolExecutor

    cc = hipcc()
    inc = ["-I", os.path.join(ROOT, "include"), "-I", HERE]
    objdir = os.path.join(HERE, "_build")
    os.makedirs(objdir, exist_ok=True)
    compile_flags = [f for f in FLAGS if f != "-shared"]
    objs = [os.path.join(objdir, src.replace(".hip", ".o")) for src in SOURCES]
    cmds = [[cc, *compile_flags, *inc, "-c", os.path.join(HERE, src), "-o", obj] for src, obj in zip(SOURCES, objs)]
    jobs = jobs or min(8, len(os.sched_getaffinity(0)))
    if verbose:
        for cmd in cmds:
            print(" ".join(cmd), flush=True)
    with ThreadPoolExecutor(max_workers=jobs) as pool:
        results = list(pool.map(lambda cmd: subprocess.run(cmd).returncode, cmds))
    for cmd, rc in zip(cmds, results):
        if rc != 0:
            raise subprocess.CalledProcessError(rc, cmd)
    link = [cc, "--offload-arch=gfx950", "-shared", "-fPIC", *objs, "-o", OUT + ".tmp"]
    if verbose:
        print(" ".join(link), flush=True)
    subprocess.run(link, check=True)
    os.replace(OUT + ".tmp", OUT)
    return OUT


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
