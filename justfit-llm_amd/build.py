"""Builds libjf_sampler.so (the C-ABI library) in-tree for gfx950.

Each source compiles to its own object in parallel (justfit-llm_amd/_build/),
then one link makes the shared library.

Usage: python justfit-llm_amd/build.py   (also called by __graft_entry__.build)
"""
import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
OBJ = os.path.join(HERE, "_build")
OUT = os.path.join(HERE, "jf_sampler", "libjf_sampler.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

SOURCES = ["jf_kernels.hip", "jf_draft.hip", "jf_gather.hip", "jf_noalloc.hip", "jf_penalty.hip",
           "jf_sampler.cpp", "jf_host.cpp",
           "jf_tree.cpp", "jf_mask_wire.cpp", "sampling.cpp"]
# jf_kernels.hip compiles as four objects (its JF_PART sections), in parallel.
PARTS = {"jf_kernels.hip": 4}

# -ffp-contract=off: every fp32 expression rounds as written, so the CPU
# restatement reproduces the weights bit for bit. Packed fp32 instructions are
# disabled (they have given silent wrong results on these boxes).
FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++20",
    "-fPIC",
    "-ffp-contract=off",
    "-fno-fast-math",
    "-Wall",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # Leading scalar kernel arguments arrive in SGPRs at wave launch.
    "-mllvm", "-amdgpu-kernarg-preload-count=16",
    "-I" + os.path.join(REPO, "include"),
    "-I" + CSRC,
]
NOISE = "'-packed-fp32-ops' is not a recognized feature"


BENCH_LOOP = os.path.join(os.path.dirname(OUT), "libjf_bench_loop.so")


def _run(cmd, what, verbose):
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    err = "\n".join(l for l in res.stderr.splitlines() if NOISE not in l)
    if res.returncode != 0:
        sys.stderr.write(err + "\n")
        raise RuntimeError(f"hipcc failed: {what}")
    if err.strip() and verbose:
        sys.stderr.write(err + "\n")


def build(verbose: bool = True) -> str:
    os.makedirs(OBJ, exist_ok=True)
    units = []  # (source, extra flags, object)
    for src in SOURCES:
        n = PARTS.get(src, 0)
        if n:
            units += [(src, [f"-DJF_PART={p}"], os.path.join(OBJ, f"{src}.{p}.o"))
                      for p in range(1, n + 1)]
        else:
            units.append((src, [], os.path.join(OBJ, src + ".o")))
    objs = [o for _, _, o in units]
    jobs = [([HIPCC] + FLAGS + extra + ["-c", "-o", o, os.path.join(CSRC, src)],
             f"{src} {' '.join(extra)}", verbose) for src, extra, o in units]
    workers = min(len(jobs), int(os.environ.get("MAX_JOBS", os.cpu_count() or 4)))
    with ThreadPoolExecutor(max_workers=max(1, workers)) as pool:
        for f in [pool.submit(_run, *j) for j in jobs]:
            f.result()
    tmp = OUT + ".tmp"
    _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp] + objs,
         "link libjf_sampler.so", verbose)
    os.replace(tmp, OUT)
    # bench.py's C++ timing loop, a separate library over libjf_sampler.so.
    loop_obj = os.path.join(OBJ, "jf_bench_loop.cpp.o")
    _run([HIPCC] + FLAGS + ["-c", "-o", loop_obj, os.path.join(CSRC, "jf_bench_loop.cpp")],
         "jf_bench_loop.cpp", verbose)
    tmp = BENCH_LOOP + ".tmp"
    _run([HIPCC, "-shared", "-fPIC", "-o", tmp, loop_obj, "-L" + os.path.dirname(OUT),
          "-ljf_sampler", "-Wl,-rpath,$ORIGIN"], "link libjf_bench_loop.so", verbose)
    os.replace(tmp, BENCH_LOOP)
    return OUT


if __name__ == "__main__":
    print(build())
