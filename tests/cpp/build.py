"""Builds tests/cpp/_build/sampling_mirror, the driver of the C++ operator
mirror, against the in-tree libjf_sampler.so (build that first)."""
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
LIBDIR = os.path.join(REPO, "justfit-llm_amd", "jf_sampler")
OUT = os.path.join(HERE, "_build", "sampling_mirror")


def build(verbose=True):
    os.makedirs(os.path.dirname(OUT), exist_ok=True)
    cmd = [os.environ.get("HIPCC", "/opt/rocm/bin/hipcc"), "-O2", "-std=c++20",
           "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
           "-I" + os.path.join(REPO, "include"),
           "-I" + os.path.join(REPO, "justfit-llm_amd", "csrc"),
           os.path.join(HERE, "sampling_mirror.cpp"),
           "-L" + LIBDIR, "-ljf_sampler",
           "-Wl,-rpath,$ORIGIN/../../../justfit-llm_amd/jf_sampler",
           "-o", OUT]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    err = "\n".join(l for l in res.stderr.splitlines()
                    if "'-packed-fp32-ops' is not a recognized feature" not in l)
    if res.returncode != 0:
        sys.stderr.write(err + "\n")
        raise RuntimeError("building the C++ mirror driver failed")
    return OUT


if __name__ == "__main__":
    print(build())
