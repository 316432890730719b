"""The host-only sources (jf_host.cpp, jf_tree.cpp, jf_mask_wire.cpp) and the
CPU oracle built with AddressSanitizer and UndefinedBehaviorSanitizer by the
host compiler (no HIP code), driven by tests/cpp/sanitize_host.cpp over
seeded random and malformed inputs; the driver also checks the penalty
table's in-place device updates against fresh uploads of the host rows."""
import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(HERE)
CSRC = os.path.join(REPO, "justfit-llm_amd", "csrc")
ORACLE = os.path.join(REPO, "oracle")
OUT = os.path.join(HERE, "cpp", "_build", "sanitize_host")
SAN = ["-fsanitize=address,undefined", "-fno-sanitize-recover=all", "-fno-omit-frame-pointer"]


def _build():
    os.makedirs(os.path.dirname(OUT), exist_ok=True)
    obj = OUT + "_oracle.o"
    subprocess.run(["gcc", "-O1", "-g", "-std=gnu11", "-ffp-contract=off", *SAN, "-c",
                    os.path.join(ORACLE, "jf_oracle.c"), "-o", obj], check=True)
    subprocess.run(["g++", "-O1", "-g", "-std=c++20", *SAN,
                    "-I" + os.path.join(REPO, "include"), "-I" + CSRC, "-I" + ORACLE,
                    os.path.join(HERE, "cpp", "sanitize_host.cpp"),
                    os.path.join(CSRC, "jf_host.cpp"), os.path.join(CSRC, "jf_tree.cpp"),
                    os.path.join(CSRC, "jf_mask_wire.cpp"), obj,
                    "-pthread", "-lm", "-o", OUT], check=True)


@pytest.mark.skipif(shutil.which("g++") is None or shutil.which("gcc") is None,
                    reason="no host compiler")
def test_host_sources_and_oracle_run_clean_under_asan_ubsan():
    _build()
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=0",
               UBSAN_OPTIONS="print_stacktrace=1")
    r = subprocess.run([OUT], capture_output=True, text=True, env=env, timeout=300)
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-4000:]
    assert "sanitized host checks passed" in r.stdout
    assert "runtime error" not in r.stderr
