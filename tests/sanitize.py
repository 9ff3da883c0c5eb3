"""Run the CPU test suite over AddressSanitizer/UndefinedBehaviorSanitizer
builds of the C oracle (oracle/pocr_oracle.c) and of the host-only library
sources (rapidocrvl_amd/csrc/quant_host.cpp, gguf.cpp).

    python tests/sanitize.py [extra pytest arguments]

Builds both (oracle/Makefile ``sanitize``, rapidocrvl_amd.build.
build_host_sanitized), then starts ``pytest -m "not gpu"`` in a child process
with libasan preloaded (ASan must come first in a Python process), leak
checking off (the interpreter's own allocations are not freed at exit) and
POCR_ORACLE_LIB / POCR_HOST_LIB naming the sanitized libraries.  A memory
error or undefined behaviour in those sources aborts the run with the
sanitizer's report.

A second pass runs the oracle's worker-pool driver (tests/test_oracle_pool.py)
over a ThreadSanitizer build of the oracle (oracle/Makefile ``tsan``), so a
data race in the pool fails the run.  The exit status is the first failing
pass's, else 0.
"""
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)


def main(argv):
    from rapidocrvl_amd import build

    subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "oracle"), "sanitize"], check=True)
    host = build.build_host_sanitized()
    oracle_lib = os.path.join(ROOT, "oracle", "_build", "san", "libpocr_oracle.so")
    asan = subprocess.run(["gcc", "-print-file-name=libasan.so"], capture_output=True, text=True,
                          check=True).stdout.strip()
    env = dict(os.environ)
    env.update({
        "LD_PRELOAD": asan,
        "ASAN_OPTIONS": "detect_leaks=0:abort_on_error=1:halt_on_error=1",
        "UBSAN_OPTIONS": "print_stacktrace=1:halt_on_error=1",
        "POCR_ORACLE_LIB": oracle_lib,
        "POCR_HOST_LIB": host,
    })
    cmd = [sys.executable, "-m", "pytest", os.path.join(ROOT, "tests"), "-q", "-m", "not gpu", "-p", "no:cacheprovider",
           *argv]
    rc = subprocess.run(cmd, env=env, cwd=ROOT).returncode
    if rc != 0:
        return rc

    subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "oracle"), "tsan"], check=True)
    tsan = subprocess.run(["gcc", "-print-file-name=libtsan.so"], capture_output=True, text=True,
                          check=True).stdout.strip()
    env = dict(os.environ)
    env.update({
        "LD_PRELOAD": tsan,
        "TSAN_OPTIONS": "halt_on_error=1:report_signal_unsafe=0",
        "POCR_ORACLE_LIB": os.path.join(ROOT, "oracle", "_build", "tsan", "libpocr_oracle.so"),
    })
    # The pool driver runs directly (no pytest): under TSan, forking a process
    # whose pool threads exist deadlocks inside the sanitizer runtime.
    driver = os.path.join(ROOT, "tests", "test_oracle_pool.py")
    for mode, threads, iters in (("restart", 2, 300), ("restart", 8, 100), ("concurrent", 4, 100)):
        r = subprocess.run([sys.executable, driver, mode, str(threads), str(iters)], env=env, cwd=ROOT,
                           timeout=600)
        print(f"tsan pool {mode} threads={threads} iters={iters}: rc={r.returncode}", flush=True)
        if r.returncode != 0:
            return r.returncode
    return 0


if __name__ == "__main__":
    sys.exit(main(sys.argv[1:]))
