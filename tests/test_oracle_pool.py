"""The oracle's worker pool (a restatement of parallelForMax,
internal/tensor/ops.go:570-614) must never lose a job: every job posted right
after a resize, and every job posted while another thread is mid-call, has to
complete. These tests restart the pool thousands of times and post one
parallel matvec after each restart, then drive it from several Python threads
at once (ctypes releases the GIL, so the calls really overlap).

Each case runs this file as a child process under a time limit, so a lost
wake-up shows as a failed test rather than a hung suite:

    python tests/test_oracle_pool.py restart|concurrent THREADS ITERS
"""
import os
import subprocess
import sys
import threading

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def drive(mode: str, threads: int, iters: int) -> None:
    if ROOT not in sys.path:
        sys.path.insert(0, ROOT)
    import oracle

    rng = np.random.default_rng(7)
    # 512 rows x 256 cols: rows >= 512 and rows*cols >= 2^17 takes the
    # parallel branch of shouldParallelQuantMatVec (quant.go:563-599)
    w = rng.standard_normal((512, 256)).astype(np.float32)
    sc, data = oracle.quantize_matrix(oracle.Q8, w)
    x = rng.standard_normal(256).astype(np.float32)
    oracle.set_threads(1)
    want = oracle.matvec(oracle.Q8, sc, data, x)
    if mode == "restart":
        for i in range(iters):
            oracle.set_threads(threads)
            got = oracle.matvec(oracle.Q8, sc, data, x)
            assert np.array_equal(got, want), i
    elif mode == "concurrent":
        oracle.set_threads(threads)
        errs = []

        def run():
            try:
                for _ in range(iters):
                    if not np.array_equal(oracle.matvec(oracle.Q8, sc, data, x), want):
                        errs.append("mismatch")
            except Exception as e:  # reported below
                errs.append(repr(e))

        ts = [threading.Thread(target=run) for _ in range(4)]
        for t in ts:
            t.start()
        for t in ts:
            t.join()
        assert not errs, errs[:3]
    else:
        raise ValueError(mode)
    oracle.set_threads(1)


def _run(mode, threads, iters, limit):
    r = subprocess.run([sys.executable, os.path.abspath(__file__), mode, str(threads), str(iters)],
                       capture_output=True, text=True, timeout=limit)
    assert r.returncode == 0 and r.stdout.strip().endswith("ok"), (r.returncode, r.stdout[-500:], r.stderr[-2000:])


@pytest.mark.parametrize("threads", [2, 4, 8, 16])
def test_pool_restart_then_job(threads):
    # 2,500 restarts per thread count, 10,000 in all; a pool whose worker read
    # its starting generation only once scheduled stalled after 250-1,500
    # restarts at 2 threads
    _run("restart", threads, 2500, limit=120)


@pytest.mark.parametrize("threads", [2, 8])
def test_pool_concurrent_callers(threads):
    _run("concurrent", threads, 300, limit=120)


def test_pool_results_independent_of_threads(orc):
    rng = np.random.default_rng(3)
    w = rng.standard_normal((1024, 512)).astype(np.float32)
    for qt in (orc.Q8, orc.Q4, orc.Q6):
        sc, data = orc.quantize_matrix(qt, w)
        x = rng.standard_normal(512).astype(np.float32)
        outs = []
        for t in (1, 3, 16):
            orc.set_threads(t)
            outs.append(orc.matvec(qt, sc, data, x))
            outs.append(orc.matvec(qt, sc, data, x, vnni=True))
        assert np.array_equal(outs[0], outs[2]) and np.array_equal(outs[0], outs[4])
        assert np.array_equal(outs[1], outs[3]) and np.array_equal(outs[1], outs[5])
    from tests.conftest import ORACLE_THREADS

    orc.set_threads(ORACLE_THREADS)


if __name__ == "__main__":
    drive(sys.argv[1], int(sys.argv[2]), int(sys.argv[3]))
    print("ok", flush=True)
