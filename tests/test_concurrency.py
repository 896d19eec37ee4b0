"""Operators called from many threads at once, as the reference's Taskflow
scheduler does (src/passes/sched/taskflow/taskflow.cpp:157-181, 474-513).

* CPU: the host-side paths of the operator layer (registry, views, shape
  arrays, element reads, equality, printing, per-thread error text) run from
  8 threads under ThreadSanitizer (tests/tsan/: the layer's C++ built with
  -fsanitize=thread, linked to the HIP library as built).
* GPU: device operators from 8 threads sharing one weight tensor; every
  result must equal the single-threaded one bit for bit (the kernels are
  deterministic and the library serialises launches on its stream).
"""
import os
import shutil
import subprocess
import threading

import numpy as np
import pytest

from camel_amd import tensor as T

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
TSAN_DIR = os.path.join(ROOT, "tests", "tsan")
DRIVER = os.path.join(ROOT, "_build", "tsan", "concurrency_driver")


@pytest.fixture(autouse=True)
def _release():
    yield
    T.release_all()


def test_host_paths_race_free_under_thread_sanitizer():
    if shutil.which("g++") is None or shutil.which("make") is None:
        pytest.skip("g++/make not available")
    if not os.path.exists(os.path.join(ROOT, "camel_amd", "lib", "libcamel_hip.so")):
        pytest.skip("libcamel_hip.so is not built")
    b = subprocess.run(["make", "-s", "-C", TSAN_DIR, "-j8"], capture_output=True, text=True,
                       timeout=600)
    assert b.returncode == 0, b.stdout + b.stderr
    env = dict(os.environ, TSAN_OPTIONS="halt_on_error=1 exitcode=66")
    r = subprocess.run([DRIVER, "8", "100"], capture_output=True, text=True, timeout=600, env=env)
    assert "ThreadSanitizer" not in r.stderr, r.stderr[-4000:]
    assert r.returncode == 0, r.stdout + r.stderr[-4000:]
    assert "failures=0" in r.stdout


@pytest.mark.gpu
def test_device_operators_from_many_threads():
    rng = np.random.default_rng(11)
    w = T.Tensor.from_numpy(rng.uniform(-1, 1, (96, 40)).astype(np.float32))  # shared by all
    inputs = [rng.uniform(-1, 1, (64 + 8 * i, 96)).astype(np.float32) for i in range(8)]

    def chain(x):
        h = T.call("dense_relu", T.Tensor.from_numpy(x), with_=(w,))
        return T.call("softmax", T.call("multiply", h, 2.0)).numpy()

    want = [chain(x) for x in inputs]
    errors = []

    def worker(i):
        try:
            for _ in range(10):
                got = chain(inputs[i])
                if not np.array_equal(got.view(np.uint32), want[i].view(np.uint32)):
                    errors.append(f"thread {i}: result differs")
                    return
        except Exception as e:  # noqa: BLE001 - reported below
            errors.append(f"thread {i}: {e!r}")

    threads = [threading.Thread(target=worker, args=(i,)) for i in range(8)]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=120)
    assert not any(t.is_alive() for t in threads), "a worker did not finish"
    assert not errors, errors
