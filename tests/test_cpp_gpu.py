"""The C++20 host classes (include/vdbg.hpp) on the GPU: tests/cpp/gpu_index_test, whose
cases follow the reference's flat_test.cc, index_test.cc, pq_test.cc and filter_test.cc and
compare with the oracle bit for bit."""
import os
import subprocess

import pytest

pytestmark = pytest.mark.gpu

BIN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "cpp", "gpu_index_test")


def test_cpp_host_classes():
    if not os.path.exists(BIN):
        pytest.fail(f"{BIN} is not built; run __graft_entry__.build() (make -C tests/cpp)")
    print("running tests/cpp/gpu_index_test", flush=True)
    r = subprocess.run([BIN], capture_output=True, text=True, timeout=240)
    print(r.stdout)
    print(r.stderr)
    assert r.returncode == 0, r.stdout[-3000:] + r.stderr[-3000:]
