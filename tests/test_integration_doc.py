"""The C++ layers compile: include/vdbg.hpp on its own, and the vdb-side adapter shown in
INTEGRATION.md against vdb's own headers (skipped where the reference sources are absent)."""
import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REF = "/root/reference"


def _gxx():
    g = shutil.which("g++")
    if g is None:
        pytest.skip("g++ not available")
    return g


def test_host_header_compiles(tmp_path):
    src = tmp_path / "use.cc"
    src.write_text('#include "vdbg.hpp"\nint main() { vdbg::DenseRowFilter f(100); f.Allow(3);'
                   ' return f.allowed(3) ? 0 : 1; }\n')
    r = subprocess.run([_gxx(), "-std=c++20", "-Wall", "-Wextra", "-Werror", "-fsyntax-only",
                        "-I", os.path.join(ROOT, "include"), str(src)],
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stderr


def test_integration_adapter_compiles_against_vdb_headers(tmp_path):
    if not os.path.isdir(os.path.join(REF, "src", "index")):
        pytest.skip("the reference sources are not present here")
    doc = open(os.path.join(ROOT, "INTEGRATION.md")).read()
    m = re.search(r"<!-- adapter:begin -->\s*```cpp\n(.*?)```\s*<!-- adapter:end -->", doc, re.S)
    assert m, "adapter block not found in INTEGRATION.md"
    src = tmp_path / "gpu_index.cc"
    src.write_text(m.group(1))
    r = subprocess.run([_gxx(), "-std=c++20", "-fsyntax-only", "-I", os.path.join(REF, "include"),
                        "-I", os.path.join(REF, "src"), "-I", os.path.join(ROOT, "include"),
                        str(src)], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr


def test_integration_search_batch_compiles_against_vdb_headers(tmp_path):
    """The SearchBatch device branch, with the adapter header where vdb would keep it."""
    if not os.path.isdir(os.path.join(REF, "src", "index")):
        pytest.skip("the reference sources are not present here")
    doc = open(os.path.join(ROOT, "INTEGRATION.md")).read()
    a = re.search(r"<!-- adapter:begin -->\s*```cpp\n(.*?)```\s*<!-- adapter:end -->", doc, re.S)
    b = re.search(r"<!-- batch:begin -->\s*```cpp\n(.*?)```\s*<!-- batch:end -->", doc, re.S)
    assert a and b, "adapter or batch block not found in INTEGRATION.md"
    hdr = tmp_path / "index" / "gpu"
    hdr.mkdir(parents=True)
    (hdr / "gpu_index.h").write_text(a.group(1))
    src = tmp_path / "gpu_search_batch.cc"
    src.write_text(b.group(1))
    r = subprocess.run([_gxx(), "-std=c++20", "-Wall", "-fsyntax-only", "-I", str(tmp_path),
                        "-I", os.path.join(REF, "include"), "-I", os.path.join(REF, "src"),
                        "-I", os.path.join(ROOT, "include"), str(src)],
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stderr


def test_integration_segment_open_compiles_against_vdb_headers(tmp_path):
    """The GPU branch of Segment::Open, which keeps a segment whose index the GPU does not
    hold (VDBHNSW1, vdb's default index type) on the CPU path instead of failing its open."""
    if not os.path.isdir(os.path.join(REF, "src", "index")):
        pytest.skip("the reference sources are not present here")
    doc = open(os.path.join(ROOT, "INTEGRATION.md")).read()
    a = re.search(r"<!-- adapter:begin -->\s*```cpp\n(.*?)```\s*<!-- adapter:end -->", doc, re.S)
    o = re.search(r"<!-- open:begin -->\s*```cpp\n(.*?)```\s*<!-- open:end -->", doc, re.S)
    assert a and o, "adapter or Segment::Open block not found in INTEGRATION.md"
    assert "VDBG_NOT_SUPPORTED" in o.group(1), "NotSupported must mean no GPU copy"
    hdr = tmp_path / "index" / "gpu"
    hdr.mkdir(parents=True)
    (hdr / "gpu_index.h").write_text(a.group(1))
    src = tmp_path / "gpu_segment_open.cc"
    src.write_text(o.group(1))
    r = subprocess.run([_gxx(), "-std=c++20", "-Wall", "-fsyntax-only", "-I", str(tmp_path),
                        "-I", os.path.join(REF, "include"), "-I", os.path.join(REF, "src"),
                        "-I", os.path.join(ROOT, "include"), str(src)],
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
