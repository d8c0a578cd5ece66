"""The C++ shim that keeps the reference's qw::gpu names (shown for
maintainers in the integration guide) compiles against include/qw/q4ops.h,
and the Python ctypes stub there declares the argument count the C-ABI has."""
import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
GUIDE = os.path.join(ROOT, "INTEGRATION.md")


def blocks(lang):
    return re.findall(r"```" + re.escape(lang) + r"\n(.*?)```", open(GUIDE).read(), flags=re.S)


@pytest.mark.skipif(shutil.which("hipcc") is None, reason="hipcc not on PATH")
def test_shim_compiles(tmp_path):
    shim = [b for b in blocks("c++") if "#pragma once" in b and "namespace qw::gpu" in b]
    assert len(shim) == 1
    src = tmp_path / "shim_check.hip"
    src.write_text(shim[0].replace("#pragma once\n", "") +
                   "\nint main() { return &qw::gpu::gemv_rows_q4 == nullptr; }\n")
    r = subprocess.run(["hipcc", "--offload-arch=gfx950", "-std=c++17", "-fsyntax-only",
                        "-I", os.path.join(ROOT, "include"), str(src)], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr[-2000:]


def test_ctypes_stub_arity_matches_header():
    stub = [b for b in blocks("python") if "argtypes" in b][0]
    n_stub = len(re.search(r"qw_q4_gemv\.argtypes = \[(.*?)\]", stub).group(1).split(","))
    header = open(os.path.join(ROOT, "include", "qw", "q4ops.h")).read()
    decl = re.search(r"int qw_q4_gemv\((.*?)\);", header, flags=re.S).group(1)
    assert n_stub == len(decl.split(","))
