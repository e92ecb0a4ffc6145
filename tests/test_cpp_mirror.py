"""The C++ host mirror (include/vdx_sampler.hpp) and its port of the
reference's sampler testbed (tests/cpp/test_sampler_testbed.cpp, after
testbed/UTest.Sampler.pas:53-327).

CPU: the testbed builds against the library and, with no GPU, reports
Create's fatal error and a failing Process (exit 77).  GPU: every section
of the reference's testbed passes through the C ABI.
"""
import os
import subprocess

import pytest

from vindexllm_amd import build as B


def test_cpp_testbed_without_gpu(tmp_path):
    if not os.path.exists(B.LIB):
        pytest.skip("library not built (run __graft_entry__.build())")
    exe = B.build_cpp_testbed(str(tmp_path / "testbed"), rpath=B.LIBDIR)
    env = dict(os.environ, HIP_VISIBLE_DEVICES="-1", ROCR_VISIBLE_DEVICES="-1")
    r = subprocess.run([exe], capture_output=True, text=True, env=env, timeout=120)
    if r.returncode == 0:
        pytest.skip("a GPU is visible here: the GPU test covers this run")
    assert r.returncode == 77, r.stdout + r.stderr
    assert "[PASS] Create recorded a fatal error" in r.stdout
    assert "[PASS] Process returns a negative code" in r.stdout


@pytest.mark.gpu
def test_cpp_testbed_on_gpu():
    # the binary is built in-tree by __graft_entry__.build(); a missing one is a failure
    assert os.path.exists(B.CPP_TESTBED), "C++ testbed not built: run __graft_entry__.build()"
    r = subprocess.run([B.CPP_TESTBED], capture_output=True, text=True, timeout=120)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "0 failed" in r.stdout and "FAIL" not in r.stdout
