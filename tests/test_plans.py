"""CPU checks of the GEMV launch planning (infer_amd/csrc/iq_plan.h),
compiled with g++ and run here: split-K partial sums always fit the
workspace a launch is given (the static no-allocation scratch's 16 MiB and
a per-stream workspace's 64 MiB), and the K ranges cover every group."""
import os
import subprocess
import tempfile

HERE = os.path.dirname(os.path.abspath(__file__))


def test_gemvq_plans_fit_the_workspace():
    with tempfile.TemporaryDirectory() as d:
        exe = os.path.join(d, "test_plans")
        subprocess.run(["g++", "-std=c++17", "-O1", "-Wall", "-o", exe, os.path.join(HERE, "cpp", "test_plans.cpp")],
                       check=True)
        r = subprocess.run([exe], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "0 failures" in r.stdout
