"""Runs the C++ test executables (reference-style asserts) built by llmengine_amd.build.

test_host_cpu   graph / registry / executor / adapter validation, no GPU needed
test_hip_q8_0   the HipBackend + HipExecutor end to end on an MI355X
"""
import os
import subprocess

import pytest

BIN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "cpp", "bin")


def run(name, timeout):
    exe = os.path.join(BIN, name)
    if not os.path.exists(exe):
        pytest.fail(f"{exe} not built: run `python -m llmengine_amd.build`")
    print(f"[case] {name}", flush=True)
    p = subprocess.run([exe], stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True,
                       timeout=timeout)
    print(p.stdout)
    assert p.returncode == 0, p.stdout


def test_host_cpu_suite():
    run("test_host_cpu", 120)


@pytest.mark.gpu
def test_hip_q8_0_suite():
    run("test_hip_q8_0", 240)
