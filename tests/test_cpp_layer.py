"""Runs the C++ test driver of the reference-shaped layer interface
(tests/cpp/test_layer.cpp): construction by tensor name through the model.bin
loader, init_gpu / forward_gpu / forward / route_tokens against the oracle."""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BIN = os.path.join(ROOT, "tests", "cpp", "test_layer")


def run(mode, cwd):
    p = subprocess.run([BIN, mode], cwd=cwd, capture_output=True, text=True, timeout=300)
    print(p.stdout)
    print(p.stderr)
    assert p.returncode == 0, p.stderr
    assert " 0 failed" in p.stdout


def test_cpp_layer_cpu(tmp_path):
    subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "tests", "cpp")], check=True)
    run("cpu", tmp_path)


@pytest.mark.gpu
def test_cpp_layer_gpu(tmp_path):
    assert os.path.exists(BIN), "tests/cpp/test_layer is built by __graft_entry__.build()"
    run("gpu", tmp_path)
