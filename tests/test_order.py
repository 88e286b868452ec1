"""CPU: the workgroup order of the MFMA pass kernels (poly-attention_amd/csrc/pa_order.h).

The kernels find their (batch, head) unit and block from the workgroup id with
``pa::block_map``.  ``tests/native/order_check.cpp`` includes that header as is, builds with
g++ and checks, over 3840 grid shapes (batch 1-8, heads 1-64, GQA groups 1-8, 1-64 blocks per
unit, causal and not), that the map is a bijection onto (unit, block), that a causal grid
dispatches each XCD's blocks heaviest first, that a non-causal grid keeps a unit's blocks
consecutive on one XCD, and that where the spread order applies every XCD runs the same number
of heads of every batch row and whole GQA groups.  A planted mistake (batch row and head
swapped) must fail the same checks."""

import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.fixture(scope="module")
def order_check(tmp_path_factory):
    gxx = shutil.which("g++")
    if gxx is None:
        pytest.skip("no g++")
    exe = str(tmp_path_factory.mktemp("order") / "order_check")
    subprocess.run([gxx, "-O2", "-std=c++17", "-I", os.path.join(ROOT, "poly-attention_amd", "csrc"),
                    os.path.join(ROOT, "tests", "native", "order_check.cpp"), "-o", exe],
                   check=True, capture_output=True, text=True)
    return exe


def test_block_map_bijective_heavy_first_and_spread(order_check):
    r = subprocess.run([order_check], capture_output=True, text=True)
    assert r.returncode == 0 and r.stdout.startswith("ok "), r.stdout + r.stderr


def test_block_map_check_rejects_a_planted_mistake(order_check):
    r = subprocess.run([order_check, "mutant"], capture_output=True, text=True)
    assert r.returncode != 0 and "FAIL" in r.stdout, r.stdout
