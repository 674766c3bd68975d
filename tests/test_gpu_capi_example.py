"""The C ABI without Python on the device path: the C++ host program
ernie-evolve-results_amd/examples/moe_step.cpp (built next to the library by
moe_route.build) runs route -> permute -> combine on raw hipMalloc buffers
and checks the step's invariants itself (counts, offsets, bijective stable
permutation, gathered rows, identity-expert combine)."""
import os
import subprocess

import pytest

pytestmark = pytest.mark.gpu

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BIN = os.path.join(REPO, "ernie-evolve-results_amd", "moe_route", "moe_step")


@pytest.mark.parametrize("T", [1, 333, 2048])
def test_cpp_host_program_through_the_c_abi(cuda, T):
    if not os.path.exists(BIN):
        raise RuntimeError("%s is not built; run __graft_entry__.build()" % BIN)
    r = subprocess.run([BIN, str(T)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "moe_step OK" in r.stdout
