"""The plain C99 client (tests/c_client/relax_client.c) on the GPU: relax,
the allocation-free entry point, ragged requests with the relative exit and an
argument error, through include/pcdevice.h alone, each checked against the
oracle inside the program (its bounds are stated there)."""
import os
import subprocess

import pytest

pytestmark = pytest.mark.gpu

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "c_client")


def test_c_client_against_oracle():
    binary = os.path.join(HERE, "relax_client")
    if not os.path.exists(binary):
        subprocess.run(["make", "-s", "-C", HERE], check=True)
    res = subprocess.run([binary], capture_output=True, text=True, timeout=100)
    print(res.stdout, res.stderr, flush=True)
    assert res.returncode == 0, res.stdout + res.stderr
    assert "c-client: OK" in res.stdout
