"""The C-ABI from a plain C host (tests/c_consumer/ppk_c_consumer.c): device memory from the HIP runtime,
quantize and attention calls through include/ppk_int8_kv.h, no Python or torch in the process. The
program checks codes and scales bit for bit and attention within the north-star bar (max abs <= 2e-3,
max relative <= 1e-2) against the CPU oracle, on a ragged batch (past = 257 and 100 of capacity 300,
H = 4, D = 128) under the library's plan, 8-token splits (merge kernel) and host lengths, a refused call,
dequantize (bit-exact) and the fused decode step (output, committed codes and scales, flags)."""
import os
import subprocess

import pytest

EXE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "c_consumer", "ppk_c_consumer")


@pytest.mark.gpu
def test_plain_c_host_matches_the_oracle():
    assert os.path.exists(EXE), "tests/c_consumer/ppk_c_consumer is not built: run __graft_entry__.build()"
    res = subprocess.run([EXE], capture_output=True, text=True, timeout=100)
    print(res.stdout)
    print(res.stderr)
    assert res.returncode == 0, res.stdout + res.stderr
    assert "c consumer ok" in res.stdout
    assert "FAIL" not in res.stdout
