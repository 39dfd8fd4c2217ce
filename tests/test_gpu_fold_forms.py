"""The Q4_0 record fold in its two forms (adaforge_amd/csrc/fold_forms.hip): the int8 matrix-core
form the decode kernels use (device.h:q4_mfma_tile, a digit image of the input and two
v_mfma_i32_16x16x64_i8 per record) and a plain fp32 FMA form (one nibble conversion and one FMA per
weight) give the same row sums on random Q4_0 records and a random input, to within 1e-5 of the
largest sum: the digit image's rounding (|x - image| <= 2^-27 max|x_b| per element).  The program
makes that check itself before it times both forms; the times are printed, not asserted."""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BIN = os.path.join(ROOT, "adaforge_amd", "fold_forms")


@pytest.mark.gpu
def test_mfma_and_fma_record_folds_agree():
    assert os.path.exists(BIN), "adaforge_amd/fold_forms is not built (make -C adaforge_amd/csrc)"
    r = subprocess.run([BIN], capture_output=True, text=True, timeout=120)
    print(r.stdout, flush=True)
    assert r.returncode == 0, r.stdout + r.stderr
    assert ": agree" in r.stdout
