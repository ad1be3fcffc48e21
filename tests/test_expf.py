"""The restatement of glibc's expf in the device's output post-processing (expf_glibc in
katago-rs_amd/csrc/kgx_post.hip, its constants in kgx_expf.h) against the host's glibc expf, which the reference's
port reproduces (crates/katago-core/src/port/math.rs:634-680): tests/expf_check.cpp repeats the same steps with the
same constants over every 61st float bit pattern of [-110, 90] and the special inputs, bit for bit. (Every float of
that range was checked the same way once, with no mismatch; the GPU tests hold the device's results to the oracle,
which calls the host's expf, bit for bit.)"""

import os
import shutil
import subprocess
import tempfile

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))


def test_expf_restatement_matches_host_glibc():
    gxx = shutil.which("g++")
    if gxx is None:
        pytest.skip("no g++")
    with tempfile.TemporaryDirectory() as d:
        exe = os.path.join(d, "expf_check")
        subprocess.run([gxx, "-O2", "-std=c++17", "-o", exe, os.path.join(HERE, "expf_check.cpp"), "-lm"], check=True)
        out = subprocess.run([exe, "61"], capture_output=True, text=True, check=True).stdout.split()
    checked, bad = int(out[-2]), int(out[-1])
    assert checked > 30_000_000, checked
    assert bad == 0, f"{bad} of {checked} floats differ from the host's expf"
