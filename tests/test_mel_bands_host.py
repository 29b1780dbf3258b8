"""CPU check of the MelBandRoformer band construction in the C++ model
loader (host/roformer_models.cpp, host/ops.cpp): tests/cpp/test_mel_bands
compares ops::mel_filterbank_host with the oracle's filterbank bit for bit
and compute_mel_bands with bands derived from it.  No GPU."""
from __future__ import annotations

import os
import subprocess

from conftest import ROOT

BIN = os.path.join(ROOT, "tests", "cpp", "_build", "test_mel_bands")


def test_mel_bands_on_cpu(oracle):
    subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "tests", "cpp"), "_build/test_mel_bands"],
                   check=True)
    r = subprocess.run([BIN], capture_output=True, text=True, timeout=120)
    print(r.stdout[-3000:], r.stderr[-2000:])
    assert r.returncode == 0
    assert r.stdout.rstrip().splitlines()[-1] == "OK"
