"""CPU check of the FFT arithmetic the STFT kernels run (csrc/fft_core.hpp):
tests/cpp/test_fft_core runs the Stockham passes and the real-transform
pack / unpack on the host against a float64 DFT for n = 16 .. 8192.  No GPU."""
from __future__ import annotations

import os
import subprocess

from conftest import ROOT

BIN = os.path.join(ROOT, "tests", "cpp", "_build", "test_fft_core")


def test_fft_core_on_cpu():
    subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "tests", "cpp"), "_build/test_fft_core"],
                   check=True)
    r = subprocess.run([BIN], capture_output=True, text=True, timeout=120)
    print(r.stdout[-3000:])
    assert r.returncode == 0
    assert r.stdout.rstrip().splitlines()[-1] == "OK"
