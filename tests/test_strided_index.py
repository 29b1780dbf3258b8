"""CPU check of the index arithmetic the strided-view kernels run
(csrc/strided_index.hpp): tests/cpp/test_strided_index checks the
multiply-high division against hardware division and replays the kernels'
merged-axis walk against a plain multi-axis walk over random permuted,
sliced and broadcast views.  No GPU."""
from __future__ import annotations

import os
import subprocess

from conftest import ROOT

BIN = os.path.join(ROOT, "tests", "cpp", "_build", "test_strided_index")


def test_strided_index_on_cpu():
    subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "tests", "cpp"),
                    "_build/test_strided_index"], check=True)
    r = subprocess.run([BIN], capture_output=True, text=True, timeout=300)
    print(r.stdout[-3000:])
    assert r.returncode == 0
    assert r.stdout.rstrip().splitlines()[-1] == "OK"
