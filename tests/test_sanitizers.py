"""Host AddressSanitizer + UndefinedBehaviorSanitizer runs (CPU only).

`make sanitize` builds, with gcc / g++ and -fsanitize=address,undefined (no
device code is compiled with a sanitizer):
  - oracle/_build/san/libmsst_oracle.so, the CPU oracle;
  - cuda-msst-infer_amd/_build/san/libcudasep_amd.so, the C++ cudasep surface
    (host/), linked against the normal libmsst_hip.so;
  - tests/cpp/_build/san/: test_oracle_san (every oracle function at small
    ragged sizes with closed-form checks), test_fft_core and
    test_strided_index (the CPU-side FFT and index arithmetic shared with the
    kernels), test_mel_bands (the model loader's band construction through
    the sanitized libcudasep_amd.so).
Each binary must exit 0 with the sanitizers set to abort on the first
finding.  Leak detection is off for the binary that loads the HIP runtime
(its one-time initialisation allocations are not ours).
"""
from __future__ import annotations

import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HIP_LIB = os.path.join(ROOT, "cuda-msst-infer_amd", "libmsst_hip.so")
SAN_DIR = os.path.join(ROOT, "tests", "cpp", "_build", "san")

ENV = dict(os.environ,
           ASAN_OPTIONS="halt_on_error=1:abort_on_error=0:detect_leaks=1",
           UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1")


def _make(subdir: str) -> None:
    r = subprocess.run(["make", "-j8", "-C", os.path.join(ROOT, subdir), "sanitize"],
                       capture_output=True, text=True, timeout=900)
    assert r.returncode == 0, f"make sanitize in {subdir} failed:\n{r.stdout[-2000:]}\n{r.stderr[-4000:]}"


@pytest.fixture(scope="module")
def san_build():
    if shutil.which("gcc") is None or shutil.which("g++") is None:
        pytest.skip("gcc / g++ not available")
    if not os.path.exists(HIP_LIB):
        pytest.skip("libmsst_hip.so not built (run __graft_entry__.build() first)")
    for d in ("oracle", "cuda-msst-infer_amd", os.path.join("tests", "cpp")):
        _make(d)
    return SAN_DIR


@pytest.mark.parametrize("binary,leaks", [("test_oracle_san", True), ("test_fft_core", True),
                                          ("test_strided_index", True),
                                          ("test_mel_bands", False)])
def test_sanitized_binary(san_build, binary, leaks):
    env = dict(ENV)
    if not leaks:
        env["ASAN_OPTIONS"] = env["ASAN_OPTIONS"].replace("detect_leaks=1", "detect_leaks=0")
    r = subprocess.run([os.path.join(san_build, binary)], capture_output=True, text=True,
                       timeout=600, env=env, cwd=san_build)
    out = r.stdout + r.stderr
    assert r.returncode == 0, f"{binary} exited {r.returncode}:\n{out[-4000:]}"
    assert "ERROR: AddressSanitizer" not in out and "runtime error:" not in out, out[-4000:]
