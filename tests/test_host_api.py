"""The C++ drop-in surface (cudasep::Tensor / cudasep::ops, libcudasep_amd.so).

CPU: the library exports the reference's op names with the reference's
signatures (src/ops.h:56, :65-66, :83-85, :99-100, :128-135).
GPU: tests/cpp/test_host_ops checks every op against the CPU oracle, the
dtype rules and the error behaviour (see that file for the tolerances);
tests/cpp/test_tensor_views checks the Tensor view surface (permute, slice,
split, expand, cat, stack, broadcast operators) and runs the reference's own
per-op apply_attention / apply_feedforward / apply_transformer /
compute_rotary_cos_sin sequence and depth-loop permutes (model_bs_roformer.cu:
205-331, :482-534) on [62, 801, 512] against the oracle's transformer.
"""
from __future__ import annotations

import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HOST_LIB = os.path.join(ROOT, "cuda-msst-infer_amd", "libcudasep_amd.so")
TEST_BIN = os.path.join(ROOT, "tests", "cpp", "_build", "test_host_ops")
VIEWS_BIN = os.path.join(ROOT, "tests", "cpp", "_build", "test_tensor_views")

SIGNATURES = [
    "cudasep::ops::linear(cudasep::Tensor const&, cudasep::Tensor const&, cudasep::Tensor const&)",
    "cudasep::ops::linear_no_bias(cudasep::Tensor const&, cudasep::Tensor const&)",
    "cudasep::ops::linear_gelu(cudasep::Tensor const&, cudasep::Tensor const&, cudasep::Tensor const&)",
    "cudasep::ops::linear_silu(cudasep::Tensor const&, cudasep::Tensor const&, cudasep::Tensor const&)",
    "cudasep::ops::linear_sigmoid(cudasep::Tensor const&, cudasep::Tensor const&, cudasep::Tensor const&)",
    "cudasep::ops::rms_norm(cudasep::Tensor const&, cudasep::Tensor const&, float)",
    "cudasep::ops::apply_rotary_emb(cudasep::Tensor&, cudasep::Tensor&, cudasep::Tensor const&, cudasep::Tensor const&)",
    "cudasep::ops::scaled_dot_product_attention(cudasep::Tensor const&, cudasep::Tensor const&, cudasep::Tensor const&, float, float)",
    "cudasep::ops::stft(cudasep::Tensor const&, int, int, int, cudasep::Tensor const&, bool, bool)",
    "cudasep::ops::istft(cudasep::Tensor const&, int, int, int, cudasep::Tensor const&, long, bool, bool)",
    "cudasep::ops::hann_window(int)",
    "cudasep::ops::tanh_act(cudasep::Tensor const&)",
    "cudasep::ops::glu(cudasep::Tensor const&, int)",
    "cudasep::ops::BandPlan::band_split(cudasep::Tensor const&) const",
    "cudasep::ops::BandPlan::mask_estimator(cudasep::Tensor const&) const",
    "cudasep::ops::BandPlan::band_gather(cudasep::Tensor const&, long) const",
    "cudasep::ops::BandPlan::mask_merge(cudasep::Tensor const&, cudasep::Tensor const&, long, bool) const",
    "cudasep::clear_attention_graph_cache()",
    "cudasep::CudaContext::instance()",
    "cudasep::Tensor::empty(std::vector<long, std::allocator<long> >, cudasep::DType)",
    # the Tensor path subset the reference's Roformer code calls (tensor.h:75-105)
    "cudasep::Tensor::permute(std::vector<int, std::allocator<int> >) const",
    "cudasep::Tensor::transpose(int, int) const",
    "cudasep::Tensor::contiguous() const",
    "cudasep::Tensor::expand(std::vector<long, std::allocator<long> >) const",
    "cudasep::Tensor::slice(int, long, long) const",
    "cudasep::Tensor::split(int, std::vector<long, std::allocator<long> > const&) const",
    "cudasep::Tensor::unbind(int) const",
    "cudasep::Tensor::cat(std::vector<cudasep::Tensor, std::allocator<cudasep::Tensor> > const&, int)",
    "cudasep::Tensor::stack(std::vector<cudasep::Tensor, std::allocator<cudasep::Tensor> > const&, int)",
    "cudasep::Tensor::operator*(cudasep::Tensor const&) const",
    "cudasep::Tensor::operator+(cudasep::Tensor const&) const",
    "cudasep::Tensor::add_(cudasep::Tensor const&)",
    "cudasep::Tensor::is_contiguous() const",
]


def test_host_library_exports_reference_signatures():
    assert os.path.exists(HOST_LIB), "build libcudasep_amd.so first (make -C cuda-msst-infer_amd)"
    out = subprocess.run(["nm", "-DC", "--defined-only", HOST_LIB], check=True,
                         capture_output=True, text=True).stdout
    for sig in SIGNATURES:
        assert sig in out, sig
    for glob in ("cudasep::g_quantize_fp16", "cudasep::g_enable_cuda_graph_attention"):
        assert glob in out, glob


@pytest.mark.gpu
def test_host_ops_against_oracle(cuda):
    assert os.path.exists(TEST_BIN), "build tests/cpp first (make -C tests/cpp)"
    print("running", TEST_BIN, flush=True)
    r = subprocess.run([TEST_BIN], capture_output=True, text=True, timeout=300)
    print(r.stdout[-4000:])
    print(r.stderr[-2000:])
    assert r.returncode == 0
    assert r.stdout.rstrip().splitlines()[-1].startswith("OK:")


@pytest.mark.gpu
def test_tensor_views_and_reference_per_op_sequence(cuda):
    assert os.path.exists(VIEWS_BIN), "build tests/cpp first (make -C tests/cpp)"
    print("running", VIEWS_BIN, flush=True)
    r = subprocess.run([VIEWS_BIN], capture_output=True, text=True, timeout=600)
    print(r.stdout[-6000:])
    print(r.stderr[-2000:])
    assert r.returncode == 0
    assert r.stdout.rstrip().splitlines()[-1].startswith("OK:")
