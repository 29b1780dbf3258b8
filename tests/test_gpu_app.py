"""End to end through the msst_infer CLI (the reference's cudasep_infer file
path): synthetic BSRoformer and MelBandRoformer .csm files (random weights
under the reference's names), a stereo WAV in, float WAVs out, compared with
the oracle's model forward run through the oracle's chunked driver.

BSRoformer: dim 128, depth 1, 2 heads, 2 stems, 19 bands over a 256-point
STFT (hop 64), mask-estimator MLP of 2 linears.  MelBandRoformer: the same
trunk with 16 overlapping HTK-mel bands computed at load (or 16 precomputed
overlapping bands stored in the file), per-transformer norms, mask MLP of 3
linears.  Chunk 4096 with 2 overlaps, so a 10000-sample track takes the
chunked path (border reflect padding, batch 2, a zero-padded last chunk)
and a 3000-sample one the direct path.
Tolerances: fp32 (--fp32) 1e-4, fp16 weights (--fp16) 2e-2, normwise per stem.
"""
from __future__ import annotations

import copy
import os
import subprocess

import numpy as np
import pytest
from scipy.io import wavfile

import csm_file
from conftest import ROOT, TOL_F16, rel_err

pytestmark = pytest.mark.gpu

CLI = os.path.join(ROOT, "cuda-msst-infer_amd", "msst_infer")

CFG = {"model_type": "bs_roformer", "dim": 128, "depth": 1, "heads": 2, "dim_head": 64,
       "stereo": True, "num_stems": 2, "mask_estimator_depth": 2, "mlp_expansion_factor": 4,
       "zero_dc": True, "stft_n_fft": 256, "stft_hop_length": 64, "stft_win_length": 256,
       "freqs_per_bands": [4] * 8 + [8] * 8 + [16] * 2 + [1], "chunk_size": 4096,
       "num_overlap": 2, "sample_rate": 44100, "instruments": ["vocals", "other"]}


MBR_CFG = {"model_type": "mel_band_roformer", "dim": 128, "depth": 1, "heads": 2,
           "dim_head": 64, "stereo": True, "num_stems": 2, "num_bands": 16,
           "mask_estimator_depth": 2, "mlp_expansion_factor": 4, "zero_dc": True,
           "stft_n_fft": 256, "stft_hop_length": 64, "stft_win_length": 256,
           "chunk_size": 4096, "num_overlap": 2, "sample_rate": 44100,
           "instruments": ["vocals", "other"]}


def mbr_model(oracle, cfg, seed, unit_mask=False, precomputed=False):
    F = cfg["stft_n_fft"] // 2 + 1
    if precomputed:
        bands = csm_file.overlapping_bands(F, 2, cfg["num_bands"])
        return csm_file.mbr_checkpoint(cfg, bands[1], seed, unit_mask, precomputed=bands)
    _, counts = oracle.mel_bands(cfg["sample_rate"], cfg["stft_n_fft"], cfg["num_bands"], 2)
    return csm_file.mbr_checkpoint(cfg, counts, seed, unit_mask)


def run_cli(args):
    print("running", " ".join(args), flush=True)
    r = subprocess.run([CLI] + args, capture_output=True, text=True, timeout=300)
    print(r.stdout[-2000:], r.stderr[-2000:])
    assert r.returncode == 0, r.stderr
    return r.stdout


def separate(tmp_path, cfg, w, audio, mode, extra=()):
    model = tmp_path / "m.csm"
    csm_file.write_csm(model, cfg, w)
    inp = tmp_path / "mix.wav"
    wavfile.write(inp, cfg["sample_rate"], np.ascontiguousarray(audio.T))
    out = tmp_path / f"out_{mode}"
    run_cli(["--model", str(model), "--input", str(inp), "--output", str(out), "--stem", "-1",
             f"--{mode}", *extra])
    stems = []
    # A one-source model writes output.wav (inference_app.cpp:609-616).
    names = cfg["instruments"] if cfg["num_stems"] > 1 else ["output"]
    for name in names:
        sr, y = wavfile.read(out / f"{name}.wav")
        assert sr == cfg["sample_rate"] and y.dtype == np.float32
        stems.append(y.T if y.ndim == 2 else y[None])
    return np.stack(stems)  # [stems, ch, S]


def oracle_separate(oracle, cfg, w, audio, num_overlap=None):
    chunk = cfg["chunk_size"]
    step = chunk // (num_overlap or cfg["num_overlap"])
    model = oracle.melbandroformer_forward if "num_bands" in cfg else oracle.bsroformer_forward
    fwd = lambda b: model(cfg, w, b)
    if audio.shape[1] > chunk:
        y = oracle.process_chunked(audio, chunk, step, 2, fwd)
        return y.reshape(cfg["num_stems"], audio.shape[0], -1)
    return fwd(audio[None])[0]


@pytest.mark.parametrize("S", [10000, 3000])
@pytest.mark.parametrize("mode", ["fp32", "fp16"])
def test_cli_matches_oracle(tmp_path, oracle, cuda, S, mode):
    rng = np.random.default_rng(S)
    audio = (0.3 * rng.standard_normal((2, S))).astype(np.float32)
    w = csm_file.bsr_checkpoint(CFG, seed=2)
    y = separate(tmp_path, CFG, w, audio, mode)
    r = oracle_separate(oracle, CFG, _fp16_view(w, mode), audio)
    assert y.shape == r.shape
    tol = 1e-4 if mode == "fp32" else TOL_F16
    for s in range(y.shape[0]):
        assert rel_err(y[s], r[s]) < tol, (s, rel_err(y[s], r[s]))


def _fp16_view(w, mode):
    return {k: (v.astype(np.float16).astype(np.float32) if (mode == "fp16" and v.ndim == 2) else v)
            for k, v in w.items()}


@pytest.mark.parametrize("S", [10000, 3000])
@pytest.mark.parametrize("mode", ["fp32", "fp16"])
@pytest.mark.parametrize("bands", ["mel", "precomputed"])
def test_cli_melband_matches_oracle(tmp_path, oracle, cuda, S, mode, bands):
    rng = np.random.default_rng(S + 1)
    audio = (0.3 * rng.standard_normal((2, S))).astype(np.float32)
    w = mbr_model(oracle, MBR_CFG, seed=5, precomputed=bands == "precomputed")
    y = separate(tmp_path, MBR_CFG, w, audio, mode)
    r = oracle_separate(oracle, MBR_CFG, _fp16_view(w, mode), audio)
    assert y.shape == r.shape
    tol = 1e-4 if mode == "fp32" else TOL_F16
    for s in range(y.shape[0]):
        assert rel_err(y[s], r[s]) < tol, (s, rel_err(y[s], r[s]))


def test_cli_melband_detected_without_model_type(tmp_path, oracle, cuda):
    """No model_type: num_bands selects MelBandRoformer
    (inference_app.cpp:87)."""
    cfg = {k: v for k, v in MBR_CFG.items() if k != "model_type"}
    w = mbr_model(oracle, cfg, seed=6)
    model = tmp_path / "m.csm"
    csm_file.write_csm(model, cfg, w)
    out = run_cli(["--model", str(model), "--list-stems"])
    assert "Model type: MelBandRoformer" in out and "Model has 2 source(s)" in out


@pytest.mark.parametrize("bands", ["mel", "precomputed"])
def test_cli_melband_unit_mask_returns_the_mix(tmp_path, oracle, cuda, bands):
    """Masks of 1 + 0i on every band: the scatter-mean over overlapping
    bands is 1 on every bin, so every stem is the mix."""
    cfg = copy.deepcopy(MBR_CFG)
    cfg["zero_dc"] = False
    w = mbr_model(oracle, cfg, seed=7, unit_mask=True, precomputed=bands == "precomputed")
    audio = (0.5 * np.random.default_rng(10).standard_normal((2, 10000))).astype(np.float32)
    y = separate(tmp_path, cfg, w, audio, "fp16")
    for s in range(y.shape[0]):
        assert rel_err(y[s], audio) < 1e-5


def test_cli_overlap_override(tmp_path, oracle, cuda):
    """--overlap 4 (>= 1: the number of overlaps, inference_app.cpp:59-70)
    cuts chunks every chunk / 4 samples instead of the model's default 2."""
    rng = np.random.default_rng(11)
    audio = (0.3 * rng.standard_normal((2, 10000))).astype(np.float32)
    w = csm_file.bsr_checkpoint(CFG, seed=8)
    y = separate(tmp_path, CFG, w, audio, "fp32", ("--overlap", "4"))
    r = oracle_separate(oracle, CFG, w, audio, num_overlap=4)
    r2 = oracle_separate(oracle, CFG, w, audio)
    for s in range(y.shape[0]):
        assert rel_err(y[s], r[s]) < 1e-4, (s, rel_err(y[s], r[s]))
    assert rel_err(r[0], r2[0]) > 1e-3  # the override changes the result


def test_cli_mono_single_stem_melband(tmp_path, oracle, cuda):
    """A mono, one-stem MelBandRoformer (channel count 1 through the band
    gather / merge and the WAV path)."""
    cfg = copy.deepcopy(MBR_CFG)
    cfg.update(stereo=False, num_stems=1, instruments=["vocals"])
    _, counts = oracle.mel_bands(cfg["sample_rate"], cfg["stft_n_fft"], cfg["num_bands"], 1)
    w = csm_file.mbr_checkpoint(cfg, counts, seed=9)
    audio = (0.3 * np.random.default_rng(12).standard_normal((1, 10000))).astype(np.float32)
    y = separate(tmp_path, cfg, w, audio, "fp32")
    r = oracle_separate(oracle, cfg, w, audio)
    assert y.shape == r.shape == (1, 1, 10000)
    assert rel_err(y[0], r[0]) < 1e-4


def test_cli_unit_mask_returns_the_mix(tmp_path, cuda):
    """Masks of 1 + 0i with zero_dc off: every stem is the mix itself
    (STFT -> iSTFT, band gather / merge, chunk stitching), independent of
    the oracle."""
    cfg = copy.deepcopy(CFG)
    cfg["zero_dc"] = False
    w = csm_file.bsr_checkpoint(cfg, seed=3, unit_mask=True)
    audio = (0.5 * np.random.default_rng(9).standard_normal((2, 10000))).astype(np.float32)
    y = separate(tmp_path, cfg, w, audio, "fp16")
    for s in range(y.shape[0]):
        assert rel_err(y[s], audio) < 1e-5


def test_cli_list_stems_and_errors(tmp_path, cuda):
    model = tmp_path / "m.csm"
    csm_file.write_csm(model, CFG, csm_file.bsr_checkpoint(CFG, seed=4))
    out = run_cli(["--model", str(model), "--list-stems"])
    assert "[0] vocals" in out and "[1] other" in out and "Model type: BSRoformer" in out
    r = subprocess.run([CLI, "--model", str(tmp_path / "missing.csm"), "--input", "x.wav"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 1 and "cannot open" in r.stderr
    bad = tmp_path / "bad.csm"
    bad.write_bytes(b"XXXX" + bytes(12))
    r = subprocess.run([CLI, "--model", str(bad), "--list-stems"], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 1 and "magic" in r.stderr
    mdx = tmp_path / "mdx.csm"
    csm_file.write_csm(mdx, {"model_type": "mdx23c", "num_subbands": 4}, {})
    r = subprocess.run([CLI, "--model", str(mdx), "--list-stems"], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 1 and "MDX23C checkpoints are not supported" in r.stderr
    wav = tmp_path / "mix.wav"
    wavfile.write(wav, 44100, np.zeros((3000, 2), np.float32))
    r = subprocess.run([CLI, "--model", str(model), "--input", str(wav), "--output",
                        str(tmp_path / "o"), "--stem", "5"], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 1 and "Stem index out of range" in r.stderr
    # One chosen stem into an explicit .wav path; a rate mismatch only warns.
    wavfile.write(wav, 48000, np.zeros((3000, 2), np.float32))
    target = tmp_path / "single.wav"
    r = subprocess.run([CLI, "--model", str(model), "--input", str(wav), "--output", str(target),
                        "--stem", "1"], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0 and target.exists() and "sample rate" in r.stderr


@pytest.mark.parametrize("model", ["bsr", "mbr"])
@pytest.mark.parametrize("mode", ["fp32", "fp16"])
def test_cli_skip_connection_and_transformer_depth(tmp_path, oracle, cuda, model, mode):
    """Checkpoints with skip_connection and time/freq_transformer_depth 2
    (model_bs_roformer.cu:477-487, :531-535, the apply_transformer loop
    :319): depth 3, so the skip sums of two and three stored outputs run,
    against the oracle's restatement of that loop."""
    extra = {"depth": 3, "skip_connection": True, "time_transformer_depth": 2,
             "freq_transformer_depth": 2}
    rng = np.random.default_rng(77)
    audio = (0.3 * rng.standard_normal((2, 3000))).astype(np.float32)
    if model == "bsr":
        cfg = dict(CFG, **extra)
        w = csm_file.bsr_checkpoint(cfg, seed=8)
    else:
        cfg = dict(MBR_CFG, **extra)
        w = mbr_model(oracle, cfg, seed=9)
    print(f"skip/transformer-depth model {model} {mode}", flush=True)
    y = separate(tmp_path, cfg, w, audio, mode)
    r = oracle_separate(oracle, cfg, _fp16_view(w, mode), audio)
    assert y.shape == r.shape
    tol = 1e-4 if mode == "fp32" else TOL_F16
    for s in range(y.shape[0]):
        assert rel_err(y[s], r[s]) < tol, (s, rel_err(y[s], r[s]))
