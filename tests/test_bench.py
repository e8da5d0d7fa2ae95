"""bench.py's host side: the one-GPU refusal and the algorithmic work behind its roofline figures.

Each figure is checked against its closed form, written out as a number rather than recomputed from bench.py's
expression. The forms: a product of M x N x K costs 2 M N K FLOP; the attention costs 4 x clips x heads x 1500^2
x 64 (scores and P.V); a decoder step reads every cross key and value once (B x layers x 2 x 1500 x d fp16 values).
"""
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import bench  # noqa: E402
from mimizuku_amd import synth  # noqa: E402

TURBO = synth.LARGE_V3_TURBO


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stderr and "--gpus 1" in r.stderr
    assert r.stdout == ""


def test_encoder_work_per_launch_at_8_clips():
    w = bench.kernel_work(TURBO, 8)
    # M = 12,000 frames, d = 1280, ff = 5120
    assert w["fc1"] == ("mfma", 157_286_400_000.0)
    assert w["fc2"] == ("mfma", 157_286_400_000.0)
    assert w["qkv"] == ("mfma", 117_964_800_000.0)
    assert w["oproj"] == ("mfma", 39_321_600_000.0)
    assert w["attn"] == ("mfma", 92_160_000_000.0)
    # the conv stem's second product: K = 3 taps x 1280 channels
    assert w["conv2"] == ("mfma", 117_964_800_000.0)
    # every turbo decoder layer's cross k and v: N = 4 layers x 2 x 1280
    assert w["xkv"] == ("mfma", 314_572_800_000.0)
    # add + LayerNorm: x read and written in fp32, the delta read and the output written in fp16
    assert w["ln"] == ("hbm", 184_320_000)


def test_decoder_step_bytes_at_32_rows():
    total = bench.decode_step_bytes(TURBO, 32, 200, 6)
    cross = 983_040_000  # 32 rows x 4 layers x (k, v) x 1500 x 1280 x 2 bytes
    weights = 183_500_800  # 4 layers x (q/k/v, out, cross q, cross out: 6 d^2; fc1 + fc2: 2 d ff) x 2 bytes
    head = 132_776_960  # 51,866 x 1280 x 2 bytes
    self_kv = 131_727_360  # 32 rows x 4 layers x (k, v) x 201 positions x 1280 x 2 bytes
    logits = 6_638_848  # 32 x 51,866 x 4 bytes
    align = 576_000  # 32 rows x 6 heads x 1500 x 2 bytes
    assert total == pytest.approx(cross + weights + head + self_kv + logits + align, rel=0, abs=0.5)
    # the cross-attention launch: a quarter of the cross bytes plus its query weights, rows and alignment rows
    b = bench.dec_kernel_bytes(TURBO, 32, 200, 6)["dec_cross"]
    assert b == pytest.approx(cross / 4 + 1280 * 1280 * 2 + 2 * 32 * 1280 * 2 + 32 * 1.5 * 1500 * 6, rel=0, abs=0.5)
