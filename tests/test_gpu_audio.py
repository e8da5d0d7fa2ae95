"""GPU parity of the log-mel features (mz_log_mel, k_mel.hip) against the oracle's restatement of the reference's
Mel::features (oracle/audio_ref.py) and transformers' feature extractor (tests/golden/mel_*.npz)."""
import ctypes as C
import os
import sys

import numpy as np
import pytest

from mimizuku_amd import _lib as L
from mimizuku_amd import model
from oracle import audio_ref as A

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")
sys.path.insert(0, GOLDEN)
from waves import waveform  # noqa: E402

NS = 480000


@pytest.fixture(scope="module")
def ctx():
    c = model.Context(0)
    yield c
    c.close()


def log_mel(ctx, clips, n_mels, junk_tail=False):
    """Runs mz_log_mel on clips (host float32 arrays); returns features [n][n_mels][3000] and frame counts."""
    n = len(clips)
    buf = np.zeros((n, NS), np.float32)
    rng = np.random.default_rng(9)
    for i, y in enumerate(clips):
        k = min(len(y), NS)
        buf[i, :k] = y[:k]
        if junk_tail and k < NS:
            buf[i, k:] = rng.standard_normal(NS - k)  # past n_samples: must read as zero
    ns = np.array([len(y) for y in clips], np.int32)
    d_audio = ctx.upload_new(buf)
    d_mel = ctx.alloc(n * n_mels * 3000 * 4)
    frames = np.zeros(n, np.int32)
    print(f"mz_log_mel n={n} n_mels={n_mels} lengths={ns.tolist()}", flush=True)
    L.check(L.lib().mz_log_mel(ctx.h, d_audio, ns.ctypes.data_as(C.c_void_p), n, n_mels, d_mel,
                               frames.ctypes.data_as(C.c_void_p)))
    out = ctx.download(d_mel, (n, n_mels, 3000), np.float32)
    ctx.free(d_audio)
    ctx.free(d_mel)
    return out, frames


@pytest.mark.parametrize("n_mels", [80, 128])
def test_log_mel_matches_the_oracle(ctx, n_mels):
    rng = np.random.default_rng(n_mels)
    lengths = [0, 1, 159, 16000 * 7 + 123, NS, NS + 40000]
    clips = [(0.3 * rng.standard_normal(k)).astype(np.float32) for k in lengths]
    got, frames = log_mel(ctx, clips, n_mels, junk_tail=True)
    tables = A.mel_tables(n_mels)
    for i, y in enumerate(clips):
        ref, fr = A.features(y, n_mels, tables)
        assert frames[i] == fr, (i, frames[i], fr)
        err = np.abs(got[i] - ref).max()
        assert err <= 1e-6, (i, lengths[i], err)


def test_log_mel_of_silence_and_a_tone(ctx):
    """features_of_silence_and_frames (src/audio.rs:336-348) on the device."""
    t = np.sin(2 * np.pi * 1000.0 * np.arange(16000) / 16000).astype(np.float32)
    got, frames = log_mel(ctx, [np.zeros(16000, np.float32), t], 80)
    assert frames.tolist() == [100, 100]
    assert np.all(np.abs(got[0] - (-10.0 + 4.0) / 4.0) < 1e-6)
    assert 20 <= int(np.argmax(got[1][:, 50])) < 40


def test_log_mel_matches_transformers(ctx):
    for name in ("mel80_7s", "mel128_30s", "mel128_short"):
        fx = np.load(os.path.join(GOLDEN, f"{name}.npz"))
        y = waveform(int(fx["seed"]), float(fx["seconds"]))
        got, frames = log_mel(ctx, [y], int(fx["n_mels"]))
        assert frames[0] == int(fx["frames"])
        assert np.abs(got[0][:, fx["cols"]] - fx["features"]).max() < 2e-5, name
