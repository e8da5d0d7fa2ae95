"""CPU checks of the audio front end: the library's WAV reader and 16 kHz resampler (mz_wav_read,
mz_resample_16k) and its feature tables (mz_mel_tables) against the reference's KATs (src/audio.rs:255-333) and the
oracle (oracle/audio_ref.py), and the oracle's features against the reference's KATs and transformers' feature
extractor (tests/golden/mel_*.npz). The features themselves run on the GPU (tests/test_gpu_audio.py)."""
import ctypes as C
import os
import struct
import sys

import numpy as np
import pytest

from mimizuku_amd import _lib as L
from oracle import audio_ref as A

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")
sys.path.insert(0, GOLDEN)
from waves import waveform  # noqa: E402


def wav(fmt, ch, sr, bits, data: bytes) -> bytes:
    """audio.rs:258-271: a 44-byte header and the data chunk."""
    b = b"RIFF\0\0\0\0WAVEfmt " + struct.pack("<IHHIIHH", 16, fmt, ch, sr, sr * ch * bits // 8, ch * bits // 8, bits)
    return b + b"data" + struct.pack("<I", len(data)) + data


def lib_read(tmp_path, data: bytes):
    p = tmp_path / f"w{len(data)}.wav"
    p.write_bytes(data)
    n, sr = C.c_size_t(), C.c_int()
    L.check(L.lib().mz_wav_read(str(p).encode(), None, 0, C.byref(n), C.byref(sr)))
    y = np.zeros(n.value, np.float32)
    L.check(L.lib().mz_wav_read(str(p).encode(), y.ctypes.data_as(C.POINTER(C.c_float)), n.value, C.byref(n),
                                C.byref(sr)))
    return y, sr.value


def lib_resample(y, sr):
    y = np.ascontiguousarray(y, np.float32)
    n = C.c_size_t()
    fp = C.POINTER(C.c_float)
    L.check(L.lib().mz_resample_16k(y.ctypes.data_as(fp), len(y), sr, None, 0, C.byref(n)))
    out = np.zeros(n.value, np.float32)
    L.check(L.lib().mz_resample_16k(y.ctypes.data_as(fp), len(y), sr, out.ctypes.data_as(fp), n.value, C.byref(n)))
    return out


def test_wav_formats(tmp_path):
    """wav_formats (audio.rs:281-291); the oracle reads the same bytes the same way."""
    pcm16 = struct.pack("<4h", 16384, -32768, 0, 8192)
    cases = [(wav(1, 2, 48000, 16, pcm16), [-0.25, 0.125], 48000),
             (wav(3, 1, 16000, 32, struct.pack("<2f", 0.5, -1.0)), [0.5, -1.0], 16000),
             (wav(1, 1, 16000, 24, bytes([0x00, 0x00, 0x40, 0x00, 0x00, 0xC0])), [0.5, -0.5], 16000),
             (wav(1, 1, 22050, 32, struct.pack("<2i", 1 << 30, -(1 << 31))), [0.5, -1.0], 22050)]
    for b, want, rate in cases:
        y, sr = lib_read(tmp_path, b)
        assert sr == rate and y.tolist() == want
        yo, sro = A.read_wav(b)
        assert sro == rate and yo.tolist() == want
    # WAVE_FORMAT_EXTENSIBLE carrying float samples, and an odd-sized chunk before the data (padded to even)
    ext = b"RIFF\0\0\0\0WAVE" + b"LIST" + struct.pack("<I", 3) + b"abc\0" + b"fmt " + struct.pack(
        "<IHHIIHH", 40, 0xFFFE, 1, 16000, 64000, 4, 32) + struct.pack("<HHI", 22, 32, 0) + struct.pack("<H", 3) + \
        bytes(14) + b"data" + struct.pack("<I", 8) + struct.pack("<2f", 0.25, 0.75)
    assert lib_read(tmp_path, ext)[0].tolist() == [0.25, 0.75] == A.read_wav(ext)[0].tolist()


def test_wav_malformed_is_an_error(tmp_path):
    """wav_malformed_is_an_error (audio.rs:293-305), including a streaming writer's unset data size."""
    bad = [b"RIFF\0\0\0\0WAVE", wav(1, 1, 16000, 8, bytes([0, 1])), wav(1, 1, 16000, 16, b"")[:30], b"not a wav file",
           wav(1, 1, 16000, 16, bytes([0, 1, 2, 3]))[:-1], wav(1, 1, 16000, 16, bytes([0, 1, 2])),
           wav(3, 1, 16000, 32, struct.pack("<f", float("inf")))]
    for b in bad:
        with pytest.raises(L.MzError):
            lib_read(tmp_path, b)
        with pytest.raises(ValueError):
            A.read_wav(b)
    streamed = bytearray(wav(1, 1, 16000, 16, bytes([0, 0x40, 0, 0x40])))
    streamed[40:44] = struct.pack("<I", 0xFFFFFFFF)
    assert lib_read(tmp_path, bytes(streamed))[0].tolist() == [0.5, 0.5] == A.read_wav(bytes(streamed))[0].tolist()


def tone(sr, hz, secs):
    return np.sin(2 * np.pi * hz * np.arange(int(sr * secs)) / sr).astype(np.float32)


def rms(y):
    m = y[len(y) // 4:3 * len(y) // 4].astype(np.float64)
    return float(np.sqrt((m ** 2).mean()))


@pytest.mark.parametrize("sr", [8000, 22050, 44100, 48000])
def test_resampler_keeps_the_band_and_removes_aliases(sr):
    """audio.rs:318-334: DC gain 1, a 1 kHz tone at full level, a 9 kHz tone gone; the oracle agrees."""
    y = lib_resample(np.ones(sr, np.float32), sr)
    assert len(y) == 16000 and abs(y[8000] - 1.0) < 1e-4
    t = tone(sr, 1000.0, 1.0)
    got = lib_resample(t, sr)
    assert abs(rms(got) - 0.5 ** 0.5) < 0.01
    np.testing.assert_allclose(got, A.to_16k(t, sr), rtol=0, atol=2e-6)
    if sr > 16000:
        assert rms(lib_resample(tone(sr, 9000.0, 1.0), sr)) < 1e-3


def test_resampler_limits():
    with pytest.raises(L.MzError):
        lib_resample(np.zeros(10, np.float32), 100)
    # 767,999 Hz: 16,000 phases of 9,460 taps, computed per sample instead of tabulated
    assert len(lib_resample(np.zeros(96, np.float32), 767999)) == 3
    y = np.arange(5, dtype=np.float32)
    assert lib_resample(y, 16000).tolist() == y.tolist()


@pytest.mark.parametrize("n_mels", [80, 128])
def test_mel_tables_match_the_oracle(n_mels):
    f = np.zeros((201, n_mels), np.float32)
    cb, sb = np.zeros((400, 201)), np.zeros((400, 201))
    d = C.POINTER(C.c_double)
    L.check(L.lib().mz_mel_tables(n_mels, f.ctypes.data_as(C.POINTER(C.c_float)), cb.ctypes.data_as(d),
                                  sb.ctypes.data_as(d)))
    fo, co, so = A.mel_tables(n_mels)
    np.testing.assert_allclose(f, fo, rtol=1e-6, atol=1e-9)
    np.testing.assert_allclose(cb, co, rtol=0, atol=1e-15)
    np.testing.assert_allclose(sb, so, rtol=0, atol=1e-15)
    # each filter is a triangle: non-negative, one peak, area-normalised (Slaney)
    assert (f >= 0).all() and (f.max(0) > 0).all()


def test_oracle_features_of_silence_and_frames():
    """features_of_silence_and_frames (audio.rs:336-348)."""
    m, frames = A.features(np.zeros(16000, np.float32), 80)
    assert m.shape == (80, 3000) and frames == 100
    assert np.all(np.abs(m - (-10.0 + 4.0) / 4.0) < 1e-6)
    m, _ = A.features(tone(16000, 1000.0, 1.0), 80)
    assert 20 <= int(np.argmax(m[:, 50])) < 40


@pytest.mark.parametrize("name", ["mel80_7s", "mel128_30s", "mel128_short"])
def test_oracle_features_match_transformers(name):
    fx = np.load(os.path.join(GOLDEN, f"{name}.npz"))
    y = waveform(int(fx["seed"]), float(fx["seconds"]))
    m, frames = A.features(y, int(fx["n_mels"]))
    assert frames == int(fx["frames"])
    assert np.abs(m[:, fx["cols"]] - fx["features"]).max() < 2e-5
    if frames < 3000:
        assert np.all(m[:, fx["cols"][-1]:] == m[0, -1]) and abs(m[0, -1] - float(fx["pad_value"])) < 2e-5
