"""CPU oracle for the audio front end — TEST INFRASTRUCTURE ONLY.

Only tests/ may import this module, and only to check results. Nothing in the mimizuku_amd package imports it.

A numpy restatement of the reference's features (src/audio.rs): WAV reading (read_wav, :14-75), resampling to
16 kHz (to_16k, :77-145), the mel filters and windowed DFT basis (Mel::new, :146-193) and the log-mel features
(Mel::features, :195-249). `features` keeps the reference's order of operations where it fixes the result bits:
each bin's real and imaginary parts are accumulated in float64 one sample at a time (vectorised over frames and
bins, never over samples), the power is rounded to float32, and each mel value is a float32 sum over bins in bin
order; only log10 is numpy's.

How it is pinned (tests/test_audio.py):
  * read_wav, to_16k: the reference's KATs (src/audio.rs:255-316: formats, malformed files, DC gain, pass-band
    level, stop-band leakage, rate limits);
  * mel_tables, features: the reference's KATs (:318-333: silence, the 1 kHz tone's band, audio frame counts), and
    transformers' WhisperFeatureExtractor (tests/golden/make_mel_golden.py, mel_*.npz), an independent
    implementation (its own STFT and Slaney filters), to 2e-4.
"""
from __future__ import annotations

import math
import struct

import numpy as np

SR = 16000
N_SAMPLES = 30 * SR
N_FRAMES = 3000
N_FFT = 400
HOP = 160
N_BINS = N_FFT // 2 + 1


def read_wav(data: bytes):
    """(mono float32 samples, sample rate) of a RIFF/WAVE byte string; ValueError when malformed (audio.rs:14-75)."""
    b = data
    if len(b) < 12 or b[0:4] != b"RIFF" or b[8:12] != b"WAVE":
        raise ValueError("not a RIFF/WAVE file")
    fmt = ch = sr = bits = 0
    i = 12
    while i + 8 <= len(b):
        cid = b[i:i + 4]
        n = struct.unpack_from("<I", b, i + 4)[0]
        body = i + 8
        if body + n > len(b) and cid != b"data":
            raise ValueError("truncated chunk")
        if cid == b"fmt ":
            fmt0 = struct.unpack_from("<H", b, body)[0] if body + 2 <= len(b) else 0
            if n < 16 or (fmt0 == 0xFFFE and n < 26):
                raise ValueError("short fmt chunk")
            fmt, ch, sr, _, _, bits = struct.unpack_from("<HHIIHH", b, body)
            if fmt == 0xFFFE:
                fmt = struct.unpack_from("<H", b, body + 24)[0]
        elif cid == b"data":
            if ch == 0 or bits == 0:
                raise ValueError("data before fmt")
            if (fmt, bits) not in ((1, 16), (1, 24), (1, 32), (3, 32)):
                raise ValueError("unsupported WAV format")
            frame = ch * bits // 8
            streamed = n == 0xFFFFFFFF
            if not streamed and (body + n > len(b) or n % frame):
                raise ValueError("data chunk is truncated or not whole frames")
            d = b[body:] if streamed else b[body:body + n]
            nf = len(d) // frame
            d = d[:nf * frame]
            if (fmt, bits) == (1, 16):
                s = np.frombuffer(d, "<i2").astype(np.float32) / np.float32(32768.0)
            elif (fmt, bits) == (1, 24):
                u = np.frombuffer(d, np.uint8).reshape(-1, 3).astype(np.int32)
                v = ((u[:, 0] << 8) | (u[:, 1] << 16) | (u[:, 2] << 24)) >> 8
                s = v.astype(np.float32) / np.float32(8388608.0)
            elif (fmt, bits) == (1, 32):
                s = np.frombuffer(d, "<i4").astype(np.float32) / np.float32(2147483648.0)
            else:
                s = np.frombuffer(d, "<f4").astype(np.float32)
            s = s.reshape(nf, ch)
            acc = np.zeros(nf, np.float32)
            for c in range(ch):  # channels summed in order, then averaged
                acc = (acc + s[:, c]).astype(np.float32)
            y = (acc / np.float32(ch)).astype(np.float32)
            if not np.isfinite(y).all():
                raise ValueError("samples that are not finite numbers")
            return y, sr
        i = body + n + (n & 1)
    raise ValueError("no data chunk")


def _bessel_i0(x: float) -> float:
    s = t = k = 1.0
    while t > 1e-12 * s:
        t *= (x / (2.0 * k)) ** 2
        s += t
        k += 1.0
    return s


def to_16k(y: np.ndarray, sr: int) -> np.ndarray:
    """Kaiser-windowed sinc resampling to 16 kHz (audio.rs:97-145), float64 arithmetic."""
    y = np.asarray(y, np.float32)
    if sr == SR:
        return y.copy()
    if not 1000 <= sr <= 768000:
        raise ValueError(f"unsupported sample rate {sr}")
    g = math.gcd(sr, SR)
    up, down = SR // g, sr // g
    scale = min(SR / sr, 1.0)
    fc = 0.95 * scale / 2.0
    half = math.ceil(32.0 / scale)
    beta = 9.0
    i0b = _bessel_i0(beta)
    i0v = np.vectorize(_bessel_i0)

    def taps(ph: int) -> np.ndarray:
        t = np.arange(-half, half + 2, dtype=np.float64) - ph / up
        with np.errstate(divide="ignore", invalid="ignore"):
            sinc = np.where(t == 0.0, 2.0 * fc, np.sin(2.0 * math.pi * fc * t) / (math.pi * t))
        r = t / half
        w = np.where(np.abs(r) > 1.0, 0.0, sinc * i0v(beta * np.sqrt(np.maximum(1.0 - r * r, 0.0))) / i0b)
        return w / w.sum()

    n_out = -(-len(y) * up // down)
    k = np.arange(n_out)
    pos = k * down
    c, ph = pos // up, pos % up
    out = np.zeros(n_out, np.float64)
    yp = np.concatenate([np.zeros(half + 2), y.astype(np.float64), np.zeros(half + 2)])
    for p in np.unique(ph):
        sel = ph == p
        w = taps(int(p))
        idx = c[sel][:, None] + np.arange(len(w))[None, :] - half + (half + 2)
        out[sel] = (yp[idx] * w[None, :]).sum(1)
    return out.astype(np.float32)


def _hz_to_mel(f):
    logstep = 27.0 / math.log(6.4)
    return np.where(f >= 1000.0, 15.0 + np.log(np.maximum(f, 1e-300) / 1000.0) * logstep, 3.0 * f / 200.0)


def _mel_to_hz(m):
    logstep = math.log(6.4) / 27.0
    return np.where(m >= 15.0, 1000.0 * np.exp(logstep * (m - 15.0)), 200.0 * m / 3.0)


def mel_tables(n_mels: int):
    """(filters float32 [201][n_mels], cos and sin float64 [400][201]) as Mel::new (audio.rs:161-189) builds them
    (the basis stored sample-major)."""
    fft_freqs = np.arange(N_BINS, dtype=np.float64) * (SR / 2.0) / (N_BINS - 1)
    m0, m1 = float(_hz_to_mel(np.float64(0.0))), float(_hz_to_mel(np.float64(8000.0)))
    ff = _mel_to_hz(m0 + (m1 - m0) * np.arange(n_mels + 2, dtype=np.float64) / (n_mels + 1))
    down = (fft_freqs[:, None] - ff[None, :-2]) / (ff[1:-1] - ff[:-2])[None, :]
    up = (ff[None, 2:] - fft_freqs[:, None]) / (ff[2:] - ff[1:-1])[None, :]
    enorm = 2.0 / (ff[2:] - ff[:-2])
    filters = (np.maximum(np.minimum(down, up), 0.0) * enorm[None, :]).astype(np.float32)
    n = np.arange(N_FFT)
    win = 0.5 - 0.5 * np.cos(2.0 * math.pi * n / N_FFT)
    a = 2.0 * math.pi * ((np.arange(N_BINS)[None, :] * n[:, None]) % N_FFT) / N_FFT
    return filters, win[:, None] * np.cos(a), win[:, None] * np.sin(a)


def features(y: np.ndarray, n_mels: int, tables=None):
    """(log-mel float32 [n_mels][3000], audio frames) of the first 30 s (Mel::features, audio.rs:195-249)."""
    filters, cosb, sinb = tables if tables is not None else mel_tables(n_mels)
    y = np.asarray(y, np.float32)
    n = min(len(y), N_SAMPLES)
    live = min(-(-(n + N_FFT // 2) // HOP), N_FRAMES)
    logmel = np.full((n_mels, N_FRAMES), -10.0, np.float32)
    if live > 0:
        # the 30 s buffer (zero padded) with centre reflect padding of N_FFT / 2
        idx = np.arange(live)[:, None] * HOP + np.arange(N_FFT)[None, :] - N_FFT // 2
        idx = np.where(idx < 0, -idx, idx)
        idx = np.where(idx >= N_SAMPLES, 2 * (N_SAMPLES - 1) - idx, idx)
        buf = np.zeros(N_SAMPLES, np.float64)
        buf[:n] = y[:n]
        frames = buf[idx]  # [live][400] float64
        re = np.zeros((live, N_BINS))
        im = np.zeros((live, N_BINS))
        for j in range(N_FFT):  # one sample at a time: the reference's summation order
            x = frames[:, j:j + 1]
            re = re + x * cosb[j][None, :]
            im = im + x * sinb[j][None, :]
        power = (re * re + im * im).astype(np.float32)
        acc = np.zeros((live, n_mels), np.float32)
        for k in range(N_BINS):  # float32 filter sums in bin order
            acc = (acc + filters[k][None, :] * power[:, k:k + 1]).astype(np.float32)
        logmel[:, :live] = np.log10(np.maximum(acc, np.float32(1e-10))).T
    mx = logmel.max()
    logmel = ((np.maximum(logmel, mx - np.float32(8.0)) + np.float32(4.0)) / np.float32(4.0)).astype(np.float32)
    return logmel, min(-(-n // HOP), N_FRAMES)
