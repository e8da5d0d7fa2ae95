"""Synthetic test waveforms, shared by the mel fixture generator (make_mel_golden.py, build container only) and the
GPU tests (numpy only: nothing here imports torch or transformers)."""
import numpy as np


def waveform(seed: int, seconds: float) -> np.ndarray:
    """A chirp plus a tone plus noise at 16 kHz, peak amplitude 0.5, float32."""
    rng = np.random.default_rng(seed)
    t = np.arange(int(16000 * seconds)) / 16000.0
    y = 0.3 * np.sin(2 * np.pi * (200 + 300 * t) * t) + 0.1 * np.sin(2 * np.pi * 2500 * t) \
        + 0.05 * rng.standard_normal(len(t))
    return (0.5 * y / max(1e-9, np.abs(y).max())).astype(np.float32)
