"""Writes log-mel golden vectors from transformers' WhisperFeatureExtractor (its numpy path and its torch path).

Run where transformers 5.15.0 is installed (the GPU tests only read the vectors it writes):
    PYTHONPATH=. python tests/golden/make_mel_golden.py

The waveforms are synthetic and regenerated from `waves.waveform(seed, seconds)`: a chirp plus a tone plus noise,
amplitude 0.5. Each fixture holds the seed and length, the 80- or 128-bin features of the default (torch) path at
the frames `cols` (every frame of the live part for short clips, every 7th for the 30 s one), the largest
difference between the numpy and torch paths, and the attention-mask frame count.
"""
import os

import numpy as np
import torch
from transformers import WhisperFeatureExtractor

from waves import waveform

HERE = os.path.dirname(os.path.abspath(__file__))
CASES = {"mel80_7s": (80, 11, 7.3), "mel128_30s": (128, 12, 30.0), "mel128_short": (128, 13, 0.9)}


def main():
    for name, (n_mels, seed, secs) in CASES.items():
        fe = WhisperFeatureExtractor(feature_size=n_mels)
        y = waveform(seed, secs)
        np_feat = fe._np_extract_fbank_features(y[None, :].copy() if len(y) >= 480000 else
                                                np.pad(y, (0, 480000 - len(y)))[None, :], "cpu")[0]
        out = fe(y, sampling_rate=16000, return_tensors="np", return_attention_mask=True)
        with torch.no_grad():
            torch_feat = out["input_features"][0]
        live = int(out["attention_mask"].sum())
        cols = np.arange(0, 3000, 7) if live >= 3000 else np.arange(min(3000, live + 4))
        np.savez_compressed(os.path.join(HERE, f"{name}.npz"), seed=seed, seconds=secs, n_mels=n_mels, cols=cols,
                            features=torch_feat[:, cols].astype(np.float32), pad_value=float(torch_feat[0, -1]),
                            np_vs_torch=float(np.abs(np_feat - torch_feat).max()), frames=live)
        print(name, np_feat.shape, float(np.abs(np_feat - torch_feat).max()))


if __name__ == "__main__":
    main()
