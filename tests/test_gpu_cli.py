"""GPU end-to-end check of the command line (mz_cli, the reference's main.rs): WAV files in three formats and rates,
a model directory with a vocab.json, JSON out. The same clips through the Python API (library WAV reader and
resampler, device log-mel, Engine.new, transcribe) and the oracle's restatement of the text side
(oracle/text_ref.py) must give the same JSON document."""
import ctypes as C
import json
import os
import struct

import numpy as np
import pytest

from mimizuku_amd import _lib as L
from mimizuku_amd import model, synth, transcribe
from oracle import text_ref as T

pytestmark = pytest.mark.gpu
G = synth.TINY
NS = 480000


def wav_bytes(y: np.ndarray, sr: int, fmt: str) -> bytes:
    """y [frames][channels] float in [-1, 1) as 16-bit PCM, 24-bit PCM or 32-bit float."""
    ch = y.shape[1]
    if fmt == "pcm16":
        data, code, bits = (np.clip(y, -1, 1 - 2 ** -15) * 32768).astype("<i2").tobytes(), 1, 16
    elif fmt == "pcm24":
        v = (np.clip(y, -1, 1 - 2 ** -23) * 8388608).astype(np.int32).reshape(-1)
        data, code, bits = np.stack([v & 255, (v >> 8) & 255, (v >> 16) & 255], 1).astype(np.uint8).tobytes(), 1, 24
    else:
        data, code, bits = y.astype("<f4").tobytes(), 3, 32
    hdr = struct.pack("<IHHIIHH", 16, code, ch, sr, sr * ch * bits // 8, ch * bits // 8, bits)
    return b"RIFF" + struct.pack("<I", 36 + len(data)) + b"WAVEfmt " + hdr + b"data" + struct.pack("<I", len(data)) + data


def synthetic_vocab(eos: int, seed: int = 0) -> list[bytes]:
    """Byte-level entries: ids 0..255 the single bytes, the rest unique random 2-3 byte strings."""
    rng = np.random.default_rng(seed)
    out, seen = [bytes([b]) for b in range(256)], set()
    while len(out) < eos:
        b = bytes(rng.integers(32, 256, rng.integers(2, 4)).astype(np.uint8))
        if b not in seen:
            seen.add(b)
            out.append(b)
    return out


@pytest.fixture(scope="module")
def setup(tmp_path_factory):
    d = tmp_path_factory.mktemp("cli")
    W = synth.random_weights(G, seed=5, bias_std=0.02)
    gen = synth.generation_config(G)
    synth.write_model_dir(str(d / "model"), G, W, gen)
    entries = synthetic_vocab(gen["eos_token_id"])
    table = T.bytes_to_unicode()
    vocab = {"".join(table[b] for b in e): i for i, e in enumerate(entries)}
    (d / "model" / "vocab.json").write_text(json.dumps(vocab, ensure_ascii=False))
    rng = np.random.default_rng(3)
    clips = []
    for name, sr, secs, ch, fmt in [("a.wav", 16000, 4.0, 1, "pcm16"), ("b.wav", 44100, 2.5, 1, "float"),
                                    ("c.wav", 48000, 6.0, 2, "pcm24")]:
        t = np.arange(int(sr * secs)) / sr
        y = 0.2 * np.sin(2 * np.pi * (300 + 80 * t) * t)[:, None] + 0.05 * rng.standard_normal((len(t), ch))
        (d / name).write_bytes(wav_bytes(y, sr, fmt))
        clips.append(str(d / name))
    return d, clips, entries, gen


def cli(*args) -> int:
    argv = [b"mimizuku"] + [a.encode() for a in args]
    print("mz_cli", " ".join(args), flush=True)
    return L.lib().mz_cli(len(argv), (C.c_char_p * len(argv))(*argv))


def expected(model_dir, paths, entries, gen, bmax, language="auto", graph=True):
    """The same work through the Python API, then the oracle's JSON."""
    lib = L.lib()
    ys = []
    for p in paths:
        n, sr = C.c_size_t(), C.c_int()
        L.check(lib.mz_wav_read(p.encode(), None, 0, C.byref(n), C.byref(sr)))
        raw = np.zeros(n.value, np.float32)
        L.check(lib.mz_wav_read(p.encode(), raw.ctypes.data, n.value, C.byref(n), C.byref(sr)))
        m = C.c_size_t()
        L.check(lib.mz_resample_16k(raw.ctypes.data, n.value, sr.value, None, 0, C.byref(m)))
        y = np.zeros(m.value, np.float32)
        L.check(lib.mz_resample_16k(raw.ctypes.data, n.value, sr.value, y.ctypes.data, m.value, C.byref(m)))
        ys.append(y)
    ctx = model.Context(0)
    try:
        e = model.Engine.new(model_dir, bmax, bmax, ctx=ctx)
        p = transcribe.Prompt(e.gc, language)
        res = []
        for c0 in range(0, len(ys), bmax):
            chunk = ys[c0:c0 + bmax]
            buf = np.zeros((len(chunk), NS), np.float32)
            for i, y in enumerate(chunk):
                buf[i, :len(y)] = y
            ns = np.array([len(y) for y in chunk], np.int32)
            frames = np.zeros(len(chunk), np.int32)
            da, dm = ctx.upload_new(buf), ctx.alloc(len(chunk) * G.n_mels * 3000 * 4)
            L.check(lib.mz_log_mel(ctx.h, da, ns.ctypes.data, len(chunk), G.n_mels, dm, frames.ctypes.data))
            out, _ = transcribe.transcribe(e, dm, p, frames=frames, graph=graph, n=len(chunk))
            res += out
            ctx.free(da)
            ctx.free(dm)
        e.close()
    finally:
        ctx.close()
    lm = {v: k[2:-2] for k, v in gen["lang_to_id"].items()}
    return T.results(entries, gen["eos_token_id"], lm, [(paths[i], r.seq, r.ts, r.lang) for i, r in enumerate(res)])


def test_cli_end_to_end(setup, tmp_path):
    d, clips, entries, gen = setup
    out = tmp_path / "out.json"
    assert cli("--model", str(d / "model"), "--batch", "2", "--enc-group", "2", "--out", str(out), "--quiet",
               *clips) == 0
    got = json.loads(out.read_text())
    assert list(got) == clips
    want = expected(str(d / "model"), clips, entries, gen, 2)
    assert got == want


def test_cli_dir_language_and_no_graph(setup, tmp_path, capfd):
    d, clips, entries, gen = setup
    out = tmp_path / "out.json"
    assert cli("--model", str(d / "model"), "--dir", str(d), "--prefix", "b", "--language", "en", "--no-graph",
               "--out", str(out)) == 0
    err = capfd.readouterr().err
    assert "model on the GPU:" in err and "decoded 1 clips:" in err and "1 clips (2.5s of audio), batch 1" in err
    got = json.loads(out.read_text())
    assert got == expected(str(d / "model"), [os.path.join(str(d), "b.wav")], entries, gen, 1, "en", graph=False)
    assert got[os.path.join(str(d), "b.wav")]["language"] == "en"
