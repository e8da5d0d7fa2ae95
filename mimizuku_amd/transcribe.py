"""The batch transcription API (src/transcribe.rs): prompts, then encode + greedy decode + token timestamps.

The loop itself runs in the library (mz_transcribe, a C++ restatement of transcribe.rs:104-167: encoder groups,
reset, optional language detection, one captured step graph replayed until every row is done, alignment rows to
DTW). This module mirrors the Rust types around it.
"""
from __future__ import annotations

import ctypes as C
import dataclasses

import numpy as np

from . import _lib as L
from ._lib import MzError, check, ptr
from .model import NFRAMES, Engine, GenCfg


class Prompt:
    """start, language, task, no timestamps; English-only models: start, no timestamps (transcribe.rs:58-93)."""

    def __init__(self, gc: GenCfg, language: str = "auto", task: str = "transcribe"):
        self.multilingual = bool(gc.langs)
        self.sot, self.no_timestamps = gc.sot, gc.no_timestamps
        if not self.multilingual:
            if language not in ("auto", "en") or task != "transcribe":
                raise MzError("this English-only model takes only --language en (or auto) and --task transcribe")
            self.task, self.lang = -1, None
            return
        if language == "auto":
            self.lang = None
        else:
            self.lang = gc.lang_token(language)
            if self.lang is None:
                raise MzError(f"--language {language}: not a language of this model")
        t = [tok for n, tok in gc.tasks if n == task]
        if not t:
            raise MzError(f"--task {task}: unknown task")
        self.task = t[0]

    def tokens(self, lang: int) -> list[int]:
        return [self.sot, lang, self.task, self.no_timestamps] if self.multilingual else [self.sot, self.no_timestamps]

    def detect(self) -> bool:
        return self.multilingual and self.lang is None


@dataclasses.dataclass
class Decoded:
    """One clip's result: language token, the whole sequence (prompt included) and each token's start time."""
    lang: int
    seq: list
    ts: list


@dataclasses.dataclass
class Times:
    enc: float = 0.0
    dec: float = 0.0
    post: float = 0.0
    steps: int = 0


def transcribe(e: Engine, mels, p: Prompt, frames=None, graph: bool = True, max_new: int = 0,
               half_align: bool = True, n: int | None = None) -> tuple[list[Decoded], Times]:
    """Encode and decode up to e.bmax clips; returns their tokens with timestamps (src/transcribe.rs:104-167).

    mels is log-mel f32 [n][n_mels][3000], either a host array or, with n given, the address of such an array in
    device memory (then nothing crosses PCIe before the encoder).
    max_new > 0 caps the generated tokens (the reference decodes until every row ends or max_t - 1 steps).
    half_align rounds the timestamp arithmetic through fp16 where an fp16 model does (src/align.rs).
    """
    m, n = _mels(e, mels, n)
    return _decode(e, n, p, frames, graph, max_new, half_align,
                   lambda args: L.lib().mz_transcribe_device(e.h, m, *args) if isinstance(m, int)
                   else L.lib().mz_transcribe(e.h, ptr(m), *args))


def _mels(e: Engine, mels, n):
    if isinstance(mels, int):
        if n is None:
            raise MzError("transcribe: the clip count n is needed with device-resident mels")
        return mels, n
    m = np.ascontiguousarray(mels, np.float32)
    if m.ndim != 3 or m.shape[1:] != (e.dims.n_mels, NFRAMES):
        raise MzError(f"mels must be [n][{e.dims.n_mels}][{NFRAMES}], got {m.shape}")
    return m, m.shape[0]


def _decode(e: Engine, n: int, p: Prompt, frames, graph, max_new, half_align, call):
    fr = np.ascontiguousarray(np.full(n, NFRAMES, np.int32) if frames is None else np.array(frames, np.int32))
    if fr.shape != (n,):
        raise MzError(f"frames must hold {n} counts, got {fr.shape}")
    prompt = np.array(p.tokens(p.lang if p.lang is not None else p.sot), np.int32)
    mt = e.dims.max_t
    seq = np.zeros((n, mt), np.int32)
    seq_len = np.zeros(n, np.int32)
    ts = np.zeros((n, mt), np.float32)
    langs = np.zeros(n, np.int32)
    tm = L.Times()
    check(call((ptr(fr), n, ptr(prompt), len(prompt), int(p.detect()), int(graph), int(max_new), int(half_align),
                ptr(seq), ptr(seq_len), ptr(ts), ptr(langs), C.byref(tm))))
    out = [Decoded(int(langs[i]), seq[i, :seq_len[i]].tolist(), ts[i, :seq_len[i]].tolist()) for i in range(n)]
    return out, Times(tm.enc, tm.dec, tm.post, tm.steps)


def submit(e: Engine, mels, n: int | None = None) -> int:
    """Enqueue the encoder of one chunk of up to e.bmax clips and return its clip count (mz_transcribe_submit);
    collect it before submitting another."""
    m, n = _mels(e, mels, n)
    check(L.lib().mz_transcribe_submit_device(e.h, m, n) if isinstance(m, int)
          else L.lib().mz_transcribe_submit(e.h, ptr(m), n))
    return n


def collect(e: Engine, n: int, p: Prompt, frames=None, graph: bool = True, max_new: int = 0,
            half_align: bool = True) -> tuple[list[Decoded], Times]:
    """Decode the submitted chunk (n clips) and return what transcribe returns for it (mz_transcribe_collect)."""
    return _decode(e, n, p, frames, graph, max_new, half_align,
                   lambda args: L.lib().mz_transcribe_collect(e.h, *args))


def transcribe_all(e: Engine, mels, p: Prompt, frames=None, graph: bool = True, max_new: int = 0,
                   half_align: bool = True, n: int | None = None) -> tuple[list[Decoded], Times]:
    """Any number of clips in chunks of e.bmax, in order (the loop of src/main.rs:195-200), one transcribe per
    chunk; the stage times are summed over the chunks."""
    m, n = _mels(e, mels, n)
    fr = np.full(n, NFRAMES, np.int32) if frames is None else np.asarray(frames, np.int32)
    step = e.dims.n_mels * NFRAMES
    out, tm = [], Times()
    for c0 in range(0, n, e.bmax):
        cn = min(e.bmax, n - c0)
        o, t = transcribe(e, m + 4 * c0 * step if isinstance(m, int) else m[c0:c0 + cn], p, fr[c0:c0 + cn], graph,
                          max_new, half_align, cn)
        out += o
        tm = Times(tm.enc + t.enc, tm.dec + t.dec, tm.post + t.post, tm.steps + t.steps)
    return out, tm


def jump_times(w: np.ndarray, cols: int, width: int = 7, half: bool = True) -> np.ndarray:
    """Token start times from alignment-head weights w [rows][heads][cols_full] (src/align.rs:8-63)."""
    w = np.ascontiguousarray(w, np.float32)
    rows, heads, full = w.shape
    out = np.zeros(rows, np.float32)
    check(L.lib().mz_jump_times(ptr(w), rows, heads, full, cols, width, int(half), ptr(out)))
    return out


def align_cost(w: np.ndarray, cols: int, width: int = 7, half: bool = True) -> np.ndarray:
    """The cost jump_times hands to the DTW, float64 [rows][cols] (src/align.rs:14-52)."""
    w = np.ascontiguousarray(w, np.float32)
    rows, heads, full = w.shape
    out = np.zeros((rows, cols), np.float64)
    check(L.lib().mz_align_cost(ptr(w), rows, heads, full, cols, width, int(half), ptr(out)))
    return out


def jump_times_device(ctx, w: int, clip_stride: int, rows, cols, heads: int, cols_full: int, width: int = 7,
                      half: bool = True) -> list[np.ndarray]:
    """Token start times of several clips on the device (the same bits as jump_times per clip): clip c's weights are
    rows[c] x heads x cols_full floats at device address w + 4 * c * clip_stride, cropped to cols[c] frames."""
    rows = np.ascontiguousarray(rows, np.int32)
    cols = np.ascontiguousarray(cols, np.int32)
    n = len(rows)
    stride = max(int(rows.max()) if n else 0, 1)
    out = np.zeros((n, stride), np.float32)
    check(L.lib().mz_jump_times_device(ctx.h, w, clip_stride, n, ptr(rows), ptr(cols), heads, cols_full, width,
                                       int(half), ptr(out), stride))
    return [out[c, :rows[c]] for c in range(n)]


def jump_times_device_noalloc(ctx, w: int, clip_stride: int, rows, cols, heads: int, cols_full: int, width: int = 7,
                              half: bool = True) -> list[np.ndarray]:
    """jump_times_device through the entry point that allocates no device memory (its scratch is a static array per
    device): the same times, bit for bit."""
    rows = np.ascontiguousarray(rows, np.int32)
    cols = np.ascontiguousarray(cols, np.int32)
    n = len(rows)
    stride = max(int(rows.max()) if n else 0, 1)
    out = np.zeros((n, stride), np.float32)
    check(L.lib().mz_jump_times_device_noalloc(ctx.h, w, clip_stride, n, ptr(rows), ptr(cols), heads, cols_full,
                                               width, int(half), ptr(out), stride))
    return [out[c, :rows[c]] for c in range(n)]


def dtw(m: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """DTW path (text, time indices) over cost m [rows][cols] (src/align.rs:66-106)."""
    m = np.ascontiguousarray(m, np.float64)
    rows, cols = m.shape
    text = np.zeros(rows + cols, np.int32)
    time = np.zeros(rows + cols, np.int32)
    n = np.zeros(1, np.int32)
    check(L.lib().mz_dtw(ptr(m), rows, cols, ptr(text), ptr(time), ptr(n)))
    return text[:n[0]], time[:n[0]]
