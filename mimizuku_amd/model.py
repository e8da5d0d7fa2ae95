"""Host-side mirror of the reference's engine surface (src/model.rs, src/gpu.rs) over the C ABI.

    ctx = Context()                                    # Gpu::new (src/gpu.rs:122-137)
    e = Engine.new(model_dir, bmax=32, eg=8)           # Engine::new (src/model.rs:333-514)
    e.encode(mels, slot0)                              # Engine::encode (:545-625)
    e.reset(prompts); e.detect(b); e.step(b, lang, np) # :628-736
"""
from __future__ import annotations

import ctypes as C
import dataclasses
import weakref

import numpy as np

from . import _lib as L
from ._lib import MzError, check, ptr

TENC = 1500
NFRAMES = 3000


class Context:
    """One device and its stream (the reference's `Gpu`). Closing it first closes the engines built on it."""

    def __init__(self, device: int = 0):
        self.h = C.c_void_p()
        self.engines = weakref.WeakSet()
        check(L.lib().mz_init(device, C.byref(self.h)))

    def close(self):
        if self.h:
            for e in list(self.engines):
                e.close()
            L.lib().mz_ctx_free(self.h)
            self.h = C.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # memory (device addresses are ints, as the reference's Ptr = u64)
    def alloc(self, nbytes: int) -> int:
        p = C.c_uint64()
        check(L.lib().mz_alloc(self.h, nbytes, C.byref(p)))
        return p.value

    def free(self, p: int):
        check(L.lib().mz_free(self.h, p))

    def upload(self, dst: int, a: np.ndarray):
        a = np.ascontiguousarray(a)
        check(L.lib().mz_upload(self.h, dst, ptr(a), a.nbytes))

    def upload_new(self, a: np.ndarray) -> int:
        p = self.alloc(a.nbytes)
        self.upload(p, a)
        return p

    def download(self, src: int, shape, dtype) -> np.ndarray:
        out = np.empty(shape, dtype)
        check(L.lib().mz_download(self.h, ptr(out), src, out.nbytes))
        return out

    def sync(self):
        check(L.lib().mz_sync(self.h))

    def mem_info(self) -> tuple[int, int]:
        f, t = C.c_size_t(), C.c_size_t()
        check(L.lib().mz_mem_info(self.h, C.byref(f), C.byref(t)))
        return f.value, t.value

    def event(self) -> int:
        e = C.c_uint64()
        check(L.lib().mz_event_create(self.h, C.byref(e)))
        return e.value

    def record(self, ev: int):
        check(L.lib().mz_event_record(self.h, ev))

    @staticmethod
    def elapsed_ms(a: int, b: int) -> float:
        ms = C.c_float()
        check(L.lib().mz_event_elapsed_ms(a, b, C.byref(ms)))
        return ms.value


@dataclasses.dataclass
class Dims:
    """Model dimensions from config.json (src/model.rs:14-62)."""
    d: int
    ff: int
    nh: int
    enc_layers: int
    dec_layers: int
    n_mels: int
    vocab: int
    max_t: int

    @staticmethod
    def load(model_dir: str) -> "Dims":
        """config.json through the library's own reader (mz_model_open: strict JSON, the same range checks)."""
        return ModelDir(model_dir).dims

    def c(self) -> L.Dims:
        return L.Dims(*dataclasses.astuple(self))


@dataclasses.dataclass
class GenCfg:
    """Prompt and decoding settings from generation_config.json (src/model.rs:64-156)."""
    sot: int
    eos: int
    no_timestamps: int
    langs: list  # [(code, token)]
    tasks: list  # [(name, token)]
    suppress: list
    begin_suppress: list
    align_heads: list  # [(layer, head)]

    @staticmethod
    def from_dict(g: dict, dims: Dims) -> "GenCfg":
        def tok(v):
            if not isinstance(v, int) or isinstance(v, bool) or not (0 <= v < dims.vocab):
                raise MzError(f"generation_config.json: {v!r} is not a token id")
            return v

        heads = g.get("alignment_heads")
        if heads is None:  # openai/whisper's default: every head of the second half of the decoder layers
            heads = [(l, h) for l in range(dims.dec_layers // 2, dims.dec_layers) for h in range(dims.nh)]
        heads = [tuple(x) for x in heads]
        if any(len(x) != 2 or not (0 <= x[0] < dims.dec_layers and 0 <= x[1] < dims.nh) for x in heads):
            raise MzError("generation_config.json: alignment_heads must be [layer, head] pairs within the model")
        if not heads or len(set(heads)) != len(heads):
            raise MzError("generation_config.json: alignment_heads is empty or has duplicates")
        multilingual = g.get("is_multilingual", True)
        bs = [tok(t) for t in (g.get("begin_suppress_tokens") or [])]
        if len(bs) > 2:
            raise MzError("generation_config.json: more than two begin_suppress_tokens are not supported")
        strip = lambda s: s[2:-2] if s.startswith("<|") and s.endswith("|>") else s  # noqa: E731
        langs = [(strip(k), tok(v)) for k, v in (g.get("lang_to_id") or {}).items()] if multilingual else []
        tasks = [(k, tok(v)) for k, v in (g.get("task_to_id") or {}).items()]
        if multilingual and (not langs or not tasks):
            raise MzError("generation_config.json: a multilingual model needs lang_to_id and task_to_id")
        return GenCfg(tok(g.get("decoder_start_token_id")), tok(g.get("eos_token_id")),
                      tok(g.get("no_timestamps_token_id")), langs, tasks,
                      [tok(t) for t in (g.get("suppress_tokens") or [])], bs, heads)

    @staticmethod
    def load(model_dir: str, dims: Dims | None = None) -> "GenCfg":
        """generation_config.json through the library's own reader (mz_model_open)."""
        return ModelDir(model_dir).gencfg

    def lang_token(self, code: str):
        return next((t for c, t in self.langs if c == code), None)

    def lang_code(self, tok: int):
        return next((c for c, t in self.langs if t == tok), None)

    def c(self):
        """ctypes struct plus the arrays it points into (keep both alive)."""
        arrs = [np.ascontiguousarray(np.array(x, np.int32).reshape(-1)) for x in
                (self.suppress, self.begin_suppress, [t for _, t in self.langs], self.align_heads)]
        p = [a.ctypes.data_as(C.POINTER(C.c_int32)) for a in arrs]
        s = L.GenCfgC(self.sot, self.eos, self.no_timestamps, p[0], len(self.suppress), p[1], len(self.begin_suppress),
                      p[2], len(self.langs), p[3], len(self.align_heads))
        return s, arrs


class ModelDir:
    """A Hugging Face model directory read by the library (mz_model_open: config.json -> Dims, src/model.rs:33-61;
    generation_config.json -> GenCfg, :78-146). from_dict above is the same reading of an in-memory dict."""

    def __init__(self, model_dir: str):
        h = C.c_void_p()
        check(L.lib().mz_model_open(model_dir.encode(), C.byref(h)))
        try:
            lib = L.lib()
            dc = L.Dims()
            check(lib.mz_model_dims(h, C.byref(dc)))
            self.dims = Dims(*[getattr(dc, f.name) for f in dataclasses.fields(Dims)])
            g = L.GenCfgC()
            check(lib.mz_model_gencfg(h, C.byref(g)))
            arr = lambda p, n: [int(p[i]) for i in range(n)]  # noqa: E731
            heads = arr(g.align_heads, 2 * g.n_align)

            def entries(fn, n):
                out = []
                for i in range(n):
                    name, tok = C.c_char_p(), C.c_int32()
                    check(fn(h, i, C.byref(name), C.byref(tok)))
                    out.append((name.value.decode(), tok.value))
                return out
            langs = entries(lib.mz_model_lang, g.n_langs)
            tasks, i = [], 0
            while True:  # task_to_id entries (the count is not part of mz_gencfg)
                name, tok = C.c_char_p(), C.c_int32()
                if lib.mz_model_task(h, i, C.byref(name), C.byref(tok)) != 0:
                    break
                tasks.append((name.value.decode(), tok.value))
                i += 1
            self.gencfg = GenCfg(g.sot, g.eos, g.no_timestamps, langs, tasks, arr(g.suppress, g.n_suppress),
                                 arr(g.begin_suppress, g.n_begin_suppress),
                                 [(heads[2 * k], heads[2 * k + 1]) for k in range(g.n_align)])
        finally:
            L.lib().mz_model_free(h)


def scratch_bytes(dims: Dims, na: int, bmax: int, eg: int) -> int:
    """Device bytes the engine allocates besides the weights (src/model.rs:324-330)."""
    dc = dims.c()
    return int(L.lib().mz_scratch_bytes(C.byref(dc), na, bmax, eg))


class Engine:
    """Whisper on one MI355X: encoder for groups of clips, cross k/v for every decoder layer, and one greedy
    decoding step for up to bmax rows (src/model.rs:267-322 `Engine`)."""

    def __init__(self, ctx: Context, dims: Dims, gc: GenCfg, bmax: int, eg: int):
        self.ctx, self.dims, self.gc, self.bmax, self.eg = ctx, dims, gc, bmax, eg
        self.h = C.c_void_p()
        dc = dims.c()
        gcs, keep = gc.c()
        check(L.lib().mz_engine_new(ctx.h, C.byref(dc), C.byref(gcs), bmax, eg, C.byref(self.h)))
        del keep
        ctx.engines.add(self)

    @staticmethod
    def new(model_dir: str, bmax: int, eg: int, ctx: Context | None = None) -> "Engine":
        """Engine for a Hugging Face model directory (config.json, generation_config.json, model.safetensors), read
        by the library: the configs through mz_model_open, the mapped checkpoint through mz_engine_load."""
        md = ModelDir(model_dir)
        e = Engine(ctx or Context(), md.dims, md.gencfg, bmax, eg)
        check(L.lib().mz_engine_load(e.h, model_dir.encode()))
        return e

    def load(self, weights: dict):
        """Place every checkpoint tensor (F16 or F32) and check none is missing (Loader, src/model.rs:200-265)."""
        for name, a in weights.items():
            self.put(name, a)
        check(L.lib().mz_engine_finish(self.h))

    def put(self, name: str, a: np.ndarray):
        a = np.ascontiguousarray(a)
        if a.dtype == np.float16:
            dt = L.DT_F16
        elif a.dtype == np.float32:
            dt = L.DT_F32
        else:
            raise MzError(f"{name}: unsupported dtype {a.dtype}")
        shp = (C.c_int64 * a.ndim)(*a.shape)
        check(L.lib().mz_engine_put(self.h, name.encode(), dt, ptr(a), shp, a.ndim))

    def close(self):
        if self.h:
            if self.ctx.h:  # the context frees its engines' device memory itself when it is closed first
                L.lib().mz_engine_free(self.h)
            self.h = C.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # ---- the reference's engine API
    def encode(self, mels: np.ndarray, slot0: int = 0):
        m = np.ascontiguousarray(mels, np.float32)
        assert m.ndim == 3 and m.shape[1:] == (self.dims.n_mels, NFRAMES), m.shape
        check(L.lib().mz_engine_encode(self.h, ptr(m), m.shape[0], slot0))

    def encode_device(self, mels: int, n: int, slot0: int = 0):
        """Encoder for n clips whose log-mel f32 [n][n_mels][3000] is already in device memory at address mels."""
        check(L.lib().mz_engine_encode_device(self.h, mels, n, slot0))

    # ---- kernel timing (events on the engine's stream)
    def profile(self, on: bool = True):
        """Clear the timing records and switch event timing of encoder launches and step replays on or off."""
        check(L.lib().mz_engine_profile(self.h, int(on)))

    def profile_read(self) -> dict:
        """{kernel class: (total ms, launches)} over the records since the last profile() call."""
        out = {}
        for i, name in enumerate(L.K_NAMES):
            ms, n = C.c_double(), C.c_int()
            check(L.lib().mz_engine_profile_read(self.h, i, C.byref(ms), C.byref(n)))
            out[name] = (ms.value, n.value)
        return out

    def reset(self, prompts):
        p = np.ascontiguousarray(np.array(prompts, np.int32))
        check(L.lib().mz_engine_reset(self.h, ptr(p), p.shape[0], p.shape[1]))

    def detect(self, b: int) -> list[int]:
        out = np.zeros(b, np.int32)
        check(L.lib().mz_engine_detect(self.h, b, ptr(out)))
        return out.tolist()

    def step(self, b: int, lang: bool = False, prompt_len: int = 4):
        check(L.lib().mz_engine_step(self.h, b, int(lang), prompt_len))

    def capture(self, b: int, prompt_len: int):
        check(L.lib().mz_engine_capture(self.h, b, prompt_len))

    def replay(self):
        check(L.lib().mz_engine_replay(self.h))

    def set_trace(self, on: bool = True):
        check(L.lib().mz_engine_set_trace(self.h, int(on)))

    # ---- buffers
    def buffer(self, which: int) -> tuple[int, int]:
        p, n = C.c_uint64(), C.c_size_t()
        check(L.lib().mz_engine_buffer(self.h, which, C.byref(p), C.byref(n)))
        return p.value, n.value

    def read(self, which: int, dtype, shape, offset: int = 0) -> np.ndarray:
        """An array of `shape` read from an engine buffer at byte offset `offset` (after the stream's work)."""
        out = np.empty(shape, dtype)
        check(L.lib().mz_engine_read(self.h, which, ptr(out), offset, out.nbytes))
        return out

    def tokens(self) -> np.ndarray:
        return self.read(L.BUF_TOK, np.int32, (self.bmax, self.dims.max_t))

    def done(self) -> np.ndarray:
        return self.read(L.BUF_DONE, np.int32, (self.bmax,))

    def position(self) -> int:
        return int(self.read(L.BUF_CTR, np.int32, (4,))[0])

    def logits(self) -> np.ndarray:
        return self.read(L.BUF_LOGITS, np.float32, (self.bmax, self.dims.vocab))

    def align(self) -> np.ndarray:
        """[bmax][max_t][n_align][1500] alignment-head probabilities (fp32)."""
        return self.read(L.BUF_ALIGN, np.float32, (self.bmax, self.dims.max_t, len(self.gc.align_heads), TENC))

    def enc_out(self, n: int | None = None) -> np.ndarray:
        n = n or self.eg
        out = np.empty((n, TENC, self.dims.d), np.float16)
        check(L.lib().mz_engine_read(self.h, L.BUF_ENC_OUT, ptr(out), 0, out.nbytes))
        return out

    def trace(self, n: int | None = None) -> np.ndarray:
        """[enc_layers][eg][1500][d] fp32 inputs of every encoder layer of the last encode (set_trace first)."""
        return self.read(L.BUF_TRACE, np.float32, (self.dims.enc_layers, self.eg, TENC, self.dims.d))[:, :n or self.eg]

    def dec_x(self) -> np.ndarray:
        return self.read(L.BUF_DEC_X, np.float32, (self.bmax, self.dims.d))

    def dec_trace(self) -> np.ndarray:
        """[dec_layers + 1][bmax][d] fp32 decoder residual entering every layer (and after the last) of the last
        eager step (set_trace first)."""
        return self.read(L.BUF_DEC_TRACE, np.float32, (self.dims.dec_layers + 1, self.bmax, self.dims.d))

    def self_kv(self) -> tuple[np.ndarray, np.ndarray]:
        """Self-attention caches, fp16 [dec_layers][bmax][nh][max_t][64] each (keys, values)."""
        shp = (self.dims.dec_layers, self.bmax, self.dims.nh, self.dims.max_t, 64)
        return self.read(L.BUF_SELF_K, np.float16, shp), self.read(L.BUF_SELF_V, np.float16, shp)

    def xkv(self) -> np.ndarray:
        """Cross-attention keys / values of every decoder layer, fp16 [bmax][dec_layers][2][nh][1536][64]."""
        return self.read(L.BUF_XKV, np.float16, (self.bmax, self.dims.dec_layers, 2, self.dims.nh, 1536, 64))
