"""CPU checks of the text side and the command line: the library's tokenizer decoding (mz_tok_*) and JSON result
(mz_json_time, mz_results_json) against the reference's KATs (src/tok.rs:87-122) and the oracle
(oracle/text_ref.py), vocab.json validation (Tok::load, tok.rs:25-45), and mz_cli's argument handling
(src/main.rs:52-95) up to the point where it would need a GPU."""
import ctypes as C
import json
import os

import numpy as np
import pytest

from mimizuku_amd import _lib as L
from mimizuku_amd import synth
from oracle import text_ref as T


class Tok:
    def __init__(self, entries: list[bytes] | None = None, model_dir: str | None = None, vocab=0, eos=0):
        self.h = C.c_void_p()
        if model_dir is not None:
            L.check(L.lib().mz_tok_open(model_dir.encode(), vocab, eos, C.byref(self.h)))
        else:
            self.keep = [C.create_string_buffer(e, len(e)) for e in entries]
            arr = (C.c_char_p * len(entries))(*[C.cast(b, C.c_char_p) for b in self.keep])
            lens = (C.c_size_t * len(entries))(*[len(e) for e in entries])
            L.check(L.lib().mz_tok_from_bytes(arr, lens, len(entries), C.byref(self.h)))

    def __del__(self):
        if self.h:
            L.lib().mz_tok_free(self.h)

    def decode(self, ids) -> str:
        a = np.array(ids, np.int32)
        n = C.c_size_t()
        L.check(L.lib().mz_tok_decode(self.h, a.ctypes.data, len(a), None, 0, C.byref(n)))
        buf = C.create_string_buffer(n.value + 1)
        L.check(L.lib().mz_tok_decode(self.h, a.ctypes.data, len(a), buf, n.value + 1, C.byref(n)))
        return buf.raw[:n.value].decode()

    def pieces(self, ids, ts, eos):
        a, t = np.array(ids, np.int32), np.array(ts, np.float32)
        k, n = C.c_int(), C.c_size_t()
        L.check(L.lib().mz_tok_pieces(self.h, a.ctypes.data, t.ctypes.data, len(a), eos, None, 0, C.byref(n), None,
                                      None, None, C.byref(k)))
        buf = C.create_string_buffer(n.value + 1)
        off = np.zeros(k.value + 1, np.int32)
        t0, t1 = np.zeros(k.value, np.float32), np.zeros(k.value, np.float32)
        L.check(L.lib().mz_tok_pieces(self.h, a.ctypes.data, t.ctypes.data, len(a), eos, buf, n.value + 1,
                                      C.byref(n), off.ctypes.data, t0.ctypes.data, t1.ctypes.data, C.byref(k)))
        raw = buf.raw[:n.value]
        return [(raw[off[i]:off[i + 1]].decode(), float(t0[i]), float(t1[i])) for i in range(k.value)]


def test_byte_table_is_a_bijection(tmp_path):
    """byte_table_is_a_bijection (tok.rs:92-100): every byte's printable character, read from a vocab.json, decodes
    to that byte; Ġ is the space."""
    table = T.bytes_to_unicode()
    assert len(table) == 256 and table[ord(" ")] == "Ġ" and table[ord("!")] == "!"
    vocab = {table[b]: b for b in range(256)}
    (tmp_path / "vocab.json").write_text(json.dumps(vocab, ensure_ascii=False))
    t = Tok(model_dir=str(tmp_path), vocab=256, eos=256)
    for b in range(256):
        got = t.decode([b])
        assert got == bytes([b]).decode("utf-8", errors="replace"), b


def test_decode_joins_bytes_and_cleans_spaces():
    """decode_joins_bytes_and_cleans_spaces (tok.rs:102-113), library and oracle."""
    entries = [b" Hello", b" .", bytes([0xE6, 0x97]), bytes([0xA5]), b" n't"]
    t = Tok(entries)
    for ids, want in [([0, 1], " Hello."), ([2], "�"), ([2, 3], "日"), ([0, 4], " Hellon't"), ([99], ""),
                      ([-1], "")]:
        assert t.decode(ids) == want == T.decode(entries, ids)


def test_pieces_are_whole_characters():
    """pieces_are_whole_characters (tok.rs:115-122), library and oracle."""
    entries = [b" a", bytes([0xE6, 0x97]), bytes([0xA5]), bytes([0xFF]), bytes([0xE6])]
    ts = [0.0, 0.1, 0.2, 0.3, 0.4, 0.5]
    want = [(" a", 0.0, 0.1), ("日", 0.1, 0.3), ("�", 0.3, 0.4), ("�", 0.5, 0.5)]
    got = Tok(entries).pieces([0, 1, 2, 3, 9, 4], ts, 5)
    assert [(s, round(a, 6), round(b, 6)) for s, a, b in got] == want
    assert T.pieces(entries, [0, 1, 2, 3, 9, 4], ts, 5) == want


def test_decode_matches_the_oracle_on_random_bytes():
    rng = np.random.default_rng(0)
    entries = [bytes(rng.integers(0, 256, rng.integers(0, 4)).astype(np.uint8)) for _ in range(300)]
    entries += [" ẞ".encode(), "😀".encode()[:2], "😀".encode()[2:], b" 's", b" '", b" "]
    t = Tok(entries)
    for _ in range(200):
        ids = rng.integers(-2, len(entries) + 2, rng.integers(0, 12)).tolist()
        ts = np.sort(rng.random(len(ids))).astype(np.float32).tolist()
        assert t.decode(ids) == T.decode(entries, ids), ids
        got = t.pieces(ids, ts, len(entries) - 3)
        ref = T.pieces(entries, ids, ts, len(entries) - 3)
        assert [g[0] for g in got] == [r[0] for r in ref], ids
        assert [g[1:] for g in got] == [(float(np.float32(a)), float(np.float32(b))) for _, a, b in ref], ids


def lib_time(x) -> str:
    n = C.c_size_t()
    buf = C.create_string_buffer(64)
    L.check(L.lib().mz_json_time(float(x), buf, 64, C.byref(n)))
    return buf.value.decode()


def test_json_times_print_as_python_does():
    rng = np.random.default_rng(1)
    xs = np.concatenate([np.arange(0, 1502) * np.float32(0.02), rng.random(2000).astype(np.float32) * 30,
                         np.array([0, 1, 2, 10, 12, 29.99, 30, 100, 1234.5, 0.005, 0.015, 1e-3], np.float32)])
    for x in xs.astype(np.float32):
        assert lib_time(x) == T.json_time(x), float(x)


def test_vocab_json_checks(tmp_path):
    """Tok::load's refusals (tok.rs:25-45): an id at or past the vocabulary, an id used twice, a character outside
    the byte table, a text id (below eos) without an entry."""
    table = T.bytes_to_unicode()
    base = {table[b]: b for b in range(256)}
    for extra, vocab, eos, what in [({"x!": 300}, 256, 256, "not below"), ({"Ġa": 5}, 256, 256, "used twice"),
                                    ({"一": 256}, 300, 256, "char"), ({}, 300, 257, "no entry for text token 256"),
                                    ({"ab": -1}, 300, 256, "not below")]:
        (tmp_path / "vocab.json").write_text(json.dumps({**base, **extra}, ensure_ascii=False))
        with pytest.raises(L.MzError, match=what):
            Tok(model_dir=str(tmp_path), vocab=vocab, eos=eos)


def test_results_json_matches_the_oracle(tmp_path):
    g = synth.TINY
    synth.write_model_dir(str(tmp_path), g, {"x": np.zeros(1, np.float16)})
    gen = json.load(open(tmp_path / "generation_config.json"))
    rng = np.random.default_rng(2)
    entries = [bytes(rng.integers(32, 127, rng.integers(1, 4)).astype(np.uint8)) for _ in range(50257)]
    entries[7] = b' "q\\\n\t'
    t = Tok(entries)
    m = C.c_void_p()
    L.check(L.lib().mz_model_open(str(tmp_path).encode(), C.byref(m)))
    try:
        mt = 448
        paths = [b"/a/one.wav", "/b/zwei ü.wav".encode()]
        seqs = [[50258, 50259, 50359, 50363, 7, 100, 2000, 50257], [50258, 50266, 50359, 50363, 3, 4]]
        seq = np.zeros((2, mt), np.int32)
        ts = np.zeros((2, mt), np.float32)
        lens = np.array([len(s) for s in seqs], np.int32)
        for i, s in enumerate(seqs):
            seq[i, :len(s)] = s
            ts[i, :len(s)] = np.float32(0.02) * np.arange(len(s), dtype=np.float32) * 7
        langs = np.array([50259, 50266], np.int32)
        parr = (C.c_char_p * 2)(*paths)
        n = C.c_size_t()
        L.check(L.lib().mz_results_json(t.h, m, 2, parr, seq.ctypes.data, lens.ctypes.data, mt, ts.ctypes.data,
                                        langs.ctypes.data, None, 0, C.byref(n)))
        buf = C.create_string_buffer(n.value + 1)
        L.check(L.lib().mz_results_json(t.h, m, 2, parr, seq.ctypes.data, lens.ctypes.data, mt, ts.ctypes.data,
                                        langs.ctypes.data, buf, n.value + 1, C.byref(n)))
        text = buf.raw[:n.value].decode()
    finally:
        L.lib().mz_model_free(m)
    assert text.endswith("}\n") and text.startswith('{"/a/one.wav": {"language": "en", "text": ')
    lm = {v: k[2:-2] for k, v in gen["lang_to_id"].items()}
    want = T.results(entries, 50257, lm, [(p.decode(), seqs[i], ts[i, :len(seqs[i])].tolist(), int(langs[i]))
                                          for i, p in enumerate(paths)])
    assert json.loads(text) == want


def cli(*args) -> int:
    argv = [b"mimizuku"] + [a.encode() for a in args]
    return L.lib().mz_cli(len(argv), (C.c_char_p * len(argv))(*argv))


def test_cli_arguments(tmp_path, capfd):
    assert cli("--help") == 0
    assert "usage: mimizuku --model DIR" in capfd.readouterr().out
    for args, what in [(["--bogus"], "unknown option --bogus"), (["a.wav"], "--model is required"),
                       (["--model"], "--model needs a value"), (["--model", str(tmp_path)], "no input files"),
                       (["--model", str(tmp_path), "a.wav"], "config.json: cannot read"),
                       (["--model", str(tmp_path), "--dir", str(tmp_path / "nope")], "cannot read the directory"),
                       (["--model", str(tmp_path), "--enc-attn", "cublas", "a.wav"], "fused encoder attention"),
                       (["--model", str(tmp_path), "--ref", "r.safetensors", "a.wav"], "not supported by this tool")]:
        assert cli(*args) == 1, args
        assert what in capfd.readouterr().err, args
    synth.write_model_dir(str(tmp_path), synth.TINY, {"x": np.zeros(1, np.float16)})
    (tmp_path / "bad.wav").write_bytes(b"not a wav")
    assert cli("--model", str(tmp_path), "--batch", "0", str(tmp_path / "bad.wav")) == 1
    assert "--batch: expected a positive integer, got 0" in capfd.readouterr().err
    assert cli("--model", str(tmp_path), "--dir", str(tmp_path), "--prefix", "bad") == 1
    assert "not a RIFF/WAVE file" in capfd.readouterr().err
