"""CPU checks of the library's model-directory readers against the reference's KATs: the strict JSON parser
(src/json.rs:222-266), the safetensors reader (src/st.rs:197-219), and the config readers (Dims::load and
GenCfg::load, src/model.rs:33-146) against their Python restatement in mimizuku_amd.model on the same files.
No GPU work is launched here."""
import ctypes as C
import json
import os
import struct

import numpy as np
import pytest

from mimizuku_amd import _lib as L
from mimizuku_amd import model, synth


def json_ok(text: bytes) -> bool:
    return L.lib().mz_json_check(text, len(text)) == 0


def st_file(header: str, data: bytes) -> bytes:
    """st.rs:191-196: little-endian header length, the JSON header, the data."""
    h = header.encode()
    return struct.pack("<Q", len(h)) + h + data


class St:
    def __init__(self, path):
        self.h = C.c_void_p()
        L.check(L.lib().mz_st_open(str(path).encode(), C.byref(self.h)))

    def __del__(self):
        if self.h:
            L.lib().mz_st_close(self.h)

    def names(self):
        n = C.c_int()
        L.check(L.lib().mz_st_count(self.h, C.byref(n)))
        return [self.info(i)[0] for i in range(n.value)]

    def info(self, i):
        name, dt, nd, shp, data, nb = C.c_char_p(), C.c_char_p(), C.c_int(), C.POINTER(C.c_int64)(), C.c_void_p(), \
            C.c_uint64()
        L.check(L.lib().mz_st_info(self.h, i, C.byref(name), C.byref(dt), C.byref(nd), C.byref(shp), C.byref(data),
                                   C.byref(nb)))
        raw = C.string_at(data.value, nb.value) if nb.value else b""
        return name.value.decode(), dt.value.decode(), tuple(shp[k] for k in range(nd.value)), raw

    def get(self, name):
        i = C.c_int()
        L.check(L.lib().mz_st_find(self.h, name.encode(), C.byref(i)))
        return self.info(i.value)

    def meta(self, key):
        v = C.c_char_p()
        L.check(L.lib().mz_st_meta(self.h, key.encode(), C.byref(v)))
        return v.value.decode()


# ---------------------------------------------------------------- JSON (src/json.rs:222-266)

def test_json_values_through_the_safetensors_header(tmp_path):
    """json_values: escapes, \\u00e9, a surrogate pair and \\r arrive as UTF-8; [0, 7] reads as integers while
    [1, 2.5, -3e2] does not; nested objects and literals parse."""
    hdr = (r'{"__metadata__": {"b": "x\"é😀\r", "u": "\ud800A", "n": null},'
           r' "t": {"dtype": "U8", "shape": [0, 7], "data_offsets": [0, 0], "extra": {"c": true, "d": null, "e": {}}}}')
    p = tmp_path / "v.safetensors"
    p.write_bytes(st_file(hdr, b""))
    f = St(p)
    assert f.meta("b") == "x\"é\U0001F600\r"
    # json_unpaired_surrogate_keeps_what_follows
    assert f.meta("u") == "�A"
    assert f.meta("n") == ""  # a non-string metadata value reads as empty (st.rs:110-114)
    assert f.get("t")[:3] == ("t", "U8", (0, 7))
    bad = hdr.replace("[0, 7]", "[1, 2.5, -3e2]")
    p.write_bytes(st_file(bad, b""))
    with pytest.raises(L.MzError, match="shape of t"):
        St(p)


@pytest.mark.parametrize("text", [b"{", b"[1,", b'{"a" 1}', b'"abc', b"[1] x", b"tru", b'"\\u12"', b"-", b"", b"01",
                                  b"1.", b".5", b"1e", b"+1", b"1e999", b'"\\q"', b'"a\tb"', b'"\\u+041"'])
def test_json_malformed_is_an_error(text):
    assert not json_ok(text)


def test_json_depth_limit_and_valid_forms():
    assert not json_ok(b"[" * 1000 + b"]" * 1000)
    assert json_ok(b"[" * 64 + b"]" * 64)  # 64 levels below the top value: the limit itself
    assert not json_ok(b"[" * 66 + b"]" * 66)
    for t in [b" {\"a\": [1, 2.5, -3e2], \"c\": true, \"d\": null, \"e\": {}} ", b"-0", b"0.5e+3", b"[0, 7]",
              b'"\\/\\b\\f\\n\\r\\t"', "\"é😀\"".encode()]:
        assert json_ok(t), t
    assert not json_ok(b'"\xff"')  # a string that is not UTF-8 (String::from_utf8 fails, json.rs:112)
    assert not json_ok(b'"\xed\xa0\x80"')  # an encoded surrogate is not UTF-8 either


# ---------------------------------------------------------------- safetensors (src/st.rs:188-219)

def test_safetensors_checks_offsets(tmp_path):
    p = tmp_path / "t.safetensors"
    p.write_bytes(st_file('{"x":{"dtype":"F32","shape":[2],"data_offsets":[0,8]}}', bytes([0, 0, 128, 63, 0, 0, 0, 64])))
    name, dt, shape, raw = St(p).get("x")
    assert (name, dt, shape) == ("x", "F32", (2,))
    assert list(np.frombuffer(raw, "<f4")) == [1.0, 2.0]
    for bad in [
        st_file('{"x":{"dtype":"F32","shape":[2],"data_offsets":[0,16]}}', bytes(8)),
        st_file('{"x":{"dtype":"F32","shape":[3],"data_offsets":[0,8]}}', bytes(8)),
        st_file('{"x":{"dtype":"F32","shape":[2],"data_offsets":[8,0]}}', bytes(8)),
        st_file('{"x":{"dtype":"F32","shape":[2,"a"],"data_offsets":[0,8]}}', bytes(8)),
        st_file('{"x":{"dtype":"F32","shape":[2],"data_offsets":[0,8]},"y":{"dtype":"F32","shape":[1],'
                '"data_offsets":[4,8]}}', bytes(8)),
        bytes([255] * 12),
        bytes([1, 2]),
    ]:
        p.write_bytes(bad)
        with pytest.raises(L.MzError):
            St(p)


def test_safetensors_more_header_errors(tmp_path):
    p = tmp_path / "t.safetensors"
    ok = '{"x":{"dtype":"F16","shape":[2],"data_offsets":[0,4]}}'
    for hdr, what in [('["x"]', "not an object"), ('{"x":{"dtype":"Q4","shape":[1],"data_offsets":[0,1]}}', "offsets"),
                      ('{"x":{"shape":[1],"data_offsets":[0,2]}}', "dtype"),
                      ('{"x":{"dtype":"F16","shape":[2]}}', "offsets"),
                      ('{"x":{"dtype":"F16","shape":[2],"data_offsets":[0,4]},'
                       '"x":{"dtype":"F16","shape":[2],"data_offsets":[4,8]}}', "twice")]:
        p.write_bytes(st_file(hdr, bytes(8)))
        with pytest.raises(L.MzError, match=what):
            St(p)
    p.write_bytes(st_file(ok, bytes(4))[:-1])  # data cut short
    with pytest.raises(L.MzError, match="offsets"):
        St(p)
    with pytest.raises(L.MzError, match="cannot open"):
        St(tmp_path / "missing.safetensors")


def test_safetensors_matches_the_python_library(tmp_path):
    """A checkpoint written by the safetensors package: the same names, dtypes, shapes and bytes, header order."""
    from safetensors.numpy import save_file
    rng = np.random.default_rng(0)
    w = {"a.weight": rng.standard_normal((3, 5)).astype(np.float32), "b": rng.standard_normal(7).astype(np.float16),
         "c.idx": np.arange(6, dtype=np.int32).reshape(2, 3), "z": np.zeros((0, 4), np.float32)}
    p = tmp_path / "m.safetensors"
    save_file(w, str(p), metadata={"format": "np"})
    f = St(p)
    assert sorted(f.names()) == sorted(w)
    for k, a in w.items():
        name, dt, shape, raw = f.get(k)
        assert shape == a.shape and dt == {np.float32: "F32", np.float16: "F16", np.int32: "I32"}[a.dtype.type]
        np.testing.assert_array_equal(np.frombuffer(raw, a.dtype).reshape(a.shape), a)
    assert f.meta("format") == "np"


# ---------------------------------------------------------------- Dims / GenCfg (src/model.rs:33-146)

@pytest.mark.parametrize("geom", ["TINY", "LARGE_V3_TURBO", "LARGE_V3"])
def test_model_dir_matches_the_python_reading(tmp_path, geom):
    g = getattr(synth, geom)
    synth.write_model_dir(str(tmp_path), g, {"x": np.zeros(1, np.float16)})
    md = model.ModelDir(str(tmp_path))
    assert md.dims == model.Dims(g.d, g.ff, g.nh, g.enc_layers, g.dec_layers, g.n_mels, g.vocab, 448)
    gen = json.load(open(tmp_path / "generation_config.json"))
    assert md.gencfg == model.GenCfg.from_dict(gen, md.dims)
    assert md.gencfg.tasks == list(gen["task_to_id"].items()) and len(md.gencfg.langs) == len(gen["lang_to_id"])


def write_dir(tmp_path, cfg_patch=None, gen_patch=None, g=synth.TINY):
    synth.write_model_dir(str(tmp_path), g, {"x": np.zeros(1, np.float16)})
    if cfg_patch:
        c = json.load(open(tmp_path / "config.json"))
        c.update(cfg_patch)
        json.dump(c, open(tmp_path / "config.json", "w"))
    if gen_patch:
        j = json.load(open(tmp_path / "generation_config.json"))
        for k, v in gen_patch.items():
            if v is None:
                j.pop(k, None)
            else:
                j[k] = v
        json.dump(j, open(tmp_path / "generation_config.json", "w"))
    return str(tmp_path)


@pytest.mark.parametrize("patch,what", [
    ({"max_target_positions": 8}, "unsupported shape"),
    ({"max_target_positions": 449}, "unsupported shape"),
    ({"d_model": 448, "encoder_attention_heads": 7, "decoder_attention_heads": 7}, "unsupported shape"),
    ({"decoder_attention_heads": 3}, "64-wide heads"),
    ({"decoder_ffn_dim": 1024}, "equal encoder/decoder"),
    ({"max_source_positions": 1000}, "unsupported shape"),
    ({"encoder_layers": 65}, "unsupported shape"),
    ({"vocab_size": 0}, "vocab_size missing or out of range"),
    ({"d_model": 384.5}, "d_model missing or out of range"),
    ({"num_mel_bins": "80"}, "num_mel_bins missing or out of range"),
])
def test_config_json_checks(tmp_path, patch, what):
    with pytest.raises(L.MzError, match=what):
        model.ModelDir(write_dir(tmp_path, cfg_patch=patch))


@pytest.mark.parametrize("patch,what", [
    ({"alignment_heads": [[9, 0]]}, "pairs within the model"),
    ({"alignment_heads": [[2, 2], [2, 2]]}, "duplicates"),
    ({"alignment_heads": []}, "empty"),
    ({"alignment_heads": {"a": 1}}, "not a list"),
    ({"begin_suppress_tokens": [220, 50257, 1]}, "more than two"),
    ({"lang_to_id": None}, "needs lang_to_id"),
    ({"eos_token_id": 51865}, "eos_token_id missing or not a token id"),
    ({"suppress_tokens": [1, -2]}, "suppress_tokens has an invalid token id"),
    ({"task_to_id": [1]}, "task_to_id is not an object"),
    ({"lang_to_id": {"<|en|>": 99999}}, "is not a token id"),
])
def test_generation_config_checks(tmp_path, patch, what):
    with pytest.raises(L.MzError, match=what):
        model.ModelDir(write_dir(tmp_path, gen_patch=patch))


def test_generation_config_defaults(tmp_path):
    """No alignment_heads: every head of the second half of the decoder layers; an English-only model has no
    languages (is_multilingual false) and needs no lang_to_id."""
    md = model.ModelDir(write_dir(tmp_path, gen_patch={"alignment_heads": None, "is_multilingual": False,
                                                       "lang_to_id": None}))
    assert md.gencfg.align_heads == [(l, h) for l in (2, 3) for h in range(6)]
    assert md.gencfg.langs == []
    assert model.GenCfg.load(str(tmp_path)) == md.gencfg and model.Dims.load(str(tmp_path)) == md.dims
