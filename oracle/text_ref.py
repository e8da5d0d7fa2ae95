"""CPU oracle for the text side — TEST INFRASTRUCTURE ONLY.

Only tests/ may import this module, and only to check results. Nothing in the mimizuku_amd package imports it.

A Python restatement of the reference's tokenizer decoding (src/tok.rs: GPT-2's byte table, decode with the clean-up
of spaces, whole-character pieces with times) and of the CLI's JSON result (src/main.rs:97-138). Pinned by the
reference's KATs (tok.rs:87-122), which tests/test_text.py runs against both this module and the library, and by
GPT-2's published byte table (bytes_to_unicode in openai/gpt-2 encoder.py, restated independently below).
"""
from __future__ import annotations

import json


def bytes_to_unicode() -> dict[int, str]:
    """GPT-2's byte -> printable character table (openai/gpt-2 src/encoder.py, bytes_to_unicode)."""
    bs = list(range(ord("!"), ord("~") + 1)) + list(range(ord("¡"), ord("¬") + 1)) + list(range(ord("®"), ord("ÿ") + 1))
    cs = bs[:]
    n = 0
    for b in range(256):
        if b not in bs:
            bs.append(b)
            cs.append(256 + n)
            n += 1
    return dict(zip(bs, map(chr, cs)))


CLEANUP = [(" .", "."), (" ?", "?"), (" !", "!"), (" ,", ","), (" ' ", "'"), (" n't", "n't"), (" 'm", "'m"),
           (" 's", "'s"), (" 've", "'ve"), (" 're", "'re")]


def decode(table: list[bytes], ids) -> str:
    """Tok::decode (tok.rs:47-57)."""
    b = b"".join(table[i] for i in ids if 0 <= i < len(table))
    s = b.decode("utf-8", errors="replace")
    for a, r in CLEANUP:
        s = s.replace(a, r)
    return s


def _utf8_state(b: bytes) -> int:
    """0 valid, 1 incomplete at the end only, 2 invalid."""
    try:
        b.decode("utf-8")
        return 0
    except UnicodeDecodeError as e:
        return 1 if e.reason == "unexpected end of data" else 2


def pieces(table: list[bytes], ids, ts, eos: int):
    """Tok::pieces (tok.rs:63-86): [(text, start, end)]."""
    out, buf, by, t0 = [], [], b"", 0.0
    for i, (tok, t) in enumerate(zip(ids, ts)):
        if tok >= eos:
            continue
        if not buf:
            t0 = t
        buf.append(tok)
        by += table[tok] if 0 <= tok < len(table) else b""
        if _utf8_state(by) != 1:
            out.append((decode(table, buf), t0, ts[i + 1] if i + 1 < len(ts) else t))
            buf, by = [], b""
    if buf:
        out.append((decode(table, buf), t0, ts[-1] if len(ts) else t0))
    return out


def json_time(x) -> str:
    """Python's round(x, 2) as json.dumps prints it (main.rs:113-117)."""
    return json.dumps(round(float(x), 2))


def results(table: list[bytes], eos: int, langs_map: dict, clips) -> dict:
    """to_json (main.rs:121-138) as a dict: clips = [(path, seq, ts, lang_token)]; langs_map token -> code ({}
    for an English-only model)."""
    out = {}
    for path, seq, ts, lang in clips:
        words = [[w, round(float(a), 2), round(float(b), 2)] for w, a, b in pieces(table, seq, ts, eos)]
        text = decode(table, [t for t in seq if t < eos])
        out[path] = {"language": "en" if not langs_map else langs_map.get(lang, ""), "text": text, "words": words}
    return out
