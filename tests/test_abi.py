"""CPU checks of the C ABI: the library loads, exports every declared symbol, fails cleanly without a device, and its
host helpers (fp16 conversion, DTW, token timestamps, config readers) match the reference's KATs and the oracle.
No GPU work is launched here."""
import os
import re

import numpy as np
import pytest

from mimizuku_amd import _lib as L
from mimizuku_amd import model, synth, transcribe
from oracle import whisper_ref as R

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "mimizuku.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(mz_[a-z0-9_]+)\s*\(", text)))


def test_header_constants_match_the_python_mirror():
    """Every buffer id, epilogue, data type and kernel class that the header defines has the same value in the Python
    mirror (a caller binding the header and these tests read the same buffers)."""
    defs = {k: int(v) for k, v in re.findall(r"#define MZ_([A-Z0-9_]+)\s+(\d+)", open(HEADER).read())}
    groups = [k for k in defs if k.startswith(("BUF_", "EPI_", "DT_"))]
    assert len(groups) >= 14 + 5 + 2
    for k in groups:
        assert getattr(L, k) == defs[k], k
    kinds = sorted((v, k) for k, v in defs.items() if k.startswith("K_"))
    assert [v for v, _ in kinds] == list(range(len(L.K_NAMES)))
    assert [k[2:].lower() for _, k in kinds] == L.K_NAMES


def test_library_exports_every_declared_function():
    lib = L.lib()
    names = declared_functions()
    assert len(names) > 40
    for n in names:
        assert hasattr(lib, n), n
    # and the Python binding declares a signature for each of them
    assert set(names) == set(L.SIGNATURES), set(names) ^ set(L.SIGNATURES)


def test_version_and_empty_error():
    assert b"gfx950" in L.lib().mz_version()


@pytest.mark.skipif(os.path.exists("/dev/kfd"), reason="checks the no-device path")
def test_init_without_device_is_a_clean_error():
    with pytest.raises(L.MzError, match="device"):
        model.Context()


def test_fp16_conversion_exhaustive():
    """src/gpu.rs:380-397: every binary16 pattern round-trips; RNE ties; overflow; subnormal ties."""
    lib = L.lib()
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    f = h.view(np.float16).astype(np.float32)
    for i in range(0, 65536, 1):
        x = float(f[i])
        y = lib.mz_h2f(int(h[i]))
        if np.isnan(x):
            assert np.isnan(y)
            assert np.isnan(lib.mz_h2f(lib.mz_f2h(y)))
        else:
            assert y == x, hex(i)
            assert lib.mz_f2h(y) == int(h[i]), hex(i)
    assert lib.mz_f2h(1.0 + 1.0 / 2048.0) == 0x3C00
    assert lib.mz_f2h(1.0 + 3.0 / 2048.0) == 0x3C02
    assert lib.mz_f2h(65520.0) == 0x7C00
    assert lib.mz_f2h(65519.0) == 0x7BFF
    assert lib.mz_f2h(2.0 ** -25) == 0
    assert lib.mz_f2h(3.0 * 2.0 ** -25) == 2
    assert lib.mz_h2f(lib.mz_f2h(0.1)) == 1638.0 / 16384.0


def test_fp16_conversion_matches_numpy_on_random_floats():
    lib = L.lib()
    rng = np.random.default_rng(0)
    x = np.concatenate([rng.standard_normal(3000) * s for s in (1e-6, 1e-3, 1, 1e3, 6e4)]).astype(np.float32)
    want = x.astype(np.float16).view(np.uint16)
    got = np.array([lib.mz_f2h(float(v)) for v in x], np.uint16)
    np.testing.assert_array_equal(got, want)


def test_dtw_kat_and_oracle():
    m = np.array([[-1.0 if (j // 2) == i else 1.0 for j in range(6)] for i in range(3)])
    text, time = transcribe.dtw(m)
    assert text.tolist() == [0, 0, 1, 1, 2, 2] and time.tolist() == [0, 1, 2, 3, 4, 5]
    rng = np.random.default_rng(1)
    for rows, cols in [(1, 1), (1, 9), (7, 3), (12, 40)]:
        m = rng.standard_normal((rows, cols))
        a, b = transcribe.dtw(m)
        c, d = R.dtw(m)
        np.testing.assert_array_equal(a, c)
        np.testing.assert_array_equal(b, d)


def test_jump_times_kat():
    """src/align.rs:122-139"""
    rows, full, cols = 4, 60, 40
    w = np.zeros((rows, 1, full), np.float32)
    for i in range(rows):
        w[i, 0, 10 * i:10 * i + 10] = 0.1
    for half in (True, False):
        t = transcribe.jump_times(w, cols, 7, half)
        assert np.all(np.abs(t - 0.2 * np.arange(rows)) < 0.03)
        assert transcribe.jump_times(w, 0, 7, half).tolist() == [0.0] * rows
        assert transcribe.jump_times(w[:1], cols, 7, half).tolist() == [0.0]


@pytest.mark.parametrize("half", [False, True])
def test_jump_times_match_oracle_on_softmax_weights(half):
    rng = np.random.default_rng(2 + half)
    for rows, heads, cols in [(5, 2, 30), (9, 6, 200), (3, 1, 2)]:
        s = rng.standard_normal((rows, heads, 64)) * 3
        w = np.exp(s - s.max(-1, keepdims=True))
        w = (w / w.sum(-1, keepdims=True)).astype(np.float16).astype(np.float32)
        np.testing.assert_array_equal(transcribe.jump_times(w, cols if cols <= 64 else 64, 7, half),
                                      R.jump_times(w, cols if cols <= 64 else 64, 7, half))


def align_rs_cost(w, cols, width, f64_sums=False):
    """src/align.rs:14-52 line by line with float32 scalars (the fp16 mode the reference always runs): sequential
    float sums over the rows, fp16 roundings of the mean, the deviation and the z-scores, a sorted window for the
    median, float sums over the heads. f64_sums takes the two column sums in float64 instead (the variant the
    fp16 mode must not be)."""
    f = np.float32
    rh = lambda x: f(np.float16(f(x)))  # noqa: E731
    rows, heads, _ = w.shape
    pad = width // 2
    avg = np.zeros((rows, cols), np.float32)
    for a in range(heads):
        z = np.zeros((rows, cols), np.float32)
        for j in range(cols):
            col = [f(w[i, a, j]) for i in range(rows)]
            if f64_sums:
                mean_f = f(sum(float(x) for x in col) / rows)
                var = f(sum(float(f(x - mean_f)) ** 2 for x in col) / rows)
            else:
                acc = f(0)
                for x in col:
                    acc = f(acc + x)
                mean_f = f(acc / f(rows))
                acc = f(0)
                for x in col:
                    d = f(x - mean_f)
                    acc = f(acc + f(d * d))
                var = f(acc / f(rows))
            mean, std = rh(mean_f), rh(np.sqrt(var))
            for i in range(rows):
                z[i, j] = rh(f(rh(f(col[i] - mean)) / std)) if std > 0 else f(0)
        for i in range(rows):
            for j in range(cols):
                if cols <= pad:
                    v = z[i, j]
                else:
                    idx = [abs(j + k - pad) for k in range(width)]
                    idx = [t if t < cols else 2 * (cols - 1) - t for t in idx]
                    v = sorted(z[i, t] for t in idx)[pad]
                avg[i, j] = f(avg[i, j] + v)
    return -np.array([[float(rh(f(avg[i, j] / f(heads)))) for j in range(cols)] for i in range(rows)])


def test_align_cost_is_align_rs_arithmetic():
    """The fp16 mode's cost, library and oracle, equals align.rs's own arithmetic bit for bit (brute force on small
    inputs), including a column built so that float32 sequential sums and float64 sums round the mean to different
    fp16 values: 4 + 2^-9 followed by three 2^-23 terms that a float32 running sum drops (mean 1 + 2^-11, an fp16
    tie, rounds to 1.0) while float64 keeps them (rounds up to 1 + 2^-10)."""
    rng = np.random.default_rng(5)
    for rows, heads, cols, width in [(4, 1, 3, 1), (5, 2, 9, 7), (3, 3, 2, 7), (6, 2, 20, 15), (1, 1, 5, 7)]:
        s = rng.standard_normal((rows, heads, cols + 3)) * 3
        w = np.exp(s - s.max(-1, keepdims=True))
        w = (w / w.sum(-1, keepdims=True)).astype(np.float32)
        if (rows, width) == (4, 1):
            w[:, 0, 0] = [4 + 2.0 ** -9, 2.0 ** -23, 2.0 ** -23, 2.0 ** -23]
        ref = align_rs_cost(w, cols, width)
        np.testing.assert_array_equal(R.align_cost(w, cols, width, half=True), ref)
        np.testing.assert_array_equal(transcribe.align_cost(w, cols, width, half=True), ref)
        np.testing.assert_array_equal(transcribe.align_cost(w, cols, width, half=False),
                                      R.align_cost(w, cols, width, half=False))
        if (rows, width) == (4, 1):
            assert not np.array_equal(align_rs_cost(w, cols, width, f64_sums=True)[:, 0], ref[:, 0])


def test_jump_times_of_the_golden_weights():
    fx = np.load(os.path.join(ROOT, "tests", "golden", "tiny_hfinit.npz"))
    w = fx["align_w"][0].transpose(1, 0, 2)[4:]
    np.testing.assert_array_equal(transcribe.jump_times(w, 1500, 7, half=False), fx["token_timestamps"][0][4:4 + len(w)])


def test_config_readers(tmp_path):
    g = synth.TINY
    synth.write_model_dir(str(tmp_path), g, {"x": np.zeros(1, np.float16)})
    d = model.Dims.load(str(tmp_path))
    assert (d.d, d.nh, d.vocab, d.max_t) == (384, 6, 51865, 448)
    gc = model.GenCfg.load(str(tmp_path), d)
    assert gc.sot == 50258 and gc.eos == 50257 and gc.align_heads[0] == (2, 2)
    assert gc.lang_token("ja") == 50266 and gc.lang_code(50259) == "en"
    p = transcribe.Prompt(gc, "en", "transcribe")
    assert p.tokens(p.lang) == [50258, 50259, 50359, 50363] and not p.detect()
    assert transcribe.Prompt(gc).detect()
    with pytest.raises(L.MzError):
        transcribe.Prompt(gc, "xx")
    bad = synth.generation_config(g)
    bad["alignment_heads"] = [[9, 0]]
    with pytest.raises(L.MzError):
        model.GenCfg.from_dict(bad, d)


def test_scratch_bytes_scales_with_batch():
    d = model.Dims(1280, 5120, 20, 32, 32, 128, 51866, 448)
    a = model.scratch_bytes(d, 10, 32, 8)
    b = model.scratch_bytes(d, 10, 16, 8)
    assert a > b > 0
    # the cross k/v cache dominates the decoder's share: 32 rows x 32 layers x 2 x 20 heads x 1536 x 64 x 2 bytes
    assert a - b >= 16 * 32 * 2 * 20 * 1536 * 64 * 2
