"""mz_jump_times_device_noalloc, the timestamp entry point that allocates no device memory, against
mz_jump_times_device (which allocates its scratch per call): bit-identical times on two calls in a row, the second
smaller (the static scratch keeps the first call's contents), on a batch that needs several passes through the static
scratch, and a clip too large for the scratch refused with an error."""
import numpy as np
import pytest

from mimizuku_amd import _lib as L
from mimizuku_amd import model, transcribe

pytestmark = pytest.mark.gpu


def softmax_rows(rng, shape, scale=3.0):
    s = rng.standard_normal(shape, dtype=np.float32) * scale
    w = np.exp(s - s.max(-1, keepdims=True))
    return (w / w.sum(-1, keepdims=True)).astype(np.float32)


@pytest.fixture(scope="module")
def ctx():
    c = model.Context(0)
    yield c
    c.close()


@pytest.mark.parametrize("half", [True, False])
def test_noalloc_equals_allocating_entry_point(ctx, half):
    rng = np.random.default_rng(17 + half)
    heads, full = 6, 1500
    cases = [
        (32, 230),  # the benchmark's batch: 32 clips of up to 224 + a few rows
        (5, 60),    # then a smaller call (stale contents of the first call in the array)
        (70, 40),   # more clips than one pass takes (64)
        (20, 500),  # long clips: two passes for lack of room (about 5 MB of scratch each)
    ]
    for n, rmax in cases:
        rows = rng.integers(0, rmax + 1, size=n).astype(np.int32)
        rows[0] = rmax
        cols = rng.integers(1, full + 1, size=n).astype(np.int32)
        cols[1 % n] = full
        w = softmax_rows(rng, (n, rmax, heads, full))
        dw = ctx.upload_new(w)
        stride = rmax * heads * full
        ref = transcribe.jump_times_device(ctx, dw, stride, rows, cols, heads, full, 7, half)
        got = transcribe.jump_times_device_noalloc(ctx, dw, stride, rows, cols, heads, full, 7, half)
        for c in range(n):
            np.testing.assert_array_equal(got[c], ref[c], err_msg=f"case {n} x {rmax}, clip {c}")
        ctx.free(dw)


def test_noalloc_refuses_a_clip_beyond_its_scratch(ctx):
    heads, full = 6000, 1500  # column statistics alone: 2 x 6000 x 1500 x 4 bytes = 72 MB > 64 MiB
    w = np.full((1, heads, full), 1.0 / full, np.float32)
    dw = ctx.upload_new(w)
    with pytest.raises(L.MzError, match="static scratch"):
        transcribe.jump_times_device_noalloc(ctx, dw, heads * full, [1], [full], heads, full, 7, True)
    ctx.free(dw)


def test_noalloc_two_threads_on_one_context(ctx):
    """Two host threads calling the entry point on one context share the device's one static array: the library
    holds a per-device lock for each whole call, so every result equals the allocating entry point's."""
    import threading
    rng = np.random.default_rng(41)
    heads, full = 6, 1500
    jobs = []
    for t in range(2):
        n, rmax = (24, 200) if t == 0 else (9, 90)
        rows = rng.integers(1, rmax + 1, size=n).astype(np.int32)
        cols = rng.integers(1, full + 1, size=n).astype(np.int32)
        w = softmax_rows(rng, (n, rmax, heads, full))
        dw = ctx.upload_new(w)
        stride = rmax * heads * full
        ref = transcribe.jump_times_device(ctx, dw, stride, rows, cols, heads, full, 7, True)
        jobs.append((dw, stride, rows, cols, ref))
    results = [[None] * 4 for _ in range(2)]
    errors = []

    def run(t):
        dw, stride, rows, cols, _ = jobs[t]
        try:
            for k in range(4):
                results[t][k] = transcribe.jump_times_device_noalloc(ctx, dw, stride, rows, cols, heads, full, 7, True)
        except Exception as ex:  # reported below, in the main thread
            errors.append(ex)

    threads = [threading.Thread(target=run, args=(t,)) for t in range(2)]
    for th in threads:
        th.start()
    for th in threads:
        th.join(timeout=100)
    assert not any(th.is_alive() for th in threads), "a thread did not finish"
    assert not errors, errors
    for t in range(2):
        ref = jobs[t][4]
        for k in range(4):
            for c in range(len(ref)):
                np.testing.assert_array_equal(results[t][k][c], ref[c], err_msg=f"thread {t} call {k} clip {c}")
        ctx.free(jobs[t][0])
