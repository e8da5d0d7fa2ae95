"""Chunked transcription as a pipeline: the reference's loop over the inputs in chunks of bmax clips
(src/main.rs:195-200) with chunk i + 1's encoder enqueued before chunk i decodes, on two streams restricted to 3/4 of
the CUs (hipExtStreamCreateWithCUMask), filling a second set of cross keys/values beside chunk i's decode.

SKIPPED: the library does not have this path. Its first GPU run stalled in the first test below (nothing printed for
180 s, the run killed, the GPU still answering), and reading the code showed no wait that could not be satisfied in
the order the host enqueued it. Without a cause that can be shown, the path was taken out: mz_transcribe_submit
refuses a second pending chunk, and transcribe_all runs the chunks one after the other. These tests state what the
path must do and stay skipped until it comes back with a shown cause and fix.

* On the golden tiny case, three copies of the clip in chunks of 2 and 1 give transformers' sequence and timestamps.
* At the large-v3-turbo widths (d 1280, 20 heads, 128 mels, 51,866 ids; 4 + 4 layers), 20 ragged clips in chunks of
  8, 8 and 4 give the same tokens, timestamps and languages, bit for bit, as one mz_transcribe per chunk.
* The protocol's errors with two chunks pending.
"""
import os

import numpy as np
import pytest

from mimizuku_amd import _lib as L
from mimizuku_amd import model, synth, transcribe

pytestmark = [pytest.mark.gpu, pytest.mark.skip(reason="pipelined chunks are not in the library: their first GPU run "
                                                    "stalled with no cause shown (module docstring)")]

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")
TINY = synth.TINY


@pytest.fixture(scope="module")
def ctx():
    c = model.Context(0)
    yield c
    c.close()


def engine(ctx, g, W, bmax, eg, seed_gen=None):
    gen = synth.generation_config(g)
    dims = model.Dims(g.d, g.ff, g.nh, g.enc_layers, g.dec_layers, g.n_mels, g.vocab, g.max_t)
    e = model.Engine(ctx, dims, model.GenCfg.from_dict(gen, dims), bmax, eg)
    e.load(W)
    return e


def test_chunks_of_the_golden_case(ctx):
    """Three copies of the golden clip in chunks of 2 and 1: every copy gives transformers' sequence and timestamps
    (the oracle's top-2 margin on this clip is >= 0.0135 at every step, so greedy decoding has one answer)."""
    fx = np.load(os.path.join(GOLDEN, "tiny_hfinit.npz"))
    W = synth.random_weights(TINY, seed=int(fx["seed"]), bias_std=float(fx["bias_std"]), ln_std=float(fx["ln_std"]))
    assert synth.weights_digest(W) == str(fx["weights_digest"])
    mel = np.repeat(synth.synthetic_mel(1, TINY.n_mels, seed=int(fx["mel_seed"])), 3, axis=0)
    max_new = fx["sequences"].shape[1] - 4
    e = engine(ctx, TINY, W, 2, 1)
    p = transcribe.Prompt(e.gc, "en")
    for half in (True, False):
        out, tm = transcribe.transcribe_all(e, mel, p, max_new=max_new, half_align=half)
        assert len(out) == 3 and tm.steps == 2 * (fx["sequences"].shape[1] - 1)
        for d in out:
            assert d.seq == fx["sequences"][0].tolist()
            np.testing.assert_array_equal(np.array(d.ts, np.float32), fx["token_timestamps"][0])
    e.close()


def test_pipeline_equals_one_call_per_chunk_at_turbo_widths(ctx):
    g = synth.Geometry(d=1280, ff=5120, nh=20, enc_layers=4, dec_layers=4, n_mels=128, vocab=51866)
    W = synth.random_weights(g, seed=21, bias_std=0.02, ln_std=0.1)
    n, bmax, eg = 20, 8, 4
    mel = synth.synthetic_mel(n, g.n_mels, seed=22)
    frames = np.random.default_rng(23).integers(200, 3001, size=n).astype(np.int32)
    e = engine(ctx, g, W, bmax, eg)
    p = transcribe.Prompt(e.gc, "auto")
    piped, tp = transcribe.transcribe_all(e, mel, p, frames=frames, max_new=24)
    one = []
    for c0 in range(0, n, bmax):
        o, _ = transcribe.transcribe(e, mel[c0:c0 + bmax], p, frames=frames[c0:c0 + bmax], max_new=24)
        one += o
    # and again through the device-resident entry points, the pipeline's second set now in use for chunk 2
    dmel = ctx.upload_new(mel)
    dev, _ = transcribe.transcribe_all(e, dmel, p, frames=frames, max_new=24, n=n)
    e.close()
    assert len(piped) == len(one) == len(dev) == n
    for c in range(n):
        assert (piped[c].lang, piped[c].seq, piped[c].ts) == (one[c].lang, one[c].seq, one[c].ts), c
        assert (dev[c].lang, dev[c].seq, dev[c].ts) == (one[c].lang, one[c].seq, one[c].ts), c
    assert tp.steps > 0
    print("turbo widths, 20 clips in chunks of 8: pipelined == one call per chunk; steps", tp.steps,
          "enc wait %.1f ms dec %.1f ms" % (tp.enc * 1e3, tp.dec * 1e3))


def test_protocol_errors(ctx):
    g = synth.Geometry(d=384, ff=1536, nh=6, enc_layers=1, dec_layers=1, n_mels=80, vocab=51865)
    W = synth.random_weights(g, seed=3)
    e = engine(ctx, g, W, 2, 2)
    p = transcribe.Prompt(e.gc, "en")
    mel = synth.synthetic_mel(2, g.n_mels, seed=4)
    with pytest.raises(L.MzError, match="no chunk submitted"):
        transcribe.collect(e, 2, p)
    transcribe.submit(e, mel)
    transcribe.submit(e, mel[:1])
    with pytest.raises(L.MzError, match="two chunks"):
        transcribe.submit(e, mel)
    with pytest.raises(L.MzError, match="not collected"):
        transcribe.transcribe(e, mel, p)
    with pytest.raises(L.MzError, match="oldest submitted chunk has 2"):
        transcribe.collect(e, 1, p)
    a, _ = transcribe.collect(e, 2, p, max_new=6)
    b, _ = transcribe.collect(e, 1, p, max_new=6)
    c, _ = transcribe.transcribe(e, mel, p, max_new=6)
    assert [d.seq for d in a] == [d.seq for d in c] and b[0].seq == c[0].seq
    e.close()
