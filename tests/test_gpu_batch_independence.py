"""Batch independence at turbo widths (the batch API, src/transcribe.rs:104-167).

Every kernel on the path computes a clip (encoder, cross keys / values, timestamps) or a decoder row on its own, and
accumulates in an order that does not depend on the clips beside it (the products sum K in the same 64-wide steps
whatever tile shape the batch size selects). So a clip's language, tokens and token timestamps are the same bits
whether it is transcribed alone or in a batch: a property that holds at any batch size, checked here on six clips
(two encoder groups on two lanes) against three of them alone (one group, smaller product tiles), in both timestamp
modes, for graph replay against eager steps, and for encoder groups of 2 and of 6 against groups of 4. Turbo widths (d 1280, 20 heads, 4 decoder layers, 128 mels, the
51866-token vocabulary) with 2 encoder layers; random weights with non-zero biases and LayerNorm parameters.
"""
import numpy as np
import pytest

from mimizuku_amd import model, synth, transcribe

pytestmark = pytest.mark.gpu

G = synth.Geometry(d=1280, ff=5120, nh=20, enc_layers=2, dec_layers=4, n_mels=128, vocab=51866)
N, EG, MAX_NEW = 6, 4, 24


@pytest.fixture(scope="module")
def parts():
    W = synth.random_weights(G, seed=3, bias_std=0.02, ln_std=0.05)
    heads = synth.generation_config(synth.LARGE_V3_TURBO)["alignment_heads"]
    gen = synth.generation_config(G, align_heads=heads)
    dims = model.Dims(G.d, G.ff, G.nh, G.enc_layers, G.dec_layers, G.n_mels, G.vocab, G.max_t)
    gc = model.GenCfg.from_dict(gen, dims)
    ctx = model.Context(0)

    def engine(eg: int) -> model.Engine:
        e = model.Engine(ctx, dims, gc, N, eg)
        e.load(W)
        return e
    mel = synth.synthetic_mel(N, G.n_mels, seed=5)
    prompt = transcribe.Prompt(gc, "auto", "transcribe")
    yield engine, mel, prompt


@pytest.fixture(scope="module")
def setup(parts):
    engine, mel, prompt = parts
    e = engine(EG)
    yield e, mel, prompt
    e.close()


def same(a: transcribe.Decoded, b: transcribe.Decoded, what: str):
    assert a.lang == b.lang, what
    assert a.seq == b.seq, what
    np.testing.assert_array_equal(np.array(a.ts, np.float32), np.array(b.ts, np.float32), err_msg=what)


@pytest.mark.parametrize("half", [True, False])
def test_clip_alone_equals_clip_in_batch(setup, half):
    e, mel, prompt = setup
    batch, tm = transcribe.transcribe(e, mel, prompt, max_new=MAX_NEW, half_align=half)
    assert tm.steps > MAX_NEW // 2
    for c in (0, 3, 5):
        alone, _ = transcribe.transcribe(e, mel[c:c + 1], prompt, max_new=MAX_NEW, half_align=half)
        same(alone[0], batch[c], f"clip {c} half {half}")


def test_graph_replay_equals_eager_steps(setup):
    e, mel, prompt = setup
    graph, _ = transcribe.transcribe(e, mel, prompt, max_new=MAX_NEW, graph=True)
    eager, _ = transcribe.transcribe(e, mel, prompt, max_new=MAX_NEW, graph=False)
    for c in range(N):
        same(graph[c], eager[c], f"clip {c}")


def test_encoder_group_size_does_not_change_results(setup, parts):
    """The six clips encoded in groups of 2 (three groups over the two lanes) and in one group of 6 (one lane, larger
    products) give the same bits as in groups of 4."""
    e, mel, prompt = setup
    engine = parts[0]
    ref, _ = transcribe.transcribe(e, mel, prompt, max_new=MAX_NEW)
    for eg in (2, N):
        other = engine(eg)
        try:
            got, _ = transcribe.transcribe(other, mel, prompt, max_new=MAX_NEW)
        finally:
            other.close()
        for c in range(N):
            same(got[c], ref[c], f"clip {c}, groups of {eg}")
