"""GPU parity of the whole path (engine + transcription loop) on the Whisper-tiny geometry, against the oracle and
the golden vectors transformers wrote (tests/golden/*.npz).

* encoder: every layer checked layer-local — the oracle's layer applied to the engine's own fp32 input of that layer
  — at max-abs error <= 2e-3 x RMS; the conv stem and the final LayerNorm likewise;
* decoder: teacher-forced on the golden sequence, logits and alignment-head weights against the oracle at every
  step, and the greedy choice equal wherever the oracle's top-2 margin exceeds 1e-2;
* the batch API (graph replay) reproduces the golden token sequences and 20 ms-grid timestamps, and graph replay is
  bit-identical to eager steps.
"""
import os

import numpy as np
import pytest

from mimizuku_amd import _lib as L
from mimizuku_amd import model, synth, transcribe
from oracle import whisper_ref as R

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")
G = synth.TINY
TOL = 2e-3
MARGIN = 1e-2
PROMPT_EN = [50258, 50259, 50359, 50363]


def rel_err(got, ref):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    return np.abs(got - ref).max() / np.sqrt((ref ** 2).mean())


class Case:
    def __init__(self, name):
        self.name = name
        fx = np.load(os.path.join(GOLDEN, f"{name}.npz"))
        self.fx = fx
        self.W = synth.random_weights(G, seed=int(fx["seed"]), bias_std=float(fx["bias_std"]),
                                      ln_std=float(fx["ln_std"]))
        assert synth.weights_digest(self.W) == str(fx["weights_digest"])
        self.Wf = {k: v.astype(np.float32) for k, v in self.W.items()}
        self.n = int(fx["n_clips"])
        self.mel = synth.synthetic_mel(self.n, G.n_mels, seed=int(fx["mel_seed"]))
        self.gen = synth.generation_config(G)
        self.detect = bool(fx["detect"])
        self.seq = fx["sequences"]
        self.dims = model.Dims(G.d, G.ff, G.nh, G.enc_layers, G.dec_layers, G.n_mels, G.vocab, G.max_t)
        self.gc = model.GenCfg.from_dict(self.gen, self.dims)
        # the oracle teacher-forced on the golden sequence (equal to its own greedy run, pinned in test_oracle.py)
        self.ref = R.greedy(self.Wf, G, self.gen, self.mel, PROMPT_EN, self.seq.shape[1] - 4, detect=self.detect,
                            teacher=self.seq)

    def engine(self, ctx, bmax=None):
        e = model.Engine(ctx, self.dims, self.gc, bmax or self.n, self.n)
        e.load(self.W)
        return e


@pytest.fixture(scope="module")
def ctx():
    c = model.Context(0)
    yield c
    c.close()


@pytest.fixture(scope="module", params=["tiny_hfinit", "tiny_bias_detect"])
def case(request):
    return Case(request.param)


def test_encoder_layer_local(ctx, case):
    e = case.engine(ctx)
    e.set_trace(True)
    e.encode(case.mel, 0)
    tr = e.trace(case.n)  # [L][n][1500][d] inputs of every layer
    xl = e.read(L.BUF_ENC_X, np.float32, (case.n, 1500, G.d))  # residual after the last layer
    out = e.enc_out(case.n).astype(np.float32)
    W = case.Wf
    for c in range(case.n):
        m16 = case.mel[c].astype(np.float16).astype(np.float32)  # the engine takes the mel to fp16 first
        errs = [rel_err(tr[0, c], R.conv_stem(m16, W))]
        for i in range(G.enc_layers):
            nxt = tr[i + 1, c] if i + 1 < G.enc_layers else xl[c]
            errs.append(rel_err(nxt, R.encoder_layer(tr[i, c], W, i, G.nh)))
        errs.append(rel_err(out[c], R.layer_norm(xl[c], W["model.encoder.layer_norm.weight"],
                                                 W["model.encoder.layer_norm.bias"])))
        print(case.name, c, ["%.2e" % x for x in errs])
        assert max(errs) < TOL, errs
    e.close()


def test_decoder_teacher_forced(ctx, case):
    """Reset with the whole golden sequence as the prompt: every step then feeds the golden token, and the logits
    and alignment rows of each position are compared with the oracle's at that position."""
    e = case.engine(ctx)
    e.encode(case.mel, 0)
    seq = case.seq.astype(np.int32)
    T = seq.shape[1]
    e.reset(seq)
    sup = set(case.gen["suppress_tokens"])
    bsup = case.gen["begin_suppress_tokens"]
    worst = 0.0
    for p in range(T - 1):
        e.step(case.n, False, T)
        if p + 1 < 4:
            continue
        lg = e.logits()[:case.n]
        ref = case.ref["logits"][p + 1 - 4]
        worst = max(worst, rel_err(lg, ref))
        for b in range(case.n):
            first = p + 1 == 4
            if case.ref["margins"][p + 1 - 4][b] > MARGIN:
                assert R.choose(lg[b], sup, bsup, first, 50257, False) == int(seq[b, p + 1]), (p, b)
    print(case.name, "logits max-abs / RMS", worst)
    assert worst < 2e-2
    al = e.align()[:case.n, :T - 1].astype(np.float32)  # [n][rows][heads][1500]
    probs = case.ref["probs"]  # [n][rows][L][nh][1500]
    for s, (l, h) in enumerate(case.gen["alignment_heads"]):
        ref = probs[:, :T - 1, l, h]
        err = np.abs(al[:, :, s] - ref).max()
        assert err < 1e-3 * ref.max(), (s, err)
        np.testing.assert_allclose(al[:, :, s].sum(-1), 1.0, atol=3e-3)
    assert e.position() == T - 1
    e.close()


def test_decoder_layer_local(ctx, case):
    """Every decoder layer layer-local at every teacher-forced position: the oracle's layer applied to the engine's own
    fp32 residual entering it, with the engine's own (fp16) self-attention cache of the earlier positions and its
    cross keys / values, against the residual the engine produced, max-abs <= 2e-3 x RMS; the new cache rows
    against the oracle's k / v within fp16 rounding; the logits against the final LayerNorm and the tied LM head
    applied to the engine's own final residual, 2e-3 x RMS."""
    e = case.engine(ctx)
    e.set_trace(True)
    e.encode(case.mel, 0)
    seq = case.seq.astype(np.int32)
    T = seq.shape[1]
    e.reset(seq)
    n, nh, nl = case.n, G.nh, G.dec_layers
    xkv = e.xkv()[:n].astype(np.float32)
    worst = worst_kv = worst_lg = 0.0
    W = case.Wf
    for p in range(T - 1):
        e.step(n, False, T)
        tr = e.dec_trace()[:, :n]
        h = R.layer_norm(tr[nl], W["model.decoder.layer_norm.weight"], W["model.decoder.layer_norm.bias"])
        err = rel_err(e.logits()[:n], R.linear(h, W["model.decoder.embed_tokens.weight"]))
        worst_lg = max(worst_lg, err)
        assert err <= TOL, (p, "logits", err)
        kc, vc = e.self_kv()
        for i in range(nl):
            cache = [(kc[i, b, :, :p].astype(np.float32), vc[i, b, :, :p].astype(np.float32)) if p else (None, None)
                     for b in range(n)]
            cross = [(xkv[b, i, 0, :, :1500], xkv[b, i, 1, :, :1500]) for b in range(n)]
            out, k, v, _ = R.decoder_layer(tr[i], case.Wf, i, nh, cache, cross)
            err = rel_err(tr[i + 1], out)
            worst = max(worst, err)
            assert err <= TOL, (p, i, err)
            for got, ref in ((kc[i, :n, :, p], k), (vc[i, :n, :, p], v)):
                ref = ref.reshape(n, nh, 64)
                worst_kv = max(worst_kv, float(np.abs(got.astype(np.float32) - ref).max() / np.sqrt((ref ** 2).mean())))
    print(case.name, "decoder layer-local max-abs / RMS", worst, "new k/v", worst_kv, "LM head", worst_lg)
    assert worst_kv <= TOL
    e.close()


@pytest.mark.parametrize("half", [False, True])
def test_transcribe_matches_golden(ctx, case, half):
    """The batch API against transformers' greedy sequences and token timestamps: both timestamp modes (fp32
    arithmetic, and align.rs's fp16 roundings) give transformers' times on the 20 ms grid."""
    e = case.engine(ctx)
    p = transcribe.Prompt(e.gc, "auto" if case.detect else "en")
    out, tm = transcribe.transcribe(e, case.mel, p, max_new=case.seq.shape[1] - 4, half_align=half)
    for b, d in enumerate(out):
        if case.detect:
            assert d.lang == int(case.seq[b, 1])
        want = case.seq[b].tolist()
        # identical up to the first generating step whose oracle margin is within 1e-2 (where a different but
        # equally likely token is allowed and the rest of the sequence follows from it)
        low = [s for s, m in enumerate(case.ref["margins"][:, b]) if m <= MARGIN]
        upto = 4 + (low[0] if low else len(want))
        assert d.seq[:upto] == want[:upto], (b, d.seq, want)
        if not low:
            assert d.seq == want[:len(d.seq)]
            np.testing.assert_array_equal(np.array(d.ts, np.float32), case.fx["token_timestamps"][b][:len(d.ts)])
    assert tm.steps == case.seq.shape[1] - 1
    e.close()


def test_graph_replay_equals_eager(ctx, case):
    res = []
    for graph in (True, False):
        e = case.engine(ctx)
        p = transcribe.Prompt(e.gc, "auto" if case.detect else "en")
        out, _ = transcribe.transcribe(e, case.mel, p, graph=graph, max_new=20)
        res.append((out, e.logits(), e.align(), e.dec_x()))
        e.close()
    (o1, l1, a1, x1), (o2, l2, a2, x2) = res
    assert [d.seq for d in o1] == [d.seq for d in o2]
    assert [d.ts for d in o1] == [d.ts for d in o2]
    np.testing.assert_array_equal(l1, l2)
    np.testing.assert_array_equal(a1, a2)
    np.testing.assert_array_equal(x1, x2)


def test_submit_collect_is_transcribe(ctx, case):
    """mz_transcribe_submit + mz_transcribe_collect (the encoder half enqueued, then the decode half) return what
    mz_transcribe returns, bit for bit; one chunk at a time, with the protocol's errors; transcribe_all over the clips
    in chunks of one equals one call per clip."""
    e = case.engine(ctx)
    p = transcribe.Prompt(e.gc, "auto" if case.detect else "en")
    with pytest.raises(L.MzError, match="no chunk submitted"):
        transcribe.collect(e, case.n, p)
    ref, _ = transcribe.transcribe(e, case.mel, p, max_new=12)
    assert transcribe.submit(e, case.mel) == case.n
    with pytest.raises(L.MzError, match="a chunk is pending"):
        transcribe.submit(e, case.mel)
    with pytest.raises(L.MzError, match="not collected"):
        transcribe.transcribe(e, case.mel, p)
    with pytest.raises(L.MzError, match="the submitted chunk has"):
        transcribe.collect(e, case.n + 1, p)
    got, tm = transcribe.collect(e, case.n, p, max_new=12)
    assert [(d.lang, d.seq, d.ts) for d in got] == [(d.lang, d.seq, d.ts) for d in ref]
    assert tm.enc > 0 and tm.steps > 0
    e.close()
    e = model.Engine(ctx, case.dims, case.gc, 1, 1)
    e.load(case.W)
    one = [transcribe.transcribe(e, case.mel[c:c + 1], p, max_new=12)[0][0] for c in range(case.n)]
    allc, tm = transcribe.transcribe_all(e, case.mel, p, max_new=12)
    assert [(d.lang, d.seq, d.ts) for d in allc] == [(d.lang, d.seq, d.ts) for d in one]
    e.close()


def test_engine_from_model_dir_equals_put(ctx, case, tmp_path):
    """Engine.new reads the directory in the library (configs, mapped safetensors, F32 -> F16 on the host) and
    places the same bits as tensors handed over one by one: identical tokens, logits and alignment rows."""
    W32 = {k: v.astype(np.float32) for k, v in case.W.items()}  # the checkpoint in F32, converted by the library
    synth.write_model_dir(str(tmp_path), G, W32, case.gen)
    res = []
    for from_dir in (True, False):
        e = model.Engine.new(str(tmp_path), case.n, case.n, ctx=ctx) if from_dir else case.engine(ctx)
        assert e.dims == case.dims and e.gc == case.gc
        p = transcribe.Prompt(e.gc, "auto" if case.detect else "en")
        out, _ = transcribe.transcribe(e, case.mel, p, max_new=12)
        res.append(([d.seq for d in out], [d.ts for d in out], e.logits(), e.align()))
        e.close()
    (s1, t1, l1, a1), (s2, t2, l2, a2) = res
    assert s1 == s2 and t1 == t2
    np.testing.assert_array_equal(l1, l2)
    np.testing.assert_array_equal(a1, a2)


def test_step_beyond_the_cache_is_refused(ctx):
    case_dims = model.Dims(G.d, G.ff, G.nh, 1, 1, G.n_mels, G.vocab, 16)
    gen = synth.generation_config(G, align_heads=[[0, 0]])
    gc = model.GenCfg.from_dict(gen, case_dims)
    W = {k: v for k, v in synth.random_weights(synth.Geometry(G.d, G.ff, G.nh, 1, 1, G.n_mels, G.vocab, 16)).items()}
    e = model.Engine(ctx, case_dims, gc, 1, 1)
    e.load(W)
    e.encode(synth.synthetic_mel(1, G.n_mels), 0)
    e.reset([PROMPT_EN])
    for _ in range(15):
        e.step(1, False, 4)
    with pytest.raises(L.MzError, match="cache"):
        e.step(1, False, 4)
    assert e.position() == 15
    e.close()
