"""Large-v3 end to end at its benchmark shape: 32 clips x 30 s, encoder groups of 8, language detection, greedy
decoding of up to 224 tokens by graph replay, token timestamps (the batch API, src/transcribe.rs:104-167, as
src/main.rs:195-200 drives it with --batch 32 --enc-group 8).

No oracle finishes this whole workload on the host within a test, so the full-size run is checked through properties
that hold at any size, and the oracle checks a subsample of it layer-local:

* tokens: the prompt kept, every token within the vocabulary, no suppressed token generated, no begin-suppressed
  token at the first generated position, nothing after an eos, at most 224 generated tokens;
* encoder groups: the batch API runs two groups at once on two streams; each clip's cross keys / values of the first
  and last decoder layer are bit-equal to those of its group encoded again alone on the engine's stream;
* alignment rows of every fed position: finite, non-negative, each summing to 1;
* timestamps: zero over the prompt, non-decreasing, within the clip, the last token repeating the one before, and
  bit-equal to the host routine (mz_jump_times) on the downloaded alignment rows;
* the oracle: the conv stem and encoder layers 0, 16 and 31 of one clip layer-local; decoder layers 0, 15 and 31 of
  two rows layer-local at two teacher-forced positions of their own transcription (max-abs error <= 2e-3 x RMS); and
  for every row at every teacher-forced generated position (12 per row), the LM head layer-local (the final LayerNorm
  and the tied head on the engine's own final residual, <= 2e-3 x RMS) and the transcription's token equal to the
  oracle's choice on those logits wherever the oracle's top-2 margin exceeds 1e-2.
"""
import inspect

import numpy as np
import pytest

from mimizuku_amd import _lib as L
from mimizuku_amd import model, synth, transcribe
from oracle import whisper_ref as R

pytestmark = pytest.mark.gpu

G = synth.LARGE_V3
B, EG, MAX_NEW, NP = 32, 8, 224, 4
TPAD, TENC = 1536, 1500
KEEP = [0, 9, 18, 27, 31]  # clips whose alignment rows are downloaded
HALF = inspect.signature(transcribe.transcribe).parameters["half_align"].default  # the product's timestamp mode


def rel_err(got, ref):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    return np.abs(got - ref).max() / np.sqrt((ref ** 2).mean())


@pytest.fixture(scope="module")
def run(large_v3_weights):
    W = large_v3_weights
    gen = synth.generation_config(G)
    dims = model.Dims(G.d, G.ff, G.nh, G.enc_layers, G.dec_layers, G.n_mels, G.vocab, G.max_t)
    gc = model.GenCfg.from_dict(gen, dims)
    ctx = model.Context(0)
    e = model.Engine(ctx, dims, gc, B, EG)
    e.load(W)
    mel = synth.synthetic_mel(B, G.n_mels, seed=2)
    prompt = transcribe.Prompt(gc, "auto", "transcribe")
    out, tm = transcribe.transcribe(e, mel, prompt, max_new=MAX_NEW)
    print(f"large-v3 end to end: encoder {tm.enc * 1e3:.1f} ms, decoder {tm.dec * 1e3:.1f} ms for {tm.steps} steps, "
          f"timestamps {tm.post * 1e3:.1f} ms", flush=True)
    na = len(gen["alignment_heads"])
    row = G.max_t * na * TENC * 4
    align = {c: e.read(L.BUF_ALIGN, np.float32, (G.max_t, na, TENC), c * row) for c in KEEP}
    yield dict(W=W, gen=gen, gc=gc, ctx=ctx, e=e, mel=mel, out=out, tm=tm, align=align, na=na)
    e.close()
    ctx.close()


def test_tokens(run):
    gen, gc, out, tm = run["gen"], run["gc"], run["out"], run["tm"]
    sup, bsup, eos = set(gen["suppress_tokens"]), set(gen["begin_suppress_tokens"]), gen["eos_token_id"]
    langs = {t for _, t in gc.langs}
    assert tm.steps <= 1 + NP - 1 + MAX_NEW
    for c, d in enumerate(out):
        s = d.seq
        assert s[0] == gc.sot and s[1] == d.lang and d.lang in langs and s[3] == gc.no_timestamps, (c, s[:4])
        assert s[2] == dict(gc.tasks)["transcribe"]
        g = s[NP:]
        assert 1 <= len(g) <= MAX_NEW, (c, len(g))
        assert all(0 <= t < G.vocab for t in g)
        assert not sup & set(g), (c, sup & set(g))
        assert g[0] not in bsup
        assert eos not in g[:-1], c


def test_alignment_rows(run):
    for c, a in run["align"].items():
        n = len(run["out"][c].seq)
        rows = a[:n - 1]  # every fed position wrote its row
        assert np.isfinite(rows).all() and (rows >= 0).all(), c
        np.testing.assert_allclose(rows.sum(-1), 1.0, atol=1e-4)


def test_timestamps(run):
    for c, d in enumerate(run["out"]):
        ts, n = np.array(d.ts, np.float32), len(d.seq)
        assert not ts[:NP].any()
        gen_ts = ts[NP:n - 1]
        assert (np.diff(gen_ts) >= 0).all() and gen_ts.min() >= 0 and gen_ts.max() <= 30.0, c
        assert ts[n - 1] == ts[n - 2]
        if c in run["align"]:
            w = np.ascontiguousarray(run["align"][c][NP:n - 1])  # [rows][heads][1500]
            np.testing.assert_array_equal(gen_ts, transcribe.jump_times(w, TENC, 7, HALF))


def test_encoder_groups_are_independent(run):
    e, mel = run["e"], run["mel"]
    nl, nh = G.dec_layers, G.nh
    tile = 2 * nh * TPAD * 64  # halves of one (clip, layer): k and v of every head

    def layers():
        return {(c, l): e.read(L.BUF_XKV, np.float16, (tile,), ((c * nl + l) * tile) * 2)
                for c in range(B) for l in (0, nl - 1)}
    before = layers()
    for g0 in range(0, B, EG):
        e.encode(mel[g0:g0 + EG], g0)
    after = layers()
    for k in before:
        assert np.array_equal(before[k], after[k]), k


def test_oracle_subsample_layer_local(run):
    W, e, mel, out = run["W"], run["e"], run["mel"], run["out"]
    gen = run["gen"]
    d, nl, nh = G.d, G.dec_layers, G.nh
    f32 = lambda keys: {k: W[k].astype(np.float32) for k in keys}  # noqa: E731

    # encoder: clip 13 (group 1, clip 5) through the conv stem and layers 0, 16 and 31
    c, g0 = 5, 8
    enc_layers = (0, 16, 31)
    We = f32([k for k in W if k.startswith("model.encoder.") and
              (not k.startswith("model.encoder.layers.") or int(k.split(".")[3]) in enc_layers)])
    e.set_trace(True)
    e.encode(mel[g0:g0 + EG], g0)
    plane = TENC * d * 4

    def trace(l):
        return e.read(L.BUF_TRACE, np.float32, (TENC, d), (l * EG + c) * plane)
    xl = e.read(L.BUF_ENC_X, np.float32, (TENC, d), c * plane)
    errs = [rel_err(trace(0), R.conv_stem(mel[g0 + c].astype(np.float16).astype(np.float32), We))]
    for l in enc_layers:
        nxt = trace(l + 1) if l + 1 < G.enc_layers else xl
        errs.append(rel_err(nxt, R.encoder_layer(trace(l), We, l, nh)))
    print("large-v3 e2e, clip 13: conv stem, encoder layers 0 / 16 / 31:", ["%.2e" % x for x in errs])
    assert max(errs) <= 2e-3, errs
    del We

    # decoder: every row teacher-forced on its own transcription (all 32 rows stepped eagerly); rows 3 and 20
    # through decoder layers 0, 15 and 31 at the last two positions
    rows, T, dec_layers = [3, 20], NP + 12, (0, 15, 31)
    Wd = f32([k for k in W if k.startswith("model.decoder.") and
              (not k.startswith("model.decoder.layers.") or int(k.split(".")[3]) in dec_layers)])
    seqs = np.array([(s.seq + [gen["eos_token_id"]] * T)[:T] for s in out], np.int32)
    e.reset(seqs)
    tile = 2 * nh * TPAD * 64
    cross = {(l, r): e.read(L.BUF_XKV, np.float16, (2, nh, TPAD, 64), ((r * nl + l) * tile) * 2)
             for l in dec_layers for r in rows}
    kv_plane = nh * G.max_t * 64
    sup, bsup = set(gen["suppress_tokens"]), gen["begin_suppress_tokens"]
    emb = Wd["model.decoder.embed_tokens.weight"]
    worst = worst_lg = 0.0
    checked, rows_checked = 0, set()
    for p in range(T - 1):
        e.step(B, False, T)
        if p < NP - 1:
            continue
        # every row: the LM head layer-local, and the transcription's token against the oracle's choice
        xf = e.dec_x()[:B]
        h = R.layer_norm(xf, Wd["model.decoder.layer_norm.weight"], Wd["model.decoder.layer_norm.bias"])
        ref_all = R.linear(h, emb)
        lg_all = e.logits()[:B]
        err = rel_err(lg_all, ref_all)
        worst_lg = max(worst_lg, err)
        assert err <= 2e-3, (p, "logits", err)
        first = p + 1 == NP
        for r in range(B):
            if len(out[r].seq) > p + 1 and R.top2_margin(ref_all[r], sup, bsup, first) > 1e-2:
                assert out[r].seq[p + 1] == R.choose(ref_all[r], sup, bsup, first, gen["eos_token_id"], False), (p, r)
                checked += 1
                rows_checked.add(r)
        if p < T - 3:
            continue
        tr = e.dec_trace()[:, rows]
        for l in dec_layers:
            cache, xkv = [], []
            for r in rows:
                k = e.read(L.BUF_SELF_K, np.float16, (nh, G.max_t, 64), ((l * B + r) * kv_plane) * 2)
                v = e.read(L.BUF_SELF_V, np.float16, (nh, G.max_t, 64), ((l * B + r) * kv_plane) * 2)
                cache.append((k[:, :p].astype(np.float32), v[:, :p].astype(np.float32)))
                x = cross[(l, r)]
                xkv.append((x[0, :, :TENC].astype(np.float32), x[1, :, :TENC].astype(np.float32)))
            ref, _, _, _ = R.decoder_layer(tr[l], Wd, l, nh, cache, xkv)
            err = rel_err(tr[l + 1], ref)
            worst = max(worst, err)
            assert err <= 2e-3, (p, l, err)
    e.set_trace(False)
    print("large-v3 e2e, rows 3 and 20: decoder layers 0 / 15 / 31 max-abs / RMS", worst, "; LM head (32 rows,",
          T - NP, "positions)", worst_lg, "; choices checked", checked, "in", len(rows_checked), "rows")
    assert len(rows_checked) >= 8 and checked >= 8 * 8
