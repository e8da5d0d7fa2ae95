"""Pins the CPU oracle (oracle/whisper_ref.py) before results are checked against it.

* against the golden vectors transformers 5.15.0 wrote for the tiny geometry (tests/golden/make_golden.py);
* against the reference's own known-answer tests (src/align.rs:112-139);
* against closed forms, brute force and invariants chosen so that a dropped term, a wrong index or a transposed
  operand fails.
"""
import math
import os

import numpy as np
import pytest

from mimizuku_amd import synth
from oracle import whisper_ref as R

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")
G = synth.TINY


def _fixture(name):
    fx = np.load(os.path.join(GOLDEN, f"{name}.npz"))
    W = synth.random_weights(G, seed=int(fx["seed"]), bias_std=float(fx["bias_std"]), ln_std=float(fx["ln_std"]))
    assert synth.weights_digest(W) == str(fx["weights_digest"]), "weight generator drifted from the fixture"
    Wf = {k: v.astype(np.float32) for k, v in W.items()}
    mel = synth.synthetic_mel(int(fx["n_clips"]), G.n_mels, seed=int(fx["mel_seed"]))
    return fx, Wf, mel


@pytest.fixture(scope="module", params=["tiny_hfinit", "tiny_bias_detect"])
def golden(request):
    return request.param, *_fixture(request.param)


def test_encoder_matches_transformers(golden):
    name, fx, W, mel = golden
    for b in range(int(fx["n_clips"])):
        hidden, out = R.encoder(mel[b], W, G.nh, G.enc_layers)
        states = hidden + [out]
        for i, h in enumerate(states):
            ref = fx["enc_hidden_rows"][i, b]
            rms = np.sqrt((ref ** 2).mean())
            assert np.abs(h[fx["rows"]] - ref).max() < 1e-5 * max(rms, 1), (name, b, i)
            assert abs(h.astype(np.float64).sum() - fx["enc_hidden_sum"][i, b]) < 1e-2 + 1e-6 * h.size
            assert abs((h.astype(np.float64) ** 2).sum() - fx["enc_hidden_sumsq"][i, b]) < 1e-6 * fx["enc_hidden_sumsq"][i, b]


def test_greedy_tokens_logits_timestamps_match_transformers(golden):
    name, fx, W, mel = golden
    gen = synth.generation_config(G)
    prompt = [50258, 50259, 50359, 50363]
    r = R.greedy(W, G, gen, mel, prompt, 32, detect=bool(fx["detect"]))
    np.testing.assert_array_equal(r["tokens"], fx["sequences"])
    lg = r["logits"]  # [steps][B][V]
    assert np.abs(lg[..., fx["vocab_sub"]] - fx["logits_sub"]).max() < 2e-5
    np.testing.assert_allclose(np.take_along_axis(lg, fx["top2_ids"].astype(np.int64), -1), fx["top2_val"], atol=2e-5)
    n_seq = fx["sequences"].shape[1]
    for b in range(int(fx["n_clips"])):
        ts = R.token_timestamps(r["probs"][b], gen["alignment_heads"], len(prompt), n_seq, 3000, half=False)
        np.testing.assert_array_equal(ts, fx["token_timestamps"][b])
        # alignment-head weights of the fed-back rows equal transformers' cross-attentions
        w = np.stack([r["probs"][b][:, l, h] for l, h in gen["alignment_heads"]], axis=0)  # [heads][rows][1500]
        assert np.abs(w[:, :fx["align_w"].shape[2]] - fx["align_w"][b]).max() < 1e-6


def test_jump_times_from_transformers_weights(golden):
    name, fx, W, mel = golden
    for b in range(int(fx["n_clips"])):
        w = fx["align_w"][b].transpose(1, 0, 2)[4:]  # rows of the generated tokens fed back
        jt = R.jump_times(w, 1500, 7, half=False)
        np.testing.assert_array_equal(jt, fx["token_timestamps"][b][4:4 + len(jt)])


# ---------------------------------------------------------------- reference KATs (src/align.rs:112-139)

def test_dtw_follows_the_cheap_diagonal():
    rows, cols = 3, 6
    m = np.array([[-1.0 if (j // 2) == i else 1.0 for j in range(cols)] for i in range(rows)])
    text, time = R.dtw(m)
    assert text.tolist() == [0, 0, 1, 1, 2, 2]
    assert time.tolist() == [0, 1, 2, 3, 4, 5]


def test_jump_times_of_a_clean_alignment():
    rows, full, cols = 4, 60, 40
    w = np.zeros((rows, 1, full), np.float32)
    for i in range(rows):
        w[i, 0, 10 * i:10 * i + 10] = 0.1
    for half in (False, True):
        t = R.jump_times(w, cols, 7, half)
        assert len(t) == rows
        assert np.all(np.abs(t - 0.2 * np.arange(rows)) < 0.03)
        assert R.jump_times(w, 0, 7, half).tolist() == [0.0] * rows
        assert R.jump_times(w[:1], cols, 7, half).tolist() == [0.0]


# ---------------------------------------------------------------- closed forms and brute force

def test_layer_norm_closed_form():
    rng = np.random.default_rng(0)
    x = rng.standard_normal((5, 256)).astype(np.float32) * 3 + 1
    w = rng.standard_normal(256).astype(np.float32)
    b = rng.standard_normal(256).astype(np.float32)
    y = R.layer_norm(x, np.ones(256, np.float32), np.zeros(256, np.float32))
    np.testing.assert_allclose(y.mean(-1), 0, atol=1e-5)
    np.testing.assert_allclose(y.var(-1), 1 - 1e-5 / x.var(-1), rtol=1e-4)
    ref = []
    for r in x.astype(np.float64).tolist():
        mu = sum(r) / len(r)
        sd = math.sqrt(sum((v - mu) ** 2 for v in r) / len(r) + 1e-5)
        ref.append([(v - mu) / sd for v in r])
    np.testing.assert_allclose(R.layer_norm(x, w, b), np.array(ref) * w + b, rtol=1e-4, atol=1e-4)


def test_gelu_closed_form():
    xs = [-5.0, -1.5, -0.3, 0.0, 0.7, 2.0, 6.0]
    got = R.gelu(np.array(xs, np.float32))
    want = [0.5 * x * (1 + math.erf(x / math.sqrt(2))) for x in xs]
    np.testing.assert_allclose(got, want, rtol=1e-6, atol=1e-7)


def test_attention_closed_form_and_key_permutation():
    rng = np.random.default_rng(1)
    q = rng.standard_normal((3, 7, 64))
    k = rng.standard_normal((3, 11, 64))
    v = rng.standard_normal((3, 11, 64))
    o = R.attention(q, k, v, dtype=np.float64)
    s = np.einsum("hqd,hkd->hqk", q, k) / 8.0
    p = np.exp(s - s.max(-1, keepdims=True))
    p /= p.sum(-1, keepdims=True)
    np.testing.assert_allclose(o, np.einsum("hqk,hkd->hqd", p, v), rtol=1e-10, atol=1e-14)
    perm = rng.permutation(11)
    np.testing.assert_allclose(R.attention(q, k[:, perm], v[:, perm], dtype=np.float64), o, rtol=1e-10, atol=1e-14)
    # one key: the output is that key's value, whatever the query
    np.testing.assert_allclose(R.attention(q, k[:, :1], v[:, :1], dtype=np.float64), np.broadcast_to(v[:, :1], o.shape))


def test_conv1d_brute_force():
    rng = np.random.default_rng(2)
    x = rng.standard_normal((3, 9)).astype(np.float32)
    w = rng.standard_normal((4, 3, 3)).astype(np.float32)
    b = rng.standard_normal(4).astype(np.float32)
    for stride in (1, 2):
        y = R.conv1d(x, w, b, stride, 1)
        tout = (9 + 2 - 3) // stride + 1
        assert y.shape == (4, tout)
        for o in range(4):
            for t in range(tout):
                s = b[o]
                for ci in range(3):
                    for k in range(3):
                        tt = stride * t + k - 1
                        if 0 <= tt < 9:
                            s += w[o, ci, k] * x[ci, tt]
                assert abs(y[o, t] - s) < 1e-5


def test_median_filter_brute_force():
    rng = np.random.default_rng(3)
    z = rng.standard_normal((2, 3, 13)).astype(np.float32)
    f = R.median_filter(z, 7)
    for idx in np.ndindex(2, 3):
        row = z[idx]
        padded = np.concatenate([row[1:4][::-1], row, row[-4:-1][::-1]])
        for j in range(13):
            assert f[idx][j] == np.median(padded[j:j + 7])
    small = z[..., :3]
    np.testing.assert_array_equal(R.median_filter(small, 7), small)


def test_choose_rules():
    lg = np.array([1.0, 3.0, 3.0, 2.0, 5.0], np.float32)
    assert R.choose(lg, {4}, [], False, 0, False) == 1  # tie -> lowest id
    assert R.choose(lg, {4}, [1], True, 0, False) == 2  # begin-suppress only at the first position
    assert R.choose(lg, {4}, [1], False, 0, False) == 1
    assert R.choose(lg, {0, 1, 2, 3, 4}, [], False, 7, False) == 7  # all suppressed -> eos
    assert R.choose(lg, set(), [], False, 7, True) == 7  # finished row -> eos


def test_top2_margin_closed_form():
    lg = np.array([0.5, 3.0, -1.0, 2.25, 7.0], np.float32)
    assert R.top2_margin(lg, {4}, [], False) == 0.75  # 3.0 - 2.25 once id 4 is suppressed
    assert R.top2_margin(lg, set(), [4], True) == 0.75  # begin-suppressed at the first position
    assert R.top2_margin(lg, set(), [4], False) == 4.0  # but not later: 7.0 - 3.0


def test_fp16_rounding_known_answers():
    assert R.rh(1.0 + 2.0 ** -11) == 1.0  # a tie rounds to even
    assert R.rh(1.0 + 3.0 * 2.0 ** -11) == 1.0 + 2.0 ** -9
    assert R.rh(65519.0) == 65504.0 and np.isinf(R.rh(65520.0))
    assert R.rh(2.0 ** -25) == 0.0 and R.rh(3.0 * 2.0 ** -25) == 2.0 ** -23  # subnormal ties
