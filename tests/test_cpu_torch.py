"""The torch restatement that times the CPU baseline (oracle/cpu_torch.py) computes what the numpy oracle computes:
encoder layer, conv stem, cross keys/values, a decoder layer with self-attention cache and cross-attention, and the
final LayerNorm + tied LM head, on a small geometry with non-zero biases and LayerNorm parameters (fp32, max-abs error
within 1e-5 x RMS: only the summation order differs). torch is imported inside the tests, so a GPU test run, which
collects this module, never loads it."""
import numpy as np
import pytest

from mimizuku_amd import synth
from oracle import whisper_ref as R

G = synth.Geometry(d=128, ff=256, nh=2, enc_layers=1, dec_layers=2, n_mels=16, vocab=51865, max_t=32)


def rel_err(got, ref):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    return np.abs(got - ref).max() / np.sqrt((ref ** 2).mean())


@pytest.fixture(scope="module")
def weights():
    W = synth.random_weights(G, seed=4, bias_std=0.02, ln_std=0.1)
    return {k: v.astype(np.float32) for k, v in W.items()}


def test_encoder_side(weights):
    torch = pytest.importorskip("torch")
    from oracle import cpu_torch as T
    Wt = {k: torch.from_numpy(v) for k, v in weights.items()}
    rng = np.random.default_rng(0)
    x = rng.standard_normal((2, 1500, G.d)).astype(np.float32)
    got = T.encoder_layer(torch.from_numpy(x), Wt, "model.encoder.layers.0", G.nh).numpy()
    for c in range(2):
        assert rel_err(got[c], R.encoder_layer(x[c], weights, 0, G.nh)) < 1e-5
    mel = synth.synthetic_mel(2, G.n_mels, seed=3)
    stem = T.conv_stem(torch.from_numpy(mel), Wt).numpy()
    for c in range(2):
        assert rel_err(stem[c], R.conv_stem(mel[c], weights)) < 1e-5
    kv = T.cross_kv(torch.from_numpy(x), Wt, [0, 1], G.nh)
    for c in range(2):
        ref = R.cross_kv(x[c], weights, 2, G.nh)
        for i in range(2):
            for j in range(2):
                assert rel_err(kv[i][j][c].numpy(), ref[i][j]) < 1e-5


def test_decoder_side(weights):
    torch = pytest.importorskip("torch")
    from oracle import cpu_torch as T
    Wt = {k: torch.from_numpy(v) for k, v in weights.items()}
    rng = np.random.default_rng(1)
    B, pos = 3, 5
    x = rng.standard_normal((B, G.d)).astype(np.float32)
    kc = rng.standard_normal((B, G.nh, G.max_t, 64)).astype(np.float32)
    vc = rng.standard_normal((B, G.nh, G.max_t, 64)).astype(np.float32)
    xk = rng.standard_normal((B, G.nh, 1500, 64)).astype(np.float32)
    xv = rng.standard_normal((B, G.nh, 1500, 64)).astype(np.float32)
    kt, vt = torch.from_numpy(kc.copy()), torch.from_numpy(vc.copy())
    got = T.decoder_layer(torch.from_numpy(x), Wt, 1, G.nh, kt, vt, pos, torch.from_numpy(xk),
                          torch.from_numpy(xv)).numpy()
    ref, k, v, _ = R.decoder_layer(x, weights, 1, G.nh, [(kc[b, :, :pos], vc[b, :, :pos]) for b in range(B)],
                                   [(xk[b], xv[b]) for b in range(B)])
    assert rel_err(got, ref) < 1e-5
    assert rel_err(kt[:, :, pos].numpy(), k.reshape(B, G.nh, 64)) < 1e-5
    assert rel_err(vt[:, :, pos].numpy(), v.reshape(B, G.nh, 64)) < 1e-5
    lg = T.lm_head(torch.from_numpy(ref), Wt).numpy()
    h = R.layer_norm(ref, weights["model.decoder.layer_norm.weight"], weights["model.decoder.layer_norm.bias"])
    assert rel_err(lg, R.linear(h, weights["model.decoder.embed_tokens.weight"])) < 1e-5
