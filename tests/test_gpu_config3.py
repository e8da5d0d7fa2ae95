"""One large-v3 encoder layer on a group of 8 clips (8 x 1500 = 12,000 tokens, d 1280, 20 heads, ff 5120): the
workload the encoder's products and attention are measured on, at its own size.

The engine encodes 8 clips through the conv stem and one layer with the trace on, so every kernel of a layer runs at
M = 12,000 exactly as the benchmark launches it: the fused QKV product scattering q (scaled by log2(e) / 8), k and v^T
into per-head tiles of 8 clips, the attention over 8 x 20 (clip, head) pairs, the out-projection, the residual add +
LayerNorm, fc1 + GELU, fc2 and the last add + LayerNorm (here the encoder's final LayerNorm), then the cross keys /
values of the decoder layer for all 8 clip slots. Checked for every clip against the oracle:

* the layer layer-local (the oracle's layer on the engine's own fp32 input) at max-abs error <= 2e-3 x RMS;
* the final LayerNorm's fp16 output within one fp16 ulp of a float64 LayerNorm of the engine's residual, plus the
  float32 evaluation error of its terms (4 float32 ulps of (|x - mean| + |mean|) rstd |w| + |b|), which exceeds the
  fp16 spacing only for outputs near zero;
* the cross keys / values (head-scatter product, kind 2) within one fp16 ulp of the float64 product of the engine's
  fp16 encoder output, plus 1e-5 x RMS for results that cancel to near zero.
"""
import numpy as np
import pytest

from mimizuku_amd import _lib as L
from mimizuku_amd import model, synth
from oracle import whisper_ref as R

pytestmark = pytest.mark.gpu

G = synth.Geometry(d=1280, ff=5120, nh=20, enc_layers=1, dec_layers=1, n_mels=128, vocab=51866)
N = 8
TPAD = 1536


def rel_err(got, ref):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    return np.abs(got - ref).max() / np.sqrt((ref ** 2).mean())


def ulp_excess(got, ref, ulps=1.0, cancel=0.0):
    """Largest |got - ref| beyond `ulps` fp16 units in the last place of the exact value ref (plus `cancel`)."""
    ref = np.asarray(ref, np.float64)
    ulp = np.spacing(np.abs(ref).astype(np.float16)).astype(np.float64)
    return float((np.abs(np.asarray(got, np.float64) - ref) - ulps * ulp - cancel).max())


def ln_f64(x, w, b):
    """float64 LayerNorm of x and the size of the terms an fp32 evaluation rounds: (|x - mean| + |mean|) rstd |w| +
    |b| (the deviation is formed from x and the mean, each known to an fp32 ulp)."""
    x64 = x.astype(np.float64)
    mu = x64.mean(-1, keepdims=True)
    r = 1.0 / np.sqrt(((x64 - mu) ** 2).mean(-1, keepdims=True) + 1e-5)
    return (x64 - mu) * r * w + b, (np.abs(x64 - mu) + np.abs(mu)) * r * np.abs(w) + np.abs(b)


def test_large_v3_layer_on_8_clips():
    W = synth.random_weights(G, seed=14, bias_std=0.02, ln_std=0.1)
    Wf = {k: v.astype(np.float32) for k, v in W.items() if k.startswith("model.encoder")}
    gen = synth.generation_config(G, align_heads=[[0, 0]])
    dims = model.Dims(G.d, G.ff, G.nh, G.enc_layers, G.dec_layers, G.n_mels, G.vocab, G.max_t)
    ctx = model.Context(0)
    e = model.Engine(ctx, dims, model.GenCfg.from_dict(gen, dims), N, N)
    e.load(W)
    mel = synth.synthetic_mel(N, G.n_mels, seed=15)
    e.set_trace(True)
    e.encode(mel, 0)
    tr = e.trace(N)[0]  # [8][1500][d] input of layer 0
    xl = e.read(L.BUF_ENC_X, np.float32, (N, 1500, G.d))  # residual after the layer
    out = e.enc_out(N)  # final LayerNorm, fp16
    xkv = e.xkv()[:N, 0]  # [8][k|v][nh][1536][64]
    lw = W["model.encoder.layer_norm.weight"].astype(np.float64)
    lb = W["model.encoder.layer_norm.bias"].astype(np.float64)
    pre = "model.decoder.layers.0.encoder_attn"
    wk = W[f"{pre}.k_proj.weight"].astype(np.float64)
    wv = W[f"{pre}.v_proj.weight"].astype(np.float64)
    bv = W[f"{pre}.v_proj.bias"].astype(np.float64)
    errs, worst_ln = [], 0.0
    for c in range(N):
        err = rel_err(xl[c], R.encoder_layer(tr[c], Wf, 0, G.nh))
        errs.append(err)
        ln64, terms = ln_f64(xl[c], lw, lb)
        assert ulp_excess(out[c], ln64, cancel=2.0 ** -22 * terms) <= 0, (c, "final LayerNorm beyond one fp16 ulp")
        lnu = np.spacing(np.abs(ln64).astype(np.float16)).astype(np.float64)
        worst_ln = max(worst_ln, float(np.max(np.abs(out[c] - ln64) / lnu)))
        eh = out[c].astype(np.float64)
        for which, ref in ((0, eh @ wk.T), (1, eh @ wv.T + bv)):
            tiles = xkv[c, which]  # [nh][1536][64]
            assert not tiles[:, 1500:].any()
            got = tiles[:, :1500].transpose(1, 0, 2).reshape(1500, G.d)
            rms = np.sqrt((ref ** 2).mean())
            assert ulp_excess(got, ref, cancel=1e-5 * rms) <= 0, (c, which, "cross k/v beyond one fp16 ulp")
    print("large-v3 layer, 8 clips: layer-local max-abs / RMS per clip", ["%.2e" % x for x in errs],
          "; final LayerNorm largest error", worst_ln, "fp16 ulps of the float64 value")
    assert max(errs) <= 2e-3, errs
    e.close()
    ctx.close()
