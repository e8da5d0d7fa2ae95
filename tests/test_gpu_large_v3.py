"""GPU parity at the full large-v3 geometry: 32 encoder and 32 decoder layers, d 1280, 20 heads, ff 5120, 128 mels,
vocabulary 51,866 (the end-to-end large-v3 workload's model; the turbo tests cover the same widths at 4 decoder
layers).

Encoder: one clip through the conv stem and all 32 layers with the trace on; the conv stem and every fourth layer
checked layer-local (the oracle's layer on the engine's own fp32 input of that layer) at max-abs error <= 2e-3 x RMS.

Decoder: 4 rows teacher-forced on random prompts over random cross keys/values, through all 32 layers in one step:
at every position every fourth layer layer-local on the engine's residual trace (2e-3 x RMS), the LM head
layer-local on the engine's final residual (2e-3 x RMS), the logits against the oracle's 32-layer decoder (2e-2 x
RMS) and alignment heads spread over layers 16 .. 31 against the oracle's probabilities (2e-3 x the largest). Bars as
in test_gpu_turbo_widths.py.
"""
import numpy as np
import pytest

from mimizuku_amd import _lib as L
from mimizuku_amd import model, synth
from oracle import whisper_ref as R

pytestmark = pytest.mark.gpu

G = synth.LARGE_V3
TPAD = 1536
ALIGN = [[16, 3], [19, 11], [22, 0], [25, 7], [28, 19], [31, 14]]


def rel_err(got, ref):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    return np.abs(got - ref).max() / np.sqrt((ref ** 2).mean())


@pytest.fixture(scope="module")
def large(large_v3_weights):
    W = large_v3_weights
    gen = synth.generation_config(G, align_heads=ALIGN)
    dims = model.Dims(G.d, G.ff, G.nh, G.enc_layers, G.dec_layers, G.n_mels, G.vocab, G.max_t)
    ctx = model.Context(0)
    e = model.Engine(ctx, dims, model.GenCfg.from_dict(gen, dims), 4, 1)
    e.load(W)
    yield W, gen, ctx, e
    e.close()
    ctx.close()


def test_encoder_large_v3_32_layers(large):
    W, _, ctx, e = large
    Wf = {k: v.astype(np.float32) for k, v in W.items() if k.startswith("model.encoder")}
    mel = synth.synthetic_mel(1, G.n_mels, seed=10)
    e.set_trace(True)
    e.encode(mel, 0)
    tr = e.trace(1)[:, 0]  # [32][1500][d] inputs of every layer
    xl = e.read(L.BUF_ENC_X, np.float32, (1500, G.d))
    e.set_trace(False)
    errs = [rel_err(tr[0], R.conv_stem(mel[0].astype(np.float16).astype(np.float32), Wf))]
    for i in range(0, G.enc_layers, 4):
        nxt = tr[i + 1] if i + 1 < G.enc_layers else xl
        errs.append(rel_err(nxt, R.encoder_layer(tr[i], Wf, i, G.nh)))
    i = G.enc_layers - 1  # the last layer, into the residual the final LayerNorm reads
    errs.append(rel_err(xl, R.encoder_layer(tr[i], Wf, i, G.nh)))
    print("large-v3 encoder: conv stem and layers 0, 4, .., 28, 31:", ["%.2e" % x for x in errs])
    assert max(errs) < 2e-3, errs


def test_decoder_large_v3_32_layers(large):
    W, gen, ctx, e = large
    B, NP = 4, 6
    rng = np.random.default_rng(23)
    Wf = {k: v.astype(np.float32) for k, v in W.items() if k.startswith("model.decoder")}
    xkv = np.zeros((B, G.dec_layers, 2, G.nh, TPAD, 64), np.float16)
    for b in range(B):
        xkv[b, :, :, :, :1500] = rng.standard_normal((G.dec_layers, 2, G.nh, 1500, 64), dtype=np.float32)
    prompts = rng.integers(0, 50000, size=(B, NP)).astype(np.int32)
    p, n = e.buffer(L.BUF_XKV)
    assert n >= xkv.nbytes
    ctx.upload(p, xkv)
    cross = [[(xkv[b, i, 0, :, :1500].astype(np.float32), xkv[b, i, 1, :, :1500].astype(np.float32))
              for b in range(B)] for i in range(G.dec_layers)]
    dec = R.Decoder(Wf, G.nh, G.dec_layers, [[cross[i][b] for i in range(G.dec_layers)] for b in range(B)])
    del xkv
    e.set_trace(True)
    e.reset(prompts)
    worst = worst_lg = worst_ll = 0.0
    for pos in range(NP):
        e.step(B, False, NP)
        ref, probs = dec.step(prompts[:, pos].tolist(), pos)
        lg = e.logits()[:B]
        worst_lg = max(worst_lg, rel_err(lg, ref))
        h = R.layer_norm(e.dec_trace()[-1, :B], Wf["model.decoder.layer_norm.weight"],
                         Wf["model.decoder.layer_norm.bias"])
        worst_ll = max(worst_ll, rel_err(lg, R.linear(h, Wf["model.decoder.embed_tokens.weight"])))
        al = e.align()[:B, pos].astype(np.float32)
        for s, (l, h) in enumerate(ALIGN):
            r = probs[:, l, h]
            assert np.abs(al[:, s] - r).max() < 2e-3 * r.max(), (pos, s)
        tr = e.dec_trace()[:, :B]
        kc, vc = e.self_kv()
        for i in range(0, G.dec_layers, 4):
            cache = [(kc[i, b, :, :pos].astype(np.float32), vc[i, b, :, :pos].astype(np.float32)) for b in range(B)]
            out, _, _, _ = R.decoder_layer(tr[i], Wf, i, G.nh, cache, cross[i])
            err = rel_err(tr[i + 1], out)
            worst = max(worst, err)
            assert err <= 2e-3, (pos, i, err)
    e.set_trace(False)
    print("large-v3 decoder, B = 4: layer-local max-abs / RMS", worst, "; logits", worst_lg, "; LM head layer-local",
          worst_ll)
    assert worst_ll <= 2e-3
    assert worst_lg < 2e-2  # through all 32 layers from the oracle's own residual stream
