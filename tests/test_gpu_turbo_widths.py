"""GPU parity at the large-v3-turbo widths (d 1280, 20 heads, ff 5120, 128 mels, vocab 51866).

Encoder: two clips through the conv stem and two layers, every part checked layer-local against the oracle (the
oracle's layer applied to the engine's own fp32 input of that layer) at max-abs error <= 2e-3 x RMS, as
test_gpu_engine.py does on the tiny geometry, and the final LayerNorm's fp16 output within one fp16 ulp: this covers
the products and the attention at the full widths with the clip and head indexing of a group of more than one clip.

Decoder: the benchmark's batch of 32 rows through 4 layers, against the oracle's decoder on the same fp16 weights and
cross keys/values.

The tiny geometry of test_gpu_engine.py runs every decoder kernel, but only at its own sizes: this file covers the
configurations the benchmark runs and the tiny model never reaches — split-K slices of 256 and 1024, the QKV and fc1
products at K = 1280, the persistent LM head's full-K weight ring over 250 workgroups, cross-attention over 1500 keys
for 32 x 20 (row, head) pairs. Teacher-forced: reset with a 10-token prompt per row, then every step's logits and
alignment-head rows are compared with the oracle's, and the greedy choice after the prompt wherever the oracle's
top-2 margin exceeds 1e-2. Bars as in test_gpu_engine.py, except the alignment rows: max-abs error <= 2e-3 x the
largest probability. These rows are nearly uniform (the largest ~0.01), and each probability carries the relative
error of its score, ~1e-3 here from the fp16 rounding of the LayerNorm output that feeds the query (the oracle keeps
it in fp32; the reference rounds it, as the kernels here do).

At the benchmark's own positions (200 .. 203, the self-attention cache holding 200+ keys) every decoder layer is
checked layer-local on the engine's residual trace, and the logits of its final residual against the oracle's head;
and the step as the benchmark runs it, one captured graph replayed through positions 0 .. 205 of a 200-token prompt,
gives the same bits as eager steps.
"""
import numpy as np
import pytest

from mimizuku_amd import _lib as L
from mimizuku_amd import model, synth
from oracle import whisper_ref as R

pytestmark = pytest.mark.gpu

B, NP, TPAD = 32, 10, 1536
G = synth.Geometry(d=1280, ff=5120, nh=20, enc_layers=1, dec_layers=4, n_mels=128, vocab=51866)


def rel_err(got, ref):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    return np.abs(got - ref).max() / np.sqrt((ref ** 2).mean())


def test_encoder_turbo_widths_layer_local():
    g = synth.Geometry(d=1280, ff=5120, nh=20, enc_layers=2, dec_layers=1, n_mels=128, vocab=51866)
    W = synth.random_weights(g, seed=6, bias_std=0.02, ln_std=0.1)
    Wf = {k: v.astype(np.float32) for k, v in W.items() if k.startswith("model.encoder")}
    gen = synth.generation_config(g, align_heads=[[0, 0]])
    dims = model.Dims(g.d, g.ff, g.nh, g.enc_layers, g.dec_layers, g.n_mels, g.vocab, g.max_t)
    ctx = model.Context(0)
    e = model.Engine(ctx, dims, model.GenCfg.from_dict(gen, dims), 2, 2)
    e.load(W)
    mel = synth.synthetic_mel(2, g.n_mels, seed=9)
    e.set_trace(True)
    e.encode(mel, 0)
    tr = e.trace(2)  # [L][n][1500][d] inputs of every layer
    xl = e.read(L.BUF_ENC_X, np.float32, (2, 1500, g.d))
    out = e.enc_out(2).astype(np.float32)
    for c in range(2):
        m16 = mel[c].astype(np.float16).astype(np.float32)
        errs = [rel_err(tr[0, c], R.conv_stem(m16, Wf))]
        for i in range(g.enc_layers):
            nxt = tr[i + 1, c] if i + 1 < g.enc_layers else xl[c]
            errs.append(rel_err(nxt, R.encoder_layer(tr[i, c], Wf, i, g.nh)))
        # the final LayerNorm's fp16 output within one fp16 ulp of a float64 LayerNorm of the same residual, plus the
        # float32 evaluation error of its terms (4 fp32 ulps of (|x - mean| + |mean|) rstd |w| + |b|; it exceeds the
        # fp16 spacing only for outputs near zero)
        lw = W["model.encoder.layer_norm.weight"].astype(np.float64)
        lb = W["model.encoder.layer_norm.bias"].astype(np.float64)
        x64 = xl[c].astype(np.float64)
        mu = x64.mean(-1, keepdims=True)
        r = 1.0 / np.sqrt(((x64 - mu) ** 2).mean(-1, keepdims=True) + 1e-5)
        ref = (x64 - mu) * r * lw + lb
        terms = (np.abs(x64 - mu) + np.abs(mu)) * r * np.abs(lw) + np.abs(lb)
        ulp = np.spacing(np.abs(ref).astype(np.float16)).astype(np.float64)
        excess = np.abs(out[c] - ref) - ulp - 2.0 ** -22 * terms
        assert np.all(excess <= 0), (np.unravel_index(np.argmax(excess), excess.shape), excess.max())
        print("turbo widths, clip", c, "final LayerNorm: largest error", float(np.max(np.abs(out[c] - ref) / ulp)),
              "fp16 ulps of the float64 value")
        print("turbo widths, clip", c, ["%.2e" % x for x in errs])
        assert max(errs) < 2e-3, errs
    e.close()
    ctx.close()


def test_decoder_turbo_widths_batch32():
    rng = np.random.default_rng(21)
    W = synth.random_weights(G, seed=5, bias_std=0.02, ln_std=0.1)
    Wf = {k: v.astype(np.float32) for k, v in W.items() if k.startswith("model.decoder")}
    gen = synth.generation_config(G, align_heads=[[2, 4], [2, 11], [3, 3], [3, 6], [3, 11], [3, 14]])
    dims = model.Dims(G.d, G.ff, G.nh, G.enc_layers, G.dec_layers, G.n_mels, G.vocab, G.max_t)
    gc = model.GenCfg.from_dict(gen, dims)
    # cross keys/values [B][layer][k|v][head][1536][64] (rows past 1500 zero), N(0, 1) on the fp16 grid
    xkv = np.zeros((B, G.dec_layers, 2, G.nh, TPAD, 64), np.float16)
    for b in range(B):
        xkv[b, :, :, :, :1500] = rng.standard_normal((G.dec_layers, 2, G.nh, 1500, 64), dtype=np.float32)
    prompts = rng.integers(0, 50000, size=(B, NP)).astype(np.int32)

    ctx = model.Context(0)
    e = model.Engine(ctx, dims, gc, B, 8)
    e.load(W)
    e.set_trace(True)
    p, n = e.buffer(L.BUF_XKV)
    assert n >= xkv.nbytes
    ctx.upload(p, xkv)
    dec = R.Decoder(Wf, G.nh, G.dec_layers,
                    [[(xkv[b, l, 0, :, :1500].astype(np.float32), xkv[b, l, 1, :, :1500].astype(np.float32))
                      for l in range(G.dec_layers)] for b in range(B)])
    del xkv
    e.reset(prompts)
    sup = set(gen["suppress_tokens"])
    bsup = gen["begin_suppress_tokens"]
    worst, worst_ll, checked = 0.0, 0.0, 0
    for pos in range(NP):
        e.step(B, False, NP)
        ref, probs = dec.step(prompts[:, pos].tolist(), pos)
        lg = e.logits()[:B]
        worst = max(worst, rel_err(lg, ref))
        # layer-local: the final LayerNorm and the tied LM head on the engine's own final residual
        h = R.layer_norm(e.dec_trace()[-1, :B], Wf["model.decoder.layer_norm.weight"],
                         Wf["model.decoder.layer_norm.bias"])
        worst_ll = max(worst_ll, rel_err(lg, R.linear(h, Wf["model.decoder.embed_tokens.weight"])))
        al = e.align()[:B, pos].astype(np.float32)  # [B][slots][1500]
        for s, (l, h) in enumerate(gen["alignment_heads"]):
            r = probs[:, l, h]
            assert np.abs(al[:, s] - r).max() < 2e-3 * r.max(), (pos, s)
        if pos == NP - 1:  # the first generated position: the engine's choice against the rules on the oracle's logits
            toks = e.tokens()[:B, NP]
            for b in range(B):
                top = np.sort(ref[b][np.setdiff1d(np.arange(G.vocab), list(sup) + list(bsup))])[-2:]
                if top[1] - top[0] > 1e-2:
                    assert toks[b] == R.choose(ref[b], sup, bsup, True, gen["eos_token_id"], False), b
                    checked += 1
    print("turbo widths, B = 32: logits max-abs / RMS", worst, "; layer-local", worst_ll, "; greedy choices checked",
          checked)
    assert worst_ll <= 2e-3
    assert worst < 2e-2  # through the whole 4-layer decoder from the oracle's own residual stream
    assert checked >= B // 2
    e.close()
    ctx.close()


@pytest.mark.parametrize("nb", [32, 8, 1])
def test_decoder_turbo_widths_at_position_200(nb):
    """The benchmark's decoder step shape: 32 rows at positions 200 .. 203, the self-attention cache holding 200+
    keys; and the same with 8 rows and with 1 (a single clip, or the last partial chunk of a batch: the skinny
    products then run with most of their 32-row MFMA operand zero). Every decoder layer layer-local (the oracle's layer
    on the engine's own residual, cache and cross keys / values) within 2e-3 x RMS, and the logits of the engine's
    final residual (the final LayerNorm and the tied LM head, layer-local) within 2e-3 x RMS."""
    B = nb
    rng = np.random.default_rng(22 + nb)
    W = synth.random_weights(G, seed=6, bias_std=0.02, ln_std=0.1)
    Wf = {k: v.astype(np.float32) for k, v in W.items() if k.startswith("model.decoder")}
    gen = synth.generation_config(G, align_heads=[[2, 4], [2, 11], [3, 3], [3, 6], [3, 11], [3, 14]])
    dims = model.Dims(G.d, G.ff, G.nh, G.enc_layers, G.dec_layers, G.n_mels, G.vocab, G.max_t)
    gc = model.GenCfg.from_dict(gen, dims)
    xkv = np.zeros((B, G.dec_layers, 2, G.nh, TPAD, 64), np.float16)
    for b in range(B):
        xkv[b, :, :, :, :1500] = rng.standard_normal((G.dec_layers, 2, G.nh, 1500, 64), dtype=np.float32)
    npr = 204
    prompts = rng.integers(0, 50000, size=(B, npr)).astype(np.int32)
    ctx = model.Context(0)
    e = model.Engine(ctx, dims, gc, B, min(8, B))
    e.load(W)
    e.set_trace(True)
    p, _ = e.buffer(L.BUF_XKV)
    ctx.upload(p, xkv)
    cross = [[(xkv[b, i, 0, :, :1500].astype(np.float32), xkv[b, i, 1, :, :1500].astype(np.float32))
              for b in range(B)] for i in range(G.dec_layers)]
    del xkv
    e.reset(prompts)
    worst = worst_lg = 0.0
    for pos in range(npr):
        e.step(B, False, npr)
        if pos < 200:
            continue
        tr = e.dec_trace()[:, :B]
        kc, vc = e.self_kv()
        for i in range(G.dec_layers):
            cache = [(kc[i, b, :, :pos].astype(np.float32), vc[i, b, :, :pos].astype(np.float32)) for b in range(B)]
            out, _, _, _ = R.decoder_layer(tr[i], Wf, i, G.nh, cache, cross[i])
            err = rel_err(tr[i + 1], out)
            worst = max(worst, err)
            assert err <= 2e-3, (pos, i, err)
        h = R.layer_norm(tr[-1], Wf["model.decoder.layer_norm.weight"], Wf["model.decoder.layer_norm.bias"])
        ref = R.linear(h, Wf["model.decoder.embed_tokens.weight"])
        worst_lg = max(worst_lg, rel_err(e.logits()[:B], ref))
    print(f"turbo widths, B = {B}, positions 200..203: layer-local max-abs / RMS", worst, "; logits", worst_lg)
    assert worst_lg <= 2e-3
    e.close()
    ctx.close()


def test_graph_replay_at_position_200_equals_eager():
    """The benchmark's replayed step against eager steps at its own shape: 32 rows, a 200-token prompt, 206 steps
    (positions 0 .. 205, greedy choices from position 200 on). One captured graph replayed 206 times gives the same
    bits as 206 eager launches of the same kernels: every token, the final residual and logits of the last step, the
    alignment rows of positions 196 .. 205 and both self-attention caches."""
    rng = np.random.default_rng(23)
    W = synth.random_weights(G, seed=7, bias_std=0.02, ln_std=0.1)
    gen = synth.generation_config(G, align_heads=[[2, 4], [2, 11], [3, 3], [3, 6], [3, 11], [3, 14]])
    dims = model.Dims(G.d, G.ff, G.nh, G.enc_layers, G.dec_layers, G.n_mels, G.vocab, G.max_t)
    gc = model.GenCfg.from_dict(gen, dims)
    xkv = np.zeros((B, G.dec_layers, 2, G.nh, TPAD, 64), np.float16)
    for b in range(B):
        xkv[b, :, :, :, :1500] = rng.standard_normal((G.dec_layers, 2, G.nh, 1500, 64), dtype=np.float32)
    npr, steps = 200, 206
    prompts = rng.integers(0, 50000, size=(B, npr)).astype(np.int32)
    ctx = model.Context(0)
    e = model.Engine(ctx, dims, gc, B, 8)
    e.load(W)
    p, _ = e.buffer(L.BUF_XKV)
    ctx.upload(p, xkv)
    del xkv

    def state():
        kc, vc = e.self_kv()
        return (e.tokens()[:B, :steps + 1], e.dec_x()[:B], e.logits()[:B], e.align()[:B, steps - 10:steps],
                kc[:, :B, :, :steps], vc[:, :B, :, :steps])

    e.reset(prompts)
    for _ in range(steps):
        e.step(B, False, npr)
    eager = state()
    e.reset(prompts)
    e.capture(B, npr)
    for _ in range(steps):
        e.replay()
    graph = state()
    names = ("tokens", "final residual", "logits", "alignment rows", "self keys", "self values")
    for n, a, g in zip(names, eager, graph):
        np.testing.assert_array_equal(a, g, err_msg=n)
    assert np.all(eager[0][:, :npr] == prompts)
    print("turbo widths, B = 32: graph replay = eager steps over positions 0 ..", steps - 1, "; generated",
          eager[0][:4, npr:].tolist(), "...")
    e.close()
    ctx.close()


def test_cross_attention_variants_give_the_same_bits():
    """The cross-attention runs as one of two forms chosen by the batch: more than 12 rows (three workgroups per CU,
    half a batch of keys staged) or at most 12 (one workgroup per CU, two batches staged). Where the keys come from
    does not change the arithmetic: the first rows stepped in a batch of 32 and alone in batches of 12, 3, 2 and 1
    give the same bits (tokens, logits, alignment rows, residual stream), greedy from a 4-token prompt through 6
    positions."""
    rng = np.random.default_rng(24)
    W = synth.random_weights(G, seed=9, bias_std=0.02, ln_std=0.1)
    gen = synth.generation_config(G, align_heads=[[2, 4], [2, 11], [3, 3], [3, 6], [3, 11], [3, 14]])
    dims = model.Dims(G.d, G.ff, G.nh, G.enc_layers, G.dec_layers, G.n_mels, G.vocab, G.max_t)
    gc = model.GenCfg.from_dict(gen, dims)
    xkv = np.zeros((B, G.dec_layers, 2, G.nh, TPAD, 64), np.float16)
    for b in range(B):
        xkv[b, :, :, :, :1500] = rng.standard_normal((G.dec_layers, 2, G.nh, 1500, 64), dtype=np.float32)
    npr, steps, few = 4, 10, 12
    prompts = rng.integers(0, 50000, size=(B, npr)).astype(np.int32)
    ctx = model.Context(0)
    e = model.Engine(ctx, dims, gc, B, 8)
    e.load(W)
    p, _ = e.buffer(L.BUF_XKV)
    ctx.upload(p, xkv)
    del xkv
    out = {}
    for nb in (B, few, 3, 2, 1):
        e.reset(prompts[:nb])
        for _ in range(steps):
            e.step(nb, False, npr)
        out[nb] = (e.tokens()[:nb, :steps + 1], e.logits()[:nb], e.align()[:nb, :steps], e.dec_x()[:nb])
    for nb in (few, 3, 2, 1):
        for n, a, g in zip(("tokens", "logits", "alignment rows", "residual"), out[B], out[nb]):
            np.testing.assert_array_equal(a[:nb], g, err_msg=f"{n}, {nb} rows")
    print("cross-attention forms: the first rows of a batch of 32 and alone in batches of 12, 3, 2 and 1 give the same "
          "bits over", steps, "steps")
    e.close()
    ctx.close()
