"""Greedy tokens and token timestamps at the benchmark's widths against the oracle (large-v3-turbo decoder: d 1280,
20 heads, 4 layers, vocabulary 51866, 6 alignment heads), 32 rows, 44 generated tokens by graph replay.

The acceptance rule: identical greedy token ids and 20 ms-grid timestamps wherever the oracle's top-2 logit margin
exceeds 1e-2. The engine decodes greedily (the captured step replayed, as the product does); the oracle is then
teacher-forced on the engine's sequences, and for every row, up to its first position where the oracle's margin is
at most 1e-2:

* every generated token equals the oracle's greedy choice (src/model.rs:650-736, kernels/whisper.cu:451-493 rules);
* every token's start time from the engine's alignment rows, computed on the device (the product's timestamp path),
  equals the one R.token_timestamps computes from the oracle's own cross-attention probabilities in the reference's
  fp16 arithmetic (src/transcribe.rs:147-162, src/align.rs:8-106);
* the fp16 alignment buffer (the reference's own, src/model.rs:455) holds the fp32 rows rounded to fp16, bit for bit,
  and the times a reference caller computes from it (download_h, then align.rs) equal the oracle's from its
  probabilities rounded to fp16.

Alignment that DTW can resolve. With random weights and random cross keys the alignment heads' rows are nearly
uniform (the largest probability ~0.01) and DTW on them is decided by differences at the level of the fp16 rounding
of the query: two correct evaluations disagree there (simulated on the host: 2 of 20 random tables move a time when
the scores get 1e-3 relative noise). Real alignment heads attend to a few frames that advance with the tokens. The
cross keys of the alignment heads are built that way: the positional embedding dominates the decoder's residual
(std 5, the token embedding std 0.03), so the query of position p of head (l, h) is close to
q_p = Wq_h LN_l(pe[p]) + bq_h; row b gives generated position p a block of tau_b frames (20..32, from a start
offset of 0..59) whose keys are 20 q_p / |q_p| plus N(0, 1) noise, and the other frames get keys N(0, 0.3^2). The
oracle's times then follow the blocks, and its rows survive 2e-3 relative noise with every time unchanged (simulated
on the host). The other heads keep N(0, 1) keys, the values are N(0, 1).
"""
import numpy as np
import pytest

from mimizuku_amd import _lib as L
from mimizuku_amd import model, synth, transcribe
from oracle import whisper_ref as R

pytestmark = pytest.mark.gpu

B, NP, GEN, TPAD, TENC = 32, 4, 44, 1536, 1500
G = synth.Geometry(d=1280, ff=5120, nh=20, enc_layers=1, dec_layers=4, n_mels=128, vocab=51866)
AH = [[2, 4], [2, 11], [3, 3], [3, 6], [3, 11], [3, 14]]  # large-v3-turbo's alignment heads
MARGIN = 1e-2


def test_greedy_tokens_and_timestamps_turbo_widths():
    rng = np.random.default_rng(31)
    W = synth.random_weights(G, seed=8, bias_std=0.02, ln_std=0.1)
    pe_key, emb_key = "model.decoder.embed_positions.weight", "model.decoder.embed_tokens.weight"
    W[pe_key] = (rng.standard_normal(W[pe_key].shape, dtype=np.float32) * 5).astype(np.float16)
    W[emb_key] = (rng.standard_normal(W[emb_key].shape, dtype=np.float32) * 0.03).astype(np.float16)
    Wf = {k: v.astype(np.float32) for k, v in W.items() if k.startswith("model.decoder")}
    gen = synth.generation_config(G, align_heads=AH)
    sup, bsup, eos = set(gen["suppress_tokens"]), gen["begin_suppress_tokens"], gen["eos_token_id"]
    dims = model.Dims(G.d, G.ff, G.nh, G.enc_layers, G.dec_layers, G.n_mels, G.vocab, G.max_t)
    gc = model.GenCfg.from_dict(gen, dims)

    # the query direction of every generated position, per alignment layer (from the positional embedding alone)
    qdir = {}
    for l in sorted({l for l, _ in AH}):
        pre = f"model.decoder.layers.{l}"
        x = R.layer_norm(Wf[pe_key][NP:NP + GEN], Wf[f"{pre}.encoder_attn_layer_norm.weight"],
                         Wf[f"{pre}.encoder_attn_layer_norm.bias"])
        qdir[l] = R.linear(x, Wf[f"{pre}.encoder_attn.q_proj.weight"], Wf[f"{pre}.encoder_attn.q_proj.bias"])
    xkv = np.zeros((B, G.dec_layers, 2, G.nh, TPAD, 64), np.float16)
    blocks = []
    for b in range(B):
        xkv[b, :, :, :, :TENC] = rng.standard_normal((G.dec_layers, 2, G.nh, TENC, 64), dtype=np.float32)
        tau, s0 = int(rng.integers(20, 33)), int(rng.integers(0, 60))
        blocks.append((s0, tau))
        for l, h in AH:
            k = rng.standard_normal((TENC, 64), dtype=np.float32) * 0.3
            for j in range(GEN):
                q = qdir[l][j, h * 64:(h + 1) * 64]
                k[s0 + j * tau:s0 + (j + 1) * tau] = 20 * q / np.linalg.norm(q) + \
                    rng.standard_normal((tau, 64), dtype=np.float32)
            xkv[b, l, 0, h, :TENC] = k
    prompts = rng.integers(0, 50000, size=(B, NP)).astype(np.int32)

    # the engine: greedy decoding by replaying the captured step
    ctx = model.Context(0)
    e = model.Engine(ctx, dims, gc, B, 8)
    e.load(W)
    p, n = e.buffer(L.BUF_XKV)
    assert n >= xkv.nbytes
    ctx.upload(p, xkv)
    cross = [[(xkv[b, l, 0, :, :TENC].astype(np.float32), xkv[b, l, 1, :, :TENC].astype(np.float32))
              for l in range(G.dec_layers)] for b in range(B)]
    del xkv
    e.reset(prompts)
    e.capture(B, NP)
    for _ in range(NP + GEN - 1):
        e.replay()
    toks = e.tokens()[:B, :NP + GEN].copy()
    assert np.array_equal(toks[:, :NP], prompts)
    assert not e.done()[:B].any(), "a row finished early: the comparison assumes 44 generated tokens"
    na = len(AH)
    ap, _ = e.buffer(L.BUF_ALIGN)
    rows = np.full(B, GEN - 1, np.int32)  # the generated tokens fed back: positions NP .. NP + GEN - 2
    ts_dev = transcribe.jump_times_device(ctx, ap + NP * na * TENC * 4, G.max_t * na * TENC, rows,
                                          np.full(B, TENC, np.int32), na, TENC, 7, True)
    al = e.align()[:B, NP:NP + GEN - 1].astype(np.float32)  # [B][rows][slots][1500]
    # the fp16 rows of the reference's own buffer (src/model.rs:455): the fp32 rows rounded, bit for bit
    ah = e.read(L.BUF_ALIGN_H, np.float16, (B, G.max_t, na, TENC))
    np.testing.assert_array_equal(ah[:, NP:NP + GEN - 1].view(np.uint16), al.astype(np.float16).view(np.uint16))
    ah = ah[:, NP:NP + GEN - 1].astype(np.float32)
    e.close()
    ctx.close()

    # the oracle, teacher-forced on the engine's sequences
    dec = R.Decoder(Wf, G.nh, G.dec_layers, cross)
    probs = np.zeros((B, NP + GEN, na, TENC), np.float32)
    margin = np.full((B, NP + GEN), np.inf)
    choice = np.zeros((B, NP + GEN), np.int64)
    for pos in range(NP + GEN - 1):
        ref, pr = dec.step(toks[:, pos].tolist(), pos)
        for s, (l, h) in enumerate(AH):
            probs[:, pos, s] = pr[:, l, h]
        if pos >= NP - 1:
            first = pos + 1 == NP
            for b in range(B):
                margin[b, pos + 1] = R.top2_margin(ref[b], sup, bsup, first)
                choice[b, pos + 1] = R.choose(ref[b], sup, bsup, first, eos, False)
    # the engine's alignment rows against the oracle's (as test_decoder_turbo_widths_batch32)
    worst_al = float(np.max(np.abs(al - probs[:, NP:NP + GEN - 1]) / probs[:, NP:NP + GEN - 1].max(-1, keepdims=True)))
    assert worst_al < 2e-3, worst_al

    tok_checked = ts_checked = ts_equal_all = 0
    for b in range(B):
        low = np.nonzero(margin[b, NP:NP + GEN] <= MARGIN)[0]
        span = int(low[0]) if len(low) else GEN  # generated tokens before the first low-margin position
        np.testing.assert_array_equal(toks[b, NP:NP + span], choice[b, NP:NP + span], err_msg=f"row {b} tokens")
        tok_checked += span
        ts_ref = R.token_timestamps(probs[b][:, :, None], [(s, 0) for s in range(na)], NP, NP + GEN, 2 * TENC,
                                    half=True)[NP:NP + GEN - 1]
        k = min(span, GEN - 1)
        np.testing.assert_array_equal(ts_dev[b][:k], ts_ref[:k], err_msg=f"row {b} timestamps (blocks {blocks[b]})")
        ts_checked += k
        ts_equal_all += int(np.sum(ts_dev[b] == ts_ref))
        # a caller that keeps src/transcribe.rs:147-162 as it is: the fp16 rows (download_h) into align.rs's
        # arithmetic, against the oracle's probabilities rounded to fp16 as the reference's kernel rounds them
        ts_h = transcribe.jump_times(ah[b], TENC, 7, True)
        probs_h = probs[b].astype(np.float16).astype(np.float32)
        ts_href = R.token_timestamps(probs_h[:, :, None], [(s, 0) for s in range(na)], NP, NP + GEN, 2 * TENC,
                                     half=True)[NP:NP + GEN - 1]
        np.testing.assert_array_equal(ts_h[:k], ts_href[:k], err_msg=f"row {b} timestamps from fp16 rows")
    print(f"turbo widths, 32 rows x {GEN} generated tokens (graph replay): tokens equal to the oracle's choices at "
          f"{tok_checked} positions, timestamps equal at {ts_checked} rows before each row's first margin <= "
          f"{MARGIN} ({ts_equal_all} of {B * (GEN - 1)} rows equal over the whole table); alignment rows max error "
          f"{worst_al:.2e} x the row's largest probability")
    assert tok_checked >= 8 * B  # on average at least 8 generated positions per row before a low margin
