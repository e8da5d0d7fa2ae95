"""The greedy-choice rules through the device kernels (dec_lmhead_kernel's per-workgroup partials and
dec_argmax_kernel), the engine's batch limits, and graph replay at the benchmark's decoder shape.

The rules are kernels/whisper.cu:451-493 (argmax_tok): positions inside the prompt keep their token; suppressed ids
are never chosen; the begin-suppressed ids only at the first generated position (p + 1 == prompt_len); ties go to
the lowest id; a finished row, or one whose every id is masked, gets eos and is marked done. Each check compares
the token the kernels wrote with the oracle's `choose` applied to the logits the same step wrote (bit-exact: the
choice is a pure function of the fp32 logits), on cases built so that each rule decides the outcome:

* ties: embed_tokens rows duplicated (the tied LM head then gives equal logits, checked bit for bit) in other
  LM-head workgroups below and above the natural winner, and in its own 16-id tile;
* an all-suppressed vocabulary: eos at the first generated position, then eos again for the finished row;
* a row marked done from the host before a step: eos, whatever its logits;
* begin-suppress: a natural first choice in the list is replaced by the runner-up, while a later natural choice in
  the list stands.
"""
import numpy as np
import pytest

from mimizuku_amd import _lib as L
from mimizuku_amd import model, synth
from mimizuku_amd._lib import MzError
from oracle import whisper_ref as R

pytestmark = pytest.mark.gpu

G = synth.TINY
TPAD = 1536
NP = 4
EOS = 50257


@pytest.fixture(scope="module")
def ctx():
    c = model.Context(0)
    yield c
    c.close()


@pytest.fixture(scope="module")
def setup():
    rng = np.random.default_rng(31)
    W = synth.random_weights(G, seed=3, bias_std=0.02, ln_std=0.1)
    B = 8
    xkv = np.zeros((B, G.dec_layers, 2, G.nh, TPAD, 64), np.float16)
    xkv[..., :1500, :] = rng.standard_normal((B, G.dec_layers, 2, G.nh, 1500, 64), dtype=np.float32)
    prompts = rng.integers(0, 50000, size=(B, NP)).astype(np.int32)
    return W, xkv, prompts


def make_engine(ctx, W, xkv, gen, bmax):
    dims = model.Dims(G.d, G.ff, G.nh, G.enc_layers, G.dec_layers, G.n_mels, G.vocab, G.max_t)
    gc = model.GenCfg.from_dict(gen, dims)
    e = model.Engine(ctx, dims, gc, bmax, min(bmax, 8))
    e.load(W)
    p, n = e.buffer(L.BUF_XKV)
    rows = np.concatenate([xkv] * (bmax // len(xkv)) + [xkv[:bmax % len(xkv)]])
    assert n >= rows.nbytes
    ctx.upload(p, rows)
    return e, gc


def run_checked(e, gc, prompts, steps, first_pos=NP):
    """Steps the engine, checking every chosen token against choose() on the step's own logits; returns the tokens
    [rows][steps + 1] from position NP - 1 on and the logits of the first generated position."""
    b = prompts.shape[0]
    e.reset(prompts)
    sup, bs = set(gc.suppress), list(gc.begin_suppress)
    first_logits = None
    for p in range(steps):
        done_before = e.done()[:b].copy()
        e.step(b, False, NP)
        if p + 1 < NP:
            assert np.array_equal(e.tokens()[:b, p + 1], prompts[:, p + 1])  # the prompt stays
            continue
        lg = e.logits()[:b]
        if p + 1 == first_pos:
            first_logits = lg.copy()
        toks = e.tokens()[:b, p + 1]
        for r in range(b):
            want = R.choose(lg[r], sup, bs, p + 1 == NP, gc.eos, bool(done_before[r]))
            assert toks[r] == want, (p, r, toks[r], want)
        assert np.array_equal(e.done()[:b], (done_before != 0) | (toks == gc.eos))
    return e.tokens()[:b, NP - 1:NP + steps - NP + 1], first_logits


def test_choice_rules_on_the_device(ctx, setup):
    W, xkv, prompts = setup
    gen = synth.generation_config(G)
    e, gc = make_engine(ctx, W, xkv, gen, len(prompts))
    toks, lg0 = run_checked(e, gc, prompts, NP + 3)
    g1, g2 = toks[:, 1], toks[:, 2]  # first and second generated tokens of every row

    # a row marked done from the host before the first generated position gets eos
    e.reset(prompts)
    for _ in range(NP - 1):
        e.step(len(prompts), False, NP)
    pd, _ = e.buffer(L.BUF_DONE)
    marked = np.zeros(len(prompts), np.int32)
    marked[1] = 1
    ctx.upload(pd, marked)
    e.step(len(prompts), False, NP)
    t = e.tokens()[:len(prompts), NP]
    assert t[1] == EOS and np.array_equal(np.delete(t, 1), np.delete(g1, 1)), (t, g1)
    e.close()

    # begin-suppress: row 0's natural first choice is suppressed at the first generated position (the runner-up
    # follows); a row r whose natural second choice is in the list keeps it there (not the first generated
    # position). Row r is one whose first choice the new list leaves unchanged, so its second step sees the same
    # history and logits as before.
    sup = set(gen["suppress_tokens"])
    cands = [i for i in range(1, len(prompts)) if g2[i] not in (g1[i], g1[0], EOS) and
             R.choose(lg0[i], sup, [int(g1[0]), int(g2[i])], True, EOS, False) == g1[i]]
    assert cands, (g1, g2)
    r = cands[0]
    gen_bs = dict(gen, begin_suppress_tokens=[int(g1[0]), int(g2[r])])
    e, gc = make_engine(ctx, W, xkv, gen_bs, len(prompts))
    toks_b, lg_b = run_checked(e, gc, prompts, NP + 2)
    assert np.array_equal(lg_b, lg0)  # same model, same inputs: the list changes only the choice
    assert toks_b[0, 1] != g1[0]
    assert toks_b[r, 1] == g1[r] and toks_b[r, 2] == g2[r], (toks_b[r], g1[r], g2[r])
    e.close()


def test_ties_go_to_the_lowest_id(ctx, setup):
    W, xkv, prompts = setup
    gen = synth.generation_config(G)
    sup = set(gen["suppress_tokens"]) | set(gen["begin_suppress_tokens"]) | set(prompts.ravel().tolist())
    e, gc = make_engine(ctx, W, xkv, gen, len(prompts))
    _, lg0 = run_checked(e, gc, prompts, NP)
    e.close()
    w = int(R.choose(lg0[0], set(gen["suppress_tokens"]), gen["begin_suppress_tokens"], True, EOS, False))

    def free(c):
        while c in sup or c == w:
            c += 1
        return c if c < G.vocab else None
    # copies of row w: its neighbour in the same 16-id tile, one far above (another LM-head workgroup), and in a
    # second engine also one far below
    mate = w ^ 1 if (w ^ 1) not in sup and (w ^ 1) < G.vocab else None
    hi = free(w + (G.vocab - w) // 2) if w < G.vocab - 600 else None
    lo = free(w // 3) if w > 600 else None
    for copies in ([mate, hi], [lo, mate, hi]):
        copies = [c for c in copies if c is not None]
        W2 = dict(W)
        emb = W["model.decoder.embed_tokens.weight"].copy()
        for c in copies:
            emb[c] = emb[w]
        W2["model.decoder.embed_tokens.weight"] = emb
        e, gc = make_engine(ctx, W2, xkv, gen, len(prompts))
        _, lg = run_checked(e, gc, prompts, NP)
        assert all(lg[0, c] == lg[0, w] for c in copies)  # equal rows give bit-equal logits
        assert e.tokens()[0, NP] == min(copies + [w]), (e.tokens()[0, NP], w, copies)
        e.close()


def test_all_suppressed_vocabulary_gives_eos(ctx, setup):
    W, xkv, prompts = setup
    gen = dict(synth.generation_config(G), suppress_tokens=list(range(G.vocab)))
    e, gc = make_engine(ctx, W, xkv, gen, len(prompts))
    toks, _ = run_checked(e, gc, prompts, NP + 2)
    assert np.all(toks[:, 1:] == EOS), toks
    assert np.all(e.done()[:len(prompts)] == 1)
    e.close()


def test_batch_above_32_rows(ctx, setup):
    """40 rows: the LM head's second 32-row block. Rows 32..39 repeat rows 0..7's prompts and cross keys/values, so
    their logits and tokens equal those rows' bit for bit, and every choice follows the rules."""
    W, xkv, prompts = setup
    gen = synth.generation_config(G)
    B = 40
    pr = np.concatenate([prompts] * (B // len(prompts)))
    e, gc = make_engine(ctx, W, xkv, gen, B)
    toks, lg = run_checked(e, gc, pr, NP + 2)
    assert np.array_equal(lg[32:40], lg[0:8])
    assert np.array_equal(toks[32:40], toks[0:8])
    e.close()


def test_widths_above_1280_are_refused(ctx):
    dims = model.Dims(1408, 5632, 22, 2, 2, 128, 51866, 448)
    gen = synth.generation_config(synth.Geometry(1408, 5632, 22, 2, 2, 128, 51866), align_heads=[[1, 0]])
    with pytest.raises(MzError, match="1280"):
        model.Engine(ctx, dims, model.GenCfg.from_dict(gen, dims), 4, 4)


def test_graph_replay_bit_identical_at_the_bench_shape(ctx):
    """large-v3-turbo widths, 32 rows at positions 200..202 (a random self-attention cache of 200 positions): three
    replays of the captured step write the same logits, tokens, cache rows and alignment rows as three eager steps,
    bit for bit."""
    g = synth.Geometry(d=1280, ff=5120, nh=20, enc_layers=1, dec_layers=4, n_mels=128, vocab=51866)
    rng = np.random.default_rng(41)
    W = synth.random_weights(g, seed=12, bias_std=0.02, ln_std=0.1)
    gen = synth.generation_config(g, align_heads=[[2, 4], [2, 11], [3, 3], [3, 6], [3, 11], [3, 14]])
    dims = model.Dims(g.d, g.ff, g.nh, g.enc_layers, g.dec_layers, g.n_mels, g.vocab, g.max_t)
    gc = model.GenCfg.from_dict(gen, dims)
    B, P0 = 32, 200
    e = model.Engine(ctx, dims, gc, B, 8)
    e.load(W)
    px, n = e.buffer(L.BUF_XKV)
    xkv = np.zeros((B, g.dec_layers, 2, g.nh, TPAD, 64), np.float16)
    xkv[..., :1500, :] = rng.standard_normal((B, g.dec_layers, 2, g.nh, 1500, 64), dtype=np.float32)
    ctx.upload(px, xkv)
    del xkv
    kv_shape = (g.dec_layers, B, g.nh, g.max_t, 64)
    for which in (L.BUF_SELF_K, L.BUF_SELF_V):
        p, n = e.buffer(which)
        ctx.upload(p, rng.standard_normal(kv_shape, dtype=np.float32).astype(np.float16))
    toks = np.zeros((B, g.max_t), np.int32)
    toks[:, :P0 + 1] = rng.integers(0, 50000, size=(B, P0 + 1))
    pt, _ = e.buffer(L.BUF_TOK)
    pd, _ = e.buffer(L.BUF_DONE)
    pc, _ = e.buffer(L.BUF_CTR)

    def start():
        e.reset(toks[:, :1])  # prompt length 1: every later position is chosen
        ctx.upload(pt, toks)
        ctx.upload(pd, np.zeros(B, np.int32))
        ctx.upload(pc, np.array([P0, 0, 0, 0], np.int32))

    def outputs(i):
        """What step i (position P0 + i) wrote."""
        kc, vc = e.self_kv()
        return [e.logits(), e.tokens(), e.done(), kc[:, :, :, P0 + i].copy(), vc[:, :, :, P0 + i].copy(),
                e.align()[:, P0 + i].copy(), e.dec_x()]

    start()
    eager = []
    for i in range(3):
        e.step(B, False, 1)
        eager.append(outputs(i))
    start()
    e.capture(B, 1)
    for i in range(3):
        e.replay()
        ctx.sync()
        got = outputs(i)
        for k, (a, b) in enumerate(zip(got, eager[i])):
            assert np.array_equal(a, b), (i, k)
    assert e.position() == P0 + 3
    e.close()
