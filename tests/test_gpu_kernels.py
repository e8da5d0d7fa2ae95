"""GPU parity of the individual kernels through the C ABI, against float64 closed forms on the same fp16 inputs (or
the oracle's functions), at small shapes and at the full large-v3 shapes with subsampled checks.

Tolerances: an fp16 output is the exact result rounded to fp16 within one ulp (assert_f16); an fp32 output within
max-abs error <= 2e-3 x RMS of the reference; the attention output (whose P operand the kernel rounds to fp16) within
the larger of that and 1.5 x the error of the same attention computed exactly but with fp16 probabilities.
"""
import numpy as np
import pytest

from mimizuku_amd import _lib as L
from mimizuku_amd import model
from oracle import whisper_ref as R

pytestmark = pytest.mark.gpu

TOL = 2e-3
TPAD = 1536


@pytest.fixture(scope="module")
def ctx():
    c = model.Context(0)
    yield c
    c.close()


def rel_err(got, ref):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    return np.abs(got - ref).max() / np.sqrt((ref ** 2).mean())


def assert_f16(got, ref, ulps=1.0):
    """An fp16 output must be the exact value rounded to fp16, within `ulps` units in the last place of that value
    (correct rounding is half an ulp; fp32 accumulation order may flip a rounding), plus 1e-5 x RMS for results that
    cancel to near zero."""
    ref = np.asarray(ref, np.float64)
    got = np.asarray(got, np.float64)
    ulp = np.spacing(np.abs(ref).astype(np.float16)).astype(np.float64)
    bound = ulps * ulp + 1e-5 * np.sqrt((ref ** 2).mean())
    bad = np.abs(got - ref) > bound
    assert not bad.any(), f"{bad.sum()} of {bad.size} outside {ulps} ulp: worst at {np.argwhere(bad)[:3].tolist()}"


def f16(rng, shape, scale=1.0):
    return (rng.standard_normal(shape, dtype=np.float32) * scale).astype(np.float16)


# ---------------------------------------------------------------- encoder attention

def pack_qkvh(q, k, v):
    """q, k, v [G][nh][1500][64] fp16 -> [G][3][nh][1536 * 64] with v transposed, zero padded."""
    G, nh = q.shape[:2]
    out = np.zeros((G, 3, nh, TPAD * 64), np.float16)
    for a, x in enumerate((q, k)):
        t = np.zeros((G, nh, TPAD, 64), np.float16)
        t[:, :, :1500] = x
        out[:, a] = t.reshape(G, nh, -1)
    t = np.zeros((G, nh, 64, TPAD), np.float16)
    t[:, :, :, :1500] = v.transpose(0, 1, 3, 2)
    out[:, 2] = t.reshape(G, nh, -1)
    return out


QSCALE = 0.125 * np.log2(np.e)  # the QKV product stores q multiplied by the attention's exponent scale


def prescaled(q):
    """(q as the QKV product stores it: fp16(q x log2(e) / 8), the query that stored value stands for) - the kernel's
    input and the reference's."""
    qs = (q.astype(np.float64) * QSCALE).astype(np.float16)
    return qs, qs.astype(np.float64) / QSCALE


def run_attention(ctx, qs, k, v):
    """qs: prescaled(q)[0]"""
    G, nh = qs.shape[:2]
    dq = ctx.upload_new(pack_qkvh(qs, k, v))
    do = ctx.alloc(G * 1500 * nh * 64 * 2)
    L.check(L.lib().mz_enc_attention(ctx.h, dq, do, G, nh))
    out = ctx.download(do, (G, 1500, nh, 64), np.float16)
    ctx.free(dq)
    ctx.free(do)
    return out.transpose(0, 2, 1, 3)  # [G][nh][1500][64]


def attention64(q, k, v):
    return R.attention(q, k, v, 0.125, dtype=np.float64)


def attention_p16(q, k, v):
    """The fp16-probability arithmetic the kernel (and the reference's fused attention) uses, otherwise exact:
    P = fp16(exp(s - max)), O = fp16(P v / sum P)."""
    s = (q.astype(np.float64) * 0.125) @ np.swapaxes(k.astype(np.float64), -1, -2)
    p = np.exp(s - s.max(-1, keepdims=True)).astype(np.float16).astype(np.float64)
    return ((p @ v.astype(np.float64)) / p.sum(-1, keepdims=True)).astype(np.float16)


def attention_bar(q, k, v, ref):
    """Error bar of an fp16-probability attention: the larger of TOL and 1.5 x the error of attention_p16, whose fp16
    rounding of P and of the output alone reaches about 2e-3 x RMS on near-uniform softmaxes. The max-abs metric
    moves by about +-25% with where the running max stands when each P is rounded (blockwise vs exact max)."""
    return max(TOL, 1.5 * rel_err(attention_p16(q, k, v), ref))


def test_enc_attention_small(ctx):
    rng = np.random.default_rng(10)
    q, k, v = (f16(rng, (1, 2, 1500, 64)) for _ in range(3))
    qs, q = prescaled(q)
    out = run_attention(ctx, qs, k, v)
    ref = attention64(q, k, v)
    assert rel_err(out, ref) < attention_bar(q, k, v, ref)
    # a transposed V (a plausible layout mistake) is far outside the bar
    assert rel_err(out, attention64(q, k, v[..., ::-1])) > 0.1


def test_enc_attention_peaked_scores(ctx):
    """Large logits (scale 4 x N(0,1) inputs): the online max/rescale path dominates."""
    rng = np.random.default_rng(11)
    q, k = f16(rng, (1, 1, 1500, 64), 4.0), f16(rng, (1, 1, 1500, 64), 4.0)
    v = f16(rng, (1, 1, 1500, 64))
    qs, q = prescaled(q)
    out = run_attention(ctx, qs, k, v)
    ref = attention64(q, k, v)
    assert rel_err(out, ref) < attention_bar(q, k, v, ref)


def test_enc_attention_late_peak(ctx):
    """Every query's largest scores far past the running max in late blocks: a peak at key 700 and a dominant one at
    key 1490 (the padded last tile, whose keys past 1500 are masked), so each of those blocks is recomputed against
    a raised max with O rescaled (its probabilities would sum far past 2^12, or overflow fp16, otherwise)."""
    rng = np.random.default_rng(13)
    q, k, v = (f16(rng, (1, 2, 1500, 64)) for _ in range(3))
    c = np.full(64, 1.0, np.float32)
    q = (q.astype(np.float32) + c).astype(np.float16)
    k = k.astype(np.float32)
    k[:, :, 700] += 3.0 * c
    k[:, :, 1490] += 6.0 * c
    k = k.astype(np.float16)
    qs, q = prescaled(q)
    out = run_attention(ctx, qs, k, v)
    ref = attention64(q, k, v)
    assert rel_err(out, ref) < attention_bar(q, k, v, ref)
    # the output is dominated by v[1490] (a kernel that missed the late peak would not be)
    assert rel_err(out, np.broadcast_to(v[:, :, 1490:1491].astype(np.float64), out.shape)) < 0.05


def test_enc_attention_large_v3_shape(ctx):
    """8 clips x 20 heads x 1500 x 1500, head 64 (the encoder group's attention); every (clip, head) checked on 48
    query rows spread over the window, including the last ones of the padded tile."""
    rng = np.random.default_rng(12)
    shape = (8, 20, 1500, 64)
    q, k, v = (f16(rng, shape) for _ in range(3))
    qs, q = prescaled(q)
    out = run_attention(ctx, qs, k, v)
    rows = np.r_[np.arange(0, 1500, 37), 1496, 1497, 1498, 1499]
    ref = attention64(q[:, :, rows], k, v)
    assert rel_err(out[:, :, rows], ref) < attention_bar(q[:, :, rows], k, v, ref)
    assert np.isfinite(out).all()


# ---------------------------------------------------------------- GEMMs

def linear_args(**kw):
    a = L.LinearArgs()
    for k_, v_ in kw.items():
        setattr(a, k_, v_)
    return a


@pytest.mark.parametrize("m,n,k", [(1, 64, 64), (7, 100, 384), (32, 1280, 1280), (33, 96, 128), (3000, 768, 384),
                                   (1500, 1284, 448)])
def test_gemm_f16(ctx, m, n, k):
    rng = np.random.default_rng(m * 7 + n)
    x, w, b = f16(rng, (m, k)), f16(rng, (n, k), 0.05), f16(rng, (n,), 0.1)
    dx, dw, db = ctx.upload_new(x), ctx.upload_new(w), ctx.upload_new(b)
    dy = ctx.alloc(m * n * 2)
    L.check(L.lib().mz_gemm(ctx.h, dx, k, dw, dy, n, m, n, k, db))
    y = ctx.download(dy, (m, n), np.float16)
    ref = x.astype(np.float64) @ w.astype(np.float64).T + b
    assert_f16(y, ref)
    for p in (dx, dw, db, dy):
        ctx.free(p)


def test_gemm_epilogues(ctx):
    rng = np.random.default_rng(3)
    m, n, k = 3000, 512, 640
    x, w, b = f16(rng, (m, k)), f16(rng, (n, k), 0.05), f16(rng, (n,), 0.1)
    res = rng.standard_normal((m, n)).astype(np.float32)
    pos = f16(rng, (1500, n))
    acc = x.astype(np.float64) @ w.astype(np.float64).T + b
    dx, dw, db, dpos = (ctx.upload_new(a) for a in (x, w, b, pos))
    # GELU -> fp16
    dy = ctx.alloc(m * n * 2)
    L.check(L.lib().mz_linear(ctx.h, linear_args(epilogue=L.EPI_GELU_F16, a=dx, lda=k, w=dw, bias=db, m=m, n=n, k=k,
                                                 out=dy, ldo=n)))
    assert_f16(ctx.download(dy, (m, n), np.float16), R.gelu(acc.astype(np.float32)))
    # residual add into fp32
    dr = ctx.upload_new(res)
    L.check(L.lib().mz_linear(ctx.h, linear_args(epilogue=L.EPI_RESID_F32, a=dx, lda=k, w=dw, bias=db, m=m, n=n, k=k,
                                                 out=dr, ldo=n)))
    got = ctx.download(dr, (m, n), np.float32)
    ref = res + acc
    assert rel_err(got, ref) < 1e-5
    # GELU + positions (the conv2 epilogue) exists only on the implicit-conv load: refused on a plain product
    with pytest.raises(L.MzError):
        L.check(L.lib().mz_linear(ctx.h, linear_args(epilogue=L.EPI_GELU_POS, a=dx, lda=k, w=dw, bias=db, m=m, n=n,
                                                     k=k, out=dr, ldo=n, pos=dpos)))
    for p in (dx, dw, db, dpos, dy, dr):
        ctx.free(p)


def test_gemm_gelu_every_fp16_value(ctx):
    """The GELU epilogue on every finite fp16 input: row m of x holds value m in column 0 and w is 1 there, so each
    accumulator is exactly that value; no bias (a missing bias reads zeros). Against 0.5 v erfc(-v / sqrt 2) in float64:
    within 0.6 fp16 ulp everywhere (0.505 measured, at v = 0.0036; an emulation of the fp32 arithmetic on the host
    gives the same, with exp2 correctly rounded or one ulp off) and correctly rounded for all but a few hundred values
    (164 measured; 157-171 in the emulation). Every column of a row is the same value, and the 64 columns cover both
    the whole-block and the column-checked stores."""
    from scipy.special import erfc
    v = np.arange(65536, dtype=np.uint32).astype(np.uint16).view(np.float16)
    v = v[np.isfinite(v)]
    m, n, k = v.size, 64, 64
    x = np.zeros((m, k), np.float16)
    x[:, 0] = v
    w = np.zeros((n, k), np.float16)
    w[:, 0] = 1
    dx, dw = ctx.upload_new(x), ctx.upload_new(w)
    dy = ctx.alloc(m * n * 2)
    L.check(L.lib().mz_linear(ctx.h, linear_args(epilogue=L.EPI_GELU_F16, a=dx, lda=k, w=dw, m=m, n=n, k=k, out=dy,
                                                 ldo=n)))
    y = ctx.download(dy, (m, n), np.float16)
    for p in (dx, dw, dy):
        ctx.free(p)
    bits = y.view(np.uint16)
    assert (bits == bits[:, :1]).all()
    vd = v.astype(np.float64)
    ref = 0.5 * vd * erfc(-vd / np.sqrt(2))
    got = y[:, 0].astype(np.float64)
    ulp = 2.0 ** (np.maximum(np.floor(np.log2(np.maximum(np.abs(ref), 1e-300))), -14) - 10)
    err = np.abs(got - ref) / ulp
    sub = np.abs(vd) < 2.0 ** -14  # fp16 subnormal inputs (and zeros)
    worst = int(np.argmax(err))
    print("GELU over %d fp16 values: max %.3f ulp at v = %g; %d not correctly rounded" %
          (v.size, err[worst], vd[worst], int((y[:, 0] != ref.astype(np.float16)).sum())))
    assert err[~sub].max() <= 0.6, ("normal inputs", vd[~sub][np.argmax(err[~sub])])
    assert err[sub].max() <= 0.6, ("subnormal inputs", vd[sub][np.argmax(err[sub])])
    assert (y[:, 0] != ref.astype(np.float16)).sum() < 300


@pytest.mark.parametrize("kind", [3, 2])
def test_gemm_head_scatter(ctx, kind):
    """kind 3: [q|k|v][head] tiles of the encoder self-attention (v tiles transposed, q tiles multiplied by
    log2(e) / 8); kind 2: [layer][k|v][head] of the cross k/v (all tiles row-major); both into clip slots (slot0
    offset)."""
    rng = np.random.default_rng(kind)
    nh, clips, slot0 = 2, 2, 1
    groups = 3 if kind == 3 else 2 * 2  # kind 2: two decoder layers
    n, k, m = groups * nh * 64, 128, clips * 1500
    x, w, b = f16(rng, (m, k)), f16(rng, (n, k), 0.1), f16(rng, (n,), 0.1)
    dx, dw, db = (ctx.upload_new(a) for a in (x, w, b))
    bpc = groups * nh
    nslots = slot0 + clips + 1  # one slot past the call's clips, which must stay untouched
    dh = ctx.alloc(nslots * bpc * TPAD * 64 * 2)
    L.check(L.lib().mz_linear(ctx.h, linear_args(epilogue=L.EPI_HEADS, a=dx, lda=k, w=dw, bias=db, m=m, n=n, k=k,
                                                 heads=dh, blocks_per_clip=bpc, nh=nh, kind=kind, slot0=slot0)))
    got = ctx.download(dh, (nslots, bpc, TPAD * 64), np.float16)
    ref = (x.astype(np.float64) @ w.astype(np.float64).T + b).reshape(clips, 1500, bpc, 64)
    if kind == 3:
        ref[:, :, :nh] *= QSCALE
    assert not got[:slot0].any(), "a slot before slot0 was written"
    assert not got[slot0 + clips:].any(), "a slot after the last clip was written"
    for c in range(clips):
        for blk in range(bpc):
            tile = got[slot0 + c, blk]
            if kind == 3 and blk // nh == 2:  # encoder v: [64][1536]
                t = tile.reshape(64, TPAD)
                assert not t[:, 1500:].any()
                assert_f16(t[:, :1500].T, ref[c, :, blk])
            else:
                t = tile.reshape(TPAD, 64)
                assert not t[1500:].any()
                assert_f16(t[:1500], ref[c, :, blk])
    for p in (dx, dw, db, dh):
        ctx.free(p)


def test_gemm_large_qkv_shape(ctx):
    """The encoder group's fused QKV product, M = 12000, N = 3840, K = 1280, 256 rows checked."""
    rng = np.random.default_rng(5)
    m, n, k = 12000, 3840, 1280
    x, w, b = f16(rng, (m, k)), f16(rng, (n, k), 0.02), f16(rng, (n,), 0.02)
    dx, dw, db = (ctx.upload_new(a) for a in (x, w, b))
    dy = ctx.alloc(m * n * 2)
    L.check(L.lib().mz_gemm(ctx.h, dx, k, dw, dy, n, m, n, k, db))
    y = ctx.download(dy, (m, n), np.float16)
    rows = np.r_[rng.choice(m, 250, replace=False), m - 6:m]
    ref = x[rows].astype(np.float64) @ w.astype(np.float64).T + b
    assert_f16(y[rows], ref)
    for p in (dx, dw, db, dy):
        ctx.free(p)


@pytest.mark.parametrize("m,n,k", [(9000, 2304, 320), (12000, 768, 448), (6000, 1000, 192)])
def test_gemm_persistent_shapes(ctx, m, n, k):
    """Products with more tiles than CUs, so each workgroup of the persistent grid walks several tiles (requesting the
    next tile's first K tile before each epilogue): 256 x 256 tiles with a partial last block row and an odd count
    of 64-wide K tiles (9000 x 2304 x 320), 256 x 128 tiles (12000 x 768 x 448), 128 x 128 tiles with partial block
    rows and columns (6000 x 1000 x 192); fp16 output against float64 on sampled rows, and on the first shape also
    the GELU and fp32 residual epilogues."""
    rng = np.random.default_rng(m + n + k)
    x, w, b = f16(rng, (m, k)), f16(rng, (n, k), 0.05), f16(rng, (n,), 0.1)
    dx, dw, db = (ctx.upload_new(a) for a in (x, w, b))
    rows = np.r_[rng.choice(m, 300, replace=False), m - 40:m]
    acc = x[rows].astype(np.float64) @ w.astype(np.float64).T + b
    dy = ctx.alloc(m * n * 2)
    L.check(L.lib().mz_gemm(ctx.h, dx, k, dw, dy, n, m, n, k, db))
    assert_f16(ctx.download(dy, (m, n), np.float16)[rows], acc)
    if m == 9000:
        L.check(L.lib().mz_linear(ctx.h, linear_args(epilogue=L.EPI_GELU_F16, a=dx, lda=k, w=dw, bias=db, m=m, n=n,
                                                     k=k, out=dy, ldo=n)))
        assert_f16(ctx.download(dy, (m, n), np.float16)[rows], R.gelu(acc.astype(np.float32)))
        res = rng.standard_normal((m, n)).astype(np.float32)
        dr = ctx.upload_new(res)
        L.check(L.lib().mz_linear(ctx.h, linear_args(epilogue=L.EPI_RESID_F32, a=dx, lda=k, w=dw, bias=db, m=m, n=n,
                                                     k=k, out=dr, ldo=n)))
        got = ctx.download(dr, (m, n), np.float32)
        assert rel_err(got[rows], res[rows] + acc) < 1e-5
        ctx.free(dr)
    for p in (dx, dw, db, dy):
        ctx.free(p)


def test_conv_stem_implicit_gemm(ctx):
    """mel transpose + conv1 (k 3, pad 1) + GELU, conv2 (stride 2) + GELU + positions, against the oracle's conv1d."""
    rng = np.random.default_rng(6)
    nm, d, clips = 80, 384, 2
    mel = np.clip(rng.normal(-0.3, 0.4, (clips, nm, 3000)), -1.5, 1.5).astype(np.float32)
    w1, b1 = f16(rng, (d, nm, 3), 0.05), f16(rng, (d,), 0.05)
    w2, b2 = f16(rng, (d, d, 3), 0.02), f16(rng, (d,), 0.05)
    pos = f16(rng, (1500, d), 0.5)
    k1 = ((3 * nm + 63) // 64) * 64
    w1t = np.zeros((d, k1), np.float16)
    w1t[:, :3 * nm] = w1.transpose(0, 2, 1).reshape(d, 3 * nm)
    w2t = np.ascontiguousarray(w2.transpose(0, 2, 1).reshape(d, 3 * d))
    dmel = ctx.upload_new(mel)
    dmt = ctx.alloc(clips * 3000 * nm * 2)
    L.check(L.lib().mz_mel_transpose(ctx.h, dmel, dmt, clips, nm))
    mt = ctx.download(dmt, (clips, 3000, nm), np.float16)
    np.testing.assert_array_equal(mt, mel.transpose(0, 2, 1).astype(np.float16))
    dw1, db1, dw2, db2, dpos = (ctx.upload_new(a) for a in (w1t, b1, w2t, b2, pos))
    dh1 = ctx.alloc(clips * 3000 * d * 2)
    L.check(L.lib().mz_linear(ctx.h, linear_args(epilogue=L.EPI_GELU_F16, a=dmt, w=dw1, bias=db1, m=clips * 3000, n=d,
                                                 k=k1, out=dh1, ldo=d, conv_cin=nm, conv_tin=3000, conv_tout=3000,
                                                 conv_stride=1)))
    h1 = ctx.download(dh1, (clips, 3000, d), np.float16)
    dx = ctx.alloc(clips * 1500 * d * 4)
    L.check(L.lib().mz_linear(ctx.h, linear_args(epilogue=L.EPI_GELU_POS, a=dh1, w=dw2, bias=db2, m=clips * 1500, n=d,
                                                 k=3 * d, out=dx, ldo=d, pos=dpos, conv_cin=d, conv_tin=3000,
                                                 conv_tout=1500, conv_stride=2)))
    x = ctx.download(dx, (clips, 1500, d), np.float32)
    for c in range(clips):
        m16 = mel[c].astype(np.float16).astype(np.float64)
        r1 = R.gelu(R.conv1d(m16, w1.astype(np.float64), b1.astype(np.float64), 1, 1).astype(np.float32))
        assert_f16(h1[c].T, r1)
        # conv2 on the kernel's own fp16 conv1 output (layer-local)
        r2 = R.gelu(R.conv1d(h1[c].T.astype(np.float64), w2.astype(np.float64), b2.astype(np.float64), 2, 1)
                    .astype(np.float32)).T + pos.astype(np.float32)
        assert rel_err(x[c], r2) < 1e-4
    for p in (dmel, dmt, dw1, db1, dw2, db2, dpos, dh1, dx):
        ctx.free(p)


# ---------------------------------------------------------------- LayerNorm

@pytest.mark.parametrize("dim", [384, 1280, 2048])
def test_layernorm_and_add_layernorm(ctx, dim):
    rng = np.random.default_rng(dim)
    rows = 301
    x = (rng.standard_normal((rows, dim)) * 3 + 1).astype(np.float32)
    dlt = f16(rng, (rows, dim))
    w, b = f16(rng, (dim,), 0.1) + np.float16(1), f16(rng, (dim,), 0.1)
    dxx, dd, dw, db = (ctx.upload_new(a) for a in (x, dlt, w, b))
    dy = ctx.alloc(rows * dim * 2)
    L.check(L.lib().mz_layernorm(ctx.h, dxx, dim, dw, db, dy, dim, rows, dim, 1e-5))
    y = ctx.download(dy, (rows, dim), np.float16)
    assert_f16(y, R.layer_norm(x.astype(np.float64), w, b))
    L.check(L.lib().mz_add_layernorm(ctx.h, dxx, dd, dw, db, dy, rows, dim, 1e-5))
    xs = ctx.download(dxx, (rows, dim), np.float32)
    np.testing.assert_allclose(xs, x + dlt.astype(np.float32), rtol=0, atol=0)
    y = ctx.download(dy, (rows, dim), np.float16)
    assert_f16(y, R.layer_norm((x + dlt.astype(np.float32)).astype(np.float64), w, b))
    for p in (dxx, dd, dw, db, dy):
        ctx.free(p)


# ---------------------------------------------------------------- token timestamps (median filter + DTW)

def softmax_rows(rng, shape, peak=3.0):
    s = rng.standard_normal(shape) * peak
    w = np.exp(s - s.max(-1, keepdims=True))
    return (w / w.sum(-1, keepdims=True)).astype(np.float16).astype(np.float32)


@pytest.mark.parametrize("half", [False, True])
def test_timestamps_device_match_host_bits(ctx, half):
    """k_align.hip against the host routine mz_jump_times (itself pinned to the oracle and to the golden vectors):
    identical floats for every clip, with ragged row and column counts, clips without rows or columns, fewer
    columns than the filter's half width, constant columns (zero deviation) and a diagonal alignment."""
    from mimizuku_amd import transcribe
    rng = np.random.default_rng(11 + half)
    heads, full = 6, 1500
    rows = [40, 1, 0, 223, 17, 5, 60, 33]
    cols = [1500, 700, 300, 1500, 3, 0, 911, 64]
    rmax = max(rows)
    w = softmax_rows(rng, (len(rows), rmax, heads, full))
    w[4, :, 2, :] = 0.25                       # constant columns in one head
    for i in range(rows[6]):                   # a clean diagonal in clip 6
        w[6, i, :, 15 * i:15 * i + 15] += 0.5
    dw = ctx.upload_new(w)
    got = transcribe.jump_times_device(ctx, dw, rmax * heads * full, rows, cols, heads, full, 7, half)
    for c in range(len(rows)):
        ref = transcribe.jump_times(w[c, :rows[c]], cols[c], 7, half)
        np.testing.assert_array_equal(got[c], ref, err_msg=f"clip {c}")
        if 0 < rows[c] <= 40 and cols[c] <= 64:
            np.testing.assert_array_equal(got[c], R.jump_times(w[c, :rows[c]], cols[c], 7, half))


@pytest.mark.parametrize("rows,cols", [([255, 3, 128], [1500, 1500, 1]),      # one wave per clip, its largest table
                                       ([300, 256, 9], [1500, 1499, 77])])   # more rows than a wave holds
def test_timestamps_device_row_limits(ctx, rows, cols):
    """Tables at and past 256 rows, where the one-wave DTW hands over to the workgroup DTW: identical floats."""
    from mimizuku_amd import transcribe
    rng = np.random.default_rng(sum(rows))
    heads, full, rmax = 2, 1500, max(rows)
    w = softmax_rows(rng, (len(rows), rmax, heads, full))
    dw = ctx.upload_new(w)
    got = transcribe.jump_times_device(ctx, dw, rmax * heads * full, rows, cols, heads, full, 7, True)
    for c in range(len(rows)):
        np.testing.assert_array_equal(got[c], transcribe.jump_times(w[c, :rows[c]], cols[c], 7, True),
                                      err_msg=f"clip {c}")


def test_timestamps_device_nan_costs(ctx):
    """A column whose values overflow fp16 (0 and 2e5 alternating: mean and deviation round to inf, z = inf / inf)
    gives NaN DTW costs in half mode. The DTW must then choose its moves with the reference's comparisons as written
    (a NaN neighbour loses every comparison, align.rs:77-83), in the one-wave kernel (<= 255 rows) as in the
    workgroup kernel and the host routine: identical floats."""
    from mimizuku_amd import transcribe
    rng = np.random.default_rng(29)
    heads, full = 6, 1500
    rows, cols = [40, 255, 7, 300], [1500, 1500, 900, 1500]
    rmax = max(rows)
    w = softmax_rows(rng, (len(rows), rmax, heads, full))
    for c, col in enumerate((700, 1201, 450, 333)):
        w[c, 0::2, :, col] = 0.0
        w[c, 1::2, :, col] = 2e5
    for c in range(len(rows)):
        assert np.isnan(transcribe.align_cost(w[c, :rows[c]], cols[c], 7, True)).any(), f"clip {c}: no NaN cost"
    dw = ctx.upload_new(w)
    got = transcribe.jump_times_device(ctx, dw, rmax * heads * full, rows, cols, heads, full, 7, True)
    for c in range(len(rows)):
        np.testing.assert_array_equal(got[c], transcribe.jump_times(w[c, :rows[c]], cols[c], 7, True),
                                      err_msg=f"clip {c} ({rows[c]} rows)")


@pytest.mark.parametrize("full", [1500, 203])
def test_timestamps_device_column_layouts(ctx, full):
    """Rows of 1500 columns (four columns per thread in the column statistics) and of an odd count (one per thread):
    identical floats in both modes."""
    from mimizuku_amd import transcribe
    rng = np.random.default_rng(full)
    heads, rows, cols = 3, [12, 30, 7], [full, full - 1, full // 2]
    w = softmax_rows(rng, (3, 30, heads, full))
    dw = ctx.upload_new(w)
    for half in (False, True):
        got = transcribe.jump_times_device(ctx, dw, 30 * heads * full, rows, cols, heads, full, 7, half)
        for c in range(3):
            np.testing.assert_array_equal(got[c], transcribe.jump_times(w[c, :rows[c]], cols[c], 7, half),
                                          err_msg=f"clip {c} half {half}")


def test_timestamps_device_other_widths(ctx):
    from mimizuku_amd import transcribe
    rng = np.random.default_rng(5)
    heads, full, rows, cols = 3, 200, [12, 30], [200, 150]
    w = softmax_rows(rng, (2, 30, heads, full))
    dw = ctx.upload_new(w)
    for width in (1, 5, 9, 15):
        got = transcribe.jump_times_device(ctx, dw, 30 * heads * full, rows, cols, heads, full, width, True)
        for c in range(2):
            np.testing.assert_array_equal(got[c], transcribe.jump_times(w[c, :rows[c]], cols[c], width, True))
