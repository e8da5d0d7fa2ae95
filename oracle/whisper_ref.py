"""CPU oracle for the Whisper compute path — TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this module, and only as the
reference that device results are compared against (or the timed CPU baseline). Nothing in the mimizuku_amd package
imports it.

An fp32 numpy restatement of transformers 5.15.0's Whisper modules (the oracle the reference verifies against,
scripts/hf_reference.py:26-45), plus the reference's own greedy-choice rules (kernels/whisper.cu:451-493) and
prompt handling (src/transcribe.rs:58-93, src/model.rs:628-646). Each function cites what it follows.
`TF/` = transformers/models/whisper/ in the installed transformers package.

How each part is pinned (tests/test_oracle.py):
  * encoder, decoder, greedy tokens, logits, alignment-head weights, token timestamps: against golden vectors that
    transformers itself wrote for the tiny geometry (tests/golden/make_golden.py, tiny_*.npz);
  * attention: against a float64 closed form and against permutation invariance of keys;
  * layer_norm / gelu: against closed forms (math.erf) and invariants (zero mean, unit variance);
  * conv1d: against a brute-force loop on a tiny input;
  * dtw / median filter / jump_times: against the reference's KATs (src/align.rs:112-139) and brute force;
  * choose / top2_margin: hand-made logit vectors with known answers (ties, suppression, begin-suppression);
  * rh (fp16 rounding): known answers of IEEE round-to-nearest-even (ties, overflow, subnormal ties).
"""
from __future__ import annotations

import math

import numpy as np

HD = 64
TENC = 1500
EPS = 1e-5  # src/model.rs:12, TF modeling_whisper layer_norm default


# ---------------------------------------------------------------- elementwise and small ops

def layer_norm(x: np.ndarray, w: np.ndarray, b: np.ndarray, eps: float = EPS) -> np.ndarray:
    """nn.LayerNorm over the last axis, biased variance (TF/modeling_whisper.py self_attn_layer_norm)."""
    x = x.astype(np.float32)
    mu = x.mean(-1, keepdims=True, dtype=np.float64).astype(np.float32)
    xc = x - mu
    var = (xc.astype(np.float64) ** 2).mean(-1, keepdims=True).astype(np.float32)
    return xc / np.sqrt(var + np.float32(eps)) * w.astype(np.float32) + b.astype(np.float32)


def gelu(x: np.ndarray) -> np.ndarray:
    """Exact erf GELU, as nn.GELU() / ACT2FN['gelu'] (kernels/whisper.cu:107)."""
    from scipy.special import erf
    x = x.astype(np.float32)
    return (0.5 * x * (1.0 + erf(x / np.float32(math.sqrt(2.0))))).astype(np.float32)


def linear(x: np.ndarray, w: np.ndarray, b: np.ndarray | None = None) -> np.ndarray:
    """y = x Wᵀ + b in fp32 (nn.Linear)."""
    # (np.asarray: no copy of a weight that is already float32)
    y = np.asarray(x, np.float32) @ np.asarray(w, np.float32).T
    if b is not None:
        y = y + np.asarray(b, np.float32)
    return y


def conv1d(x: np.ndarray, w: np.ndarray, b: np.ndarray, stride: int = 1, pad: int = 1) -> np.ndarray:
    """nn.Conv1d for x [C_in][T], w [C_out][C_in][k]; returns [C_out][T_out] (TF/modeling_whisper.py conv1/conv2)."""
    cin, t = x.shape
    k = w.shape[2]
    xp = np.zeros((cin, t + 2 * pad), np.float32)
    xp[:, pad:pad + t] = x
    tout = (t + 2 * pad - k) // stride + 1
    cols = np.stack([xp[:, j:j + stride * (tout - 1) + 1:stride] for j in range(k)], axis=1)  # [cin][k][tout]
    y = w.astype(np.float32).reshape(w.shape[0], -1) @ cols.reshape(cin * k, tout)
    return y + b.astype(np.float32)[:, None]


def attention(q: np.ndarray, k: np.ndarray, v: np.ndarray, scale: float = 0.125, mask: np.ndarray | None = None,
              return_probs: bool = False, dtype=np.float32):
    """softmax(q kᵀ · scale) v over the last two axes; q [.., Tq, 64], k/v [.., Tk, 64] (TF eager_attention_forward).

    transformers scales q before the product (q_proj(x) * scaling); that is the same number up to rounding.
    """
    q = q.astype(dtype)
    s = (q * dtype(scale)) @ np.swapaxes(k.astype(dtype), -1, -2)
    if mask is not None:
        s = np.where(mask, s, -np.inf)
    s = s - s.max(-1, keepdims=True)
    p = np.exp(s)
    p = p / p.sum(-1, keepdims=True)
    o = p @ v.astype(dtype)
    return (o, p) if return_probs else o


# ---------------------------------------------------------------- encoder

def _heads(x: np.ndarray, nh: int) -> np.ndarray:
    """[T, d] -> [nh, T, 64]"""
    t, d = x.shape
    return x.reshape(t, nh, d // nh).transpose(1, 0, 2)


def _merge(x: np.ndarray) -> np.ndarray:
    """[nh, T, 64] -> [T, d]"""
    nh, t, hd = x.shape
    return x.transpose(1, 0, 2).reshape(t, nh * hd)


def self_attention_block(h: np.ndarray, W: dict, p: str, nh: int) -> np.ndarray:
    """WhisperAttention without cache, non-causal (TF/modeling_whisper.py WhisperAttention.forward, encoder case)."""
    q = linear(h, W[f"{p}.q_proj.weight"], W[f"{p}.q_proj.bias"])
    k = linear(h, W[f"{p}.k_proj.weight"])
    v = linear(h, W[f"{p}.v_proj.weight"], W[f"{p}.v_proj.bias"])
    o = attention(_heads(q, nh), _heads(k, nh), _heads(v, nh))
    return linear(_merge(o), W[f"{p}.out_proj.weight"], W[f"{p}.out_proj.bias"])


def encoder_layer(x: np.ndarray, W: dict, i: int, nh: int) -> np.ndarray:
    """Pre-LN WhisperEncoderLayer on one clip's [1500, d] hidden states (TF/modeling_whisper.py:391-411)."""
    p = f"model.encoder.layers.{i}"
    h = layer_norm(x, W[f"{p}.self_attn_layer_norm.weight"], W[f"{p}.self_attn_layer_norm.bias"])
    x = x + self_attention_block(h, W, f"{p}.self_attn", nh)
    h = layer_norm(x, W[f"{p}.final_layer_norm.weight"], W[f"{p}.final_layer_norm.bias"])
    f = gelu(linear(h, W[f"{p}.fc1.weight"], W[f"{p}.fc1.bias"]))
    return x + linear(f, W[f"{p}.fc2.weight"], W[f"{p}.fc2.bias"])


def conv_stem(mel: np.ndarray, W: dict) -> np.ndarray:
    """GELU(conv1) -> GELU(conv2, stride 2) -> transpose -> + positions (TF/modeling_whisper.py:618-627)."""
    h = gelu(conv1d(mel, W["model.encoder.conv1.weight"], W["model.encoder.conv1.bias"], 1, 1))
    h = gelu(conv1d(h, W["model.encoder.conv2.weight"], W["model.encoder.conv2.bias"], 2, 1))
    return h.T + W["model.encoder.embed_positions.weight"].astype(np.float32)


def encoder(mel: np.ndarray, W: dict, nh: int, n_layers: int):
    """One clip: returns (inputs of every layer [L][1500][d], final-LN output [1500][d])."""
    x = conv_stem(mel, W)
    hidden = []
    for i in range(n_layers):
        hidden.append(x)
        x = encoder_layer(x, W, i, nh)
    out = layer_norm(x, W["model.encoder.layer_norm.weight"], W["model.encoder.layer_norm.bias"])
    return hidden, out


def cross_kv(eh: np.ndarray, W: dict, n_dec: int, nh: int):
    """Per decoder layer, the cross-attention keys and values [nh][1500][64] of one clip (src/model.rs:614-623)."""
    out = []
    for i in range(n_dec):
        p = f"model.decoder.layers.{i}.encoder_attn"
        k = linear(eh, W[f"{p}.k_proj.weight"])
        v = linear(eh, W[f"{p}.v_proj.weight"], W[f"{p}.v_proj.bias"])
        out.append((_heads(k, nh), _heads(v, nh)))
    return out


# ---------------------------------------------------------------- decoder

class Decoder:
    """Incremental WhisperDecoder for a batch of rows with a KV cache (TF/modeling_whisper.py:469-503, 737-790).

    One `step` feeds one token per row at position p and returns fp32 logits (tied LM head) and the
    cross-attention probabilities of every (layer, head) for that query.
    """

    def __init__(self, W: dict, nh: int, n_layers: int, xkv: list):
        self.W, self.nh, self.nl = W, nh, n_layers
        self.xkv = xkv  # per row: list over layers of (K [nh][1500][64], V)
        self.kc = [[[] for _ in range(n_layers)] for _ in xkv]
        self.vc = [[[] for _ in range(n_layers)] for _ in xkv]

    def step(self, toks: list[int], p: int):
        W, nh = self.W, self.nh
        emb = W["model.decoder.embed_tokens.weight"]
        pe = W["model.decoder.embed_positions.weight"]
        x = np.stack([emb[t].astype(np.float32) + pe[p].astype(np.float32) for t in toks])  # [B, d]
        probs = np.zeros((len(toks), self.nl, nh, TENC), np.float32)
        for i in range(self.nl):
            cache = [(_heads(np.stack(self.kc[b][i]), nh) if self.kc[b][i] else None,
                      _heads(np.stack(self.vc[b][i]), nh) if self.vc[b][i] else None) for b in range(len(toks))]
            x, k, v, probs[:, i] = decoder_layer(x, W, i, nh, cache, [self.xkv[b][i] for b in range(len(toks))])
            for b in range(len(toks)):
                self.kc[b][i].append(k[b])
                self.vc[b][i].append(v[b])
        h = layer_norm(x, W["model.decoder.layer_norm.weight"], W["model.decoder.layer_norm.bias"])
        logits = linear(h, W["model.decoder.embed_tokens.weight"])
        return logits, probs


def decoder_layer(x: np.ndarray, W: dict, i: int, nh: int, cache: list, xkv: list):
    """One WhisperDecoderLayer for one new position of B rows (TF/modeling_whisper.py:469-503): x [B][d] the residual
    entering the layer; cache[b] = (K, V) [nh][p][64] of the earlier positions of row b (None at position 0);
    xkv[b] = (K, V) [nh][1500][64] of the encoder. Returns the residual after the layer, the new key and value rows
    [B][d] and the cross-attention probabilities [B][nh][1500]."""
    pr = f"model.decoder.layers.{i}"
    B = x.shape[0]
    h = layer_norm(x, W[f"{pr}.self_attn_layer_norm.weight"], W[f"{pr}.self_attn_layer_norm.bias"])
    sa = f"{pr}.self_attn"
    q = linear(h, W[f"{sa}.q_proj.weight"], W[f"{sa}.q_proj.bias"])
    k = linear(h, W[f"{sa}.k_proj.weight"])
    v = linear(h, W[f"{sa}.v_proj.weight"], W[f"{sa}.v_proj.bias"])
    att = np.zeros_like(q)
    for b in range(B):
        K, V = _heads(k[b:b + 1], nh), _heads(v[b:b + 1], nh)
        if cache[b][0] is not None:
            K = np.concatenate([cache[b][0], K], 1)
            V = np.concatenate([cache[b][1], V], 1)
        att[b] = _merge(attention(_heads(q[b:b + 1], nh), K, V))[0]
    x = x + linear(att, W[f"{sa}.out_proj.weight"], W[f"{sa}.out_proj.bias"])
    h = layer_norm(x, W[f"{pr}.encoder_attn_layer_norm.weight"], W[f"{pr}.encoder_attn_layer_norm.bias"])
    ca = f"{pr}.encoder_attn"
    q = linear(h, W[f"{ca}.q_proj.weight"], W[f"{ca}.q_proj.bias"])
    att = np.zeros_like(q)
    probs = np.zeros((B, nh, TENC), np.float32)
    for b in range(B):
        K, V = xkv[b]
        o, pb = attention(_heads(q[b:b + 1], nh), K, V, return_probs=True)
        att[b] = _merge(o)[0]
        probs[b] = pb[:, 0, :]
    x = x + linear(att, W[f"{ca}.out_proj.weight"], W[f"{ca}.out_proj.bias"])
    h = layer_norm(x, W[f"{pr}.final_layer_norm.weight"], W[f"{pr}.final_layer_norm.bias"])
    f = gelu(linear(h, W[f"{pr}.fc1.weight"], W[f"{pr}.fc1.bias"]))
    x = x + linear(f, W[f"{pr}.fc2.weight"], W[f"{pr}.fc2.bias"])
    return x, k, v, probs


def choose(logits: np.ndarray, suppress, begin_suppress, first: bool, eos: int, done: bool) -> int:
    """Greedy choice with the reference's rules (kernels/whisper.cu:451-493): suppressed ids and, at the first
    generated position, begin-suppressed ids are excluded; ties go to the lowest id; a finished row, or a row whose
    every id is suppressed, gets eos."""
    if done:
        return eos
    lg = logits.astype(np.float32).copy()
    lg[list(suppress)] = -np.inf
    if first:
        lg[[t for t in begin_suppress if t >= 0]] = -np.inf
    if not np.isfinite(lg).any() and np.all(lg == -np.inf):
        return eos
    return int(np.argmax(lg))  # first maximum = lowest id


def top2_margin(logits: np.ndarray, suppress, begin_suppress, first: bool) -> float:
    lg = logits.astype(np.float64).copy()
    lg[list(suppress)] = -np.inf
    if first:
        lg[[t for t in begin_suppress if t >= 0]] = -np.inf
    a = np.sort(lg)[-2:]
    return float(a[1] - a[0])


def greedy(W: dict, geom, gen: dict, mels: np.ndarray, prompt: list[int], max_new: int,
           detect: bool = False, teacher: np.ndarray | None = None):
    """Greedy decoding of a batch of clips, as src/transcribe.rs:104-145 drives src/model.rs:650-736.

    mels [B][n_mels][3000]. prompt = [sot, lang, task, notimestamps]; with detect=True the language token (position
    1) is chosen per row by one step on sot restricted to language tokens (src/model.rs:641-646). Generates up to
    max_new tokens after the prompt. teacher [B][T] forces the fed-back tokens (used to compare later steps without
    one low-margin divergence cascading); the choices are still reported.

    Returns dict: tokens [B][np+max_new], logits [steps][B][V] for each generating step, margins, probs
    (cross-attention of every (layer, head), [B][rows][L][nh][1500]) for every fed position, and lang.
    """
    nh, nl = geom.nh, geom.dec_layers
    B = mels.shape[0]
    eos = gen["eos_token_id"]
    sup = set(gen.get("suppress_tokens") or [])
    bsup = list(gen.get("begin_suppress_tokens") or [])
    xkv, enc_out = [], []
    for b in range(B):
        _, eh = encoder(mels[b], W, nh, geom.enc_layers)
        enc_out.append(eh)
        xkv.append(cross_kv(eh, W, nl, nh))
    npr = len(prompt)
    toks = np.array([list(prompt) + [eos] * max_new for _ in range(B)], np.int64)
    langs = [prompt[1]] * B if npr > 1 else [-1] * B
    if detect:
        langset = set(gen["lang_to_id"].values())
        d0 = Decoder(W, nh, nl, xkv)
        lg, _ = d0.step([prompt[0]] * B, 0)
        notlang = [t for t in range(geom.vocab) if t not in langset]
        for b in range(B):
            langs[b] = choose(lg[b], notlang, [], False, eos, False)
            toks[b, 1] = langs[b]
    dec = Decoder(W, nh, nl, xkv)
    done = [False] * B
    all_logits, margins, probs = [], [], []
    for p in range(npr + max_new - 1):
        feed = [int(teacher[b, p]) if teacher is not None else int(toks[b, p]) for b in range(B)]
        lg, pr = dec.step(feed, p)
        probs.append(pr)
        if p + 1 < npr:
            continue
        first = p + 1 == npr
        all_logits.append(lg)
        margins.append([top2_margin(lg[b], sup, bsup, first) for b in range(B)])
        for b in range(B):
            t = choose(lg[b], sup, bsup, first, eos, done[b])
            toks[b, p + 1] = t
            if t == eos:
                done[b] = True
    probs = np.stack(probs, axis=1)  # [B][rows][L][nh][1500]
    return {"tokens": toks, "logits": np.stack(all_logits), "margins": np.array(margins), "probs": probs,
            "lang": langs, "enc_out": enc_out}


# ---------------------------------------------------------------- token timestamps

def rh(x):
    """Round through fp16 (src/gpu.rs:117-119)."""
    return np.asarray(x, np.float32).astype(np.float16).astype(np.float32)


def median_filter(z: np.ndarray, width: int = 7) -> np.ndarray:
    """Median over a width-`width` window of the last axis with reflect padding (TF/generation_whisper.py:43-61)."""
    pad = width // 2
    if z.shape[-1] <= pad:
        return z
    zp = np.concatenate([z[..., 1:pad + 1][..., ::-1], z, z[..., -pad - 1:-1][..., ::-1]], axis=-1)
    win = np.stack([zp[..., i:i + z.shape[-1]] for i in range(width)], axis=-1)
    return np.sort(win, axis=-1)[..., pad]


def dtw(m: np.ndarray):
    """Dynamic time warping with a float32 cost table, ties towards the horizontal move
    (TF/generation_whisper.py:64-115; src/align.rs:65-106). m [rows][cols] (the cost, i.e. minus the scores)."""
    rows, cols = m.shape
    cost = np.full((rows + 1, cols + 1), np.inf, np.float32)
    trace = -np.ones((rows + 1, cols + 1), np.int8)
    cost[0, 0] = 0
    for j in range(1, cols + 1):
        for i in range(1, rows + 1):
            c0, c1, c2 = cost[i - 1, j - 1], cost[i - 1, j], cost[i, j - 1]
            if c0 < c1 and c0 < c2:
                c, t = c0, 0
            elif c1 < c0 and c1 < c2:
                c, t = c1, 1
            else:
                c, t = c2, 2
            cost[i, j] = np.float32(np.float64(m[i - 1, j - 1]) + np.float64(c))
            trace[i, j] = t
    trace[0, :] = 2
    trace[:, 0] = 1
    i, j = rows, cols
    text, time = [], []
    while i > 0 or j > 0:
        text.append(i - 1)
        time.append(j - 1)
        t = trace[i, j]
        if t == 0:
            i, j = i - 1, j - 1
        elif t == 1:
            i -= 1
        else:
            j -= 1
    return np.array(text[::-1]), np.array(time[::-1])


def jump_times(w: np.ndarray, cols: int, width: int = 7, half: bool = False) -> np.ndarray:
    """Start time (s) of each row from alignment-head weights w [rows][heads][cols_full]
    (TF/generation_whisper.py:241-379 `_extract_token_timestamps`; src/align.rs:8-63): DTW over align_cost."""
    rows = w.shape[0]
    if cols == 0:
        return np.zeros(rows, np.float32)
    text, time = dtw(align_cost(w, cols, width, half))
    jumps = np.concatenate([[True], np.diff(text) != 0])
    out = (time[jumps] * 0.02).astype(np.float32)
    if len(out) < rows:  # degenerate scores bend the path (src/align.rs:60-61)
        out = np.concatenate([out, np.full(rows - len(out), out[-1] if len(out) else 0, np.float32)])
    return out[:rows]


def align_cost(w: np.ndarray, cols: int, width: int = 7, half: bool = False) -> np.ndarray:
    """The DTW cost of jump_times, float64 [rows][cols] (src/align.rs:14-52).

    Columns are cropped to `cols` (= audio frames // 2), each head is normalised over rows, median-filtered over
    time, the heads are averaged and DTW runs on minus the average. half=True is src/align.rs:18-23, 52 exactly: the
    column sum and the sum of squared deviations from the unrounded mean accumulate in float32 in row order (a
    sequential fold, np.add.accumulate), then the mean, the deviation and every z-score are rounded through fp16, as
    a model run in fp16 does. half=False is the fp32 model's arithmetic with the two sums taken in float64. A
    constant column scores 0 (the fp32/fp16 model divides by zero there, src/align.rs:22).
    """
    rows, heads, _ = w.shape
    x = w[:, :, :cols].astype(np.float32)
    if half:
        n = np.float32(rows)
        mean = np.add.accumulate(x, axis=0, dtype=np.float32)[-1:] / n
        dev = (x - mean).astype(np.float32)
        var = np.add.accumulate(dev * dev, axis=0, dtype=np.float32)[-1:] / n
        std = np.sqrt(var.astype(np.float32))
    else:
        mean = x.mean(0, keepdims=True, dtype=np.float64).astype(np.float32)
        var = ((x - mean).astype(np.float64) ** 2).mean(0, keepdims=True).astype(np.float32)
        std = np.sqrt(var)
    if half:
        mean, std = rh(mean), rh(std)
        num = rh(x - mean)
        z = np.where(std > 0, rh(num / np.where(std > 0, std, 1)), 0).astype(np.float32)
    else:
        z = np.where(std > 0, (x - mean) / np.where(std > 0, std, 1), 0).astype(np.float32)
    z = median_filter(z.transpose(1, 0, 2), width)  # [heads][rows][cols]
    avg = z.astype(np.float32).sum(0, dtype=np.float32) / np.float32(heads)
    if half:
        avg = rh(avg)
    return -avg.astype(np.float64)


def token_timestamps(probs_rows: np.ndarray, align_heads, n_prompt: int, n_seq: int, frames: int,
                     half: bool = False) -> np.ndarray:
    """Per-token start times of one clip's sequence of n_seq tokens (src/transcribe.rs:147-162): the rows of the
    generated tokens that were fed back (positions n_prompt .. n_seq-2) go to DTW; prompt tokens get 0 and the
    last token repeats the time of the one before it. probs_rows [rows][L][nh][1500] indexed by position."""
    ts = np.zeros(n_seq, np.float32)
    rows = max(n_seq - 1 - n_prompt, 0)
    if rows > 0:
        w = np.stack([probs_rows[n_prompt:n_prompt + rows, l, h] for l, h in align_heads], axis=1)
        jt = jump_times(w, frames // 2, 7, half)
        ts[n_prompt:n_prompt + rows] = jt
        ts[n_seq - 1] = jt[rows - 1]
    return ts
