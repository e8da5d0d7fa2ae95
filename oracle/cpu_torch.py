"""CPU baseline of the benchmark workloads: an fp32 torch restatement of transformers' Whisper modules, timed on the
host's cores.

Test and measurement infrastructure only (like the rest of oracle/): bench.py runs it in a child process,

    python -m oracle.cpu_torch --steps 227        # prints one JSON object

so torch is never loaded into the process that drives the GPU. The functions follow the same semantics as the numpy
oracle (oracle/whisper_ref.py), against which tests/test_cpu_torch.py checks them:
  * encoder layer: pre-LN self-attention (q_proj(x) * 1/8, k_proj without bias, eager matmul -> softmax -> matmul)
    and GELU FFN (TF/models/whisper/modeling_whisper.py:391-411, 279-282, 228-235);
  * decoder layer for one new token per row: self-attention over a key/value cache, cross-attention over
    precomputed encoder keys/values, FFN (:469-503); the tied LM head with the final LayerNorm (:965, 970, 1080).

Workloads (the benchmark configurations, synthetic fp32 inputs and seeded weights N(0, 0.02)):
  config 2  eager attention over [8, 20, 1500, 64]
  config 3  one large-v3 encoder layer on [8, 1500, 1280]
  config 4  one large-v3-turbo decoder step at B = 32: 4 layers with the self cache at 200 positions and cross
            keys/values [32, 20, 1500, 64] per layer, the final LayerNorm, the tied LM head over 51,866 ids, argmax
  config 5  large-v3-turbo end to end on 32 clips, extrapolated from a measured subset: the conv stem of one group
            of 8 clips, config 3 (one layer of that group) and the cross keys/values of that group, times 4 groups and
            32 layers, plus `steps` decoder steps at config 4's time
torch.set_num_threads(threads), threads = OMP_NUM_THREADS when set (the host's CPU share), else os.cpu_count();
torch.inference_mode(); one warm-up, then the median of `reps` runs.
"""
from __future__ import annotations

import argparse
import json
import os
import platform
import time

import torch
import torch.nn.functional as F

EPS = 1e-5


def layer_norm(x, w, b):
    return F.layer_norm(x, (x.shape[-1],), w, b, EPS)


def linear(x, w, b=None):
    return F.linear(x, w, b)


def attention(q, k, v, scale=0.125):
    """Eager softmax(q k^T * scale) v over the last two axes (q scaled before the product, as transformers)."""
    s = torch.matmul(q * scale, k.transpose(-1, -2))
    return torch.matmul(torch.softmax(s, dim=-1), v)


def heads(x, nh):
    *lead, t, d = x.shape
    return x.reshape(*lead, t, nh, d // nh).transpose(-3, -2)


def merge(x):
    *lead, nh, t, hd = x.shape
    return x.transpose(-3, -2).reshape(*lead, t, nh * hd)


def encoder_layer(x, W: dict, p: str, nh: int):
    """One WhisperEncoderLayer on x [..., T, d]; p = 'model.encoder.layers.i'."""
    h = layer_norm(x, W[f"{p}.self_attn_layer_norm.weight"], W[f"{p}.self_attn_layer_norm.bias"])
    a = f"{p}.self_attn"
    q = heads(linear(h, W[f"{a}.q_proj.weight"], W[f"{a}.q_proj.bias"]), nh)
    k = heads(linear(h, W[f"{a}.k_proj.weight"]), nh)
    v = heads(linear(h, W[f"{a}.v_proj.weight"], W[f"{a}.v_proj.bias"]), nh)
    x = x + linear(merge(attention(q, k, v)), W[f"{a}.out_proj.weight"], W[f"{a}.out_proj.bias"])
    h = layer_norm(x, W[f"{p}.final_layer_norm.weight"], W[f"{p}.final_layer_norm.bias"])
    h = F.gelu(linear(h, W[f"{p}.fc1.weight"], W[f"{p}.fc1.bias"]))
    return x + linear(h, W[f"{p}.fc2.weight"], W[f"{p}.fc2.bias"])


def conv_stem(mel, W: dict):
    """GELU(conv1) -> GELU(conv2, stride 2) -> + positions, mel [B, n_mels, 3000] -> [B, 1500, d]."""
    h = F.gelu(F.conv1d(mel, W["model.encoder.conv1.weight"], W["model.encoder.conv1.bias"], padding=1))
    h = F.gelu(F.conv1d(h, W["model.encoder.conv2.weight"], W["model.encoder.conv2.bias"], stride=2, padding=1))
    return h.transpose(1, 2) + W["model.encoder.embed_positions.weight"]


def cross_kv(eh, W: dict, layers: list[int], nh: int):
    """Cross-attention keys and values [B, nh, 1500, 64] of each decoder layer from the encoder output [B, 1500, d]."""
    out = []
    for i in layers:
        a = f"model.decoder.layers.{i}.encoder_attn"
        out.append((heads(linear(eh, W[f"{a}.k_proj.weight"]), nh),
                    heads(linear(eh, W[f"{a}.v_proj.weight"], W[f"{a}.v_proj.bias"]), nh)))
    return out


def decoder_layer(x, W: dict, i: int, nh: int, kc, vc, pos: int, xk, xv):
    """One WhisperDecoderLayer for one new token per row at position pos: x [B, d]; the self-attention cache
    kc / vc [B, nh, max_t, 64] gets the new key/value at pos and is attended over 0 .. pos; xk / xv [B, nh, 1500,
    64] are the cross keys/values."""
    p = f"model.decoder.layers.{i}"
    a = f"{p}.self_attn"
    h = layer_norm(x, W[f"{a}_layer_norm.weight"], W[f"{a}_layer_norm.bias"])
    q = heads(linear(h, W[f"{a}.q_proj.weight"], W[f"{a}.q_proj.bias"])[:, None], nh)  # [B, nh, 1, 64]
    kc[:, :, pos] = heads(linear(h, W[f"{a}.k_proj.weight"])[:, None], nh)[:, :, 0]
    vc[:, :, pos] = heads(linear(h, W[f"{a}.v_proj.weight"], W[f"{a}.v_proj.bias"])[:, None], nh)[:, :, 0]
    o = attention(q, kc[:, :, :pos + 1], vc[:, :, :pos + 1])
    x = x + linear(merge(o)[:, 0], W[f"{a}.out_proj.weight"], W[f"{a}.out_proj.bias"])
    c = f"{p}.encoder_attn"
    h = layer_norm(x, W[f"{c}_layer_norm.weight"], W[f"{c}_layer_norm.bias"])
    q = heads(linear(h, W[f"{c}.q_proj.weight"], W[f"{c}.q_proj.bias"])[:, None], nh)
    o = attention(q, xk, xv)
    x = x + linear(merge(o)[:, 0], W[f"{c}.out_proj.weight"], W[f"{c}.out_proj.bias"])
    h = layer_norm(x, W[f"{p}.final_layer_norm.weight"], W[f"{p}.final_layer_norm.bias"])
    h = F.gelu(linear(h, W[f"{p}.fc1.weight"], W[f"{p}.fc1.bias"]))
    return x + linear(h, W[f"{p}.fc2.weight"], W[f"{p}.fc2.bias"])


def lm_head(x, W: dict):
    """Final LayerNorm and the tied LM head (logits over the vocabulary) of x [B, d]."""
    h = layer_norm(x, W["model.decoder.layer_norm.weight"], W["model.decoder.layer_norm.bias"])
    return linear(h, W["model.decoder.embed_tokens.weight"])


# ---------------------------------------------------------------- the timed workloads

D, FF, NH, VOCAB, NMELS, MAXT, TENC = 1280, 5120, 20, 51866, 128, 448, 1500


def _weights(gen: torch.Generator, enc_layers: list[int], dec_layers: list[int]) -> dict:
    n = lambda *shape: torch.randn(*shape, generator=gen) * 0.02  # noqa: E731
    W = {"model.encoder.conv1.weight": n(D, NMELS, 3), "model.encoder.conv1.bias": torch.zeros(D),
         "model.encoder.conv2.weight": n(D, D, 3), "model.encoder.conv2.bias": torch.zeros(D),
         "model.encoder.embed_positions.weight": n(TENC, D),
         "model.decoder.embed_tokens.weight": n(VOCAB, D), "model.decoder.embed_positions.weight": n(MAXT, D),
         "model.decoder.layer_norm.weight": torch.ones(D), "model.decoder.layer_norm.bias": torch.zeros(D)}

    def attn(a):
        for m in ("q_proj", "k_proj", "v_proj", "out_proj"):
            W[f"{a}.{m}.weight"] = n(D, D)
            if m != "k_proj":
                W[f"{a}.{m}.bias"] = torch.zeros(D)

    def block(p, names):
        for ln in names:
            W[f"{p}.{ln}.weight"], W[f"{p}.{ln}.bias"] = torch.ones(D), torch.zeros(D)
        W[f"{p}.fc1.weight"], W[f"{p}.fc1.bias"] = n(FF, D), torch.zeros(FF)
        W[f"{p}.fc2.weight"], W[f"{p}.fc2.bias"] = n(D, FF), torch.zeros(D)

    for i in enc_layers:
        p = f"model.encoder.layers.{i}"
        attn(f"{p}.self_attn")
        block(p, ["self_attn_layer_norm", "final_layer_norm"])
    for i in dec_layers:
        p = f"model.decoder.layers.{i}"
        attn(f"{p}.self_attn")
        attn(f"{p}.encoder_attn")
        block(p, ["self_attn_layer_norm", "encoder_attn_layer_norm", "final_layer_norm"])
    return W


def _time(f, reps: int):
    f()  # warm-up
    ts = []
    for _ in range(reps):
        t = time.perf_counter()
        f()
        ts.append(time.perf_counter() - t)
    ts.sort()
    return ts[len(ts) // 2]


def run(steps: int, reps: int = 3) -> dict:
    threads = int(os.environ.get("OMP_NUM_THREADS") or os.cpu_count() or 1)
    torch.set_num_threads(threads)
    gen = torch.Generator().manual_seed(0)
    B, G, NL = 32, 8, 4
    W = _weights(gen, [0], list(range(NL)))
    out = {"threads": torch.get_num_threads(), "host_cpus": os.cpu_count(),
           "cpu": platform.processor() or platform.machine()}
    try:
        with open("/proc/cpuinfo") as f:
            out["cpu"] = next(l.split(":", 1)[1].strip() for l in f if l.startswith("model name"))
    except (OSError, StopIteration):
        pass
    with torch.inference_mode():
        # config 2: the attention op alone
        q, k, v = (torch.randn(G, NH, TENC, 64, generator=gen) for _ in range(3))
        out["config2_attention_s"] = _time(lambda: attention(q, k, v), reps)
        del q, k, v
        # config 3: one large-v3 encoder layer on 8 clips
        x = torch.randn(G, TENC, D, generator=gen)
        out["config3_layer_s"] = _time(lambda: encoder_layer(x, W, "model.encoder.layers.0", NH), reps)
        # the rest of one group's encoder pass: conv stem and the cross keys/values of the 4 decoder layers
        mel = torch.clamp(torch.randn(G, NMELS, 2 * TENC, generator=gen) * 0.4 - 0.3, -1.5, 1.5)
        out["stem_s"] = _time(lambda: conv_stem(mel, W), reps)
        out["cross_kv_s"] = _time(lambda: cross_kv(x, W, list(range(NL)), NH), reps)
        del x, mel
        # config 4: one turbo decoder step at B = 32, position 200
        xkv = [(torch.randn(B, NH, TENC, 64, generator=gen), torch.randn(B, NH, TENC, 64, generator=gen))
               for _ in range(NL)]
        caches = [(torch.randn(B, NH, MAXT, 64, generator=gen), torch.randn(B, NH, MAXT, 64, generator=gen))
                  for _ in range(NL)]
        toks = torch.randint(0, 50000, (B,), generator=gen)

        def step():
            x = W["model.decoder.embed_tokens.weight"][toks] + W["model.decoder.embed_positions.weight"][200]
            for i in range(NL):
                x = decoder_layer(x, W, i, NH, caches[i][0], caches[i][1], 200, xkv[i][0], xkv[i][1])
            return lm_head(x, W).argmax(-1)
        out["config4_step_s"] = _time(step, reps)
    enc_group = out["stem_s"] + 32 * out["config3_layer_s"] + out["cross_kv_s"]
    total = 4 * enc_group + steps * out["config4_step_s"]
    out.update({"config5_total_s": total, "config5_audio_s_per_s": 32 * 30.0 / total, "steps": steps,
                "config5_note": f"extrapolated: 4 groups x (conv stem + 32 x one encoder layer + cross k/v of 8 "
                                f"clips) + {steps} decoder steps at config 4's time"})
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--steps", type=int, default=227, help="decoder steps of the end-to-end extrapolation")
    ap.add_argument("--reps", type=int, default=3)
    a = ap.parse_args()
    print(json.dumps(run(a.steps, a.reps)), flush=True)


if __name__ == "__main__":
    main()
