"""Seeded random-init Whisper checkpoints, generation configs and log-mel inputs.

There are no checkpoints on disk and no network, so every workload runs on weights drawn here. Tensor names and
shapes are the Hugging Face ones the reference's loader reads (src/model.rs:343-407), so the same dictionary feeds
the engine, the oracle and transformers. Initialisation follows transformers' Whisper `_init_weights`
(Linear/Conv weights and Embeddings N(0, 0.02), biases 0, LayerNorm gamma 1 beta 0, padding row of the token
embedding zeroed, encoder positions sinusoidal). Weights are rounded to the fp16 grid once, so an fp16 engine and an
fp32 oracle read the same numbers.
"""
from __future__ import annotations

import dataclasses
import json

import numpy as np

TENC = 1500   # encoder positions of a 30 s window (src/model.rs:10)
NFRAMES = 3000  # log-mel frames of a 30 s window


@dataclasses.dataclass(frozen=True)
class Geometry:
    """Model geometry, as src/model.rs:14-25 reads it from config.json."""
    d: int
    ff: int
    nh: int
    enc_layers: int
    dec_layers: int
    n_mels: int
    vocab: int
    max_t: int = 448

    def config_json(self) -> dict:
        return {
            "d_model": self.d, "encoder_ffn_dim": self.ff, "decoder_ffn_dim": self.ff,
            "encoder_attention_heads": self.nh, "decoder_attention_heads": self.nh,
            "encoder_layers": self.enc_layers, "decoder_layers": self.dec_layers,
            "num_mel_bins": self.n_mels, "vocab_size": self.vocab, "max_target_positions": self.max_t,
            "max_source_positions": TENC, "pad_token_id": 50257, "bos_token_id": 50257, "eos_token_id": 50257,
            "decoder_start_token_id": 50258, "activation_function": "gelu", "scale_embedding": False,
            "median_filter_width": 7, "model_type": "whisper",
        }


TINY = Geometry(d=384, ff=1536, nh=6, enc_layers=4, dec_layers=4, n_mels=80, vocab=51865)
LARGE_V3 = Geometry(d=1280, ff=5120, nh=20, enc_layers=32, dec_layers=32, n_mels=128, vocab=51866)
LARGE_V3_TURBO = Geometry(d=1280, ff=5120, nh=20, enc_layers=32, dec_layers=4, n_mels=128, vocab=51866)

# Special-token layout of the multilingual vocabularies (51865: tiny..medium; 51866: large-v3 adds one language).
_LANGS = ["en", "zh", "de", "es", "ru", "ko", "fr", "ja", "pt", "tr", "pl", "ca", "nl", "ar", "sv", "it"]


def generation_config(g: Geometry, align_heads=None) -> dict:
    """A generation_config.json for geometry g with the token ids of the real vocabularies of that size."""
    v3 = g.vocab == 51866
    sot, eos = 50258, 50257
    translate, transcribe, notime = (50359, 50360, 50364) if v3 else (50358, 50359, 50363)
    if align_heads is None:
        if g == LARGE_V3_TURBO:
            align_heads = [[2, 4], [2, 11], [3, 3], [3, 6], [3, 11], [3, 14]]
        elif g == LARGE_V3:
            align_heads = [[7, 0], [10, 17], [12, 18], [13, 12], [16, 1], [17, 14], [19, 11], [21, 4], [24, 1], [25, 6]]
        elif g == TINY:
            align_heads = [[2, 2], [3, 0], [3, 2], [3, 3], [3, 4], [3, 5]]
        else:  # openai/whisper's default: every head of the second half of the decoder layers (src/model.rs:101)
            align_heads = [[layer, h] for layer in range(g.dec_layers // 2, g.dec_layers) for h in range(g.nh)]
    suppress = [1, 2, 7, 8, 9, 10, 14, 25, 26, 27, 28, 29, 31, 58, 59, 60, 61, 62, 63, 90, 91, 92, 93, 359, 503,
                522, 542, 873, 893, 902, 918, 922, 931, 1350, 1853, 1982, 2460, 2627, 3246, 3253, 3268, 3536, 3846,
                3961, 4183, 4667, 6585, 6647, 7273, 9061, 9383, 10428, 10929, 11938, 12033, 12331, 12562, 13793,
                14157, 14635, 15265, 15618, 16553, 16604, 18362, 18956, 20075, 21675, 22520, 26130, 26161, 26435,
                28279, 29464, 31650, 32302, 32470, 36865, 42863, 47425, 49870, 50254, sot, translate, transcribe,
                translate + 2, translate + 3, translate + 4]
    return {
        "decoder_start_token_id": sot, "eos_token_id": eos, "pad_token_id": eos, "bos_token_id": eos,
        "no_timestamps_token_id": notime, "is_multilingual": True,
        "lang_to_id": {f"<|{c}|>": 50259 + i for i, c in enumerate(_LANGS)},
        "task_to_id": {"translate": translate, "transcribe": transcribe},
        "suppress_tokens": sorted(set(suppress)), "begin_suppress_tokens": [220, eos],
        "alignment_heads": align_heads, "max_length": g.max_t,
    }


def sinusoids(length: int, channels: int, max_timescale: float = 10000.0) -> np.ndarray:
    """Encoder positional table (transformers modeling_whisper.py `sinusoids`): [sin | cos] halves."""
    inc = np.log(max_timescale) / (channels // 2 - 1)
    inv = np.exp(-inc * np.arange(channels // 2, dtype=np.float64))
    t = np.arange(length, dtype=np.float64)[:, None] * inv[None, :]
    return np.concatenate([np.sin(t), np.cos(t)], axis=1).astype(np.float32)


def tensor_shapes(g: Geometry) -> dict[str, tuple]:
    """Every stored tensor of a Whisper checkpoint (proj_out is tied to embed_tokens and not stored)."""
    d, ff = g.d, g.ff
    s: dict[str, tuple] = {}
    s["model.encoder.conv1.weight"] = (d, g.n_mels, 3)
    s["model.encoder.conv1.bias"] = (d,)
    s["model.encoder.conv2.weight"] = (d, d, 3)
    s["model.encoder.conv2.bias"] = (d,)
    s["model.encoder.embed_positions.weight"] = (TENC, d)

    def attn(p, ln):
        for n in ("q_proj", "k_proj", "v_proj", "out_proj"):
            s[f"{p}.{n}.weight"] = (d, d)
            if n != "k_proj":
                s[f"{p}.{n}.bias"] = (d,)
        s[f"{ln}.weight"] = (d,)
        s[f"{ln}.bias"] = (d,)

    def ffn(p):
        s[f"{p}.fc1.weight"] = (ff, d)
        s[f"{p}.fc1.bias"] = (ff,)
        s[f"{p}.fc2.weight"] = (d, ff)
        s[f"{p}.fc2.bias"] = (d,)
        s[f"{p}.final_layer_norm.weight"] = (d,)
        s[f"{p}.final_layer_norm.bias"] = (d,)

    for i in range(g.enc_layers):
        p = f"model.encoder.layers.{i}"
        attn(f"{p}.self_attn", f"{p}.self_attn_layer_norm")
        ffn(p)
    s["model.encoder.layer_norm.weight"] = (d,)
    s["model.encoder.layer_norm.bias"] = (d,)
    s["model.decoder.embed_tokens.weight"] = (g.vocab, d)
    s["model.decoder.embed_positions.weight"] = (g.max_t, d)
    for i in range(g.dec_layers):
        p = f"model.decoder.layers.{i}"
        attn(f"{p}.self_attn", f"{p}.self_attn_layer_norm")
        attn(f"{p}.encoder_attn", f"{p}.encoder_attn_layer_norm")
        ffn(p)
    s["model.decoder.layer_norm.weight"] = (d,)
    s["model.decoder.layer_norm.bias"] = (d,)
    return s


def random_weights(g: Geometry, seed: int = 0, std: float = 0.02, bias_std: float = 0.0,
                   ln_std: float = 0.0) -> dict[str, np.ndarray]:
    """Seeded weights on the fp16 grid, stored as float16 arrays.

    bias_std > 0 draws biases N(0, bias_std) instead of zeros (so the q/v-bias and zero-k-bias paths matter);
    ln_std > 0 perturbs LayerNorm gamma around 1 and beta around 0 likewise.
    """
    rng = np.random.default_rng(seed)
    out: dict[str, np.ndarray] = {}
    for name, shape in tensor_shapes(g).items():
        if name == "model.encoder.embed_positions.weight":
            a = sinusoids(TENC, g.d)
        elif "layer_norm" in name:
            base = 1.0 if name.endswith(".weight") else 0.0
            a = base + (rng.standard_normal(shape, dtype=np.float32) * ln_std if ln_std else np.zeros(shape, np.float32))
        elif name.endswith(".bias"):
            a = rng.standard_normal(shape, dtype=np.float32) * bias_std if bias_std else np.zeros(shape, np.float32)
        else:
            a = rng.standard_normal(shape, dtype=np.float32) * std
            if name == "model.decoder.embed_tokens.weight":
                a[50257] = 0.0  # padding_idx row
        out[name] = np.ascontiguousarray(a.astype(np.float16))
    return out


def synthetic_mel(n_clips: int, n_mels: int, seed: int = 1) -> np.ndarray:
    """Log-mel inputs [n][n_mels][3000] ~ N(-0.3, 0.4) clamped to [-1.5, 1.5], float32."""
    rng = np.random.default_rng(seed)
    m = rng.normal(-0.3, 0.4, size=(n_clips, n_mels, NFRAMES)).astype(np.float32)
    return np.clip(m, -1.5, 1.5)


def weights_digest(w: dict[str, np.ndarray]) -> str:
    """Short content hash of a weight dictionary (to detect generator drift against stored fixtures)."""
    import hashlib
    h = hashlib.sha256()
    for k in sorted(w):
        h.update(k.encode())
        h.update(np.ascontiguousarray(w[k]).tobytes())
    return h.hexdigest()[:16]


def write_model_dir(path: str, g: Geometry, w: dict[str, np.ndarray], gen: dict | None = None) -> None:
    """A Hugging Face style model directory (config.json, generation_config.json, model.safetensors)."""
    import os
    from safetensors.numpy import save_file
    os.makedirs(path, exist_ok=True)
    with open(os.path.join(path, "config.json"), "w") as f:
        json.dump(g.config_json(), f)
    with open(os.path.join(path, "generation_config.json"), "w") as f:
        json.dump(gen if gen is not None else generation_config(g), f)
    save_file(w, os.path.join(path, "model.safetensors"))
