"""Writes the tiny-geometry golden vectors from transformers' Whisper modules (fp32, CPU).

Run where transformers 5.15.0 is installed (the GPU tests only read the vectors it writes):
    PYTHONPATH=. python tests/golden/make_golden.py

The model is built offline from a local WhisperConfig and loaded with the seeded weights of mimizuku_amd.synth (no
hub access). Each fixture holds the greedy sequence generate() produces with its own logits processors, raw logits at
a subset of ids plus the top-2 of every step, the encoder's per-layer inputs at a subset of rows (with whole-tensor
checksums), the alignment-head cross-attention weights, and transformers' token timestamps.
"""
import os
import sys

import numpy as np
import torch
from transformers import GenerationConfig, WhisperConfig, WhisperForConditionalGeneration

sys.path.insert(0, os.path.join(os.path.dirname(__file__), "..", ".."))
from mimizuku_amd import synth  # noqa: E402

HERE = os.path.dirname(os.path.abspath(__file__))
ROWS = np.arange(0, 1500, 30)          # encoder rows kept
VOCAB_SUB = np.arange(0, 51865, 97)    # logit ids kept
MAX_NEW = 32

CASES = {
    # HF init: biases 0, LayerNorm gamma 1 beta 0; language forced to en
    "tiny_hfinit": dict(seed=0, bias_std=0.0, ln_std=0.0, mel_seed=1, n_clips=1, language="en"),
    # non-zero biases and LayerNorm parameters, language detected, two clips in one batch
    "tiny_bias_detect": dict(seed=3, bias_std=0.02, ln_std=0.02, mel_seed=4, n_clips=2, language=None),
}


def build(g, W, gen):
    cfg = WhisperConfig(**{k: v for k, v in g.config_json().items() if k != "model_type"})
    m = WhisperForConditionalGeneration(cfg).eval()
    sd = {k: torch.from_numpy(v.astype(np.float32)) for k, v in W.items()}
    sd["proj_out.weight"] = sd["model.decoder.embed_tokens.weight"]
    missing, unexpected = m.load_state_dict(sd, strict=False)
    assert not missing and not unexpected, (missing, unexpected)
    m.generation_config = GenerationConfig(**gen)
    return m


def main():
    torch.manual_seed(0)
    g = synth.TINY
    for name, c in CASES.items():
        W = synth.random_weights(g, seed=c["seed"], bias_std=c["bias_std"], ln_std=c["ln_std"])
        gen = synth.generation_config(g)
        m = build(g, W, gen)
        mel = synth.synthetic_mel(c["n_clips"], g.n_mels, seed=c["mel_seed"])
        x = torch.from_numpy(mel)
        with torch.no_grad():
            eo = m.model.encoder(x, output_hidden_states=True)
            kw = dict(task="transcribe", return_token_timestamps=True, max_new_tokens=MAX_NEW,
                      return_dict_in_generate=True, output_logits=True,
                      attention_mask=torch.ones(c["n_clips"], 3000, dtype=torch.long))
            if c["language"]:
                kw["language"] = c["language"]
            out = m.generate(x, **kw)
        hs = torch.stack(eo.hidden_states).numpy()  # [L+1][B][1500][d]; last = after the final LN
        seq = out["sequences"].numpy().astype(np.int32)
        logits = torch.stack(out["logits"], 0).numpy()  # [steps][B][V] raw logits
        top2_ids = np.argsort(-logits, axis=-1)[..., :2].astype(np.int32)
        top2_val = np.take_along_axis(logits, top2_ids, -1)
        heads = gen["alignment_heads"]
        ca = [torch.cat([st[i] for st in out["cross_attentions"]], dim=2) for i in range(g.dec_layers)]
        align_w = torch.stack([ca[l][:, h] for l, h in heads], 1).numpy()  # [B][heads][rows][1500]
        np.savez_compressed(
            os.path.join(HERE, f"{name}.npz"),
            weights_digest=np.array(synth.weights_digest(W)),
            seed=c["seed"], bias_std=c["bias_std"], ln_std=c["ln_std"], mel_seed=c["mel_seed"],
            n_clips=c["n_clips"], detect=np.array(c["language"] is None),
            rows=ROWS, enc_hidden_rows=hs[:, :, ROWS, :].astype(np.float32),
            enc_hidden_sum=hs.astype(np.float64).sum(axis=(2, 3)),
            enc_hidden_sumsq=(hs.astype(np.float64) ** 2).sum(axis=(2, 3)),
            sequences=seq, vocab_sub=VOCAB_SUB, logits_sub=logits[..., VOCAB_SUB].astype(np.float32),
            top2_ids=top2_ids, top2_val=top2_val.astype(np.float32),
            align_heads=np.array(heads, np.int32), align_w=align_w.astype(np.float32),
            token_timestamps=out["token_timestamps"].numpy().astype(np.float32),
            transformers_version=np.array(__import__("transformers").__version__),
        )
        print(name, seq.tolist())


if __name__ == "__main__":
    main()
