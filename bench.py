"""Throughput of the Whisper compute path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu]

One step = one pass of the batch transcription API over 32 synthetic 30 s clips with large-v3-turbo geometry and
seeded random-init fp16 weights: the encoder in groups of 8 clips (conv stem, 32 layers, every decoder layer's cross
k/v), language detection, greedy decoding of up to 224 tokens by replaying one captured step graph, and token
timestamps from the alignment heads (median filter + DTW on the host). The log-mel inputs are resident in device
memory before the timed region. Prints one JSON line: audio-seconds per second (value), with the encoder TFLOP/s, the
decoder step time, per-kernel event timings, the roofline of the dominant kernel and the CPU oracle on a bounded
sample of the same workload.
"""
from __future__ import annotations

import argparse
import json
import os
import platform
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_F16 = 2.5e15  # dense fp16 MFMA, FLOP/s
PEAK_HBM = 8.0e12  # bytes/s
N_CLIPS, EG, MAX_NEW = 32, 8, 224
METRIC = "audio-sec/sec, large-v3-turbo fp16 batch 32; encoder TFLOP/s; decode step µs"


def log(msg: str):
    print(msg, file=sys.stderr, flush=True)


def kernel_work(g, G: int) -> dict:
    """Algorithmic work of one launch of each encoder kernel class for a group of G clips: ('mfma', FLOP) or
    ('hbm', bytes)."""
    d, ff, nh, nm, nl = g.d, g.ff, g.nh, g.n_mels, g.dec_layers
    M = G * 1500
    return {
        "mel": ("hbm", G * nm * 3000 * (4 + 2)),
        "conv1": ("mfma", 2.0 * G * 3000 * d * 3 * nm),
        "conv2": ("mfma", 2.0 * M * d * 3 * d),
        "ln": ("hbm", M * d * (4 + 2 + 4 + 2)),  # add + LayerNorm: read x (f32) and the fp16 delta, write x and h
        "qkv": ("mfma", 2.0 * M * 3 * d * d),
        "attn": ("mfma", 4.0 * G * nh * 1500 * 1500 * 64),
        "oproj": ("mfma", 2.0 * M * d * d),
        "fc1": ("mfma", 2.0 * M * ff * d),
        "fc2": ("mfma", 2.0 * M * d * ff),
        "xkv": ("mfma", 2.0 * M * nl * 2 * d * d),
    }


def encoder_flops(g, n: int) -> float:
    w = kernel_work(g, 1)
    per_clip = w["conv1"][1] + w["conv2"][1] + w["xkv"][1] + g.enc_layers * sum(
        w[k][1] for k in ("qkv", "attn", "oproj", "fc1", "fc2"))
    return n * per_clip


def decode_step_bytes(g, B: int, p: int, na: int) -> float:
    """HBM bytes one decoder step must move at position p for B rows: cross k/v, decoder weights, the tied LM head,
    the self-attention cache (read) and its new entry, logits (fp32) and the alignment rows."""
    d, ff, nl, V = g.d, g.ff, g.dec_layers, g.vocab
    cross = B * nl * 2 * 1500 * d * 2
    weights = nl * 2 * (3 * d * d + 3 * d * d + 2 * d * ff)  # qkv, o, xq, xo, fc1, fc2 (fp16)
    head = V * d * 2
    selfkv = B * nl * 2 * (p + 1) * d * 2
    return cross + weights + head + selfkv + B * V * 4 + B * na * 1500 * 2


def cpu_baseline(g, W16: dict, gen: dict, mel: np.ndarray, steps: int) -> dict:
    """The oracle (fp32 numpy) on a bounded sample: the conv stem, one encoder layer and the cross k/v of one clip,
    and two decoder steps of the 32-row batch; extrapolated to the whole workload (32 clips x 32 layers, `steps`
    decoder steps)."""
    from oracle import whisper_ref as R
    try:
        from threadpoolctl import threadpool_info
        threads = max([i.get("num_threads", 1) for i in threadpool_info() if i.get("user_api") == "blas"] or [1])
    except Exception:  # pragma: no cover
        threads = os.cpu_count() or 1
    keep = [k for k in W16 if not k.startswith("model.encoder.layers.") or k.startswith("model.encoder.layers.0.")]
    W = {k: W16[k].astype(np.float32) for k in keep}

    def med(f, n=3):
        ts = []
        for _ in range(n):
            t = time.perf_counter()
            f()
            ts.append(time.perf_counter() - t)
        return float(np.median(ts)), ts

    m0 = mel[0].astype(np.float32)
    t_stem, _ = med(lambda: R.conv_stem(m0, W))
    x = R.conv_stem(m0, W)
    t_layer, _ = med(lambda: R.encoder_layer(x, W, 0, g.nh))
    t_xkv, _ = med(lambda: R.cross_kv(x, W, g.dec_layers, g.nh))
    xkv = R.cross_kv(x, W, g.dec_layers, g.nh)
    dec = R.Decoder(W, g.nh, g.dec_layers, [xkv] * N_CLIPS)
    toks = [gen["decoder_start_token_id"]] * N_CLIPS
    t0 = time.perf_counter()
    for p in range(2):
        dec.step(toks, p)
    t_step = (time.perf_counter() - t0) / 2
    enc = N_CLIPS * (t_stem + g.enc_layers * t_layer + t_xkv)
    total = enc + steps * t_step
    return {"value": N_CLIPS * 30.0 / total, "unit": "audio-sec/sec", "cores": int(threads), "kind": "port",
            "sample": (f"oracle fp32 numpy on {threads} BLAS threads ({os.cpu_count()} host cpus, "
                       f"{platform.processor() or platform.machine()}): conv stem {t_stem:.3f}s, one encoder layer "
                       f"{t_layer:.3f}s and cross k/v {t_xkv:.3f}s of one clip (median of 3), decoder step at "
                       f"B=32 {t_step:.3f}s (mean of 2); extrapolated to 32 clips x {g.enc_layers} layers + "
                       f"{steps} steps = {total:.1f}s")}


def probe(name: str, reps: int = 5):
    """Runs one encoder kernel class at the bench's shape (8 clips x 1500 frames, large-v3-turbo widths), or a plain
    device-to-device copy of known size, for counter runs (rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE)."""
    import ctypes as C
    from mimizuku_amd import _lib as L, model, synth
    g = synth.LARGE_V3_TURBO
    d, ff, nh = g.d, g.ff, g.nh
    M = EG * 1500
    ctx = model.Context(0)
    rng = np.random.default_rng(0)

    def f16(shape, sc=1.0):
        return (rng.standard_normal(shape, dtype=np.float32) * sc).astype(np.float16)

    if name == "copy":
        nbytes = 512 << 20
        a, b = ctx.alloc(nbytes), ctx.alloc(nbytes)
        for _ in range(reps):
            L.check(L.lib().mz_copy(ctx.h, b, a, nbytes))
        ctx.sync()
        print(json.dumps({"probe": "copy", "bytes_read": nbytes, "bytes_written": nbytes, "launches": reps}))
        return
    la = L.LinearArgs()
    x = ctx.upload_new(f16((M, ff)))
    w = ctx.upload_new(f16((g.dec_layers * 2 * d, 3 * d), 0.02))
    bias = ctx.upload_new(f16((g.dec_layers * 2 * d,), 0.02))
    out = ctx.alloc(M * max(ff, g.dec_layers * 2 * d) * 4)
    heads = ctx.alloc(EG * max(3, 2 * g.dec_layers) * nh * 1536 * 64 * 2)
    pos = ctx.upload_new(f16((1500, d)))
    for k, v in dict(a=x, lda=d, w=w, bias=bias, m=M, n=d, k=d, out=out, ldo=d).items():
        setattr(la, k, v)
    if name == "qkv":
        la.epilogue, la.n, la.heads, la.blocks_per_clip, la.nh, la.kind = L.EPI_HEADS, 3 * d, heads, 3 * nh, nh, 3
    elif name == "oproj":
        la.epilogue = L.EPI_F16
    elif name == "fc1":
        la.epilogue, la.n, la.ldo = L.EPI_GELU_F16, ff, ff
    elif name == "fc2":
        la.epilogue, la.k, la.lda = L.EPI_F16, ff, ff
    elif name == "conv1":
        la.epilogue, la.m, la.k = L.EPI_GELU_F16, EG * 3000, ((3 * g.n_mels + 63) // 64) * 64
        la.conv_cin, la.conv_tin, la.conv_tout, la.conv_stride = g.n_mels, 3000, 3000, 1
    elif name == "conv2":
        la.epilogue, la.k, la.pos = L.EPI_GELU_POS, 3 * d, pos
        la.conv_cin, la.conv_tin, la.conv_tout, la.conv_stride = d, 3000, 1500, 2
    elif name == "xkv":
        la.epilogue, la.n, la.heads, la.blocks_per_clip, la.nh, la.kind = (L.EPI_HEADS, g.dec_layers * 2 * d, heads,
                                                                         g.dec_layers * 2 * nh, nh, 2)
    elif name not in ("attn", "ln"):
        raise SystemExit(f"unknown probe {name}")
    lw, lb = ctx.upload_new(np.ones(d, np.float16)), ctx.upload_new(np.zeros(d, np.float16))
    for _ in range(reps):
        if name == "attn":
            L.check(L.lib().mz_enc_attention(ctx.h, heads, out, EG, nh))
        elif name == "ln":
            L.check(L.lib().mz_add_layernorm(ctx.h, out, x, lw, lb, heads, M, d, 1e-5))
        else:
            L.check(L.lib().mz_linear(ctx.h, C.byref(la)))
    ctx.sync()
    bound, amount = kernel_work(g, EG)[name]
    print(json.dumps({"probe": name, "launches": reps, "algorithmic": amount, "bound": bound}))


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=5)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU oracle baseline")
    ap.add_argument("--no-graph", action="store_true",
                    help="launch every decoder step's kernels instead of replaying the captured graph (as the "
                         "reference's --no-graph; for kernel tracers that do not follow graph launches)")
    ap.add_argument("--probe", default=None,
                    help="run one kernel class at the bench shape (or 'copy') for counter runs, then exit")
    a = ap.parse_args()
    if a.probe:
        probe(a.probe)
        return
    if a.gpus != 1:
        print("bench.py measures one GPU: this path shards over clips with no exchange step, and multi-GPU runs "
              "are not part of this build (use --gpus 1)", file=sys.stderr)
        sys.exit(2)

    import ctypes as C

    from mimizuku_amd import _lib as L
    from mimizuku_amd import model, synth, transcribe

    g = synth.LARGE_V3_TURBO
    log(f"bench: drawing large-v3-turbo weights (seed 0) and {N_CLIPS} log-mel clips")
    W = synth.random_weights(g, seed=0)
    gen = synth.generation_config(g)
    mel = synth.synthetic_mel(N_CLIPS, g.n_mels, seed=1)
    dims = model.Dims(g.d, g.ff, g.nh, g.enc_layers, g.dec_layers, g.n_mels, g.vocab, g.max_t)
    gc = model.GenCfg.from_dict(gen, dims)
    ctx = model.Context(0)
    e = model.Engine(ctx, dims, gc, N_CLIPS, EG)
    e.load(W)
    dmel = ctx.upload_new(mel)
    prompt = transcribe.Prompt(gc, "auto", "transcribe")
    log("bench: engine ready")

    def step():
        return transcribe.transcribe(e, dmel, prompt, max_new=MAX_NEW, n=N_CLIPS, graph=not a.no_graph)

    for i in range(a.warmup):
        out, tm = step()
        log(f"bench: warmup {i}: enc {tm.enc * 1e3:.1f} ms, dec {tm.dec * 1e3:.1f} ms ({tm.steps} steps), "
            f"post {tm.post * 1e3:.1f} ms")
    ctx.sync()
    t0 = time.perf_counter()
    tms = []
    for i in range(a.steps):
        out, tm = step()
        tms.append(tm)
    ctx.sync()
    dt = time.perf_counter() - t0
    ms_step = dt / a.steps * 1e3
    value = N_CLIPS * 30.0 / (dt / a.steps)
    enc_s = float(np.mean([t.enc for t in tms]))
    dec_s = float(np.mean([t.dec for t in tms]))
    post_s = float(np.mean([t.post for t in tms]))
    nsteps = tms[-1].steps
    log(f"bench: {a.steps} steps in {dt:.3f}s = {ms_step:.1f} ms/step, {value:.0f} audio-s/s")

    # Per-kernel timings: the transcription overlaps two encoder groups on two streams, so its launches share the GPU;
    # each kernel class is timed instead in one more encoder pass over the same clips with the groups one after the
    # other on the engine's stream (HIP events around every launch).
    e.profile(True)
    for g0 in range(0, N_CLIPS, EG):
        e.encode_device(dmel + g0 * g.n_mels * 3000 * 4, min(EG, N_CLIPS - g0), g0)
    ctx.sync()
    prof = e.profile_read()
    e.profile(False)
    work = kernel_work(g, EG)
    kernels = {}
    for name, (ms, n) in prof.items():
        if not n or name == "step":
            continue
        avg = ms / n * 1e-3
        bound, amount = work[name]
        peak = PEAK_F16 if bound == "mfma" else PEAK_HBM
        kernels[name] = {"launches": n, "avg_us": round(avg * 1e6, 2), "total_ms": round(ms, 3), "bound": bound,
                         ("tflops" if bound == "mfma" else "gbps"): round(amount / avg / (1e12 if bound == "mfma" else 1e9), 2),
                         "frac": round(amount / avg / peak, 4)}
    dom = max(kernels, key=lambda k: kernels[k]["total_ms"])
    dk = kernels[dom]
    bound, amount = work[dom]
    avg = dk["avg_us"] * 1e-6
    traffic, traffic_src = None, None
    tf = os.path.join(ROOT, "profiles", "traffic.json")  # HBM bytes per launch from rocprofv3 FETCH/WRITE_SIZE runs
    if os.path.exists(tf):
        with open(tf) as f:
            t = json.load(f).get(dom)
        if t:
            traffic, traffic_src = t["bytes_per_launch"], t["source"]
    roof = {"kernel": dom, "bound": bound, "achieved": round(amount / avg / (1e12 if bound == "mfma" else 1e9), 2),
            "peak": 2500.0 if bound == "mfma" else 8000.0, "unit": "TFLOP/s" if bound == "mfma" else "GB/s",
            "frac": dk["frac"], "traffic": traffic, "traffic_source": traffic_src,
            "per_launch": f"{amount / 1e9:.2f} G{'FLOP' if bound == 'mfma' else 'B'} ({EG} clips x 1500 frames)"}

    # decoder step alone at the 32-row batch, positions 200..219 (self-attention cache of 201..220 entries)
    rng = np.random.default_rng(7)
    nprompt = 200
    pr = rng.integers(0, 50000, size=(N_CLIPS, nprompt)).astype(np.int32)
    e.reset(pr)
    if a.no_graph:
        for _ in range(200):
            e.step(N_CLIPS, False, nprompt)
        ctx.sync()
        ev0, ev1 = ctx.event(), ctx.event()
        ctx.record(ev0)
        for _ in range(20):
            e.step(N_CLIPS, False, nprompt)
        ctx.record(ev1)
        step_us = ctx.elapsed_ms(ev0, ev1) / 20 * 1e3
    else:
        e.capture(N_CLIPS, nprompt)
        for _ in range(200):
            e.replay()
        ctx.sync()
        e.profile(True)
        for _ in range(20):
            e.replay()
        st_ms, st_n = e.profile_read()["step"]
        e.profile(False)
        step_us = st_ms / st_n * 1e3
    na = len(gen["alignment_heads"])
    step_bytes = float(np.mean([decode_step_bytes(g, N_CLIPS, p, na) for p in range(200, 220)]))
    log(f"bench: decode step at B=32, p=200..219: {step_us:.1f} us, "
        f"{step_bytes / (step_us * 1e-6) / 1e9:.0f} GB/s")

    # off the metric: the log-mel front end on the device for the same 32 clips as 30 s of 16 kHz audio
    rng = np.random.default_rng(3)
    audio = (0.1 * rng.standard_normal((N_CLIPS, 480000))).astype(np.float32)
    d_audio = ctx.upload_new(audio)
    d_feat = ctx.alloc(N_CLIPS * g.n_mels * 3000 * 4)
    ns = np.full(N_CLIPS, 480000, np.int32)
    fms = []
    for _ in range(3):
        t1 = time.perf_counter()
        L.check(L.lib().mz_log_mel(ctx.h, d_audio, ns.ctypes.data_as(C.c_void_p), N_CLIPS, g.n_mels, d_feat, None))
        fms.append((time.perf_counter() - t1) * 1e3)
    ctx.free(d_audio)
    ctx.free(d_feat)
    log(f"bench: log-mel of {N_CLIPS} x 30 s on the device: {min(fms):.2f} ms")

    res = {
        "metric": METRIC, "value": round(value, 2), "unit": "audio-sec/sec", "n_gpus": 1, "steps": a.steps,
        "warmup": a.warmup, "ms_per_step": round(ms_step, 3), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "f16",
        "data": "synthetic log-mel N(-0.3,0.4) clamped, seeded random-init weights (no checkpoint)",
        "config": {"workload": "large-v3-turbo end to end: 32 clips x 30 s, encoder groups of 8 (two at a time on two "
                               "streams), language detection, greedy <= 224 tokens (graph replay), token timestamps",
                   "batch": N_CLIPS, "enc_group": EG, "max_new_tokens": MAX_NEW, "decode_steps": nsteps,
                   "graph": not a.no_graph},
        "encoder_tflops": round(encoder_flops(g, N_CLIPS) / enc_s / 1e12, 2),
        "encoder_ms": round(enc_s * 1e3, 3), "decode_ms": round(dec_s * 1e3, 3), "post_ms": round(post_s * 1e3, 3),
        "decode_step_us": round(step_us, 2),
        "decode_step_hbm_frac": round(step_bytes / (step_us * 1e-6) / PEAK_HBM, 4),
        "decode_step_us_e2e_avg": round(dec_s / nsteps * 1e6, 2),
        "kernels": kernels,
        "kernel_timing": "HIP events around every launch of one extra encoder pass over the 32 clips with the groups "
                         "one after the other on one stream (the timed steps overlap two groups)",
        "roofline": roof,
        "features": {"clips": N_CLIPS, "ms": round(min(fms), 3),
                     "scope": "off the metric (the workload feeds log-mel): mz_log_mel over 32 x 30 s of 16 kHz audio "
                              "already in device memory, wall time of the synchronous call (tables, scratch, three "
                              "kernels), best of 3"},
    }
    if not a.no_cpu:
        log("bench: CPU oracle sample")
        res["cpu_baseline"] = cpu_baseline(g, W, gen, mel, nsteps)
    else:
        res["cpu_baseline"] = None
    e.close()
    ctx.close()
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
