"""mimizuku_amd: the Whisper compute path of hayatree/mimizuku, native to MI355X (gfx950).

The compute lives in `libmimizuku_amd.so` (hand-written HIP kernels + a C++ engine behind a C ABI, declared in
include/mimizuku.h). This package is the host-side mirror of the reference's Rust surface: `model` (Dims, GenCfg,
Engine), `transcribe` (Prompt, transcribe) and `synth` (seeded random-init checkpoints and inputs).
"""
