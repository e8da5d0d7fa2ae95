"""The host code that reads untrusted input, built with AddressSanitizer and UndefinedBehaviorSanitizer (ROCm's
clang++ as a plain host C++ compiler: no offload, the device code stays out of the build) and run over mutated inputs
(tests/fuzz/fuzz_host.cpp): the strict JSON parser, the safetensors reader, the config readers, the WAV reader and
resampler, the tokenizer's decoding and the token-timestamp routines. The functions these sources call from the rest
of the library (the engine, for the model-directory loader) resolve against libmimizuku_amd.so; only the listed
sources are instrumented."""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "mimizuku_amd", "csrc")
SOURCES = ["json.cpp", "st.cpp", "tok.cpp", "audio.cpp", "align.cpp"]


CXX = "/opt/rocm/llvm/bin/clang++"


@pytest.mark.skipif(not os.path.exists(CXX), reason="ROCm clang++ not installed")
def test_host_parsers_under_sanitizers(tmp_path):
    lib = os.path.join(ROOT, "mimizuku_amd", "libmimizuku_amd.so")
    if not os.path.exists(lib):
        pytest.skip("libmimizuku_amd.so is not built")
    exe = str(tmp_path / "fuzz_host")
    san = ["-fsanitize=address,undefined", "-fno-sanitize-recover=undefined", "-fno-omit-frame-pointer"]
    cmd = ([CXX, "-std=c++17", "-O1", "-g", *san, "-mf16c", "-mavx2", "-D__HIP_PLATFORM_AMD__",
            "-I/opt/rocm/include", "-Wno-deprecated-declarations"]
           + [os.path.join(CSRC, s) for s in SOURCES]
           + [os.path.join(ROOT, "tests", "fuzz", "fuzz_host.cpp"), "-o", exe,
              f"-L{os.path.dirname(lib)}", "-lmimizuku_amd", f"-Wl,-rpath,{os.path.dirname(lib)}",
              "-L/opt/rocm/lib", "-lamdhip64", "-Wl,-rpath,/opt/rocm/lib", "-lpthread"])
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-4000:]
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=0:abort_on_error=1",
               UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1")
    r = subprocess.run([exe, "1"], capture_output=True, text=True, env=env, timeout=600)
    assert r.returncode == 0, (r.stdout[-2000:], r.stderr[-6000:])
    assert "no sanitizer report" in r.stdout
