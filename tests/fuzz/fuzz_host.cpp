// Mutation fuzzing of the host code that reads untrusted input, for an AddressSanitizer + UndefinedBehaviorSanitizer
// build (tests/test_host_sanitizers.py builds and runs it): the strict JSON parser, the safetensors reader, the model
// directory's config readers, the WAV reader and resampler, the tokenizer's decoding, and the token-timestamp
// routines on odd shapes. Each input starts from a valid document and takes random byte flips, insertions, deletions
// and truncations (a fixed seed, so a failure reproduces). A sanitizer report aborts the run; the exit status is 0
// otherwise. Return codes of the library calls are not checked: malformed input must be refused, never crash.
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/stat.h>
#include <unistd.h>

#include <random>
#include <string>
#include <vector>

#include "../../include/mimizuku.h"

static std::mt19937_64 rng(12345);
static size_t rnd(size_t n) { return n ? (size_t)(rng() % n) : 0; }

static std::string mutate(std::string s) {
    const int k = 1 + (int)rnd(6);
    for (int i = 0; i < k; i++) {
        switch (rnd(6)) {
            case 0: if (!s.empty()) s[rnd(s.size())] ^= (char)(1 << rnd(8)); break;
            case 1: s.insert(s.begin() + rnd(s.size() + 1), (char)rnd(256)); break;
            case 2: if (!s.empty()) s.erase(rnd(s.size()), 1 + rnd(8)); break;
            case 3: s.resize(rnd(s.size() + 1)); break;
            case 4: { static const char* toks[] = {"{", "}", "[", "]", "\"", ",", ":", "-1", "1e999", "\\u", "\\ud800",
                                                   "null", "99999999999999999999", "\xff", "\xc0\x80", "0.5"};
                      s.insert(rnd(s.size() + 1), toks[rnd(16)]); break; }
            default: if (s.size() > 1) { size_t a = rnd(s.size()), b = rnd(s.size()); std::swap(s[a], s[b]); } break;
        }
    }
    return s;
}

static void write_file(const std::string& path, const std::string& data) {
    FILE* f = fopen(path.c_str(), "wb");
    if (!f) { perror(path.c_str()); exit(2); }
    fwrite(data.data(), 1, data.size(), f);
    fclose(f);
}

static std::string le(uint64_t v, int n) {
    std::string s;
    for (int i = 0; i < n; i++) s.push_back((char)(v >> (8 * i)));
    return s;
}

static std::string safetensors(const std::string& header, size_t data_bytes) {
    return le(header.size(), 8) + header + std::string(data_bytes, '\x11');
}

static std::string wav(int fmt, int bits, int ch, int sr, int frames) {
    const int bpf = ch * bits / 8;
    std::string d;
    for (int i = 0; i < frames * bpf; i++) d.push_back((char)rnd(256));
    std::string fmtc = le(fmt, 2) + le(ch, 2) + le(sr, 4) + le((uint64_t)sr * bpf, 4) + le(bpf, 2) + le(bits, 2);
    std::string body = "WAVE" + std::string("fmt ") + le(fmtc.size(), 4) + fmtc + "data" + le(d.size(), 4) + d;
    return "RIFF" + le(body.size(), 4) + body;
}

int main(int argc, char** argv) {
    const int scale = argc > 1 ? atoi(argv[1]) : 1;
    char tmpl[] = "/tmp/mz_fuzz_XXXXXX";
    const std::string dir = mkdtemp(tmpl);
    long n_calls = 0;

    // ---- JSON
    const std::string docs[] = {
        R"({"d_model": 384, "encoder_layers": 4, "decoder_layers": 4, "encoder_attention_heads": 6, "decoder_attention_heads": 6, "encoder_ffn_dim": 1536, "num_mel_bins": 80, "vocab_size": 51865, "max_target_positions": 448, "max_source_positions": 1500})",
        R"({"alignment_heads": [[2, 2], [3, 0]], "begin_suppress_tokens": [220, 50257], "suppress_tokens": [1, 2, 7], "lang_to_id": {"<|en|>": 50259, "<|zh|>": 50260}, "task_to_id": {"transcribe": 50359}, "is_multilingual": true, "decoder_start_token_id": 50258, "eos_token_id": 50257, "no_timestamps_token_id": 50363})",
        R"({"__metadata__": {"format": "pt"}, "a": {"dtype": "F16", "shape": [2, 3], "data_offsets": [0, 12]}, "b": {"dtype": "F32", "shape": [1], "data_offsets": [12, 16]}})",
        R"(["é😀", 1.5e-3, -0, true, false, null, {"k": [[[]]]}])"};
    for (int it = 0; it < 20000 * scale; it++) {
        const std::string s = mutate(docs[rnd(4)]);
        mz_json_check(s.data(), s.size());
        n_calls++;
    }

    // ---- safetensors files
    const std::string st_path = dir + "/model.safetensors";
    for (int it = 0; it < 1500 * scale; it++) {
        std::string f = rnd(4) ? safetensors(mutate(docs[2]), 16) : mutate(safetensors(docs[2], 16));
        if (rnd(8) == 0) f = le(rnd(1u << 20), 8) + f.substr(std::min<size_t>(8, f.size()));
        write_file(st_path, f);
        mz_st* st = nullptr;
        if (mz_st_open(st_path.c_str(), &st) == MZ_OK) {
            int n = 0;
            mz_st_count(st, &n);
            for (int i = 0; i < n; i++) {
                const char *name, *dt;
                int nd;
                const int64_t* shape;
                const void* data;
                uint64_t bytes;
                if (mz_st_info(st, i, &name, &dt, &nd, &shape, &data, &bytes) == MZ_OK) {
                    volatile unsigned char sink = 0;
                    for (uint64_t b = 0; b < bytes; b++) sink ^= ((const unsigned char*)data)[b];
                    for (int d = 0; d < nd; d++) sink ^= (unsigned char)shape[d];
                    int j;
                    mz_st_find(st, name, &j);
                }
            }
            const char* v;
            mz_st_meta(st, "format", &v);
            mz_st_close(st);
        }
        n_calls++;
    }

    // ---- model directory configs
    for (int it = 0; it < 1000 * scale; it++) {
        write_file(dir + "/config.json", rnd(3) ? mutate(docs[0]) : docs[0]);
        write_file(dir + "/generation_config.json", rnd(3) ? mutate(docs[1]) : docs[1]);
        mz_model* m = nullptr;
        if (mz_model_open(dir.c_str(), &m) == MZ_OK) {
            mz_dims d;
            mz_gencfg g;
            mz_model_dims(m, &d);
            mz_model_gencfg(m, &g);
            for (int i = 0; i < g.n_langs + 2; i++) {
                const char* c;
                int32_t t;
                mz_model_lang(m, i, &c, &t);
                mz_model_task(m, i, &c, &t);
            }
            mz_model_free(m);
        }
        n_calls++;
    }

    // ---- WAV files and the resampler
    const std::string wav_path = dir + "/a.wav";
    const int fmts[][2] = {{1, 16}, {1, 24}, {1, 32}, {3, 32}, {1, 8}, {3, 64}};
    for (int it = 0; it < 800 * scale; it++) {
        const int* fb = fmts[rnd(6)];
        std::string w = wav(fb[0], fb[1], 1 + (int)rnd(3), (int)(1000 + rnd(50000)), (int)rnd(400));
        if (rnd(3)) w = mutate(w);
        write_file(wav_path, w);
        size_t n = 0;
        int sr = 0;
        if (mz_wav_read(wav_path.c_str(), nullptr, 0, &n, &sr) == MZ_OK && n < (1u << 24)) {
            std::vector<float> y(n + 1);
            if (mz_wav_read(wav_path.c_str(), y.data(), y.size(), &n, &sr) == MZ_OK) {
                size_t no = 0;
                if (mz_resample_16k(y.data(), n, sr, nullptr, 0, &no) == MZ_OK && no < (1u << 24)) {
                    std::vector<float> out(no + 1);
                    mz_resample_16k(y.data(), n, sr, out.data(), out.size(), &no);
                }
            }
        }
        n_calls++;
    }

    // ---- tokenizer decoding over random byte strings and ids
    for (int it = 0; it < 2000 * scale; it++) {
        const int nv = 1 + (int)rnd(300);
        std::vector<std::string> ent(nv);
        std::vector<const char*> ptrs(nv);
        std::vector<size_t> lens(nv);
        for (int i = 0; i < nv; i++) {
            ent[i].resize(rnd(6));
            for (auto& c : ent[i]) c = (char)rnd(256);
            ptrs[i] = ent[i].data();
            lens[i] = ent[i].size();
        }
        mz_tok* t = nullptr;
        if (mz_tok_from_bytes(ptrs.data(), lens.data(), nv, &t) == MZ_OK) {
            const int n = (int)rnd(40);
            std::vector<int32_t> ids(n);
            std::vector<float> ts(n);
            for (int i = 0; i < n; i++) {
                ids[i] = (int32_t)rnd(nv + 20) - 5;
                ts[i] = (float)i * 0.02f;
            }
            char buf[512];
            size_t len;
            mz_tok_decode(t, ids.data(), n, buf, rnd(2) ? sizeof buf : rnd(8), &len);
            std::vector<int32_t> off(n + 1);
            std::vector<float> t0(n), t1(n);
            int np;
            mz_tok_pieces(t, ids.data(), ts.data(), n, (int)rnd(nv + 1), buf, rnd(2) ? sizeof buf : rnd(8), &len,
                          off.data(), t0.data(), t1.data(), &np);
            mz_tok_free(t);
        }
        char jt[32];
        size_t jl;
        const float vals[] = {0.f, 0.125f, 29.999f, -1.f, 1e30f, 3.005f};
        mz_json_time(vals[rnd(6)], jt, rnd(2) ? sizeof jt : rnd(4), &jl);
        n_calls++;
    }

    // ---- token timestamps on odd shapes
    for (int it = 0; it < 1500 * scale; it++) {
        const int rows = 1 + (int)rnd(12), heads = 1 + (int)rnd(4), full = 1 + (int)rnd(40), cols = (int)rnd(full + 1);
        const int width = 1 + 2 * (int)rnd(8);
        std::vector<float> w((size_t)rows * heads * full);
        for (auto& v : w) v = rnd(10) == 0 ? 0.f : (float)rnd(1000) / 1000.f;
        std::vector<float> out(rows);
        mz_jump_times(w.data(), rows, heads, full, cols, width, (int)rnd(2), out.data());
        if (cols > 0) {
            std::vector<double> m((size_t)rows * cols);
            mz_align_cost(w.data(), rows, heads, full, cols, width, (int)rnd(2), m.data());
            std::vector<int32_t> a(rows + cols), b(rows + cols);
            int32_t len;
            mz_dtw(m.data(), rows, cols, a.data(), b.data(), &len);
        }
        n_calls++;
    }
    unlink(st_path.c_str());
    unlink(wav_path.c_str());
    unlink((dir + "/config.json").c_str());
    unlink((dir + "/generation_config.json").c_str());
    rmdir(dir.c_str());
    printf("fuzz_host: %ld inputs, no sanitizer report\n", n_calls);
    return 0;
}
