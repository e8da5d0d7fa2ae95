// The mimizuku command line (src/main.rs:1-224) as a library call, mz_cli(argc, argv), over the library's own C ABI:
// WAV files -> 16 kHz (host threads) -> log-mel (device) -> encoder groups and graph-replayed greedy decoding in
// batches -> token timestamps -> {path: {"language", "text", "words": [[piece, start, end], ...]}}. The executable
// mimizuku_amd/mimizuku is a main() around it; callers that already drive the GPU run it in their own process.
#include <dirent.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <atomic>
#include <chrono>
#include <string>
#include <thread>
#include <vector>

#include "../../include/mimizuku.h"
#include "mz_internal.h"

namespace {

const char* USAGE =
    "usage: mimizuku --model DIR [options] FILE.wav...\n"
    "       mimizuku --model DIR [options] --dir DIR\n"
    "\n"
    "Transcribes WAV clips of up to 30 s with a Whisper checkpoint in Hugging Face format (model.safetensors,\n"
    "config.json, generation_config.json, vocab.json), greedy decoding, with a start and end time for every\n"
    "character or word piece. Writes JSON: {path: {\"language\", \"text\", \"words\": [[piece, start, end], ...]}}.\n"
    "\n"
    "options:\n"
    "  --model DIR        model directory (required)\n"
    "  --dir DIR          every .wav file in DIR, sorted by name\n"
    "  --prefix STR       with --dir: only files whose name starts with STR\n"
    "  --language CODE    language code such as en or ja; auto (default) detects it per clip\n"
    "  --task NAME        transcribe (default) or translate (into English)\n"
    "  --out FILE         write the JSON to FILE instead of standard output\n"
    "  --batch N          clips decoded together (default 32); lower it if GPU memory is short\n"
    "  --enc-group N      clips per encoder pass (default 8)\n"
    "  --quiet            no progress or timing on standard error\n"
    "development:\n"
    "  --no-graph         launch every decoding step's kernels instead of replaying a HIP graph\n";

constexpr int NS = 480000;  // 30 s at 16 kHz

struct Err {
    std::string msg;
};

void check(int rc) {
    if (rc != MZ_OK) throw Err{mz_last_error()};
}

double now() {
    return std::chrono::duration<double>(std::chrono::steady_clock::now().time_since_epoch()).count();
}

struct Args {
    std::vector<std::pair<std::string, std::string>> opts;
    std::vector<std::string> flags, files;

    static Args parse(int argc, const char* const* argv) {
        static const char* WITH_VALUE[] = {"--model", "--dir", "--prefix", "--language", "--task", "--out",
                                           "--batch", "--enc-group", "--ref", "--enc-attn"};
        static const char* FLAGS[] = {"--quiet", "--no-graph", "--help", "-h"};
        Args a;
        for (int i = 1; i < argc; i++) {
            const std::string s = argv[i];
            bool done = false;
            for (const char* w : WITH_VALUE)
                if (s == w) {
                    if (i + 1 >= argc) throw Err{s + " needs a value"};
                    a.opts.emplace_back(s, argv[++i]);
                    done = true;
                }
            for (const char* f : FLAGS)
                if (!done && s == f) {
                    a.flags.push_back(s);
                    done = true;
                }
            if (done) continue;
            if (!s.empty() && s[0] == '-') throw Err{"unknown option " + s + " (see --help)"};
            a.files.push_back(s);
        }
        return a;
    }
    const char* get(const char* k) const {  // the last occurrence wins
        for (auto it = opts.rbegin(); it != opts.rend(); ++it)
            if (it->first == k) return it->second.c_str();
        return nullptr;
    }
    bool flag(const char* k) const { return std::find(flags.begin(), flags.end(), k) != flags.end(); }
    int positive(const char* k, int dflt) const {
        const char* v = get(k);
        if (!v) return dflt;
        char* end = nullptr;
        const long n = strtol(v, &end, 10);
        if (!*v || *end || n <= 0 || n > (1 << 20)) throw Err{std::string(k) + ": expected a positive integer, got " + v};
        return (int)n;
    }
};

std::vector<std::string> list_dir(const std::string& d, const std::string& prefix) {
    DIR* dir = opendir(d.c_str());
    if (!dir) throw Err{d + ": cannot read the directory"};
    std::vector<std::string> v;
    std::string base = d;
    while (!base.empty() && base.back() == '/') base.pop_back();
    while (dirent* e = readdir(dir)) {
        std::string n = e->d_name, low = n;
        for (char& c : low) c = (char)tolower((unsigned char)c);
        if (n.compare(0, prefix.size(), prefix) == 0 && low.size() >= 4 && low.compare(low.size() - 4, 4, ".wav") == 0)
            v.push_back(base + "/" + n);
    }
    closedir(dir);
    std::sort(v.begin(), v.end());
    return v;
}

struct Clip {
    std::string path;
    std::vector<float> y;  // 16 kHz samples, at most 30 s
    std::string err;
};

// WAV -> 16 kHz for every file, on all cores (features, src/transcribe.rs:27-55, minus the log-mel)
std::vector<Clip> load_audio(const std::vector<std::string>& paths) {
    std::vector<Clip> clips(paths.size());
    std::atomic<size_t> next{0};
    const size_t workers = std::max<size_t>(1, std::min<size_t>(std::thread::hardware_concurrency(), paths.size()));
    std::vector<std::thread> pool;
    for (size_t w = 0; w < workers; w++)
        pool.emplace_back([&] {
            for (size_t i; (i = next.fetch_add(1)) < paths.size();) {
                Clip& c = clips[i];
                c.path = paths[i];
                size_t n = 0, m = 0;
                int sr = 0;
                if (mz_wav_read(c.path.c_str(), nullptr, 0, &n, &sr) != MZ_OK) {
                    c.err = mz_last_error();
                    continue;
                }
                std::vector<float> raw(n);
                if (mz_wav_read(c.path.c_str(), raw.data(), n, &n, &sr) != MZ_OK ||
                    mz_resample_16k(raw.data(), n, sr, nullptr, 0, &m) != MZ_OK) {
                    c.err = c.path + ": " + mz_last_error();
                    continue;
                }
                if (m > (size_t)NS) {
                    char b[256];
                    snprintf(b, sizeof b, ": %.1f s is longer than Whisper's 30 s window; split it into shorter clips",
                             m / 16000.0);
                    c.err = c.path + b;
                    continue;
                }
                c.y.resize(m);
                if (mz_resample_16k(raw.data(), n, sr, c.y.data(), m, &m) != MZ_OK) c.err = c.path + ": " + mz_last_error();
            }
        });
    for (auto& t : pool) t.join();
    for (auto& c : clips)
        if (!c.err.empty()) throw Err{c.err};
    return clips;
}

int run(int argc, const char* const* argv) {
    const Args args = Args::parse(argc, argv);
    if (args.flag("--help") || args.flag("-h")) {
        fputs(USAGE, stdout);
        return 0;
    }
    const bool quiet = args.flag("--quiet");
    auto log = [&](const char* fmt, auto... v) {
        if (!quiet) {
            fprintf(stderr, fmt, v...);
            fputc('\n', stderr);
        }
    };
    const char* model_dir = args.get("--model");
    if (!model_dir) throw Err{"--model is required (see --help)"};
    if (args.get("--ref")) throw Err{"--ref: the reference-comparison mode is not supported by this tool"};
    if (args.get("--enc-attn") && !strcmp(args.get("--enc-attn"), "cublas"))
        throw Err{"--enc-attn cublas: only the fused encoder attention is available"};
    const double t_start = now();

    std::vector<std::string> paths = args.files;
    if (const char* d = args.get("--dir")) {
        auto more = list_dir(d, args.get("--prefix") ? args.get("--prefix") : "");
        paths.insert(paths.end(), more.begin(), more.end());
    }
    if (paths.empty()) throw Err{"no input files (see --help)"};
    mz_model* md = nullptr;
    check(mz_model_open(model_dir, &md));
    mz_dims dims;
    mz_gencfg gc;
    check(mz_model_dims(md, &dims));
    check(mz_model_gencfg(md, &gc));
    const int bmax = std::min<int>(args.positive("--batch", 32), (int)paths.size());
    const int eg = std::min(args.positive("--enc-group", 8), bmax);

    double t0 = now();
    std::vector<Clip> clips = load_audio(paths);
    double t_feat = now() - t0;

    t0 = now();
    mz_ctx* ctx = nullptr;
    check(mz_init(0, &ctx));
    size_t free0 = 0, total = 0, free1 = 0;
    check(mz_mem_info(ctx, &free0, &total));
    const double t_setup = now() - t0;
    mz_engine* e = nullptr;
    check(mz_engine_open(ctx, model_dir, bmax, eg, &e));
    mz_tok* tk = nullptr;
    check(mz_tok_open(model_dir, dims.vocab, gc.eos, &tk));
    check(mz_mem_info(ctx, &free1, &total));
    const double t_load = now() - t0;
    log("model on the GPU: %.1f GB allocated in %.1fs (HIP setup %.1fs, weights %.1fs)", (free0 - free1) / 1e9, t_load,
        t_setup, t_load - t_setup);

    // the prompt (Prompt::new, src/transcribe.rs:69-84)
    const char* language = args.get("--language") ? args.get("--language") : "auto";
    const char* task = args.get("--task") ? args.get("--task") : "transcribe";
    const bool multilingual = gc.n_langs > 0;
    int32_t lang = -1, task_tok = -1;
    if (!multilingual) {
        if ((strcmp(language, "auto") && strcmp(language, "en")) || strcmp(task, "transcribe"))
            throw Err{"this English-only model takes only --language en (or auto) and --task transcribe"};
    } else {
        if (strcmp(language, "auto")) {
            for (int i = 0; i < gc.n_langs; i++) {
                const char* code;
                int32_t t;
                check(mz_model_lang(md, i, &code, &t));
                if (!strcmp(code, language)) lang = t;
            }
            if (lang < 0) throw Err{std::string("--language ") + language + ": not a language of this model"};
        }
        for (int i = 0;; i++) {
            const char* name;
            int32_t t;
            if (mz_model_task(md, i, &name, &t) != MZ_OK) break;
            if (!strcmp(name, task)) {
                task_tok = t;
                break;
            }
        }
        if (task_tok < 0) throw Err{std::string("--task ") + task + ": unknown task"};
    }
    std::vector<int32_t> prompt = multilingual ? std::vector<int32_t>{gc.sot, lang >= 0 ? lang : gc.sot, task_tok,
                                                                      gc.no_timestamps}
                                               : std::vector<int32_t>{gc.sot, gc.no_timestamps};
    const int detect = multilingual && lang < 0;

    // device buffers for one batch: 16 kHz audio and its log-mel
    uint64_t d_audio = 0, d_mel = 0;
    check(mz_alloc(ctx, (size_t)bmax * NS * 4, &d_audio));
    check(mz_alloc(ctx, (size_t)bmax * dims.n_mels * 3000 * 4, &d_mel));
    const int mt = dims.max_t;
    const int n = (int)clips.size();
    std::vector<int32_t> seq((size_t)n * mt), seq_len(n), langs(n), frames(n);
    std::vector<float> ts((size_t)n * mt);
    mz_times tm{};
    std::vector<float> host((size_t)bmax * NS);
    for (int c0 = 0; c0 < n; c0 += bmax) {
        const int cn = std::min(bmax, n - c0);
        t0 = now();
        std::vector<int32_t> ns(cn);
        std::fill(host.begin(), host.end(), 0.f);
        for (int i = 0; i < cn; i++) {
            const auto& y = clips[c0 + i].y;
            std::copy(y.begin(), y.end(), host.begin() + (size_t)i * NS);
            ns[i] = (int32_t)y.size();
        }
        check(mz_upload(ctx, d_audio, host.data(), (size_t)cn * NS * 4));
        check(mz_log_mel(ctx, d_audio, ns.data(), cn, dims.n_mels, d_mel, frames.data() + c0));
        t_feat += now() - t0;
        mz_times ct{};
        check(mz_transcribe_device(e, d_mel, frames.data() + c0, cn, prompt.data(), (int)prompt.size(), detect,
                                   !args.flag("--no-graph"), 0, 1, seq.data() + (size_t)c0 * mt, seq_len.data() + c0,
                                   ts.data() + (size_t)c0 * mt, langs.data() + c0, &ct));
        tm.enc += ct.enc;
        tm.dec += ct.dec;
        tm.post += ct.post;
        tm.steps += ct.steps;
        log("decoded %d clips: %d steps in %.2fs = %.1f ms/step", cn, ct.steps, ct.dec,
            ct.steps ? 1000.0 * ct.dec / ct.steps : 0.0);
    }

    t0 = now();
    std::vector<const char*> cpaths(n);
    for (int i = 0; i < n; i++) cpaths[i] = clips[i].path.c_str();
    size_t len = 0;
    check(mz_results_json(tk, md, n, cpaths.data(), seq.data(), seq_len.data(), mt, ts.data(), langs.data(), nullptr,
                          0, &len));
    std::string out(len + 1, '\0');
    check(mz_results_json(tk, md, n, cpaths.data(), seq.data(), seq_len.data(), mt, ts.data(), langs.data(), &out[0],
                          out.size(), &len));
    out.resize(len);
    if (const char* p = args.get("--out")) {
        FILE* f = fopen(p, "wb");
        if (!f || fwrite(out.data(), 1, out.size(), f) != out.size()) {
            if (f) fclose(f);
            throw Err{std::string(p) + ": cannot write"};
        }
        fclose(f);
    } else {
        fwrite(out.data(), 1, out.size(), stdout);
    }
    tm.post += now() - t0;
    double audio_s = 0;
    for (int f : frames) audio_s += f / 100.0;
    log("%d clips (%.1fs of audio), batch %d, encoder group %d: features %.2fs | model load %.1fs | encoder %.2fs | "
        "decode %.2fs (%d steps) | timestamps+text %.2fs | without load %.2fs | total %.1fs",
        n, audio_s, bmax, eg, t_feat, t_load, tm.enc, tm.dec, tm.steps, tm.post, t_feat + tm.enc + tm.dec + tm.post,
        now() - t_start);
    mz_tok_free(tk);
    mz_engine_free(e);
    mz_model_free(md);
    mz_ctx_free(ctx);
    return 0;
}

}  // namespace

extern "C" int mz_cli(int argc, const char* const* argv) {
    int rc;
    try {
        rc = run(argc, argv);
    } catch (const Err& e) {
        fprintf(stderr, "error: %s\n", e.msg.c_str());
        rc = 1;
    }
    // the caller's process goes on: hand everything written so far to the file descriptors
    fflush(stdout);
    fflush(stderr);
    return rc;
}
