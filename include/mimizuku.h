/* mimizuku_amd — C ABI of the MI355X (gfx950) Whisper compute path.
 *
 * This is the drop-in boundary that replaces the reference's cudarc-based device layer (src/gpu.rs), its CUDA
 * kernels (kernels/whisper.cu) and its engine (src/model.rs, src/transcribe.rs). Plain C: opaque handles, device
 * pointers as uint64_t (as the reference's `Ptr = u64`, src/gpu.rs:12), sizes in bytes or elements as stated.
 * Every function returns 0 on success or a nonzero MZ_ERR_* code; mz_last_error() then holds a message for the
 * calling thread (the reference returns R<T> = Result<T, Box<dyn Error>>, src/gpu.rs:11).
 *
 * Work is enqueued on the context's one non-default stream (src/gpu.rs:125); functions that return host data
 * synchronise it. One host thread drives one context.
 */
#ifndef MIMIZUKU_H
#define MIMIZUKU_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MZ_OK 0
#define MZ_ERR_HIP 1   /* HIP runtime error or no device */
#define MZ_ERR_ARG 2   /* invalid argument, shape or size */
#define MZ_ERR_STATE 3 /* call out of order (e.g. step before weights are loaded) */

typedef struct mz_ctx mz_ctx;
typedef struct mz_graph mz_graph;
typedef struct mz_engine mz_engine;

/* Message of the last failed call on this thread ("" if none). */
const char* mz_last_error(void);
const char* mz_version(void);

/* ------------------------------------------------------------------ runtime (src/gpu.rs `Gpu`) */

/* Device `device`, one non-blocking stream. Replaces Gpu::new (src/gpu.rs:122-137); no library handles. */
int mz_init(int device, mz_ctx** out);
int mz_ctx_free(mz_ctx* c);
/* Zero-filled device buffer of max(bytes, 16) bytes (Gpu::alloc, src/gpu.rs:140-145). Freed by mz_free or at
 * mz_ctx_free. */
int mz_alloc(mz_ctx* c, size_t bytes, uint64_t* dptr);
int mz_free(mz_ctx* c, uint64_t dptr);
/* (free, total) device bytes (Gpu::mem_info, src/gpu.rs:152-154). */
int mz_mem_info(mz_ctx* c, size_t* free_bytes, size_t* total_bytes);
/* Host -> device, then synchronise (Gpu::upload, src/gpu.rs:160-163). */
int mz_upload(mz_ctx* c, uint64_t dst, const void* src, size_t bytes);
/* Device -> host after the stream's work (Gpu::download, src/gpu.rs:171-176). */
int mz_download(mz_ctx* c, void* dst, uint64_t src, size_t bytes);
/* Device -> device, asynchronous and capturable (Gpu::copy, src/gpu.rs:249-252). */
int mz_copy(mz_ctx* c, uint64_t dst, uint64_t src, size_t bytes);
int mz_sync(mz_ctx* c); /* Gpu::sync, src/gpu.rs:182-185 */
/* Timing events on the context's stream. */
int mz_event_create(mz_ctx* c, uint64_t* ev);
int mz_event_record(mz_ctx* c, uint64_t ev);
int mz_event_elapsed_ms(uint64_t start, uint64_t stop, float* ms);
int mz_event_destroy(uint64_t ev);

/* Stream capture into a replayable graph (cudarc begin_capture / end_capture / Graph::{upload, launch},
 * src/transcribe.rs:123-135): thread-local capture mode, graph uploaded once, one launch per replay. */
int mz_graph_begin(mz_ctx* c);
int mz_graph_end(mz_ctx* c, mz_graph** out);
int mz_graph_launch(mz_ctx* c, mz_graph* g);
int mz_graph_free(mz_graph* g);

/* ------------------------------------------------------------------ kernels (device pointers, the ctx stream) */

/* y[m][n] (row stride ldy, fp16) = x[m][k] (row stride ldx) . W[n][k]^T + bias[n] (bias may be 0), fp32
 * accumulation, one rounding — the semantics of Gpu::gemm (src/gpu.rs:208-236). k % 64 == 0, n % 4 == 0.
 * m <= 32 per tile uses the decode-sized kernel (the reference's gemv_* for m <= 8), larger m the tiled MFMA GEMM
 * (cuBLAS there). */
int mz_gemm(mz_ctx* c, uint64_t x, int ldx, uint64_t w, uint64_t y, int ldy, int m, int n, int k, uint64_t bias);

#define MZ_EPI_F16 0       /* out f16 [m][ldo] = acc + bias */
#define MZ_EPI_GELU_F16 1  /* out f16 [m][ldo] = gelu(acc + bias) (fc1; gelu_inplace fused, whisper.cu:106-113) */
#define MZ_EPI_RESID_F32 2 /* out f32 [m][ldo] += acc + bias (residual add fused into out-proj / fc2) */
#define MZ_EPI_GELU_POS 3  /* out f32 [m][ldo] = gelu(acc + bias) + pos[m % 1500][n] (conv2 + add_pos, whisper.cu:115-119) */
#define MZ_EPI_HEADS 4     /* scatter into 1536 x 64 per-head tiles (see mz_linear_args) */

/* One encoder-sized product on the tiled MFMA kernel (replaces fill_bias + cublasGemmStridedBatchedEx,
 * src/gpu.rs:229-235, and im2col1/im2col2, whisper.cu:121-139, when conv_cin > 0). */
typedef struct {
    int epilogue;
    uint64_t a;   /* f16 [m][lda]; with conv_cin > 0 the conv source rows [clips * conv_tin][conv_cin] */
    long lda;
    uint64_t w;   /* f16 [n][k]; for a conv, columns ordered tap-major: w'[co][tap * cin + ci] */
    uint64_t bias;
    int m, n, k;
    uint64_t out;
    long ldo;
    uint64_t pos; /* MZ_EPI_GELU_POS: f16 [1500][n] */
    /* MZ_EPI_HEADS: column n -> block n / 64, row m -> clip m / 1500, time m % 1500; the block's tile is at
     * heads + ((slot0 + clip) * blocks_per_clip + block) * 1536 * 64 halves. kind 3: blocks [q|k|v][head] (encoder
     * self-attention; the q tiles stored multiplied by log2(e) / 8, the v tiles transposed [64][1536]), kind 2:
     * [layer][k|v][head] (cross-attention; every tile row-major [1536][64]). Requires n % 64 == 0, m a whole number
     * of clips and 1 <= blocks_per_clip <= 4096 (large-v3's cross k/v: 32 x 2 x 20 = 1280). */
    uint64_t heads;
    int blocks_per_clip, nh, kind, slot0;
    /* implicit conv1d (kernel 3, padding 1): A[clip * conv_tout + t][tap * cin + ci] =
     * src[(clip * conv_tin + conv_stride * t + tap - 1) * cin + ci], zero outside; k >= 3 * cin padded with 0 */
    int conv_cin, conv_tin, conv_tout, conv_stride;
} mz_linear_args;
int mz_linear(mz_ctx* c, const mz_linear_args* a);

/* y[r] = LayerNorm(x[r]) for fp32 rows x (row stride ldx) into fp16 y (layernorm, whisper.cu:65-69). */
int mz_layernorm(mz_ctx* c, uint64_t x, long ldx, uint64_t w, uint64_t b, uint64_t y, long ldy, int rows, int dim,
                 float eps);
/* x[r] += d[r] (fp32 x, fp16 d) in place, then y[r] = LayerNorm(x[r]) (add_layernorm, whisper.cu:71-82). */
int mz_add_layernorm(mz_ctx* c, uint64_t x, uint64_t d, uint64_t w, uint64_t b, uint64_t y, int rows, int dim,
                     float eps);
/* Encoder self-attention (enc_flash, whisper.cu:168-299): qkvh [clips][3][nh] tiles of 1536 x 64 halves
 * (q, k as [t][64]; v transposed [64][t]; t >= 1500 zero) -> out f16 [clips * 1500][nh * 64]; scale 1/8. The q tiles
 * hold q multiplied by log2(e) / 8, as the QKV product (mz_linear, EPI_HEADS, kind 3) writes them. */
int mz_enc_attention(mz_ctx* c, uint64_t qkvh, uint64_t out, int clips, int nh);
/* log-mel f32 [clips][n_mels][3000] -> f16 [clips][3000][n_mels] (the conv stem's source layout). */
int mz_mel_transpose(mz_ctx* c, uint64_t mel, uint64_t melT, int clips, int n_mels);

/* ------------------------------------------------------------------ engine (src/model.rs, src/transcribe.rs) */

/* Model geometry (Dims, src/model.rs:14-25). */
typedef struct {
    int d, ff, nh, enc_layers, dec_layers, n_mels, vocab, max_t;
} mz_dims;

/* Generation settings (GenCfg, src/model.rs:64-76), as plain arrays. */
typedef struct {
    int sot, eos, no_timestamps;
    const int32_t* suppress;
    int n_suppress;
    const int32_t* begin_suppress; /* at most 2 */
    int n_begin_suppress;
    const int32_t* lang_tokens; /* language tokens (detection restricts the choice to these) */
    int n_langs;
    const int32_t* align_heads; /* (layer, head) pairs */
    int n_align;
} mz_gencfg;

/* Device bytes the engine allocates besides the weights (scratch_bytes, src/model.rs:324-330). */
size_t mz_scratch_bytes(const mz_dims* d, int n_align, int bmax, int eg);
/* Validates the geometry (Dims::load checks, src/model.rs:47-59) and allocates the engine for bmax decoded rows and
 * eg clips per encoder pass (Engine::new, src/model.rs:333-514, minus reading files). Beyond the reference's limits
 * the library needs d % 128 == 0 and d <= 1280 (every Whisper size; larger widths are refused with MZ_ERR_ARG);
 * bmax has no upper limit besides memory, as the reference's --batch. */
int mz_engine_new(mz_ctx* c, const mz_dims* d, const mz_gencfg* g, int bmax, int eg, mz_engine** out);
#define MZ_DT_F16 0
#define MZ_DT_F32 1
/* Places one checkpoint tensor by its Hugging Face name (Loader, src/model.rs:200-265): shape-checked, F32
 * converted to F16, q/k/v fused (zero k bias), every decoder layer's cross k/v fused, conv weights reordered
 * tap-major. Unknown names are ignored. The data is converted into two pinned 32 MB staging buffers in turn, each
 * one's copy to the device in flight while the next chunk is converted (the reference's Arena, src/gpu.rs:289-374);
 * `data` may be reused when the call returns. */
int mz_engine_put(mz_engine* e, const char* name, int dtype, const void* data, const int64_t* shape, int ndim);
/* Checks every tensor was placed, waits for the uploads and frees the staging buffers (Arena::finish,
 * src/gpu.rs:363-373). */
int mz_engine_finish(mz_engine* e);
/* Every tensor of <model_dir>/model.safetensors through mz_engine_put, then mz_engine_finish (the Loader over the
 * mapped checkpoint, src/model.rs:200-265 with src/st.rs; F16 and F32 tensors, anything else is an error). */
int mz_engine_load(mz_engine* e, const char* model_dir);
/* Engine::new (src/model.rs:333-514) from a Hugging Face model directory: config.json and generation_config.json
 * through mz_model_open, mz_engine_new, then mz_engine_load. */
int mz_engine_open(mz_ctx* c, const char* model_dir, int bmax, int eg, mz_engine** out);
/* Encoder for n <= eg clips of log-mel f32 [n][n_mels][3000] (host); writes every decoder layer's cross k/v into
 * decoder slots slot0 .. slot0 + n - 1 (Engine::encode, src/model.rs:545-625). The log-mel goes through a pinned
 * buffer of the engine and an asynchronous copy (the host array may be reused when the call returns). */
int mz_engine_encode(mz_engine* e, const float* mels, int n, int slot0);
/* As mz_engine_encode with the log-mel already in device memory (f32 [n][n_mels][3000] at `mels`): no host copy. */
int mz_engine_encode_device(mz_engine* e, uint64_t mels, int n, int slot0);
/* Prompt tokens [n][prompt_len] into rows 0..n-1, every row unfinished, position 0 (Engine::reset, :628-637). */
int mz_engine_reset(mz_engine* e, const int32_t* prompts, int n, int prompt_len);
/* One step on the start token restricted to language tokens; writes token 1 of each row and returns them in
 * langs[b] (Engine::detect, :641-646). */
int mz_engine_detect(mz_engine* e, int b, int32_t* langs);
/* One greedy step for rows 0..b-1: feed token p, choose token p + 1 (positions below prompt_len stay), p += 1
 * (Engine::step, :650-736). lang != 0 restricts the choice to language tokens. */
int mz_engine_step(mz_engine* e, int b, int lang, int prompt_len);
/* Capture step(b, 0, prompt_len) once as a graph and upload it; replay launches it (transcribe.rs:123-142). */
int mz_engine_capture(mz_engine* e, int b, int prompt_len);
int mz_engine_replay(mz_engine* e);
/* Keep a copy of every encoder layer's input (fp32 residual stream) of the next encode (Engine::trace), and of the
 * decoder residual entering every layer of each eager step (MZ_BUF_DEC_TRACE). */
int mz_engine_set_trace(mz_engine* e, int on);

/* Kernel timing (the reference's stage timings, src/main.rs:213-222, at kernel granularity): with profiling on, every
 * encoder launch, every kernel of an eager decoder step and every graph replay is bracketed by events on the
 * engine's stream. mz_engine_profile clears the records; mz_engine_profile_read sums the elapsed time and counts the
 * launches of one kernel class. */
#define MZ_K_MEL 0   /* log-mel layout change */
#define MZ_K_CONV1 1 /* conv1 + GELU (implicit GEMM) */
#define MZ_K_CONV2 2 /* conv2 + GELU + positions */
#define MZ_K_LN 3    /* encoder LayerNorm */
#define MZ_K_QKV 4   /* fused q/k/v projection into per-head tiles */
#define MZ_K_ATTN 5  /* encoder self-attention */
#define MZ_K_OPROJ 6 /* out-projection + residual */
#define MZ_K_FC1 7   /* fc1 + GELU */
#define MZ_K_FC2 8   /* fc2 + residual */
#define MZ_K_XKV 9   /* every decoder layer's cross k/v */
#define MZ_K_STEP 10 /* one replay of the captured decoder step */
#define MZ_K_DEC_EMBED 11  /* decoder step kernels (eager steps): token + position embedding + LayerNorm */
#define MZ_K_DEC_QKV 12    /* self-attention q/k/v projection (k, v into the cache) */
#define MZ_K_DEC_SELF 13   /* self-attention over the cache */
#define MZ_K_DEC_OPROJ 14  /* self-attention out-projection (split-K partials) */
#define MZ_K_DEC_ADDLN 15  /* residual add of the partials + LayerNorm */
#define MZ_K_DEC_CROSS 16  /* cross-attention (its query projection and the alignment rows included) */
#define MZ_K_DEC_XO 17     /* cross-attention out-projection */
#define MZ_K_DEC_FC1 18    /* fc1 + GELU */
#define MZ_K_DEC_FC2 19    /* fc2 (split-K partials) */
#define MZ_K_DEC_LM 20     /* tied LM head with the per-workgroup argmax partials */
#define MZ_K_DEC_ARGMAX 21 /* greedy choice */
int mz_engine_profile(mz_engine* e, int on);
int mz_engine_profile_read(mz_engine* e, int kernel, double* total_ms, int* count);

#define MZ_BUF_TOK 0     /* i32 [bmax][max_t] */
#define MZ_BUF_DONE 1    /* i32 [bmax] */
#define MZ_BUF_CTR 2     /* i32 [4]; ctr[0] = position of the next step */
#define MZ_BUF_ALIGN 3   /* f32 [bmax][max_t][n_align][1500] alignment-head probabilities */
#define MZ_BUF_ENC_OUT 4 /* f16 [eg * 1500][d] final-LN encoder output of the last encode */
#define MZ_BUF_LOGITS 5  /* f32 [bmax][vocab] logits of the last step */
#define MZ_BUF_TRACE 6   /* f32 [enc_layers][eg * 1500][d] encoder layer inputs (set_trace) */
#define MZ_BUF_XKV 7     /* f16 [bmax][dec_layers][2][nh] tiles of 1536 x 64 (k, v as [t][64]) */
#define MZ_BUF_DEC_X 8   /* f32 [bmax][d] decoder residual stream */
#define MZ_BUF_ENC_X 9   /* f32 [eg * 1500][d] encoder residual stream */
#define MZ_BUF_DEC_TRACE 10 /* f32 [dec_layers + 1][bmax][d]: with the trace on, the decoder residual entering each
                             * layer and after the last one, of the last eager step (not recorded by graph replays) */
#define MZ_BUF_SELF_K 11 /* f16 [dec_layers][bmax][nh][max_t][64] self-attention key cache */
#define MZ_BUF_SELF_V 12 /* f16 [dec_layers][bmax][nh][max_t][64] self-attention value cache */
#define MZ_BUF_ALIGN_H 13 /* f16 [bmax][max_t][n_align][1500]: MZ_BUF_ALIGN's rows rounded to fp16, written by the
                           * same kernels; the reference's own align buffer (src/model.rs:455), which
                           * src/transcribe.rs:158 reads with download_h */
/* Device address and size of an engine buffer. */
int mz_engine_buffer(mz_engine* e, int which, uint64_t* dptr, size_t* bytes);
/* Synchronise, then copy bytes at byte offset `offset` of an engine buffer to host memory. */
int mz_engine_read(mz_engine* e, int which, void* dst, size_t offset, size_t bytes);
/* Frees the engine's device and host memory; call it before mz_ctx_free of its context. */
int mz_engine_free(mz_engine* e);

/* Wall times of the stages, seconds (Times, src/transcribe.rs:95-101). */
typedef struct {
    double enc, dec, post;
    int steps;
} mz_times;

/* Encode and greedily decode n <= bmax clips of log-mel f32 [n][n_mels][3000] with token timestamps
 * (transcribe, src/transcribe.rs:104-167). frames[i] = 10 ms frames of audio in clip i (3000 for a full window).
 * prompt = [sot, lang, task, notimestamps] (lang ignored when detect != 0). max_new caps the generated tokens
 * (<= 0: up to max_t - prompt_len, as the reference). half_align != 0 rounds the timestamp arithmetic through fp16
 * as the reference does (src/align.rs). Outputs per clip i: seq[i * max_t ..] tokens, seq_len[i], ts[i * max_t ..]
 * start times, langs[i]. The decoding loop tests the done flags every 8 steps, as the reference's (transcribe.rs:
 * 136-141), but reads flags copied two steps earlier so that the device never waits for the host: a batch whose last
 * row finishes in the last two steps before a multiple of 8 runs 8 steps more than the reference's loop, and
 * times->steps is then 8 larger. Tokens, lengths and times are the same (finished rows keep eos). */
int mz_transcribe(mz_engine* e, const float* mels, const int32_t* frames, int n, const int32_t* prompt,
                  int prompt_len, int detect, int use_graph, int max_new, int half_align, int32_t* seq,
                  int32_t* seq_len, float* ts, int32_t* langs, mz_times* times);
/* As mz_transcribe with the log-mel already in device memory (f32 [n][n_mels][3000] at `mels`). */
int mz_transcribe_device(mz_engine* e, uint64_t mels, const int32_t* frames, int n, const int32_t* prompt,
                         int prompt_len, int detect, int use_graph, int max_new, int half_align, int32_t* seq,
                         int32_t* seq_len, float* ts, int32_t* langs, mz_times* times);
/* mz_transcribe in two halves (transcribe, src/transcribe.rs:107-116 and 118-167): submit enqueues the encoder of a
 * chunk of n <= bmax clips and returns at once, so the caller's host work (reading and resampling the next files)
 * overlaps it; collect decodes that chunk and returns exactly what mz_transcribe returns (same arguments and outputs;
 * n must be the submitted count). One chunk at a time: submit refuses while a chunk is pending, and so does
 * mz_transcribe. A host log-mel is copied before submit returns; a device log-mel must stay unchanged until collect.
 * times->enc = the host's time in submit plus its wait in collect for the encoder. */
int mz_transcribe_submit(mz_engine* e, const float* mels, int n);
int mz_transcribe_submit_device(mz_engine* e, uint64_t mels, int n);
int mz_transcribe_collect(mz_engine* e, const int32_t* frames, int n, const int32_t* prompt, int prompt_len,
                          int detect, int use_graph, int max_new, int half_align, int32_t* seq, int32_t* seq_len,
                          float* ts, int32_t* langs, mz_times* times);

/* Token start times of n clips on the device, the same bits as mz_jump_times on each clip (jump_times,
 * src/align.rs:8-63; the reference runs it on the host after downloading the weights, transcribe.rs:150-158).
 * Clip c's alignment-head weights are rows[c] rows of heads x cols_full floats at device address
 * w + c * clip_stride * 4, cropped to cols[c] frames; its times go to host out[c * out_stride + k], k < rows[c].
 * Odd width <= 15. Allocates and frees its own device scratch; synchronous on the context's stream. */
int mz_jump_times_device(mz_ctx* c, uint64_t w, int64_t clip_stride, int n, const int32_t* rows, const int32_t* cols,
                         int heads, int cols_full, int width, int half, float* out, int64_t out_stride);

/* mz_jump_times_device without any device allocation: no counterpart in the reference; for callers that cannot
 * allocate device memory (code under graph capture, tight serving loops, harnesses that forbid hipMalloc). Same
 * arguments and results as mz_jump_times_device (bit for bit). Its scratch is a static 64 MiB array per device
 * (held until the process ends), located by mz_init; the clips go through it in passes of at most 64 that fit, and a
 * clip whose own scratch exceeds 64 MiB is refused with MZ_ERR_ARG (e.g. more than about 1,200 rows at 1500 frames).
 * Every call on a device shares that device's array (one copy per process and GPU), so the library serialises them:
 * a call holds a per-device lock from its first use of the array until its results are on the host, and calls from
 * other threads or contexts on the same GPU wait for it. Synchronous on the context's stream. */
int mz_jump_times_device_noalloc(mz_ctx* c, uint64_t w, int64_t clip_stride, int n, const int32_t* rows,
                                 const int32_t* cols, int heads, int cols_full, int width, int half, float* out,
                                 int64_t out_stride);

/* ------------------------------------------------------------------ model directory (host only) */

/* Safetensors file (st::File, src/st.rs:77-181): mapped read-only (read into memory if mapping fails), header
 * checked as st.rs:93-142 does (header length, an object header, known dtypes, integer shapes, two data offsets
 * in order and inside the data, size = elements x element size, no duplicate names, no overlapping ranges).
 * Tensors keep the header's order; data pointers stay valid until mz_st_close. */
typedef struct mz_st mz_st;
int mz_st_open(const char* path, mz_st** out);
int mz_st_count(const mz_st* f, int* n);
/* Tensor i: name, dtype ("F16", "F32", ...), rank, shape, data and byte count (any output may be null). */
int mz_st_info(const mz_st* f, int i, const char** name, const char** dtype, int* ndim, const int64_t** shape,
               const void** data, uint64_t* bytes);
/* Index of a tensor by name (File::get's lookup, st.rs:144-147); MZ_ERR_ARG "missing tensor" if absent. */
int mz_st_find(const mz_st* f, const char* name, int* i);
/* A __metadata__ string entry (File::meta). */
int mz_st_meta(const mz_st* f, const char* key, const char** value);
int mz_st_close(mz_st* f);
/* MZ_OK if s[0 .. n) is one JSON value under the strict grammar of src/json.rs:1-218, else MZ_ERR_ARG with the
 * parser's message (the same parser reads the safetensors header and the configs). */
int mz_json_check(const char* s, size_t n);

/* A model directory's configs: Dims::load (src/model.rs:33-61) on config.json and GenCfg::load (:78-146) on
 * generation_config.json, with the same range checks and defaults (alignment heads: every head of the second half
 * of the decoder layers). The arrays mz_model_gencfg points to live until mz_model_free. */
typedef struct mz_model mz_model;
int mz_model_open(const char* model_dir, mz_model** out);
int mz_model_dims(const mz_model* m, mz_dims* d);
int mz_model_gencfg(const mz_model* m, mz_gencfg* g);
/* Language i (code with "<|" "|>" stripped, token) of lang_to_id, and task i (name, token) of task_to_id, in file
 * order (GenCfg::langs / tasks). */
int mz_model_lang(const mz_model* m, int i, const char** code, int32_t* token);
int mz_model_task(const mz_model* m, int i, const char** name, int32_t* token);
int mz_model_free(mz_model* m);

/* ------------------------------------------------------------------ audio front end (src/audio.rs) */

/* read_wav (src/audio.rs:14-75): mono samples of a RIFF/WAVE file (16/24/32-bit PCM or 32-bit float, channels
 * averaged; a data size of 0xFFFFFFFF runs to the end of the file) and its sample rate. *n and *sr are always set;
 * the samples are written only when y is non-null and cap >= *n (call once with y = NULL to size the buffer). */
int mz_wav_read(const char* path, float* y, size_t cap, size_t* n, int* sr);
/* to_16k (src/audio.rs:77-145): Kaiser-windowed sinc resampling to 16 kHz in double, rates 1 kHz .. 768 kHz;
 * *n_out always set, out written when non-null and cap >= *n_out. */
int mz_resample_16k(const float* y, size_t n, int sr, float* out, size_t cap, size_t* n_out);
/* Mel::new's tables (src/audio.rs:161-189): Slaney filters f32 [201][n_mels] up to 8 kHz, and the
 * periodic-Hann-windowed DFT basis cos / sin f64 [400][201] (sample-major); any output may be null. */
int mz_mel_tables(int n_mels, float* filters, double* cosb, double* sinb);
/* Mel::features (src/audio.rs:195-249) of n clips on the device: audio f32 [n][480000] at device address `audio`
 * (16 kHz; samples at or past n_samples[i] read as zero) -> normalised log-mel f32 [n][n_mels][3000] at `mel`;
 * frames[i] (may be null) = 10 ms frames that hold audio. The power spectra equal the reference's bit for bit
 * (double sums in sample order); log10 is the device library's. Synchronous; allocates and frees its scratch. */
int mz_log_mel(mz_ctx* c, uint64_t audio, const int32_t* n_samples, int n, int n_mels, uint64_t mel, int32_t* frames);

/* ------------------------------------------------------------------ text (src/tok.rs, src/main.rs) */

/* Decoding side of the byte-level BPE tokenizer (Tok, src/tok.rs): <model_dir>/vocab.json through the GPT-2
 * byte table; ids must be below vocab and every id below eos needs an entry (Tok::load, :25-45). */
typedef struct mz_tok mz_tok;
int mz_tok_open(const char* model_dir, int vocab, int eos, mz_tok** out);
/* A tokenizer over raw byte strings entries[i] of lens[i] bytes (id i), for callers with their own vocabulary. */
int mz_tok_from_bytes(const char* const* entries, const size_t* lens, int n, mz_tok** out);
int mz_tok_free(mz_tok* t);
/* Tok::decode (:47-57): the ids' bytes (unknown ids dropped) as UTF-8 with invalid sequences replaced by U+FFFD,
 * then the clean-up of spaces before punctuation and contractions. Text out NUL-terminated when cap > *len. */
int mz_tok_decode(const mz_tok* t, const int32_t* ids, int n, char* out, size_t cap, size_t* len);
/* Tok::pieces (:63-86): whole UTF-8 pieces of the tokens below eos with start / end times; the pieces' text is
 * concatenated into text (NUL-terminated when cap > *len), piece k spanning offsets[k] .. offsets[k + 1]
 * (offsets holds n + 1 entries, t0 / t1 n), *n_pieces set; any of text / offsets / t0 / t1 may be null. */
int mz_tok_pieces(const mz_tok* t, const int32_t* ids, const float* ts, int n, int eos, char* text, size_t cap,
                  size_t* len, int32_t* offsets, float* t0, float* t1, int* n_pieces);
/* A time as the CLI's JSON prints it: Python's round(x, 2) as json.dumps writes a float (json_t, main.rs:113-117). */
int mz_json_time(float x, char* out, size_t cap, size_t* len);
/* to_json (src/main.rs:121-138): {path: {"language", "text", "words": [[piece, start, end], ...]}, ...} plus a
 * newline for n clips; clip i's tokens seq[i * stride ..] (seq_len[i] of them, prompt included), times ts likewise,
 * detected language token langs[i] ("en" for an English-only model). Out NUL-terminated when cap > *len. */
int mz_results_json(const mz_tok* t, const mz_model* m, int n, const char* const* paths, const int32_t* seq,
                    const int32_t* seq_len, int stride, const float* ts, const int32_t* langs, char* out, size_t cap,
                    size_t* len);

/* ------------------------------------------------------------------ command line (src/main.rs) */

/* The mimizuku command line (main.rs:17-224): argv[0] is the program name; --model DIR, input WAV files or --dir /
 * --prefix, --language, --task, --out, --batch, --enc-group, --quiet, --no-graph, --help. Prints the JSON to
 * stdout (or --out) and the reference's progress and timing lines to stderr; returns the process exit status
 * (errors print "error: ..." and return 1). Uses device 0 with its own context. */
int mz_cli(int argc, const char* const* argv);

/* ------------------------------------------------------------------ host helpers */

/* Token start times from alignment-head weights w [rows][heads][cols_full] (f32), cropped to cols frames
 * (jump_times, src/align.rs:8-63); out[rows]. */
int mz_jump_times(const float* w, int rows, int heads, int cols_full, int cols, int width, int half, float* out);
/* The cost jump_times hands to the DTW (src/align.rs:14-52): m[i][j] = minus the head average of the width-`width`
 * median-filtered per-column z-scores of w [rows][heads][cols_full] cropped to cols columns (rows, cols >= 1).
 * half != 0 is align.rs's arithmetic: column sums in float in row order, fp16 roundings of the mean, deviation,
 * z-scores and average; half == 0 takes the column sums in double and rounds nothing. */
int mz_align_cost(const float* w, int rows, int heads, int cols_full, int cols, int width, int half, double* m);
/* Dynamic time warping on cost m [rows][cols] (dtw, src/align.rs:66-106); path written to text/time (capacity
 * rows + cols), its length to *len. */
int mz_dtw(const double* m, int rows, int cols, int32_t* text, int32_t* time, int32_t* len);
/* IEEE binary16 conversions, round to nearest even (h2f / f2h, src/gpu.rs:79-114). */
uint16_t mz_f2h(float x);
float mz_h2f(uint16_t h);

#ifdef __cplusplus
}
#endif
#endif /* MIMIZUKU_H */
