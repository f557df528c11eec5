/* seoul_hip.h — C ABI of libseoul_hip.so, the MI355X (gfx950) implementation of imi's brain step.
 *
 * This is the boundary a host engine binds to: plain pointers and sizes, int status codes, no exceptions, no torch
 * or HIP types. Host buffers passed in are borrowed for the call; outputs are written into caller buffers before the
 * call returns. A context owns one model on one device and one HIP stream; calls on one context are not
 * thread-safe. A state (one conversation's memory) or table is valid only with the context that made it.
 * Destroying a context releases the device memory of its remaining states and tables; their handles must still be
 * released with sh_state_free / sh_q4_free, which then only free the handle.
 *
 * Reference interfaces replaced (paths relative to the reference repository):
 *   imi_seoul / imi_brain engine    imi/core/seoul.h:28-94, imi/brain.h:20-65
 *   imi_seoul_state                 imi/core/seoul.h:21-26
 *   imi_file (GGUF read + repack)   imi/model.h:12-36, imi/core/tables.cpp:67-97
 *   imi_q4x8 kernel API (cfg 0)     imi/kernels/q4x8.h:8-18
 *   imi_q4 table reads              imi/core/tables.h:103-138
 *   imi_voice generator             imi/core/voice.h:17-51
 *   imi_codec decoder               imi/core/codec.h:17-65
 *   imi_ears audio encoder          imi/core/ears.h:17-51, imi_wg tables imi/core/tables.h:84-95
 */
#ifndef SEOUL_HIP_H
#define SEOUL_HIP_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* status codes */
#define SH_OK 0
#define SH_E_ARG (-1)           /* bad argument (null pointer, out-of-range id, wrong size) */
#define SH_E_HIP (-2)           /* a HIP runtime call failed; sh_last_error() names it */
#define SH_E_FILE (-3)          /* model file unreadable or malformed (imi: load() returns false) */
#define SH_E_SHAPE (-4)         /* a table or shape the kernels do not take (imi/core/seoul.cpp:162) */
#define SH_E_CONTEXT_FULL (-5)  /* position would pass n_ctx; nothing was stepped (imi/core/seoul.cpp:209,353,498) */
#define SH_E_STATE (-6)         /* state belongs to another context, or no model loaded */
#define SH_E_NOMEM (-7)         /* device or host allocation failed */

typedef struct sh_ctx sh_ctx;       /* one model on one device */
typedef struct sh_state sh_state;   /* one conversation's memory: K/V caches, conv memory, position */
typedef struct sh_q4 sh_q4;         /* one Q4_0 table on the device (kernel-level API) */
typedef struct sh_voice sh_voice;   /* the Q8_0 voice generator on the device */
typedef struct sh_file sh_file;     /* one GGUF file read into host memory (imi_file) */
typedef struct sh_codec sh_codec;   /* the codec decoder on the device (codes -> 24 kHz samples) */
typedef struct sh_ears sh_ears;     /* the ears (audio encoder) on the device (16 kHz samples -> prefill rows) */

typedef struct {
    int n_embd, n_vocab, n_head, n_head_kv, head_dim, n_ff, d_conv, n_ctx, n_layer, n_attn, n_swa;
    long long table_bytes;          /* bytes of all layer tables + word table in the device layout */
    long long vector_bytes;         /* bytes a step reads besides the tables and K/V: fp32 norm weights and conv
                                       taps, plus the conv memory read and written */
} sh_model_info;

/* Message of the last error on this thread ("" if none). */
const char* sh_last_error(void);

/* ---- codec decoder: imi_codec::load / reset / frame / flush (imi/core/codec.h:17-65) ---- */
typedef struct {
    int n_embd, n_ff, n_head, n_head_kv, head_dim, d_conv, n_layer, n_bins, n_lvl, n_q, n_codes;
    long long table_bytes;          /* Q8_0 table bytes read per frame */
} sh_codec_shape;

/* Read a GGUF codec ("a.gen.wav." tensors: FSQ level table, quantizer projection, Q8_0 in_proj / out_proj and LFM
 * layers of short conv or gated attention) onto `device` (imi/core/codec.cpp:41-108). n_embd up to 512, head_dim up
 * to 128, 2 to 8 conv taps, 641 bins (n_fft 1280, hop 320). Own stream; independent of any brain context. */
int sh_codec_load(int device, const char* gguf_path, sh_codec** out);
int sh_codec_free(sh_codec* c);                                   /* imi_codec::~imi_codec (codec.cpp:279-282) */
int sh_codec_info(const sh_codec* c, sh_codec_shape* out);
/* codec.cpp:110-119: conv memory, attention window and overlap cleared, position 0, start padding re-armed */
int sh_codec_reset(sh_codec* c);
/* One frame of 12 codes (each in [0, n_codes)) -> its samples (codec.cpp:121-127): pcm needs room for 1920;
 * *n_out = 1920, less the start padding on the first frames after a reset (1440 on the first). */
int sh_codec_frame(sh_codec* c, const int32_t* codes, float* pcm, int* n_out);
/* The end of speech (codec.cpp:271-277): the tail the overlap holds back, 480 samples; then a reset. */
int sh_codec_flush(sh_codec* c, float* pcm, int* n_out);

/* ---- ears (audio encoder): imi_ears::load / encode (imi/core/ears.h:17-51) ---- */
typedef struct {
    int n_mel, n_ch, n_embd, n_ff, n_head, n_head_kv, head_dim, window, n_out, d_conv, n_layer;
    int n_attn;                     /* attention layers (the others are short-conv layers) */
    int n_mid;                      /* projector width (mm.a.mlp.1 rows) */
    long long table_bytes;          /* float table bytes (F16 / F32 as in the file, plus the 402 x 400 DFT) */
} sh_ears_shape;

/* Read a GGUF ears file ("a.conv1d.*" F32 downsampler, "a.pre_encode.out", "a.blk.N.*" layers of short conv or
 * windowed attention on F16 / F32 tables, "a.post_ln", "mm.a.mlp.*" projector; keys clip.audio.num_mel_bins,
 * window_size, attention.head_count, attention.layer_norm_epsilon) onto `device` (imi/core/ears.cpp:40-138).
 * n_mel a multiple of 8, n_embd a multiple of 32 up to 4096, head_dim a multiple of 32 up to 128, window 1 to 64. */
int sh_ears_load(int device, const char* gguf_path, sh_ears** out);
int sh_ears_free(sh_ears* e);
int sh_ears_info(const sh_ears* e, sh_ears_shape* out);
/* Positions and mel frames a clip of n_samples gives (ears.cpp:203-205); either pointer may be null. */
int sh_ears_positions(const sh_ears* e, int n_samples, int* n_pos, int* n_frames);
/* imi_ears::encode (ears.cpp:198-407): 16 kHz samples from the clip's start -> out [n_pos][n_out] (host memory,
 * room for sh_ears_positions' count). Blocking. */
int sh_ears_encode(sh_ears* e, const float* pcm, int n_samples, float* out, int* n_pos);
/* The last encode's mel frames [n_frames][n_mel] (imi_ears::last_mel), into host memory that holds cap_frames
 * frames: SH_E_ARG (nothing written) when the last encode has more. mel may be null to ask for *n_frames only. */
int sh_ears_mel(const sh_ears* e, float* mel, int cap_frames, int* n_frames);

/* ---- GGUF file: imi_file::load / get / key_i / key_f / keep / drop_data (imi/model.h:12-36) ---- */
/* The ggml_tensor fields imi's callers read. name points into the file object; data is the tensor's bytes in host
 * memory: in the file's block, or in a copy of its own after sh_file_keep, or null once sh_file_drop_data let the
 * block go and the tensor was not kept (its shape stays readable). */
typedef struct {
    const char* name;
    int type;          /* ggml type id: 0 F32, 1 F16, 2 Q4_0, 3 Q4_1, 8 Q8_0, 14 Q6_K */
    int n_dims;
    int64_t ne[4];     /* ne[0] innermost; unused dimensions are 1 */
    size_t nb[4];      /* ggml byte strides: nb[0] one element or block, nb[1] one row, ... */
    void* data;
} sh_tensor;

/* imi_file::load (imi/model.cpp:48-106): header, keys and tensor table read, every tensor's bytes mapped. The
 * repack argument of imi (a CPU kernel layout) has no counterpart: the engine makes the device layout itself. */
int sh_file_load(const char* path, sh_file** out);
int sh_file_free(sh_file* f);
/* imi_file::get (model.cpp:108-115): SH_E_ARG when the file has no such tensor (imi stops when it is required) */
int sh_file_get(const sh_file* f, const char* name, sh_tensor* out);
/* imi_file::key_i (model.cpp:117-126): a u32, i32 or u64 key's value, else def */
int64_t sh_file_key_i(const sh_file* f, const char* key, int64_t def);
/* imi_file::key_f (model.cpp:128-131): an f32 key's value, else def */
float sh_file_key_f(const sh_file* f, const char* key, float def);
/* imi_file::keep (model.cpp:138-150): the tensor gets a 64-byte aligned copy of its bytes of its own */
int sh_file_keep(sh_file* f, const char* name, sh_tensor* out);
/* imi_file::drop_data (model.cpp:152-163): the file's block is let go; tensors not kept get data = null */
int sh_file_drop_data(sh_file* f);
/* the tensors in file order (imi walks them with ggml_get_first_tensor / ggml_get_next_tensor) */
int sh_file_n_tensors(const sh_file* f);
int sh_file_tensor(const sh_file* f, int i, sh_tensor* out);
/* a key holding an array of integers or bools (imi reads these from the file's gguf context, e.g. the sliding-window
 * pattern, imi/brain.cpp:32-36): its length (0 when absent or not an array); the first cap values go to out */
int sh_file_key_arr(const sh_file* f, const char* key, int64_t* out, int cap);
/* imi_file::data / size: every tensor's bytes as one block (null and 0 after drop_data) */
int sh_file_block(const sh_file* f, const void** data, size_t* size);

/* ---- engine: imi_seoul::load / reset / step / step2 / step_batch / new_state / swap_state ---- */
int sh_create(int device, sh_ctx** out);
int sh_destroy(sh_ctx* ctx);
/* Read a GGUF brain file, repack every Q4_0 table into the device layout and upload it; n_ctx = context length of
 * states made afterwards (imi/core/seoul.cpp:93-186). */
int sh_load(sh_ctx* ctx, const char* gguf_path, int n_ctx);
int sh_info(const sh_ctx* ctx, sh_model_info* out);
/* Check a GGUF brain file on the host, without a device: its keys, and every table's type, rows and columns against
 * what the kernels take (the same kv head count and FFN width in every layer), and that the attention kernels hold
 * n_ctx positions at its head shape. sh_load runs the same check before it uploads anything (imi's load reads the
 * same keys and tensors, imi/core/seoul.cpp:93-162, and returns false on a file it cannot use). out (nullable) gets
 * the shape; table_bytes and vector_bytes are left 0. Returns SH_OK, SH_E_FILE or SH_E_SHAPE. */
int sh_check_model(const char* gguf_path, int n_ctx, sh_model_info* out);

int sh_state_new(sh_ctx* ctx, sh_state** out);          /* imi_seoul::new_state (seoul.cpp:193-201) */
int sh_state_free(sh_state* st);
int sh_state_reset(sh_state* st);                        /* imi_seoul::reset (seoul.cpp:188-191): pos 0, conv zeroed */
int sh_state_pos(const sh_state* st, int* pos);
int sh_state_set_pos(sh_state* st, int pos);             /* rewind (imi/core/hear_pieces.cpp:8-11) */

/* One position (imi_seoul::step, seoul.cpp:352-357): token >= 0 reads that word's row, else embd[n_embd].
 * hidden[n_embd] (nullable) gets the hidden state; if want_logits, logits[n_vocab] (nullable) gets the word scores
 * and best (nullable) the first index of their maximum. */
int sh_step(sh_ctx* ctx, sh_state* st, int32_t token, const float* embd, int want_logits,
            float* hidden, float* logits, int32_t* best);

/* Two conversations, one read of every table (imi_seoul::step2, seoul.cpp:208-220). Each conversation gets the
 * numbers its own sh_step would give. */
int sh_step2(sh_ctx* ctx, sh_state* a, int32_t token_a, const float* embd_a, int logits_a,
             sh_state* b, int32_t token_b, const float* embd_b, int logits_b,
             float* hidden_a, float* logits_a_out, int32_t* best_a,
             float* hidden_b, float* logits_b_out, int32_t* best_b);

/* n positions at once (imi_seoul::step_batch, seoul.cpp:490-517): tokens[n] or embd[n][n_embd]. hidden_last
 * gets the last position's hidden state, hidden_all[n][n_embd] (nullable) every position's; logits/best are the
 * last position's. For n >= 2 the positions go through each table together on the int8 matrix cores (the
 * prefill); every number equals n single steps. The whole batch must fit the context, else nothing is stepped. */
int sh_step_batch(sh_ctx* ctx, sh_state* st, const int32_t* tokens, const float* embd, int n, int want_logits,
                  float* hidden_last, float* logits, float* hidden_all, int32_t* best);

/* Greedy decode on the device: n_steps steps, each feeding back the argmax of its word scores, for one (b null)
 * or two conversations (step2). out_a/out_b[n_steps] get the chosen ids; seconds (nullable) the device time.
 * Equivalent to the greedy loops of imi/core/hear.cpp:66-72 with no host round trip per token. */
int sh_generate(sh_ctx* ctx, sh_state* a, sh_state* b, int32_t first_a, int32_t first_b, int n_steps,
                int32_t* out_a, int32_t* out_b, double* seconds);

/* Every layer table read back to back with ncol (1 or 2) inputs riding each read, reps passes
 * (imi_seoul::bench_tables, seoul.cpp:657-685). ms_per_pass = best pass; avg_launch_us = mean GEMV launch
 * duration over all passes; bytes_per_pass = table bytes read per pass. */
int sh_bench_tables(sh_ctx* ctx, int ncol, int reps, double* ms_per_pass, double* avg_launch_us,
                    double* bytes_per_pass, int* launches_per_pass);

/* The step's own GEMV kernel for one table kind (0: FFN gate|up with norm prologue and SwiGLU epilogue, 1: FFN
 * down, 2: word scores), launched reps times with real layer arguments rotating over the layers; avg_us = mean
 * kernel duration (events recorded around each kernel), bytes_per_launch = table + input + output bytes. */
int sh_bench_kernel(sh_ctx* ctx, int kind, int n_in, int reps, double* avg_us, double* bytes_per_launch);

/* The same kernels timed inside whole steps: two untimed, then `steps` timed steps (n_in conversations on fresh
 * states, seeded token ids) enqueued without the graph, each launch of table kind `kind` (2: Q4_0 word table only)
 * recording the events of its own dispatch; its input is what the step's previous kernel has just written, its
 * table is read from HBM. avg_us = mean over the `launches` timed launches. */
int sh_bench_step_kernel(sh_ctx* ctx, int kind, int n_in, int steps, double* avg_us, double* bytes_per_launch,
                         int* launches);

/* ---- kernel-level Q4_0 tables (imi/kernels/q4x8.h:14-18, imi/core/tables.h:103-138) ---- */
/* q4_0: rows * cols/32 Q4_0 blocks (fp16 scale + 16 nibble bytes) as stored in GGUF; rows % 8 == 0. */
int sh_q4_create(sh_ctx* ctx, const void* q4_0, int rows, int cols, sh_q4** out);
int sh_q4_free(sh_q4* t);
/* y[n_in][rows] = W x[n_in][cols] for n_in in {1, 2}; the input is cut to int8 per 32 columns with round half to
 * even (cut_mode 0, imi/core/vec.h:47-75) or half away from zero (cut_mode 1, imi/kernels/q4x8.cpp:38-48). */
int sh_q4_gemv(sh_ctx* ctx, const sh_q4* t, const float* x, int n_in, float* y, int cut_mode);
/* y[n][rows] = W x[n][cols] for 1 <= n <= 512 inputs through the prefill's int8 matrix-core product: each input cut
 * to int8 per 32 columns (round half to even), each 32-column block's integer sum exact, then imi's per-row chains
 * over the blocks (imi_q4_group_batch, imi/core/tables.cpp:419-454); bit for bit sh_q4_gemv per input. */
int sh_q4_gemm(sh_ctx* ctx, const sh_q4* t, const float* x, int n, float* y);
/* sh_q4_gemm on device-resident buffers with no device allocation: x_dev[n][cols] in, y_dev[n][rows] out, the same
 * numbers bit for bit. No counterpart in the reference; it is for callers that cannot allocate (code under HIP
 * graph capture, serving loops with a fixed memory budget). The int8 cut of the input goes to a fixed scratch array
 * of device memory the library holds on every device it runs on until the process ends (1.25 MiB per device), so
 * n * cols <= 1048576 (else SH_E_ARG, nothing launched) and 1 <= n <= 512. Calls on one device share that scratch:
 * calls of one context are ordered by its stream, and a call from a context other than the device's last user waits on
 * its own stream for an event recorded after that call (an event made at sh_create, no device memory). Under graph
 * capture of the context's stream no event is used: captured calls of two contexts replaying at once on one device
 * race. Enqueued on the context's stream without waiting (sh_sync waits). */
int sh_q4_gemm_noalloc(sh_ctx* ctx, const sh_q4* t, const float* x_dev, int n, float* y_dev);
/* Dequantized rows: out[n][cols] = (code - 8) * d of rows ids[n] (the input-row lookup of a tied word table,
 * imi/core/seoul.cpp:363, ggml_get_rows in imi/brain.cpp:161). Bit-exact. */
int sh_q4_rows(sh_ctx* ctx, const sh_q4* t, const int32_t* ids, int n, float* out);
/* Same on device-resident buffers (no copies, no synchronisation): x_dev, y_dev are device pointers. */
int sh_q4_gemv_dev(sh_ctx* ctx, const sh_q4* t, const float* x_dev, int n_in, float* y_dev, int cut_mode);
/* Several tables at once (a layer's linears, each with its own input): y[i][n_in][rows_i] = tables[i] x[i][n_in][cols_i]
 * for i < n, each output bit for bit sh_q4_gemv's for that table (the same kernel body and operands). Widths
 * 2048, 4096 or 8192 columns; up to 8 tables per launch (one width per launch for two inputs), so a layer's seven
 * linears cost one dispatch (two at n_in = 2) instead of seven. The reference runs the same
 * products table by table (imi_q4_group / imi_q4_group2, imi/core/tables.h:103-138); this entry point has no single
 * counterpart there. Host buffers; the call waits. */
int sh_q4_gemv_group(sh_ctx* ctx, int n, sh_q4* const* tables, const float* const* x, float* const* y, int n_in,
                     int cut_mode);
/* Same on device-resident buffers, enqueued on the context's stream without waiting. */
int sh_q4_gemv_group_dev(sh_ctx* ctx, int n, sh_q4* const* tables, const float* const* x_dev, float* const* y_dev,
                         int n_in, int cut_mode);
/* Time `reps` grouped calls over n_sets sets of n tables (tables[s * n + i]: table i of set s), the sets in
 * rotation so that none is resident in the 256 MB MALL when they are larger; inputs resident, zeros.
 * avg_us = mean time per call (all of a set's launches, back to back). */
int sh_q4_group_bench(sh_ctx* ctx, int n_sets, int n, sh_q4* const* tables, int n_in, int cut_mode, int reps,
                      double* avg_us);
/* Time `reps` launches of the GEMV over `n_tables` tables in turn (tables[i] read in rotation so that none is
 * resident in the 256 MB MALL when the set is larger), inputs resident; avg_launch_us = mean launch duration. */
int sh_q4_bench(sh_ctx* ctx, sh_q4* const* tables, int n_tables, int n_in, int cut_mode, int reps, double* avg_launch_us);
/* The kernel's own duration: each launch timed alone by events recorded around the kernel (no dispatch gap in
 * front of it), averaged over `reps`; after sh_q4_bench on the same tables (which sizes the device input/output). */
int sh_q4_bench_kernel(sh_ctx* ctx, sh_q4* const* tables, int n_tables, int n_in, int cut_mode, int reps, double* avg_kernel_us);
/* The same launches back to back replayed from a captured HIP graph: one pass over the tables (one launch each, in
 * order) captured once and replayed `passes` times; avg_launch_us = the replays' event time over passes * n_tables.
 * After sh_q4_bench on the same tables. */
int sh_q4_bench_graph(sh_ctx* ctx, sh_q4* const* tables, int n_tables, int n_in, int cut_mode, int passes, double* avg_launch_us);

/* Calibration: an empty kernel of `grid` x 256 threads launched `reps` times back to back on one stream (the
 * dispatch cost any kernel pays), and a pure read of `bytes` (copies distinct buffers in rotation, so with
 * copies * bytes above the 256 MB last-level cache every launch reads HBM; 2 x 16-byte loads in flight per thread,
 * grid x 256 threads): microseconds per launch. stamps (nullable, 3 doubles) gets one more launch's timeline from the
 * device clock: the last workgroup's start, the median workgroup's first loads back, the last workgroup's end, each in
 * microseconds after the first workgroup started. No counterpart in the reference; they bound what a kernel reading
 * the same bytes can reach. */
int sh_bench_empty(int device, int grid, int reps, double* us_per_launch);
int sh_bench_read(int device, long long bytes, int copies, int grid, int reps, double* us_per_launch, double* stamps);
/* Calibration: `launches` launches of `grid` workgroups back to back on one stream; xcc[l * grid + b] = the XCD
 * (hardware register XCC_ID) workgroup b of launch l ran on. Calibration: whether a launch finds in the L2 what the
 * launch before it read: `pairs` times, launch A and then launch B read the same 72 KB slot per workgroup (256
 * workgroups, 18.9 MB, cached loads; *same_xcd counts workgroups of B on the XCD of A's workgroup with the same index,
 * summed over pairs), and B alone reads slots no launch has read. us_second / us_alone: B's event time, averaged.
 * Under rocprofv3's TCC_HIT / TCC_MISS counters B misses every line either way. No counterpart in the reference. */
int sh_bench_xcc(int device, int grid, int launches, int* xcc);
int sh_bench_l2_reuse(int device, int pairs, double* us_second, double* us_alone, int* same_xcd);

/* y[i] = e^x[i] with the exponential the kernels use (softmax, SiLU, head gates): bit for bit the C library's expf
 * that imi runs on (imi/core/seoul.cpp:48,447,451). */
int sh_expf(sh_ctx* ctx, const float* x, long long n, float* y);

/* ---- voice generator: imi_voice::load / begin_frame / pass / feedback (imi/core/voice.h:17-51) ---- */
typedef struct {
    int n_embd, n_vocab, n_cb, n_in, n_head, n_head_kv, head_dim, n_ff, n_layer;
    long long table_bytes;          /* bytes of every 8-bit table in the device layout (layers, score tables,
                                       input projection) */
    long long feedback_bytes;       /* bytes of the feedback rows (Q8_0 as stored) */
} sh_voice_shape;

/* Read a GGUF voice generator ("a.gen.code." tensors, Q8_0 tables) onto `device` (imi/core/voice.cpp:27-88). The
 * generator has its own stream; it takes 2 to 12 codebooks and head_dim 32 or 64. */
int sh_voice_load(int device, const char* gguf_path, sh_voice** out);
int sh_voice_free(sh_voice* v);                                   /* imi_voice::~imi_voice (voice.cpp:208-212) */
int sh_voice_info(const sh_voice* v, sh_voice_shape* out);
/* The frame's input projection from the brain's hidden state hidden[n_in] (voice.cpp:99-111). */
int sh_voice_begin_frame(sh_voice* v, const float* hidden);
/* The frame's projected input, [n_cb][n_embd] (imi_voice::base, voice.h:30). */
int sh_voice_base(sh_voice* v, float* out);
/* One masked pass (voice.cpp:113-206): codes[n_cb], < 0 = still masked; out[n_need][n_vocab] gets the scores of
 * codebooks need[0..n_need) (0 <= n_need <= n_cb). out may be NULL: the scores then stay on the device for
 * sh_voice_sample and the call returns without waiting for the pass (its errors show at the next call that waits). */
int sh_voice_pass(sh_voice* v, const int32_t* codes, const int32_t* need, int n_need, float* out);
/* The brain's next input after a frame: the sum, codebook by codebook, of the chosen codes' feedback rows,
 * out[n_in] (voice.cpp:90-97). codes[n_cb] must all be chosen (0 <= code < n_vocab). */
int sh_voice_feedback(sh_voice* v, const int32_t* codes, float* out);
/* Temperature sampling with a repeat penalty of the codebooks the last sh_voice_pass scored, on the device
 * (imi_talker::next, imi/core/talk.cpp:147-164). For score row j (codebook need[j] of that pass): every distinct
 * code c the codebook took in hist (n_frames rows of n_cb codes, oldest first, as imi's last min(frames, rep_win)
 * frames; codes outside [0, n_vocab) are skipped) is penalised once, l = l > 0 ? l / rep : l * rep; then
 * p[v] = exp((double)(l[v] - max l) / temp), sum = the sum of p in code order, keep[j] = 1 - p[n_vocab - 1] / sum
 * (the chance that this pick is not end-of-audio), and picks[j] = the first v at which r = u[j] * sum minus
 * p[0], p[1], ... p[v] in double reaches <= 0 (n_vocab - 1 if none). u[j] in [0, 1) is the caller's uniform draw
 * for pick j (imi draws std::uniform_real_distribution<double>(0, 1) from its std::mt19937, pick by pick, after
 * the frame's shuffle). The penalised scores stay in the device score rows, so a pass is sampled once: a second
 * call before the next sh_voice_pass fails with SH_E_ARG. 0 <= n_frames <= 256,
 * n_vocab <= 4096, temp > 0, rep > 0. */
int sh_voice_sample(sh_voice* v, const int32_t* hist, int n_frames, const double* u, float temp, float rep,
                    int32_t* picks, double* keep);

/* Synchronise the context's stream (for callers of the _dev entry points). */
int sh_sync(sh_ctx* ctx);

#ifdef __cplusplus
}
#endif
#endif
