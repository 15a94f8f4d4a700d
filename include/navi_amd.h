/*
 * navi_amd.h - the C ABI between navi-tts's C++ host (Device, DeviceWeights,
 * KvCache/Talker, Frame, Vocoder) and this library's gfx950 kernels.
 *
 * The reference has no FFI: its boundary is the pimpl `Impl` behind each C++
 * class, which calls HIP directly. Each entry point below replaces one of those
 * Impl operations (cited per function); the C++ classes in
 * navi-tts_amd/csrc/host keep the reference's public signatures and call these.
 *
 * Conventions
 *  - Plain C types only: opaque handles, pointers and sizes. Device buffers are
 *    `void *` / typed device pointers that the caller owns unless stated.
 *  - Every call returns a navi_status; no C++ exception crosses the ABI.
 *    Functions taking (char *err, size_t errlen) write a NUL-terminated
 *    message on failure (errlen may be 0).
 *  - One host thread drives one handle at a time; all work is ordered on the
 *    library's stream for the current device (runtime/device/device.cpp:96-97),
 *    and every call that returns results to the host is synchronous on return.
 */
#ifndef NAVI_AMD_H
#define NAVI_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define NAVI_AMD_ABI_VERSION 1

typedef enum {
    NAVI_OK = 0,
    NAVI_ERR_TIMEOUT = 1,        /* a dataflow wait hit its spin cap (frame.hip:673 "timed out") */
    NAVI_ERR_LAUNCH = 2,         /* frame launch refused (the reference's cooperative launch, frame.hip:664) */
    NAVI_ERR_KV_FULL = 3,        /* n_past >= max_pos (frame.hip:800) */
    NAVI_ERR_INVALID = 4,        /* bad argument / shape / missing tensor */
    NAVI_ERR_HIP = 5,            /* a HIP runtime call failed */
    NAVI_ERR_UNSUPPORTED = 6,    /* model shape or device this build does not run */
    NAVI_ERR_CANCELLED = 7       /* the PCM consumer stopped the request (navi_synth's callback) */
} navi_status;

/* ---- device (runtime/device/device.h:43-66) ------------------------------ */

typedef struct {
    int32_t index;
    char    name[64];
    char    arch[32];                 /* gcnArchName without feature suffix, e.g. "gfx950" */
    int32_t multiprocessors;          /* CUs on CDNA */
    int32_t warp_size;                /* 64 */
    int32_t cooperative_launch;
    int32_t max_threads_per_block;
    uint64_t lds_per_block;
    int32_t clock_khz, mem_clock_khz, mem_bus_width;
    uint64_t vram_total, vram_free, l2_bytes;
    int32_t hip_runtime_version;
} navi_device_info;

/* Device::open (device.cpp:77-108): first visible gfx950 GPU, made current,
 * spin scheduling, one non-blocking stream owned by the library. */
navi_status navi_device_open(navi_device_info *out, char *err, size_t errlen);
/* The library stream (hipStream_t) for callers that enqueue their own work. */
void *navi_device_stream(void);
navi_status navi_device_synchronize(void);
/* Device::~Device (device.cpp:117-119): waits for the library stream and destroys it. Destroy
 * every handle first. A host calls it before the process exits, while the HIP runtime (and any
 * tool attached to it) is still up; a later call that needs the device opens it again. */
navi_status navi_device_close(void);
const char *navi_build_arch(void);    /* the offload arch the kernels were built for */

/* ---- device memory (DeviceWeights arena, device_weights.cpp:18-76; Impl::alloc) */

navi_status navi_mem_alloc(void **dptr, size_t bytes);   /* zero-filled */
navi_status navi_mem_free(void *dptr);
navi_status navi_mem_h2d(void *dst, const void *src, size_t bytes);
navi_status navi_mem_d2h(void *dst, const void *src, size_t bytes);
navi_status navi_mem_d2d(void *dst, const void *src, size_t bytes);
navi_status navi_mem_zero(void *dptr, size_t bytes);

/* ---- model description ----------------------------------------------------- */

typedef struct {                       /* params.h:16-27 TransformerParams */
    int32_t hidden, n_layer, n_head, n_kv_head, head_dim, ff, vocab;
    float   rms_eps;
    double  rope_theta;
} navi_xformer_params;

typedef struct {                       /* the fields of params.h:29-73 the path reads */
    navi_xformer_params talker, cp;
    int32_t n_code_groups;             /* 16 */
    int32_t codec_eos_id;              /* 2050 */
    int32_t text_hidden, text_vocab;   /* 2048, 151936 */
    int32_t tts_bos_id, tts_eos_id, tts_pad_id;
    int32_t codec_bos_id, codec_pad_id, codec_think_id, codec_nothink_id, codec_think_bos_id, codec_think_eos_id;
} navi_model_params;

typedef enum { NAVI_DT_F32 = 0, NAVI_DT_F16 = 1, NAVI_DT_BF16 = 2, NAVI_DT_I32 = 3, NAVI_DT_U8 = 4 } navi_dtype;

/* One device-resident weight (DeviceTensor, device_weights.h:17-21): the C
 * stand-in for DeviceWeights::get(name). Shapes are checked by each create(). */
typedef struct {
    const char *name;
    const void *ptr;
    int32_t     dtype;                 /* navi_dtype */
    int32_t     ndim;
    uint64_t    dims[4];
} navi_tensor_ref;

/* KV cache view (talker.h:20-24): per layer [max_pos][kv_dim] f16, caller-owned. */
typedef struct {
    int32_t   n_layer, max_pos, kv_dim;
    uint16_t *const *k;
    uint16_t *const *v;
} navi_kv_view;

/* ---- frame: talker step + cb0 sampling + code predictor (frame.h:24-71) ---- */

typedef struct {                       /* frame.h:24-31 */
    float   temperature;               /* <= 0: greedy */
    int32_t top_k;
    float   repetition_penalty;        /* <= 0: off */
    float   cp_temperature;
    int32_t cp_top_k;
    int32_t min_frames;
} navi_sampling;

typedef struct {                       /* frame.h:33-36 */
    int32_t  blocks_per_mp;            /* must be 1: one persistent block per CU */
    uint64_t spin_cap;                 /* polls per wait before the frame is failed; 0 = default */
} navi_frame_options;

typedef struct {                       /* frame.h:38-44 */
    int32_t ok;
    int32_t eos;                       /* codes[0] == codec_eos */
    int32_t codes[16];
    double  us;                        /* device time of the launch (hipEvent) */
    int32_t status;                    /* navi_status */
    char    error[160];
} navi_frame_result;

typedef struct navi_frame navi_frame;

/* Frame::create (frame.hip:684-774): binds weights by tensor name, allocates
 * the work buffers, sizes the persistent grid (one block per CU). */
navi_status navi_frame_create(const navi_model_params *p, const navi_tensor_ref *tensors, int32_t n_tensors,
                              const navi_frame_options *opt, navi_frame **out, char *err, size_t errlen);
void navi_frame_destroy(navi_frame *f);
/* Frame::reset (frame.hip:783-785): clears the repetition set. */
navi_status navi_frame_reset(navi_frame *f);
/* Frame::run_first / Frame::run (frame.hip:787-810) with Impl::launch (653-681).
 * skip_talker != 0: frame 0 from the prefill's post-norm hidden and logits
 * (kv may be NULL); else a talker step on the previous frame's step embedding at
 * position n_past (writes KV row n_past; the caller sets n_used = n_past + 1). */
navi_status navi_frame_run(navi_frame *f, const navi_kv_view *kv, int32_t n_past, int32_t skip_talker,
                           const float *d_hidden, const float *d_logits, const float *d_trailing,
                           const navi_sampling *s, uint64_t seed, int32_t frame_index, navi_frame_result *out);
/* The on-device frame loop (the "next" step after Frame::run: graph.cpp:90-105 calls run once per
 * frame and syncs on each): up to n_frames frames enqueued back to back, no host round trip between
 * them. Frame i runs as navi_frame_run would with frame index frame_index0 + i, trailing row i of
 * d_trailing (n_trailing rows of f32 [hidden]) then d_tts_pad, the same seeds; with skip_first,
 * frame 0 is run_first from d_hidden / d_logits, else frame i is a talker step at n_past0 + i
 * (writing KV row n_past0 + i). A frame that samples EOS ends the loop on the device (it is
 * counted: *eos = 1, its codes are the last row); a timed-out frame ends it with
 * NAVI_ERR_TIMEOUT. codes_out: host i32 [n_frames][16], the first *n_done rows valid; *us: device
 * time of the whole loop (may be NULL). n_frames <= 4096. */
navi_status navi_frame_run_many(navi_frame *f, const navi_kv_view *kv, int32_t n_past0, int32_t skip_first,
                                const float *d_hidden, const float *d_logits, const float *d_trailing, int32_t n_trailing,
                                const float *d_tts_pad, const navi_sampling *s, uint64_t seed, int32_t frame_index0,
                                int32_t n_frames, int32_t *codes_out, int32_t *n_done, int32_t *eos, double *us, char *err,
                                size_t errlen);
/* Frame::d_step_out (frame.hip:812): next frame's step embedding, f32[hidden]. */
float *navi_frame_step_out(navi_frame *f);
int32_t navi_frame_grid_blocks(const navi_frame *f);
int32_t navi_frame_occupancy_per_mp(const navi_frame *f);
/* Test/diagnostic taps (no reference counterpart; off unless enabled): the talker's
 * post-norm hidden f32[hidden], its logits f32[vocab] and the 15 cp logit rows
 * f32[15][cp vocab] of the last frame run with taps on. */
navi_status navi_frame_set_taps(navi_frame *f, int32_t enabled);
const float *navi_frame_tap_hidden(const navi_frame *f);
const float *navi_frame_tap_logits(const navi_frame *f);
const float *navi_frame_tap_cp_logits(const navi_frame *f);
/* Phase profile (the reference's NAVI_FRAME_PROFILE, frame.hip:71-73, as a runtime switch):
 * with profiling on, thread 0 of every block stamps the 100 MHz real-time counter at the start
 * and end of every wait of the next runs; navi_frame_profile copies the first n_slots stamps of
 * blocks 0..n_blocks-1 (slots past a block's last stamp are 0 for a fresh buffer). */
navi_status navi_frame_set_profile(navi_frame *f, int32_t enabled);
navi_status navi_frame_profile(const navi_frame *f, uint64_t *out, int32_t n_blocks, int32_t n_slots);
/* Test hooks for the launch epoch and the spin cap (no reference counterpart). Each launch uses
 * the epoch after the current one (+4096); epochs wrap after 2^20 launches, and the wrap clears
 * the mailboxes and the abort word first. set_epoch takes a multiple of 4096 up to 2^32 - 4096 so
 * a test can reach the wrap; set_spin_cap changes the polls per wait (0 = the default). */
navi_status navi_frame_set_epoch(navi_frame *f, uint32_t epoch);
uint32_t navi_frame_epoch(const navi_frame *f);
navi_status navi_frame_set_spin_cap(navi_frame *f, uint64_t spin_cap);

/* ---- talker: prompt rows, prefill, KV cache (talker.h:34-67) ----------------- */

typedef struct navi_talker navi_talker;

typedef struct {                       /* talker.h:26-32 Prompt: device rows owned by the talker */
    const float *prefill;              /* f32 [n_prefill][hidden] */
    const float *trailing;             /* f32 [n_trailing][hidden] */
    const float *tts_pad;              /* f32 [hidden] */
    int32_t n_prefill, n_trailing;
} navi_prompt;

/* Talker::create (talker.hip:200-274): binds the talker's weights by name (text embedding,
 * text projection, layers, final norm, codec head, codec embedding), allocates the KV cache
 * (max_positions rows per layer, f16 [max_positions][kv_dim]) and the prompt/prefill work
 * buffers for up to max_prompt_tokens rows. */
navi_status navi_talker_create(const navi_model_params *p, const navi_tensor_ref *tensors, int32_t n_tensors,
                               int32_t max_prompt_tokens, int32_t max_positions, navi_talker **out,
                               char *err, size_t errlen);
void navi_talker_destroy(navi_talker *t);
/* Talker::build_prompt (talker.hip:283-352). ids: host i32[n_ids] = role header (3), text,
 * trailer (5); language_id: the codec id of the language (the `talker.language.<name>` key),
 * or < 0 for "auto" (no language row); speaker: host f32[hidden]. The returned rows stay
 * valid until the next build_prompt. */
navi_status navi_talker_build_prompt(navi_talker *t, const int32_t *ids, int32_t n_ids, int32_t language_id,
                                     const float *speaker, navi_prompt *out, char *err, size_t errlen);
/* Talker::prefill (talker.hip:354-399): d_rows f32 [n_rows][hidden] (device) at positions
 * 0..n_rows-1; writes KV rows 0..n_rows-1, keeps the last row's post-norm hidden and its
 * logits, and sets the cache's n_used to n_rows. */
navi_status navi_talker_prefill(navi_talker *t, const float *d_rows, int32_t n_rows, char *err, size_t errlen);
/* enabled != 0: the prefill's layers for each row count are captured once as a HIP graph and
 * replayed; 0 (the default): every kernel is launched from the host (on MI355X the replays measured
 * no faster). Results are identical either way. No reference counterpart. */
navi_status navi_talker_set_graphs(navi_talker *t, int32_t enabled);
/* Talker::kv (talker.h:57): the cache as the view navi_frame_run takes; *n_used (may be NULL)
 * is the number of rows the last prefill wrote. The pointer arrays live as long as t. */
navi_status navi_talker_kv(navi_talker *t, navi_kv_view *out, int32_t *n_used);
const float *navi_talker_hidden(const navi_talker *t);   /* Talker::d_hidden: f32[hidden] */
const float *navi_talker_logits(const navi_talker *t);   /* Talker::d_logits: f32[vocab] */
double navi_talker_last_ms(const navi_talker *t);         /* Talker::last_ms: device time of the last prefill */

/* ---- linear layer (Talker::Impl::gemm, talker.hip:158-187; k_gemm_skinny / k_conv<K=1>,
 * kernels.h:73-330) -----------------------------------------------------------------------
 * d_y[m][n] = act(bias[n] + sum_k d_x[m][k] * w[n][k]) + residual[m][n] for m < M, n < N.
 * d_x f32 rows with stride ldx, w f16 [N][K] row-major (nn.Linear layout), d_y f32 rows with
 * stride ldy. bias, residual may be NULL; residual may alias d_y. act: 0 none, 1 SiLU.
 * Requires K % 32 == 0, N % 64 == 0, ldx % 4 == 0, 16-byte aligned d_x and w, and
 * |x| < 65504 (the activations travel as f16 hi + lo pairs through the matrix cores; a larger
 * value fails with NAVI_ERR_INVALID). Runs on the library stream and returns when done. */
navi_status navi_linear(const float *d_x, int32_t ldx, int32_t M, const uint16_t *w, int32_t K, int32_t N,
                        const float *bias, const float *residual, int32_t act, float *d_y, int32_t ldy,
                        char *err, size_t errlen);
/* navi_linear without any allocation. No counterpart in the reference: it is for callers that
 * cannot allocate device memory (serving loops or harnesses that forbid hipMalloc). It runs on
 * the library stream and synchronizes it, so it does not belong in a graph the caller captures.
 * Same arguments, kernels and results (bit-identical) as navi_linear, but the
 * split-K partials live in a fixed 8 MiB array of the library on each GPU (held until the process
 * ends) instead of a workspace the library allocates: S x M x N floats must fit in its
 * 2,097,088 floats (S, navi_linear's K-split count, is at most K / 256 and falls as the output
 * tiles grow), else NAVI_ERR_INVALID says so. The device must already be open
 * (navi_device_open). Every call on a GPU shares that array and leaves its partials there; calls
 * that overlap on one GPU (several host threads or streams) race. */
navi_status navi_linear_noalloc(const float *d_x, int32_t ldx, int32_t M, const uint16_t *w, int32_t K, int32_t N,
                                const float *bias, const float *residual, int32_t act, float *d_y, int32_t ldy,
                                char *err, size_t errlen);

/* ---- vocoder: codes -> 24 kHz PCM (vocoder.h:27-55) -------------------------- */

typedef struct navi_vocoder navi_vocoder;

typedef struct {                       /* the codec decoder fields of params.h (params.cpp:106-117) */
    navi_xformer_params xf;            /* pre-transformer: hidden 512, 8 layers, 16 x 64 heads, ff 1024,
                                          rms eps 1e-5, rope theta 1e4 (vocab unused) */
    int32_t latent_dim;                /* 1024 */
    int32_t codebook_dim;              /* 512 (the RVQ works on codebook_dim / 2) */
    int32_t codebook_size;             /* 2048 */
    int32_t n_q, n_semantic;           /* 16, 1 */
    int32_t decoder_dim;               /* 1536 */
    int32_t sliding_window;            /* 72 */
    int32_t upsampling_ratios[2];      /* 2, 2 */
    int32_t upsample_rates[4];         /* 8, 5, 4, 3 */
    int32_t samples_per_frame;         /* 1920 = the product of the ratios and rates */
} navi_vocoder_params;

/* Vocoder::create (vocoder.hip:427-602): binds the codec.decoder.* tensors by name, prepares
 * the device-side copies the kernels read (concatenated projections and codebooks, tap-major
 * conv weights, phase-split transposed convs, exp'd Snake parameters) and the streaming state
 * for chunks of up to max_chunk_frames frames. */
navi_status navi_vocoder_create(const navi_vocoder_params *p, const navi_tensor_ref *tensors, int32_t n_tensors,
                                int32_t max_chunk_frames, navi_vocoder **out, char *err, size_t errlen);
void navi_vocoder_destroy(navi_vocoder *v);
/* Vocoder::reset (vocoder.hip:604-615): a new utterance (clears the causal histories, position 0). */
navi_status navi_vocoder_reset(navi_vocoder *v);
/* Vocoder::decode (vocoder.hip:617-636): codes host i32 [n_frames][n_q] in [0, codebook_size),
 * continuing the utterance; writes n_frames * samples_per_frame samples to host pcm (where
 * the reference appends to a vector). Decodes in chunks of max_chunk_frames; synchronous. */
navi_status navi_vocoder_decode(navi_vocoder *v, const int32_t *codes, int32_t n_frames, float *pcm, char *err,
                                size_t errlen);
/* Vocoder::set_stage_hook (vocoder.h:46-48; vocoder.hip:180-185, 638): fn (NULL = off) is called
 * after every stage of a chunk with the stage's name (the reference's names: "rvq", "pre_conv",
 * "in_proj", "norm1_<l>", "qkv_<l>" (before RoPE), "attnraw<l>", "xattn_<l>", "layer<l>",
 * "pre_transformer", "up<j>_t", "up<j>_ln", "up<j>_cnx", "dec0", "dec<b>_b1".."dec<b>_b4", "pcm")
 * and its device buffer f32 [rows][cols], after the stream has drained; the buffer is valid
 * during the call. For debugging: every stage then synchronizes. */
typedef void (*navi_stage_fn)(void *user, const char *name, const float *d_buf, int32_t rows, int32_t cols);
navi_status navi_vocoder_set_stage_hook(navi_vocoder *v, navi_stage_fn fn, void *user);
/* enabled != 0: each chunk size's launch sequence is captured once per history parity as a HIP
 * graph and replayed (the stage hook always runs eagerly); 0 (the default): every kernel is
 * launched from the host (on MI355X the replays measured no faster). The PCM is identical either
 * way. No reference counterpart. */
navi_status navi_vocoder_set_graphs(navi_vocoder *v, int32_t enabled);
/* vocoder_owns_tensor (vocoder.hip:413-425): whether DeviceWeights::upload may skip a tensor
 * because the vocoder reads it from the file itself. Always 0 here: navi_vocoder_create makes
 * its re-laid-out copies on the device from the arena, so the arena must hold every
 * codec.decoder.* tensor. */
int32_t navi_vocoder_owns_tensor(const char *name);
int32_t navi_vocoder_samples_per_frame(const navi_vocoder *v);   /* Vocoder::samples_per_frame */
int32_t navi_vocoder_max_chunk_frames(const navi_vocoder *v);    /* Vocoder::max_chunk_frames */
double navi_vocoder_last_ms(const navi_vocoder *v);              /* Vocoder::last_ms: device time of the last decode */

/* ---- speaker encoder: 24 kHz audio -> speaker embedding (speaker.h:17-38) ------------ */

typedef struct navi_speaker navi_speaker;

typedef struct {                       /* the speaker fields of params.h:53-55 (params.cpp:97-104) */
    int32_t sample_rate;               /* 24000 */
    int32_t enc_dim;                   /* 1024: the embedding width (the talker's hidden) */
    int32_t n_fft, num_mels, hop, win; /* 1024, 128, 256, 1024 (win must equal n_fft, a power of 2) */
    float   fmin, fmax;                /* 0, 12000 */
} navi_speaker_params;

/* SpeakerEncoder::mel (speaker.hip:269-303): host log-mel [num_mels][*n_frames] of a mono
 * waveform in [-1, 1] (reflect padding (n_fft - hop) / 2, periodic Hann, |FFT|, slaney
 * filterbank, log(max(., 1e-5))). mel_out == NULL only sets *n_frames; otherwise capacity (in
 * floats) must hold num_mels * n_frames. Fails with NAVI_ERR_INVALID ("too short") when
 * n <= (n_fft - hop) / 2. No device work. */
navi_status navi_speaker_mel(const navi_speaker_params *p, const float *wav, int64_t n, float *mel_out, int64_t capacity,
                             int32_t *n_frames, char *err, size_t errlen);
/* SpeakerEncoder::create (speaker.hip:219-260): binds the speaker_encoder.* tensors by name
 * (shapes as params.cpp:165-194) and sizes the work buffers for max_seconds of audio. */
navi_status navi_speaker_create(const navi_speaker_params *p, const navi_tensor_ref *tensors, int32_t n_tensors,
                                double max_seconds, navi_speaker **out, char *err, size_t errlen);
void navi_speaker_destroy(navi_speaker *h);
/* SpeakerEncoder::embed_mel (speaker.hip:305-321): host mel [num_mels][n_frames] -> host
 * emb[enc_dim]. n_frames in [5, the max_seconds bound] (longer: "longer than the encoder's
 * max_seconds", as the reference). Synchronous. */
navi_status navi_speaker_embed_mel(navi_speaker *h, const float *mel, int32_t n_frames, float *emb, char *err, size_t errlen);
/* SpeakerEncoder::embed (speaker.hip:323-327): the log-mel of navi_speaker_mel, computed on the
 * device in the same double precision (equal to float rounding), then the network.
 * Errors as navi_speaker_mel and navi_speaker_embed_mel. Synchronous. */
navi_status navi_speaker_embed(navi_speaker *h, const float *wav, int64_t n, float *emb, char *err, size_t errlen);
int32_t navi_speaker_dim(const navi_speaker *h);         /* the embedding width (enc_dim) embed writes */
double navi_speaker_last_ms(const navi_speaker *h);      /* SpeakerEncoder::last_ms: device time of the last embed
                                                            (front end included for navi_speaker_embed) */
/* Diagnostics: the device log-mel of the last embed, time-major f32 [*n_frames][num_mels]. */
const float *navi_speaker_tap_mel(const navi_speaker *h, int32_t *n_frames);

/* ---- one request end to end (Graph::synth, graph.cpp:52-111) ------------------------ */

typedef struct {                       /* graph.h SynthRequest, with the text already tokenized */
    const int32_t *ids;                /* host i32[n_ids]: role header, text, trailer (build_prompt's input) */
    int32_t n_ids;
    int32_t language_id;               /* codec language id, < 0 = auto */
    const float *speaker;              /* host f32[hidden] */
    /* Optional prompt given as device rows instead of ids (prefill, trailing, tts_pad): used when
     * d_prefill != NULL, e.g. to prefill the text itself. */
    const float *d_prefill, *d_trailing, *d_tts_pad;
    int32_t n_prefill, n_trailing;
    uint64_t seed;
    int32_t max_frames;                /* cap (600 = 48 s at 12.5 Hz) */
    navi_sampling sampling;
    int32_t vocoder_batch;             /* frames per vocoder call; 0 = the vocoder's max chunk */
    int32_t first_batch;               /* frames in the first call (time to first audio); 0 = vocoder_batch */
} navi_synth_request;

typedef struct {                       /* graph.h SynthStats */
    int32_t n_tokens, n_frames, hit_cap, eos;
    double prefill_ms, frames_ms, vocoder_ms, total_ms, ttfa_ms, audio_s, rtf;
} navi_synth_stats;

/* PCM of each vocoder batch, in order; n samples at 24 kHz. Returns 0 to go on; non-zero stops
 * the request, which is how an exception thrown by Graph::synth's on_pcm (the server's "client
 * stopped reading", server.cpp:431-437) ends it: no further frame runs and navi_synth returns
 * NAVI_ERR_CANCELLED with the stats of what was delivered. */
typedef int32_t (*navi_pcm_callback)(const float *pcm, int32_t n, void *user);

/* Graph::synth: prompt -> prefill -> frames until EOS or max_frames -> vocoder in batches
 * (first_batch frames first, then vocoder_batch), PCM handed to on_pcm per batch on the calling
 * thread. Frame and vocoder are reset first; the frame runs on the talker's KV cache. Wall-clock
 * stats. */
navi_status navi_synth(navi_talker *t, navi_frame *f, navi_vocoder *v, const navi_synth_request *req,
                       navi_pcm_callback on_pcm, void *user, navi_synth_stats *stats, char *err, size_t errlen);

/* ---- multi-stream batched decode -------------------------------------
 * No counterpart in the reference, which decodes one request at a time: this is the batch-1
 * frame (navi_frame_run; k_frame, frame.hip:517-579) applied to n independent streams at once,
 * for servers that hold many requests. Stream i computes the frame navi_frame_run computes for
 * it alone (same seeds, sampling rules and step assembly), up to the summation order of the
 * projections, which run as GEMMs over the streams on the matrix cores. */

typedef struct navi_streams navi_streams;

/* Binds the talker and code-predictor weights by name (the names navi_frame_create binds) and
 * allocates the work buffers for up to max_streams streams whose contexts reach max_positions. */
navi_status navi_streams_create(const navi_model_params *p, const navi_tensor_ref *tensors, int32_t n_tensors,
                                int32_t max_streams, int32_t max_positions, navi_streams **out, char *err, size_t errlen);
void navi_streams_destroy(navi_streams *h);
/* Clears the repetition set of one stream (stream >= 0) or of all (stream < 0): Frame::reset. */
navi_status navi_streams_reset(navi_streams *h, int32_t stream);
/* One frame for streams 0..n-1. Host arrays of n: kv (each stream's cache, borrowed; row n_past[i]
 * is written), n_past, seeds, frame_index. d_step_in: device f32 [n][hidden] step inputs, or NULL
 * to continue from this handle's step_out rows; d_trailing: device f32 [n][hidden] (each stream's
 * trailing text row). codes_out: host i32 [n][16]; stream i ended when codes_out[i][0] is the EOS
 * id. Errors as navi_frame_run's: NAVI_ERR_KV_FULL names the stream. Synchronous. */
navi_status navi_streams_run(navi_streams *h, int32_t n, const navi_kv_view *kv, const int32_t *n_past, const float *d_step_in,
                             const float *d_trailing, const navi_sampling *s, const uint64_t *seeds,
                             const int32_t *frame_index, int32_t *codes_out, char *err, size_t errlen);
float *navi_streams_step_out(navi_streams *h);           /* device f32 [max_streams][hidden]: the next step inputs */
/* Diagnostics (as navi_frame_set_taps): when on, each run copies the talker's post-norm hidden
 * [max_streams][hidden], raw codec logits [max_streams][talker vocab] and the 15 cp logit rows
 * [max_streams][15][cp vocab] to device buffers. */
navi_status navi_streams_set_taps(navi_streams *h, int32_t on);
/* Replays each run from a captured HIP graph (on by default; runs with taps on are always
 * enqueued directly). Off: every kernel is launched by the host each run, the reference point
 * the graph replays are tested against. */
navi_status navi_streams_set_graphs(navi_streams *h, int32_t on);
const float *navi_streams_tap_hidden(const navi_streams *h);
const float *navi_streams_tap_logits(const navi_streams *h);
const float *navi_streams_tap_cp_logits(const navi_streams *h);
int32_t navi_streams_max_streams(const navi_streams *h);
double navi_streams_last_ms(const navi_streams *h);      /* device time of the last navi_streams_run */

#ifdef __cplusplus
}
#endif

#endif /* NAVI_AMD_H */
