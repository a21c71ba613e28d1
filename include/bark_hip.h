/*
 * bark_hip — C ABI of the MI355X (gfx950) Conformer encoder backend, with the
 * log-mel front end and the greedy TDT decoder on either side of it.
 *
 * The reference (eclipse005/bark3-wgpu, Rust) drives its GPU encoder through
 * `AsrInference::load` -> `Encoder::load_with` -> `Encoder::encode[_pre]`, its
 * conv front end through `SubGpu::run`, its features through
 * `MelFrontend::compute` and its decoder through `TdtDecoder::decode` /
 * `GpuTdtDecoder::decode_async`. These entry points are what a `Backend::Hip`
 * arm binds over FFI in place of those calls, through a Rust `extern "C"`
 * block that declares them as below.
 *
 * Conventions
 *  - Every function returns 0 on success and a negative code on error; the
 *    message is available from bark_hip_last_error() (thread-local), the
 *    counterpart of the reference's `anyhow::Error`.
 *  - Host pointers are borrowed for the duration of the call only.
 *  - Calls on one handle are serialised by an internal mutex (the reference
 *    shares `&AsrInference` across threads, src/inference.rs:17-18). The
 *    mutex orders the host side; the device side is ordered too: every call
 *    records an event on the stream it queued its work on, and a call on a
 *    different stream waits for that event before its first kernel, because
 *    all calls share the handle's workspace buffers. So device-form calls on
 *    several streams are safe, but calls on one handle never overlap on the
 *    device; use one handle per stream for concurrent encodes.
 *  - A device-form call returns without synchronising with the device, also
 *    when the batch packing changes (the plan tables are staged in pinned
 *    host memory). It blocks only when a workspace buffer must grow (the old
 *    buffer may still be in use), i.e. the first time a larger batch is seen.
 *  - No C++ exceptions cross this boundary.
 */
#ifndef BARK_HIP_H
#define BARK_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct BarkHip BarkHip;

enum {
  BARK_HIP_OK = 0,
  BARK_HIP_EINVAL = -1,  /* bad argument / shape / unknown tensor name */
  BARK_HIP_ESTATE = -2,  /* call out of order (e.g. encode before finalize) */
  BARK_HIP_EDEVICE = -3, /* HIP runtime error, no device */
  BARK_HIP_EINTERNAL = -4
};

/* Thread-local description of the last error on this thread. */
const char *bark_hip_last_error(void);

/* Number of visible HIP devices (0 when none): the probe behind
 * `Backend::Auto`'s fall-back to the CPU path (src/inference.rs:219-229). */
int bark_hip_device_count(void);

/* Replaces Gpu::new_with + the start of Encoder::load_with
 * (src/gpu.rs:448, src/encoder.rs:412). `n_layers` is 24 for the real model;
 * fewer blocks are accepted for tests. */
int bark_hip_create(int device, int n_layers, BarkHip **out);
void bark_hip_destroy(BarkHip *h);

/* ---- weight ingest: one call per reference tensor name -----------------
 * Names are the reference's (src/encoder.rs:423-604, src/sub.rs:85-89), e.g.
 * "encoder.layers.3.feed_forward1.linear1.weight". Values are the checkpoint
 * values in the stated encoding; the library keeps its own copy. */

/* f32 values (RawTensor::to_f32, src/raw.rs:23-48). Linear weights given this
 * way are rounded to f16 (RNE) like RawTensor::to_f16_words (src/raw.rs:66-97). */
int bark_hip_set_f32(BarkHip *h, const char *name, const float *v, const int64_t *shape,
                     int ndim);
/* f16 bits (rows, cols) row-major (RawTensor::to_f16_words, src/raw.rs:66-97). */
int bark_hip_set_f16(BarkHip *h, const char *name, const uint16_t *v, int64_t rows,
                     int64_t cols);
/* The reference's low-bit layout (LowBitTensor, src/bark.rs:31-48;
 * upload_lowbit, src/encoder.rs:288-317): codes rows x ceil(cols/8) u32, nibble
 * col&7 of word col>>3; levels rows x 4 f16, k_lev in 1..3. Expanded on load
 * to the 16-entry table lut[c] = expand(c, k_lev, levels) (src/bark.rs:597-611). */
int bark_hip_set_lowbit(BarkHip *h, const char *name, const uint32_t *codes,
                        const uint16_t *levels, uint32_t k_lev, int64_t rows, int64_t cols);
/* Generic 4-bit format: codes rows x cols/2 bytes (two per byte, low nibble =
 * even column), lut16 rows x 16 f16. Byte-identical code layout to the above. */
int bark_hip_set_lut4(BarkHip *h, const char *name, const uint8_t *codes,
                      const uint16_t *lut16, int64_t rows, int64_t cols);
/* TensorReader::open_model + read (src/weights_io.rs:46-127) feeding the
 * calls above: stages every tensor this handle reads (front end, encoder
 * blocks below n_layers, projector, TDT decoder and joint) from a safetensors
 * checkpoint. `path` is a .safetensors file or a model directory holding
 * model.safetensors, or model.safetensors.index.json and its shards. F32 and
 * F16 entries are taken as stored, BF16 widened exactly to f32 (linears are
 * then rounded to f16 as with bark_hip_set_f32); integer entries are skipped.
 * Tensors are read one at a time. Call before bark_hip_finalize. */
int bark_hip_load_safetensors(BarkHip *h, const char *path);
/* probe (src/weights_io.rs:208-297): what a safetensors checkpoint holds,
 * from its header(s) alone, as JSON {"release": string|null, "layout":
 * "bf16"|"f16"|"f32"|"low-bit", "tensors", "weights", "layers", "hidden",
 * "ffn", "vocab"} (4-bit code words count eight weights; ".levels" tables are
 * not weights) written to buf (cap bytes). Needs no device. */
int bark_hip_probe(const char *path, char *buf, size_t cap);
/* Fuses q|k|v (load_qkv, src/encoder.rs:342-402), folds BatchNorm
 * (src/encoder.rs:546-557), interleaves pw1 rows for the GLU epilogue and
 * uploads everything. Returns BARK_HIP_EINVAL naming a missing tensor. */
int bark_hip_finalize(BarkHip *h);

/* ---- forward ------------------------------------------------------------ */

/* Encoder::encode (src/encoder.rs:1985-2001): sub_rows (t, 4096) f32 host ->
 * pooler (t, 640) f32 host. block: if dump_layer >= 0, receives the pre-norm
 * residual (t, 1024) of that block (src/encoder.rs:2598-2606); may be NULL. */
int bark_hip_encode_sub(BarkHip *h, const float *sub_rows, int32_t t, int32_t dump_layer,
                        float *pooler, float *block);

/* SubGpu::run + Encoder::encode_pre (src/sub_gpu.rs:574-776,
 * src/encoder.rs:2005-2657): mel (n_frames, 128) f32 host -> pooler. t_out
 * receives T = conv_len^3(n_frames); pooler_cap is the capacity in floats. */
int bark_hip_encode_mel(BarkHip *h, const float *mel, int32_t n_frames, int32_t n_valid,
                        int32_t *t_out, float *pooler, size_t pooler_cap);

/* Batched form for chunked / multi-utterance input (src/inference.rs:311-326
 * runs the chunks one after another). mel holds the utterances back to back;
 * each result equals that utterance's own bark_hip_encode_mel. Sequences are
 * packed without padding between them apart from 64-row alignment; weights
 * are streamed once per batch. pooler receives sum(t_out[i]) rows. */
int bark_hip_encode_mel_batch(BarkHip *h, const float *mel, const int32_t *n_frames,
                              const int32_t *n_valid, int32_t batch, int32_t *t_out,
                              float *pooler, size_t pooler_cap);

/* Device-resident form of bark_hip_encode_mel_batch: d_mel and d_pooler are
 * device pointers, work is queued on `stream` (a hipStream_t; NULL = the
 * handle's stream) and the call returns without synchronising. */
int bark_hip_encode_mel_batch_device(BarkHip *h, const float *d_mel, const int32_t *n_frames,
                                     const int32_t *n_valid, int32_t batch, int32_t *t_out,
                                     float *d_pooler, size_t pooler_cap, void *stream);

/* ---- TDT decoder ---------------------------------------------------------
 * Present when the decoder's tensors were set before bark_hip_finalize, under
 * the reference's names (TdtDecoder::from_source, src/tdt.rs:130-162):
 * "decoder.embedding.weight" (8193, 640), "decoder.lstm.weight_ih_l0/_l1",
 * "decoder.lstm.weight_hh_l0/_l1" (2560, 640), "decoder.lstm.bias_ih_l0/_l1",
 * "decoder.lstm.bias_hh_l0/_l1" (2560), "decoder.decoder_projector.weight"
 * (640, 640) and ".bias", "joint.head.weight" (8198, 640) and ".bias". Matrices
 * are kept as f16 (RNE) like the reference's pack16. */

/* TdtDecoder::decode (src/tdt.rs:318-414): greedy TDT decoding of a host
 * pooler (t_len, 640) f32. tokens receives n_tokens {id, frame, dur} u32
 * triples (tdt::Token, src/tdt.rs:31-41); cap counts triples, and a count above
 * it is an error (BARK_HIP_EINVAL, n_tokens still set). t_len * 14 + 64
 * triples always suffice. t_len == 0 gives no tokens. */
int bark_hip_tdt_decode(BarkHip *h, const float *pooler, int32_t t_len, uint32_t *tokens, size_t cap,
                        int32_t *n_tokens);

/* GpuTdtDecoder::decode_async (src/tdt_gpu.rs:206-300): the same on a device
 * pooler (e.g. the output of bark_hip_encode_mel_batch_device), queued on
 * `stream` (NULL = the handle's stream). The decoder state stays on the device;
 * the call synchronises once per chunk of steps and returns with the tokens
 * in host memory. */
int bark_hip_tdt_decode_device(BarkHip *h, const float *d_pooler, int32_t t_len, uint32_t *tokens,
                               size_t cap, int32_t *n_tokens, void *stream);

/* Batched form (utterances decoded together: every launch advances all of
 * them, so a batch costs about as many launches as its longest member): the
 * poolers of `batch` utterances back to back, t_lens[u] rows each (the layout
 * bark_hip_encode_mel_batch writes). n_tokens[u] receives utterance u's count;
 * tokens receives every utterance's triples back to back in order; cap counts
 * triples (sum of t_lens[u] * 14 + 64 always suffices). Chunked transcription
 * (src/inference.rs:311-326) decodes its chunks one after another; the result
 * per chunk is the same. */
int bark_hip_tdt_decode_batch(BarkHip *h, const float *pooler, const int32_t *t_lens, int32_t batch,
                              uint32_t *tokens, size_t cap, int32_t *n_tokens);
/* Device-pointer form of bark_hip_tdt_decode_batch, queued on `stream`. */
int bark_hip_tdt_decode_batch_device(BarkHip *h, const float *d_pooler, const int32_t *t_lens,
                                     int32_t batch, uint32_t *tokens, size_t cap, int32_t *n_tokens,
                                     void *stream);

/* Transcription up to the tokens (AsrInference::transcribe's mel -> encoder
 * -> decoder, src/transcription.rs:56-224, over the VAD chunks of
 * src/inference.rs:298-386): log-mel of each 16 kHz wave, one batched encode,
 * and one batched greedy TDT decode of the waves' poolers in device memory (the pooler
 * never leaves the device, as with the reference's pooler_buf,
 * src/transcription.rs:200-209). t_out[i] (may be NULL) receives wave i's T;
 * n_tokens[i] its token count; tokens receives every wave's {id, frame, dur}
 * triples back to back in wave order (cap counts triples; sum of
 * T_i * 14 + 64 always suffices). Needs the decoder's tensors. */
int bark_hip_transcribe_wave_batch(BarkHip *h, const float *waves, const int64_t *n_samples,
                                   int32_t batch, int32_t *t_out, uint32_t *tokens, size_t cap,
                                   int32_t *n_tokens);

/* Per-operator GPU timing, the counterpart of BARK3_ENC_PROFILE
 * (src/encoder/prof.rs:1-127, src/encoder.rs:823-827): while enabled, every
 * launch of the forward is bracketed by HIP events on its stream. Enabling or
 * disabling discards what was recorded. */
int bark_hip_profile(BarkHip *h, int enable);
/* Restricts the per-operator timing to launches labelled `label` (NULL or ""
 * = every launch), so a benchmark can time one kernel inside its timed region
 * without timing all the others; with a label, every 8th launch of it is
 * timed (a timed launch costs a few microseconds of dispatch). Discards what
 * was recorded. */
int bark_hip_profile_only(BarkHip *h, const char *label);
/* Writes JSON {label: {count, ms, flops, bytes}} aggregated over everything
 * recorded since the last report (flops/bytes are the algorithmic work of the
 * launches) and clears it. Synchronises with the recorded work. */
int bark_hip_profile_report(BarkHip *h, char *buf, size_t cap);

/* Isolated 4-bit level-table linear (one bm64_lb dispatch of Ctx::gemm_f32,
 * src/encoder.rs:1039-1100, in the generic table format): device pointers
 * A (T, K) activations, codes (N, K/2) bytes, lut16 (N, 16) f16, C (T, N).
 * a_dtype: 0 = f16, 1 = bf16. c_dtype: 0 = f32, 1 = f16, 2 = bf16.
 * K % 256 == 0, N % 128 == 0. Queued on `stream`, not synchronised.
 * The product runs on f16 MFMA (the levels are f16, so dequantisation is
 * exact; accumulation is f32). bf16 activations are converted to f16 on the
 * way into the tile: exact for 0 and for 6.104e-5 <= |a| <= 65504 (every bf16
 * value in the f16 normal range); smaller magnitudes are rounded to f16
 * subnormals (absolute error <= 3e-8, below 3e-8 they become 0) and larger
 * ones overflow to +-inf. */
int bark_hip_lowbit_linear(const void *A, int32_t a_dtype, const uint8_t *codes,
                           const uint16_t *lut16, void *C, int32_t c_dtype, int32_t T,
                           int32_t K, int32_t N, void *stream);

/* No counterpart in the reference. For callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc): bark_hip_lowbit_linear with the same arguments, kernels
 * and results, which calls no allocating routine. Where that entry point
 * splits K over a grow-only workspace (small T, or a long K), this one keeps
 * the partial sums in a fixed device array of 24 MiB per GPU, held from the
 * first call on a GPU until the process ends; a shape whose partial sums need
 * more (split count x T x N x 4 bytes) is rejected with BARK_HIP_EINVAL. Every
 * call on one GPU shares that GPU's array: calls that overlap on one GPU (on
 * different streams) race and must be ordered by the caller. */
int bark_hip_lowbit_linear_noalloc(const void *A, int32_t a_dtype, const uint8_t *codes,
                                   const uint16_t *lut16, void *C, int32_t c_dtype, int32_t T,
                                   int32_t K, int32_t N, void *stream);

/* Log-mel front end, the counterpart of MelFrontend (src/mel.rs:10-140).
 * bark_hip_set_mel_filters takes the 128 x 257 row-major f32 filterbank, as
 * MelFrontend::new does (src/mel.rs:25; the reference loads it from
 * data/mel_filters.f32, src/inference.rs:46,480). */
int bark_hip_set_mel_filters(BarkHip *h, const float *filters);
/* MelFrontend::compute (src/mel.rs:41): features of a 16 kHz mono wave of
 * n_samples f32 samples. Writes n_frames = 1 + n/160 rows x 128 f32 into
 * `features` (capacity `cap` floats; padded rows >= n_valid = n/160 are zero)
 * and the two counts — the Features struct (src/mel.rs:17-22). Host buffers;
 * synchronises. */
int bark_hip_mel(BarkHip *h, const float *wave, int64_t n_samples, float *features, size_t cap,
                 int32_t *n_frames, int32_t *n_valid);
/* Device-resident form: d_wave and d_features are device pointers, work is
 * queued on `stream` (hipStream_t; NULL = the handle's stream), no host copies,
 * not synchronised; the output can feed bark_hip_encode_mel_batch_device. */
int bark_hip_mel_device(BarkHip *h, const float *d_wave, int64_t n_samples, float *d_features, size_t cap,
                        int32_t *n_frames, int32_t *n_valid, void *stream);
/* Batched chunk encode: the log-mel features (as bark_hip_mel) of each of
 * `batch` 16 kHz waves, concatenated in `waves` with n_samples[i] samples
 * each, encoded by one bark_hip_encode_mel_batch call — the per-chunk mel and
 * encoder work of the reference's chunked transcription (src/inference.rs:
 * 298-386, src/transcription.rs:56-122) as one batched call; each result equals
 * that wave's own bark_hip_mel + bark_hip_encode_mel. pooler receives
 * sum(t_out[i]) rows x 640 f32. Host buffers; synchronises. */
int bark_hip_encode_wave_batch(BarkHip *h, const float *waves, const int64_t *n_samples, int32_t batch,
                               int32_t *t_out, float *pooler, size_t pooler_cap);

#ifdef __cplusplus
}
#endif
#endif
