/*
 * yuf_engine.h -- C ABI of libyufhip.so, the MI355X (gfx950) backend for the
 * YufMusicGen recurrent hot path.
 *
 * The entry points mirror the reference's engine and operator surfaces:
 *   - the Rust/Vulkan engine API of YufeiV/YufMusicGen (`vulkan/`): checkpoint
 *     load, model creation, per-token step, state reset, sampling;
 *   - the Python operators `rwkv7_cuda` and `rosa_householder_scan`
 *     (`yufmusicgen/cuda_ops.py`, `yufmusicgen/rosa_cuda.py`).
 * Each declaration cites the reference interface it replaces (file:line).
 *
 * Conventions
 *   - Every int-returning call returns YUF_OK (0) or a negative yuf_status;
 *     yuf_last_error() then describes the failure (thread-local string).
 *     Nothing throws or aborts across the ABI.
 *   - "stream" arguments are hipStream_t passed as void* (NULL = the null
 *     stream).  Kernel-level calls are asynchronous on that stream.
 *   - Pointers documented as "device" must point to device memory; "host"
 *     buffers are caller-owned and only read/written during the call.
 *   - An engine is single-owner: calls on one engine must not overlap
 *     (like the reference `Model`, `vulkan/src/compute/model.rs:13-21`).
 */
#ifndef YUF_ENGINE_H
#define YUF_ENGINE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum {
    YUF_OK = 0,
    YUF_ERR_INVALID = -1,     /* bad argument / shape / unsupported size */
    YUF_ERR_IO = -2,          /* file could not be opened or read */
    YUF_ERR_FORMAT = -3,      /* malformed .yuf (magic, version, header, size) */
    YUF_ERR_HIP = -4,         /* a HIP runtime call failed */
    YUF_ERR_OOM = -5,         /* device or host allocation failed */
    YUF_ERR_RANGE = -6        /* index out of range (token id, stream slot) */
} yuf_status;

/* Last error message of the calling thread ("" if none). */
const char *yuf_last_error(void);
/* Library version string. */
const char *yuf_version(void);

/* ---------------------------------------------------------------------------
 * Kernel-level operators (device pointers, asynchronous on `stream`).
 * ------------------------------------------------------------------------- */

/*
 * WKV-7 forward scan over B x H independent N x N fp32 states.
 * Replaces `rwkv7_cuda(r, w, k, v, a, b)` (yufmusicgen/cuda_ops.py:256-266,
 * op `yufmusicgen_rwkv7::forward`, yufmusicgen/cuda/rwkv7_clampw.cpp:18-33)
 * and extends it with a non-zero initial state (the stateful path of
 * yufmusicgen/model.py:145-165).
 *   r, w_raw, k, v, a, b : device [B, T, H, N] fp32, contiguous.
 *   state_in             : device [B, H, N, N] (row i = value, col j = key) or
 *                          NULL for a zero initial state.
 *   state_out            : device [B, H, N, N] final state or NULL; may alias
 *                          state_in.
 *   y                    : device [B, T, H, N] output.
 * Per step: d = exp(-exp(-0.5) * sigmoid(w_raw)); sa = S a;
 *           S = S diag(d) + sa b^T + v k^T; y = S r.
 * Supported N: 8, 16, 32, 40, 48, 64, 128.  T >= 0 (any length, no padding).
 */
int yuf_wkv7_scan_f32(int B, int T, int H, int N,
                      const float *r, const float *w_raw, const float *k,
                      const float *v, const float *a, const float *b,
                      const float *state_in, float *state_out, float *y,
                      void *stream);

/*
 * ROSA Householder memory scan.
 * Replaces `rosa_householder_scan(cand, write, read_raw, decay, direction,
 * memory)` (yufmusicgen/rosa_cuda.py:157-180, op `yufmusicgen_rosa::forward`,
 * yufmusicgen/cuda/rosa_householder.cpp:24-50).
 *   cand, write          : device [B, T, D] pre-activations.
 *   read_raw             : device [B, T, D] read-gate pre-activation, or NULL.
 *   decay                : device [D], post-sigmoid lambda.
 *   direction            : device [D], unit Householder vector u.
 *   memory_in            : device [B, D] or NULL (zero).
 *   memory_out           : device [B, D] or NULL; may alias memory_in.
 *   read_out             : device [B, T, D].
 * m_t = lambda * H(m_{t-1}) + sigmoid(write_t) * tanh(cand_t), H(x) = x - 2(x.u)u;
 * read_t = H(m_t), times sigmoid(read_raw_t) when read_raw is not NULL
 * (the gated read of yufmusicgen/model.py:281-287).
 * Supported D: 1 .. 1024.
 */
int yuf_rosa_scan_f32(int B, int T, int D,
                      const float *cand, const float *write, const float *read_raw,
                      const float *decay, const float *direction,
                      const float *memory_in, float *memory_out, float *read_out,
                      void *stream);

/*
 * yuf_rosa_scan_f32 without any allocation: no hipMalloc, hipFree or other
 * allocating call.  No counterpart in the reference; for callers that cannot
 * allocate device memory (code under HIP graph capture, serving loops and
 * harnesses that forbid hipMalloc).  Same arguments, semantics and results.
 * The segmented form (T % 64 == 0, T >= 128, D in {64, 128, 256}) keeps its
 * scratch -- D * D + 2 * B * (T / 64) * D floats -- in a static 16 MiB device
 * array (4,194,304 floats) that every GPU the library runs on holds until the
 * process ends; larger calls fail with YUF_ERR_INVALID.  Other shapes use no
 * scratch.  All calls on one GPU share that array: calls that overlap on one
 * GPU (other streams, other host threads) race and must be ordered by the
 * caller.  The first call on a device resolves the array's address there
 * (hipGetSymbolAddress, not a stream operation).  YUF_ROSA_SEGMENTED does
 * not apply to this entry point: shapes that admit the segmented form always
 * take it, so the capacity check above runs before any launch.
 */
int yuf_rosa_scan_f32_noalloc(int B, int T, int D,
                              const float *cand, const float *write, const float *read_raw,
                              const float *decay, const float *direction,
                              const float *memory_in, float *memory_out, float *read_out,
                              void *stream);

/*
 * Linear layer on the matrix cores: C = act(A W^T + bias) + residual, fp32.
 * The projection primitive of every nn.Linear on the path
 * (yufmusicgen/model.py:107-112, :196, :306-342, :377, :421).
 *   A [M, K], W [N, K] (nn.Linear weight layout), C [M, N], all row-major,
 *   device pointers; bias [N] or NULL; residual [M, N] or NULL (may alias C);
 *   act: 0 none, 1 tanh, 2 sigmoid.
 */
int yuf_linear_f32(int M, int N, int K, const float *A, const float *W, const float *bias, int act,
                   const float *residual, float *C, void *stream);

/*
 * Pre-split weights for yuf_linear_f32 (no counterpart in the reference: a
 * one-time preparation of an nn.Linear weight, as the engine does for every
 * projection matrix at creation).  The large-tile products (M > 64, K % 32
 * == 0) run fp32 as six bf16 matrix-core products over three-part splits of
 * A and W; yuf_x3_split_planes stores W's three parts once, in the layout the
 * kernel streams into LDS directly, so products that pass them skip W's
 * split and stage both operands by direct memory -> LDS loads.
 *   yuf_x3_planes_elems: uint16 elements of the planes of an [N, K] W, 0
 *     unless N % 16 == 0 and K % 32 == 0.
 *   yuf_x3_split_planes: W [N, K] fp32 (16-byte aligned) -> planes (16-byte
 *     aligned device buffer of yuf_x3_planes_elems(N, K) elements), on
 *     `stream`.
 *   yuf_linear_f32_planes: yuf_linear_f32 with W's planes as well as W; the
 *     results are bit-identical to yuf_linear_f32's (the planes are used where
 *     the large-tile X3 path runs and A's rows are 16-byte aligned, W
 *     elsewhere).
 */
size_t yuf_x3_planes_elems(int N, int K);
int yuf_x3_split_planes(int N, int K, const float *W, uint16_t *planes, void *stream);
int yuf_linear_f32_planes(int M, int N, int K, const float *A, const float *W, const uint16_t *Wp,
                          const float *bias, int act, const float *residual, float *C, void *stream);

/*
 * LayerNorm -> (gate) -> Linear in one kernel, for short products (M <= 64, the
 * decode shapes): C = (LayerNorm(A) * gamma + beta) [* gate] W^T + bias + residual.
 * The norm -> projection pairs of a block: out_norm(y) * g -> output
 * (yufmusicgen/model.py:195-196), the ROSA and FFN pre-norms
 * (model.py:306, :377), the final norm -> LM head (model.py:390-391).
 * LayerNorm over the K columns of each A row, eps 1e-5 (torch.nn.LayerNorm).
 *   A [M, K], gate [M, K] or NULL, gamma / beta [K], W [N, K], C [M, N];
 *   bias [N] or NULL; residual [M, N] or NULL (may alias C).
 * Requires 1 <= M <= 64, K % 4 == 0, K <= 1024 (else YUF_ERR_INVALID).
 */
int yuf_ln_linear_f32(int M, int N, int K, const float *A, const float *gamma, const float *beta,
                      const float *gate, const float *W, const float *bias, const float *residual, float *C,
                      void *stream);

/*
 * bf16-weight forms of yuf_linear_f32 / yuf_ln_linear_f32 (the C5
 * configuration's weight type; no counterpart in the fp32 reference kernels,
 * they replace the same nn.Linear call sites).  W is [N, K] bf16 (raw 16-bit
 * patterns, uint16_t); A, bias, residual and C are fp32.  The result is the
 * fp32 product A x W up to accumulation order: each A value enters the bf16
 * matrix cores as two bf16 parts (hi = bf16(a), lo = bf16(a - hi), within
 * 2^-16 of a) and accumulation is fp32.
 * Needs K % 8 == 0; for M > 64, N % 64 == 0 or N % 160 == 0.
 */
int yuf_linear_bf16w(int M, int N, int K, const float *A, const uint16_t *W,
                     const float *bias, int act, const float *residual, float *C,
                     void *stream);
int yuf_ln_linear_bf16w(int M, int N, int K, const float *A, const float *gamma,
                        const float *beta, const float *gate, const uint16_t *W,
                        const float *bias, const float *residual, float *C,
                        void *stream);

/* ---------------------------------------------------------------------------
 * Checkpoints (.yuf).  Replaces `Checkpoint::load / tensor / tensor_dims`
 * (vulkan/src/checkpoint.rs:90-176).
 * ------------------------------------------------------------------------- */

typedef struct yuf_ckpt yuf_ckpt;

typedef struct {
    int32_t vocab_size;
    int32_t d_model;
    int32_t n_layers;
    int32_t n_heads;
    int32_t head_size;
    int32_t rosa_size;
    int32_t low_rank;       /* from the w1 tensor's shape, not a formula */
    int32_t tie_embeddings; /* 0 / 1 */
    float dropout;
    int32_t midi_offset;    /* header "midi.midi_offset" (260) */
    int32_t midi_vocab_size;
} yuf_model_config;

/* Load and validate a .yuf file (checkpoint.rs:90-149): magic "YUFM", a u32
 * version, a u64 header length, the UTF-8 JSON header, then the payload.
 * Version 1 is the reference's format (f32 payload whose size must equal
 * 4 * sum(count)); version 2 is this library's extension for bf16 weights
 * (per-tensor "dtype" and byte "offset", a "payload_bytes" the file size must
 * match; bf16 tensors are widened to f32 on load). */
int yuf_ckpt_load(const char *path, yuf_ckpt **out);
void yuf_ckpt_free(yuf_ckpt *ckpt);
int yuf_ckpt_config(const yuf_ckpt *ckpt, yuf_model_config *out);
/* The file's JSON header, verbatim (NUL-terminated; *len bytes without the
 * NUL), and its container version.  Replaces the reference's parsed
 * `checkpoint.header` (checkpoint.rs:60-81: format, model_config, midi{
 * tokenization, midi_offset, midi_vocab_size, vocab[], tokenizer_json},
 * source, lm_head_alias, tensors[]), which its generation loop reads to build
 * the codec and check the vocabulary (vulkan/src/generation.rs:102-117).
 * The pointer stays valid until yuf_ckpt_free.  len / version may be NULL. */
int yuf_ckpt_header_json(const yuf_ckpt *ckpt, const char **json, size_t *len, uint32_t *version);
/* Borrow a tensor by name (checkpoint.rs:151-176): host pointer valid until
 * yuf_ckpt_free; dims receives up to 8 sizes. */
int yuf_ckpt_tensor(const yuf_ckpt *ckpt, const char *name, const float **data,
                    int64_t *count, int32_t *ndim, int64_t dims[8]);

/* ---------------------------------------------------------------------------
 * Engine: device-resident weights and per-stream recurrent state.
 * Replaces `Model::new / step / reset_state` (vulkan/src/compute/model.rs:24-65),
 * batched over many streams and with a real prefill.
 * ------------------------------------------------------------------------- */

typedef struct yuf_engine yuf_engine;

enum { YUF_LOGITS_NONE = 0, YUF_LOGITS_LAST = 1, YUF_LOGITS_ALL = 2 };

/* Copy the checkpoint's weights to the device (the checkpoint may be freed
 * afterwards, like model.rs:24-51).  max_streams = state slots kept in HBM;
 * max_tokens = largest n * T processed per internal pass (longer prefills
 * are split into T-chunks that carry the state). */
int yuf_engine_create(const yuf_ckpt *ckpt, int max_streams, int max_tokens, yuf_engine **out);

/* Projection-weight type for yuf_engine_create_ex. */
enum { YUF_WEIGHTS_F32 = 0, YUF_WEIGHTS_BF16 = 1 };

/* yuf_engine_create with a projection-weight type (the `weight_dtype`
 * argument of the engine API; the C5 configuration runs bf16 weights with
 * fp32 WKV / ROSA state, yufmusicgen/config.py:73-93).  YUF_WEIGHTS_BF16 keeps
 * a bf16 copy (round to nearest even, or the file's own bf16 values) of every
 * nn.Linear weight and the tied LM head and runs the projections on the bf16
 * matrix cores with fp32-precision activations (see yuf_linear_bf16w): the
 * result is the fp32 model on bf16-valued weights.  Everything else
 * (LayerNorm, the WKV-7 and ROSA recurrences, state) is fp32.  Needs d_model,
 * the low-rank width and rosa_size to be multiples of 8, and the prefill GEMM
 * widths (d, low rank, 3 rosa_size, vocab) multiples of 64 or 160. */
int yuf_engine_create_ex(const yuf_ckpt *ckpt, int max_streams, int max_tokens, int weight_type,
                         yuf_engine **out);
void yuf_engine_destroy(yuf_engine *eng);
int yuf_engine_config(const yuf_engine *eng, yuf_model_config *out);
/* The HIP stream the engine runs its work on (hipStream_t as void*). */
void *yuf_engine_stream(yuf_engine *eng);

/* Batched prefill of n streams (slots[i] in [0, max_streams)), each by T
 * tokens, continuing from each stream's current state (the full-sequence
 * forward of yufmusicgen/model.py:406-422, replacing the reference engine's
 * per-token prefill loop, vulkan/src/generation.rs:176-185).
 *   slots  : host [n] int32
 *   tokens : host [n * T] int32 (row-major [n, T])
 *   logits : host output, [n, V] for LAST, [n, T, V] for ALL, ignored for NONE.
 * Synchronous. */
int yuf_prefill(yuf_engine *eng, int n, const int32_t *slots, int T,
                const int32_t *tokens, float *logits, int logits_mode);

/* Same with device-resident tokens and logits, asynchronous on the engine's
 * stream (slots stay host).  Use for throughput measurements.  Token ids are
 * read on the device: an id outside [0, vocab) embeds as zeros and sets the
 * engine's device-error flag, reported by yuf_engine_take_error (the host
 * entry points validate ids on the host and keep a flag of their own). */
int yuf_prefill_device(yuf_engine *eng, int n, const int32_t *slots, int T,
                       const int32_t *tokens_dev, float *logits_dev, int logits_mode);

/* One token for each of n streams; logits [n, V] (model.py:424-431;
 * Model::step, model.rs:54-60).  Host buffers, synchronous. */
int yuf_step(yuf_engine *eng, int n, const int32_t *slots, const int32_t *tokens, float *logits);

/* Same with device tokens / logits, asynchronous on the engine's stream.
 * The step is replayed from a captured HIP graph that reads tokens_dev and
 * writes logits_dev in place; the graph is captured again whenever n,
 * tokens_dev or logits_dev differ from the previous call, so a decode loop
 * should reuse one token buffer and one logits buffer.  tokens_dev must hold
 * its ids when the engine stream reaches the step (write it on that stream,
 * or synchronise first).  Out-of-range ids: see yuf_prefill_device. */
int yuf_step_device(yuf_engine *eng, int n, const int32_t *slots, const int32_t *tokens_dev,
                    float *logits_dev);

/* Synchronise the engine stream and report (then clear) the device-error flag
 * of the device entry points: YUF_ERR_RANGE if a yuf_prefill_device /
 * yuf_step_device call since the last check read a token id outside
 * [0, vocab) (its embedding row was zeroed), else YUF_OK.  No counterpart in
 * the reference, whose engine takes host token ids only (model.rs:54-60). */
int yuf_engine_take_error(yuf_engine *eng);

/*
 * Measurement hook (no reference counterpart): times the decode step's
 * first-layer WKV-7 step kernel -- the fused form with the second low-rank
 * stage, as the last decode step launched it (same inputs, streams and
 * launch shape) -- `iters` times, captured as one HIP graph and replayed on
 * the engine's stream between HIP events (the decode step is graph-replayed
 * too), writing the new state to a scratch buffer so the engine's state does
 * not change.  *avg_us receives the mean time per launch, the graph's
 * dispatch gap between kernels included; *streams (if not NULL) the number
 * of streams of that launch.  Needs a prior decode step with fp32 weights
 * and the fused low-rank step (else YUF_ERR_INVALID); allocates and frees
 * its scratch.
 */
int yuf_engine_time_wkv_step(yuf_engine *eng, int iters, float *avg_us, int *streams);

/* Zero all recurrent state of one slot (slot = -1: every slot), including
 * the token-shift `previous` vector the reference reset leaves stale
 * (Model::reset_state, model.rs:62-65). */
int yuf_state_reset(yuf_engine *eng, int slot);
/* Bytes of one stream's state blob: per layer [prev d | wkv H*N*N (i,j) | rosa D]
 * fp32, the order of BlockState (yufmusicgen/model.py:29-38). */
size_t yuf_state_size(const yuf_engine *eng);
int yuf_state_save(yuf_engine *eng, int slot, void *host_buf);
int yuf_state_load(yuf_engine *eng, int slot, const void *host_buf);

/* ---------------------------------------------------------------------------
 * Sampling.  Replaces `Mt19937` and `sample_token` / `argmax`
 * (vulkan/src/sampler.rs:22-82, :131-271) and Python `sample_token`
 * (yufmusicgen/cli/generate.py:45-56).
 * ------------------------------------------------------------------------- */

/* MT19937 state, caller-owned (the generator of torch.manual_seed). */
typedef struct {
    uint32_t mt[624];
    uint32_t index;
} yuf_rng;

void yuf_rng_seed(yuf_rng *rng, uint64_t seed);
uint32_t yuf_rng_next_u32(yuf_rng *rng);
/* 53-bit uniform in [0,1) from two words (hi << 32 | lo). */
double yuf_rng_next_uniform(yuf_rng *rng);

/* Host sampling over V logits following torch's CPU `sample_token` under the
 * same seed: temperature <= 0 -> argmax (first maximum); otherwise scale,
 * optional top_k (> 0: keep the k largest), sort descending, softmax, drop
 * where cumulative - p > top_p, renormalise, and torch.multinomial's
 * single-sample path argmax(p / q), q ~ Exp(1) -- V draws from the generator
 * per call, as torch consumes them.  The draws are bit-identical to torch's;
 * the softmax uses correctly rounded float exps and sums in the 16-lane order
 * of torch's AVX-512 kernel (the reference's Rust sampler assumes 8 lanes,
 * sampler.rs:145-170), so on hosts where torch dispatches another vector
 * width a token can differ from torch's only where two candidates tie to the
 * last bit.  Returns the token id, or a negative yuf_status. */
int32_t yuf_sample(const float *logits, int V, float temperature, float top_p, int top_k,
                   yuf_rng *rng);
/* First index of the maximum (torch.argmax semantics). */
int32_t yuf_argmax(const float *logits, int V);

/* The generation loop's logit mask (vulkan/src/generation.rs:195-203,
 * yufmusicgen/cli/generate.py:139-148): allowed_out[i] = logits[i] for MIDI
 * ids i >= midi_offset, -inf elsewhere; ids midi_offset + blocked_raw_ids[j]
 * are -inf; the EOS id keeps its logit once index >= min_before_eos (16 in
 * the reference).  allowed_out may alias logits.  Host buffers [V]. */
int yuf_generation_mask(const float *logits, int V, int index, int midi_offset, int eos_id,
                        int min_before_eos, const int32_t *blocked_raw_ids, int n_blocked,
                        float *allowed_out);

/* Device sampling for n streams at once (no logits copy to the host):
 * temperature <= 0 -> argmax; otherwise the top_k in [1, 64] largest scaled
 * logits (top_k 0 or >= V: all of them, V <= 24576), softmax over them and a
 * draw argmax p / q with q = -log u, u from a
 * counter-based generator keyed by (seed, counter, stream, token id) -- the
 * distribution of torch.multinomial, not its stream.  logits_dev [n, V];
 * tokens_dev [n] int32.  yuf_sample_device_masked(..., midi_offset = -1,
 * top_p = 1, exp_draws_dev = NULL, ...) with the same arguments. */
int yuf_sample_device(int n, int V, const float *logits_dev, float temperature, int top_k,
                      uint64_t seed, uint64_t counter, int32_t *tokens_dev, void *stream);

/* The generation loop's mask and sampler on the device, for n streams at once
 * (vulkan/src/generation.rs:195-203 then sampler.rs:131-256; Python
 * cli/generate.py:139-154): no logits copy, no host sort.
 *   mask: midi_offset >= 0 applies yuf_generation_mask's rule per stream --
 *     ids below midi_offset and midi_offset + blocked_raw_ids[j] are -inf, the
 *     EOS id keeps its logit once the stream's index >= min_before_eos; the
 *     index is index_dev[s] (device [n] int32) or, if index_dev is NULL, the
 *     host `index` for every stream.  blocked_raw_ids: host array, at most 256
 *     raw ids, each below 32768 and midi_offset + id < V.  midi_offset < 0: no
 *     mask.
 *   draw: temperature <= 0 -> the first maximum of the masked logits;
 *     otherwise top_k in [1, 64] (the k largest masked logits / temperature),
 *     or top_k = 0 (or >= V) for the whole vocabulary -- the reference's
 *     sampling, temperature 1 and top_p 0.95 with no top-k
 *     (cli/generate.py:39-56; vulkan/src/main.rs:78-82), for V <= 24576 --
 *     then top_p and the draw exactly as yuf_sample computes them.
 *     exp_draws_dev (device [n, top_k] float, or [n, V] when top_k = 0 or
 *     >= V) and first_zero_dev (device [n] int32; not read when top_k = 0 or
 *     >= V), filled from each stream's generator by yuf_rng_exp_draws(rng, V,
 *     k, ...) with k the number of draws per stream, make the token equal
 *     yuf_sample(masked logits, temperature, top_p, top_k, rng) for the same
 *     generator state; with exp_draws_dev NULL the counter-based draws of
 *     yuf_sample_device are used (first_zero_dev ignored).
 * Asynchronous on `stream`; tokens_dev [n] int32. */
int yuf_sample_device_masked(int n, int V, const float *logits_dev, float temperature, float top_p,
                             int top_k, int midi_offset, int eos_id, int min_before_eos, int index,
                             const int32_t *index_dev, const int32_t *blocked_raw_ids, int n_blocked,
                             const float *exp_draws_dev, const int32_t *first_zero_dev, uint64_t seed,
                             uint64_t counter, int32_t *tokens_dev, void *stream);

/* The generator draws one host sample consumes, for the device's exact mode:
 * takes V uniforms from `rng` (exactly what yuf_sample takes for V logits),
 * writes q_out[i] = (float)(-log1p(-u_i)) for the first k of them (k <= V),
 * and *first_zero = the first position i >= k whose uniform is 0 (its score
 * p / q would be NaN on the host), else -1.  first_zero may be NULL. */
int yuf_rng_exp_draws(yuf_rng *rng, int V, int k, float *q_out, int32_t *first_zero);

#ifdef __cplusplus
}
#endif

#endif /* YUF_ENGINE_H */
