/*
 * vxs_sampler.h — C ABI of the MI355X (gfx950) token sampler.
 *
 * One call turns each row of fp32 logits into a token id with the semantics of voxwerk's
 * Sampler (src/Voxwerk/Talker/Sampler.cs:1-96) plus the talker's suppression glue
 * (src/Voxwerk/Talker/TalkerGenerator.cs:246-249, :370-373):
 *   repetition penalty -> suppression -> (greedy argmax | temperature -> top-k -> softmax
 *   -> top-p -> inverse-CDF draw from a caller-supplied uniform).
 *
 * The reference is managed C# with no native boundary; these entry points are what its
 * P/Invoke layer binds (DllImport style of src/Voxwerk/Numerics/NativeBuffer.cs:78-92).
 * Plain pointers and sizes only. No C++ exceptions cross this boundary.
 *
 * Threading: one context owns one HIP stream and may be used by one thread at a time.
 * Separate contexts may run concurrently.
 */
#ifndef VXS_SAMPLER_H
#define VXS_SAMPLER_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#if defined(__GNUC__)
#define VXS_API __attribute__((visibility("default")))
#else
#define VXS_API
#endif

/* Return codes. A row that fails gets the code in its out_ids slot (all codes are < 0). */
#define VXS_OK 0
#define VXS_ERR_INVALID_ARG (-1)     /* bad pointer/shape/option (C#: ArgumentException family)          */
#define VXS_ERR_ID_OUT_OF_RANGE (-2) /* history id < 0 or >= vocab (C#: Span indexer at Sampler.cs:30)   */
#define VXS_ERR_NONFINITE (-3)       /* NaN or +inf logit after temperature: outside the contract        */
#define VXS_ERR_HIP (-4)             /* HIP runtime failure; text in vxs_last_error                      */
#define VXS_ERR_UNSUPPORTED (-5)     /* shape outside what the library implements; text in vxs_last_error */
#define VXS_ERR_NO_DEVICE (-6)       /* no usable gfx950 device                                          */
#define VXS_ERR_HISTORY_FULL (-7)    /* resident history slot already holds `cap` ids (vxs_sample_batch)  */

/* flags for vxs_sample / vxs_sample_device */
#define VXS_FLAG_NONE 0u
/* Kernel selection; without either flag the library chooses (one wave per row for batches of at
 * least 1024 rows with vocab <= 3072, else one workgroup per row). Results are identical. */
#define VXS_FLAG_PATH_BLOCK (1u << 8) /* one 256-thread workgroup per row                      */
#define VXS_FLAG_PATH_WAVE (1u << 9)  /* one wave per row first, 4 rows per workgroup (vocab <= 3072) */
/* vxs_sample_batch / vxs_sample_batch_device only: instead of reading `u` (which may be NULL),
 * each sampled row draws its uniform on the device from its slot's generator (vxs_history_seed):
 * the talker's new Random(Seed) or the code predictor's new Random(Seed + 1). A greedy row draws
 * nothing, as Select consumes no NextDouble when DoSample is false (Sampler.cs:37,77). */
#define VXS_FLAG_RNG_TALKER (1u << 10)
#define VXS_FLAG_RNG_SUB (1u << 11)

/*
 * Per-row sampling parameters (blittable; 36 bytes, 4-byte aligned).
 * Mirrors SamplingOptions (Sampler.cs:4-13), GenerationOptions.RepetitionPenalty
 * (TalkerGenerator.cs:11) and the talker's suppression rule (TalkerGenerator.cs:247-248).
 */
typedef struct vxs_params {
    int32_t do_sample;   /* SamplingOptions.DoSample; 0 = first-index argmax, no draw consumed      */
    int32_t top_k;       /* SamplingOptions.TopK; applied only when 0 < top_k < vocab               */
    float top_p;         /* SamplingOptions.TopP; applied only when top_p < 1                       */
    float temperature;   /* SamplingOptions.Temperature; logits are multiplied by fl32(1/T)         */
    float rep_penalty;   /* repetition penalty over the distinct history ids; 1 = off               */
    int32_t supp_begin;  /* ids in [supp_begin, supp_end) except keep_id are set to -inf            */
    int32_t supp_end;    /*   (talker: [vocab-1024, vocab) except EOS); empty range = off           */
    int32_t keep_id;     /* exempt from suppression (EOS); -1 = none                                */
    int32_t ban_id;      /* set to -inf after suppression (EOS while step < 2); -1 = none           */
} vxs_params;

typedef struct vxs_ctx vxs_ctx;

/*
 * Create a context on HIP device `device` (ordinal among visible devices). Capacities are
 * hints: buffers grow on demand and are freed by vxs_destroy.
 * Replaces: construction of Sampler (Sampler.cs:21) — the RNG stays with the caller, which
 * passes one NextDouble() per sampled row as `u`.
 */
VXS_API int vxs_create(vxs_ctx** out, int device, int max_rows, int max_vocab, int64_t max_hist);
VXS_API void vxs_destroy(vxs_ctx* ctx);

/* Text of the last error on this context ("" if none). Valid until the next call on ctx. */
VXS_API const char* vxs_last_error(const vxs_ctx* ctx);

/* Library version string, e.g. "vxs 0.1.0 gfx950". */
VXS_API const char* vxs_version(void);

/*
 * Use an external HIP stream (hipStream_t passed as void*) for all work of this context.
 * NULL restores the context's own stream. The caller keeps ownership of the stream.
 */
VXS_API int vxs_set_stream(vxs_ctx* ctx, void* hip_stream);
/* The hipStream_t (as void*) this context currently launches on. */
VXS_API void* vxs_get_stream(const vxs_ctx* ctx);

/*
 * Host-pointer sampling call; synchronous.
 * Replaces, for each row: Sampler.ApplyRepetitionPenalty (Sampler.cs:25-33), the suppression
 * loops (TalkerGenerator.cs:247-248, :371-372) and Sampler.Select (Sampler.cs:35-88) as
 * called at TalkerGenerator.cs:246-249, :268, :370-373, :419-420.
 *
 *   logits     [rows][ld] fp32, host memory; only the first `vocab` entries of a row are read
 *   hist_off   [rows+1] CSR offsets into hist_ids (hist_off[0] need not be 0); NULL = no history
 *   hist_ids   int32 generated-code history; duplicates allowed (applied once per distinct id)
 *   params     params[r * params_stride]; params_stride 0 broadcasts one struct to all rows
 *   u          [rows] uniforms in [0,1) (Random.NextDouble() per sampled row); may be NULL
 *              when no row samples
 *   out_ids    [rows] sampled ids; a failing row receives its negative error code
 *   out_logits NULL or [rows][vocab]: the row as Select leaves the caller's span (after
 *              penalty, suppression, temperature and the top-k -inf mask); may be `logits` itself
 *              when ld == vocab (in place); a row that fails keeps its contents
 *   out_probs  NULL or [rows][vocab] fp64: final probabilities the draw used (parity/debug)
 * Returns VXS_OK, or the first (lowest row) error code.
 */
VXS_API int vxs_sample(vxs_ctx* ctx, int rows, int vocab, const float* logits, int64_t ld,
                       const int32_t* hist_off, const int32_t* hist_ids,
                       const vxs_params* params, int params_stride, const double* u,
                       int32_t* out_ids, float* out_logits, double* out_probs, uint32_t flags);

/*
 * Device-pointer sampling call; asynchronous on the context stream. Every pointer is device
 * memory (params included). Per-row errors land in out_ids as negative codes; call
 * vxs_synchronize to wait. For callers whose logits are already resident on the GPU (logit
 * heads on device) and for kernel-only timing.
 */
VXS_API int vxs_sample_device(vxs_ctx* ctx, int rows, int vocab, const float* d_logits, int64_t ld,
                              const int32_t* d_hist_off, const int32_t* d_hist_ids,
                              const vxs_params* d_params, int params_stride, const double* d_u,
                              int32_t* d_out_ids, float* d_out_logits, double* d_out_probs,
                              uint32_t flags);

/*
 * vxs_sample for callers that cannot allocate (tight serving loops, harnesses that forbid hipMalloc):
 * no counterpart in the reference. Same arguments, semantics and errors as vxs_sample without the
 * write-back and probability outputs; synchronous. It allocates nothing: the inputs are copied from
 * the caller's memory into a fixed 16 MiB device scratch (one per GPU, held until the process ends),
 * the kernels read them there and write the ids there, and the ids are copied back. A call that
 * needs more than the scratch (about rows * vocab * 4 bytes plus the histories, params and
 * uniforms) fails with VXS_ERR_UNSUPPORTED. Every context on one GPU shares that GPU's scratch, so
 * the library serialises the calls on one GPU (from any threads or contexts) with a per-device lock
 * held for the whole call: concurrent calls wait for each other.
 */
VXS_API int vxs_sample_noalloc(vxs_ctx* ctx, int rows, int vocab, const float* logits, int64_t ld,
                               const int32_t* hist_off, const int32_t* hist_ids, const vxs_params* params,
                               int params_stride, const double* u, int32_t* out_ids, uint32_t flags);

/*
 * Parity/debug variant of vxs_sample_device (no counterpart in the reference): no write-back or
 * probabilities; instead, for every row sampled by the one-wave nucleus regime (sampled rows,
 * vocab <= 3072, whose top-k masks nothing and that keep more than 256 finite entries),
 *   d_stats[4r + 0] = kept fraction of the probability mass (after top-p; 1 without top-p),
 *   d_stats[4r + 1] = smallest kept probability (the top-p cut),
 *   d_stats[4r + 2] = number of kept entries (entries whose mass is 0 on the 2^-F grid excluded),
 *   d_stats[4r + 3] = 0,
 * so that the nucleus is checked beyond the id; all four are NaN for every other row (greedy,
 * exact regime, rows the one-workgroup algorithm samples). d_stats is [rows][4] fp64 device memory.
 * d_probs (optional, [rows][vocab] fp64 device memory): for the same rows, every entry's final
 * probability as the draw used it (its mass over the kept mass, 0 for removed entries); NaN for
 * every other row.
 */
VXS_API int vxs_sample_stats_device(vxs_ctx* ctx, int rows, int vocab, const float* d_logits, int64_t ld,
                                    const int32_t* d_hist_off, const int32_t* d_hist_ids,
                                    const vxs_params* d_params, int params_stride, const double* d_u,
                                    int32_t* d_out_ids, double* d_stats, double* d_probs, uint32_t flags);

/* Wait for all work queued on the context stream. */
VXS_API int vxs_synchronize(vxs_ctx* ctx);

/*
 * In-place repetition penalty on host rows (Sampler.ApplyRepetitionPenalty, Sampler.cs:25-33):
 * each distinct history id's logit s becomes s*penalty if s < 0, else s/penalty.
 * penalty == 1 is a no-op. Synchronous.
 */
VXS_API int vxs_apply_repetition_penalty(vxs_ctx* ctx, int rows, int vocab, float* logits, int64_t ld,
                                         const int32_t* hist_off, const int32_t* hist_ids,
                                         float penalty);

/* First index of the maximum of each host row (Sampler.ArgMax, Sampler.cs:90-95). Synchronous. */
VXS_API int vxs_argmax(vxs_ctx* ctx, int rows, int vocab, const float* logits, int64_t ld,
                       int32_t* out_ids);

/*
 * Resident histories for batched generation (TalkerGenerator.GenerateBatch,
 * TalkerGenerator.cs:322-455). A store holds `slots` sequence histories of at most `cap` ids each
 * in device memory of the context's device; one slot replaces one Active.History list
 * (TalkerGenerator.cs:304). The sampler reads a row's history from its slot and appends the id it
 * draws there (History.Add, TalkerGenerator.cs:374), so histories never cross PCIe per step.
 * A sequence appends one id per step and retires after MaxNewTokens steps (:375), so
 * cap = MaxNewTokens always suffices. slots * cap must not exceed 2^31 - 1. All slots start empty.
 */
typedef struct vxs_history vxs_history;
VXS_API int vxs_history_create(vxs_ctx* ctx, int slots, int cap, vxs_history** out);
/* Frees the store; no work that uses it may still be queued. */
VXS_API void vxs_history_destroy(vxs_history* h);
/* Replace slot `slot`'s history with ids[0..n) (0 <= n <= cap; n = 0 empties it, as a refilled
 * job starts with an empty History, TalkerGenerator.cs:336-349). Stream-ordered; synchronous. */
VXS_API int vxs_history_set(vxs_ctx* ctx, vxs_history* h, int slot, const int32_t* ids, int n);
/* Copy slot `slot`'s history into ids[0..max_ids) and its length into *n. Synchronous. */
VXS_API int vxs_history_get(vxs_ctx* ctx, vxs_history* h, int slot, int32_t* ids, int max_ids, int* n);
/* Seed slot `slot`'s two generators as a sequence's samplers are built (TalkerGenerator.cs:217-218,
 * :345-346): new Random(seed) for the talker, new Random(seed + 1) for the code predictor, with
 * .NET's seeded generator (Sampler.cs:21) and C#'s wrapping int arithmetic. A job without a seed
 * passes one of its own choosing. Synchronous. */
VXS_API int vxs_history_seed(vxs_ctx* ctx, vxs_history* h, int slot, int32_t seed);
/* The next n NextDouble() values (Sampler.cs:77) of slot `slot`'s talker (stream 0) or
 * code-predictor (stream 1) generator, drawn on the device into out[0..n). Synchronous. */
VXS_API int vxs_history_draw(vxs_ctx* ctx, vxs_history* h, int slot, int stream, int n, double* out);

/*
 * One batched sampling stage over host rows whose histories live in `h`: row r penalises with
 * slot slots[r]'s history, then (append != 0) its sampled id is appended to that slot.
 * Replaces the serial per-row loops of GenerateBatch: the talker stage (TalkerGenerator.cs:366-375:
 * ApplyRepetitionPenalty, suppression, a.Sampler.Select, History.Add; append = 1) and the
 * code-predictor stage (:419-420: SubSampler.Select, no penalty; pass rep_penalty 1 and append = 0).
 * Arguments as vxs_sample, with `slots` [rows] host memory: distinct slot indices in [0, slots of h).
 * A row that fails keeps its error code in out_ids and appends nothing; a full slot fails the row
 * with VXS_ERR_HISTORY_FULL. Synchronous.
 */
VXS_API int vxs_sample_batch(vxs_ctx* ctx, vxs_history* h, int rows, int vocab, const float* logits,
                             int64_t ld, const int32_t* slots, int append, const vxs_params* params,
                             int params_stride, const double* u, int32_t* out_ids, uint32_t flags);

/*
 * vxs_sample_batch with device pointers (logits, slots, params, u, out_ids); asynchronous on the
 * context stream like vxs_sample_device. A slot outside the store fails its row with
 * VXS_ERR_INVALID_ARG. Slots must be distinct within one call: the store stays in bounds if they
 * are not, but keeps only one of the ids appended to a repeated slot.
 */
VXS_API int vxs_sample_batch_device(vxs_ctx* ctx, vxs_history* h, int rows, int vocab,
                                    const float* d_logits, int64_t ld, const int32_t* d_slots,
                                    int append, const vxs_params* d_params, int params_stride,
                                    const double* d_u, int32_t* d_out_ids, uint32_t flags);

/*
 * Logit heads on the GPU, the step before the sampler: CodecHead and CodePredictorHead
 * (TalkerModel.cs:133-137, Gemm.Multiply over a bf16 PackedMatrix, WeightPrecision.BFloat16):
 *   out[r][j] = sum_k x[r][k] * W[j][k],   r < rows, j < n, k < k
 * x fp32 [rows][ldx], W bf16 [n][ldw] (the checkpoint's [out, in] layout: talker.codec_head.weight,
 * talker.code_predictor.lm_head.{g}.weight), out fp32 [rows][ldo], all device memory, so the
 * logits stay on the GPU for vxs_sample_device / vxs_sample_batch_device. fp32 products and sums
 * in an order of this library's own: each entry is within k * 2^-24 * sum_k |x w| of the exact
 * dot product, as the reference's is. Needs k <= 2048, k and ldw multiples of 8, ldx a multiple
 * of 4, 16-byte aligned x and W (else VXS_ERR_UNSUPPORTED). Asynchronous on the context stream.
 */
VXS_API int vxs_head_device(vxs_ctx* ctx, int rows, int k, int n, const float* d_x, int64_t ldx,
                            const uint16_t* d_w, int64_t ldw, float* d_out, int64_t ldo);

/*
 * The same heads with int8 weights (WeightPrecision.Int8, DecoderStack.cs:7-16; the reference packs
 * codec_head and every code_predictor.lm_head this way when asked, TalkerModel.cs:37,55):
 *   out[r][j] = scale[j] * sum_k x[r][k] * q[j][k]
 * the decode path's form (Gemm.cs:602-680: SmallM, PanelPairDotInt8 / PanelDotInt8, the scale
 * applied to the fp32 dot). q int8 [n][ldq], scale fp32 [n], as vxs_head_pack_int8_device writes
 * them. Each entry is within (k + 1) * 2^-24 * scale[j] * sum_k |x q| of the exact value, a bound
 * the reference's decode form and its batched form (Gemm.cs:95-98, which dequantizes q * scale
 * first) both satisfy. Needs k <= 2048, k and ldq multiples of 8, ldx a multiple of 4, 16-byte
 * aligned x and q (else VXS_ERR_UNSUPPORTED). Asynchronous on the context stream.
 */
VXS_API int vxs_head_int8_device(vxs_ctx* ctx, int rows, int k, int n, const float* d_x, int64_t ldx,
                                 const int8_t* d_q, int64_t ldq, const float* d_scale, float* d_out, int64_t ldo);

/*
 * int8 packing of a bf16 head weight on the GPU, PackedMatrix.FromBf16LinearInt8
 * (src/Voxwerk/Numerics/PackedMatrix.cs:124-154), bit for bit: per output row j, amax = max_k |W[j][k]|,
 * scale[j] = amax / 127 (1 when amax is 0), q[j][k] = clamp(round-half-even(W[j][k] * (1 / scale[j])),
 * -127, 127), in correctly rounded fp32, the (int) conversion saturating as in .NET 9 and later (a
 * row whose 1 / scale overflows gets +-127 and 0). W bf16 [n][ldw], q int8 [n][ldq], scale fp32 [n];
 * finite weights. Asynchronous on the context stream.
 */
VXS_API int vxs_head_pack_int8_device(vxs_ctx* ctx, int k, int n, const uint16_t* d_w, int64_t ldw, int8_t* d_q,
                                      int64_t ldq, float* d_scale);

/*
 * Embedding rows of sampled ids, the step after the sampler, so that ids need not return to the
 * host between sampling and the next forward pass. Tables are bf16 [vocab][hidden], widened to
 * fp32 exactly (Bf16.ToFloat, src/Voxwerk/Numerics/Bf16.cs:13); sums run in the reference's order,
 * so rows are bit-identical. Device pointers, asynchronous on the context stream. status[r] gets 0,
 * or VXS_ERR_ID_OUT_OF_RANGE for a row holding an id outside its table, which is then not written
 * (the reference throws ArgumentOutOfRangeException, TalkerModel.cs:102,109).
 *
 * vxs_embed_device replaces CodecEmbedding / CodePredictorEmbedding (TalkerModel.cs:100-111):
 * out[r] = table[ids[r]] (add = 0) or out[r] += table[ids[r]] (add = 1), as called at
 * TalkerGenerator.cs:258, :271, :411 and :422.
 */
VXS_API int vxs_embed_device(vxs_ctx* ctx, int rows, int hidden, const int32_t* d_ids, const uint16_t* d_table,
                             int vocab, float* d_out, int64_t ld_out, int add, int32_t* d_status);

/*
 * FrameEmbedding (TalkerModel.cs:113-117) for `rows` frames, plus the talker step's text row
 * (TalkerGenerator.cs:280-283, :435-439): out[r] = E0[codes[r][0]] + E1[codes[r][1]] + ... +
 * E_{groups-1}[codes[r][groups-1]] (+ addend[r] when d_addend is not NULL), left to right in fp32.
 * E0 = d_codec_table [vocab][hidden]; E_g = d_cp_tables + (g-1) * cp_vocab * hidden, g >= 1, the
 * code predictor's tables stored back to back. Code g of frame r is d_codes[r * ld_codes +
 * g * group_stride]: a [rows][groups] matrix has ld_codes = groups, group_stride = 1; the ids of one
 * sampling call per codebook, stage g at d_codes + g * rows, have ld_codes = 1, group_stride = rows.
 */
VXS_API int vxs_frame_embed_device(vxs_ctx* ctx, int rows, int groups, int hidden, const int32_t* d_codes,
                                   int64_t ld_codes, int64_t group_stride, const uint16_t* d_codec_table, int vocab,
                                   const uint16_t* d_cp_tables, int cp_vocab, const float* d_addend,
                                   int64_t ld_addend, float* d_out, int64_t ld_out, int32_t* d_status);

#ifdef __cplusplus
}
#endif

#endif /* VXS_SAMPLER_H */
