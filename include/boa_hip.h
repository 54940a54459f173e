/*
 * boa_hip.h -- C ABI of libboa_hip.so, the MI355X (gfx950) implementation of BoaConstrictor's batched
 * compress/decompress hot path.
 *
 * Conventions
 *   - Every entry point returns an int status: BOA_OK (0) or a BOA_ERR_* code; boa_last_error() returns a
 *     thread-local message for the last failure on the calling thread.
 *   - Pointers named d_* are device pointers (HBM of the current HIP device); h_* are host pointers.
 *   - Every call is asynchronous on the stream it is given (or the context's stream) unless it says that it
 *     synchronizes.  A context is not re-entrant: one context per stream, one call at a time.
 *   - No torch or C++ types cross this boundary.
 *
 * Each declaration names the reference interface it replaces (paths into the reference checkout).
 */
#ifndef BOA_HIP_H
#define BOA_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define BOA_OK 0
#define BOA_ERR_ARG 1       /* invalid argument (shape, size, null pointer)                        */
#define BOA_ERR_HIP 2       /* a HIP runtime call failed                                            */
#define BOA_ERR_OVERFLOW 3  /* an output buffer (stream pitch, payload capacity) is too small      */
#define BOA_ERR_STATE 4     /* call out of order (e.g. decode before init)                          */

/* Library identity and last error (replaces the reference's exit(1) on CUDA errors, gemm_gpu.hpp:36-43). */
const char* boa_last_error(void);
int boa_abi_version(void);  /* 2 (boa_decompress takes the payload length since version 2) */
/* Reports whether d_ptr is device memory of the HIP runtime this library is bound to (1 yes, 0 no). */
int boa_is_device_pointer(const void* d_ptr);

/* ------------------------------------------------------------------------------------------------ */
/* Model configuration: MambaConfig, gemm_gpu.hpp:9-34 (use_rmsnorm is always off: the model uses
 * LayerNorm, model.py:45,51). dt_rank 0 means ceil(d_model/16); d_inner = expand * d_model.            */
typedef struct boa_model_cfg {
    int32_t d_model;
    int32_t n_layers;
    int32_t vocab;      /* <= 256 */
    int32_t d_state;    /* 16 */
    int32_t d_conv;     /* 4 */
    int32_t expand;     /* 2 */
    int32_t dt_rank;    /* 0 = ceil(d_model / 16) */
} boa_model_cfg;

/* GEMM arithmetic of a context.  The weight blob passed in is always float32
 * (convert_boa_weights.py:22-133 order).
 *   BOA_PREC_F32     fp32 MFMA (v_mfma_f32_16x16x4_f32).
 *   BOA_PREC_BF16X3  activations and weights each split into two bfloat16 parts; three bf16 MFMA products
 *                    (lo*hi + hi*lo + hi*hi) accumulated in fp32.
 *   BOA_PREC_BF16W   GEMM weight matrices rounded to bfloat16 (bf16-weight models); activations split as
 *                    above; two products.
 * Encoder and decoder must use the same mode: the logits (and so the streams) depend on it.              */
#define BOA_PREC_F32 0
#define BOA_PREC_BF16X3 1
#define BOA_PREC_BF16W 2

typedef struct boa_ctx boa_ctx;

/* Size in bytes of the flat float32 weight blob for cfg (convert_boa_weights.py:22-133 order). */
int64_t boa_weights_nbytes(const boa_model_cfg* cfg);

/* Creates a model context: uploads the weights (host float32 blob) and allocates the recurrent state and
 * workspace for up to max_lanes chunks processed tile_len (1..256) positions at a time.  precision is a
 * BOA_PREC_* mode; stream may be NULL.  Replaces BoaPredictorGPU's constructor + load_weights
 * (boa_gpu.hpp:489-555) and the nvcc-at-import RangeCoderBatch holder's allocations
 * (gpu_range_coder.py:212-236).                                                                        */
int boa_ctx_create(const boa_model_cfg* cfg, const void* h_weights_f32, int64_t nbytes, int precision,
                   int32_t max_lanes, int32_t tile_len, void* stream, boa_ctx** out);
int boa_ctx_destroy(boa_ctx* ctx);
/* Bytes of device memory the context holds. */
int64_t boa_ctx_device_bytes(const boa_ctx* ctx);
/* Bytes of device memory boa_ctx_create would allocate for this shape (exact: creation checks its total
 * against it).  For sizing waves of chunks from free device memory.  Replaces
 * BoaPredictorGPU::estimate_memory_static (boa_gpu.hpp:625-662) as used by auto_size_params
 * (boa.cpp:103-150).                                                                                  */
int boa_ctx_plan_bytes(const boa_model_cfg* cfg, int precision, int32_t max_lanes, int32_t tile_len,
                       int64_t* out_bytes);

/* Zeroes the conv and SSM state of lanes [0, lanes) (MambaBlockGPU::reset_cache, boa_gpu.hpp:220-223;
 * model.py:68-73 zero initial cache).                                                                  */
int boa_state_reset(boa_ctx* ctx, int32_t lanes);

/* One recurrent step for `lanes` chunks: d_tokens int32 [lanes] -> d_logits float32 [lanes][vocab].
 * Advances the state.  Replaces BoaBytePredictor.step (model.py:109-117 / 124-131) and
 * BoaPredictorGPU::step_batch (boa_gpu.hpp:560-578).                                                   */
int boa_model_step(boa_ctx* ctx, const int32_t* d_tokens, int32_t lanes, float* d_logits);

/* Teacher-forced forward from the current state: d_tokens int32 [lanes][len] (row stride tok_stride)
 * -> d_logits float32 [lanes][len][vocab].  Advances the state by len positions.  Replaces
 * BoaBytePredictor.forward (model.py:97-101) and BoaPredictorGPU::forward_chunk (boa_gpu.hpp:606-624). */
int boa_model_forward(boa_ctx* ctx, const int32_t* d_tokens, int64_t tok_stride, int32_t lanes,
                      int32_t len, float* d_logits);

/* Opt-in per-kernel-class timing with HIP events recorded on the context's stream around each launch
 * (first BOA_PROF_SAMPLES launches of each class per profiling window).  No reference counterpart: it
 * replaces the reference's cudaEvent forward/encode split (boa.cpp:366-380) for measurement.            */
#define BOA_PROF_SAMPLES 4096
typedef struct boa_prof_entry {
    char name[32];        /* kernel class, e.g. "gemm_ff1"                                          */
    int64_t launches;     /* launches in the window                                                 */
    int64_t sampled;      /* launches that were timed                                               */
    double ms;            /* summed duration of the timed launches                                  */
    double flops;         /* algorithmic flops of the timed launches                                */
    double bytes;         /* algorithmic HBM bytes of the timed launches                            */
} boa_prof_entry;
/* enable != 0 starts a fresh window; 0 stops recording. */
int boa_profile(boa_ctx* ctx, int enable);
/* Synchronizes, resolves the recorded events and copies up to cap entries; *n receives the count.      */
int boa_profile_read(boa_ctx* ctx, boa_prof_entry* out, int32_t cap, int32_t* n);

/* ------------------------------------------------------------------------------------------------ */
/* Fused batched compress: chunk i is d_bytes[i*byte_stride .. +d_lens[i]).  Byte 0 of each chunk is not
 * coded (stored raw by the caller, codec.py:38); bytes 1..len-1 are range coded (PRECISION 24) under the
 * fused quantiser from the model's logits.  Output: d_words [lanes][pitch_words] and d_nwords[lanes].
 * Runs the model parallel in time, tile_len positions per launch sequence.  Fails with BOA_ERR_OVERFLOW
 * if a stream exceeds pitch_words (pitch_words >= max_len + 8 always suffices).
 * Replaces codec.compress_GPU (codec.py:11-86) and compress_v2's GPU section (boa.cpp:333-398).        */
int boa_compress(boa_ctx* ctx, const uint8_t* d_bytes, int64_t byte_stride, const int32_t* d_lens,
                 int32_t lanes, int32_t max_len, uint32_t* d_words, int64_t pitch_words,
                 int32_t* d_nwords);

/* Fused batched decompress of boa_compress output held contiguously: stream i is
 * d_payload[d_word_off[i] .. + d_nwords[i]), clamped to the payload's payload_words words (offsets or
 * counts past the payload read zeros, as reads past a stream's end do; nothing outside the payload is
 * read: the bound decompress_v2 checks on the host, boa.cpp:240).  d_first[i] is chunk i's raw first
 * byte.  Writes d_out[i*out_stride + t] for t < d_lens[i].  Strictly sequential per chunk: one model
 * step per byte.  Replaces codec.decompress_GPU (codec.py:89-151) and decompress_v2's GPU loop
 * (boa.cpp:535-574).                                                                                    */
int boa_decompress(boa_ctx* ctx, const uint32_t* d_payload, int64_t payload_words, const int64_t* d_word_off,
                   const int32_t* d_nwords, const uint8_t* d_first, const int32_t* d_lens, int32_t lanes,
                   int32_t max_len, uint8_t* d_out, int64_t out_stride);

/* Fused quantiser tables for parity tests: d_logits float32 [rows][vocab] -> d_cdf uint32
 * [rows][vocab+1] at `precision` bits.  No reference counterpart (the reference quantisers are Q2,
 * gpu_range_coder.py:57-79, and the warp-scan one in range_coder_kernels.cu:640-702).                  */
int boa_xq_cdf(const float* d_logits, int64_t rows, int32_t vocab, int32_t precision, uint32_t* d_cdf,
               void* stream);

/* Bitstream compaction: exclusive prefix sum of d_nwords into d_word_off (int64 [lanes]) and a gather of
 * each lane's words from the pitched buffer into the contiguous d_payload (capacity payload_cap words).
 * Every d_nwords[i] must lie in [0, pitch_words]: otherwise BOA_ERR_ARG, with nothing gathered (the check
 * runs on the device, in the scan).
 * *h_total_words receives the total; this call synchronizes the stream.  The scan's partial sums live in a
 * buffer the library allocates on the first call per device and stream (and enlarges for a larger wave).
 * Replaces the per-lane D2H copy of the full pitch (gpu_range_coder.py:278-292; boa.cpp:388-395).      */
int boa_compact(const uint32_t* d_words, int64_t pitch_words, const int32_t* d_nwords, int32_t lanes,
                int64_t* d_word_off, uint32_t* d_payload, int64_t payload_cap, int64_t* h_total_words,
                void* stream);

/* boa_compact without any device allocation: the same scan and gather, with the scan's partial sums in a
 * fixed array in the library's device memory (one copy per GPU, held until the process ends) instead of a
 * buffer the library allocates.  lanes <= 262144 (BOA_COMPACT_NOALLOC_MAX_LANES), else BOA_ERR_ARG.  Calls
 * that overlap on one GPU share that array and race: issue them one at a time per GPU.  Call it with the
 * stream's device current.  No counterpart in the reference: it is for callers that cannot allocate
 * device memory (code under HIP graph capture, serving loops, harnesses that forbid hipMalloc).          */
#define BOA_COMPACT_NOALLOC_MAX_LANES 262144
int boa_compact_noalloc(const uint32_t* d_words, int64_t pitch_words, const int32_t* d_nwords, int32_t lanes,
                        int64_t* d_word_off, uint32_t* d_payload, int64_t payload_cap, int64_t* h_total_words,
                        void* stream);

/* ------------------------------------------------------------------------------------------------ */
/* Range coder on precomputed CDF tables (the configs' "range coder alone" case).  d_cdf holds
 * [streams][len][K] entries of cdf_bytes (2 or 4) each: cdf[0..K-1] of each step, cdf[K] = 2^precision
 * implied.  d_syms uint8 [streams][len].  precision is 16 or 24.  Integer core identical to
 * gpu_range_coder.py:88-210 (encode_kernel, finalize_kernel, init_dec_kernel, decode_step_kernel).     */
int rc_encode_tables(int32_t precision, int32_t cdf_bytes, const void* d_cdf, int32_t K,
                     const uint8_t* d_syms, int32_t streams, int32_t len, uint32_t* d_words,
                     int64_t pitch_words, int32_t* d_nwords, void* stream);
int rc_decode_tables(int32_t precision, int32_t cdf_bytes, const void* d_cdf, int32_t K,
                     const uint32_t* d_words, int64_t pitch_words, const int32_t* d_nwords,
                     int32_t streams, int32_t len, uint8_t* d_syms, void* stream);
/* Synthetic tables for the range-coder-alone workload: per (stream, step) logits ~ N(0, sigma^2) from a
 * counter-based generator keyed by (seed, stream, step), quantised with the fused quantiser at
 * `precision`, and a symbol drawn by inverse CDF from a uniform integer in [0, 2^precision).           */
int rc_synth_tables(uint64_t seed, float sigma, int32_t precision, int32_t cdf_bytes, int32_t K,
                    int32_t streams, int32_t len, void* d_cdf, uint8_t* d_syms, void* stream);

/* ------------------------------------------------------------------------------------------------ */
/* Per-step batch coder with the reference's Q2 quantiser from probabilities (PRECISION 24):
 * gpu.queue.RangeCoderBatch and its pybind holder (gpu_range_coder.py:212-324, 488-550).               */
typedef struct rcb rcb;
int rcb_create(int32_t n, int32_t k, int64_t pitch_words, void* stream, rcb** out);   /* RangeCoderBatch(N,K,pitch) */
int rcb_destroy(rcb* b);
/* encode_step_from_device (gpu_range_coder.py:265-272): d_syms int32 [n], d_probs float32 [n][k],
 * d_mask uint8 [n] or NULL.  Lanes with mask 0 or a symbol outside [0, k) are skipped.                 */
int rcb_encode_step(rcb* b, const int32_t* d_syms, const float* d_probs, const uint8_t* d_mask);
int rcb_finalize(rcb* b);                                                            /* :273-276 */
int rcb_get_sizes(rcb* b, int32_t* h_sizes);                                         /* :293-297 */
/* Compacted copy of all streams to the host: h_words receives sum(sizes) words, lane after lane.       */
int rcb_get_words(rcb* b, uint32_t* h_words, int64_t cap_words, int64_t* h_total);   /* :278-292 */
/* load_compressed_from_host (:237-253): h_words holds the streams back to back, h_sizes their lengths. */
int rcb_load(rcb* b, const uint32_t* h_words, const int32_t* h_sizes);
int rcb_init_decoder(rcb* b);                                                        /* :293-297 */
int rcb_decode_step(rcb* b, const float* d_probs, int32_t* d_out_syms, const uint8_t* d_mask); /* :298-305 */

#ifdef __cplusplus
}
#endif
#endif /* BOA_HIP_H */
