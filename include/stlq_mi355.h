/*
 * stlq_mi355 — MI355X (gfx950) multi-codebook beam-search encoder, C ABI.
 *
 * Drop-in device implementation of STLQ's basic-encode stage (float vectors -> m codes per
 * vector by prefix-least-squares beam search, optional ICM sweeps). Each entry point names the
 * reference routine it replaces (paths relative to the ighxiy/STLQ tree).
 *
 * Conventions
 *  - Matrices use the reference's column-major ColMajorMatrix layout
 *    (include/stlq/common/types.h:35-51): X is d x n (vector i at X + i*d), C_all is d x H
 *    (codeword f at C_all + f*d), G is H x H (G(row,col) at G[col*H + row]), xC is H x n,
 *    codes is m x n uint8 (vector i at codes + i*m), coefficients a are m x n float.
 *  - Host pointers unless the entry point says "device". The caller owns every host buffer;
 *    the context owns every device buffer.
 *  - Every call returns STLQ_MI355_OK (0) or an error code; stlq_mi355_last_error() returns a
 *    thread-local message for the last failure. No exception crosses the ABI.
 *  - One context per host thread (a context is not thread-safe). Calls on one context are
 *    serialised on its own HIP stream; host-pointer calls return after the results are copied.
 *  - Strict arithmetic: the candidate-cost math, LS solves and costs run in fp32 with no FMA
 *    contraction and IEEE division/sqrt, in the reference's operation order; G and ||x||^2 are
 *    sequential fp32 sums; xC = C_all^T X runs on fp32 MFMA.
 */
#ifndef STLQ_MI355_H_
#define STLQ_MI355_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define STLQ_MI355_OK 0
#define STLQ_MI355_ERR_INVALID 1     /* bad argument or shape */
#define STLQ_MI355_ERR_HIP 2         /* HIP runtime failure */
#define STLQ_MI355_ERR_STATE 3       /* call order (e.g. no codebooks set) */
#define STLQ_MI355_ERR_UNSUPPORTED 4 /* outside the supported envelope */
#define STLQ_MI355_ERR_CALLBACK 5    /* a streaming callback returned non-zero */

/* Supported envelope: m <= 20 (include/stlq/core/model_limits.h:5), every layer's codebook
 * size <= 256 (uint8 codes; include/stlq/common/types.h:20-32) except the large-root layer 0,
 * 1 <= H_beam <= 64. */
#define STLQ_MI355_MAX_M 20
#define STLQ_MI355_MAX_K 256
#define STLQ_MI355_MAX_BEAM 64

typedef struct stlq_mi355_ctx stlq_mi355_ctx;

/* Encoder knobs of base.encode.* (include/stlq/common/config.h:473-482). */
typedef struct stlq_mi355_encode_params {
    int H_beam;      /* beam width; values < 1 are treated as 1 (encoder_encode_base.inc:39) */
    int icm_iters;   /* ICM sweeps after the beam (0 = none) */
    int ils_iters;   /* ILS rounds after the ICM (0 = none; icm.cpp:944-1001) */
    int perturb_k;   /* codes perturbed per vector and ILS round (min(perturb_k, m)) */
    int use_abs;     /* |score| in the ICM code pick (DynamicIcmWithIlsAbsNoNormal) */
    uint32_t seed;   /* ICM layer-order seed (std::mt19937) and ILS perturbation seed */
    int want_coeffs; /* also produce LS coefficients a and per-vector cost */
} stlq_mi355_encode_params;

/* Per-call device timings in milliseconds (HIP events on the context stream). */
typedef struct stlq_mi355_timings {
    double xnorm_ms;
    double gemm_ms;   /* xC = C_all^T X (fp32 MFMA) */
    double beam_ms;   /* all beam layers */
    double ls_ms;     /* LS refit + costs */
    double icm_ms;    /* ICM and ILS */
    double total_ms;
    int64_t n;
    int gemm_launches;
    int beam_launches;
    double layer_ms[STLQ_MI355_MAX_M]; /* beam layer l (one launch per tile) */
    int64_t beam_reruns; /* vectors the full-precomp beam re-ran in the reference's slot order
                            (ties the best-first pass cannot settle); included in beam_ms */
} stlq_mi355_timings;

const char* stlq_mi355_last_error(void);

/* Library/version string (ABI guard for loaders). */
const char* stlq_mi355_version(void);

/* Replaces the CudaStreamKernels / beam-session construction of PrepareKernelRuntimeStage
 * (src/pipeline/stlq_entry_stages.cpp:57-75). device: HIP ordinal. */
int stlq_mi355_ctx_create(int device, stlq_mi355_ctx** out);
int stlq_mi355_ctx_destroy(stlq_mi355_ctx* ctx);

/* BuildPrecomp (src/quantizer/encoder_precomp.inc:1-53): uploads C_all (d x H), computes on the
 * device G = C_all^T C_all (sequential fp32 dot products, exactly symmetric) and
 * invnorm[f] = 1/sqrt(||c_f||^2) (0 for a zero codeword). h_vec[l] <= 256 for every layer. */
int stlq_mi355_set_codebooks(stlq_mi355_ctx* ctx, int d, int m, const int* h_vec,
                             const float* C_all);

/* Same as above with a caller-built Precomp (include/stlq/common/types.h:62-75): G is the
 * reference's column-major H x H Gram, invnorm the H-vector invnorm_flat. G need not be
 * symmetric; every read uses the reference's (row, col) element. */
int stlq_mi355_set_precomp(stlq_mi355_ctx* ctx, int d, int m, const int* h_vec,
                           const float* C_all, const float* G, const float* invnorm);

/* Copies the device precomp back (G column-major H x H, invnorm H). Either may be NULL. */
int stlq_mi355_get_precomp(stlq_mi355_ctx* ctx, float* G, float* invnorm);

/* ComputeXNorm2 (src/quantizer/cost_utils.cpp:88-110, cost_utils.h:12) in the reference build's
 * omp-simd order. X is d x n; no codebooks are needed. */
int stlq_mi355_xnorm2(stlq_mi355_ctx* ctx, const float* X, int d, int64_t n, float* out);

/* StreamKernelProvider::Gemm(true,false,C_all,X) (include/stlq/core/kernel_provider.h:54-77,
 * call site encoder_encode_base.inc:86-90): xC = C_all^T X on fp32 MFMA. */
int stlq_mi355_gemm_xc(stlq_mi355_ctx* ctx, const float* X, int64_t n, float* xC);

/* BeamSearchPrefixLS (src/quantizer/beam_search.cpp:196-422,
 * include/stlq/quantizer/beam_search.h:18-22): the caller supplies xC (H x n) as the reference
 * does. nx2 may be NULL (then ||x||^2 is computed from X); when nx2 is given X may be NULL.
 * best_err (n floats, nullable) receives the selected beam's error. */
int stlq_mi355_beam_search(stlq_mi355_ctx* ctx, const float* X, const float* nx2,
                           const float* xC, int64_t n, int H_beam, uint8_t* codes,
                           float* best_err);

/* SolveLeastSquaresAll (src/quantizer/least_squares.cpp:406-565). fail_count nullable. */
int stlq_mi355_solve_ls_all(stlq_mi355_ctx* ctx, const float* xC, const uint8_t* codes,
                            int64_t n, float* a, int64_t* fail_count);

/* ComputeCosts (src/quantizer/cost_utils.cpp:139-158). */
int stlq_mi355_compute_costs(stlq_mi355_ctx* ctx, const float* xC, const uint8_t* codes,
                             const float* a, const float* nx2, int64_t n, float* cost);

/* DynamicIcmWithIls{Abs,NoAbs}NoNormal with ils_iters = 0 (src/quantizer/icm.cpp:872-899,
 * 1132-1170; include/stlq/quantizer/icm.h:15-43): LS refit + costs, then icm_iters sweeps
 * (RunIcm, icm.cpp:89-344). codes is updated in place; a (m x n) and cost (n) are outputs.
 * nx2 nullable (computed from X). */
int stlq_mi355_icm(stlq_mi355_ctx* ctx, const float* X, const float* nx2, const float* xC,
                   int64_t n, int icm_iters, int use_abs, uint32_t seed, uint8_t* codes,
                   float* a, float* cost);

/* DynamicIcmWithIls{Abs,NoAbs}NoNormal with the ILS outer loop (src/quantizer/icm.cpp:872-1003;
 * include/stlq/quantizer/icm.h:15-43, the sample_id_offset argument): the ICM above, then
 * ils_iters rounds of perturbing min(perturb_k, m) codes of layers 1..m-1 per vector (SplitMix64
 * stream keyed by seed, round and sample_id_offset + i), ICM on the perturbed codes and
 * accept-if-better (cand + 1e-6 < cost). ils_iters = 0 or perturb_k = 0 or m = 1 is the ICM. */
int stlq_mi355_icm_ils(stlq_mi355_ctx* ctx, const float* X, const float* nx2, const float* xC,
                       int64_t n, int icm_iters, int ils_iters, int perturb_k, int use_abs,
                       uint32_t seed, uint64_t sample_id_offset, uint8_t* codes, float* a,
                       float* cost);

/* EncodeBase (src/quantizer/encoder_encode_base.inc:1-106, include/stlq/quantizer/encoder.h:
 * 66-74) without the ILS outer loop: xC GEMM, beam, [ICM], [LS refit + costs], all on the
 * device. a/cost are written when params->want_coeffs (or icm_iters > 0) and non-NULL.
 * beam_mse/final_mse (nullable) receive the means of the per-vector costs before and after ICM
 * (MeanMseFromPrecomp semantics, double accumulation). */
int stlq_mi355_encode(stlq_mi355_ctx* ctx, const float* X, int64_t n,
                      const stlq_mi355_encode_params* params, uint8_t* codes, float* a,
                      float* cost, double* beam_mse, double* final_mse);

/* Device-pointer variant of stlq_mi355_encode on the caller's HIP stream (hipStream_t passed as
 * void*; NULL = the context stream). Inputs and outputs are device pointers; the call is
 * asynchronous with respect to the host. */
int stlq_mi355_encode_device(stlq_mi355_ctx* ctx, const float* dX, int64_t n,
                             const stlq_mi355_encode_params* params, uint8_t* dcodes,
                             float* da, float* dcost, void* stream);

/* No counterpart in the reference. For callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc): the same encode as
 * stlq_mi355_encode_device (same arguments, same results bit for bit), with every work buffer
 * (||x||^2, xC, beam records, best-first flags and counters, LS/ICM/ILS state) taken from a
 * 256 MiB static device array held by each device for the life of the process. The call
 * allocates no device or pinned memory and records no events (stlq_mi355_last_timings then
 * reports nothing). n must fit that scratch in one tile: about 16k vectors at d=128, M=8,
 * K=256, beam 16; a larger n fails with STLQ_MI355_ERR_UNSUPPORTED and a message naming the
 * capacity for the shape. Every call on a device shares that device's scratch, so calls that
 * overlap in time on one device (two contexts, two streams, two threads) race; calls that are
 * ordered on one stream are safe. */
int stlq_mi355_encode_device_noalloc(stlq_mi355_ctx* ctx, const float* dX, int64_t n,
                                     const stlq_mi355_encode_params* params, uint8_t* dcodes,
                                     float* da, float* dcost, void* stream);

/* Streaming encode (EncodeBaseStreaming / EncodeBaseStreamingF32,
 * src/quantizer/encode_base_streaming.cpp:1913 and :4544-4579, tile loop :2534-2620): vectors
 * are produced by `fill` into pinned host chunks of `chunk` vectors, copied to the device
 * through two buffers on a copy stream (double-buffered hipMemcpyAsync) while the previous chunk
 * encodes on the context stream, and the results are handed to `sink` in chunk order.
 *  input_u8: fill writes uint8 vectors (d bytes each) that the device widens to fp32
 *            (ConvertU8ToF32AndRotatePtr, kernel_provider_cuda_stream_impl.inc:3730+);
 *            otherwise fp32 (d floats each).
 *  R:        d x d column-major rotation applied to every vector before the encode, Xblk = R X
 *            (encode_base_streaming.cpp:817-833, :1367-1390), on fp32 MFMA; NULL for R = I.
 *  large_root: encode with the large-root codebooks (stlq_mi355_set_large_root): the beam of
 *            BeamSearchPrefixLSLargeRoot with root_mode 0 (top-H_beam roots) or 1 (nearest
 *            root); the chunk output then carries cluster_id, B_small and best_err, and, when
 *            encode asks for coefficients or ICM/ILS, a and cost from the large-root refit
 *            (SolveLeastSquaresAllLargeRoot + ComputeCostsLargeRoot, or
 *            DynamicIcmWithIls*NoNormalLargeRoot; encode_base_streaming.cpp:1117-1210).
 *            Otherwise the full-precomp EncodeBase of `encode` (codes, and a/cost when wanted).
 * fill/sink return 0 on success. */
typedef struct stlq_mi355_stream_params {
    stlq_mi355_encode_params encode;
    int input_u8;
    int large_root;
    int root_mode;
    const float* R;
    /* Global id of the first streamed vector (EncodeBaseStreaming's start_id,
     * encode_base_streaming.cpp:1913-1936): the stream covers ids start_id .. start_id + n_total - 1,
     * fill and sink receive global ids, and the ILS perturbations are keyed by them
     * (sample_id_offset = res.start + t0, :874). A resumed stream reproduces the whole one. */
    uint64_t start_id;
} stlq_mi355_stream_params;

typedef struct stlq_mi355_chunk_out {
    const uint8_t* codes;       /* full precomp: m x count */
    const float* a;             /* with coefficients (or ICM/ILS): m x count, else NULL */
    const float* cost;          /* with coefficients (or ICM/ILS): count, else NULL */
    const uint32_t* cluster_id; /* large root: count */
    const uint8_t* B_small;     /* large root: (m-1) x count */
    const float* best_err;      /* large root: count */
    const void* input;          /* the chunk's input as fill wrote it (d x count, uint8 with input_u8,
                                   else float; before any rotation), valid during the sink call */
} stlq_mi355_chunk_out;

/* first: the global id (start_id + offset in the stream) of the chunk's first vector. */
typedef int (*stlq_mi355_fill_fn)(void* user, int64_t first, int64_t count, void* dst);
typedef int (*stlq_mi355_sink_fn)(void* user, int64_t first, int64_t count,
                                  const stlq_mi355_chunk_out* out);

typedef struct stlq_mi355_stream_stats {
    double wall_ms;      /* whole call */
    double h2d_ms;       /* sum of H2D copy durations (copy stream) */
    double compute_ms;   /* sum of chunk encode durations incl. result D2H (context stream) */
    double fill_ms;      /* host time inside fill callbacks */
    double sink_ms;      /* host time inside sink callbacks */
    double h2d_bytes;
    int64_t chunks;
} stlq_mi355_stream_stats;

int stlq_mi355_encode_stream(stlq_mi355_ctx* ctx, int64_t n_total, int64_t chunk,
                             const stlq_mi355_stream_params* params, stlq_mi355_fill_fn fill,
                             stlq_mi355_sink_fn sink, void* user,
                             stlq_mi355_stream_stats* stats);

/* Timings of the last encode / beam_search / icm call on this context. */
int stlq_mi355_last_timings(stlq_mi355_ctx* ctx, stlq_mi355_timings* out);

/* BuildPrecompLargeRoot (src/quantizer/precomp_large_root.cpp:27-157,
 * include/stlq/quantizer/precomp_large_root.h:52-56): layer 0 is a large root codebook
 * C0 (d x h0, 1 <= h0 <= 2^26 - 2), layers 1..m-1 are C_small (d x Hs, h_vec[l] <= 256). Computes
 * norm0, G_small and G0S (h0 x Hs) on the device. */
int stlq_mi355_set_large_root(stlq_mi355_ctx* ctx, int d, int m, const int* h_vec,
                              const float* C0, const float* C_small);

/* BeamSearchPrefixLSLargeRoot (src/quantizer/beam_search.cpp:579-726) with the expansion of
 * BeamSearchPrefixLSLargeRootExpandFromRootCandidates (:728-992).
 *  forced_root (n, nullable): per-vector root; the root layer then contributes exactly that one
 *    candidate (a forced root).
 *  root_mode: with forced_root == NULL, 0 = top-H_beam root candidates (reference semantics),
 *    1 = force the nearest root (top-1 by the root-layer LS error).
 *  X (d x n) and xC_small (Hs x n) host pointers; xC_small may be NULL (computed on the device
 *  by MFMA). Outputs: cluster_id (n), B_small ((m-1) x n), best_err (n, nullable). */
int stlq_mi355_beam_search_large_root(stlq_mi355_ctx* ctx, const float* X, const float* xC_small,
                                      int64_t n, int H_beam, const uint32_t* forced_root,
                                      int root_mode, uint32_t* cluster_id, uint8_t* B_small,
                                      float* best_err);

/* StreamKernelProvider::ConvertU8ToF32AndRotatePtr (include/stlq/core/kernel_provider.h:44-52,
 * CPU version src/core/kernel_provider_cpu.cpp:48-80): out = R * float(in), where in is a
 * column-major uint8 tile of `rows` x `cols` with column stride ld_in >= rows, R is rows x rows
 * column-major (NULL: R = I, out = float(in)), and out is rows x cols column-major. Host
 * buffers; the product runs on fp32 MFMA with a fused k-ascending accumulation. */
int stlq_mi355_convert_u8_rotate(stlq_mi355_ctx* ctx, const uint8_t* in, int ld_in, int rows, int cols,
                                 const float* R, float* out);

/* Large-root refit. Layer 0 of vector i is its root cluster_id[i] (< h0); B_small ((m-1) x n)
 * holds layers 1..m-1. X (d x n) host; xC_small (Hs x n) host or NULL (device MFMA GEMM); nx2
 * host or NULL (formed from X). b0 = <C0[:,root], x> is formed on the device in the reference's
 * omp-simd order. */

/* SolveLeastSquaresAllLargeRoot (src/quantizer/least_squares.cpp:667-745,
 * include/stlq/quantizer/least_squares.h:54-59): a (m x n); a vector whose system fails even with
 * the diagonal bumps gets a = 0 and is counted in fail_count (nullable). */
int stlq_mi355_solve_ls_all_large_root(stlq_mi355_ctx* ctx, const float* X, const float* xC_small,
                                       int64_t n, const uint32_t* cluster_id, const uint8_t* B_small,
                                       float* a, int64_t* fail_count);

/* ComputeCostsLargeRoot (src/quantizer/cost_utils.cpp:211-233, cost_utils.h:37-44): cost (n). */
int stlq_mi355_compute_costs_large_root(stlq_mi355_ctx* ctx, const float* X, const float* xC_small,
                                        int64_t n, const uint32_t* cluster_id, const uint8_t* B_small,
                                        const float* a, const float* nx2, float* cost);

/* DynamicIcmWithIls{Abs,NoAbs}NoNormalLargeRoot (src/quantizer/icm.cpp:1005-1120,
 * include/stlq/quantizer/icm.h:45-75): LS refit and costs, icm_iters sweeps over layers 1..m-1
 * (the roots stay), then ils_iters perturbation rounds keyed by (seed, round,
 * sample_id_offset + i). B_small is updated in place; a (m x n) and cost (n) are outputs. */
int stlq_mi355_icm_ils_large_root(stlq_mi355_ctx* ctx, const float* X, const float* nx2,
                                  const float* xC_small, int64_t n, const uint32_t* cluster_id,
                                  int icm_iters, int ils_iters, int perturb_k, int use_abs,
                                  uint32_t seed, uint64_t sample_id_offset, uint8_t* B_small,
                                  float* a, float* cost);

#ifdef __cplusplus
}
#endif

#endif /* STLQ_MI355_H_ */
