/*
 * CPU oracle for the STLQ basic-encode path — TEST INFRASTRUCTURE ONLY.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load this
 * library, and only as the checker (or as the timed CPU baseline). The product path in
 * stlq_amd/ never links or calls it.
 *
 * Every function restates a reference routine (file:line relative to the ighxiy/STLQ tree).
 * Matrices follow the reference's column-major ColMajorMatrix convention
 * (include/stlq/common/types.h:35-51): element (row, col) lives at data[col*rows + row].
 *   X      d x n   (vector i = X + i*d)
 *   C_all  d x H   (codeword f = C_all + f*d)
 *   G      H x H   (G(row, col) = G[col*H + row])
 *   xC     H x n   (xC + i*H holds <x_i, c_f> for all flat codes f)
 *   codes  m x n   uint8 (codes + i*m)
 *   a      m x n   float
 */
#pragma once
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* encoder_precomp.inc:1-53 (C_all concat, invnorm, G = C_all^T C_all). */
int orc_build_precomp(int d, int m, const int* h_vec, const float* C_all,
                      float* G, float* invnorm, int nthreads);

/* cost_utils.cpp:88-110 (||x||^2 in the reference Release build's OpenMP-simd order: four
 * interleaved partial sums, tail into lane 0, lanes added in order). */
void orc_xnorm2(const float* X, int d, int64_t n, float* out, int nthreads);

/* blas.cpp:33-54 call site encoder_encode_base.inc:33-37 (xC = C_all^T X).
 * mode 0: sequential mul+add (no FMA), r ascending.
 * mode 1: fused k-ordered accumulation s = fma(c[r], x[r], s), r ascending — the order of the
 *         device's fp32 MFMA GEMM. */
void orc_gemm_xc(const float* C_all, int d, int H, const float* X, int64_t n,
                 float* xC, int mode, int nthreads);

/* beam_search.cpp:196-422 BeamSearchPrefixLS. best_err may be NULL. */
int orc_beam_search(const float* nx2, const float* xC, const float* G, int H, int m,
                    const int* h_vec, int H_beam, int64_t n, uint8_t* codes,
                    float* best_err, int nthreads);

/* least_squares.cpp:406-565 SolveLeastSquaresAll. Returns the failure count. */
int64_t orc_solve_ls_all(const float* xC, const float* G, int H, int m, const int* h_vec,
                         const uint8_t* codes, int64_t n, float* a, int nthreads);

/* cost_utils.cpp:112-158 SampleCost / ComputeCosts. */
void orc_compute_costs(const float* xC, const float* G, int H, int m, const int* h_vec,
                       const uint8_t* codes, const float* a, const float* nx2, int64_t n,
                       float* cost, int nthreads);

/* icm.cpp:89-344 RunIcm + icm.cpp:872-899 DynamicIcmWithIlsImpl with ils_iters = 0:
 * LS refit, costs, then icm_iters sweeps. codes/a/cost are updated in place
 * (a and cost are outputs; codes is input/output). */
int64_t orc_icm(const float* xC, const float* G, const float* invnorm, int H, int m,
                const int* h_vec, const float* nx2, int64_t n, int icm_iters, int use_abs,
                uint32_t seed, uint8_t* codes, float* a, float* cost, int nthreads);

/* DynamicIcmWithIls{Abs,NoAbs}NoNormal (icm.cpp:872-1003) with ILS: RunIcm, then ils_iters rounds
 * of a SplitMix64 perturbation of min(perturb_k, m) codes in layers 1..m-1 (keyed by seed, round
 * and sample_id_offset + i), RunIcm on the perturbed codes, and accept-if-better
 * (cand + 1e-6 < cost). One std::mt19937(seed) stream supplies every RunIcm's layer orders. */
int64_t orc_icm_ils(const float* xC, const float* G, const float* invnorm, int H, int m, const int* h_vec,
                    const float* nx2, int64_t n, int icm_iters, int ils_iters, int perturb_k, int use_abs,
                    uint32_t seed, uint64_t sample_id_offset, uint8_t* codes, float* a, float* cost,
                    int nthreads);

/* The layer order RunIcm uses on iteration `it` (std::shuffle with std::mt19937(seed),
 * icm.cpp:137/242/890). order_out has m * icm_iters entries. */
void orc_icm_orders(int m, int icm_iters, uint32_t seed, int* order_out);

/* linkage_tools.cpp:170-221 MeanMseFromPrecomp (double accumulation, per-vector). */
void orc_mse_from_precomp(const float* X, int d, const float* xC, const float* G, int H,
                          int m, const int* h_vec, const uint8_t* codes, const float* a,
                          int64_t n, double* per_vec, int nthreads);

/* Independent fp64 evaluator (not a reference routine): LS-refit the given codes in fp64
 * and return ||x - sum_l a_l c_l||^2 per vector by explicit reconstruction. */
void orc_mse_fp64_refit(const float* X, int d, const float* C_all, int H, int m,
                        const int* h_vec, const uint8_t* codes, int64_t n, double* per_vec,
                        int nthreads);

/* precomp_large_root.cpp:27-157 BuildPrecompLargeRoot. norm0[h0], G_small (Hs x Hs),
 * G0S (h0 x Hs, column-major: G0S(root, flat) = G0S[flat*h0 + root]). */
int orc_build_precomp_large_root(int d, int h0, int Hs, const float* C0,
                                 const float* C_small, float* norm0, float* G_small,
                                 float* G0S, int nthreads);

/* beam_search.cpp:579-726 BeamSearchPrefixLSLargeRoot, root scores from fused k-ordered
 * dot products (the device GEMM's order) instead of GemmRaw; expansion via
 * beam_search.cpp:728-992.
 * h_vec has m entries (h_vec[0] = h0); xC_small is Hs x n.
 * forced_root: NULL for the full large-root beam; otherwise a per-vector root id and the
 * root layer contributes exactly one finite candidate (the forced root).
 * root_mode: when forced_root is NULL and root_mode == 1, the nearest root by the
 * root-layer LS error is forced (one finite slot). */
int orc_beam_search_large_root(const float* X, int d, const float* nx2, const float* C0,
                               const float* norm0, const float* xC_small,
                               const float* G_small, const float* G0S, int h0, int Hs,
                               int m, const int* h_vec, int H_beam, int64_t n,
                               const uint32_t* forced_root, int root_mode,
                               uint32_t* cluster_id, uint8_t* B_small, float* best_err,
                               int nthreads);

/* The root stage of the above alone (beam_search.cpp:639-709): per vector, H_beam slots
 * [n, H_beam] of (error, code, a0, r00) in the layout ExpandFromRootCandidates takes
 * (beam_search.h:36-47); unused slots hold error +inf. */
int orc_large_root_candidates(const float* X, int d, const float* nx2, const float* C0,
                              const float* norm0, int h0, int H_beam, int64_t n,
                              const uint32_t* forced_root, int root_mode, float* root_errs,
                              int* root_codes, float* root_a0, float* root_r00, int nthreads);

/* precomp_large_root.cpp:101-114: invnorm_small_flat = 1/sqrt(Norm2(c)) (0 for a zero codeword),
 * Norm2 in the OpenMP-simd order of ||x||^2. */
void orc_invnorm_small(const float* C_small, int d, int Hs, float* out);

/* Large root (layer 0 = the vector's root cluster_id[i], layers 1..m-1 = B_small, (m-1) x n).
 * G_small Hs x Hs and G0S h0 x Hs as in orc_build_precomp_large_root; xC_small Hs x n.
 * b0 = <C0[:,cid], x> is the reference's omp-simd dot (same four-lane order as ||x||^2). */

/* least_squares.cpp:667-745 SolveLeastSquaresAllLargeRoot. Returns the failure count. */
int64_t orc_solve_ls_all_large_root(const float* X, int d, const float* C0, const float* norm0, int h0,
                                    const float* xC_small, const float* G_small, const float* G0S, int Hs, int m,
                                    const int* h_vec, const uint32_t* cluster_id, const uint8_t* B_small, int64_t n,
                                    float* a, int nthreads);

/* cost_utils.cpp:42-84, :160-233 ComputeCostsLargeRoot. */
void orc_compute_costs_large_root(const float* X, int d, const float* C0, const float* norm0, int h0,
                                  const float* xC_small, const float* G_small, const float* G0S, int Hs, int m,
                                  const int* h_vec, const uint32_t* cluster_id, const uint8_t* B_small,
                                  const float* a, const float* nx2, int64_t n, float* cost, int nthreads);

/* icm.cpp:347-870 RunIcmLargeRoot + :1005-1120 DynamicIcmWithIlsLargeRootImpl: LS refit, costs,
 * icm_iters sweeps over layers 1..m-1 (the root stays), then ils_iters perturb + ICM + accept
 * rounds. B_small is updated in place; a (m x n) and cost (n) are outputs. */
int64_t orc_icm_ils_large_root(const float* X, int d, const float* C0, const float* norm0, int h0,
                               const float* xC_small, const float* G_small, const float* G0S,
                               const float* invnorm_small, int Hs, int m, const int* h_vec,
                               const uint32_t* cluster_id, const float* nx2, int64_t n, int icm_iters, int ils_iters,
                               int perturb_k, int use_abs, uint32_t seed, uint64_t sample_id_offset,
                               uint8_t* B_small, float* a, float* cost, int nthreads);

#ifdef __cplusplus
}
#endif
