// Candidate pruning for the prefix-LS beam (src/quantizer/beam_search.cpp:286-333, :728-992).
//
// A candidate (slot h, codeword k) of layer L is rejected by the reference when the error e it
// computes in fp32 satisfies e >= worst (beam_search.cpp:320). Prunable() shows e > W for the worst
// W at the start of the candidate's scan (the worst only falls during a layer) from quantities far
// cheaper than the candidate's two triangular solves. A pruned candidate is therefore one the
// reference rejects, and its computed error is finite and positive (never NaN or -0), so no
// fast-path or best-first bookkeeping depends on it.
//
// Notation. R is the slot's stored upper Cholesky factor (L x L); its prefix codewords f_t carry
// sw_t = RN(1/RN(sqrt(G(f_t, f_t)))) and isw_t = RN(sqrt(G(f_t, f_t))) (so isw_t sw_t = 1 + eps,
// |eps| <= u = 2^-24). S = diag(1/sw_t) (the real numbers), M = R S^-1, b = S^-1 A (b_t = A_t sw_t),
// kap >= ||M^-1||_F^2 and phi >= ||M||_F^2 (per slot, rounded up), gamma_n = n u / (1 - n u).
// Gs is G with row f scaled by sw_f, so Gs(f_t, k) = b_t (1 + eps).
//
// Theorem. Triangular substitution with division (or multiplication by RN(1/R_ii), the large-root
// form) computes y, v with (R^T + E1) y = A, (R + E2) v = y, |E1|, |E2| <= gamma_{L+1} |R|
// (Higham, Accuracy and Stability of Numerical Algorithms, 2nd ed., Thm 8.5, with one more rounding
// on the diagonal for the reciprocal form). With F_i = E_i S^-1 (|F_i| <= gamma |M|, so
// ||F_i||_2 <= gamma sqrt(phi)) and nu = sqrt(kap) / (1 - gamma_{L+1} sqrt(kap phi)):
//   S v = (M + F2)^-1 (M^T + F1)^-1 b,  ||(M + F)^-1||_2 <= nu,
// so the reference's delta = fl(sum_t A_t v_t) <= (1 + gamma_L) nu^2 ||b||^2 (+ 2^-63 absolute for
// gradual underflow within the ranges below), denom = fl(alpha - delta) >= D (1 - u) with
// D = alpha - (1 + gamma_L) nu^2 ||b||^2 > 0, and
//   e >= fl(E_old - diff * fl(diff / denom)) >= (E_old - diff^2 (1+u)^2 / (D (1-u))) (1 - u).
// diff = fl(gamma - eta), eta the reference's fp32 A.a_old. The test forms eta~ = sum_t
// Gs(f_t, k) ahat_t by fma with ahat_t = fl(a_t isw_t); |eta~ - eta| <= 2 gamma_24 ||ahat|| ||b||
// (both sums approximate sum_t A_t a_t within gamma_{L+4} sum_t |A_t a_t|, and
// sum |A_t a_t| <= ||b|| ||a / sw||), so with d = fl(gamma - eta~):
//   diff^2 <= (1 + 2^-10.9) d^2 + cq b2,  cq >= 2^-25.8 ||ahat||^2 (per slot, rounded up).
// The per-candidate test
//   fl(gp * D_c) > fma(d, d, fl(cq * b2))  and  fl(gp * D_c) > 2^-80,
// with gp = fl(fl(E_old - W) (1 - 2^-8)), D_c = fl(fl(alpha (1 - 2^-20)) - fma(kb, b2, 2^-60)),
// b2 = the fma sum of Gs(f_t, k)^2 (>= (1 - gamma_{L+2}) ||b||^2) and
// kb >= (1+gamma_L) nu^2 / ((1 - gamma_{L+2})(1 - u)), together with E_old - W >= 2^-10 W, implies
// e > W strictly: the 2^-8 slack covers the 2^-10.9 cross term and every rounding of the chain
// (about 2^-18 more).
//
// Diagonal split (a second bound on delta, tighter when the prefix codewords are far from
// orthogonal, as at the deep layers of a d = 128 encode). Write M^-1 = Dg^-1 + U with Dg = diag(M)
// and U strictly upper. The reference's delta = sum_t b*_t w_t (1 + theta_t) with
// b* = (M^T + F1) y and (M + F2) w = y, so delta <= ||y||^2 (1 + 3 g sqrt(phi) nu) (g = 2^-19 >=
// gamma_21 (1 + 4u)), and ||y|| <= ||M^-T b*|| (1 + g sqrt(phi) nu). Then
//   ||M^-T b*|| <= ||Dg^-1 b*|| + ||U||_F ||b*||,  (sqrt(X) + nF B)^2 <= (1 + nF)(X + nF B^2)
// (AM-GM with theta = nF), X = sum_t (b*_t / M_tt)^2, B = ||b*||. The test forms X~ by fma from
// u_t = fl(c_t b_t), c_t = fl(RN(1/R_tt) isw_t) = (1 + 3.01u) / M_tt, so X <= X~ (1 + gamma_{L+11}),
// and B^2 <= b2 (1 + gamma_{L+3}). With nF2 >= ||U||_F^2 per slot (appending a column adds
// ||S q||^2 / rLL^2, the squared norm of the new off-diagonal column -S q / rLL of M^-1, bounded
// through v as for kap) and K = (1 + 2^-18)(1 + g sqrt(phi) nu)^2 (1 + 3 g sqrt(phi) nu)(1 + 2^-20),
//   delta <= k1 X~ + k2 b2,  k1 = K (1 + nF), k2 = K (1 + nF) nF  (per slot, rounded up),
// where the last factor of K covers the two roundings of fma(k1, X~, fma(k2, b2, .)). The test
// takes the smaller of the two bounds: D_c = fl(alpha (1 - 2^-20)) - min(fma(kb, b2, 2^-60),
// fma(k1, X~, fma(k2, b2, 2^-60))); everything else is as above.
//
// Ranges (overflow and underflow). max |G| <= 2^30 over the precomp (checked when the codebooks are
// set, else pruning is off), so every codeword has ||c||^2 <= 2^30 (1 + gamma_d) and sw_t >= 2^-15.
// Checked when a slot's constants are formed (else kb = +inf): sw_t <= 2^40 (prefix codewords of
// norm down to 2^-40: the beam does pick near-zero codewords at deep layers, where they cost
// nothing), kap <= 2^20, phi <= 2^10, cq <= 2^40. Then:
//  * |b_t| <= (1 + 2 gamma_d) ||c_k|| by Cauchy-Schwarz, so ||b|| < 2^17.3 for L <= 20; nu^2 < 2^21;
//    1 / M_tt^2 <= kap, so |c_t| < 2^10.1, |u_t| < 2^27.4 and X~ < 2^60;
//    y = (M^T + F1)^-1 b has ||y|| < 2^28, w = S v has ||w|| < 2^39 and |v_t| = sw_t |w_t| < 2^79;
//    the solves' products are R_ct y_c = M_ct y_c / sw_t and R_tc v_c = M_tc w_c, the delta sum's
//    A_t v_t = b_t w_t: every intermediate of the reference's candidate arithmetic stays below
//    2^120 (apart from gamma, eta, diff and e, whose overflow the reference and the test meet
//    alike: an infinite d never prunes).
//  * Gradual underflow adds at most tau/2 = 2^-150 absolute to a product or quotient (sums of
//    floats are exact in the subnormal range). In the forward solve equation t gains at most
//    (t + |R_tt|) tau/2 (1 + gamma), which sw_t scales into the system M^T y = b as at most
//    (L 2^40 + 2^5) tau/2 (1 + gamma) < 2^-105.6 (sw_t |R_tt| = |M_tt| <= 2^5); in the backward
//    solve row t gains at most (L + |R_tt|) tau/2 < 2^-129.9 (|R_tt| = |M_tt| / sw_t <= 2^20); the
//    delta sum L tau/2. Through (M + F2)^-1 (M^T + F1)^-1 these move delta by at most
//    nu^2 ||b|| sqrt(L) 2^-105.6 + nu ||b|| sqrt(L) 2^-129.9 + L 2^-150 < 2^-63, inside the absolute
//    slack 2^-60 (kAbsSlack) of D_c. Underflow in b2 and cq * b2 (terms below 2^-105) stays under
//    2^-25 of the 2^-80 floor on fl(gp * D_c).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace stlq_mi355 {
namespace prune {

constexpr float kKapCap = 0x1p20f;
constexpr float kPhiCap = 0x1p10f;
constexpr float kSwLo = 0x1p-15f;
constexpr float kSwHi = 0x1p40f;
constexpr uint32_t kGAbsMaxBits = 0x4E800000u;  // 2^30: envelope of max |G|
constexpr float kAlphaScale = 1.0f - 0x1p-20f;
constexpr float kAbsSlack = 0x1p-60f;
constexpr float kGapScale = 1.0f - 0x1p-8f;
constexpr float kGapMinRel = 0x1p-10f;
constexpr float kProdMin = 0x1p-80f;
constexpr double kCqCap = 0x1p40;
// 2^-19 >= gamma_{21} (1 + 4u): the solves' backward-error factor for any L <= 20, with room for
// the roundings of sqrt(kap * phi).
constexpr float kGammaSolve = 0x1p-19f;
// (1 + 2^-17) >= (1 + gamma_20)(1 + 2^-29) / ((1 - gamma_22)(1 - u)) times the roundings of
// SlotKb's own fp32 operations.
constexpr float kNuScale = 1.0f + 0x1p-17f;
constexpr double kCq = 0x1p-25;                 // >= 2^-25.8 with rounding room
constexpr double kStoreScale = 1.0 + 0x1p-22;  // fp64 -> fp32 rounded up with margin
// Layers from which the bound also tries the diagonal split (Prunable2): two more fma per prefix
// term and L more registers, which pay once the prefix codewords stop being nearly orthogonal (on
// the M=8, d=128 encode the Frobenius bound alone already prunes 86-91% up to layer 7).
constexpr int kDiagMinL = 9;

__host__ __device__ inline bool SwOk(float s) { return s >= kSwLo && s <= kSwHi; }

// The bound factor kb a slot carries for its use as a parent (+inf: never prune below it).
__host__ __device__ inline float SlotKb(float kap, float phi) {
    if (!(kap <= kKapCap) || !(phi <= kPhiCap)) return __builtin_huge_valf();
    const float den = 1.0f - kGammaSolve * sqrtf(kap * phi);
    return (kap * kNuScale) / (den * den);
}

// Per parent slot: gp = (E_old - W)(1 - 2^-8), or false when its candidates may not be pruned
// (a slot still empty, or a gap below 2^-10 W).
__host__ __device__ inline bool ParentGap(float E_old, float W, float& gp) {
    if (!(W < __builtin_huge_valf())) return false;
    const float g = E_old - W;
    if (!(g > 0.0f) || !(g >= W * kGapMinRel)) return false;
    gp = g * kGapScale;
    return true;
}

// True: the reference rejects this candidate. alc = fl(alpha * kAlphaScale); b2 and d as above.
__host__ __device__ inline bool Prunable(float alc, float b2, float d, float kb, float cq, float gp) {
    const float t2 = __builtin_fmaf(kb, b2, kAbsSlack);
    const float prod = gp * (alc - t2);
    const float q = __builtin_fmaf(d, d, cq * b2);
    return prod > q && prod > kProdMin;
}

// The diagonal-split test (see the file comment): x is the fma sum of fl(c_t b_t)^2.
__host__ __device__ inline bool Prunable2(float alc, float b2, float x, float d, float kb, float k1, float k2, float cq,
                                          float gp) {
    const float t1 = __builtin_fmaf(kb, b2, kAbsSlack);
    const float t2 = __builtin_fmaf(k1, x, __builtin_fmaf(k2, b2, kAbsSlack));
    const float prod = gp * (alc - __builtin_fminf(t1, t2));
    const float q = __builtin_fmaf(d, d, cq * b2);
    return prod > q && prod > kProdMin;
}

// c_t of the diagonal split from the slot's stored RN(1/R_tt) and the codeword's isw.
__host__ __device__ inline float DiagCoef(float rinv, float isw) { return rinv * isw; }

struct SlotBounds {
    float kap, phi, kb, cq, nf2;
};

__host__ __device__ inline SlotBounds NoBounds() {
    const float inf = __builtin_huge_valf();
    return SlotBounds{inf, inf, inf, inf, inf};
}

// The diagonal split's per-slot factors k1 = K (1 + nF) and k2 = K (1 + nF) nF (see the file
// comment), from the stored (rounded-up) kap, phi and nF2, in fp32 with every rounding covered:
// the ranges give den = 1 - g sqrt(kap phi) >= 15/16, so g sqrt(phi) nu <= g sqrt(kap phi) 16/15
// =: gs; each fp32 result below is within u of its value and the last factor 2^-18 of K absorbs
// them. +inf for a slot without bounds.
__host__ __device__ inline void DiagConsts(const SlotBounds& b, float& k1, float& k2) {
    if (!(b.kb < __builtin_huge_valf())) {
        k1 = k2 = __builtin_huge_valf();
        return;
    }
    const float gs = kGammaSolve * sqrtf(b.kap * b.phi) * (16.0f / 15.0f);
    const float K = (1.0f + 0x1p-18f) * (1.0f + gs) * (1.0f + gs) * (1.0f + 3.0f * gs) * (1.0f + 0x1p-20f) *
                    (1.0f + 0x1p-18f);
    const float nf = sqrtf(b.nf2) * (1.0f + 0x1p-22f);
    k1 = K * (1.0f + nf) * (1.0f + 0x1p-21f);
    k2 = K * (1.0f + nf) * nf * (1.0f + 0x1p-21f);
}

// Rounds the fp64 sums up into fp32 and derives kb (all +inf when out of range).
__host__ __device__ inline SlotBounds StoreBounds(double kap, double phi, double nf2, double asq, bool ok) {
    if (!(ok && kap <= static_cast<double>(kKapCap) && phi <= static_cast<double>(kPhiCap) && kCq * asq <= kCqCap &&
          nf2 <= kap))
        return NoBounds();
    SlotBounds b;
    b.kap = static_cast<float>(kap * kStoreScale);
    b.phi = static_cast<float>(phi * kStoreScale);
    b.kb = SlotKb(b.kap, b.phi);
    b.cq = static_cast<float>(kCq * asq * kStoreScale);
    b.nf2 = static_cast<float>(nf2 * kStoreScale);
    return b;
}

// A one-column slot (layer 0 or a root): R = [r00], kap = 1 / (sw0 r00)^2, phi = (sw0 r00)^2,
// nF2 = 0, ||ahat||^2 = (a0 isw0)^2.
__host__ __device__ inline SlotBounds FirstBounds(float r00, float sw0, float a0, float isw0) {
    const double m = static_cast<double>(r00) * static_cast<double>(sw0);
    const double ah = static_cast<double>(a0) * static_cast<double>(isw0);
    return StoreBounds(1.0 / (m * m), m * m, 0.0, ah * ah, SwOk(sw0) && m > 0.0);
}

// The slot made by appending column (y, rLL) to a parent with constants (kap_src, phi_src, nf2_src), from
// the parent's solve of the chosen candidate: y and v are the reference's forward and backward
// solutions ((R^T + E1) y = A, (R + E2) v = y, |E2| <= gamma_{L+1} |R|), sw(t) the prefix scalings,
// swL the new codeword's, asq = ||ahat||^2 of the new slot's coefficients.
// The new last column of M^-1 = S R_new^-1 is (-S q / rLL, 1 / (swL rLL)) with q = R^-1 y, and
// S q = S v + M^-1 F2 (S v) (F2 = E2 S^-1), so ||S q|| <= ||S v|| (1 + gamma_{L+1} sqrt(kap phi)):
// kap grows by at most ((||S v|| (1 + rho))^2 + 1 / swL^2) / rLL^2, rho = 2^-19 sqrt(kap phi), and
// nF2 by the first of those two terms.
// The new column of M adds exactly (|y|^2 + rLL^2) swL^2 to phi. The sums run in fp64.
template <int L, typename SwFn>
__host__ __device__ inline SlotBounds NextBounds(const float (&y)[L], const float (&v)[L], float rLL, SwFn sw, float swL,
                                                 float kap_src, float phi_src, float nf2_src, double asq) {
    bool ok = kap_src <= kKapCap && phi_src <= kPhiCap && nf2_src <= kap_src && SwOk(swL);
    double vs = 0.0, ysq = 0.0;
#pragma unroll
    for (int i = 0; i < L; ++i) {
        const float swi = sw(i);
        ok = ok && SwOk(swi);
        const double si = static_cast<double>(v[i]) / static_cast<double>(swi);
        vs += si * si;
        ysq += static_cast<double>(y[i]) * static_cast<double>(y[i]);
    }
    const double rho = static_cast<double>(kGammaSolve) *
                       (static_cast<double>(kap_src) * static_cast<double>(phi_src) >= 0.0
                            ? __builtin_sqrt(static_cast<double>(kap_src) * static_cast<double>(phi_src))
                            : 0.0);
    const double sq = __builtin_sqrt(vs) * (1.0 + rho);
    const double r2 = static_cast<double>(rLL) * static_cast<double>(rLL);
    const double s2 = static_cast<double>(swL) * static_cast<double>(swL);
    const double kap = static_cast<double>(kap_src) + (sq * sq + 1.0 / s2) / r2;
    const double phi = static_cast<double>(phi_src) + (ysq + r2) * s2;
    const double nf2 = static_cast<double>(nf2_src) + sq * sq / r2;
    return StoreBounds(kap, phi, nf2, asq, ok && r2 > 0.0);
}

}  // namespace prune
}  // namespace stlq_mi355
