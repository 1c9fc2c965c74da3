// Checker of the beam's candidate pruning (stlq_amd/csrc/prune_bound.hpp) on the CPU, built with
// hipcc as host code so that it runs the product's own bound functions.
//
// It replays the reference's BeamSearchPrefixLS (src/quantizer/beam_search.cpp:196-422: slot
// order, replace-first-worst, IEEE division, non-fused arithmetic, the all-skipped fallback) with
// each slot carrying the pruning constants the device computes (FirstBounds for layer 0,
// NextBounds from the chosen candidate's y and v), and for every evaluated candidate:
//  * evaluates the pruning test against the worst at the start of its slot's scan, exactly as the
//    device forms it (eta~ and b2 by fma from the row-scaled Gram, gp, kb, cq), and counts the
//    candidates it would skip and those among them the reference would have inserted (must be 0);
//  * evaluates the test with the threshold at the candidate's own error, where it must keep it
//    (the bound is a strict lower bound of the error the reference computes);
// and runs the beam again skipping the pruned candidates: codes and best errors must be identical.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <limits>
#include <vector>

#include "prune_bound.hpp"

using stlq_mi355::prune::FirstBounds;
using stlq_mi355::prune::NextBounds;
using stlq_mi355::prune::NoBounds;
using stlq_mi355::prune::ParentGap;
using stlq_mi355::prune::Prunable;
using stlq_mi355::prune::Prunable2;
using stlq_mi355::prune::SlotBounds;

namespace {

constexpr float kInf = std::numeric_limits<float>::infinity();

struct Slot {
    float err = kInf;
    std::vector<int> code;
    std::vector<float> a, R;  // R row-major m x m, upper
    SlotBounds bd = NoBounds();
};

struct Stats {
    int64_t candidates = 0, tested = 0, pruned = 0, violations = 0, self_kept_fail = 0, mismatches = 0;
    // the last layer's minimum rule (LastPick in beam_kernels.hpp): vectors it decides, vectors it would
    // flag for a re-run, decided vectors whose pick differs from the reference's, and the last
    // layer's candidates and how many of them the bound against the running minimum prunes
    int64_t lp_decided = 0, lp_flagged = 0, lp_mismatches = 0, lp_candidates = 0, lp_pruned = 0;
    int64_t last_pruned_worst = 0;  // the last layer's candidates the top-H bound prunes
};

// One candidate with the reference's arithmetic (beam_search.cpp:286-318).
bool EvalRef(const Slot& s, int L, int m, const float* A, float alpha, float gamma, float* y, float* v, float& e,
             float& denom, float& a_last) {
    for (int r = 0; r < L; ++r) {
        float q = A[r];
        for (int j = 0; j < r; ++j) q = q - s.R[j * m + r] * y[j];
        y[r] = q / s.R[r * m + r];
    }
    for (int r = L - 1; r >= 0; --r) {
        float q = y[r];
        for (int j = r + 1; j < L; ++j) q = q - s.R[r * m + j] * v[j];
        v[r] = q / s.R[r * m + r];
    }
    float delta = 0.0f, eta = 0.0f;
    for (int t = 0; t < L; ++t) {
        delta = delta + A[t] * v[t];
        eta = eta + A[t] * s.a[t];
    }
    denom = alpha - delta;
    if (denom == 0.0f) return false;
    const float diff = gamma - eta;
    a_last = diff / denom;
    const float ee = s.err - diff * a_last;
    e = ee < 0.0f ? 0.0f : ee;
    return true;
}

int FirstMax(const std::vector<float>& e, int Hb, float& worst) {
    int wi = 0;
    worst = e[0];
    for (int h = 1; h < Hb; ++h) {
        if (e[h] > worst) {
            worst = e[h];
            wi = h;
        }
    }
    return wi;
}

// The device's test for candidate k of slot s at threshold W (prune_bound.hpp).
bool DeviceTest(const Slot& s, int L, int m, const float* Gs, const float* sw, const float* isw, const int* off, int H,
                int fk, float alpha, float gamma, float W) {
    float gp = 0.0f;
    if (!(s.bd.kb < kInf) || !ParentGap(s.err, W, gp)) return false;
    float et = 0.0f, b2 = 0.0f, xs = 0.0f;
    for (int t = 0; t < L; ++t) {
        const int f = off[t] + s.code[t];
        const float bt = Gs[static_cast<int64_t>(f) * H + fk];
        const float ah = s.a[t] * isw[f];
        // c_t from the slot's RN(1/R_tt), as the device stores it
        const float ut = stlq_mi355::prune::DiagCoef(1.0f / s.R[t * m + t], isw[f]) * bt;
        et = t == 0 ? bt * ah : std::fma(bt, ah, et);
        b2 = t == 0 ? bt * bt : std::fma(bt, bt, b2);
        xs = t == 0 ? ut * ut : std::fma(ut, ut, xs);
    }
    (void)sw;
    const float alc = alpha * stlq_mi355::prune::kAlphaScale;
    if (L >= stlq_mi355::prune::kDiagMinL) {
        float k1, k2;
        stlq_mi355::prune::DiagConsts(s.bd, k1, k2);
        return Prunable2(alc, b2, xs, gamma - et, s.bd.kb, k1, k2, s.bd.cq, gp);
    }
    return Prunable(alc, b2, gamma - et, s.bd.kb, s.bd.cq, gp);
}

}  // namespace

extern "C" {

// G is the reference's column-major H x H Gram (symmetric here), xC H x n, nx2 n. Outputs
// stats[6] = {candidates, tested (slot had finite constants and a full beam), pruned, violations,
// self-threshold failures, vectors whose pruned beam differs}.
int prune_check(const float* G, const float* xC, const float* nx2, int H, int m, const int* h_vec, int64_t n,
                int Hb, int64_t* stats) {
    std::vector<int> off(m, 0);
    for (int l = 1; l < m; ++l) off[l] = off[l - 1] + h_vec[l - 1];
    // The device's scalings and row-scaled Gram (PruneScaleKernel, RowScaleKernel).
    std::vector<float> gd(H), sw(H), isw(H), Gs(static_cast<size_t>(H) * H);
    for (int f = 0; f < H; ++f) {
        gd[f] = G[static_cast<int64_t>(f) * H + f];
        isw[f] = std::sqrt(gd[f]);
        sw[f] = 1.0f / isw[f];
    }
    for (int r = 0; r < H; ++r)
        for (int c = 0; c < H; ++c) Gs[static_cast<int64_t>(r) * H + c] = G[static_cast<int64_t>(c) * H + r] * sw[r];
    Stats st;
    std::vector<float> A(m), y(m), v(m);
    for (int64_t i = 0; i < n; ++i) {
        const float* xc = xC + i * H;
        std::vector<int> codes_run[2];
        float err_run[2] = {kInf, kInf};
        std::vector<Slot> last_parents;  // the last layer's parent slots (pass 0)
        std::vector<float> last_e;       // their candidates' errors, parent-major
        std::vector<uint8_t> last_elig;
        for (int pass = 0; pass < 2; ++pass) {  // pass 1 skips the pruned candidates
            std::vector<Slot> cur;
            {  // layer 0 (beam_search.cpp:240-263), reference slot order
                std::vector<float> e(Hb, kInf);
                std::vector<int> kk(Hb, -1);
                float worst;
                int wi = FirstMax(e, Hb, worst);
                for (int k = 0; k < h_vec[0]; ++k) {
                    const float al = gd[off[0] + k];
                    if (al == 0.0f) continue;
                    const float g = xc[off[0] + k];
                    const float a1 = g / al;
                    const float e1 = nx2[i] - g * a1;
                    if (!(e1 < worst)) continue;
                    e[wi] = e1;
                    kk[wi] = k;
                    wi = FirstMax(e, Hb, worst);
                }
                for (int h = 0; h < Hb; ++h) {
                    if (!(e[h] < kInf)) continue;
                    Slot s;
                    s.err = e[h];
                    s.code = {kk[h]};
                    const float al = gd[off[0] + kk[h]];
                    s.a = {xc[off[0] + kk[h]] / al};
                    s.R.assign(static_cast<size_t>(m) * m, 0.0f);
                    s.R[0] = std::sqrt(al);
                    s.bd = FirstBounds(s.R[0], sw[off[0] + kk[h]], s.a[0], isw[off[0] + kk[h]]);
                    cur.push_back(s);
                }
            }
            for (int L = 1; L < m && !cur.empty(); ++L) {
                if (pass == 0 && L == m - 1) {
                    last_parents = cur;
                    last_e.assign(cur.size() * static_cast<size_t>(h_vec[L]), kInf);
                    last_elig.assign(cur.size() * static_cast<size_t>(h_vec[L]), 0);
                }
                struct Pick {
                    int h = -1, k = 0;
                    float denom = 0, a_last = 0;
                    std::vector<float> y, v;
                };
                std::vector<float> e(Hb, kInf);
                std::vector<Pick> pk(Hb);
                float worst;
                int wi = FirstMax(e, Hb, worst);
                for (int h = 0; h < static_cast<int>(cur.size()); ++h) {
                    const Slot& s = cur[h];
                    const float W0 = worst;
                    for (int k = 0; k < h_vec[L]; ++k) {
                        const int fk = off[L] + k;
                        for (int t = 0; t < L; ++t) A[t] = G[static_cast<int64_t>(fk) * H + off[t] + s.code[t]];
                        float ec, dn, al;
                        const bool elig = EvalRef(s, L, m, A.data(), gd[fk], xc[fk], y.data(), v.data(), ec, dn, al);
                        const bool pruned = DeviceTest(s, L, m, Gs.data(), sw.data(), isw.data(), off.data(), H, fk,
                                                       gd[fk], xc[fk], W0);
                        if (pass == 0 && L == m - 1) {
                            last_e[static_cast<size_t>(h) * h_vec[L] + k] = ec;
                            last_elig[static_cast<size_t>(h) * h_vec[L] + k] = elig ? 1 : 0;
                            if (pruned) ++st.last_pruned_worst;
                        }
                        if (pass == 0) {
                            ++st.candidates;
                            if (s.bd.kb < kInf && W0 < kInf) ++st.tested;
                            if (pruned) {
                                ++st.pruned;
                                if (elig && !(ec >= worst)) ++st.violations;
                            }
                            // at its own error the test must keep the candidate
                            if (elig && std::isfinite(ec) &&
                                DeviceTest(s, L, m, Gs.data(), sw.data(), isw.data(), off.data(), H, fk, gd[fk], xc[fk],
                                           ec))
                                ++st.self_kept_fail;
                        }
                        if (pass == 1 && pruned) continue;
                        if (!elig || ec >= worst) continue;
                        e[wi] = ec;
                        pk[wi].h = h;
                        pk[wi].k = k;
                        pk[wi].denom = dn;
                        pk[wi].a_last = al;
                        pk[wi].y.assign(y.begin(), y.begin() + L);
                        pk[wi].v.assign(v.begin(), v.begin() + L);
                        wi = FirstMax(e, Hb, worst);
                    }
                }
                std::vector<Slot> nxt;
                int finite = 0;
                for (int q = 0; q < Hb; ++q) finite += std::isfinite(e[q]) ? 1 : 0;
                if (finite == 0) {  // all-skipped fallback: the parents with a zero new column
                    for (int h = 0; h < static_cast<int>(cur.size()) && h < Hb; ++h) {
                        Slot s = cur[h];
                        s.code.push_back(0);
                        s.a.push_back(0.0f);
                        s.bd = NoBounds();
                        nxt.push_back(s);
                    }
                } else {
                    for (int q = 0; q < Hb; ++q) {
                        if (!(e[q] < kInf) && !std::isnan(e[q])) continue;
                        const Slot& src = cur[pk[q].h];
                        Slot s;
                        s.err = e[q];
                        s.code = src.code;
                        s.code.push_back(pk[q].k);
                        s.a.resize(L + 1);
                        for (int t = 0; t < L; ++t) s.a[t] = src.a[t] - pk[q].v[t] * pk[q].a_last;
                        s.a[L] = pk[q].a_last;
                        s.R = src.R;
                        for (int t = 0; t < L; ++t) s.R[t * m + L] = pk[q].y[t];
                        s.R[L * m + L] = std::sqrt(pk[q].denom);
                        double asq = 0.0;
                        for (int t = 0; t <= L; ++t) {
                            const double ah = static_cast<double>(s.a[t]) * static_cast<double>(isw[off[t] + s.code[t]]);
                            asq += ah * ah;
                        }
                        float yy[32], vv[32];
                        for (int t = 0; t < L; ++t) {
                            yy[t] = pk[q].y[t];
                            vv[t] = pk[q].v[t];
                        }
                        // NextBounds is templated on L; dispatch the layers this checker runs.
                        auto swf = [&](int t) { return sw[off[t] + src.code[t]]; };
                        const float swL = sw[off[L] + pk[q].k];
                        switch (L) {
#define STLQ_NB(LL)                                                                                            \
    case LL: {                                                                                                  \
        float ya[LL], va[LL];                                                                                   \
        for (int t = 0; t < LL; ++t) {                                                                          \
            ya[t] = yy[t];                                                                                      \
            va[t] = vv[t];                                                                                      \
        }                                                                                                       \
        s.bd = NextBounds<LL>(ya, va, s.R[L * m + L], swf, swL, src.bd.kap, src.bd.phi, src.bd.nf2, asq);                   \
        break;                                                                                                  \
    }
                            STLQ_NB(1) STLQ_NB(2) STLQ_NB(3) STLQ_NB(4) STLQ_NB(5) STLQ_NB(6) STLQ_NB(7) STLQ_NB(8)
                            STLQ_NB(9) STLQ_NB(10) STLQ_NB(11) STLQ_NB(12) STLQ_NB(13) STLQ_NB(14) STLQ_NB(15)
                            STLQ_NB(16) STLQ_NB(17) STLQ_NB(18) STLQ_NB(19)
#undef STLQ_NB
                            default:
                                s.bd = NoBounds();
                        }
                        nxt.push_back(s);
                    }
                }
                cur.swap(nxt);
            }
            // final pick: first minimum over the slots (beam_search.cpp:409-416)
            int best = 0;
            for (int h = 1; h < static_cast<int>(cur.size()); ++h)
                if (cur[h].err < cur[best].err) best = h;
            if (!cur.empty()) {
                codes_run[pass] = cur[best].code;
                err_run[pass] = cur[best].err;
            }
        }
        if (codes_run[0] != codes_run[1] ||
            std::memcmp(&err_run[0], &err_run[1], sizeof(float)) != 0)
            ++st.mismatches;
        if (m >= 2 && !last_parents.empty()) {
            // The minimum rule: parents in ascending error order (the best-first pass's), each
            // candidate bound-tested against the running minimum at its parent's start; flagged
            // on a tie for the minimum, an eligible NaN or -0, or no finite candidate.
            const int L = m - 1, K = h_vec[L];
            std::vector<int> ord(last_parents.size());
            for (size_t q = 0; q < ord.size(); ++q) ord[q] = static_cast<int>(q);
            std::stable_sort(ord.begin(), ord.end(),
                             [&](int a, int b) { return last_parents[a].err < last_parents[b].err; });
            float best = kInf;
            int bh = -1, bk = 0;
            bool tie = false, bad = false;
            for (int h : ord) {
                const Slot& s = last_parents[h];
                const float W0 = best;
                for (int k = 0; k < K; ++k) {
                    const int fk = off[L] + k;
                    ++st.lp_candidates;
                    if (DeviceTest(s, L, m, Gs.data(), sw.data(), isw.data(), off.data(), H, fk, gd[fk], xc[fk], W0)) {
                        ++st.lp_pruned;
                        continue;
                    }
                    if (!last_elig[static_cast<size_t>(h) * K + k]) continue;
                    const float ec = last_e[static_cast<size_t>(h) * K + k];
                    if (std::isnan(ec) || (ec == 0.0f && std::signbit(ec))) bad = true;
                    if (!(ec < kInf)) continue;
                    if (ec < best) {
                        best = ec;
                        bh = h;
                        bk = k;
                        tie = false;
                    } else if (ec == best) {
                        tie = true;
                    }
                }
            }
            if (bad || tie || bh < 0) {
                ++st.lp_flagged;
            } else {
                ++st.lp_decided;
                std::vector<int> codes = last_parents[bh].code;
                codes.push_back(bk);
                if (codes != codes_run[0] || std::memcmp(&best, &err_run[0], sizeof(float)) != 0) ++st.lp_mismatches;
            }
        }
    }
    stats[0] = st.candidates;
    stats[1] = st.tested;
    stats[2] = st.pruned;
    stats[3] = st.violations;
    stats[4] = st.self_kept_fail;
    stats[5] = st.mismatches;
    stats[6] = st.lp_decided;
    stats[7] = st.lp_flagged;
    stats[8] = st.lp_mismatches;
    stats[9] = st.lp_candidates;
    stats[10] = st.lp_pruned;
    stats[11] = st.last_pruned_worst;
    return 0;
}

}  // extern "C"
