// CPU oracle for the STLQ basic-encode path — TEST INFRASTRUCTURE ONLY.
//
// This file restates the reference CPU encoder (ighxiy/STLQ, C++20 + OpenMP) so that the
// HIP encoder in stlq_amd/ can be checked against it. It is loaded only by tests/,
// __graft_entry__.smoke() and bench.py's cpu_baseline leg; nothing in the product links it.
//
// Build flags (oracle/Makefile): -O2 -ffp-contract=off, no -ffast-math, no -march, so every
// float operation below is one IEEE-rounded op, as in the reference build (CMakeLists.txt:9-21
// targets baseline x86-64 without FMA).
//
// Deviations from the reference that are forced by unpinned third-party arithmetic:
//  * G = C_all^T C_all and xC = C_all^T X come from cblas_sgemm in the reference
//    (src/core/blas.cpp:33-54, un-vendored BLAS), whose summation order is unpinned. Here G is
//    a sequential mul+add dot product (exactly symmetric), and xC is either sequential mul+add
//    (mode 0) or a fused k-ordered accumulation (mode 1), the order of the device GEMM.
//  * ||x||^2 and the large-root ||c0||^2 are `omp simd` reductions in the reference
//    (beam_search.cpp:218-223, :629-633, cost_utils.cpp:99-109, precomp_large_root.cpp:14-23).
//    OpenMP leaves their order open; the reference's own Release build (GCC, -O3 -fopenmp, no
//    -march, so SSE2 with 4 float lanes) sums element t into lane t mod 4 over the first
//    floor(d/4)*4 elements, adds the remaining elements to lane 0, and then adds the lanes in
//    order to the initial 0. SimdLane4SumSq restates that order; it was checked bit for bit
//    against that build for d = 1..131 (tests/test_ref_cpu.py).
//  * SolveLeastSquaresAll for m not in {5,10} calls LAPACK spotrf/spotrs
//    (least_squares.cpp:512-564); here every m uses the hand-written Cholesky of
//    least_squares.cpp:44-84, with LAPACK's failure test (pivot <= 0 or NaN) for m not in
//    {5,10} — parity for those m is unpinned.
//  * The all-candidates-skipped fallback of the beam (beam_search.cpp:385-400) copies a code
//    slot the reference never wrote for the current vector (stale per-thread workspace); the
//    workspace here is zeroed per vector, so that code is 0.

#include "stlq_oracle.h"

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <limits>
#include <numeric>
#include <random>
#include <vector>

#include <omp.h>

namespace {

using u8 = std::uint8_t;
constexpr float kInf = std::numeric_limits<float>::infinity();
constexpr float kEps = 1e-6f;  // least_squares.cpp:19, icm.cpp:29

inline float GAt(const float* G, int H, int row, int col) {  // linear_algebra.h:17-19
    return G[static_cast<std::size_t>(col) * H + row];
}

std::vector<int> Offsets(int m, const int* h_vec) {
    std::vector<int> off(m);
    int o = 0;
    for (int l = 0; l < m; ++l) {
        off[l] = o;
        o += h_vec[l];
    }
    return off;
}

void SetThreads(int nthreads) {
    if (nthreads > 0) omp_set_num_threads(nthreads);
}

// beam_search.cpp:101-113 RecomputeWorst: first slot holding the max, strict '>' scan.
inline int FirstMaxSlot(const float* e, int Hb, float* out) {
    int w = 0;
    float we = e[0];
    for (int s = 1; s < Hb; ++s) {
        if (e[s] > we) {
            we = e[s];
            w = s;
        }
    }
    *out = we;
    return w;
}

// beam_search.cpp:115-125 CountFinite.
inline int CountFinite(const float* e, int Hb) {
    int c = 0;
    for (int s = 0; s < Hb; ++s) c += (e[s] < kInf);
    return c;
}

// beam_search.cpp:127-162 SolveCholUpperRawFixed / linear_algebra.cpp:57-77:
// forward U^T y = b then backward U x = y, subtraction in index order, true division.
inline void SolveUpper(const float* R, int L, int ld, const float* b, float* x, float* y) {
    for (int i = 0; i < L; ++i) {
        float s = b[i];
        for (int j = 0; j < i; ++j) s -= R[j * ld + i] * y[j];
        y[i] = s / R[i * ld + i];
    }
    for (int i = L - 1; i >= 0; --i) {
        float s = y[i];
        for (int j = i + 1; j < L; ++j) s -= R[i * ld + j] * x[j];
        x[i] = s / R[i * ld + i];
    }
}

// beam_search.cpp:517-575 SolveCholUpperRawBatched (large-root expansion): same order,
// but scaled by the reciprocal of the diagonal instead of divided by it.
inline void SolveUpperRecip(const float* R, int L, int ld, const float* b, float* x, float* y) {
    for (int i = 0; i < L; ++i) {
        float s = b[i];
        for (int j = 0; j < i; ++j) s -= R[j * ld + i] * y[j];
        const float inv = 1.0f / R[i * ld + i];
        y[i] = s * inv;
    }
    for (int i = L - 1; i >= 0; --i) {
        float s = y[i];
        for (int j = i + 1; j < L; ++j) s -= R[i * ld + j] * x[j];
        const float inv = 1.0f / R[i * ld + i];
        x[i] = s * inv;
    }
}

// Per-thread beam workspace; two ping-pong buffers of H_beam slots
// (beam_search.cpp:28-82 BeamWorkspace, same slot-major layout).
struct Beam {
    int m = 0, Hb = 0;
    std::vector<u8> code[2];
    std::vector<std::uint32_t> root[2];
    std::vector<float> err[2], coef[2], chol[2];
    std::vector<int> pick_src, pick_k;
    std::vector<std::uint32_t> pick_root;
    std::vector<float> pick_denom, pick_alast, pick_v, pick_y;
    std::vector<float> A, v, y;

    Beam(int m_, int Hb_) : m(m_), Hb(Hb_) {
        for (int b = 0; b < 2; ++b) {
            code[b].assign(static_cast<std::size_t>(m) * Hb, 0);
            root[b].assign(Hb, 0);
            err[b].assign(Hb, kInf);
            coef[b].assign(static_cast<std::size_t>(m) * Hb, 0.0f);
            chol[b].assign(static_cast<std::size_t>(m) * m * Hb, 0.0f);
        }
        pick_src.assign(Hb, -1);
        pick_k.assign(Hb, 0);
        pick_root.assign(Hb, 0);
        pick_denom.assign(Hb, 0.0f);
        pick_alast.assign(Hb, 0.0f);
        pick_v.assign(static_cast<std::size_t>(m) * Hb, 0.0f);
        pick_y.assign(static_cast<std::size_t>(m) * Hb, 0.0f);
        A.assign(m, 0.0f);
        v.assign(m, 0.0f);
        y.assign(m, 0.0f);
    }
    void Reset() {
        for (int b = 0; b < 2; ++b) {
            std::fill(code[b].begin(), code[b].end(), 0);
            std::fill(root[b].begin(), root[b].end(), 0);
            std::fill(err[b].begin(), err[b].end(), kInf);
            std::fill(coef[b].begin(), coef[b].end(), 0.0f);
            std::fill(chol[b].begin(), chol[b].end(), 0.0f);
        }
    }
    u8& Code(int b, int slot, int layer) { return code[b][static_cast<std::size_t>(slot) * m + layer]; }
    float& Coef(int b, int slot, int layer) { return coef[b][static_cast<std::size_t>(slot) * m + layer]; }
    float* Chol(int b, int slot) { return chol[b].data() + static_cast<std::size_t>(slot) * m * m; }
};

// Prefix-LS candidate evaluation of one (beam, code) pair for layers >= 1
// (beam_search.cpp:286-318). Returns false when denom == 0 (candidate skipped).
struct CandOut {
    float e, denom, a_last;
};

template <bool Recip>
inline bool EvalCandidate(const float* R, int L, int m, const float* A, const float* a_old,
                          float E_old, float alpha, float gamma, float* v, float* y,
                          CandOut* out) {
    if (Recip) {
        SolveUpperRecip(R, L, m, A, v, y);
    } else {
        SolveUpper(R, L, m, A, v, y);
    }
    float delta = 0.0f;
    float eta = 0.0f;
    for (int t = 0; t < L; ++t) {
        const float at = A[t];
        delta += at * v[t];
        eta += at * a_old[t];
    }
    const float denom = alpha - delta;
    if (denom == 0.0f) return false;
    const float diff = gamma - eta;
    const float a_last = diff / denom;
    float e = E_old - diff * a_last;
    if (e < 0.0f) e = 0.0f;
    out->e = e;
    out->denom = denom;
    out->a_last = a_last;
    return true;
}

// Deferred write-back of the selected candidates (beam_search.cpp:337-383, :896-947) and the
// all-skipped fallback (beam_search.cpp:385-400, :949-966).
inline int Materialize(Beam& W, int cur, int nxt, int L, int curH) {
    const int m = W.m, Hb = W.Hb;
    for (int out = 0; out < Hb; ++out) {
        if (W.err[nxt][out] >= kInf) continue;
        const int src = W.pick_src[out];
        const int k = W.pick_k[out];
        const float denom = W.pick_denom[out];
        const float a_last = W.pick_alast[out];
        W.root[nxt][out] = W.pick_root[out];
        for (int t = 0; t < L; ++t) W.Code(nxt, out, t) = W.Code(cur, src, t);
        W.Code(nxt, out, L) = static_cast<u8>(k);
        for (int t = 0; t < L; ++t) {
            const float vt = W.pick_v[static_cast<std::size_t>(t) * Hb + out];
            W.Coef(nxt, out, t) = W.Coef(cur, src, t) - vt * a_last;
        }
        W.Coef(nxt, out, L) = a_last;
        const float* Rp = W.Chol(cur, src);
        float* Rn = W.Chol(nxt, out);
        std::memcpy(Rn, Rp, sizeof(float) * static_cast<std::size_t>(L) * m);
        for (int t = 0; t < L; ++t) Rn[t * m + L] = W.pick_y[static_cast<std::size_t>(t) * Hb + out];
        Rn[L * m + L] = std::sqrt(denom);
    }
    int newH = CountFinite(W.err[nxt].data(), Hb);
    if (newH == 0) {
        newH = std::min(curH, Hb);
        for (int h = 0; h < newH; ++h) {
            W.err[nxt][h] = W.err[cur][h];
            W.root[nxt][h] = W.root[cur][h];
            for (int t = 0; t <= L; ++t) {
                W.Code(nxt, h, t) = W.Code(cur, h, t);
                W.Coef(nxt, h, t) = W.Coef(cur, h, t);
            }
            std::copy(W.Chol(cur, h), W.Chol(cur, h) + m * m, W.Chol(nxt, h));
        }
    }
    return std::max(1, newH);
}

// Layers 1..m-1 of the prefix-LS beam, common to the full-precomp and large-root variants.
// gather(h, t, k) returns A_t for candidate k of layer L under beam h.
template <bool Recip, typename AlphaFn, typename GammaFn, typename GatherFn>
int ExpandLayer(Beam& W, int cur, int nxt, int L, int K, int curH, AlphaFn alpha_of,
                GammaFn gamma_of, GatherFn gather) {
    const int m = W.m, Hb = W.Hb;
    std::fill(W.err[nxt].begin(), W.err[nxt].end(), kInf);
    std::fill(W.pick_src.begin(), W.pick_src.end(), -1);
    float worst;
    int wi = FirstMaxSlot(W.err[nxt].data(), Hb, &worst);
    for (int h = 0; h < curH; ++h) {
        const float* R = W.Chol(cur, h);
        const float* a_old = W.coef[cur].data() + static_cast<std::size_t>(h) * m;
        const float E_old = W.err[cur][h];
        for (int k = 0; k < K; ++k) {
            for (int t = 0; t < L; ++t) W.A[t] = gather(h, t, k);
            CandOut c;
            if (!EvalCandidate<Recip>(R, L, m, W.A.data(), a_old, E_old, alpha_of(k), gamma_of(k),
                                      W.v.data(), W.y.data(), &c)) {
                continue;
            }
            if (c.e >= worst) continue;
            W.err[nxt][wi] = c.e;
            W.pick_src[wi] = h;
            W.pick_k[wi] = k;
            W.pick_root[wi] = W.root[cur][h];
            W.pick_denom[wi] = c.denom;
            W.pick_alast[wi] = c.a_last;
            for (int t = 0; t < L; ++t) {
                W.pick_v[static_cast<std::size_t>(t) * Hb + wi] = W.v[t];
                W.pick_y[static_cast<std::size_t>(t) * Hb + wi] = W.y[t];
            }
            wi = FirstMaxSlot(W.err[nxt].data(), Hb, &worst);
        }
    }
    return Materialize(W, cur, nxt, L, curH);
}

// beam_search.cpp:409-416 final pick: first minimum over the live slots.
inline int BestSlot(const float* e, int curH) {
    int best = 0;
    float be = e[0];
    for (int h = 1; h < curH; ++h) {
        if (e[h] < be) {
            be = e[h];
            best = h;
        }
    }
    return best;
}

// least_squares.cpp:44-66 CholeskyUpperFixed (row-major upper, A[r*m+c]).
// lapack_test selects LAPACK's failure criterion (pivot <= 0 or NaN) used for m not in {5,10}.
bool CholUpper(float* A, int m, bool lapack_test) {
    for (int k = 0; k < m; ++k) {
        float sum = A[k * m + k];
        for (int j = 0; j < k; ++j) {
            const float v = A[j * m + k];
            sum -= v * v;
        }
        if (lapack_test ? !(sum > 0.0f) : (sum <= kEps)) return false;
        const float diag = std::sqrt(sum);
        A[k * m + k] = diag;
        for (int i = k + 1; i < m; ++i) {
            float s = A[k * m + i];
            for (int j = 0; j < k; ++j) s -= A[j * m + k] * A[j * m + i];
            A[k * m + i] = s / diag;
        }
    }
    return true;
}

// least_squares.cpp:86-129 SolveLeastSquaresSampleFixed (one vector); a_out untouched on failure.
bool SolveLsSample(const float* xCi, const float* G, int H, int m, const int* off,
                   const u8* code, float* a_out, float* A, float* b, float* x, float* y) {
    const bool lapack_test = !(m == 5 || m == 10);
    auto fill = [&](float lambda) {
        std::fill(A, A + m * m, 0.0f);
        for (int j = 0; j < m; ++j) {
            const int fj = off[j] + code[j];
            b[j] = xCi[fj];
            for (int k = 0; k <= j; ++k) {
                const int fk = off[k] + code[k];
                A[k * m + j] = GAt(G, H, fk, fj);
            }
            A[j * m + j] += lambda;
        }
    };
    fill(0.0f);
    bool ok = CholUpper(A, m, lapack_test);
    if (!ok) {
        float bump = kEps;
        for (int attempt = 0; attempt < 3 && !ok; ++attempt) {
            fill(bump);
            ok = CholUpper(A, m, lapack_test);
            bump *= 10.0f;
        }
    }
    if (!ok) return false;
    SolveUpper(A, m, m, b, x, y);
    std::copy(x, x + m, a_out);
    return true;
}

// cost_utils.cpp:112-137 SampleCost.
inline float SampleCost(const float* xCi, const float* G, int H, int m, const int* off,
                        const u8* code, const float* a, float nx2) {
    float term1 = 0.0f;
    float term2 = 0.0f;
    for (int l = 0; l < m; ++l) {
        const int fl = off[l] + code[l];
        const float al = a[l];
        term1 += al * xCi[fl];
        for (int k = 0; k < m; ++k) {
            const int fk = off[k] + code[k];
            term2 += al * a[k] * GAt(G, H, fl, fk);
        }
    }
    return nx2 - 2.0f * term1 + term2;
}

// Fused k-ordered dot product: s = fma(c[r], x[r], s) for r ascending, one rounding per term.
// This is the accumulation order of the device GEMM (v_mfma_f32_16x16x4_f32 issued over
// ascending k: each product is fused into the running fp32 sum), so xC and root scores computed
// here match the device bit for bit. The reference's own order is BLAS's (unpinned).
// Sum of squares in the reference build's OpenMP-simd order (see the file comment).
inline float SimdLane4SumSq(const float* x, int d) {
    float p0 = 0.0f, p1 = 0.0f, p2 = 0.0f, p3 = 0.0f;
    const int d4 = d & ~3;
    for (int t = 0; t < d4; t += 4) {
        p0 += x[t] * x[t];
        p1 += x[t + 1] * x[t + 1];
        p2 += x[t + 2] * x[t + 2];
        p3 += x[t + 3] * x[t + 3];
    }
    for (int t = d4; t < d; ++t) p0 += x[t] * x[t];
    float s = 0.0f;
    s += p0;
    s += p1;
    s += p2;
    s += p3;
    return s;
}

__attribute__((target("fma"))) inline float FusedDot(const float* c, const float* x, int d) {
    float s = 0.0f;
    for (int r = 0; r < d; ++r) s = std::fma(c[r], x[r], s);
    return s;
}

__attribute__((target("fma"))) void FusedDots(const float* C, int d, int H, const float* x, float* out) {
    for (int f = 0; f < H; ++f) out[f] = FusedDot(C + static_cast<std::size_t>(f) * d, x, d);
}

// Root candidates of one vector (beam_search.cpp:639-709): streaming top-`slots` over the root
// codes in ascending order, or the one given root (a forced root is a single finite slot).
// Root scores <c0_code, x> come from GemmRaw in the reference (beam_search.cpp:665); here they
// are the fused k-ordered dot of the device's root GEMM.
void RootCandidates(const float* x, int d, float nx2, const float* C0, const float* norm0, int h0, int slots,
                    const uint32_t* forced, float* rerr, int* rcode, float* ra0, float* rr00) {
    std::fill(rerr, rerr + slots, kInf);
    std::fill(rcode, rcode + slots, 0);
    std::fill(ra0, ra0 + slots, 0.0f);
    std::fill(rr00, rr00 + slots, 0.0f);
    auto root_score = [&](int code) { return FusedDot(C0 + static_cast<std::size_t>(code) * d, x, d); };
    if (forced) {
        const int code = static_cast<int>(*forced);
        const float alpha = norm0[code];
        if (alpha != 0.0f) {
            const float gamma = root_score(code);
            const float a1 = gamma / alpha;
            rerr[0] = nx2 - gamma * a1;
            rcode[0] = code;
            ra0[0] = a1;
            rr00[0] = std::sqrt(alpha);
        }
        return;
    }
    float worst;
    int wi = FirstMaxSlot(rerr, slots, &worst);
    for (int code = 0; code < h0; ++code) {
        const float alpha = norm0[code];
        if (alpha == 0.0f) continue;
        const float gamma = root_score(code);
        const float a1 = gamma / alpha;
        const float e1 = nx2 - gamma * a1;
        if (e1 >= worst) continue;
        rerr[wi] = e1;
        rcode[wi] = code;
        ra0[wi] = a1;
        rr00[wi] = std::sqrt(alpha);
        wi = FirstMaxSlot(rerr, slots, &worst);
    }
}

}  // namespace

extern "C" {

int orc_build_precomp(int d, int m, const int* h_vec, const float* C_all, float* G,
                      float* invnorm, int nthreads) {
    if (d <= 0 || m <= 0) return -1;
    SetThreads(nthreads);
    int H = 0;
    for (int l = 0; l < m; ++l) H += h_vec[l];
    // encoder_precomp.inc:28-40: invnorm = 1/sqrt(sum c^2) (0 for a zero codeword).
    for (int f = 0; f < H; ++f) {
        const float* c = C_all + static_cast<std::size_t>(f) * d;
        float norm_sq = 0.0f;
        for (int r = 0; r < d; ++r) norm_sq += c[r] * c[r];
        invnorm[f] = norm_sq > 0.0f ? 1.0f / std::sqrt(norm_sq) : 0.0f;
    }
    // encoder_precomp.inc:44-47: G = C_all^T C_all (sequential dot; symmetric by construction).
    #pragma omp parallel for schedule(dynamic, 16)
    for (int j = 0; j < H; ++j) {
        const float* cj = C_all + static_cast<std::size_t>(j) * d;
        for (int i = 0; i <= j; ++i) {
            const float* ci = C_all + static_cast<std::size_t>(i) * d;
            float s = 0.0f;
            for (int r = 0; r < d; ++r) s += ci[r] * cj[r];
            G[static_cast<std::size_t>(j) * H + i] = s;
            G[static_cast<std::size_t>(i) * H + j] = s;
        }
    }
    return 0;
}

void orc_xnorm2(const float* X, int d, int64_t n, float* out, int nthreads) {
    SetThreads(nthreads);
    #pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; ++i) {
        out[i] = SimdLane4SumSq(X + static_cast<std::size_t>(i) * d, d);
    }
}

void orc_gemm_xc(const float* C_all, int d, int H, const float* X, int64_t n, float* xC,
                 int mode, int nthreads) {
    SetThreads(nthreads);
    if (mode == 0) {
        #pragma omp parallel for schedule(static)
        for (int64_t i = 0; i < n; ++i) {
            const float* x = X + static_cast<std::size_t>(i) * d;
            float* out = xC + static_cast<std::size_t>(i) * H;
            for (int f = 0; f < H; ++f) {
                const float* c = C_all + static_cast<std::size_t>(f) * d;
                float s = 0.0f;
                for (int r = 0; r < d; ++r) s += c[r] * x[r];
                out[f] = s;
            }
        }
    } else {
        #pragma omp parallel for schedule(static)
        for (int64_t i = 0; i < n; ++i) {
            FusedDots(C_all, d, H, X + static_cast<std::size_t>(i) * d, xC + static_cast<std::size_t>(i) * H);
        }
    }
}

int orc_beam_search(const float* nx2, const float* xC, const float* G, int H, int m,
                    const int* h_vec, int H_beam, int64_t n, uint8_t* codes, float* best_err,
                    int nthreads) {
    if (m <= 0 || n < 0) return -1;
    SetThreads(nthreads);
    const int Hb = std::max(1, H_beam);
    const std::vector<int> off = Offsets(m, h_vec);
    #pragma omp parallel
    {
        Beam W(m, Hb);
        #pragma omp for schedule(static)
        for (int64_t i = 0; i < n; ++i) {
            const float* xCi = xC + static_cast<std::size_t>(i) * H;
            W.Reset();
            int cur = 0, nxt = 1;
            // Layer 0 (beam_search.cpp:240-261): e1 = ||x||^2 - gamma^2/alpha, alpha==0 skipped.
            float worst;
            int wi = FirstMaxSlot(W.err[nxt].data(), Hb, &worst);
            for (int k = 0; k < h_vec[0]; ++k) {
                const int f = off[0] + k;
                const float alpha = GAt(G, H, f, f);
                if (alpha == 0.0f) continue;
                const float gamma = xCi[f];
                const float a1 = gamma / alpha;
                const float e1 = nx2[i] - gamma * a1;
                if (e1 >= worst) continue;
                W.err[nxt][wi] = e1;
                W.Code(nxt, wi, 0) = static_cast<u8>(k);
                W.Coef(nxt, wi, 0) = a1;
                W.Chol(nxt, wi)[0] = std::sqrt(alpha);
                wi = FirstMaxSlot(W.err[nxt].data(), Hb, &worst);
            }
            int curH = CountFinite(W.err[nxt].data(), Hb);
            std::swap(cur, nxt);
            // Layers 1..m-1 (beam_search.cpp:272-407).
            for (int L = 1; L < m; ++L) {
                const int offL = off[L];
                const int cur_c = cur;
                curH = ExpandLayer<false>(
                    W, cur, nxt, L, h_vec[L], curH,
                    [&](int k) { return GAt(G, H, offL + k, offL + k); },
                    [&](int k) { return xCi[offL + k]; },
                    [&](int h, int t, int k) {
                        const int ft = off[t] + W.Code(cur_c, h, t);
                        return GAt(G, H, ft, offL + k);
                    });
                std::swap(cur, nxt);
            }
            const int best = BestSlot(W.err[cur].data(), curH);
            for (int L = 0; L < m; ++L) codes[static_cast<std::size_t>(i) * m + L] = W.Code(cur, best, L);
            if (best_err) best_err[i] = W.err[cur][best];
        }
    }
    return 0;
}

int64_t orc_solve_ls_all(const float* xC, const float* G, int H, int m, const int* h_vec,
                         const uint8_t* codes, int64_t n, float* a, int nthreads) {
    SetThreads(nthreads);
    const std::vector<int> off = Offsets(m, h_vec);
    int64_t fails = 0;
    #pragma omp parallel reduction(+ : fails)
    {
        std::vector<float> A(static_cast<std::size_t>(m) * m), b(m), x(m), y(m);
        #pragma omp for schedule(static)
        for (int64_t i = 0; i < n; ++i) {
            float* ai = a + static_cast<std::size_t>(i) * m;
            if (!SolveLsSample(xC + static_cast<std::size_t>(i) * H, G, H, m, off.data(),
                               codes + static_cast<std::size_t>(i) * m, ai, A.data(), b.data(),
                               x.data(), y.data())) {
                std::fill(ai, ai + m, 0.0f);  // least_squares.cpp:452-455
                ++fails;
            }
        }
    }
    return fails;
}

void orc_compute_costs(const float* xC, const float* G, int H, int m, const int* h_vec,
                       const uint8_t* codes, const float* a, const float* nx2, int64_t n,
                       float* cost, int nthreads) {
    SetThreads(nthreads);
    const std::vector<int> off = Offsets(m, h_vec);
    #pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; ++i) {
        cost[i] = SampleCost(xC + static_cast<std::size_t>(i) * H, G, H, m, off.data(),
                             codes + static_cast<std::size_t>(i) * m,
                             a + static_cast<std::size_t>(i) * m, nx2[i]);
    }
}

void orc_icm_orders(int m, int icm_iters, uint32_t seed, int* order_out) {
    std::mt19937 rng(static_cast<std::mt19937::result_type>(seed));
    std::vector<int> order(m);
    std::iota(order.begin(), order.end(), 0);
    for (int it = 0; it < icm_iters; ++it) {
        std::shuffle(order.begin(), order.end(), rng);
        std::copy(order.begin(), order.end(), order_out + static_cast<std::size_t>(it) * m);
    }
}

}  // extern "C"

namespace {

// RunIcm (icm.cpp:89-344) on codes/a/cost in place, with the layer order of each sweep given:
// LS refit and costs of the incoming codes, then icm_iters sweeps over the active vectors.
int64_t RunIcmOrders(const float* xC, const float* G, const float* invnorm, int H, int m, const int* h_vec,
                     const float* nx2, int64_t n, int icm_iters, int use_abs, const int* orders, uint8_t* codes,
                     float* a, float* cost, int nthreads) {
    const std::vector<int> off = Offsets(m, h_vec);
    // icm.cpp:109-114: LS refit and costs of the incoming codes.
    int64_t ls_fail = orc_solve_ls_all(xC, G, H, m, h_vec, codes, n, a, nthreads);
    orc_compute_costs(xC, G, H, m, h_vec, codes, a, nx2, n, cost, nthreads);
    std::vector<u8> active(static_cast<std::size_t>(n), 1), changed(static_cast<std::size_t>(n), 0);
    int max_h = 0;
    for (int l = 0; l < m; ++l) max_h = std::max(max_h, h_vec[l]);
    for (int it = 0; it < icm_iters; ++it) {
        std::fill(changed.begin(), changed.end(), 0);
        for (int oi = 0; oi < m; ++oi) {
            const int j = orders[static_cast<std::size_t>(it) * m + oi];
            if (j == 0) continue;  // icm.cpp:249-251: layer 0 is frozen
            const int startf = off[j];
            const int hj = h_vec[j];
            if (hj <= 1) continue;
            #pragma omp parallel reduction(+ : ls_fail)
            {
                std::vector<float> tmp(max_h), backup(m), A(static_cast<std::size_t>(m) * m), b(m), x(m), y(m);
                #pragma omp for schedule(static)
                for (int64_t i = 0; i < n; ++i) {
                    if (!active[i]) continue;
                    u8* ci = codes + static_cast<std::size_t>(i) * m;
                    float* ai = a + static_cast<std::size_t>(i) * m;
                    const float* xCi = xC + static_cast<std::size_t>(i) * H;
                    const int old_code = ci[j];
                    // icm.cpp:272-288: tmp = xC - sum_{l != j} a_l G(:, flat_l), l ascending.
                    for (int t = 0; t < hj; ++t) tmp[t] = xCi[startf + t];
                    for (int l = 0; l < m; ++l) {
                        if (l == j) continue;
                        const float al = ai[l];
                        const float* Gcol = G + static_cast<std::size_t>(off[l] + ci[l]) * H + startf;
                        for (int t = 0; t < hj; ++t) tmp[t] -= al * Gcol[t];
                    }
                    // icm.cpp:290-300: first max of (|)tmp*invnorm(|).
                    int best_code = old_code;
                    float best_score = -kInf;
                    for (int t = 0; t < hj; ++t) {
                        const float val = tmp[t] * invnorm[startf + t];
                        const float score = use_abs ? std::fabs(val) : val;
                        if (score > best_score) {
                            best_score = score;
                            best_code = t;
                        }
                    }
                    if (best_code == old_code) continue;
                    std::copy(ai, ai + m, backup.begin());
                    ci[j] = static_cast<u8>(best_code);
                    if (!SolveLsSample(xCi, G, H, m, off.data(), ci, ai, A.data(), b.data(), x.data(), y.data())) {
                        ci[j] = static_cast<u8>(old_code);
                        std::copy(backup.begin(), backup.end(), ai);
                        ++ls_fail;
                        continue;
                    }
                    const float new_cost = SampleCost(xCi, G, H, m, off.data(), ci, ai, nx2[i]);
                    if (new_cost + kEps < cost[i]) {  // icm.cpp:321-327
                        cost[i] = new_cost;
                        changed[i] = 1;
                    } else {
                        ci[j] = static_cast<u8>(old_code);
                        std::copy(backup.begin(), backup.end(), ai);
                    }
                }
            }
        }
        for (int64_t i = 0; i < n; ++i) {
            if (active[i] && !changed[i]) active[i] = 0;
        }
    }
    return ls_fail;
}

// icm.cpp:136-137 with the order reset of :121-123: each RunIcm starts from the identity order
// and shuffles it once per sweep with the caller's std::mt19937 stream.
std::vector<int> NextOrders(std::mt19937& rng, int m, int icm_iters) {
    std::vector<int> order(static_cast<std::size_t>(m)), out;
    std::iota(order.begin(), order.end(), 0);
    for (int it = 0; it < icm_iters; ++it) {
        std::shuffle(order.begin(), order.end(), rng);
        out.insert(out.end(), order.begin(), order.end());
    }
    return out;
}

// SplitMix64 and UniformBelow (icm.cpp:55-87): the ILS perturbation stream.
struct SplitMix64 {
    uint64_t state;
    uint64_t Next() {
        uint64_t z = (state += 0x9e3779b97f4a7c15ULL);
        z = (z ^ (z >> 30U)) * 0xbf58476d1ce4e5b9ULL;
        z = (z ^ (z >> 27U)) * 0x94d049bb133111ebULL;
        return z ^ (z >> 31U);
    }
};
inline uint32_t UniformBelow(SplitMix64& r, uint32_t bound) {
    return static_cast<uint32_t>((static_cast<unsigned __int128>(r.Next()) * bound) >> 64);
}

}  // namespace

extern "C" {

int64_t orc_icm(const float* xC, const float* G, const float* invnorm, int H, int m,
                const int* h_vec, const float* nx2, int64_t n, int icm_iters, int use_abs,
                uint32_t seed, uint8_t* codes, float* a, float* cost, int nthreads) {
    SetThreads(nthreads);
    std::vector<int> orders(static_cast<std::size_t>(m) * std::max(0, icm_iters));
    orc_icm_orders(m, icm_iters, seed, orders.data());
    return RunIcmOrders(xC, G, invnorm, H, m, h_vec, nx2, n, icm_iters, use_abs, orders.data(), codes, a, cost,
                        nthreads);
}

int64_t orc_icm_ils(const float* xC, const float* G, const float* invnorm, int H, int m, const int* h_vec,
                    const float* nx2, int64_t n, int icm_iters, int ils_iters, int perturb_k, int use_abs,
                    uint32_t seed, uint64_t sample_id_offset, uint8_t* codes, float* a, float* cost,
                    int nthreads) {
    SetThreads(nthreads);
    // DynamicIcmWithIlsImpl (icm.cpp:872-1003)
    std::mt19937 rng(static_cast<std::mt19937::result_type>(seed));
    std::vector<int> ord = NextOrders(rng, m, std::max(0, icm_iters));
    int64_t fails = RunIcmOrders(xC, G, invnorm, H, m, h_vec, nx2, n, icm_iters, use_abs, ord.data(), codes, a,
                                 cost, nthreads);
    if (ils_iters <= 0 || perturb_k <= 0 || m <= 1) return fails;
    const int ksel = std::min(perturb_k, m);
    const int layer_span = m - 1;
    std::vector<uint8_t> Bc(static_cast<std::size_t>(n) * m);
    std::vector<float> ac(static_cast<std::size_t>(n) * m), cc(static_cast<std::size_t>(n));
    for (int outer = 0; outer < ils_iters; ++outer) {
        std::memcpy(Bc.data(), codes, Bc.size());
        #pragma omp parallel for schedule(static)
        for (int64_t i = 0; i < n; ++i) {
            const uint64_t ig = sample_id_offset + static_cast<uint64_t>(i);
            SplitMix64 r{static_cast<uint64_t>(seed) ^ (static_cast<uint64_t>(outer + 1) * 0x9e3779b97f4a7c15ULL) ^
                         ((ig + 1) * 0xbf58476d1ce4e5b9ULL)};
            uint8_t* ci = Bc.data() + static_cast<std::size_t>(i) * m;
            for (int k = 0; k < ksel; ++k) {
                const int layer = 1 + static_cast<int>(UniformBelow(r, static_cast<uint32_t>(layer_span)));
                const int h = h_vec[layer];
                if (h <= 1) continue;
                const int old = ci[layer];
                const int raw = static_cast<int>(UniformBelow(r, static_cast<uint32_t>(h - 1)));
                ci[layer] = static_cast<uint8_t>(raw >= old ? raw + 1 : raw);
            }
        }
        ord = NextOrders(rng, m, std::max(0, icm_iters));
        fails += RunIcmOrders(xC, G, invnorm, H, m, h_vec, nx2, n, icm_iters, use_abs, ord.data(), Bc.data(),
                              ac.data(), cc.data(), nthreads);
        // accept if better (icm.cpp:977-987)
        #pragma omp parallel for schedule(static)
        for (int64_t i = 0; i < n; ++i) {
            if (cc[i] + kEps < cost[i]) {
                std::memcpy(codes + static_cast<std::size_t>(i) * m, Bc.data() + static_cast<std::size_t>(i) * m, m);
                std::memcpy(a + static_cast<std::size_t>(i) * m, ac.data() + static_cast<std::size_t>(i) * m,
                            sizeof(float) * m);
                cost[i] = cc[i];
            }
        }
    }
    return fails;
}

void orc_mse_from_precomp(const float* X, int d, const float* xC, const float* G, int H, int m,
                          const int* h_vec, const uint8_t* codes, const float* a, int64_t n,
                          double* per_vec, int nthreads) {
    SetThreads(nthreads);
    const std::vector<int> off = Offsets(m, h_vec);
    #pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; ++i) {
        const float* xi = X + static_cast<std::size_t>(i) * d;
        double nx = 0.0;
        for (int r = 0; r < d; ++r) nx += static_cast<double>(xi[r]) * xi[r];
        const u8* ci = codes + static_cast<std::size_t>(i) * m;
        const float* ai = a + static_cast<std::size_t>(i) * m;
        double t1 = 0.0, t2 = 0.0;
        for (int j = 0; j < m; ++j) t1 += static_cast<double>(ai[j]) * xC[static_cast<std::size_t>(i) * H + off[j] + ci[j]];
        for (int j = 0; j < m; ++j)
            for (int k = 0; k < m; ++k)
                t2 += static_cast<double>(ai[j]) * ai[k] * GAt(G, H, off[j] + ci[j], off[k] + ci[k]);
        double err = nx - 2.0 * t1 + t2;
        per_vec[i] = err < 0.0 ? 0.0 : err;
    }
}

void orc_mse_fp64_refit(const float* X, int d, const float* C_all, int H, int m,
                        const int* h_vec, const uint8_t* codes, int64_t n, double* per_vec,
                        int nthreads) {
    (void)H;
    SetThreads(nthreads);
    const std::vector<int> off = Offsets(m, h_vec);
    #pragma omp parallel
    {
        std::vector<double> Gm(static_cast<std::size_t>(m) * m), b(m), L(static_cast<std::size_t>(m) * m), z(m), w(m), rec(d);
        #pragma omp for schedule(static)
        for (int64_t i = 0; i < n; ++i) {
            const float* xi = X + static_cast<std::size_t>(i) * d;
            const u8* ci = codes + static_cast<std::size_t>(i) * m;
            std::vector<const float*> c(m);
            for (int l = 0; l < m; ++l) c[l] = C_all + static_cast<std::size_t>(off[l] + ci[l]) * d;
            double trace = 0.0;
            for (int p = 0; p < m; ++p) {
                double s = 0.0;
                for (int r = 0; r < d; ++r) s += static_cast<double>(c[p][r]) * xi[r];
                b[p] = s;
                for (int q = 0; q <= p; ++q) {
                    double g = 0.0;
                    for (int r = 0; r < d; ++r) g += static_cast<double>(c[p][r]) * c[q][r];
                    Gm[p * m + q] = g;
                    Gm[q * m + p] = g;
                }
                trace += Gm[p * m + p];
            }
            // Cholesky in fp64 with a tiny relative ridge for (near-)dependent code tuples.
            double ridge = 0.0;
            for (int attempt = 0; attempt < 8; ++attempt) {
                bool ok = true;
                for (int p = 0; p < m && ok; ++p) {
                    for (int q = 0; q <= p; ++q) {
                        double s = Gm[p * m + q] + (p == q ? ridge : 0.0);
                        for (int k = 0; k < q; ++k) s -= L[p * m + k] * L[q * m + k];
                        if (p == q) {
                            if (!(s > 0.0)) { ok = false; break; }
                            L[p * m + p] = std::sqrt(s);
                        } else {
                            L[p * m + q] = s / L[q * m + q];
                        }
                    }
                }
                if (ok) break;
                ridge = (ridge == 0.0 ? 1e-12 * (trace > 0 ? trace : 1.0) : ridge * 100.0);
            }
            for (int p = 0; p < m; ++p) {
                double s = b[p];
                for (int k = 0; k < p; ++k) s -= L[p * m + k] * z[k];
                z[p] = s / L[p * m + p];
            }
            for (int p = m - 1; p >= 0; --p) {
                double s = z[p];
                for (int k = p + 1; k < m; ++k) s -= L[k * m + p] * w[k];
                w[p] = s / L[p * m + p];
            }
            double err = 0.0;
            for (int r = 0; r < d; ++r) {
                double rr = 0.0;
                for (int l = 0; l < m; ++l) rr += w[l] * c[l][r];
                const double diff = static_cast<double>(xi[r]) - rr;
                err += diff * diff;
            }
            per_vec[i] = err;
        }
    }
}

int orc_build_precomp_large_root(int d, int h0, int Hs, const float* C0, const float* C_small,
                                 float* norm0, float* G_small, float* G0S, int nthreads) {
    SetThreads(nthreads);
    // precomp_large_root.cpp:82-90: norm0 = Norm2(c0) (the OpenMP-simd order of :14-23).
    for (int c = 0; c < h0; ++c) norm0[c] = SimdLane4SumSq(C0 + static_cast<std::size_t>(c) * d, d);
    // precomp_large_root.cpp:126-130: G_small = C_small^T C_small, G0S = C0^T C_small.
    #pragma omp parallel for schedule(dynamic, 16)
    for (int j = 0; j < Hs; ++j) {
        const float* cj = C_small + static_cast<std::size_t>(j) * d;
        for (int i = 0; i <= j; ++i) {
            const float* ci = C_small + static_cast<std::size_t>(i) * d;
            float s = 0.0f;
            for (int r = 0; r < d; ++r) s += ci[r] * cj[r];
            G_small[static_cast<std::size_t>(j) * Hs + i] = s;
            G_small[static_cast<std::size_t>(i) * Hs + j] = s;
        }
        for (int c = 0; c < h0; ++c) {
            const float* c0 = C0 + static_cast<std::size_t>(c) * d;
            float s = 0.0f;
            for (int r = 0; r < d; ++r) s += c0[r] * cj[r];
            G0S[static_cast<std::size_t>(j) * h0 + c] = s;
        }
    }
    return 0;
}

int orc_beam_search_large_root(const float* X, int d, const float* nx2, const float* C0,
                               const float* norm0, const float* xC_small, const float* G_small,
                               const float* G0S, int h0, int Hs, int m, const int* h_vec,
                               int H_beam, int64_t n, const uint32_t* forced_root, int root_mode,
                               uint32_t* cluster_id, uint8_t* B_small, float* best_err,
                               int nthreads) {
    if (m <= 0 || h0 <= 0) return -1;
    SetThreads(nthreads);
    const int Hb = std::max(1, H_beam);
    std::vector<int> small_off(m, 0);  // precomp_large_root.cpp:104-109
    {
        int o = 0;
        for (int l = 1; l < m; ++l) {
            small_off[l] = o;
            o += h_vec[l];
        }
    }
    const bool one_root = (forced_root != nullptr) || root_mode == 1;
    const int root_slots = one_root ? 1 : Hb;
    #pragma omp parallel
    {
        Beam W(m, Hb);
        std::vector<float> rerr(root_slots), ra0(root_slots), rr00(root_slots);
        std::vector<int> rcode(root_slots);
        #pragma omp for schedule(static)
        for (int64_t i = 0; i < n; ++i) {
            const float* x = X + static_cast<std::size_t>(i) * d;
            const float* xCi = xC_small + static_cast<std::size_t>(i) * Hs;
            RootCandidates(x, d, nx2[i], C0, norm0, h0, root_slots, forced_root ? &forced_root[i] : nullptr,
                           rerr.data(), rcode.data(), ra0.data(), rr00.data());
            // ExpandFromRootCandidates seeding (beam_search.cpp:760-793).
            W.Reset();
            int cur = 0, nxt = 1;
            int curH = 0;
            for (int h = 0; h < root_slots; ++h) {
                if (rerr[h] >= kInf) continue;
                W.err[cur][h] = rerr[h];
                W.root[cur][h] = static_cast<std::uint32_t>(rcode[h]);
                W.Coef(cur, h, 0) = ra0[h];
                W.Chol(cur, h)[0] = rr00[h];
                ++curH;
            }
            curH = std::max(1, curH);
            for (int L = 1; L < m; ++L) {
                const int offL = small_off[L];
                const int cur_c = cur;
                curH = ExpandLayer<true>(
                    W, cur, nxt, L, h_vec[L], curH,
                    [&](int k) { return GAt(G_small, Hs, offL + k, offL + k); },
                    [&](int k) { return xCi[offL + k]; },
                    [&](int h, int t, int k) {
                        if (t == 0) return GAt(G0S, h0, static_cast<int>(W.root[cur_c][h]), offL + k);
                        const int ft = small_off[t] + W.Code(cur_c, h, t);
                        return GAt(G_small, Hs, ft, offL + k);
                    });
                std::swap(cur, nxt);
            }
            const int best = BestSlot(W.err[cur].data(), curH);
            cluster_id[i] = W.root[cur][best];
            for (int L = 1; L < m; ++L)
                B_small[static_cast<std::size_t>(i) * (m - 1) + (L - 1)] = W.Code(cur, best, L);
            if (best_err) best_err[i] = W.err[cur][best];
        }
    }
    return 0;
}

int orc_large_root_candidates(const float* X, int d, const float* nx2, const float* C0, const float* norm0, int h0,
                              int H_beam, int64_t n, const uint32_t* forced_root, int root_mode, float* root_errs,
                              int* root_codes, float* root_a0, float* root_r00, int nthreads) {
    if (h0 <= 0 || H_beam <= 0) return -1;
    SetThreads(nthreads);
    const int slots = (forced_root != nullptr || root_mode == 1) ? 1 : H_beam;
    #pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; ++i) {
        const std::size_t o = static_cast<std::size_t>(i) * H_beam;
        std::fill(root_errs + o, root_errs + o + H_beam, kInf);
        std::fill(root_codes + o, root_codes + o + H_beam, 0);
        std::fill(root_a0 + o, root_a0 + o + H_beam, 0.0f);
        std::fill(root_r00 + o, root_r00 + o + H_beam, 0.0f);
        RootCandidates(X + static_cast<std::size_t>(i) * d, d, nx2[i], C0, norm0, h0, slots,
                       forced_root ? &forced_root[i] : nullptr, root_errs + o, root_codes + o, root_a0 + o,
                       root_r00 + o);
    }
    return 0;
}

}  // extern "C"

// ---------------------------------------------------------------------------------------------
// Large root: LS refit, costs and ICM/ILS with layer 0 fixed to the vector's root code.
namespace {

// Dot product in the reference build's OpenMP-simd order (least_squares.cpp:35-42 Dot,
// icm.cpp:67-74 DotF32, cost_utils.cpp:55-60): the four-lane order of SimdLane4SumSq.
inline float SimdLane4Dot(const float* a, const float* b, int d) {
    float p0 = 0.0f, p1 = 0.0f, p2 = 0.0f, p3 = 0.0f;
    const int d4 = d & ~3;
    for (int t = 0; t < d4; t += 4) {
        p0 += a[t] * b[t];
        p1 += a[t + 1] * b[t + 1];
        p2 += a[t + 2] * b[t + 2];
        p3 += a[t + 3] * b[t + 3];
    }
    for (int t = d4; t < d; ++t) p0 += a[t] * b[t];
    float s = 0.0f;
    s += p0;
    s += p1;
    s += p2;
    s += p3;
    return s;
}

// The large-root precomp and per-vector inputs (precomp_large_root.h:12-38). G0S is the
// reference's h0 x Hs column-major matrix: G0S(root, flat) = G0S[flat*h0 + root]; G_small is
// Hs x Hs column-major; B_small holds m-1 codes per vector (layers 1..m-1).
struct LrView {
    const float* X;
    int d;
    const float* C0;
    const float* norm0;
    int h0;
    const float* xCs;
    const float* Gs;
    const float* G0S;
    int Hs;
    int m;
    const int* h_vec;
    std::vector<int> soff;
    const uint32_t* cid;

    float G0SAt(uint32_t root, int flat) const { return G0S[static_cast<std::size_t>(flat) * h0 + root]; }
    float GsAt(int row, int col) const { return Gs[static_cast<std::size_t>(col) * Hs + row]; }
    const float* XCol(int64_t i) const { return xCs + static_cast<std::size_t>(i) * Hs; }
    float RootDot(int64_t i) const {
        return SimdLane4Dot(C0 + static_cast<std::size_t>(cid[i]) * d, X + static_cast<std::size_t>(i) * d, d);
    }
};

LrView MakeLrView(const float* X, int d, const float* C0, const float* norm0, int h0, const float* xCs,
                  const float* Gs, const float* G0S, int Hs, int m, const int* h_vec, const uint32_t* cid) {
    LrView v{X, d, C0, norm0, h0, xCs, Gs, G0S, Hs, m, h_vec, std::vector<int>(static_cast<std::size_t>(m), 0), cid};
    int o = 0;
    for (int l = 1; l < m; ++l) {  // precomp_large_root.cpp:95-98
        v.soff[l] = o;
        o += h_vec[l];
    }
    return v;
}

// least_squares.cpp:131-190 SolveLeastSquaresSampleLargeRootFixed (and its WithB0 twin,
// :192-250; the LAPACK variant :567-665 fills the same system): row 0 of the system is the
// root (norm0[cid], G0S(cid, .), b0 = <C0[:,cid], x>), rows 1..m-1 the small layers.
bool SolveLsSampleLargeRoot(const LrView& v, int64_t i, float b0, const u8* bs, float* a_out, float* A, float* b,
                            float* x, float* y) {
    const int m = v.m;
    const bool lapack_test = !(m == 5 || m == 10);
    const uint32_t c = v.cid[i];
    const float* xCi = v.XCol(i);
    auto fill = [&](float lambda) {
        std::fill(A, A + m * m, 0.0f);
        b[0] = b0;
        A[0] = v.norm0[c] + lambda;
        for (int j = 1; j < m; ++j) {
            const int fj = v.soff[j] + bs[j - 1];
            b[j] = xCi[fj];
            A[j] = v.G0SAt(c, fj);
            for (int k = 1; k <= j; ++k) A[k * m + j] = v.GsAt(v.soff[k] + bs[k - 1], fj);
            A[j * m + j] += lambda;
        }
    };
    fill(0.0f);
    bool ok = CholUpper(A, m, lapack_test);
    if (!ok) {
        float bump = kEps;
        for (int attempt = 0; attempt < 3 && !ok; ++attempt) {
            fill(bump);
            ok = CholUpper(A, m, lapack_test);
            bump *= 10.0f;
        }
    }
    if (!ok) return false;
    SolveUpper(A, m, m, b, x, y);
    std::copy(x, x + m, a_out);
    return true;
}

// cost_utils.cpp:42-84 SampleCostLargeRootFixed (the generic :160-209 has the same order):
// nx2 - 2*(a0*<c0,x> + sum_l a_l xC_l) + (a0*a0*norm0 + sum_j (2*a0*a_j*G0S + sum_k a_j a_k G)).
float SampleCostLargeRoot(const LrView& v, int64_t i, float xc0, const u8* bs, const float* a, float nx2) {
    const int m = v.m;
    const uint32_t c = v.cid[i];
    const float* xCi = v.XCol(i);
    float term1 = a[0] * xc0;
    for (int l = 1; l < m; ++l) term1 += a[l] * xCi[v.soff[l] + bs[l - 1]];
    float term2 = 0.0f;
    term2 += a[0] * a[0] * v.norm0[c];
    for (int j = 1; j < m; ++j) {
        const float aj = a[j];
        const int fj = v.soff[j] + bs[j - 1];
        term2 += 2.0f * a[0] * aj * v.G0SAt(c, fj);
        for (int k = 1; k < m; ++k) term2 += aj * a[k] * v.GsAt(fj, v.soff[k] + bs[k - 1]);
    }
    return nx2 - 2.0f * term1 + term2;
}

int64_t LsAllLargeRoot(const LrView& v, const u8* Bs, int64_t n, float* a) {
    const int m = v.m, mb = std::max(m - 1, 0);
    int64_t fails = 0;
    #pragma omp parallel reduction(+ : fails)
    {
        std::vector<float> A(static_cast<std::size_t>(m) * m), b(m), x(m), y(m);
        #pragma omp for schedule(static)
        for (int64_t i = 0; i < n; ++i) {
            float* ai = a + static_cast<std::size_t>(i) * m;
            if (!SolveLsSampleLargeRoot(v, i, v.RootDot(i), Bs + static_cast<std::size_t>(i) * mb, ai, A.data(),
                                        b.data(), x.data(), y.data())) {
                std::fill(ai, ai + m, 0.0f);  // least_squares.cpp:690-694
                ++fails;
            }
        }
    }
    return fails;
}

void CostsLargeRoot(const LrView& v, const u8* Bs, const float* a, const float* nx2, int64_t n, float* cost) {
    const int m = v.m, mb = std::max(m - 1, 0);
    #pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; ++i)
        cost[i] = SampleCostLargeRoot(v, i, v.RootDot(i), Bs + static_cast<std::size_t>(i) * mb,
                                      a + static_cast<std::size_t>(i) * m, nx2[i]);
}

// RunIcmLargeRoot (icm.cpp:347-870) with the sweep orders given: LS refit and costs, then
// icm_iters sweeps over layers 1..m-1 of the active vectors. The score of code t of layer j is
// (xC_small(t) - a0*G0S(cid, t) - sum_{l>=1, l!=j} a_l G_small(t, flat_l)) * invnorm_small(t),
// subtractions in that order (:437-503); b0 is cached once per vector (:381-389).
int64_t RunIcmLargeRootOrders(const LrView& v, const float* invs, const float* nx2, int64_t n, int icm_iters,
                              int use_abs, const int* orders, u8* Bs, float* a, float* cost) {
    const int m = v.m, mb = std::max(m - 1, 0);
    int64_t ls_fail = LsAllLargeRoot(v, Bs, n, a);
    CostsLargeRoot(v, Bs, a, nx2, n, cost);
    std::vector<float> b0(static_cast<std::size_t>(n));
    for (int64_t i = 0; i < n; ++i) b0[i] = v.RootDot(i);
    std::vector<u8> active(static_cast<std::size_t>(n), 1), changed(static_cast<std::size_t>(n), 0);
    int max_h = 0;
    for (int l = 0; l < m; ++l) max_h = std::max(max_h, v.h_vec[l]);
    for (int it = 0; it < icm_iters; ++it) {
        std::fill(changed.begin(), changed.end(), 0);
        for (int oi = 0; oi < m; ++oi) {
            const int j = orders[static_cast<std::size_t>(it) * m + oi];
            if (j == 0) continue;
            const int startf = v.soff[j];
            const int hj = v.h_vec[j];
            if (hj <= 1) continue;
            #pragma omp parallel reduction(+ : ls_fail)
            {
                std::vector<float> tmp(max_h), backup(m), A(static_cast<std::size_t>(m) * m), b(m), x(m), y(m);
                #pragma omp for schedule(static)
                for (int64_t i = 0; i < n; ++i) {
                    if (!active[i]) continue;
                    u8* bi = Bs + static_cast<std::size_t>(i) * mb;
                    float* ai = a + static_cast<std::size_t>(i) * m;
                    const float* xCi = v.XCol(i);
                    const uint32_t c = v.cid[i];
                    const int old_code = bi[j - 1];
                    for (int t = 0; t < hj; ++t) tmp[t] = xCi[startf + t];
                    const float a0 = ai[0];
                    for (int t = 0; t < hj; ++t) tmp[t] -= a0 * v.G0SAt(c, startf + t);
                    for (int l = 1; l < m; ++l) {
                        if (l == j) continue;
                        const float al = ai[l];
                        const int fl = v.soff[l] + bi[l - 1];
                        for (int t = 0; t < hj; ++t) tmp[t] -= al * v.GsAt(startf + t, fl);
                    }
                    int best_code = old_code;
                    float best_score = -kInf;
                    for (int t = 0; t < hj; ++t) {
                        const float val = tmp[t] * invs[startf + t];
                        const float score = use_abs ? std::fabs(val) : val;
                        if (score > best_score) {
                            best_score = score;
                            best_code = t;
                        }
                    }
                    if (best_code == old_code) continue;
                    std::copy(ai, ai + m, backup.begin());
                    bi[j - 1] = static_cast<u8>(best_code);
                    if (!SolveLsSampleLargeRoot(v, i, b0[i], bi, ai, A.data(), b.data(), x.data(), y.data())) {
                        bi[j - 1] = static_cast<u8>(old_code);
                        std::copy(backup.begin(), backup.end(), ai);
                        ++ls_fail;
                        continue;
                    }
                    const float new_cost = SampleCostLargeRoot(v, i, v.RootDot(i), bi, ai, nx2[i]);
                    if (new_cost + kEps < cost[i]) {  // icm.cpp:522-531, :601-611
                        cost[i] = new_cost;
                        changed[i] = 1;
                    } else {
                        bi[j - 1] = static_cast<u8>(old_code);
                        std::copy(backup.begin(), backup.end(), ai);
                    }
                }
            }
        }
        for (int64_t i = 0; i < n; ++i) {
            if (active[i] && !changed[i]) active[i] = 0;
        }
    }
    return ls_fail;
}

}  // namespace

extern "C" {

void orc_invnorm_small(const float* C_small, int d, int Hs, float* out) {
    for (int f = 0; f < Hs; ++f) {
        const float n2 = SimdLane4SumSq(C_small + static_cast<std::size_t>(f) * d, d);
        out[f] = n2 > 0.0f ? 1.0f / std::sqrt(n2) : 0.0f;
    }
}

int64_t orc_solve_ls_all_large_root(const float* X, int d, const float* C0, const float* norm0, int h0,
                                    const float* xC_small, const float* G_small, const float* G0S, int Hs, int m,
                                    const int* h_vec, const uint32_t* cluster_id, const uint8_t* B_small, int64_t n,
                                    float* a, int nthreads) {
    SetThreads(nthreads);
    const LrView v = MakeLrView(X, d, C0, norm0, h0, xC_small, G_small, G0S, Hs, m, h_vec, cluster_id);
    return LsAllLargeRoot(v, B_small, n, a);
}

void orc_compute_costs_large_root(const float* X, int d, const float* C0, const float* norm0, int h0,
                                  const float* xC_small, const float* G_small, const float* G0S, int Hs, int m,
                                  const int* h_vec, const uint32_t* cluster_id, const uint8_t* B_small,
                                  const float* a, const float* nx2, int64_t n, float* cost, int nthreads) {
    SetThreads(nthreads);
    const LrView v = MakeLrView(X, d, C0, norm0, h0, xC_small, G_small, G0S, Hs, m, h_vec, cluster_id);
    CostsLargeRoot(v, B_small, a, nx2, n, cost);
}

int64_t orc_icm_ils_large_root(const float* X, int d, const float* C0, const float* norm0, int h0,
                               const float* xC_small, const float* G_small, const float* G0S,
                               const float* invnorm_small, int Hs, int m, const int* h_vec,
                               const uint32_t* cluster_id, const float* nx2, int64_t n, int icm_iters, int ils_iters,
                               int perturb_k, int use_abs, uint32_t seed, uint64_t sample_id_offset,
                               uint8_t* B_small, float* a, float* cost, int nthreads) {
    SetThreads(nthreads);
    const LrView v = MakeLrView(X, d, C0, norm0, h0, xC_small, G_small, G0S, Hs, m, h_vec, cluster_id);
    // DynamicIcmWithIlsLargeRootImpl (icm.cpp:1005-1120)
    std::mt19937 rng(static_cast<std::mt19937::result_type>(seed));
    std::vector<int> ord = NextOrders(rng, m, std::max(0, icm_iters));
    int64_t fails = RunIcmLargeRootOrders(v, invnorm_small, nx2, n, icm_iters, use_abs, ord.data(), B_small, a, cost);
    if (ils_iters <= 0 || perturb_k <= 0 || m <= 1) return fails;
    const int mb = m - 1;
    const int ksel = std::min(perturb_k, m);
    std::vector<uint8_t> Bc(static_cast<std::size_t>(n) * mb);
    std::vector<float> ac(static_cast<std::size_t>(n) * m), cc(static_cast<std::size_t>(n));
    for (int outer = 0; outer < ils_iters; ++outer) {
        std::memcpy(Bc.data(), B_small, Bc.size());
        #pragma omp parallel for schedule(static)
        for (int64_t i = 0; i < n; ++i) {  // icm.cpp:1079-1098
            const uint64_t ig = sample_id_offset + static_cast<uint64_t>(i);
            SplitMix64 r{static_cast<uint64_t>(seed) ^ (static_cast<uint64_t>(outer + 1) * 0x9e3779b97f4a7c15ULL) ^
                         ((ig + 1) * 0xbf58476d1ce4e5b9ULL)};
            uint8_t* bi = Bc.data() + static_cast<std::size_t>(i) * mb;
            for (int k = 0; k < ksel; ++k) {
                const int layer = 1 + static_cast<int>(UniformBelow(r, static_cast<uint32_t>(mb)));
                const int h = h_vec[layer];
                if (h <= 1) continue;
                const int old = bi[layer - 1];
                const int raw = static_cast<int>(UniformBelow(r, static_cast<uint32_t>(h - 1)));
                bi[layer - 1] = static_cast<uint8_t>(raw >= old ? raw + 1 : raw);
            }
        }
        ord = NextOrders(rng, m, std::max(0, icm_iters));
        fails += RunIcmLargeRootOrders(v, invnorm_small, nx2, n, icm_iters, use_abs, ord.data(), Bc.data(),
                                       ac.data(), cc.data());
        #pragma omp parallel for schedule(static)
        for (int64_t i = 0; i < n; ++i) {  // icm.cpp:1104-1116
            if (cc[i] + kEps < cost[i]) {
                std::memcpy(B_small + static_cast<std::size_t>(i) * mb, Bc.data() + static_cast<std::size_t>(i) * mb,
                            mb);
                std::memcpy(a + static_cast<std::size_t>(i) * m, ac.data() + static_cast<std::size_t>(i) * m,
                            sizeof(float) * m);
                cost[i] = cc[i];
            }
        }
    }
    return fails;
}

}  // extern "C"
