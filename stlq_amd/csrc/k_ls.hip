// Per-vector least-squares refit, cost, and ICM layer sweeps.
//
//  * LsAllKernel     SolveLeastSquaresAll (src/quantizer/least_squares.cpp:406-565)
//  * CostsKernel     ComputeCosts / SampleCost (src/quantizer/cost_utils.cpp:112-158)
//  * IcmLayerKernel  one layer of RunIcm (src/quantizer/icm.cpp:249-329)
//  * *LargeRoot*     the same for a large root: SolveLeastSquaresAllLargeRoot
//                    (least_squares.cpp:667-745), ComputeCostsLargeRoot (cost_utils.cpp:211-233),
//                    one layer of RunIcmLargeRoot (icm.cpp:347-870)
//  * PerturbKernel, IlsAcceptKernel   the ILS rounds (icm.cpp:944-1001, :1070-1116)
//
// The Cholesky is the hand-written one of least_squares.cpp:44-84 (row-major upper factor,
// true division, retry with diagonal bumps 1e-6, 1e-5, 1e-4). Its failure test is the
// reference's `sum <= 1e-6` for m in {5,10}; for other m the reference calls LAPACK spotrf,
// whose failure test (pivot <= 0 or NaN) is used here with the same hand-written arithmetic.
#include "internal.hpp"

namespace stlq_mi355 {
namespace {

constexpr float kEps = 1e-6f;
constexpr float kInfF = __builtin_huge_valf();

template <int M>
__device__ __forceinline__ bool CholUpper(float (&A)[M * M]) {
    constexpr bool kLapackTest = !(M == 5 || M == 10);
#pragma unroll
    for (int k = 0; k < M; ++k) {
        float sum = A[k * M + k];
#pragma unroll
        for (int j = 0; j < k; ++j) {
            const float v = A[j * M + k];
            sum = sum - v * v;
        }
        if (kLapackTest ? !(sum > 0.0f) : (sum <= kEps)) return false;
        const float diag = sqrtf(sum);
        A[k * M + k] = diag;
#pragma unroll
        for (int i = k + 1; i < M; ++i) {
            float s = A[k * M + i];
#pragma unroll
            for (int j = 0; j < k; ++j) s = s - A[j * M + k] * A[j * M + i];
            A[k * M + i] = s / diag;
        }
    }
    return true;
}

template <int M>
__device__ __forceinline__ void SolveUpper(const float (&A)[M * M], const float (&b)[M], float (&x)[M]) {
    float y[M];
#pragma unroll
    for (int i = 0; i < M; ++i) {
        float s = b[i];
#pragma unroll
        for (int k = 0; k < i; ++k) s = s - A[k * M + i] * y[k];
        y[i] = s / A[i * M + i];
    }
#pragma unroll
    for (int i = M - 1; i >= 0; --i) {
        float s = y[i];
#pragma unroll
        for (int k = i + 1; k < M; ++k) s = s - A[i * M + k] * x[k];
        x[i] = s / A[i * M + i];
    }
}

// Flat code of each layer of one vector. Large root: layer 0 is the root (flat[0] unused) and
// the stored codes start at layer 1.
template <int M, bool LR>
__device__ __forceinline__ void Flats(const LsArgs& p, const uint8_t* __restrict__ c, int (&flat)[M]) {
#pragma unroll
    for (int l = 0; l < M; ++l) {
        if constexpr (LR) {
            flat[l] = l == 0 ? 0 : p.off[l] + c[l - 1];
        } else {
            flat[l] = p.off[l] + c[l];
        }
    }
}

// SolveLeastSquaresSampleFixed (least_squares.cpp:86-129) for one vector; for a large root
// SolveLeastSquaresSampleLargeRootFixed[WithB0] (:131-250), whose row 0 is the root:
// A(0,0) = norm0[root], A(0,j) = G0S(root, flat_j), b0 = <C0[:,root], x>.
template <int M, bool LR>
__device__ __forceinline__ bool SolveLs(const LsArgs& p, const float* __restrict__ xCi, const int (&flat)[M],
                                        uint32_t root, float b0, float (&x)[M]) {
    float A[M * M];
    float b[M];
    auto fill = [&](float lambda) {
#pragma unroll
        for (int q = 0; q < M * M; ++q) A[q] = 0.0f;
        if constexpr (LR) {
            const float* g0 = p.G0S_rm + static_cast<int64_t>(root) * p.H;
            b[0] = b0;
            A[0] = p.norm0[root] + lambda;
#pragma unroll
            for (int j = 1; j < M; ++j) {
                b[j] = xCi[flat[j]];
                A[j] = g0[flat[j]];
#pragma unroll
                for (int k = 1; k <= j; ++k) A[k * M + j] = p.G_rm[static_cast<int64_t>(flat[k]) * p.H + flat[j]];
                A[j * M + j] = A[j * M + j] + lambda;
            }
        } else {
#pragma unroll
            for (int j = 0; j < M; ++j) {
                b[j] = xCi[flat[j]];
#pragma unroll
                for (int k = 0; k <= j; ++k) A[k * M + j] = p.G_rm[static_cast<int64_t>(flat[k]) * p.H + flat[j]];
                A[j * M + j] = A[j * M + j] + lambda;
            }
        }
    };
    fill(0.0f);
    bool ok = CholUpper<M>(A);
    if (!ok) {
        float bump = kEps;
        for (int attempt = 0; attempt < 3 && !ok; ++attempt) {
            fill(bump);
            ok = CholUpper<M>(A);
            bump = bump * 10.0f;
        }
    }
    if (!ok) return false;
    SolveUpper<M>(A, b, x);
    return true;
}

// SampleCost (cost_utils.cpp:112-137): nx2 - 2*sum a_l xC_l + sum_l sum_k a_l a_k G(l,k).
// Large root (SampleCostLargeRootFixed, :42-84): term1 = a0*<c0,x> + sum_{l>=1} a_l xC_l and
// term2 = a0*a0*norm0 + sum_{j>=1} (2*a0*a_j*G0S(root,j) + sum_{k>=1} a_j a_k G(j,k)).
template <int M, bool LR>
__device__ __forceinline__ float Cost(const LsArgs& p, const float* __restrict__ xCi, const int (&flat)[M],
                                      uint32_t root, float xc0, const float (&a)[M], float nx2) {
    if constexpr (LR) {
        const float* g0 = p.G0S_rm + static_cast<int64_t>(root) * p.H;
        float term1 = a[0] * xc0;
#pragma unroll
        for (int l = 1; l < M; ++l) term1 = term1 + a[l] * xCi[flat[l]];
        float term2 = 0.0f;
        term2 = term2 + (a[0] * a[0]) * p.norm0[root];
#pragma unroll
        for (int j = 1; j < M; ++j) {
            const float aj = a[j];
            term2 = term2 + ((2.0f * a[0]) * aj) * g0[flat[j]];
            const float* Grow = p.G_rm + static_cast<int64_t>(flat[j]) * p.H;
#pragma unroll
            for (int k = 1; k < M; ++k) term2 = term2 + (aj * a[k]) * Grow[flat[k]];
        }
        return nx2 - 2.0f * term1 + term2;
    } else {
        float term1 = 0.0f, term2 = 0.0f;
#pragma unroll
        for (int l = 0; l < M; ++l) {
            const float al = a[l];
            term1 = term1 + al * xCi[flat[l]];
            const float* Grow = p.G_rm + static_cast<int64_t>(flat[l]) * p.H;
#pragma unroll
            for (int k = 0; k < M; ++k) term2 = term2 + (al * a[k]) * Grow[flat[k]];
        }
        return nx2 - 2.0f * term1 + term2;
    }
}

template <int M, bool LR>
__device__ __forceinline__ void LsAllBody(const LsArgs& p) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= p.n) return;
    int flat[M];
    Flats<M, LR>(p, p.codes + i * p.cstride, flat);
    const uint32_t root = LR ? p.root[i] : 0u;
    const float b0 = LR ? p.b0[i] : 0.0f;
    const float* xCi = p.xC + i * p.ldx;
    float x[M];
    float* ai = p.a + i * M;
    if (SolveLs<M, LR>(p, xCi, flat, root, b0, x)) {
#pragma unroll
        for (int l = 0; l < M; ++l) ai[l] = x[l];
    } else {
#pragma unroll
        for (int l = 0; l < M; ++l) ai[l] = 0.0f;  // least_squares.cpp:452-455, :690-694
        if (p.fails) atomicAdd(p.fails, 1);
    }
}

template <int M, bool LR>
__device__ __forceinline__ void CostsBody(const LsArgs& p) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= p.n) return;
    int flat[M];
    Flats<M, LR>(p, p.codes + i * p.cstride, flat);
    float a[M];
#pragma unroll
    for (int l = 0; l < M; ++l) a[l] = p.a[i * M + l];
    p.cost[i] = Cost<M, LR>(p, p.xC + i * p.ldx, flat, LR ? p.root[i] : 0u, LR ? p.b0[i] : 0.0f, a, p.nx2[i]);
}

template <int M>
__global__ __launch_bounds__(256) void LsAllKernel(LsArgs p) { LsAllBody<M, false>(p); }
template <int M>
__global__ __launch_bounds__(256) void LsAllLargeRootKernel(LsArgs p) { LsAllBody<M, true>(p); }
template <int M>
__global__ __launch_bounds__(256) void CostsKernel(LsArgs p) { CostsBody<M, false>(p); }
template <int M>
__global__ __launch_bounds__(256) void CostsLargeRootKernel(LsArgs p) { CostsBody<M, true>(p); }

__device__ __forceinline__ float ReadLane(float v, int l) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}
template <int CTRL>
__device__ __forceinline__ float Dpp(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float WaveMax(float v) {
    v = fmaxf(v, Dpp<0xB1>(v));
    v = fmaxf(v, Dpp<0x4E>(v));
    v = fmaxf(v, Dpp<0x141>(v));
    v = fmaxf(v, Dpp<0x140>(v));
    return fmaxf(fmaxf(ReadLane(v, 0), ReadLane(v, 16)), fmaxf(ReadLane(v, 32), ReadLane(v, 48)));
}

// One ICM layer update (icm.cpp:259-328), one wave per vector. Lanes score codes
// t = lane + 64*jj of layer j:
//   val(t) = (xC(start+t) - sum_{l != j} a_l G(start+t, flat_l)) * invnorm(start+t)
// (subtractions in ascending l), pick the first maximum of val (or |val|), and if it differs
// from the current code, propose it in pend[i]; IcmSolveBody then re-solves LS and accepts iff
// new_cost + 1e-6 < cost. For a large root
// (RunIcmLargeRoot, icm.cpp:437-611) layer 0's term is a0*G0S(root, start+t), the G and
// invnorm arrays are the small layers' (G_small is symmetric, so its rows serve as columns),
// and b0 is the vector's cached <C0[:,root], x>.
template <int M, bool LR>
__device__ __forceinline__ void IcmLayerBody(const IcmArgs& q) {
    const LsArgs& p = q.ls;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int64_t i = static_cast<int64_t>(blockIdx.x) * 4 + wave;
    if (i >= p.n) return;
    // The vector's flag, codes and coefficients are read together, before the flag is tested,
    // so an active vector waits for one memory round trip here, not two.
    const bool active = q.active[i] != 0;
    const int j = q.j, hj = q.hj;
    const int start = p.off[j];
    uint8_t* ci = q.codes_rw + i * p.cstride;
    const int jc = LR ? j - 1 : j;  // position of layer j among the stored codes
    float* ai = p.a + i * M;
    const float* xCi = p.xC + i * p.ldx;
    const uint32_t root = LR ? p.root[i] : 0u;
    int flat[M];
    float a[M];
    Flats<M, LR>(p, ci, flat);
#pragma unroll
    for (int l = 0; l < M; ++l) a[l] = ai[l];
    const int old_code = ci[jc];
    if (!active) return;
    const float* g0 = LR ? p.G0S_rm + static_cast<int64_t>(root) * p.H : nullptr;

    // All (at most four) chunks of 64 codes are scored before any reduction, so their loads are
    // in flight together.
    constexpr int kChunks = 4;  // layers hold at most 256 codewords
    float score[kChunks];
#pragma unroll
    for (int c = 0; c < kChunks; ++c) {
        const int t = 64 * c + lane;
        score[c] = -kInfF;
        if (t < hj) {
            float tmp = xCi[start + t];
            if constexpr (LR) tmp = tmp - a[0] * g0[start + t];
            // Layer j's own term is loaded and multiplied but not subtracted (x - (+0) == x), so
            // all M loads are unconditional and in flight together.
#pragma unroll
            for (int l = LR ? 1 : 0; l < M; ++l) {
                const float prod = a[l] * q.G_cm[static_cast<int64_t>(flat[l]) * p.H + start + t];
                tmp = tmp - (l == j ? 0.0f : prod);
            }
            const float val = tmp * q.invnorm[start + t];
            const float sc = q.use_abs ? fabsf(val) : val;
            score[c] = __builtin_isnan(sc) ? -kInfF : sc;  // NaN never wins a strict '>' scan
        }
    }
    // The scan's first maximum (strict '>' in ascending code order): the wave maximum, then the
    // lowest code that attains it.
    float lane_max = score[0];
#pragma unroll
    for (int c = 1; c < kChunks; ++c) lane_max = fmaxf(lane_max, score[c]);
    const float best_val = WaveMax(lane_max);
    int best_t = 0x7fffffff;
    if (best_val > -kInfF) {
#pragma unroll
        for (int c = kChunks - 1; c >= 0; --c) {
            const uint64_t eq = __ballot(64 * c + lane < hj && score[c] == best_val);
            if (eq) best_t = 64 * c + static_cast<int>(__builtin_ctzll(eq));
        }
    }
    const int best_code = (best_val > -kInfF) ? best_t : old_code;
    if (lane == 0) q.pend[i] = best_code == old_code ? -1 : best_code;
}

// The LS re-solve and acceptance of one ICM layer update (icm.cpp:300-328), one thread per
// vector: the scoring above proposed code pend[i] (or nothing). A thread per vector instead of
// lane 0 of the scoring wave keeps 64 times more of these latency-bound solves in flight.
template <int M, bool LR>
__device__ __forceinline__ void IcmSolveBody(const IcmArgs& q) {
    const LsArgs& p = q.ls;
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= p.n) return;
    if (!q.active[i]) return;
    const int best_code = q.pend[i];
    if (best_code < 0) return;
    const int j = q.j;
    const int start = p.off[j];
    uint8_t* ci = q.codes_rw + i * p.cstride;
    const int jc = LR ? j - 1 : j;
    float* ai = p.a + i * M;
    const float* xCi = p.xC + i * p.ldx;
    const uint32_t root = LR ? p.root[i] : 0u;
    const float b0 = LR ? p.b0[i] : 0.0f;
    int flat[M];
    Flats<M, LR>(p, ci, flat);
    int nflat[M];
#pragma unroll
    for (int l = 0; l < M; ++l) nflat[l] = (l == j) ? start + best_code : flat[l];
    float x[M];
    if (!SolveLs<M, LR>(p, xCi, nflat, root, b0, x)) {
        atomicAdd(q.fails, 1);
        return;  // icm.cpp:313-318: roll back (nothing was written)
    }
    const float new_cost = Cost<M, LR>(p, xCi, nflat, root, b0, x, p.nx2[i]);
    if (new_cost + kEps < p.cost[i]) {
        ci[jc] = static_cast<uint8_t>(best_code);
#pragma unroll
        for (int l = 0; l < M; ++l) ai[l] = x[l];
        p.cost[i] = new_cost;
        q.changed[i] = 1;
    }
}

template <int M>
__global__ __launch_bounds__(256) void IcmLayerKernel(IcmArgs q) { IcmLayerBody<M, false>(q); }
template <int M>
__global__ __launch_bounds__(256) void IcmLayerLargeRootKernel(IcmArgs q) { IcmLayerBody<M, true>(q); }
template <int M>
__global__ __launch_bounds__(256) void IcmSolveKernel(IcmArgs q) { IcmSolveBody<M, false>(q); }
template <int M>
__global__ __launch_bounds__(256) void IcmSolveLargeRootKernel(IcmArgs q) { IcmSolveBody<M, true>(q); }

__global__ void DeactivateKernel(uint8_t* active, const uint8_t* changed, int64_t n) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i < n && active[i] && !changed[i]) active[i] = 0;
}

// ILS perturbation (icm.cpp:946-972): per vector a SplitMix64 stream keyed by the seed, the round
// and the global sample id picks min(perturb_k, m) (layer, new code) pairs in layers 1..m-1,
// each new code uniform over the layer's codes other than the current one (Lemire multiply-high).
struct PerturbArgs {
    uint8_t* codes;  // [n*cstride], perturbed in place
    int64_t n;
    int m, ksel;
    int cstride, lfirst;  // codes per vector and the layer of the first stored code
    int h_vec[kMaxM];
    uint32_t seed;
    int outer;
    uint64_t id0;  // global id of vector 0
};

__device__ __forceinline__ uint64_t SplitMixNext(uint64_t& st) {
    uint64_t z = (st += 0x9e3779b97f4a7c15ULL);
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ULL;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebULL;
    return z ^ (z >> 31);
}
__device__ __forceinline__ uint32_t UniformBelow(uint64_t& st, uint32_t bound) {
    return static_cast<uint32_t>(__umul64hi(SplitMixNext(st), static_cast<uint64_t>(bound)));
}

__global__ __launch_bounds__(256) void PerturbKernel(PerturbArgs p) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= p.n) return;
    const uint64_t ig = p.id0 + static_cast<uint64_t>(i);
    uint64_t st = static_cast<uint64_t>(p.seed) ^ (static_cast<uint64_t>(p.outer + 1) * 0x9e3779b97f4a7c15ULL) ^
                  ((ig + 1ULL) * 0xbf58476d1ce4e5b9ULL);
    uint8_t* ci = p.codes + i * p.cstride;  // layer l's code at ci[l - lfirst]
    const uint32_t span = static_cast<uint32_t>(p.m - 1);
    for (int r = 0; r < p.ksel; ++r) {
        const int layer = 1 + static_cast<int>(UniformBelow(st, span));
        const int h = p.h_vec[layer];
        if (h <= 1) continue;
        const int old = ci[layer - p.lfirst];
        const int raw = static_cast<int>(UniformBelow(st, static_cast<uint32_t>(h - 1)));
        ci[layer - p.lfirst] = static_cast<uint8_t>(raw >= old ? raw + 1 : raw);
    }
}

// Accept-if-better of one ILS round (icm.cpp:977-987, :1104-1116): the candidate replaces the
// vector's codes (cstride per vector), coefficients (m) and cost when cand + 1e-6 < cost.
__global__ __launch_bounds__(256) void IlsAcceptKernel(uint8_t* codes, float* a, float* cost, const uint8_t* cc,
                                                      const float* ca, const float* ccost, int64_t n, int m,
                                                      int cstride) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= n) return;
    if (ccost[i] + kEps < cost[i]) {
        for (int l = 0; l < cstride; ++l) codes[i * cstride + l] = cc[i * cstride + l];
        for (int l = 0; l < m; ++l) a[i * m + l] = ca[i * m + l];
        cost[i] = ccost[i];
    }
}

#define STLQ_LAUNCH_M(KER, M_, grid, block, s, a) \
    hipLaunchKernelGGL((KER<M_>), grid, block, 0, s, a)

#define STLQ_SWITCH_M(KER, m, grid, block, s, a)                  \
    switch (m) {                                                  \
        case 1: STLQ_LAUNCH_M(KER, 1, grid, block, s, a); break;  \
        case 2: STLQ_LAUNCH_M(KER, 2, grid, block, s, a); break;  \
        case 3: STLQ_LAUNCH_M(KER, 3, grid, block, s, a); break;  \
        case 4: STLQ_LAUNCH_M(KER, 4, grid, block, s, a); break;  \
        case 5: STLQ_LAUNCH_M(KER, 5, grid, block, s, a); break;  \
        case 6: STLQ_LAUNCH_M(KER, 6, grid, block, s, a); break;  \
        case 7: STLQ_LAUNCH_M(KER, 7, grid, block, s, a); break;  \
        case 8: STLQ_LAUNCH_M(KER, 8, grid, block, s, a); break;  \
        case 9: STLQ_LAUNCH_M(KER, 9, grid, block, s, a); break;  \
        case 10: STLQ_LAUNCH_M(KER, 10, grid, block, s, a); break; \
        case 11: STLQ_LAUNCH_M(KER, 11, grid, block, s, a); break; \
        case 12: STLQ_LAUNCH_M(KER, 12, grid, block, s, a); break; \
        case 13: STLQ_LAUNCH_M(KER, 13, grid, block, s, a); break; \
        case 14: STLQ_LAUNCH_M(KER, 14, grid, block, s, a); break; \
        case 15: STLQ_LAUNCH_M(KER, 15, grid, block, s, a); break; \
        case 16: STLQ_LAUNCH_M(KER, 16, grid, block, s, a); break; \
        case 17: STLQ_LAUNCH_M(KER, 17, grid, block, s, a); break; \
        case 18: STLQ_LAUNCH_M(KER, 18, grid, block, s, a); break; \
        case 19: STLQ_LAUNCH_M(KER, 19, grid, block, s, a); break; \
        case 20: STLQ_LAUNCH_M(KER, 20, grid, block, s, a); break; \
        default: return hipErrorInvalidValue;                     \
    }

}  // namespace

hipError_t LaunchLsAll(const LsArgs& a, hipStream_t s) {
    if (a.n <= 0) return hipSuccess;
    const dim3 grid(static_cast<unsigned>((a.n + 255) / 256)), block(256);
    if (a.root) {
        STLQ_SWITCH_M(LsAllLargeRootKernel, a.m, grid, block, s, a);
    } else {
        STLQ_SWITCH_M(LsAllKernel, a.m, grid, block, s, a);
    }
    return hipGetLastError();
}

hipError_t LaunchCosts(const LsArgs& a, hipStream_t s) {
    if (a.n <= 0) return hipSuccess;
    const dim3 grid(static_cast<unsigned>((a.n + 255) / 256)), block(256);
    if (a.root) {
        STLQ_SWITCH_M(CostsLargeRootKernel, a.m, grid, block, s, a);
    } else {
        STLQ_SWITCH_M(CostsKernel, a.m, grid, block, s, a);
    }
    return hipGetLastError();
}

hipError_t LaunchIcmLayer(const IcmArgs& a, hipStream_t s) {
    if (a.ls.n <= 0) return hipSuccess;
    const dim3 grid(static_cast<unsigned>((a.ls.n + 3) / 4)), block(256);
    const dim3 grid_solve(static_cast<unsigned>((a.ls.n + 255) / 256));
    if (a.ls.root) {
        STLQ_SWITCH_M(IcmLayerLargeRootKernel, a.ls.m, grid, block, s, a);
        STLQ_SWITCH_M(IcmSolveLargeRootKernel, a.ls.m, grid_solve, block, s, a);
    } else {
        STLQ_SWITCH_M(IcmLayerKernel, a.ls.m, grid, block, s, a);
        STLQ_SWITCH_M(IcmSolveKernel, a.ls.m, grid_solve, block, s, a);
    }
    return hipGetLastError();
}

hipError_t LaunchPerturb(uint8_t* codes, int64_t n, int m, int cstride, int lfirst, const int* h_vec, int perturb_k,
                         uint32_t seed, int outer, uint64_t id0, hipStream_t s) {
    if (n <= 0 || m <= 1 || perturb_k <= 0) return hipSuccess;
    PerturbArgs p;
    p.codes = codes;
    p.n = n;
    p.m = m;
    p.cstride = cstride;
    p.lfirst = lfirst;
    p.ksel = perturb_k < m ? perturb_k : m;
    for (int l = 0; l < m; ++l) p.h_vec[l] = h_vec[l];
    p.seed = seed;
    p.outer = outer;
    p.id0 = id0;
    hipLaunchKernelGGL(PerturbKernel, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0, s, p);
    return hipGetLastError();
}

hipError_t LaunchIlsAccept(uint8_t* codes, float* a, float* cost, const uint8_t* cc, const float* ca, const float* ccost,
                           int64_t n, int m, int cstride, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(IlsAcceptKernel, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0, s, codes, a, cost,
                       cc, ca, ccost, n, m, cstride);
    return hipGetLastError();
}

hipError_t LaunchIcmDeactivate(uint8_t* active, const uint8_t* changed, int64_t n, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(DeactivateKernel, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0, s, active,
                       changed, n);
    return hipGetLastError();
}

}  // namespace stlq_mi355
