// Beam launchers (BeamSearchPrefixLS and the large-root expansion): layer 0, the root seed and
// its NaN fix-up, the re-run list, and the dispatch of layers 1..19 to the translation units
// that build them (beam_kernels.hpp holds the kernels and the method).
#include "beam_kernels.hpp"

namespace stlq_mi355 {
namespace {

// Root candidates of the large-root beam (beam_search.cpp:639-709) seeded into beam records the
// way BeamSearchPrefixLSLargeRootExpandFromRootCandidates does (:760-793).
//  forced != null: the vector's root is given; its gamma is p.scores[i] (a 1-wide score row).
//  otherwise: streaming top-`root_slots` over ascending root codes of the score row
//  (root_slots == 1 forces the nearest root).
// e1 = ||x||^2 - gamma*(gamma/alpha), alpha = ||c0||^2, alpha == 0 skipped. A slot is seeded when
// its error is not +inf (NaN is seeded, as `errs0[h] >= inf` is false for NaN); curH = max(1, #seeded).
__global__ __launch_bounds__(256) void RootSeedKernel(RootArgs p) {
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    // i: the vector; w: its beam-state index (i, or its position in the re-run list)
    const int64_t w = static_cast<int64_t>(blockIdx.x) * kBeamWavesPerBlock + wave;
    int64_t i = w;
    if (p.list) {
        if (w >= *p.list_n) return;
        i = p.list[w];
    } else if (w >= p.n) {
        return;
    }
    const int m = p.m, Hb = p.Hb, rs = p.root_slots;
    const Rec rc(m);
    const float nx2 = p.nx2[i];
    float s_err = kInfF;
    int s_cand = -1;
    if (p.forced) {
        if (lane == 0 && p.forced[i] != kNoRoot) {
            const int code = static_cast<int>(p.forced[i]);
            const float alpha = p.norm0[code];
            if (alpha != 0.0f) {
                const float gamma = p.scores[i * p.ldx];
                const float a1 = gamma / alpha;
                s_err = nx2 - gamma * a1;
                s_cand = code;
            }
        }
    } else {
        const float* sc = p.scores + i * p.ldx;
        bool unused_flag = false;
        SelectTopH<false, false, false>(
            rs, lane,
            [&](auto&& replay, auto, auto) {
                for (int c0 = 0; c0 < p.h0; c0 += kWave) {
                    const int code = c0 + lane;
                    const bool act = code < p.h0;
                    const float alpha = act ? p.norm0[code] : 0.0f;
                    const bool ok = act && alpha != 0.0f;
                    const float gamma = act ? sc[code] : 0.0f;
                    const float a1 = gamma / alpha;
                    const float e1 = nx2 - gamma * a1;
                    if (!replay(ok, e1, c0 + lane)) return false;
                }
                return true;
            },
            s_err, s_cand, unused_flag);
    }
    const bool seeded = lane < rs && !(s_err >= kInfF);
    const int curH = max(1, __popcll(__ballot(seeded)));
    float a0 = 0.0f, r00 = 0.0f;
    prune::SlotBounds bd = prune::NoBounds();
    uint32_t root = 0;
    if (seeded) {
        root = static_cast<uint32_t>(s_cand);
        const float alpha = p.norm0[s_cand];
        const float gamma = p.forced ? p.scores[i * p.ldx] : p.scores[i * p.ldx + s_cand];
        a0 = gamma / alpha;
        r00 = sqrtf(alpha);
        bd = prune::FirstBounds(r00, p.sw0[s_cand], a0, p.isw0[s_cand]);
    }
    if (lane < Hb) {
        float* rec = p.out.rec + (w * Hb + lane) * rc.stride;
        rec[0] = seeded ? s_err : kInfF;
        rec[rc.coef] = a0;
        rec[Rec::R(0, 0)] = r00;
        rec[Rec::Rinv(0)] = 1.0f / r00;
        reinterpret_cast<uint32_t*>(rec + rc.code)[0] = 0u;
        reinterpret_cast<uint32_t*>(rec)[rc.root] = root;
        rc.PutBounds(rec, bd);
    }
    if (lane == 0) p.out.curH[w] = curH;
    if (p.is_last) {  // m == 1: the root is the whole code
        const int best = BestSlot(seeded ? s_err : kInfF, curH, lane);
        if (lane == best) {
            p.cluster_out[i] = root;
            if (p.best_err) p.best_err[i] = seeded ? s_err : kInfF;
        }
    }
}

// gamma of a given root per vector: fused k-ordered dot product s = fma(c0[r], x[r], s), the
// accumulation order of the MFMA score GEMM, so forced and scanned roots see the same gamma.
__global__ __launch_bounds__(256) void GatherRootDotKernel(const float* __restrict__ X, int d,
                                                           const float* __restrict__ C0,
                                                           const uint32_t* __restrict__ roots, int64_t n,
                                                           float* __restrict__ out) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= n) return;
    if (roots[i] == kNoRoot) {
        out[i] = 0.0f;
        return;
    }
    const float* x = X + i * d;
    const float* c = C0 + static_cast<int64_t>(roots[i]) * d;
    float s = 0.0f;
    for (int r = 0; r < d; ++r) s = __builtin_fmaf(c[r], x[r], s);
    out[i] = s;
}

// The vectors NearestRootKernel flagged (a NaN error met): the root scan of RootSeedKernel with
// one slot, in ascending code order with the reference's NaN rules, on root scores computed here
// as fused k-ordered dot products (GatherRootDotKernel's order, the MFMA GEMM's bits). A grid of
// waves strides over the vectors; unflagged ones cost one byte read.
__global__ __launch_bounds__(256) void NearestRootFixupKernel(const float* __restrict__ X, int d,
                                                              const float* __restrict__ C0, int h0,
                                                              const float* __restrict__ norm0,
                                                              const float* __restrict__ nx2,
                                                              const uint8_t* __restrict__ flag, int64_t n,
                                                              uint32_t* __restrict__ root_out) {
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kBeamWavesPerBlock;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * kBeamWavesPerBlock + wave; i < n; i += stride) {
        if (!flag[i]) continue;
        const float* x = X + i * d;
        const float xn = nx2[i];
        float s_err;
        int s_cand;
        bool unused_flag = false;
        SelectTopH<false, false, false>(
            1, lane,
            [&](auto&& replay, auto, auto) {
                for (int c0 = 0; c0 < h0; c0 += kWave) {
                    const int code = c0 + lane;
                    const bool act = code < h0;
                    const float alpha = act ? norm0[code] : 0.0f;
                    const bool ok = act && alpha != 0.0f;
                    float gamma = 0.0f;
                    if (act) {
                        const float* c = C0 + static_cast<int64_t>(code) * d;
                        for (int r = 0; r < d; ++r) gamma = __builtin_fmaf(c[r], x[r], gamma);
                    }
                    const float a1 = gamma / alpha;
                    const float e1 = xn - gamma * a1;
                    if (!replay(ok, e1, c0 + lane)) return false;
                }
                return true;
            },
            s_err, s_cand, unused_flag);
        (void)s_err;
        if (lane == 0) root_out[i] = s_cand >= 0 ? static_cast<uint32_t>(s_cand) : kNoRoot;
    }
}

}  // namespace


int BeamRecordStride(int m) { return Rec(m).stride; }

namespace {

// Appends the index of every flagged vector to list (in no particular order) and adds the count
// to counts[0] and counts[1]. One atomic add per wave that holds a flagged vector.
__global__ __launch_bounds__(256) void CollectFlaggedKernel(const uint8_t* __restrict__ flags, int64_t n,
                                                            int* __restrict__ list, int* __restrict__ counts) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    const int lane = threadIdx.x & 63;
    const bool f = i < n && flags[i] != 0;
    const uint64_t mask = Ballot(f);
    if (mask == 0ull) return;
    int base = 0;
    if (lane == 0) {
        base = atomicAdd(&counts[0], __popcll(mask));
        atomicAdd(&counts[1], __popcll(mask));
    }
    base = __shfl(base, 0);
    if (f) list[base + __popcll(mask & ((1ull << lane) - 1ull))] = static_cast<int>(i);
}

}  // namespace

hipError_t LaunchCollectFlagged(const uint8_t* flags, int64_t n, int* list, int* counts, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(CollectFlaggedKernel, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0, s, flags, n,
                       list, counts);
    return hipGetLastError();
}

hipError_t LaunchRootSeed(const RootArgs& a, hipStream_t s) {
    if (a.n <= 0) return hipSuccess;
    const unsigned blocks = static_cast<unsigned>((a.n + kBeamWavesPerBlock - 1) / kBeamWavesPerBlock);
    hipLaunchKernelGGL(RootSeedKernel, dim3(blocks), dim3(kWave * kBeamWavesPerBlock), 0, s, a);
    return hipGetLastError();
}

hipError_t LaunchNearestRootFixup(const float* X, int d, const float* C0, int h0, const float* norm0,
                                  const float* nx2, const uint8_t* flag, int64_t n, uint32_t* root_out, hipStream_t s) {
    if (n <= 0 || h0 <= 0) return hipSuccess;
    const int64_t waves = std::min<int64_t>(n, 8192);
    const unsigned blocks = static_cast<unsigned>((waves + kBeamWavesPerBlock - 1) / kBeamWavesPerBlock);
    hipLaunchKernelGGL(NearestRootFixupKernel, dim3(blocks), dim3(kBeamWavesPerBlock * kWave), 0, s, X, d, C0, h0,
                       norm0, nx2, flag, n, root_out);
    return hipGetLastError();
}

hipError_t LaunchGatherRootDot(const float* X, int d, const float* C0, const uint32_t* roots, int64_t n, float* out,
                               hipStream_t s) {
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(GatherRootDotKernel, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0, s, X, d, C0,
                       roots, n, out);
    return hipGetLastError();
}

hipError_t LaunchBeamLayer0(const LayerArgs& a, hipStream_t s) {
    if (a.n <= 0) return hipSuccess;
    const unsigned blocks = static_cast<unsigned>((a.n + kBeamWavesPerBlock - 1) / kBeamWavesPerBlock);
    if (a.flags) hipLaunchKernelGGL(Layer0Kernel<true>, dim3(blocks), dim3(kWave * kBeamWavesPerBlock), 0, s, a);
    else hipLaunchKernelGGL(Layer0Kernel<false>, dim3(blocks), dim3(kWave * kBeamWavesPerBlock), 0, s, a);
    return hipGetLastError();
}

hipError_t LaunchBeamLayer(int L, bool large_root, const LayerArgs& a, hipStream_t s) {
    if (a.n <= 0) return hipSuccess;
    if (L >= 1 && L <= kQueueMaxL) return LaunchQueueLayer(L, large_root, a, s);
    if (L <= 13) return LaunchStagedLayerA(L, large_root, a, s);
    return LaunchStagedLayerB(L, large_root, a, s);
}

}  // namespace stlq_mi355
