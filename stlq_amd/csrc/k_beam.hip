// Prefix-least-squares beam search, one layer per launch (src/quantizer/beam_search.cpp:196-422
// for the full precomp, :728-992 for the large-root expansion).
//
// Mapping: one wave64 owns one vector. For every live beam (slot order) the 64 lanes evaluate
// the layer's codewords k = lane + 64*j with the reference's exact arithmetic (no FMA
// contraction, IEEE division, same operation order), so every candidate error is bit-identical
// to the CPU encoder's given the same xC, G and ||x||^2. The reference keeps the beam with a
// streaming "replace the first worst slot" rule (beam_search.cpp:101-113, :320-333); lanes
// 0..H_beam-1 hold those slots and the wave replays the rule in scan order: a ballot finds the
// next candidate that beats the current worst, it is written into the worst slot, and the worst
// is recomputed with a DPP max reduction. The surviving candidates are then re-evaluated once
// (same arithmetic, so same bits) to build the next layer's codes, LS coefficients and
// Cholesky factor.
#include "internal.hpp"

namespace stlq_mi355 {
namespace {

constexpr float kInfF = __builtin_huge_valf();
constexpr int kMaxChunks = kMaxK / kWave;  // 4 chunks of 64 codewords

__device__ __forceinline__ float ReadLane(float v, int l) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}
__device__ __forceinline__ int ReadLaneI(int v, int l) { return __builtin_amdgcn_readlane(v, l); }

template <int CTRL>
__device__ __forceinline__ float Dpp(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), CTRL, 0xF, 0xF, false));
}

// Max over the 64 lanes, returned wave-uniform. quad_perm(1,0,3,2), quad_perm(2,3,0,1),
// row_half_mirror, row_mirror reduce each 16-lane row; the four row results are combined.
__device__ __forceinline__ float WaveMax(float v) {
    v = fmaxf(v, Dpp<0xB1>(v));
    v = fmaxf(v, Dpp<0x4E>(v));
    v = fmaxf(v, Dpp<0x141>(v));
    v = fmaxf(v, Dpp<0x140>(v));
    return fmaxf(fmaxf(ReadLane(v, 0), ReadLane(v, 16)), fmaxf(ReadLane(v, 32), ReadLane(v, 48)));
}
__device__ __forceinline__ float WaveMin(float v) {
    v = fminf(v, Dpp<0xB1>(v));
    v = fminf(v, Dpp<0x4E>(v));
    v = fminf(v, Dpp<0x141>(v));
    v = fminf(v, Dpp<0x140>(v));
    return fminf(fminf(ReadLane(v, 0), ReadLane(v, 16)), fminf(ReadLane(v, 32), ReadLane(v, 48)));
}

// RecomputeWorst (beam_search.cpp:101-113): scan from slot 0 keeping the first slot whose error
// is strictly greater. Comparisons with NaN are false, so a NaN in slot 0 pins the worst to
// (NaN, 0) and a NaN elsewhere is never chosen.
__device__ __forceinline__ void RecomputeWorst(float s_err, int Hb, int lane, float& worst, int& widx) {
    const float e0 = ReadLane(s_err, 0);
    if (__builtin_isnan(e0)) {
        worst = e0;
        widx = 0;
        return;
    }
    const bool in = lane < Hb;
    const float v = (in && !__builtin_isnan(s_err)) ? s_err : -kInfF;
    const float mx = WaveMax(v);
    const uint64_t eq = __ballot(in && s_err == mx);
    widx = static_cast<int>(__builtin_ctzll(eq));
    worst = mx;
}

// Replays the streaming top-H over one chunk of 64 candidates in lane (= scan) order.
// Candidate `lane` is eligible when ok; it is inserted when !(e >= worst)
// (beam_search.cpp:320: `if (e >= worst_err) continue;`).
__device__ __forceinline__ void ReplayChunk(bool ok, float e, int cand_base, int Hb, int lane,
                                            float& s_err, int& s_cand, float& worst, int& widx) {
    uint64_t mask = __ballot(ok && !(e >= worst));
    while (mask) {
        const int l = static_cast<int>(__builtin_ctzll(mask));
        const float ev = ReadLane(e, l);
        if (lane == widx) {
            s_err = ev;
            s_cand = cand_base + l;
        }
        RecomputeWorst(s_err, Hb, lane, worst, widx);
        const uint64_t later = (l >= 63) ? 0ull : (~0ull << (l + 1));
        mask = __ballot(ok && !(e >= worst)) & later;
    }
}

// BestSlot (beam_search.cpp:409-416): first minimum over slots [0, curH) with strict '<'.
__device__ __forceinline__ int BestSlot(float err, int curH, int lane) {
    if (curH <= 1) return 0;
    const float e0 = ReadLane(err, 0);
    if (__builtin_isnan(e0)) return 0;
    const bool in = lane < curH;
    const float v = (in && !__builtin_isnan(err)) ? err : kInfF;
    const float mn = WaveMin(v);
    const uint64_t eq = __ballot(in && err == mn);
    return eq ? static_cast<int>(__builtin_ctzll(eq)) : 0;
}

// One prefix-LS candidate (beam_search.cpp:291-318): forward U^T y = A, backward U v = y
// (linear_algebra.cpp:57-77; the large-root expansion multiplies by 1/diag instead,
// beam_search.cpp:544-547/569-572), delta = A.v, eta = A.a_old, then
// a_last = (gamma - eta)/(alpha - delta), e = max(E_old - diff*a_last, 0).
template <int L, bool RECIP, typename RFn, typename RinvFn>
__device__ __forceinline__ void EvalCand(RFn R, RinvFn rinv, const float (&A)[L], const float (&aold)[L],
                                         float E_old, float alpha, float gamma, float (&y)[L],
                                         float (&v)[L], float& e, float& denom, float& a_last,
                                         bool& ok) {
#pragma unroll
    for (int r = 0; r < L; ++r) {
        float s = A[r];
#pragma unroll
        for (int j = 0; j < r; ++j) s = s - R(j, r) * y[j];
        y[r] = RECIP ? s * rinv(r) : s / R(r, r);
    }
#pragma unroll
    for (int r = L - 1; r >= 0; --r) {
        float s = y[r];
#pragma unroll
        for (int j = r + 1; j < L; ++j) s = s - R(r, j) * v[j];
        v[r] = RECIP ? s * rinv(r) : s / R(r, r);
    }
    float delta = 0.0f, eta = 0.0f;
#pragma unroll
    for (int t = 0; t < L; ++t) {
        delta = delta + A[t] * v[t];
        eta = eta + A[t] * aold[t];
    }
    denom = alpha - delta;
    ok = denom != 0.0f;
    const float diff = gamma - eta;
    a_last = diff / denom;
    const float ee = E_old - diff * a_last;
    e = ee < 0.0f ? 0.0f : ee;
}

// Layer 0 of the full-precomp beam (beam_search.cpp:240-263).
__global__ __launch_bounds__(256) void Layer0Kernel(LayerArgs p) {
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int64_t i = static_cast<int64_t>(blockIdx.x) * kBeamWavesPerBlock + wave;
    if (i >= p.n) return;
    const int m = p.m, Hb = p.Hb, K = p.K, off0 = p.offL;
    const int TRI = TriSize(m), CS = CodeStride(m);
    const float nx2 = p.nx2[i];
    const float* xCi = p.xC + i * p.ldx;

    float s_err = kInfF;
    int s_cand = -1;
    float worst = kInfF;
    int widx = 0;
    const int nch = (K + kWave - 1) / kWave;
    for (int j = 0; j < nch; ++j) {
        const int k = lane + kWave * j;
        const bool act = k < K;
        const float alpha = act ? p.gdiag[off0 + k] : 0.0f;
        const bool ok = act && alpha != 0.0f;
        const float gamma = act ? xCi[off0 + k] : 0.0f;
        const float a1 = gamma / alpha;
        const float e1 = nx2 - gamma * a1;
        ReplayChunk(ok, e1, kWave * j, Hb, lane, s_err, s_cand, worst, widx);
    }

    const int curH = __popcll(__ballot(lane < Hb && s_err < kInfF));  // CountFinite, no max(1,.)
    // Insertion-time write-back of the surviving slot contents (beam_search.cpp:253-258).
    uint8_t c0 = 0;
    float a0 = 0.0f, r00 = 0.0f;
    if (lane < Hb && s_cand >= 0) {
        const float alpha = p.gdiag[off0 + s_cand];
        const float gamma = xCi[off0 + s_cand];
        c0 = static_cast<uint8_t>(s_cand);
        a0 = gamma / alpha;
        r00 = sqrtf(alpha);
    }
    if (lane < Hb) {
        const int64_t so = i * Hb + lane;
        p.out.err[so] = s_err;
        p.out.code[so * CS] = c0;
        p.out.coef[so * m] = a0;
        p.out.R[so * TRI] = r00;
    }
    if (lane == 0) p.out.curH[i] = curH;
    if (p.is_last) {
        const int best = BestSlot(s_err, curH, lane);
        if (lane == best) {
            p.codes_out[i * m] = c0;
            if (p.best_err) p.best_err[i] = s_err;
        }
    }
}

// Layers L >= 1. LR selects the large-root cross-term source and reciprocal solves.
template <int L, bool LR>
__global__ __launch_bounds__(256) void LayerKernel(LayerArgs p) {
    constexpr bool RECIP = LR;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int64_t i = static_cast<int64_t>(blockIdx.x) * kBeamWavesPerBlock + wave;
    if (i >= p.n) return;
    const int m = p.m, Hb = p.Hb, K = p.K, offL = p.offL;
    const int TRI = TriSize(m), CS = CodeStride(m);
    const int64_t ld = p.gram.ld;
    const float* xCi = p.xC + i * p.ldx;
    const int nch = (K + kWave - 1) / kWave;

    float gam[kMaxChunks], alp[kMaxChunks];
#pragma unroll
    for (int j = 0; j < kMaxChunks; ++j) {
        const int k = lane + kWave * j;
        const bool act = j < nch && k < K;
        gam[j] = act ? xCi[offL + k] : 0.0f;
        alp[j] = act ? p.gdiag[offL + k] : 0.0f;
    }

    float s_err = kInfF;
    int s_cand = -1;
    float worst = kInfF;
    int widx = 0;
    const int curH = p.in.curH[i];

    for (int h = 0; h < curH; ++h) {
        const int64_t sb = i * Hb + h;
        const float E_old = p.in.err[sb];
        const float* Rp = p.in.R + sb * TRI;
        const float* ap = p.in.coef + sb * m;
        const uint8_t* cp = p.in.code + sb * CS;
        float aold[L];
        const float* rows[L];
#pragma unroll
        for (int t = 0; t < L; ++t) {
            aold[t] = ap[t];
            if (LR && t == 0) {
                rows[t] = p.gram.G0S + static_cast<int64_t>(p.in.root[sb]) * ld + offL;
            } else {
                rows[t] = p.gram.G + static_cast<int64_t>(p.gram.off[t] + cp[t]) * ld + offL;
            }
        }
        float Rv[L][L];
        float Ri[L];
#pragma unroll
        for (int r = 0; r < L; ++r) {
#pragma unroll
            for (int c = r; c < L; ++c) Rv[r][c] = Rp[TriIdx(m, r, c)];
            Ri[r] = RECIP ? 1.0f / Rv[r][r] : 0.0f;
        }
        auto Rf = [&](int r, int c) { return Rv[r][c]; };
        auto Rif = [&](int r) { return Ri[r]; };

        float ech[kMaxChunks];
        bool okc[kMaxChunks];
#pragma unroll
        for (int j = 0; j < kMaxChunks; ++j) {
            ech[j] = kInfF;
            okc[j] = false;
            if (j < nch) {
                const int k = lane + kWave * j;
                const bool act = k < K;
                float A[L];
#pragma unroll
                for (int t = 0; t < L; ++t) A[t] = act ? rows[t][k] : 0.0f;
                float y[L], v[L], denom, a_last;
                bool ok;
                EvalCand<L, RECIP>(Rf, Rif, A, aold, E_old, alp[j], gam[j], y, v, ech[j], denom, a_last, ok);
                okc[j] = act && ok;
            }
        }
#pragma unroll
        for (int j = 0; j < kMaxChunks; ++j) {
            if (j < nch) ReplayChunk(okc[j], ech[j], h * K + kWave * j, Hb, lane, s_err, s_cand, worst, widx);
        }
    }

    // Deferred write-back (beam_search.cpp:337-383) or the all-skipped fallback (:385-400).
    const int newH = __popcll(__ballot(lane < Hb && s_err < kInfF));
    int outH;
    float out_err = kInfF;
    uint8_t ncode[L + 1];
    uint32_t nroot = 0;
#pragma unroll
    for (int t = 0; t <= L; ++t) ncode[t] = 0;
    if (newH == 0) {
        const int nh = min(curH, Hb);
        outH = max(1, nh);
        if (lane < nh) {
            const int64_t si = i * Hb + lane;
            const int64_t so = si;
            out_err = p.in.err[si];
            const uint8_t* cp = p.in.code + si * CS;
            const float* ap = p.in.coef + si * m;
            const float* Rp = p.in.R + si * TRI;
            uint8_t* co = p.out.code + so * CS;
            float* ao = p.out.coef + so * m;
            float* Ro = p.out.R + so * TRI;
#pragma unroll
            for (int t = 0; t < L; ++t) {
                ncode[t] = cp[t];
                co[t] = cp[t];
                ao[t] = ap[t];
            }
            co[L] = 0;
            ao[L] = 0.0f;
#pragma unroll
            for (int r = 0; r < L; ++r) {
#pragma unroll
                for (int c = r; c < L; ++c) Ro[TriIdx(m, r, c)] = Rp[TriIdx(m, r, c)];
                Ro[TriIdx(m, r, L)] = 0.0f;
            }
            Ro[TriIdx(m, L, L)] = 0.0f;
            if (LR) {
                nroot = p.in.root[si];
                p.out.root[so] = nroot;
            }
        } else if (nh == 0 && lane == 0) {
            // No beam at all (layer 0 had no finite candidate): the reference's next-buffer slot 0
            // keeps its never-written (zero) state with error +inf.
            const int64_t so = i * Hb;
            uint8_t* co = p.out.code + so * CS;
            float* ao = p.out.coef + so * m;
            float* Ro = p.out.R + so * TRI;
#pragma unroll
            for (int t = 0; t <= L; ++t) {
                co[t] = 0;
                ao[t] = 0.0f;
            }
#pragma unroll
            for (int r = 0; r <= L; ++r)
#pragma unroll
                for (int c = r; c <= L; ++c) Ro[TriIdx(m, r, c)] = 0.0f;
            if (LR) p.out.root[so] = 0;
        }
    } else {
        outH = max(1, newH);
        const bool live = lane < Hb && !(s_err >= kInfF);
        if (live) {
            const int src = s_cand / K;
            const int k = s_cand - src * K;
            const int64_t si = i * Hb + src;
            const int64_t so = i * Hb + lane;
            const float* Rp = p.in.R + si * TRI;
            const float* ap = p.in.coef + si * m;
            const uint8_t* cp = p.in.code + si * CS;
            float Rv[L][L], Ri[L], aold[L], A[L];
            if (LR) nroot = p.in.root[si];
#pragma unroll
            for (int r = 0; r < L; ++r) {
#pragma unroll
                for (int c = r; c < L; ++c) Rv[r][c] = Rp[TriIdx(m, r, c)];
                Ri[r] = RECIP ? 1.0f / Rv[r][r] : 0.0f;
            }
#pragma unroll
            for (int t = 0; t < L; ++t) {
                aold[t] = ap[t];
                ncode[t] = cp[t];
                const float* row = (LR && t == 0)
                                       ? p.gram.G0S + static_cast<int64_t>(nroot) * ld + offL
                                       : p.gram.G + static_cast<int64_t>(p.gram.off[t] + cp[t]) * ld + offL;
                A[t] = row[k];
            }
            ncode[L] = static_cast<uint8_t>(k);
            auto Rf = [&](int r, int c) { return Rv[r][c]; };
            auto Rif = [&](int r) { return Ri[r]; };
            float y[L], v[L], e, denom, a_last;
            bool ok;
            EvalCand<L, RECIP>(Rf, Rif, A, aold, p.in.err[si], p.gdiag[offL + k], xCi[offL + k], y, v, e,
                               denom, a_last, ok);
            out_err = s_err;
            uint8_t* co = p.out.code + so * CS;
            float* ao = p.out.coef + so * m;
            float* Ro = p.out.R + so * TRI;
#pragma unroll
            for (int t = 0; t < L; ++t) {
                co[t] = ncode[t];
                ao[t] = aold[t] - v[t] * a_last;
            }
            co[L] = ncode[L];
            ao[L] = a_last;
#pragma unroll
            for (int r = 0; r < L; ++r) {
#pragma unroll
                for (int c = r; c < L; ++c) Ro[TriIdx(m, r, c)] = Rv[r][c];
                Ro[TriIdx(m, r, L)] = y[r];
            }
            Ro[TriIdx(m, L, L)] = sqrtf(denom);
            if (LR) p.out.root[so] = nroot;
        }
    }
    if (lane < Hb) p.out.err[i * Hb + lane] = out_err;
    if (lane == 0) p.out.curH[i] = outH;

    if (p.is_last) {
        const int best = BestSlot(out_err, outH, lane);
        if (lane == best) {
            if (LR) {
                p.cluster_out[i] = nroot;
#pragma unroll
                for (int t = 1; t <= L; ++t) p.codes_out[i * (m - 1) + (t - 1)] = ncode[t];
            } else {
#pragma unroll
                for (int t = 0; t <= L; ++t) p.codes_out[i * m + t] = ncode[t];
            }
            if (p.best_err) p.best_err[i] = out_err;
        }
    }
}

template <int L>
hipError_t LaunchL(bool lr, const LayerArgs& a, hipStream_t s) {
    const unsigned blocks = static_cast<unsigned>((a.n + kBeamWavesPerBlock - 1) / kBeamWavesPerBlock);
    if (lr) {
        hipLaunchKernelGGL((LayerKernel<L, true>), dim3(blocks), dim3(kWave * kBeamWavesPerBlock), 0, s, a);
    } else {
        hipLaunchKernelGGL((LayerKernel<L, false>), dim3(blocks), dim3(kWave * kBeamWavesPerBlock), 0, s, a);
    }
    return hipGetLastError();
}

}  // namespace

hipError_t LaunchBeamLayer0(const LayerArgs& a, hipStream_t s) {
    if (a.n <= 0) return hipSuccess;
    const unsigned blocks = static_cast<unsigned>((a.n + kBeamWavesPerBlock - 1) / kBeamWavesPerBlock);
    hipLaunchKernelGGL(Layer0Kernel, dim3(blocks), dim3(kWave * kBeamWavesPerBlock), 0, s, a);
    return hipGetLastError();
}

hipError_t LaunchBeamLayer(int L, bool large_root, const LayerArgs& a, hipStream_t s) {
    if (a.n <= 0) return hipSuccess;
    switch (L) {
        case 1: return LaunchL<1>(large_root, a, s);
        case 2: return LaunchL<2>(large_root, a, s);
        case 3: return LaunchL<3>(large_root, a, s);
        case 4: return LaunchL<4>(large_root, a, s);
        case 5: return LaunchL<5>(large_root, a, s);
        case 6: return LaunchL<6>(large_root, a, s);
        case 7: return LaunchL<7>(large_root, a, s);
        case 8: return LaunchL<8>(large_root, a, s);
        case 9: return LaunchL<9>(large_root, a, s);
        case 10: return LaunchL<10>(large_root, a, s);
        case 11: return LaunchL<11>(large_root, a, s);
        case 12: return LaunchL<12>(large_root, a, s);
        case 13: return LaunchL<13>(large_root, a, s);
        case 14: return LaunchL<14>(large_root, a, s);
        case 15: return LaunchL<15>(large_root, a, s);
        case 16: return LaunchL<16>(large_root, a, s);
        case 17: return LaunchL<17>(large_root, a, s);
        case 18: return LaunchL<18>(large_root, a, s);
        case 19: return LaunchL<19>(large_root, a, s);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace stlq_mi355
