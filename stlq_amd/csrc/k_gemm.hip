// xC = C_all^T X on fp32 MFMA (v_mfma_f32_16x16x4_f32): the codeword-distance contraction
// (StreamKernelProvider::Gemm call sites encoder_encode_base.inc:86-90,
// encode_base_streaming.cpp:846/2610; cuBLAS in the reference, kernel_provider_cuda_stream_impl.inc:392-444).
//
// Output layout is the reference's xC column: for vector i, xC[i*ldx + f] = <x_i, c_f>.
// Both operands are K-contiguous (d), so the kernel is an "NT" GEMM: rows = vectors,
// cols = codewords. A 256-thread workgroup computes a 128x128 tile; each wave owns a 64x64
// sub-tile as 4x4 MFMA blocks. d is staged through LDS in slices of 16 with double buffering;
// inside a slice each lane's float4 LDS read feeds four consecutive MFMAs (k = 4s + lane/16),
// so the accumulation order over k is strictly ascending in blocks of 4.
#include "internal.hpp"

namespace stlq_mi355 {
namespace {

typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int kBM = 128;
constexpr int kBN = 128;
constexpr int kBK = 16;
constexpr int kLdsStride = kBK + 4;  // 20 floats: conflict-free float4 reads across 8 rows

struct Staged {
    float v[2][4];
};

// Loads this thread's share of a 128 x 16 slice (2 rows x 4 consecutive k) of a K-contiguous
// matrix with `rows` rows and row length d. kInterior: the tile is known to lie inside the matrix
// and d is a multiple of 16, so every load is an unconditional float4 (no exec-mask branches).
template <bool kInterior>
__device__ __forceinline__ void LoadSlice(const float* __restrict__ M, int64_t rows, int d, int64_t r0,
                                          int k0, bool vec4, Staged& st) {
    const int t = threadIdx.x;
    const int quad = t & 3;
#pragma unroll
    for (int q = 0; q < 2; ++q) {
        const int64_t row = r0 + (t >> 2) + 64 * q;
        const int k = k0 + 4 * quad;
        if (kInterior || (row < rows && vec4 && k + 3 < d)) {
            const float4 x = *reinterpret_cast<const float4*>(M + row * d + k);
            st.v[q][0] = x.x;
            st.v[q][1] = x.y;
            st.v[q][2] = x.z;
            st.v[q][3] = x.w;
        } else {
#pragma unroll
            for (int e = 0; e < 4; ++e) st.v[q][e] = (row < rows && k + e < d) ? M[row * d + k + e] : 0.0f;
        }
    }
}

// Stores a staged slice into LDS with k permuted: local k = 4s + g lands at position 4g + s.
__device__ __forceinline__ void StoreSlice(float (*S)[kLdsStride], const Staged& st) {
    const int t = threadIdx.x;
    const int quad = t & 3;
#pragma unroll
    for (int q = 0; q < 2; ++q) {
        const int row = (t >> 2) + 64 * q;
#pragma unroll
        for (int e = 0; e < 4; ++e) S[row][4 * e + quad] = st.v[q][e];
    }
}

// One 128 x 128 tile of X C^T into acc; kInterior as for LoadSlice. D block (a, c) of acc: lane
// holds rows wm*64 + 16a + 4g + r (r = 0..3) of column wn*64 + 16c + r16. Ends with a barrier,
// so the LDS buffers are free for the next tile.
template <bool kInterior>
__device__ __forceinline__ void GemmAcc(const float* __restrict__ X, int64_t n, int d, const float* __restrict__ C,
                                        int H, int64_t i0, int64_t h0, float (*As)[kBM][kLdsStride],
                                        float (*Bs)[kBN][kLdsStride], floatx4 (&acc)[4][4]) {

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int g = lane >> 4, r16 = lane & 15;
    // float4 loads need 16-byte aligned rows: d % 4 == 0 and 16-byte aligned bases
    const bool vec4 = (d & 3) == 0 && ((reinterpret_cast<uintptr_t>(X) | reinterpret_cast<uintptr_t>(C)) & 15u) == 0;

#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
        for (int c = 0; c < 4; ++c) acc[a][c] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};

    const int nk = (d + kBK - 1) / kBK;
    Staged sa, sb;
    LoadSlice<kInterior>(X, n, d, i0, 0, vec4, sa);
    LoadSlice<kInterior>(C, H, d, h0, 0, vec4, sb);
    StoreSlice(As[0], sa);
    StoreSlice(Bs[0], sb);
    __syncthreads();

    for (int kt = 0; kt < nk; ++kt) {
        const int cur = kt & 1;
        const bool more = kt + 1 < nk;
        if (more) {
            LoadSlice<kInterior>(X, n, d, i0, (kt + 1) * kBK, vec4, sa);
            LoadSlice<kInterior>(C, H, d, h0, (kt + 1) * kBK, vec4, sb);
        }
        floatx4 af[4], bf[4];
#pragma unroll
        for (int a = 0; a < 4; ++a)
            af[a] = *reinterpret_cast<const floatx4*>(&As[cur][wm * 64 + a * 16 + r16][4 * g]);
#pragma unroll
        for (int c = 0; c < 4; ++c)
            bf[c] = *reinterpret_cast<const floatx4*>(&Bs[cur][wn * 64 + c * 16 + r16][4 * g]);
#pragma unroll
        for (int s = 0; s < 4; ++s)
#pragma unroll
            for (int a = 0; a < 4; ++a)
#pragma unroll
                for (int c = 0; c < 4; ++c)
                    acc[a][c] = __builtin_amdgcn_mfma_f32_16x16x4f32(af[a][s], bf[c][s], acc[a][c], 0, 0, 0);
        if (more) {
            StoreSlice(As[cur ^ 1], sa);
            StoreSlice(Bs[cur ^ 1], sb);
        }
        __syncthreads();
    }
}

// One 128 x 128 output tile of xC; kInterior as for LoadSlice (and no bounds checks on the stores).
template <bool kInterior>
__device__ __forceinline__ void GemmTile(const float* __restrict__ X, int64_t n, int d, const float* __restrict__ C,
                                         int H, float* __restrict__ xC, int64_t ldx, int64_t i0, int64_t h0,
                                         float (*As)[kBM][kLdsStride], float (*Bs)[kBN][kLdsStride]) {
    floatx4 acc[4][4];
    GemmAcc<kInterior>(X, n, d, C, H, i0, h0, As, Bs, acc);
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int g = lane >> 4, r16 = lane & 15;
#pragma unroll
    for (int a = 0; a < 4; ++a) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int64_t row = i0 + wm * 64 + a * 16 + 4 * g + r;
            if (!kInterior && row >= n) continue;
            float* dst = xC + row * ldx;
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const int64_t col = h0 + wn * 64 + c * 16 + r16;
                if (kInterior || col < H) dst[col] = acc[a][c][r];
            }
        }
    }
}

__global__ __launch_bounds__(256) void GemmXcKernel(const float* __restrict__ X, int64_t n, int d,
                                                     const float* __restrict__ C, int H,
                                                     float* __restrict__ xC, int64_t ldx,
                                                     int tiles_h, int64_t tiles_total,
                                                     int64_t per_xcd) {
    __shared__ float As[2][kBM][kLdsStride];
    __shared__ float Bs[2][kBN][kLdsStride];
    // XCD-aware tile order: workgroups are dispatched round-robin over the 8 XCDs, so block b
    // runs on XCD b % 8. Give each XCD a contiguous run of tiles so the 128-vector slices of X
    // that neighbouring codeword tiles share stay in that XCD's L2.
    const int64_t b = blockIdx.x;
    const int64_t tile = (b & 7) * per_xcd + (b >> 3);
    if (tile >= tiles_total) return;
    const int64_t tx = tile / tiles_h;
    const int th = static_cast<int>(tile - tx * tiles_h);
    const int64_t i0 = tx * kBM;
    const int64_t h0 = static_cast<int64_t>(th) * kBN;
    // Full tiles with d % 16 == 0 and aligned operands (every tile of the encoder's shapes but the
    // last row tile) take the branch-free path.
    const bool interior = i0 + kBM <= n && h0 + kBN <= H && (d % kBK) == 0 &&
                          ((reinterpret_cast<uintptr_t>(X) | reinterpret_cast<uintptr_t>(C)) & 15u) == 0;
    if (interior) {
        GemmTile<true>(X, n, d, C, H, xC, ldx, i0, h0, As, Bs);
    } else {
        GemmTile<false>(X, n, d, C, H, xC, ldx, i0, h0, As, Bs);
    }
}

// The nearest-root epilogue of one 128 x 128 score tile: for each of the lane's 16 rows, the
// running first strict minimum of e1 over this tile's columns (ascending code order within a lane;
// the cross-lane order is restored by the final reduction), NaN errors flagged in nanm.
__device__ __forceinline__ void RootTileEpilogue(const floatx4 (&acc)[4][4], const float (&alpha_c)[4], int64_t hb,
                                                 int wn, int r16, const float (&xn)[4][4], float (&be)[4][4],
                                                 uint32_t (&bc)[4][4], uint32_t& nanm) {
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        const int col = static_cast<int>(hb) + wn * 64 + c * 16 + r16;
        const float alpha = alpha_c[c];
        if (alpha == 0.0f) continue;  // beam_search.cpp: alpha == 0 roots are skipped
        // a1 = RN(gam / alpha) without a division per element: gam/alpha = (gam*sc)/(alpha*sc)
        // with sc a power of two and alpha*sc = ap in [1, 2), so q0 = sp*yp,
        // q = fma(-fma(ap, q0, -sp), yp, q0) with yp = RN(1/ap) is the correctly rounded
        // quotient whenever sp = gam*sc is exact and |sp| lies in [2^-100, 2^100] (the identity
        // tests/division_check.c verifies, as for the beam's quotients). Any lane outside that
        // range sends the column back to IEEE division.
        int ex;
        const float mant = frexpf(alpha, &ex);
        const bool colfast = alpha >= 0x1p-60f && alpha <= 0x1p60f;
        const float ap = 2.0f * mant;
        const float sc = colfast ? ldexpf(1.0f, 1 - ex) : 0.0f;  // 0: always the IEEE path
        const float yp = 1.0f / ap;
        float a1v[4][4];
        float lo = __builtin_huge_valf(), hi = 0.0f;
#pragma unroll
        for (int a = 0; a < 4; ++a)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float sp = acc[a][c][r] * sc;
                const float q0 = sp * yp;
                const float rr = __builtin_fmaf(ap, q0, -sp);
                a1v[a][r] = __builtin_fmaf(-rr, yp, q0);
                lo = __builtin_fminf(lo, __builtin_fabsf(sp));
                hi = __builtin_fmaxf(hi, __builtin_fabsf(sp));
            }
        if (__builtin_amdgcn_ballot_w64(!(lo >= 0x1p-100f && hi <= 0x1p100f)) != 0ull) {
#pragma unroll
            for (int a = 0; a < 4; ++a)
#pragma unroll
                for (int r = 0; r < 4; ++r) a1v[a][r] = acc[a][c][r] / alpha;
        }
#pragma unroll
        for (int a = 0; a < 4; ++a)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float gam = acc[a][c][r];
                const float a1 = a1v[a][r];
                const float e1 = xn[a][r] - gam * a1;
                if (__builtin_isnan(e1)) nanm |= 1u << (4 * a + r);
                if (e1 < be[a][r]) {
                    be[a][r] = e1;
                    bc[a][r] = static_cast<uint32_t>(col);
                }
            }
    }
}

// The block's answer from the per-lane running minima: first minimum over the 16 lanes that
// share the lane's rows (codes differ, so ties go to the lower code), then over the two column
// waves through LDS; rows of the block at or past `nrows` are not written.
__device__ __forceinline__ void RootFinish(const float (&be)[4][4], const uint32_t (&bc)[4][4], uint32_t nanm,
                                           int64_t i0, int64_t nrows, float (*red_e)[kBM], uint32_t (*red_c)[kBM],
                                           uint32_t (*red_f)[kBM], uint32_t* __restrict__ root_out,
                                           uint8_t* __restrict__ flag) {
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int g = lane >> 4, r16 = lane & 15;
    // first minimum over the 16 lanes that share these rows (codes differ, so ties go to the
    // lower code), then over the two column waves through LDS
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            float e = be[a][r];
            uint32_t cd = bc[a][r];
            uint32_t f = (nanm >> (4 * a + r)) & 1u;
#pragma unroll
            for (int sh = 1; sh < 16; sh <<= 1) {
                const float e2 = __shfl_xor(e, sh, 16);
                const uint32_t c2 = __shfl_xor(cd, sh, 16);
                f |= __shfl_xor(f, sh, 16);
                if (e2 < e || (e2 == e && c2 < cd)) {
                    e = e2;
                    cd = c2;
                }
            }
            if (r16 == 0) {
                const int lr = wm * 64 + a * 16 + 4 * g + r;
                red_e[wn][lr] = e;
                red_c[wn][lr] = cd;
                red_f[wn][lr] = f;
            }
        }
    __syncthreads();
    const int t = threadIdx.x;
    if (t < kBM && i0 + t < nrows) {
        float e = red_e[0][t];
        uint32_t cd = red_c[0][t];
        const float e2 = red_e[1][t];
        const uint32_t c2 = red_c[1][t];
        if (e2 < e || (e2 == e && c2 < cd)) cd = c2;
        root_out[i0 + t] = cd;
        flag[i0 + t] = static_cast<uint8_t>(red_f[0][t] | red_f[1][t]);
    }
}

// Nearest root of the large-root beam (beam_search.cpp:639-709 with one root slot, the forced
// nearest root): per vector, the first root code in ascending order with the smallest
// e1 = ||x||^2 - g*(g/alpha), g = <x, C0[:,code]>, alpha = ||C0[:,code]||^2 != 0, where a later
// code replaces the current one only when strictly smaller (so ties keep the lower code, and +0
// and -0 tie). The root scores come from the same MFMA tiles as GemmXcKernel (identical g bits),
// but each block sweeps every root tile for its 128 vectors and keeps a running per-row minimum
// in registers instead of writing the n x h0 score matrix.
// A NaN e1 has no such reduction (the reference lets it in and then accepts the next candidate
// whatever it is), so a vector that meets one is flagged for NearestRootFixupKernel.
// root_out: code or kNoRoot; flag: 1 where a NaN was met.
// Two waves per SIMD asked of the register allocator: the accumulators, the per-row minima and
// the epilogue take about 250 registers, and left alone the allocator can land just above 256.
template <bool kInteriorRows>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 8))) void NearestRootKernel(const float* __restrict__ X, int64_t n, int d,
                                                         const float* __restrict__ C0, int h0,
                                                         const float* __restrict__ norm0,
                                                         const float* __restrict__ nx2, uint32_t* __restrict__ root_out,
                                                         uint8_t* __restrict__ flag) {
    __shared__ float As[2][kBM][kLdsStride];
    __shared__ float Bs[2][kBN][kLdsStride];
    __shared__ float red_e[2][kBM];
    __shared__ uint32_t red_c[2][kBM];
    __shared__ uint32_t red_f[2][kBM];
    const int64_t i0 = static_cast<int64_t>(blockIdx.x) * kBM;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int g = lane >> 4, r16 = lane & 15;

    float be[4][4], xn[4][4];
    uint32_t bc[4][4];
    uint32_t nanm = 0;  // bit 4a+r: a NaN e1 met on that row
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int64_t row = i0 + wm * 64 + a * 16 + 4 * g + r;
            be[a][r] = __builtin_huge_valf();
            bc[a][r] = kNoRoot;
            xn[a][r] = (kInteriorRows || row < n) ? nx2[row] : 0.0f;
        }
    const int tiles = (h0 + kBN - 1) / kBN;
    const bool aligned = (d % kBK) == 0 && ((reinterpret_cast<uintptr_t>(X) | reinterpret_cast<uintptr_t>(C0)) & 15u) == 0;
    for (int th = 0; th < tiles; ++th) {
        const int64_t hb = static_cast<int64_t>(th) * kBN;
        const bool interior = kInteriorRows && aligned && hb + kBN <= h0;
        // The tile's ||c0||^2 values are read before its k-loop, so they have arrived by the time
        // the epilogue needs them.
        float alpha_c[4];
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const int col = static_cast<int>(hb) + wn * 64 + c * 16 + r16;
            alpha_c[c] = col < h0 ? norm0[col] : 0.0f;
        }
        floatx4 acc[4][4];
        if (interior) {
            GemmAcc<true>(X, n, d, C0, h0, i0, hb, As, Bs, acc);
        } else {
            GemmAcc<false>(X, n, d, C0, h0, i0, hb, As, Bs, acc);
        }
        RootTileEpilogue(acc, alpha_c, hb, wn, r16, xn, be, bc, nanm);
    }
    RootFinish(be, bc, nanm, i0, n, red_e, red_c, red_f, root_out, flag);
}

// NearestRootKernel for the all-interior case (every row and root tile full, d a multiple of 16,
// 16-byte aligned operands: the C5 shape), with the k-loop run across the root tiles as one
// pipeline: the last slice of a root tile prefetches the next tile's first slice, so a tile starts
// from data already in LDS instead of waiting on its first global loads behind a barrier. The MFMA
// order over k, and so every score's bits, the epilogue and the reduction are NearestRootKernel's.
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 8))) void NearestRootFlatKernel(const float* __restrict__ X, int64_t n, int d,
                                                             const float* __restrict__ C0, int h0,
                                                             const float* __restrict__ norm0,
                                                             const float* __restrict__ nx2,
                                                             uint32_t* __restrict__ root_out,
                                                             uint8_t* __restrict__ flag) {
    __shared__ float As[2][kBM][kLdsStride];
    __shared__ float Bs[2][kBN][kLdsStride];
    __shared__ float red_e[2][kBM];
    __shared__ uint32_t red_c[2][kBM];
    __shared__ uint32_t red_f[2][kBM];
    const int64_t i0 = static_cast<int64_t>(blockIdx.x) * kBM;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int g = lane >> 4, r16 = lane & 15;

    float be[4][4], xn[4][4];
    uint32_t bc[4][4];
    uint32_t nanm = 0;  // bit 4a+r: a NaN e1 met on that row
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            be[a][r] = __builtin_huge_valf();
            bc[a][r] = kNoRoot;
            xn[a][r] = nx2[i0 + wm * 64 + a * 16 + 4 * g + r];
        }
    const int tiles = h0 / kBN;
    const int nk = d / kBK;
    Staged sa, sb;
    LoadSlice<true>(X, n, d, i0, 0, true, sa);
    LoadSlice<true>(C0, h0, d, 0, 0, true, sb);
    StoreSlice(As[0], sa);
    StoreSlice(Bs[0], sb);
    __syncthreads();
    int cur = 0;
    for (int th = 0; th < tiles; ++th) {
        const int64_t hb = static_cast<int64_t>(th) * kBN;
        float alpha_c[4];
#pragma unroll
        for (int c = 0; c < 4; ++c) alpha_c[c] = norm0[static_cast<int>(hb) + wn * 64 + c * 16 + r16];
        floatx4 acc[4][4];
#pragma unroll
        for (int a = 0; a < 4; ++a)
#pragma unroll
            for (int c = 0; c < 4; ++c) acc[a][c] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
        for (int kt = 0; kt < nk; ++kt) {
            // the next slice: this tile's, or the next tile's first (none after the last)
            const bool last_k = kt + 1 == nk;
            const bool more = !last_k || th + 1 < tiles;
            if (more) {
                LoadSlice<true>(X, n, d, i0, last_k ? 0 : (kt + 1) * kBK, true, sa);
                LoadSlice<true>(C0, h0, d, last_k ? hb + kBN : hb, last_k ? 0 : (kt + 1) * kBK, true, sb);
            }
            floatx4 af[4], bf[4];
#pragma unroll
            for (int a = 0; a < 4; ++a)
                af[a] = *reinterpret_cast<const floatx4*>(&As[cur][wm * 64 + a * 16 + r16][4 * g]);
#pragma unroll
            for (int c = 0; c < 4; ++c)
                bf[c] = *reinterpret_cast<const floatx4*>(&Bs[cur][wn * 64 + c * 16 + r16][4 * g]);
#pragma unroll
            for (int s = 0; s < 4; ++s)
#pragma unroll
                for (int a = 0; a < 4; ++a)
#pragma unroll
                    for (int c = 0; c < 4; ++c)
                        acc[a][c] = __builtin_amdgcn_mfma_f32_16x16x4f32(af[a][s], bf[c][s], acc[a][c], 0, 0, 0);
            if (more) {
                StoreSlice(As[cur ^ 1], sa);
                StoreSlice(Bs[cur ^ 1], sb);
            }
            __syncthreads();
            cur ^= 1;
        }
        RootTileEpilogue(acc, alpha_c, hb, wn, r16, xn, be, bc, nanm);
    }
    RootFinish(be, bc, nanm, i0, n, red_e, red_c, red_f, root_out, flag);
}

}  // namespace

hipError_t LaunchNearestRoot(const float* X, int64_t n, int d, const float* C0, int h0, const float* norm0,
                             const float* nx2, uint32_t* root_out, uint8_t* flag, hipStream_t s) {
    if (n <= 0 || h0 <= 0) return hipSuccess;
    const int64_t full = n / kBM;
    const bool flat = (h0 % kBN) == 0 && (d % kBK) == 0 &&
                      ((reinterpret_cast<uintptr_t>(X) | reinterpret_cast<uintptr_t>(C0)) & 15u) == 0;
    if (full > 0 && flat)
        hipLaunchKernelGGL(NearestRootFlatKernel, dim3(static_cast<unsigned>(full)), dim3(256), 0, s, X, n, d, C0, h0,
                           norm0, nx2, root_out, flag);
    else if (full > 0)
        hipLaunchKernelGGL(NearestRootKernel<true>, dim3(static_cast<unsigned>(full)), dim3(256), 0, s, X, n, d, C0,
                           h0, norm0, nx2, root_out, flag);
    if (full * kBM < n) {
        // the partial last row tile: blockIdx 0 of this launch is tile `full`
        hipLaunchKernelGGL(NearestRootKernel<false>, dim3(1), dim3(256), 0, s, X + full * kBM * d, n - full * kBM, d,
                           C0, h0, norm0, nx2 + full * kBM, root_out + full * kBM, flag + full * kBM);
    }
    return hipGetLastError();
}

hipError_t LaunchGemmXc(const float* X, int64_t n, int d, const float* C, int H, float* xC, int64_t ldx,
                        hipStream_t s) {
    if (n <= 0 || H <= 0) return hipSuccess;
    const int tiles_h = (H + kBN - 1) / kBN;
    const int64_t tiles_x = (n + kBM - 1) / kBM;
    const int64_t total = tiles_x * tiles_h;
    const int64_t per_xcd = (total + 7) / 8;
    const int64_t blocks = per_xcd * 8;
    hipLaunchKernelGGL(GemmXcKernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, s, X, n, d, C, H, xC,
                       ldx, tiles_h, total, per_xcd);
    return hipGetLastError();
}

}  // namespace stlq_mi355
