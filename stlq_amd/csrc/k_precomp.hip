// Precomputation kernels: Gram matrices, codeword norms, ||x||^2.
//
// All sums here run in a fixed sequential order (r = 0..d-1), one IEEE-rounded multiply and
// one IEEE-rounded add per term (the library is compiled with -ffp-contract=off), so the
// results are reproducible bit-for-bit by a scalar CPU loop and the Gram is exactly symmetric.
#include "internal.hpp"

#include <algorithm>

namespace stlq_mi355 {
namespace {

// out[i*ldo + j] = sum_r A[i*d + r] * B[j*d + r], r ascending.
// 256 threads compute a 64x64 output tile, 4x4 per thread; d is staged through LDS in chunks of
// 32 so every thread keeps its own sequential accumulation order.
constexpr int kDotTile = 64;
constexpr int kDotChunk = 32;

__global__ __launch_bounds__(256) void SeqDotKernel(const float* __restrict__ A, int M,
                                                    const float* __restrict__ B, int N, int d,
                                                    float* __restrict__ out, int64_t ldo) {
    __shared__ float sA[kDotTile][kDotChunk + 1];
    __shared__ float sB[kDotTile][kDotChunk + 1];
    const int tx = threadIdx.x & 15;  // j sub-block
    const int ty = threadIdx.x >> 4;  // i sub-block
    const int64_t i0 = static_cast<int64_t>(blockIdx.y) * kDotTile;
    const int64_t j0 = static_cast<int64_t>(blockIdx.x) * kDotTile;
    float acc[4][4];
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
        for (int b = 0; b < 4; ++b) acc[a][b] = 0.0f;

    for (int r0 = 0; r0 < d; r0 += kDotChunk) {
        const int rl = min(kDotChunk, d - r0);
        for (int idx = threadIdx.x; idx < kDotTile * kDotChunk; idx += 256) {
            const int row = idx / kDotChunk;
            const int col = idx % kDotChunk;
            const int64_t gi = i0 + row, gj = j0 + row;
            sA[row][col] = (gi < M && col < rl) ? A[gi * d + r0 + col] : 0.0f;
            sB[row][col] = (gj < N && col < rl) ? B[gj * d + r0 + col] : 0.0f;
        }
        __syncthreads();
        for (int r = 0; r < rl; ++r) {
            float av[4], bv[4];
#pragma unroll
            for (int a = 0; a < 4; ++a) av[a] = sA[ty + 16 * a][r];
#pragma unroll
            for (int b = 0; b < 4; ++b) bv[b] = sB[tx + 16 * b][r];
#pragma unroll
            for (int a = 0; a < 4; ++a)
#pragma unroll
                for (int b = 0; b < 4; ++b) acc[a][b] = acc[a][b] + av[a] * bv[b];
        }
        __syncthreads();
    }
#pragma unroll
    for (int a = 0; a < 4; ++a) {
        const int64_t gi = i0 + ty + 16 * a;
        if (gi >= M) continue;
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            const int64_t gj = j0 + tx + 16 * b;
            if (gj < N) out[gi * ldo + gj] = acc[a][b];
        }
    }
}

// Sum of squares in the order the reference's Release build gives its `omp simd` reductions
// (GCC, -O3 -fopenmp, baseline x86-64 = 4 float lanes): element t goes to lane t mod 4 over the
// first floor(d/4)*4 elements, the rest to lane 0, then the lanes are added in order to 0.
__device__ __forceinline__ float SimdLane4SumSq(const float* __restrict__ x, int d) {
    float p0 = 0.0f, p1 = 0.0f, p2 = 0.0f, p3 = 0.0f;
    const int d4 = d & ~3;
    for (int t = 0; t < d4; t += 4) {
        p0 = p0 + x[t] * x[t];
        p1 = p1 + x[t + 1] * x[t + 1];
        p2 = p2 + x[t + 2] * x[t + 2];
        p3 = p3 + x[t + 3] * x[t + 3];
    }
    for (int t = d4; t < d; ++t) p0 = p0 + x[t] * x[t];
    return (((0.0f + p0) + p1) + p2) + p3;
}

// Dot product in the same `omp simd` order (least_squares.cpp:35-42 Dot, icm.cpp:67-74 DotF32,
// cost_utils.cpp:55-60): the large-root LS right-hand side b0 = <C0[:,root], x>.
__device__ __forceinline__ float SimdLane4Dot(const float* __restrict__ a, const float* __restrict__ b, int d) {
    float p0 = 0.0f, p1 = 0.0f, p2 = 0.0f, p3 = 0.0f;
    const int d4 = d & ~3;
    for (int t = 0; t < d4; t += 4) {
        p0 = p0 + a[t] * b[t];
        p1 = p1 + a[t + 1] * b[t + 1];
        p2 = p2 + a[t + 2] * b[t + 2];
        p3 = p3 + a[t + 3] * b[t + 3];
    }
    for (int t = d4; t < d; ++t) p0 = p0 + a[t] * b[t];
    return (((0.0f + p0) + p1) + p2) + p3;
}

// b0[i] = <C0[:,root[i]], x_i>, one thread per vector (d mul+adds; the C0 rows are shared
// through L2, the X rows are read once).
__global__ __launch_bounds__(256) void RootDotKernel(const float* __restrict__ X, int d, const float* __restrict__ C0,
                                                     const uint32_t* __restrict__ root, int64_t n,
                                                     float* __restrict__ out) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= n) return;
    out[i] = SimdLane4Dot(C0 + static_cast<int64_t>(root[i]) * d, X + i * d, d);
}

// ||c||^2 and 1/sqrt(||c||^2) per codeword. lane4 = false: the sequential loop of
// encoder_precomp.inc:31-39 (invnorm_flat); lane4 = true: Norm2 of precomp_large_root.cpp:14-23
// (norm0, invnorm_small_flat), an `omp simd` reduction.
__global__ void NormsKernel(const float* __restrict__ C, int d, int H, bool lane4, float* __restrict__ norm2,
                            float* __restrict__ invnorm) {
    const int f = blockIdx.x * blockDim.x + threadIdx.x;
    if (f >= H) return;
    const float* c = C + static_cast<int64_t>(f) * d;
    float s = 0.0f;
    if (lane4) {
        s = SimdLane4SumSq(c, d);
    } else {
        for (int r = 0; r < d; ++r) s = s + c[r] * c[r];
    }
    if (norm2) norm2[f] = s;
    if (invnorm) invnorm[f] = s > 0.0f ? 1.0f / sqrtf(s) : 0.0f;
}

__global__ void DiagKernel(const float* __restrict__ G, int H, float* __restrict__ diag) {
    const int f = blockIdx.x * blockDim.x + threadIdx.x;
    if (f < H) diag[f] = G[static_cast<int64_t>(f) * H + f];
}

__global__ void PruneScaleKernel(const float* __restrict__ g, int64_t n, float* __restrict__ sw,
                                 float* __restrict__ isw) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const float r = sqrtf(g[i]);
    isw[i] = r;
    sw[i] = 1.0f / r;
}

__global__ void RowScaleKernel(const float* __restrict__ G, int64_t rows, int cols, const float* __restrict__ sw,
                               float* __restrict__ Gs) {
    const int64_t r = blockIdx.y + static_cast<int64_t>(gridDim.y) * blockIdx.z;
    const int c = blockIdx.x * blockDim.x + threadIdx.x;
    if (r >= rows || c >= cols) return;
    Gs[r * cols + c] = G[r * cols + c] * sw[r];
}

// Largest |x| as float bits (NaN payloads sort above +inf): per-thread max over a grid stride,
// wave max by shuffles, one atomic per wave.
__global__ __launch_bounds__(256) void AbsMaxBitsKernel(const float* __restrict__ x, int64_t n, unsigned* out) {
    unsigned m = 0;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
         i += static_cast<int64_t>(gridDim.x) * blockDim.x)
        m = max(m, __float_as_uint(x[i]) & 0x7FFFFFFFu);
    for (int o = 32; o > 0; o >>= 1) m = max(m, static_cast<unsigned>(__shfl_xor(static_cast<int>(m), o)));
    if ((threadIdx.x & 63) == 0) atomicMax(out, m);
}

__global__ void TransposeKernel(const float* __restrict__ in, int rows, int cols,
                                float* __restrict__ out) {
    __shared__ float t[32][33];
    const int c0 = blockIdx.x * 32, r0 = blockIdx.y * 32;
    for (int k = threadIdx.y; k < 32; k += 8) {
        const int r = r0 + k, c = c0 + threadIdx.x;
        if (r < rows && c < cols) t[k][threadIdx.x] = in[static_cast<int64_t>(r) * cols + c];
    }
    __syncthreads();
    for (int k = threadIdx.y; k < 32; k += 8) {
        const int c = c0 + k, r = r0 + threadIdx.x;
        if (r < rows && c < cols) out[static_cast<int64_t>(c) * rows + r] = t[threadIdx.x][k];
    }
}

// ||x||^2 per vector (cost_utils.cpp:99-109, beam_search.cpp:218-223) in the reference build's
// OpenMP-simd order (SimdLane4SumSq above). A wave stages 64 vectors' rows through LDS in chunks
// so the global reads are coalesced; each lane keeps its vector's four partial sums. The chunk
// length is a multiple of 4, so lane t mod 4 is the same within and across chunks.
constexpr int kNormChunk = 32;
__global__ __launch_bounds__(256) void XNorm2Kernel(const float* __restrict__ X, int d, int64_t n,
                                                    float* __restrict__ out) {
    __shared__ float tile[4][kWave][kNormChunk + 1];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int64_t v0 = (static_cast<int64_t>(blockIdx.x) * 4 + wave) * kWave;
    const int nv = v0 < n ? static_cast<int>(min<int64_t>(kWave, n - v0)) : 0;
    const int d4 = d & ~3;
    float p0 = 0.0f, p1 = 0.0f, p2 = 0.0f, p3 = 0.0f;
    for (int t0 = 0; t0 < d; t0 += kNormChunk) {
        const int tl = min(kNormChunk, d - t0);
        for (int r = 0; r < nv; ++r) {
            if (lane < tl) tile[wave][r][lane] = X[(v0 + r) * d + t0 + lane];
        }
        __syncthreads();
        if (lane < nv) {
            const float* row = tile[wave][lane];
            const int main = max(0, min(tl, d4 - t0));  // multiple of 4
            for (int t = 0; t < main; t += 4) {
                p0 = p0 + row[t] * row[t];
                p1 = p1 + row[t + 1] * row[t + 1];
                p2 = p2 + row[t + 2] * row[t + 2];
                p3 = p3 + row[t + 3] * row[t + 3];
            }
            for (int t = main; t < tl; ++t) p0 = p0 + row[t] * row[t];
        }
        __syncthreads();
    }
    if (lane < nv) out[v0 + lane] = (((0.0f + p0) + p1) + p2) + p3;
}

__global__ void Fill8Kernel(uint8_t* p, uint8_t v, int64_t n) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i < n) p[i] = v;
}

// Plain streaming copy, 16 bytes per thread per iteration (grid-stride).
__global__ __launch_bounds__(256) void Copy16Kernel(uint4* __restrict__ dst, const uint4* __restrict__ src, size_t n16) {
    const size_t stride = static_cast<size_t>(gridDim.x) * blockDim.x;
    for (size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n16; i += stride) dst[i] = src[i];
}

// uint8 -> fp32 widening of a streamed chunk (U8ToF32Kernel1D, kernel_provider_cuda_stream_kernels.inc:16),
// four bytes per thread per iteration.
__global__ __launch_bounds__(256) void U8ToF32Kernel(const uint8_t* __restrict__ in, float* __restrict__ out, size_t count) {
    const size_t stride = static_cast<size_t>(gridDim.x) * blockDim.x * 4;
    for (size_t i = (static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x) * 4; i < count; i += stride) {
        if (i + 3 < count) {
            const uchar4 v = *reinterpret_cast<const uchar4*>(in + i);
            *reinterpret_cast<float4*>(out + i) = make_float4(v.x, v.y, v.z, v.w);
        } else {
            for (size_t k = i; k < count; ++k) out[k] = static_cast<float>(in[k]);
        }
    }
}

}  // namespace

hipError_t LaunchU8ToF32(const uint8_t* in, float* out, size_t count, hipStream_t s) {
    if (count == 0) return hipSuccess;
    const size_t blocks = std::min<size_t>((count / 4 + 255) / 256 + 1, 256 * 64);
    hipLaunchKernelGGL(U8ToF32Kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, s, in, out, count);
    return hipGetLastError();
}

hipError_t LaunchCopy16(void* dst, const void* src, size_t n16, hipStream_t s) {
    if (n16 == 0) return hipSuccess;
    const size_t blocks = std::min<size_t>((n16 + 255) / 256, 256 * 32);
    hipLaunchKernelGGL(Copy16Kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, s,
                       static_cast<uint4*>(dst), static_cast<const uint4*>(src), n16);
    return hipGetLastError();
}

hipError_t LaunchGram(const float* C, int d, int H, float* G_rm, hipStream_t s) {
    if (H <= 0) return hipSuccess;
    dim3 grid((H + kDotTile - 1) / kDotTile, (H + kDotTile - 1) / kDotTile);
    hipLaunchKernelGGL(SeqDotKernel, grid, dim3(256), 0, s, C, H, C, H, d, G_rm, static_cast<int64_t>(H));
    return hipGetLastError();
}

hipError_t LaunchCross(const float* C0, int h0, const float* Cs, int Hs, int d, float* G0S_rm,
                       hipStream_t s) {
    if (h0 <= 0 || Hs <= 0) return hipSuccess;
    dim3 grid((Hs + kDotTile - 1) / kDotTile, (h0 + kDotTile - 1) / kDotTile);
    hipLaunchKernelGGL(SeqDotKernel, grid, dim3(256), 0, s, C0, h0, Cs, Hs, d, G0S_rm, static_cast<int64_t>(Hs));
    return hipGetLastError();
}

hipError_t LaunchRootDot(const float* X, int d, const float* C0, const uint32_t* root, int64_t n, float* out,
                         hipStream_t s) {
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(RootDotKernel, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0, s, X, d, C0, root,
                       n, out);
    return hipGetLastError();
}

hipError_t LaunchNorms(const float* C, int d, int H, bool lane4, float* norm2, float* invnorm, hipStream_t s) {
    if (H <= 0) return hipSuccess;
    hipLaunchKernelGGL(NormsKernel, dim3((H + 255) / 256), dim3(256), 0, s, C, d, H, lane4, norm2, invnorm);
    return hipGetLastError();
}

hipError_t LaunchDiag(const float* G_rm, int H, float* diag, hipStream_t s) {
    if (H <= 0) return hipSuccess;
    hipLaunchKernelGGL(DiagKernel, dim3((H + 255) / 256), dim3(256), 0, s, G_rm, H, diag);
    return hipGetLastError();
}

hipError_t LaunchPruneScale(const float* g, int64_t n, float* sw, float* isw, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(PruneScaleKernel, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0, s, g, n, sw, isw);
    return hipGetLastError();
}

hipError_t LaunchRowScale(const float* G, int64_t rows, int cols, const float* sw, float* Gs, hipStream_t s) {
    if (rows <= 0 || cols <= 0) return hipSuccess;
    const int64_t ry = std::min<int64_t>(rows, 32768);
    const dim3 grid(static_cast<unsigned>((cols + 255) / 256), static_cast<unsigned>(ry),
                    static_cast<unsigned>((rows + ry - 1) / ry));
    hipLaunchKernelGGL(RowScaleKernel, grid, dim3(256), 0, s, G, rows, cols, sw, Gs);
    return hipGetLastError();
}

hipError_t LaunchAbsMaxBits(const float* x, int64_t n, unsigned* out, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    const int64_t blocks = std::min<int64_t>((n + 255) / 256, 2048);
    hipLaunchKernelGGL(AbsMaxBitsKernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, s, x, n, out);
    return hipGetLastError();
}

hipError_t LaunchTranspose(const float* in, int rows, int cols, float* out, hipStream_t s) {
    if (rows <= 0 || cols <= 0) return hipSuccess;
    dim3 grid((cols + 31) / 32, (rows + 31) / 32);
    hipLaunchKernelGGL(TransposeKernel, grid, dim3(32, 8), 0, s, in, rows, cols, out);
    return hipGetLastError();
}

hipError_t LaunchXNorm2(const float* X, int d, int64_t n, float* out, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    const int64_t blocks = (n + 4 * kWave - 1) / (4 * kWave);
    hipLaunchKernelGGL(XNorm2Kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, s, X, d, n, out);
    return hipGetLastError();
}

hipError_t LaunchFill8(uint8_t* p, uint8_t v, int64_t n, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(Fill8Kernel, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0, s, p, v, n);
    return hipGetLastError();
}

}  // namespace stlq_mi355
