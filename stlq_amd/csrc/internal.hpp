// Internal declarations shared by the HIP translation units of libstlq_mi355.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <string>

namespace stlq_mi355 {

constexpr int kMaxM = 20;     // include/stlq/core/model_limits.h:5
constexpr int kMaxK = 256;    // uint8 codes (include/stlq/common/types.h:20-32)
constexpr int kMaxBeam = 64;  // slot state lives in one wave64 lane per slot
constexpr int kWave = 64;
constexpr int kBeamWavesPerBlock = 4;  // one vector per wave, four vectors per workgroup

__host__ __device__ inline int CodeStride(int m) { return (m + 3) & ~3; }

// Beam state of one tile of vectors, slot-major (vector i, slot s at i*Hb + s). Each slot is
// one record of BeamRecordStride(m) dwords: [err, the Cholesky factor R column by column with
// each column followed by the reciprocal of its diagonal (m(m+3)/2), coef[m],
// codes (CodeStride(m) bytes), root id, the two pruning constants kap and phi, padding to
// 16 bytes].
struct BeamState {
    float* rec = nullptr;        // [n*Hb*BeamRecordStride(m)]
    int* curH = nullptr;         // [n]
};
int BeamRecordStride(int m);

// Gram access for the prefix-LS cross terms. A_t(k) of a beam with prefix codes code_t is
// row[(off_t + code_t) * ld + offL + k] of a row-major matrix whose element (r, c) is the
// reference's G(r, c) (linear_algebra.h:17-19 GAt(G, row=flat_t, col=flat)).
// Large-root: t = 0 reads row `root` of G0S (h0 x Hs, row-major), t >= 1 reads G_small.
struct GramView {
    const float* G = nullptr;    // row-major H x H (or Hs x Hs)
    int ld = 0;
    const float* G0S = nullptr;  // large-root only: row-major h0 x Hs
    int off[kMaxM] = {};         // flat offset of each layer inside G's index space
};

struct LayerArgs {
    GramView gram;
    const float* xC = nullptr;    // [n*ldx] per-vector <x, c_f> rows (xC_small for large-root)
    int64_t ldx = 0;
    const float* nx2 = nullptr;   // [n]
    const float* gdiag = nullptr; // G diagonal over the same flat index space
    // Candidate pruning (prune_bound.hpp), over the same flat index space as gdiag:
    // isw[f] = RN(sqrt(gdiag[f])), sw[f] = RN(1/isw[f]), Gs = G with row f scaled by sw[f]
    // (row-major, same ld; the large root's prefix 0 is scaled by sw0[root] on the fly);
    // sw0/isw0 the same for the roots of a large root. prune = 0 turns it off.
    const float* Gs = nullptr;
    const float* sw = nullptr;
    const float* isw = nullptr;
    const float* sw0 = nullptr;
    const float* isw0 = nullptr;
    int prune = 0;
    BeamState in, out;
    int64_t n = 0;
    int m = 0, Hb = 0, K = 0, offL = 0;
    // final pick (last layer): codes [n*m] (or B_small [n*(m-1)] for large-root), best_err [n]
    uint8_t* codes_out = nullptr;
    float* best_err = nullptr;
    uint32_t* cluster_out = nullptr;
    int is_last = 0;
    // Best-first pass (full precomp): parents are scanned in ascending error order instead of
    // the reference's slot order, which keeps the reference's top-H sets whenever no two
    // candidates tie at the top-H boundary. flags[i] = 1 marks a vector where that could fail
    // (a boundary tie, a tie for the final minimum, a NaN or -0 error); those vectors are
    // re-run in the reference order. null: the reference order.
    uint8_t* flags = nullptr;
    // Re-run over a list: wave w encodes vector list[w] for w < *list_n, with its beam state at
    // index w. null: wave w encodes vector w.
    const int* list = nullptr;
    const int* list_n = nullptr;
};

struct RootArgs {
    const float* scores = nullptr;  // [n*ldx] root scores <x, c0_r> (nullable when forced)
    int64_t ldx = 0;
    const float* nx2 = nullptr;
    const float* norm0 = nullptr;   // [h0]
    const float* sw0 = nullptr;     // [h0] pruning scalings of the roots (LayerArgs::sw0, isw0)
    const float* isw0 = nullptr;
    const uint32_t* forced = nullptr;
    BeamState out;
    int64_t n = 0;
    int m = 0, Hb = 0, h0 = 0, root_slots = 0;
    uint8_t* codes_out = nullptr;
    float* best_err = nullptr;
    uint32_t* cluster_out = nullptr;
    int is_last = 0;
    // Seed over a list (the best-first pass's re-run, as LayerArgs::list): wave w seeds vector
    // list[w] for w < *list_n into beam-state index w. null: wave w seeds vector w.
    const int* list = nullptr;
    const int* list_n = nullptr;
};

// ---- launchers (each defined in the .hip file that holds the kernel) ----
hipError_t LaunchGram(const float* C, int d, int H, float* G_rm, hipStream_t s);
hipError_t LaunchCross(const float* C0, int h0, const float* Cs, int Hs, int d, float* G0S_rm, hipStream_t s);
hipError_t LaunchNorms(const float* C, int d, int H, bool lane4, float* norm2, float* invnorm, hipStream_t s);
hipError_t LaunchRootDot(const float* X, int d, const float* C0, const uint32_t* root, int64_t n, float* out,
                         hipStream_t s);
hipError_t LaunchDiag(const float* G_rm, int H, float* diag, hipStream_t s);
// Pruning scalings of n codewords from their squared norms g: isw = RN(sqrt(g)), sw = RN(1/isw).
hipError_t LaunchPruneScale(const float* g, int64_t n, float* sw, float* isw, hipStream_t s);
// Gs(r, c) = G(r, c) * sw[r] for a row-major rows x cols matrix (row stride cols).
hipError_t LaunchRowScale(const float* G, int64_t rows, int cols, const float* sw, float* Gs, hipStream_t s);
// *out = max over i of the bits of |x[i]| (NaN above +inf); *out must be cleared beforehand.
hipError_t LaunchAbsMaxBits(const float* x, int64_t n, unsigned* out, hipStream_t s);
hipError_t LaunchTranspose(const float* in, int rows, int cols, float* out, hipStream_t s);
hipError_t LaunchXNorm2(const float* X, int d, int64_t n, float* out, hipStream_t s);
hipError_t LaunchGemmXc(const float* X, int64_t n, int d, const float* C, int H, float* xC, int64_t ldx,
                        hipStream_t s);

hipError_t LaunchBeamLayer0(const LayerArgs& a, hipStream_t s);
hipError_t LaunchBeamLayer(int L, bool large_root, const LayerArgs& a, hipStream_t s);
// Indices of the vectors with flags[i] != 0 into list; counts[0] and counts[1] grow by their
// number (both must be cleared beforehand as the caller needs).
hipError_t LaunchCollectFlagged(const uint8_t* flags, int64_t n, int* list, int* counts, hipStream_t s);
hipError_t LaunchRootSeed(const RootArgs& a, hipStream_t s);
// No root for the vector (every root skipped or worse than +inf): the forced-root paths seed
// nothing, as the root scan does.
constexpr uint32_t kNoRoot = 0xFFFFFFFFu;
// Nearest root per vector from fused MFMA root scores (no score matrix); flag = 1 where a NaN
// error was met (those vectors are redone by LaunchNearestRootFixup).
hipError_t LaunchNearestRoot(const float* X, int64_t n, int d, const float* C0, int h0, const float* norm0,
                             const float* nx2, uint32_t* root_out, uint8_t* flag, hipStream_t s);
hipError_t LaunchNearestRootFixup(const float* X, int d, const float* C0, int h0, const float* norm0,
                                  const float* nx2, const uint8_t* flag, int64_t n, uint32_t* root_out, hipStream_t s);
hipError_t LaunchGatherRootDot(const float* X, int d, const float* C0, const uint32_t* roots, int64_t n, float* out,
                               hipStream_t s);

struct LsArgs {
    const float* xC = nullptr;
    int64_t ldx = 0;
    const float* G_rm = nullptr;
    int H = 0;
    int m = 0;
    int off[kMaxM] = {};
    const uint8_t* codes = nullptr;  // [n*m]
    float* a = nullptr;              // [n*m]
    const float* nx2 = nullptr;
    float* cost = nullptr;
    int* fails = nullptr;            // device counter
    int64_t n = 0;
    int cstride = 0;                 // codes per vector: m, or m-1 for a large root
    // Large root: layer 0 is the vector's root code root[i] from C0 (h0 codewords) and codes
    // holds layers 1..m-1; H, G_rm, off and xC then describe the small layers. Null for the full
    // precomp.
    const uint32_t* root = nullptr;  // [n]
    const float* b0 = nullptr;       // [n] <C0[:,root], x>
    const float* norm0 = nullptr;    // [h0] ||C0[:,r]||^2
    const float* G0S_rm = nullptr;   // [h0*H] row r: <C0[:,r], C_small[:,f]>
};
hipError_t LaunchLsAll(const LsArgs& a, hipStream_t s);
hipError_t LaunchCosts(const LsArgs& a, hipStream_t s);

struct IcmArgs {
    LsArgs ls;                       // codes (mutable through codes_rw), a, cost, nx2
    uint8_t* codes_rw = nullptr;
    const float* G_cm = nullptr;     // column-major reference G: G(row, col) at [col*H + row]
    const float* invnorm = nullptr;
    uint8_t* active = nullptr;       // [n]
    uint8_t* changed = nullptr;      // [n]
    int* fails = nullptr;
    int* pend = nullptr;             // [n] the layer's proposed code, or -1 (scoring -> re-solve)
    int j = 0;                       // layer updated by this launch
    int use_abs = 1;
    int hj = 0;
};
hipError_t LaunchIcmLayer(const IcmArgs& a, hipStream_t s);
hipError_t LaunchIcmDeactivate(uint8_t* active, const uint8_t* changed, int64_t n, hipStream_t s);
// Codes are stored `cstride` per vector starting at layer `lfirst` (0, or 1 for a large root).
hipError_t LaunchPerturb(uint8_t* codes, int64_t n, int m, int cstride, int lfirst, const int* h_vec, int perturb_k,
                         uint32_t seed, int outer, uint64_t id0, hipStream_t s);
hipError_t LaunchIlsAccept(uint8_t* codes, float* a, float* cost, const uint8_t* cc, const float* ca, const float* ccost,
                           int64_t n, int m, int cstride, hipStream_t s);
hipError_t LaunchFill8(uint8_t* p, uint8_t v, int64_t n, hipStream_t s);
hipError_t LaunchCopy16(void* dst, const void* src, size_t n16, hipStream_t s);
hipError_t LaunchU8ToF32(const uint8_t* in, float* out, size_t count, hipStream_t s);

}  // namespace stlq_mi355
