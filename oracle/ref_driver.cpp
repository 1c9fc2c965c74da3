// Test infrastructure: a C-ABI driver around the reference's own CPU encoder functions, compiled
// from the reference sources where they lie (oracle/Makefile, target `ref`) into
// oracle/_ref/libstlq_ref.so. Tests use it to check the oracle restatement against the real
// reference; nothing in the product links or loads it.
//
// Compiled with the reference's translation units
//   src/quantizer/beam_search.cpp, linear_algebra.cpp, cost_utils.cpp, least_squares.cpp,
//   icm.cpp, src/common/timer.cpp, logger.cpp, src/io/base_store.cpp (the BaseBasicStore writer)
//   and src/pipeline/main_virtual_helpers.cpp (its checkpoint helpers)
// and linked against the image's MKL runtime for LAPACK spotrf_/spotrs_ (least_squares.cpp).
// blas.cpp is not buildable here (it includes cblas.h, which the image lacks), so GemmRaw and
// BlasSetThreads stay unresolved. They are only reached from the root-score GEMM of
// BeamSearchPrefixLSLargeRoot (beam_search.cpp:623-690), which this driver never calls; the
// library is loaded with lazy binding.
//
// Array conventions (all column-major as in the reference's ColMajorMatrix):
//   X d x n, xC H x n, G H x H, codes m x n (uint8), a m x n.
#include <algorithm>
#include <cstdint>
#include <cstring>
#include <vector>

#include "stlq/common/types.h"
#include "stlq/quantizer/beam_search.h"
#include "stlq/quantizer/cost_utils.h"
#include "stlq/quantizer/icm.h"
#include "stlq/quantizer/least_squares.h"
#include "stlq/quantizer/precomp_large_root.h"
#include "stlq/io/base_store.h"
#include "stlq/pipeline/main_virtual_helpers.h"

#include <string>

namespace {

stlq::Precomp MakePrecomp(const float* G, int H, const int* h_vec, int m, int d) {
    stlq::Precomp p;
    p.m = m;
    p.d = d;
    p.H = H;
    p.h_vec.assign(h_vec, h_vec + m);
    int off = 0;
    for (int l = 0; l < m; ++l) {
        p.offsets.push_back(off);
        for (int k = 0; k < h_vec[l]; ++k) p.flat_layer.push_back(l);
        off += h_vec[l];
    }
    p.G = stlq::ColMajorMatrix<float>(H, H);
    std::memcpy(p.G.data.data(), G, sizeof(float) * static_cast<std::size_t>(H) * H);
    return p;
}

template <typename T>
stlq::ColMajorMatrix<T> Wrap(const T* src, int rows, int cols) {
    stlq::ColMajorMatrix<T> M(rows, cols);
    if (src) std::memcpy(M.data.data(), src, sizeof(T) * M.data.size());
    return M;
}

// A PrecompLargeRoot (precomp_large_root.h:12-38) from arrays built by the caller: C0 d x h0,
// norm0 h0, G_small Hs x Hs, G0S h0 x Hs, invnorm_small Hs (may be null), no G0S_T.
stlq::PrecompLargeRoot MakePrecompLargeRoot(int d, int m, const int* h_vec, const float* C0, const float* norm0,
                                            const float* G_small, int Hs, const float* G0S,
                                            const float* invnorm_small) {
    stlq::PrecompLargeRoot pre;
    pre.d = d;
    pre.m = m;
    pre.h_vec.assign(h_vec, h_vec + m);
    int off = 0;
    for (int l = 0; l < m; ++l) {
        pre.offsets.push_back(off);
        off += h_vec[l];
    }
    const int h0 = h_vec[0];
    pre.C0 = Wrap(C0, d, h0);
    pre.norm0.assign(norm0, norm0 + h0);
    pre.H_small = Hs;
    pre.small_offsets.assign(m, 0);
    int so = 0;
    for (int l = 1; l < m; ++l) {
        pre.small_offsets[l] = so;
        so += h_vec[l];
    }
    pre.G_small = Wrap(G_small, Hs, Hs);
    pre.G0S = Wrap(G0S, h0, Hs);
    if (invnorm_small) pre.invnorm_small_flat.assign(invnorm_small, invnorm_small + Hs);
    pre.ready = true;
    return pre;
}

}  // namespace

extern "C" {

// stlq::ComputeXNorm2 (cost_utils.cpp:88-110).
void ref_xnorm2(const float* X, int d, int n, float* out) {
    const auto Xm = Wrap(X, d, n);
    std::vector<float> v;
    stlq::ComputeXNorm2(Xm, &v);
    std::memcpy(out, v.data(), sizeof(float) * static_cast<std::size_t>(n));
}

// stlq::BeamSearchPrefixLS (beam_search.cpp:196-422); ||x||^2 is computed inside from X.
void ref_beam_search(const float* X, int d, int n, const float* xC, const float* G, int H, const int* h_vec, int m,
                     int H_beam, uint8_t* codes) {
    const auto pre = MakePrecomp(G, H, h_vec, m, d);
    const auto Xm = Wrap(X, d, n);
    const auto xCm = Wrap(xC, H, n);
    stlq::ColMajorMatrix<stlq::FullCode> B;
    stlq::BeamSearchPrefixLS(Xm, pre, xCm, H_beam, &B);
    std::memcpy(codes, B.data.data(), B.data.size());
}

// stlq::ComputeCosts (cost_utils.cpp:139-158).
void ref_compute_costs(const float* xC, const float* G, int H, const int* h_vec, int m, const uint8_t* codes,
                       const float* a, const float* nx2, int n, float* cost) {
    const auto pre = MakePrecomp(G, H, h_vec, m, 0);
    const auto xCm = Wrap(xC, H, n);
    const auto B = Wrap(codes, m, n);
    const auto am = Wrap(a, m, n);
    const std::vector<float> xn(nx2, nx2 + n);
    std::vector<float> out;
    stlq::ComputeCosts(pre, xCm, B, am, xn, &out);
    std::memcpy(cost, out.data(), sizeof(float) * static_cast<std::size_t>(n));
}

// stlq::SolveLeastSquaresAll (least_squares.cpp:406-565; LAPACK for m not in {5, 10}).
void ref_solve_ls_all(const float* xC, const float* G, int H, const int* h_vec, int m, const uint8_t* codes, int n,
                      float* a) {
    const auto pre = MakePrecomp(G, H, h_vec, m, 0);
    const auto xCm = Wrap(xC, H, n);
    const auto B = Wrap(codes, m, n);
    stlq::ColMajorMatrix<float> am;
    stlq::SolveLeastSquaresAll(pre, xCm, B, &am);
    std::memcpy(a, am.data.data(), sizeof(float) * am.data.size());
}

// stlq::DynamicIcmWithIls{Abs,NoAbs}NoNormal (icm.cpp:1132-1170): LS refit, costs, icm_iters
// RunIcm sweeps, then ils_iters perturb + RunIcm + accept rounds. codes (m x n) are updated in
// place. invnorm (H) is the precomp's invnorm_flat.
void ref_icm(const float* X, int d, int n, const float* xC, const float* G, const float* invnorm, int H,
             const int* h_vec, int m, int icm_iters, int ils_iters, int perturb_k, int use_abs, uint32_t seed,
             uint64_t sample_id_offset, uint8_t* codes, float* a, float* cost) {
    auto pre = MakePrecomp(G, H, h_vec, m, d);
    pre.invnorm_flat.assign(invnorm, invnorm + H);
    const auto Xm = Wrap(X, d, n);
    const auto xCm = Wrap(xC, H, n);
    auto B = Wrap(codes, m, n);
    stlq::ColMajorMatrix<float> am;
    std::vector<float> xn2, cst;
    if (use_abs)
        stlq::DynamicIcmWithIlsAbsNoNormal(Xm, pre, xCm, icm_iters, ils_iters, perturb_k, seed, &B, &am, &xn2, &cst,
                                           false, sample_id_offset);
    else
        stlq::DynamicIcmWithIlsNoAbsNoNormal(Xm, pre, xCm, icm_iters, ils_iters, perturb_k, seed, &B, &am, &xn2,
                                             &cst, false, sample_id_offset);
    std::memcpy(codes, B.data.data(), B.data.size());
    std::memcpy(a, am.data.data(), sizeof(float) * am.data.size());
    std::memcpy(cost, cst.data(), sizeof(float) * cst.size());
}

// stlq::BeamSearchPrefixLSLargeRootExpandFromRootCandidates (beam_search.cpp:728-992) for all
// n vectors. G_small Hs x Hs, G0S h0 x Hs, xC_small Hs x n; root_* are [n, H_beam] row-major.
void ref_expand_large_root(const float* G_small, int Hs, const float* G0S, int h0, const int* h_vec, int m,
                           const float* xC_small, int n, int H_beam, const float* root_errs, const int* root_codes,
                           const float* root_a0, const float* root_r00, uint32_t* cluster_id, uint8_t* B_small) {
    stlq::PrecompLargeRoot pre;
    pre.m = m;
    pre.h_vec.assign(h_vec, h_vec + m);
    int off = 0;
    for (int l = 0; l < m; ++l) {
        pre.offsets.push_back(off);
        off += h_vec[l];
    }
    pre.H_small = Hs;
    pre.small_offsets.assign(m, 0);
    int so = 0;
    for (int l = 1; l < m; ++l) {
        pre.small_offsets[l] = so;
        so += h_vec[l];
    }
    pre.G_small = Wrap(G_small, Hs, Hs);
    pre.G0S = Wrap(G0S, h0, Hs);
    pre.ready = true;
    const auto xs = Wrap(xC_small, Hs, n);
    std::vector<std::uint32_t> cid(static_cast<std::size_t>(n), 0u);  // the callee writes, not resizes
    stlq::ColMajorMatrix<stlq::Code> Bs(m - 1, n);
    stlq::BeamSearchPrefixLSLargeRootExpandFromRootCandidates(pre, xs, 0, n, H_beam, root_errs, root_codes, root_a0,
                                                             root_r00, &cid, &Bs);
    std::memcpy(cluster_id, cid.data(), sizeof(uint32_t) * static_cast<std::size_t>(n));
    std::memcpy(B_small, Bs.data.data(), Bs.data.size());
}

// stlq::SolveLeastSquaresAllLargeRoot (least_squares.cpp:667-745). B_small (m-1) x n.
void ref_solve_ls_all_large_root(const float* X, int d, int n, const float* C0, const float* norm0,
                                 const float* G_small, int Hs, const float* G0S, const int* h_vec, int m,
                                 const float* xC_small, const uint32_t* cluster_id, const uint8_t* B_small, float* a) {
    const auto pre = MakePrecompLargeRoot(d, m, h_vec, C0, norm0, G_small, Hs, G0S, nullptr);
    const auto Xm = Wrap(X, d, n);
    const auto xs = Wrap(xC_small, Hs, n);
    const std::vector<std::uint32_t> cid(cluster_id, cluster_id + n);
    const auto Bs = Wrap(B_small, m - 1, n);
    stlq::ColMajorMatrix<float> am;
    stlq::SolveLeastSquaresAllLargeRoot(pre, Xm, xs, cid, Bs, &am);
    std::memcpy(a, am.data.data(), sizeof(float) * am.data.size());
}

// stlq::ComputeCostsLargeRoot (cost_utils.cpp:211-233).
void ref_compute_costs_large_root(const float* X, int d, int n, const float* C0, const float* norm0,
                                  const float* G_small, int Hs, const float* G0S, const int* h_vec, int m,
                                  const float* xC_small, const uint32_t* cluster_id, const uint8_t* B_small,
                                  const float* a, const float* nx2, float* cost) {
    const auto pre = MakePrecompLargeRoot(d, m, h_vec, C0, norm0, G_small, Hs, G0S, nullptr);
    const auto Xm = Wrap(X, d, n);
    const auto xs = Wrap(xC_small, Hs, n);
    const std::vector<std::uint32_t> cid(cluster_id, cluster_id + n);
    const auto Bs = Wrap(B_small, m - 1, n);
    const auto am = Wrap(a, m, n);
    const std::vector<float> xn(nx2, nx2 + n);
    std::vector<float> out;
    stlq::ComputeCostsLargeRoot(pre, Xm, xs, cid, Bs, am, xn, &out);
    std::memcpy(cost, out.data(), sizeof(float) * static_cast<std::size_t>(n));
}

// stlq::DynamicIcmWithIls{Abs,NoAbs}NoNormalLargeRoot (icm.cpp:1005-1120, wrappers below it):
// LS refit, costs, ICM sweeps and ILS rounds with the roots fixed. B_small is updated in place.
void ref_icm_large_root(const float* X, int d, int n, const float* C0, const float* norm0, const float* G_small,
                        int Hs, const float* G0S, const float* invnorm_small, const int* h_vec, int m,
                        const float* xC_small, const uint32_t* cluster_id, int icm_iters, int ils_iters,
                        int perturb_k, int use_abs, uint32_t seed, uint64_t sample_id_offset, uint8_t* B_small,
                        float* a, float* cost) {
    const auto pre = MakePrecompLargeRoot(d, m, h_vec, C0, norm0, G_small, Hs, G0S, invnorm_small);
    const auto Xm = Wrap(X, d, n);
    const auto xs = Wrap(xC_small, Hs, n);
    const std::vector<std::uint32_t> cid(cluster_id, cluster_id + n);
    auto Bs = Wrap(B_small, m - 1, n);
    stlq::ColMajorMatrix<float> am;
    std::vector<float> xn2, cst;
    if (use_abs)
        stlq::DynamicIcmWithIlsAbsNoNormalLargeRoot(Xm, pre, xs, icm_iters, ils_iters, perturb_k, seed, cid, &Bs, &am,
                                                   &xn2, &cst, false, sample_id_offset);
    else
        stlq::DynamicIcmWithIlsNoAbsNoNormalLargeRoot(Xm, pre, xs, icm_iters, ils_iters, perturb_k, seed, cid, &Bs,
                                                     &am, &xn2, &cst, false, sample_id_offset);
    std::memcpy(B_small, Bs.data.data(), Bs.data.size());
    std::memcpy(a, am.data.data(), sizeof(float) * am.data.size());
    std::memcpy(cost, cst.data(), sizeof(float) * cst.size());
}


// Writes a store with the reference's io::BaseBasicWriter (src/io/base_store.cpp): Open (or, with
// resume, OpenResume at resume_start with the given committed bucket sizes), then one append per
// block (block b: vectors off_b .. off_b + counts[b] - 1 of the concatenated arrays, global ids
// from starts[b]) by the variant raw_kind selects (0 AppendBlock without vectors, 1
// AppendBlockRawU8, 2 AppendBlockRawF32, 3 AppendBlock with a d x count uint8 matrix), each
// followed, when ckpt_path is set, by the pipeline's commit (writer Flush, then
// app::OnCommitBaseBasicCkpt with next id = block end). Close at the end. Returns 1, or 0 with
// the reference's message in err; out_bucket_bytes (nbucket entries) gets bucket_file_bytes().
int ref_store_write(const char* dir, int d, int m, const int* h_vec, int h_len, int shard_size, int bucket_size,
                    int flush_mb, int wvb, int wbb, int raw_bytes, int resume, uint64_t resume_start,
                    const uint64_t* bucket_sizes, int nbucket, int nblocks, const uint64_t* starts,
                    const int64_t* counts, const uint32_t* cluster_id, const uint8_t* B_small, const float* a,
                    int raw_kind, const void* raw, const char* ckpt_path, uint64_t* out_bucket_bytes, char* err,
                    int err_len) {
    stlq::io::BaseBasicStoreConfig cfg;
    cfg.dir = dir;
    cfg.d = d;
    cfg.m = m;
    cfg.h_vec.assign(h_vec, h_vec + h_len);
    cfg.shard_size = shard_size;
    cfg.bucket_size = bucket_size;
    cfg.bucket_flush_mb = flush_mb;
    cfg.write_vector_bucket = wvb != 0;
    cfg.write_basic_to_bucket = wbb != 0;
    cfg.raw_bytes_per_vec = raw_bytes;
    std::string e;
    auto done = [&](int ok) {
        if (err && err_len > 0) {
            std::strncpy(err, e.c_str(), static_cast<std::size_t>(err_len) - 1);
            err[err_len - 1] = 0;
        }
        return ok;
    };
    stlq::io::BaseBasicWriter w;
    const bool opened = resume ? w.OpenResume(cfg, resume_start,
                                              std::vector<std::uint64_t>(bucket_sizes, bucket_sizes + nbucket), &e)
                               : w.Open(cfg, &e);
    if (!opened) return done(0);
    stlq::app::BaseBasicCkptCtx hook;
    if (ckpt_path) {
        hook.path = ckpt_path;
        hook.nbucket = static_cast<std::uint32_t>(stlq::app::ComputeNbucketsForBasic(cfg));
    }
    const int mc = std::max(0, m - 1);
    const std::size_t esz = raw_kind == 2 ? sizeof(float) : 1;
    std::size_t off = 0;
    for (int b = 0; b < nblocks; ++b) {
        const int cnt = static_cast<int>(counts[b]);
        const std::vector<std::uint32_t> cid(cluster_id + off, cluster_id + off + cnt);
        const auto Bs = Wrap(B_small ? B_small + off * mc : nullptr, mc, cnt);
        const auto am = Wrap(a + off * m, m, cnt);
        const auto* rp = raw ? static_cast<const std::uint8_t*>(raw) + off * static_cast<std::size_t>(d) * esz : nullptr;
        bool ok = false;
        if (raw_kind == 1) {
            ok = w.AppendBlockRawU8(starts[b], cid, Bs, am, rp, d, &e);
        } else if (raw_kind == 2) {
            ok = w.AppendBlockRawF32(starts[b], cid, Bs, am, reinterpret_cast<const float*>(rp), d, &e);
        } else if (raw_kind == 3) {
            const auto xm = Wrap(rp, d, cnt);
            ok = w.AppendBlock(starts[b], cid, Bs, am, &xm, &e);
        } else {
            ok = w.AppendBlock(starts[b], cid, Bs, am, nullptr, &e);
        }
        if (!ok) return done(0);
        if (ckpt_path) {
            if (!w.Flush(&e)) return done(0);
            if (!stlq::app::OnCommitBaseBasicCkpt(starts[b] + static_cast<std::uint64_t>(cnt), &w, &hook, &e))
                return done(0);
        }
        off += static_cast<std::size_t>(cnt);
    }
    if (!w.Close(&e)) return done(0);
    if (out_bucket_bytes)
        for (std::size_t i = 0; i < w.bucket_file_bytes().size() && static_cast<int>(i) < nbucket; ++i)
            out_bucket_bytes[i] = w.bucket_file_bytes()[i];
    return done(1);
}

// app::ReadBaseBasicCheckpoint + app::TruncateBaseBasicToCheckpoint
// (src/pipeline/main_virtual_helpers.cpp:126-275): reads ckpt_path, cuts the store back to it and
// returns the checkpoint's next id and bucket sizes (cap entries). Returns 1, or 0 with err.
int ref_store_truncate(const char* dir, int m, const int* h_vec, int h_len, int shard_size, int bucket_size,
                       const char* ckpt_path, uint64_t* next_id, uint64_t* bucket_sizes, int cap, int* nbucket,
                       char* err, int err_len) {
    stlq::io::BaseBasicStoreConfig cfg;
    cfg.dir = dir;
    cfg.m = m;
    cfg.h_vec.assign(h_vec, h_vec + h_len);
    cfg.shard_size = shard_size;
    cfg.bucket_size = bucket_size;
    std::string e;
    stlq::app::BaseBasicCheckpoint ck;
    bool ok = stlq::app::ReadBaseBasicCheckpoint(ckpt_path, &ck, &e) &&
              stlq::app::TruncateBaseBasicToCheckpoint(dir, cfg, ck, &e);
    if (ok) {
        *next_id = ck.next_id;
        *nbucket = static_cast<int>(ck.bucket_sizes.size());
        for (int i = 0; i < cap && i < *nbucket; ++i) bucket_sizes[i] = ck.bucket_sizes[static_cast<std::size_t>(i)];
    }
    if (err && err_len > 0) {
        std::strncpy(err, e.c_str(), static_cast<std::size_t>(err_len) - 1);
        err[err_len - 1] = 0;
    }
    return ok ? 1 : 0;
}

}  // extern "C"
