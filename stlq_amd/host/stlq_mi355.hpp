// C++ host mirror of STLQ's encoder interface on top of the libstlq_mi355 C ABI.
//
// The types and free functions below carry the reference's names, argument order and meaning
// (include/stlq/common/types.h, include/stlq/quantizer/{encoder,beam_search,icm,least_squares,
// cost_utils,precomp_large_root}.h) so that an EncodeBase-style caller can switch to the MI355X
// encoder by changing a namespace. They live in stlq_mi355::stlq to avoid clashing with the
// reference's own definitions when both are linked into one program.
//
// Device state: one context per host thread (thread_local, device 0 unless SetDevice is called
// first). The codebook precomp is uploaded once per Precomp::build_tag, the way the reference's
// CUDA sessions cache device copies (beam_search_cuda_api.inc:34, :244-245).
//
// Errors: the reference's CPU functions return void/bool and its CUDA paths throw
// std::runtime_error (beam_search_cuda_kernels.inc:5-14); here every failure of the C ABI throws
// std::runtime_error with the library's message.
#pragma once

#include <algorithm>
#include <cstdint>
#include <memory>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

#include "stlq_mi355.h"
#include "stlq_mi355_store.h"

namespace stlq_mi355 {
namespace stlq {

using Code = std::uint8_t;
using FullCode = Code;

template <typename T>
struct ColMajorMatrix {  // include/stlq/common/types.h:35-51
    int rows = 0;
    int cols = 0;
    std::vector<T> data;
    ColMajorMatrix() = default;
    ColMajorMatrix(int r, int c) : rows(r), cols(c), data(static_cast<std::size_t>(r) * c) {}
    T* Col(int j) { return data.data() + static_cast<std::size_t>(j) * rows; }
    const T* Col(int j) const { return data.data() + static_cast<std::size_t>(j) * rows; }
    T& operator()(int i, int j) { return data[static_cast<std::size_t>(j) * rows + i]; }
    const T& operator()(int i, int j) const { return data[static_cast<std::size_t>(j) * rows + i]; }
};

struct CodebookPack {  // types.h:53-60
    int d = 0;
    std::vector<int> h_vec;
    std::vector<ColMajorMatrix<float>> books;
    std::uint64_t build_tag = 0;
};

struct Precomp {  // types.h:62-75
    ColMajorMatrix<float> C_all;
    ColMajorMatrix<float> G;
    std::vector<int> offsets;
    std::vector<int> flat_layer;
    std::vector<int> h_vec;
    std::vector<float> invnorm_flat;
    int H = 0;
    int d = 0;
    int m = 0;
    std::uint64_t build_tag = 0;
};

struct BaseEncoding {  // types.h:77-80
    ColMajorMatrix<FullCode> B;
    ColMajorMatrix<float> a;
};

struct EncodeOptions {  // base.encode.* (config.h:473-482)
    bool use_abs = true;
    int H_beam = 2;
    int ils_iters = 0;
    int icm_iters = 4;
    int perturb_k = 3;
    int seed = 38251450;
};

namespace detail {

inline void Check(int rc) {
    if (rc != STLQ_MI355_OK) throw std::runtime_error(std::string("stlq_mi355: ") + stlq_mi355_last_error());
}

struct Session {
    stlq_mi355_ctx* ctx = nullptr;
    const void* owner = nullptr;     // Precomp bound to ctx
    std::uint64_t tag = 0;
    int d = 0;
    const void* lr_owner = nullptr;  // PrecompLargeRoot bound to ctx
    std::uint64_t lr_tag = 0;
    ~Session() {
        if (ctx) stlq_mi355_ctx_destroy(ctx);
    }
};

inline int& DeviceOrdinal() {
    static thread_local int dev = 0;
    return dev;
}

inline Session& ThreadSession() {
    static thread_local Session s;
    if (!s.ctx) Check(stlq_mi355_ctx_create(DeviceOrdinal(), &s.ctx));
    return s;
}

inline std::uint64_t NextBuildTag() {
    static std::uint64_t tag = 0;
    return ++tag;
}

// Uploads the precomp unless this thread's context already holds the one with this build tag.
inline stlq_mi355_ctx* Bind(const Precomp& pre) {
    Session& s = ThreadSession();
    if (s.owner != &pre || s.tag != pre.build_tag || pre.build_tag == 0) {
        Check(stlq_mi355_set_precomp(s.ctx, pre.d, pre.m, pre.h_vec.data(), pre.C_all.data.data(),
                                     pre.G.data.data(), pre.invnorm_flat.data()));
        s.owner = &pre;
        s.tag = pre.build_tag;
        s.d = pre.d;
    }
    return s.ctx;
}

}  // namespace detail

// Selects the HIP device of the calling thread's context (before its first use).
inline void SetDevice(int device) { detail::DeviceOrdinal() = device; }

// BuildPrecomp (src/quantizer/encoder_precomp.inc:1-53): C_all, offsets, invnorm and
// G = C_all^T C_all, computed on the device and copied back.
inline bool BuildPrecomp(const CodebookPack& codebooks, Precomp* precomp) {
    if (!precomp || codebooks.books.empty()) return false;
    const int m = static_cast<int>(codebooks.books.size());
    const int d = codebooks.books.front().rows;
    Precomp& p = *precomp;
    p.m = m;
    p.d = d;
    p.h_vec.clear();
    p.offsets.assign(m, 0);
    int H = 0;
    for (int l = 0; l < m; ++l) {
        p.offsets[l] = H;
        p.h_vec.push_back(codebooks.books[l].cols);
        H += codebooks.books[l].cols;
    }
    p.H = H;
    p.C_all = ColMajorMatrix<float>(d, H);
    p.flat_layer.assign(H, 0);
    for (int l = 0; l < m; ++l) {
        const auto& b = codebooks.books[l];
        std::copy(b.data.begin(), b.data.end(), p.C_all.Col(p.offsets[l]));
        for (int c = 0; c < b.cols; ++c) p.flat_layer[p.offsets[l] + c] = l;
    }
    p.G = ColMajorMatrix<float>(H, H);
    p.invnorm_flat.assign(H, 0.0f);
    detail::Session& s = detail::ThreadSession();
    detail::Check(stlq_mi355_set_codebooks(s.ctx, d, m, p.h_vec.data(), p.C_all.data.data()));
    detail::Check(stlq_mi355_get_precomp(s.ctx, p.G.data.data(), p.invnorm_flat.data()));
    p.build_tag = detail::NextBuildTag();
    s.owner = &p;
    s.tag = p.build_tag;
    s.d = d;
    return true;
}

// ComputeXNorm2 (src/quantizer/cost_utils.cpp:88-110, cost_utils.h:12), on this thread's context.
inline void ComputeXNorm2(const ColMajorMatrix<float>& X, std::vector<float>* X_norm2) {
    X_norm2->resize(static_cast<std::size_t>(X.cols));
    detail::Check(stlq_mi355_xnorm2(detail::ThreadSession().ctx, X.data.data(), X.rows, X.cols, X_norm2->data()));
}

// xC = C_all^T X (StreamKernelProvider::Gemm call site, encoder_encode_base.inc:86-90).
inline void ComputeXc(const Precomp& pre, const ColMajorMatrix<float>& X, ColMajorMatrix<float>* xC) {
    *xC = ColMajorMatrix<float>(pre.H, X.cols);
    detail::Check(stlq_mi355_gemm_xc(detail::Bind(pre), X.data.data(), X.cols, xC->data.data()));
}

// BeamSearchPrefixLS (src/quantizer/beam_search.cpp:196-422).
inline void BeamSearchPrefixLS(const ColMajorMatrix<float>& X, const Precomp& precomp,
                               const ColMajorMatrix<float>& xC, int H_beam, ColMajorMatrix<FullCode>* B) {
    *B = ColMajorMatrix<FullCode>(precomp.m, X.cols);
    detail::Check(stlq_mi355_beam_search(detail::Bind(precomp), X.data.data(), nullptr, xC.data.data(), X.cols,
                                         std::max(1, H_beam), B->data.data(), nullptr));
}

// SolveLeastSquaresAll (src/quantizer/least_squares.cpp:406-565).
inline void SolveLeastSquaresAll(const Precomp& precomp, const ColMajorMatrix<float>& xC,
                                 const ColMajorMatrix<FullCode>& B, ColMajorMatrix<float>* a) {
    *a = ColMajorMatrix<float>(precomp.m, B.cols);
    int64_t fails = 0;
    detail::Check(stlq_mi355_solve_ls_all(detail::Bind(precomp), xC.data.data(), B.data.data(), B.cols,
                                          a->data.data(), &fails));
}

// ComputeCosts (src/quantizer/cost_utils.cpp:139-158).
inline void ComputeCosts(const Precomp& precomp, const ColMajorMatrix<float>& xC, const ColMajorMatrix<FullCode>& B,
                         const ColMajorMatrix<float>& a, const std::vector<float>& X_norm2,
                         std::vector<float>* out_cost) {
    out_cost->resize(static_cast<std::size_t>(B.cols));
    detail::Check(stlq_mi355_compute_costs(detail::Bind(precomp), xC.data.data(), B.data.data(), a.data.data(),
                                           X_norm2.data(), B.cols, out_cost->data()));
}

namespace detail {
inline void DynamicIcm(const ColMajorMatrix<float>& X, const Precomp& precomp, const ColMajorMatrix<float>& xC,
                       int icm_iters, int ils_iters, int perturb_k, std::uint32_t seed, bool use_abs,
                       ColMajorMatrix<FullCode>* B, ColMajorMatrix<float>* a, std::vector<float>* X_norm2,
                       std::vector<float>* cost, std::uint64_t sample_id_offset) {
    stlq_mi355_ctx* ctx = Bind(precomp);
    if (X_norm2 && X_norm2->empty()) ComputeXNorm2(X, X_norm2);
    std::vector<float> cost_local;
    std::vector<float>* c = cost ? cost : &cost_local;
    c->resize(static_cast<std::size_t>(B->cols));
    *a = ColMajorMatrix<float>(precomp.m, B->cols);
    Check(stlq_mi355_icm_ils(ctx, X.data.data(), X_norm2 ? X_norm2->data() : nullptr, xC.data.data(), B->cols,
                             icm_iters, ils_iters, perturb_k, use_abs ? 1 : 0, seed, sample_id_offset,
                             B->data.data(), a->data.data(), c->data()));
}
}  // namespace detail

// DynamicIcmWithIlsAbsNoNormal / ...NoAbsNoNormal (src/quantizer/icm.cpp:1132-1170, icm.h:15-43).
inline void DynamicIcmWithIlsAbsNoNormal(const ColMajorMatrix<float>& X, const Precomp& precomp,
                                         const ColMajorMatrix<float>& xC, int icm_iters, int ils_iters, int perturb_k,
                                         std::uint32_t seed, ColMajorMatrix<FullCode>* B, ColMajorMatrix<float>* a,
                                         std::vector<float>* X_norm2, std::vector<float>* cost,
                                         bool print_progress = true, std::uint64_t sample_id_offset = 0) {
    (void)print_progress;
    detail::DynamicIcm(X, precomp, xC, icm_iters, ils_iters, perturb_k, seed, true, B, a, X_norm2, cost,
                       sample_id_offset);
}

inline void DynamicIcmWithIlsNoAbsNoNormal(const ColMajorMatrix<float>& X, const Precomp& precomp,
                                           const ColMajorMatrix<float>& xC, int icm_iters, int ils_iters,
                                           int perturb_k, std::uint32_t seed, ColMajorMatrix<FullCode>* B,
                                           ColMajorMatrix<float>* a, std::vector<float>* X_norm2,
                                           std::vector<float>* cost, bool print_progress = true,
                                           std::uint64_t sample_id_offset = 0) {
    (void)print_progress;
    detail::DynamicIcm(X, precomp, xC, icm_iters, ils_iters, perturb_k, seed, false, B, a, X_norm2, cost,
                       sample_id_offset);
}

// EncodeBase (src/quantizer/encoder_encode_base.inc:1-106); the whole pipeline (xC GEMM, beam,
// LS, ICM, ILS, costs) runs on the device.
inline bool EncodeBase(const EncodeOptions& opt, const ColMajorMatrix<float>& Xb, const CodebookPack& codebooks,
                       const Precomp& precomp, BaseEncoding* base, float* out_beam_mse, float* out_final_mse,
                       std::string* error) {
    if (!base) {
        if (error) *error = "BaseEncoding output is null.";
        return false;
    }
    if (Xb.rows <= 0 || Xb.cols <= 0) {
        if (error) *error = "Empty base dataset.";
        return false;
    }
    if (precomp.d != Xb.rows || precomp.m != static_cast<int>(codebooks.books.size())) {
        if (error) *error = "Precomp dimensions do not match codebooks or dataset.";
        return false;
    }
    stlq_mi355_encode_params p{std::max(1, opt.H_beam), opt.icm_iters, opt.ils_iters, opt.perturb_k,
                               opt.use_abs ? 1 : 0, static_cast<std::uint32_t>(opt.seed), 1};
    base->B = ColMajorMatrix<FullCode>(precomp.m, Xb.cols);
    base->a = ColMajorMatrix<float>(precomp.m, Xb.cols);
    double bm = 0.0, fm = 0.0;
    const int rc = stlq_mi355_encode(detail::Bind(precomp), Xb.data.data(), Xb.cols, &p, base->B.data.data(),
                                     base->a.data.data(), nullptr, &bm, &fm);
    if (rc != STLQ_MI355_OK) {
        if (error) *error = stlq_mi355_last_error();
        return false;
    }
    if (out_beam_mse) *out_beam_mse = static_cast<float>(bm);
    if (out_final_mse) *out_final_mse = static_cast<float>(fm);
    return true;
}

// The configuration fields the encoder reads (include/stlq/common/config.h: base.encode.*,
// :473-482; large.base_block, :573; runtime.*, :60-67). Defaults are the reference's.
struct BaseEncodeConfig {
    bool use_abs = true;
    int H_beam = 2;
    int ils_iters = 0;
    int icm_iters = 4;
    int perturb_k = 3;
    int seed = 38251450;
};
struct BaseConfig {
    BaseEncodeConfig encode;
};
struct LargeConfig {
    int base_block = 200000;
    bool write_vector_bucket = true;  // config.h:583: store raw vectors beside the codes
};
struct RuntimeConfig {
    bool use_cuda = false;
    int cuda_device = 0;
    std::string cuda_mode = "strict";
};
struct Config {
    BaseConfig base;
    LargeConfig large;
    RuntimeConfig runtime;
};

struct Dataset {  // types.h:190-195
    ColMajorMatrix<float> Xt;
    ColMajorMatrix<float> Xb;
    ColMajorMatrix<float> Xq;
    std::vector<int> gt;
};

class KernelProvider;  // legacy provider; EncodeBase ignores it (encoder_encode_base.inc:10)

// EncodeBase with the reference's signature (include/stlq/quantizer/encoder.h:66-74): encodes
// dataset.Xb with config.base.encode.
inline bool EncodeBase(const Config& config, const Dataset& dataset, const CodebookPack& codebooks,
                       const Precomp& precomp, KernelProvider* kernels, BaseEncoding* base, float* out_beam_mse,
                       float* out_final_mse, std::string* error) {
    (void)kernels;
    const BaseEncodeConfig& e = config.base.encode;
    EncodeOptions opt;
    opt.use_abs = e.use_abs;
    opt.H_beam = e.H_beam;
    opt.ils_iters = e.ils_iters;
    opt.icm_iters = e.icm_iters;
    opt.perturb_k = e.perturb_k;
    opt.seed = e.seed;
    return EncodeBase(opt, dataset.Xb, codebooks, precomp, base, out_beam_mse, out_final_mse, error);
}

class StreamKernelProvider;  // the reference's GEMM provider; unused here (the device runs the GEMMs)

struct PrecompLargeRootBuildOptions {  // precomp_large_root.h:40-47 (CPU-only options)
    bool build_g0s_transpose = false;
    int g0s_transpose_max_mb = 0;
};

// PrecompLargeRoot (precomp_large_root.h:12-39). norm0, G_small, invnorm_small_flat and G0S are
// computed on the device and stay there; the host copies of those members remain empty.
struct PrecompLargeRoot {
    int d = 0;
    int m = 0;
    std::vector<int> h_vec;
    std::vector<int> offsets;
    std::uint64_t build_tag = 0;
    ColMajorMatrix<float> C0;
    std::vector<float> norm0;
    int H_small = 0;
    std::vector<int> small_offsets;
    ColMajorMatrix<float> C_small;
    ColMajorMatrix<float> G_small;
    std::vector<float> invnorm_small_flat;
    ColMajorMatrix<float> G0S;
    ColMajorMatrix<float> G0S_T;
    bool ready = false;
};

struct BeamSearchLargeRootTiming {  // beam_search.h:11-16
    double norm_x2 = 0.0;
    double root_gemm = 0.0;
    double root_update = 0.0;
    double expand = 0.0;
};

namespace detail {
inline stlq_mi355_ctx* BindLargeRoot(const PrecompLargeRoot& pre) {
    if (!pre.ready) throw std::runtime_error("stlq_mi355: PrecompLargeRoot is not built");
    Session& s = ThreadSession();
    if (s.lr_owner != &pre || s.lr_tag != pre.build_tag || pre.build_tag == 0) {
        Check(stlq_mi355_set_large_root(s.ctx, pre.d, pre.m, pre.h_vec.data(), pre.C0.data.data(),
                                        pre.C_small.data.data()));
        s.lr_owner = &pre;
        s.lr_tag = pre.build_tag;
    }
    return s.ctx;
}
}  // namespace detail

// BuildPrecompLargeRoot (src/quantizer/precomp_large_root.cpp:27-157): layer 0 of C_root is
// the large root codebook, layers 1..m-1 the small ones (at most 256 codewords each).
inline bool BuildPrecompLargeRoot(const CodebookPack& C_root, StreamKernelProvider* kernels,
                                  const PrecompLargeRootBuildOptions& opts, PrecompLargeRoot* out,
                                  std::string* err) {
    (void)kernels;
    (void)opts;
    if (!out || C_root.books.size() < 2) {
        if (err) *err = "large-root precomp needs a root and at least one small codebook";
        return false;
    }
    PrecompLargeRoot& p = *out;
    p = PrecompLargeRoot();
    p.m = static_cast<int>(C_root.books.size());
    p.d = C_root.books.front().rows;
    int H = 0;
    for (int l = 0; l < p.m; ++l) {
        p.offsets.push_back(H);
        p.h_vec.push_back(C_root.books[l].cols);
        H += C_root.books[l].cols;
    }
    p.C0 = C_root.books[0];
    p.small_offsets.assign(p.m, 0);
    for (int l = 1; l < p.m; ++l) {
        p.small_offsets[l] = p.H_small;
        p.H_small += p.h_vec[l];
    }
    p.C_small = ColMajorMatrix<float>(p.d, p.H_small);
    for (int l = 1; l < p.m; ++l) {
        const auto& b = C_root.books[l];
        std::copy(b.data.begin(), b.data.end(), p.C_small.Col(p.small_offsets[l]));
    }
    p.ready = true;
    p.build_tag = detail::NextBuildTag();
    try {
        detail::Session& s = detail::ThreadSession();
        const int rc = stlq_mi355_set_large_root(s.ctx, p.d, p.m, p.h_vec.data(), p.C0.data.data(),
                                                 p.C_small.data.data());
        if (rc != STLQ_MI355_OK) {
            if (err) *err = stlq_mi355_last_error();
            p.ready = false;
            return false;
        }
        s.lr_owner = &p;
        s.lr_tag = p.build_tag;
    } catch (const std::exception& e) {
        if (err) *err = e.what();
        p.ready = false;
        return false;
    }
    return true;
}

// BeamSearchPrefixLSLargeRoot (src/quantizer/beam_search.cpp:579-726, beam_search.h:26-32).
// An empty xC_small (rows == 0) has the device compute C_small^T X itself.
inline void BeamSearchPrefixLSLargeRoot(const ColMajorMatrix<float>& X, const PrecompLargeRoot& pre,
                                        const ColMajorMatrix<float>& xC_small, int H_beam,
                                        std::vector<std::uint32_t>* cluster_id, ColMajorMatrix<Code>* B_small,
                                        BeamSearchLargeRootTiming* timing = nullptr) {
    stlq_mi355_ctx* ctx = detail::BindLargeRoot(pre);
    cluster_id->assign(static_cast<std::size_t>(X.cols), 0u);
    *B_small = ColMajorMatrix<Code>(pre.m - 1, X.cols);
    const float* xcs = xC_small.rows > 0 ? xC_small.data.data() : nullptr;
    detail::Check(stlq_mi355_beam_search_large_root(ctx, X.data.data(), xcs, X.cols, std::max(1, H_beam), nullptr, 0,
                                                    cluster_id->data(), B_small->data.data(), nullptr));
    if (timing) {
        stlq_mi355_timings t{};
        detail::Check(stlq_mi355_last_timings(ctx, &t));
        timing->norm_x2 = 0.0;
        timing->root_gemm = t.gemm_ms * 1e-3;
        timing->root_update = 0.0;
        timing->expand = t.beam_ms * 1e-3;
    }
}

// SolveLeastSquaresAllLargeRoot (src/quantizer/least_squares.cpp:667-745, least_squares.h:54-59).
// An empty xC_small (rows == 0) has the device compute C_small^T X itself.
inline void SolveLeastSquaresAllLargeRoot(const PrecompLargeRoot& pre, const ColMajorMatrix<float>& X,
                                          const ColMajorMatrix<float>& xC_small,
                                          const std::vector<std::uint32_t>& cluster_id,
                                          const ColMajorMatrix<Code>& B_small, ColMajorMatrix<float>* a) {
    stlq_mi355_ctx* ctx = detail::BindLargeRoot(pre);
    *a = ColMajorMatrix<float>(pre.m, X.cols);
    const float* xcs = xC_small.rows > 0 ? xC_small.data.data() : nullptr;
    detail::Check(stlq_mi355_solve_ls_all_large_root(ctx, X.data.data(), xcs, X.cols, cluster_id.data(),
                                                     B_small.data.data(), a->data.data(), nullptr));
}

// ComputeCostsLargeRoot (src/quantizer/cost_utils.cpp:211-233, cost_utils.h:37-44).
inline void ComputeCostsLargeRoot(const PrecompLargeRoot& pre, const ColMajorMatrix<float>& X,
                                  const ColMajorMatrix<float>& xC_small, const std::vector<std::uint32_t>& cluster_id,
                                  const ColMajorMatrix<Code>& B_small, const ColMajorMatrix<float>& a,
                                  const std::vector<float>& X_norm2, std::vector<float>* out_cost) {
    if (!out_cost) return;
    stlq_mi355_ctx* ctx = detail::BindLargeRoot(pre);
    out_cost->resize(static_cast<std::size_t>(std::max(0, B_small.cols)));
    const float* xcs = xC_small.rows > 0 ? xC_small.data.data() : nullptr;
    const float* nx2 = X_norm2.empty() ? nullptr : X_norm2.data();
    detail::Check(stlq_mi355_compute_costs_large_root(ctx, X.data.data(), xcs, X.cols, cluster_id.data(),
                                                      B_small.data.data(), a.data.data(), nx2, out_cost->data()));
}

namespace detail {
inline void DynamicIcmLargeRoot(const ColMajorMatrix<float>& X, const PrecompLargeRoot& pre,
                                const ColMajorMatrix<float>& xC_small, int icm_iters, int ils_iters, int perturb_k,
                                std::uint32_t seed, bool use_abs, const std::vector<std::uint32_t>& cluster_id,
                                ColMajorMatrix<Code>* B_small, ColMajorMatrix<float>* a, std::vector<float>* X_norm2,
                                std::vector<float>* cost, std::uint64_t sample_id_offset) {
    if (!B_small || !a) return;  // icm.cpp:1020-1022
    stlq_mi355_ctx* ctx = BindLargeRoot(pre);
    if (X_norm2->empty()) {  // icm.cpp:368-370
        X_norm2->resize(static_cast<std::size_t>(X.cols));
        Check(stlq_mi355_xnorm2(ctx, X.data.data(), X.rows, X.cols, X_norm2->data()));
    }
    *a = ColMajorMatrix<float>(pre.m, B_small->cols);
    std::vector<float> local;
    std::vector<float>* c = cost ? cost : &local;
    c->resize(static_cast<std::size_t>(B_small->cols));
    const float* xcs = xC_small.rows > 0 ? xC_small.data.data() : nullptr;
    Check(stlq_mi355_icm_ils_large_root(ctx, X.data.data(), X_norm2->data(), xcs, X.cols, cluster_id.data(),
                                        icm_iters, ils_iters, perturb_k, use_abs ? 1 : 0, seed, sample_id_offset,
                                        B_small->data.data(), a->data.data(), c->data()));
}
}  // namespace detail

// DynamicIcmWithIls{NoAbs,Abs}NoNormalLargeRoot (src/quantizer/icm.cpp:1005-1120, icm.h:45-75).
inline void DynamicIcmWithIlsNoAbsNoNormalLargeRoot(const ColMajorMatrix<float>& X, const PrecompLargeRoot& pre,
                                                    const ColMajorMatrix<float>& xC_small, int icm_iters,
                                                    int ils_iters, int perturb_k, std::uint32_t seed,
                                                    const std::vector<std::uint32_t>& cluster_id,
                                                    ColMajorMatrix<Code>* B_small, ColMajorMatrix<float>* a,
                                                    std::vector<float>* X_norm2, std::vector<float>* cost,
                                                    bool print_progress = true, std::uint64_t sample_id_offset = 0) {
    (void)print_progress;
    detail::DynamicIcmLargeRoot(X, pre, xC_small, icm_iters, ils_iters, perturb_k, seed, false, cluster_id, B_small,
                                a, X_norm2, cost, sample_id_offset);
}

inline void DynamicIcmWithIlsAbsNoNormalLargeRoot(const ColMajorMatrix<float>& X, const PrecompLargeRoot& pre,
                                                  const ColMajorMatrix<float>& xC_small, int icm_iters,
                                                  int ils_iters, int perturb_k, std::uint32_t seed,
                                                  const std::vector<std::uint32_t>& cluster_id,
                                                  ColMajorMatrix<Code>* B_small, ColMajorMatrix<float>* a,
                                                  std::vector<float>* X_norm2, std::vector<float>* cost,
                                                  bool print_progress = true, std::uint64_t sample_id_offset = 0) {
    (void)print_progress;
    detail::DynamicIcmLargeRoot(X, pre, xC_small, icm_iters, ils_iters, perturb_k, seed, true, cluster_id, B_small, a,
                                X_norm2, cost, sample_id_offset);
}

namespace io {

// io::BaseBasicStoreConfig (include/stlq/io/base_store.h:12-25), the reference's defaults.
struct BaseBasicStoreConfig {
    std::string dir;
    int d = 0;
    int m = 0;
    std::vector<int> h_vec;
    int shard_size = 2000000;
    int bucket_size = 256;
    int bucket_flush_mb = 256;
    bool write_vector_bucket = true;
    bool write_basic_to_bucket = true;
    int raw_bytes_per_vec = 0;
};

// io::BaseBasicWriter (include/stlq/io/base_store.h:28-100) over include/stlq_mi355_store.h:
// the reference's on-disk BaseBasicStore, byte for byte. Methods return false and set *err.
class BaseBasicWriter {
public:
    BaseBasicWriter() = default;
    BaseBasicWriter(const BaseBasicWriter&) = delete;
    BaseBasicWriter& operator=(const BaseBasicWriter&) = delete;
    ~BaseBasicWriter() {
        std::string ignored;
        (void)Close(&ignored);
    }

    bool Open(const BaseBasicStoreConfig& cfg, std::string* err) {
        std::string ignored;
        (void)Close(&ignored);
        const stlq_mi355_store_config c = ToC(cfg);
        return Ok(stlq_mi355_store_open(&c, &h_), err);
    }
    bool OpenResume(const BaseBasicStoreConfig& cfg, std::uint64_t start_id,
                    const std::vector<std::uint64_t>& bucket_sizes, std::string* err) {
        std::string ignored;
        (void)Close(&ignored);
        const stlq_mi355_store_config c = ToC(cfg);
        return Ok(stlq_mi355_store_open_resume(&c, start_id, bucket_sizes.data(),
                                               static_cast<std::int64_t>(bucket_sizes.size()), &h_),
                  err);
    }
    bool Close(std::string* err) {
        if (!h_) return true;
        const bool flushed = Ok(stlq_mi355_store_flush(h_), err);  // Close's own write-out, kept readable
        if (flushed) committed_ = Committed();
        stlq_mi355_store* h = h_;
        h_ = nullptr;
        return Ok(stlq_mi355_store_close(h), err) && flushed;
    }
    bool Flush(std::string* err) { return Ok(stlq_mi355_store_flush(h_), err); }

    const std::vector<std::uint64_t>& bucket_file_bytes() const {
        if (h_) committed_ = Committed();
        return committed_;
    }

    bool AppendBlock(std::uint64_t start_id, const std::vector<std::uint32_t>& cluster_id,
                     const ColMajorMatrix<Code>& B_small, const ColMajorMatrix<float>& a,
                     const ColMajorMatrix<std::uint8_t>* x_u8_optional, std::string* err) {
        if (x_u8_optional && x_u8_optional->cols != static_cast<int>(cluster_id.size())) {
            if (err) *err = "BaseBasicWriter::AppendBlock: x_u8 shape mismatch.";
            return false;
        }
        return Append(start_id, cluster_id, B_small, a,
                      x_u8_optional ? STLQ_MI355_RAW_U8 : STLQ_MI355_RAW_NONE,
                      x_u8_optional ? x_u8_optional->data.data() : nullptr,
                      x_u8_optional ? x_u8_optional->rows : 0, err);
    }
    bool AppendBlockRawU8(std::uint64_t start_id, const std::vector<std::uint32_t>& cluster_id,
                          const ColMajorMatrix<Code>& B_small, const ColMajorMatrix<float>& a,
                          const std::uint8_t* x_u8, int ld_x_u8, std::string* err) {
        return Append(start_id, cluster_id, B_small, a, STLQ_MI355_RAW_U8, x_u8, ld_x_u8, err);
    }
    bool AppendBlockRawF32(std::uint64_t start_id, const std::vector<std::uint32_t>& cluster_id,
                           const ColMajorMatrix<Code>& B_small, const ColMajorMatrix<float>& a,
                           const float* x_f32, int ld_x_f32, std::string* err) {
        return Append(start_id, cluster_id, B_small, a, STLQ_MI355_RAW_F32, x_f32, ld_x_f32, err);
    }

    stlq_mi355_store* handle() const { return h_; }

private:
    static stlq_mi355_store_config ToC(const BaseBasicStoreConfig& cfg) {
        stlq_mi355_store_config c{};
        c.dir = cfg.dir.c_str();
        c.d = cfg.d;
        c.m = cfg.m;
        c.h_vec = cfg.h_vec.data();
        c.h_len = static_cast<int>(cfg.h_vec.size());
        c.shard_size = cfg.shard_size;
        c.bucket_size = cfg.bucket_size;
        c.bucket_flush_mb = cfg.bucket_flush_mb;
        c.write_vector_bucket = cfg.write_vector_bucket ? 1 : 0;
        c.write_basic_to_bucket = cfg.write_basic_to_bucket ? 1 : 0;
        c.raw_bytes_per_vec = cfg.raw_bytes_per_vec;
        return c;
    }
    static bool Ok(int rc, std::string* err) {
        if (rc == STLQ_MI355_OK) return true;
        if (err) *err = stlq_mi355_last_error();
        return false;
    }
    std::vector<std::uint64_t> Committed() const {
        std::int64_t nb = 0;
        stlq_mi355_store_bucket_bytes(h_, nullptr, 0, &nb);
        std::vector<std::uint64_t> v(static_cast<std::size_t>(nb));
        stlq_mi355_store_bucket_bytes(h_, v.data(), nb, &nb);
        return v;
    }
    bool Append(std::uint64_t start_id, const std::vector<std::uint32_t>& cluster_id,
                const ColMajorMatrix<Code>& B_small, const ColMajorMatrix<float>& a, int kind, const void* raw,
                int ld, std::string* err) {
        const int n = static_cast<int>(cluster_id.size());
        if (n > 0 && (B_small.cols != n || a.cols != n)) {
            if (err) *err = "BaseBasicWriter::AppendBlock: B/a shape mismatch.";
            return false;
        }
        return Ok(stlq_mi355_store_append(h_, start_id, n, cluster_id.data(), B_small.rows, B_small.data.data(),
                                          a.rows, a.data.data(), kind, raw, ld),
                  err);
    }

    stlq_mi355_store* h_ = nullptr;
    mutable std::vector<std::uint64_t> committed_;
};

}  // namespace io

namespace app {

// The pipeline's BaseBasic checkpoint (include/stlq/pipeline/main_virtual_helpers.h:35-69).
struct BaseBasicCheckpoint {
    static constexpr std::uint32_t kMagic = 0x544b4342u;  // "BCKT"
    std::uint32_t magic = kMagic;
    std::uint32_t version = 1;
    std::uint32_t nbucket = 0;
    std::uint32_t reserved = 0;
    std::uint64_t next_id = 0;
    std::vector<std::uint64_t> bucket_sizes;
};

inline int ComputeNbucketsForBasic(const io::BaseBasicStoreConfig& cfg) {
    const int h0 = cfg.h_vec.empty() ? 0 : cfg.h_vec.front();
    const int bs = std::max(1, cfg.bucket_size);
    return h0 > 0 ? (h0 + bs - 1) / bs : 0;
}

inline std::string BaseBasicCheckpointPath(const std::string& base_basic_dir) {
    return base_basic_dir + "/checkpoint/base_basic/ckpt.bin";
}

inline bool ReadBaseBasicCheckpoint(const std::string& path, BaseBasicCheckpoint* out, std::string* err) {
    std::int64_t nb = 0;
    std::uint64_t next = 0;
    if (stlq_mi355_checkpoint_read(path.c_str(), &next, nullptr, 0, &nb) != STLQ_MI355_OK) {
        if (err) *err = stlq_mi355_last_error();
        return false;
    }
    BaseBasicCheckpoint ck;
    ck.bucket_sizes.resize(static_cast<std::size_t>(nb));
    stlq_mi355_checkpoint_read(path.c_str(), &next, ck.bucket_sizes.data(), nb, &nb);
    ck.nbucket = static_cast<std::uint32_t>(nb);
    ck.next_id = next;
    *out = std::move(ck);
    return true;
}

inline bool WriteBaseBasicCheckpointAtomic(const std::string& path, const BaseBasicCheckpoint& ck, std::string* err) {
    if (stlq_mi355_checkpoint_write(path.c_str(), ck.next_id, ck.bucket_sizes.data(),
                                    static_cast<std::int64_t>(ck.bucket_sizes.size())) == STLQ_MI355_OK)
        return true;
    if (err) *err = stlq_mi355_last_error();
    return false;
}

inline bool TruncateBaseBasicToCheckpoint(const std::string& out_dir, const io::BaseBasicStoreConfig& store_cfg,
                                          const BaseBasicCheckpoint& ck, std::string* err) {
    stlq_mi355_store_config c{};
    c.dir = out_dir.c_str();
    c.d = store_cfg.d;
    c.m = store_cfg.m;
    c.h_vec = store_cfg.h_vec.data();
    c.h_len = static_cast<int>(store_cfg.h_vec.size());
    c.shard_size = store_cfg.shard_size;
    c.bucket_size = store_cfg.bucket_size;
    if (ck.bucket_sizes.size() != ck.nbucket) {
        if (err) *err = "Checkpoint bucket layout mismatch.";
        return false;
    }
    if (stlq_mi355_store_truncate_to_checkpoint(&c, ck.next_id, ck.bucket_sizes.data(),
                                                static_cast<std::int64_t>(ck.bucket_sizes.size())) == STLQ_MI355_OK)
        return true;
    if (err) *err = stlq_mi355_last_error();
    return false;
}

struct BaseBasicCkptCtx {
    std::string path;
    std::uint32_t nbucket = 0;
};

// The commit hook the pipeline installs (main_virtual_helpers.cpp:277-297).
inline bool OnCommitBaseBasicCkpt(std::uint64_t next_id, io::BaseBasicWriter* writer, void* vctx, std::string* err) {
    auto* ctx = static_cast<BaseBasicCkptCtx*>(vctx);
    if (!ctx || !writer) {
        if (err) *err = "OnCommitBaseBasicCkpt: ctx or writer is null.";
        return false;
    }
    BaseBasicCheckpoint ck;
    ck.nbucket = ctx->nbucket;
    ck.next_id = next_id;
    ck.bucket_sizes = writer->bucket_file_bytes();
    if (ck.bucket_sizes.size() != ck.nbucket) {
        if (err) *err = "OnCommitBaseBasicCkpt: bucket sizes length mismatch.";
        return false;
    }
    return WriteBaseBasicCheckpointAtomic(ctx->path, ck, err);
}

}  // namespace app

// Optional hook after each committed output block (include/stlq/quantizer/encode_base_streaming.h:25-28).
template <class Writer>
struct StreamingBasicCommitHookT {
    void* ctx = nullptr;
    bool (*OnCommit)(std::uint64_t next_id, Writer* writer, void* ctx, std::string* err) = nullptr;
};
using StreamingBasicCommitHook = StreamingBasicCommitHookT<io::BaseBasicWriter>;

namespace detail {

template <class Reader, class Writer>
struct StreamUser {
    const Reader* reader;
    Writer* writer;
    const StreamingBasicCommitHookT<Writer>* hook;
    int d, m;
    bool large;
    std::string* err;
    bool keep_raw;
    bool u8;
    double cost_sum = 0.0;
    std::int64_t cost_n = 0;
};

template <class Reader, class Writer, class T>
int StreamFill(void* u, std::int64_t first, std::int64_t count, void* dst) {
    auto* s = static_cast<StreamUser<Reader, Writer>*>(u);
    const std::size_t len = static_cast<std::size_t>(count) * static_cast<std::size_t>(s->d);
    return s->reader->ReadBlockInto(static_cast<std::uint64_t>(first), static_cast<std::uint32_t>(count),
                                    static_cast<T*>(dst), len * sizeof(T), s->err)
               ? 0
               : 1;
}

// One block to the writer (encode_base_streaming.cpp:3112-3135, :4393-4414), then CommitBlock
// (:2054-2059): Flush, then the hook with next id = block end.
template <class Reader, class Writer>
int StreamSink(void* u, std::int64_t first, std::int64_t count, const stlq_mi355_chunk_out* out) {
    auto* s = static_cast<StreamUser<Reader, Writer>*>(u);
    const int m = s->m;
    const std::size_t n = static_cast<std::size_t>(count);
    std::vector<std::uint32_t> cluster_id(n);
    ColMajorMatrix<Code> B_small(std::max(0, m - 1), static_cast<int>(count));
    ColMajorMatrix<float> a(m, static_cast<int>(count));
    if (s->large) {  // the large-root beam's roots and small codes
        std::copy(out->cluster_id, out->cluster_id + n, cluster_id.begin());
        if (m > 1) std::copy(out->B_small, out->B_small + n * (m - 1), B_small.data.begin());
    } else {  // full precomp: layer 0's code is the cluster id (ExtractClusterIdAndCodesSmall)
        for (std::size_t i = 0; i < n; ++i) {
            cluster_id[i] = out->codes[i * m];
            for (int l = 1; l < m; ++l) B_small.data[i * (m - 1) + (l - 1)] = out->codes[i * m + l];
        }
    }
    if (out->a) std::copy(out->a, out->a + n * m, a.data.begin());
    if (out->cost) {
        for (std::size_t i = 0; i < n; ++i) s->cost_sum += out->cost[i] < 0.0f ? 0.0 : out->cost[i];
        s->cost_n += count;
    }
    bool ok;
    if (s->keep_raw && s->u8)
        ok = s->writer->AppendBlockRawU8(static_cast<std::uint64_t>(first), cluster_id, B_small, a,
                                         static_cast<const std::uint8_t*>(out->input), s->d, s->err);
    else if (s->keep_raw)
        ok = s->writer->AppendBlockRawF32(static_cast<std::uint64_t>(first), cluster_id, B_small, a,
                                          static_cast<const float*>(out->input), s->d, s->err);
    else
        ok = s->writer->AppendBlock(static_cast<std::uint64_t>(first), cluster_id, B_small, a, nullptr, s->err);
    if (!ok) return 1;
    if (s->hook && s->hook->OnCommit) {
        if (!s->writer->Flush(s->err)) return 1;
        if (!s->hook->OnCommit(static_cast<std::uint64_t>(first + count), s->writer, s->hook->ctx, s->err)) return 1;
    }
    return 0;
}

template <class T, class Reader, class Writer>
bool EncodeStreaming(const Config& cfg, const Reader& base_reader, const ColMajorMatrix<float>& R,
                     const Precomp& pre_full, const PrecompLargeRoot* pre_large, Writer* writer, float* out_beam_mse,
                     float* out_final_mse, std::string* err, std::uint64_t start_id,
                     const StreamingBasicCommitHookT<Writer>* commit_hook) {
    if (!writer) {
        if (err) *err = "EncodeBaseStreaming: writer is null.";
        return false;
    }
    const std::uint64_t nbase = base_reader.n();
    if (start_id > nbase) {
        if (err) *err = "EncodeBaseStreaming: start_id out of range.";
        return false;
    }
    const int d = base_reader.d();
    if (d <= 0 || nbase == 0) {
        if (err) *err = "EncodeBaseStreaming: empty base reader.";
        return false;
    }
    const std::uint64_t block = static_cast<std::uint64_t>(std::max(1, cfg.large.base_block));
    if (commit_hook && commit_hook->OnCommit && start_id % block != 0) {
        if (err) *err = "EncodeBaseStreaming: start_id must be a multiple of large.base_block when using checkpointing.";
        return false;
    }
    if (start_id == nbase) return true;
    const BaseEncodeConfig& e = cfg.base.encode;
    stlq_mi355_stream_params sp{};
    sp.encode = stlq_mi355_encode_params{std::max(1, e.H_beam), e.icm_iters, e.ils_iters, e.perturb_k,
                                          e.use_abs ? 1 : 0, static_cast<std::uint32_t>(e.seed), 1};
    sp.input_u8 = sizeof(T) == 1 ? 1 : 0;
    sp.large_root = pre_large ? 1 : 0;
    sp.root_mode = 1;
    sp.R = (R.rows == d && R.cols == d) ? R.data.data() : nullptr;
    sp.start_id = start_id;
    StreamUser<Reader, Writer> u{&base_reader, writer, commit_hook, d, pre_large ? pre_large->m : pre_full.m,
                                 pre_large != nullptr, err, cfg.large.write_vector_bucket, sizeof(T) == 1};
    stlq_mi355_ctx* ctx = pre_large ? BindLargeRoot(*pre_large) : Bind(pre_full);
    stlq_mi355_stream_stats st{};
    const int rc = stlq_mi355_encode_stream(ctx, static_cast<std::int64_t>(nbase - start_id),
                                            static_cast<std::int64_t>(block), &sp, &StreamFill<Reader, Writer, T>,
                                            &StreamSink<Reader, Writer>, &u, &st);
    if (rc != STLQ_MI355_OK) {
        if (err && err->empty()) *err = stlq_mi355_last_error();
        return false;
    }
    const float mse = u.cost_n > 0 ? static_cast<float>(u.cost_sum / static_cast<double>(u.cost_n)) : 0.0f;
    if (out_final_mse) *out_final_mse = mse;
    if (out_beam_mse) *out_beam_mse = mse;
    return true;
}

}  // namespace detail

// EncodeBaseStreaming (include/stlq/quantizer/encode_base_streaming.h:32-44,
// src/quantizer/encode_base_streaming.cpp:1913-2060 and :3060-3212): encodes the reader's uint8
// vectors start_id..n()-1 in blocks of config.large.base_block, double-buffered on the device
// (uint8 widened there), and appends each block's cluster ids, small codes and LS coefficients to
// the writer in order, then calls the commit hook (after writer->Flush).
// Reader is io::BvecsReader-like (d(), n(), ReadBlockInto(start, count, uint8_t* dst, bytes, err));
// Writer is io::BaseBasicWriter (or one with its AppendBlock/AppendBlockRawU8/Flush): with
// config.large.write_vector_bucket the raw uint8 tile goes into the bucket records (:3114-3124),
// else AppendBlock(..., nullptr, ...). pre_large selects the large-root beam with the nearest root
// forced and its refit (:1005-1210); otherwise the full precomp is used and layer 0's code is the
// cluster id. The rotation R (d x d) is applied on the device (empty R: none). out_final_mse
// receives the mean cost; out_beam_mse the same (the streamed refit is final).
template <class Reader, class Writer>
bool EncodeBaseStreaming(const Config& cfg, const Reader& base_reader, const ColMajorMatrix<float>& R,
                         const CodebookPack& C_root, const Precomp& pre_full, const PrecompLargeRoot* pre_large,
                         StreamKernelProvider* kernels, Writer* writer, float* out_beam_mse, float* out_final_mse,
                         std::string* err, std::uint64_t start_id = 0,
                         const StreamingBasicCommitHookT<Writer>* commit_hook = nullptr) {
    (void)C_root;
    (void)kernels;
    return detail::EncodeStreaming<std::uint8_t>(cfg, base_reader, R, pre_full, pre_large, writer, out_beam_mse,
                                                 out_final_mse, err, start_id, commit_hook);
}

// EncodeBaseStreamingF32 (include/stlq/quantizer/encode_base_streaming.h:46-58,
// src/quantizer/encode_base_streaming.cpp:3285-3420, :4544-4579): as EncodeBaseStreaming for float
// vectors. Reader is io::FvecsReader-like (ReadBlockInto(start, count, float* dst, bytes, err));
// with write_vector_bucket the raw (unrotated) float tile goes into the bucket records through
// AppendBlockRawF32 (:4396-4404).
template <class Reader, class Writer>
bool EncodeBaseStreamingF32(const Config& cfg, const Reader& base_reader, const ColMajorMatrix<float>& R,
                            const CodebookPack& C_root, const Precomp& pre_full, const PrecompLargeRoot* pre_large,
                            StreamKernelProvider* kernels, Writer* writer, float* out_beam_mse, float* out_final_mse,
                            std::string* err, std::uint64_t start_id = 0,
                            const StreamingBasicCommitHookT<Writer>* commit_hook = nullptr) {
    (void)C_root;
    (void)kernels;
    return detail::EncodeStreaming<float>(cfg, base_reader, R, pre_full, pre_large, writer, out_beam_mse,
                                          out_final_mse, err, start_id, commit_hook);
}

}  // namespace stlq
}  // namespace stlq_mi355
