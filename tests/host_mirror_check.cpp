// Test driver for the C++ host mirror (stlq_amd/host/stlq_mi355.hpp): runs the reference-named
// functions on caller-supplied arrays and exports the results through a C ABI so that pytest
// can compare them with the oracle. Built by stlq_amd/build.py next to libstlq_mi355.so.
#include <cstdint>
#include <cstring>
#include <exception>
#include <string>
#include <vector>

#include "../stlq_amd/host/stlq_mi355.hpp"

namespace s = stlq_mi355::stlq;

namespace {

void PutError(const std::string& msg, char* err, int errlen) {
    if (!err || errlen <= 0) return;
    std::strncpy(err, msg.c_str(), static_cast<std::size_t>(errlen - 1));
    err[errlen - 1] = '\0';
}

s::CodebookPack MakePack(int d, int m, const int* h_vec, const float* C_all) {
    s::CodebookPack pack;
    pack.d = d;
    std::size_t off = 0;
    for (int l = 0; l < m; ++l) {
        s::ColMajorMatrix<float> b(d, h_vec[l]);
        std::memcpy(b.data.data(), C_all + off, b.data.size() * sizeof(float));
        off += b.data.size();
        pack.h_vec.push_back(h_vec[l]);
        pack.books.push_back(std::move(b));
    }
    return pack;
}

}  // namespace

extern "C" {

// BuildPrecomp -> ComputeXc -> BeamSearchPrefixLS -> ComputeXNorm2 -> DynamicIcmWithIls*NoNormal,
// then EncodeBase on the same inputs, which must reproduce the staged result exactly (return 3
// otherwise). C_all: d x H column-major (layer after layer); X: d x n column-major.
// Outputs: G (H x H), codes_beam and codes_final (m x n), a (m x n), cost (n), mse[2].
int mirror_encode(int d, int m, const int* h_vec, const float* C_all, const float* X, int n, int H_beam,
                  int icm_iters, int use_abs, uint32_t seed, float* G, uint8_t* codes_beam,
                  uint8_t* codes_final, float* a, float* cost, float* mse, char* err, int errlen) {
    try {
        const s::CodebookPack pack = MakePack(d, m, h_vec, C_all);
        s::Precomp pre;
        if (!s::BuildPrecomp(pack, &pre)) {
            PutError("BuildPrecomp failed", err, errlen);
            return 1;
        }
        std::memcpy(G, pre.G.data.data(), pre.G.data.size() * sizeof(float));
        s::ColMajorMatrix<float> Xm(d, n);
        std::memcpy(Xm.data.data(), X, Xm.data.size() * sizeof(float));
        s::ColMajorMatrix<float> xC;
        s::ComputeXc(pre, Xm, &xC);
        s::ColMajorMatrix<s::FullCode> B;
        s::BeamSearchPrefixLS(Xm, pre, xC, H_beam, &B);
        std::memcpy(codes_beam, B.data.data(), B.data.size());
        std::vector<float> xn2;
        s::ComputeXNorm2(Xm, &xn2);
        s::ColMajorMatrix<float> am;
        std::vector<float> cst;
        if (use_abs)
            s::DynamicIcmWithIlsAbsNoNormal(Xm, pre, xC, icm_iters, 0, 3, seed, &B, &am, &xn2, &cst);
        else
            s::DynamicIcmWithIlsNoAbsNoNormal(Xm, pre, xC, icm_iters, 0, 3, seed, &B, &am, &xn2, &cst);
        std::memcpy(codes_final, B.data.data(), B.data.size());
        std::memcpy(a, am.data.data(), am.data.size() * sizeof(float));
        std::memcpy(cost, cst.data(), cst.size() * sizeof(float));

        s::EncodeOptions opt;
        opt.use_abs = use_abs != 0;
        opt.H_beam = H_beam;
        opt.icm_iters = icm_iters;
        opt.seed = static_cast<int>(seed);
        s::BaseEncoding base;
        std::string e;
        if (!s::EncodeBase(opt, Xm, pack, pre, &base, &mse[0], &mse[1], &e)) {
            PutError("EncodeBase: " + e, err, errlen);
            return 2;
        }
        if (base.B.data != B.data || std::memcmp(base.a.data.data(), am.data.data(), am.data.size() * 4) != 0) {
            PutError("EncodeBase differs from the staged pipeline", err, errlen);
            return 3;
        }
        return 0;
    } catch (const std::exception& ex) {
        PutError(ex.what(), err, errlen);
        return 4;
    }
}

// BuildPrecompLargeRoot -> BeamSearchPrefixLSLargeRoot (xC_small computed on the device).
// C0: d x h_vec[0]; C_small: d x sum(h_vec[1..m-1]); outputs cluster_id (n), B_small ((m-1) x n).
// BuildPrecompLargeRoot + BeamSearchPrefixLSLargeRoot, then (when a is not NULL)
// DynamicIcmWithIlsAbsNoNormalLargeRoot with the given ICM/ILS settings, as the streaming
// encode's large-root branch calls them.
int mirror_large_root(int d, int m, const int* h_vec, const float* C0, const float* C_small, const float* X, int n,
                      int H_beam, int icm_iters, int ils_iters, uint32_t* cluster_id, uint8_t* B_small, float* a,
                      float* cost, char* err, int errlen) {
    try {
        s::CodebookPack pack;
        pack.d = d;
        s::ColMajorMatrix<float> root(d, h_vec[0]);
        std::memcpy(root.data.data(), C0, root.data.size() * sizeof(float));
        pack.books.push_back(std::move(root));
        pack.h_vec.push_back(h_vec[0]);
        std::size_t off = 0;
        for (int l = 1; l < m; ++l) {
            s::ColMajorMatrix<float> b(d, h_vec[l]);
            std::memcpy(b.data.data(), C_small + off, b.data.size() * sizeof(float));
            off += b.data.size();
            pack.books.push_back(std::move(b));
            pack.h_vec.push_back(h_vec[l]);
        }
        s::PrecompLargeRoot pre;
        std::string e;
        if (!s::BuildPrecompLargeRoot(pack, nullptr, s::PrecompLargeRootBuildOptions{}, &pre, &e)) {
            PutError("BuildPrecompLargeRoot: " + e, err, errlen);
            return 1;
        }
        s::ColMajorMatrix<float> Xm(d, n);
        std::memcpy(Xm.data.data(), X, Xm.data.size() * sizeof(float));
        std::vector<std::uint32_t> cid;
        s::ColMajorMatrix<s::Code> Bs;
        s::BeamSearchLargeRootTiming timing;
        s::BeamSearchPrefixLSLargeRoot(Xm, pre, s::ColMajorMatrix<float>(), H_beam, &cid, &Bs, &timing);
        if (a) {
            s::ColMajorMatrix<float> am;
            std::vector<float> xn2, cst;
            s::DynamicIcmWithIlsAbsNoNormalLargeRoot(Xm, pre, s::ColMajorMatrix<float>(), icm_iters, ils_iters, 3,
                                                    38251450u, cid, &Bs, &am, &xn2, &cst, false, 0);
            std::memcpy(a, am.data.data(), am.data.size() * sizeof(float));
            std::memcpy(cost, cst.data(), cst.size() * sizeof(float));
        }
        std::memcpy(cluster_id, cid.data(), cid.size() * sizeof(std::uint32_t));
        std::memcpy(B_small, Bs.data.data(), Bs.data.size());
        return 0;
    } catch (const std::exception& ex) {
        PutError(ex.what(), err, errlen);
        return 4;
    }
}

}  // extern "C"
