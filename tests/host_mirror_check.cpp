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

// FvecsReader-like view of a caller array (d x n column-major).
struct MemReader {
    int d_;
    std::uint64_t n_;
    const float* x;
    int d() const { return d_; }
    std::uint64_t n() const { return n_; }
    bool ReadBlockInto(std::uint64_t start, std::uint32_t count, float* dst, std::size_t bytes, std::string* err) const {
        const std::size_t want = static_cast<std::size_t>(count) * static_cast<std::size_t>(d_) * sizeof(float);
        if (start + count > n_ || bytes < want) {
            if (err) *err = "MemReader: block out of range";
            return false;
        }
        std::memcpy(dst, x + start * static_cast<std::uint64_t>(d_), want);
        return true;
    }
};

// BaseBasicWriter-like recorder: places each block's records at their global ids and checks that
// blocks arrive in order.
struct MemWriter {
    int d, m;
    std::uint64_t next = 0;
    int blocks = 0;
    std::uint32_t* cluster_id;
    std::uint8_t* B_small;
    float* a;
    float* raw;  // may be null
    bool Put(std::uint64_t start, const std::vector<std::uint32_t>& cid, const s::ColMajorMatrix<s::Code>& Bs,
             const s::ColMajorMatrix<float>& am, const float* x, int ld, std::string* err) {
        if (start != next || Bs.cols != static_cast<int>(cid.size()) || am.cols != Bs.cols || am.rows != m ||
            Bs.rows != m - 1) {
            if (err) *err = "MemWriter: block out of order or misshapen";
            return false;
        }
        const std::size_t n = cid.size();
        std::memcpy(cluster_id + start, cid.data(), n * sizeof(std::uint32_t));
        std::memcpy(B_small + start * (m - 1), Bs.data.data(), Bs.data.size());
        std::memcpy(a + start * m, am.data.data(), am.data.size() * sizeof(float));
        if (x && raw)
            for (std::size_t i = 0; i < n; ++i)
                std::memcpy(raw + (start + i) * d, x + i * static_cast<std::size_t>(ld), sizeof(float) * d);
        next = start + n;
        ++blocks;
        return true;
    }
    bool AppendBlock(std::uint64_t start, const std::vector<std::uint32_t>& cid, const s::ColMajorMatrix<s::Code>& Bs,
                     const s::ColMajorMatrix<float>& am, const s::ColMajorMatrix<std::uint8_t>*, std::string* err) {
        return Put(start, cid, Bs, am, nullptr, 0, err);
    }
    bool AppendBlockRawF32(std::uint64_t start, const std::vector<std::uint32_t>& cid,
                           const s::ColMajorMatrix<s::Code>& Bs, const s::ColMajorMatrix<float>& am, const float* x,
                           int ld, std::string* err) {
        if (!x) {
            if (err) *err = "MemWriter: raw tile missing";
            return false;
        }
        return Put(start, cid, Bs, am, x, ld, err);
    }
    bool AppendBlockRawU8(std::uint64_t, const std::vector<std::uint32_t>&, const s::ColMajorMatrix<s::Code>&,
                          const s::ColMajorMatrix<float>&, const std::uint8_t*, int, std::string* err) {
        if (err) *err = "MemWriter: float stream gave a uint8 tile";
        return false;
    }
    bool Flush(std::string*) { return true; }
};

// BvecsReader-like (uint8) view of a caller array (d x n column-major).
struct MemReaderU8 {
    int d_;
    std::uint64_t n_;
    const std::uint8_t* x;
    int d() const { return d_; }
    std::uint64_t n() const { return n_; }
    bool ReadBlockInto(std::uint64_t start, std::uint32_t count, std::uint8_t* dst, std::size_t bytes,
                       std::string* err) const {
        const std::size_t want = static_cast<std::size_t>(count) * static_cast<std::size_t>(d_);
        if (start + count > n_ || bytes < want) {
            if (err) *err = "MemReaderU8: block out of range";
            return false;
        }
        std::memcpy(dst, x + start * static_cast<std::uint64_t>(d_), want);
        return true;
    }
};

struct HookLog {
    std::uint64_t last = 0;
    int calls = 0;
    bool ordered = true;
};

bool OnCommit(std::uint64_t next_id, MemWriter* w, void* ctx, std::string*) {
    auto* h = static_cast<HookLog*>(ctx);
    h->ordered = h->ordered && next_id == w->next && next_id > h->last;
    h->last = next_id;
    ++h->calls;
    return true;
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

        s::Config cfg;  // the reference-signature EncodeBase (encoder.h:66-74)
        cfg.base.encode.use_abs = use_abs != 0;
        cfg.base.encode.H_beam = H_beam;
        cfg.base.encode.icm_iters = icm_iters;
        cfg.base.encode.seed = static_cast<int>(seed);
        s::Dataset ds;
        ds.Xb = Xm;
        s::BaseEncoding base;
        std::string e;
        if (!s::EncodeBase(cfg, ds, pack, pre, nullptr, &base, &mse[0], &mse[1], &e)) {
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

// EncodeBaseStreamingF32 over an in-memory reader and a recording writer. large != 0: C_all holds
// the root layer then the small layers and the large-root beam runs; else the full precomp. The
// writer's arrays are indexed by global id (entries below start_id stay untouched); raw (d x n) gets
// the raw tiles when write_raw. hook_calls (out) counts the commit hook's calls (-1: out of order).
// Return 0 on success, 1 when the call returned false (err holds its message), 4 on an exception.
int mirror_stream(int d, int m, const int* h_vec, const float* C_all, const float* X, int n, int large, int H_beam,
                  int icm_iters, int ils_iters, int base_block, uint64_t start_id, int write_raw, int use_hook,
                  uint32_t* cluster_id, uint8_t* B_small, float* a, float* raw, float* mse, int* hook_calls,
                  char* err, int errlen) {
    try {
        s::Config cfg;
        cfg.base.encode.H_beam = H_beam;
        cfg.base.encode.icm_iters = icm_iters;
        cfg.base.encode.ils_iters = ils_iters;
        cfg.large.base_block = base_block;
        cfg.large.write_vector_bucket = write_raw != 0;
        const s::CodebookPack pack = MakePack(d, m, h_vec, C_all);
        s::Precomp pre_full;
        s::PrecompLargeRoot pre_large;
        std::string e;
        if (d > 0 && m > 0) {
            if (large) {
                if (!s::BuildPrecompLargeRoot(pack, nullptr, s::PrecompLargeRootBuildOptions{}, &pre_large, &e)) {
                    PutError("BuildPrecompLargeRoot: " + e, err, errlen);
                    return 4;
                }
            } else if (!s::BuildPrecomp(pack, &pre_full)) {
                PutError("BuildPrecomp failed", err, errlen);
                return 4;
            }
        }
        const MemReader reader{d, static_cast<std::uint64_t>(n), X};
        MemWriter writer{d, m, start_id, 0, cluster_id, B_small, a, raw};
        HookLog log;
        s::StreamingBasicCommitHookT<MemWriter> hook;
        hook.ctx = &log;
        hook.OnCommit = &OnCommit;
        const bool ok = s::EncodeBaseStreamingF32(cfg, reader, s::ColMajorMatrix<float>(), pack, pre_full,
                                                  large ? &pre_large : nullptr, nullptr, &writer, &mse[0], &mse[1],
                                                  &e, start_id, use_hook ? &hook : nullptr);
        *hook_calls = log.ordered ? log.calls : -1;
        if (!ok) {
            PutError(e, err, errlen);
            return 1;
        }
        if (writer.next != static_cast<std::uint64_t>(n)) {
            PutError("stream ended before the last id", err, errlen);
            return 4;
        }
        return 0;
    } catch (const std::exception& ex) {
        PutError(ex.what(), err, errlen);
        return 4;
    }
}


// EncodeBaseStreaming (u8 != 0, uint8 X) or EncodeBaseStreamingF32 (float X) writing a real
// BaseBasicStore at dir through io::BaseBasicWriter, with the pipeline's checkpoint hook
// (app::OnCommitBaseBasicCkpt at app::BaseBasicCheckpointPath(dir)) when use_ckpt. resume != 0
// continues the store the way the pipeline does (stlq_large_base_stages.cpp:321-390): read the
// checkpoint, cut the store back to it, OpenResume at its next id and stream from there. stop_at > 0
// stops the stream at that id (a run cut short). Store layout: shard_size, bucket_size, flush_mb
// and write_raw (vector buckets). Return 0 on success, 1 when a call returned false, 4 on an exception.
int mirror_stream_store(const char* dir, int d, int m, const int* h_vec, const float* C_all, const void* X, int u8,
                        int n, int large, int H_beam, int icm_iters, int ils_iters, int base_block, int shard_size,
                        int bucket_size, int flush_mb, int write_raw, int use_ckpt, int resume, int stop_at,
                        char* err, int errlen) {
    try {
        s::Config cfg;
        cfg.base.encode.H_beam = H_beam;
        cfg.base.encode.icm_iters = icm_iters;
        cfg.base.encode.ils_iters = ils_iters;
        cfg.large.base_block = base_block;
        cfg.large.write_vector_bucket = write_raw != 0;
        const s::CodebookPack pack = MakePack(d, m, h_vec, C_all);
        s::Precomp pre_full;
        s::PrecompLargeRoot pre_large;
        std::string e;
        if (large) {
            if (!s::BuildPrecompLargeRoot(pack, nullptr, s::PrecompLargeRootBuildOptions{}, &pre_large, &e)) {
                PutError("BuildPrecompLargeRoot: " + e, err, errlen);
                return 4;
            }
        } else if (!s::BuildPrecomp(pack, &pre_full)) {
            PutError("BuildPrecomp failed", err, errlen);
            return 4;
        }
        s::io::BaseBasicStoreConfig sc;
        sc.dir = dir;
        sc.d = d;
        sc.m = m;
        sc.h_vec.assign(h_vec, h_vec + m);
        sc.shard_size = shard_size;
        sc.bucket_size = bucket_size;
        sc.bucket_flush_mb = flush_mb;
        sc.write_vector_bucket = write_raw != 0;
        sc.raw_bytes_per_vec = write_raw ? (u8 ? d : d * static_cast<int>(sizeof(float))) : 0;
        const std::string ckpt = s::app::BaseBasicCheckpointPath(dir);
        s::io::BaseBasicWriter writer;
        std::uint64_t start_id = 0;
        bool ok = true;
        if (resume) {
            s::app::BaseBasicCheckpoint ck;
            ok = s::app::ReadBaseBasicCheckpoint(ckpt, &ck, &e) && s::app::TruncateBaseBasicToCheckpoint(dir, sc, ck, &e) &&
                 writer.OpenResume(sc, ck.next_id, ck.bucket_sizes, &e);
            start_id = ck.next_id;
        } else {
            ok = writer.Open(sc, &e);
            if (ok && use_ckpt) {
                s::app::BaseBasicCheckpoint init;
                init.nbucket = static_cast<std::uint32_t>(s::app::ComputeNbucketsForBasic(sc));
                init.bucket_sizes.assign(init.nbucket, 0);
                ok = s::app::WriteBaseBasicCheckpointAtomic(ckpt, init, &e);
            }
        }
        if (!ok) {
            PutError(e, err, errlen);
            return 1;
        }
        s::app::BaseBasicCkptCtx hook_ctx;
        hook_ctx.path = ckpt;
        hook_ctx.nbucket = static_cast<std::uint32_t>(s::app::ComputeNbucketsForBasic(sc));
        s::StreamingBasicCommitHook hook;
        hook.ctx = &hook_ctx;
        hook.OnCommit = &s::app::OnCommitBaseBasicCkpt;
        const std::uint64_t end = stop_at > 0 ? static_cast<std::uint64_t>(stop_at) : static_cast<std::uint64_t>(n);
        float mse[2];
        if (u8) {
            const MemReaderU8 reader{d, end, static_cast<const std::uint8_t*>(X)};
            ok = s::EncodeBaseStreaming(cfg, reader, s::ColMajorMatrix<float>(), pack, pre_full,
                                        large ? &pre_large : nullptr, nullptr, &writer, &mse[0], &mse[1], &e, start_id,
                                        use_ckpt ? &hook : nullptr);
        } else {
            const MemReader reader{d, end, static_cast<const float*>(X)};
            ok = s::EncodeBaseStreamingF32(cfg, reader, s::ColMajorMatrix<float>(), pack, pre_full,
                                           large ? &pre_large : nullptr, nullptr, &writer, &mse[0], &mse[1], &e,
                                           start_id, use_ckpt ? &hook : nullptr);
        }
        ok = ok && writer.Close(&e);
        if (!ok) {
            PutError(e, err, errlen);
            return 1;
        }
        return 0;
    } catch (const std::exception& ex) {
        PutError(ex.what(), err, errlen);
        return 4;
    }
}

}  // extern "C"
