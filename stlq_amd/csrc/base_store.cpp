// BaseBasicStore output of the streaming base encode (host code of libstlq_mi355).
//
// Writes the files of the reference's io::BaseBasicWriter (src/io/base_store.cpp) and its
// checkpoint helpers (src/pipeline/main_virtual_helpers.cpp:100-297) byte for byte: the file
// names, the meta formats, the record layout, the order of bytes in every file and the
// committed-byte accounting are the reference's. Files are plain stdio streams; each bucket keeps
// its records in a memory buffer that is written out when it reaches bucket_flush_mb, on Flush
// and on Close (only the on-disk bytes count as committed).
#include "stlq_mi355_store.h"

#include "errors.hpp"

#include <algorithm>
#include <cstdio>
#include <cstring>
#include <filesystem>
#include <memory>
#include <string>
#include <system_error>
#include <vector>

namespace {

namespace fs = std::filesystem;
using stlq_mi355::SetLastError;

int Invalid(const std::string& msg) { return SetLastError(STLQ_MI355_ERR_INVALID, msg); }

// Zero-padded 4-digit tag of shard and bucket file names (wider numbers keep every digit).
std::string Tag4(int v) {
    char buf[24];
    std::snprintf(buf, sizeof(buf), "%04d", v);
    return buf;
}

std::string Under(const std::string& dir, const std::string& name) {
    if (dir.empty()) return name;
    const char last = dir.back();
    return (last == '/' || last == '\\') ? dir + name : dir + "/" + name;
}

// One output file. `good` turns false on the first failed open, write or flush.
class OutFile {
public:
    OutFile() = default;
    OutFile(const OutFile&) = delete;
    OutFile& operator=(const OutFile&) = delete;
    ~OutFile() { Close(); }

    bool Open(const std::string& path, bool append) {
        Close();
        f_ = std::fopen(path.c_str(), append ? "ab" : "wb");
        good_ = f_ != nullptr;
        return good_;
    }
    bool IsOpen() const { return f_ != nullptr; }
    bool Write(const void* p, size_t bytes) {
        if (!f_) return good_ = false;
        if (bytes && std::fwrite(p, 1, bytes, f_) != bytes) good_ = false;
        return good_;
    }
    bool Flush() {
        if (f_ && std::fflush(f_) != 0) good_ = false;
        return good_;
    }
    void Close() {
        if (f_) {
            if (std::fclose(f_) != 0) good_ = false;
            f_ = nullptr;
        }
    }

private:
    std::FILE* f_ = nullptr;
    bool good_ = true;
};

struct Params {
    std::string dir;
    int d = 0, m = 0;
    std::vector<int> h_vec;
    int shard_size = 0, bucket_size = 0, bucket_flush_mb = 0;
    bool vector_bucket = false, basic_bucket = false;
    int raw_bytes = 0;
};

int ReadConfig(const stlq_mi355_store_config* cfg, Params* p, const char* who) {
    if (!cfg) return Invalid(std::string(who) + ": config is null");
    if (cfg->h_len < 0 || (cfg->h_len > 0 && !cfg->h_vec)) return Invalid(std::string(who) + ": bad h_vec");
    p->dir = cfg->dir ? cfg->dir : "";
    p->d = cfg->d;
    p->m = cfg->m;
    p->h_vec.assign(cfg->h_vec, cfg->h_vec + cfg->h_len);
    p->shard_size = cfg->shard_size;
    p->bucket_size = cfg->bucket_size;
    p->bucket_flush_mb = cfg->bucket_flush_mb;
    p->vector_bucket = cfg->write_vector_bucket != 0;
    p->basic_bucket = cfg->write_basic_to_bucket != 0;
    p->raw_bytes = cfg->raw_bytes_per_vec;
    if (p->dir.empty() || p->d <= 0 || p->m <= 0) return Invalid(std::string(who) + ": invalid config");
    // Raw bytes per record: d (uint8) unless set; none without vector buckets (base_store.cpp:101-107).
    p->raw_bytes = p->vector_bucket ? (p->raw_bytes <= 0 ? p->d : p->raw_bytes) : 0;
    return STLQ_MI355_OK;
}

// Buckets of a layout: ceil(h0 / bucket_size) for the root codebook size h0.
int64_t BucketCount(const std::vector<int>& h_vec, int bucket_size) {
    const int64_t h0 = h_vec.empty() ? 0 : h_vec.front();
    const int64_t bs = std::max(1, bucket_size);
    return h0 > 0 ? (h0 + bs - 1) / bs : 0;
}

bool MakeDirs(const std::string& dir) {
    std::error_code ec;
    fs::create_directories(dir, ec);
    return !ec;
}

// meta.json as the reference writes it (base_store.cpp:134-156).
bool WriteMetaJson(const Params& p, int bucket_size_as_given) {
    OutFile f;
    if (!f.Open(Under(p.dir, "meta.json"), false)) return false;
    std::string s = "{\n";
    s += "  \"d\": " + std::to_string(p.d) + ",\n";
    s += "  \"m\": " + std::to_string(p.m) + ",\n";
    s += "  \"m_codes\": " + std::to_string(std::max(0, p.m - 1)) + ",\n";
    s += "  \"shard_size\": " + std::to_string(p.shard_size) + ",\n";
    s += "  \"bucket_size\": " + std::to_string(bucket_size_as_given) + ",\n";
    s += std::string("  \"write_vector_bucket\": ") + (p.vector_bucket ? "true" : "false") + ",\n";
    s += std::string("  \"write_basic_to_bucket\": ") + (p.basic_bucket ? "true" : "false") + ",\n";
    s += "  \"raw_bytes_per_vec\": " + std::to_string(p.raw_bytes) + ",\n";
    s += "  \"h_vec\": [";
    for (size_t i = 0; i < p.h_vec.size(); ++i) s += (i ? ", " : "") + std::to_string(p.h_vec[i]);
    s += "]\n}\n";
    f.Write(s.data(), s.size());
    f.Close();
    return true;  // the reference does not check this stream after opening it
}

// meta.bin (base_store.cpp:39-84): ten little-endian 32-bit fields, then h_vec.
bool WriteMetaBin(const Params& p, int bucket_size_as_given) {
    const uint32_t flags = (p.vector_bucket ? 1u : 0u) | (p.basic_bucket ? 2u : 0u);
    const int32_t raw = p.vector_bucket ? (p.raw_bytes > 0 ? p.raw_bytes : p.d) : 0;
    const uint32_t head[10] = {0x53414243u /* "CBAS" */, 2u,
                               static_cast<uint32_t>(p.d), static_cast<uint32_t>(p.m),
                               static_cast<uint32_t>(std::max(0, p.m - 1)), static_cast<uint32_t>(p.shard_size),
                               static_cast<uint32_t>(bucket_size_as_given), flags,
                               static_cast<uint32_t>(p.h_vec.size()), static_cast<uint32_t>(raw)};
    OutFile f;
    if (!f.Open(Under(p.dir, "meta.bin"), false)) return false;
    f.Write(head, sizeof(head));
    if (!p.h_vec.empty()) f.Write(p.h_vec.data(), p.h_vec.size() * sizeof(int));
    const bool ok = f.Flush();
    f.Close();
    return ok;
}

bool ResizeFile(const std::string& path, uint64_t bytes) {
    {
        OutFile touch;  // create when missing, keep the contents otherwise
        if (!touch.Open(path, true)) return false;
    }
    std::error_code ec;
    fs::resize_file(path, bytes, ec);
    return !ec;
}

}  // namespace

struct stlq_mi355_store {
    struct Bucket {
        bool open = false;
        OutFile file;
        std::vector<uint8_t> pending;  // records not yet written to the file
    };

    Params p;
    size_t flush_bytes = 0;
    OutFile cluster_ids;
    int shard = -1;
    OutFile codes, coeffs;
    bool resume = false;
    uint64_t resume_id = 0;
    int resume_shard = 0;
    int64_t resume_in_shard = 0;
    std::vector<std::unique_ptr<Bucket>> buckets;  // grows past the layout for out-of-range ids
    std::vector<uint64_t> committed;               // on-disk bytes, one per bucket of the layout

    void SizeBuckets(int64_t n) {
        buckets.clear();
        for (int64_t b = 0; b < n; ++b) buckets.push_back(std::make_unique<Bucket>());
    }

    // The shard files of global id `gid` (base_store.cpp:332-372).
    int SelectShard(uint64_t gid) {
        const uint64_t ss = static_cast<uint64_t>(std::max(1, p.shard_size));
        const int s = static_cast<int>(gid / ss);
        if (s == shard) return STLQ_MI355_OK;
        if (resume && gid < resume_id) return Invalid("BaseBasicWriter: global id before the resume point");
        shard = s;
        codes.Close();
        coeffs.Close();
        const bool append = resume && s == resume_shard && resume_in_shard > 0;
        const std::string tag = Tag4(s);
        const bool ok_codes = codes.Open(Under(p.dir, "codes_shard_" + tag + ".bin"), append);
        const bool ok_coeffs = coeffs.Open(Under(p.dir, "coeffs_shard_" + tag + ".bin"), append);
        if (!ok_codes || !ok_coeffs) return Invalid("BaseBasicWriter: cannot open the shard files of shard " + tag);
        return STLQ_MI355_OK;
    }

    int OpenBucket(int b) {
        if (b < 0) return Invalid("BaseBasicWriter: invalid bucket id");
        while (static_cast<int64_t>(buckets.size()) <= b) buckets.push_back(std::make_unique<Bucket>());
        Bucket& bk = *buckets[static_cast<size_t>(b)];
        if (bk.open) return STLQ_MI355_OK;
        const std::string path = Under(p.dir, "bucket_" + Tag4(b) + ".bin");
        if (!bk.file.Open(path, resume)) return Invalid("BaseBasicWriter: cannot open bucket file " + path);
        bk.open = true;
        bk.pending.clear();
        return STLQ_MI355_OK;
    }

    int WriteOut(size_t b) {
        if (b >= buckets.size()) return STLQ_MI355_OK;
        Bucket& bk = *buckets[b];
        if (!bk.open || bk.pending.empty()) return STLQ_MI355_OK;
        if (!bk.file.Write(bk.pending.data(), bk.pending.size()))
            return Invalid("BaseBasicWriter: bucket write failed");
        if (b < committed.size()) committed[b] += bk.pending.size();
        bk.pending.clear();
        return STLQ_MI355_OK;
    }
};

extern "C" {

void stlq_mi355_store_config_init(stlq_mi355_store_config* cfg) {
    if (!cfg) return;
    cfg->shard_size = 2000000;
    cfg->bucket_size = 256;
    cfg->bucket_flush_mb = 256;
    cfg->write_vector_bucket = 1;
    cfg->write_basic_to_bucket = 1;
    cfg->raw_bytes_per_vec = 0;
}

int stlq_mi355_store_open(const stlq_mi355_store_config* cfg, stlq_mi355_store** out) {
    if (!out) return Invalid("store_open: out is null");
    *out = nullptr;
    auto st = std::make_unique<stlq_mi355_store>();
    if (int rc = ReadConfig(cfg, &st->p, "BaseBasicWriter::Open")) return rc;
    Params& p = st->p;
    st->flush_bytes = static_cast<size_t>(std::max(1, p.bucket_flush_mb)) << 20;
    if (!MakeDirs(p.dir)) return Invalid("BaseBasicWriter: failed to create dir: " + p.dir);
    // Empty every bucket file of the layout so no earlier run's records survive (:117-132).
    const int64_t nb = BucketCount(p.h_vec, p.bucket_size);
    st->SizeBuckets(nb);
    st->committed.assign(static_cast<size_t>(nb), 0);
    for (int64_t b = 0; b < nb; ++b) {
        OutFile f;
        f.Open(Under(p.dir, "bucket_" + Tag4(static_cast<int>(b)) + ".bin"), false);
    }
    if (!WriteMetaJson(p, p.bucket_size)) return Invalid("BaseBasicWriter::Open: failed to open meta.json");
    if (!WriteMetaBin(p, p.bucket_size)) return Invalid("BaseBasicWriter: failed to write meta.bin");
    if (!st->cluster_ids.Open(Under(p.dir, "cluster_id.u32"), false))
        return Invalid("BaseBasicWriter::Open: failed to open cluster_id.u32");
    if (p.bucket_size <= 0) p.bucket_size = 256;
    *out = st.release();
    return STLQ_MI355_OK;
}

int stlq_mi355_store_open_resume(const stlq_mi355_store_config* cfg, uint64_t start_id, const uint64_t* bucket_sizes,
                                 int64_t nbucket, stlq_mi355_store** out) {
    if (!out) return Invalid("store_open_resume: out is null");
    *out = nullptr;
    auto st = std::make_unique<stlq_mi355_store>();
    if (int rc = ReadConfig(cfg, &st->p, "BaseBasicWriter::OpenResume")) return rc;
    Params& p = st->p;
    st->resume = true;
    st->resume_id = start_id;
    st->flush_bytes = static_cast<size_t>(std::max(1, p.bucket_flush_mb)) << 20;
    if (p.bucket_size <= 0) p.bucket_size = 256;
    if (!MakeDirs(p.dir)) return Invalid("BaseBasicWriter: failed to create dir: " + p.dir);
    const uint64_t ss = static_cast<uint64_t>(std::max(1, p.shard_size));
    st->resume_shard = static_cast<int>(start_id / ss);
    st->resume_in_shard = static_cast<int64_t>(start_id % ss);
    const int64_t nb = BucketCount(p.h_vec, p.bucket_size);
    st->SizeBuckets(nb);
    if (nbucket != nb || (nb > 0 && !bucket_sizes))
        return Invalid("BaseBasicWriter::OpenResume: bucket_sizes length mismatch (got=" + std::to_string(nbucket) +
                       ", expected=" + std::to_string(nb) + ")");
    st->committed.assign(bucket_sizes, bucket_sizes + nb);
    const std::string ids = Under(p.dir, "cluster_id.u32");
    std::error_code ec;
    if (!fs::exists(ids, ec)) return Invalid("BaseBasicWriter::OpenResume: missing cluster_id.u32 under: " + p.dir);
    if (!st->cluster_ids.Open(ids, true)) return Invalid("BaseBasicWriter::OpenResume: cannot open " + ids);
    *out = st.release();
    return STLQ_MI355_OK;
}

int stlq_mi355_store_append(stlq_mi355_store* st, uint64_t start_id, int64_t count, const uint32_t* cluster_id,
                            int b_rows, const uint8_t* B_small, int a_rows, const float* a, int raw_kind,
                            const void* raw, int64_t ld_raw) {
    if (!st) return Invalid("store_append: store is null");
    if (count < 0) return Invalid("store_append: negative count");
    if (count == 0) return STLQ_MI355_OK;
    const Params& p = st->p;
    const int m_codes = std::max(0, p.m - 1);
    if (b_rows != m_codes || a_rows != p.m) return Invalid("BaseBasicWriter::AppendBlock: B/a shape mismatch");
    if (!cluster_id || !a || (m_codes > 0 && !B_small)) return Invalid("store_append: null block array");
    if (raw_kind != STLQ_MI355_RAW_NONE && raw_kind != STLQ_MI355_RAW_U8 && raw_kind != STLQ_MI355_RAW_F32)
        return Invalid("store_append: unknown raw_kind");
    const size_t esz = raw_kind == STLQ_MI355_RAW_F32 ? sizeof(float) : 1;
    if (raw_kind != STLQ_MI355_RAW_NONE && p.vector_bucket) {  // AppendBlockRawU8/F32 check first
        if (!raw) return Invalid("BaseBasicWriter::AppendBlockRaw: write_vector_bucket=true but the raw tile is null");
        if (ld_raw < p.d) return Invalid("BaseBasicWriter::AppendBlockRaw: invalid leading dimension");
        if (static_cast<size_t>(p.raw_bytes) != static_cast<size_t>(p.d) * esz)
            return Invalid("BaseBasicWriter::AppendBlockRaw: raw_bytes_per_vec does not match the raw element type");
    }
    const size_t n = static_cast<size_t>(count);
    if (!st->cluster_ids.Write(cluster_id, n * sizeof(uint32_t)))
        return Invalid("BaseBasicWriter::AppendBlock: failed to write cluster_id file");
    if (int rc = st->SelectShard(start_id)) return rc;
    const bool ok_codes = st->codes.Write(B_small, static_cast<size_t>(m_codes) * n);
    const bool ok_coeffs = st->coeffs.Write(a, static_cast<size_t>(p.m) * n * sizeof(float));
    if (!ok_codes || !ok_coeffs) return Invalid("BaseBasicWriter::AppendBlock: failed to write shard outputs");
    if (!p.vector_bucket && !p.basic_bucket) return STLQ_MI355_OK;
    if (p.vector_bucket && raw_kind == STLQ_MI355_RAW_NONE)
        return Invalid("BaseBasicWriter::AppendBlock: write_vector_bucket=true but no raw vectors were given");

    // Record: uint32 global id, uint32 cluster id, [raw vector], [m-1 codes, m coefficients].
    const size_t raw_b = p.vector_bucket ? static_cast<size_t>(p.raw_bytes) : 0;
    const size_t basic_b = p.basic_bucket ? static_cast<size_t>(m_codes) + static_cast<size_t>(p.m) * sizeof(float) : 0;
    const size_t rec = 2 * sizeof(uint32_t) + raw_b + basic_b;
    const uint32_t per_bucket = static_cast<uint32_t>(std::max(1, p.bucket_size));
    const auto* raw_bytes = static_cast<const uint8_t*>(raw);
    const size_t raw_stride = static_cast<size_t>(ld_raw) * esz;
    for (size_t i = 0; i < n; ++i) {
        const uint32_t cid = cluster_id[i];
        const int b = static_cast<int>(cid / per_bucket);
        if (int rc = st->OpenBucket(b)) return rc;
        std::vector<uint8_t>& buf = st->buckets[static_cast<size_t>(b)]->pending;
        const size_t at = buf.size();
        buf.resize(at + rec);
        uint8_t* w = buf.data() + at;
        const uint32_t gid = static_cast<uint32_t>(start_id + i);
        std::memcpy(w, &gid, 4);
        std::memcpy(w + 4, &cid, 4);
        w += 8;
        if (raw_b) {
            std::memcpy(w, raw_bytes + i * raw_stride, raw_b);
            w += raw_b;
        }
        if (basic_b) {
            if (m_codes) std::memcpy(w, B_small + i * static_cast<size_t>(m_codes), static_cast<size_t>(m_codes));
            std::memcpy(w + m_codes, a + i * static_cast<size_t>(p.m), static_cast<size_t>(p.m) * sizeof(float));
        }
        if (buf.size() >= st->flush_bytes)
            if (int rc = st->WriteOut(static_cast<size_t>(b))) return rc;
    }
    return STLQ_MI355_OK;
}

int stlq_mi355_store_flush(stlq_mi355_store* st) {
    if (!st) return Invalid("store_flush: store is null");
    for (size_t b = 0; b < st->buckets.size(); ++b) {
        if (int rc = st->WriteOut(b)) return rc;
        auto& bk = *st->buckets[b];
        if (bk.open && !bk.file.Flush()) return Invalid("BaseBasicWriter::Flush: bucket flush failed");
    }
    if (st->codes.IsOpen() && !st->codes.Flush()) return Invalid("BaseBasicWriter::Flush: codes shard flush failed");
    if (st->coeffs.IsOpen() && !st->coeffs.Flush()) return Invalid("BaseBasicWriter::Flush: coeffs shard flush failed");
    if (st->cluster_ids.IsOpen() && !st->cluster_ids.Flush())
        return Invalid("BaseBasicWriter::Flush: cluster_id flush failed");
    return STLQ_MI355_OK;
}

int stlq_mi355_store_bucket_bytes(const stlq_mi355_store* st, uint64_t* out, int64_t cap, int64_t* nbucket) {
    if (!st) return Invalid("store_bucket_bytes: store is null");
    const int64_t n = static_cast<int64_t>(st->committed.size());
    if (nbucket) *nbucket = n;
    if (out)
        for (int64_t i = 0; i < std::min(cap, n); ++i) out[i] = st->committed[static_cast<size_t>(i)];
    return STLQ_MI355_OK;
}

int stlq_mi355_store_info(const stlq_mi355_store* st, int* d, int* m, int* h0, int* write_vector_bucket,
                          int* raw_bytes_per_vec) {
    if (!st) return Invalid("store_info: store is null");
    if (d) *d = st->p.d;
    if (m) *m = st->p.m;
    if (h0) *h0 = st->p.h_vec.empty() ? 0 : st->p.h_vec.front();
    if (write_vector_bucket) *write_vector_bucket = st->p.vector_bucket ? 1 : 0;
    if (raw_bytes_per_vec) *raw_bytes_per_vec = st->p.raw_bytes;
    return STLQ_MI355_OK;
}

int stlq_mi355_store_close(stlq_mi355_store* st) {
    if (!st) return STLQ_MI355_OK;
    std::unique_ptr<stlq_mi355_store> own(st);
    for (size_t b = 0; b < st->buckets.size(); ++b) {
        if (int rc = st->WriteOut(b)) return rc;
        auto& bk = *st->buckets[b];
        bk.file.Close();
        bk.open = false;
        bk.pending.clear();
    }
    st->codes.Close();
    st->coeffs.Close();
    st->cluster_ids.Flush();
    st->cluster_ids.Close();
    st->shard = -1;
    return STLQ_MI355_OK;
}

int stlq_mi355_checkpoint_write(const char* path, uint64_t next_id, const uint64_t* bucket_sizes, int64_t nbucket) {
    if (!path || nbucket < 0 || nbucket > UINT32_MAX || (nbucket > 0 && !bucket_sizes))
        return Invalid("checkpoint_write: bad arguments");
    const fs::path target(path);
    std::error_code ec;
    if (target.has_parent_path()) fs::create_directories(target.parent_path(), ec);
    if (ec) return Invalid("WriteBaseBasicCheckpoint: failed to create dir: " + target.parent_path().string());
    const fs::path tmp = target.parent_path() / (target.filename().string() + ".tmp");
    {
        OutFile f;
        if (!f.Open(tmp.string(), false)) return Invalid("WriteBaseBasicCheckpoint: failed to open tmp: " + tmp.string());
        const uint32_t head[4] = {0x544b4342u /* "BCKT" */, 1u, static_cast<uint32_t>(nbucket), 0u};
        f.Write(head, sizeof(head));
        f.Write(&next_id, sizeof(next_id));
        if (nbucket > 0) f.Write(bucket_sizes, static_cast<size_t>(nbucket) * sizeof(uint64_t));
        if (!f.Flush()) return Invalid("WriteBaseBasicCheckpoint: write failed");
    }
    fs::rename(tmp, target, ec);
    if (ec) return Invalid("WriteBaseBasicCheckpoint: rename failed");
    return STLQ_MI355_OK;
}

int stlq_mi355_checkpoint_read(const char* path, uint64_t* next_id, uint64_t* bucket_sizes, int64_t cap,
                               int64_t* nbucket) {
    if (!path) return Invalid("checkpoint_read: path is null");
    std::FILE* f = std::fopen(path, "rb");
    if (!f) return Invalid(std::string("ReadBaseBasicCheckpoint: failed to open: ") + path);
    uint32_t head[4];
    uint64_t next = 0;
    bool ok = std::fread(head, sizeof(head), 1, f) == 1 && std::fread(&next, sizeof(next), 1, f) == 1;
    if (!ok) {
        std::fclose(f);
        return Invalid("ReadBaseBasicCheckpoint: header read failed");
    }
    if (head[0] != 0x544b4342u || head[1] != 1u) {
        std::fclose(f);
        return Invalid("ReadBaseBasicCheckpoint: bad magic/version");
    }
    std::vector<uint64_t> sizes(head[2]);
    if (!sizes.empty() && std::fread(sizes.data(), sizeof(uint64_t), sizes.size(), f) != sizes.size()) {
        std::fclose(f);
        return Invalid("ReadBaseBasicCheckpoint: bucket sizes read failed");
    }
    std::fclose(f);
    if (next_id) *next_id = next;
    if (nbucket) *nbucket = static_cast<int64_t>(sizes.size());
    if (bucket_sizes)
        for (int64_t i = 0; i < std::min<int64_t>(cap, static_cast<int64_t>(sizes.size())); ++i)
            bucket_sizes[i] = sizes[static_cast<size_t>(i)];
    return STLQ_MI355_OK;
}

int stlq_mi355_store_truncate_to_checkpoint(const stlq_mi355_store_config* cfg, uint64_t next_id,
                                            const uint64_t* bucket_sizes, int64_t nbucket) {
    if (!cfg || !cfg->dir || (cfg->h_len > 0 && !cfg->h_vec) || cfg->h_len < 0)
        return Invalid("truncate_to_checkpoint: bad config");
    const std::string dir = cfg->dir;
    const std::vector<int> h_vec(cfg->h_vec, cfg->h_vec + cfg->h_len);
    if (!ResizeFile(Under(dir, "cluster_id.u32"), next_id * sizeof(uint32_t)))
        return Invalid("Failed to truncate: " + Under(dir, "cluster_id.u32"));
    const uint64_t ss = static_cast<uint64_t>(std::max(1, cfg->shard_size));
    const uint64_t in_shard = next_id % ss;
    const std::string tag = Tag4(static_cast<int>(next_id / ss));
    const uint64_t m = static_cast<uint64_t>(std::max(1, cfg->m));
    const uint64_t m_codes = static_cast<uint64_t>(std::max(0, cfg->m - 1));
    if (!ResizeFile(Under(dir, "codes_shard_" + tag + ".bin"), in_shard * m_codes) ||
        !ResizeFile(Under(dir, "coeffs_shard_" + tag + ".bin"), in_shard * m * sizeof(float)))
        return Invalid("Failed to truncate shard outputs");
    const int64_t nb = BucketCount(h_vec, cfg->bucket_size);
    if (nbucket != nb || (nb > 0 && !bucket_sizes)) return Invalid("Checkpoint bucket layout mismatch");
    for (int64_t b = 0; b < nb; ++b) {
        const std::string path = Under(dir, "bucket_" + Tag4(static_cast<int>(b)) + ".bin");
        if (!ResizeFile(path, bucket_sizes[b])) return Invalid("Failed to truncate bucket: " + path);
    }
    return STLQ_MI355_OK;
}

}  // extern "C"
