// Host-sanitizer driver of the BaseBasicStore writer (stlq_amd/csrc/base_store.cpp), built by
// tests/test_sanitizers_cpu.py with -fsanitize=address,undefined: opens, appends with every raw
// kind, flushes mid-stream, checkpoints, truncates, resumes and walks the error paths. Exits 0
// when every call behaved as expected; any sanitizer report aborts the process.
#include <algorithm>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "errors.hpp"
#include "stlq_mi355_store.h"

namespace {
thread_local std::string g_err;
}

int stlq_mi355::SetLastError(int code, const std::string& msg) {
    g_err = msg;
    return code;
}
extern "C" const char* stlq_mi355_last_error(void) { return g_err.c_str(); }

#define EXPECT(cond)                                                             \
    do {                                                                         \
        if (!(cond)) {                                                           \
            std::fprintf(stderr, "line %d: %s (%s)\n", __LINE__, #cond, g_err.c_str()); \
            return 1;                                                            \
        }                                                                        \
    } while (0)

int main(int argc, char** argv) {
    if (argc < 2) return 2;
    const std::string root = argv[1];
    const int d = 24, m = 4, n = 5000, block = 700;
    const int h_vec[m] = {1000, 16, 16, 16};
    std::vector<uint32_t> cid(n);
    std::vector<uint8_t> B(static_cast<size_t>(n) * (m - 1)), xu8(static_cast<size_t>(n) * d);
    std::vector<float> a(static_cast<size_t>(n) * m), xf(static_cast<size_t>(n) * d);
    uint32_t s = 12345;
    auto next = [&]() { return s = s * 1664525u + 1013904223u; };
    for (int i = 0; i < n; ++i) cid[i] = next() % 1300;  // some ids past the 4-bucket layout
    for (auto& v : B) v = static_cast<uint8_t>(next());
    for (auto& v : xu8) v = static_cast<uint8_t>(next());
    for (auto& v : a) v = static_cast<float>(next() % 1000) * 0.01f;
    for (auto& v : xf) v = static_cast<float>(next() % 1000) * 0.5f;

    for (int kind = 0; kind < 3; ++kind) {
        const std::string dir = root + "/k" + std::to_string(kind);
        stlq_mi355_store_config cfg{};
        stlq_mi355_store_config_init(&cfg);
        cfg.dir = dir.c_str();
        cfg.d = d;
        cfg.m = m;
        cfg.h_vec = h_vec;
        cfg.h_len = m;
        cfg.shard_size = 1400;
        cfg.bucket_flush_mb = 1;
        cfg.write_vector_bucket = kind != 0;
        cfg.raw_bytes_per_vec = kind == 2 ? d * 4 : 0;
        stlq_mi355_store* st = nullptr;
        EXPECT(stlq_mi355_store_open(&cfg, &st) == 0);
        const std::string ck = dir + "/checkpoint/base_basic/ckpt.bin";
        for (int b0 = 0; b0 < 3 * block; b0 += block) {
            const void* raw = kind == 1 ? static_cast<const void*>(xu8.data() + static_cast<size_t>(b0) * d)
                                        : static_cast<const void*>(xf.data() + static_cast<size_t>(b0) * d);
            EXPECT(stlq_mi355_store_append(st, b0, block, cid.data() + b0, m - 1, B.data() + static_cast<size_t>(b0) * (m - 1),
                                           m, a.data() + static_cast<size_t>(b0) * m, kind, kind ? raw : nullptr, d) == 0);
            EXPECT(stlq_mi355_store_flush(st) == 0);
            int64_t nb = 0;
            EXPECT(stlq_mi355_store_bucket_bytes(st, nullptr, 0, &nb) == 0 && nb == 4);
            std::vector<uint64_t> sizes(static_cast<size_t>(nb));
            EXPECT(stlq_mi355_store_bucket_bytes(st, sizes.data(), nb, &nb) == 0);
            EXPECT(stlq_mi355_checkpoint_write(ck.c_str(), b0 + block, sizes.data(), nb) == 0);
        }
        EXPECT(stlq_mi355_store_append(st, 3 * block, 100, cid.data(), m - 1, B.data(), m, a.data(), kind,
                                       kind == 1 ? static_cast<const void*>(xu8.data()) : xf.data(), d) == 0);
        EXPECT(stlq_mi355_store_close(st) == 0);  // a block past the checkpoint
        uint64_t nid = 0;
        int64_t nb = 0;
        uint64_t sizes[8] = {};
        EXPECT(stlq_mi355_checkpoint_read(ck.c_str(), &nid, sizes, 8, &nb) == 0 && nid == 3u * block && nb == 4);
        EXPECT(stlq_mi355_store_truncate_to_checkpoint(&cfg, nid, sizes, nb) == 0);
        EXPECT(stlq_mi355_store_open_resume(&cfg, nid, sizes, nb, &st) == 0);
        for (int b0 = static_cast<int>(nid); b0 < n; b0 += block) {
            const int cnt = std::min(block, n - b0);
            const void* raw = kind == 1 ? static_cast<const void*>(xu8.data() + static_cast<size_t>(b0) * d)
                                        : static_cast<const void*>(xf.data() + static_cast<size_t>(b0) * d);
            EXPECT(stlq_mi355_store_append(st, b0, cnt, cid.data() + b0, m - 1, B.data() + static_cast<size_t>(b0) * (m - 1),
                                           m, a.data() + static_cast<size_t>(b0) * m, kind, kind ? raw : nullptr, d) == 0);
        }
        EXPECT(stlq_mi355_store_close(st) == 0);
        // error paths
        EXPECT(stlq_mi355_store_open_resume(&cfg, 0, sizes, 3, &st) != 0 && st == nullptr);
        EXPECT(stlq_mi355_store_open(&cfg, &st) == 0);
        EXPECT(stlq_mi355_store_append(st, 0, 10, cid.data(), m, B.data(), m, a.data(), kind, xf.data(), d) != 0);
        EXPECT(stlq_mi355_store_append(st, 0, 10, cid.data(), m - 1, B.data(), m, a.data(), 7, nullptr, 0) != 0);
        if (kind) EXPECT(stlq_mi355_store_append(st, 0, 10, cid.data(), m - 1, B.data(), m, a.data(), kind, nullptr, d) != 0);
        if (kind) EXPECT(stlq_mi355_store_append(st, 0, 10, cid.data(), m - 1, B.data(), m, a.data(), kind, xf.data(), d - 1) != 0);
        EXPECT(stlq_mi355_store_close(st) == 0);
    }
    stlq_mi355_store* st = nullptr;
    stlq_mi355_store_config bad{};
    EXPECT(stlq_mi355_store_open(&bad, &st) != 0 && st == nullptr);
    EXPECT(stlq_mi355_store_open(nullptr, &st) != 0);
    EXPECT(stlq_mi355_checkpoint_read((root + "/missing.bin").c_str(), nullptr, nullptr, 0, nullptr) != 0);
    EXPECT(stlq_mi355_store_close(nullptr) == 0);
    std::puts("store sanitizer run ok");
    return 0;
}
