// C ABI of libstlq_mi355: context, device precomp, tiled encode orchestration, streaming.
// The reference routine each entry point replaces is named in include/stlq_mi355.h.
#include "stlq_mi355.h"
#include "stlq_mi355_tools.h"
#include "stlq_mi355_store.h"
#include "errors.hpp"
#include "internal.hpp"
#include "prune_bound.hpp"

#include <algorithm>
#include <climits>
#include <chrono>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <numeric>
#include <random>
#include <string>
#include <vector>

using namespace stlq_mi355;

namespace {

thread_local std::string g_err;

int Fail(int code, const std::string& msg) {
    g_err = msg;
    return code;
}

#define HIP_TRY(expr)                                                                         \
    do {                                                                                      \
        hipError_t e_ = (expr);                                                               \
        if (e_ != hipSuccess)                                                                 \
            return Fail(STLQ_MI355_ERR_HIP, std::string(#expr) + ": " + hipGetErrorString(e_)); \
    } while (0)

#define RC_TRY(expr)                   \
    do {                               \
        int rc_ = (expr);              \
        if (rc_ != STLQ_MI355_OK) return rc_; \
    } while (0)

struct DevBuf {
    void* p = nullptr;
    size_t bytes = 0;
    // A range of the static no-allocation scratch lent for one call: never freed or regrown.
    bool borrowed = false;
    hipError_t Ensure(size_t want) {
        if (want <= bytes && p) return hipSuccess;
        if (borrowed) return hipErrorOutOfMemory;
        if (p) {
            hipError_t e = hipFree(p);
            if (e != hipSuccess) return e;
        }
        p = nullptr;
        bytes = 0;
        if (want == 0) want = 256;
        hipError_t e = hipMalloc(&p, want);
        if (e == hipSuccess) bytes = want;
        return e;
    }
    void Release() {
        if (p && !borrowed) (void)hipFree(p);
        p = nullptr;
        bytes = 0;
        borrowed = false;
    }
    template <class T>
    T* as() const {
        return static_cast<T*>(p);
    }
};

// One tile's event set; resolved lazily when timings are read.
struct TileEvents {
    hipEvent_t e[7] = {};  // start, xnorm, gemm, beam, ls, icm, end
    hipEvent_t gemm_end = nullptr;  // set when the GEMM ran on the aux stream (then e[2] = beam start)
    hipEvent_t lay[kMaxM + 1] = {};  // before layer 0, after each beam layer
    int layers = 0;
    int64_t n = 0;
    int gemm_launches = 0;
    int beam_launches = 0;
};

int64_t EnvWorkspaceBytes() {
    const char* s = std::getenv("STLQ_MI355_WORKSPACE_GB");
    double gb = s ? std::atof(s) : 24.0;
    if (!(gb > 0.0)) gb = 24.0;
    return static_cast<int64_t>(gb * 1024.0 * 1024.0 * 1024.0);
}

// Static device scratch of stlq_mi355_encode_device_noalloc: every work buffer of that entry
// point (||x||^2, xC, beam records, flags, counters, ICM/ILS state) is a range of this array, so
// the call allocates nothing. Each device holds its own copy for the life of the process; host
// code reaches it only through the address hipGetSymbolAddress returns for that device
// (ScratchAddress), never through the symbol itself.
constexpr size_t kScratchBytes = size_t{256} << 20;
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

}  // namespace

static __device__ __align__(256) unsigned char scratch[kScratchBytes];

namespace {

// The device address of `scratch` on `device` (which must be current), looked up once per device.
hipError_t ScratchAddress(int device, void** out) {
    *out = nullptr;
    if (device < 0 || device >= kMaxDevices) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[device]) {
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return e;
        g_scratch_ptr[device] = p;
    }
    *out = g_scratch_ptr[device];
    return hipSuccess;
}

}  // namespace

struct stlq_mi355_ctx {
    int device = 0;
    hipStream_t stream = nullptr;
    hipStream_t copy_stream = nullptr;
    hipStream_t aux_stream = nullptr;  // xC GEMM of the next sub-tile while the current one's beam runs

    // Full precomp (BuildPrecomp).
    bool has_pre = false;
    int d = 0, m = 0, H = 0;
    int h_vec[kMaxM] = {}, off[kMaxM] = {};
    DevBuf C_all, G_rm, G_cm, gdiag, invnorm;
    bool g_shared = true;  // G_cm aliases G_rm (symmetric G built on the device)
    // Beam candidate pruning (prune_bound.hpp): the codewords' scalings sw, isw and the row-scaled
    // Gram Gs; allowed when max |G| <= 2^30.
    DevBuf Gs, sw, isw, absmax;
    bool prune_full = false;

    // Large-root precomp (BuildPrecompLargeRoot).
    bool has_lr = false;
    int lr_d = 0, lr_m = 0, h0 = 0, Hs = 0;
    int lr_h[kMaxM] = {}, soff[kMaxM] = {};
    DevBuf C0, Cs, norm0, G_small, G0S, gdiag_small, invnorm_small;
    DevBuf Gs_small, sw_small, isw_small, sw0, isw0;  // the same for the small layers and the roots
    bool prune_lr = false;      // max |G_small|, |G0S| <= 2^30

    // Work buffers (grown on demand, reused across calls).
    DevBuf X, nx2, xC, xC_in, codes, a, cost, best, fails, active, changed, mse, gam0, roots, scores, b0;
    DevBuf ils_codes, ils_a, ils_cost;  // ILS candidate state
    DevBuf R_in, R_rm;                  // rotation: as given (column-major) and row-major
    DevBuf nearest, nearest_flag;       // large root: nearest root per vector, NaN flags
    DevBuf icm_pend;                    // ICM: the layer's proposed code per vector
    DevBuf st_rec[2], st_curH[2];
    // Best-first beam pass: per-vector flags, the list of flagged vectors, and two counters
    // (this tile's count, and the total since the timings were last reset).
    DevBuf bf_flags, bf_list, bf_count;
    bool bf_reset = true;  // clear the total at the next best-first pass
    bool bf_used = false;  // a best-first pass ran since the timings were reset
    int* bf_host = nullptr;  // pinned copy of bf_count, refreshed after every best-first pass

    void* scratch = nullptr;  // this device's address of the static no-allocation scratch
    bool noalloc = false;     // inside stlq_mi355_encode_device_noalloc: no pinned copies, no events

    std::vector<TileEvents> tiles;
    std::vector<hipEvent_t> event_pool;
    size_t event_next = 0;

    hipEvent_t NextEvent() {
        if (event_next == event_pool.size()) {
            hipEvent_t e = nullptr;
            if (hipEventCreate(&e) != hipSuccess) return nullptr;
            event_pool.push_back(e);
        }
        return event_pool[event_next++];
    }
    bool overlapped = false;  // tiles of the last call overlapped in time (total = envelope)
    void ResetTimings() {
        tiles.clear();
        event_next = 0;
        overlapped = false;
        bf_reset = true;
        bf_used = false;
    }
};

namespace {

// Candidate pruning in the beam (on unless STLQ_MI355_PRUNE=0). It never changes a result: a
// pruned candidate is one the reference's rule rejects.
bool PruneEnv() {
    const char* v = std::getenv("STLQ_MI355_PRUNE");
    return !(v && std::strcmp(v, "0") == 0);
}

// Whether max |x| over the n floats at x (device) lies within the pruning envelope (2^30).
int GramInEnvelope(stlq_mi355_ctx* c, const float* const* mats, const int64_t* counts, int nm, bool* ok) {
    HIP_TRY(c->absmax.Ensure(4));
    HIP_TRY(LaunchFill8(c->absmax.as<uint8_t>(), 0, 4, c->stream));
    for (int i = 0; i < nm; ++i) HIP_TRY(LaunchAbsMaxBits(mats[i], counts[i], c->absmax.as<unsigned>(), c->stream));
    unsigned bits = 0xFFFFFFFFu;
    HIP_TRY(hipMemcpyAsync(&bits, c->absmax.p, 4, hipMemcpyDeviceToHost, c->stream));
    HIP_TRY(hipStreamSynchronize(c->stream));
    *ok = bits <= prune::kGAbsMaxBits;
    return STLQ_MI355_OK;
}

int CheckCtx(stlq_mi355_ctx* ctx) {
    if (!ctx) return Fail(STLQ_MI355_ERR_INVALID, "null context");
    HIP_TRY(hipSetDevice(ctx->device));
    return STLQ_MI355_OK;
}

int CheckPre(stlq_mi355_ctx* ctx) {
    RC_TRY(CheckCtx(ctx));
    if (!ctx->has_pre) return Fail(STLQ_MI355_ERR_STATE, "codebooks not set (call stlq_mi355_set_codebooks)");
    return STLQ_MI355_OK;
}

int CheckBeam(int Hb) {
    if (Hb < 1 || Hb > kMaxBeam)
        return Fail(STLQ_MI355_ERR_UNSUPPORTED, "H_beam must be in [1, 64], got " + std::to_string(Hb));
    return STLQ_MI355_OK;
}

int ValidateLayers(int d, int m, const int* h_vec, int first_max) {
    if (d <= 0) return Fail(STLQ_MI355_ERR_INVALID, "d must be positive");
    if (m < 1 || m > kMaxM) return Fail(STLQ_MI355_ERR_UNSUPPORTED, "m must be in [1, 20]");
    if (!h_vec) return Fail(STLQ_MI355_ERR_INVALID, "h_vec is null");
    for (int l = 0; l < m; ++l) {
        const int lim = (l == 0) ? first_max : kMaxK;
        if (h_vec[l] < 1 || h_vec[l] > lim)
            return Fail(STLQ_MI355_ERR_UNSUPPORTED,
                        "codebook size of layer " + std::to_string(l) + " out of range: " + std::to_string(h_vec[l]));
    }
    return STLQ_MI355_OK;
}

// Per-vector device bytes of one encode tile.
int64_t PerVectorBytes(int d, int m, int H, int Hb) {
    const int64_t state = static_cast<int64_t>(Hb) * 4 * BeamRecordStride(m);
    // ... + 5: best-first flag + list; + 4: ICM proposal
    return 4LL * d + 4 + 4LL * H + m + 4LL * m + 4 + 4 + 2 + 8 + 5 + 4 + 2 * (state + 4);
}

int64_t TileVectors(int64_t n, int d, int m, int H, int Hb) {
    const int64_t per = PerVectorBytes(d, m, H, Hb);
    int64_t t = EnvWorkspaceBytes() / std::max<int64_t>(per, 1);
    t = std::max<int64_t>(t, 1024);
    t = std::min<int64_t>(t, std::max<int64_t>(n, 1));
    return t;
}

int EnsureState(stlq_mi355_ctx* c, int64_t n, int m, int Hb) {
    const size_t slots = static_cast<size_t>(n) * Hb;
    for (int b = 0; b < 2; ++b) {
        HIP_TRY(c->st_rec[b].Ensure(slots * 4 * BeamRecordStride(m)));
        HIP_TRY(c->st_curH[b].Ensure(static_cast<size_t>(n) * 4));
    }
    return STLQ_MI355_OK;
}

BeamState StateOf(stlq_mi355_ctx* c, int b) {
    BeamState s;
    s.rec = c->st_rec[b].as<float>();
    s.curH = c->st_curH[b].as<int>();
    return s;
}

// Scan order of the full-precomp beam: best-first pass plus a reference-order re-run of the
// vectors it flags (the default), or the reference order throughout (STLQ_MI355_BEAM_ORDER=reference).
bool BestFirstBeam() {
    const char* v = std::getenv("STLQ_MI355_BEAM_ORDER");
    return !(v && std::strcmp(v, "reference") == 0);
}

// Full-precomp beam over one tile: layer 0 then layers 1..m-1 (BeamSearchPrefixLS).
//
// By default the layers first run best-first (LayerArgs::flags): parents in ascending error
// order, which admits far fewer candidates into the top-H on the way (about 80 instead of 115 per
// vector and layer at C2) and gives the reference's top-H sets, records and final pick except
// where candidates tie at the top-H boundary or for the final minimum (or an error is NaN or -0).
// Every such vector is flagged and then re-run on its own in the reference's slot order, so the
// results are the reference's in every case.
int RunBeam(stlq_mi355_ctx* c, const float* dxC, int64_t ldx, const float* dnx2, int64_t n, int Hb,
            uint8_t* dcodes, float* dbest, hipStream_t s, int* launches, TileEvents* te = nullptr) {
    RC_TRY(EnsureState(c, n, c->m, Hb));
    const bool best = c->m >= 2 && BestFirstBeam();
    if (best) {
        HIP_TRY(c->bf_flags.Ensure(static_cast<size_t>(n)));
        HIP_TRY(c->bf_list.Ensure(static_cast<size_t>(n) * 4));
        HIP_TRY(c->bf_count.Ensure(8));
        if (!c->bf_host && !c->noalloc)
            HIP_TRY(hipHostMalloc(reinterpret_cast<void**>(&c->bf_host), 8, hipHostMallocDefault));
        HIP_TRY(LaunchFill8(c->bf_flags.as<uint8_t>(), 0, n, s));
        HIP_TRY(LaunchFill8(c->bf_count.as<uint8_t>(), 0, (c->bf_reset || c->noalloc) ? 8 : 4, s));
        c->bf_reset = c->noalloc;  // (the no-allocation call's counters are its own)
        c->bf_used = !c->noalloc;
    }
    auto mark = [&](int k) -> hipError_t {
        if (!te) return hipSuccess;
        te->lay[k] = c->NextEvent();
        te->layers = k;
        return hipEventRecord(te->lay[k], s);
    };
    HIP_TRY(mark(0));
    LayerArgs a;
    a.gram.G = c->G_rm.as<float>();
    a.gram.ld = c->H;
    for (int l = 0; l < c->m; ++l) a.gram.off[l] = c->off[l];
    a.xC = dxC;
    a.ldx = ldx;
    a.nx2 = dnx2;
    a.gdiag = c->gdiag.as<float>();
    a.Gs = c->Gs.as<float>();
    a.sw = c->sw.as<float>();
    a.isw = c->isw.as<float>();
    a.prune = (c->prune_full && PruneEnv()) ? 1 : 0;
    a.n = n;
    a.m = c->m;
    a.Hb = Hb;
    a.codes_out = dcodes;
    a.best_err = dbest;
    a.flags = best ? c->bf_flags.as<uint8_t>() : nullptr;
    int nl = 0;
    auto layers = [&](bool timed) -> int {
        int cur = 0;
        a.out = StateOf(c, cur);
        a.K = c->h_vec[0];
        a.offL = c->off[0];
        a.is_last = (c->m == 1);
        HIP_TRY(LaunchBeamLayer0(a, s));
        if (timed) HIP_TRY(mark(1));
        ++nl;
        for (int L = 1; L < c->m; ++L) {
            a.in = StateOf(c, cur);
            a.out = StateOf(c, cur ^ 1);
            a.K = c->h_vec[L];
            a.offL = c->off[L];
            a.is_last = (L == c->m - 1);
            HIP_TRY(LaunchBeamLayer(L, false, a, s));
            if (timed) HIP_TRY(mark(L + 1));
            cur ^= 1;
            ++nl;
        }
        return STLQ_MI355_OK;
    };
    RC_TRY(layers(true));
    if (best) {
        // Re-run the flagged vectors in the reference order: one wave per listed vector, the
        // grid sized for all n (waves past the list's length exit at once).
        int* counts = c->bf_count.as<int>();
        HIP_TRY(LaunchCollectFlagged(c->bf_flags.as<uint8_t>(), n, c->bf_list.as<int>(), counts, s));
        a.flags = nullptr;
        a.list = c->bf_list.as<int>();
        a.list_n = counts;
        RC_TRY(layers(false));
        // for stlq_mi355_last_timings, without a synchronous copy there
        if (!c->noalloc) HIP_TRY(hipMemcpyAsync(c->bf_host, counts, 8, hipMemcpyDeviceToHost, s));
    }
    if (launches) *launches += nl;
    return STLQ_MI355_OK;
}

LsArgs MakeLs(stlq_mi355_ctx* c, const float* dxC, int64_t ldx, const uint8_t* dcodes, float* da, const float* dnx2,
              float* dcost, int64_t n) {
    LsArgs p;
    p.xC = dxC;
    p.ldx = ldx;
    p.G_rm = c->G_rm.as<float>();
    p.H = c->H;
    p.m = c->m;
    for (int l = 0; l < c->m; ++l) p.off[l] = c->off[l];
    p.codes = dcodes;
    p.a = da;
    p.nx2 = dnx2;
    p.cost = dcost;
    p.fails = c->fails.as<int>();
    p.n = n;
    p.cstride = c->m;
    return p;
}

// What one ICM / ILS run works on: the full precomp (G, invnorm, m codes per vector), or a large
// root (the small layers' G and invnorm, the roots' G0S rows and b0, m-1 codes per vector).
struct IcmProblem {
    LsArgs ls;  // all but codes, a and cost
    const float* G_cm = nullptr;
    const float* invnorm = nullptr;
    const int* h_vec = nullptr;  // host, m entries
    int lfirst = 0;              // layer of the first stored code
};

IcmProblem FullProblem(stlq_mi355_ctx* c, const float* dxC, int64_t ldx, const float* dnx2, int64_t n) {
    IcmProblem P;
    P.ls = MakeLs(c, dxC, ldx, nullptr, nullptr, dnx2, nullptr, n);
    P.G_cm = c->G_cm.as<float>();
    P.invnorm = c->invnorm.as<float>();
    P.h_vec = c->h_vec;
    return P;
}

// droot/db0: per-vector root ids and <C0[:,root], x> on the device; dxs: xC_small (Hs per vector).
IcmProblem LargeRootProblem(stlq_mi355_ctx* c, const float* dxs, const float* dnx2, const uint32_t* droot,
                            const float* db0, int64_t n) {
    IcmProblem P;
    LsArgs& p = P.ls;
    p.xC = dxs;
    p.ldx = c->Hs;
    p.G_rm = c->G_small.as<float>();
    p.H = c->Hs;
    p.m = c->lr_m;
    for (int l = 0; l < c->lr_m; ++l) p.off[l] = c->soff[l];
    p.nx2 = dnx2;
    p.fails = c->fails.as<int>();
    p.n = n;
    p.cstride = c->lr_m - 1;
    p.root = droot;
    p.b0 = db0;
    p.norm0 = c->norm0.as<float>();
    p.G0S_rm = c->G0S.as<float>();
    P.G_cm = c->G_small.as<float>();  // symmetric: its rows are its columns
    P.invnorm = c->invnorm_small.as<float>();
    P.h_vec = c->lr_h;
    P.lfirst = 1;
    return P;
}

std::vector<int> IcmOrders(int m, int iters, uint32_t seed) {
    // icm.cpp:119-122, :137/:242, :890: order = iota(m) shuffled in place once per iteration
    // with one std::mt19937(seed) stream.
    std::mt19937 rng(static_cast<std::mt19937::result_type>(seed));
    std::vector<int> order(m), all;
    std::iota(order.begin(), order.end(), 0);
    for (int it = 0; it < iters; ++it) {
        std::shuffle(order.begin(), order.end(), rng);
        all.insert(all.end(), order.begin(), order.end());
    }
    return all;
}

// RunIcm (icm.cpp:89-344) / RunIcmLargeRoot (:347-870) on one tile: LS refit + costs, then
// `iters` sweeps with the layer order of every sweep given (iters x m).
int RunIcmOrders(stlq_mi355_ctx* c, const IcmProblem& P, int iters, int use_abs, const std::vector<int>& orders,
                 uint8_t* dcodes, float* da, float* dcost, hipStream_t s) {
    LsArgs ls = P.ls;
    ls.codes = dcodes;
    ls.a = da;
    ls.cost = dcost;
    const int64_t n = ls.n;
    const int m = ls.m;
    HIP_TRY(LaunchLsAll(ls, s));
    HIP_TRY(LaunchCosts(ls, s));
    if (iters <= 0) return STLQ_MI355_OK;
    HIP_TRY(c->active.Ensure(static_cast<size_t>(n)));
    HIP_TRY(c->changed.Ensure(static_cast<size_t>(n)));
    HIP_TRY(c->icm_pend.Ensure(static_cast<size_t>(n) * 4));
    HIP_TRY(LaunchFill8(c->active.as<uint8_t>(), 1, n, s));
    IcmArgs q;
    q.pend = c->icm_pend.as<int>();
    q.ls = ls;
    q.codes_rw = dcodes;
    q.G_cm = P.G_cm;
    q.invnorm = P.invnorm;
    q.active = c->active.as<uint8_t>();
    q.changed = c->changed.as<uint8_t>();
    q.fails = c->fails.as<int>();
    q.use_abs = use_abs ? 1 : 0;
    for (int it = 0; it < iters; ++it) {
        HIP_TRY(LaunchFill8(q.changed, 0, n, s));
        for (int oi = 0; oi < m; ++oi) {
            const int j = orders[static_cast<size_t>(it) * m + oi];
            if (j == 0) continue;             // icm.cpp:250: layer 0 frozen (the root, for a large root)
            if (P.h_vec[j] <= 1) continue;    // icm.cpp:255
            q.j = j;
            q.hj = P.h_vec[j];
            HIP_TRY(LaunchIcmLayer(q, s));
        }
        HIP_TRY(LaunchIcmDeactivate(q.active, q.changed, n, s));
    }
    return STLQ_MI355_OK;
}

int RunIcm(stlq_mi355_ctx* c, const IcmProblem& P, int iters, int use_abs, uint32_t seed, uint8_t* dcodes, float* da,
           float* dcost, hipStream_t s) {
    return RunIcmOrders(c, P, iters, use_abs, IcmOrders(P.ls.m, iters, seed), dcodes, da, dcost, s);
}

// DynamicIcmWithIls{Abs,NoAbs}NoNormal[LargeRoot] (icm.cpp:872-1003, :1005-1120): RunIcm, then
// ils_iters rounds of perturb (PerturbKernel) -> RunIcm on the candidate codes ->
// accept-if-better. One std::mt19937(seed) stream supplies every RunIcm's layer orders, each
// RunIcm starting from the identity order (icm.cpp:121-137). id0 is the global id of vector 0
// (the reference's sample_id_offset), so a tile of a larger set perturbs exactly as the whole set
// would.
int RunIcmIls(stlq_mi355_ctx* c, const IcmProblem& P, int icm_iters, int ils_iters, int perturb_k, int use_abs,
              uint32_t seed, uint64_t id0, uint8_t* dcodes, float* da, float* dcost, hipStream_t s) {
    std::mt19937 rng(static_cast<std::mt19937::result_type>(seed));
    const int m = P.ls.m;
    const int64_t n = P.ls.n;
    auto next_orders = [&]() {
        std::vector<int> order(static_cast<size_t>(m)), out;
        std::iota(order.begin(), order.end(), 0);
        for (int it = 0; it < icm_iters; ++it) {
            std::shuffle(order.begin(), order.end(), rng);
            out.insert(out.end(), order.begin(), order.end());
        }
        return out;
    };
    RC_TRY(RunIcmOrders(c, P, icm_iters, use_abs, next_orders(), dcodes, da, dcost, s));
    if (ils_iters <= 0 || perturb_k <= 0 || m <= 1) return STLQ_MI355_OK;
    const size_t ncodes = static_cast<size_t>(n) * static_cast<size_t>(P.ls.cstride);
    const size_t nm = static_cast<size_t>(n) * static_cast<size_t>(m);
    HIP_TRY(c->ils_codes.Ensure(ncodes));
    HIP_TRY(c->ils_a.Ensure(nm * 4));
    HIP_TRY(c->ils_cost.Ensure(static_cast<size_t>(n) * 4));
    uint8_t* cc = c->ils_codes.as<uint8_t>();
    float* ca = c->ils_a.as<float>();
    float* ccost = c->ils_cost.as<float>();
    for (int outer = 0; outer < ils_iters; ++outer) {
        HIP_TRY(hipMemcpyAsync(cc, dcodes, ncodes, hipMemcpyDeviceToDevice, s));
        HIP_TRY(LaunchPerturb(cc, n, m, P.ls.cstride, P.lfirst, P.h_vec, perturb_k, seed, outer, id0, s));
        RC_TRY(RunIcmOrders(c, P, icm_iters, use_abs, next_orders(), cc, ca, ccost, s));
        HIP_TRY(LaunchIlsAccept(dcodes, da, dcost, cc, ca, ccost, n, m, P.ls.cstride, s));
    }
    return STLQ_MI355_OK;
}

struct EncodeOut {
    uint8_t* codes;  // device [n*m]
    float* a;        // device [n*m] or null
    float* cost;     // device [n] or null
    float* best;     // device [n] or null
};

// One tile of EncodeBase on device-resident X.
// Beam, LS refit + costs and ICM of one tile whose ||x||^2 and xC are already on the device.
int BeamAndRefit(stlq_mi355_ctx* c, const float* dxC, const float* dnx2, int64_t n, const stlq_mi355_encode_params& P,
                 const EncodeOut& o, hipStream_t s, TileEvents* te, uint64_t id0) {
    const int Hb = std::max(1, P.H_beam);
    auto rec = [&](int k) -> hipError_t {
        if (!te) return hipSuccess;
        te->e[k] = c->NextEvent();
        return hipEventRecord(te->e[k], s);
    };
    RC_TRY(RunBeam(c, dxC, c->H, dnx2, n, Hb, o.codes, o.best, s, te ? &te->beam_launches : nullptr, te));
    HIP_TRY(rec(3));
    const bool refine = P.icm_iters > 0 || P.ils_iters > 0;
    const bool need_ls = P.want_coeffs || refine;
    float* da = o.a;
    float* dcost = o.cost;
    if (need_ls) {
        if (!da) {
            HIP_TRY(c->a.Ensure(static_cast<size_t>(n) * c->m * 4));
            da = c->a.as<float>();
        }
        if (!dcost) {
            HIP_TRY(c->cost.Ensure(static_cast<size_t>(n) * 4));
            dcost = c->cost.as<float>();
        }
        if (!refine) {  // with refinement, RunIcm starts with this same refit
            LsArgs ls = MakeLs(c, dxC, c->H, o.codes, da, dnx2, dcost, n);
            HIP_TRY(LaunchLsAll(ls, s));
            HIP_TRY(LaunchCosts(ls, s));
        }
    }
    HIP_TRY(rec(4));
    if (refine) {
        RC_TRY(RunIcmIls(c, FullProblem(c, dxC, c->H, dnx2, n), P.icm_iters, P.ils_iters, P.perturb_k, P.use_abs,
                         P.seed, id0,
                         o.codes, da, dcost, s));
    }
    HIP_TRY(rec(5));
    HIP_TRY(rec(6));
    return STLQ_MI355_OK;
}

// Sub-tiles of a large tile: the xC GEMM (MFMA-bound) of sub-tile i+1 runs on the aux stream while
// the beam (VALU-bound) of sub-tile i runs on `s`, so the two share the CUs. Two xC/||x||^2
// buffers alternate; GEMM i+2 waits until sub-tile i's beam, LS and ICM are done with its buffer.
// Sub-tile length, from STLQ_MI355_PIPE_SUB; unset or 0 keeps one tile. Off by default: on the
// 1M-vector, 8 x 256, beam-16 encode the overlap saved about 1% of the wall time while the beam
// layers ran slower beside the GEMM, and the GEMM's own timing stops being measurable.
int64_t PipeSub() {
    const char* v = std::getenv("STLQ_MI355_PIPE_SUB");
    if (!v) return 0;
    const long long x = std::atoll(v);
    return x > 0 ? static_cast<int64_t>(x) : 0;
}

int EncodeTilePipelined(stlq_mi355_ctx* c, const float* dX, int64_t n, const stlq_mi355_encode_params& P,
                        const EncodeOut& o, hipStream_t s, bool record, uint64_t id0) {
    const int64_t sub = PipeSub();
    const int64_t nsub = (n + sub - 1) / sub;
    const size_t H = static_cast<size_t>(c->H), m = static_cast<size_t>(c->m);
    HIP_TRY(c->nx2.Ensure(2 * static_cast<size_t>(sub) * 4));
    HIP_TRY(c->xC.Ensure(2 * static_cast<size_t>(sub) * H * 4));
    float* xcb[2] = {c->xC.as<float>(), c->xC.as<float>() + static_cast<size_t>(sub) * H};
    float* nxb[2] = {c->nx2.as<float>(), c->nx2.as<float>() + sub};
    hipStream_t aux = c->aux_stream;
    std::vector<TileEvents> tes(static_cast<size_t>(nsub));
    std::vector<hipEvent_t> gemm_done(static_cast<size_t>(nsub)), tile_done(static_cast<size_t>(nsub));
    auto ev = [&](hipStream_t st) -> hipEvent_t {
        hipEvent_t e = c->NextEvent();
        if (e) (void)hipEventRecord(e, st);
        return e;
    };
    // the aux stream starts after everything already queued on s (input copies, earlier calls)
    hipEvent_t entry = ev(s);
    if (!entry) return Fail(STLQ_MI355_ERR_HIP, "event creation failed");
    HIP_TRY(hipStreamWaitEvent(aux, entry, 0));
    auto launch_front = [&](int64_t i) -> int {
        const int b = static_cast<int>(i & 1);
        const int64_t off = i * sub, ni = std::min(sub, n - off);
        if (i >= 2) HIP_TRY(hipStreamWaitEvent(aux, tile_done[static_cast<size_t>(i - 2)], 0));
        TileEvents& te = tes[static_cast<size_t>(i)];
        te.n = ni;
        te.e[0] = ev(aux);
        HIP_TRY(LaunchXNorm2(dX + off * c->d, c->d, ni, nxb[b], aux));
        te.e[1] = ev(aux);
        HIP_TRY(LaunchGemmXc(dX + off * c->d, ni, c->d, c->C_all.as<float>(), c->H, xcb[b], c->H, aux));
        te.gemm_launches = 1;
        te.gemm_end = gemm_done[static_cast<size_t>(i)] = ev(aux);
        if (!te.e[0] || !te.e[1] || !te.gemm_end) return Fail(STLQ_MI355_ERR_HIP, "event creation failed");
        return STLQ_MI355_OK;
    };
    RC_TRY(launch_front(0));
    for (int64_t i = 0; i < nsub; ++i) {
        if (i + 1 < nsub) RC_TRY(launch_front(i + 1));  // queued ahead of beam i so the two overlap
        const int b = static_cast<int>(i & 1);
        const int64_t off = i * sub, ni = std::min(sub, n - off);
        HIP_TRY(hipStreamWaitEvent(s, gemm_done[static_cast<size_t>(i)], 0));
        TileEvents& te = tes[static_cast<size_t>(i)];
        te.e[2] = ev(s);
        EncodeOut oi{o.codes + off * m, o.a ? o.a + off * m : nullptr, o.cost ? o.cost + off : nullptr,
                     o.best ? o.best + off : nullptr};
        RC_TRY(BeamAndRefit(c, xcb[b], nxb[b], ni, P, oi, s, &te, id0 + static_cast<uint64_t>(off)));
        tile_done[static_cast<size_t>(i)] = te.e[6];
        if (!te.e[6]) return Fail(STLQ_MI355_ERR_HIP, "event creation failed");
    }
    if (record) {
        for (const TileEvents& te : tes) c->tiles.push_back(te);
        c->overlapped = true;
    }
    return STLQ_MI355_OK;
}

// allow_overlap = false keeps the whole tile's xC and ||x||^2 in c->xC / c->nx2 afterwards.
// allow_overlap = false keeps the whole tile's xC and ||x||^2 in c->xC / c->nx2 afterwards.
// id0: global id of the tile's first vector (ILS perturbation stream).
int EncodeTile(stlq_mi355_ctx* c, const float* dX, int64_t n, const stlq_mi355_encode_params& P,
               const EncodeOut& o, hipStream_t s, bool record, bool allow_overlap = true, uint64_t id0 = 0) {
    const int64_t pipe = PipeSub();
    if (allow_overlap && pipe > 0 && n >= 2 * pipe) return EncodeTilePipelined(c, dX, n, P, o, s, record, id0);
    HIP_TRY(c->nx2.Ensure(static_cast<size_t>(n) * 4));
    HIP_TRY(c->xC.Ensure(static_cast<size_t>(n) * c->H * 4));
    TileEvents te;
    te.n = n;
    auto rec = [&](int k) -> hipError_t {
        if (!record) return hipSuccess;
        te.e[k] = c->NextEvent();
        return hipEventRecord(te.e[k], s);
    };
    HIP_TRY(rec(0));
    HIP_TRY(LaunchXNorm2(dX, c->d, n, c->nx2.as<float>(), s));
    HIP_TRY(rec(1));
    HIP_TRY(LaunchGemmXc(dX, n, c->d, c->C_all.as<float>(), c->H, c->xC.as<float>(), c->H, s));
    te.gemm_launches = 1;
    HIP_TRY(rec(2));
    RC_TRY(BeamAndRefit(c, c->xC.as<float>(), c->nx2.as<float>(), n, P, o, s, record ? &te : nullptr, id0));
    if (record) c->tiles.push_back(te);
    return STLQ_MI355_OK;
}

int CheckParams(const stlq_mi355_encode_params* p) {
    if (!p) return Fail(STLQ_MI355_ERR_INVALID, "params is null");
    if (p->icm_iters < 0 || p->ils_iters < 0 || p->perturb_k < 0)
        return Fail(STLQ_MI355_ERR_INVALID, "icm_iters, ils_iters and perturb_k must be >= 0");
    return CheckBeam(std::max(1, p->H_beam));
}

// Uploads a d x d column-major rotation and stores it row-major (R(r, k) at [r*d + k]), the
// operand layout of GemmXcKernel, so that GemmXc(X, R_rm) = R X per vector.
int UploadRotation(stlq_mi355_ctx* c, const float* R, int d, hipStream_t s) {
    const size_t bytes = static_cast<size_t>(d) * d * 4;
    HIP_TRY(c->R_in.Ensure(bytes));
    HIP_TRY(c->R_rm.Ensure(bytes));
    HIP_TRY(hipMemcpyAsync(c->R_in.p, R, bytes, hipMemcpyHostToDevice, s));
    HIP_TRY(LaunchTranspose(c->R_in.as<float>(), d, d, c->R_rm.as<float>(), s));
    return STLQ_MI355_OK;
}

double Mean(const std::vector<float>& v) {
    // MeanMseFromPrecomp accumulates in double and clamps each error at 0 (linkage_tools.cpp:170-221).
    double s = 0.0;
    for (float x : v) s += x < 0.0f ? 0.0 : static_cast<double>(x);
    return v.empty() ? 0.0 : s / static_cast<double>(v.size());
}

}  // namespace

int stlq_mi355::SetLastError(int code, const std::string& msg) { return Fail(code, msg); }

extern "C" {

const char* stlq_mi355_last_error(void) { return g_err.c_str(); }

const char* stlq_mi355_version(void) { return "stlq_mi355 1.0 gfx950"; }

int stlq_mi355_ctx_create(int device, stlq_mi355_ctx** out) {
    if (!out) return Fail(STLQ_MI355_ERR_INVALID, "out is null");
    *out = nullptr;
    int count = 0;
    HIP_TRY(hipGetDeviceCount(&count));
    if (device < 0 || device >= count) return Fail(STLQ_MI355_ERR_INVALID, "no HIP device " + std::to_string(device));
    HIP_TRY(hipSetDevice(device));
    auto* c = new stlq_mi355_ctx();
    c->device = device;
    if (hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking) != hipSuccess ||
        hipStreamCreateWithFlags(&c->copy_stream, hipStreamNonBlocking) != hipSuccess ||
        hipStreamCreateWithFlags(&c->aux_stream, hipStreamNonBlocking) != hipSuccess) {
        delete c;
        return Fail(STLQ_MI355_ERR_HIP, "stream creation failed");
    }
    if (c->fails.Ensure(256) != hipSuccess) {
        delete c;
        return Fail(STLQ_MI355_ERR_HIP, "allocation failed");
    }
    // Once per device, with the device current: the address of the no-allocation scratch.
    const hipError_t se = ScratchAddress(device, &c->scratch);
    if (se != hipSuccess) {
        stlq_mi355_ctx_destroy(c);
        return Fail(STLQ_MI355_ERR_HIP, std::string("hipGetSymbolAddress(scratch): ") + hipGetErrorString(se));
    }
    *out = c;
    return STLQ_MI355_OK;
}

int stlq_mi355_ctx_destroy(stlq_mi355_ctx* c) {
    if (!c) return STLQ_MI355_OK;
    (void)hipSetDevice(c->device);
    (void)hipStreamSynchronize(c->stream);
    (void)hipStreamSynchronize(c->copy_stream);
    (void)hipStreamSynchronize(c->aux_stream);
    DevBuf* bufs[] = {&c->C_all, &c->G_rm, &c->G_cm, &c->gdiag, &c->invnorm, &c->C0, &c->Cs, &c->norm0,
                      &c->G_small, &c->G0S, &c->gdiag_small, &c->X, &c->nx2, &c->xC, &c->xC_in, &c->codes, &c->a,
                      &c->cost, &c->best, &c->fails, &c->active, &c->changed, &c->mse, &c->gam0, &c->roots,
                      &c->scores, &c->ils_codes, &c->ils_a, &c->ils_cost, &c->b0, &c->invnorm_small,
                      &c->R_in, &c->R_rm, &c->nearest, &c->nearest_flag, &c->bf_flags, &c->bf_list,
                      &c->bf_count, &c->icm_pend, &c->Gs, &c->sw, &c->isw, &c->absmax, &c->Gs_small,
                      &c->sw_small, &c->isw_small, &c->sw0, &c->isw0};
    if (c->g_shared) c->G_cm.p = nullptr;
    for (DevBuf* b : bufs) b->Release();
    for (int b = 0; b < 2; ++b) {
        c->st_rec[b].Release();
        c->st_curH[b].Release();
    }
    for (hipEvent_t e : c->event_pool) (void)hipEventDestroy(e);
    if (c->bf_host) (void)hipHostFree(c->bf_host);
    (void)hipStreamDestroy(c->stream);
    (void)hipStreamDestroy(c->copy_stream);
    (void)hipStreamDestroy(c->aux_stream);
    delete c;
    return STLQ_MI355_OK;
}

// The pruning scalings, the row-scaled Gram and the pruning envelope of the full precomp
// (synchronizes the stream).
static int SetPruneFull(stlq_mi355_ctx* c) {
    const size_t H = static_cast<size_t>(c->H);
    HIP_TRY(c->sw.Ensure(H * 4));
    HIP_TRY(c->isw.Ensure(H * 4));
    HIP_TRY(c->Gs.Ensure(H * H * 4));
    HIP_TRY(LaunchPruneScale(c->gdiag.as<float>(), c->H, c->sw.as<float>(), c->isw.as<float>(), c->stream));
    HIP_TRY(LaunchRowScale(c->G_rm.as<float>(), c->H, c->H, c->sw.as<float>(), c->Gs.as<float>(), c->stream));
    const float* mats[1] = {c->G_rm.as<float>()};
    const int64_t counts[1] = {static_cast<int64_t>(H * H)};
    return GramInEnvelope(c, mats, counts, 1, &c->prune_full);
}

static int SetPrecompCommon(stlq_mi355_ctx* c, int d, int m, const int* h_vec, const float* C_all) {
    RC_TRY(CheckCtx(c));
    RC_TRY(ValidateLayers(d, m, h_vec, kMaxK));
    if (!C_all) return Fail(STLQ_MI355_ERR_INVALID, "C_all is null");
    c->has_pre = false;
    c->d = d;
    c->m = m;
    int o = 0;
    for (int l = 0; l < m; ++l) {
        c->h_vec[l] = h_vec[l];
        c->off[l] = o;
        o += h_vec[l];
    }
    c->H = o;
    const size_t H = static_cast<size_t>(c->H);
    HIP_TRY(c->C_all.Ensure(H * d * 4));
    HIP_TRY(c->G_rm.Ensure(H * H * 4));
    HIP_TRY(c->gdiag.Ensure(H * 4));
    HIP_TRY(c->invnorm.Ensure(H * 4));
    HIP_TRY(hipMemcpyAsync(c->C_all.p, C_all, H * d * 4, hipMemcpyHostToDevice, c->stream));
    return STLQ_MI355_OK;
}

int stlq_mi355_set_codebooks(stlq_mi355_ctx* c, int d, int m, const int* h_vec, const float* C_all) {
    RC_TRY(SetPrecompCommon(c, d, m, h_vec, C_all));
    if (!c->g_shared) c->G_cm.Release();
    c->g_shared = true;
    c->G_cm.p = c->G_rm.p;
    c->G_cm.bytes = 0;  // alias, never freed through G_cm
    HIP_TRY(LaunchGram(c->C_all.as<float>(), d, c->H, c->G_rm.as<float>(), c->stream));
    HIP_TRY(LaunchNorms(c->C_all.as<float>(), d, c->H, false, nullptr, c->invnorm.as<float>(), c->stream));
    HIP_TRY(LaunchDiag(c->G_rm.as<float>(), c->H, c->gdiag.as<float>(), c->stream));
    RC_TRY(SetPruneFull(c));
    c->has_pre = true;
    return STLQ_MI355_OK;
}

int stlq_mi355_set_precomp(stlq_mi355_ctx* c, int d, int m, const int* h_vec, const float* C_all,
                           const float* G, const float* invnorm) {
    if (!G || !invnorm) return Fail(STLQ_MI355_ERR_INVALID, "G and invnorm are required");
    RC_TRY(SetPrecompCommon(c, d, m, h_vec, C_all));
    const size_t H = static_cast<size_t>(c->H);
    if (c->g_shared) c->G_cm.p = nullptr;
    c->g_shared = false;
    c->G_cm.bytes = 0;
    HIP_TRY(c->G_cm.Ensure(H * H * 4));
    HIP_TRY(hipMemcpyAsync(c->G_cm.p, G, H * H * 4, hipMemcpyHostToDevice, c->stream));
    // Row-major copy of the reference element G(row, col) = G[col*H + row].
    HIP_TRY(LaunchTranspose(c->G_cm.as<float>(), c->H, c->H, c->G_rm.as<float>(), c->stream));
    HIP_TRY(hipMemcpyAsync(c->invnorm.p, invnorm, H * 4, hipMemcpyHostToDevice, c->stream));
    HIP_TRY(LaunchDiag(c->G_rm.as<float>(), c->H, c->gdiag.as<float>(), c->stream));
    RC_TRY(SetPruneFull(c));
    c->has_pre = true;
    return STLQ_MI355_OK;
}

int stlq_mi355_get_precomp(stlq_mi355_ctx* c, float* G, float* invnorm) {
    RC_TRY(CheckPre(c));
    const size_t H = static_cast<size_t>(c->H);
    if (G) HIP_TRY(hipMemcpyAsync(G, c->G_cm.p, H * H * 4, hipMemcpyDeviceToHost, c->stream));
    if (invnorm) HIP_TRY(hipMemcpyAsync(invnorm, c->invnorm.p, H * 4, hipMemcpyDeviceToHost, c->stream));
    HIP_TRY(hipStreamSynchronize(c->stream));
    return STLQ_MI355_OK;
}

int stlq_mi355_xnorm2(stlq_mi355_ctx* c, const float* X, int d, int64_t n, float* out) {
    RC_TRY(CheckCtx(c));
    if (d < 1 || n < 0 || (n > 0 && (!X || !out))) return Fail(STLQ_MI355_ERR_INVALID, "bad arguments");
    if (n == 0) return STLQ_MI355_OK;
    HIP_TRY(c->X.Ensure(static_cast<size_t>(n) * d * 4));
    HIP_TRY(c->nx2.Ensure(static_cast<size_t>(n) * 4));
    HIP_TRY(hipMemcpyAsync(c->X.p, X, static_cast<size_t>(n) * d * 4, hipMemcpyHostToDevice, c->stream));
    HIP_TRY(LaunchXNorm2(c->X.as<float>(), d, n, c->nx2.as<float>(), c->stream));
    HIP_TRY(hipMemcpyAsync(out, c->nx2.p, static_cast<size_t>(n) * 4, hipMemcpyDeviceToHost, c->stream));
    HIP_TRY(hipStreamSynchronize(c->stream));
    return STLQ_MI355_OK;
}

int stlq_mi355_gemm_xc(stlq_mi355_ctx* c, const float* X, int64_t n, float* xC) {
    RC_TRY(CheckPre(c));
    if (n < 0 || (n > 0 && (!X || !xC))) return Fail(STLQ_MI355_ERR_INVALID, "bad arguments");
    if (n == 0) return STLQ_MI355_OK;
    HIP_TRY(c->X.Ensure(static_cast<size_t>(n) * c->d * 4));
    HIP_TRY(c->xC.Ensure(static_cast<size_t>(n) * c->H * 4));
    HIP_TRY(hipMemcpyAsync(c->X.p, X, static_cast<size_t>(n) * c->d * 4, hipMemcpyHostToDevice, c->stream));
    HIP_TRY(LaunchGemmXc(c->X.as<float>(), n, c->d, c->C_all.as<float>(), c->H, c->xC.as<float>(), c->H, c->stream));
    HIP_TRY(hipMemcpyAsync(xC, c->xC.p, static_cast<size_t>(n) * c->H * 4, hipMemcpyDeviceToHost, c->stream));
    HIP_TRY(hipStreamSynchronize(c->stream));
    return STLQ_MI355_OK;
}

int stlq_mi355_beam_search(stlq_mi355_ctx* c, const float* X, const float* nx2, const float* xC, int64_t n,
                           int H_beam, uint8_t* codes, float* best_err) {
    RC_TRY(CheckPre(c));
    const int Hb = std::max(1, H_beam);
    RC_TRY(CheckBeam(Hb));
    if (n < 0 || (n > 0 && (!xC || !codes || (!X && !nx2)))) return Fail(STLQ_MI355_ERR_INVALID, "bad arguments");
    if (n == 0) return STLQ_MI355_OK;
    c->ResetTimings();
    const int64_t tile = TileVectors(n, c->d, c->m, c->H, Hb);
    HIP_TRY(c->xC.Ensure(static_cast<size_t>(tile) * c->H * 4));
    HIP_TRY(c->nx2.Ensure(static_cast<size_t>(tile) * 4));
    HIP_TRY(c->codes.Ensure(static_cast<size_t>(tile) * c->m));
    HIP_TRY(c->best.Ensure(static_cast<size_t>(tile) * 4));
    if (!nx2) HIP_TRY(c->X.Ensure(static_cast<size_t>(tile) * c->d * 4));
    for (int64_t t0 = 0; t0 < n; t0 += tile) {
        const int64_t nt = std::min(tile, n - t0);
        HIP_TRY(hipMemcpyAsync(c->xC.p, xC + t0 * c->H, static_cast<size_t>(nt) * c->H * 4, hipMemcpyHostToDevice,
                               c->stream));
        if (nx2) {
            HIP_TRY(hipMemcpyAsync(c->nx2.p, nx2 + t0, static_cast<size_t>(nt) * 4, hipMemcpyHostToDevice, c->stream));
        } else {
            HIP_TRY(hipMemcpyAsync(c->X.p, X + t0 * c->d, static_cast<size_t>(nt) * c->d * 4, hipMemcpyHostToDevice,
                                   c->stream));
            HIP_TRY(LaunchXNorm2(c->X.as<float>(), c->d, nt, c->nx2.as<float>(), c->stream));
        }
        TileEvents te;
        te.n = nt;
        te.e[0] = te.e[1] = te.e[2] = c->NextEvent();
        HIP_TRY(hipEventRecord(te.e[0], c->stream));
        RC_TRY(RunBeam(c, c->xC.as<float>(), c->H, c->nx2.as<float>(), nt, Hb, c->codes.as<uint8_t>(),
                       c->best.as<float>(), c->stream, &te.beam_launches, &te));
        te.e[3] = te.e[4] = te.e[5] = te.e[6] = c->NextEvent();
        HIP_TRY(hipEventRecord(te.e[3], c->stream));
        c->tiles.push_back(te);
        HIP_TRY(hipMemcpyAsync(codes + t0 * c->m, c->codes.p, static_cast<size_t>(nt) * c->m, hipMemcpyDeviceToHost,
                               c->stream));
        if (best_err)
            HIP_TRY(hipMemcpyAsync(best_err + t0, c->best.p, static_cast<size_t>(nt) * 4, hipMemcpyDeviceToHost,
                                   c->stream));
        HIP_TRY(hipStreamSynchronize(c->stream));
    }
    return STLQ_MI355_OK;
}

// Host-side check that caller-supplied codes index their layer's codebook (the kernels gather
// G rows by code; an out-of-range code would read outside G).
static int CheckCodes(const stlq_mi355_ctx* c, const uint8_t* codes, int64_t n) {
    for (int64_t i = 0; i < n; ++i) {
        const uint8_t* ci = codes + i * c->m;
        for (int l = 0; l < c->m; ++l) {
            if (ci[l] >= c->h_vec[l])
                return Fail(STLQ_MI355_ERR_INVALID, "code " + std::to_string(ci[l]) + " of vector " + std::to_string(i) +
                                                        " exceeds layer " + std::to_string(l) + " size " +
                                                        std::to_string(c->h_vec[l]));
        }
    }
    return STLQ_MI355_OK;
}

static int LsCommon(stlq_mi355_ctx* c, const float* xC, const uint8_t* codes, const float* a_in, const float* nx2,
                    int64_t n, float* a_out, float* cost_out, int64_t* fail_count) {
    RC_TRY(CheckPre(c));
    if (n < 0 || (n > 0 && (!xC || !codes))) return Fail(STLQ_MI355_ERR_INVALID, "bad arguments");
    RC_TRY(CheckCodes(c, codes, n));
    if (fail_count) *fail_count = 0;
    if (n == 0) return STLQ_MI355_OK;
    const size_t m = static_cast<size_t>(c->m);
    HIP_TRY(c->xC.Ensure(static_cast<size_t>(n) * c->H * 4));
    HIP_TRY(c->codes.Ensure(static_cast<size_t>(n) * m));
    HIP_TRY(c->a.Ensure(static_cast<size_t>(n) * m * 4));
    HIP_TRY(c->nx2.Ensure(static_cast<size_t>(n) * 4));
    HIP_TRY(c->cost.Ensure(static_cast<size_t>(n) * 4));
    HIP_TRY(hipMemcpyAsync(c->xC.p, xC, static_cast<size_t>(n) * c->H * 4, hipMemcpyHostToDevice, c->stream));
    HIP_TRY(hipMemcpyAsync(c->codes.p, codes, static_cast<size_t>(n) * m, hipMemcpyHostToDevice, c->stream));
    HIP_TRY(LaunchFill8(c->fails.as<uint8_t>(), 0, 4, c->stream));  // a kernel, not a memset node, if captured
    LsArgs ls = MakeLs(c, c->xC.as<float>(), c->H, c->codes.as<uint8_t>(), c->a.as<float>(), c->nx2.as<float>(),
                       c->cost.as<float>(), n);
    if (a_out) {
        HIP_TRY(LaunchLsAll(ls, c->stream));
        HIP_TRY(hipMemcpyAsync(a_out, c->a.p, static_cast<size_t>(n) * m * 4, hipMemcpyDeviceToHost, c->stream));
    }
    if (cost_out) {
        HIP_TRY(hipMemcpyAsync(c->a.p, a_in, static_cast<size_t>(n) * m * 4, hipMemcpyHostToDevice, c->stream));
        HIP_TRY(hipMemcpyAsync(c->nx2.p, nx2, static_cast<size_t>(n) * 4, hipMemcpyHostToDevice, c->stream));
        HIP_TRY(LaunchCosts(ls, c->stream));
        HIP_TRY(hipMemcpyAsync(cost_out, c->cost.p, static_cast<size_t>(n) * 4, hipMemcpyDeviceToHost, c->stream));
    }
    int fails = 0;
    HIP_TRY(hipMemcpyAsync(&fails, c->fails.p, 4, hipMemcpyDeviceToHost, c->stream));
    HIP_TRY(hipStreamSynchronize(c->stream));
    if (fail_count) *fail_count = fails;
    return STLQ_MI355_OK;
}

int stlq_mi355_solve_ls_all(stlq_mi355_ctx* c, const float* xC, const uint8_t* codes, int64_t n, float* a,
                            int64_t* fail_count) {
    if (n > 0 && !a) return Fail(STLQ_MI355_ERR_INVALID, "a is null");
    return LsCommon(c, xC, codes, nullptr, nullptr, n, a, nullptr, fail_count);
}

int stlq_mi355_compute_costs(stlq_mi355_ctx* c, const float* xC, const uint8_t* codes, const float* a,
                             const float* nx2, int64_t n, float* cost) {
    if (n > 0 && (!a || !nx2 || !cost)) return Fail(STLQ_MI355_ERR_INVALID, "bad arguments");
    return LsCommon(c, xC, codes, a, nx2, n, nullptr, cost, nullptr);
}

int stlq_mi355_icm(stlq_mi355_ctx* c, const float* X, const float* nx2, const float* xC, int64_t n, int icm_iters,
                   int use_abs, uint32_t seed, uint8_t* codes, float* a, float* cost) {
    RC_TRY(CheckPre(c));
    if (n < 0 || (n > 0 && (!xC || !codes || !a || !cost || (!X && !nx2))))
        return Fail(STLQ_MI355_ERR_INVALID, "bad arguments");
    if (icm_iters < 0) return Fail(STLQ_MI355_ERR_INVALID, "icm_iters must be >= 0");
    if (n == 0) return STLQ_MI355_OK;
    RC_TRY(CheckCodes(c, codes, n));
    c->ResetTimings();
    const size_t m = static_cast<size_t>(c->m);
    HIP_TRY(c->xC.Ensure(static_cast<size_t>(n) * c->H * 4));
    HIP_TRY(c->codes.Ensure(static_cast<size_t>(n) * m));
    HIP_TRY(c->a.Ensure(static_cast<size_t>(n) * m * 4));
    HIP_TRY(c->nx2.Ensure(static_cast<size_t>(n) * 4));
    HIP_TRY(c->cost.Ensure(static_cast<size_t>(n) * 4));
    HIP_TRY(hipMemcpyAsync(c->xC.p, xC, static_cast<size_t>(n) * c->H * 4, hipMemcpyHostToDevice, c->stream));
    HIP_TRY(hipMemcpyAsync(c->codes.p, codes, static_cast<size_t>(n) * m, hipMemcpyHostToDevice, c->stream));
    if (nx2) {
        HIP_TRY(hipMemcpyAsync(c->nx2.p, nx2, static_cast<size_t>(n) * 4, hipMemcpyHostToDevice, c->stream));
    } else {
        HIP_TRY(c->X.Ensure(static_cast<size_t>(n) * c->d * 4));
        HIP_TRY(hipMemcpyAsync(c->X.p, X, static_cast<size_t>(n) * c->d * 4, hipMemcpyHostToDevice, c->stream));
        HIP_TRY(LaunchXNorm2(c->X.as<float>(), c->d, n, c->nx2.as<float>(), c->stream));
    }
    HIP_TRY(LaunchFill8(c->fails.as<uint8_t>(), 0, 4, c->stream));  // a kernel, not a memset node, if captured
    TileEvents te;
    te.n = n;
    te.e[0] = te.e[1] = te.e[2] = te.e[3] = te.e[4] = c->NextEvent();
    HIP_TRY(hipEventRecord(te.e[0], c->stream));
    RC_TRY(RunIcm(c, FullProblem(c, c->xC.as<float>(), c->H, c->nx2.as<float>(), n), icm_iters, use_abs, seed,
                  c->codes.as<uint8_t>(), c->a.as<float>(), c->cost.as<float>(), c->stream));
    te.e[5] = te.e[6] = c->NextEvent();
    HIP_TRY(hipEventRecord(te.e[5], c->stream));
    c->tiles.push_back(te);
    HIP_TRY(hipMemcpyAsync(codes, c->codes.p, static_cast<size_t>(n) * m, hipMemcpyDeviceToHost, c->stream));
    HIP_TRY(hipMemcpyAsync(a, c->a.p, static_cast<size_t>(n) * m * 4, hipMemcpyDeviceToHost, c->stream));
    HIP_TRY(hipMemcpyAsync(cost, c->cost.p, static_cast<size_t>(n) * 4, hipMemcpyDeviceToHost, c->stream));
    HIP_TRY(hipStreamSynchronize(c->stream));
    return STLQ_MI355_OK;
}

int stlq_mi355_icm_ils(stlq_mi355_ctx* c, const float* X, const float* nx2, const float* xC, int64_t n,
                       int icm_iters, int ils_iters, int perturb_k, int use_abs, uint32_t seed,
                       uint64_t sample_id_offset, uint8_t* codes, float* a, float* cost) {
    RC_TRY(CheckPre(c));
    if (n < 0 || (n > 0 && (!xC || !codes || !a || !cost || (!X && !nx2))))
        return Fail(STLQ_MI355_ERR_INVALID, "bad arguments");
    if (icm_iters < 0 || ils_iters < 0 || perturb_k < 0)
        return Fail(STLQ_MI355_ERR_INVALID, "icm_iters, ils_iters and perturb_k must be >= 0");
    if (n == 0) return STLQ_MI355_OK;
    RC_TRY(CheckCodes(c, codes, n));
    c->ResetTimings();
    const size_t m = static_cast<size_t>(c->m);
    HIP_TRY(c->xC.Ensure(static_cast<size_t>(n) * c->H * 4));
    HIP_TRY(c->codes.Ensure(static_cast<size_t>(n) * m));
    HIP_TRY(c->a.Ensure(static_cast<size_t>(n) * m * 4));
    HIP_TRY(c->nx2.Ensure(static_cast<size_t>(n) * 4));
    HIP_TRY(c->cost.Ensure(static_cast<size_t>(n) * 4));
    HIP_TRY(hipMemcpyAsync(c->xC.p, xC, static_cast<size_t>(n) * c->H * 4, hipMemcpyHostToDevice, c->stream));
    HIP_TRY(hipMemcpyAsync(c->codes.p, codes, static_cast<size_t>(n) * m, hipMemcpyHostToDevice, c->stream));
    if (nx2) {
        HIP_TRY(hipMemcpyAsync(c->nx2.p, nx2, static_cast<size_t>(n) * 4, hipMemcpyHostToDevice, c->stream));
    } else {
        HIP_TRY(c->X.Ensure(static_cast<size_t>(n) * c->d * 4));
        HIP_TRY(hipMemcpyAsync(c->X.p, X, static_cast<size_t>(n) * c->d * 4, hipMemcpyHostToDevice, c->stream));
        HIP_TRY(LaunchXNorm2(c->X.as<float>(), c->d, n, c->nx2.as<float>(), c->stream));
    }
    HIP_TRY(LaunchFill8(c->fails.as<uint8_t>(), 0, 4, c->stream));  // a kernel, not a memset node, if captured
    TileEvents te;
    te.n = n;
    te.e[0] = te.e[1] = te.e[2] = te.e[3] = te.e[4] = c->NextEvent();
    HIP_TRY(hipEventRecord(te.e[0], c->stream));
    RC_TRY(RunIcmIls(c, FullProblem(c, c->xC.as<float>(), c->H, c->nx2.as<float>(), n), icm_iters, ils_iters,
                     perturb_k, use_abs,
                     seed, sample_id_offset, c->codes.as<uint8_t>(), c->a.as<float>(), c->cost.as<float>(),
                     c->stream));
    te.e[5] = te.e[6] = c->NextEvent();
    HIP_TRY(hipEventRecord(te.e[5], c->stream));
    c->tiles.push_back(te);
    HIP_TRY(hipMemcpyAsync(codes, c->codes.p, static_cast<size_t>(n) * m, hipMemcpyDeviceToHost, c->stream));
    HIP_TRY(hipMemcpyAsync(a, c->a.p, static_cast<size_t>(n) * m * 4, hipMemcpyDeviceToHost, c->stream));
    HIP_TRY(hipMemcpyAsync(cost, c->cost.p, static_cast<size_t>(n) * 4, hipMemcpyDeviceToHost, c->stream));
    HIP_TRY(hipStreamSynchronize(c->stream));
    return STLQ_MI355_OK;
}

int stlq_mi355_encode(stlq_mi355_ctx* c, const float* X, int64_t n, const stlq_mi355_encode_params* params,
                      uint8_t* codes, float* a, float* cost, double* beam_mse, double* final_mse) {
    RC_TRY(CheckPre(c));
    RC_TRY(CheckParams(params));
    if (n < 0 || (n > 0 && (!X || !codes))) return Fail(STLQ_MI355_ERR_INVALID, "bad arguments");
    if (n == 0) return STLQ_MI355_OK;
    c->ResetTimings();
    stlq_mi355_encode_params P = *params;
    const bool want_mse = beam_mse || final_mse;
    const bool need_ls = P.want_coeffs || P.icm_iters > 0 || P.ils_iters > 0 || want_mse;
    const int Hb = std::max(1, P.H_beam);
    const size_t m = static_cast<size_t>(c->m);
    const int64_t tile = TileVectors(n, c->d, c->m, c->H, Hb);
    HIP_TRY(c->X.Ensure(static_cast<size_t>(tile) * c->d * 4));
    HIP_TRY(c->codes.Ensure(static_cast<size_t>(tile) * m));
    HIP_TRY(c->a.Ensure(static_cast<size_t>(tile) * m * 4));
    HIP_TRY(c->cost.Ensure(static_cast<size_t>(tile) * 4));
    HIP_TRY(LaunchFill8(c->fails.as<uint8_t>(), 0, 4, c->stream));  // a kernel, not a memset node, if captured
    std::vector<float> beam_cost, fin_cost;
    double beam_sum = 0.0, fin_sum = 0.0;
    for (int64_t t0 = 0; t0 < n; t0 += tile) {
        const int64_t nt = std::min(tile, n - t0);
        HIP_TRY(hipMemcpyAsync(c->X.p, X + t0 * c->d, static_cast<size_t>(nt) * c->d * 4, hipMemcpyHostToDevice,
                               c->stream));
        EncodeOut o{c->codes.as<uint8_t>(), c->a.as<float>(), c->cost.as<float>(), nullptr};
        stlq_mi355_encode_params Pt = P;
        Pt.want_coeffs = need_ls ? 1 : 0;
        if (want_mse && (P.icm_iters > 0 || P.ils_iters > 0)) {
            // Beam MSE before ICM/ILS: run the beam + LS alone first, then ICM/ILS on the same codes.
            Pt.icm_iters = 0;
            Pt.ils_iters = 0;
            RC_TRY(EncodeTile(c, c->X.as<float>(), nt, Pt, o, c->stream, true, /*allow_overlap=*/false,
                              static_cast<uint64_t>(t0)));
            beam_cost.resize(static_cast<size_t>(nt));
            HIP_TRY(hipMemcpyAsync(beam_cost.data(), c->cost.p, static_cast<size_t>(nt) * 4, hipMemcpyDeviceToHost,
                                   c->stream));
            HIP_TRY(hipStreamSynchronize(c->stream));
            beam_sum += Mean(beam_cost) * static_cast<double>(nt);
            RC_TRY(RunIcmIls(c, FullProblem(c, c->xC.as<float>(), c->H, c->nx2.as<float>(), nt), P.icm_iters,
                             P.ils_iters,
                             P.perturb_k, P.use_abs, P.seed, static_cast<uint64_t>(t0), o.codes, o.a, o.cost,
                             c->stream));
        } else {
            RC_TRY(EncodeTile(c, c->X.as<float>(), nt, Pt, o, c->stream, true, true, static_cast<uint64_t>(t0)));
        }
        HIP_TRY(hipMemcpyAsync(codes + t0 * m, c->codes.p, static_cast<size_t>(nt) * m, hipMemcpyDeviceToHost,
                               c->stream));
        if (a && need_ls)
            HIP_TRY(hipMemcpyAsync(a + t0 * m, c->a.p, static_cast<size_t>(nt) * m * 4, hipMemcpyDeviceToHost,
                                   c->stream));
        if (need_ls) {
            fin_cost.resize(static_cast<size_t>(nt));
            HIP_TRY(hipMemcpyAsync(fin_cost.data(), c->cost.p, static_cast<size_t>(nt) * 4, hipMemcpyDeviceToHost,
                                   c->stream));
        }
        HIP_TRY(hipStreamSynchronize(c->stream));
        if (need_ls) {
            if (cost) std::memcpy(cost + t0, fin_cost.data(), static_cast<size_t>(nt) * 4);
            fin_sum += Mean(fin_cost) * static_cast<double>(nt);
            if (P.icm_iters == 0) beam_sum += Mean(fin_cost) * static_cast<double>(nt);
        }
    }
    if (beam_mse) *beam_mse = beam_sum / static_cast<double>(n);
    if (final_mse) *final_mse = fin_sum / static_cast<double>(n);
    return STLQ_MI355_OK;
}

int stlq_mi355_encode_device(stlq_mi355_ctx* c, const float* dX, int64_t n, const stlq_mi355_encode_params* params,
                             uint8_t* dcodes, float* da, float* dcost, void* stream) {
    RC_TRY(CheckPre(c));
    RC_TRY(CheckParams(params));
    if (n < 0 || (n > 0 && (!dX || !dcodes))) return Fail(STLQ_MI355_ERR_INVALID, "bad arguments");
    if (n == 0) return STLQ_MI355_OK;
    c->ResetTimings();
    hipStream_t s = stream ? static_cast<hipStream_t>(stream) : c->stream;
    const int Hb = std::max(1, params->H_beam);
    const int64_t tile = TileVectors(n, c->d, c->m, c->H, Hb);
    const size_t m = static_cast<size_t>(c->m);
    HIP_TRY(LaunchFill8(c->fails.as<uint8_t>(), 0, 4, s));  // a kernel, not a memset node, if captured
    for (int64_t t0 = 0; t0 < n; t0 += tile) {
        const int64_t nt = std::min(tile, n - t0);
        EncodeOut o{dcodes + t0 * m, da ? da + t0 * m : nullptr, dcost ? dcost + t0 : nullptr, nullptr};
        RC_TRY(EncodeTile(c, dX + t0 * c->d, nt, *params, o, s, true, true, static_cast<uint64_t>(t0)));
    }
    return STLQ_MI355_OK;
}

}  // extern "C"

namespace {

// The work buffers one full-precomp encode tile of n vectors asks for (EncodeTile without the
// sub-tile overlap, BeamAndRefit, RunBeam, RunIcmIls), with their sizes: the no-allocation entry
// point lends each of them a 256-byte-aligned range of the static scratch.
constexpr int kMaxLease = 24;
struct LeaseItem {
    DevBuf* buf;
    size_t bytes;
};

int NoAllocPlan(stlq_mi355_ctx* c, int64_t n, const stlq_mi355_encode_params& P, bool has_a, bool has_cost,
                LeaseItem (&items)[kMaxLease], int* count, size_t* total) {
    const size_t N = static_cast<size_t>(n), m = static_cast<size_t>(c->m), H = static_cast<size_t>(c->H);
    const size_t Hb = static_cast<size_t>(std::max(1, P.H_beam));
    const size_t rec = N * Hb * 4 * static_cast<size_t>(BeamRecordStride(c->m));
    const bool refine = P.icm_iters > 0 || P.ils_iters > 0;
    const bool need_ls = P.want_coeffs || refine;
    int k = 0;
    auto add = [&](DevBuf& b, size_t bytes) { items[k++] = LeaseItem{&b, std::max<size_t>(bytes, 1)}; };
    add(c->nx2, N * 4);
    add(c->xC, N * H * 4);
    for (int b = 0; b < 2; ++b) {
        add(c->st_rec[b], rec);
        add(c->st_curH[b], N * 4);
    }
    add(c->bf_flags, N);
    add(c->bf_list, N * 4);
    add(c->bf_count, 8);
    add(c->fails, 4);
    if (need_ls && !has_a) add(c->a, N * m * 4);
    if (need_ls && !has_cost) add(c->cost, N * 4);
    if (P.icm_iters > 0) {
        add(c->active, N);
        add(c->changed, N);
        add(c->icm_pend, N * 4);
    }
    if (P.ils_iters > 0 && P.perturb_k > 0 && c->m > 1) {
        add(c->ils_codes, N * m);
        add(c->ils_a, N * m * 4);
        add(c->ils_cost, N * 4);
    }
    size_t t = 0;
    for (int i = 0; i < k; ++i) t += (items[i].bytes + 255) & ~size_t{255};
    *count = k;
    *total = t;
    return STLQ_MI355_OK;
}

// Lends the planned ranges of the scratch to the context's buffers for one call and gives the
// context its own buffers back afterwards.
class ScratchLease {
   public:
    ScratchLease(stlq_mi355_ctx* c, const LeaseItem* items, int count) : c_(c), count_(count) {
        char* base = static_cast<char*>(c->scratch);
        size_t off = 0;
        for (int i = 0; i < count; ++i) {
            saved_[i] = *items[i].buf;
            bufs_[i] = items[i].buf;
            DevBuf lent;
            lent.p = base + off;
            lent.bytes = items[i].bytes;
            lent.borrowed = true;
            *items[i].buf = lent;
            off += (items[i].bytes + 255) & ~size_t{255};
        }
        c->noalloc = true;
    }
    ~ScratchLease() {
        for (int i = 0; i < count_; ++i) *bufs_[i] = saved_[i];
        c_->noalloc = false;
    }

   private:
    stlq_mi355_ctx* c_;
    int count_;
    DevBuf* bufs_[kMaxLease] = {};
    DevBuf saved_[kMaxLease];
};

}  // namespace

extern "C" {

int stlq_mi355_encode_device_noalloc(stlq_mi355_ctx* c, const float* dX, int64_t n,
                                     const stlq_mi355_encode_params* params, uint8_t* dcodes, float* da,
                                     float* dcost, void* stream) {
    RC_TRY(CheckPre(c));
    RC_TRY(CheckParams(params));
    if (n < 0 || (n > 0 && (!dX || !dcodes))) return Fail(STLQ_MI355_ERR_INVALID, "bad arguments");
    if (!c->scratch) return Fail(STLQ_MI355_ERR_STATE, "no-allocation scratch unavailable on this device");
    if (n == 0) return STLQ_MI355_OK;
    LeaseItem items[kMaxLease];
    int count = 0;
    size_t total = 0;
    RC_TRY(NoAllocPlan(c, n, *params, da != nullptr, dcost != nullptr, items, &count, &total));
    if (total > kScratchBytes) {
        // capacity for this shape: the largest tile whose plan fits the scratch
        int64_t lo = 0, hi = n;
        while (lo < hi) {
            const int64_t mid = lo + (hi - lo + 1) / 2;
            LeaseItem tmp[kMaxLease];
            int cnt = 0;
            size_t tot = 0;
            RC_TRY(NoAllocPlan(c, mid, *params, da != nullptr, dcost != nullptr, tmp, &cnt, &tot));
            if (tot <= kScratchBytes) lo = mid;
            else hi = mid - 1;
        }
        return Fail(STLQ_MI355_ERR_UNSUPPORTED,
                    "n = " + std::to_string(n) + " exceeds the no-allocation capacity of " + std::to_string(lo) +
                        " vectors for this shape (" + std::to_string(kScratchBytes >> 20) + " MiB device scratch); "
                        "use stlq_mi355_encode_device or smaller batches");
    }
    c->ResetTimings();
    hipStream_t s = stream ? static_cast<hipStream_t>(stream) : c->stream;
    ScratchLease lease(c, items, count);
    HIP_TRY(LaunchFill8(c->fails.as<uint8_t>(), 0, 4, s));  // the scratch keeps the previous call's bytes
    EncodeOut o{dcodes, da, dcost, nullptr};
    return EncodeTile(c, dX, n, *params, o, s, /*record=*/false, /*allow_overlap=*/false, 0);
}

int stlq_mi355_last_timings(stlq_mi355_ctx* c, stlq_mi355_timings* out) {
    RC_TRY(CheckCtx(c));
    if (!out) return Fail(STLQ_MI355_ERR_INVALID, "out is null");
    std::memset(out, 0, sizeof(*out));
    for (const TileEvents& te : c->tiles) {
        if (!te.e[0] || !te.e[6]) continue;
        HIP_TRY(hipEventSynchronize(te.e[6]));
        float ms[6] = {};
        for (int k = 0; k < 6; ++k) {
            if (te.e[k] && te.e[k + 1] && te.e[k] != te.e[k + 1]) HIP_TRY(hipEventElapsedTime(&ms[k], te.e[k], te.e[k + 1]));
        }
        if (te.gemm_end) HIP_TRY(hipEventElapsedTime(&ms[1], te.e[1], te.gemm_end));
        float tot = 0.0f;
        HIP_TRY(hipEventElapsedTime(&tot, te.e[0], te.e[6]));
        out->xnorm_ms += ms[0];
        out->gemm_ms += ms[1];
        out->beam_ms += ms[2];
        out->ls_ms += ms[3];
        out->icm_ms += ms[4];
        out->total_ms += tot;
        out->n += te.n;
        out->gemm_launches += te.gemm_launches;
        out->beam_launches += te.beam_launches;
        for (int l = 0; l < te.layers && l < kMaxM; ++l) {
            float lm = 0.0f;
            HIP_TRY(hipEventElapsedTime(&lm, te.lay[l], te.lay[l + 1]));
            out->layer_ms[l] += lm;
        }
    }
    if (c->bf_used && c->bf_host && !c->tiles.empty()) out->beam_reruns = c->bf_host[1];  // tiles synchronized above
    if (c->overlapped && !c->tiles.empty()) {
        float env = 0.0f;
        HIP_TRY(hipEventElapsedTime(&env, c->tiles.front().e[0], c->tiles.back().e[6]));
        out->total_ms = env;
    }
    return STLQ_MI355_OK;
}

}  // extern "C"

namespace {
int CheckLargeRoot(stlq_mi355_ctx* c, int H_beam, int root_mode);
int64_t LargeRootTileVectors(stlq_mi355_ctx* c, int64_t n, int Hb, bool one_score);
int LargeRootTile(stlq_mi355_ctx* c, const float* dX, int64_t nt, int Hb, int root_mode, const uint32_t* d_forced,
                  const float* dxC_given, uint32_t* d_cluster, uint8_t* d_codes, float* d_best, hipStream_t s,
                  TileEvents* te, const stlq_mi355_encode_params* refine = nullptr, float* d_a = nullptr,
                  float* d_cost = nullptr, uint64_t id0 = 0);
}  // namespace

extern "C" {

// ---------------------------------------------------------------------------------------------
// Streaming encode: pinned host chunks -> two device buffers on the copy stream, encode on the
// context stream, pinned outputs handed to the sink in chunk order.
int stlq_mi355_encode_stream(stlq_mi355_ctx* c, int64_t n_total, int64_t chunk, const stlq_mi355_stream_params* sp,
                             stlq_mi355_fill_fn fill, stlq_mi355_sink_fn sink, void* user,
                             stlq_mi355_stream_stats* stats) {
    RC_TRY(CheckCtx(c));
    if (!sp) return Fail(STLQ_MI355_ERR_INVALID, "params is null");
    const bool lr = sp->large_root != 0;
    if (lr) {
        RC_TRY(CheckLargeRoot(c, sp->encode.H_beam, sp->root_mode));
        RC_TRY(CheckParams(&sp->encode));
    } else {
        RC_TRY(CheckPre(c));
        RC_TRY(CheckParams(&sp->encode));
    }
    if (n_total < 0 || chunk <= 0 || !fill || !sink) return Fail(STLQ_MI355_ERR_INVALID, "bad arguments");
    const uint64_t gid0 = sp->start_id;  // global id of the stream's first vector
    if (gid0 > static_cast<uint64_t>(INT64_MAX) - static_cast<uint64_t>(n_total))
        return Fail(STLQ_MI355_ERR_INVALID, "start_id + n_total overflows");
    if (stats) std::memset(stats, 0, sizeof(*stats));
    if (n_total == 0) return STLQ_MI355_OK;
    c->ResetTimings();
    const auto t_begin = std::chrono::steady_clock::now();
    const int Hb = std::max(1, sp->encode.H_beam);
    const size_t m = static_cast<size_t>(lr ? c->lr_m : c->m);
    const size_t d = static_cast<size_t>(lr ? c->lr_d : c->d);
    const size_t esz = sp->input_u8 ? 1 : 4;
    if (sp->R) RC_TRY(UploadRotation(c, sp->R, static_cast<int>(d), c->stream));
    chunk = std::min(chunk, n_total);
    const size_t ch = static_cast<size_t>(chunk);
    const bool want = sp->encode.want_coeffs || sp->encode.icm_iters > 0 || sp->encode.ils_iters > 0;
    const size_t code_b = lr ? std::max<size_t>(m - 1, 1) : m;
    struct Slot {
        void* hin = nullptr;
        uint8_t* hcodes = nullptr;
        float* ha = nullptr;
        float* hcost = nullptr;
        uint32_t* hcluster = nullptr;
        float* hbest = nullptr;
        DevBuf din, dX, dXr, dcodes, da, dcost, dcluster, dbest;
        hipEvent_t copied = nullptr, done = nullptr, c0 = nullptr, c1 = nullptr, k0 = nullptr;
        int64_t first = 0, count = 0;
        bool busy = false;
    } slot[2];
    int rc = STLQ_MI355_OK;
    auto hip_ok = [&](hipError_t e, const char* what) {
        if (e == hipSuccess) return true;
        rc = Fail(STLQ_MI355_ERR_HIP, std::string(what) + ": " + hipGetErrorString(e));
        return false;
    };
    auto cleanup = [&]() {
        (void)hipStreamSynchronize(c->copy_stream);
        (void)hipStreamSynchronize(c->stream);
        for (Slot& sl : slot) {
            for (void* p : {sl.hin, static_cast<void*>(sl.hcodes), static_cast<void*>(sl.ha), static_cast<void*>(sl.hcost),
                            static_cast<void*>(sl.hcluster), static_cast<void*>(sl.hbest)})
                if (p) (void)hipHostFree(p);
            for (DevBuf* b : {&sl.din, &sl.dX, &sl.dXr, &sl.dcodes, &sl.da, &sl.dcost, &sl.dcluster, &sl.dbest})
                b->Release();
            for (hipEvent_t e : {sl.copied, sl.done, sl.c0, sl.c1, sl.k0})
                if (e) (void)hipEventDestroy(e);
        }
    };
    auto hmalloc = [&](void** p, size_t bytes) {
        return hip_ok(hipHostMalloc(p, std::max<size_t>(bytes, 16), hipHostMallocDefault), "hipHostMalloc");
    };
    for (Slot& sl : slot) {
        bool ok = hmalloc(&sl.hin, ch * d * esz) && hmalloc(reinterpret_cast<void**>(&sl.hcodes), ch * code_b) &&
                  hip_ok(sl.din.Ensure(ch * d * esz), "hipMalloc") && hip_ok(sl.dcodes.Ensure(ch * code_b), "hipMalloc");
        if (ok && sp->input_u8) ok = hip_ok(sl.dX.Ensure(ch * d * 4), "hipMalloc");
        if (ok && sp->R) ok = hip_ok(sl.dXr.Ensure(ch * d * 4), "hipMalloc");
        if (ok && want)
            ok = hmalloc(reinterpret_cast<void**>(&sl.ha), ch * m * 4) && hmalloc(reinterpret_cast<void**>(&sl.hcost), ch * 4) &&
                 hip_ok(sl.da.Ensure(ch * m * 4), "hipMalloc") && hip_ok(sl.dcost.Ensure(ch * 4), "hipMalloc");
        if (ok && lr)
            ok = hmalloc(reinterpret_cast<void**>(&sl.hcluster), ch * 4) && hmalloc(reinterpret_cast<void**>(&sl.hbest), ch * 4) &&
                 hip_ok(sl.dcluster.Ensure(ch * 4), "hipMalloc") && hip_ok(sl.dbest.Ensure(ch * 4), "hipMalloc");
        for (hipEvent_t* e : {&sl.copied, &sl.done, &sl.c0, &sl.c1, &sl.k0})
            if (ok) ok = hip_ok(hipEventCreate(e), "hipEventCreate");
        if (!ok) {
            cleanup();
            return rc;
        }
    }
    double fill_ms = 0.0, sink_ms = 0.0, h2d_ms = 0.0, comp_ms = 0.0, h2d_bytes = 0.0;
    int64_t nchunks = 0;
    auto drain = [&](Slot& sl) -> bool {
        if (!sl.busy) return true;
        if (!hip_ok(hipEventSynchronize(sl.done), "hipEventSynchronize")) return false;
        float ms = 0.0f;
        if (hip_ok(hipEventElapsedTime(&ms, sl.c0, sl.c1), "hipEventElapsedTime")) h2d_ms += ms;
        if (hip_ok(hipEventElapsedTime(&ms, sl.k0, sl.done), "hipEventElapsedTime")) comp_ms += ms;
        sl.busy = false;
        stlq_mi355_chunk_out out{};
        out.input = sl.hin;  // not refilled before the next fill, which follows this sink call
        if (lr) {
            out.cluster_id = sl.hcluster;
            out.B_small = m > 1 ? sl.hcodes : nullptr;
            out.best_err = sl.hbest;
            out.a = want ? sl.ha : nullptr;
            out.cost = want ? sl.hcost : nullptr;
        } else {
            out.codes = sl.hcodes;
            out.a = want ? sl.ha : nullptr;
            out.cost = want ? sl.hcost : nullptr;
        }
        const auto s0 = std::chrono::steady_clock::now();
        const int src = sink(user, static_cast<int64_t>(gid0) + sl.first, sl.count, &out);
        sink_ms += std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - s0).count();
        if (src != 0) {
            rc = Fail(STLQ_MI355_ERR_CALLBACK, "sink callback failed");
            return false;
        }
        return true;
    };
    int64_t ci = 0;
    for (int64_t first = 0; first < n_total; first += chunk, ++ci) {
        Slot& sl = slot[ci & 1];
        if (!drain(sl)) break;  // the slot's buffers are free once its previous chunk is done
        sl.first = first;
        sl.count = std::min(chunk, n_total - first);
        const size_t cnt = static_cast<size_t>(sl.count);
        const auto f0 = std::chrono::steady_clock::now();
        if (fill(user, static_cast<int64_t>(gid0) + sl.first, sl.count, sl.hin) != 0) {
            rc = Fail(STLQ_MI355_ERR_CALLBACK, "fill callback failed");
            break;
        }
        fill_ms += std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - f0).count();
        const size_t xb = cnt * d * esz;
        if (!hip_ok(hipEventRecord(sl.c0, c->copy_stream), "hipEventRecord") ||
            !hip_ok(hipMemcpyAsync(sl.din.p, sl.hin, xb, hipMemcpyHostToDevice, c->copy_stream), "hipMemcpyAsync") ||
            !hip_ok(hipEventRecord(sl.c1, c->copy_stream), "hipEventRecord") ||
            !hip_ok(hipEventRecord(sl.copied, c->copy_stream), "hipEventRecord") ||
            !hip_ok(hipStreamWaitEvent(c->stream, sl.copied, 0), "hipStreamWaitEvent") ||
            !hip_ok(hipEventRecord(sl.k0, c->stream), "hipEventRecord"))
            break;
        h2d_bytes += static_cast<double>(xb);
        const float* dX = sl.din.as<float>();
        if (sp->input_u8) {
            if (!hip_ok(LaunchU8ToF32(sl.din.as<uint8_t>(), sl.dX.as<float>(), cnt * d, c->stream), "U8ToF32")) break;
            dX = sl.dX.as<float>();
        }
        if (sp->R) {  // Xblk = R X (encode_base_streaming.cpp:817-833)
            if (!hip_ok(LaunchGemmXc(dX, sl.count, static_cast<int>(d), c->R_rm.as<float>(), static_cast<int>(d),
                                     sl.dXr.as<float>(), static_cast<int64_t>(d), c->stream), "rotation GEMM"))
                break;
            dX = sl.dXr.as<float>();
        }
        // Encode the chunk in workspace-bounded tiles (sequential on the context stream).
        const int64_t tile = lr ? LargeRootTileVectors(c, sl.count, Hb, sp->root_mode == 1)
                                : TileVectors(sl.count, c->d, c->m, c->H, Hb);
        for (int64_t t0 = 0; t0 < sl.count && rc == STLQ_MI355_OK; t0 += tile) {
            const int64_t nt = std::min(tile, sl.count - t0);
            if (lr) {
                TileEvents te;
                rc = LargeRootTile(c, dX + t0 * d, nt, Hb, sp->root_mode, nullptr, nullptr,
                                   sl.dcluster.as<uint32_t>() + t0, sl.dcodes.as<uint8_t>() + t0 * code_b,
                                   sl.dbest.as<float>() + t0, c->stream, &te, want ? &sp->encode : nullptr,
                                   want ? sl.da.as<float>() + t0 * m : nullptr,
                                   want ? sl.dcost.as<float>() + t0 : nullptr,
                                   gid0 + static_cast<uint64_t>(sl.first + t0));
                if (rc == STLQ_MI355_OK) c->tiles.push_back(te);
            } else {
                EncodeOut o{sl.dcodes.as<uint8_t>() + t0 * m, want ? sl.da.as<float>() + t0 * m : nullptr,
                            want ? sl.dcost.as<float>() + t0 : nullptr, nullptr};
                rc = EncodeTile(c, dX + t0 * d, nt, sp->encode, o, c->stream, true, true,
                                gid0 + static_cast<uint64_t>(sl.first + t0));
            }
        }
        if (rc != STLQ_MI355_OK) break;
        if (!hip_ok(hipMemcpyAsync(sl.hcodes, sl.dcodes.p, cnt * code_b, hipMemcpyDeviceToHost, c->stream), "hipMemcpyAsync"))
            break;
        if (want && (!hip_ok(hipMemcpyAsync(sl.ha, sl.da.p, cnt * m * 4, hipMemcpyDeviceToHost, c->stream), "hipMemcpyAsync") ||
                     !hip_ok(hipMemcpyAsync(sl.hcost, sl.dcost.p, cnt * 4, hipMemcpyDeviceToHost, c->stream), "hipMemcpyAsync")))
            break;
        if (lr && (!hip_ok(hipMemcpyAsync(sl.hcluster, sl.dcluster.p, cnt * 4, hipMemcpyDeviceToHost, c->stream), "hipMemcpyAsync") ||
                   !hip_ok(hipMemcpyAsync(sl.hbest, sl.dbest.p, cnt * 4, hipMemcpyDeviceToHost, c->stream), "hipMemcpyAsync")))
            break;
        if (!hip_ok(hipEventRecord(sl.done, c->stream), "hipEventRecord")) break;
        sl.busy = true;
        ++nchunks;
        // Hand the previous chunk to the sink while this one copies and encodes.
        if (!drain(slot[(ci + 1) & 1])) break;
    }
    if (rc == STLQ_MI355_OK) {
        for (int k = 0; k < 2 && rc == STLQ_MI355_OK; ++k) {
            Slot* older = nullptr;
            for (Slot& sl : slot)
                if (sl.busy && (!older || sl.first < older->first)) older = &sl;
            if (older && !drain(*older)) break;
        }
    }
    cleanup();
    if (stats) {
        stats->wall_ms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t_begin).count();
        stats->h2d_ms = h2d_ms;
        stats->compute_ms = comp_ms;
        stats->fill_ms = fill_ms;
        stats->sink_ms = sink_ms;
        stats->h2d_bytes = h2d_bytes;
        stats->chunks = nchunks;
    }
    return rc;
}

namespace {

// The stream-to-store adapter: every chunk the sink receives becomes one block of the store,
// then (with a checkpoint path) a committed block.
struct StoreSink {
    stlq_mi355_fill_fn fill;
    void* user;
    stlq_mi355_store* store;
    const char* ckpt;
    bool lr;
    int m;
    int raw_kind;
    int d;
    std::vector<uint32_t> cluster;
    std::vector<uint8_t> small;
    std::vector<uint64_t> bucket_bytes;
    int rc = STLQ_MI355_OK;
    std::string err;
};

int StoreFill(void* u, int64_t first, int64_t count, void* dst) {
    auto* s = static_cast<StoreSink*>(u);
    return s->fill(s->user, first, count, dst);
}

int StoreSinkChunk(void* u, int64_t first, int64_t count, const stlq_mi355_chunk_out* out) {
    auto* s = static_cast<StoreSink*>(u);
    const size_t n = static_cast<size_t>(count);
    const size_t mc = static_cast<size_t>(std::max(0, s->m - 1));
    const uint32_t* cluster = out->cluster_id;
    const uint8_t* small = out->B_small;
    if (!s->lr) {  // full precomp: layer 0's code is the cluster id (ExtractClusterIdAndCodesSmall)
        s->cluster.resize(n);
        s->small.resize(n * mc);
        const size_t m = static_cast<size_t>(s->m);
        for (size_t i = 0; i < n; ++i) {
            s->cluster[i] = out->codes[i * m];
            std::memcpy(s->small.data() + i * mc, out->codes + i * m + 1, mc);
        }
        cluster = s->cluster.data();
        small = s->small.data();
    }
    auto fail = [&](int rc) {
        s->rc = rc;
        s->err = stlq_mi355_last_error();
        return 1;
    };
    if (int rc = stlq_mi355_store_append(s->store, static_cast<uint64_t>(first), count, cluster, static_cast<int>(mc),
                                         small, s->m, out->a, s->raw_kind, out->input, s->d))
        return fail(rc);
    if (!s->ckpt) return 0;
    int64_t nb = 0;
    if (int rc = stlq_mi355_store_flush(s->store)) return fail(rc);
    if (int rc = stlq_mi355_store_bucket_bytes(s->store, nullptr, 0, &nb)) return fail(rc);
    s->bucket_bytes.resize(static_cast<size_t>(nb));
    if (int rc = stlq_mi355_store_bucket_bytes(s->store, s->bucket_bytes.data(), nb, &nb)) return fail(rc);
    if (int rc = stlq_mi355_checkpoint_write(s->ckpt, static_cast<uint64_t>(first + count), s->bucket_bytes.data(), nb))
        return fail(rc);
    return 0;
}

}  // namespace

int stlq_mi355_encode_stream_store(stlq_mi355_ctx* c, int64_t n_total, int64_t chunk,
                                   const stlq_mi355_stream_params* sp, stlq_mi355_fill_fn fill, void* user,
                                   stlq_mi355_store* store, const char* checkpoint_path,
                                   stlq_mi355_stream_stats* stats) {
    RC_TRY(CheckCtx(c));
    if (!sp || !fill || !store) return Fail(STLQ_MI355_ERR_INVALID, "encode_stream_store: null argument");
    const bool lr = sp->large_root != 0;
    if (lr) {
        RC_TRY(CheckLargeRoot(c, sp->encode.H_beam, sp->root_mode));
    } else {
        RC_TRY(CheckPre(c));
    }
    if (chunk <= 0) return Fail(STLQ_MI355_ERR_INVALID, "encode_stream_store: chunk must be positive");
    const int m = lr ? c->lr_m : c->m;
    const int d = lr ? c->lr_d : c->d;
    const int h0 = lr ? c->h0 : c->h_vec[0];
    int sd = 0, sm = 0, sh0 = 0, svb = 0, sraw = 0;
    RC_TRY(stlq_mi355_store_info(store, &sd, &sm, &sh0, &svb, &sraw));
    if (sd != d || sm != m || sh0 != h0)
        return Fail(STLQ_MI355_ERR_INVALID, "encode_stream_store: the store's d, m or h_vec[0] (" + std::to_string(sd) +
                                                ", " + std::to_string(sm) + ", " + std::to_string(sh0) +
                                                ") differ from the codebooks' (" + std::to_string(d) + ", " +
                                                std::to_string(m) + ", " + std::to_string(h0) + ")");
    const int esz = sp->input_u8 ? 1 : 4;
    if (svb && sraw != d * esz)
        return Fail(STLQ_MI355_ERR_INVALID, "encode_stream_store: raw_bytes_per_vec must be d for uint8 input and 4d "
                                            "for float input");
    if (checkpoint_path && sp->start_id % static_cast<uint64_t>(chunk) != 0)
        return Fail(STLQ_MI355_ERR_INVALID, "EncodeBaseStreaming: start_id must be a multiple of large.base_block when "
                                            "using checkpointing.");
    stlq_mi355_stream_params p = *sp;
    p.encode.want_coeffs = 1;
    StoreSink sink{fill, user, store, checkpoint_path, lr, m,
                   svb ? (sp->input_u8 ? STLQ_MI355_RAW_U8 : STLQ_MI355_RAW_F32) : STLQ_MI355_RAW_NONE, d};
    const int rc = stlq_mi355_encode_stream(c, n_total, chunk, &p, &StoreFill, &StoreSinkChunk, &sink, stats);
    if (rc == STLQ_MI355_ERR_CALLBACK && sink.rc != STLQ_MI355_OK) return Fail(sink.rc, sink.err);
    return rc;
}

// ---------------------------------------------------------------------------------------------
// Large root.
}  // extern "C"

namespace {

int CheckLargeRoot(stlq_mi355_ctx* c, int H_beam, int root_mode) {
    RC_TRY(CheckCtx(c));
    if (!c->has_lr) return Fail(STLQ_MI355_ERR_STATE, "large-root codebooks not set (call stlq_mi355_set_large_root)");
    RC_TRY(CheckBeam(std::max(1, H_beam)));
    if (root_mode != 0 && root_mode != 1) return Fail(STLQ_MI355_ERR_INVALID, "root_mode must be 0 or 1");
    return STLQ_MI355_OK;
}

// one_score: the root stage keeps one score per vector (forced or nearest root), not h0.
int64_t LargeRootTileVectors(stlq_mi355_ctx* c, int64_t n, int Hb, bool one_score) {
    const int m = c->lr_m;
    const int64_t per = 4LL * c->lr_d + 4 + 8LL * std::max(c->Hs, 1) + (one_score ? 16 : 4LL * c->h0) +
                        2 * (4LL * Hb * BeamRecordStride(m) + 4) + m + 16 +
                        (5LL * m + 20);  // refit: b0, ICM flags and proposals, ILS candidate codes/coefficients/cost
    // A multiple of 128 vectors: the nearest-root kernel sweeps all h0 roots for 128 vectors per
    // block, and a partial last block runs as a launch of its own on one CU (7.8 ms per tile at
    // C5 against 48 ms for the full blocks), so only the last tile of a call may have one.
    int64_t t = std::max<int64_t>(EnvWorkspaceBytes() / per, 1024) / 128 * 128;
    return std::min<int64_t>(t, std::max<int64_t>(n, 1));
}

// One tile of BeamSearchPrefixLSLargeRoot on device-resident fp32 X (nt x d): ||x||^2, xC_small
// (MFMA GEMM unless given), root candidates (forced root, nearest root or top-H roots from the
// MFMA score GEMM), then the expansion layers. Outputs cluster ids, B_small ((m-1) x nt) and the
// selected errors, all device pointers. With `refine`, the streaming encode's refit follows
// (encode_base_streaming.cpp:1117-1210): SolveLeastSquaresAllLargeRoot + ComputeCostsLargeRoot,
// or DynamicIcmWithIls*NoNormalLargeRoot when ICM/ILS is asked for, into d_a / d_cost; id0 is
// the global id of the tile's first vector.
int LargeRootTile(stlq_mi355_ctx* c, const float* dX, int64_t nt, int Hb, int root_mode, const uint32_t* d_forced,
                  const float* dxC_given, uint32_t* d_cluster, uint8_t* d_codes, float* d_best, hipStream_t s,
                  TileEvents* te, const stlq_mi355_encode_params* refine, float* d_a, float* d_cost, uint64_t id0) {
    const int m = c->lr_m, Hs = c->Hs, h0 = c->h0, d = c->lr_d;
    HIP_TRY(c->nx2.Ensure(static_cast<size_t>(nt) * 4));
    HIP_TRY(c->xC.Ensure(static_cast<size_t>(nt) * std::max(Hs, 1) * 4));
    const bool one_score = d_forced || root_mode == 1;  // the seed reads one score per vector
    HIP_TRY(c->scores.Ensure(static_cast<size_t>(nt) * (one_score ? 1 : h0) * 4));
    RC_TRY(EnsureState(c, nt, m, Hb));
    auto rec = [&](int k) -> hipError_t {
        if (!te) return hipSuccess;
        te->e[k] = c->NextEvent();
        return hipEventRecord(te->e[k], s);
    };
    if (te) te->n = nt;
    HIP_TRY(rec(0));
    HIP_TRY(LaunchXNorm2(dX, d, nt, c->nx2.as<float>(), s));
    HIP_TRY(rec(1));
    const float* dxs = dxC_given;
    if (Hs > 0 && !dxs) {
        HIP_TRY(LaunchGemmXc(dX, nt, d, c->Cs.as<float>(), Hs, c->xC.as<float>(), Hs, s));
        dxs = c->xC.as<float>();
        if (te) ++te->gemm_launches;
    }
    RootArgs ra;
    ra.nx2 = c->nx2.as<float>();
    ra.norm0 = c->norm0.as<float>();
    ra.sw0 = c->sw0.as<float>();
    ra.isw0 = c->isw0.as<float>();
    ra.out = StateOf(c, 0);
    ra.n = nt;
    ra.m = m;
    ra.Hb = Hb;
    ra.h0 = h0;
    ra.is_last = (m == 1);
    ra.cluster_out = d_cluster;
    ra.best_err = d_best;
    ra.scores = c->scores.as<float>();
    if (d_forced) {
        HIP_TRY(LaunchGatherRootDot(dX, d, c->C0.as<float>(), d_forced, nt, c->scores.as<float>(), s));
        ra.ldx = 1;
        ra.forced = d_forced;
        ra.root_slots = 1;
    } else if (root_mode == 1) {
        // Nearest root: the root-score GEMM with a first-minimum epilogue (no n x h0 score matrix),
        // vectors that met a NaN error redone by the exact scan, then the chosen root seeded as a
        // forced root (the same records as the one-slot scan of the scores).
        HIP_TRY(c->nearest.Ensure(static_cast<size_t>(nt) * 4));
        HIP_TRY(c->nearest_flag.Ensure(static_cast<size_t>(nt)));
        uint32_t* dn = c->nearest.as<uint32_t>();
        uint8_t* df = c->nearest_flag.as<uint8_t>();
        HIP_TRY(LaunchNearestRoot(dX, nt, d, c->C0.as<float>(), h0, c->norm0.as<float>(), c->nx2.as<float>(), dn, df,
                                  s));
        if (te) ++te->gemm_launches;
        HIP_TRY(LaunchNearestRootFixup(dX, d, c->C0.as<float>(), h0, c->norm0.as<float>(), c->nx2.as<float>(), df, nt,
                                       dn, s));
        HIP_TRY(LaunchGatherRootDot(dX, d, c->C0.as<float>(), dn, nt, c->scores.as<float>(), s));
        ra.ldx = 1;
        ra.forced = dn;
        ra.root_slots = 1;
    } else {
        HIP_TRY(LaunchGemmXc(dX, nt, d, c->C0.as<float>(), h0, c->scores.as<float>(), h0, s));
        if (te) ++te->gemm_launches;
        ra.ldx = h0;
        ra.root_slots = root_mode == 1 ? 1 : Hb;
    }
    HIP_TRY(rec(2));
    // Best-first pass over the expansion (as RunBeam's): with one root slot per vector the seed is
    // trivially in rank order, and every small layer must be full (the pass's kernels are built
    // for K = 256). Flagged vectors are re-seeded and re-run in the reference order below.
    bool best = m >= 2 && ra.root_slots == 1 && BestFirstBeam();
    for (int L = 1; L < m && best; ++L) best = c->lr_h[L] == kMaxK;
    if (best) {
        HIP_TRY(c->bf_flags.Ensure(static_cast<size_t>(nt)));
        HIP_TRY(c->bf_list.Ensure(static_cast<size_t>(nt) * 4));
        HIP_TRY(c->bf_count.Ensure(8));
        if (!c->bf_host && !c->noalloc)
            HIP_TRY(hipHostMalloc(reinterpret_cast<void**>(&c->bf_host), 8, hipHostMallocDefault));
        HIP_TRY(LaunchFill8(c->bf_flags.as<uint8_t>(), 0, nt, s));
        HIP_TRY(LaunchFill8(c->bf_count.as<uint8_t>(), 0, (c->bf_reset || c->noalloc) ? 8 : 4, s));
        c->bf_reset = c->noalloc;
        c->bf_used = !c->noalloc;
    }
    HIP_TRY(LaunchRootSeed(ra, s));
    if (te) {
        te->lay[0] = te->e[2];
        te->lay[1] = c->NextEvent();
        te->layers = 1;
        HIP_TRY(hipEventRecord(te->lay[1], s));
    }
    LayerArgs a;
    a.gram.G = c->G_small.as<float>();
    a.gram.ld = Hs;
    a.gram.G0S = c->G0S.as<float>();
    for (int l = 0; l < m; ++l) a.gram.off[l] = c->soff[l];
    a.xC = dxs;
    a.ldx = Hs;
    a.nx2 = c->nx2.as<float>();
    a.gdiag = c->gdiag_small.as<float>();
    a.Gs = c->Gs_small.as<float>();
    a.sw = c->sw_small.as<float>();
    a.isw = c->isw_small.as<float>();
    a.sw0 = c->sw0.as<float>();
    a.isw0 = c->isw0.as<float>();
    a.prune = (c->prune_lr && PruneEnv()) ? 1 : 0;
    a.n = nt;
    a.m = m;
    a.Hb = Hb;
    a.codes_out = d_codes;
    a.cluster_out = d_cluster;
    a.best_err = d_best;
    a.flags = best ? c->bf_flags.as<uint8_t>() : nullptr;
    auto expand = [&](bool timed) -> int {
        int cur = 0;
        for (int L = 1; L < m; ++L) {
            a.in = StateOf(c, cur);
            a.out = StateOf(c, cur ^ 1);
            a.K = c->lr_h[L];
            a.offL = c->soff[L];
            a.is_last = (L == m - 1);
            HIP_TRY(LaunchBeamLayer(L, true, a, s));
            cur ^= 1;
            if (te) ++te->beam_launches;
            if (te && timed) {
                te->lay[L + 1] = c->NextEvent();
                te->layers = L + 1;
                HIP_TRY(hipEventRecord(te->lay[L + 1], s));
            }
        }
        return STLQ_MI355_OK;
    };
    RC_TRY(expand(true));
    if (best) {
        // the flagged vectors: seeded again and expanded in the reference order, one wave per
        // listed vector (grids sized for all nt; waves past the list's length exit at once)
        int* counts = c->bf_count.as<int>();
        HIP_TRY(LaunchCollectFlagged(c->bf_flags.as<uint8_t>(), nt, c->bf_list.as<int>(), counts, s));
        ra.list = c->bf_list.as<int>();
        ra.list_n = counts;
        HIP_TRY(LaunchRootSeed(ra, s));
        a.flags = nullptr;
        a.list = ra.list;
        a.list_n = counts;
        RC_TRY(expand(false));
        if (!c->noalloc) HIP_TRY(hipMemcpyAsync(c->bf_host, counts, 8, hipMemcpyDeviceToHost, s));
    }
    HIP_TRY(rec(3));
    if (!refine || !d_a || !d_cost) {
        if (te) te->e[4] = te->e[5] = te->e[6] = te->e[3];
        return STLQ_MI355_OK;
    }
    HIP_TRY(c->b0.Ensure(static_cast<size_t>(nt) * 4));
    HIP_TRY(LaunchRootDot(dX, d, c->C0.as<float>(), d_cluster, nt, c->b0.as<float>(), s));
    const IcmProblem P = LargeRootProblem(c, dxs, c->nx2.as<float>(), d_cluster, c->b0.as<float>(), nt);
    const bool icm = refine->icm_iters > 0 || refine->ils_iters > 0;
    if (!icm) {
        LsArgs ls = P.ls;
        ls.codes = d_codes;
        ls.a = d_a;
        ls.cost = d_cost;
        HIP_TRY(LaunchLsAll(ls, s));
        HIP_TRY(LaunchCosts(ls, s));
    }
    HIP_TRY(rec(4));
    if (icm)
        RC_TRY(RunIcmIls(c, P, refine->icm_iters, refine->ils_iters, refine->perturb_k, refine->use_abs, refine->seed,
                         id0, d_codes, d_a, d_cost, s));
    HIP_TRY(rec(5));
    HIP_TRY(rec(6));
    return STLQ_MI355_OK;
}

}  // namespace

extern "C" {

int stlq_mi355_set_large_root(stlq_mi355_ctx* c, int d, int m, const int* h_vec, const float* C0,
                              const float* C_small) {
    RC_TRY(CheckCtx(c));
    // root ids travel in the 26-bit candidate field of the beam's selection keys
    RC_TRY(ValidateLayers(d, m, h_vec, (1 << 26) - 2));
    if (!C0 || (m > 1 && !C_small)) return Fail(STLQ_MI355_ERR_INVALID, "null codebooks");
    c->has_lr = false;
    c->lr_d = d;
    c->lr_m = m;
    c->h0 = h_vec[0];
    int o = 0;
    for (int l = 0; l < m; ++l) c->lr_h[l] = h_vec[l];
    c->soff[0] = 0;
    for (int l = 1; l < m; ++l) {
        c->soff[l] = o;
        o += h_vec[l];
    }
    c->Hs = o;
    const size_t h0 = static_cast<size_t>(c->h0), Hs = static_cast<size_t>(std::max(c->Hs, 1));
    HIP_TRY(c->C0.Ensure(h0 * d * 4));
    HIP_TRY(c->norm0.Ensure(h0 * 4));
    HIP_TRY(c->Cs.Ensure(Hs * d * 4));
    HIP_TRY(c->G_small.Ensure(Hs * Hs * 4));
    HIP_TRY(c->G0S.Ensure(h0 * Hs * 4));
    HIP_TRY(c->gdiag_small.Ensure(Hs * 4));
    HIP_TRY(c->invnorm_small.Ensure(Hs * 4));
    HIP_TRY(hipMemcpyAsync(c->C0.p, C0, h0 * d * 4, hipMemcpyHostToDevice, c->stream));
    HIP_TRY(LaunchNorms(c->C0.as<float>(), d, c->h0, true, c->norm0.as<float>(), nullptr, c->stream));
    if (c->Hs > 0) {
        HIP_TRY(hipMemcpyAsync(c->Cs.p, C_small, static_cast<size_t>(c->Hs) * d * 4, hipMemcpyHostToDevice, c->stream));
        HIP_TRY(LaunchGram(c->Cs.as<float>(), d, c->Hs, c->G_small.as<float>(), c->stream));
        HIP_TRY(LaunchCross(c->C0.as<float>(), c->h0, c->Cs.as<float>(), c->Hs, d, c->G0S.as<float>(), c->stream));
        HIP_TRY(LaunchDiag(c->G_small.as<float>(), c->Hs, c->gdiag_small.as<float>(), c->stream));
        // precomp_large_root.cpp:101-114: invnorm_small_flat from the omp-simd Norm2
        HIP_TRY(LaunchNorms(c->Cs.as<float>(), d, c->Hs, true, nullptr, c->invnorm_small.as<float>(), c->stream));
    }
    // Beam candidate pruning: the roots' and small codewords' scalings, the row-scaled small Gram,
    // and the envelope.
    HIP_TRY(c->sw0.Ensure(h0 * 4));
    HIP_TRY(c->isw0.Ensure(h0 * 4));
    HIP_TRY(c->sw_small.Ensure(Hs * 4));
    HIP_TRY(c->isw_small.Ensure(Hs * 4));
    HIP_TRY(c->Gs_small.Ensure(Hs * Hs * 4));
    HIP_TRY(LaunchPruneScale(c->norm0.as<float>(), c->h0, c->sw0.as<float>(), c->isw0.as<float>(), c->stream));
    if (c->Hs > 0) {
        HIP_TRY(LaunchPruneScale(c->gdiag_small.as<float>(), c->Hs, c->sw_small.as<float>(), c->isw_small.as<float>(),
                                 c->stream));
        HIP_TRY(LaunchRowScale(c->G_small.as<float>(), c->Hs, c->Hs, c->sw_small.as<float>(), c->Gs_small.as<float>(),
                               c->stream));
        const float* mats[2] = {c->G_small.as<float>(), c->G0S.as<float>()};
        const int64_t counts[2] = {static_cast<int64_t>(c->Hs) * c->Hs, static_cast<int64_t>(h0) * c->Hs};
        RC_TRY(GramInEnvelope(c, mats, counts, 2, &c->prune_lr));
    } else {
        c->prune_lr = false;
    }
    HIP_TRY(hipStreamSynchronize(c->stream));
    c->has_lr = true;
    return STLQ_MI355_OK;
}

int stlq_mi355_beam_search_large_root(stlq_mi355_ctx* c, const float* X, const float* xC_small, int64_t n,
                                      int H_beam, const uint32_t* forced_root, int root_mode, uint32_t* cluster_id,
                                      uint8_t* B_small, float* best_err) {
    RC_TRY(CheckLargeRoot(c, H_beam, root_mode));
    const int Hb = std::max(1, H_beam);
    const int m = c->lr_m, Hs = c->Hs, d = c->lr_d;
    if (n < 0 || (n > 0 && (!X || !cluster_id || (m > 1 && !B_small))))
        return Fail(STLQ_MI355_ERR_INVALID, "bad arguments");
    if (n == 0) return STLQ_MI355_OK;
    if (forced_root) {
        for (int64_t i = 0; i < n; ++i)
            if (forced_root[i] >= static_cast<uint32_t>(c->h0))
                return Fail(STLQ_MI355_ERR_INVALID, "forced root " + std::to_string(forced_root[i]) + " of vector " +
                                                        std::to_string(i) + " >= h0");
    }
    c->ResetTimings();
    const int64_t tile = LargeRootTileVectors(c, n, Hb, forced_root != nullptr || root_mode == 1);
    HIP_TRY(c->X.Ensure(static_cast<size_t>(tile) * d * 4));
    HIP_TRY(c->roots.Ensure(static_cast<size_t>(tile) * 4 * 2));
    HIP_TRY(c->codes.Ensure(static_cast<size_t>(tile) * std::max(m - 1, 1)));
    HIP_TRY(c->best.Ensure(static_cast<size_t>(tile) * 4));
    if (xC_small) HIP_TRY(c->xC_in.Ensure(static_cast<size_t>(tile) * std::max(Hs, 1) * 4));
    uint32_t* d_roots = c->roots.as<uint32_t>();
    uint32_t* d_cluster = d_roots + tile;
    hipStream_t s = c->stream;
    for (int64_t t0 = 0; t0 < n; t0 += tile) {
        const int64_t nt = std::min(tile, n - t0);
        HIP_TRY(hipMemcpyAsync(c->X.p, X + t0 * d, static_cast<size_t>(nt) * d * 4, hipMemcpyHostToDevice, s));
        if (forced_root)
            HIP_TRY(hipMemcpyAsync(d_roots, forced_root + t0, static_cast<size_t>(nt) * 4, hipMemcpyHostToDevice, s));
        if (xC_small)
            HIP_TRY(hipMemcpyAsync(c->xC_in.p, xC_small + t0 * Hs, static_cast<size_t>(nt) * Hs * 4,
                                   hipMemcpyHostToDevice, s));
        TileEvents te;
        RC_TRY(LargeRootTile(c, c->X.as<float>(), nt, Hb, root_mode, forced_root ? d_roots : nullptr,
                             xC_small ? c->xC_in.as<float>() : nullptr, d_cluster, c->codes.as<uint8_t>(),
                             c->best.as<float>(), s, &te));
        c->tiles.push_back(te);
        HIP_TRY(hipMemcpyAsync(cluster_id + t0, d_cluster, static_cast<size_t>(nt) * 4, hipMemcpyDeviceToHost, s));
        if (m > 1)
            HIP_TRY(hipMemcpyAsync(B_small + t0 * (m - 1), c->codes.p, static_cast<size_t>(nt) * (m - 1),
                                   hipMemcpyDeviceToHost, s));
        if (best_err)
            HIP_TRY(hipMemcpyAsync(best_err + t0, c->best.p, static_cast<size_t>(nt) * 4, hipMemcpyDeviceToHost, s));
        HIP_TRY(hipStreamSynchronize(s));
    }
    return STLQ_MI355_OK;
}

}  // extern "C"

namespace {

enum class LrOp { kLs, kCosts, kIcm };

struct LrIcm {
    int icm_iters, ils_iters, perturb_k, use_abs;
    uint32_t seed;
    uint64_t id0;
};

// Host-buffer large-root refit, tiled over the workspace budget: per tile X, the roots and B_small
// (and xC_small, ||x||^2 and a when given) go up, b0 = <C0[:,root], x> is formed on the device,
// the op runs and its results come back. B_small is written only by kIcm.
int LargeRootRefit(stlq_mi355_ctx* c, LrOp op, const float* X, const float* nx2, const float* xC_small, int64_t n,
                   const uint32_t* cluster_id, uint8_t* B_small, const float* a_in, const LrIcm* ip, float* a_out,
                   float* cost_out, int64_t* fail_count) {
    RC_TRY(CheckLargeRoot(c, 1, 0));
    const int m = c->lr_m, Hs = c->Hs, d = c->lr_d, mb = c->lr_m - 1;
    if (n < 0 || (n > 0 && (!X || !cluster_id || (mb > 0 && !B_small)))) return Fail(STLQ_MI355_ERR_INVALID, "bad arguments");
    if (fail_count) *fail_count = 0;
    if (n == 0) return STLQ_MI355_OK;
    for (int64_t i = 0; i < n; ++i) {
        if (cluster_id[i] >= static_cast<uint32_t>(c->h0))
            return Fail(STLQ_MI355_ERR_INVALID, "root " + std::to_string(cluster_id[i]) + " of vector " +
                                                    std::to_string(i) + " >= h0");
        for (int l = 0; l < mb; ++l)
            if (B_small[i * mb + l] >= c->lr_h[l + 1])
                return Fail(STLQ_MI355_ERR_INVALID, "code " + std::to_string(B_small[i * mb + l]) + " of vector " +
                                                        std::to_string(i) + " exceeds layer " + std::to_string(l + 1) +
                                                        " size " + std::to_string(c->lr_h[l + 1]));
    }
    c->ResetTimings();
    const int64_t per = 4LL * d + 4LL * Hs + 16 + 2LL * mb + 12LL * m + 16;
    const int64_t tile = std::min<int64_t>(std::max<int64_t>(EnvWorkspaceBytes() / per, 1024), n);
    const size_t T = static_cast<size_t>(tile);
    HIP_TRY(c->X.Ensure(T * d * 4));
    HIP_TRY(c->xC.Ensure(T * std::max(Hs, 1) * 4));
    HIP_TRY(c->roots.Ensure(T * 4));
    HIP_TRY(c->codes.Ensure(T * std::max(mb, 1)));
    HIP_TRY(c->a.Ensure(T * m * 4));
    HIP_TRY(c->cost.Ensure(T * 4));
    HIP_TRY(c->nx2.Ensure(T * 4));
    HIP_TRY(c->b0.Ensure(T * 4));
    hipStream_t s = c->stream;
    HIP_TRY(LaunchFill8(c->fails.as<uint8_t>(), 0, 4, s));
    for (int64_t t0 = 0; t0 < n; t0 += tile) {
        const int64_t nt = std::min(tile, n - t0);
        const size_t N = static_cast<size_t>(nt);
        HIP_TRY(hipMemcpyAsync(c->X.p, X + t0 * d, N * d * 4, hipMemcpyHostToDevice, s));
        HIP_TRY(hipMemcpyAsync(c->roots.p, cluster_id + t0, N * 4, hipMemcpyHostToDevice, s));
        if (mb > 0) HIP_TRY(hipMemcpyAsync(c->codes.p, B_small + t0 * mb, N * mb, hipMemcpyHostToDevice, s));
        if (xC_small) {
            if (Hs > 0) HIP_TRY(hipMemcpyAsync(c->xC.p, xC_small + t0 * Hs, N * Hs * 4, hipMemcpyHostToDevice, s));
        } else if (Hs > 0) {
            HIP_TRY(LaunchGemmXc(c->X.as<float>(), nt, d, c->Cs.as<float>(), Hs, c->xC.as<float>(), Hs, s));
        }
        if (op != LrOp::kLs) {
            if (nx2) {
                HIP_TRY(hipMemcpyAsync(c->nx2.p, nx2 + t0, N * 4, hipMemcpyHostToDevice, s));
            } else {
                HIP_TRY(LaunchXNorm2(c->X.as<float>(), d, nt, c->nx2.as<float>(), s));
            }
        }
        HIP_TRY(LaunchRootDot(c->X.as<float>(), d, c->C0.as<float>(), c->roots.as<uint32_t>(), nt, c->b0.as<float>(), s));
        const IcmProblem P =
            LargeRootProblem(c, c->xC.as<float>(), c->nx2.as<float>(), c->roots.as<uint32_t>(), c->b0.as<float>(), nt);
        LsArgs ls = P.ls;
        ls.codes = c->codes.as<uint8_t>();
        ls.a = c->a.as<float>();
        ls.cost = c->cost.as<float>();
        if (op == LrOp::kLs) {
            HIP_TRY(LaunchLsAll(ls, s));
            HIP_TRY(hipMemcpyAsync(a_out + t0 * m, c->a.p, N * m * 4, hipMemcpyDeviceToHost, s));
        } else if (op == LrOp::kCosts) {
            HIP_TRY(hipMemcpyAsync(c->a.p, a_in + t0 * m, N * m * 4, hipMemcpyHostToDevice, s));
            HIP_TRY(LaunchCosts(ls, s));
            HIP_TRY(hipMemcpyAsync(cost_out + t0, c->cost.p, N * 4, hipMemcpyDeviceToHost, s));
        } else {
            TileEvents te;
            te.n = nt;
            te.e[0] = te.e[1] = te.e[2] = te.e[3] = te.e[4] = c->NextEvent();
            HIP_TRY(hipEventRecord(te.e[0], s));
            RC_TRY(RunIcmIls(c, P, ip->icm_iters, ip->ils_iters, ip->perturb_k, ip->use_abs, ip->seed,
                             ip->id0 + static_cast<uint64_t>(t0), c->codes.as<uint8_t>(), ls.a, ls.cost, s));
            te.e[5] = te.e[6] = c->NextEvent();
            HIP_TRY(hipEventRecord(te.e[5], s));
            c->tiles.push_back(te);
            if (mb > 0) HIP_TRY(hipMemcpyAsync(B_small + t0 * mb, c->codes.p, N * mb, hipMemcpyDeviceToHost, s));
            HIP_TRY(hipMemcpyAsync(a_out + t0 * m, c->a.p, N * m * 4, hipMemcpyDeviceToHost, s));
            HIP_TRY(hipMemcpyAsync(cost_out + t0, c->cost.p, N * 4, hipMemcpyDeviceToHost, s));
        }
        HIP_TRY(hipStreamSynchronize(s));
    }
    int fails = 0;
    HIP_TRY(hipMemcpyAsync(&fails, c->fails.p, 4, hipMemcpyDeviceToHost, s));
    HIP_TRY(hipStreamSynchronize(s));
    if (fail_count) *fail_count = fails;
    return STLQ_MI355_OK;
}

}  // namespace

extern "C" {

int stlq_mi355_convert_u8_rotate(stlq_mi355_ctx* c, const uint8_t* in, int ld_in, int rows, int cols, const float* R,
                                 float* out) {
    RC_TRY(CheckCtx(c));
    if (rows < 0 || cols < 0 || ld_in < rows || (rows > 0 && cols > 0 && (!in || !out)))
        return Fail(STLQ_MI355_ERR_INVALID, "bad arguments");
    if (rows == 0 || cols == 0) return STLQ_MI355_OK;
    const size_t r = static_cast<size_t>(rows), n = static_cast<size_t>(cols);
    hipStream_t s = c->stream;
    HIP_TRY(c->codes.Ensure(r * n));
    HIP_TRY(c->X.Ensure(r * n * 4));
    HIP_TRY(hipMemcpy2DAsync(c->codes.p, r, in, static_cast<size_t>(ld_in), r, n, hipMemcpyHostToDevice, s));
    HIP_TRY(LaunchU8ToF32(c->codes.as<uint8_t>(), c->X.as<float>(), r * n, s));
    const float* res = c->X.as<float>();
    if (R) {
        RC_TRY(UploadRotation(c, R, rows, s));
        HIP_TRY(c->xC.Ensure(r * n * 4));
        HIP_TRY(LaunchGemmXc(c->X.as<float>(), cols, rows, c->R_rm.as<float>(), rows, c->xC.as<float>(), rows, s));
        res = c->xC.as<float>();
    }
    HIP_TRY(hipMemcpyAsync(out, res, r * n * 4, hipMemcpyDeviceToHost, s));
    HIP_TRY(hipStreamSynchronize(s));
    return STLQ_MI355_OK;
}

int stlq_mi355_solve_ls_all_large_root(stlq_mi355_ctx* c, const float* X, const float* xC_small, int64_t n,
                                       const uint32_t* cluster_id, const uint8_t* B_small, float* a,
                                       int64_t* fail_count) {
    if (n > 0 && !a) return Fail(STLQ_MI355_ERR_INVALID, "a is null");
    return LargeRootRefit(c, LrOp::kLs, X, nullptr, xC_small, n, cluster_id, const_cast<uint8_t*>(B_small), nullptr,
                          nullptr, a, nullptr, fail_count);
}

int stlq_mi355_compute_costs_large_root(stlq_mi355_ctx* c, const float* X, const float* xC_small, int64_t n,
                                        const uint32_t* cluster_id, const uint8_t* B_small, const float* a,
                                        const float* nx2, float* cost) {
    if (n > 0 && (!a || !cost)) return Fail(STLQ_MI355_ERR_INVALID, "bad arguments");
    return LargeRootRefit(c, LrOp::kCosts, X, nx2, xC_small, n, cluster_id, const_cast<uint8_t*>(B_small), a,
                          nullptr, nullptr, cost, nullptr);
}

int stlq_mi355_icm_ils_large_root(stlq_mi355_ctx* c, const float* X, const float* nx2, const float* xC_small,
                                  int64_t n, const uint32_t* cluster_id, int icm_iters, int ils_iters, int perturb_k,
                                  int use_abs, uint32_t seed, uint64_t sample_id_offset, uint8_t* B_small, float* a,
                                  float* cost) {
    if (n > 0 && (!a || !cost)) return Fail(STLQ_MI355_ERR_INVALID, "bad arguments");
    if (icm_iters < 0 || ils_iters < 0 || perturb_k < 0)
        return Fail(STLQ_MI355_ERR_INVALID, "icm_iters, ils_iters and perturb_k must be >= 0");
    const LrIcm ip{icm_iters, ils_iters, perturb_k, use_abs, seed, sample_id_offset};
    return LargeRootRefit(c, LrOp::kIcm, X, nx2, xC_small, n, cluster_id, B_small, nullptr, &ip, a, cost, nullptr);
}

}  // extern "C"

// ---------------------------------------------------------------------------------------------
// Device-buffer helpers (include/stlq_mi355_tools.h).
extern "C" {

int stlq_mi355_dev_alloc(stlq_mi355_ctx* c, size_t bytes, void** out) {
    RC_TRY(CheckCtx(c));
    if (!out) return Fail(STLQ_MI355_ERR_INVALID, "out is null");
    *out = nullptr;
    HIP_TRY(hipMalloc(out, bytes ? bytes : 256));
    return STLQ_MI355_OK;
}

int stlq_mi355_dev_free(stlq_mi355_ctx* c, void* p) {
    RC_TRY(CheckCtx(c));
    if (p) {
        HIP_TRY(hipStreamSynchronize(c->stream));
        HIP_TRY(hipFree(p));
    }
    return STLQ_MI355_OK;
}

int stlq_mi355_copy_h2d(stlq_mi355_ctx* c, void* dst, const void* src, size_t bytes) {
    RC_TRY(CheckCtx(c));
    HIP_TRY(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, c->stream));
    HIP_TRY(hipStreamSynchronize(c->stream));
    return STLQ_MI355_OK;
}

int stlq_mi355_copy_d2h(stlq_mi355_ctx* c, void* dst, const void* src, size_t bytes) {
    RC_TRY(CheckCtx(c));
    HIP_TRY(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, c->stream));
    HIP_TRY(hipStreamSynchronize(c->stream));
    return STLQ_MI355_OK;
}

int stlq_mi355_dev_copy_kernel(stlq_mi355_ctx* c, void* dst, const void* src, size_t bytes) {
    RC_TRY(CheckCtx(c));
    if (bytes % 16 != 0) return Fail(STLQ_MI355_ERR_INVALID, "bytes must be a multiple of 16");
    HIP_TRY(LaunchCopy16(dst, src, bytes / 16, c->stream));
    HIP_TRY(hipStreamSynchronize(c->stream));
    return STLQ_MI355_OK;
}

int stlq_mi355_synchronize(stlq_mi355_ctx* c) {
    RC_TRY(CheckCtx(c));
    HIP_TRY(hipStreamSynchronize(c->stream));
    return STLQ_MI355_OK;
}

int stlq_mi355_device_info(stlq_mi355_ctx* c, char* name, int name_len, int* cu_count) {
    RC_TRY(CheckCtx(c));
    hipDeviceProp_t prop;
    HIP_TRY(hipGetDeviceProperties(&prop, c->device));
    if (name && name_len > 0) {
        std::strncpy(name, prop.gcnArchName, static_cast<size_t>(name_len) - 1);
        name[name_len - 1] = '\0';
    }
    if (cu_count) *cu_count = prop.multiProcessorCount;
    return STLQ_MI355_OK;
}

}  // extern "C"
