// Beam-layer kernels and their launch templates, shared by the translation units that
// instantiate them (k_beam.hip, k_beam_queue.hip, k_beam_staged_a.hip, k_beam_staged_b.hip),
// so the deep layers compile in parallel. Everything here has internal linkage.
//
// Prefix-least-squares beam search, one layer per launch (src/quantizer/beam_search.cpp:196-422
// for the full precomp, :728-992 for the large-root expansion).
//
// Mapping: one wave64 owns one vector. For every live beam (slot order) the 64 lanes evaluate
// the layer's codewords k = lane + 64*j with the reference's arithmetic (no FMA contraction, same
// operation order, IEEE-exact quotients), so every candidate error is bit-identical to the CPU
// encoder's given the same xC, G and ||x||^2. The beam's prefix state (error, LS coefficients,
// Cholesky factor, codes) is one contiguous record. It is wave-uniform, but the factor and the
// coefficients are read into VGPRs (every lane the same values): on gfx950 a VALU instruction
// with two VGPR sources issues in half the cycles of one with a scalar source.
// The reference keeps the beam with a streaming "replace the first worst slot" rule
// (beam_search.cpp:101-113, :320-333); the wave replays it in scan order on sorted keys (see
// SelectTopH below). The surviving candidates are then re-evaluated once (same arithmetic, same
// bits) to build the next layer's records.
//
// Quotients by the Cholesky diagonal. Within one beam every forward/backward step divides by
// the same R(i,i), so y = RN(1/R(i,i)) is computed once with an IEEE division and each quotient
// s/R(i,i) is formed as q0 = s*y, r = fma(R(i,i), q0, -s), q = fma(-r, y, q0). With y the
// correctly rounded reciprocal this correction returns the correctly rounded quotient
// (Markstein's theorem) as long as nothing over- or underflows; the kernel takes it only when
// R(i,i) lies in [2^-20, 2^20] and every numerator magnitude in [2^-100, 2^100], and otherwise
// re-evaluates the chunk with IEEE division. tests/division_check.c verifies the identity.
#pragma once

#include <type_traits>

#include "internal.hpp"
#include "prune_bound.hpp"

namespace stlq_mi355 {
namespace {


constexpr float kInfF = __builtin_huge_valf();
constexpr int kMaxChunks = kMaxK / kWave;  // 4 chunks of 64 codewords

__device__ __forceinline__ float ReadLane(float v, int l) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}

// A value every lane holds (an LDS broadcast read), moved to a scalar register.
__device__ __forceinline__ float Uniform(float v) {
    return __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(v)));
}

template <int CTRL>
__device__ __forceinline__ float Dpp(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), CTRL, 0xF, 0xF, false));
}

// Max over a 16-lane row, broadcast to every lane of the row: quad_perm(1,0,3,2),
// quad_perm(2,3,0,1), row_half_mirror, row_mirror.
__device__ __forceinline__ float RowMax(float v) {
    v = fmaxf(v, Dpp<0xB1>(v));
    v = fmaxf(v, Dpp<0x4E>(v));
    v = fmaxf(v, Dpp<0x141>(v));
    return fmaxf(v, Dpp<0x140>(v));
}
__device__ __forceinline__ float RowMin(float v) {
    v = fminf(v, Dpp<0xB1>(v));
    v = fminf(v, Dpp<0x4E>(v));
    v = fminf(v, Dpp<0x141>(v));
    return fminf(v, Dpp<0x140>(v));
}
// Wave-uniform max/min over the first `rows` 16-lane rows.
__device__ __forceinline__ float SlotMax(float v, int rows) {
    v = RowMax(v);
    float r = ReadLane(v, 0);
    if (rows > 1) r = fmaxf(r, ReadLane(v, 16));
    if (rows > 2) r = fmaxf(fmaxf(r, ReadLane(v, 32)), ReadLane(v, 48));
    return r;
}
__device__ __forceinline__ float SlotMin(float v, int rows) {
    v = RowMin(v);
    float r = ReadLane(v, 0);
    if (rows > 1) r = fminf(r, ReadLane(v, 16));
    if (rows > 2) r = fminf(fminf(r, ReadLane(v, 32)), ReadLane(v, 48));
    return r;
}

// RecomputeWorst (beam_search.cpp:101-113): scan from slot 0 keeping the first slot whose error
// is strictly greater. Comparisons with NaN are false, so a NaN in slot 0 pins the worst to
// (NaN, 0) and a NaN elsewhere is never chosen.
__device__ __forceinline__ void RecomputeWorst(float s_err, int Hb, int rows, int lane, float& worst, int& widx) {
    const float e0 = ReadLane(s_err, 0);
    if (__builtin_isnan(e0)) {
        worst = e0;
        widx = 0;
        return;
    }
    const bool in = lane < Hb;
    const float v = (in && !__builtin_isnan(s_err)) ? s_err : -kInfF;
    const float mx = SlotMax(v, rows);
    const uint64_t eq = __ballot(in && s_err == mx);
    widx = static_cast<int>(__builtin_ctzll(eq));
    worst = mx;
}

// Lane mask of a predicate (the raw wave ballot: no bool-to-int round trip through a VGPR).
__device__ __forceinline__ uint64_t Ballot(bool b) { return __builtin_amdgcn_ballot_w64(b); }

// Order-preserving unsigned image of a non-NaN float (negative values reversed below the
// positive ones). -0 is kept out of the fast path, so equal errors have equal images.
__device__ __forceinline__ uint32_t OrderBits(float v) {
    const uint32_t b = __float_as_uint(v);
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
__device__ __forceinline__ float FromOrderBits(uint32_t o) {
    return __uint_as_float((o & 0x80000000u) ? (o & 0x7FFFFFFFu) : ~o);
}

// Streaming top-H of one vector (beam_search.cpp:301-333), in two forms.
//  TopKeys (fast path): lane q (< Hb) holds one slot's 64-bit key [image(err) | 63-slot
//    (6 bits) | candidate (26 bits)], kept in descending key order. A larger key is the slot
//    RecomputeWorst (beam_search.cpp:101-113) would pick first: larger error, and among equal
//    errors the lower slot. Lane 0 is therefore the worst slot, and an insertion is a rank (one
//    64-bit compare and a ballot), a one-lane shift of the keys above the rank, and a select.
//    Valid while no eligible candidate is NaN or -0. The error image is OrderBits, or, where
//    the errors are clamped at zero (layers >= 1: never negative), the float bits themselves,
//    which order non-negative floats as unsigned integers.
//  TopSlots (slow path): slot h in lane h with the reference's first-max RecomputeWorst scan and
//    its NaN comparisons. A layer whose candidates include an eligible NaN or -0 is replayed from
//    its start on this path.
constexpr uint32_t kNoCand = (1u << 26) - 1u;

template <bool kNonNeg>
__device__ __forceinline__ uint32_t KeyImage(float e) {
    return kNonNeg ? __float_as_uint(e) : OrderBits(e);
}
template <bool kNonNeg>
__device__ __forceinline__ float KeyError(uint32_t o) {
    return kNonNeg ? __uint_as_float(o) : FromOrderBits(o);
}

template <bool kNonNeg>
struct TopKeys {
    uint64_t key;
    uint32_t whi, wlo;  // key of lane 0 (the worst slot)
    bool empty = true;  // no candidate has entered yet
    __device__ explicit TopKeys(int lane)
        : key((static_cast<uint64_t>(KeyImage<kNonNeg>(__builtin_huge_valf())) << 32) |
              (static_cast<uint64_t>(63 - lane) << 26) | kNoCand),
          whi(KeyImage<kNonNeg>(__builtin_huge_valf())),
          wlo((63u << 26) | kNoCand) {}
};

// Lane (lane ^ J)'s value, J a power of two below 64: DPP quad permutations for 1 and 2, LDS
// swizzle (xor mode, within 32 lanes) for 4 to 16, bpermute for 32.
template <int J>
__device__ __forceinline__ uint32_t XorLane(uint32_t v, int lane) {
    if constexpr (J == 1) {
        return static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0xB1, 0xF, 0xF, false));
    } else if constexpr (J == 2) {
        return static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x4E, 0xF, 0xF, false));
    } else if constexpr (J < 32) {
        return static_cast<uint32_t>(__builtin_amdgcn_ds_swizzle(static_cast<int>(v), (J << 10) | 0x1F));
    } else {
        return static_cast<uint32_t>(__builtin_amdgcn_ds_bpermute((lane ^ 32) << 2, static_cast<int>(v)));
    }
}

// One compare-exchange step of a bitonic sort over the wave: sequences of K lanes, partners J
// lanes apart; lanes whose K-block is even sort ascending.
template <int K, int J>
__device__ __forceinline__ void BitonicStep(uint64_t& x, int lane) {
    const uint64_t y = (static_cast<uint64_t>(XorLane<J>(static_cast<uint32_t>(x >> 32), lane)) << 32) |
                       XorLane<J>(static_cast<uint32_t>(x), lane);
    const bool take_min = ((lane & K) == 0) == ((lane & J) == 0);
    x = (take_min == (y < x)) ? y : x;
}

// The 64 lanes' keys sorted ascending (lane 0 the smallest).
__device__ __forceinline__ uint64_t SortWave(uint64_t x, int lane) {
    BitonicStep<2, 1>(x, lane);
    BitonicStep<4, 2>(x, lane);
    BitonicStep<4, 1>(x, lane);
    BitonicStep<8, 4>(x, lane);
    BitonicStep<8, 2>(x, lane);
    BitonicStep<8, 1>(x, lane);
    BitonicStep<16, 8>(x, lane);
    BitonicStep<16, 4>(x, lane);
    BitonicStep<16, 2>(x, lane);
    BitonicStep<16, 1>(x, lane);
    BitonicStep<32, 16>(x, lane);
    BitonicStep<32, 8>(x, lane);
    BitonicStep<32, 4>(x, lane);
    BitonicStep<32, 2>(x, lane);
    BitonicStep<32, 1>(x, lane);
    BitonicStep<64, 32>(x, lane);
    BitonicStep<64, 16>(x, lane);
    BitonicStep<64, 8>(x, lane);
    BitonicStep<64, 4>(x, lane);
    BitonicStep<64, 2>(x, lane);
    BitonicStep<64, 1>(x, lane);
    return x;
}

struct TopSlots {
    float s_err = __builtin_huge_valf();
    int s_cand = -1;
    float worst = __builtin_huge_valf();
    int widx = 0;
};

// Lanes l+1..63.
__device__ __forceinline__ uint64_t AboveLane(int l) { return l >= 63 ? 0ull : (~0ull << (l + 1)); }

// Lane i receives lane i+1's value across the whole wave (DPP wave_shl:1); lane 63 keeps its own.
// (bound_ctrl: lane 63 reads 0; callers never take lane 63's value.)
__device__ __forceinline__ uint64_t WaveShl1(uint64_t v) {
    const int lo = __builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x130, 0xF, 0xF, true);
    const int hi = __builtin_amdgcn_update_dpp(0, static_cast<int>(v >> 32), 0x130, 0xF, 0xF, true);
    return (static_cast<uint64_t>(static_cast<uint32_t>(hi)) << 32) | static_cast<uint32_t>(lo);
}

// Slot-indexed view of the sorted keys: lane h receives the error and candidate of slot h.
template <bool kNonNeg>
__device__ __forceinline__ void ToSlots(const TopKeys<kNonNeg>& t, float& s_err, int& s_cand) {
    const uint32_t lo = static_cast<uint32_t>(t.key);
    const int slot = 63 - static_cast<int>((lo >> 26) & 63u);
    const uint32_t c = lo & kNoCand;
    const float err = KeyError<kNonNeg>(static_cast<uint32_t>(t.key >> 32));
    s_err = __int_as_float(__builtin_amdgcn_ds_permute(slot << 2, __float_as_int(err)));
    const int cand = __builtin_amdgcn_ds_permute(slot << 2, static_cast<int>(c));
    s_cand = cand == static_cast<int>(kNoCand) ? -1 : cand;
}

// Replays the streaming top-H over one group of 64 candidates in lane (= scan) order; lane l
// carries candidate id `cand` (ids ascend with the lane among the eligible lanes).
// Candidate `lane` is eligible when ok; it is inserted when !(e >= worst)
// (beam_search.cpp:320: `if (e >= worst_err) continue;`), into the worst slot.
// cand must stay below 2^26 - 1 (callers check).
//
// Fast path: returns false, leaving t as it was, when an eligible candidate is NaN or -0 (the
// caller then replays the layer with ReplaySlow). Otherwise e < worst exactly when
// image(e) < image(worst). With kNonNeg the errors are +0..+inf, NaN or -0, and NaN and -0 are
// exactly the bit patterns above +inf's.
// Best-first pass bookkeeping: the smallest key image among eligible candidates that did not
// enter (rej, per lane) or were evicted (ev).
struct OutTrack {
    uint32_t rej = 0xFFFFFFFFu;
    uint32_t ev = 0xFFFFFFFFu;
};

template <bool kNonNeg, bool kTrack, bool kSortFirst>
__device__ __forceinline__ bool ReplayFast(bool ok, float e, int cand, int Hb, int lane, TopKeys<kNonNeg>& t,
                                           OutTrack& ot) {
    const uint64_t okm = Ballot(ok);
    const bool bad = kNonNeg ? (__float_as_uint(e) > 0x7F800000u) : __builtin_amdgcn_classf(e, 0x23);
    if ((Ballot(bad) & okm) != 0ull) return false;
    const uint32_t oe = KeyImage<kNonNeg>(e);
    uint64_t mask = okm & Ballot(oe < t.whi);
    if (kTrack && kSortFirst && t.empty) {
        // Best-first pass, first group into an empty top-H: the group's keys sorted at once
        // instead of inserted one by one. Every entering candidate would enter in turn, so the
        // top-H after the group is its min(n, H) smallest keys: the same set the insertions give
        // (among equal errors the earlier candidate, which has the smaller key, stays), and the
        // smallest key left out counts as evicted for the tie check. Slots still empty keep their
        // placeholder keys, which sort above every candidate's.
        const int n = __popcll(mask);
        if (n == 0) return true;
        const bool in = ((mask >> lane) & 1ull) != 0ull;
        const uint64_t x = SortWave(in ? ((static_cast<uint64_t>(oe) << 32) | static_cast<uint32_t>(cand)) : ~0ull,
                                    lane);
        const int src = (Hb - 1 - lane) & 63;  // lane h (< Hb) takes the (Hb-1-h)-th smallest
        const uint64_t y =
            (static_cast<uint64_t>(static_cast<uint32_t>(
                 __builtin_amdgcn_ds_bpermute(src << 2, static_cast<int>(static_cast<uint32_t>(x >> 32)))))
             << 32) |
            static_cast<uint32_t>(__builtin_amdgcn_ds_bpermute(src << 2, static_cast<int>(static_cast<uint32_t>(x))));
        if (lane < Hb && lane >= Hb - n) t.key = y;
        if (n > Hb) {
            const uint32_t out = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(x >> 32), Hb));
            ot.ev = ot.ev < out ? ot.ev : out;
        }
        t.whi = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(t.key >> 32), 0));
        t.wlo = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(t.key), 0));
        t.empty = false;
        const uint32_t img = __builtin_amdgcn_inverse_ballot_w64(okm & ~mask) ? oe : 0xFFFFFFFFu;
        ot.rej = img < ot.rej ? img : ot.rej;
        return true;
    }
    uint64_t entered = 0;
    // lanes 1..Hb-1 of the sorted keys: the ones that stay when lane 0 (the worst) is evicted
    const uint64_t keep = (Hb >= 64 ? ~0ull : ((1ull << Hb) - 1ull)) & ~1ull;
    while (mask) {
        const int l = static_cast<int>(__builtin_ctzll(mask));
        if (kTrack) {
            entered |= 1ull << l;
            ot.ev = ot.ev < t.whi ? ot.ev : t.whi;
        }
        // the new pair takes the evicted slot: the slot field of lane 0's key
        const uint32_t hi = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(oe), l));
        const uint32_t lo = (t.wlo & 0xFC000000u) | static_cast<uint32_t>(__builtin_amdgcn_readlane(cand, l));
        const uint64_t nk = (static_cast<uint64_t>(hi) << 32) | lo;
        const int r = __popcll(Ballot(t.key > nk) & keep);
        const uint64_t sh = WaveShl1(t.key);
        t.key = lane < r ? sh : (lane == r ? nk : t.key);
        t.whi = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(t.key >> 32), 0));
        t.wlo = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(t.key), 0));
        mask = okm & AboveLane(l) & Ballot(oe < t.whi);
    }
    if (kTrack) {
        const uint32_t img = __builtin_amdgcn_inverse_ballot_w64(okm & ~entered) ? oe : 0xFFFFFFFFu;
        ot.rej = img < ot.rej ? img : ot.rej;
    }
    return true;
}

template <int CTRL>
__device__ __forceinline__ uint32_t DppU(uint32_t v) {
    return static_cast<uint32_t>(
        __builtin_amdgcn_update_dpp(static_cast<int>(v), static_cast<int>(v), CTRL, 0xF, 0xF, false));
}

// Wave-uniform minimum: DPP within each 16-lane row (as RowMin), then the four row results.
__device__ __forceinline__ uint32_t WaveMinU32(uint32_t v) {
    v = min(v, DppU<0xB1>(v));
    v = min(v, DppU<0x4E>(v));
    v = min(v, DppU<0x141>(v));
    v = min(v, DppU<0x140>(v));
    const uint32_t a = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v), 0));
    const uint32_t b = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v), 16));
    const uint32_t c = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v), 32));
    const uint32_t d = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v), 48));
    return min(min(a, b), min(c, d));
}

// Rank-indexed view of the sorted keys: lane q receives the q-th smallest key's error and
// candidate (placeholders last).
template <bool kNonNeg>
__device__ __forceinline__ void ToRanks(const TopKeys<kNonNeg>& t, int Hb, int lane, float& s_err, int& s_cand) {
    const uint32_t lo = static_cast<uint32_t>(t.key);
    const uint32_t c = lo & kNoCand;
    const float err = KeyError<kNonNeg>(static_cast<uint32_t>(t.key >> 32));
    const int tgt = lane < Hb ? Hb - 1 - lane : lane;
    s_err = __int_as_float(__builtin_amdgcn_ds_permute(tgt << 2, __float_as_int(err)));
    const int cand = __builtin_amdgcn_ds_permute(tgt << 2, static_cast<int>(c));
    s_cand = cand == static_cast<int>(kNoCand) ? -1 : cand;
}

// Slow path: the reference's scan on slot arrays (NaN enters; RecomputeWorst after each insert).
// The worst can rise here (to NaN), so the eligible lanes after an insertion are re-tested from
// all ok lanes behind it, not only from the ones that were eligible before.
__device__ __forceinline__ void ReplaySlow(bool ok, float e, int cand, int Hb, int rows, int lane, TopSlots& t) {
    const uint64_t okm = Ballot(ok);
    uint64_t mask = okm & Ballot(!(e >= t.worst));
    while (mask) {
        const int l = static_cast<int>(__builtin_ctzll(mask));
        const float ev = ReadLane(e, l);
        const int cl = __builtin_amdgcn_readlane(cand, l);
        if (lane == t.widx) {
            t.s_err = ev;
            t.s_cand = cl;
        }
        RecomputeWorst(t.s_err, Hb, rows, lane, t.worst, t.widx);
        mask = okm & AboveLane(l) & Ballot(!(e >= t.worst));
    }
}

// Runs `chunks(replay)` with the fast replay and, if it reports a NaN or -0, again from the start
// with the slow one; returns the slot-indexed (error, candidate) of the final top-H.
// chunks(replay, tag, worst) must call replay(ok, e, cand) for every group of candidates in scan
// order, stop and return false as soon as a call returns false, and return true otherwise.
// The second argument of chunks is std::false_type on the fast pass and std::true_type on the
// slow one; the third returns the current worst error (+inf while a slot is empty), which only
// falls during the fast pass.
//
// kRank: the fast pass's result comes out rank-indexed (lane q the q-th smallest key).
// kBest (the best-first pass; implies kRank): no slow pass, and `flag` is set when the result
// may differ from the reference's: an eligible NaN or -0, or an eligible candidate left out (or
// evicted) with the same error as the final worst of a full top-H. Without such a tie the top-H
// set does not depend on the scan order: every candidate with an error below the final worst
// enters when it is scanned and is never evicted, whatever came before it.
template <bool kNonNeg, bool kBest, bool kRank, bool kSortFirst = kBest, class Chunks>
__device__ __forceinline__ void SelectTopH(int Hb, int lane, Chunks&& chunks, float& s_err, int& s_cand, bool& flag) {
    TopKeys<kNonNeg> tk(lane);
    OutTrack ot;
    const bool fast = chunks(
        [&](bool ok, float e, int cand) { return ReplayFast<kNonNeg, kBest, kSortFirst>(ok, e, cand, Hb, lane, tk, ot); },
        std::false_type(), [&]() { return KeyError<kNonNeg>(tk.whi); });
    if constexpr (kBest) {
        if (!fast) {
            flag = true;
            s_err = kInfF;
            s_cand = -1;
            return;
        }
        const uint32_t rej = WaveMinU32(ot.rej);
        const uint32_t out_min = rej < ot.ev ? rej : ot.ev;
        if (tk.whi < KeyImage<kNonNeg>(kInfF) && out_min == tk.whi) flag = true;
        ToRanks(tk, Hb, lane, s_err, s_cand);
    } else {
        if (fast) {
            if (kRank) ToRanks(tk, Hb, lane, s_err, s_cand);
            else ToSlots(tk, s_err, s_cand);
            return;
        }
        TopSlots ts;
        const int rows = (Hb + 15) >> 4;
        chunks(
            [&](bool ok, float e, int cand) {
                ReplaySlow(ok, e, cand, Hb, rows, lane, ts);
                return true;
            },
            std::true_type(), [&]() { return ts.worst; });
        s_err = ts.s_err;
        s_cand = ts.s_cand;
    }
}

// BestSlot (beam_search.cpp:409-416): first minimum over slots [0, curH) with strict '<'.
__device__ __forceinline__ int BestSlot(float err, int curH, int lane) {
    if (curH <= 1) return 0;
    const float e0 = ReadLane(err, 0);
    if (__builtin_isnan(e0)) return 0;
    const bool in = lane < curH;
    const float v = (in && !__builtin_isnan(err)) ? err : kInfF;
    const float mn = SlotMin(v, (curH + 15) >> 4);
    const uint64_t eq = __ballot(in && err == mn);
    return eq ? static_cast<int>(__builtin_ctzll(eq)) : 0;
}

// Record layout of one beam slot (dword offsets); stride dwords per slot:
// [err, R column by column, coef[m], codes, root id, kap, phi, kb, cq, (nf2, k1, k2 when a layer
// of the encode uses the diagonal split), padding to 16 bytes].
// Column c of the Cholesky factor holds R(0..c, c) followed by RN(1/R(c,c)) (formed once when the
// slot is made), so the first L columns sit at offsets that depend on L only and a layer-L kernel
// reads them with immediate offsets. kap, phi, kb, cq, nf2, k1 and k2 are the slot's pruning
// constants (prune_bound.hpp).
struct Rec {
    int coef, code, root, kap, phi, kb, cq, nf2, k1, k2, stride;
    bool diag;
    __host__ __device__ explicit Rec(int m) {
        coef = 1 + m * (m + 3) / 2;
        code = coef + m;
        root = code + CodeStride(m) / 4;
        kap = root + 1;
        phi = root + 2;
        kb = root + 3;
        cq = root + 4;
        // the diagonal split's constants only where a layer uses it
        diag = m - 1 >= prune::kDiagMinL;
        nf2 = root + 5;
        k1 = root + 6;
        k2 = root + 7;
        stride = (root + (diag ? 8 : 5) + 3) & ~3;
    }
    __device__ void PutBounds(float* rec, const prune::SlotBounds& b) const {
        rec[kap] = b.kap;
        rec[phi] = b.phi;
        rec[kb] = b.kb;
        rec[cq] = b.cq;
        if (diag) {
            float c1, c2;
            prune::DiagConsts(b, c1, c2);
            rec[nf2] = b.nf2;
            rec[k1] = c1;
            rec[k2] = c2;
        }
    }
    // nF2 of a stored slot (0 where the record carries none: the split is never used below it)
    __device__ float Nf2(const float* rec) const { return diag ? rec[nf2] : 0.0f; }
    __host__ __device__ static constexpr int R(int r, int c) { return 1 + c * (c + 3) / 2 + r; }
    __host__ __device__ static constexpr int Rinv(int c) { return 1 + c * (c + 3) / 2 + c + 1; }
};

// A zero the compiler has to treat as lane-varying. Loads through `p + VZero()` land in VGPRs:
// arithmetic with two VGPR sources issues twice as fast as with a scalar source on gfx950
// (v_mul_f32 / v_sub_f32: 2 cycles per wave64 instruction against 4). The asm is not volatile:
// a volatile one counts as a possible memory write and turns every later uniform load of the
// kernel into a vector load.
__device__ __forceinline__ int VZero() {
    int z;
    asm("v_mov_b32 %0, 0" : "=v"(z));
    return z;
}

// Raw buffer access to a row-major Gram (G, Gs or G_small: ld x ld floats, ld <= 20 * 256): a
// row's byte offset rides in a scalar register and the column in the lane's offset, so a row
// address costs one 32-bit scalar multiply instead of 64-bit pointer arithmetic. Reads past
// `bytes` return 0 (the buffer's range check).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t GramRsrc(const float* g, int ld) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(g), 0, ld * ld * static_cast<int>(sizeof(float)),
                                             0x00020000);
}
__device__ __forceinline__ float GramLd(__amdgpu_buffer_rsrc_t r, uint32_t lane_bytes, uint32_t row_bytes) {
    return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, static_cast<int>(lane_bytes),
                                                                static_cast<int>(row_bytes), 0));
}

__device__ __forceinline__ int CodeAt(const float* rec, int code_off, int t) {
    const uint32_t w = reinterpret_cast<const uint32_t*>(rec + code_off)[t >> 2];
    return static_cast<int>((w >> (8 * (t & 3))) & 0xFFu);
}

// Quotient s/d given y = RN(1/d); exact when every numerator's magnitude lies in
// [2^-100, 2^100] (see the file comment), which the caller checks from the running extremes
// lo = min |s| and hi = max |s|. A NaN numerator leaves lo/hi untouched: its quotient and every
// value that depends on it are NaN on either path.
__device__ __forceinline__ float QuotFast(float s, float d, float y, float& lo, float& hi) {
    const float q0 = s * y;
    const float r = __builtin_fmaf(d, q0, -s);
    const float q = __builtin_fmaf(-r, y, q0);
    const float as = __builtin_fabsf(s);
    lo = __builtin_fminf(lo, as);
    hi = __builtin_fmaxf(hi, as);
    return q;
}

__device__ __forceinline__ bool DiagFastOk(float d) { return d >= 0x1p-20f && d <= 0x1p20f; }

// One prefix-LS candidate (beam_search.cpp:291-318): forward U^T y = A, backward U v = y
// (linear_algebra.cpp:57-77; the large-root expansion multiplies by 1/diag instead,
// beam_search.cpp:544-547/569-572), delta = A.v, eta = A.a_old, then
// a_last = (gamma - eta)/(alpha - delta), e = max(E_old - diff*a_last, 0).
// MODE 0: IEEE division; 1: Markstein quotient with reciprocal table `rinv` (clears `safe` when
// a numerator leaves the exact range);
// 2: reciprocal multiply (large-root semantics).
// Element i of an array or of an accessor (a callable taking the index).
template <typename T>
__device__ __forceinline__ float At(const T& x, int i) {
    if constexpr (std::is_invocable_v<const T&, int>) return x(i);
    else return x[i];
}

template <int L, int MODE, typename RFn, typename RiT, typename AoT>
__device__ __forceinline__ void EvalCand(RFn R, const RiT& rinv, const float (&A)[L], const AoT& aold, float E_old,
                                         float alpha, float gamma, float (&y)[L], float (&v)[L], float& e,
                                         float& denom, float& a_last, bool& ok, bool& safe) {
    float lo = __builtin_huge_valf(), hi = 0.0f;
#pragma unroll
    for (int r = 0; r < L; ++r) {
        float s = A[r];
#pragma unroll
        for (int j = 0; j < r; ++j) s = s - R(j, r) * y[j];
        if (MODE == 0) y[r] = s / R(r, r);
        else if (MODE == 1) y[r] = QuotFast(s, R(r, r), At(rinv, r), lo, hi);
        else y[r] = s * At(rinv, r);
    }
#pragma unroll
    for (int r = L - 1; r >= 0; --r) {
        float s = y[r];
#pragma unroll
        for (int j = r + 1; j < L; ++j) s = s - R(r, j) * v[j];
        if (MODE == 0) v[r] = s / R(r, r);
        else if (MODE == 1) v[r] = QuotFast(s, R(r, r), At(rinv, r), lo, hi);
        else v[r] = s * At(rinv, r);
    }
    if (MODE == 1) safe = safe && (lo >= 0x1p-100f) && (hi <= 0x1p100f);
    float delta = 0.0f, eta = 0.0f;
#pragma unroll
    for (int t = 0; t < L; ++t) {
        delta = delta + A[t] * v[t];
        eta = eta + A[t] * At(aold, t);
    }
    denom = alpha - delta;
    ok = denom != 0.0f;
    const float diff = gamma - eta;
    a_last = diff / denom;
    const float ee = E_old - diff * a_last;
    e = ee < 0.0f ? 0.0f : ee;
}

// A zero that depends on `dep`: an address offset by it cannot be read before `dep` exists.
__device__ __forceinline__ int ZeroAfter(float dep) {
    int z;
    asm("v_mov_b32 %0, 0" : "=v"(z) : "v"(dep));
    return z;
}

// EvalCand with the slot's factor in LDS at f, laid out as the record from dword 1 (R(0..c, c) then
// RN(1/R(c,c)) for c < L), followed by a_old. The same operations in the same order, so the same
// bits. The reads of column r (forward) and row r (backward) wait for the quotient two steps back:
// the compiler then keeps about two rows of the factor in registers instead of all of it.
template <int L, int MODE>
__device__ __forceinline__ void EvalStaged(const float* f, const float (&A)[L], float E_old, float alpha, float gamma,
                                           float (&y)[L], float (&v)[L], float& e, float& denom, float& a_last,
                                           bool& ok, bool& safe) {
    constexpr int kRWords = L * (L + 3) / 2;
    float lo = __builtin_huge_valf(), hi = 0.0f;
#pragma unroll
    for (int r = 0; r < L; ++r) {
        const float* fr = r >= 2 ? f + ZeroAfter(y[r - 2]) : f;
        float s = A[r];
#pragma unroll
        for (int j = 0; j < r; ++j) s = s - fr[Rec::R(j, r) - 1] * y[j];
        const float d = fr[Rec::R(r, r) - 1];
        if (MODE == 0) y[r] = s / d;
        else if (MODE == 1) y[r] = QuotFast(s, d, fr[Rec::Rinv(r) - 1], lo, hi);
        else y[r] = s * fr[Rec::Rinv(r) - 1];
    }
#pragma unroll
    for (int r = L - 1; r >= 0; --r) {
        const float* fr = f + ZeroAfter(r + 2 < L ? v[r + 2] : y[L - 1]);
        float s = y[r];
#pragma unroll
        for (int j = r + 1; j < L; ++j) s = s - fr[Rec::R(r, j) - 1] * v[j];
        const float d = fr[Rec::R(r, r) - 1];
        if (MODE == 0) v[r] = s / d;
        else if (MODE == 1) v[r] = QuotFast(s, d, fr[Rec::Rinv(r) - 1], lo, hi);
        else v[r] = s * fr[Rec::Rinv(r) - 1];
    }
    if (MODE == 1) safe = safe && (lo >= 0x1p-100f) && (hi <= 0x1p100f);
    const float* fa = f + ZeroAfter(v[0]);
    float delta = 0.0f, eta = 0.0f;
#pragma unroll
    for (int t = 0; t < L; ++t) {
        delta = delta + A[t] * v[t];
        eta = eta + A[t] * fa[kRWords + t];
    }
    denom = alpha - delta;
    ok = denom != 0.0f;
    const float diff = gamma - eta;
    a_last = diff / denom;
    const float ee = E_old - diff * a_last;
    e = ee < 0.0f ? 0.0f : ee;
}

// The queue kernel's per-slot state in LDS: EvalStaged's factor layout (record dwords 1 ..
// L(L+3)/2: R(0..c, c) then RN(1/R(c,c)) for c < L), then a_old[L], then E_old, then the pruning
// bound's per-slot operands: ahat[L] (a_t * isw_t), kb, cq and the large root's sw0[root]. The
// stride is odd, so the slots that different lanes read at one offset sit in different LDS banks.
template <int L>
struct QStage {
    static constexpr int kRWords = L * (L + 3) / 2;
    static constexpr int kEold = kRWords + L;
    static constexpr int kAhat = kEold + 1;
    static constexpr int kKb = kAhat + L;
    static constexpr int kCq = kKb + 1;
    static constexpr int kSw0 = kCq + 1;
    static constexpr int kBoundWords = L + 3;  // ahat[L], kb, cq, sw0
    static constexpr int kStride = (kSw0 + 1) | 1;
    // dynamic LDS of one workgroup for beam width Hb
    static constexpr size_t Bytes(int Hb) {
        return sizeof(float) * static_cast<size_t>(kBeamWavesPerBlock) * static_cast<size_t>(Hb) * kStride;
    }
};

// Vector index i and beam-state index w of this wave (see LayerArgs::list); false when the wave
// has no vector.
__device__ __forceinline__ bool WaveItem(const LayerArgs& p, int wave, int64_t& i, int64_t& w) {
    w = static_cast<int64_t>(blockIdx.x) * kBeamWavesPerBlock + wave;
    if (p.list) {
        if (w >= *p.list_n) return false;
        i = p.list[w];
        return true;
    }
    i = w;
    return w < p.n;
}

// Best-first pass, last layer: the final pick is the first minimum over slots, so a tie for the
// minimum makes it depend on the slot order. `err` is rank-indexed (lane 0 the smallest).
__device__ __forceinline__ bool FinalTie(float err, int curH) {
    return curH >= 2 && ReadLane(err, 0) == ReadLane(err, 1);
}

// Layer 0 of the full-precomp beam (beam_search.cpp:240-263). BEST: the best-first pass
// (LayerArgs::flags); its records come out rank-indexed.
template <bool BEST>
__global__ __launch_bounds__(256) void Layer0Kernel(LayerArgs p) {
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    int64_t i, w;
    if (!WaveItem(p, wave, i, w)) return;
    const int m = p.m, Hb = p.Hb, K = p.K, off0 = p.offL;
    const Rec rc(m);
    const float nx2 = p.nx2[i];
    const float* xCi = p.xC + i * p.ldx;

    const int nch = (K + kWave - 1) / kWave;
    float s_err;
    int s_cand;
    bool flagged = false;
    // BEST: the first group is sorted into the empty top-H at once and ties at its boundary are
    // flagged, as in the later layers (the scan itself is the reference's code order).
    SelectTopH<false, BEST, BEST>(
        Hb, lane,
        [&](auto&& replay, auto, auto) {
            for (int j = 0; j < nch; ++j) {
                const int k = lane + kWave * j;
                const bool act = k < K;
                const float alpha = act ? p.gdiag[off0 + k] : 0.0f;
                const bool ok = act && alpha != 0.0f;
                const float gamma = act ? xCi[off0 + k] : 0.0f;
                const float a1 = gamma / alpha;
                const float e1 = nx2 - gamma * a1;
                if (!replay(ok, e1, kWave * j + lane)) return false;
            }
            return true;
        },
        s_err, s_cand, flagged);

    if (BEST && flagged) {  // re-run in the reference order; the next layers see an empty beam
        if (lane == 0) {
            p.flags[i] = 1;
            p.out.curH[w] = 0;
        }
        return;
    }
    const int curH = __popcll(__ballot(lane < Hb && s_err < kInfF));  // CountFinite, no max(1,.)
    if (BEST && p.is_last && FinalTie(s_err, curH)) {
        if (lane == 0) p.flags[i] = 1;
        return;
    }
    // Insertion-time write-back of the surviving slot contents (beam_search.cpp:253-258).
    uint8_t c0 = 0;
    float a0 = 0.0f, r00 = 0.0f;
    prune::SlotBounds bd = prune::NoBounds();
    if (lane < Hb && s_cand >= 0) {
        const float alpha = p.gdiag[off0 + s_cand];
        const float gamma = xCi[off0 + s_cand];
        c0 = static_cast<uint8_t>(s_cand);
        a0 = gamma / alpha;
        r00 = sqrtf(alpha);
        bd = prune::FirstBounds(r00, p.sw[off0 + s_cand], a0, p.isw[off0 + s_cand]);
    }
    if (lane < Hb) {
        float* rec = p.out.rec + (w * Hb + lane) * rc.stride;
        rec[0] = s_err;
        rec[rc.coef] = a0;
        rec[Rec::R(0, 0)] = r00;
        rec[Rec::Rinv(0)] = 1.0f / r00;
        reinterpret_cast<uint32_t*>(rec + rc.code)[0] = c0;
        reinterpret_cast<uint32_t*>(rec)[rc.root] = 0u;
        rc.PutBounds(rec, bd);
    }
    if (lane == 0) p.out.curH[w] = curH;
    if (p.is_last) {
        const int best = BestSlot(s_err, curH, lane);
        if (lane == best) {
            p.codes_out[i * m] = c0;
            if (p.best_err) p.best_err[i] = s_err;
        }
    }
}

// Last layer of the best-first pass (LayerKernel and LayerKernelStaged built with LAST): only the
// final pick leaves the layer, the first minimum over the top-H slots (beam_search.cpp:409-419).
// When the smallest eligible error is unique and finite, that candidate enters whenever it is
// scanned (every slot then holds a larger error) and is never evicted (it is never the worst), so
// it is the pick in any scan order. So the scan only tracks the running minimum, and the pruning
// bound tests against it: a pruned candidate's error exceeds the minimum of its moment, so it can
// neither be the pick nor tie with it. Everything else is flagged and re-run in the reference
// order: a tie for the minimum, an eligible NaN or -0, or no finite candidate (the all-skipped
// fallback).
struct LastPick {
    uint32_t best_img = 0x7F800000u;  // the minimum's float bits (+inf: nothing yet)
    int best_cand = -1;
    bool tie = false;
    // One group of candidates in scan order (lane = scan position); false: flag the vector.
    __device__ bool Take(bool ok, float e, int cand) {
        const uint32_t img = __float_as_uint(e);
        // errors are clamped at +0 here, so NaN and -0 are the images above +inf's
        if (Ballot(ok && img > 0x7F800000u) != 0ull) return false;
        const uint32_t mine = ok ? img : 0xFFFFFFFFu;
        const uint32_t mn = WaveMinU32(mine);
        if (mn >= 0x7F800000u) return true;  // no finite error in this group
        const uint64_t at = Ballot(mine == mn);
        if (mn < best_img) {
            best_img = mn;
            best_cand = __builtin_amdgcn_readlane(cand, static_cast<int>(__builtin_ctzll(at)));
            tie = __popcll(at) > 1;
        } else if (mn == best_img) {
            tie = true;
        }
        return true;
    }
    __device__ float Now() const { return __uint_as_float(best_img); }
};

// The pick's codes (and the large root's cluster id) and error, or the vector's re-run flag.
template <int L, bool LR>
__device__ __forceinline__ void WriteLastPick(bool fine, const LastPick& lp, const LayerArgs& p, const Rec& rc,
                                              const float* recs_in, int K, int64_t i, int lane) {
    if (lane != 0) return;
    if (!fine || lp.tie || lp.best_cand < 0) {
        p.flags[i] = 1;
        return;
    }
    const int m = p.m;
    const int src = lp.best_cand / K;
    const int knew = lp.best_cand - src * K;
    const float* ri = recs_in + src * rc.stride;
    if (LR) {
        p.cluster_out[i] = reinterpret_cast<const uint32_t*>(ri)[rc.root];
#pragma unroll
        for (int t = 1; t < L; ++t) p.codes_out[i * (m - 1) + (t - 1)] = CodeAt(ri, rc.code, t);
        p.codes_out[i * (m - 1) + (L - 1)] = static_cast<uint8_t>(knew);
    } else {
#pragma unroll
        for (int t = 0; t < L; ++t) p.codes_out[i * m + t] = CodeAt(ri, rc.code, t);
        p.codes_out[i * m + L] = static_cast<uint8_t>(knew);
    }
    if (p.best_err) p.best_err[i] = __uint_as_float(lp.best_img);
}

// Layers L >= 1. LR selects the large-root cross-term source and reciprocal solves.
// FULL: the layer has exactly 256 codewords (no partial chunk).
// Minimum waves per SIMD asked of the register allocator by the queue kernel (layers 1-8),
// measured on the M=8, K=256, beam-16 encode: layers 1-3 at 8, 4-5 at 7, 6 at 6 (7 waves ran 1%
// slower), 7 at 5 (the allocator alone gives it 101 VGPRs and 4 waves, 3% slower); the last layer's
// minimum-only build (LAST) of layer 7 at 6 (80 VGPRs with a small spill: 8.87 against 9.33 ms at
// 5 waves); layer 8 at the allocator's choice (4 waves). The large root: layers 1-2 at 8 (the best-first
// pass's sorted first group takes the SGPRs to 106, which gives 7), the others at the allocator's
// choice (forcing 6-8 waves ran 2-9% slower on the beam-32 encode).
template <int L, bool LR, bool BEST, bool LAST>
constexpr int LayerMinWaves() {
    if (LR) return L <= 2 ? 8 : 1;
    if (LAST && L == 7) return 6;
    return L <= 3 ? 8 : (L <= 5 ? 7 : (L == 6 ? 6 : (L == 7 ? 5 : 1)));
}

// Layers up to kVStateMaxL read the slot state into VGPRs (see process() in LayerKernel): on the
// M=8 and M=16 encodes that is 1-2% faster for layers 1-3 and slower from layer 4 on, where the
// extra VGPRs cost occupancy.
constexpr int kVStateMaxL = 3;

// Layers 1..kQueueMaxL scan through a queue (LayerKernel, scan_queue): the survivors of the pruning
// bound from every parent go into one FIFO and are evaluated 64 at a time, each lane reading its own
// parent's state from LDS. At layer 1 too: there a solve costs little more than the bound, but the
// queue's full groups and the staged state cut the layer from 5.7 to 4.2 ms on the M=8, beam-16
// encode against evaluating every candidate slot by slot.
constexpr int kQueueMaxL = 8;
constexpr int kQueueCap = 128;  // ring capacity: at most 63 carried over plus one chunk of 64
// Layers above kQueueMaxL run the staged kernel (pruned, factors staged in LDS a window of slots
// at a time), the full-precomp and the large-root beam alike.

// BEST: the best-first pass (LayerArgs::flags). Its input records are rank-indexed, so slots are
// scanned in ascending error order, and so are its output records. A vector flagged by an earlier
// layer arrives with an empty beam. LAST: built for the last layer of the best-first pass only
// (p.is_last): the running minimum of LastPick instead of the top-H, and no write-back (on the M=8,
// beam-16 encode the last layer took 9.35 against 11.38 ms).
template <int L, bool LR, bool FULL, bool BEST, bool LAST = false>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(LayerMinWaves<L, LR, BEST, LAST>(), 8))) void LayerKernel(
    LayerArgs p) {
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    int64_t i, w;
    if (!WaveItem(p, wave, i, w)) return;
    const int m = p.m, Hb = p.Hb, K = FULL ? kMaxK : p.K, offL = p.offL;
    const Rec rc(m);
    const int ld = p.gram.ld;
    const float* xCi = p.xC + i * p.ldx;
    const int nch = FULL ? kMaxChunks : (K + kWave - 1) / kWave;
    const float* __restrict__ recs_in = p.in.rec + w * Hb * rc.stride;
    float* __restrict__ recs_out = p.out.rec + w * Hb * rc.stride;
    const int vz = VZero();


    // Per codeword of the layer: gamma = <x, c_k> and fl(alpha (1 - 2^-20)) for the pruning bound.
    float gam[kMaxChunks], alc[kMaxChunks];
#pragma unroll
    for (int j = 0; j < kMaxChunks; ++j) {
        const int k = lane + kWave * j;
        const bool act = FULL || (j < nch && k < K);
        gam[j] = act ? xCi[offL + k] : 0.0f;
        alc[j] = (act ? p.gdiag[offL + k] : 0.0f) * prune::kAlphaScale;
    }

    const int curH = p.in.curH[w];

    // Beam slot h's codes (and root) sit in lane h, read with one vector load per word for all
    // slots at once, so a slot's G rows can be addressed without waiting for its record.
    constexpr int kCodeWords = (L + 3) / 4;
    uint32_t cw[kCodeWords];
    uint32_t rootw = 0;
    {
        const uint32_t* rl = reinterpret_cast<const uint32_t*>(recs_in + (lane < curH ? lane : 0) * rc.stride);
#pragma unroll
        for (int w = 0; w < kCodeWords; ++w) cw[w] = rl[rc.code + w];
        if (LR) rootw = rl[rc.root];
    }
    // Per wave: the layer's codewords that go to the exact evaluation, in scan order.
    __shared__ int s_pack[kBeamWavesPerBlock][kMaxK];
    int* __restrict__ pack = s_pack[wave];
    const bool prune_on = p.prune != 0;

    // The queue scan's exact evaluations read each lane's parent state from LDS (QStage), staged
    // here for every slot: the factor is then read row by row as the solves need it (EvalStaged)
    // instead of being held whole in registers, which keeps the kernel's VGPRs, and so its
    // occupancy, near the bound stage's. The write-back reads each new slot's parent from here too.
    // diag_mask bit h: slot h's diagonal is in the range where the Markstein quotients are exact.
    HIP_DYNAMIC_SHARED(float, s_stage)
    float* __restrict__ stage = s_stage + static_cast<size_t>(wave) * Hb * QStage<L>::kStride;
    uint64_t diag_mask = 0;
    {
        constexpr int kW = QStage<L>::kEold + 1;
        for (int q = lane; q < curH * kW; q += kWave) {
            const int h = q / kW, o = q - h * kW;
            const float* src = recs_in + h * rc.stride;
            stage[h * QStage<L>::kStride + o] =
                o < QStage<L>::kRWords ? src[1 + o] : (o < QStage<L>::kEold ? src[rc.coef + o - QStage<L>::kRWords] : src[0]);
        }
        // the bound's operands: one pass over all slots here instead of a dependent isw[f] gather
        // per slot in the scan
        for (int q = lane; q < curH * QStage<L>::kBoundWords; q += kWave) {
            const int h = q / QStage<L>::kBoundWords, o = q - h * QStage<L>::kBoundWords;
            const float* src = recs_in + h * rc.stride;
            float val;
            if (o < L) {
                const float isw_t = (LR && o == 0) ? p.isw0[reinterpret_cast<const uint32_t*>(src)[rc.root]]
                                                   : p.isw[p.gram.off[o] + CodeAt(src, rc.code, o)];
                val = src[rc.coef + o] * isw_t;
            } else if (o == L) {
                val = src[rc.kb];
            } else if (o == L + 1) {
                val = src[rc.cq];
            } else {
                val = LR ? p.sw0[reinterpret_cast<const uint32_t*>(src)[rc.root]] : 1.0f;
            }
            stage[h * QStage<L>::kStride + QStage<L>::kAhat + o] = val;
        }
        bool dok = lane < curH;
        if (dok) {
            const float* src = recs_in + lane * rc.stride;
#pragma unroll
            for (int r = 0; r < L; ++r) dok = dok && DiagFastOk(src[Rec::R(r, r)]);
        }
        diag_mask = Ballot(dok);
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }

    // Evaluates slot h's candidates and replays them into the top-H (scan order: slot, then code).
    // Returns false when the replay asks for the slow pass.
    //
    // Pruning (prune_bound.hpp): once every slot of the top-H holds a candidate, a candidate whose
    // bound shows e > worst is one the reference rejects; the others are listed in `pack` in
    // ascending code order and evaluated exactly, 64 per group. While a slot is still empty the
    // chunks are listed one at a time without a bound, so the worst can become finite after each.
    auto process = [&](int h, auto&& replay, auto slow_tag, auto&& worst_now) -> bool {
        constexpr bool kSlow = decltype(slow_tag)::value;
        const float* rec = recs_in + h * rc.stride;
        const float E_old = rec[0];
        // Rows of the slot's prefix codewords from this layer's first column: G for the exact
        // evaluation, Gs (rows scaled by sw) for the bound. The large root's prefix 0 reads
        // G0S(root, .), scaled by sw0[root] in the bound.
        const float* rowb[L];
        const float* rows[L];
        float ahat[L];  // a_t * isw_t
        float cdg[L];   // c_t of the diagonal split
        uint32_t root = 0;
#pragma unroll
        for (int t = 0; t < L; ++t) {
            float isw_t;
            if (LR && t == 0) {
                root = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(rootw), h));
                rowb[t] = p.gram.G0S + static_cast<int64_t>(root) * ld + offL;
                rows[t] = rowb[t];
                isw_t = p.isw0[root];
            } else {
                const uint32_t word = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(cw[t >> 2]), h));
                const int f = p.gram.off[t] + static_cast<int>((word >> (8 * (t & 3))) & 0xFFu);
                rowb[t] = p.gram.G + static_cast<int64_t>(f) * ld + offL;
                rows[t] = p.Gs + static_cast<int64_t>(f) * ld + offL;
                isw_t = p.isw[f];
            }
            ahat[t] = rec[rc.coef + t] * isw_t;
            cdg[t] = prune::DiagCoef(rec[Rec::Rinv(t)], isw_t);
        }
        const float sw0 = LR ? p.sw0[root] : 1.0f;
        const float kb = rec[rc.kb], cq = rec[rc.cq];
        const float k1 = L >= prune::kDiagMinL ? rec[rc.k1] : 0.0f, k2 = L >= prune::kDiagMinL ? rec[rc.k2] : 0.0f;

        int next = 0;  // first chunk not yet listed
        while (next < nch) {
            float gp = 0.0f;
            const float W = worst_now();
            const bool bounded = !kSlow && prune_on && kb < kInfF && prune::ParentGap(E_old, W, gp);
            const bool filling = !kSlow && prune_on && !(W < kInfF);
            const int last = (bounded || !filling) ? nch : next + 1;
            int total = 0;
            // One chunk at a time (no unrolling): the bound stage then holds one chunk's L values.
#pragma unroll 1
            for (int j = next; j < last; ++j) {
                const int k = lane + kWave * j;
                const bool act = FULL || k < K;
                bool keep = act;
                if (bounded) {
                    // eta~ = sum_t b_t ahat_t, b2 = sum_t b_t^2 and X~ = sum_t (c_t b_t)^2 by fma,
                    // b_t = Gs(f_t, k)
                    float et = 0.0f, b2 = 0.0f, xs = 0.0f;
#pragma unroll
                    for (int t = 0; t < L; ++t) {
                        float bt = act ? rows[t][static_cast<uint32_t>(k)] : 0.0f;
                        if (LR && t == 0) bt = bt * sw0;
                        et = t == 0 ? bt * ahat[t] : __builtin_fmaf(bt, ahat[t], et);
                        b2 = t == 0 ? bt * bt : __builtin_fmaf(bt, bt, b2);
                        if (L >= prune::kDiagMinL) {
                            const float ut = cdg[t] * bt;
                            xs = t == 0 ? ut * ut : __builtin_fmaf(ut, ut, xs);
                        }
                    }
                    const float alc = (act ? p.gdiag[offL + k] : 0.0f) * prune::kAlphaScale;
                    const float gm = act ? xCi[offL + k] : 0.0f;
                    keep = act && !(L >= prune::kDiagMinL ? prune::Prunable2(alc, b2, xs, gm - et, kb, k1, k2, cq, gp)
                                                   : prune::Prunable(alc, b2, gm - et, kb, cq, gp));
                }
                const uint64_t km = Ballot(keep);
                if (keep) pack[total + __popcll(km & ((1ull << lane) - 1ull))] = k;
                total += __popcll(km);
            }
            next = last;
            if (total == 0) continue;
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            // The slot's R, 1/diag and coefficients (wave-uniform) for the exact evaluation. Up to
            // kVStateMaxL they are read into VGPRs, so the solves' products have two VGPR
            // sources; beyond it they stay in SGPRs, where they cost no occupancy.
            const float* recv = kVStateMaxL >= L ? rec + vz : rec;
            float aold[L];
            float Rv[L][L];
            float Ri[L];
#pragma unroll
            for (int t = 0; t < L; ++t) aold[t] = recv[rc.coef + t];
            bool diag_ok = true;
#pragma unroll
            for (int r = 0; r < L; ++r) {
#pragma unroll
                for (int c = r; c < L; ++c) Rv[r][c] = recv[Rec::R(r, c)];
                Ri[r] = recv[Rec::Rinv(r)];
                diag_ok = diag_ok && DiagFastOk(Rv[r][r]);
            }
            const bool diag_fast = !LR && Ballot(!diag_ok) == 0ull;
            auto Rf = [&](int r, int c) { return Rv[r][c]; };
            for (int b = 0; b < total; b += kWave) {
                const int idx = b + lane;
                const bool act = idx < total;
                const uint32_t k = static_cast<uint32_t>(act ? pack[idx] : 0);
                float A[L];
#pragma unroll
                for (int t = 0; t < L; ++t) A[t] = rowb[t][k];
                const float alpha = p.gdiag[offL + k];
                const float gamma = xCi[offL + k];
                float y[L], v[L], denom, a_last, e;
                bool ok, safe = true;
                if (LR) {
                    EvalCand<L, 2>(Rf, Ri, A, aold, E_old, alpha, gamma, y, v, e, denom, a_last, ok, safe);
                } else {
                    // Markstein quotients where they are exact (every numerator in range), IEEE
                    // division otherwise (the rare slow pass, a diagonal out of range, or a
                    // numerator that left the range: the group is evaluated again).
                    bool ieee = kSlow || !diag_fast;
                    if (!ieee) {
                        EvalCand<L, 1>(Rf, Ri, A, aold, E_old, alpha, gamma, y, v, e, denom, a_last, ok, safe);
                        ieee = Ballot(!safe) != 0ull;
                    }
                    if (ieee) EvalCand<L, 0>(Rf, Ri, A, aold, E_old, alpha, gamma, y, v, e, denom, a_last, ok, safe);
                }
                if (!replay(ok && act, e, h * K + static_cast<int>(k))) return false;
            }
        }
        return true;
    };

    // The queue scan (layers up to kQueueMaxL, fast pass with pruning): candidates are bound-
    // tested chunk by chunk in scan order against the worst of that moment, the survivors
    // (parent h, codeword k) are appended to a per-wave FIFO in scan order, and every full 64 of
    // them (then the rest) are evaluated exactly and replayed. The worst only falls between a
    // test and the evaluation, so a pruned candidate stays one the reference rejects.
    __shared__ int s_queue[kBeamWavesPerBlock][kQueueCap];
    int* __restrict__ queue = s_queue[wave];
    auto scan_queue = [&](auto&& replay, auto&& worst_now) -> bool {
        int qhead = 0, qlen = 0;
        const __amdgpu_buffer_rsrc_t g_rsrc = GramRsrc(p.gram.G, ld);
        const __amdgpu_buffer_rsrc_t gs_rsrc = GramRsrc(p.Gs, ld);
        // Exact evaluation of the first n queued candidates, one per lane, each with its own
        // parent's state.
        auto flush = [&](int n) -> bool {
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            const bool act = lane < n;
            const int ent = act ? queue[(qhead + lane) & (kQueueCap - 1)] : 0;
            const int hl = ent >> 8;
            const uint32_t k = static_cast<uint32_t>(ent & 0xFF);
            const float* f = stage + hl * QStage<L>::kStride;
            float A[L];
            const bool diag_ok = ((diag_mask >> hl) & 1ull) != 0ull;
            const float E_old = f[QStage<L>::kEold];
            const uint32_t rootl =
                LR ? static_cast<uint32_t>(__builtin_amdgcn_ds_bpermute(hl << 2, static_cast<int>(rootw))) : 0u;
            // the parent's codes from its lane (lane h holds slot h's code words)
            uint32_t cwl[kCodeWords];
#pragma unroll
            for (int q = 0; q < kCodeWords; ++q)
                cwl[q] = static_cast<uint32_t>(__builtin_amdgcn_ds_bpermute(hl << 2, static_cast<int>(cw[q])));
            const uint32_t kb4 = (k + static_cast<uint32_t>(offL)) * 4u;
#pragma unroll
            for (int t = 0; t < L; ++t) {
                const uint32_t code = (cwl[t >> 2] >> (8 * (t & 3))) & 0xFFu;
                if (LR && t == 0) {
                    A[t] = p.gram.G0S[static_cast<int64_t>(rootl) * ld + offL + k];
                } else {
                    const uint32_t f = static_cast<uint32_t>(p.gram.off[t]) + code;
                    A[t] = GramLd(g_rsrc, f * static_cast<uint32_t>(ld) * 4u + kb4, 0u);
                }
            }
            const float alpha = p.gdiag[offL + k];
            const float gamma = xCi[offL + k];
            float y[L], v[L], denom, a_last, e;
            bool ok, safe = true;
            if (LR) {
                EvalStaged<L, 2>(f, A, E_old, alpha, gamma, y, v, e, denom, a_last, ok, safe);
            } else {
                bool ieee = Ballot(act && !diag_ok) != 0ull;
                if (!ieee) {
                    EvalStaged<L, 1>(f, A, E_old, alpha, gamma, y, v, e, denom, a_last, ok, safe);
                    ieee = Ballot(act && !safe) != 0ull;
                }
                if (ieee) EvalStaged<L, 0>(f, A, E_old, alpha, gamma, y, v, e, denom, a_last, ok, safe);
            }
            qhead = (qhead + n) & (kQueueCap - 1);
            qlen -= n;
            return replay(ok && act, e, hl * K + static_cast<int>(k));
        };
        static_assert(kQueueMaxL < prune::kDiagMinL, "the queue scan uses the Frobenius bound only");
        for (int h = 0; h < curH; ++h) {
            // The slot's bound operands, staged in LDS (wave-uniform reads).
            const float* sp = stage + h * QStage<L>::kStride;
            const float E_old = Uniform(sp[QStage<L>::kEold]);
            const float kb = Uniform(sp[QStage<L>::kKb]), cq = Uniform(sp[QStage<L>::kCq]);
            float ahat[L];
#pragma unroll
            for (int t = 0; t < L; ++t) ahat[t] = sp[QStage<L>::kAhat + t];
            const float sw0 = LR ? sp[QStage<L>::kSw0] : 1.0f;
            // Gs row byte offsets of the slot's prefix codewords (the large root's prefix 0:
            // G0S(root, .), scaled by sw0[root] in the bound).
            uint32_t rowb[L];
            const float* row0 = nullptr;
#pragma unroll
            for (int t = 0; t < L; ++t) {
                rowb[t] = 0;
                if (LR && t == 0) {
                    const uint32_t root = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(rootw), h));
                    row0 = p.gram.G0S + static_cast<int64_t>(root) * ld + offL;
                } else {
                    const uint32_t word =
                        static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(cw[t >> 2]), h));
                    const uint32_t f = static_cast<uint32_t>(p.gram.off[t]) + ((word >> (8 * (t & 3))) & 0xFFu);
                    rowb[t] = f * static_cast<uint32_t>(ld) * 4u;
                }
            }
            // b_t = Gs(f_t, k) of chunk j's codeword k = lane + 64 j. Reads past the Gram return 0
            // (buffer range check); a codeword beyond K is masked by the caller.
            auto gs_of = [&](int j, int t) -> float {
                const uint32_t k = static_cast<uint32_t>(lane + kWave * j);
                if (LR && t == 0) return (FULL || static_cast<int>(k) < K) ? row0[k] * sw0 : 0.0f;
                return GramLd(gs_rsrc, (k + static_cast<uint32_t>(offL)) * 4u, rowb[t]);
            };
            // Whether chunk j's candidate survives the bound (true when it may enter the top-H):
            // eta~ = sum_t b_t ahat_t and b2 = sum_t b_t^2 by fma.
            auto keep_b = [&](int j, const float (&b)[L], float gp) -> bool {
                const bool act = FULL || lane + kWave * j < K;
                float et = 0.0f, b2 = 0.0f;
#pragma unroll
                for (int t = 0; t < L; ++t) {
                    et = t == 0 ? b[t] * ahat[t] : __builtin_fmaf(b[t], ahat[t], et);
                    b2 = t == 0 ? b[t] * b[t] : __builtin_fmaf(b[t], b[t], b2);
                }
                return act && !prune::Prunable(alc[j], b2, gam[j] - et, kb, cq, gp);
            };
            auto enqueue = [&](int j, bool keep, uint64_t km) -> bool {
                if (keep) {
                    const int pos = (qhead + qlen + __popcll(km & ((1ull << lane) - 1ull))) & (kQueueCap - 1);
                    queue[pos] = (h << 8) | (lane + kWave * j);
                }
                qlen += __popcll(km);
                return qlen < kWave || flush(kWave);
            };
            const float W0 = worst_now();
            if (!(W0 < kInfF)) {
                // A slot is still empty: chunk by chunk, each tested against the worst after the
                // previous one was evaluated.
                for (int j = 0; j < nch; ++j) {
                    const bool act = FULL || lane + kWave * j < K;
                    float gp = 0.0f;
                    const bool bounded = kb < kInfF && prune::ParentGap(E_old, worst_now(), gp);
                    bool keep = act;
#pragma unroll
                    for (int jj = 0; jj < kMaxChunks; ++jj) {
                        if (jj == j && bounded) {
                            float b[L];
#pragma unroll
                            for (int t = 0; t < L; ++t) b[t] = gs_of(jj, t);
                            keep = keep_b(jj, b, gp);
                        }
                    }
                    if (!enqueue(j, keep, Ballot(keep))) return false;
                }
            } else {
                // The whole slot against the worst at its start (it only falls from there). Every
                // chunk's values are read in one go and tested without branches, so the slot costs
                // one memory round trip; the tests are discarded when the slot is not bounded.
                float b[kMaxChunks][L];
#pragma unroll
                for (int j = 0; j < kMaxChunks; ++j) {
                    if (!FULL && j >= nch) continue;
#pragma unroll
                    for (int t = 0; t < L; ++t) b[j][t] = gs_of(j, t);
                }
                float gp = 0.0f;
                const bool bounded = kb < kInfF && prune::ParentGap(E_old, W0, gp);
                // All four ballots before the first enqueue: the tests cannot then be moved past
                // a flush, where their operands would hold registers.
                bool keep[kMaxChunks];
                uint64_t km[kMaxChunks];
#pragma unroll
                for (int j = 0; j < kMaxChunks; ++j) {
                    if (!FULL && j >= nch) continue;
                    const bool kt = keep_b(j, b[j], gp);
                    keep[j] = bounded ? kt : (FULL || lane + kWave * j < K);
                    km[j] = Ballot(keep[j]);
                }
#pragma unroll
                for (int j = 0; j < kMaxChunks; ++j) {
                    if (!FULL && j >= nch) continue;
                    if (!enqueue(j, keep[j], km[j])) return false;
                }
            }
        }
        if (qlen > 0 && !flush(qlen)) return false;
        return true;
    };

    if constexpr (LAST && BEST) {
        if (prune_on) {  // the final pick only (LastPick)
            LastPick lp;
            auto track = [&](bool ok, float e, int cand) { return lp.Take(ok, e, cand); };
            auto min_now = [&]() { return lp.Now(); };
            const bool fine = scan_queue(track, min_now);
            WriteLastPick<L, LR>(fine, lp, p, rc, recs_in, K, i, lane);
            return;
        }
    }

    float s_err;
    int s_cand;
    bool flagged = false;
    SelectTopH<true, BEST, BEST>(  // errors clamped at zero (EvalCand)
        Hb, lane,
        [&](auto&& replay, auto slow_tag, auto&& worst_now) {
            if constexpr (L <= kQueueMaxL && !decltype(slow_tag)::value) {
                if (prune_on) return scan_queue(replay, worst_now);
            }
            for (int h = 0; h < curH; ++h) {
                if (!process(h, replay, slow_tag, worst_now)) return false;
            }
            return true;
        },
        s_err, s_cand, flagged);
    if (BEST && flagged) {
        // No records: the next layers see an empty beam (curH = 0), do no work for this vector
        // and keep it well-formed until its re-run.
        if (lane == 0) {
            p.flags[i] = 1;
            p.out.curH[w] = 0;
        }
        return;
    }

    // Deferred write-back (beam_search.cpp:337-383; the large root :896-947) or the all-skipped
    // fallback (:385-400, :949-966). A slot holding a candidate is built even when its error is
    // NaN (Materialize skips only errors >= +inf); the beam's new size counts the finite errors
    // (CountFinite), and with none the parent slots are copied instead. The last layer needs no
    // records, only the final pick.
    const bool live = lane < Hb && !(s_err >= kInfF);
    const int newH = __popcll(Ballot(lane < Hb && s_err < kInfF));
    const int outH = newH == 0 ? max(1, min(curH, Hb)) : newH;  // CountFinite and max(1, .)
    if (lane == 0) p.out.curH[w] = outH;
    float out_err = kInfF;
    int src = -1, knew = 0;
    if (newH == 0) {
        if (lane < min(curH, Hb)) {
            src = lane;
            out_err = recs_in[lane * rc.stride];
        }
    } else if (live) {
        src = s_cand / K;
        knew = s_cand - src * K;
        out_err = s_err;
    }
    if (!LAST && !p.is_last) {
        float* ro = recs_out + lane * rc.stride;
        const float* ri = recs_in + (src < 0 ? 0 : src) * rc.stride;
        // the parent's code words (and root) from the lane that holds them, the whole wave active
        const int srcl = (src < 0 ? 0 : src) << 2;
        uint32_t pcw[kCodeWords];
#pragma unroll
        for (int q = 0; q < kCodeWords; ++q)
            pcw[q] = static_cast<uint32_t>(__builtin_amdgcn_ds_bpermute(srcl, static_cast<int>(cw[q])));
        const uint32_t prootw =
            LR ? static_cast<uint32_t>(__builtin_amdgcn_ds_bpermute(srcl, static_cast<int>(rootw))) : 0u;
        auto put_codes = [&](bool from_parent, int kc, uint32_t root) {
            uint32_t* cwo = reinterpret_cast<uint32_t*>(ro + rc.code);
#pragma unroll
            for (int qq = 0; qq <= L / 4; ++qq) {
                uint32_t word = 0;
#pragma unroll
                for (int b = 0; b < 4; ++b) {
                    const int t = 4 * qq + b;
                    const uint32_t c = t < L ? (from_parent ? static_cast<uint32_t>(CodeAt(ri, rc.code, t)) : 0u)
                                             : (t == L ? static_cast<uint32_t>(kc) : 0u);
                    word |= c << (8 * b);
                }
                cwo[qq] = word;
            }
            reinterpret_cast<uint32_t*>(ro)[rc.root] = root;
        };
        if (newH == 0) {
            const int nh = min(curH, Hb);
            if (lane < nh) {
                // parent slot `lane` with a zero new column
                ro[0] = ri[0];
#pragma unroll
                for (int t = 0; t < L; ++t) ro[rc.coef + t] = ri[rc.coef + t];
                ro[rc.coef + L] = 0.0f;
#pragma unroll
                for (int r = 0; r < L; ++r) {
#pragma unroll
                    for (int c = r; c < L; ++c) ro[Rec::R(r, c)] = ri[Rec::R(r, c)];
                    ro[Rec::R(r, L)] = 0.0f;
                    ro[Rec::Rinv(r)] = ri[Rec::Rinv(r)];
                }
                ro[Rec::R(L, L)] = 0.0f;
                ro[Rec::Rinv(L)] = 1.0f / 0.0f;
                put_codes(true, 0, reinterpret_cast<const uint32_t*>(ri)[rc.root]);
                rc.PutBounds(ro, prune::NoBounds());
            } else if (nh == 0 && lane == 0) {
                // No beam at all (layer 0 had no finite candidate): the reference's next-buffer
                // slot 0 keeps its never-written (zero) state with error +inf.
                ro[0] = kInfF;
#pragma unroll
                for (int t = 0; t <= L; ++t) ro[rc.coef + t] = 0.0f;
#pragma unroll
                for (int r = 0; r <= L; ++r) {
#pragma unroll
                    for (int c = r; c <= L; ++c) ro[Rec::R(r, c)] = 0.0f;
                    ro[Rec::Rinv(r)] = 1.0f / 0.0f;
                }
                put_codes(false, 0, 0u);
                rc.PutBounds(ro, prune::NoBounds());
            }
        } else if (live) {
            // The chosen candidate once more with the reference's arithmetic (IEEE division, or the
            // large root's reciprocal multiply): its new coefficients, Cholesky column and bounds.
            // The parent's factor, coefficients and error come from the LDS stage and its codes
            // from the lane that holds them (no per-lane gathers from the parent's record); the
            // record's first columns, at offsets fixed by L, leave as 16-byte stores.
            const float* sf = stage + src * QStage<L>::kStride;
            const uint32_t root = LR ? prootw : 0u;
            float A[L];
            int fl[L];  // flat index of each prefix codeword (the root for a large root's prefix 0)
#pragma unroll
            for (int t = 0; t < L; ++t) {
                const uint32_t code = (pcw[t >> 2] >> (8 * (t & 3))) & 0xFFu;
                fl[t] = (LR && t == 0) ? static_cast<int>(root) : p.gram.off[t] + static_cast<int>(code);
                const float* row = (LR && t == 0) ? p.gram.G0S + static_cast<int64_t>(root) * ld + offL
                                                  : p.gram.G + static_cast<int64_t>(fl[t]) * ld + offL;
                A[t] = row[knew];
            }
            // EvalCand's operations on the staged factor (IEEE division, or the large root's
            // reciprocal multiply), so no copy of the factor is held in registers
            const float E_old = sf[QStage<L>::kEold];
            float y[L], v[L], e, denom, a_last;
            bool ok, unused = true;
            if (LR) {
                EvalStaged<L, 2>(sf, A, E_old, p.gdiag[offL + knew], xCi[offL + knew], y, v, e, denom, a_last, ok,
                                 unused);
            } else {
                EvalStaged<L, 0>(sf, A, E_old, p.gdiag[offL + knew], xCi[offL + knew], y, v, e, denom, a_last, ok,
                                 unused);
            }
            double asq = 0.0;  // ||ahat||^2 of the new coefficients
#pragma unroll
            for (int t = 0; t <= L; ++t) {
                const float at = t < L ? sf[QStage<L>::kRWords + t] - v[t] * a_last : a_last;
                ro[rc.coef + t] = at;
                const float iswt = t < L ? ((LR && t == 0) ? p.isw0[fl[t]] : p.isw[fl[t]]) : p.isw[offL + knew];
                const double ah = static_cast<double>(at) * static_cast<double>(iswt);
                asq += ah * ah;
            }
            const float rLL = sqrtf(denom);
            // Dwords 0 .. Rinv(L): the error and columns 0..L of the factor with their 1/diag,
            // rounded up to whole 16-byte words. The padding falls in column L+1 (L < m-1 here),
            // which the next layer writes into its own output and never reads from this record.
            constexpr int kHead = (Rec::Rinv(L) + 1 + 3) / 4;
            float hd[4 * kHead];
#pragma unroll
            for (int q = 0; q < 4 * kHead; ++q) hd[q] = 0.0f;
            hd[0] = s_err;
#pragma unroll
            for (int q = 1; q <= QStage<L>::kRWords; ++q) hd[q] = sf[q - 1];  // columns 0..L-1
#pragma unroll
            for (int r = 0; r < L; ++r) hd[Rec::R(r, L)] = y[r];
            hd[Rec::R(L, L)] = rLL;
            hd[Rec::Rinv(L)] = 1.0f / rLL;
            float4* ro4 = reinterpret_cast<float4*>(ro);
#pragma unroll
            for (int q = 0; q < kHead; ++q) ro4[q] = make_float4(hd[4 * q], hd[4 * q + 1], hd[4 * q + 2], hd[4 * q + 3]);
            // the parent's code bytes below L, the new code at L, zeros above (as put_codes)
            uint32_t* cwo = reinterpret_cast<uint32_t*>(ro + rc.code);
#pragma unroll
            for (int qq = 0; qq <= L / 4; ++qq) {
                const uint32_t low = qq < L / 4 ? 0xFFFFFFFFu : ((1u << (8 * (L & 3))) - 1u);
                const uint32_t par = qq < kCodeWords ? pcw[qq < kCodeWords ? qq : 0] & low : 0u;
                cwo[qq] = par | (qq == L / 4 ? static_cast<uint32_t>(knew) << (8 * (L & 3)) : 0u);
            }
            reinterpret_cast<uint32_t*>(ro)[rc.root] = root;
            auto swf = [&](int t) { return (LR && t == 0) ? p.sw0[fl[t]] : p.sw[fl[t]]; };
            rc.PutBounds(ro, prune::NextBounds<L>(y, v, rLL, swf, p.sw[offL + knew], ri[rc.kap], ri[rc.phi], rc.Nf2(ri),
                                                  asq));
        } else if (lane < Hb) {
            ro[0] = kInfF;  // an empty slot: never read by the next layer
        }
        return;
    }

    // Last layer: the final pick (beam_search.cpp:409-419) over the slots the write-back would
    // build; with no finite candidate (the fallback) those are the parent slots with code 0.
    if (BEST && FinalTie(out_err, outH)) {
        if (lane == 0) p.flags[i] = 1;
        return;
    }
    const int best = BestSlot(out_err, outH, lane);
    if (lane == best) {
        // src < 0: no beam at all (the reference's never-written slot 0: codes 0, error +inf)
        const float* ri = recs_in + (src < 0 ? 0 : src) * rc.stride;
        const uint32_t root = src < 0 ? 0u : reinterpret_cast<const uint32_t*>(ri)[rc.root];
        if (LR) {
            p.cluster_out[i] = root;
#pragma unroll
            for (int t = 1; t < L; ++t) p.codes_out[i * (m - 1) + (t - 1)] = src < 0 ? 0 : CodeAt(ri, rc.code, t);
            p.codes_out[i * (m - 1) + (L - 1)] = static_cast<uint8_t>(knew);
        } else {
#pragma unroll
            for (int t = 0; t < L; ++t) p.codes_out[i * m + t] = src < 0 ? 0 : CodeAt(ri, rc.code, t);
            p.codes_out[i * m + L] = static_cast<uint8_t>(knew);
        }
        if (p.best_err) p.best_err[i] = out_err;
    }
}

// Layers above kQueueMaxL (the deep layers of the M=16 and large-root encodes). Per slot of the
// beam, the candidates are bound-tested chunk by chunk (prune_bound.hpp) and the survivors listed
// in ascending code order, then solved 64 at a time with the slot's factor, 1/diag and
// coefficients staged once in the wave's LDS. Every lane reads the same LDS address, so the
// solves' products take VGPR operands and the factor holds no registers (a factor in SGPRs or
// VGPRs would outgrow the register files from layer 11 on). The new slots are written back with
// the parents' factor columns copied by the whole wave, coalesced, and each new column solved by
// the lane that owns the slot, reading its parent's factor from memory.
template <int L>
constexpr int StagedWords() {
    return L * (L + 3) / 2 + L;  // R(0..c, c) and 1/R(c,c) for c < L (record dwords 1..), then a_old
}
constexpr int kWbSlots = 8;  // slots whose new column is solved per write-back round
template <int L>
constexpr int WbStride() {
    return StagedWords<L>() | 1;  // odd: the lanes of a round read distinct banks
}
// Deepest large-root staged layer whose best-first pass sorts its first group into the empty top-H
// (ReplayFast): on the large-root beam-32 encode layers 15 and 16 ran 3% and 2% slower with it,
// its layers up to 14 and every layer of the M=16, beam-8 encode 1-3% faster.
constexpr int kLrSortFirstMaxL = 14;
// The windowed queue scan stages kStagedWin slots at a time: factor, a_old and error per slot (odd
// stride: the lanes of a group read distinct banks), then ahat and c per slot, after the FIFO.
constexpr int kStagedWin = 8;
template <int L>
constexpr int StagedQStride() {
    return (StagedWords<L>() + 1) | 1;
}
template <int L>
constexpr int StagedWaveWords() {
    constexpr int scan = kMaxK + StagedWords<L>() + 2 * L;
    constexpr int win = kQueueCap + kStagedWin * (StagedQStride<L>() + 2 * L);
    constexpr int wb = kWbSlots * WbStride<L>();
    return scan > win ? (scan > wb ? scan : wb) : (win > wb ? win : wb);
}

// Waves per SIMD asked of the register allocator: the kernel needs about 5L + 60 VGPRs, so 4 waves
// (128) hold it without spills up to layer 10 and with spills of up to 46 VGPRs above, 3 waves
// (168) without spills up to layer 18. 4 waves up to layer 16 ran layers 13-16 5-15% faster than 3
// on the large-root beam-32 encode and the M=16, beam-8 encode (the large root's layer 15: 84.3
// against 92.5 ms per 1M vectors); 5 waves at layers 9-10 ran 8-9% slower. The last layer's
// minimum-only build (LAST) takes the same setting.
template <int L>
constexpr int StagedMinWaves() {
    return L <= 16 ? 4 : 3;
}

// LAST: built for the last layer of the best-first pass only (LastPick), as LayerKernel's.
template <int L, bool LR, bool FULL, bool BEST, bool LAST = false>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(StagedMinWaves<L>(), 8))) void LayerKernelStaged(
    LayerArgs p) {
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    int64_t i, w;
    if (!WaveItem(p, wave, i, w)) return;
    const int m = p.m, Hb = p.Hb, K = FULL ? kMaxK : p.K, offL = p.offL;
    const Rec rc(m);
    const int ld = p.gram.ld;
    const float* xCi = p.xC + i * p.ldx;
    const int nch = FULL ? kMaxChunks : (K + kWave - 1) / kWave;
    const float* __restrict__ recs_in = p.in.rec + w * Hb * rc.stride;
    float* __restrict__ recs_out = p.out.rec + w * Hb * rc.stride;
    const bool prune_on = p.prune != 0;

    // Per codeword of the layer: gamma = <x, c_k> and fl(alpha (1 - 2^-20)) for the pruning bound.
    float gam[kMaxChunks], alc[kMaxChunks];
#pragma unroll
    for (int j = 0; j < kMaxChunks; ++j) {
        const int k = lane + kWave * j;
        const bool act = FULL || (j < nch && k < K);
        gam[j] = act ? xCi[offL + k] : 0.0f;
        alc[j] = (act ? p.gdiag[offL + k] : 0.0f) * prune::kAlphaScale;
    }

    const int curH = p.in.curH[w];
    // Beam slot h's codes (and root) sit in lane h.
    constexpr int kCodeWords = (L + 3) / 4;
    uint32_t cw[kCodeWords];
    uint32_t rootw = 0;
    {
        const uint32_t* rl = reinterpret_cast<const uint32_t*>(recs_in + (lane < curH ? lane : 0) * rc.stride);
#pragma unroll
        for (int q = 0; q < kCodeWords; ++q) cw[q] = rl[rc.code + q];
        if (LR) rootw = rl[rc.root];
    }
    constexpr int kRWords = L * (L + 3) / 2;
    // Per wave: the survivor list and the staged factor during the scan, the write-back's staged
    // factors after it.
    __shared__ float s_wave[kBeamWavesPerBlock][StagedWaveWords<L>()];
    float* __restrict__ wbuf = s_wave[wave];
    int* __restrict__ pack = reinterpret_cast<int*>(wbuf);
    float* __restrict__ fac = wbuf + kMaxK;
    float* __restrict__ cf = fac + StagedWords<L>();  // per slot: ahat[L], then c[L]

    // 32-bit byte offsets from one base (H <= 5120, so H * ld * 4 < 2^32): the loads take the
    // scalar-base form with one VGPR offset instead of a 64-bit address per row.
    auto ld32 = [](const float* base, uint32_t elem) {
        return *reinterpret_cast<const float*>(reinterpret_cast<const char*>(base) + (elem << 2));
    };
    // Evaluates slot h's candidates and replays them into the top-H (scan order: slot, then code).
    // Returns false when the replay asks for the slow pass. While a slot of the top-H is still
    // empty the chunks are listed one at a time without a bound, so the worst can become finite
    // after each; after that every chunk is bound-tested against the worst of that moment.
    auto process = [&](int h, auto&& replay, auto slow_tag, auto&& worst_now) -> bool {
        constexpr bool kSlow = decltype(slow_tag)::value;
        const float* rec = recs_in + h * rc.stride;
        const float E_old = rec[0];
        // Element offsets of the slot's prefix rows in G (and Gs, same layout); the large root's
        // prefix 0 reads G0S(root, .), scaled by sw0[root] in the bound. ahat_t = a_t * isw_t.
        uint32_t rowo[L];
        const float* row0 = nullptr;
        float sw0 = 1.0f;
        uint32_t root = 0;
#pragma unroll
        for (int t = 0; t < L; ++t) {
            if (LR && t == 0) {
                root = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(rootw), h));
                row0 = p.gram.G0S + static_cast<int64_t>(root) * ld + offL;
                rowo[0] = 0;
                sw0 = p.sw0[root];
            } else {
                const uint32_t word = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(cw[t >> 2]), h));
                const uint32_t f = static_cast<uint32_t>(p.gram.off[t]) + ((word >> (8 * (t & 3))) & 0xFFu);
                rowo[t] = f * static_cast<uint32_t>(ld) + static_cast<uint32_t>(offL);
            }
        }
        // ahat_t = a_t * isw_t and the diagonal split's c_t, formed by lane t into the wave's LDS
        // and read back by all lanes at one address (no registers held across the slot).
        {
            uint32_t wsel = 0;
            int offl = 0;
#pragma unroll
            for (int q = 0; q < kCodeWords; ++q) {
                const uint32_t wq = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(cw[q]), h));
                if ((lane >> 2) == q) wsel = wq;
            }
#pragma unroll
            for (int t = 0; t < L; ++t) {
                if (lane == t) offl = p.gram.off[t];
            }
            if (lane < L) {
                const int t = lane;
                const float isw_t = (LR && t == 0) ? p.isw0[root]
                                                   : p.isw[offl + static_cast<int>((wsel >> (8 * (t & 3))) & 0xFFu)];
                cf[t] = rec[rc.coef + t] * isw_t;
                cf[L + t] = prune::DiagCoef(rec[Rec::Rinv(t)], isw_t);
            }
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        }
        auto gv = [&](int t, uint32_t k) { return (LR && t == 0) ? ld32(row0, k) : ld32(p.gram.G, rowo[t] + k); };
        auto gs = [&](int t, uint32_t k) { return (LR && t == 0) ? ld32(row0, k) * sw0 : ld32(p.Gs, rowo[t] + k); };
        const float kb = rec[rc.kb], cq = rec[rc.cq];
        const float k1 = L >= prune::kDiagMinL ? rec[rc.k1] : 0.0f, k2 = L >= prune::kDiagMinL ? rec[rc.k2] : 0.0f;

        bool staged = false, diag_fast = false;
        int next = 0;  // first chunk not yet listed
        while (next < nch) {
            float gp = 0.0f;
            const float W = worst_now();
            const bool bounded = !kSlow && prune_on && kb < kInfF && prune::ParentGap(E_old, W, gp);
            const bool filling = !kSlow && prune_on && !(W < kInfF);
            const int last = (bounded || !filling) ? nch : next + 1;
            int total = 0;
            // Whether candidate (this slot, lane + 64 j) survives the bound: eta~ = sum_t b_t ahat_t,
            // b2 = sum_t b_t^2 and X~ = sum_t (c_t b_t)^2 by fma, b_t = Gs(f_t, k).
            auto keep_of = [&](int j, float alj, float gmj) -> bool {
                const uint32_t k = static_cast<uint32_t>(lane + kWave * j);
                const bool act = FULL || static_cast<int>(k) < K;
                float et = 0.0f, b2 = 0.0f, xs = 0.0f;
#pragma unroll
                for (int t = 0; t < L; ++t) {
                    const float bt = act ? gs(t, k) : 0.0f;
                    const float ut = cf[L + t] * bt;
                    et = t == 0 ? bt * cf[t] : __builtin_fmaf(bt, cf[t], et);
                    b2 = t == 0 ? bt * bt : __builtin_fmaf(bt, bt, b2);
                    xs = t == 0 ? ut * ut : __builtin_fmaf(ut, ut, xs);
                }
                return act && !prune::Prunable2(alj, b2, xs, gmj - et, kb, k1, k2, cq, gp);
            };
            auto list = [&](int j, bool keep) {
                const uint64_t km = Ballot(keep);
                if (keep) pack[total + __popcll(km & ((1ull << lane) - 1ull))] = lane + kWave * j;
                total += __popcll(km);
            };
            {
#pragma unroll 1
                for (int j = next; j < last; ++j) {
                    bool keep = FULL || lane + kWave * j < K;
                    if (bounded) {
                        float alj = 0.0f, gmj = 0.0f;
#pragma unroll
                        for (int jj = 0; jj < kMaxChunks; ++jj) {
                            if (jj == j) {
                                alj = alc[jj];
                                gmj = gam[jj];
                            }
                        }
                        keep = keep_of(j, alj, gmj);
                    }
                    list(j, keep);
                }
            }
            next = last;
            if (total == 0) continue;
            if (!staged) {
                // the slot's factor columns with 1/diag (record dwords 1..kRWords) and coefficients
#pragma unroll
                for (int q0 = 0; q0 < kRWords; q0 += kWave) {
                    if (q0 + lane < kRWords) fac[q0 + lane] = rec[1 + q0 + lane];
                }
                if (lane < L) fac[kRWords + lane] = rec[rc.coef + lane];
                staged = true;
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
                bool diag_ok = true;
#pragma unroll
                for (int r = 0; r < L; ++r) diag_ok = diag_ok && DiagFastOk(fac[Rec::R(r, r) - 1]);
                diag_fast = !LR && diag_ok;
            } else {
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            }
            for (int b = 0; b < total; b += kWave) {
                const int idx = b + lane;
                const bool act = idx < total;
                const uint32_t k = static_cast<uint32_t>(act ? pack[idx] : 0);
                float A[L];
#pragma unroll
                for (int t = 0; t < L; ++t) A[t] = gv(t, k);
                const float alpha = p.gdiag[offL + k];
                const float gamma = xCi[offL + k];
                float y[L], v[L], denom, a_last, e;
                bool ok, safe = true;
                if (LR) {
                    EvalStaged<L, 2>(fac, A, E_old, alpha, gamma, y, v, e, denom, a_last, ok, safe);
                } else {
                    bool ieee = kSlow || !diag_fast;
                    if (!ieee) {
                        EvalStaged<L, 1>(fac, A, E_old, alpha, gamma, y, v, e, denom, a_last, ok, safe);
                        ieee = Ballot(!safe) != 0ull;
                    }
                    if (ieee) EvalStaged<L, 0>(fac, A, E_old, alpha, gamma, y, v, e, denom, a_last, ok, safe);
                }
                if (!replay(ok && act, e, h * K + static_cast<int>(k))) return false;
            }
        }
        return true;
    };

    // The windowed queue scan (fast pass with pruning): slots are taken kStagedWin at a time. A
    // window's factors, coefficients and errors are staged in LDS, its slots are bound-tested in
    // scan order against the worst of that moment, and the survivors (slot, codeword) of all its
    // slots go into one FIFO, evaluated exactly 64 at a time (each lane reading its own slot's
    // factor) and replayed in scan order; the window's last survivors are evaluated before the
    // next window is staged. The worst only falls between a test and the replay, so a pruned
    // candidate stays one the reference rejects.
    auto scan_windows = [&](auto&& replay, auto&& worst_now) -> bool {
        int* __restrict__ queue = reinterpret_cast<int*>(wbuf);
        float* __restrict__ wst = wbuf + kQueueCap;                    // factor, a_old, E_old per slot
        float* __restrict__ wcf = wst + kStagedWin * StagedQStride<L>();  // ahat[L], c[L] per slot
        int qhead = 0, qlen = 0, base = 0;
        uint64_t diag_mask = 0;
        auto flush = [&](int n) -> bool {
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            const bool act = lane < n;
            const int ent = act ? queue[(qhead + lane) & (kQueueCap - 1)] : 0;
            const int sl = ent >> 8;
            const int hl = base + sl;
            const uint32_t k = static_cast<uint32_t>(ent & 0xFF);
            const float* f = wst + sl * StagedQStride<L>();
            const float E_old = f[StagedWords<L>()];
            const bool diag_ok = ((diag_mask >> sl) & 1ull) != 0ull;
            const uint32_t rootl =
                LR ? static_cast<uint32_t>(__builtin_amdgcn_ds_bpermute(hl << 2, static_cast<int>(rootw))) : 0u;
            uint32_t cwl[kCodeWords];
#pragma unroll
            for (int q = 0; q < kCodeWords; ++q)
                cwl[q] = static_cast<uint32_t>(__builtin_amdgcn_ds_bpermute(hl << 2, static_cast<int>(cw[q])));
            float A[L];
#pragma unroll
            for (int t = 0; t < L; ++t) {
                if (LR && t == 0) {
                    A[t] = p.gram.G0S[static_cast<int64_t>(rootl) * ld + offL + k];
                } else {
                    const uint32_t fi = static_cast<uint32_t>(p.gram.off[t]) + ((cwl[t >> 2] >> (8 * (t & 3))) & 0xFFu);
                    A[t] = ld32(p.gram.G, fi * static_cast<uint32_t>(ld) + static_cast<uint32_t>(offL) + k);
                }
            }
            const float alpha = p.gdiag[offL + k];
            const float gamma = xCi[offL + k];
            float y[L], v[L], denom, a_last, e;
            bool ok, safe = true;
            if (LR) {
                EvalStaged<L, 2>(f, A, E_old, alpha, gamma, y, v, e, denom, a_last, ok, safe);
            } else {
                bool ieee = Ballot(act && !diag_ok) != 0ull;
                if (!ieee) {
                    EvalStaged<L, 1>(f, A, E_old, alpha, gamma, y, v, e, denom, a_last, ok, safe);
                    ieee = Ballot(act && !safe) != 0ull;
                }
                if (ieee) EvalStaged<L, 0>(f, A, E_old, alpha, gamma, y, v, e, denom, a_last, ok, safe);
            }
            qhead = (qhead + n) & (kQueueCap - 1);
            qlen -= n;
            return replay(ok && act, e, hl * K + static_cast<int>(k));
        };
        for (base = 0; base < curH; base += kStagedWin) {
            const int nw = min(kStagedWin, curH - base);
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            {
                // the window's factor columns with 1/diag, coefficients and error
                constexpr int kW1 = StagedWords<L>() + 1;
                for (int q = lane; q < nw * kW1; q += kWave) {
                    const int hw = q / kW1, o = q - hw * kW1;
                    const float* src = recs_in + (base + hw) * rc.stride;
                    wst[hw * StagedQStride<L>() + o] =
                        o < kRWords ? src[1 + o] : (o < StagedWords<L>() ? src[rc.coef + o - kRWords] : src[0]);
                }
                // ahat_t = a_t * isw_t and the diagonal split's c_t of every window slot
                for (int q = lane; q < nw * L; q += kWave) {
                    const int hw = q / L, t = q - hw * L;
                    const float* src = recs_in + (base + hw) * rc.stride;
                    const float isw_t = (LR && t == 0) ? p.isw0[reinterpret_cast<const uint32_t*>(src)[rc.root]]
                                                       : p.isw[p.gram.off[t] + CodeAt(src, rc.code, t)];
                    wcf[hw * 2 * L + t] = src[rc.coef + t] * isw_t;
                    wcf[hw * 2 * L + L + t] = prune::DiagCoef(src[Rec::Rinv(t)], isw_t);
                }
                bool dok = lane < nw;
                if (dok) {
                    const float* src = recs_in + (base + lane) * rc.stride;
#pragma unroll
                    for (int r = 0; r < L; ++r) dok = dok && DiagFastOk(src[Rec::R(r, r)]);
                }
                diag_mask = Ballot(dok);
            }
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            for (int hw = 0; hw < nw; ++hw) {
                const int h = base + hw;
                const float* rec = recs_in + h * rc.stride;
                const float E_old = rec[0];
                const float kb = rec[rc.kb], cq = rec[rc.cq], k1 = rec[rc.k1], k2 = rec[rc.k2];
                const float* cfh = wcf + hw * 2 * L;
                uint32_t rowo[L];
                const float* row0 = nullptr;
                float sw0 = 1.0f;
#pragma unroll
                for (int t = 0; t < L; ++t) {
                    if (LR && t == 0) {
                        const uint32_t root = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(rootw), h));
                        row0 = p.gram.G0S + static_cast<int64_t>(root) * ld + offL;
                        rowo[0] = 0;
                        sw0 = p.sw0[root];
                    } else {
                        const uint32_t word =
                            static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(cw[t >> 2]), h));
                        const uint32_t fi = static_cast<uint32_t>(p.gram.off[t]) + ((word >> (8 * (t & 3))) & 0xFFu);
                        rowo[t] = fi * static_cast<uint32_t>(ld) + static_cast<uint32_t>(offL);
                    }
                }
                auto gsw = [&](int t, uint32_t k) {
                    return (LR && t == 0) ? ld32(row0, k) * sw0 : ld32(p.Gs, rowo[t] + k);
                };
                auto test = [&](const float (&b)[L], float alj, float gmj, float gp) -> bool {
                    float et = 0.0f, b2 = 0.0f, xs = 0.0f;
#pragma unroll
                    for (int t = 0; t < L; ++t) {
                        const float bt = b[t];
                        const float ut = cfh[L + t] * bt;
                        et = t == 0 ? bt * cfh[t] : __builtin_fmaf(bt, cfh[t], et);
                        b2 = t == 0 ? bt * bt : __builtin_fmaf(bt, bt, b2);
                        xs = t == 0 ? ut * ut : __builtin_fmaf(ut, ut, xs);
                    }
                    return !prune::Prunable2(alj, b2, xs, gmj - et, kb, k1, k2, cq, gp);
                };
                auto enqueue = [&](int j, bool keep, uint64_t km) -> bool {
                    if (keep) {
                        const int pos = (qhead + qlen + __popcll(km & ((1ull << lane) - 1ull))) & (kQueueCap - 1);
                        queue[pos] = (hw << 8) | (lane + kWave * j);
                    }
                    qlen += __popcll(km);
                    return qlen < kWave || flush(kWave);
                };

                const float W0 = worst_now();
                if (!FULL || !(W0 < kInfF)) {
                    // A slot of the top-H is still empty (or a partial layer): chunk by chunk,
                    // each tested against the worst after the previous one was queued.
#pragma unroll 1
                    for (int j = 0; j < nch; ++j) {
                        const bool act = FULL || lane + kWave * j < K;
                        float gp = 0.0f;
                        const bool bounded = kb < kInfF && prune::ParentGap(E_old, worst_now(), gp);
                        bool keep = act;
                        if (bounded) {
                            const uint32_t k = static_cast<uint32_t>(lane + kWave * j);
                            float b[L];
#pragma unroll
                            for (int t = 0; t < L; ++t) b[t] = act ? gsw(t, k) : 0.0f;
                            // chunk j's alc and gamma read again (an index into alc/gam, j being
                            // a loop variable here, would put them in scratch)
                            const float alj = (act ? p.gdiag[offL + k] : 0.0f) * prune::kAlphaScale;
                            const float gmj = act ? xCi[offL + k] : 0.0f;
                            keep = act && test(b, alj, gmj, gp);
                        }
                        if (!enqueue(j, keep, Ballot(keep))) return false;
                    }
                } else {
                    // The whole slot against the worst at its start (it only falls from there),
                    // two chunks per step (a scheduling barrier keeps the second pair's reads
                    // from being hoisted into the first, where they would hold registers).
                    float gp = 0.0f;
                    const bool bounded = kb < kInfF && prune::ParentGap(E_old, W0, gp);
#pragma unroll
                    for (int j0 = 0; j0 < kMaxChunks; j0 += 2) {
                        __builtin_amdgcn_sched_barrier(0);
                        bool keep[2];
                        uint64_t km[2];
                        if (bounded) {
                            float b[2][L];
#pragma unroll
                            for (int jj = 0; jj < 2; ++jj) {
#pragma unroll
                                for (int t = 0; t < L; ++t) b[jj][t] = gsw(t, static_cast<uint32_t>(lane + kWave * (j0 + jj)));
                            }
#pragma unroll
                            for (int jj = 0; jj < 2; ++jj) keep[jj] = test(b[jj], alc[j0 + jj], gam[j0 + jj], gp);
                        } else {
                            keep[0] = keep[1] = true;
                        }
                        km[0] = Ballot(keep[0]);
                        km[1] = Ballot(keep[1]);
                        if (!enqueue(j0, keep[0], km[0])) return false;
                        if (!enqueue(j0 + 1, keep[1], km[1])) return false;
                    }
                }
            }
            if (qlen > 0 && !flush(qlen)) return false;
        }
        return true;
    };

    if constexpr (LAST && BEST) {
        if (prune_on) {  // the final pick only (LastPick)
            LastPick lp;
            auto track = [&](bool ok, float e, int cand) { return lp.Take(ok, e, cand); };
            auto min_now = [&]() { return lp.Now(); };
            const bool fine = scan_windows(track, min_now);
            WriteLastPick<L, LR>(fine, lp, p, rc, recs_in, K, i, lane);
            return;
        }
    }

    float s_err;
    int s_cand;
    bool flagged = false;
    SelectTopH<true, BEST, BEST, BEST && (!LR || L <= kLrSortFirstMaxL)>(  // errors clamped at zero (EvalCand)
        Hb, lane,
        [&](auto&& replay, auto slow_tag, auto&& worst_now) {
            if constexpr (!decltype(slow_tag)::value) {
                if (prune_on) return scan_windows(replay, worst_now);
            }
            for (int h = 0; h < curH; ++h) {
                if (!process(h, replay, slow_tag, worst_now)) return false;
            }
            return true;
        },
        s_err, s_cand, flagged);
    if (BEST && flagged) {
        // No records: the next layers see an empty beam (curH = 0), do no work for this vector
        // and keep it well-formed until its re-run.
        if (lane == 0) {
            p.flags[i] = 1;
            p.out.curH[w] = 0;
        }
        return;
    }

    // Deferred write-back (beam_search.cpp:337-383; the large root :896-947) or the all-skipped
    // fallback (:385-400, :949-966), as in LayerKernel.
    const bool live = lane < Hb && !(s_err >= kInfF);
    const int newH = __popcll(Ballot(lane < Hb && s_err < kInfF));
    const int outH = newH == 0 ? max(1, min(curH, Hb)) : newH;  // CountFinite and max(1, .)
    if (lane == 0) p.out.curH[w] = outH;
    float out_err = kInfF;
    int src = -1, knew = 0;
    if (newH == 0) {
        if (lane < min(curH, Hb)) {
            src = lane;
            out_err = recs_in[lane * rc.stride];
        }
    } else if (live) {
        src = s_cand / K;
        knew = s_cand - src * K;
        out_err = s_err;
    }
    if (!p.is_last) {
        float* ro = recs_out + lane * rc.stride;
        const float* ri = recs_in + (src < 0 ? 0 : src) * rc.stride;
        auto put_codes = [&](bool from_parent, int kc, uint32_t root) {
            uint32_t* cwo = reinterpret_cast<uint32_t*>(ro + rc.code);
#pragma unroll
            for (int qq = 0; qq <= L / 4; ++qq) {
                uint32_t word = 0;
#pragma unroll
                for (int b = 0; b < 4; ++b) {
                    const int t = 4 * qq + b;
                    const uint32_t c = t < L ? (from_parent ? static_cast<uint32_t>(CodeAt(ri, rc.code, t)) : 0u)
                                             : (t == L ? static_cast<uint32_t>(kc) : 0u);
                    word |= c << (8 * b);
                }
                cwo[qq] = word;
            }
            reinterpret_cast<uint32_t*>(ro)[rc.root] = root;
        };
        if (newH == 0) {
            const int nh = min(curH, Hb);
            // the parents' factor columns 0..L-1 with 1/diag, copied by the whole wave
            for (int q = 0; q < nh; ++q) {
                const float* rs = recs_in + q * rc.stride + 1;
                float* rd = recs_out + q * rc.stride + 1;
#pragma unroll
                for (int q0 = 0; q0 < kRWords; q0 += kWave) {
                    if (q0 + lane < kRWords) rd[q0 + lane] = rs[q0 + lane];
                }
            }
            if (lane < nh) {
                // parent slot `lane` with a zero new column
                ro[0] = ri[0];
#pragma unroll
                for (int t = 0; t < L; ++t) ro[rc.coef + t] = ri[rc.coef + t];
                ro[rc.coef + L] = 0.0f;
#pragma unroll
                for (int r = 0; r < L; ++r) ro[Rec::R(r, L)] = 0.0f;
                ro[Rec::R(L, L)] = 0.0f;
                ro[Rec::Rinv(L)] = 1.0f / 0.0f;
                put_codes(true, 0, reinterpret_cast<const uint32_t*>(ri)[rc.root]);
                rc.PutBounds(ro, prune::NoBounds());
            } else if (nh == 0 && lane == 0) {
                // No beam at all (layer 0 had no finite candidate): the reference's next-buffer
                // slot 0 keeps its never-written (zero) state with error +inf.
                ro[0] = kInfF;
#pragma unroll
                for (int t = 0; t <= L; ++t) ro[rc.coef + t] = 0.0f;
#pragma unroll
                for (int r = 0; r <= L; ++r) {
#pragma unroll
                    for (int c = r; c <= L; ++c) ro[Rec::R(r, c)] = 0.0f;
                    ro[Rec::Rinv(r)] = 1.0f / 0.0f;
                }
                put_codes(false, 0, 0u);
                rc.PutBounds(ro, prune::NoBounds());
            }
        } else {
            // In rounds of kWbSlots slots: the whole wave copies each slot's parent factor columns
            // 0..L-1 (with 1/diag) into the new record and stages them with the parent's
            // coefficients in LDS; then each slot's lane solves its chosen candidate once more
            // with the reference's arithmetic (IEEE division, or the large root's reciprocal
            // multiply) for the new coefficients, Cholesky column and bounds.
            for (int q0 = 0; q0 < Hb; q0 += kWbSlots) {
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
                const int qn = min(Hb - q0, kWbSlots);
                for (int q = 0; q < qn; ++q) {
                    const int sq = __builtin_amdgcn_readlane(src, q0 + q);
                    if (sq < 0) continue;
                    const float* rs = recs_in + sq * rc.stride;
                    float* rd = recs_out + (q0 + q) * rc.stride + 1;
                    float* st = wbuf + q * WbStride<L>();
#pragma unroll
                    for (int c0 = 0; c0 < kRWords + L; c0 += kWave) {
                        const int c = c0 + lane;
                        if (c < kRWords) {
                            const float x = rs[1 + c];
                            rd[c] = x;
                            st[c] = x;
                        } else if (c < kRWords + L) {
                            st[c] = rs[rc.coef + (c - kRWords)];
                        }
                    }
                }
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
                if (live && lane >= q0 && lane < q0 + qn) {
                    const float* st = wbuf + (lane - q0) * WbStride<L>();
                    const uint32_t root = reinterpret_cast<const uint32_t*>(ri)[rc.root];
                    float A[L];
                    int fl[L];  // flat index of each prefix codeword (the root for a large root's prefix 0)
#pragma unroll
                    for (int t = 0; t < L; ++t) {
                        fl[t] = (LR && t == 0) ? static_cast<int>(root) : p.gram.off[t] + CodeAt(ri, rc.code, t);
                        const float* row = (LR && t == 0) ? p.gram.G0S + static_cast<int64_t>(root) * ld + offL
                                                          : p.gram.G + static_cast<int64_t>(fl[t]) * ld + offL;
                        A[t] = row[knew];
                    }
                    float y[L], v[L], e, denom, a_last;
                    bool ok, unused = true;
                    if (LR) {
                        EvalStaged<L, 2>(st, A, ri[0], p.gdiag[offL + knew], xCi[offL + knew], y, v, e, denom, a_last,
                                         ok, unused);
                    } else {
                        EvalStaged<L, 0>(st, A, ri[0], p.gdiag[offL + knew], xCi[offL + knew], y, v, e, denom, a_last,
                                         ok, unused);
                    }
                    ro[0] = s_err;
                    double asq = 0.0;  // ||ahat||^2 of the new coefficients
#pragma unroll
                    for (int t = 0; t <= L; ++t) {
                        const float at = t < L ? st[kRWords + t] - v[t] * a_last : a_last;
                        ro[rc.coef + t] = at;
                        const float iswt =
                            t < L ? ((LR && t == 0) ? p.isw0[fl[t]] : p.isw[fl[t]]) : p.isw[offL + knew];
                        const double ah = static_cast<double>(at) * static_cast<double>(iswt);
                        asq += ah * ah;
                    }
#pragma unroll
                    for (int r = 0; r < L; ++r) ro[Rec::R(r, L)] = y[r];
                    const float rLL = sqrtf(denom);
                    ro[Rec::R(L, L)] = rLL;
                    ro[Rec::Rinv(L)] = 1.0f / rLL;
                    put_codes(true, knew, root);
                    auto swf = [&](int t) { return (LR && t == 0) ? p.sw0[fl[t]] : p.sw[fl[t]]; };
                    rc.PutBounds(ro, prune::NextBounds<L>(y, v, rLL, swf, p.sw[offL + knew], ri[rc.kap], ri[rc.phi],
                                                          rc.Nf2(ri), asq));
                }
            }
            if (!live && lane < Hb) ro[0] = kInfF;  // an empty slot: never read by the next layer
        }
        return;
    }

    // Last layer: the final pick (beam_search.cpp:409-419) over the slots the write-back would
    // build; with no finite candidate (the fallback) those are the parent slots with code 0.
    if (BEST && FinalTie(out_err, outH)) {
        if (lane == 0) p.flags[i] = 1;
        return;
    }
    const int best = BestSlot(out_err, outH, lane);
    if (lane == best) {
        // src < 0: no beam at all (the reference's never-written slot 0: codes 0, error +inf)
        const float* ri = recs_in + (src < 0 ? 0 : src) * rc.stride;
        const uint32_t root = src < 0 ? 0u : reinterpret_cast<const uint32_t*>(ri)[rc.root];
        if (LR) {
            p.cluster_out[i] = root;
#pragma unroll
            for (int t = 1; t < L; ++t) p.codes_out[i * (m - 1) + (t - 1)] = src < 0 ? 0 : CodeAt(ri, rc.code, t);
            p.codes_out[i * (m - 1) + (L - 1)] = static_cast<uint8_t>(knew);
        } else {
#pragma unroll
            for (int t = 0; t < L; ++t) p.codes_out[i * m + t] = src < 0 ? 0 : CodeAt(ri, rc.code, t);
            p.codes_out[i * m + L] = static_cast<uint8_t>(knew);
        }
        if (p.best_err) p.best_err[i] = out_err;
    }
}

template <int L, template <int, bool, bool, bool> class KernelSel>
hipError_t LaunchWith(bool lr, const LayerArgs& a, hipStream_t s) {
    const unsigned blocks = static_cast<unsigned>((a.n + kBeamWavesPerBlock - 1) / kBeamWavesPerBlock);
    const dim3 block(kWave * kBeamWavesPerBlock);
    const bool full = a.K == kMaxK;
    const unsigned lds = static_cast<unsigned>(KernelSel<L, false, true, false>::DynamicLds(a.Hb));
    if (lr) {  // the large-root beam's best-first pass is built for full layers (K = 256) only
        if (a.flags && !full) return hipErrorInvalidValue;
        if (a.flags && a.is_last)
            hipLaunchKernelGGL((KernelSel<L, true, true, true>::kernel_last), dim3(blocks), block, lds, s, a);
        else if (a.flags) hipLaunchKernelGGL((KernelSel<L, true, true, true>::kernel), dim3(blocks), block, lds, s, a);
        else if (full) hipLaunchKernelGGL((KernelSel<L, true, true, false>::kernel), dim3(blocks), block, lds, s, a);
        else hipLaunchKernelGGL((KernelSel<L, true, false, false>::kernel), dim3(blocks), block, lds, s, a);
    } else if (a.flags) {
        // the last layer of the best-first pass over full layers: the final pick only
        if (full && a.is_last)
            hipLaunchKernelGGL((KernelSel<L, false, true, true>::kernel_last), dim3(blocks), block, lds, s, a);
        else if (full) hipLaunchKernelGGL((KernelSel<L, false, true, true>::kernel), dim3(blocks), block, lds, s, a);
        else hipLaunchKernelGGL((KernelSel<L, false, false, true>::kernel), dim3(blocks), block, lds, s, a);
    } else {
        if (full) hipLaunchKernelGGL((KernelSel<L, false, true, false>::kernel), dim3(blocks), block, lds, s, a);
        else hipLaunchKernelGGL((KernelSel<L, false, false, false>::kernel), dim3(blocks), block, lds, s, a);
    }
    return hipGetLastError();
}

template <int L, bool LR, bool FULL, bool BEST>
struct QueueSel {
    static constexpr auto kernel = LayerKernel<L, LR, FULL, BEST>;
    static constexpr auto kernel_last = LayerKernel<L, LR, FULL, BEST, true>;
    static constexpr size_t DynamicLds(int Hb) { return QStage<L>::Bytes(Hb); }  // the staged slot states
};

template <int L, bool LR, bool FULL, bool BEST>
struct StagedSel {
    static constexpr auto kernel = LayerKernelStaged<L, LR, FULL, BEST>;
    static constexpr auto kernel_last = LayerKernelStaged<L, LR, FULL, BEST, true>;
    static constexpr size_t DynamicLds(int) { return 0; }
};

template <int L>
hipError_t LaunchL(bool lr, const LayerArgs& a, hipStream_t s) {
    if constexpr (L <= kQueueMaxL) {
        return LaunchWith<L, QueueSel>(lr, a, s);
    } else {
        return LaunchWith<L, StagedSel>(lr, a, s);
    }
}

}  // namespace

// Layer launchers by range of L, one per translation unit.
hipError_t LaunchQueueLayer(int L, bool large_root, const LayerArgs& a, hipStream_t s);   // 1..8
hipError_t LaunchStagedLayerA(int L, bool large_root, const LayerArgs& a, hipStream_t s);  // 9..13
hipError_t LaunchStagedLayerB(int L, bool large_root, const LayerArgs& a, hipStream_t s);  // 14..19

}  // namespace stlq_mi355
