// vxs_wave.h — the one-wave fast path of the sampler (vocabularies up to 3072).
//
// One wave64 owns a row: lane l holds elements c*256 + 4l + j of sweep c, loaded once from HBM and
// kept in VGPRs to the sampled id (first the logits, then their nucleus masses). Every reduction,
// scan and select is wave-local (DPP, readlane, ballot); LDS holds the penalty staging, one
// histogram and a short ranking list, small enough for 16 rows per CU. The path covers what
// full-vocabulary sampling needs — penalty, suppression, greedy, temperature, the nucleus regime
// with or without top-p — and hands a row back untouched (return value 1) when it needs the general
// algorithm: a top-k above 64 or one whose entries at or above the k-th largest exceed 64, a history
// longer than 2048 ids, 65 to 256 candidates (the exact regime beyond one wave), a top-p cut whose
// crossing bucket holds more than 64 entries, a cut inside a group of
// equal masses far from where equal masses imply equal logits, a draw that finds no crossing, or a
// call that asks for the write-back logits or the probabilities. Every decision depends on the row
// alone, so results do not depend on the batch.
//
//   S1 penalty      the row is staged into LDS in parts of up to 6 sweeps; the wave reads the
//                   original logit of every history id of the part, then writes s*rho or the
//                   correctly rounded s/rho back (a repeated id rewrites the same value, so
//                   each distinct id is penalised once)                         Sampler.cs:25-33
//   S2 suppression  [supp_begin, supp_end) except keep_id, then ban_id -> -inf  TalkerGenerator.cs:247-248
//   S3 greedy       first index of the max, no temperature                      Sampler.cs:37,90-95
//   S4 temperature  x * fl32(1/T)                                               Sampler.cs:39-40
//   S6-S8 nucleus   fp32 masses exp(d), d = x - max, rounded to multiples of 2^-F (exact,
//                   order-independent double sums); the masses replace the logits in VGPRs.
//                   A histogram over the top bits of the masses (1024 LDS buckets, a log scale)
//                   gives the total and the bucket where the ascending cumulative mass crosses
//                   floor(fl32(1 - top_p) * total); that bucket's entries are ranked by
//                   (mass, index) for the exact cut. The draw sums the kept masses per sweep,
//                   finds the sweep, then the lane, then the entry holding
//                   floor(u * kept mass) in index order.                        Sampler.cs:51-87
#pragma once

#include <stdint.h>

#include "vxs_device.h"
#include "vxs_internal.h"

namespace vxs {
namespace wave {

using namespace dev;

constexpr int kSweep = 256;  // elements per sweep: 64 lanes x 4
constexpr int kPart = 6;     // sweeps staged in LDS at once for the penalty
constexpr int kNB = 1024;    // top-p histogram buckets (16 per lane)
constexpr int kBPL = kNB / 64;
static_assert(kNB == 1024, "bucket index is a 10-bit field of the mass bits");
constexpr int kL = 64;       // crossing-bucket entries ranked exactly (one per lane); top-k bound
static_assert(kL == kWaveMaxTopK, "the one-wave top-k capacity is its lane count");
constexpr int kExact = 256;  // rows with at most this many candidates take the exact regime
constexpr int kHP = 8;       // history ids per lane fetched with the row (512 per row)
constexpr int kHMax = 2048;  // longest history the wave path takes (the rest in chunks of 8 per lane)
constexpr int kDeadId = 1 << 14;  // history slot past the row's ids: above every vocabulary the path takes

typedef double dbl2 __attribute__((ext_vector_type(2)));

struct Sel {
    alignas(16) uint64_t hist[kNB];     // mass per bucket in units of 2^-F; then the draw's per-lane sweep sums
    uint32_t key[kL + 8];   // crossing-bucket entries (32-bit keys), then pads
    uint32_t skey[kL];      // the same in rank order
    double ws[kL];          // their masses in rank order
    double stot;            // total mass, kept for the optional nucleus statistics
};

// LDS ordering inside one wave.
__device__ __forceinline__ void wsync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__device__ __forceinline__ float opaque(float x) {
    asm volatile("" : "+v"(x));
    return x;
}
__device__ __forceinline__ int opaque_i(int x) {
    asm volatile("" : "+v"(x));
    return x;
}

// Lane position among the set bits of `bal` below this lane.
__device__ __forceinline__ uint32_t mbcnt(uint64_t bal) {
    return __builtin_amdgcn_mbcnt_hi((uint32_t)(bal >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)bal, 0u));
}

// The wave's issue priority at a step of its row, in the instance that steps it (kPrio): 3 once
// the row's loads are issued; in the nucleus regime 2 after the masses, 1 at the crossing bucket,
// 0 at the draw; with top-k 2 at the gather above the bound, 1 at the k-th value, 0 at the exact
// regime. A SIMD then issues first for the rows with the most work left instead of for its oldest
// waves. A compile-time switch: a run-time test would split the code into more scheduling regions.
template <bool kPrio, int L>
__device__ __forceinline__ void row_prio() {
    if constexpr (kPrio) __builtin_amdgcn_s_setprio(L);
}

}  // namespace wave

template <int NS>
struct WaveSmem {
    union {
        // penalty staging, one spare slot per lane, then a 4096-bit id bitmap for long histories
        float xs[wave::kPart * wave::kSweep + 64 + 128];
        wave::Sel sel;
    } u;
};

template <int NS>
struct WaveRow {
    float v[4 * NS];     // the row: lane l holds elements c*256 + 4l + j
    int pre[wave::kHP];  // history ids h0 + lane + 64k
    int h0, h1;          // the row's history range
    bool pen_on;         // penalty active
};

// The loads of row r (in the batch), issued without waiting.
template <int NS>
__device__ __forceinline__ void wave_load_row(const SampleArgs& a, int vec, int r, int lane, WaveRow<NS>& w) {
    using namespace wave;
    const int V = a.vocab;
    const float* __restrict__ xrow = a.logits + (int64_t)r * a.ld;
    const int lane4 = lane * 4;
#pragma unroll
    for (int c = 0; c < NS; c++) {
        if (vec && (c + 1) * kSweep <= V) {  // whole sweep inside the row (wave-uniform)
            typedef float f4 __attribute__((ext_vector_type(4)));
            const f4 q = __builtin_nontemporal_load((const f4*)(xrow + c * kSweep + lane4));
            w.v[c * 4 + 0] = q.x;
            w.v[c * 4 + 1] = q.y;
            w.v[c * 4 + 2] = q.z;
            w.v[c * 4 + 3] = q.w;
        } else {
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int i = c * kSweep + lane4 + j;
                w.v[c * 4 + j] = i < V ? xrow[i] : kNegInf;
            }
        }
    }
}

// The checks that hand a row back to the general algorithm, then the loads of its history, issued
// without waiting. Returns 1 to hand the row back, else 0.
template <int NS>
__device__ __forceinline__ int wave_prepare(const SampleArgs& a, int r, int lane, const vxs_params& P, WaveRow<NS>& w) {
    using namespace wave;
    // outputs, the penalty alone and resident stores (whose step ends in put_id) take the general path
    if (a.out_logits || a.out_probs || (a.kflags & KF_STOP_AFTER_PENALTY) || a.store) return 1;
    if (P.do_sample && P.top_k > kL && P.top_k < a.vocab) return 1;  // top-k beyond one wave's candidates
    const bool pen_on = P.rep_penalty != 1.0f && has_history(a);
    HistRange hr{0, 0};
    if (pen_on) hr = history_range(a, r);
    w.pen_on = pen_on;  // each field written once: no selected-address stores
    w.h0 = hr.h0;
    w.h1 = hr.h1;
    if (hr.h1 - hr.h0 > kHMax) return 1;  // very long history
    if (pen_on) {
#pragma unroll
        for (int k = 0; k < kHP; k++) {
            const int h = w.h0 + lane + k * 64;
            w.pre[k] = h < w.h1 ? a.hist_ids[h] : kDeadId;
        }
    }
    return 0;
}

// Second half: samples row r from its loaded logits. Returns 0 when the row is done (its id
// written) and 1, having written nothing, when it must go to the general algorithm.
template <int NS, bool kStats, bool kPrio>
__device__ __forceinline__ int wave_finish(const SampleArgs& a, int r, int lane, const vxs_params& P, WaveRow<NS>& w,
                                           WaveSmem<NS>& sm) {
    using namespace wave;
    constexpr int NE = 4 * NS;
    const int V = a.vocab;
    // element index of register slot e; the base is re-materialised at each use so the compiler
    // does not keep an index register per element alive
    const int lane4 = lane * 4;
    auto eidx = [&](int e) { return (e >> 2) * kSweep + opaque_i(lane4) + (e & 3); };
    float (&v)[NE] = w.v;
    const int(&pre)[kHP] = w.pre;
    const int h0 = w.h0, h1 = w.h1;
    const bool pen_on = w.pen_on;
    // entries past the vocabulary (pads) hold -inf: they never win, carry no mass, are never written

    row_prio<kPrio, 3>();  // the row's loads are issued: all of its work is ahead
    // ---- S1: repetition penalty over the distinct history ids
    // Per staged part, every lane first reads the original logit of each of its ids, then writes
    // the penalised value back: a wave's LDS operations execute in order, so all reads precede all
    // writes and a repeated id writes the same value again instead of being penalised twice. The
    // reads and writes are unmasked: an id outside the part uses the lane's own spare slot.
    // The quotient is the Markstein-corrected one (penalize_fast): correctly rounded for rho with
    // |rho| in [2^-20, 2^20] (other rows go to the general path) and logits in [2^-60, 2^60] or
    // not positive (zeros keep their sign). A positive logit below 2^-60 becomes a value below
    // 2^-40 that may be off by at most 2^-83. That cannot change the sampled id: it gives the same
    // d = fl32(x - max) when the maximum is at least 2^-30 (a row whose maximum lies in (0, 2^-30)
    // or at or above 2^100, or is not finite, goes to the general path after the statistics
    // below), and a top-k row whose k-th largest value lies in [0, 2^-39), the only place such an
    // entry could fall on the wrong side of the k-th value, goes to the general path there.
    if (pen_on && h1 > h0) {
        const float rho = P.rep_penalty;
        const float arho = __builtin_fabsf(rho);
        if (!(arho >= 0x1p-20f && arho <= 0x1p20f)) return 1;
        const float rinv = 1.0f / rho;
        float* xs = sm.u.xs;
        typedef float f4 __attribute__((ext_vector_type(4)));
        if (h1 - h0 > kHP * 64) {
            // A history over 512 ids: the ids are taken in chunks of eight per lane (the first chunk
            // fetched with the row), and an LDS bitmap keeps them distinct: the lane whose atomicOr
            // first sets an id's bit penalises that entry of the staged part. Per part, every id is
            // tested; an id outside the vocabulary fails the row (checked over all ids in part 0).
            uint32_t* bm = reinterpret_cast<uint32_t*>(xs + kPart * kSweep + 64);
            typedef uint32_t u2v __attribute__((ext_vector_type(2)));
            *(u2v*)&bm[2 * lane] = u2v{0u, 0u};  // 128 words: 4096 bits
#pragma unroll
            for (int p0 = 0; p0 < NS; p0 += kPart) {
#pragma unroll
                for (int c = 0; c < kPart; c++)
                    if (p0 + c < NS)
                        *(f4*)(xs + c * kSweep + lane4) =
                            f4{v[(p0 + c) * 4 + 0], v[(p0 + c) * 4 + 1], v[(p0 + c) * 4 + 2], v[(p0 + c) * 4 + 3]};
                wsync();
                const int lo = p0 * kSweep, span = (p0 + kPart < NS ? kPart : NS - p0) * kSweep;
                bool bad = false;
#pragma unroll 1
                for (int k0 = 0; k0 < kHMax / 64; k0 += kHP) {
                    if (h0 + 64 * k0 >= h1) break;  // uniform: no ids left
                    int id[kHP];
#pragma unroll
                    for (int k = 0; k < kHP; k++) {
                        const int h = h0 + lane + 64 * (k0 + k);
                        id[k] = k0 == 0 ? pre[k] : (h < h1 ? a.hist_ids[h] : 0);
                    }
#pragma unroll
                    for (int k = 0; k < kHP; k++) {
                        const bool lv = h0 + lane + 64 * (k0 + k) < h1;
                        bad |= lv && (unsigned)id[k] >= (unsigned)V;
                        if (lv && (unsigned)id[k] < (unsigned)V && (unsigned)(id[k] - lo) < (unsigned)span) {
                            const uint32_t bit = 1u << (id[k] & 31);
                            if (!(atomicOr(&bm[id[k] >> 5], bit) & bit)) {
                                float* px = xs + (id[k] - lo);
                                *px = penalize_fast(*px, rho, rinv);
                            }
                        }
                    }
                }
                if (p0 == 0 && __ballot(bad)) {
                    if (lane == 0) a.out_ids[r] = VXS_ERR_ID_OUT_OF_RANGE;
                    return 0;
                }
                wsync();
#pragma unroll
                for (int c = 0; c < kPart; c++)
                    if (p0 + c < NS) {
                        const f4 q = *(const f4*)(xs + c * kSweep + lane4);
                        v[(p0 + c) * 4 + 0] = q.x;
                        v[(p0 + c) * 4 + 1] = q.y;
                        v[(p0 + c) * 4 + 2] = q.z;
                        v[(p0 + c) * 4 + 3] = q.w;
                    }
                wsync();  // the next part (or phase) overwrites the staging area
            }
        } else {
        bool live[kHP];
        bool bad = false;
#pragma unroll
        for (int k = 0; k < kHP; k++) {
            live[k] = h0 + lane + k * 64 < h1;
            bad |= live[k] && (unsigned)pre[k] >= (unsigned)V;
        }
        if (__ballot(bad)) {
            if (lane == 0) a.out_ids[r] = VXS_ERR_ID_OUT_OF_RANGE;
            return 0;
        }
        auto stage = [&](int p0) {
#pragma unroll
            for (int c = 0; c < kPart; c++)
                if (p0 + c < NS)
                    *(f4*)(xs + c * kSweep + lane4) =
                        f4{v[(p0 + c) * 4 + 0], v[(p0 + c) * 4 + 1], v[(p0 + c) * 4 + 2], v[(p0 + c) * 4 + 3]};
        };
        auto unstage = [&](int p0) {
#pragma unroll
            for (int c = 0; c < kPart; c++)
                if (p0 + c < NS) {
                    const f4 q = *(const f4*)(xs + c * kSweep + lane4);
                    v[(p0 + c) * 4 + 0] = q.x;
                    v[(p0 + c) * 4 + 1] = q.y;
                    v[(p0 + c) * 4 + 2] = q.z;
                    v[(p0 + c) * 4 + 3] = q.w;
                }
        };
        static_assert(NS <= 2 * kPart, "the penalty stages at most two parts");
        if (NS <= kPart) {
            // one part: every read of an original logit precedes every write of a penalised one;
            // dead slots clamp to the dummy slot past the staged sweeps
            uint32_t at[kHP];
            float pv[kHP];
            stage(0);
            wsync();
#pragma unroll
            for (int k = 0; k < kHP; k++) {
                at[k] = min((uint32_t)pre[k], (uint32_t)(kPart * kSweep));
                pv[k] = penalize_fast(xs[at[k]], rho, rinv);
            }
#pragma unroll
            for (int k = 0; k < kHP; k++) xs[at[k]] = pv[k];
            wsync();
            unstage(0);
            wsync();
        } else {
            // Two parts of kPart sweeps, one after the other: the staged part is read at every id,
            // the values penalised and written back (all reads of the part before its writes), and
            // the part unstaged. Ids outside the staged part and dead slots clamp to the dummy slot
            // kSpan, so every id's quotient is computed for both parts: eight more per lane than
            // staging part 0 a second time, and measured faster (6 KB less LDS traffic per row).
            constexpr uint32_t kSpan = kPart * kSweep;
            uint32_t at0[kHP], at1[kHP];
            float pv[kHP];
#pragma unroll
            for (int k = 0; k < kHP; k++) {
                at0[k] = min((uint32_t)pre[k], kSpan);
                at1[k] = min((uint32_t)pre[k] - kSpan, kSpan);
            }
            stage(0);
            wsync();
#pragma unroll
            for (int k = 0; k < kHP; k++) pv[k] = opaque(xs[at0[k]]);
#pragma unroll
            for (int k = 0; k < kHP; k++) pv[k] = penalize_fast(pv[k], rho, rinv);
#pragma unroll
            for (int k = 0; k < kHP; k++) xs[at0[k]] = pv[k];
            wsync();
            unstage(0);
            wsync();
            stage(kPart);
            wsync();
#pragma unroll
            for (int k = 0; k < kHP; k++) pv[k] = opaque(xs[at1[k]]);
#pragma unroll
            for (int k = 0; k < kHP; k++) pv[k] = penalize_fast(pv[k], rho, rinv);
#pragma unroll
            for (int k = 0; k < kHP; k++) xs[at1[k]] = pv[k];
            wsync();
            unstage(kPart);
            wsync();  // the next phase overwrites the staging area
        }
        }
    }

    // ---- S2: suppression
    if (P.supp_begin < P.supp_end || P.ban_id >= 0) {
        const int sb = max(P.supp_begin, 0), se = min(P.supp_end, V);
#pragma unroll
        for (int e = 0; e < NE; e++) {
            const int i = eidx(e);
            if ((i >= sb && i < se && i != P.keep_id) || i == P.ban_id) v[e] = kNegInf;
        }
    }

    // ---- S3: greedy (a lane's elements ascend in index, so a strict > keeps the first maximum)
    if (!P.do_sample) {
        float bv = v[0];
        int bi = eidx(0);
        bool nan = v[0] != v[0];
#pragma unroll
        for (int e = 1; e < NE; e++) {
            nan |= v[e] != v[e];
            const bool gt = v[e] > bv;
            bv = gt ? v[e] : bv;
            bi = gt ? eidx(e) : bi;
        }
        wave_argmax(bv, bi);
        const bool anynan = __ballot(nan) != 0;
        if (pen_on && (anynan || bv >= 0x1p100f || (bv > 0.0f && bv < 0x1p-30f))) return 1;  // see S1
        if (lane == 0) a.out_ids[r] = anynan ? VXS_ERR_NONFINITE : bi;
        return 0;
    }

    // ---- S4: temperature (x * 1 is x, so the common T = 1 skips the pass)
    const float invT = P.temperature == 1.0f ? 1.0f : 1.0f / P.temperature;
    if (invT != 1.0f) {
#pragma unroll
        for (int e = 0; e < NE; e++) v[e] *= invT;
        if (!(invT > 0.0f)) {  // negative or NaN scale: pads go back to -inf
#pragma unroll
            for (int e = 0; e < NE; e++)
                if (eidx(e) >= V) v[e] = kNegInf;
        }
    }
    float mx, mn;  // max; min including -inf
    float fmn;     // min over finite entries
    uint32_t cnt;  // finite entries
    float lmx;     // this lane's maximum
    {
        // the NaN-propagating maximum turns a NaN or +inf anywhere in a lane into a non-finite max
        float tmx = v[0], tmn = v[0];
#pragma unroll
        for (int e = 1; e < NE; e++) {
            tmx = __builtin_elementwise_maximum(tmx, v[e]);
            tmn = fminf(tmn, v[e]);
        }
        if (__ballot(!(tmx < kPosInf))) {
            if (pen_on) return 1;  // a penalised non-finite logit: the general path reports it
            if (lane == 0) a.out_ids[r] = VXS_ERR_NONFINITE;
            return 0;
        }
        lmx = tmx;
        mx = wave_fmax(tmx);
        if (pen_on && (mx >= 0x1p100f || (mx > 0.0f && mx < 0x1p-30f))) return 1;  // see S1
        mn = wave_fmin(tmn);
        fmn = mn;
        cnt = (uint32_t)V;
        if (mn == kNegInf) {  // some entries are -inf (suppressed or pads): count the rest
            uint32_t cl = 0;
            float fl = kPosInf;
#pragma unroll
            for (int e = 0; e < NE; e++) {
                const bool fin = v[e] != kNegInf;
                cl += fin ? 1u : 0u;
                fl = fin ? fminf(fl, v[e]) : fl;
            }
            cnt = wave_sum(cl);
            fmn = wave_fmin(fl);
        }
    }
    if (cnt == 0) {  // every entry is -inf: p = 0/0 and the reference's draw returns the last id
        if (lane == 0) a.out_ids[r] = V - 1;
        return 0;
    }
    // ================= top-k and the exact regime on one wave =================
    // Rows whose candidates fit one wave: top-k with K <= 64 (the entries >= the k-th largest, ties
    // kept), or at most 64 finite entries. The entries above a lower bound of the k-th largest (the
    // k-th largest lane maximum: at least K entries reach it) are gathered in index order (at most
    // kCand), the exact k-th largest among them is found by bisection over their keys, and the
    // reference's fp64 arithmetic runs on the final candidates, one per lane (wave_exact).
    const int K = P.top_k;
    const bool topk_on = K > 0 && K < V && (uint32_t)K < cnt;  // else top-k masks nothing (Sampler.cs:42)
    if (topk_on || cnt <= (uint32_t)kL) {
        constexpr int kCand = 256;
        float* cval = sm.u.xs;                                             // gathered values
        int32_t* cidx = reinterpret_cast<int32_t*>(sm.u.xs + kCand);       // ... and their indices
        float* fx = sm.u.xs + 2 * kCand;                                   // final candidates
        int32_t* fid = reinterpret_cast<int32_t*>(sm.u.xs + 2 * kCand + kL);
        double* scr = reinterpret_cast<double*>(sm.u.xs + 2 * kCand + 2 * kL);  // wave_exact's 193 doubles
        // lower bound: the K-th largest lane maximum (exact unless ties), or every finite entry
        float tf = -3.402823466e38f;
        if (topk_on) {
            const uint32_t lk[1] = {f2key(lmx)};
            // any t with K to K + slack lane maxima at or above it: the search stops sooner, and a
            // small slack keeps the gathered set small (talker batch, K = 50: exact 29.4 us, slack
            // 8 28.8 us, slack 16 or more 40 us, when the bound falls to the smallest lane maximum)
            const int slack = min(8, (kL - K) >> 1);
            tf = key2f(wave_bound_regs<1>(lk, wave_umin(lk[0]), wave_umax(lk[0]), K, slack));
        }
        row_prio<kPrio, 2>();
        // gather the entries >= tf in index order: per sweep, each lane's count (0..4) in a 16-bit
        // field, four sweeps per 64-bit scan
        constexpr int NH = (NS + 3) / 4;
        uint64_t exc[NH], tot[NH];
#pragma unroll
        for (int h = 0; h < NH; h++) {
            uint64_t mine = 0;
#pragma unroll
            for (int c = 4 * h; c < NS && c < 4 * h + 4; c++) {
                uint32_t m = 0;
#pragma unroll
                for (int j = 0; j < 4; j++) m += v[c * 4 + j] >= tf ? 1u : 0u;
                mine |= (uint64_t)m << (16 * (c - 4 * h));
            }
            const uint64_t incl = wave_incl_sum(mine);
            exc[h] = incl - mine;
            tot[h] = readlane64(incl, 63);
        }
        uint32_t n = 0;
#pragma unroll
        for (int c = 0; c < NS; c++) {
            const int f = 16 * (c % 4);
            uint32_t off = n + (uint32_t)((exc[c / 4] >> f) & 0xffffu);
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int e = c * 4 + j;
                if (v[e] >= tf) {
                    if (off < (uint32_t)kCand) {
                        cval[off] = v[e];
                        cidx[off] = eidx(e);
                    }
                    off++;
                }
            }
            n += (uint32_t)((tot[c / 4] >> f) & 0xffffu);
        }
        if (n > (uint32_t)kCand) return 1;  // too many entries above the bound: general path
        wsync();
        uint32_t nf = n;
        if (topk_on) {
            row_prio<kPrio, 1>();
            // the exact k-th largest key among the gathered entries (all entries >= it are here)
            uint32_t kq[4];
            float cv[4];
            int32_t ci[4];
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const int pq = lane + 64 * q;
                const bool in = pq < (int)n;
                cv[q] = in ? cval[pq] : 0.0f;
                ci[q] = in ? cidx[pq] : 0;
                kq[q] = in ? f2key(cv[q]) : 0u;
            }
            uint32_t lo = f2key(tf), hi = f2key(mx);
#pragma unroll 1
            while (lo < hi) {
                const uint32_t mid = lo + ((hi - lo + 1) >> 1);
                int c = 0;
#pragma unroll
                for (int q = 0; q < 4; q++) c += __builtin_popcountll(__ballot(kq[q] >= mid));
                if (c >= K) lo = mid;
                else hi = mid - 1;
            }
            // the k-th value near a penalised positive logit below 2^-60 (see S1)
            if (pen_on && h1 > h0 && lo >= f2key(0.0f) && lo < f2key(0x1p-39f)) return 1;
            // the final candidates (>= the k-th largest), still in index order
            nf = 0;
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const bool keep = kq[q] >= lo;  // empty slots hold 0 < lo
                const uint64_t bal = __ballot(keep);
                if (keep) {
                    const uint32_t pos = nf + mbcnt(bal);
                    if (pos < (uint32_t)kL) {
                        fx[pos] = cv[q];
                        fid[pos] = ci[q];
                    }
                }
                nf += (uint32_t)__builtin_popcountll(bal);
            }
            if (nf > (uint32_t)kL) return 1;  // ties at the k-th value beyond one wave
            wsync();
        } else {
            fx = cval;  // at most 64 finite entries: every one is a candidate
            fid = cidx;
        }
        row_prio<kPrio, 0>();  // the exact regime's fp64 chain
        const double uu = a.u ? a.u[r] : 0.0;
        const float xl = lane < (int)nf ? fx[lane] : 0.0f;
        const int pick = wave_exact(xl, fid, (int)nf, mx, P.top_p < 1.0f, P.top_p, uu, scr, nullptr, lane);
        if (lane == 0) a.out_ids[r] = pick;
        return 0;
    }
    if (cnt <= (uint32_t)kExact) return 1;  // exact regime beyond one wave

    // ================= nucleus regime =================
    const double thr = (double)(1.0f - P.top_p);
    const bool topp = P.top_p < 1.0f;
    if (topp && !(thr < 1.0)) return 1;  // top_p <= 0: every entry but the last in order goes
    // F fraction bits: vocab * 2^F <= 2^53, so sums of masses (multiples of 2^-F) are exact
    const int F = min(51, 53 - (32 - __clz(V - 1)));
    const float Cb = mass_bias(F);
    // 2^F and 2^-F built from their bits, so they stay in scalar registers
    const double gF = __longlong_as_double((long long)(1023 + F) << 52);
    const double gFi = __longlong_as_double((long long)(1023 - F) << 52);
    // d = x - max replaces the logits (-inf stays -inf)
#pragma unroll
    for (int e = 0; e < NE; e++) v[e] = v[e] - mx;
    // masses replace d: nucleus_exp(d), on the 2^-F grid. When the smallest is at least 2^(23-F)
    // (and no entry is -inf) every mass is a multiple of 2^-F already and the rounding is skipped.
    const float qmin = mass_of(nucleus_exp(fmn - mx), Cb);
    const bool ongrid = mn != kNegInf && qmin >= Cb;
    float qc = 0.0f;  // cut: keep masses >= qc
    double Skept;
    if (topp) {
        Sel& s = sm.u.sel;
        // Buckets: bits(mass) >> sh, a log scale, 1024 of them from `base` up. Every nonzero mass
        // lies in [lb, bits(1) + 8]; zero masses land anywhere and add nothing. The physical
        // bucket is the low 10 bits of the index, so no clamp is needed.
        const float qlow = qmin - qmin * 0x1p-18f - __uint_as_float((uint32_t)(127 - F) << 23);
        const uint32_t lb = max(__float_as_uint(qlow), (uint32_t)(127 - F) << 23);
        constexpr uint32_t kTop = 0x3f800000u + 8u;
        int sh = max(0, (32 - __clz(kTop - lb)) - 10);
        if ((kTop >> sh) + 2 - ((lb >> sh) & ~15u) > (uint32_t)kNB - 1) sh++;
        const uint32_t base = (lb >> sh) & ~15u;
        const uint32_t pbase = (base + (uint32_t)(kBPL * lane)) & (kNB - 1);
        // Packed buckets when every mass is on the grid and a bucket lies inside one binade
        // (sh <= 19: a lane's 16 buckets then share their exponent): each entry adds 2^40 (its
        // count) plus its mass bits above its lane's smallest value (below 2^(sh+4), so below 2^35
        // for 3072 entries), from which a bucket's or a lane's mass follows exactly. Otherwise each
        // entry adds its mass in units of 2^-F.
        const bool packed = ongrid && sh <= 19;
#pragma unroll
        for (int i = 0; i < kNB / 128; i++) *(dbl2*)&s.hist[(i * 64 + lane) * 2] = dbl2{0.0, 0.0};  // zero bits
        wsync();
        // the masses and their histogram atomics in one pass, so the atomics drain while the
        // remaining masses are computed
        if (packed) {
            const uint32_t lmask = (1u << (sh + 4)) - 1u;
#pragma unroll
            for (int e = 0; e < NE; e++) {
                const float q = nucleus_exp(v[e]);
                v[e] = q;
                const uint32_t qb = __float_as_uint(q);
                atomicAdd((unsigned long long*)&s.hist[__builtin_amdgcn_ubfe(qb, (uint32_t)sh, 10u)],
                          (unsigned long long)(qb & lmask) | (1ull << 40));
            }
        } else {
            // Integer atomics (LDS adds u64 faster than f64): a mass below 2^(52-F) added to
            // 2^(52-F) in double precision leaves mass * 2^F, an integer below 2^52, in the
            // mantissa bits (the sum keeps the exponent of 2^(52-F), so the high word just loses
            // its exponent bits).
            const double big = __longlong_as_double((long long)(1023 + 52 - F) << 52);
#pragma unroll
            for (int e = 0; e < NE; e++) {
                const float q = ongrid ? nucleus_exp(v[e]) : mass_of(nucleus_exp(v[e]), Cb);
                v[e] = q;
                const uint64_t tb = (uint64_t)__double_as_longlong((double)q + big);
                const uint64_t iq = (tb & 0xffffffffull) | ((uint64_t)((uint32_t)(tb >> 32) & 0xfffffu) << 32);
                atomicAdd((unsigned long long*)&s.hist[__builtin_amdgcn_ubfe(__float_as_uint(q), (uint32_t)sh, 10u)],
                          (unsigned long long)iq);
            }
        }
        wsync();
        row_prio<kPrio, 2>();
        // mass in units of 2^-F of packed entries (one bucket's, or a sum over buckets) of lane bl,
        // whose values are (2^23 + mantissa of the lane's smallest) + offset, times 2^(exponent - 150)
        auto packed_units = [&](uint32_t bl, uint64_t ent) -> uint64_t {
            const uint32_t t = (base + 16u * bl) << sh;  // bits of the lane's smallest value
            const int sft = (int)(t >> 23) + F - 150;
            const uint64_t m = (uint64_t)((t & 0x7fffffu) | 0x800000u) * (ent >> 40) + (ent & ((1ull << 40) - 1));
            return sft >= 0 ? m << sft : 0ull;  // empty below the range
        };
        // lane totals in ascending bucket order, then the crossing lane, then the crossing bucket;
        // lane l reads its 16 buckets in the order j xor (l/2 mod 16), which spreads every read of
        // the wave over all LDS banks
        uint64_t lti = 0;
        const int rot = (lane >> 1) & (kBPL - 1);
        if (packed) {
            uint64_t ent = 0;
#pragma unroll
            for (int j = 0; j < kBPL; j++) ent += s.hist[pbase + (j ^ rot)];
            lti = packed_units((uint32_t)lane, ent);  // the 16 buckets share their exponent
        } else {
#pragma unroll
            for (int j = 0; j < kBPL; j++) lti += s.hist[pbase + (j ^ rot)];
        }
        const double lt = (double)lti * gFi;  // exact: below 2^53 units of 2^-F
        const double incl = wave_incl_sum(lt);
        const double S = readlane_d(incl, 63);
        if constexpr (kStats) s.stot = S;
        const double T = floor(thr * S * gF) * gFi;
        const double run = incl - lt;
        const uint64_t cb = __ballot(run <= T && T - run < lt);
        if (!cb) return 1;
        const int L = (int)__builtin_ctzll(cb);
        const double runL = readlane_d(run, L);
        const uint32_t pL = (base + (uint32_t)(kBPL * L)) & (kNB - 1);
        const uint64_t hent = s.hist[pL + (lane & (kBPL - 1))];
        const uint64_t hu = packed ? packed_units((uint32_t)L, hent) : hent;
        const double hj = lane < kBPL ? (double)hu * gFi : 0.0;
        const double ij = row_incl_sum(hj);  // lanes 0..15 form one DPP row
        const double xj = runL + (ij - hj);
        const uint64_t jb = __ballot(lane < kBPL && xj <= T && T - xj < hj);
        if (!jb) return 1;
        const int jl = (int)__builtin_ctzll(jb);
        const double below = readlane_d(xj, jl);
        uint32_t glo = (base + (uint32_t)(kBPL * L + jl)) << sh;  // bits of the bucket's masses
        asm volatile("" : "+s"(glo));  // one subtraction per compare below
        const uint32_t gw = 1u << sh;
        // gather the crossing bucket (ballot compaction); the compares of a batch of eight slots
        // are issued before their ballots are consumed. An entry's 32-bit key is its mass bits
        // above the bucket's smallest (below 2^sh <= 2^19) shifted over its index (12 bits): key
        // order is (mass, index) order inside the bucket.
        row_prio<kPrio, 1>();
        if (sh > 19) return 1;
        uint32_t n = 0;
        uint32_t gwo = gw;
        asm volatile("" : "+s"(gwo));  // a plain unsigned compare (not rewritten into a shift and a test)
        uint32_t* kw = s.key;
#pragma unroll
        for (int e0 = 0; e0 < NE; e0 += 8) {
            bool p[8];
            uint32_t t[8];
            uint64_t bal[8];
#pragma unroll
            for (int k = 0; k < 8; k++) {
                t[k] = __float_as_uint(v[e0 + k]) - glo;
                p[k] = t[k] < gwo;
                bal[k] = __ballot(p[k]);
            }
#pragma unroll
            for (int k = 0; k < 8; k++) {
                if (bal[k]) {
                    const uint32_t pos = n + mbcnt(bal[k]);
                    if (p[k] && pos < (uint32_t)kL) kw[pos] = (t[k] << 12) | (uint32_t)eidx(e0 + k);
                    n += (uint32_t)__builtin_popcountll(bal[k]);
                }
            }
        }
        if (n > (uint32_t)kL) return 1;
        if (lane < 8) kw[n + lane] = ~0u;
        wsync();
        // rank by (mass, index): every lane compares its entry with all of them (broadcast reads)
        const int nn = (int)n;
        const uint32_t ka = lane < nn ? kw[lane] : ~0u;
        uint32_t rk = 0;
#pragma unroll 1
        for (int b = 0; b < nn; b += 8) {
            const uint32_t* kp = &kw[b];
            rk += (kp[0] < ka) + (kp[1] < ka) + (kp[2] < ka) + (kp[3] < ka);
            rk += (kp[4] < ka) + (kp[5] < ka) + (kp[6] < ka) + (kp[7] < ka);
        }
        if (lane < nn) {
            s.ws[rk] = (double)__uint_as_float(glo + (ka >> 12));
            s.skey[rk] = ka;
        }
        wsync();
        const double w0 = lane < nn ? s.ws[lane] : 0.0;
        const double c0 = below + (wave_incl_sum(w0) - w0);
        const uint64_t rb = __ballot(lane < nn && c0 <= T && T - c0 < w0);
        if (!rb) return 1;
        const int rl = (int)__builtin_ctzll(rb);
        const uint32_t kk = s.skey[rl];
        const uint32_t kc = glo + (kk >> 12);
        qc = __uint_as_float(kc);
        // The masses are a monotone function of d (nucleus_exp is monotone on gfx950 — checked over
        // every float in [-128, 0] — and so is the rounding to the 2^-F grid), so (mass, index)
        // order is the reference's (d, index) order except inside a group of equal masses, whose d
        // may differ (one rounding of d * log2 e can merge neighbouring values of d). When members
        // of the cut's group rank before it (removed while the cut entry is kept), the group's d
        // are recomputed from the caller's logits exactly as above: equal d order by index, as
        // ranked here, and the removed members' masses are zeroed in their owner lanes. Unequal d
        // (so the order is not known here): the general path takes the row.
        if (rl > 0 && (s.skey[rl - 1] >> 12) == (kk >> 12)) {
            if (h1 - h0 > kHP * 64) return 1;  // the history ids are not all in registers
            const uint32_t kl = lane < nn ? s.skey[lane] : 0u;  // rank order
            const bool grp = lane < nn && (kl >> 12) == (kk >> 12);
            const int id = (int)(kl & 0xfffu);
            // penalty membership of the members from an LDS bitmap of the history
            typedef uint32_t u2w __attribute__((ext_vector_type(2)));
            uint32_t* hbm = reinterpret_cast<uint32_t*>(s.hist);  // free after the scan: 4096 bits
            *(u2w*)&hbm[2 * lane] = u2w{0u, 0u};
            wsync();
            if (pen_on) {  // the ids are read again (not kept in registers for this rare case)
#pragma unroll
                for (int k = 0; k < kHP; k++) {
                    const int h = h0 + lane + 64 * k;
                    if (h < h1) {
                        const int hid = a.hist_ids[h];
                        atomicOr(&hbm[hid >> 5], 1u << (hid & 31));
                    }
                }
            }
            wsync();
            float d = 0.0f;
            if (grp) {
                float x = a.logits[(int64_t)r * a.ld + id];
                if (pen_on && ((hbm[id >> 5] >> (id & 31)) & 1u)) {
                    const float rho = P.rep_penalty;
                    x = penalize_fast(x, rho, 1.0f / rho);
                }
                if (invT != 1.0f) x *= invT;
                d = x - mx;
            }
            if (wave_fmin(grp ? d : kPosInf) != wave_fmax(grp ? d : kNegInf)) return 1;
            // zero the removed members (ranks below rl): each sets its bit in its owner lane's mask
            wsync();
            uint64_t* msk = reinterpret_cast<uint64_t*>(s.hist);
            msk[lane] = 0;
            wsync();
            if (grp && lane < rl)
                atomicOr((unsigned long long*)&msk[(id >> 2) & 63], 1ull << ((id >> 8) * 4 + (id & 3)));
            wsync();
            const uint64_t mz = msk[lane];
#pragma unroll
            for (int e = 0; e < NE; e++)
                if ((mz >> e) & 1ull) v[e] = 0.0f;
            wsync();  // the draw reuses the histogram area
        }
        Skept = S - readlane_d(c0, rl);
    } else {
        if (ongrid) {
#pragma unroll
            for (int e = 0; e < NE; e++) v[e] = nucleus_exp(v[e]);
        } else {
#pragma unroll
            for (int e = 0; e < NE; e++) v[e] = mass_of(nucleus_exp(v[e]), Cb);
        }
        double ls = 0.0;
#pragma unroll
        for (int e = 0; e < NE; e++) ls += (double)v[e];
        Skept = wave_sum(ls);
    }

    row_prio<kPrio, 0>();
    // ---- draw: first index (index order) whose inclusive kept-mass prefix exceeds floor(u * Skept).
    // Per lane and sweep, the kept masses are summed left to right in fp32 (relative error below
    // 2e-7, inside the 1e-6 band where a draw may differ from the reference's); sweep totals and
    // prefixes add those fp32 sums exactly in double precision, and the final walk recomputes the
    // same fp32 partial sums, so the lane found always holds the crossing.
    const double u = a.u ? a.u[r] : 0.0;  // read here: a double live across the cut would spill
    const double D = floor(u * Skept * gF) * gFi;
    int pick;
    {
        float* ps = reinterpret_cast<float*>(sm.u.sel.hist);  // [NS][64]: sweep-major, conflict-free
        float ls[NS];
#pragma unroll
        for (int c = 0; c < NS; c++) {
            float a = v[c * 4] >= qc ? v[c * 4] : 0.0f;  // masses are >= +0, so 0 + a would be a
#pragma unroll
            for (int j = 1; j < 4; j++) {
                const float q = v[c * 4 + j];
                a += q >= qc ? q : 0.0f;
            }
            ls[c] = a;
            ps[c * 64 + lane] = a;
        }
        wsync();
        // sweep totals: lanes 4c..4c+3 each add 16 lanes' sums of sweep c, then combine in the quad
        const int sc = lane >> 2;
        double t = 0.0;
        if (sc < NS) {
            typedef float f4 __attribute__((ext_vector_type(4)));
            const f4* col = reinterpret_cast<const f4*>(ps + sc * 64 + (lane & 3) * 16);
            const f4 q0 = col[0], q1 = col[1], q2 = col[2], q3 = col[3];
            t = (((double)q0.x + (double)q0.y) + ((double)q0.z + (double)q0.w)) +
                (((double)q1.x + (double)q1.y) + ((double)q1.z + (double)q1.w)) +
                ((((double)q2.x + (double)q2.y) + ((double)q2.z + (double)q2.w)) +
                 (((double)q3.x + (double)q3.y) + ((double)q3.z + (double)q3.w)));
        }
        t = quad_sum(t);
        const double x = (lane & 3) == 0 ? t : 0.0;  // lanes past 4*NS hold 0
        const double xi = wave_incl_sum(x);
        const uint64_t sb = __ballot((lane & 3) == 0 && sc < NS && D < xi);
        if (!sb) return 1;  // no crossing (rounding at the top of the range): general path
        const int sl = (int)__builtin_ctzll(sb);
        const int cs = __builtin_amdgcn_readfirstlane(sl >> 2);
        const double before = readlane_d(xi, sl) - readlane_d(x, sl);
        // sweep cs's partial sum and masses: a uniform switch (register arrays indexed by a
        // runtime value would go to scratch)
        float mine = 0.0f, q4[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        switch (cs) {
#define VXS_SWEEP(C)                                                                   \
    case C:                                                                            \
        if constexpr (C < NS) {                                                        \
            mine = ls[C];                                                              \
            q4[0] = v[C * 4]; q4[1] = v[C * 4 + 1]; q4[2] = v[C * 4 + 2]; q4[3] = v[C * 4 + 3]; \
        }                                                                              \
        break;
            VXS_SWEEP(0) VXS_SWEEP(1) VXS_SWEEP(2) VXS_SWEEP(3) VXS_SWEEP(4) VXS_SWEEP(5)
            VXS_SWEEP(6) VXS_SWEEP(7) VXS_SWEEP(8) VXS_SWEEP(9) VXS_SWEEP(10) VXS_SWEEP(11)
#undef VXS_SWEEP
            default: break;
        }
        static_assert(NS <= 12, "the switch covers 12 sweeps");
        const double md = (double)mine;
        const double li = before + wave_incl_sum(md);
        const uint64_t lb2 = __ballot(D < li);
        if (!lb2) return 1;
        const int L2 = (int)__builtin_ctzll(lb2);
        pick = -1;
        {
            const double b0 = li - md;
            float a = 0.0f;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const float q = q4[j];
                a += q >= qc ? q : 0.0f;
                pick = (pick < 0 && D < b0 + (double)a) ? cs * kSweep + lane * 4 + j : pick;
            }
        }
        pick = (int)readlane((uint32_t)pick, L2);
    }
    if (pick < 0) return 1;
    if (lane == 0) a.out_ids[r] = pick;
    if constexpr (kStats) {  // the nucleus the draw used: kept fraction, smallest kept probability, size
        const double St = topp ? sm.u.sel.stot : Skept;
        uint32_t kn = 0;
        float kmin = __builtin_inff();
#pragma unroll
        for (int e = 0; e < NE; e++) {
            const bool k = v[e] >= qc && v[e] > 0.0f;
            kn += k ? 1u : 0u;
            kmin = k ? fminf(kmin, v[e]) : kmin;
        }
        kn = wave_sum(kn);
        kmin = wave_fmin(kmin);
        if (lane == 0) {
            double* o = a.out_stats + 4 * (int64_t)r;
            o[0] = Skept / St;
            o[1] = (double)kmin / St;
            o[2] = (double)kn;
            o[3] = 0.0;
        }
        if (a.out_stat_probs) {  // the probabilities the draw used: kept masses over the kept mass
            double* pr = a.out_stat_probs + (int64_t)r * a.vocab;
#pragma unroll
            for (int e = 0; e < NE; e++) {
                const int i = (e >> 2) * kSweep + lane * 4 + (e & 3);
                if (i < a.vocab) pr[i] = v[e] >= qc && v[e] > 0.0f ? (double)v[e] / Skept : 0.0;
            }
        }
    }
    return 0;
}

// Samples row r (r < a.rows) with one wave: 0 when done, 1 when handed back.
template <int NS, bool kStats, bool kPrio>
__device__ __forceinline__ int wave_fast_row(const SampleArgs& a, int vec, int r, int lane, WaveSmem<NS>& sm) {
    WaveRow<NS> w;
    const vxs_params P = a.params[(int64_t)r * a.params_stride];
    if (wave_prepare<NS>(a, r, lane, P, w)) return 1;
    wave_load_row<NS>(a, vec, r, lane, w);  // after the history loads: measured faster than before them
    return wave_finish<NS, kStats, kPrio>(a, r, lane, P, w, sm);
}

}  // namespace vxs
