// vxs_wave.h — the one-wave fast path of the sampler (vocabularies up to 3072).
//
// One wave64 owns a row: lane l holds elements c*256 + 4l + j of sweep c, loaded once from HBM and
// kept in VGPRs to the sampled id. Every reduction, scan and select is wave-local (DPP, readlane,
// ballot); LDS holds the penalty staging, one histogram and a short ranking list, small enough
// for 16 rows per CU. The path covers what full-vocabulary sampling needs — penalty, suppression,
// greedy, temperature, the nucleus regime with or without top-p — and hands a row back untouched
// (return value 1) when it needs the general algorithm: an active top-k, a history longer than
// 512 ids, at most 256 candidates (the exact regime), a top-p cut whose crossing bucket holds more
// than 64 entries or is not found, a draw that finds no crossing, or a call that asks for the
// write-back logits or the probabilities. Every decision depends on the row alone, so results do not depend on the batch.
//
//   S1 penalty      the row is staged into LDS in parts of up to 6 sweeps; the wave reads the
//                   original logit of every history id of the part, then writes s*rho or the
//                   correctly rounded s/rho back (a repeated id rewrites the same value, so
//                   each distinct id is penalised once)                         Sampler.cs:25-33
//   S2 suppression  [supp_begin, supp_end) except keep_id, then ban_id -> -inf  TalkerGenerator.cs:247-248
//   S3 greedy       first index of the max, no temperature                      Sampler.cs:37,90-95
//   S4 temperature  x * fl32(1/T)                                               Sampler.cs:39-40
//   S6-S8 nucleus   fp32 masses exp(d), d = x - max, rounded to multiples of 2^-F as integer-valued
//                   doubles (exact, order-independent sums). A histogram of the masses over d
//                   (512 LDS buckets) gives the total and the bucket where the ascending
//                   cumulative mass crosses floor(fl32(1 - top_p) * total); that bucket's entries
//                   are ranked by (d, index) for the exact cut. The draw scans the kept masses in
//                   index order a sweep at a time and stops in the sweep holding
//                   floor(u * kept mass).                                       Sampler.cs:51-87
#pragma once

#include <stdint.h>

#include "vxs_device.h"
#include "vxs_internal.h"

namespace vxs {
namespace wave {

using namespace dev;

constexpr int kSweep = 256;  // elements per sweep: 64 lanes x 4
constexpr int kPart = 6;     // sweeps staged in LDS at once for the penalty
constexpr int kNB = 512;     // top-p histogram buckets (8 per lane)
constexpr int kBPL = kNB / 64;
constexpr int kL = 64;       // crossing-bucket entries ranked exactly (one per lane)
constexpr int kExact = 256;  // rows with at most this many candidates take the exact regime
constexpr int kHP = 8;       // history ids per lane fetched with the row (512 per row)

struct Sel {
    double hist[kNB];
    uint32_t key[kL];
    int32_t idx[kL];
    double ws[kL];
    int32_t at[kL];
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

}  // namespace wave

template <int NS>
struct WaveSmem {
    union {
        float xs[wave::kPart * wave::kSweep];  // penalty staging
        wave::Sel sel;
    } u;
};

// Samples row r with one wave. Returns 0 when the row is done (its id written) and 1, having
// written nothing, when it must go to the general algorithm.
template <int NS>
__device__ __forceinline__ int wave_fast_row(const SampleArgs& a, int vec, int r, int lane, WaveSmem<NS>& sm) {
    using namespace wave;
    constexpr int NE = 4 * NS;
    const int V = a.vocab;
    if (a.out_logits || a.out_probs || (a.kflags & KF_STOP_AFTER_PENALTY)) return 1;
    const vxs_params P = a.params[(int64_t)r * a.params_stride];
    if (P.do_sample && P.top_k > 0 && P.top_k < V) return 1;

    const float* __restrict__ xrow = a.logits + (int64_t)r * a.ld;
    const bool pen_on = P.rep_penalty != 1.0f && a.hist_off != nullptr;
    if (pen_on && a.hist_off[r + 1] - a.hist_off[r] > kHP * 64) return 1;  // long history
    // element index of register slot e; the base is re-materialised at each use so the compiler
    // does not keep an index register per element alive
    const int lane4 = lane * 4;
    auto eidx = [&](int e) { return (e >> 2) * kSweep + opaque_i(lane4) + (e & 3); };

    // ---- issue the history prefetch and the row loads together
    int h0 = 0, h1 = 0;
    int pre[kHP];
    if (pen_on) {
        h0 = a.hist_off[r];
        h1 = a.hist_off[r + 1];
#pragma unroll
        for (int k = 0; k < kHP; k++) {
            const int h = h0 + lane + k * 64;
            pre[k] = h < h1 ? a.hist_ids[h] : 0;
        }
    }
    float v[NE];
#pragma unroll
    for (int c = 0; c < NS; c++) {
        if (vec && (c + 1) * kSweep <= V) {  // whole sweep inside the row (wave-uniform)
            typedef float f4 __attribute__((ext_vector_type(4)));
            const f4 q = __builtin_nontemporal_load((const f4*)(xrow + c * kSweep + lane4));
            v[c * 4 + 0] = q.x;
            v[c * 4 + 1] = q.y;
            v[c * 4 + 2] = q.z;
            v[c * 4 + 3] = q.w;
        } else {
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int i = c * kSweep + lane4 + j;
                v[c * 4 + j] = i < V ? xrow[i] : kNegInf;
            }
        }
    }
    // entries past the vocabulary (pads) hold -inf: they never win, carry no mass, are never written

    // ---- S1: repetition penalty over the distinct history ids
    // Per staged part, every lane first reads the original logit of each of its ids, then writes
    // the penalised value back: a wave's LDS operations execute in order, so all reads precede all
    // writes and a repeated id writes the same value again instead of being penalised twice.
    if (pen_on && h1 > h0) {
        const float rho = P.rep_penalty;
        const float rinv = 1.0f / rho;
        const float arho = __builtin_fabsf(rho);
        const bool fast = arho >= 0x1p-60f && arho <= 0x1p60f;
        bool bad = false;
        float* xs = sm.u.xs;
        typedef float f4 __attribute__((ext_vector_type(4)));
#pragma unroll
        for (int p0 = 0; p0 < NS; p0 += kPart) {
#pragma unroll
            for (int c = 0; c < kPart; c++)
                if (p0 + c < NS)
                    *(f4*)(xs + c * kSweep + lane4) =
                        f4{v[(p0 + c) * 4 + 0], v[(p0 + c) * 4 + 1], v[(p0 + c) * 4 + 2], v[(p0 + c) * 4 + 3]};
            wsync();
            const int lo = p0 * kSweep, hi = (p0 + kPart < NS ? p0 + kPart : NS) * kSweep;
            {
                float sv[kHP];
#pragma unroll
                for (int k = 0; k < kHP; k++) {
                    const int id = pre[k];
                    const bool in = h0 + lane + k * 64 < h1 && id >= lo && id < hi;
                    sv[k] = in ? xs[id - lo] : 0.0f;
                }
#pragma unroll
                for (int k = 0; k < kHP; k++) {
                    const int id = pre[k];
                    const bool live = h0 + lane + k * 64 < h1;
                    bad |= live && (unsigned)id >= (unsigned)V;
                    if (live && id >= lo && id < hi) xs[id - lo] = penalize(sv[k], rho, rinv, fast);
                }
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
        if (__ballot(bad)) {
            if (lane == 0) a.out_ids[r] = VXS_ERR_ID_OUT_OF_RANGE;
            return 0;
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
        if (lane == 0) a.out_ids[r] = anynan ? VXS_ERR_NONFINITE : bi;
        return 0;
    }

    // ---- S4: temperature (always multiplied: x * 1 is x), and the finite-input contract
    const float invT = P.temperature == 1.0f ? 1.0f : 1.0f / P.temperature;
#pragma unroll
    for (int e = 0; e < NE; e++) v[e] *= invT;
    if (!(invT > 0.0f)) {  // negative or NaN scale: pads go back to -inf
#pragma unroll
        for (int e = 0; e < NE; e++)
            if (eidx(e) >= V) v[e] = kNegInf;
    }
    float mx, mn;  // max; min including -inf
    float fmn;     // min over finite entries
    uint32_t cnt;  // finite entries
    {
        bool bad = false;
        float tmx = kNegInf, tmn = kPosInf;
#pragma unroll
        for (int e = 0; e < NE; e++) {
            bad |= __builtin_amdgcn_class(v[e], 0x203);  // NaN or +inf
            tmx = fmaxf(tmx, v[e]);
            tmn = fminf(tmn, v[e]);
        }
        if (__ballot(bad)) {
            if (lane == 0) a.out_ids[r] = VXS_ERR_NONFINITE;
            return 0;
        }
        mx = wave_fmax(tmx);
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
    if (cnt <= (uint32_t)kExact) return 1;  // exact regime

    // ================= nucleus regime =================
    const float m = mx;
    const double u = a.u ? a.u[r] : 0.0;
    // F fraction bits: vocab * 2^F <= 2^53 (exact double sums) and e * 2^F < 2^52.
    const int F = min(51, 53 - (32 - __clz(V - 1)));
    const double scaleF = __builtin_ldexp(1.0, F);
#pragma unroll
    for (int e = 0; e < NE; e++) v[e] = v[e] - m;  // d = x - max; -inf stays -inf
    // masses are recomputed from d where needed: the row and its masses together would not fit
    auto qof = [&](int e) -> float { return exp_neg(opaque(v[e])); };
    auto wof = [&](int e) -> double { return fixed_point((double)qof(e), scaleF); };
    float dc = kNegInf;  // cut: keep d > dc, or d == dc with index >= ic
    int ic = 0;
    double Skept;
    if (P.top_p < 1.0f) {
        Sel& s = sm.u.sel;
        for (int b = lane; b < kNB; b += 64) s.hist[b] = 0.0;
        // buckets linear in d over [lo, 0]; masses below d = -32 round to zero
        const float lo = fmaxf(fmn - m, -32.0f);
        const float scale = lo < -1e-30f ? (float)kNB / -lo : 0.0f;
        const float off = -lo * scale;
        auto bucket = [&](float d) -> int {
            return (int)__builtin_amdgcn_fmed3f(__builtin_fmaf(d, scale, off), 0.0f, (float)(kNB - 1));
        };
        wsync();
#pragma unroll
        for (int e = 0; e < NE; e++)  // -inf entries add 0
            atomicAdd(&s.hist[bucket(v[e])], fixed_point((double)exp_neg(v[e]), scaleF));
        wsync();
        // scan: lane l owns buckets [l*kBPL, (l+1)*kBPL)
        double h[kBPL];
        double lt = 0.0;
#pragma unroll
        for (int j = 0; j < kBPL; j++) {
            h[j] = s.hist[lane * kBPL + j];
            lt += h[j];
        }
        const double incl = wave_incl_sum(lt);
        const double S = readlane_d(incl, 63);
        const double thr = (double)(1.0f - P.top_p);
        if (!(thr < 1.0)) return 1;  // top_p <= 0: every entry but the last in order goes
        const double T = floor(thr * S);
        double run = incl - lt;
        int mine = -1;
        double mbelow = 0.0;
#pragma unroll
        for (int j = 0; j < kBPL; j++) {
            const bool hit = run <= T && T - run < h[j];
            mine = hit ? lane * kBPL + j : mine;
            mbelow = hit ? run : mbelow;
            run += h[j];
        }
        const uint64_t cb = __ballot(mine >= 0);
        if (!cb) return 1;  // total <= T
        const int pl = (int)__builtin_ctzll(cb);
        const int bstar = (int)readlane((uint32_t)mine, pl);
        const double below = readlane_d(mbelow, pl);
        // gather the crossing bucket in index order (ballot compaction)
        uint32_t n = 0;
#pragma unroll
        for (int e = 0; e < NE; e++) {
            const float d = opaque(v[e]);
            const bool p = d != kNegInf && bucket(d) == bstar;
            const uint64_t bal = __ballot(p);
            if (bal) {
                const uint32_t pos = n + mbcnt(bal);
                if (p && pos < (uint32_t)kL) {
                    s.key[pos] = f2key(d);
                    s.idx[pos] = eidx(e);
                }
                n += (uint32_t)__builtin_popcountll(bal);
            }
        }
        if (n > (uint32_t)kL) return 1;
        wsync();
        // rank by (key, index): lane l holds entry l and compares it with every entry
        const int nn = (int)n;
        const uint32_t ka = lane < nn ? s.key[lane] : 0xffffffffu;
        const int ia = lane < nn ? s.idx[lane] : 0x7fffffff;
        const double wa = lane < nn ? fixed_point((double)exp_neg(key2f(ka)), scaleF) : 0.0;
        int rk = 0;
        for (int b = 0; b < nn; b++) {
            const uint32_t kb = readlane(ka, b);
            const int ib = (int)readlane((uint32_t)ia, b);
            rk += (kb < ka) || (kb == ka && ib < ia);
        }
        if (lane < nn) {
            s.ws[rk] = wa;
            s.at[rk] = lane;
        }
        wsync();
        const double w0 = lane < nn ? s.ws[lane] : 0.0;
        const double c0 = below + wave_incl_sum(w0) - w0;
        const uint64_t rb = __ballot(lane < nn && T >= c0 && T - c0 < w0);
        if (!rb) return 1;
        const int rl = (int)__builtin_ctzll(rb);
        const int at = s.at[rl];
        dc = key2f(s.key[at]);
        ic = s.idx[at];
        Skept = S - readlane_d(c0, rl);
    } else {
        double ls = 0.0;
#pragma unroll
        for (int e = 0; e < NE; e++) ls += wof(e);
        Skept = wave_sum(ls);
    }
    auto kept = [&](int e) { return v[e] > dc || (v[e] == dc && eidx(e) >= ic); };

    // ---- draw: first kept index (index order) whose inclusive prefix mass exceeds floor(u * Skept)
    const double D = floor(u * Skept);
    int pick = -1;
    double run = 0.0;
#pragma unroll
    for (int c = 0; c < NS; c++) {
        if (pick < 0) {
            double w4[4];
            double mine = 0.0;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                w4[j] = kept(c * 4 + j) ? wof(c * 4 + j) : 0.0;
                mine += w4[j];
            }
            const double incl = wave_incl_sum(mine);
            const double tot = readlane_d(incl, 63);
            if (D < run + tot) {
                double acc = run + incl - mine;
                int hit = -1;
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    acc += w4[j];
                    hit = (hit < 0 && w4[j] > 0.0 && D < acc) ? eidx(c * 4 + j) : hit;
                }
                const uint64_t bal = __ballot(hit >= 0);
                pick = (int)readlane((uint32_t)hit, bal ? (int)__builtin_ctzll(bal) : 0);
            } else {
                run += tot;
            }
        }
    }
    if (pick < 0) return 1;  // no crossing (rounding at the top of the range): general path
    if (lane == 0) a.out_ids[r] = pick;
    return 0;
}

}  // namespace vxs
