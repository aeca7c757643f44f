// vxs_wide.hip — the sampler for vocabularies above 8192 (up to 2^19), one 256-thread workgroup
// per row, streaming the row from HBM instead of holding it in registers.
//
// One kernel (sample_wide_kernel), two algorithms. The ordered pass (wide_ordered_row) serves the
// common sampled top-k rows in one read of the row; the general algorithm (wide_general_row) serves
// every other row and the rows the ordered pass hands back, in the same workgroup, as follows.
//
// Pass A reads the row once (16-byte loads, 1024 entries per sweep) and applies, per entry:
//   S1 penalty      an LDS bitmap of the history ids marks the entries to rescale (s*rho, or the
//                   correctly rounded s/rho); each distinct id once by construction  Sampler.cs:25-33
//   S2 suppression  [supp_begin, supp_end) except keep_id, then ban_id -> -inf       TalkerGenerator.cs:247-248
//   S3 greedy       running first-index argmax, no temperature                       Sampler.cs:37,90-95
//   S4 temperature  x * fl32(1/T)                                                    Sampler.cs:39-40
//   S5 top-k        (0 < k <= 256) a candidate buffer in LDS keeps every entry >= tau, where tau is
//                   the k-th largest value seen so far: whenever the buffer fills, an exact radix
//                   select finds the k-th largest buffered key, tau rises to it and the buffer is
//                   compacted. tau never exceeds the row's k-th largest value, so the buffer ends
//                   holding every entry the reference keeps.                        Sampler.cs:42-49
// With at most 256 candidates left after the exact k-th largest, the reference's sequential fp64
// arithmetic runs on them in index order (S6-S8, Sampler.cs:51-87) and the row is done after one
// read. Any other row (top-k off or above 256, or ties overflowing the buffer) takes the general
// path: a radix select of the k-th largest over the row, then a mass-weighted radix select of the
// top-p cut over the fixed-point masses exp(d) (exact, order-independent sums, as in the other
// kernels), ties at the cut resolved in index order, and an index-order draw; each step re-reads
// the row (L2/HBM), so the general path costs several passes.
#include <math.h>
#include <stdint.h>

#include "vxs_device.h"
#include "vxs_internal.h"

namespace vxs {
namespace {

using namespace dev;

constexpr int kTW = 256;          // threads per row
constexpr int kWW = kTW / 64;     // waves
constexpr int kSweepW = 4 * kTW;  // entries per sweep
constexpr int kCapW = 512;        // candidate buffer entries per wave
constexpr int kPerL = kCapW / 64;  // ... per lane
constexpr int kKMax = 256;        // largest top-k of the streaming path
constexpr int kCandW = 256;       // exact-regime capacity
constexpr int kRB = 256;          // radix buckets (8-bit digits)
// zero words after the history bitmap: a sweep's lanes past the row end (up to 255 entries) read
// bitmap words within the allocation
constexpr int kBmPad = 8;

struct WideSmem {
    alignas(16) uint32_t wkey[kWW][kCapW];  // per-wave candidate keys (f2key of the value)
    int32_t widx[kWW][kCapW];   // per-wave candidate indices
    // The radix histograms are done with before the exact-regime arrays are filled, so the two
    // share their storage: with the history bitmap of a 151936-entry row this keeps a workgroup
    // within 40 KB of LDS, four workgroups (16 waves) per CU.
    union {
        union {
            alignas(16) uint32_t hcnt[kRB];
            double hmass[kRB];
            alignas(16) uint32_t h3[3 * kRB];  // ordered pass: the k-th largest select's histograms
        } h;
        struct {
            float cx[kCandW];
            int32_t ci[kCandW];
            double cp[kCandW];  // also the (d, index) sort keys before the probabilities
            int16_t cs[kCandW];
        } ex;
    };
    uint64_t slot[4][kWW];
    int32_t wcnt[kWW];  // per-wave candidate counts after pass A (-1: the wave's buffer overflowed)
    int32_t wcomp[kWW]; // per-wave: the buffer was compacted at least once (ordered pass)
    int32_t wslot[kWW]; // per-wave: the wave's SIMD matches the workgroup's slot on its CU (ordered pass)
    uint32_t wklo[kWW], wkhi[kWW];  // ordered pass, per wave: smallest and largest buffered key ...
    int32_t wbad[kWW];              // ... a NaN or fl(x * 1/T) = +inf in its range ...
    int32_t wcand[kWW];             // ... and its candidates at or above the k-th largest
    uint32_t tau_key;   // the largest k-th largest any wave has found so far (a shared lower bound)
    uint32_t qkey[kWW]; // ordered pass, per wave: a key with at least ceil(k/4) of the wave's entries at or above it
    int32_t n;          // exact-regime candidates
};

// Workgroup combines that may be reused in a loop: a barrier before and after the slot read.
struct BlkW {
    int lane, wv, t;
    WideSmem* s;
    template <class Op>
    __device__ __forceinline__ uint64_t combine(uint64_t w, Op op, int site = 0) const {
        if (lane == 0) s->slot[site][wv] = w;
        __syncthreads();
        uint64_t r = s->slot[site][0];
#pragma unroll
        for (int i = 1; i < kWW; i++) r = op(r, s->slot[site][i]);
        __syncthreads();
        return r;
    }
    __device__ __forceinline__ uint32_t usum(uint32_t x) const {
        return (uint32_t)combine(wave_sum(x), [](uint64_t p, uint64_t q) { return p + q; });
    }
    __device__ __forceinline__ double dsum(double x) const {
        return __longlong_as_double((long long)combine((uint64_t)__double_as_longlong(wave_sum(x)),
                                                       [](uint64_t p, uint64_t q) {
                                                           return (uint64_t)__double_as_longlong(
                                                               __longlong_as_double((long long)p) +
                                                               __longlong_as_double((long long)q));
                                                       }));
    }
    __device__ __forceinline__ uint32_t umax(uint32_t x) const {
        return (uint32_t)combine(wave_umax(x), [](uint64_t p, uint64_t q) { return p > q ? p : q; });
    }
    __device__ __forceinline__ uint32_t umin(uint32_t x) const {
        return (uint32_t)combine(wave_umin(x), [](uint64_t p, uint64_t q) { return p < q ? p : q; });
    }
    __device__ __forceinline__ bool any(bool p) const {
        return combine(wave_any(p) ? 1u : 0u, [](uint64_t a, uint64_t b) { return a | b; }) != 0;
    }
    // exclusive prefix over threads; integer-valued doubles (exact)
    __device__ __forceinline__ double excl(double v, double& total) const {
        const double incl = wave_incl_sum(v);
        if (lane == 0) s->slot[1][wv] = (uint64_t)__double_as_longlong(readlane_d(incl, 63));
        __syncthreads();
        double base = 0.0, tot = 0.0;
#pragma unroll
        for (int i = 0; i < kWW; i++) {
            const double x = __longlong_as_double((long long)s->slot[1][i]);
            base += i < wv ? x : 0.0;
            tot += x;
        }
        __syncthreads();
        total = tot;
        return base + incl - v;
    }
    __device__ __forceinline__ uint32_t excl(uint32_t v, uint32_t& total) const {
        const uint32_t incl = wave_incl_sum(v);
        if (lane == 0) s->slot[1][wv] = readlane(incl, 63);
        __syncthreads();
        uint32_t base = 0, tot = 0;
#pragma unroll
        for (int i = 0; i < kWW; i++) {
            const uint32_t x = (uint32_t)s->slot[1][i];
            base += i < wv ? x : 0;
            tot += x;
        }
        __syncthreads();
        total = tot;
        return base + incl - v;
    }
};

// One row's transform of a raw logit: penalty, suppression, and (when sampling) temperature.
struct RowX {
    const uint32_t* bm;  // penalised-id bitmap (LDS) or null
    float rho, rinv;
    bool fastdiv;
    int sb, se, keep, ban;
    float invT;  // 1 for greedy rows
    __device__ __forceinline__ float operator()(int i, float x) const {
        if (bm && ((bm[i >> 5] >> (i & 31)) & 1u)) x = penalize(x, rho, rinv, fastdiv);
        if ((i >= sb && i < se && i != keep) || i == ban) x = kNegInf;
        return x * invT;
    }
};

// Visits every entry of the row in index order groups: f(i, x) for the transformed value x of
// entry i (i < V). Each thread handles 4 consecutive entries of every 1024-entry sweep.
template <class F>
__device__ __forceinline__ void for_row(const float* __restrict__ xrow, int V, int vec, int t, const RowX& X, F f) {
    for (int base = 0; base < V; base += kSweepW) {
        const int i0 = base + 4 * t;
        float x[4];
        if (vec && i0 + 3 < V) {
            typedef float f4 __attribute__((ext_vector_type(4)));
            const f4 q = __builtin_nontemporal_load((const f4*)(xrow + i0));
            x[0] = q.x;
            x[1] = q.y;
            x[2] = q.z;
            x[3] = q.w;
        } else {
#pragma unroll
            for (int j = 0; j < 4; j++) x[j] = i0 + j < V ? xrow[i0 + j] : kNegInf;
        }
#pragma unroll
        for (int j = 0; j < 4; j++)
            if (i0 + j < V) f(i0 + j, X(i0 + j, x[j]));
    }
}

// Orders a wave's LDS accesses: its earlier writes are visible to all its lanes afterwards.
__device__ __forceinline__ void wave_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// The largest key K with at least k of the wave's register-held keys >= K (the k-th largest with
// multiplicity), by bisection over [lo, hi], the smallest and largest valid key. Empty slots hold
// 0, below every valid key. Counts come from ballots, so a step costs one compare per slot.
template <int N>
__device__ __forceinline__ uint32_t wave_kth_regs(const uint32_t (&kk)[N], uint32_t lo, uint32_t hi, int k) {
#pragma unroll 1
    while (lo < hi) {
        const uint32_t mid = lo + ((hi - lo + 1) >> 1);
        int c = 0;
#pragma unroll
        for (int q = 0; q < N; q++) c += __builtin_popcountll(__ballot(kk[q] >= mid));
        if (c >= k) lo = mid;
        else hi = mid - 1;
    }
    return lo;
}

// k-th largest (1-based, with multiplicity) of a wave's n >= k buffered keys; wave-local.
__device__ __forceinline__ uint32_t wave_kth(const uint32_t* keys, int lane, int n, int k) {
    uint32_t kk[kPerL];
    uint32_t lo = 0xffffffffu, hi = 0;
#pragma unroll
    for (int q = 0; q < kPerL; q++) {
        const int j = lane + 64 * q;
        kk[q] = j < n ? keys[j] : 0;
        if (j < n) {
            lo = min(lo, kk[q]);
            hi = max(hi, kk[q]);
        }
    }
    return wave_kth_regs(kk, wave_umin(lo), wave_umax(hi), k);
}

// Keep a wave's buffered entries with key >= kmin (order kept). Returns the new count.
__device__ __forceinline__ int wave_filter(uint32_t* keys, int32_t* idx, int lane, int n, uint32_t kmin) {
    uint32_t kk[kPerL];
    int32_t ii[kPerL];
#pragma unroll
    for (int q = 0; q < kPerL; q++) {
        const int j = lane + 64 * q;
        kk[q] = j < n ? keys[j] : 0;
        ii[q] = j < n ? idx[j] : 0;
    }
    wave_sync();
    uint32_t m = 0;
#pragma unroll
    for (int q = 0; q < kPerL; q++) {
        const bool keep = lane + 64 * q < n && kk[q] >= kmin;
        const uint64_t bal = __ballot(keep);
        if (keep) {
            const uint32_t pos = m + __builtin_amdgcn_mbcnt_hi((uint32_t)(bal >> 32),
                                                               __builtin_amdgcn_mbcnt_lo((uint32_t)bal, 0u));
            keys[pos] = kk[q];
            idx[pos] = ii[q];
        }
        m += (uint32_t)__builtin_popcountll(bal);
    }
    wave_sync();
    return (int)m;
}

// Exact regime on n <= kCandW candidates in index order (cx values, ci indices): the reference's
// sequential fp64 arithmetic. Sequential phases run redundantly in every thread on LDS broadcasts.
__device__ __forceinline__ int exact_block(const BlkW& g, WideSmem& s, int n, float m, bool topp, float top_p,
                                           double u, double* prow) {
    auto& ex = s.ex;
    for (int j = g.t; j < n; j += kTW) ex.cp[j] = exp((double)(ex.cx[j] - m));  // Sampler.cs:57
    __syncthreads();
    const double sum = seq_sum(ex.cp, n);  // sequential in index order                  :58
    __syncthreads();
    for (int j = g.t; j < n; j += kTW) ex.cp[j] = ex.cp[j] / sum;  //                   :60
    __syncthreads();
    if (topp) {  //                                                                    :62-75
        for (int j = g.t; j < n; j += kTW) ex.cs[seq_rank(ex.cp, n, j)] = (int16_t)j;
        __syncthreads();
        // the last sorted position is never removed (the reference's loop runs j < n - 1)
        const int nrem = seq_topp_cut(ex.cp, ex.cs, n, (double)(1.0f - top_p));
        __syncthreads();
        for (int q = g.t; q < nrem; q += kTW) ex.cp[ex.cs[q]] = 0.0;
        __syncthreads();
        const double s2 = seq_sum(ex.cp, n);
        __syncthreads();
        for (int j = g.t; j < n; j += kTW) ex.cp[j] = ex.cp[j] / s2;
        __syncthreads();
    }
    const int pick = seq_draw(ex.cp, ex.ci, n, u);  // inverse-CDF draw in index order    :77-87
    if (prow)
        for (int j = g.t; j < n; j += kTW) prow[ex.ci[j]] = ex.cp[j];
    return pick;
}

// fl32(1/T) of a row, 1 for greedy rows                                     Sampler.cs:39-40
__device__ __forceinline__ float row_inv_temp(const vxs_params& P) {
    return !P.do_sample ? 1.0f : (P.temperature == 1.0f ? 1.0f : 1.0f / P.temperature);
}

// Rows the ordered pass serves: sampled, 0 < k <= kKMax and k < V, 1/T finite and positive, and
// no penalty or one that never raises a value (rho >= 1). For them fl(x * 1/T) bounds the
// transformed value from above and is monotone in the raw value x.
__device__ __forceinline__ bool row_ordered(const SampleArgs& a, const vxs_params& P) {
    if (a.kflags & KF_STOP_AFTER_PENALTY) return false;
    const float invT = row_inv_temp(P);
    const bool has_pen = P.rep_penalty != 1.0f && has_history(a);
    return P.do_sample && P.top_k > 0 && P.top_k <= kKMax && P.top_k < a.vocab && invT > 0.0f &&
           invT < kPosInf && (!has_pen || P.rep_penalty >= 1.0f);
}

// The LDS bitmap of row r's history ids (S1), with kBmPad zero words after it. All threads call
// it; false (with the error id written) when an id lies outside [0, V).
__device__ __forceinline__ bool build_bitmap(const BlkW& g, const SampleArgs& a, int r, int V, uint32_t* bm) {
    const int words = ((V + 31) >> 5) + kBmPad;
    for (int w = g.t; w < words; w += kTW) bm[w] = 0;
    __syncthreads();
    const HistRange hr = history_range(a, r);
    const int h0 = hr.h0, h1 = hr.h1;
    bool bad = false;
    for (int hb = h0; hb < h1; hb += 8 * kTW) {  // eight ids per thread in flight
        int id[8];
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const int h = hb + k * kTW + g.t;
            id[k] = h < h1 ? a.hist_ids[h] : 0;
        }
#pragma unroll
        for (int k = 0; k < 8; k++) {
            if (hb + k * kTW + g.t >= h1) continue;
            if ((unsigned)id[k] >= (unsigned)V) bad = true;
            else atomicOr(&bm[id[k] >> 5], 1u << (id[k] & 31));
        }
    }
    if (g.any(bad)) {
        if (g.t == 0) put_id(a, r, VXS_ERR_ID_OUT_OF_RANGE);
        return false;
    }
    return true;
}

// The general algorithm for row r (every option mix; the rows the ordered pass leaves).
__device__ __forceinline__ void wide_general_row(const SampleArgs& a, int vec, int r, BlkW& g, WideSmem& s,
                                                 uint32_t* bm_dyn) {
    const int V = a.vocab;
    const vxs_params P = a.params[(int64_t)r * a.params_stride];
    const float* __restrict__ xrow = a.logits + (int64_t)r * a.ld;
    float* orow = a.out_logits ? a.out_logits + (int64_t)r * V : nullptr;
    double* prow = a.out_probs ? a.out_probs + (int64_t)r * V : nullptr;
    const bool stop_pen = (a.kflags & KF_STOP_AFTER_PENALTY) != 0;

    // ---- history bitmap (S1)
    RowX X;
    X.bm = nullptr;
    X.rho = P.rep_penalty;
    X.rinv = 1.0f / P.rep_penalty;
    X.fastdiv = __builtin_fabsf(P.rep_penalty) >= 0x1p-60f && __builtin_fabsf(P.rep_penalty) <= 0x1p60f;
    if (P.rep_penalty != 1.0f && has_history(a)) {
        if (!build_bitmap(g, a, r, V, bm_dyn)) return;
        X.bm = bm_dyn;
    }
    if (stop_pen) {  // ApplyRepetitionPenalty alone: write the penalised row
        RowX P1 = X;
        P1.sb = P1.se = 0;
        P1.keep = P1.ban = -1;
        P1.invT = 1.0f;
        for_row(xrow, V, vec, g.t, P1, [&](int i, float x) { orow[i] = x; });
        if (g.t == 0) put_id(a, r, 0);
        return;
    }
    X.sb = max(P.supp_begin, 0);
    X.se = min(P.supp_end, V);
    if (!(P.supp_begin < P.supp_end)) X.sb = X.se = 0;
    X.keep = P.keep_id;
    X.ban = P.ban_id;
    const bool greedy = !P.do_sample;
    X.invT = row_inv_temp(P);
    if (g.t == 0) s.tau_key = 0;
    __syncthreads();

    // ---- pass A: each wave streams its own quarter of the row (no workgroup barrier inside):
    // statistics, greedy argmax and its own top-k candidate buffer. A wave's buffer keeps every
    // entry >= the k-th largest the wave has seen, which never exceeds the row's k-th largest, so
    // the four buffers together hold every entry the reference keeps.
    const int K = P.top_k;
    const bool kstream = !greedy && K > 0 && K <= kKMax && K < V;
    // With rho >= 1 the penalty never raises a value and with 1/T > 0 scaling keeps order, so an
    // entry below tau before its penalty stays below after it: the penalty is then applied to the
    // few candidates only. Otherwise every entry is penalised as it streams.
    const bool pen_late = X.bm && P.rep_penalty >= 1.0f && X.invT > 0.0f && !greedy;
    // wave-uniform switches (readfirstlane lets the compiler branch on them instead of masking)
    const bool pen_each = __builtin_amdgcn_readfirstlane(X.bm != nullptr && !pen_late);
    const bool supp_any = __builtin_amdgcn_readfirstlane(X.se > X.sb || X.ban >= 0);
    const int Q = ((V + kTW * 4 - 1) / (kTW * 4)) * 256;  // a wave's range, a multiple of 256
    const int lo = g.wv * Q, hi = min(V, lo + Q);
    uint32_t* wkey = s.wkey[g.wv];
    int32_t* widx = s.widx[g.wv];
    bool collect = kstream;  // false once ties overflow the wave's buffer
    int wn = 0;               // wave-uniform buffer fill
    float tau = -3.402823466e38f;  // entries below tau are not candidates (-inf never is)
    float bv = kNegInf, tmx = kNegInf, xmin = kPosInf;
    int bi = 0x7fffffff;
    bool bad = false;
    uint32_t ninf = 0;  // wave-uniform count of -inf entries
    // Raw buffer loads bounded by the end of the wave's range: loads past it read zeros without
    // fetching (lanes past the row end, the prefetch beyond the range), so every sweep is one
    // branch-free 16-byte load per lane (entries at or past `hi` are masked) and the next wave's
    // entries are not fetched twice.
    typedef float f4 __attribute__((ext_vector_type(4)));
    const __amdgpu_buffer_rsrc_t rowbuf =
        __builtin_amdgcn_make_buffer_rsrc((void*)xrow, (short)0, hi * (int)sizeof(float), 0x00020000);
    auto load4 = [&](int base) -> f4 {
        return __builtin_bit_cast(f4, __builtin_amdgcn_raw_buffer_load_b128(rowbuf, (base + 4 * g.lane) * 4, 0, 2));
    };
    // raw entries of one sweep -> values after penalty (unless deferred), suppression, temperature
    auto prep = [&](int base, f4 q, float* x, float* v) {
        const int i0 = base + 4 * g.lane;
        x[0] = q.x;
        x[1] = q.y;
        x[2] = q.z;
        x[3] = q.w;
#pragma unroll
        for (int j = 0; j < 4; j++) v[j] = x[j];
        if (pen_each) {
            const uint32_t word = X.bm[i0 >> 5];  // the 4 entries share one bitmap word
#pragma unroll
            for (int j = 0; j < 4; j++)
                if ((word >> ((i0 + j) & 31)) & 1u) v[j] = penalize(v[j], X.rho, X.rinv, X.fastdiv);
        }
        if (supp_any &&
            __builtin_amdgcn_readfirstlane((base < X.se && base + 256 > X.sb) || (X.ban >= base && X.ban < base + 256))) {
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int i = i0 + j;
                if ((i >= X.sb && i < X.se && i != X.keep) || i == X.ban) v[j] = kNegInf;
            }
        }
#pragma unroll
        for (int j = 0; j < 4; j++) v[j] *= X.invT;
        if (__builtin_amdgcn_readfirstlane(base + 256 > hi)) {  // the range's last sweep: mask its end
#pragma unroll
            for (int j = 0; j < 4; j++) v[j] = i0 + j < hi ? v[j] : kNegInf;
        }
    };
    auto sweep_greedy = [&](int base, f4 q) {  // a lane's indices ascend: strict > keeps its first max
        float x[4], v[4];
        prep(base, q, x, v);
        const int i0 = base + 4 * g.lane;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            bad |= v[j] != v[j];
            const bool take = i0 + j < hi && (v[j] > bv || bi == 0x7fffffff);
            bv = take ? v[j] : bv;
            bi = take ? i0 + j : bi;
        }
    };
    auto sweep_sample = [&](int base, f4 q) {
        float x[4], v[4];
        prep(base, q, x, v);
        const int i0 = base + 4 * g.lane;
        bool cand[4];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            bad |= __builtin_amdgcn_class(v[j], 0x203);  // NaN or +inf
            xmin = fminf(xmin, x[j]);
            tmx = fmaxf(tmx, v[j]);
            ninf += (uint32_t)__builtin_popcountll(__ballot(v[j] == kNegInf && i0 + j < hi));
            cand[j] = v[j] >= tau;
        }
        if (!collect) return;
        if (!__ballot(cand[0] || cand[1] || cand[2] || cand[3])) return;
        // another wave may have raised the shared bound: use it too
        const float ts = key2f(__hip_atomic_load(&s.tau_key, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP));
        if (ts > tau) {
            tau = ts;
#pragma unroll
            for (int j = 0; j < 4; j++) cand[j] = cand[j] && v[j] >= tau;
        }
        if (pen_late) {  // the candidates' exact values
            const uint32_t word = X.bm[i0 >> 5];
#pragma unroll
            for (int j = 0; j < 4; j++)
                if (cand[j] && ((word >> ((i0 + j) & 31)) & 1u)) {
                    v[j] = penalize(x[j], X.rho, X.rinv, X.fastdiv) * X.invT;
                    cand[j] = v[j] >= tau;
                }
        }
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const bool c = collect && cand[j] && v[j] >= tau;
            const uint64_t bal = __ballot(c);
            if (bal) {
                if (c) {
                    const uint32_t pos = (uint32_t)wn + __builtin_amdgcn_mbcnt_hi(
                                                            (uint32_t)(bal >> 32),
                                                            __builtin_amdgcn_mbcnt_lo((uint32_t)bal, 0u));
                    wkey[pos] = f2key(v[j]);
                    widx[pos] = i0 + j;
                }
                wn += __builtin_popcountll(bal);
                if (wn > kCapW - 64) {  // room for less than one more slot: raise tau and compact
                    wave_sync();
                    const uint32_t kth = wave_kth(wkey, g.lane, wn, K);
                    wn = wave_filter(wkey, widx, g.lane, wn, kth);
                    tau = fmaxf(tau, key2f(kth));
                    if (g.lane == 0) atomicMax(&s.tau_key, kth);
                    if (wn > kCapW - 64) collect = false;  // ties: the general path below
                }
            }
        }
    };
    // kPF sweeps in flight per lane: the next group's loads are issued before this group is used
    // (loads past the row return zeros, so they are issued unconditionally: no branch around a
    // load keeps the wait counters exact)
    constexpr int kPF = 8;
    auto stream = [&](auto sweep) {
        f4 cur[kPF];
#pragma unroll
        for (int q = 0; q < kPF; q++) cur[q] = load4(lo + q * 256);
        for (int gb = lo; gb < hi; gb += kPF * 256) {
            f4 nxt[kPF];
#pragma unroll
            for (int q = 0; q < kPF; q++) nxt[q] = load4(gb + (kPF + q) * 256);
#pragma unroll
            for (int q = 0; q < kPF; q++)
                if (gb + q * 256 < hi) sweep(gb + q * 256, cur[q]);
#pragma unroll
            for (int q = 0; q < kPF; q++) cur[q] = nxt[q];
        }
    };
    if (greedy) stream(sweep_greedy);
    else stream(sweep_sample);
    const bool huge = xmin < -1.0e37f;  // a deferred penalty might overflow such a value to -inf
    if (g.lane == 0) s.wcnt[g.wv] = collect ? wn : -1;
    if (g.any(bad)) {
        if (g.t == 0) put_id(a, r, VXS_ERR_NONFINITE);
        return;
    }
    if (greedy) {
        // first index of the maximum across the workgroup (wave ranges ascend in index)
        const float wbv = wave_fmax(bv);
        const uint32_t wbi = wave_umin(bv == wbv ? (uint32_t)bi : 0xffffffffu);
        if (g.lane == 0) {
            s.slot[2][g.wv] = __float_as_uint(wbv);
            s.slot[3][g.wv] = wbi;
        }
        __syncthreads();
        float best = __uint_as_float((uint32_t)s.slot[2][0]);
        uint32_t besti = (uint32_t)s.slot[3][0];
#pragma unroll
        for (int w = 1; w < kWW; w++) {
            const float ov = __uint_as_float((uint32_t)s.slot[2][w]);
            const uint32_t oi = (uint32_t)s.slot[3][w];
            if (ov > best || (ov == best && oi < besti)) {
                best = ov;
                besti = oi;
            }
        }
        if (g.t == 0) put_id(a, r, (int)besti);
        if (orow) for_row(xrow, V, vec, g.t, X, [&](int i, float x) { orow[i] = x; });
        if (prow)
            for (int i = g.t; i < V; i += kTW) prow[i] = 0.0;
        return;
    }
    // Statistics of pass A are exact unless the penalty was deferred to candidates: then the max
    // comes from the candidates (the maximum is always one) and, if a penalty could overflow a
    // value to -inf, the general path recounts with the full transform.
    float mx = key2f(g.umax(f2key(wave_fmax(tmx))));
    uint32_t cnt = (uint32_t)V -
                   (uint32_t)g.combine(g.lane == 0 ? ninf : 0u, [](uint64_t p, uint64_t q) { return p + q; });
    const bool restat = pen_late && g.any(huge);
    if (restat) {
        float m2 = kNegInf;
        uint32_t c2 = 0;
        for_row(xrow, V, vec, g.t, X, [&](int, float v) {
            m2 = fmaxf(m2, v);
            c2 += v != kNegInf ? 1u : 0u;
        });
        mx = key2f(g.umax(f2key(wave_fmax(m2))));
        cnt = g.usum(c2);
    }
    const double u = row_uniform(a, r);
    if (cnt == 0) {  // every entry -inf: the reference's draw returns the last id
        if (g.t == 0) put_id(a, r, V - 1);
        if (orow) for_row(xrow, V, vec, g.t, X, [&](int i, float x) { orow[i] = x; });
        if (prow)
            for (int i = g.t; i < V; i += kTW) prow[i] = __builtin_nan("");
        return;
    }

    // ---- streaming top-k result: exact k-th largest over the four buffers, then the exact regime
    const bool topk_on = K > 0 && K < V && (uint32_t)K < cnt;
    bool fast = kstream && !restat;
#pragma unroll
    for (int w = 0; w < kWW; w++) fast = fast && s.wcnt[w] >= 0;
    float kth = kNegInf;
    if (fast) {
        int wc[kWW];
#pragma unroll
        for (int w = 0; w < kWW; w++) wc[w] = s.wcnt[w];
        // thread t looks at entries t, t+256, ... of the concatenated buffers
        auto valid = [&](int j) { return (j % kCapW) < wc[j / kCapW]; };
        const uint32_t* keys = &s.wkey[0][0];
        const int32_t* idxs = &s.widx[0][0];
        uint32_t kthkey = 0;
        if (topk_on) {  // radix select over the union
            uint32_t prefix = 0, mask = 0;
            int need = K;
#pragma unroll 1
            for (int shift = 24; shift >= 0; shift -= 8) {
                for (int b = g.t; b < kRB; b += kTW) s.h.hcnt[b] = 0;
                __syncthreads();
                for (int j = g.t; j < kWW * kCapW; j += kTW)
                    if (valid(j) && (keys[j] & mask) == prefix) atomicAdd(&s.h.hcnt[(keys[j] >> shift) & 0xff], 1u);
                __syncthreads();
                const uint32_t c = s.h.hcnt[kRB - 1 - g.t];
                uint32_t tot;
                const uint32_t above = g.excl(c, tot);
                int mine = -1;
                if ((int)above < need && (int)(above + c) >= need) mine = kRB - 1 - g.t;
                const uint32_t dg = g.umax((uint32_t)(mine + 1)) - 1;
                const uint32_t ab = g.umax(mine >= 0 ? above + 1 : 0) - 1;
                need -= (int)ab;
                prefix |= dg << shift;
                mask |= 0xffu << shift;
            }
            kthkey = prefix;
            kth = key2f(kthkey);
        }
        if (pen_late) {  // the exact maximum: the largest candidate
            uint32_t km = 0;
            for (int j = g.t; j < kWW * kCapW; j += kTW)
                if (valid(j)) km = max(km, keys[j]);
            mx = key2f(g.umax(km));
        }
        // the candidates (key >= kth) into the exact-regime arrays, then index order
        if (g.t == 0) s.n = 0;
        __syncthreads();
        for (int j = g.t; j < kWW * kCapW; j += kTW)
            if (valid(j) && keys[j] >= kthkey) {
                const int q = atomicAdd(&s.n, 1);
                if (q < kCandW) {
                    s.ex.ci[q] = idxs[j];
                    s.ex.cx[q] = key2f(keys[j]);
                }
            }
        __syncthreads();
        const int n = s.n;
        if (n <= kCandW) {
            int ij = 0;
            float xj = 0.0f;
            if (g.t < n) {
                ij = s.ex.ci[g.t];
                xj = s.ex.cx[g.t];
            }
            int rank = 0;
#pragma unroll 8
            for (int l = 0; l < n; l++) rank += s.ex.ci[l] < ij;  // batched LDS reads
            __syncthreads();
            if (g.t < n) {
                s.ex.ci[rank] = ij;
                s.ex.cx[rank] = xj;
            }
            __syncthreads();
            if (orow) for_row(xrow, V, vec, g.t, X, [&](int i, float x) { orow[i] = x < kth ? kNegInf : x; });
            if (prow)
                for (int i = g.t; i < V; i += kTW) prow[i] = 0.0;
            __syncthreads();
            const int id = exact_block(g, s, n, mx, P.top_p < 1.0f, P.top_p, u, prow);
            if (g.t == 0) put_id(a, r, id);
            return;
        }
    }

    // =================== general path: several passes over the row ===================
    if (pen_late && !restat) {  // the exact maximum with the full transform
        float m2 = kNegInf;
        for_row(xrow, V, vec, g.t, X, [&](int, float v) { m2 = fmaxf(m2, v); });
        mx = key2f(g.umax(f2key(wave_fmax(m2))));
    }
    // exact k-th largest over the whole row (radix select on keys), when top-k is active
    if (topk_on) {
        uint32_t prefix = 0, mask = 0;
        int need = K;
#pragma unroll 1
        for (int shift = 24; shift >= 0; shift -= 8) {
            for (int b = g.t; b < kRB; b += kTW) s.h.hcnt[b] = 0;
            __syncthreads();
            for_row(xrow, V, vec, g.t, X, [&](int, float v) {
                const uint32_t key = f2key(v);
                if (v != kNegInf && (key & mask) == prefix) atomicAdd(&s.h.hcnt[(key >> shift) & 0xff], 1u);
            });
            __syncthreads();
            const uint32_t c = s.h.hcnt[kRB - 1 - g.t];
            uint32_t tot;
            const uint32_t above = g.excl(c, tot);
            int mine = -1;
            if ((int)above < need && (int)(above + c) >= need) mine = kRB - 1 - g.t;
            const uint32_t dg = g.umax((uint32_t)(mine + 1)) - 1;
            const uint32_t ab = g.umax(mine >= 0 ? above + 1 : 0) - 1;
            need -= (int)ab;
            prefix |= dg << shift;
            mask |= 0xffu << shift;
        }
        kth = key2f(prefix);
    }
    auto val = [&](int i, float x) -> float { return x < kth ? kNegInf : x; };  // top-k mask
    if (orow) for_row(xrow, V, vec, g.t, X, [&](int i, float x) { orow[i] = val(i, x); });
    // fixed-point masses of d = x - max
    const int F = min(51, 53 - (32 - __clz(V - 1)));
    const double scaleF = __builtin_ldexp(1.0, F);
    const float Cb = mass_bias(F);
    auto wof = [&](float v) -> double { return fixed_mass(exp_neg(v - mx), Cb, scaleF); };
    float dc = kNegInf;  // cut: keep d > dc, or d == dc with index >= ic
    int ic = 0;
    double Skept;
    if (P.top_p < 1.0f) {
        // mass-weighted radix select over f2key(d): first entry in ascending (d, index) order whose
        // inclusive cumulative mass exceeds T = floor(thr * S)
        const double thr = (double)(1.0f - P.top_p);
        uint32_t prefix = 0, mask = 0;
        double below = 0.0, T = 0.0, S = 0.0;
        bool last_only = false;
#pragma unroll 1
        for (int shift = 24; shift >= 0; shift -= 8) {
            for (int b = g.t; b < kRB; b += kTW) s.h.hmass[b] = 0.0;
            __syncthreads();
            for_row(xrow, V, vec, g.t, X, [&](int i, float x) {
                const float v = val(i, x);
                if (v == kNegInf) return;
                const float d = v - mx;
                const uint32_t key = f2key(d);
                if ((key & mask) == prefix) atomicAdd(&s.h.hmass[(key >> shift) & 0xff], wof(v));
            });
            __syncthreads();
            const double hb = s.h.hmass[g.t];  // thread b owns digit b (ascending)
            double tot;
            const double run = g.excl(hb, tot);
            if (shift == 24) {
                S = tot;
                if (!(thr < 1.0)) {
                    last_only = true;
                    break;
                }
                T = floor(thr * S);
                if (T >= S) {
                    last_only = true;
                    break;
                }
            }
            const double rest = T - below;
            int mine = -1;
            if (run <= rest && rest - run < hb) mine = g.t;
            const uint32_t dg = g.umax((uint32_t)(mine + 1)) - 1;
            if (g.t == (int)dg) s.slot[0][0] = (uint64_t)__double_as_longlong(run);
            __syncthreads();
            below += __longlong_as_double((long long)s.slot[0][0]);
            __syncthreads();
            prefix |= dg << shift;
            mask |= 0xffu << shift;
        }
        if (last_only) {
            // the last entry in (d, index) order: the maximum with the highest index
            int li = -1;
            for_row(xrow, V, vec, g.t, X, [&](int i, float x) {
                if (val(i, x) == mx) li = max(li, i);
            });
            ic = (int)g.umax((uint32_t)(li + 1)) - 1;
            dc = 0.0f;
            double wl = 0.0;
            if (g.t == 0) wl = wof(mx);
            below = S - g.dsum(wl);
        } else {
            // ties at the cut key: the crossing follows index order among them
            dc = key2f(prefix);
            ic = -1;
            double run = below;
            for (int base = 0; base < V && ic < 0; base += kSweepW) {
                const int i0 = base + 4 * g.t;
                double w4[4];
                double mine = 0.0;
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const int i = i0 + j;
                    w4[j] = 0.0;
                    if (i < V) {
                        const float v = val(i, X(i, xrow[i]));
                        if (v != kNegInf && v - mx == dc) w4[j] = wof(v);
                    }
                    mine += w4[j];
                }
                double tot;
                const double ex0 = g.excl(mine, tot);
                int hit = -1;
                double hb = 0.0;
                if (T >= run + ex0 && T - (run + ex0) < mine) {
                    double acc = run + ex0;
#pragma unroll
                    for (int j = 0; j < 4; j++) {
                        if (hit < 0 && w4[j] > 0.0 && T - acc < w4[j]) {
                            hit = i0 + j;
                            hb = acc;
                        }
                        acc += w4[j];
                    }
                }
                const int h = (int)g.umax((uint32_t)(hit + 1)) - 1;
                if (h >= 0) {
                    if (hit == h) s.slot[0][0] = (uint64_t)__double_as_longlong(hb);
                    __syncthreads();
                    below = __longlong_as_double((long long)s.slot[0][0]);
                    __syncthreads();
                    ic = h;
                }
                run += tot;
            }
            if (ic < 0) ic = 0x7fffffff;  // unreachable for a crossing key range
        }
        Skept = S - below;
    } else {
        double ls = 0.0;
        for_row(xrow, V, vec, g.t, X, [&](int i, float x) {
            const float v = val(i, x);
            if (v != kNegInf) ls += wof(v);
        });
        Skept = g.dsum(ls);
    }
    auto kept = [&](int i, float v) {
        if (v == kNegInf) return false;
        const float d = v - mx;
        return d > dc || (d == dc && i >= ic);
    };
    // draw: first kept index whose inclusive prefix mass exceeds floor(u * Skept)
    const double D = floor(u * Skept);
    double run = 0.0;
    int pick = -1;
    for (int base = 0; base < V && pick < 0; base += kSweepW) {
        const int i0 = base + 4 * g.t;
        double w4[4];
        double mine = 0.0;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int i = i0 + j;
            w4[j] = 0.0;
            if (i < V) {
                const float v = val(i, X(i, xrow[i]));
                if (kept(i, v)) w4[j] = wof(v);
            }
            mine += w4[j];
        }
        double tot;
        const double ex0 = g.excl(mine, tot);
        int hit = -1;
        if (D >= run + ex0 && D - (run + ex0) < mine) {
            double acc = run + ex0;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                acc += w4[j];
                if (hit < 0 && w4[j] > 0.0 && D < acc) hit = i0 + j;
            }
        }
        pick = (int)g.umax((uint32_t)(hit + 1)) - 1;
        run += tot;
    }
    if (pick < 0) {  // no crossing: the last kept id with p > 0
        int li = -1;
        for_row(xrow, V, vec, g.t, X, [&](int i, float x) {
            const float v = val(i, x);
            if (kept(i, v) && v - mx >= -745.1331787109375f) li = max(li, i);
        });
        pick = max((int)g.umax((uint32_t)(li + 1)) - 1, 0);
    }
    if (g.t == 0) put_id(a, r, pick);
    if (prow) {
        double se = 0.0;
        for_row(xrow, V, vec, g.t, X, [&](int i, float x) {
            const float v = val(i, x);
            if (kept(i, v)) se += exp_neg_prob(v - mx);
        });
        se = g.dsum(se);
        for_row(xrow, V, vec, g.t, X, [&](int i, float x) {
            const float v = val(i, x);
            prow[i] = kept(i, v) ? exp_neg_prob(v - mx) / se : 0.0;
        });
    }
}


// The smallest float x with fl(x * invT) >= tau, for finite tau and invT in (0, inf): then
// x >= xt  <=>  fl(x * invT) >= tau  for every x (fl(x * invT) is monotone in x, NaN fails both).
// Found from the quotient by a few steps in key order, with a bisection as the fallback.
__device__ __forceinline__ float x_threshold(float tau, float invT) {
    auto ok = [&](uint32_t k) { return key2f(k) * invT >= tau; };
    uint32_t k = f2key(tau / invT);
    if (k >= 0xff800001u) k = 0xff800000u;  // +inf at most
    if (k <= 0x007fffffu) k = 0x00800000u;  // above -inf
#pragma unroll 1
    for (int i = 0; i < 4 && ok(k - 1) && k > 0x00800000u; i++) k--;
#pragma unroll 1
    for (int i = 0; i < 4 && !ok(k); i++) k++;
    if (!(ok(k) && (k == 0x00800000u || !ok(k - 1)))) {  // not settled: bisect over [-FLT_MAX, +inf]
        uint32_t lo = 0x00800000u, hi = 0xff800000u;  // ok(hi) holds (tau is finite)
#pragma unroll 1
        while (lo < hi) {
            const uint32_t mid = lo + ((hi - lo) >> 1);
            if (ok(mid)) hi = mid;
            else lo = mid + 1;
        }
        k = lo;
    }
    return key2f(k);
}

// =====================================================================================
// The ordered pass: the rows row_ordered() selects, in one read of the row. Returns true when the
// general algorithm must serve the row instead.
//
// Pass A: each wave streams its quarter of the row and keeps a buffer of raw values and indices,
// in index order. The exact transformed value v (penalty, suppression, temperature) is at most
// fl(x * 1/T), which is monotone in the raw x, so an entry joins the buffer when x >= xt, the
// smallest float with fl(xt * 1/T) >= tau: one compare per entry. tau is a lower bound of the row's
// k-th largest, shared between the waves, from two rules: whenever a wave's buffer cannot take a
// sweep's entries, the exact values of its entries are formed (suppressed entries and those past
// the wave's range become -inf) and the buffer is cut to a lower bound of its k-th largest (k to
// k + 32 entries stay); and each wave publishes a key with at least ceil(k/4) of its entries at or
// above it (first from the sweeps in registers before the stream starts), so the smallest of the
// four has at least k of the row's entries at or above it. NaN and +inf reach the NaN-propagating
// maximum M of the raw values; M NaN or fl(M * 1/T) = +inf sends the row through an exact check
// with the full transform (suppression or the penalty may have removed or lowered that value).
// Tail: the four waves hold their buffers' exact keys in registers; a radix select over all of them
// (block_kth_radix) gives the row's k-th largest; the candidates are written in index order; each
// thread ranks its candidate by (d, index), d = v - max, and forms exp(d); one wave runs the
// reference's sequential fp64 arithmetic (S6-S8, Sampler.cs:51-87), its top-p cut from a wave scan
// checked against a rounding bound (wave_topp_cut_par) and its second sum and draw over the kept
// entries only. The (d, index) order is the reference's (p, index) order whenever each adjacent pair
// is in (p, index) order (p = exp(d) / sum never decreases with d for a monotone exp); otherwise the
// candidates are ranked by p directly. Rows that end with too many tied candidates go to the general
// algorithm.
// =====================================================================================
__device__ __forceinline__ bool wide_ordered_row(const SampleArgs& a, int vec, int r, BlkW& g, WideSmem& s,
                                                 uint32_t* bm_dyn) {
    const int V = a.vocab;
    const vxs_params P = a.params[(int64_t)r * a.params_stride];
    if (!row_ordered(a, P)) return true;  // the general algorithm serves it
    const float* __restrict__ xrow = a.logits + (int64_t)r * a.ld;
    const float invT = row_inv_temp(P);
    const int K = P.top_k;
    // HW_ID: SIMD_ID in bits 5:4, the workgroup's slot on its CU in bits 19:16. The wave whose
    // SIMD equals the slot runs this row's sequential tail, so the tails of the workgroups sharing a
    // CU land on different SIMDs (checked below: exactly one such wave, else wave 0).
    const uint32_t hw = __builtin_amdgcn_s_getreg((31 << 11) | 4);
    const uint32_t slot = (hw >> 16) & 3u;
    if (g.lane == 0) s.wslot[g.wv] = ((hw >> 4) & 3u) == slot ? 1 : 0;

    // the wave ranges and the row loads (the first sweeps are in flight while the bitmap is built)
    const int Q = ((V + kTW * 4 - 1) / (kTW * 4)) * 256;  // a wave's range, a multiple of 256
    const int lo = g.wv * Q, hi = min(V, lo + Q);
    typedef float f4 __attribute__((ext_vector_type(4)));
    // raw buffer loads bounded by the end of the wave's range: loads past it (the prefetch beyond the
    // range, lanes past the row end) read zeros without fetching, so the next wave's entries are
    // not fetched twice
    const __amdgpu_buffer_rsrc_t rowbuf =
        __builtin_amdgcn_make_buffer_rsrc((void*)xrow, (short)0, hi * (int)sizeof(float), 0x00020000);
    auto load4 = [&](int base) -> f4 {
        return __builtin_bit_cast(f4, __builtin_amdgcn_raw_buffer_load_b128(rowbuf, (base + 4 * g.lane) * 4, 0, 2));
    };
    constexpr int kPF = 6;  // sweeps in flight per lane
    f4 cur[kPF];
#pragma unroll
    for (int q = 0; q < kPF; q++) cur[q] = load4(lo + q * 256);

    RowX X;
    X.bm = nullptr;
    X.rho = P.rep_penalty;
    X.rinv = 1.0f / P.rep_penalty;
    X.fastdiv = __builtin_fabsf(P.rep_penalty) >= 0x1p-60f && __builtin_fabsf(P.rep_penalty) <= 0x1p60f;
    if (P.rep_penalty != 1.0f && has_history(a)) {
        if (!build_bitmap(g, a, r, V, bm_dyn)) return false;
        X.bm = bm_dyn;
    }
    X.sb = max(P.supp_begin, 0);
    X.se = min(P.supp_end, V);
    if (!(P.supp_begin < P.supp_end)) X.sb = X.se = 0;
    X.keep = P.keep_id;
    X.ban = P.ban_id;
    X.invT = invT;
    if (g.t == 0) s.tau_key = 0;
    // The exact value of entry i: the full transform (penalty, suppression, temperature); entries
    // past the wave's range (the zeros loaded beyond the row end) are -inf.
    auto vexact = [&](int i, float x) -> float { return i < hi ? X(i, x) : kNegInf; };
    // The quarter bounds: a wave with at least kq = ceil(k/4) entries at or above key b_w publishes
    // b_w (0 = none yet); the four waves' ranges are disjoint, so the row holds at least 4 kq >= k
    // entries at or above min_w b_w, a lower bound of its k-th largest. A wave's b_w only rises (it
    // is taken over more of the wave's entries each time). The first ones come from the kPF sweeps
    // already in registers.
    const int Kq = (K + 3) / 4;
    {
        uint32_t kk[kPF * 4];
        uint32_t klo = 0xffffffffu, khi = 0;
        int nf = 0;
#pragma unroll
        for (int q = 0; q < kPF; q++) {
            const float xv[4] = {cur[q].x, cur[q].y, cur[q].z, cur[q].w};
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const float v = vexact(lo + q * 256 + 4 * g.lane + j, xv[j]);
                const bool fin = v > kNegInf;
                kk[4 * q + j] = fin ? f2key(v) : 0u;
                klo = fin ? min(klo, kk[4 * q + j]) : klo;
                khi = fin ? max(khi, kk[4 * q + j]) : khi;
                nf += __builtin_popcountll(__ballot(fin));
            }
        }
        const uint32_t b = nf >= Kq ? wave_bound_regs(kk, wave_umin(klo), wave_umax(khi), Kq, 16) : 0u;
        if (g.lane == 0) s.qkey[g.wv] = b;
    }
    __syncthreads();

    // ---- pass A
    uint32_t* wkey = s.wkey[g.wv];
    int32_t* widx = s.widx[g.wv];
    // kStop: the wave stopped collecting (the general algorithm then serves the row); kCompacted: its
    // buffer does not hold every finite entry it has seen (it was compacted, or a bound applied from
    // the start). One word, only ever or-ed: two flag variables had their stores merged behind a
    // selected address, which kept them in scratch memory.
    constexpr uint32_t kStop = 1u, kCompacted = 2u;
    uint32_t state = 0;
    int wn = 0;                     // wave-uniform buffer fill
    float tau = -3.402823466e38f;   // entries with fl(x * 1/T) < tau are not candidates ...
    float M = kNegInf;              // NaN-propagating maximum of the raw entries
    auto qmin = [&]() {
        uint32_t m = 0xffffffffu;
#pragma unroll
        for (int w = 0; w < kWW; w++)
            m = min(m, __hip_atomic_load(&s.qkey[w], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP));
        return m;
    };
    {
        const uint32_t t0 = qmin();
        if (t0 != 0u) {
            tau = key2f(t0);
            state |= kCompacted;
            if (g.lane == 0) atomicMax(&s.tau_key, t0);
        }
    }
    float xt = x_threshold(tau, invT);  // entries with x < xt are not candidates
    // Keep the buffered entries whose exact value is >= a lower bound of the k-th largest exact
    // value buffered (one that leaves k to k + 32 of them, ties aside), or the shared bound if that
    // is larger; tau rises to it. With fewer than k finite values buffered the wave stops
    // collecting.
    auto compact = [&]() {
        wave_sync();
        uint32_t kk[kPerL];
        float xr[kPerL];
        int32_t ii[kPerL];
        uint32_t klo = 0xffffffffu, khi = 0;
        int nf = 0;
#pragma unroll
        for (int q = 0; q < kPerL; q++) {
            const int j = g.lane + 64 * q;
            xr[q] = __uint_as_float(wkey[j]);
            ii[q] = widx[j];
            const bool in = j < wn;
            const float v = vexact(in ? ii[q] : lo, xr[q]);
            const bool fin = in && v > kNegInf;
            kk[q] = fin ? f2key(v) : 0u;
            klo = fin ? min(klo, kk[q]) : klo;
            khi = fin ? max(khi, kk[q]) : khi;
            nf += __builtin_popcountll(__ballot(fin));
        }
        if (nf < K) {
            state |= kStop;
            return;
        }
        // a lower bound of the row's k-th largest that keeps at most k + 32 entries (untied), and
        // this wave's quarter bound (the buffer holds every seen entry at or above its k-th largest)
        const uint32_t kmax = wave_umax(khi);
        const uint32_t kown = wave_bound_regs(kk, wave_umin(klo), kmax, K, 32);
        const uint32_t qb = wave_bound_regs(kk, kown, kmax, Kq, 16);
        if (g.lane == 0) {
            atomicMax(&s.qkey[g.wv], qb);
            atomicMax(&s.tau_key, max(kown, qmin()));
        }
        const uint32_t kth = max(kown, __hip_atomic_load(&s.tau_key, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP));
        wave_sync();
        uint32_t m = 0;
#pragma unroll
        for (int q = 0; q < kPerL; q++) {
            const bool keep = kk[q] >= kth;  // empty and -inf slots hold 0 < kth
            const uint64_t bal = __ballot(keep);
            if (keep) {
                const uint32_t pos = m + __builtin_amdgcn_mbcnt_hi((uint32_t)(bal >> 32),
                                                                   __builtin_amdgcn_mbcnt_lo((uint32_t)bal, 0u));
                wkey[pos] = __float_as_uint(xr[q]);
                widx[pos] = ii[q];
            }
            m += (uint32_t)__builtin_popcountll(bal);
        }
        wave_sync();
        wn = __builtin_amdgcn_readfirstlane((int)m);
        tau = key2f(kth);
        xt = x_threshold(tau, invT);
        if (g.lane == 0) atomicMax(&s.tau_key, kth);
        state |= kCompacted;
    };
    // kPF sweeps in flight per lane: the next group's loads are issued before this group is used
    // (loads past the row return zeros, so they are issued unconditionally)
    {
        for (int gb = lo; gb < hi; gb += kPF * 256) {
            // The workgroups sharing a CU take turns at the highest wave priority, about 10 us
            // each (s_memrealtime counts at 100 MHz): with equal priorities the oldest workgroup's
            // loads issue first and the rows finish pass A in order of age, 90 to 112 us into the
            // wide workload's step, so the last rows' tails end the step; in turns the rows finish
            // it together (99 to 108 us) and the step takes 129 instead of 132 us.
            {
                const uint32_t turn = ((uint32_t)(__builtin_amdgcn_s_memrealtime() >> 10) + slot) & 3u;
                if (turn == 0) __builtin_amdgcn_s_setprio(0);
                else if (turn == 1) __builtin_amdgcn_s_setprio(1);
                else if (turn == 2) __builtin_amdgcn_s_setprio(2);
                else __builtin_amdgcn_s_setprio(3);
            }
            // another wave may have raised the shared bound: use it too
            const uint32_t ts = __hip_atomic_load(&s.tau_key, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
            f4 nxt[kPF];
#pragma unroll
            for (int q = 0; q < kPF; q++) nxt[q] = load4(gb + (kPF + q) * 256);
            if (ts > f2key(tau)) {
                tau = key2f(ts);
                xt = x_threshold(tau, invT);
            }
#pragma unroll
            for (int q = 0; q < kPF; q++) {
                const int base = gb + q * 256;
                if (base >= hi || (state & kStop)) continue;  // (no early exits: they cost structurizer state)
                const float xv[4] = {cur[q].x, cur[q].y, cur[q].z, cur[q].w};
                M = __builtin_elementwise_maximum(M, __builtin_elementwise_maximum(xv[0], xv[1]));
                M = __builtin_elementwise_maximum(M, __builtin_elementwise_maximum(xv[2], xv[3]));
                int cnt = 0;
#pragma unroll
                for (int j = 0; j < 4; j++) cnt += __builtin_popcountll(__ballot(xv[j] >= xt));
                if (wn + cnt > kCapW) {  // full: compact, then test again against the raised bound
                    compact();
                    cnt = 0;
#pragma unroll
                    for (int j = 0; j < 4; j++) cnt += __builtin_popcountll(__ballot(xv[j] >= xt));
                    if (wn + cnt > kCapW) state |= kStop;  // ties: the general algorithm
                }
                if (cnt == 0 || (state & kStop)) continue;
                // in index order: a lane's position is the buffer fill plus the candidates of the lower
                // lanes, counted from the three bits of each lane's count (0..4)
                const int i0 = base + 4 * g.lane;
                int c = 0;
#pragma unroll
                for (int j = 0; j < 4; j++) c += xv[j] >= xt ? 1 : 0;
                const uint64_t b0 = __ballot(c & 1), b1 = __ballot(c & 2), b2 = __ballot(c & 4);
                auto below = [](uint64_t b) {
                    return __builtin_amdgcn_mbcnt_hi((uint32_t)(b >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)b, 0u));
                };
                uint32_t pos = (uint32_t)wn + below(b0) + 2 * below(b1) + 4 * below(b2);
#pragma unroll
                for (int j = 0; j < 4; j++)
                    if (xv[j] >= xt) {
                        wkey[pos] = __float_as_uint(xv[j]);
                        widx[pos] = i0 + j;
                        pos++;
                    }
                wn = __builtin_amdgcn_readfirstlane(wn + cnt);
            }
            state = __builtin_amdgcn_readfirstlane(state);
            if (state & kStop) break;
#pragma unroll
            for (int q = 0; q < kPF; q++) cur[q] = nxt[q];
        }
    }
    // The buffered entries as keys of their exact values, in registers in index order (slot
    // lane + 64 q), those below the shared bound dropped (0: no entry). The bound never exceeds the
    // row's k-th largest, so every entry the reference keeps stays.
    uint32_t kk[kPerL];
    int32_t ii[kPerL];
    uint32_t klo = 0xffffffffu, khi = 0;
    int nf = 0;
    {
        wave_sync();
        const uint32_t ts = __hip_atomic_load(&s.tau_key, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
#pragma unroll
        for (int q = 0; q < kPerL; q++) {
            const int j = g.lane + 64 * q;
            ii[q] = widx[j];
            const bool in = j < wn && !(state & kStop);
            const float v = vexact(in ? ii[q] : lo, __uint_as_float(wkey[j]));
            const uint32_t key = f2key(v);
            const bool keep = in && v > kNegInf && key >= ts;
            kk[q] = keep ? key : 0u;
            klo = keep ? min(klo, key) : klo;
            khi = keep ? max(khi, key) : khi;
            nf += __builtin_popcountll(__ballot(keep));
        }
        klo = wave_umin(klo);
        khi = wave_umax(khi);
    }
    // The row's tail after its pass runs at wave priority 1, and from the rank on at 0: the rows of
    // the CU still streaming their pass (at turns 2 and 3) keep the issue slots, and the tail fills
    // the ones they leave (wide workload 128.4 -> 127.0 us; the tail at priorities 3, 2, 1, 0 by
    // phase measured 128.1, at 0 throughout 127.8).
    __builtin_amdgcn_s_setprio(1);
    // NaN or fl(M * 1/T) = +inf in a wave's range: the row is checked exactly below
    const bool wbad = wave_any(M != M || M * invT == kPosInf);
    if (g.lane == 0) {
        s.wcnt[g.wv] = (state & kStop) ? -1 : nf;
        s.wcomp[g.wv] = (state & kCompacted) ? 1 : 0;
        s.wklo[g.wv] = klo;
        s.wkhi[g.wv] = khi;
        s.wbad[g.wv] = wbad ? 1 : 0;
    }
    s.h.h3[g.t] = 0u;  // the first histogram of the k-th largest select
    __syncthreads();
    // The finite count is the buffered total unless some wave's buffer does not hold every finite
    // entry of its range (compacted, or a bound applied), which takes at least k finite entries (a
    // count of "many" decides top-k the same way).
    bool all = true, comp = false, anybad = false;
    uint32_t tot = 0;
    klo = 0xffffffffu;
    khi = 0;
#pragma unroll
    for (int w = 0; w < kWW; w++) {
        all = all && s.wcnt[w] >= 0;
        comp = comp || s.wcomp[w] != 0;
        anybad = anybad || s.wbad[w] != 0;
        tot += (uint32_t)max(s.wcnt[w], 0);
        klo = min(klo, s.wklo[w]);
        khi = max(khi, s.wkhi[w]);
    }
    // check the row exactly with the full transform (suppression, or a penalty, may have removed or
    // lowered that value)
    if (anybad) {
        bool bad = false;
        for_row(xrow, V, vec, g.t, X, [&](int, float v) { bad |= __builtin_amdgcn_class(v, 0x203); });
        if (g.any(bad)) {
            if (g.t == 0) put_id(a, r, VXS_ERR_NONFINITE);
            return false;
        }
    }
    if (!all) return true;  // a wave stopped collecting: the general algorithm takes the row
    const uint32_t cnt = comp ? (uint32_t)V : tot;
    float* orow = a.out_logits ? a.out_logits + (int64_t)r * V : nullptr;
    double* prow = a.out_probs ? a.out_probs + (int64_t)r * V : nullptr;
    if (cnt == 0) {  // every entry -inf: the reference's draw returns the last id
        if (g.t == 0) put_id(a, r, V - 1);
        if (orow) for_row(xrow, V, vec, g.t, X, [&](int i, float x) { orow[i] = x; });
        if (prow)
            for (int i = g.t; i < V; i += kTW) prow[i] = __builtin_nan("");
        return false;
    }
    const bool topk_on = (uint32_t)K < cnt;

    bool worker = g.wv == 0;  // the wave that runs the sequential tail
    {
        int nw = 0;
#pragma unroll
        for (int w = 0; w < kWW; w++) nw += s.wslot[w];
        if (nw == 1) worker = s.wslot[g.wv] != 0;
    }
    // ---- all waves: the k-th largest of the buffered keys, the maximum, the candidates
    const uint32_t kthkey = topk_on ? block_kth_radix(kk, klo, khi, K, s.h.h3, g.t, g.lane) : 1u;
    const float mx = key2f(khi);
    // the candidates (keys >= the k-th largest; 0 < 1 <= every valid key) in index order: the
    // waves' counts, then each wave writes its own after those of the waves before it
    {
        uint32_t mine = 0;
#pragma unroll
        for (int q = 0; q < kPerL; q++) mine += (uint32_t)__builtin_popcountll(__ballot(kk[q] >= kthkey));
        if (g.lane == 0) s.wcand[g.wv] = (int32_t)mine;
    }
    __syncthreads();
    int n = 0, off = 0;
#pragma unroll
    for (int w = 0; w < kWW; w++) {
        off += w < g.wv ? s.wcand[w] : 0;
        n += s.wcand[w];
    }
    if (n > kCandW) return true;  // ties beyond the exact-regime capacity: the general algorithm
    // (d, index) keys, d = v - max, over the wave buffers (every wave has read its own into registers)
    uint64_t* ckey = reinterpret_cast<uint64_t*>(&s.wkey[0][0]);
    {
        uint32_t m = (uint32_t)off;
#pragma unroll
        for (int q = 0; q < kPerL; q++) {
            const bool keep = kk[q] >= kthkey;
            const uint64_t bal = __ballot(keep);
            if (keep) {
                const uint32_t pos = m + __builtin_amdgcn_mbcnt_hi((uint32_t)(bal >> 32),
                                                                   __builtin_amdgcn_mbcnt_lo((uint32_t)bal, 0u));
                const float v = key2f(kk[q]);
                s.ex.cx[pos] = v;
                s.ex.ci[pos] = ii[q];
                ckey[pos] = ((uint64_t)f2key(v - mx) << 32) | (uint32_t)ii[q];
            }
            m += (uint32_t)__builtin_popcountll(bal);
        }
        if (g.t < 8) ckey[n + g.t] = ~0ull;  // above every key: the rank loop reads whole groups of eight
    }
    const float kth = topk_on ? key2f(kthkey) : kNegInf;
    if (orow) for_row(xrow, V, vec, g.t, X, [&](int i, float x) { orow[i] = x < kth ? kNegInf : x; });
    if (prow)
        for (int i = g.t; i < V; i += kTW) prow[i] = 0.0;
    __syncthreads();

    __builtin_amdgcn_s_setprio(0);
    // ---- all waves: thread t holds candidate t (index order); its position in (d, index) order,
    // counted over the keys eight at a time, and its exp(d)                        Sampler.cs:57
    if (g.t < n) {
        const uint64_t kt = ckey[g.t];
        typedef unsigned long long u64x2 __attribute__((ext_vector_type(2)));
        const u64x2* kp = reinterpret_cast<const u64x2*>(ckey);
        auto below = [&](const u64x2 (&q)[4]) {
            int c = 0;
#pragma unroll
            for (int k = 0; k < 4; k++) c += (q[k].x < kt ? 1 : 0) + (q[k].y < kt ? 1 : 0);
            return c;
        };
        // the next group's reads are issued before the current group is counted
        u64x2 ga[4], gb[4];
#pragma unroll
        for (int k = 0; k < 4; k++) ga[k] = kp[k];
        int po = 0, l = 8;
        for (; l + 8 < n; l += 16) {
#pragma unroll
            for (int k = 0; k < 4; k++) gb[k] = kp[l / 2 + k];
            po += below(ga);
#pragma unroll
            for (int k = 0; k < 4; k++) ga[k] = kp[l / 2 + 4 + k];
            po += below(gb);
        }
        if (l < n) {
#pragma unroll
            for (int k = 0; k < 4; k++) gb[k] = kp[l / 2 + k];
            po += below(ga);
#pragma unroll
            for (int k = 0; k < 4; k++) ga[k] = gb[k];
        }
        po += below(ga);
        s.ex.cs[po] = (int16_t)g.t;
        s.ex.cp[g.t] = exp((double)(s.ex.cx[g.t] - mx));
    }
    __syncthreads();
    if (!worker) return false;

    // ---- the worker wave: the reference's fp64 arithmetic on the candidates in index order
    double* cp = s.ex.cp;
    const double sum = seq_sum_pipe(cp, n);  // sequential in index order              :58
    for (int j = g.lane; j < n; j += 64) cp[j] = cp[j] / sum;  //                         :60
    wave_sync();
    if (P.top_p < 1.0f) {  //                                                          :62-75
        bool ok = true;
        for (int q = g.lane; q < n - 1; q += 64) {
            const int a0 = s.ex.cs[q], b0 = s.ex.cs[q + 1];
            const double pa = cp[a0], pb = cp[b0];
            ok = ok && (pa < pb || (pa == pb && a0 < b0));
        }
        if (__ballot(!ok)) {  // rank by (p, index) directly
            int rk[kCandW / 64];
#pragma unroll
            for (int k = 0; k < kCandW / 64; k++) {
                const int j = g.lane + 64 * k;
                rk[k] = j < n ? seq_rank(cp, n, j) : 0;
            }
            wave_sync();
#pragma unroll
            for (int k = 0; k < kCandW / 64; k++) {
                const int j = g.lane + 64 * k;
                if (j < n) s.ex.cs[rk[k]] = (int16_t)j;
            }
            wave_sync();
        }
        // the last sorted position is never removed (the reference's loop runs j < n - 1)
        double* ps = reinterpret_cast<double*>(&s.widx[0][0]);  // p in (p, index) order
        for (int q = g.lane; q < n; q += 64) ps[q] = cp[s.ex.cs[q]];
        wave_sync();
        const int nrem = wave_topp_cut_par(ps, n, (double)(1.0f - P.top_p), g.lane);
        for (int q = g.lane; q < nrem; q += 64) cp[s.ex.cs[q]] = 0.0;
        wave_sync();
        // The entries left with p > 0 (or NaN), in index order: the second sum and the draw over
        // them alone are the reference's over all n (adding zero changes no sum; the draw skips
        // p <= 0).
        double* kp = ps;  // the sorted copy is no longer needed
        int32_t* kid = &s.widx[2][0];
        int nk = 0;
        for (int b = 0; b < n; b += 64) {
            const int j = b + g.lane;
            const double pj = j < n ? cp[j] : 0.0;
            const bool keep = j < n && !(pj <= 0.0);
            const uint64_t bal = __ballot(keep);
            if (keep) {
                const int pos = nk + (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(bal >> 32),
                                                                    __builtin_amdgcn_mbcnt_lo((uint32_t)bal, 0u));
                kp[pos] = pj;
                kid[pos] = s.ex.ci[j];
            }
            nk += __builtin_popcountll(bal);
        }
        wave_sync();
        const double s2 = seq_sum(kp, nk);  // probs.Sum() in index order               :73
        for (int q = g.lane; q < nk; q += 64) kp[q] = kp[q] / s2;  //                  :74
        if (prow)
            for (int j = g.lane; j < n; j += 64) cp[j] = cp[j] / s2;
        wave_sync();
        const double u = row_uniform(a, r);
        const int pick = wave_draw(kp, kid, nk, u);  // inverse-CDF draw in index order :77-87
        if (g.lane == 0) put_id(a, r, pick);
    } else {
        const double u = row_uniform(a, r);
        const int pick = wave_draw(cp, s.ex.ci, n, u);  // inverse-CDF draw in index order :77-87
        if (g.lane == 0) put_id(a, r, pick);
    }
    if (prow)
        for (int j = g.lane; j < n; j += 64) prow[s.ex.ci[j]] = cp[j];
    return false;
}

// One workgroup per row: the ordered pass when the row's options allow it, else (or when that pass
// hands the row back) the general algorithm, in the same workgroup.
__global__ __launch_bounds__(kTW) __attribute__((amdgpu_waves_per_eu(4))) void sample_wide_kernel(SampleArgs a,
                                                                                                 int vec) {
    extern __shared__ uint32_t bm_dyn[];  // penalised-id bitmap, ceil(vocab / 32) words
    __shared__ WideSmem s;
    BlkW g;
    g.t = threadIdx.x;
    g.lane = g.t & 63;
    g.wv = __builtin_amdgcn_readfirstlane(g.t >> 6);  // wave-uniform: wave ranges live in SGPRs
    g.s = &s;
    const int r = blockIdx.x;
    if (!wide_ordered_row(a, vec, r, g, s, bm_dyn)) return;
    __syncthreads();  // the ordered pass is done with the LDS
    wide_general_row(a, vec, r, g, s, bm_dyn);
}

}  // namespace

hipError_t launch_sample_wide(const SampleArgs& a, hipStream_t stream) {
    if (a.rows <= 0) return hipSuccess;
    if (a.vocab <= 0 || a.vocab > kWideMaxVocab) return hipErrorNotSupported;
    const int vec = (a.ld % 4 == 0) && (((uintptr_t)a.logits & 15u) == 0) ? 1 : 0;
    const size_t dyn = sizeof(uint32_t) * (size_t)((a.vocab + 31) / 32 + kBmPad);
    hipLaunchKernelGGL(sample_wide_kernel, dim3(a.rows), dim3(kTW), dyn, stream, a, vec);
    return hipGetLastError();
}

}  // namespace vxs
