// vxs_kernels.hip — gfx950 kernels of the token sampler.
//
// Row-resident sampler: one 256-thread workgroup (4 wave64) owns one row of up to 1024*NC logits
// and keeps it in VGPRs from the single HBM read (16-byte non-temporal loads; thread t holds the
// elements c*1024 + 4t + j) to the sampled id.
//
//   S1 penalty      the row is staged in LDS; distinct history ids are found with an LDS bitmap
//                   (atomicOr) and the first setter of each id rescales that logit in place
//                   (fp32 s*rho, or the correctly rounded s/rho)                 Sampler.cs:25-33
//   S2 suppression  [supp_begin, supp_end) except keep_id, then ban_id -> -inf   TalkerGenerator.cs:247-248
//   S3 greedy       first index of the max, no temperature                       Sampler.cs:37,90-95
//   S4 temperature  x * fl32(1/T)                                                Sampler.cs:39-40
//   S5 top-k        k-th largest value (ties kept) by a count-weighted bucket select  Sampler.cs:42-49
//   S6-S8, two regimes after top-k:
//     exact      <= 256 candidates: compacted in index order; the reference's sequential fp64
//                arithmetic runs on them (exp, index-order sum, stable (p, index) order, top-p
//                cut, renormalisation, index-order draw)                          Sampler.cs:51-87
//     nucleus    more candidates (full-vocabulary top-p): masses exp(x - max) are evaluated in
//                fp32 (relative error ~2e-7) and rounded to multiples of 2^-F held in doubles, so
//                every sum (histogram atomics, totals, prefixes) is exact and order-independent.
//                One pass fills per-sweep LDS histograms over d = x - max; wave 0 scans them for
//                the bucket where the ascending cumulative mass crosses (1 - top_p) * total and
//                ranks that bucket's few elements by (d, index) for the exact cut; the sweep
//                totals above the cut give the kept mass per sweep, so the index-order draw for
//                floor(u * kept mass) only revisits the one sweep that contains it.
//
// Per-row errors are reported in out_ids[row] as negative VXS_ERR_* codes.
#include <atomic>
#include <math.h>
#include <stdint.h>

#include "vxs_device.h"
#include "vxs_internal.h"
#include "vxs_wave.h"

namespace vxs {
namespace {

using namespace dev;

constexpr int kT = 256;         // threads per row (one workgroup)
constexpr int kWaves = kT / 64;
constexpr int kSW = 4 * kT;     // elements per float4 sweep
constexpr int kCandMax = 256;   // candidate count of the exact sequential regime
constexpr int kLMax = 2 * kT;   // generic select: elements ranked exactly after bucketing
constexpr int kNB = 1024;       // generic select: buckets (4 per thread)
constexpr int kNBLog = 10;
constexpr int kNLMax = 128;     // nucleus cut: crossing-bucket elements ranked by wave 0

template <int NC>
struct Cfg {
    static constexpr int NE = 4 * NC;   // elements per thread
    static constexpr int VMAX = NC * kSW;
    static constexpr int BMW = VMAX / 32;
    static constexpr int NBP = NC <= 3 ? 1024 : (NC <= 6 ? 512 : 256);  // nucleus buckets per sweep
    static constexpr int BPL = NBP / 64;                                // ... per lane of wave 0
    static_assert(NE <= 64, "element masks are 64-bit");
};

// Workgroup-combine sites: each is written once per row, so no trailing barrier is needed; the
// refinement loop reuses its sites with an explicit barrier.
enum Site : int {
    kSiteErr,
    kSiteErr2,
    kSiteNan,
    kSiteArgV,
    kSiteArgI,
    kSiteStat0,  // + 4
    kSiteFmin = kSiteStat0 + 4,
    kSiteCnt2,
    kSiteScanK,
    kSiteLRankK,
    kSiteLRankP,
    kSiteScanP,
    kSiteDraw,
    kSiteLast,
    kSitePSum,
    kSiteRefine,
    kSiteRefine2,
    kSiteRefine3,
    kSiteTk0,    // + 3
    kSiteComp0 = kSiteTk0 + 3,  // + NC
    kSiteChunk0 = kSiteComp0 + 8,  // + NC
    kSiteNScan0 = kSiteChunk0 + 8,  // + NC + 1
    kSites = kSiteNScan0 + 9,
};

struct Blk {
    int lane, wv, t;
    uint64_t (*slot)[4];

    __device__ __forceinline__ void sync() const { __syncthreads(); }
    // combine one wave-uniform 64-bit value per wave across the workgroup
    template <class Op>
    __device__ __forceinline__ uint64_t combine(uint64_t w, int site, Op op) const {
        if (lane == 0) slot[site][wv] = w;
        __syncthreads();
        uint64_t r = slot[site][0];
#pragma unroll
        for (int i = 1; i < kWaves; i++) r = op(r, slot[site][i]);
        return r;
    }
    __device__ __forceinline__ uint32_t sum(uint32_t x, int site) const {
        return (uint32_t)combine(wave_sum(x), site, [](uint64_t p, uint64_t q) { return p + q; });
    }
    __device__ __forceinline__ uint32_t wsum_u(uint32_t w, int site) const {  // w wave-uniform
        return (uint32_t)combine(w, site, [](uint64_t p, uint64_t q) { return p + q; });
    }
    __device__ __forceinline__ double dsum(double x, int site) const {
        return __longlong_as_double((long long)combine((uint64_t)__double_as_longlong(wave_sum(x)), site,
                                                       [](uint64_t p, uint64_t q) {
                                                           return (uint64_t)__double_as_longlong(
                                                               __longlong_as_double((long long)p) +
                                                               __longlong_as_double((long long)q));
                                                       }));
    }
    __device__ __forceinline__ float fmin_(float x, int site) const {
        return __uint_as_float((uint32_t)combine(__float_as_uint(wave_min(x)), site, [](uint64_t p, uint64_t q) {
            return (uint64_t)__float_as_uint(fminf(__uint_as_float((uint32_t)p), __uint_as_float((uint32_t)q)));
        }));
    }
    __device__ __forceinline__ uint32_t umax(uint32_t x, int site) const {
        return (uint32_t)combine(wave_umax(x), site, [](uint64_t p, uint64_t q) { return p > q ? p : q; });
    }
    __device__ __forceinline__ uint32_t umin(uint32_t x, int site) const {
        return (uint32_t)combine(wave_umin(x), site, [](uint64_t p, uint64_t q) { return p < q ? p : q; });
    }
    __device__ __forceinline__ int imax(int x, int site) const {  // x >= -1
        return (int)umax((uint32_t)(x + 1), site) - 1;
    }
    __device__ __forceinline__ bool any(bool p, int site) const {
        return combine(wave_any(p) ? 1u : 0u, site, [](uint64_t a, uint64_t b) { return a | b; }) != 0;
    }
    // workgroup-wide exclusive prefix sums in thread order
    __device__ __forceinline__ uint32_t excl_scan(uint32_t v, int site, uint32_t& total) const {
        const uint32_t incl = wave_incl_sum(v);
        if (lane == 0) slot[site][wv] = readlane(incl, 63);
        __syncthreads();
        uint32_t base = 0, tot = 0;
#pragma unroll
        for (int i = 0; i < kWaves; i++) {
            const uint32_t s = (uint32_t)slot[site][i];
            base += i < wv ? s : 0;
            tot += s;
        }
        total = tot;
        return base + incl - v;
    }
    __device__ __forceinline__ uint64_t excl_scan(uint64_t v, int site, uint64_t& total) const {
        const uint64_t incl = wave_incl_sum(v);
        if (lane == 0) slot[site][wv] = readlane64(incl, 63);
        __syncthreads();
        uint64_t base = 0, tot = 0;
#pragma unroll
        for (int i = 0; i < kWaves; i++) {
            const uint64_t s = slot[site][i];
            base += i < wv ? s : 0;
            tot += s;
        }
        total = tot;
        return base + incl - v;
    }
    __device__ __forceinline__ double excl_scan(double v, int site, double& total) const {
        const double incl = wave_incl_sum(v);
        if (lane == 0) slot[site][wv] = (uint64_t)__double_as_longlong(readlane_d(incl, 63));
        __syncthreads();
        double base = 0, tot = 0;
#pragma unroll
        for (int i = 0; i < kWaves; i++) {
            const double s = __longlong_as_double((long long)slot[site][i]);
            base += i < wv ? s : 0.0;
            tot += s;
        }
        total = tot;
        return base + incl - v;  // exact: integer-valued doubles below 2^53
    }
};

struct Ctl {
    int32_t sel_b;
    uint32_t list_n;
    double sel_below;
    uint32_t sel_key;
    int32_t sel_idx;
    double sel_cbelow;
    int32_t found;
    // nucleus cut (written by wave 0)
    double S, T, below;
    int32_t bstar;
    double kept[8];
    float tk_kth;  // top-k: the k-th largest value ...
    int32_t tk_cnt;  // ... and the count of entries at or above it
};

template <int NC>
struct RowSmem {
    float tmax[kT];  // the threads' largest values (published with the row statistics, read by top-k)
    using C = Cfg<NC>;
    uint32_t bm[C::BMW];
    union {
        float xs[C::VMAX];  // staged row for the penalty
        struct {
            double hist[kNB];
            uint32_t lkey[kLMax];
            int32_t lidx[kLMax];
            double lw[kLMax];
            double lws[kLMax];   // weights in rank order
            int16_t lat[kLMax];  // list entry at each rank
        } sel;
        double nh[NC][C::NBP];  // nucleus histograms, one per sweep
        struct {
            alignas(16) float cx[kCandMax];
            int32_t ci[kCandMax];
            double cp[kCandMax];
            double ps[kCandMax];   // p in (p, index) order, for the top-p cut
            double pre[kCandMax];  // the running sums of the cut and of the draw
            int16_t cs[kCandMax];
            int32_t nrem;
        } ex;
    } u;
    struct {
        uint32_t key[kNLMax];
        int32_t idx[kNLMax];
        double w[kNLMax];
        double ws[kNLMax];
        int16_t at[kNLMax];
    } nl;
    Ctl ctl;
    uint64_t slot[kSites][4];
};

// First element, in ascending (key, index) order over the `act` elements, at which the inclusive
// cumulative weight exceeds T (weights and T are integer-valued doubles below 2^53); `sel.hist`
// must be zero on entry. Returns key, index (only if need_idx) and the cumulative weight strictly
// before the element. When the total weight is <= T the last element is returned. Level 1 spreads
// the elements over kNB buckets with `b1` (monotone in key); a bucket with more than kLMax elements
// is split in the u32 key space until few elements or a single key remain; the survivors are ranked
// exactly.
template <int NC, class KeyF, class WtF, class B1F>
__device__ __forceinline__ void block_select(const Blk& g, RowSmem<NC>& sm, uint64_t act, double T, bool need_idx,
                                             KeyF key, WtF wt, B1F b1, int scan_site, int rank_site,
                                             uint32_t& okey, int& oidx, double& obelow) {
    constexpr int NE = Cfg<NC>::NE;
    auto& s = sm.u.sel;
    auto eidx = [&](int e) { return (e >> 2) * kSW + g.t * 4 + (e & 3); };

#pragma unroll
    for (int e = 0; e < NE; e++)
        if ((act >> e) & 1u) atomicAdd(&s.hist[b1(e)], wt(e));
    if (g.t == 0) {
        sm.ctl.sel_b = -1;
        sm.ctl.list_n = 0;
    }
    g.sync();
    double below;
    int bstar;
    {
        double h[4];
        double tot = 0.0;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            h[j] = s.hist[g.t * 4 + j];
            tot += h[j];
        }
        double all;
        const double excl = g.excl_scan(tot, scan_site, all);
        if (all <= T) {  // no crossing: the last element in (key, index) order
            uint32_t km = 0;
#pragma unroll
            for (int e = 0; e < NE; e++)
                if ((act >> e) & 1u) km = max(km, key(e));
            km = g.umax(km, kSiteRefine);
            g.sync();
            int im = -1;
#pragma unroll
            for (int e = 0; e < NE; e++)
                if (((act >> e) & 1u) && key(e) == km) im = max(im, eidx(e));
            im = g.imax(im, kSiteRefine2);
            g.sync();
            double wl = 0.0;
#pragma unroll
            for (int e = 0; e < NE; e++)
                if (((act >> e) & 1u) && eidx(e) == im) wl = wt(e);
            wl = g.dsum(wl, kSiteRefine3);
            g.sync();
            okey = km;
            oidx = im;
            obelow = all - wl;
            return;
        }
        if (excl <= T && T - excl < tot) {
            double run = excl;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                if (T - run < h[j]) {
                    sm.ctl.sel_b = g.t * 4 + j;
                    sm.ctl.sel_below = run;
                    break;
                }
                run += h[j];
            }
        }
        g.sync();
        bstar = sm.ctl.sel_b;
        below = sm.ctl.sel_below;
    }
    uint64_t in = 0;
#pragma unroll
    for (int e = 0; e < NE; e++)
        if (((act >> e) & 1u) && b1(e) == bstar) in |= 1ull << e;

    // gather the bucket's elements (slots beyond kLMax are only counted)
#pragma unroll
    for (int e = 0; e < NE; e++)
        if ((in >> e) & 1u) {
            const uint32_t k = atomicAdd(&sm.ctl.list_n, 1u);
            if (k < (uint32_t)kLMax) {
                s.lkey[k] = key(e);
                s.lidx[k] = eidx(e);
                s.lw[k] = wt(e);
            }
        }
    g.sync();
    uint32_t n = sm.ctl.list_n;

    if (n > (uint32_t)kLMax) {
        // ---- crowded bucket: split its key interval until <= kLMax elements or a single key remain
        uint32_t klo, khi;
        {
            uint32_t mn = 0xffffffffu, mx = 0;
#pragma unroll
            for (int e = 0; e < NE; e++)
                if ((in >> e) & 1u) {
                    mn = min(mn, key(e));
                    mx = max(mx, key(e));
                }
            klo = g.umin(mn, kSiteRefine);
            khi = g.umax(mx, kSiteRefine2);
            g.sync();
        }
        while (n > (uint32_t)kLMax && klo != khi) {
            const uint32_t range = khi - klo;
            const int bits = 32 - __clz(range);
            const int shift = bits > kNBLog ? bits - kNBLog : 0;
            for (int b = g.t; b < kNB; b += kT) s.hist[b] = 0.0;
            if (g.t == 0) sm.ctl.sel_b = -1;
            g.sync();
#pragma unroll
            for (int e = 0; e < NE; e++)
                if ((in >> e) & 1u) atomicAdd(&s.hist[(key(e) - klo) >> shift], wt(e));
            g.sync();
            const double T2 = T - below;
            double h[4];
            double tot = 0.0;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                h[j] = s.hist[g.t * 4 + j];
                tot += h[j];
            }
            double all;
            const double excl = g.excl_scan(tot, kSiteRefine, all);
            if (excl <= T2 && T2 - excl < tot) {
                double run = excl;
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    if (T2 - run < h[j]) {
                        sm.ctl.sel_b = g.t * 4 + j;
                        sm.ctl.sel_below = run;
                        break;
                    }
                    run += h[j];
                }
            }
            g.sync();
            const int b2 = sm.ctl.sel_b;
            below += sm.ctl.sel_below;
            const uint64_t lo2 = (uint64_t)klo + ((uint64_t)b2 << shift);
            const uint64_t hi2 = min((uint64_t)khi, lo2 + ((1ull << shift) - 1));
            uint64_t in2 = 0;
            uint32_t mn = 0xffffffffu, mx = 0, cnt = 0;
#pragma unroll
            for (int e = 0; e < NE; e++)
                if (((in >> e) & 1u) && key(e) >= lo2 && key(e) <= hi2) {
                    in2 |= 1ull << e;
                    mn = min(mn, key(e));
                    mx = max(mx, key(e));
                    cnt++;
                }
            in = in2;
            klo = g.umin(mn, kSiteRefine2);
            khi = g.umax(mx, kSiteRefine3);
            g.sync();
            n = g.sum(cnt, kSiteRefine);
            g.sync();
        }
        if (klo == khi && n > (uint32_t)kLMax) {
            // ties: every remaining element has key klo and the same weight; order is by index
            okey = klo;
            oidx = -1;
            double mine = 0.0;
#pragma unroll
            for (int e = 0; e < NE; e++)
                if ((in >> e) & 1u) mine = wt(e);
            const uint64_t mb = (uint64_t)__double_as_longlong(mine);  // non-negative: bits order as values
            const uint64_t wb = ((uint64_t)g.umax((uint32_t)(mb >> 32), kSiteRefine) << 32) |
                                g.umax((uint32_t)mb, kSiteRefine2);
            g.sync();
            const double wtie = __longlong_as_double((long long)wb);
            if (!need_idx) {
                obelow = below;
                return;
            }
            const uint64_t nth = (uint64_t)(T - below) / (uint64_t)wtie;
            obelow = below + (double)nth * wtie;
            uint32_t base = 0;
            if (g.t == 0) sm.ctl.found = -1;
#pragma unroll
            for (int c = 0; c < NC; c++) {
                const uint32_t mine4 = (uint32_t)(in >> (c * 4)) & 0xfu;
                const uint32_t cnt = (uint32_t)__builtin_popcount(mine4);
                uint32_t total;
                const uint32_t excl = g.excl_scan(cnt, kSiteRefine3, total);
                if (nth >= (uint64_t)base + excl && nth < (uint64_t)base + excl + cnt) {
                    uint64_t k = nth - base - excl;
#pragma unroll
                    for (int j = 0; j < 4; j++)
                        if ((mine4 >> j) & 1u) {
                            if (k == 0) {
                                sm.ctl.found = c * kSW + g.t * 4 + j;
                                break;
                            }
                            k--;
                        }
                }
                base += total;
                g.sync();
            }
            oidx = sm.ctl.found;
            g.sync();
            return;
        }
        // gather the (now small) interval
        if (g.t == 0) sm.ctl.list_n = 0;
        g.sync();
#pragma unroll
        for (int e = 0; e < NE; e++)
            if ((in >> e) & 1u) {
                const uint32_t k = atomicAdd(&sm.ctl.list_n, 1u);
                s.lkey[k] = key(e);
                s.lidx[k] = eidx(e);
                s.lw[k] = wt(e);
            }
        g.sync();
        n = sm.ctl.list_n;
    }

    // ---- rank the list by (key, index); thread t then owns ranks 2t and 2t+1
    for (int a = g.t; a < (int)n; a += kT) {
        const uint32_t ka = s.lkey[a];
        const int ia = s.lidx[a];
        int rank = 0;
#pragma unroll 8
        for (int b = 0; b < (int)n; b++) {
            const uint32_t kb = s.lkey[b];
            const int ib = s.lidx[b];
            rank += (int)((kb < ka) | ((kb == ka) & (ib < ia)));  // bitwise: no branch per comparison
        }
        s.lws[rank] = s.lw[a];
        s.lat[rank] = (int16_t)a;
    }
    if (g.t == 0) sm.ctl.sel_idx = -1;
    g.sync();
    const int r0 = 2 * g.t;
    const double w0 = r0 < (int)n ? s.lws[r0] : 0.0;
    const double w1 = r0 + 1 < (int)n ? s.lws[r0 + 1] : 0.0;
    double tot;
    const double ex = g.excl_scan(w0 + w1, rank_site, tot);
    {
        const double c0 = below + ex;  // cumulative weight before rank r0
        int prank = -1;
        double pbelow = 0.0;
        if (r0 < (int)n && T >= c0 && T - c0 < w0) {
            prank = r0;
            pbelow = c0;
        } else if (r0 + 1 < (int)n && T >= c0 + w0 && T - (c0 + w0) < w1) {
            prank = r0 + 1;
            pbelow = c0 + w0;
        }
        if (prank >= 0) {
            const int at = s.lat[prank];
            sm.ctl.sel_key = s.lkey[at];
            sm.ctl.sel_idx = s.lidx[at];
            sm.ctl.sel_cbelow = pbelow;
        }
    }
    g.sync();
    okey = sm.ctl.sel_key;
    oidx = sm.ctl.sel_idx;
    obelow = sm.ctl.sel_cbelow;
    g.sync();
}

// Occupancy target: 4 waves per SIMD where 128 VGPRs hold the row without spills.
template <int NC>
constexpr int kWavesPerEu = NC <= 3 ? 4 : 1;

// One row by the whole 256-thread workgroup (every thread calls it; it returns uniformly).
template <int NC>
__device__ __forceinline__ void row_block(const SampleArgs& a, int vec, int r, RowSmem<NC>& sm) {
    using C = Cfg<NC>;
    constexpr int NE = C::NE;

    Blk g;
    g.lane = threadIdx.x & 63;
    g.wv = threadIdx.x >> 6;
    g.t = threadIdx.x;
    g.slot = sm.slot;
    auto eidx = [&](int e) { return (e >> 2) * kSW + g.t * 4 + (e & 3); };

    const int V = a.vocab;
    const float* __restrict__ xrow = a.logits + (int64_t)r * a.ld;

    // ---- the row loads first, then the options and the history range (independent of each
    // other, so that inputs read over PCIe cost one round trip before the history ids)
    // No lane branches around these loads: a divergent branch runs both sides under exec masks,
    // and the compiler then waits for the loads of one side before the other side's next load,
    // which puts one round trip per sweep on a row read over PCIe.
    float v[NE];
#pragma unroll
    for (int c = 0; c < NC; c++) {
        const int i0 = c * kSW + g.t * 4;
        if (vec && (c + 1) * kSW <= V) {  // uniform: a full sweep, one aligned quad per thread
            typedef float f4 __attribute__((ext_vector_type(4)));
            const f4 q = __builtin_nontemporal_load((const f4*)(xrow + i0));
            v[c * 4 + 0] = q.x;
            v[c * 4 + 1] = q.y;
            v[c * 4 + 2] = q.z;
            v[c * 4 + 3] = q.w;
        } else {  // unaligned rows and the partial last sweep: element loads at in-row addresses
#pragma unroll
            for (int j = 0; j < 4; j++) v[c * 4 + j] = xrow[min(i0 + j, V - 1)];
        }
    }
    vxs_params P;
    if (a.row_direct)
        P = a.direct_params;
    else
        P = a.params[(int64_t)r * a.params_stride];
    HistRange hr{0, 0};
    if (has_history(a)) hr = history_range(a, r);
    const bool pen_on = P.rep_penalty != 1.0f && has_history(a);
    constexpr int HP = 8;  // ids per thread fetched up front (2048 per row), in flight with the row
    const int h0 = hr.h0, h1 = pen_on ? hr.h1 : hr.h0;
    int pre[HP];
    if (pen_on) {
#pragma unroll
        for (int k = 0; k < HP; k++) {
            const int h = h0 + g.t + k * kT;
            pre[k] = h < h1 ? a.hist_ids[h] : 0;
        }
    }
    // entries past the vocabulary (pads of the last sweep) hold -inf: they never win, carry no mass
    // and are never written back (masked here, with the loads above all in flight)
#pragma unroll
    for (int e = 0; e < NE; e++)
        if ((e >> 2) * kSW + kSW > V && eidx(e) >= V) v[e] = kNegInf;

    // ---- S1: repetition penalty over the distinct history ids
    if (pen_on && h1 > h0) {
        const float rho = P.rep_penalty;
        const float rinv = 1.0f / rho;
        const float arho = __builtin_fabsf(rho);
        const bool fast = arho >= 0x1p-60f && arho <= 0x1p60f;
        // The row is staged in LDS. The first HP * kT ids (prefetched with the row): every thread
        // reads the staged logit of each of its ids, the workgroup synchronises, then every thread
        // writes the penalised value back, so a repeated id writes the same value again and each
        // distinct id is penalised once, with no atomics. A longer history marks those ids in an LDS
        // bitmap, and the thread whose atomicOr first sets a later id's bit rescales that one. Then
        // every thread reloads its elements.
        float* xs = sm.u.xs;
        typedef float f4 __attribute__((ext_vector_type(4)));
#pragma unroll
        for (int c = 0; c < NC; c++)
            *(f4*)(xs + c * kSW + g.t * 4) = f4{v[c * 4 + 0], v[c * 4 + 1], v[c * 4 + 2], v[c * 4 + 3]};
        const bool longer = h1 - h0 > HP * kT;  // uniform
        if (longer)
            for (int w = g.t; w < C::BMW; w += kT) sm.bm[w] = 0;
        g.sync();
        bool live[HP];
        float xv[HP];
        bool bad = false;
#pragma unroll
        for (int k = 0; k < HP; k++) {
            const bool in = h0 + g.t + k * kT < h1;
            bad |= in && (unsigned)pre[k] >= (unsigned)V;
            live[k] = in && (unsigned)pre[k] < (unsigned)V;
            xv[k] = live[k] ? xs[pre[k]] : 0.0f;
        }
        if (g.any(bad, kSiteErr)) {  // its barrier also orders every read above before the writes
            if (g.t == 0) put_id(a, r, VXS_ERR_ID_OUT_OF_RANGE);
            return;
        }
#pragma unroll
        for (int k = 0; k < HP; k++)
            if (live[k]) xs[pre[k]] = penalize(xv[k], rho, rinv, fast);
        if (longer) {
#pragma unroll
            for (int k = 0; k < HP; k++)
                if (live[k]) atomicOr(&sm.bm[pre[k] >> 5], 1u << (pre[k] & 31));
            g.sync();
            auto own = [&](int id) {
                if ((unsigned)id >= (unsigned)V) {
                    bad = true;
                    return;
                }
                const uint32_t bit = 1u << (id & 31);
                if (!(atomicOr(&sm.bm[id >> 5], bit) & bit)) xs[id] = penalize(xs[id], rho, rinv, fast);
            };
            for (int hb = h0 + HP * kT; hb < h1; hb += 4 * kT) {  // four ids per thread in flight
                int id[4];
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    const int h = hb + k * kT + g.t;
                    id[k] = h < h1 ? a.hist_ids[h] : 0;
                }
#pragma unroll
                for (int k = 0; k < 4; k++)
                    if (hb + k * kT + g.t < h1) own(id[k]);
            }
            if (g.any(bad, kSiteErr2)) {
                if (g.t == 0) put_id(a, r, VXS_ERR_ID_OUT_OF_RANGE);
                return;
            }
        } else {
            g.sync();  // every write above lands before the reload
        }
#pragma unroll
        for (int c = 0; c < NC; c++) {
            const f4 q = *(const f4*)(xs + c * kSW + g.t * 4);
            v[c * 4 + 0] = q.x;
            v[c * 4 + 1] = q.y;
            v[c * 4 + 2] = q.z;
            v[c * 4 + 3] = q.w;
        }
        g.sync();  // LDS is reused below
    }

    float* orow = a.out_logits ? a.out_logits + (int64_t)r * V : nullptr;
    double* prow = a.out_probs ? a.out_probs + (int64_t)r * V : nullptr;
    auto write_logits = [&]() {
        if (!orow) return;
#pragma unroll
        for (int e = 0; e < NE; e++)
            if (eidx(e) < V) orow[eidx(e)] = v[e];
    };

    if (a.kflags & KF_STOP_AFTER_PENALTY) {
        write_logits();
        if (g.t == 0) put_id(a, r, 0);
        return;
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

    // ---- S3: greedy
    if (!P.do_sample) {
        float bv = kNegInf;
        int bi = 0x7fffffff;
        bool nan = false;
#pragma unroll
        for (int e = 0; e < NE; e++) {
            nan |= v[e] != v[e];
            if (v[e] > bv || (v[e] == bv && eidx(e) < bi)) {
                bv = v[e];
                bi = eidx(e);
            }
        }
        wave_argmax(bv, bi);
        if (g.lane == 0) {
            g.slot[kSiteArgV][g.wv] = __float_as_uint(bv);
            g.slot[kSiteArgI][g.wv] = (uint32_t)bi;
        }
        const bool anynan = g.any(nan, kSiteNan);  // its barrier also publishes the argmax slots
        bv = __uint_as_float((uint32_t)g.slot[kSiteArgV][0]);
        bi = (int)g.slot[kSiteArgI][0];
#pragma unroll
        for (int i = 1; i < kWaves; i++) {
            const float ov = __uint_as_float((uint32_t)g.slot[kSiteArgV][i]);
            const int oi = (int)g.slot[kSiteArgI][i];
            if (ov > bv || (ov == bv && oi < bi)) {
                bv = ov;
                bi = oi;
            }
        }
        if (g.t == 0) put_id(a, r, anynan ? VXS_ERR_NONFINITE : bi);
        write_logits();
        if (prow)
#pragma unroll
            for (int e = 0; e < NE; e++)
                if (eidx(e) < V) prow[eidx(e)] = 0.0;
        return;
    }

    // ---- S4: temperature, and the finite-input contract
    const float invT = P.temperature == 1.0f ? 1.0f : 1.0f / P.temperature;
    if (invT != 1.0f) {
#pragma unroll
        for (int e = 0; e < NE; e++) v[e] *= invT;
        if (!(invT > 0.0f))  // negative or NaN scale: pads go back to -inf
#pragma unroll
            for (int e = 0; e < NE; e++)
                if (eidx(e) >= V) v[e] = kNegInf;
    }
    const bool topp = P.top_p < 1.0f;
    float mx, mn;  // max; min (including -inf entries)
    uint32_t cnt;  // finite entries
    {
        uint64_t badm = 0;
        float tmx = kNegInf, tmn = kPosInf;
#pragma unroll
        for (int e = 0; e < NE; e++) {
            badm |= __ballot((v[e] != v[e]) || v[e] == kPosInf);
            tmx = fmaxf(tmx, v[e]);
            tmn = fminf(tmn, v[e]);
        }
        sm.tmax[g.t] = tmx;
        const float wmx = wave_fmax(tmx);
        const float wmn = wave_fmin(tmn);
        if (g.lane == 0) {
            g.slot[kSiteStat0 + 0][g.wv] = __float_as_uint(wmx);
            g.slot[kSiteStat0 + 1][g.wv] = __float_as_uint(wmn);
            g.slot[kSiteStat0 + 3][g.wv] = badm != 0;
        }
        // zero the nucleus histograms while the statistics are published
        if (topp)
            for (int b = g.t; b < NC * C::NBP; b += kT) (&sm.u.nh[0][0])[b] = 0.0;
        g.sync();
        mx = kNegInf;
        mn = kPosInf;
        uint64_t anybad = 0;
#pragma unroll
        for (int i = 0; i < kWaves; i++) {
            mx = fmaxf(mx, __uint_as_float((uint32_t)g.slot[kSiteStat0 + 0][i]));
            mn = fminf(mn, __uint_as_float((uint32_t)g.slot[kSiteStat0 + 1][i]));
            anybad |= g.slot[kSiteStat0 + 3][i];
        }
        if (anybad) {
            if (g.t == 0) put_id(a, r, VXS_ERR_NONFINITE);
            return;
        }
        cnt = (uint32_t)V;
        if (mn == kNegInf) {  // some entries are -inf (suppressed, masked or pads): count the rest
            uint32_t cntw = 0;
#pragma unroll
            for (int e = 0; e < NE; e++) cntw += (uint32_t)__builtin_popcountll(__ballot(v[e] != kNegInf));
            cnt = g.wsum_u(cntw, kSiteStat0 + 2);
        }
    }

    // every entry is -inf: p = 0/0 everywhere and the reference's draw returns the last id
    if (cnt == 0) {
        if (g.t == 0) put_id(a, r, V - 1);
        write_logits();
        if (prow)
#pragma unroll
            for (int e = 0; e < NE; e++)
                if (eidx(e) < V) prow[eidx(e)] = __builtin_nan("");
        return;
    }

    // ---- S5: top-k (ties at the k-th value are kept)
    const int K = P.top_k;
    bool cands = false;  // the exact-regime arrays already hold the candidates in index order
    int ncand = 0;
    if (K > 0 && K < V && (uint32_t)K < cnt && K <= kCandMax) {
        // A lower bound T of the k-th largest: at least K of the 256 thread maxima (a subset of
        // the row) are >= T, and at most K + 8 unless ties force more (a tighter stop measured
        // faster than K + 32: fewer candidates to gather and count). When the entries >= T
        // fit the exact-regime capacity they are the candidates: all entries >= the k-th largest
        // are among them, so their own k-th largest is the row's.
        uint32_t mk[kT / 64];
        uint32_t mlo = 0xffffffffu, mhi = 0;
#pragma unroll
        for (int q = 0; q < kT / 64; q++) {
            mk[q] = f2key(sm.tmax[g.lane + 64 * q]);
            mlo = min(mlo, mk[q]);
            mhi = max(mhi, mk[q]);
        }
        const float Tb = key2f(wave_bound_regs4(mk, wave_umin(mlo), wave_umax(mhi), K, 8));
        // the entries >= Tb in index order: 16-bit counts per sweep, four sweeps per scan
        auto& ex = sm.u.ex;
        uint32_t tot = 0;
        uint64_t excl[(NC + 3) / 4], totals[(NC + 3) / 4];
#pragma unroll
        for (int h = 0; h < (NC + 3) / 4; h++) {
            uint64_t mine = 0;
#pragma unroll
            for (int c = 4 * h; c < NC && c < 4 * h + 4; c++) {
                uint32_t m = 0;
#pragma unroll
                for (int j = 0; j < 4; j++) m += v[c * 4 + j] >= Tb ? 1u : 0u;
                mine |= (uint64_t)m << (16 * (c - 4 * h));
            }
            excl[h] = g.excl_scan(mine, kSiteTk0 + h, totals[h]);
#pragma unroll
            for (int c = 4 * h; c < NC && c < 4 * h + 4; c++) tot += (uint32_t)((totals[h] >> (16 * (c - 4 * h))) & 0xffffu);
        }
        if (tot <= (uint32_t)kCandMax) {
            uint32_t base = 0;
#pragma unroll
            for (int c = 0; c < NC; c++) {
                const int h = c / 4, f = 16 * (c % 4);
                uint32_t off = base + (uint32_t)((excl[h] >> f) & 0xffffu);
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const int e = c * 4 + j;
                    if (v[e] >= Tb) {
                        ex.cx[off] = v[e];
                        ex.ci[off] = eidx(e);
                        off++;
                    }
                }
                base += (uint32_t)((totals[h] >> f) & 0xffffu);
            }
            g.sync();
            // the k-th largest with multiplicity: #{> x} < K <= #{>= x}
            const int n = (int)tot;
            if (g.t < n) {
                const float x = ex.cx[g.t];
                int gt = 0, ge = 0;
                typedef float f4v __attribute__((ext_vector_type(4)));
                const int n4 = n & ~3;
#pragma unroll 4
                for (int l = 0; l < n4; l += 4) {
                    const f4v y = *reinterpret_cast<const f4v*>(&ex.cx[l]);
                    gt += (y.x > x ? 1 : 0) + (y.y > x ? 1 : 0) + (y.z > x ? 1 : 0) + (y.w > x ? 1 : 0);
                    ge += (y.x >= x ? 1 : 0) + (y.y >= x ? 1 : 0) + (y.z >= x ? 1 : 0) + (y.w >= x ? 1 : 0);
                }
                for (int l = n4; l < n; l++) {
                    const float y = ex.cx[l];
                    gt += y > x ? 1 : 0;
                    ge += y >= x ? 1 : 0;
                }
                if (gt < K && K <= ge) {
                    sm.ctl.tk_kth = x;
                    sm.ctl.tk_cnt = ge;
                }
            }
            g.sync();
            const float kth = sm.ctl.tk_kth;
            cnt = (uint32_t)sm.ctl.tk_cnt;
#pragma unroll
            for (int e = 0; e < NE; e++)
                if (v[e] < kth) v[e] = kNegInf;
            g.sync();  // every thread has read the candidates: mask them
            if (g.t < n && ex.cx[g.t] < kth) ex.cx[g.t] = kNegInf;  // masked: probability 0
            mn = kth;
            cands = true;
            ncand = n;
        }
    }
    if (!cands && K > 0 && K < V && (uint32_t)K < cnt) {
        for (int b = g.t; b < kNB; b += kT) sm.u.sel.hist[b] = 0.0;
        uint64_t act = 0;
        float fmn = kPosInf;  // smallest finite value
#pragma unroll
        for (int e = 0; e < NE; e++)
            if (v[e] != kNegInf) {
                act |= 1ull << e;
                fmn = fminf(fmn, v[e]);
            }
        const float lo = g.fmin_(fmn, kSiteFmin);  // its barrier publishes the zeroed histogram
        const float span = mx - lo;                // may round; any monotone bucket map is exact here
        const float scale = (span > 0.0f && span < kPosInf) ? (float)kNB / span : 0.0f;
        auto b1 = [&](int e) -> int {
            float x = v[e];
            asm volatile("" : "+v"(x));
            return (int)fminf(fmaxf((x - lo) * scale, 0.0f), (float)(kNB - 1));
        };
        auto key = [&](int e) -> uint32_t {
            float x = v[e];
            asm volatile("" : "+v"(x));
            return f2key(x);
        };
        auto wt = [&](int) -> double { return 1.0; };
        uint32_t kkey;
        int kidx;
        double kbelow;
        block_select<NC>(g, sm, act, (double)(cnt - (uint32_t)K), false, key, wt, b1, kSiteScanK, kSiteLRankK, kkey,
                         kidx, kbelow);
        const float kth = key2f(kkey);
        uint32_t c2 = 0;
#pragma unroll
        for (int e = 0; e < NE; e++) {
            if (v[e] < kth) v[e] = kNegInf;
            c2 += (uint32_t)__builtin_popcountll(__ballot(v[e] != kNegInf));
        }
        if (topp)
            for (int b = g.t; b < NC * C::NBP; b += kT) (&sm.u.nh[0][0])[b] = 0.0;
        cnt = g.wsum_u(c2, kSiteCnt2);
        mn = kth;  // every kept value is >= kth; masked entries are -inf and carry no mass
    }
    write_logits();

    const float m = mx;
    const double u = row_uniform(a, r);

    if (cnt <= (uint32_t)kCandMax) {
        // ================= exact regime: the reference's sequential fp64 arithmetic =================
        auto& ex = sm.u.ex;
        if (cands) {
            // the top-k candidates, in index order (those below the k-th largest hold -inf)
        } else if constexpr (NC <= 4) {
            g.sync();
            // one scan for every sweep: 16-bit counts per sweep (at most kCandMax candidates)
            uint64_t mine = 0;
#pragma unroll
            for (int c = 0; c < NC; c++) {
                uint32_t m = 0;
#pragma unroll
                for (int j = 0; j < 4; j++) m += v[c * 4 + j] != kNegInf ? 1u : 0u;
                mine |= (uint64_t)m << (16 * c);
            }
            uint64_t total;
            const uint64_t excl = g.excl_scan(mine, kSiteComp0, total);
            uint32_t base = 0;
#pragma unroll
            for (int c = 0; c < NC; c++) {
                uint32_t off = base + (uint32_t)((excl >> (16 * c)) & 0xffffu);
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const int e = c * 4 + j;
                    if (v[e] != kNegInf) {
                        ex.cx[off] = v[e];
                        ex.ci[off] = eidx(e);
                        off++;
                    }
                }
                base += (uint32_t)((total >> (16 * c)) & 0xffffu);
            }
        } else {
            g.sync();
            uint32_t base = 0;
#pragma unroll
            for (int c = 0; c < NC; c++) {
                uint32_t mine = 0;
#pragma unroll
                for (int j = 0; j < 4; j++) mine += v[c * 4 + j] != kNegInf ? 1u : 0u;
                uint32_t total;
                uint32_t off = base + g.excl_scan(mine, kSiteComp0 + c, total);
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const int e = c * 4 + j;
                    if (v[e] != kNegInf) {
                        ex.cx[off] = v[e];
                        ex.ci[off] = eidx(e);
                        off++;
                    }
                }
                base += total;
            }
        }
        if (prow)
#pragma unroll
            for (int e = 0; e < NE; e++)
                if (eidx(e) < V && v[e] == kNegInf) prow[eidx(e)] = 0.0;
        g.sync();
        const int n = cands ? ncand : (int)cnt;
        if (cnt <= 64u) {
            // One wave takes the row; the other waves are done with it. The live candidates (the
            // top-k path also gathers entries below the k-th value, masked to -inf) are compacted
            // in index order into ex.cp's storage, one per lane.
            if (g.wv == 0) {
                float* cx = reinterpret_cast<float*>(ex.cp);
                int32_t* ci = reinterpret_cast<int32_t*>(ex.cp + 32);
                uint32_t base = 0;
                for (int q = 0; q < n; q += 64) {  // n uniform (a count every thread computed)
                    const int j = q + g.lane;
                    const float xj = j < n ? ex.cx[j] : kNegInf;
                    const bool live = xj != kNegInf;
                    const uint64_t bal = __ballot(live);
                    const uint32_t at = base + (uint32_t)__builtin_amdgcn_mbcnt_hi(
                                                   (uint32_t)(bal >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)bal, 0u));
                    if (live) {
                        cx[at] = xj;
                        ci[at] = ex.ci[j];
                    }
                    base += (uint32_t)__builtin_popcountll(bal);
                }
                wave_lds_sync();
                const int nl = (int)cnt;
                const float xl = g.lane < nl ? cx[g.lane] : 0.0f;
                const int pick = wave_exact(xl, ci, nl, m, topp, P.top_p, u, ex.ps, prow, g.lane);
                if (g.lane == 0) put_id(a, r, pick);
            }
            return;
        }
        // Parallel phases stride the candidates over the workgroup; sequential phases run
        // redundantly in every thread on LDS broadcast reads, so each yields a uniform value.
        for (int j = g.t; j < n; j += kT) ex.cp[j] = exp((double)(ex.cx[j] - m));  // Sampler.cs:57
        g.sync();
        double sum = seq_sum(ex.cp, n);  // sequential in index order                      :58
        g.sync();
        for (int j = g.t; j < n; j += kT) ex.cp[j] = ex.cp[j] / sum;  //                 :60
        g.sync();
        if (topp) {  //                                                                 :62-75
            // Stable ascending (p, index) order of the candidates (slot order == index order).
            // p = exp(d) / sum never decreases with d = fl32(x - m), so (d, index) order is the
            // (p, index) order whenever each adjacent pair is in (p, index) order; that is checked,
            // and the candidates are ranked by p directly otherwise.
            uint64_t* dkey = reinterpret_cast<uint64_t*>(ex.pre);
            for (int j = g.t; j < n; j += kT)
                dkey[j] = ((uint64_t)f2key(ex.cx[j] - m) << 32) | (uint32_t)j;
            g.sync();
            for (int j = g.t; j < n; j += kT) {
                const uint64_t kj = dkey[j];
                int rank = 0;
#pragma unroll 8
                for (int l = 0; l < n; l++) rank += dkey[l] < kj ? 1 : 0;
                ex.cs[rank] = (int16_t)j;
            }
            g.sync();
            bool ok = true;
            for (int q = g.t; q < n - 1; q += kT) {
                const int a0 = ex.cs[q], b0 = ex.cs[q + 1];
                const double pa = ex.cp[a0], pb = ex.cp[b0];
                ok = ok && (pa < pb || (pa == pb && a0 < b0));
            }
            if (g.any(!ok, kSiteTk0 + 2)) {
                for (int j = g.t; j < n; j += kT) ex.cs[seq_rank(ex.cp, n, j)] = (int16_t)j;
                g.sync();
            }
            const double thr = (double)(1.0f - P.top_p);
            // The largest (p, index) entry is the reference's last sorted position, which its
            // loop (j < n - 1) never visits; masked entries sort first with p = 0 and change
            // nothing. Wave 0 runs the cut on p gathered into sorted order; the removed prefix is
            // zeroed after a barrier.
            for (int q = g.t; q < n; q += kT) ex.ps[q] = ex.cp[ex.cs[q]];
            g.sync();
            if (g.wv == 0) {
                const int nr = wave_topp_cut(ex.ps, n, thr);
                if (g.lane == 0) ex.nrem = nr;
            }
            g.sync();
            const int nrem = ex.nrem;
            for (int s = g.t; s < nrem; s += kT) ex.cp[ex.cs[s]] = 0.0;
            g.sync();
            double s2 = seq_sum(ex.cp, n);  // probs.Sum(), sequential
            g.sync();
            for (int j = g.t; j < n; j += kT) ex.cp[j] = ex.cp[j] / s2;
            g.sync();
        }
        if (g.wv == 0) {  // inverse-CDF draw in index order                              :77-87
            const int pick = wave_draw(ex.cp, ex.ci, n, u);
            if (g.lane == 0) put_id(a, r, pick);
        }
        if (prow)
            for (int j = g.t; j < n; j += kT) prow[ex.ci[j]] = ex.cp[j];
        return;
    }

    // =========== nucleus regime: exact fixed-point masses, histogram-located top-p cut ===========
    // F fraction bits: vocab * 2^F <= 2^53 (exact double sums) and e * 2^F < 2^52.
    const int F = min(51, 53 - (32 - __clz(V - 1)));
    const double scaleF = __builtin_ldexp(1.0, F);
    const float Cb = mass_bias(F);
#pragma unroll
    for (int e = 0; e < NE; e++) v[e] = v[e] - m;  // d = x - max; -inf stays -inf
    // Masses and keys are recomputed where they are needed (a few VALU ops) instead of being kept
    // live; the empty asm stops the compiler from caching them in VGPRs.
    auto qof = [&](int e) -> double {
        float x = v[e];
        asm volatile("" : "+v"(x));
        return fixed_mass(nucleus_exp(x), Cb, scaleF);
    };
    auto keyof = [&](int e) -> uint32_t {
        float x = v[e];
        asm volatile("" : "+v"(x));
        return f2key(x);
    };
    float dc = kNegInf;  // cut: keep d > dc, or d == dc with index >= ic
    int ic = 0x7fffffff;
    auto kept = [&](int e) { return v[e] > dc || (v[e] == dc && eidx(e) >= ic); };
    double S = 0.0, Skept = 0.0;
    double kc[NC];  // kept mass per sweep (uniform)
    if (topp) {
        constexpr int NBP = C::NBP, BPT = NBP / kT;
        // buckets linear in d over [lo, 0]; lo is the row minimum, or -64 when lower
        const float lo = fmaxf(mn - m, -64.0f);
        const float scale = lo < -1e-30f ? (float)NBP / -lo : 0.0f;
        const float off = -lo * scale;
        auto bk = [&](int e) -> int {
            float x = v[e];
            asm volatile("" : "+v"(x));
            return (int)__builtin_amdgcn_fmed3f(__builtin_fmaf(x, scale, off), 0.0f, (float)(NBP - 1));
        };
#pragma unroll
        for (int e = 0; e < NE; e++)  // -inf entries add 0 to bucket 0
            atomicAdd(&sm.u.nh[e >> 2][bk(e)], fixed_mass(nucleus_exp(v[e]), Cb, scaleF));
        if (g.t == 0) {
            sm.ctl.bstar = -1;
            sm.ctl.list_n = 0;
        }
        g.sync();
        // Thread t owns buckets [t*BPT, (t+1)*BPT) of every sweep. One combined exclusive scan over
        // threads of (all sweeps, each sweep) gives the total S, the crossing bucket and, per sweep,
        // the mass of the buckets above it.
        double hs[NC + 1];
        hs[0] = 0.0;
#pragma unroll
        for (int c = 0; c < NC; c++) {
            double lt = 0.0;
#pragma unroll
            for (int j = 0; j < BPT; j++) lt += sm.u.nh[c][g.t * BPT + j];
            hs[c + 1] = lt;
            hs[0] += lt;
        }
        double incl[NC + 1];
#pragma unroll
        for (int i = 0; i <= NC; i++) {
            incl[i] = wave_incl_sum(hs[i]);
            if (g.lane == 0) g.slot[kSiteNScan0 + i][g.wv] = (uint64_t)__double_as_longlong(readlane_d(incl[i], 63));
        }
        g.sync();
        double exs[NC + 1], tts[NC + 1];
#pragma unroll
        for (int i = 0; i <= NC; i++) {
            double base = 0.0, tt = 0.0;
#pragma unroll
            for (int w = 0; w < kWaves; w++) {
                const double sv = __longlong_as_double((long long)g.slot[kSiteNScan0 + i][w]);
                base += w < g.wv ? sv : 0.0;
                tt += sv;
            }
            exs[i] = base + incl[i] - hs[i];
            tts[i] = tt;
        }
        S = tts[0];
        const double thr = (double)(1.0f - P.top_p);
        const double T = thr >= 1.0 ? 1e300 : floor(thr * S);
        if (exs[0] <= T && T - exs[0] < hs[0]) {  // this thread holds the crossing bucket
            double run = exs[0];
            double pre[NC];
#pragma unroll
            for (int c = 0; c < NC; c++) pre[c] = exs[c + 1];
#pragma unroll
            for (int j = 0; j < BPT; j++) {
                double hb = 0.0;
#pragma unroll
                for (int c = 0; c < NC; c++) hb += sm.u.nh[c][g.t * BPT + j];
                if (T - run < hb) {
                    sm.ctl.bstar = g.t * BPT + j;
                    sm.ctl.below = run;
#pragma unroll
                    for (int c = 0; c < NC; c++)  // sweep mass above the crossing bucket
                        sm.ctl.kept[c] = tts[c + 1] - (pre[c] + sm.u.nh[c][g.t * BPT + j]);
                    break;
                }
                run += hb;
#pragma unroll
                for (int c = 0; c < NC; c++) pre[c] += sm.u.nh[c][g.t * BPT + j];
            }
        }
        g.sync();
        const int bstar = sm.ctl.bstar;
        double cbelow = 0.0;
        bool fast = bstar >= 0;
        if (fast) {
            const double below = sm.ctl.below;
            // gather the crossing bucket
#pragma unroll
            for (int e = 0; e < NE; e++)
                if (v[e] != kNegInf && bk(e) == bstar) {
                    const uint32_t k = atomicAdd(&sm.ctl.list_n, 1u);
                    if (k < (uint32_t)kNLMax) {
                        sm.nl.key[k] = keyof(e);
                        sm.nl.idx[k] = eidx(e);
                        sm.nl.w[k] = qof(e);
                    }
                }
            g.sync();
            const int n = (int)sm.ctl.list_n;
            fast = n <= kNLMax;
            if (fast) {
                if (g.wv == 0) {
                    // rank by (key, index) in wave 0: lane l holds list entries l and l+64 in
                    // registers and compares them with every entry broadcast by readlane; lane l
                    // then owns ranks 2l and 2l+1
                    const int lane = g.lane;
                    const uint32_t ka0 = lane < n ? sm.nl.key[lane] : 0xffffffffu;
                    const int ia0 = lane < n ? sm.nl.idx[lane] : 0x7fffffff;
                    const uint32_t ka1 = lane + 64 < n ? sm.nl.key[lane + 64] : 0xffffffffu;
                    const int ia1 = lane + 64 < n ? sm.nl.idx[lane + 64] : 0x7fffffff;
                    int rk0 = 0, rk1 = 0;
                    const int n0 = min(n, 64);
                    for (int b = 0; b < n0; b++) {
                        const uint32_t kb = readlane(ka0, b);
                        const int ib = (int)readlane((uint32_t)ia0, b);
                        rk0 += (kb < ka0) || (kb == ka0 && ib < ia0);
                        rk1 += (kb < ka1) || (kb == ka1 && ib < ia1);
                    }
                    for (int b = 64; b < n; b++) {
                        const uint32_t kb = readlane(ka1, b - 64);
                        const int ib = (int)readlane((uint32_t)ia1, b - 64);
                        rk0 += (kb < ka0) || (kb == ka0 && ib < ia0);
                        rk1 += (kb < ka1) || (kb == ka1 && ib < ia1);
                    }
                    if (lane < n) {
                        sm.nl.ws[rk0] = sm.nl.w[lane];
                        sm.nl.at[rk0] = (int16_t)lane;
                    }
                    if (lane + 64 < n) {
                        sm.nl.ws[rk1] = sm.nl.w[lane + 64];
                        sm.nl.at[rk1] = (int16_t)(lane + 64);
                    }
                    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                    __builtin_amdgcn_wave_barrier();
                    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
                    const int r0 = 2 * lane;
                    const double w0 = r0 < n ? sm.nl.ws[r0] : 0.0;
                    const double w1 = r0 + 1 < n ? sm.nl.ws[r0 + 1] : 0.0;
                    const double c0 = below + wave_incl_sum(w0 + w1) - (w0 + w1);  // before rank r0
                    int prank = -1;
                    if (r0 < n && T >= c0 && T - c0 < w0) prank = r0;
                    else if (r0 + 1 < n && T >= c0 + w0 && T - (c0 + w0) < w1) prank = r0 + 1;
                    const uint64_t bal = __ballot(prank >= 0);
                    // the bucket holds the crossing, so exactly one rank qualifies
                    const int pl = bal ? (int)__builtin_ctzll(bal) : 0;
                    const double pbelow = readlane_d(prank == r0 ? c0 : c0 + w0, pl);
                    prank = bal ? (int)readlane((uint32_t)prank, pl) : n - 1;
                    // the crossing bucket's kept part (ranks >= prank) joins its sweeps' kept mass
                    if (r0 < n && r0 >= prank) atomicAdd(&sm.ctl.kept[sm.nl.idx[sm.nl.at[r0]] / kSW], w0);
                    if (r0 + 1 < n && r0 + 1 >= prank) atomicAdd(&sm.ctl.kept[sm.nl.idx[sm.nl.at[r0 + 1]] / kSW], w1);
                    if (lane == 0) {
                        const int at = sm.nl.at[prank];
                        sm.ctl.sel_key = sm.nl.key[at];
                        sm.ctl.sel_idx = sm.nl.idx[at];
                        sm.ctl.sel_cbelow = pbelow;
                    }
                }
                g.sync();
                dc = key2f(sm.ctl.sel_key);
                ic = sm.ctl.sel_idx;
                cbelow = sm.ctl.sel_cbelow;
#pragma unroll
                for (int c = 0; c < NC; c++) kc[c] = sm.ctl.kept[c];
            }
        }
        if (!fast) {
            // no crossing (top_p at or below 0), or a crowded crossing bucket: the general select
            // over the whole row, then the kept mass per sweep by a full pass
            for (int b = g.t; b < kNB; b += kT) sm.u.sel.hist[b] = 0.0;
            uint64_t act = 0;
#pragma unroll
            for (int e = 0; e < NE; e++)
                if (v[e] != kNegInf) act |= 1ull << e;
            const float sc2 = lo < -1e-30f ? (float)kNB / -lo : 0.0f;
            const float of2 = -lo * sc2;
            auto b1 = [&](int e) -> int {
                float x = v[e];
                asm volatile("" : "+v"(x));
                return (int)__builtin_amdgcn_fmed3f(__builtin_fmaf(x, sc2, of2), 0.0f, (float)(kNB - 1));
            };
            g.sync();
            uint32_t ck;
            block_select<NC>(g, sm, act, T, true, keyof, qof, b1, kSiteScanP, kSiteLRankP, ck, ic, cbelow);
            dc = key2f(ck);
#pragma unroll
            for (int c = 0; c < NC; c++) {
                double s2 = 0.0;
#pragma unroll
                for (int j = 0; j < 4; j++)
                    if (kept(c * 4 + j)) s2 += qof(c * 4 + j);
                const double w = wave_sum(s2);
                if (g.lane == 0) g.slot[kSiteChunk0 + c][g.wv] = (uint64_t)__double_as_longlong(w);
            }
            g.sync();
#pragma unroll
            for (int c = 0; c < NC; c++) {
                double s2 = 0.0;
#pragma unroll
                for (int w = 0; w < kWaves; w++) s2 += __longlong_as_double((long long)g.slot[kSiteChunk0 + c][w]);
                kc[c] = s2;
            }
        }
        Skept = S - cbelow;
    } else {
        // no top-p: every finite entry is kept; per-sweep totals from one pass
#pragma unroll
        for (int c = 0; c < NC; c++) {
            double s2 = 0.0;
#pragma unroll
            for (int j = 0; j < 4; j++) s2 += fixed_mass(nucleus_exp(v[c * 4 + j]), Cb, scaleF);
            const double w = wave_sum(s2);
            if (g.lane == 0) g.slot[kSiteChunk0 + c][g.wv] = (uint64_t)__double_as_longlong(w);
        }
        g.sync();
#pragma unroll
        for (int c = 0; c < NC; c++) {
            double s2 = 0.0;
#pragma unroll
            for (int w = 0; w < kWaves; w++) s2 += __longlong_as_double((long long)g.slot[kSiteChunk0 + c][w]);
            kc[c] = s2;
            S += s2;
        }
        Skept = S;
    }

    // ---- draw: first kept index (index order) whose inclusive prefix mass exceeds floor(u * Skept)
    const double D = floor(u * Skept);
    int cstar = -1;
    double run = 0.0;
#pragma unroll
    for (int c = 0; c < NC; c++)
        if (cstar < 0) {
            if (D >= run && D - run < kc[c]) cstar = c;
            else run += kc[c];
        }
    int pick = -1;
    if (cstar >= 0) {
        double w4[4];
#pragma unroll
        for (int j = 0; j < 4; j++) w4[j] = 0.0;
#pragma unroll
        for (int c = 0; c < NC; c++)
            if (c == cstar) {  // uniform: only the sweep holding the draw is revisited
#pragma unroll
                for (int j = 0; j < 4; j++)
                    if (kept(c * 4 + j)) w4[j] = qof(c * 4 + j);
            }
        const double mine = w4[0] + w4[1] + w4[2] + w4[3];
        if (g.t == 0) sm.ctl.found = -1;
        double total;
        const double excl = g.excl_scan(mine, kSiteDraw, total);
        if (D >= run + excl && D - (run + excl) < mine) {
            double acc = run + excl;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                acc += w4[j];
                if (w4[j] > 0.0 && D < acc) {
                    sm.ctl.found = cstar * kSW + g.t * 4 + j;
                    break;
                }
            }
        }
        g.sync();
        pick = sm.ctl.found;
    }
    if (pick < 0) {  // no crossing: the last kept id with p > 0 (exp underflows below -745.133)
        int li = -1;
#pragma unroll
        for (int e = 0; e < NE; e++)
            if (kept(e) && v[e] >= -745.1331787109375f) li = max(li, eidx(e));
        pick = g.imax(li, kSiteLast);
        if (pick < 0) pick = 0;
    }
    if (g.t == 0) put_id(a, r, pick);
    if (prow) {
        double se = 0.0;
#pragma unroll
        for (int e = 0; e < NE; e++)
            if (kept(e)) se += exp_neg_prob(v[e]);
        se = g.dsum(se, kSitePSum);
#pragma unroll
        for (int e = 0; e < NE; e++)
            if (eidx(e) < V) prow[eidx(e)] = kept(e) ? exp_neg_prob(v[e]) / se : 0.0;
    }
}

// The last workgroup of the grid publishes a.done_seq to the host (see SampleArgs::done_flag).
__device__ __forceinline__ void signal_done(const SampleArgs& a) {
    __threadfence_system();  // this thread's id store is visible to the host before the count
    __syncthreads();
    if (threadIdx.x == 0) {
        const int prev = gridDim.x == 1 ? 0 : atomicAdd(a.done_count, 1);  // one workgroup: no count
        if (prev == (int)gridDim.x - 1) {
            *a.done_count = 0;  // the next call (stream-ordered after this one) starts from zero
            __threadfence_system();
            __hip_atomic_store(a.done_flag, a.done_seq, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
        }
    }
}

template <int NC>
__global__ __launch_bounds__(kT) __attribute__((amdgpu_waves_per_eu(kWavesPerEu<NC>))) void sample_rows_kernel(
    SampleArgs a, int vec) {
    __shared__ RowSmem<NC> sm;
    row_block<NC>(a, vec, blockIdx.x, sm);
    if (a.done_flag) signal_done(a);
}

// Four rows per workgroup, one per wave, through the one-wave fast path (vxs_wave.h). The rows the
// fast path hands back (every sampled row with top-k, few candidates, crowded or degenerate cuts,
// requested outputs) are then sampled by the same workgroup with the general algorithm, one after
// the other, in the LDS the waves no longer need: no second kernel, so nothing to launch when no
// row is handed back, and a batch whose rows are all handed back runs one workgroup per four rows.
template <int NS, int NC>
union QuadSmem {
    WaveSmem<NS> wave[kWaves];
    RowSmem<NC> row;
};

template <int NS, int NC, bool kStats, bool kPrio>
__global__ __launch_bounds__(kT) __attribute__((amdgpu_waves_per_eu(4))) void sample_quad_kernel(SampleArgs a,
                                                                                                int vec) {
    __shared__ QuadSmem<NS, NC> sm;
    __shared__ int32_t back[kWaves];
    const int wv = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    const int r0 = blockIdx.x * kWaves;
    const int r = r0 + wv;
    // Staggered halves (launch_quad sets the split): when the whole grid is resident at once (at
    // most four workgroups per CU, one wave of each per SIMD), the second half of the workgroups
    // starts its loads after a delay proportional to the first half's bytes and issues them at a
    // lower wave priority, so the first half's rows arrive first and compute while the second half
    // loads; from then on every wave's priority follows its row's remaining work (kPrio).
    // Larger grids run in several rounds, which stagger by themselves, and take no delay.
    if (a.stagger_sleeps) {
        const bool late = (int)blockIdx.x >= a.stagger_from;
        if (!late) __builtin_amdgcn_s_setprio(3);
        for (int i = 0; late && i < a.stagger_sleeps; i++) __builtin_amdgcn_s_sleep(32);
    }
    int b = 0;
    if (r < a.rows) b = wave_fast_row<NS, kStats, kPrio>(a, vec, r, lane, sm.wave[wv]);
    if (lane == 0) back[wv] = b;
    __syncthreads();  // every wave is done with its LDS, and the flags are visible
    const int b0 = back[0], b1 = back[1], b2 = back[2], b3 = back[3];  // workgroup-uniform
    static_assert(kWaves == 4, "four rows per workgroup");
    if constexpr (kPrio)
        if (b0 | b1 | b2 | b3) __builtin_amdgcn_s_setprio(3);  // the slowest rows: all four waves alike
    if (b0) row_block<NC>(a, vec, r0, sm.row);
    if (b0 && (b1 | b2 | b3)) __syncthreads();  // LDS is reused by the next row
    if (b1) row_block<NC>(a, vec, r0 + 1, sm.row);
    if (b1 && (b2 | b3)) __syncthreads();
    if (b2) row_block<NC>(a, vec, r0 + 2, sm.row);
    if (b2 && b3) __syncthreads();
    if (b3) row_block<NC>(a, vec, r0 + 3, sm.row);
}

template <int NC>
hipError_t launch_nc(const SampleArgs& a, int vec, hipStream_t stream) {
    hipLaunchKernelGGL((sample_rows_kernel<NC>), dim3(a.rows), dim3(kT), 0, stream, a, vec);
    return hipGetLastError();
}

// Compute units of the current device (cached per device; calls from several threads may each
// query it once, and store the same value).
int device_cus() {
    static std::atomic<int> cus[64] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    int n = cus[dev].load(std::memory_order_relaxed);
    if (!n) {
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
        cus[dev].store(n, std::memory_order_relaxed);
    }
    return n;
}

template <int NS, int NC>
hipError_t launch_quad(const SampleArgs& a_in, int vec, hipStream_t stream) {
    SampleArgs a = a_in;
    const dim3 grid((a.rows + kWaves - 1) / kWaves);
    // The stagger of sample_quad_kernel: a grid resident in one round with three or four
    // workgroups per CU delays its second half by about 2.6 us per full round of 4 x CUs
    // workgroups (3 x 2048 cycles of s_sleep at 4096 rows on 256 CUs). Measured, 3072-entry
    // rows, staggered / not: 2049 rows (none) 15.6 us, 3072 rows 18.27 / 18.52, 4096 rows 21.04 /
    // 21.60; 6144 and 8192 rows run in two rounds and take none.
    const int g = (int)grid.x, cus = device_cus();
    a.stagger_from = g;
    a.stagger_sleeps = 0;
    // Priority by remaining work (the kPrio instance) for a grid resident in one round with more
    // than one workgroup per CU (measured, 3072-entry rows, with / without: 2048 rows 14.8 / 15.2
    // us, 3072 rows 17.3 / 18.0, 4096 rows 19.7 / 20.7); a grid of several rounds is faster with
    // the oldest waves first (6144 rows 31.8 / 28.6 us), as they free the slots the next
    // workgroups wait for.
    const bool prio = g > cus && g <= 4 * cus;
    if (g <= 4 * cus && g >= 3 * cus) {
        a.stagger_from = g / 2;
        a.stagger_sleeps = (3 * g + 2 * cus) / (4 * cus);
    }
    if (a.out_stats)  // a separate instance, so the statistics cost the sampling kernel nothing
        hipLaunchKernelGGL((sample_quad_kernel<NS, NC, true, false>), grid, dim3(kT), 0, stream, a, vec);
    else if (prio)
        hipLaunchKernelGGL((sample_quad_kernel<NS, NC, false, true>), grid, dim3(kT), 0, stream, a, vec);
    else
        hipLaunchKernelGGL((sample_quad_kernel<NS, NC, false, false>), grid, dim3(kT), 0, stream, a, vec);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_sample(const SampleArgs& a, hipStream_t stream) {
    if (a.rows <= 0) return hipSuccess;
    if (a.vocab > kRowResidentMaxVocab) return launch_sample_wide(a, stream);
    if (a.vocab <= 0) return hipErrorNotSupported;
    const int vec = (a.ld % 4 == 0) && (((uintptr_t)a.logits & 15u) == 0) ? 1 : 0;
    const int V = a.vocab;
    if (a.path == kPathQuad && V <= kWaveMaxVocab) {
        if (V <= 1024) return launch_quad<4, 1>(a, vec, stream);
        if (V <= 2048) return launch_quad<8, 2>(a, vec, stream);
        return launch_quad<12, 3>(a, vec, stream);
    }
    if (V <= 1024) return launch_nc<1>(a, vec, stream);
    if (V <= 2048) return launch_nc<2>(a, vec, stream);
    if (V <= 3072) return launch_nc<3>(a, vec, stream);
    if (V <= 4096) return launch_nc<4>(a, vec, stream);
    if (V <= 6144) return launch_nc<6>(a, vec, stream);
    return launch_nc<8>(a, vec, stream);
}

}  // namespace vxs
