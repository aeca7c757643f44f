// vxs_kernels.hip — gfx950 kernels of the token sampler.
//
// Row-resident kernel: one 256-thread workgroup (4 wave64) owns one row of up to 8192 logits.
// The row is read from HBM once, with 16-byte non-temporal loads in sweeps of 1024 elements
// (thread t holds elements c*1024 + 4t + j), and stays in VGPRs for every step:
//
//   S1 penalty     distinct history ids via an LDS bitmap (atomicOr picks one owner per id);
//                  the owner rescales the logit (true fp32 divide / multiply)  Sampler.cs:25-33
//   S2 suppression [supp_begin, supp_end) except keep_id, then ban_id -> -inf TalkerGenerator.cs:247-248
//   S3 greedy      first index of the max, no temperature                    Sampler.cs:37,90-95
//   S4 temperature x * fl32(1/T)                                             Sampler.cs:39-40
//   S5 top-k       k-th largest (ties kept) by a count-weighted bucket select Sampler.cs:42-49
//   S6-S8          two regimes after top-k:
//     exact        <= 256 candidates: candidates are compacted in index order and wave 0 runs the
//                  reference's sequential fp64 arithmetic on them (softmax sum, stable (p, index)
//                  order, cumulative top-p cut, renormalisation, index-order draw)  Sampler.cs:51-87
//     parallel     more candidates (full-vocab nucleus): masses exp(x-m) as 2^-F fixed point
//                  (exact, order-independent integer sums), top-p cut by a mass-weighted bucket
//                  select over (d = x-m, index), draw by an index-order integer prefix search.
//
// Bucket select: level 1 spreads elements linearly over the value range (1024 LDS buckets),
// refinement levels split the surviving key interval in the order-preserving u32 key space, and
// the last <= 512 elements are ranked exactly. It finds the first element, in ascending
// (key, index) order, at which the cumulative weight exceeds a target.
//
// Per-row errors are reported in out_ids[row] as negative VXS_ERR_* codes.
#include <math.h>
#include <stdint.h>

#include "vxs_internal.h"

namespace vxs {
namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int kSweep = kThreads * 4;  // elements per float4 sweep of the workgroup
constexpr int kBuckets = 1024;
constexpr int kBucketsLog2 = 10;
constexpr int kList = 512;     // elements ranked exactly at the end of a bucket select
constexpr int kCandMax = 256;  // candidate count of the exact sequential regime
constexpr float kNegInf = -__builtin_huge_valf();
constexpr float kPosInf = __builtin_huge_valf();

typedef float f4 __attribute__((ext_vector_type(4)));

// ---- keys ------------------------------------------------------------------------------------
// Order-preserving u32 image of a float; -0 maps to +0 because C# compares them equal.
__device__ __forceinline__ uint32_t f2key(float f) {
    if (f == 0.0f) f = 0.0f;
    const uint32_t u = __float_as_uint(f);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float key2f(uint32_t k) {
    const uint32_t u = (k & 0x80000000u) ? (k & 0x7fffffffu) : ~k;
    return __uint_as_float(u);
}

// Round-to-nearest integer of e * 2^F for 0 <= e*2^F < 2^52, via the 2^52 magic constant.
__device__ __forceinline__ uint64_t fixed_point(double e, double scale) {
    const double t = __builtin_fma(e, scale, 4503599627370496.0);
    return (uint64_t)__double_as_longlong(t) - 0x4330000000000000ull;
}

// ---- wave / workgroup primitives ----------------------------------------------------------
template <typename T>
__device__ __forceinline__ T wave_sum(T v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}
__device__ __forceinline__ float wave_min(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fminf(v, __shfl_xor(v, o, 64));
    return v;
}
__device__ __forceinline__ uint32_t wave_umin(uint32_t v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = min(v, (uint32_t)__shfl_xor((int)v, o, 64));
    return v;
}
__device__ __forceinline__ uint32_t wave_umax(uint32_t v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = max(v, (uint32_t)__shfl_xor((int)v, o, 64));
    return v;
}
__device__ __forceinline__ int wave_imax(int v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = max(v, __shfl_xor(v, o, 64));
    return v;
}

// Workgroup-wide scratch for reductions and control values.
struct Ctl {
    uint64_t r64[kWaves * 8];
    double rd[kWaves];
    float rf[kWaves * 2];
    uint32_t ru[kWaves * 4];
    int32_t ri[kWaves * 2];
    int32_t err;
    int32_t sel_b;
    int32_t sel_idx;
    uint32_t sel_key;
    uint64_t sel_below;
    int32_t found_idx;
    uint32_t list_n;
};

template <typename T>
__device__ __forceinline__ T block_sum(T v, T* scratch) {
    v = wave_sum(v);
    if ((threadIdx.x & 63) == 0) scratch[threadIdx.x >> 6] = v;
    __syncthreads();
    T r = scratch[0];
#pragma unroll
    for (int i = 1; i < kWaves; i++) r += scratch[i];
    __syncthreads();
    return r;
}

template <int N>
__device__ __forceinline__ void block_sum_vec(uint64_t (&v)[N], uint64_t* scratch) {
    static_assert(N <= 8, "scratch holds 8 values per wave");
#pragma unroll
    for (int c = 0; c < N; c++) v[c] = wave_sum(v[c]);
    if ((threadIdx.x & 63) == 0)
#pragma unroll
        for (int c = 0; c < N; c++) scratch[(threadIdx.x >> 6) * 8 + c] = v[c];
    __syncthreads();
#pragma unroll
    for (int c = 0; c < N; c++) {
        uint64_t r = 0;
#pragma unroll
        for (int i = 0; i < kWaves; i++) r += scratch[i * 8 + c];
        v[c] = r;
    }
    __syncthreads();
}

__device__ __forceinline__ uint32_t block_umin(uint32_t v, uint32_t* scratch) {
    v = wave_umin(v);
    if ((threadIdx.x & 63) == 0) scratch[threadIdx.x >> 6] = v;
    __syncthreads();
    uint32_t r = scratch[0];
#pragma unroll
    for (int i = 1; i < kWaves; i++) r = min(r, scratch[i]);
    __syncthreads();
    return r;
}
__device__ __forceinline__ uint32_t block_umax(uint32_t v, uint32_t* scratch) {
    v = wave_umax(v);
    if ((threadIdx.x & 63) == 0) scratch[threadIdx.x >> 6] = v;
    __syncthreads();
    uint32_t r = scratch[0];
#pragma unroll
    for (int i = 1; i < kWaves; i++) r = max(r, scratch[i]);
    __syncthreads();
    return r;
}
__device__ __forceinline__ int block_imax(int v, int32_t* scratch) {
    v = wave_imax(v);
    if ((threadIdx.x & 63) == 0) scratch[threadIdx.x >> 6] = v;
    __syncthreads();
    int r = scratch[0];
#pragma unroll
    for (int i = 1; i < kWaves; i++) r = max(r, scratch[i]);
    __syncthreads();
    return r;
}

// Exclusive prefix sum over the workgroup in thread order; `total` gets the full sum.
template <typename T>
__device__ __forceinline__ T block_excl_scan(T v, T* scratch, T& total) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    T x = v;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const T y = __shfl_up(x, o, 64);
        if (lane >= o) x += y;
    }
    if (lane == 63) scratch[w] = x;
    __syncthreads();
    T base = 0;
    total = 0;
#pragma unroll
    for (int i = 0; i < kWaves; i++) {
        const T s = scratch[i];
        if (i < w) base += s;
        total += s;
    }
    __syncthreads();
    return base + x - v;
}

// ---- shared memory -------------------------------------------------------------------------
template <int NC>
struct SmemPenalty {
    uint32_t bm[NC * kSweep / 32];
    float pen[NC * kSweep];
};
struct SmemSelect {
    uint64_t hist[kBuckets];
    uint32_t lkey[kList];
    int32_t lidx[kList];
    uint64_t lw[kList];
    int16_t lsorted[kList];
};
struct SmemExact {
    float cx[kCandMax];
    int32_t ci[kCandMax];
    double cp[kCandMax];
    int32_t csorted[kCandMax];
};
template <int NC>
union Smem {
    SmemPenalty<NC> pen;
    SmemSelect sel;
    SmemExact ex;
};

// Element index of register slot e = c*4 + j.
__device__ __forceinline__ int elem_index(int e) { return (e >> 2) * kSweep + (int)threadIdx.x * 4 + (e & 3); }

// Finds the first element, in ascending (key, index) order over the elements whose bit is set in
// `active`, at which the inclusive cumulative weight exceeds T. Returns its key and index (index
// only when need_idx). When the total weight is <= T the result is the last active element.
// `b1(e)` is the level-1 bucket of slot e: monotone non-decreasing in key, in [0, kBuckets).
template <int NC, class B1>
__device__ void weighted_select(const uint32_t (&key)[NC * 4], const uint64_t (&w)[NC * 4], uint32_t active,
                                uint64_t T, bool need_idx, B1 b1, SmemSelect& s, Ctl& ctl, uint32_t& out_key,
                                int& out_idx) {
    constexpr int NE = NC * 4;
    const int tid = threadIdx.x;

    // ---- level 1: linear buckets over the value range
    for (int b = tid; b < kBuckets; b += kThreads) s.hist[b] = 0;
    if (tid == 0) ctl.sel_b = -1;
    __syncthreads();
#pragma unroll
    for (int e = 0; e < NE; e++)
        if ((active >> e) & 1u) atomicAdd((unsigned long long*)&s.hist[b1(e)], (unsigned long long)w[e]);
    __syncthreads();
    uint64_t below;
    {
        uint64_t h[4];
#pragma unroll
        for (int j = 0; j < 4; j++) h[j] = s.hist[tid * 4 + j];
        const uint64_t tot = h[0] + h[1] + h[2] + h[3];
        uint64_t all;
        const uint64_t excl = block_excl_scan(tot, ctl.r64, all);
        if (excl <= T && T - excl < tot) {
            uint64_t run = excl;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                if (T - run < h[j]) {
                    ctl.sel_b = tid * 4 + j;
                    ctl.sel_below = run;
                    break;
                }
                run += h[j];
            }
        }
        __syncthreads();
        if (ctl.sel_b < 0) {  // total weight <= T: the last active element
            uint32_t kmax = 0;
#pragma unroll
            for (int e = 0; e < NE; e++)
                if ((active >> e) & 1u) kmax = max(kmax, key[e]);
            kmax = block_umax(kmax, ctl.ru);
            int imax = -1;
#pragma unroll
            for (int e = 0; e < NE; e++)
                if (((active >> e) & 1u) && key[e] == kmax) imax = max(imax, elem_index(e));
            imax = block_imax(imax, ctl.ri);
            out_key = kmax;
            out_idx = imax;
            return;
        }
        below = ctl.sel_below;
    }
    const int bstar = ctl.sel_b;
    // active elements of the chosen bucket
    uint32_t in = 0;
#pragma unroll
    for (int e = 0; e < NE; e++)
        if (((active >> e) & 1u) && b1(e) == bstar) in |= 1u << e;

    uint32_t klo, khi, L;
    {
        uint32_t mn = 0xffffffffu, mx = 0;
#pragma unroll
        for (int e = 0; e < NE; e++)
            if ((in >> e) & 1u) {
                mn = min(mn, key[e]);
                mx = max(mx, key[e]);
            }
        klo = block_umin(mn, ctl.ru);
        khi = block_umax(mx, ctl.ru + kWaves);
        L = block_sum((uint32_t)__builtin_popcount(in), ctl.ru + 2 * kWaves);
    }

    // ---- refinement in key space until few elements or a single key remain
    while (L > (uint32_t)kList && klo != khi) {
        const uint32_t range = khi - klo;
        const int bits = 32 - __clz(range);
        const int shift = bits > kBucketsLog2 ? bits - kBucketsLog2 : 0;
        for (int b = tid; b < kBuckets; b += kThreads) s.hist[b] = 0;
        if (tid == 0) ctl.sel_b = -1;
        __syncthreads();
#pragma unroll
        for (int e = 0; e < NE; e++)
            if ((in >> e) & 1u) atomicAdd((unsigned long long*)&s.hist[(key[e] - klo) >> shift], (unsigned long long)w[e]);
        __syncthreads();
        const uint64_t T2 = T - below;
        uint64_t h[4];
#pragma unroll
        for (int j = 0; j < 4; j++) h[j] = s.hist[tid * 4 + j];
        const uint64_t tot = h[0] + h[1] + h[2] + h[3];
        uint64_t all;
        const uint64_t excl = block_excl_scan(tot, ctl.r64, all);
        if (excl <= T2 && T2 - excl < tot) {
            uint64_t run = excl;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                if (T2 - run < h[j]) {
                    ctl.sel_b = tid * 4 + j;
                    ctl.sel_below = run;
                    break;
                }
                run += h[j];
            }
        }
        __syncthreads();
        const int b2 = ctl.sel_b;  // always found: the interval holds the crossing element
        below += ctl.sel_below;
        const uint64_t lo2 = (uint64_t)klo + ((uint64_t)b2 << shift);
        const uint64_t hi2 = min((uint64_t)khi, lo2 + ((1ull << shift) - 1));
        uint32_t in2 = 0, mn = 0xffffffffu, mx = 0;
#pragma unroll
        for (int e = 0; e < NE; e++)
            if (((in >> e) & 1u) && key[e] >= lo2 && key[e] <= hi2) {
                in2 |= 1u << e;
                mn = min(mn, key[e]);
                mx = max(mx, key[e]);
            }
        in = in2;
        klo = block_umin(mn, ctl.ru);
        khi = block_umax(mx, ctl.ru + kWaves);
        L = block_sum((uint32_t)__builtin_popcount(in), ctl.ru + 2 * kWaves);
    }

    if (klo == khi) {  // a single key remains: ties, ordered by index
        out_key = klo;
        out_idx = -1;
        if (!need_idx) return;
        // every tied element has the same (non-zero) weight: take it from any holder
        uint64_t mine = 0;
#pragma unroll
        for (int e = 0; e < NE; e++)
            if ((in >> e) & 1u) mine = w[e];
        const uint32_t whi = block_umax((uint32_t)(mine >> 32), ctl.ru);
        const uint32_t wlo = block_umax((uint32_t)mine, ctl.ru + kWaves);
        const uint64_t wt = ((uint64_t)whi << 32) | wlo;
        const uint64_t nth = (T - below) / wt;  // 0-based position among the ties, index order
        // locate the nth tied element in index order, sweep by sweep
        uint64_t base = 0;
        if (tid == 0) ctl.found_idx = -1;
#pragma unroll
        for (int c = 0; c < NC; c++) {
            const uint32_t mine = (in >> (c * 4)) & 0xfu;
            const uint64_t cnt = (uint64_t)__builtin_popcount(mine);
            uint64_t total;
            const uint64_t excl = block_excl_scan(cnt, ctl.r64, total);
            if (nth >= base + excl && nth < base + excl + cnt) {
                uint64_t k = nth - base - excl;
#pragma unroll
                for (int j = 0; j < 4; j++)
                    if ((mine >> j) & 1u) {
                        if (k == 0) {
                            ctl.found_idx = c * kSweep + tid * 4 + j;
                            break;
                        }
                        k--;
                    }
            }
            base += total;
        }
        __syncthreads();
        out_idx = ctl.found_idx;
        return;
    }

    // ---- at most kList elements remain: rank them exactly by (key, index)
    if (tid == 0) ctl.list_n = 0;
    __syncthreads();
#pragma unroll
    for (int e = 0; e < NE; e++)
        if ((in >> e) & 1u) {
            const uint32_t slot = atomicAdd(&ctl.list_n, 1u);
            s.lkey[slot] = key[e];
            s.lidx[slot] = elem_index(e);
            s.lw[slot] = w[e];
        }
    __syncthreads();
    const int n = (int)ctl.list_n;
    for (int a = tid; a < n; a += kThreads) {
        const uint32_t ka = s.lkey[a];
        const int ia = s.lidx[a];
        int rank = 0;
        for (int b = 0; b < n; b++) {
            const uint32_t kb = s.lkey[b];
            rank += (kb < ka) || (kb == ka && s.lidx[b] < ia);
        }
        s.lsorted[rank] = (int16_t)a;
    }
    __syncthreads();
    if (tid == 0) {
        uint64_t cum = below;
        int pick = s.lsorted[n - 1];
        for (int r = 0; r < n; r++) {
            const int a = s.lsorted[r];
            cum += s.lw[a];
            if (cum > T) {
                pick = a;
                break;
            }
        }
        ctl.sel_key = s.lkey[pick];
        ctl.sel_idx = s.lidx[pick];
    }
    __syncthreads();
    out_key = ctl.sel_key;
    out_idx = ctl.sel_idx;
    __syncthreads();
}

// ---- the row-resident kernel ----------------------------------------------------------------
template <int NC, bool VEC>
__global__ __launch_bounds__(kThreads) void sample_rows_kernel(SampleArgs a) {
    constexpr int NE = NC * 4;
    __shared__ Smem<NC> sm;
    __shared__ Ctl ctl;

    const int tid = threadIdx.x;
    const int r = blockIdx.x;
    const int V = a.vocab;
    const vxs_params P = a.params[(int64_t)r * a.params_stride];
    const float* __restrict__ xrow = a.logits + (int64_t)r * a.ld;

    float v[NE];
#pragma unroll
    for (int c = 0; c < NC; c++) {
        const int i0 = c * kSweep + tid * 4;
        if (VEC) {
            if (i0 < V) {
                const f4 q = __builtin_nontemporal_load((const f4*)(xrow + i0));
                v[c * 4 + 0] = q.x;
                v[c * 4 + 1] = q.y;
                v[c * 4 + 2] = q.z;
                v[c * 4 + 3] = q.w;
            } else {
#pragma unroll
                for (int j = 0; j < 4; j++) v[c * 4 + j] = kNegInf;
            }
        } else {
#pragma unroll
            for (int j = 0; j < 4; j++) v[c * 4 + j] = (i0 + j < V) ? xrow[i0 + j] : kNegInf;
        }
    }
    uint32_t valid = 0;
#pragma unroll
    for (int e = 0; e < NE; e++)
        if (elem_index(e) < V) valid |= 1u << e;

    // ---- S1: repetition penalty over the distinct history ids
    if (P.rep_penalty != 1.0f && a.hist_off != nullptr) {
        const int h0 = a.hist_off[r], h1 = a.hist_off[r + 1];
        if (h1 > h0) {
            uint32_t* bm = sm.pen.bm;
            float* pen = sm.pen.pen;
            for (int w = tid; w < NC * kSweep / 32; w += kThreads) bm[w] = 0;
            if (tid == 0) ctl.err = 0;
            __syncthreads();
            const float rho = P.rep_penalty;
            for (int h = h0 + tid; h < h1; h += kThreads) {
                const int id = a.hist_ids[h];
                if ((unsigned)id >= (unsigned)V) {
                    ctl.err = VXS_ERR_ID_OUT_OF_RANGE;
                    continue;
                }
                const uint32_t bit = 1u << (id & 31);
                const uint32_t old = atomicOr(&bm[id >> 5], bit);
                if (!(old & bit)) {
                    const float sv = xrow[id];
                    pen[id] = sv < 0.0f ? sv * rho : sv / rho;
                }
            }
            __syncthreads();
            if (ctl.err != 0) {
                if (tid == 0) a.out_ids[r] = ctl.err;
                return;
            }
#pragma unroll
            for (int e = 0; e < NE; e++) {
                const int i = elem_index(e);
                if (((valid >> e) & 1u) && ((bm[i >> 5] >> (i & 31)) & 1u)) v[e] = pen[i];
            }
            __syncthreads();
        }
    }

    float* orow = a.out_logits ? a.out_logits + (int64_t)r * V : nullptr;
    double* prow = a.out_probs ? a.out_probs + (int64_t)r * V : nullptr;
    auto write_logits = [&]() {
        if (!orow) return;
#pragma unroll
        for (int e = 0; e < NE; e++)
            if ((valid >> e) & 1u) orow[elem_index(e)] = v[e];
    };

    if (a.kflags & KF_STOP_AFTER_PENALTY) {
        write_logits();
        if (tid == 0) a.out_ids[r] = 0;
        return;
    }

    // ---- S2: suppression
    {
        const int sb = max(P.supp_begin, 0), se = min(P.supp_end, V);
#pragma unroll
        for (int e = 0; e < NE; e++) {
            const int i = elem_index(e);
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
            if (!((valid >> e) & 1u)) continue;
            const int i = elem_index(e);
            nan |= v[e] != v[e];
            if (v[e] > bv || (v[e] == bv && i < bi)) {
                bv = v[e];
                bi = i;
            }
        }
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) {
            const float ov = __shfl_xor(bv, o, 64);
            const int oi = __shfl_xor(bi, o, 64);
            if (ov > bv || (ov == bv && oi < bi)) {
                bv = ov;
                bi = oi;
            }
        }
        const int lane = tid & 63, wid = tid >> 6;
        if (lane == 0) {
            ctl.rf[wid] = bv;
            ctl.ri[wid] = bi;
        }
        const int anynan = block_sum((uint32_t)nan, ctl.ru + 3 * kWaves);
        if (tid == 0) {
            float gv = ctl.rf[0];
            int gi = ctl.ri[0];
            for (int i = 1; i < kWaves; i++)
                if (ctl.rf[i] > gv || (ctl.rf[i] == gv && ctl.ri[i] < gi)) {
                    gv = ctl.rf[i];
                    gi = ctl.ri[i];
                }
            a.out_ids[r] = anynan ? VXS_ERR_NONFINITE : gi;
        }
        write_logits();
        if (prow)
#pragma unroll
            for (int e = 0; e < NE; e++)
                if ((valid >> e) & 1u) prow[elem_index(e)] = 0.0;
        return;
    }

    // ---- S4: temperature, and the finite-input contract
    const float invT = 1.0f / P.temperature;
    bool bad = false;
#pragma unroll
    for (int e = 0; e < NE; e++)
        if ((valid >> e) & 1u) {
            v[e] *= invT;
            bad |= (v[e] != v[e]) || v[e] == kPosInf;
        }
    float mx = kNegInf, mn = kPosInf;
    uint32_t cnt = 0;
#pragma unroll
    for (int e = 0; e < NE; e++)
        if (((valid >> e) & 1u) && v[e] != kNegInf) {
            mx = fmaxf(mx, v[e]);
            mn = fminf(mn, v[e]);
            cnt++;
        }
    {
        mx = wave_max(mx);
        mn = wave_min(mn);
        cnt = wave_sum(cnt);
        uint32_t b = wave_sum((uint32_t)bad);
        const int lane = tid & 63, wid = tid >> 6;
        if (lane == 0) {
            ctl.rf[wid] = mx;
            ctl.rf[kWaves + wid] = mn;
            ctl.ru[wid] = cnt;
            ctl.ru[kWaves + wid] = b;
        }
        __syncthreads();
        mx = ctl.rf[0];
        mn = ctl.rf[kWaves];
        cnt = ctl.ru[0];
        b = ctl.ru[kWaves];
        for (int i = 1; i < kWaves; i++) {
            mx = fmaxf(mx, ctl.rf[i]);
            mn = fminf(mn, ctl.rf[kWaves + i]);
            cnt += ctl.ru[i];
            b += ctl.ru[kWaves + i];
        }
        __syncthreads();
        if (b) {
            if (tid == 0) a.out_ids[r] = VXS_ERR_NONFINITE;
            return;
        }
    }

    // every entry is -inf: p = 0/0 everywhere and the reference's draw returns the last id
    if (cnt == 0) {
        if (tid == 0) a.out_ids[r] = V - 1;
        write_logits();
        if (prow)
#pragma unroll
            for (int e = 0; e < NE; e++)
                if ((valid >> e) & 1u) prow[elem_index(e)] = __builtin_nan("");
        return;
    }

    // ---- S5: top-k (ties at the k-th value are kept)
    uint32_t key[NE];
    uint64_t wgt[NE];
    const int K = P.top_k;
    if (K > 0 && K < V && (uint32_t)K < cnt) {
        uint32_t act = 0;
#pragma unroll
        for (int e = 0; e < NE; e++) {
            key[e] = f2key(v[e]);
            wgt[e] = 1;
            if (((valid >> e) & 1u) && v[e] != kNegInf) act |= 1u << e;
        }
        const double lo = (double)mn;
        const double scale = mx > mn ? (double)kBuckets / ((double)mx - lo) : 0.0;
        auto b1 = [&](int e) -> int {
            const int b = (int)(((double)v[e] - lo) * scale);
            return min(max(b, 0), kBuckets - 1);
        };
        uint32_t kkey;
        int kidx;
        weighted_select<NC>(key, wgt, act, (uint64_t)(cnt - (uint32_t)K), false, b1, sm.sel, ctl, kkey, kidx);
        const float kth = key2f(kkey);
        uint32_t c2 = 0;
        float mn2 = kPosInf;
#pragma unroll
        for (int e = 0; e < NE; e++)
            if ((valid >> e) & 1u) {
                if (v[e] < kth) v[e] = kNegInf;
                if (v[e] != kNegInf) {
                    c2++;
                    mn2 = fminf(mn2, v[e]);
                }
            }
        cnt = block_sum(c2, ctl.ru);
        mn = kth;  // the smallest kept value
    }
    write_logits();

    const float m = mx;
    const double u = a.u ? a.u[r] : 0.0;

    if (cnt <= (uint32_t)kCandMax) {
        // ================= exact regime: the reference's sequential fp64 arithmetic =================
        SmemExact& ex = sm.ex;
        // compact candidates in index order
        uint32_t base = 0;
#pragma unroll
        for (int c = 0; c < NC; c++) {
            uint32_t mine = 0;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int e = c * 4 + j;
                if (((valid >> e) & 1u) && v[e] != kNegInf) mine++;
            }
            uint32_t total;
            uint32_t off = base + block_excl_scan(mine, ctl.ru, total);
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int e = c * 4 + j;
                if (((valid >> e) & 1u) && v[e] != kNegInf) {
                    ex.cx[off] = v[e];
                    ex.ci[off] = elem_index(e);
                    off++;
                }
            }
            base += total;
        }
        if (prow)
#pragma unroll
            for (int e = 0; e < NE; e++)
                if (((valid >> e) & 1u) && v[e] == kNegInf) prow[elem_index(e)] = 0.0;
        __syncthreads();
        // Parallel phases stride the candidates over the workgroup; sequential phases are run
        // redundantly by every thread on LDS broadcast reads, so each yields a uniform value.
        const int n = (int)cnt;
        // e_i = exp((double)fl32(x_i - max))                                  Sampler.cs:57
        for (int j = tid; j < n; j += kThreads) ex.cp[j] = exp((double)(ex.cx[j] - m));
        __syncthreads();
        double sum = 0.0;  // sequential in index order                                 :58
        for (int j = 0; j < n; j++) sum += ex.cp[j];
        __syncthreads();
        for (int j = tid; j < n; j += kThreads) ex.cp[j] = ex.cp[j] / sum;  //          :60
        __syncthreads();
        if (P.top_p < 1.0f) {  //                                                      :62-75
            // stable ascending (p, index) order of the candidates (index order == slot order)
            for (int j = tid; j < n; j += kThreads) {
                const double pj = ex.cp[j];
                int rank = 0;
                for (int l = 0; l < n; l++) {
                    const double pl = ex.cp[l];
                    rank += (pl < pj) || (pl == pj && l < j);
                }
                ex.csorted[rank] = j;
            }
            __syncthreads();
            const double thr = (double)(1.0f - P.top_p);
            double cum = 0.0;
            // The largest (p, index) entry is the reference's last sorted position, which its
            // loop (j < n - 1) never visits; masked entries sort first with p = 0 and change
            // nothing. The scan only reads; the removed prefix is zeroed after a barrier.
            int nrem = n - 1;
            for (int s = 0; s < n - 1; s++) {
                cum += ex.cp[ex.csorted[s]];
                if (!(cum <= thr)) {
                    nrem = s;
                    break;
                }
            }
            __syncthreads();
            for (int s = tid; s < nrem; s += kThreads) ex.cp[ex.csorted[s]] = 0.0;
            __syncthreads();
            double s2 = 0.0;  // probs.Sum(), sequential
            for (int j = 0; j < n; j++) s2 += ex.cp[j];
            __syncthreads();
            for (int j = tid; j < n; j += kThreads) ex.cp[j] = ex.cp[j] / s2;
            __syncthreads();
        }
        // inverse-CDF draw in index order                                              :77-87
        double acc = 0.0;
        int last = 0, pick = -1;
        for (int j = 0; j < n; j++) {
            const double pj = ex.cp[j];
            if (pj <= 0.0) continue;
            acc += pj;
            last = ex.ci[j];
            if (u < acc) {
                pick = last;
                break;
            }
        }
        if (tid == 0) a.out_ids[r] = pick >= 0 ? pick : last;
        if (prow)
            for (int j = tid; j < n; j += kThreads) prow[ex.ci[j]] = ex.cp[j];
        return;
    }

    // ================= parallel regime: fixed-point masses, bucket-selected nucleus =================
    // F fraction bits so that vocab * 2^F < 2^62 and e * 2^F < 2^52.
    const int F = min(51, 62 - (32 - __clz(V - 1)));
    const double scaleF = __builtin_ldexp(1.0, F);
    uint32_t member = 0, positive = 0;
    uint64_t sq = 0;
#pragma unroll
    for (int e = 0; e < NE; e++) {
        wgt[e] = 0;
        key[e] = 0;
        if (((valid >> e) & 1u) && v[e] != kNegInf) {
            const float d = v[e] - m;
            const double ee = exp((double)d);
            key[e] = f2key(d);
            wgt[e] = fixed_point(ee, scaleF);
            member |= 1u << e;
            if (ee > 0.0) positive |= 1u << e;
            sq += wgt[e];
        }
    }
    const uint64_t S = block_sum(sq, ctl.r64);
    uint32_t kept = member;
    if (P.top_p < 1.0f) {
        const double thr = (double)(1.0f - P.top_p);
        const uint64_t T = thr >= 1.0 ? ~0ull : (uint64_t)(thr * (double)S);
        const float dmin = mn - m;
        const double lo = fmax((double)dmin, -64.0);
        const double scale = lo < 0.0 ? (double)kBuckets / (-lo) : 0.0;
        auto b1 = [&](int e) -> int {
            const int b = (int)(((double)key2f(key[e]) - lo) * scale);
            return min(max(b, 0), kBuckets - 1);
        };
        uint32_t ckey;
        int cidx;
        weighted_select<NC>(key, wgt, member, T, true, b1, sm.sel, ctl, ckey, cidx);
        kept = 0;
#pragma unroll
        for (int e = 0; e < NE; e++)
            if (((member >> e) & 1u) && (key[e] > ckey || (key[e] == ckey && elem_index(e) >= cidx)))
                kept |= 1u << e;
    }
    // draw: first kept index (index order) whose inclusive prefix mass exceeds floor(u * S_kept)
    uint64_t cs[NC];
#pragma unroll
    for (int c = 0; c < NC; c++) {
        cs[c] = 0;
#pragma unroll
        for (int j = 0; j < 4; j++)
            if ((kept >> (c * 4 + j)) & 1u) cs[c] += wgt[c * 4 + j];
    }
    uint64_t ct[NC];
#pragma unroll
    for (int c = 0; c < NC; c++) ct[c] = cs[c];
    block_sum_vec<NC>(ct, ctl.r64);
    uint64_t Skept = 0;
#pragma unroll
    for (int c = 0; c < NC; c++) Skept += ct[c];
    const uint64_t D = (uint64_t)(u * (double)Skept);
    int cstar = -1;
    uint64_t run = 0;
#pragma unroll
    for (int c = 0; c < NC; c++) {
        if (cstar < 0) {
            if (D - run < ct[c] && D >= run) cstar = c;
            else run += ct[c];
        }
    }
    int pick = -1;
    if (cstar >= 0) {
        uint64_t mine = 0;
#pragma unroll
        for (int c = 0; c < NC; c++)
            if (c == cstar) mine = cs[c];
        uint64_t total;
        const uint64_t excl = block_excl_scan(mine, ctl.r64, total);
        if (tid == 0) ctl.found_idx = -1;
        __syncthreads();
        if (D >= run + excl && D - (run + excl) < mine) {
            uint64_t acc = run + excl;
#pragma unroll
            for (int c = 0; c < NC; c++)
                if (c == cstar)
#pragma unroll
                    for (int j = 0; j < 4; j++) {
                        const int e = c * 4 + j;
                        if ((kept >> e) & 1u) {
                            acc += wgt[e];
                            if (D < acc) {
                                ctl.found_idx = elem_index(e);
                                break;
                            }
                        }
                    }
        }
        __syncthreads();
        pick = ctl.found_idx;
    }
    if (pick < 0) {  // no crossing: the last kept id with p > 0
        int li = -1;
#pragma unroll
        for (int e = 0; e < NE; e++)
            if (((kept >> e) & 1u) && ((positive >> e) & 1u)) li = max(li, elem_index(e));
        pick = block_imax(li, ctl.ri);
        if (pick < 0) pick = 0;
    }
    if (tid == 0) a.out_ids[r] = pick;
    if (prow) {
        double se = 0.0;
#pragma unroll
        for (int e = 0; e < NE; e++)
            if ((kept >> e) & 1u) se += exp((double)(v[e] - m));
        se = block_sum(se, ctl.rd);
#pragma unroll
        for (int e = 0; e < NE; e++)
            if ((valid >> e) & 1u) prow[elem_index(e)] = ((kept >> e) & 1u) ? exp((double)(v[e] - m)) / se : 0.0;
    }
}

template <int NC>
hipError_t launch_nc(const SampleArgs& a, bool vec, hipStream_t stream) {
    const dim3 grid(a.rows), block(kThreads);
    if (vec)
        hipLaunchKernelGGL((sample_rows_kernel<NC, true>), grid, block, 0, stream, a);
    else
        hipLaunchKernelGGL((sample_rows_kernel<NC, false>), grid, block, 0, stream, a);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_sample(const SampleArgs& a, hipStream_t stream) {
    if (a.rows <= 0) return hipSuccess;
    if (a.vocab <= 0 || a.vocab > kRowResidentMaxVocab) return hipErrorNotSupported;
    const int nc = (a.vocab + kSweep - 1) / kSweep;
    const bool vec = (a.vocab % 4 == 0) && (a.ld % 4 == 0) && (((uintptr_t)a.logits & 15u) == 0);
    switch (nc) {
        case 1: return launch_nc<1>(a, vec, stream);
        case 2: return launch_nc<2>(a, vec, stream);
        case 3: return launch_nc<3>(a, vec, stream);
        case 4: return launch_nc<4>(a, vec, stream);
        case 5: return launch_nc<5>(a, vec, stream);
        case 6: return launch_nc<6>(a, vec, stream);
        case 7: return launch_nc<7>(a, vec, stream);
        case 8: return launch_nc<8>(a, vec, stream);
        default: return hipErrorNotSupported;
    }
}

}  // namespace vxs
