// vxs_device.h — gfx950 device primitives of the sampler: DPP wave scans/reductions, group
// (W-wave) combines, order-preserving keys, exact 2^-F fixed-point masses, the correctly rounded
// penalty division and the fp32 exponential used for full-vocabulary masses.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace vxs {
namespace dev {

constexpr float kNegInf = -__builtin_huge_valf();
constexpr float kPosInf = __builtin_huge_valf();

// ---- DPP (gfx9 encodings) ------------------------------------------------------------------
enum : int {
    kRowShr1 = 0x111,
    kRowShr2 = 0x112,
    kRowShr4 = 0x114,
    kRowShr8 = 0x118,
    kRowBcast15 = 0x142,
    kRowBcast31 = 0x143,
    kQuadSwap1 = 0xb1,  // quad_perm [1,0,3,2]
    kQuadSwap2 = 0x4e,  // quad_perm [2,3,0,1]
};

// Lane value moved by DPP; lanes whose source is outside the row/mask keep `old`.
template <int CTRL, int ROW_MASK = 0xf>
__device__ __forceinline__ uint32_t dpp(uint32_t old, uint32_t x) {
    return (uint32_t)__builtin_amdgcn_update_dpp((int)old, (int)x, CTRL, ROW_MASK, 0xf, false);
}
template <int CTRL, int ROW_MASK = 0xf>
__device__ __forceinline__ uint64_t dpp64(uint64_t old, uint64_t x) {
    const uint32_t lo = dpp<CTRL, ROW_MASK>((uint32_t)old, (uint32_t)x);
    const uint32_t hi = dpp<CTRL, ROW_MASK>((uint32_t)(old >> 32), (uint32_t)(x >> 32));
    return ((uint64_t)hi << 32) | lo;
}

// The same for a full row and bank mask with bound_ctrl: lanes whose source is outside the row read
// 0, and no `old` value needs to be set up.
template <int CTRL>
__device__ __forceinline__ uint64_t dpp64z(uint64_t x) {
    const uint32_t lo = (uint32_t)__builtin_amdgcn_mov_dpp((int)(uint32_t)x, CTRL, 0xf, 0xf, true);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_mov_dpp((int)(uint32_t)(x >> 32), CTRL, 0xf, 0xf, true);
    return ((uint64_t)hi << 32) | lo;
}

__device__ __forceinline__ uint32_t readlane(uint32_t x, int lane) {
    return (uint32_t)__builtin_amdgcn_readlane((int)x, lane);
}
__device__ __forceinline__ uint64_t readlane64(uint64_t x, int lane) {
    return ((uint64_t)readlane((uint32_t)(x >> 32), lane) << 32) | readlane((uint32_t)x, lane);
}

// Inclusive prefix sum over the 64 lanes (Hillis-Steele inside rows of 16, then row broadcasts).
__device__ __forceinline__ uint32_t wave_incl_sum(uint32_t x) {
    x += dpp<kRowShr1>(0, x);
    x += dpp<kRowShr2>(0, x);
    x += dpp<kRowShr4>(0, x);
    x += dpp<kRowShr8>(0, x);
    x += dpp<kRowBcast15, 0xa>(0, x);
    x += dpp<kRowBcast31, 0xc>(0, x);
    return x;
}
__device__ __forceinline__ uint64_t wave_incl_sum(uint64_t x) {
    x += dpp64<kRowShr1>(0, x);
    x += dpp64<kRowShr2>(0, x);
    x += dpp64<kRowShr4>(0, x);
    x += dpp64<kRowShr8>(0, x);
    x += dpp64<kRowBcast15, 0xa>(0, x);
    x += dpp64<kRowBcast31, 0xc>(0, x);
    return x;
}
__device__ __forceinline__ uint32_t wave_sum(uint32_t x) { return readlane(wave_incl_sum(x), 63); }
__device__ __forceinline__ uint64_t wave_sum(uint64_t x) { return readlane64(wave_incl_sum(x), 63); }

__device__ __forceinline__ double wave_incl_sum(double x) {
#define VXS_FSTEPZ(C) x += __longlong_as_double((long long)dpp64z<C>((uint64_t)__double_as_longlong(x)));
#define VXS_FSTEP(C, M) \
    x += __longlong_as_double((long long)dpp64<C, M>(0, (uint64_t)__double_as_longlong(x)));
    VXS_FSTEPZ(kRowShr1)
    VXS_FSTEPZ(kRowShr2)
    VXS_FSTEPZ(kRowShr4)
    VXS_FSTEPZ(kRowShr8)
    VXS_FSTEP(kRowBcast15, 0xa)
    VXS_FSTEP(kRowBcast31, 0xc)
#undef VXS_FSTEP
#undef VXS_FSTEPZ
    return x;
}
// Inclusive prefix sum inside each row of 16 lanes.
__device__ __forceinline__ double row_incl_sum(double x) {
#define VXS_FSTEP(C) x += __longlong_as_double((long long)dpp64z<C>((uint64_t)__double_as_longlong(x)));
    VXS_FSTEP(kRowShr1)
    VXS_FSTEP(kRowShr2)
    VXS_FSTEP(kRowShr4)
    VXS_FSTEP(kRowShr8)
#undef VXS_FSTEP
    return x;
}
// Sum over each quad of lanes, in every lane of the quad.
__device__ __forceinline__ double quad_sum(double x) {
    x += __longlong_as_double((long long)dpp64z<kQuadSwap1>((uint64_t)__double_as_longlong(x)));
    x += __longlong_as_double((long long)dpp64z<kQuadSwap2>((uint64_t)__double_as_longlong(x)));
    return x;
}
__device__ __forceinline__ double readlane_d(double x, int lane) {
    return __longlong_as_double((long long)readlane64((uint64_t)__double_as_longlong(x), lane));
}
__device__ __forceinline__ double wave_sum(double x) { return readlane_d(wave_incl_sum(x), 63); }

#define VXS_MSTEP(OP, IDENT, C, M) x = OP(x, __uint_as_float(dpp<C, M>(__float_as_uint(IDENT), __float_as_uint(x))));
__device__ __forceinline__ float wave_max(float x) {
    VXS_MSTEP(fmaxf, kNegInf, kRowShr1, 0xf)
    VXS_MSTEP(fmaxf, kNegInf, kRowShr2, 0xf)
    VXS_MSTEP(fmaxf, kNegInf, kRowShr4, 0xf)
    VXS_MSTEP(fmaxf, kNegInf, kRowShr8, 0xf)
    VXS_MSTEP(fmaxf, kNegInf, kRowBcast15, 0xa)
    VXS_MSTEP(fmaxf, kNegInf, kRowBcast31, 0xc)
    return __uint_as_float(readlane(__float_as_uint(x), 63));
}
__device__ __forceinline__ float wave_min(float x) {
    VXS_MSTEP(fminf, kPosInf, kRowShr1, 0xf)
    VXS_MSTEP(fminf, kPosInf, kRowShr2, 0xf)
    VXS_MSTEP(fminf, kPosInf, kRowShr4, 0xf)
    VXS_MSTEP(fminf, kPosInf, kRowShr8, 0xf)
    VXS_MSTEP(fminf, kPosInf, kRowBcast15, 0xa)
    VXS_MSTEP(fminf, kPosInf, kRowBcast31, 0xc)
    return __uint_as_float(readlane(__float_as_uint(x), 63));
}
#undef VXS_MSTEP

#define VXS_USTEP(OP, IDENT, C, M) x = OP(x, dpp<C, M>(IDENT, x));
__device__ __forceinline__ uint32_t wave_umax(uint32_t x) {
    VXS_USTEP(max, 0u, kRowShr1, 0xf)
    VXS_USTEP(max, 0u, kRowShr2, 0xf)
    VXS_USTEP(max, 0u, kRowShr4, 0xf)
    VXS_USTEP(max, 0u, kRowShr8, 0xf)
    VXS_USTEP(max, 0u, kRowBcast15, 0xa)
    VXS_USTEP(max, 0u, kRowBcast31, 0xc)
    return readlane(x, 63);
}
__device__ __forceinline__ uint32_t wave_umin(uint32_t x) {
    VXS_USTEP(min, 0xffffffffu, kRowShr1, 0xf)
    VXS_USTEP(min, 0xffffffffu, kRowShr2, 0xf)
    VXS_USTEP(min, 0xffffffffu, kRowShr4, 0xf)
    VXS_USTEP(min, 0xffffffffu, kRowShr8, 0xf)
    VXS_USTEP(min, 0xffffffffu, kRowBcast15, 0xa)
    VXS_USTEP(min, 0xffffffffu, kRowBcast31, 0xc)
    return readlane(x, 63);
}
#undef VXS_USTEP

// Max value with the lowest index among equal values (Sampler.ArgMax tie rule).
__device__ __forceinline__ void wave_argmax(float& v, int& i) {
#define VXS_ASTEP(C, M)                                                                \
    {                                                                                  \
        const float ov = __uint_as_float(dpp<C, M>(__float_as_uint(kNegInf), __float_as_uint(v))); \
        const int oi = (int)dpp<C, M>(0x7fffffffu, (uint32_t)i);                       \
        if (ov > v || (ov == v && oi < i)) {                                           \
            v = ov;                                                                    \
            i = oi;                                                                    \
        }                                                                              \
    }
    VXS_ASTEP(kRowShr1, 0xf)
    VXS_ASTEP(kRowShr2, 0xf)
    VXS_ASTEP(kRowShr4, 0xf)
    VXS_ASTEP(kRowShr8, 0xf)
    VXS_ASTEP(kRowBcast15, 0xa)
    VXS_ASTEP(kRowBcast31, 0xc)
#undef VXS_ASTEP
    v = __uint_as_float(readlane(__float_as_uint(v), 63));
    i = (int)readlane((uint32_t)i, 63);
}

__device__ __forceinline__ bool wave_any(bool p) { return __ballot(p) != 0; }

// Order-preserving int image of a non-NaN float (for signed-int max/min): negative values get
// their magnitude bits flipped. The DPP max/min on this image fuses into one instruction per step.
__device__ __forceinline__ int f2ord(float x) {
    const int k = __float_as_int(x);
    return k ^ ((k >> 31) & 0x7fffffff);
}
__device__ __forceinline__ float ord2f(int k) { return __int_as_float(k ^ ((k >> 31) & 0x7fffffff)); }

#define VXS_ISTEP(OP, IDENT, C, M) x = OP(x, (int)dpp<C, M>((uint32_t)(IDENT), (uint32_t)x));
__device__ __forceinline__ int wave_imax_ord(int x) {
    VXS_ISTEP(max, 0x80000000, kRowShr1, 0xf)
    VXS_ISTEP(max, 0x80000000, kRowShr2, 0xf)
    VXS_ISTEP(max, 0x80000000, kRowShr4, 0xf)
    VXS_ISTEP(max, 0x80000000, kRowShr8, 0xf)
    VXS_ISTEP(max, 0x80000000, kRowBcast15, 0xa)
    VXS_ISTEP(max, 0x80000000, kRowBcast31, 0xc)
    return (int)readlane((uint32_t)x, 63);
}
__device__ __forceinline__ int wave_imin_ord(int x) {
    VXS_ISTEP(min, 0x7fffffff, kRowShr1, 0xf)
    VXS_ISTEP(min, 0x7fffffff, kRowShr2, 0xf)
    VXS_ISTEP(min, 0x7fffffff, kRowShr4, 0xf)
    VXS_ISTEP(min, 0x7fffffff, kRowShr8, 0xf)
    VXS_ISTEP(min, 0x7fffffff, kRowBcast15, 0xa)
    VXS_ISTEP(min, 0x7fffffff, kRowBcast31, 0xc)
    return (int)readlane((uint32_t)x, 63);
}
#undef VXS_ISTEP
// max / min of non-NaN floats over the wave
__device__ __forceinline__ float wave_fmax(float x) { return ord2f(wave_imax_ord(f2ord(x))); }
__device__ __forceinline__ float wave_fmin(float x) { return ord2f(wave_imin_ord(f2ord(x))); }

// ---- keys, fixed point, arithmetic ----------------------------------------------------------
// Order-preserving u32 image of a float; -0 maps to +0 (C# compares them equal).
__device__ __forceinline__ uint32_t f2key(float f) {
    if (f == 0.0f) f = 0.0f;
    const uint32_t u = __float_as_uint(f);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float key2f(uint32_t k) {
    const uint32_t u = (k & 0x80000000u) ? (k & 0x7fffffffu) : ~k;
    return __uint_as_float(u);
}

// A key K with at least k of the register-held keys >= K and at most k + slack of them (or the
// exact k-th largest, where ties leave no such K): a bisection over [lo, hi] that stops as soon
// as the count falls in that window. Any such K is a lower bound of the k-th largest.
template <int N>
__device__ __forceinline__ uint32_t wave_bound_regs(const uint32_t (&kk)[N], uint32_t lo, uint32_t hi, int k,
                                                    int slack) {
#pragma unroll 1
    while (lo < hi) {
        const uint32_t mid = lo + ((hi - lo + 1) >> 1);
        int c = 0;
#pragma unroll
        for (int q = 0; q < N; q++) c += __builtin_popcountll(__ballot(kk[q] >= mid));
        if (c >= k) {
            lo = mid;
            if (c <= k + slack) break;
        } else {
            hi = mid - 1;
        }
    }
    return lo;
}

// wave_bound_regs by a four-way search: three thresholds per step (counted independently, so one
// step costs about the latency of one bisection step) narrow [lo, hi] four times over. For rows
// sampled by one workgroup, where the step's dependent chain is the row's time.
template <int N>
__device__ __forceinline__ uint32_t wave_bound_regs4(const uint32_t (&kk)[N], uint32_t lo, uint32_t hi, int k,
                                                     int slack) {
#pragma unroll 1
    while (lo < hi) {
        const uint32_t w = hi - lo + 1;          // at least 2 (valid keys never span all 2^32)
        const uint32_t t1 = lo + (w >> 2);       // lo when w < 4
        const uint32_t t2 = lo + (w >> 1);       // above lo
        const uint32_t t3 = t2 + ((hi - t2 + 1) >> 1);
        int c1 = 0, c2 = 0, c3 = 0;
#pragma unroll
        for (int q = 0; q < N; q++) {
            c1 += __builtin_popcountll(__ballot(kk[q] >= t1));
            c2 += __builtin_popcountll(__ballot(kk[q] >= t2));
            c3 += __builtin_popcountll(__ballot(kk[q] >= t3));
        }
        if (c3 >= k) {
            lo = t3;
            if (c3 <= k + slack) break;
        } else if (c2 >= k) {
            lo = t2;
            hi = t3 - 1;
            if (c2 <= k + slack) break;
        } else if (c1 >= k) {
            lo = t1;
            hi = t2 - 1;
            if (c1 <= k + slack) break;
        } else {
            hi = t1 - 1;
        }
    }
    return lo;
}

// The digit of the need-th largest counted key, from a 256-bin histogram of the current digit read
// by one wave (lane l takes bins 255 - 4l down to 252 - 4l, the counts in descending digit order);
// need drops by the count of keys in higher digits.
__device__ __forceinline__ uint32_t hist_digit(const uint32_t* hist, int lane, int& need) {
    typedef uint32_t u4 __attribute__((ext_vector_type(4)));
    const u4 h4 = reinterpret_cast<const u4*>(hist)[63 - lane];
    const uint32_t c[4] = {h4.w, h4.z, h4.y, h4.x};
    const uint32_t tot = c[0] + c[1] + c[2] + c[3];
    const uint32_t incl = wave_incl_sum(tot);
    uint32_t run = incl - tot;  // entries in higher digits than this lane's
    int digit = -1;
    uint32_t above = 0;
#pragma unroll
    for (int b = 0; b < 4; b++) {
        if (digit < 0 && run < (uint32_t)need && run + c[b] >= (uint32_t)need) {
            digit = 255 - 4 * lane - b;
            above = run;
        }
        run += c[b];
    }
    const uint64_t who = __ballot(digit >= 0);
    const int src = __builtin_ctzll(who);
    need -= (int)__builtin_amdgcn_readlane(above, src);
    return (uint32_t)__builtin_amdgcn_readlane(digit, src);
}

// The exact k-th largest (with multiplicity) of the keys all waves of the workgroup hold in registers
// (0 = empty slot; at least k valid ones in [klo, khi], the workgroup's smallest and largest valid
// key), by the same radix select: every wave counts its keys into one LDS histogram, and after the
// barrier each wave finds the digit from the whole histogram itself (all find the same one), so a
// digit costs one barrier. Three histograms rotate: while one is filled the next is cleared, and the
// one before may still be read by a wave that has not reached this digit. The caller clears the
// first one (h3[0..255]) before a barrier; the workgroup has 256 threads.
template <int N>
__device__ __forceinline__ uint32_t block_kth_radix(const uint32_t (&kk)[N], uint32_t klo, uint32_t khi, int k,
                                                    uint32_t* h3, int t, int lane) {
    constexpr int kRB = 256;  // buckets per digit; the workgroup has 256 threads (one clear each)
    if (klo == khi) return khi;
    const int top = 31 - __clz(klo ^ khi);                        // highest bit that differs
    uint32_t mask = top == 31 ? 0u : ~((2u << top) - 1u);          // the bits every valid key shares ...
    uint32_t prefix = khi & mask;                                  // ... and their value
    int need = k;
    int cur = 0;
#pragma unroll 1
    for (int lo_bit = top - 7;; lo_bit -= 8) {
        const int sh = lo_bit > 0 ? lo_bit : 0;
        const uint32_t dmask = (lo_bit >= 0 ? 0xffu : (0xffu >> -lo_bit));
        uint32_t* hist = h3 + kRB * cur;
        const int nxt = cur == 2 ? 0 : cur + 1;
#pragma unroll
        for (int q = 0; q < N; q++)
            if (kk[q] != 0u && (kk[q] & mask) == prefix) atomicAdd(&hist[(kk[q] >> sh) & dmask], 1u);
        h3[kRB * nxt + t] = 0u;
        __syncthreads();
        const uint32_t d = hist_digit(hist, lane, need);
        prefix |= d << sh;
        mask |= dmask << sh;
        cur = nxt;
        if (sh == 0) break;
    }
    return prefix;
}

// ---- sequential phases of the exact regime (the reference's fp64 loops, Sampler.cs:58-87) ----
// They run redundantly in every thread on LDS broadcast reads; LDS is read 8 entries at a time so
// one read latency covers eight steps, and the steps are branch-free.

// A zero the compiler cannot prove wave-uniform. Indexing the LDS reads of a sequential loop with
// it keeps the loop's running counts in vector registers: otherwise every compare result of a
// broadcast value is moved to a scalar register (a read-first-lane and a dependent scalar add per
// step, several times slower than the vector count).
__device__ __forceinline__ int lane_zero() {
    int z;
    asm volatile("v_mov_b32 %0, 0" : "=v"(z));
    return z;
}

// Left-to-right double sum of x[0..n) (the reference's sequential Sum).
__device__ __forceinline__ double seq_sum(const double* x, int n) {
    double s = 0.0;
    int j = 0;
    for (; j + 8 <= n; j += 8) {
        double b[8];
#pragma unroll
        for (int k = 0; k < 8; k++) b[k] = x[j + k];
#pragma unroll
        for (int k = 0; k < 8; k++) s += b[k];
    }
    for (; j < n; j++) s += x[j];
    return s;
}

// seq_sum with the next batch of eight read while the current one is added (x 16-byte aligned): for
// long sums, where the read latency of each batch would otherwise add to the chain.
__device__ __forceinline__ double seq_sum_pipe(const double* x, int n) {
    typedef double d2 __attribute__((ext_vector_type(2)));
    const d2* v = reinterpret_cast<const d2*>(x);
    double s = 0.0;
    int j = 0;
    if (n >= 8) {
        // b holds the batch before j, read but not yet added
        d2 b[4], c[4];
#pragma unroll
        for (int k = 0; k < 4; k++) b[k] = v[k];
        j = 8;
        for (; j + 16 <= n; j += 16) {
#pragma unroll
            for (int k = 0; k < 4; k++) c[k] = v[j / 2 + k];
#pragma unroll
            for (int k = 0; k < 4; k++) {
                s += b[k].x;
                s += b[k].y;
            }
#pragma unroll
            for (int k = 0; k < 4; k++) b[k] = v[j / 2 + 4 + k];
#pragma unroll
            for (int k = 0; k < 4; k++) {
                s += c[k].x;
                s += c[k].y;
            }
        }
        if (j + 8 <= n) {
#pragma unroll
            for (int k = 0; k < 4; k++) c[k] = v[j / 2 + k];
#pragma unroll
            for (int k = 0; k < 4; k++) {
                s += b[k].x;
                s += b[k].y;
            }
#pragma unroll
            for (int k = 0; k < 4; k++) b[k] = c[k];
            j += 8;
        }
#pragma unroll
        for (int k = 0; k < 4; k++) {
            s += b[k].x;
            s += b[k].y;
        }
    }
    for (; j < n; j++) s += x[j];
    return s;
}

// Top-p cut over the (p, index)-sorted order (order[s] = entry at sorted position s): the number
// of leading positions, among the first n - 1, whose running sum stays <= thr (Sampler.cs:66-73).
// The running sum never decreases until it turns NaN (and stays NaN), so the reference's first
// position with !(cum <= thr) equals the number of prefixes with cum <= thr, counted off the
// critical path of the additions; the scan stops after the deciding batch.
__device__ __forceinline__ int seq_topp_cut(const double* p, const int16_t* order, int n, double thr) {
    const int z = lane_zero();
    double cum = 0.0;
    int nrem = 0;
    for (int s0 = 0; s0 < n - 1 && nrem == s0; s0 += 8) {
        double pb[8];
#pragma unroll
        for (int k = 0; k < 8; k++) {  // clamped indices: the reads are unconditional and overlap
            const double pk = p[order[min(s0 + k, n - 1) + z]];
            pb[k] = s0 + k < n - 1 ? pk : 0.0;
        }
#pragma unroll
        for (int k = 0; k < 8; k++) {
            cum += pb[k];
            nrem += (s0 + k < n - 1 && cum <= thr) ? 1 : 0;
        }
    }
    return nrem;
}

// Inverse-CDF draw in index order over p[0..n) with ids id[0..n) (Sampler.cs:77-87): the first
// entry whose running sum exceeds u, skipping entries with p <= 0 (NaN is not skipped); without
// one, the last entry visited (0 when none). Skipped entries add 0, which leaves the running sum
// unchanged, and it never decreases until it turns NaN, so the first crossing is the number of
// prefixes <= u, provided that is below the first NaN prefix.
__device__ __forceinline__ int seq_draw(const double* p, const int32_t* id, int n, double u) {
    const int z = lane_zero();
    double acc = 0.0;
    int below_u = 0, nan_prefixes = 0, lastj = -1, scanned = 0;
    for (int j0 = 0; j0 < n && below_u == j0 && nan_prefixes == 0; j0 += 8) {
        scanned = min(n, j0 + 8);
        double pb[8];
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const double pk = p[min(j0 + k, n - 1) + z];  // clamped: unconditional reads
            const double pj = j0 + k < n ? pk : 0.0;
            const bool take = !(pj <= 0.0);
            pb[k] = take ? pj : 0.0;
            lastj = take ? j0 + k : lastj;
        }
#pragma unroll
        for (int k = 0; k < 8; k++) {
            acc += pb[k];
            below_u += (j0 + k < n && acc <= u) ? 1 : 0;
            nan_prefixes += (j0 + k < n && acc != acc) ? 1 : 0;
        }
    }
    // After an early stop `lastj` may have missed later entries; it only matters without a pick,
    // and then every batch was scanned or a NaN prefix appeared (the reference keeps visiting
    // entries after it): `lastj` is finished over all entries in that case.
    const int first_nan = nan_prefixes > 0 ? scanned - nan_prefixes : n;
    if (below_u < first_nan) return id[below_u];
    if (nan_prefixes > 0)
        for (int j = 0; j < n; j++) lastj = !(p[j] <= 0.0) ? j : lastj;
    return lastj >= 0 ? id[lastj] : 0;
}

// ---- one-wave forms of the top-p cut and the draw: every lane runs the same dependent chain of
// additions over LDS reads in batches of eight (the reads of a batch issued before its adds); the
// running sum never decreases until it turns NaN, so the batch that holds the deciding prefix is
// the first whose last prefix decides, and the prefix is found among that batch's eight. Same
// results as seq_topp_cut and seq_draw.

// seq_topp_cut by one wave, on the probabilities already gathered into sorted order
// (ps[s] = p[order[s]]): the number of leading positions, among the first n - 1, whose running sum
// stays <= thr.
__device__ __forceinline__ int wave_topp_cut(const double* ps, int n, double thr) {
    const int m = n - 1;  // the positions the reference may remove
    double cum = 0.0;
    int j = 0;
    for (; j + 8 <= m; j += 8) {
        double b[8], c[8];
#pragma unroll
        for (int k = 0; k < 8; k++) b[k] = ps[j + k];
#pragma unroll
        for (int k = 0; k < 8; k++) {
            cum += b[k];
            c[k] = cum;
        }
        if (!(cum <= thr)) {
            int f = 8;
#pragma unroll
            for (int k = 7; k >= 0; k--) f = !(c[k] <= thr) ? k : f;
            return j + f;
        }
    }
    for (; j < m; j++) {
        cum += ps[j];
        if (!(cum <= thr)) return j;
    }
    return m;
}

// wave_topp_cut for n <= 256 without the dependent chain, same result. Lane l sums positions
// 4l..4l+3 and a wave scan adds the lanes before it: every prefix sum P_j of the first n - 1
// probabilities with at most 10 roundings on any term's path, so |P_j - T_j| <= 10 u T_j for the
// exact prefix sum T_j (u = 2^-53, the terms are non-negative). The reference's running sum C_j,
// j + 1 <= 255 terms added left to right, has |C_j - T_j| <= 254 u T_j (Higham, Accuracy and
// Stability of Numerical Algorithms, 2nd ed., 4.2), so |C_j - P_j| < 2^-44 P_j. C_j never decreases,
// so the first j with C_j > thr is the first j with P_j > thr whenever P_j (1 - 2^-40) > thr and
// P_{j-1} (1 + 2^-40) <= thr (no crossing: P_{m-1} (1 + 2^-40) <= thr). With thr that close to a
// prefix sum, or NaN, the sequential form decides.
__device__ __forceinline__ int wave_topp_cut_par(const double* ps, int n, double thr, int lane) {
    const int m = n - 1;  // the positions the reference may remove
    if (n > 256) return wave_topp_cut(ps, n, thr);
    if (m <= 0) return 0;
    const int j0 = 4 * lane;
    double P[4];
#pragma unroll
    for (int k = 0; k < 4; k++) P[k] = j0 + k < m ? ps[j0 + k] : 0.0;
    P[1] += P[0];
    P[2] += P[1];
    P[3] += P[2];
    const double incl = wave_incl_sum(P[3]);
    double excl = __shfl_up(incl, 1);
    excl = lane == 0 ? 0.0 : excl;
#pragma unroll
    for (int k = 0; k < 4; k++) P[k] += excl;
    int f = 4;  // this lane's first position with P_j > thr (or NaN)
#pragma unroll
    for (int k = 3; k >= 0; k--) f = (j0 + k < m && !(P[k] <= thr)) ? k : f;
    const uint64_t bal = __ballot(f < 4);
    constexpr double kUp = 1.0 + 0x1p-40, kDown = 1.0 - 0x1p-40;
    if (bal == 0) {  // no P_j above thr: C_j stays <= thr for every j < m if P_{m-1} is clear of it
        const int lm = (m - 1) >> 2, km = (m - 1) & 3;
        const double pl = km == 0 ? P[0] : km == 1 ? P[1] : km == 2 ? P[2] : P[3];
        const double last = readlane_d(pl, lm);
        if (last * kUp <= thr) return m;
        return wave_topp_cut(ps, n, thr);
    }
    const int src = __builtin_ctzll(bal);
    const double pf = f == 0 ? P[0] : f == 1 ? P[1] : f == 2 ? P[2] : P[3];
    const double pb = f == 0 ? excl : f == 1 ? P[0] : f == 2 ? P[1] : P[2];  // the prefix before it
    const int js = 4 * src + __builtin_amdgcn_readlane(f, src);
    const double pj = readlane_d(pf, src), pp = readlane_d(pb, src);
    if (pj * kDown > thr && (js == 0 || pp * kUp <= thr)) return js;
    return wave_topp_cut(ps, n, thr);
}

// seq_draw by one wave over p[0..n) with ids id[0..n): the first entry whose running sum exceeds u,
// or without one the last entry with p > 0 or NaN (0 when none). Skipped entries (p <= 0) hold +0
// here (the probabilities are exp(d) / sum >= +0, removed ones +0), so adding them leaves the
// running sum unchanged and the chain adds every entry.
__device__ __forceinline__ int wave_draw(const double* p, const int32_t* id, int n, double u) {
    double acc = 0.0;
    int j = 0, pick = -1;
    for (; j + 8 <= n; j += 8) {
        double b[8], c[8];
#pragma unroll
        for (int k = 0; k < 8; k++) b[k] = p[j + k];
#pragma unroll
        for (int k = 0; k < 8; k++) {
            acc += b[k];
            c[k] = acc;
        }
        if (!(acc <= u)) {  // the crossing, or a NaN prefix, is in this batch
            int f = 8;
#pragma unroll
            for (int k = 7; k >= 0; k--) f = !(c[k] <= u) ? k : f;
            if (u < c[f]) pick = j + f;  // a NaN prefix first: no crossing at all
            break;
        }
    }
    if (pick < 0 && acc <= u)
        for (; j < n; j++) {
            acc += p[j];
            if (!(acc <= u)) {
                if (u < acc) pick = j;
                break;
            }
        }
    if (pick >= 0) return id[pick];
    int last = -1;
    for (int q = 0; q < n; q++) last = !(p[q] <= 0.0) ? q : last;
    return last >= 0 ? id[last] : 0;
}

// The draw over q (lane j: candidate j in index order, `keep` for p > 0) by a wave prefix sum in
// place of the sequential running sum. q is p / s with s any fp64 sum of the kept p (or p itself
// when it was already divided by the reference's sum); both the sequential loop's running sums and
// the scan's lie within 64 * 2^-52 of the exact partial sums of p / (exact sum p), relative to 1
// (at most 64 terms, each sum within gamma_63 of its exact value in any order, one rounding per
// quotient), so a crossing that clears u by more than 2^-40 is the sequential loop's crossing, and
// u clearing every kept sum by that much means no crossing (the last kept entry is drawn).
// Returns the lane drawn, or -1 when u lies within 2^-40 of a deciding sum, u is NaN or a kept q is
// not in (0, 1]: the caller then runs the sequential form.
__device__ __forceinline__ int wave_draw_par(double q, bool keep, double u) {
    constexpr double kBand = 0x1p-40;
    const double c = wave_incl_sum(keep ? q : 0.0);
    const uint64_t kb = __ballot(keep);
    // NaN, beyond 1, or a kept p whose quotient underflowed to 0 (the reference's draw skips it)
    const uint64_t bad = __ballot(keep && !(q > 0.0 && q <= 1.0));
    const uint64_t sure = __ballot(keep && u < c - kBand);
    const uint64_t maybe = __ballot(keep && u < c + kBand);
    if (bad || !kb) return -1;
    if (!maybe) return !(u >= 0.0) ? -1 : 63 - __builtin_clzll(kb);
    if (sure && __builtin_ctzll(sure) == __builtin_ctzll(maybe)) return __builtin_ctzll(sure);
    return -1;
}

// LDS ordering inside one wave.
__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// The reference's sequential fp64 arithmetic (Sampler.cs:51-87) on n <= 64 candidates by one wave,
// candidate j (index order) in lane j: x = its logit after temperature and the top-k mask, m = the
// row maximum; ids[0..n) their vocabulary indices (LDS). Entries outside the candidates have p = 0:
// they add nothing to any sum, sort first in the top-p order (where the loop passes over them) and
// are never drawn. The sequential sums read their terms from LDS in batches (the reads of a batch
// issued before its adds), every lane adding the same terms in the reference's order; ranks and the
// crossings are found in register batches. The first sum (the divisor of every probability) is
// always the sequential one; the draw, and without prow the second sum before it, are decided by
// wave sums (wave_draw_par) unless u lies within their rounding band of a deciding running sum,
// when the sequential forms run. scr: 193 doubles of wave-private LDS. Returns the sampled id
// (uniform); with prow, lanes < n store their final probability to prow[ids[lane]].
__device__ __forceinline__ int wave_exact(float x, const int32_t* ids, int n, float m, bool topp, float top_p,
                                          double u, double* scr, double* prow, int lane) {
    n = __builtin_amdgcn_readfirstlane(n);  // uniform in fact; so the compiler keeps the loops scalar
    double* cp = scr;                                        // p in index order
    double* ps = scr + 64;                                   // p in (p, index) order
    uint64_t* key = reinterpret_cast<uint64_t*>(scr + 128);  // sort keys, then lanes by sorted position
    const bool in = lane < n;
    double p = in ? exp((double)(x - m)) : 0.0;  // :57, x - m in fp32, then Math.Exp
    cp[lane] = p;
    wave_lds_sync();
    p = in ? p / seq_sum_pipe(cp, n) : 0.0;  // :58-60, the sum in index order
    if (!topp) {
        if (prow && in) prow[ids[lane]] = p;
        const int jp = wave_draw_par(p, in && !(p <= 0.0), u);
        if (jp >= 0) return ids[jp];
        cp[lane] = p;
        wave_lds_sync();
        return wave_draw(cp, ids, n, u);  // :77-87
    }
    // :62-75. Stable ascending (p, index) order. p = exp(d) / sum never decreases with
    // d = fl32(x - m), so the (d, index) order is taken when every adjacent pair of it is in
    // (p, index) order, else the entries are ranked by p directly.
    const uint64_t k = in ? ((uint64_t)f2key(x - m) << 32) | (uint32_t)lane : ~0ull;
    key[lane] = k;
    if (lane == 0) key[n] = ~0ull;  // above every key: the rank loop reads pairs
    cp[lane] = p;
    wave_lds_sync();
    int rank = 0;
    {
        typedef unsigned long long u64x2 __attribute__((ext_vector_type(2)));
        const u64x2* kp = reinterpret_cast<const u64x2*>(key);
#pragma unroll 4
        for (int l = 0; l < n; l += 2) {
            const u64x2 q = kp[l / 2];
            rank += (q.x < k ? 1 : 0) + (q.y < k ? 1 : 0);
        }
    }
    wave_lds_sync();  // every lane has read the keys
    int* at = reinterpret_cast<int*>(key);
    if (in) {
        ps[rank] = p;
        at[rank] = lane;
    }
    wave_lds_sync();
    const bool has_next = in && rank + 1 < n;
    const double pn = ps[has_next ? rank + 1 : 0];
    const int ln = at[has_next ? rank + 1 : 0];
    if (__ballot(has_next && !(p < pn || (p == pn && lane < ln)))) {
        rank = 0;
#pragma unroll 8
        for (int l = 0; l < n; l++) {
            const double pl = cp[l];
            rank += (pl < p || (pl == p && l < lane)) ? 1 : 0;
        }
        wave_lds_sync();  // every lane has read ps above
        if (in) ps[rank] = p;
        wave_lds_sync();
    }
    // positions 0 .. n - 2 are removed while the running sum stays <= 1 - top_p
    const int nrem = wave_topp_cut_par(ps, n, (double)(1.0f - top_p), lane);
    if (in && rank < nrem) p = 0.0;
    // The entries left with p > 0 (or NaN), in index order: the second sum and the draw over them
    // alone are the reference's over all n (adding zero changes no sum; the draw skips p <= 0).
    const bool keep = in && !(p <= 0.0);
    if (!prow) {  // the draw decided by a parallel sum and scan (the probabilities are not returned)
        const double s2p = wave_sum(keep ? p : 0.0);
        const int jp = wave_draw_par(keep ? p / s2p : 0.0, keep, u);
        if (jp >= 0) return ids[jp];
    }
    const uint64_t kb = __ballot(keep);
    const int nk = (int)__builtin_popcountll(kb);
    const int pos = (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(kb >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)kb, 0u));
    double* kp = ps;  // the cut has read ps (its result is uniform, so every lane is past it)
    int32_t* kid = reinterpret_cast<int32_t*>(key);
    wave_lds_sync();
    if (keep) {
        kp[pos] = p;
        kid[pos] = ids[lane];
    }
    wave_lds_sync();
    const double s2 = seq_sum(kp, nk);  // probs.Sum() in index order
    p = in ? p / s2 : 0.0;              // :74
    if (prow && in) prow[ids[lane]] = p;
    wave_lds_sync();  // every lane has read kp
    if (keep) kp[pos] = p;
    wave_lds_sync();
    return wave_draw(kp, kid, nk, u);  // :77-87
}

// Stable ascending (p, index) rank of entry j among p[0..n).
__device__ __forceinline__ int seq_rank(const double* p, int n, int j) {
    const double pj = p[j];
    int rank = 0;
#pragma unroll 8
    for (int l = 0; l < n; l++) {
        const double pl = p[l];
        rank += (int)((pl < pj) | ((pl == pj) & (l < j)));
    }
    return rank;
}

// Nucleus mass of a weight q in [0, 1], a multiple of 2^-F: q itself when q >= Cb = 2^(23 - F) (every
// fp32 value there is a multiple of 2^-F), else fl32(fl32(q + Cb) - Cb), q rounded to the nearest
// multiple of 2^-F (fl32(q + Cb) lies in [Cb, 2 Cb], where the ulp is 2^-F, and the subtraction is
// exact). Monotone in q. Sums of up to 2^(53-F) such masses are exact in double precision, so
// partial sums and LDS atomics are order-independent.
__device__ __forceinline__ float mass_bias(int F) { return __uint_as_float((uint32_t)(150 - F) << 23); }
__device__ __forceinline__ float mass_of(float q, float Cb) { return q >= Cb ? q : (q + Cb) - Cb; }
// The same mass as an integer-valued double (units of 2^-F).
__device__ __forceinline__ double fixed_mass(float q, float Cb, double scaleF) { return (double)mass_of(q, Cb) * scaleF; }

// Repetition penalty of one logit (Sampler.cs:31): s*rho if s < 0, else s/rho correctly rounded.
// The quotient uses rinv = RN(1/rho) and one fma correction (Markstein): with s and rho in
// [2^-60, 2^60] no intermediate leaves the normal range, so the result is the correctly rounded
// s/rho; every other case (zeros, tiny or huge values, `fast` false) takes the IEEE division.
__device__ __forceinline__ float penalize(float s, float rho, float rinv, bool fast) {
    if (s < 0.0f) return s * rho;
    if (!(fast && s >= 0x1p-60f && s <= 0x1p60f)) return s / rho;
    const float t0 = s * rinv;
    const float rem = __builtin_fmaf(-t0, rho, s);
    return __builtin_fmaf(rem, rinv, t0);
}

// The same penalty without branches for the common case: s*rho for s <= 0, else the Markstein
// quotient, which is the correctly rounded s/rho unless penalize_needs_division(s, fast).
__device__ __forceinline__ float penalize_fast(float s, float rho, float rinv) {
    const float t0 = s * rinv;
    const float q = __builtin_fmaf(__builtin_fmaf(-t0, rho, s), rinv, t0);
    return s <= 0.0f ? s * rho : q;  // zeros keep their sign, as s / rho keeps it
}
__device__ __forceinline__ bool penalize_needs_division(float s, bool fast) {
    return !(s < 0.0f) && !(fast && s >= 0x1p-60f && s <= 0x1p60f);
}

// Nucleus weight of d = x - max <= 0 for vocabularies up to 8192 (the one-wave and one-workgroup
// kernels): 2^fl32(d * fl32(log2 e)) with the hardware 2^x, three VALU operations. Monotone
// non-decreasing in d (one rounding of a product by a positive constant, then a monotone 2^x; both
// checked on every float of [-128, 0] by vxs_selfcheck). Relative error at most |d| * 7.4e-8 plus
// the 2^x rounding: the rounding of d * log2e to fp32 (half an ulp of |d| * 1.44) and the 1.3e-8
// relative error of the constant, each scaled by ln 2. Over a row the mass-weighted error of any
// cumulative sum is at most E_p[|d|] * 7.4e-8 + 1.2e-7 relative to the total, below 6e-7 for every
// row of at most 8192 entries (E_p[|d|] <= 6.3 there), inside the 1e-6 band in which a draw or a
// top-p cut may differ from the reference's. -inf gives 0.
__device__ __forceinline__ float nucleus_exp(float d) {
    return __builtin_amdgcn_exp2f(d * 1.44269502162933349609375f);
}

// exp(d) for d <= 0 in fp32: 2^(d log2 e) with the product carried in two parts (the rounding
// error of d*L2E recovered by fma, plus d times the tail of log2 e) and the hardware 2^x. Relative
// error about 1e-7; 0 for d = -inf or results below 2^-126 (d is clamped at -256 first).
__device__ __forceinline__ float exp_neg_unclamped(float d);
__device__ __forceinline__ float exp_neg(float d) { return exp_neg_unclamped(__builtin_fmaxf(d, -256.0f)); }
// The same without the clamp, for d in [-256, 0] (where the clamp changes nothing).
__device__ __forceinline__ float exp_neg_unclamped(float d) {
    constexpr float kL2E = 1.44269502162933349609375f;          // fl32(log2 e)
    constexpr float kL2ELo = 1.925963033500011079e-8f;          // log2 e - kL2E
    constexpr float kLn2 = 0.693147180559945309f;
    const float y = d * kL2E;
    float yl = __builtin_fmaf(d, kL2E, -y);
    yl = __builtin_fmaf(d, kL2ELo, yl);
    const float e = __builtin_amdgcn_exp2f(y);
    return __builtin_fmaf(e, yl * kLn2, e);
}

// exp(d) for d <= 0 as a probability's numerator in fp64: the fp32 form where its result is a normal
// number (relative error about 1e-7), the fp64 exponential below that (d < -87, where the fp32 form
// returns 0 and the reference's fp64 Math.Exp still gives a positive value, down to its own
// underflow at d = -745.13).
__device__ __forceinline__ double exp_neg_prob(float d) { return d >= -87.0f ? (double)exp_neg(d) : exp((double)d); }

}  // namespace dev
}  // namespace vxs
