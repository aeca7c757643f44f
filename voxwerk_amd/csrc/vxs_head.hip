// vxs_head.hip — the logit heads on the GPU, the step before the sampler.
//
// CodecHead and CodePredictorHead (src/Voxwerk/Talker/TalkerModel.cs:133-137) multiply a few fp32
// hidden rows by a bf16 weight (the checkpoint's [out, in] layout, WeightPrecision.BFloat16,
// DecoderStack.cs:7-15): out[r][n] = sum_k x[r][k] * W[n][k]. With the rows of a decode step
// (1-24) this is a GEMV; the logits stay in HBM for the sampler. From 8 rows the matrix cores take it
// (head_mfma_kernel, with x split exactly into three bf16 parts); below, the VALU form with fp32
// products.
//
// VALU layout: a wave owns R = 8 consecutive outputs (4 when k > 1024, 2 for one or two rows); lane l
// holds W[n][k] for k = 512 j + 8 l + 0..7
// (one 16-byte load per output and j, 1 KiB contiguous per wave instruction), all of its rows in
// registers for the whole call. Per hidden row the lane loads its x slice (the next row's loads
// issued before the current row's products), forms 8 partial dots and reduces them across the
// wave by halving exchanges (xor 32, 16, 8: each lane keeps half of its partials and adds its
// partner's other half) and then plain butterflies (xor 4, 2, 1): with R = 8, lane l ends with
// output 4 b5 + 2 b4 + b3 of the wave, summed over all 64 lanes. The fp32 sum order is this kernel's own;
// it differs from the reference's AVX-512 order by rounding only (bounded by K 2^-24 sum |x w|).
//
// The int8 form (WeightPrecision.Int8, DecoderStack.cs:7-16) keeps W as q[n][k] in [-127, 127] and
// one fp32 scale per output (PackedMatrix.FromBf16LinearInt8, PackedMatrix.cs:124-154):
// out[r][n] = scale[n] * sum_k x[r][k] * q[n][k], the scale applied to the fp32 dot as the decode
// path does (Gemm.cs:650-680, PanelPairDotInt8 / PanelDotInt8). Same layout and reduction, half the
// weight bytes; a lane widens its int8 slice to fp32 once (exact) and keeps it in registers for
// every row, so a row costs one FMA per weight. The packing itself runs on the GPU too
// (head_pack_i8_kernel): per output the largest |w|, scale = amax / 127 (1 for an all-zero row),
// q = clamp(round-half-even(w * (1 / scale)), -127, 127), all in correctly rounded fp32.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <type_traits>

#include "vxs_internal.h"

namespace vxs {
namespace {

constexpr int kHT = 256;  // threads per workgroup

typedef float f4 __attribute__((ext_vector_type(4)));
typedef unsigned int u4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float lo16(unsigned w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float hi16(unsigned w) { return __uint_as_float(w & 0xFFFF0000u); }

// 8 bf16 (packed in u4) times 8 fp32, added to acc in k order.
__device__ __forceinline__ float dot8(u4 w, f4 xa, f4 xb, float acc) {
    acc = __builtin_fmaf(lo16(w.x), xa.x, acc);
    acc = __builtin_fmaf(hi16(w.x), xa.y, acc);
    acc = __builtin_fmaf(lo16(w.y), xa.z, acc);
    acc = __builtin_fmaf(hi16(w.y), xa.w, acc);
    acc = __builtin_fmaf(lo16(w.z), xb.x, acc);
    acc = __builtin_fmaf(hi16(w.z), xb.y, acc);
    acc = __builtin_fmaf(lo16(w.w), xb.z, acc);
    acc = __builtin_fmaf(hi16(w.w), xb.w, acc);
    return acc;
}

// One lane's slice of hidden row m: x[m][512 j + 8 lane + 0..7] for each j. FULL: k = 512 KJ, every
// slice inside the row; otherwise slices past k read the row's start and are zeroed (a select that
// waits for the load, so only the partial shapes pay it).
template <int KJ>
struct XSlice {
    f4 a[KJ], b[KJ];
};

template <int KJ, bool FULL>
__device__ __forceinline__ XSlice<KJ> load_x(const HeadArgs& h, int m, int lane) {
    XSlice<KJ> r;
#pragma unroll
    for (int j = 0; j < KJ; j++) {
        const int k = 512 * j + 8 * lane;
        const bool in = FULL || k < h.k;
        const float* p = h.x + (int64_t)m * h.ldx + (in ? k : 0);
        const f4 a = *reinterpret_cast<const f4*>(p);
        const f4 b = *reinterpret_cast<const f4*>(p + 4);
        r.a[j] = FULL || in ? a : f4{0.f, 0.f, 0.f, 0.f};
        r.b[j] = FULL || in ? b : f4{0.f, 0.f, 0.f, 0.f};
    }
    return r;
}

// One halving exchange over lane bit `mask`: of 2H partials (outputs 2H apart in the lane pair),
// each lane keeps the half its bit selects and adds the partner's copy of it.
template <int H>
__device__ __forceinline__ void halve(const float (&in)[2 * H], float (&out)[H], int lane, int mask) {
    const bool bit = (lane & mask) != 0;
#pragma unroll
    for (int i = 0; i < H; i++) {
        const float lo = in[i], hi = in[i + H];
        out[i] = (bit ? hi : lo) + __shfl_xor(bit ? lo : hi, mask);
    }
}

// The wave's R partial dots of one row reduced to one output per lane group (see the layout note).
template <int R>
__device__ __forceinline__ float reduce_outputs(const float (&v)[R], int lane) {
    constexpr int kGroup = 64 / R;
    float sum;
    if constexpr (R == 8) {
        float q[4], t[2], s1[1];
        halve<4>(v, q, lane, 32);
        halve<2>(q, t, lane, 16);
        halve<1>(t, s1, lane, 8);
        sum = s1[0];
    } else if constexpr (R == 4) {
        float q[2], s1[1];
        halve<2>(v, q, lane, 32);
        halve<1>(q, s1, lane, 16);
        sum = s1[0];
    } else {
        float s1[1];
        halve<1>(v, s1, lane, 32);
        sum = s1[0];
    }
#pragma unroll
    for (int mask = kGroup / 2; mask >= 1; mask /= 2) sum += __shfl_xor(sum, mask);
    return sum;
}

// R outputs per wave (8 or 4), KJ slices of 8 per lane (k <= 512 KJ).
template <int KJ, int R, bool FULL>
__global__ __launch_bounds__(kHT) void head_kernel(HeadArgs a) {
    static_assert(R == 8 || R == 4 || R == 2, "eight, four or two outputs per wave");
    constexpr int kGroup = 64 / R;  // lanes that share an output after the halving exchanges
    const int lane = threadIdx.x & 63;
    const int n0 = (blockIdx.x * (kHT / 64) + (threadIdx.x >> 6)) * R;
    if (n0 >= a.n) return;  // whole wave past the last output (wave-uniform)

    // this lane's weights, kept as bf16 pairs
    u4 w[R][KJ];
#pragma unroll
    for (int o = 0; o < R; o++)
#pragma unroll
        for (int j = 0; j < KJ; j++) {
            const int k = 512 * j + 8 * lane;
            const bool in = n0 + o < a.n && (FULL || k < a.k);
            // every lane loads from inside W (a clamped address) and zeroes what lies outside
            const uint16_t* p = a.w + (int64_t)min(n0 + o, a.n - 1) * a.ldw + (FULL || k < a.k ? k : 0);
            const u4 v = __builtin_nontemporal_load(reinterpret_cast<const u4*>(p));
            w[o][j] = in ? v : u4{0u, 0u, 0u, 0u};
        }

    // output this lane holds after the halving exchanges (lane bits 5, 4[, 3], most significant first)
    const int o_mine = R == 8   ? 4 * ((lane >> 5) & 1) + 2 * ((lane >> 4) & 1) + ((lane >> 3) & 1)
                       : R == 4 ? 2 * ((lane >> 5) & 1) + ((lane >> 4) & 1)
                                : (lane >> 5) & 1;
    // rows two at a time with two slice buffers, each reloaded in place while the other is used,
    // so a row's loads are in flight during the previous row's products and exchanges
    auto row = [&](int m, const XSlice<KJ>& x) {
        if constexpr (KJ > 2) {  // keep the weights packed (widened per row): half the registers
#pragma unroll
            for (int o = 0; o < R; o++)
#pragma unroll
                for (int j = 0; j < KJ; j++) asm volatile("" : "+v"(w[o][j]));
        }
        float v[R];
#pragma unroll
        for (int o = 0; o < R; o++) {
            float acc = 0.f;
#pragma unroll
            for (int j = 0; j < KJ; j++) acc = dot8(w[o][j], x.a[j], x.b[j], acc);
            v[o] = acc;
        }
        const float sum = reduce_outputs<R>(v, lane);
        if ((lane & (kGroup - 1)) == 0 && n0 + o_mine < a.n) a.out[(int64_t)m * a.ldo + n0 + o_mine] = sum;
    };
    // this workgroup's rows: group blockIdx.y of a.row_group rows
    const int first = blockIdx.y * a.row_group;
    const int last = min(a.rows, first + a.row_group) - 1;
    XSlice<KJ> x0 = load_x<KJ, FULL>(a, first, lane);
    for (int m = first; m <= last; m += 2) {
        XSlice<KJ> x1 = load_x<KJ, FULL>(a, min(m + 1, last), lane);
        row(m, x0);
        if (m + 1 > last) break;
        x0 = load_x<KJ, FULL>(a, min(m + 2, last), lane);
        row(m + 1, x1);
    }
}

typedef unsigned int u2 __attribute__((ext_vector_type(2)));

// int8 weights, widened once: R outputs per wave, KJ slices of 8 per lane (k <= 512 KJ).
template <int KJ, int R, bool FULL>
__global__ __launch_bounds__(kHT) void head_i8_kernel(HeadArgs a) {
    static_assert(R == 8 || R == 4 || R == 2, "eight, four or two outputs per wave");
    constexpr int kGroup = 64 / R;
    const int lane = threadIdx.x & 63;
    const int n0 = (blockIdx.x * (kHT / 64) + (threadIdx.x >> 6)) * R;
    if (n0 >= a.n) return;  // whole wave past the last output (wave-uniform)

    // every lane loads from inside q (a clamped address) and zeroes what lies outside; all loads
    // are issued before the first conversion
    u2 raw[R][KJ];
#pragma unroll
    for (int o = 0; o < R; o++)
#pragma unroll
        for (int j = 0; j < KJ; j++) {
            const int k = 512 * j + 8 * lane;
            const int8_t* p = a.q + (int64_t)min(n0 + o, a.n - 1) * a.ldw + (FULL || k < a.k ? k : 0);
            raw[o][j] = __builtin_nontemporal_load(reinterpret_cast<const u2*>(p));
        }
    // q = (q + 128) - 128: the biased byte (sign bit flipped) converted as unsigned, then an exact
    // fp32 subtraction. (A sign-extended byte fed straight to the conversion was compiled here into
    // an unsigned conversion of the extended value.)
    float w[R][KJ][8];
#pragma unroll
    for (int o = 0; o < R; o++)
#pragma unroll
        for (int j = 0; j < KJ; j++) {
            const int k = 512 * j + 8 * lane;
            const bool in = n0 + o < a.n && (FULL || k < a.k);
            const uint32_t lo = raw[o][j].x ^ 0x80808080u, hi = raw[o][j].y ^ 0x80808080u;
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const float f = (float)(((i < 4 ? lo : hi) >> (8 * (i & 3))) & 0xffu) - 128.0f;
                w[o][j][i] = in ? f : 0.0f;
            }
        }
    const int o_mine = R == 8   ? 4 * ((lane >> 5) & 1) + 2 * ((lane >> 4) & 1) + ((lane >> 3) & 1)
                       : R == 4 ? 2 * ((lane >> 5) & 1) + ((lane >> 4) & 1)
                                : (lane >> 5) & 1;
    const float sc = a.scale[min(n0 + o_mine, a.n - 1)];
    auto row = [&](int m, const XSlice<KJ>& x) {
        float v[R];
#pragma unroll
        for (int o = 0; o < R; o++) {
            float acc = 0.f;
#pragma unroll
            for (int j = 0; j < KJ; j++) {
                const float xs[8] = {x.a[j].x, x.a[j].y, x.a[j].z, x.a[j].w, x.b[j].x, x.b[j].y, x.b[j].z, x.b[j].w};
#pragma unroll
                for (int i = 0; i < 8; i++) acc = __builtin_fmaf(w[o][j][i], xs[i], acc);
            }
            v[o] = acc;
        }
        const float sum = reduce_outputs<R>(v, lane) * sc;
        if ((lane & (kGroup - 1)) == 0 && n0 + o_mine < a.n) a.out[(int64_t)m * a.ldo + n0 + o_mine] = sum;
    };
    const int first = blockIdx.y * a.row_group;
    const int last = min(a.rows, first + a.row_group) - 1;
    XSlice<KJ> x0 = load_x<KJ, FULL>(a, first, lane);
    for (int m = first; m <= last; m += 2) {
        XSlice<KJ> x1 = load_x<KJ, FULL>(a, min(m + 1, last), lane);
        row(m, x0);
        if (m + 1 > last) break;
        x0 = load_x<KJ, FULL>(a, min(m + 2, last), lane);
        row(m + 1, x1);
    }
}

// ---- matrix-core form, for 8 or more rows -------------------------------------------------------
// The hidden rows are fp32 and v_mfma_f32_16x16x32_bf16 multiplies bf16, so each x is split exactly
// into three bf16 parts, x = h + m + l: h keeps the top 8 significand bits (truncation), m the next
// 8 of the remainder x - h (exact in fp32), l what is left (at most 8 bits: exact in bf16), exact
// whenever |x| >= 2^-110 or x = 0. A bf16 weight times a part is exact in fp32, so the matrix cores
// sum exact products: out = W h + W m + W l, with fp32 roundings only in the accumulation (a chain
// of at most 3 K / 32 + 2 matrix operations and NW wave partials per output; the test bound is that
// of K sequential fp32 additions). An int8 weight widens to bf16 exactly (|q| <= 127).
//
// Tile: a workgroup owns 16 TM outputs and all rows, 32 at a time; its NW waves split K in chunks
// of 64 (two 32-deep steps), chunk c to wave c % NW, and their 16 TM x 32 partial sums are added in
// LDS in wave order. MFMA operand layout (16x16x32): lane l supplies A[l % 16][8 (l / 16) + 0..7] and
// B[8 (l / 16) + 0..7][l % 16], and holds C[4 (l / 16) + i][l % 16], i = 0..3. Here A = W (outputs by
// k), B = x^T (k by rows), so lane l reads 8 consecutive k of one weight row and of one hidden row.
typedef __bf16 bf8 __attribute__((ext_vector_type(8)));

// three exact bf16 parts of 8 fp32 values. With NONFINITE, +-inf and NaN are their own high part (a
// NaN keeps a payload bit in the bf16 half) with zero remainders, so the products follow IEEE
// (inf w = +-inf, inf 0 = NaN, NaN w = NaN); without it such a value would turn into NaN parts.
template <bool NONFINITE>
__device__ __forceinline__ void split3(const f4& a, const f4& b, bf8& h, bf8& m, bf8& l) {
    const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
    uint32_t th[8], tm[8], tl[8];
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const uint32_t u = __float_as_uint(v[i]);
        float r1;
        if constexpr (NONFINITE) {
            const bool fin = (u & 0x7F800000u) != 0x7F800000u;
            th[i] = fin || !(u & 0x007FFFFFu) ? u & 0xFFFF0000u : u | 0x00400000u;
            r1 = fin ? v[i] - __uint_as_float(th[i]) : 0.0f;
        } else {
            th[i] = u & 0xFFFF0000u;
            r1 = v[i] - __uint_as_float(th[i]);
        }
        tm[i] = __float_as_uint(r1) & 0xFFFF0000u;
        tl[i] = __float_as_uint(r1 - __uint_as_float(tm[i]));
    }
    u4 ph, pm, pl;
#pragma unroll
    for (int i = 0; i < 4; i++) {  // high halves of elements 2i (low) and 2i + 1 (high)
        ph[i] = __builtin_amdgcn_perm(th[2 * i + 1], th[2 * i], 0x07060302u);
        pm[i] = __builtin_amdgcn_perm(tm[2 * i + 1], tm[2 * i], 0x07060302u);
        pl[i] = __builtin_amdgcn_perm(tl[2 * i + 1], tl[2 * i], 0x07060302u);
    }
    h = __builtin_bit_cast(bf8, ph);
    m = __builtin_bit_cast(bf8, pm);
    l = __builtin_bit_cast(bf8, pl);
}

// split3 with the non-finite handling only when the wave holds such a value (one class test per
// value; the rare case takes the longer form)
__device__ __forceinline__ void split3_any(const f4& a, const f4& b, bf8& h, bf8& m, bf8& l) {
    bool nf = false;
#pragma unroll
    for (int i = 0; i < 4; i++)
        nf |= __builtin_amdgcn_class(a[i], 0x207) | __builtin_amdgcn_class(b[i], 0x207);  // NaN, +-inf
    if (__ballot(nf))
        split3<true>(a, b, h, m, l);
    else
        split3<false>(a, b, h, m, l);
}

// 8 int8 weights (two dwords) as 8 bf16: the biased byte converted, 128 subtracted (exact), the
// high halves packed
__device__ __forceinline__ bf8 i8_to_bf16(uint32_t lo, uint32_t hi) {
    lo ^= 0x80808080u;
    hi ^= 0x80808080u;
    uint32_t f[8];
#pragma unroll
    for (int i = 0; i < 8; i++)
        f[i] = __float_as_uint((float)(((i < 4 ? lo : hi) >> (8 * (i & 3))) & 0xffu) - 128.0f);
    u4 p;
#pragma unroll
    for (int i = 0; i < 4; i++) p[i] = __builtin_amdgcn_perm(f[2 * i + 1], f[2 * i], 0x07060302u);
    return __builtin_bit_cast(bf8, p);
}

template <int TM, int NW, bool I8>
__global__ __launch_bounds__(64 * NW) void head_mfma_kernel(HeadArgs a) {
    __shared__ f4 part[NW][TM * 2][64];  // each wave's accumulators, per (output tile, row tile)
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int g = lane >> 4, c16 = lane & 15;
    const int n0 = blockIdx.x * 16 * TM;
    const int nchunks = (a.k + 63) / 64;
    for (int r0 = 0; r0 < a.rows; r0 += 32) {
        f4 acc[TM][2];
#pragma unroll
        for (int tm = 0; tm < TM; tm++)
#pragma unroll
            for (int tn = 0; tn < 2; tn++) acc[tm][tn] = f4{0.f, 0.f, 0.f, 0.f};
        for (int c = wv; c < nchunks; c += NW) {
            // every load of the chunk is issued before the first product: the weights of both steps
            // and output tiles, the hidden rows' slices of both steps and row tiles (lane l: 8
            // consecutive k from 64 c + 32 step + 8 (l / 16), weight row / hidden row l % 16 of the tile)
            typedef typename std::conditional<I8, u2, u4>::type WRaw;
            WRaw wr[2][TM];
            f4 xr[2][2][2];
            bool kin[2];
#pragma unroll
            for (int st = 0; st < 2; st++) {
                const int k = 64 * c + 32 * st + 8 * g;  // k % 8 == 0: the 8 are all inside or all past k
                kin[st] = k < a.k;
#pragma unroll
                for (int tm = 0; tm < TM; tm++) {
                    const int n = n0 + 16 * tm + c16;
                    const int64_t off = (int64_t)min(n, a.n - 1) * a.ldw + (kin[st] ? k : 0);
                    if constexpr (I8)
                        wr[st][tm] = *reinterpret_cast<const u2*>(a.q + off);
                    else
                        wr[st][tm] = __builtin_nontemporal_load(reinterpret_cast<const u4*>(a.w + off));
                }
#pragma unroll
                for (int tn = 0; tn < 2; tn++) {
                    const int r = r0 + 16 * tn + c16;
                    const float* px = a.x + (int64_t)min(r, a.rows - 1) * a.ldx + (kin[st] ? k : 0);
                    xr[st][tn][0] = *reinterpret_cast<const f4*>(px);
                    xr[st][tn][1] = *reinterpret_cast<const f4*>(px + 4);
                }
            }
#pragma unroll
            for (int st = 0; st < 2; st++) {
                bf8 wa[TM];
#pragma unroll
                for (int tm = 0; tm < TM; tm++) {
                    const bool in = kin[st] && n0 + 16 * tm + c16 < a.n;
                    if constexpr (I8)
                        wa[tm] = i8_to_bf16(in ? wr[st][tm].x : 0u, in ? wr[st][tm].y : 0u);
                    else
                        wa[tm] = __builtin_bit_cast(bf8, in ? wr[st][tm] : u4{0u, 0u, 0u, 0u});
                }
#pragma unroll
                for (int tn = 0; tn < 2; tn++) {
                    const bool in = kin[st] && r0 + 16 * tn + c16 < a.rows;
                    const f4 z = {0.f, 0.f, 0.f, 0.f};
                    bf8 h, m, l;
                    split3_any(in ? xr[st][tn][0] : z, in ? xr[st][tn][1] : z, h, m, l);
#pragma unroll
                    for (int tm = 0; tm < TM; tm++) {
                        acc[tm][tn] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wa[tm], h, acc[tm][tn], 0, 0, 0);
                        acc[tm][tn] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wa[tm], m, acc[tm][tn], 0, 0, 0);
                        acc[tm][tn] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wa[tm], l, acc[tm][tn], 0, 0, 0);
                    }
                }
            }
        }
#pragma unroll
        for (int tm = 0; tm < TM; tm++)
#pragma unroll
            for (int tn = 0; tn < 2; tn++) part[wv][2 * tm + tn][lane] = acc[tm][tn];
        __syncthreads();
        // (output, row) pairs of the tile, consecutive threads on consecutive outputs: the waves'
        // partials added in wave order, scaled (int8), stored
        for (int p = threadIdx.x; p < 16 * TM * 32; p += 64 * NW) {
            const int nl = p % (16 * TM), rl = p / (16 * TM);
            const int tm = nl / 16, mi = nl % 16, tn = rl / 16;
            const int l = 16 * (mi / 4) + rl % 16;
            float sum = 0.f;
#pragma unroll
            for (int w = 0; w < NW; w++) sum += part[w][2 * tm + tn][l][mi % 4];
            const int n = n0 + nl, r = r0 + rl;
            if (n < a.n && r < a.rows) {
                if constexpr (I8) sum *= a.scale[n];
                a.out[(int64_t)r * a.ldo + n] = sum;
            }
        }
        __syncthreads();  // the partials are read before the next row group writes them
    }
}

template <int TM, int NW>
hipError_t launch_mfma(const HeadArgs& a, hipStream_t stream) {
    const dim3 grid((a.n + 16 * TM - 1) / (16 * TM));
    if (a.q)
        hipLaunchKernelGGL((head_mfma_kernel<TM, NW, true>), grid, dim3(64 * NW), 0, stream, a);
    else
        hipLaunchKernelGGL((head_mfma_kernel<TM, NW, false>), grid, dim3(64 * NW), 0, stream, a);
    return hipGetLastError();
}

// FromBf16LinearInt8 for one output row per workgroup.
__global__ __launch_bounds__(kHT) void head_pack_i8_kernel(int k, const uint16_t* __restrict__ w, int64_t ldw,
                                                          int8_t* __restrict__ q, int64_t ldq, float* __restrict__ scale) {
    __shared__ float wmax[kHT / 64];
    const int n = blockIdx.x;
    const uint16_t* row = w + (int64_t)n * ldw;
    float amax = 0.0f;
    for (int i = threadIdx.x; i < k; i += kHT) amax = fmaxf(amax, fabsf(__uint_as_float((uint32_t)row[i] << 16)));
#pragma unroll
    for (int mask = 32; mask >= 1; mask /= 2) amax = fmaxf(amax, __shfl_xor(amax, mask));
    if ((threadIdx.x & 63) == 0) wmax[threadIdx.x >> 6] = amax;
    __syncthreads();
    amax = fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3]));
    const float scl = amax > 0.0f ? amax / 127.0f : 1.0f;  // correctly rounded fp32 divisions
    const float inv = 1.0f / scl;
    int8_t* qr = q + (int64_t)n * ldq;
    for (int i = threadIdx.x; i < k; i += kHT) {
        const float t = rintf(__uint_as_float((uint32_t)row[i] << 16) * inv);  // half to even, as MathF.Round
        // (int) then Math.Clamp, with .NET's saturating conversion: NaN (0 * inf, when 1 / scale
        // overflowed) gives 0, +-inf the clamp's ends; clamped in fp32 first, so the cast is exact
        qr[i] = (int8_t)(t != t ? 0 : (int)fminf(fmaxf(t, -127.0f), 127.0f));
    }
    if (threadIdx.x == 0) scale[n] = scl;
}

// Rows are split into groups, one grid row each, so that the launch has about 2048 waves for the
// chip's 1024 SIMDs; a group keeps at least two rows (the loads of one overlap the other's work).
// Every group reads the weight again, from the last-level cache after the first.
template <int KJ, int R>
hipError_t launch_kr(HeadArgs a, hipStream_t stream) {
    const int tiles = (a.n + (kHT / 64) * R - 1) / ((kHT / 64) * R);
    const int waves = tiles * (kHT / 64);
    const int groups = std::max(1, std::min(2048 / waves, a.rows / 2));
    a.row_group = (a.rows + groups - 1) / groups;
    const dim3 grid(tiles, (a.rows + a.row_group - 1) / a.row_group);
    if (a.q) {
        if (a.k == 512 * KJ)
            hipLaunchKernelGGL((head_i8_kernel<KJ, R, true>), grid, dim3(kHT), 0, stream, a);
        else
            hipLaunchKernelGGL((head_i8_kernel<KJ, R, false>), grid, dim3(kHT), 0, stream, a);
    } else if (a.k == 512 * KJ) {
        hipLaunchKernelGGL((head_kernel<KJ, R, true>), grid, dim3(kHT), 0, stream, a);
    } else {
        hipLaunchKernelGGL((head_kernel<KJ, R, false>), grid, dim3(kHT), 0, stream, a);
    }
    return hipGetLastError();
}

}  // namespace

hipError_t launch_head(const HeadArgs& a, hipStream_t stream) {
    if (a.rows <= 0 || a.n <= 0) return hipSuccess;
    // The matrix-core form for 8 to 32 rows and at least 2560 outputs (160 or more workgroups of
    // 16 outputs). Measured, 24 rows x 1024, matrix cores / VALU: 3072 outputs 6.8 / 7.9 us, 2048
    // outputs 6.8 / 6.4 us; 8 rows x 3072 5.4 / 6.1 us; 64 rows (two row groups in turn) 13.4 /
    // 12.6 us at 3072 outputs and 13.3 / 9.4 us at 2048.
    if (a.rows >= 8 && a.rows <= 32 && a.n >= 2560 && a.k >= 64) return launch_mfma<1, 16>(a, stream);
    // Outputs per wave: eight up to k = 1024 (four above, for registers); with one or two rows, two,
    // so that the single pass over the weight is spread over four times as many waves.
    const bool few = a.rows <= 2;
    switch ((a.k + 511) / 512) {
        case 1: return few ? launch_kr<1, 2>(a, stream) : launch_kr<1, 8>(a, stream);
        case 2: return few ? launch_kr<2, 2>(a, stream) : launch_kr<2, 8>(a, stream);
        case 3: return few ? launch_kr<3, 2>(a, stream) : launch_kr<3, 4>(a, stream);
        case 4: return few ? launch_kr<4, 2>(a, stream) : launch_kr<4, 4>(a, stream);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_head_pack_int8(int k, int n, const uint16_t* w, int64_t ldw, int8_t* q, int64_t ldq, float* scale,
                                 hipStream_t stream) {
    if (n <= 0 || k <= 0) return hipSuccess;
    hipLaunchKernelGGL(head_pack_i8_kernel, dim3(n), dim3(kHT), 0, stream, k, w, ldw, q, ldq, scale);
    return hipGetLastError();
}

}  // namespace vxs
