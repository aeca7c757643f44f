// vxs_head.hip — the logit heads on the GPU, the step before the sampler.
//
// CodecHead and CodePredictorHead (src/Voxwerk/Talker/TalkerModel.cs:133-137) multiply a few fp32
// hidden rows by a bf16 weight (the checkpoint's [out, in] layout, WeightPrecision.BFloat16,
// DecoderStack.cs:7-15): out[r][n] = sum_k x[r][k] * W[n][k]. With the rows of a decode step
// (1-24) this is a GEMV bound by reading W once from HBM; the products stay fp32 (no MFMA, which
// would round x to bf16), and the logits stay in HBM for the sampler.
//
// Layout: a wave owns R = 8 consecutive outputs (4 when k > 1024); lane l holds W[n][k] for
// k = 512 j + 8 l + 0..7
// (one 16-byte load per output and j, 1 KiB contiguous per wave instruction), all of its rows in
// registers for the whole call. Per hidden row the lane loads its x slice (the next row's loads
// issued before the current row's products), forms 8 partial dots and reduces them across the
// wave by halving exchanges (xor 32, 16, 8: each lane keeps half of its partials and adds its
// partner's other half) and then plain butterflies (xor 4, 2, 1): with R = 8, lane l ends with
// output 4 b5 + 2 b4 + b3 of the wave, summed over all 64 lanes. The fp32 sum order is this kernel's own;
// it differs from the reference's AVX-512 order by rounding only (bounded by K 2^-24 sum |x w|).
#include <hip/hip_runtime.h>

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

// One lane's slice of hidden row m: x[m][512 j + 8 lane + 0..7] for each j (zero past k).
template <int KJ>
struct XSlice {
    f4 a[KJ], b[KJ];
};

template <int KJ>
__device__ __forceinline__ XSlice<KJ> load_x(const HeadArgs& h, int m, int lane) {
    XSlice<KJ> r;
#pragma unroll
    for (int j = 0; j < KJ; j++) {
        const int k = 512 * j + 8 * lane;
        const bool in = k < h.k;
        const float* p = h.x + (int64_t)m * h.ldx + (in ? k : 0);
        const f4 a = *reinterpret_cast<const f4*>(p);
        const f4 b = *reinterpret_cast<const f4*>(p + 4);
        r.a[j] = in ? a : f4{0.f, 0.f, 0.f, 0.f};
        r.b[j] = in ? b : f4{0.f, 0.f, 0.f, 0.f};
    }
    return r;
}

// R outputs per wave (a power of two <= 8), KJ slices of 8 per lane (k <= 512 KJ).
template <int KJ, int R>
__global__ __launch_bounds__(kHT) void head_kernel(HeadArgs a) {
    constexpr int kSteps = R == 8 ? 3 : R == 4 ? 2 : R == 2 ? 1 : 0;  // halving exchanges
    constexpr int kGroup = 64 >> kSteps;                                // lanes sharing an output after them
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
            const bool in = n0 + o < a.n && k < a.k;
            // every lane loads from inside W (a clamped address) and zeroes what lies outside
            const uint16_t* p = a.w + (int64_t)min(n0 + o, a.n - 1) * a.ldw + (k < a.k ? k : 0);
            const u4 v = __builtin_nontemporal_load(reinterpret_cast<const u4*>(p));
            w[o][j] = in ? v : u4{0u, 0u, 0u, 0u};
        }

    int o_mine = 0;  // output this lane holds after the halving exchanges
#pragma unroll
    for (int s = 0; s < kSteps; s++) o_mine |= ((lane >> (5 - s)) & 1) << (kSteps - 1 - s);
    XSlice<KJ> x = load_x<KJ>(a, 0, lane);
    for (int m = 0; m < a.rows; m++) {
        const XSlice<KJ> y = load_x<KJ>(a, m + 1 < a.rows ? m + 1 : m, lane);  // the next row, in flight
        // the widening is redone per row: kept packed, the weights take half the registers
#pragma unroll
        for (int o = 0; o < R; o++)
#pragma unroll
            for (int j = 0; j < KJ; j++) asm volatile("" : "+v"(w[o][j]));
        float v[R];
#pragma unroll
        for (int o = 0; o < R; o++) {
            float acc = 0.f;
#pragma unroll
            for (int j = 0; j < KJ; j++) acc = dot8(w[o][j], x.a[j], x.b[j], acc);
            v[o] = acc;
        }
        // halving exchanges over lane bits 5, 4, ...: keep the half of the outputs the bit selects
#pragma unroll
        for (int s = 0, half = R / 2; s < kSteps; s++, half /= 2) {
            const int mask = 32 >> s;
            const bool bit = (lane & mask) != 0;
#pragma unroll
            for (int i = 0; i < half; i++) {
                const float send = bit ? v[i] : v[i + half];
                const float keep = bit ? v[i + half] : v[i];
                v[i] = keep + __shfl_xor(send, mask);
            }
        }
        float sum = v[0];
#pragma unroll
        for (int mask = kGroup / 2; mask >= 1; mask /= 2) sum += __shfl_xor(sum, mask);
        if ((lane & (kGroup - 1)) == 0 && n0 + o_mine < a.n) a.out[(int64_t)m * a.ldo + n0 + o_mine] = sum;
        x = y;
    }
}

}  // namespace

hipError_t launch_head(const HeadArgs& a, hipStream_t stream) {
    if (a.rows <= 0 || a.n <= 0) return hipSuccess;
    const int kj = (a.k + 511) / 512;
    auto grid = [&](int r) { return dim3((a.n + (kHT / 64) * r - 1) / ((kHT / 64) * r)); };
    switch (kj) {  // eight outputs per wave up to k = 1024, four above (register budget)
        case 1: hipLaunchKernelGGL((head_kernel<1, 8>), grid(8), dim3(kHT), 0, stream, a); break;
        case 2: hipLaunchKernelGGL((head_kernel<2, 8>), grid(8), dim3(kHT), 0, stream, a); break;
        case 3: hipLaunchKernelGGL((head_kernel<3, 4>), grid(4), dim3(kHT), 0, stream, a); break;
        case 4: hipLaunchKernelGGL((head_kernel<4, 4>), grid(4), dim3(kHT), 0, stream, a); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace vxs
