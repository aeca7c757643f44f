// vxs_embed.hip — embedding rows of sampled ids, the step after the sampler.
//
// The talker feeds each sampled code back through bf16 embedding tables (src/Voxwerk/Talker/
// TalkerModel.cs:100-131): CodecEmbedding / CodePredictorEmbedding write or add one widened table
// row, FrameEmbedding sums a frame's 16 codebook rows (codebook 0 from the talker table, 1..15
// from the code predictor's), and the talker step then adds a text embedding row
// (TalkerGenerator.cs:280-283, :435-439). bf16 -> fp32 widening is exact (the bits shifted left by 16,
// Bf16.cs:13), and the fp32 sums run in the reference's order with no contraction, so the rows are
// bit-identical to the reference's.
//
// Layout: one 256-thread workgroup per output row, each thread four consecutive entries per
// 1024-entry sweep (8-byte bf16 loads, 16-byte fp32 stores); the codes of a row are read once per
// workgroup. HBM-bound gathers of whole 2 KiB table rows; at the batch sizes of generation the
// launch dominates.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "vxs_internal.h"

namespace vxs {
namespace {

constexpr int kET = 256;

typedef float f4 __attribute__((ext_vector_type(4)));
typedef unsigned short us4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float widen(unsigned short b) { return __uint_as_float((uint32_t)b << 16); }

__device__ __forceinline__ f4 widen4(const uint16_t* p) {
    const us4 w = *reinterpret_cast<const us4*>(p);
    return f4{widen(w.x), widen(w.y), widen(w.z), widen(w.w)};
}

// Four fp32 entries (fewer at the end of a row); 16-byte accesses when the layout allows (vec).
__device__ __forceinline__ void store4(float* p, f4 v, int n, bool vec) {
    if (vec && n >= 4) {
        *reinterpret_cast<f4*>(p) = v;
        return;
    }
    if (n > 0) p[0] = v.x;
    if (n > 1) p[1] = v.y;
    if (n > 2) p[2] = v.z;
    if (n > 3) p[3] = v.w;
}

__device__ __forceinline__ f4 load4(const float* p, int n, bool vec) {
    if (vec && n >= 4) return *reinterpret_cast<const f4*>(p);
    f4 r{0.f, 0.f, 0.f, 0.f};
    if (n > 0) r.x = p[0];
    if (n > 1) r.y = p[1];
    if (n > 2) r.z = p[2];
    if (n > 3) r.w = p[3];
    return r;
}

__device__ __forceinline__ f4 gather4(const uint16_t* p, int n, bool vec) {
    if (vec && n >= 4) return widen4(p);
    f4 r{0.f, 0.f, 0.f, 0.f};
    if (n > 0) r.x = widen(p[0]);
    if (n > 1) r.y = widen(p[1]);
    if (n > 2) r.z = widen(p[2]);
    if (n > 3) r.w = widen(p[3]);
    return r;
}

// out[r] (+)= table[ids[r]] (CodecEmbedding / CodePredictorEmbedding).
__global__ __launch_bounds__(kET) void embed_kernel(EmbedArgs a) {
    const int r = blockIdx.x;
    const int id = a.ids[r];
    const bool ok = (unsigned)id < (unsigned)a.vocab;
    if (threadIdx.x == 0) a.status[r] = ok ? 0 : VXS_ERR_ID_OUT_OF_RANGE;
    if (!ok) return;  // the row is left as it was (the reference throws before writing)
    const uint16_t* src = a.table + (int64_t)id * a.hidden;
    float* dst = a.out + (int64_t)r * a.ld_out;
    const bool vec = a.vec;
    for (int i = threadIdx.x * 4; i < a.hidden; i += kET * 4) {
        const int n = a.hidden - i;
        const f4 e = gather4(src + i, n, vec);
        store4(dst + i, a.add ? load4(dst + i, n, vec) + e : e, n, vec);
    }
}

// out[r] = E0[c0] + E1[c1] + ... + E_{G-1}[c_{G-1}] (+ addend[r]), in that order (FrameEmbedding,
// then the talker step's text row).
__global__ __launch_bounds__(kET) void frame_embed_kernel(FrameEmbedArgs a) {
    const int r = blockIdx.x;
    const int32_t* codes = a.codes + (int64_t)r * a.ld_codes;
    auto code = [&](int g) { return codes[(int64_t)g * a.group_stride]; };
    bool ok = (unsigned)code(0) < (unsigned)a.vocab;
    for (int g = 1; g < a.groups; g++) ok = ok && (unsigned)code(g) < (unsigned)a.cp_vocab;
    if (threadIdx.x == 0) a.status[r] = ok ? 0 : VXS_ERR_ID_OUT_OF_RANGE;
    if (!ok) return;
    float* dst = a.out + (int64_t)r * a.ld_out;
    const float* add = a.addend ? a.addend + (int64_t)r * a.ld_addend : nullptr;
    const bool vec = a.vec;
    for (int i = threadIdx.x * 4; i < a.hidden; i += kET * 4) {
        const int n = a.hidden - i;
        f4 acc = gather4(a.codec_table + (int64_t)code(0) * a.hidden + i, n, vec);
        for (int g = 1; g < a.groups; g++)
            acc = acc + gather4(a.cp_tables + ((int64_t)(g - 1) * a.cp_vocab + code(g)) * a.hidden + i, n, vec);
        if (add) acc = acc + load4(add + i, n, vec);
        store4(dst + i, acc, n, vec);
    }
}

// The same for the talker's 16 codebooks with all codes read up front and every table row of a
// sweep in flight before the sums (the general loop waits on each gather in turn).
constexpr int kGroups = 16;
__global__ __launch_bounds__(kET) void frame_embed16_kernel(FrameEmbedArgs a) {
    const int r = blockIdx.x;
    const int32_t* codes = a.codes + (int64_t)r * a.ld_codes;
    int c[kGroups];
#pragma unroll
    for (int g = 0; g < kGroups; g++) c[g] = codes[(int64_t)g * a.group_stride];
    bool ok = (unsigned)c[0] < (unsigned)a.vocab;
#pragma unroll
    for (int g = 1; g < kGroups; g++) ok = ok && (unsigned)c[g] < (unsigned)a.cp_vocab;
    if (threadIdx.x == 0) a.status[r] = ok ? 0 : VXS_ERR_ID_OUT_OF_RANGE;
    if (!ok) return;
    float* dst = a.out + (int64_t)r * a.ld_out;
    const float* add = a.addend ? a.addend + (int64_t)r * a.ld_addend : nullptr;
    const bool vec = a.vec;
    for (int i = threadIdx.x * 4; i < a.hidden; i += kET * 4) {
        const int n = a.hidden - i;
        f4 e[kGroups];
        e[0] = gather4(a.codec_table + (int64_t)c[0] * a.hidden + i, n, vec);
#pragma unroll
        for (int g = 1; g < kGroups; g++)
            e[g] = gather4(a.cp_tables + ((int64_t)(g - 1) * a.cp_vocab + c[g]) * a.hidden + i, n, vec);
        const f4 t = add ? load4(add + i, n, vec) : f4{0.f, 0.f, 0.f, 0.f};
        f4 acc = e[0];
#pragma unroll
        for (int g = 1; g < kGroups; g++) acc = acc + e[g];
        if (add) acc = acc + t;
        store4(dst + i, acc, n, vec);
    }
}

}  // namespace

hipError_t launch_embed(const EmbedArgs& a, hipStream_t stream) {
    if (a.rows <= 0) return hipSuccess;
    hipLaunchKernelGGL(embed_kernel, dim3(a.rows), dim3(kET), 0, stream, a);
    return hipGetLastError();
}

hipError_t launch_frame_embed(const FrameEmbedArgs& a, hipStream_t stream) {
    if (a.rows <= 0) return hipSuccess;
    if (a.groups == kGroups)
        hipLaunchKernelGGL(frame_embed16_kernel, dim3(a.rows), dim3(kET), 0, stream, a);
    else
        hipLaunchKernelGGL(frame_embed_kernel, dim3(a.rows), dim3(kET), 0, stream, a);
    return hipGetLastError();
}

}  // namespace vxs
