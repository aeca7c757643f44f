// vxs_history.hip — resident histories for batched generation.
//
// In continuous batching (src/Voxwerk/Talker/TalkerGenerator.cs:322-455) every active sequence
// owns a history of the codes it has sampled (Active.History, :304), penalised before each talker
// draw (:369) and grown by one id after it (:374). Here the histories stay in device memory, one
// fixed-capacity slot per sequence ([slots][cap] ids plus [slots] lengths), and this kernel runs
// after the sampler to append each row's id to its slot, so no history crosses PCIe per step.
// A slot also holds its sequence's two generators, new Random(seed) for the talker and
// new Random(seed + 1) for the code predictor (:345-346), so the uniforms can be drawn here too.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "vxs_internal.h"

namespace vxs {
namespace {

constexpr int kAT = 256;

__global__ __launch_bounds__(kAT) void history_append_kernel(AppendArgs a) {
    for (int r = blockIdx.x * kAT + threadIdx.x; r < a.rows; r += gridDim.x * kAT) {
        int id = a.out_ids[r];
        const int s = a.slot[r];
        if ((unsigned)s >= (unsigned)a.slots) {
            id = VXS_ERR_INVALID_ARG;  // the sampler read this row's history as empty
        } else if (a.append && id >= 0) {
            const int n = a.len[s];
            if ((unsigned)n >= (unsigned)a.cap) {
                id = VXS_ERR_HISTORY_FULL;
            } else {
                a.ids[(int64_t)s * a.cap + n] = id;
                a.len[s] = n + 1;
            }
        }
        a.out_ids[r] = id;
        if (a.host_ids) a.host_ids[r] = id;
    }
    if (a.done_flag) {  // one workgroup: every id is in host memory before the flag
        __threadfence_system();
        __syncthreads();
        if (threadIdx.x == 0) __hip_atomic_store(a.done_flag, a.done_seq, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
    }
}

// One NextDouble() of a .NET seeded Random (InternalSample() * (1.0 / int.MaxValue)) with C#'s
// wrapping int arithmetic; advances the state in place.
__device__ __forceinline__ double next_double(int32_t* st) {
    constexpr int32_t kMbig = 0x7FFFFFFF;
    int i = st[56] + 1;
    if (i >= 56) i = 1;
    int j = st[57] + 1;
    if (j >= 56) j = 1;
    int32_t v = (int32_t)((uint32_t)st[i] - (uint32_t)st[j]);
    if (v == kMbig) v--;
    if (v < 0) v = (int32_t)((uint32_t)v + (uint32_t)kMbig);
    st[i] = v;
    st[56] = i;
    st[57] = j;
    return (double)v * (1.0 / 2147483647.0);
}

__global__ __launch_bounds__(kAT) void draw_uniforms_kernel(DrawArgs a) {
    for (int r = blockIdx.x * kAT + threadIdx.x; r < a.rows; r += gridDim.x * kAT) {
        const int s = a.slot[r];
        const int sampled = a.params[(int64_t)r * a.params_stride].do_sample;
        double u = 0.0;
        if (sampled && (unsigned)s < (unsigned)a.slots) u = next_double(a.rng + ((int64_t)s * 2 + a.stream) * kRngWords);
        a.u[r] = u;
    }
}

__global__ void draw_sequence_kernel(int32_t* st, int n, double* out) {
    if (threadIdx.x == 0)
        for (int k = 0; k < n; k++) out[k] = next_double(st);
}

}  // namespace

hipError_t launch_draw_uniforms(const DrawArgs& a, hipStream_t stream) {
    if (a.rows <= 0) return hipSuccess;
    const int blocks = std::min((a.rows + kAT - 1) / kAT, 1024);
    hipLaunchKernelGGL(draw_uniforms_kernel, dim3(blocks), dim3(kAT), 0, stream, a);
    return hipGetLastError();
}

hipError_t launch_draw_sequence(int32_t* state, int n, double* out, hipStream_t stream) {
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(draw_sequence_kernel, dim3(1), dim3(64), 0, stream, state, n, out);
    return hipGetLastError();
}

hipError_t launch_history_append(const AppendArgs& a, hipStream_t stream) {
    if (a.rows <= 0) return hipSuccess;
    const int blocks = a.done_flag ? 1 : std::min((a.rows + kAT - 1) / kAT, 1024);
    hipLaunchKernelGGL(history_append_kernel, dim3(blocks), dim3(kAT), 0, stream, a);
    return hipGetLastError();
}

}  // namespace vxs
