// vxs_history.hip — resident histories for batched generation.
//
// In continuous batching (src/Voxwerk/Talker/TalkerGenerator.cs:322-455) every active sequence
// owns a history of the codes it has sampled (Active.History, :304), penalised before each talker
// draw (:369) and grown by one id after it (:374). Here the histories stay in device memory, one
// fixed-capacity slot per sequence ([slots][cap] ids plus [slots] lengths), and this kernel runs
// after the sampler to append each row's id to its slot, so no history crosses PCIe per step.
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

}  // namespace

hipError_t launch_history_append(const AppendArgs& a, hipStream_t stream) {
    if (a.rows <= 0) return hipSuccess;
    const int blocks = a.done_flag ? 1 : std::min((a.rows + kAT - 1) / kAT, 1024);
    hipLaunchKernelGGL(history_append_kernel, dim3(blocks), dim3(kAT), 0, stream, a);
    return hipGetLastError();
}

}  // namespace vxs
