// vxs_history.hip — the generators of resident histories, drawn in sequence.
//
// In continuous batching (src/Voxwerk/Talker/TalkerGenerator.cs:322-455) every active sequence owns
// a history of the codes it has sampled (Active.History, :304), penalised before each talker draw
// (:369) and grown by one id after it (:374), and two generators, new Random(seed) for the talker and
// new Random(seed + 1) for the code predictor (:345-346). A resident store keeps both in device
// memory, one slot per sequence; the sampling kernels read a row's slot and end its step themselves
// (put_id in vxs_internal.h: draw, append, slot check), so a batched stage is one launch. This file
// holds the one kernel left outside them: n successive NextDouble() of one generator
// (vxs_history_draw), for callers that want the uniforms themselves.
#include <hip/hip_runtime.h>

#include "vxs_internal.h"

namespace vxs {
namespace {

__global__ void draw_sequence_kernel(int32_t* st, int n, double* out) {
    if (threadIdx.x == 0)
        for (int k = 0; k < n; k++) {
            const RngStep t = rng_peek(st);
            rng_commit(st, t);
            out[k] = rng_double(t.v);
        }
}

}  // namespace

hipError_t launch_draw_sequence(int32_t* state, int n, double* out, hipStream_t stream) {
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(draw_sequence_kernel, dim3(1), dim3(64), 0, stream, state, n, out);
    return hipGetLastError();
}

}  // namespace vxs
