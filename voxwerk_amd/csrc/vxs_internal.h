// vxs_internal.h — shared declarations between the HIP kernels and the C-ABI layer.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/vxs_sampler.h"

namespace vxs {

// Kernel-side flags (not part of the public ABI).
enum : uint32_t {
    KF_STOP_AFTER_PENALTY = 1u,  // apply penalty (+ write-back) only: ApplyRepetitionPenalty
};

struct SampleArgs {
    int rows;
    int vocab;
    int64_t ld;
    const float* logits;
    const int32_t* hist_off;
    const int32_t* hist_ids;
    const vxs_params* params;
    int params_stride;
    const double* u;
    int32_t* out_ids;
    float* out_logits;   // optional [rows][vocab]
    double* out_probs;   // optional [rows][vocab]
    uint32_t kflags;
};

// Largest vocabulary handled by the row-resident kernel (one workgroup keeps a row in VGPRs).
constexpr int kRowResidentMaxVocab = 8192;

// Enqueue the sampler on `stream`. Returns hipSuccess or the launch error.
hipError_t launch_sample(const SampleArgs& a, hipStream_t stream);

}  // namespace vxs
