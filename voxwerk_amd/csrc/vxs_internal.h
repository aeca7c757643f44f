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
    int path;            // kPathBlock or kPathQuad
    // kPathQuad: rows the one-wave path hands back, appended by it and sampled by a second
    // kernel. Calls alternate between two counters: this call appends at *defer_count, and its
    // second kernel zeroes *defer_next, the counter of the following call.
    int32_t* defer_list;  // [rows]
    int32_t* defer_count;
    int32_t* defer_next;
    // Host-visible completion for small host calls (one workgroup per row): after its row, every
    // workgroup counts itself in *done_count (device memory, zero between calls); the last one
    // resets the count and stores done_seq to *done_flag (pinned host memory), which the host
    // polls instead of synchronising the stream. Unused when done_flag is null.
    int32_t* done_count;
    int32_t* done_flag;
    int32_t done_seq;
};

enum : int {
    kPathBlock = 0,  // one 256-thread workgroup per row
    kPathQuad = 1,   // one wave per row first, four rows per workgroup (vocab <= kWaveMaxVocab)
};

// Largest vocabulary handled by the row-resident kernels (a row stays in VGPRs).
constexpr int kRowResidentMaxVocab = 8192;
// Largest vocabulary of the one-wave-per-row fast path (vxs_wave.h).
constexpr int kWaveMaxVocab = 3072;
// Largest vocabulary of the streaming kernel (vxs_wide.hip); its history bitmap lives in LDS.
constexpr int kWideMaxVocab = 1 << 19;

// Enqueue the sampler on `stream`. Returns hipSuccess or the launch error.
hipError_t launch_sample(const SampleArgs& a, hipStream_t stream);
hipError_t launch_sample_wide(const SampleArgs& a, hipStream_t stream);

}  // namespace vxs
