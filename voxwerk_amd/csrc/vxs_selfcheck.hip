// vxs_selfcheck.hip — exhaustive check of the sampler's fp32 exponential on the device it runs on.
//
// The one-wave path ranks top-p candidates by their nucleus masses instead of their logits. That
// order equals the reference's (logit, index) order only if exp_neg is monotone non-decreasing,
// which depends on the hardware exp2 instruction. This program evaluates exp_neg on every float d
// in [-128, 0] (about 1.1e9 values), in increasing order per chunk, and reports the largest step
// back (in units of the result's last place) and the largest error against the double-precision
// exp, also in ulps. Output: one JSON line. Exit status 0 when the run completed.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>

#include "vxs_device.h"

namespace {

constexpr uint32_t kChunk = 4096;   // floats per thread, walked with increasing d
constexpr uint32_t kOverlap = 64;   // each chunk starts this many values early to see its left edge

__global__ void check(uint32_t n, uint32_t* step_back, float* err_ulp) {
    const uint32_t t = blockIdx.x * blockDim.x + threadIdx.x;
    const uint64_t b0 = (uint64_t)t * kChunk;
    if (b0 >= n) return;
    const uint64_t b1 = b0 + kChunk < n ? b0 + kChunk : n;
    uint32_t run_max = 0, worst = 0;
    float emax = 0.0f;
    for (uint64_t k = b0 >= kOverlap ? b0 - kOverlap : 0; k < b1; k++) {
        // k = 0 is d = -128 (bits 0xc3000000); k = n - 1 is d = -0 (bits 0x80000000)
        const float d = __uint_as_float(0x80000000u + (uint32_t)(n - 1 - k));
        const uint32_t qb = __float_as_uint(vxs::dev::exp_neg(d));
        if (k >= b0) {
            if (run_max > qb && run_max - qb > worst) worst = run_max - qb;
            const double e = exp((double)d);
            if (e >= 1e-37) {  // normal results only: ulps below are not comparable
                const float ef = (float)e;
                const double ulp = (double)(__uint_as_float(__float_as_uint(ef) + 1) - ef);
                const float er = (float)(fabs((double)__uint_as_float(qb) - e) / ulp);
                emax = er > emax ? er : emax;
            }
        }
        run_max = qb > run_max ? qb : run_max;
    }
    step_back[t] = worst;
    err_ulp[t] = emax;
}

bool ok(hipError_t e, const char* what) {
    if (e == hipSuccess) return true;
    fprintf(stderr, "vxs_selfcheck: %s: %s\n", what, hipGetErrorString(e));
    return false;
}

}  // namespace

int main() {
    const uint32_t n = 0x43000000u + 1;  // |d| bits from 0 to those of 128.0
    const uint32_t threads = (n + kChunk - 1) / kChunk;
    uint32_t* d_step = nullptr;
    float* d_err = nullptr;
    if (!ok(hipMalloc(&d_step, threads * sizeof(uint32_t)), "hipMalloc") ||
        !ok(hipMalloc(&d_err, threads * sizeof(float)), "hipMalloc"))
        return 1;
    hipLaunchKernelGGL(check, dim3((threads + 255) / 256), dim3(256), 0, 0, n, d_step, d_err);
    if (!ok(hipGetLastError(), "launch") || !ok(hipDeviceSynchronize(), "kernel")) return 1;
    uint32_t* step = (uint32_t*)malloc(threads * sizeof(uint32_t));
    float* err = (float*)malloc(threads * sizeof(float));
    if (!step || !err) return 1;
    if (!ok(hipMemcpy(step, d_step, threads * sizeof(uint32_t), hipMemcpyDeviceToHost), "copy") ||
        !ok(hipMemcpy(err, d_err, threads * sizeof(float), hipMemcpyDeviceToHost), "copy"))
        return 1;
    uint32_t worst = 0;
    uint64_t chunks_with_steps = 0;
    float emax = 0.0f;
    for (uint32_t i = 0; i < threads; i++) {
        worst = step[i] > worst ? step[i] : worst;
        chunks_with_steps += step[i] != 0;
        emax = err[i] > emax ? err[i] : emax;
    }
    printf("{\"values\": %u, \"max_step_back_ulp\": %u, \"chunks_with_step_back\": %llu, \"max_err_ulp\": %.4f}\n", n,
           worst, (unsigned long long)chunks_with_steps, emax);
    free(step);
    free(err);
    return ok(hipFree(d_step), "hipFree") && ok(hipFree(d_err), "hipFree") ? 0 : 1;
}
