// vxs_selfcheck.hip — exhaustive check of the sampler's fp32 exponentials on the device it runs on.
//
// The one-wave path ranks top-p candidates by their nucleus masses instead of their logits. That
// order equals the reference's (logit, index) order only if the mass function is monotone
// non-decreasing, which depends on the hardware exp2 instruction. This program evaluates both
// exponentials, nucleus_exp (the masses of vocabularies up to 8192) and exp_neg (the streaming
// kernel's), on every float d in [-128, 0] (about 1.1e9 values), in increasing order per chunk, and
// reports for each the largest step back (in units of the result's last place) and the error
// against the double-precision exp: exp_neg's in ulps, nucleus_exp's as the largest relative error
// and the largest excess of the relative error over the bound's |d| term (|d| * 7.4e-8).
// Output: one JSON line. Exit status 0 when the run completed.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>

#include "vxs_device.h"

namespace {

constexpr uint32_t kChunk = 4096;   // floats per thread, walked with increasing d
constexpr uint32_t kOverlap = 64;   // each chunk starts this many values early to see its left edge

constexpr double kDTerm = 7.4e-8;  // the |d| coefficient of nucleus_exp's relative error bound

__global__ void check(uint32_t n, uint32_t* step_back, float* err_ulp, uint32_t* nstep_back, double* nrel,
                      double* nexcess) {
    const uint32_t t = blockIdx.x * blockDim.x + threadIdx.x;
    const uint64_t b0 = (uint64_t)t * kChunk;
    if (b0 >= n) return;
    const uint64_t b1 = b0 + kChunk < n ? b0 + kChunk : n;
    uint32_t run_max = 0, worst = 0, nrun_max = 0, nworst = 0;
    float emax = 0.0f;
    double rmax = 0.0, xmax = -1.0;
    for (uint64_t k = b0 >= kOverlap ? b0 - kOverlap : 0; k < b1; k++) {
        // k = 0 is d = -128 (bits 0xc3000000); k = n - 1 is d = -0 (bits 0x80000000)
        const float d = __uint_as_float(0x80000000u + (uint32_t)(n - 1 - k));
        const uint32_t qb = __float_as_uint(vxs::dev::exp_neg(d));
        const uint32_t nb = __float_as_uint(vxs::dev::nucleus_exp(d));
        if (k >= b0) {
            if (run_max > qb && run_max - qb > worst) worst = run_max - qb;
            if (nrun_max > nb && nrun_max - nb > nworst) nworst = nrun_max - nb;
            const double e = exp((double)d);
            if (e >= 1e-37) {  // normal results only: ulps below are not comparable
                const float ef = (float)e;
                const double ulp = (double)(__uint_as_float(__float_as_uint(ef) + 1) - ef);
                const float er = (float)(fabs((double)__uint_as_float(qb) - e) / ulp);
                emax = er > emax ? er : emax;
                const double rel = fabs((double)__uint_as_float(nb) - e) / e;
                rmax = rel > rmax ? rel : rmax;
                const double ex = rel - kDTerm * fabs((double)d);
                xmax = ex > xmax ? ex : xmax;
            }
        }
        run_max = qb > run_max ? qb : run_max;
        nrun_max = nb > nrun_max ? nb : nrun_max;
    }
    step_back[t] = worst;
    err_ulp[t] = emax;
    nstep_back[t] = nworst;
    nrel[t] = rmax;
    nexcess[t] = xmax;
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
    uint32_t *d_step = nullptr, *d_nstep = nullptr;
    float* d_err = nullptr;
    double *d_nrel = nullptr, *d_nex = nullptr;
    if (!ok(hipMalloc(&d_step, threads * sizeof(uint32_t)), "hipMalloc") ||
        !ok(hipMalloc(&d_err, threads * sizeof(float)), "hipMalloc") ||
        !ok(hipMalloc(&d_nstep, threads * sizeof(uint32_t)), "hipMalloc") ||
        !ok(hipMalloc(&d_nrel, threads * sizeof(double)), "hipMalloc") ||
        !ok(hipMalloc(&d_nex, threads * sizeof(double)), "hipMalloc"))
        return 1;
    hipLaunchKernelGGL(check, dim3((threads + 255) / 256), dim3(256), 0, 0, n, d_step, d_err, d_nstep, d_nrel, d_nex);
    if (!ok(hipGetLastError(), "launch") || !ok(hipDeviceSynchronize(), "kernel")) return 1;
    uint32_t* step = (uint32_t*)malloc(threads * sizeof(uint32_t));
    uint32_t* nstep = (uint32_t*)malloc(threads * sizeof(uint32_t));
    float* err = (float*)malloc(threads * sizeof(float));
    double* nrel = (double*)malloc(threads * sizeof(double));
    double* nex = (double*)malloc(threads * sizeof(double));
    if (!step || !err || !nstep || !nrel || !nex) return 1;
    if (!ok(hipMemcpy(step, d_step, threads * sizeof(uint32_t), hipMemcpyDeviceToHost), "copy") ||
        !ok(hipMemcpy(err, d_err, threads * sizeof(float), hipMemcpyDeviceToHost), "copy") ||
        !ok(hipMemcpy(nstep, d_nstep, threads * sizeof(uint32_t), hipMemcpyDeviceToHost), "copy") ||
        !ok(hipMemcpy(nrel, d_nrel, threads * sizeof(double), hipMemcpyDeviceToHost), "copy") ||
        !ok(hipMemcpy(nex, d_nex, threads * sizeof(double), hipMemcpyDeviceToHost), "copy"))
        return 1;
    uint32_t worst = 0, nworst = 0;
    uint64_t chunks_with_steps = 0;
    float emax = 0.0f;
    double rmax = 0.0, xmax = -1.0;
    for (uint32_t i = 0; i < threads; i++) {
        worst = step[i] > worst ? step[i] : worst;
        nworst = nstep[i] > nworst ? nstep[i] : nworst;
        chunks_with_steps += step[i] != 0;
        emax = err[i] > emax ? err[i] : emax;
        rmax = nrel[i] > rmax ? nrel[i] : rmax;
        xmax = nex[i] > xmax ? nex[i] : xmax;
    }
    printf("{\"values\": %u, \"max_step_back_ulp\": %u, \"chunks_with_step_back\": %llu, \"max_err_ulp\": %.4f, "
           "\"nucleus_max_step_back_ulp\": %u, \"nucleus_max_rel_err\": %.4e, \"nucleus_max_excess\": %.4e}\n",
           n, worst, (unsigned long long)chunks_with_steps, emax, nworst, rmax, xmax);
    free(step);
    free(err);
    free(nstep);
    free(nrel);
    free(nex);
    return ok(hipFree(d_step), "hipFree") && ok(hipFree(d_err), "hipFree") && ok(hipFree(d_nstep), "hipFree") &&
                   ok(hipFree(d_nrel), "hipFree") && ok(hipFree(d_nex), "hipFree")
               ? 0
               : 1;
}
