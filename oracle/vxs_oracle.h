/* vxs_oracle.h — CPU restatement of voxwerk's sampler. TEST INFRASTRUCTURE ONLY (see vxs_oracle.c). */
#ifndef VXS_ORACLE_H
#define VXS_ORACLE_H

#include <stdint.h>

#include "../include/vxs_sampler.h"

#ifdef __cplusplus
extern "C" {
#endif

#define VXS_ORACLE_TOPK_APPLIED 1
#define VXS_ORACLE_TOPP_APPLIED 2

/* Per-row diagnostics used to classify GPU/oracle id differences. */
typedef struct vxs_oracle_info {
    double draw_margin;   /* min |u - CDF edge| around the drawn id (inf if greedy)          */
    double topp_margin;   /* min |cum - thr| around the top-p cutoff (inf if top-p inactive) */
    int32_t n_candidates; /* entries with p > 0 after top-k                                  */
    int32_t n_kept;       /* entries with p > 0 after top-p                                  */
    float kth;            /* top-k threshold when applied, else -inf                         */
    int32_t flags;        /* VXS_ORACLE_* bits                                               */
} vxs_oracle_info;

int vxs_oracle_argmax(int n, const float* x);

/* Same argument meaning as vxs_sample (include/vxs_sampler.h); `threads` splits rows statically. */
int vxs_oracle_sample(int rows, int vocab, const float* logits, int64_t ld, const int32_t* hist_off,
                      const int32_t* hist_ids, const vxs_params* params, int params_stride,
                      const double* u, int32_t* out_ids, float* out_logits, double* out_probs,
                      vxs_oracle_info* info, int threads);

int vxs_oracle_apply_penalty(int rows, int vocab, float* logits, int64_t ld, const int32_t* hist_off,
                             const int32_t* hist_ids, float penalty);

/* .NET's seeded System.Random (vxs_oracle_random.c): the 56-entry table and its two cursors. */
typedef struct vxs_oracle_random {
    int32_t table[56];
    int next, nextp;
} vxs_oracle_random;

void vxs_oracle_random_seed(vxs_oracle_random* g, int32_t seed);    /* new Random(seed)      */
int32_t vxs_oracle_random_sample(vxs_oracle_random* g);              /* InternalSample()/Next() */
double vxs_oracle_random_next_double(vxs_oracle_random* g);          /* NextDouble()          */
/* The first n draws of new Random(seed): Next() values into samples and NextDouble() values into
 * doubles (either may be NULL). */
int vxs_oracle_random_stream(int32_t seed, int64_t n, int32_t* samples, double* doubles);

#ifdef __cplusplus
}
#endif

#endif
