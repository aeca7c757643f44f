/*
 * vxs_oracle.c — CPU restatement of voxwerk's token sampler. TEST INFRASTRUCTURE ONLY.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load this file's
 * library, and only as the checker / the timed CPU baseline. It is never part of the product
 * path (the product is the HIP library under voxwerk_amd/).
 *
 * It restates, scalar and in the reference's evaluation order:
 *   Sampler.ApplyRepetitionPenalty  src/Voxwerk/Talker/Sampler.cs:25-33
 *   suppression + min-new-tokens    src/Voxwerk/Talker/TalkerGenerator.cs:247-248 (:371-372)
 *   Sampler.Select                  src/Voxwerk/Talker/Sampler.cs:35-88
 *   Sampler.ArgMax                  src/Voxwerk/Talker/Sampler.cs:90-95
 * Build with -O2 -ffp-contract=off and without fast-math: every float op below is one IEEE
 * binary32 operation and every double op one binary64 operation, as RyuJIT emits them.
 *
 * How each step is pinned (checks live in tests/test_oracle.py):
 *   penalty    — HF RepetitionPenaltyLogitsProcessor on CPU torch (same formula), order and
 *                duplicate invariance, rho = 1 identity;
 *   top-k      — HF TopKLogitsWarper masks, brute-force k-th order statistic, k=1 == argmax;
 *   softmax    — closed form, sum to 1;
 *   top-p      — brute force on tiny rows, p -> 0 keeps the highest-index maximum, HF
 *                TopPLogitsWarper away from ties/boundaries;
 *   draw       — u = 0 picks the first kept id, uniform rows pick kept[floor(u*m)], chi-square;
 *   a second, independent numpy restatement (oracle/sampler_np.py) must agree bit for bit.
 * The .NET BCL parts (Math.Exp last ulp, Enumerable.Sum order, OrderBy stability) cannot be
 * run here (no .NET runtime): those stay "parity unpinned" beyond the documented semantics.
 */
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "../include/vxs_sampler.h"
#include "vxs_oracle.h"

/* Sampler.ApplyRepetitionPenalty, Sampler.cs:25-33. `seen` has vocab bytes of scratch. */
static int penalty_row(int vocab, float* x, const int32_t* hist, int64_t nhist, float penalty,
                       unsigned char* seen) {
    if (penalty == 1.0f) return VXS_OK; /* Sampler.cs:27 */
    memset(seen, 0, (size_t)vocab);
    for (int64_t h = 0; h < nhist; h++) { /* foreach id in history.Distinct() — :28 */
        int32_t id = hist[h];
        if (id < 0 || id >= vocab) return VXS_ERR_ID_OUT_OF_RANGE; /* Span bounds check, :30 */
        if (seen[id]) continue;
        seen[id] = 1;
        float s = x[id];                                 /* :30 */
        x[id] = s < 0 ? s * penalty : s / penalty;       /* :31 */
    }
    return VXS_OK;
}

/* Suppression, TalkerGenerator.cs:247-248: [begin,end) except keep -> -inf; then ban -> -inf. */
static void suppress_row(int vocab, float* x, const vxs_params* p) {
    int b = p->supp_begin < 0 ? 0 : p->supp_begin;
    int e = p->supp_end > vocab ? vocab : p->supp_end;
    for (int i = b; i < e; i++)
        if (i != p->keep_id) x[i] = -INFINITY;
    if (p->ban_id >= 0 && p->ban_id < vocab) x[p->ban_id] = -INFINITY;
}

/* Sampler.ArgMax, Sampler.cs:90-95: first index of the maximum (strict >). */
int vxs_oracle_argmax(int n, const float* x) {
    int best = 0;
    for (int i = 1; i < n; i++)
        if (x[i] > x[best]) best = i;
    return best;
}

/* Array.Sort(float[]) order for Sampler.cs:46 (NaN would sort first; rows with NaN are rejected). */
static int cmp_float(const void* a, const void* b) {
    float fa = *(const float*)a, fb = *(const float*)b;
    return (fa > fb) - (fa < fb);
}

/* Enumerable.Range(0,n).OrderBy(i => probs[i]) (Sampler.cs:65): stable ascending, so ties keep
 * index order. Comparer<double>.Default orders NaN below every number. */
typedef struct {
    double p;
    int32_t i;
} pidx;

static int cmp_pidx(const void* a, const void* b) {
    const pidx* x = (const pidx*)a;
    const pidx* y = (const pidx*)b;
    int xn = isnan(x->p), yn = isnan(y->p);
    if (xn || yn) {
        if (xn && !yn) return -1;
        if (!xn && yn) return 1;
    } else {
        if (x->p < y->p) return -1;
        if (x->p > y->p) return 1;
    }
    return (x->i > y->i) - (x->i < y->i);
}

static double mind(double a, double b) { return a < b ? a : b; }

/*
 * One row. x is modified in place exactly as the C# caller's span is. probs (n doubles) is
 * always written when sampling. Scratch: ws_f (n floats), ws_pi (n pidx), seen (n bytes).
 */
static int sample_row(int n, float* x, const int32_t* hist, int64_t nhist, const vxs_params* p,
                      double u, int32_t* out_id, double* probs, vxs_oracle_info* info, float* ws_f,
                      pidx* ws_pi, unsigned char* seen) {
    if (info) {
        info->draw_margin = INFINITY;
        info->topp_margin = INFINITY;
        info->n_candidates = 0;
        info->n_kept = 0;
        info->kth = -INFINITY;
        info->flags = 0;
    }
    int rc = penalty_row(n, x, hist, nhist, p->rep_penalty, seen);
    if (rc != VXS_OK) return rc;
    suppress_row(n, x, p);

    if (!p->do_sample) { /* Sampler.cs:37 — greedy, no temperature, no draw */
        for (int i = 0; i < n; i++) /* the ABI rejects NaN (outside the C# contract) */
            if (isnan(x[i])) return VXS_ERR_NONFINITE;
        *out_id = vxs_oracle_argmax(n, x);
        return VXS_OK;
    }

    float invT = 1.0f / p->temperature; /* Sampler.cs:39 */
    for (int i = 0; i < n; i++) x[i] *= invT; /* :40 */
    for (int i = 0; i < n; i++) /* the ABI rejects NaN / +inf (outside the C# contract) */
        if (isnan(x[i]) || x[i] == INFINITY) return VXS_ERR_NONFINITE;

    if (p->top_k > 0 && p->top_k < n) { /* Sampler.cs:42-49 */
        memcpy(ws_f, x, (size_t)n * sizeof(float));
        qsort(ws_f, (size_t)n, sizeof(float), cmp_float);
        float kth = ws_f[n - p->top_k];
        for (int i = 0; i < n; i++)
            if (x[i] < kth) x[i] = -INFINITY;
        if (info) {
            info->kth = kth;
            info->flags |= VXS_ORACLE_TOPK_APPLIED;
        }
    }

    float max = -INFINITY; /* Sampler.cs:51-52 */
    for (int i = 0; i < n; i++) max = x[i] > max ? x[i] : max;
    double sum = 0; /* :54-59, sequential in index order */
    for (int i = 0; i < n; i++) {
        probs[i] = x[i] == -INFINITY ? 0.0 : exp((double)(float)(x[i] - max));
        sum += probs[i];
    }
    for (int i = 0; i < n; i++) probs[i] /= sum; /* :60 */
    if (info)
        for (int i = 0; i < n; i++) info->n_candidates += probs[i] > 0;

    if (p->top_p < 1.0f) { /* Sampler.cs:62-75 */
        for (int i = 0; i < n; i++) {
            ws_pi[i].p = probs[i];
            ws_pi[i].i = i;
        }
        qsort(ws_pi, (size_t)n, sizeof(pidx), cmp_pidx);
        double thr = (double)(1.0f - p->top_p); /* C#: int - float is evaluated in float */
        double cum = 0;
        int broke = 0;
        for (int j = 0; j < n - 1; j++) {
            double prev = cum;
            cum += probs[ws_pi[j].i];
            if (cum <= thr) {
                probs[ws_pi[j].i] = 0;
            } else {
                if (info) info->topp_margin = mind(cum - thr, thr - prev);
                broke = 1;
                break;
            }
        }
        if (!broke && info) info->topp_margin = thr - cum;
        sum = 0; /* probs.Sum(): sequential */
        for (int i = 0; i < n; i++) sum += probs[i];
        for (int i = 0; i < n; i++) probs[i] /= sum;
        if (info) info->flags |= VXS_ORACLE_TOPP_APPLIED;
    }
    if (info)
        for (int i = 0; i < n; i++) info->n_kept += probs[i] > 0;

    double r = u; /* Sampler.cs:77-87 */
    double acc = 0;
    int last = 0;
    for (int i = 0; i < n; i++) {
        if (probs[i] <= 0) continue;
        double prev = acc;
        acc += probs[i];
        last = i;
        if (r < acc) {
            if (info) info->draw_margin = mind(acc - r, r - prev);
            *out_id = i;
            return VXS_OK;
        }
    }
    if (info) info->draw_margin = isnan(acc) ? INFINITY : r - acc;
    *out_id = last;
    return VXS_OK;
}

typedef struct {
    int row0, row1, vocab;
    const float* logits;
    int64_t ld;
    const int32_t* hist_off;
    const int32_t* hist_ids;
    const vxs_params* params;
    int params_stride;
    const double* u;
    int32_t* out_ids;
    float* out_logits;
    double* out_probs;
    vxs_oracle_info* info;
    int rc;
} batch_job;

static void* run_rows(void* arg) {
    batch_job* j = (batch_job*)arg;
    int n = j->vocab;
    float* x = (float*)malloc((size_t)n * sizeof(float));
    float* wsf = (float*)malloc((size_t)n * sizeof(float));
    pidx* wsp = (pidx*)malloc((size_t)n * sizeof(pidx));
    unsigned char* seen = (unsigned char*)malloc((size_t)n);
    double* probs = (double*)malloc((size_t)n * sizeof(double));
    j->rc = VXS_OK;
    if (!x || !wsf || !wsp || !seen || !probs) {
        j->rc = VXS_ERR_INVALID_ARG;
        goto done;
    }
    for (int r = j->row0; r < j->row1; r++) {
        memcpy(x, j->logits + (int64_t)r * j->ld, (size_t)n * sizeof(float));
        const int32_t* h = NULL;
        int64_t nh = 0;
        if (j->hist_off) {
            h = j->hist_ids + j->hist_off[r];
            nh = (int64_t)j->hist_off[r + 1] - j->hist_off[r];
        }
        const vxs_params* p = j->params + (int64_t)r * j->params_stride;
        double u = j->u ? j->u[r] : 0.0;
        int32_t id = 0;
        for (int i = 0; i < n; i++) probs[i] = 0;
        int rc = sample_row(n, x, h, nh, p, u, &id, probs, j->info ? j->info + r : NULL, wsf, wsp,
                            seen);
        j->out_ids[r] = rc == VXS_OK ? id : rc;
        if (rc != VXS_OK && j->rc == VXS_OK) j->rc = rc;
        if (j->out_logits) memcpy(j->out_logits + (int64_t)r * n, x, (size_t)n * sizeof(float));
        if (j->out_probs) memcpy(j->out_probs + (int64_t)r * n, probs, (size_t)n * sizeof(double));
    }
done:
    free(x);
    free(wsf);
    free(wsp);
    free(seen);
    free(probs);
    return NULL;
}

int vxs_oracle_sample(int rows, int vocab, const float* logits, int64_t ld, const int32_t* hist_off,
                      const int32_t* hist_ids, const vxs_params* params, int params_stride,
                      const double* u, int32_t* out_ids, float* out_logits, double* out_probs,
                      vxs_oracle_info* info, int threads) {
    if (rows < 0 || vocab <= 0 || !logits || ld < vocab || !params || !out_ids ||
        params_stride < 0 || (hist_off && !hist_ids))
        return VXS_ERR_INVALID_ARG;
    if (rows == 0) return VXS_OK;
    if (threads < 1) threads = 1;
    if (threads > rows) threads = rows;
    batch_job jobs[256];
    pthread_t tid[256];
    if (threads > 256) threads = 256;
    for (int t = 0; t < threads; t++) {
        batch_job* j = &jobs[t];
        j->row0 = (int)((int64_t)rows * t / threads);
        j->row1 = (int)((int64_t)rows * (t + 1) / threads);
        j->vocab = vocab;
        j->logits = logits;
        j->ld = ld;
        j->hist_off = hist_off;
        j->hist_ids = hist_ids;
        j->params = params;
        j->params_stride = params_stride;
        j->u = u;
        j->out_ids = out_ids;
        j->out_logits = out_logits;
        j->out_probs = out_probs;
        j->info = info;
    }
    if (threads == 1) {
        run_rows(&jobs[0]);
        return jobs[0].rc;
    }
    for (int t = 0; t < threads; t++) pthread_create(&tid[t], NULL, run_rows, &jobs[t]);
    int rc = VXS_OK;
    for (int t = 0; t < threads; t++) {
        pthread_join(tid[t], NULL);
        if (jobs[t].rc != VXS_OK && rc == VXS_OK) rc = jobs[t].rc;
    }
    return rc;
}

/* The repetition penalty alone, in place (Sampler.ApplyRepetitionPenalty). */
int vxs_oracle_apply_penalty(int rows, int vocab, float* logits, int64_t ld, const int32_t* hist_off,
                             const int32_t* hist_ids, float penalty) {
    unsigned char* seen = (unsigned char*)malloc((size_t)vocab);
    if (!seen) return VXS_ERR_INVALID_ARG;
    int rc = VXS_OK;
    for (int r = 0; r < rows && rc == VXS_OK; r++) {
        const int32_t* h = hist_ids + hist_off[r];
        int64_t nh = (int64_t)hist_off[r + 1] - hist_off[r];
        rc = penalty_row(vocab, logits + (int64_t)r * ld, h, nh, penalty, seen);
    }
    free(seen);
    return rc;
}
