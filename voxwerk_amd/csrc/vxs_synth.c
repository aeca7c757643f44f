/*
 * vxs_synth.c — deterministic synthetic sampler workloads (CPU).
 *
 * Produces the logits, histories, parameters and uniforms of the five benchmark workloads of
 * the voxwerk sampler (talker step, code-predictor frame, batched talker step, full-vocab
 * nucleus, wide vocab). Every value comes from SplitMix64 streams keyed by (seed, step, row,
 * purpose) and from IEEE +,-,*,/,sqrt only: the logarithm and cosine used by Box–Muller are
 * written here as polynomials, so the bytes are identical on every x86-64 host (no libm
 * version or CPU dispatch involved). Build with -ffp-contract=off.
 */
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "../../include/vxs_sampler.h"

#define VXS_SYNTH_API __attribute__((visibility("default")))

/* ---- SplitMix64 (Steele, Lea, Flood 2014) ---------------------------------------------------- */
static inline uint64_t sm64_next(uint64_t* s) {
    uint64_t z = (*s += 0x9e3779b97f4a7c15ull);
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}

static inline uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}

/* Stream state for (seed, step, row, purpose). */
static uint64_t stream_state(uint64_t seed, uint64_t step, uint64_t row, uint64_t purpose) {
    uint64_t s = mix64(seed + 0x632be59bd9b4e019ull);
    s = mix64(s ^ (step * 0x9e3779b97f4a7c15ull + 0x1234567ull));
    s = mix64(s ^ (row * 0xd1b54a32d192ed03ull + 0x89abcdefull));
    s = mix64(s ^ (purpose * 0x8cb92ba72f3d8dd7ull + 0x5555ull));
    return s;
}

/* Uniform double in [0,1) with 53 random bits. */
static inline double u01(uint64_t* s) { return (double)(sm64_next(s) >> 11) * 0x1.0p-53; }

/* Uniform integer in [0,n) (multiply-shift on 32 high bits; n < 2^31). */
static inline int32_t uint_below(uint64_t* s, int32_t n) {
    uint64_t r = sm64_next(s) >> 32;
    return (int32_t)((r * (uint64_t)n) >> 32);
}

/* ---- deterministic log and cos ---------------------------------------------------------------- */
static const double LN2 = 0.6931471805599453094;

/* Natural log of a positive normal double: x = 2^k * m, m in [sqrt(1/2), sqrt(2)),
 * log m = 2 atanh(s), s = (m-1)/(m+1), series to s^21 (|s| < 0.1716: error < 1e-17). */
static double det_log(double x) {
    uint64_t b;
    memcpy(&b, &x, 8);
    int k = (int)((b >> 52) & 0x7ff) - 1023;
    b = (b & 0x000fffffffffffffull) | 0x3ff0000000000000ull;
    double m;
    memcpy(&m, &b, 8);
    if (m > 1.4142135623730951) {
        m = m * 0.5;
        k += 1;
    }
    double s = (m - 1.0) / (m + 1.0);
    double z = s * s;
    double t = 1.0 / 21;
    t = 1.0 / 19 + z * t;
    t = 1.0 / 17 + z * t;
    t = 1.0 / 15 + z * t;
    t = 1.0 / 13 + z * t;
    t = 1.0 / 11 + z * t;
    t = 1.0 / 9 + z * t;
    t = 1.0 / 7 + z * t;
    t = 1.0 / 5 + z * t;
    t = 1.0 / 3 + z * t;
    t = 1.0 + z * t;
    return (double)k * LN2 + 2.0 * s * t;
}

/* cos(2*pi*v) for v in [0,1): quarter-turn reduction is exact on the dyadic v, then Taylor
 * series for sin/cos of a in [0, pi/2) to degree 22 (error < 1e-16). */
static double det_cos_turn(double v) {
    double t = v * 4.0; /* exact */
    int q = (int)t;
    double f = t - (double)q; /* exact, in [0,1) */
    double a = f * 1.5707963267948966;
    double z = a * a;
    double c = 1.0, s = 1.0;
    /* cos a = sum (-1)^n z^n/(2n)!, sin a = a * sum (-1)^n z^n/(2n+1)! (Horner from n=11) */
    double cn = 0.0, sn = 0.0;
    for (int n = 11; n >= 1; n--) {
        double fc = 1.0, fs = 1.0;
        for (int i = 1; i <= 2 * n; i++) fc *= (double)i;
        for (int i = 1; i <= 2 * n + 1; i++) fs *= (double)i;
        double sign = (n & 1) ? -1.0 : 1.0;
        cn = (cn + sign / fc) * z;
        sn = (sn + sign / fs) * z;
    }
    c = 1.0 + cn;
    s = a * (1.0 + sn);
    switch (q & 3) {
        case 0: return c;
        case 1: return -s;
        case 2: return -c;
        default: return s;
    }
}

/* Standard normal by Box–Muller (cosine branch; one normal per two uniforms). */
static double normal01(uint64_t* s) {
    double u1 = 1.0 - u01(s); /* (0,1] */
    double u2 = u01(s);
    return sqrt(-2.0 * det_log(u1)) * det_cos_turn(u2);
}

/* ---- workloads --------------------------------------------------------------------------------- */
enum { P_LOGITS = 0, P_HIST = 1, P_SPECIAL = 2, P_UNIFORM = 3, P_MIX = 4, P_PERM = 5 };

typedef struct vxs_workload {
    int32_t id;       /* 1..5 */
    int32_t rows;     /* rows per step */
    int32_t vocab;
    int32_t steps;    /* sequential steps (code-predictor frame: 15) */
    int32_t hist_len; /* history ids per row (0 = none) */
    uint64_t seed;
    vxs_params params;
} vxs_workload;

static int workload_of(int id, vxs_workload* w) {
    memset(w, 0, sizeof(*w));
    w->id = id;
    w->steps = 1;
    vxs_params p;
    memset(&p, 0, sizeof(p));
    p.do_sample = 1;
    p.keep_id = -1;
    p.ban_id = -1;
    switch (id) {
        case 1: /* single talker step */
            w->rows = 1, w->vocab = 3072, w->hist_len = 256, w->seed = 42;
            p.top_k = 50, p.top_p = 1.0f, p.temperature = 0.9f, p.rep_penalty = 1.05f;
            break;
        case 2: /* code-predictor sub-sampling, 15 sequential codebook steps */
            w->rows = 16, w->vocab = 2048, w->hist_len = 0, w->seed = 7, w->steps = 15;
            p.top_k = 50, p.top_p = 1.0f, p.temperature = 0.9f, p.rep_penalty = 1.0f;
            break;
        case 3: /* batched talker step with suppression */
            w->rows = 256, w->vocab = 3072, w->hist_len = 2048, w->seed = 123;
            p.top_k = 50, p.top_p = 0.9f, p.temperature = 0.9f, p.rep_penalty = 1.05f;
            p.supp_begin = 2048, p.supp_end = 3072, p.keep_id = 2150;
            break;
        case 4: /* bandwidth-bound full-vocab nucleus */
            w->rows = 4096, w->vocab = 3072, w->hist_len = 512, w->seed = 2024;
            p.top_k = 0, p.top_p = 0.95f, p.temperature = 1.0f, p.rep_penalty = 1.1f;
            break;
        case 5: /* wide-vocab stress */
            w->rows = 1024, w->vocab = 151936, w->hist_len = 4096, w->seed = 99;
            p.top_k = 200, p.top_p = 0.8f, p.temperature = 0.7f, p.rep_penalty = 1.05f;
            p.supp_begin = 151936 - 1024, p.supp_end = 151936, p.keep_id = 151936 - 1024 + 102;
            break;
        default:
            return VXS_ERR_INVALID_ARG;
    }
    w->params = p;
    return VXS_OK;
}

VXS_SYNTH_API int vxs_synth_workload(int id, vxs_workload* out) { return workload_of(id, out); }

/* One row's logits. `perm` is vocab int32 scratch (wide-vocab workload only). */
static void gen_row_logits(const vxs_workload* w, int step, int64_t row, float* x, int32_t* perm) {
    int V = w->vocab;
    uint64_t s = stream_state(w->seed, (uint64_t)step, (uint64_t)row, P_LOGITS);
    switch (w->id) {
        case 1:
        case 3:
            for (int i = 0; i < V; i++) x[i] = (float)(3.0 * normal01(&s));
            break;
        case 2:
            for (int i = 0; i < V; i++) x[i] = (float)(2.5 * normal01(&s));
            break;
        case 4: {
            uint64_t m = stream_state(w->seed, (uint64_t)step, (uint64_t)row, P_MIX);
            for (int i = 0; i < V; i++) {
                double mean = u01(&m) < 0.1 ? 4.0 : 0.0;
                x[i] = (float)(mean + normal01(&s));
            }
            break;
        }
        case 5: {
            /* logit = -1.1 ln(rank) + N(0, 0.5^2), ranks 1..V under a Fisher–Yates permutation */
            uint64_t ps = stream_state(w->seed, (uint64_t)step, (uint64_t)row, P_PERM);
            for (int i = 0; i < V; i++) perm[i] = i + 1;
            for (int i = V - 1; i > 0; i--) {
                int j = uint_below(&ps, i + 1);
                int32_t t = perm[i];
                perm[i] = perm[j];
                perm[j] = t;
            }
            for (int i = 0; i < V; i++)
                x[i] = (float)(-1.1 * det_log((double)perm[i]) + 0.5 * normal01(&s));
            break;
        }
    }
    if (w->id == 1) { /* 8 distinct ids set to +10 */
        uint64_t sp = stream_state(w->seed, (uint64_t)step, (uint64_t)row, P_SPECIAL);
        int32_t chosen[8];
        int n = 0;
        while (n < 8) {
            int32_t id = uint_below(&sp, V);
            int dup = 0;
            for (int k = 0; k < n; k++) dup |= chosen[k] == id;
            if (!dup) chosen[n++] = id;
        }
        for (int k = 0; k < 8; k++) x[chosen[k]] = 10.0f;
    } else if (w->id == 2) { /* one peak per row at +8 */
        uint64_t sp = stream_state(w->seed, (uint64_t)step, (uint64_t)row, P_SPECIAL);
        x[uint_below(&sp, V)] = 8.0f;
    }
}

typedef struct {
    const vxs_workload* w;
    int step;
    int64_t r0, r1, row_base;
    float* logits;
    int64_t ld;
    int32_t* hist;
    double* u;
    int rc;
} gen_job;

static void* gen_rows(void* arg) {
    gen_job* j = (gen_job*)arg;
    const vxs_workload* w = j->w;
    int32_t* perm = w->id == 5 ? (int32_t*)malloc((size_t)w->vocab * sizeof(int32_t)) : NULL;
    j->rc = VXS_OK;
    if (w->id == 5 && !perm) {
        j->rc = VXS_ERR_INVALID_ARG;
        return NULL;
    }
    for (int64_t r = j->r0; r < j->r1; r++) {
        int64_t gr = j->row_base + r; /* absolute row within the workload */
        if (j->logits) gen_row_logits(w, j->step, gr, j->logits + r * j->ld, perm);
        if (j->hist && w->hist_len > 0) {
            uint64_t s = stream_state(w->seed, (uint64_t)j->step, (uint64_t)gr, P_HIST);
            int32_t* h = j->hist + r * w->hist_len;
            for (int k = 0; k < w->hist_len; k++) h[k] = uint_below(&s, w->vocab);
        }
        if (j->u) {
            uint64_t s = stream_state(w->seed, (uint64_t)j->step, (uint64_t)gr, P_UNIFORM);
            j->u[r] = u01(&s);
        }
    }
    free(perm);
    return NULL;
}

/*
 * Generate rows [row_begin, row_begin+rows) of step `step` of workload `id`.
 * logits: [rows][ld] (NULL to skip); hist: [rows][hist_len] (NULL to skip); u: [rows] (NULL to
 * skip). Rows are independent streams, so any row subset reproduces the full batch's rows.
 */
VXS_SYNTH_API int vxs_synth_generate(int id, int step, int64_t row_begin, int64_t rows, float* logits,
                                     int64_t ld, int32_t* hist, double* u, int threads) {
    vxs_workload w;
    if (workload_of(id, &w) != VXS_OK) return VXS_ERR_INVALID_ARG;
    if (step < 0 || step >= w.steps || row_begin < 0 || rows < 0 || row_begin + rows > w.rows)
        return VXS_ERR_INVALID_ARG;
    if (logits && ld < w.vocab) return VXS_ERR_INVALID_ARG;
    if (threads < 1) threads = 1;
    if (threads > 64) threads = 64;
    if (threads > rows) threads = rows > 0 ? (int)rows : 1;
    gen_job jobs[64];
    pthread_t tid[64];
    for (int t = 0; t < threads; t++) {
        jobs[t].w = &w;
        jobs[t].step = step;
        jobs[t].r0 = rows * t / threads;
        jobs[t].r1 = rows * (t + 1) / threads;
        jobs[t].row_base = row_begin;
        jobs[t].logits = logits;
        jobs[t].ld = ld;
        jobs[t].hist = hist;
        jobs[t].u = u;
    }
    if (threads == 1) {
        gen_rows(&jobs[0]);
        return jobs[0].rc;
    }
    for (int t = 0; t < threads; t++) pthread_create(&tid[t], NULL, gen_rows, &jobs[t]);
    int rc = VXS_OK;
    for (int t = 0; t < threads; t++) {
        pthread_join(tid[t], NULL);
        if (jobs[t].rc != VXS_OK) rc = jobs[t].rc;
    }
    return rc;
}

/* Exposed for tests of the generator itself. */
VXS_SYNTH_API double vxs_synth_log(double x) { return det_log(x); }
VXS_SYNTH_API double vxs_synth_cos_turn(double v) { return det_cos_turn(v); }
