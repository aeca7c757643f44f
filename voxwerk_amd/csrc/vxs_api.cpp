// vxs_api.cpp — the C ABI of include/vxs_sampler.h: contexts, device buffers, pinned staging,
// argument validation and error mapping. No C++ exception crosses the boundary.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cstdio>
#include <cstring>
#include <new>
#include <string>
#include <vector>

#include "vxs_internal.h"

namespace {

constexpr size_t kAlign = 256;
constexpr int kPolledMaxRows = 1024;                        // host calls below this complete by polling
constexpr std::chrono::seconds kPollLimit{2};              // then a stream synchronisation takes over
// Polled calls staging at most this many bytes skip the host-to-device copy: the kernel reads its
// inputs straight from the coherent pinned staging block over PCIe (one pass, so nothing is lost),
// which saves the copy's latency (a DMA engine handoff of ~10 us once a copy exceeds a few KiB).
constexpr size_t kZeroCopyMaxBytes = size_t(2) << 20;
size_t align_up(size_t x) { return (x + kAlign - 1) & ~(kAlign - 1); }

// Device buffer that only grows.
struct DevBuf {
    void* p = nullptr;
    size_t cap = 0;
    hipError_t reserve(size_t n) {
        if (n <= cap) return hipSuccess;
        if (p) {
            hipError_t e = hipFree(p);
            p = nullptr;
            cap = 0;
            if (e != hipSuccess) return e;
        }
        size_t want = std::max(n, cap + cap / 2);
        hipError_t e = hipMalloc(&p, want);
        if (e != hipSuccess) return e;
        cap = want;
        return hipSuccess;
    }
    void release() {
        if (p) (void)hipFree(p);
        p = nullptr;
        cap = 0;
    }
};

// Pinned host buffer that only grows.
struct HostBuf {
    void* p = nullptr;
    size_t cap = 0;
    unsigned flags = hipHostMallocDefault;
    hipError_t reserve(size_t n) {
        if (n <= cap) return hipSuccess;
        if (p) {
            hipError_t e = hipHostFree(p);
            p = nullptr;
            cap = 0;
            if (e != hipSuccess) return e;
        }
        size_t want = std::max(n, cap + cap / 2);
        hipError_t e = hipHostMalloc(&p, want, flags);
        if (e != hipSuccess) return e;
        cap = want;
        return hipSuccess;
    }
    void release() {
        if (p) (void)hipHostFree(p);
        p = nullptr;
        cap = 0;
    }
};

}  // namespace

struct vxs_ctx {
    int device = 0;
    hipStream_t own_stream = nullptr;
    hipStream_t stream = nullptr;
    std::string err;
    DevBuf d_in, d_ids, d_logits_out, d_probs_out;
    DevBuf d_draw;   // uniforms drawn on the device by vxs_history_draw
    HostBuf h_in, h_ids, h_out;  // h_in is coherent: polled calls' kernels read it in place
    void* h_in_dev = nullptr;    // device address of h_in.p
    void* h_in_dev_of = nullptr;  // the h_in.p that h_in_dev belongs to
    // completion by polling (small host calls on the one-workgroup-per-row path): a device counter,
    // zeroed once, and coherent pinned memory holding the flag (word 0) and the ids (from word 16)
    DevBuf d_done;
    bool done_ready = false;
    HostBuf h_done;
    uint32_t done_seq = 0;  // wraps; the completion word is reset to seq - 1 before each launch
    void* noalloc = nullptr;  // this device's fixed scratch (vxs_sample_noalloc), looked up at create
};

struct vxs_history {
    int device = 0;
    int slots = 0;
    int cap = 0;
    int32_t* ids = nullptr;  // [slots][cap]
    int32_t* len = nullptr;  // [slots]
    int32_t* rng = nullptr;  // [slots][2][kRngWords]: talker and code-predictor generators
    vxs::StoreDesc* desc = nullptr;  // the three pointers and the shape, in device memory
    std::vector<uint8_t> seeded;  // host record of vxs_history_seed per slot
};

namespace {

int fail(vxs_ctx* ctx, int code, const std::string& msg) {
    if (ctx) ctx->err = msg;
    return code;
}

int hip_fail(vxs_ctx* ctx, hipError_t e, const char* what) {
    std::string m = std::string(what) + ": " + hipGetErrorString(e);
    return fail(ctx, VXS_ERR_HIP, m);
}

#define VXS_HIP(ctx, call)                                         \
    do {                                                           \
        hipError_t e_ = (call);                                    \
        if (e_ != hipSuccess) return hip_fail((ctx), e_, #call);   \
    } while (0)

const char* code_text(int code) {
    switch (code) {
        case VXS_ERR_INVALID_ARG: return "invalid argument";
        case VXS_ERR_ID_OUT_OF_RANGE: return "history id out of range [0, vocab)";
        case VXS_ERR_NONFINITE: return "NaN or +inf logit after temperature";
        case VXS_ERR_HIP: return "HIP error";
        case VXS_ERR_UNSUPPORTED: return "unsupported shape";
        case VXS_ERR_NO_DEVICE: return "no gfx950 device";
        case VXS_ERR_HISTORY_FULL: return "resident history slot is full";
        default: return "error";
    }
}

// Validation shared by the host and device entry points (host-side facts only).
int check_shape(vxs_ctx* ctx, int rows, int vocab, const void* logits, int64_t ld, const void* params,
                int params_stride, const void* out_ids) {
    if (!ctx) return VXS_ERR_INVALID_ARG;
    if (rows < 0) return fail(ctx, VXS_ERR_INVALID_ARG, "rows < 0");
    if (vocab <= 0) return fail(ctx, VXS_ERR_INVALID_ARG, "vocab <= 0");
    if (ld < vocab) return fail(ctx, VXS_ERR_INVALID_ARG, "ld < vocab");
    if (params_stride < 0) return fail(ctx, VXS_ERR_INVALID_ARG, "params_stride < 0");
    if (rows > 0 && (!logits || !params || !out_ids))
        return fail(ctx, VXS_ERR_INVALID_ARG, "null logits, params or out_ids");
    if (vocab > vxs::kWideMaxVocab)
        return fail(ctx, VXS_ERR_UNSUPPORTED,
                    "vocab " + std::to_string(vocab) + " exceeds the limit " + std::to_string(vxs::kWideMaxVocab));
    return VXS_OK;
}

int check_params_host(vxs_ctx* ctx, int rows, const vxs_params* params, int stride, const double* u) {
    const int np = stride == 0 ? 1 : rows;
    for (int i = 0; i < np; i++) {
        const vxs_params& p = params[(int64_t)i * stride];
        if (p.do_sample && !u) return fail(ctx, VXS_ERR_INVALID_ARG, "u is NULL but a row samples");
    }
    return VXS_OK;
}

int first_row_error(vxs_ctx* ctx, const int32_t* ids, int rows) {
    for (int r = 0; r < rows; r++)
        if (ids[r] < 0) {
            char buf[96];
            std::snprintf(buf, sizeof buf, "row %d: %s", r, code_text(ids[r]));
            return fail(ctx, ids[r], buf);
        }
    return VXS_OK;
}

// Pack host inputs into the pinned staging block; returns byte offsets of each section.
struct Layout {
    size_t params, u, hoff, hids, logits, total;
    int64_t ld_dev;
    int np;
    int64_t nh;
};

Layout plan(int rows, int vocab, int params_stride, const int32_t* hist_off) {
    Layout L{};
    L.np = params_stride == 0 ? 1 : rows;
    L.nh = hist_off ? (int64_t)hist_off[rows] - hist_off[0] : 0;
    L.ld_dev = ((int64_t)vocab + 3) & ~(int64_t)3;
    size_t off = 0;
    L.params = off;
    off = align_up(off + sizeof(vxs_params) * (size_t)std::max(L.np, 1));
    L.u = off;
    off = align_up(off + sizeof(double) * (size_t)rows);
    L.hoff = off;
    off = align_up(off + sizeof(int32_t) * (size_t)(rows + 1));
    L.hids = off;
    off = align_up(off + sizeof(int32_t) * (size_t)L.nh);
    L.logits = off;
    off = align_up(off + sizeof(float) * (size_t)rows * (size_t)L.ld_dev);
    L.total = off;
    return L;
}

int check_hist_host(vxs_ctx* ctx, int rows, const int32_t* hist_off, const int32_t* hist_ids) {
    if (!hist_off) return VXS_OK;
    for (int r = 0; r < rows; r++)
        if (hist_off[r + 1] < hist_off[r]) return fail(ctx, VXS_ERR_INVALID_ARG, "hist_off not monotone");
    if (hist_off[rows] > hist_off[0] && !hist_ids) return fail(ctx, VXS_ERR_INVALID_ARG, "hist_ids is NULL");
    return VXS_OK;
}

constexpr uint32_t kPathFlags = VXS_FLAG_PATH_BLOCK | VXS_FLAG_PATH_WAVE;

// Kernel path: the one-wave path needs a vocabulary it can hold and enough rows to fill the GPU
// at four rows per workgroup; the caller may force either.
int choose_path(uint32_t flags, int rows, int vocab) {
    if (vocab > vxs::kWaveMaxVocab || (flags & VXS_FLAG_PATH_BLOCK)) return vxs::kPathBlock;
    if (flags & VXS_FLAG_PATH_WAVE) return vxs::kPathQuad;
    return rows >= 1024 ? vxs::kPathQuad : vxs::kPathBlock;
}

// Host calls know their options: when most rows sample with a top-k above 64, which the one-wave
// path hands back, go to the one-workgroup-per-row kernel directly.
int choose_path_host(uint32_t flags, int rows, int vocab, const vxs_params* params, int stride) {
    const int path = choose_path(flags, rows, vocab);
    if (path != vxs::kPathQuad || (flags & VXS_FLAG_PATH_WAVE)) return path;
    const int np = stride == 0 ? 1 : rows;
    int topk = 0;
    for (int i = 0; i < np; i++) {
        const vxs_params& p = params[(int64_t)i * stride];
        topk += p.do_sample && p.top_k > vxs::kWaveMaxTopK && p.top_k < vocab;
    }
    return 2 * topk > np ? vxs::kPathBlock : path;
}

int check_flags(vxs_ctx* ctx, uint32_t flags) {
    if (flags & ~kPathFlags) return fail(ctx, VXS_ERR_INVALID_ARG, "unknown flags");
    if ((flags & kPathFlags) == kPathFlags) return fail(ctx, VXS_ERR_INVALID_ARG, "both path flags set");
    return VXS_OK;
}

// A call whose histories live in a resident store: host slot indices (staged with the inputs),
// whether to append, the generator stream, and the completion words of a polled call.
struct ResidentCall {
    const vxs_history* store = nullptr;
    const int32_t* slots = nullptr;
    int append = 0;
    int rng_stream = -1;  // 0 / 1: draw the uniforms from the slots' talker / code-predictor generators
    const vxs::SampleArgs* done = nullptr;
};

constexpr uint32_t kRngFlags = VXS_FLAG_RNG_TALKER | VXS_FLAG_RNG_SUB;

int rng_stream_of(uint32_t flags) {
    return (flags & VXS_FLAG_RNG_TALKER) ? 0 : (flags & VXS_FLAG_RNG_SUB) ? 1 : -1;
}

// new Random(seed) of .NET (the seeded, legacy subtractive generator), into st[0..kRngWords):
// SeedArray[1..55], then inext = 0 and inextp = 21. Every step wraps to 32 bits, as C#'s unchecked
// int arithmetic does (seeds above 161803398 overflow during seeding).
void dotnet_seed(int32_t seed, int32_t* st) {
    constexpr int32_t kMbig = 0x7FFFFFFF, kMseed = 161803398;
    auto sub = [](int32_t a, int32_t b) { return (int32_t)((uint32_t)a - (uint32_t)b); };
    auto add = [](int32_t a, int32_t b) { return (int32_t)((uint32_t)a + (uint32_t)b); };
    for (int i = 0; i < vxs::kRngWords; i++) st[i] = 0;
    const int32_t subtraction = seed == INT32_MIN ? kMbig : (seed < 0 ? -seed : seed);
    int32_t mj = sub(kMseed, subtraction);
    st[55] = mj;
    int32_t mk = 1;
    int ii = 0;
    for (int i = 1; i < 55; i++) {
        ii += 21;
        if (ii >= 55) ii -= 55;
        st[ii] = mk;
        mk = sub(mj, mk);
        if (mk < 0) mk = add(mk, kMbig);
        mj = st[ii];
    }
    for (int k = 1; k < 5; k++)
        for (int i = 1; i < 56; i++) {
            int n = i + 30;
            if (n >= 55) n -= 55;
            st[i] = sub(st[i], st[1 + n]);
            if (st[i] < 0) st[i] = add(st[i], kMbig);
        }
    st[56] = 0;
    st[57] = 21;
}

// Row histories of a resident call: the sampler reads each row's slot and ends its step itself
// (draw from the slot's generator when rng_stream >= 0, append when `append`, slot check).
void set_resident(vxs::SampleArgs& a, const vxs_history* h, const int32_t* d_slots, int append, int rng_stream) {
    a.hist_off = nullptr;
    a.hist_ids = h->ids;
    a.hist_slot = d_slots;
    a.hist_len = h->len;
    a.hist_cap = h->cap;
    a.hist_slots = h->slots;
    a.store = h->desc;
    if (append) a.kflags |= vxs::KF_APPEND;
    if (rng_stream >= 0) a.kflags |= vxs::KF_RNG | (rng_stream == 1 ? vxs::KF_RNG_SUB : 0u);
}

// Stage inputs and launch. On success the kernels are queued on ctx->stream.
int stage_and_launch(vxs_ctx* ctx, int rows, int vocab, const float* logits, int64_t ld, const int32_t* hist_off,
                     const int32_t* hist_ids, const vxs_params* params, int params_stride, const double* u,
                     bool want_logits, bool want_probs, uint32_t kflags, uint32_t flags = 0,
                     const vxs::SampleArgs* done = nullptr, const ResidentCall* res = nullptr) {
    const Layout L = plan(rows, vocab, params_stride, hist_off);
    const bool zero_copy = (done || (res && res->done)) && L.total <= kZeroCopyMaxBytes;
    VXS_HIP(ctx, ctx->h_in.reserve(L.total));
    if (!zero_copy) VXS_HIP(ctx, ctx->d_in.reserve(L.total));
    char* h = static_cast<char*>(ctx->h_in.p);
    for (int i = 0; i < L.np; i++)
        std::memcpy(h + L.params + sizeof(vxs_params) * i, params + (int64_t)i * params_stride, sizeof(vxs_params));
    if (u) std::memcpy(h + L.u, u, sizeof(double) * rows);
    else std::memset(h + L.u, 0, sizeof(double) * rows);
    int32_t* hoff = reinterpret_cast<int32_t*>(h + L.hoff);
    if (hist_off) {
        for (int r = 0; r <= rows; r++) hoff[r] = hist_off[r] - hist_off[0];
        if (L.nh) std::memcpy(h + L.hids, hist_ids + hist_off[0], sizeof(int32_t) * L.nh);
    } else if (res) {
        std::memcpy(hoff, res->slots, sizeof(int32_t) * rows);  // slot indices use the offsets' room
    }
    float* lg = reinterpret_cast<float*>(h + L.logits);
    if (ld == L.ld_dev) {  // one copy that ends at the last row's last entry (its pads are not read)
        std::memcpy(lg, logits, sizeof(float) * ((size_t)(rows - 1) * (size_t)ld + (size_t)vocab));
    } else {
        for (int r = 0; r < rows; r++) std::memcpy(lg + (int64_t)r * L.ld_dev, logits + (int64_t)r * ld, sizeof(float) * vocab);
    }
    VXS_HIP(ctx, ctx->d_ids.reserve(sizeof(int32_t) * (size_t)rows));
    if (want_logits) VXS_HIP(ctx, ctx->d_logits_out.reserve(sizeof(float) * (size_t)rows * vocab));
    if (want_probs) VXS_HIP(ctx, ctx->d_probs_out.reserve(sizeof(double) * (size_t)rows * vocab));
    char* d;
    if (zero_copy) {
        if (ctx->h_in_dev_of != ctx->h_in.p) {
            VXS_HIP(ctx, hipHostGetDevicePointer(&ctx->h_in_dev, ctx->h_in.p, 0));
            ctx->h_in_dev_of = ctx->h_in.p;
        }
        d = static_cast<char*>(ctx->h_in_dev);
    } else {
        VXS_HIP(ctx, hipMemcpyAsync(ctx->d_in.p, ctx->h_in.p, L.total, hipMemcpyHostToDevice, ctx->stream));
        d = static_cast<char*>(ctx->d_in.p);
    }
    vxs::SampleArgs a{};
    a.rows = rows;
    a.vocab = vocab;
    a.ld = L.ld_dev;
    a.logits = reinterpret_cast<const float*>(d + L.logits);
    a.hist_off = hist_off ? reinterpret_cast<const int32_t*>(d + L.hoff) : nullptr;
    a.hist_ids = reinterpret_cast<const int32_t*>(d + L.hids);
    a.params = reinterpret_cast<const vxs_params*>(d + L.params);
    a.params_stride = params_stride == 0 ? 0 : 1;
    a.u = reinterpret_cast<const double*>(d + L.u);
    a.out_ids = static_cast<int32_t*>(ctx->d_ids.p);
    a.out_logits = want_logits ? static_cast<float*>(ctx->d_logits_out.p) : nullptr;
    a.out_probs = want_probs ? static_cast<double*>(ctx->d_probs_out.p) : nullptr;
    a.kflags = kflags;
    a.path = choose_path_host(flags, rows, vocab, params, params_stride);
    if (res && res->done) done = res->done;
    if (done) {
        a.out_ids = done->out_ids;
        if (done->out_logits) a.out_logits = done->out_logits;
        a.done_count = done->done_count;
        a.done_flag = done->done_flag;
        a.done_seq = done->done_seq;
    }
    if (res) set_resident(a, res->store, reinterpret_cast<const int32_t*>(d + L.hoff), res->append, res->rng_stream);
    if (zero_copy && rows == 1 && !res && a.path == vxs::kPathBlock) {
        // one row read in place over PCIe: its scalars travel in the kernel arguments
        a.row_direct = 1;
        a.direct_params = params[0];
        a.direct_h0 = 0;
        a.direct_h1 = hist_off ? hoff[1] : 0;
        a.direct_u = u ? u[0] : 0.0;
    }
    VXS_HIP(ctx, vxs::launch_sample(a, ctx->stream));
    return VXS_OK;
}

// Host calls that can complete by polling: the one-workgroup-per-row kernel alone, ids and (up to
// kZeroCopyMaxBytes of them) write-back logits, which the kernel then stores into coherent host memory.
bool polled_call(int rows, int vocab, uint32_t flags, bool want_logits, bool want_probs) {
    return !want_probs && vocab <= vxs::kRowResidentMaxVocab &&
           choose_path(flags, rows, vocab) == vxs::kPathBlock && rows <= kPolledMaxRows &&
           (!want_logits || sizeof(float) * (size_t)rows * (size_t)vocab <= kZeroCopyMaxBytes);
}

// Completion state for a polled call of `rows` rows: the device counter (zeroed when first used and
// after any failure) and the coherent host words the kernel writes: the completion word, the ids
// and, when logit_count > 0, that many write-back logits from a 256-byte boundary.
hipError_t ensure_done(vxs_ctx* ctx, int rows, vxs::SampleArgs& a, size_t logit_count = 0) {
    if (!ctx->done_ready) {
        hipError_t e = ctx->d_done.reserve(sizeof(int32_t));
        if (e != hipSuccess) return e;
        if ((e = hipMemset(ctx->d_done.p, 0, sizeof(int32_t))) != hipSuccess) return e;
        ctx->done_ready = true;
    }
    ctx->h_done.flags = hipHostMallocCoherent;
    const size_t logits_at = align_up(sizeof(int32_t) * (16 + (size_t)rows));
    hipError_t e = ctx->h_done.reserve(logits_at + sizeof(float) * logit_count);
    if (e != hipSuccess) return e;
    int32_t* w = static_cast<int32_t*>(ctx->h_done.p);
    const uint32_t seq = ++ctx->done_seq;
    // the word the host polls can never hold the new sequence before this call's kernel writes
    // it, also in a freshly allocated (or recycled) block: the previous call's kernel has finished
    __atomic_store_n(w, (int32_t)(seq - 1u), __ATOMIC_RELEASE);
    a.done_count = static_cast<int32_t*>(ctx->d_done.p);
    a.done_flag = w;
    a.done_seq = (int32_t)seq;
    a.out_ids = w + 16;
    a.out_logits = logit_count ? reinterpret_cast<float*>(static_cast<char*>(ctx->h_done.p) + logits_at) : nullptr;
    return hipSuccess;
}

// Spin until the kernel publishes `seq`; after kPollLimit fall back to a stream synchronisation,
// which reports a failed kernel.
int wait_done(vxs_ctx* ctx, int32_t seq) {
    const int32_t* flag = static_cast<const int32_t*>(ctx->h_done.p);
    const auto t0 = std::chrono::steady_clock::now();
    while (__atomic_load_n(flag, __ATOMIC_ACQUIRE) != seq) {
        if (std::chrono::steady_clock::now() - t0 > kPollLimit) {
            const hipError_t e = hipStreamSynchronize(ctx->stream);
            if (e != hipSuccess) {
                ctx->done_ready = false;
                return hip_fail(ctx, e, "hipStreamSynchronize");
            }
            if (__atomic_load_n(flag, __ATOMIC_ACQUIRE) != seq) {
                ctx->done_ready = false;
                return fail(ctx, VXS_ERR_HIP, "kernel finished without publishing its completion");
            }
            break;
        }
    }
    return VXS_OK;
}

int check_batch_flags(vxs_ctx* ctx, uint32_t flags) {
    if (flags & ~(kPathFlags | kRngFlags)) return fail(ctx, VXS_ERR_INVALID_ARG, "unknown flags");
    if ((flags & kPathFlags) == kPathFlags) return fail(ctx, VXS_ERR_INVALID_ARG, "both path flags set");
    if ((flags & kRngFlags) == kRngFlags) return fail(ctx, VXS_ERR_INVALID_ARG, "both generator flags set");
    return VXS_OK;
}

int check_store(vxs_ctx* ctx, const vxs_history* h) {
    if (!h) return fail(ctx, VXS_ERR_INVALID_ARG, "history store is NULL");
    if (h->device != ctx->device) return fail(ctx, VXS_ERR_INVALID_ARG, "history store belongs to another device");
    return VXS_OK;
}

// Host slot indices of a resident call: each in [0, slots), no slot twice.
int check_slots_host(vxs_ctx* ctx, const vxs_history* h, int rows, const int32_t* slots) {
    if (!slots) return fail(ctx, VXS_ERR_INVALID_ARG, "slots is NULL");
    std::vector<int32_t> sorted(slots, slots + rows);
    for (int r = 0; r < rows; r++)
        if ((unsigned)slots[r] >= (unsigned)h->slots)
            return fail(ctx, VXS_ERR_INVALID_ARG, "row " + std::to_string(r) + ": slot outside the store");
    std::sort(sorted.begin(), sorted.end());
    if (std::adjacent_find(sorted.begin(), sorted.end()) != sorted.end())
        return fail(ctx, VXS_ERR_INVALID_ARG, "a slot appears twice in one call");
    return VXS_OK;
}

// Copy `bytes` of device results into host memory through pinned staging.
int fetch(vxs_ctx* ctx, void* dst, const void* src, size_t bytes) {
    if (!bytes) return VXS_OK;
    VXS_HIP(ctx, ctx->h_out.reserve(bytes));
    VXS_HIP(ctx, hipMemcpyAsync(ctx->h_out.p, src, bytes, hipMemcpyDeviceToHost, ctx->stream));
    VXS_HIP(ctx, hipStreamSynchronize(ctx->stream));
    std::memcpy(dst, ctx->h_out.p, bytes);
    return VXS_OK;
}

// Copy the rows of `src` whose id is a token (>= 0) into `dst`; a failed row of `dst` keeps what the
// caller had there.
void copy_ok_rows(void* dst, const void* src, const int32_t* ids, int rows, size_t row_bytes) {
    bool all = true;
    for (int r = 0; r < rows && all; r++) all = ids[r] >= 0;
    if (all) {
        std::memcpy(dst, src, row_bytes * (size_t)rows);
        return;
    }
    for (int r = 0; r < rows; r++)
        if (ids[r] >= 0)
            std::memcpy(static_cast<char*>(dst) + row_bytes * r, static_cast<const char*>(src) + row_bytes * r, row_bytes);
}

// fetch() of write-back rows, skipping the rows that failed.
int fetch_ok_rows(vxs_ctx* ctx, void* dst, const void* src, const int32_t* ids, int rows, size_t row_bytes) {
    const size_t bytes = row_bytes * (size_t)rows;
    if (!bytes) return VXS_OK;
    VXS_HIP(ctx, ctx->h_out.reserve(bytes));
    VXS_HIP(ctx, hipMemcpyAsync(ctx->h_out.p, src, bytes, hipMemcpyDeviceToHost, ctx->stream));
    VXS_HIP(ctx, hipStreamSynchronize(ctx->stream));
    copy_ok_rows(dst, ctx->h_out.p, ids, rows, row_bytes);
    return VXS_OK;
}

}  // namespace

extern "C" {

VXS_API const char* vxs_version(void) { return "vxs 0.1.0 gfx950"; }

VXS_API int vxs_create(vxs_ctx** out, int device, int max_rows, int max_vocab, int64_t max_hist) {
    if (!out) return VXS_ERR_INVALID_ARG;
    *out = nullptr;
    if (max_rows < 0 || max_vocab < 0 || max_hist < 0) return VXS_ERR_INVALID_ARG;
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) return VXS_ERR_NO_DEVICE;
    if (device < 0 || device >= n) return VXS_ERR_NO_DEVICE;
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, device) != hipSuccess) return VXS_ERR_NO_DEVICE;
    if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0) return VXS_ERR_NO_DEVICE;
    vxs_ctx* ctx = new (std::nothrow) vxs_ctx();
    if (!ctx) return VXS_ERR_INVALID_ARG;
    ctx->device = device;
    ctx->h_in.flags = hipHostMallocCoherent;
    if (hipSetDevice(device) != hipSuccess ||
        hipStreamCreateWithFlags(&ctx->own_stream, hipStreamNonBlocking) != hipSuccess) {
        delete ctx;
        return VXS_ERR_HIP;
    }
    ctx->stream = ctx->own_stream;
    // the fixed scratch's device address on this device (the device is current)
    if (vxs::noalloc_scratch(device, &ctx->noalloc) != hipSuccess) {
        vxs_destroy(ctx);
        return VXS_ERR_HIP;
    }
    if (max_rows > 0 && max_vocab > 0) {
        const int32_t* no_hist = nullptr;
        Layout L = plan(max_rows, max_vocab, 1, no_hist);
        size_t hist_bytes = align_up(sizeof(int32_t) * (size_t)max_hist);
        if (ctx->d_in.reserve(L.total + hist_bytes) != hipSuccess || ctx->h_in.reserve(L.total + hist_bytes) != hipSuccess ||
            ctx->d_ids.reserve(sizeof(int32_t) * (size_t)max_rows) != hipSuccess ||
            ctx->h_out.reserve(sizeof(int32_t) * (size_t)max_rows) != hipSuccess) {
            vxs_destroy(ctx);
            return VXS_ERR_HIP;
        }
    }
    *out = ctx;
    return VXS_OK;
}

VXS_API void vxs_destroy(vxs_ctx* ctx) {
    if (!ctx) return;
    (void)hipSetDevice(ctx->device);
    if (ctx->stream) (void)hipStreamSynchronize(ctx->stream);
    ctx->d_in.release();
    ctx->d_ids.release();
    ctx->d_draw.release();
    ctx->d_done.release();
    ctx->h_done.release();
    ctx->d_logits_out.release();
    ctx->d_probs_out.release();
    ctx->h_in.release();
    ctx->h_ids.release();
    ctx->h_out.release();
    if (ctx->own_stream) (void)hipStreamDestroy(ctx->own_stream);
    delete ctx;
}

VXS_API const char* vxs_last_error(const vxs_ctx* ctx) { return ctx ? ctx->err.c_str() : "null context"; }

VXS_API int vxs_set_stream(vxs_ctx* ctx, void* hip_stream) {
    if (!ctx) return VXS_ERR_INVALID_ARG;
    ctx->stream = hip_stream ? static_cast<hipStream_t>(hip_stream) : ctx->own_stream;
    return VXS_OK;
}

VXS_API void* vxs_get_stream(const vxs_ctx* ctx) { return ctx ? static_cast<void*>(ctx->stream) : nullptr; }

VXS_API int vxs_synchronize(vxs_ctx* ctx) {
    if (!ctx) return VXS_ERR_INVALID_ARG;
    VXS_HIP(ctx, hipSetDevice(ctx->device));
    VXS_HIP(ctx, hipStreamSynchronize(ctx->stream));
    return VXS_OK;
}

VXS_API int vxs_sample(vxs_ctx* ctx, int rows, int vocab, const float* logits, int64_t ld, const int32_t* hist_off,
                       const int32_t* hist_ids, const vxs_params* params, int params_stride, const double* u,
                       int32_t* out_ids, float* out_logits, double* out_probs, uint32_t flags) {
    try {
        int rc = check_shape(ctx, rows, vocab, logits, ld, params, params_stride, out_ids);
        if (rc != VXS_OK) return rc;
        if ((rc = check_flags(ctx, flags)) != VXS_OK) return rc;
        if (rows == 0) return VXS_OK;
        if ((rc = check_params_host(ctx, rows, params, params_stride, u)) != VXS_OK) return rc;
        if ((rc = check_hist_host(ctx, rows, hist_off, hist_ids)) != VXS_OK) return rc;
        VXS_HIP(ctx, hipSetDevice(ctx->device));
        if (polled_call(rows, vocab, flags, out_logits != nullptr, out_probs != nullptr)) {
            vxs::SampleArgs done{};
            const size_t nlog = out_logits ? (size_t)rows * (size_t)vocab : 0;
            VXS_HIP(ctx, ensure_done(ctx, rows, done, nlog));
            rc = stage_and_launch(ctx, rows, vocab, logits, ld, hist_off, hist_ids, params, params_stride, u, false,
                                  false, 0, flags, &done);
            if (rc != VXS_OK) {
                ctx->done_ready = false;
                return rc;
            }
            if ((rc = wait_done(ctx, done.done_seq)) != VXS_OK) return rc;
            std::memcpy(out_ids, done.out_ids, sizeof(int32_t) * (size_t)rows);
            if (nlog) copy_ok_rows(out_logits, done.out_logits, out_ids, rows, sizeof(float) * (size_t)vocab);
            ctx->err.clear();
            return first_row_error(ctx, out_ids, rows);
        }
        rc = stage_and_launch(ctx, rows, vocab, logits, ld, hist_off, hist_ids, params, params_stride, u,
                              out_logits != nullptr, out_probs != nullptr, 0, flags);
        if (rc != VXS_OK) return rc;
        if ((rc = fetch(ctx, out_ids, ctx->d_ids.p, sizeof(int32_t) * (size_t)rows)) != VXS_OK) return rc;
        if (out_logits && (rc = fetch_ok_rows(ctx, out_logits, ctx->d_logits_out.p, out_ids, rows,
                                              sizeof(float) * (size_t)vocab)) != VXS_OK)
            return rc;
        if (out_probs && (rc = fetch(ctx, out_probs, ctx->d_probs_out.p, sizeof(double) * (size_t)rows * vocab)) != VXS_OK)
            return rc;
        ctx->err.clear();
        return first_row_error(ctx, out_ids, rows);
    } catch (const std::exception& e) {
        return fail(ctx, VXS_ERR_INVALID_ARG, e.what());
    } catch (...) {
        return fail(ctx, VXS_ERR_INVALID_ARG, "unknown exception");
    }
}

VXS_API int vxs_sample_noalloc(vxs_ctx* ctx, int rows, int vocab, const float* logits, int64_t ld,
                               const int32_t* hist_off, const int32_t* hist_ids, const vxs_params* params,
                               int params_stride, const double* u, int32_t* out_ids, uint32_t flags) {
    try {
        int rc = check_shape(ctx, rows, vocab, logits, ld, params, params_stride, out_ids);
        if (rc != VXS_OK) return rc;
        if ((rc = check_flags(ctx, flags)) != VXS_OK) return rc;
        if (rows == 0) return VXS_OK;
        if ((rc = check_params_host(ctx, rows, params, params_stride, u)) != VXS_OK) return rc;
        if ((rc = check_hist_host(ctx, rows, hist_off, hist_ids)) != VXS_OK) return rc;
        if (!ctx->noalloc) return fail(ctx, VXS_ERR_HIP, "no fixed scratch on this device");
        // the staged layout of vxs_sample, then the ids, all inside the fixed scratch
        const Layout L = plan(rows, vocab, params_stride, hist_off);
        const size_t ids_at = L.total;
        const size_t need = align_up(ids_at + sizeof(int32_t) * (size_t)rows);
        if (need > vxs::kNoAllocScratchBytes)
            return fail(ctx, VXS_ERR_UNSUPPORTED,
                        "vxs_sample_noalloc: this call stages " + std::to_string(need) + " bytes; the fixed scratch holds " +
                            std::to_string(vxs::kNoAllocScratchBytes));
        // one call at a time per device: the scratch is the device's, not the context's
        std::lock_guard<std::mutex> hold(vxs::noalloc_lock(ctx->device));
        VXS_HIP(ctx, hipSetDevice(ctx->device));
        char* d = static_cast<char*>(ctx->noalloc);
        hipStream_t st = ctx->stream;
        // inputs straight from the caller's memory (no pinned staging)
        if (params_stride <= 1) {
            VXS_HIP(ctx, hipMemcpyAsync(d + L.params, params, sizeof(vxs_params) * (size_t)L.np, hipMemcpyHostToDevice, st));
        } else {
            VXS_HIP(ctx, hipMemcpy2DAsync(d + L.params, sizeof(vxs_params), params, sizeof(vxs_params) * (size_t)params_stride,
                                          sizeof(vxs_params), (size_t)rows, hipMemcpyHostToDevice, st));
        }
        if (u) VXS_HIP(ctx, hipMemcpyAsync(d + L.u, u, sizeof(double) * (size_t)rows, hipMemcpyHostToDevice, st));
        const int32_t* k_hoff = nullptr;
        const int32_t* k_hids = nullptr;
        if (hist_off) {
            // the offsets as given; the ids from hist_off[0] on, so the kernel's base is shifted back
            VXS_HIP(ctx, hipMemcpyAsync(d + L.hoff, hist_off, sizeof(int32_t) * (size_t)(rows + 1), hipMemcpyHostToDevice, st));
            if (L.nh)
                VXS_HIP(ctx, hipMemcpyAsync(d + L.hids, hist_ids + hist_off[0], sizeof(int32_t) * (size_t)L.nh,
                                            hipMemcpyHostToDevice, st));
            k_hoff = reinterpret_cast<const int32_t*>(d + L.hoff);
            k_hids = reinterpret_cast<const int32_t*>(reinterpret_cast<uintptr_t>(d + L.hids) -
                                                      sizeof(int32_t) * (uintptr_t)(int64_t)hist_off[0]);
        }
        if (ld == L.ld_dev) {
            VXS_HIP(ctx, hipMemcpyAsync(d + L.logits, logits, sizeof(float) * ((size_t)(rows - 1) * (size_t)ld + (size_t)vocab),
                                        hipMemcpyHostToDevice, st));
        } else {
            VXS_HIP(ctx, hipMemcpy2DAsync(d + L.logits, sizeof(float) * (size_t)L.ld_dev, logits, sizeof(float) * (size_t)ld,
                                          sizeof(float) * (size_t)vocab, (size_t)rows, hipMemcpyHostToDevice, st));
        }
        vxs::SampleArgs a{};
        a.rows = rows;
        a.vocab = vocab;
        a.ld = L.ld_dev;
        a.logits = reinterpret_cast<const float*>(d + L.logits);
        a.hist_off = k_hoff;
        a.hist_ids = k_hids;
        a.params = reinterpret_cast<const vxs_params*>(d + L.params);
        a.params_stride = params_stride == 0 ? 0 : 1;
        a.u = u ? reinterpret_cast<const double*>(d + L.u) : nullptr;
        a.out_ids = reinterpret_cast<int32_t*>(d + ids_at);
        a.kflags = 0;
        a.path = choose_path_host(flags, rows, vocab, params, params_stride);
        VXS_HIP(ctx, vxs::launch_sample(a, st));
        VXS_HIP(ctx, hipMemcpyAsync(out_ids, d + ids_at, sizeof(int32_t) * (size_t)rows, hipMemcpyDeviceToHost, st));
        VXS_HIP(ctx, hipStreamSynchronize(st));
        ctx->err.clear();
        return first_row_error(ctx, out_ids, rows);
    } catch (...) {
        return fail(ctx, VXS_ERR_INVALID_ARG, "unknown exception");
    }
}

VXS_API int vxs_sample_device(vxs_ctx* ctx, int rows, int vocab, const float* d_logits, int64_t ld,
                              const int32_t* d_hist_off, const int32_t* d_hist_ids, const vxs_params* d_params,
                              int params_stride, const double* d_u, int32_t* d_out_ids, float* d_out_logits,
                              double* d_out_probs, uint32_t flags) {
    try {
        int rc = check_shape(ctx, rows, vocab, d_logits, ld, d_params, params_stride, d_out_ids);
        if (rc != VXS_OK) return rc;
        if ((rc = check_flags(ctx, flags)) != VXS_OK) return rc;
        if (rows == 0) return VXS_OK;
        if (d_hist_off && !d_hist_ids) return fail(ctx, VXS_ERR_INVALID_ARG, "hist_ids is NULL");
        if (params_stride > 1) return fail(ctx, VXS_ERR_INVALID_ARG, "device params_stride must be 0 or 1");
        VXS_HIP(ctx, hipSetDevice(ctx->device));
        vxs::SampleArgs a{};
        a.rows = rows;
        a.vocab = vocab;
        a.ld = ld;
        a.logits = d_logits;
        a.hist_off = d_hist_off;
        a.hist_ids = d_hist_ids;
        a.params = d_params;
        a.params_stride = params_stride;
        a.u = d_u;
        a.out_ids = d_out_ids;
        a.out_logits = d_out_logits;
        a.out_probs = d_out_probs;
        a.kflags = 0;
        a.path = choose_path(flags, rows, vocab);
        VXS_HIP(ctx, vxs::launch_sample(a, ctx->stream));
        ctx->err.clear();
        return VXS_OK;
    } catch (...) {
        return fail(ctx, VXS_ERR_INVALID_ARG, "unknown exception");
    }
}

VXS_API int vxs_sample_stats_device(vxs_ctx* ctx, int rows, int vocab, const float* d_logits, int64_t ld,
                                    const int32_t* d_hist_off, const int32_t* d_hist_ids, const vxs_params* d_params,
                                    int params_stride, const double* d_u, int32_t* d_out_ids, double* d_stats,
                                    double* d_probs, uint32_t flags) {
    try {
        int rc = check_shape(ctx, rows, vocab, d_logits, ld, d_params, params_stride, d_out_ids);
        if (rc != VXS_OK) return rc;
        if ((rc = check_flags(ctx, flags)) != VXS_OK) return rc;
        if (!d_stats) return fail(ctx, VXS_ERR_INVALID_ARG, "stats is NULL");
        if (rows == 0) return VXS_OK;
        if (d_hist_off && !d_hist_ids) return fail(ctx, VXS_ERR_INVALID_ARG, "hist_ids is NULL");
        if (params_stride > 1) return fail(ctx, VXS_ERR_INVALID_ARG, "device params_stride must be 0 or 1");
        VXS_HIP(ctx, hipSetDevice(ctx->device));
        // all-ones bytes: every double NaN, for the rows the one-wave nucleus regime does not sample
        VXS_HIP(ctx, hipMemsetAsync(d_stats, 0xff, sizeof(double) * 4 * (size_t)rows, ctx->stream));
        if (d_probs) VXS_HIP(ctx, hipMemsetAsync(d_probs, 0xff, sizeof(double) * (size_t)rows * vocab, ctx->stream));
        vxs::SampleArgs a{};
        a.rows = rows;
        a.vocab = vocab;
        a.ld = ld;
        a.logits = d_logits;
        a.hist_off = d_hist_off;
        a.hist_ids = d_hist_ids;
        a.params = d_params;
        a.params_stride = params_stride;
        a.u = d_u;
        a.out_ids = d_out_ids;
        a.out_stats = d_stats;
        a.out_stat_probs = d_probs;
        a.kflags = 0;
        a.path = choose_path(flags, rows, vocab);
        VXS_HIP(ctx, vxs::launch_sample(a, ctx->stream));
        ctx->err.clear();
        return VXS_OK;
    } catch (...) {
        return fail(ctx, VXS_ERR_INVALID_ARG, "unknown exception");
    }
}

VXS_API int vxs_apply_repetition_penalty(vxs_ctx* ctx, int rows, int vocab, float* logits, int64_t ld,
                                         const int32_t* hist_off, const int32_t* hist_ids, float penalty) {
    try {
        vxs_params p{};
        p.do_sample = 0;
        p.rep_penalty = penalty;
        p.keep_id = -1;
        p.ban_id = -1;
        int32_t dummy = 0;
        int rc = check_shape(ctx, rows, vocab, logits, ld, &p, 0, &dummy);
        if (rc != VXS_OK) return rc;
        if (rows == 0 || penalty == 1.0f || !hist_off) return VXS_OK;  // Sampler.cs:27
        if ((rc = check_hist_host(ctx, rows, hist_off, hist_ids)) != VXS_OK) return rc;
        VXS_HIP(ctx, hipSetDevice(ctx->device));
        const size_t row_bytes = sizeof(float) * (size_t)vocab;
        if (rows <= kPolledMaxRows && vocab <= vxs::kRowResidentMaxVocab && row_bytes * rows <= kZeroCopyMaxBytes) {
            // completes by polling, the penalised rows written straight into coherent host memory
            vxs::SampleArgs done{};
            VXS_HIP(ctx, ensure_done(ctx, rows, done, (size_t)rows * (size_t)vocab));
            rc = stage_and_launch(ctx, rows, vocab, logits, ld, hist_off, hist_ids, &p, 0, nullptr, false, false,
                                  vxs::KF_STOP_AFTER_PENALTY, VXS_FLAG_PATH_BLOCK, &done);
            if (rc != VXS_OK) {
                ctx->done_ready = false;
                return rc;
            }
            if ((rc = wait_done(ctx, done.done_seq)) != VXS_OK) return rc;
            ctx->err.clear();
            if ((rc = first_row_error(ctx, done.out_ids, rows)) != VXS_OK) return rc;
            for (int r = 0; r < rows; r++)
                std::memcpy(logits + (int64_t)r * ld, reinterpret_cast<const char*>(done.out_logits) + row_bytes * r,
                            row_bytes);
            return VXS_OK;
        }
        rc = stage_and_launch(ctx, rows, vocab, logits, ld, hist_off, hist_ids, &p, 0, nullptr, true, false,
                              vxs::KF_STOP_AFTER_PENALTY, VXS_FLAG_PATH_BLOCK);
        if (rc != VXS_OK) return rc;
        VXS_HIP(ctx, ctx->h_ids.reserve(sizeof(int32_t) * (size_t)rows));
        if ((rc = fetch(ctx, ctx->h_ids.p, ctx->d_ids.p, sizeof(int32_t) * (size_t)rows)) != VXS_OK) return rc;
        ctx->err.clear();
        if ((rc = first_row_error(ctx, static_cast<int32_t*>(ctx->h_ids.p), rows)) != VXS_OK) return rc;
        VXS_HIP(ctx, ctx->h_out.reserve(row_bytes * rows));
        VXS_HIP(ctx, hipMemcpyAsync(ctx->h_out.p, ctx->d_logits_out.p, row_bytes * rows, hipMemcpyDeviceToHost, ctx->stream));
        VXS_HIP(ctx, hipStreamSynchronize(ctx->stream));
        for (int r = 0; r < rows; r++)
            std::memcpy(logits + (int64_t)r * ld, static_cast<char*>(ctx->h_out.p) + row_bytes * r, row_bytes);
        return VXS_OK;
    } catch (...) {
        return fail(ctx, VXS_ERR_INVALID_ARG, "unknown exception");
    }
}

VXS_API int vxs_argmax(vxs_ctx* ctx, int rows, int vocab, const float* logits, int64_t ld, int32_t* out_ids) {
    try {
        vxs_params p{};
        p.do_sample = 0;
        p.rep_penalty = 1.0f;
        p.keep_id = -1;
        p.ban_id = -1;
        // a greedy row of vxs_sample: no history, no draw (polled completion for small calls)
        return vxs_sample(ctx, rows, vocab, logits, ld, nullptr, nullptr, &p, 0, nullptr, out_ids, nullptr, nullptr,
                          VXS_FLAG_NONE);
    } catch (...) {
        return fail(ctx, VXS_ERR_INVALID_ARG, "unknown exception");
    }
}

VXS_API int vxs_history_create(vxs_ctx* ctx, int slots, int cap, vxs_history** out) {
    try {
        if (!ctx) return VXS_ERR_INVALID_ARG;
        if (!out) return fail(ctx, VXS_ERR_INVALID_ARG, "out is NULL");
        *out = nullptr;
        if (slots <= 0 || cap <= 0) return fail(ctx, VXS_ERR_INVALID_ARG, "slots and cap must be positive");
        if ((int64_t)slots * cap > INT32_MAX) return fail(ctx, VXS_ERR_INVALID_ARG, "slots * cap exceeds 2^31 - 1");
        VXS_HIP(ctx, hipSetDevice(ctx->device));
        vxs_history* h = new (std::nothrow) vxs_history();
        if (!h) return fail(ctx, VXS_ERR_INVALID_ARG, "out of host memory");
        h->device = ctx->device;
        h->slots = slots;
        h->cap = cap;
        try {
            h->seeded.assign((size_t)slots, 0);
        } catch (...) {
            delete h;
            return fail(ctx, VXS_ERR_INVALID_ARG, "out of host memory");
        }
        const size_t rng_bytes = sizeof(int32_t) * (size_t)slots * 2 * vxs::kRngWords;
        hipError_t e = hipMalloc(&h->ids, sizeof(int32_t) * (size_t)slots * (size_t)cap);
        if (e == hipSuccess) e = hipMalloc(&h->len, sizeof(int32_t) * (size_t)slots);
        if (e == hipSuccess) e = hipMalloc(&h->rng, rng_bytes);
        if (e == hipSuccess) e = hipMemsetAsync(h->len, 0, sizeof(int32_t) * (size_t)slots, ctx->stream);
        if (e == hipSuccess) e = hipMemsetAsync(h->rng, 0, rng_bytes, ctx->stream);
        if (e == hipSuccess) e = hipMalloc(&h->desc, sizeof(vxs::StoreDesc));
        if (e == hipSuccess) {
            const vxs::StoreDesc d{h->ids, h->len, h->rng, cap, slots};
            e = hipMemcpyAsync(h->desc, &d, sizeof d, hipMemcpyHostToDevice, ctx->stream);
            if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
        }
        if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
        if (e != hipSuccess) {
            vxs_history_destroy(h);
            return hip_fail(ctx, e, "vxs_history_create");
        }
        *out = h;
        ctx->err.clear();
        return VXS_OK;
    } catch (...) {
        return fail(ctx, VXS_ERR_INVALID_ARG, "unknown exception");
    }
}

VXS_API void vxs_history_destroy(vxs_history* h) {
    if (!h) return;
    (void)hipSetDevice(h->device);
    if (h->ids) (void)hipFree(h->ids);
    if (h->len) (void)hipFree(h->len);
    if (h->rng) (void)hipFree(h->rng);
    if (h->desc) (void)hipFree(h->desc);
    delete h;
}

VXS_API int vxs_history_set(vxs_ctx* ctx, vxs_history* h, int slot, const int32_t* ids, int n) {
    try {
        if (!ctx) return VXS_ERR_INVALID_ARG;
        int rc = check_store(ctx, h);
        if (rc != VXS_OK) return rc;
        if ((unsigned)slot >= (unsigned)h->slots) return fail(ctx, VXS_ERR_INVALID_ARG, "slot outside the store");
        if (n < 0 || n > h->cap) return fail(ctx, VXS_ERR_INVALID_ARG, "n outside [0, cap]");
        if (n > 0 && !ids) return fail(ctx, VXS_ERR_INVALID_ARG, "ids is NULL");
        VXS_HIP(ctx, hipSetDevice(ctx->device));
        VXS_HIP(ctx, ctx->h_ids.reserve(sizeof(int32_t) * ((size_t)n + 1)));
        int32_t* st = static_cast<int32_t*>(ctx->h_ids.p);
        st[0] = n;
        if (n) std::memcpy(st + 1, ids, sizeof(int32_t) * (size_t)n);
        if (n)
            VXS_HIP(ctx, hipMemcpyAsync(h->ids + (int64_t)slot * h->cap, st + 1, sizeof(int32_t) * (size_t)n,
                                        hipMemcpyHostToDevice, ctx->stream));
        VXS_HIP(ctx, hipMemcpyAsync(h->len + slot, st, sizeof(int32_t), hipMemcpyHostToDevice, ctx->stream));
        VXS_HIP(ctx, hipStreamSynchronize(ctx->stream));
        ctx->err.clear();
        return VXS_OK;
    } catch (...) {
        return fail(ctx, VXS_ERR_INVALID_ARG, "unknown exception");
    }
}

VXS_API int vxs_history_get(vxs_ctx* ctx, vxs_history* h, int slot, int32_t* ids, int max_ids, int* n) {
    try {
        if (!ctx) return VXS_ERR_INVALID_ARG;
        int rc = check_store(ctx, h);
        if (rc != VXS_OK) return rc;
        if ((unsigned)slot >= (unsigned)h->slots) return fail(ctx, VXS_ERR_INVALID_ARG, "slot outside the store");
        if (max_ids < 0 || (max_ids > 0 && !ids)) return fail(ctx, VXS_ERR_INVALID_ARG, "bad ids / max_ids");
        VXS_HIP(ctx, hipSetDevice(ctx->device));
        int32_t len = 0;
        if ((rc = fetch(ctx, &len, h->len + slot, sizeof(int32_t))) != VXS_OK) return rc;
        len = std::min(std::max(len, 0), h->cap);
        const int k = std::min(len, max_ids);
        if (k && (rc = fetch(ctx, ids, h->ids + (int64_t)slot * h->cap, sizeof(int32_t) * (size_t)k)) != VXS_OK)
            return rc;
        if (n) *n = len;
        ctx->err.clear();
        return VXS_OK;
    } catch (...) {
        return fail(ctx, VXS_ERR_INVALID_ARG, "unknown exception");
    }
}

VXS_API int vxs_history_seed(vxs_ctx* ctx, vxs_history* h, int slot, int32_t seed) {
    try {
        if (!ctx) return VXS_ERR_INVALID_ARG;
        int rc = check_store(ctx, h);
        if (rc != VXS_OK) return rc;
        if ((unsigned)slot >= (unsigned)h->slots) return fail(ctx, VXS_ERR_INVALID_ARG, "slot outside the store");
        VXS_HIP(ctx, hipSetDevice(ctx->device));
        VXS_HIP(ctx, ctx->h_ids.reserve(sizeof(int32_t) * 2 * vxs::kRngWords));
        int32_t* st = static_cast<int32_t*>(ctx->h_ids.p);
        dotnet_seed(seed, st);
        dotnet_seed((int32_t)((uint32_t)seed + 1u), st + vxs::kRngWords);  // Seed + 1, unchecked
        VXS_HIP(ctx, hipMemcpyAsync(h->rng + (int64_t)slot * 2 * vxs::kRngWords, st, sizeof(int32_t) * 2 * vxs::kRngWords,
                                    hipMemcpyHostToDevice, ctx->stream));
        VXS_HIP(ctx, hipStreamSynchronize(ctx->stream));
        h->seeded[slot] = 1;
        ctx->err.clear();
        return VXS_OK;
    } catch (...) {
        return fail(ctx, VXS_ERR_INVALID_ARG, "unknown exception");
    }
}

VXS_API int vxs_history_draw(vxs_ctx* ctx, vxs_history* h, int slot, int stream, int n, double* out) {
    try {
        if (!ctx) return VXS_ERR_INVALID_ARG;
        int rc = check_store(ctx, h);
        if (rc != VXS_OK) return rc;
        if ((unsigned)slot >= (unsigned)h->slots) return fail(ctx, VXS_ERR_INVALID_ARG, "slot outside the store");
        if (stream != 0 && stream != 1) return fail(ctx, VXS_ERR_INVALID_ARG, "stream must be 0 or 1");
        if (n < 0 || (n > 0 && !out)) return fail(ctx, VXS_ERR_INVALID_ARG, "bad n / out");
        if (!h->seeded[slot]) return fail(ctx, VXS_ERR_INVALID_ARG, "slot's generators are not seeded");
        if (n == 0) return VXS_OK;
        VXS_HIP(ctx, hipSetDevice(ctx->device));
        VXS_HIP(ctx, ctx->d_draw.reserve(sizeof(double) * (size_t)n));
        VXS_HIP(ctx, vxs::launch_draw_sequence(h->rng + ((int64_t)slot * 2 + stream) * vxs::kRngWords, n,
                                               static_cast<double*>(ctx->d_draw.p), ctx->stream));
        if ((rc = fetch(ctx, out, ctx->d_draw.p, sizeof(double) * (size_t)n)) != VXS_OK) return rc;
        ctx->err.clear();
        return VXS_OK;
    } catch (...) {
        return fail(ctx, VXS_ERR_INVALID_ARG, "unknown exception");
    }
}

VXS_API int vxs_sample_batch(vxs_ctx* ctx, vxs_history* h, int rows, int vocab, const float* logits, int64_t ld,
                             const int32_t* slots, int append, const vxs_params* params, int params_stride,
                             const double* u, int32_t* out_ids, uint32_t flags) {
    try {
        int rc = check_shape(ctx, rows, vocab, logits, ld, params, params_stride, out_ids);
        if (rc != VXS_OK) return rc;
        if ((rc = check_batch_flags(ctx, flags)) != VXS_OK) return rc;
        if ((rc = check_store(ctx, h)) != VXS_OK) return rc;
        if (rows == 0) return VXS_OK;
        const int stream = rng_stream_of(flags);
        if (stream < 0 && (rc = check_params_host(ctx, rows, params, params_stride, u)) != VXS_OK) return rc;
        if ((rc = check_slots_host(ctx, h, rows, slots)) != VXS_OK) return rc;
        if (stream >= 0)
            for (int r = 0; r < rows; r++)
                if (!h->seeded[slots[r]])
                    return fail(ctx, VXS_ERR_INVALID_ARG, "row " + std::to_string(r) + ": slot's generators are not seeded");
        VXS_HIP(ctx, hipSetDevice(ctx->device));
        ResidentCall res;
        res.store = h;
        res.slots = slots;
        res.append = append != 0;
        res.rng_stream = stream;
        if (polled_call(rows, vocab, flags, false, false)) {
            vxs::SampleArgs done{};
            VXS_HIP(ctx, ensure_done(ctx, rows, done));
            res.done = &done;
            rc = stage_and_launch(ctx, rows, vocab, logits, ld, nullptr, nullptr, params, params_stride, u, false,
                                  false, 0, flags, nullptr, &res);
            if (rc != VXS_OK) {
                ctx->done_ready = false;
                return rc;
            }
            if ((rc = wait_done(ctx, done.done_seq)) != VXS_OK) return rc;
            std::memcpy(out_ids, done.out_ids, sizeof(int32_t) * (size_t)rows);
            ctx->err.clear();
            return first_row_error(ctx, out_ids, rows);
        }
        rc = stage_and_launch(ctx, rows, vocab, logits, ld, nullptr, nullptr, params, params_stride, u, false, false,
                              0, flags, nullptr, &res);
        if (rc != VXS_OK) return rc;
        if ((rc = fetch(ctx, out_ids, ctx->d_ids.p, sizeof(int32_t) * (size_t)rows)) != VXS_OK) return rc;
        ctx->err.clear();
        return first_row_error(ctx, out_ids, rows);
    } catch (const std::exception& e) {
        return fail(ctx, VXS_ERR_INVALID_ARG, e.what());
    } catch (...) {
        return fail(ctx, VXS_ERR_INVALID_ARG, "unknown exception");
    }
}

VXS_API int vxs_sample_batch_device(vxs_ctx* ctx, vxs_history* h, int rows, int vocab, const float* d_logits,
                                    int64_t ld, const int32_t* d_slots, int append, const vxs_params* d_params,
                                    int params_stride, const double* d_u, int32_t* d_out_ids, uint32_t flags) {
    try {
        int rc = check_shape(ctx, rows, vocab, d_logits, ld, d_params, params_stride, d_out_ids);
        if (rc != VXS_OK) return rc;
        if ((rc = check_batch_flags(ctx, flags)) != VXS_OK) return rc;
        if ((rc = check_store(ctx, h)) != VXS_OK) return rc;
        if (rows == 0) return VXS_OK;
        if (!d_slots) return fail(ctx, VXS_ERR_INVALID_ARG, "slots is NULL");
        if (params_stride > 1) return fail(ctx, VXS_ERR_INVALID_ARG, "device params_stride must be 0 or 1");
        VXS_HIP(ctx, hipSetDevice(ctx->device));
        vxs::SampleArgs a{};
        a.rows = rows;
        a.vocab = vocab;
        a.ld = ld;
        a.logits = d_logits;
        a.params = d_params;
        a.params_stride = params_stride;
        a.u = d_u;
        a.out_ids = d_out_ids;
        a.kflags = 0;
        a.path = choose_path(flags, rows, vocab);
        set_resident(a, h, d_slots, append != 0, rng_stream_of(flags));
        VXS_HIP(ctx, vxs::launch_sample(a, ctx->stream));
        ctx->err.clear();
        return VXS_OK;
    } catch (...) {
        return fail(ctx, VXS_ERR_INVALID_ARG, "unknown exception");
    }
}

VXS_API int vxs_embed_device(vxs_ctx* ctx, int rows, int hidden, const int32_t* d_ids, const uint16_t* d_table,
                             int vocab, float* d_out, int64_t ld_out, int add, int32_t* d_status) {
    try {
        if (!ctx) return VXS_ERR_INVALID_ARG;
        if (rows < 0 || hidden <= 0 || vocab <= 0 || ld_out < hidden)
            return fail(ctx, VXS_ERR_INVALID_ARG, "bad rows, hidden, vocab or ld_out");
        if (rows == 0) return VXS_OK;
        if (!d_ids || !d_table || !d_out || !d_status) return fail(ctx, VXS_ERR_INVALID_ARG, "null pointer");
        VXS_HIP(ctx, hipSetDevice(ctx->device));
        vxs::EmbedArgs a{};
        a.rows = rows;
        a.hidden = hidden;
        a.vocab = vocab;
        a.add = add != 0;
        a.vec = hidden % 4 == 0 && ld_out % 4 == 0 && ((uintptr_t)d_table & 7u) == 0 && ((uintptr_t)d_out & 15u) == 0;
        a.ids = d_ids;
        a.table = d_table;
        a.out = d_out;
        a.ld_out = ld_out;
        a.status = d_status;
        VXS_HIP(ctx, vxs::launch_embed(a, ctx->stream));
        ctx->err.clear();
        return VXS_OK;
    } catch (...) {
        return fail(ctx, VXS_ERR_INVALID_ARG, "unknown exception");
    }
}

VXS_API int vxs_frame_embed_device(vxs_ctx* ctx, int rows, int groups, int hidden, const int32_t* d_codes,
                                   int64_t ld_codes, int64_t group_stride, const uint16_t* d_codec_table, int vocab,
                                   const uint16_t* d_cp_tables, int cp_vocab, const float* d_addend,
                                   int64_t ld_addend, float* d_out, int64_t ld_out, int32_t* d_status) {
    try {
        if (!ctx) return VXS_ERR_INVALID_ARG;
        if (rows < 0 || groups < 1 || hidden <= 0 || vocab <= 0 || ld_codes < 0 || group_stride < 0 || ld_out < hidden)
            return fail(ctx, VXS_ERR_INVALID_ARG, "bad rows, groups, hidden, vocab, ld_codes, group_stride or ld_out");
        if (groups > 1 && (cp_vocab <= 0 || !d_cp_tables))
            return fail(ctx, VXS_ERR_INVALID_ARG, "code predictor tables missing");
        if (d_addend && ld_addend < hidden) return fail(ctx, VXS_ERR_INVALID_ARG, "ld_addend < hidden");
        if (rows == 0) return VXS_OK;
        if (!d_codes || !d_codec_table || !d_out || !d_status) return fail(ctx, VXS_ERR_INVALID_ARG, "null pointer");
        VXS_HIP(ctx, hipSetDevice(ctx->device));
        vxs::FrameEmbedArgs a{};
        a.rows = rows;
        a.groups = groups;
        a.hidden = hidden;
        a.vocab = vocab;
        a.cp_vocab = cp_vocab;
        a.vec = hidden % 4 == 0 && ld_out % 4 == 0 && ((uintptr_t)d_codec_table & 7u) == 0 &&
                ((uintptr_t)d_cp_tables & 7u) == 0 && ((uintptr_t)d_out & 15u) == 0 &&
                (!d_addend || (ld_addend % 4 == 0 && ((uintptr_t)d_addend & 15u) == 0));
        a.codes = d_codes;
        a.ld_codes = ld_codes;
        a.group_stride = group_stride;
        a.codec_table = d_codec_table;
        a.cp_tables = d_cp_tables;
        a.addend = d_addend;
        a.ld_addend = ld_addend;
        a.out = d_out;
        a.ld_out = ld_out;
        a.status = d_status;
        VXS_HIP(ctx, vxs::launch_frame_embed(a, ctx->stream));
        ctx->err.clear();
        return VXS_OK;
    } catch (...) {
        return fail(ctx, VXS_ERR_INVALID_ARG, "unknown exception");
    }
}

VXS_API int vxs_head_device(vxs_ctx* ctx, int rows, int k, int n, const float* d_x, int64_t ldx, const uint16_t* d_w,
                            int64_t ldw, float* d_out, int64_t ldo) {
    try {
        if (!ctx) return VXS_ERR_INVALID_ARG;
        if (rows < 0 || k <= 0 || n <= 0 || ldx < k || ldw < k || ldo < n)
            return fail(ctx, VXS_ERR_INVALID_ARG, "bad rows, k, n or leading dimensions");
        if (k > 2048 || k % 8 != 0 || ldw % 8 != 0 || ldx % 4 != 0 || ((uintptr_t)d_x & 15u) || ((uintptr_t)d_w & 15u))
            return fail(ctx, VXS_ERR_UNSUPPORTED,
                        "head needs k <= 2048, k and ldw multiples of 8, ldx a multiple of 4, 16-byte aligned x and w");
        if (rows == 0) return VXS_OK;
        if (!d_x || !d_w || !d_out) return fail(ctx, VXS_ERR_INVALID_ARG, "null pointer");
        VXS_HIP(ctx, hipSetDevice(ctx->device));
        vxs::HeadArgs a{rows, k, n, d_x, ldx, d_w, ldw, d_out, ldo, 0, nullptr, nullptr};
        VXS_HIP(ctx, vxs::launch_head(a, ctx->stream));
        ctx->err.clear();
        return VXS_OK;
    } catch (...) {
        return fail(ctx, VXS_ERR_INVALID_ARG, "unknown exception");
    }
}

VXS_API int vxs_head_int8_device(vxs_ctx* ctx, int rows, int k, int n, const float* d_x, int64_t ldx, const int8_t* d_q,
                                 int64_t ldq, const float* d_scale, float* d_out, int64_t ldo) {
    try {
        if (!ctx) return VXS_ERR_INVALID_ARG;
        if (rows < 0 || k <= 0 || n <= 0 || ldx < k || ldq < k || ldo < n)
            return fail(ctx, VXS_ERR_INVALID_ARG, "bad rows, k, n or leading dimensions");
        if (k > 2048 || k % 8 != 0 || ldq % 8 != 0 || ldx % 4 != 0 || ((uintptr_t)d_x & 15u) || ((uintptr_t)d_q & 15u))
            return fail(ctx, VXS_ERR_UNSUPPORTED,
                        "int8 head needs k <= 2048, k and ldq multiples of 8, ldx a multiple of 4, 16-byte aligned x and q");
        if (rows == 0) return VXS_OK;
        if (!d_x || !d_q || !d_scale || !d_out) return fail(ctx, VXS_ERR_INVALID_ARG, "null pointer");
        VXS_HIP(ctx, hipSetDevice(ctx->device));
        vxs::HeadArgs a{rows, k, n, d_x, ldx, nullptr, ldq, d_out, ldo, 0, d_q, d_scale};
        VXS_HIP(ctx, vxs::launch_head(a, ctx->stream));
        ctx->err.clear();
        return VXS_OK;
    } catch (...) {
        return fail(ctx, VXS_ERR_INVALID_ARG, "unknown exception");
    }
}

VXS_API int vxs_head_pack_int8_device(vxs_ctx* ctx, int k, int n, const uint16_t* d_w, int64_t ldw, int8_t* d_q,
                                      int64_t ldq, float* d_scale) {
    try {
        if (!ctx) return VXS_ERR_INVALID_ARG;
        if (k <= 0 || n <= 0 || ldw < k || ldq < k) return fail(ctx, VXS_ERR_INVALID_ARG, "bad k, n or leading dimensions");
        if (!d_w || !d_q || !d_scale) return fail(ctx, VXS_ERR_INVALID_ARG, "null pointer");
        VXS_HIP(ctx, hipSetDevice(ctx->device));
        VXS_HIP(ctx, vxs::launch_head_pack_int8(k, n, d_w, ldw, d_q, ldq, d_scale, ctx->stream));
        ctx->err.clear();
        return VXS_OK;
    } catch (...) {
        return fail(ctx, VXS_ERR_INVALID_ARG, "unknown exception");
    }
}

}  // extern "C"
