// vxs_internal.h — shared declarations between the HIP kernels and the C-ABI layer.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <mutex>

#include "../../include/vxs_sampler.h"

namespace vxs {

// Kernel-side flags (not part of the public ABI).
enum : uint32_t {
    KF_STOP_AFTER_PENALTY = 1u,  // apply penalty (+ write-back) only: ApplyRepetitionPenalty
    KF_APPEND = 2u,              // resident store: append each sampled id to its row's slot
    KF_RNG = 4u,                 // resident store: draw the uniforms from the slots' generators
    KF_RNG_SUB = 8u,             //   the code predictor's (else the talker's)
};

// A resident store as the kernels see it (vxs_history, one copy in device memory per store):
// ids [slots][cap], lengths [slots], generators [slots][2][kRngWords].
struct StoreDesc {
    int32_t* ids;
    int32_t* len;
    int32_t* rng;
    int cap;
    int slots;
};

struct SampleArgs {
    int rows;
    int vocab;
    int64_t ld;
    const float* logits;
    const int32_t* hist_off;
    const int32_t* hist_ids;
    // Resident histories (vxs_history), used instead of hist_off when hist_len is set: row r reads
    // slot s = hist_slot[r], the ids hist_ids[s * hist_cap, s * hist_cap + min(hist_len[s], hist_cap)).
    // A slot outside [0, hist_slots) reads as empty, and put_id then fails the row.
    const int32_t* hist_slot;
    const int32_t* hist_len;
    int hist_cap;
    int hist_slots;
    // With a resident store (`store`, in device memory), the row's step ends in the kernel
    // (put_id): with KF_APPEND the slot takes the sampled id, and with KF_RNG a sampled row's
    // uniform is the next NextDouble() of generator 2 * slot + (KF_RNG_SUB ? 1 : 0) instead of u[r]
    // (read by row_uniform, advanced once by put_id).
    const struct StoreDesc* store;
    const vxs_params* params;
    int params_stride;
    const double* u;
    int32_t* out_ids;
    float* out_logits;   // optional [rows][vocab]
    double* out_probs;   // optional [rows][vocab]
    // Optional [rows][4] (parity/debug): for a row the one-wave nucleus regime samples, its kept
    // fraction of the mass, smallest kept probability, kept count and 0; other rows are untouched.
    double* out_stats;
    // Optional [rows][vocab] with out_stats: for the same rows, every entry's final probability
    // (its mass over the kept mass; 0 for removed entries).
    double* out_stat_probs;
    uint32_t kflags;
    int path;            // kPathBlock or kPathQuad
    // Host-visible completion for small host calls (one workgroup per row): after its row, every
    // workgroup counts itself in *done_count (device memory, zero between calls); the last one
    // resets the count and stores done_seq to *done_flag (pinned host memory), which the host
    // polls instead of synchronising the stream. Unused when done_flag is null.
    int32_t* done_count;
    int32_t* done_flag;
    int32_t done_seq;
    // One-wave kernel launch stagger (set by its launcher): workgroups from stagger_from on start
    // their loads after stagger_sleeps x 2048 cycles of s_sleep.
    int stagger_from;
    int stagger_sleeps;
    // A single-row host call's scalars by value (row_direct = 1, one-workgroup kernel): the options,
    // the history range and the uniform, so the kernel reads none of them from host memory over
    // PCIe before its history ids (or at the draw).
    int row_direct;
    int direct_h0, direct_h1;
    double direct_u;
    vxs_params direct_params;
};

enum : int {
    kPathBlock = 0,  // one 256-thread workgroup per row
    kPathQuad = 1,   // one wave per row first, four rows per workgroup (vocab <= kWaveMaxVocab)
};

// Largest vocabulary handled by the row-resident kernels (a row stays in VGPRs).
constexpr int kRowResidentMaxVocab = 8192;
// Largest vocabulary of the one-wave-per-row fast path (vxs_wave.h).
constexpr int kWaveMaxVocab = 3072;
// Largest top-k the one-wave path samples itself (its final candidates are one per lane).
constexpr int kWaveMaxTopK = 64;
// Largest vocabulary of the streaming kernel (vxs_wide.hip); its history bitmap lives in LDS.
constexpr int kWideMaxVocab = 1 << 19;

// Whether row histories are given (CSR offsets or a resident store).
__device__ __forceinline__ bool has_history(const SampleArgs& a) {
    return a.hist_off != nullptr || a.hist_len != nullptr;
}

// The history of row r: ids a.hist_ids[h0, h1). Wave-uniform (scalar loads).
struct HistRange {
    int h0, h1;
};
__device__ __forceinline__ HistRange history_range(const SampleArgs& a, int r) {
    if (a.row_direct) return {a.direct_h0, a.direct_h1};
    if (!a.hist_len) return {a.hist_off[r], a.hist_off[r + 1]};
    const int s = a.hist_slot[r];
    const bool ok = (unsigned)s < (unsigned)a.hist_slots;
    const int h0 = ok ? s * a.hist_cap : 0;
    const int n = ok ? a.hist_len[s] : 0;
    return {h0, h0 + min(max(n, 0), a.hist_cap)};
}

// Per-sequence generators of a resident store: .NET's seeded System.Random state, kRngWords int32
// per generator (SeedArray[1..55] at [1..55], inext at [56], inextp at [57]), two per slot (the
// talker's at 2s, the code predictor's at 2s + 1).
constexpr int kRngWords = 64;

// The next InternalSample() of generator state `st` (Random.InternalSample with C#'s wrapping int
// arithmetic): the value and the table slot it replaces. Nothing is written.
struct RngStep {
    int32_t v;
    int i, j;
};
__device__ __forceinline__ RngStep rng_peek(const int32_t* st) {
    constexpr int32_t kMbig = 0x7FFFFFFF;
    int i = st[56] + 1;
    if (i >= 56) i = 1;
    int j = st[57] + 1;
    if (j >= 56) j = 1;
    int32_t v = (int32_t)((uint32_t)st[i] - (uint32_t)st[j]);
    if (v == kMbig) v--;
    if (v < 0) v = (int32_t)((uint32_t)v + (uint32_t)kMbig);
    return {v, i, j};
}
__device__ __forceinline__ void rng_commit(int32_t* st, const RngStep& t) {
    st[t.i] = t.v;
    st[56] = t.i;
    st[57] = t.j;
}
// NextDouble() = InternalSample() * (1.0 / int.MaxValue) (Sampler.cs:77).
__device__ __forceinline__ double rng_double(int32_t v) { return (double)v * (1.0 / 2147483647.0); }

// The uniform row r's draw uses: u[r], or with a resident store's generators the next NextDouble()
// of its slot's generator, read without advancing it (put_id advances it once for the row). Any
// number of threads may call it before the row's put_id. 0 for a slot outside the store.
__device__ __forceinline__ int32_t* slot_rng(const SampleArgs& a, const StoreDesc& d, int s) {
    return d.rng + ((int64_t)s * 2 + ((a.kflags & KF_RNG_SUB) ? 1 : 0)) * kRngWords;
}
__device__ __forceinline__ double row_uniform(const SampleArgs& a, int r) {
    if (a.kflags & KF_RNG) {
        const StoreDesc d = *a.store;
        const int s = a.hist_slot[r];
        if ((unsigned)s >= (unsigned)d.slots) return 0.0;
        return rng_double(rng_peek(slot_rng(a, d, s)).v);
    }
    if (a.row_direct) return a.direct_u;
    return a.u ? a.u[r] : 0.0;
}

// The one store of row r's result, by one thread after every thread of the row has taken its
// uniform. With a resident store it also ends the row's step (the order of the batched
// generator's loop, TalkerGenerator.cs:369-374): a row whose slot lies outside the store fails with
// VXS_ERR_INVALID_ARG; a sampled row advances its slot's generator (one NextDouble per sampled
// Select, whatever the outcome, Sampler.cs:77); with `append` a sampled id joins the slot's
// history (History.Add), or the row fails with VXS_ERR_HISTORY_FULL when the slot is full.
__device__ __forceinline__ void put_id(const SampleArgs& a, int r, int id) {
    if (a.store) {  // the descriptor is read here, at the row's end
        const StoreDesc d = *a.store;
        const int s = a.hist_slot[r];
        if ((unsigned)s >= (unsigned)d.slots) {
            id = VXS_ERR_INVALID_ARG;
        } else {
            if ((a.kflags & KF_RNG) && a.params[(int64_t)r * a.params_stride].do_sample) {
                int32_t* st = slot_rng(a, d, s);
                rng_commit(st, rng_peek(st));
            }
            if ((a.kflags & KF_APPEND) && id >= 0) {
                const int n = d.len[s];
                if ((unsigned)n >= (unsigned)d.cap) {
                    id = VXS_ERR_HISTORY_FULL;
                } else {
                    d.ids[(int64_t)s * d.cap + n] = id;
                    d.len[s] = n + 1;
                }
            }
        }
    }
    a.out_ids[r] = id;
}

// Embedding of sampled ids (vxs_embed.hip). `vec`: hidden % 4 == 0 and every base pointer and
// leading dimension allows 8-byte bf16 and 16-byte fp32 accesses. status[r] = 0 or
// VXS_ERR_ID_OUT_OF_RANGE (the row is then not written).
struct EmbedArgs {
    int rows, hidden, vocab, add, vec;
    const int32_t* ids;
    const uint16_t* table;  // [vocab][hidden] bf16
    float* out;             // [rows][ld_out]
    int64_t ld_out;
    int32_t* status;
};
struct FrameEmbedArgs {
    int rows, groups, hidden, vocab, cp_vocab, vec;
    const int32_t* codes;  // code g of row r at codes[r * ld_codes + g * group_stride]
    int64_t ld_codes, group_stride;
    const uint16_t* codec_table;  // [vocab][hidden] bf16: codebook 0
    const uint16_t* cp_tables;    // [groups - 1][cp_vocab][hidden] bf16: codebooks 1..groups-1
    const float* addend;          // optional [rows][ld_addend], added last
    int64_t ld_addend;
    float* out;
    int64_t ld_out;
    int32_t* status;
};
hipError_t launch_embed(const EmbedArgs& a, hipStream_t stream);

// Logit heads (vxs_head.hip): out[r][n] = sum_k x[r][k] * W[n][k], W bf16 [n][ldw].
// k <= 2048, k % 8 == 0, ldw % 8 == 0, ldx % 4 == 0, x and w 16-byte aligned.
struct HeadArgs {
    int rows, k, n;
    const float* x;
    int64_t ldx;
    const uint16_t* w;    // bf16 weight [n][ldw], or null for the int8 form
    int64_t ldw;          // leading dimension of w or q, in elements
    float* out;
    int64_t ldo;
    int row_group;        // rows per workgroup (set by the launcher)
    const int8_t* q;      // int8 weight [n][ldw] (WeightPrecision.Int8), or null
    const float* scale;   // its per-output scale [n]
};
hipError_t launch_head(const HeadArgs& a, hipStream_t stream);
// int8 packing of a bf16 weight: q[n][ldq], scale[n] (PackedMatrix.FromBf16LinearInt8).
hipError_t launch_head_pack_int8(int k, int n, const uint16_t* w, int64_t ldw, int8_t* q, int64_t ldq, float* scale,
                                 hipStream_t stream);
hipError_t launch_frame_embed(const FrameEmbedArgs& a, hipStream_t stream);

// Fixed device scratch of vxs_sample_noalloc (vxs_noalloc.hip): its size, and its device address on
// `device`, which must be the current device (looked up once per device, then cached).
constexpr size_t kNoAllocScratchBytes = size_t(16) << 20;
hipError_t noalloc_scratch(int device, void** out);
// The lock a call holds while it uses `device`'s scratch (device as accepted by noalloc_scratch).
std::mutex& noalloc_lock(int device);

// Enqueue the sampler on `stream`. Returns hipSuccess or the launch error.
hipError_t launch_sample(const SampleArgs& a, hipStream_t stream);
hipError_t launch_sample_wide(const SampleArgs& a, hipStream_t stream);
// n successive NextDouble() of one generator into out[0..n) (one thread; a check and debug aid).
hipError_t launch_draw_sequence(int32_t* state, int n, double* out, hipStream_t stream);

}  // namespace vxs
