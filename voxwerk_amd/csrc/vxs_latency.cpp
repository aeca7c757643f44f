// vxs_latency.cpp — host-to-host latency of vxs_sample through the C ABI, timed in native code (the
// way a P/Invoke caller sees it: host logits in, host id out, no interpreter in between).
//
// usage: vxs_latency <input file> <iterations> [steps]
// input file (little-endian): int32 rows, int32 vocab, int32 hist_len, then rows*vocab float32 logits,
// rows*hist_len int32 history ids, rows vxs_params, rows float64 uniforms.
// With `steps` S > 1 the rows are S consecutive blocks of rows / S, one call each in order (the
// dependent steps of a frame, e.g. the 15 code-predictor stages of TalkerGenerator.cs:262-269), and
// an iteration is one frame of S calls.
// output: one JSON line {"p50_us": .., "p99_us": .., "iters": .., "id0": ..} per call, plus
// "frame_p50_us", "frame_p99_us", "steps" when S > 1.
//
// usage: vxs_latency --binding-frame <frames> [writeback]
// One frame of single-sequence generation (TalkerGenerator.Generate, TalkerGenerator.cs:241-272) as the
// C# binding issues it: one SelectTalker (1 x 3072: penalty over the sequence's history, suppression of
// the last 1024 ids except EOS, EOS ban for the first two frames, draw) and 15 Select (1 x 2048, top-k
// 50, T 0.9, draw), each one synchronous vxs_sample. With "writeback", Select also writes the row back
// into the caller's span (the reference's in-place Select); by default it does not, as no caller reads
// the span after Select. Output {"p50_us": per call, "talker_p50_us", "select_p50_us", "frame_p50_us", ..}.
//
// usage: vxs_latency --frame <rows> <iterations> [serial]
// One frame step of batched generation (TalkerGenerator.GenerateBatch, TalkerGenerator.cs:362-426)
// over `rows` sequences: the talker stage (rows x 3072, penalty over resident histories, suppression,
// append) and 15 code-predictor stages (rows x 2048), each one batched call. With "serial", the same
// work as the reference's per-row loops: one single-row call per sequence and stage, histories
// passed from the host. Synthetic logits; output {"p50_us": .., "p99_us": .., "iters": .., "calls": ..}.
#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>

#include "vxs_sampler.h"

namespace {

constexpr int kTalkerVocab = 3072, kCpVocab = 2048, kGroups = 16, kEos = 2150;

// xorshift64* in [0, 1)
struct Rng {
    uint64_t s;
    double next() {
        s ^= s >> 12;
        s ^= s << 25;
        s ^= s >> 27;
        return (double)((s * 0x2545F4914F6CDD1DULL) >> 11) * 0x1.0p-53;
    }
};

int frame_mode(int rows, int iters, bool serial) {
    Rng rng{0x9E3779B97F4A7C15ULL};
    std::vector<float> talker((size_t)rows * kTalkerVocab), cp((size_t)kGroups * rows * kCpVocab);
    for (float& x : talker) x = (float)(6.0 * rng.next() - 3.0);
    for (float& x : cp) x = (float)(6.0 * rng.next() - 3.0);
    const vxs_params tp{1, 50, 1.0f, 0.9f, 1.05f, kTalkerVocab - 1024, kTalkerVocab, kEos, -1};
    const vxs_params cpp{1, 50, 1.0f, 0.9f, 1.0f, 0, 0, -1, -1};
    std::vector<vxs_params> tps(rows, tp), cps(rows, cpp);
    std::vector<double> u(rows);
    std::vector<int32_t> ids(rows), slots(rows);
    for (int r = 0; r < rows; r++) slots[r] = r;
    const int warm = 50, total = warm + iters;

    vxs_ctx* ctx = nullptr;
    if (vxs_create(&ctx, 0, rows, kTalkerVocab, 0) != VXS_OK) {
        std::fprintf(stderr, "vxs_create failed\n");
        return 1;
    }
    vxs_history* store = nullptr;
    if (vxs_history_create(ctx, rows, total + 1, &store) != VXS_OK) {
        std::fprintf(stderr, "vxs_history_create failed: %s\n", vxs_last_error(ctx));
        vxs_destroy(ctx);
        return 1;
    }
    std::vector<std::vector<int32_t>> hist(rows);  // host histories of the serial loop
    long calls = 0;
    auto step = [&]() -> int {
        for (int r = 0; r < rows; r++) u[r] = rng.next();
        int rc;
        if (!serial) {
            rc = vxs_sample_batch(ctx, store, rows, kTalkerVocab, talker.data(), kTalkerVocab, slots.data(), 1,
                                  tps.data(), 1, u.data(), ids.data(), 0);
            calls++;
            for (int g = 1; g < kGroups && rc == VXS_OK; g++, calls++) {
                for (int r = 0; r < rows; r++) u[r] = rng.next();
                rc = vxs_sample(ctx, rows, kCpVocab, cp.data() + (size_t)g * rows * kCpVocab, kCpVocab, nullptr,
                                nullptr, cps.data(), 1, u.data(), ids.data(), nullptr, nullptr, 0);
            }
            return rc;
        }
        for (int r = 0; r < rows; r++, calls++) {
            const int32_t off[2] = {0, (int32_t)hist[r].size()};
            int32_t id = 0;
            rc = vxs_sample(ctx, 1, kTalkerVocab, talker.data() + (size_t)r * kTalkerVocab, kTalkerVocab, off,
                            hist[r].data(), &tp, 0, &u[r], &id, nullptr, nullptr, 0);
            if (rc != VXS_OK) return rc;
            hist[r].push_back(id);
        }
        for (int g = 1; g < kGroups; g++)
            for (int r = 0; r < rows; r++, calls++) {
                const double ur = rng.next();
                int32_t id = 0;
                rc = vxs_sample(ctx, 1, kCpVocab, cp.data() + ((size_t)g * rows + r) * kCpVocab, kCpVocab, nullptr,
                                nullptr, &cpp, 0, &ur, &id, nullptr, nullptr, 0);
                if (rc != VXS_OK) return rc;
            }
        return VXS_OK;
    };
    std::vector<double> t;
    int rc = VXS_OK;
    for (int i = 0; i < total && rc == VXS_OK; i++) {
        const auto a = std::chrono::steady_clock::now();
        rc = step();
        if (i >= warm) t.push_back(std::chrono::duration<double, std::micro>(std::chrono::steady_clock::now() - a).count());
    }
    if (rc != VXS_OK) std::fprintf(stderr, "sampling failed: %s\n", vxs_last_error(ctx));
    vxs_history_destroy(store);
    vxs_destroy(ctx);
    if (rc != VXS_OK) return 1;
    std::sort(t.begin(), t.end());
    std::printf("{\"p50_us\": %.2f, \"p99_us\": %.2f, \"iters\": %d, \"calls_per_frame\": %ld}\n", t[t.size() / 2],
                t[(size_t)(t.size() * 0.99)], iters, calls / total);
    return 0;
}

int binding_frame_mode(int frames, bool writeback) {
    Rng rng{0xD1B54A32D192ED03ULL};
    constexpr int kRot = 8;  // distinct synthetic rows per stage, used in turn
    std::vector<float> talker((size_t)kRot * kTalkerVocab), cp((size_t)kRot * kCpVocab), span(kCpVocab);
    for (float& x : talker) x = (float)(6.0 * rng.next() - 3.0);
    for (float& x : cp) x = (float)(6.0 * rng.next() - 3.0);
    const vxs_params cpp{1, 50, 1.0f, 0.9f, 1.0f, 0, 0, -1, -1};
    vxs_ctx* ctx = nullptr;
    if (vxs_create(&ctx, 0, 64, kTalkerVocab, 1 << 16) != VXS_OK) {
        std::fprintf(stderr, "vxs_create failed\n");
        return 1;
    }
    std::vector<int32_t> history;
    std::vector<double> tt, ts, tf;
    const int warm = 50;
    int rc = VXS_OK;
    for (int f = 0; f < warm + frames && rc == VXS_OK; f++) {
        const int t = f % 256;  // a sequence of 256 frames, then a new one
        if (t == 0) history.clear();
        const vxs_params tp{1, 50, 1.0f, 0.9f, 1.05f, kTalkerVocab - 1024, kTalkerVocab, kEos, t < 2 ? kEos : -1};
        const auto f0 = std::chrono::steady_clock::now();
        const int32_t off[2] = {0, (int32_t)history.size()};
        double u = rng.next();
        int32_t id = 0;
        rc = vxs_sample(ctx, 1, kTalkerVocab, talker.data() + (size_t)(f % kRot) * kTalkerVocab, kTalkerVocab, off,
                        history.data(), &tp, 0, &u, &id, nullptr, nullptr, 0);
        const auto f1 = std::chrono::steady_clock::now();
        if (rc != VXS_OK) break;
        history.push_back(id);
        if (f >= warm) tt.push_back(std::chrono::duration<double, std::micro>(f1 - f0).count());
        for (int g = 1; g < kGroups && rc == VXS_OK; g++) {
            // the caller's span: the head writes fresh logits into it before every Select
            std::memcpy(span.data(), cp.data() + (size_t)((f + g) % kRot) * kCpVocab, sizeof(float) * kCpVocab);
            u = rng.next();
            const auto s0 = std::chrono::steady_clock::now();
            rc = vxs_sample(ctx, 1, kCpVocab, span.data(), kCpVocab, nullptr, nullptr, &cpp, 0, &u, &id,
                            writeback ? span.data() : nullptr, nullptr, 0);
            if (f >= warm)
                ts.push_back(std::chrono::duration<double, std::micro>(std::chrono::steady_clock::now() - s0).count());
        }
        if (f >= warm && rc == VXS_OK) {
            double frame = tt.back();
            for (int g = 1; g < kGroups; g++) frame += ts[ts.size() - kGroups + g];
            tf.push_back(frame);
        }
    }
    if (rc != VXS_OK) std::fprintf(stderr, "sampling failed: %s\n", vxs_last_error(ctx));
    vxs_destroy(ctx);
    if (rc != VXS_OK) return 1;
    std::vector<double> all(tt);
    all.insert(all.end(), ts.begin(), ts.end());
    auto pct = [](std::vector<double>& v, double q) {
        std::sort(v.begin(), v.end());
        return v[std::min(v.size() - 1, (size_t)(v.size() * q))];
    };
    std::printf("{\"p50_us\": %.2f, \"p99_us\": %.2f, \"talker_p50_us\": %.2f, \"select_p50_us\": %.2f, "
                "\"select_p99_us\": %.2f, \"frame_p50_us\": %.2f, \"frames\": %d, \"calls_per_frame\": %d, "
                "\"writeback\": %s}\n",
                pct(all, 0.5), pct(all, 0.99), pct(tt, 0.5), pct(ts, 0.5), pct(ts, 0.99), pct(tf, 0.5), frames, kGroups,
                writeback ? "true" : "false");
    return 0;
}

}  // namespace

int main(int argc, char** argv) {
    if (argc >= 3 && std::strcmp(argv[1], "--binding-frame") == 0) {
        const int frames = std::atoi(argv[2]);
        if (frames <= 0) return 2;
        return binding_frame_mode(frames, argc >= 4 && std::strcmp(argv[3], "writeback") == 0);
    }
    if (argc >= 4 && std::strcmp(argv[1], "--frame") == 0) {
        const int rows = std::atoi(argv[2]), iters = std::atoi(argv[3]);
        if (rows <= 0 || iters <= 0) return 2;
        return frame_mode(rows, iters, argc >= 5 && std::strcmp(argv[4], "serial") == 0);
    }
    if (argc < 3) {
        std::fprintf(stderr, "usage: %s <input file> <iterations> [steps] | --frame <rows> <iterations> [serial] | --binding-frame <frames> "
                     "[writeback]\n", argv[0]);
        return 2;
    }
    std::FILE* f = std::fopen(argv[1], "rb");
    if (!f) {
        std::fprintf(stderr, "cannot open %s\n", argv[1]);
        return 2;
    }
    int32_t hdr[3];
    if (std::fread(hdr, sizeof hdr, 1, f) != 1) return 2;
    const int rows = hdr[0], vocab = hdr[1], hlen = hdr[2];
    if (rows <= 0 || vocab <= 0 || hlen < 0) return 2;
    std::vector<float> logits((size_t)rows * vocab);
    std::vector<int32_t> hist((size_t)rows * hlen), off(rows + 1);
    std::vector<vxs_params> params(rows);
    std::vector<double> u(rows);
    std::vector<int32_t> ids(rows);
    bool ok = std::fread(logits.data(), sizeof(float), logits.size(), f) == logits.size() &&
              std::fread(hist.data(), sizeof(int32_t), hist.size(), f) == hist.size() &&
              std::fread(params.data(), sizeof(vxs_params), params.size(), f) == params.size() &&
              std::fread(u.data(), sizeof(double), u.size(), f) == u.size();
    std::fclose(f);
    if (!ok) {
        std::fprintf(stderr, "short input file\n");
        return 2;
    }
    for (int r = 0; r <= rows; r++) off[r] = r * hlen;
    const int iters = std::max(1, std::atoi(argv[2]));
    const int steps = argc >= 4 ? std::atoi(argv[3]) : 1;
    if (steps <= 0 || rows % steps) {
        std::fprintf(stderr, "steps must divide the rows\n");
        return 2;
    }
    const int rs = rows / steps;  // rows per call

    vxs_ctx* ctx = nullptr;
    if (vxs_create(&ctx, 0, rs, vocab, (int64_t)rs * hlen) != VXS_OK) {
        std::fprintf(stderr, "vxs_create failed\n");
        return 1;
    }
    // call k: rows [k * rs, (k + 1) * rs); the offsets index the whole history array
    auto call = [&](int k) {
        const size_t r0 = (size_t)k * rs;
        return vxs_sample(ctx, rs, vocab, logits.data() + r0 * vocab, vocab, hlen ? off.data() + r0 : nullptr,
                          hlen ? hist.data() : nullptr, params.data() + r0, 1, u.data() + r0, ids.data() + r0, nullptr,
                          nullptr, 0);
    };
    for (int i = 0; i < 200; i++)
        if (call(i % steps) != VXS_OK) {
            std::fprintf(stderr, "vxs_sample failed: %s\n", vxs_last_error(ctx));
            vxs_destroy(ctx);
            return 1;
        }
    std::vector<double> t((size_t)iters * steps), fr(iters);
    for (int i = 0; i < iters; i++) {
        const auto f0 = std::chrono::steady_clock::now();
        for (int k = 0; k < steps; k++) {
            const auto a = std::chrono::steady_clock::now();
            const int rc = call(k);
            t[(size_t)i * steps + k] = std::chrono::duration<double, std::micro>(std::chrono::steady_clock::now() - a).count();
            if (rc != VXS_OK) {
                std::fprintf(stderr, "vxs_sample failed: %s\n", vxs_last_error(ctx));
                vxs_destroy(ctx);
                return 1;
            }
        }
        fr[i] = std::chrono::duration<double, std::micro>(std::chrono::steady_clock::now() - f0).count();
    }
    vxs_destroy(ctx);
    std::sort(t.begin(), t.end());
    std::sort(fr.begin(), fr.end());
    const size_t n = t.size();
    if (steps == 1) {
        std::printf("{\"p50_us\": %.2f, \"p99_us\": %.2f, \"iters\": %d, \"id0\": %d}\n", t[n / 2],
                    t[(size_t)(n * 0.99)], iters, ids[0]);
    } else {
        std::printf("{\"p50_us\": %.2f, \"p99_us\": %.2f, \"iters\": %zu, \"steps\": %d, \"frame_p50_us\": %.2f, "
                    "\"frame_p99_us\": %.2f, \"frames\": %d, \"id0\": %d}\n",
                    t[n / 2], t[(size_t)(n * 0.99)], n, steps, fr[iters / 2], fr[(size_t)(iters * 0.99)], iters, ids[0]);
    }
    return 0;
}
