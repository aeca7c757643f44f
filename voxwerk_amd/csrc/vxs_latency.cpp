// vxs_latency.cpp — host-to-host latency of vxs_sample through the C ABI, timed in native code (the
// way a P/Invoke caller sees it: host logits in, host id out, no interpreter in between).
//
// usage: vxs_latency <input file> <iterations>
// input file (little-endian): int32 rows, int32 vocab, int32 hist_len, then rows*vocab float32 logits,
// rows*hist_len int32 history ids, rows vxs_params, rows float64 uniforms.
// output: one JSON line {"p50_us": .., "p99_us": .., "iters": .., "id0": ..}
#include <algorithm>
#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <vector>

#include "vxs_sampler.h"

int main(int argc, char** argv) {
    if (argc < 3) {
        std::fprintf(stderr, "usage: %s <input file> <iterations>\n", argv[0]);
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

    vxs_ctx* ctx = nullptr;
    if (vxs_create(&ctx, 0, rows, vocab, (int64_t)rows * hlen) != VXS_OK) {
        std::fprintf(stderr, "vxs_create failed\n");
        return 1;
    }
    auto call = [&]() {
        return vxs_sample(ctx, rows, vocab, logits.data(), vocab, hlen ? off.data() : nullptr,
                          hlen ? hist.data() : nullptr, params.data(), 1, u.data(), ids.data(), nullptr, nullptr, 0);
    };
    for (int i = 0; i < 200; i++)
        if (call() != VXS_OK) {
            std::fprintf(stderr, "vxs_sample failed: %s\n", vxs_last_error(ctx));
            vxs_destroy(ctx);
            return 1;
        }
    std::vector<double> t(iters);
    for (int i = 0; i < iters; i++) {
        const auto a = std::chrono::steady_clock::now();
        const int rc = call();
        t[i] = std::chrono::duration<double, std::micro>(std::chrono::steady_clock::now() - a).count();
        if (rc != VXS_OK) {
            std::fprintf(stderr, "vxs_sample failed: %s\n", vxs_last_error(ctx));
            vxs_destroy(ctx);
            return 1;
        }
    }
    vxs_destroy(ctx);
    std::sort(t.begin(), t.end());
    std::printf("{\"p50_us\": %.2f, \"p99_us\": %.2f, \"iters\": %d, \"id0\": %d}\n", t[iters / 2],
                t[(size_t)(iters * 0.99)], iters, ids[0]);
    return 0;
}
