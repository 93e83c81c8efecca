// Host-only driver for the AddressSanitizer / UndefinedBehaviorSanitizer build
// of the library's CPU code (the .yuf loader and the host sampler).  Built and
// run by tests/test_host_sanitizers.py with g++; never part of libyufhip.so.
//
//   host_sanitize ckpt FILE [NAME ...]   load FILE, read its config, header
//                                        JSON and the named tensors; prints
//                                        "ok" or "status <code>"
//   host_sanitize sampler SEED CASES     random logits through yuf_sample,
//                                        yuf_argmax, yuf_generation_mask and
//                                        yuf_rng_exp_draws, edge cases included
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>

#include "../include/yuf_engine.h"

namespace {

int run_ckpt(int argc, char **argv) {
    yuf_ckpt *ck = nullptr;
    const int st = yuf_ckpt_load(argv[2], &ck);
    if (st != YUF_OK) {
        // The message must be a readable string.
        std::printf("status %d %zu\n", st, std::strlen(yuf_last_error()));
        return 0;
    }
    yuf_model_config cfg;
    if (yuf_ckpt_config(ck, &cfg) != YUF_OK) return 2;
    const char *json = nullptr;
    size_t len = 0;
    uint32_t version = 0;
    if (yuf_ckpt_header_json(ck, &json, &len, &version) != YUF_OK || std::strlen(json) != len) return 3;
    double checksum = 0.0;
    for (int i = 3; i < argc; ++i) {
        const float *data = nullptr;
        int64_t count = 0, dims[8] = {0};
        int32_t ndim = 0;
        if (yuf_ckpt_tensor(ck, argv[i], &data, &count, &ndim, dims) != YUF_OK) continue;
        for (int64_t j = 0; j < count; ++j) checksum += data[j];
    }
    const float *none = nullptr;
    if (yuf_ckpt_tensor(ck, "no.such.tensor", &none, nullptr, nullptr, nullptr) == YUF_OK) return 4;
    yuf_ckpt_free(ck);
    std::printf("ok %u %d %.6e\n", version, cfg.vocab_size, checksum);
    return 0;
}

// xorshift for the driver's own inputs (independent of the MT19937 under test).
uint64_t g_state = 88172645463325252ull;
uint64_t next_u64() {
    g_state ^= g_state << 13;
    g_state ^= g_state >> 7;
    g_state ^= g_state << 17;
    return g_state;
}
float uniform01() { return (float)((next_u64() >> 40) * (1.0 / 16777216.0)); }

int run_sampler(int seed, int cases) {
    g_state += (uint64_t)seed * 0x9e3779b97f4a7c15ull;
    yuf_rng rng;
    yuf_rng_seed(&rng, (uint64_t)seed);
    for (int c = 0; c < cases; ++c) {
        const int V = 1 + (int)(next_u64() % 600);
        std::vector<float> logits(V), masked(V);
        const int kind = c % 5;
        for (int i = 0; i < V; ++i) {
            float x = 8.0f * (uniform01() - 0.5f);
            if (kind == 1 && i % 3 == 0) x = -INFINITY;   // masked entries
            if (kind == 2) x = 1.0f;                       // all ties
            if (kind == 3 && i == V / 2) x = NAN;          // a NaN logit
            logits[i] = x;
        }
        const float temperature = (kind == 4) ? 0.0f : 0.25f + 2.0f * uniform01();
        const float top_p = (c % 7 == 0) ? 1.0f : 0.05f + 0.95f * uniform01();
        const int top_k = (c % 3 == 0) ? 0 : 1 + (int)(next_u64() % (uint64_t)V);
        const int32_t tok = yuf_sample(logits.data(), V, temperature, top_p, top_k, &rng);
        if (tok < 0 || tok >= V) return 10;
        const int32_t am = yuf_argmax(logits.data(), V);
        if (am < 0 || am >= V) return 11;

        // Generation mask: MIDI ids from an offset, a few blocked raw ids, EOS.
        const int offset = (int)(next_u64() % (uint64_t)(V + 1));
        const int room = V - offset;
        std::vector<int32_t> blocked;
        for (int j = 0; room > 0 && j < 4; ++j) blocked.push_back((int32_t)(next_u64() % (uint64_t)room));
        const int eos = (int)(next_u64() % (uint64_t)V);
        const int index = (int)(next_u64() % 32);
        int st = yuf_generation_mask(logits.data(), V, index, offset, eos, 16, blocked.data(),
                                     (int)blocked.size(), masked.data());
        if (st != YUF_OK) return 12;
        // Rejected inputs must come back as status codes.
        const int32_t bad_id = (int32_t)room;
        if (yuf_generation_mask(logits.data(), V, index, offset, eos, 16, &bad_id, 1, masked.data()) == YUF_OK)
            return 13;
        if (yuf_generation_mask(logits.data(), V, 20, offset, V, 16, nullptr, 0, masked.data()) == YUF_OK) return 14;

        // Exponential draws for the exact device mode.
        const int k = (int)(next_u64() % (uint64_t)(V + 1));
        std::vector<float> q(k > 0 ? k : 1);
        int32_t first_zero = 0;
        if (yuf_rng_exp_draws(&rng, V, k, q.data(), &first_zero) != YUF_OK) return 15;
        for (int i = 0; i < k; ++i)
            if (!(q[i] >= 0.0f)) return 16;
    }
    if (yuf_sample(nullptr, 4, 1.0f, 1.0f, 0, &rng) != YUF_ERR_INVALID) return 17;
    if (yuf_rng_exp_draws(&rng, 0, 0, nullptr, nullptr) != YUF_ERR_INVALID) return 18;
    std::printf("ok %d\n", cases);
    return 0;
}

}  // namespace

int main(int argc, char **argv) {
    if (argc >= 3 && std::strcmp(argv[1], "ckpt") == 0) return run_ckpt(argc, argv);
    if (argc == 4 && std::strcmp(argv[1], "sampler") == 0) return run_sampler(std::atoi(argv[2]), std::atoi(argv[3]));
    std::fprintf(stderr, "usage: host_sanitize ckpt FILE [NAME ...] | sampler SEED CASES\n");
    return 1;
}
