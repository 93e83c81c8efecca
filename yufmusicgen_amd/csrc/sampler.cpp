// Host token sampling, following torch's CPU arithmetic step by step.
//
// Replaces the reference's Rust sampler (vulkan/src/sampler.rs:22-82 MT19937,
// :131-256 sample_token, :264-271 argmax) and mirrors the Python
// `sample_token` (yufmusicgen/cli/generate.py:45-56) it was written to match:
//   scale by 1/temperature -> [top_k] -> sort descending -> softmax ->
//   cumsum (accumulated in double, as torch's CPU cumsum does for float) ->
//   drop where cumulative - p > top_p -> softmax of the masked logits ->
//   torch.multinomial(p, 1): q ~ Exp(1) for every entry (53-bit uniforms from
//   two MT19937 words, -log1p(-u) in double, cast to float), argmax(p / q).
// The Gumbel/exponential stream is bit-identical to torch.manual_seed's; the
// softmax exponentials are correctly rounded float exps (the double exp
// rounded once), which torch's vectorised exp matches to within an ulp, so a
// token can differ from torch only when two candidates are tied to the last
// bit.  The device sampler's exact mode (yuf_sample_device_masked with host
// draws) computes the same floats.
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <numeric>
#include <string>
#include <vector>

#include "../../include/yuf_engine.h"

namespace yuf {
int fail(int status, const std::string &msg);
}

namespace {

constexpr int kN = 624, kM = 397;
constexpr uint32_t kMatrixA = 0x9908b0dfu, kUpper = 0x80000000u, kLower = 0x7fffffffu;

void twist(yuf_rng *r) {
    for (int j = 0; j < kN; ++j) {
        const uint32_t y = (r->mt[j] & kUpper) | (r->mt[(j + 1) % kN] & kLower);
        uint32_t next = y >> 1;
        if (y & 1u) next ^= kMatrixA;
        r->mt[j] = r->mt[(j + kM) % kN] ^ next;
    }
    r->index = 0;
}

// Sum of a float array the way an AVX-512 horizontal reduction of 16-lane
// partial sums orders it (acc = first chunk, += later chunks, partial tail
// into the low lanes, then halves folded 8/4/2/1).
float vec_sum(const float *x, size_t n) {
    constexpr size_t W = 16;
    if (n == 0) return 0.0f;
    float acc[W];
    if (n < W) {
        std::fill(acc, acc + W, 0.0f);
        for (size_t i = 0; i < n; ++i) acc[i] = x[i];
    } else {
        std::copy(x, x + W, acc);
        size_t i = W;
        for (; i + W <= n; i += W)
            for (size_t l = 0; l < W; ++l) acc[l] += x[i + l];
        for (size_t l = 0; i + l < n; ++l) acc[l] += x[i + l];
    }
    for (size_t half = W / 2; half >= 1; half /= 2)
        for (size_t l = 0; l < half; ++l) acc[l] = acc[l] + acc[l + half];
    return acc[0];
}

// softmax over x (with -inf entries), result into p.
void softmax(const std::vector<float> &x, std::vector<float> &p) {
    const size_t n = x.size();
    float mx = -INFINITY;
    for (float v : x) mx = std::max(mx, v);
    p.resize(n);
    for (size_t i = 0; i < n; ++i) p[i] = (float)std::exp((double)(x[i] - mx));
    const float inv = 1.0f / vec_sum(p.data(), n);
    for (size_t i = 0; i < n; ++i) p[i] = p[i] * inv;
}

}  // namespace

extern "C" void yuf_rng_seed(yuf_rng *r, uint64_t seed) {
    r->mt[0] = (uint32_t)(seed & 0xffffffffu);
    for (int j = 1; j < kN; ++j) {
        const uint32_t prev = r->mt[j - 1];
        r->mt[j] = (uint32_t)(1812433253ull * (uint64_t)(prev ^ (prev >> 30)) + (uint64_t)j);
    }
    r->index = kN;
}

extern "C" uint32_t yuf_rng_next_u32(yuf_rng *r) {
    if (r->index >= (uint32_t)kN) twist(r);
    uint32_t y = r->mt[r->index++];
    y ^= y >> 11;
    y ^= (y << 7) & 0x9d2c5680u;
    y ^= (y << 15) & 0xefc60000u;
    y ^= y >> 18;
    return y;
}

extern "C" double yuf_rng_next_uniform(yuf_rng *r) {
    const uint64_t hi = yuf_rng_next_u32(r), lo = yuf_rng_next_u32(r);
    const uint64_t composite = (hi << 32) | lo;
    return (double)(composite & ((1ull << 53) - 1)) * (1.0 / (double)(1ull << 53));
}

extern "C" int yuf_rng_exp_draws(yuf_rng *r, int V, int k, float *q_out, int32_t *first_zero) {
    if (!r || V <= 0 || k < 0 || (k > 0 && !q_out)) return yuf::fail(YUF_ERR_INVALID, "yuf_rng_exp_draws: bad arguments");
    int32_t fz = -1;
    for (int i = 0; i < V; ++i) {
        const double u = yuf_rng_next_uniform(r);
        if (i < k) q_out[i] = (float)(-std::log1p(-u));
        else if (u == 0.0 && fz < 0) fz = i;
    }
    if (first_zero) *first_zero = fz;
    return YUF_OK;
}

extern "C" int32_t yuf_argmax(const float *logits, int V) {
    if (!logits || V <= 0) return yuf::fail(YUF_ERR_INVALID, "yuf_argmax: empty logits");
    int best = 0;
    for (int i = 1; i < V; ++i) {
        // torch.argmax: NaN counts as the maximum, otherwise the first maximum wins.
        if (std::isnan(logits[best])) break;
        if (std::isnan(logits[i]) || logits[i] > logits[best]) best = i;
    }
    return best;
}

extern "C" int yuf_generation_mask(const float *logits, int V, int index, int midi_offset, int eos_id,
                                   int min_before_eos, const int32_t *blocked_raw_ids, int n_blocked,
                                   float *allowed_out) {
    if (!logits || !allowed_out || V <= 0) return yuf::fail(YUF_ERR_INVALID, "yuf_generation_mask: empty logits");
    if (midi_offset < 0 || midi_offset > V) return yuf::fail(YUF_ERR_RANGE, "yuf_generation_mask: midi_offset outside [0, V]");
    if (n_blocked < 0 || (n_blocked > 0 && !blocked_raw_ids))
        return yuf::fail(YUF_ERR_INVALID, "yuf_generation_mask: bad blocked id list");
    for (int j = 0; j < n_blocked; ++j)
        if (blocked_raw_ids[j] < 0 || midi_offset + (int64_t)blocked_raw_ids[j] >= V)
            return yuf::fail(YUF_ERR_RANGE, "yuf_generation_mask: blocked id outside the MIDI range");
    if (index >= min_before_eos && (eos_id < 0 || eos_id >= V))
        return yuf::fail(YUF_ERR_RANGE, "yuf_generation_mask: EOS id outside [0, V)");
    const float eos_logit = (eos_id >= 0 && eos_id < V) ? logits[eos_id] : 0.0f;
    for (int i = 0; i < midi_offset; ++i) allowed_out[i] = -INFINITY;
    if (allowed_out != logits)
        for (int i = midi_offset; i < V; ++i) allowed_out[i] = logits[i];
    for (int j = 0; j < n_blocked; ++j) allowed_out[midi_offset + blocked_raw_ids[j]] = -INFINITY;
    if (index >= min_before_eos) allowed_out[eos_id] = eos_logit;
    return YUF_OK;
}

extern "C" int32_t yuf_sample(const float *logits, int V, float temperature, float top_p, int top_k, yuf_rng *rng) {
    if (!logits || V <= 0) return yuf::fail(YUF_ERR_INVALID, "yuf_sample: empty logits");
    if (!(temperature > 0.0f)) return yuf_argmax(logits, V);
    if (!rng) return yuf::fail(YUF_ERR_INVALID, "yuf_sample: null rng");
    std::vector<float> scaled(V);
    for (int i = 0; i < V; ++i) scaled[i] = logits[i] / temperature;
    if (top_k > 0 && top_k < V) {
        std::vector<int> idx(V);
        std::iota(idx.begin(), idx.end(), 0);
        std::nth_element(idx.begin(), idx.begin() + top_k, idx.end(), [&](int a, int b) {
            return scaled[a] > scaled[b] || (scaled[a] == scaled[b] && a < b);
        });
        std::vector<float> masked(V, -INFINITY);
        for (int i = 0; i < top_k; ++i) masked[idx[i]] = scaled[idx[i]];
        scaled.swap(masked);
    }
    // Descending order; equal keys keep index order.
    std::vector<int> order(V);
    std::iota(order.begin(), order.end(), 0);
    std::stable_sort(order.begin(), order.end(), [&](int a, int b) { return scaled[a] > scaled[b]; });
    std::vector<float> sorted(V);
    for (int i = 0; i < V; ++i) sorted[i] = scaled[order[i]];
    std::vector<float> probs;
    softmax(sorted, probs);
    double cum = 0.0;
    for (int i = 0; i < V; ++i) {
        cum += (double)probs[i];
        const float cum_f = (float)cum;
        if (cum_f - probs[i] > top_p) sorted[i] = -INFINITY;
    }
    std::vector<float> p2;
    softmax(sorted, p2);
    // torch.multinomial(p2, 1): q ~ Exp(1) for every entry, argmax(p2 / q).
    int best = -1;
    float best_score = 0.0f;
    for (int i = 0; i < V; ++i) {
        const double u = yuf_rng_next_uniform(rng);
        const float q = (float)(-std::log1p(-u));
        const float score = p2[i] / q;
        if (best < 0 || (!std::isnan(best_score) && (std::isnan(score) || score > best_score))) {
            best = i;
            best_score = score;
        }
    }
    return order[best];
}
