// Device-side sampling for many decode streams at once (gfx950).
//
// The reference samples on the host after copying every stream's logits back
// (cli/generate.py:45-56, :139-154; vulkan/src/sampler.rs:131-256 after the
// generation mask of vulkan/src/generation.rs:195-203).  Here one workgroup
// per stream runs the same steps on the device:
//
//   1. the generation mask (optional): MIDI ids i >= midi_offset keep their
//      logit, ids midi_offset + blocked[j] and every id below midi_offset are
//      -inf, and the EOS id keeps its logit once the stream's index >=
//      min_before_eos (cli/generate.py:142-148);
//   2. temperature <= 0: the first maximum (torch.argmax); otherwise
//      s_i = x_i / temperature (IEEE division, as the host's float divide);
//   3. the top_k (1..64) largest s (ties: lower token id first) in descending
//      order -- the first positions of the host's stable descending sort;
//   4. softmax over them, the cumulative top-p cut (cumulative sum in double,
//      cut where (float)cum - p > top_p), softmax of the survivors: the
//      arithmetic of the host sampler (yuf_sample) step by step -- exp as the
//      correctly rounded float exp, sums in its 16-lane order, 1 / sum;
//   5. the draw argmax_i p_i / q_i (the first maximum; a NaN score wins), the
//      single-sample path of torch.multinomial, with q_i either
//        - exact mode: Exp(1) draws the host took from the stream's MT19937
//          generator (yuf_rng_exp_draws: the first top_k of the V draws a host
//          sample consumes, and the first later position whose draw is 0),
//          so the token equals yuf_sample's under the same generator state;
//        - counter mode: -log u with u from a counter-based hash of (seed,
//          counter, stream, token id) -- the same distribution, no host work.
//
// Selection: the k-th largest of the 256 per-group maxima is a lower bound of
// the k-th largest value (k groups hold a value at least that large), so one
// pass collects the few values at or above it into LDS and their exact ranks
// (by value, then token id) pick the top k.  If more than kPoolCap values pass
// the bound (heavy ties), a 4-pass 8-bit radix select over order-preserving
// integer keys (histograms in LDS) is used instead; it keeps the lowest ids
// among the ties at the k-th value.
#include "common.h"
#include "kernels.h"

namespace yuf {
namespace {

constexpr int kThreads = 256;
constexpr int kMaxTopK = 64;

__device__ __forceinline__ uint32_t order_key(float x) {
    const uint32_t u = __float_as_uint(x);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ uint64_t mix64(uint64_t z) {
    z += 0x9e3779b97f4a7c15ull;
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}

// Uniform in (0, 1) from 24 random bits.
__device__ __forceinline__ float uniform01(uint64_t seed, uint64_t counter, int stream, int token) {
    const uint64_t h = mix64(seed ^ mix64(counter * 0x100000001b3ull + (uint64_t)stream * 0x9e3779b97f4a7c15ull +
                                          (uint64_t)token));
    return ((float)(h >> 40) + 0.5f) * (1.0f / 16777216.0f);
}

// exp rounded once to float: the double exponential is accurate to about an
// ulp of double, so the float result is the correctly rounded one (the host
// sampler computes the same value).
__device__ __forceinline__ float exp_rn(float x) { return (float)exp((double)x); }

constexpr int kPoolCap = 1024;

// Fallback selection (many ties at the bound): 4-pass 8-bit radix select of the
// k-th largest key, then the keys above it and the lowest ids among its ties.
// `val(i)` is the (masked, scaled) value of token i.
template <int NTH, typename Val>
__device__ void radix_topk(Val &&val, int V, int k, int tid, uint32_t *hist, uint32_t &sh_prefix,
                           uint32_t &sh_remaining, uint32_t &sh_gt, float *cand_val, int *cand_idx) {
    uint32_t prefix = 0, mask = 0;
    if (tid == 0) sh_remaining = (uint32_t)k;
    for (int shift = 24; shift >= 0; shift -= 8) {
        for (int hb = tid; hb < 256; hb += NTH) hist[hb] = 0;
        __syncthreads();
        for (int i = tid; i < V; i += NTH) {
            const uint32_t key = order_key(val(i));
            if ((key & mask) == prefix) atomicAdd(&hist[(key >> shift) & 255u], 1u);
        }
        __syncthreads();
        if (tid == 0) {
            uint32_t cum = 0, rem = sh_remaining;
            int b = 255;
            for (; b > 0; --b) {
                if (cum + hist[b] >= rem) break;
                cum += hist[b];
            }
            sh_remaining = rem - cum;
            sh_prefix = prefix | ((uint32_t)b << shift);
        }
        __syncthreads();
        prefix = sh_prefix;
        mask |= 255u << shift;
    }
    // prefix = key of the k-th largest; sh_remaining = how many of its ties to keep.
    if (tid == 0) sh_gt = 0;
    __syncthreads();
    const uint32_t n_eq = sh_remaining;
    const uint32_t n_gt = (uint32_t)k - n_eq;
    for (int i = tid; i < V; i += NTH) {
        const float x = val(i);
        if (order_key(x) > prefix) {
            const uint32_t slot = atomicAdd(&sh_gt, 1u);
            cand_val[slot] = x;
            cand_idx[slot] = i;
        }
    }
    __syncthreads();
    // Ties at the k-th key: the n_eq lowest ids.  Wave 0 walks the row in
    // 64-id blocks in id order; a ballot numbers each block's ties.
    if (tid < 64) {
        uint32_t taken = 0;
        for (int base = 0; base < V && taken < n_eq; base += 64) {
            const int i = base + tid;
            const float x = i < V ? val(i) : 0.0f;
            const bool tie = i < V && order_key(x) == prefix;
            const uint64_t bits = __ballot(tie);
            const uint32_t before = (uint32_t)__popcll(bits & ((1ull << tid) - 1ull));
            if (tie && taken + before < n_eq) {
                cand_val[n_gt + taken + before] = x;
                cand_idx[n_gt + taken + before] = i;
            }
            taken += (uint32_t)__popcll(bits);
        }
    }
    __syncthreads();
    // Order the candidates by (value, then id): rank each one.
    float v = 0.0f;
    int ix = 0, rank = 0;
    if (tid < k) {
        v = cand_val[tid];
        ix = cand_idx[tid];
        const uint32_t key = order_key(v);
        for (int j = 0; j < k; ++j) {
            const uint32_t o = order_key(cand_val[j]);
            rank += (o > key || (o == key && cand_idx[j] < ix)) ? 1 : 0;
        }
    }
    __syncthreads();
    if (tid < k) {
        cand_val[rank] = v;
        cand_idx[rank] = ix;
    }
}

// Sum of p[0..63] (zeros past the kept candidates) in the host sampler's
// order: 16 lane accumulators over consecutive chunks of 16, then the halves
// folded 8 / 4 / 2 / 1 (the zeros the host adds for positions >= 64 change
// nothing).  One thread.
__device__ __forceinline__ float sum16(const float *p) {
    float acc[16];
#pragma unroll
    for (int l = 0; l < 16; ++l) acc[l] = ((p[l] + p[l + 16]) + p[l + 32]) + p[l + 48];
#pragma unroll
    for (int half = 8; half >= 1; half /= 2)
#pragma unroll
        for (int l = 0; l < half; ++l) acc[l] = acc[l] + acc[l + half];
    return acc[0];
}

constexpr int kRegElems = 24576;  // rows up to this many logits are held in registers
constexpr int kRegThreads = 1024;  // threads per row on that path (four waves per SIMD)

template <int NTH, bool REG>
__global__ void __launch_bounds__(NTH) sample_kernel(SampleParams p) {
    static_assert(NTH % kThreads == 0, "bound groups of NTH / 256 threads");
    constexpr int kRegF4 = kRegElems / 4 / NTH;  // float4 per thread on the register path
    constexpr int GRP = NTH / kThreads;          // threads per bound group (one key per group)
    static_assert(GRP == 1 || GRP == 2 || GRP == 4, "bound group size");
    __shared__ uint32_t hist[256];
    __shared__ uint32_t sh_prefix, sh_remaining, sh_gt;
    __shared__ float cand_val[kMaxTopK];
    __shared__ int cand_idx[kMaxTopK];
    __shared__ float red_val[NTH / 64];
    __shared__ int red_idx[NTH / 64];
    __shared__ uint32_t sh_thresh, sh_n;
    __shared__ __attribute__((aligned(16))) uint32_t tkey[kThreads];
    __shared__ uint32_t pool_key[kPoolCap];
    __shared__ int pool_idx[kPoolCap];
    __shared__ float pool_val[kPoolCap];
    __shared__ uint32_t blocked_bits[kSampleMaskWords];
    __shared__ float sm[kMaxTopK], sp[kMaxTopK];
    __shared__ float sh_sum;
    __shared__ int sh_keep[kMaxTopK];
    const int s = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int V = p.V;
    const float *row = p.logits + (size_t)s * V;

    // Generation mask: blocked MIDI ids as a bitmap over raw ids.
    const bool masked = p.midi_offset >= 0;
    const int mo = p.midi_offset;
    const bool eos_ok = masked && (p.index ? p.index[s] : p.index_all) >= p.min_before_eos;
    if (masked) {
        for (int w = tid; w < kSampleMaskWords; w += NTH) blocked_bits[w] = 0u;
        __syncthreads();
        for (int j = tid; j < p.n_blocked; j += NTH) {
            const int raw = p.blocked[j];
            atomicOr(&blocked_bits[raw >> 5], 1u << (raw & 31));
        }
        __syncthreads();
    }
    const bool greedy = !(p.temperature > 0.0f);
    // The value the selection ranks: the masked logit, divided by the
    // temperature unless greedy.
    auto value = [&](int i, float x) {
        if (masked) {
            const int raw = i - mo;
            const bool blocked =
                raw >= 0 && raw < 32 * kSampleMaskWords && ((blocked_bits[raw >> 5] >> (raw & 31)) & 1u);
            const bool allowed = (raw >= 0 && !blocked) ||
                                 (i == p.eos_id && eos_ok);
            x = allowed ? x : -INFINITY;
        }
        return greedy ? x : x / p.temperature;
    };

    // REG: the whole row is read once, as 16-byte loads all in flight together,
    // into registers (thread t holds elements 4 (t + NTH j) .. + 3), and
    // replaced there by the values the selection ranks.
    float4 vals[REG ? kRegF4 : 1];
    if constexpr (REG) {
        const auto rr = make_rsrc(row, (uint32_t)V * 4u);
#pragma unroll
        for (int j = 0; j < kRegF4; ++j)
            vals[j] = __builtin_bit_cast(
                float4, __builtin_amdgcn_raw_buffer_load_b128(rr, (uint32_t)(tid + j * NTH) * 16u, 0, 0));
#pragma unroll
        for (int j = 0; j < kRegF4; ++j) {
            const int i0 = 4 * (tid + j * NTH);
            vals[j].x = value(i0, vals[j].x);
            vals[j].y = value(i0 + 1, vals[j].y);
            vals[j].z = value(i0 + 2, vals[j].z);
            vals[j].w = value(i0 + 3, vals[j].w);
        }
    }
    auto visit = [&](auto &&fn) {
        if constexpr (REG) {
#pragma unroll
            for (int j = 0; j < kRegF4; ++j) {
                const int i0 = 4 * (tid + j * NTH);
                if (i0 < V) fn(i0, vals[j].x);
                if (i0 + 1 < V) fn(i0 + 1, vals[j].y);
                if (i0 + 2 < V) fn(i0 + 2, vals[j].z);
                if (i0 + 3 < V) fn(i0 + 3, vals[j].w);
            }
        } else {
            for (int i = tid; i < V; i += NTH) fn(i, value(i, row[i]));
        }
    };

    if (greedy) {
        float best = -INFINITY;
        int bi = 0x7fffffff;
        visit([&](int i, float x) {
            if (x > best || (x == best && i < bi) || (isnan(x) && !isnan(best))) { best = x; bi = i; }
        });
        // Wave then block reduction of (value, index): larger value, then smaller index.
        for (int off = 32; off >= 1; off >>= 1) {
            const float ov = __shfl_xor(best, off);
            const int oi = __shfl_xor(bi, off);
            if (ov > best || (ov == best && oi < bi) || (isnan(ov) && !isnan(best))) { best = ov; bi = oi; }
        }
        if (lane == 0) { red_val[wave] = best; red_idx[wave] = bi; }
        __syncthreads();
        if (tid == 0) {
            for (int w = 1; w < NTH / 64; ++w)
                if (red_val[w] > best || (red_val[w] == best && red_idx[w] < bi) || (isnan(red_val[w]) && !isnan(best))) {
                    best = red_val[w];
                    bi = red_idx[w];
                }
            p.tokens[s] = bi < V ? bi : 0;
        }
        return;
    }

    const int k = p.top_k < V ? p.top_k : V;
    // Lower bound: the k-th largest of the 256 group maxima (a group is GRP
    // adjacent threads; rank by key, then group): k groups hold a value at
    // least that large.
    uint32_t mk = 0;
    visit([&](int, float x) { mk = max(mk, order_key(x)); });
    if constexpr (GRP >= 2)
        mk = max(mk, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)mk, dpp::kQuadXor1, 0xF, 0xF, false));
    if constexpr (GRP >= 4)
        mk = max(mk, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)mk, dpp::kQuadXor2, 0xF, 0xF, false));
    if (tid % GRP == 0) tkey[tid / GRP] = mk;
    if (tid == 0) sh_n = 0;
    __syncthreads();
    if (tid < kThreads) {
        mk = tkey[tid];
        uint32_t rank = 0;
        const uint4 *t4 = reinterpret_cast<const uint4 *>(tkey);
#pragma unroll 8
        for (int j = 0; j < kThreads / 4; ++j) {
            const uint4 o = t4[j];  // broadcast reads, batched by the unroll
            rank += (o.x > mk || (o.x == mk && 4 * j < tid)) ? 1u : 0u;
            rank += (o.y > mk || (o.y == mk && 4 * j + 1 < tid)) ? 1u : 0u;
            rank += (o.z > mk || (o.z == mk && 4 * j + 2 < tid)) ? 1u : 0u;
            rank += (o.w > mk || (o.w == mk && 4 * j + 3 < tid)) ? 1u : 0u;
        }
        if (rank == (uint32_t)(k - 1)) sh_thresh = mk;
    }
    __syncthreads();
    const uint32_t thresh = sh_thresh;
    visit([&](int i, float x) {
        const uint32_t key = order_key(x);
        if (key >= thresh) {
            const uint32_t slot = atomicAdd(&sh_n, 1u);
            if (slot < (uint32_t)kPoolCap) {
                pool_key[slot] = key;
                pool_idx[slot] = i;
                pool_val[slot] = x;
            }
        }
    });
    __syncthreads();
    const uint32_t n_pool = sh_n;
    if (n_pool <= (uint32_t)kPoolCap) {
        // Exact rank of each pooled value; ranks below k are the top k in
        // descending order (a rank depends only on (key, token id)).
        for (uint32_t c = tid; c < n_pool; c += NTH) {
            const uint32_t key = pool_key[c];
            const int idx = pool_idx[c];
            uint32_t rank = 0;
#pragma unroll 8
            for (uint32_t j = 0; j < n_pool; ++j) {
                const uint32_t o = pool_key[j];
                rank += (o > key || (o == key && pool_idx[j] < idx)) ? 1u : 0u;
            }
            if (rank < (uint32_t)k) {
                cand_val[rank] = pool_val[c];
                cand_idx[rank] = idx;
            }
        }
    } else {
        radix_topk<NTH>([&](int i) { return value(i, row[i]); }, V, k, tid, hist, sh_prefix, sh_remaining, sh_gt,
                        cand_val, cand_idx);
    }
    __syncthreads();
    if (wave != 0) return;

    // Candidates in descending order (position = lane).  Softmax, top-p cut,
    // softmax, draw -- the host sampler's arithmetic.
    const bool live = lane < k;
    const float v = live ? cand_val[lane] : -INFINITY;
    const int ix = live ? cand_idx[lane] : 0x7fffffff;
    const float mx = __shfl(v, 0);  // position 0 holds the maximum
    sm[lane] = live ? exp_rn(v - mx) : 0.0f;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
    if (lane == 0) sh_sum = sum16(sm);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
    const float pr = sm[lane] * (1.0f / sh_sum);
    sp[lane] = pr;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
    if (lane == 0) {
        double cum = 0.0;
        for (int i = 0; i < k; ++i) {
            cum += (double)sp[i];
            sh_keep[i] = !((float)cum - sp[i] > p.top_p);
        }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
    const float v2 = live && sh_keep[lane] ? v : -INFINITY;
    float mx2 = v2;
    for (int off = 32; off >= 1; off >>= 1) mx2 = fmaxf(mx2, __shfl_xor(mx2, off));
    sm[lane] = live ? exp_rn(v2 - mx2) : 0.0f;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
    if (lane == 0) sh_sum = sum16(sm);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
    const float p2 = sm[lane] * (1.0f / sh_sum);
    float q = 1.0f;
    if (live) q = p.exp_draws ? p.exp_draws[(size_t)s * p.top_k + lane] : -logf(uniform01(p.seed, p.counter, s, ix));
    sp[lane] = p2 / q;  // the score
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
    if (lane == 0) {
        // First maximum in position order; a NaN score takes the place unless
        // the best is already NaN (the host's loop over all V positions:
        // positions >= k score 0, or NaN where their draw is 0).
        int best = 0;
        float best_score = sp[0];
        for (int i = 1; i < k; ++i) {
            const float sc = sp[i];
            if (!isnan(best_score) && (isnan(sc) || sc > best_score)) {
                best = i;
                best_score = sc;
            }
        }
        const int fz = p.first_zero ? p.first_zero[s] : -1;
        if (fz >= k && !isnan(best_score)) best = fz;
        int token;
        if (best < k) {
            token = cand_idx[best];
        } else {
            // Position best >= k of the host's order: the t-th (t = best - k,
            // from 0) smallest id outside the candidates (all -inf, in id
            // order).  That id is the least x >= t with x = t + #{candidate
            // ids <= x}; iterating x <- t + count(x) from x = t climbs to it
            // (count is non-decreasing) in at most k + 1 rounds, with no
            // sorted copy of the ids (a private array would live in scratch).
            const int t = best - k;
            int x = t;
            for (int round = 0; round <= k; ++round) {
                int c = 0;
                for (int i = 0; i < k; ++i) c += cand_idx[i] <= x ? 1 : 0;
                if (t + c == x) break;
                x = t + c;
            }
            token = x;
        }
        p.tokens[s] = token < V ? token : 0;
    }
}

}  // namespace

hipError_t launch_sample(const SampleParams &p, int n, hipStream_t stream) {
    if (n <= 0) return hipSuccess;
    if (p.temperature > 0.0f && (p.top_k < 1 || p.top_k > kMaxTopK)) return hipErrorInvalidValue;
    if (p.V <= kRegElems)
        hipLaunchKernelGGL((sample_kernel<kRegThreads, true>), dim3(n), dim3(kRegThreads), 0, stream, p);
    else
        hipLaunchKernelGGL((sample_kernel<kThreads, false>), dim3(n), dim3(kThreads), 0, stream, p);
    return hipGetLastError();
}

}  // namespace yuf

namespace {
int check_sample_args(int n, int V, const float *logits_dev, float temperature, int top_k, const int32_t *tokens_dev) {
    using namespace yuf;
    if (n < 0 || V <= 0) return fail(YUF_ERR_INVALID, "sample_device: bad sizes");
    if (temperature > 0.0f && (top_k < 1 || top_k > 64))
        return fail(YUF_ERR_INVALID, "sample_device: top_k must be in [1, 64] when temperature > 0");
    if (n > 0 && (!logits_dev || !tokens_dev)) return fail(YUF_ERR_INVALID, "sample_device: null pointer");
    return YUF_OK;
}

int launch_checked(const yuf::SampleParams &sp, int n, void *stream) {
    using namespace yuf;
    hipError_t err = launch_sample(sp, n, static_cast<hipStream_t>(stream));
    if (err != hipSuccess) return fail(YUF_ERR_HIP, std::string("sample launch: ") + hipGetErrorString(err));
    return YUF_OK;
}
}  // namespace

extern "C" int yuf_sample_device(int n, int V, const float *logits_dev, float temperature, int top_k, uint64_t seed,
                                 uint64_t counter, int32_t *tokens_dev, void *stream) {
    using namespace yuf;
    int rc = check_sample_args(n, V, logits_dev, temperature, top_k, tokens_dev);
    if (rc != YUF_OK) return rc;
    SampleParams sp;
    sp.V = V; sp.logits = logits_dev; sp.temperature = temperature; sp.top_p = 1.0f; sp.top_k = top_k;
    sp.seed = seed; sp.counter = counter; sp.tokens = tokens_dev;
    return launch_checked(sp, n, stream);
}

extern "C" int yuf_sample_device_masked(int n, int V, const float *logits_dev, float temperature, float top_p,
                                        int top_k, int midi_offset, int eos_id, int min_before_eos, int index,
                                        const int32_t *index_dev, const int32_t *blocked_raw_ids, int n_blocked,
                                        const float *exp_draws_dev, const int32_t *first_zero_dev, uint64_t seed,
                                        uint64_t counter, int32_t *tokens_dev, void *stream) {
    using namespace yuf;
    int rc = check_sample_args(n, V, logits_dev, temperature, top_k, tokens_dev);
    if (rc != YUF_OK) return rc;
    SampleParams sp;
    sp.V = V; sp.logits = logits_dev; sp.temperature = temperature; sp.top_p = top_p; sp.top_k = top_k;
    sp.seed = seed; sp.counter = counter; sp.tokens = tokens_dev;
    sp.exp_draws = exp_draws_dev; sp.first_zero = first_zero_dev;
    if (midi_offset >= 0) {
        if (midi_offset > V) return fail(YUF_ERR_RANGE, "sample_device_masked: midi_offset outside [0, V]");
        if (n_blocked < 0 || n_blocked > kSampleMaxBlocked || (n_blocked > 0 && !blocked_raw_ids))
            return fail(YUF_ERR_INVALID, "sample_device_masked: blocked ids: at most " +
                                             std::to_string(kSampleMaxBlocked) + ", host array");
        for (int j = 0; j < n_blocked; ++j) {
            const int raw = blocked_raw_ids[j];
            if (raw < 0 || raw >= 32 * kSampleMaskWords || (int64_t)midi_offset + raw >= V)
                return fail(YUF_ERR_RANGE, "sample_device_masked: blocked id " + std::to_string(raw) +
                                               " outside the MIDI range");
            sp.blocked[j] = raw;
        }
        if (index >= min_before_eos || index_dev) {
            if (eos_id < 0 || eos_id >= V) return fail(YUF_ERR_RANGE, "sample_device_masked: EOS id outside [0, V)");
        }
        sp.midi_offset = midi_offset; sp.eos_id = eos_id; sp.min_before_eos = min_before_eos;
        sp.index_all = index; sp.index = index_dev; sp.n_blocked = n_blocked;
    }
    return launch_checked(sp, n, stream);
}
