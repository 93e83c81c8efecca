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

// ---------------------------------------------------------------------------
// Full vocabulary (top_k = 0, or top_k >= V): the reference's own parameters
// (temperature 1, top_p 0.95, no top-k: cli/generate.py:39-56,
// vulkan/src/sampler.rs:131-256).  The host sampler sorts all V scaled logits
// (stable, descending) and its softmax sums run over all of them in its
// 16-lane order, so every value's position matters.  One workgroup of 1024
// threads per stream:
//   1. mask + scale, then a stable LSD radix sort of (key, token id) in LDS:
//      4-bit digits, eight passes (a pass whose digit is the same for every
//      value is skipped); element e of a pass is handled by thread e % 1024
//      in round e / 1024, so a ballot ranks it among its wave's equal digits
//      and an exclusive scan over (digit, round, wave) counts places it;
//   2. e_i = exp(x_i - max) rounded once to float, their sum by 16 lanes in
//      the host's order, p_i = e_i * (1 / sum);
//   3. the cut (float)cum_i - p_i > top_p with cum the host's sequential
//      double sum: while every p is a multiple of 2^-53 and the running sum
//      stays <= 1, each double addition is exact, so cum_i is the integer
//      prefix sum of p * 2^53 (one block scan); elsewhere a position whose
//      approximate prefix is more than 2^-20 away from top_p is decided by
//      the bound, and any other position makes one lane redo the host's
//      sequential loop up to it;
//   4. the second softmax over the kept positions (the maximum is position
//      0's, which the cut always keeps for top_p >= 0) and the draw argmax
//      p / q over all V positions, q the host's Exp(1) draws (exact mode,
//      [n, V]) or the counter hash.
constexpr int kFullThreads = 1024;
constexpr int kFullWaves = kFullThreads / 64;
constexpr int kFullMaxV = 24576;
constexpr int kFullMaxRounds = kFullMaxV / kFullThreads;
constexpr uint16_t kDropBit = 0x8000;  // top-p cut flag in the id array (ids < 32768)

// Ascending keys = the host's descending order of values; -0.0 counts as +0.0
// (the host's comparison cannot tell them apart).
__device__ __forceinline__ uint32_t desc_key(float x) { return ~order_key(x == 0.0f ? 0.0f : x); }

__device__ __forceinline__ float from_desc_key(uint32_t k) {
    const uint32_t o = ~k;
    return __uint_as_float((o & 0x80000000u) ? (o & 0x7fffffffu) : ~o);
}

template <typename T>
__device__ __forceinline__ T wave_incl_scan(T x, int lane) {
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const T y = __shfl_up(x, off);
        if (lane >= off) x += y;
    }
    return x;
}

// Exclusive scan of one value per thread in thread order (sh: kFullWaves
// slots).  Ends with a barrier, so sh can be reused at once.
template <typename T>
__device__ __forceinline__ T block_excl_scan(T x, T *sh, int lane, int wave) {
    const T incl = wave_incl_scan(x, lane);
    T excl = __shfl_up(incl, 1);
    if (lane == 0) excl = T(0);
    if (lane == 63) sh[wave] = incl;
    __syncthreads();
    T base = T(0);
    for (int w = 0; w < wave; ++w) base += sh[w];
    __syncthreads();
    return base + excl;
}

// Sum of e[0..n) in the host sampler's order (16 lane accumulators over
// consecutive chunks of 16, then halves folded 8 / 4 / 2 / 1), skipping
// positions whose id carries the drop flag when `cut`.  Lanes 0..15 of one
// wave; lane 0 returns the sum.
__device__ __forceinline__ float sum16_lds(const float *e, const uint16_t *ids, int n, bool cut, int lane) {
    float acc = 0.0f;
    if (lane < 16) {
        int i = lane;
        for (; i + 7 * 16 < n; i += 8 * 16) {
            float v[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                v[u] = e[i + 16 * u];
                if (cut && (ids[i + 16 * u] & kDropBit)) v[u] = 0.0f;
            }
#pragma unroll
            for (int u = 0; u < 8; ++u) acc += v[u];
        }
        for (; i < n; i += 16) acc += (cut && (ids[i] & kDropBit)) ? 0.0f : e[i];
    }
#pragma unroll
    for (int half = 8; half >= 1; half >>= 1) {
        const float o = __shfl_down(acc, half);
        if (lane < half) acc = acc + o;
    }
    return acc;
}

__global__ void __launch_bounds__(kFullThreads) sample_full_kernel(SampleParams p) {
    __shared__ uint32_t skey[kFullMaxV];  // sort keys; after the sort, e_i as float bits
    __shared__ uint16_t sidx[kFullMaxV];  // token ids; kDropBit once cut by top-p
    // Digit counts, then their offsets, per (digit, round, wave); before the
    // sort, the blocked-id bitmap of the generation mask.
    __shared__ uint32_t scnt32[16 * kFullMaxRounds * kFullWaves / 2];
    __shared__ uint64_t sh_u64[kFullWaves];
    __shared__ double sh_f64[kFullWaves];
    __shared__ int sh_int[kFullWaves], sh_int2[kFullWaves];
    __shared__ float sh_flt[kFullWaves];
    __shared__ float sh_sum;
    static_assert(kSampleMaskWords <= 16 * kFullMaxRounds * kFullWaves / 2, "bitmap fits the count array");
    uint16_t *scnt = reinterpret_cast<uint16_t *>(scnt32);
    float *se = reinterpret_cast<float *>(skey);

    const int s = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int V = p.V;
    const int R = (V + kFullThreads - 1) / kFullThreads;
    const float *row = p.logits + (size_t)s * V;
    const uint64_t lt_mask = (1ull << lane) - 1ull;

    // 1. Generation mask and temperature (as sample_kernel).
    uint32_t *blocked_bits = scnt32;
    const bool masked = p.midi_offset >= 0;
    const int mo = p.midi_offset;
    const bool eos_ok = masked && (p.index ? p.index[s] : p.index_all) >= p.min_before_eos;
    if (masked) {
        for (int w = tid; w < kSampleMaskWords; w += kFullThreads) blocked_bits[w] = 0u;
        __syncthreads();
        for (int j = tid; j < p.n_blocked; j += kFullThreads) {
            const int raw = p.blocked[j];
            atomicOr(&blocked_bits[raw >> 5], 1u << (raw & 31));
        }
        __syncthreads();
    }
    for (int r = 0; r < R; ++r) {
        const int i = r * kFullThreads + tid;
        uint32_t key = 0xffffffffu;  // padding: after every value
        if (i < V) {
            float x = row[i];
            if (masked) {
                const int raw = i - mo;
                const bool blocked =
                    raw >= 0 && raw < 32 * kSampleMaskWords && ((blocked_bits[raw >> 5] >> (raw & 31)) & 1u);
                const bool allowed = (raw >= 0 && !blocked) || (i == p.eos_id && eos_ok);
                x = allowed ? x : -INFINITY;
            }
            key = desc_key(x / p.temperature);
        }
        skey[i] = key;
        sidx[i] = (uint16_t)i;
    }
    __syncthreads();

    // Stable LSD radix sort of (key, id), 4 bits per pass.
    const int n_cnt = 16 * R * kFullWaves;
    const int per = (n_cnt + kFullThreads - 1) / kFullThreads;
    for (int shift = 0; shift < 32; shift += 4) {
        uint32_t kr[kFullMaxRounds], ir[kFullMaxRounds];
#pragma unroll
        for (int r = 0; r < kFullMaxRounds; ++r)
            if (r < R) {
                kr[r] = skey[r * kFullThreads + tid];
                ir[r] = sidx[r * kFullThreads + tid];
            }
#pragma unroll
        for (int r = 0; r < kFullMaxRounds; ++r)
            if (r < R) {
                const uint32_t dg = (kr[r] >> shift) & 15u;
                uint64_t bal[4];
                uint64_t same = ~0ull;
#pragma unroll
                for (int b = 0; b < 4; ++b) {
                    bal[b] = __ballot((dg >> b) & 1u);
                    same &= ((dg >> b) & 1u) ? bal[b] : ~bal[b];
                }
                ir[r] |= (uint32_t)__popcll(same & lt_mask) << 16;
                if (lane < 16) {
                    uint64_t m = ~0ull;
#pragma unroll
                    for (int b = 0; b < 4; ++b) m &= ((lane >> b) & 1) ? bal[b] : ~bal[b];
                    scnt[(lane * R + r) * kFullWaves + wave] = (uint16_t)__popcll(m);
                }
            }
        __syncthreads();
        // Exclusive scan of the counts in (digit, round, wave) order.
        {
            int loc[8];
            int tot = 0;
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int c = tid * per + j;
                loc[j] = (j < per && c < n_cnt) ? (int)scnt[c] : 0;
                tot += loc[j];
            }
            int base = block_excl_scan(tot, sh_int, lane, wave);
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int c = tid * per + j;
                if (j < per && c < n_cnt) scnt[c] = (uint16_t)base;
                base += loc[j];
            }
        }
        __syncthreads();
        // A digit that every element shares leaves the order unchanged.
        bool trivial = false;
        const int np = R * kFullThreads;
        for (int d = 0; d < 16; ++d) {
            const int lo = scnt[d * R * kFullWaves], hi = d < 15 ? (int)scnt[(d + 1) * R * kFullWaves] : np;
            trivial |= hi - lo == np;
        }
        if (!trivial) {
#pragma unroll
            for (int r = 0; r < kFullMaxRounds; ++r)
                if (r < R) {
                    const uint32_t dg = (kr[r] >> shift) & 15u;
                    const int pos = (int)scnt[(dg * R + r) * kFullWaves + wave] + (int)(ir[r] >> 16);
                    skey[pos] = kr[r];
                    sidx[pos] = (uint16_t)(ir[r] & 0xffffu);
                }
        }
        __syncthreads();
    }

    // 2. First softmax.  Thread t owns the R consecutive positions from t R.
    const float mx = from_desc_key(skey[0]);
    __syncthreads();
    const int p0 = tid * R;
#pragma unroll
    for (int j = 0; j < kFullMaxRounds; ++j)
        if (j < R) {
            const int pos = p0 + j;
            se[pos] = pos < V ? exp_rn(from_desc_key(skey[pos]) - mx) : 0.0f;
        }
    __syncthreads();
    if (wave == 0) {
        const float sum = sum16_lds(se, sidx, V, false, lane);
        if (lane == 0) sh_sum = sum;
    }
    __syncthreads();
    const float inv = 1.0f / sh_sum;

    // 3. The top-p cut.  Exact prefix sums of p * 2^53 where every p so far is
    // a multiple of 2^-53; approximate double prefix sums for the bounds.
    uint64_t nloc = 0;
    double aloc = 0.0;
    int first_inexact = 0x7fffffff;
#pragma unroll
    for (int j = 0; j < kFullMaxRounds; ++j)
        if (j < R) {
            const float pr = se[p0 + j] * inv;
            const double t = (double)pr * 0x1p53;
            const bool exact = t >= 0.0 && t <= 0x1p62 && t == floor(t);
            if (exact) nloc += (uint64_t)t;
            else first_inexact = min(first_inexact, p0 + j);
            aloc += (double)pr;
        }
    const uint64_t nbase = block_excl_scan(nloc, sh_u64, lane, wave);
    const double abase = block_excl_scan(aloc, sh_f64, lane, wave);
    for (int off = 32; off >= 1; off >>= 1) first_inexact = min(first_inexact, __shfl_xor(first_inexact, off));
    if (lane == 0) sh_int[wave] = first_inexact;
    __syncthreads();
    int fb = sh_int[0];
    for (int w = 1; w < kFullWaves; ++w) fb = min(fb, sh_int[w]);
    __syncthreads();
    int last_uncertain = -1, last_kept = -1;
    {
        uint64_t nsum = nbase;
        double asum = abase;  // approximate sum before position
#pragma unroll
        for (int j = 0; j < kFullMaxRounds; ++j)
            if (j < R) {
                const int pos = p0 + j;
                if (pos >= V) continue;  // padding
                const float pr = se[pos] * inv;
                const double aprev = asum;
                asum += (double)pr;
                bool drop;
                if (pos < fb) nsum += (uint64_t)((double)pr * 0x1p53);
                if (pos < fb && nsum <= (1ull << 53)) {
                    const double cum = (double)nsum * 0x1p-53;  // the host's running sum, exactly
                    drop = (float)cum - pr > p.top_p;
                } else if (aprev > (double)p.top_p + 0x1p-20) {
                    drop = true;
                } else if (aprev < (double)p.top_p - 0x1p-20) {
                    drop = false;
                } else {
                    drop = false;
                    last_uncertain = pos;
                }
                const uint16_t id = sidx[pos] & (uint16_t)~kDropBit;
                sidx[pos] = drop ? (uint16_t)(id | kDropBit) : id;
                if (!drop) last_kept = pos;
            }
    }
    for (int off = 32; off >= 1; off >>= 1) {
        last_uncertain = max(last_uncertain, __shfl_xor(last_uncertain, off));
        last_kept = max(last_kept, __shfl_xor(last_kept, off));
    }
    if (lane == 0) {
        sh_int[wave] = last_uncertain;
        sh_int2[wave] = last_kept;
    }
    __syncthreads();
    int lu = -1, lk = -1;
    for (int w = 0; w < kFullWaves; ++w) {
        lu = max(lu, sh_int[w]);
        lk = max(lk, sh_int2[w]);
    }
    if (lu >= 0) {
        // Undecided positions: the host's loop itself, up to the last of them.
        __syncthreads();  // every thread has read sh_int / sh_int2
        if (tid == 0) {
            double cum = 0.0;
            int kept = -1;
            for (int pos = 0; pos <= lu && pos < V; ++pos) {
                const float pr = se[pos] * inv;
                cum += (double)pr;
                const bool drop = (float)cum - pr > p.top_p;
                const uint16_t id = sidx[pos] & (uint16_t)~kDropBit;
                sidx[pos] = drop ? (uint16_t)(id | kDropBit) : id;
                if (!drop) kept = pos;
            }
            sh_int[0] = kept;
        }
        __syncthreads();
        lk = max(lk, sh_int[0]);
        // Positions after lu keep their bounded decisions; the last kept one
        // may now lie before lu: recount from the flags.
        if (tid == 0) {
            int k2 = -1;
            for (int pos = min(V, kFullMaxV) - 1; pos >= 0; --pos)
                if (!(sidx[pos] & kDropBit)) { k2 = pos; break; }
            sh_int[1] = k2;
        }
        __syncthreads();
        lk = sh_int[1];
    }
    __syncthreads();
    if (lk < 0 || (sidx[0] & kDropBit)) {
        // Everything cut (top_p < 0): the host's second softmax is NaN at every
        // position and its draw keeps position 0.
        if (tid == 0) p.tokens[s] = (int)(sidx[0] & (uint16_t)~kDropBit);
        return;
    }

    // 4. Second softmax over the kept positions (same maximum, so the same
    // exponentials), then the draw.
    if (wave == 0) {
        const float sum2 = sum16_lds(se, sidx, lk + 1, true, lane);
        if (lane == 0) sh_sum = sum2;
    }
    __syncthreads();
    const float inv2 = 1.0f / sh_sum;
    int nan_pos = 0x7fffffff, best_pos = 0x7fffffff;
    float best = -1.0f;
#pragma unroll
    for (int j = 0; j < kFullMaxRounds; ++j)
        if (j < R) {
            const int pos = p0 + j;
            if (pos < V) {
                const uint16_t raw = sidx[pos];
                const float p2 = (raw & kDropBit) ? 0.0f : se[pos] * inv2;
                float sc;
                if (p.exp_draws) {
                    sc = p2 / p.exp_draws[(size_t)s * V + pos];
                } else {
                    sc = p2 == 0.0f ? 0.0f : p2 / -logf(uniform01(p.seed, p.counter, s, raw & (uint16_t)~kDropBit));
                }
                if (isnan(sc)) nan_pos = min(nan_pos, pos);
                else if (sc > best) { best = sc; best_pos = pos; }
            }
        }
    for (int off = 32; off >= 1; off >>= 1) {
        nan_pos = min(nan_pos, __shfl_xor(nan_pos, off));
        const float ob = __shfl_xor(best, off);
        const int op = __shfl_xor(best_pos, off);
        if (ob > best || (ob == best && op < best_pos)) { best = ob; best_pos = op; }
    }
    if (lane == 0) {
        sh_int[wave] = nan_pos;
        sh_int2[wave] = best_pos;
        sh_flt[wave] = best;
    }
    __syncthreads();
    if (tid == 0) {
        int np_ = sh_int[0], bp = sh_int2[0];
        float bs = sh_flt[0];
        for (int w = 1; w < kFullWaves; ++w) {
            np_ = min(np_, sh_int[w]);
            if (sh_flt[w] > bs || (sh_flt[w] == bs && sh_int2[w] < bp)) { bs = sh_flt[w]; bp = sh_int2[w]; }
        }
        const int pos = np_ != 0x7fffffff ? np_ : bp;
        p.tokens[s] = pos < V ? (int)(sidx[pos] & (uint16_t)~kDropBit) : 0;
    }
}

}  // namespace

bool sample_full_vocab(int top_k, int V) { return top_k == 0 || top_k >= V; }

hipError_t launch_sample(const SampleParams &p, int n, hipStream_t stream) {
    if (n <= 0) return hipSuccess;
    if (p.temperature > 0.0f && sample_full_vocab(p.top_k, p.V)) {
        if (p.V > kFullMaxV) return hipErrorInvalidValue;
        hipLaunchKernelGGL(sample_full_kernel, dim3(n), dim3(kFullThreads), 0, stream, p);
        return hipGetLastError();
    }
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
    if (temperature > 0.0f && sample_full_vocab(top_k, V)) {
        if (V > kFullMaxV)
            return fail(YUF_ERR_INVALID, "sample_device: the full-vocabulary path (top_k = 0 or >= V) needs V <= " +
                                             std::to_string(kFullMaxV));
    } else if (temperature > 0.0f && (top_k < 1 || top_k > 64)) {
        return fail(YUF_ERR_INVALID, "sample_device: top_k must be 0 (all V), in [1, 64] or >= V when temperature > 0");
    }
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
