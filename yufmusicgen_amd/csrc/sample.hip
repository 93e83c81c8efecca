// Device-side top-k sampling for many decode streams at once (gfx950).
//
// The reference samples on the host after copying every stream's logits back
// (cli/generate.py:45-56; vulkan/src/sampler.rs:131-256).  Here one workgroup
// per stream: temperature <= 0 takes the first maximum (torch.argmax); else the
// top_k largest logits (ties: lower token id first) are selected and a
// Gumbel-max draw argmax(x_i / T - log(-log u_i)) picks among them -- the same
// distribution as softmax(top-k(x / T)) sampling.  u_i comes from a
// counter-based hash of (seed, counter, stream, token id), so results do not
// depend on launch order.
//
// Selection: the k-th largest of the 256 per-thread maxima is a lower bound of
// the k-th largest logit (k threads hold a value at least that large), so one
// pass collects the few logits at or above it into LDS and their exact ranks
// (by value, then token id) pick the top k.  If more than kPoolCap logits pass
// the bound (heavy ties), a 4-pass 8-bit radix select over order-preserving
// integer keys (histograms in LDS) is used instead; it keeps the ties at the
// k-th value in arrival order.
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

constexpr int kPoolCap = 1024;

// Fallback selection (many ties at the bound): 4-pass 8-bit radix select of the
// k-th largest key, then the keys above it and ties up to k in arrival order.
template <int NTH>
__device__ void radix_topk(const float *row, int V, int k, int tid, uint32_t *hist, uint32_t &sh_prefix,
                           uint32_t &sh_remaining, uint32_t &sh_gt, uint32_t &sh_eq, float *cand_val, int *cand_idx) {
    uint32_t prefix = 0, mask = 0;
    if (tid == 0) sh_remaining = (uint32_t)k;
    for (int shift = 24; shift >= 0; shift -= 8) {
        for (int hb = tid; hb < 256; hb += NTH) hist[hb] = 0;
        __syncthreads();
        for (int i = tid; i < V; i += NTH) {
            const uint32_t key = order_key(row[i]);
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
    if (tid == 0) { sh_gt = 0; sh_eq = 0; }
    __syncthreads();
    const uint32_t n_eq = sh_remaining;
    const uint32_t n_gt = (uint32_t)k - n_eq;
    for (int i = tid; i < V; i += NTH) {
        const float x = row[i];
        const uint32_t key = order_key(x);
        if (key > prefix) {
            const uint32_t slot = atomicAdd(&sh_gt, 1u);
            cand_val[slot] = x; cand_idx[slot] = i;
        } else if (key == prefix) {
            const uint32_t slot = atomicAdd(&sh_eq, 1u);
            if (slot < n_eq) { cand_val[n_gt + slot] = x; cand_idx[n_gt + slot] = i; }
        }
    }
}

constexpr int kRegElems = 24576;  // rows up to this many logits are held in registers
constexpr int kRegThreads = 1024;  // threads per row on that path (four waves per SIMD)

template <int NTH, bool REG>
__global__ void __launch_bounds__(NTH) sample_kernel(int V, const float *logits, float temperature, int top_k,
                                                    uint64_t seed, uint64_t counter, int32_t *tokens) {
    static_assert(NTH % kThreads == 0, "bound groups of NTH / 256 threads");
    constexpr int kRegF4 = kRegElems / 4 / NTH;  // float4 per thread on the register path
    constexpr int GRP = NTH / kThreads;          // threads per bound group (one key per group)
    static_assert(GRP == 1 || GRP == 2 || GRP == 4, "bound group size");
    __shared__ uint32_t hist[256];
    __shared__ uint32_t sh_prefix, sh_remaining, sh_gt, sh_eq;
    __shared__ float cand_val[kMaxTopK];
    __shared__ int cand_idx[kMaxTopK];
    __shared__ float red_val[NTH / 64];
    __shared__ int red_idx[NTH / 64];
    __shared__ uint32_t sh_thresh, sh_n;
    __shared__ __attribute__((aligned(16))) uint32_t tkey[kThreads];
    __shared__ uint32_t pool_key[kPoolCap];
    __shared__ int pool_idx[kPoolCap];
    __shared__ float pool_val[kPoolCap];
    const int s = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const float *row = logits + (size_t)s * V;
    // REG: the whole row is read once, as 16-byte loads all in flight together,
    // into registers (thread t holds elements 4 (t + 256 j) .. + 3); every pass
    // below then visits (index, value) pairs from there.
    float4 vals[REG ? kRegF4 : 1];
    if constexpr (REG) {
        const auto rr = make_rsrc(row, (uint32_t)V * 4u);
#pragma unroll
        for (int j = 0; j < kRegF4; ++j)
            vals[j] = __builtin_bit_cast(
                float4, __builtin_amdgcn_raw_buffer_load_b128(rr, (uint32_t)(tid + j * NTH) * 16u, 0, 0));
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
            for (int i = tid; i < V; i += NTH) fn(i, row[i]);
        }
    };

    if (!(temperature > 0.0f)) {
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
                if (red_val[w] > best || (red_val[w] == best && red_idx[w] < bi)) { best = red_val[w]; bi = red_idx[w]; }
            tokens[s] = bi < V ? bi : 0;
        }
        return;
    }

    const int k = top_k < V ? top_k : V;
    // Lower bound: the k-th largest of the 256 group maxima (a group is GRP
    // adjacent threads; rank by key, then group): k groups hold a logit at
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
        // Exact rank of each pooled logit; ranks below k are the top k (the pool
        // order does not matter: a rank depends only on (key, token id)).
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
        radix_topk<NTH>(row, V, k, tid, hist, sh_prefix, sh_remaining, sh_gt, sh_eq, cand_val, cand_idx);
    }
    __syncthreads();
    if (wave == 0) {
        float best = -INFINITY;
        int bi = 0x7fffffff;
        if (lane < k) {
            const float u = uniform01(seed, counter, s, cand_idx[lane]);
            best = cand_val[lane] / temperature - __logf(-__logf(u));
            bi = cand_idx[lane];
        }
        for (int off = 32; off >= 1; off >>= 1) {
            const float ov = __shfl_xor(best, off);
            const int oi = __shfl_xor(bi, off);
            if (ov > best || (ov == best && oi < bi)) { best = ov; bi = oi; }
        }
        if (lane == 0) tokens[s] = bi < V ? bi : 0;
    }
}

}  // namespace

hipError_t launch_sample(int n, int V, const float *logits, float temperature, int top_k, uint64_t seed,
                         uint64_t counter, int32_t *tokens, hipStream_t stream) {
    if (n <= 0) return hipSuccess;
    if (temperature > 0.0f && (top_k < 1 || top_k > kMaxTopK)) return hipErrorInvalidValue;
    if (V <= kRegElems)
        hipLaunchKernelGGL((sample_kernel<kRegThreads, true>), dim3(n), dim3(kRegThreads), 0, stream, V, logits,
                           temperature, top_k, seed, counter, tokens);
    else
        hipLaunchKernelGGL((sample_kernel<kThreads, false>), dim3(n), dim3(kThreads), 0, stream, V, logits,
                           temperature, top_k, seed, counter, tokens);
    return hipGetLastError();
}

}  // namespace yuf

extern "C" int yuf_sample_device(int n, int V, const float *logits_dev, float temperature, int top_k, uint64_t seed,
                                 uint64_t counter, int32_t *tokens_dev, void *stream) {
    using namespace yuf;
    if (n < 0 || V <= 0) return fail(YUF_ERR_INVALID, "sample_device: bad sizes");
    if (temperature > 0.0f && (top_k < 1 || top_k > kMaxTopK))
        return fail(YUF_ERR_INVALID, "sample_device: top_k must be in [1, 64] when temperature > 0");
    if (n > 0 && (!logits_dev || !tokens_dev)) return fail(YUF_ERR_INVALID, "sample_device: null pointer");
    hipError_t err = launch_sample(n, V, logits_dev, temperature, top_k, seed, counter, tokens_dev,
                                   static_cast<hipStream_t>(stream));
    if (err != hipSuccess) return fail(YUF_ERR_HIP, std::string("sample launch: ") + hipGetErrorString(err));
    return YUF_OK;
}
