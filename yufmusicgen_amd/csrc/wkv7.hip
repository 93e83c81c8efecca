// WKV-7 TimeMix scan for gfx950 (MI355X).
//
// Semantics: yufmusicgen/model.py:145-165 (the stateful PyTorch recurrence) and
// yufmusicgen/cuda/rwkv7_clampw.cu:20-75 (decay form :16,:42).  Per (b, h):
//     d = exp(-e^{-0.5} sigmoid(w_raw)),  sa = S a,
//     S <- S diag(d) + sa b^T + v k^T,    y = S r,
// with S in R^{N x N}, row i = value index, column j = key index.
//
// Design (not a translation of the CUDA kernel, which gives one thread a whole
// row and uses 2 block barriers per token):
//   * Rows of S are independent given the per-token column vectors, so a head
//     is split over W = N / R single-wave workgroups of R rows each; B*H*W
//     waves spread over all CUs (C2: 640 waves) instead of B*H blocks.
//   * Inside a wave, a row is held by L consecutive lanes, E = N / L columns
//     each (N = 40: L = 8, E = 5).  The two row reductions per token (S a and
//     S r) are L-lane DPP butterflies -- no LDS round trip, no barrier.
//   * Tokens are processed in 16-token chunks.  A chunk's column vectors
//     (a, decay, b, k, r) are staged in LDS in a per-lane-contiguous layout
//     so each lane fetches its 5E values per token with ds_read_b128; the next
//     chunk's HBM loads are issued before the current chunk is computed
//     (register prefetch, double-buffered LDS).  Decay exponentials are
//     computed once per (token, column) during staging.
//   * Waves of one head get consecutive flat indices laid out per XCD, so the
//     shared column vectors are read from HBM once and then hit that XCD's L2.
//   * Any T (no padding), optional non-zero initial state, optional state
//     slots (decode / stateful prefill), and a fused-prep mode that builds
//     kappa = normalize(k * k_k), a = -kappa, b = kappa * alpha and
//     k_hat = k (1 + (alpha - 1) k_a) from the projections during staging
//     (yufmusicgen/model.py:114-122), so the model path never materialises them.
#include "common.h"
#include "kernels.h"

namespace yuf {
namespace {

constexpr float kWScale = 0.6065306597f;  // exp(-0.5)
constexpr int kChunk = 16;
constexpr int kWave = 64;
constexpr int kXcds = 8;

// Lanes per row (L) and columns per lane (E) for each supported head size.
template <int N> struct Shape;
template <> struct Shape<8> { static constexpr int L = 8, E = 1; };
template <> struct Shape<16> { static constexpr int L = 4, E = 4; };
template <> struct Shape<32> { static constexpr int L = 8, E = 4; };
template <> struct Shape<40> { static constexpr int L = 8, E = 5; };
template <> struct Shape<48> { static constexpr int L = 8, E = 6; };
template <> struct Shape<64> { static constexpr int L = 8, E = 8; };
template <> struct Shape<128> { static constexpr int L = 16, E = 8; };

template <int N>
struct Layout {
    static constexpr int L = Shape<N>::L;
    static constexpr int E = Shape<N>::E;
    static constexpr int R = kWave / L;                  // rows per wave
    static constexpr int W = (N + R - 1) / R;            // waves per head
    static constexpr int P = ((5 * E + 3) / 4) * 4;      // floats per (token, lane-column)
    static constexpr int kCols = kChunk * L * P;         // one LDS buffer of column vectors
    static constexpr int kItems = (kChunk * N + kWave - 1) / kWave;  // staging items per lane
    static constexpr int kVItems = (kChunk * R + kWave - 1) / kWave;
};

// Vector slots inside a lane's P floats: [a | d | b | k | r], E each.
enum : int { kA = 0, kD = 1, kB = 2, kK = 3, kR = 4 };

template <int N, bool PREP>
struct Stage {
    using Lay = Layout<N>;
    float r[Lay::kItems], w[Lay::kItems], k[Lay::kItems], a[Lay::kItems], b[Lay::kItems];
    float v[Lay::kVItems];
};

template <int N, bool PREP>
__device__ __forceinline__ void stage_load(Stage<N, PREP> &st, const WkvParams &p, int bb, int h,
                                           int row0, int t0, int nt, int lane) {
    using Lay = Layout<N>;
    // Token t of this chunk starts t * H * N floats after `base`; tokens past
    // the chunk end fall outside the descriptor range and load as 0.
    const size_t base = ((size_t)(bb * p.T + t0) * p.H + h) * N;
    const uint32_t bytes = nt > 0 ? (uint32_t)(((nt - 1) * p.H * N + N) * 4) : 0u;
    const auto rr_ = make_rsrc(p.r + base, bytes), rw_ = make_rsrc(p.w + base, bytes);
    const auto rk_ = make_rsrc(p.k + base, bytes), ra_ = make_rsrc(p.a + base, bytes);
    const auto rv_ = make_rsrc(p.v + base, bytes);
    const int stride = p.H * N;
#pragma unroll
    for (int it = 0; it < Lay::kItems; ++it) {
        const int q = lane + it * kWave;
        const int t = q / N, j = q - t * N;
        const uint32_t off = (uint32_t)(t * stride + j) * 4u;
        st.r[it] = buf_load(rr_, off);
        st.w[it] = buf_load(rw_, off);
        st.k[it] = buf_load(rk_, off);
        st.a[it] = buf_load(ra_, off);
        if constexpr (!PREP) st.b[it] = buf_load(make_rsrc(p.b + base, bytes), off);
    }
#pragma unroll
    for (int it = 0; it < Lay::kVItems; ++it) {
        const int q = lane + it * kWave;
        const int t = q / Lay::R, rr = q - t * Lay::R;
        const bool ok = row0 + rr < N && q < kChunk * Lay::R;
        st.v[it] = buf_load(rv_, ok ? (uint32_t)(t * stride + row0 + rr) * 4u : kBufferOob);
    }
}

// Transform the prefetched registers into the LDS layout of buffer `cols`.
template <int N, bool PREP>
__device__ __forceinline__ void stage_store(Stage<N, PREP> &st, const WkvParams &p, int h, int nt,
                                            int lane, float *cols, float *vbuf, float *sq, float *inv_norm) {
    using Lay = Layout<N>;
    constexpr int E = Lay::E, P = Lay::P, L = Lay::L;
    float kk[Lay::kItems];
    if constexpr (PREP) {
        // Per-token L2 norm of k * k_k over the head (F.normalize, eps 1e-12),
        // summed in a fixed order so results are deterministic.
#pragma unroll
        for (int it = 0; it < Lay::kItems; ++it) {
            const int q = lane + it * kWave;
            const int t = q / N, j = q - t * N;
            kk[it] = 0.0f;
            if (q < kChunk * N && t < nt) {
                kk[it] = st.k[it] * p.k_k[h * N + j];
                sq[q] = kk[it] * kk[it];
            }
        }
        __syncthreads();
        if (lane < nt) {
            float acc = 0.0f;
            for (int j = 0; j < N; ++j) acc += sq[lane * N + j];
            inv_norm[lane] = 1.0f / fmaxf(sqrtf(acc), 1e-12f);
        }
        __syncthreads();
    }
#pragma unroll
    for (int it = 0; it < Lay::kItems; ++it) {
        const int q = lane + it * kWave;
        const int t = q / N, j = q - t * N;
        if (q < kChunk * N && t < nt) {
            float av, bv, kv;
            if constexpr (PREP) {
                const float kap = kk[it] * inv_norm[t];
                const float alpha = st.a[it];
                av = -kap;
                bv = kap * alpha;
                kv = st.k[it] * (1.0f + (alpha - 1.0f) * p.k_a[h * N + j]);
            } else {
                av = st.a[it];
                bv = st.b[it];
                kv = st.k[it];
            }
            const float dv = expf(-kWScale / (1.0f + expf(-st.w[it])));
            const int cl = j / E, e = j - cl * E;
            float *dst = cols + (t * L + cl) * P + e;
            dst[kA * E] = av;
            dst[kD * E] = dv;
            dst[kB * E] = bv;
            dst[kK * E] = kv;
            dst[kR * E] = st.r[it];
        }
    }
#pragma unroll
    for (int it = 0; it < Lay::kVItems; ++it) {
        const int q = lane + it * kWave;
        if (q < kChunk * Lay::R) vbuf[q] = st.v[it];
    }
}

template <int N>
__device__ __forceinline__ void load_step(float (&col)[Layout<N>::P], float &vi, const float *base,
                                          const float *vbuf, int t, int rl) {
    using Lay = Layout<N>;
    const float4 *src = reinterpret_cast<const float4 *>(base + t * Lay::L * Lay::P);
#pragma unroll
    for (int q = 0; q < Lay::P / 4; ++q) reinterpret_cast<float4 *>(col)[q] = src[q];
    vi = vbuf[t * Lay::R + rl];
}

// One chunk of the recurrence.  The LDS operands of token t+1 are fetched
// while token t is computed, so LDS latency stays off the sequential chain.
template <int N, bool FULL>
__device__ __forceinline__ void chunk_steps(float (&s)[Layout<N>::E], const float *cols, const float *vbuf,
                                            float *ybuf, int nt, int rl, int cl) {
    using Lay = Layout<N>;
    constexpr int E = Lay::E, P = Lay::P, L = Lay::L, R = Lay::R;
    const float *base = cols + cl * P;
    const int steps = FULL ? kChunk : nt;
    float cur[P], nxt[P];
    float vcur, vnxt = 0.0f;
    load_step<N>(cur, vcur, base, vbuf, 0, rl);
    constexpr int kUnroll = FULL ? kChunk : 1;
#pragma unroll kUnroll
    for (int t = 0; t < steps; ++t) {
        if (t + 1 < steps) load_step<N>(nxt, vnxt, base, vbuf, t + 1, rl);
        float sa = 0.0f;
#pragma unroll
        for (int e = 0; e < E; ++e) sa = fmaf(s[e], cur[kA * E + e], sa);
        sa = group_sum<L>(sa);
        float yv = 0.0f;
#pragma unroll
        for (int e = 0; e < E; ++e) {
            s[e] = fmaf(s[e], cur[kD * E + e], fmaf(sa, cur[kB * E + e], cur[kK * E + e] * vcur));
            yv = fmaf(s[e], cur[kR * E + e], yv);
        }
        yv = group_sum<L>(yv);
        // Every lane of the row holds the same sum; all write the same word.
        ybuf[t * R + rl] = yv;
#pragma unroll
        for (int q = 0; q < P; ++q) cur[q] = nxt[q];
        vcur = vnxt;
    }
}

template <int N, bool PREP>
__global__ void __launch_bounds__(kWave) wkv7_scan_kernel(WkvParams p, int waves_total, int per_xcd) {
    using Lay = Layout<N>;
    constexpr int E = Lay::E, L = Lay::L, R = Lay::R, W = Lay::W;
    __shared__ __attribute__((aligned(16))) float cols[2][Lay::kCols];
    __shared__ float vbuf[2][kChunk * R];
    __shared__ float ybuf[kChunk * R];
    __shared__ float sq[PREP ? kChunk * N : 1];
    __shared__ float inv_norm[kChunk];

    // XCD-aware flat index: blocks are dealt round-robin over the XCDs, so
    // give each XCD a contiguous range of (head, wave) indices.
    const int flat = (blockIdx.x % kXcds) * per_xcd + blockIdx.x / kXcds;
    if (flat >= waves_total) return;
    const int head = flat / W, wave = flat - head * W;
    const int bb = head / p.H, h = head - bb * p.H;
    const int lane = threadIdx.x;
    const int rl = lane / L, cl = lane - rl * L;
    const int row0 = wave * R;
    const int i = row0 + rl;
    const bool row_ok = i < N;
    const int slot = p.slot ? p.slot[bb] : bb;
    const size_t state_off = ((size_t)slot * p.H + h) * N * N;

    float s[E];
#pragma unroll
    for (int e = 0; e < E; ++e)
        s[e] = (p.state_in && row_ok) ? p.state_in[state_off + (size_t)i * N + cl * E + e] : 0.0f;

    const int n_chunks = (p.T + kChunk - 1) / kChunk;
    Stage<N, PREP> st;
    if (n_chunks > 0) {
        const int nt0 = min(kChunk, p.T);
        stage_load<N, PREP>(st, p, bb, h, row0, 0, nt0, lane);
        stage_store<N, PREP>(st, p, h, nt0, lane, cols[0], vbuf[0], sq, inv_norm);
    }
    __syncthreads();
    for (int c = 0; c < n_chunks; ++c) {
        const int t0 = c * kChunk;
        const int nt = min(kChunk, p.T - t0);
        const int buf = c & 1;
        const bool more = c + 1 < n_chunks;
        const int nt_next = more ? min(kChunk, p.T - t0 - kChunk) : 0;
        if (more) stage_load<N, PREP>(st, p, bb, h, row0, t0 + kChunk, nt_next, lane);
        if (nt == kChunk)
            chunk_steps<N, true>(s, cols[buf], vbuf[buf], ybuf, nt, rl, cl);
        else
            chunk_steps<N, false>(s, cols[buf], vbuf[buf], ybuf, nt, rl, cl);
        __syncthreads();
        // Write this chunk's outputs: R contiguous rows per token.
        for (int q = lane; q < nt * R; q += kWave) {
            const int t = q / R, rr = q - t * R;
            if (row0 + rr < N) p.y[((size_t)(bb * p.T + t0 + t) * p.H + h) * N + row0 + rr] = ybuf[q];
        }
        if (more) stage_store<N, PREP>(st, p, h, nt_next, lane, cols[buf ^ 1], vbuf[buf ^ 1], sq, inv_norm);
        __syncthreads();
    }
    if (p.state_out && row_ok) {
#pragma unroll
        for (int e = 0; e < E; ++e) p.state_out[state_off + (size_t)i * N + cl * E + e] = s[e];
    }
}

template <int N>
hipError_t launch_n(const WkvParams &p, bool prep, hipStream_t stream) {
    using Lay = Layout<N>;
    const int waves = p.B * p.H * Lay::W;
    const int per_xcd = (waves + kXcds - 1) / kXcds;
    const dim3 grid(per_xcd * kXcds), block(kWave);
    if (prep)
        hipLaunchKernelGGL((wkv7_scan_kernel<N, true>), grid, block, 0, stream, p, waves, per_xcd);
    else
        hipLaunchKernelGGL((wkv7_scan_kernel<N, false>), grid, block, 0, stream, p, waves, per_xcd);
    return hipGetLastError();
}

}  // namespace

bool wkv7_supported(int N) {
    return N == 8 || N == 16 || N == 32 || N == 40 || N == 48 || N == 64 || N == 128;
}

hipError_t launch_wkv7(const WkvParams &p, int N, bool prep, hipStream_t stream) {
    if (p.B <= 0 || p.H <= 0) return hipSuccess;
    switch (N) {
        case 8: return launch_n<8>(p, prep, stream);
        case 16: return launch_n<16>(p, prep, stream);
        case 32: return launch_n<32>(p, prep, stream);
        case 40: return launch_n<40>(p, prep, stream);
        case 48: return launch_n<48>(p, prep, stream);
        case 64: return launch_n<64>(p, prep, stream);
        case 128: return launch_n<128>(p, prep, stream);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace yuf

// --------------------------------------------------------------------- C ABI
extern "C" int yuf_wkv7_scan_f32(int B, int T, int H, int N, const float *r, const float *w_raw,
                                 const float *k, const float *v, const float *a, const float *b,
                                 const float *state_in, float *state_out, float *y, void *stream) {
    using namespace yuf;
    if (B < 0 || T < 0 || H < 0) return fail(YUF_ERR_INVALID, "wkv7: negative size");
    if (!wkv7_supported(N)) return fail(YUF_ERR_INVALID, "wkv7: unsupported head size N=" + std::to_string(N));
    if (T > 0 && (!r || !w_raw || !k || !v || !a || !b || !y))
        return fail(YUF_ERR_INVALID, "wkv7: null input/output pointer");
    WkvParams p;
    p.B = B; p.T = T; p.H = H;
    p.r = r; p.w = w_raw; p.k = k; p.v = v; p.a = a; p.b = b;
    p.state_in = state_in; p.state_out = state_out; p.y = y;
    hipError_t err = launch_wkv7(p, N, false, static_cast<hipStream_t>(stream));
    if (err != hipSuccess) return fail(YUF_ERR_HIP, std::string("wkv7 launch: ") + hipGetErrorString(err));
    return YUF_OK;
}
