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
#include <cstdlib>
#include <cstring>

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
    static constexpr int R = kWave / L;                        // rows per wave
    static constexpr int W = (N + R - 1) / R;                  // waves per head
    static constexpr int P = ((5 * E + 3) / 4) * 4;            // floats per (token, lane-column)
    static constexpr int kCols = kChunk * L * P;               // staged operands of one chunk
    static constexpr int kF4 = N / 4;                          // float4 per token row of a head
    static constexpr int kItems = (kChunk * kF4 + kWave - 1) / kWave;
    static constexpr int kVF4 = R / 4;                         // float4 of v per token
    static constexpr int kVItems = (kChunk * kVF4 + kWave - 1) / kWave;
};

// Operand slots inside a lane's P floats: [a | d | b | k | r], E each.
enum : int { kA = 0, kD = 1, kB = 2, kK = 3, kR = 4 };
// Raw per-token vectors staged before the decay pass.
enum : int { kRawR = 0, kRawW = 1, kRawK = 2, kRawA = 3, kRawB = 4, kNumRaw = 5 };

template <int N>
struct Stage {
    using Lay = Layout<N>;
    float4 x[kNumRaw][Lay::kItems];
    float4 v[Lay::kVItems];
};

__device__ __forceinline__ float4 buf_load4(__amdgpu_buffer_rsrc_t rsrc, uint32_t byte_offset) {
    return __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(rsrc, byte_offset, 0, 0));
}

// Issue the HBM reads of one chunk (16-byte bounds-checked buffer loads; tokens
// past the chunk end fall outside the descriptors and read as 0).
template <int N, bool PREP>
__device__ __forceinline__ void stage_load(Stage<N> &st, const WkvParams &p, int bb, int h, int row0, int t0,
                                           int nt, int lane) {
    using Lay = Layout<N>;
    const size_t base = ((size_t)(bb * p.T + t0) * p.H + h) * N;
    const uint32_t bytes = nt > 0 ? (uint32_t)(((nt - 1) * p.H * N + N) * 4) : 0u;
    const float *src[kNumRaw] = {p.r, p.w, p.k, p.a, PREP ? p.a : p.b};
    const int stride = p.H * N;
#pragma unroll
    for (int c = 0; c < (PREP ? kNumRaw - 1 : kNumRaw); ++c) {
        const auto rs = make_rsrc(src[c] + base, bytes);
#pragma unroll
        for (int it = 0; it < Lay::kItems; ++it) {
            const int q = lane + it * kWave;
            const int t = q / Lay::kF4, f = q - t * Lay::kF4;
            st.x[c][it] = buf_load4(rs, q < kChunk * Lay::kF4 ? (uint32_t)(t * stride + f * 4) * 4u : kBufferOob);
        }
    }
    const auto rv = make_rsrc(p.v + base, bytes);
#pragma unroll
    for (int it = 0; it < Lay::kVItems; ++it) {
        const int q = lane + it * kWave;
        const int t = q / Lay::kVF4, f = q - t * Lay::kVF4;
        const bool ok = q < kChunk * Lay::kVF4 && row0 + f * 4 < N;
        st.v[it] = buf_load4(rv, ok ? (uint32_t)(t * stride + row0 + f * 4) * 4u : kBufferOob);
    }
}

// Turn a staged chunk into the per-lane operand layout: for token t and lane
// column group cl, P contiguous floats [a | d | b | k | r] (E each), so a lane
// fetches one token's operands with ds_read_b128.  Work is spread over all
// lanes as (token, 4-column) items.
template <int N, bool PREP>
__device__ __forceinline__ void stage_store(const Stage<N> &st, const WkvParams &p, int h, int nt, int lane,
                                            float *raw, float *cols, float *vbuf, float *psq, float *inv_norm) {
    using Lay = Layout<N>;
    constexpr int E = Lay::E, P = Lay::P, L = Lay::L, F4 = Lay::kF4;
#pragma unroll
    for (int c = 0; c < (PREP ? kNumRaw - 1 : kNumRaw); ++c)
#pragma unroll
        for (int it = 0; it < Lay::kItems; ++it) {
            const int q = lane + it * kWave;
            if (q < kChunk * F4) reinterpret_cast<float4 *>(raw + c * kChunk * N)[q] = st.x[c][it];
        }
#pragma unroll
    for (int it = 0; it < Lay::kVItems; ++it) {
        const int q = lane + it * kWave;
        if (q < kChunk * Lay::kVF4) reinterpret_cast<float4 *>(vbuf)[q] = st.v[it];
    }
    if constexpr (PREP) {
        // Per-token L2 norm of k * k_k over the head (F.normalize, eps 1e-12):
        // partial sums of squares per 4 columns, then one lane per token.
#pragma unroll
        for (int it = 0; it < Lay::kItems; ++it) {
            const int q = lane + it * kWave;
            if (q < kChunk * F4) {
                const int f = q - (q / F4) * F4;
                const float4 kv = st.x[kRawK][it];
                const float4 kk = *reinterpret_cast<const float4 *>(p.k_k + h * N + f * 4);
                const float x0 = kv.x * kk.x, x1 = kv.y * kk.y, x2 = kv.z * kk.z, x3 = kv.w * kk.w;
                psq[q] = fmaf(x0, x0, fmaf(x1, x1, fmaf(x2, x2, x3 * x3)));
            }
        }
        lds_barrier();
        if (lane < nt) {
            float acc = 0.0f;
            for (int f = 0; f < F4; ++f) acc += psq[lane * F4 + f];
            inv_norm[lane] = 1.0f / fmaxf(sqrtf(acc), 1e-12f);
        }
    }
    lds_barrier();
    for (int q = lane; q < nt * F4; q += kWave) {
        const int t = q / F4, f = q - t * F4;
        const float4 r4 = reinterpret_cast<const float4 *>(raw + kRawR * kChunk * N)[q];
        const float4 w4 = reinterpret_cast<const float4 *>(raw + kRawW * kChunk * N)[q];
        const float4 k4 = reinterpret_cast<const float4 *>(raw + kRawK * kChunk * N)[q];
        const float4 a4 = reinterpret_cast<const float4 *>(raw + kRawA * kChunk * N)[q];
        float4 b4 = a4;
        if constexpr (!PREP) b4 = reinterpret_cast<const float4 *>(raw + kRawB * kChunk * N)[q];
        const float rr[4] = {r4.x, r4.y, r4.z, r4.w}, ww[4] = {w4.x, w4.y, w4.z, w4.w};
        const float kk[4] = {k4.x, k4.y, k4.z, k4.w}, aa[4] = {a4.x, a4.y, a4.z, a4.w};
        const float bb[4] = {b4.x, b4.y, b4.z, b4.w};
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int j = f * 4 + u;
            // d = exp(-e^{-0.5} sigmoid(w)) = exp2(-e^{-0.5} log2(e) sigmoid(w)).
            const float sig = __frcp_rn(1.0f + __expf(-ww[u]));
            const float dv = exp2f(-0.8750387749f * sig);
            float av, bv, kv;
            if constexpr (PREP) {
                const float kap = kk[u] * p.k_k[h * N + j] * inv_norm[t];
                av = -kap;
                bv = kap * aa[u];
                kv = kk[u] * (1.0f + (aa[u] - 1.0f) * p.k_a[h * N + j]);
            } else {
                av = aa[u];
                bv = bb[u];
                kv = kk[u];
            }
            const int cl = j / E, e = j - cl * E;
            float *dst = cols + (t * L + cl) * P + e;
            dst[kA * E] = av;
            dst[kD * E] = dv;
            dst[kB * E] = bv;
            dst[kK * E] = kv;
            dst[kR * E] = rr[u];
        }
    }
    lds_barrier();
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
    __shared__ __attribute__((aligned(16))) float raw[kNumRaw * kChunk * N];
    __shared__ __attribute__((aligned(16))) float cols[Lay::kCols];
    __shared__ __attribute__((aligned(16))) float vbuf[kChunk * R];
    __shared__ float ybuf[kChunk * R];
    __shared__ float psq[PREP ? kChunk * Lay::kF4 : 1];
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
    {
        const auto rs = make_rsrc(p.state_in ? p.state_in + state_off : nullptr, p.state_in ? N * N * 4 : 0u);
#pragma unroll
        for (int e = 0; e < E; ++e)
            s[e] = buf_load(rs, row_ok ? (uint32_t)(i * N + cl * E + e) * 4u : kBufferOob);
    }
    wait_vmem();

    const int n_chunks = (p.T + kChunk - 1) / kChunk;
    Stage<N> st;
    if (n_chunks > 0) stage_load<N, PREP>(st, p, bb, h, row0, 0, min(kChunk, p.T), lane);
    for (int c = 0; c < n_chunks; ++c) {
        const int t0 = c * kChunk;
        const int nt = min(kChunk, p.T - t0);
        stage_store<N, PREP>(st, p, h, nt, lane, raw, cols, vbuf, psq, inv_norm);
        if (c + 1 < n_chunks) stage_load<N, PREP>(st, p, bb, h, row0, t0 + kChunk, min(kChunk, p.T - t0 - kChunk), lane);
        if (nt == kChunk)
            chunk_steps<N, true>(s, cols, vbuf, ybuf, nt, rl, cl);
        else
            chunk_steps<N, false>(s, cols, vbuf, ybuf, nt, rl, cl);
        lds_barrier();
        // This chunk's outputs: R contiguous rows per token, stored through a
        // buffer descriptor (stores past the chunk end or past row N drop).
        {
            const size_t ybase = ((size_t)(bb * p.T + t0) * p.H + h) * N;
            const auto ry = make_rsrc(p.y + ybase, (uint32_t)(((nt - 1) * p.H * N + N) * 4));
#pragma unroll
            for (int it = 0; it < (kChunk * R + kWave - 1) / kWave; ++it) {
                const int q = lane + it * kWave;
                const int t = q / R, rr = q - t * R;
                const bool ok = q < kChunk * R && t < nt && row0 + rr < N;
                buf_store(ybuf[ok ? q : 0], ry, ok ? (uint32_t)(t * p.H * N + row0 + rr) * 4u : kBufferOob);
            }
        }
    }
    if (p.state_out && row_ok) {
#pragma unroll
        for (int e = 0; e < E; ++e) p.state_out[state_off + (size_t)i * N + cl * E + e] = s[e];
    }
}

// Single-token step (T = 1, decode): 256 threads per (stream, head), SPW
// streams of one head per workgroup.  The state streams in and out as 16-byte
// runs (float4 q of the row-major N x N state is row 4q / N, columns 4q % N ..
// + 3; N % 4 == 0); the per-token vectors are prepared once per head in LDS
// (decay, and in the model path kappa = normalize(k k_k), a = -kappa, b = kappa
// alpha, k^ = k (1 + (alpha - 1) k_a)); the row sums S a and S' r go through
// per-float4 partials in LDS.  Every global load is issued before the first
// barrier, so a step costs one HBM round trip plus four barriers.
//
// LR (model decode path): the second low-rank stage runs here instead of as a
// GEMM -- w, alpha and the output gate g of the head's N channels are dot
// products of the stream's rank-L rows with the head's N x L slices of w2t,
// a2t, g2t, staged once per workgroup in LDS and shared by its SPW streams.
constexpr int kStepThreads = 256;
constexpr int kStepLrSpw = 4;       // streams per workgroup of the LR form
constexpr int kStepLrMaxL = 128;  // an LDS weight row holds kStepLrMaxL + 2 floats (even / odd lanes on distinct banks)
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

template <int N, bool PREP, int SPW, bool LR>
__global__ void __launch_bounds__(kStepThreads * SPW) wkv7_step_kernel(WkvParams p) {
    static_assert(!LR || (PREP && 3 * N <= kStepThreads), "fused low-rank layout");
    constexpr int Q = N * N / 4;                                 // float4 of the state
    constexpr int QM = (Q + kStepThreads - 1) / kStepThreads;   // per thread
    constexpr int RQ = N / 4;                                    // float4 per row
    constexpr int LP = kStepLrMaxL + 2;                          // padded LDS row of a weight slice
    __shared__ __attribute__((aligned(16))) float vec[SPW][6][N];  // a, b, k^, d, r, v
    __shared__ float part[SPW][Q];                                 // per-float4 partial row sums
    __shared__ float rowv[SPW][N];                                 // S a, then y
    __shared__ float red[SPW][kStepThreads / 64];
    __shared__ float wl[LR ? 3 * N : 1][LR ? LP : 1];              // w2t | a2t | g2t rows of the head
    __shared__ float lrs[LR ? SPW : 1][LR ? 3 : 1][LR ? kStepLrMaxL : 1];
    __shared__ float lrv[LR ? SPW : 1][2][LR ? N : 1];             // w, alpha

    const int sub = threadIdx.x / kStepThreads, tid = threadIdx.x % kStepThreads;
    const int lane = tid & 63, wave = tid >> 6;
    const int h = blockIdx.x % p.H, bb = (blockIdx.x / p.H) * SPW + sub;
    const bool live = bb < p.B;  // idle streams of the last workgroup still meet every barrier
    const int slot = live ? (p.slot ? p.slot[bb] : bb) : 0;
    const size_t state_off = ((size_t)slot * p.H + h) * N * N;
    const size_t base = ((size_t)(live ? bb : 0) * p.H + h) * N;  // token (bb, 0)

    // All global loads first: the state's float4s, then one column / row per thread.
    const auto rs = make_rsrc(live && p.state_in ? p.state_in + state_off : nullptr,
                              live && p.state_in ? N * N * 4 : 0u);
    float4 sq[QM];
#pragma unroll
    for (int m = 0; m < QM; ++m) {
        const int q = tid + m * kStepThreads;
        sq[m] = buf_load4(rs, q < Q ? (uint32_t)q * 16u : kBufferOob);
    }
    const bool col = tid < N;
    const uint32_t off = col && live ? (uint32_t)tid * 4u : kBufferOob;
    const float rv = buf_load(make_rsrc(p.r + base, N * 4), off);
    float wv = 0.0f, av = 0.0f;
    if constexpr (!LR) {
        wv = buf_load(make_rsrc(p.w + base, N * 4), off);
        av = buf_load(make_rsrc(p.a + base, N * 4), off);
    }
    float kv = buf_load(make_rsrc(p.k + base, N * 4), off);
    const float vv = buf_load(make_rsrc(p.v + base, N * 4), off);
    float bv = 0.0f, kk = 0.0f, ka = 0.0f;
    if constexpr (PREP) {
        kk = buf_load(make_rsrc(p.k_k + h * N, N * 4), off);
        ka = buf_load(make_rsrc(p.k_a + h * N, N * 4), off);
    } else {
        bv = buf_load(make_rsrc(p.b + base, N * 4), off);
    }
    if constexpr (LR) {
        // Stage the head's weight rows (3 N rows of L, contiguous N x L blocks)
        // and the streams' rank-L rows: every load is issued before the first
        // LDS write, so staging costs one memory latency.
        constexpr int kT = kStepThreads * SPW;
        constexpr int kW4 = (N * kStepLrMaxL / 4 + kT - 1) / kT;  // float4 per thread and matrix
        constexpr int kL1 = (SPW * 3 * kStepLrMaxL + kT - 1) / kT;
        const int L = p.L, nl4 = N * L / 4, flat = threadIdx.x;
        float4 wreg[3][kW4];
#pragma unroll
        for (int m = 0; m < 3; ++m) {
            const float *src = m == 0 ? p.w2t : (m == 1 ? p.a2t : p.g2t);
            const auto rw = make_rsrc(src + (size_t)h * N * L, (uint32_t)(N * L * 4));
#pragma unroll
            for (int i = 0; i < kW4; ++i) {
                const int e4 = flat + i * kT;
                wreg[m][i] = buf_load4(rw, e4 < nl4 ? (uint32_t)e4 * 16u : kBufferOob);
            }
        }
        float lreg[kL1];
#pragma unroll
        for (int i = 0; i < kL1; ++i) {
            const int e = flat + i * kT;
            const int sb = e / (3 * L), rem = e - sb * 3 * L, m = rem / L, j = rem - m * L;
            const int b2 = (blockIdx.x / p.H) * SPW + sb;
            const bool ok = sb < SPW && b2 < p.B;
            lreg[i] = ok ? p.lr[m * p.lr_plane + (size_t)b2 * L + j] : 0.0f;
        }
        const float w0c = col ? p.w0[h * N + tid] : 0.0f, a0c = col ? p.a0[h * N + tid] : 0.0f;
#pragma unroll
        for (int m = 0; m < 3; ++m)
#pragma unroll
            for (int i = 0; i < kW4; ++i) {
                const int e4 = flat + i * kT;
                if (e4 < nl4) {
                    const int c = (4 * e4) / L, j = 4 * e4 - c * L;  // L % 8 == 0
                    float *dst = &wl[m * N + c][j];
                    dst[0] = wreg[m][i].x; dst[1] = wreg[m][i].y; dst[2] = wreg[m][i].z; dst[3] = wreg[m][i].w;
                }
            }
#pragma unroll
        for (int i = 0; i < kL1; ++i) {
            const int e = flat + i * kT;
            const int sb = e / (3 * L), rem = e - sb * 3 * L, m = rem / L, j = rem - m * L;
            if (sb < SPW) lrs[sb][m][j] = lreg[i];
        }
        lds_barrier();
        // One dot per thread (PAIR = false) or per lane pair, the even and odd
        // j of a dot on lanes 2q and 2q + 1, summed through a DPP swap.
        constexpr bool PAIR = 6 * N <= kStepThreads;
        constexpr int TPD = PAIR ? 2 : 1;
        if (tid < 3 * N * TPD) {
            const int dq = tid / TPD, hj = tid % TPD, m = dq / N, c = dq - m * N;
            const float *wrow = &wl[m * N + c][hj];
            const float *lrow = &lrs[sub][m][hj];
            float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll 4
            for (int i = 0; i < L / TPD; i += 4)  // L % 8 == 0
#pragma unroll
                for (int t = 0; t < 4; ++t) acc[t] = fmaf(lrow[TPD * (i + t)], wrow[TPD * (i + t)], acc[t]);
            float dot = (acc[0] + acc[1]) + (acc[2] + acc[3]);
            if constexpr (PAIR) dot += dpp_move<dpp::kQuadXor1>(dot);
            if (hj == 0) {
                if (m == 2) {
                    if (live)
                        p.g_out[p.tiled_out ? tile_index(bb, h * N + c, p.H * N) : (size_t)bb * p.H * N + h * N + c] =
                            1.0f / (1.0f + expf(-dot));
                } else {
                    lrv[sub][m][c] = dot;
                }
            }
        }
        lds_barrier();
        if (col) {
            wv = w0c + lrv[sub][0][tid];
            av = 1.0f / (1.0f + expf(-(a0c + lrv[sub][1][tid])));
        }
    }
    if constexpr (PREP) {
        // kappa = normalize(k * k_k) over the head (F.normalize, eps 1e-12).
        const float x = kv * kk;
        const float ws = wave_sum(x * x);
        if (lane == 0) red[sub][wave] = ws;
        lds_barrier();
        float sq2 = 0.0f;
#pragma unroll
        for (int w = 0; w < (N + 63) / 64; ++w) sq2 += red[sub][w];
        const float inv = 1.0f / fmaxf(sqrtf(sq2), 1e-12f);
        const float kap = x * inv, alpha = av;
        av = -kap;
        bv = kap * alpha;
        kv = kv * (1.0f + (alpha - 1.0f) * ka);
    }
    if (col) {
        // d = exp(-e^{-0.5} sigmoid(w)) = exp2(-e^{-0.5} log2(e) sigmoid(w)).
        const float sig = __frcp_rn(1.0f + __expf(-wv));
        vec[sub][0][tid] = av;
        vec[sub][1][tid] = bv;
        vec[sub][2][tid] = kv;
        vec[sub][3][tid] = exp2f(-0.8750387749f * sig);
        vec[sub][4][tid] = rv;
        vec[sub][5][tid] = vv;
    }
    lds_barrier();
    // sa_i = sum_j S_ij a_j.
#pragma unroll
    for (int m = 0; m < QM; ++m) {
        const int q = tid + m * kStepThreads;
        if (q < Q) {
            const float4 a4 = *reinterpret_cast<const float4 *>(&vec[sub][0][(4 * q) % N]);
            part[sub][q] = (sq[m].x * a4.x + sq[m].y * a4.y) + (sq[m].z * a4.z + sq[m].w * a4.w);
        }
    }
    lds_barrier();
    if (tid < N) {
        float sa = 0.0f;
#pragma unroll
        for (int u = 0; u < RQ; ++u) sa += part[sub][tid * RQ + u];
        rowv[sub][tid] = sa;
    }
    lds_barrier();
    // S'_ij = S_ij d_j + sa_i b_j + v_i k^_j;  y_i = sum_j S'_ij r_j.
    const auto ro = make_rsrc(live && p.state_out ? p.state_out + state_off : nullptr,
                              live && p.state_out ? N * N * 4 : 0u);
#pragma unroll
    for (int m = 0; m < QM; ++m) {
        const int q = tid + m * kStepThreads;
        if (q < Q) {
            const int i = (4 * q) / N, c = (4 * q) % N;
            const float sa = rowv[sub][i], vi = vec[sub][5][i];
            const float4 b4 = *reinterpret_cast<const float4 *>(&vec[sub][1][c]);
            const float4 k4 = *reinterpret_cast<const float4 *>(&vec[sub][2][c]);
            const float4 d4 = *reinterpret_cast<const float4 *>(&vec[sub][3][c]);
            const float4 r4 = *reinterpret_cast<const float4 *>(&vec[sub][4][c]);
            float4 x;
            x.x = fmaf(sq[m].x, d4.x, fmaf(sa, b4.x, k4.x * vi));
            x.y = fmaf(sq[m].y, d4.y, fmaf(sa, b4.y, k4.y * vi));
            x.z = fmaf(sq[m].z, d4.z, fmaf(sa, b4.z, k4.z * vi));
            x.w = fmaf(sq[m].w, d4.w, fmaf(sa, b4.w, k4.w * vi));
            part[sub][q] = (x.x * r4.x + x.y * r4.y) + (x.z * r4.z + x.w * r4.w);
            if (p.state_out)
                __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, x), ro, (uint32_t)q * 16u, 0, 0);
        }
    }
    lds_barrier();
    if (tid < N && live) {
        float yv = 0.0f;
#pragma unroll
        for (int u = 0; u < RQ; ++u) yv += part[sub][tid * RQ + u];
        p.y[p.tiled_out ? tile_index(bb, h * N + tid, p.H * N) : base + tid] = yv;
    }
}

template <int N>
hipError_t launch_step_n(const WkvParams &p, bool prep, hipStream_t stream) {
    static_assert(N % 4 == 0 && N <= kStepThreads, "step kernel layout");
    if (p.lr) {
        if constexpr (3 * N <= kStepThreads) {
            if (!prep || !wkv7_step_lowrank_ok(N, p.L)) return hipErrorInvalidValue;
            const dim3 grid(((p.B + kStepLrSpw - 1) / kStepLrSpw) * p.H), block(kStepThreads * kStepLrSpw);
            hipLaunchKernelGGL((wkv7_step_kernel<N, true, kStepLrSpw, true>), grid, block, 0, stream, p);
            return hipGetLastError();
        } else {
            return hipErrorInvalidValue;
        }
    }
    const dim3 grid(p.B * p.H), block(kStepThreads);
    if (prep)
        hipLaunchKernelGGL((wkv7_step_kernel<N, true, 1, false>), grid, block, 0, stream, p);
    else
        hipLaunchKernelGGL((wkv7_step_kernel<N, false, 1, false>), grid, block, 0, stream, p);
    return hipGetLastError();
}

template <int N>
hipError_t launch_n(const WkvParams &p, bool prep, hipStream_t stream) {
    if (p.T == 1) return launch_step_n<N>(p, prep, stream);
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

bool wkv7_step_lowrank_ok(int N, int L) {
    return (N == 8 || N == 16 || N == 32 || N == 40 || N == 48 || N == 64) && L >= 8 && L <= kStepLrMaxL &&
           L % 8 == 0;
}

bool wkv7_supported(int N) {
    return N == 8 || N == 16 || N == 32 || N == 40 || N == 48 || N == 64 || N == 128;
}

hipError_t launch_wkv7(const WkvParams &p, int N, bool prep, hipStream_t stream) {
    if (p.B <= 0 || p.H <= 0) return hipSuccess;
    const char *force = std::getenv("YUF_WKV7_KERNEL");
    const bool want_serial = force && std::strcmp(force, "serial") == 0;
    const bool want_chunked = force && std::strcmp(force, "chunked") == 0;
    // The fused low-rank form is the single-token step kernel only, and so are
    // tiled outputs (which the fused form's callers use).
    if (p.lr && (p.T != 1 || !prep)) return hipErrorInvalidValue;
    if (p.tiled_out && !p.lr) return hipErrorInvalidValue;
    if (!p.lr && wkv7_chunk_supported(N) && !want_serial && (want_chunked || p.T >= kWkvChunkMinT))
        return launch_wkv7_chunked(p, N, prep, stream);
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
