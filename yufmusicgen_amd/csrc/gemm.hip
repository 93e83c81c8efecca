// fp32 GEMM on the gfx950 matrix cores: C = epilogue(A W^T) (nn.Linear).
//
// Used for every projection of the model (r/k/v/output, the low-rank w/a/g
// pairs, ROSA in/out, the FFN and the tied LM head) -- the only dense
// contractions of the path.  Semantics of each call site: yufmusicgen/model.py
// :107-112 (TimeMix projections), :196 (output), :306-342 (ROSA), :377 (FFN),
// :421 (LM head).
//
// Kernel: 256 threads = 4 waves in a 2 x 2 arrangement; block tile 128 x 128,
// K tile 32, double-buffered LDS.  Each wave owns a 64 x 64 sub-tile as 2 x 2
// v_mfma_f32_32x32x2f32 accumulators (16 fp32 per lane each).  Operands are
// fetched from LDS with ds_read_b128: within a K tile, lanes 0-31 contract
// k in [0, 16) and lanes 32-63 k in [16, 32) (each MFMA sums one k of each
// half), so a lane's 16 A values for one 32-row fragment are contiguous.
// Global tiles are loaded with bounds-checked buffer loads (rows past M/N and
// the K tail read as zero) one K tile ahead of the MFMAs.  Blocks are dealt to
// XCDs so that consecutive tile indices share an XCD (and its L2).
//
// Epilogues fused into the store: + bias[n], tanh / sigmoid, + residual, and
// the paired SiLU gate of the FFN (W rows interleaved in blocks of 32 "in"
// then 32 "gate" rows; output silu(in) * gate).
#include "common.h"
#include "kernels.h"

namespace yuf {
namespace {

typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int kBM = 128, kBN = 128, kBK = 32, kPad = 4, kLd = kBK + kPad;
constexpr int kThreads = 256;
constexpr int kXcds = 8;

struct TileLoad {
    float4 v[4];
};

// 128 rows x 32 k: thread t loads rows t/8 + 32 i (i < 4), float4 column t % 8.
__device__ __forceinline__ void load_tile(TileLoad &tl, const float *base, int ld, int rows_left, int k0, int K,
                                          int tid) {
    const int rows = rows_left < kBM ? rows_left : kBM;
    const uint32_t bytes = rows > 0 ? (uint32_t)(((size_t)(rows - 1) * ld + K) * 4) : 0u;
    const auto rsrc = make_rsrc(base, bytes);
    const int c4 = tid & 7;
    const int k = k0 + c4 * 4;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int row = (tid >> 3) + 32 * i;
        float4 val;
        if (k + 3 < K) {
            const uint32_t off = (uint32_t)((size_t)row * ld + k) * 4u;
            const auto raw = __builtin_amdgcn_raw_buffer_load_b128(rsrc, off, 0, 0);
            val = __builtin_bit_cast(float4, raw);
        } else {
            // K tail (K % 4 may be non-zero): element-wise with explicit masks.
            float e[4];
#pragma unroll
            for (int q = 0; q < 4; ++q)
                e[q] = buf_load(rsrc, k + q < K ? (uint32_t)((size_t)row * ld + k + q) * 4u : kBufferOob);
            val = make_float4(e[0], e[1], e[2], e[3]);
        }
        tl.v[i] = val;
    }
}

__device__ __forceinline__ void store_tile(const TileLoad &tl, float *lds, int tid) {
    const int c4 = tid & 7;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int row = (tid >> 3) + 32 * i;
        *reinterpret_cast<float4 *>(lds + row * kLd + c4 * 4) = tl.v[i];
    }
}

__device__ __forceinline__ float apply_act(float x, int act) {
    if (act == ACT_TANH) return tanhf(x);
    if (act == ACT_SIGMOID) return 1.0f / (1.0f + expf(-x));
    return x;
}

__global__ void __launch_bounds__(kThreads) gemm_f32_kernel(GemmParams p, int tiles_m, int tiles_n, int per_xcd) {
    __shared__ __attribute__((aligned(16))) float As[2][kBM * kLd];
    __shared__ __attribute__((aligned(16))) float Bs[2][kBN * kLd];

    const int total = tiles_m * tiles_n;
    const int flat = (blockIdx.x % kXcds) * per_xcd + blockIdx.x / kXcds;
    if (flat >= total) return;
    const int bm = flat / tiles_n, bn = flat - bm * tiles_n;
    const int m0 = bm * kBM, n0 = bn * kBN;

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int wm = wave >> 1, wn = wave & 1;
    const float *a_base = p.A + (size_t)m0 * p.lda;
    const float *w_base = p.W + (size_t)n0 * p.ldw;

    floatx16 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = floatx16{};

    const int k_tiles = (p.K + kBK - 1) / kBK;
    TileLoad ta, tb;
    load_tile(ta, a_base, p.lda, p.M - m0, 0, p.K, tid);
    load_tile(tb, w_base, p.ldw, p.N - n0, 0, p.K, tid);
    store_tile(ta, As[0], tid);
    store_tile(tb, Bs[0], tid);
    __syncthreads();

    const int frag_row = lane & 31, frag_k = (lane >> 5) * 16;
    for (int kt = 0; kt < k_tiles; ++kt) {
        const int cur = kt & 1;
        const bool more = kt + 1 < k_tiles;
        if (more) {
            load_tile(ta, a_base, p.lda, p.M - m0, (kt + 1) * kBK, p.K, tid);
            load_tile(tb, w_base, p.ldw, p.N - n0, (kt + 1) * kBK, p.K, tid);
        }
        float af[2][16], bf[2][16];
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const float *pa = As[cur] + (wm * 64 + i * 32 + frag_row) * kLd + frag_k;
            const float *pb = Bs[cur] + (wn * 64 + i * 32 + frag_row) * kLd + frag_k;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                *reinterpret_cast<float4 *>(&af[i][q * 4]) = *reinterpret_cast<const float4 *>(pa + q * 4);
                *reinterpret_cast<float4 *>(&bf[i][q * 4]) = *reinterpret_cast<const float4 *>(pb + q * 4);
            }
        }
#pragma unroll
        for (int s = 0; s < 16; ++s)
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(af[i][s], bf[j][s], acc[i][j], 0, 0, 0);
        if (more) {
            store_tile(ta, As[cur ^ 1], tid);
            store_tile(tb, Bs[cur ^ 1], tid);
        }
        __syncthreads();
    }

    // Epilogue.  Accumulator element r of lane l holds
    // row = 8 (r / 4) + 4 (l / 32) + r % 4, column = l % 32 of its 32 x 32 tile.
    const int col_in_tile = lane & 31;
    const int row_base = (lane >> 5) * 4;
    if (p.silu_pair) {
        // Wave columns [0, 32) are "in", [32, 64) the matching "gate" rows.
        const int hcol = (n0 + wn * 64) / 2 + col_in_tile;
        if (hcol < p.N / 2) {
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int row = m0 + wm * 64 + i * 32 + (r >> 2) * 8 + row_base + (r & 3);
                    if (row < p.M) {
                        const float x = acc[i][0][r], g = acc[i][1][r];
                        p.C[(size_t)row * p.ldc + hcol] = x / (1.0f + expf(-x)) * g;
                    }
                }
        }
        return;
    }
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int col = n0 + wn * 64 + j * 32 + col_in_tile;
        if (col >= p.N) continue;
        const float bias = p.bias ? p.bias[col] : 0.0f;
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int row = m0 + wm * 64 + i * 32 + (r >> 2) * 8 + row_base + (r & 3);
                if (row < p.M) {
                    float x = apply_act(acc[i][j][r] + bias, p.act);
                    if (p.residual) x += p.residual[(size_t)row * p.ldr + col];
                    p.C[(size_t)row * p.ldc + col] = x;
                }
            }
    }
}

}  // namespace

hipError_t launch_gemm(const GemmParams &p, hipStream_t stream) {
    if (p.M <= 0 || p.N <= 0) return hipSuccess;
    if (p.K <= 0 || p.lda < p.K || p.ldw < p.K) return hipErrorInvalidValue;
    if (p.silu_pair && (p.N % 64) != 0) return hipErrorInvalidValue;
    // Buffer descriptors address at most 2^31 bytes per 128-row panel.
    if ((size_t)kBM * p.lda * 4 >= (1u << 31) || (size_t)kBN * p.ldw * 4 >= (1u << 31)) return hipErrorInvalidValue;
    const int tiles_m = (p.M + kBM - 1) / kBM, tiles_n = (p.N + kBN - 1) / kBN;
    const int total = tiles_m * tiles_n;
    const int per_xcd = (total + kXcds - 1) / kXcds;
    hipLaunchKernelGGL(gemm_f32_kernel, dim3(per_xcd * kXcds), dim3(kThreads), 0, stream, p, tiles_m, tiles_n,
                       per_xcd);
    return hipGetLastError();
}

}  // namespace yuf

extern "C" int yuf_linear_f32(int M, int N, int K, const float *A, const float *W, const float *bias, int act,
                              const float *residual, float *C, void *stream) {
    using namespace yuf;
    if (M < 0 || N < 0 || K < 1) return fail(YUF_ERR_INVALID, "linear: bad sizes");
    if (act < ACT_NONE || act > ACT_SIGMOID) return fail(YUF_ERR_INVALID, "linear: bad activation");
    if (M > 0 && N > 0 && (!A || !W || !C)) return fail(YUF_ERR_INVALID, "linear: null pointer");
    GemmParams p;
    p.M = M; p.N = N; p.K = K; p.A = A; p.lda = K; p.W = W; p.ldw = K; p.C = C; p.ldc = N;
    p.bias = bias; p.act = act; p.residual = residual; p.ldr = N;
    hipError_t err = launch_gemm(p, static_cast<hipStream_t>(stream));
    if (err != hipSuccess) return fail(YUF_ERR_HIP, std::string("linear launch: ") + hipGetErrorString(err));
    return YUF_OK;
}
