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
//
// bf16 weights (GemmParams::Wh, the C5 configuration's weight type): the
// large-tile and decode kernels take a WB flag.  W streams as bf16 and A stays
// fp32 in memory.  As A enters the matrix core it is split into two bf16
// parts, hi = bf16(a) and lo = bf16(a - hi) (round to nearest even, the gfx950
// v_cvt_pk_bf16_f32), and each k-step runs two v_mfma_f32_16x16x32_bf16,
// hi x W then lo x W (lane l: A[m = l % 16][k = 8 (l / 16) + j],
// B[k = 8 (l / 16) + j][n = l % 16], j < 8; accumulator layout as for
// v_mfma_f32_16x16x4f32), so the epilogues are shared.  A product of two bf16
// values is exact in fp32 and |a - hi - lo| <= 2^-16 |a|, so the result is the
// fp32 product A x bf16(W) up to fp32 accumulation order: the activations keep
// fp32 precision (a single bf16 rounding of A moves C5 logits by up to ~0.2
// over 24 layers, against the configuration's 2e-2).  Needs K % 8 == 0.
#include <algorithm>
#include <cstdlib>
#include <cstring>
#include <type_traits>

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

struct GemmGroup {
    GemmParams p[kMaxGroup];
    int tiles_n[kMaxGroup];
    int total[kMaxGroup];
};

// blockIdx.y selects the product of a group; blockIdx.x its output tile.
__global__ void __launch_bounds__(kThreads) gemm_f32_kernel(GemmGroup g, int per_xcd) {
    __shared__ __attribute__((aligned(16))) float As[2][kBM * kLd];
    __shared__ __attribute__((aligned(16))) float Bs[2][kBN * kLd];

    const GemmParams &p = g.p[blockIdx.y];
    const int tiles_n = g.tiles_n[blockIdx.y];
    const int flat = (blockIdx.x % kXcds) * per_xcd + blockIdx.x / kXcds;
    if (flat >= g.total[blockIdx.y]) return;
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
    lds_barrier();

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
        lds_barrier();
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

// ---------------------------------------------------------------------------
// Large-tile path for the prefill shapes (M a multiple of 256 in practice):
// 512 threads = 8 waves in a 4 x 2 arrangement over a 256 x BN block tile
// (BN = 256 for N % 256 == 0, BN = 160 for the d_model = 640 outputs, 128 and
// 64 for the narrow ROSA input and low-rank products), K tile
// 16, double-buffered LDS, one workgroup per CU.  The tile sizes make the tile
// count a multiple of the 256 CUs for every prefill product of the 0.1B model
// (N = 640: 64 x 4 tiles; N = 5120: 64 x 20; N = 20480: 64 x 80), so no CU
// idles through a partial last wave of tiles.  Each wave owns 64 x BN/2 as
// 16 x 16 tiles of v_mfma_f32_16x16x4f32; for 4 consecutive k-steps a lane
// reads its 4 k values of a row with one ds_read_b128 (k-step r uses k = 4 g + r
// for lane group g on both operands).
// ---------------------------------------------------------------------------
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

// Eight fp32 values (k order) rounded to bf16 for one MFMA operand.
__device__ __forceinline__ bf16x8 to_bf16x8(floatx4 lo, floatx4 hi) {
    bf16x8 r;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        r[q] = (__bf16)lo[q];
        r[4 + q] = (__bf16)hi[q];
    }
    return r;
}

// The three bf16 parts of eight fp32 values: p1 = bf16(x), p2 = bf16(x - p1),
// p3 = bf16(x - p1 - p2) (both differences exact in fp32); |x - p1 - p2 - p3|
// <= 2^-24 |x| up to fp32 underflow.  Two values at a time: one packed
// v_cvt_pk_bf16_f32 per part, shifts / masks back to fp32.
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float floatx2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ void split3_pair(floatx2 x, bf16x2 &p1, bf16x2 &p2, bf16x2 &p3) {
    p1 = __builtin_convertvector(x, bf16x2);
    const floatx2 r1 = x - __builtin_convertvector(p1, floatx2);
    p2 = __builtin_convertvector(r1, bf16x2);
    const floatx2 r2 = r1 - __builtin_convertvector(p2, floatx2);
    p3 = __builtin_convertvector(r2, bf16x2);
}

// The two bf16 parts of eight fp32 values: hi = bf16(x), lo = bf16(x - hi).
__device__ __forceinline__ void split_bf16x8(floatx4 x0, floatx4 x1, bf16x8 &hi, bf16x8 &lo) {
    hi = to_bf16x8(x0, x1);
    floatx4 r0, r1;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        r0[q] = x0[q] - (float)hi[q];
        r1[q] = x1[q] - (float)hi[4 + q];
    }
    lo = to_bf16x8(r0, r1);
}
constexpr int kBigBM = 256, kBigThreads = 512;
// K tile: 32 where the accumulators leave room for the larger load set, else 16.
template <int BN> constexpr int big_bk() { return BN >= 256 ? 16 : 32; }

template <int ROWS, int BK>
struct BigLoad {
    static constexpr int kF4 = ROWS * (BK / 4);                        // float4 per tile
    static constexpr int kPer = (kF4 + kBigThreads - 1) / kBigThreads;  // per thread
    float4 v[kPer];
};

template <int ROWS, int BK>
__device__ __forceinline__ void big_load(BigLoad<ROWS, BK> &t, __amdgpu_buffer_rsrc_t rsrc, int ld, int k0, int K,
                                         int tid) {
#pragma unroll
    for (int i = 0; i < BigLoad<ROWS, BK>::kPer; ++i) {
        const int q = tid + i * kBigThreads;
        const int row = q / (BK / 4), k = k0 + (q % (BK / 4)) * 4;
        // K % 4 == 0 on this path: a float4 is wholly inside or outside [0, K).
        const uint32_t off = (q < BigLoad<ROWS, BK>::kF4 && k < K) ? (uint32_t)((size_t)row * ld + k) * 4u : kBufferOob;
        t.v[i] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(rsrc, off, 0, 0));
    }
}

template <int ROWS, int BK>
__device__ __forceinline__ void big_store(const BigLoad<ROWS, BK> &t, float *lds, int tid) {
    constexpr int LD = BK + 4;
#pragma unroll
    for (int i = 0; i < BigLoad<ROWS, BK>::kPer; ++i) {
        const int q = tid + i * kBigThreads;
        if (q < BigLoad<ROWS, BK>::kF4) *reinterpret_cast<float4 *>(lds + (q / (BK / 4)) * LD + (q % (BK / 4)) * 4) = t.v[i];
    }
}

// bf16 tiles of the WB and X3 paths: rows of 32 k (64 bytes) padded to
// kLdh = 48 elements (96 bytes) in LDS (measured ~2 % faster on every
// prefill product than 80-byte rows).
constexpr int kLdh = 48;

template <int ROWS>
struct BigLoadH {
    static constexpr int kChunks = ROWS * 4;                               // 16-byte runs per tile
    static constexpr int kPer = (kChunks + kBigThreads - 1) / kBigThreads;  // per thread
    floatx4 v[kPer];                                                        // raw bf16 bits
};

template <int ROWS>
__device__ __forceinline__ void big_load_h(BigLoadH<ROWS> &t, __amdgpu_buffer_rsrc_t rsrc, int ld, int k0, int K,
                                           int tid) {
#pragma unroll
    for (int i = 0; i < BigLoadH<ROWS>::kPer; ++i) {
        const int q = tid + i * kBigThreads;
        const int row = q / 4, k = k0 + (q % 4) * 8;
        // K % 8 == 0 on this path: a run of 8 is wholly inside or outside [0, K).
        const uint32_t off = (q < BigLoadH<ROWS>::kChunks && k < K) ? (uint32_t)((size_t)row * ld + k) * 2u : kBufferOob;
        t.v[i] = __builtin_bit_cast(floatx4, __builtin_amdgcn_raw_buffer_load_b128(rsrc, off, 0, 0));
    }
}

template <int ROWS>
__device__ __forceinline__ void big_store_h(const BigLoadH<ROWS> &t, __bf16 *lds, int tid) {
#pragma unroll
    for (int i = 0; i < BigLoadH<ROWS>::kPer; ++i) {
        const int q = tid + i * kBigThreads;
        if (q < BigLoadH<ROWS>::kChunks) *reinterpret_cast<floatx4 *>(lds + (q / 4) * kLdh + (q % 4) * 8) = t.v[i];
    }
}

// fp32 A tile (32 k) split into its bf16 parts on the way into LDS: hi into
// `hi`, lo = bf16(a - hi) into `lo` (same layout).
template <int ROWS>
__device__ __forceinline__ void big_store_a_h(const BigLoad<ROWS, 32> &t, __bf16 *hi, __bf16 *lo, int tid) {
    typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
#pragma unroll
    for (int i = 0; i < BigLoad<ROWS, 32>::kPer; ++i) {
        const int q = tid + i * kBigThreads;
        if (q < BigLoad<ROWS, 32>::kF4) {
            const float4 x = t.v[i];
            const bf16x4 h = {(__bf16)x.x, (__bf16)x.y, (__bf16)x.z, (__bf16)x.w};
            const bf16x4 l = {(__bf16)(x.x - (float)h[0]), (__bf16)(x.y - (float)h[1]), (__bf16)(x.z - (float)h[2]),
                              (__bf16)(x.w - (float)h[3])};
            const int o = (q / 8) * kLdh + (q % 8) * 4;
            *reinterpret_cast<bf16x4 *>(hi + o) = h;
            *reinterpret_cast<bf16x4 *>(lo + o) = l;
        }
    }
}

// Epilogue of the large-tile path through LDS: 16 accumulator rows of a wave at
// a time are written to LDS and read back row-contiguous, so every global
// access (C, residual, bias) is a 16-byte run along a row.  Needs 16-byte
// aligned C / residual / bias and row strides that are multiples of 4 floats.
template <int WN>
__device__ __forceinline__ float4 stage_read(const float *stage, int row, int c4) {
    return *reinterpret_cast<const float4 *>(stage + row * (WN + 4) + 4 * c4);
}

// Epilogue of the large-tile kernels: waves 4 x 2 over a 64 MI x BN tile, wave
// (wm, wn) owns rows m0 + 16 MI wm + [0, 16 MI) and columns n0 + (BN / 2) wn +
// [0, BN / 2), accumulator acc[i][j] the 16 x 16 block (i, j) of it (MI = 4:
// 256-row tiles; MI = 1: 64-row tiles).  `lds` is free when it is called
// (STAGED: wave-private staging areas of 16 x (BN / 2 + 4) floats).
template <int BN, bool STAGED, int MI = 4>
__device__ __forceinline__ void big_epilogue(const GemmParams &p, floatx4 (&acc)[MI][BN / 32], float *lds, int m0,
                                             int n0, int wave, int lane) {
    constexpr int WN = BN / 2, NT = WN / 16;
    const int wm = wave >> 1, wn = wave & 1;
    const int g4 = lane >> 4, li = lane & 15;
    // Accumulator register r of lane l: row 4 (l / 16) + r, column l % 16 of its 16 x 16 tile.
    // The parameters are read once, ahead of the LDS fences below (after a
    // fence the compiler would load each kernel-argument field again).
    const int M = p.M, ldc = p.ldc, ldr = p.ldr, act = p.act;
    float *const C = p.C;
    const float *const bias_p = p.bias, *const res_p = p.residual;
    if constexpr (STAGED) {
        // The K loop ended with a barrier: LDS is free.  Wave-private staging areas.
        constexpr int SW = WN + 4;
        float *stage = lds + wave * 16 * SW;
        const int row0 = m0 + wm * 16 * MI;
        if (p.silu_pair) {
            if constexpr (BN % 128 == 0) {
                constexpr int HW = WN / 2;  // output columns of the wave
                const int hcol0 = (n0 + wn * WN) / 2;
#pragma unroll
                for (int i = 0; i < MI; ++i) {
#pragma unroll
                    for (int b = 0; b < WN / 64; ++b)
#pragma unroll
                        for (int h = 0; h < 2; ++h)
#pragma unroll
                            for (int r = 0; r < 4; ++r) {
                                const float x = acc[i][4 * b + h][r], gt = acc[i][4 * b + 2 + h][r];
                                stage[(4 * g4 + r) * SW + 32 * b + 16 * h + li] = x / (1.0f + expf(-x)) * gt;
                            }
                    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
                    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
#pragma unroll
                    for (int t = 0; t < 16 * HW / 4 / 64; ++t) {
                        const int q = lane + 64 * t, row = q / (HW / 4), c4 = q % (HW / 4);
                        const int grow = row0 + i * 16 + row;
                        if (grow < M)
                            *reinterpret_cast<float4 *>(C + (size_t)grow * ldc + hcol0 + 4 * c4) =
                                stage_read<WN>(stage, row, c4);
                    }
                    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
                    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
                }
            }
            return;
        }
        const int col0 = n0 + wn * WN;
        // One copy of the row loop per activation (a uniform branch outside it).
        auto rows = [&](auto act_c) {
            constexpr int ACT = decltype(act_c)::value;
#pragma unroll
            for (int i = 0; i < MI; ++i) {
#pragma unroll
                for (int j = 0; j < NT; ++j)
#pragma unroll
                    for (int r = 0; r < 4; ++r) stage[(4 * g4 + r) * SW + 16 * j + li] = acc[i][j][r];
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
#pragma unroll
                for (int t = 0; t < 16 * WN / 4 / 64; ++t) {
                    const int q = lane + 64 * t, row = q / (WN / 4), c4 = q % (WN / 4);
                    const int grow = row0 + i * 16 + row, col = col0 + 4 * c4;
                    if (grow < M) {
                        float4 x = stage_read<WN>(stage, row, c4);
                        if (bias_p) {
                            const float4 b4 = *reinterpret_cast<const float4 *>(bias_p + col);
                            x.x += b4.x; x.y += b4.y; x.z += b4.z; x.w += b4.w;
                        }
                        x.x = apply_act(x.x, ACT); x.y = apply_act(x.y, ACT);
                        x.z = apply_act(x.z, ACT); x.w = apply_act(x.w, ACT);
                        if (res_p) {
                            const float4 r4 = *reinterpret_cast<const float4 *>(res_p + (size_t)grow * ldr + col);
                            x.x += r4.x; x.y += r4.y; x.z += r4.z; x.w += r4.w;
                        }
                        *reinterpret_cast<float4 *>(C + (size_t)grow * ldc + col) = x;
                    }
                }
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
            }
        };
        if (act == ACT_TANH) rows(std::integral_constant<int, ACT_TANH>{});
        else if (act == ACT_SIGMOID) rows(std::integral_constant<int, ACT_SIGMOID>{});
        else rows(std::integral_constant<int, ACT_NONE>{});
        return;
    }
    if constexpr (BN % 128 == 0) {
        if (p.silu_pair) {
            // Each wave's columns are whole 64-row blocks [32 "in" | 32 "gate"].
#pragma unroll
            for (int b = 0; b < WN / 64; ++b)
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const int hcol = (n0 + wn * WN + 64 * b) / 2 + 16 * h + li;
                    if (hcol >= p.N / 2) continue;
#pragma unroll
                    for (int i = 0; i < MI; ++i)
#pragma unroll
                        for (int r = 0; r < 4; ++r) {
                            const int row = m0 + wm * 16 * MI + i * 16 + 4 * g4 + r;
                            if (row < p.M) {
                                const float x = acc[i][4 * b + h][r], gt = acc[i][4 * b + 2 + h][r];
                                p.C[(size_t)row * p.ldc + hcol] = x / (1.0f + expf(-x)) * gt;
                            }
                        }
                }
            return;
        }
    }
#pragma unroll
    for (int j = 0; j < NT; ++j) {
        const int col = n0 + wn * WN + j * 16 + li;
        if (col >= p.N) continue;
        const float bias = p.bias ? p.bias[col] : 0.0f;
#pragma unroll
        for (int i = 0; i < MI; ++i)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int row = m0 + wm * 16 * MI + i * 16 + 4 * g4 + r;
                if (row < p.M) {
                    float x = apply_act(acc[i][j][r] + bias, p.act);
                    if (p.residual) x += p.residual[(size_t)row * p.ldr + col];
                    p.C[(size_t)row * p.ldc + col] = x;
                }
            }
    }
}

// X3 (fp32 A and W, K % 32 == 0): each staged fp32 value is split once, when
// its tile is written to LDS, into three bf16 parts (split3_pair), kept as
// three bf16 planes of A and of W in one LDS buffer (two barriers per K tile);
// every 16 x 16 x 32 block then takes six v_mfma_f32_16x16x32_bf16 -- a3 w1,
// a1 w3, a2 w2, a2 w1, a1 w2, a1 w1 (the terms below 2^-24 relative, a2 w3,
// a3 w2 and a3 w3, are dropped) -- so the result is the fp32 product up to
// about 3 * 2^-24 relative per term and fp32 accumulation order.  On gfx950
// the bf16 matrix cores run a 32-k block in about 17 cycles against 256 for
// eight 16 x 16 x 4 fp32 MFMAs.
template <int BN, bool STAGED, bool WB, bool X3 = false>
__global__ void __launch_bounds__(kBigThreads) gemm_big_kernel(GemmGroup g, int per_xcd) {
    static_assert(!(WB && X3), "X3 takes fp32 weights");
    constexpr int WN = BN / 2, NT = WN / 16;
    constexpr int kBigBK = (WB || X3) ? 32 : big_bk<BN>(), kBigLd = kBigBK + 4;
    // X3: one buffer of three bf16 planes each for A and W ([plane][row][kLdh]).
    constexpr int kLdsFloats = WB   ? (2 * (2 * kBigBM + BN) * kLdh) / 2
                               : X3 ? (3 * (kBigBM + BN) * kLdh) / 2
                                    : 2 * (kBigBM + BN) * kBigLd;
    static_assert(kLdsFloats >= kBigThreads / 64 * 16 * (WN + 4), "LDS too small for the staged epilogue");
    __shared__ __attribute__((aligned(16))) float lds[kLdsFloats];
    float(*As)[kBigBM * kBigLd] = reinterpret_cast<float(*)[kBigBM * kBigLd]>(lds);
    float(*Bs)[BN * kBigLd] = reinterpret_cast<float(*)[BN * kBigLd]>(lds + 2 * kBigBM * kBigLd);
    __bf16 *Ah = reinterpret_cast<__bf16 *>(lds);  // WB: A hi [2][kBigBM * kLdh], A lo [2][kBigBM * kLdh],
    __bf16 *Al = Ah + 2 * kBigBM * kLdh;            // then W [2][BN * kLdh]
    __bf16 *Bh = Al + 2 * kBigBM * kLdh;
    __bf16 *Ap = reinterpret_cast<__bf16 *>(lds);  // X3: A planes [3][kBigBM * kLdh], then W planes [3][BN * kLdh]
    __bf16 *Wp = Ap + 3 * kBigBM * kLdh;

    const GemmParams &p = g.p[blockIdx.y];
    const int tiles_n = g.tiles_n[blockIdx.y];
    const int flat = (blockIdx.x % kXcds) * per_xcd + blockIdx.x / kXcds;
    if (flat >= g.total[blockIdx.y]) return;
    const int bm = flat / tiles_n, bn = flat - bm * tiles_n;
    const int m0 = bm * kBigBM, n0 = bn * BN;

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int wm = wave >> 1, wn = wave & 1;
    const int g4 = lane >> 4, li = lane & 15;
    const int rows_a = min(kBigBM, p.M - m0), rows_w = min(BN, p.N - n0);
    const auto ra = make_rsrc(p.A + (size_t)m0 * p.lda, (uint32_t)(((size_t)(rows_a - 1) * p.lda + p.K) * 4));
    const auto rw = WB ? make_rsrc(p.Wh + (size_t)n0 * p.ldw, (uint32_t)(((size_t)(rows_w - 1) * p.ldw + p.K) * 2))
                       : make_rsrc(p.W + (size_t)n0 * p.ldw, (uint32_t)(((size_t)(rows_w - 1) * p.ldw + p.K) * 4));

    floatx4 acc[4][NT];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < NT; ++j) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};

    const int k_tiles = (p.K + kBigBK - 1) / kBigBK;
    BigLoad<kBigBM, kBigBK> ta;
    std::conditional_t<WB, BigLoadH<BN>, BigLoad<BN, kBigBK>> tb;
    auto load_w = [&](int k0) {
        if constexpr (WB) big_load_h(tb, rw, p.ldw, k0, p.K, tid);
        else big_load(tb, rw, p.ldw, k0, p.K, tid);
    };
    // X3: split each staged float4 into its three bf16 parts (one ds_write_b64 per plane).
    auto store_planes = [&](const auto &t, __bf16 *dst, int plane_elems) {
        using T = std::decay_t<decltype(t)>;
#pragma unroll
        for (int i = 0; i < T::kPer; ++i) {
            const int q = tid + i * kBigThreads;
            if (q < T::kF4) {
                bf16x2 a0, b0, c0, a1, b1, c1;
                split3_pair(floatx2{t.v[i].x, t.v[i].y}, a0, b0, c0);
                split3_pair(floatx2{t.v[i].z, t.v[i].w}, a1, b1, c1);
                __bf16 *o = dst + (q / 8) * kLdh + (q % 8) * 4;
                typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
                *reinterpret_cast<bf16x4 *>(o) = __builtin_shufflevector(a0, a1, 0, 1, 2, 3);
                *reinterpret_cast<bf16x4 *>(o + plane_elems) = __builtin_shufflevector(b0, b1, 0, 1, 2, 3);
                *reinterpret_cast<bf16x4 *>(o + 2 * plane_elems) = __builtin_shufflevector(c0, c1, 0, 1, 2, 3);
            }
        }
    };
    auto store_tiles = [&](int buf) {
        if constexpr (X3) {
            store_planes(ta, Ap, kBigBM * kLdh);
            store_planes(tb, Wp, BN * kLdh);
        } else if constexpr (WB) {
            big_store_a_h(ta, Ah + buf * kBigBM * kLdh, Al + buf * kBigBM * kLdh, tid);
            big_store_h(tb, Bh + buf * BN * kLdh, tid);
        } else {
            big_store(ta, As[buf], tid);
            big_store(tb, Bs[buf], tid);
        }
    };
    big_load(ta, ra, p.lda, 0, p.K, tid);
    load_w(0);
    store_tiles(0);
    lds_barrier();

    for (int kt = 0; kt < k_tiles; ++kt) {
        const int cur = X3 ? 0 : kt & 1;
        const bool more = kt + 1 < k_tiles;
        if (more) {
            big_load(ta, ra, p.lda, (kt + 1) * kBigBK, p.K, tid);
            load_w((kt + 1) * kBigBK);
        }
        if constexpr (WB) {
            // One 32-k step: a lane's 8 k of a row are one ds_read_b128 per part.
            const __bf16 *Ac = Ah + cur * kBigBM * kLdh, *Alc = Al + cur * kBigBM * kLdh, *Bc = Bh + cur * BN * kLdh;
            bf16x8 af[4], al[4], bf[NT];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                af[i] = *reinterpret_cast<const bf16x8 *>(Ac + (wm * 64 + i * 16 + li) * kLdh + 8 * g4);
                al[i] = *reinterpret_cast<const bf16x8 *>(Alc + (wm * 64 + i * 16 + li) * kLdh + 8 * g4);
            }
#pragma unroll
            for (int j = 0; j < NT; ++j) bf[j] = *reinterpret_cast<const bf16x8 *>(Bc + (wn * WN + j * 16 + li) * kLdh + 8 * g4);
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < NT; ++j) {
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[i], bf[j], acc[i][j], 0, 0, 0);
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al[i], bf[j], acc[i][j], 0, 0, 0);
                }
        }
        if constexpr (X3) {
            // One 32-k step from the split planes: a lane's 8 consecutive k of a
            // row are one ds_read_b128 per plane.
            constexpr int PA = kBigBM * kLdh, PW = BN * kLdh;
            bf16x8 a1[4], a2[4], a3[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const __bf16 *ap = Ap + (wm * 64 + i * 16 + li) * kLdh + 8 * g4;
                a1[i] = *reinterpret_cast<const bf16x8 *>(ap);
                a2[i] = *reinterpret_cast<const bf16x8 *>(ap + PA);
                a3[i] = *reinterpret_cast<const bf16x8 *>(ap + 2 * PA);
            }
            // W fragments one ahead of their MFMAs, so the LDS latency of
            // fragment j + 1 overlaps the products of fragment j.
            const __bf16 *bp0 = Wp + (wn * WN + li) * kLdh + 8 * g4;
            bf16x8 nw1 = *reinterpret_cast<const bf16x8 *>(bp0);
            bf16x8 nw2 = *reinterpret_cast<const bf16x8 *>(bp0 + PW);
            bf16x8 nw3 = *reinterpret_cast<const bf16x8 *>(bp0 + 2 * PW);
            __builtin_amdgcn_sched_group_barrier(0x100, 15, 0);  // A fragments and W fragment 0 first
#pragma unroll
            for (int j = 0; j < NT; ++j) {
                const bf16x8 w1 = nw1, w2 = nw2, w3 = nw3;
                if (j + 1 < NT) {
                    const __bf16 *bp = bp0 + (j + 1) * 16 * kLdh;
                    nw1 = *reinterpret_cast<const bf16x8 *>(bp);
                    nw2 = *reinterpret_cast<const bf16x8 *>(bp + PW);
                    nw3 = *reinterpret_cast<const bf16x8 *>(bp + 2 * PW);
                }
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    floatx4 c = acc[i][j];
                    c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a3[i], w1, c, 0, 0, 0);
                    c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1[i], w3, c, 0, 0, 0);
                    c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a2[i], w2, c, 0, 0, 0);
                    c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a2[i], w1, c, 0, 0, 0);
                    c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1[i], w2, c, 0, 0, 0);
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1[i], w1, c, 0, 0, 0);
                }
                // Keep the next fragment's reads ahead of this fragment's products.
                if (j + 1 < NT) __builtin_amdgcn_sched_group_barrier(0x100, 3, 0);  // DS reads
                __builtin_amdgcn_sched_group_barrier(0x008, 24, 0);                 // MFMA
            }
        }
#pragma unroll
        for (int h = 0; h < ((WB || X3) ? 0 : kBigBK / 16); ++h) {  // 16 k per half: one ds_read_b128 per operand fragment
            floatx4 af[4], bf[NT];
#pragma unroll
            for (int i = 0; i < 4; ++i)
                af[i] = *reinterpret_cast<const floatx4 *>(As[cur] + (wm * 64 + i * 16 + li) * kBigLd + 16 * h + 4 * g4);
#pragma unroll
            for (int j = 0; j < NT; ++j)
                bf[j] = *reinterpret_cast<const floatx4 *>(Bs[cur] + (wn * WN + j * 16 + li) * kBigLd + 16 * h + 4 * g4);
#pragma unroll
            for (int r = 0; r < 4; ++r)
#pragma unroll
                for (int i = 0; i < 4; ++i)
#pragma unroll
                    for (int j = 0; j < NT; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(af[i][r], bf[j][r], acc[i][j], 0, 0, 0);
        }
        if constexpr (X3) {
            // One buffer: every wave is done with this tile before it is replaced.
            if (more) {
                lds_barrier();
                store_tiles(0);
            }
        } else if (more) {
            store_tiles(cur ^ 1);
        }
        lds_barrier();
    }

    big_epilogue<BN, STAGED>(p, acc, lds, m0, n0, wave, lane);
}

// ---------------------------------------------------------------------------
// X3 with pre-split weight planes (GemmParams::Wp).  The engine splits every
// fp32 projection matrix once, at creation, into the three bf16 parts the X3
// form uses (split3_pair), stored as "planes": for each 16-row block rb and
// 32-k tile kt, three 1-KB blocks (part 1, 2, 3) of 16 rows x 32 bf16, at
// element ((rb * (K / 32) + kt) * 3 + part) * 512; inside a block, row r's
// 16-byte chunk c (k 8c .. 8c + 7) sits at r * 32 + 8 (c ^ x3p_swz(r)), which
// spreads the 16 rows a fragment read touches over all LDS banks.
//
// The kernel then never writes LDS from registers: each k tile arrives by
// direct buffer -> LDS loads (64 lanes x 16 bytes per instruction) into one of
// two buffers while the MFMAs run on the other -- A as fp32 in 8-row x 32-k
// blocks (chunk c of row R at c ^ (R & 7) ^ ((R >> 3) & 1), conflict-free for
// the fragment reads), W as its plane blocks -- with one barrier per k tile.
// Each wave splits its own 16 MI A rows into parts (two waves share rows: the
// split is done twice), W's parts come ready from LDS.  Tile 64 MI x BN,
// waves 4 x 2 as in gemm_big_kernel (MI = 4: 256 rows; MI = 1: 64 rows for the
// memory-bound shapes); the per-32-k product order and the split are the X3
// form's, so the results are bit-identical to it.  LDS: two buffers of 8 MI
// KB (A) + 6 BN / 16 KB (W planes): 160 KB at BN = 256, MI = 4.
__host__ __device__ constexpr int x3p_swz(int r) { return ((r >> 1) ^ (r >> 3)) & 3; }

__device__ __forceinline__ void split3_x8(floatx4 x0, floatx4 x1, bf16x8 &p1, bf16x8 &p2, bf16x8 &p3) {
    bf16x2 a[4], b[4], c[4];
    split3_pair(floatx2{x0[0], x0[1]}, a[0], b[0], c[0]);
    split3_pair(floatx2{x0[2], x0[3]}, a[1], b[1], c[1]);
    split3_pair(floatx2{x1[0], x1[1]}, a[2], b[2], c[2]);
    split3_pair(floatx2{x1[2], x1[3]}, a[3], b[3], c[3]);
#pragma unroll
    for (int h = 0; h < 4; ++h) {
        p1[2 * h] = a[h][0]; p1[2 * h + 1] = a[h][1];
        p2[2 * h] = b[h][0]; p2[2 * h + 1] = b[h][1];
        p3[2 * h] = c[h][0]; p3[2 * h + 1] = c[h][1];
    }
}

typedef __attribute__((address_space(3))) void lds_void_t;
constexpr uint32_t kWaitVm0 = 0x0F70;  // s_waitcnt vmcnt(0) (expcnt / lgkmcnt left free)

template <int BN, bool STAGED, int MI = 4>
__global__ void __launch_bounds__(kBigThreads) gemm_x3p_kernel(GemmGroup g, int per_xcd) {
    constexpr int WN = BN / 2, NT = WN / 16;
    constexpr int BM = 64 * MI;          // MI 16-row sub-tiles per wave, waves 4 x 2
    constexpr int AB = BM / 8;           // fp32 A blocks per k tile (8 rows x 32 k = 1 KB)
    constexpr int WB = BN / 16 * 3;      // W plane blocks per k tile
    constexpr int NB = AB + WB;          // 1-KB blocks per buffer
    constexpr int PER = (NB + 7) / 8;    // direct loads per wave and k tile
    constexpr int GM = 8;                // row tiles walked together (L2 reuse of W inside an XCD)
    static_assert(2 * NB * 1024 <= 160 * 1024, "two k-tile buffers must fit in LDS");
    static_assert(2 * NB * 256 >= 8 * 16 * (WN + 4), "LDS too small for the staged epilogue");
    __shared__ __attribute__((aligned(1024))) float lds[2 * NB * 256];

    const GemmParams &p = g.p[blockIdx.y];
    const int tiles_n = g.tiles_n[blockIdx.y], total = g.total[blockIdx.y];
    const int flat = (blockIdx.x % kXcds) * per_xcd + blockIdx.x / kXcds;
    if (flat >= total) return;
    const int tiles_m = total / tiles_n;
    const int grp = flat / (GM * tiles_n), rem = flat - grp * GM * tiles_n;
    const int gm = min(GM, tiles_m - grp * GM);
    const int bm = grp * GM + rem % gm, bn = rem / gm;
    const int m0 = bm * BM, n0 = bn * BN;

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: the LDS destination goes in M0
    const int wm = wave >> 1, wn = wave & 1;
    const int g4 = lane >> 4, li = lane & 15;
    // Kernel-argument fields read once: the loop's direct LDS loads count as
    // memory writes to the compiler, which would otherwise reload them (a
    // scalar-memory wait) before every k tile's loads.
    const int lda = __builtin_amdgcn_readfirstlane(p.lda), K = __builtin_amdgcn_readfirstlane(p.K);
    const int KT = K / 32;
    const int rows_a = min(BM, p.M - m0);
    const auto ra = make_rsrc(p.A + (size_t)m0 * lda, (uint32_t)(((size_t)(rows_a - 1) * lda + K) * 4));
    const auto rw = make_rsrc(p.Wp, (uint32_t)((size_t)(p.N / 16) * KT * 3 * 1024));
    const int ar = lane >> 3, apos = lane & 7;  // lane's row / LDS chunk inside an 8-row A block

    auto issue = [&](int kt, int buf) {
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const int b = wave + 8 * i;
            if (b >= NB) break;
            lds_void_t *dst = (lds_void_t *)(lds + (buf * NB + b) * 256);
            if (b < AB) {
                const int c = apos ^ ar ^ (b & 1);
                const uint32_t off = (uint32_t)(((b * 8 + ar) * lda + kt * 32 + 4 * c) * 4);
                __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, dst, 16, off, 0, 0, 0);
            } else {
                const int bb = b - AB, rb = bn * (BN / 16) + bb / 3, part = bb % 3;
                const uint32_t blk = (uint32_t)(((rb * KT + kt) * 3 + part) * 1024);
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rw, dst, 16, (uint32_t)lane * 16u, blk, 0, 0);
            }
        }
    };

    floatx4 acc[MI][NT];
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int j = 0; j < NT; ++j) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};
    // Fragment offsets: A rows wm 16 MI + 16 i + li (float index), W rows wn WN + 16 j + li (bf16 index).
    const int fa = (li & 7) ^ (li >> 3);
    const int offa0 = (wm * 2 * MI + (li >> 3)) * 256 + (li & 7) * 32 + (((2 * g4) ^ fa) * 4);
    const int offa1 = (wm * 2 * MI + (li >> 3)) * 256 + (li & 7) * 32 + (((2 * g4 + 1) ^ fa) * 4);
    const int offw = (AB + wn * NT * 3) * 512 + li * 32 + ((g4 ^ x3p_swz(li)) * 8);

    issue(0, 0);
    __builtin_amdgcn_s_waitcnt(kWaitVm0);
    lds_barrier();
    for (int kt = 0; kt < KT; ++kt) {
        const int cur = kt & 1;
        if (kt + 1 < KT) issue(kt + 1, cur ^ 1);
        const float *base = lds + cur * NB * 256;
        const __bf16 *bh = reinterpret_cast<const __bf16 *>(base);
        bf16x8 a1[MI], a2[MI], a3[MI];
#pragma unroll
        for (int i = 0; i < MI; ++i) {
            const floatx4 x0 = *reinterpret_cast<const floatx4 *>(base + offa0 + i * 512);
            const floatx4 x1 = *reinterpret_cast<const floatx4 *>(base + offa1 + i * 512);
            split3_x8(x0, x1, a1[i], a2[i], a3[i]);
        }
        bf16x8 nw1 = *reinterpret_cast<const bf16x8 *>(bh + offw);
        bf16x8 nw2 = *reinterpret_cast<const bf16x8 *>(bh + offw + 512);
        bf16x8 nw3 = *reinterpret_cast<const bf16x8 *>(bh + offw + 1024);
#pragma unroll
        for (int j = 0; j < NT; ++j) {
            const bf16x8 w1 = nw1, w2 = nw2, w3 = nw3;
            if (j + 1 < NT) {
                const __bf16 *bp = bh + offw + (j + 1) * 1536;
                nw1 = *reinterpret_cast<const bf16x8 *>(bp);
                nw2 = *reinterpret_cast<const bf16x8 *>(bp + 512);
                nw3 = *reinterpret_cast<const bf16x8 *>(bp + 1024);
            }
#pragma unroll
            for (int i = 0; i < MI; ++i) {
                floatx4 c = acc[i][j];
                c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a3[i], w1, c, 0, 0, 0);
                c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1[i], w3, c, 0, 0, 0);
                c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a2[i], w2, c, 0, 0, 0);
                c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a2[i], w1, c, 0, 0, 0);
                c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1[i], w2, c, 0, 0, 0);
                acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1[i], w1, c, 0, 0, 0);
            }
        }
        // This wave's loads of the next tile have landed; after the barrier
        // every wave's have, and nobody reads this tile's buffer any more.
        __builtin_amdgcn_s_waitcnt(kWaitVm0);
        lds_barrier();
    }
    big_epilogue<BN, STAGED, MI>(p, acc, lds, m0, n0, wave, lane);
}

// fp32 W [N][ldw] -> X3 planes (layout above): one thread per 8 consecutive k of a row.
__global__ void x3_split_planes_kernel(const float *W, int ldw, int N, int K, uint16_t *planes) {
    const int chunks = K / 8;
    const long long q = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (q >= (long long)N * chunks) return;
    const int n = (int)(q / chunks), c8 = (int)(q % chunks);
    const float *src = W + (size_t)n * ldw + 8 * c8;
    const floatx4 x0 = *reinterpret_cast<const floatx4 *>(src), x1 = *reinterpret_cast<const floatx4 *>(src + 4);
    bf16x8 p1, p2, p3;
    split3_x8(x0, x1, p1, p2, p3);
    const int rb = n / 16, r = n % 16, kt = c8 / 4, c = c8 % 4;
    uint16_t *dst = planes + ((size_t)(rb * (K / 32) + kt) * 3) * 512 + r * 32 + ((c ^ x3p_swz(r)) * 8);
    *reinterpret_cast<bf16x8 *>(dst) = p1;
    *reinterpret_cast<bf16x8 *>(dst + 512) = p2;
    *reinterpret_cast<bf16x8 *>(dst + 1024) = p3;
}

// ---------------------------------------------------------------------------
// Decode path (M <= 64 rows, one token per stream).  The product is latency-
// bound, so the unit of work is small: one workgroup owns a 16-column slice of
// the output (two slices, in + gate, for the paired SiLU layout) for a tile of
// 16 * MI rows, and the 8 waves of the workgroup split K.  A 64-row,
// 640-column product is then 160 workgroups (MI = 1) instead of 40.  The row
// tiles of one slice are dealt to the same XCD, so its W rows come from HBM
// once and then hit that XCD's L2.  A wave issues the loads of up to S 16-k
// steps before its first MFMA (v_mfma_f32_16x16x4f32, A and W straight from
// global memory as 16-byte runs; rows past M and k past K read as zero through
// the buffer descriptors), so a wave's whole K range is in flight at once.
// The 8 partial tiles are summed in LDS in a fixed order and the epilogue is
// applied once: no workspace, no second kernel.  Up to kMaxDecode independent
// products with the same flags share one launch through a flat unit index.
//
// Optional A-side prologue (PRO): LayerNorm over the K columns of each A row
// (eps 1e-5; the same float expressions as layernorm_kernel, so the result
// equals LN-then-GEMM) and, for PRO = 2, an elementwise gate:
//   A' = (LN(A) * gamma + beta) [* gate],
// so the LN -> Linear pairs of a block run as one kernel
// (yufmusicgen/model.py:195-196 out_norm * g -> output, :306 ROSA norm,
// :377 FFN norm, :390-391 final norm -> LM head).
// ---------------------------------------------------------------------------
constexpr int kDecWaves = 8, kDecThreads = kDecWaves * 64;
constexpr int kMaxDecode = kMaxGroup;
constexpr int kDecLnPerLane = 16;  // LayerNorm prologue: K <= 1024
static_assert(64 * kDecLnPerLane <= 2 * kDecThreads, "gamma / beta: at most two columns per thread");

struct DecodeGroup {
    GemmParams p[kMaxDecode];
    int unit_end[kMaxDecode];  // running sum of units (slice x row tile) per product
    int mtiles[kMaxDecode];    // row tiles per product
    int count, units, per_xcd;
};

// Largest S (k steps in flight per wave) that keeps the prefetched operands
// within the register budget of a 512-thread workgroup.
// A WB step covers 32 k and holds 8 A floats per m-tile (4 for fp32 W).
constexpr int dec_cap(int NT, int MI, int PRO, bool WB = false) {
    const int c = MI == 1 ? (NT == 1 && PRO < 2 ? 10 : 6) : (NT == 1 ? (PRO == 0 ? 4 : 3) : 3);
    return WB ? (c >= 6 ? c - 4 : c - 1) : c;
}

// MULTI = false: a single product, whose parameters sit at fixed kernel-argument
// offsets (no dependent argument load to find the product of a unit).
template <int NT, int MI, int S, int PRO, bool MULTI, bool WB>
__global__ void __launch_bounds__(kDecThreads) gemm_decode_kernel(DecodeGroup g) {
    constexpr int RT = 16 * MI;  // rows per workgroup
    constexpr int KS = WB ? 32 : 16;  // k per step
    constexpr int RL = KS / 4;        // consecutive k per lane and step
    constexpr int AH = RL / 4;        // floatx4 per lane, m-tile and step
    __shared__ __attribute__((aligned(16))) float red[kDecWaves][NT][RT * 17];
    __shared__ float stats[PRO > 0 ? RT : 1][2];
    __shared__ float part[2][PRO > 0 ? kDecWaves : 1][PRO > 0 ? RT : 1];  // per-wave row partial sums
    __shared__ __attribute__((aligned(16))) float affine[PRO > 0 ? 2 * 64 * kDecLnPerLane : 4];  // gamma | beta

    const int u = (blockIdx.x % kXcds) * g.per_xcd + blockIdx.x / kXcds;
    if (u >= g.units) return;
    int pi = 0;
    if constexpr (MULTI) {
#pragma unroll
        for (int i = 1; i < kMaxDecode; ++i) pi += (i < g.count && u >= g.unit_end[i - 1]) ? 1 : 0;
    }
    const GemmParams &p = g.p[MULTI ? pi : 0];
    const int local = MULTI && pi > 0 ? u - g.unit_end[pi - 1] : u;
    const int mtiles = g.mtiles[MULTI ? pi : 0];
    const int slice = local / mtiles, mt = local - slice * mtiles;
    // NT = 1 -> 16 consecutive W rows; NT = 2 (SiLU pair) -> rows c and c + 32
    // of one 64-row [in | gate] block.
    const int w_row0 = NT == 1 ? slice * 16 : (slice / 2) * 64 + (slice % 2) * 16;
    const int row0 = mt * RT;
    const int rows = min(p.M - row0, RT);
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: k ranges and step guards are scalar
    const int g4 = lane >> 4, li = lane & 15;
    const int spw = ((p.K + KS - 1) / KS + kDecWaves - 1) / kDecWaves;  // k steps per wave
    const int k_begin = min(p.K, wave * spw * KS), k_end = min(p.K, k_begin + spw * KS);
    const auto ra = make_rsrc(p.A + (size_t)row0 * p.lda, p.a_tiled ? (uint32_t)((size_t)RT * p.lda * 4)
                                                                     : (uint32_t)(((size_t)(rows - 1) * p.lda + p.K) * 4));
    // Tiled W when given (contiguous 1 KB per wave load), else row-major W.
    const bool tiled = WB ? p.Wht != nullptr : p.Wt != nullptr;
    const uint32_t tiles_bytes = (uint32_t)((size_t)((p.N + 15) / 16) * p.wt_ld * (WB ? 2 : 4));
    const auto rw = tiled ? make_rsrc(WB ? (const void *)p.Wht : (const void *)p.Wt, tiles_bytes)
                  : WB    ? make_rsrc(p.Wh, (uint32_t)(((size_t)(p.N - 1) * p.ldw + p.K) * 2))
                          : make_rsrc(p.W, (uint32_t)(((size_t)(p.N - 1) * p.ldw + p.K) * 4));

    floatx4 acc[NT][MI];
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int i = 0; i < MI; ++i) acc[t][i] = floatx4{0.f, 0.f, 0.f, 0.f};
    floatx4 a[S][MI][AH], b[S][NT];  // b: 4 fp32 W values, or 8 bf16 ones (raw bits)
    floatx4 gt[PRO == 2 ? S : 1][MI][AH];
    // The loaders are forced inline: left as calls (the inliner's choice at
    // S = 10 and at MI = 4), a and b are passed by address and live in scratch
    // memory, which made those instantiations about 13x slower.
    auto load4 =[](__amdgpu_buffer_rsrc_t rs, uint32_t off) __attribute__((always_inline)) {
        return __builtin_bit_cast(floatx4, __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, 0));
    };
    const auto rt = make_rsrc(PRO == 2 ? p.a_gate + (size_t)row0 * p.ldg : nullptr,
                              PRO == 2 ? (p.a_tiled ? (uint32_t)((size_t)RT * p.ldg * 4)
                                                    : (uint32_t)(((size_t)(rows - 1) * p.ldg + p.K) * 4))
                                       : 0u);
    auto load_w = [&](int s, int k0) __attribute__((always_inline)) {
        const int k = k0 + KS * s + RL * g4;
        const bool kin = k < k_end;  // K % RL == 0 on this path
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            const int wr = w_row0 + 32 * t + li;
            const size_t e = tiled ? (size_t)(wr >> 4) * p.wt_ld + (size_t)(k / KS) * (16 * KS) + (wr & 15) * KS + (k % KS)
                                   : (size_t)wr * p.ldw + k;
            b[s][t] = load4(rw, (kin && wr < p.N) ? (uint32_t)e * (WB ? 2u : 4u) : kBufferOob);
        }
    };
    auto load_a = [&](int s, int k0) __attribute__((always_inline)) {
        const int k = k0 + KS * s + RL * g4;
        const bool kin = k < k_end;
#pragma unroll
        for (int i = 0; i < MI; ++i)
#pragma unroll
            for (int hh = 0; hh < AH; ++hh)
                a[s][i][hh] = load4(ra, kin ? (uint32_t)(p.a_tiled ? tile_index(16 * i + li, k + 4 * hh, p.lda)
                                                                   : (size_t)(16 * i + li) * p.lda + k + 4 * hh) * 4u
                                            : kBufferOob);
        if constexpr (PRO == 2) {
#pragma unroll
            for (int i = 0; i < MI; ++i)
#pragma unroll
                for (int hh = 0; hh < AH; ++hh)
                    gt[s][i][hh] = load4(rt, kin ? (uint32_t)(p.a_tiled ? tile_index(16 * i + li, k + 4 * hh, p.ldg)
                                                                        : (size_t)(16 * i + li) * p.ldg + k + 4 * hh) * 4u
                                                 : kBufferOob);
        }
    };
    // Issue order: with a prologue, all A (and gate) loads of the round first,
    // so the row statistics wait for A only while W is still in flight.
    auto load_round = [&](int k0) __attribute__((always_inline)) {
        if constexpr (PRO > 0) {
#pragma unroll
            for (int s = 0; s < S; ++s) load_a(s, k0);
#pragma unroll
            for (int s = 0; s < S; ++s) load_w(s, k0);
        } else {
#pragma unroll
            for (int s = 0; s < S; ++s) {
                load_w(s, k0);
                load_a(s, k0);
            }
        }
    };
    // gamma and beta of the K columns (K <= 2 * kDecThreads), loaded between
    // the round's A and W loads.
    float gam[2], bet[2];
    if constexpr (PRO > 0) {
#pragma unroll
        for (int s = 0; s < S; ++s) load_a(s, k_begin);
        const auto rg = make_rsrc(p.ln_gamma, (uint32_t)p.K * 4u), rb = make_rsrc(p.ln_beta, (uint32_t)p.K * 4u);
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int c = tid + j * kDecThreads;
            gam[j] = buf_load(rg, c < p.K ? (uint32_t)c * 4u : kBufferOob);
            bet[j] = buf_load(rb, c < p.K ? (uint32_t)c * 4u : kBufferOob);
        }
#pragma unroll
        for (int s = 0; s < S; ++s) load_w(s, k_begin);
    } else {
        load_round(k_begin);
    }

    float mean[MI], rstd[MI];
    if constexpr (PRO > 0) {
        // gamma and beta of the K columns, shared by every row of the tile.
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int c = tid + j * kDecThreads;
            if (c < p.K) {
                affine[c] = gam[j];
                affine[64 * kDecLnPerLane + c] = bet[j];
            }
        }
        if (spw <= S) {
            // One round covers this wave's K range, so the row statistics come
            // from the A values already in registers: per-wave partial sums over
            // the wave's columns, combined across the waves through LDS (two
            // passes: the mean, then the squared deviations from it).
            float ps[MI];
#pragma unroll
            for (int i = 0; i < MI; ++i) {
                ps[i] = 0.0f;
#pragma unroll
                for (int s = 0; s < S; ++s)
#pragma unroll
                    for (int hh = 0; hh < AH; ++hh) ps[i] += (a[s][i][hh][0] + a[s][i][hh][1]) + (a[s][i][hh][2] + a[s][i][hh][3]);
                ps[i] += __shfl_xor(ps[i], 16);
                ps[i] += __shfl_xor(ps[i], 32);
                if (g4 == 0) part[0][wave][16 * i + li] = ps[i];
            }
            lds_barrier();
#pragma unroll
            for (int i = 0; i < MI; ++i) {
                float sum = 0.0f;
#pragma unroll
                for (int w = 0; w < kDecWaves; ++w) sum += part[0][w][16 * i + li];
                mean[i] = sum / (float)p.K;
                float sq = 0.0f;
#pragma unroll
                for (int s = 0; s < S; ++s) {
                    if (k_begin + KS * s + RL * g4 < k_end) {
#pragma unroll
                        for (int hh = 0; hh < AH; ++hh)
#pragma unroll
                            for (int q = 0; q < 4; ++q) {
                                const float dv = a[s][i][hh][q] - mean[i];
                                sq = fmaf(dv, dv, sq);
                            }
                    }
                }
                sq += __shfl_xor(sq, 16);
                sq += __shfl_xor(sq, 32);
                if (g4 == 0) part[1][wave][16 * i + li] = sq;
            }
            lds_barrier();
#pragma unroll
            for (int i = 0; i < MI; ++i) {
                float sq = 0.0f;
#pragma unroll
                for (int w = 0; w < kDecWaves; ++w) sq += part[1][w][16 * i + li];
                rstd[i] = rsqrtf(sq / (float)p.K + 1e-5f);
            }
        } else {
            // Row statistics: wave w normalises rows w, w + 16, ... of the tile.
            for (int rr = wave; rr < RT; rr += kDecWaves) {
                float v[kDecLnPerLane];
                float sum = 0.0f;
#pragma unroll
                for (int e = 0; e < kDecLnPerLane; ++e) {
                    const int c = lane + e * 64;
                    v[e] = buf_load(ra, c < p.K ? (uint32_t)((size_t)rr * p.lda + c) * 4u : kBufferOob);
                    sum += v[e];
                }
                const float mu = wave_sum(sum) / (float)p.K;
                float sq = 0.0f;
#pragma unroll
                for (int e = 0; e < kDecLnPerLane; ++e) {
                    const int c = lane + e * 64;
                    const float dv = c < p.K ? v[e] - mu : 0.0f;
                    sq = fmaf(dv, dv, sq);
                }
                const float rs = rsqrtf(wave_sum(sq) / (float)p.K + 1e-5f);
                if (lane == 0) {
                    stats[rr][0] = mu;
                    stats[rr][1] = rs;
                }
            }
            lds_barrier();
#pragma unroll
            for (int i = 0; i < MI; ++i) {
                mean[i] = stats[16 * i + li][0];
                rstd[i] = stats[16 * i + li][1];
            }
        }
    }

    for (int k0 = k_begin;;) {
#pragma unroll
        for (int s = 0; s < S; ++s) {
            if (k0 + KS * s >= k_end) break;  // steps past this wave's K range: no MFMAs on zeros
            if constexpr (PRO > 0) {
#pragma unroll
                for (int hh = 0; hh < AH; ++hh) {
                const int k = k0 + KS * s + RL * g4 + 4 * hh;
                if (k < k_end) {
                    const floatx4 gm = *reinterpret_cast<const floatx4 *>(affine + k);
                    const floatx4 bt = *reinterpret_cast<const floatx4 *>(affine + 64 * kDecLnPerLane + k);
#pragma unroll
                    for (int i = 0; i < MI; ++i)
#pragma unroll
                        for (int q = 0; q < 4; ++q) {
                            float y = (a[s][i][hh][q] - mean[i]) * rstd[i] * gm[q] + bt[q];
                            if constexpr (PRO == 2) y *= gt[s][i][hh][q];
                            a[s][i][hh][q] = y;
                        }
                }
                }
            }
            if constexpr (WB) {
#pragma unroll
                for (int i = 0; i < MI; ++i) {
                    bf16x8 ah, al;
                    split_bf16x8(a[s][i][0], a[s][i][AH - 1], ah, al);
#pragma unroll
                    for (int t = 0; t < NT; ++t) {
                        acc[t][i] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, __builtin_bit_cast(bf16x8, b[s][t]), acc[t][i], 0, 0, 0);
                        acc[t][i] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al, __builtin_bit_cast(bf16x8, b[s][t]), acc[t][i], 0, 0, 0);
                    }
                }
            } else {
#pragma unroll
                for (int r = 0; r < 4; ++r)
#pragma unroll
                    for (int t = 0; t < NT; ++t)
#pragma unroll
                        for (int i = 0; i < MI; ++i)
                            acc[t][i] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[s][i][0][r], b[s][t][r], acc[t][i], 0, 0, 0);
            }
        }
        k0 += KS * S;
        if (k0 >= k_end) break;
        load_round(k0);
    }
    // Register r of lane l in m-tile i: row 16 i + 4 (l / 16) + r, column l % 16.
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int i = 0; i < MI; ++i)
#pragma unroll
            for (int r = 0; r < 4; ++r) red[wave][t][(16 * i + 4 * g4 + r) * 17 + li] = acc[t][i][r];
    lds_barrier();
    for (int q = tid; q < RT * 16; q += kDecThreads) {
        const int rl = q >> 4, c = q & 15;
        if (rl >= rows) continue;
        const int row = row0 + rl;
        float x[NT];
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            float sum = 0.0f;
#pragma unroll
            for (int w = 0; w < kDecWaves; ++w) sum += red[w][t][rl * 17 + c];
            x[t] = sum;
        }
        if constexpr (NT == 2) {
            const int hcol = (w_row0 / 64) * 32 + (w_row0 % 64) + c;
            p.C[p.c_tiled ? tile_index(row, hcol, p.ldc) : (size_t)row * p.ldc + hcol] = x[0] / (1.0f + expf(-x[0])) * x[NT - 1];
        } else {
            const int col = w_row0 + c;
            if (col < p.N) {
                float y = apply_act(x[0] + (p.bias ? p.bias[col] : 0.0f), p.act);
                if (p.residual) y += p.residual[(size_t)row * p.ldr + col];
                p.C[(size_t)row * p.ldc + col] = y;
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Wide decode products (the LM head, yufmusicgen/model.py:421
// lm_head(final_norm(hidden)): M <= 64, far more 16-column slices than
// CUs, K <= 640, fp32 W).  The decode kernel above re-reads the 64 x K block of
// A once per slice (1,280 times for the LM head); here one workgroup per CU
// keeps its 8 waves' K ranges of all 64 rows in registers (S steps of 16 k;
// LayerNorm applied there once) and walks the slices g, g + G, ...: the next
// slice's W is in flight during the current slice's MFMAs, and the 8 partial
// tiles are summed through two alternating LDS buffers (one barrier a slice).
template <int S, bool LN>
__global__ void __launch_bounds__(kDecThreads) gemm_wide_kernel(GemmParams p, int slices) {
    __shared__ __attribute__((aligned(16))) float red[2][kDecWaves][64 * 17];
    __shared__ float part[2][kDecWaves][LN ? 64 : 1];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int g4 = lane >> 4, li = lane & 15;
    const int K = p.K, M = p.M, k0 = wave * 16 * S;
    const auto ra = make_rsrc(p.A, (uint32_t)(((size_t)(M - 1) * p.lda + K) * 4));
    const bool tiled = p.Wt != nullptr;  // 16 x 16 tiles: one contiguous 1 KB run per wave load
    const auto rw = tiled ? make_rsrc(p.Wt, (uint32_t)((size_t)((p.N + 15) / 16) * p.wt_ld * 4))
                          : make_rsrc(p.W, (uint32_t)(((size_t)(p.N - 1) * p.ldw + K) * 4));
    auto load4 = [](__amdgpu_buffer_rsrc_t rs, uint32_t off) __attribute__((always_inline)) {
        return __builtin_bit_cast(floatx4, __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, 0));
    };
    floatx4 a[S][4];
#pragma unroll
    for (int s = 0; s < S; ++s)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int k = k0 + 16 * s + 4 * g4, row = 16 * i + li;
            a[s][i] = load4(ra, row < M && k < K ? (uint32_t)((size_t)row * p.lda + k) * 4u : kBufferOob);
        }
    floatx4 b0[S], b1[S];
    auto load_w = [&](floatx4 (&b)[S], int slice) __attribute__((always_inline)) {
        const int wr = slice * 16 + li;
#pragma unroll
        for (int s = 0; s < S; ++s) {
            const int k = k0 + 16 * s + 4 * g4;
            const size_t e = tiled ? (size_t)slice * p.wt_ld + (size_t)(k >> 4) * 256 + li * 16 + (k & 15)
                                   : (size_t)wr * p.ldw + k;
            b[s] = load4(rw, slice < slices && wr < p.N && k < K ? (uint32_t)e * 4u : kBufferOob);
        }
    };
    int j = blockIdx.x;
    if constexpr (LN) {
        floatx4 gm[S], bt[S];
        const auto rg = make_rsrc(p.ln_gamma, (uint32_t)K * 4u), rb = make_rsrc(p.ln_beta, (uint32_t)K * 4u);
#pragma unroll
        for (int s = 0; s < S; ++s) {
            const int k = k0 + 16 * s + 4 * g4;
            gm[s] = load4(rg, k < K ? (uint32_t)k * 4u : kBufferOob);
            bt[s] = load4(rb, k < K ? (uint32_t)k * 4u : kBufferOob);
        }
        load_w(b0, j);
        // Row statistics (two passes, the decode kernel's expressions).
        float mean[4], rstd[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            float ps = 0.0f;
#pragma unroll
            for (int s = 0; s < S; ++s) ps += (a[s][i][0] + a[s][i][1]) + (a[s][i][2] + a[s][i][3]);
            ps += __shfl_xor(ps, 16);
            ps += __shfl_xor(ps, 32);
            if (g4 == 0) part[0][wave][16 * i + li] = ps;
        }
        lds_barrier();
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            float sum = 0.0f;
#pragma unroll
            for (int w = 0; w < kDecWaves; ++w) sum += part[0][w][16 * i + li];
            mean[i] = sum / (float)K;
            float sq = 0.0f;
#pragma unroll
            for (int s = 0; s < S; ++s)
                if (k0 + 16 * s + 4 * g4 < K) {
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const float dv = a[s][i][q] - mean[i];
                        sq = fmaf(dv, dv, sq);
                    }
                }
            sq += __shfl_xor(sq, 16);
            sq += __shfl_xor(sq, 32);
            if (g4 == 0) part[1][wave][16 * i + li] = sq;
        }
        lds_barrier();
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            float sq = 0.0f;
#pragma unroll
            for (int w = 0; w < kDecWaves; ++w) sq += part[1][w][16 * i + li];
            rstd[i] = rsqrtf(sq / (float)K + 1e-5f);
        }
#pragma unroll
        for (int s = 0; s < S; ++s) {
            const bool kin = k0 + 16 * s + 4 * g4 < K;
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int q = 0; q < 4; ++q)
                    a[s][i][q] = kin ? (a[s][i][q] - mean[i]) * rstd[i] * gm[s][q] + bt[s][q] : 0.0f;
        }
    } else {
        load_w(b0, j);
    }
    // One slice: MFMAs on b, the 8 partial tiles through red[RB], the epilogue.
    auto slice_step = [&](const floatx4 (&b)[S], int slice, float (*rbuf)[64 * 17]) {
        floatx4 acc[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[i] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < S; ++s)
#pragma unroll
            for (int r = 0; r < 4; ++r)
#pragma unroll
                for (int i = 0; i < 4; ++i) acc[i] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[s][i][r], b[s][r], acc[i], 0, 0, 0);
        // Register r of lane l in m-tile i: row 16 i + 4 (l / 16) + r, column l % 16.
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int r = 0; r < 4; ++r) rbuf[wave][(16 * i + 4 * g4 + r) * 17 + li] = acc[i][r];
        lds_barrier();
#pragma unroll
        for (int e = 0; e < 2; ++e) {
            const int q = tid + e * kDecThreads, rl = q >> 4, c = q & 15, col = slice * 16 + c;
            if (rl < M && col < p.N) {
                float x = 0.0f;
#pragma unroll
                for (int w = 0; w < kDecWaves; ++w) x += rbuf[w][rl * 17 + c];
                float y = apply_act(x + (p.bias ? p.bias[col] : 0.0f), p.act);
                if (p.residual) y += p.residual[(size_t)rl * p.ldr + col];
                p.C[(size_t)rl * p.ldc + col] = y;
            }
        }
    };
    const int G = gridDim.x;
    while (j < slices) {
        load_w(b1, j + G);
        slice_step(b0, j, red[0]);
        j += G;
        if (j >= slices) break;
        load_w(b0, j + G);
        slice_step(b1, j, red[1]);
        j += G;
    }
}

// ---------------------------------------------------------------------------
// Decode ROSA output projection with the ROSA step as its A prologue
// (yufmusicgen/model.py:296-311: output(H(m_t) * sigmoid(read_gate)), the step
// of yufmusicgen/cuda/rosa_householder.cu:63-101 for T = 1).  The
// unit of work is the decode GEMM's (16-column slice, 16-row tile) with the 8
// waves splitting K = D (S steps of 16 k per wave); each lane holds 4 k of one
// row per step.  The step's two projections u.m and u.m' are summed in double
// (lane partials -> the row's 4 lanes through the row swaps -> the 8 waves in
// a fixed order through LDS), then the read A[m][k] feeds the MFMAs directly,
// so the separate step kernel and its read buffer go away.  Every workgroup of
// a row tile computes the tile's new memory rows; the last one to finish (a
// device-scope counter per tile, incremented after the tile's reads) stores
// them in place and resets the counter.  Cross-workgroup traffic is only that
// counter: the stores never race a read of the old rows.
template <int S>
__global__ void __launch_bounds__(kDecThreads) rosa_out_decode_kernel(RosaOutParams p, int mtiles, int units,
                                                                      int per_xcd) {
    __shared__ __attribute__((aligned(16))) float red[kDecWaves][16 * 17];
    __shared__ double pd[2][kDecWaves][16];
    __shared__ int last;
    const int u = (blockIdx.x % kXcds) * per_xcd + blockIdx.x / kXcds;
    if (u >= units) return;
    const int slice = u / mtiles, mt = u - slice * mtiles;
    const int row0 = mt * 16, rows = min(p.M - row0, 16);
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int g4 = lane >> 4, li = lane & 15;
    const bool rv = li < rows;
    const int slot = rv ? (p.slot ? p.slot[row0 + li] : row0 + li) : 0;
    const int D = p.D, kw = wave * 16 * S;
    const auto rm = make_rsrc(p.mem, (uint32_t)((size_t)p.mem_rows * D * 4));
    const auto rp = make_rsrc(p.pre + (size_t)row0 * p.ld_pre, (uint32_t)(((size_t)(rows - 1) * p.ld_pre + 3 * D) * 4));
    const auto ru = make_rsrc(p.u, (uint32_t)D * 4u), rl = make_rsrc(p.lam, (uint32_t)D * 4u);
    const bool tiled = p.Wt != nullptr;  // one contiguous 1 KB run per wave load
    const auto rw = tiled ? make_rsrc(p.Wt, (uint32_t)((size_t)((p.N + 15) / 16) * p.wt_ld * 4))
                          : make_rsrc(p.W, (uint32_t)((size_t)p.N * D * 4));
    auto load4 = [](__amdgpu_buffer_rsrc_t rs, uint32_t off) {
        return __builtin_bit_cast(floatx4, __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, 0));
    };
    const int wr = slice * 16 + li;
    floatx4 m[S], e[S], gw[S], rr[S], uu[S], ll[S], b[S];
#pragma unroll
    for (int s = 0; s < S; ++s) {
        const int k = kw + 16 * s + 4 * g4;
        const size_t we = tiled ? (size_t)slice * p.wt_ld + (size_t)(k >> 4) * 256 + li * 16 + (k & 15) : (size_t)wr * D + k;
        b[s] = load4(rw, wr < p.N ? (uint32_t)we * 4u : kBufferOob);
        m[s] = load4(rm, rv ? (uint32_t)((size_t)slot * D + k) * 4u : kBufferOob);
        e[s] = load4(rp, rv ? (uint32_t)((size_t)li * p.ld_pre + k) * 4u : kBufferOob);
        gw[s] = load4(rp, rv ? (uint32_t)((size_t)li * p.ld_pre + D + k) * 4u : kBufferOob);
        rr[s] = load4(rp, rv ? (uint32_t)((size_t)li * p.ld_pre + 2 * D + k) * 4u : kBufferOob);
        uu[s] = load4(ru, (uint32_t)k * 4u);
        ll[s] = load4(rl, (uint32_t)k * 4u);
    }
    // Gates (the single-token kernel's expressions): e <- tanh(e) sigmoid(write),
    // rr <- sigmoid(read_raw); first projection u.m.
    double f = 0.0;
#pragma unroll
    for (int s = 0; s < S; ++s)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const float th = 1.0f - 2.0f * __frcp_rn(__expf(2.0f * e[s][q]) + 1.0f);
            e[s][q] = th * __frcp_rn(1.0f + __expf(-gw[s][q]));
            rr[s][q] = __frcp_rn(1.0f + __expf(-rr[s][q]));
            f = fma((double)uu[s][q], (double)m[s][q], f);
        }
    f = rows_sum_f64(f);
    if (g4 == 0) pd[0][wave][li] = f;
    lds_barrier();
    double t = 0.0;
#pragma unroll
    for (int w = 0; w < kDecWaves; ++w) t += pd[0][w][li];
    const float p1 = (float)t;
    double f2 = 0.0;
#pragma unroll
    for (int s = 0; s < S; ++s)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            m[s][q] = fmaf(ll[s][q], fmaf(-2.0f * p1, uu[s][q], m[s][q]), e[s][q]);
            f2 = fma((double)uu[s][q], (double)m[s][q], f2);
        }
    f2 = rows_sum_f64(f2);
    if (g4 == 0) pd[1][wave][li] = f2;
    lds_barrier();
    t = 0.0;
#pragma unroll
    for (int w = 0; w < kDecWaves; ++w) t += pd[1][w][li];
    const float p2 = (float)t;
    floatx4 acc = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < S; ++s) {
        floatx4 a;
#pragma unroll
        for (int q = 0; q < 4; ++q) a[q] = fmaf(-2.0f * p2, uu[s][q], m[s][q]) * rr[s][q];
#pragma unroll
        for (int r = 0; r < 4; ++r) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[r], b[s][r], acc, 0, 0, 0);
    }
    // Register r of lane l: row 4 (l / 16) + r, column l % 16.
#pragma unroll
    for (int r = 0; r < 4; ++r) red[wave][(4 * g4 + r) * 17 + li] = acc[r];
    lds_barrier();
    if (tid < 256) {
        const int rl = tid >> 4, c = tid & 15, col = slice * 16 + c;
        if (rl < rows && col < p.N) {
            float x = 0.0f;
#pragma unroll
            for (int w = 0; w < kDecWaves; ++w) x += red[w][rl * 17 + c];
            const int row = row0 + rl;
            if (p.bias) x += p.bias[col];
            if (p.residual) x += p.residual[(size_t)row * p.ldr + col];
            p.C[(size_t)row * p.ldc + col] = x;
        }
    }
    // Every wave has consumed its old memory values (p1 needed them): count
    // this workgroup; the tile's last one writes the new rows.
    if (tid == 0) last = atomicAdd(&p.counter[mt], 1) == units / mtiles - 1;
    lds_barrier();
    if (last) {
        if (rv) {
#pragma unroll
            for (int s = 0; s < S; ++s) {
                const int k = kw + 16 * s + 4 * g4;
                __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, m[s]), rm,
                                                       (uint32_t)((size_t)slot * D + k) * 4u, 0, 0);
            }
        }
        if (tid == 0) atomicExch(&p.counter[mt], 0);
    }
}

// ---------------------------------------------------------------------------
// Short-M path (decode: M <= 64 rows, one token per stream).  The product is
// bound by streaming W from HBM, so parallelism comes from N and K instead of
// M: each wave owns 64 rows x 64 columns (2 x 2 MFMA 32x32 tiles) over a K
// slice, reading A (small, L2-resident) and W directly from global memory with
// 16-float contiguous runs per lane; split-K partials go to a workspace and a
// second kernel sums them in a fixed order and applies the epilogue.
// ---------------------------------------------------------------------------
constexpr int kSkinnyWaves = 4;
constexpr int kSkinnyTargetWaves = 1024;

struct SkinnyFrag {
    float v[16];
};

__device__ __forceinline__ void skinny_load(SkinnyFrag &f, __amdgpu_buffer_rsrc_t rsrc, int row, int ld, int k,
                                            int K) {
    if (k + 15 < K) {
        const uint32_t off = (uint32_t)((size_t)row * ld + k) * 4u;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const auto raw = __builtin_amdgcn_raw_buffer_load_b128(rsrc, off + q * 16, 0, 0);
            const float4 x = __builtin_bit_cast(float4, raw);
            f.v[4 * q] = x.x; f.v[4 * q + 1] = x.y; f.v[4 * q + 2] = x.z; f.v[4 * q + 3] = x.w;
        }
    } else {
#pragma unroll
        for (int q = 0; q < 16; ++q)
            f.v[q] = buf_load(rsrc, k + q < K ? (uint32_t)((size_t)row * ld + k + q) * 4u : kBufferOob);
    }
}

__device__ __forceinline__ void store_out(const GemmParams &p, int row, int col, float x) {
    x = apply_act(x + (p.bias ? p.bias[col] : 0.0f), p.act);
    if (p.residual) x += p.residual[(size_t)row * p.ldr + col];
    p.C[(size_t)row * p.ldc + col] = x;
}

__global__ void __launch_bounds__(64 * kSkinnyWaves) gemm_skinny_kernel(GemmParams p, int k_chunk, int splits) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int n0 = (blockIdx.x * kSkinnyWaves + wave) * 64;
    if (n0 >= p.N) return;
    const int split = blockIdx.y;
    const int k_begin = split * k_chunk;
    const int k_end = min(p.K, k_begin + k_chunk);
    const int rows = min(p.M, 64);
    const auto ra = make_rsrc(p.A, (uint32_t)(((size_t)(rows - 1) * p.lda + p.K) * 4));
    const int ncols = min(64, p.N - n0);
    const auto rw = make_rsrc(p.W + (size_t)n0 * p.ldw, (uint32_t)(((size_t)(ncols - 1) * p.ldw + p.K) * 4));

    floatx16 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = floatx16{};
    const int r_in = lane & 31, k_half = (lane >> 5) * 16;
    SkinnyFrag a[2], w[2], an[2], wn[2];
    int k = k_begin;
    if (k < k_end) {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            skinny_load(a[i], ra, i * 32 + r_in, p.lda, k + k_half, k_end);
            skinny_load(w[i], rw, i * 32 + r_in, p.ldw, k + k_half, k_end);
        }
    }
    for (; k < k_end; k += 32) {
        const bool more = k + 32 < k_end;
        if (more) {
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                skinny_load(an[i], ra, i * 32 + r_in, p.lda, k + 32 + k_half, k_end);
                skinny_load(wn[i], rw, i * 32 + r_in, p.ldw, k + 32 + k_half, k_end);
            }
        }
#pragma unroll
        for (int s = 0; s < 16; ++s)
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[i].v[s], w[j].v[s], acc[i][j], 0, 0, 0);
        if (more) {
#pragma unroll
            for (int i = 0; i < 2; ++i) { a[i] = an[i]; w[i] = wn[i]; }
        }
    }
    const int col_in_tile = lane & 31, row_base = (lane >> 5) * 4;
    if (splits > 1) {
        float *part = p.workspace + (size_t)split * p.M * p.N;
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int col = n0 + j * 32 + col_in_tile;
            if (col >= p.N) continue;
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int row = i * 32 + (r >> 2) * 8 + row_base + (r & 3);
                    if (row < p.M) part[(size_t)row * p.N + col] = acc[i][j][r];
                }
        }
        return;
    }
    if (p.silu_pair) {
        const int hcol = n0 / 2 + col_in_tile;
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int row = i * 32 + (r >> 2) * 8 + row_base + (r & 3);
                if (row < p.M) {
                    const float x = acc[i][0][r], g = acc[i][1][r];
                    p.C[(size_t)row * p.ldc + hcol] = x / (1.0f + expf(-x)) * g;
                }
            }
        return;
    }
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int col = n0 + j * 32 + col_in_tile;
        if (col >= p.N) continue;
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int row = i * 32 + (r >> 2) * 8 + row_base + (r & 3);
                if (row < p.M) store_out(p, row, col, acc[i][j][r]);
            }
    }
}

// Sum the split-K partials in split order and apply the epilogue.
__global__ void gemm_splitk_reduce_kernel(GemmParams p, int splits) {
    const int out_cols = p.silu_pair ? p.N / 2 : p.N;
    const size_t total = (size_t)p.M * out_cols;
    const size_t plane = (size_t)p.M * p.N;
    for (size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
         idx += (size_t)gridDim.x * blockDim.x) {
        const int row = (int)(idx / out_cols), c = (int)(idx - (size_t)row * out_cols);
        if (p.silu_pair) {
            const int q = c / 32, cc = c - q * 32;
            const int cin = q * 64 + cc, cgate = cin + 32;
            float x = 0.0f, g = 0.0f;
            for (int s = 0; s < splits; ++s) {
                x += p.workspace[s * plane + (size_t)row * p.N + cin];
                g += p.workspace[s * plane + (size_t)row * p.N + cgate];
            }
            p.C[(size_t)row * p.ldc + c] = x / (1.0f + expf(-x)) * g;
        } else {
            float x = 0.0f;
            for (int s = 0; s < splits; ++s) x += p.workspace[s * plane + (size_t)row * p.N + c];
            store_out(p, row, c, x);
        }
    }
}

template <int BN, bool WB, bool X3 = false>
void launch_big(const GemmGroup &g, int per_xcd, bool staged, dim3 grid, hipStream_t stream) {
    if (staged)
        hipLaunchKernelGGL((gemm_big_kernel<BN, true, WB, X3>), grid, dim3(kBigThreads), 0, stream, g, per_xcd);
    else
        hipLaunchKernelGGL((gemm_big_kernel<BN, false, WB, X3>), grid, dim3(kBigThreads), 0, stream, g, per_xcd);
}

template <int BN, int MI = 4>
void launch_x3p(const GemmGroup &g, int per_xcd, bool staged, dim3 grid, hipStream_t stream) {
    if (staged)
        hipLaunchKernelGGL((gemm_x3p_kernel<BN, true, MI>), grid, dim3(kBigThreads), 0, stream, g, per_xcd);
    else
        hipLaunchKernelGGL((gemm_x3p_kernel<BN, false, MI>), grid, dim3(kBigThreads), 0, stream, g, per_xcd);
}

// The X3 form from pre-split weight planes when every product of the group
// has them and its A rows can be loaded straight into LDS (16-byte aligned
// rows); otherwise gemm_big_kernel splits W itself.
bool use_x3p(const GemmGroup &g, int n) {
    for (int i = 0; i < n; ++i) {
        const GemmParams &p = g.p[i];
        if (!p.Wp || p.K % 32 != 0 || p.N % 16 != 0 || p.lda % 4 != 0 ||
            (reinterpret_cast<uintptr_t>(p.A) & 15) != 0 || x3_planes_elems(p.N, p.K) * 2 >= (1ull << 32))
            return false;
    }
    return true;
}

// fp32 products on the bf16 matrix cores through three-part splits (the X3
// form of gemm_big_kernel) when every K of the group is a multiple of 32;
// YUF_GEMM_X3=0 keeps the fp32 MFMA form.
bool use_x3(const GemmGroup &g, int n) {
    static const bool enabled = [] {
        const char *e = std::getenv("YUF_GEMM_X3");
        return !(e && std::strcmp(e, "0") == 0);
    }();
    if (!enabled) return false;
    for (int i = 0; i < n; ++i)
        if (g.p[i].K % 32 != 0) return false;
    return true;
}

template <int NT, int MI, int PRO, bool WB, int S>
void launch_dec_s(const DecodeGroup &g, dim3 grid, hipStream_t stream) {
    if constexpr (S <= dec_cap(NT, MI, PRO, WB)) {
        if (g.count == 1)
            hipLaunchKernelGGL((gemm_decode_kernel<NT, MI, S, PRO, false, WB>), grid, dim3(kDecThreads), 0, stream, g);
        else if constexpr (PRO == 0)
            hipLaunchKernelGGL((gemm_decode_kernel<NT, MI, S, PRO, true, WB>), grid, dim3(kDecThreads), 0, stream, g);
    }
}

template <int NT, int MI, int PRO, bool WB>
void launch_dec(const DecodeGroup &g, int S, dim3 grid, hipStream_t stream) {
    switch (S) {
        case 1: launch_dec_s<NT, MI, PRO, WB, 1>(g, grid, stream); break;
        case 2: launch_dec_s<NT, MI, PRO, WB, 2>(g, grid, stream); break;
        case 3: launch_dec_s<NT, MI, PRO, WB, 3>(g, grid, stream); break;
        case 4: launch_dec_s<NT, MI, PRO, WB, 4>(g, grid, stream); break;
        case 5: launch_dec_s<NT, MI, PRO, WB, 5>(g, grid, stream); break;
        case 6: launch_dec_s<NT, MI, PRO, WB, 6>(g, grid, stream); break;
        default: launch_dec_s<NT, MI, PRO, WB, 10>(g, grid, stream); break;
    }
}

template <bool WB>
void launch_dec_kind(const DecodeGroup &g, int NT, int MI, int PRO, int S, dim3 grid, hipStream_t stream) {
    if (PRO == 0) {
        if (NT == 1) {
            if (MI == 1) launch_dec<1, 1, 0, WB>(g, S, grid, stream);
            else launch_dec<1, 4, 0, WB>(g, S, grid, stream);
        } else {
            if (MI == 1) launch_dec<2, 1, 0, WB>(g, S, grid, stream);
            else launch_dec<2, 4, 0, WB>(g, S, grid, stream);
        }
    } else if (PRO == 1) {
        if (NT == 2) launch_dec<2, 1, 1, WB>(g, S, grid, stream);
        else if (MI == 1) launch_dec<1, 1, 1, WB>(g, S, grid, stream);
        else launch_dec<1, 4, 1, WB>(g, S, grid, stream);
    } else {
        launch_dec<1, 1, 2, WB>(g, S, grid, stream);
    }
}

// Smallest instantiated S >= min(steps per wave, cap).
int pick_steps(int spw, int cap) {
    const int want = std::min(spw, cap);
    for (int s : {1, 2, 3, 4, 5, 6, 10})
        if (s >= want && s <= cap) return s;
    return cap;
}

int dec_prologue(const GemmParams &p) { return p.ln_gamma ? (p.a_gate ? 2 : 1) : 0; }

// Decode products (M <= 64, K % 4 == 0; K % 8 == 0 for bf16 W): one launch per
// group; all products of a group share the SiLU-pair flag, the prologue kind
// and the weight type.
hipError_t launch_decode(const GemmParams *ps, int count, hipStream_t stream) {
    if (count < 1 || count > kMaxDecode) return hipErrorInvalidValue;
    const int NT = ps[0].silu_pair ? 2 : 1, PRO = dec_prologue(ps[0]);
    const bool WB = ps[0].Wh != nullptr;
    const int KS = WB ? 32 : 16;
    if (PRO > 0 && count > 1) {  // grouped launches exist for plain products only
        for (int i = 0; i < count; ++i) {
            const hipError_t e = launch_decode(ps + i, 1, stream);
            if (e != hipSuccess) return e;
        }
        return hipSuccess;
    }
    int units1 = 0, spw = 1;
    for (int i = 0; i < count; ++i) {
        const GemmParams &p = ps[i];
        const int slices = p.silu_pair ? p.N / 32 : (p.N + 15) / 16;
        units1 += slices * ((p.M + 15) / 16);
        spw = std::max(spw, ((p.K + KS - 1) / KS + kDecWaves - 1) / kDecWaves);
    }
    // Wide products (the LM head) already fill the chip with 64-row tiles.
    // (Measured: the LN + SiLU-pair FFN input is slower with them, 17.7 against
    // 15.1 us at 64 x 5120 x 640, so it keeps 16-row tiles.)
    const int MI = (units1 > 1024 && PRO < 2 && !(PRO == 1 && NT == 2)) ? 4 : 1;
    DecodeGroup g{};
    g.count = count;
    for (int i = 0; i < count; ++i) {
        const GemmParams &p = ps[i];
        const int slices = p.silu_pair ? p.N / 32 : (p.N + 15) / 16;
        g.p[i] = p;
        g.mtiles[i] = (p.M + 16 * MI - 1) / (16 * MI);
        g.units += slices * g.mtiles[i];
        g.unit_end[i] = g.units;
    }
    g.per_xcd = (g.units + kXcds - 1) / kXcds;
    const dim3 grid(g.per_xcd * kXcds);
    const int cap = dec_cap(NT, MI, PRO, WB);
    const int S = pick_steps(spw, cap);
    if (PRO == 2 && NT == 2) return hipErrorInvalidValue;
    // A tiled A is read in the MFMA layout only: one round of k steps per wave
    // (no later rounds and no row re-reads for the LayerNorm statistics).
    for (int i = 0; i < count; ++i)
        if ((ps[i].a_tiled || ps[i].c_tiled) && spw > S) return hipErrorInvalidValue;
    if (WB) launch_dec_kind<true>(g, NT, MI, PRO, S, grid, stream);
    else launch_dec_kind<false>(g, NT, MI, PRO, S, grid, stream);
    return hipGetLastError();
}

bool decode_ok(const GemmParams &p) { return p.M <= 64 && p.K % (p.Wh ? 8 : 4) == 0; }

// The A-side prologue exists on the decode path only, for K <= 1024.
bool prologue_ok(const GemmParams &p) {
    if (!p.ln_gamma && !p.a_gate) return true;
    return p.ln_gamma && p.ln_beta && decode_ok(p) && p.K <= 64 * kDecLnPerLane && !(p.a_gate && p.silu_pair) &&
           (!p.a_gate || p.ldg >= p.K);
}

int skinny_splits(int N, int K) {
    const int wave_tiles = (N + 63) / 64;
    const int max_splits = (K + 31) / 32;
    int s = (kSkinnyTargetWaves + wave_tiles - 1) / wave_tiles;
    s = s < 1 ? 1 : (s > max_splits ? max_splits : s);
    return s > 64 ? 64 : s;
}

}  // namespace

// The wide form: single plain or LN-prologue products, fp32 W, 32 < M <= 64,
// K <= 640, at least 512 slices (the LM head).
static int wide_steps(const GemmParams &p) {
    if (p.Wh || p.silu_pair || p.a_gate || p.M <= 32 || p.M > 64 || p.K % 4 != 0 || p.K > 640) return 0;
    if ((p.N + 15) / 16 < 512) return 0;
    return ((p.K + 15) / 16 + kDecWaves - 1) / kDecWaves;
}

template <int S>
static void launch_wide_s(const GemmParams &p, int slices, hipStream_t stream) {
    const dim3 grid(std::min(slices, 256)), block(kDecThreads);
    if (p.ln_gamma)
        hipLaunchKernelGGL((gemm_wide_kernel<S, true>), grid, block, 0, stream, p, slices);
    else
        hipLaunchKernelGGL((gemm_wide_kernel<S, false>), grid, block, 0, stream, p, slices);
}

static hipError_t launch_wide(const GemmParams &p, int steps, hipStream_t stream) {
    const int slices = (p.N + 15) / 16;
    switch (steps) {
        case 1: launch_wide_s<1>(p, slices, stream); break;
        case 2: launch_wide_s<2>(p, slices, stream); break;
        case 3: launch_wide_s<3>(p, slices, stream); break;
        case 4: launch_wide_s<4>(p, slices, stream); break;
        case 5: launch_wide_s<5>(p, slices, stream); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

bool rosa_out_decode_ok(int M, int D) { return M >= 1 && M <= 64 && (D == 128 || D == 256); }

hipError_t launch_rosa_out_decode(const RosaOutParams &p, hipStream_t stream) {
    if (p.M <= 0 || p.N <= 0) return hipSuccess;
    if (!rosa_out_decode_ok(p.M, p.D) || !p.pre || !p.mem || !p.u || !p.lam || !p.W || !p.C || !p.counter ||
        p.ld_pre < 3 * p.D || p.mem_rows < 1)
        return hipErrorInvalidValue;
    const int mtiles = (p.M + 15) / 16, units = ((p.N + 15) / 16) * mtiles;
    const int per_xcd = (units + kXcds - 1) / kXcds;
    const dim3 grid(per_xcd * kXcds), block(kDecThreads);
    if (p.D == 128)
        hipLaunchKernelGGL(rosa_out_decode_kernel<1>, grid, block, 0, stream, p, mtiles, units, per_xcd);
    else
        hipLaunchKernelGGL(rosa_out_decode_kernel<2>, grid, block, 0, stream, p, mtiles, units, per_xcd);
    return hipGetLastError();
}

hipError_t launch_gemm(const GemmParams &p, hipStream_t stream) {
    if (p.M <= 0 || p.N <= 0) return hipSuccess;
    if (p.K <= 0 || p.lda < p.K || p.ldw < p.K) return hipErrorInvalidValue;
    if (p.silu_pair && (p.N % 64) != 0) return hipErrorInvalidValue;
    // Buffer descriptors address at most 2^31 bytes per 128-row panel.
    if ((size_t)kBM * p.lda * 4 >= (1u << 31) || (size_t)kBN * p.ldw * 4 >= (1u << 31)) return hipErrorInvalidValue;
    if (!prologue_ok(p)) return hipErrorInvalidValue;
    if ((p.a_tiled || p.c_tiled) && (!decode_ok(p) || wide_steps(p))) return hipErrorInvalidValue;  // decode kernel only
    if (const int ws = wide_steps(p)) return launch_wide(p, ws, stream);
    if (decode_ok(p)) return launch_decode(&p, 1, stream);
    if (p.Wh) return launch_gemm_group(&p, 1, stream);  // bf16 W: large-tile path or an error
    if (p.M <= 64) {
        int splits = skinny_splits(p.N, p.K);
        if (!p.workspace || (size_t)splits * p.M * p.N > p.workspace_floats) splits = 1;
        const int k_chunk = ((p.K + splits - 1) / splits + 31) / 32 * 32;
        splits = (p.K + k_chunk - 1) / k_chunk;
        const int wave_tiles = (p.N + 63) / 64;
        const dim3 grid((wave_tiles + kSkinnyWaves - 1) / kSkinnyWaves, splits);
        hipLaunchKernelGGL(gemm_skinny_kernel, grid, dim3(64 * kSkinnyWaves), 0, stream, p, k_chunk, splits);
        if (splits > 1) {
            const size_t outs = (size_t)p.M * (p.silu_pair ? p.N / 2 : p.N);
            const int blocks = (int)std::min<size_t>((outs + 255) / 256, 4096);
            hipLaunchKernelGGL(gemm_splitk_reduce_kernel, dim3(blocks), dim3(256), 0, stream, p, splits);
        }
        return hipGetLastError();
    }
    return launch_gemm_group(&p, 1, stream);
}

hipError_t launch_gemm_group(const GemmParams *ps, int count, hipStream_t stream) {
    if (count < 1 || count > kMaxGroup) return hipErrorInvalidValue;
    for (int i = 0; i < count; ++i) {
        if (ps[i].M > 0 && ps[i].N > 0 && !prologue_ok(ps[i])) return hipErrorInvalidValue;
        if ((ps[i].a_tiled || ps[i].c_tiled) && !decode_ok(ps[i])) return hipErrorInvalidValue;  // decode kernel only
    }
    {
        // Decode-shaped products: one launch per (SiLU flag, prologue kind, W type).
        GemmParams dec[12][kMaxGroup];
        int nd[12] = {};
        for (int i = 0; i < count; ++i) {
            const GemmParams &p = ps[i];
            if (p.M <= 0 || p.N <= 0 || !decode_ok(p)) continue;
            if (p.K <= 0 || p.lda < p.K || p.ldw < p.K) return hipErrorInvalidValue;
            if (p.silu_pair && (p.N % 64) != 0) return hipErrorInvalidValue;
            const int key = (p.Wh ? 6 : 0) + (p.silu_pair ? 3 : 0) + dec_prologue(p);
            dec[key][nd[key]++] = p;
        }
        for (int f = 0; f < 12; ++f)
            if (nd[f] > 0) {
                hipError_t e = launch_decode(dec[f], nd[f], stream);
                if (e != hipSuccess) return e;
            }
    }
    // bf16-weight products: the large-tile kernel for any M, or an error.
    {
        GemmGroup gh{};
        int nh = 0, hmax = 0;
        bool f256 = true, f160 = true, f128 = true, f64 = true;
        for (int i = 0; i < count; ++i) {
            const GemmParams &p = ps[i];
            if (p.M <= 0 || p.N <= 0 || !p.Wh || decode_ok(p)) continue;
            if (p.K <= 0 || p.K % 8 != 0 || p.lda < p.K || p.ldw < p.K) return hipErrorInvalidValue;
            if (p.silu_pair && (p.N % 64) != 0) return hipErrorInvalidValue;
            if ((size_t)kBigBM * p.lda * 4 >= (1u << 31) || (size_t)256 * p.ldw * 2 >= (1u << 31)) return hipErrorInvalidValue;
            f256 = f256 && p.N % 256 == 0;
            f160 = f160 && p.N % 160 == 0 && !p.silu_pair;
            f128 = f128 && p.N % 128 == 0;
            f64 = f64 && p.N % 64 == 0 && !p.silu_pair;
            gh.p[nh++] = p;
        }
        if (nh > 0) {
            if (!(f256 || f160 || f128 || f64)) return hipErrorInvalidValue;
            const int bn = f256 ? 256 : f160 ? 160 : f128 ? 128 : 64;
            bool staged = true;
            for (int i = 0; i < nh; ++i) {
                const GemmParams &p = gh.p[i];
                gh.tiles_n[i] = p.N / bn;
                gh.total[i] = ((p.M + kBigBM - 1) / kBigBM) * gh.tiles_n[i];
                hmax = std::max(hmax, gh.total[i]);
                const uintptr_t bits = reinterpret_cast<uintptr_t>(p.C) | reinterpret_cast<uintptr_t>(p.residual) |
                                       reinterpret_cast<uintptr_t>(p.bias);
                staged = staged && (bits & 15) == 0 && p.ldc % 4 == 0 && (!p.residual || p.ldr % 4 == 0);
            }
            const int per_xcd = (hmax + kXcds - 1) / kXcds;
            const dim3 grid(per_xcd * kXcds, nh);
            switch (bn) {
                case 256: launch_big<256, true>(gh, per_xcd, staged, grid, stream); break;
                case 160: launch_big<160, true>(gh, per_xcd, staged, grid, stream); break;
                case 128: launch_big<128, true>(gh, per_xcd, staged, grid, stream); break;
                default: launch_big<64, true>(gh, per_xcd, staged, grid, stream); break;
            }
            const hipError_t e = hipGetLastError();
            if (e != hipSuccess) return e;
        }
    }
    GemmGroup g{};
    int max_total = 0, n = 0;
    for (int i = 0; i < count; ++i) {
        const GemmParams &p = ps[i];
        if (p.M <= 0 || p.N <= 0) continue;
        if (decode_ok(p) || p.Wh) continue;  // launched above
        if (p.M <= 64) {  // short-M products take the split-K path one by one
            hipError_t e = launch_gemm(p, stream);
            if (e != hipSuccess) return e;
            continue;
        }
        if (p.K <= 0 || p.lda < p.K || p.ldw < p.K) return hipErrorInvalidValue;
        if (p.silu_pair && (p.N % 64) != 0) return hipErrorInvalidValue;
        if ((size_t)kBM * p.lda * 4 >= (1u << 31) || (size_t)kBN * p.ldw * 4 >= (1u << 31)) return hipErrorInvalidValue;
        g.p[n] = p;
        g.tiles_n[n] = (p.N + kBN - 1) / kBN;
        g.total[n] = ((p.M + kBM - 1) / kBM) * g.tiles_n[n];
        max_total = std::max(max_total, g.total[n]);
        ++n;
    }
    if (n == 0) return hipSuccess;
    // Large-tile path when every product of the group fits one of its tile widths.
    bool fit256 = true, fit160 = true, fit128 = true, fit64 = true;
    for (int i = 0; i < n; ++i) {
        const GemmParams &p = g.p[i];
        const bool big_ok = p.M >= kBigBM && p.K % 4 == 0 &&
                            (size_t)kBigBM * p.lda * 4 < (1u << 31) && (size_t)256 * p.ldw * 4 < (1u << 31);
        fit256 = fit256 && big_ok && p.N % 256 == 0;
        fit160 = fit160 && big_ok && p.N % 160 == 0 && !p.silu_pair;
        fit128 = fit128 && big_ok && p.N % 128 == 0;
        fit64 = fit64 && big_ok && p.N % 64 == 0 && !p.silu_pair;
    }
    if (fit256 || fit160 || fit128 || fit64) {
        const int bn = fit256 ? 256 : fit160 ? 160 : fit128 ? 128 : 64;
        int big_max = 0;
        for (int i = 0; i < n; ++i) {
            g.tiles_n[i] = g.p[i].N / bn;
            g.total[i] = ((g.p[i].M + kBigBM - 1) / kBigBM) * g.tiles_n[i];
            big_max = std::max(big_max, g.total[i]);
        }
        const int per_xcd = (big_max + kXcds - 1) / kXcds;
        bool staged = true;  // 16-byte epilogue accesses need aligned C / residual / bias rows
        for (int i = 0; i < n; ++i) {
            const GemmParams &p = g.p[i];
            const uintptr_t bits = reinterpret_cast<uintptr_t>(p.C) | reinterpret_cast<uintptr_t>(p.residual) |
                                   reinterpret_cast<uintptr_t>(p.bias);
            staged = staged && (bits & 15) == 0 && p.ldc % 4 == 0 && (!p.residual || p.ldr % 4 == 0);
        }
        const dim3 grid(per_xcd * kXcds, n), block(kBigThreads);
        if (use_x3(g, n) && use_x3p(g, n)) {
            // Memory-bound shapes -- products of at most 64 columns (A read once
            // per 64 outputs) or K <= 128 (the output write dominates) -- take
            // 64-row tiles when the tile is at most 160 wide: four times the
            // workgroups, each with at most 76 KB of LDS, so two or more share
            // a CU and more loads and stores are in flight.  (64 x 256 tiles
            // hold 112 KB, one per CU, and 64 x 128 tiles in place of 256 x
            // 256 ones were measured slower.)  Same per-element product order:
            // bit-identical.
            int kmax = 0;
            for (int i = 0; i < n; ++i) kmax = std::max(kmax, g.p[i].K);
            if (bn == 64 || (kmax <= 128 && bn <= 160)) {
                int small_max = 0;
                for (int i = 0; i < n; ++i) {
                    g.total[i] = ((g.p[i].M + 63) / 64) * g.tiles_n[i];
                    small_max = std::max(small_max, g.total[i]);
                }
                const int px = (small_max + kXcds - 1) / kXcds;
                const dim3 sgrid(px * kXcds, n);
                switch (bn) {
                    case 160: launch_x3p<160, 1>(g, px, staged, sgrid, stream); break;
                    case 128: launch_x3p<128, 1>(g, px, staged, sgrid, stream); break;
                    default: launch_x3p<64, 1>(g, px, staged, sgrid, stream); break;
                }
                return hipGetLastError();
            }
            switch (bn) {
                case 256: launch_x3p<256>(g, per_xcd, staged, grid, stream); break;
                case 160: launch_x3p<160>(g, per_xcd, staged, grid, stream); break;
                case 128: launch_x3p<128>(g, per_xcd, staged, grid, stream); break;
                default: launch_x3p<64>(g, per_xcd, staged, grid, stream); break;
            }
            return hipGetLastError();
        }
        if (use_x3(g, n)) {
            switch (bn) {
                case 256: launch_big<256, false, true>(g, per_xcd, staged, grid, stream); break;
                case 160: launch_big<160, false, true>(g, per_xcd, staged, grid, stream); break;
                case 128: launch_big<128, false, true>(g, per_xcd, staged, grid, stream); break;
                default: launch_big<64, false, true>(g, per_xcd, staged, grid, stream); break;
            }
            return hipGetLastError();
        }
        switch (bn) {
            case 256: launch_big<256, false>(g, per_xcd, staged, grid, stream); break;
            case 160: launch_big<160, false>(g, per_xcd, staged, grid, stream); break;
            case 128: launch_big<128, false>(g, per_xcd, staged, grid, stream); break;
            default: launch_big<64, false>(g, per_xcd, staged, grid, stream); break;
        }
        return hipGetLastError();
    }
    const int per_xcd = (max_total + kXcds - 1) / kXcds;
    hipLaunchKernelGGL(gemm_f32_kernel, dim3(per_xcd * kXcds, n), dim3(kThreads), 0, stream, g, per_xcd);
    return hipGetLastError();
}

size_t gemm_workspace_floats(int N, int K) { return (size_t)skinny_splits(N, K) * 64 * N; }

size_t x3_planes_elems(int N, int K) {
    if (N <= 0 || K <= 0 || N % 16 != 0 || K % 32 != 0) return 0;
    return (size_t)N * K * 3;
}

hipError_t launch_x3_split_planes(const float *W, int ldw, int N, int K, uint16_t *planes, hipStream_t stream) {
    if (!x3_planes_elems(N, K) || ldw < K || ldw % 4 != 0 || !W || !planes ||
        (reinterpret_cast<uintptr_t>(W) & 15) != 0 || (reinterpret_cast<uintptr_t>(planes) & 15) != 0)
        return hipErrorInvalidValue;
    const long long items = (long long)N * (K / 8);
    hipLaunchKernelGGL(x3_split_planes_kernel, dim3((unsigned)((items + 255) / 256)), dim3(256), 0, stream, W, ldw, N,
                       K, planes);
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

extern "C" size_t yuf_x3_planes_elems(int N, int K) { return yuf::x3_planes_elems(N, K); }

extern "C" int yuf_x3_split_planes(int N, int K, const float *W, uint16_t *planes, void *stream) {
    using namespace yuf;
    if (!x3_planes_elems(N, K)) return fail(YUF_ERR_INVALID, "x3_split_planes: needs N % 16 == 0, K % 32 == 0");
    if (!W || !planes) return fail(YUF_ERR_INVALID, "x3_split_planes: null pointer");
    if ((reinterpret_cast<uintptr_t>(W) & 15) != 0 || (reinterpret_cast<uintptr_t>(planes) & 15) != 0)
        return fail(YUF_ERR_INVALID, "x3_split_planes: W and planes must be 16-byte aligned");
    hipError_t err = launch_x3_split_planes(W, K, N, K, planes, static_cast<hipStream_t>(stream));
    if (err != hipSuccess) return fail(YUF_ERR_HIP, std::string("x3_split_planes launch: ") + hipGetErrorString(err));
    return YUF_OK;
}

extern "C" int yuf_linear_f32_planes(int M, int N, int K, const float *A, const float *W, const uint16_t *Wp,
                                     const float *bias, int act, const float *residual, float *C, void *stream) {
    using namespace yuf;
    if (M < 0 || N < 0 || K < 1) return fail(YUF_ERR_INVALID, "linear_planes: bad sizes");
    if (act < ACT_NONE || act > ACT_SIGMOID) return fail(YUF_ERR_INVALID, "linear_planes: bad activation");
    if (M > 0 && N > 0 && (!A || !W || !Wp || !C)) return fail(YUF_ERR_INVALID, "linear_planes: null pointer");
    if (M > 0 && N > 0 && !x3_planes_elems(N, K))
        return fail(YUF_ERR_INVALID, "linear_planes: planes need N % 16 == 0, K % 32 == 0");
    GemmParams p;
    p.M = M; p.N = N; p.K = K; p.A = A; p.lda = K; p.W = W; p.ldw = K; p.C = C; p.ldc = N;
    p.bias = bias; p.act = act; p.residual = residual; p.ldr = N;
    if (M > 64) p.Wp = Wp;
    hipError_t err = launch_gemm(p, static_cast<hipStream_t>(stream));
    if (err != hipSuccess) return fail(YUF_ERR_HIP, std::string("linear_planes launch: ") + hipGetErrorString(err));
    return YUF_OK;
}

extern "C" int yuf_ln_linear_f32(int M, int N, int K, const float *A, const float *gamma, const float *beta,
                                 const float *gate, const float *W, const float *bias, const float *residual, float *C,
                                 void *stream) {
    using namespace yuf;
    if (M < 1 || M > 64 || N < 0 || K < 4 || K % 4 != 0 || K > 1024)
        return fail(YUF_ERR_INVALID, "ln_linear: needs 1 <= M <= 64, K % 4 == 0, 4 <= K <= 1024");
    if (N > 0 && (!A || !gamma || !beta || !W || !C)) return fail(YUF_ERR_INVALID, "ln_linear: null pointer");
    GemmParams p;
    p.M = M; p.N = N; p.K = K; p.A = A; p.lda = K; p.W = W; p.ldw = K; p.C = C; p.ldc = N;
    p.bias = bias; p.residual = residual; p.ldr = N;
    p.ln_gamma = gamma; p.ln_beta = beta; p.a_gate = gate; p.ldg = gate ? K : 0;
    hipError_t err = launch_gemm(p, static_cast<hipStream_t>(stream));
    if (err != hipSuccess) return fail(YUF_ERR_HIP, std::string("ln_linear launch: ") + hipGetErrorString(err));
    return YUF_OK;
}

extern "C" int yuf_linear_bf16w(int M, int N, int K, const float *A, const uint16_t *W, const float *bias, int act,
                                const float *residual, float *C, void *stream) {
    using namespace yuf;
    if (M < 0 || N < 0 || K < 8 || K % 8 != 0) return fail(YUF_ERR_INVALID, "linear_bf16w: needs K % 8 == 0, K >= 8");
    if (act < ACT_NONE || act > ACT_SIGMOID) return fail(YUF_ERR_INVALID, "linear_bf16w: bad activation");
    if (M > 0 && N > 0 && (!A || !W || !C)) return fail(YUF_ERR_INVALID, "linear_bf16w: null pointer");
    if (M > 64 && N % 64 != 0 && N % 160 != 0)
        return fail(YUF_ERR_INVALID, "linear_bf16w: M > 64 needs N % 64 == 0 or N % 160 == 0");
    GemmParams p;
    p.M = M; p.N = N; p.K = K; p.A = A; p.lda = K; p.Wh = W; p.ldw = K; p.C = C; p.ldc = N;
    p.bias = bias; p.act = act; p.residual = residual; p.ldr = N;
    hipError_t err = launch_gemm(p, static_cast<hipStream_t>(stream));
    if (err != hipSuccess) return fail(YUF_ERR_HIP, std::string("linear_bf16w launch: ") + hipGetErrorString(err));
    return YUF_OK;
}

extern "C" int yuf_ln_linear_bf16w(int M, int N, int K, const float *A, const float *gamma, const float *beta,
                                   const float *gate, const uint16_t *W, const float *bias, const float *residual,
                                   float *C, void *stream) {
    using namespace yuf;
    if (M < 1 || M > 64 || N < 0 || K < 8 || K % 8 != 0 || K > 1024)
        return fail(YUF_ERR_INVALID, "ln_linear_bf16w: needs 1 <= M <= 64, K % 8 == 0, 8 <= K <= 1024");
    if (N > 0 && (!A || !gamma || !beta || !W || !C)) return fail(YUF_ERR_INVALID, "ln_linear_bf16w: null pointer");
    GemmParams p;
    p.M = M; p.N = N; p.K = K; p.A = A; p.lda = K; p.Wh = W; p.ldw = K; p.C = C; p.ldc = N;
    p.bias = bias; p.residual = residual; p.ldr = N;
    p.ln_gamma = gamma; p.ln_beta = beta; p.a_gate = gate; p.ldg = gate ? K : 0;
    hipError_t err = launch_gemm(p, static_cast<hipStream_t>(stream));
    if (err != hipSuccess) return fail(YUF_ERR_HIP, std::string("ln_linear_bf16w launch: ") + hipGetErrorString(err));
    return YUF_OK;
}
