// WKV-7 scan in chunk-parallel form on the fp32 matrix cores (gfx950 MFMA).
//
// Same recurrence as wkv7.hip (yufmusicgen/model.py:145-165): per (b, h)
//     S_t = S_{t-1} (diag(d_t) + a_t b_t^T) + v_t k_t^T,   y_t = S_t r_t,
// with d = exp(-e^{-0.5} sigmoid(w_raw)) in (0.545, 1].
//
// Chunk algebra (16 tokens, t = 0..15 inside the chunk; g_t = prod_{s<=t} d_s
// per key column, g_{-1} = 1; S0 = state at the chunk start):
//     A~_t = a_t g_{t-1},  R~_t = r_t g_t,  B^_t = b_t / g_t,  K^_t = k_t / g_t
//     Gab = strict(A~ B^T),  P = strict(A~ K^T),  Qb = incl(R~ B^T),  Qk = incl(R~ K^T)
//     U  = (I - Gab)^{-1} (A~ S0^T + P V)        rows u_t = S_{t-1} a_t  (the "sa" vectors)
//     Y  = R~ S0^T + Qb U + Qk V                 rows y_t
//     S_16^T = diag(g_15) (S0^T + B^^T U + K^^T V)
// (U, Y as [token][value row]).  The decays enter only as sequential running
// products in fp32 (4-token runs chained by their end products), so ratios g_t / g_s keep
// their shared prefix exactly; a tree-shaped scan costs ~25% more error.
// d >= 0.545 keeps 1/g below 2^14 inside a chunk.  An fp32 emulation of this
// sequence stays within 0.65 of the 1e-4/1e-5 tolerance of the fp64
// recurrence at C2 size.
//
// Work split for one head (one workgroup), NB = ceil(N/16) 16-row blocks:
//   NB waves       consumers: wave q owns S^T[:, 16q..16q+15] as NB 16x16
//                  accumulator tiles and runs the S-dependent products above,
//                  16 NB + 16 v_mfma_f32_16x16x4f32 per chunk;
//   one wave       stage B1: the four 16x16 Gram matrices (MFMA; B^ and K^
//                  read from stage A's [key][token] tiles);
//   NB waves       stage A: loads r, w, k, a, b, v (16-byte runs along the
//                  columns; all but v transposed through LDS), decays, running
//                  products (quarters joined by gfx950 row swaps) and the
//                  scaled operands -> LDS (16 columns each);
//                  model path: kappa = normalize(k k_k), a = -kappa,
//                  b = kappa alpha, k^ = k (1 + (alpha - 1) k_a) first;
//   one wave       stage B2: (I - Gab)^{-1} by forward substitution, and in
//                  the model path the per-token key norms of a later chunk.
// Iteration i runs B2's norms on chunk i+4, A on i+3, B1 on i+2, B2's inverse
// on i+1 and the consumers on chunk i, with one workgroup barrier per
// iteration and ring buffers in LDS.  The consumers apply the chunk decay to
// the state last:  S^T <- diag(g_15) (S0^T + B^^T U + K^^T V).
// Global loads run two chunks ahead of their use in two register sets (loops
// unrolled by two), so an HBM round trip (~1 us under load) spans two
// iterations.  Only stage A and B2 load; the consumers read v from the ring
// and only store, so no wave waits on a load issued after its own stores, and
// the order of loads before each loop matches the loop's steady state (the
// compiler's wait counts then allow the newer register set to stay in flight).
//
// MFMA operand layouts (16x16x4 f32; lane l, g = l / 16, li = l % 16):
//   A operand A[m = li][k = g], B operand B[k = g][n = li],
//   accumulator register r holds D[m = 4 g + r][n = li].
// A product whose B operand is a previous accumulator uses k-step r to mean
// rows {4 g + r}: register r of that accumulator is the B operand as is, and
// the matching A operand is one ds_read_b128 of 4 consecutive k per lane.
#include "common.h"
#include "kernels.h"

#include <cstdlib>
#include <cstring>

namespace yuf {
namespace {

typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kC = 16;       // tokens per chunk
constexpr int kWave = 64;
constexpr int kXcds = 8;
constexpr int kST = 20;      // row stride of 16-wide LDS tiles (floats, 16-byte aligned rows)

__device__ __forceinline__ floatx4 mfma(float a, float b, floatx4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ floatx4 ld4(const float *p) { return *reinterpret_cast<const floatx4 *>(p); }

typedef float floatx2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ floatx2 ld2(const float *p) { return *reinterpret_cast<const floatx2 *>(p); }

__device__ __forceinline__ floatx4 buf_load4(__amdgpu_buffer_rsrc_t rsrc, uint32_t byte_offset) {
    return __builtin_bit_cast(floatx4, __builtin_amdgcn_raw_buffer_load_b128(rsrc, byte_offset, 0, 0));
}

__device__ __forceinline__ void buf_store4(floatx4 v, __amdgpu_buffer_rsrc_t rsrc, uint32_t byte_offset) {
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), rsrc, byte_offset, 0, 0);
}

template <int NB, bool SPLIT>
struct Lds {
    // Ring depths: a split workgroup's Y wave reads chunk c - 1's ring entries
    // while stage A writes chunk c + 3 and stage B1 chunk c + 2.
    static constexpr int kRA = SPLIT ? 5 : 4, kRG = SPLIT ? 4 : 3;
    static constexpr int NP = 16 * NB;        // padded head size
    static constexpr int SA = NP + 4;         // row stride of [token][column] tiles
    // Ring A (4 chunks in flight): A~, R~ [16][SA]; B^^T, K^^T [NP][kST]; g_15 [NP];
    // V^T [NP][kST] (value row, token).
    static constexpr int oAs = 0, oRs = 16 * SA, oBhT = 32 * SA, oKhT = oBhT + NP * kST, oGl = oKhT + NP * kST;
    static constexpr int oV = oGl + NP;
    static constexpr int kSlotA = oV + NP * kST;
    // Ring G (3): Gab^T [s][t], P, Qb, Qk [t][s], all [16][kST].
    static constexpr int oGabT = 0, oP = 16 * kST, oQb = 32 * kST, oQk = 48 * kST, kSlotG = 64 * kST;
    // Ring T (2): (I - Gab)^{-1} [16][kST].
    static constexpr int kSlotT = 16 * kST;
    // Ring N (2): per-token 1 / max(|k k_k|, 1e-12) (model path).
    static constexpr int kSlotN = 16;
    // Stage A transpose (one region per stage-A wave): up to 5 inputs x
    // [16 tokens][16 columns], rows padded to kST floats.
    static constexpr int kSlotR = 5 * 16 * kST;
    // Split: consumer -> Y wave exchange, [chunk parity][value tile][vector k]
    // [lane] floatx4: k < NB the chunk-start state S0^T rows, k = NB the U tile.
    static constexpr int kSlotX = SPLIT ? 2 * 2 * 4 * 64 * 4 : 0;
    static constexpr int kFloats =
        kRA * kSlotA + kRG * kSlotG + 2 * kSlotT + 2 * kSlotN + NB * kSlotR + kSlotX;
};

// Wave roles.  Waves w and w + 4 of a workgroup share a SIMD, and a wave
// issuing MFMAs halves the VALU issue rate of its SIMD neighbour, so each
// MFMA-heavy wave (consumer or B1) is paired with one VALU-heavy wave
// (stage A or B2): NB = 3 gives cons0+A0, cons1+A1, B1+B2, cons2+A2.
enum : int { kRoleB1 = 8, kRoleB2 = 9, kRoleIdle = 10, kRoleY = 11, kRoleA = 12 };
template <int NB> struct Roles {
    static constexpr int kWaves = 2 * NB + 2;
    __device__ static int of(int w) {
        constexpr int A = kRoleA;
        if constexpr (NB == 1) { constexpr int r[] = {0, kRoleB1, A, kRoleB2}; return r[w]; }
        if constexpr (NB == 2) { constexpr int r[] = {0, 1, kRoleB1, A, A + 1, kRoleB2}; return r[w]; }
        if constexpr (NB == 3) { constexpr int r[] = {0, 1, kRoleB1, 2, A, A + 1, kRoleB2, A + 2}; return r[w]; }
        constexpr int r[] = {0, 1, 2, 3, A, A + 1, A + 2, A + 3, kRoleB1, kRoleB2};
        return r[w];
    }
};
// Split heads (two workgroups per head, each with the consumers of its own
// value tiles and the whole key-space pipeline, NB <= 3).  On gfx950 an fp32
// MFMA stream and the VALU / LDS work of any wave on the same SIMD run one
// after the other (measured: no overlap), so the work is spread for equal
// per-SIMD sums: the consumers keep only the state chain (X, U, the state
// update) and hand the chunk-start state and U to a Y wave that forms the
// outputs one chunk later.  NB = 3: cons0 + A0, cons1 + A1, B1 + B2, Y + A2.
// Consumer roles past the workgroup's tile count idle (they keep the barrier
// count only).
template <int NB> struct SplitRoles {
    static constexpr int kWaves = NB == 2 ? 6 : 8;
    __device__ static int of(int w) {
        constexpr int A = kRoleA;
        if constexpr (NB == 2) { constexpr int r[] = {0, kRoleB1, kRoleY, A, A + 1, kRoleB2}; return r[w]; }
        constexpr int r[] = {0, 1, kRoleB1, kRoleY, A, A + 1, kRoleB2, A + 2};
        return r[w];
    }
};
template <int NB, bool SPLIT> struct RoleMap : Roles<NB> {};
template <int NB> struct RoleMap<NB, true> : SplitRoles<NB> {
    static_assert(NB == 2 || NB == 3, "split heads need NB in {2, 3}");
};

// SPLIT: two workgroups per head; the first owns value tiles [0, (NB + 1) / 2),
// the second the rest.
// HALF (N % 16 == 8): the last key tile holds 8 keys.  Its accumulator row
// m = 4 g + r stands for key 16 (NB - 1) + 8 (r >> 1) + 2 g + (r & 1), so the
// real keys sit in registers r = 0, 1 of every lane group, and every product
// over the keys takes k-steps r = 0, 1 only on that tile (k-step r of lane
// group g: key 2 g + r of the tile) instead of four k-steps of which half
// would multiply zeros.
template <int NB, bool PREP, bool SPLIT, bool HALF>
__global__ void __launch_bounds__((RoleMap<NB, SPLIT>::kWaves) * kWave)
    wkv7_chunk_kernel(WkvParams p, int N, int units, int per_xcd) {
    using Ly = Lds<NB, SPLIT>;
    constexpr int NP = Ly::NP, SA = Ly::SA, kRA = Ly::kRA, kRG = Ly::kRG;
    constexpr int kExtra = SPLIT ? 1 : 0;  // iterations after the consumers' last chunk (the Y wave's)
    __shared__ __attribute__((aligned(16))) float lds[Ly::kFloats];
    float *ringA = lds;
    float *ringG = ringA + kRA * Ly::kSlotA;
    float *ringT = ringG + kRG * Ly::kSlotG;
    float *ringN = ringT + 2 * Ly::kSlotT;
    float *stageR = ringN + 2 * Ly::kSlotN;
    floatx4 *xch = reinterpret_cast<floatx4 *>(stageR + NB * Ly::kSlotR);  // split only

    // XCD-aware unit index: consecutive units (the two halves of a head, then
    // consecutive heads of a batch row) share an XCD's L2.
    const int unit = (blockIdx.x % kXcds) * per_xcd + blockIdx.x / kXcds;
    if (unit >= units) return;  // uniform over the workgroup
    const int flat = SPLIT ? unit >> 1 : unit, part = SPLIT ? unit & 1 : 0;
    constexpr int kNv0 = SPLIT ? (NB + 1) / 2 : NB;  // value tiles of the first workgroup
    const int vb0 = part ? kNv0 : 0, nv = part ? NB - kNv0 : kNv0;
    const int bb = flat / p.H, h = flat - bb * p.H;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    int role = RoleMap<NB, SPLIT>::of(wave);
    if (role < NB && role >= nv) role = kRoleIdle;
    const int g = lane >> 4, li = lane & 15;
    const int T = p.T, HN = p.H * N;
    constexpr int kLast = NB - 1;
    auto half_tile = [](int jb) { return HALF && jb == kLast; };
    auto ksteps = [&](int jb) { return half_tile(jb) ? 2 : 4; };
    // Key of accumulator row m of tile jb.
    auto rowkey = [&](int jb, int m) {
        return 16 * jb + (half_tile(jb) ? ((m & 2) << 2) + 2 * (m >> 2) + (m & 1) : m);
    };
    // The k-step values of lane group g over tile jb of a [token][key] row.
    auto ldk = [&](const float *row, int jb) -> floatx4 {
        if (half_tile(jb)) {
            const floatx2 v = ld2(row + 16 * jb + 2 * g);
            return floatx4{v[0], v[1], 0.0f, 0.0f};
        }
        return ld4(row + 16 * jb + 4 * g);
    };
    // g_15 of the four accumulator rows of lane group g in tile jb.
    auto ldg = [&](const float *gl, int jb) -> floatx4 {
        if (half_tile(jb)) {
            const floatx2 a = ld2(gl + 16 * jb + 2 * g), b = ld2(gl + 16 * jb + 8 + 2 * g);
            return floatx4{a[0], a[1], b[0], b[1]};
        }
        return ld4(gl + 16 * jb + 4 * g);
    };
    const int n_chunks = (T + kC - 1) / kC;
    // Per-(b, h) token-major views: element (t, c) at t * HN + c.  Tokens past
    // T fall outside the descriptor range and read as 0.
    const size_t tok_base = ((size_t)bb * T * p.H + h) * N;
    const uint32_t tok_bytes = T > 0 ? (uint32_t)(((size_t)(T - 1) * HN + N) * 4) : 0u;
    const int chunk_bytes = kC * HN * 4;
    const int slot = p.slot ? p.slot[bb] : bb;
    const size_t state_off = ((size_t)slot * p.H + h) * N * N;

    if (role == kRoleIdle) {
        for (int it = -4; it < n_chunks + kExtra; ++it) lds_barrier();
    } else if (SPLIT && role == kRoleY) {
        // ------------------------------------------------------------ Y wave
        // Chunk c = it - 1 of each owned value tile: Y = R~ S0^T + Qb U + Qk V
        // from the consumer's exchange (S0^T, U), then the y rows.
        const auto ry = make_rsrc(p.y + tok_base, tok_bytes);
        for (int it = -4; it < n_chunks + kExtra; ++it) {
            const int c = it - 1;
            if (c >= 0) {
                const float *sA = ringA + (c % kRA) * Ly::kSlotA;
                const float *sG = ringG + (c % kRG) * Ly::kSlotG;
                const floatx4 *xc = xch + (c & 1) * 2 * 4 * 64;
                for (int tl = 0; tl < nv; ++tl) {
                    const int i = 16 * (vb0 + tl) + li;
                    const floatx4 *xt = xc + tl * 4 * 64;
                    const floatx4 v = ld4(sA + Ly::oV + i * kST + 4 * g);
                    const floatx4 U = xt[NB * 64 + lane];
                    floatx4 Y0 = {0.f, 0.f, 0.f, 0.f}, Y1 = Y0;
#pragma unroll
                    for (int jb = 0; jb < NB; ++jb) {
                        const floatx4 r4 = ldk(sA + Ly::oRs + li * SA, jb);
                        const floatx4 s0 = xt[jb * 64 + lane];
#pragma unroll
                        for (int r = 0; r < 4; ++r) {
                            if (r >= ksteps(jb)) break;
                            if (r & 1) Y1 = mfma(r4[r], s0[r], Y1);
                            else Y0 = mfma(r4[r], s0[r], Y0);
                        }
                    }
                    const floatx4 qk4 = ld4(sG + Ly::oQk + li * kST + 4 * g);
                    const floatx4 qb4 = ld4(sG + Ly::oQb + li * kST + 4 * g);
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        Y0 = mfma(qk4[r], v[r], Y0);
                        Y1 = mfma(qb4[r], U[r], Y1);
                    }
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const int t = c * kC + 4 * g + r;
                        buf_store(Y0[r] + Y1[r], ry, (t < T && i < N) ? (uint32_t)(t * HN + i) * 4u : kBufferOob);
                    }
                }
            }
            lds_barrier();
        }
    } else if (role < NB) {
        // ------------------------------------------------------------ consumer
        const int q = vb0 + role;
        const int i = 16 * q + li;  // value row owned by this lane's column of the tiles
        floatx4 S[NB];
        {
            const auto rs = make_rsrc(p.state_in ? p.state_in + state_off : nullptr,
                                      p.state_in ? (uint32_t)(N * N * 4) : 0u);
#pragma unroll
            for (int jb = 0; jb < NB; ++jb) {
                if (half_tile(jb)) {
                    const int j0 = 16 * jb + 2 * g;  // rows r = 0, 1; rows 2, 3 are padding keys
                    S[jb] = floatx4{buf_load(rs, i < N ? (uint32_t)(i * N + j0) * 4u : kBufferOob),
                                    buf_load(rs, i < N ? (uint32_t)(i * N + j0 + 1) * 4u : kBufferOob), 0.0f, 0.0f};
                    continue;
                }
                const int j0 = 16 * jb + 4 * g;
                S[jb] = buf_load4(rs, (i < N && j0 < N) ? (uint32_t)(i * N + j0) * 4u : kBufferOob);
            }
        }
        const auto ry = make_rsrc(p.y + tok_base, tok_bytes);
        wait_vmem();
        for (int it = -4; it < n_chunks + kExtra; ++it) {
            if (SPLIT && it >= 0 && it < n_chunks) {
                // The state chain only: X = A~ S0^T + P V, U = (I - Gab)^{-1} X,
                // S^T <- diag(g_15) (S^T + B^^T U + K^^T V); S0^T and U go to the Y wave.
                const int c = it;
                const float *sA = ringA + (c % kRA) * Ly::kSlotA;
                const float *sG = ringG + (c % kRG) * Ly::kSlotG;
                const float *sT = ringT + (c & 1) * Ly::kSlotT;
                floatx4 *xt = xch + ((c & 1) * 2 + role) * 4 * 64;
                const floatx4 v = ld4(sA + Ly::oV + i * kST + 4 * g);  // V[4 g + r][i]
                floatx4 X0 = {0.f, 0.f, 0.f, 0.f}, X1 = X0;
#pragma unroll
                for (int jb = 0; jb < NB; ++jb) {
                    const floatx4 a4 = ldk(sA + Ly::oAs + li * SA, jb);
                    xt[jb * 64 + lane] = S[jb];
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        if (r >= ksteps(jb)) break;
                        if (r & 1) X1 = mfma(a4[r], S[jb][r], X1);
                        else X0 = mfma(a4[r], S[jb][r], X0);
                    }
                }
                const floatx4 p4 = ld4(sG + Ly::oP + li * kST + 4 * g);
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    if (r & 1) X1 = mfma(p4[r], v[r], X1);
                    else X0 = mfma(p4[r], v[r], X0);
                }
                const floatx4 X = X0 + X1;
                const floatx4 ti4 = ld4(sT + li * kST + 4 * g);
                floatx4 U = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int r = 0; r < 4; ++r) U = mfma(ti4[r], X[r], U);
                xt[NB * 64 + lane] = U;
#pragma unroll
                for (int jb = 0; jb < NB; ++jb) {
                    const floatx4 gl4 = ldg(sA + Ly::oGl, jb);
                    const int brow = rowkey(jb, li);
                    const floatx4 bh4 = ld4(sA + Ly::oBhT + brow * kST + 4 * g);
                    const floatx4 kh4 = ld4(sA + Ly::oKhT + brow * kST + 4 * g);
                    floatx4 acc = S[jb];
#pragma unroll
                    for (int r = 0; r < 4; ++r) acc = mfma(bh4[r], U[r], acc);
#pragma unroll
                    for (int r = 0; r < 4; ++r) acc = mfma(kh4[r], v[r], acc);
                    S[jb] = acc * gl4;
                }
            } else if (!SPLIT && it >= 0) {
                const int c = it;
                const float *sA = ringA + (c % kRA) * Ly::kSlotA;
                const float *sG = ringG + (c % kRG) * Ly::kSlotG;
                const float *sT = ringT + (c & 1) * Ly::kSlotT;
                const floatx4 v = ld4(sA + Ly::oV + i * kST + 4 * g);  // V[4 g + r][i]
                floatx4 X = {0.f, 0.f, 0.f, 0.f}, Y = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int jb = 0; jb < NB; ++jb) {
                    const floatx4 a4 = ldk(sA + Ly::oAs + li * SA, jb);
                    const floatx4 r4 = ldk(sA + Ly::oRs + li * SA, jb);
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        if (r >= ksteps(jb)) break;
                        X = mfma(a4[r], S[jb][r], X);
                        Y = mfma(r4[r], S[jb][r], Y);
                    }
                }
                const floatx4 p4 = ld4(sG + Ly::oP + li * kST + 4 * g);
                const floatx4 qk4 = ld4(sG + Ly::oQk + li * kST + 4 * g);
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    X = mfma(p4[r], v[r], X);
                    Y = mfma(qk4[r], v[r], Y);
                }
                const floatx4 ti4 = ld4(sT + li * kST + 4 * g);
                floatx4 U = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int r = 0; r < 4; ++r) U = mfma(ti4[r], X[r], U);
                const floatx4 qb4 = ld4(sG + Ly::oQb + li * kST + 4 * g);
#pragma unroll
                for (int r = 0; r < 4; ++r) Y = mfma(qb4[r], U[r], Y);
                // S^T <- diag(g_15) (S^T + B^^T U + K^^T V)
#pragma unroll
                for (int jb = 0; jb < NB; ++jb) {
                    const floatx4 gl4 = ldg(sA + Ly::oGl, jb);
                    const int brow = rowkey(jb, li);
                    const floatx4 bh4 = ld4(sA + Ly::oBhT + brow * kST + 4 * g);
                    const floatx4 kh4 = ld4(sA + Ly::oKhT + brow * kST + 4 * g);
                    floatx4 acc = S[jb];
#pragma unroll
                    for (int r = 0; r < 4; ++r) acc = mfma(bh4[r], U[r], acc);
#pragma unroll
                    for (int r = 0; r < 4; ++r) acc = mfma(kh4[r], v[r], acc);
                    S[jb] = acc * gl4;
                }
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int t = c * kC + 4 * g + r;
                    buf_store(Y[r], ry, (t < T && i < N) ? (uint32_t)(t * HN + i) * 4u : kBufferOob);
                }
            }
            lds_barrier();
        }
        if (p.state_out) {
            const auto rs = make_rsrc(p.state_out + state_off, (uint32_t)(N * N * 4));
#pragma unroll
            for (int jb = 0; jb < NB; ++jb) {
                if (half_tile(jb)) {
                    const int j0 = 16 * jb + 2 * g;
                    buf_store(S[jb][0], rs, i < N ? (uint32_t)(i * N + j0) * 4u : kBufferOob);
                    buf_store(S[jb][1], rs, i < N ? (uint32_t)(i * N + j0 + 1) * 4u : kBufferOob);
                    continue;
                }
                const int j0 = 16 * jb + 4 * g;
                buf_store4(S[jb], rs, (i < N && j0 < N) ? (uint32_t)(i * N + j0) * 4u : kBufferOob);
            }
        }
    } else if (role >= kRoleA) {
        // ------------------------------------------------------------- stage A
        // NB waves, 16 columns each; lane = (token quarter qg, column): tokens
        // 4 qg .. 4 qg + 3 of column j.  Decay products run sequentially over
        // the 4 tokens; quarters are chained by a 2-step scan over lane groups.
        const int qg = lane >> 4;
        const int j = (role - kRoleA) * 16 + li;
        // Loads: lane = (token li, 4-column group qg) reads 16 bytes per input,
        // and the tile is transposed through LDS into the compute layout.
        const int lc0 = (role - kRoleA) * 16 + 4 * qg;
        const uint32_t voff = lc0 < N ? (uint32_t)((li * HN + lc0) * 4) : kBufferOob;
        float *stR = stageR + (role - kRoleA) * Ly::kSlotR;
        constexpr int kT = PREP ? 4 : 5;  // transposed inputs r, w, k, a(lpha) [, b]
        constexpr int kIn = kT + 1;       // + v (input kT), stored untransposed
        const float *src[6] = {p.r, p.w, p.k, p.a, PREP ? p.v : p.b, p.v};
        __amdgpu_buffer_rsrc_t rs[kIn];
#pragma unroll
        for (int x = 0; x < kIn; ++x) rs[x] = make_rsrc(src[x] + tok_base, tok_bytes);
        float kk_w = 0.0f, ka_w = 0.0f;
        if constexpr (PREP) {
            const bool col_ok = j < N;
            kk_w = col_ok ? p.k_k[h * N + j] : 0.0f;
            ka_w = col_ok ? p.k_a[h * N + j] : 0.0f;
        }
        // Inputs of even and odd chunks (two register sets).
        floatx4 ld0[kIn], ld1[kIn];
        float raw[kT][4];
        auto load_chunk = [&](floatx4 (&ld)[kIn], int c) {
#pragma unroll
            for (int x = 0; x < kIn; ++x) ld[x] = buf_load4(rs[x], voff + c * chunk_bytes);
        };
        // ld (token li, columns 4 qg..) -> LDS -> raw (tokens 4 qg.., column li).
        auto transpose = [&](const floatx4 (&ld)[kIn]) {
#pragma unroll
            for (int x = 0; x < kT; ++x)
                *reinterpret_cast<floatx4 *>(stR + x * 16 * kST + li * kST + 4 * qg) = ld[x];
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
#pragma unroll
            for (int x = 0; x < kT; ++x)
#pragma unroll
                for (int tt = 0; tt < 4; ++tt) raw[x][tt] = stR[x * 16 * kST + (4 * qg + tt) * kST + li];
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
        };
        // Unconditional (a chunk past T reads zeros) and not interleaved (the
        // scheduling barrier): the compiler's wait counts at the loop head
        // follow the order of these loads.
        load_chunk(ld0, 0);
        __builtin_amdgcn_sched_barrier(0);
        load_chunk(ld1, 1);
        const int rowbase = 4 * qg * SA + j;  // LDS [token][column] index of (4 qg, j)
        // Chunk c (iteration c - 3); its set is reloaded with chunk c + 2.
        auto body = [&](int c, floatx4 (&ld)[kIn], bool load_next) {
            {
                float *sA = ringA + (c % kRA) * Ly::kSlotA;
                transpose(ld);
#pragma unroll
                for (int e = 0; e < 4; ++e) sA[Ly::oV + (lc0 + e) * kST + li] = ld[kT][e];
                if (load_next) load_chunk(ld, c + 2);
                const int nt = min(kC, T - c * kC);
                float av[4], bv[4], kv[4], rv[4], dv[4];
#pragma unroll
                for (int tt = 0; tt < 4; ++tt) {
                    rv[tt] = raw[0][tt];
                    // d = exp(-e^{-0.5} sigmoid(w)) = exp2(-e^{-0.5} log2(e) sigmoid(w)); padded tokens keep g.
                    const float sig = __builtin_amdgcn_rcpf(1.0f + __expf(-raw[1][tt]));
                    const float d = __builtin_amdgcn_exp2f(-0.8750387749f * sig);
                    dv[tt] = nt == kC || 4 * qg + tt < nt ? d : 1.0f;
                }
                if constexpr (PREP) {
                    const float *inv = ringN + (c & 1) * Ly::kSlotN + 4 * qg;
#pragma unroll
                    for (int tt = 0; tt < 4; ++tt) {
                        const float alpha = raw[3][tt];
                        const float kap = raw[2][tt] * kk_w * inv[tt];
                        av[tt] = -kap;
                        bv[tt] = kap * alpha;
                        kv[tt] = raw[2][tt] * (1.0f + (alpha - 1.0f) * ka_w);
                    }
                } else {
#pragma unroll
                    for (int tt = 0; tt < 4; ++tt) {
                        av[tt] = raw[3][tt];
                        bv[tt] = raw[4][tt];
                        kv[tt] = raw[2][tt];
                    }
                }
                float gl[4];
                {
                    float gacc = 1.0f;
#pragma unroll
                    for (int tt = 0; tt < 4; ++tt) {
                        gacc *= dv[tt];
                        gl[tt] = gacc;
                    }
                }
                // base = product of d over the earlier quarters (exclusive scan of
                // the quarter end products e_q over the four 16-lane rows), with
                // the gfx950 row swaps: P = {e0, e0, e2, e2}, Q = {e1, e1, e3, e3},
                // R = e0 e1 on every row.  (Run on every lane, outside any condition.)
                const float eq = gl[3];
                const auto sw16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(eq), __float_as_uint(eq), false, false);
                const float P = __uint_as_float(sw16[0]), Q = __uint_as_float(sw16[1]);
                const float m01 = P * Q;
                const auto sw32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(m01), __float_as_uint(m01), false, false);
                const float R = __uint_as_float(sw32[0]);
                const float base = qg == 0 ? 1.0f : qg == 1 ? P : qg == 2 ? R : R * P;
                float bh[4], kh[4];
                float *pAs = sA + Ly::oAs + rowbase, *pRs = sA + Ly::oRs + rowbase;
#pragma unroll
                for (int tt = 0; tt < 4; ++tt) {
                    const float gprev = tt == 0 ? base : base * gl[tt - 1];
                    const float gam = base * gl[tt];
                    const float ig = __builtin_amdgcn_rcpf(gam);
                    bh[tt] = bv[tt] * ig;
                    kh[tt] = kv[tt] * ig;
                    pAs[tt * SA] = av[tt] * gprev;
                    pRs[tt * SA] = rv[tt] * gam;
                }
                *reinterpret_cast<floatx4 *>(sA + Ly::oBhT + j * kST + 4 * qg) = floatx4{bh[0], bh[1], bh[2], bh[3]};
                *reinterpret_cast<floatx4 *>(sA + Ly::oKhT + j * kST + 4 * qg) = floatx4{kh[0], kh[1], kh[2], kh[3]};
                if (qg == 3) sA[Ly::oGl + j] = base * gl[3];
            }
            lds_barrier();
        };
        // Iteration -4 has no stage-A chunk.  The steady loop loads
        // unconditionally (the same issue order as before the loop: the even
        // set, then the odd one); the last chunks and the three iterations
        // after stage A's last chunk follow it.
        lds_barrier();
        int c = 0;
        for (; c + 3 < n_chunks; c += 2) {
            body(c, ld0, true);
            body(c + 1, ld1, true);
        }
        if (c < n_chunks) body(c, ld0, c + 2 < n_chunks);
        if (c + 1 < n_chunks) body(c + 1, ld1, false);
        if (c + 2 < n_chunks) body(c + 2, ld0, false);
        for (int k = 0; k < 3 + kExtra; ++k) lds_barrier();
    } else if (role == kRoleB1) {
        // ------------------------------------------------------------ stage B1
        for (int it = -4; it < n_chunks + kExtra; ++it) {
            const int c = it + 2;
            if (c >= 0 && c < n_chunks) {
                const float *sA = ringA + (c % kRA) * Ly::kSlotA;
                float *sG = ringG + (c % kRG) * Ly::kSlotG;
                floatx4 gab = {0.f, 0.f, 0.f, 0.f}, gp = gab, gqb = gab, gqk = gab;
#pragma unroll
                for (int jb = 0; jb < NB; ++jb) {
                    const floatx4 a4 = ldk(sA + Ly::oAs + li * SA, jb), r4 = ldk(sA + Ly::oRs + li * SA, jb);
                    // B^[s = li][key of k-step r] from the [key][token] tiles.
                    const int oT = (16 * jb + (half_tile(jb) ? 2 : 4) * g) * kST + li;
                    floatx4 b4 = {0.f, 0.f, 0.f, 0.f}, k4 = b4;
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        if (r >= ksteps(jb)) break;
                        b4[r] = sA[Ly::oBhT + oT + r * kST];
                        k4[r] = sA[Ly::oKhT + oT + r * kST];
                    }
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        if (r >= ksteps(jb)) break;
                        gab = mfma(a4[r], b4[r], gab);
                        gp = mfma(a4[r], k4[r], gp);
                        gqb = mfma(r4[r], b4[r], gqb);
                        gqk = mfma(r4[r], k4[r], gqk);
                    }
                }
                // Register r: row t = 4 g + r, column s = li.
                floatx4 gt;
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int t = 4 * g + r, o = t * kST + li;
                    gt[r] = li < t ? gab[r] : 0.0f;
                    sG[Ly::oP + o] = li < t ? gp[r] : 0.0f;
                    sG[Ly::oQb + o] = li <= t ? gqb[r] : 0.0f;
                    sG[Ly::oQk + o] = li <= t ? gqk[r] : 0.0f;
                }
                *reinterpret_cast<floatx4 *>(sG + Ly::oGabT + li * kST + 4 * g) = gt;  // Gab^T[s = li][t]
            }
            lds_barrier();
        }
    } else {
        // ------------------------------------------------------------ stage B2
        // (model path) per-token inverse key norms one iteration ahead of stage A:
        // lane = (token li, column group g + 4 m), partial sums folded over the
        // four lane groups.
        __amdgpu_buffer_rsrc_t rk = make_rsrc(p.k + tok_base, tok_bytes);
        floatx4 kkw[NB], kraw0[NB], kraw1[NB];  // k of even / odd chunks
        if constexpr (PREP) {
#pragma unroll
            for (int m = 0; m < NB; ++m) {
                const int j0 = 4 * (g + 4 * m);
#pragma unroll
                for (int e = 0; e < 4; ++e) kkw[m][e] = j0 < N ? p.k_k[h * N + j0 + e] : 0.0f;
            }
        }
        auto load_k = [&](floatx4 (&kraw)[NB], int c) {
#pragma unroll
            for (int m = 0; m < NB; ++m) {
                const int j0 = 4 * (g + 4 * m);
                const uint32_t off = j0 < N ? (uint32_t)((li * HN + j0) * 4) : kBufferOob;
                kraw[m] = __builtin_bit_cast(floatx4, __builtin_amdgcn_raw_buffer_load_b128(rk, off, c * chunk_bytes, 0));
            }
        };
        if constexpr (PREP) {  // unconditional and in order, as in stage A
            load_k(kraw0, 0);
            __builtin_amdgcn_sched_barrier(0);
            load_k(kraw1, 1);
        }
        auto step = [&](int it, floatx4 (&kraw)[NB], bool load_next) {
            if constexpr (PREP) {
                const int cn = it + 4;
                if (cn < n_chunks) {
                    float sq = 0.0f;
#pragma unroll
                    for (int m = 0; m < NB; ++m)
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            const float x = kraw[m][e] * kkw[m][e];
                            sq = fmaf(x, x, sq);
                        }
                    if (load_next) load_k(kraw, cn + 2);
                    // Sum over the four 16-lane rows with the gfx950 row swaps.
                    const auto p16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(sq), __float_as_uint(sq), false, false);
                    sq = __uint_as_float(p16[0]) + __uint_as_float(p16[1]);
                    const auto p32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(sq), __float_as_uint(sq), false, false);
                    sq = __uint_as_float(p32[0]) + __uint_as_float(p32[1]);
                    if (lane < kC) ringN[(cn & 1) * Ly::kSlotN + lane] = 1.0f / fmaxf(sqrtf(sq), 1e-12f);
                }
            }
            const int c = it + 1;
            if (c >= 0 && c < n_chunks) {
                const float *GT = ringG + (c % kRG) * Ly::kSlotG + Ly::oGabT;
                float *sT = ringT + (c & 1) * Ly::kSlotT;
                // Column `lane` (< 16) of (I - Gab)^{-1}, right-looking: once x_s is
                // final, x_t += Gab[t][s] x_s for every t > s.
                float x[kC];
#pragma unroll
                for (int t = 0; t < kC; ++t) x[t] = lane == t ? 1.0f : 0.0f;
#pragma unroll
                for (int s = 0; s < kC - 1; ++s) {
                    float col[kC];
#pragma unroll
                    for (int m = 0; m < 4; ++m) {
                        const floatx4 c4 = ld4(GT + s * kST + 4 * m);
                        col[4 * m] = c4[0]; col[4 * m + 1] = c4[1]; col[4 * m + 2] = c4[2]; col[4 * m + 3] = c4[3];
                    }
#pragma unroll
                    for (int t = s + 1; t < kC; ++t) x[t] = fmaf(col[t], x[s], x[t]);
                }
                if (lane < kC) {
#pragma unroll
                    for (int t = 0; t < kC; ++t) sT[t * kST + lane] = x[t];
                }
            }
            lds_barrier();
        };
        // Chunk cn = it + 4 is even for even it, so kraw0 (loaded first) is used
        // first; the steady loop loads unconditionally, the tail as needed.
        int it = -4;
        for (; it + 7 < n_chunks; it += 2) {
            step(it, kraw0, true);
            step(it + 1, kraw1, true);
        }
        for (; it < n_chunks; it += 2) {
            step(it, kraw0, it + 6 < n_chunks);
            if (it + 1 < n_chunks) step(it + 1, kraw1, it + 7 < n_chunks);
        }
        for (int k = 0; k < kExtra; ++k) lds_barrier();
    }
}

// Heads at or below this many per GPU are split over two workgroups each (the
// MI355X has 256 CUs; one workgroup per head would leave half of them idle).
constexpr int kSplitMaxHeads = 128;

template <int NB, bool SPLIT, bool HALF>
void launch_nb_form(const WkvParams &p, int N, bool prep, int units, int per_xcd, hipStream_t stream) {
    const dim3 grid(per_xcd * kXcds), block(RoleMap<NB, SPLIT>::kWaves * kWave);
    if (prep)
        hipLaunchKernelGGL((wkv7_chunk_kernel<NB, true, SPLIT, HALF>), grid, block, 0, stream, p, N, units, per_xcd);
    else
        hipLaunchKernelGGL((wkv7_chunk_kernel<NB, false, SPLIT, HALF>), grid, block, 0, stream, p, N, units, per_xcd);
}

// Half-padded last key tile (N % 16 == 8) unless YUF_WKV7_HALF=0.
bool half_tile_form(int N) {
    if (N % 16 != 8) return false;
    const char *e = std::getenv("YUF_WKV7_HALF");
    return !(e && std::strcmp(e, "0") == 0);
}

template <int NB, bool SPLIT>
hipError_t launch_nb_split(const WkvParams &p, int N, bool prep, hipStream_t stream) {
    const int heads = p.B * p.H, units = SPLIT ? 2 * heads : heads;
    const int per_xcd = (units + kXcds - 1) / kXcds;
    if (half_tile_form(N)) launch_nb_form<NB, SPLIT, true>(p, N, prep, units, per_xcd, stream);
    else launch_nb_form<NB, SPLIT, false>(p, N, prep, units, per_xcd, stream);
    return hipGetLastError();
}

bool split_heads(int heads) {
    if (const char *e = std::getenv("YUF_WKV7_SPLIT")) return std::strcmp(e, "0") != 0;
    return heads <= kSplitMaxHeads;
}

template <int NB>
hipError_t launch_nb(const WkvParams &p, int N, bool prep, hipStream_t stream) {
    if constexpr (NB == 2 || NB == 3) {
        if (split_heads(p.B * p.H)) return launch_nb_split<NB, true>(p, N, prep, stream);
    }
    return launch_nb_split<NB, false>(p, N, prep, stream);
}

}  // namespace

bool wkv7_chunk_supported(int N) { return N >= 4 && N <= 64 && N % 4 == 0; }

hipError_t launch_wkv7_chunked(const WkvParams &p, int N, bool prep, hipStream_t stream) {
    if (p.B <= 0 || p.H <= 0) return hipSuccess;
    if (!wkv7_chunk_supported(N)) return hipErrorInvalidValue;
    switch ((N + 15) / 16) {
        case 1: return launch_nb<1>(p, N, prep, stream);
        case 2: return launch_nb<2>(p, N, prep, stream);
        case 3: return launch_nb<3>(p, N, prep, stream);
        default: return launch_nb<4>(p, N, prep, stream);
    }
}

}  // namespace yuf
