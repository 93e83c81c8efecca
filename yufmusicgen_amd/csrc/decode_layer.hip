// One decode layer per launch, persistent over the XCDs of gfx950 (MI355X).
//
// The per-token layer of the reference's Vulkan graph (vulkan/src/compute/
// model.rs:425-757: LN0 -> mix -> r/k/v/w/a/g -> fused TimeMix recurrence
// (shaders/timemix_recurrence.glsl:26-89) -> LN(o) * g -> W_o (+res) -> LN1 ->
// ROSA linears -> rosa_update / rosa_read -> ROSA out (+res) -> LN2 -> FFN
// in/gate -> silu * gate -> FFN out (+res)), for many streams at once, as one
// kernel instead of eight dependent launches.
//
// The streams of a step are split into one group per XCD (at most kDlRows
// each).  A workgroup reads the XCD it runs on from the hardware (XCC_ID) and
// works only on that XCD's group, so every exchange between its workgroups
// stays in that XCD's L2:
//   - the workgroups of an XCD split each stage's work items (16-column
//     slices of a product, or one WKV head of four streams) statically by
//     their rank b / groups (the dispatcher deals workgroups to the XCDs
//     round-robin, so b / groups is unique within an XCD; every workgroup
//     registers its (XCD, rank) and one that finds its slot taken twice
//     flags an error);
//   - a stage ends at a barrier of its group: each workgroup adds the items it
//     finished to the stage's counter once its stores have completed, and
//     waits until the counter reaches the stage's item count (agent-scope
//     atomics; every wait gives up after kPollCap polls and flags an error,
//     so no launch can hang);
//   - values another workgroup wrote in this launch (activations, the
//     residual h) are read with device-scope loads (sc1): on MI355X plain and
//     sc0 loads of such values returned stale data from the CU's L1.
// Measured on MI355X: such a barrier costs about 1.0 us (about 4 us across
// the whole device).  Everything a stage needs that does not depend on the
// previous stage -- its first weight batch, LayerNorm parameters, the WKV
// state and head weights, the ROSA memory rows -- is loaded before the
// workgroup waits at the previous barrier, and weight batches stream through
// two register buffers, the next batch (of the same item or the next one)
// loading during the current one's MFMAs.
//
// Stages per group (rows m < M = the group's streams; MFMA tiles of 16 rows,
// rows >= M read as zero):
//   1 LN_t + token shift + r/k/v/w1/a1/g1 products  (3 d / 16 + 3 L / 16 items)
//   2 WKV step with the second low-rank stage       (H x ceil(M / 4) items)
//   3 LN_o(y) * g -> W_o, + h                       (d / 16)
//   4 LN_r(h) -> ROSA input | write | read, + bias  (3 D / 16)
//   5 ROSA step -> ROSA out, + h                    (d / 16)
//   6 LN_f(h) -> FFN in / gate, silu(in) * gate     (4 d / 16)
//   7 FFN out, + h                                  (d / 16)
// The new `previous` rows (stage 1's normed input) and ROSA memory rows
// (stage 5) are written by the rank-0 workgroup after the next barrier, when
// no workgroup can still read the old rows.
#include "common.h"
#include "kernels.h"

namespace yuf {
namespace {

typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256, kWaves = 4;
constexpr int kSc1 = 16;            // buffer-load cache policy: device scope (misses the CU's L1)
constexpr int kPollCap = 400000;    // barrier polls (~40 ms) before a wait gives up
constexpr int kCh = 10;             // k tiles per wave per weight batch
constexpr int kMaxPer = kDlMaxD / 64;  // row elements per lane in the LayerNorm staging

// LDS regions (floats).
constexpr int kLdA = 4 * kDlMaxD + 4;  // row stride of the widest staged A (FFN out)
constexpr int kRegA = kDlRows * kLdA;
constexpr int kLdX = kDlMaxD + 4;
constexpr int kRegX = kDlRows * kLdX;   // stage 1's normed rows (kept for the `previous` write)
constexpr int kRegM = kDlRows * 256;    // stage 5's new ROSA memory rows (kept for their write)
constexpr int kTile = 16 * 17;          // a 16 x 16 partial tile, padded rows
constexpr int kRegR = 2 * kWaves * kTile;
constexpr int kLp = 64 + 4;             // LDS row of a WKV head weight (L <= 64)

enum : int { kS1 = 0, kS2, kS3, kS4, kS5, kS6, kS7 };

__device__ __forceinline__ int atom_add(int *p, int v) {
    return __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ floatx4 lds4(const float *p) { return *reinterpret_cast<const floatx4 *>(p); }
__device__ __forceinline__ void sts4(float *p, floatx4 v) { *reinterpret_cast<floatx4 *>(p) = v; }
__device__ __forceinline__ floatx4 ldg4(const float *p) { return *reinterpret_cast<const floatx4 *>(p); }

__device__ __forceinline__ float ld_sc1(__amdgpu_buffer_rsrc_t r, uint32_t byte_off) {
    return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, byte_off, 0, kSc1));
}
__device__ __forceinline__ floatx4 ld4_sc1(__amdgpu_buffer_rsrc_t r, uint32_t byte_off) {
    return __builtin_bit_cast(floatx4, __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, kSc1));
}

// LDS ordering between the lanes of one wave.
__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Per-group activations: [3][R][d] r, k, v | [3][R][L] lw, la, lg | [R][d] y |
// [R][d] g | [R][3D] ROSA pre-activations | [R][4d] FFN hidden.
struct GroupOff {
    size_t rkv, lr, y, g, pre, hid;
};
__device__ __forceinline__ GroupOff group_off(int d, int L, int D) {
    constexpr size_t R = kDlRows;
    GroupOff o;
    o.rkv = 0;
    o.lr = o.rkv + 3 * R * d;
    o.y = o.lr + 3 * R * L;
    o.g = o.y + R * d;
    o.pre = o.g + R * d;
    o.hid = o.pre + R * 3 * D;
    return o;
}

// ------------------------------------------------------------- LayerNorm staging
// LayerNorm (eps 1e-5) of the group's rows into LDS, in three parts so the
// loads are all in flight together: the parameters (before the previous
// barrier), the rows (device-scope loads), then the statistics and the write.
// Wave w takes rows w and w + 4.
struct LnPar {
    float g[kMaxPer], b[kMaxPer];
};
struct LnRows {
    float v[2][kMaxPer], gv[2][kMaxPer];
};

__device__ __forceinline__ void ln_par(LnPar &P, const float *gamma, const float *beta, int cols, int lane) {
#pragma unroll
    for (int e = 0; e < kMaxPer; ++e) {
        const int k = lane + 64 * e;
        P.g[e] = k < cols ? gamma[k] : 0.0f;
        P.b[e] = k < cols ? beta[k] : 0.0f;
    }
}

// Row m of the source at element offset row_off(m) of src (and its gate at
// row_off(m) + gate_off of gsrc when gated).
template <typename RowOff>
__device__ __forceinline__ void ln_rows(LnRows &R, __amdgpu_buffer_rsrc_t src, RowOff row_off, int cols, int M,
                                        __amdgpu_buffer_rsrc_t gsrc, bool gated, size_t gate_off, int lane, int wave) {
#pragma unroll
    for (int half = 0; half < 2; ++half) {
        const int m = wave + kWaves * half;
#pragma unroll
        for (int e = 0; e < kMaxPer; ++e) {
            const int k = lane + 64 * e;
            const bool ok = m < M && k < cols;
            R.v[half][e] = ok ? ld_sc1(src, (uint32_t)((row_off(m) + k) * 4)) : 0.0f;
            R.gv[half][e] = ok && gated ? ld_sc1(gsrc, (uint32_t)((row_off(m) + gate_off + k) * 4)) : 0.0f;
        }
    }
}

__device__ __forceinline__ void ln_write(const LnRows &R, const LnPar &P, int cols, int M, bool gated, float *dst,
                                         int ldd, int lane, int wave) {
#pragma unroll
    for (int half = 0; half < 2; ++half) {
        const int m = wave + kWaves * half;
        float sum = 0.0f;
#pragma unroll
        for (int e = 0; e < kMaxPer; ++e) sum += R.v[half][e];
        const float mean = wave_sum(sum) / (float)cols;
        float sq = 0.0f;
#pragma unroll
        for (int e = 0; e < kMaxPer; ++e) {
            const float dv = lane + 64 * e < cols ? R.v[half][e] - mean : 0.0f;
            sq = fmaf(dv, dv, sq);
        }
        const float rstd = rsqrtf(wave_sum(sq) / (float)cols + 1e-5f);
#pragma unroll
        for (int e = 0; e < kMaxPer; ++e) {
            const int k = lane + 64 * e;
            if (k < cols) {
                float o = 0.0f;
                if (m < M) {
                    o = (R.v[half][e] - mean) * rstd * P.g[e] + P.b[e];
                    if (gated) o *= R.gv[half][e];
                }
                dst[m * ldd + k] = o;
            }
        }
    }
}

// ------------------------------------------------------------- product tiles
// A 16-row x 16-column product tile is the sum over KT k tiles of 16 of A
// (afrag(kt): the floatx4 k = 16 kt + 4 (lane / 16) .. + 3 of row lane % 16)
// times a tiled weight slice w0 (and w1, the gate half of a SiLU pair): one
// contiguous 1 KB tile per wave load, the k order inside a tile permuted alike
// for A and W.  Wave w takes k tiles w, w + 4, ..., in batches of kCh.
struct WBuf {
    floatx4 a[kCh], b[kCh];
};

template <bool PAIR>
__device__ __forceinline__ void load_batch(WBuf &B, const float *w0, const float *w1, int nt, int i0, int wave,
                                           int off) {
#pragma unroll
    for (int c = 0; c < kCh; ++c) {
        const int i = i0 + c;
        if (i < nt) {
            const size_t o = (size_t)(wave + kWaves * i) * 256 + off;
            B.a[c] = ldg4(w0 + o);
            if (PAIR) B.b[c] = ldg4(w1 + o);
        }
    }
}

template <bool PAIR, typename AF>
__device__ __forceinline__ void mma_batch(const WBuf &B, AF &af, int nt, int i0, int wave, floatx4 &c0,
                                          floatx4 &c1) {
#pragma unroll
    for (int c = 0; c < kCh; ++c) {
        const int i = i0 + c;
        if (i < nt) {
            const floatx4 a = af(wave + kWaves * i);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                c0 = __builtin_amdgcn_mfma_f32_16x16x4f32(a[j], B.a[c][j], c0, 0, 0, 0);
                if (PAIR) c1 = __builtin_amdgcn_mfma_f32_16x16x4f32(a[j], B.b[c][j], c1, 0, 0, 0);
            }
        }
    }
}

// Items first, first + stride, ... below total of a product stage with KT k
// tiles.  Each item takes nb batches per wave (the same count for every wave,
// so the reductions' barriers line up); batches stream through P and Q, the
// next one loading while the current one's MFMAs run.  P must hold the first
// item's batch 0 on entry (prefetch_first).  wof(item, w0, w1) sets the
// item's weight slice, afrag(item, kt) gives its A fragments, fin(item, c0,
// c1) reduces and stores the tile.
// The XCDs walk a stage's items rotated by rot (x total / groups for XCD x):
// the same slice requested by all XCDs at once would queue eight requests on
// the same memory channels; rotated, they read different slices and a slice
// read later by another XCD comes from the memory-side cache.
struct Stream {
    int first, stride, total, KT, rot;
    __device__ __forceinline__ int nt(int wave) const { return KT > wave ? (KT - wave + kWaves - 1) / kWaves : 0; }
    __device__ __forceinline__ int nb() const { return ((KT + kWaves - 1) / kWaves + kCh - 1) / kCh; }
    __device__ __forceinline__ int items() const { return first < total ? (total - first + stride - 1) / stride : 0; }
    __device__ __forceinline__ int item(int k) const {
        const int i = first + k * stride + rot;
        return i < total ? i : i - total;
    }
};

template <bool PAIR, typename WOf>
__device__ __forceinline__ void prefetch_first(WBuf &P, const Stream &S, WOf &wof, int lane, int wave) {
    if (S.items() == 0) return;
    const float *w0, *w1;
    wof(S.item(0), w0, w1);
    load_batch<PAIR>(P, w0, w1, S.nt(wave), 0, wave, (lane & 15) * 16 + 4 * (lane >> 4));
}

template <bool PAIR, typename WOf, typename AFrag, typename Fin>
__device__ __forceinline__ void product_stream(WBuf &P, WBuf &Q, const Stream &S, WOf &wof, AFrag &afrag, Fin &fin,
                                               int lane, int wave) {
    const int off = (lane & 15) * 16 + 4 * (lane >> 4);
    const int nt = S.nt(wave), nb = S.nb();
    const int tb = S.items() * nb;
    floatx4 c0 = {0.0f, 0.0f, 0.0f, 0.0f}, c1 = c0;
    auto load = [&](WBuf &B, int b) __attribute__((always_inline)) {
        const float *w0, *w1;
        wof(S.item(b / nb), w0, w1);
        load_batch<PAIR>(B, w0, w1, nt, (b % nb) * kCh, wave, off);
    };
    auto step = [&](const WBuf &B, int b) __attribute__((always_inline)) {
        const int item = S.item(b / nb);
        auto af = [&](int kt) __attribute__((always_inline)) { return afrag(item, kt); };
        mma_batch<PAIR>(B, af, nt, (b % nb) * kCh, wave, c0, c1);
        if (b % nb == nb - 1) {
            fin(item, c0, c1);
            c0 = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
            c1 = c0;
        }
    };
    for (int b = 0; b < tb; b += 2) {
        if (b + 1 < tb) load(Q, b + 1);
        step(P, b);
        if (b + 1 >= tb) break;
        if (b + 2 < tb) load(P, b + 2);
        step(Q, b + 1);
    }
}

// The waves' partial tiles summed in a fixed order: out(row, col, x, g) for
// rows < kDlRows (g: the gate half of a SiLU pair).
template <bool PAIR, typename Out>
__device__ __forceinline__ void reduce_tile(float *sR, const floatx4 &c0, const floatx4 &c1, int tid, int lane,
                                            int wave, Out &&out) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int row = 4 * (lane >> 4) + r;
        sR[wave * kTile + row * 17 + (lane & 15)] = c0[r];
        if (PAIR) sR[(kWaves + wave) * kTile + row * 17 + (lane & 15)] = c1[r];
    }
    __syncthreads();
    if (tid < kDlRows * 16) {
        const int row = tid >> 4, col = tid & 15;
        float x = 0.0f, g = 0.0f;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) {
            x += sR[w * kTile + row * 17 + col];
            if (PAIR) g += sR[(kWaves + w) * kTile + row * 17 + col];
        }
        out(row, col, x, g);
    }
    __syncthreads();
}

template <int N, int EPL>
__global__ void __launch_bounds__(kThreads) decode_layer_kernel(DecodeLayerParams p, size_t gfloats) {
    __shared__ __attribute__((aligned(16))) float sA[kRegA];
    __shared__ __attribute__((aligned(16))) float sX[kRegX];
    __shared__ __attribute__((aligned(16))) float sM[kRegM];
    __shared__ __attribute__((aligned(16))) float sR[kRegR];
    __shared__ int sOk;

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    unsigned xraw;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xraw));
    const int x = (int)(xraw & 15u) % p.groups;
    const int rank = blockIdx.x / p.groups, per = gridDim.x / p.groups;
    const int b0 = (int)((long long)p.n * x / p.groups);
    const int M = (int)((long long)p.n * (x + 1) / p.groups) - b0;
    const int d = p.d, L = p.L, D = p.D, H = p.H, hid = 4 * d;
    const GroupOff go = group_off(d, L, D);
    float *const gb = p.buf + (size_t)x * gfloats;
    const auto rg = make_rsrc(gb, (uint32_t)(gfloats * 4));
    const auto rh = make_rsrc(p.h, (uint32_t)((size_t)p.n * d * 4));
    auto slot_of = [&](int m) { return p.slot ? p.slot[b0 + m] : b0 + m; };
    auto done = [&](int s) { return p.sync + (size_t)(s * p.groups + x) * kDlCounterStride; };
    int *const reg = p.sync + (size_t)kDlStages * p.groups * kDlCounterStride + (size_t)x * per + rank;
    const int items[kDlStages] = {M ? 3 * (d / 16) + 3 * (L / 16) : 0, M ? H * ((M + 3) / 4) : 0, M ? d / 16 : 0,
                                  M ? 3 * D / 16 : 0, M ? d / 16 : 0, M ? hid / 16 : 0, M ? d / 16 : 0};
    auto rot_of = [&](int s) { return (int)((long long)items[s] * x / p.groups); };
    auto stream = [&](int s, int KT) { return Stream{rank, per, items[s], KT, rot_of(s)}; };

    // This workgroup's (XCD, rank) slot; read back at the first barrier and
    // checked at the second.
    if (tid == 0) (void)atom_add(reg, 1);
    int reg_seen = 1;

    // Stage barrier of the group (see the file comment).
    auto barrier = [&](int s, int cnt) -> bool {
        wait_vmem();
        __syncthreads();
        if (tid == 0) {
            bool good = s != kS2 || reg_seen == 1;  // a shared (XCD, rank): two workgroups on one item
            if (cnt) atom_add(done(s), cnt);
            int n = 0;
            for (; n < kPollCap; ++n) {
                if (atom_add(done(s), 0) >= items[s]) break;
                __builtin_amdgcn_s_sleep(1);
            }
            good = good && n < kPollCap;
            if (!good) __hip_atomic_fetch_or(p.error, 2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            // Every workgroup of the group registered before it arrived here.
            if (s == kS1) reg_seen = atom_add(reg, 0);
            sOk = good;
        }
        __syncthreads();
        return sOk;
    };

    WBuf P, Q;
    LnPar lp;
    LnRows lr;
    const float *const wt6[6] = {p.wt_rkv[0], p.wt_rkv[1], p.wt_rkv[2], p.wt_lr1[0], p.wt_lr1[1], p.wt_lr1[2]};
    const int kq1 = 3 * (d / 16);
    // Stage 1 item -> product c (r, k, v, w1, a1, g1) and column slice j.
    auto item1 = [&](int it, int &c, int &j) {
        if (it < kq1) {
            c = it / (d / 16);
            j = it - c * (d / 16);
        } else {
            c = 3 + (it - kq1) / (L / 16);
            j = (it - kq1) - (c - 3) * (L / 16);
        }
    };

    // ---------------------------------------------------------------- stage 1
    // A_c = xn + (xn - prev) * mix_c (model.py:98-105), xn = LN_t(h).
    const Stream s1 = stream(kS1, d / 16);
    auto wof1 = [&](int it, const float *&w0, const float *&w1) {
        int c, j;
        item1(it, c, j);
        w0 = w1 = wt6[c] + (size_t)j * 16 * d;
    };
    {
        float *sPv = sA, *sMix = sA + kRegX;
        ln_par(lp, p.ln_t_w, p.ln_t_b, d, lane);
        prefetch_first<false>(P, s1, wof1, lane, wave);
        if (s1.items()) {
            ln_rows(lr, rh, [&](int m) { return (size_t)(b0 + m) * d; }, d, M, rh, false, 0, lane, wave);
            for (int e = tid; e < kDlRows * d / 4; e += kThreads) {
                const int m = e / (d / 4), k = 4 * (e - m * (d / 4));
                floatx4 v = {0.0f, 0.0f, 0.0f, 0.0f};
                if (m < M) v = ldg4(p.prev + (size_t)slot_of(m) * d + k);
                sts4(sPv + m * kLdX + k, v);
            }
            for (int e = tid; e < 6 * d / 4; e += kThreads) sts4(sMix + 4 * e, ldg4(p.mix6 + 4 * e));
            ln_write(lr, lp, d, M, false, sX, kLdX, lane, wave);
            __syncthreads();
        }
        // mix6 holds mix_r, mix_w, mix_k, mix_v, mix_a, mix_g; products
        // c = r, k, v, w1, a1, g1 take mixes 0, 2, 3, 1, 4, 5.
        auto af = [&](int it, int kt) __attribute__((always_inline)) {
            constexpr int kMixOf[6] = {0, 2, 3, 1, 4, 5};
            int c, j;
            item1(it, c, j);
            const float *mixc = sMix + kMixOf[c] * d;
            const int row = lane & 15, k = kt * 16 + 4 * (lane >> 4);
            floatx4 a = {0.0f, 0.0f, 0.0f, 0.0f};
            if (row < kDlRows) {
                const floatx4 xv = lds4(sX + row * kLdX + k), pv = lds4(sPv + row * kLdX + k), mv = lds4(mixc + k);
#pragma unroll
                for (int q = 0; q < 4; ++q) a[q] = fmaf(xv[q] - pv[q], mv[q], xv[q]);
            }
            return a;
        };
        auto fin = [&](int it, const floatx4 &c0, const floatx4 &c1) {
            int c, j;
            item1(it, c, j);
            reduce_tile<false>(sR, c0, c1, tid, lane, wave, [&](int m, int col, float v, float) {
                if (m >= M) return;
                const int cc = j * 16 + col;
                if (c < 3) gb[go.rkv + ((size_t)c * kDlRows + m) * d + cc] = v;
                else gb[go.lr + ((size_t)(c - 3) * kDlRows + m) * L + cc] = c == 3 ? tanhf(v) : v;
            });
        };
        product_stream<false>(P, Q, s1, wof1, af, fin, lane, wave);
    }

    // Stage 2's inputs that stage 1 does not produce: the WKV state of this
    // workgroup's first item and its head's w2t | a2t | g2t rows.
    constexpr int Q4 = N * N / 4, QM = (Q4 + 63) / 64;
    constexpr int kW4 = (3 * N * 64 / 4 + kThreads - 1) / kThreads;
    floatx4 sq[QM], wreg[kW4];
    auto wkv_prefetch = [&](int it) {
        const int hh = it % H, m = (it / H) * 4 + wave;
        const bool live = m < M;
        const float *st = live ? p.wkv + ((size_t)slot_of(m) * H + hh) * N * N : nullptr;
#pragma unroll
        for (int i = 0; i < QM; ++i) {
            const int q = lane + 64 * i;
            sq[i] = live && q < Q4 ? ldg4(st + 4 * q) : floatx4{0.0f, 0.0f, 0.0f, 0.0f};
        }
        const int nl4 = N * L / 4;
#pragma unroll
        for (int i = 0; i < kW4; ++i) {
            const int e = tid + kThreads * i;
            if (e < 3 * nl4) {
                const int mat = e / nl4, r4 = e - mat * nl4;
                const float *src = mat == 0 ? p.w2t : (mat == 1 ? p.a2t : p.g2t);
                wreg[i] = ldg4(src + (size_t)hh * N * L + 4 * r4);
            }
        }
    };
    auto wkv_item = [&](int it) {
        const int i = it + rot_of(kS2);
        return i < items[kS2] ? i : i - items[kS2];
    };
    if (rank < items[kS2]) wkv_prefetch(wkv_item(rank));
    if (!barrier(kS1, s1.items())) return;
    if (rank == 0 && items[kS1] > 0) {
        // The new `previous` rows: LN_t(h) (model.py:197), read by nobody now.
        for (int e = tid; e < M * d; e += kThreads) {
            const int m = e / d, k = e - m * d;
            p.prev[(size_t)slot_of(m) * d + k] = sX[m * kLdX + k];
        }
    }

    // ---------------------------------------------------------------- stage 2
    // WKV step of four streams of one head, one wave per stream, with the
    // second low-rank stage (model.py:108-122, :145-165).
    int cnt2 = 0;
    {
        float *sW = sA;                         // [3][N][kLp]: w2t | a2t | g2t rows of the head
        float *sIn = sW + 3 * N * kLp;          // [4][3][N]: r, k, v
        float *sLr = sIn + 4 * 3 * N;           // [4][3][64]: lw, la, lg
        float *sWave = sLr + 4 * 3 * 64;        // per wave: vec[6][N], part[Q4], rowv[N]
        constexpr int kWaveF = 6 * N + Q4 + N;
        const int ni = items[kS2];
        for (int k = rank; k < ni; k += per) {
            const int it = wkv_item(k);
            if (k != rank) {
                __syncthreads();  // the previous item's LDS reads are done
                wkv_prefetch(it);
            }
            const int hh = it % H, quad = it / H;
            const int m = quad * 4 + wave;
            const bool live = m < M;
            const int nl4 = N * L / 4;
#pragma unroll
            for (int i = 0; i < kW4; ++i) {
                const int e = tid + kThreads * i;
                if (e < 3 * nl4) {
                    const int mat = e / nl4, r4 = e - mat * nl4;
                    const int c = (4 * r4) / L, jj = 4 * r4 - c * L;
                    sts4(sW + (mat * N + c) * kLp + jj, wreg[i]);
                }
            }
            for (int e = tid; e < 4 * 3 * N; e += kThreads) {
                const int s4 = e / (3 * N), rem = e - s4 * 3 * N, c3 = rem / N, c = rem - c3 * N;
                const int ms = quad * 4 + s4;
                sIn[e] = ms < M ? ld_sc1(rg, (uint32_t)((go.rkv + ((size_t)c3 * kDlRows + ms) * d + hh * N + c) * 4))
                                : 0.0f;
            }
            for (int e = tid; e < 4 * 3 * L; e += kThreads) {
                const int s4 = e / (3 * L), rem = e - s4 * 3 * L, c3 = rem / L, jj = rem - c3 * L;
                const int ms = quad * 4 + s4;
                sLr[(s4 * 3 + c3) * 64 + jj] =
                    ms < M ? ld_sc1(rg, (uint32_t)((go.lr + ((size_t)c3 * kDlRows + ms) * L + jj) * 4)) : 0.0f;
            }
            __syncthreads();
            float *vec = sWave + wave * kWaveF, *part = vec + 6 * N, *rowv = part + Q4;
            const bool col = lane < N;
            const int hc = hh * N + lane;
            float dw = 0.0f, da = 0.0f, dg = 0.0f;
            if (col) {
                const float *lw = sLr + (wave * 3) * 64;
                const float *w2 = sW + lane * kLp, *a2 = sW + (N + lane) * kLp, *g2 = sW + (2 * N + lane) * kLp;
                for (int jj = 0; jj < L; jj += 4) {
                    const floatx4 l0 = lds4(lw + jj), l1 = lds4(lw + 64 + jj), l2 = lds4(lw + 128 + jj);
                    const floatx4 x0 = lds4(w2 + jj), x1 = lds4(a2 + jj), x2 = lds4(g2 + jj);
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        dw = fmaf(l0[q], x0[q], dw);
                        da = fmaf(l1[q], x1[q], da);
                        dg = fmaf(l2[q], x2[q], dg);
                    }
                }
            }
            const float rv = col ? sIn[(wave * 3 + 0) * N + lane] : 0.0f;
            float kv = col ? sIn[(wave * 3 + 1) * N + lane] : 0.0f;
            const float vv = col ? sIn[(wave * 3 + 2) * N + lane] : 0.0f;
            const float wv = col ? p.w0[hc] + dw : 0.0f;
            const float alpha = col ? 1.0f / (1.0f + expf(-(p.a0[hc] + da))) : 0.0f;
            if (col && live) gb[go.g + (size_t)m * d + hc] = 1.0f / (1.0f + expf(-dg));
            // kappa = normalize(k * k_k) over the head (eps 1e-12), a = -kappa,
            // b = kappa * alpha, k^ = k (1 + (alpha - 1) k_a).
            const float xk = col ? kv * p.k_k[hc] : 0.0f;
            const float inv = 1.0f / fmaxf(sqrtf(wave_sum(xk * xk)), 1e-12f);
            const float kap = xk * inv;
            if (col) {
                kv = kv * (1.0f + (alpha - 1.0f) * p.k_a[hc]);
                const float sig = __frcp_rn(1.0f + __expf(-wv));
                vec[0 * N + lane] = -kap;
                vec[1 * N + lane] = kap * alpha;
                vec[2 * N + lane] = kv;
                vec[3 * N + lane] = exp2f(-0.8750387749f * sig);  // exp(-e^-0.5 sigmoid(w))
                vec[4 * N + lane] = rv;
                vec[5 * N + lane] = vv;
            }
            wave_lds_sync();
            // sa_i = sum_j S_ij a_j.
#pragma unroll
            for (int i = 0; i < QM; ++i) {
                const int q = lane + 64 * i;
                if (q < Q4) {
                    const floatx4 a4 = lds4(vec + (4 * q) % N);
                    part[q] = (sq[i][0] * a4[0] + sq[i][1] * a4[1]) + (sq[i][2] * a4[2] + sq[i][3] * a4[3]);
                }
            }
            wave_lds_sync();
            if (col) {
                float sa = 0.0f;
#pragma unroll
                for (int u = 0; u < N / 4; ++u) sa += part[lane * (N / 4) + u];
                rowv[lane] = sa;
            }
            wave_lds_sync();
            // S'_ij = S_ij d_j + sa_i b_j + v_i k^_j;  y_i = sum_j S'_ij r_j.
            float *st = live ? p.wkv + ((size_t)slot_of(m) * H + hh) * N * N : nullptr;
#pragma unroll
            for (int i = 0; i < QM; ++i) {
                const int q = lane + 64 * i;
                if (q < Q4) {
                    const int ri = (4 * q) / N, c = (4 * q) % N;
                    const float sa = rowv[ri], vi = vec[5 * N + ri];
                    const floatx4 b4 = lds4(vec + N + c), k4 = lds4(vec + 2 * N + c), d4 = lds4(vec + 3 * N + c),
                                  r4 = lds4(vec + 4 * N + c);
                    floatx4 s2;
#pragma unroll
                    for (int t = 0; t < 4; ++t) s2[t] = fmaf(sq[i][t], d4[t], fmaf(sa, b4[t], k4[t] * vi));
                    part[q] = (s2[0] * r4[0] + s2[1] * r4[1]) + (s2[2] * r4[2] + s2[3] * r4[3]);
                    if (live) *reinterpret_cast<floatx4 *>(st + 4 * q) = s2;
                }
            }
            wave_lds_sync();
            if (col && live) {
                float yv = 0.0f;
#pragma unroll
                for (int u = 0; u < N / 4; ++u) yv += part[lane * (N / 4) + u];
                gb[go.y + (size_t)m * d + hc] = yv;
            }
            ++cnt2;
        }
    }

    // Residual add into h: the current row value was written by another
    // workgroup in this launch, so it is read past the L1.
    auto add_h = [&](int m, int col, float v) {
        const size_t o = (size_t)(b0 + m) * d + col;
        p.h[o] = v + ld_sc1(rh, (uint32_t)(o * 4));
    };
    // A fragments of the A rows staged in sA (row stride lda).
    auto af_lds = [&](int lda) {
        return [&, lda](int, int kt) __attribute__((always_inline)) {
            const int row = lane & 15;
            floatx4 a = {0.0f, 0.0f, 0.0f, 0.0f};
            if (row < kDlRows) a = lds4(sA + row * lda + kt * 16 + 4 * (lane >> 4));
            return a;
        };
    };

    // ---------------------------------------------------------------- stage 3
    // W_o(LN_o(y) * g) + h (model.py:195-196).
    const Stream s3 = stream(kS3, d / 16);
    auto wof3 = [&](int it, const float *&w0, const float *&w1) { w0 = w1 = p.wt_o + (size_t)it * 16 * d; };
    ln_par(lp, p.ln_o_w, p.ln_o_b, d, lane);
    prefetch_first<false>(P, s3, wof3, lane, wave);
    if (!barrier(kS2, cnt2)) return;
    {
        if (s3.items()) {
            ln_rows(lr, rg, [&](int m) { return go.y + (size_t)m * d; }, d, M, rg, true, go.g - go.y, lane, wave);
            ln_write(lr, lp, d, M, true, sA, d + 4, lane, wave);
            __syncthreads();
        }
        auto af = af_lds(d + 4);
        auto fin = [&](int it, const floatx4 &c0, const floatx4 &c1) {
            reduce_tile<false>(sR, c0, c1, tid, lane, wave,
                               [&](int m, int col, float v, float) { if (m < M) add_h(m, it * 16 + col, v); });
        };
        product_stream<false>(P, Q, s3, wof3, af, fin, lane, wave);
    }

    // ---------------------------------------------------------------- stage 4
    // ROSA input | write | read pre-activations of LN_r(h) (model.py:306-311).
    const Stream s4 = stream(kS4, d / 16);
    auto wof4 = [&](int it, const float *&w0, const float *&w1) { w0 = w1 = p.wt_rin + (size_t)it * 16 * d; };
    ln_par(lp, p.ln_r_w, p.ln_r_b, d, lane);
    prefetch_first<false>(P, s4, wof4, lane, wave);
    if (!barrier(kS3, s3.items())) return;
    {
        if (s4.items()) {
            ln_rows(lr, rh, [&](int m) { return (size_t)(b0 + m) * d; }, d, M, rh, false, 0, lane, wave);
            ln_write(lr, lp, d, M, false, sA, d + 4, lane, wave);
            __syncthreads();
        }
        auto af = af_lds(d + 4);
        auto fin = [&](int it, const floatx4 &c0, const floatx4 &c1) {
            reduce_tile<false>(sR, c0, c1, tid, lane, wave, [&](int m, int col, float v, float) {
                const int cc = it * 16 + col;
                if (m < M) gb[go.pre + (size_t)m * 3 * D + cc] = v + p.b_rin[cc];
            });
        };
        product_stream<false>(P, Q, s4, wof4, af, fin, lane, wave);
    }

    // ---------------------------------------------------------------- stage 5
    // ROSA step (model.py:282-288 with the sigmoid read gate) as the A operand
    // of ROSA out: m' = lambda (m - 2 (u.m) u) + tanh(c) sigmoid(w),
    // read = (m' - 2 (u.m') u) sigmoid(rho); dot products in double.
    const Stream s5 = stream(kS5, D / 16);
    auto wof5 = [&](int it, const float *&w0, const float *&w1) { w0 = w1 = p.wt_rout + (size_t)it * 16 * D; };
    float mm[2][EPL], uu[EPL], ll[EPL];
    prefetch_first<false>(P, s5, wof5, lane, wave);
    if (s5.items()) {
#pragma unroll
        for (int q = 0; q < EPL; ++q) {
            uu[q] = p.rosa_u[lane + 64 * q];
            ll[q] = p.rosa_lam[lane + 64 * q];
        }
#pragma unroll
        for (int half = 0; half < 2; ++half) {
            const int m = wave + kWaves * half;
#pragma unroll
            for (int q = 0; q < EPL; ++q) mm[half][q] = m < M ? p.rosa[(size_t)slot_of(m) * D + lane + 64 * q] : 0.0f;
        }
    }
    if (!barrier(kS4, s4.items())) return;
    {
        if (s5.items()) {
            float er[2][EPL], wr[2][EPL], rho[2][EPL];
#pragma unroll
            for (int half = 0; half < 2; ++half) {
                const int m = wave + kWaves * half;
#pragma unroll
                for (int q = 0; q < EPL; ++q) {
                    const size_t pre = go.pre + (size_t)m * 3 * D + lane + 64 * q;
                    const bool ok = m < M;
                    er[half][q] = ok ? ld_sc1(rg, (uint32_t)(pre * 4)) : 0.0f;
                    wr[half][q] = ok ? ld_sc1(rg, (uint32_t)((pre + D) * 4)) : 0.0f;
                    rho[half][q] = ok ? ld_sc1(rg, (uint32_t)((pre + 2 * D) * 4)) : 0.0f;
                }
            }
#pragma unroll
            for (int half = 0; half < 2; ++half) {
                const int m = wave + kWaves * half;
                const bool ok = m < M;
                float e[EPL], rr[EPL];
                double f = 0.0;
#pragma unroll
                for (int q = 0; q < EPL; ++q) {
                    const float th = 1.0f - 2.0f * __frcp_rn(__expf(2.0f * er[half][q]) + 1.0f);
                    e[q] = th * __frcp_rn(1.0f + __expf(-wr[half][q]));
                    rr[q] = __frcp_rn(1.0f + __expf(-rho[half][q]));
                    f = fma((double)uu[q], (double)mm[half][q], f);
                }
                const float p1 = (float)wave_sum_f64(f);
                double f2 = 0.0;
#pragma unroll
                for (int q = 0; q < EPL; ++q) {
                    mm[half][q] = fmaf(ll[q], fmaf(-2.0f * p1, uu[q], mm[half][q]), e[q]);
                    f2 = fma((double)uu[q], (double)mm[half][q], f2);
                }
                const float p2 = (float)wave_sum_f64(f2);
#pragma unroll
                for (int q = 0; q < EPL; ++q) {
                    const int k = lane + 64 * q;
                    sA[m * (D + 4) + k] = ok ? fmaf(-2.0f * p2, uu[q], mm[half][q]) * rr[q] : 0.0f;
                    sM[m * D + k] = mm[half][q];
                }
            }
            __syncthreads();
        }
        auto af = af_lds(D + 4);
        auto fin = [&](int it, const floatx4 &c0, const floatx4 &c1) {
            reduce_tile<false>(sR, c0, c1, tid, lane, wave,
                               [&](int m, int col, float v, float) { if (m < M) add_h(m, it * 16 + col, v); });
        };
        product_stream<false>(P, Q, s5, wof5, af, fin, lane, wave);
    }

    // ---------------------------------------------------------------- stage 6
    // FFN in / gate of LN_f(h), silu(in) * gate (model.py:377); weight rows in
    // 64-row blocks of 32 in then 32 gate rows.
    const Stream s6 = stream(kS6, d / 16);
    auto wof6 = [&](int it, const float *&w0, const float *&w1) {
        w0 = p.wt_fin + (size_t)(4 * (it / 2) + (it & 1)) * 16 * d;
        w1 = w0 + (size_t)2 * 16 * d;
    };
    ln_par(lp, p.ln_f_w, p.ln_f_b, d, lane);
    prefetch_first<true>(P, s6, wof6, lane, wave);
    if (!barrier(kS5, s5.items())) return;
    if (rank == 0 && items[kS5] > 0) {
        // The new ROSA memory rows, read by nobody now.
        for (int e = tid; e < M * D; e += kThreads) {
            const int m = e / D, k = e - m * D;
            p.rosa[(size_t)slot_of(m) * D + k] = sM[m * D + k];
        }
    }
    {
        if (s6.items()) {
            ln_rows(lr, rh, [&](int m) { return (size_t)(b0 + m) * d; }, d, M, rh, false, 0, lane, wave);
            ln_write(lr, lp, d, M, false, sA, d + 4, lane, wave);
            __syncthreads();
        }
        auto af = af_lds(d + 4);
        auto fin = [&](int it, const floatx4 &c0, const floatx4 &c1) {
            reduce_tile<true>(sR, c0, c1, tid, lane, wave, [&](int m, int col, float v, float g) {
                if (m < M) gb[go.hid + (size_t)m * hid + it * 16 + col] = v / (1.0f + expf(-v)) * g;
            });
        };
        product_stream<true>(P, Q, s6, wof6, af, fin, lane, wave);
    }

    // ---------------------------------------------------------------- stage 7
    // FFN out + h; the launch's end orders it before the next layer.
    const Stream s7 = stream(kS7, hid / 16);
    auto wof7 = [&](int it, const float *&w0, const float *&w1) { w0 = w1 = p.wt_fout + (size_t)it * 16 * hid; };
    prefetch_first<false>(P, s7, wof7, lane, wave);
    if (!barrier(kS6, s6.items())) return;
    if (s7.items()) {
        const int q4 = hid / 4;
        for (int e = tid; e < kDlRows * q4; e += kThreads) {
            const int m = e / q4, k = 4 * (e - m * q4);
            floatx4 v = {0.0f, 0.0f, 0.0f, 0.0f};
            if (m < M) v = ld4_sc1(rg, (uint32_t)((go.hid + (size_t)m * hid + k) * 4));
            sts4(sA + m * (hid + 4) + k, v);
        }
        __syncthreads();
    }
    auto af7 = af_lds(hid + 4);
    auto fin7 = [&](int it, const floatx4 &c0, const floatx4 &c1) {
        reduce_tile<false>(sR, c0, c1, tid, lane, wave,
                           [&](int m, int col, float v, float) { if (m < M) add_h(m, it * 16 + col, v); });
    };
    product_stream<false>(P, Q, s7, wof7, af7, fin7, lane, wave);
}

}  // namespace

bool decode_layer_ok(int d, int H, int N, int L, int D) {
    const bool n_ok = N == 16 || N == 32 || N == 40 || N == 64;
    return n_ok && d == H * N && d % 16 == 0 && d <= kDlMaxD && L % 16 == 0 && L >= 16 && L <= 64 &&
           (D == 64 || D == 128 || D == 256);
}

size_t decode_layer_group_floats(int d, int L, int D) {
    return (size_t)kDlRows * (3 * (size_t)d + 3 * (size_t)L + 2 * (size_t)d + 3 * (size_t)D + 4 * (size_t)d);
}

size_t decode_layer_sync_ints(int groups, int grid) {
    return (size_t)kDlStages * groups * kDlCounterStride + (size_t)grid;
}

hipError_t launch_decode_layer(const DecodeLayerParams &p, int grid, hipStream_t stream) {
    if (!decode_layer_ok(p.d, p.H, p.N, p.L, p.D) || p.groups < 1 || p.n < 1 || p.n > kDlRows * p.groups ||
        grid < p.groups || grid % p.groups != 0 || !p.sync || !p.error || !p.buf || !p.h)
        return hipErrorInvalidValue;
    const size_t gf = decode_layer_group_floats(p.d, p.L, p.D);
    const int epl = p.D / 64;
#define YUF_DL_LAUNCH(NN)                                                                                      \
    do {                                                                                                       \
        if (epl == 1)                                                                                          \
            hipLaunchKernelGGL((decode_layer_kernel<NN, 1>), dim3(grid), dim3(kThreads), 0, stream, p, gf);   \
        else if (epl == 2)                                                                                     \
            hipLaunchKernelGGL((decode_layer_kernel<NN, 2>), dim3(grid), dim3(kThreads), 0, stream, p, gf);   \
        else                                                                                                   \
            hipLaunchKernelGGL((decode_layer_kernel<NN, 4>), dim3(grid), dim3(kThreads), 0, stream, p, gf);   \
    } while (0)
    switch (p.N) {
        case 16: YUF_DL_LAUNCH(16); break;
        case 32: YUF_DL_LAUNCH(32); break;
        case 40: YUF_DL_LAUNCH(40); break;
        default: YUF_DL_LAUNCH(64); break;
    }
#undef YUF_DL_LAUNCH
    return hipGetLastError();
}

}  // namespace yuf
