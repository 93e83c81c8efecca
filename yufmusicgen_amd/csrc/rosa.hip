// ROSA Householder memory scan for gfx950 (MI355X).
//
// Semantics: yufmusicgen/model.py:260-288 (reference recurrence) and the read
// of model.py:303-311 / yufmusicgen/cuda/rosa_householder.cu:30-101:
//     m_t    = lambda * H(m_{t-1}) + e_t,   e_t = sigmoid(write_t) tanh(cand_t)
//     read_t = H(m_t) [* sigmoid(read_raw_t)],     H(x) = x - 2 (x.u) u.
//
// The transition diag(lambda) H = diag(lambda) - 2 (lambda u) u^T is diagonal
// plus rank one, so with p_t = u.m_{t-1} the recurrence is
//     m_t = lambda (m_{t-1} - 2 p_t u) + e_t.
// Over a chunk of C tokens starting from m_0 (1-based tau):
//     m_tau = y_tau - 2 c_tau,  y_tau = lambda^tau m_0 + z_tau,
//     z_tau = lambda z_{tau-1} + e_tau (z_0 = 0),  c_tau = lambda (c_{tau-1} + p_tau u),
// and the projections solve a lower-triangular Toeplitz system
//     p_tau + 2 sum_{s<tau} kappa_{tau-s} p_s = f_tau := u.y_{tau-1},
//     kappa_n = sum_j u_j^2 lambda_j^n,   p = L f,  L[tau][s] = ell_{tau-s},
//     ell_0 = 1, ell_n = -2 sum_{k=1..n} kappa_k ell_{n-k}.
// So the only cross-channel reductions are the C+1 dot products f (one batch
// per chunk), not one wave reduction per token as in the direct recurrence.
//
// One workgroup per stream, 1 consumer wave + 6 producer waves, three LDS
// stages in flight (chunk i+1 staged, chunk i solved, chunk i-1 emitted):
//   producers, A(i+1): turn chunk i+1's pre-activations (loaded one iteration
//       earlier with bounds-checked buffer loads) into e and the gate in LDS --
//       or take e and the gate as computed by the model's input projection --
//       and run the per-channel z recurrence;
//   consumer, B(i):   f = u.(lambda^tau m_0 + z_tau) for tau = 0..C (per-lane
//       partials, transposed through LDS), p = L f, then the chunk-end state;
//   producers, O(i-1): per channel, m_tau = lambda (m_{tau-1} - 2 p_tau u) + e_tau
//       with the now-known p, and read_tau = (m_tau - 2 p_{tau+1} u) g_tau.
// All waves meet at one barrier per chunk.
#include "common.h"
#include "kernels.h"

#include <cstdlib>
#include <cstring>
#include <map>
#include <mutex>
#include <utility>

namespace yuf {
namespace {

constexpr int kWave = 64;
// Waves w and w + 4 of a workgroup share a SIMD: the consumer (wave 0) keeps its
// SIMD to itself (wave 4 only joins the barriers), six producers take waves
// 1-3 and 5-7.
constexpr int kProducerWaves = 6;
constexpr int kThreads = 8 * kWave;
constexpr int kStages = 3;

template <int EPL>
struct Cfg {
    static constexpr int C = EPL <= 2 ? 16 : (EPL == 4 ? 8 : (EPL == 8 ? 4 : 2));  // tokens per chunk
    static constexpr int DP = EPL * kWave;                                          // padded channels
    static constexpr int ZS = C + 1;          // odd row stride of the transposed z / partial arrays
    static constexpr int CH = (DP + kProducerWaves - 1) / kProducerWaves;  // channels per producer wave
    static constexpr int CPL = (CH + kWave - 1) / kWave;                   // channels per producer lane
    static constexpr int kItems = (C * CH + kWave - 1) / kWave;            // (token, channel) loads per lane
};

// LDS-only ordering between lanes of one wave (no s_barrier).
__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Column j of A^L, A = diag(lambda) (I - 2 u u^T) (lambda post-sigmoid, u
// unit), in double, by one wave: A applied L times to e_j through the
// rank-one form A x = lambda (x - 2 (u.x) u); AL[i][j] = x_i.  PER =
// ceil(D / 64) rows per lane; the L projections u.x are the chain, each one
// DPP / row-swap reduction.
template <int PER>
__device__ __forceinline__ void power_column(int D, int L, const float *lambda, const float *u, float *AL, int j,
                                             int lane) {
    double x[PER], uu[PER], lam[PER];
#pragma unroll
    for (int e = 0; e < PER; ++e) {
        const int i = lane + 64 * e;
        const bool in = i < D;
        x[e] = in && i == j ? 1.0 : 0.0;
        uu[e] = in ? (double)u[i] : 0.0;
        lam[e] = in ? (double)lambda[i] : 0.0;
    }
    for (int step = 0; step < L; ++step) {
        double pr = 0.0;
#pragma unroll
        for (int e = 0; e < PER; ++e) pr += uu[e] * x[e];
        pr = wave_sum_f64(pr);
#pragma unroll
        for (int e = 0; e < PER; ++e) x[e] = lam[e] * (x[e] - 2.0 * pr * uu[e]);
    }
#pragma unroll
    for (int e = 0; e < PER; ++e) {
        const int i = lane + 64 * e;
        if (i < D) AL[(size_t)i * D + j] = (float)x[e];
    }
}

// EMIT = false: end states only (the first pass of the segmented scan), so
// neither the reads nor their gate are computed and the gate input is not
// loaded.  A compile-time switch: as a run-time flag its tests inside the
// unrolled load loops made the scan ~35 % slower at D = 256.
template <int EPL, bool EMIT>
__global__ void __launch_bounds__(kThreads) rosa_scan_kernel(RosaParams p) {
    using K = Cfg<EPL>;
    constexpr int C = K::C, DP = K::DP, ZS = K::ZS, CH = K::CH, CPL = K::CPL;
    __shared__ __attribute__((aligned(16))) float ew[kStages][C * DP];  // e_tau   [tau][c]
    __shared__ __attribute__((aligned(16))) float gt[kStages][C * DP];  // gate    [tau][c]
    __shared__ float zt[kStages][DP * ZS];                              // z_tau   [c][tau], tau = 0..C
    __shared__ float pv[kStages][ZS];                                   // p_{tau+1}, tau = 0..C
    __shared__ float m0b[kStages][DP];                                  // chunk-start state
    __shared__ float lam_s[DP], u_s[DP];
    // Consumer-only: per-lane partial dot products [lane][tau], f, and the Toeplitz
    // inverse ell, in double: ell alternates in sign with |ell_n| up to 2 when the
    // decay is near 1, so p = L f adds up to C rounding errors of f with weight 2.
    __shared__ double part[kWave * ZS];
    __shared__ double fv[ZS], ell[ZS];

    const int bb = blockIdx.x;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int D = p.D;
    const int slot = p.slot ? p.slot[bb] : bb;
    const bool gated = p.read_raw != nullptr || p.e_pre != nullptr;
    const int n_chunks = (p.T + C - 1) / C;

    // ------------------------------------------------------------ producers
    const int pw = wave < 4 ? wave - 1 : wave - 2;  // producer index on waves 1-3, 5-7
    const bool producer = wave != 0 && wave != 4;
    const bool prepared = p.e_pre != nullptr;
    // Next chunk's inputs, loaded one iteration ahead: (cand, write, read_raw) or,
    // prepared, (e, gate).  Every load is issued; an input that is not needed
    // has a zero-size descriptor and reads 0 without touching memory.
    float in0[K::kItems], in1[K::kItems], in2[K::kItems];
    auto load_in = [&](int ch) {
        const int t0 = ch * C, nt = min(C, p.T - t0);
        const size_t base = (size_t)(bb * p.T + t0) * p.ld;
        const uint32_t bytes = (uint32_t)(((nt - 1) * p.ld + D) * 4);
        const auto r0 = make_rsrc((prepared ? p.e_pre : p.cand) + base, bytes);
        const auto r1 = make_rsrc((prepared ? p.g_pre : p.write) + base, EMIT || !prepared ? bytes : 0u);
        const auto r2 = make_rsrc(gated && !prepared ? p.read_raw + base : p.cand + base,
                                  gated && !prepared ? bytes : 0u);
#pragma unroll
        for (int it = 0; it < K::kItems; ++it) {
            const int q = lane + it * kWave;
            const int tau = q / CH, c = pw * CH + (q - tau * CH);
            const uint32_t off = (q < C * CH && c < D && tau < nt) ? (uint32_t)(tau * p.ld + c) * 4u : kBufferOob;
            in0[it] = buf_load(r0, off);
            in1[it] = buf_load(r1, off);
            in2[it] = EMIT ? buf_load(r2, off) : 0.0f;
        }
    };
    auto stage_in = [&](int ch) {  // A(ch), from the registers load_in(ch) filled
        const int s = ch % kStages;
#pragma unroll
        for (int it = 0; it < K::kItems; ++it) {
            const int q = lane + it * kWave;
            const int tau = q / CH, c = pw * CH + (q - tau * CH);
            if (q < C * CH && c < DP) {
                float e, gv;
                if (prepared) {
                    e = in0[it];
                    gv = EMIT ? in1[it] : 1.0f;
                } else {
                    // tanh(x) = 1 - 2 / (e^{2x} + 1); sigmoid(x) = 1 / (1 + e^{-x}).  Out-of-range
                    // tokens and channels read 0 and give e = 0.
                    const float th = 1.0f - 2.0f * __frcp_rn(__expf(2.0f * in0[it]) + 1.0f);
                    e = th * __frcp_rn(1.0f + __expf(-in1[it]));
                    gv = EMIT && gated ? __frcp_rn(1.0f + __expf(-in2[it])) : 1.0f;
                }
                ew[s][tau * DP + c] = e;
                gt[s][tau * DP + c] = gv;
            }
        }
        wave_lds_sync();
#pragma unroll
        for (int k = 0; k < CPL; ++k) {
            const int cc = lane + k * kWave;
            const int c = pw * CH + cc;
            if (cc < CH && c < DP) {
                const float lam = lam_s[c];
                float z = 0.0f;
                zt[s][c * ZS] = 0.0f;
#pragma unroll
                for (int tau = 0; tau < C; ++tau) {
                    z = fmaf(lam, z, ew[s][tau * DP + c]);
                    zt[s][c * ZS + tau + 1] = z;
                }
            }
        }
    };
    auto emit = [&](int ch) {  // O(ch)
        if constexpr (!EMIT) return;
        const int s = ch % kStages, t0 = ch * C, nt = min(C, p.T - t0);
        const size_t obase = (size_t)(bb * p.T + t0) * D;
        const auto ro = make_rsrc(p.read_out + obase, (uint32_t)(nt * D * 4));
#pragma unroll
        for (int k = 0; k < CPL; ++k) {
            const int cc = lane + k * kWave;
            const int c = pw * CH + cc;
            if (cc < CH && c < DP) {
                const float lam = lam_s[c], u = u_s[c];
                float m = m0b[s][c];
                // All C steps run (tokens past nt have e = 0 and are not stored), so
                // the LDS reads are independent of the chain and issue up front.
#pragma unroll
                for (int tau = 0; tau < C; ++tau) {
                    m = fmaf(lam, fmaf(-2.0f * pv[s][tau], u, m), ew[s][tau * DP + c]);
                    const float rv = fmaf(-2.0f * pv[s][tau + 1], u, m) * gt[s][tau * DP + c];
                    buf_store(rv, ro, (c < D && tau < nt) ? (uint32_t)(tau * D + c) * 4u : kBufferOob);
                }
            }
        }
    };

    // ------------------------------------------------------------- consumer
    float lam[EPL], u[EPL], m0[EPL];
    if (wave == 0) {
        float nrm = 0.0f;
#pragma unroll
        for (int e = 0; e < EPL; ++e) {
            const int c = lane + e * kWave;
            const bool ok = c < D;
            u[e] = ok ? p.direction[c] : 0.0f;
            lam[e] = ok ? p.decay[c] : 0.0f;
            m0[e] = (ok && p.memory_in) ? p.memory_in[(size_t)slot * D + c] : 0.0f;
            nrm = fmaf(u[e], u[e], nrm);
        }
        if (p.raw_params) {
            // Model path: u = householder / max(|householder|, 1e-12), lambda = sigmoid(decay)
            // (model.py:300-301).
            const float inv = 1.0f / fmaxf(sqrtf(wave_sum(nrm)), 1e-12f);
#pragma unroll
            for (int e = 0; e < EPL; ++e) {
                const int c = lane + e * kWave;
                u[e] *= inv;
                lam[e] = c < D ? 1.0f / (1.0f + expf(-lam[e])) : 0.0f;
            }
        }
#pragma unroll
        for (int e = 0; e < EPL; ++e) {
            lam_s[lane + e * kWave] = lam[e];
            u_s[lane + e * kWave] = u[e];
        }
        // kappa_n = sum_j u_j^2 lambda_j^n, n = 1..C, then the Toeplitz inverse ell.
        {
            double pw_[EPL];
#pragma unroll
            for (int e = 0; e < EPL; ++e) pw_[e] = (double)u[e] * u[e];
            for (int n = 1; n <= C; ++n) {
                double acc = 0.0;
#pragma unroll
                for (int e = 0; e < EPL; ++e) {
                    pw_[e] *= lam[e];
                    acc += pw_[e];
                }
                part[lane * ZS + n] = acc;
            }
            wave_lds_sync();
            if (lane >= 1 && lane <= C) {
                double acc = 0.0;
                for (int k = 0; k < kWave; ++k) acc += part[k * ZS + lane];
                fv[lane] = acc;  // kappa_lane
            }
            wave_lds_sync();
            if (lane == 0) {
                ell[0] = 1.0;
                for (int n = 1; n <= C; ++n) {
                    double acc = 0.0;
                    for (int k = 1; k <= n; ++k) acc = fma(fv[k], ell[n - k], acc);
                    ell[n] = -2.0 * acc;
                }
            }
            wave_lds_sync();
        }
        wait_vmem();
    }
    lds_barrier();  // lam_s / u_s visible to the producers
    if (producer && n_chunks > 0) {
        load_in(0);
        stage_in(0);
        if (n_chunks > 1) load_in(1);
    }
    lds_barrier();

    for (int i = 0; i <= n_chunks; ++i) {
        if (wave == 0) {
            if (i < n_chunks) {
                const int s = i % kStages, nt = min(C, p.T - i * C);
                // f_{tau+1} = u . (lambda^tau m_0 + z_tau), tau = 0..C: per-lane partials.
                float y[EPL];
#pragma unroll
                for (int e = 0; e < EPL; ++e) y[e] = m0[e];
                for (int tau = 0; tau <= C; ++tau) {
                    double acc = 0.0;
#pragma unroll
                    for (int e = 0; e < EPL; ++e) {
                        const double ud = u[e];
                        acc = fma(ud, (double)y[e], fma(ud, (double)zt[s][(lane + e * kWave) * ZS + tau], acc));
                        y[e] *= lam[e];
                    }
                    part[lane * ZS + tau] = acc;
                }
                wave_lds_sync();
                // Sums over the 64 lanes' partials and the Toeplitz products use
                // independent accumulators: these chains are the scan's critical path.
                if (lane <= C) {
                    double a8[8] = {0.0, 0.0, 0.0, 0.0, 0.0, 0.0, 0.0, 0.0};
#pragma unroll
                    for (int k = 0; k < kWave; k += 8)
#pragma unroll
                        for (int m = 0; m < 8; ++m) a8[m] += part[(k + m) * ZS + lane];
                    fv[lane] = ((a8[0] + a8[1]) + (a8[2] + a8[3])) + ((a8[4] + a8[5]) + (a8[6] + a8[7]));
                }
                wave_lds_sync();
                if (lane <= C) {
                    double a4[4] = {0.0, 0.0, 0.0, 0.0};
#pragma unroll
                    for (int sg = 0; sg <= C; ++sg) {
                        const double coef = sg <= lane ? ell[sg <= lane ? lane - sg : 0] : 0.0;
                        a4[sg & 3] = fma(coef, fv[sg], a4[sg & 3]);
                    }
                    pv[s][lane] = (float)((a4[0] + a4[1]) + (a4[2] + a4[3]));
                }
#pragma unroll
                for (int e = 0; e < EPL; ++e) m0b[s][lane + e * kWave] = m0[e];
                wave_lds_sync();
                // State after the chunk's nt real tokens:
                // m_nt = lambda^nt m_0 + z_nt - 2 sum_{s<=nt} p_s lambda^{nt-s+1} u.
                float acc[EPL], pwr[EPL];
#pragma unroll
                for (int e = 0; e < EPL; ++e) { acc[e] = 0.0f; pwr[e] = m0[e]; }
#pragma unroll
                for (int sg = 0; sg < C; ++sg) {
                    const float ps = pv[s][sg];
#pragma unroll
                    for (int e = 0; e < EPL; ++e) {
                        if (sg < nt) {
                            acc[e] = lam[e] * fmaf(ps, u[e], acc[e]);
                            pwr[e] *= lam[e];
                        }
                    }
                }
#pragma unroll
                for (int e = 0; e < EPL; ++e)
                    m0[e] = fmaf(-2.0f, acc[e], pwr[e] + zt[s][(lane + e * kWave) * ZS + nt]);
            }
        } else if (producer) {
            if (i >= 1) emit(i - 1);
            if (i + 1 < n_chunks) {
                stage_in(i + 1);
                if (i + 2 < n_chunks) load_in(i + 2);
            }
        }
        lds_barrier();
    }
    // End state: every row, or (segmented second pass) each chain's last segment.
    int out_row = slot;
    bool write_out = p.memory_out != nullptr;
    if (p.seg > 0) {
        const int chain = bb / p.seg;
        write_out = write_out && bb - chain * p.seg == p.seg - 1;
        out_row = p.seg_slot ? p.seg_slot[chain] : chain;
    }
    if (wave == 0 && write_out) {
#pragma unroll
        for (int e = 0; e < EPL; ++e) {
            const int c = lane + e * kWave;
            if (c < D) p.memory_out[(size_t)out_row * D + c] = m0[e];
        }
    }
}

}  // namespace


// Single-token step (T = 1, decode): one wave per stream, EPL channels per
// lane, the direct recurrence with its two projections (u.m_{t-1} and u.m_t)
// summed in double across the wave, and the gates computed from the raw
// pre-activations in place (the same float expressions as the scan's
// activation path) -- one kernel, no separate gate pass.
template <int EPL>
__global__ void __launch_bounds__(256) rosa_step_kernel(RosaParams p) {
    const int bb = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (bb >= p.B) return;
    const int D = p.D;
    const int slot = p.slot ? p.slot[bb] : bb;
    const bool prepared = p.e_pre != nullptr;
    const bool gated = p.read_raw != nullptr || prepared;
    const size_t base = (size_t)bb * p.ld;
    float u[EPL], lam[EPL], m[EPL], ev[EPL], gv[EPL];
    float nrm = 0.0f;
#pragma unroll
    for (int e = 0; e < EPL; ++e) {
        const int c = lane + e * kWave;
        const bool ok = c < D;
        u[e] = ok ? p.direction[c] : 0.0f;
        lam[e] = ok ? p.decay[c] : 0.0f;
        m[e] = (ok && p.memory_in) ? p.memory_in[(size_t)slot * D + c] : 0.0f;
        ev[e] = ok ? (prepared ? p.e_pre : p.cand)[base + c] : 0.0f;
        gv[e] = ok ? (prepared ? p.g_pre : p.write)[base + c] : 0.0f;
        nrm = fmaf(u[e], u[e], nrm);
    }
    float rr[EPL];
#pragma unroll
    for (int e = 0; e < EPL; ++e) {
        const int c = lane + e * kWave;
        rr[e] = (c < D && gated && !prepared) ? p.read_raw[base + c] : 0.0f;
    }
    if (p.raw_params) {
        const float inv = 1.0f / fmaxf(sqrtf(wave_sum(nrm)), 1e-12f);
#pragma unroll
        for (int e = 0; e < EPL; ++e) {
            const int c = lane + e * kWave;
            u[e] *= inv;
            lam[e] = c < D ? 1.0f / (1.0f + expf(-lam[e])) : 0.0f;
        }
    }
    if (!prepared) {
#pragma unroll
        for (int e = 0; e < EPL; ++e) {
            const float th = 1.0f - 2.0f * __frcp_rn(__expf(2.0f * ev[e]) + 1.0f);
            ev[e] = th * __frcp_rn(1.0f + __expf(-gv[e]));
            gv[e] = gated ? __frcp_rn(1.0f + __expf(-rr[e])) : 1.0f;
        }
    }
    double f = 0.0;
#pragma unroll
    for (int e = 0; e < EPL; ++e) f = fma((double)u[e], (double)m[e], f);
    const float p1 = (float)wave_sum_f64(f);
    double f2 = 0.0;
#pragma unroll
    for (int e = 0; e < EPL; ++e) {
        m[e] = fmaf(lam[e], fmaf(-2.0f * p1, u[e], m[e]), ev[e]);
        f2 = fma((double)u[e], (double)m[e], f2);
    }
    const float p2 = (float)wave_sum_f64(f2);
#pragma unroll
    for (int e = 0; e < EPL; ++e) {
        const int c = lane + e * kWave;
        if (c < D) {
            p.read_out[(size_t)bb * D + c] = fmaf(-2.0f * p2, u[e], m[e]) * gv[e];
            if (p.memory_out) p.memory_out[(size_t)slot * D + c] = m[e];
        }
    }
}

// Segmented scan, carry pass.  With a constant transition A = diag(lambda) H,
// the state after segment s of length L is m_{s+1} = A^L m_s + z_s, where z_s
// is the segment's end state from a zero start.  One workgroup per chain walks
// its P segments: it records each segment's start state (carry) and applies
// A^L (row-major [D][D]) plus z_s.  D in {64, 128, 256}: blockDim = D * D / 64;
// thread (h, r) = (tid / D, tid % D) keeps the 64 entries of row r in column
// block h in registers, so the 64 lanes of a wave read the same 64 state
// values (LDS broadcasts).  The P steps are the chain, so a step only touches
// registers and LDS: the z rows are staged into LDS in blocks before the
// steps that use them (no global-load wait inside the chain, which would also
// wait for the carry stores in flight), the 64 state values are read before
// the FMAs (four independent chains), and the column blocks' partial sums
// meet in LDS in a fixed order.  Measured at the C3 layer shape (P = 32, D =
// 128): 21.5 -> 16.6 us, all of it from the launch bounds sized to the
// workgroup (the compiler had capped registers for 1024 threads and kept one
// or two state reads in flight); the z staging alone changed nothing.
template <int D>
__global__ void __launch_bounds__(D * D / 64) rosa_carry_kernel(int P, const float *AL, const float *z,
                                                                const float *memory_in, const int *slot, float *carry) {
    constexpr int kZFloats = 16384;  // staged z rows (64 KB)
    constexpr int nthr = D * D / 64, nb = D / 64;
    __shared__ __attribute__((aligned(16))) float st[2][D];
    __shared__ float part[nb][D];
    __shared__ __attribute__((aligned(16))) float zs[kZFloats];
    const int b = blockIdx.x, tid = threadIdx.x;
    const int h = tid / D, r = tid - h * D;
    float arow[64];
    const float4 *arow4 = reinterpret_cast<const float4 *>(AL + (size_t)r * D + h * 64);
#pragma unroll
    for (int j = 0; j < 16; ++j) {
        const float4 a4 = arow4[j];
        arow[4 * j] = a4.x; arow[4 * j + 1] = a4.y; arow[4 * j + 2] = a4.z; arow[4 * j + 3] = a4.w;
    }
    const int sl = slot ? slot[b] : b;
    if (tid < D) st[0][tid] = memory_in ? memory_in[(size_t)sl * D + tid] : 0.0f;
    constexpr int zb = kZFloats / D;  // steps per staged block
    for (int s0 = 0; s0 < P; s0 += zb) {
        const int n = min(zb, P - s0);
        const float4 *z4 = reinterpret_cast<const float4 *>(z + ((size_t)b * P + s0) * D);
        float4 *zs4 = reinterpret_cast<float4 *>(zs);
        const int total4 = n * D / 4;
        for (int i0 = 0; i0 < total4; i0 += 8 * nthr) {  // eight loads in flight per thread
            float4 t4[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) t4[u] = z4[min(i0 + u * nthr + tid, total4 - 1)];  // in bounds; extras unused
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const int i = i0 + u * nthr + tid;
                if (i < total4) zs4[i] = t4[u];
            }
        }
        // LDS-only barriers: the carry stores below stay in flight across them.
        lds_barrier();
        for (int k = 0; k < n; ++k) {
            const int s = s0 + k, cur = s & 1;
            const size_t v = (size_t)b * P + s;
            if (tid < D) carry[v * D + tid] = st[cur][tid];
            float x[64];
            const float4 *x4 = reinterpret_cast<const float4 *>(st[cur] + h * 64);
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                const float4 t = x4[j];
                x[4 * j] = t.x; x[4 * j + 1] = t.y; x[4 * j + 2] = t.z; x[4 * j + 3] = t.w;
            }
            float d4[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int j = 0; j < 64; j += 4)
#pragma unroll
                for (int q = 0; q < 4; ++q) d4[q] = fmaf(arow[j + q], x[j + q], d4[q]);
            const float dot = (d4[0] + d4[1]) + (d4[2] + d4[3]);
            if constexpr (nb == 1) {
                st[cur ^ 1][r] = dot + zs[k * D + r];
            } else {
                part[h][r] = dot;
                lds_barrier();
                if (h == 0) {
                    float sum = part[0][r];
#pragma unroll
                    for (int q = 1; q < nb; ++q) sum += part[q][r];
                    st[cur ^ 1][r] = sum + zs[k * D + r];
                }
            }
            lds_barrier();
        }
    }
}

// A^L of the ROSA transition for the operator path on its own (lambda
// post-sigmoid, u unit): wave w of workgroup g computes column 4 g + w.
template <int PER>
__global__ void __launch_bounds__(256) rosa_power_kernel(int D, int L, const float *lambda, const float *u, float *AL) {
    const int j = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (j >= D) return;  // uniform over the wave
    power_column<PER>(D, L, lambda, u, AL, j, lane);
}

hipError_t launch_rosa_power(int D, int L, const float *lambda, const float *u, float *AL, hipStream_t stream) {
    if (D < 1 || D > 1024 || L < 1) return hipErrorInvalidValue;
    const dim3 grid((D + 3) / 4), block(256);
    const int per = (D + 63) / 64;
    if (per <= 1) hipLaunchKernelGGL(rosa_power_kernel<1>, grid, block, 0, stream, D, L, lambda, u, AL);
    else if (per <= 2) hipLaunchKernelGGL(rosa_power_kernel<2>, grid, block, 0, stream, D, L, lambda, u, AL);
    else if (per <= 4) hipLaunchKernelGGL(rosa_power_kernel<4>, grid, block, 0, stream, D, L, lambda, u, AL);
    else if (per <= 8) hipLaunchKernelGGL(rosa_power_kernel<8>, grid, block, 0, stream, D, L, lambda, u, AL);
    else hipLaunchKernelGGL(rosa_power_kernel<16>, grid, block, 0, stream, D, L, lambda, u, AL);
    return hipGetLastError();
}

bool rosa_segmented_ok(int T, int D, int L) {
    return L > 0 && T % L == 0 && T / L >= 2 && (D == 64 || D == 128 || D == 256);
}

hipError_t launch_rosa_segmented(const RosaParams &p, const float *AL, int L, float *z, float *carry,
                                 hipStream_t stream) {
    if (p.B <= 0) return hipSuccess;
    if (!rosa_segmented_ok(p.T, p.D, L)) return hipErrorInvalidValue;
    const int P = p.T / L;
    // 1. every segment from a zero state: end states only.
    RosaParams a = p;
    a.B = p.B * P; a.T = L;
    a.memory_in = nullptr; a.slot = nullptr; a.memory_out = z; a.read_out = nullptr;
    hipError_t e = launch_rosa(a, stream);
    if (e != hipSuccess) return e;
    // 2. chain the segment start states.
    switch (p.D) {
        case 64: hipLaunchKernelGGL(rosa_carry_kernel<64>, dim3(p.B), dim3(64), 0, stream, P, AL, z, p.memory_in, p.slot, carry); break;
        case 128: hipLaunchKernelGGL(rosa_carry_kernel<128>, dim3(p.B), dim3(256), 0, stream, P, AL, z, p.memory_in, p.slot, carry); break;
        default: hipLaunchKernelGGL(rosa_carry_kernel<256>, dim3(p.B), dim3(1024), 0, stream, P, AL, z, p.memory_in, p.slot, carry); break;
    }
    if ((e = hipGetLastError()) != hipSuccess) return e;
    // 3. every segment again from its true start: the reads, and the last
    // segment's end state as the chain's new state.
    RosaParams c = p;
    c.B = p.B * P; c.T = L;
    c.memory_in = carry; c.slot = nullptr;
    c.seg = P; c.seg_slot = p.slot;
    return launch_rosa(c, stream);
}

namespace {
// Operator path: segment length of the segmented scan, and its scratch, one
// growing buffer per (device, stream) kept for the life of the process (a
// launch on a stream only ever waits on that stream's earlier work).
constexpr int kOpRosaSeg = 64;
std::mutex g_rosa_mu;
std::map<std::pair<int, hipStream_t>, std::pair<float *, size_t>> g_rosa_scratch;

bool op_rosa_sequential() {
    const char *e = std::getenv("YUF_ROSA_SEGMENTED");
    return e && std::strcmp(e, "0") == 0;
}

hipError_t op_rosa_scratch(hipStream_t stream, size_t floats, float **out) {
    int dev = 0;
    hipError_t err = hipGetDevice(&dev);
    if (err != hipSuccess) return err;
    std::lock_guard<std::mutex> lock(g_rosa_mu);
    auto &slot = g_rosa_scratch[{dev, stream}];
    if (slot.second < floats) {
        if (slot.first) {
            // Earlier launches on this stream may still read the old buffer.
            if ((err = hipStreamSynchronize(stream)) != hipSuccess) return err;
            (void)hipFree(slot.first);
            slot = {nullptr, 0};
        }
        float *p = nullptr;
        if ((err = hipMalloc(&p, floats * sizeof(float))) != hipSuccess) return err;
        slot = {p, floats};
    }
    *out = slot.first;
    return hipSuccess;
}
}  // namespace

hipError_t launch_rosa(const RosaParams &p, hipStream_t stream) {
    if (p.B <= 0) return hipSuccess;
    if (p.T == 1) {
        const dim3 grid((p.B + 3) / 4), block(256);
        const int epl = (p.D + kWave - 1) / kWave;
        if (epl <= 1) hipLaunchKernelGGL(rosa_step_kernel<1>, grid, block, 0, stream, p);
        else if (epl <= 2) hipLaunchKernelGGL(rosa_step_kernel<2>, grid, block, 0, stream, p);
        else if (epl <= 4) hipLaunchKernelGGL(rosa_step_kernel<4>, grid, block, 0, stream, p);
        else if (epl <= 8) hipLaunchKernelGGL(rosa_step_kernel<8>, grid, block, 0, stream, p);
        else if (epl <= 16) hipLaunchKernelGGL(rosa_step_kernel<16>, grid, block, 0, stream, p);
        else return hipErrorInvalidValue;
        return hipGetLastError();
    }
    const dim3 grid(p.B), block(kThreads);
    const int epl = (p.D + kWave - 1) / kWave;
    if (p.read_out) {
        if (epl <= 1) hipLaunchKernelGGL((rosa_scan_kernel<1, true>), grid, block, 0, stream, p);
        else if (epl <= 2) hipLaunchKernelGGL((rosa_scan_kernel<2, true>), grid, block, 0, stream, p);
        else if (epl <= 4) hipLaunchKernelGGL((rosa_scan_kernel<4, true>), grid, block, 0, stream, p);
        else if (epl <= 8) hipLaunchKernelGGL((rosa_scan_kernel<8, true>), grid, block, 0, stream, p);
        else if (epl <= 16) hipLaunchKernelGGL((rosa_scan_kernel<16, true>), grid, block, 0, stream, p);
        else return hipErrorInvalidValue;
    } else {
        if (epl <= 1) hipLaunchKernelGGL((rosa_scan_kernel<1, false>), grid, block, 0, stream, p);
        else if (epl <= 2) hipLaunchKernelGGL((rosa_scan_kernel<2, false>), grid, block, 0, stream, p);
        else if (epl <= 4) hipLaunchKernelGGL((rosa_scan_kernel<4, false>), grid, block, 0, stream, p);
        else if (epl <= 8) hipLaunchKernelGGL((rosa_scan_kernel<8, false>), grid, block, 0, stream, p);
        else if (epl <= 16) hipLaunchKernelGGL((rosa_scan_kernel<16, false>), grid, block, 0, stream, p);
        else return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace yuf

namespace yuf {
namespace {

// The no-allocation operator variant (yuf_rosa_scan_f32_noalloc) keeps the
// segmented scan's scratch -- A^L and the z / carry segment rows -- in
// this file-scope device array: every device the library runs on holds one
// copy, at its own address, until the process ends.  Nothing in it needs to
// start at zero (each pass writes its rows before the next reads them).
constexpr size_t kNoAllocScratchFloats = (size_t)4 << 20;  // 16 MiB
__device__ __align__(256) float scratch[kNoAllocScratchFloats];

// Device address of `scratch` per device, resolved once per device with that
// device current (the array's name is a host-side stand-in, never passed to a
// kernel).  Fixed storage: no host or device allocation on this path.
constexpr int kNoAllocMaxDevices = 64;
std::mutex g_noalloc_mu;
float *g_noalloc_ptr[kNoAllocMaxDevices] = {};

int noalloc_scratch(float **out) {
    int dev = 0;
    hipError_t err = hipGetDevice(&dev);
    if (err != hipSuccess) return fail(YUF_ERR_HIP, std::string("rosa noalloc: hipGetDevice: ") + hipGetErrorString(err));
    if (dev < 0 || dev >= kNoAllocMaxDevices) return fail(YUF_ERR_INVALID, "rosa noalloc: device index above 63");
    std::lock_guard<std::mutex> lock(g_noalloc_mu);
    if (!g_noalloc_ptr[dev]) {
        void *ptr = nullptr;
        err = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (err != hipSuccess || !ptr)
            return fail(YUF_ERR_HIP, std::string("rosa noalloc: hipGetSymbolAddress: ") + hipGetErrorString(err));
        g_noalloc_ptr[dev] = static_cast<float *>(ptr);
    }
    *out = g_noalloc_ptr[dev];
    return YUF_OK;
}

// The operator: argument checks, then the segmented form (scratch from the
// growing per-stream buffer, or from `scratch` when noalloc) or the
// sequential chunked scan (no scratch).  The no-allocation variant does not
// read YUF_ROSA_SEGMENTED: its scratch capacity is checked on every call that
// can take the segmented form, before any launch, whatever the switch says.
int rosa_operator(int B, int T, int D, const float *cand, const float *write, const float *read_raw,
                  const float *decay, const float *direction, const float *memory_in, float *memory_out,
                  float *read_out, void *stream, bool noalloc) {
    if (B < 0 || T < 0) return fail(YUF_ERR_INVALID, "rosa: negative size");
    if (D < 1 || D > 1024) return fail(YUF_ERR_INVALID, "rosa: D must be in [1, 1024], got " + std::to_string(D));
    if (!decay || !direction) return fail(YUF_ERR_INVALID, "rosa: null decay/direction");
    if (T > 0 && (!cand || !write || !read_out)) return fail(YUF_ERR_INVALID, "rosa: null input/output pointer");
    RosaParams p;
    p.B = B; p.T = T; p.D = D; p.ld = D;
    p.cand = cand; p.write = write; p.read_raw = read_raw;
    p.decay = decay; p.direction = direction;
    p.memory_in = memory_in; p.memory_out = memory_out; p.read_out = read_out;
    const hipStream_t st = static_cast<hipStream_t>(stream);
    hipError_t err;
    if (B > 0 && rosa_segmented_ok(T, D, kOpRosaSeg) && (noalloc || !op_rosa_sequential())) {
        // Segmented form (as the engine's prefill): A^L on the device, then
        // segments from zero, the carry chain, and segments from their starts.
        float *buf = nullptr;
        const size_t seg = (size_t)B * (T / kOpRosaSeg) * D;
        const size_t need = (size_t)D * D + 2 * seg;
        if (noalloc) {
            if (need > kNoAllocScratchFloats)
                return fail(YUF_ERR_INVALID, "rosa noalloc: B * (T / 64) * D = " + std::to_string(seg) +
                                                 " needs " + std::to_string(need) + " scratch floats (D^2 + 2 B (T / 64) D); "
                                                 "the static buffer holds " + std::to_string(kNoAllocScratchFloats) +
                                                 " -- split the batch or use yuf_rosa_scan_f32");
            int rc = noalloc_scratch(&buf);
            if (rc != YUF_OK) return rc;
        } else if ((err = op_rosa_scratch(st, need, &buf)) != hipSuccess) {
            return fail(YUF_ERR_OOM, std::string("rosa scratch: ") + hipGetErrorString(err));
        }
        float *AL = buf, *z = AL + (size_t)D * D, *carry = z + seg;
        // A^L in its own launch (as extra workgroups of the first pass it
        // measured no faster: 21.2-21.4 us against 8.5 + 13.9 us).
        err = launch_rosa_power(D, kOpRosaSeg, decay, direction, AL, st);
        if (err == hipSuccess) err = launch_rosa_segmented(p, AL, kOpRosaSeg, z, carry, st);
    } else {
        err = launch_rosa(p, st);
    }
    if (err != hipSuccess) return fail(YUF_ERR_HIP, std::string("rosa launch: ") + hipGetErrorString(err));
    return YUF_OK;
}

}  // namespace
}  // namespace yuf

extern "C" int yuf_rosa_scan_f32(int B, int T, int D, const float *cand, const float *write,
                                 const float *read_raw, const float *decay, const float *direction,
                                 const float *memory_in, float *memory_out, float *read_out, void *stream) {
    return yuf::rosa_operator(B, T, D, cand, write, read_raw, decay, direction, memory_in, memory_out, read_out,
                              stream, false);
}

extern "C" int yuf_rosa_scan_f32_noalloc(int B, int T, int D, const float *cand, const float *write,
                                         const float *read_raw, const float *decay, const float *direction,
                                         const float *memory_in, float *memory_out, float *read_out, void *stream) {
    return yuf::rosa_operator(B, T, D, cand, write, read_raw, decay, direction, memory_in, memory_out, read_out,
                              stream, true);
}
