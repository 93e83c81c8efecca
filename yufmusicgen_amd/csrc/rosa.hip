// ROSA Householder memory scan for gfx950 (MI355X).
//
// Semantics: yufmusicgen/model.py:260-288 (reference recurrence) and the read
// of model.py:303-311 / yufmusicgen/cuda/rosa_householder.cu:30-101:
//     m_t    = lambda * H(m_{t-1}) + sigmoid(write_t) * tanh(cand_t)
//     read_t = H(m_t) [* sigmoid(read_raw_t)],     H(x) = x - 2 (x.u) u.
//
// Design: one 4-wave workgroup per stream.  Wave 0 runs the sequential chain
// and nothing else: per token one FMA pair per channel, ONE wave reduction (the
// projection m_t.u serves both the read of token t and the update of token
// t+1 -- the reference recomputes two O(D) dot products in every thread), the
// gated read and a buffer store.  Waves 1-3 are producers: while wave 0 runs
// chunk c they load chunk c+1's pre-activations from HBM and turn them into
// the write term sigmoid(w) tanh(c) and the gate sigmoid(rho) in LDS (double
// buffered), so no transcendental and no HBM latency sits on the chain.  Chunk
// length is 32 tokens for D <= 256 and shrinks for wider memories so the two
// LDS buffers stay within 128 KB.
#include "common.h"
#include "kernels.h"

namespace yuf {
namespace {

constexpr int kWave = 64;
constexpr int kWaves = 4;
constexpr int kProducers = (kWaves - 1) * kWave;

template <int EPL>
constexpr int chunk_len() { return EPL <= 4 ? 32 : 64 / EPL; }

template <int EPL>
__global__ void __launch_bounds__(kWaves * kWave) rosa_scan_kernel(RosaParams p) {
    constexpr int C = chunk_len<EPL>();
    constexpr int DP = EPL * kWave;  // padded channel count
    // [buffer][token][channel] write term and read gate.
    __shared__ __attribute__((aligned(16))) float ew[2][C * DP];
    __shared__ __attribute__((aligned(16))) float gt[2][C * DP];

    const int bb = blockIdx.x;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int D = p.D;
    const int slot = p.slot ? p.slot[bb] : bb;
    const bool gated = p.read_raw != nullptr;
    const int n_chunks = (p.T + C - 1) / C;

    // Producers: chunk -> LDS buffer.  Channels past D and tokens past T are 0.
    auto produce = [&](int ch, int buf) {
        const int t0 = ch * C, nt = min(C, p.T - t0);
        const size_t base = (size_t)(bb * p.T + t0) * p.ld;
        const uint32_t bytes = (uint32_t)(((nt - 1) * p.ld + D) * 4);
        const auto rc = make_rsrc(p.cand + base, bytes), rw = make_rsrc(p.write + base, bytes);
        const auto rr = make_rsrc(gated ? p.read_raw + base : p.cand + base, gated ? bytes : 0u);
        for (int q = tid - kWave; q < C * DP; q += kProducers) {
            const int t = q / DP, c = q - t * DP;
            const uint32_t off = (c < D && t < nt) ? (uint32_t)(t * p.ld + c) * 4u : kBufferOob;
            const float cv = buf_load(rc, off), wv = buf_load(rw, off), rv = buf_load(rr, off);
            // tanh(x) = 1 - 2 / (e^{2x} + 1); sigmoid(x) = 1 / (1 + e^{-x}).
            const float th = 1.0f - 2.0f * __frcp_rn(__expf(2.0f * cv) + 1.0f);
            ew[buf][q] = th * __frcp_rn(1.0f + __expf(-wv));
            gt[buf][q] = gated ? __frcp_rn(1.0f + __expf(-rv)) : 1.0f;
        }
    };

    // Consumer state: lane owns channels lane + 64 e.
    float lam[EPL], u[EPL], m[EPL];
    float proj = 0.0f;
    if (wave == 0) {
        float nrm = 0.0f;
#pragma unroll
        for (int e = 0; e < EPL; ++e) {
            const int c = lane + e * kWave;
            const bool ok = c < D;
            u[e] = ok ? p.direction[c] : 0.0f;
            lam[e] = ok ? p.decay[c] : 0.0f;
            m[e] = (ok && p.memory_in) ? p.memory_in[(size_t)slot * D + c] : 0.0f;
            nrm = fmaf(u[e], u[e], nrm);
        }
        if (p.raw_params) {
            // Model path: u = householder / max(|householder|, 1e-12), lambda = sigmoid(decay)
            // (model.py:300-301).
            const float inv = 1.0f / fmaxf(sqrtf(wave_sum(nrm)), 1e-12f);
#pragma unroll
            for (int e = 0; e < EPL; ++e) {
                u[e] *= inv;
                lam[e] = 1.0f / (1.0f + expf(-lam[e]));
            }
        }
#pragma unroll
        for (int e = 0; e < EPL; ++e) proj = fmaf(m[e], u[e], proj);
        proj = wave_sum(proj);
        wait_vmem();
    } else if (n_chunks > 0) {
        produce(0, 0);
    }
    lds_barrier();

    for (int ch = 0; ch < n_chunks; ++ch) {
        const int buf = ch & 1;
        if (wave == 0) {
            const int t0 = ch * C, nt = min(C, p.T - t0);
            const size_t obase = (size_t)(bb * p.T + t0) * D;
            const auto ro = make_rsrc(p.read_out + obase, (uint32_t)(nt * D * 4));
            const float *e_row = ew[buf] + lane;
            const float *g_row = gt[buf] + lane;
            for (int t = 0; t < nt; ++t) {
                float q = 0.0f;
                const float two_p = 2.0f * proj;
#pragma unroll
                for (int e = 0; e < EPL; ++e) {
                    m[e] = fmaf(lam[e], fmaf(-two_p, u[e], m[e]), e_row[t * DP + e * kWave]);
                    q = fmaf(m[e], u[e], q);
                }
                proj = wave_sum(q);
                const float two_q = 2.0f * proj;
#pragma unroll
                for (int e = 0; e < EPL; ++e) {
                    const int c = lane + e * kWave;
                    const float rv = fmaf(-two_q, u[e], m[e]) * g_row[t * DP + e * kWave];
                    buf_store(rv, ro, c < D ? (uint32_t)(t * D + c) * 4u : kBufferOob);
                }
            }
        } else if (ch + 1 < n_chunks) {
            produce(ch + 1, buf ^ 1);
        }
        lds_barrier();
    }
    if (wave == 0 && p.memory_out) {
#pragma unroll
        for (int e = 0; e < EPL; ++e) {
            const int c = lane + e * kWave;
            if (c < D) p.memory_out[(size_t)slot * D + c] = m[e];
        }
    }
}

}  // namespace

hipError_t launch_rosa(const RosaParams &p, hipStream_t stream) {
    if (p.B <= 0) return hipSuccess;
    const dim3 grid(p.B), block(kWaves * kWave);
    const int epl = (p.D + kWave - 1) / kWave;
    if (epl <= 1) hipLaunchKernelGGL(rosa_scan_kernel<1>, grid, block, 0, stream, p);
    else if (epl <= 2) hipLaunchKernelGGL(rosa_scan_kernel<2>, grid, block, 0, stream, p);
    else if (epl <= 4) hipLaunchKernelGGL(rosa_scan_kernel<4>, grid, block, 0, stream, p);
    else if (epl <= 8) hipLaunchKernelGGL(rosa_scan_kernel<8>, grid, block, 0, stream, p);
    else if (epl <= 16) hipLaunchKernelGGL(rosa_scan_kernel<16>, grid, block, 0, stream, p);
    else return hipErrorInvalidValue;
    return hipGetLastError();
}

}  // namespace yuf

extern "C" int yuf_rosa_scan_f32(int B, int T, int D, const float *cand, const float *write,
                                 const float *read_raw, const float *decay, const float *direction,
                                 const float *memory_in, float *memory_out, float *read_out, void *stream) {
    using namespace yuf;
    if (B < 0 || T < 0) return fail(YUF_ERR_INVALID, "rosa: negative size");
    if (D < 1 || D > 1024) return fail(YUF_ERR_INVALID, "rosa: D must be in [1, 1024], got " + std::to_string(D));
    if (!decay || !direction) return fail(YUF_ERR_INVALID, "rosa: null decay/direction");
    if (T > 0 && (!cand || !write || !read_out)) return fail(YUF_ERR_INVALID, "rosa: null input/output pointer");
    RosaParams p;
    p.B = B; p.T = T; p.D = D; p.ld = D;
    p.cand = cand; p.write = write; p.read_raw = read_raw;
    p.decay = decay; p.direction = direction;
    p.memory_in = memory_in; p.memory_out = memory_out; p.read_out = read_out;
    hipError_t err = launch_rosa(p, static_cast<hipStream_t>(stream));
    if (err != hipSuccess) return fail(YUF_ERR_HIP, std::string("rosa launch: ") + hipGetErrorString(err));
    return YUF_OK;
}
