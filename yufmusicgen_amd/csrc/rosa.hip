// ROSA Householder memory scan for gfx950 (MI355X).
//
// Semantics: yufmusicgen/model.py:260-288 (reference recurrence) and the read
// of model.py:303-311 / yufmusicgen/cuda/rosa_householder.cu:30-101:
//     m_t    = lambda * H(m_{t-1}) + sigmoid(write_t) * tanh(cand_t)
//     read_t = H(m_t) [* sigmoid(read_raw_t)],     H(x) = x - 2 (x.u) u.
//
// Design: one wave per stream; a lane owns D / 64 memory channels (strided,
// so every per-token HBM access is a coalesced 256 B row).  The reference
// kernel recomputes two O(D) dot products in every thread for every token
// (O(D^2) work per token); here each token needs exactly ONE wave reduction,
// because the projection used by the read at token t, m_t.u, is also the
// projection the update at token t+1 needs.  The write term and the read gate
// are computed in the 16-token staging pass (off the sequential chain), and the
// next chunk's pre-activations are loaded while the current chunk runs.
#include "common.h"
#include "kernels.h"

namespace yuf {
namespace {

constexpr int kWave = 64;
// Tokens per staging chunk: 16, fewer for wide memories to bound registers.
template <int EPL>
constexpr int chunk_len() { return EPL <= 2 ? 16 : 32 / EPL; }

template <int EPL>
__global__ void __launch_bounds__(kWave) rosa_scan_kernel(RosaParams p) {
    constexpr int kChunk = chunk_len<EPL>();
    const int bb = blockIdx.x;
    const int lane = threadIdx.x;
    const int D = p.D;
    const int slot = p.slot ? p.slot[bb] : bb;

    float lam[EPL], u[EPL], m[EPL];
    // Direction and decay.  Model path: u = householder / max(|householder|, 1e-12),
    // lambda = sigmoid(decay_param) (model.py:300-301).
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
        const float inv = 1.0f / fmaxf(sqrtf(wave_sum(nrm)), 1e-12f);
#pragma unroll
        for (int e = 0; e < EPL; ++e) {
            u[e] *= inv;
            lam[e] = 1.0f / (1.0f + expf(-lam[e]));
        }
    }
    // Projection of the incoming memory.
    float proj = 0.0f;
#pragma unroll
    for (int e = 0; e < EPL; ++e) proj = fmaf(m[e], u[e], proj);
    proj = wave_sum(proj);

    const bool gated = p.read_raw != nullptr;
    float pc[kChunk][EPL], pw[kChunk][EPL], pr[kChunk][EPL];
    auto load_chunk = [&](int t0, int nt) {
        // Rows past the chunk end and channels past D fall outside the buffer
        // descriptors and load as 0, so they contribute nothing to reductions.
        const size_t base = (size_t)(bb * p.T + t0) * p.ld;
        const uint32_t bytes = nt > 0 ? (uint32_t)(((nt - 1) * p.ld + D) * 4) : 0u;
        const auto rc = make_rsrc(p.cand + base, bytes), rw = make_rsrc(p.write + base, bytes);
        const auto rr = make_rsrc(gated ? p.read_raw + base : p.cand + base, gated ? bytes : 0u);
#pragma unroll
        for (int t = 0; t < kChunk; ++t) {
#pragma unroll
            for (int e = 0; e < EPL; ++e) {
                const int c = lane + e * kWave;
                const uint32_t off = c < D ? (uint32_t)(t * p.ld + c) * 4u : kBufferOob;
                pc[t][e] = buf_load(rc, off);
                pw[t][e] = buf_load(rw, off);
                pr[t][e] = buf_load(rr, off);
            }
        }
    };
    const int n_chunks = (p.T + kChunk - 1) / kChunk;
    if (n_chunks > 0) load_chunk(0, min(kChunk, p.T));
    for (int ch = 0; ch < n_chunks; ++ch) {
        const int t0 = ch * kChunk;
        const int nt = min(kChunk, p.T - t0);
        // Off-chain transforms of this chunk: write term and read gate.
        float ew[kChunk][EPL], g[kChunk][EPL];
#pragma unroll
        for (int t = 0; t < kChunk; ++t) {
#pragma unroll
            for (int e = 0; e < EPL; ++e) {
                // tanh(x) = 1 - 2 / (e^{2x} + 1); sigmoid(x) = 1 / (1 + e^{-x}).
                const float th = 1.0f - 2.0f * __frcp_rn(__expf(2.0f * pc[t][e]) + 1.0f);
                ew[t][e] = th * __frcp_rn(1.0f + __expf(-pw[t][e]));
                g[t][e] = gated ? __frcp_rn(1.0f + __expf(-pr[t][e])) : 1.0f;
            }
        }
        if (ch + 1 < n_chunks) load_chunk(t0 + kChunk, min(kChunk, p.T - t0 - kChunk));
        for (int t = 0; t < nt; ++t) {
            float q = 0.0f;
#pragma unroll
            for (int e = 0; e < EPL; ++e) {
                m[e] = fmaf(lam[e], m[e] - 2.0f * proj * u[e], ew[t][e]);
                q = fmaf(m[e], u[e], q);
            }
            proj = wave_sum(q);
            const size_t row = (size_t)(bb * p.T + t0 + t) * D;
#pragma unroll
            for (int e = 0; e < EPL; ++e) {
                const int c = lane + e * kWave;
                if (c < D) p.read_out[row + c] = (m[e] - 2.0f * proj * u[e]) * g[t][e];
            }
        }
    }
    if (p.memory_out) {
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
    const dim3 grid(p.B), block(kWave);
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
