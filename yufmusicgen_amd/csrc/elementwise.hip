// Memory-bound helper kernels of the model path (gfx950): embedding gather,
// LayerNorm (+ gate), token shift, state bookkeeping, fills.
//
// Semantics: yufmusicgen/model.py:417 (embedding), nn.LayerNorm eps 1e-5
// (model.py:89, :346-356, :391), token shift model.py:98-105 (sign of
// x + (x - x_prev) * mu), the carried `previous` of model.py:197 and the
// gated output norm of model.py:195-196.
#include "common.h"
#include "kernels.h"

namespace yuf {
namespace {

constexpr int kWave = 64;

// One wave per row; rows of width d <= 64 * kMaxPerLane.
constexpr int kMaxPerLane = 32;

template <int PER>
__global__ void __launch_bounds__(256) layernorm_kernel(const float *x, int M, int d, const float *gamma,
                                                        const float *beta, const float *gate, float *out) {
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= M) return;
    const float *xr = x + (size_t)row * d;
    float v[PER];
    float sum = 0.0f;
#pragma unroll
    for (int e = 0; e < PER; ++e) {
        const int c = lane + e * kWave;
        v[e] = c < d ? xr[c] : 0.0f;
        sum += v[e];
    }
    const float mean = wave_sum(sum) / (float)d;
    float sq = 0.0f;
#pragma unroll
    for (int e = 0; e < PER; ++e) {
        const int c = lane + e * kWave;
        const float dv = c < d ? v[e] - mean : 0.0f;
        sq = fmaf(dv, dv, sq);
    }
    const float rstd = rsqrtf(wave_sum(sq) / (float)d + 1e-5f);
    float *orow = out + (size_t)row * d;
    const float *grow = gate ? gate + (size_t)row * d : nullptr;
#pragma unroll
    for (int e = 0; e < PER; ++e) {
        const int c = lane + e * kWave;
        if (c < d) {
            float y = (v[e] - mean) * rstd * gamma[c] + beta[c];
            if (grow) y *= grow[c];
            orow[c] = y;
        }
    }
}

// Single-token step (T = 1): LayerNorm of row b, the six token-shift mixes
// against prev_state[slot[b]] (as token_shift_kernel), and prev_state[slot[b]]
// <- the normed row (yufmusicgen/model.py:97-105, :197), one 256-thread
// workgroup per row.  Every load (row, previous row, affine, mixes) is issued
// before the first store, so the kernel costs one memory round trip; each
// thread reads a column's previous value before it overwrites it.
constexpr int kMaxParts = 4;  // K-split partial planes ln_shift_kernel can add

template <int PER>
__global__ void __launch_bounds__(256) ln_shift_kernel(float *__restrict__ x, int d,
                                                       const float *__restrict__ gamma,
                                                       const float *__restrict__ beta, float *__restrict__ prev_state,
                                                       const int *__restrict__ slot, const float *__restrict__ mix6,
                                                       float *__restrict__ out6, size_t out_stride,
                                                       const float *__restrict__ parts, size_t part_stride,
                                                       int nparts, bool out_tiled) {
    __shared__ float part[2][4];
    const int row = blockIdx.x, tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    float *xr = x + (size_t)row * d;
    float *prow = prev_state + (size_t)(slot ? slot[row] : row) * d;
    float v[PER], pv[PER], gm[PER], bt[PER], mx[6][PER];
    float sum = 0.0f;
#pragma unroll
    for (int e = 0; e < PER; ++e) {
        const int c = tid + e * 256;
        const bool ok = c < d;
        v[e] = ok ? xr[c] : 0.0f;
        pv[e] = ok ? prow[c] : 0.0f;
        gm[e] = ok ? gamma[c] : 0.0f;
        bt[e] = ok ? beta[c] : 0.0f;
#pragma unroll
        for (int q = 0; q < 6; ++q) mx[q][e] = ok ? mix6[q * d + c] : 0.0f;
    }
    // Pending K-split partial sums of the previous product (h += P0 + P1 + ...,
    // in order): loaded with the row (unused parts read as zero outside the
    // descriptor), the row is completed and written back before it is normed.
    float pp[kMaxParts][PER];
    const auto rpart = make_rsrc(parts ? parts + (size_t)row * d : nullptr,
                                 parts ? (uint32_t)(((size_t)(kMaxParts - 1) * part_stride + d) * 4) : 0u);
#pragma unroll
    for (int q = 0; q < kMaxParts; ++q)
#pragma unroll
        for (int e = 0; e < PER; ++e) {
            const int c = tid + e * 256;
            pp[q][e] = buf_load(rpart, q < nparts && c < d ? (uint32_t)((size_t)q * part_stride + c) * 4u : kBufferOob);
        }
#pragma unroll
    for (int q = 0; q < kMaxParts; ++q)
        if (q < nparts) {
#pragma unroll
            for (int e = 0; e < PER; ++e) v[e] += pp[q][e];
        }
#pragma unroll
    for (int e = 0; e < PER; ++e) {
        const int c = tid + e * 256;
        if (nparts > 0 && c < d) xr[c] = v[e];
        sum += v[e];
    }
    sum = wave_sum(sum);
    if (lane == 0) part[0][wave] = sum;
    lds_barrier();
    const float mean = ((part[0][0] + part[0][1]) + (part[0][2] + part[0][3])) / (float)d;
    float sq = 0.0f;
#pragma unroll
    for (int e = 0; e < PER; ++e) {
        const float dv = tid + e * 256 < d ? v[e] - mean : 0.0f;
        sq = fmaf(dv, dv, sq);
    }
    sq = wave_sum(sq);
    if (lane == 0) part[1][wave] = sq;
    lds_barrier();
    const float rstd = rsqrtf(((part[1][0] + part[1][1]) + (part[1][2] + part[1][3])) / (float)d + 1e-5f);
#pragma unroll
    for (int e = 0; e < PER; ++e) {
        const int c = tid + e * 256;
        if (c < d) {
            const float xv = (v[e] - mean) * rstd * gm[e] + bt[e];
            const float delta = xv - pv[e];
            const size_t o = out_tiled ? tile_index(row, c, d) : (size_t)row * d + c;
#pragma unroll
            for (int q = 0; q < 6; ++q) out6[q * out_stride + o] = fmaf(delta, mx[q][e], xv);
            prow[c] = xv;
        }
    }
}

__global__ void embed_kernel(const int *tokens, int M, const float *table, int d, int vocab, float *out,
                             int *bad) {
    const int row = blockIdx.x;
    if (row >= M) return;
    const int tok = tokens[row];
    const bool ok = tok >= 0 && tok < vocab;
    if (!ok && threadIdx.x == 0 && bad) atomicOr(bad, 1);
    const float *src = table + (size_t)(ok ? tok : 0) * d;
    float *dst = out + (size_t)row * d;
    for (int c = threadIdx.x; c < d; c += blockDim.x) dst[c] = ok ? src[c] : 0.0f;
}

// Prefill (T > 1) fusion of layernorm_kernel -> token_shift_kernel: each wave
// walks a run of R consecutive tokens of one sequence, normalizing every row
// with layernorm_kernel's expressions and reduction order (same bits) and
// mixing it against the previous normed row it still holds in registers (the
// run's first row against prev_state[slot[b]] at t = 0, else against its
// recomputed predecessor); the normed rows never go to memory.  The wave whose
// run ends the sequence writes that row to last_xn[b] for save_prev, which
// runs afterwards (no wave overwrites prev_state while another may read it).
template <int PER>
__global__ void __launch_bounds__(256) ln_shift_seq_kernel(const float *__restrict__ x, int Bn, int T, int d, int R,
                                                           const float *__restrict__ gamma,
                                                           const float *__restrict__ beta,
                                                           const float *__restrict__ prev_state,
                                                           const int *__restrict__ slot,
                                                           const float *__restrict__ mix6, float *__restrict__ out6,
                                                           size_t out_stride, float *__restrict__ last_xn) {
    const int runs = (T + R - 1) / R;
    const int gw = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (gw >= Bn * runs) return;  // uniform over the wave; no barriers below
    const int b = gw / runs, t0 = (gw - b * runs) * R, t1 = min(T, t0 + R);
    float gm[PER], bt[PER], mx[6][PER];
#pragma unroll
    for (int e = 0; e < PER; ++e) {
        const int c = lane + e * kWave;
        const bool ok = c < d;
        gm[e] = ok ? gamma[c] : 0.0f;
        bt[e] = ok ? beta[c] : 0.0f;
#pragma unroll
        for (int q = 0; q < 6; ++q) mx[q][e] = ok ? mix6[q * d + c] : 0.0f;
    }
    auto load_row = [&](int t, float (&v)[PER]) {
        const float *xr = x + ((size_t)b * T + t) * d;
#pragma unroll
        for (int e = 0; e < PER; ++e) {
            const int c = lane + e * kWave;
            v[e] = c < d ? xr[c] : 0.0f;
        }
    };
    auto norm = [&](float (&v)[PER]) {
        float sum = 0.0f;
#pragma unroll
        for (int e = 0; e < PER; ++e) sum += v[e];
        const float mean = wave_sum(sum) / (float)d;
        float sq = 0.0f;
#pragma unroll
        for (int e = 0; e < PER; ++e) {
            const float dv = lane + e * kWave < d ? v[e] - mean : 0.0f;
            sq = fmaf(dv, dv, sq);
        }
        const float rstd = rsqrtf(wave_sum(sq) / (float)d + 1e-5f);
#pragma unroll
        for (int e = 0; e < PER; ++e) v[e] = (v[e] - mean) * rstd * gm[e] + bt[e];
    };
    float pv[PER], cur[PER], nxt[PER] = {};
    if (t0 == 0) {
        const float *prow = prev_state + (size_t)(slot ? slot[b] : b) * d;
#pragma unroll
        for (int e = 0; e < PER; ++e) {
            const int c = lane + e * kWave;
            pv[e] = c < d ? prow[c] : 0.0f;
        }
    } else {
        load_row(t0 - 1, pv);
        norm(pv);
    }
    load_row(t0, cur);
    for (int t = t0; t < t1; ++t) {
        if (t + 1 < t1) load_row(t + 1, nxt);
        norm(cur);
        float *orow = out6 + ((size_t)b * T + t) * d;
#pragma unroll
        for (int e = 0; e < PER; ++e) {
            const int c = lane + e * kWave;
            if (c < d) {
                const float delta = cur[e] - pv[e];
#pragma unroll
                for (int q = 0; q < 6; ++q) orow[q * out_stride + c] = fmaf(delta, mx[q][e], cur[e]);
            }
            pv[e] = cur[e];
            cur[e] = nxt[e];
        }
    }
    if (t1 == T) {
#pragma unroll
        for (int e = 0; e < PER; ++e) {
            const int c = lane + e * kWave;
            if (c < d) last_xn[(size_t)b * d + c] = pv[e];
        }
    }
}

__global__ void token_shift_kernel(const float *x, int Bn, int T, int d, const float *prev_state, const int *slot,
                                   const float *mix6, float *out6, size_t out_stride) {
    const size_t total = (size_t)Bn * T * d;
    for (size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
         idx += (size_t)gridDim.x * blockDim.x) {
        const size_t m = idx / d;
        const int c = (int)(idx - m * d);
        const int b = (int)(m / T), t = (int)(m - (size_t)b * T);
        const float xv = x[idx];
        const float pv = t > 0 ? x[idx - d] : prev_state[(size_t)(slot ? slot[b] : b) * d + c];
        const float delta = xv - pv;
#pragma unroll
        for (int q = 0; q < 6; ++q) out6[q * out_stride + idx] = fmaf(delta, mix6[q * d + c], xv);
    }
}

__global__ void save_prev_kernel(const float *x, int Bn, int T, int d, float *prev_state, const int *slot) {
    const int b = blockIdx.x;
    if (b >= Bn) return;
    const float *src = x + ((size_t)b * T + T - 1) * d;
    float *dst = prev_state + (size_t)(slot ? slot[b] : b) * d;
    for (int c = threadIdx.x; c < d; c += blockDim.x) dst[c] = src[c];
}

__global__ void gather_last_kernel(const float *x, int Bn, int T, int d, float *out) {
    const int b = blockIdx.x;
    if (b >= Bn) return;
    const float *src = x + ((size_t)b * T + T - 1) * d;
    for (int c = threadIdx.x; c < d; c += blockDim.x) out[(size_t)b * d + c] = src[c];
}

__global__ void fill_kernel(float *p, size_t n, float value) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
        p[i] = value;
}

// ROSA gates in place: row r of x holds [cand | write | read_raw] (D each, row
// stride ld); cand becomes e = tanh(cand) sigmoid(write) and write becomes the
// read gate sigmoid(read_raw) (yufmusicgen/model.py:303-311; the same float
// expressions as the scan kernel's own activation path).
__global__ void rosa_gates_kernel(float *x, int M, int D, int ld) {
    const size_t n = (size_t)M * D;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
        const int r = (int)(i / D), c = (int)(i - (size_t)r * D);
        float *row = x + (size_t)r * ld;
        const float cv = row[c], wv = row[D + c], rv = row[2 * D + c];
        const float th = 1.0f - 2.0f * __frcp_rn(__expf(2.0f * cv) + 1.0f);
        row[c] = th * __frcp_rn(1.0f + __expf(-wv));
        row[D + c] = __frcp_rn(1.0f + __expf(-rv));
    }
}

int grid_for(size_t n, int block) {
    size_t g = (n + block - 1) / block;
    return (int)(g < 65536 ? (g > 0 ? g : 1) : 65536);
}

}  // namespace

hipError_t launch_layernorm(const float *x, int M, int d, const float *gamma, const float *beta, const float *gate,
                            float *out, hipStream_t stream) {
    if (M <= 0) return hipSuccess;
    const int per = (d + kWave - 1) / kWave;
    const dim3 grid((M + 3) / 4), block(256);
    if (per <= 2) hipLaunchKernelGGL(layernorm_kernel<2>, grid, block, 0, stream, x, M, d, gamma, beta, gate, out);
    else if (per <= 4) hipLaunchKernelGGL(layernorm_kernel<4>, grid, block, 0, stream, x, M, d, gamma, beta, gate, out);
    else if (per <= 8) hipLaunchKernelGGL(layernorm_kernel<8>, grid, block, 0, stream, x, M, d, gamma, beta, gate, out);
    else if (per <= 10) hipLaunchKernelGGL(layernorm_kernel<10>, grid, block, 0, stream, x, M, d, gamma, beta, gate, out);
    else if (per <= 16) hipLaunchKernelGGL(layernorm_kernel<16>, grid, block, 0, stream, x, M, d, gamma, beta, gate, out);
    else if (per <= kMaxPerLane)
        hipLaunchKernelGGL(layernorm_kernel<kMaxPerLane>, grid, block, 0, stream, x, M, d, gamma, beta, gate, out);
    else return hipErrorInvalidValue;
    return hipGetLastError();
}

hipError_t launch_ln_shift(float *x, int n, int d, const float *gamma, const float *beta, float *prev_state,
                           const int *slot, const float *mix6, float *out6, size_t out_stride, const float *parts,
                           size_t part_stride, int nparts, bool out_tiled, hipStream_t stream) {
    if (n <= 0) return hipSuccess;
    if (nparts < 0 || nparts > kMaxParts || (nparts > 0 && !parts)) return hipErrorInvalidValue;
    if (out_tiled && (d % 16 != 0 || out_stride < (size_t)((n + 15) / 16) * 16 * d)) return hipErrorInvalidValue;
    const dim3 grid(n), block(256);
    const int per = (d + 255) / 256;
    if (per <= 1) hipLaunchKernelGGL(ln_shift_kernel<1>, grid, block, 0, stream, x, d, gamma, beta, prev_state, slot, mix6, out6, out_stride, parts, part_stride, nparts, out_tiled);
    else if (per <= 2) hipLaunchKernelGGL(ln_shift_kernel<2>, grid, block, 0, stream, x, d, gamma, beta, prev_state, slot, mix6, out6, out_stride, parts, part_stride, nparts, out_tiled);
    else if (per <= 3) hipLaunchKernelGGL(ln_shift_kernel<3>, grid, block, 0, stream, x, d, gamma, beta, prev_state, slot, mix6, out6, out_stride, parts, part_stride, nparts, out_tiled);
    else if (per <= 4) hipLaunchKernelGGL(ln_shift_kernel<4>, grid, block, 0, stream, x, d, gamma, beta, prev_state, slot, mix6, out6, out_stride, parts, part_stride, nparts, out_tiled);
    else return hipErrorInvalidValue;
    return hipGetLastError();
}

// x[m, c] += parts[0][m, c] + parts[1][m, c] + ... (in order), rows of width d.
__global__ void add_parts_kernel(float *x, size_t n, const float *parts, size_t part_stride, int nparts) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
        float v = x[i];
        for (int q = 0; q < nparts; ++q) v += parts[q * part_stride + i];
        x[i] = v;
    }
}

hipError_t launch_add_parts(float *x, int M, int d, const float *parts, size_t part_stride, int nparts,
                            hipStream_t stream) {
    const size_t n = (size_t)M * d;
    if (n == 0 || nparts <= 0) return hipSuccess;
    hipLaunchKernelGGL(add_parts_kernel, dim3(grid_for(n, 256)), dim3(256), 0, stream, x, n, parts, part_stride, nparts);
    return hipGetLastError();
}

hipError_t launch_embed(const int *tokens, int M, const float *table, int d, int vocab, float *out, int *bad,
                        hipStream_t stream) {
    if (M <= 0) return hipSuccess;
    hipLaunchKernelGGL(embed_kernel, dim3(M), dim3(256), 0, stream, tokens, M, table, d, vocab, out, bad);
    return hipGetLastError();
}

hipError_t launch_ln_shift_seq(const float *x, int Bn, int T, int d, const float *gamma, const float *beta,
                               const float *prev_state, const int *slot, const float *mix6, float *out6,
                               size_t out_stride, float *last_xn, hipStream_t stream) {
    if (Bn <= 0 || T <= 0) return hipSuccess;
    constexpr int R = 16;  // tokens per wave: one extra LayerNorm per 16 rows
    const int waves = Bn * ((T + R - 1) / R), per = (d + kWave - 1) / kWave;
    const dim3 grid((waves + 3) / 4), block(256);
    if (per <= 2)
        hipLaunchKernelGGL(ln_shift_seq_kernel<2>, grid, block, 0, stream, x, Bn, T, d, R, gamma, beta, prev_state, slot,
                           mix6, out6, out_stride, last_xn);
    else if (per <= 4)
        hipLaunchKernelGGL(ln_shift_seq_kernel<4>, grid, block, 0, stream, x, Bn, T, d, R, gamma, beta, prev_state, slot,
                           mix6, out6, out_stride, last_xn);
    else if (per <= 10)
        hipLaunchKernelGGL(ln_shift_seq_kernel<10>, grid, block, 0, stream, x, Bn, T, d, R, gamma, beta, prev_state,
                           slot, mix6, out6, out_stride, last_xn);
    else if (per <= 16)
        hipLaunchKernelGGL(ln_shift_seq_kernel<16>, grid, block, 0, stream, x, Bn, T, d, R, gamma, beta, prev_state,
                           slot, mix6, out6, out_stride, last_xn);
    else
        return hipErrorInvalidValue;
    return hipGetLastError();
}

hipError_t launch_token_shift(const float *x, int Bn, int T, int d, const float *prev_state, const int *slot,
                              const float *mix6, float *out6, size_t out_stride, hipStream_t stream) {
    const size_t n = (size_t)Bn * T * d;
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(token_shift_kernel, dim3(grid_for(n, 256)), dim3(256), 0, stream, x, Bn, T, d, prev_state,
                       slot, mix6, out6, out_stride);
    return hipGetLastError();
}

hipError_t launch_save_prev(const float *x, int Bn, int T, int d, float *prev_state, const int *slot,
                            hipStream_t stream) {
    if (Bn <= 0 || T <= 0) return hipSuccess;
    hipLaunchKernelGGL(save_prev_kernel, dim3(Bn), dim3(256), 0, stream, x, Bn, T, d, prev_state, slot);
    return hipGetLastError();
}

hipError_t launch_gather_last(const float *x, int Bn, int T, int d, float *out, hipStream_t stream) {
    if (Bn <= 0 || T <= 0) return hipSuccess;
    hipLaunchKernelGGL(gather_last_kernel, dim3(Bn), dim3(256), 0, stream, x, Bn, T, d, out);
    return hipGetLastError();
}

hipError_t launch_rosa_gates(float *x, int M, int D, int ld, hipStream_t stream) {
    const size_t n = (size_t)M * D;
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(rosa_gates_kernel, dim3(grid_for(n, 256)), dim3(256), 0, stream, x, M, D, ld);
    return hipGetLastError();
}

hipError_t launch_fill(float *p, size_t n, float value, hipStream_t stream) {
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(fill_kernel, dim3(grid_for(n, 256)), dim3(256), 0, stream, p, n, value);
    return hipGetLastError();
}

}  // namespace yuf
