// Internal launch interfaces of the HIP kernels (not part of the C ABI).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace yuf {

// ----------------------------------------------------------------- WKV-7 scan
struct WkvParams {
    int B = 0, T = 0, H = 0;
    // Per-token inputs, [B, T, H, N] contiguous.
    const float *r = nullptr, *w = nullptr, *k = nullptr, *v = nullptr;
    const float *a = nullptr, *b = nullptr;
    // Fused-prep mode (the model path): `a` holds the post-sigmoid gate alpha,
    // `k` the raw key; kk = normalize(k * k_k) per head, a = -kk, b = kk * alpha,
    // k_hat = k * (1 + (alpha - 1) * k_a)  (yufmusicgen/model.py:114-122).
    const float *k_k = nullptr, *k_a = nullptr;  // [H * N]
    // State [slots, H, N, N]; stream b uses slot `slot[b]` (slot == nullptr: b).
    const float *state_in = nullptr;
    float *state_out = nullptr;
    const int *slot = nullptr;
    float *y = nullptr;  // [B, T, H, N]
    // Decode step (T = 1, fused prep) with the second low-rank stage folded in:
    // when `lr` is set, `w` and `a` are not read; instead, per channel c,
    //   w = w0 + lw . w2t[c],  alpha = sigmoid(a0 + la . a2t[c]),
    //   g = sigmoid(lg . g2t[c])  (written to g_out [B, H * N]),
    // from the rank-L rows lw = lr + b * L, la = lw + lr_plane, lg = la + lr_plane
    // and the [H * N, L] matrices w2t, a2t, g2t (yufmusicgen/model.py:108-112).
    const float *lr = nullptr;
    size_t lr_plane = 0;
    int L = 0;
    const float *w2t = nullptr, *a2t = nullptr, *g2t = nullptr, *w0 = nullptr, *a0 = nullptr;
    float *g_out = nullptr;
    // T = 1 step only: y and g_out written in 16 x 16 tiles (tile_index with
    // row = sequence, column = h * N + channel, ld = H * N) for the decode GEMM.
    bool tiled_out = false;
};
bool wkv7_supported(int N);
// The fused low-rank step exists for N <= 64 and L <= 128 with L % 8 == 0.
bool wkv7_step_lowrank_ok(int N, int L);
// Picks the chunked MFMA kernel (N <= 64, N % 4 == 0, T >= kWkvChunkMinT) or
// the per-token VALU kernel; YUF_WKV7_KERNEL=serial|chunked forces one.
hipError_t launch_wkv7(const WkvParams &p, int N, bool prep, hipStream_t stream);
constexpr int kWkvChunkMinT = 32;
bool wkv7_chunk_supported(int N);
hipError_t launch_wkv7_chunked(const WkvParams &p, int N, bool prep, hipStream_t stream);

// ------------------------------------------------------------------ ROSA scan
struct RosaParams {
    int B = 0, T = 0, D = 0;
    // Pre-activations; element (b, t, c) at base[(b * T + t) * ld + c].
    const float *cand = nullptr, *write = nullptr, *read_raw = nullptr;
    int ld = 0;
    const float *decay = nullptr, *direction = nullptr;  // [D]
    // Model path: derive lambda = sigmoid(decay_param), u = normalize(householder).
    bool raw_params = false;
    const float *memory_in = nullptr;
    float *memory_out = nullptr;
    const int *slot = nullptr;
    float *read_out = nullptr;  // [(b * T + t) * D + c]
    // Prepared inputs (model path): e = sigmoid(write) tanh(cand) and the read
    // gate sigmoid(read_raw), same indexing as the pre-activations; when set,
    // cand / write / read_raw are ignored and the read is gated.
    const float *e_pre = nullptr, *g_pre = nullptr;
    // Segmented second pass: the B rows are chains of `seg` consecutive
    // segments, and only each chain's last segment writes its end state, to
    // memory_out row seg_slot[chain] (or chain).
    int seg = 0;
    const int *seg_slot = nullptr;
};
hipError_t launch_rosa(const RosaParams &p, hipStream_t stream);
// Long sequences with the model's constant transition A = diag(lambda) H: the
// T tokens of each chain split into T / L segments scanned in parallel (zero
// start, then true start) around a carry pass with AL = A^L ([D][D] row-major,
// fp32).  Scratch: z, carry of B * (T / L) * D floats each.
bool rosa_segmented_ok(int T, int D, int L);
// A^L of A = diag(lambda) (I - 2 u u^T) into AL [D][D] (column j = A^L e_j),
// computed in double on the device (lambda post-sigmoid, u unit).
hipError_t launch_rosa_power(int D, int L, const float *lambda, const float *u, float *AL, hipStream_t stream);
hipError_t launch_rosa_segmented(const RosaParams &p, const float *AL, int L, float *z, float *carry,
                                 hipStream_t stream);

// ----------------------------------------------------------------------- GEMM
// C[m, n] = epilogue( sum_k A[m, k] * W[n, k] )   (nn.Linear: y = x W^T)
enum GemmAct : int { ACT_NONE = 0, ACT_TANH = 1, ACT_SIGMOID = 2 };
struct GemmParams {
    int M = 0, N = 0, K = 0;
    const float *A = nullptr;
    int lda = 0;
    const float *W = nullptr;
    int ldw = 0;
    // bf16 weights (raw bits, [N][ldw]) instead of W: the large-tile and decode
    // kernels split A into bf16 hi + lo parts and accumulate in fp32; needs
    // K % 8 == 0.
    const uint16_t *Wh = nullptr;
    float *C = nullptr;
    int ldc = 0;
    const float *bias = nullptr;      // [N] added before the activation
    int act = ACT_NONE;
    const float *residual = nullptr;  // [M, ldr] added after the activation (may alias C)
    int ldr = 0;
    // Paired SiLU-gate output: W rows come in blocks of 64 = 32 "in" rows then
    // 32 "gate" rows; C[m, 32 q + c] = silu(in) * gate.  N counts W rows.
    bool silu_pair = false;
    // Optional scratch for the split-K path of short-M (decode) products:
    // `workspace_floats` floats of device memory; nullptr disables splitting.
    float *workspace = nullptr;
    size_t workspace_floats = 0;
    // Optional A-side prologue (M <= 64, K % 4 == 0, K <= 1024 only): each A row
    // is replaced by LayerNorm(row) * ln_gamma + ln_beta over its K columns
    // (eps 1e-5), then multiplied elementwise by a_gate (row stride ldg) if set.
    const float *ln_gamma = nullptr;
    const float *ln_beta = nullptr;
    const float *a_gate = nullptr;
    int ldg = 0;
    // Optional copy of W for the decode kernels (M <= 64) in 16-row tiles: row
    // tile rt, k tile kt (16 k for fp32, 32 k for bf16) at rt * wt_ld + kt *
    // 256 (fp32, 16 x 16 row-major) or kt * 512 (bf16, 16 x 32) elements, so
    // the 16 rows x 16 k (32 k) a wave reads per k step are one contiguous
    // 1 KB run -- about 4x the vector-load issue rate of 16 rows x 64 bytes.
    const float *Wt = nullptr;
    const uint16_t *Wht = nullptr;
    int wt_ld = 0;
    // Optional pre-split copy of an fp32 W for the large-tile X3 products
    // (M > 64): its three bf16 parts in the plane layout of
    // launch_x3_split_planes (N % 16 == 0, K % 32 == 0).  Same results as
    // without it.
    const uint16_t *Wp = nullptr;
    // Decode kernels only: A (and a_gate) stored in 16 x 16 tiles (tile_index,
    // row strides lda / ldg), and, for the SiLU-pair product, C written that way
    // (row stride ldc).  A tiled A needs one round of k steps per wave.
    bool a_tiled = false, c_tiled = false;
};
hipError_t launch_gemm(const GemmParams &p, hipStream_t stream);

// Decode ROSA output projection with the ROSA single-token step as its A
// prologue (M <= 64, fp32 W [N][D], D in {128, 256}): per row m, from the
// memory row mem[slot[m]] and the pre-activations e | write | read_raw at
// pre + m * ld_pre,
//   m' = lambda (m - 2 (u.m) u) + tanh(e) sigmoid(write),
//   A[m] = (m' - 2 (u.m') u) sigmoid(read_raw),
// then C = A W^T (+ bias) (+ residual).  The last workgroup of each 16-row tile
// to finish (counter[tile], left at zero) writes m' back to mem[slot[m]], after
// every workgroup of the tile has read the old row.
struct RosaOutParams {
    int M = 0, N = 0, D = 0;
    const float *pre = nullptr;
    int ld_pre = 0;
    float *mem = nullptr;
    int mem_rows = 0;
    const int *slot = nullptr;
    const float *u = nullptr, *lam = nullptr;  // unit direction, sigmoid(decay) [D]
    const float *W = nullptr;
    const float *Wt = nullptr;  // optional 16 x 16-tiled W (GemmParams::Wt layout), wt_ld floats per row tile
    int wt_ld = 0;
    const float *bias = nullptr;
    const float *residual = nullptr;
    int ldr = 0;
    float *C = nullptr;
    int ldc = 0;
    int *counter = nullptr;  // ceil(M / 16) ints, zero between launches
};
bool rosa_out_decode_ok(int M, int D);
hipError_t launch_rosa_out_decode(const RosaOutParams &p, hipStream_t stream);
// Up to kMaxGroup independent products in one launch (M > 64: one launch for
// the group; M <= 64: one launch per SiLU flag and prologue kind).
constexpr int kMaxGroup = 6;
hipError_t launch_gemm_group(const GemmParams *ps, int count, hipStream_t stream);
// Workspace the short-M path can use for an N-column product (floats).
size_t gemm_workspace_floats(int N, int K);
// Pre-split weight planes (GemmParams::Wp): elements (uint16) for an [N, K]
// matrix, 0 unless N % 16 == 0 and K % 32 == 0; the split of fp32 W [N][ldw]
// (16-byte aligned, ldw % 4 == 0) into them.
size_t x3_planes_elems(int N, int K);
hipError_t launch_x3_split_planes(const float *W, int ldw, int N, int K, uint16_t *planes, hipStream_t stream);

// --------------------------------------------------- persistent decode layer
// One decode layer (T = 1) of up to kDlRows streams per XCD group in one
// launch: the streams are split into `groups` groups (one per XCD), and the
// workgroups running on XCD x (read from the hardware's XCC_ID) work through
// group x's seven stages -- LN + token shift + r/k/v/w1/a1/g1 products; the
// WKV step with the second low-rank stage; LN * g -> W_o (+h); LN -> ROSA
// in; the ROSA step -> ROSA out (+h); LN -> FFN in (silu * gate); FFN out
// (+h) -- taking work items from per-group queues and meeting at per-group
// barriers (agent-scope counters; activations written by one workgroup are
// read by another with L1-bypassing loads, which the XCD's shared L2 serves).
constexpr int kDlRows = 8;
constexpr int kDlMaxD = 640;
constexpr int kDlStages = 7;
constexpr int kDlCounterStride = 32;  // ints between counters (one per 128-byte line)
// The launch takes `grid` workgroups, a multiple of `groups`: the workgroups
// of an XCD split each stage's items by their rank blockIdx.x / groups.
struct DecodeLayerParams {
    int n = 0, groups = 0;
    int d = 0, H = 0, N = 0, L = 0, D = 0;
    const int *slot = nullptr;
    const float *ln_t_w = nullptr, *ln_t_b = nullptr, *mix6 = nullptr;
    // 16 x 16-tiled weights (GemmParams::Wt layout); K = d matrices have
    // 16 d floats per row tile.
    const float *wt_rkv[3] = {}, *wt_lr1[3] = {};  // r, k, v [d][d]; w1t, a1t, g1t [L][d]
    const float *w2t = nullptr, *a2t = nullptr, *g2t = nullptr;  // row-major [d][L]
    const float *w0 = nullptr, *a0 = nullptr, *k_k = nullptr, *k_a = nullptr;
    const float *ln_o_w = nullptr, *ln_o_b = nullptr, *wt_o = nullptr;
    const float *ln_r_w = nullptr, *ln_r_b = nullptr, *wt_rin = nullptr, *b_rin = nullptr;  // [3D][d], [3D]
    const float *rosa_u = nullptr, *rosa_lam = nullptr, *wt_rout = nullptr;              // [d][D]
    const float *ln_f_w = nullptr, *ln_f_b = nullptr, *wt_fin = nullptr;  // [8d][d], 64-row in/gate blocks
    const float *wt_fout = nullptr;                                      // [d][4d]
    // This layer's state slots and the step's activations.
    float *prev = nullptr, *wkv = nullptr, *rosa = nullptr;
    float *h = nullptr;       // [n][d]
    float *buf = nullptr;     // groups x decode_layer_group_floats(d, L, D)
    int *sync = nullptr;      // this launch's counters (decode_layer_sync_ints), zero at launch
    int *error = nullptr;     // bit 1 set when a barrier wait gives up
};
bool decode_layer_ok(int d, int H, int N, int L, int D);
size_t decode_layer_group_floats(int d, int L, int D);
// Counter ints of one launch: the stage counters of every group and one
// (XCD, rank) registration slot per workgroup of the `grid`.
size_t decode_layer_sync_ints(int groups, int grid);
hipError_t launch_decode_layer(const DecodeLayerParams &p, int grid, hipStream_t stream);

// ---------------------------------------------------------------- elementwise
hipError_t launch_embed(const int *tokens, int M, const float *table, int d, int vocab, float *out,
                        int *bad_token_flag, hipStream_t stream);
// out = LayerNorm(x) * gamma + beta, rows of width d (eps 1e-5); optional
// row gather (`rows`), optional multiply by `gate` after the affine.
hipError_t launch_layernorm(const float *x, int M, int d, const float *gamma, const float *beta,
                            const float *gate, float *out, hipStream_t stream);
// Token shift: six outputs out[c][m, :] = x[m] + (x[m] - x_prev(m)) * mix[c],
// x_prev(m) = x[m - 1] inside a row of T tokens, prev_state[slot[b]] at t = 0.
hipError_t launch_token_shift(const float *x, int Bn, int T, int d, const float *prev_state,
                              const int *slot, const float *mix6, float *out6, size_t out_stride,
                              hipStream_t stream);
// T = 1 fusion of layernorm -> token_shift -> save_prev: out6 from the normed
// rows and prev_state[slot[b]] <- LayerNorm(x[b]); d <= 1024.
// nparts > 0: x[b] += parts[0][b] + parts[1][b] + ... (part planes part_stride
// floats apart, rows of width d) first, and the completed row is written back.
hipError_t launch_ln_shift(float *x, int n, int d, const float *gamma, const float *beta, float *prev_state,
                           const int *slot, const float *mix6, float *out6, size_t out_stride, const float *parts,
                           size_t part_stride, int nparts, bool out_tiled, hipStream_t stream);
// x[m] += parts[0][m] + parts[1][m] + ... in order (M rows of width d).
hipError_t launch_add_parts(float *x, int M, int d, const float *parts, size_t part_stride, int nparts,
                            hipStream_t stream);
// T > 1 fusion of layernorm -> token_shift: out6 from the normed rows (the
// normed rows themselves are not stored) and last_xn[b] <- the normed row
// t = T - 1 (for launch_save_prev with T = 1 afterwards); d <= 1024.
hipError_t launch_ln_shift_seq(const float *x, int Bn, int T, int d, const float *gamma, const float *beta,
                               const float *prev_state, const int *slot, const float *mix6, float *out6,
                               size_t out_stride, float *last_xn, hipStream_t stream);
// prev_state[slot[b]] = x[b, T - 1, :]
hipError_t launch_save_prev(const float *x, int Bn, int T, int d, float *prev_state, const int *slot,
                            hipStream_t stream);
// Gather the last token of each row: out[b] = x[b, T - 1].
hipError_t launch_gather_last(const float *x, int Bn, int T, int d, float *out, hipStream_t stream);
// state blob pack/unpack and clearing.
hipError_t launch_fill(float *p, size_t n, float value, hipStream_t stream);
// In place on rows [cand | write | read_raw] of stride ld: cand <- e, write <- gate.
hipError_t launch_rosa_gates(float *x, int M, int D, int ld, hipStream_t stream);

// -------------------------------------------------------------------- sampling
// One workgroup per stream (row of `logits`, [n, V]): optional generation
// mask, temperature, top-k (1..64) and top-p, then the draw argmax p / q with
// q = exp_draws[stream][position] (host MT19937 Exp(1) draws) or, when
// exp_draws is null, -log u from a counter-based hash.
constexpr int kSampleMaxBlocked = 256;  // blocked raw ids carried in the kernel arguments
constexpr int kSampleMaskWords = 1024;  // blocked-id bitmap: raw ids below 32768
struct SampleParams {
    int V = 0;
    const float *logits = nullptr;
    float temperature = 1.0f, top_p = 1.0f;
    int top_k = 0;
    // Generation mask (midi_offset < 0: none).  The EOS id is allowed once the
    // stream's index (index[s], or index_all when index is null) reaches
    // min_before_eos.
    int midi_offset = -1, eos_id = 0, min_before_eos = 0, index_all = 0;
    const int32_t *index = nullptr;
    int n_blocked = 0;
    int blocked[kSampleMaxBlocked] = {};
    const float *exp_draws = nullptr;     // [n, top_k]
    const int32_t *first_zero = nullptr;  // [n]: first position >= top_k whose draw is 0, else -1
    uint64_t seed = 0, counter = 0;
    int32_t *tokens = nullptr;  // [n]
};
hipError_t launch_sample(const SampleParams &p, int n, hipStream_t stream);

}  // namespace yuf
