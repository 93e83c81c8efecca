// The inference engine behind the C ABI: device-resident weights, per-stream
// recurrent state in HBM, batched prefill and multi-stream decode.
//
// Replaces the reference's Vulkan `Model` (vulkan/src/compute/model.rs:24-65,
// op order :425-757) and the Python forward/step (yufmusicgen/model.py:97-445):
//   embedding -> per layer [LN_t -> token shift -> r/k/v/w/a/g projections ->
//   WKV-7 scan -> LN_out * g -> W_o (+res) -> LN_r -> ROSA c/w/rho -> ROSA scan
//   -> W_out (+res) -> LN_f -> FFN in/gate (silu * gate) -> W_ffn_out (+res)]
//   -> final LN -> tied LM head.
// State per stream and layer: previous normed input [d], WKV state [H, N, N]
// (row = value index), ROSA memory [D] -- the BlockState of model.py:29-38.
//
// Differences by design: prefill is one batched pass per T-chunk instead of a
// per-token loop (generation.rs:176-185); any number of streams share the
// engine through state slots; `previous` is part of the state that
// yuf_state_reset clears (the Rust reset leaves it stale, mod.rs:706-724).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstdlib>
#include <cstring>
#include <memory>
#include <set>
#include <string>
#include <vector>

#include "../../include/yuf_engine.h"
#include "checkpoint.h"
#include "common.h"
#include "kernels.h"

namespace yuf {

namespace {

struct LayerW {
    const float *ln_t_w, *ln_t_b, *mix6;
    const float *w_r, *w_k, *w_v, *w_o;
    const float *w1t, *w2t, *a1t, *a2t, *g1t, *g2t;  // low-rank pairs as [out, in]
    const float *w0, *a0, *k_k, *k_a;
    const float *ln_o_w, *ln_o_b, *ln_r_w, *ln_r_b;
    const float *rosa_w3, *rosa_b3, *rosa_hh, *rosa_decay, *rosa_out;
    const float *ln_f_w, *ln_f_b, *ffn_cat, *ffn_out;
    const float *rosa_al;  // A^kRosaSeg of the ROSA transition, [D][D] row-major
    const float *rosa_u, *rosa_lam;  // u = normalize(householder), lambda = sigmoid(decay), [D]
};

// Segment length of the segmented ROSA prefill scan.
constexpr int kRosaSeg = 64;
constexpr int kFfnParts = 4;  // K split of the decode FFN output product (partials summed by their consumer)

struct DeviceBuf {
    void *p = nullptr;
    ~DeviceBuf() {
        if (p) (void)hipFree(p);
    }
};

}  // namespace

struct Engine {
    ModelShape s;
    int max_streams = 0, max_tokens = 0;
    hipStream_t stream = nullptr;
    DeviceBuf weights, weights_h, weights_t, weights_p, state, work, io, dl;
    // bf16 mode: a bf16 image of the weight buffer (same element offsets); the
    // GEMMs of weights inside [w_base, w_base + w_floats) read it instead.
    const float *w_base = nullptr;
    size_t w_floats = 0;
    const uint16_t *w_h = nullptr;
    // The projection matrices again in 16-row tiles for the decode kernels
    // (GemmParams::Wt / Wht): fp32 16 x 16 tiles, or bf16 16 x 32 tiles in
    // bf16 mode.  `base` is the row-major matrix in the weight buffer.
    struct Tiled {
        const float *base;
        long long rows, cols;
        const void *tiles;
        int wt_ld;  // elements per row tile
        // fp32 mode: the matrix's three bf16 parts for the large-tile X3
        // products (GemmParams::Wp), or nullptr.
        const uint16_t *planes;
    };
    std::vector<Tiled> tiled;
    std::vector<LayerW> layers;
    const float *emb = nullptr, *ln_fin_w = nullptr, *ln_fin_b = nullptr, *head = nullptr;
    // state arrays, [layer][slot][...]
    float *st_prev = nullptr, *st_wkv = nullptr, *st_rosa = nullptr;
    // workspace (sized for max_tokens rows)
    float *h = nullptr, *xn = nullptr, *mix = nullptr, *r = nullptr, *k = nullptr, *v = nullptr, *wr = nullptr,
          *al = nullptr, *g = nullptr, *lr = nullptr, *y = nullptr, *z = nullptr, *rosa3 = nullptr, *rread = nullptr,
          *ffn = nullptr, *hl = nullptr;
    float *rz = nullptr, *rcarry = nullptr;  // segmented ROSA scratch
    float *kpart = nullptr;  // [kFfnParts][max_streams][d]: K-split partials of the decode FFN output
    bool rosa_segmented = true;                                // YUF_ROSA_SEGMENTED=0 disables
    bool decode_fusion = true;                                 // YUF_DECODE_FUSION=0: separate low-rank GEMM and ROSA step
    bool act_tiles = true;                                     // YUF_DECODE_TILES=0: row-major decode activations
    // Persistent decode layers (launch_decode_layer): one launch per layer for
    // steps of at most kDlRows streams per XCD.  YUF_DECODE_LAYER=1 enables.
    bool decode_layer = false;
    int dl_groups = 0, dl_grid = 0;  // XCDs of the device, workgroups per launch (its CU count)
    float *dl_buf = nullptr;         // per-XCD group activations
    int *dl_sync = nullptr;          // per-layer counter blocks, zeroed at the start of each step
    size_t dl_sync_ints = 0;         // per layer
    int prefill_groups = 0;                                    // YUF_PREFILL_GROUPS=1..4: streams for the batch's parts (0: automatic)
    // The first layer's WKV-7 step launch of the last decode pass (fused
    // low-rank form), kept for yuf_engine_time_wkv_step.
    WkvParams wkv_probe;
    bool wkv_probe_set = false;
    float *gemm_ws = nullptr;  // split-K partials of short-M (decode) products
    size_t gemm_ws_floats = 0;
    // Out-of-range token flags set by the embedding kernel: bad_host for the
    // host-buffer entry points (ids already validated on the host), bad_dev
    // for the device entry points (read by yuf_engine_take_error).
    int *slots_dev = nullptr, *tokens_dev = nullptr, *bad_dev = nullptr, *bad_host = nullptr;
    int *rosa_count = nullptr;  // [max_streams]: 16-row tile counters of the fused ROSA-out kernel, by first stream
    int *slots_host = nullptr;  // pinned
    std::vector<int> last_slots;
    // Device staging for the host-buffer entry points (grown on demand).
    DeviceBuf host_tokens, host_logits;
    size_t host_tokens_cap = 0, host_logits_cap = 0;
    // Decode step captured as a HIP graph (about ten kernels per layer and
    // group, replayed with one launch); rebuilt when n or the token / logit
    // buffers change.
    // YUF_NO_GRAPH=1 runs every step eagerly.
    bool use_graphs = true;
    hipGraphExec_t step_exec[5] = {};  // one per branch + the LM head (one graph when unbranched)
    int step_n = 0;
    const int32_t *step_tok = nullptr;
    float *step_logits = nullptr;
    // The step can split its streams into groups replayed on their own HIP
    // streams (fork / join events): independent chains of small kernels that
    // the hardware queues overlap.  branches = 0: automatic (two groups when
    // n is a multiple of 32 and at least 64, else one); YUF_DECODE_BRANCHES=1..4
    // forces that many groups.
    static constexpr int kMaxBranches = 4;
    int branches = 0;
    hipStream_t side[kMaxBranches - 1] = {};
    hipEvent_t fork = nullptr, join[kMaxBranches - 1] = {};

    ~Engine() {
        for (auto g : step_exec)
            if (g) (void)hipGraphExecDestroy(g);
        for (int i = 0; i < kMaxBranches - 1; ++i) {
            if (side[i]) (void)hipStreamDestroy(side[i]);
            if (join[i]) (void)hipEventDestroy(join[i]);
        }
        if (fork) (void)hipEventDestroy(fork);
        if (stream) {
            (void)hipStreamSynchronize(stream);
            (void)hipStreamDestroy(stream);
        }
        if (slots_host) (void)hipHostFree(slots_host);
    }

    size_t wkv_floats() const { return (size_t)s.heads * s.head_size * s.head_size; }
    size_t state_floats() const { return (size_t)s.layers * (s.d + wkv_floats() + s.rosa); }
};

namespace {

int hip_fail(hipError_t e, const char *what) {
    return fail(YUF_ERR_HIP, std::string(what) + ": " + hipGetErrorString(e));
}

#define ENG_TRY(expr, what)                                  \
    do {                                                     \
        hipError_t e_ = (expr);                              \
        if (e_ != hipSuccess) return hip_fail(e_, what);     \
    } while (0)

// x rounded to the nearest bf16 value (ties to even; NaN stays NaN), as float.
float bf16_round(float x) {
    uint32_t u;
    std::memcpy(&u, &x, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) return x;
    u = ((u + 0x7fffu + ((u >> 16) & 1u)) >> 16) << 16;
    std::memcpy(&x, &u, 4);
    return x;
}

// Host-side weight preparation: the device layout the kernels want.  With
// round_projections (bf16 weights) every projection matrix -- the nn.Linear
// weights, the low-rank pairs and the LM head -- is stored as its bf16 value,
// so kernels that read the fp32 copy (the decode folds) multiply exactly the
// weights the bf16 products use.
int build_weights(const Checkpoint &ck, std::vector<float> &host, std::vector<size_t> &offsets, std::string &err,
                  bool round_projections = false) {
    const ModelShape &s = ck.shape;
    const long long d = s.d, L = s.low_rank, D = s.rosa, V = s.vocab, hid = 4LL * s.d;
    std::vector<std::pair<size_t, size_t>> projections;  // (offset, count) of each projection matrix
    auto append = [&](const float *src, size_t n) {
        // Keep every tensor 256-byte aligned for vector loads.
        size_t off = (host.size() + 63) & ~size_t(63);
        host.resize(off + n);
        std::memcpy(host.data() + off, src, n * sizeof(float));
        offsets.push_back(off);
    };
    auto append_proj = [&](const float *src, size_t n) {
        append(src, n);
        projections.emplace_back(offsets.back(), n);
    };
    auto get = [&](const std::string &name, std::vector<long long> dims) -> const float * {
        return ck.tensor(name, dims, err);
    };
    auto transposed = [&](const float *src, long long rows, long long cols) {
        std::vector<float> t((size_t)(rows * cols));
        for (long long i = 0; i < rows; ++i)
            for (long long j = 0; j < cols; ++j) t[(size_t)(j * rows + i)] = src[i * cols + j];
        return t;
    };
    const float *e = get("token_embedding.weight", {V, d});
    if (!e) return YUF_ERR_FORMAT;
    append(e, (size_t)(V * d));
    const float *head = e;
    if (!s.tie) {
        head = get("lm_head.weight", {V, d});
        if (!head) return YUF_ERR_FORMAT;
    }
    append_proj(head, (size_t)(V * d));
    for (const char *n : {"final_norm.weight", "final_norm.bias"}) {
        const float *p = get(n, {d});
        if (!p) return YUF_ERR_FORMAT;
        append(p, (size_t)d);
    }
    for (int l = 0; l < s.layers; ++l) {
        const std::string pre = "blocks." + std::to_string(l) + ".";
        auto vec = [&](const std::string &n) -> bool {
            const float *p = get(pre + n, {n.find("rosa.") == 0 ? D : d});
            if (!p) return false;
            append(p, (size_t)(n.find("rosa.") == 0 ? D : d));
            return true;
        };
        auto mat = [&](const std::string &n, long long rows, long long cols) -> bool {
            const float *p = get(pre + n, {rows, cols});
            if (!p) return false;
            append_proj(p, (size_t)(rows * cols));
            return true;
        };
        auto mat_t = [&](const std::string &n, long long rows, long long cols) -> bool {
            const float *p = get(pre + n, {rows, cols});
            if (!p) return false;
            std::vector<float> t = transposed(p, rows, cols);
            append_proj(t.data(), t.size());
            return true;
        };
        if (!vec("norm_time.weight") || !vec("norm_time.bias")) return YUF_ERR_FORMAT;
        {
            std::vector<float> mix6((size_t)(6 * d));
            const char *names[6] = {"mix_r", "mix_w", "mix_k", "mix_v", "mix_a", "mix_g"};
            for (int c = 0; c < 6; ++c) {
                const float *p = get(pre + "time_mix." + names[c], {d});
                if (!p) return YUF_ERR_FORMAT;
                std::memcpy(mix6.data() + c * d, p, d * sizeof(float));
            }
            append(mix6.data(), mix6.size());
        }
        if (!mat("time_mix.receptance.weight", d, d) || !mat("time_mix.key.weight", d, d) ||
            !mat("time_mix.value.weight", d, d) || !mat("time_mix.output.weight", d, d))
            return YUF_ERR_FORMAT;
        if (!mat_t("time_mix.w1", d, L) || !mat_t("time_mix.w2", L, d) || !mat_t("time_mix.a1", d, L) ||
            !mat_t("time_mix.a2", L, d) || !mat_t("time_mix.g1", d, L) || !mat_t("time_mix.g2", L, d))
            return YUF_ERR_FORMAT;
        if (!vec("time_mix.w0") || !vec("time_mix.a0") || !vec("time_mix.k_k") || !vec("time_mix.k_a"))
            return YUF_ERR_FORMAT;
        if (!vec("time_mix.out_norm.weight") || !vec("time_mix.out_norm.bias") || !vec("norm_rosa.weight") ||
            !vec("norm_rosa.bias"))
            return YUF_ERR_FORMAT;
        {
            std::vector<float> w3((size_t)(3 * D * d)), b3((size_t)(3 * D));
            const char *names[3] = {"rosa.input", "rosa.write_gate", "rosa.read_gate"};
            for (int c = 0; c < 3; ++c) {
                const float *w = get(pre + names[c] + ".weight", {D, d});
                const float *b = get(pre + names[c] + ".bias", {D});
                if (!w || !b) return YUF_ERR_FORMAT;
                std::memcpy(w3.data() + c * D * d, w, (size_t)(D * d) * sizeof(float));
                std::memcpy(b3.data() + c * D, b, (size_t)D * sizeof(float));
            }
            append_proj(w3.data(), w3.size());
            append(b3.data(), b3.size());
        }
        if (!vec("rosa.householder") || !vec("rosa.decay") || !mat("rosa.output.weight", d, D)) return YUF_ERR_FORMAT;
        if (!vec("norm_ffn.weight") || !vec("norm_ffn.bias")) return YUF_ERR_FORMAT;
        {
            const float *wi = get(pre + "ffn_in.weight", {hid, d});
            const float *wg = get(pre + "ffn_gate.weight", {hid, d});
            if (!wi || !wg) return YUF_ERR_FORMAT;
            if (hid % 32 != 0) {
                err = "ffn hidden width must be a multiple of 32";
                return YUF_ERR_FORMAT;
            }
            // Rows in blocks of 64: 32 rows of ffn_in, then the same 32 of ffn_gate.
            std::vector<float> cat((size_t)(2 * hid * d));
            for (long long q = 0; q < hid / 32; ++q) {
                std::memcpy(cat.data() + (size_t)(q * 64) * d, wi + (size_t)(q * 32) * d, 32 * d * sizeof(float));
                std::memcpy(cat.data() + (size_t)(q * 64 + 32) * d, wg + (size_t)(q * 32) * d, 32 * d * sizeof(float));
            }
            append_proj(cat.data(), cat.size());
        }
        if (!mat("ffn_out.weight", d, hid)) return YUF_ERR_FORMAT;
        {
            // A^L for the segmented ROSA scan, A = diag(lambda) (I - 2 u u^T) with
            // lambda = sigmoid(decay), u = householder / max(|householder|, 1e-12)
            // (yufmusicgen/model.py:300-301): column j is A applied L times to e_j,
            // in double precision through the rank-one form A x = lambda (x - 2 (u.x) u).
            const float *hh = get(pre + "rosa.householder", {D});
            const float *dec = get(pre + "rosa.decay", {D});
            if (!hh || !dec) return YUF_ERR_FORMAT;
            std::vector<double> u((size_t)D), lam((size_t)D), x((size_t)D);
            double nrm = 0.0;
            for (long long j = 0; j < D; ++j) nrm += (double)hh[j] * hh[j];
            nrm = std::max(std::sqrt(nrm), 1e-12);
            for (long long j = 0; j < D; ++j) {
                u[(size_t)j] = hh[j] / nrm;
                lam[(size_t)j] = 1.0 / (1.0 + std::exp(-(double)dec[j]));
            }
            std::vector<float> al((size_t)(D * D));
            for (long long j = 0; j < D; ++j) {
                std::fill(x.begin(), x.end(), 0.0);
                x[(size_t)j] = 1.0;
                for (int step = 0; step < kRosaSeg; ++step) {
                    double pr = 0.0;
                    for (long long i = 0; i < D; ++i) pr += u[(size_t)i] * x[(size_t)i];
                    for (long long i = 0; i < D; ++i) x[(size_t)i] = lam[(size_t)i] * (x[(size_t)i] - 2.0 * pr * u[(size_t)i]);
                }
                for (long long i = 0; i < D; ++i) al[(size_t)(i * D + j)] = (float)x[(size_t)i];
            }
            append(al.data(), al.size());
            std::vector<float> uf((size_t)D), lf((size_t)D);
            for (long long j = 0; j < D; ++j) {
                uf[(size_t)j] = (float)u[(size_t)j];
                lf[(size_t)j] = (float)lam[(size_t)j];
            }
            append(uf.data(), uf.size());
            append(lf.data(), lf.size());
        }
    }
    if (round_projections)
        for (const auto &[off, n] : projections)
            for (size_t i = 0; i < n; ++i) host[off + i] = bf16_round(host[off + i]);
    return YUF_OK;
}

template <typename T>
T *carve(char *&cursor, size_t count) {
    T *p = reinterpret_cast<T *>(cursor);
    cursor += ((count * sizeof(T) + 255) / 256) * 256;
    return p;
}

// The tiled copy of W (a tile-aligned block of one of e.tiled's matrices, row
// stride ldw) for the decode kernels, or nullptr; *wt_ld receives its row-tile
// stride.
const void *tiled_copy(const Engine &e, const float *W, int ldw, int *wt_ld) {
    for (const Engine::Tiled &t : e.tiled) {
        if (W < t.base || W >= t.base + t.rows * t.cols || ldw != t.cols) continue;
        const long long off = W - t.base, r0 = off / t.cols, c0 = off % t.cols;
        const int kt = e.w_h ? 32 : 16, esz = e.w_h ? 2 : 4;
        if (r0 % 16 != 0 || c0 % kt != 0) return nullptr;
        *wt_ld = t.wt_ld;
        return static_cast<const char *>(t.tiles) + ((size_t)(r0 / 16) * t.wt_ld + (size_t)(c0 / kt) * 16 * kt) * esz;
    }
    return nullptr;
}

// The pre-split planes of W (rows r0 .. r0 + N of one of e.tiled's matrices,
// all of its columns, r0 % 16 == 0) for the large-tile X3 products, or nullptr.
const uint16_t *planes_copy(const Engine &e, const float *W, int ldw, int N, int K) {
    for (const Engine::Tiled &t : e.tiled) {
        if (!t.planes || W < t.base || W >= t.base + t.rows * t.cols || ldw != t.cols || K != t.cols) continue;
        const long long off = W - t.base, r0 = off / t.cols, c0 = off % t.cols;
        if (c0 != 0 || r0 % 16 != 0 || r0 + N > t.rows) return nullptr;
        return t.planes + (size_t)(r0 / 16) * (t.cols / 32) * 3 * 512;
    }
    return nullptr;
}

GemmParams make_gemm(Engine &e, int M, int N, int K, const float *A, int lda, const float *W, int ldw, float *C,
                     int ldc, const float *bias = nullptr, int act = ACT_NONE, const float *residual = nullptr,
                     int ldr = 0, bool silu_pair = false) {
    GemmParams p;
    p.M = M; p.N = N; p.K = K; p.A = A; p.lda = lda; p.W = W; p.ldw = ldw; p.C = C; p.ldc = ldc;
    p.bias = bias; p.act = act; p.residual = residual; p.ldr = ldr; p.silu_pair = silu_pair;
    p.workspace = e.gemm_ws; p.workspace_floats = e.gemm_ws_floats;
    if (e.w_h && W >= e.w_base && W < e.w_base + e.w_floats) p.Wh = e.w_h + (W - e.w_base);
    if (!e.w_h && M > 64) p.Wp = planes_copy(e, W, ldw, N, K);
    if (M <= 64) {
        const void *t = tiled_copy(e, W, ldw, &p.wt_ld);
        if (e.w_h) p.Wht = static_cast<const uint16_t *>(t);
        else p.Wt = static_cast<const float *>(t);
    }
    return p;
}

int gemm(Engine &e, hipStream_t st, int M, int N, int K, const float *A, int lda, const float *W, int ldw, float *C,
         int ldc, const float *bias = nullptr, int act = ACT_NONE, const float *residual = nullptr, int ldr = 0,
         bool silu_pair = false) {
    ENG_TRY(launch_gemm(make_gemm(e, M, N, K, A, lda, W, ldw, C, ldc, bias, act, residual, ldr, silu_pair), st),
            "gemm");
    return YUF_OK;
}

// LayerNorm(A) [* gate] -> Linear.  Short products (M <= 64) fold the norm into
// the GEMM's A prologue; otherwise -- and for the wide LM head, whose many
// workgroups would each recompute the row statistics -- the normed rows go
// through `scratch` first.
int ln_gemm(Engine &e, hipStream_t st, int M, int N, int K, const float *A, int lda, const float *gamma,
            const float *beta, const float *gate, float *scratch, const float *W, float *C, int ldc,
            const float *bias = nullptr, const float *residual = nullptr, int ldr = 0, bool silu_pair = false,
            bool a_tiled = false, bool c_tiled = false) {
    // Wide N fuses only where the wide decode kernel runs (fp32 W, 32 < M, K <= 640).
    if (M <= 64 && K % 4 == 0 && K <= 1024 && (N <= 8192 || (M > 32 && K <= 640 && !e.w_h))) {
        GemmParams p = make_gemm(e, M, N, K, A, lda, W, K, C, ldc, bias, ACT_NONE, residual, ldr, silu_pair);
        p.ln_gamma = gamma; p.ln_beta = beta; p.a_gate = gate; p.ldg = gate ? lda : 0;
        p.a_tiled = a_tiled; p.c_tiled = c_tiled;
        ENG_TRY(launch_gemm(p, st), "ln gemm");
        return YUF_OK;
    }
    if (a_tiled || c_tiled) return fail(YUF_ERR_INVALID, "ln_gemm: tiled operands need the fused path");
    if (lda != K) return fail(YUF_ERR_INVALID, "ln_gemm: strided rows need the fused path");
    ENG_TRY(launch_layernorm(A, M, K, gamma, beta, gate, scratch, st), "layernorm");
    return gemm(e, st, M, N, K, scratch, K, W, K, C, ldc, bias, ACT_NONE, residual, ldr, silu_pair);
}

// Several independent products in one launch (the short-M split-K path runs
// them one after another: its workspace holds one product at a time).
int gemm_group(hipStream_t st, const GemmParams *ps, int count) {
    ENG_TRY(launch_gemm_group(ps, count, st), "gemm group");
    return YUF_OK;
}

// The activation rows of one forward pass: the engine's workspace from stream
// s0 on (token row s0 * Tc), and the HIP stream its kernels go to.  A decode
// step splits its batch into groups of streams whose passes touch disjoint
// rows, so they can run as parallel branches of one graph.
struct Act {
    hipStream_t st = nullptr;
    float *h, *xn, *mix, *r, *k, *v, *wr, *al, *g, *lr, *y, *z, *rosa3, *rread, *ffn, *hl;
    float *rz, *rcarry;  // segmented ROSA scratch (segment rows of kRosaSeg tokens)
    const int *tokens, *slots;
    int *bad;     // out-of-range token flag the embedding sets
    int *rcount;  // fused ROSA-out tile counters of this group of streams
    float *kpart;  // FFN-out K-split partials of these streams, planes kplane floats apart
    size_t kplane;
    bool tile_aligned;  // the rows start at a multiple of 16 (16 x 16-tiled decode activations possible)
    bool grouped = false;  // one of several stream groups of a step (parallel graph branches)
};

Act act_at(Engine &e, hipStream_t st, int s0, int Tc) {
    const ModelShape &s = e.s;
    const size_t m0 = (size_t)s0 * Tc, d = s.d;
    Act a;
    a.st = st;
    a.h = e.h + m0 * d; a.xn = e.xn + m0 * d; a.mix = e.mix + m0 * d;
    a.r = e.r + m0 * d; a.k = e.k + m0 * d; a.v = e.v + m0 * d; a.wr = e.wr + m0 * d; a.al = e.al + m0 * d;
    a.g = e.g + m0 * d; a.y = e.y + m0 * d; a.z = e.z + m0 * d;
    a.lr = e.lr + m0 * s.low_rank;
    a.rosa3 = e.rosa3 + m0 * 3 * s.rosa; a.rread = e.rread + m0 * s.rosa;
    a.ffn = e.ffn + m0 * 4 * d;
    a.hl = e.hl + (size_t)s0 * d;
    const size_t seg0 = (m0 / kRosaSeg) * s.rosa;
    a.rz = e.rz + seg0; a.rcarry = e.rcarry + seg0;
    a.tokens = e.tokens_dev + m0;
    a.slots = e.slots_dev + s0;
    a.bad = e.bad_dev;
    a.rcount = e.rosa_count + s0;
    a.kpart = e.kpart + (size_t)s0 * d;
    a.kplane = (size_t)e.max_streams * d;
    a.tile_aligned = m0 % 16 == 0;
    return a;
}

// Final norm and tied LM head on the last token of each of n streams.
int lm_head_last(Engine &e, const Act &a, int n, int Tc, float *logits) {
    const int d = e.s.d, V = e.s.vocab;
    const float *last = a.h;
    if (Tc > 1) {
        ENG_TRY(launch_gather_last(a.h, n, Tc, d, a.hl, a.st), "gather_last");
        last = a.hl;
    }
    return ln_gemm(e, a.st, n, V, d, last, d, e.ln_fin_w, e.ln_fin_b, nullptr, a.xn, e.head, logits, V);
}

// Single-token passes of at most kDlRows streams per XCD take the persistent
// decode layers.
bool decode_layer_applies(const Engine &e, int n) {
    return e.decode_layer && n >= 1 && n <= kDlRows * e.dl_groups;
}

// Internal logits mode of a prefill part: gather the last rows into a.hl for
// one LM head over all parts after they join.
constexpr int kLogitsGather = -1;

// One forward pass over n streams x Tc tokens whose ids and slots are in
// a.tokens / a.slots.  logits: LAST -> [n, V] at `logits`; ALL -> row (b, t) at
// logits + (b * row_stride_T + t0 + t) * V.  [l_begin, l_end) limits the pass
// to those layers: the embedding runs with l_begin = 0, the LM head with the
// last layer (l_end = -1: through the last layer).
int forward_pass(Engine &e, const Act &a, int n, int Tc, float *logits, int mode, int row_stride_T, int t0,
                 int l_begin = 0, int l_end = -1) {
    const ModelShape &s = e.s;
    const int M = n * Tc, d = s.d, L = s.low_rank, D = s.rosa, V = s.vocab, hid = 4 * s.d;
    const size_t plane = (size_t)e.max_tokens * d, lplane = (size_t)e.max_tokens * L;
    hipStream_t st = a.st;
    if (l_end < 0 || l_end > s.layers) l_end = s.layers;
    if (l_begin == 0) ENG_TRY(launch_embed(a.tokens, M, e.emb, d, V, a.h, a.bad, st), "embed");
    // Decode: the FFN output product is split over K into kFfnParts products
    // (four times the workgroups); the partial sums stay in a.kpart until the
    // next layer's ln_shift (or, after the last layer, add_parts) adds them to h.
    const bool ffn_split = Tc == 1 && e.decode_fusion && M <= 64 && d <= 1024 &&
                           hid % (16 * kFfnParts) == 0 && !decode_layer_applies(e, n);
    // Decode activations that only feed the decode GEMMs (the token-shift mixes,
    // the WKV output and gate, the FFN hidden rows) are written in 16 x 16 tiles
    // (tile_index), so those GEMMs read their A rows as contiguous 1 KB runs.
    // Needs the fused step (low-rank stage and FFN split), one round of k steps
    // per wave (d <= 768) and room for whole 16-row tiles.
    // With several stream groups (parallel graph branches) a group's tiles must
    // not cover another group's rows: whole tiles only.
    // (d <= 768 with fp32 weights, 16-k steps; d <= 512 with bf16 weights,
    // 32-k steps: W_o's gated LN prologue and the SiLU-pair FFN input hold at
    // most 6 and 2 steps per wave in registers.)
    const bool tl = ffn_split && e.act_tiles && a.tile_aligned && (!a.grouped || M % 16 == 0) && d % 16 == 0 &&
                    d <= (e.w_h ? 512 : 768) && wkv7_step_lowrank_ok(s.head_size, L) && ((M + 15) / 16) * 16 <= e.max_tokens;
    if (Tc == 1 && decode_layer_applies(e, n)) {
        // One launch per layer; its counters start at zero (a fill kernel, not
        // a memset node, so the step can be captured and replayed).
        if (l_begin == 0)
            ENG_TRY(launch_fill(reinterpret_cast<float *>(e.dl_sync), e.dl_sync_ints * s.layers, 0.0f, st),
                    "decode layer counters");
        for (int l = l_begin; l < l_end; ++l) {
            const LayerW &w = e.layers[l];
            DecodeLayerParams dp;
            dp.n = n; dp.groups = e.dl_groups;
            dp.d = d; dp.H = s.heads; dp.N = s.head_size; dp.L = L; dp.D = D;
            dp.slot = a.slots;
            dp.ln_t_w = w.ln_t_w; dp.ln_t_b = w.ln_t_b; dp.mix6 = w.mix6;
            int ld = 0;
            const float *mats[6] = {w.w_r, w.w_k, w.w_v, w.w1t, w.a1t, w.g1t};
            for (int c = 0; c < 6; ++c) {
                const float *t = static_cast<const float *>(tiled_copy(e, mats[c], d, &ld));
                if (!t) return fail(YUF_ERR_INVALID, "decode layer: missing tiled weights");
                if (c < 3) dp.wt_rkv[c] = t;
                else dp.wt_lr1[c - 3] = t;
            }
            dp.w2t = w.w2t; dp.a2t = w.a2t; dp.g2t = w.g2t;
            dp.w0 = w.w0; dp.a0 = w.a0; dp.k_k = w.k_k; dp.k_a = w.k_a;
            dp.ln_o_w = w.ln_o_w; dp.ln_o_b = w.ln_o_b;
            dp.wt_o = static_cast<const float *>(tiled_copy(e, w.w_o, d, &ld));
            dp.ln_r_w = w.ln_r_w; dp.ln_r_b = w.ln_r_b;
            dp.wt_rin = static_cast<const float *>(tiled_copy(e, w.rosa_w3, d, &ld));
            dp.b_rin = w.rosa_b3;
            dp.rosa_u = w.rosa_u; dp.rosa_lam = w.rosa_lam;
            dp.wt_rout = static_cast<const float *>(tiled_copy(e, w.rosa_out, D, &ld));
            dp.ln_f_w = w.ln_f_w; dp.ln_f_b = w.ln_f_b;
            dp.wt_fin = static_cast<const float *>(tiled_copy(e, w.ffn_cat, d, &ld));
            dp.wt_fout = static_cast<const float *>(tiled_copy(e, w.ffn_out, hid, &ld));
            if (!dp.wt_o || !dp.wt_rin || !dp.wt_rout || !dp.wt_fin || !dp.wt_fout)
                return fail(YUF_ERR_INVALID, "decode layer: missing tiled weights");
            dp.prev = e.st_prev + (size_t)l * e.max_streams * d;
            dp.wkv = e.st_wkv + (size_t)l * e.max_streams * e.wkv_floats();
            dp.rosa = e.st_rosa + (size_t)l * e.max_streams * D;
            dp.h = a.h;
            dp.buf = e.dl_buf;
            dp.sync = e.dl_sync + (size_t)l * e.dl_sync_ints;
            dp.error = a.bad;
            ENG_TRY(launch_decode_layer(dp, e.dl_grid, st), "decode layer");
        }
        l_begin = l_end;  // the layer loop below has nothing left to do
    }
    for (int l = l_begin; l < l_end; ++l) {
        const LayerW &w = e.layers[l];
        float *prev = e.st_prev + (size_t)l * e.max_streams * d;
        float *wkv = e.st_wkv + (size_t)l * e.max_streams * e.wkv_floats();
        float *ros = e.st_rosa + (size_t)l * e.max_streams * D;
        // TimeMix
        if (Tc == 1 && d <= 1024) {
            // The previous layer's FFN output may be pending as K-split partials.
            const int np = ffn_split && l > 0 ? kFfnParts : 0;
            ENG_TRY(launch_ln_shift(a.h, n, d, w.ln_t_w, w.ln_t_b, prev, a.slots, w.mix6, a.mix, plane,
                                    np ? a.kpart : nullptr, a.kplane, np, tl, st), "ln_shift");
        } else if (d <= 1024) {
            // LayerNorm + token shift in one pass; the last normed row of each
            // stream goes through a.hl (free until the LM head) to prev.
            ENG_TRY(launch_ln_shift_seq(a.h, n, Tc, d, w.ln_t_w, w.ln_t_b, prev, a.slots, w.mix6, a.mix, plane, a.hl,
                                        st), "ln_shift_seq");
            ENG_TRY(launch_save_prev(a.hl, n, 1, d, prev, a.slots, st), "save_prev");
        } else {
            ENG_TRY(launch_layernorm(a.h, M, d, w.ln_t_w, w.ln_t_b, nullptr, a.xn, st), "ln_time");
            ENG_TRY(launch_token_shift(a.xn, n, Tc, d, prev, a.slots, w.mix6, a.mix, plane, st), "token_shift");
            ENG_TRY(launch_save_prev(a.xn, n, Tc, d, prev, a.slots, st), "save_prev");
        }
        const float *mr = a.mix, *mw = a.mix + plane, *mk = a.mix + 2 * plane, *mv = a.mix + 3 * plane,
                    *ma = a.mix + 4 * plane, *mg = a.mix + 5 * plane;
        int rc;
        // Decode: the second low-rank stage runs inside the WKV step (which reads
        // the fp32 copy of w2t / a2t / g2t; bf16-valued in bf16 mode).
        const bool fuse_lr = Tc == 1 && e.decode_fusion && wkv7_step_lowrank_ok(s.head_size, L);
        {
            // r, k, v and the three low-rank first stages (one launch for short
            // products, two otherwise: the tile widths differ); then the second stages.
            float *lw = a.lr, *la = a.lr + lplane, *lg = a.lr + 2 * lplane;
            GemmParams g6[6] = {make_gemm(e, M, d, d, mr, d, w.w_r, d, a.r, d),
                                make_gemm(e, M, d, d, mk, d, w.w_k, d, a.k, d),
                                make_gemm(e, M, d, d, mv, d, w.w_v, d, a.v, d),
                                make_gemm(e, M, L, d, mw, d, w.w1t, d, lw, L, nullptr, ACT_TANH),
                                make_gemm(e, M, L, d, ma, d, w.a1t, d, la, L),
                                make_gemm(e, M, L, d, mg, d, w.g1t, d, lg, L)};
            if (M <= 64) {
                for (GemmParams &gp : g6) gp.a_tiled = tl;
                if ((rc = gemm_group(st, g6, 6)) != YUF_OK) return rc;
            } else {
                if ((rc = gemm_group(st, g6, 3)) != YUF_OK) return rc;
                if ((rc = gemm_group(st, g6 + 3, 3)) != YUF_OK) return rc;
            }
            if (!fuse_lr) {
                GemmParams l2[3] = {make_gemm(e, M, d, L, lw, L, w.w2t, L, a.wr, d, w.w0),
                                    make_gemm(e, M, d, L, la, L, w.a2t, L, a.al, d, w.a0, ACT_SIGMOID),
                                    make_gemm(e, M, d, L, lg, L, w.g2t, L, a.g, d, nullptr, ACT_SIGMOID)};
                if ((rc = gemm_group(st, l2, 3)) != YUF_OK) return rc;
            }
        }
        WkvParams wp;
        wp.B = n; wp.T = Tc; wp.H = s.heads;
        wp.r = a.r; wp.w = a.wr; wp.k = a.k; wp.v = a.v; wp.a = a.al;
        wp.k_k = w.k_k; wp.k_a = w.k_a;
        wp.state_in = wkv; wp.state_out = wkv; wp.slot = a.slots; wp.y = a.y;
        if (fuse_lr) {
            // The step kernel computes w, alpha and g from the rank-L rows.
            wp.lr = a.lr; wp.lr_plane = lplane; wp.L = L;
            wp.w2t = w.w2t; wp.a2t = w.a2t; wp.g2t = w.g2t; wp.w0 = w.w0; wp.a0 = w.a0; wp.g_out = a.g;
            wp.tiled_out = tl;
        }
        ENG_TRY(launch_wkv7(wp, s.head_size, true, st), "wkv7");
        if (fuse_lr && l == 0) {
            e.wkv_probe = wp;
            e.wkv_probe_set = true;
        }
        if ((rc = ln_gemm(e, st, M, d, d, a.y, d, w.ln_o_w, w.ln_o_b, a.g, a.z, w.w_o, a.h, d, nullptr, a.h, d, false,
                          tl)) != YUF_OK)
            return rc;
        // ROSA
        if ((rc = ln_gemm(e, st, M, 3 * D, d, a.h, d, w.ln_r_w, w.ln_r_b, nullptr, a.xn, w.rosa_w3, a.rosa3, 3 * D,
                          w.rosa_b3)) != YUF_OK)
            return rc;
        if (Tc == 1 && e.decode_fusion && rosa_out_decode_ok(M, D)) {
            // Decode: the ROSA step runs as the A prologue of the ROSA-out product.
            RosaOutParams ro;
            ro.M = M; ro.N = d; ro.D = D;
            ro.pre = a.rosa3; ro.ld_pre = 3 * D;
            ro.mem = ros; ro.mem_rows = e.max_streams; ro.slot = a.slots;
            ro.u = w.rosa_u; ro.lam = w.rosa_lam; ro.W = w.rosa_out;
            if (!e.w_h) ro.Wt = static_cast<const float *>(tiled_copy(e, w.rosa_out, D, &ro.wt_ld));
            ro.residual = a.h; ro.ldr = d; ro.C = a.h; ro.ldc = d;
            ro.counter = a.rcount;
            ENG_TRY(launch_rosa_out_decode(ro, st), "rosa out (fused step)");
        } else {
            RosaParams rp;
            rp.B = n; rp.T = Tc; rp.D = D; rp.ld = 3 * D;
            if (Tc == 1) {
                // The single-token kernel applies the gates itself.
                rp.cand = a.rosa3; rp.write = a.rosa3 + D; rp.read_raw = a.rosa3 + 2 * D;
            } else {
                // Gates on all M rows in parallel, so the sequential scan only loads e and the gate.
                ENG_TRY(launch_rosa_gates(a.rosa3, M, D, 3 * D, st), "rosa_gates");
                rp.e_pre = a.rosa3; rp.g_pre = a.rosa3 + D;
            }
            rp.decay = w.rosa_decay; rp.direction = w.rosa_hh; rp.raw_params = true;
            rp.memory_in = ros; rp.memory_out = ros; rp.slot = a.slots; rp.read_out = a.rread;
            if (e.rosa_segmented && Tc > 1 && rosa_segmented_ok(Tc, D, kRosaSeg)) {
                ENG_TRY(launch_rosa_segmented(rp, w.rosa_al, kRosaSeg, a.rz, a.rcarry, st), "rosa segmented");
            } else {
                ENG_TRY(launch_rosa(rp, st), "rosa");
            }
            if ((rc = gemm(e, st, M, d, D, a.rread, D, w.rosa_out, D, a.h, d, nullptr, ACT_NONE, a.h, d)) != YUF_OK)
                return rc;
        }
        // FFN
        if ((rc = ln_gemm(e, st, M, 2 * hid, d, a.h, d, w.ln_f_w, w.ln_f_b, nullptr, a.xn, w.ffn_cat, a.ffn, hid,
                          nullptr, nullptr, 0, true, false, tl)) != YUF_OK)
            return rc;
        if (ffn_split) {
            const int kp = hid / kFfnParts;
            GemmParams parts[kFfnParts];
            for (int q = 0; q < kFfnParts; ++q) {
                // Column q kp of the hidden rows: tile column q kp / 16 when tiled.
                const float *aq = a.ffn + (tl ? tile_index(0, q * kp, hid) : (size_t)q * kp);
                parts[q] = make_gemm(e, M, d, kp, aq, hid, w.ffn_out + (size_t)q * kp, hid,
                                     a.kpart + (size_t)q * a.kplane, d);
                parts[q].a_tiled = tl;
            }
            if ((rc = gemm_group(st, parts, kFfnParts)) != YUF_OK) return rc;
        } else if ((rc = gemm(e, st, M, d, hid, a.ffn, hid, w.ffn_out, hid, a.h, d, nullptr, ACT_NONE, a.h, d)) !=
                   YUF_OK) {
            return rc;
        }
    }
    if (l_end < s.layers) return YUF_OK;  // more layers follow in another call
    if (ffn_split && s.layers > 0)
        ENG_TRY(launch_add_parts(a.h, M, d, a.kpart, a.kplane, kFfnParts, st), "ffn partials");
    if (mode == YUF_LOGITS_LAST) return lm_head_last(e, a, n, Tc, logits);
    if (mode == kLogitsGather) {  // a part of a prefill: its last rows only
        if (Tc > 1) ENG_TRY(launch_gather_last(a.h, n, Tc, d, a.hl, st), "gather_last");
        return YUF_OK;
    }
    if (mode == YUF_LOGITS_ALL) {
        ENG_TRY(launch_layernorm(a.h, M, d, e.ln_fin_w, e.ln_fin_b, nullptr, a.xn, st), "ln_final");
        if (row_stride_T == Tc && t0 == 0) return gemm(e, st, M, V, d, a.xn, d, e.head, d, logits, V);
        for (int b = 0; b < n; ++b) {
            int rc = gemm(e, st, Tc, V, d, a.xn + (size_t)b * Tc * d, d, e.head, d,
                          logits + ((size_t)b * row_stride_T + t0) * V, V);
            if (rc != YUF_OK) return rc;
        }
    }
    return YUF_OK;
}

int check_slots(const Engine &e, int n, const int32_t *slots) {
    if (n <= 0) return fail(YUF_ERR_INVALID, "n must be positive");
    if (n > e.max_streams) return fail(YUF_ERR_RANGE, "more streams than the engine's max_streams");
    if (!slots) return fail(YUF_ERR_INVALID, "null slots");
    std::set<int> seen;
    for (int i = 0; i < n; ++i) {
        if (slots[i] < 0 || slots[i] >= e.max_streams)
            return fail(YUF_ERR_RANGE, "stream slot " + std::to_string(slots[i]) + " out of range");
        if (!seen.insert(slots[i]).second) return fail(YUF_ERR_INVALID, "duplicate stream slot in one call");
    }
    return YUF_OK;
}

int upload_slots(Engine &e, int n, const int32_t *slots) {
    std::vector<int> cur(slots, slots + n);
    if (cur == e.last_slots) return YUF_OK;
    std::memcpy(e.slots_host, slots, n * sizeof(int));
    ENG_TRY(hipMemcpyAsync(e.slots_dev, e.slots_host, n * sizeof(int), hipMemcpyHostToDevice, e.stream), "slots upload");
    ENG_TRY(hipStreamSynchronize(e.stream), "slots upload sync");
    e.last_slots = cur;
    return YUF_OK;
}

// The embedding's error flag for a call whose ids are at `tokens`: the host
// entry points stage their (validated) ids in host_tokens.
int *flag_for(Engine &e, const int32_t *tokens) {
    return tokens == static_cast<const int32_t *>(e.host_tokens.p) ? e.bad_host : e.bad_dev;
}

// Prefill n x T tokens (device pointer), splitting T into chunks of at most max_tokens / n.
int prefill_impl(Engine &e, int n, int T, const int32_t *tokens_dev, float *logits_dev, int mode) {
    const int tc_max = std::max(1, e.max_tokens / n);
    if (n > e.max_tokens) return fail(YUF_ERR_RANGE, "n exceeds max_tokens");
    for (int t0 = 0; t0 < T; t0 += tc_max) {
        const int tc = std::min(tc_max, T - t0);
        // Gather this chunk's token ids into [n, tc] rows.
        if (tc == T) {
            ENG_TRY(hipMemcpyAsync(e.tokens_dev, tokens_dev, (size_t)n * T * sizeof(int), hipMemcpyDeviceToDevice, e.stream),
                    "tokens copy");
        } else {
            ENG_TRY(hipMemcpy2DAsync(e.tokens_dev, (size_t)tc * sizeof(int), tokens_dev + t0, (size_t)T * sizeof(int),
                                     (size_t)tc * sizeof(int), n, hipMemcpyDeviceToDevice, e.stream),
                    "tokens copy");
        }
        const bool last_chunk = t0 + tc >= T;
        int chunk_mode = mode == YUF_LOGITS_ALL ? YUF_LOGITS_ALL : (last_chunk ? mode : YUF_LOGITS_NONE);
        // Parts of the batch on their own HIP streams when each part has at
        // least 256 rows: one part's latency-bound kernels (the scans, the
        // LayerNorms) run beside another part's GEMMs.  The parts touch
        // disjoint workspace rows, state slots and logit rows.  Automatic
        // count, measured on MI355X: four parts when the batch has at most 128
        // heads (C3, 8 x 2048: 25.5 ms per step as one part, 25.2 as two, 24.3
        // as three, 24.0 as four), else two (C5, 32 x 2048 chunks: bf16
        // prefill 722 ms as one part, 672 as two, 698 as four).
        int G = e.prefill_groups > 0 ? e.prefill_groups : ((size_t)n * e.s.heads <= 128 ? 4 : 2);
        G = std::min(G, n);
        while (G > 1 && (size_t)(n / G) * tc < 256) --G;
        if (G > 1) ENG_TRY(hipEventRecord(e.fork, e.stream), "fork record");
        // Join every side stream that waited on the fork back into e.stream,
        // on the error paths too: the next call's token copy and workspace
        // writes on e.stream must not overtake a side stream's kernels.
        int forked = 0;
        auto join_forked = [&]() -> hipError_t {
            hipError_t first = hipSuccess;
            for (int g = 1; g <= forked; ++g) {
                hipError_t err = hipEventRecord(e.join[g - 1], e.side[g - 1]);
                if (err == hipSuccess) err = hipStreamWaitEvent(e.stream, e.join[g - 1], 0);
                if (first == hipSuccess) first = err;
            }
            forked = 0;
            return first;
        };
        // Last-position logits of a split batch: the parts gather their last
        // rows and one LM head runs over all of them after the join (the same
        // kernel, so the same values, as for the whole batch in one part).
        const bool head_after = G > 1 && chunk_mode == YUF_LOGITS_LAST;
        if (head_after) chunk_mode = kLogitsGather;
        Act acts[Engine::kMaxBranches];
        float *lgs[Engine::kMaxBranches];
        int ns[Engine::kMaxBranches];
        for (int g = 0; g < G; ++g) {
            const int s0 = (int)((long long)n * g / G), s1 = (int)((long long)n * (g + 1) / G);
            hipStream_t st = g == 0 ? e.stream : e.side[g - 1];
            if (g > 0) {
                const hipError_t err = hipStreamWaitEvent(st, e.fork, 0);
                if (err != hipSuccess) {
                    (void)join_forked();
                    return hip_fail(err, "fork wait");
                }
                forked = g;
            }
            acts[g] = act_at(e, st, s0, tc);
            acts[g].bad = flag_for(e, tokens_dev);
            lgs[g] = logits_dev;
            if (lgs[g] && chunk_mode == YUF_LOGITS_ALL) lgs[g] += (size_t)s0 * T * e.s.vocab;
            else if (lgs[g] && chunk_mode == YUF_LOGITS_LAST) lgs[g] += (size_t)s0 * e.s.vocab;
            ns[g] = s1 - s0;
        }
        // Submitted a layer at a time across the parts, so every part starts
        // at once instead of waiting for the host to enqueue the whole pass of
        // the parts before it.
        const int layers = e.s.layers;
        for (int l = 0; l == 0 || l < layers; ++l) {
            const int l1 = G > 1 ? std::min(l + 1, layers) : layers;
            for (int g = 0; g < G; ++g) {
                const int rc = forward_pass(e, acts[g], ns[g], tc, lgs[g], chunk_mode, T, t0, l, l1);
                if (rc != YUF_OK) {
                    (void)join_forked();
                    return rc;
                }
            }
            if (l1 == layers) break;
        }
        ENG_TRY(join_forked(), "join");
        if (head_after) {
            const Act a0 = act_at(e, e.stream, 0, tc);
            const int rc = ln_gemm(e, e.stream, n, e.s.vocab, e.s.d, tc > 1 ? e.hl : e.h, e.s.d, e.ln_fin_w,
                                   e.ln_fin_b, nullptr, a0.xn, e.head, logits_dev, e.s.vocab);
            if (rc != YUF_OK) return rc;
        }
    }
    return YUF_OK;
}

// Capture `body` (launches on stream st) into an executable graph.
template <typename F>
int capture(hipStream_t st, F &&body, hipGraphExec_t *out) {
    ENG_TRY(hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal), "capture begin");
    const int rc = body();
    hipGraph_t graph = nullptr;
    const hipError_t ce = hipStreamEndCapture(st, &graph);
    if (rc != YUF_OK || ce != hipSuccess) {
        if (graph) (void)hipGraphDestroy(graph);
        return rc != YUF_OK ? rc : hip_fail(ce, "capture end");
    }
    const hipError_t ie = hipGraphInstantiate(out, graph, nullptr, nullptr, 0);
    (void)hipGraphDestroy(graph);
    if (ie != hipSuccess) {
        *out = nullptr;
        return hip_fail(ie, "graph instantiate");
    }
    return YUF_OK;
}

int drop_step_graphs(Engine &e) {
    for (auto &g : e.step_exec)
        if (g) {
            ENG_TRY(hipGraphExecDestroy(g), "graph destroy");
            g = nullptr;
        }
    return YUF_OK;
}

// One decode step (T = 1, last-position logits) of n streams whose slots are
// already on the device, replayed from captured graphs (kernel nodes only: no
// memset or copy nodes, no host synchronisation; the graphs read the caller's
// token ids in place and are captured again when n, the token pointer or the
// logits pointer changes).
// With one branch the whole step is one graph.  With G > 1 the streams are
// split into G groups whose layers are G graphs launched on G HIP streams
// (forked from and joined back into the engine stream with events, so the
// hardware queues run them side by side), then one graph with the final norm
// and the LM head over all n streams (its weights are read once per step).
int step_impl(Engine &e, int n, const int32_t *tokens_dev, float *logits_dev) {
    if (!e.use_graphs) return prefill_impl(e, n, 1, tokens_dev, logits_dev, YUF_LOGITS_LAST);
    // Measured on MI355X (0.1B model, 64 streams): one group 0.975 ms per step,
    // two 0.953, three 1.068 (21-row groups: no whole tiles), four 1.030.
    // Groups run concurrently and share e.gemm_ws, the split-K workspace of
    // short products, so they are used only when no decode product can take
    // the split-K path (every K a multiple of the decode kernel's k step).
    const int kq = e.w_h ? 8 : 4;
    const bool no_split_k = e.s.d % kq == 0 && e.s.low_rank % kq == 0 && e.s.rosa % kq == 0;
    int G = e.branches > 0 ? std::max(1, std::min(e.branches, n)) : (n >= 64 && n % 32 == 0 ? 2 : 1);
    if (!no_split_k || decode_layer_applies(e, n)) G = 1;
    auto group = [&](int g) { return std::make_pair((int)((long long)n * g / G), (int)((long long)n * (g + 1) / G)); };
    auto stream_of = [&](int g) { return g == 0 ? e.stream : e.side[g - 1]; };
    if (!(e.step_exec[0] && e.step_n == n && e.step_tok == tokens_dev && e.step_logits == logits_dev)) {
        int rc = drop_step_graphs(e);
        if (rc != YUF_OK) return rc;
        // The graphs read the caller's token ids in place (a graph is re-captured
        // when that pointer changes), so a replay needs no copy node.
        if (G == 1) {
            rc = capture(e.stream, [&]() {
                Act a = act_at(e, e.stream, 0, 1);
                a.tokens = tokens_dev;
                a.bad = flag_for(e, tokens_dev);
                return forward_pass(e, a, n, 1, logits_dev, YUF_LOGITS_LAST, 1, 0);
            }, &e.step_exec[0]);
        } else {
            for (int g = 0; g < G && rc == YUF_OK; ++g) {
                const auto [s0, s1] = group(g);
                hipStream_t st = stream_of(g);
                rc = capture(st, [&]() {
                    Act a = act_at(e, st, s0, 1);
                    a.grouped = true;
                    a.tokens = tokens_dev + s0;
                    a.bad = flag_for(e, tokens_dev);
                    return forward_pass(e, a, s1 - s0, 1, nullptr, YUF_LOGITS_NONE, 1, 0);
                }, &e.step_exec[g]);
            }
            if (rc == YUF_OK)
                rc = capture(e.stream, [&]() { return lm_head_last(e, act_at(e, e.stream, 0, 1), n, 1, logits_dev); },
                             &e.step_exec[G]);
        }
        if (rc != YUF_OK) {
            (void)drop_step_graphs(e);
            return rc;
        }
        e.step_n = n;
        e.step_tok = tokens_dev;
        e.step_logits = logits_dev;
    }
    if (G == 1) {
        ENG_TRY(hipGraphLaunch(e.step_exec[0], e.stream), "graph launch");
        return YUF_OK;
    }
    ENG_TRY(hipEventRecord(e.fork, e.stream), "fork record");
    // Every side stream that waited on the fork is joined back into e.stream,
    // also when a later launch fails.
    int forked = 0;
    hipError_t err = hipSuccess;
    for (int g = 1; g < G && err == hipSuccess; ++g)
        if ((err = hipStreamWaitEvent(e.side[g - 1], e.fork, 0)) == hipSuccess) forked = g;
    for (int g = 0; g < G && err == hipSuccess; ++g) err = hipGraphLaunch(e.step_exec[g], stream_of(g));
    for (int g = 1; g <= forked; ++g) {
        hipError_t je = hipEventRecord(e.join[g - 1], e.side[g - 1]);
        if (je == hipSuccess) je = hipStreamWaitEvent(e.stream, e.join[g - 1], 0);
        if (err == hipSuccess) err = je;
    }
    if (err != hipSuccess) return hip_fail(err, "step branches");
    ENG_TRY(hipGraphLaunch(e.step_exec[G], e.stream), "graph launch");
    return YUF_OK;
}

}  // namespace

}  // namespace yuf

// --------------------------------------------------------------------- C ABI
struct yuf_engine {
    yuf::Engine e;
};

using yuf::fail;

namespace {
const char *const kDecodeLayerTimeout =
    "a persistent decode layer gave up waiting at a stage barrier (its results are invalid; "
    "without YUF_DECODE_LAYER=1 the per-kernel decode path runs)";
}  // namespace

namespace {
// fp32 -> bf16 bits, round to nearest even (NaN stays NaN), as v_cvt_pk_bf16_f32.
uint16_t bf16_bits(float x) {
    uint32_t u;
    std::memcpy(&u, &x, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
    return (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}
}  // namespace

extern "C" int yuf_engine_create(const yuf_ckpt *ckpt, int max_streams, int max_tokens, yuf_engine **out) {
    return yuf_engine_create_ex(ckpt, max_streams, max_tokens, YUF_WEIGHTS_F32, out);
}

extern "C" int yuf_engine_create_ex(const yuf_ckpt *ckpt, int max_streams, int max_tokens, int weight_type,
                                    yuf_engine **out) {
    using namespace yuf;
    if (!ckpt || !out) return fail(YUF_ERR_INVALID, "yuf_engine_create: null argument");
    *out = nullptr;
    if (weight_type != YUF_WEIGHTS_F32 && weight_type != YUF_WEIGHTS_BF16)
        return fail(YUF_ERR_INVALID, "weight_type must be YUF_WEIGHTS_F32 or YUF_WEIGHTS_BF16");
    if (max_streams < 1 || max_tokens < 1) return fail(YUF_ERR_INVALID, "max_streams and max_tokens must be >= 1");
    const Checkpoint &ck = checkpoint_of(ckpt);
    const ModelShape &s = ck.shape;
    if (!wkv7_supported(s.head_size))
        return fail(YUF_ERR_INVALID, "head_size " + std::to_string(s.head_size) + " has no scan kernel");
    if (s.d > 64 * 32) return fail(YUF_ERR_INVALID, "d_model above 2048 is not supported");
    if (s.rosa > 1024) return fail(YUF_ERR_INVALID, "rosa_size above 1024 is not supported");
    if (weight_type == YUF_WEIGHTS_BF16) {
        auto wide_ok = [](long long n) { return n % 64 == 0 || n % 160 == 0; };
        if (s.d % 8 != 0 || s.low_rank % 8 != 0 || s.rosa % 8 != 0)
            return fail(YUF_ERR_INVALID, "bf16 weights need d_model, the low-rank width and rosa_size % 8 == 0");
        if (!wide_ok(s.d) || !wide_ok(s.low_rank) || !wide_ok(3LL * s.rosa) || !wide_ok(s.vocab))
            return fail(YUF_ERR_INVALID, "bf16 weights need d_model, the low-rank width, 3 rosa_size and the vocabulary "
                                         "to be multiples of 64 or 160");
    }
    std::unique_ptr<yuf_engine> h(new (std::nothrow) yuf_engine());
    if (!h) return fail(YUF_ERR_OOM, "host allocation failed");
    Engine &e = h->e;
    e.s = s;
    if (const char *ng = std::getenv("YUF_NO_GRAPH")) e.use_graphs = std::strcmp(ng, "1") != 0;
    if (const char *rs = std::getenv("YUF_ROSA_SEGMENTED")) e.rosa_segmented = std::strcmp(rs, "0") != 0;
    if (const char *dt = std::getenv("YUF_DECODE_TILES")) e.act_tiles = std::strcmp(dt, "0") != 0;
    if (const char *pg = std::getenv("YUF_PREFILL_GROUPS")) e.prefill_groups = std::max(1, std::min(std::atoi(pg), Engine::kMaxBranches));
    if (const char *df = std::getenv("YUF_DECODE_FUSION")) e.decode_fusion = std::strcmp(df, "0") != 0;
    // Opt-in: measured at 1.94 ms per 64-stream 0.1B step against 0.955 ms for
    // the per-kernel step (every XCD streams every weight).
    bool want_dl = false;
    if (const char *dl = std::getenv("YUF_DECODE_LAYER")) want_dl = std::strcmp(dl, "1") == 0;
    e.max_streams = max_streams;
    e.max_tokens = max_tokens;

    std::vector<float> host;
    std::vector<size_t> offs;
    std::string err;
    try {
        int rc = build_weights(ck, host, offs, err, weight_type == YUF_WEIGHTS_BF16);
        if (rc != YUF_OK) return fail(rc, err);
    } catch (const std::bad_alloc &) {
        return fail(YUF_ERR_OOM, "out of host memory preparing weights");
    }
    ENG_TRY(hipStreamCreateWithFlags(&e.stream, hipStreamNonBlocking), "stream create");
    e.branches = 0;  // automatic
    if (const char *b = std::getenv("YUF_DECODE_BRANCHES"))
        e.branches = std::max(1, std::min(std::atoi(b), (int)Engine::kMaxBranches));
    for (int i = 0; i + 1 < Engine::kMaxBranches; ++i) {
        ENG_TRY(hipStreamCreateWithFlags(&e.side[i], hipStreamNonBlocking), "side stream create");
        ENG_TRY(hipEventCreateWithFlags(&e.join[i], hipEventDisableTiming), "event create");
    }
    ENG_TRY(hipEventCreateWithFlags(&e.fork, hipEventDisableTiming), "event create");
    ENG_TRY(hipMalloc(&e.weights.p, host.size() * sizeof(float)), "weights alloc");
    ENG_TRY(hipMemcpy(e.weights.p, host.data(), host.size() * sizeof(float), hipMemcpyHostToDevice), "weights upload");
    const float *base = static_cast<const float *>(e.weights.p);
    if (weight_type == YUF_WEIGHTS_BF16) {
        std::vector<uint16_t> hb;
        try {
            hb.resize(host.size());
        } catch (const std::bad_alloc &) {
            return fail(YUF_ERR_OOM, "out of host memory preparing bf16 weights");
        }
        for (size_t i = 0; i < host.size(); ++i) hb[i] = bf16_bits(host[i]);
        ENG_TRY(hipMalloc(&e.weights_h.p, hb.size() * sizeof(uint16_t)), "bf16 weights alloc");
        ENG_TRY(hipMemcpy(e.weights_h.p, hb.data(), hb.size() * sizeof(uint16_t), hipMemcpyHostToDevice),
                "bf16 weights upload");
        e.w_base = base;
        e.w_floats = host.size();
        e.w_h = static_cast<const uint16_t *>(e.weights_h.p);
    }
    size_t oi = 0;
    auto nxt = [&]() { return base + offs[oi++]; };
    e.emb = nxt();
    e.head = nxt();
    e.ln_fin_w = nxt();
    e.ln_fin_b = nxt();
    e.layers.resize(s.layers);
    for (int l = 0; l < s.layers; ++l) {
        LayerW &w = e.layers[l];
        w.ln_t_w = nxt(); w.ln_t_b = nxt(); w.mix6 = nxt();
        w.w_r = nxt(); w.w_k = nxt(); w.w_v = nxt(); w.w_o = nxt();
        w.w1t = nxt(); w.w2t = nxt(); w.a1t = nxt(); w.a2t = nxt(); w.g1t = nxt(); w.g2t = nxt();
        w.w0 = nxt(); w.a0 = nxt(); w.k_k = nxt(); w.k_a = nxt();
        w.ln_o_w = nxt(); w.ln_o_b = nxt(); w.ln_r_w = nxt(); w.ln_r_b = nxt();
        w.rosa_w3 = nxt(); w.rosa_b3 = nxt(); w.rosa_hh = nxt(); w.rosa_decay = nxt(); w.rosa_out = nxt();
        w.ln_f_w = nxt(); w.ln_f_b = nxt(); w.ffn_cat = nxt(); w.ffn_out = nxt();
        w.rosa_al = nxt();
        w.rosa_u = nxt(); w.rosa_lam = nxt();
    }
    {
        // Tiled copies of the decode products' matrices (from the host image).
        const long long d = s.d, L = s.low_rank, D = s.rosa, V = s.vocab, hid = 4LL * s.d;
        std::vector<Engine::Tiled> mats;
        mats.push_back({e.head, V, d, nullptr, 0, nullptr});
        for (const LayerW &w : e.layers) {
            for (const float *m : {w.w_r, w.w_k, w.w_v, w.w_o}) mats.push_back({m, d, d, nullptr, 0, nullptr});
            for (const float *m : {w.w1t, w.a1t, w.g1t}) mats.push_back({m, L, d, nullptr, 0, nullptr});
            for (const float *m : {w.w2t, w.a2t, w.g2t}) mats.push_back({m, d, L, nullptr, 0, nullptr});
            mats.push_back({w.rosa_w3, 3 * D, d, nullptr, 0, nullptr});
            mats.push_back({w.rosa_out, d, D, nullptr, 0, nullptr});
            mats.push_back({w.ffn_cat, 2 * hid, d, nullptr, 0, nullptr});
            mats.push_back({w.ffn_out, d, hid, nullptr, 0, nullptr});
        }
        const bool bf16 = e.w_h != nullptr;
        const int kt = bf16 ? 32 : 16, esz = bf16 ? 2 : 4;
        size_t total = 0;
        std::vector<size_t> at;
        for (Engine::Tiled &t : mats) {
            t.wt_ld = (int)(((t.cols + kt - 1) / kt) * 16 * kt);
            at.push_back(total);
            total += (((size_t)((t.rows + 15) / 16) * t.wt_ld * esz + 255) / 256) * 256 / esz;
        }
        std::vector<uint16_t> th;
        std::vector<float> tf;
        try {
            if (bf16) th.assign(total, 0);
            else tf.assign(total, 0.0f);
        } catch (const std::bad_alloc &) {
            return fail(YUF_ERR_OOM, "out of host memory preparing tiled weights");
        }
        for (size_t i = 0; i < mats.size(); ++i) {
            const Engine::Tiled &t = mats[i];
            const float *src = host.data() + (t.base - base);
            for (long long r = 0; r < t.rows; ++r)
                for (long long c = 0; c < t.cols; ++c) {
                    const size_t o = at[i] + (size_t)(r / 16) * t.wt_ld + (size_t)(c / kt) * 16 * kt + (r % 16) * kt + c % kt;
                    if (bf16) th[o] = bf16_bits(src[r * t.cols + c]);
                    else tf[o] = src[r * t.cols + c];
                }
        }
        ENG_TRY(hipMalloc(&e.weights_t.p, total * esz), "tiled weights alloc");
        ENG_TRY(hipMemcpy(e.weights_t.p, bf16 ? (const void *)th.data() : (const void *)tf.data(), total * esz,
                          hipMemcpyHostToDevice),
                "tiled weights upload");
        for (size_t i = 0; i < mats.size(); ++i)
            mats[i].tiles = static_cast<const char *>(e.weights_t.p) + at[i] * esz;
        e.tiled = std::move(mats);
        // fp32 mode: every projection matrix pre-split for the prefill's X3
        // products (1.5 x the matrices' fp32 bytes; YUF_GEMM_PLANES=0 skips it).
        const char *pe = std::getenv("YUF_GEMM_PLANES");
        if (!bf16 && !(pe && std::strcmp(pe, "0") == 0)) {
            size_t ptotal = 0;
            std::vector<size_t> pat;
            for (const Engine::Tiled &t : e.tiled) {
                const size_t n = x3_planes_elems((int)t.rows, (int)t.cols);
                pat.push_back(n ? ptotal : SIZE_MAX);
                ptotal += ((n * 2 + 255) / 256) * 128;
            }
            if (ptotal) {
                ENG_TRY(hipMalloc(&e.weights_p.p, ptotal * 2), "weight planes alloc");
                uint16_t *pb = static_cast<uint16_t *>(e.weights_p.p);
                for (size_t i = 0; i < e.tiled.size(); ++i) {
                    Engine::Tiled &t = e.tiled[i];
                    if (pat[i] == SIZE_MAX) continue;
                    t.planes = pb + pat[i];
                    ENG_TRY(launch_x3_split_planes(t.base, (int)t.cols, (int)t.rows, (int)t.cols, pb + pat[i], e.stream),
                            "weight planes split");
                }
                ENG_TRY(hipStreamSynchronize(e.stream), "weight planes sync");
            }
        }
    }

    // State: [layer][slot][...] for each of prev, wkv, rosa.
    const size_t n_prev = (size_t)s.layers * max_streams * s.d;
    const size_t n_wkv = (size_t)s.layers * max_streams * e.wkv_floats();
    const size_t n_rosa = (size_t)s.layers * max_streams * s.rosa;
    const size_t state_bytes = (n_prev + n_wkv + n_rosa) * sizeof(float) + 3 * 256;
    ENG_TRY(hipMalloc(&e.state.p, state_bytes), "state alloc");
    {
        char *cur = static_cast<char *>(e.state.p);
        e.st_prev = carve<float>(cur, n_prev);
        e.st_wkv = carve<float>(cur, n_wkv);
        e.st_rosa = carve<float>(cur, n_rosa);
    }
    ENG_TRY(hipMemsetAsync(e.state.p, 0, state_bytes, e.stream), "state clear");

    // Workspace.
    const size_t Mx = (size_t)max_tokens, d = s.d;
    size_t ws = 0;
    {
        const int D = s.rosa, L = s.low_rank, dd = s.d;
        const int shapes[][2] = {{dd, dd}, {L, dd}, {dd, L}, {3 * D, dd}, {dd, D}, {8 * dd, dd}, {dd, 4 * dd},
                                 {s.vocab, dd}};
        for (auto &nk : shapes) ws = std::max(ws, gemm_workspace_floats(nk[0], nk[1]));
    }
    e.gemm_ws_floats = ws;
    const size_t sizes[] = {Mx * d, Mx * d, 6 * Mx * d, Mx * d, Mx * d, Mx * d, Mx * d, Mx * d, Mx * d,
                            3 * Mx * s.low_rank, Mx * d, Mx * d, Mx * 3 * s.rosa, Mx * s.rosa, Mx * 4 * d,
                            (size_t)max_streams * d, ws, Mx / kRosaSeg * s.rosa + s.rosa, Mx / kRosaSeg * s.rosa + s.rosa,
                            (size_t)kFfnParts * max_streams * d};
    size_t total = 0;
    for (size_t z : sizes) total += ((z * sizeof(float) + 255) / 256) * 256;
    ENG_TRY(hipMalloc(&e.work.p, total), "workspace alloc");
    {
        char *cur = static_cast<char *>(e.work.p);
        float **dst[] = {&e.h, &e.xn, &e.mix, &e.r, &e.k, &e.v, &e.wr, &e.al, &e.g, &e.lr, &e.y, &e.z, &e.rosa3,
                         &e.rread, &e.ffn, &e.hl, &e.gemm_ws, &e.rz, &e.rcarry, &e.kpart};
        for (size_t i = 0; i < sizeof(sizes) / sizeof(sizes[0]); ++i) *dst[i] = carve<float>(cur, sizes[i]);
    }
    const size_t io_bytes = 256 * 5 + (size_t)(2 * max_streams + max_tokens + 2) * sizeof(int);
    ENG_TRY(hipMalloc(&e.io.p, io_bytes), "io alloc");
    {
        char *cur = static_cast<char *>(e.io.p);
        e.slots_dev = carve<int>(cur, max_streams);
        e.tokens_dev = carve<int>(cur, max_tokens);
        e.bad_dev = carve<int>(cur, 1);
        e.bad_host = carve<int>(cur, 1);
        e.rosa_count = carve<int>(cur, max_streams);
    }
    ENG_TRY(hipHostMalloc(reinterpret_cast<void **>(&e.slots_host), max_streams * sizeof(int)), "pinned alloc");
    // Persistent decode layers: fp32 weights (their tiled copies), a supported
    // shape, and the device's XCD count; one workgroup per CU.
    if (want_dl && weight_type == YUF_WEIGHTS_F32 && decode_layer_ok(s.d, s.heads, s.head_size, s.low_rank, s.rosa)) {
        int dev = 0, xccs = 0, cus = 0;
        ENG_TRY(hipGetDevice(&dev), "device query");
        if (hipDeviceGetAttribute(&xccs, hipDeviceAttributeNumberOfXccs, dev) != hipSuccess) xccs = 0;
        ENG_TRY(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev), "device query");
        (void)hipGetLastError();
        if (xccs >= 1 && xccs <= 16 && cus >= xccs) {
            e.dl_groups = xccs;
            e.dl_grid = cus / xccs * xccs;
            e.dl_sync_ints = decode_layer_sync_ints(xccs, e.dl_grid);
            const size_t gf = decode_layer_group_floats(s.d, s.low_rank, s.rosa);
            const size_t bytes = ((gf * xccs * sizeof(float) + 255) / 256) * 256 + e.dl_sync_ints * s.layers * sizeof(int);
            ENG_TRY(hipMalloc(&e.dl.p, bytes), "decode layer buffers");
            e.dl_buf = static_cast<float *>(e.dl.p);
            e.dl_sync = reinterpret_cast<int *>(static_cast<char *>(e.dl.p) + ((gf * xccs * sizeof(float) + 255) / 256) * 256);
            e.decode_layer = true;
        }
    }
    ENG_TRY(hipMemsetAsync(e.bad_dev, 0, sizeof(int), e.stream), "flag clear");
    ENG_TRY(hipMemsetAsync(e.bad_host, 0, sizeof(int), e.stream), "flag clear");
    // Tile counters of the fused ROSA-out decode kernel: zero here, and every
    // launch leaves them at zero (outside any captured graph).
    ENG_TRY(hipMemsetAsync(e.rosa_count, 0, (size_t)max_streams * sizeof(int), e.stream), "counter clear");
    ENG_TRY(hipStreamSynchronize(e.stream), "engine init sync");
    *out = h.release();
    return YUF_OK;
}

extern "C" void yuf_engine_destroy(yuf_engine *eng) { delete eng; }

extern "C" int yuf_engine_config(const yuf_engine *eng, yuf_model_config *out) {
    if (!eng || !out) return fail(YUF_ERR_INVALID, "yuf_engine_config: null argument");
    yuf::fill_config(eng->e.s, *out);
    return YUF_OK;
}

extern "C" void *yuf_engine_stream(yuf_engine *eng) { return eng ? static_cast<void *>(eng->e.stream) : nullptr; }

namespace {

int check_tokens_host(const yuf::Engine &e, const int32_t *tokens, size_t count) {
    if (!tokens) return fail(YUF_ERR_INVALID, "null tokens");
    for (size_t i = 0; i < count; ++i)
        if (tokens[i] < 0 || tokens[i] >= e.s.vocab)
            return fail(YUF_ERR_RANGE, "token id " + std::to_string(tokens[i]) + " out of range [0, " +
                                           std::to_string(e.s.vocab) + ")");
    return YUF_OK;
}

}  // namespace

extern "C" int yuf_prefill_device(yuf_engine *eng, int n, const int32_t *slots, int T, const int32_t *tokens_dev,
                                  float *logits_dev, int logits_mode) {
    using namespace yuf;
    if (!eng) return fail(YUF_ERR_INVALID, "null engine");
    Engine &e = eng->e;
    int rc = check_slots(e, n, slots);
    if (rc != YUF_OK) return rc;
    if (T < 0) return fail(YUF_ERR_INVALID, "negative T");
    if (T == 0) return YUF_OK;
    if (logits_mode < YUF_LOGITS_NONE || logits_mode > YUF_LOGITS_ALL) return fail(YUF_ERR_INVALID, "bad logits mode");
    if (!tokens_dev || (logits_mode != YUF_LOGITS_NONE && !logits_dev)) return fail(YUF_ERR_INVALID, "null buffer");
    if ((rc = upload_slots(e, n, slots)) != YUF_OK) return rc;
    return prefill_impl(e, n, T, tokens_dev, logits_dev, logits_mode);
}

extern "C" int yuf_prefill(yuf_engine *eng, int n, const int32_t *slots, int T, const int32_t *tokens, float *logits,
                           int logits_mode) {
    using namespace yuf;
    if (!eng) return fail(YUF_ERR_INVALID, "null engine");
    Engine &e = eng->e;
    int rc = check_slots(e, n, slots);
    if (rc != YUF_OK) return rc;
    if (T < 0) return fail(YUF_ERR_INVALID, "negative T");
    if (T == 0) return YUF_OK;
    if (logits_mode < YUF_LOGITS_NONE || logits_mode > YUF_LOGITS_ALL) return fail(YUF_ERR_INVALID, "bad logits mode");
    if ((rc = check_tokens_host(e, tokens, (size_t)n * T)) != YUF_OK) return rc;
    if (logits_mode != YUF_LOGITS_NONE && !logits) return fail(YUF_ERR_INVALID, "null logits");
    const size_t n_logits =
        logits_mode == YUF_LOGITS_ALL ? (size_t)n * T * e.s.vocab : (logits_mode == YUF_LOGITS_LAST ? (size_t)n * e.s.vocab : 0);
    const size_t n_tok = (size_t)n * T;
    if (n_tok > e.host_tokens_cap) {
        if (e.host_tokens.p) ENG_TRY(hipFree(e.host_tokens.p), "token buffer");
        e.host_tokens.p = nullptr;
        e.host_tokens_cap = 0;
        ENG_TRY(hipMalloc(&e.host_tokens.p, n_tok * sizeof(int)), "token buffer");
        e.host_tokens_cap = n_tok;
    }
    if (n_logits > e.host_logits_cap) {
        if (e.host_logits.p) ENG_TRY(hipFree(e.host_logits.p), "logits buffer");
        e.host_logits.p = nullptr;
        e.host_logits_cap = 0;
        ENG_TRY(hipMalloc(&e.host_logits.p, n_logits * sizeof(float)), "logits buffer");
        e.host_logits_cap = n_logits;
    }
    ENG_TRY(hipMemcpyAsync(e.host_tokens.p, tokens, n_tok * sizeof(int), hipMemcpyHostToDevice, e.stream),
            "tokens upload");
    if ((rc = upload_slots(e, n, slots)) != YUF_OK) return rc;
    if (T == 1 && logits_mode == YUF_LOGITS_LAST)
        rc = step_impl(e, n, static_cast<int *>(e.host_tokens.p), static_cast<float *>(e.host_logits.p));
    else
        rc = prefill_impl(e, n, T, static_cast<int *>(e.host_tokens.p), static_cast<float *>(e.host_logits.p),
                          logits_mode);
    if (rc != YUF_OK) return rc;
    if (n_logits)
        ENG_TRY(hipMemcpyAsync(logits, e.host_logits.p, n_logits * sizeof(float), hipMemcpyDeviceToHost, e.stream),
                "logits download");
    int bad = 0;
    ENG_TRY(hipMemcpyAsync(&bad, e.bad_host, sizeof(int), hipMemcpyDeviceToHost, e.stream), "flag read");
    ENG_TRY(hipStreamSynchronize(e.stream), "prefill sync");
    if (bad) {
        ENG_TRY(hipMemsetAsync(e.bad_host, 0, sizeof(int), e.stream), "flag clear");
        ENG_TRY(hipStreamSynchronize(e.stream), "flag clear sync");
        if (bad & 2) return fail(YUF_ERR_HIP, kDecodeLayerTimeout);
        return fail(YUF_ERR_RANGE, "a token id was out of range on the device (its embedding was zeroed)");
    }
    return YUF_OK;
}

extern "C" int yuf_engine_time_wkv_step(yuf_engine *eng, int iters, float *avg_us, int *streams) {
    using namespace yuf;
    if (!eng || !avg_us || iters < 1) return fail(YUF_ERR_INVALID, "time_wkv_step: bad arguments");
    Engine &e = eng->e;
    if (!e.wkv_probe_set) return fail(YUF_ERR_INVALID, "time_wkv_step: no decode step has run the fused WKV-7 step yet");
    // Same launch as the step's first layer, but the new state goes to a
    // scratch copy, so the engine's state is not advanced.
    WkvParams wp = e.wkv_probe;
    const size_t floats = (size_t)e.max_streams * e.wkv_floats();
    DeviceBuf scratch;
    ENG_TRY(hipMalloc(&scratch.p, floats * sizeof(float)), "time_wkv_step scratch");
    wp.state_out = static_cast<float *>(scratch.p);
    // The launches are captured into one HIP graph and replayed, as the
    // decode step replays its own: back-to-back launches from the host leave
    // a dispatch gap of ~5 us after each ~8 us kernel, which events would
    // count as kernel time; graph-replayed kernels are ~2 us apart.
    hipEvent_t t0 = nullptr, t1 = nullptr;
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    ENG_TRY(hipEventCreate(&t0), "event");
    hipError_t err = hipEventCreate(&t1);
    if (err == hipSuccess) err = launch_wkv7(wp, e.s.head_size, true, e.stream);  // warm-up
    if (err == hipSuccess) err = hipStreamBeginCapture(e.stream, hipStreamCaptureModeThreadLocal);
    if (err == hipSuccess) {
        for (int i = 0; i < iters && err == hipSuccess; ++i) err = launch_wkv7(wp, e.s.head_size, true, e.stream);
        const hipError_t end = hipStreamEndCapture(e.stream, &graph);  // always ends the capture
        if (err == hipSuccess) err = end;
    }
    if (err == hipSuccess) err = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
    if (err == hipSuccess) err = hipGraphLaunch(exec, e.stream);  // warm-up replay
    if (err == hipSuccess) err = hipEventRecord(t0, e.stream);
    if (err == hipSuccess) err = hipGraphLaunch(exec, e.stream);
    if (err == hipSuccess) err = hipEventRecord(t1, e.stream);
    if (err == hipSuccess) err = hipEventSynchronize(t1);
    float ms = 0.f;
    if (err == hipSuccess) err = hipEventElapsedTime(&ms, t0, t1);
    if (exec) (void)hipGraphExecDestroy(exec);
    if (graph) (void)hipGraphDestroy(graph);
    hipEventDestroy(t0);
    if (t1) hipEventDestroy(t1);
    if (err != hipSuccess) return fail(YUF_ERR_HIP, std::string("time_wkv_step: ") + hipGetErrorString(err));
    *avg_us = ms * 1e3f / iters;
    if (streams) *streams = wp.B;
    return YUF_OK;
}

extern "C" int yuf_engine_take_error(yuf_engine *eng) {
    using namespace yuf;
    if (!eng) return fail(YUF_ERR_INVALID, "null engine");
    Engine &e = eng->e;
    int bad = 0;
    ENG_TRY(hipMemcpyAsync(&bad, e.bad_dev, sizeof(int), hipMemcpyDeviceToHost, e.stream), "flag read");
    ENG_TRY(hipStreamSynchronize(e.stream), "flag read sync");
    if (!bad) return YUF_OK;
    ENG_TRY(hipMemsetAsync(e.bad_dev, 0, sizeof(int), e.stream), "flag clear");
    ENG_TRY(hipStreamSynchronize(e.stream), "flag clear sync");
    if (bad & 2) return fail(YUF_ERR_HIP, kDecodeLayerTimeout);
    return fail(YUF_ERR_RANGE, "a device-side token id was out of range in a yuf_prefill_device / yuf_step_device call "
                               "(its embedding was zeroed)");
}

extern "C" int yuf_step_device(yuf_engine *eng, int n, const int32_t *slots, const int32_t *tokens_dev,
                               float *logits_dev) {
    using namespace yuf;
    if (!eng) return fail(YUF_ERR_INVALID, "null engine");
    Engine &e = eng->e;
    int rc = check_slots(e, n, slots);
    if (rc != YUF_OK) return rc;
    if (!tokens_dev || !logits_dev) return fail(YUF_ERR_INVALID, "null buffer");
    if ((rc = upload_slots(e, n, slots)) != YUF_OK) return rc;
    return step_impl(e, n, tokens_dev, logits_dev);
}

extern "C" int yuf_step(yuf_engine *eng, int n, const int32_t *slots, const int32_t *tokens, float *logits) {
    return yuf_prefill(eng, n, slots, 1, tokens, logits, YUF_LOGITS_LAST);
}

extern "C" int yuf_state_reset(yuf_engine *eng, int slot) {
    using namespace yuf;
    if (!eng) return fail(YUF_ERR_INVALID, "null engine");
    Engine &e = eng->e;
    if (slot < -1 || slot >= e.max_streams) return fail(YUF_ERR_RANGE, "slot out of range");
    const int first = slot < 0 ? 0 : slot, count = slot < 0 ? e.max_streams : 1;
    for (int l = 0; l < e.s.layers; ++l) {
        struct { float *base; size_t per; } parts[3] = {
            {e.st_prev + (size_t)l * e.max_streams * e.s.d, (size_t)e.s.d},
            {e.st_wkv + (size_t)l * e.max_streams * e.wkv_floats(), e.wkv_floats()},
            {e.st_rosa + (size_t)l * e.max_streams * e.s.rosa, (size_t)e.s.rosa}};
        for (auto &p : parts)
            ENG_TRY(launch_fill(p.base + (size_t)first * p.per, (size_t)count * p.per, 0.0f, e.stream), "state reset");
    }
    ENG_TRY(hipStreamSynchronize(e.stream), "state reset sync");
    return YUF_OK;
}

extern "C" size_t yuf_state_size(const yuf_engine *eng) {
    return eng ? eng->e.state_floats() * sizeof(float) : 0;
}

namespace {
int state_copy(yuf::Engine &e, int slot, float *host, bool save) {
    using namespace yuf;
    if (slot < 0 || slot >= e.max_streams) return fail(YUF_ERR_RANGE, "slot out of range");
    if (!host) return fail(YUF_ERR_INVALID, "null state buffer");
    size_t off = 0;
    for (int l = 0; l < e.s.layers; ++l) {
        struct { float *dev; size_t n; } parts[3] = {
            {e.st_prev + ((size_t)l * e.max_streams + slot) * e.s.d, (size_t)e.s.d},
            {e.st_wkv + ((size_t)l * e.max_streams + slot) * e.wkv_floats(), e.wkv_floats()},
            {e.st_rosa + ((size_t)l * e.max_streams + slot) * e.s.rosa, (size_t)e.s.rosa}};
        for (auto &p : parts) {
            if (save)
                ENG_TRY(hipMemcpyAsync(host + off, p.dev, p.n * sizeof(float), hipMemcpyDeviceToHost, e.stream), "state save");
            else
                ENG_TRY(hipMemcpyAsync(p.dev, host + off, p.n * sizeof(float), hipMemcpyHostToDevice, e.stream), "state load");
            off += p.n;
        }
    }
    ENG_TRY(hipStreamSynchronize(e.stream), "state copy sync");
    return YUF_OK;
}
}  // namespace

extern "C" int yuf_state_save(yuf_engine *eng, int slot, void *host_buf) {
    if (!eng) return fail(YUF_ERR_INVALID, "null engine");
    return state_copy(eng->e, slot, static_cast<float *>(host_buf), true);
}

extern "C" int yuf_state_load(yuf_engine *eng, int slot, const void *host_buf) {
    if (!eng) return fail(YUF_ERR_INVALID, "null engine");
    return state_copy(eng->e, slot, static_cast<float *>(const_cast<void *>(host_buf)), false);
}
