// Shared helpers for the libyufhip.so sources: error reporting across the C
// ABI, HIP status checks and wavefront (wave64) reduction primitives.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <string>

#include "../../include/yuf_engine.h"

namespace yuf {

// Thread-local message behind yuf_last_error().
void set_error(const std::string &msg);
int fail(int status, const std::string &msg);

#define YUF_HIP_TRY(expr)                                                              \
    do {                                                                               \
        hipError_t yuf_err_ = (expr);                                                  \
        if (yuf_err_ != hipSuccess)                                                    \
            return ::yuf::fail(YUF_ERR_HIP, std::string(#expr " failed: ") +           \
                                                hipGetErrorString(yuf_err_));          \
    } while (0)

// Launch-time check: a kernel launch reports configuration errors through
// hipGetLastError.
#define YUF_LAUNCH_CHECK(what)                                                         \
    do {                                                                               \
        hipError_t yuf_err_ = hipGetLastError();                                       \
        if (yuf_err_ != hipSuccess)                                                    \
            return ::yuf::fail(YUF_ERR_HIP, std::string(what " launch failed: ") +     \
                                                hipGetErrorString(yuf_err_));          \
    } while (0)

// ---------------------------------------------------------------------------
// DPP lane permutations (gfx9 encodings).  All lanes enabled, bound_ctrl off:
// every lane reads an in-range source lane for the patterns used here.
// ---------------------------------------------------------------------------
namespace dpp {
constexpr int kQuadXor1 = 0xB1;       // quad_perm [1,0,3,2]
constexpr int kQuadXor2 = 0x4E;       // quad_perm [2,3,0,1]
constexpr int kRowHalfMirror = 0x141; // lane k <-> 7-k inside each 8-lane half row
constexpr int kRowMirror = 0x140;     // lane k <-> 15-k inside each 16-lane row
}  // namespace dpp

template <int CTRL>
__device__ __forceinline__ float dpp_move(float x) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xF, 0xF, false));
}

// Sum over aligned groups of G consecutive lanes (G in {1,2,4,8,16}); every
// lane of the group receives the group sum.  Pure DPP, no LDS traffic.
template <int G>
__device__ __forceinline__ float group_sum(float x) {
    static_assert(G == 1 || G == 2 || G == 4 || G == 8 || G == 16, "group size");
    if constexpr (G >= 2) x += dpp_move<dpp::kQuadXor1>(x);
    if constexpr (G >= 4) x += dpp_move<dpp::kQuadXor2>(x);
    if constexpr (G >= 8) x += dpp_move<dpp::kRowHalfMirror>(x);
    if constexpr (G >= 16) x += dpp_move<dpp::kRowMirror>(x);
    return x;
}

// Full 64-lane sum, returned (uniform) to every lane.
__device__ __forceinline__ float wave_sum(float x) {
    x = group_sum<16>(x);
    const float s0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 0));
    const float s1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 16));
    const float s2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 32));
    const float s3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 48));
    return (s0 + s1) + (s2 + s3);
}

// Full 64-lane sum of a double, returned to every lane with the same bits:
// DPP inside each 16-lane row (each step adds a pair of partial sums that both
// lanes of the pair see, so commutativity keeps them equal), then the gfx950
// row swaps pair rows (0,1) (2,3) and then (0,2) (1,3).  No LDS traffic.
template <int CTRL>
__device__ __forceinline__ double dpp_move_f64(double x) {
    const uint64_t b = __builtin_bit_cast(uint64_t, x);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)b, CTRL, 0xF, 0xF, false);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)(b >> 32), CTRL, 0xF, 0xF, false);
    return __builtin_bit_cast(double, ((uint64_t)hi << 32) | lo);
}

// Sum over the four lanes l % 16 == const (one per 16-lane row), returned to
// those four lanes with the same bits.
__device__ __forceinline__ double rows_sum_f64(double x) {
    uint64_t b = __builtin_bit_cast(uint64_t, x);
    const auto l16 = __builtin_amdgcn_permlane16_swap((uint32_t)b, (uint32_t)b, false, false);
    const auto h16 = __builtin_amdgcn_permlane16_swap((uint32_t)(b >> 32), (uint32_t)(b >> 32), false, false);
    x = __builtin_bit_cast(double, ((uint64_t)h16[0] << 32) | l16[0]) +
        __builtin_bit_cast(double, ((uint64_t)h16[1] << 32) | l16[1]);
    b = __builtin_bit_cast(uint64_t, x);
    const auto l32 = __builtin_amdgcn_permlane32_swap((uint32_t)b, (uint32_t)b, false, false);
    const auto h32 = __builtin_amdgcn_permlane32_swap((uint32_t)(b >> 32), (uint32_t)(b >> 32), false, false);
    return __builtin_bit_cast(double, ((uint64_t)h32[0] << 32) | l32[0]) +
           __builtin_bit_cast(double, ((uint64_t)h32[1] << 32) | l32[1]);
}

__device__ __forceinline__ double wave_sum_f64(double x) {
    x += dpp_move_f64<dpp::kQuadXor1>(x);
    x += dpp_move_f64<dpp::kQuadXor2>(x);
    x += dpp_move_f64<dpp::kRowHalfMirror>(x);
    x += dpp_move_f64<dpp::kRowMirror>(x);
    return rows_sum_f64(x);
}

__device__ __forceinline__ float sigmoidf_(float x) { return 1.0f / (1.0f + expf(-x)); }

// Workgroup barrier that orders LDS only.  __syncthreads() also releases
// global memory at workgroup scope, which makes every wave wait for its
// outstanding global loads -- including prefetches meant to stay in flight
// across the barrier.  The kernels here exchange data through LDS only.
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// ---------------------------------------------------------------------------
// Raw buffer loads: the hardware bounds-checks every access against the
// descriptor's byte range and returns 0 outside it, so staging loops need no
// per-element branches (branches around loads make the compiler serialise
// them with conservative vmcnt waits).  `base` must be wave-uniform.
// ---------------------------------------------------------------------------
constexpr uint32_t kBufferOob = 0x80000000u;  // an offset past any range used here

// Decode activations in 16 x 16 tiles: element (r, c) of a [rows][ld] matrix at
// [r / 16][c / 16][r % 16][c % 16] (row-tile stride 16 ld floats), so the 16
// rows x 16 columns a wave reads per k step are one contiguous 1 KB run.
__host__ __device__ __forceinline__ size_t tile_index(int r, int c, int ld) {
    return (size_t)(r >> 4) * 16 * ld + (size_t)(c >> 4) * 256 + (r & 15) * 16 + (c & 15);
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void *base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), 0, bytes, 0x00020000);
}

__device__ __forceinline__ float buf_load(__amdgpu_buffer_rsrc_t rsrc, uint32_t byte_offset) {
    return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rsrc, byte_offset, 0, 0));
}

__device__ __forceinline__ void buf_store(float value, __amdgpu_buffer_rsrc_t rsrc, uint32_t byte_offset) {
    __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, value), rsrc, byte_offset, 0, 0);
}

// s_waitcnt vmcnt(0): retire this wave's outstanding global loads here, so the
// compiler's conservative wait insertion does not place a full wait inside a
// later loop (where it would also wait for prefetches issued in that loop).
__device__ __forceinline__ void wait_vmem() { __builtin_amdgcn_s_waitcnt(0x0F70); }

inline int ceil_div(int a, int b) { return (a + b - 1) / b; }

}  // namespace yuf
