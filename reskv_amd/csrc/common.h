// Shared device helpers for the ResKV gfx950 library.
//
// Wave64 conventions used throughout: a "lane" is one of the 64 work-items of a
// wavefront; lane L usually owns head channels L and L + 64, which is exactly a
// rotate-half RoPE pair (frequency index L).
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

namespace reskv {

constexpr int kDim = 128;
constexpr int kHalf = 64;
constexpr int kWave = 64;
constexpr int kMaxClusters = 64;

// ---------------------------------------------------------------------------
// bit casts and fp16 conversions (round-to-nearest-even)
// ---------------------------------------------------------------------------
__device__ __forceinline__ float h2f(uint16_t bits) {
    return __half2float(__ushort_as_half(bits));
}
__device__ __forceinline__ uint16_t f2h(float x) {
    return __half_as_ushort(__float2half_rn(x));
}
__device__ __forceinline__ int f2i(float x) { return __builtin_bit_cast(int, x); }
__device__ __forceinline__ float i2f(int x) { return __builtin_bit_cast(float, x); }

// ---------------------------------------------------------------------------
// cross-lane helpers (DPP row operations + readlane), wave64 only
// ---------------------------------------------------------------------------
// dpp_ctrl encodings (GCN/CDNA DPP): quad_perm xor1 = 0xB1, quad_perm xor2 = 0x4E,
// row_half_mirror = 0x141, row_mirror = 0x140.
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
    return i2f(__builtin_amdgcn_update_dpp(0, f2i(v), CTRL, 0xF, 0xF, false));
}
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xF, 0xF, false);
}

__device__ __forceinline__ float readlane(float v, int lane) {
    return i2f(__builtin_amdgcn_readlane(f2i(v), lane));
}

// Sum of v over the 16 lanes of each DPP row, returned in every lane of the row.
__device__ __forceinline__ float row_sum16(float v) {
    v += dpp<0xB1>(v);
    v += dpp<0x4E>(v);
    v += dpp<0x141>(v);
    v += dpp<0x140>(v);
    return v;
}
__device__ __forceinline__ float row_max16(float v) {
    v = fmaxf(v, dpp<0xB1>(v));
    v = fmaxf(v, dpp<0x4E>(v));
    v = fmaxf(v, dpp<0x141>(v));
    v = fmaxf(v, dpp<0x140>(v));
    return v;
}
// Wave-wide sum, uniform result.  Fixed association order: ((r0+r1)+(r2+r3)).
__device__ __forceinline__ float wave_sum(float v) {
    v = row_sum16(v);
    const float r0 = readlane(v, 0), r1 = readlane(v, 16);
    const float r2 = readlane(v, 32), r3 = readlane(v, 48);
    return (r0 + r1) + (r2 + r3);
}
__device__ __forceinline__ float wave_max(float v) {
    v = row_max16(v);
    const float r0 = readlane(v, 0), r1 = readlane(v, 16);
    const float r2 = readlane(v, 32), r3 = readlane(v, 48);
    return fmaxf(fmaxf(r0, r1), fmaxf(r2, r3));
}

// Orders this wave's LDS traffic: writes before the call are visible to every
// lane of the same wave after it.
__device__ __forceinline__ void wave_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// 64-bit lane mask of lanes where pred holds (wave-uniform result).
__device__ __forceinline__ uint64_t ballot(bool pred) {
    return __builtin_amdgcn_ballot_w64(pred);
}
// Number of set bits of mask in lanes below this lane.
__device__ __forceinline__ uint32_t lanes_below(uint64_t mask) {
    return __builtin_amdgcn_mbcnt_hi((uint32_t)(mask >> 32),
                                     __builtin_amdgcn_mbcnt_lo((uint32_t)mask, 0u));
}
__device__ __forceinline__ int lane_id() { return (int)__builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u)); }

// ---------------------------------------------------------------------------
// RoPE angle: theta = fl32(position * frequency), evaluated by an accurate
// sincos (the device libm, correctly range-reduced for large arguments).
// ---------------------------------------------------------------------------
__device__ __forceinline__ void rope_sincos(float position, float freq, float* s, float* c) {
    const float theta = __fmul_rn(position, freq);
    sincosf(theta, s, c);
}

}  // namespace reskv

// Host-side error reporting shared by all translation units.
namespace reskv_host {
void set_error(const char* fmt, ...);
int check_launch(const char* what);
}  // namespace reskv_host

#define RESKV_REQUIRE(cond, ...)                   \
    do {                                           \
        if (!(cond)) {                             \
            reskv_host::set_error(__VA_ARGS__);    \
            return 1;                              \
        }                                          \
    } while (0)
