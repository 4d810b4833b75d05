// Shared device/host helpers for the gfx950 routed-attention kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/hga.h"

namespace hga {

constexpr int kWave = 64;

// ---------------------------------------------------------------------------------------------
// host-side error reporting (per thread)
// ---------------------------------------------------------------------------------------------
void set_error(const char* fmt, ...);
int launch_status(const char* what);  // HGA_OK or HGA_ERR_LAUNCH after a kernel launch

#define HGA_REQUIRE(cond, code, ...)   \
    do {                               \
        if (!(cond)) {                 \
            ::hga::set_error(__VA_ARGS__); \
            return (code);             \
        }                              \
    } while (0)

int check_config(const hga_config* cfg);

// ---------------------------------------------------------------------------------------------
// element access.  bf16 values travel as raw uint16 bit patterns.
// ---------------------------------------------------------------------------------------------
__device__ __forceinline__ float bf16_to_f(uint16_t h) { return __uint_as_float((uint32_t)h << 16); }

// round-to-nearest-even float -> bf16 bits (NaN kept quiet)
__device__ __forceinline__ uint16_t f_to_bf16(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7f800000u) == 0x7f800000u) return (uint16_t)((u >> 16) | ((u & 0xffffu) ? 0x40u : 0u));
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

__device__ __forceinline__ float round_dt(float x, int dt) {
    return dt == HGA_DTYPE_BF16 ? bf16_to_f(f_to_bf16(x)) : x;
}

template <int DT>
struct Elem;
template <>
struct Elem<HGA_DTYPE_F32> {
    typedef float T;
    static __device__ __forceinline__ float ld(const T* p, int64_t i) { return p[i]; }
    static __device__ __forceinline__ void st(T* p, int64_t i, float v) { p[i] = v; }
};
template <>
struct Elem<HGA_DTYPE_BF16> {
    typedef uint16_t T;
    static __device__ __forceinline__ float ld(const T* p, int64_t i) { return bf16_to_f(p[i]); }
    static __device__ __forceinline__ void st(T* p, int64_t i, float v) { p[i] = f_to_bf16(v); }
};

// ---------------------------------------------------------------------------------------------
// wave-wide helpers (64 lanes)
// ---------------------------------------------------------------------------------------------
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, kWave));
    return v;
}
__device__ __forceinline__ float wave_min(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fminf(v, __shfl_xor(v, o, kWave));
    return v;
}
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
    return v;
}
__device__ __forceinline__ int wave_sum_i(int v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
    return v;
}

__device__ __forceinline__ int lane_id() { return (int)(threadIdx.x & (kWave - 1)); }

// Number of set bits of `mask` in lanes below the calling lane.
__device__ __forceinline__ int lanes_below(uint64_t mask) {
    return __popcll(mask & ((1ull << lane_id()) - 1ull));
}

// Orderable unsigned key of a float (larger float -> larger key); -0 maps to +0's key.
__device__ __forceinline__ uint32_t okey(float f) {
    if (f == 0.0f) f = 0.0f;
    uint32_t u = __float_as_uint(f);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float okey_inv(uint32_t k) {
    uint32_t u = (k & 0x80000000u) ? (k & 0x7fffffffu) : ~k;
    return __uint_as_float(u);
}

// Window ranges for a query chunk / decode step with `n` earlier chunks
// (vectorized.py:246-253; chunk_placement_policy.py:27-38).
// Chunks of a block of S tokens (S up to INT32_MAX: computed in 64 bits).
__host__ __device__ __forceinline__ int chunks_of(int64_t S, int C) { return (int)((S + C - 1) / C); }

__host__ __device__ __forceinline__ void windows(int n, int kf, int kl, int* f_hi, int* l_lo) {
    *f_hi = kf > 0 ? (n < kf ? n : kf) : 0;
    if (kl > 0) {
        int x = n - kl > kf ? n - kl : kf;
        *l_lo = x < n ? x : n;
    } else {
        *l_lo = n;
    }
}

}  // namespace hga
