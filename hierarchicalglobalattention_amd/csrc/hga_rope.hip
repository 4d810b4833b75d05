// Rotate-half RoPE applied in fp32 and rounded to the activation dtype
// (HierarchicalGlobalAttentionRouted.py:156-157, 219-223), or with every step rounded to the
// activation dtype (x*cos, rotate_half(x)*sin and their sum, as transformers'
// apply_rotary_pos_emb computes them on bf16 tensors: qwen_routed_attention.py:176, :80-84).
// HBM-bound elementwise kernel:
// each thread owns 4 consecutive dims of the first half and the matching 4 of the second half
// of one row, so every load/store is an 8-byte (bf16) or 16-byte (fp32) vector access.
// Built with -ffp-contract=off: x*cos and rot*sin are rounded separately, then added, as torch's
// eager ops do.
#include "hga_common.h"

namespace hga {
namespace {

template <int DT>
struct Vec4;
template <>
struct Vec4<HGA_DTYPE_BF16> {
    static __device__ __forceinline__ void ld(const void* p, float* v) {
        uint2 u = *reinterpret_cast<const uint2*>(p);
        v[0] = __uint_as_float(u.x << 16);
        v[1] = __uint_as_float(u.x & 0xffff0000u);
        v[2] = __uint_as_float(u.y << 16);
        v[3] = __uint_as_float(u.y & 0xffff0000u);
    }
    static __device__ __forceinline__ void st(void* p, const float* v) {
        uint2 u;
        u.x = (uint32_t)f_to_bf16(v[0]) | ((uint32_t)f_to_bf16(v[1]) << 16);
        u.y = (uint32_t)f_to_bf16(v[2]) | ((uint32_t)f_to_bf16(v[3]) << 16);
        *reinterpret_cast<uint2*>(p) = u;
    }
    static constexpr int kBytes = 2;
};
template <>
struct Vec4<HGA_DTYPE_F32> {
    static __device__ __forceinline__ void ld(const void* p, float* v) {
        float4 u = *reinterpret_cast<const float4*>(p);
        v[0] = u.x; v[1] = u.y; v[2] = u.z; v[3] = u.w;
    }
    static __device__ __forceinline__ void st(void* p, const float* v) {
        *reinterpret_cast<float4*>(p) = make_float4(v[0], v[1], v[2], v[3]);
    }
    static constexpr int kBytes = 4;
};

template <int DT, bool STEPS>
__global__ __launch_bounds__(256) void rope_kernel(const char* x, int64_t x_sb, int64_t x_sh,
                                                   int64_t x_ss, char* out, int64_t o_sb,
                                                   int64_t o_sh, int64_t o_ss, const float* cos,
                                                   const float* sin, int64_t cos_bstride, int X,
                                                   int S, int Dh, int64_t nrows) {
    const int half = Dh / 2, tpr = half / 4, rpb = 256 / tpr;
    const int64_t row = (int64_t)blockIdx.x * rpb + threadIdx.x / tpr;
    if (row >= nrows) return;
    const int d0 = (threadIdx.x % tpr) * 4;
    // rows in (position, batch, head) order, heads fastest: the heads of one position share
    // its cos/sin row while it is in cache (head-major order would stream the whole table
    // once per head)
    const int64_t BX = nrows / S;
    const int s = (int)(row / BX);
    const int64_t bx = row % BX;
    const int h = (int)(bx % X);
    const int64_t b = bx / X;
    constexpr int E = Vec4<DT>::kBytes;
    const char* xr = x + (b * x_sb + h * x_sh + s * x_ss) * E;
    char* orow = out + (b * o_sb + h * o_sh + s * o_ss) * E;
    const float* cr = cos + b * cos_bstride + (int64_t)s * Dh;
    const float* sr = sin + b * cos_bstride + (int64_t)s * Dh;
    float x1[4], x2[4], o1[4], o2[4];
    Vec4<DT>::ld(xr + d0 * E, x1);
    Vec4<DT>::ld(xr + (d0 + half) * E, x2);
    const float4 c1 = *reinterpret_cast<const float4*>(cr + d0);
    const float4 c2 = *reinterpret_cast<const float4*>(cr + d0 + half);
    const float4 s1 = *reinterpret_cast<const float4*>(sr + d0);
    const float4 s2 = *reinterpret_cast<const float4*>(sr + d0 + half);
    const float cc1[4] = {c1.x, c1.y, c1.z, c1.w}, cc2[4] = {c2.x, c2.y, c2.z, c2.w};
    const float ss1[4] = {s1.x, s1.y, s1.z, s1.w}, ss2[4] = {s2.x, s2.y, s2.z, s2.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        float a = x1[e] * cc1[e];
        float r1 = -x2[e] * ss1[e];
        float c = x2[e] * cc2[e];
        float r2 = x1[e] * ss2[e];
        if constexpr (STEPS) {
            a = round_dt(a, DT);
            r1 = round_dt(r1, DT);
            c = round_dt(c, DT);
            r2 = round_dt(r2, DT);
        }
        o1[e] = a + r1;
        o2[e] = c + r2;
    }
    Vec4<DT>::st(orow + d0 * E, o1);
    Vec4<DT>::st(orow + (d0 + half) * E, o2);
}

}  // namespace
}  // namespace hga

extern "C" int hga_rope(const hga_config* cfg, int32_t nheads, int32_t S, const void* x,
                        int64_t x_sb, int64_t x_sh, int64_t x_ss, void* out, int64_t o_sb,
                        int64_t o_sh, int64_t o_ss, const float* cos, const float* sin,
                        int64_t cos_bstride, int32_t flags, void* stream) {
    using namespace hga;
    int rc = check_config(cfg);
    if (rc) return rc;
    HGA_REQUIRE(x && out && cos && sin, HGA_ERR_ARG, "hga_rope: NULL pointer");
    HGA_REQUIRE(nheads > 0 && S >= 0, HGA_ERR_ARG, "hga_rope: bad nheads/S");
    HGA_REQUIRE((flags & ~HGA_ROPE_STEPS_IN_DTYPE) == 0, HGA_ERR_ARG, "hga_rope: unknown flags");
    if (S == 0) return HGA_OK;
    const int Dh = cfg->head_dim;
    const int E = cfg->dtype == HGA_DTYPE_BF16 ? 2 : 4;
    const uintptr_t al = (uintptr_t)x | (uintptr_t)out;
    HGA_REQUIRE((al % (4 * E)) == 0 && ((x_sb | x_sh | x_ss | o_sb | o_sh | o_ss) % 4) == 0 &&
                    ((uintptr_t)cos % 16) == 0 && ((uintptr_t)sin % 16) == 0 &&
                    (cos_bstride % 4) == 0,
                HGA_ERR_ARG, "hga_rope: pointers/strides must allow 4-element vector access");
    const int tpr = Dh / 8, rpb = 256 / tpr;
    const int64_t nrows = (int64_t)cfg->batch * nheads * S;
    const int64_t grid = (nrows + rpb - 1) / rpb;
    hipStream_t st = (hipStream_t)stream;
    const bool steps = (flags & HGA_ROPE_STEPS_IN_DTYPE) != 0;
    auto launch = [&](auto kern) {
        kern<<<dim3((unsigned)grid), dim3(256), 0, st>>>((const char*)x, x_sb, x_sh, x_ss,
                                                         (char*)out, o_sb, o_sh, o_ss, cos, sin,
                                                         cos_bstride, nheads, S, Dh, nrows);
    };
    if (cfg->dtype == HGA_DTYPE_BF16) {
        if (steps) launch(rope_kernel<HGA_DTYPE_BF16, true>);
        else launch(rope_kernel<HGA_DTYPE_BF16, false>);
    } else {
        launch(rope_kernel<HGA_DTYPE_F32, false>);   // fp32: every step is already fp32
    }
    return launch_status("hga_rope");
}
