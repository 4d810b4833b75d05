// Rotate-half RoPE applied in fp32 and rounded to the activation dtype
// (HierarchicalGlobalAttentionRouted.py:156-157, 219-223), or with every step rounded to the
// activation dtype (x*cos, rotate_half(x)*sin and their sum, as transformers'
// apply_rotary_pos_emb computes them on bf16 tensors: qwen_routed_attention.py:176, :80-84).
// HBM-bound elementwise kernel:
// each thread owns 8 (bf16) or 4 (fp32) consecutive dims of the first half and the matching ones
// of the second half of one row, so every load/store is a 16-byte vector access.
// Built with -ffp-contract=off: x*cos and rot*sin are rounded separately, then added, as torch's
// eager ops do.
#include "hga_common.h"

namespace hga {
namespace {

// VEC consecutive elements of a row per access: 8 bf16 (16 bytes) or 4 fp32 (16 bytes).
template <int DT>
struct Vec;
template <>
struct Vec<HGA_DTYPE_BF16> {
    static constexpr int N = 8, kBytes = 2;
    static __device__ __forceinline__ void ld(const void* p, float* v) {
        const uint4 u = *reinterpret_cast<const uint4*>(p);
        const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            v[2 * e] = __uint_as_float(w[e] << 16);
            v[2 * e + 1] = __uint_as_float(w[e] & 0xffff0000u);
        }
    }
    static __device__ __forceinline__ void st(void* p, const float* v) {
        uint32_t w[4];
#pragma unroll
        for (int e = 0; e < 4; ++e)
            w[e] = (uint32_t)f_to_bf16(v[2 * e]) | ((uint32_t)f_to_bf16(v[2 * e + 1]) << 16);
        *reinterpret_cast<uint4*>(p) = make_uint4(w[0], w[1], w[2], w[3]);
    }
};
template <>
struct Vec<HGA_DTYPE_F32> {
    static constexpr int N = 4, kBytes = 4;
    static __device__ __forceinline__ void ld(const void* p, float* v) {
        const float4 u = *reinterpret_cast<const float4*>(p);
        v[0] = u.x; v[1] = u.y; v[2] = u.z; v[3] = u.w;
    }
    static __device__ __forceinline__ void st(void* p, const float* v) {
        *reinterpret_cast<float4*>(p) = make_float4(v[0], v[1], v[2], v[3]);
    }
};

template <int N>
__device__ __forceinline__ void ld_tab(const float* p, float* v) {
#pragma unroll
    for (int e = 0; e < N; e += 4) {
        const float4 u = *reinterpret_cast<const float4*>(p + e);
        v[e] = u.x; v[e + 1] = u.y; v[e + 2] = u.z; v[e + 3] = u.w;
    }
}

// One tensor's rows: [B, X, S, Dh] input and output views (element strides b, head, position).
struct RopeSet {
    const char* x;
    char* out;
    int64_t x_sb, x_sh, x_ss, o_sb, o_sh, o_ss, nrows;
    int X;
};

// HPT rows per thread: consecutive heads of one (position, batch), so the position's cos/sin
// slices are loaded once for all of them (HPT divides the head count).  blk: the workgroup's
// index within this tensor's part of the grid.
template <int DT, bool STEPS, int HPT>
__device__ __forceinline__ void rope_rows(const RopeSet& R, int64_t blk, const float* cos,
                                          const float* sin, int64_t cos_bstride, int S, int Dh) {
    constexpr int N = Vec<DT>::N, E = Vec<DT>::kBytes;
    const int half = Dh / 2, tpr = half / N, rpb = 256 / tpr;
    const int64_t row0 = (blk * rpb + threadIdx.x / tpr) * HPT;
    if (row0 >= R.nrows) return;
    const int d0 = (threadIdx.x % tpr) * N;
    // rows in (position, batch, head) order, heads fastest: the heads of one position share
    // its cos/sin row while it is in cache (head-major order would stream the whole table
    // once per head)
    const int64_t BX = R.nrows / S;
    const int s = (int)(row0 / BX);
    const int64_t bx = row0 % BX;
    const int h0 = (int)(bx % R.X);
    const int64_t b = bx / R.X;
    const float* cr = cos + b * cos_bstride + (int64_t)s * Dh;
    const float* sr = sin + b * cos_bstride + (int64_t)s * Dh;
    float x1[HPT][N], x2[HPT][N], c1[N], c2[N], s1[N], s2[N];
#pragma unroll
    for (int k = 0; k < HPT; ++k) {
        const char* xr = R.x + (b * R.x_sb + (h0 + k) * R.x_sh + s * R.x_ss) * E;
        Vec<DT>::ld(xr + d0 * E, x1[k]);
        Vec<DT>::ld(xr + (d0 + half) * E, x2[k]);
    }
    ld_tab<N>(cr + d0, c1);
    ld_tab<N>(cr + d0 + half, c2);
    ld_tab<N>(sr + d0, s1);
    ld_tab<N>(sr + d0 + half, s2);
#pragma unroll
    for (int k = 0; k < HPT; ++k) {
        float o1[N], o2[N];
#pragma unroll
        for (int e = 0; e < N; ++e) {
            float a = x1[k][e] * c1[e];
            float r1 = -x2[k][e] * s1[e];
            float c = x2[k][e] * c2[e];
            float r2 = x1[k][e] * s2[e];
            if constexpr (STEPS) {
                a = round_dt(a, DT);
                r1 = round_dt(r1, DT);
                c = round_dt(c, DT);
                r2 = round_dt(r2, DT);
            }
            o1[e] = a + r1;
            o2[e] = c + r2;
        }
        char* orow = R.out + (b * R.o_sb + (h0 + k) * R.o_sh + s * R.o_ss) * E;
        Vec<DT>::st(orow + d0 * E, o1);
        Vec<DT>::st(orow + (d0 + half) * E, o2);
    }
}

// Workgroups [0, g0) rotate set 0 (H0 heads per thread), the rest set 1 (H1): q and k of a
// block in one launch, so k's small grid fills q's tail instead of running after it.
template <int DT, bool STEPS, int H0, int H1>
__global__ __launch_bounds__(256) void rope_kernel(RopeSet r0, RopeSet r1, int64_t g0,
                                                   const float* cos, const float* sin,
                                                   int64_t cos_bstride, int S, int Dh) {
    const int64_t blk = blockIdx.x;
    if (blk < g0) rope_rows<DT, STEPS, H0>(r0, blk, cos, sin, cos_bstride, S, Dh);
    else rope_rows<DT, STEPS, H1>(r1, blk - g0, cos, sin, cos_bstride, S, Dh);
}

}  // namespace
}  // namespace hga

namespace hga {
namespace {

int rope_launch(const hga_config* cfg, int S, RopeSet* sets, int nsets, const float* cos,
                const float* sin, int64_t cos_bstride, int32_t flags, void* stream,
                const char* what) {
    int rc = check_config(cfg);
    if (rc) return rc;
    HGA_REQUIRE(cos && sin, HGA_ERR_ARG, "%s: NULL pointer", what);
    HGA_REQUIRE(S >= 0, HGA_ERR_ARG, "%s: bad S", what);
    HGA_REQUIRE((flags & ~HGA_ROPE_STEPS_IN_DTYPE) == 0, HGA_ERR_ARG, "%s: unknown flags", what);
    const int Dh = cfg->head_dim;
    const bool bf = cfg->dtype == HGA_DTYPE_BF16;
    const int N = bf ? 8 : 4;   // elements per 16-byte access
    HGA_REQUIRE((Dh / 2) % N == 0, HGA_ERR_UNSUPPORTED, "%s: head_dim %d not a multiple of %d",
                what, Dh, 2 * N);
    HGA_REQUIRE(((uintptr_t)cos % 16) == 0 && ((uintptr_t)sin % 16) == 0 && (cos_bstride % 4) == 0,
                HGA_ERR_ARG, "%s: rotary tables must allow 16-byte vector access", what);
    const int tpr = Dh / 2 / N, rpb = 256 / tpr;
    int hpt[2] = {1, 1};
    int64_t g[2] = {0, 0};
    for (int i = 0; i < nsets; ++i) {
        RopeSet& R = sets[i];
        HGA_REQUIRE(R.x && R.out, HGA_ERR_ARG, "%s: NULL pointer", what);
        HGA_REQUIRE(R.X > 0, HGA_ERR_ARG, "%s: bad head count", what);
        const uintptr_t al = (uintptr_t)R.x | (uintptr_t)R.out;
        HGA_REQUIRE((al % 16) == 0 &&
                        ((R.x_sb | R.x_sh | R.x_ss | R.o_sb | R.o_sh | R.o_ss) % N) == 0,
                    HGA_ERR_ARG, "%s: pointers/strides must allow 16-byte vector access", what);
        R.nrows = (int64_t)cfg->batch * R.X * S;
        // heads per thread (rows stay within a position); four only while the tensor's grid
        // keeps at least 2048 workgroups (8 per CU)
        hpt[i] = R.X % 4 == 0 && R.nrows / 4 >= (int64_t)2048 * rpb ? 4 : 1;
        g[i] = (R.nrows / hpt[i] + rpb - 1) / rpb;
    }
    if (S == 0) return HGA_OK;
    RopeSet none{};
    const RopeSet& r1 = nsets > 1 ? sets[1] : none;
    const int64_t grid = g[0] + g[1];
    hipStream_t st = (hipStream_t)stream;
    const bool steps = (flags & HGA_ROPE_STEPS_IN_DTYPE) != 0;
    auto launch = [&](auto kern) {
        kern<<<dim3((unsigned)grid), dim3(256), 0, st>>>(sets[0], r1, g[0], cos, sin, cos_bstride,
                                                         S, Dh);
    };
    auto by_heads = [&](auto k11, auto k14, auto k41, auto k44) {
        if (hpt[0] == 4) hpt[1] == 4 ? launch(k44) : launch(k41);
        else hpt[1] == 4 ? launch(k14) : launch(k11);
    };
    constexpr int B16 = HGA_DTYPE_BF16, F32 = HGA_DTYPE_F32;
    if (bf && steps)
        by_heads(rope_kernel<B16, true, 1, 1>, rope_kernel<B16, true, 1, 4>,
                 rope_kernel<B16, true, 4, 1>, rope_kernel<B16, true, 4, 4>);
    else if (bf)
        by_heads(rope_kernel<B16, false, 1, 1>, rope_kernel<B16, false, 1, 4>,
                 rope_kernel<B16, false, 4, 1>, rope_kernel<B16, false, 4, 4>);
    else   // fp32: every step is already fp32
        by_heads(rope_kernel<F32, false, 1, 1>, rope_kernel<F32, false, 1, 4>,
                 rope_kernel<F32, false, 4, 1>, rope_kernel<F32, false, 4, 4>);
    return launch_status(what);
}

}  // namespace
}  // namespace hga

extern "C" int hga_rope(const hga_config* cfg, int32_t nheads, int32_t S, const void* x,
                        int64_t x_sb, int64_t x_sh, int64_t x_ss, void* out, int64_t o_sb,
                        int64_t o_sh, int64_t o_ss, const float* cos, const float* sin,
                        int64_t cos_bstride, int32_t flags, void* stream) {
    using namespace hga;
    HGA_REQUIRE(x && out, HGA_ERR_ARG, "hga_rope: NULL pointer");
    RopeSet r{(const char*)x, (char*)out, x_sb, x_sh, x_ss, o_sb, o_sh, o_ss, 0, nheads};
    return rope_launch(cfg, S, &r, 1, cos, sin, cos_bstride, flags, stream, "hga_rope");
}

extern "C" int hga_rope_qk(const hga_config* cfg, int32_t S, const void* q, int64_t q_sb,
                           int64_t q_sh, int64_t q_ss, void* q_out, int64_t qo_sb, int64_t qo_sh,
                           int64_t qo_ss, const void* k, int64_t k_sb, int64_t k_sh, int64_t k_ss,
                           void* k_out, int64_t ko_sb, int64_t ko_sh, int64_t ko_ss,
                           const float* cos, const float* sin, int64_t cos_bstride,
                           int32_t flags, void* stream) {
    using namespace hga;
    HGA_REQUIRE(q && q_out && k && k_out, HGA_ERR_ARG, "hga_rope_qk: NULL pointer");
    RopeSet r[2] = {
        {(const char*)q, (char*)q_out, q_sb, q_sh, q_ss, qo_sb, qo_sh, qo_ss, 0, cfg ? cfg->heads : 0},
        {(const char*)k, (char*)k_out, k_sb, k_sh, k_ss, ko_sb, ko_sh, ko_ss, 0,
         cfg ? cfg->kv_heads : 0}};
    return rope_launch(cfg, S, r, 2, cos, sin, cos_bstride, flags, stream, "hga_rope_qk");
}
