// Mixed-RoPE chunk/group key summaries at KV-head granularity
// (vectorized._rope_summary, vectorized.py:146-183 applied at :265-287; store twin
//  ChunkRouter._rope_summary_at, chunk_router.py:575-585, 631-652, 693-735).
//
// One workgroup per (chunk n, kv head, batch).  Each thread owns a pair of adjacent dims of one
// group and sums the group's valid tokens sequentially in fp32 (k_raw and k_rope at once, two
// coalesced 4/8-byte loads per token row); chunk sums are the sequential fp32 sum of the four
// unrounded group sums.  Then the reference's dtype roundings, the anchor rotation in fp32 and
// the mixed tokenwise/anchor select.  The reference computes this at query-head granularity
// after repeat_interleave (chunk_router.py:540), i.e. rep times over; KV heads suffice.
// Built with -ffp-contract=off so each product/sum rounds exactly as the oracle does.
#include "hga_common.h"

namespace hga {
namespace {

constexpr int kSumThreads = 256;

template <int DT>
__global__ __launch_bounds__(kSumThreads) void summarize_kernel(
    const typename Elem<DT>::T* k_raw, int64_t kr_sb, int64_t kr_sh, int64_t kr_ss,
    const typename Elem<DT>::T* k_rope, int64_t kp_sb, int64_t kp_sh, int64_t kp_ss,
    const float* cos_a, const float* sin_a, typename Elem<DT>::T* ck_a,
    typename Elem<DT>::T* gk_a, const float* cos_b, const float* sin_b,
    typename Elem<DT>::T* ck_b, typename Elem<DT>::T* gk_b, int64_t ck_sb, int64_t ck_sh,
    int64_t gk_sb, int64_t gk_sh, int64_t pos0, int S, int Dh, int C, int gs, int cutoff,
    float gscale) {
    typedef Elem<DT> E;
    extern __shared__ float smem[];
    const int n = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
    const int M = C / gs, half = Dh / 2;
    float* graw = smem;              // [M][Dh] unrounded group sums
    float* grope = graw + M * Dh;
    float* traw = grope + M * Dh;    // [M+1][Dh] rounded, scaled raw sums (row M = chunk)
    float* ttok = traw + (M + 1) * Dh;
    int len = S - n * C;
    if (len > C) len = C;

    const typename E::T* kr = k_raw + b * kr_sb + h * kr_sh;
    const typename E::T* kp = k_rope + b * kp_sb + h * kp_sh;
    for (int task = threadIdx.x; task < M * half; task += kSumThreads) {
        const int m = task / half, d = 2 * (task % half);
        int glen = len - m * gs;
        glen = glen < 0 ? 0 : (glen > gs ? gs : glen);
        float r0 = 0.0f, r1 = 0.0f, p0 = 0.0f, p1 = 0.0f;
        const int64_t t0 = (int64_t)n * C + m * gs;
#pragma unroll 4
        for (int t = 0; t < glen; ++t) {
            const int64_t offr = (t0 + t) * kr_ss + d, offp = (t0 + t) * kp_ss + d;
            r0 = r0 + E::ld(kr, offr);
            r1 = r1 + E::ld(kr, offr + 1);
            p0 = p0 + E::ld(kp, offp);
            p1 = p1 + E::ld(kp, offp + 1);
        }
        graw[m * Dh + d] = r0;
        graw[m * Dh + d + 1] = r1;
        grope[m * Dh + d] = p0;
        grope[m * Dh + d + 1] = p1;
    }
    __syncthreads();
    for (int task = threadIdx.x; task < (M + 1) * Dh; task += kSumThreads) {
        const int m = task / Dh, d = task % Dh;
        if (m < M) {
            traw[task] = round_dt(round_dt(graw[m * Dh + d], DT) * gscale, DT);
            ttok[task] = round_dt(round_dt(grope[m * Dh + d], DT) * gscale, DT);
        } else {
            float sr = 0.0f, sp = 0.0f;
            for (int g = 0; g < M; ++g) {
                sr = sr + graw[g * Dh + d];
                sp = sp + grope[g * Dh + d];
            }
            traw[task] = round_dt(sr, DT);
            ttok[task] = round_dt(sp, DT);
        }
    }
    __syncthreads();
    for (int task = threadIdx.x; task < (M + 1) * Dh; task += kSumThreads) {
        const int m = task / Dh, d = task % Dh;
        int64_t a;
        if (m < M) {
            int glen = len - m * gs;
            glen = glen < 0 ? 0 : (glen > gs ? gs : glen);
            a = (int64_t)n * C + m * gs + ((glen > 1 ? glen : 1) - 1) / 2;
        } else {
            a = (int64_t)n * C + ((len > 1 ? len : 1) - 1) / 2;
        }
        if (a > S - 1) a = S - 1;
        const float* row = traw + m * Dh;
        const float x = row[d];
        const float rot = d < half ? -row[d + half] : row[d - half];
        const bool tokenwise = (d % half) < cutoff;
        const float tok = ttok[task];
        {
            const float c = cos_a[(pos0 + a) * Dh + d], s = sin_a[(pos0 + a) * Dh + d];
            const float p = x * c;
            const float q = rot * s;
            const float v = tokenwise ? tok : round_dt(p + q, DT);
            if (m < M)
                E::st(gk_a, b * gk_sb + h * gk_sh + ((int64_t)n * M + m) * Dh + d, v);
            else
                E::st(ck_a, b * ck_sb + h * ck_sh + (int64_t)n * Dh + d, v);
        }
        if (cos_b) {
            const float c = cos_b[(pos0 + a) * Dh + d], s = sin_b[(pos0 + a) * Dh + d];
            const float p = x * c;
            const float q = rot * s;
            const float v = tokenwise ? tok : round_dt(p + q, DT);
            if (m < M)
                E::st(gk_b, b * gk_sb + h * gk_sh + ((int64_t)n * M + m) * Dh + d, v);
            else
                E::st(ck_b, b * ck_sb + h * ck_sh + (int64_t)n * Dh + d, v);
        }
    }
}

}  // namespace
}  // namespace hga

extern "C" int hga_summarize(const hga_config* cfg, int32_t S, int64_t pos0, const void* k_raw,
                             int64_t kr_sb, int64_t kr_sh, int64_t kr_ss, const void* k_rope,
                             int64_t kp_sb, int64_t kp_sh, int64_t kp_ss, const float* cos_tab,
                             const float* sin_tab, void* chunk_k, int64_t ck_sb, int64_t ck_sh,
                             void* group_k, int64_t gk_sb, int64_t gk_sh, const float* cos_b,
                             const float* sin_b, void* chunk_k_b, void* group_k_b,
                             void* stream) {
    using namespace hga;
    int rc = check_config(cfg);
    if (rc) return rc;
    HGA_REQUIRE(k_raw && k_rope && cos_tab && sin_tab && chunk_k && group_k, HGA_ERR_ARG,
                "hga_summarize: NULL pointer");
    const bool two = cos_b || sin_b || chunk_k_b || group_k_b;
    HGA_REQUIRE(!two || (cos_b && sin_b && chunk_k_b && group_k_b), HGA_ERR_ARG,
                "hga_summarize: second table/output must be all set or all NULL");
    HGA_REQUIRE(S >= 0 && pos0 >= 0 && pos0 % cfg->chunk_size == 0, HGA_ERR_ARG,
                "hga_summarize: S >= 0 and pos0 a multiple of chunk_size required");
    if (S == 0) return HGA_OK;
    const int C = cfg->chunk_size, gs = cfg->group_size, M = C / gs, Dh = cfg->head_dim;
    const int N = chunks_of(S, C);
    const size_t lds = sizeof(float) * (size_t)(2 * M * Dh + 2 * (M + 1) * Dh);
    HGA_REQUIRE(lds <= 65536, HGA_ERR_UNSUPPORTED, "hga_summarize: group layout too large");
    dim3 grid(N, cfg->kv_heads, cfg->batch);
    hipStream_t st = (hipStream_t)stream;
    if (cfg->dtype == HGA_DTYPE_BF16) {
        typedef uint16_t T;
        summarize_kernel<HGA_DTYPE_BF16><<<grid, kSumThreads, lds, st>>>(
            (const T*)k_raw, kr_sb, kr_sh, kr_ss, (const T*)k_rope, kp_sb, kp_sh, kp_ss, cos_tab,
            sin_tab, (T*)chunk_k, (T*)group_k, cos_b, sin_b, (T*)chunk_k_b, (T*)group_k_b, ck_sb,
            ck_sh, gk_sb, gk_sh, pos0, S, Dh, C, gs, cfg->cutoff_pair, cfg->group_scale);
    } else {
        typedef float T;
        summarize_kernel<HGA_DTYPE_F32><<<grid, kSumThreads, lds, st>>>(
            (const T*)k_raw, kr_sb, kr_sh, kr_ss, (const T*)k_rope, kp_sb, kp_sh, kp_ss, cos_tab,
            sin_tab, (T*)chunk_k, (T*)group_k, cos_b, sin_b, (T*)chunk_k_b, (T*)group_k_b, ck_sb,
            ck_sh, gk_sb, gk_sh, pos0, S, Dh, C, gs, cfg->cutoff_pair, cfg->group_scale);
    }
    return launch_status("hga_summarize");
}
