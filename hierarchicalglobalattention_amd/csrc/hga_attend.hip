// Exact attention over the routed working set of a prefill block (vectorized.py:404-490 and
// RoutedKV.attend chunked, chunk_router.py:149-158, fused; no K/V or mask is materialised).
//
// Key sequence of query chunk n (row t sees key k iff t >= thr(k)):
//   [first window 0..f_hi*C)            thr 0
//   [last window l_lo*C..n*C)           thr 0
//   [opened groups, gs tokens each]     thr = the group's first visible row
//   [own chunk n*C + j, j < rows]       thr = j   (causal)
// Masked scores become -inf (the reference's -1e4 fill underflows to exactly 0 in its fp32
// softmax), the softmax is accumulated online in fp32.
//
// bf16 path (head_dim 64/128): one 128-thread workgroup per (batch, head, chunk); wave w owns
// query rows 32w..32w+31.  64-key tiles are staged in LDS (K row-major, V transposed); scores
// are computed as S^T = K Q^T with v_mfma_f32_32x32x16_bf16 so each lane holds 32 scores of a
// single query row, and the output as O^T = V^T P^T so the online-softmax rescale is a per-lane
// scalar.  Workgroups of the H/KVH heads that share a KV head and chunk are placed on the same
// XCD (consecutive in that XCD's dispatch order) so their common window/current tiles are L2
// hits.
// fp32 path (and head_dim 16/32): one wave per query row at a time, VALU dot products, online
// softmax across the wave.
#include "hga_common.h"

namespace hga {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int kNever = 1 << 28;

struct AttnArgs {
    const void* q;
    int64_t q_sb, q_sh, q_ss;
    const void* k;
    int64_t k_sb, k_sh, k_ss;
    const void* v;
    int64_t v_sb, v_sh, v_ss;
    void* out;
    int64_t o_sb, o_sh, o_ss;
    const int32_t* open_grp;
    const int32_t* open_thr;
    int B, H, KVH, S, N, C, gs, M, kf, kl, Kg;
    float scale;
};

struct KeySeq {
    int a1, a2, a3, a4, l_lo, n, C, gs, M;
    const int* og;
    const int* ot;
    __device__ __forceinline__ void get(int k, int& pos, int& thr) const {
        if (k < a1) {
            pos = k;
            thr = 0;
        } else if (k < a2) {
            pos = l_lo * C + (k - a1);
            thr = 0;
        } else if (k < a3) {
            const int g = (k - a2) / gs, e = (k - a2) % gs;
            const int grp = og[g];
            pos = (grp / M) * C + (grp % M) * gs + e;
            thr = ot[g];
        } else if (k < a4) {
            pos = n * C + (k - a3);
            thr = k - a3;
        } else {
            pos = 0;
            thr = kNever;
        }
    }
};

// Maps a dispatch index to (b, h, n) such that the rep heads of one (b, kv head, n) are
// consecutive blocks of one XCD (blocks are dispatched round-robin over the 8 XCDs).
__device__ __forceinline__ void block_coords(int nblk, int B, int H, int N, int* b, int* h,
                                             int* n) {
    const int bid = blockIdx.x, xcd = bid % 8, slot = bid / 8;
    const int q = nblk / 8, r = nblk % 8;
    const int logical = xcd < r ? xcd * (q + 1) + slot : r * (q + 1) + (xcd - r) * q + slot;
    // logical = ((b * N + n) * H + h): heads innermost (heads of a KV head are contiguous)
    *h = logical % H;
    const int bn = logical / H;
    *n = bn % N;
    *b = bn / N;
}

__device__ __forceinline__ void setup_keys(const AttnArgs& A, int b, int h, int n, int rows,
                                           int* sOG, int* sOT, KeySeq& ks, int nthreads) {
    int f_hi, l_lo;
    windows(n, A.kf, A.kl, &f_hi, &l_lo);
    const int Kgw = A.Kg > 0 ? A.Kg : 1;
    const int32_t* og = A.open_grp + (((int64_t)b * A.H + h) * A.N + n) * Kgw;
    const int32_t* ot = A.open_thr + (((int64_t)b * A.H + h) * A.N + n) * Kgw;
    // opened groups with a valid first row, compacted (lists are -1 padded at the end)
    for (int i = threadIdx.x; i < A.Kg; i += nthreads) {
        sOG[i] = og[i];
        sOT[i] = ot[i];
    }
    __syncthreads();
    int nopen = 0;
    for (int i = 0; i < A.Kg; ++i)
        if (sOG[i] >= 0 && sOT[i] >= 0) nopen = i + 1;
    ks.a1 = f_hi * A.C;
    ks.a2 = ks.a1 + (n - l_lo) * A.C;
    ks.a3 = ks.a2 + nopen * A.gs;
    ks.a4 = ks.a3 + rows;
    ks.l_lo = l_lo;
    ks.n = n;
    ks.C = A.C;
    ks.gs = A.gs;
    ks.M = A.M;
    ks.og = sOG;
    ks.ot = sOT;
}

// ------------------------------------------------------------------------------------------
// bf16 MFMA kernel
// ------------------------------------------------------------------------------------------
constexpr int kAT = 128;   // threads
constexpr int kKT = 64;    // keys per tile

template <int DH>
__global__ __launch_bounds__(kAT) void attend_mfma_kernel(AttnArgs A) {
    constexpr int KS = DH / 16, DB = DH / 32;
    constexpr int KSTR = DH + 8;     // sK row stride (elements)
    constexpr int VSTR = kKT + 4;    // sVt row stride (elements)
    __shared__ __align__(16) uint16_t sK[kKT * KSTR];
    __shared__ __align__(16) uint16_t sVt[DH * VSTR];
    __shared__ int sThrK[kKT];
    __shared__ int sPos[kKT];
    extern __shared__ int sOpen[];   // [2 * Kg]
    int* sOG = sOpen;
    int* sOT = sOpen + (A.Kg > 0 ? A.Kg : 1);

    int b, h, n;
    block_coords(A.B * A.H * A.N, A.B, A.H, A.N, &b, &h, &n);
    const int kvh = h / (A.H / A.KVH);
    int rows = A.S - n * A.C;
    if (rows > A.C) rows = A.C;
    KeySeq ks;
    setup_keys(A, b, h, n, rows, sOG, sOT, ks, kAT);

    const int w = threadIdx.x / kWave, l = lane_id();
    const int row = w * 32 + (l % 32);       // chunk-local query row of this lane
    const bool wave_active = w * 32 < rows;
    const uint16_t* qp = reinterpret_cast<const uint16_t*>(A.q) + b * A.q_sb + h * A.q_sh;
    const uint16_t* kp = reinterpret_cast<const uint16_t*>(A.k) + b * A.k_sb + kvh * A.k_sh;
    const uint16_t* vp = reinterpret_cast<const uint16_t*>(A.v) + b * A.v_sb + kvh * A.v_sh;

    bf16x8 qb[KS];
#pragma unroll
    for (int s = 0; s < KS; ++s) {
        uint4 u = make_uint4(0u, 0u, 0u, 0u);
        if (row < rows)
            u = *reinterpret_cast<const uint4*>(qp + ((int64_t)A.C * n + row) * A.q_ss + s * 16 +
                                                8 * (l / 32));
        qb[s] = __builtin_bit_cast(bf16x8, u);
    }
    floatx16 acc[DB];
#pragma unroll
    for (int d = 0; d < DB; ++d) acc[d] = floatx16{};
    float m_run = -INFINITY, l_run = 0.0f;
    const float c2 = A.scale * 1.4426950408889634f;

    const int ntiles = (ks.a4 + kKT - 1) / kKT;
    for (int tile = 0; tile < ntiles; ++tile) {
        const int kbase = tile * kKT;
        if (threadIdx.x < kKT) {
            int pos, thr;
            ks.get(kbase + threadIdx.x, pos, thr);
            sPos[threadIdx.x] = pos;
            sThrK[threadIdx.x] = thr;
        }
        __syncthreads();
        // K tile (row-major) and V tile (transposed) into LDS
        constexpr int CPR = DH / 8;   // 16-byte pieces per key row
        for (int c = threadIdx.x; c < kKT * CPR; c += kAT) {
            const int kk = c / CPR, dp = c % CPR;
            const uint4 u = *reinterpret_cast<const uint4*>(kp + (int64_t)sPos[kk] * A.k_ss + dp * 8);
            *reinterpret_cast<uint4*>(&sK[kk * KSTR + dp * 8]) = u;
        }
        for (int c = threadIdx.x; c < (kKT / 2) * CPR; c += kAT) {
            const int kp2 = c / CPR, dg = c % CPR;
            const uint4 u0 = *reinterpret_cast<const uint4*>(vp + (int64_t)sPos[2 * kp2] * A.v_ss + dg * 8);
            const uint4 u1 = *reinterpret_cast<const uint4*>(vp + (int64_t)sPos[2 * kp2 + 1] * A.v_ss + dg * 8);
            const uint32_t a0[4] = {u0.x, u0.y, u0.z, u0.w}, a1[4] = {u1.x, u1.y, u1.z, u1.w};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const uint32_t lo = (a0[e] & 0xffffu) | (a1[e] << 16);
                const uint32_t hi = (a0[e] >> 16) | (a1[e] & 0xffff0000u);
                *reinterpret_cast<uint32_t*>(&sVt[(dg * 8 + 2 * e) * VSTR + 2 * kp2]) = lo;
                *reinterpret_cast<uint32_t*>(&sVt[(dg * 8 + 2 * e + 1) * VSTR + 2 * kp2]) = hi;
            }
        }
        __syncthreads();
        if (wave_active) {
            floatx16 s0 = {}, s1 = {};
#pragma unroll
            for (int s = 0; s < KS; ++s) {
                const int col = s * 16 + 8 * (l / 32);
                const bf16x8 k0 = __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4*>(&sK[(l % 32) * KSTR + col]));
                const bf16x8 k1 = __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4*>(&sK[(32 + l % 32) * KSTR + col]));
                s0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(k0, qb[s], s0, 0, 0, 0);
                s1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(k1, qb[s], s1, 0, 0, 0);
            }
            // mask + running max
            float mx = -INFINITY;
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int kk = 8 * (i / 4) + 4 * (l / 32) + (i % 4);
                s0[i] = row >= sThrK[kk] ? s0[i] * c2 : -INFINITY;
                s1[i] = row >= sThrK[32 + kk] ? s1[i] * c2 : -INFINITY;
                mx = fmaxf(mx, fmaxf(s0[i], s1[i]));
            }
            mx = fmaxf(mx, __shfl_xor(mx, 32, kWave));
            const float m_new = fmaxf(m_run, mx);
            const float m_use = m_new == -INFINITY ? 0.0f : m_new;
            const float alpha = exp2f(m_run - m_use);
            float rs = 0.0f;
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                s0[i] = exp2f(s0[i] - m_use);
                s1[i] = exp2f(s1[i] - m_use);
                rs += s0[i] + s1[i];
            }
            rs += __shfl_xor(rs, 32, kWave);
            l_run = l_run * alpha + rs;
            m_run = m_new;
#pragma unroll
            for (int d = 0; d < DB; ++d)
#pragma unroll
                for (int i = 0; i < 16; ++i) acc[d][i] *= alpha;
            // P^T operands (bf16), 4 k-steps of 16 keys
            bf16x8 pb[4];
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                pb[0][j] = (__bf16)s0[j];
                pb[1][j] = (__bf16)s0[8 + j];
                pb[2][j] = (__bf16)s1[j];
                pb[3][j] = (__bf16)s1[8 + j];
            }
#pragma unroll
            for (int st = 0; st < 4; ++st) {
                const int kb = 16 * st + 4 * (l / 32);
#pragma unroll
                for (int d = 0; d < DB; ++d) {
                    const uint16_t* vr = &sVt[(d * 32 + l % 32) * VSTR];
                    const uint2 lo = *reinterpret_cast<const uint2*>(vr + kb);
                    const uint2 hi = *reinterpret_cast<const uint2*>(vr + kb + 8);
                    const uint4 u = make_uint4(lo.x, lo.y, hi.x, hi.y);
                    acc[d] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
                        __builtin_bit_cast(bf16x8, u), pb[st], acc[d], 0, 0, 0);
                }
            }
        }
        __syncthreads();
    }
    if (wave_active && row < rows) {
        const float inv = l_run > 0.0f ? 1.0f / l_run : 0.0f;
        uint16_t* op = reinterpret_cast<uint16_t*>(A.out) + b * A.o_sb + h * A.o_sh +
                       ((int64_t)A.C * n + row) * A.o_ss;
#pragma unroll
        for (int d = 0; d < DB; ++d)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const int dim = d * 32 + 8 * g + 4 * (l / 32);
                uint2 u;
                u.x = (uint32_t)f_to_bf16(acc[d][4 * g] * inv) |
                      ((uint32_t)f_to_bf16(acc[d][4 * g + 1] * inv) << 16);
                u.y = (uint32_t)f_to_bf16(acc[d][4 * g + 2] * inv) |
                      ((uint32_t)f_to_bf16(acc[d][4 * g + 3] * inv) << 16);
                *reinterpret_cast<uint2*>(op + dim) = u;
            }
    }
}

// ------------------------------------------------------------------------------------------
// VALU kernel (fp32 activations, or head_dim 16/32)
// ------------------------------------------------------------------------------------------
constexpr int kVT = 256;

template <int DT, int DH>
__global__ __launch_bounds__(kVT) void attend_valu_kernel(AttnArgs A) {
    typedef Elem<DT> E;
    typedef typename E::T T;
    constexpr int DPL = DH > 64 ? DH / 64 : 1;  // dims per lane
    __shared__ float sQ[64 * DH];
    extern __shared__ int sOpen[];
    int* sOG = sOpen;
    int* sOT = sOpen + (A.Kg > 0 ? A.Kg : 1);
    int b, h, n;
    block_coords(A.B * A.H * A.N, A.B, A.H, A.N, &b, &h, &n);
    const int kvh = h / (A.H / A.KVH);
    int rows = A.S - n * A.C;
    if (rows > A.C) rows = A.C;
    const T* qp = reinterpret_cast<const T*>(A.q) + b * A.q_sb + h * A.q_sh;
    for (int idx = threadIdx.x; idx < rows * DH; idx += kVT) {
        const int t = idx / DH, d = idx % DH;
        sQ[idx] = E::ld(qp, ((int64_t)A.C * n + t) * A.q_ss + d);
    }
    KeySeq ks;
    setup_keys(A, b, h, n, rows, sOG, sOT, ks, kVT);   // contains a barrier
    const T* kp = reinterpret_cast<const T*>(A.k) + b * A.k_sb + kvh * A.k_sh;
    const T* vp = reinterpret_cast<const T*>(A.v) + b * A.v_sb + kvh * A.v_sh;
    const int w = threadIdx.x / kWave, l = lane_id();
    for (int t = w; t < rows; t += kVT / kWave) {
        const float* qr = sQ + t * DH;
        float m_run = -INFINITY, l_run = 0.0f, acc[DPL];
#pragma unroll
        for (int e = 0; e < DPL; ++e) acc[e] = 0.0f;
        for (int base = 0; base < ks.a4; base += kWave) {
            int pos, thr;
            ks.get(base + l, pos, thr);
            float s = -INFINITY;
            if (t >= thr) {
                const T* kr = kp + (int64_t)pos * A.k_ss;
                float d0 = 0.0f;
                for (int d = 0; d < DH; ++d) d0 = fmaf(qr[d], E::ld(kr, d), d0);
                s = d0 * A.scale;
            }
            const float mx = wave_max(s);
            const float m_new = fmaxf(m_run, mx);
            const float m_use = m_new == -INFINITY ? 0.0f : m_new;
            const float alpha = expf(m_run - m_use);
            const float p = expf(s - m_use);
            l_run = l_run * alpha + wave_sum(p);
            m_run = m_new;
#pragma unroll
            for (int e = 0; e < DPL; ++e) acc[e] *= alpha;
            const int lim = ks.a4 - base < kWave ? ks.a4 - base : kWave;
            for (int kk = 0; kk < lim; ++kk) {
                const float pk = __shfl(p, kk, kWave);
                if (pk == 0.0f) continue;
                const int pos2 = __shfl(pos, kk, kWave);
                const T* vr = vp + (int64_t)pos2 * A.v_ss;
#pragma unroll
                for (int e = 0; e < DPL; ++e) {
                    const int d = l + 64 * e;
                    if (d < DH) acc[e] = fmaf(pk, E::ld(vr, d), acc[e]);
                }
            }
        }
        T* op = reinterpret_cast<T*>(A.out) + b * A.o_sb + h * A.o_sh;
        const float inv = l_run > 0.0f ? 1.0f / l_run : 0.0f;
#pragma unroll
        for (int e = 0; e < DPL; ++e) {
            const int d = l + 64 * e;
            if (d < DH) E::st(op, ((int64_t)A.C * n + t) * A.o_ss + d, acc[e] * inv);
        }
    }
}

}  // namespace
}  // namespace hga

extern "C" int hga_attend_prefill(const hga_config* cfg, int32_t S, const void* q, int64_t q_sb,
                                  int64_t q_sh, int64_t q_ss, const void* k, int64_t k_sb,
                                  int64_t k_sh, int64_t k_ss, const void* v, int64_t v_sb,
                                  int64_t v_sh, int64_t v_ss, const int32_t* open_grp,
                                  const int32_t* open_thr, int32_t Kg, void* out, int64_t o_sb,
                                  int64_t o_sh, int64_t o_ss, void* stream) {
    using namespace hga;
    int rc = check_config(cfg);
    if (rc) return rc;
    HGA_REQUIRE(q && k && v && out && open_grp && open_thr, HGA_ERR_ARG,
                "hga_attend_prefill: NULL pointer");
    HGA_REQUIRE(S >= 0 && Kg >= 0, HGA_ERR_ARG, "hga_attend_prefill: negative S/Kg");
    if (S == 0) return HGA_OK;
    AttnArgs a{};
    a.q = q; a.q_sb = q_sb; a.q_sh = q_sh; a.q_ss = q_ss;
    a.k = k; a.k_sb = k_sb; a.k_sh = k_sh; a.k_ss = k_ss;
    a.v = v; a.v_sb = v_sb; a.v_sh = v_sh; a.v_ss = v_ss;
    a.out = out; a.o_sb = o_sb; a.o_sh = o_sh; a.o_ss = o_ss;
    a.open_grp = open_grp; a.open_thr = open_thr;
    a.B = cfg->batch; a.H = cfg->heads; a.KVH = cfg->kv_heads; a.S = S;
    a.C = cfg->chunk_size; a.gs = cfg->group_size; a.M = a.C / a.gs;
    a.N = (S + a.C - 1) / a.C; a.kf = cfg->keep_first; a.kl = cfg->keep_last;
    a.Kg = Kg; a.scale = cfg->scale;
    int nN, nKc, nKg;
    hga_prefill_widths(cfg, S, &nN, &nKc, &nKg);
    HGA_REQUIRE(Kg == nKg, HGA_ERR_ARG, "hga_attend_prefill: Kg %d != routing width %d", Kg, nKg);
    const int D = cfg->head_dim;
    const unsigned grid = (unsigned)(a.B * a.H * a.N);
    const size_t lds = sizeof(int) * 2 * (size_t)(Kg > 0 ? Kg : 1);
    hipStream_t st = (hipStream_t)stream;
    if (cfg->dtype == HGA_DTYPE_BF16 && (D == 64 || D == 128)) {
        const uintptr_t al = (uintptr_t)q | (uintptr_t)k | (uintptr_t)v | (uintptr_t)out;
        HGA_REQUIRE(al % 16 == 0 && ((q_sb | q_sh | q_ss | k_sb | k_sh | k_ss | v_sb | v_sh |
                                      v_ss | o_sb | o_sh | o_ss) % 8) == 0,
                    HGA_ERR_ARG, "hga_attend_prefill: 16-byte aligned rows required");
        if (D == 128) attend_mfma_kernel<128><<<grid, kAT, lds, st>>>(a);
        else attend_mfma_kernel<64><<<grid, kAT, lds, st>>>(a);
        return launch_status("hga_attend_prefill");
    }
#define HGA_VALU_CASE(DTV, DHV) \
    if (cfg->dtype == DTV && D == DHV) { attend_valu_kernel<DTV, DHV><<<grid, kVT, lds, st>>>(a); return launch_status("hga_attend_prefill"); }
    HGA_VALU_CASE(HGA_DTYPE_F32, 128)
    HGA_VALU_CASE(HGA_DTYPE_F32, 64)
    HGA_VALU_CASE(HGA_DTYPE_F32, 32)
    HGA_VALU_CASE(HGA_DTYPE_F32, 16)
    HGA_VALU_CASE(HGA_DTYPE_BF16, 32)
    HGA_VALU_CASE(HGA_DTYPE_BF16, 16)
#undef HGA_VALU_CASE
    set_error("hga_attend_prefill: unsupported dtype/head_dim");
    return HGA_ERR_UNSUPPORTED;
}
