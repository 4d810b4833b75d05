// Backward of the exact attention over the routed working set of a prefill block.  The reference
// trains through its routed attention with torch autograd (HierarchicalGlobalAttentionRouted
// forward, :137-177, over the working set gathered by vectorized.py:404-490); the routing
// decisions carry no gradient, so the gradient is that of softmax attention over each row's key
// sequence (hga_keys.h).  For row i and key j of its sequence:
//   p_ij = softmax_j(scale q_i.k_j),  dp_ij = dO_i.v_j,  D_i = dO_i.O_i,  ds_ij = p_ij (dp_ij - D_i)
//   dq_i = scale sum_j ds_ij k_j,  dk_j += scale ds_ij q_i,  dv_j += p_ij dO_i.
//
// One workgroup per (b, h, query chunk): pass 1 recomputes the rows' softmax statistics
// (log-sum-exp) over the key sequence, pass 2 recomputes P, forms dS, accumulates dq in
// registers and adds each key tile's dk/dv (summed over the chunk's rows) into fp32 accumulators
// with hardware float atomics: a key is reached from many query chunks and heads (the windows
// from every later chunk, opened groups from any chunk that routes to them), so the sums are
// scattered.  A final kernel writes the accumulators in the caller's dtype and strides.
//
// bf16 head_dim 64/128: MFMA kernel (v_mfma_f32_32x32x16_bf16; S^T = K Q^T and dP^T = V dO^T
// leave one query row per lane, dQ^T = K^T dS^T reads dS^T from registers, dK = dS^T Q and
// dV = P^T dO read P and dS through LDS).  Other shapes: VALU kernel.
#include <algorithm>

#include "hga_common.h"
#include "hga_keys.h"

namespace hga {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

struct BwdArgs {
    AttnArgs a;        // q, k, v, out = the forward output O, routing lists, shape, scale
    const void* dout;
    int64_t g_sb, g_sh, g_ss;
    void* dq;
    int64_t dq_sb, dq_sh, dq_ss;
    float* dk;         // fp32 accumulators [B, KVH, S, Dh], zeroed
    float* dv;
};

constexpr int kBR = 64;   // query rows per workgroup (chunk_size <= 64)

__global__ void zero_kernel(float4* p, int64_t n4) {
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n4;
         i += (int64_t)gridDim.x * blockDim.x)
        p[i] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
}

// acc [B, KVH, S, DH] fp32 -> out (caller dtype and strides)
template <int DT>
__global__ void acc_out_kernel(const float* __restrict__ acc, void* out, int64_t sb, int64_t sh,
                               int64_t ss, int KVH, int S, int DH, int64_t total) {
    typedef Elem<DT> E;
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * blockDim.x) {
        const int d = (int)(i % DH);
        const int64_t t = i / DH;
        const int s = (int)(t % S);
        const int64_t bk = t / S;
        const int kvh = (int)(bk % KVH), b = (int)(bk / KVH);
        E::st(reinterpret_cast<typename E::T*>(out), b * sb + kvh * sh + s * ss + d, acc[i]);
    }
}

// ------------------------------------------------------------------------------------------
// VALU kernel: 256 threads; scores as 4 threads x 8 keys per row, fp32 operands in LDS
// ------------------------------------------------------------------------------------------
constexpr int kBT = 256;
constexpr int kBK = 32;   // keys per tile

template <int DH>
__host__ __device__ constexpr size_t valu_lds_floats() {
    return 2 * (size_t)kBR * (DH + 1) + 2 * (size_t)kBK * (DH + 1) + 2 * (size_t)kBR * (kBK + 1) +
           kBR;
}

template <int DT, int DH>
__global__ __launch_bounds__(kBT) void attend_bwd_valu_kernel(BwdArgs P) {
    typedef Elem<DT> E;
    typedef typename E::T T;
    const AttnArgs& A = P.a;
    constexpr int QS = DH + 1, PS = kBK + 1;
    extern __shared__ __align__(16) float smem[];
    float* sQ = smem;                    // [kBR][QS]
    float* sG = sQ + kBR * QS;           // dO rows
    float* sK = sG + kBR * QS;           // [kBK][QS]
    float* sV = sK + kBK * QS;
    float* sP = sV + kBK * QS;           // [kBR][PS]
    float* sDS = sP + kBR * PS;
    float* sD = sDS + kBR * PS;          // [kBR]
    int* sPos = reinterpret_cast<int*>(sD + kBR);
    int* sThr = sPos + kBK;
    int* sOG = sThr + kBK;
    int* sOT = sOG + (A.Kg > 0 ? A.Kg : 1);

    int b, h, n;
    block_coords(A.B * A.H * A.N, A.B, A.H, A.KVH, A.N, &b, &h, &n);
    const int kvh = h / (A.H / A.KVH);
    int rows = A.S - n * A.C;
    if (rows > A.C) rows = A.C;
    KeySeq ks;
    setup_keys(A, b, h, n, rows, sOG, sOT, ks, kBT);

    const int64_t r0 = (int64_t)n * A.C;
    const T* qp = reinterpret_cast<const T*>(A.q) + b * A.q_sb + h * A.q_sh + r0 * A.q_ss;
    const T* op = reinterpret_cast<const T*>(A.out) + b * A.o_sb + h * A.o_sh + r0 * A.o_ss;
    const T* gp = reinterpret_cast<const T*>(P.dout) + b * P.g_sb + h * P.g_sh + r0 * P.g_ss;
    const T* kp = reinterpret_cast<const T*>(A.k) + b * A.k_sb + kvh * A.k_sh;
    const T* vp = reinterpret_cast<const T*>(A.v) + b * A.v_sb + kvh * A.v_sh;
    for (int i = threadIdx.x; i < kBR * DH; i += kBT) {
        const int r = i / DH, d = i % DH;
        const bool in = r < rows;
        sQ[r * QS + d] = in ? E::ld(qp, r * A.q_ss + d) : 0.0f;
        sG[r * QS + d] = in ? E::ld(gp, r * P.g_ss + d) : 0.0f;
    }
    const int r = threadIdx.x >> 2, kq = threadIdx.x & 3;   // score rows / key lanes
    {
        float acc = 0.0f;
        if (r < rows)
            for (int d = kq; d < DH; d += 4)
                acc = fmaf(E::ld(gp, r * P.g_ss + d), E::ld(op, r * A.o_ss + d), acc);
        acc += __shfl_xor(acc, 1, kWave);
        acc += __shfl_xor(acc, 2, kWave);
        if (kq == 0) sD[r] = acc;
    }
    __syncthreads();

    const float c2 = A.scale * 1.4426950408889634f;
    const int ntiles = (ks.a4 + kBK - 1) / kBK;
    auto load_tile = [&](int tile, bool with_v) {
        if (threadIdx.x < kBK) {
            int pos, thr;
            ks.get(tile * kBK + threadIdx.x, pos, thr);
            sPos[threadIdx.x] = pos;
            sThr[threadIdx.x] = thr;
        }
        __syncthreads();
        for (int i = threadIdx.x; i < kBK * DH; i += kBT) {
            const int kk = i / DH, d = i % DH;
            const int64_t pos = sPos[kk];
            sK[kk * QS + d] = E::ld(kp, pos * A.k_ss + d);
            if (with_v) sV[kk * QS + d] = E::ld(vp, pos * A.v_ss + d);
        }
        __syncthreads();
    };
    auto dots = [&](const float* sa, const float* sb, float (&s)[8]) {
#pragma unroll
        for (int i = 0; i < 8; ++i) s[i] = 0.0f;
        for (int d = 0; d < DH; ++d) {
            const float a = sa[r * QS + d];
#pragma unroll
            for (int i = 0; i < 8; ++i) s[i] = fmaf(a, sb[(kq + 4 * i) * QS + d], s[i]);
        }
    };

    // pass 1: log2-domain softmax statistics of each row (the forward's, when it kept them)
    float m = -INFINITY, lsum = 0.0f;
    for (int tile = 0; tile < (A.lse ? 0 : ntiles); ++tile) {
        load_tile(tile, false);
        float s[8];
        dots(sQ, sK, s);
        float mx = -INFINITY;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            s[i] = (r < rows && r >= sThr[kq + 4 * i]) ? s[i] * c2 : -INFINITY;
            mx = fmaxf(mx, s[i]);
        }
        mx = fmaxf(mx, __shfl_xor(mx, 1, kWave));
        mx = fmaxf(mx, __shfl_xor(mx, 2, kWave));
        const float mn = fmaxf(m, mx);
        if (mn != -INFINITY) {
            float add = 0.0f;
#pragma unroll
            for (int i = 0; i < 8; ++i) add += exp2f(s[i] - mn);
            add += __shfl_xor(add, 1, kWave);
            add += __shfl_xor(add, 2, kWave);
            lsum = lsum * exp2f(m - mn) + add;
            m = mn;
        }
        __syncthreads();
    }
    const float lse = A.lse ? (r < rows ? A.lse[((int64_t)b * A.H + h) * A.S + r0 + r] : INFINITY)
                            : (lsum > 0.0f ? m + log2f(lsum) : INFINITY);
    const float Dr = sD[r];

    // pass 2
    constexpr int QJ = DH / 4, KJ = DH / 8;
    float dq[QJ];
#pragma unroll
    for (int j = 0; j < QJ; ++j) dq[j] = 0.0f;
    const int kk2 = threadIdx.x >> 3, dpart = threadIdx.x & 7;   // dk/dv: key, dim lane
    float* dkb = P.dk + ((int64_t)b * A.KVH + kvh) * A.S * DH;
    float* dvb = P.dv + ((int64_t)b * A.KVH + kvh) * A.S * DH;
    for (int tile = 0; tile < ntiles; ++tile) {
        load_tile(tile, true);
        float s[8], dp[8];
        dots(sQ, sK, s);
        dots(sG, sV, dp);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int kk = kq + 4 * i;
            const bool vis = r < rows && r >= sThr[kk];
            const float p = vis ? exp2f(s[i] * c2 - lse) : 0.0f;
            sP[r * PS + kk] = p;
            sDS[r * PS + kk] = p * (dp[i] - Dr);
        }
        __syncthreads();
        for (int kk = 0; kk < kBK; ++kk) {
            const float ds = sDS[r * PS + kk];
#pragma unroll
            for (int j = 0; j < QJ; ++j) dq[j] = fmaf(ds, sK[kk * QS + kq + 4 * j], dq[j]);
        }
        if (sThr[kk2] < kNever) {
            float gk[KJ], gv[KJ];
#pragma unroll
            for (int j = 0; j < KJ; ++j) gk[j] = gv[j] = 0.0f;
            for (int rr = 0; rr < kBR; ++rr) {
                const float ds = sDS[rr * PS + kk2], p = sP[rr * PS + kk2];
#pragma unroll
                for (int j = 0; j < KJ; ++j) {
                    gk[j] = fmaf(ds, sQ[rr * QS + dpart + 8 * j], gk[j]);
                    gv[j] = fmaf(p, sG[rr * QS + dpart + 8 * j], gv[j]);
                }
            }
            const int64_t o = (int64_t)sPos[kk2] * DH + dpart;
#pragma unroll
            for (int j = 0; j < KJ; ++j) {
                unsafeAtomicAdd(dkb + o + 8 * j, gk[j] * A.scale);
                unsafeAtomicAdd(dvb + o + 8 * j, gv[j]);
            }
        }
        __syncthreads();
    }
    if (r < rows) {
        T* dqp = reinterpret_cast<T*>(P.dq) + b * P.dq_sb + h * P.dq_sh + (r0 + r) * P.dq_ss;
#pragma unroll
        for (int j = 0; j < QJ; ++j) E::st(dqp, kq + 4 * j, dq[j] * A.scale);
    }
}

// ------------------------------------------------------------------------------------------
// bf16 MFMA kernel: 128 threads, wave w owns query rows 32w..32w+31, 32-key tiles
// ------------------------------------------------------------------------------------------
constexpr int kMT = 128;
constexpr int kMK = 32;                 // keys per tile

template <int DH>
struct MfmaLds {
    static constexpr int KSTR = DH + 8;      // sK / sV row stride (bf16 elements)
    static constexpr int KTSTR = kMK + 4;    // sKt row stride
    static constexpr int QTSTR = kBR + 8;    // sQt / sGt row stride
    static constexpr int PSTR = kBR + 8;     // sP / sDS row stride
    static constexpr size_t bytes = 2 * (2 * (size_t)DH * QTSTR + 2 * (size_t)kMK * KSTR +
                                         (size_t)DH * KTSTR + 2 * (size_t)kMK * PSTR);
};

__device__ __forceinline__ bf16x8 ld8(const uint16_t* p) {
    return __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4*>(p));
}

// rows [r0, r0 + 2*npairs) of a [rows][DH] bf16 matrix (row stride ss) -> dst[d][row]
template <int DH, int STR>
__device__ __forceinline__ void transpose_rows(const uint16_t* src, int64_t ss, int rows,
                                               uint16_t* dst) {
    constexpr int CPR = DH / 8;
    for (int c = threadIdx.x; c < (kBR / 2) * CPR; c += kMT) {
        const int rp = c / CPR, dg = c % CPR;
        const int ra = 2 * rp, rb = 2 * rp + 1;
        uint4 u0 = make_uint4(0u, 0u, 0u, 0u), u1 = u0;
        if (ra < rows) u0 = *reinterpret_cast<const uint4*>(src + ra * ss + dg * 8);
        if (rb < rows) u1 = *reinterpret_cast<const uint4*>(src + rb * ss + dg * 8);
        auto put = [&](int e, uint32_t x0, uint32_t x1) {
            *reinterpret_cast<uint32_t*>(&dst[(dg * 8 + 2 * e) * STR + ra]) =
                (x0 & 0xffffu) | (x1 << 16);
            *reinterpret_cast<uint32_t*>(&dst[(dg * 8 + 2 * e + 1) * STR + ra]) =
                (x0 >> 16) | (x1 & 0xffff0000u);
        };
        put(0, u0.x, u1.x);
        put(1, u0.y, u1.y);
        put(2, u0.z, u1.z);
        put(3, u0.w, u1.w);
    }
}

template <int DH>
__global__ __launch_bounds__(kMT) void attend_bwd_mfma_kernel(BwdArgs P) {
    typedef MfmaLds<DH> L;
    constexpr int KS = DH / 16, DB = DH / 32, CPR = DH / 8;
    const AttnArgs& A = P.a;
    extern __shared__ __align__(16) uint16_t lds[];
    uint16_t* sQt = lds;                           // [DH][QTSTR] Q^T of the chunk's rows
    uint16_t* sGt = sQt + DH * L::QTSTR;           // dO^T
    uint16_t* sK = sGt + DH * L::QTSTR;            // [kMK][KSTR]
    uint16_t* sV = sK + kMK * L::KSTR;
    uint16_t* sKt = sV + kMK * L::KSTR;            // [DH][KTSTR]
    uint16_t* sP = sKt + DH * L::KTSTR;            // [kMK][PSTR] P^T (bf16)
    uint16_t* sDS = sP + kMK * L::PSTR;            // dS^T
    int* sPos = reinterpret_cast<int*>(sDS + kMK * L::PSTR);
    int* sThr = sPos + kMK;
    int* sOG = sThr + kMK;
    int* sOT = sOG + (A.Kg > 0 ? A.Kg : 1);

    int b, h, n;
    block_coords(A.B * A.H * A.N, A.B, A.H, A.KVH, A.N, &b, &h, &n);
    const int kvh = h / (A.H / A.KVH);
    int rows = A.S - n * A.C;
    if (rows > A.C) rows = A.C;
    KeySeq ks;
    setup_keys(A, b, h, n, rows, sOG, sOT, ks, kMT);

    const int w = threadIdx.x / kWave, l = lane_id(), hl = l / 32;
    const int row = w * 32 + (l % 32);
    const bool rv = row < rows;
    const int64_t r0 = (int64_t)n * A.C;
    const uint16_t* qp = reinterpret_cast<const uint16_t*>(A.q) + b * A.q_sb + h * A.q_sh + r0 * A.q_ss;
    const uint16_t* op = reinterpret_cast<const uint16_t*>(A.out) + b * A.o_sb + h * A.o_sh + r0 * A.o_ss;
    const uint16_t* gp = reinterpret_cast<const uint16_t*>(P.dout) + b * P.g_sb + h * P.g_sh + r0 * P.g_ss;
    const uint16_t* kp = reinterpret_cast<const uint16_t*>(A.k) + b * A.k_sb + kvh * A.k_sh;
    const uint16_t* vp = reinterpret_cast<const uint16_t*>(A.v) + b * A.v_sb + kvh * A.v_sh;

    // this lane's query row as MFMA B operands (8 dims of each 16-dim step), D_row = dO.O
    bf16x8 qb[KS], gb[KS];
    float Dr = 0.0f;
#pragma unroll
    for (int s = 0; s < KS; ++s) {
        const int col = s * 16 + 8 * hl;
        uint4 uq = make_uint4(0u, 0u, 0u, 0u), ug = uq, uo = uq;
        if (rv) {
            uq = *reinterpret_cast<const uint4*>(qp + row * A.q_ss + col);
            ug = *reinterpret_cast<const uint4*>(gp + row * P.g_ss + col);
            uo = *reinterpret_cast<const uint4*>(op + row * A.o_ss + col);
        }
        qb[s] = __builtin_bit_cast(bf16x8, uq);
        gb[s] = __builtin_bit_cast(bf16x8, ug);
        const uint32_t g4[4] = {ug.x, ug.y, ug.z, ug.w}, o4[4] = {uo.x, uo.y, uo.z, uo.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            Dr = fmaf(bf16_to_f((uint16_t)(g4[e] & 0xffffu)), bf16_to_f((uint16_t)(o4[e] & 0xffffu)), Dr);
            Dr = fmaf(bf16_to_f((uint16_t)(g4[e] >> 16)), bf16_to_f((uint16_t)(o4[e] >> 16)), Dr);
        }
    }
    Dr += __shfl_xor(Dr, 32, kWave);
    transpose_rows<DH, L::QTSTR>(qp, A.q_ss, rows, sQt);
    transpose_rows<DH, L::QTSTR>(gp, P.g_ss, rows, sGt);

    const float c2 = A.scale * 1.4426950408889634f;
    const int ntiles = (ks.a4 + kMK - 1) / kMK;
    auto load_tile = [&](int tile, bool bwd) {
        if (threadIdx.x < kMK) {
            int pos, thr;
            ks.get(tile * kMK + threadIdx.x, pos, thr);
            sPos[threadIdx.x] = pos;
            sThr[threadIdx.x] = thr;
        }
        __syncthreads();
        for (int c = threadIdx.x; c < kMK * CPR; c += kMT) {
            const int kk = c / CPR, dp = c % CPR;
            const int64_t pos = sPos[kk];
            *reinterpret_cast<uint4*>(&sK[kk * L::KSTR + dp * 8]) =
                *reinterpret_cast<const uint4*>(kp + pos * A.k_ss + dp * 8);
            if (bwd)
                *reinterpret_cast<uint4*>(&sV[kk * L::KSTR + dp * 8]) =
                    *reinterpret_cast<const uint4*>(vp + pos * A.v_ss + dp * 8);
        }
        if (bwd) {
            for (int c = threadIdx.x; c < (kMK / 2) * CPR; c += kMT) {
                const int kp2 = c / CPR, dg = c % CPR;
                const uint4 u0 = *reinterpret_cast<const uint4*>(kp + (int64_t)sPos[2 * kp2] * A.k_ss + dg * 8);
                const uint4 u1 = *reinterpret_cast<const uint4*>(kp + (int64_t)sPos[2 * kp2 + 1] * A.k_ss + dg * 8);
                const uint32_t a0[4] = {u0.x, u0.y, u0.z, u0.w}, a1[4] = {u1.x, u1.y, u1.z, u1.w};
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    *reinterpret_cast<uint32_t*>(&sKt[(dg * 8 + 2 * e) * L::KTSTR + 2 * kp2]) =
                        (a0[e] & 0xffffu) | (a1[e] << 16);
                    *reinterpret_cast<uint32_t*>(&sKt[(dg * 8 + 2 * e + 1) * L::KTSTR + 2 * kp2]) =
                        (a0[e] >> 16) | (a1[e] & 0xffff0000u);
                }
            }
        }
        __syncthreads();
    };
    // S^T (keys x this wave's rows): lane holds keys 8*(i/4) + 4*hl + i%4 of query row `row`
    auto scores = [&](const uint16_t* sA, const bf16x8 (&bq)[KS]) {
        floatx16 acc = {};
#pragma unroll
        for (int s = 0; s < KS; ++s)
            acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
                ld8(&sA[(l % 32) * L::KSTR + s * 16 + 8 * hl]), bq[s], acc, 0, 0, 0);
        return acc;
    };
    auto key_of = [&](int i) { return 8 * (i / 4) + 4 * hl + (i % 4); };

    // pass 1: log2-domain softmax statistics of each row (the forward's, when it kept them)
    float m_run = -INFINITY, l_run = 0.0f;
    for (int tile = 0; tile < (A.lse ? 0 : ntiles); ++tile) {
        load_tile(tile, false);
        floatx16 sc = scores(sK, qb);
        float mx = -INFINITY;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            sc[i] = (rv && row >= sThr[key_of(i)]) ? sc[i] * c2 : -INFINITY;
            mx = fmaxf(mx, sc[i]);
        }
        mx = fmaxf(mx, __shfl_xor(mx, 32, kWave));
        const float m_new = fmaxf(m_run, mx);
        const float m_use = m_new == -INFINITY ? 0.0f : m_new;
        float rs = 0.0f;
#pragma unroll
        for (int i = 0; i < 16; ++i) rs += exp2f(sc[i] - m_use);
        rs += __shfl_xor(rs, 32, kWave);
        l_run = l_run * exp2f(m_run - m_use) + rs;
        m_run = m_new;
        __syncthreads();
    }
    const float lse = A.lse ? (rv ? A.lse[((int64_t)b * A.H + h) * A.S + r0 + row] : INFINITY)
                            : (l_run > 0.0f ? m_run + log2f(l_run) : INFINITY);

    // pass 2
    floatx16 dq[DB];
#pragma unroll
    for (int d = 0; d < DB; ++d) dq[d] = floatx16{};
    float* dkb = P.dk + ((int64_t)b * A.KVH + kvh) * A.S * DH;
    float* dvb = P.dv + ((int64_t)b * A.KVH + kvh) * A.S * DH;
    for (int tile = 0; tile < ntiles; ++tile) {
        load_tile(tile, true);
        floatx16 sc = scores(sK, qb);
        const floatx16 dp = scores(sV, gb);
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int kk = key_of(i);
            const float p = (rv && row >= sThr[kk]) ? exp2f(sc[i] * c2 - lse) : 0.0f;
            sc[i] = p * (dp[i] - Dr);                       // dS
            sP[kk * L::PSTR + row] = f_to_bf16(p);
            sDS[kk * L::PSTR + row] = f_to_bf16(sc[i]);
        }
        bf16x8 dsb[2];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            dsb[0][j] = (__bf16)sc[j];
            dsb[1][j] = (__bf16)sc[8 + j];
        }
        // dQ^T += K^T dS^T: A = K^T rows (dims), k = keys in the order the score MFMA left them
#pragma unroll
        for (int st = 0; st < 2; ++st) {
            const int kb = 16 * st + 4 * hl;
#pragma unroll
            for (int d = 0; d < DB; ++d) {
                const uint16_t* kr = &sKt[(d * 32 + l % 32) * L::KTSTR];
                const uint2 lo = *reinterpret_cast<const uint2*>(kr + kb);
                const uint2 hi = *reinterpret_cast<const uint2*>(kr + kb + 8);
                dq[d] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
                    __builtin_bit_cast(bf16x8, make_uint4(lo.x, lo.y, hi.x, hi.y)), dsb[st], dq[d],
                    0, 0, 0);
            }
        }
        __syncthreads();
        // wave 0: dK = dS^T Q, wave 1: dV = P^T dO over the chunk's 64 rows; then scatter
        {
            const uint16_t* sA = w == 0 ? sDS : sP;
            const uint16_t* sB = w == 0 ? sQt : sGt;
            float* dst = w == 0 ? dkb : dvb;
            const float mul = w == 0 ? A.scale : 1.0f;
            // two 32-dim blocks at a time keep the accumulators to 32 registers
#pragma unroll
            for (int d0 = 0; d0 < DB; d0 += 2) {
                floatx16 acc[2] = {floatx16{}, floatx16{}};
#pragma unroll
                for (int st = 0; st < kBR / 16; ++st) {
                    const bf16x8 a = ld8(&sA[(l % 32) * L::PSTR + 16 * st + 8 * hl]);
#pragma unroll
                    for (int d = 0; d < 2; ++d)
                        acc[d] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
                            a, ld8(&sB[((d0 + d) * 32 + l % 32) * L::QTSTR + 16 * st + 8 * hl]),
                            acc[d], 0, 0, 0);
                }
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    const int kk = key_of(i);
                    if (sThr[kk] < kNever) {
                        float* o = dst + (int64_t)sPos[kk] * DH + (d0 * 32 + l % 32);
                        unsafeAtomicAdd(o, acc[0][i] * mul);
                        unsafeAtomicAdd(o + 32, acc[1][i] * mul);
                    }
                }
            }
        }
        __syncthreads();
    }
    if (rv) {
        uint16_t* dqp = reinterpret_cast<uint16_t*>(P.dq) + b * P.dq_sb + h * P.dq_sh +
                        (r0 + row) * P.dq_ss;
#pragma unroll
        for (int d = 0; d < DB; ++d)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const int dim = d * 32 + 8 * g + 4 * hl;
                uint2 u;
                u.x = (uint32_t)f_to_bf16(dq[d][4 * g] * A.scale) |
                      ((uint32_t)f_to_bf16(dq[d][4 * g + 1] * A.scale) << 16);
                u.y = (uint32_t)f_to_bf16(dq[d][4 * g + 2] * A.scale) |
                      ((uint32_t)f_to_bf16(dq[d][4 * g + 3] * A.scale) << 16);
                *reinterpret_cast<uint2*>(dqp + dim) = u;
            }
    }
}

}  // namespace
}  // namespace hga

extern "C" int hga_attend_prefill_bwd_workspace(const hga_config* cfg, int32_t S,
                                                int64_t* bytes) {
    using namespace hga;
    int rc = check_config(cfg);
    if (rc) return rc;
    HGA_REQUIRE(S >= 0 && bytes, HGA_ERR_ARG, "hga_attend_prefill_bwd_workspace: bad S/bytes");
    // fp32 dk and dv accumulators
    *bytes = 2 * (int64_t)cfg->batch * cfg->kv_heads * S * cfg->head_dim * (int64_t)sizeof(float);
    return HGA_OK;
}

extern "C" int hga_attend_prefill_bwd(
    const hga_config* cfg, int32_t S, const void* q, int64_t q_sb, int64_t q_sh, int64_t q_ss,
    const void* k, int64_t k_sb, int64_t k_sh, int64_t k_ss, const void* v, int64_t v_sb,
    int64_t v_sh, int64_t v_ss, const void* out, int64_t o_sb, int64_t o_sh, int64_t o_ss,
    const void* dout, int64_t g_sb, int64_t g_sh, int64_t g_ss, const float* lse,
    const int32_t* open_grp, const int32_t* open_thr, int32_t Kg, void* dq, int64_t dq_sb, int64_t dq_sh, int64_t dq_ss,
    void* dk, int64_t dk_sb, int64_t dk_sh, int64_t dk_ss, void* dv, int64_t dv_sb,
    int64_t dv_sh, int64_t dv_ss, void* workspace, int64_t workspace_bytes, void* stream) {
    using namespace hga;
    int rc = check_config(cfg);
    if (rc) return rc;
    HGA_REQUIRE(q && k && v && out && dout && open_grp && open_thr && dq && dk && dv, HGA_ERR_ARG,
                "hga_attend_prefill_bwd: NULL pointer");
    HGA_REQUIRE(S >= 0 && Kg >= 0, HGA_ERR_ARG, "hga_attend_prefill_bwd: negative S/Kg");
    if (S == 0) return HGA_OK;
    HGA_REQUIRE(cfg->chunk_size <= kBR, HGA_ERR_UNSUPPORTED,
                "hga_attend_prefill_bwd: chunk_size %d > %d", cfg->chunk_size, kBR);
    int nN, nKc, nKg;
    hga_prefill_widths(cfg, S, &nN, &nKc, &nKg);
    HGA_REQUIRE(Kg == nKg, HGA_ERR_ARG, "hga_attend_prefill_bwd: Kg %d != routing width %d", Kg,
                nKg);
    int64_t need = 0;
    hga_attend_prefill_bwd_workspace(cfg, S, &need);
    HGA_REQUIRE(workspace && workspace_bytes >= need && (uintptr_t)workspace % 16 == 0,
                HGA_ERR_ARG,
                "hga_attend_prefill_bwd: 16-byte aligned workspace of %lld bytes required (got %lld)",
                (long long)need, (long long)workspace_bytes);
    BwdArgs p{};
    AttnArgs& a = p.a;
    a.q = q; a.q_sb = q_sb; a.q_sh = q_sh; a.q_ss = q_ss;
    a.k = k; a.k_sb = k_sb; a.k_sh = k_sh; a.k_ss = k_ss;
    a.v = v; a.v_sb = v_sb; a.v_sh = v_sh; a.v_ss = v_ss;
    a.out = const_cast<void*>(out); a.o_sb = o_sb; a.o_sh = o_sh; a.o_ss = o_ss;
    a.open_grp = open_grp; a.open_thr = open_thr;
    a.B = cfg->batch; a.H = cfg->heads; a.KVH = cfg->kv_heads; a.S = S;
    a.C = cfg->chunk_size; a.gs = cfg->group_size; a.M = a.C / a.gs;
    a.N = chunks_of(S, a.C); a.kf = cfg->keep_first; a.kl = cfg->keep_last;
    a.Kg = Kg; a.scale = cfg->scale; a.lse = const_cast<float*>(lse);
    p.dout = dout; p.g_sb = g_sb; p.g_sh = g_sh; p.g_ss = g_ss;
    p.dq = dq; p.dq_sb = dq_sb; p.dq_sh = dq_sh; p.dq_ss = dq_ss;
    const int D = cfg->head_dim;
    const int64_t nacc = (int64_t)a.B * a.KVH * S * D;
    p.dk = (float*)workspace;
    p.dv = p.dk + nacc;
    hipStream_t st = (hipStream_t)stream;
    zero_kernel<<<1024, 256, 0, st>>>((float4*)workspace, 2 * nacc / 4);
    rc = launch_status("hga_attend_prefill_bwd");
    if (rc) return rc;
    const unsigned grid = (unsigned)(a.B * a.H * a.N);
    const size_t open_lds = sizeof(int) * (2 * (size_t)kBK + 2 * (size_t)(Kg > 0 ? Kg : 1));
    bool launched = false;
    const uintptr_t al = (uintptr_t)q | (uintptr_t)k | (uintptr_t)v | (uintptr_t)out |
                         (uintptr_t)dout | (uintptr_t)dq;
    const bool aligned = al % 16 == 0 && ((q_sb | q_sh | q_ss | k_sb | k_sh | k_ss | v_sb | v_sh |
                                           v_ss | o_sb | o_sh | o_ss | g_sb | g_sh | g_ss | dq_sb |
                                           dq_sh | dq_ss) % 8) == 0;
    if (cfg->dtype == HGA_DTYPE_BF16 && (D == 64 || D == 128) && aligned) {
        const size_t lds = (D == 128 ? MfmaLds<128>::bytes : MfmaLds<64>::bytes) + open_lds;
        HGA_REQUIRE(lds <= 163840, HGA_ERR_UNSUPPORTED,
                    "hga_attend_prefill_bwd: %d opened groups too many", Kg);
        static bool attr = false;
        if (!attr) {
            (void)hipFuncSetAttribute((const void*)attend_bwd_mfma_kernel<128>,
                                      hipFuncAttributeMaxDynamicSharedMemorySize, 163840);
            (void)hipFuncSetAttribute((const void*)attend_bwd_mfma_kernel<64>,
                                      hipFuncAttributeMaxDynamicSharedMemorySize, 163840);
            attr = true;
        }
        if (D == 128) attend_bwd_mfma_kernel<128><<<grid, kMT, lds, st>>>(p);
        else attend_bwd_mfma_kernel<64><<<grid, kMT, lds, st>>>(p);
        launched = true;
    }
#define HGA_BWD_VALU(DTV, DHV)                                                                   \
    if (!launched && cfg->dtype == DTV && D == DHV) {                                            \
        const size_t lds = sizeof(float) * valu_lds_floats<DHV>() + open_lds;                    \
        HGA_REQUIRE(lds <= 163840, HGA_ERR_UNSUPPORTED,                                          \
                    "hga_attend_prefill_bwd: %d opened groups too many", Kg);                    \
        static bool attr = false;                                                                \
        if (!attr) {                                                                             \
            (void)hipFuncSetAttribute((const void*)attend_bwd_valu_kernel<DTV, DHV>,             \
                                      hipFuncAttributeMaxDynamicSharedMemorySize, 163840);       \
            attr = true;                                                                         \
        }                                                                                        \
        attend_bwd_valu_kernel<DTV, DHV><<<grid, kBT, lds, st>>>(p);                             \
        launched = true;                                                                         \
    }
    HGA_BWD_VALU(HGA_DTYPE_F32, 128)
    HGA_BWD_VALU(HGA_DTYPE_F32, 64)
    HGA_BWD_VALU(HGA_DTYPE_F32, 32)
    HGA_BWD_VALU(HGA_DTYPE_F32, 16)
    HGA_BWD_VALU(HGA_DTYPE_BF16, 128)
    HGA_BWD_VALU(HGA_DTYPE_BF16, 64)
    HGA_BWD_VALU(HGA_DTYPE_BF16, 32)
    HGA_BWD_VALU(HGA_DTYPE_BF16, 16)
#undef HGA_BWD_VALU
    if (!launched) {
        set_error("hga_attend_prefill_bwd: unsupported dtype/head_dim");
        return HGA_ERR_UNSUPPORTED;
    }
    rc = launch_status("hga_attend_prefill_bwd");
    if (rc) return rc;
    const unsigned cg = (unsigned)std::min<int64_t>((nacc + 255) / 256, 4096);
    if (cfg->dtype == HGA_DTYPE_BF16) {
        acc_out_kernel<HGA_DTYPE_BF16><<<cg, 256, 0, st>>>(p.dk, dk, dk_sb, dk_sh, dk_ss, a.KVH, S, D, nacc);
        acc_out_kernel<HGA_DTYPE_BF16><<<cg, 256, 0, st>>>(p.dv, dv, dv_sb, dv_sh, dv_ss, a.KVH, S, D, nacc);
    } else {
        acc_out_kernel<HGA_DTYPE_F32><<<cg, 256, 0, st>>>(p.dk, dk, dk_sb, dk_sh, dk_ss, a.KVH, S, D, nacc);
        acc_out_kernel<HGA_DTYPE_F32><<<cg, 256, 0, st>>>(p.dv, dv, dv_sb, dv_sh, dv_ss, a.KVH, S, D, nacc);
    }
    return launch_status("hga_attend_prefill_bwd");
}
