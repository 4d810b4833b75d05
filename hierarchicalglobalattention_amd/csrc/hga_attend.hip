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
// bf16 path, group and chunk sizes multiples of 16 (head_dim 64/128): kernel v3 below -- the
// query heads of one KV head share a workgroup and the LDS-staged window / own-chunk K/V tiles,
// each head's opened groups are staged per head; S^T = K Q^T and O^T = V^T P^T on
// v_mfma_f32_32x32x16_bf16, software-pipelined.  Other bf16 head_dim 64/128 shapes: a 128-thread
// workgroup per (batch, head, chunk) with 64-key tiles staged in LDS (K row-major, V transposed).
// fp32 path (and head_dim 16/32): one wave per query row at a time, VALU dot products, online
// softmax across the wave.
#include <algorithm>
#include <type_traits>

#include "hga_common.h"
#include "hga_keys.h"

namespace hga {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

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
    block_coords(A.B * A.H * A.N, A.B, A.H, A.KVH, A.N, &b, &h, &n);
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
        if (A.lse && l < 32)                // both half-waves hold the row
            A.lse[((int64_t)b * A.H + h) * A.S + (int64_t)A.C * n + row] = m_run + log2f(l_run);
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
    block_coords(A.B * A.H * A.N, A.B, A.H, A.KVH, A.N, &b, &h, &n);
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
        if (A.lse && l == 0)
            A.lse[((int64_t)b * A.H + h) * A.S + (int64_t)A.C * n + t] =
                (m_run + logf(l_run)) * 1.4426950408889634f;
        const float inv = l_run > 0.0f ? 1.0f / l_run : 0.0f;
#pragma unroll
        for (int e = 0; e < DPL; ++e) {
            const int d = l + 64 * e;
            if (d < DH) E::st(op, ((int64_t)A.C * n + t) * A.o_ss + d, acc[e] * inv);
        }
    }
}

// ------------------------------------------------------------------------------------------
// bf16 MFMA path (group_size and chunk_size multiples of 16): blocked K/V copies + kernel v3
// ------------------------------------------------------------------------------------------
// Blocked operand copies of K and V (one pass per call): a 16-key block is one contiguous run
// that a stage copy takes verbatim, laid out so that every 16-byte operand read of a wave from
// LDS is conflict-free (eight consecutive lanes read 128 consecutive bytes):
//   kb[b][kvh][blk][s][2 halves][16 keys][8 dims]     K[16 blk + key][16 s + 8 half + j]
//   vb[b][kvh][blk][d/32][2 halves][32 dims][8 slots] V[16 blk + vt_key(8 half + j)][d]
// with keys of a 16-key block stored in the order {0-3, 8-11, 4-7, 12-15} in vb: the order in
// which a lane half holds P after the score MFMA.  Keys >= S are zero.  Sp = keys per (b, kvh),
// a multiple of 64.
constexpr int kVtKeys = 64;

__device__ __forceinline__ int vt_key(int slot) {   // key stored at slot (0..15) of a block
    const int g = slot >> 3, j = slot & 7;
    return j < 4 ? 4 * g + j : 8 + 4 * g + (j - 4);
}

template <int DH>
__global__ __launch_bounds__(256) void kv_block_kernel(const uint16_t* __restrict__ k,
                                                       int64_t k_sb, int64_t k_sh, int64_t k_ss,
                                                       const uint16_t* __restrict__ v,
                                                       int64_t v_sb, int64_t v_sh, int64_t v_ss,
                                                       uint16_t* __restrict__ kb,
                                                       uint16_t* __restrict__ vb, int S, int Sp,
                                                       int KVH) {
    constexpr int RS = DH + 8;     // LDS row stride (elements), 16-byte multiple
    constexpr int KS = DH / 16;
    __shared__ __align__(16) uint16_t sK[kVtKeys * RS];
    __shared__ __align__(16) uint16_t sV[kVtKeys * RS];
    const int k0 = blockIdx.x * kVtKeys, kvh = blockIdx.y, b = blockIdx.z;
    const uint16_t* kg = k + b * k_sb + kvh * k_sh;
    const uint16_t* vg = v + b * v_sb + kvh * v_sh;
    constexpr int CPR = DH / 8;
    for (int c = threadIdx.x; c < kVtKeys * CPR; c += 256) {
        const int kk = c / CPR, dp = c % CPR;
        uint4 uk = make_uint4(0u, 0u, 0u, 0u), uv = uk;
        if (k0 + kk < S) {
            uk = *reinterpret_cast<const uint4*>(kg + (int64_t)(k0 + kk) * k_ss + dp * 8);
            uv = *reinterpret_cast<const uint4*>(vg + (int64_t)(k0 + kk) * v_ss + dp * 8);
        }
        *reinterpret_cast<uint4*>(&sK[kk * RS + dp * 8]) = uk;
        *reinterpret_cast<uint4*>(&sV[kk * RS + dp * 8]) = uv;
    }
    __syncthreads();
    const int64_t base = ((int64_t)b * KVH + kvh) * (int64_t)Sp * DH + (int64_t)k0 * DH;
    // kb: 16-byte piece c -> (blk, s, half, key): dims 16s + 8half .. +7 of one key
    for (int c = threadIdx.x; c < kVtKeys * DH / 8; c += 256) {
        const int key = c & 15, half = (c >> 4) & 1, sb = c >> 5;   // sb = blk * KS + s
        const int blk = sb / KS, st = sb % KS;
        const uint4 u = *reinterpret_cast<const uint4*>(&sK[(16 * blk + key) * RS + 16 * st + 8 * half]);
        *reinterpret_cast<uint4*>(kb + base + (int64_t)c * 8) = u;
    }
    // vb: 16-byte piece c -> (blk, dim group, half, dim): slots 8half .. +7 of dim 32*group + dim
    constexpr int DB = DH / 32;
    for (int c = threadIdx.x; c < kVtKeys * DH / 8; c += 256) {
        const int half = (c >> 5) & 1, d = 32 * ((c >> 6) % DB) + (c & 31), blk = (c >> 6) / DB;
        uint32_t w[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int ka = 16 * blk + vt_key(8 * half + 2 * j);
            const int kb2 = 16 * blk + vt_key(8 * half + 2 * j + 1);
            w[j] = (uint32_t)sV[ka * RS + d] | ((uint32_t)sV[kb2 * RS + d] << 16);
        }
        *reinterpret_cast<uint4*>(vb + base + (int64_t)c * 8) = make_uint4(w[0], w[1], w[2], w[3]);
    }
}

// Direct global->LDS copy of 16 bytes per lane: lane i's 16 bytes at sbase + voff land at the
// wave-uniform LDS byte address lds_addr + 16 * i (sbase wave-uniform in SGPRs, voff the lane's
// 32-bit byte offset).  Issued as inline assembly so that the compiler, which cannot prove that
// a copy into one stage does not alias reads of the other, inserts no waits for it; the caller
// waits (vmcnt) before the barrier that publishes a stage.  M0 holds the LDS address; nothing
// else in these kernels uses M0.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void lds_copy16_s(const void* sbase, uint32_t voff, uint32_t lds_addr) {
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2"
                 :: "s"(lds_addr), "v"(voff), "s"(sbase) : "memory", "m0");
}
#pragma clang diagnostic pop

constexpr float kRescaleLog2 = 8.0f;   // a row's softmax reference may trail its max by 2^8
// ------------------------------------------------------------------------------------------
// bf16 MFMA kernel v3: HP query heads of one KV head per workgroup, software-pipelined
// ------------------------------------------------------------------------------------------
// The query heads of a KV head see the same windows and own chunk (the reference repeats K/V
// per head, chunk_router.py:540, vectorized.py:443-472); only their opened groups differ.  A
// workgroup of 2*HP waves takes HP heads of one (batch, KV head, query chunk), wave w = head
// slot w/2, rows 32*(w%2)..+31.  Its key sequence is walked in steps of one 32-key tile
// (two 16-key blocks), in the order
//   window steps (first window | last window): one tile staged in LDS serves the waves of all
//     HP heads (copied once, by all threads);
//   opened steps: each head's two waves compute on that head's own tile of opened groups,
//     staged in a slot of its own (copied by that head's threads);
//   own-chunk steps (causal), shared like the windows, last.
// Software pipeline: step s computes the scores of step s+1 (S = K Q^T, one MFMA chain) in
// the same straight-line block as the softmax and the O^T += V^T P^T product of step s, so a
// wave issues its VALU work between its own MFMAs.  K tiles are therefore staged two steps
// ahead and V tiles one step ahead: the LDS ring holds two K and two V tiles per head slot,
// and after the barrier that opens step s the slots of K_s and V_{s-1} are refilled with
// K_{s+2} and V_{s+1}.  Masks: a window or opened block is visible from one row on, so its
// mask is the exp offset (-inf for a row that does not see the block) and the row maximum
// is taken over the visible block halves; own-chunk tiles are masked per key.  A row's
// running sum adds the bf16 P values the PV product uses, two at a time (v_dot2_f32_bf16),
// except in the variant that stores the log-sum-exp for the backward (fp32 sums).
// (b, kv head, query chunk, head group) of a v3 workgroup.  Workgroups reach the 8 XCDs
// round-robin by linear id; each XCD takes a contiguous range of
// logical = ((b*KVH + kvh)*N + n)*G + hg, so the chunks in flight on one L2 share a KV head.
__device__ __forceinline__ void group_coords(int nitems, int KVH, int N, int G, int* b, int* kvh,
                                             int* n, int* hg) {
    const int bid = blockIdx.x, xcd = bid % 8, slot = bid / 8;
    const int q = nitems / 8, r = nitems % 8;
    const int logical = xcd < r ? xcd * (q + 1) + slot : r * (q + 1) + (xcd - r) * q + slot;
    *hg = logical % G;
    const int t = logical / G;
    *n = t % N;
    const int bk = t / N;
    *b = bk / KVH;
    *kvh = bk % KVH;
}

template <int DH, int HP, bool LSE>
__global__ __launch_bounds__(128 * HP) void attend_v3_kernel(AttnArgs A,
                                                             const uint16_t* __restrict__ kbl,
                                                             const uint16_t* __restrict__ vbl,
                                                             int Sp, int capS, int capO) {
    constexpr int NT = 128 * HP;
    constexpr int KS = DH / 16, DB = DH / 32;
    constexpr int BB = 32 * DH;       // bytes of one 16-key block of K or of V
    constexpr int HT = 2 * BB;        // a half tile: the two K (or V) blocks of one step
    constexpr int RUNS = HT / 1024;   // 1 KiB runs (64 lanes x 16 bytes) per half tile
    static_assert(HP == 1 || HP == 2, "sMeta holds one entry per wave, at most four waves");
    extern __shared__ __align__(16) int sTab[];
    int* sPosS = sTab;                     // shared blocks: first position, first visible row
    int* sThrS = sPosS + capS;
    int* sPosO = sThrS + capS;             // opened blocks of each head slot: [HP][capO]
    int* sThrO = sPosO + HP * capO;
    int* sMeta = sThrO + HP * capO;        // [4]: last valid list entry seen by each wave
    unsigned char* sK = reinterpret_cast<unsigned char*>(sMeta + 4);   // [2][HP][HT]
    unsigned char* sV = sK + 2 * HP * HT;                              // [2][HP][HT]

    const int rep = A.H / A.KVH, G = rep / HP;
    int b, kvh, n, hg;
    group_coords(A.B * A.KVH * A.N * G, A.KVH, A.N, G, &b, &kvh, &n, &hg);
    const int C = A.C, gs = A.gs, M = A.M;
    int rows = A.S - n * C;
    if (rows > C) rows = C;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const int j = w >> 1, rh = w & 1;
    const int h = kvh * rep + hg * HP + j;
    const int l = lane_id(), g = l >> 5, lr = l & 31;
    const int row = 32 * rh + lr;                  // chunk-local query row of this lane
    const int Kgw = A.Kg > 0 ? A.Kg : 1;
    const int gpb = gs / 16, bpc = C / 16;

    // q rows first: their loads overlap the list reads and the table build
    const int kcol = 8 * g;                        // this lane's 8 dims per k-step
    bf16x8 qb[KS];
    {
        const uint16_t* qp = reinterpret_cast<const uint16_t*>(A.q) + b * A.q_sb + h * A.q_sh +
                             ((int64_t)n * C + row) * A.q_ss;
#pragma unroll
        for (int k = 0; k < KS; ++k) {
            uint4 u = make_uint4(0u, 0u, 0u, 0u);
            if (row < rows) u = *reinterpret_cast<const uint4*>(qp + 16 * k + kcol);
            qb[k] = __builtin_bit_cast(bf16x8, u);
        }
    }
    // Head slot j's opened list, read once by its two waves (entry i by thread i % 128 of the
    // slot), goes straight into the slot's table: entry i's blocks at i*gpb.., an invalid entry
    // (group or first row < 0: the router compacts valid entries to the front) and the table's
    // padding never visible.  The slot's opened steps end after its last valid entry.
    const int32_t* ogp = A.open_grp + (((int64_t)b * A.H + h) * A.N + n) * Kgw;
    const int32_t* otp = A.open_thr + (((int64_t)b * A.H + h) * A.N + n) * Kgw;
    {
        const int tl = threadIdx.x - 128 * j;
        int* pj = sPosO + j * capO;
        int* tj = sThrO + j * capO;
        int last = -1;
        for (int i = tl; i < A.Kg; i += 128) {
            const int grp = ogp[i], t = otp[i];
            const bool ok = grp >= 0 && t >= 0;
            if (ok) last = i;
            for (int e = 0; e < gpb; ++e) {
                pj[i * gpb + e] = ok ? (grp / M) * C + (grp % M) * gs + 16 * e : 0;
                tj[i * gpb + e] = ok ? t : kNever;
            }
        }
        for (int gb = A.Kg * gpb + tl; gb < capO; gb += 128) {
            pj[gb] = 0;
            tj[gb] = kNever;
        }
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) last = max(last, __shfl_xor(last, o, kWave));
        if (l == 0) sMeta[w] = last;               // per wave (2 * HP <= 4)
    }
    int f_hi, l_lo;
    windows(n, A.kf, A.kl, &f_hi, &l_lo);
    const int nbF = f_hi * bpc, nbW = nbF + (n - l_lo) * bpc;
    const int nWs = (nbW + 1) / 2;                 // window steps
    const int nbOwn = (rows + 15) / 16;
    const int nCs = (nbOwn + 1) / 2;               // own-chunk steps
    // shared table: window blocks padded to whole tiles, then own-chunk blocks (padding
    // blocks read block 0 and are never visible)
    for (int gb = threadIdx.x; gb < 2 * (nWs + nCs); gb += NT) {
        int pos = 0, thr = kNever;
        if (gb < nbF) {
            pos = gb * 16;
            thr = 0;
        } else if (gb < nbW) {
            pos = l_lo * C + (gb - nbF) * 16;
            thr = 0;
        } else if (gb >= 2 * nWs && gb - 2 * nWs < nbOwn) {
            pos = n * C + 16 * (gb - 2 * nWs);
            thr = 16 * (gb - 2 * nWs);
        }
        sPosS[gb] = pos;
        sThrS[gb] = thr;
    }
    // q is in registers and the list reads are done: the direct LDS copies below are the only
    // vector memory operations in flight inside the step loop
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();                               // tables complete
    int nbO = 0;
#pragma unroll
    for (int jj = 0; jj < 2 * HP; ++jj) nbO = max(nbO, (sMeta[jj] + 1) * gpb);
    const int nOs = (nbO + 1) / 2;                 // opened steps (the longest list of the heads)
    const int T = nWs + nOs + nCs;                 // >= 1: rows >= 1
    const int sC = nWs + nOs;                      // first own-chunk step

    const uint32_t k_lds = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) unsigned char*)sK;
    const uint32_t v_lds = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) unsigned char*)sV;
    const int64_t kvbase = ((int64_t)b * A.KVH + kvh) * (int64_t)Sp * DH;
    const unsigned char* kblk = reinterpret_cast<const unsigned char*>(kbl + kvbase);
    const unsigned char* vblk = reinterpret_cast<const unsigned char*>(vbl + kvbase);
    // index in sTab of step s's table entries (first positions; the first visible rows follow
    // at + capS for shared steps, + HP * capO for opened ones), and the head slot its tile is
    // staged in (0 for shared steps)
    auto step_tab = [&](int s, int& pi, int& ti, int& hs) __attribute__((always_inline)) {
        const bool opened = s >= nWs && s < sC;
        const int i = opened ? 2 * (s - nWs) : 2 * (s < nWs ? s : s - nOs);
        pi = opened ? 2 * capS + j * capO + i : i;
        ti = opened ? pi + HP * capO : pi + capS;
        hs = opened ? j : 0;
    };
    // Copy the K (or V) blocks of step s into ring slot s & 1: a shared tile by all waves, an
    // opened tile by head slot j's two waves.  Run r (1 KiB) of the half tile lies in block
    // r / (RUNS/2); the direct load writes lane i's 16 bytes at the wave-uniform base + 16 i.
    auto copy_half = [&](int s, const unsigned char* src, uint32_t lds) __attribute__((always_inline)) {
        int pi, ti, hs;
        step_tab(s, pi, ti, hs);
        const int2 p2 = *reinterpret_cast<const int2*>(&sTab[pi]);
        const int64_t ba = (int64_t)(__builtin_amdgcn_readfirstlane(p2.x) >> 4) * BB;
        const int64_t bbk = (int64_t)(__builtin_amdgcn_readfirstlane(p2.y) >> 4) * BB;
        const uint32_t dst = lds + (uint32_t)(((s & 1) * HP + hs) * HT);
        auto run = [&](int r) __attribute__((always_inline)) {
            const int blk = r / (RUNS / 2), off = 1024 * (r % (RUNS / 2));
            const uint64_t sa = (uint64_t)(uintptr_t)src + (uint64_t)(blk ? bbk : ba);
            // (readfirstlane returns int: widen through uint32_t, never by sign extension)
            const uint64_t su =
                ((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(sa >> 32)) << 32) |
                (uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)sa);
            lds_copy16_s(reinterpret_cast<const void*>(su), (uint32_t)(off + 16 * l),
                         __builtin_amdgcn_readfirstlane(dst + (uint32_t)(blk * BB + off)));
        };
        if (s < nWs || s >= sC) {                  // shared: all 2*HP waves
#pragma unroll
            for (int rr = 0; rr < (RUNS + 2 * HP - 1) / (2 * HP); ++rr)
                if (w + 2 * HP * rr < RUNS) run(w + 2 * HP * rr);
        } else {                                   // opened: head slot j's two waves
#pragma unroll
            for (int rr = 0; rr < RUNS / 2; ++rr) run(rh + 2 * rr);
        }
    };

    // operand reads from a slot: K lane = key lr of the tile (block lr/16), V lane = dim lr of
    // each 32-dim group; g selects the 8-element half
    const int koff = ((lr >> 4) ? BB : 0) + 256 * g + 16 * (lr & 15);
    const int voff = 512 * g + 16 * lr;
    const float c2 = A.scale * 1.4426950408889634f;
    typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
    const bf16x2 ones = {(__bf16)1.0f, (__bf16)1.0f};

    auto read_k = [&](int s, bf16x8 (&kr)[KS]) {
        int pi, ti, hs;
        step_tab(s, pi, ti, hs);
        const unsigned char* base = sK + ((s & 1) * HP + hs) * HT + koff;
#pragma unroll
        for (int k = 0; k < KS; ++k)
            kr[k] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4*>(base + 512 * k));
    };
    auto read_v = [&](int s, bf16x8 (&vr)[DB][2]) {
        int pi, ti, hs;
        step_tab(s, pi, ti, hs);
        const unsigned char* base = sV + ((s & 1) * HP + hs) * HT + voff;
#pragma unroll
        for (int ks = 0; ks < 2; ++ks)
#pragma unroll
            for (int d = 0; d < DB; ++d)
                vr[d][ks] = __builtin_bit_cast(
                    bf16x8, *reinterpret_cast<const uint4*>(base + ks * BB + 1024 * d));
    };
    auto score = [&](const bf16x8 (&kr)[KS]) {
        floatx16 x = {};
#pragma unroll
        for (int k = 0; k < KS; ++k) x = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kr[k], qb[k], x, 0, 0, 0);
        return x;
    };
    // Mask step s's raw scores: a block visible from row th is masked through the exp offset
    // (vA/vB: does this row see block a/b); own-chunk tiles per key.  Returns the row maximum
    // over the visible scores (-inf if none).
    auto finish = [&](int s, auto causal_tag, floatx16& x, bool& vA, bool& vB) __attribute__((always_inline)) {
        constexpr bool CAUSAL = decltype(causal_tag)::value;
        int pi, ti, hs;
        step_tab(s, pi, ti, hs);
        const int2 t2 = *reinterpret_cast<const int2*>(&sTab[ti]);
        const int thA = __builtin_amdgcn_readfirstlane(t2.x);
        const int thB = __builtin_amdgcn_readfirstlane(t2.y);
        float m;
        if constexpr (CAUSAL) {
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int within = 8 * ((i >> 2) & 1) + 4 * g + (i & 3);
                x[i] = row >= (i < 8 ? thA : thB) + within ? x[i] : -INFINITY;
            }
            vA = vB = true;
            m = -INFINITY;
#pragma unroll
            for (int i = 0; i < 16; ++i) m = fmaxf(m, x[i]);
        } else {
            vA = row >= thA;
            vB = row >= thB;
            float ma = -INFINITY, mb = -INFINITY;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                ma = fmaxf(ma, x[i]);
                mb = fmaxf(mb, x[8 + i]);
            }
            m = fmaxf(vA ? ma : -INFINITY, vB ? mb : -INFINITY);
        }
        return fmaxf(m, __shfl_xor(m, 32, kWave));
    };

    floatx16 acc[DB];
#pragma unroll
    for (int d = 0; d < DB; ++d) acc[d] = floatx16{};
    float m_ref = -INFINITY, l_run = 0.0f;
    // Adopt a tile's row maximum as the softmax reference: the first finite one (the
    // accumulators are still zero then), or one beyond the reference by more than 2^8, which
    // rescales the accumulators and running sum (rare: a wave-uniform branch skips it).
    auto adopt = [&](float m) __attribute__((always_inline)) {
        bool jump = false;
        if (m_ref == -INFINITY) m_ref = m;
        else jump = (m - m_ref) * c2 > kRescaleLog2;
        if (__builtin_amdgcn_ballot_w64(jump)) {
            if (jump) {
                const float f = __builtin_amdgcn_exp2f((m_ref - m) * c2);
#pragma unroll
                for (int d = 0; d < DB; ++d)
#pragma unroll
                    for (int i = 0; i < 16; ++i) acc[d][i] *= f;
                l_run *= f;
                m_ref = m;
            }
        }
    };
    // softmax numerators of the current tile (bf16) and the running sum
    auto softmax = [&](const floatx16& x, bool vA, bool vB, bf16x8 (&pt)[2]) {
        const float nb = m_ref == -INFINITY ? 0.0f : -m_ref * c2;
        const float nA = vA ? nb : -INFINITY, nB = vB ? nb : -INFINITY;
        if constexpr (LSE) {   // the backward's log-sum-exp: fp32 sums of the fp32 values
            float rs = 0.0f;
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const float e = __builtin_amdgcn_exp2f(fmaf(x[i], c2, i < 8 ? nA : nB));
                pt[i >> 3][i & 7] = (__bf16)e;
                rs += e;
            }
            l_run += rs;
        } else {
#pragma unroll
            for (int i = 0; i < 16; ++i)
                pt[i >> 3][i & 7] = (__bf16)__builtin_amdgcn_exp2f(fmaf(x[i], c2, i < 8 ? nA : nB));
#pragma unroll
            for (int k2 = 0; k2 < 2; ++k2)
#pragma unroll
                for (int pr = 0; pr < 4; ++pr) {
                    const bf16x2 two = {pt[k2][2 * pr], pt[k2][2 * pr + 1]};
                    l_run = __builtin_amdgcn_fdot2_f32_bf16(two, ones, l_run, false);
                }
        }
    };
    auto pv = [&](const bf16x8 (&vr)[DB][2], const bf16x8 (&pt)[2]) {
#pragma unroll
        for (int ks = 0; ks < 2; ++ks)
#pragma unroll
            for (int d = 0; d < DB; ++d)
                acc[d] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vr[d][ks], pt[ks], acc[d], 0, 0, 0);
    };

    // prologue: K_0, V_0 and K_1 staged, scores of step 0
    copy_half(0, kblk, k_lds);
    copy_half(0, vblk, v_lds);
    if (T > 1) copy_half(1, kblk, k_lds);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    floatx16 sc;
    bool vA, vB;
    {
        bf16x8 kr[KS];
        read_k(0, kr);
        sc = score(kr);
        const float m = sC == 0 ? finish(0, std::true_type{}, sc, vA, vB)
                                : finish(0, std::false_type{}, sc, vA, vB);
        adopt(m);
    }
    // step s: stage K_{s+2} and V_{s+1}; scores of step s+1 with the softmax and PV of step s
    auto step = [&](int s, auto causal_next) __attribute__((always_inline)) {
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");   // K_{s+1}, V_s copied (this thread)
        __syncthreads();                                    // by everyone; K_s, V_{s-1} read
        if (s + 2 < T) copy_half(s + 2, kblk, k_lds);
        copy_half(s + 1, vblk, v_lds);
        bf16x8 kr[KS];
        read_k(s + 1, kr);
        bf16x8 vr[DB][2];
        read_v(s, vr);
        floatx16 sn = score(kr);
        bf16x8 pt[2];
        softmax(sc, vA, vB, pt);
        pv(vr, pt);
        const float m = finish(s + 1, causal_next, sn, vA, vB);
        sc = sn;
        adopt(m);
    };
    int s = 0;
    for (; s + 1 < sC; ++s) step(s, std::false_type{});
    for (; s + 1 < T; ++s) step(s, std::true_type{});
    {   // last step: softmax and PV only
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        bf16x8 vr[DB][2];
        read_v(s, vr);
        bf16x8 pt[2];
        softmax(sc, vA, vB, pt);
        pv(vr, pt);
    }

    const float lt = l_run + __shfl_xor(l_run, 32, kWave);
    if (row >= rows) return;
    if constexpr (LSE)
        if (g == 0) A.lse[((int64_t)b * A.H + h) * A.S + (int64_t)C * n + row] = m_ref * c2 + log2f(lt);
    const float inv = lt > 0.0f ? 1.0f / lt : 0.0f;
    uint16_t* op = reinterpret_cast<uint16_t*>(A.out) + b * A.o_sb + h * A.o_sh +
                   ((int64_t)C * n + row) * A.o_ss;
    typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
#pragma unroll
    for (int d = 0; d < DB; ++d)
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4) {
            const int dim = d * 32 + 8 * q4 + 4 * g;
            bf16x4 o;   // hardware round-to-nearest-even conversion
            o[0] = (__bf16)(acc[d][4 * q4] * inv);
            o[1] = (__bf16)(acc[d][4 * q4 + 1] * inv);
            o[2] = (__bf16)(acc[d][4 * q4 + 2] * inv);
            o[3] = (__bf16)(acc[d][4 * q4 + 3] * inv);
            *reinterpret_cast<uint2*>(op + dim) = __builtin_bit_cast(uint2, o);
        }
}

}  // namespace
}  // namespace hga

namespace {
// v3 applies to bf16, head_dim 64/128, group and chunk sizes that are multiples of 16.
bool use_v3(const hga_config* cfg) {
    return cfg->dtype == HGA_DTYPE_BF16 && (cfg->head_dim == 64 || cfg->head_dim == 128) &&
           cfg->group_size % 16 == 0 && cfg->chunk_size % 16 == 0;
}
template <int DH, int HP, bool LSE>
int launch_v3_t(const hga::AttnArgs& a, const uint16_t* kbl, const uint16_t* vbl, int Sp,
                int capS, int capO, unsigned grid, size_t lds, hipStream_t st) {
    auto kern = hga::attend_v3_kernel<DH, HP, LSE>;
    if (lds > 65536)
        HGA_REQUIRE(hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                        hipFuncAttributeMaxDynamicSharedMemorySize,
                                        (int)lds) == hipSuccess,
                    HGA_ERR_LAUNCH, "hga_attend_prefill: %zu bytes of LDS refused", lds);
    kern<<<grid, 128 * HP, lds, st>>>(a, kbl, vbl, Sp, capS, capO);
    return hga::launch_status("hga_attend_prefill");
}
template <int DH, int HP>
int launch_v3_h(const hga::AttnArgs& a, const uint16_t* kbl, const uint16_t* vbl, int Sp,
                int capS, int capO, bool lse, unsigned grid, size_t lds, hipStream_t st) {
    return lse ? launch_v3_t<DH, HP, true>(a, kbl, vbl, Sp, capS, capO, grid, lds, st)
               : launch_v3_t<DH, HP, false>(a, kbl, vbl, Sp, capS, capO, grid, lds, st);
}
template <int DH>
int launch_v3_d(const hga::AttnArgs& a, const uint16_t* kbl, const uint16_t* vbl, int Sp,
                int capS, int capO, int HP, bool lse, unsigned grid, size_t lds, hipStream_t st) {
    if (HP == 2) return launch_v3_h<DH, 2>(a, kbl, vbl, Sp, capS, capO, lse, grid, lds, st);
    return launch_v3_h<DH, 1>(a, kbl, vbl, Sp, capS, capO, lse, grid, lds, st);
}
// v3 launch: head_dim 64/128, HP = query heads of one KV head per workgroup (1 or 2)
int launch_v3(const hga::AttnArgs& a, const uint16_t* kbl, const uint16_t* vbl, int Sp, int capS,
              int capO, int D, int HP, bool lse, unsigned grid, size_t lds, hipStream_t st) {
    return D == 128 ? launch_v3_d<128>(a, kbl, vbl, Sp, capS, capO, HP, lse, grid, lds, st)
                    : launch_v3_d<64>(a, kbl, vbl, Sp, capS, capO, HP, lse, grid, lds, st);
}
int64_t vt_keys(const hga_config* cfg, int32_t S) {   // Sp: keys per V^T row
    const int64_t NC = (int64_t)hga::chunks_of(S, cfg->chunk_size) * cfg->chunk_size;
    return (NC + hga::kVtKeys - 1) / hga::kVtKeys * hga::kVtKeys;
}
}  // namespace

extern "C" int hga_attend_prefill_workspace(const hga_config* cfg, int32_t S, int64_t* bytes) {
    using namespace hga;
    int rc = check_config(cfg);
    if (rc) return rc;
    HGA_REQUIRE(S >= 0 && bytes, HGA_ERR_ARG, "hga_attend_prefill_workspace: bad S/bytes");
    // blocked copies of K and V
    *bytes = use_v3(cfg) && S > 0
                 ? 2 * (int64_t)cfg->batch * cfg->kv_heads * cfg->head_dim * vt_keys(cfg, S) * 2
                 : 0;
    return HGA_OK;
}

extern "C" int hga_attend_prefill(const hga_config* cfg, int32_t S, const void* q, int64_t q_sb,
                                  int64_t q_sh, int64_t q_ss, const void* k, int64_t k_sb,
                                  int64_t k_sh, int64_t k_ss, const void* v, int64_t v_sb,
                                  int64_t v_sh, int64_t v_ss, const int32_t* open_grp,
                                  const int32_t* open_thr, int32_t Kg, void* out, int64_t o_sb,
                                  int64_t o_sh, int64_t o_ss, float* lse, void* workspace,
                                  int64_t workspace_bytes, void* stream) {
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
    a.N = chunks_of(S, a.C); a.kf = cfg->keep_first; a.kl = cfg->keep_last;
    a.Kg = Kg; a.scale = cfg->scale; a.lse = lse;
    int nN, nKc, nKg;
    hga_prefill_widths(cfg, S, &nN, &nKc, &nKg);
    HGA_REQUIRE(Kg == nKg, HGA_ERR_ARG, "hga_attend_prefill: Kg %d != routing width %d", Kg, nKg);
    const int D = cfg->head_dim;
    const unsigned grid = (unsigned)(a.B * a.H * a.N);
    const size_t lds = sizeof(int) * 2 * (size_t)(Kg > 0 ? Kg : 1);
    hipStream_t st = (hipStream_t)stream;
    if (use_v3(cfg)) {
        const uintptr_t al = (uintptr_t)q | (uintptr_t)k | (uintptr_t)v | (uintptr_t)out |
                             (uintptr_t)workspace;
        HGA_REQUIRE(al % 16 == 0 && ((q_sb | q_sh | q_ss | k_sb | k_sh | k_ss | v_sb | v_sh |
                                      v_ss | o_sb | o_sh | o_ss) % 8) == 0,
                    HGA_ERR_ARG, "hga_attend_prefill: 16-byte aligned rows required");
        int64_t need = 0;
        hga_attend_prefill_workspace(cfg, S, &need);
        HGA_REQUIRE(workspace && workspace_bytes >= need, HGA_ERR_ARG,
                    "hga_attend_prefill: workspace of %lld bytes required (got %lld)",
                    (long long)need, (long long)workspace_bytes);
        const int Sp = (int)vt_keys(cfg, S);
        uint16_t* kbl = (uint16_t*)workspace;
        uint16_t* vbl = kbl + (int64_t)a.B * a.KVH * Sp * D;
        // the windows of chunk n cover min(kf, n) + (n - l_lo) <= min(kf + kl, N - 1) chunks
        const int bpc = a.C / 16;
        const int64_t wch = std::min<int64_t>((int64_t)a.kf + a.kl, a.N - 1);
        // query heads of one KV head per workgroup: two (two 2-wave heads share the window and
        // own-chunk tiles; four heads would fit only one workgroup per CU by LDS), else one
        const int rep = a.H / a.KVH;
        const int HP = rep % 2 == 0 ? 2 : 1;
        // tables of the shared blocks (windows, own chunk) and of each head's opened blocks,
        // each padded to whole tiles
        const int capS = (int)(2 * ((wch * bpc + 1) / 2 + (bpc + 1) / 2));
        const int capO = std::max(2, (Kg * (a.gs / 16) + 1) / 2 * 2);
        // tables, then K and V rings of two half tiles per head slot
        const size_t lds3 = sizeof(int) * (2 * (size_t)capS + 2 * (size_t)HP * capO + 4) +
                            2 * (size_t)HP * 4 * 32 * D;
        HGA_REQUIRE(lds3 <= 160 * 1024, HGA_ERR_UNSUPPORTED,
                    "hga_attend_prefill: key sequence too long for the LDS tables");
        HGA_REQUIRE((int64_t)Sp * D * 2 < ((int64_t)1 << 32), HGA_ERR_UNSUPPORTED,
                    "hga_attend_prefill: block of %d tokens too long", S);
        dim3 tg((unsigned)(Sp / kVtKeys), (unsigned)a.KVH, (unsigned)a.B);
        if (D == 128)
            kv_block_kernel<128><<<tg, 256, 0, st>>>((const uint16_t*)k, k_sb, k_sh, k_ss,
                                                     (const uint16_t*)v, v_sb, v_sh, v_ss, kbl,
                                                     vbl, S, Sp, a.KVH);
        else
            kv_block_kernel<64><<<tg, 256, 0, st>>>((const uint16_t*)k, k_sb, k_sh, k_ss,
                                                    (const uint16_t*)v, v_sb, v_sh, v_ss, kbl,
                                                    vbl, S, Sp, a.KVH);
        const unsigned grid3 = (unsigned)(a.B * a.KVH * a.N * (rep / HP));
        return launch_v3(a, kbl, vbl, Sp, capS, capO, D, HP, lse != nullptr, grid3, lds3, st);
    }
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
