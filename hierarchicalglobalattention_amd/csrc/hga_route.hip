// Two-level prefill router (vectorized.py:242-396) for gfx950.
//
// Stage 1: one 512-thread workgroup per (batch, query head, query chunk n), at most ~80 KB of LDS
// so that two share a CU; stage 2: one 256-thread workgroup per chunk.  Nothing is materialised
// in HBM except the routing lists.
//
//   1. Stage 1, per 32-row block of the chunk: scores of the block's query rows against every
//      candidate of the routing pool P(n) = [f_hi, l_lo) are produced into LDS by bf16 MFMA
//      (S^T = K * Q^T, v_mfma_f32_32x32x16_bf16, fp32 accumulate, both operands straight from
//      global memory), or by the canonical fp32 FMA chain for fp32 inputs / HGA_ROUTE_CANONICAL.
//   2. Per-row top-min(Kc,|P|) by row groups: 16 lanes own one row (four rows per wave), hold
//      its scores in registers as order-preserving keys and run an interpolation search for a
//      separating threshold (seeded from the row's mean and standard deviation, secant steps on
//      DPP-reduced counts, then key-space bisection), ties to the lower chunk id.  MFMA scores
//      differ from the canonical chain by at most delta = 2^-16 * |q| * |k| * scale (both are
//      fp32 accumulations of the same exact bf16 products); a row whose k-th and (k+1)-th scores
//      are closer than 2*delta goes to the canonical path: the candidates inside the band are
//      re-scored with the canonical chain and the remaining slots filled exactly, so selections
//      equal the canonical oracle's.
//   3. Requests are pooled per chunk (max score, first requesting row) with LDS atomics; one
//      wave takes the top-Kc pooled chunks (same certification; ambiguous pooled maxima are
//      recomputed canonically over the requesting rows), forces in chunk n-1 when it lies in the
//      pool, and writes the sorted (chunk, first row) list.
//   4. Stage 2 repeats 1-3 for all rows at once over the M groups of each selected chunk, a
//      group being visible to a row from its parent's first row on; top-Kgr requests per row,
//      top-Kg opened.
#include "hga_common.h"
#include "hga_select.h"

namespace hga {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int kThreads = 512;
constexpr int kWaves = kThreads / kWave;
constexpr int kRows = 64;     // query rows per chunk (C <= 64)
constexpr int kBlk = 32;      // stage-1 row block
constexpr int kJ = 8;         // candidates per lane in a prefill selection: <= 512 candidates
constexpr int kMaxSel = 64;   // Kc bound
constexpr float kDeltaRel = 1.0f / 65536.0f;

struct RouteArgs {
    const void* q;
    int64_t q_sb, q_sh, q_ss;
    const void* ck;
    int64_t ck_sb, ck_sh;
    const void* gk;
    int64_t gk_sb, gk_sh;
    int32_t *sel_chunk, *sel_thr, *n_sel, *open_grp, *open_thr, *n_open;
    int32_t* stats;
    int B, H, KVH, S, N, C, M, kf, kl, Kc, Kg, Kgr;
    int n_hi;                // fused launches: query chunks n_hi - 1, n_hi - 2, ... of the grid
    int SP, SP2, SSZ, SPP, BW, SPP2, BW2, VT2, canonical;
    float scale;
};

// ------------------------------------------------------------------------------------------
// scores
// ------------------------------------------------------------------------------------------
// Canonical score: sequential fp32 FMA chain over d = 0..DH-1, then * scale (-0 -> +0).
// q and k are read with 16-byte vector loads (LDS or global); the chain order is unchanged.
template <int DT, int DH>
__device__ __forceinline__ float canon_dot(const typename Elem<DT>::T* q,
                                           const typename Elem<DT>::T* k, float scale) {
    float acc = 0.0f;
    if constexpr (DT == HGA_DTYPE_BF16) {
        for (int p = 0; p < DH / 32; ++p) {          // 32 dims per step, 16-byte loads
            uint4 kr[4], qr[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                kr[i] = *reinterpret_cast<const uint4*>(k + 32 * p + 8 * i);
                qr[i] = *reinterpret_cast<const uint4*>(q + 32 * p + 8 * i);
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t qw[4] = {qr[i].x, qr[i].y, qr[i].z, qr[i].w};
                const uint32_t kw[4] = {kr[i].x, kr[i].y, kr[i].z, kr[i].w};
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    acc = fmaf(__uint_as_float(qw[e] << 16), __uint_as_float(kw[e] << 16), acc);
                    acc = fmaf(__uint_as_float(qw[e] & 0xffff0000u),
                               __uint_as_float(kw[e] & 0xffff0000u), acc);
                }
            }
        }
        if constexpr (DH % 32 != 0) {                 // DH == 16
            const uint4 kr0 = *reinterpret_cast<const uint4*>(k), kr1 = *reinterpret_cast<const uint4*>(k + 8);
            const uint4 qr0 = *reinterpret_cast<const uint4*>(q), qr1 = *reinterpret_cast<const uint4*>(q + 8);
            const uint32_t qw[8] = {qr0.x, qr0.y, qr0.z, qr0.w, qr1.x, qr1.y, qr1.z, qr1.w};
            const uint32_t kw[8] = {kr0.x, kr0.y, kr0.z, kr0.w, kr1.x, kr1.y, kr1.z, kr1.w};
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                acc = fmaf(__uint_as_float(qw[e] << 16), __uint_as_float(kw[e] << 16), acc);
                acc = fmaf(__uint_as_float(qw[e] & 0xffff0000u), __uint_as_float(kw[e] & 0xffff0000u), acc);
            }
        }
    } else {
        for (int p = 0; p < DH / 16; ++p) {
            float4 kr[4], qr[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                kr[i] = *reinterpret_cast<const float4*>(k + 16 * p + 4 * i);
                qr[i] = *reinterpret_cast<const float4*>(q + 16 * p + 4 * i);
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                acc = fmaf(qr[i].x, kr[i].x, acc);
                acc = fmaf(qr[i].y, kr[i].y, acc);
                acc = fmaf(qr[i].z, kr[i].z, acc);
                acc = fmaf(qr[i].w, kr[i].w, acc);
            }
        }
    }
    const float s = acc * scale;
    return s == 0.0f ? 0.0f : s;
}

__device__ __forceinline__ bf16x8 as_bf16x8(uint4 u) { return __builtin_bit_cast(bf16x8, u); }

// Sum of squares of the 8 bf16 values of a 16-byte word (packed bf16 dot products).  Only used
// for the certification bound, which carries a 1% margin for its rounding.
__device__ __forceinline__ float sumsq_bf16x8(uint4 u) {
    typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
    float s = 0.0f;
#pragma unroll
    for (int e = 0; e < 4; ++e)
        s = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, w[e]),
                                            __builtin_bit_cast(bf16x2, w[e]), s, false);
    return s;
}

// bf16 MFMA scores (scaled; -0 folded into +0) of the query rows [32*rb, 32*rb + 32) (rb < nrb)
// against all candidates, written row-major to sRows[row * stride + c].  Computed as
// S^T = K * Q^T with v_mfma_f32_32x32x16_bf16 (candidates on the M side, query rows on the N
// side), so a lane's 16 results are four runs of four consecutive candidates of one query row
// and are written with 16-byte stores at constant offsets (stride: a multiple of 4 covering
// every candidate tile).  Both operands are read from global memory: candidate rows through
// rowptr, query row t at qg + t*q_ss (rows >= `rows` read as zero).  Wave w takes the jobs
// (row block, candidate tile) w, w+NW, ..., row block fastest.  The wave holding tile 0 of a row
// block writes the block's query norms to sQn[t]; with knmax the largest candidate norm (row
// block 0's tiles) is folded into *knmax (uint bits of a non-negative float).  VIS: candidate c
// of row t gets -inf unless vthr[c] <= t.
template <int DH, int NW, bool VIS, class RowPtr>
__device__ __forceinline__ void scores_st(const uint16_t* qg, int64_t q_ss, int rows, int nrb, int ncand,
                          RowPtr rowptr, const int* vthr, float* sRows, int stride, float scale,
                          uint32_t* knmax, float* sQn) {
    constexpr int KS = DH / 16;
    const int w = threadIdx.x / kWave, l = lane_id(), j = l % 32, hh = l / 32;
    const int ntile = (ncand + 31) / 32;
    int cur = -1;
    bf16x8 b[KS];
    for (int job = w; job < nrb * ntile; job += NW) {
        const int rb = job % nrb, ct = job / nrb;
        const int t = 32 * rb + j;
        if (rb != cur) {            // wave-uniform: query operand of the row block
            cur = rb;
            uint4 u[KS];
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
                u[ks] = make_uint4(0u, 0u, 0u, 0u);
                if (t < rows)
                    u[ks] = *reinterpret_cast<const uint4*>(qg + (int64_t)t * q_ss + ks * 16 + 8 * hh);
            }
            if (ct == 0) {
                float x = 0.0f;
#pragma unroll
                for (int ks = 0; ks < KS; ++ks) x += sumsq_bf16x8(u[ks]);
                x += __shfl_xor(x, 32, kWave);
                if (hh == 0) sQn[t] = __builtin_sqrtf(x);
            }
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) b[ks] = as_bf16x8(u[ks]);
        }
        const int c = ct * 32 + j;
        const bool cv = c < ncand;
        const uint16_t* kp = rowptr(cv ? c : 0);
        uint4 a[KS];
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            a[ks] = make_uint4(0u, 0u, 0u, 0u);
            if (cv) a[ks] = *reinterpret_cast<const uint4*>(kp + ks * 16 + 8 * hh);
        }
        floatx16 acc = {};
#pragma unroll
        for (int ks = 0; ks < KS; ++ks)
            acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(a[ks]), b[ks], acc, 0, 0, 0);
        if (knmax && rb == 0) {
            float nsq = 0.0f;
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) nsq += sumsq_bf16x8(a[ks]);
            nsq += __shfl_xor(nsq, 32, kWave);
            if (cv && hh == 0) atomicMax(knmax, __float_as_uint(__builtin_sqrtf(nsq)));
        }
        float* dst = sRows + t * stride + ct * 32 + 4 * hh;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            float4 o;
            o.x = fmaf(acc[4 * g + 0], scale, 0.0f);
            o.y = fmaf(acc[4 * g + 1], scale, 0.0f);
            o.z = fmaf(acc[4 * g + 2], scale, 0.0f);
            o.w = fmaf(acc[4 * g + 3], scale, 0.0f);
            if constexpr (VIS) {
                const int4 th = *reinterpret_cast<const int4*>(vthr + ct * 32 + 8 * g + 4 * hh);
                o.x = th.x <= t ? o.x : -INFINITY;
                o.y = th.y <= t ? o.y : -INFINITY;
                o.z = th.z <= t ? o.z : -INFINITY;
                o.w = th.w <= t ? o.w : -INFINITY;
            }
            *reinterpret_cast<float4*>(dst + 8 * g) = o;
        }
    }
}

// One query row's requests: members raise the candidate's pooled key to okey(score), lower its
// first row to t, and set bit (t, i).  v: the row's approximate scores (-inf = not visible).
template <int J, class Canon>
__device__ __forceinline__ void row_request(int t, const float (&v)[J], int k, float delta,
                                            Canon canon, uint32_t* sPk, int* sFirst,
                                            uint32_t* sBits, int BW, int* amb) {
    const int l = lane_id();
    const uint32_t mem = select_certified<J>(v, k, delta, canon, amb);
#pragma unroll
    for (int j = 0; j < J; ++j) {
        const bool m = (mem >> j) & 1u;
        if (m) {
            const int i = l + 64 * j;
            atomicMax(&sPk[i], okey(v[j]));
            atomicMin(&sFirst[i], t);
        }
        const uint64_t bal = __ballot(m);
        if (l == 0) {
            if (2 * j < BW) sBits[t * BW + 2 * j] = (uint32_t)bal;
            if (2 * j + 1 < BW) sBits[t * BW + 2 * j + 1] = (uint32_t)(bal >> 32);
        }
    }
}

// Canonical pooled value of candidate i: max of the canonical scores over the rows that
// requested it.
template <class Canon>
__device__ float pooled_exact(int i, int rows, const uint32_t* sBits, int BW, Canon canon_row) {
    float best = -INFINITY;
    for (int t = 0; t < rows; ++t)
        if ((sBits[t * BW + i / 32] >> (i % 32)) & 1u) best = fmaxf(best, canon_row(t, i));
    return best;
}

// Wave 0: top-k of the requested candidates by pooled score (certified), optional forced
// candidate `ip` (evicting the last-ranked one when full), written ascending to sSel/sThr with
// ids base_id + i; returns the count (wave-uniform).
template <int J, class Canon>
__device__ __forceinline__ int pooled_select(int ncand, int k, int rows, const uint32_t* sBits, int BW,
                             const uint32_t* sPk, const int* sFirst, float dpool,
                             Canon canon_row, int ip, int base_id, int* sSel, int* sThr,
                             int* amb) {
    const int l = lane_id();
    float v[J];
#pragma unroll
    for (int j = 0; j < J; ++j) {
        const int i = l + 64 * j;
        v[j] = (i < ncand && sFirst[i] < kNoRow) ? okey_inv(sPk[i]) : -INFINITY;
    }
    auto canon_pool = [&](int i) { return pooled_exact(i, rows, sBits, BW, canon_row); };
    uint32_t sel = select_certified<J>(v, k, dpool, canon_pool, amb);
    if (ip >= 0) {
        const bool have = __ballot(((sel >> (ip / 64)) & 1u) && l == ip % 64) != 0;
        if (!have) {
            int nsel = 0;
#pragma unroll
            for (int j = 0; j < J; ++j) nsel += __popcll(__ballot((sel >> j) & 1u));
            if (nsel >= k) {
                // evict the last-ranked selected candidate: lowest pooled, then highest id
                float mn = INFINITY;
#pragma unroll
                for (int j = 0; j < J; ++j)
                    if ((sel >> j) & 1u) mn = fminf(mn, v[j]);
                mn = wmin(mn);
                uint32_t ev[J];
                uint32_t best = 0u;
#pragma unroll
                for (int j = 0; j < J; ++j) {
                    const bool cand = ((sel >> j) & 1u) && v[j] <= mn + 2.0f * dpool;
                    const float e = cand ? (dpool > 0.0f ? canon_pool(l + 64 * j) : v[j]) : 0.0f;
                    ev[j] = cand ? ~okey(e) : 0u;
                    best = max(best, ev[j]);
                }
                best = (uint32_t)wave_reduce_bits((int)best, [](int a, int b) {
                    return (int)max((uint32_t)a, (uint32_t)b);
                });
                int victim = -1;
#pragma unroll
                for (int j = J - 1; j >= 0; --j) {
                    const uint64_t m = __ballot(ev[j] == best && best != 0u);
                    if (victim < 0 && m) victim = 64 * j + 63 - __clzll(m);
                }
                if (victim >= 0 && l == victim % 64) sel &= ~(1u << (victim / 64));
            }
            if (l == ip % 64) sel |= 1u << (ip / 64);
        }
    }
    int base = 0;
#pragma unroll
    for (int j = 0; j < J; ++j) {
        const bool m = (sel >> j) & 1u;
        const uint64_t bal = __ballot(m);
        if (m) {
            const int i = l + 64 * j;
            const int pos = base + lanes_below(bal);
            sSel[pos] = base_id + i;
            sThr[pos] = i == ip ? 0 : sFirst[i];
        }
        base += __popcll(bal);
    }
    return base;
}

// ------------------------------------------------------------------------------------------
// row-group selection: one query row per 16-lane DPP row, four rows per wave in lockstep
// ------------------------------------------------------------------------------------------
// Lane `seg` (= lane % 16) of a row holds JJ candidates in registers: with W = min(JJ, 4),
// register W*g + e holds candidate 16*W*g + W*seg + e (g < JJ/W, e < W), so that a lane reads
// W consecutive scores at once.  The per-row count of keys >= x is a 16-lane DPP reduction, so
// a search step costs 2*JJ + 8 VALU operations for four rows at once.
// DPP source with the operation's identity as the "old" value and bound_ctrl set (every lane
// reads a valid source in these patterns), so the compiler can fold the move into the op.
template <int CTRL, int IDENT>
__device__ __forceinline__ int dppi(int x) {
    return __builtin_amdgcn_update_dpp(IDENT, x, CTRL, 0xf, 0xf, true);
}
// Butterfly over the 16 lanes of a DPP row: every step pairs each lane with a partner that
// pairs back with it (xor 1, xor 2, then the half-row and row mirrors, which act as xor 4 and
// xor 8 once values are uniform within quads and half-rows), so with a commutative op all 16
// lanes end bit-identical even for floating-point sums (a rotation pattern would add the
// partial sums in a lane-dependent order and leave lanes of one row with different roundings).
template <int IDENT, class Op>
__device__ __forceinline__ int row16_reduce(int x, Op op) {
    x = op(x, dppi<0xB1, IDENT>(x));    // quad_perm [1,0,3,2]
    x = op(x, dppi<0x4E, IDENT>(x));    // quad_perm [2,3,0,1]
    x = op(x, dppi<0x141, IDENT>(x));   // row_half_mirror
    x = op(x, dppi<0x140, IDENT>(x));   // row_mirror
    return x;
}
__device__ __forceinline__ int r16_sum(int x) { return row16_reduce<0>(x, [](int a, int b) { return a + b; }); }
__device__ __forceinline__ float r16_fsum(float x) {
    return __int_as_float(row16_reduce<0>(__float_as_int(x), [](int a, int b) {
        return __float_as_int(__int_as_float(a) + __int_as_float(b));
    }));
}
__device__ __forceinline__ uint32_t r16_umin(uint32_t x) {
    return (uint32_t)row16_reduce<-1>((int)x, [](int a, int b) { return (int)min((uint32_t)a, (uint32_t)b); });
}
__device__ __forceinline__ uint32_t r16_umax(uint32_t x) {
    return (uint32_t)row16_reduce<0>((int)x, [](int a, int b) { return (int)max((uint32_t)a, (uint32_t)b); });
}

template <int JJ>
__device__ __forceinline__ int r16_count_ge(const uint32_t (&kv)[JJ], uint32_t x) {
    int c = 0;
#pragma unroll
    for (int i = 0; i < JJ; ++i) c += kv[i] >= x ? 1 : 0;
    return r16_sum(c);
}

// Order-preserving key in three operations; differs from okey only for -0, which the score
// producers never emit (the MFMA epilogue adds +0, canon_dot folds -0).
__device__ __forceinline__ uint32_t okey_fast(float f) {
    const uint32_t u = __float_as_uint(f);
    return u ^ ((uint32_t)((int32_t)u >> 31) | 0x80000000u);
}

// Upper-tail normal quantile (Abramowitz & Stegun 26.2.23) with hardware log/sqrt/rcp: a search
// seed only, so approximate transcendental instructions are fine.
__device__ __forceinline__ float z_upper_fast(float p) {
    p = fminf(fmaxf(p, 1e-6f), 1.0f - 1e-6f);
    const bool lower = p > 0.5f;
    const float pp = lower ? 1.0f - p : p;
    const float t = __builtin_amdgcn_sqrtf(-2.0f * 0.69314718f * __builtin_amdgcn_logf(pp));
    const float z = t - (2.515517f + 0.802853f * t + 0.010328f * t * t) *
                            __builtin_amdgcn_rcpf(1.0f + 1.432788f * t + 0.189269f * t * t +
                                                  0.001308f * t * t * t);
    return lower ? -z : z;
}

// Row statistics gathered while loading: nv valid candidates; the search seed's sample (the
// row's first read group, at most 64 candidates): ns values, their sum and sum of squares.
struct RowStats {
    int nv, ns;
    float s1, s2;
};

// Top-k of the row's keys (0 = not a candidate; larger key first).  Every lane of the wave
// must call it (DPP reads neighbours).  Returns the member bits (bit i <-> register i: keys >=
// the separating key vsep_out) when the search separated exactly k keys; tie_out reports rows
// whose k-th and (k+1)-th keys are equal (their bits are not a selection: such rows take the
// canonical path, which orders equal keys by candidate index).  Keys are below 0xffffffff
// (okey of a NaN with an all-ones payload, which no score producer emits).
template <int JJ>
__device__ __forceinline__ uint32_t rowgroup_topk(const uint32_t (&kv)[JJ], int k, const RowStats& rs,
                                                  uint32_t& vsep_out, bool& tie_out) {
    const int nv = rs.nv;
    // state per row: threshold vsep (members: key >= vsep, or > vsep plus ties when tie).
    // Bracket [lo, hi) with clo = count(>= lo) > k > chi = count(>= hi): key 1 (every valid
    // candidate) and the largest key value (none).  lf/hf only steer the interpolation: they
    // start as mean -/+ 8 standard deviations of the sample and become probe values.
    bool done = nv <= k, tie = false;
    uint32_t vsep = 1u, lo = 1u, hi = 0xffffffffu;
    int clo = nv, chi = 0;
    float lf, hf, guess;
    {
        const float rn = __builtin_amdgcn_rcpf((float)(rs.ns > 0 ? rs.ns : 1));
        const float mu = rs.s1 * rn;
        const float sd = __builtin_amdgcn_sqrtf(fmaxf(rs.s2 * rn - mu * mu, 0.0f));
        const float rv = __builtin_amdgcn_rcpf((float)(nv > 0 ? nv : 1));
        guess = mu + z_upper_fast((k + 0.5f) * rv) * sd;
        lf = mu - 8.0f * sd - 1e-30f;
        hf = mu + 8.0f * sd + 1e-30f;
    }
    for (int it = 0; __ballot(!done) != 0; ++it) {
        uint32_t mid = lo + (hi - lo) / 2u;
        float midf = 0.0f;
        if (it < 8) {
            // interpolated probe (only steers the search: approximate reciprocal is enough),
            // kept at least 1/16 of the span inside the bracket and clamped into (lo, hi) in
            // key space
            const float span = hf - lf;
            float x = it == 0 ? guess
                              : lf + span * (float)(clo - k) * __builtin_amdgcn_rcpf((float)(clo - chi));
            x = fminf(fmaxf(x, lf + span * 0.0625f), hf - span * 0.0625f);
            mid = min(max(okey_fast(x), lo + 1u), hi - 1u);
            midf = x;
        } else {
            midf = okey_inv(mid);
        }
        const int c = r16_count_ge<JJ>(kv, mid);
        if (!done) {
            if (c == k) {
                vsep = mid;
                done = true;
            } else {
                if (c > k) {
                    lo = mid;
                    clo = c;
                    lf = midf;
                } else {
                    hi = mid;
                    chi = c;
                    hf = midf;
                }
                if (hi - lo <= 1u) {
                    vsep = lo;
                    tie = true;
                    done = true;
                }
            }
        }
    }
    tie_out = tie;
    vsep_out = vsep;
    uint32_t bits = 0;
#pragma unroll
    for (int i = JJ - 1; i >= 0; --i) bits = 2u * bits + (kv[i] >= vsep ? 1u : 0u);
    return bits;
}

// ------------------------------------------------------------------------------------------
// Compacted selection (k <= kCompactK): one or a few counting probes find a threshold T that
// leaves k < count(key >= T) <= kCap keys in the row; those keys are compacted into a per-row
// LDS buffer (kCap slots + one discard slot) and sorted by a 32-element bitonic network over the
// row's 16 lanes (2 keys per lane, element e = 2*seg + r, DPP partner exchanges); the k-th and
// (k+1)-th largest keys are then read off exactly.  This replaces the full-row search and its
// certification count.  Rows whose probes do not land within a few steps make the whole wave
// fall back to the full-row search.
// ------------------------------------------------------------------------------------------
constexpr int kCap = 32;         // compacted keys per row
constexpr int kCmpStride = 34;   // per-row buffer: kCap slots, a discard slot, 8-byte aligned
constexpr int kCompactK = 16;

// (the permutations used here read a lane of the same DPP row, so no lane is out of bounds)
template <int CTRL>
__device__ __forceinline__ uint32_t dppu(uint32_t x) {
    return (uint32_t)__builtin_amdgcn_mov_dpp((int)x, CTRL, 0xf, 0xf, true);
}
// Compare-exchange of this lane's x with partner value p: the lower element (hi = 0) keeps the
// minimum, the upper one (hi = 0xffffffff) the maximum.  max(min(x, p), min(max(x, p), hi)) is
// the median of {x, p, hi}: one v_med3_u32 instead of a min, a max and a select.
__device__ __forceinline__ uint32_t cx_mask(bool lower) { return lower ? 0u : 0xffffffffu; }
__device__ __forceinline__ uint32_t cx(uint32_t x, uint32_t p, uint32_t hi) {
    return max(min(x, p), min(max(x, p), hi));
}
// Ascending bitonic sort of the 32 keys (a = element 2*seg, b = 2*seg + 1) of each 16-lane
// row: for block sizes 2..32 a flip step (element e against e ^ (size-1), a lane mirror that
// swaps a and b) then half-cleaners e against e ^ j for j = size/4 .. 1.
__device__ __forceinline__ void sort32_row(uint32_t& a, uint32_t& b, int seg) {
    auto inlane = [&]() { const uint32_t lo = min(a, b); b = max(a, b); a = lo; };
    auto flip = [&](auto pa_fn, int lowbit) {
        const uint32_t lw = cx_mask((seg & lowbit) == 0);
        const uint32_t pa = pa_fn(b), pb = pa_fn(a);
        a = cx(a, pa, lw);
        b = cx(b, pb, lw);
    };
    auto half = [&](auto p_fn, int lowbit) {
        const uint32_t lw = cx_mask((seg & lowbit) == 0);
        a = cx(a, p_fn(a), lw);
        b = cx(b, p_fn(b), lw);
    };
    auto x1 = [](uint32_t v) { return dppu<0xB1>(v); };     // lane ^ 1 (quad_perm [1,0,3,2])
    auto x2 = [](uint32_t v) { return dppu<0x4E>(v); };     // lane ^ 2 (quad_perm [2,3,0,1])
    auto m3 = [](uint32_t v) { return dppu<0x1B>(v); };     // lane ^ 3 (quad_perm [3,2,1,0])
    auto m7 = [](uint32_t v) { return dppu<0x141>(v); };    // lane ^ 7 (row_half_mirror)
    auto m15 = [](uint32_t v) { return dppu<0x140>(v); };   // lane ^ 15 (row_mirror)
    auto x4 = [](uint32_t v) {                              // lane ^ 4 (swizzle, xor mask 4)
        return (uint32_t)__builtin_amdgcn_ds_swizzle((int)v, 0x101f);
    };
    inlane();                                                      // size 2
    flip(x1, 1); inlane();                                         // size 4
    flip(m3, 2); half(x1, 1); inlane();                            // size 8
    flip(m7, 4); half(x2, 2); half(x1, 1); inlane();               // size 16
    flip(m15, 8); half(x4, 4); half(x2, 2); half(x1, 1); inlane(); // size 32
}

// Ascending bitonic sort of the 64 keys of each 16-lane row, element e = 4*seg + r held in
// R[r] (the row-group layout of 64 candidates): in-lane steps pair r with r ^ m; cross-lane
// steps pair lane seg with seg ^ mh (DPP / swizzle) and register r with r ^ ml.
template <int M>
__device__ __forceinline__ void sort_inlane4(uint32_t (&R)[4]) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int p = r ^ M;
        if (p > r) {
            const uint32_t lo = min(R[r], R[p]);
            R[p] = max(R[r], R[p]);
            R[r] = lo;
        }
    }
}
template <int ML, class F>
__device__ __forceinline__ void sort_cross4(uint32_t (&R)[4], F perm, uint32_t lower) {
    uint32_t P[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) P[r] = perm(R[r ^ ML]);
#pragma unroll
    for (int r = 0; r < 4; ++r) R[r] = cx(R[r], P[r], lower);
}
__device__ __forceinline__ void sort64_row(uint32_t (&R)[4], int seg) {
    auto x1 = [](uint32_t v) { return dppu<0xB1>(v); };
    auto x2 = [](uint32_t v) { return dppu<0x4E>(v); };
    auto m3 = [](uint32_t v) { return dppu<0x1B>(v); };
    auto m7 = [](uint32_t v) { return dppu<0x141>(v); };
    auto m15 = [](uint32_t v) { return dppu<0x140>(v); };
    auto x4 = [](uint32_t v) { return (uint32_t)__builtin_amdgcn_ds_swizzle((int)v, 0x101f); };
    const uint32_t b1 = cx_mask((seg & 1) == 0), b2 = cx_mask((seg & 2) == 0),
                   b4 = cx_mask((seg & 4) == 0), b8 = cx_mask((seg & 8) == 0);
    sort_inlane4<1>(R);                                                           // size 2
    sort_inlane4<3>(R); sort_inlane4<1>(R);                                       // size 4
    sort_cross4<3>(R, x1, b1); sort_inlane4<2>(R); sort_inlane4<1>(R);            // size 8
    sort_cross4<3>(R, m3, b2); sort_cross4<0>(R, x1, b1);                         // size 16
    sort_inlane4<2>(R); sort_inlane4<1>(R);
    sort_cross4<3>(R, m7, b4); sort_cross4<0>(R, x2, b2); sort_cross4<0>(R, x1, b1); // size 32
    sort_inlane4<2>(R); sort_inlane4<1>(R);
    sort_cross4<3>(R, m15, b8); sort_cross4<0>(R, x4, b4); sort_cross4<0>(R, x2, b2); // size 64
    sort_cross4<0>(R, x1, b1); sort_inlane4<2>(R); sort_inlane4<1>(R);
}

// k-th and (k+1)-th largest keys of each row (k <= kCompactK) by compaction into rowbuf (this
// row's kCmpStride-slot LDS buffer).  Returns false (wave-uniform) when some row of the wave
// found no threshold; the caller then runs the full-row search.  Rows with at most kCap valid
// candidates (including rows with none) compact all of them.
template <int JJ>
__device__ __forceinline__ bool rowgroup_compact(const uint32_t (&kv)[JJ], int k, const RowStats& rs,
                                                 uint32_t* rowbuf, uint32_t& kth, uint32_t& k1th) {
    const int nv = rs.nv, seg = lane_id() & 15;
    bool ok = nv <= kCap;
    uint32_t T = 1u;                  // threshold: keys >= T are compacted (key 0 = no candidate)
    int cl = 0;                       // this lane's keys >= T
    {
        // probes aim at the middle of (k, kCap]: Gaussian quantile of the row's sample first,
        // then regula falsi between the probes on either side, or a Newton step on the
        // Gaussian count density (at most 2 standard deviations) while one side is missing
        const float rn = __builtin_amdgcn_rcpf((float)(rs.ns > 0 ? rs.ns : 1));
        const float mu = rs.s1 * rn;
        const float sd = __builtin_amdgcn_sqrtf(fmaxf(rs.s2 * rn - mu * mu, 0.0f));
        const float rv = __builtin_amdgcn_rcpf((float)(nv > 0 ? nv : 1));
        const float target = 0.5f * (float)(k + 1 + kCap);
        float x = mu + z_upper_fast((target + 0.5f) * rv) * sd;
        float lf = 0.0f, hf = 0.0f;
        int clo = -1, chi = -1;
        for (int it = 0; it < 6 && __ballot(!ok) != 0; ++it) {
            const uint32_t tx = min(max(okey_fast(x), 1u), 0xfffffffeu);
            int c_l = 0;
#pragma unroll
            for (int i = 0; i < JJ; ++i) c_l += kv[i] >= tx ? 1 : 0;
            const int c = r16_sum(c_l);
            if (!ok) {
                if (c > k && c <= kCap) {
                    ok = true;
                    T = tx;
                    cl = c_l;
                } else {
                    if (c > kCap) {
                        lf = x;
                        clo = c;
                    } else {
                        hf = x;
                        chi = c;
                    }
                    if (clo >= 0 && chi >= 0) {
                        x = lf + (hf - lf) * ((float)clo - target) * __builtin_amdgcn_rcpf((float)(clo - chi));
                    } else {
                        const float z = (x - mu) * __builtin_amdgcn_rcpf(sd > 0.0f ? sd : 1.0f);
                        const float dens = (float)nv * 0.39894228f * __expf(-0.5f * z * z) *
                                           __builtin_amdgcn_rcpf(sd > 0.0f ? sd : 1.0f);
                        const float step = ((float)c - target) * __builtin_amdgcn_rcpf(fmaxf(dens, 1e-30f));
                        x += fminf(fmaxf(step, -2.0f * sd), 2.0f * sd);
                    }
                }
            }
        }
    }
    if (__ballot(!ok) != 0) return false;
    if (nv <= kCap) {
        cl = 0;
#pragma unroll
        for (int i = 0; i < JJ; ++i) cl += kv[i] != 0u ? 1 : 0;
    }
    // exclusive prefix of the per-lane counts over the row (row_shr with zero fill)
    int incl = cl;
    incl += dppi<0x111, 0>(incl);
    incl += dppi<0x112, 0>(incl);
    incl += dppi<0x114, 0>(incl);
    incl += dppi<0x118, 0>(incl);
    const int cnt = r16_sum(cl);
    int pos = incl - cl;
#pragma unroll
    for (int i = 0; i < JJ; ++i) {
        const bool in = kv[i] >= T;
        rowbuf[in ? pos : kCap] = kv[i];
        pos += in ? 1 : 0;
    }
    __builtin_amdgcn_wave_barrier();
    const uint2 ab = *reinterpret_cast<const uint2*>(rowbuf + 2 * seg);
    uint32_t a = 2 * seg < cnt ? ab.x : 0u;
    uint32_t b = 2 * seg + 1 < cnt ? ab.y : 0u;
    __builtin_amdgcn_wave_barrier();
    sort32_row(a, b, seg);
    // ascending order: element kCap - k holds the k-th largest key, kCap - k - 1 the next
    const int ek = kCap - k, ek1 = ek - 1;
    kth = r16_umax(seg == (ek >> 1) ? ((ek & 1) ? b : a) : 0u);
    k1th = r16_umax(seg == (ek1 >> 1) ? ((ek1 & 1) ? b : a) : 0u);
    return true;
}

// Row-group requests of block rows [r0, r0+32): lane -> (row rr = 4w + lane/16, seg); row rr's
// candidate values are sS[rr * stride + c] for c < ncand (-inf = not visible when VIS; without
// VIS every candidate is visible).  Certified rows raise the pooled key / lower the first row of
// their members and set their request bits; rows whose k-th and (k+1)-th values lie within
// 2*delta are queued (absolute row) in sAmb for the canonical path.
template <int JJ, bool VIS>
__device__ __forceinline__ void rowgroup_requests(int r0, int brows, int ncand, const float* sS, int stride,
                                  int k, float dsc, const float* sQn, uint32_t* sPk,
                                  int* sFirst, uint32_t* sBits, int BW, int* sAmb, int* sAmbN,
                                  uint32_t* sCmp) {
    constexpr int W = JJ < 4 ? JJ : 4;
    constexpr int G = JJ / W;
    const int w = threadIdx.x / kWave, l = lane_id(), seg = l & 15;
    const int rr = 4 * w + (l >> 4), t = r0 + rr;
    const bool act = rr < brows;
    const float* rowp = sS + rr * stride;
    uint32_t kv[JJ];
    RowStats rs{0, 0, 0.0f, 0.0f};
    int nvl = 0, nsl = 0;
#pragma unroll
    for (int g = 0; g < G; ++g) {
        const int c0 = 16 * W * g + W * seg;
        float x[W];
#pragma unroll
        for (int e = 0; e < W; ++e) x[e] = 0.0f;
        if (16 * W * g < ncand) {                    // wave-uniform; rows are 16-byte aligned
            if constexpr (W == 4) {
                const float4 v4 = *reinterpret_cast<const float4*>(rowp + c0);
                x[0] = v4.x; x[1] = v4.y; x[2] = v4.z; x[3] = v4.w;
            } else if constexpr (W == 2) {
                const float2 v2 = *reinterpret_cast<const float2*>(rowp + c0);
                x[0] = v2.x; x[1] = v2.y;
            } else {
                x[0] = rowp[c0];
            }
        }
        const bool full = 16 * W * (g + 1) <= ncand;  // wave-uniform
        if (full && !VIS) {
#pragma unroll
            for (int e = 0; e < W; ++e) {
                kv[W * g + e] = okey_fast(x[e]);
                if (g == 0) {
                    rs.s1 += x[e];
                    rs.s2 = fmaf(x[e], x[e], rs.s2);
                }
            }
        } else if (16 * W * g < ncand) {
#pragma unroll
            for (int e = 0; e < W; ++e) {
                const bool valid = (full || c0 + e < ncand) && (!VIS || x[e] != -INFINITY);
                kv[W * g + e] = valid ? okey_fast(x[e]) : 0u;
                nvl += valid ? 1 : 0;
                if (g == 0) {
                    const float xm = valid ? x[e] : 0.0f;
                    nsl += valid ? 1 : 0;
                    rs.s1 += xm;
                    rs.s2 = fmaf(xm, xm, rs.s2);
                }
            }
        } else {
#pragma unroll
            for (int e = 0; e < W; ++e) kv[W * g + e] = 0u;
        }
    }
    // valid counts: without VIS every candidate below ncand is valid
    rs.nv = act ? (VIS ? r16_sum(nvl) : ncand) : 0;
    rs.ns = VIS ? r16_sum(nsl) : (ncand < 16 * W ? ncand : 16 * W);
    rs.s1 = r16_fsum(rs.s1);
    rs.s2 = r16_fsum(rs.s2);
    const bool open = act && rs.nv > k;
    bool amb = false;
    uint32_t bits = 0u;
    // exact k-th / (k+1)-th keys -- by compaction and a 32-key sort (k <= kCompactK, with a
    // compaction buffer) or, for rows of at most 64 candidates, by sorting the row's keys in
    // place -- make certification one comparison (members: keys >= the k-th; an equal (k+1)-th
    // is a boundary tie, canonical path); otherwise the full-row search
    bool exact = false;
    uint32_t kth = 0u, k1th = 0u;
    if constexpr (JJ >= 2) {
        if (sCmp != nullptr && k <= kCompactK)
            exact = rowgroup_compact<JJ>(kv, k, rs, sCmp + rr * kCmpStride, kth, k1th);
    }
    if constexpr (JJ == 4) {
        if (!exact && k < 64) {
            uint32_t R[4] = {kv[0], kv[1], kv[2], kv[3]};
            sort64_row(R, seg);
            const int ek = 64 - k, ek1 = ek - 1;   // ascending positions of the k-th, (k+1)-th
            const uint32_t vk = (ek & 3) == 0 ? R[0] : (ek & 3) == 1 ? R[1] : (ek & 3) == 2 ? R[2] : R[3];
            const uint32_t vk1 = (ek1 & 3) == 0 ? R[0] : (ek1 & 3) == 1 ? R[1] : (ek1 & 3) == 2 ? R[2] : R[3];
            kth = r16_umax(seg == (ek >> 2) ? vk : 0u);
            k1th = r16_umax(seg == (ek1 >> 2) ? vk1 : 0u);
            exact = true;
        }
    }
    if (exact) {
        const uint32_t vs = open ? kth : 1u;
#pragma unroll
        for (int i = JJ - 1; i >= 0; --i) bits = 2u * bits + (kv[i] >= vs ? 1u : 0u);
        amb = open && kth == k1th;
        if (open && !amb && dsc > 0.0f) {
            const float delta = dsc * sQn[t];
            amb = !(okey_inv(kth) - 2.0f * delta > okey_inv(k1th));
        }
    }
    if (!exact) {
    uint32_t vsep;
    bool tie;
    bits = rowgroup_topk<JJ>(kv, k, rs, vsep, tie);
    // A tie at the boundary goes to the canonical path (equal keys ordered by candidate index
    // there; with MFMA scores such a row is never certifiable anyway).  Certification: k-th and
    // (k+1)-th values at least 2*delta apart.  Rows with at most k candidates have no (k+1)-th.
    // A row that ended with count(>= vsep) == k is certified when no key lies in
    // [value(vsep) - 2 delta, vsep) (one more count); only rows failing that test get the exact
    // k-th / (k+1)-th comparison.
    amb = open && tie;
    if (dsc > 0.0f) {
        const float delta = act ? dsc * sQn[t] : 0.0f;
        const uint32_t probe = okey_fast(okey_inv(vsep) - 2.0f * delta);
        const int cp = r16_count_ge<JJ>(kv, probe);
        const bool unsure = open && !tie && cp != k;
        if (__ballot(unsure) != 0) {
            uint32_t kk = 0xffffffffu, kk1 = 0u;  // smallest member key, largest non-member key
#pragma unroll
            for (int i = 0; i < JJ; ++i) {
                if (kv[i] == 0u) continue;
                if ((bits >> i) & 1u) kk = min(kk, kv[i]);
                else kk1 = max(kk1, kv[i]);
            }
            kk = r16_umin(kk);
            kk1 = r16_umax(kk1);
            const float ak = kk == 0xffffffffu ? INFINITY : okey_inv(kk);
            const float ak1 = kk1 == 0u ? -INFINITY : okey_inv(kk1);
            if (unsure) amb = ak1 != -INFINITY && !(ak - 2.0f * delta > ak1);
        }
    }
    }
    if (amb) {
        if (seg == 0) sAmb[atomicAdd(sAmbN, 1)] = t;
        return;
    }
    if (!act) return;
    // members only (a lane holds about k/16 of them): pooled key, first row, request bit
    for (uint32_t mb = bits; mb != 0u; mb &= mb - 1u) {
        const int i = __builtin_ctz(mb);
        const int c = 16 * W * (i / W) + W * seg + (i % W);
        atomicMax(&sPk[c], okey(rowp[c]));
        atomicMin(&sFirst[c], t);
        atomicOr(&sBits[t * BW + c / 32], 1u << (c % 32));
    }
}

// Out-of-line entry for the wide variants in stage 1: called, they get the whole register
// budget instead of sharing it with the kernel's live state (fewer spills than inlined).
template <int JJ, bool VIS>
__device__ __noinline__ void rowgroup_requests_call(int r0, int brows, int ncand, const float* sS,
                                                    int stride, int k, float dsc,
                                                    const float* sQn, uint32_t* sPk,
                                                    int* sFirst, uint32_t* sBits, int BW,
                                                    int* sAmb, int* sAmbN, uint32_t* sCmp) {
    rowgroup_requests<JJ, VIS>(r0, brows, ncand, sS, stride, k, dsc, sQn, sPk, sFirst, sBits, BW,
                               sAmb, sAmbN, sCmp);
}

// Calls f(JTag<JJ>) with the smallest JJ in {1, 2, 4, 8, 12, ..., 32} such that 16*JJ >= n
// (n <= 512): rows are at most 64 slots longer than the candidate count.
template <class F>
__device__ __forceinline__ void dispatch_jj(int n, F&& f) {
    if (n <= 16) f(JTag<1>{});
    else if (n <= 32) f(JTag<2>{});
    else if (n <= 64) f(JTag<4>{});
    else if (n <= 128) f(JTag<8>{});
    else if (n <= 192) f(JTag<12>{});
    else if (n <= 256) f(JTag<16>{});
    else if (n <= 320) f(JTag<20>{});
    else if (n <= 384) f(JTag<24>{});
    else if (n <= 448) f(JTag<28>{});
    else f(JTag<32>{});
}

// ------------------------------------------------------------------------------------------
// the kernel
// ------------------------------------------------------------------------------------------
template <int DT, int DH>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(4)))
void route_stage1_kernel(RouteArgs A) {
    typedef typename Elem<DT>::T T;
    extern __shared__ __align__(16) unsigned char smem_raw[];
    const int SP = A.SP, BW = A.BW;
    float* sS = reinterpret_cast<float*>(smem_raw);                 // [32][SP] block scores
    float* sQn = sS + A.SSZ;                                         // [64] query row norms
    uint32_t* sPk = reinterpret_cast<uint32_t*>(sQn + kRows);        // [SPP] pooled key
    int* sFirst = reinterpret_cast<int*>(sPk + A.SPP);               // [SPP]
    uint32_t* sBits = reinterpret_cast<uint32_t*>(sFirst + A.SPP);   // [64][BW]
    int* sSel = reinterpret_cast<int*>(sBits + kRows * BW);          // [kMaxSel] sorted chunk ids
    int* sThr = sSel + kMaxSel;                                      // [kMaxSel]
    int* sScal = sThr + kMaxSel;                                     // [8] scalars
    int* sAmb = sScal + 8;                                           // [kRows] ambiguous rows
    uint32_t* sCmp = reinterpret_cast<uint32_t*>(sAmb + kRows);      // [32][kCmpStride] compaction

    const int N = A.N, C = A.C;
    const int n = N - 1 - (int)(blockIdx.x / (A.B * A.H));          // heavy chunks first
    const int bh = blockIdx.x % (A.B * A.H);
    const int b = bh / A.H, h = bh % A.H, kvh = h / (A.H / A.KVH);
    const int w = threadIdx.x / kWave, l = lane_id();
    int rows = A.S - n * C;
    if (rows > C) rows = C;
    int f_hi, l_lo;
    windows(n, A.kf, A.kl, &f_hi, &l_lo);
    const int P = l_lo > f_hi ? l_lo - f_hi : 0;
    const int64_t o = ((int64_t)b * A.H + h) * N + n;
    const int Kcw = A.Kc > 0 ? A.Kc : 1;
    int32_t* out_sc = A.sel_chunk + o * Kcw;
    int32_t* out_st = A.sel_thr + o * Kcw;

    if (A.Kc == 0 || P == 0) {
        for (int i = threadIdx.x; i < Kcw; i += kThreads) out_sc[i] = out_st[i] = -1;
        if (threadIdx.x == 0) A.n_sel[o] = 0;
        return;
    }
    const bool use_mfma = (DT == HGA_DTYPE_BF16) && !A.canonical;
    const float scale = A.scale;
    int amb1 = 0, amb1p = 0;
    const T* qg = reinterpret_cast<const T*>(A.q) + b * A.q_sb + h * A.q_sh + (int64_t)n * C * A.q_ss;
    const T* ckb = reinterpret_cast<const T*>(A.ck) + b * A.ck_sb + kvh * A.ck_sh;
    auto crow = [&](int i) -> const T* { return ckb + (int64_t)(f_hi + i) * DH; };
    auto canonG1 = [&](int t, int i) { return canon_dot<DT, DH>(qg + t * A.q_ss, crow(i), scale); };

    for (int i = threadIdx.x; i < A.SPP; i += kThreads) {
        sPk[i] = 0u;
        sFirst[i] = kNoRow;
    }
    for (int i = threadIdx.x; i < kRows * BW; i += kThreads) sBits[i] = 0u;
    if (threadIdx.x < 8) sScal[threadIdx.x] = 0;
    __syncthreads();

    // ---- stage 1, per 32-row block -----------------------------------------------------------
    for (int r0 = 0; r0 < rows; r0 += kBlk) {
        const int brows = rows - r0 < kBlk ? rows - r0 : kBlk;
        bool scored = false;
        if constexpr (DT == HGA_DTYPE_BF16) {
            if (use_mfma) {
                scores_st<DH, kWaves, false>(reinterpret_cast<const uint16_t*>(qg + (int64_t)r0 * A.q_ss),
                                             A.q_ss, brows, 1, P,
                                             [&](int i) { return reinterpret_cast<const uint16_t*>(crow(i)); },
                                             nullptr, sS, SP, scale,
                                             r0 == 0 ? reinterpret_cast<uint32_t*>(&sScal[1]) : nullptr,
                                             sQn + r0);
                scored = true;
            }
        }
        if (!scored) {
            for (int idx = threadIdx.x; idx < brows * P; idx += kThreads)
                sS[(idx / P) * SP + idx % P] = canonG1(r0 + idx / P, idx % P);
            if (threadIdx.x < kBlk) sQn[r0 + threadIdx.x] = 0.0f;   // no certification
        }
        if (threadIdx.x == 0) sScal[4] = 0;
        __syncthreads();
        const float ds1 = use_mfma ? kDeltaRel * __uint_as_float((uint32_t)sScal[1]) * scale * 1.01f : 0.0f;
        const int kreq = A.Kc < P ? A.Kc : P;
        dispatch_jj(P, [&](auto jt) {
            constexpr int JJ = decltype(jt)::value;
            if constexpr (JJ >= 8)
                rowgroup_requests_call<JJ, false>(r0, brows, P, sS, SP, kreq, ds1, sQn, sPk,
                                                  sFirst, sBits, BW, sAmb, &sScal[4], sCmp);
            else
                rowgroup_requests<JJ, false>(r0, brows, P, sS, SP, kreq, ds1, sQn, sPk, sFirst,
                                             sBits, BW, sAmb, &sScal[4], sCmp);
        });
        __syncthreads();
        // rows the MFMA scores could not certify: canonical re-rank (one row per wave)
        const int namb = sScal[4];
        if (namb > 0) {
            dispatch_j(P, [&](auto jt) {
                constexpr int J = decltype(jt)::value;
                for (int a = w; a < namb; a += kWaves) {
                    const int t = sAmb[a], r = t - r0;
                    float v[J];
#pragma unroll
                    for (int j = 0; j < J; ++j) {
                        const int i = l + 64 * j;
                        v[j] = i < P ? sS[r * SP + i] : -INFINITY;
                    }
                    row_request<J>(t, v, kreq, ds1 * sQn[t], [&](int i) { return canonG1(t, i); },
                                   sPk, sFirst, sBits, BW, &amb1);
                }
            });
        }
        __syncthreads();
    }
    float qnmax = 0.0f;
    {
        float x = 0.0f;
        if (l < rows) x = sQn[l];
        qnmax = wmax(x);
    }

    // ---- stage 1 pooled selection + forced previous chunk (wave 0) -------------------------
    if (w == 0) {
        const float dpool = use_mfma ? kDeltaRel * __uint_as_float((uint32_t)sScal[1]) * qnmax * scale * 1.01f : 0.0f;
        const int prev = n - 1;
        const int ip = (n > 0 && prev >= f_hi && prev < l_lo) ? prev - f_hi : -1;
        int cnt = 0;
        dispatch_j(P, [&](auto jt) {
            constexpr int J = decltype(jt)::value;
            cnt = pooled_select<J>(P, A.Kc, rows, sBits, BW, sPk, sFirst, dpool, canonG1, ip,
                                   f_hi, sSel, sThr, &amb1p);
        });
        if (l == 0) sScal[0] = cnt;
    }
    __syncthreads();
    const int nsel = sScal[0];
    for (int i = threadIdx.x; i < Kcw; i += kThreads) {
        out_sc[i] = i < nsel ? sSel[i] : -1;
        out_st[i] = i < nsel ? sThr[i] : -1;
    }
    if (threadIdx.x == 0) A.n_sel[o] = nsel;

    if (A.stats && l == 0) {
        if (amb1) atomicAdd(&A.stats[0], amb1);
        if (amb1p) atomicAdd(&A.stats[1], amb1p);
    }
}


// ------------------------------------------------------------------------------------------
// stage 2: groups of the selected chunks, all rows of a query chunk (4 waves)
// ------------------------------------------------------------------------------------------
constexpr int kThreads2 = 256;
constexpr int kWaves2 = kThreads2 / kWave;

template <int DT, int DH>
__global__ __launch_bounds__(kThreads2) __attribute__((amdgpu_waves_per_eu(4)))
void route_stage2_kernel(RouteArgs A) {
    typedef typename Elem<DT>::T T;
    extern __shared__ __align__(16) unsigned char smem_raw[];
    const int SP2 = A.SP2, BW = A.BW2;
    float* sS = reinterpret_cast<float*>(smem_raw);                 // [64][SP2] scores
    float* sQn = sS + kRows * SP2;                                   // [64] query row norms
    int* sVthr = reinterpret_cast<int*>(sQn + kRows);                // [VT2] candidate -> first row
    uint32_t* sPk = reinterpret_cast<uint32_t*>(sVthr + A.VT2);      // [SPP2] pooled key
    int* sFirst = reinterpret_cast<int*>(sPk + A.SPP2);              // [SPP2]
    uint32_t* sBits = reinterpret_cast<uint32_t*>(sFirst + A.SPP2);  // [64][BW2]
    int* sSel = reinterpret_cast<int*>(sBits + kRows * BW);          // [kMaxSel]
    int* sThr = sSel + kMaxSel;                                      // [kMaxSel]
    int* sScal = sThr + kMaxSel;                                     // [8]
    int* sAmb = sScal + 8;                                           // [kRows]

    const int N = A.N, C = A.C, M = A.M;
    const int n = N - 1 - (int)(blockIdx.x / (A.B * A.H));          // heavy chunks first
    const int bh = blockIdx.x % (A.B * A.H);
    const int b = bh / A.H, h = bh % A.H, kvh = h / (A.H / A.KVH);
    const int w = threadIdx.x / kWave, l = lane_id();
    int rows = A.S - n * C;
    if (rows > C) rows = C;
    const int64_t o = ((int64_t)b * A.H + h) * N + n;
    const int Kcw = A.Kc > 0 ? A.Kc : 1, Kgw = A.Kg > 0 ? A.Kg : 1;
    int32_t* out_og = A.open_grp + o * Kgw;
    int32_t* out_ot = A.open_thr + o * Kgw;
    const int nsel = A.Kc > 0 ? A.n_sel[o] : 0;
    if (A.Kg == 0 || A.Kgr == 0 || nsel == 0) {
        for (int i = threadIdx.x; i < Kgw; i += kThreads2) out_og[i] = out_ot[i] = -1;
        if (threadIdx.x == 0) A.n_open[o] = 0;
        return;
    }
    const bool use_mfma = (DT == HGA_DTYPE_BF16) && !A.canonical;
    const float scale = A.scale;
    int amb2 = 0, amb2p = 0;
    const T* qg = reinterpret_cast<const T*>(A.q) + b * A.q_sb + h * A.q_sh + (int64_t)n * C * A.q_ss;
    const T* gkb = reinterpret_cast<const T*>(A.gk) + b * A.gk_sb + kvh * A.gk_sh;
    const int T2 = nsel * M;
    for (int i = threadIdx.x; i < nsel; i += kThreads2) {
        sSel[i] = A.sel_chunk[o * Kcw + i];
        sThr[i] = A.sel_thr[o * Kcw + i];
    }
    for (int i = threadIdx.x; i < A.SPP2; i += kThreads2) {
        sPk[i] = 0u;
        sFirst[i] = kNoRow;
    }
    for (int i = threadIdx.x; i < kRows * BW; i += kThreads2) sBits[i] = 0u;
    if (threadIdx.x < 8) sScal[threadIdx.x] = 0;
    for (int i = threadIdx.x; i < A.VT2; i += kThreads2)   // a group is visible from its parent's row
        sVthr[i] = i < T2 ? A.sel_thr[o * Kcw + i / M] : kNoRow;
    __syncthreads();
    auto grow = [&](int i) -> const T* {
        return gkb + ((int64_t)sSel[i / M] * M + (i % M)) * DH;
    };
    auto canonG2 = [&](int t, int i) { return canon_dot<DT, DH>(qg + t * A.q_ss, grow(i), scale); };
    bool scored = false;
    if constexpr (DT == HGA_DTYPE_BF16) {
        if (use_mfma) {
            scores_st<DH, kWaves2, true>(reinterpret_cast<const uint16_t*>(qg), A.q_ss, rows,
                                         (rows + 31) / 32, T2,
                                         [&](int i) { return reinterpret_cast<const uint16_t*>(grow(i)); },
                                         sVthr, sS, SP2, scale, reinterpret_cast<uint32_t*>(&sScal[2]),
                                         sQn);
            scored = true;
        }
    }
    if (!scored) {
        for (int idx = threadIdx.x; idx < rows * T2; idx += kThreads2) {
            const int t = idx / T2, i = idx % T2;
            sS[t * SP2 + i] = sVthr[i] <= t ? canonG2(t, i) : -INFINITY;
        }
        if (threadIdx.x < kRows) sQn[threadIdx.x] = 0.0f;   // no certification
    }
    __syncthreads();
    float qnmax = 0.0f;
    {
        float x = 0.0f;
        if (l < rows) x = sQn[l];
        qnmax = wmax(x);
    }
    const float ds2 = use_mfma ? kDeltaRel * __uint_as_float((uint32_t)sScal[2]) * scale * 1.01f : 0.0f;
    // four waves x four rows per pass
    for (int r0 = 0; r0 < rows; r0 += 4 * kWaves2) {
        const int brows = rows - r0 < 4 * kWaves2 ? rows - r0 : 4 * kWaves2;
        dispatch_jj(T2, [&](auto jt) {
            constexpr int JJ = decltype(jt)::value;
            rowgroup_requests<JJ, true>(r0, brows, T2, sS + r0 * SP2, SP2, A.Kgr, ds2, sQn,
                                        sPk, sFirst, sBits, BW, sAmb, &sScal[4], nullptr);
        });
    }
    __syncthreads();
    const int namb = sScal[4];
    if (namb > 0) {
        dispatch_j(T2, [&](auto jt) {
            constexpr int J = decltype(jt)::value;
            for (int a = w; a < namb; a += kWaves2) {
                const int t = sAmb[a];
                float v[J];
#pragma unroll
                for (int j = 0; j < J; ++j) {
                    const int i = l + 64 * j;
                    v[j] = (i < T2 && sThr[i / M] <= t) ? sS[t * SP2 + i] : -INFINITY;
                }
                row_request<J>(t, v, A.Kgr, ds2 * sQn[t], [&](int i) { return canonG2(t, i); },
                               sPk, sFirst, sBits, BW, &amb2);
            }
        });
    }
    __syncthreads();
    if (w == 0) {
        const float dpool2 = ds2 * qnmax;
        int cnt = 0;
        dispatch_j(T2, [&](auto jt) {
            constexpr int J = decltype(jt)::value;
            float v[J];
#pragma unroll
            for (int j = 0; j < J; ++j) {
                const int i = l + 64 * j;
                v[j] = (i < T2 && sFirst[i] < kNoRow) ? okey_inv(sPk[i]) : -INFINITY;
            }
            auto canon_pool2 = [&](int i) { return pooled_exact(i, rows, sBits, BW, canonG2); };
            const uint32_t op = select_certified<J>(v, A.Kg, dpool2, canon_pool2, &amb2p);
            int base = 0;
#pragma unroll
            for (int j = 0; j < J; ++j) {
                const bool m = (op >> j) & 1u;
                const uint64_t bal = __ballot(m);
                if (m) {
                    const int i = l + 64 * j;
                    const int pos = base + lanes_below(bal);
                    if (pos < Kgw) {
                        out_og[pos] = sSel[i / M] * M + (i % M);
                        out_ot[pos] = sFirst[i];
                    }
                }
                base += __popcll(bal);
            }
            cnt = base;
        });
        for (int i = cnt + l; i < Kgw; i += kWave) out_og[i] = out_ot[i] = -1;
        if (l == 0) A.n_open[o] = cnt;
    }
    if (A.stats && l == 0) {
        if (amb2) atomicAdd(&A.stats[2], amb2);
        if (amb2p) atomicAdd(&A.stats[3], amb2p);
    }
}

// ==========================================================================================
// Fused router (bf16 MFMA path): stage 1 and stage 2 of one (b, h, query chunk) in one
// workgroup of four waves.  Wave w owns query rows 16w..16w+15 in both stages; its rows' scores
// never leave registers: S^T = K * Q^T by v_mfma_f32_16x16x32_bf16 puts query row l % 16 in lane
// l, with candidates 16*tau + 4*(l/16) + i (i < 4) of candidate tile tau, so the four lanes
// l % 16 + 16*qd of a row hold a quarter of its scores each.  The query rows stay in registers
// as the B operand for both stages (q is read once).
//
// Stage 1, per segment of up to 256 pool candidates: counting probes (a Gaussian quantile of a
// sample of the row, then regula falsi / Newton steps; counts summed over the row's four lanes)
// find a key threshold T with k < count(key >= T) <= 32; those keys and their candidate ids are
// appended to the row's LDS survivor list.  The survivors hold the row's top-(k+1) (each
// segment's top-(k+1) survives), so sorting them (32-key or 64-key bitonic network over the 16
// lanes of a DPP row) gives the exact k-th and (k+1)-th MFMA keys; certification and the
// canonical re-rank of uncertain rows are as in the split kernels, except that an uncertain row
// is rescored canonically in full.  Pooling, the pooled selection and stage 2 follow the split
// kernels' rules.
//
// Pools of more than 512 chunks (the LONG variant, launched for those query chunks only) take
// more segments; between segments a row list longer than 32 is cut back to its entries with
// key >= x, x its 32nd largest key (its (k+1)-th where ties at the 32nd would keep more), so
// the list still holds every candidate with key >= the largest threshold applied to the row,
// and at least k + 1 of them.
// ==========================================================================================
constexpr int kFThreads = 256;
constexpr int kFWaves = kFThreads / kWave;
constexpr int kSegTiles = 16;             // 16-candidate tiles per stage-1 segment
constexpr int kSegCand = 16 * kSegTiles;  // 256
constexpr int kSurv = 32;                 // survivors per row and segment
constexpr int kSvStride = 66;             // survivor list slots per row: 2 x 32, padded (bank spread)
constexpr int kFusedMaxPool = 2 * kSegCand;       // pools of the ordinary variant
constexpr int kFusedMaxPoolLong = 8 * kSegCand;   // pools of the LONG variant (2048 chunks)
constexpr int kFusedMaxT2 = 64;
constexpr int kFStageRows = 32;           // candidate rows per stage-1 LDS stage (two stages)

typedef float floatx4 __attribute__((ext_vector_type(4)));

// sums / maxima over the four lanes of a row (l % 16 + 16 * qd); butterflies, so all four
// lanes end bit-identical
__device__ __forceinline__ int q4_sum(int x) {
    x += __shfl_xor(x, 16, kWave);
    return x + __shfl_xor(x, 32, kWave);
}
__device__ __forceinline__ float q4_fsum(float x) {
    x += __shfl_xor(x, 16, kWave);
    return x + __shfl_xor(x, 32, kWave);
}

// Direct global->LDS copy of 16 bytes per lane: lane i's bytes at sbase + voff land at LDS byte
// address lds_addr + 16 i (lds_addr wave-uniform).  Inline assembly, so the compiler inserts no
// waits for it; the kernel waits (s_waitcnt 0) before the barrier that publishes a stage.  M0
// holds the LDS address; nothing else in this kernel uses M0.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void route_lds_copy16(const void* sbase, uint32_t voff, uint32_t lds_addr) {
    // base and LDS address are wave-uniform: make them scalar operands
    const uint64_t b64 = (uint64_t)(uintptr_t)sbase;
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)b64);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(b64 >> 32));
    const void* sb = (const void*)(uintptr_t)(((uint64_t)hi << 32) | lo);
    const uint32_t la = __builtin_amdgcn_readfirstlane(lds_addr);
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2"
                 :: "s"(la), "v"(voff), "s"(sb) : "memory", "m0");
}
#pragma clang diagnostic pop

// A stage holds ROWS (32 or 64) candidate rows (DH bf16 each, row-major) with the 16-byte pieces
// of row r XOR-swizzled: piece j at slot j ^ (r % PPR), so the 16 rows of a tile read the same
// piece from different banks.  Wave w copies rows RPW w .. RPW w + RPW - 1 (RPW = ROWS / 4): row
// r (< nrows) from sbase + off(r) bytes.
template <int DH, int ROWS, class Off>
__device__ __forceinline__ void stage_rows(const void* sbase, Off off, int nrows, uint32_t stage,
                                           int w) {
    constexpr int PPR = DH / 8;          // 16-byte pieces per row
    constexpr int RPI = 64 / PPR;        // rows per wave instruction
    constexpr int RPW = ROWS / 4;        // rows per wave
    static_assert(RPW % RPI == 0, "a wave copies whole instructions' worth of rows");
    const int l = lane_id();
#pragma unroll
    for (int r = 0; r < RPW / RPI; ++r) {
        const int row = RPW * w + RPI * r + l / PPR;
        const int j = (l % PPR) ^ (row % PPR);
        if (row < nrows)
            route_lds_copy16(sbase, off(row) + 16u * (uint32_t)j,
                             stage + (uint32_t)((RPW * w + RPI * r) * DH * 2));
    }
}

template <int DH>
__device__ __forceinline__ floatx4 tile_mfma(const uint4 (&a)[DH / 32], const bf16x8 (&qb)[DH / 32]) {
    floatx4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int ks = 0; ks < DH / 32; ++ks)
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(a[ks]), qb[ks], acc, 0, 0, 0);
    return acc;
}
template <int DH>
__device__ __forceinline__ float tile_knorm(const uint4 (&a)[DH / 32]) {
    float x = 0.0f;
#pragma unroll
    for (int ks = 0; ks < DH / 32; ++ks) x += sumsq_bf16x8(a[ks]);
    return __builtin_sqrtf(q4_fsum(x));
}

// Scores of the wave's rows against the NT tiles (16 NT candidates c0 + 16 u + ..) of a stage as
// order-preserving keys kv[4 tau + i], tau = tau0 + u (0: candidate >= ncand).  A operands from
// the stage: lane l reads candidate row 16 u + l % 16, dims 32 ks + 8 (l / 16).  Updates knmax
// with the norms of the tiles with tau % nw == w (the nw active waves see the same candidates:
// their maximum covers all) and the sample statistics (s1, s2, ns) of tiles 0..3.
template <int DH, int NK, int NT>
__device__ __forceinline__ void stage_scores(const unsigned char* stage, int tau0, int c0, int ncand,
                                             int w, int nw, const bf16x8 (&qb)[DH / 32], float scale,
                                             uint32_t (&kv)[NK], float& knmax, float& s1, float& s2,
                                             int& ns) {
    constexpr int PPR = DH / 8;
    const int l = lane_id(), r16 = l % 16, qd = l / 16;
#pragma unroll
    for (int u = 0; u < NT; ++u) {
        const int tau = tau0 + u;
        if (tau >= NK / 4) break;
        const int row = 16 * u + r16;
        uint4 a[DH / 32];
#pragma unroll
        for (int ks = 0; ks < DH / 32; ++ks) {
            const int j = (4 * ks + qd) ^ (row % PPR);
            a[ks] = *reinterpret_cast<const uint4*>(stage + row * (DH * 2) + 16 * j);
        }
        const floatx4 acc = tile_mfma<DH>(a, qb);
        const int cbase = c0 + 16 * u;
        if (tau % nw == w) {                      // wave-uniform
            const float kn = tile_knorm<DH>(a);
            if (cbase + r16 < ncand) knmax = fmaxf(knmax, kn);
        }
        const int cb = cbase + 4 * qd;
        const bool full = cbase + 16 <= ncand;    // wave-uniform
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float sc = fmaf(acc[i], scale, 0.0f);
            const bool valid = full || cb + i < ncand;
            kv[4 * tau + i] = valid ? okey_fast(sc) : 0u;
            if (tau < 4 && valid) {
                s1 += sc;
                s2 = fmaf(sc, sc, s2);
                ns += 1;
            }
        }
    }
}

// Threshold probes for the rows of a wave (four lanes per row): on success T leaves
// k < count(key >= T) <= kSurv keys in the row (rows with at most kSurv valid keys take T = 1:
// all of them).  Returns false for rows (open ones only) where no threshold was found.
template <int NK>
__device__ __forceinline__ bool fused_probe(const uint32_t (&kv)[NK], int nk, bool open, int nv,
                                            int k, float s1, float s2, int ns, uint32_t& T) {
    bool ok = !open || nv <= kSurv;
    T = 1u;
    const float rn = __builtin_amdgcn_rcpf((float)(ns > 0 ? ns : 1));
    const float mu = s1 * rn;
    const float sd = __builtin_amdgcn_sqrtf(fmaxf(s2 * rn - mu * mu, 0.0f));
    const float rv = __builtin_amdgcn_rcpf((float)(nv > 0 ? nv : 1));
    const float target = 0.5f * (float)(k + 1 + kSurv);
    float x = mu + z_upper_fast((target + 0.5f) * rv) * sd;
    float lf = 0.0f, hf = 0.0f;
    int clo = -1, chi = -1;
    for (int it = 0; it < 6 && __ballot(!ok) != 0; ++it) {
        const uint32_t tx = min(max(okey_fast(x), 1u), 0xfffffffeu);
        int cl = 0;
#pragma unroll
        for (int g = 0; g < NK / 16; ++g)
            if (16 * g < nk) {                             // wave-uniform
#pragma unroll
                for (int i = 16 * g; i < 16 * g + 16; ++i) cl += kv[i] >= tx ? 1 : 0;
            }
        const int c = q4_sum(cl);
        if (!ok) {
            if (c > k && c <= kSurv) {
                ok = true;
                T = tx;
            } else {
                if (c > kSurv) {
                    lf = x;
                    clo = c;
                } else {
                    hf = x;
                    chi = c;
                }
                if (clo >= 0 && chi >= 0) {
                    x = lf + (hf - lf) * ((float)clo - target) * __builtin_amdgcn_rcpf((float)(clo - chi));
                } else {
                    const float z = (x - mu) * __builtin_amdgcn_rcpf(sd > 0.0f ? sd : 1.0f);
                    const float dens = (float)nv * 0.39894228f * __expf(-0.5f * z * z) *
                                       __builtin_amdgcn_rcpf(sd > 0.0f ? sd : 1.0f);
                    const float step = ((float)c - target) * __builtin_amdgcn_rcpf(fmaxf(dens, 1e-30f));
                    x += fminf(fmaxf(step, -2.0f * sd), 2.0f * sd);
                }
            }
        }
    }
    return ok;
}

// Appends this lane's keys >= T (and their candidate ids id0 + 16 * (i / 4) + 4 * qd + i % 4) to
// the row's survivor list at base; returns the row's new survivor count (all four lanes).
template <int NK>
__device__ __forceinline__ int fused_compact(const uint32_t (&kv)[NK], int nk, uint32_t T, int id0,
                                             uint2* rowbuf, int base, bool on) {
    const int qd = lane_id() / 16;
    int cl = 0;
#pragma unroll
    for (int g = 0; g < NK / 16; ++g)
        if (16 * g < nk) {
#pragma unroll
            for (int i = 16 * g; i < 16 * g + 16; ++i) cl += (on && kv[i] >= T) ? 1 : 0;
        }
    // exclusive prefix over the row's lanes qd = 0..3
    const int x16 = __shfl_xor(cl, 16, kWave);
    const int pair = cl + x16;
    const int x32 = __shfl_xor(pair, 32, kWave);
    int pos = base + ((qd & 1) ? x16 : 0) + ((qd & 2) ? x32 : 0);
    // the counts above must not keep 64 compare results alive: recompute them below
    asm volatile("" : "+v"(T));
#pragma unroll
    for (int g = 0; g < NK / 16; ++g)
        if (16 * g < nk) {
#pragma unroll
            for (int i = 16 * g; i < 16 * g + 16; ++i) {
                const bool in = on && kv[i] >= T;
                if (in) rowbuf[pos] = make_uint2(kv[i], (uint32_t)(id0 + 16 * (i / 4) + 4 * qd + (i % 4)));
                pos += in ? 1 : 0;
            }
        }
    return base + pair + x32;
}

// Ascending bitonic sort of the (up to) 64 keys of each query row in the MFMA layout: a row's
// keys are held by its four lanes l % 16 + 16 qd, element e = 16 qd + i in S[i] (zeros sort
// first).  In-lane steps for block sizes 2..16, then the size-32 flip against the lane
// l ^ 16 (element e ^ 31), the size-64 flip against l ^ 48 (element e ^ 63) and its
// half-cleaner against l ^ 16 (element e ^ 16); the remaining half-cleaners are in-lane.  All 16
// rows of a wave sort at once, with no LDS round trip.
__device__ __forceinline__ void q4_ce(uint32_t& a, uint32_t& b) {
    const uint32_t lo = min(a, b);
    b = max(a, b);
    a = lo;
}
template <int M>
__device__ __forceinline__ void q4_inlane(uint32_t (&S)[16]) {
#pragma unroll
    for (int i = 0; i < 16; ++i)
        if ((i ^ M) > i) q4_ce(S[i], S[i ^ M]);
}
__device__ __forceinline__ uint32_t q4_x16(uint32_t v) {   // lane ^ 16 (swizzle, xor mask 16)
    return (uint32_t)__builtin_amdgcn_ds_swizzle((int)v, 0x401f);
}
__device__ __forceinline__ void sort64_q4(uint32_t (&S)[16], int qd) {
    q4_inlane<1>(S);                                                        // size 2
    q4_inlane<3>(S); q4_inlane<1>(S);                                       // size 4
    q4_inlane<7>(S); q4_inlane<2>(S); q4_inlane<1>(S);                      // size 8
    q4_inlane<15>(S); q4_inlane<4>(S); q4_inlane<2>(S); q4_inlane<1>(S);    // size 16
    uint32_t P[16];
    {   // size 32: e against e ^ 31 (lane ^ 16, register 15 - i); lanes with even qd keep the minimum
        const uint32_t lower = cx_mask((qd & 1) == 0);
#pragma unroll
        for (int i = 0; i < 16; ++i) P[i] = q4_x16(S[15 - i]);
#pragma unroll
        for (int i = 0; i < 16; ++i) S[i] = cx(S[i], P[i], lower);
        q4_inlane<8>(S); q4_inlane<4>(S); q4_inlane<2>(S); q4_inlane<1>(S);
    }
    {   // size 64: e against e ^ 63 (lane ^ 48, register 15 - i), then e ^ 16 (lane ^ 16)
        const uint32_t lower = cx_mask(qd < 2);
#pragma unroll
        for (int i = 0; i < 16; ++i) P[i] = (uint32_t)__shfl_xor((int)S[15 - i], 48, kWave);
#pragma unroll
        for (int i = 0; i < 16; ++i) S[i] = cx(S[i], P[i], lower);
        const uint32_t lower2 = cx_mask((qd & 1) == 0);
#pragma unroll
        for (int i = 0; i < 16; ++i) P[i] = q4_x16(S[i]);
#pragma unroll
        for (int i = 0; i < 16; ++i) S[i] = cx(S[i], P[i], lower2);
        q4_inlane<8>(S); q4_inlane<4>(S); q4_inlane<2>(S); q4_inlane<1>(S);
    }
}
// The 32nd and 33rd largest of the 64 keys of each row (the split at the middle, on all four
// lanes of the row), without the rest of the sort: the two 32-key halves are sorted (as in
// sort64_q4), and the first size-64 step leaves the 32 largest keys on lanes qd >= 2 and the 32
// smallest on lanes qd < 2, so the 32nd largest is the minimum of the upper lanes and the 33rd the
// maximum of the lower ones.
__device__ __forceinline__ void split64_q4(uint32_t (&S)[16], int qd, uint32_t& k32, uint32_t& k33) {
    q4_inlane<1>(S);
    q4_inlane<3>(S); q4_inlane<1>(S);
    q4_inlane<7>(S); q4_inlane<2>(S); q4_inlane<1>(S);
    q4_inlane<15>(S); q4_inlane<4>(S); q4_inlane<2>(S); q4_inlane<1>(S);
    uint32_t P[16];
    {
        const uint32_t lower = cx_mask((qd & 1) == 0);
#pragma unroll
        for (int i = 0; i < 16; ++i) P[i] = q4_x16(S[15 - i]);
#pragma unroll
        for (int i = 0; i < 16; ++i) S[i] = cx(S[i], P[i], lower);
        q4_inlane<8>(S); q4_inlane<4>(S); q4_inlane<2>(S); q4_inlane<1>(S);
    }
    const uint32_t lower = cx_mask(qd < 2);
#pragma unroll
    for (int i = 0; i < 16; ++i) P[i] = (uint32_t)__shfl_xor((int)S[15 - i], 48, kWave);
#pragma unroll
    for (int i = 0; i < 16; ++i) S[i] = cx(S[i], P[i], lower);
    uint32_t mn = S[0], mx = S[0];
#pragma unroll
    for (int i = 1; i < 16; ++i) {
        mn = min(mn, S[i]);
        mx = max(mx, S[i]);
    }
    mn = min(mn, q4_x16(mn));                       // lanes qd >= 2: the 32nd largest
    mx = max(mx, q4_x16(mx));                       // lanes qd < 2: the 33rd largest
    const uint32_t mn_o = (uint32_t)__shfl_xor((int)mn, 32, kWave);
    const uint32_t mx_o = (uint32_t)__shfl_xor((int)mx, 32, kWave);
    k32 = qd >= 2 ? mn : mn_o;
    k33 = qd < 2 ? mx : mx_o;
}
// Element pos (0..63, uniform) of each row after sort64_q4, on all four lanes of the row.
__device__ __forceinline__ uint32_t q4_pick(const uint32_t (&S)[16], int pos, int qd) {
    uint32_t v = 0u;
#pragma unroll
    for (int r = 0; r < 16; ++r) v = (r == (pos & 15) && qd == (pos >> 4)) ? S[r] : v;
    v = max(v, q4_x16(v));
    return max(v, (uint32_t)__shfl_xor((int)v, 32, kWave));
}

__device__ __forceinline__ void fused_request(int t, int id, uint32_t key, uint32_t* sPk,
                                              int* sFirst, uint32_t* sBits, int BW) {
    atomicMax(&sPk[id], key);
    atomicMin(&sFirst[id], t);
    atomicOr(&sBits[t * BW + id / 32], 1u << (id % 32));
}

// Exact k-th and (k+1)-th largest keys of a row list (ns <= 16 * SW entries at rowbuf): DPP row
// d (lanes 16d..16d+15) sorts one row with a 32-key (SW = 2) or 64-key (SW = 4) bitonic network.
// Returns the lane's SW entries (zero keys past ns).
template <int SW>
__device__ __forceinline__ void list_kth(const uint2* rowbuf, int ns, int k, uint32_t& kth,
                                         uint32_t& k1th, uint2 (&e)[SW]) {
    const int seg = lane_id() & 15;
#pragma unroll
    for (int r = 0; r < SW; ++r) {
        const int x = SW * seg + r;
        e[r] = x < ns ? rowbuf[x] : make_uint2(0u, 0u);
    }
    if constexpr (SW == 2) {
        uint32_t a = e[0].x, b = e[1].x;
        sort32_row(a, b, seg);
        const int ek = 32 - k, ek1 = ek - 1;
        kth = r16_umax(seg == (ek >> 1) ? ((ek & 1) ? b : a) : 0u);
        k1th = r16_umax(seg == (ek1 >> 1) ? ((ek1 & 1) ? b : a) : 0u);
    } else {
        uint32_t R[4] = {e[0].x, e[1].x, e[2].x, e[3].x};
        sort64_row(R, seg);
        const int ek = 64 - k, ek1 = ek - 1;
        const uint32_t vk = (ek & 3) == 0 ? R[0] : (ek & 3) == 1 ? R[1] : (ek & 3) == 2 ? R[2] : R[3];
        const uint32_t vk1 = (ek1 & 3) == 0 ? R[0] : (ek1 & 3) == 1 ? R[1] : (ek1 & 3) == 2 ? R[2] : R[3];
        kth = r16_umax(seg == (ek >> 2) ? vk : 0u);
        k1th = r16_umax(seg == (ek1 >> 2) ? vk1 : 0u);
    }
}

// Selections of the wave's 16 rows from their lists (stage 1: survivor lists; stage 2: the full
// candidate lists), four rows per pass: certified rows request their members; uncertain rows are
// queued in sAmb with their re-rank band key in sBand (0: rescore every candidate).
// sRowN[t]: list length, -1 no selection work (inactive, or everything valid was requested
// already), -2 probes failed (uncertain, full rescoring).  sRowT[t] (stage 1, else nullptr): the
// largest compaction threshold of the row's segments.
template <int SW>
__device__ __forceinline__ void list_rows(int w, int k, float dsc, const float* sQn, const uint2* sSv,
                                          const int* sRowN, const uint32_t* sRowT, uint32_t* sPk,
                                          int* sFirst, uint32_t* sBits, int BW, int* sAmb,
                                          int* sAmbN, uint32_t* sBand) {
    const int l = lane_id(), seg = l & 15;
    for (int p = 0; p < 4; ++p) {
        const int t = 16 * w + 4 * p + l / 16;
        const int ns = sRowN[t];
        uint32_t kth = 0u, k1th = 0u;
        uint2 e[SW];
        list_kth<SW>(sSv + t * kSvStride, ns < 0 ? 0 : ns, k, kth, k1th, e);
        if (ns == -1) continue;
        const float delta = dsc * sQn[t];
        const bool amb = ns == -2 || kth == k1th || !(okey_inv(kth) - 2.0f * delta > okey_inv(k1th));
        if (amb) {
            if (seg == 0) {
                const uint32_t band = okey_fast(okey_inv(kth) - 2.0f * delta);
                sBand[t] = (ns == -2 || !sRowT || band < sRowT[t]) ? 0u : (band > 1u ? band : 1u);
                sAmb[atomicAdd(sAmbN, 1)] = t;
            }
            continue;
        }
#pragma unroll
        for (int r = 0; r < SW; ++r)
            if (e[r].x >= kth && e[r].x != 0u) fused_request(t, (int)e[r].y, e[r].x, sPk, sFirst, sBits, BW);
    }
}

// LONG pools, between segments: the wave's rows t with sRowN[t] > 0 (their list length, more
// than kSurv) cut their survivor lists back to the entries with key >= x, four rows per pass on
// the 16-lane DPP rows; x is the row's 32nd largest key, or its (k+1)-th largest where more than
// 32 entries tie at the 32nd.  sRowN[t] becomes the new length (-2: more than 32 entries even at
// the (k+1)-th key) and sRowT[t] = x.
__device__ __forceinline__ void fused_merge(int w, int k, uint2* sSv, int* sRowN, uint32_t* sRowT) {
    const int l = lane_id(), seg = l & 15;
    const uint64_t gm = 0xffffull << (l & 48);           // this lane's DPP row
    const uint64_t below = gm & ((1ull << l) - 1ull);
    for (int p = 0; p < 4; ++p) {
        const int t = 16 * w + 4 * p + l / 16;
        const int ns = sRowN[t];
        if (__ballot(ns > 0) == 0ull) continue;          // wave-uniform
        uint2* rowbuf = sSv + t * kSvStride;
        uint2 e[4];
        uint32_t R[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int x = 4 * seg + r;
            e[r] = x < ns ? rowbuf[x] : make_uint2(0u, 0u);
            R[r] = e[r].x;
        }
        sort64_row(R, seg);                               // ascending: position 64 - j = j-th largest
        const uint32_t x32 = r16_umax(seg == 8 ? R[0] : 0u);
        const int ek1 = 63 - k;
        const uint32_t vk1 = (ek1 & 3) == 0 ? R[0] : (ek1 & 3) == 1 ? R[1] : (ek1 & 3) == 2 ? R[2] : R[3];
        const uint32_t k1th = r16_umax(seg == (ek1 >> 2) ? vk1 : 0u);
        int c32 = 0;
#pragma unroll
        for (int r = 0; r < 4; ++r) c32 += e[r].x >= x32 && e[r].x != 0u ? 1 : 0;
        c32 = r16_sum(c32);
        const uint32_t x = c32 <= kSurv ? x32 : k1th;
        int pos = 0;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const bool in = ns > 0 && e[r].x >= x && e[r].x != 0u;
            const uint64_t bal = __ballot(in);
            if (in) rowbuf[pos + __popcll(bal & below)] = e[r];
            pos += __popcll(bal & gm);
        }
        if (seg == 0 && ns > 0) {
            sRowN[t] = pos > kSurv ? -2 : pos;
            sRowT[t] = x;
        }
    }
}

// Canonical re-rank of an uncertain stage-1 row t from its survivor list (one wave): every
// survivor whose MFMA key is >= band (which holds every candidate that can be among the row's
// canonical top k: those have MFMA scores >= kth - 2 delta) is rescored with the canonical chain;
// the k best by (canonical score, lower id) are requested.
template <int DH>
__device__ __noinline__ void fused_canon_band(int t, int k, uint32_t band, const uint2* rowbuf,
                                              int ns, const uint16_t* qr, const uint16_t* kb,
                                              float scale, uint32_t* sPk, int* sFirst,
                                              uint32_t* sBits, int BW) {
    const int l = lane_id();
    const uint2 e = l < ns ? rowbuf[l] : make_uint2(0u, 0u);
    const bool in = l < ns && e.x >= band;
    const float E = in ? canon_dot<HGA_DTYPE_BF16, DH>(qr, kb + (int64_t)e.y * DH, scale) : -INFINITY;
    int rank = 0;
    for (uint64_t m = __ballot(in); m != 0ull; m &= m - 1ull) {
        const int j = __builtin_ctzll(m);
        const float Ej = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(E), j));
        const int idj = __builtin_amdgcn_readlane((int)e.y, j);
        rank += (Ej > E || (Ej == E && idj < (int)e.y)) ? 1 : 0;
    }
    if (in && rank < k) fused_request(t, (int)e.y, okey(E), sPk, sFirst, sBits, BW);
}

// Rows whose selection the MFMA scores could not certify (queued in sAmb): every candidate
// rescored with the canonical chain, one dot product at a time, and the exact top-k requested.
// Candidate i is row kb + i*DH (stage 1, sel == nullptr) or group sel[i/M]*M + i%M of kb
// (stage 2, visible to row t iff thr[i/M] <= t).  Returns the number of rows this wave took.
template <int DH, int JMAX = 8>
__device__ __noinline__ int fused_canon_rows(int w, int namb, const int* sAmb, int ncand, int k,
                                             const uint16_t* qg, int64_t q_ss, const uint16_t* kb,
                                             const int* sel, int M, const int* thr, float scale,
                                             uint32_t* sPk, int* sFirst, uint32_t* sBits, int BW) {
    const int l = lane_id();
    int taken = 0;
    auto row_of = [&](int i) -> const uint16_t* {
        return sel ? kb + ((int64_t)sel[i / M] * M + (i % M)) * DH : kb + (int64_t)i * DH;
    };
    dispatch_j<JMAX>(ncand, [&](auto jt) {
        constexpr int J = decltype(jt)::value;
        for (int a = w; a < namb; a += kFWaves) {
            const int ta = sAmb[a];
            const uint16_t* qr = qg + ta * q_ss;
            float v[J];
#pragma unroll
            for (int j = 0; j < J; ++j) {
                const int i = l + 64 * j;
                const bool vis = i < ncand && (!thr || thr[i / M] <= ta);
                v[j] = vis ? canon_dot<HGA_DTYPE_BF16, DH>(qr, row_of(vis ? i : 0), scale) : -INFINITY;
                asm volatile("" ::: "memory");    // one dot product in flight at a time
            }
            int unused = 0;
            row_request<J>(ta, v, k, 0.0f, [](int) { return 0.0f; }, sPk, sFirst, sBits, BW, &unused);
            ++taken;
        }
    });
    return taken;
}

// Canonical top-k of an uncertain stage-1 row t over a LONG pool (one wave): the pool in blocks
// of 512 candidates (kb + i * DH), each block's exact top-k (canonical score, then lower id)
// listed at `list` in ascending id order, then the top-k of the listed entries (at most 4 k <=
// 64: the same order resolves ties to the lower id) requested.  `list` is the row's survivor
// list, unused once the row is rescored in full.
template <int DH>
__device__ __noinline__ void fused_canon_row_long(int t, int ncand, int k, const uint16_t* qr,
                                                  const uint16_t* kb, float scale, uint2* list,
                                                  uint32_t* sPk, int* sFirst, uint32_t* sBits, int BW) {
    const int l = lane_id();
    int nl = 0;
    for (int c0 = 0; c0 < ncand; c0 += 512) {
        float v[8];
        uint32_t kv[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int i = c0 + l + 64 * j;
            v[j] = i < ncand ? canon_dot<HGA_DTYPE_BF16, DH>(qr, kb + (int64_t)i * DH, scale) : -INFINITY;
            kv[j] = v[j] == -INFINITY ? 0u : okey(v[j]);
            asm volatile("" ::: "memory");    // one dot product in flight at a time
        }
        const uint32_t bits = exact_topk<8>(kv, v, k);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const bool m = (bits >> j) & 1u;
            const uint64_t bal = __ballot(m);
            if (m) list[nl + lanes_below(bal)] = make_uint2(kv[j], (uint32_t)(c0 + l + 64 * j));
            nl += __popcll(bal);
        }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const uint2 e = l < nl ? list[l] : make_uint2(0u, 0u);
    uint32_t kv1[1] = {e.x};
    float v1[1] = {l < nl ? okey_inv(e.x) : -INFINITY};
    if (exact_topk<1>(kv1, v1, k) & 1u) fused_request(t, (int)e.y, e.x, sPk, sFirst, sBits, BW);
}

// Pooled selection of the fused kernel (wave 0): the certified top-k of the requested
// candidates (sFirst < kNoRow) by pooled key, the forced candidate ip, written ascending to
// sSel/sThr with ids base_id + i.  Probes (Gaussian quantile, then secant / Newton steps) find a
// threshold leaving k < count <= 32 keys; those are compacted into buf (32 slots) and sorted by
// lanes 0..15, which gives the exact k-th and (k+1)-th pooled keys.  Returns the count, or -1
// when no threshold was found, the pooled scores could not be certified or the forced
// candidate must evict a selected one (the caller then runs the general selection).
template <int J>
__device__ __forceinline__ int fused_pool_fast(int P, int k, const uint32_t* sPk, const int* sFirst,
                                               float dpool, int ip, int base_id, int* sSel,
                                               int* sThr, uint2* buf) {
    constexpr bool REG = J <= 8;            // keys held in registers; wider pools re-read LDS
    const int l = lane_id();
    uint32_t kvr[REG ? J : 1];
    int forced = -1;                        // candidate forced in (its key taken as maximal)
    auto key = [&](int j) -> uint32_t {
        const int i = l + 64 * j;
        uint32_t v;
        if constexpr (REG) v = kvr[j];
        else v = (i < P && sFirst[i] < kNoRow) ? sPk[i] : 0u;
        return i == forced ? 0xffffffffu : v;
    };
    int nreq = 0;
    float s1 = 0.0f, s2 = 0.0f;
#pragma unroll
    for (int j = 0; j < J; ++j) {
        const int i = l + 64 * j;
        uint32_t v = 0u;
        if (64 * j < P) {                                 // wave-uniform
            if (i < P && sFirst[i] < kNoRow) v = sPk[i];
            nreq += __popcll(__ballot(v != 0u));
            const float f = v != 0u ? okey_inv(v) : 0.0f;
            s1 += f;
            s2 = fmaf(f, f, s2);
        }
        if constexpr (REG) kvr[j] = v;
    }
    uint32_t x = 1u;                                      // members: keys >= x
    if (nreq > k) {
        // a threshold T leaving k < count(key >= T) <= 32 requested candidates
        // (the probe positions are a search seed only: approximate instructions are fine, the
        // threshold found is exact by its count)
        s1 = wsum(s1);
        s2 = wsum(s2);
        const float rn = __builtin_amdgcn_rcpf((float)nreq);
        const float mu = s1 * rn;
        const float sd = __builtin_amdgcn_sqrtf(fmaxf(s2 * rn - mu * mu, 0.0f));
        const float rsd = __builtin_amdgcn_rcpf(sd > 0.0f ? sd : 1.0f);
        const float target = 0.5f * (float)(k + 1 + 32);
        uint32_t T = 1u;
        bool ok = nreq <= 32;
        float xf = mu + z_upper_fast((target + 0.5f) * rn) * sd, lf = 0.0f, hf = 0.0f;
        int clo = -1, chi = -1;
        for (int it = 0; it < 8 && !ok; ++it) {
            const uint32_t tx = min(max(okey_fast(xf), 1u), 0xfffffffeu);
            int c = 0;
#pragma unroll
            for (int j = 0; j < J; ++j)
                if (64 * j < P) c += __popcll(__ballot(key(j) >= tx));
            if (c > k && c <= 32) {
                ok = true;
                T = tx;
            } else {
                if (c > 32) {
                    lf = xf;
                    clo = c;
                } else {
                    hf = xf;
                    chi = c;
                }
                if (clo >= 0 && chi >= 0) {
                    xf = lf + (hf - lf) * ((float)clo - target) * __builtin_amdgcn_rcpf((float)(clo - chi));
                } else {
                    const float z = (xf - mu) * rsd;
                    const float dens = (float)nreq * 0.39894228f * __expf(-0.5f * z * z) * rsd;
                    const float step = ((float)c - target) * __builtin_amdgcn_rcpf(fmaxf(dens, 1e-30f));
                    xf += fminf(fmaxf(step, -2.0f * sd), 2.0f * sd);
                }
            }
        }
        if (!ok) return -1;
        // compact the keys >= T (with their candidate index) and sort them on lanes 0..15
        int base = 0;
#pragma unroll
        for (int j = 0; j < J; ++j) {
            if (64 * j < P) {
                const uint32_t v = key(j);
                const bool in = v >= T && v != 0u;
                const uint64_t bal = __ballot(in);
                if (in) buf[base + lanes_below(bal)] = make_uint2(v, (uint32_t)(l + 64 * j));
                base += __popcll(bal);
            }
        }
        __builtin_amdgcn_wave_barrier();
        const int seg = l & 15;
        uint32_t a = l < 16 && 2 * seg < base ? buf[2 * seg].x : 0u;
        uint32_t bb = l < 16 && 2 * seg + 1 < base ? buf[2 * seg + 1].x : 0u;
        sort32_row(a, bb, seg);
        const int ek = 32 - k, ek1 = ek - 1;
        const uint32_t kth = (uint32_t)__builtin_amdgcn_readfirstlane(
            (int)r16_umax(seg == (ek >> 1) ? ((ek & 1) ? bb : a) : 0u));
        const uint32_t k1th = (uint32_t)__builtin_amdgcn_readfirstlane(
            (int)r16_umax(seg == (ek1 >> 1) ? ((ek1 & 1) ? bb : a) : 0u));
        if (kth == k1th || !(okey_inv(kth) - 2.0f * dpool > okey_inv(k1th))) return -1;
        x = kth;
    }
    int nsel = nreq < k ? nreq : k;
    if (ip >= 0) {
        bool have = false;
#pragma unroll
        for (int j = 0; j < J; ++j)
            if (j == ip / 64) {
                const uint32_t v = key(j);
                have = v >= x && v != 0u;                 // meaningful in lane ip % 64
            }
        const bool have_w = __ballot(l == ip % 64 && have) != 0ull;
        if (!have_w) {
            if (nsel >= k) return -1;                     // eviction: general path
            forced = ip;                                  // forced in (key >= x)
            ++nsel;
        }
    }
    int base = 0;
#pragma unroll
    for (int j = 0; j < J; ++j) {
        if (64 * j < P) {
            const uint32_t v = key(j);
            const bool m = v >= x && v != 0u;
            const uint64_t bal = __ballot(m);
            if (m) {
                const int i = l + 64 * j;
                const int pos = base + lanes_below(bal);
                sSel[pos] = base_id + i;
                sThr[pos] = i == ip ? 0 : sFirst[i];
            }
            base += __popcll(bal);
        }
    }
    return base;
}

// General pooled selection (certified with canonical pooled values, forced-candidate
// eviction): the split kernels' routine, out of line.  Returns the count in the low 16 bits and
// the number of canonically rescored pooled candidates above them (a value, not an out-pointer,
// so that the caller keeps no stack slot).
template <int DH, int J>
__device__ __noinline__ int fused_pool_general(int P, int k, int rows, const uint32_t* sBits, int BW,
                                               const uint32_t* sPk, const int* sFirst, float dpool,
                                               const uint16_t* qg, int64_t q_ss, const uint16_t* kb,
                                               float scale, int ip, int base_id, int* sSel,
                                               int* sThr) {
    auto canon = [&](int t, int i) {
        return canon_dot<HGA_DTYPE_BF16, DH>(qg + t * q_ss, kb + (int64_t)i * DH, scale);
    };
    int amb = 0;
    const int cnt = pooled_select<J>(P, k, rows, sBits, BW, sPk, sFirst, dpool, canon,
                                     ip, base_id, sSel, sThr, &amb);
    return cnt | (amb << 16);
}

// LDS: [stage region][survivors][row and selection scalars][pooled state (LONG only)].  The stage
// region holds the two stage-1 stages; the ordinary variant keeps its pooled state (pooled keys,
// first requesting rows, request bits) there once stage-1 scoring is over, and stages stage 2's
// group rows in the survivor area, which is free by then: about 51 KB (Dh 128), three
// workgroups per CU.
// The ordinary variant's layout is fixed at its largest pool (kFusedMaxPool chunks), so that every
// LDS array sits at a compile-time offset.
constexpr int kSPPo = kFusedMaxPool + 1;                       // pooled slots (ordinary variant)
constexpr int kBWo = (kSPPo + 31) / 32;                        // request-bit words per row
constexpr int kPooledO = (8 * kSPPo + 4 * kRows * kBWo + 15) & ~15;
constexpr int fused_region(int D) {
    return kPooledO > 2 * kFStageRows * D * 2 ? kPooledO : 2 * kFStageRows * D * 2;
}
size_t fused_lds(const RouteArgs& a, int D, bool lng) {
    const size_t stage = 2 * (size_t)kFStageRows * D * 2;
    const size_t pooled = 2 * sizeof(int) * (size_t)a.SPP + sizeof(uint32_t) * kRows * (size_t)a.BW;
    const size_t misc = sizeof(float) * kRows + 3 * sizeof(int) * kRows +
                        sizeof(int) * (2 * kMaxSel + 8 + kRows) + sizeof(float) * 4;
    const size_t surv = sizeof(uint2) * kRows * kSvStride;
    if (lng) return stage + surv + misc + pooled;
    return (size_t)fused_region(D) + surv + misc;
}

template <int DH, bool LONG>
__global__ __launch_bounds__(kFThreads) __attribute__((amdgpu_waves_per_eu(LONG ? 2 : 3)))
void route_fused_kernel(RouteArgs A) {
    constexpr int KS = DH / 32;
    constexpr int PJ = (LONG ? kFusedMaxPoolLong : kFusedMaxPool) / kWave;   // pool slots per lane
    constexpr int SR = kFStageRows;                                    // candidate rows per stage
    constexpr int GT = SR / 16;                                        // tiles per stage
    constexpr int kStageBytes = SR * DH * 2;
    extern __shared__ __align__(16) unsigned char smem_raw[];
    unsigned char* sStage = smem_raw;                                  // [2][SR][DH] candidate rows
    constexpr int region = LONG ? 2 * kStageBytes : fused_region(DH);
    uint2* sSv = reinterpret_cast<uint2*>(sStage + region);            // [64][kSvStride] survivors
    // stage 2's group rows: the survivor area (ordinary) or the two stages (LONG)
    unsigned char* sStage2 = LONG ? sStage : reinterpret_cast<unsigned char*>(sSv);
    float* sQn = reinterpret_cast<float*>(sSv + kRows * kSvStride);    // [64] row norms
    int* sRowN = reinterpret_cast<int*>(sQn + kRows);                  // [64] survivors of a row
    uint32_t* sBand = reinterpret_cast<uint32_t*>(sRowN + kRows);      // [64] re-rank band key
    uint32_t* sRowT = sBand + kRows;                                   // [64] compaction threshold
    int* sSel = reinterpret_cast<int*>(sRowT + kRows);                 // [kMaxSel]
    int* sThr = sSel + kMaxSel;                                        // [kMaxSel]
    int* sScal = sThr + kMaxSel;                                       // [8]
    int* sAmb = sScal + 8;                                             // [64]
    float* sKn = reinterpret_cast<float*>(sAmb + kRows);               // [4] per-wave norm maxima
    // pooled state (zeroed once stage-1 scoring is over): [SPP] pooled key, [SPP] first
    // requesting row, [64][BW] request bits
    uint32_t* sPk = LONG ? reinterpret_cast<uint32_t*>(sKn + 4) : reinterpret_cast<uint32_t*>(smem_raw);
    int* sFirst = reinterpret_cast<int*>(sPk + (LONG ? A.SPP : kSPPo));
    uint32_t* sBits = reinterpret_cast<uint32_t*>(sFirst + (LONG ? A.SPP : kSPPo));

    const int N = A.N, C = A.C, M = A.M, BW = A.BW;
    const int n = A.n_hi - 1 - (int)(blockIdx.x / (A.B * A.H));       // heavy chunks first
    const int bh = blockIdx.x % (A.B * A.H);
    const int b = bh / A.H, h = bh % A.H, kvh = h / (A.H / A.KVH);
    const int w = threadIdx.x / kWave, l = lane_id(), r16 = l % 16, qd = l / 16;
    int rows = A.S - n * C;
    if (rows > C) rows = C;
    int f_hi, l_lo;
    windows(n, A.kf, A.kl, &f_hi, &l_lo);
    const int P = l_lo > f_hi ? l_lo - f_hi : 0;
    const int64_t o = ((int64_t)b * A.H + h) * N + n;
    const int Kcw = A.Kc > 0 ? A.Kc : 1, Kgw = A.Kg > 0 ? A.Kg : 1;
    int32_t* out_sc = A.sel_chunk + o * Kcw;
    int32_t* out_st = A.sel_thr + o * Kcw;
    int32_t* out_og = A.open_grp + o * Kgw;
    int32_t* out_ot = A.open_thr + o * Kgw;
    if (A.Kc == 0 || P == 0) {
        for (int i = threadIdx.x; i < Kcw; i += kFThreads) out_sc[i] = out_st[i] = -1;
        for (int i = threadIdx.x; i < Kgw; i += kFThreads) out_og[i] = out_ot[i] = -1;
        if (threadIdx.x == 0) A.n_sel[o] = A.n_open[o] = 0;
        return;
    }
    const float scale = A.scale;
    const uint16_t* qg = reinterpret_cast<const uint16_t*>(A.q) + b * A.q_sb + h * A.q_sh +
                         (int64_t)n * C * A.q_ss;
    const uint16_t* ckb = reinterpret_cast<const uint16_t*>(A.ck) + b * A.ck_sb + kvh * A.ck_sh;
    const uint16_t* gkb = reinterpret_cast<const uint16_t*>(A.gk) + b * A.gk_sb + kvh * A.gk_sh;
    const uint16_t* pool = ckb + (int64_t)f_hi * DH;             // candidate i = chunk f_hi + i
    const int t = 16 * w + r16;                 // this lane's row (MFMA layout)
    const bool act = t < rows;
    const bool wave_act = 16 * w < rows;        // wave-uniform
    const int nwact = (rows + 15) / 16;         // active waves (they split the norm bound)
    const uint32_t stage_lds =
        (uint32_t)(uintptr_t)(__attribute__((address_space(3))) unsigned char*)sStage;

    // the first SR pool candidates go to LDS stage 0 now, so that their copy overlaps the q loads
    // (vector memory loads complete in order: the compiler's waits for q also cover them)
    stage_rows<DH, SR>(pool, [&](int r) { return (uint32_t)(r * DH * 2); }, P < SR ? P : SR,
                       stage_lds, w);
    // query rows: B operand (row l % 16, dims 32 ks + 8 qd) and norms.  The ordinary variant
    // reads q again for stage 2 (from L2: a plain load here allocates it there) rather than keep
    // it in registers through the stage-1 selection, whose out-of-line calls would have to save
    // it; the LONG variant streams q once (non-temporal, so its larger summaries stay in L2)
    auto load_q = [&](bf16x8 (&qb)[KS], const uint16_t* qp, bool nt, float* sumsq) __attribute__((always_inline)) {
        float x = 0.0f;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            uint4 u = make_uint4(0u, 0u, 0u, 0u);
            if (act) {
                typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
                const u32x4* src = reinterpret_cast<const u32x4*>(qp + (int64_t)t * A.q_ss + 32 * ks + 8 * qd);
                const u32x4 r = nt ? __builtin_nontemporal_load(src) : *src;
                u = make_uint4(r.x, r.y, r.z, r.w);
            }
            if (sumsq) x += sumsq_bf16x8(u);
            qb[ks] = as_bf16x8(u);
        }
        if (sumsq) *sumsq = x;
    };
    {
        bf16x8 qn[KS];
        float x = 0.0f;
        load_q(qn, qg, LONG, &x);
        x = q4_fsum(x);
        if (qd == 0) sQn[t] = __builtin_sqrtf(x);
    }
    if (threadIdx.x < 8) sScal[threadIdx.x] = 0;
    __syncthreads();

    // ---- stage 1: segments of up to 256 pool candidates ------------------------------------
    const int kreq = A.Kc < P ? A.Kc : P;
    const bool open = act && P > kreq;
    float knmax = 0.0f;
    int nsurv = 0;
    bool hard = false;
    uint32_t tmax = 1u;                         // largest compaction threshold of the segments
    const int nseg = (P + kSegCand - 1) / kSegCand;
    uint32_t kv[4 * kSegTiles];
    for (int sg = 0; sg < nseg; ++sg) {
        // every wave copies a quarter of each SR-candidate group into an LDS stage (double
        // buffered, one group ahead); the waves with query rows score the stage
        const int c0 = sg * kSegCand;
        const int ncs = P - c0 < kSegCand ? P - c0 : kSegCand;
        const int nt = (ncs + 15) / 16;
        const int ngr = (nt + GT - 1) / GT;
        float s1 = 0.0f, s2 = 0.0f;
        int ns = 0;
        if (sg > 0) {
            __syncthreads();                      // the previous segment's stages are read
            stage_rows<DH, SR>(pool, [&](int r) { return (uint32_t)((c0 + r) * DH * 2); }, ncs,
                               stage_lds, w);
        }
        // q as the B operand, read per segment (L2 hits after the first): held through the
        // scoring only, not through the selection of the segment's rows
        bf16x8 qb[KS];
        {
            const uint16_t* qs = qg;
            asm volatile("" : "+s"(qs));
            load_q(qb, qs, LONG, nullptr);
        }
#pragma unroll
        for (int g = 0; g < kSegTiles / GT; ++g) {
            if (g < ngr) {                                            // workgroup-uniform
                __builtin_amdgcn_s_waitcnt(0);
                __syncthreads();          // stage g % 2 complete, stage (g + 1) % 2 no longer read
                if (g + 1 < ngr)
                    stage_rows<DH, SR>(pool, [&](int r) { return (uint32_t)((c0 + SR * (g + 1) + r) * DH * 2); },
                                       ncs - SR * (g + 1), stage_lds + (uint32_t)(((g + 1) & 1) * kStageBytes), w);
                if (wave_act)
                    stage_scores<DH, 4 * kSegTiles, GT>(sStage + (g & 1) * kStageBytes, GT * g, c0 + SR * g,
                                                        P, w, nwact, qb, scale, kv, knmax, s1, s2, ns);
            } else {
#pragma unroll
                for (int i = 4 * GT * g; i < 4 * GT * (g + 1); ++i) kv[i] = 0u;
            }
        }
        if (!wave_act) continue;
        if (open) {
            s1 = q4_fsum(s1);
            s2 = q4_fsum(s2);
            ns = q4_sum(ns);
            uint32_t T;
            const bool ok = fused_probe<4 * kSegTiles>(kv, 4 * nt, !hard, ncs, kreq, s1, s2, ns, T);
            hard = hard || !ok;
            tmax = max(tmax, T);
            nsurv = fused_compact<4 * kSegTiles>(kv, 4 * nt, T, c0, sSv + t * kSvStride, nsurv, !hard);
        }
        if constexpr (LONG) {
            // lists longer than kSurv are cut back before the next segment appends its survivors
            const bool big = open && !hard && nsurv > kSurv;
            if (sg + 1 < nseg && __ballot(big) != 0ull) {             // wave-uniform
                if (qd == 0) sRowN[t] = big ? nsurv : -1;
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                __builtin_amdgcn_wave_barrier();
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
                fused_merge(w, kreq, sSv, sRowN, sRowT);
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                __builtin_amdgcn_wave_barrier();
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
                if (big) {
                    const int m = sRowN[t];
                    hard = m < 0;
                    nsurv = m < 0 ? 0 : m;
                    tmax = max(tmax, sRowT[t]);
                }
            }
        }
    }
    // the stages are read: the pooled state (in the stage region of the ordinary variant) is set up
    __syncthreads();
    for (int i = threadIdx.x; i < A.SPP; i += kFThreads) {
        sPk[i] = 0u;
        sFirst[i] = kNoRow;
    }
    for (int i = threadIdx.x; i < kRows * BW; i += kFThreads) sBits[i] = 0u;
    if (wave_act) {
        if (qd == 0) {
            sRowN[t] = !open ? -1 : (hard ? -2 : nsurv);
            sRowT[t] = tmax;
        }
        knmax = wmax(knmax);
    }
    if (l == 0) sKn[w] = knmax;
    __syncthreads();
    knmax = fmaxf(fmaxf(sKn[0], sKn[1]), fmaxf(sKn[2], sKn[3]));
    const float ds1 = kDeltaRel * knmax * scale * 1.01f;
    if (act && !open) {
        // every valid candidate requested (P <= Kc: one segment, one tile)
#pragma unroll
        for (int i = 0; i < 4; ++i)
            if (kv[i] != 0u) fused_request(t, 4 * qd + i, kv[i], sPk, sFirst, sBits, BW);
    }
    if (wave_act) {
        if (nseg > 1)
            list_rows<4>(w, kreq, ds1, sQn, sSv, sRowN, sRowT, sPk, sFirst, sBits, BW, sAmb, &sScal[4], sBand);
        else
            list_rows<2>(w, kreq, ds1, sQn, sSv, sRowN, sRowT, sPk, sFirst, sBits, BW, sAmb, &sScal[4], sBand);
    }
    __syncthreads();
    int amb1 = 0, amb1p = 0;
    {
        const int namb = sScal[4];
        for (int a = w; a < namb; a += kFWaves) {
            const int ta = sAmb[a];
            if (sBand[ta] != 0u)
                fused_canon_band<DH>(ta, kreq, sBand[ta], sSv + ta * kSvStride, sRowN[ta],
                                     qg + ta * A.q_ss, pool, scale, sPk, sFirst, sBits, BW);
            else if (LONG && P > kFusedMaxPool)
                fused_canon_row_long<DH>(ta, P, kreq, qg + ta * A.q_ss, pool, scale, sSv + ta * kSvStride,
                                         sPk, sFirst, sBits, BW);
            else
                fused_canon_rows<DH>(0, 1, sAmb + a, P, kreq, qg, A.q_ss, pool, nullptr, 0, nullptr,
                                     scale, sPk, sFirst, sBits, BW);
            ++amb1;
        }
    }
    __syncthreads();
    float qnmax = 0.0f;
    {
        float x = 0.0f;
        if (l < rows) x = sQn[l];
        qnmax = wmax(x);
    }
    if (w == 0) {
        const float dpool = kDeltaRel * knmax * qnmax * scale * 1.01f;
        const int prev = n - 1;
        const int ip = (n > 0 && prev >= f_hi && prev < l_lo) ? prev - f_hi : -1;
        int cnt = fused_pool_fast<PJ>(P, A.Kc, sPk, sFirst, dpool, ip, f_hi, sSel, sThr, sSv);
        if (cnt < 0) {
            const int r = fused_pool_general<DH, PJ>(P, A.Kc, rows, sBits, BW, sPk, sFirst, dpool, qg,
                                                     A.q_ss, pool, scale, ip, f_hi, sSel, sThr);
            cnt = r & 0xffff;
            amb1p = r >> 16;
        }
        if (l == 0) sScal[0] = cnt;
    }
    __syncthreads();
    const int nsel = sScal[0];
    for (int i = threadIdx.x; i < Kcw; i += kFThreads) {
        out_sc[i] = i < nsel ? sSel[i] : -1;
        out_st[i] = i < nsel ? sThr[i] : -1;
    }
    if (threadIdx.x == 0) A.n_sel[o] = nsel;
    if (A.stats && threadIdx.x == 0 && amb1p) atomicAdd(&A.stats[1], amb1p);
    if (A.stats && l == 0 && amb1) atomicAdd(&A.stats[0], amb1);

    // ---- stage 2: the M groups of each selected chunk --------------------------------------
    if (A.Kg == 0 || A.Kgr == 0 || nsel == 0) {
        for (int i = threadIdx.x; i < Kgw; i += kFThreads) out_og[i] = out_ot[i] = -1;
        if (threadIdx.x == 0) A.n_open[o] = 0;
        return;
    }
    const int T2 = nsel * M;
    const int BW2 = A.BW2;
    __syncthreads();                              // the stage-1 stages / survivor lists are read
    const uint32_t stage2_lds =
        (uint32_t)(uintptr_t)(__attribute__((address_space(3))) unsigned char*)sStage2;
    stage_rows<DH, 64>(gkb, [&](int r) { return (uint32_t)(((int64_t)sSel[r / M] * M + (r % M)) * DH * 2); },
                       T2, stage2_lds, w);
    bf16x8 qb2[KS];
    {
        // q again, in flight with the group rows (the wait below covers both)
        const uint16_t* qg2 = qg;
        asm volatile("" : "+s"(qg2));            // a fresh read: q is not kept from stage 1
        if (wave_act) load_q(qb2, qg2, LONG, nullptr);
    }
    for (int i = threadIdx.x; i < T2 + 1; i += kFThreads) {
        sPk[i] = 0u;
        sFirst[i] = kNoRow;
    }
    for (int i = threadIdx.x; i < kRows * BW2; i += kFThreads) sBits[i] = 0u;
    if (threadIdx.x < 8) sScal[threadIdx.x] = 0;
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    auto grow = [&](int i) -> const uint16_t* {
        return gkb + ((int64_t)sSel[i / M] * M + (i % M)) * DH;
    };
    float knmax2 = 0.0f;
    uint32_t kv2[16];
    bool open2 = false;
    uint32_t kth2 = 0u, k1th2 = 0u;
    if (wave_act) {
        int nv2 = 0;
        float s1 = 0.0f, s2 = 0.0f;
        int ns = 0;
        stage_scores<DH, 16, 4>(sStage2, 0, 0, T2, w, nwact, qb2, scale, kv2, knmax2, s1, s2, ns);
        // candidate c is visible to row t from its parent's first row on
        ns = 0;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int c = 16 * (i / 4) + 4 * qd + (i % 4);
            const int pt = c < T2 ? sThr[c / M] : kNoRow;
            kv2[i] = pt <= t ? kv2[i] : 0u;
            ns += kv2[i] != 0u ? 1 : 0;
        }
        nv2 = q4_sum(ns);
        open2 = act && nv2 > A.Kgr;
        // rows with more visible groups than Kgr: the exact Kgr-th and (Kgr+1)-th largest keys of
        // the row's T2 <= 64 keys (zeros for the invisible ones), sorted across its four lanes
        if (__ballot(open2) != 0ull) {                                // wave-uniform
            uint32_t S[16];
#pragma unroll
            for (int i = 0; i < 16; ++i) S[i] = kv2[i];
            if (A.Kgr == 32) {
                split64_q4(S, qd, kth2, k1th2);
            } else {
                sort64_q4(S, qd);
                kth2 = q4_pick(S, 64 - A.Kgr, qd);
                k1th2 = q4_pick(S, 63 - A.Kgr, qd);
            }
        }
        knmax2 = wmax(knmax2);
    }
    if (l == 0) sKn[w] = knmax2;
    __syncthreads();
    knmax2 = fmaxf(fmaxf(sKn[0], sKn[1]), fmaxf(sKn[2], sKn[3]));
    const float ds2 = kDeltaRel * knmax2 * scale * 1.01f;
    if (wave_act) {                                                   // wave-uniform
        // a row whose Kgr-th and (Kgr+1)-th MFMA scores lie within 2*delta (or tie) is rescored
        // canonically in full
        bool amb = false;
        if (open2) {
            const float delta = ds2 * sQn[t];
            amb = kth2 == k1th2 || !(okey_inv(kth2) - 2.0f * delta > okey_inv(k1th2));
            if (amb && qd == 0) {
                sBand[t] = 0u;
                sAmb[atomicAdd(&sScal[4], 1)] = t;
            }
        }
        // Requests: every visible group of a row with at most Kgr of them, the certified members
        // of the others.  A candidate sits in the same register slot of the wave's 16 rows (one
        // DPP row per lane quarter), so its pooled key (max) and first requesting row (min) over
        // those rows are 16-lane reductions and cost one atomic pair per candidate and wave;
        // each row's request bits (T2 <= 64) are stored once.
        const bool req = act && !amb;
        const uint32_t lim = open2 ? kth2 : 1u;
        uint32_t blo = 0u, bhi = 0u;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int id = 16 * (i / 4) + 4 * qd + (i % 4);
            const bool mem = req && kv2[i] >= lim && kv2[i] != 0u;
            const uint32_t mk = r16_umax(mem ? kv2[i] : 0u);
            const uint32_t fr = r16_umin(mem ? (uint32_t)t : (uint32_t)kNoRow);
            if (r16 == i && mk != 0u) {
                atomicMax(&sPk[id], mk);
                atomicMin(&sFirst[id], (int)fr);
            }
            if (mem) {
                if (id < 32) blo |= 1u << id;
                else bhi |= 1u << (id - 32);
            }
        }
        blo |= (uint32_t)__shfl_xor((int)blo, 16, kWave);
        bhi |= (uint32_t)__shfl_xor((int)bhi, 16, kWave);
        blo |= (uint32_t)__shfl_xor((int)blo, 32, kWave);
        bhi |= (uint32_t)__shfl_xor((int)bhi, 32, kWave);
        if (qd == 0 && req) {
            sBits[t * BW2] = blo;
            if (BW2 > 1) sBits[t * BW2 + 1] = bhi;
        }
    }
    __syncthreads();
    int amb2 = 0, amb2p = 0;
    const int namb2 = sScal[4];
    if (namb2 > 0)
        amb2 = fused_canon_rows<DH>(w, namb2, sAmb, T2, A.Kgr, qg, A.q_ss, gkb, sSel, M, sThr,
                                    scale, sPk, sFirst, sBits, BW2);
    __syncthreads();
    if (w == 0) {
        const float dpool2 = ds2 * qnmax;
        auto canonG2 = [&](int tt, int i) {
            return canon_dot<HGA_DTYPE_BF16, DH>(qg + tt * A.q_ss, grow(i), scale);
        };
        float v[1];
        v[0] = (l < T2 && sFirst[l] < kNoRow) ? okey_inv(sPk[l]) : -INFINITY;
        auto canon_pool2 = [&](int i) { return pooled_exact(i, rows, sBits, BW2, canonG2); };
        const uint32_t op = select_certified<1>(v, A.Kg, dpool2, canon_pool2, &amb2p);
        const bool m = op & 1u;
        const uint64_t bal = __ballot(m);
        if (m) {
            const int pos = lanes_below(bal);
            if (pos < Kgw) {
                out_og[pos] = sSel[l / M] * M + (l % M);
                out_ot[pos] = sFirst[l];
            }
        }
        const int cnt = __popcll(bal);
        for (int i = cnt + l; i < Kgw; i += kWave) out_og[i] = out_ot[i] = -1;
        if (l == 0) A.n_open[o] = cnt;
        if (A.stats && l == 0 && amb2p) atomicAdd(&A.stats[3], amb2p);
    }
    if (A.stats && l == 0 && amb2) atomicAdd(&A.stats[2], amb2);
}

template <int DH, bool LONG>
int launch_route_fused(const RouteArgs& a, size_t lds, int nchunks, hipStream_t st) {
    auto k = route_fused_kernel<DH, LONG>;
    static bool attr_done = false;
    if (!attr_done) {
        if (hipFuncSetAttribute((const void*)k, hipFuncAttributeMaxDynamicSharedMemorySize,
                                163840) != hipSuccess) {
            set_error("hga_route_prefill: cannot raise the LDS limit");
            return HGA_ERR_LAUNCH;
        }
        attr_done = true;
    }
    const unsigned grid = (unsigned)(a.B * a.H * nchunks);
    k<<<dim3(grid), dim3(kFThreads), lds, st>>>(a);
    return launch_status(LONG ? "hga_route_prefill (fused, long pools)" : "hga_route_prefill (fused)");
}

template <int DT, int DH>
int launch_route(const RouteArgs& a, size_t lds1, size_t lds2, hipStream_t st) {
    auto k1 = route_stage1_kernel<DT, DH>;
    auto k2 = route_stage2_kernel<DT, DH>;
    static bool attr_done = false;
    if (!attr_done) {
        if (hipFuncSetAttribute((const void*)k1, hipFuncAttributeMaxDynamicSharedMemorySize,
                                163840) != hipSuccess ||
            hipFuncSetAttribute((const void*)k2, hipFuncAttributeMaxDynamicSharedMemorySize,
                                163840) != hipSuccess) {
            set_error("hga_route_prefill: cannot raise the LDS limit");
            return HGA_ERR_LAUNCH;
        }
        attr_done = true;
    }
    const unsigned grid = (unsigned)(a.B * a.H * a.N);
    k1<<<dim3(grid), dim3(kThreads), lds1, st>>>(a);
    int rc = launch_status("hga_route_prefill (stage 1)");
    if (rc) return rc;
    k2<<<dim3(grid), dim3(kThreads2), lds2, st>>>(a);
    return launch_status("hga_route_prefill (stage 2)");
}

}  // namespace
}  // namespace hga

extern "C" int hga_route_prefill(const hga_config* cfg, int32_t S, const void* q, int64_t q_sb,
                                 int64_t q_sh, int64_t q_ss, const void* chunk_k, int64_t ck_sb,
                                 int64_t ck_sh, const void* group_k, int64_t gk_sb,
                                 int64_t gk_sh, int32_t* sel_chunk, int32_t* sel_thr,
                                 int32_t* n_sel, int32_t* open_grp, int32_t* open_thr,
                                 int32_t* n_open, int32_t flags, int32_t* stats, void* stream) {
    using namespace hga;
    int rc = check_config(cfg);
    if (rc) return rc;
    HGA_REQUIRE(q && chunk_k && group_k && sel_chunk && sel_thr && n_sel && open_grp &&
                    open_thr && n_open,
                HGA_ERR_ARG, "hga_route_prefill: NULL pointer");
    HGA_REQUIRE(S >= 0, HGA_ERR_ARG, "hga_route_prefill: negative S");
    if (S == 0) return HGA_OK;
    RouteArgs a{};
    a.q = q; a.q_sb = q_sb; a.q_sh = q_sh; a.q_ss = q_ss;
    a.ck = chunk_k; a.ck_sb = ck_sb; a.ck_sh = ck_sh;
    a.gk = group_k; a.gk_sb = gk_sb; a.gk_sh = gk_sh;
    a.sel_chunk = sel_chunk; a.sel_thr = sel_thr; a.n_sel = n_sel;
    a.open_grp = open_grp; a.open_thr = open_thr; a.n_open = n_open; a.stats = stats;
    a.B = cfg->batch; a.H = cfg->heads; a.KVH = cfg->kv_heads; a.S = S;
    a.C = cfg->chunk_size; a.M = cfg->chunk_size / cfg->group_size;
    a.N = chunks_of(S, a.C);
    a.kf = cfg->keep_first; a.kl = cfg->keep_last;
    a.Kc = cfg->topk_chunks > 0 ? (cfg->topk_chunks < a.N ? cfg->topk_chunks : a.N) : 0;
    const int T2max = a.Kc * a.M;
    a.Kg = cfg->topk_groups > 0 ? (cfg->topk_groups < T2max ? cfg->topk_groups : T2max) : 0;
    a.Kgr = cfg->topk_groups > 0 ? (cfg->topk_groups / 2 < T2max ? cfg->topk_groups / 2 : T2max) : 0;
    a.canonical = (flags & HGA_ROUTE_CANONICAL) ? 1 : 0;
    a.scale = cfg->scale;
    int f_hi, l_lo;
    windows(a.N - 1, a.kf, a.kl, &f_hi, &l_lo);
    const int Pmax = l_lo > f_hi ? l_lo - f_hi : 0;
    const int D = cfg->head_dim;
    HGA_REQUIRE(a.Kc <= kMaxSel, HGA_ERR_UNSUPPORTED, "hga_route_prefill: top-k chunks %d > %d",
                a.Kc, kMaxSel);
    {
        const int64_t ve = cfg->dtype == HGA_DTYPE_BF16 ? 8 : 4;   // elements per 16 bytes
        const uintptr_t al = (uintptr_t)chunk_k | (uintptr_t)group_k | (uintptr_t)q;
        HGA_REQUIRE(al % 16 == 0 && ((ck_sb | ck_sh | gk_sb | gk_sh | q_sb | q_sh | q_ss) % ve) == 0,
                    HGA_ERR_ARG, "hga_route_prefill: q and summaries need 16-byte aligned rows");
    }
    hipStream_t st = (hipStream_t)stream;
    // bf16 MFMA scoring with a chunk of at most 64 rows, top-k chunks <= 16, pools of at most
    // 2048 chunks and at most 64 group candidates: the fused kernel (one launch, q read once;
    // the query chunks whose pools exceed 512 in a launch of the LONG variant of their own)
    const bool fused = cfg->dtype == HGA_DTYPE_BF16 && !a.canonical && !(flags & HGA_ROUTE_SPLIT) &&
                       (D == 64 || D == 128) && a.Kc <= kCompactK && Pmax <= kFusedMaxPoolLong &&
                       T2max <= kFusedMaxT2;
    if (fused) {
        // n_long: the first query chunk whose pool exceeds kFusedMaxPool (pools grow with n)
        int n_long = a.N;
        while (n_long > 0) {
            int fh, ll;
            windows(n_long - 1, a.kf, a.kl, &fh, &ll);
            if (ll - fh <= kFusedMaxPool) break;
            --n_long;
        }
        auto launch = [&](int n_lo, int n_hi, bool lng) -> int {
            int fh, ll;
            windows(n_hi - 1, a.kf, a.kl, &fh, &ll);
            const int pm = ll > fh ? ll - fh : 0;
            RouteArgs f = a;
            f.n_hi = n_hi;
            f.SPP = (pm > T2max ? pm : T2max) + 1;
            f.BW = (f.SPP + 31) / 32;
            f.BW2 = (T2max + 1 + 31) / 32;
            HGA_REQUIRE(lng || (f.SPP <= kSPPo && f.BW <= kBWo), HGA_ERR_UNSUPPORTED,
                        "hga_route_prefill: pooled state of %d slots exceeds the fused layout", f.SPP);
            const size_t lds = fused_lds(f, D, lng);
            HGA_REQUIRE(lds <= 163840, HGA_ERR_UNSUPPORTED, "hga_route_prefill: %zu bytes of LDS", lds);
            if (lng)
                return D == 128 ? launch_route_fused<128, true>(f, lds, n_hi - n_lo, st)
                                : launch_route_fused<64, true>(f, lds, n_hi - n_lo, st);
            return D == 128 ? launch_route_fused<128, false>(f, lds, n_hi - n_lo, st)
                            : launch_route_fused<64, false>(f, lds, n_hi - n_lo, st);
        };
        if (n_long < a.N) {
            rc = launch(n_long, a.N, true);
            if (rc) return rc;
        }
        return n_long > 0 ? launch(0, n_long, false) : HGA_OK;
    }
    HGA_REQUIRE(Pmax <= kJ * 64 && T2max <= kJ * 64, HGA_ERR_UNSUPPORTED,
                "hga_route_prefill: routing pool %d / group candidates %d exceed %d", Pmax,
                T2max, kJ * 64);
    // Score rows: a multiple of 4 floats (16-byte stores of the MFMA epilogue) covering every
    // 64-candidate read group, = 4 mod 32 so that the epilogue's stores are conflict-free.
    auto row_stride = [](int x) { return (x + 63) / 64 * 64 + 4; };
    a.SP = row_stride(Pmax);
    a.SP2 = row_stride(T2max);
    a.VT2 = (T2max + 63) / 64 * 64;
    // stage 1: [32][SP] scores of a row block, row norms, pooled state over the pool
    a.SSZ = kBlk * a.SP;
    a.SPP = Pmax + 1;
    a.BW = (a.SPP + 31) / 32;
    const size_t lds1 = sizeof(float) * (size_t)a.SSZ + sizeof(float) * kRows +
                        2 * sizeof(int) * (size_t)a.SPP + sizeof(uint32_t) * (size_t)kRows * a.BW +
                        sizeof(int) * (2 * kMaxSel + 8 + kRows) +
                        sizeof(uint32_t) * kBlk * kCmpStride;
    // stage 2: [64][SP2] scores of all rows, row norms, visibility table, pooled state
    a.SPP2 = T2max + 1;
    a.BW2 = (a.SPP2 + 31) / 32;
    const size_t lds2 = sizeof(float) * (size_t)kRows * a.SP2 + sizeof(float) * kRows +
                        sizeof(int) * (size_t)a.VT2 + 2 * sizeof(int) * (size_t)a.SPP2 +
                        sizeof(uint32_t) * (size_t)kRows * a.BW2 +
                        sizeof(int) * (2 * kMaxSel + 8 + kRows);
    HGA_REQUIRE(lds1 <= 163840 && lds2 <= 163840, HGA_ERR_UNSUPPORTED,
                "hga_route_prefill: %zu / %zu bytes of LDS needed (pool %d, head_dim %d)", lds1,
                lds2, Pmax, D);
#define HGA_ROUTE_CASE(DTV, DHV) \
    if (cfg->dtype == DTV && D == DHV) return launch_route<DTV, DHV>(a, lds1, lds2, st);
    HGA_ROUTE_CASE(HGA_DTYPE_BF16, 128)
    HGA_ROUTE_CASE(HGA_DTYPE_BF16, 64)
    HGA_ROUTE_CASE(HGA_DTYPE_BF16, 32)
    HGA_ROUTE_CASE(HGA_DTYPE_BF16, 16)
    HGA_ROUTE_CASE(HGA_DTYPE_F32, 128)
    HGA_ROUTE_CASE(HGA_DTYPE_F32, 64)
    HGA_ROUTE_CASE(HGA_DTYPE_F32, 32)
    HGA_ROUTE_CASE(HGA_DTYPE_F32, 16)
#undef HGA_ROUTE_CASE
    set_error("hga_route_prefill: unsupported dtype/head_dim");
    return HGA_ERR_UNSUPPORTED;
}
