// Two-level prefill router (vectorized.py:242-396) for gfx950.
//
// One 512-thread workgroup per (batch, query head, query chunk n); nothing is materialised in
// HBM except the routing lists.
//
//   1. The chunk's query rows go to LDS.  Scores of every row against every candidate of the
//      routing pool P(n) = [f_hi, l_lo) are produced into LDS: by bf16 MFMA
//      (v_mfma_f32_32x32x16_bf16, fp32 accumulate) for bf16 inputs, or by the canonical fp32
//      FMA chain for fp32 inputs / HGA_ROUTE_CANONICAL.
//   2. Each wave selects, per query row, the row's top-min(Kc,|P|) candidates with an exact
//      wave-wide bisection over order-preserving score keys (ballot counts), ties to the lower
//      chunk id.  MFMA scores differ from the canonical chain by at most
//      delta = 2^-16 * |q| * |k| * scale (both are fp32 accumulations of the same exact bf16
//      products); when the k-th and (k+1)-th scores are closer than 2*delta the row is
//      re-ranked: the candidates inside the uncertainty band are re-scored with the canonical
//      chain and the remaining slots are filled from them exactly.  Selections are therefore
//      identical to the canonical oracle.
//   3. Requests are pooled per chunk (max score, first requesting row) with LDS atomics; one
//      wave takes the top-Kc pooled chunks (same certification, with the pooled maxima
//      recomputed canonically when ambiguous), forces in chunk n-1 when it lies in the pool,
//      and writes the sorted (chunk, first row) list.
//   4. Stage 2 repeats 1-3 over the M groups of each selected chunk, with a group visible to a
//      row only from its parent's first row on, top-Kgr requests per row and top-Kg opened.
#include "hga_common.h"

namespace hga {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int kThreads = 512;
constexpr int kWaves = kThreads / kWave;
constexpr int kRows = 64;   // query rows per chunk (C <= 64)
constexpr int kJ = 8;       // candidates per lane in a wave selection: <= 512 candidates
constexpr int kMaxSel = 64; // Kc bound
constexpr float kDeltaRel = 1.0f / 65536.0f;
constexpr int kNoRow = 1 << 20;

struct RouteArgs {
    const void* q;
    int64_t q_sb, q_sh, q_ss;
    const void* ck;
    int64_t ck_sb, ck_sh;
    const void* gk;
    int64_t gk_sb, gk_sh;
    int32_t *sel_chunk, *sel_thr, *n_sel, *open_grp, *open_thr, *n_open;
    int32_t* stats;
    int B, H, KVH, S, N, C, M, kf, kl, Kc, Kg, Kgr, SP, BW, canonical;
    float scale;
};

// ------------------------------------------------------------------------------------------
// wave-level exact top-k over order-preserving keys (0 = not a candidate)
// ------------------------------------------------------------------------------------------
__device__ __forceinline__ uint32_t wave_max_u(uint32_t v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = max(v, (uint32_t)__shfl_xor((int)v, o, kWave));
    return v;
}
__device__ __forceinline__ uint32_t wave_min_u(uint32_t v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = min(v, (uint32_t)__shfl_xor((int)v, o, kWave));
    return v;
}

template <int J>
__device__ __forceinline__ int count_ge(const uint32_t (&kv)[J], uint32_t x) {
    int c = 0;
#pragma unroll
    for (int j = 0; j < J; ++j) c += __popcll(__ballot(kv[j] >= x));
    return c;
}

// Members of the top-k (largest keys; equal keys -> lower candidate index lane + 64*j).
// Returns bit j set for member candidate lane + 64*j.
template <int J>
__device__ uint32_t exact_topk(const uint32_t (&kv)[J], int k) {
    const int nvalid = count_ge<J>(kv, 1u);
    uint32_t bits = 0;
    if (nvalid <= k) {
#pragma unroll
        for (int j = 0; j < J; ++j) bits |= (kv[j] != 0u ? 1u : 0u) << j;
        return bits;
    }
    if (k <= 0) return 0u;
    uint32_t lmin = 0xffffffffu, lmax = 0u;
#pragma unroll
    for (int j = 0; j < J; ++j) {
        if (kv[j] != 0u) lmin = min(lmin, kv[j]);
        lmax = max(lmax, kv[j]);
    }
    uint32_t lo = wave_min_u(lmin), hi = wave_max_u(lmax);
    uint32_t vstar;
    if (count_ge<J>(kv, hi) >= k) {
        vstar = hi;
    } else {
        // invariant: count_ge(lo) > k, count_ge(hi) < k.  The first steps bisect the float
        // values (fast for smooth score distributions), then the key space (terminates).
        int it = 0;
        while (hi - lo > 1u) {
            uint32_t mid = lo + (hi - lo) / 2u;
            if (it++ < 16) {
                const float lf = okey_inv(lo), hf = okey_inv(hi);
                const uint32_t fm = okey(lf + (hf - lf) * 0.5f);
                if (fm > lo && fm < hi) mid = fm;
            }
            const int c = count_ge<J>(kv, mid);
            if (c == k) {
#pragma unroll
                for (int j = 0; j < J; ++j) bits |= (kv[j] >= mid ? 1u : 0u) << j;
                return bits;
            }
            if (c > k) lo = mid;
            else hi = mid;
        }
        vstar = lo;
    }
    // members: keys > vstar, then the lowest-index candidates with key == vstar
    int r = k - count_ge<J>(kv, vstar + 1u);
#pragma unroll
    for (int j = 0; j < J; ++j) {
        bits |= (kv[j] > vstar ? 1u : 0u) << j;
        uint64_t m = __ballot(kv[j] == vstar);
        uint64_t take = 0;
        while (r > 0 && m) {
            const uint64_t lowest = m & (~m + 1ull);
            take |= lowest;
            m ^= lowest;
            --r;
        }
        bits |= (uint32_t)((take >> lane_id()) & 1ull) << j;
    }
    return bits;
}

// Top-k of approximate values v (-inf = not a candidate) whose canonical values are within
// +-delta.  Ambiguous boundaries are resolved with canon(candidate) (exact).  Returns member
// bits; *amb is incremented (wave-uniformly) when the canonical re-rank ran.
template <int J, class Canon>
__device__ uint32_t select_certified(const float (&v)[J], int k, float delta, Canon canon,
                                     int* amb) {
    uint32_t kv[J];
#pragma unroll
    for (int j = 0; j < J; ++j) kv[j] = (v[j] == -INFINITY) ? 0u : okey(v[j]);
    const uint32_t bits = exact_topk<J>(kv, k);
    if (!(delta > 0.0f)) return bits;
    if (count_ge<J>(kv, 1u) <= k) return bits;
    float ak = INFINITY, ak1 = -INFINITY;
#pragma unroll
    for (int j = 0; j < J; ++j) {
        if (kv[j] == 0u) continue;
        if ((bits >> j) & 1u) ak = fminf(ak, v[j]);
        else ak1 = fmaxf(ak1, v[j]);
    }
    ak = wave_min(ak);
    ak1 = wave_max(ak1);
    if (ak - 2.0f * delta > ak1) return bits;
    *amb += 1;
    const float band_lo = ak - 2.0f * delta, band_hi = ak1 + 2.0f * delta;
    uint32_t cin = 0, ck[J];
    int cc = 0;
#pragma unroll
    for (int j = 0; j < J; ++j) {
        const bool valid = kv[j] != 0u, mem = (bits >> j) & 1u;
        const bool certain = mem && v[j] > band_hi;
        const bool inA = valid && !certain && v[j] >= band_lo;
        cin |= (certain ? 1u : 0u) << j;
        ck[j] = inA ? okey(canon(lane_id() + 64 * j)) : 0u;
        cc += __popcll(__ballot(certain));
    }
    return cin | exact_topk<J>(ck, k - cc);
}

// ------------------------------------------------------------------------------------------
// scores
// ------------------------------------------------------------------------------------------
// Canonical score: sequential fp32 FMA chain over d = 0..DH-1, then * scale (-0 -> +0).
// q comes from LDS, k from global; both are read with 16-byte vector loads, the chain order is
// unchanged.
template <int DT, int DH>
__device__ __noinline__ float canon_dot(const typename Elem<DT>::T* q,
                                        const typename Elem<DT>::T* k, float scale) {
    float acc = 0.0f;
    if constexpr (DT == HGA_DTYPE_BF16) {
        uint4 kr[DH / 8];
#pragma unroll
        for (int i = 0; i < DH / 8; ++i) kr[i] = *reinterpret_cast<const uint4*>(k + 8 * i);
#pragma unroll
        for (int i = 0; i < DH / 8; ++i) {
            const uint4 qq = *reinterpret_cast<const uint4*>(q + 8 * i);
            const uint32_t qw[4] = {qq.x, qq.y, qq.z, qq.w}, kw[4] = {kr[i].x, kr[i].y, kr[i].z, kr[i].w};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                acc = fmaf(__uint_as_float(qw[e] << 16), __uint_as_float(kw[e] << 16), acc);
                acc = fmaf(__uint_as_float(qw[e] & 0xffff0000u), __uint_as_float(kw[e] & 0xffff0000u), acc);
            }
        }
    } else {
        float4 kr[DH / 4];
#pragma unroll
        for (int i = 0; i < DH / 4; ++i) kr[i] = *reinterpret_cast<const float4*>(k + 4 * i);
#pragma unroll
        for (int i = 0; i < DH / 4; ++i) {
            const float4 qq = *reinterpret_cast<const float4*>(q + 4 * i);
            acc = fmaf(qq.x, kr[i].x, acc);
            acc = fmaf(qq.y, kr[i].y, acc);
            acc = fmaf(qq.z, kr[i].z, acc);
            acc = fmaf(qq.w, kr[i].w, acc);
        }
    }
    const float s = acc * scale;
    return s == 0.0f ? 0.0f : s;
}

__device__ __forceinline__ bf16x8 as_bf16x8(uint4 u) { return __builtin_bit_cast(bf16x8, u); }

__device__ __forceinline__ float sumsq_bf16x8(uint4 u) {
    float s = 0.0f;
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const float a = __uint_as_float(w[e] << 16), b = __uint_as_float(w[e] & 0xffff0000u);
        s = fmaf(a, a, s);
        s = fmaf(b, b, s);
    }
    return s;
}

// bf16 MFMA scores (scaled) of all rows against all candidates, plus candidate norms.
// Wave w handles candidate tiles w, w+8, ... of 32 candidates; both 32-row blocks.
template <int DH, int QS, class RowPtr>
__device__ void scores_mfma(const uint16_t* sQ, int rows, int ncand, RowPtr rowptr, float* sS,
                            int SP, float* sKn, float scale) {
    constexpr int KS = DH / 16;
    const int w = threadIdx.x / kWave, l = lane_id();
    const int nrb = rows > 32 ? 2 : 1;
    bf16x8 a0[KS], a1[KS];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
        const int col = ks * 16 + 8 * (l / 32);
        a0[ks] = as_bf16x8(*reinterpret_cast<const uint4*>(sQ + (l % 32) * QS + col));
        a1[ks] = as_bf16x8(*reinterpret_cast<const uint4*>(sQ + (32 + l % 32) * QS + col));
    }
    for (int ct = w; ct * 32 < ncand; ct += kWaves) {
        const int c = ct * 32 + l % 32;
        const bool cv = c < ncand;
        const uint16_t* kp = cv ? rowptr(c) : nullptr;
        uint4 u[KS];
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            u[ks] = make_uint4(0u, 0u, 0u, 0u);
            if (cv) u[ks] = *reinterpret_cast<const uint4*>(kp + ks * 16 + 8 * (l / 32));
        }
        floatx16 acc0 = {}, acc1 = {};
        float nsq = 0.0f;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            nsq += sumsq_bf16x8(u[ks]);
            const bf16x8 bv = as_bf16x8(u[ks]);
            acc0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a0[ks], bv, acc0, 0, 0, 0);
            if (nrb > 1) acc1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a1[ks], bv, acc1, 0, 0, 0);
        }
        nsq += __shfl_xor(nsq, 32, kWave);
        if (cv) {
            if (l < 32) sKn[c] = sqrtf(nsq);
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int row = 8 * (i / 4) + 4 * (l / 32) + (i % 4);
                sS[row * SP + c] = acc0[i] * scale;
                if (nrb > 1) sS[(32 + row) * SP + c] = acc1[i] * scale;
            }
        }
    }
}

template <int J>
struct JTag {
    static constexpr int value = J;
};
// Calls f(JTag<J>) with the smallest J such that 64*J >= n (wave-uniform n).
template <class F>
__device__ __forceinline__ void dispatch_j(int n, F&& f) {
    if (n <= 64) f(JTag<1>{});
    else if (n <= 128) f(JTag<2>{});
    else if (n <= 256) f(JTag<4>{});
    else f(JTag<8>{});
}

// Per-row top-k requests for rows w, w+8, ...: every member (row t, candidate i) raises the
// candidate's pooled key to okey(score), lowers its first row to t, and sets bit (t, i).
template <int J, class Vis, class Canon>
__device__ void row_requests(const float* sS, int SP, int rows, int ncand, int k, Vis visible,
                             const float* sQn, float dscale, Canon canon_row, uint32_t* sPk,
                             int* sFirst, uint32_t* sBits, int BW, int* amb) {
    const int w = threadIdx.x / kWave, l = lane_id();
    for (int t = w; t < rows; t += kWaves) {
        float v[J];
#pragma unroll
        for (int j = 0; j < J; ++j) {
            const int i = l + 64 * j;
            v[j] = (i < ncand && visible(t, i)) ? sS[t * SP + i] : -INFINITY;
        }
        const float delta = dscale * sQn[t];
        const uint32_t mem = select_certified<J>(
            v, k, delta, [&](int i) { return canon_row(t, i); }, amb);
#pragma unroll
        for (int j = 0; j < J; ++j) {
            const bool m = (mem >> j) & 1u;
            if (m) {
                const int i = l + 64 * j;
                atomicMax(&sPk[i], okey(v[j]));
                atomicMin(&sFirst[i], t);
            }
            const uint64_t bal = __ballot(m);
            if (l == 0 && 64 * j < SP) {
                sBits[t * BW + 2 * j] = (uint32_t)bal;
                if (2 * j + 1 < BW) sBits[t * BW + 2 * j + 1] = (uint32_t)(bal >> 32);
            }
        }
    }
}

// Canonical pooled value of candidate i: max over requesting rows whose approximate score can
// still be the maximum (within 2*dpool of the approximate pooled max).
template <class Canon>
__device__ float pooled_exact(int i, int rows, const float* sS, int SP, const uint32_t* sBits,
                              int BW, const uint32_t* sPk, float dpool, Canon canon_row) {
    const float pt = okey_inv(sPk[i]) - 2.0f * dpool;
    float best = -INFINITY;
    for (int t = 0; t < rows; ++t) {
        if (!((sBits[t * BW + i / 32] >> (i % 32)) & 1u)) continue;
        if (sS[t * SP + i] < pt) continue;
        best = fmaxf(best, canon_row(t, i));
    }
    return best;
}

// Wave 0: top-k of the requested candidates by pooled score (certified), optional forced
// candidate `ip` (evicting the last-ranked one when full), written ascending to sSel/sThr with
// ids base + i; returns the count (wave-uniform).
template <int J, class Canon>
__device__ int pooled_select(int ncand, int k, int rows, const float* sS, int SP,
                             const uint32_t* sBits, int BW, const uint32_t* sPk,
                             const int* sFirst, float dpool, Canon canon_row, int ip, int base_id,
                             int* sSel, int* sThr, int* amb) {
    const int l = lane_id();
    float v[J];
#pragma unroll
    for (int j = 0; j < J; ++j) {
        const int i = l + 64 * j;
        v[j] = (i < ncand && sFirst[i] < kNoRow) ? okey_inv(sPk[i]) : -INFINITY;
    }
    auto canon_pool = [&](int i) {
        return pooled_exact(i, rows, sS, SP, sBits, BW, sPk, dpool, canon_row);
    };
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
                mn = wave_min(mn);
                uint32_t ev[J];
#pragma unroll
                for (int j = 0; j < J; ++j) {
                    const bool cand = ((sel >> j) & 1u) && v[j] <= mn + 2.0f * dpool;
                    const float e = cand ? (dpool > 0.0f ? canon_pool(l + 64 * j) : v[j]) : 0.0f;
                    ev[j] = cand ? ~okey(e) : 0u;
                }
                uint32_t best = 0u;
#pragma unroll
                for (int j = 0; j < J; ++j) best = max(best, ev[j]);
                best = wave_max_u(best);
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
// the kernel
// ------------------------------------------------------------------------------------------
template <int DT, int DH>
__global__ __launch_bounds__(kThreads) void route_prefill_kernel(RouteArgs A) {
    typedef typename Elem<DT>::T T;
    constexpr int QS = DH + 8;   // padded LDS row stride of the query tile
    extern __shared__ __align__(16) unsigned char smem_raw[];
    const int SP = A.SP, BW = A.BW;
    float* sS = reinterpret_cast<float*>(smem_raw);                 // [64][SP]
    T* sQ = reinterpret_cast<T*>(sS + kRows * SP);                   // [64][QS]
    float* sKn = reinterpret_cast<float*>(sQ + kRows * QS);          // [SP]
    float* sQn = sKn + SP;                                           // [64]
    uint32_t* sPk = reinterpret_cast<uint32_t*>(sQn + kRows);        // [SP] pooled key
    int* sFirst = reinterpret_cast<int*>(sPk + SP);                  // [SP]
    uint32_t* sBits = reinterpret_cast<uint32_t*>(sFirst + SP);      // [64][BW]
    int* sSel = reinterpret_cast<int*>(sBits + kRows * BW);          // [kMaxSel] sorted chunk ids
    int* sThr = sSel + kMaxSel;                                      // [kMaxSel]
    int* sScal = sThr + kMaxSel;                                     // [8] scalars
    // Stage-2 group selections can be up to Kc*M long; they are emitted straight to global.

    const int N = A.N, C = A.C, M = A.M;
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
    const int Kcw = A.Kc > 0 ? A.Kc : 1, Kgw = A.Kg > 0 ? A.Kg : 1;
    int32_t* out_sc = A.sel_chunk + o * Kcw;
    int32_t* out_st = A.sel_thr + o * Kcw;
    int32_t* out_og = A.open_grp + o * Kgw;
    int32_t* out_ot = A.open_thr + o * Kgw;

    if (A.Kc == 0 || P == 0) {
        for (int i = threadIdx.x; i < Kcw; i += kThreads) out_sc[i] = out_st[i] = -1;
        for (int i = threadIdx.x; i < Kgw; i += kThreads) out_og[i] = out_ot[i] = -1;
        if (threadIdx.x == 0) A.n_sel[o] = A.n_open[o] = 0;
        return;
    }
    const bool use_mfma = (DT == HGA_DTYPE_BF16) && !A.canonical;
    const float scale = A.scale;
    int amb1 = 0, amb1p = 0, amb2 = 0, amb2p = 0;

    // ---- query rows -> LDS (rows >= `rows` zero), row norms --------------------------------
    {
        constexpr int VE = 16 / (int)sizeof(T);   // elements per 16-byte vector
        const T* qb = reinterpret_cast<const T*>(A.q) + b * A.q_sb + h * A.q_sh +
                      (int64_t)n * C * A.q_ss;
        for (int idx = threadIdx.x; idx < kRows * (DH / VE); idx += kThreads) {
            const int t = idx / (DH / VE), d = (idx % (DH / VE)) * VE;
            uint4 u = make_uint4(0u, 0u, 0u, 0u);
            if (t < rows) u = *reinterpret_cast<const uint4*>(qb + (int64_t)t * A.q_ss + d);
            *reinterpret_cast<uint4*>(sQ + t * QS + d) = u;
        }
    }
    for (int i = threadIdx.x; i < SP; i += kThreads) {
        sPk[i] = 0u;
        sFirst[i] = kNoRow;
    }
    for (int i = threadIdx.x; i < kRows * BW; i += kThreads) sBits[i] = 0u;
    __syncthreads();
    for (int t = w; t < kRows; t += kWaves) {
        float s = 0.0f;
        for (int d = l; d < DH; d += kWave) {
            const float x = Elem<DT>::ld(sQ, t * QS + d);
            s = fmaf(x, x, s);
        }
        s = wave_sum(s);
        if (l == 0) sQn[t] = sqrtf(s);
    }

    // ---- stage 1 scores ----------------------------------------------------------------------
    const T* ckb = reinterpret_cast<const T*>(A.ck) + b * A.ck_sb + kvh * A.ck_sh;
    auto crow = [&](int i) -> const T* { return ckb + (int64_t)(f_hi + i) * DH; };
    auto canon1 = [&](int t, int i) { return canon_dot<DT, DH>(sQ + t * QS, crow(i), scale); };
    if (use_mfma)
        scores_mfma<DH, QS>(reinterpret_cast<const uint16_t*>(sQ), rows, P,
                            [&](int i) { return reinterpret_cast<const uint16_t*>(crow(i)); },
                            sS, SP, sKn, scale);
    else
        for (int idx = threadIdx.x; idx < rows * P; idx += kThreads)
            sS[(idx / P) * SP + idx % P] = canon1(idx / P, idx % P);
    __syncthreads();
    float knmax = 0.0f, qnmax = 0.0f;
    if (use_mfma) {
        float x = 0.0f;
        for (int i = l; i < P; i += kWave) x = fmaxf(x, sKn[i]);
        knmax = wave_max(x);
        qnmax = wave_max(l < rows ? sQn[l] : 0.0f);
    }
    const float ds1 = use_mfma ? kDeltaRel * knmax * scale * 1.01f : 0.0f;

    // ---- stage 1 per-row requests ------------------------------------------------------------
    const int kreq = A.Kc < P ? A.Kc : P;
    dispatch_j(P, [&](auto jt) {
        constexpr int J = decltype(jt)::value;
        row_requests<J>(sS, SP, rows, P, kreq, [](int, int) { return true; }, sQn, ds1, canon1,
                        sPk, sFirst, sBits, BW, &amb1);
    });
    __syncthreads();

    // ---- stage 1 pooled selection + forced previous chunk (wave 0) -------------------------
    const float dpool = ds1 * qnmax;
    if (w == 0) {
        const int prev = n - 1;
        const int ip = (n > 0 && prev >= f_hi && prev < l_lo) ? prev - f_hi : -1;
        int cnt = 0;
        dispatch_j(P, [&](auto jt) {
            constexpr int J = decltype(jt)::value;
            cnt = pooled_select<J>(P, A.Kc, rows, sS, SP, sBits, BW, sPk, sFirst, dpool, canon1,
                                   ip, f_hi, sSel, sThr, &amb1p);
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

    // ---- stage 2: groups of the selected chunks ---------------------------------------------
    const int T2 = nsel * M;
    if (A.Kg == 0 || A.Kgr == 0 || nsel == 0) {
        for (int i = threadIdx.x; i < Kgw; i += kThreads) out_og[i] = out_ot[i] = -1;
        if (threadIdx.x == 0) A.n_open[o] = 0;
    } else {
        for (int i = threadIdx.x; i < SP; i += kThreads) {
            sPk[i] = 0u;
            sFirst[i] = kNoRow;
        }
        for (int i = threadIdx.x; i < kRows * BW; i += kThreads) sBits[i] = 0u;
        const T* gkb = reinterpret_cast<const T*>(A.gk) + b * A.gk_sb + kvh * A.gk_sh;
        auto grow = [&](int i) -> const T* {
            return gkb + ((int64_t)sSel[i / M] * M + (i % M)) * DH;
        };
        auto canon2 = [&](int t, int i) { return canon_dot<DT, DH>(sQ + t * QS, grow(i), scale); };
        if (use_mfma)
            scores_mfma<DH, QS>(reinterpret_cast<const uint16_t*>(sQ), rows, T2,
                                [&](int i) { return reinterpret_cast<const uint16_t*>(grow(i)); },
                                sS, SP, sKn, scale);
        else
            for (int idx = threadIdx.x; idx < rows * T2; idx += kThreads)
                sS[(idx / T2) * SP + idx % T2] = canon2(idx / T2, idx % T2);
        __syncthreads();
        float kn2 = 0.0f;
        if (use_mfma) {
            float x = 0.0f;
            for (int i = l; i < T2; i += kWave) x = fmaxf(x, sKn[i]);
            kn2 = wave_max(x);
        }
        const float ds2 = use_mfma ? kDeltaRel * kn2 * scale * 1.01f : 0.0f;
        dispatch_j(T2, [&](auto jt) {
            constexpr int J = decltype(jt)::value;
            row_requests<J>(sS, SP, rows, T2, A.Kgr,
                            [&](int t, int i) { return sThr[i / M] <= t; }, sQn, ds2, canon2, sPk,
                            sFirst, sBits, BW, &amb2);
        });
        __syncthreads();
        if (w == 0) {
            int cnt = 0;
            const float dpool2 = ds2 * qnmax;
            dispatch_j(T2, [&](auto jt) {
                constexpr int J = decltype(jt)::value;
                const int l2 = lane_id();
                float v[J];
#pragma unroll
                for (int j = 0; j < J; ++j) {
                    const int i = l2 + 64 * j;
                    v[j] = (i < T2 && sFirst[i] < kNoRow) ? okey_inv(sPk[i]) : -INFINITY;
                }
                auto canon_pool2 = [&](int i) {
                    return pooled_exact(i, rows, sS, SP, sBits, BW, sPk, dpool2, canon2);
                };
                const uint32_t op = select_certified<J>(v, A.Kg, dpool2, canon_pool2, &amb2p);
                int base = 0;
#pragma unroll
                for (int j = 0; j < J; ++j) {
                    const bool m = (op >> j) & 1u;
                    const uint64_t bal = __ballot(m);
                    if (m) {
                        const int i = l2 + 64 * j;
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
    }
    if (A.stats && l == 0) {
        if (amb1) atomicAdd(&A.stats[0], amb1);
        if (amb1p) atomicAdd(&A.stats[1], amb1p);
        if (amb2) atomicAdd(&A.stats[2], amb2);
        if (amb2p) atomicAdd(&A.stats[3], amb2p);
    }
}

template <int DT, int DH>
int launch_route(const RouteArgs& a, size_t lds, hipStream_t st) {
    auto kern = route_prefill_kernel<DT, DH>;
    static bool attr_done = false;
    if (!attr_done) {
        if (hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize,
                                163840) != hipSuccess) {
            set_error("hga_route_prefill: cannot raise the LDS limit");
            return HGA_ERR_LAUNCH;
        }
        attr_done = true;
    }
    const unsigned grid = (unsigned)(a.B * a.H * a.N);
    kern<<<dim3(grid), dim3(kThreads), lds, st>>>(a);
    return launch_status("hga_route_prefill");
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
    a.N = (S + a.C - 1) / a.C;
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
    HGA_REQUIRE(a.Kc <= kMaxSel, HGA_ERR_UNSUPPORTED, "hga_route_prefill: top-k chunks %d > %d",
                a.Kc, kMaxSel);
    HGA_REQUIRE(Pmax <= kJ * 64 && T2max <= kJ * 64, HGA_ERR_UNSUPPORTED,
                "hga_route_prefill: routing pool %d / group candidates %d exceed %d", Pmax,
                T2max, kJ * 64);
    int SP = (Pmax > T2max ? Pmax : T2max) + 1;
    if (SP % 2 == 0) ++SP;
    a.SP = SP;
    a.BW = (SP + 31) / 32;
    const int D = cfg->head_dim;
    const size_t esz = cfg->dtype == HGA_DTYPE_BF16 ? 2 : 4;
    const size_t lds = sizeof(float) * (size_t)kRows * SP + esz * kRows * (D + 8) +
                       sizeof(float) * (SP + kRows) + sizeof(uint32_t) * SP + sizeof(int) * SP +
                       sizeof(uint32_t) * (size_t)kRows * a.BW + sizeof(int) * 2 * kMaxSel +
                       sizeof(int) * 8 + sizeof(float) * 8;
    HGA_REQUIRE(lds <= 163840, HGA_ERR_UNSUPPORTED,
                "hga_route_prefill: %zu bytes of LDS needed (pool %d, head_dim %d)", lds, Pmax, D);
    {
        const int64_t ve = cfg->dtype == HGA_DTYPE_BF16 ? 8 : 4;   // elements per 16 bytes
        const uintptr_t al = (uintptr_t)chunk_k | (uintptr_t)group_k | (uintptr_t)q;
        HGA_REQUIRE(al % 16 == 0 && ((ck_sb | ck_sh | gk_sb | gk_sh | q_sb | q_sh | q_ss) % ve) == 0,
                    HGA_ERR_ARG, "hga_route_prefill: q and summaries need 16-byte aligned rows");
    }
    hipStream_t st = (hipStream_t)stream;
#define HGA_ROUTE_CASE(DTV, DHV) \
    if (cfg->dtype == DTV && D == DHV) return launch_route<DTV, DHV>(a, lds, st);
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
