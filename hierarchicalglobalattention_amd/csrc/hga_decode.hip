// Decode path: routing of an L-token block inside the active chunk (ChunkRouter._route_decision,
// chunk_router.py:187-277) and the attention over its working set (decode_block,
// chunk_router.py:279-407).
//
// Router: one 256-thread workgroup per (batch, query head).  Decode scores are few (L rows x
// pool), so they are computed directly with the canonical fp32 FMA chain (no MFMA pre-pass, no
// certification needed).  Stage 1 is split over workgroups: route_decode_part_kernel (grid: pool
// segments x (batch, head)) scores one segment of the pool for the block's rows and writes the
// segment's exact top-Kc of every row and of the pooled (max over rows) scores into a workspace;
// route_decode_kernel merges the segments' lists with one exact wave top-k per list (top-k of a
// union = top-k of the union of the parts' top-k; segments hold ascending id ranges and their
// lists are id-sorted, so candidate order is id order and ties still go to the lower id), then
// forces the previous chunk and runs stage 2.  Any pool length routes exactly as a single pass.
//
// Attention: one 256-thread workgroup per (batch, query head); the key sequence [first window |
// last window | opened groups | active chunk] is split over the 4 waves, lanes score one key
// each (16-byte loads of the key row), the online softmax runs per wave, values are
// accumulated with lanes over the head dim, and the 4 partial states are merged in LDS.  Opened
// groups can be read straight from a pinned host record (zero copy over PCIe), so only the
// routed groups cross the link.
#include "hga_common.h"
#include "hga_select.h"

#include <mutex>

namespace hga {
namespace {

constexpr int kDT = 256;            // threads
constexpr int kDW = kDT / kWave;     // waves
constexpr int kMaxL = 64;
constexpr int kDecJ = 32;            // wave selections over <= 2048 candidates
constexpr int kDecSegJ = 32;         // stage-1 segment: <= 64 * kDecSegJ chunks

// Work item (inner, outer) of the calling workgroup in a grid (inner, outer) whose outer index
// runs over (batch, query head).  Workgroups go to the 8 XCDs round-robin by linear id and each
// XCD has its own L2; when the inner count is not a multiple of 8, adjacent heads (those sharing
// a KV head, which read the same summaries and window keys) would land on different XCDs, so the
// linear id is permuted to give XCD k the contiguous item range [k n/8, (k+1) n/8).  Otherwise
// (inner count a multiple of 8: each inner index of every head already stays on one XCD, or
// n not a multiple of 8) the identity is kept.  A bijection on [0, n) either way.
__device__ __forceinline__ void xcd_item(int& inner, int& outer) {
    const int64_t ni = gridDim.x, n = ni * gridDim.y;
    int64_t x = blockIdx.x + ni * blockIdx.y;
    if ((ni & 7) != 0 && (n & 7) == 0) x = (x & 7) * (n >> 3) + (x >> 3);
    inner = (int)(x % ni);
    outer = (int)(x / ni);
}

struct DecRouteArgs {
    const void* q;
    int64_t q_sb, q_sh, q_ss;
    const void* ck;
    int64_t ck_sb, ck_sh;
    const void* gk;
    int64_t gk_sb, gk_sh;
    int32_t *mid, *mid_thr, *n_mid, *open_grp, *open_thr, *n_open;
    int B, H, KVH, L, n_closed, M, kf, kl, Kc, Kg, Kgr, SPD;
    int seg, nseg;  // stage-1 pool segment length and count (one scoring workgroup each)
    int SPW;        // row stride of the stage-1 scores (the pool length)
    float* ws;      // workspace: stage-1 scores [B*H][L][SPW]
    float* wv;      // segments' pooled top-Kc values [B*H][nseg][Kc] (id-sorted, -inf padded)
    int32_t* wi;    // and their chunk offsets in the pool (-1 padded)
    float scale;
};

// Wave-wide exact top-k of LDS values vals[0..n) (-inf excluded); returns member bits.
template <int J>
__device__ __forceinline__ uint32_t topk_lds(const float* vals, int n, int k) {
    const int l = lane_id();
    float v[J];
    uint32_t kv[J];
#pragma unroll
    for (int j = 0; j < J; ++j) {
        const int i = l + 64 * j;
        v[j] = i < n ? vals[i] : -INFINITY;
        kv[j] = v[j] == -INFINITY ? 0u : okey(v[j]);
    }
    return exact_topk<J>(kv, v, k);
}

// Canonical scores (sequential fp32 FMA chain over d, then * scale, -0 -> +0) of one key row
// against query rows [r0, r1) held in LDS as fp32; score r goes to out[r * stride] and the max
// over those rows is returned.  The key row is widened to fp32 once and kept in registers (bf16
// widening is exact), every lane of a wave reads the same query element at a time (LDS
// broadcast), and four rows' chains are interleaved (each keeps its own order).
__device__ __forceinline__ float fin_score(float acc, float scale) {
    const float sc = acc * scale;
    return sc == 0.0f ? 0.0f : sc;
}
template <int DT, int DH>
__device__ __forceinline__ float score_key_rows(const float* sQ, int r0, int r1,
                                                const typename Elem<DT>::T* kg, float* out,
                                                int64_t stride, float scale) {
    float kf[DH];
    if constexpr (DT == HGA_DTYPE_BF16) {
#pragma unroll
        for (int v = 0; v < DH / 8; ++v) {
            const uint4 u = reinterpret_cast<const uint4*>(kg)[v];
            const uint32_t w4[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                kf[8 * v + 2 * e] = __uint_as_float(w4[e] << 16);
                kf[8 * v + 2 * e + 1] = __uint_as_float(w4[e] & 0xffff0000u);
            }
        }
    } else {
#pragma unroll
        for (int v = 0; v < DH / 4; ++v) {
            const float4 f = reinterpret_cast<const float4*>(kg)[v];
            kf[4 * v] = f.x;
            kf[4 * v + 1] = f.y;
            kf[4 * v + 2] = f.z;
            kf[4 * v + 3] = f.w;
        }
    }
    float mx = -INFINITY;
    int r = r0;
    for (; r + 4 <= r1; r += 4) {
        const float4* q0 = reinterpret_cast<const float4*>(sQ + r * DH);
        constexpr int NV = DH / 4;
        float a0 = 0.0f, a1 = 0.0f, a2 = 0.0f, a3 = 0.0f;
#pragma unroll
        for (int v = 0; v < NV; ++v) {
            const float4 x0 = q0[v], x1 = q0[NV + v], x2 = q0[2 * NV + v], x3 = q0[3 * NV + v];
            a0 = fmaf(x0.x, kf[4 * v], a0);
            a1 = fmaf(x1.x, kf[4 * v], a1);
            a2 = fmaf(x2.x, kf[4 * v], a2);
            a3 = fmaf(x3.x, kf[4 * v], a3);
            a0 = fmaf(x0.y, kf[4 * v + 1], a0);
            a1 = fmaf(x1.y, kf[4 * v + 1], a1);
            a2 = fmaf(x2.y, kf[4 * v + 1], a2);
            a3 = fmaf(x3.y, kf[4 * v + 1], a3);
            a0 = fmaf(x0.z, kf[4 * v + 2], a0);
            a1 = fmaf(x1.z, kf[4 * v + 2], a1);
            a2 = fmaf(x2.z, kf[4 * v + 2], a2);
            a3 = fmaf(x3.z, kf[4 * v + 2], a3);
            a0 = fmaf(x0.w, kf[4 * v + 3], a0);
            a1 = fmaf(x1.w, kf[4 * v + 3], a1);
            a2 = fmaf(x2.w, kf[4 * v + 3], a2);
            a3 = fmaf(x3.w, kf[4 * v + 3], a3);
        }
        const float s0 = fin_score(a0, scale), s1 = fin_score(a1, scale);
        const float s2 = fin_score(a2, scale), s3 = fin_score(a3, scale);
        out[r * stride] = s0;
        out[(r + 1) * stride] = s1;
        out[(r + 2) * stride] = s2;
        out[(r + 3) * stride] = s3;
        mx = fmaxf(mx, fmaxf(fmaxf(s0, s1), fmaxf(s2, s3)));
    }
    for (; r < r1; ++r) {
        const float4* qv = reinterpret_cast<const float4*>(sQ + r * DH);
        float acc = 0.0f;
#pragma unroll
        for (int v = 0; v < DH / 4; ++v) {
            const float4 x = qv[v];
            acc = fmaf(x.x, kf[4 * v], acc);
            acc = fmaf(x.y, kf[4 * v + 1], acc);
            acc = fmaf(x.z, kf[4 * v + 2], acc);
            acc = fmaf(x.w, kf[4 * v + 3], acc);
        }
        const float sc = fin_score(acc, scale);
        out[r * stride] = sc;
        mx = fmaxf(mx, sc);
    }
    return mx;
}

// Query rows [L][DH] of (b, h) into LDS as fp32 (exact widening of bf16).
template <int DT, int DH>
__device__ __forceinline__ void load_q_f32(const DecRouteArgs& A, int b, int h, float* sQ,
                                           int nthreads) {
    typedef typename Elem<DT>::T T;
    const T* qg = reinterpret_cast<const T*>(A.q) + b * A.q_sb + h * A.q_sh;
    for (int idx = threadIdx.x; idx < A.L * DH; idx += nthreads) {
        const int r = idx / DH, d = idx % DH;
        sQ[idx] = Elem<DT>::ld(qg, (int64_t)r * A.q_ss + d);
    }
}

// Row groups of the scoring loops: blocks of 16+ rows split a key's rows over 4 thread groups.
__host__ __device__ __forceinline__ int score_row_groups(int L) { return L >= 16 ? 4 : 1; }

// Exact top-k (ties -> lower position) of LDS values vals[0..n) (-inf excluded), written in
// position order to ov/oi (ids id0 + position), -inf / -1 past its length.
template <int J>
__device__ __forceinline__ void topk_to(const float* vals, int n, int k, int id0, float* ov,
                                        int32_t* oi) {
    const int l = lane_id();
    float v[J];
    uint32_t kv[J];
#pragma unroll
    for (int j = 0; j < J; ++j) {
        const int i = l + 64 * j;
        v[j] = i < n ? vals[i] : -INFINITY;
        kv[j] = v[j] == -INFINITY ? 0u : okey(v[j]);
    }
    const uint32_t mem = exact_topk<J>(kv, v, k);
    int base = 0;
#pragma unroll
    for (int j = 0; j < J; ++j) {
        const bool m = (mem >> j) & 1u;
        const uint64_t bal = __ballot(m);
        if (m) {
            ov[base + lanes_below(bal)] = v[j];
            oi[base + lanes_below(bal)] = id0 + l + 64 * j;
        }
        base += __popcll(bal);
    }
    for (int i = base + l; i < k; i += kWave) {
        ov[i] = -INFINITY;
        oi[i] = -1;
    }
}

// Exact top-k of the candidate lists of nseg segments (k entries each, id-sorted, -inf padded,
// consecutive): position order is id order, so ties go to the lower id.  Writes the values and
// ids in id order to LDS, -inf / -1 past its length.
template <int J>
__device__ __forceinline__ void merge_segments(const float* cv, const int32_t* ci, int n, int k,
                                               float* dv, int* di) {
    const int l = lane_id();
    float v[J];
    uint32_t kv[J];
    int id[J];
#pragma unroll
    for (int j = 0; j < J; ++j) {
        const int i = l + 64 * j;
        v[j] = i < n ? cv[i] : -INFINITY;
        id[j] = i < n ? ci[i] : -1;
        kv[j] = v[j] == -INFINITY ? 0u : okey(v[j]);
    }
    const uint32_t mem = exact_topk<J>(kv, v, k);
    int base = 0;
#pragma unroll
    for (int j = 0; j < J; ++j) {
        const bool m = (mem >> j) & 1u;
        const uint64_t bal = __ballot(m);
        if (m) {
            di[base + lanes_below(bal)] = id[j];
            dv[base + lanes_below(bal)] = v[j];
        }
        base += __popcll(bal);
    }
    for (int i = base + l; i < k; i += kWave) {
        di[i] = -1;
        dv[i] = -INFINITY;
    }
}

// Whether row `row` (values vals[0..n), candidate ids 0..n-1) ranks each of the wave's open
// candidates (lanes in `open`, lane p holding its value sp and id cp) among its top k: fewer
// than k candidates larger, or equal with a lower id -- membership in the row's exact top-k
// under the canonical ranking, without selecting it.  Returns the lanes that are members.
__device__ __forceinline__ uint64_t ranked_in(const float* vals, int n, uint64_t open, float sp,
                                              int cp, int k) {
    constexpr int U = 4;                      // 64-candidate blocks loaded together
    const int l = lane_id();
    int cnt = 0;
    for (int i0 = 0; i0 < n && open; i0 += U * kWave) {
        float v[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int i = i0 + u * kWave + l;
            v[u] = i < n ? vals[i] : -INFINITY;   // -inf never ranks above a score
        }
        uint64_t m = open;
        while (m) {
            const int p = __builtin_ctzll(m);
            m &= m - 1ull;
            const float s = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(sp), p));
            const int c = __builtin_amdgcn_readlane(cp, p);
            int add = 0;
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int i = i0 + u * kWave + l;
                add += (int)__popcll(__ballot(v[u] > s || (v[u] == s && i < c)));
            }
            if (l == p) cnt += add;
        }
        open &= __ballot(cnt < k);
    }
    return open;
}

// Stage-1 scoring of one pool segment: canonical scores of the block's L rows (to the
// workspace, row stride SPW), their max over the rows, and the segment's pooled top-Kc
// (chunk_router.py:219-231).
template <int DT, int DH>
__global__ __launch_bounds__(kDT) void route_decode_part_kernel(DecRouteArgs A) {
    typedef typename Elem<DT>::T T;
    extern __shared__ __align__(16) unsigned char smem_raw[];
    const int L = A.L, K = A.Kc;
    float* sQ = reinterpret_cast<float*>(smem_raw);             // [L][DH] fp32
    float* sPool = sQ + L * DH;                                 // [RG][seg] partial maxima
    int sg, bh;
    xcd_item(sg, bh);
    const int b = bh / A.H, h = bh % A.H;
    const int kvh = h / (A.H / A.KVH);
    int f_hi, l_lo;
    windows(A.n_closed, A.kf, A.kl, &f_hi, &l_lo);
    const int nmid = l_lo > f_hi ? l_lo - f_hi : 0;
    const int s0 = sg * A.seg, sl = min(A.seg, nmid - s0);   // s0 < nmid (host grid)
    const int NT = (int)blockDim.x;                              // 64 (L <= 4) or 256 threads
    load_q_f32<DT, DH>(A, b, h, sQ, NT);
    __syncthreads();
    const T* ckb = reinterpret_cast<const T*>(A.ck) + b * A.ck_sb + kvh * A.ck_sh +
                   (int64_t)(f_hi + s0) * DH;
    float* srow = L > 1 ? A.ws + (int64_t)bh * L * A.SPW + s0 : nullptr;
    {
        const int RG = score_row_groups(L), KP = NT / RG, rg = threadIdx.x / KP;
        const int rpg = (L + RG - 1) / RG, r0 = min(L, rg * rpg), r1 = min(L, r0 + rpg);
        // a one-row block needs only the pooled score (its rows request the whole selection)
        for (int i = threadIdx.x % KP; i < sl; i += KP)
            sPool[rg * A.seg + i] = score_key_rows<DT, DH>(
                sQ, r0, r1, ckb + (int64_t)i * DH, L == 1 ? sPool + i : srow + i, A.SPW, A.scale);
        __syncthreads();
        for (int i = threadIdx.x; i < sl; i += NT) {           // pooled over all rows (:227)
            float m = sPool[i];
            for (int g = 1; g < RG; ++g) m = fmaxf(m, sPool[g * A.seg + i]);
            sPool[i] = m;
        }
    }
    __syncthreads();
    if (threadIdx.x < kWave) {
        const int64_t o = ((int64_t)bh * A.nseg + sg) * K;
        dispatch_j<kDecSegJ>(sl, [&](auto jt) {
            constexpr int J = decltype(jt)::value;
            topk_to<J>(sPool, sl, K, s0, A.wv + o, A.wi + o);
        });
    }
}

template <int DT, int DH>
__global__ __launch_bounds__(kDT) void route_decode_kernel(DecRouteArgs A) {
    typedef typename Elem<DT>::T T;
    extern __shared__ __align__(16) unsigned char smem_raw[];
    const int SPD = A.SPD, M = A.M, L = A.L;
    float* sQ = reinterpret_cast<float*>(smem_raw);             // [L][DH] fp32
    float* sS = sQ + L * DH;                                    // [L][SPD] group scores
    float* sPool = sS + L * SPD;                                // [SPD]
    int* sFirst = reinterpret_cast<int*>(sPool + SPD);          // [SPD] first requesting row
    int* sSel = sFirst + SPD;                                   // [64] sorted chunk ids
    int* sThr = sSel + 64;                                      // [64] -1 = never visible
    int* sScal = sThr + 64;                                     // [8]
    int* sOp = sScal + 8;                                       // [256] opened candidates
    int* sPI = sOp + 256;                                       // [Kc] pooled selection ids

    int one, bh;
    xcd_item(one, bh);   // grid (1, B*H)
    const int b = bh / A.H, h = bh % A.H, kvh = h / (A.H / A.KVH);
    const int w = threadIdx.x / kWave, l = lane_id();
    int f_hi, l_lo;
    windows(A.n_closed, A.kf, A.kl, &f_hi, &l_lo);
    const int nmid = l_lo > f_hi ? l_lo - f_hi : 0;
    const int Kcw = A.Kc > 0 ? A.Kc : 1, Kgw = A.Kg > 0 ? A.Kg : 1;
    int32_t* o_mid = A.mid + (int64_t)bh * Kcw;
    int32_t* o_mth = A.mid_thr + (int64_t)bh * Kcw;
    int32_t* o_og = A.open_grp + (int64_t)bh * Kgw;
    int32_t* o_ot = A.open_thr + (int64_t)bh * Kgw;
    if (A.Kc == 0) {
        for (int i = threadIdx.x; i < Kcw; i += kDT) o_mid[i] = o_mth[i] = -1;
        for (int i = threadIdx.x; i < Kgw; i += kDT) o_og[i] = o_ot[i] = -1;
        if (threadIdx.x == 0) A.n_mid[bh] = A.n_open[bh] = 0;
        return;
    }
    const float scale = A.scale;
    const int K = A.Kc;
    load_q_f32<DT, DH>(A, b, h, sQ, kDT);
    // ---- stage 1: pooled selection = top-Kc of the segments' pooled lists (:227, :231) ------
    if (w == 0) {
        const int64_t o = (int64_t)bh * A.nseg * K;
        dispatch_j<kDecJ>(A.nseg * K, [&](auto jt) {
            constexpr int J = decltype(jt)::value;
            merge_segments<J>(A.wv + o, A.wi + o, A.nseg * K, K, sPool, sPI);
        });
    }
    __syncthreads();
    if (w == 0) {
        // forced previous chunk (:232-241); K <= 64, one list entry per lane
        const int prev = A.n_closed - 1;
        const int ip = (prev >= f_hi && prev < l_lo) ? prev - f_hi : -1;
        const int id = l < K ? sPI[l] : -1;
        bool m = id >= 0;
        const bool forced = ip >= 0 && __ballot(m && id == ip) == 0;
        if (forced) {
            // evict the last-ranked selected chunk (lowest pooled score, highest id)
            const uint32_t ok = m ? okey(sPool[l]) : 0xffffffffu;
            const uint32_t worst = (uint32_t)wave_reduce_bits((int)ok, [](int a, int c) {
                return (int)min((uint32_t)a, (uint32_t)c);
            });
            const uint64_t cand = __ballot(m && ok == worst);
            if (cand && l == 63 - __clzll(cand)) m = false;
        }
        // ip >= 0 only when the last window is empty, so ip is the pool's highest id and goes last
        const uint64_t bal = __ballot(m);
        const int nkeep = __popcll(bal);
        if (m) sSel[lanes_below(bal)] = f_hi + id;
        if (forced && l == 0) sSel[nkeep] = f_hi + ip;
        const uint64_t fb = __ballot(m && id == ip);          // ip selected on its own
        const int fl = fb ? 63 - __clzll(fb) : -1;
        const int ns = nkeep + (forced ? 1 : 0);
        if (l == 0) {
            sScal[0] = ns;
            sScal[1] = forced ? nkeep : (fl >= 0 ? __popcll(bal & ((1ull << fl) - 1ull)) : -1);
        }
        // one row: its own top-Kc is the pooled selection, so row 0 requests every selected chunk
        if (l < ns) sFirst[l] = L == 1 ? 0 : kNoRow;          // ns <= Kc < SPD
    }
    __syncthreads();
    if (L > 1) {
        // first row whose own top-Kc holds each selected chunk (:230, :243-250), by rank
        const int ns = sScal[0];
        const int c = l < ns ? sSel[l] - f_hi : 0;
        for (int r = w; r < L; r += kDW) {
            const float* row = A.ws + ((int64_t)bh * L + r) * A.SPW;
            const uint64_t open = __ballot(l < ns && sFirst[l] > r);
            if (!open) continue;
            const float sp = l < ns ? row[c] : 0.0f;
            const uint64_t req = ranked_in(row, nmid, open, sp, c, K);
            if ((req >> l) & 1ull) atomicMin(&sFirst[l], r);
        }
    }
    __syncthreads();
    if (w == 0) {
        const int ns = sScal[0], fpos = sScal[1];
        const int thr = l >= ns ? -1 : (l == fpos ? 0 : (sFirst[l] < kNoRow ? sFirst[l] : -1));
        if (l < ns) sThr[l] = thr;
        const uint64_t vb = __ballot(l < ns && thr >= 0);
        if (l < ns && thr >= 0) {
            o_mid[lanes_below(vb)] = sSel[l];
            o_mth[lanes_below(vb)] = thr;
        }
        const int nvis = __popcll(vb);
        for (int i = nvis + l; i < Kcw; i += kWave) o_mid[i] = o_mth[i] = -1;
        if (l == 0) A.n_mid[bh] = nvis;
    }
    __syncthreads();
    const int nsel = sScal[0];
    const int T2 = nsel * M;
    if (A.Kg == 0 || T2 == 0) {
        for (int i = threadIdx.x; i < Kgw; i += kDT) o_og[i] = o_ot[i] = -1;
        if (threadIdx.x == 0) A.n_open[bh] = 0;
        return;
    }
    // ---- groups of the selected chunks (:256-276) --------------------------------------------
    const T* gkb = reinterpret_cast<const T*>(A.gk) + b * A.gk_sb + kvh * A.gk_sh;
    {
        const int RG = score_row_groups(L), KP = kDT / RG, rg = threadIdx.x / KP;
        const int rpg = (L + RG - 1) / RG, r0 = min(L, rg * rpg), r1 = min(L, r0 + rpg);
        for (int i = threadIdx.x % KP; i < T2; i += KP)
            score_key_rows<DT, DH>(sQ, r0, r1, gkb + ((int64_t)sSel[i / M] * M + i % M) * DH,
                                   sS + i, SPD, scale);
    }
    __syncthreads();
    for (int i = threadIdx.x; i < T2; i += kDT) {             // pooled over all rows (:264)
        float m = -INFINITY;
        for (int r = 0; r < L; ++r) m = fmaxf(m, sS[r * SPD + i]);
        sPool[i] = m;
    }
    __syncthreads();
    if (w == 0) {
        // opened = pooled top-Kg (:265), ascending candidate order
        dispatch_j<kDecJ>(T2, [&](auto jt) {
            constexpr int J = decltype(jt)::value;
            const uint32_t op = topk_lds<J>(sPool, T2, A.Kg);
            int base = 0;
#pragma unroll
            for (int j = 0; j < J; ++j) {
                const bool m = (op >> j) & 1u;
                const uint64_t bal = __ballot(m);
                if (m) sOp[base + lanes_below(bal)] = l + 64 * j;
                base += __popcll(bal);
            }
            if (l == 0) sScal[2] = base;
        });
    }
    __syncthreads();
    const int nop = sScal[2];
    for (int i = threadIdx.x; i < nop; i += kDT) sFirst[i] = kNoRow;
    __syncthreads();
    // each row requests its own top-Kgr groups (:266); first requesting row by rank -- a one-row
    // block's requests are its top-Kgr, one selection over the candidates
    if (L == 1 && w == 0) {
        dispatch_j<kDecJ>(T2, [&](auto jt) {
            constexpr int J = decltype(jt)::value;
            const uint32_t req = topk_lds<J>(sS, T2, A.Kgr);
            // opened candidates are ascending: find each requested candidate's opened slot
#pragma unroll
            for (int j = 0; j < J; ++j)
                if ((req >> j) & 1u) {
                    const int c = l + 64 * j;
                    int lo = 0, hi = nop;
                    while (lo < hi) {
                        const int mid = (lo + hi) >> 1;
                        if (sOp[mid] < c) lo = mid + 1;
                        else hi = mid;
                    }
                    if (lo < nop && sOp[lo] == c) sFirst[lo] = 0;
                }
        });
    }
    for (int r = L == 1 ? L : w; r < L; r += kDW) {
        const float* row = sS + r * SPD;
        for (int o0 = 0; o0 < nop; o0 += kWave) {
            const int o = o0 + l;
            const uint64_t open = __ballot(o < nop && sFirst[o] > r);
            if (!open) continue;
            const int c = o < nop ? sOp[o] : 0;
            const float sp = o < nop ? row[c] : 0.0f;
            const uint64_t req = ranked_in(row, T2, open, sp, c, A.Kgr);
            if ((req >> l) & 1ull) atomicMin(&sFirst[o], r);
        }
    }
    __syncthreads();
    if (w == 0) {
        // visible from max(first request, parent threshold) (:273-276)
        int base = 0;
        for (int o0 = 0; o0 < nop; o0 += kWave) {
            const int o = o0 + l;
            int thr = -1, grp = -1;
            if (o < nop) {
                const int i = sOp[o];
                grp = sSel[i / M] * M + i % M;
                if (sFirst[o] < kNoRow && sThr[i / M] >= 0)
                    thr = sFirst[o] > sThr[i / M] ? sFirst[o] : sThr[i / M];
            }
            const uint64_t bal = __ballot(thr >= 0);
            if (thr >= 0 && base + lanes_below(bal) < Kgw) {
                o_og[base + lanes_below(bal)] = grp;
                o_ot[base + lanes_below(bal)] = thr;
            }
            base += __popcll(bal);
        }
        for (int i = base + l; i < Kgw; i += kWave) o_og[i] = o_ot[i] = -1;
        if (l == 0) A.n_open[bh] = base;
    }
}

// ------------------------------------------------------------------------------------------
// decode attention
// ------------------------------------------------------------------------------------------
struct DecAttnArgs {
    const void* q;
    int64_t q_sb, q_sh, q_ss;
    const void *kr, *vr;
    int64_t r_sb, r_sh, r_ss;
    const void *kfst, *vfst;
    int64_t f_sb, f_sh, f_ss;
    const void *kd, *vd;
    int64_t d_sb, d_sh, d_ss;
    const int32_t* open_grp;
    const int32_t* open_thr;
    void* out;
    int64_t o_sb, o_sh, o_ss;
    int64_t start_pos;
    int B, H, KVH, L, n_closed, C, gs, M, kf, kl, Kg, ring;
    float scale;
    // Dual Chunk Attention (DCA kernels only): fp32 query rows RoPE'd at the intra, successive and
    // inter positions (strides q_sb/q_sh/q_ss), the opened groups' own ids for key positions
    // (the list attention reads may hold staging slots), the DCA chunk length
    const float* q_dca[3];
    const int32_t* open_pos;
    int dca_chunk;
    // split kernels: partial slots [0, n1) hold the windows and the active chunk, [n1, n1 + n2)
    // the opened groups; phase 0 launches all of them, phase 1 the first range, phase 2 the second
    int phase, n1;
};

// The key sequence of a decode block for (b, query head): [first window | last window | opened
// groups | active chunk], key k -> (key row, value row, first visible query row).  sOG/sOT hold
// the head's opened list in LDS; nopen is its valid length.
template <class T>
struct DecKeys {
    const T *kr, *vr, *kf, *vf, *kd, *vd;
    int64_t r_ss, f_ss, d_ss, c0;
    const int *sOG, *sOT, *sOP;
    int a1, a2, a3, a4, C, gs, M, n_closed, l_lo, ring;
    int n, skip;   // keys of the phase's sequence; phase 1 skips the opened groups, 2 the rest

    // ph: 0 the whole sequence, 1 [first | last | active], 2 [opened]
    __device__ void init(const DecAttnArgs& A, int b, int kvh, const int* og, const int* ot,
                         int nopen, int ph = 0) {
        int f_hi;
        windows(A.n_closed, A.kf, A.kl, &f_hi, &l_lo);
        C = A.C; gs = A.gs; M = A.M; n_closed = A.n_closed; ring = A.ring;
        sOG = og; sOT = ot; sOP = og;
        c0 = A.start_pos - (int64_t)A.n_closed * C;
        a1 = f_hi * C;
        a2 = a1 + (A.n_closed - l_lo) * C;
        a3 = a2 + nopen * gs;
        a4 = a3 + (int)c0 + A.L;
        n = ph == 1 ? a4 - (a3 - a2) : (ph == 2 ? a3 - a2 : a4);
        skip = ph;
        kr = reinterpret_cast<const T*>(A.kr) + b * A.r_sb + kvh * A.r_sh;
        vr = reinterpret_cast<const T*>(A.vr) + b * A.r_sb + kvh * A.r_sh;
        kf = reinterpret_cast<const T*>(A.kfst) + b * A.f_sb + kvh * A.f_sh;
        vf = reinterpret_cast<const T*>(A.vfst) + b * A.f_sb + kvh * A.f_sh;
        kd = reinterpret_cast<const T*>(A.kd) + b * A.d_sb + kvh * A.d_sh;
        vd = reinterpret_cast<const T*>(A.vd) + b * A.d_sb + kvh * A.d_sh;
        r_ss = A.r_ss; f_ss = A.f_ss; d_ss = A.d_ss;
    }
    // kpos: the key's absolute position (opened groups: from sOP, the groups' own ids); k is an
    // index into the phase's sequence (phase 1: [first | last | active], phase 2: [opened])
    __device__ void locate(int k, const T*& kp, const T*& vp, int& thr, int64_t& kpos) const {
        if (skip == 1 && k >= a2) k += a3 - a2;
        else if (skip == 2) k += a2;
        if (k < a1) {
            kp = kf + (int64_t)k * f_ss;
            vp = vf + (int64_t)k * f_ss;
            thr = 0;
            kpos = k;
            return;
        }
        int64_t pos;
        if (k < a2) {
            pos = (int64_t)l_lo * C + (k - a1);
            thr = 0;
        } else if (k < a3) {
            const int g = (k - a2) / gs, e = (k - a2) % gs, grp = sOG[g];
            if (grp < 0 || grp >= n_closed * M || sOT[g] < 0) {   // padding / invalid id
                kp = vp = nullptr;
                thr = kNoRow;
                kpos = 0;
                return;
            }
            const int64_t p = (int64_t)(grp / M) * C + (grp % M) * gs + e;
            kp = kd + p * d_ss;
            vp = vd + p * d_ss;
            thr = sOT[g];
            const int gp = sOP[g];
            kpos = (int64_t)(gp / M) * C + (gp % M) * gs + e;
            return;
        } else {
            pos = (int64_t)n_closed * C + (k - a3);
            thr = (int)((k - a3) - c0);
            if (thr < 0) thr = 0;
        }
        const int64_t slot = ring > 0 ? ((pos / C) % ring) * C + pos % C : pos;
        kp = kr + slot * r_ss;
        vp = vr + slot * r_ss;
        kpos = pos;
    }
    __device__ void locate(int k, const T*& kp, const T*& vp, int& thr) const {
        int64_t kpos;
        locate(k, kp, vp, thr, kpos);
    }
};

// DCA regime of a key for a query at qpos: 0 same DCA chunk, 1 the one before, 2 older
// (qwen_routed_attention.py:274-278)
__device__ __forceinline__ int dca_regime(int64_t kpos, int64_t qpos, int L_c) {
    const int64_t ck = kpos / L_c, cq = qpos / L_c;
    return ck == cq ? 0 : (ck == cq - 1 ? 1 : 2);
}

template <int DT, int DH, bool DCA>
__global__ __launch_bounds__(kDT) void attend_decode_kernel(DecAttnArgs A) {
    typedef typename Elem<DT>::T T;
    constexpr int DPL = DH / kWave > 0 ? DH / kWave : 1;   // dims per lane
    constexpr int NQ = DCA ? 3 : 1;                          // query versions
    __shared__ float sQv[NQ][DH];
    __shared__ float sM[kDW], sLs[kDW];
    __shared__ float sAcc[kDW][DH];
    __shared__ int sOG[256], sOT[256], sOP[DCA ? 256 : 1];
    const int bh = blockIdx.x, b = bh / A.H, h = bh % A.H, kvh = h / (A.H / A.KVH);
    const int w = threadIdx.x / kWave, l = lane_id();
    const int Kgw = A.Kg > 0 ? A.Kg : 1;
    for (int i = threadIdx.x; i < A.Kg; i += kDT) {
        sOG[i] = A.open_grp[(int64_t)bh * Kgw + i];
        sOT[i] = A.open_thr[(int64_t)bh * Kgw + i];
        if constexpr (DCA) sOP[i] = A.open_pos[(int64_t)bh * Kgw + i];
    }
    __syncthreads();
    int nopen = 0;
    for (int i = 0; i < A.Kg; ++i)
        if (sOG[i] >= 0 && sOT[i] >= 0) nopen = i + 1;
    DecKeys<T> keys;
    keys.init(A, b, kvh, sOG, sOT, nopen);
    if constexpr (DCA) keys.sOP = sOP;
    const int a4 = keys.a4;
    const int per = (a4 + kDW - 1) / kDW;
    const int k_lo = w * per, k_hi = (w + 1) * per < a4 ? (w + 1) * per : a4;
    const T* qg = reinterpret_cast<const T*>(A.q) + b * A.q_sb + h * A.q_sh;
    T* og = reinterpret_cast<T*>(A.out) + b * A.o_sb + h * A.o_sh;
    for (int row = 0; row < A.L; ++row) {
        for (int d = threadIdx.x; d < DH; d += kDT) {
            const int64_t o = (int64_t)row * A.q_ss + d;
            if constexpr (DCA) {
#pragma unroll
                for (int r = 0; r < 3; ++r) sQv[r][d] = A.q_dca[r][b * A.q_sb + h * A.q_sh + o];
            } else {
                sQv[0][d] = Elem<DT>::ld(qg, o);
            }
        }
        __syncthreads();
        float m_run = -INFINITY, l_run = 0.0f, acc[DPL];
#pragma unroll
        for (int e = 0; e < DPL; ++e) acc[e] = 0.0f;
        for (int base = k_lo; base < k_hi; base += kWave) {
            const int k = base + l;
            const T* kp = nullptr;
            const T* vp = nullptr;
            int thr = kNoRow;
            int64_t kpos = 0;
            if (k < k_hi) keys.locate(k, kp, vp, thr, kpos);
            const float* sQ = sQv[DCA ? dca_regime(kpos, A.start_pos + row, A.dca_chunk) : 0];
            float s = -INFINITY;
            if (k < k_hi && row >= thr) {
                float d0 = 0.0f;
                for (int d = 0; d < DH; d += 8) {
                    if constexpr (DT == HGA_DTYPE_BF16) {
                        const uint4 u = *reinterpret_cast<const uint4*>(kp + d);
                        const uint32_t wv[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            d0 = fmaf(sQ[d + 2 * e], __uint_as_float(wv[e] << 16), d0);
                            d0 = fmaf(sQ[d + 2 * e + 1], __uint_as_float(wv[e] & 0xffff0000u), d0);
                        }
                    } else {
                        const float4 u0 = *reinterpret_cast<const float4*>(kp + d);
                        const float4 u1 = *reinterpret_cast<const float4*>(kp + d + 4);
                        d0 = fmaf(sQ[d], u0.x, d0); d0 = fmaf(sQ[d + 1], u0.y, d0);
                        d0 = fmaf(sQ[d + 2], u0.z, d0); d0 = fmaf(sQ[d + 3], u0.w, d0);
                        d0 = fmaf(sQ[d + 4], u1.x, d0); d0 = fmaf(sQ[d + 5], u1.y, d0);
                        d0 = fmaf(sQ[d + 6], u1.z, d0); d0 = fmaf(sQ[d + 7], u1.w, d0);
                    }
                }
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
            const int lim = k_hi - base < kWave ? k_hi - base : kWave;
            const uint64_t vaddr = (uint64_t)vp;
            for (int kk = 0; kk < lim; ++kk) {
                const float pk = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(p), kk));
                if (pk == 0.0f) continue;
                const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)vaddr, kk);
                const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(vaddr >> 32), kk);
                const T* vrow = reinterpret_cast<const T*>(((uint64_t)hi << 32) | lo);
#pragma unroll
                for (int e = 0; e < DPL; ++e) {
                    const int d = l + kWave * e;
                    if (d < DH) acc[e] = fmaf(pk, Elem<DT>::ld(vrow, d), acc[e]);
                }
            }
        }
        if (l == 0) {
            sM[w] = m_run;
            sLs[w] = l_run;
        }
#pragma unroll
        for (int e = 0; e < DPL; ++e)
            if (l + kWave * e < DH) sAcc[w][l + kWave * e] = acc[e];
        __syncthreads();
        if (w == 0) {
            float mt = -INFINITY;
            for (int i = 0; i < kDW; ++i) mt = fmaxf(mt, sM[i]);
            const float mu = mt == -INFINITY ? 0.0f : mt;
            float lt = 0.0f;
            for (int i = 0; i < kDW; ++i) lt += sLs[i] * expf(sM[i] - mu);
            const float inv = lt > 0.0f ? 1.0f / lt : 0.0f;
            for (int d = l; d < DH; d += kWave) {
                float o = 0.0f;
                for (int i = 0; i < kDW; ++i) o += sAcc[i][d] * expf(sM[i] - mu);
                Elem<DT>::st(og, (int64_t)row * A.o_ss + d, o * inv);
            }
        }
        __syncthreads();
    }
}

// ------------------------------------------------------------------------------------------
// split decode attention (head_dim 64 / 128): the key sequence of each (b, head) in splits of
// SK keys (kSplitKeys or kWideSplitKeys), one workgroup per split; 16 lanes per key (a lane
// holds head_dim/16 consecutive dims, so a key row is one contiguous read), SK / 16 keys per
// 16-lane group, four in flight.  Each split writes its (max, sum, accumulator) partial; decode_combine_kernel merges.
// ------------------------------------------------------------------------------------------
constexpr int kSplitKeys = 256;
// One-token steps of large batches (B * H >= kWideSplitHeads) take splits of twice as many keys:
// half the workgroups, each locating its keys and merging its groups once for twice the work.
constexpr int kWideSplitKeys = 512;
constexpr int kWideSplitHeads = 512;

// Sum over the 16 lanes of a DPP row, bit-identical in all of them (butterfly: xor 1, xor 2,
// half-row mirror, row mirror).
__device__ __forceinline__ float r16_sum_f(float x) {
    x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0xB1, 0xf, 0xf, true));
    x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x4E, 0xf, 0xf, true));
    x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x141, 0xf, 0xf, true));
    x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x140, 0xf, 0xf, true));
    return x;
}

template <int DT, int DPL>
__device__ __forceinline__ void load_slice(const typename Elem<DT>::T* p, float (&x)[DPL]) {
    if constexpr (DT == HGA_DTYPE_BF16) {
        if constexpr (DPL == 8) {
            const uint4 u = *reinterpret_cast<const uint4*>(p);
            const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                x[2 * e] = __uint_as_float(w[e] << 16);
                x[2 * e + 1] = __uint_as_float(w[e] & 0xffff0000u);
            }
        } else {
            const uint2 u = *reinterpret_cast<const uint2*>(p);
            x[0] = __uint_as_float(u.x << 16);
            x[1] = __uint_as_float(u.x & 0xffff0000u);
            x[2] = __uint_as_float(u.y << 16);
            x[3] = __uint_as_float(u.y & 0xffff0000u);
        }
    } else {
#pragma unroll
        for (int e = 0; e < DPL; e += 4) {
            const float4 u = *reinterpret_cast<const float4*>(p + e);
            x[e] = u.x; x[e + 1] = u.y; x[e + 2] = u.z; x[e + 3] = u.w;
        }
    }
}

// A lane's DPL elements of a key or value row as loaded (bf16 pairs or fp32 words), widened to
// fp32 on use exactly as load_slice does.
template <int DT, int DPL>
struct RawSlice {
    static constexpr int NW = DT == HGA_DTYPE_BF16 ? DPL / 2 : DPL;
    uint32_t w[NW];
    __device__ __forceinline__ void load(const typename Elem<DT>::T* p) {
        if constexpr (DT == HGA_DTYPE_BF16 && DPL == 8) {
            const uint4 u = *reinterpret_cast<const uint4*>(p);
            w[0] = u.x; w[1] = u.y; w[2] = u.z; w[3] = u.w;
        } else if constexpr (DT == HGA_DTYPE_BF16) {
            const uint2 u = *reinterpret_cast<const uint2*>(p);
            w[0] = u.x; w[1] = u.y;
        } else {
#pragma unroll
            for (int e = 0; e < DPL; e += 4) {
                const uint4 u = *reinterpret_cast<const uint4*>(p + e);
                w[e] = u.x; w[e + 1] = u.y; w[e + 2] = u.z; w[e + 3] = u.w;
            }
        }
    }
    __device__ __forceinline__ float at(int e) const {
        if constexpr (DT == HGA_DTYPE_BF16)
            return __uint_as_float((e & 1) ? (w[e >> 1] & 0xffff0000u) : (w[e >> 1] << 16));
        else
            return __uint_as_float(w[e]);
    }
};

template <int DT, int DH, bool DCA, int SK>
__global__ __launch_bounds__(kDT) void attend_decode_split_kernel(DecAttnArgs A, float* part,
                                                                  int nsplit) {
    typedef typename Elem<DT>::T T;
    constexpr int DPL = DH / 16;
    constexpr int NG = kDT / 16;                     // 16-lane groups per workgroup
    constexpr int KPG = SK / NG;                     // keys per group
    constexpr int U = 4;                             // keys in flight per group
    constexpr int NQ = DCA ? 3 : 1;                  // query versions
    static_assert(SK % kDT == 0, "every thread locates SK / kDT keys of a split");
    __shared__ int sOG[256], sOT[256], sOP[DCA ? 256 : 1];
    __shared__ float sM[NG], sL[NG];
    __shared__ float sAcc[NG][DH];
    // the split's keys, located once: K and V row addresses, first visible row, position
    __shared__ unsigned long long sKP[SK], sVP[SK];
    __shared__ int sKT[SK], sKX[DCA ? SK : 1];
    __shared__ int sNopen;
    int split, bh;
    xcd_item(split, bh);
    const int gsplit = A.phase == 2 ? A.n1 + split : split;           // partial slot
    const int ph = gsplit < A.n1 ? 1 : 2;
    split = ph == 1 ? gsplit : gsplit - A.n1;                          // split of the phase
    const int b = bh / A.H, h = bh % A.H;
    const int kvh = h / (A.H / A.KVH);
    const int l = lane_id(), j = l & 15, G = (int)(threadIdx.x >> 4);
    const int Kgw = A.Kg > 0 ? A.Kg : 1;
    if (threadIdx.x == 0) sNopen = 0;
    __syncthreads();
    for (int i = threadIdx.x; i < A.Kg; i += kDT) {
        const int og = A.open_grp[(int64_t)bh * Kgw + i], ot = A.open_thr[(int64_t)bh * Kgw + i];
        sOG[i] = og;
        sOT[i] = ot;
        if constexpr (DCA) sOP[i] = A.open_pos[(int64_t)bh * Kgw + i];
        if (og >= 0 && ot >= 0) atomicMax(&sNopen, i + 1);   // length of the opened list
    }
    __syncthreads();
    DecKeys<T> keys;
    keys.init(A, b, kvh, sOG, sOT, sNopen, ph);
    if constexpr (DCA) keys.sOP = sOP;
#pragma unroll
    for (int t = (int)threadIdx.x; t < SK; t += kDT) {
        const int k = split * SK + t;
        const T* kp = nullptr;
        const T* vp = nullptr;
        int thr = kNoRow;
        int64_t kpos = 0;
        if (k < keys.n) keys.locate(k, kp, vp, thr, kpos);
        sKP[t] = (unsigned long long)kp;
        sVP[t] = (unsigned long long)vp;
        sKT[t] = k < keys.n ? thr : kNoRow;
        if constexpr (DCA) sKX[t] = (int)kpos;
    }
    __syncthreads();
    const int gk0 = split * SK + G * KPG;
    const T* qg = reinterpret_cast<const T*>(A.q) + b * A.q_sb + h * A.q_sh;
    for (int row = 0; row < A.L; ++row) {
        float qvs[NQ][DPL];
#pragma unroll
        for (int e = 0; e < DPL; ++e) {
            const int64_t o = (int64_t)row * A.q_ss + j * DPL + e;
            if constexpr (DCA) {
#pragma unroll
                for (int r = 0; r < 3; ++r) qvs[r][e] = A.q_dca[r][b * A.q_sb + h * A.q_sh + o];
            } else {
                qvs[0][e] = Elem<DT>::ld(qg, o);
            }
        }
        float m_run = -INFINITY, l_run = 0.0f, acc[DPL];
#pragma unroll
        for (int e = 0; e < DPL; ++e) acc[e] = 0.0f;
        for (int i0 = 0; i0 < KPG; i0 += U) {
            // the U keys' K and V slices are loaded together: one memory round trip per U keys
            RawSlice<DT, DPL> kxs[U], vxs[U];
            bool visu[U];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int k = gk0 + i0 + u, kl = G * KPG + i0 + u;   // kl: key within the split
                visu[u] = k < keys.n && row >= sKT[kl];
                if (visu[u]) {
                    kxs[u].load(reinterpret_cast<const T*>(sKP[kl]) + j * DPL);
                    vxs[u].load(reinterpret_cast<const T*>(sVP[kl]) + j * DPL);
                }
            }
            float s[U];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int kl = G * KPG + i0 + u;
                int64_t kpos = 0;
                if constexpr (DCA) kpos = sKX[kl];
                float d = 0.0f;
                const bool vis = visu[u];
                if (vis) {
                    float kx[DPL];
#pragma unroll
                    for (int e = 0; e < DPL; ++e) kx[e] = kxs[u].at(e);
                    if constexpr (DCA) {
                        const int r = dca_regime(kpos, A.start_pos + row, A.dca_chunk);
#pragma unroll
                        for (int e = 0; e < DPL; ++e) {
                            const float qe = r == 0 ? qvs[0][e] : (r == 1 ? qvs[1][e] : qvs[2][e]);
                            d = fmaf(qe, kx[e], d);
                        }
                    } else {
#pragma unroll
                        for (int e = 0; e < DPL; ++e) d = fmaf(qvs[0][e], kx[e], d);
                    }
                }
                d = r16_sum_f(d);                    // whole group: uniform control flow
                s[u] = vis ? d * A.scale : -INFINITY;
            }
            float mx = m_run;
#pragma unroll
            for (int u = 0; u < U; ++u) mx = fmaxf(mx, s[u]);
            const float m_use = mx == -INFINITY ? 0.0f : mx;
            const float alpha = expf(m_run - m_use);
            l_run *= alpha;
#pragma unroll
            for (int e = 0; e < DPL; ++e) acc[e] *= alpha;
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const float p = expf(s[u] - m_use);
                l_run += p;
                if (visu[u]) {
#pragma unroll
                    for (int e = 0; e < DPL; ++e) acc[e] = fmaf(p, vxs[u].at(e), acc[e]);
                }
            }
            m_run = mx;
        }
        if (j == 0) {
            sM[G] = m_run;
            sL[G] = l_run;
        }
#pragma unroll
        for (int e = 0; e < DPL; ++e) sAcc[G][j * DPL + e] = acc[e];
        __syncthreads();
        // merge the 16 groups: partial of this split for this row
        float* pp = part + (((int64_t)bh * A.L + row) * nsplit + gsplit) * (DH + 2);
        float mt = -INFINITY;
        for (int g = 0; g < NG; ++g) mt = fmaxf(mt, sM[g]);
        const float mu = mt == -INFINITY ? 0.0f : mt;
        for (int d = threadIdx.x; d < DH; d += kDT) {
            float o = 0.0f;
            for (int g = 0; g < NG; ++g) o += sAcc[g][d] * expf(sM[g] - mu);
            pp[2 + d] = o;
        }
        if (threadIdx.x == 0) {
            float lt = 0.0f;
            for (int g = 0; g < NG; ++g) lt += sL[g] * expf(sM[g] - mu);
            pp[0] = mt;
            pp[1] = lt;
        }
        __syncthreads();
    }
}

// One workgroup per (b, head, row): out = sum_s e^(m_s - M) acc_s / sum_s e^(m_s - M) l_s.
// Multi-row blocks, bf16 head_dim 64/128: the split's keys are located once, staged 32 at a time
// in LDS (K row-major, V transposed) and scored for all the block's rows at once with
// v_mfma_f32_32x32x16_bf16 -- S^T = K Q^T leaves one query row per lane (wave w: rows
// 32w..32w+31), O^T = V^T P^T -- with the online softmax per row in base 2.  Writes the same
// per-split partials as attend_decode_split_kernel (natural-log maximum, sum, accumulator).
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float floatx16_t __attribute__((ext_vector_type(16)));
constexpr int kDMT = 128;   // threads: two waves of 32 rows
constexpr int kDMK = 32;    // keys per tile

// DCA (qwen_routed_attention.py:244-283): the three fp32 query versions (intra, successive,
// inter DCA chunk) are each split into bf16 hi + lo parts (q = hi + lo to about 16 mantissa
// bits) staged in LDS; a key's scores from the three versions are accumulated by two MFMAs per
// step each and the key's regime picks one (a block's rows share one DCA chunk, so the regime is
// a property of the key).
constexpr int kDcaQStr(int DH) { return DH + 8; }
template <int DH>
constexpr size_t dca_q_lds_bytes() { return 2 * 3 * 2 * 64 * (size_t)kDcaQStr(DH); }

template <int DH, bool DCA>
__global__ __launch_bounds__(kDMT) void attend_decode_mfma_kernel(DecAttnArgs A, float* part,
                                                                  int nsplit) {
    typedef uint16_t T;
    constexpr int KS = DH / 16, DB = DH / 32, CPR = DH / 8;
    constexpr int KSTR = DH + 8, VSTR = kDMK + 4, QSTR = kDcaQStr(DH);
    __shared__ __align__(16) uint16_t sK[kDMK * KSTR];
    __shared__ __align__(16) uint16_t sVt[DH * VSTR];
    __shared__ int sOG[256], sOT[256], sOP[DCA ? 256 : 1];
    __shared__ unsigned long long sKP[kSplitKeys], sVP[kSplitKeys];
    __shared__ int sKT[kSplitKeys], sKR[DCA ? kSplitKeys : 1];
    __shared__ int sNopen;
    extern __shared__ __align__(16) uint16_t sQd[];   // DCA: [version][hi, lo][64 rows][QSTR]
    int split, bh;
    xcd_item(split, bh);
    const int gsplit = A.phase == 2 ? A.n1 + split : split;           // partial slot
    const int ph = gsplit < A.n1 ? 1 : 2;
    split = ph == 1 ? gsplit : gsplit - A.n1;                          // split of the phase
    const int b = bh / A.H, h = bh % A.H;
    const int kvh = h / (A.H / A.KVH);
    const int w = threadIdx.x / kWave, l = lane_id(), hl = l / 32;
    const int row = w * 32 + (l % 32);
    const int Kgw = A.Kg > 0 ? A.Kg : 1;
    if (threadIdx.x == 0) sNopen = 0;
    __syncthreads();
    for (int i = threadIdx.x; i < A.Kg; i += kDMT) {
        const int og = A.open_grp[(int64_t)bh * Kgw + i], ot = A.open_thr[(int64_t)bh * Kgw + i];
        sOG[i] = og;
        sOT[i] = ot;
        if constexpr (DCA) sOP[i] = A.open_pos[(int64_t)bh * Kgw + i];
        if (og >= 0 && ot >= 0) atomicMax(&sNopen, i + 1);   // length of the opened list
    }
    __syncthreads();
    DecKeys<T> keys;
    keys.init(A, b, kvh, sOG, sOT, sNopen, ph);
    if constexpr (DCA) keys.sOP = sOP;
    for (int t = threadIdx.x; t < kSplitKeys; t += kDMT) {
        const int k = split * kSplitKeys + t;
        const T* kp = nullptr;
        const T* vp = nullptr;
        int thr = kNoRow;
        int64_t kpos = 0;
        if (k < keys.n) keys.locate(k, kp, vp, thr, kpos);
        sKP[t] = (unsigned long long)kp;
        sVP[t] = (unsigned long long)vp;
        sKT[t] = kp ? thr : kNoRow;
        if constexpr (DCA) sKR[t] = dca_regime(kpos, A.start_pos, A.dca_chunk);
    }
    // this lane's query row as MFMA B operands (8 dims of each 16-dim step)
    bf16x8_t qb[KS];
    if constexpr (!DCA) {
        const T* qg = reinterpret_cast<const T*>(A.q) + b * A.q_sb + h * A.q_sh;
#pragma unroll
        for (int s = 0; s < KS; ++s) {
            uint4 u = make_uint4(0u, 0u, 0u, 0u);
            if (row < A.L) u = *reinterpret_cast<const uint4*>(qg + (int64_t)row * A.q_ss + s * 16 + 8 * hl);
            qb[s] = __builtin_bit_cast(bf16x8_t, u);
        }
    } else {
        // fp32 rows of the three versions -> bf16 hi + lo parts in LDS (rows past L are zero)
        for (int idx = threadIdx.x; idx < 3 * 64 * DH; idx += kDMT) {
            const int v = idx / (64 * DH), r = (idx / DH) % 64, d = idx % DH;
            float x = 0.0f;
            if (r < A.L) x = A.q_dca[v][b * A.q_sb + h * A.q_sh + (int64_t)r * A.q_ss + d];
            const uint16_t hi = f_to_bf16(x);
            const uint16_t lo = f_to_bf16(x - bf16_to_f(hi));
            sQd[((v * 2 + 0) * 64 + r) * QSTR + d] = hi;
            sQd[((v * 2 + 1) * 64 + r) * QSTR + d] = lo;
        }
    }
    __syncthreads();
    floatx16_t acc[DB];
#pragma unroll
    for (int d = 0; d < DB; ++d) acc[d] = floatx16_t{};
    float m_run = -INFINITY, l_run = 0.0f;
    const float c2 = A.scale * 1.4426950408889634f;
    const int nk = min(kSplitKeys, keys.n - split * kSplitKeys);
    for (int t0 = 0; t0 < nk; t0 += kDMK) {
        const uint4 z = make_uint4(0u, 0u, 0u, 0u);
        for (int c = threadIdx.x; c < kDMK * CPR; c += kDMT) {
            const int kk = c / CPR, dp = c % CPR;
            const T* kp = reinterpret_cast<const T*>(sKP[t0 + kk]);
            *reinterpret_cast<uint4*>(&sK[kk * KSTR + dp * 8]) =
                kp ? *reinterpret_cast<const uint4*>(kp + dp * 8) : z;
        }
        for (int c = threadIdx.x; c < (kDMK / 2) * CPR; c += kDMT) {
            const int kp2 = c / CPR, dg = c % CPR;
            const T* v0 = reinterpret_cast<const T*>(sVP[t0 + 2 * kp2]);
            const T* v1 = reinterpret_cast<const T*>(sVP[t0 + 2 * kp2 + 1]);
            const uint4 u0 = v0 ? *reinterpret_cast<const uint4*>(v0 + dg * 8) : z;
            const uint4 u1 = v1 ? *reinterpret_cast<const uint4*>(v1 + dg * 8) : z;
            auto put = [&](int e, uint32_t x0, uint32_t x1) {
                *reinterpret_cast<uint32_t*>(&sVt[(dg * 8 + 2 * e) * VSTR + 2 * kp2]) =
                    (x0 & 0xffffu) | (x1 << 16);
                *reinterpret_cast<uint32_t*>(&sVt[(dg * 8 + 2 * e + 1) * VSTR + 2 * kp2]) =
                    (x0 >> 16) | (x1 & 0xffff0000u);
            };
            put(0, u0.x, u1.x);
            put(1, u0.y, u1.y);
            put(2, u0.z, u1.z);
            put(3, u0.w, u1.w);
        }
        __syncthreads();
        floatx16_t sc = {};
        if constexpr (!DCA) {
#pragma unroll
            for (int s = 0; s < KS; ++s)
                sc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
                    __builtin_bit_cast(bf16x8_t, *reinterpret_cast<const uint4*>(
                                                     &sK[(l % 32) * KSTR + s * 16 + 8 * hl])),
                    qb[s], sc, 0, 0, 0);
        } else {
            floatx16_t sv[3] = {floatx16_t{}, floatx16_t{}, floatx16_t{}};
#pragma unroll
            for (int s = 0; s < KS; ++s) {
                const bf16x8_t ka = __builtin_bit_cast(
                    bf16x8_t, *reinterpret_cast<const uint4*>(&sK[(l % 32) * KSTR + s * 16 + 8 * hl]));
#pragma unroll
                for (int v = 0; v < 3; ++v)
#pragma unroll
                    for (int part = 0; part < 2; ++part)
                        sv[v] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
                            ka,
                            __builtin_bit_cast(bf16x8_t, *reinterpret_cast<const uint4*>(
                                &sQd[((v * 2 + part) * 64 + w * 32 + l % 32) * QSTR + s * 16 + 8 * hl])),
                            sv[v], 0, 0, 0);
            }
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int kk = 8 * (i / 4) + 4 * hl + (i % 4);
                const int rg = t0 + kk < nk ? sKR[t0 + kk] : 0;
                sc[i] = rg == 0 ? sv[0][i] : (rg == 1 ? sv[1][i] : sv[2][i]);
            }
        }
        float mx = -INFINITY;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int kk = 8 * (i / 4) + 4 * hl + (i % 4);
            sc[i] = (row < A.L && t0 + kk < nk && row >= sKT[t0 + kk]) ? sc[i] * c2 : -INFINITY;
            mx = fmaxf(mx, sc[i]);
        }
        mx = fmaxf(mx, __shfl_xor(mx, 32, kWave));
        const float m_new = fmaxf(m_run, mx);
        const float m_use = m_new == -INFINITY ? 0.0f : m_new;
        const float alpha = exp2f(m_run - m_use);
        float rs = 0.0f;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            sc[i] = exp2f(sc[i] - m_use);
            rs += sc[i];
        }
        rs += __shfl_xor(rs, 32, kWave);
        l_run = l_run * alpha + rs;
        m_run = m_new;
#pragma unroll
        for (int d = 0; d < DB; ++d)
#pragma unroll
            for (int i = 0; i < 16; ++i) acc[d][i] *= alpha;
        bf16x8_t pb[2];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            pb[0][j] = (__bf16)sc[j];
            pb[1][j] = (__bf16)sc[8 + j];
        }
#pragma unroll
        for (int st = 0; st < 2; ++st) {
            const int kb = 16 * st + 4 * hl;
#pragma unroll
            for (int d = 0; d < DB; ++d) {
                const uint16_t* vr = &sVt[(d * 32 + l % 32) * VSTR];
                const uint2 lo = *reinterpret_cast<const uint2*>(vr + kb);
                const uint2 hi = *reinterpret_cast<const uint2*>(vr + kb + 8);
                acc[d] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
                    __builtin_bit_cast(bf16x8_t, make_uint4(lo.x, lo.y, hi.x, hi.y)), pb[st],
                    acc[d], 0, 0, 0);
            }
        }
        __syncthreads();
    }
    if (row < A.L) {
        float* pp = part + (((int64_t)bh * A.L + row) * nsplit + gsplit) * (DH + 2);
        if (hl == 0) {
            pp[0] = m_run == -INFINITY ? -INFINITY : m_run * 0.6931471805599453f;
            pp[1] = l_run;
        }
#pragma unroll
        for (int d = 0; d < DB; ++d)
#pragma unroll
            for (int i = 0; i < 16; ++i) pp[2 + d * 32 + 8 * (i / 4) + 4 * hl + (i % 4)] = acc[d][i];
    }
}

template <int DT, int DH>
__global__ __launch_bounds__(128) void decode_combine_kernel(DecAttnArgs A, const float* part,
                                                             int nsplit) {
    typedef typename Elem<DT>::T T;
    const int bhr = blockIdx.x, row = bhr % A.L, bh = bhr / A.L, b = bh / A.H, h = bh % A.H;
    const float* pp = part + (int64_t)bhr * nsplit * (DH + 2);
    float mt = -INFINITY;
    for (int s2 = 0; s2 < nsplit; ++s2) mt = fmaxf(mt, pp[s2 * (DH + 2)]);
    const float mu = mt == -INFINITY ? 0.0f : mt;
    float lt = 0.0f;
    for (int s2 = 0; s2 < nsplit; ++s2) lt += pp[s2 * (DH + 2) + 1] * expf(pp[s2 * (DH + 2)] - mu);
    const float inv = lt > 0.0f ? 1.0f / lt : 0.0f;
    T* og = reinterpret_cast<T*>(A.out) + b * A.o_sb + h * A.o_sh + (int64_t)row * A.o_ss;
    for (int d = threadIdx.x; d < DH; d += 128) {
        float o = 0.0f;
        for (int s2 = 0; s2 < nsplit; ++s2)
            o += pp[s2 * (DH + 2) + 2 + d] * expf(pp[s2 * (DH + 2)] - mu);
        Elem<DT>::st(og, d, o * inv);
    }
}

// ------------------------------------------------------------------------------------------
// decode gather: the opened groups of a step, deduplicated per (batch, KV head), copied from the
// closed-token record (pinned host memory or device) into a device staging buffer
// ------------------------------------------------------------------------------------------
constexpr int kGT = 256;

struct GatherArgs {
    const int32_t* open_grp;
    const int32_t* open_thr;
    const unsigned char* kd;
    const unsigned char* vd;
    int64_t d_sb, d_sh, d_ss;          // record strides (elements)
    unsigned char* stage_k;
    unsigned char* stage_v;
    int32_t* staged_grp;               // [B, H, Kg] staging slot of each opened group, -1 if none
    int32_t* ulist;                    // [B, KVH, U] group id of each staging slot
    int32_t* ucount;                   // [B, KVH]
    int B, H, KVH, rep, Kg, NG, U, C, gs, M, D, esz;
};

// One workgroup per (b, kv head): the valid opened groups of the kv head's rep query heads are
// marked in an LDS bitmap over group ids [0, NG); a group's staging slot is its rank among the
// marked ids (prefix popcount), so slots are dense and in ascending group order.
__global__ __launch_bounds__(kGT) void gather_plan_kernel(GatherArgs A) {
    extern __shared__ uint32_t sBm[];                  // [NW] bitmap, then [NW] prefix counts
    __shared__ int sPart[kGT];
    const int b = blockIdx.x / A.KVH, kvh = blockIdx.x % A.KVH, tid = threadIdx.x;
    const int NW = (A.NG + 31) / 32;
    int* sPre = reinterpret_cast<int*>(sBm + NW);
    for (int i = tid; i < NW; i += kGT) sBm[i] = 0u;
    __syncthreads();
    const int Kgw = A.Kg > 0 ? A.Kg : 1, n_ent = A.rep * A.Kg;
    for (int e = tid; e < n_ent; e += kGT) {
        const int h = kvh * A.rep + e / A.Kg;
        const int64_t idx = ((int64_t)b * A.H + h) * Kgw + e % A.Kg;
        const int g = A.open_grp[idx];
        if (g >= 0 && g < A.NG && A.open_thr[idx] >= 0) atomicOr(&sBm[g >> 5], 1u << (g & 31));
    }
    __syncthreads();
    // exclusive prefix of the words' popcounts: per-thread ranges, then a serial scan of the
    // kGT partial sums
    const int per = (NW + kGT - 1) / kGT;
    const int w0 = tid * per, w1 = w0 + per < NW ? w0 + per : NW;
    int part = 0;
    for (int w = w0; w < w1; ++w) part += __popc(sBm[w]);
    sPart[tid] = part;
    __syncthreads();
    if (tid == 0) {
        int run = 0;
        for (int i = 0; i < kGT; ++i) {
            const int x = sPart[i];
            sPart[i] = run;
            run += x;
        }
        A.ucount[blockIdx.x] = run;
    }
    __syncthreads();
    {
        int run = sPart[tid];
        for (int w = w0; w < w1; ++w) {
            sPre[w] = run;
            run += __popc(sBm[w]);
        }
    }
    __syncthreads();
    int32_t* ul = A.ulist + (int64_t)blockIdx.x * A.U;
    for (int w = tid; w < NW; w += kGT) {
        uint32_t bits = sBm[w];
        int slot = sPre[w];
        while (bits) {
            ul[slot++] = 32 * w + __builtin_ctz(bits);
            bits &= bits - 1u;
        }
    }
    for (int e = tid; e < n_ent; e += kGT) {
        const int h = kvh * A.rep + e / A.Kg;
        const int64_t idx = ((int64_t)b * A.H + h) * Kgw + e % A.Kg;
        const int g = A.open_grp[idx];
        int slot = -1;
        if (g >= 0 && g < A.NG && A.open_thr[idx] >= 0)
            slot = sPre[g >> 5] + __popc(sBm[g >> 5] & ((1u << (g & 31)) - 1u));
        A.staged_grp[idx] = slot;
    }
}

// Persistent copy over the valid staging slots of all (b, kv head) pairs at once: slot v of
// the flattened list (the (b, kv head) lists one after the other, an exclusive prefix of their
// counts in LDS locates v's pair) is taken by workgroup v % G, four slots in flight per thread;
// each copies the group's gs K rows and gs V rows (contiguous in a [.., T, D] record) with
// 16-byte accesses.  A small grid (kGatherWG workgroups) leaves the other CUs to the attention
// that runs beside the copy on another stream.
constexpr int kGatherWG = 128;
__global__ __launch_bounds__(kGT) void gather_copy_kernel(GatherArgs A) {
    extern __shared__ int sPre[];                      // [nbk + 1] prefix, then [kGT] partials
    const int G = gridDim.x, nbk = A.B * A.KVH, tid = threadIdx.x;
    int* sPart = sPre + nbk + 1;
    const int per = (nbk + kGT - 1) / kGT;
    const int i0 = tid * per < nbk ? tid * per : nbk, i1 = i0 + per < nbk ? i0 + per : nbk;
    int part = 0;
    for (int i = i0; i < i1; ++i) part += A.ucount[i];
    sPart[tid] = part;
    __syncthreads();
    if (tid == 0) {
        int run = 0;
        for (int i = 0; i < kGT; ++i) {
            const int x = sPart[i];
            sPart[i] = run;
            run += x;
        }
        sPre[nbk] = run;
    }
    __syncthreads();
    {
        int run = sPart[tid];
        for (int i = i0; i < i1; ++i) {
            sPre[i] = run;
            run += A.ucount[i];
        }
    }
    __syncthreads();
    const int total = sPre[nbk];
    const int vpr = A.D * A.esz / 16;                  // 16-byte pieces per row
    const int pieces = A.gs * vpr;                     // of one group's K (or V)
    for (int v0 = blockIdx.x; v0 < total; v0 += 4 * G) {
        int64_t src[4], dst[4];
        bool ok[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int v = v0 + j * G;
            ok[j] = v < total;
            // the (b, kv head) pair holding v: the last one whose prefix is <= v
            int lo = 0, hi = nbk - 1;
            while (lo < hi) {
                const int mid = (lo + hi + 1) >> 1;
                if (sPre[mid] <= v) lo = mid;
                else hi = mid - 1;
            }
            const int bk = lo, u = ok[j] ? v - sPre[bk] : 0;
            const int b = bk / A.KVH, kvh = bk % A.KVH;
            const int g = ok[j] ? A.ulist[(int64_t)bk * A.U + u] : 0;
            const int64_t p0 = (int64_t)(g / A.M) * A.C + (int64_t)(g % A.M) * A.gs;
            src[j] = ((int64_t)b * A.d_sb + (int64_t)kvh * A.d_sh + p0 * A.d_ss) * A.esz;
            dst[j] = (((int64_t)bk * A.U + u) * A.gs) * (int64_t)A.D * A.esz;
        }
        for (int c = tid; c < pieces; c += kGT) {
            const int r = c / vpr, x = (c % vpr) * 16;
            const int64_t so = (int64_t)r * A.d_ss * A.esz + x;
            const int64_t dO = (int64_t)r * A.D * A.esz + x;
            uint4 kq[4], vq[4];
#pragma unroll
            for (int j = 0; j < 4; ++j)
                if (ok[j]) {
                    kq[j] = *reinterpret_cast<const uint4*>(A.kd + src[j] + so);
                    vq[j] = *reinterpret_cast<const uint4*>(A.vd + src[j] + so);
                }
#pragma unroll
            for (int j = 0; j < 4; ++j)
                if (ok[j]) {
                    *reinterpret_cast<uint4*>(A.stage_k + dst[j] + dO) = kq[j];
                    *reinterpret_cast<uint4*>(A.stage_v + dst[j] + dO) = vq[j];
                }
        }
    }
}

// Exclusive prefix sum over the kGT threads of a workgroup (wave scans, then the wave totals).
__device__ __forceinline__ int block_excl_scan(int x, int* sWave) {
    const int l = lane_id(), w = (int)threadIdx.x / kWave;
    int inc = x;
#pragma unroll
    for (int d = 1; d < kWave; d <<= 1) {
        const int y = __shfl_up(inc, d, kWave);
        if (l >= d) inc += y;
    }
    if (l == kWave - 1) sWave[w] = inc;
    __syncthreads();
    int base = 0;
    for (int i = 0; i < w; ++i) base += sWave[i];
    return base + inc - x;
}

// Plan and copy in one launch, for B * KVH * ceil(NG / 32) <= kFusedPlanWords: every workgroup
// marks the valid opened groups of all (b, kv head) pairs in an LDS bitmap (words of pair bk at
// bk * NW ..), takes an exclusive prefix of the words' popcounts -- a group's staging slot in its
// pair is its rank among the pair's marked ids, as in gather_plan_kernel -- and copies its share
// of the flattened slots; workgroup 0 also writes every opened group's slot.
constexpr int kFusedPlanWords = 4096;
__global__ __launch_bounds__(kGT) void gather_fused_kernel(GatherArgs A) {
    extern __shared__ uint32_t sBmF[];                 // [nw] bitmap, [nw + 1] prefix, [4] waves
    const int G = gridDim.x, nbk = A.B * A.KVH, tid = threadIdx.x;
    const int NW = (A.NG + 31) / 32, nw = nbk * NW;
    int* sPre = reinterpret_cast<int*>(sBmF + nw);
    int* sWave = sPre + nw + 1;
    for (int i = tid; i < nw; i += kGT) sBmF[i] = 0u;
    __syncthreads();
    const int Kgw = A.Kg > 0 ? A.Kg : 1, n_ent = A.B * A.H * A.Kg;
    for (int e = tid; e < n_ent; e += kGT) {
        const int bh = e / A.Kg, b = bh / A.H, h = bh % A.H;
        const int64_t idx = (int64_t)bh * Kgw + e % A.Kg;
        const int g = A.open_grp[idx];
        if (g >= 0 && g < A.NG && A.open_thr[idx] >= 0)
            atomicOr(&sBmF[(b * A.KVH + h / A.rep) * NW + (g >> 5)], 1u << (g & 31));
    }
    __syncthreads();
    const int per = (nw + kGT - 1) / kGT;
    const int w0 = tid * per < nw ? tid * per : nw, w1 = w0 + per < nw ? w0 + per : nw;
    int part = 0;
    for (int i = w0; i < w1; ++i) part += __popc(sBmF[i]);
    int run = block_excl_scan(part, sWave);
    for (int i = w0; i < w1; ++i) {
        sPre[i] = run;
        run += __popc(sBmF[i]);
    }
    if (tid == kGT - 1) sPre[nw] = run;
    __syncthreads();
    const int total = sPre[nw];
    if (blockIdx.x == 0) {
        for (int e = tid; e < n_ent; e += kGT) {
            const int bh = e / A.Kg, b = bh / A.H, h = bh % A.H;
            const int64_t idx = (int64_t)bh * Kgw + e % A.Kg;
            const int g = A.open_grp[idx];
            int slot = -1;
            if (g >= 0 && g < A.NG && A.open_thr[idx] >= 0) {
                const int bk = b * A.KVH + h / A.rep, wi = bk * NW + (g >> 5);
                slot = sPre[wi] - sPre[bk * NW] + __popc(sBmF[wi] & ((1u << (g & 31)) - 1u));
            }
            A.staged_grp[idx] = slot;
        }
    }
    const int vpr = A.D * A.esz / 16;                  // 16-byte pieces per row
    const int pieces = A.gs * vpr;                     // of one group's K (or V)
    for (int v0 = blockIdx.x; v0 < total; v0 += 4 * G) {
        int64_t src[4], dst[4];
        bool ok[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int v = v0 + j * G;
            ok[j] = v < total;
            // the bitmap word holding slot v: the last one whose prefix is <= v (a word with
            // marked groups, since the prefix rises past v there)
            int lo = 0, hi = nw - 1;
            while (lo < hi) {
                const int mid = (lo + hi + 1) >> 1;
                if (sPre[mid] <= v) lo = mid;
                else hi = mid - 1;
            }
            const int bk = lo / NW;
            uint32_t bits = ok[j] ? sBmF[lo] : 0u;
            for (int r = ok[j] ? v - sPre[lo] : 0; r > 0; --r) bits &= bits - 1u;   // r-th set bit
            const int g = (lo % NW) * 32 + (bits ? __builtin_ctz(bits) : 0);
            const int u = ok[j] ? v - sPre[bk * NW] : 0;
            const int b = bk / A.KVH, kvh = bk % A.KVH;
            const int64_t p0 = (int64_t)(g / A.M) * A.C + (int64_t)(g % A.M) * A.gs;
            src[j] = ((int64_t)b * A.d_sb + (int64_t)kvh * A.d_sh + p0 * A.d_ss) * A.esz;
            dst[j] = (((int64_t)bk * A.U + u) * A.gs) * (int64_t)A.D * A.esz;
        }
        for (int c = tid; c < pieces; c += kGT) {
            const int r = c / vpr, x = (c % vpr) * 16;
            const int64_t so = (int64_t)r * A.d_ss * A.esz + x;
            const int64_t dO = (int64_t)r * A.D * A.esz + x;
            uint4 kq[4], vq[4];
#pragma unroll
            for (int j = 0; j < 4; ++j)
                if (ok[j]) {
                    kq[j] = *reinterpret_cast<const uint4*>(A.kd + src[j] + so);
                    vq[j] = *reinterpret_cast<const uint4*>(A.vd + src[j] + so);
                }
#pragma unroll
            for (int j = 0; j < 4; ++j)
                if (ok[j]) {
                    *reinterpret_cast<uint4*>(A.stage_k + dst[j] + dO) = kq[j];
                    *reinterpret_cast<uint4*>(A.stage_v + dst[j] + dO) = vq[j];
                }
        }
    }
}

}  // namespace
}  // namespace hga

namespace {
// Keys per split: kWideSplitKeys for one-token steps of B * H >= kWideSplitHeads (these take
// the VALU split kernel), else kSplitKeys.
int split_keys(const hga_config* cfg, int32_t L) {
    return L == 1 && (int64_t)cfg->batch * cfg->heads >= hga::kWideSplitHeads ? hga::kWideSplitKeys
                                                                               : hga::kSplitKeys;
}
// Splits of the split decode attention: phase 1 the windows and the active chunk, phase 2 the
// opened groups of the longest list (every slot valid), phase 0 both; the workspace holds the
// partials of all of them.
int decode_splits(const hga_config* cfg, int32_t L, int32_t n_closed, int64_t start_pos,
                  int32_t Kg, int phase) {
    const int sk = split_keys(cfg, L);
    int f_hi, l_lo;
    hga::windows(n_closed, cfg->keep_first, cfg->keep_last, &f_hi, &l_lo);
    const int64_t C = cfg->chunk_size;
    const int64_t c0 = start_pos - (int64_t)n_closed * C;
    const int64_t win = (int64_t)f_hi * C + (int64_t)(n_closed - l_lo) * C + c0 + L;
    const int64_t opened = (int64_t)(Kg > 0 ? Kg : 0) * cfg->group_size;
    auto splits = [sk](int64_t keys) { return (keys + sk - 1) / sk; };
    if (phase == 1) return (int)splits(win);
    if (phase == 2) return (int)splits(opened);
    return (int)(splits(win) + splits(opened));
}
}  // namespace

extern "C" int32_t hga_attend_decode_workspace(const hga_config* cfg, int32_t L, int32_t n_closed,
                                               int64_t start_pos, int32_t Kg, int64_t* bytes) {
    using namespace hga;
    int rc = check_config(cfg);
    if (rc) return rc;
    HGA_REQUIRE(bytes && L >= 1 && n_closed >= 0 && Kg >= 0, HGA_ERR_ARG,
                "hga_attend_decode_workspace: bad arguments");
    const int D = cfg->head_dim;
    *bytes = (D == 64 || D == 128)
                 ? 4 * (int64_t)cfg->batch * cfg->heads * L *
                       decode_splits(cfg, L, n_closed, start_pos, Kg, 0) * (D + 2)
                 : 0;
    return HGA_OK;
}

extern "C" int32_t hga_gather_decode_sizes(const hga_config* cfg, int32_t Kg,
                                           int32_t* stage_groups, int64_t* stage_bytes,
                                           int64_t* scratch_bytes) {
    using namespace hga;
    int rc = check_config(cfg);
    if (rc) return rc;
    HGA_REQUIRE(Kg >= 0 && stage_groups && stage_bytes && scratch_bytes, HGA_ERR_ARG,
                "hga_gather_decode_sizes: bad arguments");
    const int rep = cfg->heads / cfg->kv_heads;
    const int U = rep * (Kg > 0 ? Kg : 1);
    const int64_t esz = cfg->dtype == HGA_DTYPE_BF16 ? 2 : 4;
    *stage_groups = U;
    *stage_bytes = (int64_t)cfg->batch * cfg->kv_heads * U * cfg->group_size * cfg->head_dim * esz;
    *scratch_bytes = 4 * (int64_t)cfg->batch * cfg->kv_heads * (U + 1);
    return HGA_OK;
}

extern "C" int hga_gather_decode(const hga_config* cfg, int32_t n_closed, const int32_t* open_grp,
                                 const int32_t* open_thr, int32_t Kg, const void* k_record,
                                 const void* v_record, int64_t d_sb, int64_t d_sh, int64_t d_ss,
                                 int32_t record_on_host, void* stage_k, void* stage_v,
                                 int32_t stage_groups, int32_t* staged_grp, void* scratch,
                                 int64_t scratch_bytes, void* stream) {
    using namespace hga;
    int rc = check_config(cfg);
    if (rc) return rc;
    HGA_REQUIRE(open_grp && open_thr && k_record && v_record && stage_k && stage_v && staged_grp &&
                    scratch,
                HGA_ERR_ARG, "hga_gather_decode: NULL pointer");
    HGA_REQUIRE(n_closed >= 0 && Kg >= 0, HGA_ERR_ARG, "hga_gather_decode: bad n_closed/Kg");
    int32_t U = 0;
    int64_t sbytes = 0, need = 0;
    hga_gather_decode_sizes(cfg, Kg, &U, &sbytes, &need);
    // scratch: the slot list at the caller's staging capacity, then the counts
    need = 4 * (int64_t)cfg->batch * cfg->kv_heads * ((int64_t)stage_groups + 1);
    HGA_REQUIRE(stage_groups >= U && scratch_bytes >= need, HGA_ERR_ARG,
                "hga_gather_decode: staging for %d groups and %lld scratch bytes required", U,
                (long long)need);
    const int64_t ve = cfg->dtype == HGA_DTYPE_BF16 ? 8 : 4;
    HGA_REQUIRE(((uintptr_t)k_record | (uintptr_t)v_record | (uintptr_t)stage_k |
                 (uintptr_t)stage_v) % 16 == 0 && ((d_sb | d_sh | d_ss) % ve) == 0,
                HGA_ERR_ARG, "hga_gather_decode: 16-byte aligned rows required");
    GatherArgs a{};
    a.kd = static_cast<const unsigned char*>(k_record);
    a.vd = static_cast<const unsigned char*>(v_record);
    if (record_on_host) {
        void *dk = nullptr, *dv = nullptr;
        hipError_t e1 = hipHostGetDevicePointer(&dk, const_cast<void*>(k_record), 0);
        hipError_t e2 = hipHostGetDevicePointer(&dv, const_cast<void*>(v_record), 0);
        HGA_REQUIRE(e1 == hipSuccess && e2 == hipSuccess, HGA_ERR_ARG,
                    "hga_gather_decode: the host record is not pinned device-accessible memory");
        a.kd = static_cast<const unsigned char*>(dk);
        a.vd = static_cast<const unsigned char*>(dv);
    }
    a.open_grp = open_grp; a.open_thr = open_thr;
    a.d_sb = d_sb; a.d_sh = d_sh; a.d_ss = d_ss;
    a.stage_k = static_cast<unsigned char*>(stage_k);
    a.stage_v = static_cast<unsigned char*>(stage_v);
    a.staged_grp = staged_grp;
    a.B = cfg->batch; a.H = cfg->heads; a.KVH = cfg->kv_heads; a.rep = cfg->heads / cfg->kv_heads;
    a.Kg = Kg; a.C = cfg->chunk_size; a.gs = cfg->group_size; a.M = a.C / a.gs;
    a.NG = n_closed * a.M; a.U = stage_groups; a.D = cfg->head_dim;
    a.esz = cfg->dtype == HGA_DTYPE_BF16 ? 2 : 4;
    a.ulist = static_cast<int32_t*>(scratch);
    a.ucount = a.ulist + (int64_t)a.B * a.KVH * a.U;
    const int NW = (a.NG + 31) / 32;
    const size_t lds = 2 * sizeof(uint32_t) * (size_t)(NW > 0 ? NW : 1);
    HGA_REQUIRE(lds <= 65536, HGA_ERR_UNSUPPORTED, "hga_gather_decode: %d closed chunks too many",
                n_closed);
    hipStream_t st = (hipStream_t)stream;
    const int64_t nwf = (int64_t)a.B * a.KVH * NW;
    if (Kg > 0 && n_closed > 0 && nwf <= kFusedPlanWords) {
        // plan and copy in one launch
        const size_t lds_f = sizeof(uint32_t) * (2 * (size_t)nwf + 1 + kGT / kWave);
        gather_fused_kernel<<<dim3((unsigned)kGatherWG), dim3(kGT), lds_f, st>>>(a);
        return launch_status("hga_gather_decode (plan + copy)");
    }
    gather_plan_kernel<<<dim3((unsigned)(a.B * a.KVH)), dim3(kGT), lds, st>>>(a);
    rc = launch_status("hga_gather_decode (plan)");
    if (rc) return rc;
    if (Kg == 0 || n_closed == 0) return HGA_OK;
    const size_t lds_c = sizeof(int) * ((size_t)a.B * a.KVH + 1 + kGT);
    HGA_REQUIRE(lds_c <= 65536, HGA_ERR_UNSUPPORTED, "hga_gather_decode: batch x kv heads too large");
    gather_copy_kernel<<<dim3((unsigned)kGatherWG), dim3(kGT), lds_c, st>>>(a);
    return launch_status("hga_gather_decode (copy)");
}

extern "C" int32_t hga_decode_widths(const hga_config* cfg, int32_t n_closed, int32_t* Kc,
                                     int32_t* Kg) {
    using namespace hga;
    int rc = check_config(cfg);
    if (rc) return rc;
    HGA_REQUIRE(n_closed >= 0, HGA_ERR_ARG, "negative n_closed");
    int f_hi, l_lo;
    windows(n_closed, cfg->keep_first, cfg->keep_last, &f_hi, &l_lo);
    const int nmid = l_lo > f_hi ? l_lo - f_hi : 0;
    const int M = cfg->chunk_size / cfg->group_size;
    const int kc = (nmid > 0 && cfg->topk_chunks > 0) ? (cfg->topk_chunks < nmid ? cfg->topk_chunks : nmid) : 0;
    const int kg = cfg->topk_groups > 0 ? (cfg->topk_groups < kc * M ? cfg->topk_groups : kc * M) : 0;
    if (Kc) *Kc = kc;
    if (Kg) *Kg = kg;
    return HGA_OK;
}

namespace hga {
namespace {
// Stage-1 segmentation of a decode block's pool: segment length, count and the scoring kernel's
// LDS bytes.  Segments of at least 128 (L <= 4), 256 (L < 16) or 64 chunks (L >= 16: 4 row
// groups per key) give each workgroup's 256 threads work; longer segments where the grid already
// has about 1024 workgroups, or to keep the merge's candidates (nseg * Kc) within one wave
// selection.
struct DecSeg {
    int seg, nseg, spd;
    size_t lds;
};
int dec_segments(const hga_config* cfg, int L, int nmid, int Kc, DecSeg* o) {
    const int64_t room =
        ((int64_t)163840 - 16 - (int64_t)(4 * L * cfg->head_dim)) / (4 * score_row_groups(L));
    const int cap = 64 * kDecJ / (Kc > 0 ? Kc : 1);
    const int RG = score_row_groups(L);
    int seg = RG == 4 ? 64 : (L <= 4 ? 128 : 256);
    // split a pool only as far as the grid needs: about 1024 scoring workgroups in all
    const int64_t heads = (int64_t)cfg->batch * cfg->heads;
    const int64_t want = heads >= 1024 ? 1 : (1024 + heads - 1) / heads;
    if (nmid > seg * want) {
        seg = (int)((nmid + want - 1) / want);
        if (seg > 64 * kDecSegJ) seg = 64 * kDecSegJ;
        if (seg > room) seg = (int)room;
    }
    if (nmid > (int64_t)seg * cap) seg = (nmid + cap - 1) / cap;
    HGA_REQUIRE(seg <= 64 * kDecSegJ && seg <= room, HGA_ERR_UNSUPPORTED,
                "hga_route_decode: pool of %d chunks too long for L=%d x head_dim %d", nmid, L,
                cfg->head_dim);
    o->seg = seg;
    o->nseg = nmid > 0 ? (nmid + seg - 1) / seg : 0;
    o->spd = seg;   // [row groups][seg] partial maxima
    o->lds = sizeof(float) * ((size_t)L * cfg->head_dim + (size_t)RG * seg) + 16;
    return HGA_OK;
}
}  // namespace
}  // namespace hga

extern "C" int hga_route_decode_workspace(const hga_config* cfg, int32_t L, int32_t n_closed,
                                          int64_t* bytes) {
    using namespace hga;
    int rc = check_config(cfg);
    if (rc) return rc;
    HGA_REQUIRE(bytes && L >= 1 && L <= kMaxL && n_closed >= 0, HGA_ERR_ARG,
                "hga_route_decode_workspace: bad L/n_closed/bytes");
    int f_hi, l_lo, Kc, Kg;
    windows(n_closed, cfg->keep_first, cfg->keep_last, &f_hi, &l_lo);
    const int nmid = l_lo > f_hi ? l_lo - f_hi : 0;
    hga_decode_widths(cfg, n_closed, &Kc, &Kg);
    DecSeg sg{};
    if (Kc > 0) {
        rc = dec_segments(cfg, L, nmid, Kc, &sg);
        if (rc) return rc;
    }
    // stage-1 scores of every row (blocks of 2+ rows: their rank counts read them), then per
    // (b, h, segment) Kc pooled values and chunk offsets
    const int64_t score_bytes = L > 1 ? (int64_t)L * nmid * 4 : 0;
    *bytes = Kc > 0 ? (int64_t)cfg->batch * cfg->heads * (score_bytes + sg.nseg * Kc * 8) : 0;
    return HGA_OK;
}

extern "C" int hga_route_decode(const hga_config* cfg, int32_t L, int32_t n_closed, const void* q,
                                int64_t q_sb, int64_t q_sh, int64_t q_ss, const void* chunk_k,
                                int64_t ck_sb, int64_t ck_sh, const void* group_k, int64_t gk_sb,
                                int64_t gk_sh, int32_t* mid, int32_t* mid_thr, int32_t* n_mid,
                                int32_t* open_grp, int32_t* open_thr, int32_t* n_open,
                                void* workspace, int64_t workspace_bytes, void* stream) {
    using namespace hga;
    int rc = check_config(cfg);
    if (rc) return rc;
    HGA_REQUIRE(q && mid && mid_thr && n_mid && open_grp && open_thr && n_open, HGA_ERR_ARG,
                "hga_route_decode: NULL pointer");
    HGA_REQUIRE(L >= 1 && L <= kMaxL, HGA_ERR_UNSUPPORTED, "hga_route_decode: L=%d outside [1, 64]", L);
    HGA_REQUIRE(n_closed >= 0, HGA_ERR_ARG, "hga_route_decode: negative n_closed");
    DecRouteArgs a{};
    a.q = q; a.q_sb = q_sb; a.q_sh = q_sh; a.q_ss = q_ss;
    a.ck = chunk_k; a.ck_sb = ck_sb; a.ck_sh = ck_sh;
    a.gk = group_k; a.gk_sb = gk_sb; a.gk_sh = gk_sh;
    a.mid = mid; a.mid_thr = mid_thr; a.n_mid = n_mid;
    a.open_grp = open_grp; a.open_thr = open_thr; a.n_open = n_open;
    a.B = cfg->batch; a.H = cfg->heads; a.KVH = cfg->kv_heads; a.L = L; a.n_closed = n_closed;
    a.M = cfg->chunk_size / cfg->group_size; a.kf = cfg->keep_first; a.kl = cfg->keep_last;
    hga_decode_widths(cfg, n_closed, &a.Kc, &a.Kg);
    a.Kgr = cfg->topk_groups > 0 ? (cfg->topk_groups / 2 < a.Kc * a.M ? cfg->topk_groups / 2 : a.Kc * a.M) : 0;
    a.scale = cfg->scale;
    int f_hi, l_lo;
    windows(n_closed, a.kf, a.kl, &f_hi, &l_lo);
    const int nmid = l_lo > f_hi ? l_lo - f_hi : 0;
    HGA_REQUIRE(a.Kc <= 64, HGA_ERR_UNSUPPORTED, "hga_route_decode: top-k chunks %d > 64", a.Kc);
    const int T2max = a.Kc * a.M;
    HGA_REQUIRE(T2max <= kDecJ * 64, HGA_ERR_UNSUPPORTED,
                "hga_route_decode: %d candidate groups exceed %d", T2max, kDecJ * 64);
    const int D = cfg->head_dim;
    const size_t esz = cfg->dtype == HGA_DTYPE_BF16 ? 2 : 4;
    DecSeg sg{};
    if (a.Kc > 0) {
        rc = dec_segments(cfg, L, nmid, a.Kc, &sg);
        if (rc) return rc;
        int64_t need = 0;
        hga_route_decode_workspace(cfg, L, n_closed, &need);
        HGA_REQUIRE(workspace && workspace_bytes >= need && (uintptr_t)workspace % 4 == 0,
                    HGA_ERR_ARG, "hga_route_decode: workspace of %lld bytes required (got %lld)",
                    (long long)need, (long long)workspace_bytes);
        a.seg = sg.seg;
        a.nseg = sg.nseg;
        a.SPW = nmid;
        a.ws = L > 1 ? (float*)workspace : nullptr;
        a.wv = (float*)workspace + (L > 1 ? (int64_t)a.B * a.H * L * nmid : 0);
        a.wi = (int32_t*)(a.wv + (int64_t)a.B * a.H * sg.nseg * a.Kc);
    }
    // merge kernel LDS: sQ [L][D] | sS [L][SPD] | sPool, sFirst [SPD] | sSel, sThr [64] |
    // sScal [8] | sOp [256] | sPI [Kc]; SPD covers stage 2's candidate groups and the lists
    const int Kcw = a.Kc > 0 ? a.Kc : 1;
    HGA_REQUIRE(a.Kg <= 256, HGA_ERR_UNSUPPORTED, "hga_route_decode: top-k groups %d > 256", a.Kg);
    a.SPD = ((T2max > Kcw ? T2max : Kcw) + 1) | 1;
    const size_t lds = sizeof(float) * (size_t)L * D + sizeof(int) * (136 + 256 + (size_t)Kcw) +
                       16 + sizeof(float) * (size_t)(L + 2) * a.SPD;
    HGA_REQUIRE(lds <= 163840, HGA_ERR_UNSUPPORTED,
                "hga_route_decode: L=%d x head_dim %d x %d groups leave no LDS", L, D, T2max);
    if (a.Kc > 0) {
        const int64_t ve = esz == 2 ? 8 : 4;
        HGA_REQUIRE(chunk_k && group_k, HGA_ERR_ARG, "hga_route_decode: NULL summaries");
        const uintptr_t al = (uintptr_t)chunk_k | (uintptr_t)group_k | (uintptr_t)q;
        HGA_REQUIRE(al % 16 == 0 && ((ck_sb | ck_sh | gk_sb | gk_sh | q_sb | q_sh | q_ss) % ve) == 0,
                    HGA_ERR_ARG, "hga_route_decode: 16-byte aligned rows required");
    }
    hipStream_t st = (hipStream_t)stream;
    const unsigned grid = (unsigned)(a.B * a.H);
#define HGA_DEC_CASE(DTV, DHV)                                                                  \
    if (cfg->dtype == DTV && D == DHV) {                                                        \
        static bool attr = false;                                                               \
        if (!attr) {                                                                            \
            (void)hipFuncSetAttribute((const void*)route_decode_kernel<DTV, DHV>,               \
                                      hipFuncAttributeMaxDynamicSharedMemorySize, 163840);      \
            (void)hipFuncSetAttribute((const void*)route_decode_part_kernel<DTV, DHV>,          \
                                      hipFuncAttributeMaxDynamicSharedMemorySize, 163840);      \
            attr = true;                                                                        \
        }                                                                                       \
        if (a.Kc > 0) {                                                                         \
            route_decode_part_kernel<DTV, DHV><<<dim3((unsigned)sg.nseg, grid),               \
                                                 L <= 4 ? kWave : kDT, sg.lds, st>>>(a);        \
            rc = launch_status("hga_route_decode");                                             \
            if (rc) return rc;                                                                  \
        }                                                                                       \
        route_decode_kernel<DTV, DHV><<<dim3(1u, grid), kDT, lds, st>>>(a);                     \
        return launch_status("hga_route_decode");                                               \
    }
    HGA_DEC_CASE(HGA_DTYPE_BF16, 128)
    HGA_DEC_CASE(HGA_DTYPE_BF16, 64)
    HGA_DEC_CASE(HGA_DTYPE_BF16, 32)
    HGA_DEC_CASE(HGA_DTYPE_BF16, 16)
    HGA_DEC_CASE(HGA_DTYPE_F32, 128)
    HGA_DEC_CASE(HGA_DTYPE_F32, 64)
    HGA_DEC_CASE(HGA_DTYPE_F32, 32)
    HGA_DEC_CASE(HGA_DTYPE_F32, 16)
#undef HGA_DEC_CASE
    set_error("hga_route_decode: unsupported dtype/head_dim");
    return HGA_ERR_UNSUPPORTED;
}

namespace hga {
namespace {
// Body of hga_attend_decode and hga_attend_decode_dca (q_dca == nullptr: plain attention).
int attend_decode_impl(const hga_config* cfg, int32_t L, int32_t n_closed, int64_t start_pos,
                       const void* q, int64_t q_sb, int64_t q_sh, int64_t q_ss,
                       const float* const* q_dca, const int32_t* open_pos, int32_t dca_chunk,
                       const void* k_recent, const void* v_recent, int64_t r_sb, int64_t r_sh,
                       int64_t r_ss, int32_t ring_chunks, const void* k_first,
                       const void* v_first, int64_t f_sb, int64_t f_sh, int64_t f_ss,
                       const void* k_record, const void* v_record, int64_t d_sb, int64_t d_sh,
                       int64_t d_ss, int32_t record_on_host, const int32_t* open_grp,
                       const int32_t* open_thr, int32_t Kg, void* out, int64_t o_sb,
                       int64_t o_sh, int64_t o_ss, void* workspace, int64_t workspace_bytes,
                       void* stream, int32_t phase = 0) {
    int rc = check_config(cfg);
    if (rc) return rc;
    HGA_REQUIRE(phase >= 0 && phase <= 2, HGA_ERR_ARG, "hga_attend_decode_phase: phase %d", phase);
    HGA_REQUIRE(phase == 0 || cfg->head_dim == 64 || cfg->head_dim == 128, HGA_ERR_UNSUPPORTED,
                "hga_attend_decode_phase: phases need head_dim 64 or 128");
    HGA_REQUIRE((q || q_dca) && k_recent && v_recent && out && open_grp && open_thr, HGA_ERR_ARG,
                "hga_attend_decode: NULL pointer");
    HGA_REQUIRE(L >= 1 && L <= kMaxL && n_closed >= 0 && Kg >= 0 && Kg <= 256 && ring_chunks >= 0,
                HGA_ERR_ARG, "hga_attend_decode: bad L/n_closed/Kg/ring");
    const int C = cfg->chunk_size;
    const int64_t c0 = start_pos - (int64_t)n_closed * C;
    HGA_REQUIRE(c0 >= 0 && c0 + L <= C, HGA_ERR_ARG,
                "hga_attend_decode: block [%lld, +%d) is not inside active chunk %d",
                (long long)start_pos, L, n_closed);
    int f_hi, l_lo;
    windows(n_closed, cfg->keep_first, cfg->keep_last, &f_hi, &l_lo);
    HGA_REQUIRE(f_hi == 0 || (k_first && v_first), HGA_ERR_ARG, "hga_attend_decode: first window source missing");
    HGA_REQUIRE(ring_chunks == 0 || ring_chunks >= n_closed - l_lo + 1, HGA_ERR_ARG,
                "hga_attend_decode: ring of %d chunks cannot hold the last window + active chunk",
                ring_chunks);
    const bool dca = q_dca != nullptr;
    if (dca) {
        HGA_REQUIRE(q_dca[0] && q_dca[1] && q_dca[2], HGA_ERR_ARG,
                    "hga_attend_decode_dca: NULL query version");
        HGA_REQUIRE(dca_chunk > 0 && dca_chunk % C == 0, HGA_ERR_ARG,
                    "hga_attend_decode_dca: dca_chunk %d must be a positive multiple of the chunk "
                    "size %d", dca_chunk, C);
    }
    DecAttnArgs a{};
    a.q = q ? q : (dca ? q_dca[0] : nullptr);
    a.q_sb = q_sb; a.q_sh = q_sh; a.q_ss = q_ss;
    if (dca) {
        for (int r = 0; r < 3; ++r) a.q_dca[r] = q_dca[r];
        a.open_pos = open_pos ? open_pos : open_grp;
        a.dca_chunk = dca_chunk;
    }
    a.kr = k_recent; a.vr = v_recent; a.r_sb = r_sb; a.r_sh = r_sh; a.r_ss = r_ss;
    a.kfst = k_first ? k_first : k_recent; a.vfst = v_first ? v_first : v_recent;
    a.f_sb = f_sb; a.f_sh = f_sh; a.f_ss = f_ss;
    a.kd = k_record ? k_record : k_recent; a.vd = v_record ? v_record : v_recent;
    a.d_sb = d_sb; a.d_sh = d_sh; a.d_ss = d_ss;
    if (record_on_host && k_record) {
        void *dk = nullptr, *dv = nullptr;
        hipError_t e1 = hipHostGetDevicePointer(&dk, const_cast<void*>(k_record), 0);
        hipError_t e2 = hipHostGetDevicePointer(&dv, const_cast<void*>(v_record), 0);
        HGA_REQUIRE(e1 == hipSuccess && e2 == hipSuccess, HGA_ERR_ARG,
                    "hga_attend_decode: the host record is not pinned device-accessible memory");
        a.kd = dk;
        a.vd = dv;
    }
    a.open_grp = open_grp; a.open_thr = open_thr;
    a.out = out; a.o_sb = o_sb; a.o_sh = o_sh; a.o_ss = o_ss;
    a.start_pos = start_pos;
    a.B = cfg->batch; a.H = cfg->heads; a.KVH = cfg->kv_heads; a.L = L; a.n_closed = n_closed;
    a.C = C; a.gs = cfg->group_size; a.M = C / cfg->group_size; a.kf = cfg->keep_first;
    a.kl = cfg->keep_last; a.Kg = Kg; a.ring = ring_chunks; a.scale = cfg->scale;
    const int D = cfg->head_dim;
    const int64_t ve = cfg->dtype == HGA_DTYPE_BF16 ? 8 : 4;
    const uintptr_t al = (uintptr_t)a.kr | (uintptr_t)a.kfst | (uintptr_t)a.kd;
    HGA_REQUIRE(al % 16 == 0 && ((r_sb | r_sh | r_ss | f_sb | f_sh | f_ss | d_sb | d_sh | d_ss) % ve) == 0,
                HGA_ERR_ARG, "hga_attend_decode: 16-byte aligned key rows required");
    hipStream_t st = (hipStream_t)stream;
    if (D == 64 || D == 128) {
        // phase 0: one launch over all keys; phases 1 and 2: the windows and active chunk into
        // partial slots [0, n1), the opened groups into [n1, n1 + n2), then the combine
        const int n1 = decode_splits(cfg, L, n_closed, start_pos, Kg, 1);
        const int n2 = decode_splits(cfg, L, n_closed, start_pos, Kg, 2);
        const int nsplit = n1 + n2;
        const int64_t need = 4 * (int64_t)a.B * a.H * L * nsplit * (D + 2);
        HGA_REQUIRE(workspace && workspace_bytes >= need, HGA_ERR_ARG,
                    "hga_attend_decode: workspace of %lld bytes required (got %lld)",
                    (long long)need, (long long)workspace_bytes);
        float* part = static_cast<float*>(workspace);
        a.phase = phase;
        a.n1 = n1;
        const int nlaunch = phase == 0 ? nsplit : (phase == 1 ? n1 : n2);
        const dim3 g1((unsigned)(nlaunch > 0 ? nlaunch : 1), (unsigned)(a.B * a.H)),
            g2((unsigned)(a.B * a.H * L));
        // blocks of 8+ rows (bf16, aligned query rows): the MFMA split kernel
        const bool mfma = cfg->dtype == HGA_DTYPE_BF16 && L >= 8 &&
                          (dca || ((uintptr_t)q % 16 == 0 && ((q_sb | q_sh | q_ss) % 8) == 0));
        const bool wide = split_keys(cfg, L) == kWideSplitKeys;   // never with the MFMA kernel (L 1)
#define HGA_DS_CASE(DTV, DHV)                                                                    \
        if (cfg->dtype == DTV && D == DHV) {                                                   \
            if (nlaunch == 0) {                                                                 \
            } else if (mfma && DTV == HGA_DTYPE_BF16 && dca) {                                  \
                static bool attr = false;                                                       \
                if (!attr) {                                                                    \
                    (void)hipFuncSetAttribute((const void*)attend_decode_mfma_kernel<DHV, true>, \
                                              hipFuncAttributeMaxDynamicSharedMemorySize,       \
                                              (int)dca_q_lds_bytes<DHV>());                     \
                    attr = true;                                                                \
                }                                                                               \
                attend_decode_mfma_kernel<DHV, true><<<g1, kDMT, dca_q_lds_bytes<DHV>(), st>>>(  \
                    a, part, nsplit);                                                           \
            } else if (mfma && DTV == HGA_DTYPE_BF16)                                           \
                attend_decode_mfma_kernel<DHV, false><<<g1, kDMT, 0, st>>>(a, part, nsplit);    \
            else if (wide && dca)                                                               \
                attend_decode_split_kernel<DTV, DHV, true, kWideSplitKeys><<<g1, kDT, 0, st>>>(a, part, nsplit); \
            else if (wide)                                                                      \
                attend_decode_split_kernel<DTV, DHV, false, kWideSplitKeys><<<g1, kDT, 0, st>>>(a, part, nsplit); \
            else if (dca)                                                                       \
                attend_decode_split_kernel<DTV, DHV, true, kSplitKeys><<<g1, kDT, 0, st>>>(a, part, nsplit); \
            else attend_decode_split_kernel<DTV, DHV, false, kSplitKeys><<<g1, kDT, 0, st>>>(a, part, nsplit); \
            rc = launch_status("hga_attend_decode (split)");                                    \
            if (rc) return rc;                                                                  \
            if (phase == 1) return HGA_OK;                                                      \
            decode_combine_kernel<DTV, DHV><<<g2, 128, 0, st>>>(a, part, nsplit);               \
            return launch_status("hga_attend_decode (combine)");                                \
        }
        HGA_DS_CASE(HGA_DTYPE_BF16, 128)
        HGA_DS_CASE(HGA_DTYPE_BF16, 64)
        HGA_DS_CASE(HGA_DTYPE_F32, 128)
        HGA_DS_CASE(HGA_DTYPE_F32, 64)
#undef HGA_DS_CASE
    }
    const unsigned grid = (unsigned)(a.B * a.H);
#define HGA_DA_CASE(DTV, DHV)                                                                    \
    if (cfg->dtype == DTV && D == DHV) {                                                       \
        if (dca) attend_decode_kernel<DTV, DHV, true><<<grid, kDT, 0, st>>>(a);                \
        else attend_decode_kernel<DTV, DHV, false><<<grid, kDT, 0, st>>>(a);                   \
        return launch_status("hga_attend_decode");                                             \
    }
    HGA_DA_CASE(HGA_DTYPE_BF16, 128)
    HGA_DA_CASE(HGA_DTYPE_BF16, 64)
    HGA_DA_CASE(HGA_DTYPE_BF16, 32)
    HGA_DA_CASE(HGA_DTYPE_BF16, 16)
    HGA_DA_CASE(HGA_DTYPE_F32, 128)
    HGA_DA_CASE(HGA_DTYPE_F32, 64)
    HGA_DA_CASE(HGA_DTYPE_F32, 32)
    HGA_DA_CASE(HGA_DTYPE_F32, 16)
#undef HGA_DA_CASE
    set_error("hga_attend_decode: unsupported dtype/head_dim");
    return HGA_ERR_UNSUPPORTED;
}
}  // namespace
}  // namespace hga

extern "C" int hga_attend_decode(const hga_config* cfg, int32_t L, int32_t n_closed,
                                 int64_t start_pos, const void* q, int64_t q_sb, int64_t q_sh,
                                 int64_t q_ss, const void* k_recent, const void* v_recent,
                                 int64_t r_sb, int64_t r_sh, int64_t r_ss, int32_t ring_chunks,
                                 const void* k_first, const void* v_first, int64_t f_sb,
                                 int64_t f_sh, int64_t f_ss, const void* k_record,
                                 const void* v_record, int64_t d_sb, int64_t d_sh, int64_t d_ss,
                                 int32_t record_on_host, const int32_t* open_grp,
                                 const int32_t* open_thr, int32_t Kg, void* out, int64_t o_sb,
                                 int64_t o_sh, int64_t o_ss, void* workspace,
                                 int64_t workspace_bytes, void* stream) {
    HGA_REQUIRE(q, HGA_ERR_ARG, "hga_attend_decode: NULL pointer");
    return hga::attend_decode_impl(cfg, L, n_closed, start_pos, q, q_sb, q_sh, q_ss, nullptr,
                                   nullptr, 0, k_recent, v_recent, r_sb, r_sh, r_ss, ring_chunks,
                                   k_first, v_first, f_sb, f_sh, f_ss, k_record, v_record, d_sb,
                                   d_sh, d_ss, record_on_host, open_grp, open_thr, Kg, out, o_sb,
                                   o_sh, o_ss, workspace, workspace_bytes, stream);
}

extern "C" int hga_attend_decode_phase(const hga_config* cfg, int32_t L, int32_t n_closed,
                                       int64_t start_pos, const void* q, int64_t q_sb,
                                       int64_t q_sh, int64_t q_ss, const void* k_recent,
                                       const void* v_recent, int64_t r_sb, int64_t r_sh,
                                       int64_t r_ss, int32_t ring_chunks, const void* k_first,
                                       const void* v_first, int64_t f_sb, int64_t f_sh,
                                       int64_t f_ss, const void* k_record, const void* v_record,
                                       int64_t d_sb, int64_t d_sh, int64_t d_ss,
                                       int32_t record_on_host, const int32_t* open_grp,
                                       const int32_t* open_thr, int32_t Kg, void* out,
                                       int64_t o_sb, int64_t o_sh, int64_t o_ss, int32_t phase,
                                       void* workspace, int64_t workspace_bytes, void* stream) {
    HGA_REQUIRE(q, HGA_ERR_ARG, "hga_attend_decode_phase: NULL pointer");
    return hga::attend_decode_impl(cfg, L, n_closed, start_pos, q, q_sb, q_sh, q_ss, nullptr,
                                   nullptr, 0, k_recent, v_recent, r_sb, r_sh, r_ss, ring_chunks,
                                   k_first, v_first, f_sb, f_sh, f_ss, k_record, v_record, d_sb,
                                   d_sh, d_ss, record_on_host, open_grp, open_thr, Kg, out, o_sb,
                                   o_sh, o_ss, workspace, workspace_bytes, stream, phase);
}

extern "C" int hga_attend_decode_dca(const hga_config* cfg, int32_t L, int32_t n_closed,
                                     int64_t start_pos, const float* q_intra,
                                     const float* q_succ, const float* q_inter, int64_t q_sb,
                                     int64_t q_sh, int64_t q_ss, int32_t dca_chunk,
                                     const void* k_recent, const void* v_recent, int64_t r_sb,
                                     int64_t r_sh, int64_t r_ss, int32_t ring_chunks,
                                     const void* k_first, const void* v_first, int64_t f_sb,
                                     int64_t f_sh, int64_t f_ss, const void* k_record,
                                     const void* v_record, int64_t d_sb, int64_t d_sh,
                                     int64_t d_ss, int32_t record_on_host,
                                     const int32_t* open_grp, const int32_t* open_pos,
                                     const int32_t* open_thr, int32_t Kg, void* out, int64_t o_sb,
                                     int64_t o_sh, int64_t o_ss, void* workspace,
                                     int64_t workspace_bytes, void* stream) {
    const float* qd[3] = {q_intra, q_succ, q_inter};
    return hga::attend_decode_impl(cfg, L, n_closed, start_pos, nullptr, q_sb, q_sh, q_ss, qd,
                                   open_pos, dca_chunk, k_recent, v_recent, r_sb, r_sh, r_ss,
                                   ring_chunks, k_first, v_first, f_sb, f_sh, f_ss, k_record,
                                   v_record, d_sb, d_sh, d_ss, record_on_host, open_grp, open_thr,
                                   Kg, out, o_sb, o_sh, o_ss, workspace, workspace_bytes, stream);
}

// ------------------------------------------------------------------------------------------
// hga_attend_decode_noalloc: hga_attend_decode with its split partials in a static device
// array instead of a caller workspace, for callers that cannot allocate device memory
// ------------------------------------------------------------------------------------------
// The partials of every call on a device go to that device's copy of `scratch`; a call needs no
// part of it cleared (each split writes its partial before the combine reads it).  Calls that
// overlap on one device (two streams, two threads) race on it.  Host code never passes the
// array's name to a kernel: its device address comes from hipGetSymbolAddress on each device.
constexpr int64_t kNoAllocScratchBytes = 32ll << 20;     // per device, held until process exit
static __device__ __align__(256) float scratch[kNoAllocScratchBytes / 4];

namespace {
constexpr int kNoAllocMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kNoAllocMaxDevices] = {};

// Device address of the current device's scratch array (looked up once per device).
int scratch_for_current_device(void** ptr) {
    int dev = -1;
    const hipError_t e = hipGetDevice(&dev);
    HGA_REQUIRE(e == hipSuccess && dev >= 0 && dev < kNoAllocMaxDevices, HGA_ERR_LAUNCH,
                "hga_attend_decode_noalloc: no current device (%s)", hipGetErrorString(e));
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void* p = nullptr;
        const hipError_t es = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        HGA_REQUIRE(es == hipSuccess && p, HGA_ERR_LAUNCH,
                    "hga_attend_decode_noalloc: scratch address on device %d: %s", dev,
                    hipGetErrorString(es));
        g_scratch_ptr[dev] = p;
    }
    *ptr = g_scratch_ptr[dev];
    return HGA_OK;
}
}  // namespace

extern "C" int hga_attend_decode_noalloc(const hga_config* cfg, int32_t L, int32_t n_closed,
                                         int64_t start_pos, const void* q, int64_t q_sb,
                                         int64_t q_sh, int64_t q_ss, const void* k_recent,
                                         const void* v_recent, int64_t r_sb, int64_t r_sh,
                                         int64_t r_ss, int32_t ring_chunks, const void* k_first,
                                         const void* v_first, int64_t f_sb, int64_t f_sh,
                                         int64_t f_ss, const void* k_record, const void* v_record,
                                         int64_t d_sb, int64_t d_sh, int64_t d_ss,
                                         int32_t record_on_host, const int32_t* open_grp,
                                         const int32_t* open_thr, int32_t Kg, void* out,
                                         int64_t o_sb, int64_t o_sh, int64_t o_ss, void* stream) {
    using namespace hga;
    int rc = check_config(cfg);
    if (rc) return rc;
    HGA_REQUIRE(q, HGA_ERR_ARG, "hga_attend_decode_noalloc: NULL pointer");
    HGA_REQUIRE(L >= 1 && L <= kMaxL && n_closed >= 0 && Kg >= 0 && Kg <= 256, HGA_ERR_ARG,
                "hga_attend_decode_noalloc: bad L/n_closed/Kg");
    const int64_t c0 = start_pos - (int64_t)n_closed * cfg->chunk_size;
    HGA_REQUIRE(c0 >= 0 && c0 + L <= cfg->chunk_size, HGA_ERR_ARG,
                "hga_attend_decode_noalloc: block [%lld, +%d) is not inside active chunk %d",
                (long long)start_pos, L, n_closed);
    int64_t need = 0;
    rc = hga_attend_decode_workspace(cfg, L, n_closed, start_pos, Kg, &need);
    if (rc) return rc;
    HGA_REQUIRE(need <= kNoAllocScratchBytes, HGA_ERR_UNSUPPORTED,
                "hga_attend_decode_noalloc: %lld bytes of partials exceed the static scratch of "
                "%lld bytes (call hga_attend_decode with a workspace)",
                (long long)need, (long long)kNoAllocScratchBytes);
    void* ws = nullptr;
    rc = scratch_for_current_device(&ws);
    if (rc) return rc;
    return attend_decode_impl(cfg, L, n_closed, start_pos, q, q_sb, q_sh, q_ss, nullptr, nullptr,
                              0, k_recent, v_recent, r_sb, r_sh, r_ss, ring_chunks, k_first,
                              v_first, f_sb, f_sh, f_ss, k_record, v_record, d_sb, d_sh, d_ss,
                              record_on_host, open_grp, open_thr, Kg, out, o_sb, o_sh, o_ss, ws,
                              kNoAllocScratchBytes, stream);
}

// ------------------------------------------------------------------------------------------
// RAM / disk tier decode attention with the opened groups' copy overlapped (one host call)
// ------------------------------------------------------------------------------------------
namespace {
// Side stream (default priority, non-blocking) and two events per device, for the calling
// thread: created on first use, kept until the thread ends (a thread's calls are ordered, so
// its events are never recorded twice before they are waited on).
struct SideRes {
    hipStream_t st = nullptr;
    hipEvent_t ready = nullptr, done = nullptr;   // done: the side stream's work is finished
};
constexpr int kMaxDev = 64;
thread_local SideRes t_side[kMaxDev];

int side_resources(SideRes** out) {
    int dev = 0;
    HGA_REQUIRE(hipGetDevice(&dev) == hipSuccess && dev >= 0 && dev < kMaxDev, HGA_ERR_LAUNCH,
                "hga_attend_decode_overlapped: no current device");
    SideRes& r = t_side[dev];
    if (!r.st) {
        HGA_REQUIRE(hipStreamCreateWithFlags(&r.st, hipStreamNonBlocking) == hipSuccess &&
                        hipEventCreateWithFlags(&r.ready, hipEventDisableTiming) == hipSuccess &&
                        hipEventCreateWithFlags(&r.done, hipEventDisableTiming) == hipSuccess,
                    HGA_ERR_LAUNCH, "hga_attend_decode_overlapped: cannot create the side stream");
    }
    *out = &r;
    return HGA_OK;
}
}  // namespace

extern "C" int hga_attend_decode_overlapped(
    const hga_config* cfg, int32_t L, int32_t n_closed, int64_t start_pos, const void* q,
    int64_t q_sb, int64_t q_sh, int64_t q_ss, const void* k_recent, const void* v_recent,
    int64_t r_sb, int64_t r_sh, int64_t r_ss, int32_t ring_chunks, const void* k_first,
    const void* v_first, int64_t f_sb, int64_t f_sh, int64_t f_ss, const void* k_record,
    const void* v_record, int64_t d_sb, int64_t d_sh, int64_t d_ss, int32_t record_on_host,
    int32_t record_chunks, const int32_t* record_grp, const int32_t* open_grp,
    const int32_t* open_thr, int32_t Kg, void* stage_k, void* stage_v, int32_t stage_groups,
    int32_t* staged_grp, void* scratch, int64_t scratch_bytes, void* out, int64_t o_sb,
    int64_t o_sh, int64_t o_ss, void* workspace, int64_t workspace_bytes, void* stream) {
    using namespace hga;
    int rc = check_config(cfg);
    if (rc) return rc;
    HGA_REQUIRE(q && out && open_grp && open_thr && record_grp && stage_k && stage_v &&
                    staged_grp,
                HGA_ERR_ARG, "hga_attend_decode_overlapped: NULL pointer");
    HGA_REQUIRE(cfg->head_dim == 64 || cfg->head_dim == 128, HGA_ERR_UNSUPPORTED,
                "hga_attend_decode_overlapped: head_dim 64 or 128");
    SideRes* sr = nullptr;
    rc = side_resources(&sr);
    if (rc) return rc;
    hipStream_t st = (hipStream_t)stream;
    const int64_t D = cfg->head_dim, gs = cfg->group_size;
    const int64_t s_sh = (int64_t)stage_groups * gs * D, s_sb = (int64_t)cfg->kv_heads * s_sh;
    // The copy is the long pole, so it stays on `stream` right behind the routing; the window and
    // active-chunk attention (phase 1, partials into the workspace, the record not read) runs on
    // the side stream, ordered after everything issued on `stream` so far, and `stream` waits for
    // it only before phase 2, which attends the staged groups and combines all partials.
    HGA_REQUIRE(hipEventRecord(sr->ready, st) == hipSuccess &&
                    hipStreamWaitEvent(sr->st, sr->ready, 0) == hipSuccess,
                HGA_ERR_LAUNCH, "hga_attend_decode_overlapped: cannot order the side stream");
    rc = hga_attend_decode_phase(cfg, L, n_closed, start_pos, q, q_sb, q_sh, q_ss, k_recent,
                                 v_recent, r_sb, r_sh, r_ss, ring_chunks, k_first, v_first, f_sb,
                                 f_sh, f_ss, stage_k, stage_v, s_sb, s_sh, D, 0, open_grp,
                                 open_thr, Kg, out, o_sb, o_sh, o_ss, 1, workspace,
                                 workspace_bytes, sr->st);
    if (rc) return rc;
    HGA_REQUIRE(hipEventRecord(sr->done, sr->st) == hipSuccess, HGA_ERR_LAUNCH,
                "hga_attend_decode_overlapped: cannot record the window attention");
    rc = hga_gather_decode(cfg, record_chunks, record_grp, open_thr, Kg, k_record, v_record, d_sb,
                           d_sh, d_ss, record_on_host, stage_k, stage_v, stage_groups, staged_grp,
                           scratch, scratch_bytes, stream);
    if (rc) return rc;
    HGA_REQUIRE(hipStreamWaitEvent(st, sr->done, 0) == hipSuccess, HGA_ERR_LAUNCH,
                "hga_attend_decode_overlapped: cannot wait for the window attention");
    // phase 2 reads the staging as a record [B, KVH, stage_groups * gs, Dh]
    return hga_attend_decode_phase(cfg, L, n_closed, start_pos, q, q_sb, q_sh, q_ss, k_recent,
                                   v_recent, r_sb, r_sh, r_ss, ring_chunks, k_first, v_first, f_sb,
                                   f_sh, f_ss, stage_k, stage_v, s_sb, s_sh, D, 0, staged_grp,
                                   open_thr, Kg, out, o_sb, o_sh, o_ss, 2, workspace,
                                   workspace_bytes, stream);
}
