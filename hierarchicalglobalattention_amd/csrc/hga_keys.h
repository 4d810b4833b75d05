// Key sequence of a prefill query chunk and the (b, h, chunk) dispatch order, shared by the
// attention kernels and their backward.
//
// Key sequence of query chunk n (row t sees key k iff t >= thr(k)):
//   [first window 0..f_hi*C)            thr 0
//   [last window l_lo*C..n*C)           thr 0
//   [opened groups, gs tokens each]     thr = the group's first visible row
//   [own chunk n*C + j, j < rows]       thr = j   (causal)
#pragma once
#include "hga_common.h"

namespace hga {
namespace {

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
    // NULL or [B, H, S]: each row's log-sum-exp of its scores times scale*log2(e), in log2 units
    // (written by the forward kernels, read by the backward instead of recomputing it)
    float* lse;
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
            // an invalid entry inside the list (group or first row < 0) is never visible
            const int g = (k - a2) / gs, e = (k - a2) % gs;
            const int grp = og[g], t = ot[g];
            pos = grp >= 0 && t >= 0 ? (grp / M) * C + (grp % M) * gs + e : 0;
            thr = grp >= 0 && t >= 0 ? t : kNever;
        } else if (k < a4) {
            pos = n * C + (k - a3);
            thr = k - a3;
        } else {
            pos = 0;
            thr = kNever;
        }
    }
};

// Maps a dispatch index to (b, h, n).  Blocks are dispatched round-robin over the 8 XCDs, each
// with its own L2; every XCD takes a contiguous range of logical = ((b*KVH + kvh)*N + n)*rep +
// h % rep, so an XCD works on one (b, kv head) -- or a chunk range of it -- at a time and the
// opened groups its in-flight blocks share (same K/V) meet in its L2; the rep heads of one
// (b, kv head, n) are consecutive blocks (shared windows and own chunk).
__device__ __forceinline__ void block_coords(int nblk, int B, int H, int KVH, int N, int* b,
                                             int* h, int* n) {
    const int bid = blockIdx.x, xcd = bid % 8, slot = bid / 8;
    const int q = nblk / 8, r = nblk % 8;
    const int logical = xcd < r ? xcd * (q + 1) + slot : r * (q + 1) + (xcd - r) * q + slot;
    const int rep = H / KVH;
    const int t = logical / rep;
    *n = t % N;
    const int bk = t / N;
    *b = bk / KVH;
    *h = (bk % KVH) * rep + logical % rep;
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

}  // namespace
}  // namespace hga
