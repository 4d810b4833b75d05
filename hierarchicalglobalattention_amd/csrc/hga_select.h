// Wave-level exact top-k selection shared by the prefill and decode routers.
//
// Candidates are spread over a wave as candidate index lane + 64*j (j < J); a selection returns a
// bit mask (bit j <-> candidate lane + 64*j) of the top-k under the canonical ranking: larger
// score first, equal scores -> lower candidate index.  Scores are carried as order-preserving
// 32-bit keys (okey), 0 meaning "not a candidate".
#pragma once

#include "hga_common.h"

namespace hga {
namespace {

constexpr int kNoRow = 1 << 20;

// ------------------------------------------------------------------------------------------
// wave-wide reductions: DPP within rows of 16 lanes, then the four row results by lane reads
// ------------------------------------------------------------------------------------------
template <int CTRL>
__device__ __forceinline__ int dpp(int x) {
    return __builtin_amdgcn_update_dpp(x, x, CTRL, 0xf, 0xf, false);
}
template <class Op>
__device__ __forceinline__ int wave_reduce_bits(int x, Op op) {
    x = op(x, dpp<0xB1>(x));    // quad_perm [1,0,3,2]
    x = op(x, dpp<0x4E>(x));    // quad_perm [2,3,0,1]
    x = op(x, dpp<0x124>(x));   // row_ror:4
    x = op(x, dpp<0x128>(x));   // row_ror:8
    const int a = __builtin_amdgcn_readlane(x, 0), b = __builtin_amdgcn_readlane(x, 16);
    const int c = __builtin_amdgcn_readlane(x, 32), d = __builtin_amdgcn_readlane(x, 48);
    return op(op(a, b), op(c, d));
}
__device__ __forceinline__ float wmax(float v) {
    return __int_as_float(wave_reduce_bits(__float_as_int(v), [](int a, int b) {
        return __float_as_int(fmaxf(__int_as_float(a), __int_as_float(b)));
    }));
}
__device__ __forceinline__ float wmin(float v) {
    return __int_as_float(wave_reduce_bits(__float_as_int(v), [](int a, int b) {
        return __float_as_int(fminf(__int_as_float(a), __int_as_float(b)));
    }));
}
__device__ __forceinline__ float wsum(float v) {
    return __int_as_float(wave_reduce_bits(__float_as_int(v), [](int a, int b) {
        return __float_as_int(__int_as_float(a) + __int_as_float(b));
    }));
}

// ------------------------------------------------------------------------------------------
// wave-level exact top-k over order-preserving keys (0 = not a candidate)
// ------------------------------------------------------------------------------------------
template <int J>
__device__ __forceinline__ int count_ge(const uint32_t (&kv)[J], uint32_t x) {
    int c = 0;
#pragma unroll
    for (int j = 0; j < J; ++j) c += __popcll(__ballot(kv[j] >= x));
    return c;
}

// Upper-tail standard normal quantile, Abramowitz & Stegun 26.2.23 (|error| < 4.5e-4); only
// seeds the threshold search.
__device__ __forceinline__ float z_upper(float p) {
    p = fminf(fmaxf(p, 1e-6f), 1.0f - 1e-6f);
    const bool lower = p > 0.5f;
    const float pp = lower ? 1.0f - p : p;
    const float t = sqrtf(-2.0f * logf(pp));
    const float z = t - (2.515517f + 0.802853f * t + 0.010328f * t * t) /
                            (1.0f + 1.432788f * t + 0.189269f * t * t + 0.001308f * t * t * t);
    return lower ? -z : z;
}

// Members of the top-k (largest keys; equal keys -> lower candidate index lane + 64*j).
// v holds the float values of the keys (only used to steer the search).
template <int J>
__device__ __forceinline__ uint32_t exact_topk(const uint32_t (&kv)[J], const float (&v)[J], int k) {
    const int nvalid = count_ge<J>(kv, 1u);
    uint32_t bits = 0;
    if (nvalid <= k) {
#pragma unroll
        for (int j = 0; j < J; ++j) bits |= (kv[j] != 0u ? 1u : 0u) << j;
        return bits;
    }
    if (k <= 0) return 0u;
    float s1 = 0.0f, s2 = 0.0f, mn = INFINITY, mx = -INFINITY;
#pragma unroll
    for (int j = 0; j < J; ++j)
        if (kv[j] != 0u) {
            s1 += v[j];
            s2 = fmaf(v[j], v[j], s2);
            mn = fminf(mn, v[j]);
            mx = fmaxf(mx, v[j]);
        }
    s1 = wsum(s1);
    s2 = wsum(s2);
    uint32_t lo = okey(wmin(mn)), hi = okey(wmax(mx));
    int clo = nvalid, chi = count_ge<J>(kv, hi);
    uint32_t vstar;
    if (chi >= k) {
        vstar = hi;
    } else {
        // invariant: count_ge(lo) = clo > k > chi = count_ge(hi)
        const float mu = s1 / nvalid;
        const float sd = sqrtf(fmaxf(s2 / nvalid - mu * mu, 0.0f));
        const float guess = mu + z_upper((k + 0.5f) / nvalid) * sd;
        int it = 0;
        while (hi - lo > 1u) {
            uint32_t mid = lo + (hi - lo) / 2u;
            if (it < 8) {
                const float lf = okey_inv(lo), hf = okey_inv(hi), span = hf - lf;
                float x = it == 0 ? guess : lf + span * (float)(clo - k) / (float)(clo - chi);
                x = fminf(fmaxf(x, lf + span * 0.0625f), hf - span * 0.0625f);
                if (x == x && span < INFINITY) {
                    const uint32_t xm = okey(x);
                    if (xm > lo && xm < hi) mid = xm;
                }
            }
            ++it;
            const int c = count_ge<J>(kv, mid);
            if (c == k) {
#pragma unroll
                for (int j = 0; j < J; ++j) bits |= (kv[j] >= mid ? 1u : 0u) << j;
                return bits;
            }
            if (c > k) {
                lo = mid;
                clo = c;
            } else {
                hi = mid;
                chi = c;
            }
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
__device__ __forceinline__ uint32_t select_certified(const float (&v)[J], int k, float delta, Canon canon,
                                     int* amb) {
    uint32_t kv[J];
#pragma unroll
    for (int j = 0; j < J; ++j) kv[j] = (v[j] == -INFINITY) ? 0u : okey(v[j]);
    const uint32_t bits = exact_topk<J>(kv, v, k);
    if (!(delta > 0.0f)) return bits;
    if (count_ge<J>(kv, 1u) <= k) return bits;
    float ak = INFINITY, ak1 = -INFINITY;
#pragma unroll
    for (int j = 0; j < J; ++j) {
        if (kv[j] == 0u) continue;
        if ((bits >> j) & 1u) ak = fminf(ak, v[j]);
        else ak1 = fmaxf(ak1, v[j]);
    }
    ak = wmin(ak);
    ak1 = wmax(ak1);
    if (ak - 2.0f * delta > ak1) return bits;
    *amb += 1;
    const float band_lo = ak - 2.0f * delta, band_hi = ak1 + 2.0f * delta;
    uint32_t cin = 0, ck[J];
    float cv[J];
    int cc = 0;
#pragma unroll
    for (int j = 0; j < J; ++j) {
        const bool valid = kv[j] != 0u, mem = (bits >> j) & 1u;
        const bool certain = mem && v[j] > band_hi;
        const bool inA = valid && !certain && v[j] >= band_lo;
        cin |= (certain ? 1u : 0u) << j;
        cv[j] = inA ? canon(lane_id() + 64 * j) : -INFINITY;
        ck[j] = inA ? okey(cv[j]) : 0u;
        cc += __popcll(__ballot(certain));
    }
    return cin | exact_topk<J>(ck, cv, k - cc);
}

template <int J>
struct JTag {
    static constexpr int value = J;
};
// Calls f(JTag<J>) with the smallest J in {1,2,4,8(,16,32)} such that 64*J >= n (wave-uniform
// n <= 64*JMAX).
template <int JMAX = 8, class F>
__device__ __forceinline__ void dispatch_j(int n, F&& f) {
    if (n <= 64) f(JTag<1>{});
    else if (n <= 128) f(JTag<2>{});
    else if (n <= 256) f(JTag<4>{});
    else if (JMAX <= 8 || n <= 512) f(JTag<(JMAX < 8 ? JMAX : 8)>{});
    else if (JMAX <= 16 || n <= 1024) f(JTag<(JMAX < 16 ? JMAX : 16)>{});
    else f(JTag<JMAX>{});
}

}  // namespace
}  // namespace hga
