/*
 * hga_oracle.c -- TEST INFRASTRUCTURE ONLY.
 *
 * A plain-C, single-threaded restatement of the reference's routed exact-token attention path
 * (vfedosov77/HierarchicalGlobalAttention, ExistingModelFineTuning/KvRouter).  It is the parity
 * checker for the HIP kernels of hierarchicalglobalattention_amd: only tests/, the smoke check
 * and bench.py's cpu_baseline leg may load it.  The product path never calls it.
 *
 * All tensors are float32 arrays; bf16 tensors are represented by float32 values that are
 * exactly representable in bf16 (dt == DT_BF16 makes every rounding step of the reference's
 * bf16 path round to bf16 with round-to-nearest-even).  Build with -ffp-contract=off: each
 * float operation below is a single IEEE round-to-nearest step unless fmaf() is written.
 *
 * Canonical semantics (what "bit-exact selection" means):
 *   * router score s(t, c) = RN32(chain(q_t, k_c) * scale), chain = sequential fp32 FMA over
 *     d = 0..Dh-1 starting from +0; -0 is treated as +0;
 *   * ranking = (score descending, absolute index ascending);
 *   * summaries: group sums sequential over the group's tokens in fp32, chunk sums = sequential
 *     fp32 sum of the (unrounded) group sums; then the reference's dtype roundings.
 *   Masked candidates (fill -1e4 in the reference) never outrank a real score; this assumes
 *   |score| < 1e4, which holds for any normalised activations.
 *
 * Parity pins: tests/test_oracle_golden.py compares the routing, summary and attention
 * functions here against fixtures written by the reference itself (tests/golden/make_golden.py),
 * tests/test_oracle_props.py against closed forms and invariants, tests/test_oracle_dca.py the
 * Dual Chunk Attention decode against dense DCA, and tests/test_oracle_bwd.py the attention
 * gradient against float64 autograd of the masked dense attention.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define DT_F32 0
#define DT_BF16 1

static float bf16_rne(float x) {
    uint32_t u;
    memcpy(&u, &x, 4);
    if ((u & 0x7f800000u) == 0x7f800000u) return x;
    u += 0x7fffu + ((u >> 16) & 1u);
    u &= 0xffff0000u;
    memcpy(&x, &u, 4);
    return x;
}

static float rd(float x, int dt) { return dt == DT_BF16 ? bf16_rne(x) : x; }

float orc_bf16_round(float x) { return bf16_rne(x); }

/* ------------------------------------------------------------------------------------------
 * RoPE, rotate-half convention (HierarchicalGlobalAttentionRouted.py:219-223, applied in fp32
 * then cast to the activation dtype at :156-157):  out = x*cos + cat(-x2, x1)*sin.
 * x/out: [B, X, S, Dh]; cos/sin: [Bc, S, Dh] with Bc in {1, B} (cos_bstride = 0 or S*Dh).
 * ------------------------------------------------------------------------------------------ */
void orc_rope(const float* x, float* out, const float* cos_t, const float* sin_t, int B, int X,
              int S, int Dh, long cos_bstride, int dt) {
    const int half = Dh / 2;
    for (int b = 0; b < B; ++b)
        for (int h = 0; h < X; ++h)
            for (int s = 0; s < S; ++s) {
                const float* xr = x + (((long)b * X + h) * S + s) * Dh;
                float* orow = out + (((long)b * X + h) * S + s) * Dh;
                const float* cr = cos_t + b * cos_bstride + (long)s * Dh;
                const float* sr = sin_t + b * cos_bstride + (long)s * Dh;
                for (int d = 0; d < Dh; ++d) {
                    float rot = d < half ? -xr[d + half] : xr[d - half];
                    float a = xr[d] * cr[d];
                    float c = rot * sr[d];
                    orow[d] = rd(a + c, dt);
                }
            }
}

/* ------------------------------------------------------------------------------------------
 * Mixed-RoPE key summaries (vectorized.py:146-183 applied at :265-287; the store twin
 * chunk_router.py:575-585, 631-652, 693-735).  For every chunk n and group m of the block:
 *   raw_sum  = rd(rd(sum of valid k_raw) * scale)        (scale = 1 for chunks)
 *   tokenwise= rd(rd(sum of valid k_rope) * scale)
 *   endpoint = rd(raw_sum*cos[a] + rot(raw_sum)*sin[a])   (fp32 math, anchor position a)
 *   summary  = pair(d) < cutoff ? tokenwise : endpoint
 * anchors: chunk  a = min(n*C + (max(len,1)-1)/2, S-1); group a = min(n*C + m*gs +
 * (max(glen,1)-1)/2, S-1) (vectorized.py:265-270).  For full chunks these equal the store's
 * fixed anchors n*C+(C-1)/2 and n*C+m*gs+(gs-1)/2 (chunk_router.py:580,584).
 * cos_t/sin_t: fp32 table rows indexed by absolute position pos0 + local position; the caller
 * passes values already rounded the way the reference's table is (dtype table for the
 * vectorized path, fp32 for the store).
 * k_raw/k_rope: [B, KVH, S, Dh];  chunk_k: [B, KVH, N, Dh];  group_k: [B, KVH, N, M, Dh].
 * ------------------------------------------------------------------------------------------ */
void orc_summarize(const float* k_raw, const float* k_rope, const float* cos_t,
                   const float* sin_t, long pos0, int B, int KVH, int S, int Dh, int C, int gs,
                   int cutoff, float gscale, int dt, float* chunk_k, float* group_k) {
    const int N = (S + C - 1) / C, M = C / gs, half = Dh / 2;
    float* gsum_raw = (float*)malloc(sizeof(float) * M * Dh);
    float* gsum_rope = (float*)malloc(sizeof(float) * M * Dh);
    float* tmp_raw = (float*)malloc(sizeof(float) * Dh);
    float* tmp_tok = (float*)malloc(sizeof(float) * Dh);
    for (int b = 0; b < B; ++b)
        for (int h = 0; h < KVH; ++h) {
            const long base = ((long)b * KVH + h) * S * Dh;
            for (int n = 0; n < N; ++n) {
                int len = S - n * C;
                if (len > C) len = C;
                for (int m = 0; m < M; ++m) {
                    int glen = len - m * gs;
                    if (glen < 0) glen = 0;
                    if (glen > gs) glen = gs;
                    for (int d = 0; d < Dh; ++d) {
                        float ar = 0.0f, ap = 0.0f;
                        for (int t = 0; t < glen; ++t) {
                            long off = base + (long)(n * C + m * gs + t) * Dh + d;
                            ar = ar + k_raw[off];
                            ap = ap + k_rope[off];
                        }
                        gsum_raw[m * Dh + d] = ar;
                        gsum_rope[m * Dh + d] = ap;
                    }
                    /* group summary */
                    long a = (long)n * C + m * gs + ((glen > 1 ? glen : 1) - 1) / 2;
                    if (a > S - 1) a = S - 1;
                    const float* cr = cos_t + (pos0 + a) * Dh;
                    const float* sr = sin_t + (pos0 + a) * Dh;
                    for (int d = 0; d < Dh; ++d) {
                        tmp_raw[d] = rd(rd(gsum_raw[m * Dh + d], dt) * gscale, dt);
                        tmp_tok[d] = rd(rd(gsum_rope[m * Dh + d], dt) * gscale, dt);
                    }
                    float* go = group_k + ((((long)b * KVH + h) * N + n) * M + m) * Dh;
                    for (int d = 0; d < Dh; ++d) {
                        float rot = d < half ? -tmp_raw[d + half] : tmp_raw[d - half];
                        float e = rd(tmp_raw[d] * cr[d] + rot * sr[d], dt);
                        go[d] = (d % half) < cutoff ? tmp_tok[d] : e;
                    }
                }
                /* chunk summary: sequential sum of the unrounded group sums, scale 1 */
                long a = (long)n * C + ((len > 1 ? len : 1) - 1) / 2;
                if (a > S - 1) a = S - 1;
                const float* cr = cos_t + (pos0 + a) * Dh;
                const float* sr = sin_t + (pos0 + a) * Dh;
                for (int d = 0; d < Dh; ++d) {
                    float sr_ = 0.0f, sp_ = 0.0f;
                    for (int m = 0; m < M; ++m) {
                        sr_ = sr_ + gsum_raw[m * Dh + d];
                        sp_ = sp_ + gsum_rope[m * Dh + d];
                    }
                    tmp_raw[d] = rd(sr_, dt);
                    tmp_tok[d] = rd(sp_, dt);
                }
                float* co = chunk_k + (((long)b * KVH + h) * N + n) * Dh;
                for (int d = 0; d < Dh; ++d) {
                    float rot = d < half ? -tmp_raw[d + half] : tmp_raw[d - half];
                    float e = rd(tmp_raw[d] * cr[d] + rot * sr[d], dt);
                    co[d] = (d % half) < cutoff ? tmp_tok[d] : e;
                }
            }
        }
    free(gsum_raw);
    free(gsum_rope);
    free(tmp_raw);
    free(tmp_tok);
}

/* ------------------------------------------------------------------------------------------
 * Canonical router score and ranking.
 * ------------------------------------------------------------------------------------------ */
float orc_score(const float* q, const float* k, int Dh, float scale) {
    float acc = 0.0f;
    for (int d = 0; d < Dh; ++d) acc = fmaf(q[d], k[d], acc);
    float s = acc * scale;
    return s == 0.0f ? 0.0f : s;
}

typedef struct {
    float s;
    int id;
} item_t;

/* a ranks before b: higher score first, then lower index */
static int rank_cmp(const void* pa, const void* pb) {
    const item_t* a = (const item_t*)pa;
    const item_t* b = (const item_t*)pb;
    if (a->s > b->s) return -1;
    if (a->s < b->s) return 1;
    return (a->id < b->id) ? -1 : (a->id > b->id);
}

/* top-k of items (in place sort), returns count taken = min(k, n) */
static int topk_items(item_t* it, int n, int k) {
    qsort(it, (size_t)n, sizeof(item_t), rank_cmp);
    return k < n ? k : n;
}

/* Write (id, thr) pairs ascending by id into out arrays of width w, pad with -1. */
static void emit_sorted(const int* ids, const int* thr, int n, int* out_id, int* out_thr, int w,
                        int* out_n) {
    item_t* tmp = (item_t*)malloc(sizeof(item_t) * (n > 0 ? n : 1));
    for (int i = 0; i < n; ++i) {
        tmp[i].id = ids[i];
        tmp[i].s = (float)thr[i];
    }
    /* sort by id ascending */
    for (int i = 1; i < n; ++i) {
        item_t x = tmp[i];
        int j = i - 1;
        while (j >= 0 && tmp[j].id > x.id) {
            tmp[j + 1] = tmp[j];
            --j;
        }
        tmp[j + 1] = x;
    }
    for (int i = 0; i < w; ++i) {
        out_id[i] = i < n ? tmp[i].id : -1;
        out_thr[i] = i < n ? (int)tmp[i].s : -1;
    }
    *out_n = n;
    free(tmp);
}

/* ------------------------------------------------------------------------------------------
 * Prefill two-level routing for one block starting at position 0 (vectorized.py:242-396).
 * For query chunk n:  f_hi = min(kf, n) (0 if kf == 0);  l_lo = min(max(kf, n-kl), n)
 * (n if kl == 0);  routing pool P(n) = [f_hi, l_lo)  (vectorized.py:246-253, 296-301).
 * Stage 1 (:304-337): each valid row t requests its top-min(Kc,|P|) pool chunks; a chunk's
 *   pooled score is the max over requesting rows; the top-Kc requested chunks by pooled score
 *   are selected; if n-1 is in P(n) and missing, the last-ranked selected chunk is replaced
 *   by n-1.  thrA(c) = first row that requested c, and 0 for n-1.
 * Stage 2 (:339-396): candidates = groups of the selected chunks; row t sees group (c,m) iff
 *   t >= thrA(c); each row requests its top-min(Kgr, visible) groups; pooled max; the top-Kg
 *   requested groups are opened; thrD(g) = first row that requested g.
 * Kc = min(topk_chunks, N); Kg = min(topk_groups, Kc*M); Kgr = min(topk_groups/2, Kc*M).
 * Outputs (ascending ids, -1 padded):
 *   sel_chunk/sel_thr [B,H,N,Kcw], n_sel [B,H,N]; open_grp (= c*M+m)/open_thr [B,H,N,Kgw],
 *   n_open [B,H,N].  Kcw >= Kc and Kgw >= Kg are the widths of the caller's arrays.
 * ------------------------------------------------------------------------------------------ */
void orc_route_prefill(const float* q, const float* chunk_k, const float* group_k, int B, int H,
                       int KVH, int S, int Dh, int C, int gs, int kf, int kl, int topk_chunks,
                       int topk_groups, float scale, int Kcw, int Kgw, int* sel_chunk,
                       int* sel_thr, int* n_sel, int* open_grp, int* open_thr, int* n_open) {
    const int N = (S + C - 1) / C, M = C / gs, rep = H / KVH;
    const int Kc = topk_chunks > 0 ? (topk_chunks < N ? topk_chunks : N) : 0;
    const int Tgrp = Kc * M;
    const int Kg = topk_groups > 0 ? (topk_groups < Tgrp ? topk_groups : Tgrp) : 0;
    const int Kgr = topk_groups > 0 ? (topk_groups / 2 < Tgrp ? topk_groups / 2 : Tgrp) : 0;
    item_t* items = (item_t*)malloc(sizeof(item_t) * (N * M + 8));
    float* pooled = (float*)malloc(sizeof(float) * (N * M + 8));
    int* first = (int*)malloc(sizeof(int) * (N * M + 8));
    int* sel = (int*)malloc(sizeof(int) * (N + 8));
    int* thrA = (int*)malloc(sizeof(int) * (N + 8));
    int* gid = (int*)malloc(sizeof(int) * (N * M + 8));
    int* gthr = (int*)malloc(sizeof(int) * (N * M + 8));
    float* scores = (float*)malloc(sizeof(float) * (N * M + 8));
    int* oid = (int*)malloc(sizeof(int) * (N * M + 8));
    for (int b = 0; b < B; ++b)
        for (int h = 0; h < H; ++h) {
            const int kvh = h / rep;
            for (int n = 0; n < N; ++n) {
                const long o = ((long)b * H + h) * N + n;
                int* oc = sel_chunk + o * Kcw;
                int* ot = sel_thr + o * Kcw;
                int* og = open_grp + o * Kgw;
                int* ogt = open_thr + o * Kgw;
                int f_hi = kf > 0 ? (n < kf ? n : kf) : 0;
                int l_lo = n;
                if (kl > 0) {
                    int x = n - kl > kf ? n - kl : kf;
                    l_lo = x < n ? x : n;
                }
                int P = l_lo - f_hi;
                int rows = S - n * C < C ? S - n * C : C;
                int nsel = 0;
                if (Kc > 0 && P > 0) {
                    const int kreq = Kc < P ? Kc : P;
                    for (int c = 0; c < P; ++c) {
                        pooled[c] = -INFINITY;
                        first[c] = -1;
                    }
                    for (int t = 0; t < rows; ++t) {
                        const float* qr = q + (((long)b * H + h) * S + n * C + t) * Dh;
                        for (int c = 0; c < P; ++c) {
                            items[c].id = f_hi + c;
                            items[c].s = orc_score(
                                qr, chunk_k + (((long)b * KVH + kvh) * N + f_hi + c) * Dh, Dh,
                                scale);
                        }
                        topk_items(items, P, kreq);
                        for (int j = 0; j < kreq; ++j) {
                            int c = items[j].id - f_hi;
                            if (items[j].s > pooled[c]) pooled[c] = items[j].s;
                            if (first[c] < 0) first[c] = t;
                        }
                    }
                    int nu = 0;
                    for (int c = 0; c < P; ++c)
                        if (first[c] >= 0) {
                            items[nu].id = f_hi + c;
                            items[nu].s = pooled[c];
                            ++nu;
                        }
                    nsel = topk_items(items, nu, Kc); /* ranked, best first */
                    for (int j = 0; j < nsel; ++j) {
                        sel[j] = items[j].id;
                        thrA[j] = first[items[j].id - f_hi];
                    }
                    const int prev = n - 1;
                    if (n > 0 && prev >= f_hi && prev < l_lo) {
                        int have = -1;
                        for (int j = 0; j < nsel; ++j)
                            if (sel[j] == prev) have = j;
                        if (have < 0) {
                            if (nsel == Kc) have = nsel - 1; /* evict the last-ranked */
                            else have = nsel++;
                            sel[have] = prev;
                        }
                        thrA[have] = 0;
                    }
                }
                emit_sorted(sel, thrA, nsel, oc, ot, Kcw, &n_sel[o]);
                int nopen = 0;
                if (Kg > 0 && Kgr > 0 && nsel > 0) {
                    const int T2 = nsel * M;
                    for (int j = 0; j < T2; ++j) {
                        gid[j] = sel[j / M] * M + (j % M);
                        pooled[j] = -INFINITY;
                        first[j] = -1;
                    }
                    for (int t = 0; t < rows; ++t) {
                        const float* qr = q + (((long)b * H + h) * S + n * C + t) * Dh;
                        int nv = 0;
                        for (int j = 0; j < T2; ++j) {
                            if (thrA[j / M] > t) continue;
                            const int c = gid[j] / M, m = gid[j] % M;
                            items[nv].id = j; /* slot; ranking uses absolute id below */
                            items[nv].s = orc_score(
                                qr,
                                group_k + ((((long)b * KVH + kvh) * N + c) * M + m) * Dh, Dh,
                                scale);
                            scores[j] = items[nv].s;
                            ++nv;
                        }
                        for (int i = 0; i < nv; ++i) items[i].id = gid[items[i].id];
                        int kr = topk_items(items, nv, Kgr);
                        for (int i = 0; i < kr; ++i) {
                            int j = 0;
                            while (gid[j] != items[i].id) ++j;
                            if (scores[j] > pooled[j]) pooled[j] = scores[j];
                            if (first[j] < 0) first[j] = t;
                        }
                    }
                    int nu = 0;
                    for (int j = 0; j < T2; ++j)
                        if (first[j] >= 0) {
                            items[nu].id = j; /* slot */
                            items[nu].s = pooled[j];
                            ++nu;
                        }
                    for (int i = 0; i < nu; ++i) items[i].id = gid[items[i].id];
                    nopen = topk_items(items, nu, Kg);
                    for (int i = 0; i < nopen; ++i) {
                        int j = 0;
                        while (gid[j] != items[i].id) ++j;
                        gthr[i] = first[j];
                        oid[i] = items[i].id;
                    }
                }
                emit_sorted(oid, gthr, nopen, og, ogt, Kgw, &n_open[o]);
            }
        }
    free(items);
    free(pooled);
    free(first);
    free(sel);
    free(thrA);
    free(gid);
    free(gthr);
    free(scores);
    free(oid);
}

/* ------------------------------------------------------------------------------------------
 * Exact attention over the routed working set, chunk-parallel layout
 * (vectorized.py:404-490 assembles the set, RoutedKV.attend chunked at chunk_router.py:149-158
 * computes it).  Valid query row t of chunk n (absolute i = n*C + t) sees:
 *   current chunk tokens n*C + j, j <= t;  first window chunks [0, f_hi);  last window chunks
 *   [l_lo, n);  every opened group g = c*M + m with open_thr <= t (tokens c*C + m*gs + [0,gs)).
 * Masked columns in the reference carry -1e4 and vanish in the fp32 softmax; here they are
 * simply absent.  Math in double, result rounded to dt.  q/out [B,H,S,Dh], k/v [B,KVH,S,Dh].
 * ------------------------------------------------------------------------------------------ */
static void attend_row_sel(const float* const* qsel, const int* regime, const float* kb,
                           const float* vb, const long* keys, int nk, int Dh, double scale,
                           int dt, float* orow, double* p) {
    double mx = -INFINITY;
    for (int j = 0; j < nk; ++j) {
        const float* qr = qsel[regime ? regime[j] : 0];
        const float* kr = kb + keys[j] * Dh;
        double s = 0.0;
        for (int d = 0; d < Dh; ++d) s += (double)qr[d] * (double)kr[d];
        p[j] = s * scale;
        if (p[j] > mx) mx = p[j];
    }
    double den = 0.0;
    for (int j = 0; j < nk; ++j) {
        p[j] = exp(p[j] - mx);
        den += p[j];
    }
    for (int d = 0; d < Dh; ++d) {
        double acc = 0.0;
        for (int j = 0; j < nk; ++j) acc += p[j] * (double)vb[keys[j] * Dh + d];
        orow[d] = rd((float)(acc / den), dt);
    }
}

static void attend_row(const float* qr, const float* kb, const float* vb, const long* keys,
                       int nk, int Dh, double scale, int dt, float* orow, double* p) {
    const float* qsel[1] = {qr};
    attend_row_sel(qsel, NULL, kb, vb, keys, nk, Dh, scale, dt, orow, p);
}

/* Rows of the query chunks listed in chunks[0..nchunks) only (chunks == NULL: every chunk); the
 * other rows of out are left as they are.  Lets a test check a few query chunks of a long
 * sequence in seconds. */
void orc_attend_prefill_chunks(const float* q, const float* k, const float* v, int B, int H,
                               int KVH, int S, int Dh, int C, int gs, int kf, int kl,
                               const int* open_grp, const int* open_thr, int Kgw, float scale,
                               int dt, const int* chunks, int nchunks, float* out) {
    const int N = (S + C - 1) / C, M = C / gs, rep = H / KVH;
    long* keys = (long*)malloc(sizeof(long) * ((long)S + 16));
    double* p = (double*)malloc(sizeof(double) * ((long)S + 16));
    const int nlist = chunks ? nchunks : N;
    for (int b = 0; b < B; ++b)
        for (int h = 0; h < H; ++h) {
            const int kvh = h / rep;
            const float* kb = k + ((long)b * KVH + kvh) * S * Dh;
            const float* vb = v + ((long)b * KVH + kvh) * S * Dh;
            for (int ci = 0; ci < nlist; ++ci) {
                const int n = chunks ? chunks[ci] : ci;
                if (n < 0 || n >= N) continue;
                int f_hi = kf > 0 ? (n < kf ? n : kf) : 0;
                int l_lo = n;
                if (kl > 0) {
                    int x = n - kl > kf ? n - kl : kf;
                    l_lo = x < n ? x : n;
                }
                const int* og = open_grp + (((long)b * H + h) * N + n) * Kgw;
                const int* ot = open_thr + (((long)b * H + h) * N + n) * Kgw;
                int rows = S - n * C < C ? S - n * C : C;
                for (int t = 0; t < rows; ++t) {
                    int nk = 0;
                    for (long i = 0; i < (long)f_hi * C; ++i) keys[nk++] = i;
                    for (long i = (long)l_lo * C; i < (long)n * C; ++i) keys[nk++] = i;
                    for (int j = 0; j < Kgw; ++j)
                        if (og[j] >= 0 && ot[j] >= 0 && ot[j] <= t) {
                            long base = (long)(og[j] / M) * C + (og[j] % M) * gs;
                            for (int e = 0; e < gs; ++e) keys[nk++] = base + e;
                        }
                    for (int j = 0; j <= t; ++j) keys[nk++] = (long)n * C + j;
                    const long row = (long)n * C + t;
                    attend_row(q + (((long)b * H + h) * S + row) * Dh, kb, vb, keys, nk, Dh,
                               (double)scale, dt, out + (((long)b * H + h) * S + row) * Dh, p);
                }
            }
        }
    free(keys);
    free(p);
}

void orc_attend_prefill(const float* q, const float* k, const float* v, int B, int H, int KVH,
                        int S, int Dh, int C, int gs, int kf, int kl, const int* open_grp,
                        const int* open_thr, int Kgw, float scale, int dt, float* out) {
    orc_attend_prefill_chunks(q, k, v, B, H, KVH, S, Dh, C, gs, kf, kl, open_grp, open_thr, Kgw,
                              scale, dt, NULL, 0, out);
}

/* ------------------------------------------------------------------------------------------
 * Gradient of the prefill attention above (the reference trains through it with torch
 * autograd: HierarchicalGlobalAttentionRouted.forward, :137-177, over the gathered working set
 * of vectorized.py:404-490; routing decisions carry no gradient).  Same per-row key set as
 * orc_attend_prefill; for row i with keys J(i), in double precision:
 *   p_j = softmax_j(scale q_i.k_j),  dp_j = dout_i.v_j,  D_i = sum_j p_j dp_j,
 *   ds_j = p_j (dp_j - D_i),  dq_i = scale sum_j ds_j k_j,
 *   dk_j += scale ds_j q_i,  dv_j += p_j dout_i   (summed over rows and the heads of a KV head).
 * q, dout, dq [B,H,S,Dh]; k, v, dk, dv [B,KVH,S,Dh]; open lists as orc_attend_prefill.
 * ------------------------------------------------------------------------------------------ */
void orc_attend_prefill_bwd(const float* q, const float* k, const float* v, const float* dout,
                            int B, int H, int KVH, int S, int Dh, int C, int gs, int kf, int kl,
                            const int* open_grp, const int* open_thr, int Kgw, float scale,
                            float* dq, float* dk, float* dv) {
    const int N = (S + C - 1) / C, M = C / gs, rep = H / KVH;
    long* keys = (long*)malloc(sizeof(long) * ((long)S + 16));
    double* p = (double*)malloc(sizeof(double) * ((long)S + 16));
    double* dpv = (double*)malloc(sizeof(double) * ((long)S + 16));
    double* gq = (double*)malloc(sizeof(double) * (Dh + 1));
    const long nkv = (long)B * KVH * S * Dh;
    double* gk = (double*)calloc(nkv + 1, sizeof(double));
    double* gv = (double*)calloc(nkv + 1, sizeof(double));
    for (int b = 0; b < B; ++b)
        for (int h = 0; h < H; ++h) {
            const int kvh = h / rep;
            const long kvo = ((long)b * KVH + kvh) * S * Dh;
            const float* kb = k + kvo;
            const float* vb = v + kvo;
            for (int n = 0; n < N; ++n) {
                int f_hi = kf > 0 ? (n < kf ? n : kf) : 0;
                int l_lo = n;
                if (kl > 0) {
                    int x = n - kl > kf ? n - kl : kf;
                    l_lo = x < n ? x : n;
                }
                const int* og = open_grp + (((long)b * H + h) * N + n) * Kgw;
                const int* ot = open_thr + (((long)b * H + h) * N + n) * Kgw;
                int rows = S - n * C < C ? S - n * C : C;
                for (int t = 0; t < rows; ++t) {
                    int nk = 0;
                    for (long i = 0; i < (long)f_hi * C; ++i) keys[nk++] = i;
                    for (long i = (long)l_lo * C; i < (long)n * C; ++i) keys[nk++] = i;
                    for (int j = 0; j < Kgw; ++j)
                        if (og[j] >= 0 && ot[j] >= 0 && ot[j] <= t) {
                            long base = (long)(og[j] / M) * C + (og[j] % M) * gs;
                            for (int e = 0; e < gs; ++e) keys[nk++] = base + e;
                        }
                    for (int j = 0; j <= t; ++j) keys[nk++] = (long)n * C + j;
                    const long ro = (((long)b * H + h) * S + (long)n * C + t) * Dh;
                    const float* qr = q + ro;
                    const float* gr = dout + ro;
                    double mx = -INFINITY, den = 0.0, Dsum = 0.0;
                    for (int j = 0; j < nk; ++j) {
                        double sdot = 0.0, vdot = 0.0;
                        for (int d = 0; d < Dh; ++d) {
                            sdot += (double)qr[d] * (double)kb[keys[j] * Dh + d];
                            vdot += (double)gr[d] * (double)vb[keys[j] * Dh + d];
                        }
                        p[j] = sdot * scale;
                        dpv[j] = vdot;
                        if (p[j] > mx) mx = p[j];
                    }
                    for (int j = 0; j < nk; ++j) {
                        p[j] = exp(p[j] - mx);
                        den += p[j];
                    }
                    for (int j = 0; j < nk; ++j) {
                        p[j] /= den;
                        Dsum += p[j] * dpv[j];
                    }
                    for (int d = 0; d < Dh; ++d) gq[d] = 0.0;
                    for (int j = 0; j < nk; ++j) {
                        const double ds = p[j] * (dpv[j] - Dsum);
                        const long ko = keys[j] * Dh;
                        for (int d = 0; d < Dh; ++d) {
                            gq[d] += ds * (double)kb[ko + d];
                            gk[kvo + ko + d] += (double)scale * ds * (double)qr[d];
                            gv[kvo + ko + d] += p[j] * (double)gr[d];
                        }
                    }
                    for (int d = 0; d < Dh; ++d) dq[ro + d] = (float)((double)scale * gq[d]);
                }
            }
        }
    for (long i = 0; i < nkv; ++i) {
        dk[i] = (float)gk[i];
        dv[i] = (float)gv[i];
    }
    free(keys);
    free(p);
    free(dpv);
    free(gq);
    free(gk);
    free(gv);
}

/* ------------------------------------------------------------------------------------------
 * Decode routing for an L-token block inside the active chunk (ChunkRouter._route_decision,
 * chunk_router.py:187-277).  Window ranges from ChunkPlacementPolicy
 * (chunk_placement_policy.py:27-38): f_hi = min(kf, n_closed), l_lo = min(max(kf,
 * n_closed-kl), n_closed) (n_closed if kl == 0); candidates mid = [f_hi, l_lo).
 *   Kc = min(topk_chunks, |mid|);  pooled(c) = max over ALL L rows (no masking, :227);
 *   sel = top-Kc by pooled; req(l) = top-Kc of row l (:230); forced prev n_closed-1 when it is
 *   in mid (:232-241); thrA(c) = first row requesting c, 0 for prev (:246-249).
 *   Groups: candidates = all M groups of every selected chunk, scored for every row unmasked
 *   (:263); Kg = min(topk_groups, Kc*M) opened by pooled max (:264-265); row requests
 *   top-Kgr = min(topk_groups/2, Kc*M) (:266); visible at row l iff requested at some l' <= l
 *   and l >= thrA(parent) (:273-276).
 * chunk_k [B,KVH,cap,Dh], group_k [B,KVH,cap,M,Dh] (store layout), q [B,H,L,Dh].
 * Outputs: mid/mid_thr [B,H,Kcw] (visible routed chunks), open_grp/open_thr [B,H,Kgw]
 * (opened groups visible to some row), ascending, -1 padded.
 * ------------------------------------------------------------------------------------------ */
void orc_route_decode(const float* q, const float* chunk_k, const float* group_k, long cap,
                      int B, int H, int KVH, int L, int Dh, int M, int n_closed, int kf, int kl,
                      int topk_chunks, int topk_groups, float scale, int Kcw, int Kgw, int* mid,
                      int* mid_thr, int* n_mid_out, int* open_grp, int* open_thr,
                      int* n_open) {
    const int rep = H / KVH;
    int f_hi = kf < n_closed ? kf : n_closed;
    if (f_hi < 0) f_hi = 0;
    int l_lo = n_closed;
    if (kl > 0) {
        int x = n_closed - kl > kf ? n_closed - kl : kf;
        l_lo = x < n_closed ? x : n_closed;
    }
    const int nmid = l_lo - f_hi > 0 ? l_lo - f_hi : 0;
    const int Kc = (nmid > 0 && topk_chunks > 0) ? (topk_chunks < nmid ? topk_chunks : nmid) : 0;
    const int T2 = Kc * M;
    const int Kg = topk_groups > 0 ? (topk_groups < T2 ? topk_groups : T2) : 0;
    const int Kgr = topk_groups > 0 ? (topk_groups / 2 < T2 ? topk_groups / 2 : T2) : 0;
    const int W = nmid > T2 ? nmid : T2;
    item_t* items = (item_t*)malloc(sizeof(item_t) * (W + 8));
    float* sc = (float*)malloc(sizeof(float) * ((long)L * (W + 8)));
    float* pooled = (float*)malloc(sizeof(float) * (W + 8));
    int* first = (int*)malloc(sizeof(int) * (W + 8));
    int* sel = (int*)malloc(sizeof(int) * (W + 8));
    int* thrA = (int*)malloc(sizeof(int) * (W + 8));
    int* gid = (int*)malloc(sizeof(int) * (W + 8));
    int* gthr = (int*)malloc(sizeof(int) * (W + 8));
    int* oid = (int*)malloc(sizeof(int) * (W + 8));
    int* vid = (int*)malloc(sizeof(int) * (W + 8));
    int* vthr = (int*)malloc(sizeof(int) * (W + 8));
    for (int b = 0; b < B; ++b)
        for (int h = 0; h < H; ++h) {
            const int kvh = h / rep;
            const long o = (long)b * H + h;
            int nsel = 0, nopen = 0, nvis = 0;
            if (Kc > 0) {
                for (int c = 0; c < nmid; ++c) {
                    pooled[c] = -INFINITY;
                    first[c] = -1;
                }
                for (int l = 0; l < L; ++l) {
                    const float* qr = q + ((o * L) + l) * Dh;
                    for (int c = 0; c < nmid; ++c) {
                        float s = orc_score(qr, chunk_k + (((long)b * KVH + kvh) * cap + f_hi + c) * Dh,
                                            Dh, scale);
                        sc[(long)l * nmid + c] = s;
                        if (s > pooled[c]) pooled[c] = s;
                    }
                }
                for (int c = 0; c < nmid; ++c) {
                    items[c].id = f_hi + c;
                    items[c].s = pooled[c];
                }
                nsel = topk_items(items, nmid, Kc);
                for (int j = 0; j < nsel; ++j) sel[j] = items[j].id;
                for (int l = 0; l < L; ++l) {
                    for (int c = 0; c < nmid; ++c) {
                        items[c].id = f_hi + c;
                        items[c].s = sc[(long)l * nmid + c];
                    }
                    int kr = topk_items(items, nmid, Kc);
                    for (int i = 0; i < kr; ++i)
                        if (first[items[i].id - f_hi] < 0) first[items[i].id - f_hi] = l;
                }
                const int prev = n_closed - 1;
                const int prev_in = prev >= f_hi && prev < l_lo;
                if (prev_in) {
                    int have = -1;
                    for (int j = 0; j < nsel; ++j)
                        if (sel[j] == prev) have = j;
                    if (have < 0) sel[nsel - 1] = prev; /* evict the last-ranked */
                }
                for (int j = 0; j < nsel; ++j) {
                    thrA[j] = first[sel[j] - f_hi];
                    if (prev_in && sel[j] == prev) thrA[j] = 0;
                    if (thrA[j] >= 0) {
                        vid[nvis] = sel[j];
                        vthr[nvis] = thrA[j];
                        ++nvis;
                    }
                }
                if (Kg > 0) {
                    for (int j = 0; j < T2; ++j) {
                        gid[j] = sel[j / M] * M + (j % M);
                        pooled[j] = -INFINITY;
                        first[j] = -1;
                    }
                    for (int l = 0; l < L; ++l) {
                        const float* qr = q + ((o * L) + l) * Dh;
                        for (int j = 0; j < T2; ++j) {
                            const int c = gid[j] / M, m = gid[j] % M;
                            float s = orc_score(
                                qr, group_k + ((((long)b * KVH + kvh) * cap + c) * M + m) * Dh,
                                Dh, scale);
                            sc[(long)l * T2 + j] = s;
                            if (s > pooled[j]) pooled[j] = s;
                        }
                    }
                    for (int l = 0; l < L && Kgr > 0; ++l) {
                        for (int j = 0; j < T2; ++j) {
                            items[j].id = gid[j];
                            items[j].s = sc[(long)l * T2 + j];
                        }
                        int kr = topk_items(items, T2, Kgr);
                        for (int i = 0; i < kr; ++i) {
                            int j = 0;
                            while (gid[j] != items[i].id) ++j;
                            if (first[j] < 0) first[j] = l;
                        }
                    }
                    for (int j = 0; j < T2; ++j) {
                        items[j].id = gid[j];
                        items[j].s = pooled[j];
                    }
                    int ko = topk_items(items, T2, Kg);
                    for (int i = 0; i < ko; ++i) {
                        int j = 0;
                        while (gid[j] != items[i].id) ++j;
                        const int pa = thrA[j / M];
                        if (first[j] < 0 || pa < 0) continue;
                        oid[nopen] = gid[j];
                        gthr[nopen] = first[j] > pa ? first[j] : pa;
                        ++nopen;
                    }
                }
            }
            emit_sorted(vid, vthr, nvis, mid + o * Kcw, mid_thr + o * Kcw, Kcw, &n_mid_out[o]);
            emit_sorted(oid, gthr, nopen, open_grp + o * Kgw, open_thr + o * Kgw, Kgw, &n_open[o]);
        }
    free(items);
    free(sc);
    free(pooled);
    free(first);
    free(sel);
    free(thrA);
    free(gid);
    free(gthr);
    free(oid);
    free(vid);
    free(vthr);
}

/* ------------------------------------------------------------------------------------------
 * Decode attention for an L-token block (decode_block, chunk_router.py:333-401, attended flat
 * at :159-162).  Query row l sits at absolute position start_pos + l inside active chunk
 * n_closed; it sees the first window [0, f_hi*C), the last window [l_lo*C, n_closed*C), every
 * opened group with open_thr <= l, and active-chunk tokens n_closed*C + [0, c0 + l] where
 * c0 = start_pos - n_closed*C.  k/v: full token history [B,KVH,T,Dh]; q/out [B,H,L,Dh].
 * ------------------------------------------------------------------------------------------ */
/* Decode attention over the keys a block of L rows sees (chunk_router.py:333-401).  With
 * q2/q3 set (Dual Chunk Attention, Qwen3LongContext/qwen_routed_attention.py:253-283), q, q2
 * and q3 are the rows RoPE'd at the intra, successive and inter positions, and key j is scored
 * with q when its DCA chunk (position / dca_chunk) equals the row's, with q2 when it is the one
 * before, else with q3. */
static void attend_decode_impl(const float* q, const float* q2, const float* q3, const float* k,
                               const float* v, long T, int B, int H, int KVH, int L, int Dh,
                               int C, int gs, int kf, int kl, int n_closed, long start_pos,
                               const int* open_grp, const int* open_thr, int Kgw, float scale,
                               int dt, int dca_chunk, float* out) {
    const int M = C / gs, rep = H / KVH;
    int f_hi = kf < n_closed ? kf : n_closed;
    if (f_hi < 0) f_hi = 0;
    int l_lo = n_closed;
    if (kl > 0) {
        int x = n_closed - kl > kf ? n_closed - kl : kf;
        l_lo = x < n_closed ? x : n_closed;
    }
    const long c0 = start_pos - (long)n_closed * C;
    long* keys = (long*)malloc(sizeof(long) * (T + 16));
    int* regime = q2 ? (int*)malloc(sizeof(int) * (T + 16)) : NULL;
    double* p = (double*)malloc(sizeof(double) * (T + 16));
    for (int b = 0; b < B; ++b)
        for (int h = 0; h < H; ++h) {
            const int kvh = h / rep;
            const float* kb = k + ((long)b * KVH + kvh) * T * Dh;
            const float* vb = v + ((long)b * KVH + kvh) * T * Dh;
            const int* og = open_grp + ((long)b * H + h) * Kgw;
            const int* ot = open_thr + ((long)b * H + h) * Kgw;
            for (int l = 0; l < L; ++l) {
                int nk = 0;
                for (long i = 0; i < (long)f_hi * C; ++i) keys[nk++] = i;
                for (long i = (long)l_lo * C; i < (long)n_closed * C; ++i) keys[nk++] = i;
                for (int j = 0; j < Kgw; ++j)
                    if (og[j] >= 0 && ot[j] >= 0 && ot[j] <= l) {
                        long base = (long)(og[j] / M) * C + (og[j] % M) * gs;
                        for (int e = 0; e < gs; ++e) keys[nk++] = base + e;
                    }
                for (long j = 0; j <= c0 + l; ++j) keys[nk++] = (long)n_closed * C + j;
                const long ro = (((long)b * H + h) * L + l) * Dh;
                const float* qsel[3] = {q + ro, q2 ? q2 + ro : NULL, q3 ? q3 + ro : NULL};
                if (regime) {
                    const long cq = (start_pos + l) / dca_chunk;
                    for (int j = 0; j < nk; ++j) {
                        const long ck = keys[j] / dca_chunk;
                        regime[j] = ck == cq ? 0 : (ck == cq - 1 ? 1 : 2);
                    }
                }
                attend_row_sel(qsel, regime, kb, vb, keys, nk, Dh, (double)scale, dt, out + ro, p);
            }
        }
    free(keys);
    free(regime);
    free(p);
}

void orc_attend_decode(const float* q, const float* k, const float* v, long T, int B, int H,
                       int KVH, int L, int Dh, int C, int gs, int kf, int kl, int n_closed,
                       long start_pos, const int* open_grp, const int* open_thr, int Kgw,
                       float scale, int dt, float* out) {
    attend_decode_impl(q, NULL, NULL, k, v, T, B, H, KVH, L, Dh, C, gs, kf, kl, n_closed,
                       start_pos, open_grp, open_thr, Kgw, scale, dt, 1, out);
}

void orc_attend_decode_dca(const float* q, const float* q2, const float* q3, const float* k,
                           const float* v, long T, int B, int H, int KVH, int L, int Dh, int C,
                           int gs, int kf, int kl, int n_closed, long start_pos,
                           const int* open_grp, const int* open_thr, int Kgw, float scale,
                           int dt, int dca_chunk, float* out) {
    attend_decode_impl(q, q2, q3, k, v, T, B, H, KVH, L, Dh, C, gs, kf, kl, n_closed,
                       start_pos, open_grp, open_thr, Kgw, scale, dt, dca_chunk, out);
}
