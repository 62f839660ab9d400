/*
 * Oracle (test infrastructure): SplitMix64, argmax, the sparse sampling
 * chain and speculative acceptance, restated from
 * cortiq-engine/src/sampler.rs.
 */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "oracle.h"

/* sampler.rs:71-84 */
uint64_t or_rng_next_u64(or_rng* r) {
    r->state += 0x9E3779B97F4A7C15ull;
    uint64_t z = r->state;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

float or_rng_next_f32(or_rng* r) {
    if (r->seq && r->used < r->nseq) return r->seq[r->used++];
    return (float)(or_rng_next_u64(r) >> 40) / (float)(1u << 24);
}

/* sampler.rs:832-867 — four running maxima, ties to the highest index. */
uint32_t or_argmax(const float* v, int n) {
    if (n <= 0) return 0;
    int bi_[4];
    float bv_[4];
    for (int l = 0; l < 4; l++) {
        bi_[l] = l < n - 1 ? l : n - 1;
        bv_[l] = -INFINITY;
    }
    int i = 0;
    for (; i + 4 <= n; i += 4)
        for (int l = 0; l < 4; l++)
            if (v[i + l] >= bv_[l]) {
                bv_[l] = v[i + l];
                bi_[l] = i + l;
            }
    int bi = bi_[0];
    float bv = bv_[0];
    for (int l = 1; l < 4; l++)
        if (bv_[l] > bv || (bv_[l] == bv && bi_[l] > bi)) {
            bi = bi_[l];
            bv = bv_[l];
        }
    for (; i < n; i++)
        if (v[i] >= bv) {
            bv = v[i];
            bi = i;
        }
    return (uint32_t)bi;
}

/* sampler.rs:1111-1120 */
uint32_t or_categorical(const float* p, int n, float r) {
    float c = 0.0f;
    for (int i = 0; i < n; i++) {
        c += p[i];
        if (r < c) return (uint32_t)i;
    }
    for (int i = n - 1; i >= 0; i--)
        if (p[i] > 0.0f) return (uint32_t)i;
    return 0;
}

typedef struct {
    uint32_t id;
    float v;
} cand_t;

static int better(cand_t a, cand_t b) { return a.v > b.v || (a.v == b.v && a.id < b.id); }

static int cmp_desc(const void* pa, const void* pb) {
    const cand_t *a = (const cand_t*)pa, *b = (const cand_t*)pb;
    if (a->v > b->v) return -1;
    if (a->v < b->v) return 1;
    return (a->id < b->id) ? -1 : (a->id > b->id);
}

/* sampler.rs:522-622, serial arm: k-slot insertion scan, then gather every
 * value >= the k-th (capped at 4k+64), sorted by value desc, id asc. */
static int topk_serial(const float* src, int n, int k, cand_t* out /* cap 4k+64 */) {
    int cnt = 0;
    for (int i = 0; i < n; i++) {
        cand_t c = {(uint32_t)i, src[i]};
        if (cnt < k) {
            int pos = cnt;
            for (int j = 0; j < cnt; j++)
                if (better(c, out[j])) {
                    pos = j;
                    break;
                }
            memmove(out + pos + 1, out + pos, sizeof(cand_t) * (size_t)(cnt - pos));
            out[pos] = c;
            cnt++;
        } else if (better(c, out[k - 1])) {
            int pos = k - 1;
            for (int j = 0; j < k; j++)
                if (better(c, out[j])) {
                    pos = j;
                    break;
                }
            memmove(out + pos + 1, out + pos, sizeof(cand_t) * (size_t)(k - 1 - pos));
            out[pos] = c;
        }
    }
    if (cnt == 0) return 0;
    float kth = out[cnt - 1].v;
    if (!isfinite(kth)) return cnt;
    int cap = k * 4 + 64, m = 0;
    for (int i = 0; i < n; i++)
        if (src[i] >= kth) {
            out[m].id = (uint32_t)i;
            out[m].v = src[i];
            m++;
            if (m >= cap) break;
        }
    qsort(out, (size_t)m, sizeof(cand_t), cmp_desc);
    return m;
}

static void apply_penalties(float* p, int n, const or_sampler_cfg* c, const uint32_t* past,
                            int npast) {
    /* sampler.rs:363-393 (no suppress list in this build's configs) */
    if (c->repetition_penalty != 1.0f) {
        unsigned char* seen = (unsigned char*)calloc((size_t)n, 1);
        for (int i = 0; i < npast; i++) {
            uint32_t t = past[i];
            if ((int)t < n && !seen[t]) {
                seen[t] = 1;
                if (p[t] > 0.0f)
                    p[t] /= c->repetition_penalty;
                else
                    p[t] *= c->repetition_penalty;
            }
        }
        free(seen);
    }
    if (c->presence_penalty != 0.0f) {
        unsigned char* seen = (unsigned char*)calloc((size_t)n, 1);
        for (int i = 0; i < npast; i++) {
            uint32_t t = past[i];
            if ((int)t < n && !seen[t]) {
                seen[t] = 1;
                p[t] -= c->presence_penalty;
            }
        }
        free(seen);
    }
}

static int cmp_id(const void* pa, const void* pb) {
    const cand_t *a = (const cand_t*)pa, *b = (const cand_t*)pb;
    return (a->id < b->id) ? -1 : (a->id > b->id);
}

/* sampler.rs:440-514 */
int or_sparse_distribution(const float* logits, int n, const or_sampler_cfg* c,
                           const uint32_t* past, int npast, uint32_t* ids, float* probs) {
    int k = (int)c->top_k < n ? (int)c->top_k : n;
    if (k == 0) return 0;
    int penalized = c->repetition_penalty != 1.0f || c->presence_penalty != 0.0f;
    float* buf = NULL;
    const float* src = logits;
    if (penalized) {
        buf = (float*)malloc(sizeof(float) * (size_t)n);
        memcpy(buf, logits, sizeof(float) * (size_t)n);
        apply_penalties(buf, n, c, past, npast);
        src = buf;
    }
    float t = c->temperature > 0.0f ? c->temperature : 1.0f;
    cand_t* cand = (cand_t*)malloc(sizeof(cand_t) * (size_t)(4 * k + 64));
    int nc = topk_serial(src, n, k, cand);
    int cnt = 0;
    if (nc > 0 && isfinite(cand[0].v)) {
        float lmax = cand[0].v;
        float sum_all = 0.0f; /* par_sum_exp serial arm, sampler.rs:626-656 */
        for (int i = 0; i < n; i++) sum_all += expf((src[i] - lmax) / t);
        float cum = 0.0f;
        int cut = 0;
        cand_t* out = (cand_t*)malloc(sizeof(cand_t) * (size_t)nc);
        for (int i = 0; i < nc && !cut; i++) {
            float e = expf((cand[i].v - lmax) / t);
            if (c->min_p > 0.0f && e < c->min_p) continue;
            float pr = e / sum_all;
            if (pr <= 0.0f) continue;
            out[cnt].id = cand[i].id;
            out[cnt].v = pr;
            cnt++;
            cum += pr;
            if (c->top_p < 1.0f && c->top_p > 0.0f && cum >= c->top_p) cut = 1;
        }
        float sum = 0.0f;
        for (int i = 0; i < cnt; i++) sum += out[i].v;
        if (sum > 0.0f) {
            for (int i = 0; i < cnt; i++) out[i].v /= sum;
            qsort(out, (size_t)cnt, sizeof(cand_t), cmp_id);
            for (int i = 0; i < cnt; i++) {
                ids[i] = out[i].id;
                probs[i] = out[i].v;
            }
        } else {
            cnt = 0;
        }
        free(out);
    }
    free(cand);
    free(buf);
    return cnt;
}

/* sampler.rs:661-671 */
uint32_t or_draw_sparse(const uint32_t* ids, const float* p, int n, or_rng* rng) {
    float r = or_rng_next_f32(rng), cum = 0.0f;
    for (int i = 0; i < n; i++) {
        cum += p[i];
        if (r < cum) return ids[i];
    }
    for (int i = n - 1; i >= 0; i--)
        if (p[i] > 0.0f) return ids[i];
    return 0;
}

static float sparse_get(const uint32_t* ids, const float* p, int n, uint32_t id) {
    int lo = 0, hi = n - 1;
    while (lo <= hi) {
        int mid = (lo + hi) / 2;
        if (ids[mid] == id) return p[mid];
        if (ids[mid] < id)
            lo = mid + 1;
        else
            hi = mid - 1;
    }
    return 0.0f;
}

/* sampler.rs:683-711 */
int64_t or_spec_accept_sparse(const uint32_t* pid, const float* pp, int np, const uint32_t* qid,
                              const float* qp, int nq, uint32_t d, or_rng* rng) {
    float pd = sparse_get(pid, pp, np, d), qd = sparse_get(qid, qp, nq, d);
    float r = or_rng_next_f32(rng);
    if (qd > 0.0f && r * qd < pd) return -1;
    uint32_t* rid = (uint32_t*)malloc(sizeof(uint32_t) * (size_t)(np ? np : 1));
    float* rp = (float*)malloc(sizeof(float) * (size_t)(np ? np : 1));
    int nr = 0;
    float total = 0.0f;
    for (int i = 0; i < np; i++) {
        float ri = pp[i] - sparse_get(qid, qp, nq, pid[i]);
        if (ri > 0.0f) {
            rid[nr] = pid[i];
            rp[nr] = ri;
            nr++;
            total += ri;
        }
    }
    int64_t res;
    if (total <= 0.0f) {
        res = or_draw_sparse(pid, pp, np, rng);
    } else {
        for (int i = 0; i < nr; i++) rp[i] /= total;
        res = or_draw_sparse(rid, rp, nr, rng);
    }
    free(rid);
    free(rp);
    return res;
}

/* sampler.rs:771-819 */
int64_t or_spec_accept_dense(const float* p, const float* q, int n, uint32_t d, or_rng* rng) {
    float pd = (int)d < n ? p[d] : 0.0f, qd = (int)d < n ? q[d] : 0.0f;
    float r = or_rng_next_f32(rng);
    if (qd > 0.0f && r * qd < pd) return -1;
    float* res = (float*)malloc(sizeof(float) * (size_t)n);
    for (int i = 0; i < n; i++) {
        float v = p[i] - q[i];
        res[i] = v > 0.0f ? v : 0.0f;
    }
    float sum = 0.0f;
    for (int i = 0; i < n; i++) sum += res[i];
    int64_t out;
    if (sum > 0.0f) {
        float inv = 1.0f / sum;
        for (int i = 0; i < n; i++) res[i] *= inv;
        out = or_categorical(res, n, or_rng_next_f32(rng));
    } else {
        out = or_categorical(p, n, or_rng_next_f32(rng));
    }
    free(res);
    return out;
}

/* sampler.rs:161-212 — greedy short-circuit, else the sparse chain (top_k in
 * 1..=256).  The dense chain (top_k == 0) is outside this build's configs. */
uint32_t or_sample(const float* logits, int n, const or_sampler_cfg* c, const uint32_t* past,
                   int npast, or_rng* rng) {
    if (c->temperature < 1e-6f && c->repetition_penalty == 1.0f && c->presence_penalty == 0.0f)
        return or_argmax(logits, n);
    if (c->temperature < 1e-6f) {
        float* buf = (float*)malloc(sizeof(float) * (size_t)n);
        memcpy(buf, logits, sizeof(float) * (size_t)n);
        apply_penalties(buf, n, c, past, npast);
        uint32_t t = or_argmax(buf, n);
        free(buf);
        return t;
    }
    uint32_t ids[4 * 256 + 64];
    float pr[4 * 256 + 64];
    int m = or_sparse_distribution(logits, n, c, past, npast, ids, pr);
    if (m > 0) return or_draw_sparse(ids, pr, m, rng);
    return or_argmax(logits, n);
}
