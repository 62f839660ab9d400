/*
 * Oracle (test infrastructure): the Qwen3-arch forward, the MTP head, the
 * speculative decode loop and MoE routing, restated from
 * cortiq-engine/src/{inference.rs, attention.rs, kv_cache.rs, pipeline.rs}.
 */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "oracle.h"

/* inference.rs:14-16 */
float or_silu(float x) { return x / (1.0f + expf(-x)); }

/* inference.rs:33-50 (Qwen style): mean-square in f64, inv cast to f32. */
void or_rms_norm(const float* x, const float* w, int n, double eps, float* out) {
    double ms = 0.0;
    for (int i = 0; i < n; i++) ms += (double)x[i] * (double)x[i];
    ms /= (double)n;
    float inv = 1.0f / (float)sqrt(ms + eps);
    for (int i = 0; i < n; i++) out[i] = x[i] * inv * w[i];
}

/* inference.rs:55-86: h += delta, then rms_norm(h) */
static void add_rms_norm(float* h, const float* d, const float* w, int n, double eps, float* out) {
    double ms = 0.0;
    for (int i = 0; i < n; i++) {
        float v = h[i] + d[i];
        h[i] = v;
        ms += (double)v * (double)v;
    }
    ms /= (double)n;
    float inv = 1.0f / (float)sqrt(ms + eps);
    for (int i = 0; i < n; i++) out[i] = h[i] * inv * w[i];
}

/* attention.rs:606-624: qk-norm, inv computed in f64 then cast. */
/* The model's quantized matmuls under the contract it runs: exact (the
 * default, CMF_SDOT=0) or a8w8 (split_act + integer dots, qtensor.rs:9237-9281,
 * the reference's default on hosts with integer dot instructions); f32
 * weights (a dense router) always take the exact path.  m->fast routes the
 * a8w8 matmuls through the AVX-512 VNNI timing arm (fast.c), which returns
 * the scalar arm's values bit for bit.  xs / out: [b][cols] / [b][rows]. */
static void mm(const or_model* m, const or_qt* w, const float* xs, int b, float* out) {
    if (m->a8w8 && w->dtype != OR_F32) {
        if (!(m->fast && or_fast_matmat_a8w8(w, xs, b, out, m->threads) == 0))
            or_matmat_a8w8(w, xs, b, out, m->threads);
    } else {
        or_matmat(w, xs, b, out, m->threads);
    }
}

static void mv(const or_model* m, const or_qt* w, const float* x, float* out) { mm(m, w, x, 1, out); }

static void rmsnorm_head(float* x, const float* w, int n, double eps) {
    double ss = 0.0;
    for (int i = 0; i < n; i++) ss += (double)x[i] * (double)x[i];
    float inv = (float)(1.0 / sqrt(ss / (double)n + eps));
    for (int i = 0; i < n; i++) x[i] = x[i] * inv * w[i];
}

/* attention.rs:27-31 */
void or_rope_inv_freq(int hd, float theta, float* out) {
    for (int i = 0; i < hd / 2; i++) out[i] = 1.0f / powf(theta, 2.0f * (float)i / (float)hd);
}

/* attention.rs:71-81 (scale 1) */
static void rope(float* x, int pos, const float* inv_freq, int half) {
    for (int i = 0; i < half; i++) {
        float ang = (float)pos * inv_freq[i];
        float s = sinf(ang), c = cosf(ang);
        float x0 = x[i], x1 = x[i + half];
        x[i] = x0 * c - x1 * s;
        x[i + half] = x0 * s + x1 * c;
    }
}

/* attention.rs:150-182 dot_f32_avx2.  The clones only let the compiler use
 * hardware fma and wider registers; the operations and their order are the
 * same in every clone (no contraction, no reassociation). */
CLONES static float dot_f32(const float* a, const float* b, int n) {
    float s0[8] = {0}, s1[8] = {0};
    int j = 0;
    for (; j + 16 <= n; j += 16)
        for (int l = 0; l < 8; l++) {
            s0[l] = fmaf(a[j + l], b[j + l], s0[l]);
            s1[l] = fmaf(a[j + 8 + l], b[j + 8 + l], s1[l]);
        }
    float acc[8], q[4];
    for (int l = 0; l < 8; l++) acc[l] = s0[l] + s1[l];
    for (int l = 0; l < 4; l++) q[l] = acc[l] + acc[4 + l];
    float sum = (q[0] + q[2]) + (q[1] + q[3]);
    for (; j < n; j++) sum += a[j] * b[j];
    return sum;
}

void or_embed(const or_model* m, uint32_t id, float* out) {
    /* pipeline.rs:5568-5575: row_f32 of the q8 embedding table (the tied
     * lm_head unless the model carries its own) */
    int H = m->cfg.hidden;
    const or_qt* e = m->embed.q ? &m->embed : &m->lm_head;
    if ((int)id >= e->rows) {
        memset(out, 0, sizeof(float) * (size_t)H);
        return;
    }
    const int8_t* q = e->q + (size_t)id * H;
    float rs = e->row_scale[id];
    for (int i = 0; i < H; i++) out[i] = (float)q[i] * rs;
}

/* finish_projection (attention.rs:818-890: qk-norm then RoPE), the KV
 * append (kv_cache.rs:366-411) and, when ao != NULL, attend_group
 * (kv_cache.rs:521-690) over the stored rows into ao [n_heads * head_dim].
 * q / k / v: this position's projections (q and k are changed in place).
 * Heads are independent, so they are spread over the model's threads. */
/* o[d] = fma(w, v[d], o[d]) (attend_group's value accumulation) */
CLONES static void axpy(float w, const float* v, float* o, int n) {
    for (int d = 0; d < n; d++) o[d] = fmaf(w, v[d], o[d]);
}

static void attend_row(const or_model* m, const or_layer* L, or_kv* kv, const float* inv_freq, float* q,
                       float* k, const float* v, int pos, float* ao) {
    const or_cfg* c = &m->cfg;
    int nh = c->n_heads, nkv = c->n_kv, hd = c->head_dim, S = c->max_seq;
    for (int h = 0; h < nh; h++) rmsnorm_head(q + h * hd, L->q_norm, hd, c->eps);
    for (int g = 0; g < nkv; g++) rmsnorm_head(k + g * hd, L->k_norm, hd, c->eps);
    for (int h = 0; h < nh; h++) rope(q + h * hd, pos, inv_freq, hd / 2);
    for (int g = 0; g < nkv; g++) rope(k + g * hd, pos, inv_freq, hd / 2);
    int p0 = kv->len;
    for (int g = 0; g < nkv; g++) {
        memcpy(kv->k + ((size_t)g * S + p0) * hd, k + g * hd, sizeof(float) * (size_t)hd);
        memcpy(kv->v + ((size_t)g * S + p0) * hd, v + g * hd, sizeof(float) * (size_t)hd);
    }
    kv->len = p0 + 1;
    if (!ao) return;
    int stored = kv->len, hpk = nh / nkv;
    float scale = 1.0f / sqrtf((float)hd);
    memset(ao, 0, sizeof(float) * (size_t)(nh * hd));
    int nt = m->threads > 1 ? (m->threads < nh ? m->threads : nh) : 1;
#pragma omp parallel num_threads(nt)
    {
        float* sc = (float*)malloc(sizeof(float) * (size_t)stored);
#pragma omp for schedule(static)
        for (int h = 0; h < nh; h++) {
            int g = h / hpk;
            const float* K = kv->k + (size_t)g * S * hd;
            const float* V = kv->v + (size_t)g * S * hd;
            for (int p = 0; p < stored; p++) sc[p] = dot_f32(q + h * hd, K + (size_t)p * hd, hd) * scale;
            float mx = -INFINITY, sum = 0.0f;
            for (int p = 0; p < stored; p++) mx = fmaxf(mx, sc[p]);
            for (int p = 0; p < stored; p++) {
                sc[p] = expf(sc[p] - mx);
                sum += sc[p];
            }
            if (sum > 0.0f)
                for (int p = 0; p < stored; p++) sc[p] /= sum;
            float* o = ao + h * hd;
            for (int p = 0; p < stored; p++) {
                float w = sc[p];
                if (fabsf(w) < 1e-12f) continue;
                const float* vr = V + (size_t)p * hd;
                axpy(w, vr, o, hd);
            }
        }
        free(sc);
    }
}

/* qwen_attention (attention.rs:1005-1027) for b consecutive positions
 * pos0 .. pos0+b-1 over one KV: the projections of all rows at once (the
 * verify batch's matmat, pipeline.rs:4275-4505), then each row in order
 * appends its K/V and attends over the rows stored so far, then the output
 * projection of all rows.  x / out: [b][hidden]; out == NULL: append only. */
static void attention_rows(const or_model* m, const or_layer* L, or_kv* kv, const float* inv_freq,
                           const float* x, int b, int pos0, float* out) {
    const or_cfg* c = &m->cfg;
    int qd = c->n_heads * c->head_dim, kd = c->n_kv * c->head_dim;
    float* q = (float*)malloc(sizeof(float) * (size_t)b * qd);
    float* k = (float*)malloc(sizeof(float) * (size_t)b * kd);
    float* v = (float*)malloc(sizeof(float) * (size_t)b * kd);
    float* ao = out ? (float*)malloc(sizeof(float) * (size_t)b * qd) : NULL;
    mm(m, &L->wq, x, b, q);
    mm(m, &L->wk, x, b, k);
    mm(m, &L->wv, x, b, v);
    for (int i = 0; i < b; i++)
        attend_row(m, L, kv, inv_freq, q + (size_t)i * qd, k + (size_t)i * kd, v + (size_t)i * kd, pos0 + i,
                   ao ? ao + (size_t)i * qd : NULL);
    if (out) mm(m, &L->wo, ao, b, out);
    free(ao);
    free(q);
    free(k);
    free(v);
}

static void attention(const or_model* m, const or_layer* L, or_kv* kv, const float* inv_freq,
                      const float* x, int pos, float* out, int compute_out) {
    attention_rows(m, L, kv, inv_freq, x, 1, pos, compute_out ? out : NULL);
}

/* dense_ffn_cpu (pipeline.rs:9570-9661), exact arm: silu(g)*u then down,
 * for b rows at once (x / out: [b][hidden]) */
static void ffn_rows(const or_model* m, const or_layer* L, const float* x, int b, float* out) {
    size_t n = (size_t)b * L->gate.rows;
    float* g = (float*)malloc(sizeof(float) * n);
    float* u = (float*)malloc(sizeof(float) * n);
    mm(m, &L->gate, x, b, g);
    mm(m, &L->up, x, b, u);
    for (size_t i = 0; i < n; i++) g[i] = or_silu(g[i]) * u[i];
    mm(m, &L->down, g, b, out);
    free(g);
    free(u);
}

/* one transformer block over b consecutive positions (h: [b][hidden]):
 * h += attn(norm(h)); h += ffn(norm(h)) */
static void block_rows(const or_model* m, const or_layer* L, or_kv* kv, const float* inv_freq, float* h, int b,
                       int pos0) {
    int H = m->cfg.hidden;
    size_t n = (size_t)b * H;
    float* n1 = (float*)calloc(n, sizeof(float));
    float* a = (float*)malloc(sizeof(float) * n);
    float* f = (float*)malloc(sizeof(float) * n);
    for (int i = 0; i < b; i++) or_rms_norm(h + (size_t)i * H, L->input_norm, H, m->cfg.eps, n1 + (size_t)i * H);
    attention_rows(m, L, kv, inv_freq, n1, b, pos0, a);
    for (int i = 0; i < b; i++)
        add_rms_norm(h + (size_t)i * H, a + (size_t)i * H, L->post_norm, H, m->cfg.eps, n1 + (size_t)i * H);
    if (L->n_experts > 0) {
        /* moe_ffn_forward (pipeline.rs:10868-11045): router logits of the
         * normed row, routing, the routed experts' weighted sum */
        float* lg = (float*)malloc(sizeof(float) * (size_t)L->n_experts);
        for (int i = 0; i < b; i++) {
            or_matvec(&L->router, n1 + (size_t)i * H, lg, m->threads);
            or_moe_ffn(L->experts, L->n_experts, L->top_k, L->norm_topk, L->routed_scaling, lg, n1 + (size_t)i * H,
                       H, f + (size_t)i * H, m->threads);
        }
        free(lg);
    } else {
        ffn_rows(m, L, n1, b, f);
    }
    for (size_t i = 0; i < n; i++) h[i] += f[i];
    free(n1);
    free(a);
    free(f);
}

static void block(const or_model* m, const or_layer* L, or_kv* kv, const float* inv_freq, float* h, int pos) {
    block_rows(m, L, kv, inv_freq, h, 1, pos);
}

/* forward_layers_span (pipeline.rs:7981-8700) */
void or_forward(const or_model* m, or_state* s, float* h, int pos) {
    for (int li = 0; li < m->cfg.n_layers; li++) block(m, &m->layers[li], &s->trunk[li], s->inv_freq, h, pos);
}

/* forward_batch over b consecutive positions (pipeline.rs:4275-4505, the
 * verify rows as one batch): every layer's matmuls take all rows at once,
 * attention runs row by row in position order.  Under the exact contract the
 * rows equal b per-position forwards bit for bit; under a8w8 the q4t
 * matmuls take the four-input blocked order for rows 0..3 (qtensor.rs:
 * 5908-5928). */
void or_forward_rows(const or_model* m, or_state* s, float* h, int b, int pos0) {
    for (int li = 0; li < m->cfg.n_layers; li++)
        block_rows(m, &m->layers[li], &s->trunk[li], s->inv_freq, h, b, pos0);
}

void or_logits(const or_model* m, const float* h, float* logits) {
    int H = m->cfg.hidden;
    float* n = (float*)malloc(sizeof(float) * (size_t)H);
    or_rms_norm(h, m->final_norm, H, m->cfg.eps, n);
    mv(m, &m->lm_head, n, logits);
    free(n);
}

/* mtp_step_hl (pipeline.rs:3051-3160); logits == NULL is mtp_warm
 * (pipeline.rs:3532-3572: only the attention's KV append matters). */
void or_mtp_step(const or_model* m, or_state* s, const float* hidden, uint32_t tok, int pos,
                 float* logits, float* h_out) {
    int H = m->cfg.hidden;
    float* e = (float*)malloc(sizeof(float) * (size_t)H);
    float* cat = (float*)malloc(sizeof(float) * (size_t)(2 * H));
    float* x = (float*)malloc(sizeof(float) * (size_t)H);
    or_embed(m, tok, e);
    or_rms_norm(e, m->enorm, H, m->cfg.eps, cat);      /* embedding FIRST */
    or_rms_norm(hidden, m->hnorm, H, m->cfg.eps, cat + H);
    mv(m, &m->eh_proj, cat, x);
    if (logits == NULL) {
        float* n1 = (float*)malloc(sizeof(float) * (size_t)H);
        or_rms_norm(x, m->mtp.input_norm, H, m->cfg.eps, n1);
        attention(m, &m->mtp, &s->mtp, s->inv_freq, n1, pos, NULL, 0);
        free(n1);
    } else {
        block(m, &m->mtp, &s->mtp, s->inv_freq, x, pos);
        float* n = (float*)malloc(sizeof(float) * (size_t)H);
        or_rms_norm(x, m->mtp_norm, H, m->cfg.eps, n);
        mv(m, &m->lm_head, n, logits);
        free(n);
    }
    if (h_out) memcpy(h_out, x, sizeof(float) * (size_t)H);
    free(e);
    free(cat);
    free(x);
}

/* ---------------------------------------------------------------------------
 * The decode loop with graph_spec_step (pipeline.rs:2546-2980, 3582-4213).
 * The verify rows are per-position forwards, or one batch (or_forward_rows)
 * when the model asks for it; the trunk KV rows past
 * the accepted prefix are dropped (truncate_last, kv_cache.rs:883).  The
 * reference's timing-based speculation monitor (SpecMon, pipeline.rs:662)
 * is not restated: speculation is on for every round.
 * ------------------------------------------------------------------------- */

typedef struct {
    uint32_t ids[1088];
    float p[1088];
    int n;
} sparse_t;

static int is_sampling(const or_sampler_cfg* c) { return c->temperature >= 1e-6f; }

/* the draft/verify token choice for one row: greedy argmax or a draw from
 * the sparse distribution (pipeline.rs:3709-3757) */
static uint32_t choose(const float* lg, int V, const or_sampler_cfg* c, const uint32_t* past,
                       int npast, or_rng* rng, sparse_t* q) {
    if (!is_sampling(c)) return or_argmax(lg, V);
    q->n = or_sparse_distribution(lg, V, c, past, npast, q->ids, q->p);
    if (q->n > 0) return or_draw_sparse(q->ids, q->p, q->n, rng);
    uint32_t t = or_argmax(lg, V);
    q->ids[0] = t;
    q->p[0] = 1.0f;
    q->n = 1;
    return t;
}

static void truncate_kv(or_kv* kv, int n) { kv->len -= n < kv->len ? n : kv->len; }

/* The verify half of graph_spec_step (pipeline.rs:3768-4176) given the
 * drafts: the b = K + 1 rows [t_next, d_0 .. d_{K-1}] at next_pos .. as
 * ordinary per-position forwards (vlog / hid: [b][V] / [b][H]), acceptance
 * (pipeline.rs:3887-4001), the trunk rows past the accepted prefix dropped
 * (truncate_last, kv_cache.rs:883) and the accepted pairs warmed into the
 * MTP cache (pipeline.rs:4120-4176).  qs: the draft distributions
 * (sampling only); all/nall: the committed stream the sampler reads.
 * Returns a; *forced = the correction token or -1. */
static int verify_core(const or_model* m, or_state* s, int next_pos, uint32_t t_next, const uint32_t* drafts,
                       int K, const or_sampler_cfg* sc, const sparse_t* qs, or_rng* rng, uint32_t* all,
                       int nall, float* vlog, float* hid, int* forced) {
    const or_cfg* c = &m->cfg;
    int H = c->hidden, V = c->vocab, b = K + 1;
    sparse_t* ps = (sparse_t*)malloc(sizeof(sparse_t));
    if (m->batch_verify) {
        for (int i = 0; i < b; i++) or_embed(m, i == 0 ? t_next : drafts[i - 1], hid + (size_t)i * H);
        or_forward_rows(m, s, hid, b, next_pos);
        float* n = (float*)malloc(sizeof(float) * (size_t)b * H);
        for (int i = 0; i < b; i++) or_rms_norm(hid + (size_t)i * H, m->final_norm, H, c->eps, n + (size_t)i * H);
        mm(m, &m->lm_head, n, b, vlog);
        free(n);
    } else {
        for (int i = 0; i < b; i++) {
            uint32_t t = i == 0 ? t_next : drafts[i - 1];
            float* h = hid + (size_t)i * H;
            or_embed(m, t, h);
            or_forward(m, s, h, next_pos + i);
            or_logits(m, h, vlog + (size_t)i * V);
        }
    }
    int a = 0;
    *forced = -1;
    if (is_sampling(sc)) {
        int base = nall;
        while (a < K) {
            const float* row = vlog + (size_t)a * V;
            ps->n = or_sparse_distribution(row, V, sc, all, nall, ps->ids, ps->p);
            if (ps->n == 0) {
                ps->ids[0] = or_argmax(row, V);
                ps->p[0] = 1.0f;
                ps->n = 1;
            }
            int64_t r = or_spec_accept_sparse(ps->ids, ps->p, ps->n, qs[a].ids, qs[a].p, qs[a].n, drafts[a], rng);
            if (r < 0) {
                all[nall++] = drafts[a];
                a++;
            } else {
                *forced = (int)r;
                break;
            }
        }
        nall = base;
    } else {
        while (a < K && or_argmax(vlog + (size_t)a * V, V) == drafts[a]) a++;
    }
    for (int li = 0; li < c->n_layers; li++) truncate_kv(&s->trunk[li], K - a);
    if (m->has_mtp)
        for (int j = 0; j < a; j++) or_mtp_step(m, s, hid + (size_t)j * H, drafts[j], next_pos + j, NULL, NULL);
    free(ps);
    return a;
}

int or_decode(const or_model* m, or_state* s, float* hidden, int next_pos, const uint32_t* ids0,
              int nids, int max_tokens, const or_gen_cfg* g, uint64_t* rng_state, uint32_t* out,
              or_gen_stats* st) {
    const or_cfg* c = &m->cfg;
    int H = c->hidden, V = c->vocab, K = g->k;
    or_rng rng = {*rng_state};
    uint32_t* all = (uint32_t*)malloc(sizeof(uint32_t) * (size_t)(nids + max_tokens + K + 8));
    memcpy(all, ids0, sizeof(uint32_t) * (size_t)nids);
    int nall = nids, generated = 0;
    float* logits = (float*)malloc(sizeof(float) * (size_t)V);
    float* vlog = (float*)malloc(sizeof(float) * (size_t)V * (size_t)(K + 1));
    float* hid = (float*)malloc(sizeof(float) * (size_t)H * (size_t)(K + 1));
    float* hx = (float*)malloc(sizeof(float) * (size_t)H);
    float* hj = (float*)malloc(sizeof(float) * (size_t)H);
    sparse_t* qs = (sparse_t*)malloc(sizeof(sparse_t) * (size_t)(K > 0 ? K : 1));
    int have_logits = 0, forced = -1;
    memset(st, 0, sizeof(*st));
    while (generated < max_tokens) {
        uint32_t t_next;
        if (forced >= 0) {
            t_next = (uint32_t)forced;
            forced = -1;
        } else {
            if (!have_logits) or_logits(m, hidden, logits);
            have_logits = 0;
            t_next = or_sample(logits, V, &g->sc, all, nall, &rng);
        }
        all[nall++] = t_next;
        out[generated++] = t_next;
        if (generated >= max_tokens) break;
        if (g->spec && m->has_mtp && generated + 1 < max_tokens && next_pos > 0) {
            /* ---- graph_spec_step: the draft chain ---- */
            st->rounds++;
            uint32_t drafts[16];
            int base = nall;
            memcpy(hx, hidden, sizeof(float) * (size_t)H);
            for (int j = 0; j < K; j++) {
                uint32_t tin = j == 0 ? t_next : drafts[j - 1];
                or_mtp_step(m, s, hx, tin, next_pos - 1 + j, logits, hj);
                uint32_t d = choose(logits, V, &g->sc, all, nall, &rng, &qs[j]);
                if (is_sampling(&g->sc)) all[nall++] = d;
                drafts[j] = d;
                memcpy(hx, hj, sizeof(float) * (size_t)H);
            }
            nall = base;
            st->drafted += K;
            /* MTP cache: keep the first draft row (its inputs were real) */
            truncate_kv(&s->mtp, K - 1);
            int a = verify_core(m, s, next_pos, t_next, drafts, K, &g->sc, qs, &rng, all, nall, vlog, hid, &forced);
            st->accepted += a;
            st->hist[a]++;
            if (forced < 0) {
                memcpy(logits, vlog + (size_t)a * V, sizeof(float) * (size_t)V);
                have_logits = 1;
            }
            memcpy(hidden, hid + (size_t)a * H, sizeof(float) * (size_t)H);
            next_pos += a + 1;
            for (int j = 0; j < a; j++) {
                all[nall++] = drafts[j];
                out[generated++] = drafts[j];
            }
            continue;
        }
        /* vanilla: forward the sampled token */
        or_embed(m, t_next, hidden);
        or_forward(m, s, hidden, next_pos);
        next_pos++;
    }
    *rng_state = rng.state;
    free(all);
    free(logits);
    free(vlog);
    free(hid);
    free(hx);
    free(hj);
    free(qs);
    return generated;
}

int or_verify_step(const or_model* m, or_state* s, float* hidden, int pos0, const uint32_t* tokens, int b,
                   const or_sampler_cfg* sc, const uint32_t* q_ids, const float* q_p, const int* q_n,
                   int q_stride, or_rng* rng, const uint32_t* past, int npast, int warm_tip, float* logits,
                   uint32_t* argmax, uint32_t* next) {
    const or_cfg* c = &m->cfg;
    int H = c->hidden, V = c->vocab, K = b - 1;
    float* vlog = (float*)malloc(sizeof(float) * (size_t)V * (size_t)b);
    float* hid = (float*)malloc(sizeof(float) * (size_t)H * (size_t)b);
    sparse_t* qs = (sparse_t*)calloc((size_t)(K > 0 ? K : 1), sizeof(sparse_t));
    uint32_t* all = (uint32_t*)malloc(sizeof(uint32_t) * (size_t)(npast + b + 1));
    if (npast > 0) memcpy(all, past, sizeof(uint32_t) * (size_t)npast);
    if (is_sampling(sc))
        for (int j = 0; j < K; j++) {
            qs[j].n = q_n[j];
            for (int i = 0; i < q_n[j]; i++) {
                qs[j].ids[i] = q_ids[(size_t)j * q_stride + i];
                qs[j].p[i] = q_p[(size_t)j * q_stride + i];
            }
        }
    /* the MTP row of the first draft: (tip hidden, t_next) at pos0 - 1 */
    if (warm_tip && m->has_mtp && pos0 > 0) or_mtp_step(m, s, hidden, tokens[0], pos0 - 1, NULL, NULL);
    int forced = -1;
    int a = verify_core(m, s, pos0, tokens[0], tokens + 1, K, sc, qs, rng, all, npast, vlog, hid, &forced);
    if (argmax)
        for (int i = 0; i < b; i++) argmax[i] = or_argmax(vlog + (size_t)i * V, V);
    if (logits) memcpy(logits, vlog, sizeof(float) * (size_t)V * (size_t)b);
    if (forced >= 0) {
        *next = (uint32_t)forced;
    } else {
        /* the loop top picks from row a over the stream with the accepted drafts */
        int n = npast;
        for (int j = 0; j < a; j++) all[n++] = tokens[1 + j];
        *next = or_sample(vlog + (size_t)a * V, V, sc, all, n, rng);
    }
    memcpy(hidden, hid + (size_t)a * H, sizeof(float) * (size_t)H);
    free(vlog);
    free(hid);
    free(qs);
    free(all);
    return a;
}

int or_generate(const or_model* m, or_state* s, const uint32_t* prompt, int np, int max_tokens,
                const or_gen_cfg* g, uint32_t* out, or_gen_stats* st) {
    int H = m->cfg.hidden;
    float* h = (float*)malloc(sizeof(float) * (size_t)H);
    float* last = (float*)malloc(sizeof(float) * (size_t)H);
    /* prefill per position; the MTP head is warmed on (h_p, id_{p+1})
     * pairs (pipeline.rs:2275-2318) */
    for (int p = 0; p < np; p++) {
        or_embed(m, prompt[p], h);
        or_forward(m, s, h, p);
        if (m->has_mtp && p + 1 < np) or_mtp_step(m, s, h, prompt[p + 1], p, NULL, NULL);
        memcpy(last, h, sizeof(float) * (size_t)H);
    }
    uint64_t rs = g->seed;
    int n = or_decode(m, s, last, np, prompt, np, max_tokens, g, &rs, out, st);
    free(h);
    free(last);
    return n;
}

/* ---------------------------------------------------------------------------
 * MoE (pipeline.rs:10780-10841 moe_route; 11017-11045 moe_ffn_cpu)
 * ------------------------------------------------------------------------- */
int or_moe_route(const float* lg, int ne, int top_k, int norm_topk, float routed_scaling,
                 int* idx, float* w) {
    float* p = (float*)malloc(sizeof(float) * (size_t)ne);
    float mx = -INFINITY, s = 0.0f;
    for (int e = 0; e < ne; e++) mx = fmaxf(mx, lg[e]);
    for (int e = 0; e < ne; e++) p[e] = expf(lg[e] - mx);
    for (int e = 0; e < ne; e++) s += p[e];
    for (int e = 0; e < ne; e++) p[e] /= s;
    /* descending by probability, lower index wins ties */
    int* ord = (int*)malloc(sizeof(int) * (size_t)ne);
    for (int e = 0; e < ne; e++) ord[e] = e;
    for (int i = 1; i < ne; i++) {
        int v = ord[i], j = i - 1;
        while (j >= 0 && (p[ord[j]] < p[v] || (p[ord[j]] == p[v] && ord[j] > v))) {
            ord[j + 1] = ord[j];
            j--;
        }
        ord[j + 1] = v;
    }
    int k = top_k < ne ? top_k : ne;
    float wsum;
    if (norm_topk) {
        float t = 0.0f;
        for (int i = 0; i < k; i++) t += p[ord[i]];
        wsum = t / routed_scaling;
    } else {
        wsum = 1.0f / routed_scaling;
    }
    for (int i = 0; i < k; i++) {
        idx[i] = ord[i];
        w[i] = p[ord[i]] / wsum;
    }
    free(p);
    free(ord);
    return k;
}

/* moe_ffn_cpu's serial expert loop (pipeline.rs:11017-11030): out starts at
 * 0, each routed expert in routing order adds w * dense_ffn(expert, x). */
void or_moe_ffn(const or_qt* ex, int ne, int top_k, int norm_topk, float routed_scaling, const float* rl,
                const float* x, int hidden, float* out, int threads) {
    int idx[256];
    float w[256];
    int k = or_moe_route(rl, ne, top_k, norm_topk, routed_scaling, idx, w);
    int I = ex[0].rows;
    float* g = (float*)malloc(sizeof(float) * (size_t)I);
    float* u = (float*)malloc(sizeof(float) * (size_t)I);
    float* d = (float*)malloc(sizeof(float) * (size_t)hidden);
    memset(out, 0, sizeof(float) * (size_t)hidden);
    for (int i = 0; i < k; i++) {
        const or_qt* e = ex + 3 * idx[i];
        or_matvec(&e[0], x, g, threads);
        or_matvec(&e[1], x, u, threads);
        for (int j = 0; j < I; j++) g[j] = or_silu(g[j]) * u[j];
        or_matvec(&e[2], g, d, threads);
        for (int j = 0; j < hidden; j++) out[j] += w[i] * d[j];
    }
    free(g);
    free(u);
    free(d);
}
