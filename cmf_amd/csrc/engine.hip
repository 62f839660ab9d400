// The decode engine: a Qwen3-arch decoder with an MTP head resident on one
// MI355X, the batched verify forward (the counterpart of the reference's
// forward_batch_graph, gpu.rs:1466-1497) and the speculative decode loop
// (graph_spec_step, pipeline.rs:3582-4213) run device-side: drafted tokens,
// acceptance and the commit never leave HBM; the host reads back one small
// state record per round.
#include <chrono>
#include <climits>
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <cmath>

#include <string>
#include <vector>

#include "../../include/cmf_hip.h"
#include "common.h"
#include "gemv.h"
#include "layers.h"
#include "runtime.h"
#include "sample.h"
#include "wave.h"
#include "xlayer.h"

namespace cmf {

struct LayerDev {
    float *in_norm = nullptr, *post_norm = nullptr, *q_norm = nullptr, *k_norm = nullptr;
    float qk_norm_max = 0.f;  // max |q_norm|, |k_norm| (bounds the normed q / k rows)
    DevWeight qkv, wo, gu, down;
    float *kc = nullptr, *vc = nullptr;
    // routed-expert FFN (GraphFfn::Moe, gpu.rs:1248-1361): the router and the
    // caller's MoE layer (borrowed) instead of gu / down
    cmf_moe_s* moe = nullptr;
    DevWeight router;
    float* router_f32 = nullptr;  // a dense (f32 / f16 / bf16 in the file) router [ne][hidden] as f32
    int n_experts = 0;
};

// rms_norm of nb rows (inference.rs:33-50: f64 mean of squares, the inverse
// cast to f32, x * inv * w), one workgroup per row.
__global__ __launch_bounds__(256) void k_rms_rows(const float* __restrict__ x, int ldx, const float* __restrict__ w,
                                                  int H, double eps, float* __restrict__ out) {
    __shared__ double red[4];
    const int b = blockIdx.x, t = threadIdx.x;
    const float* row = x + (size_t)b * ldx;
    double ss = 0.0;
    for (int i = t; i < H; i += 256) ss += (double)row[i] * (double)row[i];
    ss = wave_sum(ss);
    if ((t & 63) == 0) red[t >> 6] = ss;
    __syncthreads();
    const double tot = red[0] + red[1] + red[2] + red[3];
    const float inv = 1.0f / (float)sqrt(tot / (double)H + eps);
    for (int i = t; i < H; i += 256) out[(size_t)b * H + i] = row[i] * inv * w[i];
}

// Router logits of a dense f32 router (QTensor::F32 matvec, pool.rs:535-548):
// logits[b][e] = sum_k W[e][k] x[b][k], one wave per expert row, the rows of
// x from L2.
__global__ __launch_bounds__(256) void k_router_f32(const float* __restrict__ W, const float* __restrict__ x,
                                                    int ne, int H, int nb, float* __restrict__ out) {
    const int e = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (e >= ne) return;  // uniform over the wave
    const float* wr = W + (size_t)e * H;
    for (int b = 0; b < nb; b++) {
        const float* xr = x + (size_t)b * H;
        float acc = 0.f;
        for (int k = lane; k < H; k += 64) acc += wr[k] * xr[k];
        acc = wave_sum(acc);
        if (lane == 0) out[(size_t)b * ne + e] = acc;
    }
}

}  // namespace cmf

using namespace cmf;

struct cmf_model_s {
    cmf_model_config c{};
    std::vector<LayerDev> L;
    bool has_head = false, has_mtp = false;
    DevWeight lm;
    DevWeight emb;  // untied embedding table (q8); empty: lm doubles as the table
    float* final_norm = nullptr;
    float *enorm = nullptr, *hnorm = nullptr, *mtp_norm = nullptr;
    DevWeight eh;
    LayerDev mtp;
    float2* rope = nullptr;
    // scratch
    float *hv = nullptr, *hm = nullptr, *attn_out = nullptr, *ffn_out = nullptr, *qkv_out = nullptr,
          *qrot = nullptr, *ao = nullptr, *xrows = nullptr, *hm2 = nullptr, *gu_out = nullptr, *logits = nullptr;
    float *pm = nullptr, *pl = nullptr, *po = nullptr;
    int nch_cap = 0;
    float* am_v = nullptr;
    int* am_i = nullptr;
    int* toks = nullptr;  // [2*MAXB] token staging
    DState* st = nullptr;
    int* out = nullptr;
    int out_cap = 0;
    float* h_tip = nullptr;
    uint8_t* plw = nullptr;  // the output projections' q8 operand, written by the attention merge
    float* plw_cs = nullptr;
    float* rlog = nullptr;  // router logits [MAXB][rlog_cap]
    int rlog_cap = 0;
    uint8_t* planes = nullptr;  // prepared GEMV operand (largest prep_bytes of the model)
    float* xs = nullptr;        // its per-row scales [16]
    SampleBufs sb;
    std::vector<void*> allocs;
    int next_pos_host = 0;
    bool prefilled = false;
    // prefill chunk buffers [prefill_chunk() rows] (allocated by the first prefill)
    float *pf_h = nullptr, *pf_qkv = nullptr, *pf_ao = nullptr, *pf_gu = nullptr, *pf_hm = nullptr, *pf_q = nullptr;
    int* pf_toks = nullptr;
    _Float16* pf_khl = nullptr;  // the prefill attention's K / V operands (f16 hi / lo keys, then f32 values)
    unsigned long long* pf_cells = nullptr;  // placement check of the XCD prefill attention
    int* pf_err = nullptr;
    unsigned long long pf_tag = 0;
    bool pf_xcd_off = false;  // a placement check failed: the grid-indexed variant from then on
    hipGraphExec_t round_graph = nullptr;
    int graph_k = 0;
    int graph_len = 0;  // attention length bound the captured round was built for
    int graph_sampling = -1;
    hipGraphExec_t plain_graph = nullptr;  // one captured plain step
    int plain_len = 0;
    int plain_sampling = -1;
    cmf_spec_state mon{};  // the speculation monitor of the last cmf_decode (spec = 2)
    bool use_graph = true;
    bool decoding = false;
    int rounds = 0;
    int emitted_host = 0;
    int accepted_host = 0;
    cmf_sampler_config sc{};
    // XCD-partitioned blocks (xlayer.hip): buffers allocated at create when
    // the shape and the device take them
    XlBufs xl;
    XlShape xls{};
    bool xl_on = false;
    int xl_fallbacks = 0;   // calls re-run on the six-launch blocks after a failed check
    float* h_save = nullptr;  // the tip hidden before such a call
};

namespace {

int dalloc(cmf_model_s* m, void** p, size_t bytes) {
    CMF_HIP(hipMalloc(p, bytes));
    CMF_HIP(hipMemset(*p, 0, bytes));
    m->allocs.push_back(*p);
    return CMF_OK;
}

template <class T>
int dalloc_t(cmf_model_s* m, T** p, size_t n) {
    return dalloc(m, (void**)p, n * sizeof(T));
}

void* xl_dalloc(void* ctx, size_t n) {
    void* p = nullptr;
    return dalloc((cmf_model_s*)ctx, &p, n) == CMF_OK ? p : nullptr;
}

int upload_f32(cmf_model_s* m, float** d, const float* h, size_t n) {
    if (!h) return fail("missing norm weights");
    if (dalloc_t(m, d, n) != CMF_OK) return CMF_ERR;
    CMF_HIP(hipMemcpy(*d, h, n * sizeof(float), hipMemcpyHostToDevice));
    return CMF_OK;
}

int check_tensor(const cmf_tensor& t, int rows, int cols, const char* name) {
    if (t.rows != rows || t.cols != cols)
        return fail(std::string(name) + ": shape mismatch (got " + std::to_string(t.rows) + "x" +
                    std::to_string(t.cols) + ", want " + std::to_string(rows) + "x" + std::to_string(cols) + ")");
    if (t.dtype == DT_Q8ROW) {
        if (!t.q || !t.row_scale) return fail(std::string(name) + ": q8 needs q and row_scale");
    } else if (t.dtype == DT_Q4T || t.dtype == DT_Q4TP) {
        if (!t.bytes) return fail(std::string(name) + ": q4 needs bytes");
        if (cols % 32) return fail(std::string(name) + ": q4 needs cols % 32 == 0");
    } else {
        return fail(std::string(name) + ": unsupported dtype");
    }
    return CMF_OK;
}

// Concatenate tensors along rows into one device weight (one launch serves
// q/k/v, or gate/up).
int build_cat(DevWeight& w, const std::vector<const cmf_tensor*>& ts) {
    const int dt = ts[0]->dtype, cols = ts[0]->cols;
    for (auto* t : ts)
        if (t->dtype != dt || t->cols != cols) return fail("fused tensors must share dtype and cols");
    if (dt == DT_Q8ROW) {
        std::vector<const int8_t*> rp;
        std::vector<float> rs;
        for (auto* t : ts)
            for (int r = 0; r < t->rows; r++) {
                rp.push_back(t->q + (size_t)r * cols);
                rs.push_back(t->row_scale[r]);
            }
        return build_q8(w, (int)rp.size(), cols, rp.data(), rs.data());
    }
    Q4Src s;
    for (auto* t : ts) fill_q4src(s, dt, t->rows, cols, t->bytes, 0);
    return build_q4(w, s);
}

int upload_layer(cmf_model_s* m, LayerDev& l, const cmf_layer_desc* d, bool kv) {
    const auto& c = m->c;
    const int H = c.hidden, hd = c.head_dim, Q = c.n_heads * hd, KV = c.n_kv * hd, I = c.inter;
    if (check_tensor(d->wq, Q, H, "wq") || check_tensor(d->wk, KV, H, "wk") ||
        check_tensor(d->wv, KV, H, "wv") || check_tensor(d->wo, H, Q, "wo") ||
        check_tensor(d->gate, I, H, "gate") || check_tensor(d->up, I, H, "up") ||
        check_tensor(d->down, H, I, "down"))
        return CMF_ERR;
    if (upload_f32(m, &l.in_norm, d->input_norm, H) || upload_f32(m, &l.post_norm, d->post_norm, H) ||
        upload_f32(m, &l.q_norm, d->q_norm, hd) || upload_f32(m, &l.k_norm, d->k_norm, hd))
        return CMF_ERR;
    l.qk_norm_max = 0.f;
    for (int i = 0; i < hd; i++)
        l.qk_norm_max = std::max(l.qk_norm_max, std::max(std::fabs(d->q_norm[i]), std::fabs(d->k_norm[i])));
    free_weight(l.qkv);
    free_weight(l.wo);
    free_weight(l.gu);
    free_weight(l.down);
    if (build_cat(l.qkv, {&d->wq, &d->wk, &d->wv}) || build_cat(l.wo, {&d->wo}) ||
        build_swiglu(l.gu, &d->gate, &d->up) || build_cat(l.down, {&d->down}))
        return CMF_ERR;
    if (kv && !l.kc) {
        const size_t n = (size_t)c.n_kv * c.max_seq * hd;
        if (dalloc_t(m, &l.kc, n) || dalloc_t(m, &l.vc, n)) return CMF_ERR;
    }
    return CMF_OK;
}

void free_layer(LayerDev& l) {
    free_weight(l.qkv);
    free_weight(l.wo);
    free_weight(l.gu);
    free_weight(l.down);
}

EmbedSrc embed_src(cmf_model_s* m) {
    const DevWeight& e = m->emb.w ? m->emb : m->lm;
    return EmbedSrc{(const int8_t*)e.w, (const float*)e.scale, e.rows, e.kchunks};
}

XSrc src_norm(const float* x, int ldx, const float* w, double eps) {
    XSrc r{};
    r.mode = XS_NORM;
    r.x = x;
    r.ldx = ldx;
    r.w = w;
    r.eps = eps;
    return r;
}

// W x with the operand of src: norm and plain rows are evaluated by every
// GEMV workgroup from raw rows loaded ahead of its weights (no producer
// launch); other producers (concat, larger operands) run as a
// one-workgroup-per-row kernel that writes the prepared planes, which the
// GEMV copies to LDS (or reads in place when they do not fit).
// Whether a batch of mb rows of src is prepared inside the GEMV workgroups
// (gemv_fuse_pays; CMF_GEMV_FUSED=n instead fuses every batch of at most n
// rows, 0: never).
static bool fuse_ok(const DevWeight& w, const XSrc& src, int mb) {
    static const int fuse_env = getenv("CMF_GEMV_FUSED") ? atoi(getenv("CMF_GEMV_FUSED")) : -1;
    if (fused_lds_bytes(w, src, mb) == 0) return false;
    return fuse_env >= 0 ? mb <= fuse_env : gemv_fuse_pays(w, mb);
}

int gemv_f(cmf_model_s* m, const DevWeight& w, XSrc src, float* y, int ldy, int nb, bool resid,
           hipStream_t s, int epi = EPI_NONE) {
    for (int b0 = 0; b0 < nb; b0 += MAXB) {
        const int mb = std::min(MAXB, nb - b0);
        XSrc sb = src;
        sb.x = src.x ? src.x + (size_t)b0 * src.ldx : nullptr;
        if (sb.toks) sb.toks = src.toks + b0;
        if (fuse_ok(w, sb, mb)) {
            const int rc = gemv(w, sb, y + (size_t)b0 * ldy, ldy, mb, 0, w.rows, resid, s, 0, 0, epi);
            if (rc != CMF_OK) return rc;
            continue;
        }
        int rc = launch_prep_src(w, sb, mb, m->planes, m->xs, s);
        if (rc != CMF_OK) return rc;
        XSrc g{};
        g.mode = XS_GLOBAL;
        g.planes = m->planes;
        g.xs = m->xs;
        rc = gemv(w, g, y + (size_t)b0 * ldy, ldy, mb, 0, w.rows, resid, s, 0, 0, epi);
        if (rc != CMF_OK) return rc;
    }
    return CMF_OK;
}

// The routed-expert FFN of a block (moe_ffn, pipeline.rs:10868-10915) over
// nb <= 16 rows of h: router logits of the normed rows (a q8 / q4 router on
// the GEMV with the norm staged inside, a dense one on k_router_f32 over
// rows normed by k_rms_rows), then routing + the routed experts, and
// h += their weighted sum.
int moe_block_ffn(cmf_model_s* m, LayerDev& l, float* h, int nb, hipStream_t s) {
    const auto& c = m->c;
    const int H = c.hidden, ne = l.n_experts;
    if (l.router_f32) {
        hipLaunchKernelGGL(k_rms_rows, dim3(nb), dim3(256), 0, s, h, H, l.post_norm, H, c.eps, m->xrows);
        hipLaunchKernelGGL(k_router_f32, dim3((ne + 3) / 4), dim3(256), 0, s, l.router_f32, m->xrows, ne, H, nb,
                           m->rlog);
        XSrc r{};
        r.mode = XS_ROWS;
        r.x = m->xrows;
        r.ldx = H;
        return moe_ffn_launch(l.moe, r, m->rlog, nb, h, H, true, s);
    }
    gemv_f(m, l.router, src_norm(h, H, l.post_norm, c.eps), m->rlog, ne, nb, false, s);
    return moe_ffn_launch(l.moe, src_norm(h, H, l.post_norm, c.eps), m->rlog, nb, h, H, true, s);
}

// One decoder block over nb rows of the residual h at positions *pb + padd
// + i (forward_layers_span, pipeline.rs:7981-8700):
//   h += Wo attn(qk-norm/RoPE(Wqkv rms_norm(h)))
//   h += Wdown (silu(Wg rms_norm(h)) * Wu rms_norm(h))
// The norms are evaluated by the GEMVs that consume them, SwiGLU is the
// gate|up GEMV's epilogue and the residual adds are epilogues too.
void run_block(cmf_model_s* m, LayerDev& l, float* h, int nb, const int* pb, int padd, int max_len,
               hipStream_t s) {
    const auto& c = m->c;
    const int H = c.hidden, hd = c.head_dim, nh = c.n_heads, nkv = c.n_kv;
    const int QKV = (nh + 2 * nkv) * hd, I = c.inter;
    gemv_f(m, l.qkv, src_norm(h, H, l.in_norm, c.eps), m->qkv_out, QKV, nb, false, s);
    // the attention kernel holds at most 32 query heads per kv head and
    // MAXB new rows
    const int rows_per = std::min(MAXB, std::max(1, 32 / (nh / nkv)));
    // a q8 output projection takes its operand straight from the merge:
    // every merge wave writes its head's two 64-column chunks as int8 planes
    // with their own chunk scales, so the wo GEMV neither stages the rows nor
    // waits for a producer launch
    const bool wo_planes = l.wo.dtype == DT_Q8ROW && (nh * hd) % 64 == 0;
    for (int b0 = 0; b0 < nb; b0 += rows_per) {
        AttnArgs at{m->qkv_out + (size_t)b0 * QKV, QKV, l.q_norm, l.k_norm, m->rope, l.kc, l.vc, c.max_seq,
                    std::min(rows_per, nb - b0), nh, nkv, c.eps, pb, padd + b0, m->pm, m->pl, m->po, m->nch_cap,
                    m->ao + (size_t)b0 * nh * hd, 1};
        if (wo_planes) {
            at.wop = m->plw;
            at.wop_cs = m->plw_cs;
            at.wop_M = nb;
            at.wop_b0 = b0;
        }
        launch_attention(at, max_len, s);
    }
    if (wo_planes) {
        XSrc pw{};
        pw.mode = XS_GLOBAL;
        pw.planes = m->plw;
        pw.cs = m->plw_cs;
        pw.cs_ld = l.wo.kchunks;
        (void)gemv(l.wo, pw, h, H, nb, 0, l.wo.rows, true, s);
    } else {
        // the merged rows (ao): prepared inside the wo GEMV for small
        // batches, by a producer launch otherwise
        XSrc ra{};
        ra.mode = XS_ROWS;
        ra.x = m->ao;
        ra.ldx = nh * hd;
        gemv_f(m, l.wo, ra, h, H, nb, true, s);
    }
    if (l.moe) {
        moe_block_ffn(m, l, h, nb, s);
        return;
    }
    // gate|up with the SwiGLU epilogue: gu_out [nb][I] = silu(g) * u
    gemv_f(m, l.gu, src_norm(h, H, l.post_norm, c.eps), m->gu_out, I, nb, false, s, EPI_SWIGLU);
    XSrc sd{};
    sd.mode = XS_ROWS;
    sd.x = m->gu_out;
    sd.ldx = I;
    gemv_f(m, l.down, sd, h, H, nb, true, s);
}

// Trunk forward of nb rows in m->hv (embeddings in, final hidden rows out,
// pre-norm as forward_layers returns them); logits when want_logits.
// Whether block l runs as the two XCD-partitioned launches for nb rows:
// q8 attention weights, q4t FFN weights, a dense FFN, a shape xlayer.hip
// is built for.
// The fused blocks score with f16 hi / lo halves of the normed, rotated q
// and k rows, which needs |q|, |k| < 65504: after the qk-norm an element is at
// most sqrt(head_dim) * max|norm weight| (|x_i| / rms(x) <= sqrt(n)), after
// RoPE sqrt(2) times that, so norm weights up to 2048 keep it below 32768.
constexpr float XL_QK_NORM_MAX = 2048.f;
bool xl_layer_ok(cmf_model_s* m, const LayerDev& l, int nb, int max_len) {
    return m->xl_on && !l.moe && l.kc && l.qkv.dtype == DT_Q8ROW && l.wo.dtype == DT_Q8ROW &&
           l.gu.dtype == DT_Q4T && l.down.dtype == DT_Q4T && l.qk_norm_max <= XL_QK_NORM_MAX &&
           xl_shape_ok(m->xls, nb, max_len);
}
XlAttnW xl_aw(const LayerDev& l) {
    return XlAttnW{l.qkv.w, l.qkv.scale, l.wo.w, l.wo.scale, l.qkv.kchunks, l.wo.kchunks,
                   l.in_norm, l.q_norm, l.k_norm, l.kc, l.vc};
}
XlFfnW xl_fw(const LayerDev& l) {
    return XlFfnW{l.gu.w, l.gu.scale, l.down.w, l.down.scale, l.gu.kchunks, l.down.kchunks, l.post_norm};
}

void trunk_forward(cmf_model_s* m, int nb, const int* pb, int padd, int max_len, bool want_logits,
                   hipStream_t s) {
    const auto& c = m->c;
    bool xl = true;
    for (int li = 0; li < c.n_layers && xl; li++) xl = xl_layer_ok(m, m->L[li], nb, max_len);
    if (xl) {
        for (int li = 0; li < c.n_layers; li++)
            xl_block(m->xl, m->xls, xl_aw(m->L[li]), xl_fw(m->L[li]), m->hv, nb, pb, padd, max_len, m->rope, li, s);
        xl_finish(m->xl, m->xls, m->hv, nb, s);
    } else {
        for (int li = 0; li < c.n_layers; li++) run_block(m, m->L[li], m->hv, nb, pb, padd, max_len, s);
    }
    if (want_logits)
        gemv_f(m, m->lm, src_norm(m->hv, c.hidden, m->final_norm, c.eps), m->logits, c.vocab, nb, false, s);
}

XSrc src_cat(cmf_model_s* m, const int* toks, const float* hid) {
    XSrc r{};
    r.mode = XS_CAT;
    r.x = hid;
    r.ldx = m->c.hidden;
    r.w = m->enorm;
    r.w2 = m->hnorm;
    r.toks = toks;
    r.emb = embed_src(m);
    r.H = m->c.hidden;
    r.K = 2 * m->c.hidden;
    r.eps = m->c.eps;
    return r;
}

// MTP warm (mtp_warm, pipeline.rs:3532-3572): eh_proj on [enorm(embed(tok));
// hnorm(h)], input norm, q/k/v, qk-norm + RoPE, KV append.  No attention.
void mtp_warm(cmf_model_s* m, const int* toks, const float* hid, int nb, const int* pb, int padd, int max_len,
              hipStream_t s) {
    const auto& c = m->c;
    const int H = c.hidden, hd = c.head_dim, nh = c.n_heads, nkv = c.n_kv;
    const int QKV = (nh + 2 * nkv) * hd;
    gemv_f(m, m->eh, src_cat(m, toks, hid), m->hm, H, nb, false, s);
    gemv_f(m, m->mtp.qkv, src_norm(m->hm, H, m->mtp.in_norm, c.eps), m->qkv_out, QKV, nb, false, s);
    AttnArgs at{m->qkv_out, QKV, m->mtp.q_norm, m->mtp.k_norm, m->rope, m->mtp.kc, m->mtp.vc, c.max_seq, nb, nh,
                nkv, c.eps, pb, padd, nullptr, nullptr, nullptr, 0, nullptr, 0};
    launch_attention(at, max_len, s);
}

// One MTP draft step (mtp_step_hl, pipeline.rs:3051-3160) for a single row:
// tok (device), hidden hin (device row) -> hout = the block's output hidden
// (hout != hin), logits row 0.
void mtp_step(cmf_model_s* m, const int* tok, const float* hin, float* hout, const int* pb, int padd,
              int max_len, hipStream_t s) {
    const auto& c = m->c;
    const int H = c.hidden;
    gemv_f(m, m->eh, src_cat(m, tok, hin), hout, H, 1, false, s);
    if (xl_layer_ok(m, m->mtp, 1, max_len)) {
        xl_block(m->xl, m->xls, xl_aw(m->mtp), xl_fw(m->mtp), hout, 1, pb, padd, max_len, m->rope, 0, s);
        xl_finish(m->xl, m->xls, hout, 1, s);
    } else {
        run_block(m, m->mtp, hout, 1, pb, padd, max_len, s);
    }
    gemv_f(m, m->lm, src_norm(hout, H, m->mtp_norm, c.eps), m->logits, c.vocab, 1, false, s);
}

int alloc_scratch(cmf_model_s* m) {
    const auto& c = m->c;
    const int H = c.hidden, hd = c.head_dim, QKV = (c.n_heads + 2 * c.n_kv) * hd;
    m->nch_cap = (c.max_seq + ATT_C - 1) / ATT_C;
    if (dalloc_t(m, &m->hv, (size_t)MAXB * H) || dalloc_t(m, &m->hm, (size_t)MAXB * H) ||
        dalloc_t(m, &m->attn_out, (size_t)MAXB * H) || dalloc_t(m, &m->ffn_out, (size_t)MAXB * H) ||
        dalloc_t(m, &m->qkv_out, (size_t)MAXB * QKV) || dalloc_t(m, &m->qrot, (size_t)MAXB * c.n_heads * hd) || dalloc_t(m, &m->ao, (size_t)MAXB * c.n_heads * hd) ||
        dalloc_t(m, &m->xrows, (size_t)MAXB * std::max(std::max(2 * H, c.inter), c.n_heads * hd)) ||
        dalloc_t(m, &m->hm2, (size_t)MAXB * H) ||
        dalloc_t(m, &m->gu_out, (size_t)MAXB * 2 * c.inter) ||
        dalloc_t(m, &m->pm, (size_t)MAXB * c.n_heads * m->nch_cap) ||
        dalloc_t(m, &m->pl, (size_t)MAXB * c.n_heads * m->nch_cap) ||
        dalloc_t(m, &m->po, (size_t)MAXB * c.n_heads * m->nch_cap * hd) ||
        dalloc_t(m, &m->toks, 4 * MAXB) || dalloc_t(m, &m->st, 1) || dalloc_t(m, &m->h_tip, H) || dalloc_t(m, &m->h_save, H) ||
        dalloc_t(m, &m->xs, 16))
        return CMF_ERR;
    {
        const size_t nk = (size_t)c.n_heads * hd / 64;  // 64-column chunks of the output projection's K
        if (dalloc(m, (void**)&m->plw, nk * 192 * MAXB) || dalloc_t(m, &m->plw_cs, nk * MAXB)) return CMF_ERR;
    }
    {
        // prepared operand of the widest GEMV: q8 K <= max(2H, nh*hd), q4 K <= max(H, I)
        const size_t k8 = ((size_t)std::max(2 * H, c.n_heads * hd) + 63) / 64;
        const size_t k4 = ((size_t)std::max(H, c.inter) + 127) / 128;
        const size_t pb = std::max(k8 * 1024 * 3, k4 * 4 * (1024 * 2 + 128));
        if (dalloc(m, (void**)&m->planes, pb)) return CMF_ERR;
    }
    // rope table (cos, sin) per (position, freq) with the host libm, as
    // rope_rotate (attention.rs:71-81) evaluates it
    const int half = hd / 2;
    std::vector<float> inv(half);
    for (int i = 0; i < half; i++) inv[i] = 1.0f / powf(c.rope_theta, 2.0f * (float)i / (float)hd);
    std::vector<float2> tab((size_t)c.max_seq * half);
    for (int p = 0; p < c.max_seq; p++)
        for (int i = 0; i < half; i++) {
            const float ang = (float)p * inv[i];
            tab[(size_t)p * half + i] = make_float2(cosf(ang), sinf(ang));
        }
    if (dalloc_t(m, &m->rope, tab.size())) return CMF_ERR;
    CMF_HIP(hipMemcpy(m->rope, tab.data(), tab.size() * sizeof(float2), hipMemcpyHostToDevice));
    return CMF_OK;
}

int ensure_logits(cmf_model_s* m) {
    if (m->logits) return CMF_OK;
    const int V = m->c.vocab;
    if (dalloc_t(m, &m->logits, (size_t)(MAXB + 1) * V)) return CMF_ERR;
    const int ns = (V + 4095) / 4096;
    if (dalloc_t(m, &m->am_v, (size_t)(MAXB + 1) * ns) || dalloc_t(m, &m->am_i, (size_t)(MAXB + 1) * ns))
        return CMF_ERR;
    return sample_alloc(m->sb, V, [&](void** p, size_t b) { return dalloc(m, p, b); });
}

// Forget the captured decode round (its nodes hold the buffer addresses).
void drop_graph(cmf_model_s* m) {
    if (m->round_graph) (void)hipGraphExecDestroy(m->round_graph);
    m->round_graph = nullptr;
    if (m->plain_graph) (void)hipGraphExecDestroy(m->plain_graph);
    m->plain_graph = nullptr;
}

int ensure_out(cmf_model_s* m, int cap) {
    if (m->out_cap >= cap) return CMF_OK;
    drop_graph(m);
    if (dalloc_t(m, &m->out, cap)) return CMF_ERR;
    m->out_cap = cap;
    return CMF_OK;
}

__global__ void k_set_int(int* p, int v) { *p = v; }

// prompt positions per prefill chunk: every weight is read once per chunk by
// the large-batch GEMMs (prefill_batch, pipeline.rs:5100-5108), which run
// far better at m = 2048 than at 256 (2048-position prefill of config 4:
// 33.9 ms in chunks of 256, 24.9 of 512, 21.7 of 1024, 18.5 of 2048); the
// CMF_PREFILL_CHUNK environment variable (read once) overrides it
static int prefill_chunk() {
    static const int v = [] {
        const char* e = getenv("CMF_PREFILL_CHUNK");
        const int c = e ? atoi(e) : 2048;
        return c >= 16 && c <= 4096 ? c : 2048;
    }();
    return v;
}

int ensure_prefill_bufs(cmf_model_s* m) {
    if (m->pf_h) return CMF_OK;
    const auto& c = m->c;
    const int H = c.hidden, QKV = (c.n_heads + 2 * c.n_kv) * c.head_dim;
    const size_t R = std::min(prefill_chunk(), c.max_seq);
    if (dalloc_t(m, &m->pf_h, R * H) || dalloc_t(m, &m->pf_qkv, R * QKV) ||
        dalloc_t(m, &m->pf_ao, R * c.n_heads * c.head_dim) || dalloc_t(m, &m->pf_gu, R * 2 * c.inter) ||
        dalloc_t(m, &m->pf_hm, R * H) || dalloc_t(m, &m->pf_toks, R) ||
        dalloc_t(m, &m->pf_q, R * c.n_heads * c.head_dim) ||
        dalloc(m, (void**)&m->pf_khl, (size_t)c.n_kv * ((c.max_seq + 127) / 128 * 128) * c.head_dim * 8) ||
        dalloc_t(m, &m->pf_cells, PREFILL_XCD_CELLS) || dalloc_t(m, &m->pf_err, 1))
        return CMF_ERR;
    // (tags start at 1, so the zeroed cells hold none)
    CMF_HIP(hipMemset(m->pf_cells, 0, PREFILL_XCD_CELLS * sizeof(unsigned long long)));
    CMF_HIP(hipMemset(m->pf_err, 0, sizeof(int)));
    return CMF_OK;
}

// Causal attention of cnt chunk rows (positions *pb + i) in groups the
// attention kernel serves (at most 32 queries per kv head); attend = 0 only
// appends their K/V (the MTP warm).
void prefill_attention(cmf_model_s* m, LayerDev& l, const float* qkv, float* ao, int cnt, const int* pb, int p0,
                       bool attend, hipStream_t s) {
    const auto& c = m->c;
    const int hd = c.head_dim, nh = c.n_heads, nkv = c.n_kv, QKV = (nh + 2 * nkv) * hd;
    static const bool tiled = !(getenv("CMF_PREFILL_ATTN") && getenv("CMF_PREFILL_ATTN")[0] == '0');
    if (tiled && prefill_attention_fits(nh, nkv, hd)) {
        // the whole chunk at once: the tiled prefill attention (one launch
        // for the norms + append, one for the attention)
        PrefillAttnArgs pa{qkv, QKV, l.q_norm, l.k_norm, m->rope, l.kc, l.vc, c.max_seq, cnt, p0, nh, nkv,
                           c.eps, m->pf_q, attend ? ao : nullptr, m->pf_khl, m->pf_cells, m->pf_err, ++m->pf_tag,
                           !m->pf_xcd_off};
        launch_prefill_attention(pa, s);
        return;
    }
    const int rows_per = std::min(MAXB, std::max(1, 32 / (nh / nkv)));
    for (int b0 = 0; b0 < cnt; b0 += rows_per) {
        const int nb = std::min(rows_per, cnt - b0);
        AttnArgs at{qkv + (size_t)b0 * QKV, QKV, l.q_norm, l.k_norm, m->rope, l.kc, l.vc, c.max_seq, nb, nh, nkv,
                    c.eps, pb, b0, attend ? m->pm : nullptr, attend ? m->pl : nullptr, attend ? m->po : nullptr,
                    attend ? m->nch_cap : 0, attend ? ao + (size_t)b0 * nh * hd : nullptr, attend ? 1 : 0};
        launch_attention(at, p0 + b0 + nb, s);
    }
}

// One decoder block over a prefill chunk of cnt rows of h (forward_layers_span
// over a batch, pipeline.rs:5100-5108 / 7981-8700) on the GEMMs: the
// norm and SwiGLU producers prepare each GEMM's operand, the residual adds
// are GEMM epilogues.
int prefill_block(cmf_model_s* m, LayerDev& l, float* h, int cnt, const int* pb, int p0, hipStream_t s) {
    const auto& c = m->c;
    const int H = c.hidden, hd = c.head_dim, nh = c.n_heads, QKV = (nh + 2 * c.n_kv) * hd, I = c.inter;
    int rc = gemm(l.qkv, src_norm(h, H, l.in_norm, c.eps), cnt, m->pf_qkv, QKV, false, s);
    if (rc != CMF_OK) return rc;
    prefill_attention(m, l, m->pf_qkv, m->pf_ao, cnt, pb, p0, true, s);
    XSrc ra{};
    ra.mode = XS_ROWS;
    ra.x = m->pf_ao;
    ra.ldx = nh * hd;
    if ((rc = gemm(l.wo, ra, cnt, h, H, true, s)) != CMF_OK) return rc;
    if (l.moe) {  // the routed experts in batches of 16 rows (the verify-batch kernels)
        for (int b0 = 0; b0 < cnt; b0 += MAXB)
            if ((rc = moe_block_ffn(m, l, h + (size_t)b0 * H, std::min(MAXB, cnt - b0), s))) return rc;
        return CMF_OK;
    }
    if ((rc = gemm(l.gu, src_norm(h, H, l.post_norm, c.eps), cnt, m->pf_gu, 2 * I, false, s)) != CMF_OK) return rc;
    XSrc sd{};
    sd.mode = XS_SILU8;
    sd.x = m->pf_gu;
    sd.ldx = 2 * I;
    sd.K = I;
    return gemm(l.down, sd, cnt, h, H, true, s);
}

__global__ void k_copy_rows_i32(int* dst, const int* src, int n) {
    const int i = threadIdx.x;
    if (i < n) dst[i] = src[i];
}

// verify batch tokens [t_next, d_0 .. d_{K-1}]
// greedy acceptance (pipeline.rs:3989-3999): a = longest prefix with
// argmax(row i) == d_i; emits [t_next, d_0..d_{a-1}]; next token argmax(row a)
__device__ __forceinline__ void accept_greedy(DState* st, int k, int* out) {
    int a = 0;
    while (a < k && st->argmax[a] == st->drafts[a]) a++;
    const int n = st->n_out;
    out[n] = st->t_next;
    for (int j = 0; j < a; j++) out[n + 1 + j] = st->drafts[j];
    st->n_out = n + 1 + a;
    st->a = a;
    st->t_new = st->argmax[a];
    st->accepted += a;
}

// The verify rows' argmax (second pass, wave r reduces row r's partials)
// followed by the greedy acceptance in the same launch: one workgroup of
// 64 (k + 1) threads, k <= 8.
__global__ __launch_bounds__(1024) void k_argmax_accept(const float* __restrict__ pv,
                                                                   const int* __restrict__ pi, int ns, DState* st,
                                                                   int k, int* out) {
    const int r = threadIdx.x >> 6, lane = threadIdx.x & 63;
    float bv = -INFINITY;
    int bi = 0;
    for (int s = lane; s < ns; s += 64) argmax_take(bv, bi, pv[(size_t)r * ns + s], pi[(size_t)r * ns + s]);
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const float v2 = __shfl_xor(bv, o);
        const int i2 = __shfl_xor(bi, o);
        argmax_take(bv, bi, v2, i2);
    }
    __shared__ int win[MAXB + 1];
    if (lane == 0) win[r] = bi;
    __syncthreads();
    if (threadIdx.x == 0) {
        // one thread writes the rows' picks and then reads them back
        for (int j = 0; j <= k; j++) st->argmax[j] = win[j];
        accept_greedy(st, k, out);
    }
}

// commit: h_tip = hidden row a, next_pos += a + 1, t_next = t_new
__global__ void k_commit(DState* st, const float* hv, float* h_tip, int H) {
    const int a = st->a;
    for (int i = threadIdx.x; i < H; i += blockDim.x) h_tip[i] = hv[(size_t)a * H + i];
    __syncthreads();
    if (threadIdx.x == 0) {
        st->next_pos += a + 1;
        st->t_next = st->t_new;
    }
}

// plain step commit: emit t_next, next token = row-0 pick
__global__ void k_plain_commit(DState* st, const float* hv, float* h_tip, int H, int* out,
                               int use_sample) {
    for (int i = threadIdx.x; i < H; i += blockDim.x) h_tip[i] = hv[i];
    __syncthreads();
    if (threadIdx.x == 0) {
        out[st->n_out] = st->t_next;
        st->n_out += 1;
        st->next_pos += 1;
        st->t_next = use_sample ? st->t_new : st->argmax[0];
    }
}

// emit t_next without advancing (the last token of a generation)
__global__ void k_emit(DState* st, int* out) { out[st->n_out++] = st->t_next; }

// after prefill: t_next = pick of the last hidden's logits
__global__ void k_first_token(DState* st, int use_sample) {
    st->t_next = use_sample ? st->t_new : st->argmax[0];
}

}  // namespace

// ---------------------------------------------------------------------------
// C ABI
// ---------------------------------------------------------------------------
extern "C" {

int cmf_model_create(const cmf_model_config* cfg, cmf_model* out) {
    if (ensure_init() != CMF_OK) return CMF_ERR;
    if (!cfg || !out) return fail("model_create: null argument");
    const auto& c = *cfg;
    if (c.n_layers < 1 || c.hidden < 64 || c.n_heads < 1 || c.n_kv < 1 || c.n_heads % c.n_kv ||
        c.vocab < 1 || c.max_seq < 8 || c.inter < 32)
        return fail("model_create: bad config");
    if (c.head_dim != 128) return fail("model_create: the attention kernels are built for head_dim 128");
    if ((c.n_heads / c.n_kv) & (c.n_heads / c.n_kv - 1))
        return fail("model_create: query heads per KV head must be a power of two");
    if (c.n_heads / c.n_kv > 32) return fail("model_create: at most 32 query heads per KV head");
    if (c.hidden > 4096 || c.inter > 12288 || c.n_heads * c.head_dim > 4096)
        return fail("model_create: hidden <= 4096, inter <= 12288, heads*head_dim <= 4096");
    if (c.hidden % 32 || c.inter % 32) return fail("model_create: hidden and inter must be multiples of 32");
    auto* m = new cmf_model_s();
    m->c = c;
    const char* g = getenv("CMF_DECODE_GRAPH");  // "0": launch every round eagerly
    m->use_graph = !(g && g[0] == '0');
    m->L.resize(c.n_layers);
    if (alloc_scratch(m) != CMF_OK) {
        cmf_model_free(m);
        return CMF_ERR;
    }
    m->xls = XlShape{c.hidden, c.inter, c.n_heads, c.n_kv, c.head_dim, c.max_seq, c.eps};
    const char* xe = getenv("CMF_XL");  // "0": the six-launch blocks only
    if (!(xe && xe[0] == '0') && xl_shape_ok(m->xls, 1, 16)) {
        if (xl_alloc(m->xl, m->xls, xl_dalloc, m) != CMF_OK) {
            cmf_model_free(m);
            return CMF_ERR;
        }
        m->xl_on = true;
    }
    *out = m;
    return CMF_OK;
}

int cmf_model_free(cmf_model m) {
    if (!m) return CMF_OK;
    (void)hipStreamSynchronize(stream());
    drop_graph(m);
    for (auto& l : m->L) {
        free_layer(l);
        free_weight(l.router);
    }
    free_layer(m->mtp);
    free_weight(m->lm);
    free_weight(m->emb);
    free_weight(m->eh);
    for (void* p : m->allocs) (void)hipFree(p);
    delete m;
    return CMF_OK;
}

int cmf_model_set_layer(cmf_model m, int li, const cmf_layer_desc* d) {
    if (m) drop_graph(m);
    if (!m || !d || li < 0 || li >= m->c.n_layers) return fail("set_layer: bad arguments");
    if (m->c.n_heads / m->c.n_kv * MAXB > 32 && m->c.n_heads / m->c.n_kv > 2)
        return fail("set_layer: the attention kernel serves <= 32 queries per KV head");
    m->L[li].moe = nullptr;
    free_weight(m->L[li].router);
    return upload_layer(m, m->L[li], d, true);
}

int cmf_model_set_layer_moe(cmf_model m, int li, const cmf_layer_desc* d, const cmf_tensor* router,
                            cmf_moe moe) {
    if (m) drop_graph(m);
    if (!m || !d || !router || !moe || li < 0 || li >= m->c.n_layers) return fail("set_layer_moe: bad arguments");
    const auto& c = m->c;
    const int H = c.hidden, hd = c.head_dim, Q = c.n_heads * hd, KV = c.n_kv * hd;
    if (moe_hidden(moe) != H) return fail("set_layer_moe: the MoE layer's hidden differs from the model's");
    const int ne = moe_experts_count(moe);
    const bool dense = router->dtype == 0 || router->dtype == 1 || router->dtype == 2;  // F32 / F16 / BF16
    if (dense) {
        if (router->rows != ne || router->cols != H || !router->bytes)
            return fail("set_layer_moe: router must be [n_experts x hidden] with its bytes");
    } else if (check_tensor(*router, ne, H, "router")) {
        return CMF_ERR;
    }
    if (check_tensor(d->wq, Q, H, "wq") || check_tensor(d->wk, KV, H, "wk") || check_tensor(d->wv, KV, H, "wv") ||
        check_tensor(d->wo, H, Q, "wo"))
        return CMF_ERR;
    LayerDev& l = m->L[li];
    if (upload_f32(m, &l.in_norm, d->input_norm, H) || upload_f32(m, &l.post_norm, d->post_norm, H) ||
        upload_f32(m, &l.q_norm, d->q_norm, hd) || upload_f32(m, &l.k_norm, d->k_norm, hd))
        return CMF_ERR;
    free_layer(l);
    free_weight(l.router);
    l.router_f32 = nullptr;
    if (build_cat(l.qkv, {&d->wq, &d->wk, &d->wv}) || build_cat(l.wo, {&d->wo})) return CMF_ERR;
    if (dense) {
        // f16 / bf16 widen exactly to f32 (dequant_tensor; load_matrix keeps an f32 QTensor)
        std::vector<float> w((size_t)ne * H);
        for (size_t i = 0; i < w.size(); i++) {
            if (router->dtype == 0) {
                memcpy(&w[i], router->bytes + 4 * i, 4);
            } else {
                uint16_t u;
                memcpy(&u, router->bytes + 2 * i, 2);
                if (router->dtype == 2) {
                    const uint32_t bits = (uint32_t)u << 16;
                    memcpy(&w[i], &bits, 4);
                } else {
                    w[i] = (float)__builtin_bit_cast(_Float16, u);
                }
            }
        }
        if (upload_f32(m, &l.router_f32, w.data(), w.size())) return CMF_ERR;
    } else if (build_cat(l.router, {router})) {
        return CMF_ERR;
    }
    l.n_experts = ne;
    if (!l.kc) {
        const size_t n = (size_t)c.n_kv * c.max_seq * hd;
        if (dalloc_t(m, &l.kc, n) || dalloc_t(m, &l.vc, n)) return CMF_ERR;
    }
    if (m->rlog_cap < ne) {
        if (dalloc_t(m, &m->rlog, (size_t)MAXB * ne)) return CMF_ERR;
        m->rlog_cap = ne;
    }
    l.moe = moe;
    return CMF_OK;
}

int cmf_model_set_head(cmf_model m, const cmf_tensor* lm, const float* final_norm) {
    if (m) drop_graph(m);
    if (!m || !lm) return fail("set_head: null argument");
    if (lm->dtype != DT_Q8ROW) return fail("set_head: the tied lm_head/embedding must be q8");
    if (check_tensor(*lm, m->c.vocab, m->c.hidden, "lm_head")) return CMF_ERR;
    if (upload_f32(m, &m->final_norm, final_norm, m->c.hidden)) return CMF_ERR;
    free_weight(m->lm);
    if (build_cat(m->lm, {lm})) return CMF_ERR;
    if (ensure_logits(m)) return CMF_ERR;
    m->has_head = true;
    return CMF_OK;
}

int cmf_model_set_embed(cmf_model m, const cmf_tensor* e) {
    if (m) drop_graph(m);
    if (!m || !e) return fail("set_embed: null argument");
    if (e->dtype != DT_Q8ROW) return fail("set_embed: the embedding table must be q8");
    if (check_tensor(*e, m->c.vocab, m->c.hidden, "embed_tokens")) return CMF_ERR;
    free_weight(m->emb);
    return build_cat(m->emb, {e});
}

int cmf_model_fused_blocks(cmf_model m) { return m && m->xl_on ? 1 : 0; }

int cmf_model_set_mtp(cmf_model m, const float* enorm, const float* hnorm, const cmf_tensor* eh,
                      const cmf_layer_desc* layer, const float* norm) {
    if (m) drop_graph(m);
    if (!m || !eh || !layer) return fail("set_mtp: null argument");
    const int H = m->c.hidden;
    if (check_tensor(*eh, H, 2 * H, "eh_proj")) return CMF_ERR;
    if (upload_f32(m, &m->enorm, enorm, H) || upload_f32(m, &m->hnorm, hnorm, H) ||
        upload_f32(m, &m->mtp_norm, norm, H))
        return CMF_ERR;
    free_weight(m->eh);
    if (build_cat(m->eh, {eh})) return CMF_ERR;
    if (upload_layer(m, m->mtp, layer, true)) return CMF_ERR;
    m->has_mtp = true;
    return CMF_OK;
}

// After a call that ran XCD-partitioned blocks (stream idle): an exchange
// wait that gave up, more attention positions than a launch's bound or two
// workgroups on one (XCD, index) slot (xlayer.h, err bits 1, 4, 8) mean the
// call wrote wrong values.  The model then switches to the six-launch
// blocks for good and XL_RETRY asks the caller to restore its state and run
// the call again.  The generation is reset before the exchange tags could
// repeat.  (CMF_XL_FORCE_FAIL=1 reports one failure, to test the fallback.)
constexpr int XL_RETRY = 2;
static int xl_check(cmf_model m) {
    if (!m->xl_on) return CMF_OK;
    uint32_t w[17] = {};  // gen at 0, err at 16
    CMF_HIP(hipMemcpy(w, m->xl.gen, sizeof(w), hipMemcpyDeviceToHost));
    int e = (int)w[16];
    static bool force = getenv("CMF_XL_FORCE_FAIL") && getenv("CMF_XL_FORCE_FAIL")[0] == '1';
    if (force) {
        force = false;
        e |= 1;
    }
    if (e != 0) {
        CMF_HIP(hipMemset(m->xl.err, 0, sizeof(int)));
        m->xl_on = false;
        m->xl_fallbacks += 1;
        drop_graph(m);
        return XL_RETRY;
    }
    if (w[0] >= XL_GEN_RESET) {
        xl_reset(m->xl, stream());
        CMF_HIP(hipStreamSynchronize(stream()));
    }
    return CMF_OK;
}
// The decode state and tip hidden before a call that may have to run again.
struct XlSnap {
    DState st;
};
static int xl_save(cmf_model m, XlSnap& sn) {
    if (!m->xl_on) return CMF_OK;
    hipStream_t s = stream();
    CMF_HIP(hipMemcpyAsync(&sn.st, m->st, sizeof(DState), hipMemcpyDeviceToHost, s));
    CMF_HIP(hipMemcpyAsync(m->h_save, m->h_tip, (size_t)m->c.hidden * sizeof(float), hipMemcpyDeviceToDevice, s));
    CMF_HIP(hipStreamSynchronize(s));
    return CMF_OK;
}
static int xl_restore(cmf_model m, const XlSnap& sn) {
    hipStream_t s = stream();
    CMF_HIP(hipMemcpyAsync(m->st, &sn.st, sizeof(DState), hipMemcpyHostToDevice, s));
    CMF_HIP(hipMemcpyAsync(m->h_tip, m->h_save, (size_t)m->c.hidden * sizeof(float), hipMemcpyDeviceToDevice, s));
    CMF_HIP(hipStreamSynchronize(s));
    return CMF_OK;
}

static int ready(cmf_model m) {
    if (!m) return fail("null model");
    if (!m->has_head) return fail("model has no lm_head (cmf_model_set_head)");
    for (auto& l : m->L) {
        if (!l.qkv.w) return fail("model has unset layers (cmf_model_set_layer)");
        if (l.moe && moe_prepare(l.moe) != CMF_OK) return CMF_ERR;  // before any captured round
    }
    return CMF_OK;
}

int cmf_prefill(cmf_model m, const int32_t* ids, int n) {
    if (ready(m)) return CMF_ERR;
    if (!ids || n < 1 || n + 1 > m->c.max_seq) return fail("prefill: 1 <= n < max_seq");
    if (ensure_prefill_bufs(m)) return CMF_ERR;
    for (int i = 0; i < n; i++)
        if (ids[i] < 0 || ids[i] >= m->c.vocab) return fail("prefill: token id out of range");
    hipStream_t s = stream();
    const auto& c = m->c;
    const int H = c.hidden, QKV = (c.n_heads + 2 * c.n_kv) * c.head_dim;
    int* pb = &m->st->next_pos;
    const int chunk = prefill_chunk();
    for (int p0 = 0; p0 < n; p0 += chunk) {
        const int cnt = std::min(chunk, n - p0);
        CMF_HIP(hipMemcpyAsync(m->pf_toks, ids + p0, cnt * sizeof(int), hipMemcpyHostToDevice, s));
        hipLaunchKernelGGL(k_set_int, dim3(1), dim3(1), 0, s, pb, p0);
        launch_embed(m->pf_toks, embed_src(m), H, m->pf_h, H, cnt, s);
        for (int li = 0; li < c.n_layers; li++)
            if (prefill_block(m, m->L[li], m->pf_h, cnt, pb, p0, s) != CMF_OK) return CMF_ERR;
        if (m->has_mtp) {
            // MTP warm on the (h_p, id_{p+1}) pairs of the chunk (pipeline.rs:2275-2318)
            const int pairs = (p0 + cnt < n) ? cnt : cnt - 1;
            if (pairs > 0) {
                CMF_HIP(hipMemcpyAsync(m->pf_toks, ids + p0 + 1, pairs * sizeof(int), hipMemcpyHostToDevice, s));
                if (gemm(m->eh, src_cat(m, m->pf_toks, m->pf_h), pairs, m->pf_hm, H, false, s) ||
                    gemm(m->mtp.qkv, src_norm(m->pf_hm, H, m->mtp.in_norm, c.eps), pairs, m->pf_qkv, QKV, false, s))
                    return CMF_ERR;
                prefill_attention(m, m->mtp, m->pf_qkv, nullptr, pairs, pb, p0, false, s);
            }
        }
        if (p0 + cnt == n)
            CMF_HIP(hipMemcpyAsync(m->h_tip, m->pf_h + (size_t)(cnt - 1) * H, H * sizeof(float),
                                   hipMemcpyDeviceToDevice, s));
        CMF_HIP(hipStreamSynchronize(s));  // the host ids of this chunk are reused
    }
    hipLaunchKernelGGL(k_set_int, dim3(1), dim3(1), 0, s, pb, n);
    CMF_HIP(hipMemsetAsync(&m->st->n_out, 0, sizeof(int), s));
    CMF_HIP(hipStreamSynchronize(s));
    CMF_HIP(hipGetLastError());
    // the XCD prefill attention's placement check: a collision means some
    // (query block, kv head) went unserved; the prefill runs again on the
    // grid-indexed variant, which the model keeps from then on
    // (CMF_PREFILL_PLACEMENT_FAIL=1 reports a collision once, to test this path)
    int perr = 0;
    CMF_HIP(hipMemcpy(&perr, m->pf_err, sizeof(int), hipMemcpyDeviceToHost));
    static const bool force_fail = getenv("CMF_PREFILL_PLACEMENT_FAIL") && getenv("CMF_PREFILL_PLACEMENT_FAIL")[0] == '1';
    if (force_fail && !m->pf_xcd_off && prefill_attention_fits(c.n_heads, c.n_kv, c.head_dim) && c.n_kv == 8)
        perr = 1;
    if (perr && !m->pf_xcd_off) {
        m->pf_xcd_off = true;
        CMF_HIP(hipMemset(m->pf_err, 0, sizeof(int)));
        return cmf_prefill(m, ids, n);
    }
    m->next_pos_host = n;
    m->prefilled = true;
    return CMF_OK;
}

int cmf_model_prefill_xcd(cmf_model m) { return m ? (m->pf_xcd_off ? 0 : 1) : CMF_ERR; }

// logits of the tip hidden -> next token (greedy argmax or device sampler)
static void pick_from_tip(cmf_model m, bool sampling, const cmf_sampler_config* sc, hipStream_t s) {
    const int H = m->c.hidden;
    gemv_f(m, m->lm, src_norm(m->h_tip, H, m->final_norm, m->c.eps), m->logits, m->c.vocab, 1, false, s);
    if (sampling) sample_rows(m->sb, m->logits, m->c.vocab, 1, *sc, m->st, SampleMode::Plain, 0, nullptr, s);
    else launch_argmax(m->logits, m->c.vocab, m->c.vocab, 1, m->am_v, m->am_i, m->st->argmax, s);
}

// One speculative round (graph_spec_step, pipeline.rs:3582-4213) on the
// device state: K chained MTP drafts, the K+1-row verify, acceptance, the
// MTP re-warm of the verified pairs and the commit.  np = next_pos (host
// mirror, sizes the attention grids).
static void spec_round(cmf_model m, int k, bool sampling, const cmf_sampler_config& sc, int np,
                       hipStream_t s, int graph_len = 0) {
    const int H = m->c.hidden, V = m->c.vocab;
    int* pb = &m->st->next_pos;
    for (int j = 0; j < k; j++) {
        const int* tok = j == 0 ? &m->st->t_next : &m->st->drafts[j - 1];
        float* bufs[2] = {m->hm, m->hm2};
        const float* hin = j == 0 ? m->h_tip : bufs[(j - 1) & 1];
        mtp_step(m, tok, hin, bufs[j & 1], pb, j - 1, graph_len ? graph_len : np + j, s);
        if (sampling) sample_rows(m->sb, m->logits, V, 1, sc, m->st, SampleMode::Draft, j, nullptr, s);
        else launch_argmax(m->logits, V, V, 1, m->am_v, m->am_i, &m->st->drafts[j], s);
    }
    launch_embed(m->st->drafts, embed_src(m), H, m->hv, H, k + 1, s, &m->st->t_next);
    trunk_forward(m, k + 1, pb, 0, graph_len ? graph_len : np + k + 1, true, s);
    if (sampling) {
        sample_rows(m->sb, m->logits, V, k + 1, sc, m->st, SampleMode::Accept, k, m->out, s);
    } else {
        const int ns = launch_argmax_part(m->logits, V, V, k + 1, m->am_v, m->am_i, s);
        hipLaunchKernelGGL(k_argmax_accept, dim3(1), dim3(64 * (k + 1)), 0, s, m->am_v, m->am_i, ns, m->st, k,
                           m->out);
    }
    mtp_warm(m, m->st->drafts, m->hv, k, pb, 0, graph_len ? graph_len : np + k + 1, s);
    hipLaunchKernelGGL(k_commit, dim3(1), dim3(256), 0, s, m->st, m->hv, m->h_tip, H);
}

// One plain decode step: forward t_next at next_pos, emit it, pick the next.
// graph_len > 0: the attention length bound of a captured step (every
// position-dependent value is read from the device state).
static void plain_step(cmf_model m, bool sampling, const cmf_sampler_config& sc, int np, hipStream_t s,
                       int graph_len = 0) {
    const int H = m->c.hidden, V = m->c.vocab;
    int* pb = &m->st->next_pos;
    launch_embed(&m->st->t_next, embed_src(m), H, m->hv, H, 1, s);
    trunk_forward(m, 1, pb, 0, graph_len ? graph_len : np + 1, true, s);
    if (sampling) sample_rows(m->sb, m->logits, V, 1, sc, m->st, SampleMode::Plain, 0, nullptr, s);
    else launch_argmax(m->logits, V, V, 1, m->am_v, m->am_i, m->st->argmax, s);
    hipLaunchKernelGGL(k_plain_commit, dim3(1), dim3(256), 0, s, m->st, m->hv, m->h_tip, H, m->out,
                       sampling ? 1 : 0);
}

static int check_sampler(cmf_model m, const cmf_sampler_config* sc) {
    if (!sc) return fail("null sampler config");
    if (sc->repetition_penalty != 1.0f || sc->presence_penalty != 0.0f) return CMF_DECLINED;
    if (sc->temperature >= 1e-6f) {
        if (sc->top_k < 1 || (int)sc->top_k > SPARSE_K_MAX) return CMF_DECLINED;
        if (m->sb.nslices * (int)sc->top_k > SLICE) return CMF_DECLINED;
    }
    return CMF_OK;
}

int cmf_decode_begin(cmf_model m, const cmf_sampler_config* sc, uint64_t seed) {
    if (ready(m)) return CMF_ERR;
    if (!m->prefilled) return fail("decode: call cmf_prefill first");
    int rc = check_sampler(m, sc);
    if (rc != CMF_OK) return rc;
    if (ensure_out(m, m->c.max_seq + 32)) return CMF_ERR;
    hipStream_t s = stream();
    DState init{};
    init.next_pos = m->next_pos_host;
    init.rng = seed;
    init.forced = -1;
    CMF_HIP(hipMemcpyAsync(m->st, &init, sizeof(DState), hipMemcpyHostToDevice, s));
    CMF_HIP(hipStreamSynchronize(s));
    m->sc = *sc;
    const bool sampling = sc->temperature >= 1e-6f;
    pick_from_tip(m, sampling, sc, s);
    hipLaunchKernelGGL(k_first_token, dim3(1), dim3(1), 0, s, m->st, sampling ? 1 : 0);
    CMF_HIP(hipStreamSynchronize(s));
    CMF_HIP(hipGetLastError());
    m->decoding = true;
    m->rounds = 0;
    m->emitted_host = 0;
    m->accepted_host = 0;
    return CMF_OK;
}

static int decode_rounds_impl(cmf_model m, int n, int spec, int k, cmf_gen_stats* stats) {
    if (ready(m)) return CMF_ERR;
    if (!m->decoding) return fail("decode_rounds: call cmf_decode_begin first");
    if (spec && !m->has_mtp) return fail("decode: speculation needs the MTP head (cmf_model_set_mtp)");
    if (spec && (k < 1 || k > 8)) return fail("decode: k must be 1..8 (CMF_GRAPH_SPEC_K range)");
    if (n < 0) return fail("decode_rounds: n < 0");
    const int per = spec ? k + 1 : 1;
    if (m->next_pos_host + (n + 1) * per + 2 > m->c.max_seq) return fail("decode: max_seq too small");
    if (m->emitted_host + (n + 1) * per + 2 > m->out_cap) return fail("decode: output buffer full");
    hipStream_t s = stream();
    const bool sampling = m->sc.temperature >= 1e-6f;
    hipEvent_t e0, e1;
    CMF_HIP(hipEventCreate(&e0));
    CMF_HIP(hipEventCreate(&e1));
    CMF_HIP(hipEventRecord(e0, s));
    DState hs{};
    int np = m->next_pos_host;
    int r0 = 0;
    if (spec && m->use_graph && n > 1) {
        // The captured round reads every position-dependent value from the
        // device state; only the attention grid is sized on the host, by a
        // bound on the positions these n rounds can reach (512-position steps).
        const int need = std::min(m->c.max_seq, ((np + (n + 1) * (k + 1) + 511) / 512) * 512);
        if (!m->round_graph || m->graph_k != k || m->graph_sampling != (int)sampling || m->graph_len < need) {
            // one eager round first: it sets the kernels' launch attributes
            spec_round(m, k, sampling, m->sc, np, s);
            r0 = 1;
            if (m->round_graph) {
                (void)hipGraphExecDestroy(m->round_graph);
                m->round_graph = nullptr;
            }
            hipGraph_t g;
            CMF_HIP(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal));
            spec_round(m, k, sampling, m->sc, np, s, need);
            CMF_HIP(hipStreamEndCapture(s, &g));
            const hipError_t ie = hipGraphInstantiate(&m->round_graph, g, nullptr, nullptr, 0);
            (void)hipGraphDestroy(g);
            CMF_HIP(ie);
            m->graph_k = k;
            m->graph_sampling = (int)sampling;
            m->graph_len = need;
        }
        for (int r = r0; r < n; r++) CMF_HIP(hipGraphLaunch(m->round_graph, s));
        r0 = n;
    }
    if (!spec && m->use_graph && n > 1) {
        // plain steps the same way: one eager step, then one captured step
        // replayed (the forward_token_graph counterpart, gpu.rs:1368)
        const int need = std::min(m->c.max_seq, ((np + n + 2 + 511) / 512) * 512);
        if (!m->plain_graph || m->plain_sampling != (int)sampling || m->plain_len < need) {
            plain_step(m, sampling, m->sc, np, s);
            np += 1;
            r0 = 1;
            if (m->plain_graph) {
                (void)hipGraphExecDestroy(m->plain_graph);
                m->plain_graph = nullptr;
            }
            hipGraph_t g;
            CMF_HIP(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal));
            plain_step(m, sampling, m->sc, np, s, need);
            CMF_HIP(hipStreamEndCapture(s, &g));
            const hipError_t ie = hipGraphInstantiate(&m->plain_graph, g, nullptr, nullptr, 0);
            (void)hipGraphDestroy(g);
            CMF_HIP(ie);
            m->plain_sampling = (int)sampling;
            m->plain_len = need;
        }
        for (int r = r0; r < n; r++) CMF_HIP(hipGraphLaunch(m->plain_graph, s));
        r0 = n;
    }
    for (int r = r0; r < n; r++) {
        if (spec) {
            spec_round(m, k, sampling, m->sc, np, s);
            CMF_HIP(hipMemcpyAsync(&hs, m->st, sizeof(DState), hipMemcpyDeviceToHost, s));
            CMF_HIP(hipStreamSynchronize(s));
            np = hs.next_pos;
        } else {
            plain_step(m, sampling, m->sc, np, s);
            np += 1;
        }
    }
    CMF_HIP(hipEventRecord(e1, s));
    CMF_HIP(hipMemcpyAsync(&hs, m->st, sizeof(DState), hipMemcpyDeviceToHost, s));
    CMF_HIP(hipStreamSynchronize(s));
    CMF_HIP(hipGetLastError());
    float ms = 0.f;
    CMF_HIP(hipEventElapsedTime(&ms, e0, e1));
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    const int xc = xl_check(m);
    if (xc != CMF_OK) return xc;
    m->next_pos_host = hs.next_pos;
    m->emitted_host = hs.n_out;
    m->rounds += spec ? n : 0;
    if (stats) {  // this call's rounds
        stats->generated = hs.n_out;
        stats->drafted = spec ? n * k : 0;
        stats->accepted = hs.accepted - m->accepted_host;
        stats->rounds = spec ? n : 0;
        stats->device_ms = ms;
    }
    m->accepted_host = hs.accepted;
    return CMF_OK;
}

// Rounds in pieces of at most 2^16 (a piece's generations stay far below
// the tag reset point, xl_check running between pieces); a piece whose
// XCD-partitioned blocks failed their check runs again from the state
// before it on the six-launch blocks.
int cmf_decode_rounds(cmf_model m, int n, int spec, int k, cmf_gen_stats* stats) {
    if (!m) return fail("null model");
    if (n < 0) return fail("decode_rounds: n < 0");
    cmf_gen_stats tot{};
    int done = 0;
    do {
        const int piece = std::min(n - done, 1 << 16);
        XlSnap sn{};
        if (xl_save(m, sn) != CMF_OK) return CMF_ERR;
        cmf_gen_stats st{};
        int rc = decode_rounds_impl(m, piece, spec, k, &st);
        if (rc == XL_RETRY) {
            if (xl_restore(m, sn) != CMF_OK) return CMF_ERR;
            rc = decode_rounds_impl(m, piece, spec, k, &st);
        }
        if (rc != CMF_OK) return rc == XL_RETRY ? fail("decode: XCD-partitioned blocks failed twice") : rc;
        tot.generated = st.generated;
        tot.drafted += st.drafted;
        tot.accepted += st.accepted;
        tot.rounds += st.rounds;
        tot.device_ms += st.device_ms;
        done += piece;
    } while (done < n);
    if (stats) *stats = tot;
    return CMF_OK;
}

int cmf_model_xl_fallbacks(cmf_model m) { return m ? m->xl_fallbacks : CMF_ERR; }

int cmf_decode_tokens(cmf_model m, int32_t* out, int cap) {
    if (!m || !out) return fail("decode_tokens: null argument");
    const int n = std::min(cap, m->emitted_host);
    if (n > 0) CMF_HIP(hipMemcpy(out, m->out, n * sizeof(int), hipMemcpyDeviceToHost));
    return n;
}

// The speculation monitor (SpecMon, pipeline.rs:661-694): exponential
// averages of a speculative round's wall time and of the tokens it produced,
// and the plain token's wall time.  A round pays when tokens * plain_ms >
// round_ms * 1.03; round 1 after a (re)start is not counted (it pays the
// one-off set-up).
namespace {
void mon_round(cmf_spec_state& s, double dt_ms, int produced) {
    s.n += 1;
    if (s.n == 1) return;
    const double a = s.n == 2 ? 1.0 : 0.3;
    s.round_ms += a * (dt_ms - s.round_ms);
    s.tokens += a * ((double)produced - s.tokens);
}
bool mon_pays(const cmf_spec_state& s) { return s.plain_ms > 0.0 && s.tokens * s.plain_ms > s.round_ms * 1.03; }

// The trial's step after one speculative round (spec_trial_round,
// pipeline.rs:3181-3230): five rounds of a trial, then the plain phase (or,
// with a known plain rate, the decision at once); a decided speculation
// re-checks the rule every round and stops after four losing rounds in a
// row, to be retried 128 tokens later.
void mon_after_round(cmf_spec_state& s, int generated, double now_ms) {
    if (s.phase == CMF_SPEC_TRIAL) {
        s.trial_rounds += 1;
        if (s.trial_rounds >= 5) {
            if (s.plain_ms > 0.0) {
                const bool keep = mon_pays(s);
                s.fails = 0;
                s.phase = keep ? CMF_SPEC_ON : CMF_SPEC_OFF;
                s.recheck_at = keep ? INT_MAX : generated + 128;
            } else {
                s.phase = CMF_SPEC_PLAIN_TRIAL;
                s.t0_ms = now_ms;
                s.gen0 = generated;
            }
        }
    } else if (s.phase == CMF_SPEC_ON) {
        if (mon_pays(s)) {
            s.fails = 0;
        } else if (++s.fails >= 4) {
            s.phase = CMF_SPEC_OFF;
            s.recheck_at = generated + 128;
        }
    }
}
// The per-token part of the trial (pipeline.rs:2655-2689): the plain phase
// ends after 8 tokens with the decision; a decided arm is re-checked at
// recheck_at by a new trial.
void mon_token(cmf_spec_state& s, int generated, double now_ms) {
    if (s.phase == CMF_SPEC_PLAIN_TRIAL && generated >= s.gen0 + 8) {
        s.plain_ms = (now_ms - s.t0_ms) / (double)(generated - s.gen0);
        const bool keep = mon_pays(s);
        s.fails = 0;
        s.phase = keep ? CMF_SPEC_ON : CMF_SPEC_OFF;
        s.recheck_at = keep ? INT_MAX : generated + 128;
    } else if ((s.phase == CMF_SPEC_ON || s.phase == CMF_SPEC_OFF) && generated >= s.recheck_at) {
        s.n = 0;
        s.phase = CMF_SPEC_TRIAL;
        s.trial_rounds = 0;
        s.gen0 = generated;
    }
}
double wall_ms() {
    return std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now().time_since_epoch()).count();
}
}  // namespace

// The reference decode loop (pipeline.rs:2546-2980) over the device rounds:
// emit t_next; a speculative round while generated + 1 < max_tokens, else a
// plain step; the last token is emitted without a forward.  spec = 2 puts
// the rounds under the speculation monitor (SpecMon and its trial,
// pipeline.rs:661-694, 2537, 2655-2760, 3181-3230): speculation stops when
// the measured rounds do not pay and is retried 128 tokens later.
int cmf_decode(cmf_model m, int max_tokens, const cmf_sampler_config* sc, uint64_t seed, int spec,
               int k, int32_t* out, cmf_gen_stats* stats) {
    if (!out || max_tokens < 1 || spec < 0 || spec > 2) return fail("decode: bad arguments");
    int rc = cmf_decode_begin(m, sc, seed);
    if (rc != CMF_OK) return rc;
    hipStream_t s = stream();
    double ms = 0.0;
    cmf_gen_stats st{}, tot{};
    int generated = 0;
    cmf_spec_state& mon = m->mon;
    mon = cmf_spec_state{};
    mon.phase = CMF_SPEC_TRIAL;
    while (true) {
        // a round that ends at or past max_tokens ends the decode (its next
        // token is not emitted: pipeline.rs's loop stops at generated >= max)
        if (generated >= max_tokens) break;
        if (generated + 1 >= max_tokens) {
            hipLaunchKernelGGL(k_emit, dim3(1), dim3(1), 0, s, m->st, m->out);
            CMF_HIP(hipStreamSynchronize(s));
            m->emitted_host += 1;
            generated += 1;
            break;
        }
        if (spec == 2) mon_token(mon, generated, wall_ms());
        const bool off = spec == 2 && (mon.phase == CMF_SPEC_PLAIN_TRIAL || mon.phase == CMF_SPEC_OFF);
        const bool sp = spec && !off && generated + 2 < max_tokens;
        const double t0 = wall_ms();
        rc = cmf_decode_rounds(m, 1, sp ? 1 : 0, k, &st);
        if (rc != CMF_OK) return rc;
        ms += st.device_ms;
        tot.drafted += st.drafted;
        tot.accepted += st.accepted;
        tot.rounds += st.rounds;
        const int produced = m->emitted_host - generated;
        generated = m->emitted_host;
        if (sp) {
            mon.spec_rounds += 1;
            if (spec == 2) {
                const double now = wall_ms();
                mon_round(mon, now - t0, produced);
                mon_after_round(mon, generated, now);
            }
        } else {
            mon.plain_steps += 1;
        }
    }
    const int n = cmf_decode_tokens(m, out, m->emitted_host);
    if (n < 0) return CMF_ERR;
    if (stats) {
        stats->generated = n;
        stats->drafted = tot.drafted;
        stats->accepted = tot.accepted;
        stats->rounds = tot.rounds;
        stats->device_ms = ms;
    }
    m->decoding = false;
    return CMF_OK;
}

int cmf_spec_monitor(cmf_model m, cmf_spec_state* out) {
    if (!m || !out) return fail("spec_monitor: null argument");
    *out = m->mon;
    return CMF_OK;
}

static int forward_batch_impl(cmf_model m, const int32_t* tokens, int b, int pos0, float* hidden, float* logits) {
    if (ready(m)) return CMF_ERR;
    if (!tokens || b < 1 || b > MAXB || pos0 < 0 || pos0 + b > m->c.max_seq)
        return fail("forward_batch: 1 <= b <= 16 and pos0 + b <= max_seq");
    hipStream_t s = stream();
    const int H = m->c.hidden;
    int* pb = &m->st->next_pos;
    CMF_HIP(hipMemcpyAsync(m->toks, tokens, b * sizeof(int), hipMemcpyHostToDevice, s));
    hipLaunchKernelGGL(k_set_int, dim3(1), dim3(1), 0, s, pb, pos0);
    launch_embed(m->toks, embed_src(m), H, m->hv, H, b, s);
    trunk_forward(m, b, pb, 0, pos0 + b, logits != nullptr, s);
    CMF_HIP(hipMemcpyAsync(m->h_tip, m->hv + (size_t)(b - 1) * H, H * sizeof(float), hipMemcpyDeviceToDevice, s));
    if (hidden) CMF_HIP(hipMemcpyAsync(hidden, m->hv, (size_t)b * H * sizeof(float), hipMemcpyDeviceToHost, s));
    if (logits)
        CMF_HIP(hipMemcpyAsync(logits, m->logits, (size_t)b * m->c.vocab * sizeof(float), hipMemcpyDeviceToHost, s));
    hipLaunchKernelGGL(k_set_int, dim3(1), dim3(1), 0, s, pb, pos0 + b);
    CMF_HIP(hipStreamSynchronize(s));
    CMF_HIP(hipGetLastError());
    const int xc = xl_check(m);
    if (xc != CMF_OK) return xc;
    m->next_pos_host = pos0 + b;
    return CMF_OK;
}
// (a call whose XCD-partitioned blocks failed their check runs again on the
// six-launch blocks: its inputs come from the host)
int cmf_forward_batch(cmf_model m, const int32_t* tokens, int b, int pos0, float* hidden, float* logits) {
    const int rc = forward_batch_impl(m, tokens, b, pos0, hidden, logits);
    return rc == XL_RETRY ? forward_batch_impl(m, tokens, b, pos0, hidden, logits) : rc;
}

static int verify_step_impl(cmf_model m, const int32_t* tokens, int b, int pos0, const cmf_sampler_config* sc,
                            const int32_t* q_ids, const float* q_probs, const int32_t* q_n, const float* uniforms,
                            int32_t* argmax_out, float* logits_out, int32_t* accepted, int32_t* next_token) {
    if (ready(m)) return CMF_ERR;
    const int k = b - 1;
    if (!tokens || k < 1 || k > 8 || pos0 < 1 || pos0 + b + 1 > m->c.max_seq)
        return fail("verify_step: 2 <= b <= 9 tokens, 1 <= pos0, pos0 + b < max_seq");
    // the tip hidden is the trunk output at the committed position - 1: the
    // verify runs at that position (positions past it would attend over
    // unwritten KV rows, earlier ones over a stale tip)
    if (!m->prefilled || pos0 != m->next_pos_host)
        return fail("verify_step: pos0 must be the committed position (" + std::to_string(m->next_pos_host) +
                    ", after cmf_prefill / cmf_forward_batch / a decode or verify step)");
    const int V = m->c.vocab, H = m->c.hidden;
    for (int i = 0; i < b; i++)
        if (tokens[i] < 0 || tokens[i] >= V) return fail("verify_step: token id out of range");
    const bool sampling = sc && sc->temperature >= 1e-6f;
    if (sampling) {
        const int rc = check_sampler(m, sc);
        if (rc != CMF_OK) return rc;
        if (!q_ids || !q_probs || !q_n || !uniforms) return fail("verify_step: sampling needs q and uniforms");
        for (int j = 0; j < k; j++)
            if (q_n[j] < 1 || q_n[j] > SPARSE_CAP) return fail("verify_step: q_n[j] must be 1..CMF_SPARSE_CAP");
    }
    if (ensure_out(m, m->c.max_seq + 32)) return CMF_ERR;
    hipStream_t s = stream();
    DState init{};
    init.next_pos = pos0;
    init.t_next = tokens[0];
    init.forced = -1;
    for (int j = 0; j < k; j++) init.drafts[j] = tokens[1 + j];
    CMF_HIP(hipMemcpyAsync(m->st, &init, sizeof(DState), hipMemcpyHostToDevice, s));
    if (sampling) {
        CMF_HIP(hipMemcpyAsync(m->sb.qid, q_ids, (size_t)k * SPARSE_CAP * 4, hipMemcpyHostToDevice, s));
        CMF_HIP(hipMemcpyAsync(m->sb.qp, q_probs, (size_t)k * SPARSE_CAP * 4, hipMemcpyHostToDevice, s));
        CMF_HIP(hipMemcpyAsync(m->sb.qn, q_n, (size_t)k * 4, hipMemcpyHostToDevice, s));
        CMF_HIP(hipMemcpyAsync(m->sb.uni, uniforms, (size_t)b * 4, hipMemcpyHostToDevice, s));
    }
    int* pb = &m->st->next_pos;
    // the MTP row of the first draft, (tip hidden, t_next) at pos0 - 1: what
    // the device draft chain writes before a round
    if (m->has_mtp) mtp_warm(m, &m->st->t_next, m->h_tip, 1, pb, -1, pos0, s);
    launch_embed(m->st->drafts, embed_src(m), H, m->hv, H, b, s, &m->st->t_next);
    trunk_forward(m, b, pb, 0, pos0 + b, true, s);
    if (sampling) {
        sample_rows(m->sb, m->logits, V, b, *sc, m->st, SampleMode::Accept, k, m->out, s, b);
        if (argmax_out) launch_argmax(m->logits, V, V, b, m->am_v, m->am_i, m->st->argmax, s);
    } else {
        const int ns = launch_argmax_part(m->logits, V, V, b, m->am_v, m->am_i, s);
        hipLaunchKernelGGL(k_argmax_accept, dim3(1), dim3(64 * b), 0, s, m->am_v, m->am_i, ns, m->st, k, m->out);
    }
    if (logits_out)
        CMF_HIP(hipMemcpyAsync(logits_out, m->logits, (size_t)b * V * sizeof(float), hipMemcpyDeviceToHost, s));
    if (m->has_mtp) mtp_warm(m, m->st->drafts, m->hv, k, pb, 0, pos0 + b, s);
    hipLaunchKernelGGL(k_commit, dim3(1), dim3(256), 0, s, m->st, m->hv, m->h_tip, H);
    DState hs{};
    CMF_HIP(hipMemcpyAsync(&hs, m->st, sizeof(DState), hipMemcpyDeviceToHost, s));
    CMF_HIP(hipStreamSynchronize(s));
    CMF_HIP(hipGetLastError());
    const int xc = xl_check(m);
    if (xc != CMF_OK) return xc;
    m->next_pos_host = hs.next_pos;
    m->prefilled = true;
    m->decoding = false;
    if (accepted) *accepted = hs.a;
    if (next_token) *next_token = hs.t_next;
    if (argmax_out)
        for (int i = 0; i < b; i++) argmax_out[i] = hs.argmax[i];
    return CMF_OK;
}

// (a call whose XCD-partitioned blocks failed their check runs again on the
// six-launch blocks from the decode state and tip hidden before it)
int cmf_verify_step(cmf_model m, const int32_t* tokens, int b, int pos0, const cmf_sampler_config* sc,
                    const int32_t* q_ids, const float* q_probs, const int32_t* q_n, const float* uniforms,
                    int32_t* argmax_out, float* logits_out, int32_t* accepted, int32_t* next_token) {
    if (!m) return fail("null model");
    XlSnap sn{};
    if (xl_save(m, sn) != CMF_OK) return CMF_ERR;
    int rc = verify_step_impl(m, tokens, b, pos0, sc, q_ids, q_probs, q_n, uniforms, argmax_out, logits_out, accepted,
                              next_token);
    if (rc == XL_RETRY) {
        if (xl_restore(m, sn) != CMF_OK) return CMF_ERR;
        rc = verify_step_impl(m, tokens, b, pos0, sc, q_ids, q_probs, q_n, uniforms, argmax_out, logits_out, accepted,
                              next_token);
    }
    return rc == XL_RETRY ? fail("verify_step: XCD-partitioned blocks failed twice") : rc;
}

int cmf_sparse_distribution(cmf_model m, const float* logits, const cmf_sampler_config* sc, int32_t* ids,
                            float* probs) {
    if (ready(m)) return CMF_ERR;
    if (!logits || !sc || !ids || !probs) return fail("sparse_distribution: null argument");
    if (sc->temperature < 1e-6f) return fail("sparse_distribution: temperature must be > 0");
    const int rc = check_sampler(m, sc);
    if (rc != CMF_OK) return rc;
    hipStream_t s = stream();
    const int V = m->c.vocab;
    int* d_n = m->toks;  // scratch
    CMF_HIP(hipMemcpyAsync(m->logits, logits, (size_t)V * sizeof(float), hipMemcpyHostToDevice, s));
    sample_distribution(m->sb, m->logits, V, *sc, m->sb.rid + MAXB * SPARSE_CAP, m->sb.rv + MAXB * SPARSE_CAP, d_n,
                        s);
    int n = 0;
    CMF_HIP(hipMemcpyAsync(&n, d_n, sizeof(int), hipMemcpyDeviceToHost, s));
    CMF_HIP(hipStreamSynchronize(s));
    if (n < 1 || n > SPARSE_CAP) return fail("sparse_distribution: bad count");
    CMF_HIP(hipMemcpy(ids, m->sb.rid + MAXB * SPARSE_CAP, n * 4, hipMemcpyDeviceToHost));
    CMF_HIP(hipMemcpy(probs, m->sb.rv + MAXB * SPARSE_CAP, n * 4, hipMemcpyDeviceToHost));
    CMF_HIP(hipGetLastError());
    return n;
}

int cmf_kv_truncate(cmf_model m, int n) {
    if (!m || n < 0) return fail("kv_truncate: bad arguments");
    const int np = std::max(0, m->next_pos_host - n);
    hipLaunchKernelGGL(k_set_int, dim3(1), dim3(1), 0, stream(), &m->st->next_pos, np);
    CMF_HIP(hipStreamSynchronize(stream()));
    m->next_pos_host = np;
    return CMF_OK;
}

int cmf_state_get(cmf_model m, int* next_pos, float* hidden) {
    if (!m) return fail("null model");
    if (next_pos) *next_pos = m->next_pos_host;
    if (hidden) CMF_HIP(hipMemcpy(hidden, m->h_tip, m->c.hidden * sizeof(float), hipMemcpyDeviceToHost));
    return CMF_OK;
}

int cmf_kv_export(cmf_model m, int li, int n, float* k, float* v) {
    if (!m || !k || !v || n < 0 || n > m->c.max_seq) return fail("kv_export: bad arguments");
    LayerDev* l = li < 0 ? &m->mtp : (li < m->c.n_layers ? &m->L[li] : nullptr);
    if (!l || !l->kc) return fail("kv_export: no such layer");
    const int hd = m->c.head_dim;
    for (int g = 0; g < m->c.n_kv; g++) {
        CMF_HIP(hipMemcpy(k + (size_t)g * n * hd, l->kc + (size_t)g * m->c.max_seq * hd, (size_t)n * hd * 4,
                          hipMemcpyDeviceToHost));
        CMF_HIP(hipMemcpy(v + (size_t)g * n * hd, l->vc + (size_t)g * m->c.max_seq * hd, (size_t)n * hd * 4,
                          hipMemcpyDeviceToHost));
    }
    return CMF_OK;
}

int cmf_time_attention(cmf_model m, int nb, int pos0, int merge, int iters, float* avg_ms) {
    if (ready(m)) return CMF_ERR;
    const auto& c = m->c;
    if (nb < 1 || nb > MAXB || pos0 < 0 || pos0 + nb > c.max_seq || iters < 1 || !avg_ms)
        return fail("time_attention: 1 <= nb <= 16, pos0 + nb <= max_seq");
    if (c.n_heads / c.n_kv * nb > 32) return fail("time_attention: at most 32 queries per kv head");
    hipStream_t s = stream();
    const int hd = c.head_dim, QKV = (c.n_heads + 2 * c.n_kv) * hd;
    int* pb = m->toks;  // position base (scratch)
    hipLaunchKernelGGL(k_set_int, dim3(1), dim3(1), 0, s, pb, pos0);
    auto one = [&](int i) {
        LayerDev& l = m->L[i % c.n_layers];
        AttnArgs at{m->qkv_out, QKV, l.q_norm, l.k_norm, m->rope, l.kc, l.vc, c.max_seq, nb, c.n_heads, c.n_kv,
                    c.eps, pb, 0, m->pm, m->pl, m->po, m->nch_cap, m->ao, 1};
        launch_attention(at, pos0 + nb, s, merge != 0);
    };
    for (int i = 0; i < 2 * c.n_layers; i++) one(i);
    int rate_khz = 100000;
    (void)hipDeviceGetAttribute(&rate_khz, hipDeviceAttributeWallClockRate, 0);
    hipEvent_t e0, e1;
    CMF_HIP(hipEventCreate(&e0));
    CMF_HIP(hipEventCreate(&e1));
    // captured into a graph, as the decode rounds run
    hipGraph_t g = nullptr;
    hipGraphExec_t ge = nullptr;
    CMF_HIP(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal));
    for (int i = 0; i < iters; i++) one(i);
    CMF_HIP(hipStreamEndCapture(s, &g));
    CMF_HIP(hipGraphInstantiate(&ge, g, nullptr, nullptr, 0));
    CMF_HIP(hipGraphLaunch(ge, s));
    CMF_HIP(hipEventRecord(e0, s));
    CMF_HIP(hipGraphLaunch(ge, s));
    CMF_HIP(hipEventRecord(e1, s));
    CMF_HIP(hipEventSynchronize(e1));
    float ms = 0.f;
    CMF_HIP(hipEventElapsedTime(&ms, e0, e1));
    (void)hipGraphExecDestroy(ge);
    (void)hipGraphDestroy(g);
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    *avg_ms = ms / iters;
    CMF_HIP(hipGetLastError());
    return CMF_OK;
}

}  // extern "C"
