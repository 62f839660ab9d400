/*
 * CPU oracle for the cortiq decode hot path — TEST INFRASTRUCTURE ONLY.
 *
 * This is a plain-C restatement of the reference's CPU path (the Rust crates
 * cortiq-core and cortiq-engine of infosave2007/cmf, which cannot be built
 * here: no Rust toolchain).  Every function cites the reference file:line it
 * follows.  Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
 * leg may load it, and only as the checker or the timed CPU baseline; the
 * product (cmf_amd/) never links or calls it.
 *
 * Numerics contract: the reference's "exact" contract (CMF_SDOT=0): f32
 * activations times dequantized weights with f32 accumulation in the
 * reference's own summation order.  The a8w8 contract (split_act + integer
 * tile dots) is restated for the single-row kernels.
 *
 * Parity pinning (what checks each part; see tests/test_oracle_*.py):
 *   f16 conversion      known answers of quant.rs:872-891 + exhaustive
 *                       round trip over all 65536 halves
 *   q8/q4t/q4tp dequant closed form on hand-built tiles; q4tp(step=0) ==
 *                       q4t with the same scale; golden fixtures
 *   exact matvecs       brute force f64 dot of the dequantized matrix,
 *                       |err| <= 1e-5 * sum|w*x| (qtensor.rs:10702-10733)
 *   a8w8 matvecs        integer dot brute-forced in int64, error bound
 *                       rel-L2 < 0.05 vs exact (qtensor.rs:10446-10481)
 *   SplitMix64          Vigna's published outputs for seeds 0 and 42
 *   argmax              tie rule of sampler.rs:1130-1154
 *   sparse chain        brute-force dense chain on small vocabularies
 *   spec acceptance     empirical L1 < 0.01 over 4e5 trials
 *                       (sampler.rs:1285-1337)
 *   model forward       spec(greedy) == vanilla greedy
 *                       (pipeline.rs:11543-11564); attention vs numpy
 *                       softmax attention; KV rows enter exactly once
 * Parity unpinned (no reference output exists to check against here):
 *   bit patterns of Rust std exp2f/expf/sin_cos/powf (glibc is used), and
 *   the pool-grain summation order of the sparse chain's denominator
 *   (sampler.rs:626-656; the serial order is used).
 */
#ifndef CMF_ORACLE_H
#define CMF_ORACLE_H

#include <stddef.h>
#include <stdint.h>

/* Hot oracle loops are built twice: for hosts with FMA/AVX2 and for any
 * x86-64 host, picked at load time.  Both clones perform the same float
 * operations in the same order (-ffp-contract=off, no fast-math). */
#if defined(__x86_64__) && defined(__GNUC__) && !defined(__clang__)
#define CLONES __attribute__((target_clones("fma", "default")))
#else
#define CLONES
#endif

#ifdef __cplusplus
extern "C" {
#endif

/* TensorDtype ids, cortiq-core/src/types.rs:10-90 */
enum { OR_F32 = 0, OR_Q8ROW = 3, OR_Q4T = 11, OR_Q4TP = 15 };

/* ---- quant.rs ---------------------------------------------------------- */
float or_f16_to_f32(uint16_t h);
uint16_t or_f32_to_f16(float x);
void or_dequant_q8_row(const uint8_t* bytes, int rows, int cols, float* dst);
void or_dequant_q4t(const uint8_t* bytes, size_t n, float* dst);
size_t or_q4tp_code_stride(size_t gpr);
void or_q4tp_sections(size_t rows, size_t cols, size_t* params_off, size_t* codes_off,
                      size_t* stride);
int or_q4tp_code(const uint8_t* codes, size_t stride, size_t g);
void or_q4tp_put_code(uint8_t* codes, size_t g, int code);
void or_q4tp_ladder(const uint8_t* params, size_t r, float* t32);
void or_dequant_q4tp(const uint8_t* bytes, int rows, int cols, float* dst);

/* ---- a quantized tensor as the engine holds it (QTensor) -------------- */
typedef struct {
    int dtype;               /* OR_Q8ROW / OR_Q4T / OR_Q4TP */
    int rows, cols;
    const int8_t* q;         /* q8: [rows*cols] */
    const float* row_scale;  /* q8: f32 per row (qtensor.rs:196-231) */
    const uint8_t* bytes;    /* q4t / q4tp payload in the quant.rs layout; F32: rows*cols floats
                              * (an f16 / bf16 file tensor converted at load, as load_matrix does,
                              * loader.rs:~510) */
} or_qt;

/* exact contract, qtensor.rs:9980-10047 / 5683-5717 / 4674-4716 */
void or_matvec(const or_qt* w, const float* x, float* out, int threads);
/* exact contract batch: out[b*rows + r], qtensor.rs:5950-5959 / 5668-5679 */
void or_matmat(const or_qt* w, const float* xs, int b, float* out, int threads);
/* a8w8 contract (split_act + integer tile dots), qtensor.rs:9237-9281,
 * 4106-4130, 4405-4413, 4517-4544, 4666-4671, 8921-8933 */
void or_matvec_a8w8(const or_qt* w, const float* x, float* out, int threads);
/* a8w8 batch (qmatmat / q4t_matmat / q4tp_matmat x86 VNNI arms): out[b*rows + r] */
void or_matmat_a8w8(const or_qt* w, const float* xs, int b, float* out, int threads);
/* fast.c, the timing arm: the same values as or_matmat_a8w8 by AVX-512 VNNI
 * intrinsics; -1 on a host without AVX-512 VNNI */
int or_fast_supported(void);
int or_fast_matmat_a8w8(const or_qt* w, const float* xs, int b, float* out, int threads);
/* split_act as a plain function (qtensor.rs:9237-9281).  xq: [n];
 * outl_idx/outl_val: capacity n.  Returns the outlier count. */
int or_split_act(const float* x, int n, int8_t* xq, float* sx, int* outl_idx, float* outl_val,
                 int32_t* xsum);

/* ---- inference.rs / attention.rs -------------------------------------- */
float or_silu(float x);
void or_rms_norm(const float* x, const float* w, int n, double eps, float* out);
void or_rope_inv_freq(int head_dim, float theta, float* out);

/* ---- sampler.rs ------------------------------------------------------- */
/* SplitMix64 state.  seq != NULL replaces the stream's uniforms: next_f32
 * returns seq[used++] (the caller's shared uniforms of a verify step) and
 * falls back to the generator once nseq are used. */
typedef struct {
    uint64_t state;
    const float* seq;
    int nseq, used;
} or_rng;
uint64_t or_rng_next_u64(or_rng* r);
float or_rng_next_f32(or_rng* r);
uint32_t or_argmax(const float* v, int n);

typedef struct {
    float temperature, top_p;
    uint32_t top_k;
    float repetition_penalty, min_p, presence_penalty;
} or_sampler_cfg;

/* sparse distribution: ids ascending, probs sum to 1.  Returns count (0 =
 * filtered everything).  sampler.rs:440-514 (serial par_topk/par_sum_exp) */
int or_sparse_distribution(const float* logits, int n, const or_sampler_cfg* cfg,
                           const uint32_t* past, int npast, uint32_t* ids, float* probs);
uint32_t or_draw_sparse(const uint32_t* ids, const float* probs, int n, or_rng* rng);
/* returns -1 = accepted, else the correction token; sampler.rs:683-711 */
int64_t or_spec_accept_sparse(const uint32_t* pid, const float* pp, int np, const uint32_t* qid,
                              const float* qp, int nq, uint32_t d, or_rng* rng);
/* dense: sampler.rs:771-819 (p, q normalised over n) */
int64_t or_spec_accept_dense(const float* p, const float* q, int n, uint32_t d, or_rng* rng);
uint32_t or_categorical(const float* probs, int n, float r);
/* sample_with_scratch_pool, sampler.rs:161-212 */
uint32_t or_sample(const float* logits, int n, const or_sampler_cfg* cfg, const uint32_t* past,
                   int npast, or_rng* rng);

/* ---- the Qwen3-arch model --------------------------------------------- */
typedef struct {
    int n_layers, hidden, n_heads, n_kv, head_dim, inter, vocab, max_seq;
    float rope_theta;
    double eps;
} or_cfg;

/* One decoder block.  n_experts > 0: the FFN is a routed MoE (MoeFfn,
 * pipeline.rs:434-470; Qwen3-MoE: softmax router, no shared expert):
 * logits = router * rms_norm(h), moe_route + moe_ffn_cpu
 * (pipeline.rs:10780-10841, 11017-11030), experts [n_experts][3] =
 * gate, up, down; gate/up/down of the layer itself are unused. */
typedef struct {
    const float *input_norm, *post_norm, *q_norm, *k_norm;
    or_qt wq, wk, wv, wo, gate, up, down;
    int n_experts, top_k, norm_topk;
    float routed_scaling;
    or_qt router;
    const or_qt* experts;
} or_layer;

typedef struct {
    or_cfg cfg;
    const or_layer* layers; /* n_layers */
    or_qt lm_head;          /* q8, tied embedding: embed row = q8 row dequant */
    const float* final_norm;
    int has_mtp;
    const float *enorm, *hnorm, *mtp_norm;
    or_qt eh_proj;          /* [hidden, 2*hidden] */
    or_layer mtp;
    int threads;
    or_qt embed;            /* untied q8 embedding table (loader.rs:714-724); q == NULL: lm_head */
    int a8w8;               /* 1: the quantized matvecs of the forward under the a8w8 contract */
    int fast;               /* 1: a8w8 matmuls through the AVX-512 VNNI timing arm (same values) */
    int batch_verify;       /* 1: the verify rows of a spec round as one batch (or_forward_rows) */
} or_model;

/* KV: per layer k[n_kv][max_seq][head_dim], same for v; len = stored rows.
 * kv_cache.rs:83-132 (head-major f32). */
typedef struct {
    float* k;
    float* v;
    int len;
} or_kv;

typedef struct {
    or_kv* trunk;   /* n_layers */
    or_kv mtp;
    float* inv_freq;
} or_state;

void or_embed(const or_model* m, uint32_t id, float* out);
/* forward_layers (pipeline.rs:5851, 7981-8700): h in/out */
void or_forward(const or_model* m, or_state* s, float* h, int pos);
/* forward_batch over positions pos0 .. pos0+b-1, h: [b][hidden] in/out */
void or_forward_rows(const or_model* m, or_state* s, float* h, int b, int pos0);
/* final norm + lm_head (pipeline.rs:5919, 8771) */
void or_logits(const or_model* m, const float* h, float* logits);
/* mtp_step_hl (pipeline.rs:3051-3160): logits (may be NULL -> warm only,
 * mtp_warm pipeline.rs:3532) and the block output hidden */
void or_mtp_step(const or_model* m, or_state* s, const float* hidden, uint32_t tok, int pos,
                 float* logits, float* h_out);

typedef struct {
    int spec;            /* 1 = graph_spec_step rounds, 0 = vanilla */
    int k;               /* drafts per round */
    or_sampler_cfg sc;
    uint64_t seed;
} or_gen_cfg;

typedef struct {
    int drafted, accepted, rounds;
    int hist[17]; /* rounds by accepted count a = 0..16 */
} or_gen_stats;

/* generate_from_ids restated (pipeline.rs:1913-2980 with the decode loop at
 * 2546-2980 and graph_spec_step at 3582-4213).  Prefill runs per position.
 * out must hold max_tokens + k entries; returns generated count. */
int or_generate(const or_model* m, or_state* s, const uint32_t* prompt, int np, int max_tokens,
                const or_gen_cfg* g, uint32_t* out, or_gen_stats* st);

/* Continue a decode from an imported state: `hidden` = trunk output at
 * next_pos-1 (the caller's KV already holds positions < next_pos and the MTP
 * KV positions < next_pos-1), all_ids = committed stream.  Runs until
 * max_tokens more are generated.  rng_state in/out. */
int or_decode(const or_model* m, or_state* s, float* hidden, int next_pos, const uint32_t* ids,
              int nids, int max_tokens, const or_gen_cfg* g, uint64_t* rng_state, uint32_t* out,
              or_gen_stats* st);

/* One verify step of graph_spec_step with caller drafts (pipeline.rs:
 * 3768-4176): rows tokens[0..b) = [t_next, d_0 .. d_{b-2}] at positions
 * pos0.. through the trunk (KV appended), acceptance (greedy argmax
 * equality, or spec_accept_or_correct_sparse against the caller's draft
 * distributions q_ids/q_p/q_n [b-1][q_stride] with rng's uniforms), the
 * trunk KV cut to pos0 + a + 1 and, with an MTP head, the MTP rows
 * (hidden, t_next) at pos0 - 1 (warm_tip = 1: the caller drafted
 * elsewhere; 0: the draft chain wrote it) and the accepted pairs.
 * hidden: in = trunk output at pos0 - 1, out = row a.  past/npast: the
 * committed stream (t_next included).  logits (b*vocab) and argmax (b)
 * may be NULL.  *next = the token after the accepted ones (correction,
 * or the pick of row a).  Returns a. */
int or_verify_step(const or_model* m, or_state* s, float* hidden, int pos0, const uint32_t* tokens, int b,
                   const or_sampler_cfg* sc, const uint32_t* q_ids, const float* q_p, const int* q_n,
                   int q_stride, or_rng* rng, const uint32_t* past, int npast, int warm_tip, float* logits,
                   uint32_t* argmax, uint32_t* next);

/* MoE routing + expert FFN for one token (pipeline.rs:10780-10841,
 * 10868-11045). experts: 3*ne tensors (gate, up, down per expert). */
int or_moe_route(const float* logits, int ne, int top_k, int norm_topk, float routed_scaling,
                 int* idx, float* w);
void or_moe_ffn(const or_qt* experts, int ne, int top_k, int norm_topk, float routed_scaling,
                const float* router_logits, const float* x, int hidden, float* out, int threads);

#ifdef __cplusplus
}
#endif
#endif
