/*
 * libcmfhip — MI355X (gfx950) backend for the cortiq decode hot path.
 *
 * A C ABI shaped like the engine's GPU backend seam
 * (infosave2007/cmf crates/cortiq-engine/src/gpu.rs): plain pointers and
 * sizes, no framework types.  Return convention of every op (gpu.rs:1-12,
 * where `false` means "declined, the caller runs the CPU path"):
 *     0  done                     (CMF_OK)
 *    >0  declined, nothing written (the caller runs its CPU path)
 *    <0  error; cmf_last_error() says why (thread-local, like
 *        cortiq_last_error in crates/cortiq-ffi/include/cortiq.h:6-24)
 * Calls on one handle are serialised by the caller (cortiq.h:3-5).  Each
 * host thread that calls the library gets its own HIP stream and its own
 * seam scratch (created on its first call), so seam ops from several
 * threads run concurrently; a model handle's work runs on the stream of the
 * thread that calls it.
 */
#ifndef CMF_HIP_H
#define CMF_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* TensorDtype ids, cortiq-core/src/types.rs:10-90 */
#define CMF_DT_Q8ROW 3
#define CMF_DT_Q4T 11
#define CMF_DT_Q4TP 15

/* ---- library -------------------------------------------------------- */
/* Thread-local message of the last failing call (cortiq.h:6-24). */
const char* cmf_last_error(void);
/* Select the device and create the calling thread's stream.  Replaces the
 * backend selection of gpu.rs:866-936.  Idempotent. */
int cmf_init(int device);
int cmf_device_count(void);
/* Wait for all work on the calling thread's stream. */
int cmf_sync(void);

/* ---- weights (residency: gpu.rs:507 weight_is_resident) -------------- */
typedef struct cmf_weight_s* cmf_weight;

/* Upload a tensor payload in the reference byte layout (quant.rs):
 *   CMF_DT_Q8ROW: [int8 rows*cols][f16 scale rows]      (quant.rs:4-5)
 *   CMF_DT_Q4T  : rows*cols/32 tiles of [f16 scale][16 B nibbles] (:322)
 *   CMF_DT_Q4TP : [nibbles][row params f16 lo,step][5-bit codes]  (:346-431)
 * The library repacks it once into its device layout. */
int cmf_weight_upload(const uint8_t* payload, size_t nbytes, int dtype, int rows, int cols,
                      cmf_weight* out);
/* q8 in the engine's in-memory form: int8 rows + f32 row_scale
 * (QTensor::from_model q8 arm, qtensor.rs:196-231). */
int cmf_weight_upload_q8(const int8_t* q, const float* row_scale, int rows, int cols,
                         cmf_weight* out);
int cmf_weight_free(cmf_weight w);
size_t cmf_weight_device_bytes(cmf_weight w);

/* ---- seam ops on host slices (gpu.rs) -------------------------------- */
/* gpu.rs:1104 q8_matvec_range: rows [row0, row0+rows) of w times x, each
 * row r scaled by row_scale[r - row0] (the caller's f32 row scales, as the
 * reference passes them with every call; NULL: the scales given at upload). */
int cmf_q8_matvec_range(cmf_weight w, int row0, const float* row_scale, const float* xs, int rows, int cols,
                        float* out);
/* gpu.rs:1155 q8_matmat: out[b*rows + r] with row_scale [rows] (NULL: the
 * upload-time scales), b <= 16 per launch (larger b is split into launches
 * of 16). */
int cmf_q8_matmat(cmf_weight w, const float* row_scale, const float* xs, int b, int rows, int cols, float* out);
/* gpu.rs:2423 / 2439 */
int cmf_q4t_matvec(cmf_weight w, const float* xs, int rows, int cols, float* out);
int cmf_q4t_matmat(cmf_weight w, const float* xs, int b, int rows, int cols, float* out);
/* gpu.rs:2400 / 2358 */
int cmf_q4tp_matvec(cmf_weight w, const float* xs, int rows, int cols, float* out);
int cmf_q4tp_matmat(cmf_weight w, const float* xs, int b, int rows, int cols, float* out);
/* The a8w8 contract of qmatvec / q4t_matvec / q4tp_matvec / their matmats
 * on x86 with VNNI (qtensor.rs:9980-10047, 5683-5717, 4674-4716): each row
 * of xs goes through split_act (qtensor.rs:9237-9281; per-vector int8 scale,
 * |x| > 8 rms kept exactly), integer tile dots, then the outliers; out
 * [b][rows] for any q8 / q4t / q4tp weight, batches of 16 per launch. */
int cmf_matmat_a8w8(cmf_weight w, const float* xs, int b, float* out);
/* gpu.rs:1773 / 1794 q4t_ffn / q4tp_ffn: out = w2 * (silu(w1 x) * (w3 x)),
 * xs [b][hidden], out [b][hidden]. */
int cmf_ffn(cmf_weight w1, cmf_weight w3, cmf_weight w2, const float* xs, int b, int hidden,
            int inter, float* out);

/* MoeJob (gpu.rs:814-841): one expert trio of a caller-routed MoE FFN.
 * gate/up [inter x cols], down [hidden x inter], all three of one codec:
 * q8 (q4t = q4tp = 0; *_row_scale [rows] or NULL = upload-time scales),
 * q4t (q4t = 1) or q4tp (q4tp = 1).  xs_gate / xs_up [cols]: the gate and
 * up inputs; w: the blending weight. */
typedef struct {
    cmf_weight gate, up, down;
    const float *gate_row_scale, *up_row_scale, *down_row_scale;
    const float *xs_gate, *xs_up;
    const float* down_col; /* q8_2f column field of down: no device kernel, must be NULL */
    float w;
    int q1, q4t, q4tp, gu_q2;
    float swiglu_limit;
} cmf_moe_job;
/* moe_block (gpu.rs:2482, wgpu arm gpu_wgpu.rs:28964): out [hidden] =
 * sum over jobs in order of w * down(silu(gate xs_gate) * (up xs_up)).
 * Declined (>0, nothing written) as the reference backends refuse: any q1,
 * gu_q2 (2-bit gate/up), swiglu_limit != 0 or down_col job, jobs of mixed
 * kinds, or a trio whose codec does not match its flags. */
int cmf_moe_block_jobs(const cmf_moe_job* jobs, int njobs, float* out);

/* BatchJob (gpu.rs:843-864): one independent matvec; layout is the
 * BatchLayout as a dtype id (CMF_DT_Q8ROW, CMF_DT_Q4T, CMF_DT_Q4TP; Q1 and
 * anything else is declined). */
typedef struct {
    cmf_weight w;
    int rows, cols;
    const float* row_scale; /* q8: [rows] or NULL (upload-time scales) */
    const float* xs;        /* [cols] */
    int layout;
} cmf_batch_job;
/* matvec_batch (gpu.rs:2494): outs[j] [rows_j] = job j's weight times its
 * xs.  Every job is validated before any runs: a declined job declines the
 * whole batch with nothing written. */
int cmf_matvec_batch(const cmf_batch_job* jobs, int njobs, float* const* outs);

/* ---- device-resident variants (inputs already in HBM) ----------------- */
void* cmf_dev_alloc(size_t bytes);
int cmf_dev_free(void* p);
int cmf_h2d(void* dst, const void* src, size_t bytes);
int cmf_d2h(void* dst, const void* src, size_t bytes);
/* Bytes of the prepared-activation buffer a GEMV on w needs (b <= 16). */
size_t cmf_prep_bytes(cmf_weight w);
/* Prepare x[b][ldx] (device f32) for w: planes (cmf_prep_bytes) + xs[16]. */
int cmf_prep_dev(cmf_weight w, const float* d_x, int ldx, int b, void* d_planes, float* d_xs);
/* y[b][ldy] = w * x from prepared activations; all pointers on the device.
 * ks = waves per workgroup splitting K (0 = heuristic). */
int cmf_gemv_prepared(cmf_weight w, const void* d_planes, const float* d_xs, int b, float* d_y,
                      int ldy, int ks);
/* y[b][ldy] = w * x[b][ldx] on device pointers with no allocation: the
 * operand is prepared into a workspace the library holds in a static device
 * array (1 310 976 B per device, set up by cmf_init), then the GEMV of
 * cmf_gemv_prepared runs on it; the same kernels and results as
 * cmf_prep_dev + cmf_gemv_prepared with a caller workspace.  Weights whose
 * operand needs more (cols > 16384) are rejected with an error.  No
 * counterpart in the reference: for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops).  Requires
 * cmf_init; calls that overlap on one device race on the workspace. */
int cmf_gemv_dev_noalloc(cmf_weight w, const float* d_x, int ldx, int b, float* d_y, int ldy);
/* Average device time (ms) of `iters` back-to-back launches of the GEMV
 * on ws[i % nw] (rotating copies defeat the 256 MB last-level cache),
 * measured with HIP events on the library stream. */
int cmf_time_gemv(const cmf_weight* ws, int nw, const void* d_planes, const float* d_xs, int b,
                  float* d_y, int ldy, int ks, int warmup, int iters, float* avg_ms);
/* Average device time (ms) of `iters` back-to-back GEMVs y[b] = ws[i % nw]
 * x'[b] whose operand x' is produced from device rows d_x [b][ldx] (the
 * layer input): rms_norm(x) * d_norm_w when d_norm_w is not NULL (eps
 * 1e-6), else the rows themselves.  fused = 1: every GEMV workgroup
 * evaluates the producer itself (fails when that path does not apply);
 * fused = 0: a producer launch before each GEMV.  No counterpart in the
 * reference: a measurement helper for the decode layer's operand paths. */
int cmf_time_gemv_rows(const cmf_weight* ws, int nw, const float* d_x, int ldx, const float* d_norm_w, int b,
                       float* d_y, int ldy, int fused, int warmup, int iters, float* avg_ms);
/* Average device time (ms) of `iters` large-batch GEMMs y[m][rows] = w x
 * (q4t / q4tp; operand preparation included), x [m][cols] and y on the
 * device.  No counterpart in the reference: a measurement helper. */
int cmf_time_gemm(cmf_weight w, const float* d_x, int m, float* d_y, int warmup, int iters, float* avg_ms);
/* Average device time (ms) of `iters` launches of a plain device copy of
 * `bytes` (16-byte vector loads and stores, a fresh source buffer each
 * launch from `nbuf` rotating ones).  No counterpart in the reference: a
 * measurement helper, the known-size kernel against which HBM traffic
 * counters (FETCH_SIZE / WRITE_SIZE) are calibrated. */
int cmf_time_copy(size_t bytes, int nbuf, int iters, float* avg_ms);
/* Diagnostic: average time of a plain read of `bytes` (a multiple of 32 KiB)
 * in the M = 1 GEMV's launch shape (workgroups of 8 waves x 4 KiB), nbuf
 * buffers rotated: the ceiling a GEMV streaming that many bytes can reach. */
int cmf_time_read(size_t bytes, int nbuf, int iters, float* avg_ms);

/* ---- model: Qwen3-arch decoder + MTP head (pipeline.rs) --------------- */
typedef struct cmf_model_s* cmf_model;
typedef struct cmf_moe_s* cmf_moe;

typedef struct {
    int n_layers, hidden, n_heads, n_kv, head_dim, inter, vocab, max_seq;
    float rope_theta;
    double eps;
} cmf_model_config;

/* A quantized tensor as the engine holds it (QTensor): q8 as int8 rows +
 * f32 row_scale, q4t / q4tp as their quant.rs payloads. */
typedef struct {
    int dtype, rows, cols;
    const int8_t* q;
    const float* row_scale;
    const uint8_t* bytes;
} cmf_tensor;

/* One decoder block (LayerWeights, AttnKind::Full + dense SwiGLU FFN). */
typedef struct {
    const float *input_norm, *post_norm, *q_norm, *k_norm;
    cmf_tensor wq, wk, wv, wo, gate, up, down;
} cmf_layer_desc;

int cmf_model_create(const cmf_model_config* cfg, cmf_model* out);
int cmf_model_free(cmf_model m);
int cmf_model_set_layer(cmf_model m, int li, const cmf_layer_desc* d);
/* A decoder block whose FFN is routed experts (FfnKind::Moe / GraphFfn::Moe,
 * pipeline.rs:434-470, gpu.rs:1248-1361; Qwen3-MoE): d supplies the norms
 * and attention weights (its gate/up/down are not read), router [n_experts x
 * hidden] scores the block's normed rows (q8 / q4t / q4tp, or a dense router
 * as the reference's converter stores it: dtype 0 f32, 1 f16, 2 bf16 in
 * bytes, widened to f32 on upload), and moe (created
 * with cmf_moe_create, experts set; hidden equal to the model's) runs
 * moe_route + the experts; h += their weighted sum.  The model borrows moe:
 * free it after the model. */
int cmf_model_set_layer_moe(cmf_model m, int li, const cmf_layer_desc* d, const cmf_tensor* router, cmf_moe moe);
/* lm_head (q8) doubles as the tied embedding table; final_norm [hidden]. */
int cmf_model_set_head(cmf_model m, const cmf_tensor* lm_head, const float* final_norm);
/* MtpModule (pipeline.rs:600-612). */
int cmf_model_set_mtp(cmf_model m, const float* enorm, const float* hnorm, const cmf_tensor* eh_proj,
                      const cmf_layer_desc* layer, const float* norm);
/* 1 when the model's dense decoder blocks run as the XCD-partitioned pair of
 * launches (MI355X with 256 CUs, hidden 1024, inter 3072, 16 query / 8 KV
 * heads of 128, q8 attention and q4t FFN weights, batches of up to 16 rows;
 * environment CMF_XL=0 at model creation turns it off), 0 when they run as
 * six launches per block.  No counterpart in the reference (a backend
 * property, not a seam). */
int cmf_model_fused_blocks(cmf_model m);
/* No reference counterpart: 1 while the model's prefill attention may run
 * the XCD-placed variant (one kv head per XCD, MI355X with 8 kv heads), 0
 * after its placement check failed once (the prefill was then re-run on the
 * grid-indexed variant, which the model keeps). */
int cmf_model_prefill_xcd(cmf_model m);
/* No reference counterpart: how many calls of the model were run again on
 * the six-launch blocks because its XCD-partitioned blocks failed their
 * check (an exchange wait gave up, a position bound was exceeded, or two
 * workgroups of a launch ran on one XCD slot); after the first, the model
 * keeps the six-launch blocks (cmf_model_fused_blocks then reports 0). */
int cmf_model_xl_fallbacks(cmf_model m);

/* ---- MoE FFN (moe_ffn / moe_block) ------------------------------------ */

/* A routed-expert FFN layer (MoeFfn, pipeline.rs:10868-11045): n_experts
 * SwiGLU experts gate/up [inter x hidden], down [hidden x inter], softmax
 * router, top_k experts per token, norm_topk_prob and routed_scaling as
 * moe_route (pipeline.rs:10780-10841).  No shared expert, expert bias, mask
 * or tau trimming (the Qwen3-MoE configuration). */
int cmf_moe_create(int n_experts, int hidden, int inter, int top_k, int norm_topk, float routed_scaling,
                   cmf_moe* out);
int cmf_moe_free(cmf_moe m);
/* Upload expert e (quant.rs layouts; q8, q4t or q4tp; every expert with the
 * same codecs).  >0 (declined) for a codec without a device kernel. */
int cmf_moe_set_expert(cmf_moe m, int e, const cmf_tensor* gate, const cmf_tensor* up, const cmf_tensor* down);
/* moe_ffn for a verify batch of b <= 16 tokens: route router_logits [b][ne],
 * run every (token, expert) pair grouped by expert, out [b][hidden] =
 * sum over the token's experts, in routing order, of w * expert(x).  Host
 * pointers; idx_out / w_out [b][top_k] (nullable) receive the routing. */
int cmf_moe_ffn(cmf_moe m, const float* x, const float* router_logits, int b, float* out, int32_t* idx_out,
                float* w_out);
/* The same on device pointers (inputs resident in HBM). */
int cmf_moe_ffn_dev(cmf_moe m, const float* d_x, const float* d_logits, int b, float* d_out);
/* Average device time (ms, HIP events on the library stream) of `iters`
 * cmf_moe_ffn_dev calls after `warmup` ones.  No counterpart in the
 * reference: a measurement helper. */
int cmf_time_moe(cmf_moe m, const float* d_x, const float* d_logits, int b, float* d_out, int warmup, int iters,
                 float* avg_ms);
/* moe_block (gpu.rs:2482): one token x [hidden], the caller's routing
 * (experts[njobs], weights[njobs], njobs <= top_k) -> out [hidden]. */
int cmf_moe_block(cmf_moe m, const float* x, const int32_t* experts, const float* weights, int njobs, float* out);

/* SamplerConfig (sampler.rs:88-121).  Penalised configs are declined by the
 * device sampler (speculation is gated off under penalties,
 * pipeline.rs:2035-2037). */
typedef struct {
    float temperature, top_p;
    uint32_t top_k;
    float repetition_penalty, min_p, presence_penalty;
} cmf_sampler_config;

/* generated: tokens emitted since cmf_decode_begin; drafted, accepted,
 * rounds and device_ms: of this call. */
typedef struct {
    int generated, drafted, accepted, rounds;
    double device_ms;
} cmf_gen_stats;

/* Prefill ids at positions 0..n-1 (trunk KV + MTP warm on the (h_p,
 * id_{p+1}) pairs, pipeline.rs:2275-2318) and reset the decode state. */
int cmf_prefill(cmf_model m, const int32_t* ids, int n);
/* Decode after cmf_prefill: samples the first token from the prefill's last
 * hidden, then runs graph_spec_step rounds (spec=1, k drafts,
 * pipeline.rs:3582-4213) or plain tokens (spec=0) until at least max_tokens
 * are produced.  out: capacity max_tokens + k + 1.  Returns via stats. */
int cmf_decode(cmf_model m, int max_tokens, const cmf_sampler_config* sc, uint64_t seed, int spec,
               int k, int32_t* out, cmf_gen_stats* st);
/* spec = 2: the rounds run under the speculation monitor (SpecMon,
 * pipeline.rs:661-694, and its trial, :2537, :2655-2760, :3181-3230): five
 * timed speculative rounds, eight timed plain tokens, then the faster arm;
 * a speculating decode re-checks tokens_per_round * plain_ms > round_ms *
 * 1.03 every round and stops after four losing rounds, and a stopped one is
 * retried 128 tokens later.  Times are host wall times, as the reference's.
 * cmf_spec_monitor reads the monitor of the model's last cmf_decode. */
enum { CMF_SPEC_TRIAL = 0, CMF_SPEC_PLAIN_TRIAL = 1, CMF_SPEC_ON = 2, CMF_SPEC_OFF = 3 };
typedef struct {
    double round_ms, tokens, plain_ms; /* SpecMon's averages (pipeline.rs:672-677) */
    int n, fails;                      /* rounds counted since the trial began; losing rounds in a row */
    int phase;                         /* CMF_SPEC_*: the SpecTrial phase (pipeline.rs:642-660) */
    int trial_rounds, gen0, recheck_at;
    double t0_ms;                      /* start of the plain phase (host wall clock) */
    int spec_rounds, plain_steps;      /* what the decode ran */
} cmf_spec_state;
int cmf_spec_monitor(cmf_model m, cmf_spec_state* out);
/* The same loop in pieces, for callers that pace it themselves:
 * begin (reset the emitted stream, sample the first token from the tip),
 * exactly n speculative rounds (spec=1) or plain steps (spec=0) with no
 * end-of-generation gating, and a copy of the emitted tokens (returns the
 * count).  device_ms in stats is the device time of that call. */
int cmf_decode_begin(cmf_model m, const cmf_sampler_config* sc, uint64_t seed);
int cmf_decode_rounds(cmf_model m, int n, int spec, int k, cmf_gen_stats* st);
int cmf_decode_tokens(cmf_model m, int32_t* out, int cap);
/* forward_batch_graph counterpart (gpu.rs:1466-1497): run b tokens at
 * positions pos0.. through the trunk (appending KV), write final hidden rows
 * [b][hidden] and logits [b][vocab] (either may be NULL). */
int cmf_forward_batch(cmf_model m, const int32_t* tokens, int b, int pos0, float* hidden,
                      float* logits);
/* Largest top_k the device sampler serves. */
#define CMF_SPARSE_K_MAX 64
/* Capacity of a sparse distribution list: par_topk keeps the top k and every
 * entry tied with the k-th value, at most 4 k + 64 (sampler.rs:515-600). */
#define CMF_SPARSE_CAP (4 * CMF_SPARSE_K_MAX + 64)

/* One verify step of graph_spec_step with the caller's drafts: the
 * forward_batch_graph + SpecTail verify (gpu.rs:1455-1497) and the
 * acceptance, commit and rollback that follow it (pipeline.rs:3885-4176,
 * kv_cache.rs:883).  tokens [b] = [t_next, d_0 .. d_{b-2}] (2 <= b <= 9) at
 * positions pos0 .. where pos0 is the committed position (the decode state's
 * tip hidden is the trunk output at pos0 - 1: after cmf_prefill,
 * cmf_forward_batch, a decode round or a previous verify step); another
 * pos0 is an error.
 *   greedy (sc NULL or temperature < 1e-6): a = the longest prefix with
 *     argmax(row i) == d_i (ties to the highest id); *next_token =
 *     argmax(row a);
 *   sampled: spec_accept_or_correct_sparse (sampler.rs:683-711) of each
 *     draft against the caller's draft distributions q_ids / q_probs
 *     [b-1][CMF_SPARSE_CAP] (ids ascending, q_n[j] entries) and the
 *     row's sparse distribution p; the uniforms [b] are consumed in the
 *     reference's order (one per tested draft, one for the correction or
 *     for the draw from row a); *next_token = the correction or that draw.
 * Commit: trunk KV holds positions [0, pos0 + a + 1), the tip hidden is row
 * a, and with an MTP head its cache holds the pairs (tip, t_next) at
 * pos0 - 1 and (row j, d_j) at pos0 + j for j < a (rows past that are
 * scratch for the next round).  argmax_out [b] (picks of every row) and
 * logits_out [b][vocab] may be NULL. */
int cmf_verify_step(cmf_model m, const int32_t* tokens, int b, int pos0, const cmf_sampler_config* sc,
                    const int32_t* q_ids, const float* q_probs, const int32_t* q_n, const float* uniforms,
                    int32_t* argmax_out, float* logits_out, int32_t* accepted, int32_t* next_token);
/* sparse_distribution_into (sampler.rs:440-514) of one logits row [vocab]
 * (host) on the device sampler: ids ascending and their probabilities
 * (capacity CMF_SPARSE_CAP); returns the count (>= 1: a fully filtered
 * row gives its argmax with probability 1, as the decode loop does). */
int cmf_sparse_distribution(cmf_model m, const float* logits, const cmf_sampler_config* sc, int32_t* ids,
                            float* probs);
/* KV rollback (kv_cache.rs:883 truncate_last / gpu.rs:1514 graph_kv_reset):
 * the decode position moves back by n. */
int cmf_kv_truncate(cmf_model m, int n);
/* Decode state after cmf_prefill / cmf_decode: next position, the tip
 * hidden [hidden] (trunk output at next_pos-1). */
int cmf_state_get(cmf_model m, int* next_pos, float* hidden);
/* Copy KV rows [0, n) of layer li (li == -1: the MTP block) into
 * k/v [n_kv][n][head_dim]. */
int cmf_kv_export(cmf_model m, int li, int n, float* k, float* v);

/* Average device time (ms) of the decode attention of nb rows at positions
 * pos0 .. pos0+nb-1 (qk-norm, RoPE, KV append, causal attention over the
 * cache; merge = 0 leaves out the merge of the chunk partials), rotating
 * over the layers of model m, `iters` launches captured in a HIP graph.
 * Writes the KV rows at those positions.  No counterpart in the reference:
 * a measurement helper. */
int cmf_time_attention(cmf_model m, int nb, int pos0, int merge, int iters, float* avg_ms);


/* ---- .cmf v2 container (cortiq-core/src/format.rs) ------------------- */
/* Error kinds of the container calls (CmfError, format.rs; the message of
 * cmf_last_error() carries the details). */
#define CMF_E_NOTFOUND (-2) /* FileNotFound */
#define CMF_E_MAGIC (-3)    /* InvalidMagic */
#define CMF_E_VERSION (-4)  /* UnsupportedVersion */
#define CMF_E_FEATURE (-5)  /* UnsupportedFeature */
#define CMF_E_BOUNDS (-6)   /* Bounds */
#define CMF_E_PARSE (-7)    /* Parse */
#define CMF_E_DTYPE (-8)    /* UnknownDtype */
#define CMF_E_IO (-9)       /* Io */
#define CMF_E_MISSING (-10) /* MissingTensor */

typedef struct CmfFileS* cmf_file;

/* Envelope of an open file: sections header, dir, data, masks, vocab,
 * index (offset, length; length 0 = absent), the stored header / directory
 * hashes (0 = absent) and the mapping's base address and length. */
typedef struct {
    uint32_t required_features;
    uint64_t off[6], len[6];
    uint64_t header_hash, dir_hash;
    const uint8_t* base;
    uint64_t file_len;
} cmf_file_sections;

/* One tensor directory record (TensorEntry, format.rs:255-269).  name is
 * not NUL-terminated; data points into the read-only mapping of the owning
 * shard (entry_bytes, format.rs:924-933) and lives until cmf_file_close. */
typedef struct {
    const char* name;
    int name_len;
    int dtype;
    int ndim;
    uint64_t shape[6];
    uint64_t off, nbytes, hash;
    int shard;
    const uint8_t* data;
} cmf_file_tensor;

/* hash64 (cortiq-core/src/hash.rs:18-35): murmur3 fmix64 over 64-bit LE
 * words with positional salt, XOR fold, length mix. */
uint64_t cmf_hash64(const void* data, size_t n);
/* CmfModel::open (format.rs:390-584): maps the file read-only and validates
 * the envelope (magic, version 2, required feature bits, section bounds,
 * 4096-aligned data), the header's JSON syntax, the directory (56-byte
 * records, name pool, UTF-8 names, known dtype ids, ndim <= 6) and every
 * tensor (64-aligned offset, inside the data section, shape product,
 * expected_nbytes of fixed-size dtypes, no duplicate names).  The header's
 * fields are read by the caller from the header section. */
int cmf_file_open(const char* path, cmf_file* out);
int cmf_file_close(cmf_file f);
int cmf_file_info(cmf_file f, cmf_file_sections* s);
int cmf_file_count(cmf_file f);
int cmf_file_entry(cmf_file f, int i, cmf_file_tensor* e);
/* tensor_index (format.rs:809-821): directory index of a tensor by name, or
 * CMF_E_MISSING. */
int cmf_file_find(cmf_file f, const char* name, size_t name_len);
/* The directory-merge step of open_sharded (format.rs:589-650): appends the
 * tensors of an opened sibling shard to f (entry.shard = 1, 2, ... in call
 * order) and takes over its mapping; shard is consumed on success.  A name
 * already present is CMF_E_PARSE and leaves both files unchanged.  The
 * caller checks the shard coordinates of the sibling's header. */
int cmf_file_attach_shard(cmf_file f, cmf_file shard);
/* verify (format.rs:1063-1110): the envelope's header and directory hashes,
 * the optional sections' hashes stored[0..2] = masks, vocab, index (0 or a
 * NULL array: not checked; they are read from the header's section_hashes
 * by the caller) and every tensor's hash.  *nproblems = count; the messages,
 * one per line, go to buf (truncated to cap). */
int cmf_file_verify(cmf_file f, const uint64_t* stored, char* buf, size_t cap, int* nproblems);
/* A model whose embedding table is not tied to lm_head (loader.rs:714-724):
 * q8 [vocab][hidden], read row by row by the embedding lookups.  Without
 * this call the lm_head doubles as the embedding table. */
int cmf_model_set_embed(cmf_model m, const cmf_tensor* embed);

#ifdef __cplusplus
}
#endif
#endif
