// Device-side decode state and the sparse sampling chain + speculative
// acceptance (sampler.rs:440-514, 661-711) run on the GPU.
#pragma once

#include <functional>

#include "../../include/cmf_hip.h"
#include "common.h"

namespace cmf {

constexpr int SPARSE_K_MAX = 64;  // largest top_k the device sampler serves
// par_topk keeps the top-k and every entry tied with the k-th value, at most
// 4 k + 64 of them (sampler.rs:515-600): the candidate lists hold that many
constexpr int SPARSE_CAP = 4 * SPARSE_K_MAX + 64;
static_assert(SPARSE_CAP % 64 == 0, "candidate lists are whole waves");
constexpr int SLICE = 4096;       // logits per selection block

// Decode state kept in HBM; kernels read positions from it so a round needs
// no host values.
struct DState {
    int next_pos;        // next trunk position (trunk KV holds [0, next_pos))
    int a;               // accepted drafts of the last round
    int t_next;          // token to emit next
    int t_new;           // token picked by the last accept / plain pick
    int n_out;           // tokens emitted
    int accepted;        // total accepted drafts
    int forced;          // correction token of the last round, -1 if none
    int pad;
    unsigned long long rng;  // SplitMix64 state (sampler.rs:54-84)
    int drafts[16];
    int argmax[17];
};

enum class SampleMode { Draft, Plain, Accept };

struct SampleBufs {
    int V = 0, nslices = 0;
    int* cid = nullptr;     // [rows][nslices][K_MAX] the slices' top-k, value desc / id asc
    float* cv = nullptr;
    int* ocnt = nullptr;    // [rows][nslices] ties at the slice's k-th value past its list
    int* oid = nullptr;     // [rows][nslices][SPARSE_CAP] their ids, index order
    float* smax = nullptr;  // [rows][nslices]
    float* ssum = nullptr;
    int* rid = nullptr;     // [rows][SPARSE_CAP] merged candidates, value desc / id asc
    float* rv = nullptr;
    int* rn = nullptr;      // [rows] their count
    float* lmax = nullptr;  // [rows]
    float* sum = nullptr;   // [rows]
    int* qid = nullptr;     // draft distributions [8][SPARSE_CAP]
    float* qp = nullptr;
    int* qn = nullptr;      // [8]
    float* uni = nullptr;   // caller uniforms of a verify step [MAXB + 1]
};

int sample_alloc(SampleBufs& b, int V, const std::function<int(void**, size_t)>& alloc);

// Selection + the sparse chain for `rows` logit rows (ld = V), then:
//   Draft : q_j from row 0, draw -> st->drafts[j]
//   Plain : p from row 0, draw -> st->t_new
//   Accept: rows 0..k against q_0..q_{k-1}; emits [t_next, accepted drafts]
//           into out, sets a, forced, t_new (correction or draw from row a)
// nuni > 0: the chain's uniforms are b.uni[0..nuni) in order (the caller's
// shared uniforms), then the SplitMix64 stream.
void sample_rows(SampleBufs& b, const float* logits, int V, int rows, const cmf_sampler_config& sc,
                 DState* st, SampleMode mode, int j_or_k, int* out, hipStream_t s, int nuni = 0);

// The sparse distribution of logits row 0 (sparse_distribution_into with the
// argmax fallback of a fully filtered row): ids ascending into ids[0..n),
// probabilities into probs (capacity SPARSE_CAP), n into *n (all device
// pointers).
void sample_distribution(SampleBufs& b, const float* logits, int V, const cmf_sampler_config& sc, int* ids,
                         float* probs, int* n, hipStream_t s);

}  // namespace cmf
