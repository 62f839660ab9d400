// The sampler's sparse chain and speculative acceptance on the GPU.
//
// Selection: every block takes SLICE logits of one row, finds the top-k by
// (value desc, id asc) with an in-LDS radix select over order-preserving
// keys, and records the slice max and sum of exp((l - max)/T); a merge block
// per row selects the row's top-k from the slice lists and combines the
// sums (sum_all = sum_s ssum_s * exp((smax_s - lmax)/T)).  The O(k) chain of
// sparse_distribution_into (sampler.rs:440-514), draw_sparse (:661-671) and
// spec_accept_or_correct_sparse (:683-711) then runs in one thread with the
// SplitMix64 state (sampler.rs:54-84) kept in HBM, consuming uniforms in the
// reference's order.  Ties at the k-th value keep the k lowest ids (the
// reference also keeps every further tie; continuous logits have none).
#include <math.h>

#include "../../include/cmf_hip.h"
#include "common.h"
#include "sample.h"

namespace cmf {

struct SampCfg {
    float t, top_p, min_p;
    int k;
};

__device__ __forceinline__ uint32_t fkey(float f) {
    const uint32_t u = __float_as_uint(f);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ bool better(float va, int ia, float vb, int ib) {
    return va > vb || (va == vb && ia < ib);
}

// Top-k of (vals, ids) in LDS, n entries, 256 threads.  Writes the k winners
// sorted by (value desc, id asc) into ov/oi.  scratch: hist[256], ties.
__device__ void select_topk(const float* vals, const int* ids, int n, int k, float* ov, int* oi,
                            int* hist, float* tv, int* ti, int* cnt) {
    const int t = threadIdx.x;
    __shared__ uint32_t s_prefix, s_mask;
    __shared__ int s_kk;
    if (t == 0) {
        s_prefix = 0;
        s_mask = 0;
        s_kk = k < n ? k : n;
    }
    __syncthreads();
    const int kk_total = k < n ? k : n;
    for (int shift = 24; shift >= 0; shift -= 8) {
        hist[t] = 0;
        __syncthreads();
        const uint32_t pre = s_prefix, msk = s_mask;
        for (int i = t; i < n; i += 256) {
            const uint32_t key = fkey(vals[i]);
            if ((key & msk) == pre) atomicAdd(&hist[(key >> shift) & 255], 1);
        }
        __syncthreads();
        if (t == 0) {
            int cum = 0, kk = s_kk, sel = 0;
            for (int d = 255; d >= 0; d--) {
                if (cum + hist[d] >= kk) {
                    sel = d;
                    kk -= cum;
                    break;
                }
                cum += hist[d];
            }
            s_prefix = pre | ((uint32_t)sel << shift);
            s_mask = msk | (0xFFu << shift);
            s_kk = kk;
        }
        __syncthreads();
    }
    const uint32_t kth = s_prefix;
    const int need_eq = s_kk;  // entries equal to kth still needed
    if (t == 0) {
        cnt[0] = 0;
        cnt[1] = 0;
    }
    __syncthreads();
    // strictly greater: all of them; equal: collect (capped) then lowest ids
    for (int i = t; i < n; i += 256) {
        const uint32_t key = fkey(vals[i]);
        if (key > kth) {
            const int p = atomicAdd(&cnt[0], 1);
            if (p < SPARSE_K_MAX) {
                tv[p] = vals[i];
                ti[p] = ids[i];
            }
        } else if (key == kth) {
            const int p = atomicAdd(&cnt[1], 1);
            if (p < 256) {
                tv[SPARSE_K_MAX + p] = vals[i];
                ti[SPARSE_K_MAX + p] = ids[i];
            }
        }
    }
    __syncthreads();
    const int ngt = cnt[0] < SPARSE_K_MAX ? cnt[0] : SPARSE_K_MAX;
    const int neq = cnt[1] < 256 ? cnt[1] : 256;
    if (t == 0) {
        // lowest ids among the ties
        for (int i = 1; i < neq; i++) {
            const int id = ti[SPARSE_K_MAX + i];
            const float v = tv[SPARSE_K_MAX + i];
            int j = i - 1;
            while (j >= 0 && ti[SPARSE_K_MAX + j] > id) {
                ti[SPARSE_K_MAX + j + 1] = ti[SPARSE_K_MAX + j];
                tv[SPARSE_K_MAX + j + 1] = tv[SPARSE_K_MAX + j];
                j--;
            }
            ti[SPARSE_K_MAX + j + 1] = id;
            tv[SPARSE_K_MAX + j + 1] = v;
        }
        int p = ngt;
        for (int i = 0; i < need_eq && i < neq && p < SPARSE_K_MAX; i++, p++) {
            tv[p] = tv[SPARSE_K_MAX + i];
            ti[p] = ti[SPARSE_K_MAX + i];
        }
        cnt[2] = p;
    }
    __syncthreads();
    const int m = cnt[2] < kk_total ? cnt[2] : kk_total;
    // rank sort
    if (t < m) {
        const float v = tv[t];
        const int id = ti[t];
        int r = 0;
        for (int j = 0; j < m; j++)
            if (better(tv[j], ti[j], v, id)) r++;
        ov[r] = v;
        oi[r] = id;
    }
    __syncthreads();
}

__global__ __launch_bounds__(256) void k_topk_slice(const float* __restrict__ logits, int V, SampCfg c,
                                                    int nslices, int* __restrict__ cid,
                                                    float* __restrict__ cv, float* __restrict__ smax,
                                                    float* __restrict__ ssum) {
    const int sl = blockIdx.x, row = blockIdx.y, t = threadIdx.x;
    __shared__ float vals[SLICE];
    __shared__ int ids[SLICE];
    __shared__ int hist[256];
    __shared__ float tv[SPARSE_K_MAX + 256];
    __shared__ int ti[SPARSE_K_MAX + 256];
    __shared__ int cnt[4];
    __shared__ float ov[SPARSE_K_MAX];
    __shared__ int oi[SPARSE_K_MAX];
    __shared__ float red[256];
    const int lo = sl * SLICE, n = min(SLICE, V - lo);
    const float* src = logits + (size_t)row * V + lo;
    float mx = -INFINITY;
    {
        float tmp[SLICE / 256];  // all loads in flight together
#pragma unroll
        for (int u = 0; u < SLICE / 256; u++) {
            const int i = t + 256 * u;
            tmp[u] = i < n ? src[i] : -INFINITY;
        }
#pragma unroll
        for (int u = 0; u < SLICE / 256; u++) {
            const int i = t + 256 * u;
            if (i < n) {
                vals[i] = tmp[u];
                ids[i] = lo + i;
                mx = fmaxf(mx, tmp[u]);
            }
        }
    }
    red[t] = mx;
    __syncthreads();
    for (int o = 128; o > 0; o >>= 1) {
        if (t < o) red[t] = fmaxf(red[t], red[t + o]);
        __syncthreads();
    }
    mx = red[0];
    __syncthreads();
    float se = 0.f;
    for (int i = t; i < n; i += 256) se += expf((vals[i] - mx) / c.t);
    red[t] = se;
    __syncthreads();
    for (int o = 128; o > 0; o >>= 1) {
        if (t < o) red[t] += red[t + o];
        __syncthreads();
    }
    select_topk(vals, ids, n, c.k, ov, oi, hist, tv, ti, cnt);
    const size_t base = ((size_t)row * nslices + sl) * SPARSE_K_MAX;
    const int m = min(c.k, n);
    if (t < SPARSE_K_MAX) {
        cid[base + t] = t < m ? oi[t] : -1;
        cv[base + t] = t < m ? ov[t] : -INFINITY;
    }
    if (t == 0) {
        smax[(size_t)row * nslices + sl] = mx;
        ssum[(size_t)row * nslices + sl] = red[0];
    }
}

__global__ __launch_bounds__(256) void k_topk_merge(int V, SampCfg c, int nslices,
                                                    const int* __restrict__ cid,
                                                    const float* __restrict__ cv,
                                                    const float* __restrict__ smax,
                                                    const float* __restrict__ ssum, int* __restrict__ rid,
                                                    float* __restrict__ rv, float* __restrict__ lmax,
                                                    float* __restrict__ sum) {
    const int row = blockIdx.x, t = threadIdx.x;
    __shared__ float vals[SLICE];
    __shared__ int ids[SLICE];
    __shared__ int hist[256];
    __shared__ float tv[SPARSE_K_MAX + 256];
    __shared__ int ti[SPARSE_K_MAX + 256];
    __shared__ int cnt[4];
    __shared__ float ov[SPARSE_K_MAX];
    __shared__ int oi[SPARSE_K_MAX];
    const int k = min(c.k, V);
    const int n = nslices * k;  // <= SLICE (checked by the host)
    {
        int ti_[SLICE / 256];
        float tv_[SLICE / 256];
#pragma unroll
        for (int u = 0; u < SLICE / 256; u++) {
            const int e = t + 256 * u, sl = e / k, i = e - sl * k;
            const size_t at = ((size_t)row * nslices + sl) * SPARSE_K_MAX + i;
            ti_[u] = e < n ? cid[at] : -1;
            tv_[u] = e < n ? cv[at] : -INFINITY;
        }
#pragma unroll
        for (int u = 0; u < SLICE / 256; u++) {
            const int e = t + 256 * u;
            if (e < n) {
                vals[e] = ti_[u] >= 0 ? tv_[u] : -INFINITY;
                ids[e] = ti_[u] >= 0 ? ti_[u] : 0x7FFFFFFF;
            }
        }
    }
    __syncthreads();
    select_topk(vals, ids, n, k, ov, oi, hist, tv, ti, cnt);
    if (t < SPARSE_K_MAX) {
        rid[(size_t)row * SPARSE_K_MAX + t] = t < k ? oi[t] : -1;
        rv[(size_t)row * SPARSE_K_MAX + t] = t < k ? ov[t] : -INFINITY;
    }
    if (t == 0) {
        const float lm = ov[0];
        float tot = 0.f;
        for (int s = 0; s < nslices; s++)
            tot += ssum[(size_t)row * nslices + s] * expf((smax[(size_t)row * nslices + s] - lm) / c.t);
        lmax[row] = lm;
        sum[row] = tot;
    }
}

// ---- the O(k) chain, one thread ----
__device__ __forceinline__ float next_f32(unsigned long long* s) {
    *s += 0x9E3779B97F4A7C15ull;
    unsigned long long z = *s;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    z ^= z >> 31;
    return (float)(z >> 40) / 16777216.0f;
}

// sparse_distribution_into over the merged candidates of one row: ids
// ascending, probabilities summing to 1.  Returns the count (0 = filtered).
__device__ int sparse_dist(const int* rid, const float* rv, float lmax, float sum_all, SampCfg c,
                           int* oid, float* op) {
    int n = 0;
    float cum = 0.f;
    bool cut = false;
    for (int i = 0; i < c.k && !cut; i++) {
        const int id = rid[i];
        if (id < 0) break;
        const float e = expf((rv[i] - lmax) / c.t);
        if (c.min_p > 0.f && e < c.min_p) continue;
        const float pr = e / sum_all;
        if (pr <= 0.f) continue;
        oid[n] = id;
        op[n] = pr;
        n++;
        cum += pr;
        if (c.top_p < 1.f && c.top_p > 0.f && cum >= c.top_p) cut = true;
    }
    float s = 0.f;
    for (int i = 0; i < n; i++) s += op[i];
    if (!(s > 0.f)) return 0;
    for (int i = 0; i < n; i++) op[i] /= s;
    for (int i = 1; i < n; i++) {  // by id
        const int id = oid[i];
        const float p = op[i];
        int j = i - 1;
        while (j >= 0 && oid[j] > id) {
            oid[j + 1] = oid[j];
            op[j + 1] = op[j];
            j--;
        }
        oid[j + 1] = id;
        op[j + 1] = p;
    }
    return n;
}

// the greedy fallback of a fully filtered row: argmax, ties to the highest id
__device__ int row_argmax(const int* rid, const float* rv, int k) {
    int best = rid[0];
    for (int i = 1; i < k && rid[i] >= 0; i++)
        if (rv[i] == rv[0] && rid[i] > best) best = rid[i];
    return best;
}

// The chain's uniform source: the caller's uniforms first (a verify step
// under shared uniforms), then the SplitMix64 stream.
struct Uni {
    unsigned long long rng;
    const float* u;
    int n, used;
    __device__ float next() { return used < n ? u[used++] : next_f32(&rng); }
};

__device__ int draw_sparse(const int* id, const float* p, int n, Uni* rng) {
    const float r = rng->next();
    float cum = 0.f;
    for (int i = 0; i < n; i++) {
        cum += p[i];
        if (r < cum) return id[i];
    }
    for (int i = n - 1; i >= 0; i--)
        if (p[i] > 0.f) return id[i];
    return 0;
}

__device__ float sparse_get(const int* id, const float* p, int n, int q) {
    for (int i = 0; i < n; i++)
        if (id[i] == q) return p[i];
    return 0.f;
}

__global__ void k_sample_finish(SampCfg c, int mode, int jk, const int* __restrict__ rid,
                                const float* __restrict__ rv, const float* __restrict__ lmax,
                                const float* __restrict__ sum, int* __restrict__ qid,
                                float* __restrict__ qp, int* __restrict__ qn, DState* st,
                                int* __restrict__ out, const float* __restrict__ uni, int nuni) {
    // the O(k) chain runs in one thread; its working lists live in LDS
    __shared__ int pid[SPARSE_K_MAX], rsid[SPARSE_K_MAX];
    __shared__ float pp[SPARSE_K_MAX], rsp[SPARSE_K_MAX];
    if (threadIdx.x != 0) return;
    Uni rng{st->rng, uni, nuni, 0};
    if (mode == 0 || mode == 1) {  // Draft / Plain: distribution of row 0, one draw
        int n = sparse_dist(rid, rv, lmax[0], sum[0], c, pid, pp);
        if (n == 0) {
            pid[0] = row_argmax(rid, rv, c.k);
            pp[0] = 1.f;
            n = 1;
        }
        const int tok = draw_sparse(pid, pp, n, &rng);
        if (mode == 0) {
            for (int i = 0; i < n; i++) {
                qid[jk * SPARSE_K_MAX + i] = pid[i];
                qp[jk * SPARSE_K_MAX + i] = pp[i];
            }
            qn[jk] = n;
            st->drafts[jk] = tok;
        } else {
            st->t_new = tok;
        }
        st->rng = rng.rng;
        return;
    }
    // Accept (pipeline.rs:3894-3934 + the loop-top sample of row a)
    const int k = jk;
    int a = 0, forced = -1;
    while (a < k) {
        const int* r_id = rid + (size_t)a * SPARSE_K_MAX;
        const float* r_v = rv + (size_t)a * SPARSE_K_MAX;
        int np = sparse_dist(r_id, r_v, lmax[a], sum[a], c, pid, pp);
        if (np == 0) {
            pid[0] = row_argmax(r_id, r_v, c.k);
            pp[0] = 1.f;
            np = 1;
        }
        const int d = st->drafts[a];
        const int* q_id = qid + a * SPARSE_K_MAX;
        const float* q_p = qp + a * SPARSE_K_MAX;
        const int nq = qn[a];
        const float pd = sparse_get(pid, pp, np, d), qd = sparse_get(q_id, q_p, nq, d);
        const float r = rng.next();
        if (qd > 0.f && r * qd < pd) {
            a++;
            continue;
        }
        int nr = 0;
        float total = 0.f;
        for (int i = 0; i < np; i++) {
            const float ri = pp[i] - sparse_get(q_id, q_p, nq, pid[i]);
            if (ri > 0.f) {
                rsid[nr] = pid[i];
                rsp[nr] = ri;
                nr++;
                total += ri;
            }
        }
        if (total <= 0.f) {
            forced = draw_sparse(pid, pp, np, &rng);
        } else {
            for (int i = 0; i < nr; i++) rsp[i] /= total;
            forced = draw_sparse(rsid, rsp, nr, &rng);
        }
        break;
    }
    int tnew = forced;
    if (forced < 0) {  // loop top: sample row a (sample_with_scratch_pool)
        const int* r_id = rid + (size_t)a * SPARSE_K_MAX;
        const float* r_v = rv + (size_t)a * SPARSE_K_MAX;
        int np = sparse_dist(r_id, r_v, lmax[a], sum[a], c, pid, pp);
        if (np > 0) tnew = draw_sparse(pid, pp, np, &rng);
        else tnew = row_argmax(r_id, r_v, c.k);
    }
    const int n0 = st->n_out;
    out[n0] = st->t_next;
    for (int j = 0; j < a; j++) out[n0 + 1 + j] = st->drafts[j];
    st->n_out = n0 + 1 + a;
    st->a = a;
    st->forced = forced;
    st->t_new = tnew;
    st->accepted += a;
    st->rng = rng.rng;
}

__global__ void k_sample_dist(SampCfg c, const int* __restrict__ rid, const float* __restrict__ rv,
                              const float* __restrict__ lmax, const float* __restrict__ sum, int* __restrict__ ids,
                              float* __restrict__ probs, int* __restrict__ n_out) {
    __shared__ int pid[SPARSE_K_MAX];
    __shared__ float pp[SPARSE_K_MAX];
    if (threadIdx.x != 0) return;
    int n = sparse_dist(rid, rv, lmax[0], sum[0], c, pid, pp);
    if (n == 0) {
        pid[0] = row_argmax(rid, rv, c.k);
        pp[0] = 1.f;
        n = 1;
    }
    for (int i = 0; i < n; i++) {
        ids[i] = pid[i];
        probs[i] = pp[i];
    }
    *n_out = n;
}

int sample_alloc(SampleBufs& b, int V, const std::function<int(void**, size_t)>& alloc) {
    b.V = V;
    b.nslices = (V + SLICE - 1) / SLICE;
    const int R = MAXB + 1;
    const size_t nc = (size_t)R * b.nslices * SPARSE_K_MAX;
    if (alloc((void**)&b.cid, nc * 4) || alloc((void**)&b.cv, nc * 4) ||
        alloc((void**)&b.smax, (size_t)R * b.nslices * 4) || alloc((void**)&b.ssum, (size_t)R * b.nslices * 4) ||
        alloc((void**)&b.rid, (size_t)R * SPARSE_K_MAX * 4) || alloc((void**)&b.rv, (size_t)R * SPARSE_K_MAX * 4) ||
        alloc((void**)&b.lmax, R * 4) || alloc((void**)&b.sum, R * 4) ||
        alloc((void**)&b.qid, 8 * SPARSE_K_MAX * 4) || alloc((void**)&b.qp, 8 * SPARSE_K_MAX * 4) ||
        alloc((void**)&b.qn, 8 * 4) || alloc((void**)&b.uni, (MAXB + 1) * 4))
        return CMF_ERR;
    return CMF_OK;
}

static SampCfg samp_cfg(const cmf_sampler_config& sc, int V) {
    SampCfg c;
    c.t = sc.temperature > 0.f ? sc.temperature : 1.0f;
    c.top_p = sc.top_p;
    c.min_p = sc.min_p;
    c.k = (int)sc.top_k < V ? (int)sc.top_k : V;
    return c;
}

void sample_distribution(SampleBufs& b, const float* logits, int V, const cmf_sampler_config& sc, int* ids,
                         float* probs, int* n, hipStream_t s) {
    const SampCfg c = samp_cfg(sc, V);
    hipLaunchKernelGGL(k_topk_slice, dim3(b.nslices, 1), dim3(256), 0, s, logits, V, c, b.nslices, b.cid, b.cv,
                       b.smax, b.ssum);
    hipLaunchKernelGGL(k_topk_merge, dim3(1), dim3(256), 0, s, V, c, b.nslices, b.cid, b.cv, b.smax, b.ssum,
                       b.rid, b.rv, b.lmax, b.sum);
    hipLaunchKernelGGL(k_sample_dist, dim3(1), dim3(64), 0, s, c, b.rid, b.rv, b.lmax, b.sum, ids, probs, n);
}

void sample_rows(SampleBufs& b, const float* logits, int V, int rows, const cmf_sampler_config& sc,
                 DState* st, SampleMode mode, int jk, int* out, hipStream_t s, int nuni) {
    const SampCfg c = samp_cfg(sc, V);
    hipLaunchKernelGGL(k_topk_slice, dim3(b.nslices, rows), dim3(256), 0, s, logits, V, c, b.nslices, b.cid,
                       b.cv, b.smax, b.ssum);
    hipLaunchKernelGGL(k_topk_merge, dim3(rows), dim3(256), 0, s, V, c, b.nslices, b.cid, b.cv, b.smax,
                       b.ssum, b.rid, b.rv, b.lmax, b.sum);
    const int m = mode == SampleMode::Draft ? 0 : (mode == SampleMode::Plain ? 1 : 2);
    hipLaunchKernelGGL(k_sample_finish, dim3(1), dim3(64), 0, s, c, m, jk, b.rid, b.rv, b.lmax, b.sum, b.qid,
                       b.qp, b.qn, st, out, b.uni, nuni);
}

}  // namespace cmf
