// The sampler's sparse chain and speculative acceptance on the GPU.
//
// Selection: every block takes SLICE logits of one row, finds the top-k by
// (value desc, id asc) with an in-LDS radix select over order-preserving
// keys (each pass's bucket found by a block-wide scan), and records the slice
// max and sum of exp((l - max)/T); a merge block per row selects the row's
// top-k from the slice lists and combines the sums (sum_all = sum_s ssum_s *
// exp((smax_s - lmax)/T), in slice order).  The O(k) chain of
// sparse_distribution_into (sampler.rs:440-514), draw_sparse (:661-671) and
// spec_accept_or_correct_sparse (:683-711) then runs on one wave (lane =
// candidate; every order-dependent float sum walks the lanes in the
// reference's order) with the SplitMix64 state (sampler.rs:54-84) kept in
// HBM, consuming uniforms in the reference's order.  As par_topk
// (sampler.rs:515-600) the candidates are the top k and every entry tied
// with the k-th value, in index order up to 4 k + 64 of them: each slice
// also lists its ties past its own top k, and the merge gathers the entries
// >= the row's k-th value in index order when there are more than k.
#include <climits>
#include <math.h>

#include "../../include/cmf_hip.h"
#include "common.h"
#include "sample.h"
#include "wave.h"

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

// Bucket selection of one radix pass: with the 256 bucket counts of the keys
// still in play (hist, 256 threads) and kk of them still needed, the bucket d
// scanning 255 -> 0 where the count above d is < kk and with d >= kk, and kk
// less the count above.  A block-wide scan replaces the serial walk over the
// buckets (a wave-level inclusive scan, then the waves' totals).  With no
// such bucket the prefix stays and kk is unchanged (d = 0).
__device__ __forceinline__ void pick_bucket(const int* hist, int shift, uint32_t* s_prefix, uint32_t* s_mask,
                                            int* s_kk, int* wsum, int kk_total, int* s_cand) {
    const int t = threadIdx.x, lane = t & 63, w = t >> 6;
    const int kk = *s_kk;
    const uint32_t pre = *s_prefix, msk = *s_mask;
    const int h = hist[255 - t];
    int p = h;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const int u = __shfl_up(p, o);
        if (lane >= o) p += u;
    }
    if (lane == 63) wsum[w] = p;
    __syncthreads();
    int base = 0;
    for (int i = 0; i < w; i++) base += wsum[i];
    p += base;
    __syncthreads();  // every thread has read kk, the prefix and wsum
    if (t == 0) {
        *s_mask = msk | (0xFFu << shift);  // prefix unchanged (d = 0) unless a bucket is picked below
    }
    if (p >= kk && p - h < kk) {
        *s_prefix = pre | ((uint32_t)(255 - t) << shift);
        *s_kk = kk - (p - h);
        *s_cand = p + (kk_total - kk);  // keys at or above the new prefix
    }
    __syncthreads();
}

// Sorts the m <= 256 entries tv/ti[0, m) by (value desc, id asc) and writes
// those ranked below k to ov/oi (256 threads).  Each entry counts the
// entries ahead of it; the list is padded to a multiple of 16 with entries
// that rank last and read four at a time (the reads in flight together
// rather than one LDS round trip per entry).  Ids are distinct.
__device__ void rank_sort_lds(float* tv, int* ti, int m, int k, float* ov, int* oi) {
    const int t = threadIdx.x;
    const int m16 = (m + 15) & ~15;
    if (t >= m && t < m16) {
        tv[t] = -INFINITY;
        ti[t] = 0x7FFFFFFF;
    }
    __syncthreads();
    if (t < m) {
        const float v = tv[t];
        const int id = ti[t];
        int r = 0;
        for (int j = 0; j < m16; j += 16) {
#pragma unroll
            for (int i = 0; i < 16; i += 4) {
                const float4 a4 = *(const float4*)&tv[j + i];
                const int4 b4 = *(const int4*)&ti[j + i];
                r += better(a4.x, b4.x, v, id) ? 1 : 0;
                r += better(a4.y, b4.y, v, id) ? 1 : 0;
                r += better(a4.z, b4.z, v, id) ? 1 : 0;
                r += better(a4.w, b4.w, v, id) ? 1 : 0;
            }
        }
        if (r < k) {
            ov[r] = v;
            oi[r] = id;
        }
    }
    __syncthreads();
}

// Sorts m <= SPARSE_CAP entries tv/ti[0, m) by (value desc, id asc) into
// ov/oi[0, m) (256 threads; rank_sort_lds with two entries per thread).
__device__ void rank_sort_cap(float* tv, int* ti, int m, float* ov, int* oi) {
    const int t = threadIdx.x;
    const int m16 = (m + 15) & ~15;
    for (int e = m + t; e < m16; e += 256) {
        tv[e] = -INFINITY;
        ti[e] = 0x7FFFFFFF;
    }
    __syncthreads();
    for (int e = t; e < m; e += 256) {
        const float v = tv[e];
        const int id = ti[e];
        int r = 0;
        for (int j = 0; j < m16; j += 4) {
            const float4 a4 = *(const float4*)&tv[j];
            const int4 b4 = *(const int4*)&ti[j];
            r += better(a4.x, b4.x, v, id) ? 1 : 0;
            r += better(a4.y, b4.y, v, id) ? 1 : 0;
            r += better(a4.z, b4.z, v, id) ? 1 : 0;
            r += better(a4.w, b4.w, v, id) ? 1 : 0;
        }
        ov[r] = v;
        oi[r] = id;
    }
    __syncthreads();
}

// Top-k by (value desc, id asc) of n entries held NPT per thread (entry i =
// thread t's slot u with i = t + 256 u; entries i >= n are not in play),
// 256 threads.  Writes the k winners sorted into ov/oi.  Radix select over
// order-preserving keys, 8 bits a pass, each pass's bucket found by a
// block-wide scan; the keys stay in registers.  The first pass counts into
// 16 copies of the histogram (lane % 16 picks the copy: at most 16 lanes of
// a wave meet on one address, where same-bucket keys, the common case
// there, used to serialize 64 deep; the copies are 257 words apart so that
// one bucket's copies sit in distinct LDS banks); the later passes count
// only the keys under the chosen prefix, into one histogram.  Once at most
// 256 keys sit at or above the chosen prefix (those above it are in the
// top-k, those on it compete), the passes stop and a rank sort of those keys
// decides.  scratch: hist[16][257], ties.
template <int NPT>
__device__ void select_topk_reg(const float (&v)[NPT], const int (&id)[NPT], int n, int k, float* ov, int* oi,
                                int (*hist)[257], float* tv, int* ti, int* cnt) {
    const int t = threadIdx.x, hc = t & 15;
    __shared__ uint32_t s_prefix, s_mask;
    __shared__ int s_kk;
    __shared__ int wsum[4];
    __shared__ int htot[256];
    __shared__ int s_cand;
    uint32_t key[NPT];
#pragma unroll
    for (int u = 0; u < NPT; u++) key[u] = t + 256 * u < n ? fkey(v[u]) : 0u;  // 0: below every real key
    if (t == 0) {
        s_prefix = 0;
        s_mask = 0;
        s_kk = k < n ? k : n;
    }
    const int kk_total = k < n ? k : n;
    for (int shift = 24; shift >= 0; shift -= 8) {
        if (shift == 24) {
            // first pass: most keys share a few top bytes, so the counts go
            // to the 16 copies
#pragma unroll
            for (int c = 0; c < 16; c++) hist[c][t] = 0;
            __syncthreads();
#pragma unroll
            for (int u = 0; u < NPT; u++)
                if (t + 256 * u < n) atomicAdd(&hist[hc][key[u] >> 24], 1);
            __syncthreads();
            int s = 0;
#pragma unroll
            for (int c = 0; c < 16; c++) s += hist[c][t];
            htot[t] = s;
        } else {
            // later passes count only the keys under the chosen prefix (few,
            // spread over the buckets): one histogram
            htot[t] = 0;
            __syncthreads();
            const uint32_t pre = s_prefix, msk = s_mask;
#pragma unroll
            for (int u = 0; u < NPT; u++)
                if (t + 256 * u < n && (key[u] & msk) == pre) atomicAdd(&htot[(key[u] >> shift) & 255], 1);
        }
        if (t == 0) s_cand = 0x7FFFFFFF;  // no bucket picked: no early stop
        __syncthreads();
        pick_bucket(htot, shift, &s_prefix, &s_mask, &s_kk, wsum, kk_total, &s_cand);
        if (s_cand <= 256) break;
    }
    if (s_cand <= 256) {
        // the keys at or above the prefix: the top-k among them by rank
        const uint32_t pre = s_prefix, msk = s_mask;
        if (t == 0) cnt[0] = 0;
        __syncthreads();
#pragma unroll
        for (int u = 0; u < NPT; u++)
            if (t + 256 * u < n && (key[u] & msk) >= pre) {
                const int p = atomicAdd(&cnt[0], 1);
                if (p < 256) {
                    tv[p] = v[u];
                    ti[p] = id[u];
                }
            }
        __syncthreads();
        rank_sort_lds(tv, ti, cnt[0] < 256 ? cnt[0] : 256, kk_total, ov, oi);
        return;
    }
    const uint32_t kth = s_prefix;
    const int need_eq = s_kk;  // entries equal to kth still needed
    if (t == 0) {
        cnt[0] = 0;
        cnt[1] = 0;
    }
    __syncthreads();
    // strictly greater: all of them; equal: collect (capped) then lowest ids
#pragma unroll
    for (int u = 0; u < NPT; u++) {
        if (t + 256 * u >= n) continue;
        if (key[u] > kth) {
            const int p = atomicAdd(&cnt[0], 1);
            if (p < SPARSE_K_MAX) {
                tv[p] = v[u];
                ti[p] = id[u];
            }
        } else if (key[u] == kth) {
            const int p = atomicAdd(&cnt[1], 1);
            if (p < 256) {
                tv[SPARSE_K_MAX + p] = v[u];
                ti[SPARSE_K_MAX + p] = id[u];
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
    rank_sort_lds(tv, ti, m, m, ov, oi);
}

__global__ __launch_bounds__(256) void k_topk_slice(const float* __restrict__ logits, int V, SampCfg c,
                                                    int nslices, int* __restrict__ cid,
                                                    float* __restrict__ cv, float* __restrict__ smax,
                                                    float* __restrict__ ssum, int* __restrict__ ocnt,
                                                    int* __restrict__ oid) {
    const int sl = blockIdx.x, row = blockIdx.y, t = threadIdx.x;
    __shared__ int hist[16][257];  // copies 257 apart: one bucket's copies fall in distinct banks
    __shared__ __align__(16) float tv[SPARSE_K_MAX + 256];
    __shared__ __align__(16) int ti[SPARSE_K_MAX + 256];
    __shared__ int cnt[4];
    __shared__ float ov[SPARSE_K_MAX];
    __shared__ int oi[SPARSE_K_MAX];
    __shared__ float red[256];
    const int lo = sl * SLICE, n = min(SLICE, V - lo);
    const float* src = logits + (size_t)row * V + lo;
    float mx = -INFINITY;
    constexpr int NPT = SLICE / 256;
    float vals[NPT];  // entry t + 256 u (all loads in flight together)
    int ids[NPT];
#pragma unroll
    for (int u = 0; u < NPT; u++) {
        const int i = t + 256 * u;
        vals[u] = i < n ? src[i] : -INFINITY;
        ids[u] = lo + i;
    }
#pragma unroll
    for (int u = 0; u < NPT; u++) mx = fmaxf(mx, vals[u]);
    // slice max and sum of exp((l - max) / T): wave reductions, then the
    // four waves' values in wave order
    const int w = t >> 6;
    mx = wave_max(mx);
    if ((t & 63) == 0) red[w] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    float se = 0.f;
#pragma unroll
    for (int u = 0; u < NPT; u++)
        if (t + 256 * u < n) se += expf((vals[u] - mx) / c.t);
    se = wave_sum(se);
    __syncthreads();  // red[] reads above are done
    if ((t & 63) == 0) red[4 + w] = se;
    select_topk_reg<NPT>(vals, ids, n, c.k, ov, oi, hist, tv, ti, cnt);  // (its barriers publish red[4..7])
    const size_t base = ((size_t)row * nslices + sl) * SPARSE_K_MAX;
    const int m = min(c.k, n);
    // ties at the slice's k-th value past its list: the list holds the lowest
    // ids among them (the first in index order); the others go to oid in
    // index order (at most SPARSE_CAP), their count to ocnt
    {
        __shared__ int s_t, s_l, wc[4];
        if (t == 0) {
            s_t = 0;
            s_l = 0;
        }
        __syncthreads();
        const float kv = m > 0 ? ov[m - 1] : -INFINITY;
        const bool full = m == c.k && m > 0 && isfinite(kv);  // (uniform: LDS values)
        int over = 0;
        if (full) {
            int mine = 0;
#pragma unroll
            for (int u = 0; u < NPT; u++) mine += (t + 256 * u < n && vals[u] == kv) ? 1 : 0;
            if (mine) atomicAdd(&s_t, mine);
            if (t < m && ov[t] == kv) atomicAdd(&s_l, 1);
            __syncthreads();
            over = s_t - s_l;
        }
        if (over > 0) {  // (rare: tied logits)
            const int L = s_l, lane = t & 63, w = t >> 6;
            int* dst = oid + ((size_t)row * nslices + sl) * SPARSE_CAP;
            int done = 0;
            for (int u = 0; u < NPT; u++) {
                const bool f = t + 256 * u < n && vals[u] == kv;
                const unsigned long long bm = __ballot(f);
                if (lane == 0) wc[w] = __popcll(bm);
                __syncthreads();
                int off = done;
                for (int q = 0; q < w; q++) off += wc[q];
                const int tot = wc[0] + wc[1] + wc[2] + wc[3];
                __syncthreads();  // every wave has read wc
                const int pos = off + __popcll(bm & ((1ull << lane) - 1ull)) - L;
                if (f && pos >= 0 && pos < SPARSE_CAP) dst[pos] = lo + 256 * u + t;
                done += tot;
            }
            over = min(over, SPARSE_CAP);
        }
        if (t == 0) ocnt[(size_t)row * nslices + sl] = over;
    }
    if (t < SPARSE_K_MAX) {
        cid[base + t] = t < m ? oi[t] : -1;
        cv[base + t] = t < m ? ov[t] : -INFINITY;
    }
    if (t == 0) {
        smax[(size_t)row * nslices + sl] = mx;
        ssum[(size_t)row * nslices + sl] = (red[4] + red[5]) + (red[6] + red[7]);
    }
}

__global__ __launch_bounds__(256) void k_topk_merge(int V, SampCfg c, int nslices,
                                                    const int* __restrict__ cid,
                                                    const float* __restrict__ cv,
                                                    const float* __restrict__ smax,
                                                    const float* __restrict__ ssum, const int* __restrict__ ocnt,
                                                    const int* __restrict__ oid, int* __restrict__ rid,
                                                    float* __restrict__ rv, int* __restrict__ rn,
                                                    float* __restrict__ lmax, float* __restrict__ sum) {
    const int row = blockIdx.x, t = threadIdx.x;
    __shared__ int hist[16][257];  // copies 257 apart: one bucket's copies fall in distinct banks
    __shared__ __align__(16) float tv[SPARSE_K_MAX + 256];
    __shared__ __align__(16) int ti[SPARSE_K_MAX + 256];
    __shared__ int cnt[4];
    __shared__ float ov[SPARSE_K_MAX];
    __shared__ int oi[SPARSE_K_MAX];
    const int k = min(c.k, V);
    const int n = nslices * k;  // <= SLICE (checked by the host)
    constexpr int NPT = SLICE / 256;
    float vals[NPT];  // candidate t + 256 u
    int ids[NPT];
#pragma unroll
    for (int u = 0; u < NPT; u++) {
        const int e = t + 256 * u, sl = e / k, i = e - sl * k;
        const size_t at = ((size_t)row * nslices + sl) * SPARSE_K_MAX + i;
        const int id = e < n ? cid[at] : -1;
        const float v = e < n ? cv[at] : -INFINITY;
        vals[u] = id >= 0 ? v : -INFINITY;
        ids[u] = id >= 0 ? id : 0x7FFFFFFF;
    }
    // tau: the largest k-th value of a full slice list.  That list holds k
    // entries >= tau, so an entry below tau ranks k or later: the rest
    // (usually few) go to a rank sort, else to the radix select.
    __shared__ float red[4];
    float tau = -INFINITY;
    for (int s2 = t; s2 < nslices; s2 += 256) {
        const size_t at = ((size_t)row * nslices + s2) * SPARSE_K_MAX + (k - 1);
        if (cid[at] >= 0) tau = fmaxf(tau, cv[at]);
    }
    tau = wave_max(tau);
    if ((t & 63) == 0) red[t >> 6] = tau;
    if (t == 0) cnt[3] = 0;
    __syncthreads();
    tau = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
#pragma unroll
    for (int u = 0; u < NPT; u++)
        if (t + 256 * u < n && vals[u] >= tau) {
            const int p = atomicAdd(&cnt[3], 1);
            if (p < 256) {
                tv[p] = vals[u];
                ti[p] = ids[u];
            }
        }
    __syncthreads();
    const int nc = cnt[3];
    __syncthreads();  // every thread has read cnt[3]
    if (nc <= 256) rank_sort_lds(tv, ti, nc, k, ov, oi);
    else select_topk_reg<NPT>(vals, ids, n, k, ov, oi, hist, tv, ti, cnt);
    // par_topk (sampler.rs:569-600, its serial arm :590-598): when entries
    // tied with the k-th value lie past the top k, the candidates are every
    // entry >= the k-th value in index order, at most 4 k + 64, sorted by
    // (value desc, id asc).  The entries >= kth are in the slice lists and,
    // for slices whose own k-th value is kth, in their overflow ties (a
    // slice's k-th value is never above kth: the slice would hold k entries
    // above it).
    __shared__ int s_ge, s_cnt;
    __shared__ __align__(16) float gv[SPARSE_CAP];
    __shared__ __align__(16) int gi[SPARSE_CAP];
    __shared__ float sav[SPARSE_K_MAX];
    __shared__ int sai[SPARSE_K_MAX];
    const float kth = k > 0 ? ov[k - 1] : -INFINITY;
    if (t == 0) s_ge = 0;
    __syncthreads();
    int ncand = k;
    if (k > 0 && isfinite(kth)) {  // (uniform)
        int mine = 0;
#pragma unroll
        for (int u = 0; u < NPT; u++) mine += (t + 256 * u < n && ids[u] != 0x7FFFFFFF && vals[u] >= kth) ? 1 : 0;
        for (int s2 = t; s2 < nslices; s2 += 256) {
            const size_t at = ((size_t)row * nslices + s2) * SPARSE_K_MAX + (k - 1);
            if (cid[at] >= 0 && cv[at] == kth) mine += ocnt[(size_t)row * nslices + s2];
        }
        if (mine) atomicAdd(&s_ge, mine);
        __syncthreads();
        ncand = s_ge;
    }
    if (ncand > k) {  // (rare: tied logits) the index-ordered gather, one thread
        const int cap = 4 * k + 64;
        if (t == 0) {
            int nout = 0;
            for (int s2 = 0; s2 < nslices && nout < cap; s2++) {
                const size_t lb = ((size_t)row * nslices + s2) * SPARSE_K_MAX;
                // the slice list's entries >= kth, by id (insertion sort)
                int na = 0;
                for (int i = 0; i < k; i++) {
                    const int id = cid[lb + i];
                    const float v = cv[lb + i];
                    if (id < 0 || !(v >= kth)) continue;
                    int j = na++;
                    while (j > 0 && sai[j - 1] > id) {
                        sai[j] = sai[j - 1];
                        sav[j] = sav[j - 1];
                        j--;
                    }
                    sai[j] = id;
                    sav[j] = v;
                }
                // its ties past the list (ids ascending), merged in by id
                const bool tied = cid[lb + k - 1] >= 0 && cv[lb + k - 1] == kth;
                const int nb = tied ? ocnt[(size_t)row * nslices + s2] : 0;
                const int* ob = oid + ((size_t)row * nslices + s2) * SPARSE_CAP;
                int ia = 0, ib = 0;
                while (nout < cap && (ia < na || ib < nb)) {
                    if (ib >= nb || (ia < na && sai[ia] < ob[ib])) {
                        gi[nout] = sai[ia];
                        gv[nout] = sav[ia];
                        ia++;
                    } else {
                        gi[nout] = ob[ib];
                        gv[nout] = kth;
                        ib++;
                    }
                    nout++;
                }
            }
            s_cnt = nout;
        }
        __syncthreads();
        ncand = s_cnt;
        for (int e = t; e < ncand; e += 256) {
            tv[e] = gv[e];
            ti[e] = gi[e];
        }
        __syncthreads();
        rank_sort_cap(tv, ti, ncand, gv, gi);
        for (int e = t; e < SPARSE_CAP; e += 256) {
            rid[(size_t)row * SPARSE_CAP + e] = e < ncand ? gi[e] : -1;
            rv[(size_t)row * SPARSE_CAP + e] = e < ncand ? gv[e] : -INFINITY;
        }
    } else {
        ncand = k;
        for (int e = t; e < SPARSE_CAP; e += 256) {
            rid[(size_t)row * SPARSE_CAP + e] = e < k ? oi[e] : -1;
            rv[(size_t)row * SPARSE_CAP + e] = e < k ? ov[e] : -INFINITY;
        }
    }
    if (t == 0) rn[row] = ncand;
    // sum_all = sum over slices (in slice order) of ssum_s exp((smax_s - lmax)/T):
    // the terms in parallel, the sum by one thread
    __shared__ float term[256];
    const float lm = ov[0];
    for (int s2 = t; s2 < nslices; s2 += 256)
        term[s2] = ssum[(size_t)row * nslices + s2] * expf((smax[(size_t)row * nslices + s2] - lm) / c.t);
    __syncthreads();
    if (t == 0) {
        float tot = 0.f;
        for (int s2 = 0; s2 < nslices; s2++) tot += term[s2];
        lmax[row] = lm;
        sum[row] = tot;
    }
}

// ---- the O(k) chain on one wave ----
// A candidate list of up to SPARSE_CAP entries over the wave: entry e sits in
// lane e % 64, slot e / 64 (NCP slots per lane).  Every order-dependent float
// sum (the top-p cumulative, the normalisation, the inverse-CDF draw, the
// residual total) is taken in the reference's order: a block of 64 entries
// starts from the serial total of the blocks before it and each lane adds
// the block's entries one at a time from the first (the rounding of the
// reference's sequential loop); ranks by id and list lookups are
// lane-parallel.
constexpr int NCP = SPARSE_CAP / 64;

__device__ __forceinline__ float next_f32(unsigned long long* s) {
    *s += 0x9E3779B97F4A7C15ull;
    unsigned long long z = *s;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    z ^= z >> 31;
    return (float)(z >> 40) / 16777216.0f;
}
__device__ __forceinline__ float lanef(float v, int i) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), i));
}
__device__ __forceinline__ int lanei(int v, int i) { return __builtin_amdgcn_readlane(v, i); }
// entry e of a slotted value (e wave-uniform)
__device__ __forceinline__ float entryf(const float (&x)[NCP], int e) {
    float r = 0.f;
#pragma unroll
    for (int j = 0; j < NCP; j++)
        if (j == (e >> 6)) r = lanef(x[j], e & 63);
    return r;
}
__device__ __forceinline__ int entryi(const int (&x)[NCP], int e) {
    int r = 0;
#pragma unroll
    for (int j = 0; j < NCP; j++)
        if (j == (e >> 6)) r = lanei(x[j], e & 63);
    return r;
}

// Orders the wave's LDS accesses before and after (one wave per workgroup).
__device__ __forceinline__ void wsync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Inclusive prefix sums of x over entries 0..e, for each entry e < n, in
// the rounding of a serial loop (entries past n count as 0, and s + 0 == s).
__device__ void wseq_prefix(const float (&x)[NCP], int n, float (&out)[NCP]) {
    __shared__ __align__(16) float buf[SPARSE_CAP];
    const int lane = threadIdx.x;
    wsync();
#pragma unroll
    for (int j = 0; j < NCP; j++) buf[64 * j + lane] = 64 * j + lane < n ? x[j] : 0.f;
    wsync();
    float tot = 0.f;  // the serial sum of the blocks before block j
#pragma unroll
    for (int j = 0; j < NCP; j++) {
        out[j] = tot;
        if (64 * j >= n) continue;  // (uniform)
        const int nb = min(64, n - 64 * j);
        float acc = tot;
        for (int i = 0; i < nb; i += 4) {
            const float4 v = *reinterpret_cast<const float4*>(&buf[64 * j + i]);
            acc = i <= lane ? acc + v.x : acc;
            acc = i + 1 <= lane ? acc + v.y : acc;
            acc = i + 2 <= lane ? acc + v.z : acc;
            acc = i + 3 <= lane ? acc + v.w : acc;
        }
        out[j] = acc;
        tot = lanef(acc, 63);
    }
}

// The first / last entry e < n where p holds (-1: none).
__device__ __forceinline__ int wfirst(const bool (&p)[NCP], int n) {
    const int lane = threadIdx.x;
#pragma unroll
    for (int j = 0; j < NCP; j++) {
        const unsigned long long m = __ballot(p[j] && 64 * j + lane < n);
        if (m) return 64 * j + __builtin_ctzll(m);
    }
    return -1;
}
__device__ __forceinline__ int wlast(const bool (&p)[NCP], int n) {
    const int lane = threadIdx.x;
    int r = -1;
#pragma unroll
    for (int j = 0; j < NCP; j++) {
        const unsigned long long m = __ballot(p[j] && 64 * j + lane < n);
        if (m) r = 64 * j + 63 - __builtin_clzll(m);
    }
    return r;
}

// A sparse list over the wave: entry e < n holds (id, p), ids ascending.
struct WList {
    int id[NCP];
    float p[NCP];
    int n;
};

// Writes the entries where keep holds, in entry order, as list entries
// 0.. of (ids, ps) (through LDS); returns their count.
__device__ int wcompact(const bool (&keep)[NCP], const int (&ids)[NCP], const float (&ps)[NCP], int n, WList& out) {
    __shared__ int sid[SPARSE_CAP];
    __shared__ float sp[SPARSE_CAP];
    const int lane = threadIdx.x;
    int base = 0;
    wsync();
#pragma unroll
    for (int j = 0; j < NCP; j++) {
        const bool k = keep[j] && 64 * j + lane < n;
        const unsigned long long m = __ballot(k);
        if (k) {
            const int slot = base + __builtin_popcountll(m & ((1ull << lane) - 1ull));
            sid[slot] = ids[j];
            sp[slot] = ps[j];
        }
        base += __builtin_popcountll(m);
    }
    wsync();
    out.n = base;
#pragma unroll
    for (int j = 0; j < NCP; j++) {
        const int e = 64 * j + lane;
        out.id[j] = e < base ? sid[e] : -1;
        out.p[j] = e < base ? sp[e] : 0.f;
    }
    wsync();
    return base;
}

// sparse_distribution_into (sampler.rs:440-514) over the merged candidates of
// one row (rn of them, value desc, id asc): min-p filter, p = e / sum_all,
// top-p cut (cumulative in candidate order), renormalised (sum in candidate
// order), then ids ascending.  n = 0: everything filtered.
__device__ WList wsparse_dist(const int* rid, const float* rv, int rn, float lmax, float sum_all, SampCfg c) {
    const int lane = threadIdx.x;
    int id[NCP];
    float pr[NCP], kp[NCP];
    bool kept[NCP];
#pragma unroll
    for (int j = 0; j < NCP; j++) {
        const int e = 64 * j + lane;
        id[j] = e < rn ? rid[e] : -1;
        const float v = e < rn ? rv[e] : -INFINITY;
        const float ex = expf((v - lmax) / c.t);
        pr[j] = ex / sum_all;
        kept[j] = e < rn && !(c.min_p > 0.f && ex < c.min_p) && pr[j] > 0.f;
        kp[j] = kept[j] ? pr[j] : 0.f;
    }
    // cumulative p of the kept candidates, in candidate order
    float cum[NCP];
    wseq_prefix(kp, rn, cum);
    // top-p: the first kept candidate at which the cumulative reaches top_p
    // ends the list (inclusive)
    int last = rn;
    if (c.top_p < 1.f && c.top_p > 0.f) {
        bool hit[NCP];
#pragma unroll
        for (int j = 0; j < NCP; j++) hit[j] = kept[j] && cum[j] >= c.top_p;
        const int h = wfirst(hit, rn);
        if (h >= 0) last = h + 1;
    }
    // the kept candidates before last are the list: its sum is the cumulative
    const float s = last > 0 ? entryf(cum, last - 1) : 0.f;
    WList out;
    bool in[NCP];
#pragma unroll
    for (int j = 0; j < NCP; j++) in[j] = kept[j] && 64 * j + lane < last;
    if (!(s > 0.f)) {
        out.n = 0;
#pragma unroll
        for (int j = 0; j < NCP; j++) {
            out.id[j] = -1;
            out.p[j] = 0.f;
        }
        return out;
    }
    // rank by id among the kept (ids are distinct), then ids ascending
    __shared__ __align__(16) int bid[SPARSE_CAP];
    __shared__ int sid[SPARSE_CAP];
    __shared__ float sp[SPARSE_CAP];
    const int l16 = (last + 3) & ~3;
    wsync();
#pragma unroll
    for (int j = 0; j < NCP; j++) {
        const int e = 64 * j + lane;
        if (e < l16) bid[e] = e < last && in[j] ? id[j] : INT_MAX;
    }
    wsync();
    int nin = 0;
#pragma unroll
    for (int j = 0; j < NCP; j++) nin += __builtin_popcountll(__ballot(in[j]));
#pragma unroll
    for (int j = 0; j < NCP; j++) {
        if (64 * j >= last) break;  // (uniform)
        int r = 0;
        for (int i = 0; i < l16; i += 4) {
            const int4 v = *reinterpret_cast<const int4*>(&bid[i]);
            r += (v.x < id[j]) + (v.y < id[j]) + (v.z < id[j]) + (v.w < id[j]);
        }
        if (in[j]) {
            sid[r] = id[j];
            sp[r] = pr[j] / s;
        }
    }
    wsync();
    out.n = nin;
#pragma unroll
    for (int j = 0; j < NCP; j++) {
        const int e = 64 * j + lane;
        out.id[j] = e < nin ? sid[e] : -1;
        out.p[j] = e < nin ? sp[e] : 0.f;
    }
    wsync();
    return out;
}

// the greedy fallback of a fully filtered row: argmax, ties to the highest id
__device__ int row_argmax(const int* rid, const float* rv, int rn) {
    int best = rid[0];
    for (int i = 1; i < rn; i++)
        if (rv[i] == rv[0] && rid[i] > best) best = rid[i];
    return best;
}
// a list of the one entry (id, 1)
__device__ __forceinline__ void wsingle(WList& l, int id) {
    const int lane = threadIdx.x;
    l.n = 1;
#pragma unroll
    for (int j = 0; j < NCP; j++) {
        l.id[j] = j == 0 && lane == 0 ? id : -1;
        l.p[j] = j == 0 && lane == 0 ? 1.f : 0.f;
    }
}

// The chain's uniform source: the caller's uniforms first (a verify step
// under shared uniforms), then the SplitMix64 stream (wave-uniform).
struct Uni {
    unsigned long long rng;
    const float* u;
    int n, used;
    __device__ float next() { return used < n ? u[used++] : next_f32(&rng); }
};

// draw_sparse (sampler.rs:661-671): inverse CDF in list order
__device__ int wdraw(const WList& l, Uni* rng) {
    const float r = rng->next();
    float cum[NCP];
    wseq_prefix(l.p, l.n, cum);
    bool hit[NCP], pos[NCP];
#pragma unroll
    for (int j = 0; j < NCP; j++) {
        hit[j] = r < cum[j];
        pos[j] = l.p[j] > 0.f;
    }
    const int h = wfirst(hit, l.n);
    if (h >= 0) return entryi(l.id, h);
    // rounding left the cumulative short of r: the last entry with p > 0
    const int lp = wlast(pos, l.n);
    if (lp >= 0) return entryi(l.id, lp);
    return 0;
}

// p in list l of each of this lane's entries' ids x (0 if absent)
__device__ void wget_each(const WList& l, const int (&x)[NCP], float (&out)[NCP]) {
    __shared__ __align__(16) int bid[SPARSE_CAP];
    __shared__ __align__(16) float bp[SPARSE_CAP];
    const int lane = threadIdx.x;
    const int n4 = (l.n + 3) & ~3;
    wsync();
#pragma unroll
    for (int j = 0; j < NCP; j++) {
        const int e = 64 * j + lane;
        if (e < n4) {
            bid[e] = e < l.n ? l.id[j] : -1;
            bp[e] = e < l.n ? l.p[j] : 0.f;
        }
    }
    wsync();
#pragma unroll
    for (int j = 0; j < NCP; j++) {
        float r = 0.f;
        for (int i = 0; i < n4; i += 4) {
            const int4 d = *reinterpret_cast<const int4*>(&bid[i]);
            const float4 q = *reinterpret_cast<const float4*>(&bp[i]);
            r = d.x == x[j] ? q.x : r;
            r = d.y == x[j] ? q.y : r;
            r = d.z == x[j] ? q.z : r;
            r = d.w == x[j] ? q.w : r;
        }
        out[j] = r;
    }
    wsync();
}

// p of id q in the list (0 if absent)
__device__ float wget(const WList& l, int q) {
    bool hit[NCP];
#pragma unroll
    for (int j = 0; j < NCP; j++) hit[j] = l.id[j] == q;
    const int e = wfirst(hit, l.n);
    return e >= 0 ? entryf(l.p, e) : 0.f;
}

__device__ void wload(WList& l, const int* ids, const float* ps, int n) {
    const int lane = threadIdx.x;
    l.n = n;
#pragma unroll
    for (int j = 0; j < NCP; j++) {
        const int e = 64 * j + lane;
        l.id[j] = e < n ? ids[e] : -1;
        l.p[j] = e < n ? ps[e] : 0.f;
    }
}

__global__ __launch_bounds__(64) void k_sample_finish(SampCfg c, int mode, int jk, const int* __restrict__ rid,
                                                      const float* __restrict__ rv, const int* __restrict__ rn,
                                                      const float* __restrict__ lmax,
                                                      const float* __restrict__ sum, int* __restrict__ qid,
                                                      float* __restrict__ qp, int* __restrict__ qn, DState* st,
                                                      int* __restrict__ out, const float* __restrict__ uni,
                                                      int nuni) {
    const int lane = threadIdx.x;
    Uni rng{st->rng, uni, nuni, 0};
    if (mode == 0 || mode == 1) {  // Draft / Plain: distribution of row 0, one draw
        WList l = wsparse_dist(rid, rv, rn[0], lmax[0], sum[0], c);
        if (l.n == 0) wsingle(l, row_argmax(rid, rv, rn[0]));
        const int tok = wdraw(l, &rng);
        if (mode == 0) {
#pragma unroll
            for (int j = 0; j < NCP; j++) {
                const int e = 64 * j + lane;
                if (e < l.n) {
                    qid[jk * SPARSE_CAP + e] = l.id[j];
                    qp[jk * SPARSE_CAP + e] = l.p[j];
                }
            }
            if (lane == 0) {
                qn[jk] = l.n;
                st->drafts[jk] = tok;
            }
        } else if (lane == 0) {
            st->t_new = tok;
        }
        if (lane == 0) st->rng = rng.rng;
        return;
    }
    // Accept (spec_accept_or_correct_sparse, sampler.rs:683-711, per verify
    // row as pipeline.rs:3894-3934, then the loop-top sample of row a)
    const int k = jk;
    int a = 0, forced = -1;
    while (a < k) {
        const int* r_id = rid + (size_t)a * SPARSE_CAP;
        const float* r_v = rv + (size_t)a * SPARSE_CAP;
        WList p = wsparse_dist(r_id, r_v, rn[a], lmax[a], sum[a], c);
        if (p.n == 0) wsingle(p, row_argmax(r_id, r_v, rn[a]));
        const int d = st->drafts[a];
        WList q;
        wload(q, qid + a * SPARSE_CAP, qp + a * SPARSE_CAP, qn[a]);
        const float pd = wget(p, d), qd = wget(q, d);
        const float r = rng.next();
        if (qd > 0.f && r * qd < pd) {
            a++;
            continue;
        }
        // residual max(0, p - q) over p's support, in p's order
        float qv[NCP], ri[NCP], rpos[NCP];
        bool pos[NCP];
        wget_each(q, p.id, qv);
#pragma unroll
        for (int j = 0; j < NCP; j++) {
            ri[j] = 64 * j + lane < p.n ? p.p[j] - qv[j] : 0.f;
            pos[j] = 64 * j + lane < p.n && ri[j] > 0.f;
            rpos[j] = pos[j] ? ri[j] : 0.f;
        }
        float cum[NCP];
        wseq_prefix(rpos, p.n, cum);
        const float total = entryf(cum, p.n - 1);
        if (total <= 0.f) {
            forced = wdraw(p, &rng);
        } else {
            // the residual list: p's order, entries with ri > 0, ri / total
            float rn_[NCP];
#pragma unroll
            for (int j = 0; j < NCP; j++) rn_[j] = ri[j] / total;
            WList rs;
            wcompact(pos, p.id, rn_, p.n, rs);
            forced = wdraw(rs, &rng);
        }
        break;
    }
    int tnew = forced;
    if (forced < 0) {  // loop top: sample row a (sample_with_scratch_pool)
        const int* r_id = rid + (size_t)a * SPARSE_CAP;
        const float* r_v = rv + (size_t)a * SPARSE_CAP;
        const WList p = wsparse_dist(r_id, r_v, rn[a], lmax[a], sum[a], c);
        if (p.n > 0) tnew = wdraw(p, &rng);
        else tnew = row_argmax(r_id, r_v, rn[a]);
    }
    if (lane == 0) {
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
}

__global__ __launch_bounds__(64) void k_sample_dist(SampCfg c, const int* __restrict__ rid,
                                                    const float* __restrict__ rv, const int* __restrict__ rn,
                                                    const float* __restrict__ lmax, const float* __restrict__ sum,
                                                    int* __restrict__ ids, float* __restrict__ probs,
                                                    int* __restrict__ n_out) {
    const int lane = threadIdx.x;
    WList l = wsparse_dist(rid, rv, rn[0], lmax[0], sum[0], c);
    if (l.n == 0) wsingle(l, row_argmax(rid, rv, rn[0]));
#pragma unroll
    for (int j = 0; j < NCP; j++) {
        const int e = 64 * j + lane;
        if (e < l.n) {
            ids[e] = l.id[j];
            probs[e] = l.p[j];
        }
    }
    if (lane == 0) *n_out = l.n;
}

int sample_alloc(SampleBufs& b, int V, const std::function<int(void**, size_t)>& alloc) {
    b.V = V;
    b.nslices = (V + SLICE - 1) / SLICE;
    if (b.nslices > 256) return CMF_ERR;  // the merge's per-slice terms (vocab <= 1 048 576)
    const int R = MAXB + 1;
    const size_t nc = (size_t)R * b.nslices * SPARSE_K_MAX;
    if (alloc((void**)&b.cid, nc * 4) || alloc((void**)&b.cv, nc * 4) ||
        alloc((void**)&b.ocnt, (size_t)R * b.nslices * 4) ||
        alloc((void**)&b.oid, (size_t)R * b.nslices * SPARSE_CAP * 4) ||
        alloc((void**)&b.smax, (size_t)R * b.nslices * 4) || alloc((void**)&b.ssum, (size_t)R * b.nslices * 4) ||
        alloc((void**)&b.rid, (size_t)R * SPARSE_CAP * 4) || alloc((void**)&b.rv, (size_t)R * SPARSE_CAP * 4) ||
        alloc((void**)&b.rn, R * 4) || alloc((void**)&b.lmax, R * 4) || alloc((void**)&b.sum, R * 4) ||
        alloc((void**)&b.qid, 8 * SPARSE_CAP * 4) || alloc((void**)&b.qp, 8 * SPARSE_CAP * 4) ||
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
                       b.smax, b.ssum, b.ocnt, b.oid);
    hipLaunchKernelGGL(k_topk_merge, dim3(1), dim3(256), 0, s, V, c, b.nslices, b.cid, b.cv, b.smax, b.ssum,
                       b.ocnt, b.oid, b.rid, b.rv, b.rn, b.lmax, b.sum);
    hipLaunchKernelGGL(k_sample_dist, dim3(1), dim3(64), 0, s, c, b.rid, b.rv, b.rn, b.lmax, b.sum, ids, probs, n);
}

void sample_rows(SampleBufs& b, const float* logits, int V, int rows, const cmf_sampler_config& sc,
                 DState* st, SampleMode mode, int jk, int* out, hipStream_t s, int nuni) {
    const SampCfg c = samp_cfg(sc, V);
    hipLaunchKernelGGL(k_topk_slice, dim3(b.nslices, rows), dim3(256), 0, s, logits, V, c, b.nslices, b.cid,
                       b.cv, b.smax, b.ssum, b.ocnt, b.oid);
    hipLaunchKernelGGL(k_topk_merge, dim3(rows), dim3(256), 0, s, V, c, b.nslices, b.cid, b.cv, b.smax,
                       b.ssum, b.ocnt, b.oid, b.rid, b.rv, b.rn, b.lmax, b.sum);
    const int m = mode == SampleMode::Draft ? 0 : (mode == SampleMode::Plain ? 1 : 2);
    hipLaunchKernelGGL(k_sample_finish, dim3(1), dim3(64), 0, s, c, m, jk, b.rid, b.rv, b.rn, b.lmax, b.sum, b.qid,
                       b.qp, b.qn, st, out, b.uni, nuni);
}

}  // namespace cmf
