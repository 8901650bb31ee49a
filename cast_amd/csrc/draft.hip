// K5: drafter top-k marginals and best-first tree build on the device.
//
// Replaces the host half of a decode round's drafting:
//   topk_marginals (cast_trees/verify.py:8-12, used at serving.py:126-128):
//     log-softmax over the vocabulary, top-k per future position, then a
//     device-to-host copy per request;
//   build_tree (cast_trees/tree.py:29-49): a best-first heap over the
//     (L x k) candidates, run on the host per request.
// Ranking follows the reference's block_topk (tree.py:20-26): descending
// log-probability, equal values in increasing index order (a stable sort).
// Log-softmax is monotone, so that is the order of the raw logits.  The
// tree build reproduces the heap exactly: entries (-score, depth, parent,
// rank, counter) popped in tuple order, scores summed in double precision as
// the reference's Python floats are.
#include <float.h>

#include "cast_common.hpp"

namespace cast {

constexpr int kTopKMax = 16;

// (v1, i1) ranks before (v2, i2): larger value, then smaller index.
__device__ __forceinline__ bool ranks_before(float v1, int i1, float v2, int i2) {
    return v1 > v2 || (v1 == v2 && i1 < i2);
}

template <bool BF16>
__device__ __forceinline__ float logit_at(const char *row, int i) {
    if constexpr (BF16)
        return bf16_to_float(reinterpret_cast<const uint16_t *>(row)[i]);
    else
        return reinterpret_cast<const float *>(row)[i];
}

// One workgroup per row: top-k (value, index) and the row's log-sum-exp.
// Every thread keeps its best kTopKMax elements (a superset of its share of
// the row's top k) in a fully unrolled sorted list; k merge rounds then pick
// the row's top k.
template <bool BF16>
__global__ __launch_bounds__(256) void draft_topk_kernel(const void *__restrict__ logits, int64_t ld, int32_t vocab,
                                                         int32_t k, int64_t *__restrict__ top_idx,
                                                         float *__restrict__ top_lp) {
    constexpr int NT = 256, K = kTopKMax;
    const int row = blockIdx.x, tid = threadIdx.x;
    const char *base = static_cast<const char *>(logits) + (size_t)row * (size_t)ld * (BF16 ? 2 : 4);
    float tv[K];
    int ti[K];
#pragma unroll
    for (int j = 0; j < K; ++j) {
        tv[j] = -INFINITY;
        ti[j] = INT_MAX;   // empty slot
    }
    // pass 1: row maximum and the thread's sorted top-K.  Elements come in
    // increasing index order, so a new one goes behind equal values.
    float mx = -INFINITY;
    for (int i = tid; i < vocab; i += NT) {
        const float v = logit_at<BF16>(base, i);
        mx = fmaxf(mx, v);
        if (v > tv[K - 1] || ti[K - 1] == INT_MAX) {
            bool placed = false;
#pragma unroll
            for (int j = K - 1; j >= 0; --j) {
                const bool stays_ahead = j > 0 && !(v > tv[j - 1] || ti[j - 1] == INT_MAX);
                if (!placed) {
                    if (j == 0 || stays_ahead) {
                        tv[j] = v;
                        ti[j] = i;
                        placed = true;
                    } else {
                        tv[j] = tv[j - 1];
                        ti[j] = ti[j - 1];
                    }
                }
            }
        }
    }
    __shared__ float red[NT / 64];
    __shared__ double dred[NT / 64];
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off));
    if ((tid & 63) == 0) red[tid >> 6] = mx;
    __syncthreads();
    mx = red[0];
#pragma unroll
    for (int w = 1; w < NT / 64; ++w) mx = fmaxf(mx, red[w]);
    // pass 2: sum of exp(x - max), accumulated in double
    double sum = 0.0;
    for (int i = tid; i < vocab; i += NT) sum += (double)expf(logit_at<BF16>(base, i) - mx);
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) sum += __shfl_xor(sum, off);
    if ((tid & 63) == 0) dred[tid >> 6] = sum;
    __syncthreads();
    double tot = 0.0;
#pragma unroll
    for (int w = 0; w < NT / 64; ++w) tot += dred[w];
    const float log_sum = (float)log(tot);
    // k merge rounds over the threads' list heads
    __shared__ float hv[NT / 64];
    __shared__ int hi[NT / 64];
    for (int r = 0; r < k; ++r) {
        float bv = tv[0];
        int bi = ti[0];
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) {
            const float ov = __shfl_xor(bv, off);
            const int oi = __shfl_xor(bi, off);
            if (ranks_before(ov, oi, bv, bi)) {
                bv = ov;
                bi = oi;
            }
        }
        __syncthreads();
        if ((tid & 63) == 0) {
            hv[tid >> 6] = bv;
            hi[tid >> 6] = bi;
        }
        __syncthreads();
        bv = hv[0];
        bi = hi[0];
#pragma unroll
        for (int w = 1; w < NT / 64; ++w)
            if (ranks_before(hv[w], hi[w], bv, bi)) {
                bv = hv[w];
                bi = hi[w];
            }
        if (ti[0] == bi && bi != INT_MAX) {   // indices are disjoint across threads: one owner pops
#pragma unroll
            for (int j = 0; j < K - 1; ++j) {
                tv[j] = tv[j + 1];
                ti[j] = ti[j + 1];
            }
            tv[K - 1] = -INFINITY;
            ti[K - 1] = INT_MAX;
        }
        if (tid == 0) {
            top_idx[(size_t)row * k + r] = bi == INT_MAX ? -1 : bi;
            top_lp[(size_t)row * k + r] = (bv - mx) - log_sum;   // log_softmax: (x - max) - log(sum)
        }
    }
}

// ---- best-first tree build, one wave per request ----

struct Cand {
    double neg;     // -(path log-probability)
    int depth, parent, rank, cnt;
};

// the heap's order: smaller tuple (neg, depth, parent, rank, cnt) pops first
__device__ __forceinline__ bool pops_before(const Cand &a, const Cand &b) {
    if (a.neg != b.neg) return a.neg < b.neg;
    if (a.depth != b.depth) return a.depth < b.depth;
    if (a.parent != b.parent) return a.parent < b.parent;
    if (a.rank != b.rank) return a.rank < b.rank;
    return a.cnt < b.cnt;
}

constexpr int kPoolMax = kTopKMax * kMaxPack;   // candidates ever pushed: k * (1 + nodes)

template <typename LP>
__global__ __launch_bounds__(64) void build_trees_kernel(const int64_t *__restrict__ top_idx,
                                                         const LP *__restrict__ top_lp, int32_t L, int32_t k,
                                                         const int32_t *__restrict__ budget, int64_t *token,
                                                         int32_t *depth, int32_t *parent, double *score,
                                                         int32_t *n_nodes, int32_t *status) {
    __shared__ double pneg[kPoolMax];
    __shared__ int pmeta[kPoolMax];   // depth | parent << 8 | rank << 20 (depth < 256, parent < 4096, rank < 16)
    __shared__ unsigned char alive[kPoolMax];
    const int b = blockIdx.x, lane = threadIdx.x;
    const int64_t *ti = top_idx + (size_t)b * L * k;
    const LP *tl = top_lp + (size_t)b * L * k;
    int want = budget[b];
    if (want < 0 || want > kMaxPack - 1) {
        if (lane == 0) raise_flag(status, CAST_FLAG_BAD_PACK);
        want = want < 0 ? 0 : kMaxPack - 1;
    }
    int64_t *tok_o = token + (size_t)b * (kMaxPack - 1);
    int32_t *dep_o = depth + (size_t)b * (kMaxPack - 1);
    int32_t *par_o = parent + (size_t)b * (kMaxPack - 1);
    double *sc_o = score + (size_t)b * (kMaxPack - 1);
    // the k roots' children: depth 1, parent -1 (stored as parent + 1)
    int cnt = 0;
    if (lane < k) {
        pneg[lane] = -(double)tl[lane];
        pmeta[lane] = 1 | (0 << 8) | (lane << 20);
        alive[lane] = 1;
    }
    cnt = k;
    int nodes = 0;
    while (nodes < want) {
        // wave argmin over the alive candidates
        Cand best;
        best.neg = DBL_MAX;
        best.depth = INT_MAX;
        best.parent = INT_MAX;
        best.rank = INT_MAX;
        best.cnt = INT_MAX;
        __syncthreads();
        for (int c = lane; c < cnt; c += 64) {
            if (!alive[c]) continue;
            const int m = pmeta[c];
            const Cand x{pneg[c], m & 0xff, ((m >> 8) & 0xfff) - 1, m >> 20, c};
            if (pops_before(x, best)) best = x;
        }
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) {
            Cand o;
            o.neg = __shfl_xor(best.neg, off);
            o.depth = __shfl_xor(best.depth, off);
            o.parent = __shfl_xor(best.parent, off);
            o.rank = __shfl_xor(best.rank, off);
            o.cnt = __shfl_xor(best.cnt, off);
            if (pops_before(o, best)) best = o;
        }
        if (best.cnt == INT_MAX) break;   // heap empty
        const int me = nodes++;
        const int d = best.depth, r = best.rank;
        if (lane == 0) {
            alive[best.cnt] = 0;
            tok_o[me] = ti[(size_t)(d - 1) * k + r];
            dep_o[me] = d;
            par_o[me] = best.parent;
            sc_o[me] = -best.neg;
        }
        if (d < L) {
            // children: the reference pushes neg - top_lp[d, r2] for r2 in rank order
            if (lane < k && cnt + lane < kPoolMax) {
                pneg[cnt + lane] = best.neg - (double)tl[(size_t)d * k + lane];
                pmeta[cnt + lane] = (d + 1) | ((me + 1) << 8) | (lane << 20);
                alive[cnt + lane] = 1;
            }
            cnt += k;
            if (cnt > kPoolMax) cnt = kPoolMax;
        }
    }
    if (lane == 0) n_nodes[b] = nodes;
}

}  // namespace cast

using namespace cast;

extern "C" int cast_draft_topk(const void *logits, int64_t logits_ld, int32_t rows, int32_t vocab, int32_t dtype,
                               int32_t k, int64_t *top_idx, float *top_lp, cast_stream_t stream) {
    if (rows < 0 || vocab <= 0 || logits_ld < vocab || k < 1 || k > kTopKMax || k > vocab) return CAST_ERR_SHAPE;
    if (dtype != CAST_BF16 && dtype != CAST_FP32) return CAST_ERR_DTYPE;
    if (rows == 0) return CAST_OK;
    if (!logits || !top_idx || !top_lp) return CAST_ERR_NULL_POINTER;
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    if (dtype == CAST_BF16)
        draft_topk_kernel<true><<<rows, 256, 0, s>>>(logits, logits_ld, vocab, k, top_idx, top_lp);
    else
        draft_topk_kernel<false><<<rows, 256, 0, s>>>(logits, logits_ld, vocab, k, top_idx, top_lp);
    return hipGetLastError() == hipSuccess ? CAST_OK : CAST_ERR_HIP;
}

extern "C" int cast_build_trees(const int64_t *top_idx, const void *top_lp, int32_t lp_dtype, int32_t batch,
                                int32_t L, int32_t k, const int32_t *budget, int64_t *token, int32_t *depth,
                                int32_t *parent, double *score, int32_t *n_nodes, int32_t *status,
                                cast_stream_t stream) {
    if (batch < 0 || L < 1 || L > 255 || k < 1 || k > kTopKMax) return CAST_ERR_SHAPE;
    if (lp_dtype != CAST_FP32 && lp_dtype != CAST_FP64) return CAST_ERR_DTYPE;
    if (batch == 0) return CAST_OK;
    if (!top_idx || !top_lp || !budget || !token || !depth || !parent || !score || !n_nodes)
        return CAST_ERR_NULL_POINTER;
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    if (lp_dtype == CAST_FP32)
        build_trees_kernel<float><<<batch, 64, 0, s>>>(top_idx, static_cast<const float *>(top_lp), L, k, budget,
                                                       token, depth, parent, score, n_nodes, status);
    else
        build_trees_kernel<double><<<batch, 64, 0, s>>>(top_idx, static_cast<const double *>(top_lp), L, k,
                                                        budget, token, depth, parent, score, n_nodes, status);
    return hipGetLastError() == hipSuccess ? CAST_OK : CAST_ERR_HIP;
}
