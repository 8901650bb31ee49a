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

// BF16: 16-bit elements, of format E (Bf16 or Fp16); else float.
template <bool BF16, typename E = Bf16>
__device__ __forceinline__ float logit_at(const char *row, int i) {
    if constexpr (BF16)
        return E::widen(reinterpret_cast<const uint16_t *>(row)[i]);
    else
        return reinterpret_cast<const float *>(row)[i];
}

// Rank keys: (value, index) pairs as one unsigned 64-bit integer whose order
// is the ranking order (larger value first, equal values by smaller index):
// the value's order-preserving bits (-0 folded into +0) above the complement
// of the index.  NaN maps to 0, the empty key, which never ranks.
__device__ __forceinline__ uint64_t rank_key(float v, int i) {
    const uint32_t b = __builtin_bit_cast(uint32_t, v + 0.0f);   // -0 + 0 = +0
    const uint32_t ord = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
    return v == v ? (uint64_t)ord << 32 | (uint32_t)~(uint32_t)i : 0;
}
__device__ __forceinline__ float key_value(uint64_t key) {
    const uint32_t ord = (uint32_t)(key >> 32);
    return __builtin_bit_cast(float, (ord & 0x80000000u) ? (ord & 0x7fffffffu) : ~ord);
}
__device__ __forceinline__ int key_index(uint64_t key) { return (int)~(uint32_t)key; }

template <int CTRL, int ROW_MASK = 0xf>
__device__ __forceinline__ uint64_t key_max_dpp(uint64_t key) {   // lanes without a source keep their own
    const uint32_t lo = (uint32_t)__builtin_amdgcn_update_dpp((int)(uint32_t)key, (int)(uint32_t)key, CTRL, ROW_MASK,
                                                              0xf, false);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_update_dpp((int)(uint32_t)(key >> 32), (int)(uint32_t)(key >> 32),
                                                              CTRL, ROW_MASK, 0xf, false);
    const uint64_t o = (uint64_t)hi << 32 | lo;
    return o > key ? o : key;
}
__device__ __forceinline__ uint64_t lane_key(uint64_t key, int lane) {
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)key, lane);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(key >> 32), lane);
    return (uint64_t)hi << 32 | lo;
}
// the wave's largest key, in every lane
__device__ __forceinline__ uint64_t wave_key_max(uint64_t key) {
    key = key_max_dpp<0x111>(key);        // row_shr:1
    key = key_max_dpp<0x112>(key);        // row_shr:2
    key = key_max_dpp<0x114>(key);        // row_shr:4
    key = key_max_dpp<0x118>(key);        // row_shr:8
    key = key_max_dpp<0x142, 0xa>(key);   // row_bcast:15 into rows 1 and 3
    key = key_max_dpp<0x143, 0xc>(key);   // row_bcast:31 into rows 2 and 3
    return lane_key(key, 63);
}
// the largest key of lanes 0..15, in every lane
__device__ __forceinline__ uint64_t row_key_max(uint64_t key) {
    key = key_max_dpp<0x111>(key);
    key = key_max_dpp<0x112>(key);
    key = key_max_dpp<0x114>(key);
    key = key_max_dpp<0x118>(key);
    return lane_key(key, 15);
}

// Partial result of one (row, split) workgroup: its slice's top-k keys and
// the slice's log-sum-exp as (max, sum of exp(x - max)).
struct TopkPart {
    uint64_t key[kTopKMax];   // descending, 0 = empty
    double sum;
    float mx;                 // -inf for a slice without elements
    float pad;
};
constexpr int kTopkNT = 512;          // threads of a top-k workgroup
constexpr int kTopkBatch = 8;         // 16-byte chunks per thread per batch
constexpr int kTopkMaxSplits = 8;

// Rank selection over candidates held in LDS: every candidate (unique keys,
// 0 = none) counts the candidates above it, and a rank below k is its slot.
// Threads 0..n-1 hold one candidate each (cand[tid]); slots stay as set.
__device__ __forceinline__ void rank_select(const uint64_t *cand, int n, int k, uint64_t *slots) {
    const int tid = threadIdx.x;
    if (tid < n) {
        const uint64_t mine = cand[tid];
        int above = 0;
        for (int j = 0; j < n; ++j) above += cand[j] > mine ? 1 : 0;
        if (above < k && mine != 0) slots[above] = mine;
    }
}

// One wave per row: the splits' top-k lists and log-sum-exp partials into
// the row's top k and log probabilities (splits * k <= 64).  A kernel of its
// own: the launch boundary makes every part visible, where a last-workgroup
// ticket would need a device-scope release (an L2 write-back) per workgroup.
__global__ __launch_bounds__(64) void draft_topk_combine_kernel(const TopkPart *__restrict__ part, int32_t splits,
                                                                int32_t k, int64_t *__restrict__ top_idx,
                                                                float *__restrict__ top_lp) {
    __shared__ uint64_t cand[64];
    __shared__ uint64_t slots[kTopKMax];
    const int row = blockIdx.x, lane = threadIdx.x;
    const TopkPart *pp = part + (size_t)row * splits;
    top_idx += (size_t)row * k;
    top_lp += (size_t)row * k;
    const int n = splits * k;
    if (lane < kTopKMax) slots[lane] = 0;
    cand[lane] = lane < n ? pp[lane / k].key[lane % k] : 0;
    const float m = lane < splits ? pp[lane].mx : -INFINITY;
    float gm = m;
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) gm = fmaxf(gm, __shfl_xor(gm, off));
    double sum = lane < splits && m != -INFINITY ? pp[lane].sum * exp((double)m - (double)gm) : 0.0;
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) sum += __shfl_xor(sum, off);
    __syncthreads();
    rank_select(cand, n, k, slots);
    __syncthreads();
    if (lane < k) {
        const float log_sum = (float)log(sum);
        const uint64_t key = slots[lane];
        top_idx[lane] = key == 0 ? -1 : key_index(key);
        top_lp[lane] = key == 0 ? NAN : (key_value(key) - gm) - log_sum;
    }
}

// One workgroup per (row, split): top-k (value, index) and log-sum-exp of the
// split's slice of the row, elements [split * per_e, +per_e) (per_e a
// multiple of the 16-byte chunk).  With one split it writes the row's log
// probabilities; with several it writes a TopkPart for the combine kernel.
//
// Each thread keeps its best K rank keys (K >= k) in a fully unrolled sorted
// list.  Only elements whose key is at least a threshold key enter the lists.
// The threshold comes from the first batch (8 chunks per thread): the k-th
// largest of the NW * R best thread keys, R per wave (2 for k <= 8, 4 for
// k > 8), a bound no final top-k element of the slice falls below since at
// least k distinct elements are at or above it.  At k = 8 two per wave were
// measured faster than four (16.3 against 17.0 us); for k > 8 four per wave
// keep the threshold the k-th of 32 keys rather than of 16, which at k = 16
// would be the smallest of them.  A chunk whose max is below the threshold's
// value skips the per-element test.  The lists' entries are then compacted
// into LDS and ranked by counting (k rounds over the list heads when more
// than kTopkNT entries survive).
//
// Log-sum-exp: a running max per thread; a chunk's exp terms are summed
// pairwise in float onto the thread's float sum, which is rescaled only when
// the running max moves.  Workgroup and split sums are combined in double.
template <bool BF16, int K, typename E = Bf16>
__global__ __launch_bounds__(kTopkNT) void draft_topk_kernel(const void *__restrict__ logits, int64_t ld,
                                                             int32_t vocab, int32_t k, int32_t per_e,
                                                             TopkPart *__restrict__ part,
                                                             int64_t *__restrict__ top_idx,
                                                             float *__restrict__ top_lp) {
    constexpr int NT = kTopkNT, NW = NT / 64, NB = kTopkBatch;
    constexpr float kLog2e = 1.4426950408889634f;
    constexpr int EPC = BF16 ? 8 : 4;
    const int row = blockIdx.x, split = blockIdx.y, tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const char *base = static_cast<const char *>(logits) + (size_t)row * (size_t)ld * (BF16 ? 2 : 4);
    const int e0 = split * per_e;
    const int e1 = max(e0, min(vocab, e0 + per_e));   // an empty last split stays empty
    const bool vec = (reinterpret_cast<uintptr_t>(base) & 15) == 0;
    const int cb = vec ? e0 / EPC : 0, ce = vec ? e1 / EPC : 0;   // this split's whole chunks
    const int tail0 = vec ? ce * EPC : e0;                         // then elements [tail0, e1)

    uint64_t tk[K];   // descending; 0 = empty
#pragma unroll
    for (int j = 0; j < K; ++j) tk[j] = 0;
    uint64_t thr = 1;           // every key but NaN's passes
    float thr_v = -INFINITY;    // the threshold's value
    auto insert = [&](uint64_t key) __attribute__((always_inline)) {   // keys are unique
        if (key > tk[K - 1]) {
            bool placed = false;
#pragma unroll
            for (int j = K - 1; j >= 0; --j) {
                if (!placed) {
                    if (j == 0 || key < tk[j - 1]) {
                        tk[j] = key;
                        placed = true;
                    } else {
                        tk[j] = tk[j - 1];
                    }
                }
            }
        }
    };
    // running max mx; fsum holds sum(2^(x * log2e - ref2)) with ref2 the
    // rounded mx * log2e (0 while mx = -inf) and eps2 = mx * log2e - ref2
    // exactly, so fsum * 2^-eps2 = sum(exp(x - mx)).  One FMA per element
    // (the product is exact inside it), however large the logits.
    float mx = -INFINITY, ref2 = 0.f, eps2 = 0.f;
    float fsum = 0.f;
    auto lse_add = [&](const auto &v, float m) __attribute__((always_inline)) {   // m = max(v)
        constexpr int n = sizeof(v) / sizeof(float);
        if (m > mx) {   // a sum of -inf terms only is 0 (a NaN sum stays NaN)
            const float r = m * kLog2e;
            fsum *= mx == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(ref2 - r);
            eps2 = fmaf(m, kLog2e, -r);
            ref2 = r;
            mx = m;
        }
        float ex[n];
#pragma unroll
        for (int e = 0; e < n; ++e) ex[e] = __builtin_amdgcn_exp2f(fmaf(v[e], kLog2e, -ref2));
#pragma unroll
        for (int w = 1; w < n; w *= 2)   // pairwise
#pragma unroll
            for (int e = 0; e + w < n; e += 2 * w) ex[e] += ex[e + w];
        fsum += ex[0];
    };
    auto unpack = [&](const u32x4 &w, float (&v)[EPC]) __attribute__((always_inline)) {
#pragma unroll
        for (int e = 0; e < EPC; ++e) {
            const uint32_t bits = w[BF16 ? (e >> 1) : e];
            if constexpr (BF16 && __is_same(E, Fp16))
                v[e] = f16_to_float((uint16_t)(bits >> ((e & 1) * 16)));
            else
                v[e] = BF16 ? __builtin_bit_cast(float, (e & 1) ? (bits & 0xffff0000u) : (bits << 16))
                            : __builtin_bit_cast(float, bits);
        }
    };
    auto chunk_max = [&](const float (&v)[EPC]) __attribute__((always_inline)) {
        float m = fmaxf(fmaxf(v[0], v[1]), fmaxf(v[2], v[3]));
        if constexpr (EPC == 8) m = fmaxf(m, fmaxf(fmaxf(v[4], v[5]), fmaxf(v[6], v[7])));
        return m;
    };
    // the chunk's elements at or above the threshold's value, in index order;
    // the exact key test (ties at the threshold value pass up to its index)
    // is made at insertion
    auto filter = [&](const float (&v)[EPC], float m, int c) __attribute__((always_inline)) {
        if (m >= thr_v) {   // no element of the chunk passes otherwise
            uint32_t pm = 0;
#pragma unroll
            for (int e = 0; e < EPC; ++e) pm |= (v[e] >= thr_v ? 1u : 0u) << e;
            while (pm) {
                const int e = __builtin_ctz(pm);
                pm &= pm - 1;
                float ve = v[0];
#pragma unroll
                for (int e2 = 1; e2 < EPC; ++e2) ve = e == e2 ? v[e2] : ve;
                const uint64_t key = rank_key(ve, c * EPC + e);
                if (key >= thr) insert(key);
            }
        }
    };
    auto chunk = [&](const u32x4 &w, int c) __attribute__((always_inline)) {
        float v[EPC];
        unpack(w, v);
        const float m = chunk_max(v);
        lse_add(v, m);
        filter(v, m, c);
    };
    auto load_batch = [&](u32x4 (&w)[NB], int c0) __attribute__((always_inline)) {
#pragma unroll
        for (int u = 0; u < NB; ++u) w[u] = *reinterpret_cast<const u32x4 *>(base + (size_t)(c0 + u * NT) * 16);
    };

    constexpr int R = K > 8 ? 4 : 2;   // best keys taken per wave for the threshold
    __shared__ uint64_t thr_keys[NW * R];
    __shared__ uint64_t thr_pick;
    int c = cb + tid;
    u32x4 nxt[NB];
    if (ce - cb >= NB * NT) {   // first batch: the threshold, then the batch through it
        u32x4 w[NB];
        load_batch(w, c);
        if (c + NB * NT + (NB - 1) * NT < ce) load_batch(nxt, c + NB * NT);
        uint64_t best = 0;
#pragma unroll
        for (int u = 0; u < NB; ++u) {
            float v[EPC];
            unpack(w[u], v);
            const float m = chunk_max(v);
            lse_add(v, m);
            int fi = EPC - 1;   // the chunk's first element equal to its max
#pragma unroll
            for (int e = EPC - 2; e >= 0; --e) fi = v[e] == m ? e : fi;
            const uint64_t key = rank_key(m, (c + u * NT) * EPC + fi);
            best = key > best ? key : best;
        }
#pragma unroll
        for (int r = 0; r < R; ++r) {   // the wave's R best thread keys (unique keys: one owner)
            const uint64_t wb = wave_key_max(best);
            if (lane == 0) thr_keys[wv * R + r] = wb;
            if (best == wb) best = 0;
        }
        if (tid == 0) thr_pick = 0;
        __syncthreads();
        // the k-th largest of the NW * R keys (distinct, or 0): k distinct
        // real elements are at or above it
        if (tid < NW * R) {
            const uint64_t mine = thr_keys[tid];
            int above = 0;
#pragma unroll
            for (int j = 0; j < NW * R; ++j) above += thr_keys[j] > mine ? 1 : 0;
            if (above == k - 1) thr_pick = mine;
        }
        __syncthreads();
        const uint64_t t = thr_pick;
        if (t != 0) {   // k distinct real elements are at or above t
            thr = t;
            thr_v = key_value(t);
        }
#pragma unroll
        for (int u = 0; u < NB; ++u) {
            float v[EPC];
            unpack(w[u], v);
            filter(v, chunk_max(v), c + u * NT);
        }
        c += NB * NT;
    } else if (c + (NB - 1) * NT < ce) {
        load_batch(nxt, c);
    }
    // the rest in batches, the next batch loading while this one is consumed
    for (; c + (NB - 1) * NT < ce; c += NB * NT) {
        u32x4 w[NB];
#pragma unroll
        for (int u = 0; u < NB; ++u) w[u] = nxt[u];
        if (c + NB * NT + (NB - 1) * NT < ce) load_batch(nxt, c + NB * NT);
#pragma unroll
        for (int u = 0; u < NB; ++u) chunk(w[u], c + u * NT);
    }
    {   // the remainder, fewer than NB chunks per thread, in one round trip
        u32x4 w[NB];
#pragma unroll
        for (int u = 0; u < NB - 1; ++u)
            if (c + u * NT < ce) w[u] = *reinterpret_cast<const u32x4 *>(base + (size_t)(c + u * NT) * 16);
#pragma unroll
        for (int u = 0; u < NB - 1; ++u)
            if (c + u * NT < ce) chunk(w[u], c + u * NT);
    }
    for (int i = tail0 + tid; i < e1; i += NT) {
        const float v[1] = {logit_at<BF16, E>(base, i)};
        lse_add(v, v[0]);
        const uint64_t key = rank_key(v[0], i);
        if (key >= thr) insert(key);
    }

    // ---- the slice's log-sum-exp: max, then the sums rescaled to it
    __shared__ float red[NW];
    __shared__ double dred[NW];
    __shared__ int n_cand;
    __shared__ uint64_t cand[NT];
    __shared__ uint64_t topk[kTopKMax];
    if (tid == 0) n_cand = 0;
    if (tid < kTopKMax) topk[tid] = 0;
    float gm = mx;
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) gm = fmaxf(gm, __shfl_xor(gm, off));
    if (lane == 0) red[wv] = gm;
    __syncthreads();
    gm = red[0];
#pragma unroll
    for (int w = 1; w < NW; ++w) gm = fmaxf(gm, red[w]);
    double sum = mx == -INFINITY ? 0.0 : (double)fsum * (double)__builtin_amdgcn_exp2f((mx - gm) * kLog2e - eps2);
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) sum += __shfl_xor(sum, off);
    if (lane == 0) dred[wv] = sum;

    // ---- the slice's top k: the lists' entries compacted into LDS, ranked
    int mine = 0;
#pragma unroll
    for (int j = 0; j < K; ++j) mine += tk[j] != 0 ? 1 : 0;
    const int at = mine ? atomicAdd(&n_cand, mine) : 0;
    __syncthreads();
    const int n = n_cand;
    double tot = 0.0;
#pragma unroll
    for (int w = 0; w < NW; ++w) tot += dred[w];
    if (n <= NT) {
#pragma unroll
        for (int j = 0; j < K; ++j)
            if (j < mine) cand[at + j] = tk[j];
        __syncthreads();
        rank_select(cand, n, k, topk);
    } else {   // many survivors: k rounds over the list heads
        for (int r = 0; r < k; ++r) {
            uint64_t best = wave_key_max(tk[0]);
            if (lane == 0) cand[(r & 1) * NW + wv] = best;
            __syncthreads();
            best = row_key_max(lane < NW ? cand[(r & 1) * NW + lane] : 0);
            if (tk[0] == best && best != 0) {   // keys are unique: one owner pops
#pragma unroll
                for (int j = 0; j < K - 1; ++j) tk[j] = tk[j + 1];
                tk[K - 1] = 0;
            }
            if (tid == 0) topk[r] = best;
        }
    }
    __syncthreads();
    if (part) {
        TopkPart *pp = part + (size_t)row * gridDim.y + split;
        if (tid < kTopKMax) pp->key[tid] = topk[tid];
        if (tid == 0) {
            pp->sum = tot;
            pp->mx = gm;
        }
    } else if (tid < k) {
        const float log_sum = (float)log(tot);
        const uint64_t key = topk[tid];
        top_idx[(size_t)row * k + tid] = key == 0 ? -1 : key_index(key);
        top_lp[(size_t)row * k + tid] = key == 0 ? NAN : (key_value(key) - gm) - log_sum;   // (x - max) - log(sum)
    }
}

// ---- best-first tree build, one wave per request ----
//
// Heap entries are (neg, depth, parent, rank, cnt), popped in tuple order.
// (parent, rank) is unique, so cnt never decides and the order is
// (neg, key) with key = depth << 16 | (parent + 1) << 4 | rank compared
// unsigned.
//
// Sorted path (every position's log-probs non-increasing in rank, as top-k
// output is): a parent's children have keys neg_p - lp[d][r] that are
// non-decreasing in r (rounding is monotone) with ties to the smaller rank,
// so they pop in rank order and only each parent's next child can be the
// heap's minimum.  The frontier - one entry per parent with a next rank - is
// kept sorted across the wave, lane i holding the i-th smallest entry: a pop
// reads lane 0, and the popped entry's next sibling and the popped node's
// first child go in by two ballots and one three-way shift.  After pop i the
// frontier holds at most i + 2 entries and want - i - 1 pops remain, so it
// only outgrows 64 lanes once fewer than 64 pops remain, and entries pushed
// past lane 63 could never pop.
// Other inputs scan the pool of every pushed candidate (up to k per node).

constexpr int kLMax = 255;
constexpr int kPoolMax = kTopKMax * kMaxPack;   // candidates ever pushed: k * (1 + nodes)
constexpr uint32_t kDead = 0xffffffffu;

__device__ __forceinline__ uint32_t heap_key(int depth, int parent, int rank) {
    return (uint32_t)depth << 16 | (uint32_t)(parent + 1) << 4 | (uint32_t)rank;
}

// (n1, k1) pops before (n2, k2)
__device__ __forceinline__ bool pops_before(double n1, uint32_t k1, double n2, uint32_t k2) {
    return (n1 < n2) | ((n1 == n2) & (k1 < k2));   // bitwise: no short-circuit branches
}

// one DPP step of the argmin: combine with the lane CTRL names (lanes
// without a source keep their own value)
template <int CTRL, int ROW_MASK = 0xf>
__device__ __forceinline__ void argmin_dpp(double &neg, uint32_t &key) {
    const uint64_t nb = __builtin_bit_cast(uint64_t, neg);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_update_dpp((int)(uint32_t)nb, (int)(uint32_t)nb, CTRL, ROW_MASK, 0xf, false);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_update_dpp((int)(uint32_t)(nb >> 32), (int)(uint32_t)(nb >> 32), CTRL,
                                                              ROW_MASK, 0xf, false);
    const uint32_t ok = (uint32_t)__builtin_amdgcn_update_dpp((int)key, (int)key, CTRL, ROW_MASK, 0xf, false);
    const double on = __builtin_bit_cast(double, (uint64_t)hi << 32 | lo);
    const bool take = pops_before(on, ok, neg, key);
    neg = take ? on : neg;
    key = take ? ok : key;
}

// the wave's minimum (neg, key), in every lane: an inclusive scan over each
// row of 16 lanes (row_shr 1, 2, 4, 8), rows chained by row_bcast 15 and 31,
// lane 63 read out
__device__ __forceinline__ void wave_argmin(double &neg, uint32_t &key) {
    argmin_dpp<0x111>(neg, key);        // row_shr:1
    argmin_dpp<0x112>(neg, key);        // row_shr:2
    argmin_dpp<0x114>(neg, key);        // row_shr:4
    argmin_dpp<0x118>(neg, key);        // row_shr:8
    argmin_dpp<0x142, 0xa>(neg, key);   // row_bcast:15 into rows 1 and 3
    argmin_dpp<0x143, 0xc>(neg, key);   // row_bcast:31 into rows 2 and 3
    const uint64_t nb = __builtin_bit_cast(uint64_t, neg);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)nb, 63);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(nb >> 32), 63);
    key = (uint32_t)__builtin_amdgcn_readlane((int)key, 63);
    neg = __builtin_bit_cast(double, (uint64_t)hi << 32 | lo);
}

// a uniform lane's double
__device__ __forceinline__ double lane_value(double x, int lane) {
    const uint64_t xb = __builtin_bit_cast(uint64_t, x);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)xb, lane);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(xb >> 32), lane);
    return __builtin_bit_cast(double, (uint64_t)hi << 32 | lo);
}

// lane i receives lane i + 1's value (wave_shl:1; lane 63 keeps its own)
__device__ __forceinline__ uint32_t shift_down(uint32_t x) {
    return (uint32_t)__builtin_amdgcn_update_dpp((int)x, (int)x, 0x130, 0xf, 0xf, false);
}
__device__ __forceinline__ double shift_down(double x) {
    const uint64_t xb = __builtin_bit_cast(uint64_t, x);
    return __builtin_bit_cast(double, (uint64_t)shift_down((uint32_t)(xb >> 32)) << 32 | shift_down((uint32_t)xb));
}
// lane i receives lane i - 1's value (wave_shr:1; lane 0 keeps its own)
__device__ __forceinline__ uint32_t shift_up(uint32_t x) {
    return (uint32_t)__builtin_amdgcn_update_dpp((int)x, (int)x, 0x138, 0xf, 0xf, false);
}
__device__ __forceinline__ double shift_up(double x) {
    const uint64_t xb = __builtin_bit_cast(uint64_t, x);
    return __builtin_bit_cast(double, (uint64_t)shift_up((uint32_t)(xb >> 32)) << 32 | shift_up((uint32_t)xb));
}

template <typename LP>
__global__ __launch_bounds__(64) void build_trees_kernel(const int64_t *__restrict__ top_idx,
                                                         const LP *__restrict__ top_lp, int32_t L, int32_t k,
                                                         const int32_t *__restrict__ budget, int64_t *token,
                                                         int32_t *depth, int32_t *parent, double *score,
                                                         int32_t *n_nodes, int32_t *status) {
    __shared__ double stl[kLMax * kTopKMax];   // the request's [L][k] log-probs
    __shared__ double nscore[kMaxPack];         // popped nodes: score
    __shared__ uint32_t nkey[kMaxPack];         // popped nodes: heap_key
    __shared__ double pneg[kPoolMax];           // pool path: every pushed candidate
    __shared__ uint32_t pkey[kPoolMax];
    const int b = blockIdx.x, lane = threadIdx.x;
    const int64_t *ti = top_idx + (size_t)b * L * k;
    const LP *tl = top_lp + (size_t)b * L * k;
    int want = budget[b];
    if (want < 0 || want > kMaxPack - 1) {
        if (lane == 0) raise_flag(status, CAST_FLAG_BAD_PACK);
        want = want < 0 ? 0 : kMaxPack - 1;
    }
    // stage the log-probs; check that each position is sorted (NaN fails)
    const int n_lp = L * k;
    bool sorted = true;
    for (int i = lane; i < n_lp; i += 64) {
        const double v = (double)tl[i];
        stl[i] = v;
        if ((i % k) != k - 1) sorted = sorted && v >= (double)tl[i + 1];
    }
    sorted = __all(sorted);
    __syncthreads();
    int nodes = 0;
    if (sorted) {
        // lane i: the i-th smallest frontier entry (en, ek); dead entries
        // (+inf, kDead) sort last.  Popped node j's neg and key stay in lane
        // j & 63 of nn[j >> 6] / nk[j >> 6].
        double en = INFINITY;
        uint32_t ek = kDead;
        if (lane == 0) {   // the root's first child
            en = -stl[0];
            ek = heap_key(1, -1, 0);
        }
        double nn[2] = {0.0, 0.0};
        uint32_t nk[2] = {kDead, kDead};
        while (nodes < want) {
            const double bn = lane_value(en, 0);
            const uint32_t bk = (uint32_t)__builtin_amdgcn_readlane((int)ek, 0);
            if (bk == kDead) break;   // heap empty
            const int me = nodes++;
            const int d = (int)(bk >> 16), par = (int)((bk >> 4) & 0xfff) - 1, r = (int)(bk & 15);
            // a: the popped entry's next sibling; c: the popped node's first
            // child (uniform LDS reads, issued first; clamped in range)
            const bool has_a = r + 1 < k, has_c = d < L;
            const double v_a = stl[(d - 1) * k + min(r + 1, k - 1)];
            const double v_c = stl[min(d, L - 1) * k];
            const bool mine = lane == (me & 63);
            nn[0] = mine && me < 64 ? bn : nn[0];
            nk[0] = mine && me < 64 ? bk : nk[0];
            nn[1] = mine && me >= 64 ? bn : nn[1];
            nk[1] = mine && me >= 64 ? bk : nk[1];
            const double pn = lane_value(par < 64 ? nn[0] : nn[1], par & 63);   // the parent's neg
            double an = !has_a ? INFINITY : par < 0 ? -v_a : pn - v_a;   // roots push -lp, children neg_p - lp
            uint32_t ak = has_a ? heap_key(d, par, r + 1) : kDead;
            double cn = has_c ? bn - v_c : INFINITY;
            uint32_t ck = has_c ? heap_key(d + 1, me, 0) : kDead;
            const bool swap = pops_before(cn, ck, an, ak);
            const double n_lo = swap ? cn : an, n_hi = swap ? an : cn;
            const uint32_t k_lo = swap ? ck : ak, k_hi = swap ? ak : ck;
            // new positions: lo at pa, hi at pb + 1, counting the old entries 1..63 before each
            const int pa = __popcll(__ballot(lane >= 1 && pops_before(en, ek, n_lo, k_lo)));
            const int pb = __popcll(__ballot(lane >= 1 && pops_before(en, ek, n_hi, k_hi)));
            const double up_n = shift_down(en), dn_n = shift_up(en);
            const uint32_t up_k = shift_down(ek), dn_k = shift_up(ek);
            const bool s_up = lane < pa, s_lo = lane == pa, s_keep = lane <= pb, s_hi = lane == pb + 1;
            en = s_up ? up_n : s_lo ? n_lo : s_keep ? en : s_hi ? n_hi : dn_n;
            ek = s_up ? up_k : s_lo ? k_lo : s_keep ? ek : s_hi ? k_hi : dn_k;
        }
        // the nodes to LDS for the write-out below
        for (int j = 0; j < 2; ++j)
            if (j * 64 + lane < nodes) {
                nscore[j * 64 + lane] = -nn[j];
                nkey[j * 64 + lane] = nk[j];
            }
    } else {
        int cnt = 0;
        for (int r = lane; r < k; r += 64) {
            pneg[r] = -stl[r];
            pkey[r] = heap_key(1, -1, r);
        }
        cnt = k;
        while (nodes < want) {
            __syncthreads();
            double bn = INFINITY;
            uint32_t bk = kDead;
            int bc = -1;
            for (int c = lane; c < cnt; c += 64) {
                if (pkey[c] != kDead && pops_before(pneg[c], pkey[c], bn, bk)) {
                    bn = pneg[c];
                    bk = pkey[c];
                    bc = c;
                }
            }
            wave_argmin(bn, bk);
            if (bk == kDead) break;   // heap empty
            const int me = nodes++;
            const int d = (int)(bk >> 16);
            if (lane == 0) {
                nscore[me] = -bn;
                nkey[me] = bk;
            }
            if (bc >= 0 && pkey[bc] == bk) pkey[bc] = kDead;   // (parent, rank) is unique: one owner
            if (d < L) {
                // the reference pushes neg - lp[d][r2] for r2 in rank order
                for (int r = lane; r < k && cnt + r < kPoolMax; r += 64) {
                    pneg[cnt + r] = bn - stl[d * k + r];
                    pkey[cnt + r] = heap_key(d + 1, me, r);
                }
                cnt += k;
                if (cnt > kPoolMax) cnt = kPoolMax;
            }
        }
    }
    __syncthreads();
    // write the nodes out in pop order
    int64_t *tok_o = token + (size_t)b * (kMaxPack - 1);
    int32_t *dep_o = depth + (size_t)b * (kMaxPack - 1);
    int32_t *par_o = parent + (size_t)b * (kMaxPack - 1);
    double *sc_o = score + (size_t)b * (kMaxPack - 1);
    for (int i = lane; i < nodes; i += 64) {
        const uint32_t key = nkey[i];
        const int d = (int)(key >> 16), r = (int)(key & 15);
        tok_o[i] = ti[(d - 1) * k + r];
        dep_o[i] = d;
        par_o[i] = (int)((key >> 4) & 0xfff) - 1;
        sc_o[i] = nscore[i];
    }
    if (lane == 0) n_nodes[b] = nodes;
}

}  // namespace cast

using namespace cast;

// Splits per row: about one workgroup per CU (a workgroup's registers fill
// most of a CU), each split at least one first batch long, and
// splits * k <= 64 for the combine wave.
static int topk_splits(int32_t rows, int32_t vocab, int32_t dtype, int32_t k, int32_t want) {
    const int per_batch = kTopkBatch * kTopkNT * (dtype == CAST_FP32 ? 4 : 8);
    int cap = vocab / per_batch;
    cap = cap < 64 / k ? cap : 64 / k;
    cap = cap < kTopkMaxSplits ? cap : kTopkMaxSplits;
    if (cap < 1) cap = 1;
    int s = want > 0 ? want : 256 / rows;
    if (s < 1) s = 1;
    return s < cap ? s : cap;
}

extern "C" size_t cast_draft_topk_workspace_size(int32_t rows, int32_t vocab, int32_t dtype, int32_t k,
                                                 int32_t splits) {
    if (rows <= 0 || vocab <= 0 || k < 1 || k > kTopKMax) return 0;
    const int s = topk_splits(rows, vocab, dtype, k, splits);
    return s > 1 ? (size_t)rows * s * sizeof(TopkPart) : 0;
}

extern "C" int cast_draft_topk(const void *logits, int64_t logits_ld, int32_t rows, int32_t vocab, int32_t dtype,
                               int32_t k, int64_t *top_idx, float *top_lp, int32_t splits, void *workspace,
                               size_t workspace_bytes, cast_stream_t stream) {
    if (rows < 0 || vocab <= 0 || logits_ld < vocab || k < 1 || k > kTopKMax || k > vocab || splits < 0)
        return CAST_ERR_SHAPE;
    if (dtype != CAST_BF16 && dtype != CAST_FP16 && dtype != CAST_FP32) return CAST_ERR_DTYPE;
    if (rows == 0) return CAST_OK;
    if (!logits || !top_idx || !top_lp) return CAST_ERR_NULL_POINTER;
    const int ns = topk_splits(rows, vocab, dtype, k, splits);
    TopkPart *part = nullptr;
    if (ns > 1) {
        if (!workspace) return CAST_ERR_NULL_POINTER;
        if (workspace_bytes < (size_t)rows * ns * sizeof(TopkPart)) return CAST_ERR_WORKSPACE;
        if (reinterpret_cast<uintptr_t>(workspace) & 15) return CAST_ERR_ALIGNMENT;
        part = static_cast<TopkPart *>(workspace);
    }
    const int epc = dtype == CAST_FP32 ? 4 : 8;
    const int32_t per_e = (int32_t)(((int64_t)vocab + ns * epc - 1) / (ns * epc) * epc);
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    const dim3 grid(rows, ns);
    if (dtype == CAST_FP16 && k <= 8)
        draft_topk_kernel<true, 8, Fp16><<<grid, kTopkNT, 0, s>>>(logits, logits_ld, vocab, k, per_e, part, top_idx,
                                                                  top_lp);
    else if (dtype == CAST_FP16)
        draft_topk_kernel<true, kTopKMax, Fp16><<<grid, kTopkNT, 0, s>>>(logits, logits_ld, vocab, k, per_e, part,
                                                                         top_idx, top_lp);
    else if (dtype == CAST_BF16 && k <= 8)
        draft_topk_kernel<true, 8><<<grid, kTopkNT, 0, s>>>(logits, logits_ld, vocab, k, per_e, part, top_idx, top_lp);
    else if (dtype == CAST_BF16)
        draft_topk_kernel<true, kTopKMax><<<grid, kTopkNT, 0, s>>>(logits, logits_ld, vocab, k, per_e, part, top_idx,
                                                                   top_lp);
    else if (k <= 8)
        draft_topk_kernel<false, 8><<<grid, kTopkNT, 0, s>>>(logits, logits_ld, vocab, k, per_e, part, top_idx, top_lp);
    else
        draft_topk_kernel<false, kTopKMax><<<grid, kTopkNT, 0, s>>>(logits, logits_ld, vocab, k, per_e, part, top_idx,
                                                                    top_lp);
    if (ns > 1) draft_topk_combine_kernel<<<rows, 64, 0, s>>>(part, ns, k, top_idx, top_lp);
    return hipGetLastError() == hipSuccess ? CAST_OK : CAST_ERR_HIP;
}

extern "C" int cast_build_trees(const int64_t *top_idx, const void *top_lp, int32_t lp_dtype, int32_t batch,
                                int32_t L, int32_t k, const int32_t *budget, int64_t *token, int32_t *depth,
                                int32_t *parent, double *score, int32_t *n_nodes, int32_t *status,
                                cast_stream_t stream) {
    if (batch < 0 || L < 1 || L > kLMax || k < 1 || k > kTopKMax) return CAST_ERR_SHAPE;
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
