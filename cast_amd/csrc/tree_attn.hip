// K2: ragged ancestor-masked tree-verification attention for gfx950.
//
// Replaces cast_trees/tree_attn.py (Triton _tree_attn_fwd, lines 17-92, and
// its host schedule/launch, lines 104-139) with the same visibility rule:
// a packed row of request b sees every prefix key [0, S_b) and pack key j iff
// bit j of its ancestor words is set (tree_attn.py:73-75); query head h reads
// KV head h / (Hq/Hkv) (tree_attn.py:30); fully masked rows give 0
// (tree_attn.py:62,89).
//
// Work unit: (request b, KV head h, key split s, row block rb).  The Q rows of
// a unit are the pack's tokens times the GQA group (row r = token*G + g), so
// one KV head's keys are streamed from HBM once per split and shared by
// G*P_b query rows.  bf16 or fp16 with head_dim 64/128/256 runs on MFMA:
//   S^T = K Q^T with v_mfma_f32_32x32x16_bf16 (_f16 for fp16 inputs; keys
//   on the M side, queries on the N side, so each lane ends up owning one
//   query column), then
//   O^T += V^T P^T with the same instruction, P^T taken straight from the
//   S^T accumulator registers (a lane's 16 score values are exactly the 8+8
//   k-slots it must supply), V^T read from a transposed LDS copy.  fp32
//   inputs with head_dim 64/128/256 run the same structure on
//   v_mfma_f32_32x32x2_f32 (tree_attn_f32_kernel); other head dims (up to
//   256) take a scalar kernel.  Head_dim 256 runs one wave per SIMD (512
//   registers a lane).
// K/V tiles of 64 keys (32 for fp32 at head_dim 256) are double-buffered
// through LDS with 16-byte loads; the ancestor words are only consulted on
// the tile(s) holding pack keys, and pack tiles past the last key any row
// of a workgroup sees are skipped.
// The online softmax works in base 2 with a lazy rescale: the running max
// moves only when a tile raises it by more than 2^8, so most tiles skip the
// O rescale.  Every workgroup decodes its unit from the device-side metadata
// (batches of up to 64 requests: longest key splits first, per XCD).  Long
// prefixes are split over keys; a combine kernel merges the per-split
// (O, lse) pairs by log-sum-exp.
#include <limits.h>
#include <math.h>

#include <mutex>
#include <type_traits>

#include "cast_common.hpp"

namespace cast {

constexpr int kNoSplit = 1 << 30;        // chunk value meaning "one split"
constexpr float kLn2 = 0.69314718055994530942f;
constexpr float kLog2e = 1.44269504088896340736f;
constexpr float kRescaleSlack = 8.0f;    // log2 headroom before the O rescale
constexpr int kCombineFast = 4;          // splits the combine loads in one round trip
constexpr int kCombineLdsSplits = 64;    // more splits: per-head weights in LDS up to this many
constexpr int kCombineLdsHeads = 64;     //   and this many heads per combine workgroup
constexpr int kCombineUnroll = 8;        // partial loads in flight per thread
// Smallest automatic split-K chunk (keys).  Short prefixes with few (request,
// head) units split down to two 64-key tiles per workgroup: a single request
// at S=2048, P=16 takes 24.7 us per call at 128 keys against 32.3 us at 512.
constexpr int kMinChunk = 128;
constexpr int kQkAhead = 4;   // K and V^T operand reads in flight ahead of their MFMAs

// Where the keys and values of request b, KV head h live.  Two layouts:
//  concat (store == 0): one ragged [total_kv, Hkv, D] tensor per K and V;
//      request b owns rows [cu_kv[b], cu_kv[b+1]) = concat(prefix, pack)
//      (cast_trees/tree_attn.py:71).  pre == pack, pre_b unused.
//  store (store == 1): the prefix stays in a per-request store
//      [B, Hkv, cap, D] (cast_trees/serving.py:191-205), key t of request b
//      at pre + b*pre_b + h*pre_h + t*pre_t; the pack comes from the
//      forward's own K/V [Hkv, total_q, D], key j at
//      pack + h*pack_h + (cu_q[b] + j)*pack_t.
struct KvSource {
    const void *k_pre, *v_pre, *k_pack, *v_pack;
    int64_t kpre_b, kpre_h, kpre_t, vpre_b, vpre_h, vpre_t;
    int64_t kpack_h, kpack_t, vpack_h, vpack_t;
    int32_t store, cap;
};

struct AttnArgs {
    const void *q;
    KvSource kv;
    void *out;
    float *lse;
    const int32_t *cu_q, *cu_kv, *prefix_len, *pack_len;
    const uint64_t *mask;
    int32_t mask_words;
    int32_t batch, total_q, total_kv, Hq, Hkv, G;
    int32_t D, esz;     // head dim, bytes per element of q/out
    int64_t q_tok, q_head, o_tok, o_head;
    float scale_log2;   // sm_scale * log2(e)
    int32_t chunk;      // keys per split, multiple of 64 (kNoSplit = no split)
    int32_t max_rows;   // longest key source (rows) the MFMA kernel can address
    int32_t xcds;       // XCDs of the device: workgroup x runs on XCD x % xcds
    int32_t sk_mode;    // stream-K schedule asked for (CAST_SPLIT_STREAM)
    int32_t sk_wgs;     // stream-K workgroups (resident at once; a multiple of 2 * xcds)
    int32_t sk_min_tiles;   // shortest stream-K lane (key tiles)
    float *sk_lse;      // stream-K partial lse [2 * sk_wgs][rows_wg] (partial O at part_o)
    int32_t rows_wg;    // query rows per workgroup
    int32_t comb_groups;  // combine kernel: head groups per packed token
    float *part_o;      // [part_rows][Hq][D] fp32, normalised partial outputs
    float *part_lse;    // [part_rows][Hq]    fp32, base-2 partial lse
    int64_t part_rows;
    int32_t *status;
};

// Per-request geometry shared by the attention and combine kernels.
struct Seq {
    int b, S, P, T, q0, kv0, ns, rb, split_len;
    int64_t part_off;   // first partial row of this request (only if ns > 1)
};

// Reads and checks request b's metadata; `report` raises the device flags.
__device__ __forceinline__ bool load_seq(const AttnArgs &a, int b, Seq &s, bool report) {
    const int S = a.prefix_len[b], P = a.pack_len[b];
    const int q0 = a.cu_q[b], q1 = a.cu_q[b + 1];
    int kv0 = 0, kv1 = S + P;
    bool bad_kv;
    if (a.kv.store) {
        bad_kv = S > a.kv.cap;
    } else {
        kv0 = a.cu_kv[b];
        kv1 = a.cu_kv[b + 1];
        bad_kv = kv0 < 0 || kv1 > a.total_kv || kv1 - kv0 != S + P;
    }
    if ((a.kv.store ? max(S, P) : S + P) > a.max_rows) {
        if (report) raise_flag(a.status, CAST_FLAG_TOO_LONG);
        return false;
    }
    if (S < 0 || q0 < 0 || q1 > a.total_q || q1 - q0 != P || bad_kv) {
        if (report) raise_flag(a.status, CAST_FLAG_BAD_OFFSETS);
        return false;
    }
    if (P < 0 || P > 64 * a.mask_words) {
        if (report) raise_flag(a.status, CAST_FLAG_BAD_PACK);
        return false;
    }
    s.b = b;
    s.S = S;
    s.P = P;
    s.T = S + P;
    s.q0 = q0;
    s.kv0 = kv0;
    s.ns = P == 0 ? 0 : (s.T + a.chunk - 1) / a.chunk;
    s.rb = (P * a.G + a.rows_wg - 1) / a.rows_wg;
    const int per = s.ns ? (s.T + s.ns - 1) / s.ns : 0;
    s.split_len = (per + 63) & ~63;
    return true;
}

// ---- batch lookups.  A wave walks the batch 64 requests at a time, lane j
// holding request b0 + j, with wave prefix sums over the lanes, so that a
// lookup costs one round of metadata loads per 64 requests.

// lane src's value in every lane, as a scalar (src wave-uniform)
__device__ __forceinline__ int bcast(int x, int src) { return __builtin_amdgcn_readlane(x, src); }
__device__ __forceinline__ int64_t bcast64(int64_t x, int src) {
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)x, src);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(x >> 32), src);
    return (int64_t)(((uint64_t)hi << 32) | lo);
}
// Inclusive scan over the 64 lanes of non-negative int32 values, saturating
// at INT32_MAX (so inconsistent metadata can never wrap a sum to a small
// value).  DPP row shifts build 16-lane scans, row broadcasts join them: all
// VALU, no LDS round trips.
__device__ __forceinline__ int wave_scan(int x) {
    auto add = [](int a, int b) { return (int)min((uint32_t)a + (uint32_t)b, 0x7fffffffu); };
    x = add(x, __builtin_amdgcn_update_dpp(0, x, 0x111, 0xf, 0xf, false));   // row_shr:1
    x = add(x, __builtin_amdgcn_update_dpp(0, x, 0x112, 0xf, 0xf, false));   // row_shr:2
    x = add(x, __builtin_amdgcn_update_dpp(0, x, 0x114, 0xf, 0xf, false));   // row_shr:4
    x = add(x, __builtin_amdgcn_update_dpp(0, x, 0x118, 0xf, 0xf, false));   // row_shr:8
    x = add(x, __builtin_amdgcn_update_dpp(0, x, 0x142, 0xa, 0xf, false));   // row_bcast:15 into rows 1, 3
    x = add(x, __builtin_amdgcn_update_dpp(0, x, 0x143, 0xc, 0xf, false));   // row_bcast:31 into rows 2, 3
    return x;
}
// The saturated sum of x over the wave, in every lane.
__device__ __forceinline__ int wave_sum(int x) { return bcast(wave_scan(x), 63); }

__device__ __forceinline__ Seq shfl_seq(const Seq &t, int src) {
    Seq s;
    s.b = bcast(t.b, src);
    s.S = bcast(t.S, src);
    s.P = bcast(t.P, src);
    s.T = bcast(t.T, src);
    s.q0 = bcast(t.q0, src);
    s.kv0 = bcast(t.kv0, src);
    s.ns = bcast(t.ns, src);
    s.rb = bcast(t.rb, src);
    s.split_len = bcast(t.split_len, src);
    return s;
}

// Work items are ordered (b, h, split, row block) with the row block fastest.
__device__ __forceinline__ int sat32(int64_t v) { return (int)min(v, (int64_t)0x7fffffff); }
__device__ __forceinline__ int items_of(const AttnArgs &a, const Seq &t) { return sat32((int64_t)a.Hkv * t.ns * t.rb); }

// Totals over the requests that pass load_seq (work items, key rows, query
// rows), and whether any request failed it.  Wave 0 of the workgroup reports
// invalid requests.
struct BatchTotals {
    int64_t items, kv_sum, q_sum;
    bool bad;          // some request failed load_seq
    bool unordered;    // cu_q decreases somewhere: accepted packs might overlap
};

// Adds the 64 requests b0 + lane (lane holding request b, ok when it passed
// load_seq) to the totals.
__device__ __forceinline__ void add_totals(BatchTotals &r, const AttnArgs &a, int b, bool ok, const Seq &t) {
    r.items += wave_sum(ok ? items_of(a, t) : 0);
    r.kv_sum += wave_sum(ok ? t.T : 0);
    r.q_sum += wave_sum(ok ? t.P : 0);
    r.bad |= __ballot(b < a.batch && !ok) != 0;
    r.unordered |= __ballot(b < a.batch && a.cu_q[b + 1] < a.cu_q[b]) != 0;
}

__device__ BatchTotals batch_totals(const AttnArgs &a) {
    const int lane = threadIdx.x & 63;
    BatchTotals r{0, 0, 0, false, false};
    for (int b0 = 0; b0 < a.batch; b0 += 64) {
        const int b = b0 + lane;
        Seq t{};
        const bool ok = b < a.batch && load_seq(a, b, t, threadIdx.x < 64);
        add_totals(r, a, b, ok, t);
    }
    return r;
}

// total_q and total_kv are host-side bounds that sized the grid and the
// workspace.  Accepted requests whose rows or keys add up past them overlap
// (or the store layout's bound is too small), and a decreasing cu_q lets
// packs overlap: such a batch is rejected whole.  Otherwise the accepted
// packs are disjoint row ranges.
__device__ __forceinline__ bool batch_fits(const AttnArgs &a, const BatchTotals &t) {
    if (t.kv_sum > a.total_kv || t.q_sum > a.total_q || t.unordered) {
        if (threadIdx.x == 0) raise_flag(a.status, CAST_FLAG_BAD_OFFSETS);
        return false;
    }
    return true;
}

__device__ bool find_request(const AttnArgs &a, int64_t w, bool by_token, Seq &s, int &local);

// Rows that no accepted request owns - those of rejected requests, rows
// outside every request, or all rows of a rejected batch - get zeros and
// lse = -inf, so an inconsistent call never returns uninitialised memory.
// Every wave of the grid takes a share of the packed rows; the kernels call
// this only when some request was rejected or the accepted ones leave rows
// uncovered.
__device__ void fill_unowned_rows(const AttnArgs &a, bool batch_ok) {
    const int lane = threadIdx.x & 63;
    const int waves = blockDim.x >> 6;
    const int64_t first = (int64_t)blockIdx.x * waves + (threadIdx.x >> 6);
    const int64_t stride = (int64_t)gridDim.x * waves;
    const int n = a.Hq * a.D;
    for (int64_t t = first; t < a.total_q; t += stride) {
        Seq s;
        int local;
        if (batch_ok && find_request(a, t, true, s, local)) continue;
        char *row = static_cast<char *>(a.out) + t * a.o_tok * a.esz;
        for (int e = lane; e < n; e += 64) {
            char *p = row + ((int64_t)(e / a.D) * a.o_head + e % a.D) * a.esz;
            if (a.esz == 2)
                *reinterpret_cast<uint16_t *>(p) = 0;
            else
                *reinterpret_cast<float *>(p) = 0.f;
        }
        if (a.lse)
            for (int h = lane; h < a.Hq; h += 64) a.lse[t * a.Hq + h] = -INFINITY;
    }
}

// The start of every attention kernel: the batch totals, the fill of
// unowned rows when needed; false when the batch is rejected whole.
__device__ bool batch_prologue(const AttnArgs &a, const BatchTotals &t) {
    const bool ok = batch_fits(a, t);
    if (!ok || t.bad || t.q_sum != a.total_q) fill_unowned_rows(a, ok);
    return ok;
}

// The request holding work item w (or, with by_token, packed row w), with its
// first partial row; local = w's index
// within the request.  Wave-uniform result.
__device__ bool find_request(const AttnArgs &a, int64_t w, bool by_token, Seq &s, int &local) {
    const int lane = threadIdx.x & 63;
    int64_t items = 0, part = 0;
    for (int b0 = 0; b0 < a.batch; b0 += 64) {
        const int b = b0 + lane;
        Seq t{};
        const bool ok = b < a.batch && load_seq(a, b, t, false);
        const int n = ok ? items_of(a, t) : 0;
        const int pp = ok && t.ns > 1 ? sat32((int64_t)t.ns * t.P) : 0;
        const int n_in = wave_scan(n), p_in = wave_scan(pp);
        const int64_t start = by_token ? (ok ? t.q0 : 0) : items + n_in - n;
        const int64_t len = by_token ? (ok ? t.P : 0) : n;
        const uint64_t hit = __ballot(ok && w >= start && w < start + len);
        if (hit) {
            const int src = __builtin_amdgcn_readfirstlane(__builtin_ctzll(hit));
            s = shfl_seq(t, src);
            s.part_off = part + bcast(p_in - pp, src);
            local = (int)(w - bcast64(start, src));
            return true;
        }
        items += bcast(n_in, 63);
        part += bcast(p_in, 63);
    }
    return false;
}

// ---- longest-first schedule (batches of up to 64 requests).  Work is
// grouped per (request, KV head, key split); a group's rb row blocks read
// the same keys.  Groups are ranked by keys per group (split_len) in
// descending order and dealt to the nx XCDs round-robin (workgroup x runs on
// XCD x % nx), each group's row blocks taking consecutive slots of one XCD so
// that they share its L2.  Within an XCD workgroups start in slot order, so
// each XCD works through its groups longest first (a greedy longest-
// processing-time schedule): short groups fill in behind long ones instead
// of trailing alone.  Every group has R = the batch's largest rb slots;
// slots past a request's own rb exit at once.

// Slot count of the longest-first grid: every one of the nx XCDs holds at
// most ceil(groups / nx) groups of at most rbmax row blocks each.
__host__ __device__ __forceinline__ int64_t sorted_slots(int64_t groups, int64_t rbmax, int nx) {
    return ((groups + nx - 1) / nx) * nx * rbmax;
}

// The (request, KV head, split, row block) of slot x, or false for an empty
// slot.  Requires batch <= 64: lane j holds request j (t, and loaded when it
// passed load_seq).  XCD x % nx takes every nx-th group of the longest-first
// order, and its slots are those groups' row blocks, packed densely in that
// order.  Wave-uniform result.
__device__ bool locate_sorted(const AttnArgs &a, int64_t x, const Seq &t, bool loaded, Seq &s, int &h, int &split,
                              int &rblk) {
    const int lane = threadIdx.x & 63;
    const bool ok = loaded && t.ns > 0;
    // partial-row offsets stay in batch order (the combine kernel's order)
    const int pp = ok && t.ns > 1 ? sat32((int64_t)t.ns * t.P) : 0;
    const int p_excl = wave_scan(pp) - pp;
    // rank key: keys per group descending, then request index (all distinct)
    const uint32_t key = ok ? ((uint32_t)((1 << 24) - 1 - t.split_len) << 6) | (uint32_t)lane : 0xffffffffu;
    const int ng = ok ? a.Hkv * t.ns : 0;                 // this request's groups
    // groups ahead of this request in longest-first order
    int off = 0;
    for (int j = 0; j < a.batch; ++j) {
        const uint32_t kj = (uint32_t)__builtin_amdgcn_readlane((int)key, j);
        const int nj = __builtin_amdgcn_readlane(ng, j);
        off += kj < key ? nj : 0;
    }
    // its groups dealt to this XCD (g in [off, off + ng), g % nx == xcd), and
    // the slots they take there
    const int nx = a.xcds;
    const int xcd = (int)(x % nx);
    const int k = (int)(x / nx);
    auto on_xcd = [xcd, nx](int n) { return (n + nx - 1 - xcd) / nx; };   // #g in [0, n) with g % nx == xcd
    const int slots = ok ? (on_xcd(off + ng) - on_xcd(off)) * t.rb : 0;
    int start = 0;
    for (int j = 0; j < a.batch; ++j) {
        const uint32_t kj = (uint32_t)__builtin_amdgcn_readlane((int)key, j);
        const int sj = __builtin_amdgcn_readlane(slots, j);
        start += kj < key ? sj : 0;
    }
    const uint64_t hit = __ballot(slots > 0 && k >= start && k < start + slots);
    if (!hit) return false;
    const int b = __builtin_amdgcn_readfirstlane(__builtin_ctzll(hit));
    s = shfl_seq(t, b);
    s.part_off = bcast(p_excl, b);
    const int kk = k - bcast(start, b);
    const int off_b = bcast(off, b);
    const int g = off_b + ((xcd - off_b) % nx + nx) % nx + nx * (kk / s.rb);   // the (kk / rb)-th of its groups here
    const int local = g - off_b;
    h = local / s.ns;
    split = local % s.ns;
    rblk = kk % s.rb;
    return true;
}

// Base pointers and token strides of the prefix and pack keys of one
// (request, KV head); key kk < S is prefix key kk, key kk >= S pack key kk - S.
template <typename T>
struct KvView {
    const T *kpre, *kpack, *vpre, *vpack;
    int64_t kpre_t, kpack_t, vpre_t, vpack_t;

    __device__ __forceinline__ KvView(const KvSource &src, const Seq &s, int h) {
        const T *kp = static_cast<const T *>(src.k_pre), *vp = static_cast<const T *>(src.v_pre);
        kpre_t = src.kpre_t;
        vpre_t = src.vpre_t;
        if (src.store) {
            kpre = kp + (int64_t)s.b * src.kpre_b + (int64_t)h * src.kpre_h;
            vpre = vp + (int64_t)s.b * src.vpre_b + (int64_t)h * src.vpre_h;
            kpack = static_cast<const T *>(src.k_pack) + (int64_t)s.q0 * src.kpack_t + (int64_t)h * src.kpack_h;
            vpack = static_cast<const T *>(src.v_pack) + (int64_t)s.q0 * src.vpack_t + (int64_t)h * src.vpack_h;
            kpack_t = src.kpack_t;
            vpack_t = src.vpack_t;
        } else {
            kpre = kp + (int64_t)s.kv0 * kpre_t + (int64_t)h * src.kpre_h;
            vpre = vp + (int64_t)s.kv0 * vpre_t + (int64_t)h * src.vpre_h;
            kpack = kpre + (int64_t)s.S * kpre_t;
            vpack = vpre + (int64_t)s.S * vpre_t;
            kpack_t = kpre_t;
            vpack_t = vpre_t;
        }
    }
    __device__ __forceinline__ const T *key(int kk, int S) const {
        return kk < S ? kpre + (int64_t)kk * kpre_t : kpack + (int64_t)(kk - S) * kpack_t;
    }
    __device__ __forceinline__ const T *val(int kk, int S) const {
        return kk < S ? vpre + (int64_t)kk * vpre_t : vpack + (int64_t)(kk - S) * vpack_t;
    }
};

__device__ __forceinline__ bool pack_bit(int j, uint64_t w0, uint64_t w1) {
    const uint64_t w = j < 64 ? w0 : w1;
    return (w >> (j & 63)) & 1ull;
}

// --------------------------------------------------------------------------
// MFMA kernel: bf16 or fp16, head_dim D in {64, 128, 256}, WAVES waves x 32
// query rows.
// --------------------------------------------------------------------------

// Bits [j0, j0+32) of the 192-bit string {w1 : w0 : 64 ones}, read from bit
// j0 + 64: pack-relative key positions j < 0 are prefix keys (all visible),
// j in [0, 128) are the row's ancestor bits.  Requires -64 <= j0 < 128.
__device__ __forceinline__ uint32_t vis_window(uint64_t w0, uint64_t w1, int j0) {
    const int p = j0 + 64;
    const int q = p >> 6, r = p & 63;
    const uint64_t lo = q == 0 ? ~0ull : (q == 1 ? w0 : w1);
    const uint64_t hi = q == 0 ? w0 : (q == 1 ? w1 : 0ull);
    const uint64_t v = (lo >> r) | (r ? hi << (64 - r) : 0ull);
    return (uint32_t)v;
}

// The highest pack key that ancestor words (w0, w1) make visible, or -1.
__device__ __forceinline__ int last_visible(uint64_t w0, uint64_t w1) {
    return w1 ? 127 - __builtin_clzll(w1) : (w0 ? 63 - __builtin_clzll(w0) : -1);
}

// Whether any row of the wave sees a key of the 32-key block that starts at
// pack key j0, of which the first `lim` keys are real.  A block that no row
// sees adds exact zeros to every row's sum and output, so it can be skipped.
__device__ __forceinline__ bool block_live(uint64_t w0, uint64_t w1, int j0, int lim) {
    uint32_t vis = vis_window(w0, w1, j0);
    vis &= lim >= 32 ? ~0u : (lim <= 0 ? 0u : ((1u << lim) - 1u));
    return __any(vis != 0u);
}

// What the MFMA kernel's epilogue needs, parked in LDS during the key loop
// so that it holds no scalar registers there.
struct EpiArgs {
    void *out;
    float *lse, *part_o, *part_lse, *sk_lse;
    int32_t *status;
    int64_t o_tok, o_head, part_rows;
    int64_t prow0;      // static partial row of token q0 + i is prow0 + q0 + i
    int32_t slot;       // stream-K partial slot (-1: static)
    int32_t final_out, Hq;
};

// Raw buffer resource over `rows` key rows of `row_bytes` stride and
// `width` bytes each, from base: loads at offsets past the last row's end
// return zeros.  The caller keeps rows * row_bytes below 2^31.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t seg_rsrc(const void *base, int rows, uint32_t row_bytes,
                                                           uint32_t width) {
    const uint32_t bytes = rows > 0 ? (uint32_t)(rows - 1) * row_bytes + width : 0u;
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), 0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ u32x4 load16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0));
}

// ---- stream-K schedule ("lanes"), batches of up to 64 requests.  The
// static schedule above cuts every request into equal key splits; when the
// requests' lengths differ, its longest item sets the call's time while
// other CUs idle.  Stream-K gives every lane the same number of key tiles
// instead:
//  - a lane is two workgroups on one XCD (x and x + xcds);
//  - the units of request b - (KV head h, row block r), unit index
//    k = h * rb + r - are paired into super-groups (2s, 2s + 1): the two row
//    blocks of one head (they read the same keys, which the lane's two
//    workgroups then share through the XCD's L2), or two heads when a head
//    has one row block;
//  - a super-group is tiles_b lane-steps (the request's key tiles: its
//    prefix in 64-key tiles, then its pack); the super-groups of all
//    requests, in batch order, make a line of C lane-steps, and lane l takes
//    steps [l * L, (l + 1) * L), L = ceil(C / lanes);
//  - member m of a lane runs unit 2s + m of every super-group its range
//    touches, over the key tiles the range covers, carrying the online
//    softmax across consecutive tiles.  A segment that covers its unit's
//    whole key range writes the output; the lane's first and last segments
//    otherwise write a partial (O, lse) into slot 2x or 2x + 1 of workgroup
//    x, which the combine kernel merges.
constexpr int kSkMaxPieces = 64;   // lanes one unit may span (the combine's LDS tables)

// A request's stream-K figures, shared through LDS during the segment loop.
struct SkReq {
    int base, cost, tiles, npre, rb, units, S, P, q0, kv0;
};

struct SkPlan {
    bool use;
    int C, L;
};

// Key tiles of a request: its prefix in 64-key tiles, then its pack.
__device__ __forceinline__ int seq_tiles_pre(const Seq &t) { return (t.S + 63) >> 6; }
__device__ __forceinline__ int seq_tiles(const Seq &t) { return ((t.S + 63) >> 6) + ((t.P + 63) >> 6); }

// The wave's maximum, as a wave-uniform (scalar) value.
__device__ __forceinline__ int wave_max(int x) {
#pragma unroll
    for (int off = 32; off; off >>= 1) x = max(x, __shfl_xor(x, off));
    return __builtin_amdgcn_readfirstlane(x);
}

// Lane and member of workgroup x, and back: the two members of a lane run
// on one XCD (workgroups are dealt to the XCDs round-robin).
__device__ __forceinline__ int sk_lane_of(int x, int nx, int &member) {
    const int k = x / nx;
    member = k & 1;
    return (k >> 1) * nx + x % nx;
}
__device__ __forceinline__ int sk_wg_of(int lane, int member, int nx) {
    return ((lane / nx) * 2 + member) * nx + lane % nx;
}

// Per-lane stream-K figures of request `lane` (t, loaded when it passed
// load_seq) and the batch's plan; every workgroup of the attention and
// combine kernels computes the same plan from the same metadata.  The
// static schedule stays when a unit would span more than kSkMaxPieces
// lanes.
__device__ SkPlan sk_plan(const AttnArgs &a, const Seq &t, bool ok, int &base, int &cost, int &tiles) {
    const bool has = ok && t.P > 0;
    tiles = has ? seq_tiles(t) : 0;
    const int units = has ? a.Hkv * t.rb : 0;
    cost = sat32((int64_t)((units + 1) >> 1) * tiles);
    const int C = wave_sum(cost);
    base = wave_scan(cost) - cost;
    SkPlan pl{false, C, 0};
    const int lanes = a.sk_wgs >> 1;
    if (a.sk_mode == 0 || lanes == 0 || C <= 0 || C == 0x7fffffff) return pl;
    pl.L = max((C + lanes - 1) / lanes, a.sk_min_tiles);
    pl.use = wave_max(tiles) <= (kSkMaxPieces - 2) * pl.L;
    return pl;
}

// One piece of work: query rows [rb * rows_wg, +rows_wg) of (request sq, KV
// head h) against its keys [k_begin, k_end), and where the result goes:
// the output (final), a static split-K partial (partial row of token q0 + i
// at prow0 + q0 + i, [part_rows][Hq][D]), or stream-K slot `slot`
// ([2 * sk_wgs][rows_wg][D]).
struct Unit {
    Seq sq;
    int h, rb, k_begin, k_end;
    int64_t prow0;
    int slot;
    bool final_out;
};

// Where a workgroup is in its stream-K lane.
struct WorkCursor {
    int64_t p, end, start;   // lane-steps: next position, lane end, lane start
    int member, x;
    bool sk;
};

// The next segment of the lane from cur.p on whose unit exists (a member
// whose super-group has one unit idles there); false at the lane's end.
__device__ bool sk_next_segment(const AttnArgs &a, WorkCursor &cur, Unit &u, const SkReq *skr) {
    const int lane = threadIdx.x & 63;
    const bool in = lane < a.batch;
    const int my_base = in ? skr[lane].base : 0, my_cost = in ? skr[lane].cost : 0;
    while (cur.p < cur.end) {
        const int64_t p = cur.p;
        const uint64_t hit = __ballot(in && my_cost > 0 && p >= my_base && p < (int64_t)my_base + my_cost);
        if (!hit) return false;
        const int b = __builtin_amdgcn_readfirstlane(__builtin_ctzll(hit));
        // wave-uniform values, kept in scalar registers
        SkReq q = skr[b];
        q.base = __builtin_amdgcn_readfirstlane(q.base);
        q.cost = __builtin_amdgcn_readfirstlane(q.cost);
        q.tiles = __builtin_amdgcn_readfirstlane(q.tiles);
        q.npre = __builtin_amdgcn_readfirstlane(q.npre);
        q.rb = __builtin_amdgcn_readfirstlane(q.rb);
        q.units = __builtin_amdgcn_readfirstlane(q.units);
        q.S = __builtin_amdgcn_readfirstlane(q.S);
        q.P = __builtin_amdgcn_readfirstlane(q.P);
        q.q0 = __builtin_amdgcn_readfirstlane(q.q0);
        q.kv0 = __builtin_amdgcn_readfirstlane(q.kv0);
        const int rel = (int)(p - q.base);
        const int sgi = rel / q.tiles, off = rel % q.tiles;
        const int64_t seg_end = min(cur.end, (int64_t)q.base + (int64_t)(sgi + 1) * q.tiles);
        const int n = (int)(seg_end - p);
        const int k = 2 * sgi + cur.member;
        const bool first = p == cur.start;
        cur.p = seg_end;
        if (k >= q.units) continue;
        Seq &sq = u.sq;
        sq.b = b;
        sq.S = q.S;
        sq.P = q.P;
        sq.T = q.S + q.P;
        sq.q0 = q.q0;
        sq.kv0 = q.kv0;
        sq.ns = 1;
        sq.rb = q.rb;
        sq.split_len = 0;
        sq.part_off = 0;
        u.h = k / q.rb;
        u.rb = k % q.rb;
        // tiles [off, off + n): prefix tiles first, then pack tiles from S
        auto key0 = [&](int i) { return i < q.npre ? i * 64 : q.S + (i - q.npre) * 64; };
        auto key1 = [&](int i) { return i < q.npre ? min(i * 64 + 64, q.S) : min(q.S + (i - q.npre) * 64 + 64, sq.T); };
        u.k_begin = key0(off);
        u.k_end = key1(off + n - 1);
        u.final_out = off == 0 && n == q.tiles;
        u.slot = u.final_out ? -1 : 2 * cur.x + (first ? 0 : 1);
        u.prow0 = 0;
        return true;
    }
    return false;
}

// The first piece of work of the calling workgroup, after the batch
// prologue; false when it has none (or the batch was rejected).  Batches of
// up to 64 requests take the stream-K lanes when the caller asked for them
// and sk_plan accepts the batch, else the longest-first schedule; larger
// ones take items in batch order, consecutive items (the row blocks of one
// key split) on one XCD so that they share its L2.  skr: LDS for the stream-K table (64 entries).
template <bool SK>   // SK: the kernel instance takes the stream-K schedule when the plan asks
__device__ bool first_unit(const AttnArgs &a, WorkCursor &cur, Unit &u, SkReq *skr) {
    cur.sk = false;
    Seq &sq = u.sq;
    int h = 0, split = 0, rb = 0;
    if (a.batch <= 64) {
        // one round of metadata loads serves the totals and the schedule
        const int lane = threadIdx.x & 63;
        Seq t{};
        const bool ok = lane < a.batch && load_seq(a, lane, t, threadIdx.x < 64);
        BatchTotals tot{0, 0, 0, false, false};
        add_totals(tot, a, lane, ok, t);
        if (!batch_prologue(a, tot)) return false;
        int base, cost, tiles;
        const SkPlan pl = SK ? sk_plan(a, t, ok, base, cost, tiles) : SkPlan{false, 0, 0};
        if (SK && pl.use) {
            if (threadIdx.x < 64 && lane < a.batch)
                skr[lane] = SkReq{base, cost, tiles, ok ? seq_tiles_pre(t) : 0, ok ? t.rb : 0,
                                  ok && t.P > 0 ? a.Hkv * t.rb : 0, t.S, t.P, t.q0, t.kv0};
            __syncthreads();
            const int x = blockIdx.x;
            if (x >= a.sk_wgs) return false;
            int member;
            const int l = sk_lane_of(x, a.xcds, member);
            cur.sk = true;
            cur.member = member;
            cur.x = x;
            cur.start = cur.p = (int64_t)l * pl.L;
            cur.end = min(cur.p + pl.L, (int64_t)pl.C);
            return sk_next_segment(a, cur, u, skr);
        }
        if (!locate_sorted(a, blockIdx.x, t, ok, sq, h, split, rb)) return false;
    } else {
        const BatchTotals tot = batch_totals(a);
        if (!batch_prologue(a, tot)) return false;
        const int64_t total = tot.items;
        const int nx = a.xcds;
        const int64_t n8 = (total + nx - 1) / nx * nx;
        const int64_t x = blockIdx.x;
        if (x >= n8) return false;
        const int64_t w = (x % nx) * (n8 / nx) + x / nx;
        if (w >= total) return false;
        int local;
        if (!find_request(a, w, false, sq, local)) return false;
        rb = local % sq.rb;
        split = (local / sq.rb) % sq.ns;
        h = local / (sq.rb * sq.ns);
    }
    u.h = h;
    u.rb = rb;
    u.k_begin = split * sq.split_len;
    u.k_end = min(sq.T, u.k_begin + sq.split_len);
    u.final_out = sq.ns == 1;
    u.slot = -1;
    u.prow0 = sq.part_off + (int64_t)split * sq.P - sq.q0;
    return true;
}

// The workgroup's next piece of work (stream-K lanes only), after a
// barrier that retires the previous piece's use of LDS.
__device__ __forceinline__ bool next_unit(const AttnArgs &a, WorkCursor &cur, Unit &u, const SkReq *skr) {
    if (!cur.sk || cur.p >= cur.end) return false;
    __syncthreads();
    return sk_next_segment(a, cur, u, skr);
}

// WPE: waves per SIMD the register budget is sized for.  2 (256 registers a
// lane) for head_dim 64 and 128; 1 (512) for head_dim 256, whose O^T
// accumulators (128 registers), Q^T operand (64), scores and staged K/V
// tiles take about 330, and for the 2-wave head_dim-128 instance, whose 128
// threads each stage four times the 8-wave instance's share of a K tile
// (about 330 registers): its 72 KB of LDS allow two such workgroups per
// CU, one wave per SIMD, either way.
// SKI: the stream-K instance (a run of segments per workgroup, the next
// segment's first tile and Q loaded during a segment's last tile); the
// static instances do one unit each.
template <int D, int WAVES, bool STORE, typename E, int WPE = 2, bool SKI = false>
__global__ __launch_bounds__(WAVES * 64) __attribute__((amdgpu_waves_per_eu(WPE)))
void tree_attn_mfma_kernel(AttnArgs a) {
    using vec8 = typename E::vec8;
    constexpr int NT = WAVES * 64;
    constexpr int BN = 64;                 // keys per tile: two 32-key MFMA blocks
    constexpr int ROWS = WAVES * 32;       // query rows per workgroup
    constexpr int KPAD = D + 8;            // K row stride in LDS (elements)
    constexpr int VPAD = BN + 8;           // V^T row stride in LDS (elements)
    constexpr int DSTEPS = D / 16;         // MFMA k-steps over the head dim
    constexpr int DB = D / 32;             // 32-row blocks of O^T
    constexpr int KCH = BN * D / 8;        // 16-byte K chunks per tile
    constexpr int K_PER_T = (KCH + NT - 1) / NT;
    constexpr int OCT = BN / 8;            // 8-key groups per tile
    constexpr int VUNITS = OCT * (D / 8);  // (8 keys x 8 d) V blocks per tile
    constexpr int V_PER_T = (VUNITS + NT - 1) / NT;

    // K tile [key][d].  V tile transposed, [d][key'], with the keys of every
    // 16-key group stored in the order (0-3, 8-11, 4-7, 12-15): a lane's eight
    // P^T k-slots are then eight consecutive columns (one 16-byte read).
    constexpr int NBUF = 2;
    __shared__ __attribute__((aligned(16))) uint16_t Ks[NBUF][BN * KPAD];
    __shared__ __attribute__((aligned(16))) uint16_t Vt[NBUF][D * VPAD];
    __shared__ EpiArgs epi;
    __shared__ int pack_hi[WAVES];   // per wave: the last pack key a row of it sees
    // Head dim 256 (one wave per SIMD, no registers to spare) has no
    // stream-K instance.
    constexpr bool kStreamK = SKI && D <= 128;
    __shared__ SkReq skr[kStreamK ? 64 : 1];

    // ---- this workgroup's work: one unit, or a run of stream-K segments
    Unit wu;
    WorkCursor cur;
    if (!first_unit<kStreamK>(a, cur, wu, skr)) return;
    const int tid = threadIdx.x;
    const int wave = tid >> 6;
    const int lane = tid & 63;
    const int g = lane >> 5;
    const int l32 = lane & 31;
    const uint16_t *qp = static_cast<const uint16_t *>(a.q);

    // ---- Q^T operand (B side): query l32, head-dim slice [ds*16 + g*8, +8)
    // of this lane's row of unit w
    vec8 qreg[DSTEPS];
    auto load_q = [&](const Unit &w) __attribute__((always_inline)) {
        const int r = w.rb * ROWS + wave * 32 + l32;
        const bool valid = r < w.sq.P * a.G;
        const int tok = w.sq.q0 + (valid ? r / a.G : 0);
        const int head = w.h * a.G + (valid ? r % a.G : 0);
        const uint16_t *src = qp + (int64_t)tok * a.q_tok + (int64_t)head * a.q_head + g * 8;
#pragma unroll
        for (int ds = 0; ds < DSTEPS; ++ds)
            qreg[ds] = valid ? *reinterpret_cast<const vec8 *>(src + ds * 16) : vec8{};
    };

    // ---- global -> register staging of one tile.  Each key source of a
    // (request, head) is one buffer resource that ends at its last row (the
    // concat layout: the request's S+P rows; the store layout: its S prefix
    // slots and its P pack rows), so rows past it read as zeros; a tile adds
    // 32-bit byte offsets (row * row stride + 16-byte chunk).  Rows past a
    // split's end but inside the request are real keys, masked below.
    u32x4 kst[K_PER_T];
    u32x4 vst[V_PER_T][8];
    // loads of one tile from one source (base, rows, byte strides); row0 is
    // the tile's first row within that source
    auto fetch_from = [&](const uint16_t *kb, const uint16_t *vb, int rows, uint32_t ksb, uint32_t vsb,
                          uint32_t row0) __attribute__((always_inline)) {
        const __amdgpu_buffer_rsrc_t krs = seg_rsrc(kb, rows, ksb, D * 2);
        const __amdgpu_buffer_rsrc_t vrs = seg_rsrc(vb, rows, vsb, D * 2);
#pragma unroll
        for (int it = 0; it < K_PER_T; ++it) {
            const int cidx = tid + it * NT;
            if (cidx >= KCH) break;
            const int key = cidx / (D / 8), dch = cidx % (D / 8);
            kst[it] = load16(krs, __umul24(row0 + key, ksb) + dch * 16);
        }
#pragma unroll
        for (int it = 0; it < V_PER_T; ++it) {
            const int u = tid + it * NT;
            if (u >= VUNITS) break;
            const int oc = u % OCT, dch = u / OCT;
            // key i of stored group oc: 16*(oc/2) + 4*(oc%2) + 8*(i/4) + i%4
            const uint32_t v0 = row0 + 16 * (oc >> 1) + 4 * (oc & 1);
#pragma unroll
            for (int i = 0; i < 8; ++i)
                vst[it][i] = load16(vrs, __umul24(v0 + 8 * (i >> 2) + (i & 3), vsb) + dch * 16);
        }
    };
    // the tile of keys [t0, t0 + 64) of (request q, head view v): its source
    // is chosen by a (wave-uniform) branch, not by selecting between the two
    // sources' values, which the compiler may lower to loads through a
    // private array
    auto fetch_tile = [&](const KvView<uint16_t> &v, const Seq &q, int t0) __attribute__((always_inline)) {
        if (!STORE || t0 < q.S)
            fetch_from(v.kpre, v.vpre, STORE ? q.S : q.T, (uint32_t)v.kpre_t * 2u, (uint32_t)v.vpre_t * 2u,
                       (uint32_t)t0);
        else
            fetch_from(v.kpack, v.vpack, q.P, (uint32_t)v.kpack_t * 2u, (uint32_t)v.vpack_t * 2u,
                       (uint32_t)(t0 - q.S));
    };

    // The first unit's Q and first tile; a stream-K segment loads the next
    // segment's during its own last tile (head dims up to 128: at 256 the
    // extra registers would spill), else at the segment's start.
    constexpr bool kPrefetchNext = kStreamK;
    load_q(wu);
    {
        const KvView<uint16_t> kv0(a.kv, wu.sq, wu.h);
        fetch_tile(kv0, wu.sq, wu.k_begin);
    }
    for (bool first_seg = true;; first_seg = false) {
    const Seq &sq = wu.sq;
    const int h = wu.h, rb = wu.rb, k_begin = wu.k_begin, k_end = wu.k_end;
    const int rows = sq.P * a.G;
    const int r = rb * ROWS + wave * 32 + l32;     // this lane's query row
    const bool active = rb * ROWS + wave * 32 < rows;
    const bool qvalid = r < rows;
    const int qtok = sq.q0 + (qvalid ? r / a.G : 0);
    const int qhead = h * a.G + (qvalid ? r % a.G : 0);
    const KvView<uint16_t> kv(a.kv, sq, h);
    if (!kPrefetchNext && !first_seg) {
        load_q(wu);
        fetch_tile(kv, sq, k_begin);
    }
    uint64_t mw0 = 0, mw1 = 0;
    if (qvalid && k_end > sq.S) {
        const uint64_t *mp = a.mask + (int64_t)qtok * a.mask_words;
        mw0 = mp[0];
        if (a.mask_words > 1) mw1 = mp[1];
    }

    floatx16 o[DB];
#pragma unroll
    for (int db = 0; db < DB; ++db) o[db] = floatx16{};
    float m = -INFINITY, msafe = 0.f, lsum = 0.f;
    const float c = a.scale_log2;

    // ---- key tiles, each covering keys [t0, t0 + valid), valid <= BN (the
    // rest of the tile is masked).  The split's prefix keys [k_begin, pre_end)
    // and pack keys [pk_begin, k_end) are tiled separately: in the store
    // layout every tile then reads one source, and both layouts add up the
    // same keys in the same order.
    const int pre_end = min(k_end, sq.S);
    const int n_pre = k_begin < pre_end ? (pre_end - k_begin + BN - 1) / BN : 0;
    const int pk_begin = max(k_begin, sq.S);
    const int n_pack = k_end > pk_begin ? (k_end - pk_begin + BN - 1) / BN : 0;
    auto tile_t0 = [&](int t) __attribute__((always_inline)) { return t < n_pre ? k_begin + t * BN : pk_begin + (t - n_pre) * BN; };
    auto tile_valid = [&](int t) __attribute__((always_inline)) { return min(BN, (t < n_pre ? pre_end : k_end) - tile_t0(t)); };
    auto fetch = [&](int t) __attribute__((always_inline)) { fetch_tile(kv, sq, tile_t0(t)); };
    // ---- register -> LDS: K as is; V as 8x8 transposed blocks
    auto publish = [&](int buf) __attribute__((always_inline)) {
#pragma unroll
        for (int it = 0; it < K_PER_T; ++it) {
            const int cidx = tid + it * NT;
            if (cidx >= KCH) break;
            const int key = cidx / (D / 8), dch = cidx % (D / 8);
            *reinterpret_cast<u32x4 *>(&Ks[buf][key * KPAD + dch * 8]) = kst[it];
        }
#pragma unroll
        for (int it = 0; it < V_PER_T; ++it) {
            const int u = tid + it * NT;
            if (u >= VUNITS) break;
            const int oc = u % OCT, dch = u / OCT;
#pragma unroll
            for (int dd = 0; dd < 8; ++dd) {
                // dword dd/2 of each key holds d = 2*(dd/2) (low) and +1 (high)
                const uint32_t sel = (dd & 1) ? 0x07060302u : 0x05040100u;
                const int k = dd >> 1;
                const u32x4 row = {__builtin_amdgcn_perm(vst[it][1][k], vst[it][0][k], sel),
                                   __builtin_amdgcn_perm(vst[it][3][k], vst[it][2][k], sel),
                                   __builtin_amdgcn_perm(vst[it][5][k], vst[it][4][k], sel),
                                   __builtin_amdgcn_perm(vst[it][7][k], vst[it][6][k], sel)};
                *reinterpret_cast<u32x4 *>(&Vt[buf][(dch * 8 + dd) * VPAD + oc * 8]) = row;
            }
        }
    };

    // the previous segment's epilogue (its reads of epi) and LDS tiles retire
    if (!first_seg) __syncthreads();
    // Pack tiles past the last pack key any row of the workgroup sees are
    // skipped: a one-unit workgroup at head dims up to 128 (the stream-K
    // segments keep their tiles; head dim 256 has no registers to spare)
    constexpr bool kTrimPack = !kStreamK && D <= 128;
    if (kTrimPack && n_pack > 0) {
        const int hi = wave_max(last_visible(mw0, mw1));
        if (lane == 0) pack_hi[wave] = hi;
    }
    if (tid == 0) {
        epi.out = a.out;
        epi.lse = a.lse;
        epi.part_o = a.part_o;
        epi.part_lse = a.part_lse;
        epi.sk_lse = a.sk_lse;
        epi.status = a.status;
        epi.o_tok = a.o_tok;
        epi.o_head = a.o_head;
        epi.part_rows = wu.slot >= 0 ? (int64_t)2 * a.sk_wgs * ROWS : a.part_rows;
        epi.prow0 = wu.prow0;
        epi.slot = wu.slot;
        epi.final_out = wu.final_out;
        epi.Hq = a.Hq;
    }
    __syncthreads();
    int n_pack_live = n_pack;
    if (kTrimPack && n_pack > 0) {
        int hi = pack_hi[0];
#pragma unroll
        for (int w = 1; w < WAVES; ++w) hi = max(hi, pack_hi[w]);
        const int pk0 = pk_begin - sq.S;
        n_pack_live = hi < pk0 ? 0 : min(n_pack, (hi - pk0) / BN + 1);
    }
    // (read from LDS, so held in a vector register: made scalar again)
    const int ntiles = __builtin_amdgcn_readfirstlane(n_pre + n_pack_live);
    // ---- the three stages of a tile
    // S^T = K Q^T: two 32-key blocks x 32 queries
    auto qk = [&](int buf, floatx16 (&s)[2]) __attribute__((always_inline)) {
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
            s[kb] = floatx16{};
#pragma unroll
            for (int ds = 0; ds < DSTEPS; ++ds) {
                const vec8 ka = *reinterpret_cast<const vec8 *>(
                    &Ks[buf][(kb * 32 + l32) * KPAD + ds * 16 + g * 8]);
                s[kb] = E::mma(ka, qreg[ds], s[kb]);
            }
        }
        // issue order: the K operand reads run kQkAhead MFMAs ahead of
        // their use (the default schedule issues them one or two ahead)
        __builtin_amdgcn_sched_group_barrier(0x100, kQkAhead, 0);   // DS reads
#pragma unroll
        for (int i = 0; i < 2 * DSTEPS - kQkAhead; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);      // one MFMA
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);      // one DS read
        }
        __builtin_amdgcn_sched_group_barrier(0x008, kQkAhead, 0);
    };
    // visibility, the online softmax in base 2 and the P^T operand of tile t
    auto softmax = [&](int t, floatx16 (&s)[2], vec8 (&pb)[2][2]) __attribute__((always_inline)) {
        // visibility (pack tiles and partial tiles only).  Element e of
        // lane (l32, g) in block kb is key t0 + 32*kb + 4*g + off(e),
        // off(e) = 8*(e/4) + e%4; in a pack tile that is pack key t0 - S + ...
        const int t0 = tile_t0(t);
        const int valid = tile_valid(t);
        const bool pack_tile = t >= n_pre;
        if (pack_tile || valid < BN) {
#pragma unroll
            for (int kb = 0; kb < 2; ++kb) {
                const int k0 = kb * 32 + 4 * g;
                const int lim = valid - k0;
                uint32_t vis = pack_tile ? vis_window(mw0, mw1, t0 - sq.S + k0) : ~0u;
                vis &= lim >= 32 ? ~0u : (lim <= 0 ? 0u : ((1u << lim) - 1u));
#pragma unroll
                for (int e = 0; e < 16; ++e) {
                    const int off = 8 * (e >> 2) + (e & 3);
                    s[kb][e] = (vis >> off) & 1u ? s[kb][e] : -INFINITY;
                }
            }
        }
        // The running max m is shared by the two lanes (l32, 0) and (l32, 1)
        // of a query; it only moves when a tile exceeds it by more than
        // 2^kRescaleSlack somewhere in the wave, so the cross-lane exchange
        // and the O rescale are rare.
        float lmax = s[0][0];
#pragma unroll
        for (int e = 1; e < 16; ++e) lmax = fmaxf(lmax, s[0][e]);
#pragma unroll
        for (int e = 0; e < 16; ++e) lmax = fmaxf(lmax, s[1][e]);
        if (__any(lmax * c > m + kRescaleSlack)) {
            const float mx = fmaxf(lmax, partner32(lmax)) * c;
            const float mn = fmaxf(m, mx);
            const float alpha = mn == -INFINITY ? 1.f : __builtin_amdgcn_exp2f(m - mn);
            lsum *= alpha;
#pragma unroll
            for (int db = 0; db < DB; ++db) o[db] *= alpha;
            m = mn;
            msafe = m == -INFINITY ? 0.f : m;
        }
        float acc = 0.f;
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
            float p[16];
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                p[e] = __builtin_amdgcn_exp2f(fmaf(s[kb][e], c, -msafe));
                acc += p[e];
            }
#pragma unroll
            for (int hf = 0; hf < 2; ++hf) {
                u32x4 w;
#pragma unroll
                for (int e = 0; e < 4; ++e) w[e] = E::pack2(p[hf * 8 + 2 * e], p[hf * 8 + 2 * e + 1]);
                pb[kb][hf] = __builtin_bit_cast(vec8, w);
            }
        }
        lsum += acc;
    };
    // O^T += V^T P^T over four 16-key slices.  Slot j of lane group g in
    // slice (kb, hf) is key 32*kb + 16*hf + 8*(j/4) + 4*g + j%4, stored at
    // column 32*kb + 16*hf + 8*g + j.
    auto pv = [&](int buf, const vec8 (&pb)[2][2]) __attribute__((always_inline)) {
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int hf = 0; hf < 2; ++hf)
#pragma unroll
                for (int db = 0; db < DB; ++db) {
                    const vec8 va = *reinterpret_cast<const vec8 *>(
                        &Vt[buf][(db * 32 + l32) * VPAD + kb * 32 + hf * 16 + g * 8]);
                    o[db] = E::mma(va, pb[kb][hf], o[db]);
                }
        // the same for the V^T operand reads of the PV product; the
        // exponentials stay free to fill the gaps
        __builtin_amdgcn_sched_group_barrier(0x100, kQkAhead, 1);
#pragma unroll
        for (int i = 0; i < 4 * DB - kQkAhead; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 1);
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 1);
        }
        __builtin_amdgcn_sched_group_barrier(0x008, kQkAhead, 1);
    };

    auto tile_body = [&](int t, int buf) __attribute__((always_inline)) {
        floatx16 s[2];
        vec8 pb[2][2];
        qk(buf, s);
        softmax(t, s, pb);
        pv(buf, pb);
    };

    // The next tile's loads are in flight during the current tile's MFMA
    // work.  During a stream-K segment's last tile, the next segment's first
    // tile and (once this tile's QK product is issued) its Q are loaded.
    // (The last tile is peeled off the loop, so that the next segment's
    // values live only there.)
    Unit nxt;
    bool has_next = false;
    if constexpr (kPrefetchNext) {
    for (int t = 0; t + 1 < ntiles; ++t) {
        const int buf = t % NBUF;
        publish(buf);
        __syncthreads();
        fetch(t + 1);
        if (!active) continue;
        tile_body(t, buf);
    }
    if (ntiles > 0) {
        const int t = ntiles - 1;
        const int buf = t % NBUF;
        publish(buf);
        __syncthreads();
        if (kStreamK && cur.sk) {
            has_next = sk_next_segment(a, cur, nxt, skr);
            if (kPrefetchNext && has_next) {
                const KvView<uint16_t> kvn(a.kv, nxt.sq, nxt.h);
                fetch_tile(kvn, nxt.sq, nxt.k_begin);
            }
        }
        if (active) tile_body(t, buf);
        // the next segment's Q: its latency overlaps this segment's epilogue
        if (kPrefetchNext && has_next) {
            __builtin_amdgcn_sched_barrier(0);
            load_q(nxt);
        }
    }
    } else {
    for (int t = 0; t < ntiles; ++t) {
        const int buf = t % NBUF;
        publish(buf);
        __syncthreads();
        if (t + 1 < ntiles) fetch(t + 1);
        if (!active) continue;
        tile_body(t, buf);
    }
    }

    // ---- epilogue: normalise, write the output or the split partial.
    // O^T element e of lane (l32, g) in block db is d = 32*db + 8*(e/4) + 4*g + e%4.
    if (active) {
        const float ltot = lsum + partner32(lsum);
        const float inv = ltot > 0.f ? 1.f / ltot : 0.f;
        const float lse2 = ltot > 0.f ? msafe + log2f(ltot) : -INFINITY;
        const EpiArgs e = epi;
        if (qvalid && e.final_out) {
            uint16_t *op = static_cast<uint16_t *>(e.out) + (int64_t)qtok * e.o_tok + (int64_t)qhead * e.o_head;
#pragma unroll
            for (int db = 0; db < DB; ++db)
#pragma unroll
                for (int r4 = 0; r4 < 4; ++r4) {
                    const int d = db * 32 + 8 * r4 + 4 * g;
                    const u32x2 w = {E::pack2(o[db][4 * r4] * inv, o[db][4 * r4 + 1] * inv),
                                     E::pack2(o[db][4 * r4 + 2] * inv, o[db][4 * r4 + 3] * inv)};
                    *reinterpret_cast<u32x2 *>(op + d) = w;
                }
            if (e.lse && g == 0) e.lse[(int64_t)qtok * e.Hq + qhead] = lse2 * kLn2;
        } else if (qvalid) {
            // static split: row (token, head) of the partial rows; stream-K:
            // row wave * 32 + l32 of the workgroup's slot
            const int64_t prow = e.slot >= 0 ? (int64_t)e.slot * ROWS + wave * 32 + l32 : e.prow0 + qtok;
            if (prow >= e.part_rows) {
                raise_flag(e.status, CAST_FLAG_BAD_OFFSETS);
            } else {
                const int64_t orow = e.slot >= 0 ? prow : prow * e.Hq + qhead;
                float *pp = e.part_o + orow * D;
#pragma unroll
                for (int db = 0; db < DB; ++db)
#pragma unroll
                    for (int r4 = 0; r4 < 4; ++r4) {
                        const int d = db * 32 + 8 * r4 + 4 * g;
                        const floatx4 w = {o[db][4 * r4] * inv, o[db][4 * r4 + 1] * inv, o[db][4 * r4 + 2] * inv,
                                           o[db][4 * r4 + 3] * inv};
                        *reinterpret_cast<floatx4 *>(pp + d) = w;
                    }
                if (g == 0) (e.slot >= 0 ? e.sk_lse : e.part_lse)[orow] = lse2;
            }
        }
    }
    if constexpr (kStreamK && !kPrefetchNext) has_next = cur.sk && sk_next_segment(a, cur, nxt, skr);
    if (!has_next) break;
    wu = nxt;
    }
}
// --------------------------------------------------------------------------
// MFMA kernel for fp32 inputs: head_dim D in {64, 128, 256}, WAVES waves x
// 32 query rows, v_mfma_f32_32x32x2_f32.  The reference hook runs its kernel on
// fp32 copies of q/k/v (cast_trees/serving.py:68-71), where p stays fp32
// for the value product (tree_attn.py:66,87 cast p to the input dtype):
// so does this kernel.  Same structure as the bf16 kernel: S^T = K Q^T with
// each lane owning one query column, P^T straight from the S^T
// accumulators, O^T += V^T P^T.  A 32x32x2 step takes one value per lane
// per operand: in the QK product lane (l32, g) supplies head-dim element
// (D/2)*g + step of its key and of its query, so a lane's K operands for
// four steps are one 16-byte LDS read; in the PV product it supplies the
// value of key 8*(e/4) + 4*g + e%4 at step e, which is exactly its own
// accumulator element e.  V sits in LDS as V'[key][vpos(l)*DB + db] =
// V[key][32*db + l], so one read gives lane l the operands of all DB
// output blocks; vpos(l) = 8*(l%4) + l/4 (a 4x8 transpose of the group
// index) puts the eight groups of a key that one staging store covers
// (l = 4*lg + i, lg = 0..7) side by side, on distinct banks; the reads
// take a permutation of the same row.  The product is MFMA-bound (16 x the
// bf16 cycles per flop): staging and softmax are small beside it.
// --------------------------------------------------------------------------
// Key tiles hold 64 keys (two 32-key blocks), or 32 at head dim 256, where
// two double-buffered 64-key K and V' tiles would not fit in LDS.
// WPE: waves per SIMD the register budget is sized for: 2, except the
// 4-wave head-dim-128 and -256 instances (1): the former's threads each
// stage twice the 8-wave instance's share of a tile, the latter holds 128
// registers of Q and 128 of O per lane; their 133-135 KB of LDS leave room
// for one workgroup (one wave per SIMD) per CU anyway.
template <int D, int WAVES, bool STORE, int WPE = 2, bool SKI = false>
__global__ __launch_bounds__(WAVES * 64) __attribute__((amdgpu_waves_per_eu(WPE)))
void tree_attn_f32_kernel(AttnArgs a) {
    constexpr int NT = WAVES * 64;
    constexpr int BN = D <= 128 ? 64 : 32;  // keys per tile
    constexpr int NKB = BN / 32;           // 32-key MFMA blocks per tile
    constexpr int ROWS = WAVES * 32;       // query rows per workgroup
    constexpr int DH = D / 2;              // k-steps per 32-key block (2 head-dim values each)
    constexpr int DB = D / 32;             // 32-row blocks of O^T
    constexpr int KPAD = D + 4;            // LDS row stride (floats)
    constexpr int KCH = BN * D / 4;        // 16-byte K chunks per tile
    constexpr int K_PER_T = (KCH + NT - 1) / NT;
    constexpr int VUNITS = BN * 8;         // (key, group of 4 l) staging units of V
    constexpr int V_PER_T = (VUNITS + NT - 1) / NT;
    typedef float floatxDB __attribute__((ext_vector_type(DB)));

    __shared__ __attribute__((aligned(16))) float Ks[2][BN * KPAD];
    __shared__ __attribute__((aligned(16))) float Vs[2][BN * KPAD];
    __shared__ EpiArgs epi;
    __shared__ int pack_hi[WAVES];   // per wave: the last pack key a row of it sees
    __shared__ SkReq skr[SKI ? 64 : 1];

    Unit wu;
    WorkCursor cur;
    if (!first_unit<SKI>(a, cur, wu, skr)) return;
    const int tid = threadIdx.x;
    const int wave = tid >> 6;
    const int lane = tid & 63;
    const int g = lane >> 5;
    const int l32 = lane & 31;
    do {
    const Seq &sq = wu.sq;
    const int h = wu.h, rb = wu.rb, k_begin = wu.k_begin, k_end = wu.k_end;
    const int rows = sq.P * a.G;
    const int r = rb * ROWS + wave * 32 + l32;
    const bool active = rb * ROWS + wave * 32 < rows;
    const bool qvalid = r < rows;
    const int qtok = sq.q0 + (qvalid ? r / a.G : 0);
    const int qhead = h * a.G + (qvalid ? r % a.G : 0);
    const KvView<float> kv(a.kv, sq, h);

    // Q operand: head-dim elements [DH*g, DH*g + DH) of this lane's query
    float qf[DH];
    {
        const float *src = static_cast<const float *>(a.q) + (int64_t)qtok * a.q_tok + (int64_t)qhead * a.q_head +
                           DH * g;
#pragma unroll
        for (int i = 0; i < DH / 4; ++i) {
            const floatx4 x = qvalid ? *reinterpret_cast<const floatx4 *>(src + 4 * i) : floatx4{};
#pragma unroll
            for (int j = 0; j < 4; ++j) qf[4 * i + j] = x[j];
        }
    }
    uint64_t mw0 = 0, mw1 = 0;
    if (qvalid && k_end > sq.S) {
        const uint64_t *mp = a.mask + (int64_t)qtok * a.mask_words;
        mw0 = mp[0];
        if (a.mask_words > 1) mw1 = mp[1];
    }

    floatx16 o[DB];
#pragma unroll
    for (int db = 0; db < DB; ++db) o[db] = floatx16{};
    float m = -INFINITY, msafe = 0.f, lsum = 0.f;
    const float c = a.scale_log2;

    const int pre_end = min(k_end, sq.S);
    const int n_pre = k_begin < pre_end ? (pre_end - k_begin + BN - 1) / BN : 0;
    const int pk_begin = max(k_begin, sq.S);
    const int n_pack = k_end > pk_begin ? (k_end - pk_begin + BN - 1) / BN : 0;
    auto tile_t0 = [&](int t) __attribute__((always_inline)) { return t < n_pre ? k_begin + t * BN : pk_begin + (t - n_pre) * BN; };
    auto tile_valid = [&](int t) __attribute__((always_inline)) { return min(BN, (t < n_pre ? pre_end : k_end) - tile_t0(t)); };

    const uint32_t ksb_pre = (uint32_t)kv.kpre_t * 4u, vsb_pre = (uint32_t)kv.vpre_t * 4u;
    const uint32_t ksb_pack = (uint32_t)kv.kpack_t * 4u, vsb_pack = (uint32_t)kv.vpack_t * 4u;
    const int rows_pre = STORE ? sq.S : sq.T;
    const __amdgpu_buffer_rsrc_t kr_pre = seg_rsrc(kv.kpre, rows_pre, ksb_pre, D * 4);
    const __amdgpu_buffer_rsrc_t vr_pre = seg_rsrc(kv.vpre, rows_pre, vsb_pre, D * 4);
    const __amdgpu_buffer_rsrc_t kr_pack = seg_rsrc(kv.kpack, STORE ? sq.P : 0, ksb_pack, D * 4);
    const __amdgpu_buffer_rsrc_t vr_pack = seg_rsrc(kv.vpack, STORE ? sq.P : 0, vsb_pack, D * 4);
    u32x4 kst[K_PER_T];
    u32x4 vst[V_PER_T][DB];
    auto fetch = [&](int t) __attribute__((always_inline)) {
        const bool pre = !STORE || t < n_pre;
        const int t0 = tile_t0(t);
        const uint32_t row0 = (uint32_t)(pre ? t0 : t0 - sq.S);
        const __amdgpu_buffer_rsrc_t krs = pre ? kr_pre : kr_pack;
        const __amdgpu_buffer_rsrc_t vrs = pre ? vr_pre : vr_pack;
        const uint32_t ksb = pre ? ksb_pre : ksb_pack;
        const uint32_t vsb = pre ? vsb_pre : vsb_pack;
#pragma unroll
        for (int it = 0; it < K_PER_T; ++it) {
            const int cidx = tid + it * NT;
            if (cidx >= KCH) break;
            const int key = cidx / (D / 4), dch = cidx % (D / 4);
            kst[it] = load16(krs, __umul24(row0 + key, ksb) + dch * 16);
        }
#pragma unroll
        for (int it = 0; it < V_PER_T; ++it) {
            const int u = tid + it * NT;
            if (u >= VUNITS) break;
            const int key = u >> 3, lg = u & 7;
#pragma unroll
            for (int db = 0; db < DB; ++db)
                vst[it][db] = load16(vrs, __umul24(row0 + key, vsb) + db * 128 + lg * 16);
        }
    };
    // register -> LDS: K as is; V with d = 32*db + l stored at vpos(l)*DB + db
    auto vpos = [](int l) __attribute__((always_inline)) { return 8 * (l & 3) + (l >> 2); };
    auto publish = [&](int buf) __attribute__((always_inline)) {
#pragma unroll
        for (int it = 0; it < K_PER_T; ++it) {
            const int cidx = tid + it * NT;
            if (cidx >= KCH) break;
            const int key = cidx / (D / 4), dch = cidx % (D / 4);
            *reinterpret_cast<u32x4 *>(&Ks[buf][key * KPAD + dch * 4]) = kst[it];
        }
#pragma unroll
        for (int it = 0; it < V_PER_T; ++it) {
            const int u = tid + it * NT;
            if (u >= VUNITS) break;
            const int key = u >> 3, lg = u & 7;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                floatxDB w;
#pragma unroll
                for (int db = 0; db < DB; ++db) {
                    // element i through a scalar: hipcc (ROCm 7.2) reads element 0
                    // for every i of __builtin_bit_cast(float, vec[db][i])
                    const uint32_t bits = vst[it][db][i];
                    w[db] = __builtin_bit_cast(float, bits);
                }
                *reinterpret_cast<floatxDB *>(&Vs[buf][key * KPAD + vpos(4 * lg + i) * DB]) = w;
            }
        }
    };

    // pack tiles past the last pack key any row of the workgroup sees are
    // skipped (a one-unit workgroup; the stream-K segments keep their tiles)
    if (!SKI && n_pack > 0) {
        const int hi = wave_max(last_visible(mw0, mw1));
        if (lane == 0) pack_hi[wave] = hi;
    }
    if (tid == 0) {
        epi.out = a.out;
        epi.lse = a.lse;
        epi.part_o = a.part_o;
        epi.part_lse = a.part_lse;
        epi.sk_lse = a.sk_lse;
        epi.status = a.status;
        epi.o_tok = a.o_tok;
        epi.o_head = a.o_head;
        epi.part_rows = wu.slot >= 0 ? (int64_t)2 * a.sk_wgs * ROWS : a.part_rows;
        epi.prow0 = wu.prow0;
        epi.slot = wu.slot;
        epi.final_out = wu.final_out;
        epi.Hq = a.Hq;
    }
    __syncthreads();
    int n_pack_live = n_pack;
    if (!SKI && n_pack > 0) {
        int hi = pack_hi[0];
#pragma unroll
        for (int w = 1; w < WAVES; ++w) hi = max(hi, pack_hi[w]);
        const int pk0 = pk_begin - sq.S;
        n_pack_live = hi < pk0 ? 0 : min(n_pack, (hi - pk0) / BN + 1);
    }
    // (read from LDS, so held in a vector register: made scalar again)
    const int ntiles = __builtin_amdgcn_readfirstlane(n_pre + n_pack_live);

    if (ntiles > 0) fetch(0);
    for (int t = 0; t < ntiles; ++t) {
        const int buf = t & 1;
        publish(buf);
        __syncthreads();
        if (t + 1 < ntiles) fetch(t + 1);
        if (!active) continue;
        const int t0 = tile_t0(t);
        const int valid = tile_valid(t);
        const bool pack_tile = t >= n_pre;
        // in a pack tile, the 32-key blocks no row of the wave sees are
        // skipped: scores -inf, no PV product
        bool live[NKB];
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb)
            live[kb] = SKI || !pack_tile || block_live(mw0, mw1, t0 - sq.S + 32 * kb, valid - 32 * kb);
        // S^T = K Q^T, the two 32-key blocks' chains interleaved
        floatx16 s[NKB];
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb) s[kb] = floatx16{};
        if (NKB == 2 && live[0] && live[NKB - 1]) {
#pragma unroll
            for (int i = 0; i < DH / 4; ++i) {
                const floatx4 k0 = *reinterpret_cast<const floatx4 *>(&Ks[buf][l32 * KPAD + DH * g + 4 * i]);
                const floatx4 k1 =
                    *reinterpret_cast<const floatx4 *>(&Ks[buf][((NKB - 1) * 32 + l32) * KPAD + DH * g + 4 * i]);
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    s[0] = __builtin_amdgcn_mfma_f32_32x32x2f32(k0[j], qf[4 * i + j], s[0], 0, 0, 0);
                    s[NKB - 1] = __builtin_amdgcn_mfma_f32_32x32x2f32(k1[j], qf[4 * i + j], s[NKB - 1], 0, 0, 0);
                }
            }
        } else {
#pragma unroll
            for (int kb = 0; kb < NKB; ++kb) {
                if (!live[kb]) {
#pragma unroll
                    for (int e = 0; e < 16; ++e) s[kb][e] = -INFINITY;
                    continue;
                }
#pragma unroll
                for (int i = 0; i < DH / 4; ++i) {
                    const floatx4 kk =
                        *reinterpret_cast<const floatx4 *>(&Ks[buf][(kb * 32 + l32) * KPAD + DH * g + 4 * i]);
#pragma unroll
                    for (int j = 0; j < 4; ++j)
                        s[kb] = __builtin_amdgcn_mfma_f32_32x32x2f32(kk[j], qf[4 * i + j], s[kb], 0, 0, 0);
                }
            }
        }
        // visibility on pack tiles and partial tiles (as in the bf16 kernel)
        if (pack_tile || valid < BN) {
#pragma unroll
            for (int kb = 0; kb < NKB; ++kb) {
                const int k0 = kb * 32 + 4 * g;
                const int lim = valid - k0;
                uint32_t vis = pack_tile ? vis_window(mw0, mw1, t0 - sq.S + k0) : ~0u;
                vis &= lim >= 32 ? ~0u : (lim <= 0 ? 0u : ((1u << lim) - 1u));
#pragma unroll
                for (int e = 0; e < 16; ++e) {
                    const int off = 8 * (e >> 2) + (e & 3);
                    s[kb][e] = (vis >> off) & 1u ? s[kb][e] : -INFINITY;
                }
            }
        }
        float lmax = s[0][0];
#pragma unroll
        for (int e = 1; e < 16; ++e) lmax = fmaxf(lmax, s[0][e]);
#pragma unroll
        for (int kb = 1; kb < NKB; ++kb)
#pragma unroll
            for (int e = 0; e < 16; ++e) lmax = fmaxf(lmax, s[kb][e]);
        if (__any(lmax * c > m + kRescaleSlack)) {
            const float mx = fmaxf(lmax, partner32(lmax)) * c;
            const float mn = fmaxf(m, mx);
            const float alpha = mn == -INFINITY ? 1.f : __builtin_amdgcn_exp2f(m - mn);
            lsum *= alpha;
#pragma unroll
            for (int db = 0; db < DB; ++db) o[db] *= alpha;
            m = mn;
            msafe = m == -INFINITY ? 0.f : m;
        }
        float acc = 0.f;
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                s[kb][e] = __builtin_amdgcn_exp2f(fmaf(s[kb][e], c, -msafe));
                acc += s[kb][e];
            }
        lsum += acc;
        // O^T += V^T P^T: step e of block kb is key 32*kb + 8*(e/4) + 4*g + e%4
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb) {
            if (!live[kb]) continue;
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int key = kb * 32 + 8 * (e >> 2) + 4 * g + (e & 3);
                const floatxDB vv = *reinterpret_cast<const floatxDB *>(&Vs[buf][key * KPAD + vpos(l32) * DB]);
#pragma unroll
                for (int db = 0; db < DB; ++db)
                    o[db] = __builtin_amdgcn_mfma_f32_32x32x2f32(vv[db], s[kb][e], o[db], 0, 0, 0);
            }
        }
    }

    if (active && qvalid) {
        const float ltot = lsum + partner32(lsum);
        const float inv = ltot > 0.f ? 1.f / ltot : 0.f;
        const float lse2 = ltot > 0.f ? msafe + log2f(ltot) : -INFINITY;
        const EpiArgs e = epi;
        float *dst = nullptr;
        if (e.final_out) {
            dst = static_cast<float *>(e.out) + (int64_t)qtok * e.o_tok + (int64_t)qhead * e.o_head;
            if (e.lse && g == 0) e.lse[(int64_t)qtok * e.Hq + qhead] = lse2 * kLn2;
        } else {
            // static split: row (token, head) of the partial rows; stream-K:
            // row wave * 32 + l32 of the workgroup's slot
            const int64_t prow = e.slot >= 0 ? (int64_t)e.slot * ROWS + wave * 32 + l32 : e.prow0 + qtok;
            if (prow >= e.part_rows) {
                raise_flag(e.status, CAST_FLAG_BAD_OFFSETS);
            } else {
                const int64_t orow = e.slot >= 0 ? prow : prow * e.Hq + qhead;
                dst = e.part_o + orow * D;
                if (g == 0) (e.slot >= 0 ? e.sk_lse : e.part_lse)[orow] = lse2;
            }
        }
        if (dst) {
#pragma unroll
            for (int db = 0; db < DB; ++db)
#pragma unroll
                for (int r4 = 0; r4 < 4; ++r4) {
                    const int d = db * 32 + 8 * r4 + 4 * g;
                    const floatx4 w = {o[db][4 * r4] * inv, o[db][4 * r4 + 1] * inv, o[db][4 * r4 + 2] * inv,
                                       o[db][4 * r4 + 3] * inv};
                    *reinterpret_cast<floatx4 *>(dst + d) = w;
                }
        }
    }
    } while (SKI && next_unit(a, cur, wu, skr));
}

// --------------------------------------------------------------------------
// Split-K combine: one workgroup per packed token, all query heads.
// --------------------------------------------------------------------------
// The stream-K merge of token tok (index i of request sq) for query heads
// [h0, hend): each head's unit (KV head, row block) sits in super-group
// s = unit / 2, lane-steps [g0, g0 + tiles) of the lane line, which lanes
// g0 / L .. (g0 + tiles - 1) / L cover; one lane means the attention kernel
// wrote the output itself.  Otherwise piece l is member (unit % 2) of lane l:
// slot 2x + 1 for the first lane when the super-group starts inside it (the
// lane's last segment), slot 2x for the others (their first segment).  The
// pieces' lse and weights go through LDS, then every 4-wide chunk of the
// heads' outputs merges its pieces.
// The LDS of the combine kernel: per (head, split) lse then weights, and
// per head max and sum; the stream-K instance adds each piece's partial row
// and each head's piece count.
struct CombineLds {
    float wgt[kCombineLdsHeads * kCombineLdsSplits];
    float hm[kCombineLdsHeads], hl[kCombineLdsHeads];
};
struct CombineLdsSk : CombineLds {
    int prow[kCombineLdsHeads * kSkMaxPieces];
    int hn[kCombineLdsHeads];
};

template <typename OutT, int D, typename E>
__device__ void combine_stream_k(const AttnArgs &a, const SkPlan &pl, const Seq &sq, int i, int tok, int h0,
                                 int hend, int base, int tiles, CombineLdsSk &sm) {
    constexpr int C = D / 4;
    constexpr int NP = kSkMaxPieces;
    static_assert(kSkMaxPieces <= kCombineLdsSplits, "pieces share the split table");
    const int nh = hend - h0;   // <= kCombineLdsHeads (the host sizes the head groups)
    const int rows_wg = a.rows_wg, G = a.G, nx = a.xcds, L = pl.L;
    // one thread per head: its unit, the lanes its super-group spans and
    // the partial row of every piece; the pieces' lse into LDS
    if (threadIdx.x < nh) {
        const int hh = threadIdx.x, hq = h0 + hh;
        const int r = i * G + hq % G;
        const int unit = (hq / G) * sq.rb + r / rows_wg;
        const int64_t g0 = (int64_t)base + (int64_t)(unit >> 1) * tiles;
        const int l0 = (int)(g0 / L), l1 = (int)((g0 + tiles - 1) / L);
        const int n = l1 > l0 ? l1 - l0 + 1 : 0;
        sm.hn[hh] = n;
        float M = -INFINITY;
        for (int p0 = 0; p0 < n; p0 += kCombineUnroll) {
            float l[kCombineUnroll];
#pragma unroll
            for (int k = 0; k < kCombineUnroll; ++k) {
                const int piece = p0 + k;
                const int x = sk_wg_of(l0 + piece, unit & 1, nx);
                const int slot = 2 * x + (piece == 0 && g0 != (int64_t)l0 * L ? 1 : 0);
                const int row = slot * rows_wg + r % rows_wg;
                if (piece < n) sm.prow[hh * NP + piece] = row;
                l[k] = piece < n ? a.sk_lse[row] : -INFINITY;
            }
#pragma unroll
            for (int k = 0; k < kCombineUnroll; ++k) {
                if (p0 + k < n) sm.wgt[hh * NP + p0 + k] = l[k];
                M = fmaxf(M, l[k]);
            }
        }
        float S = 0.f;
        for (int piece = 0; piece < n; ++piece) {
            const float w = M == -INFINITY ? 0.f : exp2f(sm.wgt[hh * NP + piece] - M);
            sm.wgt[hh * NP + piece] = w;
            S += w;
        }
        sm.hm[hh] = M;
        sm.hl[hh] = S;
    }
    __syncthreads();
    // every 4-wide chunk of the heads' outputs: all its pieces' loads in
    // flight at once (up to kCombineUnroll), then the weighted sum
    for (int c = threadIdx.x; c < nh * C; c += blockDim.x) {
        const int hh = c / C, d4 = c % C;
        const int n = sm.hn[hh];
        if (n == 0) continue;
        const float M = sm.hm[hh], S = sm.hl[hh];
        floatx4 acc = {0.f, 0.f, 0.f, 0.f};
        if (M != -INFINITY) {
            const int *rw = sm.prow + hh * NP;
            const float *w = sm.wgt + hh * NP;
            for (int s0 = 0; s0 < n; s0 += kCombineUnroll) {
                floatx4 x[kCombineUnroll];
#pragma unroll
                for (int k = 0; k < kCombineUnroll; ++k)
                    x[k] = s0 + k < n ? *reinterpret_cast<const floatx4 *>(a.part_o + (int64_t)rw[s0 + k] * D + d4 * 4)
                                      : floatx4{};
#pragma unroll
                for (int k = 0; k < kCombineUnroll; ++k)
                    if (s0 + k < n) acc += w[s0 + k] * x[k];
            }
            acc *= 1.f / S;
        }
        const int hq = h0 + hh;
        OutT *op = static_cast<OutT *>(a.out) + (int64_t)tok * a.o_tok + (int64_t)hq * a.o_head + d4 * 4;
        if constexpr (sizeof(OutT) == 2) {
            const u32x2 w2 = {E::pack2(acc[0], acc[1]), E::pack2(acc[2], acc[3])};
            *reinterpret_cast<u32x2 *>(op) = w2;
        } else {
            *reinterpret_cast<floatx4 *>(op) = acc;
        }
        if (a.lse && d4 == 0)
            a.lse[(int64_t)tok * a.Hq + hq] = M == -INFINITY ? -INFINITY : (M + log2f(S)) * kLn2;
    }
}

// E: the 16-bit format when OutT is 2 bytes; SKI: merges stream-K pieces
template <typename OutT, int D, typename E, bool SKI = false>
__global__ __launch_bounds__(256) void tree_attn_combine_kernel(AttnArgs a) {
    constexpr int C = D / 4;
    __shared__ typename std::conditional<SKI, CombineLdsSk, CombineLds>::type sm;
    const int groups = a.comb_groups;
    const int tok = blockIdx.x / groups;
    const int hpg = (a.Hq + groups - 1) / groups;
    const int h0 = (blockIdx.x % groups) * hpg;
    Seq sq;
    int i;
    // a rejected batch was zero-filled by the attention kernel
    auto rejected = [&](const BatchTotals &t) { return t.kv_sum > a.total_kv || t.q_sum > a.total_q || t.unordered; };
    if (a.batch <= 64) {
        // one round of metadata loads: the totals and the request of tok
        const int lane = threadIdx.x & 63;
        Seq t{};
        const bool ok = lane < a.batch && load_seq(a, lane, t, false);
        BatchTotals tot{0, 0, 0, false, false};
        add_totals(tot, a, lane, ok, t);
        if (rejected(tot)) return;
        const int pp = ok && t.ns > 1 ? sat32((int64_t)t.ns * t.P) : 0;
        const int p_excl = wave_scan(pp) - pp;
        int base = 0, cost = 0, tiles = 0;
        const SkPlan pl = SKI ? sk_plan(a, t, ok, base, cost, tiles) : SkPlan{false, 0, 0};
        const uint64_t hit = __ballot(ok && tok >= t.q0 && tok < t.q0 + t.P);
        if (!hit) return;
        const int src = __builtin_amdgcn_readfirstlane(__builtin_ctzll(hit));
        sq = shfl_seq(t, src);
        sq.part_off = bcast(p_excl, src);
        i = tok - sq.q0;
        if constexpr (SKI) {
            if (pl.use) {
                combine_stream_k<OutT, D, E>(a, pl, sq, i, tok, h0, min(a.Hq, h0 + hpg), bcast(base, src),
                                             bcast(tiles, src), sm);
                return;
            }
        }
    } else {
        if (rejected(batch_totals(a))) return;
        if (!find_request(a, tok, true, sq, i)) return;
    }
    if (sq.ns <= 1) return;
    if (sq.part_off + (int64_t)sq.ns * sq.P > a.part_rows) return;
    const int64_t lstride = (int64_t)sq.P * a.Hq, xstride = lstride * D;
    const int hend = min(a.Hq, h0 + hpg);
    const int ns = sq.ns;
    auto finish = [&](int c, floatx4 acc, float M, float L) {
        const int hq = h0 + c / C, d4 = c % C;
        if (M != -INFINITY) acc *= 1.f / L;
        OutT *op = static_cast<OutT *>(a.out) + (int64_t)tok * a.o_tok + (int64_t)hq * a.o_head + d4 * 4;
        if constexpr (sizeof(OutT) == 2) {
            const u32x2 w = {E::pack2(acc[0], acc[1]), E::pack2(acc[2], acc[3])};
            *reinterpret_cast<u32x2 *>(op) = w;
        } else {
            *reinterpret_cast<floatx4 *>(op) = acc;
        }
        if (a.lse && d4 == 0)
            a.lse[(int64_t)tok * a.Hq + hq] = M == -INFINITY ? -INFINITY : (M + log2f(L)) * kLn2;
    };
    const int nc = (hend - h0) * C;
    if (ns <= kCombineFast) {
        // up to kCombineFast splits: every split's LSE and partial of two
        // chunks are loaded before any is used (one round trip)
        for (int c0 = threadIdx.x; c0 < nc; c0 += 2 * 256) {
            float lv[2][kCombineFast];
            floatx4 xv[2][kCombineFast];
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                const int c = min(c0 + u * 256, nc - 1);
                const int hq = h0 + c / C, d4 = c % C;
                const float *lp = a.part_lse + (sq.part_off + i) * a.Hq + hq;
                const float *xp = a.part_o + ((sq.part_off + i) * a.Hq + hq) * D + d4 * 4;
#pragma unroll
                for (int s = 0; s < kCombineFast; ++s) {
                    lv[u][s] = s < ns ? lp[s * lstride] : -INFINITY;
                    xv[u][s] = s < ns ? *reinterpret_cast<const floatx4 *>(xp + s * xstride) : floatx4{};
                }
            }
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                const int c = c0 + u * 256;
                if (c >= nc) break;
                float M = -INFINITY;
#pragma unroll
                for (int s = 0; s < kCombineFast; ++s) M = fmaxf(M, lv[u][s]);
                floatx4 acc = {0.f, 0.f, 0.f, 0.f};
                float L = 0.f;
                if (M != -INFINITY) {
#pragma unroll
                    for (int s = 0; s < kCombineFast; ++s) {
                        const float w = s < ns ? exp2f(lv[u][s] - M) : 0.f;
                        L += w;
                        acc += w * xv[u][s];
                    }
                }
                finish(c, acc, M, L);
            }
        }
        return;
    }
    const int nh = hend - h0;
    if (ns <= kCombineLdsSplits && nh <= kCombineLdsHeads) {
        // Every split's lse of the group's heads is loaded once (one round
        // trip) and each head's max, sum and weights computed once, in LDS;
        // then each chunk loads its ns partials kCombineUnroll at a time.
        // Same operations in the same order as the loop below: same bits.
        float *wgt = sm.wgt;
        float *hm = sm.hm, *hl = sm.hl;
        const float *lp0 = a.part_lse + (sq.part_off + i) * a.Hq + h0;
        for (int t = threadIdx.x; t < nh * ns; t += 256) wgt[t] = lp0[(t / ns) + (t % ns) * lstride];
        __syncthreads();
        if (threadIdx.x < nh) {
            const float *l = wgt + threadIdx.x * ns;
            float M = -INFINITY, L = 0.f;
            for (int s = 0; s < ns; ++s) M = fmaxf(M, l[s]);
            if (M != -INFINITY)
                for (int s = 0; s < ns; ++s) L += exp2f(l[s] - M);
            hm[threadIdx.x] = M;
            hl[threadIdx.x] = L;
        }
        __syncthreads();
        for (int t = threadIdx.x; t < nh * ns; t += 256) {
            const float M = hm[t / ns];
            wgt[t] = M == -INFINITY ? 0.f : exp2f(wgt[t] - M);
        }
        __syncthreads();
        for (int c = threadIdx.x; c < nc; c += 256) {
            const int hh = c / C;
            const float *xp = a.part_o + ((sq.part_off + i) * a.Hq + h0 + hh) * D + (c % C) * 4;
            const float *w = wgt + hh * ns;
            floatx4 acc = {0.f, 0.f, 0.f, 0.f};
            if (hm[hh] != -INFINITY) {
                int s = 0;
                for (; s + kCombineUnroll <= ns; s += kCombineUnroll) {
                    floatx4 x[kCombineUnroll];
#pragma unroll
                    for (int u = 0; u < kCombineUnroll; ++u)
                        x[u] = *reinterpret_cast<const floatx4 *>(xp + (s + u) * xstride);
#pragma unroll
                    for (int u = 0; u < kCombineUnroll; ++u) acc += w[s + u] * x[u];
                }
                for (; s < ns; ++s) acc += w[s] * *reinterpret_cast<const floatx4 *>(xp + s * xstride);
            }
            finish(c, acc, hm[hh], hl[hh]);
        }
        return;
    }
    for (int c = threadIdx.x; c < nc; c += 256) {
        const int hq = h0 + c / C, d4 = c % C;
        const float *lp = a.part_lse + (sq.part_off + i) * a.Hq + hq;   // split s at + s*lstride
        const float *xp = a.part_o + ((sq.part_off + i) * a.Hq + hq) * D + d4 * 4;
        float M = -INFINITY;
#pragma unroll 4
        for (int s = 0; s < ns; ++s) M = fmaxf(M, lp[s * lstride]);
        floatx4 acc = {0.f, 0.f, 0.f, 0.f};
        float L = 0.f;
        if (M != -INFINITY) {
#pragma unroll 4
            for (int s = 0; s < ns; ++s) {
                const float w = exp2f(lp[s * lstride] - M);
                L += w;
                const floatx4 x = *reinterpret_cast<const floatx4 *>(xp + s * xstride);
                acc += w * x;
            }
        }
        finish(c, acc, M, L);
    }
}

// --------------------------------------------------------------------------
// Generic kernel: fp32, bf16 or fp16 inputs, any head_dim <= 256 (multiple of 8),
// scalar FMA.  One workgroup = 16 query rows of one (request, KV head).
// DMAX sizes the LDS tiles: 128 (42 KB) for head_dim <= 128, 256 (83 KB)
// above, as the reference kernel takes any power-of-two head_dim.
// --------------------------------------------------------------------------
template <typename T, typename E>
__device__ __forceinline__ float load_elem(const T *p) {
    if constexpr (sizeof(T) == 2)
        return E::widen(*p);
    else
        return *p;
}

// T: float or uint16_t; E: the 16-bit format when T is 2 bytes
template <typename T, int DMAX, typename E>
__global__ __launch_bounds__(256) void tree_attn_generic_kernel(AttnArgs a, int D) {
    constexpr int R = 16, BK = 32;
    __shared__ float Qs[R][DMAX];
    __shared__ float Ks[BK][DMAX + 1];
    __shared__ float Vs[BK][DMAX];
    __shared__ float Ps[R][BK];

    // items: (b, h, 16-row block); rows_wg == 16 for this kernel
    Seq sq;
    int local;
    if (!batch_prologue(a, batch_totals(a))) return;
    if (!find_request(a, blockIdx.x, false, sq, local)) return;
    const int rb = local % sq.rb;
    const int h = local / (sq.rb * sq.ns);
    const int rows = sq.P * a.G;
    const int tid = threadIdx.x;
    const int row = tid >> 4, sub = tid & 15;
    const int r = rb * R + row;
    const bool valid = r < rows;
    const int tok = sq.q0 + (valid ? r / a.G : 0);
    const int hq = h * a.G + (valid ? r % a.G : 0);
    const T *qp = static_cast<const T *>(a.q);
    const KvView<T> kv(a.kv, sq, h);
    for (int d = sub; d < D; d += 16)
        Qs[row][d] = valid ? load_elem<T, E>(qp + (int64_t)tok * a.q_tok + (int64_t)hq * a.q_head + d) : 0.f;
    uint64_t w0 = 0, w1 = 0;
    if (valid) {
        w0 = a.mask[(int64_t)tok * a.mask_words];
        if (a.mask_words > 1) w1 = a.mask[(int64_t)tok * a.mask_words + 1];
    }
    float m = -INFINITY, l = 0.f;
    float acc[DMAX / 16];
#pragma unroll
    for (int e = 0; e < DMAX / 16; ++e) acc[e] = 0.f;

    for (int t0 = 0; t0 < sq.T; t0 += BK) {
        __syncthreads();
        for (int c = tid; c < BK * D; c += 256) {
            const int key = c / D, d = c % D;
            const int kk = t0 + key;
            const bool in = kk < sq.T;
            Ks[key][d] = in ? load_elem<T, E>(kv.key(kk, sq.S) + d) : 0.f;
            Vs[key][d] = in ? load_elem<T, E>(kv.val(kk, sq.S) + d) : 0.f;
        }
        __syncthreads();
        float sv[2];
        for (int e = 0; e < 2; ++e) {
            const int key = sub + 16 * e;
            float dot = 0.f;
            for (int d = 0; d < D; ++d) dot = fmaf(Qs[row][d], Ks[key][d], dot);
            const int kk = t0 + key;
            const bool vis = kk < sq.T && (kk < sq.S || pack_bit(kk - sq.S, w0, w1));
            sv[e] = vis ? dot * a.scale_log2 : -INFINITY;
        }
        float mx = fmaxf(sv[0], sv[1]);
        for (int off = 8; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off));
        const float mn = fmaxf(m, mx);
        const float alpha = mn == -INFINITY ? 1.f : exp2f(m - mn);
        const float ms = mn == -INFINITY ? 0.f : mn;
        const float p0 = exp2f(sv[0] - ms), p1 = exp2f(sv[1] - ms);
        float ps = p0 + p1;
        for (int off = 8; off > 0; off >>= 1) ps += __shfl_xor(ps, off);
        l = l * alpha + ps;
        m = mn;
        Ps[row][sub] = p0;
        Ps[row][sub + 16] = p1;
        __syncthreads();
        for (int e = 0; e < DMAX / 16; ++e) {
            const int d = sub + 16 * e;
            if (d < D) {
                float x = acc[e] * alpha;
                for (int key = 0; key < BK; ++key) x = fmaf(Ps[row][key], Vs[key][d], x);
                acc[e] = x;
            }
        }
    }
    if (!valid) return;
    const float inv = l > 0.f ? 1.f / l : 0.f;
    T *op = static_cast<T *>(a.out) + (int64_t)tok * a.o_tok + (int64_t)hq * a.o_head;
    for (int e = 0; e < DMAX / 16; ++e) {
        const int d = sub + 16 * e;
        if (d >= D) continue;
        const float x = acc[e] * inv;
        if constexpr (sizeof(T) == 2)
            op[d] = (uint16_t)(E::pack2(x, 0.f) & 0xffffu);
        else
            op[d] = x;
    }
    if (a.lse && sub == 0)
        a.lse[(int64_t)tok * a.Hq + hq] = l > 0.f ? ((m == -INFINITY ? 0.f : m) + log2f(l)) * kLn2 : -INFINITY;
}

// --------------------------------------------------------------------------
// Host side
// --------------------------------------------------------------------------
// The current device's compute units and XCDs, looked up once per device;
// an MI355X's 256 and 8 where no device is visible (host-only size queries
// on a machine without a GPU).
struct Topology {
    int cus, xcds;
};
constexpr int kMaxTopoDevices = 64;
static Topology device_topology() {
    static std::mutex mu;
    static Topology cache[kMaxTopoDevices];
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxTopoDevices) return {256, 8};
    std::lock_guard<std::mutex> lock(mu);
    Topology &t = cache[dev];
    if (t.cus == 0) {
        int cus = 0, xcds = 0;
        if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
            cus = 256;
        if (hipDeviceGetAttribute(&xcds, hipDeviceAttributeNumberOfXccs, dev) != hipSuccess || xcds <= 0 ||
            cus % xcds)
            xcds = 1;
        t = {cus, xcds};
    }
    return t;
}

static bool mfma_path(int32_t dtype, int32_t D) {
    if (dtype == CAST_FP32) return D == 64 || D == 128 || D == 256;
    return (dtype == CAST_BF16 || dtype == CAST_FP16) && (D == 64 || D == 128 || D == 256);
}

// Waves per workgroup (32 query rows each) for the largest possible pack.
// (The fp32 kernel has no 2-wave instance: its staging registers would not
// fit beside the Q and O operands.)
// Head_dim 256 always runs 4 waves, one per SIMD: fewer threads would each
// stage more of its 32 KB tiles than the registers hold.
static int waves_for(int32_t total_q, int32_t G, int32_t dtype, int32_t D) {
    const int pmax = total_q < kMaxPack ? total_q : kMaxPack;
    const int rows = pmax * G;
    if (D == 256) return 4;
    const int w = rows <= 64 ? 2 : rows <= 128 ? 4 : 8;
    return dtype == CAST_FP32 && w < 4 ? 4 : w;
}

static int32_t resolve_chunk(int32_t batch, int32_t total_q, int32_t total_kv, int32_t Hq, int32_t Hkv,
                             int32_t D, int32_t dtype, int32_t kv_split) {
    if (!mfma_path(dtype, D) || kv_split < 0 || batch <= 0) return kNoSplit;
    if (kv_split > 0) return ((kv_split + 63) / 64) * 64;
    const int G = Hq / Hkv;
    const int rows_wg = waves_for(total_q, G, dtype, D) * 32;
    const int64_t p_avg = (total_q + batch - 1) / batch;
    const int64_t p_est = p_avg < kMaxPack ? p_avg : kMaxPack;
    const int64_t rb = (p_est * G + rows_wg - 1) / rows_wg;
    const int64_t units = (int64_t)Hkv * batch * (rb > 0 ? rb : 1);
    const int64_t t_avg = (total_kv + batch - 1) / batch;
    const int cus = device_topology().cus;
    if (units >= cus) return kNoSplit;
    int64_t chunk = (t_avg * units + cus - 1) / cus;
    chunk = ((chunk + 63) / 64) * 64;
    if (chunk < kMinChunk) chunk = kMinChunk;
    if (chunk >= t_avg) return kNoSplit;
    return (int32_t)chunk;
}

static int64_t part_rows_bound(int32_t total_q, int32_t total_kv, int32_t chunk) {
    const int64_t pmax = total_q < kMaxPack ? total_q : kMaxPack;
    return (pmax * (int64_t)total_kv + chunk - 1) / chunk + total_q;
}

static size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

// kv_split value that asks for the stream-K schedule.
constexpr int32_t kSplitStreamK = -2;

// The MFMA attention kernel instance of a call and its block size.
struct AttnKernel {
    const void *fn;
    int threads;
};
template <int DD, int W, int WPE, bool SKI>
static AttnKernel mfma_instance(bool f16, bool store) {
    const void *fn =
        f16 ? (store ? reinterpret_cast<const void *>(&tree_attn_mfma_kernel<DD, W, true, Fp16, WPE, SKI>)
                     : reinterpret_cast<const void *>(&tree_attn_mfma_kernel<DD, W, false, Fp16, WPE, SKI>))
            : (store ? reinterpret_cast<const void *>(&tree_attn_mfma_kernel<DD, W, true, Bf16, WPE, SKI>)
                     : reinterpret_cast<const void *>(&tree_attn_mfma_kernel<DD, W, false, Bf16, WPE, SKI>));
    return {fn, W * 64};
}
template <int DD, int W, int WPE, bool SKI>
static AttnKernel f32_instance(bool store) {
    const void *fn = store ? reinterpret_cast<const void *>(&tree_attn_f32_kernel<DD, W, true, WPE, SKI>)
                           : reinterpret_cast<const void *>(&tree_attn_f32_kernel<DD, W, false, WPE, SKI>);
    return {fn, W * 64};
}
template <bool SKI>
static AttnKernel attn_kernel_of(int32_t dtype, int32_t D, int waves, bool store) {
    if (dtype == CAST_FP32) {
        if (D == 128) return waves == 4 ? f32_instance<128, 4, 1, SKI>(store) : f32_instance<128, 8, 2, SKI>(store);
        return waves == 4 ? f32_instance<64, 4, 2, SKI>(store) : f32_instance<64, 8, 2, SKI>(store);
    }
    const bool f16 = dtype == CAST_FP16;
    if (D == 128) {
        if (waves == 2) return mfma_instance<128, 2, 1, SKI>(f16, store);
        return waves == 4 ? mfma_instance<128, 4, 2, SKI>(f16, store) : mfma_instance<128, 8, 2, SKI>(f16, store);
    }
    if (waves == 2) return mfma_instance<64, 2, 2, SKI>(f16, store);
    return waves == 4 ? mfma_instance<64, 4, 2, SKI>(f16, store) : mfma_instance<64, 8, 2, SKI>(f16, store);
}
// Head dims 64 and 128 run 2, 4 or 8 waves (bf16 / fp16) or 4 or 8 (fp32);
// head dim 256 runs 4 (static schedule only).  WPE (waves per
// SIMD of the register budget) as the kernels' comments give it; sk picks
// the stream-K instance.
static AttnKernel attn_kernel(int32_t dtype, int32_t D, int waves, bool store, bool sk) {
    if (D == 256)
        return dtype == CAST_FP32 ? f32_instance<256, 4, 1, false>(store)
                                  : mfma_instance<256, 4, 1, false>(dtype == CAST_FP16, store);
    return sk ? attn_kernel_of<true>(dtype, D, waves, store) : attn_kernel_of<false>(dtype, D, waves, store);
}

// Workgroups of kernel k resident on one CU of the current device (1 where
// no device is visible), looked up once per (device, kernel).
static int resident_per_cu(const AttnKernel &k) {
    struct Entry {
        int dev;
        const void *fn;
        int n;
    };
    static std::mutex mu;
    static Entry cache[256];
    static int used = 0;
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess) return 1;
    std::lock_guard<std::mutex> lock(mu);
    for (int i = 0; i < used; ++i)
        if (cache[i].dev == dev && cache[i].fn == k.fn) return cache[i].n;
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, k.fn, k.threads, 0) != hipSuccess || n < 1) n = 1;
    if (used < 256) cache[used++] = Entry{dev, k.fn, n};
    return n;
}

// Stream-K figures of a call: whether the caller asked for the schedule
// (kv_split = CAST_SPLIT_STREAM, batches of up to 64 requests, head dims 64
// and 128) and its workgroup count - every CU's resident workgroups of the
// concat-layout stream-K instance (the store-layout instance only differs
// in its addressing), a multiple of two per XCD.
struct SkHost {
    int mode, wgs, rows_wg;
};
static SkHost sk_host(int32_t batch, int32_t total_q, int32_t G, int32_t D, int32_t dtype, int32_t kv_split,
                      int32_t chunk) {
    SkHost h{0, 0, 0};
    if (!mfma_path(dtype, D) || D > 128 || batch <= 0 || batch > 64) return h;
    if (kv_split != kSplitStreamK) return h;
    h.mode = 1;
    const int waves = waves_for(total_q, G, dtype, D);
    const Topology topo = device_topology();
    const int per = resident_per_cu(attn_kernel(dtype, D, waves, false, true));
    const int step = 2 * topo.xcds;
    h.wgs = (topo.cus * per) / step * step;
    h.rows_wg = waves * 32;
    if (h.wgs < step) h.mode = 0;
    return h;
}

// Bytes of stream-K partials: O [2 * wgs][rows_wg][D] then lse [2 * wgs][rows_wg].
static size_t sk_bytes(const SkHost &h, int32_t D) {
    if (!h.mode) return 0;
    const size_t rows = (size_t)2 * h.wgs * h.rows_wg;
    return align256(rows * D * sizeof(float)) + align256(rows * sizeof(float));
}

}  // namespace cast

using namespace cast;

extern "C" int32_t cast_tree_attn_default_split(int32_t batch, int32_t total_q, int32_t total_kv,
                                                int32_t num_q_heads, int32_t num_kv_heads,
                                                int32_t head_dim, int32_t dtype) {
    if (num_kv_heads <= 0 || num_q_heads % num_kv_heads) return -1;
    const int32_t c = resolve_chunk(batch, total_q, total_kv, num_q_heads, num_kv_heads, head_dim, dtype, 0);
    return c == kNoSplit ? -1 : c;
}

extern "C" size_t cast_tree_attn_workspace_size(int32_t batch, int32_t total_q, int32_t total_kv,
                                                int32_t num_q_heads, int32_t num_kv_heads,
                                                int32_t head_dim, int32_t dtype, int32_t kv_split) {
    if (batch <= 0 || total_q <= 0 || num_kv_heads <= 0 || num_q_heads % num_kv_heads) return 0;
    const int32_t chunk = resolve_chunk(batch, total_q, total_kv, num_q_heads, num_kv_heads, head_dim,
                                        dtype, kv_split);
    size_t bytes = 0;
    if (chunk != kNoSplit) {
        const int64_t rows = part_rows_bound(total_q, total_kv, chunk);
        bytes = align256((size_t)rows * num_q_heads * head_dim * sizeof(float)) +
                align256((size_t)rows * num_q_heads * sizeof(float));
    }
    const SkHost sk = sk_host(batch, total_q, num_q_heads / num_kv_heads, head_dim, dtype, kv_split, chunk);
    const size_t skb = sk_bytes(sk, head_dim);
    return skb > bytes ? skb : bytes;
}

enum { kStageAttn = 1, kStageCombine = 2 };

static int tree_attn_run(const void *q, const KvSource &kv, void *out, float *lse, const int32_t *cu_q,
                         const int32_t *cu_kv, const int32_t *prefix_len, const int32_t *pack_len,
                         const uint64_t *mask, int32_t mask_words, int32_t batch, int32_t total_q, int32_t total_kv,
                         int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim, int64_t q_tok, int64_t q_head,
                         int64_t o_tok, int64_t o_head, int32_t dtype, float sm_scale, int32_t kv_split,
                         void *workspace, size_t workspace_bytes, int32_t *status, cast_stream_t stream, int stages) {
    if (batch < 0 || total_q < 0 || total_kv < 0 || head_dim <= 0) return CAST_ERR_SHAPE;
    if (num_q_heads <= 0 || num_kv_heads <= 0 || num_q_heads % num_kv_heads) return CAST_ERR_HEAD_RATIO;
    if (dtype != CAST_BF16 && dtype != CAST_FP16 && dtype != CAST_FP32) return CAST_ERR_DTYPE;
    if (mask_words != 1 && mask_words != 2) return CAST_ERR_SHAPE;
    if (kv.store && kv.cap < 0) return CAST_ERR_SHAPE;
    if (!(sm_scale > 0.f) || !isfinite(sm_scale)) return CAST_ERR_SCALE;
    if (batch == 0 || total_q == 0) return CAST_OK;
    if (!q || !kv.k_pre || !kv.v_pre || !kv.k_pack || !kv.v_pack || !out || !cu_q || !prefix_len || !pack_len ||
        !mask || (!kv.store && !cu_kv))
        return CAST_ERR_NULL_POINTER;
    const bool mfma = mfma_path(dtype, head_dim);
    if (!mfma && (head_dim > 256 || head_dim % 8)) return CAST_ERR_HEAD_DIM;
    const int64_t esz = dtype == CAST_FP32 ? 4 : 2;
    int32_t max_rows = INT32_MAX;
    auto a16 = [](const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
    if (mfma) {
        if (!a16(q) || !a16(kv.k_pre) || !a16(kv.v_pre) || !a16(kv.k_pack) || !a16(kv.v_pack) || !a16(out))
            return CAST_ERR_ALIGNMENT;
        const int64_t strides[14] = {q_tok,     q_head,    kv.kpre_b,  kv.kpre_h,  kv.kpre_t,
                                     kv.vpre_b, kv.vpre_h, kv.vpre_t,  kv.kpack_h, kv.kpack_t,
                                     kv.vpack_h, kv.vpack_t, o_tok,    o_head};
        for (int64_t s : strides)
            if ((s * esz) % 16) return CAST_ERR_ALIGNMENT;
        // key rows are addressed by 24-bit row index x 24-bit byte stride,
        // within 2^31 bytes of their source's first row
        const int64_t rows[4] = {kv.kpre_t, kv.vpre_t, kv.kpack_t, kv.vpack_t};
        int64_t rb = 0;
        for (int64_t r : rows) {
            if (r < 0 || r * esz >= (int64_t)1 << 24) return CAST_ERR_SHAPE;
            rb = r * esz > rb ? r * esz : rb;
        }
        const int64_t by_bytes = rb ? (((int64_t)1 << 31) - 1 - head_dim * esz) / rb : INT32_MAX;
        const int64_t by_index = ((int64_t)1 << 24) - 64;
        max_rows = (int32_t)(by_bytes < by_index ? by_bytes : by_index);
    }
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    AttnArgs a{};
    a.q = q;
    a.kv = kv;
    a.out = out;
    a.lse = lse;
    a.cu_q = cu_q;
    a.cu_kv = cu_kv;
    a.prefix_len = prefix_len;
    a.pack_len = pack_len;
    a.mask = mask;
    a.mask_words = mask_words;
    a.batch = batch;
    a.total_q = total_q;
    a.total_kv = total_kv;
    a.Hq = num_q_heads;
    a.Hkv = num_kv_heads;
    a.G = num_q_heads / num_kv_heads;
    a.D = head_dim;
    a.esz = (int32_t)esz;
    a.q_tok = q_tok;
    a.q_head = q_head;
    a.o_tok = o_tok;
    a.o_head = o_head;
    a.scale_log2 = sm_scale * kLog2e;
    a.status = status;
    a.max_rows = max_rows;

    if (!mfma) {
        a.chunk = kNoSplit;
        a.rows_wg = 16;
        const int64_t items = (int64_t)num_kv_heads * (((int64_t)total_q * a.G + 15) / 16 + batch);
        if (!(stages & kStageAttn)) return CAST_OK;
        const bool wide = head_dim > 128;
#define CAST_GENERIC(T, DM, E) tree_attn_generic_kernel<T, DM, E><<<(unsigned)items, 256, 0, st>>>(a, head_dim)
        if (dtype == CAST_FP32) {
            if (wide) CAST_GENERIC(float, 256, Bf16);
            else CAST_GENERIC(float, 128, Bf16);
        } else if (dtype == CAST_FP16) {
            if (wide) CAST_GENERIC(uint16_t, 256, Fp16);
            else CAST_GENERIC(uint16_t, 128, Fp16);
        } else {
            if (wide) CAST_GENERIC(uint16_t, 256, Bf16);
            else CAST_GENERIC(uint16_t, 128, Bf16);
        }
#undef CAST_GENERIC
        return hipGetLastError() == hipSuccess ? CAST_OK : CAST_ERR_HIP;
    }

    const int waves = waves_for(total_q, a.G, dtype, head_dim);
    a.rows_wg = waves * 32;
    a.chunk = resolve_chunk(batch, total_q, total_kv, num_q_heads, num_kv_heads, head_dim, dtype, kv_split);
    const SkHost sk = sk_host(batch, total_q, a.G, head_dim, dtype, kv_split, a.chunk);
    a.sk_mode = sk.mode;
    a.sk_wgs = sk.mode ? sk.wgs : 0;
    a.sk_min_tiles = kMinChunk / 64;
    if (a.chunk != kNoSplit || sk.mode) {
        const size_t need = cast_tree_attn_workspace_size(batch, total_q, total_kv, num_q_heads, num_kv_heads,
                                                          head_dim, dtype, kv_split);
        if (!workspace || workspace_bytes < need) return CAST_ERR_WORKSPACE;
        if (reinterpret_cast<uintptr_t>(workspace) & 255) return CAST_ERR_ALIGNMENT;
        a.part_o = static_cast<float *>(workspace);
        if (a.chunk != kNoSplit) {
            a.part_rows = part_rows_bound(total_q, total_kv, a.chunk);
            a.part_lse = reinterpret_cast<float *>(
                static_cast<char *>(workspace) + align256((size_t)a.part_rows * num_q_heads * head_dim * sizeof(float)));
        }
        if (sk.mode)
            a.sk_lse = reinterpret_cast<float *>(
                static_cast<char *>(workspace) + align256((size_t)2 * sk.wgs * sk.rows_wg * head_dim * sizeof(float)));
    }
    // Grid bound without reading device metadata: every request has at most
    // min(total_q, 128) tokens, so row blocks per (request, head, split) are
    // bounded, and splits sum to at most total_kv / chunk + batch.  The
    // stream-K schedule needs sk_wgs workgroups; the device picks one.
    const int64_t pmax = total_q < kMaxPack ? total_q : kMaxPack;
    const int64_t rbmax = (pmax * a.G + a.rows_wg - 1) / a.rows_wg;
    const int64_t nsplit = a.chunk == kNoSplit ? batch : ((int64_t)total_kv + a.chunk - 1) / a.chunk + batch;
    int64_t items = (int64_t)num_kv_heads * rbmax * nsplit;
    a.xcds = device_topology().xcds;
    items = batch <= 64 ? sorted_slots((int64_t)num_kv_heads * nsplit, rbmax, a.xcds)
                        : (items + a.xcds - 1) / a.xcds * a.xcds;
    if (a.sk_mode && items < a.sk_wgs) items = a.sk_wgs;
    if (items > 0x7fffffff) return CAST_ERR_SHAPE;
    if (stages & kStageAttn) {
        const AttnKernel k = attn_kernel(dtype, head_dim, waves, kv.store != 0, a.sk_mode != 0);
        void *args[] = {&a};
        if (hipLaunchKernel(k.fn, dim3((unsigned)items), dim3(k.threads), args, 0, st) != hipSuccess)
            return CAST_ERR_HIP;
    }
    if (hipGetLastError() != hipSuccess) return CAST_ERR_HIP;
    if ((a.chunk != kNoSplit || a.sk_mode) && (stages & kStageCombine)) {
        // about 1536 workgroups (6 per CU), each with up to 256 output chunks
        // of at most kCombineLdsHeads heads
        const int64_t max_groups = ((int64_t)num_q_heads * (head_dim / 4) + 255) / 256;
        const int64_t min_groups = (num_q_heads + kCombineLdsHeads - 1) / kCombineLdsHeads;
        int64_t g = 1536 / total_q;
        g = g < 1 ? 1 : (g > max_groups ? max_groups : g);
        g = g < min_groups ? min_groups : g;
        a.comb_groups = (int32_t)g;
        const unsigned cg = (unsigned)(total_q * g);
#define CAST_COMBINE(OT, DD, E)                                                         \
    (a.sk_mode ? tree_attn_combine_kernel<OT, DD, E, true><<<cg, 256, 0, st>>>(a) \
               : tree_attn_combine_kernel<OT, DD, E, false><<<cg, 256, 0, st>>>(a))
        if (dtype == CAST_FP32) {
            if (head_dim == 256) tree_attn_combine_kernel<float, 256, Bf16, false><<<cg, 256, 0, st>>>(a);
            else if (head_dim == 128) CAST_COMBINE(float, 128, Bf16);
            else CAST_COMBINE(float, 64, Bf16);
        } else if (dtype == CAST_FP16) {
            if (head_dim == 256) tree_attn_combine_kernel<uint16_t, 256, Fp16, false><<<cg, 256, 0, st>>>(a);
            else if (head_dim == 128) CAST_COMBINE(uint16_t, 128, Fp16);
            else CAST_COMBINE(uint16_t, 64, Fp16);
        } else {
            if (head_dim == 256) tree_attn_combine_kernel<uint16_t, 256, Bf16, false><<<cg, 256, 0, st>>>(a);
            else if (head_dim == 128) CAST_COMBINE(uint16_t, 128, Bf16);
            else CAST_COMBINE(uint16_t, 64, Bf16);
        }
#undef CAST_COMBINE
        if (hipGetLastError() != hipSuccess) return CAST_ERR_HIP;
    }
    return CAST_OK;
}

#define CAST_ATTN_PARAMS                                                                                        \
    const void *q, const void *k, const void *v, void *out, float *lse, const int32_t *cu_q,                 \
        const int32_t *cu_kv, const int32_t *prefix_len, const int32_t *pack_len, const uint64_t *mask,      \
        int32_t mask_words, int32_t batch, int32_t total_q, int32_t total_kv, int32_t num_q_heads,           \
        int32_t num_kv_heads, int32_t head_dim, int64_t q_tok, int64_t q_head, int64_t k_tok, int64_t k_head, \
        int64_t v_tok, int64_t v_head, int64_t o_tok, int64_t o_head, int32_t dtype, float sm_scale,         \
        int32_t kv_split, void *workspace, size_t workspace_bytes, int32_t *status, cast_stream_t stream

static KvSource concat_source(const void *k, const void *v, int64_t k_tok, int64_t k_head, int64_t v_tok,
                              int64_t v_head) {
    KvSource s{};
    s.k_pre = s.k_pack = k;
    s.v_pre = s.v_pack = v;
    s.kpre_t = s.kpack_t = k_tok;
    s.kpre_h = s.kpack_h = k_head;
    s.vpre_t = s.vpack_t = v_tok;
    s.vpre_h = s.vpack_h = v_head;
    s.store = 0;
    return s;
}

#define CAST_CONCAT_RUN(STAGES)                                                                                \
    tree_attn_run(q, concat_source(k, v, k_tok, k_head, v_tok, v_head), out, lse, cu_q, cu_kv, prefix_len,  \
                  pack_len, mask, mask_words, batch, total_q, total_kv, num_q_heads, num_kv_heads, head_dim,  \
                  q_tok, q_head, o_tok, o_head, dtype, sm_scale, kv_split, workspace, workspace_bytes, status, \
                  stream, STAGES)

extern "C" int cast_tree_attn_fwd(CAST_ATTN_PARAMS) { return CAST_CONCAT_RUN(kStageAttn | kStageCombine); }

extern "C" int cast_tree_attn_partial(CAST_ATTN_PARAMS) { return CAST_CONCAT_RUN(kStageAttn); }

extern "C" int cast_tree_attn_combine(CAST_ATTN_PARAMS) { return CAST_CONCAT_RUN(kStageCombine); }

extern "C" int cast_tree_attn_store_fwd(const void *q, const void *k_store, const void *v_store, const void *k_pack,
                                        const void *v_pack, void *out, float *lse, const int32_t *cu_q,
                                        const int32_t *prefix_len, const int32_t *pack_len, const uint64_t *mask,
                                        int32_t mask_words, int32_t batch, int32_t total_q, int32_t total_kv,
                                        int32_t store_cap, int32_t num_q_heads, int32_t num_kv_heads,
                                        int32_t head_dim, int64_t q_tok, int64_t q_head, int64_t ks_batch,
                                        int64_t ks_head, int64_t ks_tok, int64_t vs_batch, int64_t vs_head,
                                        int64_t vs_tok, int64_t kp_tok, int64_t kp_head, int64_t vp_tok,
                                        int64_t vp_head, int64_t o_tok, int64_t o_head, int32_t dtype,
                                        float sm_scale, int32_t kv_split, void *workspace, size_t workspace_bytes,
                                        int32_t *status, cast_stream_t stream) {
    KvSource s{};
    s.k_pre = k_store;
    s.v_pre = v_store;
    s.k_pack = k_pack;
    s.v_pack = v_pack;
    s.kpre_b = ks_batch;
    s.kpre_h = ks_head;
    s.kpre_t = ks_tok;
    s.vpre_b = vs_batch;
    s.vpre_h = vs_head;
    s.vpre_t = vs_tok;
    s.kpack_t = kp_tok;
    s.kpack_h = kp_head;
    s.vpack_t = vp_tok;
    s.vpack_h = vp_head;
    s.store = 1;
    s.cap = store_cap;
    return tree_attn_run(q, s, out, lse, cu_q, nullptr, prefix_len, pack_len, mask, mask_words, batch, total_q,
                         total_kv, num_q_heads, num_kv_heads, head_dim, q_tok, q_head, o_tok, o_head, dtype,
                         sm_scale, kv_split, workspace, workspace_bytes, status, stream, kStageAttn | kStageCombine);
}

// --------------------------------------------------------------------------
// No-allocation entry point: the split-K partials live in a static device
// array instead of a caller workspace, for callers that cannot allocate
// (code under HIP graph capture, tight serving loops, harnesses that forbid
// hipMalloc).  Each GPU the library runs on holds its own copy of the array
// until the process ends.  Nothing in it must start at zero: every partial
// row the combine reads is written by the attention kernel of the same call.
// Calls that overlap on one GPU (other streams, other host threads) share
// the array and race.
// --------------------------------------------------------------------------
namespace cast {
constexpr size_t kScratchBytes = (size_t)72 << 20;
constexpr int kMaxDevices = 64;
}  // namespace cast

static __device__ __align__(256) unsigned char scratch[cast::kScratchBytes];

namespace {
std::mutex g_scratch_mu;
void *g_scratch_ptr[cast::kMaxDevices];   // device address of `scratch` per GPU

// The array's device address on the current GPU, looked up once per device
// with that device current.  The host-side name `scratch` is only a stand-in
// and never reaches a kernel.
int scratch_for_current_device(void **out) {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= cast::kMaxDevices) return CAST_ERR_HIP;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void *p = nullptr;
        if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) return CAST_ERR_HIP;
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return CAST_OK;
}
}  // namespace

extern "C" size_t cast_tree_attn_noalloc_limit(void) { return cast::kScratchBytes; }

extern "C" int cast_tree_attn_fwd_noalloc(const void *q, const void *k, const void *v, void *out, float *lse,
                                          const int32_t *cu_q, const int32_t *cu_kv, const int32_t *prefix_len,
                                          const int32_t *pack_len, const uint64_t *mask, int32_t mask_words,
                                          int32_t batch, int32_t total_q, int32_t total_kv, int32_t num_q_heads,
                                          int32_t num_kv_heads, int32_t head_dim, int64_t q_tok, int64_t q_head,
                                          int64_t k_tok, int64_t k_head, int64_t v_tok, int64_t v_head,
                                          int64_t o_tok, int64_t o_head, int32_t dtype, float sm_scale,
                                          int32_t kv_split, int32_t *status, cast_stream_t stream) {
    const size_t need = cast_tree_attn_workspace_size(batch, total_q, total_kv, num_q_heads, num_kv_heads,
                                                      head_dim, dtype, kv_split);
    if (need > cast::kScratchBytes) return CAST_ERR_SCRATCH_LIMIT;
    void *ws = nullptr;
    if (need) {
        if (stream) {
            int cur = -1, sdev = -1;
            if (hipGetDevice(&cur) != hipSuccess ||
                hipStreamGetDevice(reinterpret_cast<hipStream_t>(stream), &sdev) != hipSuccess)
                return CAST_ERR_HIP;
            if (cur != sdev) return CAST_ERR_DEVICE;
        }
        const int st = scratch_for_current_device(&ws);
        if (st != CAST_OK) return st;
    }
    void *workspace = ws;
    const size_t workspace_bytes = need ? cast::kScratchBytes : 0;
    return CAST_CONCAT_RUN(kStageAttn | kStageCombine);
}
