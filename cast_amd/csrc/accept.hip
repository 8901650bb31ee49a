// K3: greedy accepted-path walk, entirely on the device.
//
// Replaces the temperature-0 branch of cast_trees/decode.py:85-103 and its
// pick rule (decode.py:13-15), which the reference runs per request on the
// host with one device->host sync per visited node
// (cast_trees/serving.py:326-335).
//
// Two kernels on the caller's stream:
//   row_argmax   one workgroup per packed row: first index of the row
//                maximum, NaN counting as the maximum (torch.argmax rule).
//                Streams the logits once with 16-byte loads.  bf16 and fp16
//                rows compare 16-bit order keys two at a time (see below), a
//                row holding a NaN takes the exact element-by-element scan.
//   tree_walk    one wave per request: starting at the root row, finds the
//                first child (lowest pack index, i.e. node order) whose draft
//                token equals the row's argmax with one ballot per level,
//                and follows it until no child matches.  Each step moves to
//                a strictly larger pack index, so at most P steps run.
#include <limits.h>

#include "cast_common.hpp"

namespace cast {

// (v1, i1) beats (v2, i2): NaN beats everything, larger beats smaller, ties
// go to the smaller index.
__device__ __forceinline__ bool better(float v1, int i1, float v2, int i2) {
    const bool n1 = v1 != v1, n2 = v2 != v2;
    if (n1 || n2) return n1 && (!n2 || i1 < i2);
    return v1 > v2 || (v1 == v2 && i1 < i2);
}

// Element formats of a logits row: F32 (float), or Bf16 / Fp16 (16-bit).
struct F32 {};
template <typename F>
constexpr bool kHalf = !__is_same(F, F32);

// The first index of the maximum of one row (base, vocab elements), NaN
// counting as the maximum, element by element; the workgroup's 256 threads
// call it together and thread 0 writes *out.
template <typename F>
__device__ void argmax_exact(const char *__restrict__ base, int32_t vocab, int32_t *__restrict__ out) {
    constexpr int NT = 256;
    constexpr bool BF16 = kHalf<F>;     // 16-bit elements (bf16 or fp16)
    constexpr int EPC = BF16 ? 8 : 4;   // elements per 16-byte chunk
    const int tid = threadIdx.x;
    float best = -INFINITY;
    int bi = INT_MAX;
    const bool vec = ((reinterpret_cast<uintptr_t>(base) & 15) == 0);
    const int nch = vec ? vocab / EPC : 0;
    // A thread visits its elements in increasing index order, so an element
    // replaces the running best iff it is the first, strictly greater, or the
    // first NaN: ties keep the earlier index and a NaN best is never replaced.
    // Branch-free (compares and selects only).
    auto take = [&](float v, int i) {
        const bool t = (v > best) | ((v != v) & (best == best));
        best = t ? v : best;
        bi = t ? i : bi;
    };
    auto scan_chunk = [&](const u32x4 &w, int c, bool first) {
#pragma unroll
        for (int e = 0; e < EPC; ++e) {
            float v;
            // copy the lane element to a scalar first: a bit cast of a
            // vector element expression reads the vector's first element
            const uint32_t bits = w[BF16 ? (e >> 1) : e];
            if constexpr (BF16)
                v = F::widen((uint16_t)(bits >> ((e & 1) * 16)));
            else
                v = __builtin_bit_cast(float, bits);
            if (first && e == 0) {   // the thread's first element seeds the running best
                best = v;
                bi = c * EPC;
            } else {
                take(v, c * EPC + e);
            }
        }
    };
    // UNR independent 16-byte loads in flight per thread, then the compares
    // (in increasing index order per thread, as the tie rule needs)
    constexpr int UNR = 4;
    int c = tid;
    if (c < nch) {
        scan_chunk(*reinterpret_cast<const u32x4 *>(base + (size_t)c * 16), c, true);
        c += NT;
    }
    for (; c + (UNR - 1) * NT < nch; c += UNR * NT) {
        u32x4 w[UNR];
#pragma unroll
        for (int u = 0; u < UNR; ++u) w[u] = *reinterpret_cast<const u32x4 *>(base + (size_t)(c + u * NT) * 16);
#pragma unroll
        for (int u = 0; u < UNR; ++u) scan_chunk(w[u], c + u * NT, false);
    }
    for (; c < nch; c += NT) scan_chunk(*reinterpret_cast<const u32x4 *>(base + (size_t)c * 16), c, false);
    for (int i = nch * EPC + tid; i < vocab; i += NT) {
        float v;
        if constexpr (BF16)
            v = F::widen(reinterpret_cast<const uint16_t *>(base)[i]);
        else
            v = reinterpret_cast<const float *>(base)[i];
        if (bi == INT_MAX) {     // no vector chunk seeded this thread
            best = v;
            bi = i;
        } else {
            take(v, i);
        }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const float ov = __shfl_xor(best, off);
        const int oi = __shfl_xor(bi, off);
        if (better(ov, oi, best, bi)) {
            best = ov;
            bi = oi;
        }
    }
    __shared__ float sv[NT / 64];
    __shared__ int si[NT / 64];
    if ((tid & 63) == 0) {
        sv[tid >> 6] = best;
        si[tid >> 6] = bi;
    }
    __syncthreads();
    if (tid == 0) {
        for (int w = 1; w < NT / 64; ++w)
            if (better(sv[w], si[w], best, bi)) {
                best = sv[w];
                bi = si[w];
            }
        *out = bi;
    }
}

template <typename F>
__global__ __launch_bounds__(256) void row_argmax_kernel(const void *__restrict__ logits, int64_t ld,
                                                         int32_t vocab, int32_t *__restrict__ argmax) {
    const char *base = static_cast<const char *>(logits) + (size_t)blockIdx.x * (size_t)ld * (kHalf<F> ? 2 : 4);
    argmax_exact<F>(base, vocab, argmax + blockIdx.x);
}

// ---- 16-bit rows by order keys.  A bf16 or fp16 value with magnitude bits
// m (sign cleared) gets the 16-bit two's-complement key m when non-negative
// and -m when negative: both are sign-magnitude formats whose magnitude bits
// order as the magnitudes do.  Keys order exactly as the values do for every
// non-NaN pair, and -0 and +0 share key 0, so equal values tie as the float
// compare has them.  A NaN has m above the magnitude of infinity (0x7f80 in
// bf16, 0x7c00 in fp16); a row that holds one is left to the exact scan,
// since NaN outranks every value there.
typedef short s16x2 __attribute__((ext_vector_type(2)));
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));

// The keys of the two bf16 values of one dword, and their magnitudes.  With
// s = -1 for a negative half (0 otherwise), (bits ^ (s & 0x7fff)) - s is m
// for a non-negative value and 0x8000 | (0x7fff - m), plus one, = -m mod 2^16
// for a negative one: no select needed.
__device__ __forceinline__ s16x2 bf16x2_key(uint32_t bits, u16x2 &mag) {
    mag = __builtin_bit_cast(u16x2, bits & 0x7fff7fffu);
    const s16x2 sv = __builtin_bit_cast(s16x2, bits) >> (short)15;
    const uint32_t x = bits ^ (__builtin_bit_cast(uint32_t, sv) & 0x7fff7fffu);
    return __builtin_bit_cast(s16x2, x) - sv;
}
__device__ __forceinline__ int bf16_key(uint16_t bits) {
    const int m = bits & 0x7fff;
    return (bits & 0x8000) ? -m : m;
}

// Per thread: the largest key of its 16-byte chunks (visited in increasing
// order) and the first chunk holding it; then that chunk alone is read
// again for the first element with the key.  Per element the scan costs
// about three VALU operations against about nine for the float compare.
template <typename F>   // Bf16 or Fp16
__global__ __launch_bounds__(256) void row_argmax_bf16_kernel(const void *__restrict__ logits, int64_t ld,
                                                              int32_t vocab, int32_t *__restrict__ argmax) {
    constexpr int NT = 256;
    constexpr unsigned short kInfMag = __is_same(F, Fp16) ? 0x7c00 : 0x7f80;
    constexpr int EPC = 8;
    const int row = blockIdx.x;
    const int tid = threadIdx.x;
    const char *base = static_cast<const char *>(logits) + (size_t)row * (size_t)ld * 2;
    const bool vec = ((reinterpret_cast<uintptr_t>(base) & 15) == 0);
    const int nch = vec ? vocab / EPC : 0;
    int bk = INT_MIN, bc = -1;          // best chunk key, first chunk holding it
    u16x2 magmax = {0, 0};
    auto chunk_key = [&](const u32x4 &w) {
        u16x2 m0, m1, m2, m3;
        const s16x2 k0 = bf16x2_key(w[0], m0), k1 = bf16x2_key(w[1], m1);
        const s16x2 k2 = bf16x2_key(w[2], m2), k3 = bf16x2_key(w[3], m3);
        magmax = __builtin_elementwise_max(magmax, __builtin_elementwise_max(__builtin_elementwise_max(m0, m1),
                                                                             __builtin_elementwise_max(m2, m3)));
        const s16x2 k = __builtin_elementwise_max(__builtin_elementwise_max(k0, k1), __builtin_elementwise_max(k2, k3));
        return max((int)k[0], (int)k[1]);
    };
    auto visit = [&](const u32x4 &w, int c) {
        const int k = chunk_key(w);
        if (k > bk) {
            bk = k;
            bc = c;
        }
    };
    // 8 chunks in flight per thread: 32 KB per workgroup, enough bytes in
    // flight to cover the memory latency at the four workgroups per CU of a
    // 1024-row launch
    constexpr int UNR = 8;
    int c = tid;
    for (; c + (UNR - 1) * NT < nch; c += UNR * NT) {
        u32x4 w[UNR];
#pragma unroll
        for (int u = 0; u < UNR; ++u) w[u] = *reinterpret_cast<const u32x4 *>(base + (size_t)(c + u * NT) * 16);
#pragma unroll
        for (int u = 0; u < UNR; ++u) visit(w[u], c + u * NT);
    }
    for (; c < nch; c += NT) visit(*reinterpret_cast<const u32x4 *>(base + (size_t)c * 16), c);
    // the thread's first element holding bk: inside chunk bc
    int bi = INT_MAX;
    if (bc >= 0) {
        const u32x4 w = *reinterpret_cast<const u32x4 *>(base + (size_t)bc * 16);
#pragma unroll
        for (int e = EPC - 1; e >= 0; --e) {
            const uint32_t bits = w[e >> 1];
            if (bf16_key((uint16_t)(bits >> ((e & 1) * 16))) == bk) bi = bc * EPC + e;
        }
    }
    // elements past the last whole chunk (or all of an unaligned row): their
    // indices follow every chunk's, so they win only on a larger key
    for (int i = nch * EPC + tid; i < vocab; i += NT) {
        const uint16_t bits = reinterpret_cast<const uint16_t *>(base)[i];
        const int m = bits & 0x7fff;
        magmax[0] = max(magmax[0], (unsigned short)m);
        const int k = bf16_key(bits);
        if (k > bk || bi == INT_MAX) {
            bk = k;
            bi = i;
        }
    }
    const bool nan = max(magmax[0], magmax[1]) > kInfMag;
    if (__syncthreads_or(nan)) {
        argmax_exact<F>(base, vocab, argmax + row);
        return;
    }
    // (key desc, index asc) over the workgroup
    auto wins = [](int k1, int i1, int k2, int i2) { return k1 > k2 || (k1 == k2 && i1 < i2); };
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const int ok = __shfl_xor(bk, off);
        const int oi = __shfl_xor(bi, off);
        if (wins(ok, oi, bk, bi)) {
            bk = ok;
            bi = oi;
        }
    }
    __shared__ int sk[NT / 64], si[NT / 64];
    if ((tid & 63) == 0) {
        sk[tid >> 6] = bk;
        si[tid >> 6] = bi;
    }
    __syncthreads();
    if (tid == 0) {
        for (int w = 1; w < NT / 64; ++w)
            if (wins(sk[w], si[w], bk, bi)) {
                bk = sk[w];
                bi = si[w];
            }
        argmax[row] = bi;
    }
}

__global__ __launch_bounds__(64) void tree_walk_kernel(const int32_t *__restrict__ cu_q,
                                                       const int32_t *__restrict__ parent,
                                                       const int64_t *__restrict__ token,
                                                       const int32_t *__restrict__ argmax, int32_t total_q,
                                                       int32_t *__restrict__ path, int32_t *__restrict__ path_len,
                                                       int64_t *__restrict__ bonus, int32_t *status) {
    const int b = blockIdx.x;
    const int lane = threadIdx.x;
    const int base = cu_q[b];
    const int P = cu_q[b + 1] - base;
    int32_t *my_path = path + (size_t)b * kMaxPack;
    if (base < 0 || cu_q[b + 1] > total_q || P < 1 || P > kMaxPack) {
        if (lane == 0) {
            raise_flag(status, P > kMaxPack ? CAST_FLAG_BAD_PACK : CAST_FLAG_BAD_OFFSETS);
            path_len[b] = 0;
            bonus[b] = -1;
        }
        my_path[lane] = -1;
        my_path[lane + 64] = -1;
        return;
    }
    // each lane holds pack indices lane and lane + 64
    int par[2];
    int64_t tok[2];
    bool bad = false;
#pragma unroll
    for (int e = 0; e < 2; ++e) {
        const int j = lane + 64 * e;
        par[e] = -2;
        tok[e] = 0;
        if (j < P && j > 0) {
            const int p = parent[base + j];
            if (p >= 0 && p < j) {
                par[e] = p;
                tok[e] = token[base + j];
            } else {
                bad = true;
            }
        }
    }
    if (lane == 0 && parent[base] != -1) bad = true;
    if (__any(bad) && lane == 0) raise_flag(status, CAST_FLAG_BAD_PARENT);

    int cur = 0, len = 0;
    int64_t next = argmax[base];
    for (int step = 0; step < P; ++step) {
        next = argmax[base + cur];
        const uint64_t m0 = __ballot(par[0] == cur && tok[0] == next);
        const uint64_t m1 = __ballot(par[1] == cur && tok[1] == next);
        int j;
        if (m0)
            j = __builtin_ctzll(m0);
        else if (m1)
            j = 64 + __builtin_ctzll(m1);
        else
            break;
        if (lane == 0) my_path[len] = j - 1;
        ++len;
        cur = j;
    }
    if (lane >= len) my_path[lane] = -1;
    if (lane + 64 >= len) my_path[lane + 64] = -1;
    if (lane == 0) {
        path_len[b] = len;
        bonus[b] = next;
    }
}

}  // namespace cast

using namespace cast;

extern "C" int cast_greedy_accept(const void *logits, int64_t logits_ld, int32_t vocab, int32_t dtype,
                                  const int32_t *cu_q, const int32_t *parent, const int64_t *token,
                                  int32_t batch, int32_t total_q, int32_t *argmax, int32_t *path,
                                  int32_t *path_len, int64_t *bonus, int32_t *status, cast_stream_t stream) {
    if (batch < 0 || total_q < 0 || vocab <= 0 || logits_ld < vocab) return CAST_ERR_SHAPE;
    if (dtype != CAST_BF16 && dtype != CAST_FP16 && dtype != CAST_FP32) return CAST_ERR_DTYPE;
    if (batch == 0) return CAST_OK;
    if (!logits || !cu_q || !parent || !token || !argmax || !path || !path_len || !bonus)
        return CAST_ERR_NULL_POINTER;
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    if (total_q > 0) {
        if (dtype == CAST_BF16)
            row_argmax_bf16_kernel<Bf16><<<total_q, 256, 0, s>>>(logits, logits_ld, vocab, argmax);
        else if (dtype == CAST_FP16)
            row_argmax_bf16_kernel<Fp16><<<total_q, 256, 0, s>>>(logits, logits_ld, vocab, argmax);
        else
            row_argmax_kernel<F32><<<total_q, 256, 0, s>>>(logits, logits_ld, vocab, argmax);
        if (hipGetLastError() != hipSuccess) return CAST_ERR_HIP;
    }
    tree_walk_kernel<<<batch, 64, 0, s>>>(cu_q, parent, token, argmax, total_q, path, path_len, bonus, status);
    return hipGetLastError() == hipSuccess ? CAST_OK : CAST_ERR_HIP;
}
