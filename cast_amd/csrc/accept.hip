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
//                Streams the logits once with 16-byte loads (HBM-bound).
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

template <bool BF16>
__global__ __launch_bounds__(256) void row_argmax_kernel(const void *__restrict__ logits, int64_t ld,
                                                         int32_t vocab, int32_t *__restrict__ argmax) {
    constexpr int NT = 256;
    constexpr int EPC = BF16 ? 8 : 4;   // elements per 16-byte chunk
    const int row = blockIdx.x;
    const int tid = threadIdx.x;
    float best = -INFINITY;
    int bi = INT_MAX;
    const size_t esz = BF16 ? 2 : 4;
    const char *base = static_cast<const char *>(logits) + (size_t)row * (size_t)ld * esz;
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
                v = bf16_to_float((uint16_t)(bits >> ((e & 1) * 16)));
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
            v = bf16_to_float(reinterpret_cast<const uint16_t *>(base)[i]);
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
    if (dtype != CAST_BF16 && dtype != CAST_FP32) return CAST_ERR_DTYPE;
    if (batch == 0) return CAST_OK;
    if (!logits || !cu_q || !parent || !token || !argmax || !path || !path_len || !bonus)
        return CAST_ERR_NULL_POINTER;
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    if (total_q > 0) {
        if (dtype == CAST_BF16)
            row_argmax_kernel<true><<<total_q, 256, 0, s>>>(logits, logits_ld, vocab, argmax);
        else
            row_argmax_kernel<false><<<total_q, 256, 0, s>>>(logits, logits_ld, vocab, argmax);
        if (hipGetLastError() != hipSuccess) return CAST_ERR_HIP;
    }
    tree_walk_kernel<<<batch, 64, 0, s>>>(cu_q, parent, token, argmax, total_q, path, path_len, bonus, status);
    return hipGetLastError() == hipSuccess ? CAST_OK : CAST_ERR_HIP;
}
