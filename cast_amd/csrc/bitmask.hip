// K1: packed ancestor bitmask builder.
//
// Replaces the per-round host loop of cast_trees/serving.py:213-222, which
// builds one int64 per packed row as bits[i+1] = bits[parent+1] | 1 << (i+1),
// and the dense cast_trees/tree.py:85-93 ancestor matrix that word encodes.
// One workgroup owns one pack: its parents are staged in LDS, then every
// thread walks its own row's chain to the root, setting bit j for each
// pack-local index j on the way (at most 128 steps, each checked to move to a
// strictly smaller index, so malformed input cannot loop).
#include "cast_common.hpp"

namespace cast {

template <int WORDS>
__global__ __launch_bounds__(kMaxPack) void tree_bitmask_kernel(
    const int32_t *__restrict__ parent, const int32_t *__restrict__ cu_q, int32_t total_q,
    uint64_t *__restrict__ words_out, int32_t *status) {
    __shared__ int32_t par[kMaxPack];
    const int b = blockIdx.x;
    const int base = cu_q[b];
    const int end = cu_q[b + 1];
    const int P = end - base;
    const int limit = WORDS * 64;
    if (base < 0 || end > total_q || P < 0) {
        if (threadIdx.x == 0) raise_flag(status, CAST_FLAG_BAD_OFFSETS);
        return;
    }
    if (P > limit) {
        if (threadIdx.x == 0) raise_flag(status, CAST_FLAG_BAD_PACK);
        for (int r = threadIdx.x; r < P; r += blockDim.x)
            for (int w = 0; w < WORDS; ++w) words_out[(size_t)(base + r) * WORDS + w] = 0;
        return;
    }
    const int i = threadIdx.x;
    if (i < P) par[i] = parent[base + i];
    __syncthreads();
    if (i >= P) return;
    uint64_t w[WORDS];
#pragma unroll
    for (int q = 0; q < WORDS; ++q) w[q] = 0;
    int j = i;
    bool bad = false;
    for (int step = 0; step < kMaxPack; ++step) {
        w[j >> 6] |= 1ull << (j & 63);
        const int p = par[j];
        if (p == -1) break;
        if (p < 0 || p >= j) {
            bad = true;
            break;
        }
        j = p;
    }
    if (bad) raise_flag(status, CAST_FLAG_BAD_PARENT);
#pragma unroll
    for (int q = 0; q < WORDS; ++q) words_out[(size_t)(base + i) * WORDS + q] = w[q];
}

}  // namespace cast

using namespace cast;

extern "C" int cast_abi_version(void) { return 4; }

extern "C" const char *cast_status_string(int status) {
    switch (status) {
        case CAST_OK: return "ok";
        case CAST_ERR_NULL_POINTER: return "a required pointer is NULL";
        case CAST_ERR_HEAD_RATIO: return "query heads must be a multiple of KV heads";
        case CAST_ERR_PACK_TOO_LARGE: return "a pack holds at most 128 tokens (64 with one mask word)";
        case CAST_ERR_DTYPE: return "unsupported element type";
        case CAST_ERR_HEAD_DIM: return "unsupported head dimension";
        case CAST_ERR_ALIGNMENT: return "pointers and strides must be 16-byte aligned, head dim contiguous";
        case CAST_ERR_SHAPE: return "negative or inconsistent sizes";
        case CAST_ERR_WORKSPACE: return "workspace smaller than cast_tree_attn_workspace_size";
        case CAST_ERR_SCALE: return "softmax scale must be finite and positive";
        case CAST_ERR_HIP: return "a HIP runtime call or kernel launch failed";
        case CAST_ERR_SCRATCH_LIMIT:
            return "the split-K scratch this call needs exceeds the no-allocation entry point's static array "
                   "(use a workspace, or a larger kv_split)";
        case CAST_ERR_DEVICE: return "the stream belongs to another device than the current one";
        case CAST_ERR_ALIAS: return "an output overlaps an input that the kernels still read";
        default: return "unknown status";
    }
}

extern "C" int cast_tree_bitmask(const int32_t *parent, const int32_t *cu_q, int32_t batch,
                                 int32_t total_q, int32_t words_per_row, uint64_t *words_out,
                                 int32_t *status, cast_stream_t stream) {
    if (batch < 0 || total_q < 0) return CAST_ERR_SHAPE;
    if (words_per_row != 1 && words_per_row != 2) return CAST_ERR_SHAPE;
    if (batch == 0 || total_q == 0) return CAST_OK;
    if (!parent || !cu_q || !words_out) return CAST_ERR_NULL_POINTER;
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    if (words_per_row == 1)
        tree_bitmask_kernel<1><<<batch, kMaxPack, 0, s>>>(parent, cu_q, total_q, words_out, status);
    else
        tree_bitmask_kernel<2><<<batch, kMaxPack, 0, s>>>(parent, cu_q, total_q, words_out, status);
    return hipGetLastError() == hipSuccess ? CAST_OK : CAST_ERR_HIP;
}
