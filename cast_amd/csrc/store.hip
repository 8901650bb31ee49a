// K4: accepted-path KV append into the per-request store, up to 64 layers per
// launch.
//
// Replaces the per-layer scatter of cast_trees/serving.py:264-289
// (_append_store): for every surviving request b, the pack rows it keeps -
// the root and its accepted nodes, keep = [0] + [i + 1 for i in path]
// (serving.py:328-330) - are copied from the verify pass's pack K/V of each
// layer (serving.py:62, [Hkv, total_q, D]) to store slots
// store_len[b] .. store_len[b] + len(path) of buf[layer][b] ([B, Hkv, cap, D]).
// The reference issues two advanced-indexing copies per layer; here one
// workgroup per (request, layer, KV head, column slice of at most 512 bytes
// of each row) moves 16-byte chunks, driven by the
// greedy-accept kernel's device-side path / path_len (no host round trip).
// The per-layer base addresses come from host arrays and travel in the
// kernel arguments, up to 64 layers per launch: a decode loop whose pack
// tensors are new every round pays no table upload and no host sync.
//
// Every workgroup loads all of its rows before it stores any (registers,
// then a barrier), so the copy is also correct in place: pack and store may
// be the same tensor, as in the batch-one cache compaction of
// cast_trees/verify.py:48-60 (gather_cache), where row n_prefix + keep[j]
// moves to n_prefix + j.  Different (request, layer, head, column slice)
// tuples never share an address.
#include "cast_common.hpp"

namespace cast {

// Layers per launch: their four base addresses travel in the kernel
// arguments (4 x 64 x 8 B = 2 KiB), so the call needs no device table.
constexpr int kAppendLayersPerLaunch = 64;

struct AppendArgs {
    const void *k_pack[kAppendLayersPerLaunch];   // pack K of each layer of this launch
    const void *v_pack[kAppendLayersPerLaunch];
    void *k_store[kAppendLayersPerLaunch];        // store K of each layer
    void *v_store[kAppendLayersPerLaunch];
    int32_t batch, total_q, cap, Hkv, chunks;     // chunks = 16-byte pieces per (row, head)
    int32_t slices;                               // column slices per (row, head): ceil(chunks / 32)
    int32_t first_launch;                         // writes new_len and the per-request flag
    const int32_t *src_row;      // [batch] packed row of request b's root (cu_q of its pack)
    const int32_t *path;         // [batch][path_stride] accepted node indices (-1 padded)
    int32_t path_stride;
    const int32_t *path_len;     // [batch]
    const int32_t *store_len;    // [batch] tokens already in request b's slot
    int32_t *new_len;            // [batch] out: store_len + path_len + 1 (nullable)
    int64_t kp_tok, kp_head, vp_tok, vp_head;             // bytes
    int64_t ks_batch, ks_head, ks_tok, vs_batch, vs_head, vs_tok;   // bytes
    int32_t *status;
};

constexpr int kAppendThreads = 256;
constexpr int kAppendMaxChunks = 32;   // 16-byte chunks of each row one workgroup moves (512 B)
constexpr int kAppendPerThread = kMaxPack * kAppendMaxChunks / kAppendThreads;

__global__ __launch_bounds__(kAppendThreads) void store_append_kernel(AppendArgs a) {
    const int b = blockIdx.x, layer = blockIdx.y;
    const int h = blockIdx.z / a.slices, slice = blockIdx.z % a.slices;
    // this workgroup's columns of every row: chunks [c0, c0 + width)
    const int c0 = slice * kAppendMaxChunks;
    const int width = min(kAppendMaxChunks, a.chunks - c0);
    const int n = a.path_len[b];
    const int s0 = a.store_len[b];
    const int root = a.src_row[b];
    const int count = n + 1;     // root + accepted nodes
    if (n < 0 || n >= kMaxPack || s0 < 0 || s0 + count > a.cap || root < 0 || root >= a.total_q) {
        if (threadIdx.x == 0 && layer == 0 && blockIdx.z == 0 && a.first_launch)
            raise_flag(a.status, CAST_FLAG_BAD_OFFSETS);
        return;
    }
    if (threadIdx.x == 0 && layer == 0 && blockIdx.z == 0 && a.first_launch && a.new_len) a.new_len[b] = s0 + count;
    const char *kp = static_cast<const char *>(a.k_pack[layer]) + (int64_t)h * a.kp_head;
    const char *vp = static_cast<const char *>(a.v_pack[layer]) + (int64_t)h * a.vp_head;
    char *ks = static_cast<char *>(a.k_store[layer]) + (int64_t)b * a.ks_batch + (int64_t)h * a.ks_head;
    char *vs = static_cast<char *>(a.v_store[layer]) + (int64_t)b * a.vs_batch + (int64_t)h * a.vs_head;
    const int total = count * width;   // <= kMaxPack * kAppendMaxChunks
    // phase 1: every row this workgroup moves, into registers
    u32x4 kx[kAppendPerThread], vx[kAppendPerThread];
    bool ok[kAppendPerThread];
#pragma unroll
    for (int u = 0; u < kAppendPerThread; ++u) {
        const int idx = threadIdx.x + u * kAppendThreads;
        ok[u] = false;
        if (idx < total) {
            const int j = idx / width, c = c0 + idx % width;
            // keep[j]: the root (pack index 0), then node path[j-1] at pack index path[j-1] + 1
            int pk = 0;
            if (j > 0) pk = a.path[(int64_t)b * a.path_stride + j - 1] + 1;
            if (pk >= 1 || j == 0) {
                if (root + pk < a.total_q) {
                    const int64_t src = (int64_t)(root + pk);
                    kx[u] = *reinterpret_cast<const u32x4 *>(kp + src * a.kp_tok + c * 16);
                    vx[u] = *reinterpret_cast<const u32x4 *>(vp + src * a.vp_tok + c * 16);
                    ok[u] = true;
                }
            }
            if (!ok[u]) raise_flag(a.status, CAST_FLAG_BAD_OFFSETS);
        }
    }
    __syncthreads();
    // phase 2: the stores
#pragma unroll
    for (int u = 0; u < kAppendPerThread; ++u) {
        const int idx = threadIdx.x + u * kAppendThreads;
        if (idx < total && ok[u]) {
            const int j = idx / width, c = c0 + idx % width;
            const int64_t dst = (int64_t)(s0 + j);
            *reinterpret_cast<u32x4 *>(ks + dst * a.ks_tok + c * 16) = kx[u];
            *reinterpret_cast<u32x4 *>(vs + dst * a.vs_tok + c * 16) = vx[u];
        }
    }
}

}  // namespace cast

using namespace cast;

extern "C" int cast_store_append(const void *const *k_pack, const void *const *v_pack, void *const *k_store,
                                 void *const *v_store, int32_t layers, const int32_t *src_row,
                                 const int32_t *path, int32_t path_stride, const int32_t *path_len,
                                 const int32_t *store_len, int32_t *new_len, int32_t batch, int32_t total_q,
                                 int32_t cap, int32_t num_kv_heads, int32_t head_dim, int64_t kp_tok,
                                 int64_t kp_head, int64_t vp_tok, int64_t vp_head, int64_t ks_batch,
                                 int64_t ks_head, int64_t ks_tok, int64_t vs_batch, int64_t vs_head,
                                 int64_t vs_tok, int32_t dtype, int32_t *status, cast_stream_t stream) {
    if (layers < 0 || batch < 0 || total_q < 0 || cap < 0 || num_kv_heads <= 0 || head_dim <= 0 ||
        path_stride < kMaxPack)
        return CAST_ERR_SHAPE;
    if (dtype != CAST_BF16 && dtype != CAST_FP16 && dtype != CAST_FP32) return CAST_ERR_DTYPE;
    if (layers == 0 || batch == 0) return CAST_OK;
    if (!k_pack || !v_pack || !k_store || !v_store || !src_row || !path || !path_len || !store_len)
        return CAST_ERR_NULL_POINTER;
    const int64_t esz = dtype == CAST_FP32 ? 4 : 2;   // a row copy: only the element size matters
    if ((head_dim * esz) % 16 || head_dim * esz > 16 * 1024) return CAST_ERR_HEAD_DIM;
    const int64_t slices = (head_dim * esz / 16 + kAppendMaxChunks - 1) / kAppendMaxChunks;
    if ((int64_t)num_kv_heads * slices > 65535) return CAST_ERR_SHAPE;
    // new_len is written while other workgroups (and later launches) still
    // read store_len, path_len, src_row and path: it must not overlap them
    if (new_len) {
        auto overlaps = [&](const int32_t *p, int64_t n) {
            const uintptr_t a0 = reinterpret_cast<uintptr_t>(new_len), a1 = a0 + (uintptr_t)batch * 4;
            const uintptr_t b0 = reinterpret_cast<uintptr_t>(p), b1 = b0 + (uintptr_t)n * 4;
            return a0 < b1 && b0 < a1;
        };
        if (overlaps(store_len, batch) || overlaps(path_len, batch) || overlaps(src_row, batch) ||
            overlaps(path, (int64_t)batch * path_stride))
            return CAST_ERR_ALIAS;
    }
    const int64_t strides[10] = {kp_tok, kp_head, vp_tok, vp_head, ks_batch, ks_head, ks_tok, vs_batch, vs_head, vs_tok};
    for (int64_t s : strides)
        if ((s * esz) % 16) return CAST_ERR_ALIGNMENT;
    for (int32_t l = 0; l < layers; ++l)
        if (!k_pack[l] || !v_pack[l] || !k_store[l] || !v_store[l]) return CAST_ERR_NULL_POINTER;
    AppendArgs a{};
    a.batch = batch;
    a.total_q = total_q;
    a.cap = cap;
    a.Hkv = num_kv_heads;
    a.chunks = (int32_t)(head_dim * esz / 16);
    a.slices = (a.chunks + kAppendMaxChunks - 1) / kAppendMaxChunks;
    a.src_row = src_row;
    a.path = path;
    a.path_stride = path_stride;
    a.path_len = path_len;
    a.store_len = store_len;
    a.new_len = new_len;
    a.kp_tok = kp_tok * esz;
    a.kp_head = kp_head * esz;
    a.vp_tok = vp_tok * esz;
    a.vp_head = vp_head * esz;
    a.ks_batch = ks_batch * esz;
    a.ks_head = ks_head * esz;
    a.ks_tok = ks_tok * esz;
    a.vs_batch = vs_batch * esz;
    a.vs_head = vs_head * esz;
    a.vs_tok = vs_tok * esz;
    a.status = status;
    for (int32_t l0 = 0; l0 < layers; l0 += kAppendLayersPerLaunch) {
        const int32_t n = layers - l0 < kAppendLayersPerLaunch ? layers - l0 : kAppendLayersPerLaunch;
        for (int32_t l = 0; l < n; ++l) {
            a.k_pack[l] = k_pack[l0 + l];
            a.v_pack[l] = v_pack[l0 + l];
            a.k_store[l] = k_store[l0 + l];
            a.v_store[l] = v_store[l0 + l];
        }
        a.first_launch = l0 == 0;
        store_append_kernel<<<dim3(batch, n, num_kv_heads * a.slices), kAppendThreads, 0,
                              reinterpret_cast<hipStream_t>(stream)>>>(a);
        if (hipGetLastError() != hipSuccess) return CAST_ERR_HIP;
    }
    return CAST_OK;
}
