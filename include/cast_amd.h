/*
 * cast_amd.h - C ABI of the MI355X (gfx950) tree-verification library.
 *
 * Plain pointers and sizes only.  Every pointer argument is device memory
 * unless stated otherwise; every entry point is stream-ordered on the
 * hipStream_t passed as `stream` (NULL = the null stream), performs no host
 * synchronisation and allocates nothing: scratch memory is passed in by the
 * caller.  Entry points validate their host-side arguments before touching
 * the GPU and return a cast_status code; metadata that lives on the device
 * (pack lengths, offsets, parents) is checked by the kernels, which skip the
 * offending request and raise a bit in the optional device status word.
 *
 * Packed layout (cast_trees/serving.py:211-231): request b owns query rows
 * [cu_q[b], cu_q[b+1]) = its pack (root + tree nodes, P_b = pack_len[b] <= 128
 * tokens) and key/value rows [cu_kv[b], cu_kv[b+1]) = concat(prefix of
 * S_b = prefix_len[b] tokens, pack).  Bit j of a row's ancestor words marks
 * pack-local key j visible; word w holds bits 64w..64w+63.
 */
#ifndef CAST_AMD_H
#define CAST_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void *cast_stream_t; /* a hipStream_t */

enum cast_status {
    CAST_OK = 0,
    CAST_ERR_NULL_POINTER = 1,     /* a required pointer is NULL */
    CAST_ERR_HEAD_RATIO = 2,       /* query heads not a multiple of KV heads */
    CAST_ERR_PACK_TOO_LARGE = 3,   /* a pack bound above 128 tokens (or 64 with one word) */
    CAST_ERR_DTYPE = 4,            /* unsupported element type */
    CAST_ERR_HEAD_DIM = 5,         /* unsupported head dimension */
    CAST_ERR_ALIGNMENT = 6,        /* pointer or stride breaks the 16-byte rule */
    CAST_ERR_SHAPE = 7,            /* negative or inconsistent sizes */
    CAST_ERR_WORKSPACE = 8,        /* workspace smaller than the queried size */
    CAST_ERR_SCALE = 9,            /* softmax scale not finite and positive */
    CAST_ERR_HIP = 10,             /* a HIP runtime call or launch failed */
    CAST_ERR_SCRATCH_LIMIT = 11,   /* the no-allocation entry point would need more
                                      split-K scratch than its static array holds */
    CAST_ERR_DEVICE = 12,          /* the stream's device is not the current device */
    CAST_ERR_ALIAS = 13            /* an output overlaps an input the kernels still read */
};

/* Bits a kernel ORs into the optional device status word (int32). */
enum cast_device_flag {
    CAST_FLAG_BAD_PACK = 1,        /* pack_len outside [1, 128] or beyond the mask words */
    CAST_FLAG_BAD_OFFSETS = 2,     /* cu_q / cu_kv / prefix_len inconsistent with totals */
    CAST_FLAG_BAD_PARENT = 4,      /* a parent index not in [-1, own index) */
    CAST_FLAG_TOO_LONG = 8         /* a request's key source exceeds the kernel's
                                      row addressing (bf16 MFMA path: 2^24 - 64
                                      rows and 2^31 bytes per source) */
};

enum cast_dtype { CAST_BF16 = 0, CAST_FP32 = 1, CAST_FP64 = 2, CAST_FP16 = 3 };

/* Library ABI version (bumped on any signature change). */
int cast_abi_version(void);

/* Human-readable text of a cast_status code. */
const char *cast_status_string(int status);

/* ---------------------------------------------------------------------
 * K1: packed ancestor bitmask.
 * Replaces the host loop of cast_trees/serving.py:213-222 (and the dense
 * cast_trees/tree.py:85-93 ancestor_matrix it encodes).
 *   parent     int32 [total_q]  pack-local parent of every packed row, -1 at
 *                               each pack's root (row 0 of the pack)
 *   cu_q       int32 [batch+1]  pack offsets
 *   words_out  uint64 [total_q][words_per_row]; words_per_row 1 gives the
 *                               reference's int64 word (packs <= 64 tokens),
 *                               2 covers packs <= 128 tokens
 *   status     int32*, nullable device status word (cast_device_flag bits)
 * ------------------------------------------------------------------- */
int cast_tree_bitmask(const int32_t *parent, const int32_t *cu_q, int32_t batch,
                      int32_t total_q, int32_t words_per_row, uint64_t *words_out,
                      int32_t *status, cast_stream_t stream);

/* ---------------------------------------------------------------------
 * K2: ragged ancestor-masked tree-verification attention (forward).
 * Replaces the tile schedule and kernel launch of
 * cast_trees/tree_attn.py:116-139 (kernel body tree_attn.py:17-92).
 *   q      [total_q,  Hq,  D]  strides (q_tok, q_head, 1), in elements
 *   k, v   [total_kv, Hkv, D]  strides (k_tok, k_head, 1) / (v_tok, v_head, 1)
 *   out    [total_q,  Hq,  D]  strides (o_tok, o_head, 1), same dtype as q
 *   lse    float [total_q, Hq] contiguous, natural-log log-sum-exp of the
 *                              scaled scores over visible keys; nullable
 *   cu_q, cu_kv  int32 [batch+1];  prefix_len, pack_len  int32 [batch]
 *   mask   uint64 [total_q][mask_words], mask_words 1 (int64 reference
 *          layout) or 2
 *   dtype  cast_dtype of q, k, v and out: CAST_BF16, CAST_FP16 or CAST_FP32
 *   head_dim  64, 128 or 256 on the MFMA kernels; any other multiple of 8
 *          up to 256 on a scalar kernel (the reference takes any power of
 *          two)
 *   sm_scale  > 0 (the Python layer substitutes 1/sqrt(D) for None)
 *   kv_split  keys per split-K chunk (multiple of 64); 0 lets the library
 *             choose; CAST_SPLIT_STREAM (-2) asks for the stream-K schedule;
 *             any other negative value disables split-K.  With 0 the library
 *             cuts long prefixes into equal splits so that the work items
 *             cover the device's CUs (static schedule, longest items first).
 *             Stream-K (only when asked for): pairs of workgroups on one XCD
 *             get equal ranges of key tiles over all (request, KV head, row
 *             block) units, and a combine merges the pieces of units cut
 *             between workgroups; the pieces' cut points follow the batch
 *             order.  The static schedule sums each request's keys in an
 *             order that only depends on batch totals.
 *   workspace / workspace_bytes  scratch of at least
 *             cast_tree_attn_workspace_size(...) bytes, 256-byte aligned
 *   status    int32*, nullable device status word
 * Rows with no visible key produce zeros and lse = -inf.  So do the rows of
 * every request the kernels reject on its device-side metadata (pack longer
 * than 64 * mask_words, offsets that disagree with prefix_len / pack_len,
 * keys beyond the row addressing) and rows outside every request; a batch
 * whose accepted packs or keys exceed total_q / total_kv, or whose cu_q
 * decreases, is rejected whole.  Rejections also raise *status bits.
 * ------------------------------------------------------------------- */
int cast_tree_attn_fwd(const void *q, const void *k, const void *v, void *out, float *lse,
                       const int32_t *cu_q, const int32_t *cu_kv, const int32_t *prefix_len,
                       const int32_t *pack_len, const uint64_t *mask, int32_t mask_words,
                       int32_t batch, int32_t total_q, int32_t total_kv, int32_t num_q_heads,
                       int32_t num_kv_heads, int32_t head_dim, int64_t q_tok, int64_t q_head,
                       int64_t k_tok, int64_t k_head, int64_t v_tok, int64_t v_head,
                       int64_t o_tok, int64_t o_head, int32_t dtype, float sm_scale,
                       int32_t kv_split, void *workspace, size_t workspace_bytes,
                       int32_t *status, cast_stream_t stream);

/* The two stages of cast_tree_attn_fwd, same arguments, for callers that
 * interleave other work or time the stages separately:
 *   _partial  the attention kernel; requests that are split over keys leave
 *             their rows of out/lse unwritten and their partials in workspace
 *   _combine  merges those partials into out/lse (a no-op without split-K)
 * Same-stream order partial -> combine equals cast_tree_attn_fwd.  Both
 * replace the same reference launch (cast_trees/tree_attn.py:128-138). */
int cast_tree_attn_partial(const void *q, const void *k, const void *v, void *out, float *lse,
                           const int32_t *cu_q, const int32_t *cu_kv, const int32_t *prefix_len,
                           const int32_t *pack_len, const uint64_t *mask, int32_t mask_words,
                           int32_t batch, int32_t total_q, int32_t total_kv, int32_t num_q_heads,
                           int32_t num_kv_heads, int32_t head_dim, int64_t q_tok, int64_t q_head,
                           int64_t k_tok, int64_t k_head, int64_t v_tok, int64_t v_head,
                           int64_t o_tok, int64_t o_head, int32_t dtype, float sm_scale,
                           int32_t kv_split, void *workspace, size_t workspace_bytes,
                           int32_t *status, cast_stream_t stream);
int cast_tree_attn_combine(const void *q, const void *k, const void *v, void *out, float *lse,
                           const int32_t *cu_q, const int32_t *cu_kv, const int32_t *prefix_len,
                           const int32_t *pack_len, const uint64_t *mask, int32_t mask_words,
                           int32_t batch, int32_t total_q, int32_t total_kv, int32_t num_q_heads,
                           int32_t num_kv_heads, int32_t head_dim, int64_t q_tok, int64_t q_head,
                           int64_t k_tok, int64_t k_head, int64_t v_tok, int64_t v_head,
                           int64_t o_tok, int64_t o_head, int32_t dtype, float sm_scale,
                           int32_t kv_split, void *workspace, size_t workspace_bytes,
                           int32_t *status, cast_stream_t stream);

/* ---------------------------------------------------------------------
 * K2 over a per-request KV store, read in place.
 * Replaces the per-layer ragged K/V assembly of the reference attention hook
 * (cast_trees/serving.py:61-68: prefix gathered out of buf_k/buf_v
 * [B, Hkv, cap, D], pack scattered behind it, both up-cast to fp32) and the
 * call it feeds (serving.py:69-71 -> cast_trees/tree_attn.py:116-139).
 * Request b's keys are its S_b = prefix_len[b] stored tokens followed by its
 * P_b pack tokens; nothing is copied:
 *   k_store, v_store  prefix key t of request b, head h at
 *                     base + b*ks_batch + h*ks_head + t*ks_tok (elements);
 *                     S_b <= store_cap is checked on the device
 *   k_pack, v_pack    pack key j of request b, head h at
 *                     base + (cu_q[b] + j)*kp_tok + h*kp_head, i.e. the
 *                     forward's own K/V [Hkv, total_q, D] in any strides
 *   total_kv          a bound on sum_b (S_b + P_b) (sizes grid and workspace;
 *                     a batch above it is flagged CAST_FLAG_BAD_OFFSETS)
 * Every other argument and the output are as in cast_tree_attn_fwd; the
 * workspace is cast_tree_attn_workspace_size(batch, total_q, total_kv, ...).
 * ------------------------------------------------------------------- */
int cast_tree_attn_store_fwd(const void *q, const void *k_store, const void *v_store,
                             const void *k_pack, const void *v_pack, void *out, float *lse,
                             const int32_t *cu_q, const int32_t *prefix_len, const int32_t *pack_len,
                             const uint64_t *mask, int32_t mask_words, int32_t batch, int32_t total_q,
                             int32_t total_kv, int32_t store_cap, int32_t num_q_heads,
                             int32_t num_kv_heads, int32_t head_dim, int64_t q_tok, int64_t q_head,
                             int64_t ks_batch, int64_t ks_head, int64_t ks_tok, int64_t vs_batch,
                             int64_t vs_head, int64_t vs_tok, int64_t kp_tok, int64_t kp_head,
                             int64_t vp_tok, int64_t vp_head, int64_t o_tok, int64_t o_head,
                             int32_t dtype, float sm_scale, int32_t kv_split, void *workspace,
                             size_t workspace_bytes, int32_t *status, cast_stream_t stream);

/* ---------------------------------------------------------------------
 * cast_tree_attn_fwd without a workspace argument: allocates nothing.
 * No counterpart in the reference.  For callers that cannot allocate device
 * memory during the call: code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc.  The split-K partials go to a static
 * device array of cast_tree_attn_noalloc_limit() bytes (72 MiB), which every
 * GPU the library runs on holds until the process ends.  Calls whose
 * cast_tree_attn_workspace_size(...) exceeds it return
 * CAST_ERR_SCRATCH_LIMIT before any device work (a larger kv_split, or -1,
 * needs less).  Call with the stream's device current (else
 * CAST_ERR_DEVICE).  Every call on one GPU shares that GPU's array: calls
 * that overlap on one GPU (other streams or host threads) race.  Arguments
 * and results are otherwise those of cast_tree_attn_fwd, with the same
 * kernels and the same output bits.
 * ------------------------------------------------------------------- */
int cast_tree_attn_fwd_noalloc(const void *q, const void *k, const void *v, void *out, float *lse,
                               const int32_t *cu_q, const int32_t *cu_kv, const int32_t *prefix_len,
                               const int32_t *pack_len, const uint64_t *mask, int32_t mask_words,
                               int32_t batch, int32_t total_q, int32_t total_kv, int32_t num_q_heads,
                               int32_t num_kv_heads, int32_t head_dim, int64_t q_tok, int64_t q_head,
                               int64_t k_tok, int64_t k_head, int64_t v_tok, int64_t v_head,
                               int64_t o_tok, int64_t o_head, int32_t dtype, float sm_scale,
                               int32_t kv_split, int32_t *status, cast_stream_t stream);
/* Bytes of the static split-K scratch of cast_tree_attn_fwd_noalloc. */
size_t cast_tree_attn_noalloc_limit(void);

/* kv_split value asking for the stream-K schedule (batches of up to 64
 * requests on the MFMA kernels with head dims 64 and 128; otherwise the
 * same as -1). */
#define CAST_SPLIT_STREAM (-2)

/* Workspace bytes cast_tree_attn_fwd needs for these host-known sizes (and
 * the current device's CU count: the stream-K partials take two slots of
 * rows_per_workgroup x (head_dim + 1) floats per resident workgroup). */
size_t cast_tree_attn_workspace_size(int32_t batch, int32_t total_q, int32_t total_kv,
                                     int32_t num_q_heads, int32_t num_kv_heads,
                                     int32_t head_dim, int32_t dtype, int32_t kv_split);

/* The split-K chunk (keys) the library would choose for kv_split = 0. */
int32_t cast_tree_attn_default_split(int32_t batch, int32_t total_q, int32_t total_kv,
                                     int32_t num_q_heads, int32_t num_kv_heads,
                                     int32_t head_dim, int32_t dtype);

/* ---------------------------------------------------------------------
 * K3: greedy accepted-path walk over verify logits, no host sync.
 * Replaces the temperature-0 walk of cast_trees/decode.py:85-103 (pick at
 * decode.py:13-15) called per request at cast_trees/serving.py:326-335.
 *   logits   [total_q, vocab], row stride logits_ld elements, dtype
 *            CAST_BF16, CAST_FP16 or CAST_FP32; packed row r = pack row
 *            (root first)
 *   cu_q     int32 [batch+1];  parent int32 [total_q] pack-local (-1 root)
 *   token    int64 [total_q]  draft token of every packed row (root ignored)
 *   argmax   int32 [total_q]  out: first index of each row's maximum
 *            (NaN counts as the maximum, as torch.argmax)
 *   path     int32 [batch][128] out: accepted node indices (pack index - 1),
 *            root-to-leaf, -1 padded
 *   path_len int32 [batch] out: accepted nodes per request
 *   bonus    int64 [batch] out: the target's token after the accepted path
 *   status   int32*, nullable device status word
 * ------------------------------------------------------------------- */
int cast_greedy_accept(const void *logits, int64_t logits_ld, int32_t vocab, int32_t dtype,
                       const int32_t *cu_q, const int32_t *parent, const int64_t *token,
                       int32_t batch, int32_t total_q, int32_t *argmax, int32_t *path,
                       int32_t *path_len, int64_t *bonus, int32_t *status,
                       cast_stream_t stream);

/* ---------------------------------------------------------------------
 * K4: accepted-path KV append into the per-request store, every layer in
 * one launch.  Replaces the per-layer scatter of cast_trees/serving.py:
 * 264-289 (_append_store, two indexed copies per layer).
 *   k_pack / v_pack    HOST arrays of `layers` device pointers to each
 *                      layer's pack K / V [Hkv, total_q, D] (strides kp_* /
 *                      vp_*, in elements, shared by all layers)
 *   k_store / v_store  HOST arrays of `layers` device pointers to each
 *                      layer's store [batch, Hkv, cap, D] (strides ks_* / vs_*)
 *                      The addresses travel in the kernel arguments (64
 *                      layers per launch), so the arrays may be reused or
 *                      freed as soon as the call returns.
 *   src_row   int32 [batch]  packed row of request b's root (cu_q of its pack)
 *   path      int32 [batch][path_stride >= 128]  accepted node indices, as
 *             written by cast_greedy_accept;  path_len int32 [batch]
 *   store_len int32 [batch]  tokens already in request b's slot
 *   new_len   int32 [batch]  out (nullable): store_len + path_len + 1.  It
 *             must not overlap store_len, path_len, src_row or path (other
 *             workgroups still read them when it is written): an in-place
 *             length update is refused with CAST_ERR_ALIAS
 * Request b keeps its root and its accepted nodes (keep = [0] + [i + 1 for
 * i in path], cast_trees/serving.py:328-330) at slots store_len[b] .. in
 * order.  A request that would pass `cap` is skipped and flagged
 * CAST_FLAG_BAD_OFFSETS.  head_dim * element size: a multiple of 16 bytes,
 * at most 16 KiB (rows above 512 bytes are moved in 512-byte column slices,
 * one workgroup each).
 * Pack and store may be the same memory (each (request, layer, head) is
 * read whole before it is written): this is also the batch-one in-place
 * compaction of cast_trees/verify.py:48-60 (gather_cache), with the pack
 * at row n_prefix of the cache, store_len = n_prefix and batch = 1.
 * ------------------------------------------------------------------- */
int cast_store_append(const void *const *k_pack, const void *const *v_pack, void *const *k_store,
                      void *const *v_store, int32_t layers, const int32_t *src_row,
                      const int32_t *path, int32_t path_stride, const int32_t *path_len,
                      const int32_t *store_len, int32_t *new_len, int32_t batch, int32_t total_q,
                      int32_t cap, int32_t num_kv_heads, int32_t head_dim, int64_t kp_tok,
                      int64_t kp_head, int64_t vp_tok, int64_t vp_head, int64_t ks_batch,
                      int64_t ks_head, int64_t ks_tok, int64_t vs_batch, int64_t vs_head,
                      int64_t vs_tok, int32_t dtype, int32_t *status, cast_stream_t stream);

/* ---------------------------------------------------------------------
 * K5: drafter top-k marginals and best-first tree build on the device.
 * cast_draft_topk replaces topk_marginals (cast_trees/verify.py:8-12; the
 * log_softmax + topk + .cpu() of cast_trees/serving.py:126-128):
 *   logits   [rows, vocab] bf16 / fp16 / fp32, row stride logits_ld elements
 *   top_idx  int64 [rows][k] token ids, top_lp  float [rows][k] log-probs,
 *            ranked by descending log-probability, equal values in
 *            increasing index order (cast_trees/tree.py:20-26); 1 <= k <= 16,
 *            k <= vocab.  -inf logits rank by index like any value; NaN
 *            logits never rank (a row with fewer than k non-NaN entries gets
 *            index -1 and a NaN log-prob in its last slots), and a NaN or
 *            +inf anywhere in a row makes its log-probs NaN, as log_softmax
 *            does.
 *   splits   workgroups per row (0 = chosen from rows and vocab so that the
 *            grid covers the GPU); with more than one, each writes its
 *            slice's top k and log-sum-exp into workspace and a second
 *            kernel merges them
 *   workspace / workspace_bytes  at least
 *            cast_draft_topk_workspace_size(rows, vocab, dtype, k, splits)
 *            bytes, 16-byte aligned (may be NULL when that size is 0)
 * cast_build_trees replaces build_tree (cast_trees/tree.py:29-49), one tree
 * per request, the same heap order (-score, depth, parent, rank, counter):
 *   top_idx / top_lp  [batch][L][k] as written by cast_draft_topk; top_lp
 *            float (lp_dtype CAST_FP32) or double (CAST_FP64)
 *   budget   int32 [batch] non-root nodes wanted (<= 127; larger values
 *            are clamped and flag CAST_FLAG_BAD_PACK in *status)
 *   token int64, depth int32, parent int32 (node index, -1 = root child),
 *   score double: [batch][127] nodes in pop order;  n_nodes int32 [batch]
 *   1 <= L <= 255, 1 <= k <= 16.  Log-probs must not be NaN or +inf (the
 *   reference's heap has no defined order then).  Positions whose log-probs
 *   are non-increasing in rank (top-k output) take a sorted-frontier search;
 *   others a scan of every pushed candidate; both pop the heap's order.
 * ------------------------------------------------------------------- */
int cast_draft_topk(const void *logits, int64_t logits_ld, int32_t rows, int32_t vocab,
                    int32_t dtype, int32_t k, int64_t *top_idx, float *top_lp, int32_t splits,
                    void *workspace, size_t workspace_bytes, cast_stream_t stream);
size_t cast_draft_topk_workspace_size(int32_t rows, int32_t vocab, int32_t dtype, int32_t k,
                                      int32_t splits);
int cast_build_trees(const int64_t *top_idx, const void *top_lp, int32_t lp_dtype, int32_t batch,
                     int32_t L, int32_t k, const int32_t *budget, int64_t *token, int32_t *depth,
                     int32_t *parent, double *score, int32_t *n_nodes, int32_t *status,
                     cast_stream_t stream);


#ifdef __cplusplus
}
#endif

#endif /* CAST_AMD_H */
