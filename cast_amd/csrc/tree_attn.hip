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
// G*P_b query rows.  bf16 with head_dim 64/128 runs on MFMA:
//   S^T = K Q^T with v_mfma_f32_32x32x16_bf16 (keys on the M side, queries on
//   the N side, so each lane ends up owning one query column), then
//   O^T += V^T P^T with the same instruction, P^T taken straight from the
//   S^T accumulator registers (a lane's 16 score values are exactly the 8+8
//   k-slots it must supply), V^T read from a transposed LDS copy.
// K/V tiles of 64 keys are double-buffered through LDS with 16-byte loads;
// the ancestor words are only consulted on the tile(s) holding pack keys.
// The online softmax works in base 2 with a lazy rescale: the running max
// moves only when a tile raises it by more than 2^8, so most tiles skip the
// O rescale.  Long prefixes are split over keys; a combine kernel merges the
// per-split (O, lse) pairs by log-sum-exp.
#include <math.h>

#include "cast_common.hpp"

namespace cast {

constexpr int kNumCU = 256;              // MI355X compute units
constexpr int kNoSplit = 1 << 30;        // chunk value meaning "one split"
constexpr float kLn2 = 0.69314718055994530942f;
constexpr float kLog2e = 1.44269504088896340736f;
constexpr float kRescaleSlack = 8.0f;    // log2 headroom before the O rescale

struct AttnArgs {
    const void *q, *k, *v;
    void *out;
    float *lse;
    const int32_t *cu_q, *cu_kv, *prefix_len, *pack_len;
    const uint64_t *mask;
    int32_t mask_words;
    int32_t batch, total_q, total_kv, Hq, Hkv, G;
    int64_t q_tok, q_head, k_tok, k_head, v_tok, v_head, o_tok, o_head;
    float scale_log2;   // sm_scale * log2(e)
    int32_t chunk;      // keys per split, multiple of 64 (kNoSplit = no split)
    int32_t rows_wg;    // query rows per workgroup
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

__device__ __forceinline__ bool load_seq(const AttnArgs &a, int b, Seq &s) {
    const int S = a.prefix_len[b], P = a.pack_len[b];
    const int q0 = a.cu_q[b], q1 = a.cu_q[b + 1];
    const int kv0 = a.cu_kv[b], kv1 = a.cu_kv[b + 1];
    if (S < 0 || q0 < 0 || kv0 < 0 || q1 > a.total_q || kv1 > a.total_kv || q1 - q0 != P ||
        kv1 - kv0 != S + P) {
        if (threadIdx.x == 0) raise_flag(a.status, CAST_FLAG_BAD_OFFSETS);
        return false;
    }
    if (P < 0 || P > 64 * a.mask_words) {
        if (threadIdx.x == 0) raise_flag(a.status, CAST_FLAG_BAD_PACK);
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

// Total work items and, for item w, the request and in-request index.
// Items are ordered (b, h, split, row block) with the row block fastest.
__device__ bool find_item(const AttnArgs &a, int w, Seq &s, int &local, int &total) {
    total = 0;
    bool found = false;
    int64_t part = 0;
    for (int b = 0; b < a.batch; ++b) {
        Seq t;
        if (!load_seq(a, b, t)) continue;
        const int n = a.Hkv * t.ns * t.rb;
        if (!found && w >= total && w < total + n) {
            s = t;
            s.part_off = part;
            local = w - total;
            found = true;
        }
        total += n;
        if (t.ns > 1) part += (int64_t)t.ns * t.P;
    }
    return found;
}

__device__ __forceinline__ bool pack_bit(int j, uint64_t w0, uint64_t w1) {
    const uint64_t w = j < 64 ? w0 : w1;
    return (w >> (j & 63)) & 1ull;
}

// --------------------------------------------------------------------------
// MFMA kernel: bf16, head_dim D in {64, 128}, WAVES waves x 64 query rows.
// --------------------------------------------------------------------------
template <int D, int WAVES>
__global__ __launch_bounds__(WAVES * 64, 1) void tree_attn_mfma_kernel(AttnArgs a) {
    constexpr int NT = WAVES * 64;
    constexpr int BN = 32;                 // keys per tile (one 32-row MFMA block)
    constexpr int KPAD = D + 8;            // K row stride in LDS (elements)
    constexpr int VPAD = BN + 4;           // V^T row stride in LDS (elements)
    constexpr int DSTEPS = D / 16;         // MFMA k-steps over the head dim
    constexpr int DB = D / 32;             // 32-row blocks of O^T
    constexpr int KCH = BN * D / 8;        // 16-byte K chunks per tile
    constexpr int K_PER_T = (KCH + NT - 1) / NT;
    constexpr int VUNITS = (BN / 4) * (D / 8);   // (4 keys x 8 d) V units per tile
    constexpr int V_PER_T = (VUNITS + NT - 1) / NT;
    // With four waves the next tile is prefetched into registers during the
    // MFMA work; narrower workgroups (small packs) load synchronously and rely
    // on other resident workgroups to hide the latency.
    constexpr bool PREFETCH = WAVES == 4;

    __shared__ __attribute__((aligned(16))) uint16_t Ks[2][BN * KPAD];
    __shared__ __attribute__((aligned(16))) uint16_t Vt[2][D * VPAD];

    // ---- which unit is this workgroup?  Work items are renumbered so that
    // consecutive items (the row blocks of one key split) run on one XCD
    // (workgroups are dealt to the 8 XCDs round-robin) and share its L2.
    Seq sq;
    int local, total;
    {
        Seq dummy;
        int l0;
        find_item(a, -1, dummy, l0, total);
        const int n8 = (total + 7) & ~7;
        const int x = blockIdx.x;
        if (x >= n8) return;
        const int w = (x & 7) * (n8 >> 3) + (x >> 3);
        if (w >= total) return;
        int t2;
        if (!find_item(a, w, sq, local, t2)) return;
    }
    const int rb = local % sq.rb;
    const int split = (local / sq.rb) % sq.ns;
    const int h = local / (sq.rb * sq.ns);
    const int k_begin = split * sq.split_len;
    const int k_end = min(sq.T, k_begin + sq.split_len);

    const int tid = threadIdx.x;
    const int wave = tid >> 6;
    const int lane = tid & 63;
    const int g = lane >> 5;
    const int l32 = lane & 31;
    const int rows = sq.P * a.G;
    const int row_base = rb * (WAVES * 64) + wave * 64;
    const bool active = row_base < rows;

    const uint16_t *qp = static_cast<const uint16_t *>(a.q);
    const uint16_t *kp = static_cast<const uint16_t *>(a.k);
    const uint16_t *vp = static_cast<const uint16_t *>(a.v);

    // ---- Q^T operands (B side): lane holds query l32 of each 32-row block,
    // head-dim slice [ds*16 + g*8, +8)
    bf16x8 qreg[2][DSTEPS];
    uint64_t mw0[2], mw1[2];
    int qtok[2], qhead[2];
    bool qvalid[2];
#pragma unroll
    for (int qb = 0; qb < 2; ++qb) {
        const int r = row_base + qb * 32 + l32;
        qvalid[qb] = r < rows;
        const int i = qvalid[qb] ? r / a.G : 0;
        qtok[qb] = sq.q0 + i;
        qhead[qb] = h * a.G + (qvalid[qb] ? r % a.G : 0);
        const uint16_t *src = qp + (int64_t)qtok[qb] * a.q_tok + (int64_t)qhead[qb] * a.q_head + g * 8;
#pragma unroll
        for (int ds = 0; ds < DSTEPS; ++ds) {
            if (qvalid[qb])
                qreg[qb][ds] = *reinterpret_cast<const bf16x8 *>(src + ds * 16);
            else
                qreg[qb][ds] = bf16x8{};
        }
        mw0[qb] = 0;
        mw1[qb] = 0;
        if (qvalid[qb] && k_end > sq.S) {
            const uint64_t *mp = a.mask + (int64_t)qtok[qb] * a.mask_words;
            mw0[qb] = mp[0];
            if (a.mask_words > 1) mw1[qb] = mp[1];
        }
    }

    floatx16 o[2][DB];
#pragma unroll
    for (int qb = 0; qb < 2; ++qb)
#pragma unroll
        for (int db = 0; db < DB; ++db) o[qb][db] = floatx16{};
    float m[2] = {-INFINITY, -INFINITY};
    float lsum[2] = {0.f, 0.f};

    const int64_t kbase = (int64_t)sq.kv0 * a.k_tok + (int64_t)h * a.k_head;
    const int64_t vbase = (int64_t)sq.kv0 * a.v_tok + (int64_t)h * a.v_head;

    // ---- global -> register staging of one tile
    u32x4 kst[K_PER_T];
    u32x4 vst[V_PER_T][4];
    auto fetch = [&](int t0) {
#pragma unroll
        for (int it = 0; it < K_PER_T; ++it) {
            const int c = tid + it * NT;
            if (c >= KCH) break;
            const int key = c / (D / 8), dch = c % (D / 8);
            const int kk = t0 + key;
            if (kk < k_end)
                kst[it] = *reinterpret_cast<const u32x4 *>(kp + kbase + (int64_t)kk * a.k_tok + dch * 8);
            else
                kst[it] = u32x4{0, 0, 0, 0};
        }
#pragma unroll
        for (int it = 0; it < V_PER_T; ++it) {
            const int u = tid + it * NT;
            if (u >= VUNITS) break;
            const int dch = u % (D / 8), kq = u / (D / 8);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int kk = t0 + kq * 4 + j;
                if (kk < k_end)
                    vst[it][j] = *reinterpret_cast<const u32x4 *>(vp + vbase + (int64_t)kk * a.v_tok + dch * 8);
                else
                    vst[it][j] = u32x4{0, 0, 0, 0};
            }
        }
    };
    // ---- register -> LDS (K as is, V transposed to [d][key])
    auto publish = [&](int buf) {
#pragma unroll
        for (int it = 0; it < K_PER_T; ++it) {
            const int c = tid + it * NT;
            if (c >= KCH) break;
            const int key = c / (D / 8), dch = c % (D / 8);
            *reinterpret_cast<u32x4 *>(&Ks[buf][key * KPAD + dch * 8]) = kst[it];
        }
#pragma unroll
        for (int it = 0; it < V_PER_T; ++it) {
            const int u = tid + it * NT;
            if (u >= VUNITS) break;
            const int dch = u % (D / 8), kq = u / (D / 8);
            // vst[it][j] holds d = dch*8 .. +7 of key kq*4+j as 4 dwords of bf16
            // pairs; row d of the transpose is (key0, key1, key2, key3) at d.
#pragma unroll
            for (int dw = 0; dw < 4; ++dw) {
                const uint32_t a0 = vst[it][0][dw], a1 = vst[it][1][dw];
                const uint32_t a2 = vst[it][2][dw], a3 = vst[it][3][dw];
                // low halves: d = dch*8 + 2*dw, high halves: d + 1
                const u32x2 lo = {__builtin_amdgcn_perm(a1, a0, 0x05040100u),
                                  __builtin_amdgcn_perm(a3, a2, 0x05040100u)};
                const u32x2 hi = {__builtin_amdgcn_perm(a1, a0, 0x07060302u),
                                  __builtin_amdgcn_perm(a3, a2, 0x07060302u)};
                const int d = dch * 8 + 2 * dw;
                *reinterpret_cast<u32x2 *>(&Vt[buf][d * VPAD + kq * 4]) = lo;
                *reinterpret_cast<u32x2 *>(&Vt[buf][(d + 1) * VPAD + kq * 4]) = hi;
            }
        }
    };

    const int ntiles = (k_end - k_begin + BN - 1) / BN;
    if (PREFETCH && ntiles > 0) fetch(k_begin);
    for (int t = 0; t < ntiles; ++t) {
        const int buf = t & 1;
        const int t0 = k_begin + t * BN;
        if (!PREFETCH) fetch(t0);
        publish(buf);
        __syncthreads();
        if (PREFETCH && t + 1 < ntiles) fetch(t0 + BN);
        if (!active) continue;

        // ---- S^T = K Q^T : 32 keys x (2 blocks of 32 queries)
        floatx16 s[2] = {floatx16{}, floatx16{}};
#pragma unroll
        for (int ds = 0; ds < DSTEPS; ++ds) {
            const bf16x8 ka = *reinterpret_cast<const bf16x8 *>(&Ks[buf][l32 * KPAD + ds * 16 + g * 8]);
#pragma unroll
            for (int qb = 0; qb < 2; ++qb)
                s[qb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ka, qreg[qb][ds], s[qb], 0, 0, 0);
        }

        // ---- visibility: tail of the split and the pack's ancestor words.
        // Accumulator element r of lane (l32, g) is key 8*(r/4) + 4*g + r%4.
        if (t0 + BN > sq.S || t0 + BN > k_end) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int key = t0 + 8 * (r >> 2) + 4 * g + (r & 3);
#pragma unroll
                for (int qb = 0; qb < 2; ++qb) {
                    const bool vis = key < k_end && (key < sq.S || pack_bit(key - sq.S, mw0[qb], mw1[qb]));
                    if (!vis) s[qb][r] = -INFINITY;
                }
            }
        }

        // ---- online softmax (base 2, lazy rescale)
        bool need_any = false;
        float mt[2];
#pragma unroll
        for (int qb = 0; qb < 2; ++qb) {
            float mx = s[qb][0];
#pragma unroll
            for (int r = 1; r < 16; ++r) mx = fmaxf(mx, s[qb][r]);
            mx = fmaxf(mx, partner32(mx));
            mt[qb] = mx * a.scale_log2;
            need_any |= mt[qb] > m[qb] + kRescaleSlack;
        }
        if (__any(need_any)) {
#pragma unroll
            for (int qb = 0; qb < 2; ++qb) {
                const float mn = fmaxf(m[qb], mt[qb]);
                const float alpha = mn == -INFINITY ? 1.f : __builtin_amdgcn_exp2f(m[qb] - mn);
                lsum[qb] *= alpha;
#pragma unroll
                for (int db = 0; db < DB; ++db) o[qb][db] *= alpha;
                m[qb] = mn;
            }
        }
        bf16x8 pb[2][2];   // [qb][half]: P^T operand, k-slots of 16 keys
#pragma unroll
        for (int qb = 0; qb < 2; ++qb) {
            const float msafe = m[qb] == -INFINITY ? 0.f : m[qb];
            float acc = 0.f;
            float p[16];
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                p[r] = __builtin_amdgcn_exp2f(fmaf(s[qb][r], a.scale_log2, -msafe));
                acc += p[r];
            }
#pragma unroll
            for (int half = 0; half < 2; ++half) {
                u32x4 w;
#pragma unroll
                for (int e = 0; e < 4; ++e) w[e] = pack_bf16x2(p[half * 8 + 2 * e], p[half * 8 + 2 * e + 1]);
                pb[qb][half] = __builtin_bit_cast(bf16x8, w);
            }
            lsum[qb] += acc;
        }

        // ---- O^T += V^T P^T over 2 slices of 16 keys.  Slot j of lane group
        // g is key 16*half + 8*(j/4) + 4*g + j%4 on both operands.
#pragma unroll
        for (int half = 0; half < 2; ++half) {
#pragma unroll
            for (int db = 0; db < DB; ++db) {
                const uint16_t *vrow = &Vt[buf][(db * 32 + l32) * VPAD + half * 16 + 4 * g];
                const u32x2 lo = *reinterpret_cast<const u32x2 *>(vrow);
                const u32x2 hi = *reinterpret_cast<const u32x2 *>(vrow + 8);
                const u32x4 va4 = {lo[0], lo[1], hi[0], hi[1]};
                const bf16x8 va = __builtin_bit_cast(bf16x8, va4);
#pragma unroll
                for (int qb = 0; qb < 2; ++qb)
                    o[qb][db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(va, pb[qb][half], o[qb][db], 0, 0, 0);
            }
        }
    }

    if (!active) return;
    // ---- epilogue: normalise, write the output or the split partial.
    // O^T element r of lane (l32, g) in block db is d = 32*db + 8*(r/4) + 4*g + r%4.
#pragma unroll
    for (int qb = 0; qb < 2; ++qb) {
        const float ltot = lsum[qb] + partner32(lsum[qb]);
        const float inv = ltot > 0.f ? 1.f / ltot : 0.f;
        const float lse2 = ltot > 0.f ? (m[qb] == -INFINITY ? 0.f : m[qb]) + log2f(ltot) : -INFINITY;
        if (!qvalid[qb]) continue;
        if (sq.ns == 1) {
            uint16_t *op = static_cast<uint16_t *>(a.out) + (int64_t)qtok[qb] * a.o_tok + (int64_t)qhead[qb] * a.o_head;
#pragma unroll
            for (int db = 0; db < DB; ++db)
#pragma unroll
                for (int r4 = 0; r4 < 4; ++r4) {
                    const int d = db * 32 + 8 * r4 + 4 * g;
                    const u32x2 w = {pack_bf16x2(o[qb][db][4 * r4] * inv, o[qb][db][4 * r4 + 1] * inv),
                                     pack_bf16x2(o[qb][db][4 * r4 + 2] * inv, o[qb][db][4 * r4 + 3] * inv)};
                    *reinterpret_cast<u32x2 *>(op + d) = w;
                }
            if (a.lse && g == 0) a.lse[(int64_t)qtok[qb] * a.Hq + qhead[qb]] = lse2 * kLn2;
        } else {
            const int i = qtok[qb] - sq.q0;
            const int64_t prow = sq.part_off + (int64_t)split * sq.P + i;
            if (prow >= a.part_rows) {
                raise_flag(a.status, CAST_FLAG_BAD_OFFSETS);
                continue;
            }
            float *pp = a.part_o + (prow * a.Hq + qhead[qb]) * D;
#pragma unroll
            for (int db = 0; db < DB; ++db)
#pragma unroll
                for (int r4 = 0; r4 < 4; ++r4) {
                    const int d = db * 32 + 8 * r4 + 4 * g;
                    const floatx4 w = {o[qb][db][4 * r4] * inv, o[qb][db][4 * r4 + 1] * inv,
                                       o[qb][db][4 * r4 + 2] * inv, o[qb][db][4 * r4 + 3] * inv};
                    *reinterpret_cast<floatx4 *>(pp + d) = w;
                }
            if (g == 0) a.part_lse[prow * a.Hq + qhead[qb]] = lse2;
        }
    }
}

// --------------------------------------------------------------------------
// Split-K combine: one workgroup per packed token, all query heads.
// --------------------------------------------------------------------------
template <typename OutT, int D>
__global__ __launch_bounds__(256) void tree_attn_combine_kernel(AttnArgs a) {
    const int tok = blockIdx.x;
    Seq sq;
    bool found = false;
    int64_t part = 0;
    for (int b = 0; b < a.batch && !found; ++b) {
        Seq t;
        if (!load_seq(a, b, t)) continue;
        if (tok >= t.q0 && tok < t.q0 + t.P) {
            sq = t;
            sq.part_off = part;
            found = true;
        }
        if (t.ns > 1) part += (int64_t)t.ns * t.P;
    }
    if (!found || sq.ns <= 1) return;
    const int i = tok - sq.q0;
    if (sq.part_off + (int64_t)sq.ns * sq.P > a.part_rows) return;
    constexpr int C = D / 4;
    for (int c = threadIdx.x; c < a.Hq * C; c += blockDim.x) {
        const int hq = c / C, d4 = c % C;
        float M = -INFINITY;
        for (int s = 0; s < sq.ns; ++s)
            M = fmaxf(M, a.part_lse[(sq.part_off + (int64_t)s * sq.P + i) * a.Hq + hq]);
        floatx4 acc = {0.f, 0.f, 0.f, 0.f};
        float L = 0.f;
        if (M != -INFINITY) {
            for (int s = 0; s < sq.ns; ++s) {
                const int64_t prow = sq.part_off + (int64_t)s * sq.P + i;
                const float w = exp2f(a.part_lse[prow * a.Hq + hq] - M);
                L += w;
                const floatx4 x = *reinterpret_cast<const floatx4 *>(a.part_o + (prow * a.Hq + hq) * D + d4 * 4);
                acc += w * x;
            }
            acc *= 1.f / L;
        }
        OutT *op = static_cast<OutT *>(a.out) + (int64_t)tok * a.o_tok + (int64_t)hq * a.o_head + d4 * 4;
        if constexpr (sizeof(OutT) == 2) {
            const u32x2 w = {pack_bf16x2(acc[0], acc[1]), pack_bf16x2(acc[2], acc[3])};
            *reinterpret_cast<u32x2 *>(op) = w;
        } else {
            *reinterpret_cast<floatx4 *>(op) = acc;
        }
        if (a.lse && d4 == 0) a.lse[(int64_t)tok * a.Hq + hq] = M == -INFINITY ? -INFINITY : (M + log2f(L)) * kLn2;
    }
}

// --------------------------------------------------------------------------
// Generic kernel: fp32 or bf16 inputs, any head_dim <= 128 (multiple of 8),
// scalar FMA.  One workgroup = 16 query rows of one (request, KV head).
// --------------------------------------------------------------------------
template <typename T>
__device__ __forceinline__ float load_elem(const T *p);
template <>
__device__ __forceinline__ float load_elem<float>(const float *p) { return *p; }
template <>
__device__ __forceinline__ float load_elem<uint16_t>(const uint16_t *p) { return bf16_to_float(*p); }

template <typename T>
__global__ __launch_bounds__(256) void tree_attn_generic_kernel(AttnArgs a, int D) {
    constexpr int R = 16, BK = 32, DMAX = 128;
    __shared__ float Qs[R][DMAX];
    __shared__ float Ks[BK][DMAX + 1];
    __shared__ float Vs[BK][DMAX];
    __shared__ float Ps[R][BK];

    // items: (b, h, 16-row block); rows_wg == 16 for this kernel
    Seq sq;
    int local, total;
    if (!find_item(a, blockIdx.x, sq, local, total)) return;
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
    const T *kp = static_cast<const T *>(a.k);
    const T *vp = static_cast<const T *>(a.v);
    for (int d = sub; d < D; d += 16)
        Qs[row][d] = valid ? load_elem(qp + (int64_t)tok * a.q_tok + (int64_t)hq * a.q_head + d) : 0.f;
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
            Ks[key][d] = in ? load_elem(kp + (int64_t)(sq.kv0 + kk) * a.k_tok + (int64_t)h * a.k_head + d) : 0.f;
            Vs[key][d] = in ? load_elem(vp + (int64_t)(sq.kv0 + kk) * a.v_tok + (int64_t)h * a.v_head + d) : 0.f;
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
            op[d] = (uint16_t)(pack_bf16x2(x, 0.f) & 0xffffu);
        else
            op[d] = x;
    }
    if (a.lse && sub == 0)
        a.lse[(int64_t)tok * a.Hq + hq] = l > 0.f ? ((m == -INFINITY ? 0.f : m) + log2f(l)) * kLn2 : -INFINITY;
}

// --------------------------------------------------------------------------
// Host side
// --------------------------------------------------------------------------
static bool mfma_path(int32_t dtype, int32_t D) { return dtype == CAST_BF16 && (D == 64 || D == 128); }

static int waves_for(int32_t total_q, int32_t G) {
    const int pmax = total_q < kMaxPack ? total_q : kMaxPack;
    const int rows = pmax * G;
    return rows <= 64 ? 1 : rows <= 128 ? 2 : 4;
}

static int32_t resolve_chunk(int32_t batch, int32_t total_q, int32_t total_kv, int32_t Hq, int32_t Hkv,
                             int32_t D, int32_t dtype, int32_t kv_split) {
    if (!mfma_path(dtype, D) || kv_split < 0 || batch <= 0) return kNoSplit;
    if (kv_split > 0) return ((kv_split + 63) / 64) * 64;
    const int G = Hq / Hkv;
    const int rows_wg = waves_for(total_q, G) * 64;
    const int64_t p_avg = (total_q + batch - 1) / batch;
    const int64_t p_est = p_avg < kMaxPack ? p_avg : kMaxPack;
    const int64_t rb = (p_est * G + rows_wg - 1) / rows_wg;
    const int64_t units = (int64_t)Hkv * batch * (rb > 0 ? rb : 1);
    const int64_t t_avg = (total_kv + batch - 1) / batch;
    if (units >= kNumCU) return kNoSplit;
    int64_t chunk = (t_avg * units + kNumCU - 1) / kNumCU;
    chunk = ((chunk + 63) / 64) * 64;
    if (chunk < 512) chunk = 512;
    if (chunk >= t_avg) return kNoSplit;
    return (int32_t)chunk;
}

static int64_t part_rows_bound(int32_t total_q, int32_t total_kv, int32_t chunk) {
    const int64_t pmax = total_q < kMaxPack ? total_q : kMaxPack;
    return (pmax * (int64_t)total_kv + chunk - 1) / chunk + total_q;
}

static size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

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
    if (chunk == kNoSplit) return 0;
    const int64_t rows = part_rows_bound(total_q, total_kv, chunk);
    return align256((size_t)rows * num_q_heads * head_dim * sizeof(float)) +
           align256((size_t)rows * num_q_heads * sizeof(float));
}

enum { kStageAttn = 1, kStageCombine = 2 };

static int tree_attn_run(const void *q, const void *k, const void *v, void *out, float *lse, const int32_t *cu_q,
                         const int32_t *cu_kv, const int32_t *prefix_len, const int32_t *pack_len,
                         const uint64_t *mask, int32_t mask_words, int32_t batch, int32_t total_q, int32_t total_kv,
                         int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim, int64_t q_tok, int64_t q_head,
                         int64_t k_tok, int64_t k_head, int64_t v_tok, int64_t v_head, int64_t o_tok,
                         int64_t o_head, int32_t dtype, float sm_scale, int32_t kv_split, void *workspace,
                         size_t workspace_bytes, int32_t *status, cast_stream_t stream, int stages) {
    if (batch < 0 || total_q < 0 || total_kv < 0 || head_dim <= 0) return CAST_ERR_SHAPE;
    if (num_q_heads <= 0 || num_kv_heads <= 0 || num_q_heads % num_kv_heads) return CAST_ERR_HEAD_RATIO;
    if (dtype != CAST_BF16 && dtype != CAST_FP32) return CAST_ERR_DTYPE;
    if (mask_words != 1 && mask_words != 2) return CAST_ERR_SHAPE;
    if (!(sm_scale > 0.f) || !isfinite(sm_scale)) return CAST_ERR_SCALE;
    if (batch == 0 || total_q == 0) return CAST_OK;
    if (!q || !k || !v || !out || !cu_q || !cu_kv || !prefix_len || !pack_len || !mask)
        return CAST_ERR_NULL_POINTER;
    const bool mfma = mfma_path(dtype, head_dim);
    if (!mfma && (head_dim > 128 || head_dim % 8)) return CAST_ERR_HEAD_DIM;
    const int64_t esz = dtype == CAST_BF16 ? 2 : 4;
    auto a16 = [](const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
    if (mfma) {
        if (!a16(q) || !a16(k) || !a16(v) || !a16(out)) return CAST_ERR_ALIGNMENT;
        const int64_t strides[8] = {q_tok, q_head, k_tok, k_head, v_tok, v_head, o_tok, o_head};
        for (int64_t s : strides)
            if ((s * esz) % 16) return CAST_ERR_ALIGNMENT;
    }
    (void)esz;
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    AttnArgs a{};
    a.q = q;
    a.k = k;
    a.v = v;
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
    a.q_tok = q_tok;
    a.q_head = q_head;
    a.k_tok = k_tok;
    a.k_head = k_head;
    a.v_tok = v_tok;
    a.v_head = v_head;
    a.o_tok = o_tok;
    a.o_head = o_head;
    a.scale_log2 = sm_scale * kLog2e;
    a.status = status;

    if (!mfma) {
        a.chunk = kNoSplit;
        a.rows_wg = 16;
        const int64_t items = (int64_t)num_kv_heads * (((int64_t)total_q * a.G + 15) / 16 + batch);
        if (!(stages & kStageAttn)) return CAST_OK;
        if (dtype == CAST_FP32)
            tree_attn_generic_kernel<float><<<(unsigned)items, 256, 0, st>>>(a, head_dim);
        else
            tree_attn_generic_kernel<uint16_t><<<(unsigned)items, 256, 0, st>>>(a, head_dim);
        return hipGetLastError() == hipSuccess ? CAST_OK : CAST_ERR_HIP;
    }

    const int waves = waves_for(total_q, a.G);
    a.rows_wg = waves * 64;
    a.chunk = resolve_chunk(batch, total_q, total_kv, num_q_heads, num_kv_heads, head_dim, dtype, kv_split);
    if (a.chunk != kNoSplit) {
        const size_t need = cast_tree_attn_workspace_size(batch, total_q, total_kv, num_q_heads, num_kv_heads,
                                                          head_dim, dtype, kv_split);
        if (!workspace || workspace_bytes < need) return CAST_ERR_WORKSPACE;
        if (reinterpret_cast<uintptr_t>(workspace) & 255) return CAST_ERR_ALIGNMENT;
        a.part_rows = part_rows_bound(total_q, total_kv, a.chunk);
        a.part_o = static_cast<float *>(workspace);
        a.part_lse = reinterpret_cast<float *>(static_cast<char *>(workspace) +
                                               align256((size_t)a.part_rows * num_q_heads * head_dim * sizeof(float)));
    }
    // Grid bound without reading device metadata: every request has at most
    // min(total_q, 128) tokens, so row blocks per (request, head, split) are
    // bounded, and splits sum to at most total_kv / chunk + batch.
    const int64_t pmax = total_q < kMaxPack ? total_q : kMaxPack;
    const int64_t rbmax = (pmax * a.G + a.rows_wg - 1) / a.rows_wg;
    const int64_t nsplit = a.chunk == kNoSplit ? batch : ((int64_t)total_kv + a.chunk - 1) / a.chunk + batch;
    int64_t items = (int64_t)num_kv_heads * rbmax * nsplit;
    items = (items + 7) & ~(int64_t)7;
    const unsigned grid = (unsigned)items;
#define CAST_LAUNCH(DD, W) tree_attn_mfma_kernel<DD, W><<<grid, W * 64, 0, st>>>(a)
    if (!(stages & kStageAttn)) {
    } else if (head_dim == 128) {
        if (waves == 1) CAST_LAUNCH(128, 1);
        else if (waves == 2) CAST_LAUNCH(128, 2);
        else CAST_LAUNCH(128, 4);
    } else {
        if (waves == 1) CAST_LAUNCH(64, 1);
        else if (waves == 2) CAST_LAUNCH(64, 2);
        else CAST_LAUNCH(64, 4);
    }
#undef CAST_LAUNCH
    if (hipGetLastError() != hipSuccess) return CAST_ERR_HIP;
    if (a.chunk != kNoSplit && (stages & kStageCombine)) {
        if (head_dim == 128)
            tree_attn_combine_kernel<uint16_t, 128><<<total_q, 256, 0, st>>>(a);
        else
            tree_attn_combine_kernel<uint16_t, 64><<<total_q, 256, 0, st>>>(a);
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
#define CAST_ATTN_ARGS                                                                                        \
    q, k, v, out, lse, cu_q, cu_kv, prefix_len, pack_len, mask, mask_words, batch, total_q, total_kv,        \
        num_q_heads, num_kv_heads, head_dim, q_tok, q_head, k_tok, k_head, v_tok, v_head, o_tok, o_head,      \
        dtype, sm_scale, kv_split, workspace, workspace_bytes, status, stream

extern "C" int cast_tree_attn_fwd(CAST_ATTN_PARAMS) {
    return tree_attn_run(CAST_ATTN_ARGS, kStageAttn | kStageCombine);
}

extern "C" int cast_tree_attn_partial(CAST_ATTN_PARAMS) { return tree_attn_run(CAST_ATTN_ARGS, kStageAttn); }

extern "C" int cast_tree_attn_combine(CAST_ATTN_PARAMS) { return tree_attn_run(CAST_ATTN_ARGS, kStageCombine); }
