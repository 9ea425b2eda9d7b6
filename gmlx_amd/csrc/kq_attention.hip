// Ragged GQA decode attention (one query token per row) for gfx950.
//
// Semantics: gmlx/qwen35_attn.py:395-493 (ragged_decode_attention) and the
// batched kq.sdpa_decode_gqa(starts=) route (gmlx/gemma4_batched_sdpa.py:
// 210-226): per (row b, q head hq) softmax(scale * q . K^T) . V over the row's
// visible keys, kv head h = hq / (Hq/Hkv), fp32 online softmax.
//
// Two launches (flash-decoding):
//  1. split pass: work unit = one wave = (row b, kv head h, split s of C
//     tokens).  The wave streams its K/V tokens once for all G = Hq/Hkv query
//     heads of the group (GQA sharing), 32 tokens per tile, both products on
//     v_mfma_f32_16x16x32:
//       S^T[tok, head] = K_tile[tok, d] . q^T[d, head]   (A = K rows as loaded)
//       O^T[d, head]  += V^T[d, tok] . P^T[tok, head]    (A = V^T via v_perm)
//     Lane l = 16*g + r: in the score tile it holds head r at tokens
//     {4g..4g+3, 16+4g..16+4g+3}; the P.V B-operand wants exactly those
//     tokens in the same lane, so P never leaves its lane.  K/V tiles are
//     double-buffered in registers: the next tile's loads are in flight
//     while the current one is multiplied.  A row with one split writes its
//     output directly; otherwise the split stores (O unnormalised, m, l).
//  2. merge pass: one workgroup per (row, q head) with nsplit > 1 rescales
//     the splits to the common max and sums them in split order (the
//     two-pass merge of gmlx/qwen35_attn.py:255-282), so the result does not
//     depend on scheduling.
// Cascade mode (kq.sdpa_decode_gqa_cascade, gmlx/cascade_sdpa.py:136-260):
// a prefix shared by all sequences plus a private slab per sequence, and qL
// query tokens per sequence (rows).  A prefix unit puts 16 / G rows' heads
// in the 16 MFMA columns and the row blocks of one prefix split run as the
// waves of one workgroup, so each prefix tile is fetched from HBM about
// once for all rows; private splits are ragged-mode units.  The merge sees
// one split list per row: prefix splits, then private ones.
// No cross-workgroup synchronisation happens inside a launch.
#include <mutex>

#include "kq_common.h"

int device_cus();

namespace {

struct SdpaArgs {
    const uint16_t *q, *k, *v;
    uint16_t *out;
    const int64_t *kv_off, *head_stride;
    const int32_t *row_len;
    // cascade mode (cascade != 0): k/v hold the shared prefix [Hkv][P][D]
    // (head stride shared_head_stride) seen by every row in full; k2/v2 the
    // private slabs [seq][Hkv][S][D], where row r (token i = r % qL of
    // sequence r / qL) sees keys [starts[seq], S - qL + i] after the prefix
    const int32_t *starts;
    const uint16_t *k2, *v2;
    int64_t shared_head_stride, priv_batch_stride, priv_head_stride;
    int32_t cascade, P, S, n1;  // n1 = prefix splits of every row
    int32_t split1;             // tokens per prefix split
    float *part;          // [B][Hkv][max_splits][G][D] O partials
    float *ml;            // [B][Hkv][max_splits][G][2] (m, l)
    int32_t B, Hq, Hkv, G, split, max_splits, max_len;
    int32_t qL;           // query tokens per sequence: row r is token r % qL of sequence r / qL
    // 8-bit affine KV (q8 != 0): k / v (k2 / v2) hold uint8 values, token
    // rows of D bytes, offsets and strides in bytes; ks / kb / vs / vb (and
    // ks2 .. vb2) the 16-bit scales and biases, one per 64 values, at
    // element index (byte offset) / 64
    const uint16_t *ks, *kb, *vs, *vb, *ks2, *kb2, *vs2, *vb2;
    int32_t q8;
    float scale_log2;     // scale * log2(e)
    // padded mode (padded != 0, ragged): k / v are [B, Hkv, max_len, D] at
    // batch / head strides pad_batch_stride / pad_head_stride (elements, or
    // bytes for 8-bit KV) and row b's keys are [starts[b], max_len) (starts
    // NULL: 0), so no per-row tables exist: offsets and lengths are derived
    // here from the device starts
    int32_t padded;
    int64_t pad_batch_stride, pad_head_stride;
};

template <bool BF>
__device__ __forceinline__ floatx4 mfma(const half8_t &a, const half8_t &b, const floatx4 &c) {
    if constexpr (!BF) {
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
    } else {
        typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                       __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
    }
}

template <bool BF>
__device__ __forceinline__ uint32_t pack2(float a, float b) {
    if constexpr (!BF) {
        return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)a) |
               ((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)b) << 16);
    } else {
        return (uint32_t)kq_f32_to_bf16_bits(a) | ((uint32_t)kq_f32_to_bf16_bits(b) << 16);
    }
}

template <bool BF>
__device__ __forceinline__ uint16_t from_f32(float f) {
    if constexpr (!BF) return __builtin_bit_cast(uint16_t, (_Float16)f);
    else return kq_f32_to_bf16_bits(f);
}

// Element index / D of (row, q head) in q and out, laid out [seq][Hq][qL][D]
// (qL = 1: [row][Hq][D]).
__device__ __forceinline__ int64_t qo_index(const SdpaArgs &a, int row, int hq) {
    const int sq = row / a.qL, i = row - sq * a.qL;
    return ((int64_t)sq * a.Hq + hq) * a.qL + i;
}

// First visible key of padded-mode row b, clamped to [0, max_len].
__device__ __forceinline__ int padded_start(const SdpaArgs &a, int b) {
    return a.starts ? min(max(a.starts[b], 0), a.max_len) : 0;
}

// Keys of ragged row b (rows longer than max_len are clamped to it: the
// workspace holds max_len / split splits per (row, head)).
__device__ __forceinline__ int ragged_len(const SdpaArgs &a, int b) {
    if (a.padded) return a.max_len - padded_start(a, b);
    return max(min(a.row_len[b], a.max_len), 0);
}

// Element (byte, 8-bit KV) offset of ragged row b's first visible key of kv head h.
__device__ __forceinline__ int64_t ragged_base(const SdpaArgs &a, int b, int h, int D) {
    if (a.padded)
        return (int64_t)b * a.pad_batch_stride + (int64_t)h * a.pad_head_stride + (int64_t)padded_start(a, b) * D;
    return a.kv_off[b] + (int64_t)h * a.head_stride[b];
}

__device__ __forceinline__ int row_splits(int len, int split) {
    return len <= 0 ? 1 : (len + split - 1) / split;
}

__device__ __forceinline__ int cascade_start(const SdpaArgs &a, int sq) {
    return a.starts ? min(max(a.starts[sq], 0), a.S) : 0;
}

// Private keys of cascade row r: [start, S - qL + i] (end-aligned causal).
__device__ __forceinline__ int cascade_len2(const SdpaArgs &a, int r) {
    const int sq = r / a.qL, i = r - sq * a.qL;
    return max(a.S - a.qL + i + 1 - cascade_start(a, sq), 0);
}

// Splits that map_unit hands out per (row, kv head): ragged mode, the row's
// splits; cascade mode, the private slab's (the prefix units are counted
// apart).  A row with no keys keeps one (empty) split.
__device__ __forceinline__ int row_unit_splits(const SdpaArgs &a, int b) {
    if (!a.cascade) return row_splits(ragged_len(a, b), a.split);
    const int n2 = (cascade_len2(a, b) + a.split - 1) / a.split;
    return a.n1 == 0 ? max(n2, 1) : n2;
}

// All splits of row b (the merge's count).
__device__ __forceinline__ int row_nsplit(const SdpaArgs &a, int b) {
    return a.cascade ? a.n1 + row_unit_splits(a, b) : row_unit_splits(a, b);
}

// Map unit u to (b, h, s).  Each row contributes row_unit_splits splits per
// kv head.  Returns false when u is past the last unit.
__device__ __forceinline__ bool map_unit(const SdpaArgs &a, int u, int &b, int &h, int &s) {
    const int lane = kq_lane();
    int base = 0;
    for (int c0 = 0; c0 < a.B; c0 += 64) {
        const int row = c0 + lane;
        int n = 0;
        if (row < a.B) n = row_unit_splits(a, row);
        const int units = n * a.Hkv;
        int inc = units;  // inclusive scan across the wave
        for (int off = 1; off < 64; off <<= 1) {
            const int t = __shfl_up(inc, off);
            if (lane >= off) inc += t;
        }
        const int excl = inc - units;
        const int total = __shfl(inc, 63);
        if (u < base + total) {
            const uint64_t hit = __ballot(row < a.B && u >= base + excl && u < base + inc);
            const int src = __builtin_ctzll(hit);
            b = c0 + src;
            const int nsplit = __shfl(n, src);
            const int local = u - base - __shfl(excl, src);
            h = local / nsplit;
            s = local - h * nsplit;
            return true;
        }
        base += total;
    }
    return false;
}

// Tokens per K/V tile: 32, or 16 at head dim 512, where a 32-token tile
// alone would take 256 VGPRs.  A 16-token tile fills the first half of the
// P.V MFMA's 32 k values; the other half gets zero P and zero V rows.
template <int D>
struct TileTok {
    static constexpr int TT = D > 256 ? 16 : 32;
    static constexpr int CH = TT / 16;  // 16-token chunks of the score MFMA
    static constexpr int VT = TT / 4;   // V rows per lane
};

// One K/V tile of TT tokens in registers.
template <int D>
struct KVTile {
    static constexpr int NC = D / 32;            // 32-wide d chunks for Q.K
    static constexpr int NG = (D + 127) / 128;   // 128-wide d groups for P.V
    static constexpr int CH = TileTok<D>::CH, VT = TileTok<D>::VT;
    u32x4 k[CH][NC];  // token t0 + 16*ch + r, d = 32c + 8g .. +7
    u32x4 v[NG][VT];  // token t0 + {4g+i | 16+4g+i-4}, d = 128dg + 8r .. +7

    // Tokens past t_end are read from the row's last token (a valid address);
    // their scores are masked to -inf, so they contribute p = 0.
    __device__ __forceinline__ void load(const uint16_t *kp, const uint16_t *vp, int t0, int t_end) {
        const int lane = kq_lane();
        const int r = lane & 15, g = lane >> 4;
#pragma unroll
        for (int ch = 0; ch < CH; ++ch) {
            const int tok = min(t0 + 16 * ch + r, t_end - 1);
#pragma unroll
            for (int c = 0; c < NC; ++c) k[ch][c] = *(const u32x4 *)(kp + (int64_t)tok * D + 32 * c + 8 * g);
        }
#pragma unroll
        for (int dg = 0; dg < NG; ++dg) {
            const int d0 = min(128 * dg + 8 * r, D - 8);
#pragma unroll
            for (int i = 0; i < VT; ++i) {
                const int tok = min(t0 + (i < 4 ? 4 * g + i : 16 + 4 * g + (i - 4)), t_end - 1);
                v[dg][i] = *(const u32x4 *)(vp + (int64_t)tok * D + d0);
            }
        }
    }
    __device__ __forceinline__ half8_t kfrag(int ch, int c) const { return __builtin_bit_cast(half8_t, k[ch][c]); }
    __device__ __forceinline__ void vrows(int dg, u32x4 (&out)[8]) const {
#pragma unroll
        for (int i = 0; i < 8; ++i) out[i] = i < VT ? v[dg][i] : u32x4{0u, 0u, 0u, 0u};
    }
};

// 16-bit float bits (fp16, or bf16 when BF) -> fp32
template <bool BF>
__device__ __forceinline__ float f16bits_to_f32(uint32_t h) {
    if constexpr (BF) return __builtin_bit_cast(float, h << 16);
    else return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
}

// 8 unsigned bytes -> s * q + b with one rounding to the 16-bit type: the
// affine dequantization of an 8-bit group-quantized KV cache, group of 64
// (mx.dequantize).  fp16: a byte becomes 1024 + q exactly (byte under an
// 0x64 high byte), 1024 is subtracted exactly, and a packed fp16 FMA rounds
// q * s + b once; bf16: exact byte -> fp32, fp32 FMA, rounding to bf16.
template <bool BF>
__device__ __forceinline__ u32x4 deq8(u32x2 q, uint32_t sb) {
    if constexpr (!BF) {
        const half2_t s2 = kq_as_h2(__builtin_amdgcn_perm(sb, sb, 0x01000100u));  // (s, s)
        const half2_t b2 = kq_as_h2(__builtin_amdgcn_perm(sb, sb, 0x03020302u));  // (b, b)
        const half2_t k1024 = {(_Float16)1024.f, (_Float16)1024.f};
        auto pair = [&](uint32_t w, uint32_t sel) {
            const half2_t qv = kq_as_h2(kq_bytes_to_h2_biased(w, sel)) - k1024;
            return __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(qv, s2, b2));
        };
        return u32x4{pair(q.x, KQ_SEL_B01), pair(q.x, KQ_SEL_B23), pair(q.y, KQ_SEL_B01), pair(q.y, KQ_SEL_B23)};
    } else {
        const float s = f16bits_to_f32<BF>(sb & 0xFFFFu), b = f16bits_to_f32<BF>(sb >> 16);
        float f[8];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            f[j] = fmaf((float)((q.x >> (8 * j)) & 0xFFu), s, b);
            f[4 + j] = fmaf((float)((q.y >> (8 * j)) & 0xFFu), s, b);
        }
        return u32x4{pack2<BF>(f[0], f[1]), pack2<BF>(f[2], f[3]), pack2<BF>(f[4], f[5]), pack2<BF>(f[6], f[7])};
    }
}

// The head-dim offset of the score MFMA's chunk c in lane group g: 32 c + 8 g,
// or with wide K loads (WK: 8-bit tiles, whose lanes then load 16 contiguous
// values of a token per instruction, two chunks) 64 (c / 2) + 16 g + 8 (c % 2):
// one load instruction covers 64 bytes of each of 16 token rows where
// chunk-sized loads covered 32 (C3 over an 8-bit cache: 0.225-0.229 ->
// 0.212-0.214 ms, measured).  The query fragments follow the same order.  The
// bf16 cascade form with two row blocks keeps chunk-sized loads: its 512
// registers are full, and the wide loads' 128-bit tuples spilled 12 bytes.
template <bool WK>
__device__ __forceinline__ int qk_d(int c, int g) {
    return WK ? 64 * (c >> 1) + 16 * g + 8 * (c & 1) : 32 * c + 8 * g;
}

// One tile of an 8-bit affine-quantized KV cache (uint8 values, token rows of
// D bytes; a 16-bit scale and bias per 64 values of a token), in the lane
// layout of KVTile except for K's head-dim order (qk_d<WK>); values are
// dequantized at their use.  The tile's TT x SG (token, group) scale / bias
// pairs are loaded once, pair p = 64 j + l by lane l into slot j (one 2-byte
// load of each array per lane and slot, where one load per value chunk made
// the 8-bit cache as slow as the 16-bit one), and a fragment takes its pair
// from the owning lane (ds_bpermute).  Tokens past the row's end are clamped
// to its last token, for the values and their pairs alike.
template <int D, bool BF, bool WK>
struct KVTileQ8 {
    static constexpr int NC = D / 32;
    static constexpr int NG = (D + 127) / 128;
    static constexpr int SG = D / 64;  // scale groups per token
    static constexpr int TT = TileTok<D>::TT, CH = TileTok<D>::CH, VT = TileTok<D>::VT;
    static constexpr int NP = TT * SG;         // (token, group) pairs of a tile
    static constexpr int PJ = (NP + 63) / 64;  // pair slots per lane
    u32x2 k[CH][NC];  // token t0 + 16 ch + r, d = qk_d<WK>(c, g) .. +7
    u32x2 v[NG][VT];
    uint32_t ksb[PJ], vsb[PJ];  // pair 64 j + lane: scale | bias << 16
    int tlast;                  // the tile's last valid token (local index)

    __device__ __forceinline__ void load(const uint8_t *kp, const uint8_t *vp, const uint16_t *ks, const uint16_t *kb,
                                         const uint16_t *vs, const uint16_t *vb, int t0, int t_end) {
        const int lane = kq_lane();
        const int r = lane & 15, g = lane >> 4;
        tlast = max(t_end - 1 - t0, 0);  // (a prefetched tile past the end: every token is the last)
#pragma unroll
        for (int ch = 0; ch < CH; ++ch) {
            const int tok = min(t0 + 16 * ch + r, t_end - 1);
            if constexpr (WK) {
#pragma unroll
                for (int i = 0; i < NC / 2; ++i) {
                    const u32x4 w = *(const u32x4 *)(kp + (int64_t)tok * D + 64 * i + 16 * g);
                    k[ch][2 * i] = u32x2{w.x, w.y};
                    k[ch][2 * i + 1] = u32x2{w.z, w.w};
                }
            } else {
#pragma unroll
                for (int c = 0; c < NC; ++c) k[ch][c] = *(const u32x2 *)(kp + (int64_t)tok * D + qk_d<WK>(c, g));
            }
        }
#pragma unroll
        for (int dg = 0; dg < NG; ++dg) {
            const int d0 = min(128 * dg + 8 * r, D - 8);
#pragma unroll
            for (int i = 0; i < VT; ++i) {
                const int tok = min(t0 + (i < 4 ? 4 * g + i : 16 + 4 * g + (i - 4)), t_end - 1);
                v[dg][i] = *(const u32x2 *)(vp + (int64_t)tok * D + d0);
            }
        }
#pragma unroll
        for (int j = 0; j < PJ; ++j) {
            const int p = min(64 * j + lane, NP - 1);  // (lanes past the pairs repeat the last)
            const int tok = min(t0 + p % TT, t_end - 1);
            const int64_t si = (int64_t)tok * SG + p / TT;
            ksb[j] = (uint32_t)ks[si] | ((uint32_t)kb[si] << 16);
            vsb[j] = (uint32_t)vs[si] | ((uint32_t)vb[si] << 16);
        }
    }
    // The pair of local token tl, group grp: lane (grp TT + tl) % 64 of slot
    // (grp TT + tl) / 64; the slot is uniform over the wave at every call.
    __device__ __forceinline__ static uint32_t pair(const uint32_t (&sb)[PJ], int tl, int grp) {
        const int p = grp * TT + tl;
        uint32_t w = sb[0];
#pragma unroll
        for (int j = 1; j < PJ; ++j)
            if (p >= 64 * j) w = sb[j];
        return (uint32_t)__builtin_amdgcn_ds_bpermute((p & 63) * 4, (int)w);
    }
    __device__ __forceinline__ half8_t kfrag(int ch, int c) const {
        const int r = kq_lane() & 15;
        // values qk_d<WK>(c, g) .. +7 lie in group c / 2
        return __builtin_bit_cast(half8_t, deq8<BF>(k[ch][c], pair(ksb, min(16 * ch + r, tlast), c >> 1)));
    }
    __device__ __forceinline__ void vrows(int dg, u32x4 (&out)[8]) const {
        const int lane = kq_lane(), r = lane & 15, g = lane >> 4;
        const int grp = min(128 * dg + 8 * r, D - 8) >> 6;
#pragma unroll
        for (int i = 0; i < 8; ++i)
            out[i] = i < VT ? deq8<BF>(v[dg][i], pair(vsb, min(i < 4 ? 4 * g + i : 16 + 4 * g + (i - 4), tlast), grp))
                            : u32x4{0u, 0u, 0u, 0u};
    }
};

// Query rows in LDS (QL): 16 rows of D 16-bit values, 2 D + 16 bytes apart so
// that a fragment read of 16 rows spans every bank.  The 8-bit kernels at head
// dim 512 keep the query there instead of in 64 VGPRs, and order each MFMA of
// the tile math after the one before (scheduling barriers: left free, the
// scheduler hoisted every dequantized fragment of the tile): with the query
// in registers they spilled 228 (split) and 284 (cascade) bytes per lane, with
// either change alone 0-28.
template <int D>
constexpr uint32_t q_lds_pitch() { return 2 * D + 16; }
template <int D>
constexpr uint32_t q_lds_bytes() { return 16 * q_lds_pitch<D>(); }
template <int D, bool Q8>
constexpr bool q_in_lds() { return Q8 && D > 256; }


template <int D, bool BF, bool QL = false>
struct SplitState {
    static constexpr int NC = D / 32;
    static constexpr int NG = (D + 127) / 128;
    half8_t qf[QL ? 1 : NC];
    uint32_t qrow;  // QL: LDS byte address of the lane's query row (column r)
    floatx4 o[NG][8];
    float m_run;   // running max (log2 domain), same on the 4 lanes of a head
    float l_part;  // this lane's share of the running sum

    __device__ __forceinline__ half8_t qfrag(int c, int g) const {
        if constexpr (QL)
            return __builtin_bit_cast(
                half8_t, *(const __attribute__((address_space(3))) u32x4 *)(uintptr_t)(qrow + 2u * (32 * c + 8 * g)));
        else
            return qf[c];
    }

    template <class Tile>
    __device__ __forceinline__ void tile(const Tile &kv, int t0, int t_end, bool head_ok, float scale_log2) {
        const int lane = kq_lane();
        const int g = lane >> 4;
        // ---- S = K . q^T for tokens t0 + [0, TT)
        constexpr int CH = TileTok<D>::CH;
        floatx4 sc[2];
#pragma unroll
        for (int ch = 0; ch < CH; ++ch) {
            floatx4 acc = {0, 0, 0, 0};
#pragma unroll
            for (int c = 0; c < NC; ++c) {
                acc = mfma<BF>(kv.kfrag(ch, c), qfrag(c, g), acc);
                if constexpr (QL) __builtin_amdgcn_sched_barrier(0);  // (see q_lds_pitch)
            }
            sc[ch] = acc;
        }
        // ---- online softmax over this lane's 8 scores (head r); a
        // 16-token tile has no second chunk (its scores are -inf, p = 0)
        float sv[8];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int ta = t0 + 4 * g + e, tb = t0 + 16 + 4 * g + e;
            sv[e] = (ta < t_end && head_ok) ? sc[0][e] * scale_log2 : -INFINITY;
            sv[4 + e] = (CH == 2 && tb < t_end && head_ok) ? sc[CH - 1][e] * scale_log2 : -INFINITY;
        }
        float tmax = sv[0];
#pragma unroll
        for (int i = 1; i < 8; ++i) tmax = fmaxf(tmax, sv[i]);
        tmax = fmaxf(tmax, __shfl_xor(tmax, 16));
        tmax = fmaxf(tmax, __shfl_xor(tmax, 32));
        const float m_new = fmaxf(m_run, tmax);
        // m_new == -inf only for heads >= G
        const float alpha = (m_new == -INFINITY) ? 1.f : exp2f(m_run - m_new);
        float p[8];
        float psum = 0.f;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            p[i] = (m_new == -INFINITY) ? 0.f : exp2f(sv[i] - m_new);
            psum += p[i];
        }
        l_part = l_part * alpha + psum;
        m_run = m_new;
        const half8_t pf = __builtin_bit_cast(
            half8_t, u32x4{pack2<BF>(p[0], p[1]), pack2<BF>(p[2], p[3]), pack2<BF>(p[4], p[5]),
                           pack2<BF>(p[6], p[7])});
        // ---- O^T += V^T . P^T
#pragma unroll
        for (int dg = 0; dg < NG; ++dg) {
            u32x4 vr[8];
            kv.vrows(dg, vr);
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const uint32_t sel = (j & 1) ? 0x07060302u : 0x05040100u;
                u32x4 f;
                f.x = __builtin_amdgcn_perm(vr[1][j >> 1], vr[0][j >> 1], sel);
                f.y = __builtin_amdgcn_perm(vr[3][j >> 1], vr[2][j >> 1], sel);
                f.z = __builtin_amdgcn_perm(vr[5][j >> 1], vr[4][j >> 1], sel);
                f.w = __builtin_amdgcn_perm(vr[7][j >> 1], vr[6][j >> 1], sel);
                const floatx4 acc = o[dg][j] * alpha;
                o[dg][j] = mfma<BF>(__builtin_bit_cast(half8_t, f), pf, acc);
                if constexpr (QL) __builtin_amdgcn_sched_barrier(0);  // (see q_lds_pitch)
            }
        }
        // o is read by VALU at the next tile (rescale) or after the loop
        kq_mfma_drain();
    }
};

// One split of one KV head over one token range [t_begin, t_end) of the
// buffers kp/vp, for NRB blocks of 16 query columns.  In block j, lane
// l = 16g + r holds query vector r: row row[j], q head h * G + head[j]
// (ok[j] == false: an idle column, its scores are -inf and it stores
// nothing).  Each K/V tile is loaded once into registers and multiplied
// for all NRB * 16 columns.
// Where one unit's K / V rows start: element (fp16 / bf16) or byte (q8)
// offset `base` into k / v, and for q8 the scale / bias arrays of the
// segment (index base / 64).
struct KvSrc {
    const void *k, *v;
    const uint16_t *ks, *kb, *vs, *vb;
};

template <bool Q8>
__device__ __forceinline__ KvSrc kv_src(const void *k, const void *v, const uint16_t *ks, const uint16_t *kb,
                                        const uint16_t *vs, const uint16_t *vb, int64_t base) {
    KvSrc r;
    if constexpr (Q8) {
        r.k = (const uint8_t *)k + base;
        r.v = (const uint8_t *)v + base;
        r.ks = ks + (base >> 6);
        r.kb = kb + (base >> 6);
        r.vs = vs + (base >> 6);
        r.vb = vb + (base >> 6);
    } else {
        r.k = (const uint16_t *)k + base;
        r.v = (const uint16_t *)v + base;
        r.ks = r.kb = r.vs = r.vb = nullptr;
    }
    return r;
}

template <int D, bool BF, bool Q8, bool WK>
struct TileOf {
    using type = KVTile<D>;
};
template <int D, bool BF, bool WK>
struct TileOf<D, BF, true, WK> {
    using type = KVTileQ8<D, BF, WK>;
};

template <class Tile, bool Q8>
__device__ __forceinline__ void load_tile(Tile &t, const KvSrc &src, int t0, int t_end) {
    if constexpr (Q8)
        t.load((const uint8_t *)src.k, (const uint8_t *)src.v, src.ks, src.kb, src.vs, src.vb, t0, t_end);
    else
        t.load((const uint16_t *)src.k, (const uint16_t *)src.v, t0, t_end);
}

// q_lds: the wave's query region (q_lds_bytes<D>() of LDS) when
// q_in_lds<D, Q8>(), else unused.
template <int D, bool BF, int NBUF, int NRB, bool Q8>
__device__ __forceinline__ void split_unit(const SdpaArgs &a, const KvSrc &src, int t_begin,
                                           int t_end, int h, int s, const int (&row)[NRB],
                                           const int (&head)[NRB], const bool (&ok)[NRB], uint32_t q_lds) {
    constexpr int NC = D / 32;
    constexpr int NG = (D + 127) / 128;
    constexpr bool QL = q_in_lds<D, Q8>();
    static_assert(!QL || NRB == 1, "one query block per wave in LDS");
    constexpr bool WK = Q8 && !(BF && NRB > 1);  // wide K loads (qk_d)
    using Tile = typename TileOf<D, BF, Q8, WK>::type;
    const int lane = kq_lane();
    const int g = lane >> 4;

    SplitState<D, BF, QL> st[NRB];
#pragma unroll
    for (int j = 0; j < NRB; ++j) {
        // q^T fragments: lane (column r, group g) holds q[qk_d(c, g) .. +7]
        // (in LDS: at fragment slot 32 c + 8 g of the lane's row)
        const uint16_t *qp = a.q + qo_index(a, row[j], h * a.G + head[j]) * D;
        if constexpr (QL) {
            // each lane writes its own fragments of row r; the wave reads
            // them back after its LDS writes complete
            st[j].qrow = q_lds + (uint32_t)(lane & 15) * q_lds_pitch<D>();
#pragma unroll
            for (int c = 0; c < NC; ++c) {
                const u32x4 v = ok[j] ? *(const u32x4 *)(qp + qk_d<WK>(c, g)) : u32x4{0u, 0u, 0u, 0u};
                *(__attribute__((address_space(3))) u32x4 *)(uintptr_t)(st[j].qrow + 2u * (32 * c + 8 * g)) = v;
            }
            __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
            __builtin_amdgcn_wave_barrier();
        } else {
#pragma unroll
            for (int c = 0; c < NC; ++c)
                st[j].qf[c] = __builtin_bit_cast(half8_t, *(const u32x4 *)(qp + qk_d<WK>(c, g)));
            if (!ok[j]) {
#pragma unroll
                for (int c = 0; c < NC; ++c) st[j].qf[c] = half8_t{0, 0, 0, 0, 0, 0, 0, 0};
            }
        }
#pragma unroll
        for (int dg = 0; dg < NG; ++dg)
#pragma unroll
            for (int i = 0; i < 8; ++i) st[j].o[dg][i] = floatx4{0, 0, 0, 0};
        st[j].m_run = -INFINITY;
        st[j].l_part = 0.f;
    }

    if (t_end > t_begin) {  // wave-uniform
        // Ring of NBUF tiles: tile j + NBUF - 1 is loaded while tile j is
        // multiplied.  Loads are issued unconditionally (tokens past t_end
        // read the last valid token), so the wait counts are static.
        constexpr int TT = TileTok<D>::TT;
        Tile ring[NBUF];
#pragma unroll
        for (int j = 0; j < NBUF - 1; ++j) load_tile<Tile, Q8>(ring[j], src, t_begin + TT * j, t_end);
        for (int t0 = t_begin; t0 < t_end; t0 += TT * NBUF) {
#pragma unroll
            for (int j = 0; j < NBUF; ++j) {
                load_tile<Tile, Q8>(ring[(j + NBUF - 1) % NBUF], src, t0 + TT * (j + NBUF - 1), t_end);
                __builtin_amdgcn_sched_barrier(0);
                if (t0 + TT * j < t_end) {
#pragma unroll
                    for (int k = 0; k < NRB; ++k) st[k].tile(ring[j], t0 + TT * j, t_end, ok[k], a.scale_log2);
                }
            }
        }
    }

#pragma unroll
    for (int j = 0; j < NRB; ++j) {
        // Lane (column r, g) now holds O[d] for d = 128*dg + 32*g + 8*e + i
        // (element e of o[dg][i]); l is split over the 4 lanes of a column.
        float l_tot = st[j].l_part + __shfl_xor(st[j].l_part, 16);
        l_tot += __shfl_xor(l_tot, 32);
        if (!ok[j]) continue;
        const int hq = h * a.G + head[j];
        if (row_nsplit(a, row[j]) == 1) {
            const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
            uint16_t *op = a.out + qo_index(a, row[j], hq) * D;
#pragma unroll
            for (int dg = 0; dg < NG; ++dg)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int d0 = 128 * dg + 32 * g + 8 * e;
                    if (d0 >= D) continue;
                    const floatx4 *o = st[j].o[dg];
                    u32x4 w;
                    w.x = (uint32_t)from_f32<BF>(o[0][e] * inv) | ((uint32_t)from_f32<BF>(o[1][e] * inv) << 16);
                    w.y = (uint32_t)from_f32<BF>(o[2][e] * inv) | ((uint32_t)from_f32<BF>(o[3][e] * inv) << 16);
                    w.z = (uint32_t)from_f32<BF>(o[4][e] * inv) | ((uint32_t)from_f32<BF>(o[5][e] * inv) << 16);
                    w.w = (uint32_t)from_f32<BF>(o[6][e] * inv) | ((uint32_t)from_f32<BF>(o[7][e] * inv) << 16);
                    *(u32x4 *)(op + d0) = w;
                }
            continue;
        }
        // ---- split partial: O (unnormalised), m, l
        const int64_t slot = ((int64_t)row[j] * a.Hkv + h) * a.max_splits + s;
        float *po = a.part + (slot * a.G + head[j]) * D;
#pragma unroll
        for (int dg = 0; dg < NG; ++dg)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int d0 = 128 * dg + 32 * g + 8 * e;
                if (d0 >= D) continue;
                const floatx4 *o = st[j].o[dg];
                float4 *dst = (float4 *)(po + d0);
                dst[0] = make_float4(o[0][e], o[1][e], o[2][e], o[3][e]);
                dst[1] = make_float4(o[4][e], o[5][e], o[6][e], o[7][e]);
            }
        if (g == 0) {
            float *pml = a.ml + (slot * a.G + head[j]) * 2;
            pml[0] = st[j].m_run;
            pml[1] = l_tot;
        }
    }
}

// Ragged mode: unit = one wave = (row b, kv head h, split s), the G q heads
// of the group in columns 0..G-1.
//
// Register budget: left alone the compiler gives a wave ~290 of the SIMD's
// 512 registers (one wave per SIMD).  A 16-bit wave keeps one 16 KB tile in
// flight, enough for the four waves of a CU to stream at HBM rate (C3: 0.71
// of 8 TB/s); an 8-bit tile is half the bytes, and at one wave per SIMD the
// 8-bit C3 batch ran at 4.2-4.3 TB/s.  8-bit kernels at head dim <= 128
// therefore ask for two waves per SIMD (249 VGPRs, no AGPRs, no scratch):
// 0.250 -> 0.224-0.229 ms on C3 (measured).  Three waves spill 416 B per
// lane; two waves with a three-tile ring spill 88 B; the 16-bit kernel at two
// waves measured the same as at one.
template <int D, bool BF, int NBUF, bool Q8>
__global__ __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(Q8 && D <= 128 ? 2 : 1))) void kq_sdpa_split_kernel(
    SdpaArgs a) {
    __shared__ __attribute__((aligned(16))) uint8_t qs[q_in_lds<D, Q8>() ? q_lds_bytes<D>() : 16];
    const uint32_t q_lds = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) void *)qs;
    const int r = kq_lane() & 15;
    for (int u = blockIdx.x;; u += gridDim.x) {
        int b, h, s;
        if (!map_unit(a, u, b, h, s)) return;
        const int len = ragged_len(a, b);
        const int t_begin = s * a.split;
        const int t_end = min(len, t_begin + a.split);
        const int64_t kvbase = ragged_base(a, b, h, D);
        const int rw[1] = {b}, hd[1] = {r < a.G ? r : 0};
        const bool ok[1] = {r < a.G};
        split_unit<D, BF, NBUF, 1, Q8>(a, kv_src<Q8>(a.k, a.v, a.ks, a.kb, a.vs, a.vb, kvbase), t_begin, t_end, h, s,
                                       rw, hd, ok, q_lds);
    }
}

// Cascade mode, W = blockDim / 64 waves per workgroup.
//  - Workgroup units [0, Hkv * n1): the shared prefix, unit = (kv head h,
//    prefix split s).  A row block is R = 16 / G rows whose G heads fill
//    the 16 MFMA columns; a wave takes NRB row blocks and multiplies every
//    prefix tile it loads for all of them, and wave w of the workgroup
//    takes block groups w, w + W, ...  With nrb <= NRB (the usual case: up
//    to 16 rows at G = 4) one wave streams each prefix tile once for all
//    rows.
//  - Later workgroup units: the private slabs, W consecutive units (row,
//    h, split) per workgroup, one per wave, as in ragged mode.  Splits
//    0..n1-1 of a row are the prefix's, n1.. the slab's.
template <int D, bool BF, int NBUF, int NRB, bool Q8>
__global__ __launch_bounds__(256) void kq_sdpa_cascade_kernel(SdpaArgs a) {
    __shared__ __attribute__((aligned(16))) uint8_t qs[q_in_lds<D, Q8>() ? 4 * q_lds_bytes<D>() : 16];
    const int r = kq_lane() & 15;
    const int W = blockDim.x >> 6, w = threadIdx.x >> 6;
    const uint32_t q_lds =
        (uint32_t)(uintptr_t)(__attribute__((address_space(3))) void *)qs + (uint32_t)w * q_lds_bytes<D>();
    const int R = 16 / a.G;
    const int nrb = (a.B + R - 1) / R;
    const int ngrp = (nrb + NRB - 1) / NRB;
    const int64_t U1 = (int64_t)a.Hkv * a.n1;
    const int jr = r / a.G;
    for (int64_t bu = blockIdx.x;; bu += gridDim.x) {
        if (bu < U1) {
            const int s = (int)(bu % a.n1), h = (int)(bu / a.n1);
            const int64_t kvbase = (int64_t)h * a.shared_head_stride;
            const int t_begin = s * a.split1;
            const int t_end = min(a.P, t_begin + a.split1);
            for (int grp = w; grp < ngrp; grp += W) {
                int rw[NRB], hd[NRB];
                bool ok[NRB];
#pragma unroll
                for (int j = 0; j < NRB; ++j) {
                    const int row = (grp * NRB + j) * R + jr;
                    ok[j] = jr < R && row < a.B;
                    rw[j] = ok[j] ? row : 0;
                    hd[j] = ok[j] ? r - jr * a.G : 0;
                }
                split_unit<D, BF, NBUF, NRB, Q8>(a, kv_src<Q8>(a.k, a.v, a.ks, a.kb, a.vs, a.vb, kvbase), t_begin,
                                                 t_end, h, s, rw, hd, ok, q_lds);
            }
        } else {
            const int64_t u2 = (bu - U1) * W + w;
            if (u2 >= (int64_t)1 << 30) return;
            int b, h, s;
            if (!map_unit(a, (int)u2, b, h, s)) return;
            const int sq = b / a.qL;
            const int st = cascade_start(a, sq);
            const int t_begin = s * a.split;
            const int t_end = min(cascade_len2(a, b), t_begin + a.split);
            const int64_t kvbase = (int64_t)sq * a.priv_batch_stride + (int64_t)h * a.priv_head_stride +
                                   (int64_t)st * D;
            const int rw[1] = {b}, hd[1] = {r < a.G ? r : 0};
            const bool ok[1] = {r < a.G};
            split_unit<D, BF, NBUF, 1, Q8>(a, kv_src<Q8>(a.k2, a.v2, a.ks2, a.kb2, a.vs2, a.vb2, kvbase), t_begin,
                                           t_end, h, a.n1 + s, rw, hd, ok, q_lds);
        }
    }
}

// One 256-thread workgroup per (row b, q head hq); rows with a single split
// were finished by the split pass.  Thread t handles the float4 of output
// elements 4q .. 4q + 3 (q = t % (D/4)) for the splits s = p, p + P, ...
// (p = t / (D/4), P = 256 / (D/4) parts), then the P partial sums are added
// in part order through LDS: a fixed summation order, so the merge is
// deterministic.
template <int D, bool BF>
__global__ __launch_bounds__(256) void kq_sdpa_merge_kernel(SdpaArgs a) {
    constexpr int Q = D / 4;    // float4 lanes per split
    constexpr int P = 256 / Q;  // splits summed side by side
    __shared__ float red_m[4];
    __shared__ float4 red_acc[P][Q];
    __shared__ float red_l[P];
    const int b = blockIdx.x / a.Hq;
    const int hq = blockIdx.x - b * a.Hq;
    const int nsplit = row_nsplit(a, b);
    if (nsplit == 1) return;  // uniform over the workgroup
    const int h = hq / a.G, r = hq - h * a.G;
    const int t = threadIdx.x;
    const int q = t % Q, part = t / Q;
    const int64_t slot0 = ((int64_t)b * a.Hkv + h) * a.max_splits;
    const float *ml = a.ml + (slot0 * a.G + r) * 2;                          // split s at ml[s * G * 2]
    const float4 *po = (const float4 *)(a.part + (slot0 * a.G + r) * D) + q;  // split s at po[s * G * Q]
    const int64_t ml_stride = (int64_t)a.G * 2, po_stride = (int64_t)a.G * Q;
    // common max over the splits
    float M = -INFINITY;
    for (int s = t; s < nsplit; s += 256) M = fmaxf(M, ml[s * ml_stride]);
    for (int off = 32; off > 0; off >>= 1) M = fmaxf(M, __shfl_xor(M, off));
    if ((t & 63) == 0) red_m[t >> 6] = M;
    __syncthreads();
    M = fmaxf(fmaxf(red_m[0], red_m[1]), fmaxf(red_m[2], red_m[3]));
    // D = 96: threads 240..255 hold no (q, part) pair
    if (part < P) {
        float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
        float L = 0.f;
#pragma unroll 4
        for (int s = part; s < nsplit; s += P) {
            const float ms = ml[s * ml_stride], ls = ml[s * ml_stride + 1];
            const float f = (ms == -INFINITY) ? 0.f : exp2f(ms - M);
            const float4 o = po[s * po_stride];
            L += ls * f;
            acc.x += f * o.x;
            acc.y += f * o.y;
            acc.z += f * o.z;
            acc.w += f * o.w;
        }
        red_acc[part][q] = acc;
        if (q == 0) red_l[part] = L;
    }
    __syncthreads();
    if (part != 0) return;
    float4 acc = red_acc[0][q];
    float L = red_l[0];
#pragma unroll
    for (int p = 1; p < P; ++p) {
        const float4 o = red_acc[p][q];
        acc.x += o.x;
        acc.y += o.y;
        acc.z += o.z;
        acc.w += o.w;
        L += red_l[p];
    }
    const float inv = L > 0.f ? 1.f / L : 0.f;
    uint2 w;
    w.x = (uint32_t)from_f32<BF>(acc.x * inv) | ((uint32_t)from_f32<BF>(acc.y * inv) << 16);
    w.y = (uint32_t)from_f32<BF>(acc.z * inv) | ((uint32_t)from_f32<BF>(acc.w * inv) << 16);
    *(uint2 *)(a.out + qo_index(a, b, hq) * D + 4 * q) = w;
}

int env_int(const char *name, int dflt) {
    const char *s = getenv(name);
    if (!s || !*s) return dflt;
    char *end = nullptr;
    const long v = strtol(s, &end, 10);
    return (end && *end == 0 && v > 0 && v < (1 << 24)) ? (int)v : dflt;
}

// Tokens per split (a multiple of the 32-token tile): 1024 when the launch's
// unit bound B * Hkv * ceil(max_len / 1024) gives every CU 8 waves, 512
// otherwise (longer splits halve the partials and the merge's work; measured
// on C3: 353 against 372 us); GMLX_KQ_SDPA_SPLIT forces it.  The workspace
// size follows the same rule from the same arguments.
int split_tokens(int B, int Hkv, int max_len) {
    int c = env_int("GMLX_KQ_SDPA_SPLIT", 0);
    if (c == 0) {
        const int64_t units = (int64_t)B * Hkv * (((int64_t)(max_len > 0 ? max_len : 1) + 1023) / 1024);
        c = units >= 8 * (int64_t)device_cus() ? 1024 : 512;
    }
    c = (c + 31) / 32 * 32;
    return c < 32 ? 32 : c;
}

struct WsLayout {
    size_t part_bytes, ml_bytes;
};

WsLayout ws_layout(int B, int Hq, int Hkv, int D, int max_len) {
    const int G = Hq / Hkv;
    const int C = split_tokens(B, Hkv, max_len);
    const int64_t ms = max_len <= 0 ? 1 : (max_len + C - 1) / C;
    WsLayout w;
    w.part_bytes = (((size_t)B * Hkv * ms * G * D * 4) + 255) & ~(size_t)255;
    w.ml_bytes = (size_t)B * Hkv * ms * G * 2 * 4;
    return w;
}

// Row blocks per prefix wave: 2 (GMLX_KQ_CASCADE_NRB=1 selects one).  Four
// spill; D = 256 keeps one, its tile alone being 128 VGPRs.
int cascade_nrb(int D, int nrb) {
    const int cap = D >= 256 ? 1 : env_int("GMLX_KQ_CASCADE_NRB", 2);
    return nrb >= 2 && cap >= 2 ? 2 : 1;
}

template <int D, bool BF, int NBUF, bool Q8>
void launch_n(const SdpaArgs &a, int grid, int block, bool merge, hipStream_t s) {
    if (a.cascade) {
        const int R = 16 / a.G;
        switch (cascade_nrb(D, (a.B + R - 1) / R)) {
        case 2:
            if constexpr (D < 256)
                hipLaunchKernelGGL((kq_sdpa_cascade_kernel<D, BF, NBUF, 2, Q8>), dim3(grid), dim3(block), 0, s, a);
            break;
        default:
            hipLaunchKernelGGL((kq_sdpa_cascade_kernel<D, BF, NBUF, 1, Q8>), dim3(grid), dim3(block), 0, s, a);
            break;
        }
    } else
        hipLaunchKernelGGL((kq_sdpa_split_kernel<D, BF, NBUF, Q8>), dim3(grid), dim3(64), 0, s, a);
    if (merge) hipLaunchKernelGGL((kq_sdpa_merge_kernel<D, BF>), dim3(a.B * a.Hq), dim3(256), 0, s, a);
}

// Tiles in flight per wave: 2 (D = 256 tiles are 128 VGPRs, 96 in 8 bits:
// 1).  Deeper rings put tiles in AGPRs, whose copies wait for the loads:
// measured no faster on the C3 ragged batch and the cascade shapes.  8-bit
// KV needs whole 64-value scale groups per token (D = 64, 128, 256).
template <int D, bool BF>
void launch(const SdpaArgs &a, int grid, int block, bool merge, hipStream_t s) {
    if (a.q8) {
        if constexpr (D % 64 == 0) launch_n<D, BF, D >= 256 ? 1 : 2, true>(a, grid, block, merge, s);
    } else {
        launch_n<D, BF, D >= 256 ? 1 : 2, false>(a, grid, block, merge, s);
    }
}

}  // namespace

extern "C" {

size_t kq_sdpa_workspace_bytes(int32_t B, int32_t Hq, int32_t Hkv, int32_t D, int32_t max_len) {
    if (B <= 0 || Hkv <= 0 || Hq <= 0 || Hq % Hkv || D <= 0) return 0;
    const WsLayout w = ws_layout(B, Hq, Hkv, D, max_len);
    return w.part_bytes + w.ml_bytes;
}

}  // extern "C"

namespace {

// The four scale / bias arrays of an 8-bit KV cache (all NULL: 16-bit KV).
struct Q8Scales {
    const void *ks, *kb, *vs, *vb;
};

int q8_check(const Q8Scales *q8, int D) {
    if (!q8) return KQ_OK;
    if (!q8->ks || !q8->kb || !q8->vs || !q8->vb) return KQ_ERR_NULL_POINTER;
    if (D % 64) return KQ_ERR_BAD_SHAPE;
    if (((uintptr_t)q8->ks | (uintptr_t)q8->kb | (uintptr_t)q8->vs | (uintptr_t)q8->vb) & 1) return KQ_ERR_BAD_ALIGN;
    return KQ_OK;
}

void set_q8(SdpaArgs &a, const Q8Scales *q8, const Q8Scales *q8b) {
    a.q8 = q8 != nullptr;
    a.ks = q8 ? (const uint16_t *)q8->ks : nullptr;
    a.kb = q8 ? (const uint16_t *)q8->kb : nullptr;
    a.vs = q8 ? (const uint16_t *)q8->vs : nullptr;
    a.vb = q8 ? (const uint16_t *)q8->vb : nullptr;
    a.ks2 = q8b ? (const uint16_t *)q8b->ks : nullptr;
    a.kb2 = q8b ? (const uint16_t *)q8b->kb : nullptr;
    a.vs2 = q8b ? (const uint16_t *)q8b->vs : nullptr;
    a.vb2 = q8b ? (const uint16_t *)q8b->vb : nullptr;
}

// Padded layout of kq_sdpa_decode_gqa: strides and device starts instead
// of per-row tables.
struct PaddedKv {
    int64_t batch_stride, head_stride;
    const int32_t *starts;
};

int ragged_impl(const void *q, const void *k, const void *v, const Q8Scales *q8, const int64_t *kv_off,
                const int64_t *head_stride, const int32_t *row_len, const PaddedKv *pad, int32_t B, int32_t Hq,
                int32_t Hkv, int32_t D, int32_t max_len, float scale, int dtype, void *out, void *workspace,
                size_t workspace_bytes, kq_stream_t stream) {
    if (B == 0) return KQ_OK;
    if (!q || !k || !v || !out) return KQ_ERR_NULL_POINTER;
    if (!pad && (!kv_off || !head_stride || !row_len)) return KQ_ERR_NULL_POINTER;
    if (pad) {
        // token rows of D elements (bytes for 8-bit KV), heads and rows apart
        if (pad->head_stride < (int64_t)max_len * D || pad->batch_stride < pad->head_stride * Hkv)
            return KQ_ERR_BAD_SHAPE;
        const int64_t al = q8 ? 63 : 7;
        if ((pad->head_stride & al) || (pad->batch_stride & al)) return KQ_ERR_BAD_ALIGN;
    }
    if (B < 0 || Hq <= 0 || Hkv <= 0 || Hq % Hkv || Hq / Hkv > 16 || max_len < 0) return KQ_ERR_BAD_SHAPE;
    if (D != 64 && D != 96 && D != 128 && D != 256 && D != 512) return KQ_ERR_BAD_SHAPE;
    if ((int64_t)B * Hq > (1 << 30)) return KQ_ERR_BAD_SHAPE;
    if (dtype != KQ_DTYPE_F16 && dtype != KQ_DTYPE_BF16) return KQ_ERR_UNSUPPORTED_DTYPE;
    if (const int rc = q8_check(q8, D)) return rc;
    const uintptr_t kv_align = q8 ? 7 : 15;
    if (((uintptr_t)q & 15) || ((uintptr_t)k & kv_align) || ((uintptr_t)v & kv_align) || ((uintptr_t)out & 15))
        return KQ_ERR_BAD_ALIGN;
    const size_t need = kq_sdpa_workspace_bytes(B, Hq, Hkv, D, max_len);
    if (!workspace || workspace_bytes < need) return KQ_ERR_WORKSPACE_TOO_SMALL;
    const WsLayout w = ws_layout(B, Hq, Hkv, D, max_len);
    SdpaArgs a;
    a.q = (const uint16_t *)q;
    a.k = (const uint16_t *)k;
    a.v = (const uint16_t *)v;
    a.out = (uint16_t *)out;
    a.kv_off = kv_off;
    a.head_stride = head_stride;
    a.row_len = row_len;
    a.starts = pad ? pad->starts : nullptr;
    a.padded = pad ? 1 : 0;
    a.pad_batch_stride = pad ? pad->batch_stride : 0;
    a.pad_head_stride = pad ? pad->head_stride : 0;
    a.k2 = a.v2 = nullptr;
    a.shared_head_stride = a.priv_batch_stride = a.priv_head_stride = 0;
    a.cascade = a.P = a.S = a.n1 = a.split1 = 0;
    a.qL = 1;
    set_q8(a, q8, nullptr);
    a.part = (float *)workspace;
    a.ml = (float *)((char *)workspace + w.part_bytes);
    a.B = B;
    a.Hq = Hq;
    a.Hkv = Hkv;
    a.G = Hq / Hkv;
    a.split = split_tokens(B, Hkv, max_len);
    a.max_splits = max_len <= 0 ? 1 : (max_len + a.split - 1) / a.split;
    a.max_len = max_len;
    a.scale_log2 = scale * 1.4426950408889634f;
    // one wave per unit; the unit count is bounded by B * Hkv * max_splits
    // (rows are shorter on the device side), extra waves exit at once
    const int64_t upper = (int64_t)B * Hkv * a.max_splits;
    const int grid = (int)(upper < (1 << 22) ? upper : (1 << 22));
    const bool merge = a.max_splits > 1;
    hipStream_t s = (hipStream_t)stream;
    const bool bf = dtype == KQ_DTYPE_BF16;
    switch (D) {
    case 64: bf ? launch<64, true>(a, grid, 64, merge, s) : launch<64, false>(a, grid, 64, merge, s); break;
    case 96: bf ? launch<96, true>(a, grid, 64, merge, s) : launch<96, false>(a, grid, 64, merge, s); break;
    case 128: bf ? launch<128, true>(a, grid, 64, merge, s) : launch<128, false>(a, grid, 64, merge, s); break;
    case 256: bf ? launch<256, true>(a, grid, 64, merge, s) : launch<256, false>(a, grid, 64, merge, s); break;
    default: bf ? launch<512, true>(a, grid, 64, merge, s) : launch<512, false>(a, grid, 64, merge, s); break;
    }
    return hipGetLastError() == hipSuccess ? KQ_OK : KQ_ERR_LAUNCH_FAILED;
}

}  // namespace

extern "C" {

int kq_sdpa_decode_ragged(const void *q, const void *k, const void *v, const int64_t *kv_off,
                          const int64_t *head_stride, const int32_t *row_len, int32_t B, int32_t Hq,
                          int32_t Hkv, int32_t D, int32_t max_len, float scale, int dtype, void *out,
                          void *workspace, size_t workspace_bytes, kq_stream_t stream) {
    return ragged_impl(q, k, v, nullptr, kv_off, head_stride, row_len, nullptr, B, Hq, Hkv, D, max_len, scale, dtype,
                       out, workspace, workspace_bytes, stream);
}

int kq_sdpa_decode_gqa(const void *q, const void *k, const void *v, int64_t batch_stride, int64_t head_stride,
                       int32_t L, const int32_t *starts, int32_t B, int32_t Hq, int32_t Hkv, int32_t D, float scale,
                       int dtype, void *out, void *workspace, size_t workspace_bytes, kq_stream_t stream) {
    const PaddedKv pad{batch_stride, head_stride, starts};
    return ragged_impl(q, k, v, nullptr, nullptr, nullptr, nullptr, &pad, B, Hq, Hkv, D, L, scale, dtype, out,
                       workspace, workspace_bytes, stream);
}

int kq_sdpa_decode_gqa_q8(const void *q, const void *k, const void *v, const void *const *kv_scales,
                          int64_t batch_stride, int64_t head_stride, int32_t L, const int32_t *starts, int32_t B,
                          int32_t Hq, int32_t Hkv, int32_t D, float scale, int dtype, void *out, void *workspace,
                          size_t workspace_bytes, kq_stream_t stream) {
    if (!kv_scales) return KQ_ERR_NULL_POINTER;
    const Q8Scales q8{kv_scales[0], kv_scales[1], kv_scales[2], kv_scales[3]};
    const PaddedKv pad{batch_stride, head_stride, starts};
    return ragged_impl(q, k, v, &q8, nullptr, nullptr, nullptr, &pad, B, Hq, Hkv, D, L, scale, dtype, out, workspace,
                       workspace_bytes, stream);
}

int kq_sdpa_decode_ragged_q8(const void *q, const void *k, const void *v, const void *k_scales,
                             const void *k_biases, const void *v_scales, const void *v_biases,
                             const int64_t *kv_off, const int64_t *head_stride, const int32_t *row_len, int32_t B,
                             int32_t Hq, int32_t Hkv, int32_t D, int32_t max_len, float scale, int dtype, void *out,
                             void *workspace, size_t workspace_bytes, kq_stream_t stream) {
    const Q8Scales q8{k_scales, k_biases, v_scales, v_biases};
    return ragged_impl(q, k, v, &q8, kv_off, head_stride, row_len, nullptr, B, Hq, Hkv, D, max_len, scale, dtype, out,
                       workspace, workspace_bytes, stream);
}

// Cascade launch plan.  A wave's tiles form one chain of dependent loads
// (about 1.5 us per 32-token tile when few waves run), so short batches
// want short splits, while every split costs a partial (G * D * 4 bytes
// per row and kv head, written and merged).  Chosen from a sweep of
// B 2..16, qL 1..4, P 4k-32k, private 256-1024 tokens (Hq 32, Hkv 8, D 128):
//   prefix split 512 tokens, 256 when that leaves under 384 prefix waves;
//   private split 512 tokens, 256 when that leaves under 256 private
//   waves, 128 when 256 leaves under 128.
// GMLX_KQ_CASCADE_SPLIT / GMLX_KQ_CASCADE_PSPLIT override the two splits.
struct CascadePlan {
    int split1, split2;  // tokens per prefix / private split
    int per_wave;        // row blocks per prefix wave
    int ngrp;            // prefix waves per (kv head, split)
};

static int env_split(const char *name) {
    const int env = env_int(name, 0);
    return env > 0 ? (env < 32 ? 32 : (env + 31) / 32 * 32) : 0;
}

static CascadePlan cascade_plan(int P, int S, int rows, int Hkv, int G, int D) {
    CascadePlan p;
    const int R = 16 / G;
    const int nrb = (rows + R - 1) / R;
    p.per_wave = cascade_nrb(D, nrb);
    p.ngrp = (nrb + p.per_wave - 1) / p.per_wave;
    const int64_t prefix_waves_512 = (int64_t)Hkv * ((P + 511) / 512) * p.ngrp;
    p.split1 = env_split("GMLX_KQ_CASCADE_SPLIT");
    if (!p.split1) p.split1 = prefix_waves_512 < 384 ? 256 : 512;
    p.split2 = env_split("GMLX_KQ_CASCADE_PSPLIT");
    if (!p.split2) {
        const int64_t per_row = (int64_t)rows * Hkv;
        p.split2 = per_row * ((S + 511) / 512) >= 256 ? 512 : (per_row * ((S + 255) / 256) >= 128 ? 256 : 128);
    }
    return p;
}

// Cascade splits per (row, kv head): the prefix's, then the private slab's.
static int cascade_max_splits(const CascadePlan &p, int P, int S) {
    const int n = (P + p.split1 - 1) / p.split1 + (S + p.split2 - 1) / p.split2;
    return n > 0 ? n : 1;
}

size_t kq_sdpa_cascade_workspace_bytes(int32_t B, int32_t qL, int32_t Hq, int32_t Hkv, int32_t D, int32_t P,
                                       int32_t S) {
    if (B <= 0 || qL <= 0 || Hkv <= 0 || Hq <= 0 || Hq % Hkv || D <= 0 || P < 0 || S < 0) return 0;
    const CascadePlan plan = cascade_plan(P, S, B * qL, Hkv, Hq / Hkv, D);
    const int64_t slots = (int64_t)B * qL * Hkv * cascade_max_splits(plan, P, S) * (Hq / Hkv);
    return (((size_t)slots * D * 4 + 255) & ~(size_t)255) + (size_t)slots * 2 * 4;
}

}  // extern "C"

namespace {

int cascade_impl(const void *q, const void *k_shared, const void *v_shared, const Q8Scales *q8s,
                 int64_t shared_head_stride, int32_t P, const void *k_priv, const void *v_priv, const Q8Scales *q8p,
                 int64_t priv_batch_stride, int64_t priv_head_stride, int32_t S, const int32_t *starts, int32_t B,
                 int32_t qL, int32_t Hq, int32_t Hkv, int32_t D, float scale, int dtype, void *out, void *workspace,
                 size_t workspace_bytes, kq_stream_t stream) {
    if (B == 0) return KQ_OK;
    if (!q || !k_shared || !v_shared || !k_priv || !v_priv || !out) return KQ_ERR_NULL_POINTER;
    if (B < 0 || qL < 1 || qL > 64 || Hq <= 0 || Hkv <= 0 || Hq % Hkv || Hq / Hkv > 16 || P < 0 || S < 0)
        return KQ_ERR_BAD_SHAPE;
    if (D != 64 && D != 96 && D != 128 && D != 256 && D != 512) return KQ_ERR_BAD_SHAPE;
    if ((int64_t)B * qL * Hq > (1 << 24)) return KQ_ERR_BAD_SHAPE;
    if (shared_head_stride < (int64_t)P * D || priv_head_stride < (int64_t)S * D ||
        priv_batch_stride < priv_head_stride * Hkv)
        return KQ_ERR_BAD_SHAPE;
    if (dtype != KQ_DTYPE_F16 && dtype != KQ_DTYPE_BF16) return KQ_ERR_UNSUPPORTED_DTYPE;
    if ((q8s == nullptr) != (q8p == nullptr)) return KQ_ERR_NULL_POINTER;
    if (const int rc = q8_check(q8s, D)) return rc;
    if (const int rc = q8_check(q8p, D)) return rc;
    // 16-bit KV: 16-byte rows of 8 values; 8-bit KV: 8-byte runs, and token
    // rows / strides on whole 64-value scale groups
    const uintptr_t kv_align = q8s ? 7 : 15;
    const int64_t st_align = q8s ? 63 : 7;
    if (((uintptr_t)q & 15) || ((uintptr_t)k_shared & kv_align) || ((uintptr_t)v_shared & kv_align) ||
        ((uintptr_t)k_priv & kv_align) || ((uintptr_t)v_priv & kv_align) || ((uintptr_t)out & 15) ||
        (shared_head_stride & st_align) || (priv_head_stride & st_align) || (priv_batch_stride & st_align))
        return KQ_ERR_BAD_ALIGN;
    const size_t need = kq_sdpa_cascade_workspace_bytes(B, qL, Hq, Hkv, D, P, S);
    if (!workspace || workspace_bytes < need) return KQ_ERR_WORKSPACE_TOO_SMALL;
    const int rows = B * qL;
    SdpaArgs a;
    a.q = (const uint16_t *)q;
    a.k = (const uint16_t *)k_shared;
    a.v = (const uint16_t *)v_shared;
    a.out = (uint16_t *)out;
    a.kv_off = a.head_stride = nullptr;
    a.row_len = nullptr;
    a.starts = starts;
    a.k2 = (const uint16_t *)k_priv;
    a.v2 = (const uint16_t *)v_priv;
    a.shared_head_stride = shared_head_stride;
    a.priv_batch_stride = priv_batch_stride;
    a.priv_head_stride = priv_head_stride;
    a.cascade = 1;
    a.padded = 0;
    a.pad_batch_stride = a.pad_head_stride = 0;
    set_q8(a, q8s, q8p);
    a.P = P;
    a.S = S;
    a.qL = qL;
    a.B = rows;
    a.Hq = Hq;
    a.Hkv = Hkv;
    a.G = Hq / Hkv;
    const CascadePlan plan = cascade_plan(P, S, rows, Hkv, a.G, D);
    a.split = plan.split2;
    a.split1 = plan.split1;
    a.n1 = (P + a.split1 - 1) / a.split1;
    a.max_splits = cascade_max_splits(plan, P, S);
    a.max_len = P > S ? P : S;
    a.part = (float *)workspace;
    const int64_t slots = (int64_t)rows * Hkv * a.max_splits * a.G;
    a.ml = (float *)((char *)workspace + (((size_t)slots * D * 4 + 255) & ~(size_t)255));
    a.scale_log2 = scale * 1.4426950408889634f;
    // W waves per workgroup: up to 4 row blocks of a prefix split share a
    // workgroup.  Grid: the prefix's Hkv * n1 units, then the private
    // units W at a time (an upper bound; extra waves exit at once).
    const int W = plan.ngrp < 4 ? plan.ngrp : 4;
    const int64_t priv = (int64_t)rows * Hkv * (a.max_splits - a.n1 > 0 ? a.max_splits - a.n1 : 1);
    const int64_t upper = (int64_t)Hkv * a.n1 + (priv + W - 1) / W;
    const int grid = (int)(upper < (1 << 22) ? upper : (1 << 22));
    const int block = 64 * W;
    const bool merge = a.max_splits > 1;
    const bool bf = dtype == KQ_DTYPE_BF16;
    hipStream_t s = (hipStream_t)stream;
    switch (D) {
    case 64: bf ? launch<64, true>(a, grid, block, merge, s) : launch<64, false>(a, grid, block, merge, s); break;
    case 96: bf ? launch<96, true>(a, grid, block, merge, s) : launch<96, false>(a, grid, block, merge, s); break;
    case 128:
        bf ? launch<128, true>(a, grid, block, merge, s) : launch<128, false>(a, grid, block, merge, s);
        break;
    case 256:
        bf ? launch<256, true>(a, grid, block, merge, s) : launch<256, false>(a, grid, block, merge, s);
        break;
    default:
        bf ? launch<512, true>(a, grid, block, merge, s) : launch<512, false>(a, grid, block, merge, s);
        break;
    }
    return hipGetLastError() == hipSuccess ? KQ_OK : KQ_ERR_LAUNCH_FAILED;
}

}  // namespace

extern "C" {

int kq_sdpa_decode_gqa_cascade(const void *q, const void *k_shared, const void *v_shared,
                               int64_t shared_head_stride, int32_t P, const void *k_priv, const void *v_priv,
                               int64_t priv_batch_stride, int64_t priv_head_stride, int32_t S,
                               const int32_t *starts, int32_t B, int32_t qL, int32_t Hq, int32_t Hkv, int32_t D,
                               float scale, int dtype, void *out, void *workspace, size_t workspace_bytes,
                               kq_stream_t stream) {
    return cascade_impl(q, k_shared, v_shared, nullptr, shared_head_stride, P, k_priv, v_priv, nullptr,
                        priv_batch_stride, priv_head_stride, S, starts, B, qL, Hq, Hkv, D, scale, dtype, out,
                        workspace, workspace_bytes, stream);
}

int kq_sdpa_decode_gqa_cascade_q8(const void *q, const void *k_shared, const void *v_shared,
                                  const void *const *shared_scales, int64_t shared_head_stride, int32_t P,
                                  const void *k_priv, const void *v_priv, const void *const *priv_scales,
                                  int64_t priv_batch_stride, int64_t priv_head_stride, int32_t S,
                                  const int32_t *starts, int32_t B, int32_t qL, int32_t Hq, int32_t Hkv, int32_t D,
                                  float scale, int dtype, void *out, void *workspace, size_t workspace_bytes,
                                  kq_stream_t stream) {
    if (!shared_scales || !priv_scales) return KQ_ERR_NULL_POINTER;
    const Q8Scales s8{shared_scales[0], shared_scales[1], shared_scales[2], shared_scales[3]};
    const Q8Scales p8{priv_scales[0], priv_scales[1], priv_scales[2], priv_scales[3]};
    return cascade_impl(q, k_shared, v_shared, &s8, shared_head_stride, P, k_priv, v_priv, &p8, priv_batch_stride,
                        priv_head_stride, S, starts, B, qL, Hq, Hkv, D, scale, dtype, out, workspace,
                        workspace_bytes, stream);
}

}  // extern "C"

// ---- allocation-free decode attention ------------------------------------
// The split partials (fp32 O, m, l) of kq_sdpa_decode_gqa_noalloc live in
// this file-scope device array: each GPU the library runs on holds its own
// copy, from the code object's load until the process ends.  On the host the
// array's name is a stand-in, not a device address: host code uses only the
// per-device address hipGetSymbolAddress returns (taken once per device, with
// that device current, on the entry point's first call there).  The partials
// are written before they are read, so nothing needs clearing between calls;
// calls that overlap on one GPU (two streams, or two threads) share the array
// and race.
static __device__ __align__(256) uint8_t scratch[KQ_SDPA_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int kScratchDevices = 64;
std::mutex g_scratch_mu;
void *g_scratch_ptr[kScratchDevices];

int scratch_ptr(void **out) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return KQ_ERR_LAUNCH_FAILED;
    if (dev < 0 || dev >= kScratchDevices) return KQ_ERR_BAD_ARGUMENT;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void *p = nullptr;
        if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) return KQ_ERR_LAUNCH_FAILED;
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return KQ_OK;
}

}  // namespace

extern "C" int kq_sdpa_decode_gqa_noalloc(const void *q, const void *k, const void *v, int64_t batch_stride,
                                          int64_t head_stride, int32_t L, const int32_t *starts, int32_t B,
                                          int32_t Hq, int32_t Hkv, int32_t D, float scale, int dtype, void *out,
                                          kq_stream_t stream) {
    if (B == 0) return KQ_OK;
    if (B < 0 || Hq <= 0 || Hkv <= 0 || Hq % Hkv || D <= 0 || L < 0) return KQ_ERR_BAD_SHAPE;
    const size_t need = kq_sdpa_workspace_bytes(B, Hq, Hkv, D, L);
    if (need > KQ_SDPA_NOALLOC_SCRATCH_BYTES) return KQ_ERR_WORKSPACE_TOO_SMALL;
    void *ws = nullptr;
    if (const int rc = scratch_ptr(&ws)) return rc;
    const PaddedKv pad{batch_stride, head_stride, starts};
    return ragged_impl(q, k, v, nullptr, nullptr, nullptr, nullptr, &pad, B, Hq, Hkv, D, L, scale, dtype, out, ws,
                       KQ_SDPA_NOALLOC_SCRATCH_BYTES, stream);
}
