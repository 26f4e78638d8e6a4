// Split-K flash-decode over the paged K4V4 codebook cache (gfx950).
//
// Reference contract: cda_decode_full_hmma_v3 as bound by
// cda/kernels_cuda/wrappers.py:79-124; math of cda/algorithm/attention.py:
// 426-482 (attention_compressed), split-K partials and merge of :190-272.
//
// Default form, one launch (decode_stream_kernel<..., FUSED = true>): where
// the page-streaming kernel applies (8 KV heads, 144- or 80-byte slots, one
// codebook pointer, the library's split plan), one workgroup per (sequence,
// context split, KV head) rotates that head's GQA group of q, streams the
// head's pages on eight waves over consecutive token ranges, merges the
// waves' partials in LDS and, when one split covers the sequence, applies
// R^T and writes out; with several splits the combine launch follows.
//
// Otherwise three launches on the caller's stream:
//   1. rotate_q:  q_rot = fp16(q @ R) per (b, q-head).
//   2. split:     one workgroup per (b, context split, group of 8 KV heads);
//                 wave w owns KV head 8*blockIdx.y + w and its GQA group.  Two
//                 kernels compute the same partials: decode_stream_kernel
//                 (8 KV heads, 144-byte slots, one codebook for K and V;
//                 pages stream into per-wave LDS rings by DMA, 64 tokens per
//                 step) and decode_split_kernel (any head count and slot
//                 width; 32 tokens per step loaded straight into registers).
//                 Codes are dequantised through LDS tables indexed by code
//                 byte, one table column per lane so reads do not conflict.
//                 K and V are both rebuilt as fp16(centroid * norm) per
//                 element, exactly as the reference decodes them
//                 (compression.py:355-359).  QK^T and PV run on MFMA 16x16x32
//                 f16 with the GQA group as the N=16 side, with an exp2-domain
//                 online softmax.  It writes (O_unnorm, m, l) per split.
//   3. combine:   merges the splits (attention.py:239-272), rounds O_rot to
//                 fp16 (attention.py:93), applies R^T (compression.py:293-296)
//                 and writes fp16 out.
#include "cda_common.h"

#include <atomic>
#include <mutex>
#include <string>
#include <type_traits>
#include <utility>

namespace cda {

namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int kWaves = 8;                 // KV heads per workgroup
constexpr int kThreads = 64 * kWaves;
constexpr int kChunk = 32;                // tokens per inner iteration (2 MFMA tiles)
// Dequant tables of decode_split_kernel in LDS (128 KiB), one 256-byte row per
// code byte e holding the fp32 centroid pair (cb[e >> 4], cb[e & 15]) for 32
// lane columns: K at [0, 64 KiB), V at [64 KiB, 128 KiB).  Lane l reads column
// (l & 31), so reads never conflict, and the byte address is one v_perm of the
// code byte with a per-lane constant (byte 2 of that constant carries the
// 64 KiB bit of the V table).
constexpr int kLutDwords = 2 * 256 * 64;
constexpr float kLog2e = 1.4426950408889634f;

struct SplitParams {
    const uint16_t *q_rot;      // (B, H_q, 128) fp16
    const uint8_t *kv;          // paged cache
    const int32_t *block_table; // (B, bt_stride)
    const int32_t *seq_lens;    // (B,)
    const float *cb_k;
    const float *cb_v;
    float *part_o;              // (B, S, H_q, 128)
    float *part_ml;             // (B, S, H_q, 2): m (log2 domain), l
    int64_t row_bytes;          // H_kv * slot_bytes
    int bt_stride;
    int H_q;
    int H_kv;
    int slot_bytes;
    int block_size;
    int tile_n;
    int n_splits;
    float scale_log2;           // softmax scale * log2(e)
    int levels;                 // codebook levels: 16 (4-bit codes) or 4 (2-bit codes)
    // Set when both split kernels are launched (codebooks passed as two
    // pointers): 1 if they hold equal bits.  The page-streaming kernel runs
    // only if 1, the general kernel only if 0.
    const int *cb_same;
    // Score-domain QK (decode_stream_kernel's SQK form): 1 if cb_k holds the
    // 16-level uniform codebook (2i + 1)/16 - 1, written by rotate_q_kernel.
    const int *k_uniform;
    // Single-launch form (decode_stream_kernel's FUSED form): one workgroup
    // per (sequence, split, KV head), its waves on consecutive token ranges
    // of wave_tokens each; the workgroup rotates q itself and, when the split
    // covers the whole sequence (n_splits == 1), writes out itself.
    const uint16_t *q;          // (B, H_q, 128) fp16, un-rotated
    const float *R;             // (128, 128) fp32 rotation
    uint16_t *out;              // (B, H_q, 128) fp16
    int wave_tokens;            // multiple of 64
    int xcd_map;                // 1: the 8 heads of a (sequence, split) share an XCD
};

__device__ __forceinline__ floatx4 mfma16(uint4 a, uint4 b, floatx4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, a),
                                                  __builtin_bit_cast(half8, b), c, 0, 0, 0);
}

// LDS table read: byte address = code_byte * 256 + column offset.
__device__ __forceinline__ float2 lut2_at(const uint32_t *lut, uint32_t addr) {
    return *reinterpret_cast<const float2 *>(reinterpret_cast<const char *>(lut) + addr);
}

// fp16(a), fp16(b) packed, round-to-nearest-even (v_cvt_pk_f16_f32 on gfx950).
__device__ __forceinline__ uint32_t cvt_pk_rn(float a, float b) {
    typedef float float2_ __attribute__((ext_vector_type(2)));
    typedef _Float16 half2_ __attribute__((ext_vector_type(2)));
    const half2_ h = __builtin_convertvector(float2_{a, b}, half2_);
    return __builtin_bit_cast(uint32_t, h);
}

// max of three floats, NaN-propagating (v_maximum3_f32 on gfx950; no
// canonicalisation moves).  Compiler-visible, so the MFMA-result read
// hazards before it are handled by the compiler.
__device__ __forceinline__ float max3f(float a, float b, float c) {
    return __builtin_elementwise_maximum(__builtin_elementwise_maximum(a, b), c);
}

// Table address of code byte k of `w`: byte 0 <- col.byte0, byte 1 <- w.byte[k],
// byte 2 <- col.byte2, byte 3 <- 0.
template <int k>
__device__ __forceinline__ uint32_t lut_addr(uint32_t w, uint32_t col) {
    return __builtin_amdgcn_perm(w, col, 0x0C020400u | ((4u + k) << 8));
}

// max / sum over the four 16-lane rows of a wave (lanes l, l^16, l^32, l^48)
// with the gfx950 row-swap permutes; every lane gets the result.
__device__ __forceinline__ float rows_max(float v) {
    auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
    auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}

__device__ __forceinline__ float rows_sum(float v) {
    auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = __uint_as_float(a[0]) + __uint_as_float(a[1]);
    auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

struct Chunk {
    uint4 kq[2];        // K codes: token r16 of tile t, dims [32*q4, 32*q4+32)
    float nk[2];        // K norm of token r16 of tile t
    uint32_t vw[2][4];  // V codes: token 4*q4+i of tile t, dims [8*r16, 8*r16+8)
    float nv[2][4];     // V norm of token 4*q4+i of tile t
};

typedef __amdgpu_buffer_rsrc_t rsrc_t;

// Buffer descriptor over the 16 token rows of one tile (wave-uniform base in
// SGPRs, so per-lane addressing is a constant 32-bit offset; reads past the
// range return 0).
__device__ __forceinline__ rsrc_t tile_rsrc(const uint8_t *base, int nbytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(base), 0, nbytes, 0x00020000);
}

struct LaneOffsets {
    uint32_t k, nk, v[4], nv[4];
};

// Two bytes of 2-bit codes (pack_2bit: dim 4j at bits 7:6 of byte j,
// compression.py:382-386) -> four bytes in the 4-bit layout (dim 2k in the
// high nibble of byte k), so both code widths share the 4-bit tables.
__device__ __forceinline__ uint32_t widen_2bit(uint32_t x) {
    const uint32_t y = (x & 0xFFu) | ((x & 0xFF00u) << 8);
    return ((y >> 2) & 0x00300030u) | ((y >> 4) & 0x00030003u) | ((y << 10) & 0x30003000u) |
           ((y << 8) & 0x03000300u);
}

// One 16-token tile of a chunk.  K: 16 code bytes per lane (LK = 16) or 8
// widened to the 4-bit layout (LK = 4); V likewise 4 or 2 bytes per token.
template <int LK, int LV>
__device__ __forceinline__ void load_tile(Chunk &c, int t, rsrc_t r, const LaneOffsets &o) {
    if constexpr (LK == 16) {
        c.kq[t] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, o.k, 0, 0));
    } else {
        typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
        const u32x2 k2 = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(r, o.k, 0, 0));
        c.kq[t] = make_uint4(widen_2bit(k2.x & 0xFFFFu), widen_2bit(k2.x >> 16),
                             widen_2bit(k2.y & 0xFFFFu), widen_2bit(k2.y >> 16));
    }
    c.nk[t] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, o.nk, 0, 0));
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        if constexpr (LV == 16)
            c.vw[t][i] = __builtin_amdgcn_raw_buffer_load_b32(r, o.v[i], 0, 0);
        else
            c.vw[t][i] = widen_2bit(__builtin_amdgcn_raw_buffer_load_b16(r, o.v[i], 0, 0));
        c.nv[t][i] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, o.nv[i], 0, 0));
    }
}

template <int GS, int LK, int LV>
__global__ void __launch_bounds__(kThreads, 1)
decode_split_kernel(SplitParams p) {
    if (p.cb_same && *p.cb_same) return;        // the page-streaming kernel covers this call
    __shared__ __align__(16) uint32_t lds[kLutDwords];

    const int sp = blockIdx.x;
    const int b = blockIdx.z;
    const int tid = threadIdx.x;

    // ---- dequant tables (layout above).  K holds fp32 centroids: the decoded
    // K is rounded to fp16 only after the norm multiply, as the reference
    // decode does.
    {
        __shared__ float cbs[2][16];
        // Entries past the codebook are never indexed (widened 2-bit codes
        // stay below 4); they are set to 0 rather than read out of bounds.
        if (tid < 32) {
            const int e = tid & 15;
            cbs[tid >> 4][e] = (tid < 16) ? (e < LK ? p.cb_k[e] : 0.0f) : (e < LV ? p.cb_v[e] : 0.0f);
        }
        __syncthreads();
        for (int i = tid; i < kLutDwords / 2; i += kThreads) {
            const int e = i >> 6;
            lds[i] = __float_as_uint(cbs[0][(i & 1) ? (e & 15) : (e >> 4)]);
            lds[kLutDwords / 2 + i] = __float_as_uint(cbs[1][(i & 1) ? (e & 15) : (e >> 4)]);
        }
        __syncthreads();
    }

    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);   // uniform per wave
    const int lane = tid & 63;
    const int h = blockIdx.y * kWaves + wave;
    if (h >= p.H_kv) return;
    const int r16 = lane & 15;
    const int q4 = lane >> 4;

    // Keys past the block-table row are never read, whatever seq_lens says.
    const int seq_len =
        __builtin_amdgcn_readfirstlane(min(p.seq_lens[b], p.bt_stride * p.block_size));
    const int start = sp * p.tile_n;
    const int end = min(start + p.tile_n, seq_len);
    const int64_t part_row = ((int64_t)b * p.n_splits + sp) * p.H_q + (int64_t)h * GS;

    if (start >= end) {
        if (q4 == 0 && r16 < GS) {
            p.part_ml[(part_row + r16) * 2 + 0] = -INFINITY;
            p.part_ml[(part_row + r16) * 2 + 1] = 0.0f;
        }
        for (int i = lane; i < GS * kD; i += 64) p.part_o[part_row * kD + i] = 0.0f;
        return;
    }

    // ---- query operand (B of QK^T): column g = r16, k slots = dims 32*q4+8*s+j.
    // Columns g >= GS are zero; their scores are 0, so their (unused) rows of
    // P and O stay finite.
    uint4 qb[4];
    {
        const uint4 z = make_uint4(0, 0, 0, 0);
        const uint16_t *qg = p.q_rot + ((int64_t)b * p.H_q + (int64_t)h * GS + r16) * kD + 32 * q4;
#pragma unroll
        for (int s = 0; s < 4; ++s)
            qb[s] = (r16 < GS) ? *reinterpret_cast<const uint4 *>(qg + 8 * s) : z;
    }

    const uint32_t colK = (uint32_t)(lane & 31) * 8u;
    const uint32_t colV = 0x10000u | ((uint32_t)(lane & 31) * 8u);
    // Slot: [K codes KBK | V codes KBV | K norm | V norm | pad].
    constexpr int KBK = (LK == 16) ? kD / 2 : kD / 4;
    constexpr int KBV = (LV == 16) ? kD / 2 : kD / 4;
    LaneOffsets lo;
    lo.k = (uint32_t)(r16 * p.row_bytes + q4 * (KBK / 4));
    lo.nk = (uint32_t)(r16 * p.row_bytes + KBK + KBV);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        lo.v[i] = (uint32_t)((4 * q4 + i) * p.row_bytes + KBK + (KBV / 16) * r16);
        lo.nv[i] = (uint32_t)((4 * q4 + i) * p.row_bytes + KBK + KBV + 4);
    }
    const int32_t *bt = p.block_table + (int64_t)b * p.bt_stride;
    const uint8_t *kvh = p.kv + (int64_t)h * p.slot_bytes;
    const int bs = p.block_size;
    const int tile_bytes = (int)(16 * p.row_bytes);

    auto tile_res = [&](int t0) -> rsrc_t {
        // The page id is wave-uniform: keep it (and the descriptor) in SGPRs.
        const int page = __builtin_amdgcn_readfirstlane(bt[t0 / bs]);
        const int64_t slot = (int64_t)page * bs + (t0 % bs);
        return tile_rsrc(kvh + slot * p.row_bytes, tile_bytes);
    };

    auto load_chunk = [&](Chunk &c, int c0) {
        const rsrc_t r0 = tile_res(c0);
        const rsrc_t r1 = (c0 + 16 < end) ? tile_res(c0 + 16) : r0;
        load_tile<LK, LV>(c, 0, r0, lo);
        load_tile<LK, LV>(c, 1, r1, lo);
    };

    floatx4 acc_o[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) acc_o[j] = floatx4{0.f, 0.f, 0.f, 0.f};
    float m_run = -INFINITY;   // running max of column g = r16 (log2 domain)
    float l_run = 0.0f;        // lane-partial running sum

    auto compute_chunk = [&](const Chunk &c, int c0, auto masked) {
        constexpr bool MASK = decltype(masked)::value;
        // ---- S = K Q^T: rows = 16 tokens of a tile, cols = GQA group.  The K
        // operand is fp16(centroid * norm), bit-identical to the reference's
        // decoded K (compression.py:355-359).  All 16 table reads of a tile
        // are issued before the first is used.
        floatx4 sc[2];
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            const uint32_t w[4] = {c.kq[t].x, c.kq[t].y, c.kq[t].z, c.kq[t].w};
            float2 cv[16];
#pragma unroll
            for (int s = 0; s < 4; ++s) {
                cv[4 * s + 0] = lut2_at(lds, lut_addr<0>(w[s], colK));
                cv[4 * s + 1] = lut2_at(lds, lut_addr<1>(w[s], colK));
                cv[4 * s + 2] = lut2_at(lds, lut_addr<2>(w[s], colK));
                cv[4 * s + 3] = lut2_at(lds, lut_addr<3>(w[s], colK));
            }
            const float nk = c.nk[t];
            floatx4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int s = 0; s < 4; ++s) {
                uint4 a;
                a.x = cvt_pk_rn(cv[4 * s + 0].x * nk, cv[4 * s + 0].y * nk);
                a.y = cvt_pk_rn(cv[4 * s + 1].x * nk, cv[4 * s + 1].y * nk);
                a.z = cvt_pk_rn(cv[4 * s + 2].x * nk, cv[4 * s + 2].y * nk);
                a.w = cvt_pk_rn(cv[4 * s + 3].x * nk, cv[4 * s + 3].y * nk);
                acc = mfma16(a, qb[s], acc);
            }
            sc[t] = acc;
        }
        // ---- V operand: column n = r16 of tile j holds dim 8*r16 + j; k slot
        // pairs (2p, 2p+1) = tokens (4*q4 + 2*(p%2), +1) of tile p/2.  Pair two
        // tokens' nibbles of one dim into one byte, then one table read gives
        // both fp16 values.  The 32 reads are issued here, ahead of the softmax.
        uint32_t ev[4], od[4];
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int m2 = 0; m2 < 2; ++m2) {
                const uint32_t wa = c.vw[t][2 * m2];
                const uint32_t wb = c.vw[t][2 * m2 + 1];
                ev[2 * t + m2] = (wa & 0xF0F0F0F0u) | ((wb >> 4) & 0x0F0F0F0Fu);
                od[2 * t + m2] = ((wa << 4) & 0xF0F0F0F0u) | (wb & 0x0F0F0F0Fu);
            }
        float2 vc[32];
#define CDA_V_TILE(K_, SRC_, J_)                                               \
    vc[4 * (J_) + 0] = lut2_at(lds, lut_addr<K_>(SRC_[0], colV));              \
    vc[4 * (J_) + 1] = lut2_at(lds, lut_addr<K_>(SRC_[1], colV));              \
    vc[4 * (J_) + 2] = lut2_at(lds, lut_addr<K_>(SRC_[2], colV));              \
    vc[4 * (J_) + 3] = lut2_at(lds, lut_addr<K_>(SRC_[3], colV));
        CDA_V_TILE(0, ev, 0)
        CDA_V_TILE(0, od, 1)
        CDA_V_TILE(1, ev, 2)
        CDA_V_TILE(1, od, 3)
        CDA_V_TILE(2, ev, 4)
        CDA_V_TILE(2, od, 5)
        CDA_V_TILE(3, ev, 6)
        CDA_V_TILE(3, od, 7)
#undef CDA_V_TILE
        // ---- online softmax in the log2 domain: the max is taken on the raw
        // scores (scale > 0), the scale is fused into the exponent argument.
        float raw[2][4];
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                raw[t][i] = sc[t][i];
                if (MASK && c0 + 16 * t + 4 * q4 + i >= end) raw[t][i] = -INFINITY;
            }
        float cmax = max3f(max3f(raw[0][0], raw[0][1], raw[0][2]),
                           max3f(raw[0][3], raw[1][0], raw[1][1]),
                           max3f(raw[1][2], raw[1][3], raw[1][3]));
        cmax = rows_max(cmax);
        const float m_new = fmaxf(m_run, cmax * p.scale_log2);
        const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);   // m_run = -inf -> 0
        m_run = m_new;
        // ---- P (A operand of PV): row g = r16, k slot j <-> (tile j/4, token 4*q4 + j%4).
        float pv[2][4];
        float psum = 0.0f;
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float pr = __builtin_amdgcn_exp2f(fmaf(raw[t][i], p.scale_log2, -m_new));
                psum += pr;
                // A masked token weighs 0 (its V may be garbage).
                pv[t][i] = (MASK && c0 + 16 * t + 4 * q4 + i >= end) ? 0.0f : pr;
            }
        l_run = fmaf(l_run, alpha, psum);
        uint4 pa;
        pa.x = cvt_pk_rn(pv[0][0], pv[0][1]);
        pa.y = cvt_pk_rn(pv[0][2], pv[0][3]);
        pa.z = cvt_pk_rn(pv[1][0], pv[1][1]);
        pa.w = cvt_pk_rn(pv[1][2], pv[1][3]);
        // ---- rescale O rows (row g = 4*q4 + i) when any group max moved.
        float al[GS];
        bool moved = false;
#pragma unroll
        for (int g = 0; g < GS; ++g) {
            al[g] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(alpha), g));
            moved |= (al[g] != 1.0f);
        }
        if (moved) {
            float f[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                f[i] = 1.0f;
#pragma unroll
                for (int g = 0; g < GS; ++g)
                    if (4 * q4 + i == g) f[i] = al[g];
            }
#pragma unroll
            for (int j = 0; j < 8; ++j)
#pragma unroll
                for (int i = 0; i < 4; ++i) acc_o[j][i] *= f[i];
        }
        // V rebuilt exactly as the reference decodes it: fp16(centroid * norm)
        // per element; a masked token's V is zeroed (0 * garbage could be NaN).
        float nva[2][4];
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int i = 0; i < 4; ++i)
                nva[t][i] = (MASK && c0 + 16 * t + 4 * q4 + i >= end) ? 0.0f : c.nv[t][i];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            uint4 vb;
            vb.x = cvt_pk_rn(vc[4 * j + 0].x * nva[0][0], vc[4 * j + 0].y * nva[0][1]);
            vb.y = cvt_pk_rn(vc[4 * j + 1].x * nva[0][2], vc[4 * j + 1].y * nva[0][3]);
            vb.z = cvt_pk_rn(vc[4 * j + 2].x * nva[1][0], vc[4 * j + 2].y * nva[1][1]);
            vb.w = cvt_pk_rn(vc[4 * j + 3].x * nva[1][2], vc[4 * j + 3].y * nva[1][3]);
            acc_o[j] = mfma16(pa, vb, acc_o[j]);
        }
    };

    // ---- main loop over the full 32-token chunks; loads run one chunk
    // ahead.  A partial last chunk is handled after the loop, so the loop body
    // carries no masking.
    const int nfull = (end - start) / kChunk;
    int i = 0;
    Chunk ca, cb;
    if (nfull > 0) load_chunk(ca, start);
#define CDA_STEP(CUR, NEXT)                                                    \
    {                                                                          \
        if (i >= nfull) break;                                                 \
        if (i + 1 < nfull) load_chunk(NEXT, start + (i + 1) * kChunk);         \
        compute_chunk(CUR, start + i * kChunk, std::false_type{});             \
        ++i;                                                                   \
    }
    while (true) {
        CDA_STEP(ca, cb)
        CDA_STEP(cb, ca)
    }
#undef CDA_STEP
    if (start + nfull * kChunk < end) {
        load_chunk(ca, start + nfull * kChunk);
        compute_chunk(ca, start + nfull * kChunk, std::true_type{});
    }

    // ---- partials.
    const float l = rows_sum(l_run);
    if (q4 == 0 && r16 < GS) {
        p.part_ml[(part_row + r16) * 2 + 0] = m_run;
        p.part_ml[(part_row + r16) * 2 + 1] = l;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int g = 4 * q4 + i;
        if (g < GS) {
            float4 *dst = reinterpret_cast<float4 *>(p.part_o + (part_row + g) * kD + 8 * r16);
            dst[0] = make_float4(acc_o[0][i], acc_o[1][i], acc_o[2][i], acc_o[3][i]);
            dst[1] = make_float4(acc_o[4][i], acc_o[5][i], acc_o[6][i], acc_o[7][i]);
        }
    }
}

// ---------------------------------------------------------------------------
// Page-streaming split kernel for the common cache shapes: 8 KV heads x
// 144-byte K4V4 slots (L = 16) or 80-byte K2V2 slots (L = 4), a block size
// that is a multiple of 16 and one codebook for K and V.  The K4V4 layout is
// described first; the K2V2 differences follow.
//
// Wave h (one per KV head) streams its head's share of each 16-token page
// (16 x 144 B = 2304 B) into a private 4-page LDS ring with the gfx950
// direct-to-LDS DMA (buffer_load_dwordx4 ... lds): three instructions per page
// (K codes, V codes, norms), each lane fetching one 16-byte piece.  The waves
// never wait for each other: each one waits on its own DMA counter only.  A
// step takes a chunk of four pages (64 tokens): wait for the chunk's DMAs,
// read the four pages into registers, refill the four slots with the next
// chunk (in flight while this one computes), then QK^T on the four pages
// (independent MFMA chains), one online-softmax update over the 64 tokens and
// PV over two page pairs.  Page k of a chunk lives in ring slot k, so every
// ring offset is an immediate.  Within a page the pieces are laid out so that
// every read is free of LDS bank conflicts:
//   [0, 1024)     K codes: piece 16*c + t = token t, 16-byte column c (0..3)
//   [1024, 2048)  V codes: token t's 64 bytes at 64 * vslot(t)
//   [2048, 2304)  norms:   token t's (Kn, Vn, pad) at 16 * t
// One dequant table serves K and V: row e (256 B) holds (cb[e >> 4],
// cb[e & 15]) in fp32 for 32 lane columns, read with one ds_read_b64 per code
// byte.
//
// K2V2 (1280 B per head and page, two DMA instructions):
//   [0, 512)      K codes: piece 16*c + t = token t, 16-byte column c (0..1)
//   [512, 1024)   V codes: token t's 32 bytes at 32 * vslot2(t)
//   [1024, 1280)  norms, as above
// The table row e (256 B) holds, for 16 lane columns of 16 bytes,
// (cb[e >> 6], cb[(e >> 4) & 3], cb[(e >> 2) & 3], cb[e & 3]): a byte of
// 2-bit codes (dims 4j..4j+3, first dim in bits 7:6) gives its four values in
// one ds_read_b128.  For V, four tokens' codes of one dim are first
// gathered into one byte (bit-field inserts), so one read likewise gives the
// four tokens' values of that dim.
// ---------------------------------------------------------------------------

constexpr int kHeadPage = 16 * 144;      // largest share of one head in a page (K4V4): 2304 B

template <int N>
using IC = std::integral_constant<int, N>;

constexpr int kLut2Bytes = 256 * 64 * 4;                   // 64 KiB
constexpr int kStreamMaxPages = 1024;                      // page rows staged in LDS

typedef unsigned v4u32 __attribute__((ext_vector_type(4)));

// One 16-byte-per-lane direct-to-LDS load: lane l's 16 bytes at rsrc+voff go
// to LDS address lds_base + 16*l.  Issued through asm so the compiler does not
// track these asynchronous LDS writes (its tracking is conservative and would
// serialise the ring); completion is ordered by the explicit vmcnt waits.  M0
// (the LDS base operand) is saved and restored around the load, so the
// compiler's own use of M0 is never disturbed.
__device__ __forceinline__ void dma_page_chunk(v4u32 rsrc, uint32_t voff, uint32_t lds_base) {
    uint32_t saved;
    asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %3\n\t"
                 "buffer_load_dwordx4 %1, %2, 0 offen lds\n\ts_mov_b32 m0, %0"
                 : "=&s"(saved) : "v"(voff), "s"(rsrc), "s"(lds_base) : "memory");
}

__device__ __forceinline__ uint32_t lds_u32addr(const void *p) {
    return (uint32_t)(size_t)(const __attribute__((address_space(3))) void *)p;
}

__device__ __forceinline__ uint32_t lds_b32(const uint8_t *base, uint32_t off) {
    return *reinterpret_cast<const uint32_t *>(base + off);
}

// 64-byte V slot of token t within its group of four: the four tokens read
// together (4*q4 + i, q4 = 0..3) land in four different bank quarters.
__host__ __device__ constexpr int vslot(int t) { return (t & 12) | ((t + (t >> 2)) & 3); }
__host__ __device__ constexpr int vslot_inv(int s) { return (s & 12) | ((s - (s >> 2)) & 3); }

// The score-domain form (SQK) bounds the drift between its waves with a
// workgroup barrier every 8 chunks: with the lighter K side it is bound by the
// fetched bytes, and waves that drift apart fetch the 64-byte segments shared
// by neighbouring heads twice (B=32, N=64K: 495 -> 468 us; every 2, 3, 16
// chunks 469-482 us).  The exact-dequant form runs slower with any such
// barrier (its VALU phases would fall into lockstep).
constexpr int kSqkSyncChunks = 8;
constexpr int kStreamPages = 4;
constexpr int kStreamRingOff = kLut2Bytes;
constexpr int kStreamPidOff = kStreamRingOff + kWaves * kStreamPages * kHeadPage;
constexpr int kStreamLds = kStreamPidOff + kStreamMaxPages * 4;           // 143360 B
// FUSED form: a workgroup covers up to 4096 pages of one head, and stages q
// (fp32) and q_rot (fp16) of its GQA group after the page rows.
constexpr int kFusedMaxPages = 4096;
constexpr int kFusedQOff = kStreamPidOff + kFusedMaxPages * 4;
constexpr int kFusedQrOff = kFusedQOff + 8 * kD * 4;
constexpr int kFusedLds = kFusedQrOff + 8 * kD * 2;                         // 159744 B
static_assert(kFusedLds <= 160 * 1024, "FUSED LDS");

// K2V2 V slot of token t: the four tokens read together (4*q4 + i, q4 =
// 0..3) land in four consecutive 32-byte slots (an involution).
__host__ __device__ constexpr int vslot2(int t) { return ((t & 3) << 2) | (t >> 2); }

// Bit-field insert: bits of a where m is set, of b elsewhere (v_bfi_b32).
__device__ __forceinline__ uint32_t bfi(uint32_t m, uint32_t a, uint32_t b) {
    return (m & a) | (~m & b);
}

// SQK: score-domain QK for the 16-level uniform K codebook
// (attention.py:101-152): score = Kn * (q_rot . code / 8 - 15/16 * sum(q_rot)).
// The K operand of the MFMA is the 4-bit code itself, as the fp16 bit pattern
// code (the subnormal code * 2^-24, exact; no table, no multiply), so
// q_rot . code = acc * 2^24 exactly up to fp32 accumulation; V is decoded
// as in the default form, through a table of cb_v.
template <int GS, int L, bool SQK = false, bool FUSED = false>
__global__ void __launch_bounds__(kThreads, 1)
decode_stream_kernel(SplitParams p) {
    if (!FUSED && !SQK && p.cb_same && !*p.cb_same) return;   // different codebooks: the general kernel runs
    static_assert(L == 16 || L == 4, "4-bit or 2-bit codes");
    static_assert(!SQK || L == 16, "score-domain QK: 4-bit K codes");
    static_assert(!(SQK && FUSED), "the score-domain form runs as three launches");
    static_assert(GS == 4 || GS == 8, "GQA groups of 4 or 8");
    // The MFMA's 16 score columns hold the GS heads RP times over, so every
    // lane holds every score of its head RP times.  Each lane computes the
    // softmax weights of its own share only -- pages g_own + RP*j (j < NPL),
    // g_own = r16 / GS -- and the weights are exchanged before PV.
    constexpr int RP = 16 / GS;
    constexpr int NPL = 4 / RP;
    __shared__ __align__(16) uint8_t smem[FUSED ? kFusedLds : kStreamLds];
    constexpr int S = (L == 16) ? 144 : 80;        // slot bytes
    constexpr int KB = (L == 16) ? 64 : 32;        // code bytes per role
    constexpr int kRow = 8 * S;                    // one token row, all heads
    constexpr int kPB = 16 * kRow;                 // one 16-token page, all heads
    constexpr int kHP = 16 * S;                    // one head's share of a page
    constexpr uint32_t kVo = 16 * KB;              // V codes within a ring page
    constexpr uint32_t kNo = 32 * KB;              // norms within a ring page
    static_assert(kWaves * kStreamPages * kHP + kStreamRingOff <= kStreamPidOff, "ring fits");

    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lane = tid & 63;
    const int r16 = lane & 15;
    const int q4 = lane >> 4;
    int sp, b, h;
    if constexpr (FUSED) {
        // Linear id -> (unit = (sequence, split), head).  The hardware deals
        // workgroups to the 8 XCDs round-robin by linear id; with xcd_map the
        // 8 heads of a unit go to one XCD, so the 64-byte segments that
        // neighbouring heads' slots share are fetched into one L2.
        const int pl = blockIdx.x;
        int u;
        if (p.xcd_map) {
            const int i = pl >> 3;
            h = i & 7;
            u = ((i >> 3) << 3) + (pl & 7);
        } else {
            h = pl & 7;
            u = pl >> 3;
        }
        sp = u % p.n_splits;
        b = u / p.n_splits;
    } else {
        sp = blockIdx.x;
        b = blockIdx.z;
        h = wave;
    }

    const int seq_len =
        __builtin_amdgcn_readfirstlane(min(p.seq_lens[b], p.bt_stride * p.block_size));
    const int start = sp * p.tile_n;
    const int end = min(start + p.tile_n, seq_len);
    const int64_t part_row = ((int64_t)b * p.n_splits + sp) * p.H_q + (int64_t)h * GS;
    // This wave's token range: the whole split, or (FUSED) its own share.
    const int wstart = FUSED ? min(start + wave * p.wave_tokens, end) : start;
    const int wend = FUSED ? min(wstart + p.wave_tokens, end) : end;
    if (SQK && !*p.k_uniform) {
        // Not the uniform codebook: the output is NaN rather than wrong.
        if (q4 == 0 && r16 < GS) {
            p.part_ml[(part_row + r16) * 2 + 0] = __builtin_nanf("");
            p.part_ml[(part_row + r16) * 2 + 1] = __builtin_nanf("");
        }
        for (int i = lane; i < GS * kD; i += 64) p.part_o[part_row * kD + i] = __builtin_nanf("");
        return;
    }
    if (FUSED && start >= end && p.n_splits == 1) {
        // Empty sequence: the merge of no keys is 0 (weights 0, l clamped).
        for (int i = tid; i < GS * kD; i += kThreads)
            p.out[((int64_t)b * p.H_q + (int64_t)h * GS) * kD + i] = 0;
        return;
    }
    if (start >= end) {
        if (FUSED && wave != 0) return;
        if (q4 == 0 && r16 < GS) {
            p.part_ml[(part_row + r16) * 2 + 0] = -INFINITY;
            p.part_ml[(part_row + r16) * 2 + 1] = 0.0f;
        }
        for (int i = lane; i < GS * kD; i += 64) p.part_o[part_row * kD + i] = 0.0f;
        return;
    }

    // Source offset of lane's 16-byte piece within the head's page rows.
    uint32_t src[3];
    if constexpr (L == 16) {
        src[0] = (uint32_t)((lane & 15) * kRow + (lane >> 4) * 16);
        src[1] = (uint32_t)(vslot_inv(lane >> 2) * kRow + KB + (lane & 3) * 16);
        src[2] = (uint32_t)((lane & 15) * kRow + 2 * KB);   // lanes 0..15 only
    } else {
        // lanes 0..31: K pieces; lanes 32..63: V pieces (LDS 512 + 16*(lane-32)).
        const int j = lane & 31;
        src[0] = (lane < 32) ? (uint32_t)((j & 15) * kRow + (j >> 4) * 16)
                             : (uint32_t)(vslot2(j >> 1) * kRow + KB + (j & 1) * 16);
        src[2] = (uint32_t)((lane & 15) * kRow + 2 * KB);   // lanes 0..15 only
        src[1] = 0;
    }

    const int bs = p.block_size;
    const int npages = (end - start + 15) >> 4;          // the workgroup's pages
    const int wpage0 = (wstart - start) >> 4;            // this wave's first among them
    const int wnpages = (wend - wstart + 15) >> 4;
    const uint32_t ring_w = __builtin_amdgcn_readfirstlane(lds_u32addr(smem)) + kStreamRingOff +
                            wave * (kStreamPages * kHP);
    int32_t *page_row = reinterpret_cast<int32_t *>(smem + kStreamPidOff);
    {
        const int32_t *bt = p.block_table + (int64_t)b * p.bt_stride;
        for (int t = tid; t < npages; t += kThreads) {
            const int t0 = start + 16 * t;
            page_row[t] = bt[t0 / bs] * bs + (t0 % bs);
        }
    }
    const uint8_t *kv_h = p.kv + h * S;
    // DMA of the page starting at cache row row0 into ring slot k.
    auto issue_row = [&](int64_t row0, int k) CDA_INLINE {
        const uint64_t base = (uint64_t)(kv_h + row0 * kRow);
        const v4u32 r = {(uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)base),
                         (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(base >> 32) & 0xFFFFu),
                         (uint32_t)(kPB - h * S), 0x00020000u};
        const uint32_t sb = ring_w + (uint32_t)k * kHP;
        dma_page_chunk(r, src[0], sb);
        if constexpr (L == 16) dma_page_chunk(r, src[1], sb + kVo);
        if (lane < 16) dma_page_chunk(r, src[2], sb + kNo);
    };
    // DMA of page t (row from the workgroup's table) into ring slot k.
    auto issue = [&](int t, int k) CDA_INLINE {
        issue_row(__builtin_amdgcn_readfirstlane(page_row[wpage0 + t]), k);
    };
    // The first chunk's pages straight from the block table (wave-uniform
    // loads), before the tables are built: their latency overlaps the set-up.
    {
        const int32_t *bt = p.block_table + (int64_t)b * p.bt_stride;
#pragma unroll
        for (int k = 0; k < kStreamPages; ++k)
            if (k < wnpages) {
                const int t0 = wstart + 16 * k;
                issue_row((int64_t)__builtin_amdgcn_readfirstlane(bt[t0 / bs]) * bs + t0 % bs, k);
            }
    }
    uint4 qb[4];
    if constexpr (FUSED) {
        // q of this head's GQA group as fp32, for the rotation below.
        float *qs = reinterpret_cast<float *>(smem + kFusedQOff);
        const uint16_t *qg = p.q + ((int64_t)b * p.H_q + (int64_t)h * GS) * kD;
        for (int i = tid; i < GS * kD; i += kThreads) qs[i] = h2f(qg[i]);
    } else {
        const uint16_t *qg =
            p.q_rot + ((int64_t)b * p.H_q + (int64_t)h * GS + (r16 & (GS - 1))) * kD + 32 * q4;
#pragma unroll
        for (int s = 0; s < 4; ++s) qb[s] = *reinterpret_cast<const uint4 *>(qg + 8 * s);
    }
    // -15/16 * sum(q_rot) of this lane's query column (SQK), in fp32.
    float qsum_neg = 0.0f;
    if constexpr (SQK) {
        float a = 0.0f;
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            const uint32_t w[4] = {qb[s].x, qb[s].y, qb[s].z, qb[s].w};
#pragma unroll
            for (int e = 0; e < 4; ++e) a += h2f((uint16_t)(w[e] & 0xFFFFu)) + h2f((uint16_t)(w[e] >> 16));
        }
        a += __shfl_xor(a, 16);
        a += __shfl_xor(a, 32);
        qsum_neg = -0.9375f * a;
    }
    {
        // The codebook goes through LDS first: a global load per table entry
        // would put 32 dependent memory round trips in every thread's
        // prologue.
        __shared__ float cbs[16];
        if (tid < L) cbs[tid] = SQK ? p.cb_v[tid] : p.cb_k[tid];
        __syncthreads();
        uint32_t *lut = reinterpret_cast<uint32_t *>(smem);
        for (int i = tid; i < kLut2Bytes / 4; i += kThreads) {
            const int e = i >> 6;
            if constexpr (L == 16)
                lut[i] = __float_as_uint(cbs[(i & 1) ? (e & 15) : (e >> 4)]);
            else   // quad q of row e: the code in bits 7-2q:6-2q (dims 4j + q)
                lut[i] = __float_as_uint(cbs[(e >> (6 - 2 * (i & 3))) & 3]);
        }
    }
    if constexpr (FUSED) {
        // q_rot = fp16(q @ R): the fp32 fma chain over k in ascending order,
        // as rotate_q_kernel computes it (compression.py:290-291).
        const float *qs = reinterpret_cast<const float *>(smem + kFusedQOff);
        uint16_t *qr = reinterpret_cast<uint16_t *>(smem + kFusedQrOff);
        for (int o = tid; o < GS * kD; o += kThreads) {
            const float *qrow = qs + (o >> 7) * kD;
            const float *rc = p.R + (o & (kD - 1));
            float a = 0.0f;
#pragma unroll 16
            for (int k = 0; k < kD; ++k) a = fmaf(qrow[k], rc[k * kD], a);
            qr[o] = f2h_after_f32(a);
        }
    }
    __syncthreads();
    if constexpr (FUSED) {
        const uint16_t *qr = reinterpret_cast<const uint16_t *>(smem + kFusedQrOff) +
                             (r16 & (GS - 1)) * kD + 32 * q4;
#pragma unroll
        for (int s = 0; s < 4; ++s) qb[s] = *reinterpret_cast<const uint4 *>(qr + 8 * s);
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

    const uint32_t rb0 = (uint32_t)(kStreamRingOff + wave * (kStreamPages * kHP));
    // K4V4: token r16's 16 code bytes of dims [32*q4, +32); K2V2: its 8 bytes.
    const uint32_t oK = (L == 16) ? rb0 + (uint32_t)lane * 16u
                                  : rb0 + 256u * (q4 >> 1) + 16u * r16 + 8u * (q4 & 1);
    const uint32_t oNK = rb0 + kNo + 16u * r16;
    uint32_t oV[4], oNV[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        oV[i] = (L == 16) ? rb0 + kVo + 64u * vslot(4 * q4 + i) + 4u * r16
                          : rb0 + kVo + 32u * vslot2(4 * q4 + i) + 2u * r16;
        oNV[i] = rb0 + kNo + 16u * (4 * q4 + i) + 4u;
    }
    // Table column of this lane: 32 columns of 8-byte pairs (4-bit codes) or
    // 16 columns of 16-byte quads (2-bit codes); either way a row is 256 bytes.
    const uint32_t col = (L == 16) ? (uint32_t)(lane & 31) * 8u : (uint32_t)(lane & 15) * 16u;
    const uint8_t *lutb = smem;
    const int g_own = r16 / GS;

    floatx4 acc_o[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) acc_o[j] = floatx4{0.f, 0.f, 0.f, 0.f};
    float m_run = -INFINITY;
    float l_run = 0.0f;

#define CDA_PAIR(K_, W_) (*reinterpret_cast<const float2 *>(lutb + lut_addr<K_>(W_, col)))
    struct PageRegs {
        uint4 kq;
        float nk;
        uint32_t vw[4];
        float nv[4];
        float nki[4];      // SQK: K norms of tokens 4*q4 + i
    };
    auto read_page = [&](PageRegs &r, auto slot) CDA_INLINE {
        constexpr uint32_t so = decltype(slot)::value * kHP;
        if constexpr (L == 16) {
            r.kq = *reinterpret_cast<const uint4 *>(smem + oK + so);
        } else {
            const uint2 k2 = *reinterpret_cast<const uint2 *>(smem + oK + so);
            r.kq = make_uint4(k2.x, k2.y, 0u, 0u);
        }
        r.nk = __uint_as_float(lds_b32(smem + so, oNK));
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            if constexpr (L == 16)
                r.vw[k] = lds_b32(smem + so, oV[k]);
            else
                r.vw[k] = *reinterpret_cast<const uint16_t *>(smem + so + oV[k]);
            if constexpr (SQK) {
                const float2 kv = *reinterpret_cast<const float2 *>(smem + so + oNV[k] - 4);
                r.nki[k] = kv.x;
                r.nv[k] = kv.y;
            } else {
                r.nv[k] = __uint_as_float(lds_b32(smem + so, oNV[k]));
            }
        }
    };
    // Table reads of one page's K code bytes (the centroid pairs).
    auto k_lookup = [&](const PageRegs &r, float2 (&cv)[16]) CDA_INLINE {
        if constexpr (L == 16) {
            const uint32_t w[4] = {r.kq.x, r.kq.y, r.kq.z, r.kq.w};
#pragma unroll
            for (int s = 0; s < 4; ++s) {
                cv[4 * s + 0] = CDA_PAIR(0, w[s]);
                cv[4 * s + 1] = CDA_PAIR(1, w[s]);
                cv[4 * s + 2] = CDA_PAIR(2, w[s]);
                cv[4 * s + 3] = CDA_PAIR(3, w[s]);
            }
        } else {
            // Word x holds dims [16x, 16x+16) of the lane's 32, byte k dims
            // 16x + 4k .. +3; one 16-byte table read per byte gives all four.
            // MFMA s takes bytes 2s, 2s+1 (dims 8s..8s+7).
            const uint32_t w[2] = {r.kq.x, r.kq.y};
#define CDA_QUAD(K_, W_) (*reinterpret_cast<const float4 *>(lutb + lut_addr<K_>(W_, col)))
#pragma unroll
            for (int x = 0; x < 2; ++x) {
                const float4 q0 = CDA_QUAD(0, w[x]), q1 = CDA_QUAD(1, w[x]);
                const float4 q2 = CDA_QUAD(2, w[x]), q3 = CDA_QUAD(3, w[x]);
                cv[8 * x + 0] = make_float2(q0.x, q0.y);
                cv[8 * x + 1] = make_float2(q0.z, q0.w);
                cv[8 * x + 2] = make_float2(q1.x, q1.y);
                cv[8 * x + 3] = make_float2(q1.z, q1.w);
                cv[8 * x + 4] = make_float2(q2.x, q2.y);
                cv[8 * x + 5] = make_float2(q2.z, q2.w);
                cv[8 * x + 6] = make_float2(q3.x, q3.y);
                cv[8 * x + 7] = make_float2(q3.z, q3.w);
            }
#undef CDA_QUAD
        }
    };
    // fp16(centroid * norm) of those pairs and the page's QK MFMAs.
    auto k_math = [&](const PageRegs &r, const float2 (&cv)[16]) CDA_INLINE -> floatx4 {
        const float nk = r.nk;
        floatx4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            uint4 a;
            a.x = cvt_pk_rn(cv[4 * s + 0].x * nk, cv[4 * s + 0].y * nk);
            a.y = cvt_pk_rn(cv[4 * s + 1].x * nk, cv[4 * s + 1].y * nk);
            a.z = cvt_pk_rn(cv[4 * s + 2].x * nk, cv[4 * s + 2].y * nk);
            a.w = cvt_pk_rn(cv[4 * s + 3].x * nk, cv[4 * s + 3].y * nk);
            acc = mfma16(a, qb[s], acc);
        }
        return acc;
    };
    auto page_scores = [&](const PageRegs &r) CDA_INLINE -> floatx4 {
        if constexpr (SQK) {
            // Byte j of a code word: dims 2j (high nibble), 2j + 1 (low).
            floatx4 acc = {0.f, 0.f, 0.f, 0.f};
            const uint32_t w[4] = {r.kq.x, r.kq.y, r.kq.z, r.kq.w};
#pragma unroll
            for (int s = 0; s < 4; ++s) {
                const uint32_t lo = w[s] & 0x0F0F0F0Fu, hi = (w[s] >> 4) & 0x0F0F0F0Fu;
                uint4 a;
                a.x = __builtin_amdgcn_perm(lo, hi, 0x0C040C00u);
                a.y = __builtin_amdgcn_perm(lo, hi, 0x0C050C01u);
                a.z = __builtin_amdgcn_perm(lo, hi, 0x0C060C02u);
                a.w = __builtin_amdgcn_perm(lo, hi, 0x0C070C03u);
                acc = mfma16(a, qb[s], acc);
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[i] = r.nki[i] * fmaf(acc[i], 0x1p21f, qsum_neg);
            return acc;
        }
        float2 cv[16];
        k_lookup(r, cv);
        return k_math(r, cv);
    };
    // O += P V over pages ra, rb (k slots as in decode_stream_kernel).
    auto pv_pair = [&](const uint4 &pa, const PageRegs &ra, const PageRegs &rb) CDA_INLINE {
        uint32_t ev[4], od[4];
        float2 vc[32];
#define CDA_V_TILE(K_, SRC_, J_)                                               \
    vc[4 * (J_) + 0] = CDA_PAIR(K_, SRC_[0]);                                  \
    vc[4 * (J_) + 1] = CDA_PAIR(K_, SRC_[1]);                                  \
    vc[4 * (J_) + 2] = CDA_PAIR(K_, SRC_[2]);                                  \
    vc[4 * (J_) + 3] = CDA_PAIR(K_, SRC_[3]);
        if constexpr (L == 16) {
#pragma unroll
            for (int m2 = 0; m2 < 2; ++m2) {
                ev[m2] = (ra.vw[2 * m2] & 0xF0F0F0F0u) | ((ra.vw[2 * m2 + 1] >> 4) & 0x0F0F0F0Fu);
                od[m2] = ((ra.vw[2 * m2] << 4) & 0xF0F0F0F0u) | (ra.vw[2 * m2 + 1] & 0x0F0F0F0Fu);
                ev[2 + m2] = (rb.vw[2 * m2] & 0xF0F0F0F0u) | ((rb.vw[2 * m2 + 1] >> 4) & 0x0F0F0F0Fu);
                od[2 + m2] = ((rb.vw[2 * m2] << 4) & 0xF0F0F0F0u) | (rb.vw[2 * m2 + 1] & 0x0F0F0F0Fu);
            }
            CDA_V_TILE(0, ev, 0)
            CDA_V_TILE(0, od, 1)
            CDA_V_TILE(1, ev, 2)
            CDA_V_TILE(1, od, 3)
            CDA_V_TILE(2, ev, 4)
            CDA_V_TILE(2, od, 5)
            CDA_V_TILE(3, ev, 6)
            CDA_V_TILE(3, od, 7)
        } else {
            // Four tokens' 2-bit codes of one dim in one byte, first token in
            // bits 7:6 (the quad table's order), so one 16-byte read gives
            // the four k slots of a page.  A token's 16 bits (read little
            // endian) hold dims 8*r16 .. +3 in byte 0 and +4 .. +7 in byte 1,
            // the first dim of each byte in bits 7:6.  t01 pairs tokens 0, 1
            // into nibbles (byte 0: dims 0 | 2, byte 1: dims 4 | 6), u01 the
            // odd dims; then two nibble inserts give (dim 0 | dim 4),
            // (dim 1 | dim 5), (dim 2 | dim 6), (dim 3 | dim 7) in bytes 0 | 1
            // of four words.
            auto quads = [&](const PageRegs &rr, uint32_t (&qw)[4]) CDA_INLINE {
                const uint32_t v0 = rr.vw[0], v1 = rr.vw[1], v2 = rr.vw[2], v3 = rr.vw[3];
                const uint32_t t01 = bfi(0xCCCCu, v0, v1 >> 2), u01 = bfi(0xCCCCu, v0 << 2, v1);
                const uint32_t t23 = bfi(0xCCCCu, v2, v3 >> 2), u23 = bfi(0xCCCCu, v2 << 2, v3);
                qw[0] = bfi(0xF0F0u, t01, t23 >> 4);          // dims 0 (byte 0), 4 (byte 1)
                qw[1] = bfi(0xF0F0u, u01, u23 >> 4);          // dims 1, 5
                qw[2] = bfi(0xF0F0u, t01 << 4, t23);          // dims 2, 6
                qw[3] = bfi(0xF0F0u, u01 << 4, u23);          // dims 3, 7
            };
            uint32_t qa[4], qbw[4];
            quads(ra, qa);
            quads(rb, qbw);
#define CDA_QUAD(K_, W_) (*reinterpret_cast<const float4 *>(lutb + lut_addr<K_>(W_, col)))
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                // dim j: word j & 3, byte 0 for j < 4, byte 1 otherwise
                const float4 a4 = (j < 4) ? CDA_QUAD(0, qa[j & 3]) : CDA_QUAD(1, qa[j & 3]);
                const float4 b4 = (j < 4) ? CDA_QUAD(0, qbw[j & 3]) : CDA_QUAD(1, qbw[j & 3]);
                vc[4 * j + 0] = make_float2(a4.x, a4.y);
                vc[4 * j + 1] = make_float2(a4.z, a4.w);
                vc[4 * j + 2] = make_float2(b4.x, b4.y);
                vc[4 * j + 3] = make_float2(b4.z, b4.w);
            }
#undef CDA_QUAD
            (void)ev;
            (void)od;
        }
#undef CDA_V_TILE
        // The 32 table reads above all issue before the first multiply.
        __builtin_amdgcn_sched_barrier(0);
        // V rebuilt exactly as the reference decodes it: fp16(centroid * norm)
        // per element (k slot pairs are two tokens of one dim).
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            uint4 vb;
            vb.x = cvt_pk_rn(vc[4 * j + 0].x * ra.nv[0], vc[4 * j + 0].y * ra.nv[1]);
            vb.y = cvt_pk_rn(vc[4 * j + 1].x * ra.nv[2], vc[4 * j + 1].y * ra.nv[3]);
            vb.z = cvt_pk_rn(vc[4 * j + 2].x * rb.nv[0], vc[4 * j + 2].y * rb.nv[1]);
            vb.w = cvt_pk_rn(vc[4 * j + 3].x * rb.nv[2], vc[4 * j + 3].y * rb.nv[3]);
            acc_o[j] = mfma16(pa, vb, acc_o[j]);
        }
    };

    // ---- one chunk of four pages starting at page 4c (token c0).
    auto step = [&](int c, auto masked) CDA_INLINE {
        constexpr bool MASK = decltype(masked)::value;
        const int c0 = wstart + 64 * c;
        const int p0 = 4 * c;
        __builtin_amdgcn_s_waitcnt(0x0F70);        // this chunk's DMAs (the only ones in flight)
        asm volatile("" ::: "memory");
        PageRegs r[4];
        read_page(r[0], IC<0>{});
        if (!MASK || p0 + 1 < wnpages) read_page(r[1], IC<1>{});
        if (!MASK || p0 + 2 < wnpages) read_page(r[2], IC<2>{});
        if (!MASK || p0 + 3 < wnpages) read_page(r[3], IC<3>{});
        if (MASK) {
            // Pages past the split are not read: zero codes and norms (their
            // tokens are masked out below).
#pragma unroll
            for (int k = 1; k < 4; ++k)
                if (p0 + k >= wnpages) {
                    r[k].kq = make_uint4(0, 0, 0, 0);
                    r[k].nk = 0.0f;
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        r[k].vw[i] = 0u;
                        r[k].nv[i] = 0.0f;
                        r[k].nki[i] = 0.0f;
                    }
                }
        }
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        // Refill of ring slot k with the next chunk's page k, issued once page
        // k's scores are computed rather than all four before the math: under
        // full HBM load the direct-to-LDS loads are slow to issue, and spread
        // out they stall the wave less (B=32, N=64K: 510 -> 505 us).
        auto refill = [&](int k) CDA_INLINE {
            if (!MASK && p0 + 4 + k < wnpages) issue(p0 + 4 + k, k);
        };
        floatx4 sc[4];
        if constexpr (SQK) {
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                sc[k] = page_scores(r[k]);
                refill(k);
            }
        } else {
            // All 64 table reads of the chunk's K codes first, fenced from the
            // scheduler, so their LDS latency overlaps instead of stalling
            // each page's multiplies (534 -> 525 us at B=32, N=64K).
            float2 cvk[4][16];
#pragma unroll
            for (int k = 0; k < 4; ++k) k_lookup(r[k], cvk[k]);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                sc[k] = k_math(r[k], cvk[k]);
                refill(k);
            }
        }
        float raw[4][4];
#pragma unroll
        for (int k = 0; k < 4; ++k)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                raw[k][i] = sc[k][i];
                if (MASK && c0 + 16 * k + 4 * q4 + i >= wend) raw[k][i] = -INFINITY;
            }
        float cmax = max3f(max3f(raw[0][0], raw[0][1], raw[0][2]),
                           max3f(raw[0][3], raw[1][0], raw[1][1]),
                           max3f(raw[1][2], raw[1][3], raw[2][0]));
        cmax = max3f(cmax, max3f(raw[2][1], raw[2][2], raw[2][3]),
                     max3f(raw[3][0], raw[3][1], max3f(raw[3][2], raw[3][3], raw[3][3])));
        cmax = rows_max(cmax);
        // Lazy running max (log2 domain): it moves only when a chunk's max
        // exceeds it by more than 8, so P <= 2^8 (exact enough in fp16, far
        // from its range) and the O rescale below is skipped by the whole
        // wave on almost every chunk.
        const float cm = cmax * p.scale_log2;
        const bool move = cm > m_run + 8.0f;
        if (__builtin_amdgcn_ballot_w64(move)) {
            const float alpha = move ? __builtin_amdgcn_exp2f(m_run - cm) : 1.0f;  // -inf -> 0
            m_run = move ? cm : m_run;
            l_run *= alpha;
            float al[GS];
#pragma unroll
            for (int g = 0; g < GS; ++g)
                al[g] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(alpha), g));
            float f[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                f[i] = 1.0f;
#pragma unroll
                for (int g = 0; g < GS; ++g)
                    if (4 * q4 + i == g) f[i] = al[g];
            }
#pragma unroll
            for (int j = 0; j < 8; ++j)
#pragma unroll
                for (int i = 0; i < 4; ++i) acc_o[j][i] *= f[i];
        }
        const float m_sub = (m_run == -INFINITY) ? 0.0f : m_run;
        // Softmax weights of the lane's own share (page g_own + RP*j, token
        // 4*q4 + i), as fp16 pairs.
        uint32_t pw[NPL][2];
        float psum = 0.0f;
#pragma unroll
        for (int j = 0; j < NPL; ++j) {
            float pj[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                float sv = raw[j * RP][i];
#pragma unroll
                for (int t = 1; t < RP; ++t) sv = (g_own == t) ? raw[j * RP + t][i] : sv;
                const float pr = __builtin_amdgcn_exp2f(fmaf(sv, p.scale_log2, -m_sub));
                psum += pr;
                pj[i] = (MASK && c0 + 16 * (j * RP + g_own) + 4 * q4 + i >= wend) ? 0.0f : pr;
            }
            pw[j][0] = cvt_pk_rn(pj[0], pj[1]);
            pw[j][1] = cvt_pk_rn(pj[2], pj[3]);
        }
        l_run += psum;
        // Page kk's weights of head r16 % GS are in lane (kk % RP) * GS +
        // r16 % GS of this 16-lane row, register kk / RP: ds_swizzle in
        // bit-mask mode keeps the head and row bits and sets the page bits.
        constexpr int kGMask = (RP - 1) * GS;
        uint32_t xw[4][2];
#define CDA_SWZ(KK_)                                                                    \
    {                                                                                   \
        constexpr int pat = (0x1F & ~kGMask) | ((((KK_) % RP) * GS) << 5);              \
        xw[KK_][0] = (uint32_t)__builtin_amdgcn_ds_swizzle((int)pw[(KK_) / RP][0], pat); \
        xw[KK_][1] = (uint32_t)__builtin_amdgcn_ds_swizzle((int)pw[(KK_) / RP][1], pat); \
    }
        CDA_SWZ(0)
        CDA_SWZ(1)
        CDA_SWZ(2)
        CDA_SWZ(3)
#undef CDA_SWZ
        const uint4 pa0 = make_uint4(xw[0][0], xw[0][1], xw[1][0], xw[1][1]);
        const uint4 pa1 = make_uint4(xw[2][0], xw[2][1], xw[3][0], xw[3][1]);
        if (MASK) {
            // A masked token's V is zeroed: its slot may hold garbage norms.
#pragma unroll
            for (int k = 0; k < 4; ++k)
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    if (c0 + 16 * k + 4 * q4 + i >= wend) r[k].nv[i] = 0.0f;
        }
        pv_pair(pa0, r[0], r[1]);
        pv_pair(pa1, r[2], r[3]);
    };
#undef CDA_PAIR

    const int nchunks = (wnpages + 3) >> 2;
    const int nfull = (wend - wstart) >> 6;
    for (int c = 0; c < nfull; ++c) {
        step(c, std::false_type{});
        if constexpr (SQK) {
            if (c % kSqkSyncChunks == kSqkSyncChunks - 1) __syncthreads();
        }
    }
    if (nfull < nchunks) step(nfull, std::true_type{});

    // Each lane summed its own share: add the other pages' lanes of its row.
    float l = rows_sum(l_run);
    if constexpr (GS == 4)
        l += __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(l), 0x1F | (4 << 10)));
    l += __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(l), 0x1F | (8 << 10)));
    if constexpr (FUSED) {
        // Merge the eight waves' partials of this head's GQA group
        // (attention.py:239-272, log2 domain).  Each wave parks its (O, m, l)
        // in its own ring area, idle once its last chunk is read.
        auto wave_part = [&](int w) CDA_INLINE {
            return reinterpret_cast<float *>(smem + kStreamRingOff + w * (kStreamPages * kHP));
        };
        float *mine = wave_part(wave);
        if (q4 == 0 && r16 < GS) {
            mine[GS * kD + r16] = m_run;
            mine[GS * kD + GS + r16] = l;
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int g = 4 * q4 + i;
            if (g < GS) {
                float4 *dst = reinterpret_cast<float4 *>(mine + g * kD + 8 * r16);
                dst[0] = make_float4(acc_o[0][i], acc_o[1][i], acc_o[2][i], acc_o[3][i]);
                dst[1] = make_float4(acc_o[4][i], acc_o[5][i], acc_o[6][i], acc_o[7][i]);
            }
        }
        __syncthreads();
        float *orot = reinterpret_cast<float *>(smem);   // the table area, free now
        for (int o = tid; o < GS * kD; o += kThreads) {
            const int g = o >> 7, d = o & (kD - 1);
            float mw[kWaves];
            float M = -INFINITY;
#pragma unroll
            for (int w = 0; w < kWaves; ++w) {
                mw[w] = wave_part(w)[GS * kD + g];
                M = fmaxf(M, mw[w]);
            }
            float Ls = 0.0f, Os = 0.0f;
#pragma unroll
            for (int w = 0; w < kWaves; ++w) {
                const float a = (mw[w] == -INFINITY) ? 0.0f : exp2f(mw[w] - M);
                Ls = fmaf(a, wave_part(w)[GS * kD + GS + g], Ls);
                Os = fmaf(a, wave_part(w)[g * kD + d], Os);
            }
            if (p.n_splits == 1) {
                // As the merge's epilogue: fp16(O / l) (attention.py:93).
                orot[o] = h2f(f2h_after_f32(Os * (1.0f / fmaxf(Ls, 1e-30f))));
            } else {
                p.part_o[(part_row + g) * kD + d] = Os;
                if (d == 0) {
                    p.part_ml[(part_row + g) * 2 + 0] = M;
                    p.part_ml[(part_row + g) * 2 + 1] = Ls;
                }
            }
        }
        if (p.n_splits != 1) return;                     // combine_kernel merges the splits
        __syncthreads();
        // out[j] = sum_k fp16(O_rot)[k] * R[j][k], k ascending (compression.py:293-296):
        // thread j reads row j of R once for the group's GS heads.
        if (tid < kD) {
            const float4 *rrow = reinterpret_cast<const float4 *>(p.R + tid * kD);
            float a[GS];
#pragma unroll
            for (int g = 0; g < GS; ++g) a[g] = 0.0f;
#pragma unroll 8
            for (int k4 = 0; k4 < kD / 4; ++k4) {
                const float4 x = rrow[k4];
#pragma unroll
                for (int g = 0; g < GS; ++g) {
                    const float4 o4 = *reinterpret_cast<const float4 *>(orot + g * kD + 4 * k4);
                    a[g] = fmaf(o4.x, x.x, a[g]);
                    a[g] = fmaf(o4.y, x.y, a[g]);
                    a[g] = fmaf(o4.z, x.z, a[g]);
                    a[g] = fmaf(o4.w, x.w, a[g]);
                }
            }
            const int64_t orow = (int64_t)b * p.H_q + (int64_t)h * GS;
#pragma unroll
            for (int g = 0; g < GS; ++g) p.out[(orow + g) * kD + tid] = f2h_after_f32(a[g]);
        }
        return;
    }
    if (q4 == 0 && r16 < GS) {
        p.part_ml[(part_row + r16) * 2 + 0] = m_run;
        p.part_ml[(part_row + r16) * 2 + 1] = l;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int g = 4 * q4 + i;
        if (g < GS) {
            float4 *dst = reinterpret_cast<float4 *>(p.part_o + (part_row + g) * kD + 8 * r16);
            dst[0] = make_float4(acc_o[0][i], acc_o[1][i], acc_o[2][i], acc_o[3][i]);
            dst[1] = make_float4(acc_o[4][i], acc_o[5][i], acc_o[6][i], acc_o[7][i]);
        }
    }
}

// q_rot[b, h, j] = fp16(sum_k fp32(q[b, h, k]) * R[k, j]).  One 256-thread
// block per (4 q-heads, sequence): R is staged in LDS once (all its loads in
// flight together), then wave w computes head w, two output columns per lane.
constexpr int kHeadsPerBlock = 4;

__global__ void __launch_bounds__(256)
rotate_q_kernel(const uint16_t *q, const float *R, uint16_t *q_rot, int H_q,
                const float *cb_k, const float *cb_v, int levels, int *cb_same,
                int *k_uniform) {
    __shared__ __align__(16) float Rs[kD * kD];
    __shared__ float qs[kHeadsPerBlock][kD];
    const int b = blockIdx.y, t = threadIdx.x;
    if (cb_same && blockIdx.x == 0 && blockIdx.y == 0 && t < 64) {
        // Whether the K and V codebooks hold the same bits: selects between
        // the two split kernels launched after this one.
        const bool eq = t >= levels || __float_as_uint(cb_k[t]) == __float_as_uint(cb_v[t]);
        const bool all = __builtin_amdgcn_ballot_w64(!eq) == 0;
        if (t == 0) *cb_same = all ? 1 : 0;
    }
    if (k_uniform && blockIdx.x == 0 && blockIdx.y == 0 && t >= 64 && t < 128) {
        // Whether cb_k is the uniform codebook the score-domain QK assumes.
        const int i = t - 64;
        const bool eq = i >= 16 || cb_k[i] == (float)(2 * i + 1) * 0.0625f - 1.0f;
        const bool all = __builtin_amdgcn_ballot_w64(!eq) == 0;
        if (i == 0) *k_uniform = all ? 1 : 0;
    }
    const int h0 = blockIdx.x * kHeadsPerBlock;
    const float4 *R4 = reinterpret_cast<const float4 *>(R);
    float4 *Rs4 = reinterpret_cast<float4 *>(Rs);
#pragma unroll
    for (int i = 0; i < kD * kD / 4 / 256; ++i) Rs4[t + 256 * i] = R4[t + 256 * i];
    for (int i = t; i < kHeadsPerBlock * kD; i += 256) {
        const int hh = i / kD, k = i % kD;
        qs[hh][k] = (h0 + hh < H_q) ? h2f(q[((int64_t)b * H_q + h0 + hh) * kD + k]) : 0.0f;
    }
    __syncthreads();
    const int hh = t >> 6, j = 2 * (t & 63);
    if (h0 + hh >= H_q) return;
    float a0 = 0.0f, a1 = 0.0f;
#pragma unroll 8
    for (int k = 0; k < kD; ++k) {
        const float2 r = *reinterpret_cast<const float2 *>(Rs + k * kD + j);
        a0 = fmaf(qs[hh][k], r.x, a0);
        a1 = fmaf(qs[hh][k], r.y, a1);
    }
    const int64_t row = ((int64_t)b * H_q + h0 + hh) * kD;
    q_rot[row + j] = f2h_after_f32(a0);
    q_rot[row + j + 1] = f2h_after_f32(a1);
}

constexpr int kMaxSplits = 1024;

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int m = 1; m < 64; m <<= 1) v = fmaxf(v, __shfl_xor(v, m));
    return v;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int m = 1; m < 64; m <<= 1) v += __shfl_xor(v, m);
    return v;
}

// Merge split partials (attention.py:239-272: m* = max m_i, weights
// exp(m_i - m*), empty splits weigh 0, l clamped at 1e-30), round O_rot to
// fp16 and unrotate: out[j] = sum_k fp16(O_rot)[k] * R[j][k].  One 256-thread
// block per (4 q-heads, sequence): wave w merges head w (two splits per wave
// instruction, four dims per lane, 32 splits' loads in flight at a time).  R is staged in LDS in its own row
// order with rows padded to 132 floats, so the global reads are coalesced,
// all sixteen per thread are in flight at once, and the epilogue's 16-byte
// row reads (lane j reads row j) fall in distinct banks.
constexpr int kRPad = kD + 4;

// HPB heads per 256-thread block: 4 (one wave per head) when the grid fills
// the chip, else 1 (the four waves take interleaved 32-split batches of one
// head and their partial sums are added in a fixed order).
template <int HPB>
__global__ void __launch_bounds__(256)
combine_kernel(const float *part_o, const float *part_ml, const float *R, uint16_t *out,
               int H_q, int n_splits) {
    static_assert(HPB == 4 || HPB == 1, "heads per block");
    constexpr int kWph = 4 / HPB;                  // waves per head
    __shared__ __align__(16) float Rs[kD * kRPad];
    __shared__ float wts[4][kMaxSplits];
    __shared__ __align__(16) float orot[4][kD];
    const int b = blockIdx.y, t = threadIdx.x;
    const int h0 = blockIdx.x * HPB;
    const int hh = (HPB == 4) ? (t >> 6) : 0, lane = t & 63;
    const int wsub = (HPB == 4) ? 0 : (t >> 6);   // this wave's share of the splits
    const int wslot = t >> 6;                      // this wave's rows of wts / orot
    const int h = h0 + hh;
    float4 rr[kD * kD / 4 / 256];
    {
        const float4 *R4 = reinterpret_cast<const float4 *>(R);
#pragma unroll
        for (int u = 0; u < kD * kD / 4 / 256; ++u) rr[u] = R4[t + 256 * u];
    }
    const bool live = h < H_q;
    const int64_t base = (int64_t)b * n_splits * H_q + h;
    float L = 0.0f;
    if (live) {
        // All (m, l) pairs of this head in flight at once (up to kMaxSplits).
        constexpr int kPer = kMaxSplits / 64;
        float2 ml[kPer];
#pragma unroll
        for (int i = 0; i < kPer; ++i) {
            const int s = lane + 64 * i;
            ml[i] = (s < n_splits)
                        ? *reinterpret_cast<const float2 *>(part_ml + (base + (int64_t)s * H_q) * 2)
                        : make_float2(-INFINITY, 0.0f);
        }
        float mx = -INFINITY;
#pragma unroll
        for (int i = 0; i < kPer; ++i) mx = fmaxf(mx, ml[i].x);
        mx = wave_max(mx);
        float lp = 0.0f;
#pragma unroll
        for (int i = 0; i < kPer; ++i) {
            const int s = lane + 64 * i;
            const float w = (ml[i].x == -INFINITY) ? 0.0f : exp2f(ml[i].x - mx);
            if (s < n_splits) wts[wslot][s] = w;
            if (w != 0.0f) lp += w * ml[i].y;
        }
        L = wave_sum(lp);
    }
#pragma unroll
    for (int u = 0; u < kD * kD / 4 / 256; ++u) {
        const int i = t + 256 * u;
        *reinterpret_cast<float4 *>(Rs + (i >> 5) * kRPad + 4 * (i & 31)) = rr[u];
    }
    __syncthreads();
    if (live) {
        // Empty splits store zeros, so every partial is read unconditionally.
        // Lanes 0-31 take the even splits and lanes 32-63 the odd ones, four
        // dims per lane, sixteen 16-byte loads in flight: 32 splits per batch.
        const int half = lane >> 5, d4 = 4 * (lane & 31);
        const float *po = part_o + base * kD + d4;
        const int64_t step = (int64_t)H_q * kD;
        float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
        for (int s0 = 32 * wsub; s0 < n_splits; s0 += 32 * kWph) {
            float4 v[16];
#pragma unroll
            for (int u = 0; u < 16; ++u) {
                const int s = s0 + 2 * u + half;
                v[u] = (s < n_splits) ? *reinterpret_cast<const float4 *>(po + (int64_t)s * step)
                                      : make_float4(0.f, 0.f, 0.f, 0.f);
            }
#pragma unroll
            for (int u = 0; u < 16; ++u) {
                const int s = s0 + 2 * u + half;
                const float w = (s < n_splits) ? wts[wslot][s] : 0.0f;
                o.x = fmaf(w, v[u].x, o.x);
                o.y = fmaf(w, v[u].y, o.y);
                o.z = fmaf(w, v[u].z, o.z);
                o.w = fmaf(w, v[u].w, o.w);
            }
        }
        auto sum_halves = [](float x) {
            const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x),
                                                            false, false);
            return __uint_as_float(r[0]) + __uint_as_float(r[1]);
        };
        o.x = sum_halves(o.x);
        o.y = sum_halves(o.y);
        o.z = sum_halves(o.z);
        o.w = sum_halves(o.w);
        const float inv = 1.0f / fmaxf(L, 1e-30f);
        if (HPB == 4 && half == 0) {
            orot[hh][d4 + 0] = h2f(f2h_after_f32(o.x * inv));
            orot[hh][d4 + 1] = h2f(f2h_after_f32(o.y * inv));
            orot[hh][d4 + 2] = h2f(f2h_after_f32(o.z * inv));
            orot[hh][d4 + 3] = h2f(f2h_after_f32(o.w * inv));
        }
        if (HPB == 1 && half == 0)
            *reinterpret_cast<float4 *>(&orot[wsub][d4]) = make_float4(o.x, o.y, o.z, o.w);
    }
    __syncthreads();
    if (!live || wsub != 0) return;
    if (HPB == 1) {
        // Wave 0: add the four waves' partial sums (fixed order), normalise,
        // round O_rot to fp16.
        const float inv = 1.0f / fmaxf(L, 1e-30f);
        const float s0 = ((orot[0][lane] + orot[1][lane]) + orot[2][lane]) + orot[3][lane];
        const float s1 = ((orot[0][lane + 64] + orot[1][lane + 64]) + orot[2][lane + 64]) +
                         orot[3][lane + 64];
        // Every lane has read all four rows before row 0 is overwritten.
        __builtin_amdgcn_wave_barrier();
        orot[0][lane] = h2f(f2h_after_f32(s0 * inv));
        orot[0][lane + 64] = h2f(f2h_after_f32(s1 * inv));
        __builtin_amdgcn_wave_barrier();
    }
    const float *r0 = Rs + lane * kRPad;
    const float *r1 = Rs + (lane + 64) * kRPad;
    float a0 = 0.0f, a1 = 0.0f;
#pragma unroll 8
    for (int k = 0; k < kD; k += 4) {
        const float4 o = *reinterpret_cast<const float4 *>(&orot[hh][k]);
        const float4 x = *reinterpret_cast<const float4 *>(r0 + k);
        const float4 y = *reinterpret_cast<const float4 *>(r1 + k);
        a0 = fmaf(o.x, x.x, a0);
        a0 = fmaf(o.y, x.y, a0);
        a0 = fmaf(o.z, x.z, a0);
        a0 = fmaf(o.w, x.w, a0);
        a1 = fmaf(o.x, y.x, a1);
        a1 = fmaf(o.y, y.y, a1);
        a1 = fmaf(o.z, y.z, a1);
        a1 = fmaf(o.w, y.w, a1);
    }
    const int64_t row = ((int64_t)b * H_q + h) * kD;
    out[row + lane] = f2h_after_f32(a0);
    out[row + lane + 64] = f2h_after_f32(a1);
}

struct WsLayout {
    size_t q_rot, part_o, part_ml, flag, total;
};

// Plan of the single-launch form: workgroups of one KV head over
// 8 * wave_tokens tokens (each wave at least one 64-token chunk), about one
// workgroup per CU over all sequences and heads, at most 4096 pages (64K
// tokens) per workgroup.  Never more splits than cda_decode_plan's, so its
// partials fit the same workspace.
void fused_plan(int B, int H_kv, int max_seq_len, int *wave_tokens, int *n_splits);

WsLayout ws_layout(int B, int H_q, int n_splits) {
    WsLayout w;
    size_t off = 0;
    w.q_rot = off;
    off += align256((size_t)B * H_q * kD * 2);
    w.part_o = off;
    off += align256((size_t)B * n_splits * H_q * kD * 4);
    w.part_ml = off;
    off += align256((size_t)B * n_splits * H_q * 2 * 4);
    w.flag = off;
    off += 256;
    w.total = off;
    return w;
}

// Optional profiling events recorded around the split kernel (per thread).
thread_local hipEvent_t g_split_start = nullptr;
thread_local hipEvent_t g_split_stop = nullptr;
// Lets tests run the general kernel on shapes the streaming kernel also covers.
// (Process-wide switches; atomics, since another thread may set them while a
// call reads them.)
std::atomic<bool> g_allow_stream{true};
// Lets tests and benchmarks run the three-launch form where the single-launch
// form also applies.
std::atomic<bool> g_allow_fused{true};

int num_cus() {
    static int cached = 0;
    if (!cached) {
        int dev = 0, n = 0;
        if (hipGetDevice(&dev) == hipSuccess &&
            hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess &&
            n > 0)
            cached = n;
        else
            cached = 256;
    }
    return cached;
}

void fused_plan(int B, int H_kv, int max_seq_len, int *wave_tokens, int *n_splits) {
    const int n = max_seq_len > 0 ? max_seq_len : 1;
    const int units = B * H_kv;
    int s = (num_cus() + units - 1) / units;
    const int max_by_len = (n + 8 * kStreamPages * 16 - 1) / (8 * kStreamPages * 16);
    if (s > max_by_len) s = max_by_len;
    const int min_by_len = (n + 16 * kFusedMaxPages - 1) / (16 * kFusedMaxPages);
    if (s < min_by_len) s = min_by_len;
    if (s < 1) s = 1;
    int wg = (n + s - 1) / s;
    wg = (wg + 511) / 512 * 512;
    *wave_tokens = wg / kWaves;
    *n_splits = (n + wg - 1) / wg;
}

}  // namespace

}  // namespace cda

using namespace cda;

extern "C" int cda_decode_plan(int B, int H_q, int H_kv, int max_seq_len, int tile_n,
                               int *tile_n_out, int *n_splits_out) {
    (void)H_q;
    if (B <= 0 || H_kv <= 0 || max_seq_len < 0)
        return fail(CDA_E_INVALID, "cda_decode_plan: B, H_kv must be > 0 and max_seq_len >= 0");
    const int n = max_seq_len > 0 ? max_seq_len : 1;
    int tn;
    if (tile_n > 0) {
        tn = (tile_n + kChunk - 1) / kChunk * kChunk;
    } else {
        // One workgroup per CU (the split kernels hold one per CU: their LDS
        // tables are 128-143 KiB), so every split runs in a single round and
        // the per-workgroup set-up is paid once per CU; splits of at least 64
        // tokens, at most 16384 (the streaming kernel's page-row table) and at
        // most 512 per sequence.  Measured at B=32, N=64K: 8 splits 527 us,
        // 16: 530, 32: 545, 64: 578.
        const int hg = (H_kv + kWaves - 1) / kWaves;
        const int target = num_cus();
        int splits = (target + B * hg - 1) / (B * hg);
        const int max_by_len = (n + 63) / 64;
        if (splits > max_by_len) splits = max_by_len;
        const int min_by_len = (n + 16 * kStreamMaxPages - 1) / (16 * kStreamMaxPages);
        if (splits < min_by_len) splits = min_by_len;
        if (splits > 512) splits = 512;
        if (splits < 1) splits = 1;
        tn = (n + splits - 1) / splits;
        tn = (tn + kChunk - 1) / kChunk * kChunk;
    }
    if (tile_n_out) *tile_n_out = tn;
    if (n_splits_out) *n_splits_out = (n + tn - 1) / tn;
    return CDA_OK;
}

extern "C" int cda_decode_fused_plan(int B, int H_kv, int max_seq_len, int *wave_tokens_out,
                                     int *n_splits_out) {
    if (B <= 0 || H_kv <= 0 || max_seq_len < 0)
        return fail(CDA_E_INVALID, "cda_decode_fused_plan: B, H_kv must be > 0 and max_seq_len >= 0");
    int wt = 0, ns = 0;
    fused_plan(B, H_kv, max_seq_len, &wt, &ns);
    if (wave_tokens_out) *wave_tokens_out = wt;
    if (n_splits_out) *n_splits_out = ns;
    return CDA_OK;
}

extern "C" size_t cda_decode_workspace_size(int B, int H_q, int H_kv, int max_seq_len,
                                            int tile_n) {
    int tn = 0, ns = 0;
    if (cda_decode_plan(B, H_q, H_kv, max_seq_len, tile_n, &tn, &ns) != CDA_OK) return 0;
    return ws_layout(B, H_q, ns).total;
}

namespace cda {
namespace {
// Shared body of the decode entry points.  levels_k / levels_v: 16/16 (K4V4),
// 4/4 (K2V2) or 16/4 (the legacy K4V2 104-byte slot).
int decode_impl(const void *q, const void *kv_cache, int slot_bytes, int H_kv,
                const int32_t *block_table, int bt_stride, const int32_t *seq_lens,
                const float *cb_k, const float *cb_v, int levels_k, int levels_v,
                const float *rot_f32, void *out, int B, int H_q, int group_size, int block_size,
                int tile_n, int max_seq_len, float scale, void *workspace,
                size_t workspace_bytes, void *stream, const char *fn,
                bool uniform_qk = false) {
    const std::string f(fn);
    CDA_REQUIRE(q && kv_cache && block_table && seq_lens && cb_k && cb_v && rot_f32 && out,
                f + ": null pointer argument");
    CDA_REQUIRE(B > 0 && H_kv > 0 && H_q > 0, f + ": B, H_q, H_kv must be > 0");
    CDA_REQUIRE(group_size == 4 || group_size == 8, f + ": group_size must be 4 or 8");
    CDA_REQUIRE(H_q == H_kv * group_size, f + ": H_q must equal H_kv * group_size");
    const int kbk = (levels_k == 16) ? kD / 2 : kD / 4;
    const int kbv = (levels_v == 16) ? kD / 2 : kD / 4;
    const int align = (levels_k == levels_v) ? 16 : 8;
    CDA_REQUIRE(slot_bytes >= kbk + kbv + 8 && slot_bytes % align == 0,
                f + ": slot_bytes must hold both code fields and the two norms (>= 136 for "
                    "K4V4, >= 72 for K2V2, a multiple of 16; >= 104 and a multiple of 8 for "
                    "K4V2)");
    CDA_REQUIRE(block_size > 0 && block_size % 16 == 0,
                f + ": block_size must be a positive multiple of 16");
    CDA_REQUIRE(max_seq_len >= 0 && bt_stride > 0, f + ": bad max_seq_len / block-table stride");
    CDA_REQUIRE((int64_t)16 * H_kv * slot_bytes < (int64_t)1 << 31, f + ": cache row too wide");
    CDA_REQUIRE(((uintptr_t)kv_cache & 15) == 0 && ((uintptr_t)q & 15) == 0,
                f + ": q and kv_cache must be 16-byte aligned");
    int tn = 0, ns = 0;
    int rc = cda_decode_plan(B, H_q, H_kv, max_seq_len, tile_n, &tn, &ns);
    if (rc) return rc;
    CDA_REQUIRE(ns <= kMaxSplits, f + ": tile_n gives more than 1024 context splits; use a "
                                      "larger tile_n");
    const WsLayout w = ws_layout(B, H_q, ns);
    if (!workspace || workspace_bytes < w.total || ((uintptr_t)workspace & 255))
        return fail(CDA_E_WORKSPACE, f + ": workspace missing, misaligned or smaller than "
                                         "cda_decode_workspace_size()");
    char *ws = static_cast<char *>(workspace);
    hipStream_t st = static_cast<hipStream_t>(stream);

    uint16_t *q_rot = reinterpret_cast<uint16_t *>(ws + w.q_rot);
    const dim3 head_grid((H_q + kHeadsPerBlock - 1) / kHeadsPerBlock, B);
    // The page-streaming kernel covers 8 KV heads x 144-byte (K4V4) or
    // 80-byte (K2V2) slots with one codebook for K and V, and splits of at
    // most 1024 pages.  With one codebook pointer it runs alone; with two, the
    // rotation kernel compares them on the device and both split kernels are
    // launched, each returning at once unless the comparison picks it (no
    // host round trip, so the choice is the same inside graph capture).
    const bool stream_shape = H_kv == 8 && levels_k == levels_v &&
                              ((levels_k == 16 && slot_bytes == 144) ||
                               (levels_k == 4 && slot_bytes == 80)) &&
                              tn <= 16 * kStreamMaxPages &&
                              g_allow_stream.load(std::memory_order_relaxed);
    if (uniform_qk)
        CDA_REQUIRE(stream_shape && levels_k == 16,
                    f + ": the score-domain QK runs on the page-streaming kernel: K4V4 "
                        "144-byte slots, 8 KV heads, splits of at most 16384 tokens");
    // Single launch: one workgroup per (sequence, split, KV head) rotates q,
    // streams, merges its waves and (one split per sequence) writes out; more
    // splits add the combine launch.  Taken with one codebook pointer and the
    // library's split plan (tile_n 0, or the plan's own tile_n, which the
    // reference-shaped wrapper passes).
    int plan_tn = 0;
    cda_decode_plan(B, H_q, H_kv, max_seq_len, 0, &plan_tn, nullptr);
    int wave_tokens = 0, nsf = 0;
    fused_plan(B, H_kv, max_seq_len, &wave_tokens, &nsf);
    const WsLayout wf = ws_layout(B, H_q, nsf);
    // The single-launch plan never has more splits than the three-launch one
    // (tests pin this over a sweep of shapes); were it to, the three launches
    // below run instead of failing the call.
    if (stream_shape && !uniform_qk && cb_k == cb_v && (tile_n == 0 || tile_n == plan_tn) &&
        g_allow_fused.load(std::memory_order_relaxed) && nsf <= ns && wf.total <= w.total) {
        SplitParams p{};
        p.q_rot = nullptr;
        p.kv = static_cast<const uint8_t *>(kv_cache);
        p.block_table = block_table;
        p.seq_lens = seq_lens;
        p.cb_k = cb_k;
        p.cb_v = cb_v;
        p.part_o = reinterpret_cast<float *>(ws + wf.part_o);
        p.part_ml = reinterpret_cast<float *>(ws + wf.part_ml);
        p.row_bytes = (int64_t)H_kv * slot_bytes;
        p.bt_stride = bt_stride;
        p.H_q = H_q;
        p.H_kv = H_kv;
        p.slot_bytes = slot_bytes;
        p.block_size = block_size;
        p.tile_n = kWaves * wave_tokens;
        p.n_splits = nsf;
        p.scale_log2 = scale * kLog2e;
        p.levels = levels_k;
        p.q = static_cast<const uint16_t *>(q);
        p.R = rot_f32;
        p.out = static_cast<uint16_t *>(out);
        p.wave_tokens = wave_tokens;
        const int units = B * nsf;
        p.xcd_map = (units % 8 == 0) ? 1 : 0;
        const dim3 grid(units * H_kv);
        if (g_split_start && hipEventRecord(g_split_start, st) != hipSuccess)
            return fail(CDA_E_HIP, f + ": hipEventRecord(start) failed");
        if (levels_k == 16) {
            if (group_size == 4)
                decode_stream_kernel<4, 16, false, true><<<grid, kThreads, 0, st>>>(p);
            else
                decode_stream_kernel<8, 16, false, true><<<grid, kThreads, 0, st>>>(p);
        } else {
            if (group_size == 4)
                decode_stream_kernel<4, 4, false, true><<<grid, kThreads, 0, st>>>(p);
            else
                decode_stream_kernel<8, 4, false, true><<<grid, kThreads, 0, st>>>(p);
        }
        CDA_LAUNCH_CHECK("decode_stream_kernel");
        if (g_split_stop && hipEventRecord(g_split_stop, st) != hipSuccess)
            return fail(CDA_E_HIP, f + ": hipEventRecord(stop) failed");
        if (nsf > 1) {
            if ((int64_t)head_grid.x * B < num_cus())
                combine_kernel<1><<<dim3(H_q, B), 256, 0, st>>>(p.part_o, p.part_ml, rot_f32,
                                                                p.out, H_q, nsf);
            else
                combine_kernel<4><<<head_grid, 256, 0, st>>>(p.part_o, p.part_ml, rot_f32,
                                                             p.out, H_q, nsf);
            CDA_LAUNCH_CHECK("combine_kernel");
        }
        return CDA_OK;
    }
    const bool dual = stream_shape && cb_k != cb_v && !uniform_qk;
    int *cb_same = dual ? reinterpret_cast<int *>(ws + w.flag) : nullptr;
    int *k_uniform = uniform_qk ? reinterpret_cast<int *>(ws + w.flag) + 1 : nullptr;
    rotate_q_kernel<<<head_grid, 256, 0, st>>>(static_cast<const uint16_t *>(q), rot_f32, q_rot,
                                               H_q, cb_k, cb_v, levels_k, cb_same, k_uniform);
    CDA_LAUNCH_CHECK("rotate_q_kernel");

    SplitParams p;
    p.q_rot = q_rot;
    p.kv = static_cast<const uint8_t *>(kv_cache);
    p.block_table = block_table;
    p.seq_lens = seq_lens;
    p.cb_k = cb_k;
    p.cb_v = cb_v;
    p.part_o = reinterpret_cast<float *>(ws + w.part_o);
    p.part_ml = reinterpret_cast<float *>(ws + w.part_ml);
    p.row_bytes = (int64_t)H_kv * slot_bytes;
    p.bt_stride = bt_stride;
    p.H_q = H_q;
    p.H_kv = H_kv;
    p.slot_bytes = slot_bytes;
    p.block_size = block_size;
    p.tile_n = tn;
    p.n_splits = ns;
    p.scale_log2 = scale * kLog2e;
    p.levels = levels_k;
    p.cb_same = cb_same;
    p.k_uniform = k_uniform;
    dim3 grid(ns, (H_kv + kWaves - 1) / kWaves, B);
    const bool use_stream = stream_shape;
    if (g_split_start && hipEventRecord(g_split_start, st) != hipSuccess)
        return fail(CDA_E_HIP, f + ": hipEventRecord(start) failed");
    if (uniform_qk) {
        if (group_size == 4)
            decode_stream_kernel<4, 16, true><<<grid, kThreads, 0, st>>>(p);
        else
            decode_stream_kernel<8, 16, true><<<grid, kThreads, 0, st>>>(p);
    } else if (use_stream) {
        if (levels_k == 16) {
            if (group_size == 4)
                decode_stream_kernel<4, 16><<<grid, kThreads, 0, st>>>(p);
            else
                decode_stream_kernel<8, 16><<<grid, kThreads, 0, st>>>(p);
        } else {
            if (group_size == 4)
                decode_stream_kernel<4, 4><<<grid, kThreads, 0, st>>>(p);
            else
                decode_stream_kernel<8, 4><<<grid, kThreads, 0, st>>>(p);
        }
    }
    if (!uniform_qk && (!use_stream || dual)) {
        if (levels_k == 4) {
            if (group_size == 4)
                decode_split_kernel<4, 4, 4><<<grid, kThreads, 0, st>>>(p);
            else
                decode_split_kernel<8, 4, 4><<<grid, kThreads, 0, st>>>(p);
        } else if (levels_v == 4) {
            if (group_size == 4)
                decode_split_kernel<4, 16, 4><<<grid, kThreads, 0, st>>>(p);
            else
                decode_split_kernel<8, 16, 4><<<grid, kThreads, 0, st>>>(p);
        } else if (group_size == 4) {
            decode_split_kernel<4, 16, 16><<<grid, kThreads, 0, st>>>(p);
        } else {
            decode_split_kernel<8, 16, 16><<<grid, kThreads, 0, st>>>(p);
        }
    }
    CDA_LAUNCH_CHECK("decode_split_kernel");
    if (g_split_stop && hipEventRecord(g_split_stop, st) != hipSuccess)
        return fail(CDA_E_HIP, f + ": hipEventRecord(stop) failed");

    // One head per block when four per block would leave CUs idle.
    if ((int64_t)head_grid.x * B < num_cus())
        combine_kernel<1><<<dim3(H_q, B), 256, 0, st>>>(p.part_o, p.part_ml, rot_f32,
                                                        static_cast<uint16_t *>(out), H_q, ns);
    else
        combine_kernel<4><<<head_grid, 256, 0, st>>>(p.part_o, p.part_ml, rot_f32,
                                                     static_cast<uint16_t *>(out), H_q, ns);
    CDA_LAUNCH_CHECK("combine_kernel");
    return CDA_OK;
}
}  // namespace
}  // namespace cda

extern "C" int cda_decode_full_hmma_v3(const void *q, const void *kv_cache, int64_t num_slots,
                                       int slot_bytes, int H_kv, const int32_t *block_table,
                                       int bt_stride, const int32_t *seq_lens, const float *cb_k,
                                       const float *cb_v, int levels, const float *rot_f32,
                                       const void *rot_f16, void *out, int B, int H_q,
                                       int group_size, int block_size, int tile_n,
                                       int max_seq_len, float scale, void *workspace,
                                       size_t workspace_bytes, void *stream) {
    (void)rot_f16;
    (void)num_slots;
    CDA_REQUIRE(levels == 16 || levels == 4,
                "cda_decode_full_hmma_v3: codebooks must have 16 levels (K4V4) or 4 (K2V2)");
    return decode_impl(q, kv_cache, slot_bytes, H_kv, block_table, bt_stride, seq_lens, cb_k,
                       cb_v, levels, levels, rot_f32, out, B, H_q, group_size, block_size, tile_n,
                       max_seq_len, scale, workspace, workspace_bytes, stream,
                       "cda_decode_full_hmma_v3");
}

extern "C" int cda_decode_full_hmma_v3_uniform_qk(
    const void *q, const void *kv_cache, int64_t num_slots, int slot_bytes, int H_kv,
    const int32_t *block_table, int bt_stride, const int32_t *seq_lens, const float *cb_k,
    const float *cb_v, const float *rot_f32, void *out, int B, int H_q, int group_size,
    int block_size, int tile_n, int max_seq_len, float scale, void *workspace,
    size_t workspace_bytes, void *stream) {
    (void)num_slots;
    return decode_impl(q, kv_cache, slot_bytes, H_kv, block_table, bt_stride, seq_lens, cb_k,
                       cb_v, 16, 16, rot_f32, out, B, H_q, group_size, block_size, tile_n,
                       max_seq_len, scale, workspace, workspace_bytes, stream,
                       "cda_decode_full_hmma_v3_uniform_qk", true);
}

extern "C" int cda_decode_full_hmma_v3_k4v2(const void *q, const void *kv_cache,
                                            int64_t num_slots, int slot_bytes, int H_kv,
                                            const int32_t *block_table, int bt_stride,
                                            const int32_t *seq_lens, const float *cb_k,
                                            const float *cb_v, const float *rot_f32,
                                            const void *rot_f16, void *out, int B, int H_q,
                                            int group_size, int block_size, int tile_n,
                                            int max_seq_len, float scale, void *workspace,
                                            size_t workspace_bytes, void *stream) {
    (void)rot_f16;
    (void)num_slots;
    return decode_impl(q, kv_cache, slot_bytes, H_kv, block_table, bt_stride, seq_lens, cb_k,
                       cb_v, 16, 4, rot_f32, out, B, H_q, group_size, block_size, tile_n,
                       max_seq_len, scale, workspace, workspace_bytes, stream,
                       "cda_decode_full_hmma_v3_k4v2");
}

extern "C" int cda_decode_set_timing_events(void *start_event, void *stop_event) {
    CDA_REQUIRE((start_event == nullptr) == (stop_event == nullptr),
                "cda_decode_set_timing_events: pass both events or neither");
    g_split_start = static_cast<hipEvent_t>(start_event);
    g_split_stop = static_cast<hipEvent_t>(stop_event);
    return CDA_OK;
}

extern "C" int cda_decode_set_stream_kernel(int enable) {
    g_allow_stream.store(enable != 0, std::memory_order_relaxed);
    return CDA_OK;
}

extern "C" int cda_decode_set_fused_kernel(int enable) {
    g_allow_fused.store(enable != 0, std::memory_order_relaxed);
    return CDA_OK;
}

// ------------------------------------------------- allocation-free decode --
//
// cda_decode_full_hmma_v3_noalloc: the same decode with the split-K workspace
// taken from a fixed device array of this library instead of the caller, for
// callers that cannot allocate (code under graph capture that must not call
// hipMalloc, tight serving loops, harnesses that forbid allocation).  Every
// GPU the library runs on holds its own copy of the array until the process
// ends; every call on one GPU shares it, so calls that overlap on one GPU
// (two streams, or two threads) race on it.  Nothing in it needs to start at
// zero: the kernels write q_rot and every split's partials before the
// combine reads them.

namespace cda {
namespace {

constexpr size_t kDecodeScratchBytes = size_t(16) << 20;   // 16 MiB per GPU
__device__ __align__(256) char scratch[kDecodeScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void *g_scratch_ptr[kMaxDevices] = {};

// Device address of `scratch` on the current device (looked up once per
// device, with that device current).
int decode_scratch(void **ptr) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices)
        return fail(CDA_E_HIP, "cda_decode_full_hmma_v3_noalloc: no current HIP device");
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void *p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p)
            return fail(CDA_E_HIP, std::string("cda_decode_full_hmma_v3_noalloc: "
                                               "hipGetSymbolAddress(scratch): ") +
                                       hipGetErrorString(e));
        g_scratch_ptr[dev] = p;
    }
    *ptr = g_scratch_ptr[dev];
    return CDA_OK;
}

}  // namespace
}  // namespace cda

extern "C" size_t cda_decode_noalloc_max_workspace(void) { return cda::kDecodeScratchBytes; }

extern "C" int cda_decode_full_hmma_v3_noalloc(const void *q, const void *kv_cache,
                                               int64_t num_slots, int slot_bytes, int H_kv,
                                               const int32_t *block_table, int bt_stride,
                                               const int32_t *seq_lens, const float *cb_k,
                                               const float *cb_v, int levels,
                                               const float *rot_f32, const void *rot_f16,
                                               void *out, int B, int H_q, int group_size,
                                               int block_size, int tile_n, int max_seq_len,
                                               float scale, void *stream) {
    CDA_REQUIRE(B > 0 && H_kv > 0 && H_q > 0 && max_seq_len >= 0,
                "cda_decode_full_hmma_v3_noalloc: B, H_q, H_kv must be > 0, max_seq_len >= 0");
    const size_t need = cda_decode_workspace_size(B, H_q, H_kv, max_seq_len, tile_n);
    CDA_REQUIRE(need > 0, "cda_decode_full_hmma_v3_noalloc: bad shape or tile_n");
    if (need > kDecodeScratchBytes)
        return fail(CDA_E_WORKSPACE,
                    "cda_decode_full_hmma_v3_noalloc: this shape needs " + std::to_string(need) +
                        " bytes of split-K scratch, more than the fixed " +
                        std::to_string(kDecodeScratchBytes) +
                        "; use cda_decode_full_hmma_v3 with a caller workspace");
    void *ws = nullptr;
    const int rc = decode_scratch(&ws);
    if (rc) return rc;
    return cda_decode_full_hmma_v3(q, kv_cache, num_slots, slot_bytes, H_kv, block_table,
                                   bt_stride, seq_lens, cb_k, cb_v, levels, rot_f32, rot_f16,
                                   out, B, H_q, group_size, block_size, tile_n, max_seq_len,
                                   scale, ws, kDecodeScratchBytes, stream);
}
