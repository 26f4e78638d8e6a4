// Varlen causal prefill for CDA (gfx950): flash attention whose K/V tiles are
// materialised in LDS, with the Hadamard-128 rotation of Q as a prologue and
// the inverse rotation of O as an epilogue, both on MFMA.
//
// Reference contract: fa2_cda_prefill_varlen_v1 (cda/kernels_cuda/fa2_cda.py:
// 98-230) with fuse_fa2_epilogue=True: Q is unrotated fp16, the cache holds
// Hadamard-rotated codes, the mask is causal with bottom-right alignment
// (k <= q + seq_k - seq_q per sequence), O_rot is rounded to fp16 before the
// inverse rotation (attention.py:93, :482) and the output is unrotated fp16.
// Math per (query, head): attention_reference (attention.py:60-93) on K and V
// decoded as fp16(centroid * norm) (compression.py:355-359).
//
// Two K/V sources share the kernel:
//   * Paged: the compressed K4V4 cache; each 64-token tile is dequantised by
//     the whole workgroup straight into LDS (no dense scratch in HBM).
//   * Dense: fp16 rotated K/V rows (the reference's cda_fa2_varlen_fwd_hadamard
//     over the output of paged_cache_to_dense_rotated).
//
// Workgroup = 8 waves = the GQA group of one KV head x 32*(8/GS) queries: wave
// w takes q-head h*GS + w % GS and 32 queries.  Per wave all products are
// 32x32x16 f16 MFMAs laid out so that no lane ever exchanges data:
//   q_rot^T = H q^T           (prologue; result columns = queries)
//   S^T     = K q_rot^T       (rows = 32 keys, columns = the wave's queries)
//   O^T    += V^T P^T         (P^T taken straight from the S^T accumulators)
//   out^T   = H fp16(O^T / l) (epilogue)
// The k index of each product is permuted to match the accumulator rows it is
// fed from; the other operand (H, an LDS tile) is read in the same order.
#include "cda_common.h"

#include <cmath>
#include <type_traits>

namespace cda {
namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half2 __attribute__((ext_vector_type(2)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int kD = 128;
constexpr int kBN = 64;                  // keys per tile
constexpr int kWaves = 8;
constexpr int kThreads = 64 * kWaves;
constexpr uint32_t kXcds = 8;            // MI355X: 8 XCDs, each with its own L2
constexpr float kLog2e = 1.4426950408889634f;

// LDS: two tile buffers, then the code-byte dequant tables (paged source).
//   K tile   [64 keys][128 dims] fp16, natural dim order, rows padded to 272 B.
//   V^T tile [128 dims][64 keys] fp16, rows padded to 144 B; within each
//            16-key group the keys are stored in the MFMA k order (key
//            8*jh + 4*u + jl at position 8*u + 4*jh + jl), so each MFMA
//            operand is one 16-byte read.
// The padding puts the 16 lanes of every 16-byte read (consecutive rows) in
// distinct banks, and every address is a per-lane base plus a compile-time
// offset.
constexpr int kKRow = kD * 2 + 16;                     // 272
constexpr int kVRow = kBN * 2 + 16;                    // 144
constexpr int kKTile = kBN * kKRow;                    // 17408
constexpr int kTileBytes = kKTile + kD * kVRow;         // + 18432
constexpr int kLutOff = 2 * kTileBytes;
// Code-byte tables for K and V: entry x = (cb[x >> 4], cb[x & 15]) in fp32,
// so one 8-byte read yields both values of a code byte (one copy: 1, 2 and 4
// interleaved copies measured the same).
constexpr int kLutEntry = 8;                           // bytes per code byte
constexpr int kLutBytes = 2 * 256 * kLutEntry;         // 4 KiB
// The q_rot operands stay in registers (8 x 16 bytes per lane): reading them
// from LDS every tile cost 2-3 % (dense / compressed kernel, config 3).
constexpr int kPrefillLds = kLutOff + kLutBytes;

// Dense source: the K tile is copied into LDS by the direct-to-LDS DMA, 256-
// byte rows (no pad) with the 16-byte chunks of row k permuted: chunk c of key
// k sits at chunk position c ^ (k & 15).  One DMA instruction moves four keys
// (64 lanes x 16 bytes); the lane writing position p of key k reads global
// chunk p ^ (k & 15), and the 16 lanes of an MFMA operand read (rows c32,
// chunk 2S + u) then fall in 16 distinct bank groups.
constexpr int kKRowDense = kD * 2;                      // 256

typedef unsigned v4u32 __attribute__((ext_vector_type(4)));

// One 16-byte-per-lane direct-to-LDS load: lane l's 16 bytes at rsrc+voff go
// to LDS address lds_base + 16*l.  Issued through asm so the compiler does not
// track these asynchronous LDS writes; completion is ordered by explicit vmcnt
// waits.  M0 (the LDS base operand) is saved and restored around the load.
__device__ __forceinline__ void dma_x4_to_lds(v4u32 rsrc, uint32_t voff, uint32_t lds_base) {
    uint32_t saved;
    asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %3\n\t"
                 "buffer_load_dwordx4 %1, %2, 0 offen lds\n\ts_mov_b32 m0, %0"
                 : "=&s"(saved) : "v"(voff), "s"(rsrc), "s"(lds_base) : "memory");
}

__device__ __forceinline__ uint32_t lds_addr32(const void *ptr) {
    return (uint32_t)(size_t)(const __attribute__((address_space(3))) void *)ptr;
}

__device__ __forceinline__ floatx16 mfma32(half8 a, half8 b, floatx16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ uint32_t cvt_pk(float a, float b) {
    typedef float f2 __attribute__((ext_vector_type(2)));
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f2{a, b}, h2));
}

// max of three floats (v_maximum3_f32), compiler-visible so that reads of
// MFMA results before it get their hazard waits.
__device__ __forceinline__ float max3f(float a, float b, float c) {
    return __builtin_elementwise_maximum(__builtin_elementwise_maximum(a, b), c);
}

__device__ __forceinline__ half8 pack8(const floatx16 &c, int base) {
    const uint4 v = make_uint4(cvt_pk(c[base + 0], c[base + 1]), cvt_pk(c[base + 2], c[base + 3]),
                               cvt_pk(c[base + 4], c[base + 5]), cvt_pk(c[base + 6], c[base + 7]));
    return __builtin_bit_cast(half8, v);
}

// Thread -> V share: dims [4cv, 4cv+4) of keys [4gv, 4gv+4).  Each 32-lane
// half of a wave covers 4 cv x 8 gv, so its 8-byte V^T writes land in 32
// distinct bank pairs.
__device__ __forceinline__ int v_cv(int tid) { return (((tid >> 5) & 7) << 2) | ((tid >> 3) & 3); }
__device__ __forceinline__ int v_gv(int tid) { return ((tid >> 8) << 3) | (tid & 7); }
// Byte offset of keys 4gv..4gv+3 (8 bytes) in a V^T row.
__device__ __forceinline__ uint32_t v_key_off(int gv) {
    return (uint32_t)(32 * (gv >> 2) + 16 * (gv & 1) + 8 * ((gv >> 1) & 1));
}

// A operand of a product with the unnormalised Hadamard matrix,
// A[r][k] = (-1)^popcount(k & r) for r = 32*T + c32 and k = 16*S + 8*u + e:
// the e part depends on the lane only (hbase), the rest flips all eight signs.
__device__ __forceinline__ half8 hadamard_operand(uint4 hbase, int S, int u, int T, int c32) {
    const uint32_t f = (__builtin_popcount((16 * S + 8 * u) & (32 * T + c32)) & 1) ? 0x80008000u : 0u;
    return __builtin_bit_cast(half8, make_uint4(hbase.x ^ f, hbase.y ^ f, hbase.z ^ f, hbase.w ^ f));
}

// The identity in the same operand layout (row 32T + c32, k = 16S + 8u + e):
// the prologue and epilogue then copy q and O exactly (one product each).
__device__ __forceinline__ half8 identity_operand(int S, int u, int T, int c32) {
    const int e = 32 * T + c32 - 16 * S - 8 * u;
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
        w[i] = (e == 2 * i ? 0x3C00u : 0u) | (e == 2 * i + 1 ? 0x3C000000u : 0u);
    return __builtin_bit_cast(half8, make_uint4(w[0], w[1], w[2], w[3]));
}

__device__ __forceinline__ uint4 hadamard_base(int c32) {
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t lo = (__builtin_popcount((2 * i) & c32 & 7) & 1) ? 0xBC00u : 0x3C00u;
        const uint32_t hi = (__builtin_popcount((2 * i + 1) & c32 & 7) & 1) ? 0xBC00u : 0x3C00u;
        w[i] = lo | (hi << 16);
    }
    return make_uint4(w[0], w[1], w[2], w[3]);
}

// B operand (natural k: values 16*S + 8*u + 0..7) of tile T's k-step S = 2T + s
// from a 32x32 accumulator whose rows carry those values in MFMA row order
// (row 8*g + 4*u + i in register 4*g + i of lane half u): lane half u keeps
// its own group 2s+u and takes the partner half's, scaled by `scale`.
__device__ __forceinline__ half8 acc_to_operand(const floatx16 &c, int s, int u, float scale) {
    const int g0 = 2 * s, g1 = 2 * s + 1;
    const uint32_t m0 = cvt_pk(c[4 * g0 + 0] * scale, c[4 * g0 + 1] * scale);
    const uint32_t m1 = cvt_pk(c[4 * g0 + 2] * scale, c[4 * g0 + 3] * scale);
    const uint32_t n0 = cvt_pk(c[4 * g1 + 0] * scale, c[4 * g1 + 1] * scale);
    const uint32_t n1 = cvt_pk(c[4 * g1 + 2] * scale, c[4 * g1 + 3] * scale);
    const uint32_t own0 = u ? n0 : m0, own1 = u ? n1 : m1;     // group 2s+u
    const uint32_t snd0 = u ? m0 : n0, snd1 = u ? m1 : n1;     // what the partner needs
    const uint32_t rcv0 = __shfl_xor(snd0, 32), rcv1 = __shfl_xor(snd1, 32);
    const uint4 v = u ? make_uint4(rcv0, rcv1, own0, own1) : make_uint4(own0, own1, rcv0, rcv1);
    return __builtin_bit_cast(half8, v);
}

struct PrefillParams {
    const uint16_t *q;          // (T, H_q, 128) fp16, unrotated
    uint16_t *out;              // (T, H_q, 128) fp16
    const int32_t *cu_q;        // (B+1,)
    const int32_t *seq_k;       // (B,) key length per sequence
    int H_q, H_kv, GS;
    float scale_log2;           // softmax scale * log2(e)
    // paged source
    const uint8_t *kv;
    const int32_t *block_table;
    int bt_stride, block_size, slot_bytes;
    int bs_shift;               // log2(block_size) when it is a power of two, else -1
    int64_t row_bytes;
    const float *cb_k, *cb_v;
    // dense source
    const uint16_t *k_rot, *v_rot;
    const int32_t *cu_k;        // (B+1,) first dense row of each sequence
    // key split (n_ksplit > 1): split ks of a query block takes key tiles
    // [ks * ksplit_tiles, +ksplit_tiles) and writes unnormalised partials
    // (rotated frame) instead of out; prefill_combine_kernel merges them.
    int n_ksplit;               // 1 = no split
    int ksplit_tiles;
    int T_total;                // rows of q / out
    int rotate;                 // 1: q and out unrotated (Hadamard prologue/epilogue);
                                // 0: q and out already in the rotated frame
    int causal;                 // 1: bottom-right causal mask; 0: every key visible
    // Keys of sequence b: kKeysAll = [0, seq_k[b]); kKeysPast = the first
    // seq_k[b] - (its query count) of them (the prefix before the queries);
    // kKeysChunk = as many keys as queries (the query chunk's own keys).
    int key_range;
    int ks_base;                // partial slot of split 0 (several sources merged)
    float *part_o;              // (slots, T, H_q, 128) fp32
    float *part_ml;             // (slots, T, H_q, 2): m (log2 domain), l
    // Unsplit kernel only: when set, slot 0 of part_o / part_ml holds a
    // partial over other keys of the same queries (written by an earlier
    // launch), merged in before the epilogue (attention.py:239-272).
    int merge_slot0;
    // Unsplit kernel only: when set, lse[hq * T_total + t] = the natural-log
    // sum of exp(scale * q.k) over query t's visible keys (FlashAttention-2's
    // varlen softmax_lse layout), +inf for a query with no visible key.
    float *lse;
};
constexpr int kKeysAll = 0, kKeysPast = 1, kKeysChunk = 2;

// Registers holding one tile's share of the source data for this thread:
// paged: K codes k[0..1] + nk, V codes v[0..3] (two bytes per key) + nv[];
// dense: K fp16 k[0..7], V fp16 v[2i], v[2i+1] for key i.
struct TileRegs {
    uint32_t k[8];
    uint32_t v[8];
    float nk;
    float nv[4];
};

// Block-table entries of one tile's rows for this thread (paged source): the
// K row (key tk) and the V rows (keys 4gv..4gv+3, one 16-key block).  They
// are fetched one tile ahead of the row loads that use them, so no load
// waits on a block-table load.
struct TileRows {
    int32_t bk, bv;
};

__device__ __forceinline__ int block_of(const PrefillParams &p, int kpos) {
    return p.bs_shift >= 0 ? (kpos >> p.bs_shift) : (kpos / p.block_size);
}

template <bool PAGED>
__device__ __forceinline__ TileRows fetch_rows(const PrefillParams &p, const int32_t *bt_row,
                                               int kbase, int nk_valid, int tid) {
    TileRows r{0, 0};
    if (PAGED) {
        const int tk = tid >> 3, gv = v_gv(tid);
        if (tk < nk_valid) r.bk = bt_row[block_of(p, kbase + tk)];
        if (4 * gv < nk_valid) r.bv = bt_row[block_of(p, kbase + 4 * gv)];
    }
    return r;
}

// Source loads of one tile.  K share: key tk = tid >> 3, dims [16c, 16c+16)
// with c = tid & 7.  V share: keys 4g..4g+3 with g = v_gv(tid), dims
// [4c, 4c+4) with c = v_cv(tid).  Keys at or past nk_valid are not read
// (zeros; they are masked later).  Dense rows start at dense_row0 (the
// sequence's first row of k_rot / v_rot).
template <bool PAGED>
__device__ __forceinline__ void load_tile(const PrefillParams &p, TileRegs &r, TileRows rows,
                                          int64_t dense_row0, int h, int kbase, int nk_valid,
                                          int tid) {
    const int tk = tid >> 3, ck = tid & 7;
    const int gv = v_gv(tid), cv = v_cv(tid);
    if (PAGED) {
        auto in_block = [&](int kpos) { return kpos - block_of(p, kpos) * p.block_size; };
        const uint8_t *kvh = p.kv + (int64_t)h * p.slot_bytes;
        r.k[0] = r.k[1] = 0u;
        r.nk = 0.0f;
        if (tk < nk_valid) {
            // Slot rows and row_bytes are below 2^32 and 2^31: one 32 x 32 -> 64-bit multiply.
            const uint8_t *rp =
                kvh + (uint64_t)(uint32_t)(rows.bk * p.block_size + in_block(kbase + tk)) *
                          (uint32_t)p.row_bytes;
            const uint2 w = *reinterpret_cast<const uint2 *>(rp + 8 * ck);
            r.k[0] = w.x;
            r.k[1] = w.y;
            r.nk = *reinterpret_cast<const float *>(rp + 128);
        }
        const uint8_t *vp =
            kvh + (uint64_t)(uint32_t)(rows.bv * p.block_size + in_block(kbase + 4 * gv)) *
                      (uint32_t)p.row_bytes;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            r.v[i] = 0u;
            r.nv[i] = 0.0f;
            if (4 * gv + i < nk_valid) {
                const uint8_t *rp = vp + i * p.row_bytes;
                r.v[i] = *reinterpret_cast<const uint16_t *>(rp + 64 + 2 * cv);
                r.nv[i] = *reinterpret_cast<const float *>(rp + 132);
            }
        }
    } else {
        // Dense rows and the row pitch are below 2^31: 32 x 32 -> 64-bit multiplies.
        // The K tile goes by DMA (issue_k_dma); only V passes through registers.
        (void)tk;
        (void)ck;
        const uint32_t r0 = (uint32_t)(dense_row0 + kbase);
        const uint32_t hs = (uint32_t)(p.H_kv * kD);
        const uint16_t *vrow = p.v_rot + (uint64_t)(r0 + 4 * gv) * hs + h * kD + 4 * cv;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            uint2 v = make_uint2(0u, 0u);
            if (4 * gv + i < nk_valid) v = *reinterpret_cast<const uint2 *>(vrow + (size_t)i * hs);
            r.v[2 * i] = v.x;
            r.v[2 * i + 1] = v.y;
        }
    }
}

// One code byte's two values fp16(cb[code] * norm) from the per-code table
// (16 rows x 64 lane columns of fp32).
// One code byte's two values fp16(cb[code] * norm) from the code-byte table
// (hi nibble first: the even dim).
__device__ __forceinline__ uint32_t dq_byte(const uint8_t *lut, uint32_t byte, float norm) {
    const float2 c = *reinterpret_cast<const float2 *>(lut + byte * kLutEntry);
    return cvt_pk(c.x * norm, c.y * norm);
}

// fp16(cb[a] * norm), fp16(cb[b] * norm) packed, from a table of 64 lane
// columns (row = code).
__device__ __forceinline__ uint32_t dq_codes(const uint8_t *lut, uint32_t a, uint32_t b,
                                            uint32_t col, float norm) {
    const float x = *reinterpret_cast<const float *>(lut + (a << 8) + col);
    const float y = *reinterpret_cast<const float *>(lut + (b << 8) + col);
    return cvt_pk(x * norm, y * norm);
}

__device__ __forceinline__ uint32_t dq_pair(const uint8_t *lut, uint32_t byte, uint32_t col,
                                           float norm) {
    const float hi = *reinterpret_cast<const float *>(lut + ((byte >> 4) << 8) + col);
    const float lo = *reinterpret_cast<const float *>(lut + ((byte & 15u) << 8) + col);
    return cvt_pk(hi * norm, lo * norm);
}

template <bool PAGED>
__device__ __forceinline__ void store_tile(const TileRegs &r, uint8_t *kt, uint8_t *vt,
                                           const uint8_t *lutk, const uint8_t *lutv, int tid) {
    const int tk = tid >> 3, ck = tid & 7;
    const int gv = v_gv(tid), cv = v_cv(tid);
    uint32_t kw[8];      // key tk, dims [16ck, 16ck+16) as fp16 pairs (2j, 2j+1)
    uint32_t pr[4][2];   // key 4gv+i: dims (4cv, 4cv+1), (4cv+2, 4cv+3) as fp16 pairs
    if (PAGED) {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const uint32_t byte = (r.k[j >> 2] >> (8 * (j & 3))) & 0xFFu;
            kw[j] = dq_byte(lutk, byte, r.nk);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            pr[i][0] = dq_byte(lutv, r.v[i] & 0xFFu, r.nv[i]);
            pr[i][1] = dq_byte(lutv, (r.v[i] >> 8) & 0xFFu, r.nv[i]);
        }
    } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) kw[j] = 0u;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            pr[i][0] = r.v[2 * i];
            pr[i][1] = r.v[2 * i + 1];
        }
    }
    // V^T: dim 4cv+k gets keys 4gv..4gv+3 (a 4 x 4 fp16 transpose).
    uint32_t vw[4][2];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const int w = k >> 1;
        const uint32_t sel = (k & 1) ? 0x07060302u : 0x05040100u;
        vw[k][0] = __builtin_amdgcn_perm(pr[1][w], pr[0][w], sel);
        vw[k][1] = __builtin_amdgcn_perm(pr[3][w], pr[2][w], sel);
    }
    if (PAGED) {
        uint4 *kd = reinterpret_cast<uint4 *>(kt + tk * kKRow + 32 * ck);
        kd[0] = make_uint4(kw[0], kw[1], kw[2], kw[3]);
        kd[1] = make_uint4(kw[4], kw[5], kw[6], kw[7]);
    }
    const uint32_t vo = v_key_off(gv);
#pragma unroll
    for (int k = 0; k < 4; ++k)
        *reinterpret_cast<uint2 *>(vt + (4 * cv + k) * kVRow + vo) = make_uint2(vw[k][0], vw[k][1]);
}

template <bool PAGED, int GS, bool KSPLIT = false>
__global__ void __launch_bounds__(kThreads, 1)
prefill_kernel(PrefillParams p) {
    __shared__ __align__(16) uint8_t smem[kPrefillLds];
    constexpr int QB = 32 * (kWaves / GS);          // queries per workgroup

    // XCD-aware order: workgroups are dealt to the 8 XCDs round-robin by
    // linear id, so XCD k is given the k-th contiguous eighth of the logical
    // order (query blocks of one (sequence, KV head) adjacent, longest first).
    // Workgroups reading the same keys then share one XCD's L2.
    uint32_t lx, ly, lz;
    {
        const uint32_t gx = gridDim.x, gy = gridDim.y;
        const uint32_t n = gx * gy * gridDim.z;
        const uint32_t pid = blockIdx.x + gx * (blockIdx.y + gy * blockIdx.z);
        const uint32_t xcd = pid % kXcds, slot = pid / kXcds;
        const uint32_t per = n / kXcds, rem = n % kXcds;
        const uint32_t lid = xcd < rem ? xcd * (per + 1) + slot
                                       : rem * (per + 1) + (xcd - rem) * per + slot;
        lx = lid % gx;
        ly = (lid / gx) % gy;
        lz = lid / (gx * gy);
    }
    const int b = (int)ly;
    const int h = (int)lz;
    const int ks = KSPLIT ? (int)lx % p.n_ksplit : 0;   // key split (splits of a block adjacent)
    if (KSPLIT) lx /= (uint32_t)p.n_ksplit;
    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lane = tid & 63;
    const int u = lane >> 5;
    const int c32 = lane & 31;

    const int q_begin = p.cu_q[b];
    const int seq_q = p.cu_q[b + 1] - q_begin;
    const int seq_k = p.key_range == kKeysPast    ? max(0, p.seq_k[b] - seq_q)
                      : p.key_range == kKeysChunk ? seq_q
                                                  : p.seq_k[b];
    // Longest workgroups first: blockIdx.x counts query blocks from the end.
    // Consecutive workgroups share one (sequence, KV head) and so read the
    // same keys: ordering the grid by causal work across sequences instead
    // was measured 30-40 % slower (the L2 working set grows).
    const int q0 = (int)((KSPLIT ? gridDim.x / p.n_ksplit : gridDim.x) - 1 - lx) * QB;
    if (q0 >= seq_q) return;
    // Bottom-right causal alignment; without the mask every key is visible.
    const int off = p.causal ? seq_k - seq_q : seq_k;
    const int q_last = min(q0 + QB, seq_q) - 1;
    const int kend = max(0, min(seq_k, q_last + off + 1));

    const int hq = h * GS + wave % GS;
    const int qw0 = q0 + 32 * (wave / GS);           // first query of this wave
    const bool wave_live = qw0 < seq_q;
    const int my_q = min(qw0 + c32, seq_q - 1);       // this lane's query (clamped)
    const int my_kmax = min(seq_k, my_q + off + 1);   // keys [0, my_kmax) visible
    const int wave_kend = wave_live ? max(0, min(seq_k, min(qw0 + 31, seq_q - 1) + off + 1)) : 0;
    const int wave_kfull = max(0, min(seq_k, qw0 + off + 1));   // keys visible to every lane

    // ---- tables for the paged source.
    const uint8_t *lutk = smem + kLutOff;
    const uint8_t *lutv = lutk + kLutBytes / 2;
    if (PAGED) {
        float2 *lk = reinterpret_cast<float2 *>(smem + kLutOff);
        for (int i = tid; i < 2 * 256; i += kThreads) {
            const int e = i & 255;
            const float *cb = (i < 256) ? p.cb_k : p.cb_v;
            lk[i] = make_float2(cb[e >> 4], cb[e & 15]);
        }
    }

    // ---- prologue: q_rot = fp16(q H / sqrt(128)) (compression.py:290-291) as
    // the B operand of S^T = K q_rot^T, natural k (dims 16S + 8u + 0..7).
    const bool rot = p.rotate != 0;
    const float hs = rot ? 0.08838834764831845f : 1.0f;   // 1/sqrt(128)
    const uint4 hbase = hadamard_base(c32);
    half8 qb[8];
    {
        // Clamped to the T rows of q: a cu_seqlens_q beyond T reads no memory past q.
        const uint16_t *qrow = p.q + ((int64_t)min(q_begin + my_q, p.T_total - 1) * p.H_q + hq) * kD;
        half8 qin[8];
#pragma unroll
        for (int S = 0; S < 8; ++S)
            qin[S] = *reinterpret_cast<const half8 *>(qrow + 16 * S + 8 * u);
#pragma unroll
        for (int T = 0; T < 4; ++T) {
            floatx16 acc = {};
#pragma unroll
            for (int S = 0; S < 8; ++S)
                acc = mfma32(rot ? hadamard_operand(hbase, S, u, T, c32)
                                 : identity_operand(S, u, T, c32), qin[S], acc);
            qb[2 * T] = acc_to_operand(acc, 0, u, hs);
            qb[2 * T + 1] = acc_to_operand(acc, 1, u, hs);
        }
    }

    floatx16 o[4];
#pragma unroll
    for (int T = 0; T < 4; ++T) o[T] = floatx16{};
    float m_run = -INFINITY, l_run = 0.0f;

    // Per-lane LDS bases: K rows 32*sub + c32 (16 bytes at dims 16S + 8u), V^T
    // rows 32*T + c32 (16 bytes at key group 2*sub + s, half u).
    const uint32_t k_lane = (uint32_t)(c32 * kKRow + 16 * u);
    const uint32_t v_lane = (uint32_t)(kKTile + c32 * kVRow + 16 * u);
    // Dense source: byte offset of row c32, chunk 2S + u in the permuted K tile.
    uint32_t k_off[8];
#pragma unroll
    for (int S = 0; S < 8; ++S)
        k_off[S] = PAGED ? k_lane + 32u * S
                         : (uint32_t)(c32 * kKRowDense + 16 * ((2 * S + u) ^ (c32 & 15)));

    // Per 64-key tile: S^T = K q_rot^T; online softmax in the log2 domain with
    // a lazy rescale (the running max moves only when a tile's max exceeds it
    // by more than 8, so P <= 2^8 and the O rescale is rare after the first
    // tiles); O^T += V^T P^T.  MASK: the tile crosses the causal diagonal or
    // the end of the keys.
    // |scale| in the exponent; a negative scale flips the sign of q_rot
    // instead (exact in fp16), so the running max can be taken on raw scores.
    const float scl = fabsf(p.scale_log2);
    if (p.scale_log2 < 0.0f) {
#pragma unroll
        for (int S = 0; S < 8; ++S) {
            uint4 w = __builtin_bit_cast(uint4, qb[S]);
            w.x ^= 0x80008000u; w.y ^= 0x80008000u; w.z ^= 0x80008000u; w.w ^= 0x80008000u;
            qb[S] = __builtin_bit_cast(half8, w);
        }
    }
    // Whole 64-key tile per softmax step: S^T of both 32-key halves (each q
    // operand read once for both), one running-max update, then O^T += V^T P^T.
    // The max is taken on raw scores (the scale is positive: a negative scale
    // was folded into the sign of q_rot) and the scale enters the exponent's
    // FMA.
    auto tile = [&](const uint8_t *buf, int kbase, auto masked) {
        constexpr bool MASK = decltype(masked)::value;
        floatx16 st[2];
        st[0] = floatx16{};
        st[1] = floatx16{};
        // Two k-steps per batch: the operands of the whole tile would not fit.
#pragma unroll
        for (int S0 = 0; S0 < 8; S0 += 2) {
            half8 qv[2], a0[2], a1[2];
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const int S = S0 + i;
                qv[i] = qb[S];
                a0[i] = *reinterpret_cast<const half8 *>(buf + k_off[S]);
                a1[i] = *reinterpret_cast<const half8 *>(
                    buf + k_off[S] + 32 * (PAGED ? kKRow : kKRowDense));
            }
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                st[0] = mfma32(a0[i], qv[i], st[0]);
                st[1] = mfma32(a1[i], qv[i], st[1]);
            }
            asm volatile("" ::: "memory");
        }
        if (MASK) {
#pragma unroll
            for (int sub = 0; sub < 2; ++sub)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int kpos = kbase + 32 * sub + (r & 3) + 4 * u + 8 * (r >> 2);
                    if (kpos >= my_kmax) st[sub][r] = -INFINITY;
                }
        }
        float mt = -INFINITY;
#pragma unroll
        for (int sub = 0; sub < 2; ++sub)
#pragma unroll
            for (int r = 0; r < 16; r += 2) mt = max3f(mt, st[sub][r], st[sub][r + 1]);
        {
            auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(mt), __float_as_uint(mt),
                                                       false, false);
            mt = fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1])) * scl;
        }
        const bool move = mt > m_run + 8.0f;
        if (__builtin_amdgcn_ballot_w64(move)) {
            const float alpha = move ? __builtin_amdgcn_exp2f(m_run - mt) : 1.0f;  // -inf -> 0
            m_run = move ? mt : m_run;
            l_run *= alpha;
#pragma unroll
            for (int T = 0; T < 4; ++T)
#pragma unroll
                for (int r = 0; r < 16; ++r) o[T][r] *= alpha;
        }
        const float m_sub = (m_run == -INFINITY) ? 0.0f : m_run;
#pragma unroll
        for (int sub = 0; sub < 2; ++sub)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                float e = __builtin_amdgcn_exp2f(fmaf(st[sub][r], scl, -m_sub));
                if (MASK && st[sub][r] == -INFINITY) e = 0.0f;
                st[sub][r] = e;
            }
        // P as the fp16 operand of O^T += V^T P^T; the row sum l is taken over
        // the same rounded values (v_dot2_f32_f16 against ones), per lane: the
        // two halves of a query's keys are added once after the key loop.
        half8 pbs[4];
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) pbs[ks] = pack8(st[ks >> 1], 8 * (ks & 1));
        {
            const half2 one = {(_Float16)1.0f, (_Float16)1.0f};
            float ls = 0.0f;
#pragma unroll
            for (int ks = 0; ks < 4; ++ks)
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    ls = __builtin_amdgcn_fdot2(half2{pbs[ks][2 * i], pbs[ks][2 * i + 1]}, one, ls,
                                                false);
            l_run += ls;
        }
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
            half8 a[4];
#pragma unroll
            for (int T = 0; T < 4; ++T)
                a[T] = *reinterpret_cast<const half8 *>(buf + v_lane + T * 32 * kVRow + 32 * ks);
            const half8 pb = pbs[ks];
#pragma unroll
            for (int T = 0; T < 4; ++T) o[T] = mfma32(a[T], pb, o[T]);
        }
    };

    const int ntiles = (kend + kBN - 1) / kBN;
    // This workgroup's key tiles [jt0, jt1): all of them, or one split's share.
    const int jt0 = KSPLIT ? min(ntiles, ks * p.ksplit_tiles) : 0;
    // The last split runs to the end, so a max_seq_len below some seq_lens[b]
    // costs speed, never keys.
    const int jt1 = (KSPLIT && ks < p.n_ksplit - 1) ? min(ntiles, jt0 + p.ksplit_tiles) : ntiles;
    const int32_t *bt_row = PAGED ? p.block_table + (int64_t)b * p.bt_stride : nullptr;
    const int64_t dense_row0 = PAGED ? 0 : p.cu_k[b];
    TileRegs cur;
    TileRows rows_next{0, 0};
    // Dense source: K tile j into LDS buffer j & 1 by DMA, two instructions per
    // wave (keys 8*wave .. +7).  Keys past the end of the tile's valid range
    // read the last valid key's row (in bounds; their scores are masked).
    auto issue_k_dma = [&](int j) CDA_INLINE {
        if constexpr (!PAGED) {
            const int kb = j * kBN;
            const int nk_valid = min(kBN, kend - kb);
            const uint32_t pitch = (uint32_t)(p.H_kv * kD * 2);
            const uint64_t base =
                (uint64_t)(p.k_rot + ((uint64_t)(dense_row0 + kb) * p.H_kv + h) * kD);
            const v4u32 r = {(uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)base),
                             (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(base >> 32)) & 0xFFFFu,
                             (uint32_t)(kBN * pitch), 0x00020000u};
            const uint32_t dst = __builtin_amdgcn_readfirstlane(lds_addr32(smem)) +
                                 (uint32_t)((j & 1) * kTileBytes);
#pragma unroll
            for (int t = 0; t < 2; ++t) {
                const int ins = 2 * wave + t;               // keys 4*ins .. 4*ins + 3
                const int key = 4 * ins + (lane >> 4);
                const int pos = lane & 15;
                const uint32_t voff =
                    (uint32_t)min(key, nk_valid - 1) * pitch + 16u * (uint32_t)(pos ^ (key & 15));
                dma_x4_to_lds(r, voff, dst + 1024u * (uint32_t)ins);
            }
        }
    };
    if (jt0 < jt1) {
        const int k0 = jt0 * kBN, k1 = k0 + kBN;
        issue_k_dma(jt0);
        load_tile<PAGED>(p, cur, fetch_rows<PAGED>(p, bt_row, k0, min(kBN, kend - k0), tid),
                         dense_row0, h, k0, min(kBN, kend - k0), tid);
        if (jt0 + 1 < jt1) rows_next = fetch_rows<PAGED>(p, bt_row, k1, min(kBN, kend - k1), tid);
    }
    __syncthreads();   // tables visible

    // Tile j into LDS (the whole workgroup), then the loads of tile j + 1.
    // Dense source: the K DMA of tile j (issued after the previous barrier)
    // and tile j's V loads are waited for here; the K DMA of tile j + 1 goes
    // out after this barrier, when every wave is done with buffer (j + 1) & 1.
    auto produce = [&](int j) CDA_INLINE {
        uint8_t *buf = smem + (j & 1) * kTileBytes;
        if constexpr (!PAGED) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        store_tile<PAGED>(cur, buf, buf + kKTile, lutk, lutv, tid);
        if (j + 1 < jt1) {
            const int k1 = (j + 1) * kBN, k2 = (j + 2) * kBN;
            load_tile<PAGED>(p, cur, rows_next, dense_row0, h, k1, min(kBN, kend - k1), tid);
            if (j + 2 < jt1) rows_next = fetch_rows<PAGED>(p, bt_row, k2, min(kBN, kend - k2), tid);
        }
        __syncthreads();
        if (j + 1 < jt1) issue_k_dma(j + 1);
        return buf;
    };
    // The tiles whole for every row of this wave come first, those crossing
    // the causal diagonal or the end of the keys last: two loops (the same
    // number of barriers for every wave) keep one compute path per loop body,
    // so the O accumulators stay in the same registers from tile to tile.
    const int j_mask = __builtin_amdgcn_readfirstlane(
        wave_live ? max(jt0, min(jt1, wave_kfull / kBN)) : jt1);
    for (int j = jt0; j < j_mask; ++j) {
        const uint8_t *buf = produce(j);
        if (j * kBN < wave_kend) tile(buf, j * kBN, std::false_type{});
    }
    for (int j = j_mask; j < jt1; ++j) {
        const uint8_t *buf = produce(j);
        if (wave_live && j * kBN < wave_kend) tile(buf, j * kBN, std::true_type{});
    }
    if (!wave_live) return;
    {
        // l over all of the query's keys: this lane's half plus the partner's.
        auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(l_run), __float_as_uint(l_run),
                                                   false, false);
        l_run = __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
    }

    if (KSPLIT) {
        // Partial of this split: O^T rows are dims (acc element i of tile T is
        // dim 32T + 8(i >> 2) + 4u + (i & 3)), columns queries.  A split that
        // saw no visible key writes O = 0, m = -inf, l = 0.
        if (qw0 + c32 < seq_q && q_begin + qw0 + c32 < p.T_total) {
            const int64_t row = ((int64_t)(p.ks_base + ks) * p.T_total + q_begin + qw0 + c32) * p.H_q + hq;
            float *po = p.part_o + row * kD;
#pragma unroll
            for (int T = 0; T < 4; ++T)
#pragma unroll
                for (int gi = 0; gi < 4; ++gi)
                    *reinterpret_cast<float4 *>(po + 32 * T + 8 * gi + 4 * u) =
                        make_float4(o[T][4 * gi + 0], o[T][4 * gi + 1], o[T][4 * gi + 2],
                                    o[T][4 * gi + 3]);
            if (u == 0) *reinterpret_cast<float2 *>(p.part_ml + row * 2) = make_float2(m_run, l_run);
        }
        return;
    }

    if (p.merge_slot0) {
        // Merge the partial of the other keys (same lane layout as the split
        // kernel's partial store): m = max(m1, m2), O = sum 2^(mi - m) Oi.
        const bool valid = qw0 + c32 < seq_q && q_begin + qw0 + c32 < p.T_total;
        const int64_t row = (int64_t)(q_begin + min(qw0 + c32, seq_q - 1)) * p.H_q + hq;
        const float2 ml = valid ? *reinterpret_cast<const float2 *>(p.part_ml + row * 2)
                                : make_float2(-INFINITY, 0.0f);
        const float m = fmaxf(m_run, ml.x);
        const float a = (m_run == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(m_run - m);
        const float c = (ml.x == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(ml.x - m);
        l_run = l_run * a + ml.y * c;
        m_run = m;
        const float *po = p.part_o + row * kD;
#pragma unroll
        for (int T = 0; T < 4; ++T)
#pragma unroll
            for (int gi = 0; gi < 4; ++gi) {
                const float4 v = valid ? *reinterpret_cast<const float4 *>(po + 32 * T + 8 * gi + 4 * u)
                                       : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                o[T][4 * gi + 0] = fmaf(o[T][4 * gi + 0], a, v.x * c);
                o[T][4 * gi + 1] = fmaf(o[T][4 * gi + 1], a, v.y * c);
                o[T][4 * gi + 2] = fmaf(o[T][4 * gi + 2], a, v.z * c);
                o[T][4 * gi + 3] = fmaf(o[T][4 * gi + 3], a, v.w * c);
            }
    }

    if (p.lse != nullptr && u == 0 && qw0 + c32 < seq_q && q_begin + qw0 + c32 < p.T_total) {
        // m_run is the running max of scale * s * log2(e); l_run sums 2^(that - m_run).
        constexpr float kLn2 = 0.6931471805599453f;
        p.lse[(int64_t)hq * p.T_total + q_begin + qw0 + c32] =
            l_run > 0.0f ? (m_run + log2f(l_run)) * kLn2 : INFINITY;
    }

    // ---- epilogue: O_rot = fp16(O / l) (attention.py:93), out = fp16(O_rot H / sqrt(128)).
    const float inv_l = 1.0f / fmaxf(l_run, 1e-30f);
    half8 ob[8];
#pragma unroll
    for (int T = 0; T < 4; ++T) {
        ob[2 * T] = acc_to_operand(o[T], 0, u, inv_l);
        ob[2 * T + 1] = acc_to_operand(o[T], 1, u, inv_l);
    }
    const bool store = qw0 + c32 < seq_q && q_begin + qw0 + c32 < p.T_total;
    uint16_t *orow = p.out + ((int64_t)(q_begin + qw0 + c32) * p.H_q + hq) * kD;
    // A fresh (opaque) copy of the Hadamard base, so the compiler rebuilds the
    // operands here instead of keeping the prologue's 32 of them (128 VGPRs)
    // alive through the key loop.
    uint4 hb2 = hbase;
    asm volatile("" : "+v"(hb2.x), "+v"(hb2.y), "+v"(hb2.z), "+v"(hb2.w));
#pragma unroll
    for (int T = 0; T < 4; ++T) {
        floatx16 acc = {};
#pragma unroll
        for (int S = 0; S < 8; ++S)
            acc = mfma32(rot ? hadamard_operand(hb2, S, u, T, c32)
                             : identity_operand(S, u, T, c32), ob[S], acc);
        if (store) {
#pragma unroll
            for (int gi = 0; gi < 4; ++gi) {
                const uint2 v = make_uint2(cvt_pk(acc[4 * gi + 0] * hs, acc[4 * gi + 1] * hs),
                                           cvt_pk(acc[4 * gi + 2] * hs, acc[4 * gi + 3] * hs));
                *reinterpret_cast<uint2 *>(orow + 32 * T + 8 * gi + 4 * u) = v;
            }
        }
    }
}

// Dense rotated K/V from the paged cache (fa2_cda.py:64-95): row b*max_seq + t
// of (B*max_seq, H_kv, 128) fp16 = fp16(centroid * norm) for t < seq_lens[b],
// zeros beyond.  One 256-thread block per (4 rows of one sequence); thread =
// (row, head, 16-dim chunk); the per-code tables sit in LDS (64 lane columns).
template <int LV>
__global__ void __launch_bounds__(256)
paged_to_dense_kernel(const uint8_t *kv, int64_t row_bytes, int slot_bytes, int H_kv,
                      const int32_t *block_table, int bt_stride, const int32_t *seq_lens,
                      const float *cb_k, const float *cb_v, int block_size, int max_seq,
                      uint16_t *k_out, uint16_t *v_out) {
    __shared__ float lut[2][16 * 64];
    const int tid = threadIdx.x;
    for (int i = tid; i < 2 * 16 * 64; i += 256)
        lut[i >> 10][i & 1023] = (i < 1024) ? cb_k[(i & 1023) >> 6]
                                            : (((i & 1023) >> 6) < LV ? cb_v[(i & 1023) >> 6] : 0.0f);
    __syncthreads();
    const int b = blockIdx.y;
    const int n = min(seq_lens[b], bt_stride * block_size);
    const uint32_t col = (uint32_t)(tid & 63) * 4u;
    const uint8_t *lk = reinterpret_cast<const uint8_t *>(lut[0]);
    const uint8_t *lv = reinterpret_cast<const uint8_t *>(lut[1]);
    const int per_row = H_kv * 8;                       // threads per token row
    for (int w = tid; w < 4 * per_row; w += 256) {
        const int t = blockIdx.x * 4 + w / per_row;
        if (t >= max_seq) break;
        const int h = (w % per_row) >> 3, c = w & 7;    // dims [16c, 16c+16)
        uint4 ko0 = make_uint4(0, 0, 0, 0), ko1 = ko0, vo0 = ko0, vo1 = ko0;
        if (t < n) {
            const int64_t slot =
                (int64_t)block_table[(int64_t)b * bt_stride + t / block_size] * block_size + t % block_size;
            const uint8_t *rp = kv + slot * row_bytes + (int64_t)h * slot_bytes;
            // Slot: [K codes 64 | V codes KBV | K norm | V norm].
            constexpr int KBV = LV == 16 ? 64 : 32;
            const uint2 kc = *reinterpret_cast<const uint2 *>(rp + 8 * c);
            const float nk = *reinterpret_cast<const float *>(rp + 64 + KBV);
            const float nv = *reinterpret_cast<const float *>(rp + 68 + KBV);
            uint32_t kw[8], vw[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const uint32_t kb = ((j < 4 ? kc.x : kc.y) >> (8 * (j & 3))) & 0xFFu;
                kw[j] = dq_pair(lk, kb, col, nk);
            }
            if constexpr (LV == 16) {
                const uint2 vc = *reinterpret_cast<const uint2 *>(rp + 64 + 8 * c);
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const uint32_t vb = ((j < 4 ? vc.x : vc.y) >> (8 * (j & 3))) & 0xFFu;
                    vw[j] = dq_pair(lv, vb, col, nv);
                }
            } else {
                // 2-bit codes: dim 4j at bits 7:6 of byte j (compression.py:382-386).
                const uint32_t vc = *reinterpret_cast<const uint32_t *>(rp + 64 + 4 * c);
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const uint32_t vb = (vc >> (8 * j)) & 0xFFu;
                    vw[2 * j] = dq_codes(lv, vb >> 6, (vb >> 4) & 3u, col, nv);
                    vw[2 * j + 1] = dq_codes(lv, (vb >> 2) & 3u, vb & 3u, col, nv);
                }
            }
            ko0 = make_uint4(kw[0], kw[1], kw[2], kw[3]);
            ko1 = make_uint4(kw[4], kw[5], kw[6], kw[7]);
            vo0 = make_uint4(vw[0], vw[1], vw[2], vw[3]);
            vo1 = make_uint4(vw[4], vw[5], vw[6], vw[7]);
        }
        const int64_t o = (((int64_t)b * max_seq + t) * H_kv + h) * kD + 16 * c;
        reinterpret_cast<uint4 *>(k_out + o)[0] = ko0;
        reinterpret_cast<uint4 *>(k_out + o)[1] = ko1;
        reinterpret_cast<uint4 *>(v_out + o)[0] = vo0;
        reinterpret_cast<uint4 *>(v_out + o)[1] = vo1;
    }
}

// y = fp16(scale * x H) for rows of 128 fp16 (Sylvester order, natural index):
// 16 lanes per row, 8 elements per lane; butterflies over index bits 0-2 in
// registers and bits 3-6 across lanes, in fp32.
__global__ void __launch_bounds__(256)
hadamard128_kernel(const uint16_t *x, uint16_t *y, int64_t rows, float scale) {
    const int64_t row = (int64_t)blockIdx.x * 16 + (threadIdx.x >> 4);
    const int l16 = threadIdx.x & 15;
    float v[8] = {};
    if (row < rows) {
        const uint4 w = *reinterpret_cast<const uint4 *>(x + row * kD + 8 * l16);
        const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            v[2 * i] = h2f((uint16_t)(ws[i] & 0xFFFFu));
            v[2 * i + 1] = h2f((uint16_t)(ws[i] >> 16));
        }
    }
#pragma unroll
    for (int m = 1; m < 8; m <<= 1)
#pragma unroll
        for (int i = 0; i < 8; ++i)
            if (!(i & m)) {
                const float a = v[i], c = v[i | m];
                v[i] = a + c;
                v[i | m] = a - c;
            }
#pragma unroll
    for (int m = 1; m < 16; m <<= 1) {
        const bool upper = (l16 & m) != 0;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float o = __shfl_xor(v[i], m);
            v[i] = upper ? (o - v[i]) : (v[i] + o);
        }
    }
    if (row < rows) {
        uint4 w;
        w.x = cvt_pk(v[0] * scale, v[1] * scale);
        w.y = cvt_pk(v[2] * scale, v[3] * scale);
        w.z = cvt_pk(v[4] * scale, v[5] * scale);
        w.w = cvt_pk(v[6] * scale, v[7] * scale);
        *reinterpret_cast<uint4 *>(y + row * kD + 8 * l16) = w;
    }
}

// Merge of the key-split partials of prefill_kernel, then the epilogue of the
// unsplit kernel: O_rot = fp16(O / l) (attention.py:93), out = fp16(O_rot H /
// sqrt(128)) (compression.py:293-296).  Merge as attention.py:239-272 with m
// in the log2 domain: w_i = 2^(m_i - max m), O = sum w_i O_i, l = sum w_i l_i.
// One wave per (token, q-head), two dims per lane; block = 4 q-heads.  Lane i
// loads split i's (m, l) (n_ksplit <= 64), so the weights come from two wave
// reductions, and the O loads are issued 16 splits at a time.
constexpr int kCombineBatch = 16;
__global__ void __launch_bounds__(256)
prefill_combine_kernel(const float *__restrict__ part_o, const float *__restrict__ part_ml,
                       uint16_t *__restrict__ out, int T, int H_q, int n_ksplit,
                       const int32_t *__restrict__ cu_q, int B) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int hq = blockIdx.y * 4 + wave;
    const int t = blockIdx.x;
    // Rows past the last sequence (a padded q) have no partials: leave them.
    if (t >= cu_q[B]) return;
    const int64_t split_rows = (int64_t)T * H_q;
    const int64_t row = (int64_t)t * H_q + hq;
    float mi = -INFINITY, li = 0.0f;
    if (lane < n_ksplit) {
        const float2 ml = *reinterpret_cast<const float2 *>(part_ml + (lane * split_rows + row) * 2);
        mi = ml.x;
        li = ml.y;
    }
    float m = mi;
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) m = fmaxf(m, __shfl_xor(m, d));
    // A split without a visible key (m_i = -inf) has weight 0.
    const float wi = (mi == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(mi - m);
    float l = wi * li;
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) l += __shfl_xor(l, d);
    float o0 = 0.0f, o1 = 0.0f;
    const float *po = part_o + row * kD + 2 * lane;
    for (int i0 = 0; i0 < n_ksplit; i0 += kCombineBatch) {
        float2 ov[kCombineBatch];
#pragma unroll
        for (int k = 0; k < kCombineBatch; ++k)
            ov[k] = (i0 + k < n_ksplit)
                        ? *reinterpret_cast<const float2 *>(po + (i0 + k) * split_rows * kD)
                        : make_float2(0.0f, 0.0f);
#pragma unroll
        for (int k = 0; k < kCombineBatch; ++k) {
            if (i0 + k >= n_ksplit) break;
            const float w = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(wi), i0 + k));
            if (w != 0.0f) {
                o0 = fmaf(w, ov[k].x, o0);
                o1 = fmaf(w, ov[k].y, o1);
            }
        }
    }
    const float inv_l = 1.0f / fmaxf(l, 1e-30f);
    // O_rot = fp16(O / l) (attention.py:93), then out = O_rot H / sqrt(128) by
    // a fast Walsh-Hadamard transform: lane l holds dims 2l, 2l+1; the stage
    // on index bit 0 runs in registers, bits 1-6 pair lane l with lane
    // l ^ 2^(b-1) (x_i + x_partner where bit b of i is clear, x_partner - x_i
    // where it is set): the Sylvester sum sum_k (-1)^popcount(j & k) x_k.
    float x0 = h2f(f2h_after_f32(o0 * inv_l));
    float x1 = h2f(f2h_after_f32(o1 * inv_l));
    {
        const float a = x0 + x1, b = x0 - x1;
        x0 = a;
        x1 = b;
    }
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const float p0 = __shfl_xor(x0, d), p1 = __shfl_xor(x1, d);
        const float sgn = (lane & d) ? -1.0f : 1.0f;
        x0 = fmaf(sgn, x0, p0);
        x1 = fmaf(sgn, x1, p1);
    }
    const float hs = 0.08838834764831845f;
    const uint32_t hv = (uint32_t)f2h_after_f32(x0 * hs) | ((uint32_t)f2h_after_f32(x1 * hs) << 16);
    *reinterpret_cast<uint32_t *>(out + row * kD + 2 * lane) = hv;
}

// The attention kernel alone; with `partials` it writes split partials
// (n_ksplit of them from slot ks_base on) for prefill_combine_kernel.
template <bool PAGED>
int launch_prefill_kernel(const PrefillParams &p, int B, int max_q, bool partials, hipStream_t st,
                          const char *fn) {
    const int qb = 32 * (kWaves / p.GS);
    const dim3 grid((unsigned)((max_q + qb - 1) / qb * p.n_ksplit), B, p.H_kv);
    if (grid.x == 0) return CDA_OK;
    if (partials) {
        if (p.GS == 4)
            prefill_kernel<PAGED, 4, true><<<grid, kThreads, 0, st>>>(p);
        else
            prefill_kernel<PAGED, 8, true><<<grid, kThreads, 0, st>>>(p);
    } else if (p.GS == 4) {
        prefill_kernel<PAGED, 4><<<grid, kThreads, 0, st>>>(p);
    } else {
        prefill_kernel<PAGED, 8><<<grid, kThreads, 0, st>>>(p);
    }
    CDA_LAUNCH_CHECK(std::string(fn) + ": prefill_kernel");
    return CDA_OK;
}

int launch_combine(const PrefillParams &p, int slots, int B, hipStream_t st, const char *fn) {
    prefill_combine_kernel<<<dim3((unsigned)p.T_total, (unsigned)(p.H_q / 4)), 256, 0, st>>>(
        p.part_o, p.part_ml, p.out, p.T_total, p.H_q, slots, p.cu_q, B);
    CDA_LAUNCH_CHECK(std::string(fn) + ": prefill_combine_kernel");
    return CDA_OK;
}

template <bool PAGED>
int launch_prefill(const PrefillParams &p, int B, int max_q, hipStream_t st, const char *fn) {
    const bool split = p.n_ksplit > 1;
    const int rc = launch_prefill_kernel<PAGED>(p, B, max_q, split, st, fn);
    if (rc != CDA_OK || !split) return rc;
    return launch_combine(p, p.n_ksplit, B, st, fn);
}

// Key-split plan: split only when the unsplit grid leaves CUs idle (fewer
// than 256 workgroups), into splits of at least 4 key tiles (256 keys), aiming
// at one round of ~256 workgroups (one per CU: the kernel's LDS admits one);
// at most kMaxKsplit splits.  Targets of 512 and 1024 workgroups (two and four
// rounds of shorter splits) measured 5-30 % slower.
constexpr int kMaxKsplit = 64;
static_assert(kMaxKsplit <= 64, "prefill_combine_kernel: one lane per split");
void prefill_ksplit_plan(int B, int H_q, int H_kv, int max_q, int max_k, int *n_split,
                         int *split_tiles, int max_split = kMaxKsplit) {
    const int qb = 32 * (kWaves / (H_q / H_kv));
    const int64_t wgs = (int64_t)((max_q + qb - 1) / qb) * B * H_kv;
    const int tiles = (max_k + kBN - 1) / kBN;
    int ns = 1;
    if (wgs > 0 && wgs < 256) {
        ns = (int)std::min<int64_t>((256 + wgs - 1) / wgs, tiles / 4);
        ns = std::min(ns, max_split);
    }
    if (ns < 2) {
        *n_split = 1;
        *split_tiles = tiles;
        return;
    }
    const int per = (tiles + ns - 1) / ns;
    *split_tiles = per;
    *n_split = (tiles + per - 1) / per;
}

size_t prefill_ws_bytes(int T, int H_q, int n_split) {
    const size_t o = (size_t)n_split * T * H_q * kD * 4;
    const size_t ml = (size_t)n_split * T * H_q * 2 * 4;
    return ((o + 255) & ~(size_t)255) + ((ml + 255) & ~(size_t)255);
}

}  // namespace
}  // namespace cda

using namespace cda;

namespace cda {
namespace {
// Both paged entry points; max_seq_len < 0: no key split.
int prefill_paged_impl(const char *fn, const void *q, const void *kv_cache, int slot_bytes,
                       int H_kv, const int32_t *block_table, int bt_stride,
                       const int32_t *cu_seqlens_q, const int32_t *seq_lens, int B,
                       const float *cb_k, const float *cb_v, int levels, void *out, int T,
                       int H_q, int block_size, int max_query_len, float scale, int max_seq_len,
                       void *workspace, size_t workspace_bytes, void *stream) {
    CDA_REQUIRE(q && kv_cache && block_table && cu_seqlens_q && seq_lens && cb_k && cb_v && out,
                "cda_prefill_paged_hadamard: null pointer argument");
    CDA_REQUIRE(B >= 0 && H_kv > 0 && H_q > 0 && max_query_len >= 0,
                "cda_prefill_paged_hadamard: bad B / H_q / H_kv / max_query_len");
    CDA_REQUIRE(H_q % H_kv == 0 && (H_q / H_kv == 4 || H_q / H_kv == 8),
                "cda_prefill_paged_hadamard: H_q / H_kv must be 4 or 8");
    CDA_REQUIRE(levels == 16 && slot_bytes >= 136,
                "cda_prefill_paged_hadamard: the prefill reads K4V4 caches (16 levels, slot >= 136 B)");
    CDA_REQUIRE(block_size > 0 && block_size % 16 == 0 && bt_stride > 0,
                "cda_prefill_paged_hadamard: block_size must be a positive multiple of 16");
    CDA_REQUIRE(((uintptr_t)q & 15) == 0 && ((uintptr_t)out & 15) == 0 &&
                    ((uintptr_t)kv_cache & 7) == 0 && slot_bytes % 8 == 0,
                "cda_prefill_paged_hadamard: q/out must be 16-byte and the cache 8-byte aligned");
    if (B == 0 || max_query_len == 0) return CDA_OK;
    PrefillParams p{};
    p.q = static_cast<const uint16_t *>(q);
    p.out = static_cast<uint16_t *>(out);
    p.cu_q = cu_seqlens_q;
    p.seq_k = seq_lens;
    p.H_q = H_q;
    p.H_kv = H_kv;
    p.GS = H_q / H_kv;
    p.scale_log2 = scale * kLog2e;
    p.kv = static_cast<const uint8_t *>(kv_cache);
    p.block_table = block_table;
    p.bt_stride = bt_stride;
    p.block_size = block_size;
    p.bs_shift = (block_size & (block_size - 1)) == 0 ? __builtin_ctz(block_size) : -1;
    p.slot_bytes = slot_bytes;
    p.row_bytes = (int64_t)H_kv * slot_bytes;
    p.cb_k = cb_k;
    p.cb_v = cb_v;
    p.n_ksplit = 1;
    p.T_total = T;
    p.rotate = 1;
    p.causal = 1;
    CDA_REQUIRE(T > 0 || max_query_len == 0, std::string(fn) + ": T must be the number of query rows");
    if (max_seq_len >= 0) {
        int ns, per;
        prefill_ksplit_plan(B, H_q, H_kv, max_query_len, max_seq_len, &ns, &per);
        if (ns > 1) {
            CDA_REQUIRE(T > 0, std::string(fn) + ": T must be the number of query rows");
            const size_t need = prefill_ws_bytes(T, H_q, ns);
            if (!workspace || workspace_bytes < need || ((uintptr_t)workspace & 255))
                return fail(CDA_E_WORKSPACE, std::string(fn) + ": workspace missing, misaligned "
                                             "or smaller than cda_prefill_workspace_size()");
            const size_t o_bytes = ((size_t)ns * T * H_q * kD * 4 + 255) & ~(size_t)255;
            p.n_ksplit = ns;
            p.ksplit_tiles = per;
            p.part_o = static_cast<float *>(workspace);
            p.part_ml = reinterpret_cast<float *>(static_cast<char *>(workspace) + o_bytes);
        }
    }
    return launch_prefill<true>(p, B, max_query_len, static_cast<hipStream_t>(stream), fn);
}
}  // namespace
}  // namespace cda

extern "C" int cda_prefill_paged_hadamard(const void *q, const void *kv_cache, int64_t num_slots,
                                          int slot_bytes, int H_kv, const int32_t *block_table,
                                          int bt_stride, const int32_t *cu_seqlens_q,
                                          const int32_t *seq_lens, int B, const float *cb_k,
                                          const float *cb_v, int levels, void *out, int T,
                                          int H_q, int block_size, int max_query_len,
                                          float scale, void *stream) {
    (void)num_slots;
    return prefill_paged_impl("cda_prefill_paged_hadamard", q, kv_cache, slot_bytes, H_kv,
                              block_table, bt_stride, cu_seqlens_q, seq_lens, B, cb_k, cb_v,
                              levels, out, T, H_q, block_size, max_query_len, scale, -1, nullptr,
                              0, stream);
}

extern "C" size_t cda_prefill_workspace_size(int B, int T, int H_q, int H_kv, int max_query_len,
                                             int max_seq_len) {
    if (B <= 0 || T <= 0 || H_q <= 0 || H_kv <= 0 || H_q % H_kv != 0 ||
        (H_q / H_kv != 4 && H_q / H_kv != 8) || max_query_len <= 0 || max_seq_len <= 0)
        return 0;
    int ns, per;
    prefill_ksplit_plan(B, H_q, H_kv, max_query_len, max_seq_len, &ns, &per);
    return ns > 1 ? prefill_ws_bytes(T, H_q, ns) : 0;
}

extern "C" int cda_prefill_paged_hadamard_ws(const void *q, const void *kv_cache,
                                             int64_t num_slots, int slot_bytes, int H_kv,
                                             const int32_t *block_table, int bt_stride,
                                             const int32_t *cu_seqlens_q, const int32_t *seq_lens,
                                             int B, const float *cb_k, const float *cb_v,
                                             int levels, void *out, int T, int H_q,
                                             int block_size, int max_query_len, int max_seq_len,
                                             float scale, void *workspace,
                                             size_t workspace_bytes, void *stream) {
    const char *fn = "cda_prefill_paged_hadamard_ws";
    (void)num_slots;
    CDA_REQUIRE(max_seq_len >= 0, "cda_prefill_paged_hadamard_ws: max_seq_len must be >= 0");
    return prefill_paged_impl(fn, q, kv_cache, slot_bytes, H_kv, block_table, bt_stride,
                              cu_seqlens_q, seq_lens, B, cb_k, cb_v, levels, out, T, H_q,
                              block_size, max_query_len, scale, max_seq_len, workspace,
                              workspace_bytes, stream);
}

namespace cda {
namespace {
// Causal / non-causal varlen flash attention over dense fp16 K/V rows, with
// (rotate = 1) or without the Hadamard prologue and epilogue.
int fa2_varlen_dense(const void *q, const void *k, const void *v, void *out,
                     const int32_t *cu_seqlens_q, const int32_t *cu_seqlens_k,
                     const int32_t *seqused_k, int B, int T, int H_q, int H_kv,
                     int max_query_len, float scale, int causal, int rotate, float *lse,
                     void *stream, const char *fn) {
    const std::string f(fn);
    CDA_REQUIRE(q && k && v && out && cu_seqlens_q && cu_seqlens_k && seqused_k,
                f + ": null pointer argument");
    CDA_REQUIRE(B >= 0 && H_kv > 0 && H_q > 0 && max_query_len >= 0,
                f + ": bad B / H_q / H_kv / max_query_len");
    CDA_REQUIRE(H_q % H_kv == 0 && (H_q / H_kv == 4 || H_q / H_kv == 8),
                f + ": H_q / H_kv must be 4 or 8");
    CDA_REQUIRE(((uintptr_t)q & 15) == 0 && ((uintptr_t)out & 15) == 0 &&
                    ((uintptr_t)k & 15) == 0 && ((uintptr_t)v & 15) == 0,
                f + ": tensors must be 16-byte aligned");
    if (B == 0 || max_query_len == 0) return CDA_OK;
    CDA_REQUIRE(T > 0, f + ": T must be the number of query rows");
    PrefillParams p{};
    p.q = static_cast<const uint16_t *>(q);
    p.out = static_cast<uint16_t *>(out);
    p.cu_q = cu_seqlens_q;
    p.seq_k = seqused_k;
    p.H_q = H_q;
    p.H_kv = H_kv;
    p.GS = H_q / H_kv;
    p.scale_log2 = scale * kLog2e;
    p.k_rot = static_cast<const uint16_t *>(k);
    p.v_rot = static_cast<const uint16_t *>(v);
    p.cu_k = cu_seqlens_k;
    p.n_ksplit = 1;
    p.T_total = T;
    p.rotate = rotate;
    p.causal = causal;
    p.lse = lse;
    return launch_prefill<false>(p, B, max_query_len, static_cast<hipStream_t>(stream), fn);
}

// out row r (fp16, 128 dims) = fp16(cb[code] * norm) of source row src(r):
// src(r) = r, or, with a block table, the slot of token t = r % max_seq of
// sequence b = r / max_seq (rows past seq_lens[b] are zero).  One thread per
// (row, 16-dim chunk); codes MSB-first, 4-bit (levels 16) or 2-bit (4).
__global__ void __launch_bounds__(256)
dequant_rows_kernel(const uint8_t *codes, const float *norms, int64_t rows, int H,
                    const float *cb, int levels, const int32_t *block_table, int bt_stride,
                    const int32_t *seq_lens, int block_size, int max_seq, uint16_t *out) {
    __shared__ float lut[16];
    if (threadIdx.x < 16) lut[threadIdx.x] = threadIdx.x < levels ? cb[threadIdx.x] : 0.0f;
    __syncthreads();
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;   // (row, head, chunk)
    if (i >= rows * H * 8) return;
    const int c = (int)(i & 7);
    const int64_t rh = i >> 3;
    const int h = (int)(rh % H);
    const int64_t r = rh / H;
    int64_t src = r;
    bool zero = false;
    if (block_table) {
        const int64_t b = r / max_seq;
        const int t = (int)(r - b * max_seq);
        zero = t >= seq_lens[b];
        src = zero ? 0 : (int64_t)block_table[b * bt_stride + t / block_size] * block_size +
                             t % block_size;
    }
    uint32_t w[8];
    if (zero) {
#pragma unroll
        for (int j = 0; j < 8; ++j) w[j] = 0;
    } else {
        const int cbytes = levels == 16 ? 64 : 32;
        const uint8_t *row = codes + (src * H + h) * cbytes;
        const float nrm = norms[src * H + h];
        float x[16];
        if (levels == 16) {
            const uint2 cw = *reinterpret_cast<const uint2 *>(row + 8 * c);
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const uint32_t byte = ((j < 4 ? cw.x : cw.y) >> (8 * (j & 3))) & 0xFFu;
                x[2 * j] = lut[byte >> 4];
                x[2 * j + 1] = lut[byte & 15];
            }
        } else {
            const uint32_t cw = *reinterpret_cast<const uint32_t *>(row + 4 * c);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const uint32_t byte = (cw >> (8 * j)) & 0xFFu;
#pragma unroll
                for (int e = 0; e < 4; ++e) x[4 * j + e] = lut[(byte >> (6 - 2 * e)) & 3];
            }
        }
#pragma unroll
        for (int j = 0; j < 8; ++j)
            w[j] = (uint32_t)f2h_after_f32(x[2 * j] * nrm) |
                   ((uint32_t)f2h_after_f32(x[2 * j + 1] * nrm) << 16);
    }
    uint4 *dst = reinterpret_cast<uint4 *>(out + (r * H + h) * kD + 16 * c);
    dst[0] = make_uint4(w[0], w[1], w[2], w[3]);
    dst[1] = make_uint4(w[4], w[5], w[6], w[7]);
}
}  // namespace
}  // namespace cda

extern "C" int cda_fa2_varlen_fwd_hadamard(const void *q, const void *k_rot, const void *v_rot,
                                           void *out, const int32_t *cu_seqlens_q,
                                           const int32_t *cu_seqlens_k, const int32_t *seqused_k,
                                           int B, int T, int H_q, int H_kv, int max_query_len,
                                           int max_seq_len, float scale, void *stream) {
    (void)max_seq_len;
    return fa2_varlen_dense(q, k_rot, v_rot, out, cu_seqlens_q, cu_seqlens_k, seqused_k, B, T,
                            H_q, H_kv, max_query_len, scale, 1, 1, nullptr, stream,
                            "cda_fa2_varlen_fwd_hadamard");
}

extern "C" int cda_fa2_varlen_fwd(const void *q, const void *k, const void *v, void *out,
                                  const int32_t *cu_seqlens_q, const int32_t *cu_seqlens_k,
                                  const int32_t *seqused_k, int B, int T, int H_q, int H_kv,
                                  int max_query_len, float scale, int causal, void *stream) {
    return fa2_varlen_dense(q, k, v, out, cu_seqlens_q, cu_seqlens_k, seqused_k, B, T, H_q, H_kv,
                            max_query_len, scale, causal != 0, 0, nullptr, stream,
                            "cda_fa2_varlen_fwd");
}

extern "C" int cda_fa2_varlen_fwd_lse(const void *q, const void *k, const void *v, void *out,
                                      const int32_t *cu_seqlens_q, const int32_t *cu_seqlens_k,
                                      const int32_t *seqused_k, int B, int T, int H_q, int H_kv,
                                      int max_query_len, float scale, int causal,
                                      float *softmax_lse, void *stream) {
    CDA_REQUIRE(softmax_lse != nullptr, "cda_fa2_varlen_fwd_lse: softmax_lse is null");
    return fa2_varlen_dense(q, k, v, out, cu_seqlens_q, cu_seqlens_k, seqused_k, B, T, H_q, H_kv,
                            max_query_len, scale, causal != 0, 0, softmax_lse, stream,
                            "cda_fa2_varlen_fwd_lse");
}

extern "C" int cda_dequantize_rows(const void *codes, const float *norms, int64_t rows, int H,
                                   const float *cb, int levels, const int32_t *block_table,
                                   int bt_stride, const int32_t *seq_lens, int block_size,
                                   int max_seq_len, void *out, void *stream) {
    CDA_REQUIRE(codes && norms && cb && out && rows >= 0 && H > 0,
                "cda_dequantize_rows: bad arguments");
    CDA_REQUIRE(levels == 16 || levels == 4, "cda_dequantize_rows: levels must be 16 or 4");
    CDA_REQUIRE(((uintptr_t)codes & 7) == 0 && ((uintptr_t)out & 15) == 0,
                "cda_dequantize_rows: codes must be 8-byte and out 16-byte aligned");
    if (block_table) {
        CDA_REQUIRE(seq_lens && bt_stride > 0 && block_size > 0 && max_seq_len > 0 &&
                        rows % max_seq_len == 0,
                    "cda_dequantize_rows: paged form needs seq_lens, bt_stride, block_size and "
                    "rows = B * max_seq_len");
    }
    if (rows == 0) return CDA_OK;
    const int64_t threads = rows * H * 8;
    dequant_rows_kernel<<<(unsigned)((threads + 255) / 256), 256, 0,
                          static_cast<hipStream_t>(stream)>>>(
        static_cast<const uint8_t *>(codes), norms, rows, H, cb, levels, block_table, bt_stride,
        seq_lens, block_size, max_seq_len, static_cast<uint16_t *>(out));
    CDA_LAUNCH_CHECK("dequant_rows_kernel");
    return CDA_OK;
}

namespace cda {
namespace {
int paged_to_dense_impl(const void *kv_cache, int slot_bytes, int H_kv, const int32_t *block_table,
                        int bt_stride, const int32_t *seq_lens, int B, const float *cb_k,
                        const float *cb_v, int levels_v, int block_size, int max_seq_len,
                        void *k_out, void *v_out, void *stream, const char *fn) {
    const std::string f(fn);
    CDA_REQUIRE(kv_cache && block_table && seq_lens && cb_k && cb_v && k_out && v_out,
                f + ": null pointer argument");
    CDA_REQUIRE(B >= 0 && H_kv > 0 && max_seq_len >= 0 && block_size > 0 && bt_stride > 0,
                f + ": bad shape arguments");
    const int data = 64 + (levels_v == 16 ? 64 : 32) + 8;
    CDA_REQUIRE(slot_bytes >= data && slot_bytes % 8 == 0,
                f + ": slot too small for the layout (136 B K4V4, 104 B K4V2) or not a "
                    "multiple of 8");
    CDA_REQUIRE(((uintptr_t)kv_cache & 7) == 0 && ((uintptr_t)k_out & 15) == 0 &&
                    ((uintptr_t)v_out & 15) == 0,
                f + ": misaligned pointer");
    if (B == 0 || max_seq_len == 0) return CDA_OK;
    const dim3 grid((max_seq_len + 3) / 4, B);
    hipStream_t st = static_cast<hipStream_t>(stream);
    const auto *kv = static_cast<const uint8_t *>(kv_cache);
    const int64_t row = (int64_t)H_kv * slot_bytes;
    auto *ko = static_cast<uint16_t *>(k_out);
    auto *vo = static_cast<uint16_t *>(v_out);
    if (levels_v == 16)
        paged_to_dense_kernel<16><<<grid, 256, 0, st>>>(kv, row, slot_bytes, H_kv, block_table,
                                                        bt_stride, seq_lens, cb_k, cb_v,
                                                        block_size, max_seq_len, ko, vo);
    else
        paged_to_dense_kernel<4><<<grid, 256, 0, st>>>(kv, row, slot_bytes, H_kv, block_table,
                                                       bt_stride, seq_lens, cb_k, cb_v,
                                                       block_size, max_seq_len, ko, vo);
    CDA_LAUNCH_CHECK(f + ": paged_to_dense_kernel");
    return CDA_OK;
}
}  // namespace
}  // namespace cda

extern "C" int cda_fa2_paged_cache_to_dense_rotated(const void *kv_cache, int64_t num_slots,
                                                    int slot_bytes, int H_kv,
                                                    const int32_t *block_table, int bt_stride,
                                                    const int32_t *seq_lens, int B,
                                                    const float *cb_k, const float *cb_v,
                                                    int levels, int block_size, int max_seq_len,
                                                    void *k_out, void *v_out, void *stream) {
    (void)num_slots;
    CDA_REQUIRE(levels == 16, "cda_fa2_paged_cache_to_dense_rotated: K4V4 caches only (16 levels)");
    return paged_to_dense_impl(kv_cache, slot_bytes, H_kv, block_table, bt_stride, seq_lens, B,
                               cb_k, cb_v, 16, block_size, max_seq_len, k_out, v_out, stream,
                               "cda_fa2_paged_cache_to_dense_rotated");
}

extern "C" int cda_fa2_paged_cache_to_dense_rotated_k4v2(
    const void *kv_cache, int64_t num_slots, int slot_bytes, int H_kv, const int32_t *block_table,
    int bt_stride, const int32_t *seq_lens, int B, const float *cb_k, const float *cb_v,
    int block_size, int max_seq_len, void *k_out, void *v_out, void *stream) {
    (void)num_slots;
    return paged_to_dense_impl(kv_cache, slot_bytes, H_kv, block_table, bt_stride, seq_lens, B,
                               cb_k, cb_v, 4, block_size, max_seq_len, k_out, v_out, stream,
                               "cda_fa2_paged_cache_to_dense_rotated_k4v2");
}

extern "C" int cda_hadamard128_fp16(const void *x, void *y, int64_t rows, float scale,
                                    void *stream) {
    CDA_REQUIRE(x && y && rows >= 0, "cda_hadamard128_fp16: bad arguments");
    CDA_REQUIRE(((uintptr_t)x & 15) == 0 && ((uintptr_t)y & 15) == 0,
                "cda_hadamard128_fp16: x and y must be 16-byte aligned");
    if (rows == 0) return CDA_OK;
    hadamard128_kernel<<<(unsigned)((rows + 15) / 16), 256, 0, static_cast<hipStream_t>(stream)>>>(
        static_cast<const uint16_t *>(x), static_cast<uint16_t *>(y), rows, scale);
    CDA_LAUNCH_CHECK("hadamard128_kernel");
    return CDA_OK;
}

// ---------------------------------------------------------------------------
// Hybrid chunked prefill (cda_attn_v2.py:1023-1060, 1474-1532): the queries of
// each sequence attend to its compressed prefix in the paged cache (keys
// [0, seq_lens[b] - q_len), all visible) and to the fresh fp16 K/V of the
// chunk itself (causal), merged by log-sum-exp (attention.py:239-272).
//   1. the chunk's K and V are rotated into the cache's frame,
//      fp16(x H / sqrt(128)) (fa2_cda.py:256-287), into the workspace;
//   2. the paged kernel over the prefix writes partials to slots [0, nA);
//   3. the dense kernel over the rotated chunk writes slots [nA, nA + nB);
//   4. prefill_combine_kernel merges the nA + nB slots and unrotates.
// When neither side needs a key split (nA = nB = 1) the chunk's partial goes
// to slot 0 first and the unsplit prefix kernel merges it before its own
// epilogue: no prefix partials, no combine launch.
// Workspace: the partials, then the rotated chunk K and V.
// ---------------------------------------------------------------------------
namespace cda {
namespace {
struct HybridPlan {
    int na, na_tiles, nb, nb_tiles;
    size_t part_bytes, kv_bytes;
};

HybridPlan hybrid_plan(int B, int T, int H_q, int H_kv, int max_query_len, int max_seq_len) {
    HybridPlan h{};
    prefill_ksplit_plan(B, H_q, H_kv, max_query_len, std::max(1, max_seq_len - 1), &h.na,
                        &h.na_tiles, kMaxKsplit / 2);
    prefill_ksplit_plan(B, H_q, H_kv, max_query_len, max_query_len, &h.nb, &h.nb_tiles,
                        kMaxKsplit / 2);
    h.part_bytes = prefill_ws_bytes(T, H_q, h.na + h.nb);
    h.kv_bytes = (((size_t)T * H_kv * kD * 2) + 255) & ~(size_t)255;
    return h;
}
}  // namespace
}  // namespace cda

extern "C" size_t cda_prefill_hybrid_workspace_size(int B, int T, int H_q, int H_kv,
                                                    int max_query_len, int max_seq_len) {
    if (B <= 0 || T <= 0 || H_q <= 0 || H_kv <= 0 || H_q % H_kv != 0 ||
        (H_q / H_kv != 4 && H_q / H_kv != 8) || max_query_len <= 0 || max_seq_len <= 0)
        return 0;
    const HybridPlan h = hybrid_plan(B, T, H_q, H_kv, max_query_len, max_seq_len);
    return h.part_bytes + 2 * h.kv_bytes;
}

extern "C" int cda_prefill_hybrid_rawkv(const void *q, const void *k_new, const void *v_new,
                                        const void *kv_cache, int64_t num_slots, int slot_bytes,
                                        int H_kv, const int32_t *block_table, int bt_stride,
                                        const int32_t *cu_seqlens_q, const int32_t *seq_lens,
                                        int B, const float *cb_k, const float *cb_v, int levels,
                                        void *out, int T, int H_q, int block_size,
                                        int max_query_len, int max_seq_len, float scale,
                                        void *workspace, size_t workspace_bytes, void *stream) {
    const char *fn = "cda_prefill_hybrid_rawkv";
    (void)num_slots;
    CDA_REQUIRE(q && k_new && v_new && kv_cache && block_table && cu_seqlens_q && seq_lens &&
                    cb_k && cb_v && out,
                "cda_prefill_hybrid_rawkv: null pointer argument");
    CDA_REQUIRE(B >= 0 && H_kv > 0 && H_q > 0 && max_query_len >= 0 && max_seq_len >= 0,
                "cda_prefill_hybrid_rawkv: bad B / H_q / H_kv / max_query_len / max_seq_len");
    CDA_REQUIRE(H_q % H_kv == 0 && (H_q / H_kv == 4 || H_q / H_kv == 8),
                "cda_prefill_hybrid_rawkv: H_q / H_kv must be 4 or 8");
    CDA_REQUIRE(levels == 16 && slot_bytes >= 136,
                "cda_prefill_hybrid_rawkv: the prefill reads K4V4 caches (16 levels, slot >= 136 B)");
    CDA_REQUIRE(block_size > 0 && block_size % 16 == 0 && bt_stride > 0,
                "cda_prefill_hybrid_rawkv: block_size must be a positive multiple of 16");
    CDA_REQUIRE(((uintptr_t)q & 15) == 0 && ((uintptr_t)out & 15) == 0 &&
                    ((uintptr_t)k_new & 15) == 0 && ((uintptr_t)v_new & 15) == 0 &&
                    ((uintptr_t)kv_cache & 7) == 0 && slot_bytes % 8 == 0,
                "cda_prefill_hybrid_rawkv: q/out/k_new/v_new must be 16-byte and the cache "
                "8-byte aligned");
    if (B == 0 || max_query_len == 0) return CDA_OK;
    CDA_REQUIRE(T > 0, "cda_prefill_hybrid_rawkv: T must be the number of query rows");
    const HybridPlan h = hybrid_plan(B, T, H_q, H_kv, max_query_len, std::max(1, max_seq_len));
    const size_t need = h.part_bytes + 2 * h.kv_bytes;
    if (!workspace || workspace_bytes < need || ((uintptr_t)workspace & 255))
        return fail(CDA_E_WORKSPACE, "cda_prefill_hybrid_rawkv: workspace missing, misaligned or "
                                     "smaller than cda_prefill_hybrid_workspace_size()");
    hipStream_t st = static_cast<hipStream_t>(stream);
    char *ws = static_cast<char *>(workspace);
    uint16_t *k_rot = reinterpret_cast<uint16_t *>(ws + h.part_bytes);
    uint16_t *v_rot = reinterpret_cast<uint16_t *>(ws + h.part_bytes + h.kv_bytes);
    const int64_t kv_rows = (int64_t)T * H_kv;
    const float hs = 0.08838834764831845f;
    hadamard128_kernel<<<(unsigned)((kv_rows + 15) / 16), 256, 0, st>>>(
        static_cast<const uint16_t *>(k_new), k_rot, kv_rows, hs);
    CDA_LAUNCH_CHECK("cda_prefill_hybrid_rawkv: hadamard128_kernel (K)");
    hadamard128_kernel<<<(unsigned)((kv_rows + 15) / 16), 256, 0, st>>>(
        static_cast<const uint16_t *>(v_new), v_rot, kv_rows, hs);
    CDA_LAUNCH_CHECK("cda_prefill_hybrid_rawkv: hadamard128_kernel (V)");

    PrefillParams p{};
    p.q = static_cast<const uint16_t *>(q);
    p.out = static_cast<uint16_t *>(out);
    p.cu_q = cu_seqlens_q;
    p.seq_k = seq_lens;
    p.H_q = H_q;
    p.H_kv = H_kv;
    p.GS = H_q / H_kv;
    p.scale_log2 = scale * kLog2e;
    p.kv = static_cast<const uint8_t *>(kv_cache);
    p.block_table = block_table;
    p.bt_stride = bt_stride;
    p.block_size = block_size;
    p.bs_shift = (block_size & (block_size - 1)) == 0 ? __builtin_ctz(block_size) : -1;
    p.slot_bytes = slot_bytes;
    p.row_bytes = (int64_t)H_kv * slot_bytes;
    p.cb_k = cb_k;
    p.cb_v = cb_v;
    p.T_total = T;
    p.rotate = 1;
    p.part_o = reinterpret_cast<float *>(ws);
    p.part_ml = reinterpret_cast<float *>(
        ws + (((size_t)(h.na + h.nb) * T * H_q * cda::kD * 4 + 255) & ~(size_t)255));
    if (h.na == 1 && h.nb == 1) {
        // No key split on either side: the chunk's keys go to partial slot 0,
        // then the unsplit prefix kernel merges that slot into its own result
        // before the epilogue (no prefix partials, no combine launch).
        p.causal = 1;
        p.key_range = kKeysChunk;
        p.ks_base = 0;
        p.n_ksplit = 1;
        p.ksplit_tiles = h.nb_tiles;
        p.k_rot = k_rot;
        p.v_rot = v_rot;
        p.cu_k = cu_seqlens_q;
        int rc = launch_prefill_kernel<false>(p, B, max_query_len, true, st, fn);
        if (rc != CDA_OK) return rc;
        p.causal = 0;
        p.key_range = kKeysPast;
        p.merge_slot0 = 1;
        return launch_prefill_kernel<true>(p, B, max_query_len, false, st, fn);
    }
    // The compressed prefix: every key precedes every query of the chunk.
    p.causal = 0;
    p.key_range = kKeysPast;
    p.ks_base = 0;
    p.n_ksplit = h.na;
    p.ksplit_tiles = h.na_tiles;
    int rc = launch_prefill_kernel<true>(p, B, max_query_len, true, st, fn);
    if (rc != CDA_OK) return rc;
    // The chunk's own keys, causal; dense rows of sequence b start at cu_q[b].
    p.causal = 1;
    p.key_range = kKeysChunk;
    p.ks_base = h.na;
    p.n_ksplit = h.nb;
    p.ksplit_tiles = h.nb_tiles;
    p.k_rot = k_rot;
    p.v_rot = v_rot;
    p.cu_k = cu_seqlens_q;
    rc = launch_prefill_kernel<false>(p, B, max_query_len, true, st, fn);
    if (rc != CDA_OK) return rc;
    return launch_combine(p, h.na + h.nb, B, st, fn);
}
