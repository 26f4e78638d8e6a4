/*
 * CPU restatement of the reference CDA algorithm -- TEST INFRASTRUCTURE ONLY.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load this library, and only as the checker.  The product (sub0_amd/) never
 * links or calls it.
 *
 * Reference functions restated here (file:line in the reference tree):
 *   hadamard_matrix          cda/algorithm/compression.py:43-57
 *   Compressor.rotate        cda/algorithm/compression.py:287-291
 *   Compressor.quantize_unit cda/algorithm/compression.py:298-313
 *   Compressor.encode        cda/algorithm/compression.py:315-335
 *   pack_4bit / pack_2bit    cda/algorithm/compression.py:163-179, 375-386
 *   Compressor.decode        cda/algorithm/compression.py:337-361
 *   attention_reference      cda/algorithm/attention.py:60-93
 *   attention_compressed     cda/algorithm/attention.py:426-482
 *   attention_partial_reference / merge_partials  attention.py:190-272
 *   causal_mask              cda/algorithm/attention.py:46-57
 *
 * Arithmetic contract of the encode (every rounding point and every
 * accumulation order follows the reference's CPU path, so the indices and
 * norms are bit-exact; tests/test_oracle_golden.py pins this against all of
 * the reference-written fixtures):
 *   1. x_rot_j = fp16(acc_j), acc_j the fp32 fused-multiply-add chain over
 *      k = 0..127 in order: acc = fmaf(x_k, H[k][j], acc) from acc = 0.  This
 *      is the accumulation order of the MKL sgemm behind
 *      torch.matmul(x.float(), H) for two or more rows (compression.py:290;
 *      a single-row matmul takes MKL's gemv, which rounds differently, but
 *      the paged encode always rotates H_kv >= 2 rows per token).
 *   2. norm: sq_j = fp32(x_j * x_j) (no fusion), eight lane accumulators
 *      a_l = sq_l + sq_{8+l} + ... + sq_{120+l} added in order, then
 *      s = a_0 + a_1 + ... + a_7 in order, norm = fp32 sqrt(s) correctly
 *      rounded, then clamp_min(1e-12f) (Tensor.norm(dim=-1) on the CPU,
 *      compression.py:328).
 *   3. x_unit = fp32(x_rot) / norm (IEEE fp32 division), clamp to [-1, 1]
 *      with NaN passing through (torch.clamp_ semantics).
 *   4. quantize exactly as compression.py:298-313 does in fp32:
 *      upper = #{i : !(cb[i] >= x)} (torch.bucketize, right=False; NaN -> L),
 *      upper = min(upper, L-1); lower = max(upper-1, 0);
 *      idx = |cb[upper]-x| < |x-cb[lower]| ? upper : lower (ties -> lower).
 *   5. pack MSB-first (4-bit: even dim in the high nibble; 2-bit: dim 4j at
 *      bits 7:6).
*/
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define D 128

/* ---------------------------------------------------------------- fp16 -- */

static float f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1Fu;
    uint32_t man = h & 0x3FFu;
    uint32_t bits;
    if (exp == 0) {
        if (man == 0) {
            bits = sign;
        } else { /* subnormal: value = man * 2^-24 */
            float v = (float)man * 5.9604644775390625e-8f;
            memcpy(&bits, &v, 4);
            bits |= sign;
        }
    } else if (exp == 31) {
        bits = sign | 0x7F800000u | (man << 13);
    } else {
        bits = sign | ((exp + 112u) << 23) | (man << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* Correctly rounded (nearest-even) float64 -> float16. */
uint16_t cda_oracle_f64_to_f16(double v) {
    uint64_t b;
    memcpy(&b, &v, 8);
    uint16_t sign = (uint16_t)((b >> 48) & 0x8000u);
    int e = (int)((b >> 52) & 0x7FF);
    uint64_t m = b & 0xFFFFFFFFFFFFFull;
    if (e == 0x7FF) return (uint16_t)(sign | 0x7C00u | (m ? 0x200u : 0u));
    if (e == 0 && m == 0) return sign;
    /* value = (1.m) * 2^(e-1023) for normal doubles (double subnormals are
       far below the fp16 range and round to zero). */
    if (e == 0) return sign;
    int ue = e - 1023;                    /* unbiased exponent */
    uint64_t sig = m | (1ull << 52);      /* 53-bit significand */
    if (ue > 15) return (uint16_t)(sign | 0x7C00u);
    int shift;                            /* bits to drop from sig */
    uint16_t hexp;
    if (ue >= -14) {                      /* normal fp16 */
        shift = 52 - 10;
        hexp = (uint16_t)(ue + 15);
    } else {                              /* subnormal fp16: unit 2^-24 */
        shift = 52 - 10 + (-14 - ue);
        hexp = 0;
        if (shift > 63) return sign;
    }
    uint64_t kept = sig >> shift;
    uint64_t rem = sig & ((1ull << shift) - 1);
    uint64_t half = 1ull << (shift - 1);
    if (rem > half || (rem == half && (kept & 1))) kept++;
    uint32_t out;
    if (hexp) {
        /* kept has 11 bits incl. hidden one; carry may bump the exponent */
        if (kept == (1ull << 11)) { kept >>= 1; hexp++; }
        if (hexp >= 31) return (uint16_t)(sign | 0x7C00u);
        out = ((uint32_t)hexp << 10) | (uint32_t)(kept & 0x3FFu);
    } else {
        out = (uint32_t)kept;             /* may round up into the first normal */
    }
    return (uint16_t)(sign | out);
}

uint16_t cda_oracle_f32_to_f16(float v) { return cda_oracle_f64_to_f16((double)v); }

float cda_oracle_f16_to_f32(uint16_t h) { return f16_to_f32(h); }

/* ----------------------------------------------------------- rotation -- */

static const uint32_t H32_BITS = 0x3db504f3u;   /* fp32(1/sqrt(128)) */

/* compression.py:43-57 -- the fp32 matrix the reference builds. */
void cda_oracle_hadamard128(float *H) {
    float h;
    memcpy(&h, &H32_BITS, 4);
    for (int i = 0; i < D; ++i)
        for (int j = 0; j < D; ++j)
            H[i * D + j] = (__builtin_popcount((unsigned)(i & j)) & 1) ? -h : h;
}

/* ----------------------------------------------------------- quantize -- */

/* compression.py:298-313 in fp32, torch.bucketize(right=False) semantics. */
static uint8_t quantize_one(float x, const float *cb, int L) {
    int upper = 0;
    for (int i = 0; i < L; ++i) upper += !(cb[i] >= x);
    if (upper > L - 1) upper = L - 1;
    int lower = upper - 1 < 0 ? 0 : upper - 1;
    float du = fabsf(cb[upper] - x);
    float dl = fabsf(x - cb[lower]);
    return (uint8_t)(du < dl ? upper : lower);
}

void cda_oracle_quantize(const float *x, int64_t n, const float *cb, int L, uint8_t *idx) {
    for (int64_t i = 0; i < n; ++i) idx[i] = quantize_one(x[i], cb, L);
}

/* Correctly rounded fp32 square root of a float64 value: move an
   approximation until the exact fp32 rounding midpoints (25-bit values whose
   squares are exact in float64) bracket x; ties go to even.  The HIP encoder
   takes the same midpoint test as one branch-free step from fp32(sqrt(x)),
   which is within one fp32 ulp of the answer. */
static float sqrt_f64_to_f32_rn(double x) {
    if (!(x > 0.0)) return x == 0.0 ? 0.0f : NAN;
    if (isinf(x)) return INFINITY;
    float f = (float)sqrt(x);
    for (int it = 0; it < 4; ++it) {
        float up = nextafterf(f, INFINITY);
        double mid = ((double)f + (double)up) * 0.5;
        double mm = mid * mid;
        uint32_t fb;
        memcpy(&fb, &f, 4);
        if (mm < x || (mm == x && (fb & 1))) { f = up; continue; }
        float dn = nextafterf(f, 0.0f);
        double midl = ((double)f + (double)dn) * 0.5;
        double ml = midl * midl;
        if (ml > x || (ml == x && (fb & 1))) { f = dn; continue; }
        break;
    }
    return f;
}

/* ------------------------------------------------------------- encode -- */

/* Encode `rows` vectors of 128 fp16 values (compression.py:315-335).
   bits = 4 (16 levels) or 2 (4 levels).  packed: rows x (128*bits/8) bytes.
   norm: rows fp32.  xrot (optional): rows x 128 fp16 bit patterns. */
void cda_oracle_encode_rows(const uint16_t *x, int64_t rows, const float *cb, int L,
                            uint8_t *packed, float *norm, uint16_t *xrot) {
    const int bits = (L == 16) ? 4 : 2;
    const int bpr = D * bits / 8;
    float hf;
    memcpy(&hf, &H32_BITS, 4);
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; ++r) {
        float xf[D];
        uint16_t xr[D];
        for (int i = 0; i < D; ++i) xf[i] = f16_to_f32(x[r * D + i]);
        for (int j = 0; j < D; ++j) {
            float acc = 0.0f;
            for (int k = 0; k < D; ++k) {
                const float hk = (__builtin_popcount((unsigned)(k & j)) & 1) ? -hf : hf;
                acc = fmaf(xf[k], hk, acc);
            }
            xr[j] = cda_oracle_f32_to_f16(acc);
        }
        if (xrot) memcpy(xrot + r * D, xr, sizeof(xr));
        float lanes[8];
        for (int l = 0; l < 8; ++l) {
            const float v = f16_to_f32(xr[l]);
            lanes[l] = v * v;
        }
        for (int c = 1; c < D / 8; ++c)
            for (int l = 0; l < 8; ++l) {
                const float v = f16_to_f32(xr[8 * c + l]);
                const float sq = v * v;
                lanes[l] = lanes[l] + sq;
            }
        float ss = lanes[0];
        for (int l = 1; l < 8; ++l) ss = ss + lanes[l];
        float nv = sqrt_f64_to_f32_rn((double)ss);
        if (nv < 1e-12f) nv = 1e-12f;    /* clamp_min(1e-12); NaN passes */
        norm[r] = nv;
        uint8_t idx[D];
        for (int j = 0; j < D; ++j) {
            float u = f16_to_f32(xr[j]) / nv;
            u = u < -1.0f ? -1.0f : (u > 1.0f ? 1.0f : u);
            idx[j] = quantize_one(u, cb, L);
        }
        uint8_t *out = packed + r * bpr;
        if (bits == 4) {
            for (int j = 0; j < bpr; ++j) out[j] = (uint8_t)((idx[2 * j] << 4) | idx[2 * j + 1]);
        } else {
            for (int j = 0; j < bpr; ++j)
                out[j] = (uint8_t)((idx[4 * j] << 6) | (idx[4 * j + 1] << 4) |
                                   (idx[4 * j + 2] << 2) | idx[4 * j + 3]);
        }
    }
}

/* --------------------------------------------------------- decode rows -- */

static void unpack_row(const uint8_t *p, int bits, uint8_t *idx) {
    if (bits == 4) {
        for (int j = 0; j < D / 2; ++j) { idx[2 * j] = p[j] >> 4; idx[2 * j + 1] = p[j] & 15; }
    } else {
        for (int j = 0; j < D / 4; ++j) {
            idx[4 * j] = (p[j] >> 6) & 3; idx[4 * j + 1] = (p[j] >> 4) & 3;
            idx[4 * j + 2] = (p[j] >> 2) & 3; idx[4 * j + 3] = p[j] & 3;
        }
    }
}

/* compression.py:337-361 with rotated=True: fp16(cb[idx] * norm), the
   multiply in fp32. */
static void decode_row(const uint8_t *p, float nrm, const float *cb, int bits, float *out) {
    uint8_t idx[D];
    unpack_row(p, bits, idx);
    for (int j = 0; j < D; ++j) out[j] = f16_to_f32(cda_oracle_f32_to_f16(cb[idx[j]] * nrm));
}

void cda_oracle_decode_rows(const uint8_t *packed, const float *norm, int64_t rows,
                            const float *cb, int L, uint16_t *out) {
    const int bits = (L == 16) ? 4 : 2;
    const int bpr = D * bits / 8;
    for (int64_t r = 0; r < rows; ++r) {
        float v[D];
        decode_row(packed + r * bpr, norm[r], cb, bits, v);
        for (int j = 0; j < D; ++j) out[r * D + j] = cda_oracle_f32_to_f16(v[j]);
    }
}

/* ------------------------------------------------- paged decode attention -- */

/* Slot layout (cda_attn_v2.py:20-29, generalised to 2-bit codes):
   [K codes kbk | V codes kbv | K norm f32 | V norm f32 | pad], kb = 128*bits/8:
   K4V4 64 | 64 (144-byte slots), K2V2 32 | 32, K4V2 64 | 32 (the legacy
   104-byte slot).  The level argument L of the paged functions below is the
   K codebook size, with the V codebook size in bits 8..15 when it differs. */
typedef struct {
    const uint8_t *kv;
    int64_t row_bytes;   /* H_kv * slot_bytes */
    int slot_bytes;
    int kbk, kbv;
    int bitsk, bitsv;
} cache_view;

static void init_view(cache_view *c, const uint8_t *kv, int H_kv, int slot_bytes, int L) {
    const int lk = L & 0xFF, lv = (L >> 8) ? (L >> 8) : lk;
    c->kv = kv;
    c->slot_bytes = slot_bytes;
    c->row_bytes = (int64_t)H_kv * slot_bytes;
    c->bitsk = lk == 16 ? 4 : 2;
    c->bitsv = lv == 16 ? 4 : 2;
    c->kbk = D * c->bitsk / 8;
    c->kbv = D * c->bitsv / 8;
}

static const uint8_t *slot_ptr(const cache_view *c, int64_t slot, int h) {
    return c->kv + slot * c->row_bytes + (int64_t)h * c->slot_bytes;
}

static float load_f32(const uint8_t *p) { float f; memcpy(&f, p, 4); return f; }

/* q_rot = fp16(fp32(q @ R)) with the sum in float64 (compression.py:287-291). */
static void rotate_q(const uint16_t *q, const float *R, float *qr) {
    for (int j = 0; j < D; ++j) {
        double s = 0.0;
        for (int k = 0; k < D; ++k) s += (double)f16_to_f32(q[k]) * (double)R[k * D + j];
        qr[j] = f16_to_f32(cda_oracle_f32_to_f16((float)s));
    }
}

/* Decode the keys/values [k0, k1) of sequence b / kv head h into fp16-valued
   float arrays (compression.py:337-361 with rotated=True). */
static void decode_window(const cache_view *c, const int32_t *bt_row, int block_size, int h,
                          int k0, int k1, const float *cbK, const float *cbV, float *K, float *V) {
    for (int t = k0; t < k1; ++t) {
        int64_t slot = (int64_t)bt_row[t / block_size] * block_size + t % block_size;
        const uint8_t *p = slot_ptr(c, slot, h);
        const uint8_t *nrm = p + c->kbk + c->kbv;
        decode_row(p, load_f32(nrm), cbK, c->bitsk, K + (int64_t)(t - k0) * D);
        decode_row(p + c->kbk, load_f32(nrm + 4), cbV, c->bitsv, V + (int64_t)(t - k0) * D);
    }
}

/* Attention of one rotated query over n decoded keys: the split-K partial of
   attention.py:190-236 (o_un, m in the natural-log domain, l), float64
   accumulation.  Causal masking is done by the caller through n. */
static void partial_one(const float *qr, const float *K, const float *V, int n, float scale,
                        double *o_un, double *m_out, double *l_out) {
    double m = -INFINITY, l = 0.0;
    for (int j = 0; j < D; ++j) o_un[j] = 0.0;
    if (n <= 0) { *m_out = m; *l_out = l; return; }
    double *s = (double *)malloc(sizeof(double) * (size_t)n);
    for (int t = 0; t < n; ++t) {
        double acc = 0.0;
        const float *kd = K + (int64_t)t * D;
        for (int j = 0; j < D; ++j) acc += (double)qr[j] * (double)kd[j];
        s[t] = acc * (double)scale;
        if (s[t] > m) m = s[t];
    }
    for (int t = 0; t < n; ++t) {
        double pr = exp(s[t] - m);
        const float *vd = V + (int64_t)t * D;
        l += pr;
        for (int j = 0; j < D; ++j) o_un[j] += pr * (double)vd[j];
    }
    free(s);
    *m_out = m;
    *l_out = l;
}

static void finish_row(const double *o, double l, const float *R, int rotated_io, uint16_t *ov) {
    float orot[D];
    double den = l > 1e-30 ? l : 1e-30;
    for (int j = 0; j < D; ++j) orot[j] = f16_to_f32(cda_oracle_f32_to_f16((float)(o[j] / den)));
    if (rotated_io) {
        for (int j = 0; j < D; ++j) ov[j] = cda_oracle_f32_to_f16(orot[j]);
    } else {
        for (int j = 0; j < D; ++j) {
            double acc = 0.0;
            for (int k = 0; k < D; ++k) acc += (double)orot[k] * (double)R[j * D + k];
            ov[j] = cda_oracle_f32_to_f16((float)acc);
        }
    }
}

/* Decode attention over a paged cache: the full oracle path of
   attention_compressed (attention.py:426-482) for M_q = 1, i.e.
   q_rot = fp16(q @ R); O_rot = fp16(softmax(q_rot K^T * scale) V);
   out = fp16(O_rot @ R^T).  With rotated_io != 0 the rotations are skipped
   (q is already rotated and out stays rotated).  K and V of each (b, kv head)
   are decoded once and shared by the GQA group, as the reference does.
   q: (B, H_q, 128) fp16; out: (B, H_q, 128) fp16. */
void cda_oracle_decode_paged(const uint16_t *q, const uint8_t *kv, int H_kv, int slot_bytes,
                             int L, const int32_t *block_table, int max_blocks,
                             const int32_t *seq_lens, int B, int H_q, int block_size,
                             const float *cbK, const float *cbV, const float *R, float scale,
                             int rotated_io, uint16_t *out) {
    cache_view c;
    init_view(&c, kv, H_kv, slot_bytes, L);
    const int g = H_q / H_kv;
#pragma omp parallel for collapse(2) schedule(dynamic)
    for (int b = 0; b < B; ++b)
        for (int h = 0; h < H_kv; ++h) {
            int n = seq_lens[b];
            float *K = (float *)malloc(sizeof(float) * (size_t)(n > 0 ? n : 1) * D);
            float *V = (float *)malloc(sizeof(float) * (size_t)(n > 0 ? n : 1) * D);
            decode_window(&c, block_table + (int64_t)b * max_blocks, block_size, h, 0, n, cbK,
                          cbV, K, V);
            for (int gi = 0; gi < g; ++gi) {
                int hq = h * g + gi;
                const uint16_t *qv = q + ((int64_t)b * H_q + hq) * D;
                float qr[D];
                if (rotated_io) {
                    for (int j = 0; j < D; ++j) qr[j] = f16_to_f32(qv[j]);
                } else {
                    rotate_q(qv, R, qr);
                }
                double o[D], m, l;
                partial_one(qr, K, V, n, scale, o, &m, &l);
                finish_row(o, l, R, rotated_io, out + ((int64_t)b * H_q + hq) * D);
            }
            free(K);
            free(V);
        }
}

/* Split-K partials (attention.py:190-236, 349-384) for M_q = 1 in the rotated
   frame: for each (b, hq) the keys [k0, min(k1, seq_len)).  o_un: (B,H_q,128)
   fp32, m/l: (B,H_q) fp32, natural-log domain. */
void cda_oracle_decode_partial(const uint16_t *q_rot, const uint8_t *kv, int H_kv, int slot_bytes,
                               int L, const int32_t *block_table, int max_blocks,
                               const int32_t *seq_lens, int B, int H_q, int block_size,
                               const float *cbK, const float *cbV, float scale, int k0, int k1,
                               float *o_un, float *m_out, float *l_out) {
    cache_view c;
    init_view(&c, kv, H_kv, slot_bytes, L);
    const int g = H_q / H_kv;
    for (int b = 0; b < B; ++b)
        for (int h = 0; h < H_kv; ++h) {
            int e = k1 < seq_lens[b] ? k1 : seq_lens[b];
            int n = e - k0;
            float *K = (float *)malloc(sizeof(float) * (size_t)(n > 0 ? n : 1) * D);
            float *V = (float *)malloc(sizeof(float) * (size_t)(n > 0 ? n : 1) * D);
            if (n > 0)
                decode_window(&c, block_table + (int64_t)b * max_blocks, block_size, h, k0, e,
                              cbK, cbV, K, V);
            for (int gi = 0; gi < g; ++gi) {
                int hq = h * g + gi;
                float qr[D];
                for (int j = 0; j < D; ++j)
                    qr[j] = f16_to_f32(q_rot[((int64_t)b * H_q + hq) * D + j]);
                double o[D], m, l;
                partial_one(qr, K, V, n, scale, o, &m, &l);
                for (int j = 0; j < D; ++j) o_un[((int64_t)b * H_q + hq) * D + j] = (float)o[j];
                m_out[b * H_q + hq] = (float)m;
                l_out[b * H_q + hq] = (float)l;
            }
            free(K);
            free(V);
        }
}

/* Causal varlen prefill over the paged cache (attention.py:60-93 with the
   lower-right mask of :46-57): query token i of sequence b (cu_q[b] <= row <
   cu_q[b+1], M_b = cu_q[b+1]-cu_q[b]) attends keys [0, seq_lens[b] - M_b + i].
   q: (T, H_q, 128) fp16 unrotated; out: (T, H_q, 128) fp16 unrotated. */
void cda_oracle_prefill_paged(const uint16_t *q, const int32_t *cu_q, const uint8_t *kv, int H_kv,
                              int slot_bytes, int L, const int32_t *block_table, int max_blocks,
                              const int32_t *seq_lens, int B, int H_q, int block_size,
                              const float *cbK, const float *cbV, const float *R, float scale,
                              uint16_t *out) {
    cache_view c;
    init_view(&c, kv, H_kv, slot_bytes, L);
    const int g = H_q / H_kv;
    for (int b = 0; b < B; ++b) {
        int M = cu_q[b + 1] - cu_q[b];
        int n = seq_lens[b];
        int off = n - M;
        for (int h = 0; h < H_kv; ++h) {
            float *K = (float *)malloc(sizeof(float) * (size_t)(n > 0 ? n : 1) * D);
            float *V = (float *)malloc(sizeof(float) * (size_t)(n > 0 ? n : 1) * D);
            decode_window(&c, block_table + (int64_t)b * max_blocks, block_size, h, 0, n, cbK,
                          cbV, K, V);
#pragma omp parallel for collapse(2) schedule(dynamic)
            for (int i = 0; i < M; ++i)
                for (int gi = 0; gi < g; ++gi) {
                    int hq = h * g + gi;
                    int64_t row = cu_q[b] + i;
                    float qr[D];
                    rotate_q(q + (row * H_q + hq) * D, R, qr);
                    int kend = off + i + 1;
                    if (kend > n) kend = n;
                    double o[D], m, l;
                    partial_one(qr, K, V, kend, scale, o, &m, &l);
                    finish_row(o, l, R, 0, out + (row * H_q + hq) * D);
                }
            free(K);
            free(V);
        }
    }
}

void cda_oracle_set_threads(int n) {
#ifdef _OPENMP
    omp_set_num_threads(n > 0 ? n : 1);
#else
    (void)n;
#endif
}
