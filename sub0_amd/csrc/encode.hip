// Fused paged encode: Hadamard-128 + norm + nearest centroid + pack + scatter
// into the paged slot layout (gfx950).
//
// Reference contract: cda_paged_encode_fused as bound by
// cda/kernels_cuda/wrappers.py:127-156; arithmetic of Compressor.encode
// (cda/algorithm/compression.py:287-335) and pack_4bit / pack_2bit
// (:163-179, :375-386).  The result is bit-identical to the reference's CPU
// path, which fixes three orders:
//
//  * rotation (compression.py:290-291): x_rot_j = fp16(acc_j) with acc_j the
//    fp32 fused-multiply-add chain over k = 0..127 in order,
//    acc = fma(x_k, H[k][j], acc), H[k][j] = (-1)^popcount(k & j) * h,
//    h = fp32(1/sqrt(128)) (the order of the MKL sgemm behind torch.matmul);
//  * norm (:328): eight lane sums a_l = sq_l + sq_{8+l} + ... + sq_{120+l}
//    with sq_j = fp32(x_j * x_j), then a_0 + ... + a_7 in order, a correctly
//    rounded fp32 square root, clamp_min(1e-12);
//  * x_unit = fp32(x_rot / norm), clamp to [-1, 1], then the bucketize +
//    neighbour compare of quantize_unit (:298-313) in fp32.
//
// Work layout.  P lanes share one 128-vector (P = 4 for throughput, 16 for
// small batches); lane r of a group owns the outputs j = r + P*m,
// m = 0..128/P-1.  The chains of outputs that agree in the low bits of j
// agree in their first steps: (-1)^popcount(k & j) depends only on the bits
// of j below the highest set bit of k, so for k < 2^t the chains of j and
// j + 2^t are equal.  Each lane therefore runs its chains as a binary tree:
// one chain for k < P (the lane's own sign pattern s(k & r) sits in P
// registers of signed h), which splits in two at k = P, 2P, ..., 64.  That is
// 2^7 - ... ~ 2731 fused multiply-adds per lane for P = 4 (10924 per vector,
// against 16384 for 128 independent chains), every one an exact IEEE fma
// with the sign folded into the operand, so the chain rounds exactly as the
// reference's.
//
// Quantisation without a division.  For a sorted codebook the reference's
// index is monotone in u = RN32(x / n): it equals #{i in 1..L-1 : u >= th_i}
// where th_i is the smallest fp32 in (cb[i-1], cb[i]] for which
// |RN(cb[i] - u)| < |RN(u - cb[i-1])| (found once per block by bisection over
// the ordered fp32 bit patterns).  RN32(x / n) >= th holds exactly when
// x / n >= beta (th even) or x / n > beta (th odd), beta the midpoint of th
// and its fp32 predecessor; x / n >= beta <=> x >= n * beta, and n * beta
// (24 x 25 significant bits) is exact in float64.  So each vector gets L-1
// thresholds in the x domain (rounded up to fp32, where every fp16 x lives)
// and each element a four-step bisection of compares.  Non-finite norms
// (an fp16 overflow in x_rot, or NaN input) take the reference's formula
// with a true division.
#include "cda_common.h"

namespace cda {

namespace {

struct EncodeParams {
    const uint16_t *k;
    const uint16_t *v;
    int64_t k_stride;      // elements between tokens
    int64_t v_stride;
    const int32_t *slot_mapping;
    int64_t num_tokens;
    uint8_t *cache;
    int64_t num_slots;
    int64_t row_bytes;     // H_kv * slot_bytes
    int slot_bytes;
    int H_kv;
    const float *cb_k;
    const float *cb_v;
};

constexpr int kEncWaves = 4;          // waves 2q, 2q+1: K and V of item group q

// Ordered-integer image of an fp32 value (monotone in the value; -0 < +0).
__device__ __forceinline__ uint32_t f2key(float f) {
    const uint32_t b = __float_as_uint(f);
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
__device__ __forceinline__ float key2f(uint32_t k) {
    return __uint_as_float((k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k);
}

// The neighbour compare of quantize_unit for u in bucket i (lo < u <= hi):
// true picks the upper centroid.
__device__ __forceinline__ bool pick_upper(float u, float lo, float hi) {
    return fabsf(__fsub_rn(hi, u)) < fabsf(__fsub_rn(u, lo));
}

// Decision threshold i (1 <= i < L) of a sorted codebook in the u domain,
// expressed as (beta, strict): clamp(u) selects at least level i exactly when
// u >= beta (u > beta when strict), for every u = RN32(v) with v real.
// Thresholds at or below -1 always hold after the clamp (beta = -inf);
// thresholds above 1 never do (beta = +inf).
__device__ void codebook_threshold(const float *cb, int i, double *beta, int *strict) {
    const float lo = cb[i - 1], hi = cb[i];
    uint32_t a = f2key(lo) + 1u, b = f2key(hi);
    if (a <= b) {
        while (a < b) {
            const uint32_t mid = a + ((b - a) >> 1);
            if (pick_upper(key2f(mid), lo, hi)) b = mid; else a = mid + 1u;
        }
    }
    // a: the smallest fp32 above lo that selects i (an empty bucket, lo == hi,
    // gives nextup(hi): only values above hi select it, as in the reference).
    const float th = key2f(a);
    if (th <= -1.0f) { *beta = -__builtin_inf(); *strict = 0; return; }
    if (th > 1.0f) { *beta = __builtin_inf(); *strict = 0; return; }
    uint32_t pk = a - 1u;
    if (__float_as_uint(key2f(pk)) == 0x80000000u && __float_as_uint(th) == 0u) pk -= 1u;  // pred(+0)
    *beta = ((double)key2f(pk) + (double)th) * 0.5;
    *strict = (int)(__float_as_uint(th) & 1u);
}

// Smallest fp32 >= t (t finite or infinite).
__device__ __forceinline__ float round_up_f32(double t) {
    float f = (float)t;
    if ((double)f < t) f = __uint_as_float(__float_as_uint(f) + (f >= 0.0f ? 1u : 0xFFFFFFFFu));
    return f;
}

// Next float64 above t (t finite, non-zero).
__device__ __forceinline__ double next_up(double t) {
    const long long b = __double_as_longlong(t);
    return __longlong_as_double(t > 0.0 ? b + 1 : b - 1);
}

// The reference's quantize_unit on one fp32 value (compression.py:298-313):
// only used for vectors with a non-finite norm.
template <int L>
__device__ uint32_t quantize_ref(float u, const float *cb) {
    int upper = 0;
#pragma unroll
    for (int i = 0; i < L; ++i) upper += !(cb[i] >= u) ? 1 : 0;
    upper = upper > L - 1 ? L - 1 : upper;
    const int lower = upper - 1 < 0 ? 0 : upper - 1;
    const float du = fabsf(__fsub_rn(cb[upper], u));
    const float dl = fabsf(__fsub_rn(u, cb[lower]));
    return (uint32_t)(du < dl ? upper : lower);
}

// #{i : x >= thr[i]} for the sorted thresholds thr[1..L-1] of this vector,
// by bisection with the thresholds read from LDS at computed indices (tmid =
// thr[L/2] in a register): one compare, one add and one LDS read per level
// (register selects among the thresholds measured 5 % slower for K4V4).
template <int L>
__device__ __forceinline__ uint32_t count_ge_lds(float x, const float *thr, float tmid) {
    if constexpr (L == 16) {
        uint32_t c = x >= tmid ? 8u : 0u;
        c += x >= thr[c + 4] ? 4u : 0u;
        c += x >= thr[c + 2] ? 2u : 0u;
        c += x >= thr[c + 1] ? 1u : 0u;
        return c;
    } else {
        static_assert(L == 4, "4 or 16 levels");
        uint32_t c = x >= tmid ? 2u : 0u;
        c += x >= thr[c + 1] ? 1u : 0u;
        return c;
    }
}

template <int P>
struct EncLayout {
    static constexpr int V = 64 / P;          // vectors per wave
    static constexpr int M = kD / P;          // outputs per lane
    static constexpr int kPitch = kD + P;     // floats per vector row in LDS (bank spread)
    // per wave: V rows of sq / idx, then V x 16 thresholds, V x 8 lane sums
    static constexpr int kThrPitch = 17;      // thresholds per vector (bank spread)
    static constexpr int kWaveFloats = V * kPitch + V * kThrPitch + V * 8;
};

template <int LK, int LV, int P>
__global__ void __launch_bounds__(64 * kEncWaves)
paged_encode_kernel(EncodeParams p) {
    using Lay = EncLayout<P>;
    constexpr int V = Lay::V, M = Lay::M, PITCH = Lay::kPitch;
    // Slot: [K codes KBK | V codes KBV | K norm | V norm | pad].
    constexpr int KBK = kD * (LK == 16 ? 4 : 2) / 8;
    constexpr int KBV = kD * (LV == 16 ? 4 : 2) / 8;
    __shared__ double s_beta[2][16];
    __shared__ int s_strict[2][16];
    __shared__ float s_cb[2][16];
    __shared__ float s_w[kEncWaves][Lay::kWaveFloats];

    if (threadIdx.x < 32) {
        const int r = threadIdx.x / 16, i = threadIdx.x % 16;
        const float *cb = r ? p.cb_v : p.cb_k;
        if (i < (r ? LV : LK)) {
            s_cb[r][i] = cb[i];
            if (i > 0) codebook_threshold(cb, i, &s_beta[r][i], &s_strict[r][i]);
        }
    }
    __syncthreads();

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int role = wave & 1;                        // wave-uniform: 0 = K, 1 = V
    const int g = lane / P, r = lane % P;
    float *sq_row = s_w[wave] + g * PITCH;            // this vector's 128 floats
    float *thr = s_w[wave] + V * PITCH + g * Lay::kThrPitch;
    float *lsum = s_w[wave] + V * PITCH + V * Lay::kThrPitch + g * 8;

    // (token, head) item of this lane group; fewer than 2^31 items (host check).
    const uint32_t items = (uint32_t)(p.num_tokens * p.H_kv);
    const uint32_t item = blockIdx.x * (uint32_t)(V * kEncWaves / 2) +
                          (uint32_t)(wave >> 1) * (uint32_t)V + (uint32_t)g;
    const bool valid = item < items;
    const uint32_t t32 = valid ? item / (uint32_t)p.H_kv : 0u;
    const int h = valid ? (int)(item - t32 * (uint32_t)p.H_kv) : 0;
    const int64_t t = t32;

    // ---- load the vector (all P lanes of the group read the same 256 B) ----
    // Kept as packed fp16 pairs; each x_k is widened to fp32 once, where the
    // chains use it (xf below).
    uint32_t xw[kD / 2];
    {
        const uint16_t *src = role == 0 ? p.k + t * p.k_stride + (int64_t)h * kD
                                        : p.v + t * p.v_stride + (int64_t)h * kD;
        const uint4 *s4 = reinterpret_cast<const uint4 *>(src);
#pragma unroll
        for (int q = 0; q < kD / 8; ++q) {
            uint4 w = make_uint4(0, 0, 0, 0);
            if (valid) w = s4[q];
            xw[4 * q + 0] = w.x;
            xw[4 * q + 1] = w.y;
            xw[4 * q + 2] = w.z;
            xw[4 * q + 3] = w.w;
        }
    }
    // x_k in fp32 (exact).  The empty asm makes the widened value opaque, so
    // the compiler cannot fold the conversion into every fma that uses it
    // (v_fma_mix_f32, about twice the issue cost of v_fma_f32 on gfx950).
    auto xf = [&](int k) CDA_INLINE -> float {
        float v = h2f((uint16_t)((k & 1) ? (xw[k >> 1] >> 16) : (xw[k >> 1] & 0xFFFFu)));
        asm volatile("" : "+v"(v));
        return v;
    };

    // ---- rotation: the fma chains as a tree ---------------------------------
    const float hval = __int_as_float(0x3db504f3);    // fp32(1/sqrt(128))
    float hs[P];                                      // s(k & r) * h for k mod P
#pragma unroll
    for (int q = 0; q < P; ++q) hs[q] = (__popc((uint32_t)(q & r)) & 1) ? -hval : hval;
    float ch[M];
    {
        float c = 0.0f;
#pragma unroll
        for (int k = 0; k < P; ++k) c = fmaf(xf(k), hs[k], c);
        ch[0] = c;
    }
#pragma unroll
    for (int lvl = 0; (P << lvl) < kD; ++lvl) {
        const int cnt = 1 << lvl;                     // chains so far (m mod cnt)
        const int k0 = P << lvl;                      // steps k0 .. 2 k0 - 1
#pragma unroll
        for (int m = 0; m < cnt; ++m) ch[m + cnt] = ch[m];
#pragma unroll
        for (int k = k0; k < 2 * k0; ++k) {
            const float xk = xf(k);
#pragma unroll
            for (int m = 0; m < 2 * cnt; ++m) {
                const bool neg = (__builtin_popcount((unsigned)(k & (P * m))) & 1) != 0;
                ch[m] = fmaf(xk, neg ? -hs[k % P] : hs[k % P], ch[m]);
            }
        }
    }

    // ---- fp16 rounding, squares, norm (reference order) ---------------------
    float xr[M];
#pragma unroll
    for (int m = 0; m < M; ++m) {
        // The fp32 chain value is rounded on its own, then to fp16 (the
        // reference rounds its fp32 matmul output to the input dtype); the
        // empty asm keeps the compiler from fusing the last fma with the fp16
        // conversion into one rounding (v_fma_mixlo_f16).
        asm volatile("" : "+v"(ch[m]));
        xr[m] = __half2float(__float2half_rn(ch[m]));
        sq_row[r + P * m] = __fmul_rn(xr[m], xr[m]);
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
    for (int l0 = 0; l0 < 8; l0 += P) {
        const int l = l0 + r;
        if (l < 8) {
            float a = sq_row[l];
#pragma unroll
            for (int c = 1; c < kD / 8; ++c) a = __fadd_rn(a, sq_row[8 * c + l]);
            lsum[l] = a;
        }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    float ss = lsum[0];
#pragma unroll
    for (int l = 1; l < 8; ++l) ss = __fadd_rn(ss, lsum[l]);
    float n = sqrt_f64_to_f32_rn((double)ss);
    n = (n < 1e-12f) ? 1e-12f : n;                    // clamp_min(1e-12); NaN passes

    // ---- thresholds, quantisation, packing and the store, for this role's
    // codebook (K: LK levels, V: LV levels; wave-uniform branch).
    auto finish = [&](auto levels) CDA_INLINE {
        constexpr int L = decltype(levels)::value;
        constexpr int KB = kD * (L == 16 ? 4 : 2) / 8;   // code bytes of this role
        // ---- per-vector thresholds in the x domain ------------------------------
        const bool finite_n = fabsf(n) < __builtin_inff();
    #pragma unroll
        for (int i0 = 1; i0 < L; i0 += P) {
            const int i = i0 + r;
            if (i < L) {
                const double beta = s_beta[role][i];
                double tt = (double)n * beta;             // exact: 24 x 25 significant bits
                if (s_strict[role][i] && finite_n) tt = next_up(tt);
                thr[i] = round_up_f32(tt);
            }
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

        // ---- quantise; codes go through LDS (the sq row is free again) ----------
        uint8_t *idx_row = reinterpret_cast<uint8_t *>(sq_row);
        uint32_t code[M];
        if (finite_n) {
            const float tmid = thr[L / 2];
    #pragma unroll
            for (int m = 0; m < M; ++m) code[m] = count_ge_lds<L>(xr[m], thr, tmid);
        } else {
    #pragma unroll
            for (int m = 0; m < M; ++m) {
                float u = __fdiv_rn(xr[m], n);
                u = u < -1.0f ? -1.0f : (u > 1.0f ? 1.0f : u);
                code[m] = quantize_ref<L>(u, s_cb[role]);
            }
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();                  // lane sums read before the row is reused
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    #pragma unroll
        for (int m = 0; m < M; ++m) idx_row[r + P * m] = (uint8_t)code[m];
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

        if (!valid) return;
        const int64_t slot = p.slot_mapping[t];
        if (slot < 0 || slot >= p.num_slots) return;
        uint8_t *dst = p.cache + slot * p.row_bytes + (int64_t)h * p.slot_bytes;
        uint8_t *codes = dst + (role ? KBK : 0);
        // Lane r packs code bytes [r * KB / P, (r + 1) * KB / P).
        constexpr int BPL = KB / P;                        // bytes per lane: 16/4 (K4) or 8/2 (K2)
        constexpr int EPB = L == 16 ? 2 : 4;               // elements per byte
        const uint32_t *src = reinterpret_cast<const uint32_t *>(idx_row + r * BPL * EPB);
        uint32_t packed[(BPL + 3) / 4];
    #pragma unroll
        for (int w = 0; w < (BPL + 3) / 4; ++w) packed[w] = 0;
    #pragma unroll
        for (int b = 0; b < BPL; ++b) {
            uint32_t byte;
            if constexpr (L == 16) {
                const uint32_t e = src[b / 2] >> (16 * (b & 1));      // elements 2b, 2b+1
                byte = ((e & 0xFu) << 4) | ((e >> 8) & 0xFu);
            } else {
                const uint32_t e = src[b];                           // elements 4b .. 4b+3
                byte = ((e & 3u) << 6) | (((e >> 8) & 3u) << 4) | (((e >> 16) & 3u) << 2) |
                       ((e >> 24) & 3u);
            }
            packed[b / 4] |= byte << (8 * (b & 3));
        }
        if constexpr (BPL >= 4) {
    #pragma unroll
            for (int w = 0; w < BPL / 4; ++w)
                reinterpret_cast<uint32_t *>(codes + r * BPL)[w] = packed[w];
        } else {
            *reinterpret_cast<uint16_t *>(codes + r * BPL) = (uint16_t)packed[0];
        }
        if (r == 0) *reinterpret_cast<float *>(dst + KBK + KBV + 4 * role) = n;

    };
    if (role == 0) finish(std::integral_constant<int, LK>{});
    else finish(std::integral_constant<int, LV>{});
}

template <int LK, int LV, int P>
void launch_encode(const EncodeParams &p, int64_t items, hipStream_t st) {
    constexpr int per_block = (64 / P) * kEncWaves / 2;          // items per block
    const int64_t blocks = (items + per_block - 1) / per_block;
    paged_encode_kernel<LK, LV, P><<<dim3((unsigned)blocks), 64 * kEncWaves, 0, st>>>(p);
}

}  // namespace

}  // namespace cda

using namespace cda;

namespace cda {
namespace {
int encode_impl(const void *k, const void *v, int64_t k_stride, int64_t v_stride,
                const int32_t *slot_mapping, int64_t num_tokens, void *flat_cache,
                int64_t num_slots, int slot_bytes, int H_kv, const float *cb_k, const float *cb_v,
                int levels_k, int levels_v, void *stream, const char *fn) {
    const std::string f(fn);
    CDA_REQUIRE(num_tokens >= 0, f + ": num_tokens must be >= 0");
    if (num_tokens == 0) return CDA_OK;
    CDA_REQUIRE(k && v && slot_mapping && flat_cache && cb_k && cb_v, f + ": null pointer argument");
    CDA_REQUIRE(H_kv > 0 && num_slots > 0, f + ": H_kv and num_slots must be > 0");
    const int kbk = kD * (levels_k == 16 ? 4 : 2) / 8;
    const int kbv = kD * (levels_v == 16 ? 4 : 2) / 8;
    CDA_REQUIRE(slot_bytes >= kbk + kbv + 8, f + ": slot_bytes too small for the layout");
    CDA_REQUIRE(k_stride >= (int64_t)H_kv * kD && v_stride >= (int64_t)H_kv * kD,
                f + ": token stride smaller than H_kv * 128");
    CDA_REQUIRE(((uintptr_t)k & 3) == 0 && ((uintptr_t)v & 3) == 0 && slot_bytes % 4 == 0 &&
                    ((uintptr_t)flat_cache & 3) == 0,
                f + ": k, v, cache must be 4-byte aligned");
    EncodeParams p;
    p.k = static_cast<const uint16_t *>(k);
    p.v = static_cast<const uint16_t *>(v);
    p.k_stride = k_stride;
    p.v_stride = v_stride;
    p.slot_mapping = slot_mapping;
    p.num_tokens = num_tokens;
    p.cache = static_cast<uint8_t *>(flat_cache);
    p.num_slots = num_slots;
    p.row_bytes = (int64_t)H_kv * slot_bytes;
    p.slot_bytes = slot_bytes;
    p.H_kv = H_kv;
    p.cb_k = cb_k;
    p.cb_v = cb_v;
    const int64_t items = num_tokens * H_kv;
    CDA_REQUIRE(items < ((int64_t)1 << 31), f + ": too many tokens x heads");
    hipStream_t st = static_cast<hipStream_t>(stream);
    // Four lanes per vector run the fewest instructions per vector; sixteen
    // finish a wave four times sooner.  Take 16 while the 4-lane grid would
    // leave the SIMDs with fewer than two waves each.
    const bool wide = items * 2 / 16 < 2048;
    if (levels_k == 16 && levels_v == 16) {
        if (wide) launch_encode<16, 16, 16>(p, items, st); else launch_encode<16, 16, 4>(p, items, st);
    } else if (levels_k == 4 && levels_v == 4) {
        if (wide) launch_encode<4, 4, 16>(p, items, st); else launch_encode<4, 4, 4>(p, items, st);
    } else {
        if (wide) launch_encode<16, 4, 16>(p, items, st); else launch_encode<16, 4, 4>(p, items, st);
    }
    CDA_LAUNCH_CHECK(f + ": paged_encode_kernel");
    return CDA_OK;
}
}  // namespace
}  // namespace cda

extern "C" int cda_paged_encode_fused(const void *k, const void *v, int64_t k_stride,
                                      int64_t v_stride, const int32_t *slot_mapping,
                                      int64_t num_tokens, void *flat_cache, int64_t num_slots,
                                      int slot_bytes, int H_kv, const float *cb_k,
                                      const float *cb_v, int levels, void *stream) {
    CDA_REQUIRE(levels == 16 || levels == 4, "cda_paged_encode_fused: levels must be 16 or 4");
    return encode_impl(k, v, k_stride, v_stride, slot_mapping, num_tokens, flat_cache, num_slots,
                       slot_bytes, H_kv, cb_k, cb_v, levels, levels, stream,
                       "cda_paged_encode_fused");
}

extern "C" int cda_paged_encode_fused_k4v2(const void *k, const void *v, int64_t k_stride,
                                           int64_t v_stride, const int32_t *slot_mapping,
                                           int64_t num_tokens, void *flat_cache,
                                           int64_t num_slots, int slot_bytes, int H_kv,
                                           const float *cb_k, const float *cb_v, void *stream) {
    return encode_impl(k, v, k_stride, v_stride, slot_mapping, num_tokens, flat_cache, num_slots,
                       slot_bytes, H_kv, cb_k, cb_v, 16, 4, stream, "cda_paged_encode_fused_k4v2");
}
