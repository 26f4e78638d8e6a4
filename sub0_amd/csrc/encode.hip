// Fused paged encode: Hadamard-128 + norm + nearest centroid + pack + scatter
// into the paged slot layout (gfx950).
//
// Reference contract: cda_paged_encode_fused as bound by
// cda/kernels_cuda/wrappers.py:127-156; arithmetic of Compressor.encode
// (cda/algorithm/compression.py:287-335) and pack_4bit / pack_2bit
// (:163-179, :375-386).
//
// A 16-lane row of a wave encodes one 128-vector: lane j holds elements
// 8j..8j+7 (one 16-byte load), so the first three butterfly stages and the
// first three levels of the norm tree stay in registers; an LDS transpose
// turns three of the other four butterfly stages into register stages, one
// crosses lanes (DPP within the row), as do four levels of the norm tree; a
// wave encodes four vectors of one role (K or V).  The butterfly runs in float64, where every partial sum of fp16 inputs
// is exact, so the rotated value is rounded once, to fp16, exactly as the
// reference rounds its fp32 matmul result back to the input dtype.  The
// squared norm is summed in float64 in a fixed pairwise-tree order (element
// order) and rounded to fp32 with a correctly rounded square root; the
// division, clamp and the bucketize-style nearest-centroid search give the
// reference's fp32 results.
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

// Lane l reads lane l ^ M's 32-bit value (M = 1, 2, 4, 8) with DPP within its
// row of 16 lanes, without the LDS crossbar (every source lane exists, so no
// old value is needed).
template <int M>
__device__ __forceinline__ uint32_t xor_lane(uint32_t v) {
    if constexpr (M == 1) {
        return __builtin_amdgcn_mov_dpp(v, 0xB1, 0xF, 0xF, true);   // quad_perm 1,0,3,2
    } else if constexpr (M == 2) {
        return __builtin_amdgcn_mov_dpp(v, 0x4E, 0xF, 0xF, true);   // quad_perm 2,3,0,1
    } else if constexpr (M == 4) {
        // row_half_mirror (lane a of each 8-lane half reads lane 7 - a), then
        // quad_perm 3,2,1,0 (lane a reads a ^ 3): 7 - (a ^ 3) = a ^ 4.
        const uint32_t m = __builtin_amdgcn_mov_dpp(v, 0x141, 0xF, 0xF, true);
        return __builtin_amdgcn_mov_dpp(m, 0x1B, 0xF, 0xF, true);
    } else {
        static_assert(M == 8, "lane distance within a row");
        return __builtin_amdgcn_mov_dpp(v, 0x128, 0xF, 0xF, true);   // row_ror:8
    }
}

template <int M>
__device__ __forceinline__ double xor_lane_d(double v) {
    const uint64_t b = (uint64_t)__double_as_longlong(v);
    const uint32_t lo = xor_lane<M>((uint32_t)b);
    const uint32_t hi = xor_lane<M>((uint32_t)(b >> 32));
    return __longlong_as_double((long long)(((uint64_t)hi << 32) | lo));
}

constexpr int kEncWaves = 4;

// Butterfly stage across lanes j, j ^ M (element bit log2(M) + 3): the lower
// lane keeps x + partner, the upper one partner - x (exact in float64).
template <int M>
__device__ __forceinline__ void bfly_lanes(double (&x)[8], int lane) {
    const double sg = (lane & M) ? -1.0 : 1.0;
    double pt[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) pt[i] = xor_lane_d<M>(x[i]);
#pragma unroll
    for (int i = 0; i < 8; ++i) x[i] = fma(sg, x[i], pt[i]);
}

// Nearest centroid of x among the sorted L-entry codebook: bucketize-style
// upper index upper = min(#{i : !(cb[i] >= x)}, L-1) by bisection (the
// predicate is monotone in i for a sorted codebook; NaN makes it true
// everywhere, as in the count), then the neighbour compare: the upper index
// unless the lower neighbour is at least as close (compression.py:298-313).
// cbl: the codebook in LDS (probes; one shared copy, so lanes reading
// different entries hit different banks); tri: (cb[2i-1] (cb[0] for i = 0),
// cb[2i], cb[2i+1]) triples for the last step and the compare.
template <int L>
__device__ __forceinline__ uint32_t quantize_bisect(float x, const float *cbl, const float4 *tri) {
    int pos = 0;
#pragma unroll
    for (int step = L / 2; step >= 2; step >>= 1)
        if (!(cbl[pos + step - 1] >= x)) pos += step;
    const float4 t = tri[pos >> 1];
    const bool c1 = !(t.y >= x);
    const int upper = pos + (c1 ? 1 : 0);
    const float cu = c1 ? t.z : t.y;
    const float cl = c1 ? t.y : t.x;
    const int lower = upper - 1 < 0 ? 0 : upper - 1;
    const float du = fabsf(cu - x);
    const float dl = fabsf(x - cl);
    return (uint32_t)(du < dl ? upper : lower);
}

template <int L>
__global__ void __launch_bounds__(64 * kEncWaves)
paged_encode_kernel(EncodeParams p) {
    constexpr int KB = kD * (L == 16 ? 4 : 2) / 8;   // code bytes per role
    __shared__ float4 tri[2][L / 2];
    __shared__ float cbl[2][L];
    __shared__ double xt[4 * kEncWaves][kD];      // one 128-vector per 16-lane row
    if (threadIdx.x < L) {
        const int r = threadIdx.x / (L / 2), i = threadIdx.x % (L / 2);
        const float *c = r ? p.cb_v : p.cb_k;
        tri[r][i] = make_float4(c[i ? 2 * i - 1 : 0], c[2 * i], c[2 * i + 1], 0.0f);
    }
    if (threadIdx.x < 2 * L)
        cbl[threadIdx.x / L][threadIdx.x % L] =
            (threadIdx.x < L ? p.cb_k : p.cb_v)[threadIdx.x % L];
    __syncthreads();

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int role = wave >> 1;                       // waves 0,1: K; 2,3: V (wave-uniform)
    const int j = lane & 15;
    // (token, head) item of this row; fewer than 2^31 items (checked on the host).
    const uint32_t items = (uint32_t)(p.num_tokens * p.H_kv);
    const uint32_t item = blockIdx.x * 8u + 4u * (uint32_t)(wave & 1) + (uint32_t)(lane >> 4);
    const bool valid = item < items;
    const uint32_t t32 = valid ? item / (uint32_t)p.H_kv : 0u;
    const int h = valid ? (int)(item - t32 * (uint32_t)p.H_kv) : 0;
    const int64_t t = t32;

    double x[8];
    {
        const uint16_t *src = role == 0 ? p.k + t * p.k_stride + (int64_t)h * kD
                                        : p.v + t * p.v_stride + (int64_t)h * kD;
        uint4 w = make_uint4(0, 0, 0, 0);
        if (valid) w = reinterpret_cast<const uint4 *>(src)[j];
        const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            x[2 * i] = (double)h2f((uint16_t)(ws[i] & 0xFFFFu));
            x[2 * i + 1] = (double)h2f((uint16_t)(ws[i] >> 16));
        }
    }
    // Sylvester butterflies, exact in float64 (so their order is free):
    // element bits 0-2 in registers; then a transpose through LDS gives lane
    // j the elements (j & 7) + 8 r + 64 (j >> 3), r = 0..7, so bits 3-5 are
    // register stages too and only bit 6 crosses lanes (j ^ 8); a second
    // transpose restores elements 8j..8j+7 to lane j.
    auto bfly_regs = [&]() CDA_INLINE {
#pragma unroll
        for (int m = 1; m < 8; m <<= 1)
#pragma unroll
            for (int i = 0; i < 8; ++i)
                if (!(i & m)) {
                    const double a = x[i], b = x[i | m];
                    x[i] = a + b;
                    x[i | m] = a - b;
                }
    };
    bfly_regs();
    {
        double *row = xt[threadIdx.x >> 4];       // this lane's vector (128 doubles)
        const int e0 = (j & 7) + 64 * (j >> 3);
        double2 *mine = reinterpret_cast<double2 *>(row + 8 * j);
#pragma unroll
        for (int i = 0; i < 4; ++i) mine[i] = make_double2(x[2 * i], x[2 * i + 1]);
        __builtin_amdgcn_wave_barrier();
#pragma unroll
        for (int r = 0; r < 8; ++r) x[r] = row[e0 + 8 * r];
        bfly_regs();
        bfly_lanes<8>(x, lane);
        __builtin_amdgcn_wave_barrier();
#pragma unroll
        for (int r = 0; r < 8; ++r) row[e0 + 8 * r] = x[r];
        __builtin_amdgcn_wave_barrier();
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const double2 v = mine[i];
            x[2 * i] = v.x;
            x[2 * i + 1] = v.y;
        }
    }
    const double hsc = (double)__int_as_float(0x3db504f3);   // fp32(1/sqrt(128))
    float f[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) f[i] = h2f(f64_to_f16_rn(x[i] * hsc));
    // Squared norm: the pairwise tree in element order.
    double sq[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) sq[i] = (double)f[i] * (double)f[i];
    double ss = ((sq[0] + sq[1]) + (sq[2] + sq[3])) + ((sq[4] + sq[5]) + (sq[6] + sq[7]));
    ss = ss + xor_lane_d<1>(ss);
    ss = ss + xor_lane_d<2>(ss);
    ss = ss + xor_lane_d<4>(ss);
    ss = ss + xor_lane_d<8>(ss);
    float n = sqrt_f64_to_f32_rn(ss);
    n = (n < 1e-12f) ? 1e-12f : n;     // clamp_min(1e-12); NaN passes through
    // u = RN32(f / n) as RN32(f * RN64(1 / n)): the float64 product is within
    // 2^-52 (relative) of f / n, and a quotient of two 24-bit numbers is never
    // a 25-bit rounding midpoint and, when not one, lies at least 2^-49 from
    // every midpoint, so the final rounding equals the correctly rounded
    // quotient (NaN, infinity and zero propagate as in the division).
    const double rn = 1.0 / (double)n;
    uint32_t idx[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        float u = (float)((double)f[i] * rn);
        u = u < -1.0f ? -1.0f : (u > 1.0f ? 1.0f : u);
        idx[i] = quantize_bisect<L>(u, cbl[role], tri[role]);
    }
    if (!valid) return;
    const int64_t slot = p.slot_mapping[t];
    if (slot < 0 || slot >= p.num_slots) return;
    uint8_t *dst = p.cache + slot * p.row_bytes + (int64_t)h * p.slot_bytes;
    uint8_t *codes = dst + role * KB;
    if (L == 16) {
        uint32_t wv = 0;
#pragma unroll
        for (int b = 0; b < 4; ++b) wv |= ((idx[2 * b] << 4) | idx[2 * b + 1]) << (8 * b);
        *reinterpret_cast<uint32_t *>(codes + 4 * j) = wv;
    } else {
        const uint32_t b0 = (idx[0] << 6) | (idx[1] << 4) | (idx[2] << 2) | idx[3];
        const uint32_t b1 = (idx[4] << 6) | (idx[5] << 4) | (idx[6] << 2) | idx[7];
        *reinterpret_cast<uint16_t *>(codes + 2 * j) = (uint16_t)(b0 | (b1 << 8));
    }
    if (j == 0) *reinterpret_cast<float *>(dst + 2 * KB + 4 * role) = n;
}

}  // namespace

}  // namespace cda

using namespace cda;

extern "C" int cda_paged_encode_fused(const void *k, const void *v, int64_t k_stride,
                                      int64_t v_stride, const int32_t *slot_mapping,
                                      int64_t num_tokens, void *flat_cache, int64_t num_slots,
                                      int slot_bytes, int H_kv, const float *cb_k,
                                      const float *cb_v, int levels, void *stream) {
    CDA_REQUIRE(num_tokens >= 0, "cda_paged_encode_fused: num_tokens must be >= 0");
    if (num_tokens == 0) return CDA_OK;
    CDA_REQUIRE(k && v && slot_mapping && flat_cache && cb_k && cb_v,
                "cda_paged_encode_fused: null pointer argument");
    CDA_REQUIRE(levels == 16 || levels == 4, "cda_paged_encode_fused: levels must be 16 or 4");
    CDA_REQUIRE(H_kv > 0 && num_slots > 0, "cda_paged_encode_fused: H_kv and num_slots must be > 0");
    const int kb = kD * (levels == 16 ? 4 : 2) / 8;
    CDA_REQUIRE(slot_bytes >= 2 * kb + 8, "cda_paged_encode_fused: slot_bytes too small for the layout");
    CDA_REQUIRE(k_stride >= (int64_t)H_kv * kD && v_stride >= (int64_t)H_kv * kD,
                "cda_paged_encode_fused: token stride smaller than H_kv * 128");
    CDA_REQUIRE(((uintptr_t)k & 3) == 0 && ((uintptr_t)v & 3) == 0 && slot_bytes % 4 == 0 &&
                    ((uintptr_t)flat_cache & 3) == 0,
                "cda_paged_encode_fused: k, v, cache must be 4-byte aligned");
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
    CDA_REQUIRE(items < ((int64_t)1 << 31), "cda_paged_encode_fused: too many tokens x heads");
    hipStream_t st = static_cast<hipStream_t>(stream);
    const int64_t blocks = (items + 7) / 8;
    if (levels == 16)
        paged_encode_kernel<16><<<dim3((unsigned)blocks), 64 * kEncWaves, 0, st>>>(p);
    else
        paged_encode_kernel<4><<<dim3((unsigned)blocks), 64 * kEncWaves, 0, st>>>(p);
    CDA_LAUNCH_CHECK("paged_encode_kernel");
    return CDA_OK;
}
