// Fused paged encode: Hadamard-128 + norm + nearest centroid + pack + scatter
// into the paged slot layout (gfx950).
//
// Reference contract: cda_paged_encode_fused as bound by
// cda/kernels_cuda/wrappers.py:127-156; arithmetic of Compressor.encode
// (cda/algorithm/compression.py:287-335) and pack_4bit / pack_2bit
// (:163-179, :375-386).
//
// One wave per (token, KV head); it encodes K then V.  Lane l holds
// elements 2l and 2l+1 of the 128-vector (one coalesced 256-byte read per
// vector).  The butterfly runs in float64, where every partial sum of fp16
// inputs is exact, so the rotated value is rounded once, to fp16, exactly as
// the reference rounds its fp32 matmul result back to the input dtype.  The
// squared norm is summed in float64 in a fixed lane-tree order and rounded
// to fp32 with a correctly rounded square root; the division, clamp and the
// bucketize-style nearest-centroid search run in fp32 as in the reference.
#include "cda_common.h"

namespace cda {

namespace {

constexpr int kEncWaves = 4;

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

// Lane l reads lane l ^ M's 32-bit value, without the LDS crossbar: DPP
// within a row of 16 lanes (M = 1, 2, 4, 8), the row-swap permutes across
// rows (M = 16, 32).
template <int M>
__device__ __forceinline__ uint32_t xor_lane(uint32_t v, int lane) {
    if constexpr (M == 1) {
        return __builtin_amdgcn_update_dpp(0u, v, 0xB1, 0xF, 0xF, false);   // quad_perm 1,0,3,2
    } else if constexpr (M == 2) {
        return __builtin_amdgcn_update_dpp(0u, v, 0x4E, 0xF, 0xF, false);   // quad_perm 2,3,0,1
    } else if constexpr (M == 4) {
        // row_ror:n gives lane l the value of lane (l - n) mod 16 of its row.
        const uint32_t from_below = __builtin_amdgcn_update_dpp(0u, v, 0x124, 0xF, 0xF, false);
        const uint32_t from_above = __builtin_amdgcn_update_dpp(0u, v, 0x12C, 0xF, 0xF, false);
        return (lane & 4) ? from_below : from_above;
    } else if constexpr (M == 8) {
        return __builtin_amdgcn_update_dpp(0u, v, 0x128, 0xF, 0xF, false);   // row_ror:8
    } else if constexpr (M == 16) {
        const auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
        return (lane & 16) ? r[0] : r[1];
    } else {
        static_assert(M == 32, "lane distance");
        const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
        return (lane & 32) ? r[0] : r[1];
    }
}

template <int M>
__device__ __forceinline__ double xor_lane_d(double v, int lane) {
    const uint64_t b = (uint64_t)__double_as_longlong(v);
    const uint32_t lo = xor_lane<M>((uint32_t)b, lane);
    const uint32_t hi = xor_lane<M>((uint32_t)(b >> 32), lane);
    return __longlong_as_double((long long)(((uint64_t)hi << 32) | lo));
}

// One butterfly stage across lanes l, l ^ M (element e and e ^ 2M): the lower
// lane keeps x + partner, the upper one partner - x.  Exact (every partial
// sum of fp16 values fits float64).
template <int M>
__device__ __forceinline__ void bfly_stage(double &x0, double &x1, int lane) {
    const double p0 = xor_lane_d<M>(x0, lane);
    const double p1 = xor_lane_d<M>(x1, lane);
    const double sg = (lane & M) ? -1.0 : 1.0;
    x0 = fma(sg, x0, p0);
    x1 = fma(sg, x1, p1);
}

template <int M>
__device__ __forceinline__ void tree_stage(double &ss, int lane) {
    ss = ss + xor_lane_d<M>(ss, lane);
}

// torch.bucketize(right=False) + neighbour compare (compression.py:298-313):
// upper = #{i : !(cb[i] >= x)} (NaN -> L), clamp, ties go to the lower index.
template <int L>
__device__ __forceinline__ uint32_t quantize(float x, const float *cb) {
    int upper = 0;
#pragma unroll
    for (int i = 0; i < L; ++i) upper += !(cb[i] >= x);
    upper = upper > L - 1 ? L - 1 : upper;
    const int lower = upper - 1 < 0 ? 0 : upper - 1;
    const float du = fabsf(cb[upper] - x);
    const float dl = fabsf(x - cb[lower]);
    return (uint32_t)(du < dl ? upper : lower);
}

// Encode the 128-vector whose elements (2*lane, 2*lane+1) are `pair`; returns
// the two indices (hi = element 2*lane) and the fp32 norm (same on all lanes).
template <int L>
__device__ __forceinline__ void encode_vec(uint32_t pair, const float *cb, int lane,
                                           uint32_t &i0, uint32_t &i1, float &nrm) {
    double a = (double)h2f((uint16_t)(pair & 0xFFFFu));
    double b = (double)h2f((uint16_t)(pair >> 16));
    // Sylvester butterfly, stage len=1 inside the lane.
    double x0 = a + b, x1 = a - b;
    // Stages len = 2..64: partner element e ^ len lives in lane l ^ (len/2).
    bfly_stage<1>(x0, x1, lane);
    bfly_stage<2>(x0, x1, lane);
    bfly_stage<4>(x0, x1, lane);
    bfly_stage<8>(x0, x1, lane);
    bfly_stage<16>(x0, x1, lane);
    bfly_stage<32>(x0, x1, lane);
    const double h = (double)__int_as_float(0x3db504f3);   // fp32(1/sqrt(128))
    const uint16_t r0 = f64_to_f16_rn(x0 * h);
    const uint16_t r1 = f64_to_f16_rn(x1 * h);
    const float f0 = h2f(r0), f1 = h2f(r1);
    double ss = (double)f0 * (double)f0 + (double)f1 * (double)f1;
    // Pairwise tree in element order: lanes l, l ^ m for m = 1, 2, ..., 32.
    tree_stage<1>(ss, lane);
    tree_stage<2>(ss, lane);
    tree_stage<4>(ss, lane);
    tree_stage<8>(ss, lane);
    tree_stage<16>(ss, lane);
    tree_stage<32>(ss, lane);
    float n = sqrt_f64_to_f32_rn(ss);
    n = (n < 1e-12f) ? 1e-12f : n;     // clamp_min(1e-12); NaN passes through
    nrm = n;
    float u0 = __fdiv_rn(f0, n), u1 = __fdiv_rn(f1, n);
    u0 = u0 < -1.0f ? -1.0f : (u0 > 1.0f ? 1.0f : u0);
    u1 = u1 < -1.0f ? -1.0f : (u1 > 1.0f ? 1.0f : u1);
    i0 = quantize<L>(u0, cb);
    i1 = quantize<L>(u1, cb);
}

template <int L>
__global__ void __launch_bounds__(64 * kEncWaves)
paged_encode_kernel(EncodeParams p) {
    constexpr int KB = kD * (L == 16 ? 4 : 2) / 8;   // code bytes per role
    __shared__ float cbs[2][L];
    if (threadIdx.x < 2 * L)
        cbs[threadIdx.x / L][threadIdx.x % L] =
            threadIdx.x < L ? p.cb_k[threadIdx.x] : p.cb_v[threadIdx.x - L];
    __syncthreads();

    const int lane = threadIdx.x & 63;
    const int64_t item = (int64_t)blockIdx.x * kEncWaves + (threadIdx.x >> 6);
    if (item >= p.num_tokens * p.H_kv) return;
    const int64_t t = item / p.H_kv;
    const int h = (int)(item % p.H_kv);
    const int64_t slot = p.slot_mapping[t];
    if (slot < 0 || slot >= p.num_slots) return;
    uint8_t *dst = p.cache + slot * p.row_bytes + (int64_t)h * p.slot_bytes;

#pragma unroll
    for (int role = 0; role < 2; ++role) {
        const uint16_t *src = role == 0 ? p.k + t * p.k_stride + (int64_t)h * kD
                                        : p.v + t * p.v_stride + (int64_t)h * kD;
        const uint32_t pair = reinterpret_cast<const uint32_t *>(src)[lane];
        uint32_t i0, i1;
        float nrm;
        encode_vec<L>(pair, cbs[role], lane, i0, i1, nrm);
        uint8_t *codes = dst + role * KB;
        if (L == 16) {
            codes[lane] = (uint8_t)((i0 << 4) | i1);
        } else {
            const uint32_t nib = (i0 << 2) | i1;          // dims 2l, 2l+1
            const uint32_t other = (uint32_t)__shfl_xor((int)nib, 1);
            if ((lane & 1) == 0) codes[lane >> 1] = (uint8_t)((nib << 4) | other);
        }
        if (lane == 0) *reinterpret_cast<float *>(dst + 2 * KB + 4 * role) = nrm;
    }
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
    const int64_t blocks = (items + kEncWaves - 1) / kEncWaves;
    CDA_REQUIRE(blocks < ((int64_t)1 << 31), "cda_paged_encode_fused: too many tokens");
    hipStream_t st = static_cast<hipStream_t>(stream);
    if (levels == 16)
        paged_encode_kernel<16><<<dim3((unsigned)blocks), 64 * kEncWaves, 0, st>>>(p);
    else
        paged_encode_kernel<4><<<dim3((unsigned)blocks), 64 * kEncWaves, 0, st>>>(p);
    CDA_LAUNCH_CHECK("paged_encode_kernel");
    return CDA_OK;
}
