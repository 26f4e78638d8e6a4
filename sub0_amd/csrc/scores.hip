// Score-domain QK over compressed K for the 16-level uniform codebook
// (gfx950).
//
// Reference contract: qk_scores_uniform_4bit_without_k_decode
// (cda/algorithm/attention.py:101-152).  With cb[i] = (2i + 1)/16 - 1,
//     Q . K[k] = norm[k] * ((Q . code[k]) / 8 - 15/16 * sum(Q)),
// so K stays as packed 4-bit codes plus its row norm and is never decoded.
// Scores are fp32 (B, H_q, M_q, key_end - key_start), times `scale`, with the
// bottom-right causal mask of the reference (key key_start + k visible to
// query m iff key_start + k <= m + q_offset) when `causal` is set.
//
// K layout: contiguous (B, H_kv, M_k, 64) bytes, MSB-first nibbles (the
// CompressedSlot of compression.py:163-188), norms (B, H_kv, M_k) fp32.
//
// Workgroup = 256 threads = 64 keys x 4 query-row lanes over 16 query rows of
// one (sequence, KV head): rows r = g * M_q + m of the GQA group.  The 16 rows
// of q_rot sit in LDS as fp32 (broadcast reads), each thread unpacks its key's
// codes once per 32 dims and accumulates four rows.  The paged decode form of
// the same contract runs on MFMA inside decode_stream_kernel.
#include "cda_common.h"

namespace cda {
namespace {

constexpr int kRows = 16;          // query rows per workgroup
constexpr int kKeys = 64;          // keys per workgroup

__global__ void __launch_bounds__(256)
qk_scores_uniform4_kernel(const uint16_t *__restrict__ q_rot, const uint8_t *__restrict__ k_idx,
                          const float *__restrict__ k_norm, float *__restrict__ out, int H_q,
                          int H_kv, int M_q, int gs, int64_t M_k, int64_t key_start,
                          int64_t key_end, int64_t q_offset, float scale, int causal) {
    __shared__ float qs[kRows][kD];
    __shared__ float qsum[kRows];
    const int tid = threadIdx.x;
    const int bh = blockIdx.y;                       // b * H_kv + h
    const int b = bh / H_kv, h = bh % H_kv;
    const int rows = gs * M_q;
    const int r0 = blockIdx.z * kRows;
    for (int i = tid; i < kRows * kD; i += 256) {
        const int r = r0 + i / kD, d = i % kD;
        float v = 0.0f;
        if (r < rows) {
            const int g = r / M_q, m = r % M_q;
            v = h2f(q_rot[(((int64_t)b * H_q + h * gs + g) * M_q + m) * kD + d]);
        }
        qs[i / kD][d] = v;
    }
    __syncthreads();
    if (tid < kRows) {
        float a = 0.0f;
        for (int d = 0; d < kD; ++d) a += qs[tid][d];
        qsum[tid] = a;
    }
    __syncthreads();

    const int64_t nk = key_end - key_start;
    const int64_t kl = (int64_t)blockIdx.x * kKeys + (tid & 63);   // key within the window
    const int sub = tid >> 6;                                       // rows sub, sub + 4, ...
    if (kl >= nk) return;
    const int64_t key = key_start + kl;
    const uint8_t *code = k_idx + ((int64_t)bh * M_k + key) * (kD / 2);
    const float nrm = k_norm[(int64_t)bh * M_k + key];
    float acc[kRows / 4] = {};
#pragma unroll
    for (int c = 0; c < 4; ++c) {                    // 32 dims per 16-byte chunk
        const uint4 w = *reinterpret_cast<const uint4 *>(code + 16 * c);
        const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
        float cv[32];
#pragma unroll
        for (int e = 0; e < 4; ++e)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const uint32_t byte = (ws[e] >> (8 * j)) & 0xFFu;
                cv[8 * e + 2 * j] = (float)(byte >> 4);
                cv[8 * e + 2 * j + 1] = (float)(byte & 15u);
            }
#pragma unroll
        for (int j = 0; j < kRows / 4; ++j) {
            const float *qr = qs[sub + 4 * j] + 32 * c;
#pragma unroll
            for (int d = 0; d < 32; ++d) acc[j] = fmaf(qr[d], cv[d], acc[j]);
        }
    }
#pragma unroll
    for (int j = 0; j < kRows / 4; ++j) {
        const int r = r0 + sub + 4 * j;
        if (r >= rows) break;
        const int g = r / M_q, m = r % M_q;
        float s = nrm * (acc[j] * 0.125f - qsum[sub + 4 * j] * 0.9375f) * scale;
        if (causal && key > (int64_t)m + q_offset) s = -__builtin_inff();
        out[(((int64_t)b * H_q + h * gs + g) * M_q + m) * nk + kl] = s;
    }
}

}  // namespace
}  // namespace cda

using namespace cda;

extern "C" int cda_qk_scores_uniform4(const void *q_rot, const void *k_idx, const float *k_norm,
                                      float *out, int B, int H_q, int H_kv, int M_q,
                                      int group_size, int64_t M_k, int64_t key_start,
                                      int64_t key_end, int64_t q_offset, float scale, int causal,
                                      void *stream) {
    CDA_REQUIRE(q_rot && k_idx && k_norm && out, "cda_qk_scores_uniform4: null pointer argument");
    CDA_REQUIRE(B >= 0 && H_kv > 0 && M_q >= 0 && M_k >= 0 && group_size > 0 &&
                    H_q == H_kv * group_size,
                "cda_qk_scores_uniform4: bad shape (H_q must equal H_kv * group_size)");
    CDA_REQUIRE(0 <= key_start && key_start <= key_end && key_end <= M_k,
                "cda_qk_scores_uniform4: invalid key window");
    CDA_REQUIRE(((uintptr_t)k_idx & 15) == 0, "cda_qk_scores_uniform4: K idx must be 16-byte aligned");
    const int64_t nk = key_end - key_start;
    const int64_t rows = (int64_t)group_size * M_q;
    if (B == 0 || nk == 0 || rows == 0) return CDA_OK;
    CDA_REQUIRE((int64_t)B * H_kv < 65536 && (rows + kRows - 1) / kRows < 65536,
                "cda_qk_scores_uniform4: B * H_kv and group_size * M_q / 16 must be < 65536");
    const dim3 grid((unsigned)((nk + kKeys - 1) / kKeys), (unsigned)(B * H_kv),
                    (unsigned)((rows + kRows - 1) / kRows));
    qk_scores_uniform4_kernel<<<grid, 256, 0, static_cast<hipStream_t>(stream)>>>(
        static_cast<const uint16_t *>(q_rot), static_cast<const uint8_t *>(k_idx), k_norm, out,
        H_q, H_kv, M_q, group_size, M_k, key_start, key_end, q_offset, scale, causal);
    CDA_LAUNCH_CHECK("qk_scores_uniform4_kernel");
    return CDA_OK;
}
