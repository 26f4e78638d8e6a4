// libcda_hip_torch.so -- the torch.ops registration of the MI355X CDA kernels,
// in C++ over the C ABI of libcda_hip.so (include/cda_hip.h).
//
// The reference ships its kernels as TORCH_LIBRARY extensions loaded with
// torch.ops.load_library (cda/_prebuilt_loader.py:69-80); this library is
// that artefact here: `torch.ops.load_library(".../libcda_hip_torch.so")`
// defines two namespaces with Tensor(a!) schemas, CUDA (= HIP on ROCm)
// kernels and Meta kernels (shape-only, for FakeTensor / torch.compile):
//
//   cda_hip               -- the product ops behind load_pybind_module
//                            (wrappers.py:115-124, 153-156; fa2_cda.py:51-52,
//                            85-95, 166-181), plus the score-domain QK
//                            (attention.py:101-187) and the hybrid prefill.
//   _cda_vllm_fa2_fork_C  -- the comparator namespace of the reference's vLLM
//                            FA2 fork (kernels_vllm_fa2_fork/interface.py:
//                            138-162, 234-257, 304-328, 434-461), positional
//                            signatures as there.
//
// Errors: wrong dtypes raise TypeError (TORCH_CHECK_TYPE), wrong shapes or a
// C-ABI CDA_E_INVALID raise ValueError (TORCH_CHECK_VALUE), features the
// kernels do not have raise NotImplementedError, other C-ABI failures
// RuntimeError with cda_hip_last_error().  libcda_hip.so itself stays
// torch-free; this file is the only C++ that sees torch types.
#include <ATen/ATen.h>
#include <ATen/hip/impl/HIPGuardImplMasqueradingAsCUDA.h>
#include <ATen/hip/impl/HIPStreamMasqueradingAsCUDA.h>
#include <torch/library.h>

#include <cmath>
#include <string>
#include <vector>

#include "../../include/cda_hip.h"

namespace {

using at::Tensor;

void check_rc(int rc, const char *what) {
    if (rc == CDA_OK) return;
    std::string msg = cda_hip_last_error();
    const std::string pre = std::string(what) + ": ";
    if (msg.rfind(pre, 0) == 0) msg = msg.substr(pre.size());
    TORCH_CHECK_VALUE(rc != CDA_E_INVALID, what, ": ", msg);
    TORCH_CHECK(false, what, " failed (", rc, "): ", msg);
}

// PyTorch on ROCm reports HIP devices as "cuda": the masquerading guard and
// stream types are the ones that accept them.
using DeviceGuard = c10::hip::HIPGuardMasqueradingAsCUDA;

void *stream_of(const Tensor &t) {
    return c10::hip::getCurrentHIPStreamMasqueradingAsCUDA(t.device().index()).stream();
}

// All tensors on one GPU; returns that device (the caller makes it current).
c10::Device on_gpu(std::initializer_list<const Tensor *> ts) {
    const Tensor &first = **ts.begin();
    for (const Tensor *t : ts) {
        TORCH_CHECK_VALUE(t->is_cuda(), "CDA kernels run on the GPU only; got a tensor on ",
                          t->device().str());
        TORCH_CHECK_VALUE(t->device() == first.device(), "all tensors must be on one device (",
                          t->device().str(), " vs ", first.device().str(), ")");
    }
    return first.device();
}

// 256-byte-aligned scratch of `need` bytes from torch's caching allocator.
struct Workspace {
    Tensor buf;
    void *ptr = nullptr;
    size_t bytes = 0;
};

Workspace workspace(const Tensor &like, size_t need) {
    Workspace w;
    w.buf = at::empty({(int64_t)need + 256}, like.options().dtype(at::kByte));
    const uintptr_t p = reinterpret_cast<uintptr_t>(w.buf.data_ptr());
    const size_t pad = (256 - p % 256) % 256;
    w.ptr = reinterpret_cast<void *>(p + pad);
    w.bytes = (size_t)w.buf.numel() - pad;
    return w;
}

void need_dtype(const Tensor &t, at::ScalarType s, const char *msg) {
    TORCH_CHECK_TYPE(t.scalar_type() == s, msg);
}

void check_paged(const Tensor &kv, const Tensor &bt, const Tensor &sl, const Tensor &cbk,
                 const Tensor &cbv, bool allow_k4v2) {
    TORCH_CHECK_VALUE(kv.scalar_type() == at::kByte && kv.dim() == 3 && kv.is_contiguous(),
                      "kv_cache must be a contiguous uint8 (num_slots, H_kv, slot_bytes) tensor");
    TORCH_CHECK_VALUE(bt.scalar_type() == at::kInt && bt.dim() == 2 && bt.stride(1) == 1,
                      "block_table must be int32 (B, max_blocks) with unit inner stride");
    need_dtype(sl, at::kInt, "seq_lens must be int32");
    if (allow_k4v2 && cbk.numel() == 16 && cbv.numel() == 4) return;
    TORCH_CHECK_VALUE(cbk.numel() == 16 && cbv.numel() == 16,
                      "the prefill kernels read K4V4 caches (16-level codebooks)");
}

Tensor f32c(const Tensor &t) { return t.to(at::kFloat).contiguous(); }

// ------------------------------------------------------------------ decode --

void decode_impl(const Tensor &q, const Tensor &kv, const Tensor &bt, const Tensor &sl,
                 const Tensor &cb_k_in, const Tensor &cb_v_in, const Tensor &r32,
                 const c10::optional<Tensor> &r16, const Tensor &out, int64_t gs, int64_t bs,
                 int64_t tile_n, int64_t max_seq_len, double scale, bool uniform_qk) {
    const DeviceGuard guard(on_gpu({&q, &kv, &bt, &sl, &cb_k_in, &cb_v_in, &r32, &out}));
    TORCH_CHECK_TYPE(q.scalar_type() == at::kHalf && out.scalar_type() == at::kHalf,
                     "q and out must be fp16");
    need_dtype(kv, at::kByte, "kv_cache must be uint8");
    TORCH_CHECK_TYPE(bt.scalar_type() == at::kInt && sl.scalar_type() == at::kInt,
                     "block_table and seq_lens must be int32");
    TORCH_CHECK_TYPE(cb_k_in.scalar_type() == at::kFloat && cb_v_in.scalar_type() == at::kFloat &&
                         r32.scalar_type() == at::kFloat,
                     "codebooks and rot_f32 must be fp32");
    TORCH_CHECK_VALUE(q.dim() == 3 && q.size(2) == 128 && q.is_contiguous(),
                      "q must be a contiguous (B, H_q, 128) tensor");
    TORCH_CHECK_VALUE(out.sizes() == q.sizes() && out.is_contiguous(),
                      "out must be a contiguous tensor shaped like q");
    TORCH_CHECK_VALUE(kv.dim() == 3 && kv.is_contiguous(),
                      "kv_cache must be a contiguous (num_slots, H_kv, slot_bytes) tensor");
    TORCH_CHECK_VALUE(bt.dim() == 2 && bt.stride(1) == 1,
                      "block_table must be (B, max_blocks) with unit inner stride");
    TORCH_CHECK_VALUE(r32.dim() == 2 && r32.size(0) == 128 && r32.size(1) == 128 &&
                          r32.is_contiguous(),
                      "rot_f32 must be a contiguous (128, 128) tensor");
    const bool k4v2 = cb_k_in.numel() == 16 && cb_v_in.numel() == 4;
    TORCH_CHECK_VALUE(cb_k_in.numel() == cb_v_in.numel() || k4v2,
                      "cb_K and cb_V must have the same number of levels (or 16 and 4: the "
                      "K4V2 cache)");
    const int B = (int)q.size(0), H_q = (int)q.size(1);
    const int64_t num_slots = kv.size(0);
    const int H_kv = (int)kv.size(1), slot_bytes = (int)kv.size(2);
    TORCH_CHECK_VALUE(bt.size(0) >= B && sl.numel() >= B,
                      "block_table / seq_lens have fewer rows than q");
    const Tensor cb_k = cb_k_in.contiguous();
    // One tensor for both codebooks lets the single-launch kernel run without
    // a device-side comparison of the two tables.
    const Tensor cb_v = cb_v_in.data_ptr() == cb_k_in.data_ptr() ? cb_k : cb_v_in.contiguous();
    const size_t need = cda_decode_workspace_size(B, H_q, H_kv, (int)max_seq_len, (int)tile_n);
    Workspace ws = workspace(q, need);
    void *st = stream_of(q);
    const float *pk = cb_k.data_ptr<float>(), *pv = cb_v.data_ptr<float>();
    if (uniform_qk) {
        TORCH_CHECK_VALUE(cb_k.numel() == 16 && cb_v.numel() == 16,
                          "the score-domain QK reads K4V4 caches (16-level codebooks)");
        check_rc(cda_decode_full_hmma_v3_uniform_qk(
                     q.data_ptr(), kv.data_ptr(), num_slots, slot_bytes, H_kv,
                     bt.data_ptr<int32_t>(), (int)bt.stride(0), sl.data_ptr<int32_t>(), pk, pv,
                     r32.data_ptr<float>(), out.data_ptr(), B, H_q, (int)gs, (int)bs,
                     (int)tile_n, (int)max_seq_len, (float)scale, ws.ptr, ws.bytes, st),
                 "cda_decode_full_hmma_v3_uniform_qk");
        return;
    }
    const void *p16 = r16.has_value() ? r16->data_ptr() : nullptr;
    if (k4v2) {
        check_rc(cda_decode_full_hmma_v3_k4v2(
                     q.data_ptr(), kv.data_ptr(), num_slots, slot_bytes, H_kv,
                     bt.data_ptr<int32_t>(), (int)bt.stride(0), sl.data_ptr<int32_t>(), pk, pv,
                     r32.data_ptr<float>(), p16, out.data_ptr(), B, H_q, (int)gs, (int)bs,
                     (int)tile_n, (int)max_seq_len, (float)scale, ws.ptr, ws.bytes, st),
                 "cda_decode_full_hmma_v3_k4v2");
        return;
    }
    check_rc(cda_decode_full_hmma_v3(q.data_ptr(), kv.data_ptr(), num_slots, slot_bytes, H_kv,
                                     bt.data_ptr<int32_t>(), (int)bt.stride(0),
                                     sl.data_ptr<int32_t>(), pk, pv, (int)cb_k.numel(),
                                     r32.data_ptr<float>(), p16, out.data_ptr(), B, H_q, (int)gs,
                                     (int)bs, (int)tile_n, (int)max_seq_len, (float)scale, ws.ptr,
                                     ws.bytes, st),
             "cda_decode_full_hmma_v3");
}

void decode(const Tensor &q, const Tensor &kv, const Tensor &bt, const Tensor &sl,
            const Tensor &cb_k, const Tensor &cb_v, const Tensor &r32, const Tensor &r16,
            const Tensor &out, int64_t gs, int64_t bs, int64_t tile_n, int64_t max_seq_len,
            double scale) {
    decode_impl(q, kv, bt, sl, cb_k, cb_v, r32, r16, out, gs, bs, tile_n, max_seq_len, scale,
                false);
}

void decode_uniform_qk(const Tensor &q, const Tensor &kv, const Tensor &bt, const Tensor &sl,
                       const Tensor &cb_k, const Tensor &cb_v, const Tensor &r32,
                       const Tensor &out, int64_t gs, int64_t bs, int64_t tile_n,
                       int64_t max_seq_len, double scale) {
    decode_impl(q, kv, bt, sl, cb_k, cb_v, r32, c10::nullopt, out, gs, bs, tile_n, max_seq_len,
                scale, true);
}

void qk_scores_uniform4(const Tensor &q_rot, const Tensor &k_idx, const Tensor &k_norm,
                        const Tensor &out, int64_t gs, double scale, bool causal,
                        int64_t q_offset, int64_t key_start, int64_t key_end) {
    const DeviceGuard guard(on_gpu({&q_rot, &k_idx, &k_norm, &out}));
    TORCH_CHECK_TYPE(q_rot.scalar_type() == at::kHalf && k_idx.scalar_type() == at::kByte,
                     "Q_rot must be fp16 and K idx uint8");
    TORCH_CHECK_TYPE(k_norm.scalar_type() == at::kFloat && out.scalar_type() == at::kFloat,
                     "K norm and the scores must be fp32");
    for (const Tensor *t : {&q_rot, &k_idx, &k_norm, &out})
        TORCH_CHECK_VALUE(t->is_contiguous(),
                          "Q_rot, K idx / norm and the scores must be contiguous");
    TORCH_CHECK_VALUE(q_rot.dim() == 4 && k_idx.dim() == 4, "Q_rot and K idx must be 4-D");
    const int64_t B = q_rot.size(0), H_q = q_rot.size(1), M_q = q_rot.size(2);
    const int64_t H_kv = k_idx.size(1), M_k = k_idx.size(2);
    TORCH_CHECK_VALUE(out.dim() == 4 && out.size(0) == B && out.size(1) == H_q &&
                          out.size(2) == M_q && out.size(3) == key_end - key_start,
                      "scores must be (B, H_q, M_q, key_end - key_start)");
    check_rc(cda_qk_scores_uniform4(q_rot.data_ptr(), k_idx.data_ptr(), k_norm.data_ptr<float>(),
                                    out.data_ptr<float>(), (int)B, (int)H_q, (int)H_kv, (int)M_q,
                                    (int)gs, M_k, key_start, key_end, q_offset, (float)scale,
                                    causal ? 1 : 0, stream_of(q_rot)),
             "cda_qk_scores_uniform4");
}

// ------------------------------------------------------------------ encode --

void encode(const Tensor &k, const Tensor &v, const Tensor &slot_mapping,
            const Tensor &flat_cache, const Tensor &cb_k, const Tensor &cb_v) {
    const DeviceGuard guard(on_gpu({&k, &v, &slot_mapping, &flat_cache, &cb_k, &cb_v}));
    TORCH_CHECK_TYPE(k.scalar_type() == at::kHalf && v.scalar_type() == at::kHalf,
                     "K, V must be fp16");
    need_dtype(flat_cache, at::kByte, "flat_cache must be uint8");
    need_dtype(slot_mapping, at::kInt, "slot_mapping must be int32");
    TORCH_CHECK_VALUE(k.dim() == 3 && k.sizes() == v.sizes(),
                      "K and V must be (T, H_kv, 128) tensors of one shape");
    TORCH_CHECK_VALUE(k.size(2) == 128, "D must be 128, got ", k.size(2));
    TORCH_CHECK_VALUE(k.stride(2) == 1 && k.stride(1) == 128 && v.stride(2) == 1 &&
                          v.stride(1) == 128,
                      "K and V need contiguous heads (stride (*, 128, 1))");
    TORCH_CHECK_VALUE(flat_cache.dim() == 3 && flat_cache.is_contiguous(),
                      "flat_cache must be a contiguous (num_slots, H_kv, slot_bytes) tensor");
    const int64_t T = k.size(0);
    const int H_kv = (int)k.size(1);
    TORCH_CHECK_VALUE(flat_cache.size(1) == H_kv, "flat_cache head count does not match K");
    TORCH_CHECK_VALUE(slot_mapping.numel() >= T,
                      "slot_mapping shorter than the number of tokens");
    const Tensor sm = slot_mapping.contiguous(), ck = f32c(cb_k), cv = f32c(cb_v);
    const int levels = (int)cb_k.numel();
    void *st = stream_of(k);
    if (levels == 16 && cb_v.numel() == 4) {   // the legacy K4V2 slot
        check_rc(cda_paged_encode_fused_k4v2(k.data_ptr(), v.data_ptr(), k.stride(0),
                                             v.stride(0), sm.data_ptr<int32_t>(), T,
                                             flat_cache.data_ptr(), flat_cache.size(0),
                                             (int)flat_cache.size(2), H_kv, ck.data_ptr<float>(),
                                             cv.data_ptr<float>(), st),
                 "cda_paged_encode_fused_k4v2");
        return;
    }
    TORCH_CHECK_VALUE(cb_v.numel() == levels && (levels == 4 || levels == 16),
                      "cb_K and cb_V must both have 16 (K4V4) or 4 (K2V2) levels, or 16 and 4 "
                      "(K4V2)");
    check_rc(cda_paged_encode_fused(k.data_ptr(), v.data_ptr(), k.stride(0), v.stride(0),
                                    sm.data_ptr<int32_t>(), T, flat_cache.data_ptr(),
                                    flat_cache.size(0), (int)flat_cache.size(2), H_kv,
                                    ck.data_ptr<float>(), cv.data_ptr<float>(), levels, st),
             "cda_paged_encode_fused");
}

// ----------------------------------------------------------------- prefill --

void prefill(const Tensor &q, const Tensor &kv, const Tensor &bt, const Tensor &cu_q,
             const Tensor &sl, const Tensor &cb_k, const Tensor &cb_v, const Tensor &out,
             int64_t bs, int64_t max_query_len, double scale, int64_t max_seq_len) {
    const DeviceGuard guard(on_gpu({&q, &kv, &bt, &cu_q, &sl, &cb_k, &cb_v, &out}));
    TORCH_CHECK_TYPE(q.scalar_type() == at::kHalf && out.scalar_type() == at::kHalf,
                     "Q and output must be fp16");
    TORCH_CHECK_VALUE(q.dim() == 3 && q.size(2) == 128 && q.is_contiguous(),
                      "Q must be a contiguous (T, H_q, 128) tensor");
    TORCH_CHECK_VALUE(out.sizes() == q.sizes() && out.is_contiguous(),
                      "output must be a contiguous tensor shaped like Q");
    need_dtype(cu_q, at::kInt, "cu_seqlens_q must be int32");
    check_paged(kv, bt, sl, cb_k, cb_v, false);
    const int T = (int)q.size(0), H_q = (int)q.size(1);
    const int B = (int)cu_q.numel() - 1;
    TORCH_CHECK_VALUE(sl.numel() >= B && bt.size(0) >= B,
                      "seq_lens / block_table have fewer rows than cu_seqlens_q");
    const int64_t num_slots = kv.size(0);
    const int H_kv = (int)kv.size(1), slot_bytes = (int)kv.size(2);
    const Tensor ck = f32c(cb_k), cv = f32c(cb_v);
    void *st = stream_of(q);
    size_t need = 0;
    if (max_seq_len >= 0)
        need = cda_prefill_workspace_size(B, T, H_q, H_kv, (int)max_query_len, (int)max_seq_len);
    if (need == 0) {
        check_rc(cda_prefill_paged_hadamard(q.data_ptr(), kv.data_ptr(), num_slots, slot_bytes,
                                            H_kv, bt.data_ptr<int32_t>(), (int)bt.stride(0),
                                            cu_q.data_ptr<int32_t>(), sl.data_ptr<int32_t>(), B,
                                            ck.data_ptr<float>(), cv.data_ptr<float>(), 16,
                                            out.data_ptr(), T, H_q, (int)bs, (int)max_query_len,
                                            (float)scale, st),
                 "cda_prefill_paged_hadamard");
        return;
    }
    Workspace ws = workspace(q, need);
    check_rc(cda_prefill_paged_hadamard_ws(q.data_ptr(), kv.data_ptr(), num_slots, slot_bytes,
                                           H_kv, bt.data_ptr<int32_t>(), (int)bt.stride(0),
                                           cu_q.data_ptr<int32_t>(), sl.data_ptr<int32_t>(), B,
                                           ck.data_ptr<float>(), cv.data_ptr<float>(), 16,
                                           out.data_ptr(), T, H_q, (int)bs, (int)max_query_len,
                                           (int)max_seq_len, (float)scale, ws.ptr, ws.bytes, st),
             "cda_prefill_paged_hadamard_ws");
}

void prefill_hybrid(const Tensor &q, const Tensor &k_new, const Tensor &v_new, const Tensor &kv,
                    const Tensor &bt, const Tensor &cu_q, const Tensor &sl, const Tensor &cb_k,
                    const Tensor &cb_v, const Tensor &out, int64_t bs, int64_t max_query_len,
                    int64_t max_seq_len, double scale) {
    const DeviceGuard guard(on_gpu({&q, &k_new, &v_new, &kv, &bt, &cu_q, &sl, &cb_k, &cb_v, &out}));
    const std::pair<const Tensor *, const char *> named[] = {
        {&q, "Q"}, {&k_new, "K"}, {&v_new, "V"}, {&out, "output"}};
    for (const auto &tn : named) {
        TORCH_CHECK_TYPE(tn.first->scalar_type() == at::kHalf, tn.second, " must be fp16");
        TORCH_CHECK_VALUE(tn.first->dim() == 3 && tn.first->size(2) == 128 &&
                              tn.first->is_contiguous(),
                          tn.second, " must be a contiguous (T, heads, 128) tensor");
    }
    TORCH_CHECK_VALUE(out.sizes() == q.sizes(), "output must be shaped like Q");
    TORCH_CHECK_VALUE(k_new.sizes() == v_new.sizes() && k_new.size(0) == q.size(0),
                      "K and V must be (T, H_kv, 128) with the T of Q");
    need_dtype(cu_q, at::kInt, "cu_seqlens_q must be int32");
    check_paged(kv, bt, sl, cb_k, cb_v, false);
    const int T = (int)q.size(0), H_q = (int)q.size(1);
    const int B = (int)cu_q.numel() - 1;
    TORCH_CHECK_VALUE(sl.numel() >= B && bt.size(0) >= B,
                      "seq_lens / block_table have fewer rows than cu_seqlens_q");
    const int64_t num_slots = kv.size(0);
    const int H_kv = (int)kv.size(1), slot_bytes = (int)kv.size(2);
    TORCH_CHECK_VALUE(k_new.size(1) == H_kv, "K/V have ", k_new.size(1), " heads, the cache ",
                      H_kv);
    if (B == 0 || T == 0 || max_query_len <= 0) return;
    const size_t need = cda_prefill_hybrid_workspace_size(
        B, T, H_q, H_kv, (int)max_query_len, (int)std::max<int64_t>(1, max_seq_len));
    TORCH_CHECK_VALUE(need != 0, "unsupported hybrid prefill shape (H_q / H_kv must be 4 or 8)");
    Workspace ws = workspace(q, need);
    const Tensor ck = f32c(cb_k), cv = f32c(cb_v);
    check_rc(cda_prefill_hybrid_rawkv(q.data_ptr(), k_new.data_ptr(), v_new.data_ptr(),
                                      kv.data_ptr(), num_slots, slot_bytes, H_kv,
                                      bt.data_ptr<int32_t>(), (int)bt.stride(0),
                                      cu_q.data_ptr<int32_t>(), sl.data_ptr<int32_t>(), B,
                                      ck.data_ptr<float>(), cv.data_ptr<float>(), 16,
                                      out.data_ptr(), T, H_q, (int)bs, (int)max_query_len,
                                      (int)max_seq_len, (float)scale, ws.ptr, ws.bytes,
                                      stream_of(q)),
             "cda_prefill_hybrid_rawkv");
}

void check_dense_attn(const Tensor &q, const Tensor &k, const Tensor &v, const Tensor &out,
                      const Tensor &cu_q, const Tensor &cu_k, const Tensor &seqused,
                      const char *nq, const char *nk, const char *nv, const char *no) {
    const std::pair<const Tensor *, const char *> named[] = {{&q, nq}, {&k, nk}, {&v, nv},
                                                             {&out, no}};
    for (const auto &tn : named) {
        TORCH_CHECK_TYPE(tn.first->scalar_type() == at::kHalf, tn.second, " must be fp16");
        TORCH_CHECK_VALUE(tn.first->dim() == 3 && tn.first->size(2) == 128 &&
                              tn.first->is_contiguous(),
                          tn.second, " must be a contiguous (rows, heads, 128) tensor");
    }
    TORCH_CHECK_VALUE(k.sizes() == v.sizes() && out.sizes() == q.sizes(), nk, "/", nv, " and ",
                      nq, "/", no, " must have matching shapes");
    need_dtype(cu_q, at::kInt, "cu_seqlens_q must be int32");
    need_dtype(cu_k, at::kInt, "cu_seqlens_k must be int32");
    need_dtype(seqused, at::kInt, "seqused_k must be int32");
}

void varlen_fwd(const Tensor &q, const Tensor &k, const Tensor &v, const Tensor &out,
                const Tensor &cu_q, const Tensor &cu_k, const Tensor &seqused, int64_t max_q,
                double scale, bool causal) {
    const DeviceGuard guard(on_gpu({&q, &k, &v, &out, &cu_q, &cu_k, &seqused}));
    check_dense_attn(q, k, v, out, cu_q, cu_k, seqused, "q", "k", "v", "out");
    check_rc(cda_fa2_varlen_fwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(),
                                cu_q.data_ptr<int32_t>(), cu_k.data_ptr<int32_t>(),
                                seqused.data_ptr<int32_t>(), (int)cu_q.numel() - 1,
                                (int)q.size(0), (int)q.size(1), (int)k.size(1), (int)max_q,
                                (float)scale, causal ? 1 : 0, stream_of(q)),
             "cda_fa2_varlen_fwd");
}

void varlen_fwd_hadamard(const Tensor &q, const Tensor &k_rot, const Tensor &v_rot,
                         const Tensor &out, const Tensor &cu_q, const Tensor &cu_k,
                         const Tensor &seqused, int64_t max_q, int64_t max_k, double scale) {
    const DeviceGuard guard(on_gpu({&q, &k_rot, &v_rot, &out, &cu_q, &cu_k, &seqused}));
    check_dense_attn(q, k_rot, v_rot, out, cu_q, cu_k, seqused, "Q", "k_rot", "v_rot", "output");
    check_rc(cda_fa2_varlen_fwd_hadamard(q.data_ptr(), k_rot.data_ptr(), v_rot.data_ptr(),
                                         out.data_ptr(), cu_q.data_ptr<int32_t>(),
                                         cu_k.data_ptr<int32_t>(), seqused.data_ptr<int32_t>(),
                                         (int)cu_q.numel() - 1, (int)q.size(0), (int)q.size(1),
                                         (int)k_rot.size(1), (int)max_q, (int)max_k,
                                         (float)scale, stream_of(q)),
             "cda_fa2_varlen_fwd_hadamard");
}

std::tuple<Tensor, Tensor> paged_to_dense(const Tensor &kv, const Tensor &bt, const Tensor &sl,
                                          const Tensor &cb_k, const Tensor &cb_v, int64_t bs,
                                          int64_t max_seq_len) {
    const DeviceGuard guard(on_gpu({&kv, &bt, &sl, &cb_k, &cb_v}));
    check_paged(kv, bt, sl, cb_k, cb_v, true);
    const int B = (int)sl.numel();
    const int64_t num_slots = kv.size(0);
    const int H_kv = (int)kv.size(1), slot_bytes = (int)kv.size(2);
    Tensor k_out = at::empty({B * max_seq_len, H_kv, 128}, kv.options().dtype(at::kHalf));
    Tensor v_out = at::empty_like(k_out);
    const Tensor ck = f32c(cb_k), cv = f32c(cb_v);
    void *st = stream_of(kv);
    if (cb_k.numel() == 16 && cb_v.numel() == 4) {   // the legacy K4V2 slot
        check_rc(cda_fa2_paged_cache_to_dense_rotated_k4v2(
                     kv.data_ptr(), num_slots, slot_bytes, H_kv, bt.data_ptr<int32_t>(),
                     (int)bt.stride(0), sl.data_ptr<int32_t>(), B, ck.data_ptr<float>(),
                     cv.data_ptr<float>(), (int)bs, (int)max_seq_len, k_out.data_ptr(),
                     v_out.data_ptr(), st),
                 "cda_fa2_paged_cache_to_dense_rotated_k4v2");
    } else {
        check_rc(cda_fa2_paged_cache_to_dense_rotated(
                     kv.data_ptr(), num_slots, slot_bytes, H_kv, bt.data_ptr<int32_t>(),
                     (int)bt.stride(0), sl.data_ptr<int32_t>(), B, ck.data_ptr<float>(),
                     cv.data_ptr<float>(), 16, (int)bs, (int)max_seq_len, k_out.data_ptr(),
                     v_out.data_ptr(), st),
                 "cda_fa2_paged_cache_to_dense_rotated");
    }
    return {k_out, v_out};
}

void hadamard128(const Tensor &x, const Tensor &y, double scale) {
    const DeviceGuard guard(on_gpu({&x, &y}));
    TORCH_CHECK_TYPE(x.scalar_type() == at::kHalf && y.scalar_type() == at::kHalf,
                     "x and y must be fp16");
    TORCH_CHECK_VALUE(x.size(-1) == 128 && x.sizes() == y.sizes() && x.is_contiguous() &&
                          y.is_contiguous(),
                      "x and y must be contiguous, of one shape, last dimension 128");
    check_rc(cda_hadamard128_fp16(x.data_ptr(), y.data_ptr(), x.numel() / 128, (float)scale,
                                  stream_of(x)),
             "cda_hadamard128_fp16");
}

// ------------------------------------------------- _cda_vllm_fa2_fork_C --

// fp16(cb[code] * norm) rows (compression.py:337-361), contiguous or gathered
// from paged pools through a block table.
Tensor dequant_rows(const Tensor &codes_in, const Tensor &norms_in, const Tensor &cb_in,
                    const Tensor *bt, const Tensor *sl, int64_t bs, int64_t max_seq_len) {
    TORCH_CHECK_TYPE(codes_in.scalar_type() == at::kByte && norms_in.scalar_type() == at::kFloat,
                     "codes must be uint8, norms and cb fp32");
    const Tensor codes = codes_in.contiguous(), norms = norms_in.contiguous();
    const Tensor cb = f32c(cb_in);
    const int64_t H = codes.size(-2), cbytes = codes.size(-1);
    const int levels = (int)cb.numel();
    TORCH_CHECK_VALUE(cbytes == (levels == 16 ? 64 : 32),
                      "codes must hold 64 (16 levels) or 32 (4 levels) bytes per row");
    void *st = stream_of(codes);
    if (bt == nullptr) {
        const int64_t rows = codes.numel() / (H * cbytes);
        Tensor out = at::empty({rows, H, 128}, codes.options().dtype(at::kHalf));
        check_rc(cda_dequantize_rows(codes.data_ptr(), norms.data_ptr<float>(), rows, (int)H,
                                     cb.data_ptr<float>(), levels, nullptr, 0, nullptr, 0, 0,
                                     out.data_ptr(), st),
                 "cda_dequantize_rows");
        return out;
    }
    TORCH_CHECK_TYPE(bt->scalar_type() == at::kInt && sl->scalar_type() == at::kInt,
                     "block_table and seq_lens must be int32");
    const int64_t rows = sl->numel() * max_seq_len;
    Tensor out = at::empty({rows, H, 128}, codes.options().dtype(at::kHalf));
    check_rc(cda_dequantize_rows(codes.data_ptr(), norms.data_ptr<float>(), rows, (int)H,
                                 cb.data_ptr<float>(), levels, bt->data_ptr<int32_t>(),
                                 (int)bt->stride(0), sl->data_ptr<int32_t>(), (int)bs,
                                 (int)max_seq_len, out.data_ptr(), st),
             "cda_dequantize_rows");
    return out;
}

std::tuple<Tensor, Tensor> fork_dequantize(const Tensor &k_idx, const Tensor &k_norm,
                                           const Tensor &v_idx, const Tensor &v_norm,
                                           const Tensor &cb_k, const Tensor &cb_v) {
    const DeviceGuard guard(on_gpu({&k_idx, &k_norm, &v_idx, &v_norm, &cb_k, &cb_v}));
    return {dequant_rows(k_idx, k_norm, cb_k, nullptr, nullptr, 0, 0),
            dequant_rows(v_idx, v_norm, cb_v, nullptr, nullptr, 0, 0)};
}

void fork_unsupported(double p_dropout, int64_t wl, int64_t wr, double softcap,
                      int64_t num_splits, const c10::optional<Tensor> &alibi) {
    TORCH_CHECK_NOT_IMPLEMENTED(p_dropout == 0.0, "inference only: p_dropout must be 0");
    TORCH_CHECK_NOT_IMPLEMENTED(wl == -1 && wr == -1, "sliding windows are not supported");
    TORCH_CHECK_NOT_IMPLEMENTED(softcap == 0.0, "soft-capping is not supported");
    TORCH_CHECK_NOT_IMPLEMENTED(num_splits <= 1, "split-KV is not supported");
    TORCH_CHECK_NOT_IMPLEMENTED(!alibi.has_value(), "ALiBi is not supported");
}

Tensor seqused_of(const Tensor &cu_k, const c10::optional<Tensor> &seqused) {
    if (seqused.has_value()) return seqused->to(at::kInt).contiguous();
    return (cu_k.slice(0, 1) - cu_k.slice(0, 0, cu_k.numel() - 1)).to(at::kInt).contiguous();
}

// Returns [out, softmax_lse] as the fork's varlen ops do: softmax_lse is
// (H_q, total_q) fp32, the natural-log sum of exp(scale * q.k) over each
// query's visible keys (+inf where it sees none).
std::vector<Tensor> attend(const Tensor &q, const Tensor &k, const Tensor &v,
                           const c10::optional<Tensor> &out_opt, const Tensor &cu_q,
                           const Tensor &cu_k, const Tensor &seqused, int64_t max_q,
                           double scale, bool causal) {
    Tensor out = out_opt.has_value() ? *out_opt : at::empty(q.sizes(), q.options());
    const Tensor cq = cu_q.to(at::kInt).contiguous(), ckk = cu_k.to(at::kInt).contiguous();
    const Tensor qc = q.contiguous(), kc = k.contiguous(), vc = v.contiguous();
    const DeviceGuard guard(on_gpu({&qc, &kc, &vc, &out, &cq, &ckk, &seqused}));
    check_dense_attn(qc, kc, vc, out, cq, ckk, seqused, "q", "k", "v", "out");
    Tensor lse = at::empty({qc.size(1), qc.size(0)}, qc.options().dtype(at::kFloat));
    check_rc(cda_fa2_varlen_fwd_lse(qc.data_ptr(), kc.data_ptr(), vc.data_ptr(), out.data_ptr(),
                                    cq.data_ptr<int32_t>(), ckk.data_ptr<int32_t>(),
                                    seqused.data_ptr<int32_t>(), (int)cq.numel() - 1,
                                    (int)qc.size(0), (int)qc.size(1), (int)kc.size(1),
                                    (int)max_q, (float)scale, causal ? 1 : 0,
                                    lse.data_ptr<float>(), stream_of(qc)),
             "cda_fa2_varlen_fwd_lse");
    return {out, lse};
}

std::vector<Tensor> fork_varlen_fwd(const Tensor &q, const Tensor &k, const Tensor &v,
                                    const c10::optional<Tensor> &out, const Tensor &cu_q,
                                    const Tensor &cu_k, const c10::optional<Tensor> &seqused_k,
                                    const c10::optional<Tensor> &leftpad_k,
                                    const c10::optional<Tensor> &block_table,
                                    const c10::optional<Tensor> &alibi, int64_t max_q,
                                    int64_t /*max_k*/, double p_dropout, double scale,
                                    bool /*zero_tensors*/, bool causal, int64_t wl, int64_t wr,
                                    double softcap, bool /*return_softmax*/, int64_t num_splits,
                                    c10::optional<at::Generator> /*gen*/) {
    fork_unsupported(p_dropout, wl, wr, softcap, num_splits, alibi);
    TORCH_CHECK_NOT_IMPLEMENTED(!block_table.has_value(),
                                "paged dense K/V is not supported by varlen_fwd");
    TORCH_CHECK_NOT_IMPLEMENTED(!leftpad_k.has_value(), "leftpad_k is not supported");
    return attend(q, k, v, out, cu_q, cu_k, seqused_of(cu_k, seqused_k), max_q, scale, causal);
}

std::vector<Tensor> fork_varlen_compressed(
    const Tensor &q, const Tensor &k_idx, const Tensor &k_norm, const Tensor &v_idx,
    const Tensor &v_norm, const Tensor &cb_k, const Tensor &cb_v,
    const c10::optional<Tensor> &out, const Tensor &cu_q, const Tensor &cu_k,
    const c10::optional<Tensor> &alibi, int64_t max_q, int64_t /*max_k*/, double p_dropout,
    double scale, bool /*zero_tensors*/, bool causal, int64_t wl, int64_t wr, double softcap,
    bool /*return_softmax*/, int64_t num_splits, c10::optional<at::Generator> /*gen*/) {
    fork_unsupported(p_dropout, wl, wr, softcap, num_splits, alibi);
    auto kv = fork_dequantize(k_idx, k_norm, v_idx, v_norm, cb_k, cb_v);
    return attend(q, std::get<0>(kv), std::get<1>(kv), out, cu_q, cu_k,
                  seqused_of(cu_k, c10::nullopt), max_q, scale, causal);
}

std::vector<Tensor> fork_varlen_compressed_fused(
    const Tensor &q, const Tensor &k_idx, const Tensor &k_norm, const Tensor &v_idx,
    const Tensor &v_norm, const Tensor &cb_k, const Tensor &cb_v,
    const c10::optional<Tensor> &out, const Tensor &cu_q, const Tensor &cu_k,
    const c10::optional<Tensor> &seqused_k, const c10::optional<Tensor> &block_table,
    const c10::optional<Tensor> &alibi, int64_t max_q, int64_t max_k, double p_dropout,
    double scale, bool /*zero_tensors*/, bool causal, int64_t wl, int64_t wr, double softcap,
    bool /*return_softmax*/, int64_t num_splits, bool /*uniform_codebook*/,
    c10::optional<at::Generator> /*gen*/) {
    fork_unsupported(p_dropout, wl, wr, softcap, num_splits, alibi);
    if (!block_table.has_value()) {
        auto kv = fork_dequantize(k_idx, k_norm, v_idx, v_norm, cb_k, cb_v);
        return attend(q, std::get<0>(kv), std::get<1>(kv), out, cu_q, cu_k,
                      seqused_of(cu_k, seqused_k), max_q, scale, causal);
    }
    // Paged pools (num_blocks, block_size, H_kv, D/2) + (num_blocks, block_size,
    // H_kv): each sequence's tokens gathered into dense rows b * max_k + t.
    TORCH_CHECK_VALUE(seqused_k.has_value(), "a paged call needs seqused_k");
    TORCH_CHECK_VALUE(k_idx.dim() == 4, "paged k_idx must be (num_blocks, block_size, H, D/2)");
    const int64_t nb = k_idx.size(0), bs = k_idx.size(1), H = k_idx.size(2),
                  cbytes = k_idx.size(3);
    const Tensor bt = block_table->to(at::kInt).contiguous();
    const Tensor sl = seqused_k->to(at::kInt).contiguous();
    const DeviceGuard guard(on_gpu({&q, &k_idx, &k_norm, &v_idx, &v_norm, &cb_k, &cb_v}));
    const Tensor kd = dequant_rows(k_idx.reshape({nb * bs, H, cbytes}),
                                   k_norm.reshape({nb * bs, H}), cb_k, &bt, &sl, bs, max_k);
    const Tensor vd = dequant_rows(v_idx.reshape({nb * bs, H, cbytes}),
                                   v_norm.reshape({nb * bs, H}), cb_v, &bt, &sl, bs, max_k);
    const Tensor cu_dense =
        at::arange(sl.numel() + 1, q.options().dtype(at::kInt)) * (int32_t)max_k;
    return attend(q, kd, vd, out, cu_q, cu_dense, sl, max_q, scale, causal);
}

// ------------------------------------------------------------ Meta kernels --

void nothing_decode(const Tensor &, const Tensor &, const Tensor &, const Tensor &,
                    const Tensor &, const Tensor &, const Tensor &, const Tensor &, const Tensor &,
                    int64_t, int64_t, int64_t, int64_t, double) {}
void nothing_decode_uqk(const Tensor &, const Tensor &, const Tensor &, const Tensor &,
                        const Tensor &, const Tensor &, const Tensor &, const Tensor &, int64_t,
                        int64_t, int64_t, int64_t, double) {}
void nothing_scores(const Tensor &, const Tensor &, const Tensor &, const Tensor &, int64_t,
                    double, bool, int64_t, int64_t, int64_t) {}
void nothing_encode(const Tensor &, const Tensor &, const Tensor &, const Tensor &,
                    const Tensor &, const Tensor &) {}
void nothing_prefill(const Tensor &, const Tensor &, const Tensor &, const Tensor &,
                     const Tensor &, const Tensor &, const Tensor &, const Tensor &, int64_t,
                     int64_t, double, int64_t) {}
void nothing_hybrid(const Tensor &, const Tensor &, const Tensor &, const Tensor &,
                    const Tensor &, const Tensor &, const Tensor &, const Tensor &,
                    const Tensor &, const Tensor &, int64_t, int64_t, int64_t, double) {}
void nothing_varlen(const Tensor &, const Tensor &, const Tensor &, const Tensor &,
                    const Tensor &, const Tensor &, const Tensor &, int64_t, double, bool) {}
void nothing_varlen_h(const Tensor &, const Tensor &, const Tensor &, const Tensor &,
                      const Tensor &, const Tensor &, const Tensor &, int64_t, int64_t, double) {}
void nothing_hadamard(const Tensor &, const Tensor &, double) {}

std::tuple<Tensor, Tensor> meta_paged_to_dense(const Tensor &kv, const Tensor &, const Tensor &sl,
                                               const Tensor &, const Tensor &, int64_t,
                                               int64_t max_seq_len) {
    Tensor k = at::empty({sl.numel() * max_seq_len, kv.size(1), 128},
                         kv.options().dtype(at::kHalf));
    return {k, at::empty_like(k)};
}

std::tuple<Tensor, Tensor> meta_dequantize(const Tensor &k_idx, const Tensor &, const Tensor &v_idx,
                                           const Tensor &, const Tensor &, const Tensor &) {
    return {at::empty({k_idx.size(0), k_idx.size(1), 128}, k_idx.options().dtype(at::kHalf)),
            at::empty({v_idx.size(0), v_idx.size(1), 128}, v_idx.options().dtype(at::kHalf))};
}

std::vector<Tensor> meta_fork_out(const Tensor &q, const c10::optional<Tensor> &out) {
    return {out.has_value() ? *out : at::empty_like(q),
            at::empty({q.size(1), q.size(0)}, q.options().dtype(at::kFloat))};
}

std::vector<Tensor> meta_fork_varlen(const Tensor &q, const Tensor &, const Tensor &,
                                     const c10::optional<Tensor> &out, const Tensor &,
                                     const Tensor &, const c10::optional<Tensor> &,
                                     const c10::optional<Tensor> &, const c10::optional<Tensor> &,
                                     const c10::optional<Tensor> &, int64_t, int64_t, double,
                                     double, bool, bool, int64_t, int64_t, double, bool, int64_t,
                                     c10::optional<at::Generator>) {
    return meta_fork_out(q, out);
}

std::vector<Tensor> meta_fork_compressed(const Tensor &q, const Tensor &, const Tensor &,
                                         const Tensor &, const Tensor &, const Tensor &,
                                         const Tensor &, const c10::optional<Tensor> &out,
                                         const Tensor &, const Tensor &,
                                         const c10::optional<Tensor> &, int64_t, int64_t, double,
                                         double, bool, bool, int64_t, int64_t, double, bool,
                                         int64_t, c10::optional<at::Generator>) {
    return meta_fork_out(q, out);
}

std::vector<Tensor> meta_fork_fused(const Tensor &q, const Tensor &, const Tensor &,
                                    const Tensor &, const Tensor &, const Tensor &,
                                    const Tensor &, const c10::optional<Tensor> &out,
                                    const Tensor &, const Tensor &,
                                    const c10::optional<Tensor> &, const c10::optional<Tensor> &,
                                    const c10::optional<Tensor> &, int64_t, int64_t, double,
                                    double, bool, bool, int64_t, int64_t, double, bool, int64_t,
                                    bool, c10::optional<at::Generator>) {
    return meta_fork_out(q, out);
}

}  // namespace

// Schemas mirror the reference signatures (wrappers.py:115-124, 153-156;
// fa2_cda.py:51-52, 85-95, 166-181; interface.py:154-161, 234-257, 304-328,
// 434-461), outputs written in place annotated Tensor(a!).
TORCH_LIBRARY(cda_hip, m) {
    m.def("decode(Tensor q, Tensor kv_cache, Tensor block_table, Tensor seq_lens, "
          "Tensor cb_k, Tensor cb_v, Tensor rot_f32, Tensor rot_f16, Tensor(a!) out, "
          "int group_size, int block_size, int tile_n, int max_seq_len, float scale) -> ()");
    m.def("decode_uniform_qk(Tensor q, Tensor kv_cache, Tensor block_table, Tensor seq_lens, "
          "Tensor cb_k, Tensor cb_v, Tensor rot_f32, Tensor(a!) out, int group_size, "
          "int block_size, int tile_n, int max_seq_len, float scale) -> ()");
    m.def("qk_scores_uniform4(Tensor q_rot, Tensor k_idx, Tensor k_norm, Tensor(a!) out, "
          "int group_size, float scale, bool causal, int q_offset, int key_start, "
          "int key_end) -> ()");
    m.def("encode(Tensor k, Tensor v, Tensor slot_mapping, Tensor(a!) flat_cache, Tensor cb_k, "
          "Tensor cb_v) -> ()");
    m.def("prefill(Tensor q, Tensor kv_cache, Tensor block_table, Tensor cu_seqlens_q, "
          "Tensor seq_lens, Tensor cb_k, Tensor cb_v, Tensor(a!) out, int block_size, "
          "int max_query_len, float scale, int max_seq_len=-1) -> ()");
    m.def("prefill_hybrid(Tensor q, Tensor k_new, Tensor v_new, Tensor kv_cache, "
          "Tensor block_table, Tensor cu_seqlens_q, Tensor seq_lens, Tensor cb_k, Tensor cb_v, "
          "Tensor(a!) out, int block_size, int max_query_len, int max_seq_len, float scale) -> ()");
    m.def("varlen_fwd(Tensor q, Tensor k, Tensor v, Tensor(a!) out, Tensor cu_seqlens_q, "
          "Tensor cu_seqlens_k, Tensor seqused_k, int max_seqlen_q, float scale, bool causal) "
          "-> ()");
    m.def("paged_to_dense(Tensor kv_cache, Tensor block_table, Tensor seq_lens, Tensor cb_k, "
          "Tensor cb_v, int block_size, int max_seq_len) -> (Tensor, Tensor)");
    m.def("varlen_fwd_hadamard(Tensor q, Tensor k_rot, Tensor v_rot, Tensor(a!) out, "
          "Tensor cu_seqlens_q, Tensor cu_seqlens_k, Tensor seqused_k, int max_seqlen_q, "
          "int max_seqlen_k, float scale) -> ()");
    m.def("hadamard128(Tensor x, Tensor(a!) y, float scale) -> ()");
}

TORCH_LIBRARY_IMPL(cda_hip, CUDA, m) {
    m.impl("decode", &decode);
    m.impl("decode_uniform_qk", &decode_uniform_qk);
    m.impl("qk_scores_uniform4", &qk_scores_uniform4);
    m.impl("encode", &encode);
    m.impl("prefill", &prefill);
    m.impl("prefill_hybrid", &prefill_hybrid);
    m.impl("varlen_fwd", &varlen_fwd);
    m.impl("paged_to_dense", &paged_to_dense);
    m.impl("varlen_fwd_hadamard", &varlen_fwd_hadamard);
    m.impl("hadamard128", &hadamard128);
}

TORCH_LIBRARY_IMPL(cda_hip, Meta, m) {
    m.impl("decode", &nothing_decode);
    m.impl("decode_uniform_qk", &nothing_decode_uqk);
    m.impl("qk_scores_uniform4", &nothing_scores);
    m.impl("encode", &nothing_encode);
    m.impl("prefill", &nothing_prefill);
    m.impl("prefill_hybrid", &nothing_hybrid);
    m.impl("varlen_fwd", &nothing_varlen);
    m.impl("paged_to_dense", &meta_paged_to_dense);
    m.impl("varlen_fwd_hadamard", &nothing_varlen_h);
    m.impl("hadamard128", &nothing_hadamard);
}

#define CDA_FORK_TAIL                                                                        \
    "int max_seqlen_q, int max_seqlen_k, float p_dropout, float softmax_scale, "             \
    "bool zero_tensors, bool is_causal, int window_size_left, int window_size_right, "      \
    "float softcap, bool return_softmax, int num_splits"

TORCH_LIBRARY(_cda_vllm_fa2_fork_C, m) {
    m.def("dequantize_compressed_kv(Tensor k_idx, Tensor k_norm, Tensor v_idx, Tensor v_norm, "
          "Tensor cb_k, Tensor cb_v) -> (Tensor, Tensor)");
    m.def("varlen_fwd(Tensor q, Tensor k, Tensor v, Tensor(a!)? out, Tensor cu_seqlens_q, "
          "Tensor cu_seqlens_k, Tensor? seqused_k, Tensor? leftpad_k, Tensor? block_table, "
          "Tensor? alibi_slopes, " CDA_FORK_TAIL ", Generator? gen) -> Tensor[]");
    m.def("varlen_fwd_compressed_kv(Tensor q, Tensor k_idx, Tensor k_norm, Tensor v_idx, "
          "Tensor v_norm, Tensor cb_k, Tensor cb_v, Tensor(a!)? out, Tensor cu_seqlens_q, "
          "Tensor cu_seqlens_k, Tensor? alibi_slopes, " CDA_FORK_TAIL
          ", Generator? gen) -> Tensor[]");
    m.def("varlen_fwd_compressed_kv_fused(Tensor q, Tensor k_idx, Tensor k_norm, Tensor v_idx, "
          "Tensor v_norm, Tensor cb_k, Tensor cb_v, Tensor(a!)? out, Tensor cu_seqlens_q, "
          "Tensor cu_seqlens_k, Tensor? seqused_k, Tensor? block_table, Tensor? alibi_slopes, "
          CDA_FORK_TAIL ", bool uniform_codebook, Generator? gen) -> Tensor[]");
}

TORCH_LIBRARY_IMPL(_cda_vllm_fa2_fork_C, CUDA, m) {
    m.impl("dequantize_compressed_kv", &fork_dequantize);
    m.impl("varlen_fwd", &fork_varlen_fwd);
    m.impl("varlen_fwd_compressed_kv", &fork_varlen_compressed);
    m.impl("varlen_fwd_compressed_kv_fused", &fork_varlen_compressed_fused);
}

TORCH_LIBRARY_IMPL(_cda_vllm_fa2_fork_C, Meta, m) {
    m.impl("dequantize_compressed_kv", &meta_dequantize);
    m.impl("varlen_fwd", &meta_fork_varlen);
    m.impl("varlen_fwd_compressed_kv", &meta_fork_compressed);
    m.impl("varlen_fwd_compressed_kv_fused", &meta_fork_fused);
}
