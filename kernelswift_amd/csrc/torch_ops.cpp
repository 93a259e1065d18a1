// PyTorch operator registration of the KernelSwift MI355X operators: TORCH_LIBRARY(ks_mi355x, ...).
//
// The reference registers its Ascend kernels as torch operators (sinkhorn_ops::sinkhorn_kernel_basic,
// optimized/sinkhorn_project/op_extension/sinkhorn_torch.cpp:59-66; indexer_ops::rope_inplace /
// fused_qk_reduce / topk_mask, optimized/indexer_project/op_extension/indexer_torch.cpp:272-276;
// npu::sparse_attn_megakernel_basic, optimized/sparse_attention/op_extension/register.cpp:7-16).  This
// translation unit is the same kind of boundary for the gfx950 kernels: each op validates its tensors
// (TORCH_CHECK, RuntimeError in Python), allocates its outputs and workspace with the caching allocator on
// the input's device, and enqueues the kernels through the C ABI of libkswift_amd.so (include/kswift.h) on
// the current HIP stream, without synchronising.  Host code only; built by kernelswift_amd/build.py into
// libkswift_torch.so and loaded with torch.ops.load_library.
#include <ATen/ATen.h>
#include <c10/hip/HIPStream.h>
#include <torch/library.h>

#include "../../include/kswift.h"

namespace {

void* current_stream(const at::Tensor& t) {
  return static_cast<void*>(c10::hip::getCurrentHIPStream(t.device().index()).stream());
}

void check_rc(int rc, const char* what) { TORCH_CHECK(rc == KS_OK, what, ": ", ks_last_error(), " (code ", rc, ")"); }

void check_gpu(const at::Tensor& t, const char* name, bool contiguous = true) {
  TORCH_CHECK(t.is_cuda(), name, " must be on the GPU (there is no CPU path)");
  TORCH_CHECK(!contiguous || t.is_contiguous(), name, " must be contiguous");
}

// ---------------------------------------------------------------- Sinkhorn
at::Tensor sinkhorn(const at::Tensor& x, int64_t repeat, double eps) {
  check_gpu(x, "x");
  TORCH_CHECK(x.scalar_type() == at::kFloat, "x must be float32");
  TORCH_CHECK(x.dim() >= 2 && x.size(-1) == 4 && x.size(-2) == 4, "x must be [..., 4, 4]");
  TORCH_CHECK(repeat >= 1, "repeat must be >= 1");
  at::Tensor out = at::empty_like(x);
  check_rc(ks_sinkhorn(x.data_ptr<float>(), out.data_ptr<float>(), x.numel() / 16, static_cast<int32_t>(repeat),
                       static_cast<float>(eps), current_stream(x)),
           "ks_mi355x::sinkhorn");
  return out;
}

// ---------------------------------------------------------------- indexer
void indexer_rope(at::Tensor x, const at::Tensor& freqs, int64_t rope_start, int64_t rope_dim, int64_t pos0) {
  check_gpu(x, "x");
  check_gpu(freqs, "freqs");
  TORCH_CHECK(x.scalar_type() == at::kBFloat16, "x must be bfloat16");
  TORCH_CHECK(freqs.scalar_type() == at::kFloat && freqs.dim() == 3 && freqs.size(2) == 2,
              "freqs must be float32 [rows, rope_dim/2, 2]");
  TORCH_CHECK(x.dim() == 3 || x.dim() == 4, "x must be [b, s, h, d] or [b, s, d]");
  TORCH_CHECK(rope_dim == 2 * freqs.size(1), "rope_dim must equal 2 * freqs.size(1)");
  const int64_t H = x.dim() == 4 ? x.size(2) : 1;
  check_rc(ks_rope_inplace(reinterpret_cast<uint16_t*>(x.data_ptr()), freqs.data_ptr<float>(), x.size(0), x.size(1),
                           H, x.size(-1), rope_start, rope_dim, pos0, freqs.size(0), current_stream(x)),
           "ks_mi355x::indexer_rope");
}

int32_t weights_bf16(const at::Tensor& w) {
  TORCH_CHECK(w.scalar_type() == at::kFloat || w.scalar_type() == at::kBFloat16, "weights must be float32 or bfloat16");
  return w.scalar_type() == at::kBFloat16 ? 1 : 0;
}

at::Tensor indexer_scores(const at::Tensor& q, const at::Tensor& k, const at::Tensor& weights, bool causal,
                          int64_t start_pos, int64_t ratio, c10::optional<int64_t> T_opt) {
  check_gpu(q, "q");
  check_gpu(k, "k");
  check_gpu(weights, "weights");
  TORCH_CHECK(q.scalar_type() == at::kBFloat16 && k.scalar_type() == at::kBFloat16, "q and k must be bfloat16");
  const int32_t wbf = weights_bf16(weights);
  TORCH_CHECK(q.dim() == 4 && k.dim() == 3 && weights.dim() == 3, "q [b,s,h,d], k [b,t,d], weights [b,s,h]");
  const int64_t B = q.size(0), S = q.size(1), H = q.size(2), D = q.size(3), Tk = k.size(1);
  TORCH_CHECK(k.size(0) == B && k.size(2) == D, "k shape mismatch");
  TORCH_CHECK(weights.size(0) == B && weights.size(1) == S && weights.size(2) == H, "weights shape mismatch");
  const int64_t T = T_opt.value_or(Tk);
  TORCH_CHECK(T >= 1 && T <= Tk, "T out of range");
  auto f32 = q.options().dtype(at::kFloat);
  auto i32 = q.options().dtype(at::kInt);
  at::Tensor qn = at::empty({B * S * H}, f32), qs = at::empty({B * S * H}, i32);
  at::Tensor kn = at::empty({B * Tk}, f32), ksp = at::empty({B * Tk}, i32);
  void* st = current_stream(q);
  check_rc(ks_indexer_row_stats(reinterpret_cast<const uint16_t*>(q.data_ptr()), B * S * H, D, qn.data_ptr<float>(),
                                qs.data_ptr<int32_t>(), st),
           "ks_mi355x::indexer_scores (q statistics)");
  check_rc(ks_indexer_row_stats(reinterpret_cast<const uint16_t*>(k.data_ptr()), B * Tk, D, kn.data_ptr<float>(),
                                ksp.data_ptr<int32_t>(), st),
           "ks_mi355x::indexer_scores (k statistics)");
  at::Tensor out = at::empty({B, S, T}, f32);
  check_rc(ks_indexer_scores(reinterpret_cast<const uint16_t*>(q.data_ptr()),
                             reinterpret_cast<const uint16_t*>(k.data_ptr()), weights.data_ptr(), wbf,
                             qn.data_ptr<float>(), qs.data_ptr<int32_t>(), kn.data_ptr<float>(), ksp.data_ptr<int32_t>(),
                             out.data_ptr<float>(), B, S, H, D, T, Tk, causal ? 1 : 0, start_pos,
                             static_cast<int32_t>(ratio), st),
           "ks_mi355x::indexer_scores");
  return out;
}

at::Tensor indexer_topk(const at::Tensor& scores, bool causal, int64_t ratio, int64_t actual_t, int64_t offset,
                        int64_t k, int64_t start_pos, bool out_i64) {
  check_gpu(scores, "scores", false);
  TORCH_CHECK(scores.scalar_type() == at::kFloat, "scores must be float32");
  TORCH_CHECK(scores.dim() == 3 && scores.stride(2) == 1 && scores.stride(0) == scores.size(1) * scores.stride(1),
              "scores must be [b, s, ld] with contiguous rows");
  TORCH_CHECK(actual_t >= 1 && actual_t <= scores.size(2), "actual_t=", actual_t,
              " must be in [1, scores.size(2)=", scores.size(2), "]");
  const int64_t kk = std::min(k, actual_t);
  at::Tensor out = at::empty({scores.size(0), scores.size(1), kk}, scores.options().dtype(out_i64 ? at::kLong : at::kInt));
  check_rc(ks_indexer_topk(scores.data_ptr<float>(), scores.stride(1), scores.size(0), scores.size(1), actual_t, kk,
                           causal ? 1 : 0, start_pos, static_cast<int32_t>(ratio), offset, out.data_ptr(),
                           out_i64 ? 1 : 0, current_stream(scores)),
           "ks_mi355x::indexer_topk");
  return out;
}

at::Tensor indexer(const at::Tensor& q, const at::Tensor& k, const at::Tensor& weights,
                   const c10::optional<at::Tensor>& freqs, int64_t k_top, bool causal, int64_t start_pos, int64_t ratio,
                   int64_t offset, int64_t rope_start, int64_t rope_dim, bool rope_k, bool out_i64,
                   c10::optional<int64_t> T_opt, double w_scale) {
  check_gpu(q, "q");
  check_gpu(weights, "weights");
  check_gpu(k, "k", false);
  TORCH_CHECK(q.scalar_type() == at::kBFloat16 && k.scalar_type() == at::kBFloat16, "q and k must be bfloat16");
  const int32_t wbf = weights_bf16(weights);
  TORCH_CHECK(q.dim() == 4 && k.dim() == 3 && weights.dim() == 3, "q [b,s,h,d], k [b,t,d], weights [b,s,h]");
  const int64_t B = q.size(0), S = q.size(1), H = q.size(2), D = q.size(3);
  TORCH_CHECK(k.size(0) >= B && k.size(2) == D, "k shape mismatch");
  TORCH_CHECK(weights.size(0) == B && weights.size(1) == S && weights.size(2) == H, "weights shape mismatch");
  TORCH_CHECK(k.stride(2) == 1 && k.stride(1) == D && k.stride(0) % D == 0, "k rows must be contiguous");
  const int64_t T = T_opt.value_or(k.size(1));
  TORCH_CHECK(T >= 1 && T <= k.size(1), "T out of range");
  const int64_t kbs = B > 1 ? k.stride(0) / D : std::max(k.size(1), T);
  const float* fp = nullptr;
  int64_t frows = 0;
  if (rope_dim > 0) {
    TORCH_CHECK(freqs.has_value(), "freqs is required when rope_dim > 0");
    const at::Tensor& f = *freqs;
    check_gpu(f, "freqs");
    TORCH_CHECK(f.scalar_type() == at::kFloat && f.dim() == 3 && f.size(1) * 2 == rope_dim && f.size(2) == 2,
                "freqs must be float32 [rows, rope_dim/2, 2]");
    fp = f.data_ptr<float>();
    frows = f.size(0);
  }
  const size_t need = ks_indexer_workspace_size(B, S, H, D, T);
  at::Tensor ws = at::empty({static_cast<int64_t>(std::max<size_t>(need, 1))}, q.options().dtype(at::kByte));
  const int64_t kk = std::min(k_top, T);
  at::Tensor out = at::empty({B, S, kk}, q.options().dtype(out_i64 ? at::kLong : at::kInt));
  check_rc(ks_indexer_scaled(reinterpret_cast<const uint16_t*>(q.data_ptr()),
                             reinterpret_cast<const uint16_t*>(k.data_ptr()), weights.data_ptr(), wbf,
                             static_cast<float>(w_scale), fp, frows, rope_start, rope_dim, rope_k ? 1 : 0, k_top,
                             causal ? 1 : 0, start_pos, static_cast<int32_t>(ratio), offset, out.data_ptr(),
                             out_i64 ? 1 : 0, B, S, H, D, T, kbs, ws.data_ptr(), ws.numel(), current_stream(q)),
           "ks_mi355x::indexer");
  return out;
}

// ---------------------------------------------------------------- FP8 indexer
std::tuple<at::Tensor, at::Tensor> fp8_quant(const at::Tensor& x, int64_t block, bool ue8m0) {
  check_gpu(x, "x");
  TORCH_CHECK(x.scalar_type() == at::kBFloat16, "x must be bfloat16");
  TORCH_CHECK(x.dim() >= 1 && block > 0 && x.size(-1) % block == 0, "the last dim must be a multiple of block");
  const int64_t D = x.size(-1);
  const int64_t rows = D ? x.numel() / D : 0;
  at::Tensor codes = at::empty(x.sizes(), x.options().dtype(at::kFloat8_e4m3fn));
  std::vector<int64_t> ss(x.sizes().begin(), x.sizes().end());
  ss.back() = D / block;
  at::Tensor scales = at::empty(ss, x.options().dtype(at::kFloat));
  check_rc(ks_fp8_quant_rows(reinterpret_cast<const uint16_t*>(x.data_ptr()), rows, D, block, ue8m0 ? 1 : 0,
                             reinterpret_cast<uint8_t*>(codes.data_ptr()), scales.data_ptr<float>(), current_stream(x)),
           "ks_mi355x::fp8_quant");
  return {codes, scales};
}

void check_codes(const at::Tensor& t, const char* name) {
  TORCH_CHECK(t.scalar_type() == at::kFloat8_e4m3fn || t.scalar_type() == at::kByte, name,
              " must be float8_e4m3fn (or its uint8 bits)");
}

at::Tensor indexer_fp8(const at::Tensor& q, const at::Tensor& q_scale, const at::Tensor& k, const at::Tensor& k_scale,
                       const at::Tensor& weights, int64_t k_top, bool causal, int64_t start_pos, int64_t ratio,
                       int64_t offset, bool out_i64, c10::optional<int64_t> T_opt) {
  check_gpu(q, "q");
  check_gpu(q_scale, "q_scale");
  check_gpu(weights, "weights");
  check_gpu(k, "k", false);
  check_gpu(k_scale, "k_scale", false);
  check_codes(q, "q");
  check_codes(k, "k");
  TORCH_CHECK(q_scale.scalar_type() == at::kFloat && k_scale.scalar_type() == at::kFloat, "scales must be float32");
  const int32_t wbf = weights_bf16(weights);
  TORCH_CHECK(q.dim() == 4 && k.dim() == 3 && weights.dim() == 3, "q [b,s,h,d], k [b,t,d], weights [b,s,h]");
  const int64_t B = q.size(0), S = q.size(1), H = q.size(2), D = q.size(3);
  TORCH_CHECK(k.size(0) >= B && k.size(2) == D, "k shape mismatch");
  TORCH_CHECK(weights.size(0) == B && weights.size(1) == S && weights.size(2) == H, "weights shape mismatch");
  TORCH_CHECK(q_scale.dim() == 3 && q_scale.size(0) == B && q_scale.size(1) == S && q_scale.size(2) == H,
              "q_scale must be [b, s, h]");
  TORCH_CHECK(k.stride(2) == 1 && k.stride(1) == D && k.stride(0) % D == 0, "k rows must be contiguous");
  TORCH_CHECK(k_scale.dim() == 2 && k_scale.size(0) >= B && k_scale.size(1) == k.size(1) && k_scale.stride(1) == 1,
              "k_scale must be [b, t] with contiguous rows");
  const int64_t T = T_opt.value_or(k.size(1));
  TORCH_CHECK(T >= 1 && T <= k.size(1), "T out of range");
  const int64_t kbs = B > 1 ? k.stride(0) / D : std::max(k.size(1), T);
  TORCH_CHECK(B <= 1 || k_scale.stride(0) == kbs, "k_scale must have the batch stride of k (in rows)");
  const size_t need = ks_indexer_workspace_size(B, S, H, D, T);
  at::Tensor ws = at::empty({static_cast<int64_t>(std::max<size_t>(need, 1))}, q.options().dtype(at::kByte));
  const int64_t kk = std::min(k_top, T);
  at::Tensor out = at::empty({B, S, kk}, q.options().dtype(out_i64 ? at::kLong : at::kInt));
  check_rc(ks_indexer_fp8(reinterpret_cast<const uint8_t*>(q.data_ptr()), q_scale.data_ptr<float>(),
                          reinterpret_cast<const uint8_t*>(k.data_ptr()), k_scale.data_ptr<float>(), weights.data_ptr(),
                          wbf, k_top, causal ? 1 : 0, start_pos, static_cast<int32_t>(ratio), offset, out.data_ptr(),
                          out_i64 ? 1 : 0, B, S, H, D, T, kbs, ws.data_ptr(), ws.numel(), current_stream(q)),
           "ks_mi355x::indexer_fp8");
  return out;
}

// ---------------------------------------------------------------- sparse attention
at::Tensor sparse_attn(const at::Tensor& q, const at::Tensor& kv, const at::Tensor& attn_sink,
                       const at::Tensor& topk_idxs, double softmax_scale, c10::optional<int64_t> dv_opt) {
  check_gpu(q, "q");
  check_gpu(kv, "kv");
  check_gpu(attn_sink, "attn_sink");
  check_gpu(topk_idxs, "topk_idxs");
  TORCH_CHECK(q.scalar_type() == at::kBFloat16 && kv.scalar_type() == at::kBFloat16, "q and kv must be bfloat16");
  TORCH_CHECK(attn_sink.scalar_type() == at::kFloat, "attn_sink must be float32");
  TORCH_CHECK(topk_idxs.scalar_type() == at::kInt, "topk_idxs must be int32");
  TORCH_CHECK(q.dim() == 4 && kv.dim() == 3 && attn_sink.dim() == 1 && topk_idxs.dim() == 3,
              "q [b,m,h,d], kv [b,n,d], attn_sink [h], topk_idxs [b,m,topk]");
  const int64_t B = q.size(0), M = q.size(1), H = q.size(2), D = q.size(3), N = kv.size(1), K = topk_idxs.size(2);
  TORCH_CHECK(kv.size(0) == B && kv.size(2) == D, "kv shape mismatch");
  TORCH_CHECK(attn_sink.size(0) == H, "attn_sink shape mismatch");
  TORCH_CHECK(topk_idxs.size(0) == B && topk_idxs.size(1) == M, "topk_idxs shape mismatch");
  const int64_t dv = dv_opt.value_or(D);
  at::Tensor out = at::empty({B, M, H, dv}, q.options());
  const size_t need = ks_sparse_attn_workspace_size(B, M, H, D, dv, K);
  at::Tensor ws;
  if (need) ws = at::empty({static_cast<int64_t>(need)}, q.options().dtype(at::kByte));
  check_rc(ks_sparse_attn(reinterpret_cast<const uint16_t*>(q.data_ptr()), reinterpret_cast<const uint16_t*>(kv.data_ptr()),
                          attn_sink.data_ptr<float>(), topk_idxs.data_ptr<int32_t>(),
                          reinterpret_cast<uint16_t*>(out.data_ptr()), B, M, H, D, dv, N, K,
                          static_cast<float>(softmax_scale), need ? ws.data_ptr() : nullptr, need, current_stream(q)),
           "ks_mi355x::sparse_attn");
  return out;
}

// ---------------------------------------------------------------- mHC hyper-connections
void check_streams(const at::Tensor& x) {
  check_gpu(x, "x");
  TORCH_CHECK(x.scalar_type() == at::kBFloat16, "x must be bfloat16");
  TORCH_CHECK(x.dim() == 3 && x.size(1) == 4 && x.size(2) % 8 == 0, "x must be [N, 4, C] with C a multiple of 8");
}

at::Tensor mhc_pre(const at::Tensor& x, const at::Tensor& pre_logits) {
  check_streams(x);
  check_gpu(pre_logits, "pre_logits");
  TORCH_CHECK(pre_logits.scalar_type() == at::kFloat && pre_logits.dim() == 2 && pre_logits.size(0) == x.size(0) &&
                  pre_logits.size(1) == 4,
              "pre_logits must be float32 [N, 4]");
  at::Tensor h = at::empty({x.size(0), x.size(2)}, x.options());
  check_rc(ks_mhc_pre(reinterpret_cast<const uint16_t*>(x.data_ptr()), pre_logits.data_ptr<float>(),
                      reinterpret_cast<uint16_t*>(h.data_ptr()), x.size(0), x.size(2), current_stream(x)),
           "ks_mi355x::mhc_pre");
  return h;
}

at::Tensor mhc_post(const at::Tensor& x, const at::Tensor& f, const at::Tensor& res_logits,
                    const at::Tensor& post_logits, int64_t sinkhorn_iters, double eps) {
  check_streams(x);
  check_gpu(f, "f");
  check_gpu(res_logits, "res_logits");
  check_gpu(post_logits, "post_logits");
  const int64_t N = x.size(0), C = x.size(2);
  TORCH_CHECK(f.scalar_type() == at::kBFloat16 && f.dim() == 2 && f.size(0) == N && f.size(1) == C,
              "f must be bfloat16 [N, C]");
  TORCH_CHECK(res_logits.scalar_type() == at::kFloat && res_logits.dim() == 3 && res_logits.size(0) == N &&
                  res_logits.size(1) == 4 && res_logits.size(2) == 4,
              "res_logits must be float32 [N, 4, 4]");
  TORCH_CHECK(post_logits.scalar_type() == at::kFloat && post_logits.dim() == 2 && post_logits.size(0) == N &&
                  post_logits.size(1) == 4,
              "post_logits must be float32 [N, 4]");
  at::Tensor out = at::empty_like(x);
  check_rc(ks_mhc_post(reinterpret_cast<const uint16_t*>(x.data_ptr()), reinterpret_cast<const uint16_t*>(f.data_ptr()),
                       res_logits.data_ptr<float>(), post_logits.data_ptr<float>(),
                       reinterpret_cast<uint16_t*>(out.data_ptr()), N, C, static_cast<int32_t>(sinkhorn_iters),
                       static_cast<float>(eps), current_stream(x)),
           "ks_mi355x::mhc_post");
  return out;
}

}  // namespace

TORCH_LIBRARY(ks_mi355x, m) {
  m.def("sinkhorn(Tensor x, int repeat=10, float eps=1e-06) -> Tensor");
  m.def("indexer_rope(Tensor(a!) x, Tensor freqs, int rope_start, int rope_dim, int pos0=0) -> ()");
  m.def("indexer_scores(Tensor q, Tensor k, Tensor weights, bool causal, int start_pos=0, int ratio=1, "
        "int? T=None) -> Tensor");
  m.def("indexer_topk(Tensor scores, bool causal, int ratio, int actual_t, int offset, int k, int start_pos=0, "
        "bool out_i64=True) -> Tensor");
  m.def("indexer(Tensor q, Tensor k, Tensor weights, Tensor? freqs, int k_top, bool causal, int start_pos, "
        "int ratio=1, int offset=0, int rope_start=0, int rope_dim=64, bool rope_k=True, bool out_i64=False, "
        "int? T=None, float w_scale=1.0) -> Tensor");
  m.def("sparse_attn(Tensor q, Tensor kv, Tensor attn_sink, Tensor topk_idxs, float softmax_scale, "
        "int? dv=None) -> Tensor");
  m.def("fp8_quant(Tensor x, int block=128, bool ue8m0=True) -> (Tensor, Tensor)");
  m.def("indexer_fp8(Tensor q, Tensor q_scale, Tensor k, Tensor k_scale, Tensor weights, int k_top, bool causal, "
        "int start_pos, int ratio=1, int offset=0, bool out_i64=False, int? T=None) -> Tensor");
  m.def("mhc_pre(Tensor x, Tensor pre_logits) -> Tensor");
  m.def("mhc_post(Tensor x, Tensor f, Tensor res_logits, Tensor post_logits, int sinkhorn_iters=20, "
        "float eps=1e-06) -> Tensor");
}

TORCH_LIBRARY_IMPL(ks_mi355x, CUDA, m) {
  m.impl("sinkhorn", &sinkhorn);
  m.impl("indexer_rope", &indexer_rope);
  m.impl("indexer_scores", &indexer_scores);
  m.impl("indexer_topk", &indexer_topk);
  m.impl("indexer", &indexer);
  m.impl("sparse_attn", &sparse_attn);
  m.impl("fp8_quant", &fp8_quant);
  m.impl("indexer_fp8", &indexer_fp8);
  m.impl("mhc_pre", &mhc_pre);
  m.impl("mhc_post", &mhc_post);
}
