// torch operators over the C ABI of librlt_mi355x.so: the hot-path entry points as
// ``torch.ops.rlt_mi355x.<name>`` with a fixed schema and a ROCm (CUDA dispatch key)
// implementation, the way the reference binds its native code
// (csrc/torch_bindings.cpp:7-13: TORCH_LIBRARY schema + implementation).  Argument
// checks raise ValueError (TORCH_CHECK_VALUE) with the Python wrappers' messages; a
// kernel status other than RLT_OK raises RuntimeError.  Every operator launches on
// the tensor device's current stream, allocates its workspace from torch's caching
// allocator and never synchronizes the host.  Fake (shape) implementations are
// registered from Python (vllm-rlt_amd/ops.py).

#include <ATen/ATen.h>
#include <ATen/hip/impl/HIPGuardImplMasqueradingAsCUDA.h>
#include <ATen/hip/impl/HIPStreamMasqueradingAsCUDA.h>
#include <torch/library.h>

#include <optional>
#include <tuple>

#include "rlt_mi355x.h"

namespace {

using at::Tensor;
using OptTensor = std::optional<Tensor>;

hipStream_t stream_of(const Tensor& t) {
  return c10::hip::getCurrentHIPStreamMasqueradingAsCUDA(t.device().index()).stream();
}

void check_status(int status, const char* what) {
  static const char* kNames[] = {"ok", "invalid argument", "unsupported configuration",
                                 "workspace too small", "kernel launch failed"};
  TORCH_CHECK(status == 0, what, ": ",
              (status > 0 && status < 5) ? kNames[status] : "unknown status");
}

int32_t dtype_code(at::ScalarType t) {
  switch (t) {
    case at::kFloat: return 0;
    case at::kHalf: return 1;
    case at::kBFloat16: return 2;
    case at::kFloat8_e4m3fn: return 3;
    default: TORCH_CHECK_VALUE(false, "unsupported dtype ", t);
  }
  return -1;
}

Tensor workspace(size_t bytes, const Tensor& like) {
  return at::empty({(int64_t)std::max<size_t>(bytes, 1)},
                   like.options().dtype(at::kByte));
}

void* ptr(const Tensor& t) { return t.data_ptr(); }
void* ptr(const OptTensor& t) { return t.has_value() ? t->data_ptr() : nullptr; }

// The operators copy nothing behind the caller's back: a tensor of another dtype or
// layout than the kernel reads raises ValueError.  The Python wrappers convert where
// the reference's own functions convert (``logits.float()``, ``drafts.long()``).
const Tensor& need(const Tensor& t, at::ScalarType dt, const char* name) {
  TORCH_CHECK_VALUE(t.scalar_type() == dt, name, " must be ", dt, ", got ", t.scalar_type());
  TORCH_CHECK_VALUE(t.is_contiguous(), name, " must be contiguous");
  return t;
}

OptTensor need(const OptTensor& t, at::ScalarType dt, const char* name) {
  if (t.has_value()) need(*t, dt, name);
  return t;
}

bool logit_dtype(at::ScalarType t) {
  return t == at::kFloat || t == at::kBFloat16 || t == at::kHalf;
}

// Rows with unit column stride (row stride free) in a supported logits dtype.
const Tensor& logit_rows(const Tensor& t, const char* name) {
  TORCH_CHECK_VALUE(logit_dtype(t.scalar_type()), name, " must be float32, bfloat16 or float16");
  TORCH_CHECK_VALUE(t.stride(-1) == 1, name, " must have a unit column stride");
  return t;
}

// Every tensor argument must live on the device of the first one: a host tensor's
// pointer handed to a kernel would fault the GPU instead of raising.
void device_check(const c10::Device&) {}
template <class... Rest>
void device_check(const c10::Device& dev, const Tensor& t, const Rest&... rest);
template <class... Rest>
void device_check(const c10::Device& dev, const OptTensor& t, const Rest&... rest) {
  if (t.has_value()) device_check(dev, *t);
  device_check(dev, rest...);
}
template <class... Rest>
void device_check(const c10::Device& dev, const Tensor& t, const Rest&... rest) {
  TORCH_CHECK_VALUE(t.device() == dev,
                    "the MI355X kernels require every tensor on one ROCm device: got ",
                    t.device(), " next to ", dev);
  device_check(dev, rest...);
}
template <class... Rest>
void same_device(const Tensor& first, const Rest&... rest) {
  TORCH_CHECK_VALUE(first.is_cuda(), "the MI355X kernels require ROCm device tensors");
  device_check(first.device(), first, rest...);
}

// ---------------------------------------------------------------- attention

// reference: vllm_rlt/kernels/paged_attention.py:13-90 (per-row, windowed),
// vllm_rlt/kernels/triton_attention.py:386-404 (packed window).
Tensor paged_attention(const Tensor& q, const Tensor& key_cache, const Tensor& value_cache,
                       const Tensor& block_tables, const Tensor& context_lengths,
                       const OptTensor& key_scale, const OptTensor& value_scale,
                       const OptTensor& cu_seqlens_q, int64_t max_seqlen_q, int64_t window,
                       const OptTensor& row_lengths, bool compensate) {
  TORCH_CHECK_VALUE(window >= 0, "window must be a nonnegative integer");
  TORCH_CHECK_VALUE(q.dim() == 3 && key_cache.dim() == 4 && value_cache.dim() == 4,
                    "q must be [rows, heads, dim] and caches [block, token, kv_head, dim]");
  same_device(q, key_cache, value_cache, block_tables, context_lengths, key_scale, value_scale,
              cu_seqlens_q, row_lengths);
  const int64_t head_dim = q.size(2);
  TORCH_CHECK_VALUE(head_dim <= 256, "the MI355X attention backend supports head_dim <= 256");
  TORCH_CHECK_VALUE(key_cache.sizes() == value_cache.sizes() &&
                        key_cache.scalar_type() == value_cache.scalar_type(),
                    "key and value caches must share shape and dtype");
  const int64_t num_blocks = key_cache.size(0), block_size = key_cache.size(1);
  const int64_t kv_heads = key_cache.size(2);
  TORCH_CHECK_VALUE(!compensate || block_size % 16 == 0,
                    "compensated attention needs a block size that is a multiple of 16");
  TORCH_CHECK_VALUE(key_cache.size(3) == head_dim && q.size(1) % kv_heads == 0,
                    "q heads must be a positive multiple of KV heads with equal head_dim");
  TORCH_CHECK_VALUE(key_cache.stride(3) == 1 && value_cache.stride(3) == 1,
                    "paged attention requires a contiguous head dimension");
  Tensor output = at::empty_like(q);
  const int64_t rows = q.size(0);
  if (rows == 0 || block_tables.size(0) == 0) return output;
  TORCH_CHECK_VALUE(q.stride(2) == 1, "paged attention requires a contiguous head dimension");
  const Tensor& qq = q;
  int32_t mode = 0;
  int64_t s_strides[3] = {0, 0, 0};
  TORCH_CHECK_VALUE(key_scale.has_value() == value_scale.has_value(),
                    "key_scale and value_scale must be given together");
  if (key_scale.has_value()) {
    TORCH_CHECK_VALUE(key_scale->scalar_type() == at::kFloat &&
                          value_scale->scalar_type() == at::kFloat,
                      "FP8 scales must be float32");
    if (key_scale->dim() == 0 && value_scale->dim() == 0) {
      mode = 1;
    } else {
      TORCH_CHECK_VALUE(key_scale->dim() == 3 && key_scale->strides() == value_scale->strides(),
                        "per-vector FP8 scales must be [block, token, kv_head] views sharing "
                        "strides");
      mode = 2;
      for (int i = 0; i < 3; ++i) s_strides[i] = key_scale->stride(i);
    }
  }
  TORCH_CHECK_VALUE(!(key_cache.scalar_type() == at::kFloat8_e4m3fn && mode == 0),
                    "an FP8 KV pool needs key_scale / value_scale");
  TORCH_CHECK_VALUE(block_tables.dim() == 2 && block_tables.scalar_type() == at::kInt &&
                        block_tables.stride(1) == 1,
                    "block_tables must be int32 [sequences, width] with unit column stride");
  const Tensor& tables = block_tables;
  const Tensor& lengths = need(context_lengths, at::kInt, "context_lengths");
  const int64_t num_seqs = tables.size(0);
  OptTensor cu;
  int64_t max_q = 1;
  if (!cu_seqlens_q.has_value()) {
    TORCH_CHECK_VALUE(num_seqs == rows && lengths.size(0) == rows,
                      "per-row attention needs one block table and length per q row");
  } else {
    cu = need(*cu_seqlens_q, at::kInt, "cu_seqlens_q");
    TORCH_CHECK_VALUE(cu->size(0) == num_seqs + 1 && lengths.size(0) == num_seqs,
                      "cu_seqlens_q must be [sequences + 1] and lengths [sequences]");
    max_q = max_seqlen_q;
  }
  OptTensor rl;
  if (row_lengths.has_value()) {
    TORCH_CHECK_VALUE(cu_seqlens_q.has_value(), "row_lengths needs the packed form (cu_seqlens_q)");
    TORCH_CHECK_VALUE(row_lengths->dim() == 1 && row_lengths->size(0) == rows,
                      "row_lengths must be [q rows]");
    rl = need(*row_lengths, at::kInt, "row_lengths");
  }
  const c10::hip::HIPGuardMasqueradingAsCUDA guard(q.device());
  const int64_t heads = q.size(1), width = tables.size(1);
  const Tensor ws = workspace(
      rlt_paged_attention_workspace_size((int32_t)rows, (int32_t)heads, (int32_t)head_dim,
                                         (int32_t)width, (int32_t)block_size),
      q);
  const int status = rlt_paged_attention_rows(
      ptr(qq), qq.stride(0), qq.stride(1), ptr(key_cache), ptr(value_cache), key_cache.stride(0),
      key_cache.stride(1), key_cache.stride(2), value_cache.stride(0), value_cache.stride(1),
      value_cache.stride(2), (int32_t)num_blocks, (const int32_t*)ptr(tables), tables.stride(0),
      (int32_t)width, (const int32_t*)ptr(lengths), (const int32_t*)ptr(rl),
      (const int32_t*)ptr(cu), (int32_t)num_seqs, (int32_t)max_q, (int32_t)rows,
      (const float*)ptr(key_scale), (const float*)ptr(value_scale), mode, s_strides[0],
      s_strides[1], s_strides[2], (int32_t)heads, (int32_t)kv_heads, (int32_t)head_dim,
      (int32_t)block_size, dtype_code(q.scalar_type()), dtype_code(key_cache.scalar_type()),
      (int32_t)window, compensate ? RLT_ATTN_COMPENSATE : 0, ptr(output), output.stride(0),
      output.stride(1), ptr(ws), ws.numel(), stream_of(q));
  check_status(status, "rlt_paged_attention");
  return output;
}

// ---------------------------------------------------------------- KV writes

void check_view(const Tensor& cache, const char* name) {
  TORCH_CHECK_VALUE(cache.dim() == 4 && cache.stride(-1) == 1, name,
                    " must be a [block, token, kv_head, dim] view with unit dim stride");
}

const Tensor& rows3(const Tensor& x, const char* name) {
  TORCH_CHECK_VALUE(x.dim() == 3 && x.stride(-1) == 1, name,
                    " must be [rows, kv_heads, head_dim] with unit dim stride");
  return x;
}

const Tensor& index_of(const Tensor& t, int64_t rows, const char* name) {
  TORCH_CHECK_VALUE(t.dim() == 1 && t.size(0) == rows, name, " must have shape [", rows, "]");
  return need(t, at::kLong, name);
}

// reference: vllm_rlt/kernels/routing.py:210-223, vllm_rlt/kernels/graph_kv.py:52-67.
void store_kv(const Tensor& key_cache, const Tensor& value_cache, const Tensor& k_in, const Tensor& v_in,
              const Tensor& blocks, const Tensor& offsets, const OptTensor& mask,
              const OptTensor& active) {
  check_view(key_cache, "key_cache");
  check_view(value_cache, "value_cache");
  same_device(key_cache, value_cache, k_in, v_in, blocks, offsets, mask, active);
  TORCH_CHECK_VALUE(key_cache.strides() == value_cache.strides() &&
                        key_cache.sizes() == value_cache.sizes(),
                    "key and value pools must share a layout");
  const Tensor& k = rows3(k_in, "k");
  const Tensor& v = rows3(v_in, "v");
  const int64_t rows = k.size(0);
  TORCH_CHECK_VALUE(v.sizes() == k.sizes() && k.size(1) == key_cache.size(2) &&
                        k.size(2) == key_cache.size(3),
                    "k, v must be [rows, kv_heads, head_dim] of the pool");
  TORCH_CHECK_VALUE(k.scalar_type() == key_cache.scalar_type() &&
                        v.scalar_type() == key_cache.scalar_type(),
                    "rows must have the pool's dtype");
  if (rows == 0) return;
  const Tensor& b = index_of(blocks, rows, "blocks");
  const Tensor& o = index_of(offsets, rows, "offsets");
  OptTensor m, a;
  if (mask.has_value()) {
    TORCH_CHECK_VALUE(mask->dim() == 1 && mask->size(0) == rows, "mask must have shape [", rows,
                      "]");
    const auto mt = mask->scalar_type();
    TORCH_CHECK_VALUE((mt == at::kBool || mt == at::kByte) && mask->is_contiguous(),
                      "mask must be a contiguous bool or uint8 tensor");
    m = mask;
  }
  if (active.has_value()) {
    TORCH_CHECK_VALUE(active->numel() == 1 && active->scalar_type() == at::kInt,
                      "active must be one int32 row count");
    a = active;
  }
  const c10::hip::HIPGuardMasqueradingAsCUDA guard(k.device());
  const int status = rlt_kv_store(
      ptr(k), ptr(v), k.stride(0), k.stride(1), v.stride(0), v.stride(1), ptr(key_cache),
      ptr(value_cache), key_cache.stride(0), key_cache.stride(1), key_cache.stride(2),
      key_cache.size(0), key_cache.size(1), (const int64_t*)ptr(b), (const int64_t*)ptr(o),
      (const uint8_t*)ptr(m), (const int32_t*)ptr(a), rows, (int32_t)k.size(1),
      (int32_t)k.size(2), dtype_code(k.scalar_type()), stream_of(k));
  check_status(status, "rlt_kv_store");
}

// ---------------------------------------------------------------- sampling

void check_vec(const Tensor& t, int64_t n, const char* name) {
  TORCH_CHECK_VALUE(t.dim() == 1 && t.size(0) == n, name, " must have shape [", n, "], got ",
                    t.sizes());
}

// reference: vllm_rlt/worker/speculative_sampling.py:8-56.
Tensor spec_probs(const Tensor& logits, const Tensor& temperature, const Tensor& top_k,
                  const Tensor& top_p, int64_t max_top_k, bool apply_top_p) {
  TORCH_CHECK_VALUE(logits.dim() == 2, "logits must be a 2-D [n, V] tensor");
  const int64_t n = logits.size(0), vocab = logits.size(1);
  check_vec(temperature, n, "temperature");
  check_vec(top_k, n, "top_k");
  check_vec(top_p, n, "top_p");
  TORCH_CHECK_VALUE(max_top_k >= 0, "max_top_k must be nonnegative");
  Tensor out = at::empty({n, vocab}, logits.options().dtype(at::kFloat));
  if (n == 0 || vocab == 0) return out;
  same_device(logits, temperature, top_k, top_p);
  const Tensor& x = logit_rows(logits, "logits");
  const Tensor& t = need(temperature, at::kFloat, "temperature");
  const Tensor& k = need(top_k, at::kLong, "top_k");
  const Tensor& p = need(top_p, at::kFloat, "top_p");
  const c10::hip::HIPGuardMasqueradingAsCUDA guard(x.device());
  // row-split form (several workgroups per row) when it applies to this vocabulary
  const size_t nbytes = rlt_probabilities_workspace_size(n, 0, vocab);
  const Tensor ws = workspace(nbytes, x);
  const int status = rlt_batched_probabilities(
      ptr(x), dtype_code(x.scalar_type()), x.stride(0), n, vocab, (const float*)ptr(t),
      (const int64_t*)ptr(k), (const float*)ptr(p), max_top_k, apply_top_p ? 1 : 0,
      (float*)ptr(out), out.stride(0), nbytes ? ptr(ws) : nullptr, nbytes, stream_of(x));
  check_status(status, "rlt_batched_probabilities");
  return out;
}

// reference: vllm_rlt/worker/speculative_sampling.py:59-85.
std::tuple<Tensor, Tensor> categorical(const Tensor& weights, const Tensor& u) {
  TORCH_CHECK_VALUE(weights.dim() == 2 && weights.size(1) >= 1,
                    "weights must be a 2-D [m, V] tensor with V >= 1");
  const int64_t m = weights.size(0), vocab = weights.size(1);
  check_vec(u, m, "u");
  Tensor index = at::empty({m}, weights.options().dtype(at::kLong));
  Tensor valid = at::empty({m}, weights.options().dtype(at::kBool));
  if (m == 0) return {index, valid};
  same_device(weights, u);
  const Tensor& w = need(weights, at::kFloat, "weights");
  const Tensor& uu = need(u, at::kFloat, "u");
  const c10::hip::HIPGuardMasqueradingAsCUDA guard(w.device());
  const Tensor ws = workspace(rlt_categorical_workspace_size(m, vocab), w);
  const int status = rlt_categorical((const float*)ptr(w), (const float*)ptr(uu), m, vocab,
                                     (int64_t*)ptr(index), (uint8_t*)ptr(valid), ptr(ws),
                                     ws.numel(), stream_of(w));
  check_status(status, "rlt_categorical");
  return {index, valid};
}

// reference: vllm_rlt/worker/speculative_sampling.py:104-181.
std::tuple<Tensor, Tensor, Tensor, Tensor> spec_accept(const Tensor& draft_tokens,
                                                       const Tensor& drafts, const Tensor& q,
                                                       const Tensor& p, const Tensor& u_accept,
                                                       const Tensor& u_final) {
  TORCH_CHECK_VALUE(draft_tokens.dim() == 2, "draft_tokens must be [n, W1]");
  const int64_t n = draft_tokens.size(0), w1 = draft_tokens.size(1);
  const int64_t vocab = p.size(-1);
  TORCH_CHECK_VALUE(drafts.sizes() == at::IntArrayRef{n} && u_final.sizes() == at::IntArrayRef{n} &&
                        u_accept.sizes() == at::IntArrayRef({n, w1}),
                    "drafts, u_accept and u_final must match draft_tokens [n, W1]");
  TORCH_CHECK_VALUE(q.sizes() == at::IntArrayRef({n, w1, vocab}) &&
                        p.sizes() == at::IntArrayRef({n, w1 + 1, vocab}),
                    "q must be [n, W1, V] and p must be [n, W1 + 1, V]");
  Tensor tokens = at::empty({n, w1 + 1}, p.options().dtype(at::kLong));
  Tensor accepted = at::empty({n}, p.options().dtype(at::kLong));
  Tensor final_token = at::empty({n}, p.options().dtype(at::kLong));
  Tensor error = at::empty({n}, p.options().dtype(at::kBool));
  if (n == 0) return {tokens, accepted, final_token, error};
  TORCH_CHECK_VALUE(w1 <= 32, "at most 32 draft tokens per request are supported");
  same_device(p, draft_tokens, drafts, q, u_accept, u_final);
  const Tensor& dt = need(draft_tokens, at::kLong, "draft_tokens");
  const Tensor& dr = need(drafts, at::kLong, "drafts");
  const Tensor& qq = need(q, at::kFloat, "q");
  const Tensor& pp = need(p, at::kFloat, "p");
  const Tensor& ua = need(u_accept, at::kFloat, "u_accept");
  const Tensor& uf = need(u_final, at::kFloat, "u_final");
  const c10::hip::HIPGuardMasqueradingAsCUDA guard(p.device());
  const Tensor ws = workspace(rlt_speculative_accept_workspace_size(n, (int32_t)w1, vocab), p);
  const int status = rlt_speculative_accept(
      (const int64_t*)ptr(dt), (const int64_t*)ptr(dr), (const float*)ptr(qq),
      (const float*)ptr(pp), (const float*)ptr(ua), (const float*)ptr(uf), n, (int32_t)w1, vocab,
      (int64_t*)ptr(tokens), (int64_t*)ptr(accepted), (int64_t*)ptr(final_token),
      (uint8_t*)ptr(error), ptr(ws), ws.numel(), stream_of(p));
  check_status(status, "rlt_speculative_accept");
  return {tokens, accepted, final_token, error};
}

// reference: vllm_rlt/worker/async_speculative.py:706-720.
std::tuple<Tensor, Tensor, Tensor> greedy_accept(const Tensor& draft_tokens, const Tensor& drafts,
                                                 const Tensor& target_logits) {
  TORCH_CHECK_VALUE(draft_tokens.dim() == 2, "draft_tokens must be [n, W1]");
  const int64_t n = draft_tokens.size(0), w1 = draft_tokens.size(1);
  TORCH_CHECK_VALUE(drafts.sizes() == at::IntArrayRef{n}, "drafts must have shape [n]");
  TORCH_CHECK_VALUE(target_logits.dim() == 3 && target_logits.size(0) == n &&
                        target_logits.size(1) == w1 + 1,
                    "target_logits must be [n, W1 + 1, V]");
  const int64_t vocab = target_logits.size(2);
  Tensor targets = at::empty({n, w1 + 1}, target_logits.options().dtype(at::kLong));
  Tensor accepted = at::empty({n}, target_logits.options().dtype(at::kLong));
  Tensor next_token = at::empty({n}, target_logits.options().dtype(at::kLong));
  if (n == 0) return {targets, accepted, next_token};
  TORCH_CHECK_VALUE(vocab >= 1, "target_logits must have V >= 1");
  same_device(target_logits, draft_tokens, drafts);
  const Tensor& x = logit_rows(target_logits, "target_logits");
  TORCH_CHECK_VALUE(x.stride(0) == (w1 + 1) * x.stride(1),
                    "target_logits rows of a request must be evenly strided ([n * (W1 + 1), V] view)");
  const Tensor& dt = need(draft_tokens, at::kLong, "draft_tokens");
  const Tensor& dr = need(drafts, at::kLong, "drafts");
  const c10::hip::HIPGuardMasqueradingAsCUDA guard(x.device());
  const int status = rlt_greedy_accept(
      (const int64_t*)ptr(dt), (const int64_t*)ptr(dr), ptr(x), dtype_code(x.scalar_type()),
      x.stride(1), n, (int32_t)w1, vocab, (int64_t*)ptr(targets), (int64_t*)ptr(accepted),
      (int64_t*)ptr(next_token), stream_of(x));
  check_status(status, "rlt_greedy_accept");
  return {targets, accepted, next_token};
}

// reference: vllm_rlt/worker/async_speculative.py:678-692.
std::tuple<Tensor, Tensor> verify_distributions(const Tensor& logits, const Tensor& random_rows,
                                                const Tensor& temperature, const Tensor& top_k,
                                                const Tensor& top_p, int64_t max_top_k,
                                                bool apply_top_p) {
  TORCH_CHECK_VALUE(logits.dim() == 2, "logits must be a 2-D [m, V] tensor");
  TORCH_CHECK_VALUE(random_rows.dim() == 1, "random_rows must be 1-D");
  const int64_t m = logits.size(0), vocab = logits.size(1), r = random_rows.size(0);
  if (r) {
    check_vec(temperature, r, "temperature");
    check_vec(top_k, r, "top_k");
    check_vec(top_p, r, "top_p");
  }
  TORCH_CHECK_VALUE(max_top_k >= 0, "max_top_k must be nonnegative");
  Tensor target = at::empty({m}, logits.options().dtype(at::kLong));
  Tensor p_out = at::empty({r, vocab}, logits.options().dtype(at::kFloat));
  if (m == 0 && r == 0) return {target, p_out};
  TORCH_CHECK_VALUE(vocab >= 1, "logits must have V >= 1");
  same_device(logits, random_rows, temperature, top_k, top_p);
  const Tensor& x = logit_rows(logits, "logits");
  const Tensor& rows = need(random_rows, at::kLong, "random_rows");
  OptTensor t, k, p;
  if (r) {
    t = need(temperature, at::kFloat, "temperature");
    k = need(top_k, at::kLong, "top_k");
    p = need(top_p, at::kFloat, "top_p");
  }
  const c10::hip::HIPGuardMasqueradingAsCUDA guard(x.device());
  const size_t nbytes = r ? rlt_probabilities_workspace_size(r, m, vocab) : 0;
  const Tensor ws = workspace(nbytes, x);
  const int status = rlt_verify_distributions(
      ptr(x), dtype_code(x.scalar_type()), x.stride(0), m, vocab, (const int64_t*)ptr(rows), r,
      (const float*)ptr(t), (const int64_t*)ptr(k), (const float*)ptr(p), max_top_k,
      apply_top_p ? 1 : 0, (float*)ptr(p_out), r ? p_out.stride(0) : vocab,
      (int64_t*)ptr(target), nbytes ? ptr(ws) : nullptr, nbytes, stream_of(x));
  check_status(status, "rlt_verify_distributions");
  return {target, p_out};
}

// reference: vllm_rlt/worker/async_speculative.py:678-692 then :727-734.
std::tuple<Tensor, Tensor, Tensor, Tensor, Tensor, Tensor> verify_accept(
    const Tensor& target_logits, const Tensor& temperature, const Tensor& top_k,
    const Tensor& top_p, const Tensor& draft_tokens, const Tensor& drafts, const Tensor& q,
    const Tensor& u_accept, const Tensor& u_final, int64_t max_top_k, bool apply_top_p) {
  TORCH_CHECK_VALUE(draft_tokens.dim() == 2, "draft_tokens must be [n, W1]");
  const int64_t n = draft_tokens.size(0), w1 = draft_tokens.size(1);
  TORCH_CHECK_VALUE(target_logits.dim() == 3 && target_logits.size(0) == n &&
                        target_logits.size(1) == w1 + 1,
                    "target_logits must be [n, W1 + 1, V]");
  const int64_t vocab = target_logits.size(2), rows = n * (w1 + 1);
  check_vec(temperature, rows, "temperature");
  check_vec(top_k, rows, "top_k");
  check_vec(top_p, rows, "top_p");
  TORCH_CHECK_VALUE(drafts.sizes() == at::IntArrayRef{n} && u_final.sizes() == at::IntArrayRef{n} &&
                        u_accept.sizes() == at::IntArrayRef({n, w1}),
                    "drafts, u_accept and u_final must match draft_tokens [n, W1]");
  TORCH_CHECK_VALUE(q.sizes() == at::IntArrayRef({n, w1, vocab}), "q must be [n, W1, V]");
  TORCH_CHECK_VALUE(max_top_k >= 0, "max_top_k must be nonnegative");
  TORCH_CHECK_VALUE(w1 <= 32, "at most 32 draft tokens per request are supported");
  const auto i64 = target_logits.options().dtype(at::kLong);
  Tensor target = at::empty({rows}, i64);
  Tensor p = at::empty({n, w1 + 1, vocab}, target_logits.options().dtype(at::kFloat));
  Tensor tokens = at::empty({n, w1 + 1}, i64);
  Tensor accepted = at::empty({n}, i64), final_token = at::empty({n}, i64);
  Tensor error = at::empty({n}, target_logits.options().dtype(at::kBool));
  if (n == 0) return {target, p, tokens, accepted, final_token, error};
  same_device(target_logits, temperature, top_k, top_p, draft_tokens, drafts, q, u_accept,
              u_final);
  logit_rows(target_logits, "target_logits");
  TORCH_CHECK_VALUE(target_logits.stride(0) == (w1 + 1) * target_logits.stride(1),
                    "target_logits rows of a request must be evenly strided ([n * (W1 + 1), V] view)");
  const Tensor x = target_logits.view({rows, vocab});
  const Tensor& t = need(temperature, at::kFloat, "temperature");
  const Tensor& k = need(top_k, at::kLong, "top_k");
  const Tensor& pp = need(top_p, at::kFloat, "top_p");
  const Tensor& dt = need(draft_tokens, at::kLong, "draft_tokens");
  const Tensor& dr = need(drafts, at::kLong, "drafts");
  const Tensor& qq = need(q, at::kFloat, "q");
  const Tensor& ua = need(u_accept, at::kFloat, "u_accept");
  const Tensor& uf = need(u_final, at::kFloat, "u_final");
  const c10::hip::HIPGuardMasqueradingAsCUDA guard(x.device());
  const Tensor ws = workspace(rlt_verify_accept_workspace_size(n, (int32_t)w1, vocab), x);
  const int status = rlt_verify_accept(
      ptr(x), dtype_code(x.scalar_type()), x.stride(0), (const float*)ptr(t),
      (const int64_t*)ptr(k), (const float*)ptr(pp), max_top_k, apply_top_p ? 1 : 0,
      (const int64_t*)ptr(dt), (const int64_t*)ptr(dr), (const float*)ptr(qq),
      (const float*)ptr(ua), (const float*)ptr(uf), n, (int32_t)w1, vocab, (int64_t*)ptr(target),
      (float*)ptr(p), (int64_t*)ptr(tokens), (int64_t*)ptr(accepted), (int64_t*)ptr(final_token),
      (uint8_t*)ptr(error), ptr(ws), ws.numel(), stream_of(x));
  check_status(status, "rlt_verify_accept");
  return {target, p, tokens, accepted, final_token, error};
}

// ---------------------------------------------------------------- window store + attention

// reference: vllm_rlt/kernels/graph_kv.py:52-67 (the window rows' KV write) followed by
// vllm_rlt/kernels/triton_attention.py:386-404 (packed window attention).  Row r of
// k_new / v_new goes to packed q row r's position (context_lengths[s] - q_len + i).
// bf16 / fp16 windows below the prefill tiling run as one launch pair
// (rlt_paged_attention_store); other shapes store with the scatter kernel and attend
// separately, with the same result.
Tensor paged_attention_store(const Tensor& q, const Tensor& k_new_in, const Tensor& v_new_in,
                             const Tensor& key_cache, const Tensor& value_cache,
                             const Tensor& block_tables, const Tensor& context_lengths,
                             const Tensor& cu_seqlens_q, int64_t max_seqlen_q,
                             const OptTensor& key_scale, const OptTensor& value_scale,
                             const OptTensor& row_lengths, bool compensate) {
  TORCH_CHECK_VALUE(q.dim() == 3, "q must be [rows, heads, dim]");
  check_view(key_cache, "key_cache");
  check_view(value_cache, "value_cache");
  TORCH_CHECK_VALUE(key_cache.strides() == value_cache.strides() &&
                        key_cache.sizes() == value_cache.sizes(),
                    "key and value pools must share a layout with a unit dim stride");
  same_device(q, k_new_in, v_new_in, key_cache, value_cache, block_tables, context_lengths,
              cu_seqlens_q, key_scale, value_scale, row_lengths);
  const int64_t rows = q.size(0), head_dim = q.size(2), kv_heads = key_cache.size(2);
  const Tensor& k_new = rows3(k_new_in, "k_new");
  const Tensor& v_new = rows3(v_new_in, "v_new");
  TORCH_CHECK_VALUE(k_new.size(0) == rows && k_new.size(1) == kv_heads && k_new.size(2) == head_dim &&
                        v_new.sizes() == k_new.sizes(),
                    "k_new, v_new must be [q rows, kv_heads, head_dim]");
  const bool fp8 = key_cache.scalar_type() == at::kFloat8_e4m3fn;
  const bool half = q.scalar_type() == at::kBFloat16 || q.scalar_type() == at::kHalf;
  // everything is checked before anything is stored: the attention's own checks must
  // not fail after the store
  int32_t mode = 0;
  int64_t s_strides[3] = {0, 0, 0};
  TORCH_CHECK_VALUE(key_scale.has_value() == value_scale.has_value(),
                    "key_scale and value_scale must be given together");
  if (fp8) {
    TORCH_CHECK_VALUE(half && k_new.scalar_type() == q.scalar_type() &&
                          v_new.scalar_type() == q.scalar_type(),
                      "an FP8 window store takes bfloat16 / float16 q, k_new and v_new");
    TORCH_CHECK_VALUE(key_scale.has_value(), "an FP8 KV pool needs key_scale / value_scale");
    TORCH_CHECK_VALUE(key_scale->scalar_type() == at::kFloat &&
                          value_scale->scalar_type() == at::kFloat,
                      "FP8 scales must be float32");
    if (key_scale->dim() == 0 && value_scale->dim() == 0) {
      mode = 1;
    } else {
      TORCH_CHECK_VALUE(key_scale->dim() == 3 && key_scale->strides() == value_scale->strides() &&
                            key_scale->size(0) == key_cache.size(0) &&
                            key_scale->size(1) == key_cache.size(1) &&
                            key_scale->size(2) == kv_heads,
                        "per-vector FP8 scales must be [block, token, kv_head] views of the pool "
                        "sharing strides");
      mode = 2;
      for (int i = 0; i < 3; ++i) s_strides[i] = key_scale->stride(i);
    }
  } else {
    TORCH_CHECK_VALUE(k_new.scalar_type() == key_cache.scalar_type() &&
                          v_new.scalar_type() == key_cache.scalar_type(),
                      "k_new, v_new must have the pool's dtype");
    TORCH_CHECK_VALUE(!key_scale.has_value(), "a 16-bit KV pool takes no scales");
  }
  TORCH_CHECK_VALUE(head_dim <= 256 && key_cache.size(3) == head_dim && q.size(1) % kv_heads == 0,
                    "q heads must be a positive multiple of KV heads with equal head_dim <= 256");
  TORCH_CHECK_VALUE(block_tables.dim() == 2 && context_lengths.dim() == 1 &&
                        cu_seqlens_q.dim() == 1 &&
                        cu_seqlens_q.size(0) == block_tables.size(0) + 1 &&
                        context_lengths.size(0) == block_tables.size(0),
                    "cu_seqlens_q must be [sequences + 1] and lengths [sequences]");
  TORCH_CHECK_VALUE(q.stride(2) == 1, "paged attention requires a contiguous head dimension");
  TORCH_CHECK_VALUE(block_tables.scalar_type() == at::kInt && block_tables.stride(1) == 1,
                    "block_tables must be int32 [sequences, width] with unit column stride");
  need(context_lengths, at::kInt, "context_lengths");
  need(cu_seqlens_q, at::kInt, "cu_seqlens_q");
  if (row_lengths.has_value()) {
    TORCH_CHECK_VALUE(row_lengths->dim() == 1 && row_lengths->size(0) == rows,
                      "row_lengths must be [q rows]");
    need(*row_lengths, at::kInt, "row_lengths");
  }
  TORCH_CHECK_VALUE(k_new.strides() == v_new.strides(), "k_new and v_new must share strides");
  const int32_t qd = dtype_code(q.scalar_type()), kvd = dtype_code(key_cache.scalar_type());
  // the C ABI's store-and-attend form: one launch on the verify kernels, or the window
  // store then the prefill tiling for windows that take it
  const bool abi_store = half && (fp8 || q.scalar_type() == key_cache.scalar_type()) &&
                          rlt_paged_attention_uses_mfma(qd, kvd, (int32_t)head_dim);
  TORCH_CHECK_VALUE(abi_store || !fp8,
                    "an FP8 window store needs a head_dim the MFMA kernels serve (64, 96, 128, "
                    "256): use store_fp8 and prefill");
  if (rows > 0 && abi_store) {
    const int64_t num_seqs = block_tables.size(0), width = block_tables.size(1), heads = q.size(1);
    const c10::hip::HIPGuardMasqueradingAsCUDA guard(q.device());
    Tensor output = at::empty_like(q);
    const Tensor ws = workspace(
        rlt_paged_attention_workspace_size((int32_t)rows, (int32_t)heads, (int32_t)head_dim,
                                           (int32_t)width, (int32_t)key_cache.size(1)),
        q);
    const int status = rlt_paged_attention_store_scaled(
        ptr(q), q.stride(0), q.stride(1), ptr(key_cache), ptr(value_cache), key_cache.stride(0),
        key_cache.stride(1), key_cache.stride(2), value_cache.stride(0), value_cache.stride(1),
        value_cache.stride(2), (int32_t)key_cache.size(0), (const int32_t*)ptr(block_tables),
        block_tables.stride(0), (int32_t)width, (const int32_t*)ptr(context_lengths),
        (const int32_t*)ptr(row_lengths), (const int32_t*)ptr(cu_seqlens_q), (int32_t)num_seqs,
        (int32_t)max_seqlen_q, (int32_t)rows, (float*)ptr(key_scale), (float*)ptr(value_scale),
        mode, s_strides[0], s_strides[1], s_strides[2], (int32_t)heads, (int32_t)kv_heads,
        (int32_t)head_dim, (int32_t)key_cache.size(1), qd, kvd,
        compensate ? RLT_ATTN_COMPENSATE : 0, ptr(k_new), ptr(v_new),
        k_new.stride(0), k_new.stride(1), ptr(output), output.stride(0), output.stride(1), ptr(ws),
        ws.numel(), stream_of(q));
    if (status != 2 || fp8) {  // 2: a 16-bit shape the one-launch form does not serve
      check_status(status, "rlt_paged_attention_store");
      return output;
    }
  }
  // separate store and attention (16-bit pools): positions -> (block, offset) through
  // the tables; a position whose block index falls outside the table gets block -1,
  // which the scatter skips (the one-launch form does not write such positions either)
  if (rows > 0) {
    const Tensor cu = cu_seqlens_q.to(at::kLong);
    const int64_t num_seqs = cu.size(0) - 1, width = block_tables.size(1);
    const Tensor q_len = cu.slice(0, 1) - cu.slice(0, 0, num_seqs);
    const Tensor seq = at::repeat_interleave(
        at::arange(num_seqs, cu.options()), q_len, /*dim=*/0, /*output_size=*/rows);
    const Tensor pos =
        row_lengths.has_value()
            ? row_lengths->to(at::kLong) - 1
            : context_lengths.to(at::kLong).index({seq}) - q_len.index({seq}) +
                  at::arange(rows, cu.options()) - cu.index({seq});
    const int64_t bs = key_cache.size(1);
    const Tensor idx = at::floor_divide(pos, bs);
    const Tensor inside = (pos >= 0) & (idx < width);
    const Tensor blocks =
        width == 0 ? at::full({rows}, -1, cu.options())
                   : at::where(inside, block_tables.to(at::kLong).index({seq, idx.clamp(0, width - 1)}),
                               at::full({rows}, -1, cu.options()));
    store_kv(key_cache, value_cache, k_new, v_new, blocks, at::remainder(pos, bs), std::nullopt,
             std::nullopt);
  }
  return paged_attention(q, key_cache, value_cache, block_tables, context_lengths, std::nullopt,
                         std::nullopt, cu_seqlens_q, max_seqlen_q, 0, row_lengths, compensate);
}

}  // namespace

TORCH_LIBRARY(rlt_mi355x, m) {
  m.def("paged_attention(Tensor q, Tensor key_cache, Tensor value_cache, Tensor block_tables, "
        "Tensor context_lengths, Tensor? key_scale, Tensor? value_scale, Tensor? cu_seqlens_q, "
        "int max_seqlen_q, int window, Tensor? row_lengths=None, bool compensate=False) -> Tensor");
  m.def("store_kv(Tensor(a!) key_cache, Tensor(b!) value_cache, Tensor k, Tensor v, "
        "Tensor blocks, Tensor offsets, Tensor? mask, Tensor? active) -> ()");
  m.def("spec_probs(Tensor logits, Tensor temperature, Tensor top_k, Tensor top_p, "
        "int max_top_k, bool apply_top_p) -> Tensor");
  m.def("categorical(Tensor weights, Tensor u) -> (Tensor, Tensor)");
  m.def("spec_accept(Tensor draft_tokens, Tensor drafts, Tensor q, Tensor p, Tensor u_accept, "
        "Tensor u_final) -> (Tensor, Tensor, Tensor, Tensor)");
  m.def("greedy_accept(Tensor draft_tokens, Tensor drafts, Tensor target_logits) "
        "-> (Tensor, Tensor, Tensor)");
  m.def("verify_distributions(Tensor logits, Tensor random_rows, Tensor temperature, "
        "Tensor top_k, Tensor top_p, int max_top_k, bool apply_top_p) -> (Tensor, Tensor)");
  m.def("verify_accept(Tensor target_logits, Tensor temperature, Tensor top_k, Tensor top_p, "
        "Tensor draft_tokens, Tensor drafts, Tensor q, Tensor u_accept, Tensor u_final, "
        "int max_top_k, bool apply_top_p) -> (Tensor, Tensor, Tensor, Tensor, Tensor, Tensor)");
  m.def("paged_attention_store(Tensor q, Tensor k_new, Tensor v_new, Tensor(a!) key_cache, "
        "Tensor(b!) value_cache, Tensor block_tables, Tensor context_lengths, "
        "Tensor cu_seqlens_q, int max_seqlen_q, Tensor(c!)? key_scale=None, "
        "Tensor(d!)? value_scale=None, Tensor? row_lengths=None, bool compensate=False) -> Tensor");
}

TORCH_LIBRARY_IMPL(rlt_mi355x, CUDA, m) {
  m.impl("paged_attention", &paged_attention);
  m.impl("store_kv", &store_kv);
  m.impl("spec_probs", &spec_probs);
  m.impl("categorical", &categorical);
  m.impl("spec_accept", &spec_accept);
  m.impl("greedy_accept", &greedy_accept);
  m.impl("verify_distributions", &verify_distributions);
  m.impl("verify_accept", &verify_accept);
  m.impl("paged_attention_store", &paged_attention_store);
}
