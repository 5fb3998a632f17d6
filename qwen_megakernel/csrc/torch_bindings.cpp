// torch.ops.qwen_megakernel_C -- the reference's operator library, rebuilt on
// PyTorch-ROCm over the C ABI of libqwen_megakernel_amd.so.
//
// `decode` and `generate_nosync` keep the reference's schemas exactly
// (reference csrc/torch_bindings.cpp:129-155), so callers written against
// torch.ops.qwen_megakernel_C work unchanged.  Unlike the reference, every
// tensor argument is checked (device, dtype, contiguity, size) and the
// position is range-checked before anything is launched; failures raise
// through TORCH_CHECK instead of writing out of bounds.  Additive ops:
// `decode_logits` (also returns the fp32 copy of the bf16 logits),
// `device_error`, `reset`, `set_wait_limit`, `set_trace` (phase trace),
// `phase_bench` (per-phase weight-streaming microbenchmark), and the batched
// forward `forward_tokens` (prefill, batched decode) with
// `forward_workspace_bytes` and `selftest_mfma`, `generate_eos` (stop token on
// the device), `set_graph_launch`, and sampling: `sample` over logits rows and
// the sampled loop `generate_sample`.

#include <Python.h>
#include <ATen/hip/impl/HIPGuardImplMasqueradingAsCUDA.h>
#include <ATen/hip/impl/HIPStreamMasqueradingAsCUDA.h>
#include <torch/all.h>
#include <torch/library.h>

#include "../../include/qwen_megakernel.h"

namespace {

constexpr int64_t kHidden = 1024, kInter = 3072, kQ = 2048, kKV = 1024, kHeadDim = 128, kKVHeads = 8;
constexpr int64_t kVocab = 151936, kMaxLayers = 28;

void check_cuda(const torch::Tensor& t, const char* name) {
  TORCH_CHECK(t.is_cuda(), name, " must be a GPU tensor");
  TORCH_CHECK(t.is_contiguous(), name, " must be contiguous");
}

void check_bf16(const torch::Tensor& t, const char* name, int64_t numel) {
  check_cuda(t, name);
  TORCH_CHECK(t.scalar_type() == torch::kBFloat16, name, " must be bfloat16");
  if (numel >= 0) TORCH_CHECK(t.numel() == numel, name, " must have ", numel, " elements, got ", t.numel());
}

void check_scratch(const torch::Tensor& t, const char* name, int64_t min_bytes) {
  check_cuda(t, name);
  TORCH_CHECK(t.numel() * t.element_size() >= min_bytes, name, " is smaller than ", min_bytes, " bytes");
}

struct Checked {
  int num_layers;
  int max_seq_len;
  int model;       // QMK_MODEL_*, from the embedding's row length
  int64_t hidden;
  int64_t inter;
};

Checked check_common(const torch::Tensor& embed_weight, const torch::Tensor& layer_weights_packed,
                     const torch::Tensor& final_norm_weight, const torch::Tensor& lm_head_weight,
                     const torch::Tensor& cos_table, const torch::Tensor& sin_table, const torch::Tensor& k_cache,
                     const torch::Tensor& v_cache, const torch::Tensor& hidden_buffer,
                     const torch::Tensor& normalized, int64_t num_layers, int64_t max_seq_len, double attn_scale) {
  TORCH_CHECK(num_layers >= 1 && num_layers <= kMaxLayers, "num_layers must be in [1, 28], got ", num_layers);
  TORCH_CHECK(max_seq_len >= 1 && max_seq_len <= 65536, "max_seq_len must be in [1, 65536]");
  TORCH_CHECK(attn_scale > 0.0, "attn_scale must be positive");
  // The model is Qwen3-0.6B (hidden 1024, the reference's) or Qwen3-1.7B (hidden 2048), told apart by
  // the embedding's size; every other tensor is checked against that model's dimensions.
  check_bf16(embed_weight, "embed_weight", -1);
  const int64_t hidden = embed_weight.numel() / kVocab;
  TORCH_CHECK(embed_weight.numel() == kVocab * hidden && (hidden == 1024 || hidden == 2048),
              "embed_weight must be [151936, 1024] (Qwen3-0.6B) or [151936, 2048] (Qwen3-1.7B)");
  const int model = hidden == 1024 ? QMK_MODEL_QWEN3_0_6B : QMK_MODEL_QWEN3_1_7B;
  const int64_t inter = 3 * hidden;
  check_bf16(lm_head_weight, "lm_head_weight", kVocab * hidden);
  check_bf16(final_norm_weight, "final_norm_weight", hidden);
  check_cuda(layer_weights_packed, "layer_weights_packed");
  TORCH_CHECK(layer_weights_packed.scalar_type() == torch::kUInt8, "layer_weights_packed must be uint8");
  TORCH_CHECK(layer_weights_packed.numel() >= num_layers * 11 * 8,
              "layer_weights_packed must hold 11 pointers per layer");
  TORCH_CHECK(cos_table.dim() == 2 && cos_table.size(1) == kHeadDim && cos_table.size(0) >= max_seq_len,
              "cos_table must be [>= max_seq_len, 128]");
  TORCH_CHECK(sin_table.sizes() == cos_table.sizes(), "sin_table must match cos_table");
  check_bf16(cos_table, "cos_table", -1);
  check_bf16(sin_table, "sin_table", -1);
  const int64_t kv = num_layers * kKVHeads * max_seq_len * kHeadDim;
  check_bf16(k_cache, "k_cache", -1);
  check_bf16(v_cache, "v_cache", -1);
  TORCH_CHECK(k_cache.dim() == 4 && k_cache.size(1) == kKVHeads && k_cache.size(2) == max_seq_len &&
                  k_cache.size(3) == kHeadDim && k_cache.size(0) >= num_layers,
              "k_cache must be [>= num_layers, 8, max_seq_len, 128]");
  TORCH_CHECK(v_cache.sizes() == k_cache.sizes(), "v_cache must match k_cache");
  TORCH_CHECK(k_cache.numel() >= kv, "k_cache too small");
  check_bf16(hidden_buffer, "hidden_buffer", -1);
  TORCH_CHECK(hidden_buffer.numel() >= hidden, "hidden_buffer must hold ", hidden, " bf16");
  check_cuda(normalized, "normalized");
  TORCH_CHECK(normalized.scalar_type() == torch::kFloat32 && normalized.numel() >= hidden,
              "normalized must be float32 with >= ", hidden, " elements");
  const auto dev = embed_weight.device();
  for (const torch::Tensor* t : {&layer_weights_packed, &final_norm_weight, &lm_head_weight, &cos_table, &sin_table,
                                 &k_cache, &v_cache, &hidden_buffer, &normalized})
    TORCH_CHECK(t->device() == dev, "all tensors must be on the same device");
  return Checked{(int)num_layers, (int)max_seq_len, model, hidden, inter};
}

void check_unused_scratch(const Checked& c, const torch::Tensor& activations, const torch::Tensor& residual,
                          const torch::Tensor& q, const torch::Tensor& k, const torch::Tensor& v,
                          const torch::Tensor& attn_out, const torch::Tensor& mlp_intermediate,
                          const torch::Tensor& block_max_vals, const torch::Tensor& block_max_idxs) {
  // Not used by this kernel, but the reference's callers pass them; keep the
  // contract that they are GPU tensors of the reference's sizes (for the model).
  check_scratch(activations, "activations", c.hidden * 4);
  check_scratch(residual, "residual", c.hidden * 4);
  check_scratch(q, "q", kQ * 4);
  check_scratch(k, "k", kKV * 4);
  check_scratch(v, "v", kKV * 4);
  check_scratch(attn_out, "attn_out", kQ * 4);
  check_scratch(mlp_intermediate, "mlp_intermediate", c.inter * 4);
  check_scratch(block_max_vals, "block_max_vals", 4);
  check_scratch(block_max_idxs, "block_max_idxs", 4);
}

void raise_status(const char* what) {
  const int s = qmk_last_status();
  TORCH_CHECK(s == QMK_OK, what, " failed: ", qmk_status_string(s));
}

void decode(torch::Tensor output_token, int64_t input_token_id, torch::Tensor embed_weight,
            torch::Tensor layer_weights_packed, torch::Tensor final_norm_weight, torch::Tensor lm_head_weight,
            torch::Tensor cos_table, torch::Tensor sin_table, torch::Tensor k_cache, torch::Tensor v_cache,
            torch::Tensor hidden_buffer, torch::Tensor activations, torch::Tensor residual, torch::Tensor q,
            torch::Tensor k, torch::Tensor v, torch::Tensor attn_out, torch::Tensor mlp_intermediate,
            torch::Tensor normalized, torch::Tensor block_max_vals, torch::Tensor block_max_idxs,
            int64_t num_layers, int64_t position, int64_t max_seq_len, double attn_scale) {
  const Checked c = check_common(embed_weight, layer_weights_packed, final_norm_weight, lm_head_weight, cos_table,
                                 sin_table, k_cache, v_cache, hidden_buffer, normalized, num_layers, max_seq_len,
                                 attn_scale);
  check_unused_scratch(c, activations, residual, q, k, v, attn_out, mlp_intermediate, block_max_vals, block_max_idxs);
  check_cuda(output_token, "output_token");
  TORCH_CHECK(output_token.scalar_type() == torch::kInt32 && output_token.numel() >= 1, "output_token must be int32[1]");
  TORCH_CHECK(position >= 0 && position < max_seq_len, "position ", position, " outside [0, ", max_seq_len, ")");
  TORCH_CHECK(input_token_id >= 0 && input_token_id < kVocab, "input_token_id outside the vocabulary");
  const c10::hip::HIPGuardMasqueradingAsCUDA guard(embed_weight.device());
  if (c.model != QMK_MODEL_QWEN3_0_6B) {
    qmk_decode_model(c.model, (int)input_token_id, static_cast<int*>(output_token.data_ptr()), nullptr,
                     embed_weight.data_ptr(), reinterpret_cast<const LDGLayerWeights*>(layer_weights_packed.data_ptr()),
                     final_norm_weight.data_ptr(), lm_head_weight.data_ptr(), cos_table.data_ptr(), sin_table.data_ptr(),
                     k_cache.data_ptr(), v_cache.data_ptr(), hidden_buffer.data_ptr(), normalized.data_ptr(),
                     c.num_layers, (int)position, c.max_seq_len, (float)attn_scale,
                     c10::hip::getCurrentHIPStreamMasqueradingAsCUDA().stream());
    raise_status("decode");
    return;
  }
  launch_ldg_decode_direct(
      (int)input_token_id, static_cast<int*>(output_token.data_ptr()), embed_weight.data_ptr(),
      reinterpret_cast<const LDGLayerWeights*>(layer_weights_packed.data_ptr()), final_norm_weight.data_ptr(),
      lm_head_weight.data_ptr(), cos_table.data_ptr(), sin_table.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(),
      hidden_buffer.data_ptr(), activations.data_ptr(), residual.data_ptr(), q.data_ptr(), k.data_ptr(),
      v.data_ptr(), attn_out.data_ptr(), mlp_intermediate.data_ptr(), normalized.data_ptr(),
      block_max_vals.data_ptr(), block_max_idxs.data_ptr(), c.num_layers, (int)position, c.max_seq_len,
      (float)attn_scale, c10::hip::getCurrentHIPStreamMasqueradingAsCUDA().stream());
  raise_status("decode");
}

torch::Tensor generate_nosync(int64_t first_token_id, int64_t num_steps, torch::Tensor embed_weight,
                              torch::Tensor layer_weights_packed, torch::Tensor final_norm_weight,
                              torch::Tensor lm_head_weight, torch::Tensor cos_table, torch::Tensor sin_table,
                              torch::Tensor k_cache, torch::Tensor v_cache, torch::Tensor hidden_buffer,
                              torch::Tensor activations, torch::Tensor residual, torch::Tensor q, torch::Tensor k,
                              torch::Tensor v, torch::Tensor attn_out, torch::Tensor mlp_intermediate,
                              torch::Tensor normalized, torch::Tensor block_max_vals, torch::Tensor block_max_idxs,
                              int64_t num_layers, int64_t start_position, int64_t max_seq_len, double attn_scale) {
  const Checked c = check_common(embed_weight, layer_weights_packed, final_norm_weight, lm_head_weight, cos_table,
                                 sin_table, k_cache, v_cache, hidden_buffer, normalized, num_layers, max_seq_len,
                                 attn_scale);
  check_unused_scratch(c, activations, residual, q, k, v, attn_out, mlp_intermediate, block_max_vals, block_max_idxs);
  TORCH_CHECK(num_steps >= 0, "num_steps must be non-negative");
  TORCH_CHECK(start_position >= 0 && start_position + num_steps <= max_seq_len, "steps [", start_position, ", ",
              start_position + num_steps, ") do not fit in max_seq_len ", max_seq_len);
  TORCH_CHECK(first_token_id >= 0 && first_token_id < kVocab, "first_token_id outside the vocabulary");
  const c10::hip::HIPGuardMasqueradingAsCUDA guard(embed_weight.device());
  auto stream = c10::hip::getCurrentHIPStreamMasqueradingAsCUDA().stream();
  auto output_log = torch::empty({num_steps}, torch::dtype(torch::kInt32).device(embed_weight.device()));
  if (num_steps == 0) return output_log;
  if (c.model != QMK_MODEL_QWEN3_0_6B)
    qmk_generate_model(c.model, (int)first_token_id, (int)num_steps, embed_weight.data_ptr(),
                       reinterpret_cast<const LDGLayerWeights*>(layer_weights_packed.data_ptr()),
                       final_norm_weight.data_ptr(), lm_head_weight.data_ptr(), cos_table.data_ptr(),
                       sin_table.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), hidden_buffer.data_ptr(),
                       normalized.data_ptr(), static_cast<int*>(output_log.data_ptr()), c.num_layers,
                       (int)start_position, c.max_seq_len, (float)attn_scale, stream);
  else
    launch_ldg_generate_nosync(
        (int)first_token_id, (int)num_steps, embed_weight.data_ptr(),
        reinterpret_cast<const LDGLayerWeights*>(layer_weights_packed.data_ptr()), final_norm_weight.data_ptr(),
        lm_head_weight.data_ptr(), cos_table.data_ptr(), sin_table.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(),
        hidden_buffer.data_ptr(), activations.data_ptr(), residual.data_ptr(), q.data_ptr(), k.data_ptr(),
        v.data_ptr(), attn_out.data_ptr(), mlp_intermediate.data_ptr(), normalized.data_ptr(),
        block_max_vals.data_ptr(), block_max_idxs.data_ptr(), static_cast<int*>(output_log.data_ptr()), c.num_layers,
        (int)start_position, c.max_seq_len, (float)attn_scale, stream);
  raise_status("generate_nosync");
  // Single synchronisation at the end, as the reference (csrc/torch_bindings.cpp:125).
  const uint32_t err = qmk_device_error(stream);
  TORCH_CHECK(err == 0, "generate_nosync: device error bits 0x", std::hex, err,
              " (a bounded wait expired or a position left the cache); call reset()");
  return output_log;
}

// generate_nosync that stops at eos_token_id on the device (qmk_generate_eos):
// the returned log holds the generated tokens, then eos_token_id padding.
torch::Tensor generate_eos(int64_t first_token_id, int64_t num_steps, int64_t eos_token_id,
                           torch::Tensor embed_weight, torch::Tensor layer_weights_packed,
                           torch::Tensor final_norm_weight, torch::Tensor lm_head_weight, torch::Tensor cos_table,
                           torch::Tensor sin_table, torch::Tensor k_cache, torch::Tensor v_cache,
                           torch::Tensor hidden_buffer, torch::Tensor normalized, int64_t num_layers,
                           int64_t start_position, int64_t max_seq_len, double attn_scale) {
  const Checked c = check_common(embed_weight, layer_weights_packed, final_norm_weight, lm_head_weight, cos_table,
                                 sin_table, k_cache, v_cache, hidden_buffer, normalized, num_layers, max_seq_len,
                                 attn_scale);
  TORCH_CHECK(num_steps >= 0, "num_steps must be non-negative");
  TORCH_CHECK(start_position >= 0 && start_position + num_steps <= max_seq_len, "steps [", start_position, ", ",
              start_position + num_steps, ") do not fit in max_seq_len ", max_seq_len);
  TORCH_CHECK(first_token_id >= 0 && first_token_id < kVocab, "first_token_id outside the vocabulary");
  TORCH_CHECK(eos_token_id >= 0 && eos_token_id < kVocab, "eos_token_id outside the vocabulary");
  const c10::hip::HIPGuardMasqueradingAsCUDA guard(embed_weight.device());
  auto stream = c10::hip::getCurrentHIPStreamMasqueradingAsCUDA().stream();
  auto output_log = torch::empty({num_steps}, torch::dtype(torch::kInt32).device(embed_weight.device()));
  if (num_steps == 0) return output_log;
  qmk_generate_eos(c.model, (int)first_token_id, (int)num_steps, (int)eos_token_id, embed_weight.data_ptr(),
                   reinterpret_cast<const LDGLayerWeights*>(layer_weights_packed.data_ptr()),
                   final_norm_weight.data_ptr(), lm_head_weight.data_ptr(), cos_table.data_ptr(), sin_table.data_ptr(),
                   k_cache.data_ptr(), v_cache.data_ptr(), hidden_buffer.data_ptr(), normalized.data_ptr(),
                   static_cast<int*>(output_log.data_ptr()), c.num_layers, (int)start_position, c.max_seq_len,
                   (float)attn_scale, stream);
  raise_status("generate_eos");
  const uint32_t err = qmk_device_error(stream);
  TORCH_CHECK(err == 0, "generate_eos: device error bits 0x", std::hex, err, "; call reset()");
  return output_log;
}

// Sampled generate loop (qmk_generate_sample); eos_token_id < 0: none.
torch::Tensor generate_sample(int64_t first_token_id, int64_t num_steps, int64_t eos_token_id, double temperature,
                              int64_t top_k, double top_p, int64_t seed, torch::Tensor embed_weight,
                              torch::Tensor layer_weights_packed, torch::Tensor final_norm_weight,
                              torch::Tensor lm_head_weight, torch::Tensor cos_table, torch::Tensor sin_table,
                              torch::Tensor k_cache, torch::Tensor v_cache, torch::Tensor hidden_buffer,
                              torch::Tensor normalized, int64_t num_layers, int64_t start_position,
                              int64_t max_seq_len, double attn_scale) {
  const Checked c = check_common(embed_weight, layer_weights_packed, final_norm_weight, lm_head_weight, cos_table,
                                 sin_table, k_cache, v_cache, hidden_buffer, normalized, num_layers, max_seq_len,
                                 attn_scale);
  TORCH_CHECK(num_steps >= 0, "num_steps must be non-negative");
  TORCH_CHECK(start_position >= 0 && start_position + num_steps <= max_seq_len, "steps [", start_position, ", ",
              start_position + num_steps, ") do not fit in max_seq_len ", max_seq_len);
  TORCH_CHECK(first_token_id >= 0 && first_token_id < kVocab, "first_token_id outside the vocabulary");
  TORCH_CHECK(eos_token_id < kVocab, "eos_token_id outside the vocabulary");
  TORCH_CHECK(temperature == temperature && top_p == top_p, "temperature and top_p must not be NaN");
  const c10::hip::HIPGuardMasqueradingAsCUDA guard(embed_weight.device());
  auto stream = c10::hip::getCurrentHIPStreamMasqueradingAsCUDA().stream();
  auto output_log = torch::empty({num_steps}, torch::dtype(torch::kInt32).device(embed_weight.device()));
  if (num_steps == 0) return output_log;
  qmk_generate_sample(c.model, (int)first_token_id, (int)num_steps, (int)eos_token_id, (float)temperature, (int)top_k,
                      (float)top_p, (unsigned long long)seed, embed_weight.data_ptr(),
                      reinterpret_cast<const LDGLayerWeights*>(layer_weights_packed.data_ptr()),
                      final_norm_weight.data_ptr(), lm_head_weight.data_ptr(), cos_table.data_ptr(),
                      sin_table.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), hidden_buffer.data_ptr(),
                      normalized.data_ptr(), static_cast<int*>(output_log.data_ptr()), c.num_layers,
                      (int)start_position, c.max_seq_len, (float)attn_scale, stream);
  raise_status("generate_sample");
  const uint32_t err = qmk_device_error(stream);
  TORCH_CHECK(err == 0, "generate_sample: device error bits 0x", std::hex, err, "; call reset()");
  return output_log;
}

// One sampled token per row of fp32 logits (qmk_sample_rows).
void sample(torch::Tensor logits, double temperature, int64_t top_k, double top_p, int64_t seed,
            torch::Tensor counters, torch::Tensor out_tokens) {
  check_cuda(logits, "logits");
  TORCH_CHECK(logits.scalar_type() == torch::kFloat32 && logits.dim() == 2 && logits.size(0) >= 1 &&
                  logits.size(0) <= 65535 && logits.size(1) >= 1,
              "logits must be float32 [rows, vocab]");
  check_cuda(counters, "counters");
  TORCH_CHECK(counters.scalar_type() == torch::kInt64 && counters.numel() == logits.size(0),
              "counters must be int64 [rows]");
  check_cuda(out_tokens, "out_tokens");
  TORCH_CHECK(out_tokens.scalar_type() == torch::kInt32 && out_tokens.numel() == logits.size(0),
              "out_tokens must be int32 [rows]");
  TORCH_CHECK(counters.device() == logits.device() && out_tokens.device() == logits.device(),
              "all tensors must be on the same device");
  TORCH_CHECK(temperature == temperature && top_p == top_p, "temperature and top_p must not be NaN");
  const c10::hip::HIPGuardMasqueradingAsCUDA guard(logits.device());
  const int s = qmk_sample_rows(static_cast<const float*>(logits.data_ptr()), (int)logits.size(0),
                                (int)logits.size(1), (float)temperature, (int)top_k, (float)top_p,
                                (unsigned long long)seed, static_cast<const long long*>(counters.data_ptr()),
                                static_cast<int*>(out_tokens.data_ptr()),
                                c10::hip::getCurrentHIPStreamMasqueradingAsCUDA().stream());
  TORCH_CHECK(s == QMK_OK, "sample failed: ", qmk_status_string(s));
}

void set_graph_launch(bool enable) {
  const int s = qmk_set_graph_launch(c10::hip::getCurrentHIPStreamMasqueradingAsCUDA().stream(), enable ? 1 : 0);
  TORCH_CHECK(s == QMK_OK, "set_graph_launch failed: ", qmk_status_string(s));
}

void decode_logits(torch::Tensor output_token, torch::Tensor logits, int64_t input_token_id,
                   torch::Tensor embed_weight, torch::Tensor layer_weights_packed, torch::Tensor final_norm_weight,
                   torch::Tensor lm_head_weight, torch::Tensor cos_table, torch::Tensor sin_table,
                   torch::Tensor k_cache, torch::Tensor v_cache, torch::Tensor hidden_buffer,
                   torch::Tensor normalized, int64_t num_layers, int64_t position, int64_t max_seq_len,
                   double attn_scale) {
  const Checked c = check_common(embed_weight, layer_weights_packed, final_norm_weight, lm_head_weight, cos_table,
                                 sin_table, k_cache, v_cache, hidden_buffer, normalized, num_layers, max_seq_len,
                                 attn_scale);
  check_cuda(output_token, "output_token");
  TORCH_CHECK(output_token.scalar_type() == torch::kInt32 && output_token.numel() >= 1, "output_token must be int32[1]");
  check_cuda(logits, "logits");
  TORCH_CHECK(logits.scalar_type() == torch::kFloat32 && logits.numel() == kVocab, "logits must be float32[151936]");
  TORCH_CHECK(position >= 0 && position < max_seq_len, "position ", position, " outside [0, ", max_seq_len, ")");
  TORCH_CHECK(input_token_id >= 0 && input_token_id < kVocab, "input_token_id outside the vocabulary");
  const c10::hip::HIPGuardMasqueradingAsCUDA guard(embed_weight.device());
  qmk_decode_model(c.model, (int)input_token_id, static_cast<int*>(output_token.data_ptr()),
                    static_cast<float*>(logits.data_ptr()), embed_weight.data_ptr(),
                    reinterpret_cast<const LDGLayerWeights*>(layer_weights_packed.data_ptr()),
                    final_norm_weight.data_ptr(), lm_head_weight.data_ptr(), cos_table.data_ptr(),
                    sin_table.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), hidden_buffer.data_ptr(),
                    normalized.data_ptr(), c.num_layers, (int)position, c.max_seq_len, (float)attn_scale,
                    c10::hip::getCurrentHIPStreamMasqueradingAsCUDA().stream());
  raise_status("decode_logits");
}

int64_t device_error() {
  return (int64_t)qmk_device_error(c10::hip::getCurrentHIPStreamMasqueradingAsCUDA().stream());
}

void reset() {
  const int s = qmk_reset(c10::hip::getCurrentHIPStreamMasqueradingAsCUDA().stream());
  TORCH_CHECK(s == QMK_OK, "reset failed: ", qmk_status_string(s));
}

void set_wait_limit(int64_t ticks) {
  TORCH_CHECK(ticks >= 0 && ticks <= 0xffffffffLL, "ticks out of range");
  const int s = qmk_set_wait_limit(c10::hip::getCurrentHIPStreamMasqueradingAsCUDA().stream(), (uint32_t)ticks);
  TORCH_CHECK(s == QMK_OK, "set_wait_limit failed: ", qmk_status_string(s));
}

void set_trace(std::optional<torch::Tensor> buf) {
  auto stream = c10::hip::getCurrentHIPStreamMasqueradingAsCUDA().stream();
  int s;
  if (buf.has_value()) {
    check_cuda(*buf, "trace");
    TORCH_CHECK(buf->scalar_type() == torch::kInt64, "trace buffer must be int64");
    s = qmk_set_trace(stream, reinterpret_cast<uint64_t*>(buf->data_ptr()), (size_t)buf->numel());
  } else {
    s = qmk_set_trace(stream, nullptr, 0);
  }
  TORCH_CHECK(s == QMK_OK, "set_trace failed: ", qmk_status_string(s));
}

// Per-phase weight-streaming microbenchmark (qmk_phase_bench): `weights`
// holds n_copies copies of the phase's matrices back to back.
void phase_bench(int64_t phase, torch::Tensor weights, int64_t n_copies, std::optional<torch::Tensor> norm_weight,
                 torch::Tensor act, torch::Tensor out) {
  const size_t per = qmk_phase_copy_elems((int)phase);
  TORCH_CHECK(per > 0, "phase must be 0 (QKV), 1 (O), 2 (GATE_UP), 3 (DOWN) or 4 (LM_HEAD)");
  TORCH_CHECK(n_copies >= 1 && n_copies <= (1 << 20), "n_copies out of range");
  check_bf16(weights, "weights", -1);
  TORCH_CHECK(weights.numel() >= (int64_t)per * n_copies, "weights holds fewer than n_copies copies");
  static const int64_t in_len[5] = {kHidden, kQ, kHidden, kInter, kHidden};
  check_bf16(act, "act", in_len[phase]);
  check_cuda(out, "out");
  static const int64_t out_bytes[5] = {(kQ + 2 * kKV) * 2, 8 * kHidden * 4, kInter * 2, 8 * kHidden * 4, 256 * 8 * 8};
  TORCH_CHECK(out.numel() * out.element_size() >= out_bytes[phase], "out is smaller than ", out_bytes[phase], " bytes");
  const void* nw = nullptr;
  if (phase == 0) {
    TORCH_CHECK(norm_weight.has_value(), "phase 0 needs norm_weight");
    check_bf16(*norm_weight, "norm_weight", kHidden);
    nw = norm_weight->data_ptr();
  }
  const c10::hip::HIPGuardMasqueradingAsCUDA guard(weights.device());
  const int s = qmk_phase_bench((int)phase, weights.data_ptr(), (int)n_copies, nw, act.data_ptr(), out.data_ptr(),
                                c10::hip::getCurrentHIPStreamMasqueradingAsCUDA().stream());
  TORCH_CHECK(s == QMK_OK, "phase_bench failed: ", qmk_status_string(s));
}

// Batched forward (qmk_forward_tokens): T tokens of any sequences at any
// positions through the MFMA path; prefill and batched decode.  k_cache /
// v_cache are [L, 8, S, 128] (one sequence) or [B, L, 8, S, 128];
// layer_weights is the reference's flat list of 11 tensors per layer
// (qwen_megakernel/model.py:82-89).
int model_of_hidden(int64_t hidden) {
  TORCH_CHECK(hidden == 1024 || hidden == 2048, "hidden must be 1024 (Qwen3-0.6B) or 2048 (Qwen3-1.7B)");
  return hidden == 1024 ? QMK_MODEL_QWEN3_0_6B : QMK_MODEL_QWEN3_1_7B;
}

int64_t forward_workspace_bytes(int64_t hidden, int64_t num_tokens, int64_t num_emit, int64_t max_context) {
  TORCH_CHECK(num_tokens >= 1 && num_tokens <= (1 << 20), "num_tokens out of range");
  TORCH_CHECK(num_emit >= 1 && num_emit <= 256, "num_emit must be in [1, 256]");
  TORCH_CHECK(max_context >= 1 && max_context <= 65536, "max_context must be in [1, 65536]");
  return (int64_t)qmk_forward_workspace_bytes(model_of_hidden(hidden), (int)num_tokens, (int)num_emit,
                                              (int)max_context);
}

struct BatchModel {
  int model;
  std::vector<LDGLayerWeights> table;
  int64_t num_seqs, max_seq_len, seq_stride;
};

// Checks the weights (reference flat list of 11 per layer) and the caches
// ([L, 8, S, 128] or [B, L, 8, S, 128]) of a batched call.
BatchModel check_batch_model(const torch::Tensor& embed_weight, const std::vector<torch::Tensor>& layer_weights,
                             const torch::Tensor& final_norm_weight, const torch::Tensor& lm_head_weight,
                             const torch::Tensor& cos_table, const torch::Tensor& sin_table,
                             const torch::Tensor& k_cache, const torch::Tensor& v_cache, int64_t num_layers,
                             int64_t max_context, double attn_scale) {
  check_bf16(embed_weight, "embed_weight", -1);
  const int64_t hidden = embed_weight.numel() / kVocab;
  TORCH_CHECK(embed_weight.numel() == kVocab * hidden, "embed_weight must be [151936, hidden]");
  BatchModel bm;
  bm.model = model_of_hidden(hidden);
  const int64_t inter = 3 * hidden;
  TORCH_CHECK(num_layers >= 1 && num_layers <= kMaxLayers, "num_layers must be in [1, 28], got ", num_layers);
  TORCH_CHECK(attn_scale > 0.0, "attn_scale must be positive");
  check_bf16(final_norm_weight, "final_norm_weight", hidden);
  check_bf16(lm_head_weight, "lm_head_weight", kVocab * hidden);
  TORCH_CHECK((int64_t)layer_weights.size() >= 11 * num_layers, "layer_weights must hold 11 tensors per layer");
  const int64_t sizes[11] = {hidden, kQ * hidden, kKV * hidden, kKV * hidden, kHeadDim, kHeadDim,
                             hidden * kQ, hidden, inter * hidden, inter * hidden, hidden * inter};
  bm.table.resize((size_t)num_layers);
  for (int64_t L = 0; L < num_layers; L++) {
    const void* p[11];
    for (int i = 0; i < 11; i++) {
      const torch::Tensor& t = layer_weights[(size_t)(11 * L + i)];
      check_bf16(t, "layer weight", sizes[i]);
      TORCH_CHECK(t.device() == embed_weight.device(), "all tensors must be on the same device");
      p[i] = t.data_ptr();
    }
    bm.table[(size_t)L] = LDGLayerWeights{p[0], p[1], p[2], p[3], p[4], p[5], p[6], p[7], p[8], p[9], p[10]};
  }
  check_bf16(k_cache, "k_cache", -1);
  check_bf16(v_cache, "v_cache", -1);
  TORCH_CHECK(v_cache.sizes() == k_cache.sizes(), "v_cache must match k_cache");
  TORCH_CHECK((k_cache.dim() == 4 || k_cache.dim() == 5) && k_cache.size(-3) == kKVHeads &&
                  k_cache.size(-1) == kHeadDim && k_cache.size(-4) >= num_layers,
              "k_cache must be [>= num_layers, 8, S, 128] or [B, >= num_layers, 8, S, 128]");
  bm.max_seq_len = k_cache.size(-2);
  bm.num_seqs = k_cache.dim() == 5 ? k_cache.size(0) : 1;
  TORCH_CHECK(bm.num_seqs >= 1 && bm.max_seq_len >= 1 && bm.max_seq_len <= 65536, "k_cache sizes out of range");
  bm.seq_stride = k_cache.size(-4) * kKVHeads * bm.max_seq_len * kHeadDim;
  TORCH_CHECK(max_context >= 1 && max_context <= bm.max_seq_len, "max_context must be in [1, ", bm.max_seq_len, "]");
  check_bf16(cos_table, "cos_table", -1);
  check_bf16(sin_table, "sin_table", -1);
  TORCH_CHECK(cos_table.dim() == 2 && cos_table.size(1) == kHeadDim && cos_table.size(0) >= bm.max_seq_len,
              "cos_table must be [>= max_seq_len, 128]");
  TORCH_CHECK(sin_table.sizes() == cos_table.sizes(), "sin_table must match cos_table");
  for (const torch::Tensor* t : {&final_norm_weight, &lm_head_weight, &cos_table, &sin_table, &k_cache, &v_cache})
    TORCH_CHECK(t->device() == embed_weight.device(), "all tensors must be on the same device");
  return bm;
}

int64_t decode_batch_workspace_bytes(int64_t hidden, int64_t batch, int64_t max_context) {
  TORCH_CHECK(batch >= 1 && batch <= 256, "batch must be in [1, 256]");
  TORCH_CHECK(max_context >= 1 && max_context <= 65536, "max_context must be in [1, 65536]");
  return (int64_t)qmk_decode_batch_workspace_bytes(model_of_hidden(hidden), (int)batch, (int)max_context);
}

// One batched decode step (qmk_decode_batch): tokens[b] of sequence b at positions[b].
void decode_batch(torch::Tensor tokens, torch::Tensor positions, torch::Tensor out_tokens,
                  std::optional<torch::Tensor> logits, torch::Tensor embed_weight,
                  std::vector<torch::Tensor> layer_weights, torch::Tensor final_norm_weight,
                  torch::Tensor lm_head_weight, torch::Tensor cos_table, torch::Tensor sin_table,
                  torch::Tensor k_cache, torch::Tensor v_cache, torch::Tensor workspace, int64_t num_layers,
                  int64_t max_context, double attn_scale) {
  const BatchModel bm = check_batch_model(embed_weight, layer_weights, final_norm_weight, lm_head_weight, cos_table,
                                          sin_table, k_cache, v_cache, num_layers, max_context, attn_scale);
  const int64_t B = tokens.numel();
  for (const torch::Tensor* t : {&tokens, &positions, &out_tokens}) {
    check_cuda(*t, "token arrays");
    TORCH_CHECK(t->scalar_type() == torch::kInt32, "tokens, positions, out_tokens must be int32");
    TORCH_CHECK(t->device() == embed_weight.device(), "all tensors must be on the same device");
  }
  TORCH_CHECK(B >= 1 && B <= 256, "tokens must hold 1 .. 256 entries");
  TORCH_CHECK(positions.numel() == B && out_tokens.numel() == B, "positions and out_tokens must match tokens");
  TORCH_CHECK(bm.num_seqs == B, "k_cache must hold one sequence per token (", B, "), got ", bm.num_seqs);
  // out_tokens may share memory with tokens or positions (an in-place step): qmk_decode_batch then
  // takes its multi-launch path, which reads them before writing
  float* lg = nullptr;
  if (logits.has_value()) {
    check_cuda(*logits, "logits");
    TORCH_CHECK(logits->scalar_type() == torch::kFloat32 && logits->numel() == B * kVocab,
                "logits must be float32[batch, 151936]");
    lg = static_cast<float*>(logits->data_ptr());
  }
  check_cuda(workspace, "workspace");
  TORCH_CHECK(workspace.device() == embed_weight.device(), "all tensors must be on the same device");
  const size_t need = qmk_decode_batch_workspace_bytes(bm.model, (int)B, (int)max_context);
  TORCH_CHECK((size_t)(workspace.numel() * workspace.element_size()) >= need, "workspace is smaller than ", need,
              " bytes");
  const c10::hip::HIPGuardMasqueradingAsCUDA guard(embed_weight.device());
  const int s = qmk_decode_batch(
      bm.model, (int)B, static_cast<const int*>(tokens.data_ptr()), static_cast<const int*>(positions.data_ptr()),
      static_cast<int*>(out_tokens.data_ptr()), lg, embed_weight.data_ptr(), bm.table.data(),
      final_norm_weight.data_ptr(), lm_head_weight.data_ptr(), cos_table.data_ptr(), sin_table.data_ptr(),
      k_cache.data_ptr(), v_cache.data_ptr(), (long long)bm.seq_stride, (int)num_layers, (int)bm.max_seq_len,
      (int)max_context, (float)attn_scale, workspace.data_ptr(), need,
      c10::hip::getCurrentHIPStreamMasqueradingAsCUDA().stream());
  TORCH_CHECK(s == QMK_OK, "decode_batch failed: ", qmk_status_string(s));
}

void forward_tokens(torch::Tensor tokens, torch::Tensor seq_ids, torch::Tensor positions, torch::Tensor emit_rows,
                    torch::Tensor out_tokens, std::optional<torch::Tensor> logits, torch::Tensor embed_weight,
                    std::vector<torch::Tensor> layer_weights, torch::Tensor final_norm_weight,
                    torch::Tensor lm_head_weight, torch::Tensor cos_table, torch::Tensor sin_table,
                    torch::Tensor k_cache, torch::Tensor v_cache, torch::Tensor workspace, int64_t num_layers,
                    int64_t max_context, double attn_scale) {
  check_bf16(embed_weight, "embed_weight", -1);
  const int64_t hidden = embed_weight.numel() / kVocab;
  TORCH_CHECK(embed_weight.numel() == kVocab * hidden, "embed_weight must be [151936, hidden]");
  const int model = model_of_hidden(hidden);
  const int64_t inter = 3 * hidden;
  TORCH_CHECK(num_layers >= 1 && num_layers <= kMaxLayers, "num_layers must be in [1, 28], got ", num_layers);
  TORCH_CHECK(attn_scale > 0.0, "attn_scale must be positive");
  check_bf16(final_norm_weight, "final_norm_weight", hidden);
  check_bf16(lm_head_weight, "lm_head_weight", kVocab * hidden);
  TORCH_CHECK((int64_t)layer_weights.size() >= 11 * num_layers, "layer_weights must hold 11 tensors per layer");
  const int64_t sizes[11] = {hidden, kQ * hidden, kKV * hidden, kKV * hidden, kHeadDim, kHeadDim,
                             hidden * kQ, hidden, inter * hidden, inter * hidden, hidden * inter};
  std::vector<LDGLayerWeights> table((size_t)num_layers);
  for (int64_t L = 0; L < num_layers; L++) {
    const void* p[11];
    for (int i = 0; i < 11; i++) {
      const torch::Tensor& t = layer_weights[(size_t)(11 * L + i)];
      check_bf16(t, "layer weight", sizes[i]);
      TORCH_CHECK(t.device() == embed_weight.device(), "all tensors must be on the same device");
      p[i] = t.data_ptr();
    }
    table[(size_t)L] = LDGLayerWeights{p[0], p[1], p[2], p[3], p[4], p[5], p[6], p[7], p[8], p[9], p[10]};
  }
  check_bf16(k_cache, "k_cache", -1);
  check_bf16(v_cache, "v_cache", -1);
  TORCH_CHECK(v_cache.sizes() == k_cache.sizes(), "v_cache must match k_cache");
  TORCH_CHECK((k_cache.dim() == 4 || k_cache.dim() == 5) && k_cache.size(-3) == kKVHeads &&
                  k_cache.size(-1) == kHeadDim && k_cache.size(-4) >= num_layers,
              "k_cache must be [>= num_layers, 8, S, 128] or [B, >= num_layers, 8, S, 128]");
  const int64_t max_seq_len = k_cache.size(-2);
  const int64_t num_seqs = k_cache.dim() == 5 ? k_cache.size(0) : 1;
  TORCH_CHECK(num_seqs >= 1 && max_seq_len >= 1 && max_seq_len <= 65536, "k_cache sizes out of range");
  const int64_t seq_stride = k_cache.size(-4) * kKVHeads * max_seq_len * kHeadDim;
  TORCH_CHECK(max_context >= 1 && max_context <= max_seq_len, "max_context must be in [1, ", max_seq_len, "]");
  check_bf16(cos_table, "cos_table", -1);
  check_bf16(sin_table, "sin_table", -1);
  TORCH_CHECK(cos_table.dim() == 2 && cos_table.size(1) == kHeadDim && cos_table.size(0) >= max_seq_len,
              "cos_table must be [>= max_seq_len, 128]");
  TORCH_CHECK(sin_table.sizes() == cos_table.sizes(), "sin_table must match cos_table");
  for (const torch::Tensor* t : {&tokens, &seq_ids, &positions, &emit_rows, &out_tokens}) {
    check_cuda(*t, "token arrays");
    TORCH_CHECK(t->scalar_type() == torch::kInt32, "tokens, seq_ids, positions, emit_rows, out_tokens must be int32");
    TORCH_CHECK(t->device() == embed_weight.device(), "all tensors must be on the same device");
  }
  const int64_t T = tokens.numel(), R = emit_rows.numel();
  TORCH_CHECK(T >= 1 && T <= (1 << 20), "tokens must hold 1 .. 2^20 entries");
  TORCH_CHECK(seq_ids.numel() == T && positions.numel() == T, "seq_ids and positions must match tokens");
  TORCH_CHECK(R >= 1 && R <= 256, "emit_rows must hold 1 .. 256 entries");
  TORCH_CHECK(out_tokens.numel() == R, "out_tokens must match emit_rows");
  float* lg = nullptr;
  if (logits.has_value()) {
    check_cuda(*logits, "logits");
    TORCH_CHECK(logits->scalar_type() == torch::kFloat32 && logits->numel() == R * kVocab,
                "logits must be float32[num_emit, 151936]");
    lg = static_cast<float*>(logits->data_ptr());
  }
  check_cuda(workspace, "workspace");
  const size_t need = qmk_forward_workspace_bytes(model, (int)T, (int)R, (int)max_context);
  TORCH_CHECK((size_t)(workspace.numel() * workspace.element_size()) >= need, "workspace is smaller than ", need,
              " bytes");
  for (const torch::Tensor* t : {&final_norm_weight, &lm_head_weight, &cos_table, &sin_table, &k_cache, &v_cache,
                                 &workspace})
    TORCH_CHECK(t->device() == embed_weight.device(), "all tensors must be on the same device");
  const c10::hip::HIPGuardMasqueradingAsCUDA guard(embed_weight.device());
  const int s = qmk_forward_tokens(
      model, (int)T, static_cast<const int*>(tokens.data_ptr()), static_cast<const int*>(seq_ids.data_ptr()),
      static_cast<const int*>(positions.data_ptr()), (int)R, static_cast<const int*>(emit_rows.data_ptr()),
      static_cast<int*>(out_tokens.data_ptr()), lg, embed_weight.data_ptr(), table.data(),
      final_norm_weight.data_ptr(), lm_head_weight.data_ptr(), cos_table.data_ptr(), sin_table.data_ptr(),
      k_cache.data_ptr(), v_cache.data_ptr(), (int)num_seqs, (long long)seq_stride, (int)num_layers,
      (int)max_seq_len, (int)max_context, (float)attn_scale, workspace.data_ptr(), need,
      c10::hip::getCurrentHIPStreamMasqueradingAsCUDA().stream());
  TORCH_CHECK(s == QMK_OK, "forward_tokens failed: ", qmk_status_string(s));
}

// decode_batch runs the batched persistent kernel where it applies (default), or always the
// multi-launch path (qmk_set_batch_persistent); returns the previous setting.
bool set_batch_persistent(bool enable) {
  const bool was = qmk_batch_persistent_enabled() != 0;
  qmk_set_batch_persistent(enable ? 1 : 0);
  return was;
}

void selftest_mfma(torch::Tensor a, torch::Tensor b, torch::Tensor c) {
  check_bf16(a, "a", 16 * 32);
  check_bf16(b, "b", 16 * 32);
  check_cuda(c, "c");
  TORCH_CHECK(c.scalar_type() == torch::kFloat32 && c.numel() == 256, "c must be float32[16, 16]");
  const c10::hip::HIPGuardMasqueradingAsCUDA guard(a.device());
  const int s = qmk_selftest_mfma(a.data_ptr(), b.data_ptr(), static_cast<float*>(c.data_ptr()),
                                  c10::hip::getCurrentHIPStreamMasqueradingAsCUDA().stream());
  TORCH_CHECK(s == QMK_OK, "selftest_mfma failed: ", qmk_status_string(s));
}

}  // namespace

TORCH_LIBRARY(qwen_megakernel_C, ops) {
  ops.def(
      "decode(Tensor output_token, int input_token_id, "
      "Tensor embed_weight, Tensor layer_weights_packed, "
      "Tensor final_norm_weight, Tensor lm_head_weight, "
      "Tensor cos_table, Tensor sin_table, "
      "Tensor k_cache, Tensor v_cache, "
      "Tensor hidden_buffer, Tensor activations, Tensor residual, "
      "Tensor q, Tensor k, Tensor v, Tensor attn_out, "
      "Tensor mlp_intermediate, Tensor normalized, "
      "Tensor block_max_vals, Tensor block_max_idxs, "
      "int num_layers, int position, int max_seq_len, "
      "float attn_scale) -> ()");
  ops.impl("decode", torch::kCUDA, &decode);

  ops.def(
      "generate_nosync(int first_token_id, int num_steps, "
      "Tensor embed_weight, Tensor layer_weights_packed, "
      "Tensor final_norm_weight, Tensor lm_head_weight, "
      "Tensor cos_table, Tensor sin_table, "
      "Tensor k_cache, Tensor v_cache, "
      "Tensor hidden_buffer, Tensor activations, Tensor residual, "
      "Tensor q, Tensor k, Tensor v, Tensor attn_out, "
      "Tensor mlp_intermediate, Tensor normalized, "
      "Tensor block_max_vals, Tensor block_max_idxs, "
      "int num_layers, int start_position, int max_seq_len, "
      "float attn_scale) -> Tensor");
  ops.impl("generate_nosync", torch::kCUDA, &generate_nosync);

  ops.def(
      "decode_logits(Tensor output_token, Tensor logits, int input_token_id, "
      "Tensor embed_weight, Tensor layer_weights_packed, "
      "Tensor final_norm_weight, Tensor lm_head_weight, "
      "Tensor cos_table, Tensor sin_table, Tensor k_cache, Tensor v_cache, "
      "Tensor hidden_buffer, Tensor normalized, "
      "int num_layers, int position, int max_seq_len, float attn_scale) -> ()");
  ops.impl("decode_logits", torch::kCUDA, &decode_logits);

  ops.def(
      "generate_eos(int first_token_id, int num_steps, int eos_token_id, "
      "Tensor embed_weight, Tensor layer_weights_packed, "
      "Tensor final_norm_weight, Tensor lm_head_weight, "
      "Tensor cos_table, Tensor sin_table, Tensor k_cache, Tensor v_cache, "
      "Tensor hidden_buffer, Tensor normalized, "
      "int num_layers, int start_position, int max_seq_len, float attn_scale) -> Tensor");
  ops.impl("generate_eos", torch::kCUDA, &generate_eos);
  ops.def("set_graph_launch(bool enable) -> ()", &set_graph_launch);
  ops.def(
      "generate_sample(int first_token_id, int num_steps, int eos_token_id, float temperature, int top_k, "
      "float top_p, int seed, Tensor embed_weight, Tensor layer_weights_packed, "
      "Tensor final_norm_weight, Tensor lm_head_weight, "
      "Tensor cos_table, Tensor sin_table, Tensor k_cache, Tensor v_cache, "
      "Tensor hidden_buffer, Tensor normalized, "
      "int num_layers, int start_position, int max_seq_len, float attn_scale) -> Tensor");
  ops.impl("generate_sample", torch::kCUDA, &generate_sample);
  ops.def("sample(Tensor logits, float temperature, int top_k, float top_p, int seed, Tensor counters, "
          "Tensor out_tokens) -> ()");
  ops.impl("sample", torch::kCUDA, &sample);
  ops.def("device_error() -> int", &device_error);
  ops.def("reset() -> ()", &reset);
  ops.def("set_wait_limit(int ticks) -> ()", &set_wait_limit);
  ops.def("set_trace(Tensor? buf) -> ()", &set_trace);
  ops.def("phase_bench(int phase, Tensor weights, int n_copies, Tensor? norm_weight, Tensor act, Tensor out) -> ()");
  ops.impl("phase_bench", torch::kCUDA, &phase_bench);

  ops.def("forward_workspace_bytes(int hidden, int num_tokens, int num_emit, int max_context) -> int",
          &forward_workspace_bytes);
  ops.def(
      "forward_tokens(Tensor tokens, Tensor seq_ids, Tensor positions, Tensor emit_rows, "
      "Tensor out_tokens, Tensor? logits, Tensor embed_weight, Tensor[] layer_weights, "
      "Tensor final_norm_weight, Tensor lm_head_weight, Tensor cos_table, Tensor sin_table, "
      "Tensor k_cache, Tensor v_cache, Tensor workspace, int num_layers, int max_context, "
      "float attn_scale) -> ()");
  ops.impl("forward_tokens", torch::kCUDA, &forward_tokens);
  ops.def("decode_batch_workspace_bytes(int hidden, int batch, int max_context) -> int",
          &decode_batch_workspace_bytes);
  ops.def(
      "decode_batch(Tensor tokens, Tensor positions, Tensor out_tokens, Tensor? logits, Tensor embed_weight, "
      "Tensor[] layer_weights, Tensor final_norm_weight, Tensor lm_head_weight, Tensor cos_table, "
      "Tensor sin_table, Tensor k_cache, Tensor v_cache, Tensor workspace, int num_layers, int max_context, "
      "float attn_scale) -> ()");
  ops.impl("decode_batch", torch::kCUDA, &decode_batch);
  ops.def("set_batch_persistent(bool enable) -> bool", &set_batch_persistent);
  ops.def("selftest_mfma(Tensor a, Tensor b, Tensor c) -> ()");
  ops.impl("selftest_mfma", torch::kCUDA, &selftest_mfma);
}

// Empty Python module so the shared object can also be imported by name
// (reference csrc/torch_bindings.cpp:14-19, 157).
extern "C" PyObject* PyInit_qwen_megakernel_C() {
  static struct PyModuleDef module = {PyModuleDef_HEAD_INIT, "qwen_megakernel_C", nullptr, 0, nullptr};
  return PyModule_Create(&module);
}
