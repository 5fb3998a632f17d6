// Host-side AddressSanitizer driver for the C ABI (include/qwen_megakernel.h).
//
// Test infrastructure.  Built by tests/asan/Makefile against a copy of libqwen_megakernel_amd whose
// host code is compiled with -fsanitize=address (device code unchanged), and run by
// tests/test_asan_host.py.  It calls every entry point: first the argument checks that return
// before touching a GPU (null pointers, out-of-range sizes, unknown models), then, when a GPU is
// present, real launches of every host path on a 2-layer Qwen3-0.6B with constant weights --
// decode, the reference-named launchers, generate (greedy, stop token, sampled), the
// allocation-free entry point, the batched step (persistent kernel, multi-launch path, an
// in-place call, 16 sequences), the batched forward, the row sampler, tracing, a second stream and
// the bounded-wait failure path.  The numbers are not checked (the GPU tests do that); every call's
// status is, and ASan reports any invalid host memory access.  Exit status: 0 when every status
// was as expected (ASan exits non-zero on a report).
#include <hip/hip_runtime_api.h>

#include <cstdint>
#include <cstdio>
#include <cstring>
#include <vector>

#include "../../include/qwen_megakernel.h"

namespace {

int g_fail = 0;

void expect(bool ok, const char* what) {
  if (!ok) {
    std::printf("FAIL %s (last status %d: %s)\n", what, qmk_last_status(), qmk_status_string(qmk_last_status()));
    g_fail++;
  }
}

constexpr int kV = 151936, kH = 1024, kI = 3072, kQ = 2048, kKV = 1024, kD = 128;
constexpr int kLayers = 2, kSeq = 256;

struct Buffers {
  std::vector<void*> all;
  void* get(size_t bytes, uint16_t fill) {
    void* p = nullptr;
    if (hipMalloc(&p, bytes) != hipSuccess) return nullptr;
    if (hipMemsetD16(reinterpret_cast<hipDeviceptr_t>(p), fill, bytes / 2) != hipSuccess) return nullptr;
    all.push_back(p);
    return p;
  }
  ~Buffers() {
    for (void* p : all) (void)hipFree(p);
  }
};

void host_argument_checks() {
  // every call here fails its argument checks before any GPU work
  expect(qmk_decode_model(7, 1, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr,
                          nullptr, nullptr, nullptr, 28, 0, 256, 0.088f, nullptr) != QMK_OK,
         "decode: unknown model, null pointers");
  expect(qmk_generate_model(0, 1, 4, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr,
                            nullptr, nullptr, 28, 0, 256, 0.088f, nullptr) != QMK_OK,
         "generate: null pointers");
  expect(qmk_sample_rows(nullptr, 1, 10, 1.f, 0, 1.f, 1, nullptr, nullptr, nullptr) != QMK_OK, "sample: null rows");
  expect(qmk_decode_batch(0, 0, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr,
                          nullptr, nullptr, nullptr, 0, 28, 256, 16, 0.088f, nullptr, 0, nullptr) == QMK_ERR_ARG,
         "decode_batch: batch 0");
  expect(qmk_forward_tokens(0, 0, nullptr, nullptr, nullptr, 1, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr,
                            nullptr, nullptr, nullptr, nullptr, nullptr, 1, 0, 28, 256, 16, 0.088f, nullptr, 0,
                            nullptr) != QMK_OK,
         "forward_tokens: no tokens");
  expect(qmk_forward_workspace_bytes(5, 16, 1, 64) == 0, "forward workspace: unknown model");
  expect(qmk_decode_batch_workspace_bytes(0, 0, 64) == 0, "batch workspace: batch 0");
  expect(qmk_trace_entries(28) > qmk_trace_entries(2) && qmk_trace_entries(2) > 0, "trace entries");
  expect(qmk_noalloc_set_wait_limit(1) == QMK_ERR_INIT, "noalloc wait limit before qmk_init");
  expect(qmk_noalloc_device_error(nullptr) == 0xffffffffu, "noalloc error before qmk_init");
  for (int s = 0; s <= 8; s++) expect(qmk_status_string(s) != nullptr, "status string");
  int wg = 0, th = 0;
  qmk_launch_geometry(&wg, &th);
  expect(wg == 256 && th > 0, "launch geometry");
}

void gpu_paths() {
  expect(qmk_init() == QMK_OK, "qmk_init");
  Buffers b;
  const uint16_t w = 0x3c3c, one = 0x3f80;  // bf16 0.0115 and 1.0
  void* embed = b.get((size_t)kV * kH * 2, w);
  void* fnorm = b.get(kH * 2, one);
  void* cos_t = b.get((size_t)kSeq * kD * 2, one);
  void* sin_t = b.get((size_t)kSeq * kD * 2, 0);
  std::vector<LDGLayerWeights> table(kLayers);
  for (int L = 0; L < kLayers; L++) {
    table[L].input_layernorm_weight = b.get(kH * 2, one);
    table[L].q_proj_weight = b.get((size_t)kQ * kH * 2, w);
    table[L].k_proj_weight = b.get((size_t)kKV * kH * 2, w);
    table[L].v_proj_weight = b.get((size_t)kKV * kH * 2, w);
    table[L].q_norm_weight = b.get(kD * 2, one);
    table[L].k_norm_weight = b.get(kD * 2, one);
    table[L].o_proj_weight = b.get((size_t)kH * kQ * 2, w);
    table[L].post_attn_layernorm_weight = b.get(kH * 2, one);
    table[L].gate_proj_weight = b.get((size_t)kI * kH * 2, w);
    table[L].up_proj_weight = b.get((size_t)kI * kH * 2, w);
    table[L].down_proj_weight = b.get((size_t)kH * kI * 2, w);
  }
  LDGLayerWeights* dtable = static_cast<LDGLayerWeights*>(b.get(sizeof(LDGLayerWeights) * kLayers, 0));
  expect(dtable && hipMemcpy(dtable, table.data(), sizeof(LDGLayerWeights) * kLayers, hipMemcpyHostToDevice) == hipSuccess,
         "layer table upload");
  const size_t kv_bytes = (size_t)kLayers * 8 * kSeq * kD * 2;
  void* kc = b.get(kv_bytes * 16, 0);  // room for 16 sequences
  void* vc = b.get(kv_bytes * 16, 0);
  void* hidden = b.get(kH * 2, 0);
  void* normed = b.get(kH * 4, 0);
  int* tok = static_cast<int*>(b.get(64 * 4, 0));
  float* logits = static_cast<float*>(b.get((size_t)16 * kV * 4, 0));
  int* log = static_cast<int*>(b.get(4096 * 4, 0));
  const float scale = 0.08838834764831845f;
  hipStream_t s1 = nullptr, s2 = nullptr;
  expect(hipStreamCreate(&s1) == hipSuccess && hipStreamCreate(&s2) == hipSuccess, "streams");

  for (int p = 0; p < 4; p++)
    expect(qmk_decode_model(QMK_MODEL_QWEN3_0_6B, 11 + p, tok, logits, embed, dtable, fnorm, embed, cos_t, sin_t, kc, vc,
                            hidden, normed, kLayers, p, kSeq, scale, s1) == QMK_OK,
           "decode");
  expect(qmk_decode_logits(11, tok, logits, embed, dtable, fnorm, embed, cos_t, sin_t, kc, vc, hidden, normed, kLayers,
                           4, kSeq, scale, s1) == QMK_OK,
         "decode_logits");
  launch_ldg_decode_direct(12, tok, embed, dtable, fnorm, embed, cos_t, sin_t, kc, vc, hidden, nullptr, nullptr,
                           nullptr, nullptr, nullptr, nullptr, nullptr, normed, nullptr, nullptr, kLayers, 5, kSeq, scale,
                           s1);
  expect(qmk_last_status() == QMK_OK, "launch_ldg_decode_direct");
  launch_ldg_decode_persistent(13, tok, embed, dtable, fnorm, embed, cos_t, sin_t, kc, vc, hidden, nullptr, nullptr,
                               nullptr, nullptr, nullptr, nullptr, nullptr, normed, nullptr, nullptr, kLayers, 6, 7, kSeq,
                               scale, s1);
  expect(qmk_last_status() == QMK_OK, "launch_ldg_decode_persistent");
  launch_ldg_generate_nosync(14, 40, embed, dtable, fnorm, embed, cos_t, sin_t, kc, vc, hidden, nullptr, nullptr,
                             nullptr, nullptr, nullptr, nullptr, nullptr, normed, nullptr, nullptr, log, kLayers, 7, kSeq,
                             scale, s1);
  expect(qmk_last_status() == QMK_OK, "launch_ldg_generate_nosync");
  expect(qmk_generate_model(QMK_MODEL_QWEN3_0_6B, 15, 70, embed, dtable, fnorm, embed, cos_t, sin_t, kc, vc, hidden,
                            normed, log, kLayers, 50, kSeq, scale, s1) == QMK_OK,
         "generate");
  expect(qmk_generate_eos(QMK_MODEL_QWEN3_0_6B, 15, 20, 0, embed, dtable, fnorm, embed, cos_t, sin_t, kc, vc, hidden,
                          normed, log, kLayers, 130, kSeq, scale, s1) == QMK_OK,
         "generate_eos");
  expect(qmk_generate_sample(QMK_MODEL_QWEN3_0_6B, 15, 20, -1, 0.8f, 20, 0.9f, 7, embed, dtable, fnorm, embed, cos_t,
                             sin_t, kc, vc, hidden, normed, log, kLayers, 160, kSeq, scale, s1) == QMK_OK,
         "generate_sample");
  expect(qmk_decode_model_noalloc(QMK_MODEL_QWEN3_0_6B, 11, tok, logits, embed, dtable, fnorm, embed, cos_t, sin_t, kc,
                                  vc, hidden, normed, kLayers, 3, kSeq, scale, s1) == QMK_OK,
         "noalloc");
  expect(qmk_noalloc_device_error(s1) == 0u, "noalloc error bits");
  expect(qmk_noalloc_set_wait_limit(0) == QMK_OK, "noalloc wait limit");
  expect(qmk_decode_model_noalloc(QMK_MODEL_QWEN3_0_6B, 11, tok, logits, embed, dtable, fnorm, embed, cos_t, sin_t, kc,
                                  vc, hidden, normed, 29, 3, kSeq, scale, s1) == QMK_ERR_SIZE,
         "noalloc: too many layers");

  // batched forward: a 40-token prompt of sequence 0
  {
    std::vector<int> h_tok(40), h_seq(40, 0), h_pos(40), h_emit{39};
    for (int i = 0; i < 40; i++) {
      h_tok[i] = 100 + i;
      h_pos[i] = i;
    }
    int* d = static_cast<int*>(b.get(4 * 128, 0));
    expect(hipMemcpy(d, h_tok.data(), 160, hipMemcpyHostToDevice) == hipSuccess &&
               hipMemcpy(d + 40, h_seq.data(), 160, hipMemcpyHostToDevice) == hipSuccess &&
               hipMemcpy(d + 80, h_pos.data(), 160, hipMemcpyHostToDevice) == hipSuccess &&
               hipMemcpy(d + 120, h_emit.data(), 4, hipMemcpyHostToDevice) == hipSuccess,
           "forward inputs");
    const size_t ws_bytes = qmk_forward_workspace_bytes(QMK_MODEL_QWEN3_0_6B, 40, 1, 40);
    void* ws = b.get(ws_bytes + 256, 0);
    expect(qmk_forward_tokens(QMK_MODEL_QWEN3_0_6B, 40, d, d + 40, d + 80, 1, d + 120, tok, logits, embed, table.data(),
                              fnorm, embed, cos_t, sin_t, kc, vc, 1, 0, kLayers, kSeq, 40, scale, ws, ws_bytes,
                              s1) == QMK_OK,
           "forward_tokens");
  }

  // batched decode steps: 4 sequences (persistent kernel, twice: its layer table is then cached),
  // 2 on the multi-launch path, an in-place call, 16 sequences (five-launch path)
  {
    const long long stride = (long long)kLayers * 8 * kSeq * kD;
    int* d = static_cast<int*>(b.get(4 * 64, 0));
    std::vector<int> h(32);
    for (int i = 0; i < 16; i++) {
      h[i] = 200 + i;
      h[16 + i] = 10 + i;
    }
    expect(hipMemcpy(d, h.data(), 128, hipMemcpyHostToDevice) == hipSuccess, "batch inputs");
    const size_t ws_bytes = qmk_decode_batch_workspace_bytes(QMK_MODEL_QWEN3_0_6B, 16, 64);
    void* ws = b.get(ws_bytes + 256, 0);
    for (int rep = 0; rep < 2; rep++)
      expect(qmk_decode_batch(QMK_MODEL_QWEN3_0_6B, 4, d, d + 16, tok, logits, embed, table.data(), fnorm, embed, cos_t,
                              sin_t, kc, vc, stride, kLayers, kSeq, 64, scale, ws, ws_bytes, s1) == QMK_OK,
             "decode_batch 4");
    expect(qmk_decode_batch_persistent(QMK_MODEL_QWEN3_0_6B, 3, d, d + 16, tok, nullptr, embed, table.data(), fnorm,
                                       embed, cos_t, sin_t, kc, vc, stride, kLayers, kSeq, 64, scale, s1) == QMK_OK,
           "decode_batch_persistent 3");
    expect(qmk_decode_batch_persistent(QMK_MODEL_QWEN3_0_6B, 3, d, d + 16, d, nullptr, embed, table.data(), fnorm,
                                       embed, cos_t, sin_t, kc, vc, stride, kLayers, kSeq, 64, scale, s1) == QMK_ERR_ARG,
           "decode_batch_persistent: out_tokens over tokens");
    expect(qmk_decode_batch(QMK_MODEL_QWEN3_0_6B, 4, d, d + 16, d, nullptr, embed, table.data(), fnorm, embed, cos_t,
                            sin_t, kc, vc, stride, kLayers, kSeq, 64, scale, ws, ws_bytes, s1) == QMK_OK,
           "decode_batch in place");
    expect(hipMemcpy(d, h.data(), 128, hipMemcpyHostToDevice) == hipSuccess, "batch inputs again");
    const int was = qmk_set_batch_persistent(0);
    expect(qmk_decode_batch(QMK_MODEL_QWEN3_0_6B, 2, d, d + 16, tok, logits, embed, table.data(), fnorm, embed, cos_t,
                            sin_t, kc, vc, stride, kLayers, kSeq, 64, scale, ws, ws_bytes, s1) == QMK_OK,
           "decode_batch 2, multi-launch");
    qmk_set_batch_persistent(was);
    expect(qmk_decode_batch(QMK_MODEL_QWEN3_0_6B, 16, d, d + 16, tok, logits, embed, table.data(), fnorm, embed, cos_t,
                            sin_t, kc, vc, stride, kLayers, kSeq, 64, scale, ws, ws_bytes, s1) == QMK_OK,
           "decode_batch 16");
  }

  // the row sampler over the batched logits
  {
    long long* ctr = static_cast<long long*>(b.get(16 * 8, 0));
    expect(qmk_sample_rows(logits, 4, kV, 0.7f, 50, 0.9f, 3, ctr, tok, s1) == QMK_OK, "sample_rows");
  }

  // tracing, a second stream, graph launches off, the bounded-wait failure and its reset
  {
    const size_t n = qmk_trace_entries(28);  // set_trace takes buffers sized for the deepest model
    uint64_t* tr = static_cast<uint64_t*>(b.get(n * 8, 0));
    expect(qmk_set_trace(s1, tr, n) == QMK_OK, "set_trace");
    expect(qmk_decode_model(QMK_MODEL_QWEN3_0_6B, 11, tok, nullptr, embed, dtable, fnorm, embed, cos_t, sin_t, kc, vc,
                            hidden, normed, kLayers, 8, kSeq, scale, s1) == QMK_OK,
           "traced decode");
    expect(qmk_set_trace(s1, nullptr, 0) == QMK_OK, "trace off");
    expect(qmk_set_graph_launch(s2, 0) == QMK_OK, "graph launch off");
    expect(qmk_generate_model(QMK_MODEL_QWEN3_0_6B, 15, 40, embed, dtable, fnorm, embed, cos_t, sin_t, kc, vc, hidden,
                              normed, log, kLayers, 60, kSeq, scale, s2) == QMK_OK,
           "generate on a second stream");
    expect(hipStreamSynchronize(s1) == hipSuccess && hipStreamSynchronize(s2) == hipSuccess, "synchronize");
    expect(qmk_device_error(s1) == 0 && qmk_device_error(s2) == 0, "no device error");
    expect(qmk_set_wait_limit(s2, 1) == QMK_OK, "wait limit 1 tick");
    expect(qmk_decode_model(QMK_MODEL_QWEN3_0_6B, 11, tok, nullptr, embed, dtable, fnorm, embed, cos_t, sin_t, kc, vc,
                            hidden, normed, kLayers, 8, kSeq, scale, s2) == QMK_OK,
           "decode with a one-tick wait bound");
    expect(hipStreamSynchronize(s2) == hipSuccess, "synchronize after the forced failure");
    expect((qmk_device_error(s2) & QMK_DEV_TIMEOUT) != 0, "the one-tick wait expired");
    expect(qmk_set_wait_limit(s2, 0) == QMK_OK && qmk_reset(s2) == QMK_OK, "reset");
    expect(qmk_decode_model(QMK_MODEL_QWEN3_0_6B, 11, tok, nullptr, embed, dtable, fnorm, embed, cos_t, sin_t, kc, vc,
                            hidden, normed, kLayers, 8, kSeq, scale, s2) == QMK_OK,
           "decode after reset");
    expect(hipStreamSynchronize(s2) == hipSuccess && qmk_device_error(s2) == 0, "no device error after reset");
  }
  expect(hipDeviceSynchronize() == hipSuccess, "device synchronize");
  (void)hipStreamDestroy(s1);
  (void)hipStreamDestroy(s2);
}

}  // namespace

int main() {
  host_argument_checks();
  int n = 0;
  const bool gpu = hipGetDeviceCount(&n) == hipSuccess && n > 0;
  if (gpu) gpu_paths();
  std::printf("%s: %d failed checks\n", gpu ? "host argument checks and GPU paths" : "host argument checks (no GPU)",
              g_fail);
  return g_fail == 0 ? 0 : 1;
}
