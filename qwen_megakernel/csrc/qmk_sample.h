// Sampling from logits rows: temperature, top-k, top-p (HF's logits warpers,
// transformers generation/logits_process.py TemperatureLogitsWarper,
// TopKLogitsWarper, TopPLogitsWarper), then one draw from the softmax of the
// kept scores by the Gumbel-max method.  Declarations shared by the C ABI
// (qmk_api.hip) and the kernels (qmk_sample.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "qmk_state.h"

namespace qmk {

// SplitMix64 finaliser with its golden-ratio increment (G. Steele, D. Lea,
// C. Flood, "Fast splittable pseudorandom number generators", OOPSLA 2014).
__device__ __forceinline__ uint64_t mix64(uint64_t z) {
  z += 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

// Per-draw base of the random numbers: (seed, counter).
__device__ __forceinline__ uint64_t draw_base(uint64_t seed, uint64_t counter) { return mix64(seed ^ mix64(counter)); }

// U in (0, 1) for token v: the top 24 bits of the hash, centred in their interval.
__device__ __forceinline__ float draw_uniform(uint64_t base, int v) {
  const uint64_t h = mix64(base + (uint64_t)(uint32_t)v);
  return ((float)(uint32_t)(h >> 40) + 0.5f) * (1.0f / 16777216.0f);
}

// Order-preserving uint32 key of a float.
__device__ __forceinline__ uint32_t key32(float f) {
  const uint32_t u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// Key of token v's Gumbel-perturbed score: key32(logit / T + G), G = -log(-log(U)).
__device__ __forceinline__ uint32_t gumbel_key(float logit, float temperature, uint64_t base, int v) {
  const float s = __fdiv_rn(logit, temperature);
  return key32(s + -logf(-logf(draw_uniform(base, v))));
}

struct SampleParams {
  float temperature;  // <= 0: greedy (first index of the maximum)
  int top_k;          // keep scores >= the top_k-th largest; <= 0 or >= vocab: off
  float top_p;        // keep the highest scores whose mass above them is < top_p; outside (0, 1): off
  uint64_t seed;
};

// Device work of one logits row between the launches of a sampling call: the
// row's radix histogram (counts or fixed-point masses) and selection state.
// Zero between calls: the call's last launch clears it.
struct SampleWork {
  unsigned long long hist[256];  // bins of the current 8-bit radix digit
  unsigned long long z, target, need, best;  // need: top-k rank still sought / top-p mass above the prefix
  unsigned int maxkey, prefix, mask, kmin, pmin, ticket;
};
constexpr int kSampleRowsMax = 256;  // rows per launch sequence of qmk_sample_rows

// hipMalloc + zero fill of `rows` work blocks.
int alloc_sample_work(SampleWork** out, int rows);

// Persistent-mode sampler of the generate loop: when the decode step just run
// produced `logits`, replace its greedy token in the state and the log by a
// sampled one (counter = the step's position) and set `done` for the stop token.
// `work`: one zeroed SampleWork owned by the caller's stream.
int launch_sample_state(const float* logits, int vocab, const SampleParams& sp, DecodeState* st, int* log,
                        SampleWork* work, hipStream_t stream);

}  // namespace qmk
