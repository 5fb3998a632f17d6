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

struct SampleParams {
  float temperature;  // <= 0: greedy (first index of the maximum)
  int top_k;          // keep scores >= the top_k-th largest; <= 0 or >= vocab: off
  float top_p;        // keep the highest scores whose mass above them is < top_p; outside (0, 1): off
  uint64_t seed;
};

// Persistent-mode sampler of the generate loop: when the decode step just run
// produced `logits`, replace its greedy token in the state and the log by a
// sampled one (counter = the step's position) and set `done` for the stop token.
int launch_sample_state(const float* logits, int vocab, const SampleParams& sp, DecodeState* st, int* log,
                        hipStream_t stream);

}  // namespace qmk
