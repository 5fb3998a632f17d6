// Sampling kernels: one workgroup of 1024 threads per logits row.
//
//   s_v = logit_v / T                       (HF TemperatureLogitsWarper, fp32 divide)
//   top-k: keep s_v >= the k-th largest s   (HF TopKLogitsWarper: ties at the k-th value kept)
//   top-p: keep v iff the probability mass of the kept scores strictly above s_v is < p
//          (HF TopPLogitsWarper removes sorted tokens whose ascending cumulative
//          probability is <= 1 - p; at least the top token stays)
//   draw:  argmax over kept v of s_v + G_v, G_v = -log(-log(U_v)) (Gumbel-max: a draw
//          from softmax of the kept s), U_v from a counter-based hash of (seed, counter, v)
//
// Both thresholds are found by radix descent over the order-preserving 32-bit
// key of s, 8 bits per pass: top-k over integer counts, top-p over
// probability masses held as 2^-40 fixed-point integers (exp(s_v - max)
// rounded once), so every sum is an integer sum and the result does not depend
// on thread order.  The random numbers use SplitMix64 (G. Steele, D. Lea,
// C. Flood, "Fast splittable pseudorandom number generators", OOPSLA 2014).

#include <hip/hip_runtime.h>

#include "../../include/qwen_megakernel.h"
#include "qmk_device.h"
#include "qmk_sample.h"

namespace qmk {
namespace sample {

constexpr int kThreads = 1024;
constexpr int kWaves = kThreads / 64;
constexpr double kFix = 1099511627776.0;  // 2^40

__device__ __forceinline__ uint64_t wave_sum_u64(uint64_t v) {
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

struct Shared {
  unsigned long long hist[256];
  unsigned long long red[kWaves];
  float redf[kWaves];
  uint32_t digit;
  unsigned long long carry;
};

__device__ float block_max(float v, Shared& sh) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  v = wave_max(v);
  __syncthreads();
  if (lane == 0) sh.redf[wave] = v;
  __syncthreads();
  float m = sh.redf[0];
  for (int i = 1; i < kWaves; i++) m = fmaxf(m, sh.redf[i]);
  return m;
}

__device__ unsigned long long block_sum_u64(unsigned long long v, Shared& sh) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  v = wave_sum_u64(v);
  __syncthreads();
  if (lane == 0) sh.red[wave] = v;
  __syncthreads();
  unsigned long long s = 0;
  for (int i = 0; i < kWaves; i++) s += sh.red[i];
  return s;
}

__device__ unsigned long long block_max_u64(unsigned long long v, Shared& sh) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  v = wave_max_u64(v);
  __syncthreads();
  if (lane == 0) sh.red[wave] = v;
  __syncthreads();
  unsigned long long m = 0;
  for (int i = 0; i < kWaves; i++) m = sh.red[i] > m ? sh.red[i] : m;
  return m;
}

// Token of one row (every thread returns it).
__device__ int sample_row(const float* x, int V, const SampleParams& sp, uint64_t counter, Shared& sh) {
  const float T = sp.temperature;
  if (!(T > 0.f)) {
    unsigned long long best = 0;
    for (int v = threadIdx.x; v < V; v += kThreads) {
      const unsigned long long k = ((unsigned long long)key32(x[v]) << 32) | (0xffffffffu - (uint32_t)v);
      best = k > best ? k : best;
    }
    return (int)(0xffffffffu - (uint32_t)block_max_u64(best, sh));
  }
  auto score = [&](int v) { return __fdiv_rn(x[v], T); };

  // ---- top-k: key of the k-th largest score
  uint32_t kmin = 0;
  if (sp.top_k > 0 && sp.top_k < V) {
    uint32_t prefix = 0, mask = 0;
    unsigned long long remaining = (unsigned long long)sp.top_k;
    for (int shift = 24; shift >= 0; shift -= 8) {
      for (int i = threadIdx.x; i < 256; i += kThreads) sh.hist[i] = 0;
      __syncthreads();
      for (int v = threadIdx.x; v < V; v += kThreads) {
        const uint32_t k = key32(score(v));
        if ((k & mask) == prefix) atomicAdd(&sh.hist[(k >> shift) & 255u], 1ull);
      }
      __syncthreads();
      if (threadIdx.x == 0) {
        unsigned long long cum = 0;
        int d = 255;
        for (; d > 0; d--) {
          if (cum + sh.hist[d] >= remaining) break;
          cum += sh.hist[d];
        }
        sh.digit = (uint32_t)d;
        sh.carry = cum;
      }
      __syncthreads();
      prefix |= sh.digit << shift;
      mask |= 255u << shift;
      remaining -= sh.carry;
      __syncthreads();
    }
    kmin = prefix;
  }

  // ---- masses of the kept scores (fixed point), their sum Z
  float mx = -INFINITY;
  for (int v = threadIdx.x; v < V; v += kThreads) mx = fmaxf(mx, score(v));
  mx = block_max(mx, sh);
  auto mass = [&](float s) { return (unsigned long long)((double)expf(s - mx) * kFix + 0.5); };

  // ---- top-p: smallest key whose mass strictly above is < p * Z
  uint32_t pmin = 0;
  if (sp.top_p > 0.f && sp.top_p < 1.f) {
    unsigned long long z = 0;
    for (int v = threadIdx.x; v < V; v += kThreads) {
      const float s = score(v);
      if (key32(s) >= kmin) z += mass(s);
    }
    z = block_sum_u64(z, sh);
    unsigned long long target = (unsigned long long)((double)sp.top_p * (double)z);
    if (target < 1) target = 1;
    uint32_t prefix = 0, mask = 0;
    unsigned long long above = 0;
    for (int shift = 24; shift >= 0; shift -= 8) {
      for (int i = threadIdx.x; i < 256; i += kThreads) sh.hist[i] = 0;
      __syncthreads();
      for (int v = threadIdx.x; v < V; v += kThreads) {
        const float s = score(v);
        const uint32_t k = key32(s);
        if (k >= kmin && (k & mask) == prefix) atomicAdd(&sh.hist[(k >> shift) & 255u], mass(s));
      }
      __syncthreads();
      if (threadIdx.x == 0) {
        unsigned long long a = above;
        int d = 255;
        for (; d > 0; d--) {
          if (a + sh.hist[d] >= target) break;
          a += sh.hist[d];
        }
        sh.digit = (uint32_t)d;
        sh.carry = a;
      }
      __syncthreads();
      prefix |= sh.digit << shift;
      mask |= 255u << shift;
      above = sh.carry;
      __syncthreads();
    }
    pmin = prefix;
  }

  // ---- Gumbel-max draw over the kept scores
  const uint32_t kkeep = kmin > pmin ? kmin : pmin;
  const uint64_t base = draw_base(sp.seed, counter);
  unsigned long long best = 0;
  for (int v = threadIdx.x; v < V; v += kThreads) {
    if (key32(score(v)) < kkeep) continue;
    const unsigned long long k = ((unsigned long long)gumbel_key(x[v], T, base, v) << 32) |
                                 (0xffffffffu - (uint32_t)v);
    best = k > best ? k : best;
  }
  return (int)(0xffffffffu - (uint32_t)block_max_u64(best, sh));
}

__global__ void __launch_bounds__(kThreads) sample_rows(const float* __restrict__ logits, int V, SampleParams sp,
                                                        const long long* __restrict__ counters,
                                                        int* __restrict__ out) {
  __shared__ Shared sh;
  const int r = blockIdx.x;
  const int tok = sample_row(logits + (size_t)r * V, V, sp, (uint64_t)counters[r], sh);
  if (threadIdx.x == 0) out[r] = tok;
}

// After a persistent decode step: `ran` says whether the step ran (a step
// after the stop token only pads the log); if so its greedy token in the state
// and the log is replaced by the sampled one.
__global__ void __launch_bounds__(kThreads) sample_state(const float* __restrict__ logits, int V, SampleParams sp,
                                                         DecodeState* st, int* log) {
  __shared__ Shared sh;
  __shared__ int run;
  __shared__ long long counter;
  if (threadIdx.x == 0) {
    run = st->ran != 0 && st->err == 0;
    counter = (long long)st->pos - 1;  // position of the step just run
  }
  __syncthreads();
  if (!run) return;
  const int tok = sample_row(logits, V, sp, (uint64_t)counter, sh);
  if (threadIdx.x == 0) {
    st->tok = tok;
    if (log) log[st->step - 1] = tok;
    st->done = (st->eos >= 0 && tok == st->eos) ? 1u : 0u;
  }
}

}  // namespace sample

int launch_sample_state(const float* logits, int vocab, const SampleParams& sp, DecodeState* st, int* log,
                        hipStream_t stream) {
  hipLaunchKernelGGL(sample::sample_state, dim3(1), dim3(sample::kThreads), 0, stream, logits, vocab, sp, st, log);
  return hipGetLastError() == hipSuccess ? QMK_OK : QMK_ERR_HIP;
}

}  // namespace qmk

using namespace qmk;

extern "C" int qmk_sample_rows(const float* logits, int rows, int vocab, float temperature, int top_k, float top_p,
                               unsigned long long seed, const long long* counters, int* out_tokens,
                               hipStream_t stream) {
  if (!logits || !counters || !out_tokens || rows < 1 || rows > 65535 || vocab < 1) return QMK_ERR_ARG;
  if (!(top_p == top_p) || !(temperature == temperature)) return QMK_ERR_ARG;  // NaN
  const SampleParams sp{temperature, top_k, top_p, (uint64_t)seed};
  hipLaunchKernelGGL(sample::sample_rows, dim3(rows), dim3(sample::kThreads), 0, stream, logits, vocab, sp, counters,
                     out_tokens);
  return hipGetLastError() == hipSuccess ? QMK_OK : QMK_ERR_HIP;
}
