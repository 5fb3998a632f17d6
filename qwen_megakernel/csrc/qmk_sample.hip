// Sampling kernels.  Each logits row is spread over G workgroups of 256
// threads (G from 8 to 128, so that a single row fills many CUs); the passes
// are separate launches and no workgroup ever waits for another.
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
// rounded once).  Every workgroup histograms its slice of the row in LDS and
// adds its non-zero bins to the row's histogram with integer atomics; the last
// workgroup of the pass (a ticket counter) picks the digit and prepares the
// next pass.  Integer sums and integer maxima do not depend on the order of
// the atomics, so results are deterministic.  The random numbers use
// SplitMix64 (G. Steele, D. Lea, C. Flood, "Fast splittable pseudorandom
// number generators", OOPSLA 2014).
//
// Launches per sampling call: greedy or temperature only, 1 (the draw); top-k,
// 4 + 1; top-p, 1 (the maximum score) + 4 (the first also sums the mass) + 1;
// both, 10.  In the generate loop the maximum is the decode step's own greedy
// logit over T, which saves the first launch.  (Three passes of 11 bits were
// slower: 2048-bin histograms cost more per pass than the launch they save.)

#include <hip/hip_runtime.h>

#include "../../include/qwen_megakernel.h"
#include "qmk_device.h"
#include "qmk_sample.h"

#include <map>
#include <mutex>
#include <utility>

namespace qmk {
namespace sample {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr double kFix = 1099511627776.0;  // 2^40
constexpr int kPasses = 4;
constexpr int kBins = 256;  // 8-bit digits

struct Args {
  const float* logits;
  int V;
  SampleParams sp;
  const long long* counters;  // rows mode: per-row counters, out: per-row tokens
  int* out;
  DecodeState* st;            // state mode (one row): counter = st->pos - 1; the token replaces st->tok
  int* log;
  SampleWork* work;           // one per row, zero between calls
};

__device__ __forceinline__ float from_key32(uint32_t k) {
  return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

__device__ __forceinline__ unsigned long long mass_of(float s, float mx) {
  return (unsigned long long)((double)expf(s - mx) * kFix + 0.5);
}

struct Block {
  int row;
  const float* x;
  int v0, v1;           // this workgroup's slice of the row
  uint64_t counter;
  SampleWork* w;
  uint32_t greedy_tok;  // state mode: the decode step's greedy token (its logit is the row maximum)
};

// Common prologue: the row and slice of this workgroup; false when the call
// has nothing to do (state mode after a step that only padded the log).
__device__ bool setup(const Args& a, Block& b) {
  __shared__ int run, tok;
  __shared__ long long ctr;
  b.row = blockIdx.y;
  if (threadIdx.x == 0) {
    if (a.st) {
      run = a.st->ran != 0 && a.st->err == 0;
      ctr = (long long)a.st->pos - 1;  // position of the step just run
      tok = a.st->tok;
      if (tok < 0 || tok >= a.V) run = 0;
    } else {
      run = 1;
      ctr = a.counters ? a.counters[b.row] : 0;
    }
  }
  __syncthreads();
  const int chunk = (a.V + gridDim.x - 1) / gridDim.x;
  b.x = a.logits + (size_t)b.row * a.V;
  b.v0 = min(a.V, (int)blockIdx.x * chunk);
  b.v1 = min(a.V, b.v0 + chunk);
  b.counter = (uint64_t)ctr;
  b.w = a.work + b.row;
  b.greedy_tok = a.st ? (uint32_t)tok : 0u;
  return run != 0;
}

template <class F>
__device__ unsigned long long block_reduce_u64(unsigned long long v, F&& op) {
  __shared__ unsigned long long red[kWaves];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  for (int o = 32; o >= 1; o >>= 1) v = op(v, (unsigned long long)__shfl_xor(v, o));
  if (lane == 0) red[wave] = v;
  __syncthreads();
  v = red[0];
  for (int i = 1; i < kWaves; i++) v = op(v, red[i]);
  return v;
}

// True in every thread of the last workgroup of this pass to finish; the
// other workgroups' atomics are then visible to it.  Each thread waits until
// its device-scope atomics are acknowledged before the ticket is taken, and
// the last workgroup reads the results with agent-scope atomic loads; no
// fence, which on this part would write back the L2.
__device__ bool last_block(SampleWork* w) {
  __shared__ int last;
  wait_vmcnt(0);
  __syncthreads();
  if (threadIdx.x == 0) last = atomicAdd(&w->ticket, 1u) == gridDim.x - 1;
  __syncthreads();
  return last != 0;
}

__device__ __forceinline__ unsigned long long load_u64(const unsigned long long* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ unsigned int load_u32(const unsigned int* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Maximum key of s over the row (for the masses).
__global__ void __launch_bounds__(kThreads) k_max(Args a) {
  Block b;
  if (!setup(a, b)) return;
  const float T = a.sp.temperature;
  unsigned long long m = 0;
  for (int v = b.v0 + threadIdx.x; v < b.v1; v += kThreads) {
    const unsigned long long k = key32(__fdiv_rn(b.x[v], T));
    m = k > m ? k : m;
  }
  m = block_reduce_u64(m, [](unsigned long long p, unsigned long long q) { return p > q ? p : q; });
  if (threadIdx.x == 0) atomicMax(&b.w->maxkey, (unsigned int)m);
}

// The maximum score: the decode step's greedy logit over T (state mode), else
// the k_max result.
__device__ __forceinline__ float row_max(const Args& a, const Block& b) {
  return a.st ? __fdiv_rn(b.x[b.greedy_tok], a.sp.temperature) : from_key32(load_u32(&b.w->maxkey));
}

// One radix pass of the top-k (MASS = false: counts) or top-p (MASS = true:
// fixed-point masses of the scores >= kmin) threshold.  The first top-p pass
// also sums the mass Z of the scores >= kmin and sets the target max(1, p Z).
template <bool MASS>
__global__ void __launch_bounds__(kThreads) k_hist(Args a, int pass) {
  __shared__ unsigned long long wh[kWaves][kBins];
  __shared__ unsigned long long hs[kBins];
  __shared__ unsigned int ndig;
  Block b;
  if (!setup(a, b)) return;
  const int shift = 24 - 8 * pass;
  constexpr int nb = kBins;
  const float T = a.sp.temperature;
  SampleWork* w = b.w;
  const uint32_t prefix = load_u32(&w->prefix), mask = load_u32(&w->mask);
  const uint32_t kmin = MASS ? load_u32(&w->kmin) : 0u;
  const float mx = MASS ? row_max(a, b) : 0.f;
  const bool zsum = MASS && pass == 0;
  const int wave = threadIdx.x >> 6;
  for (int i = threadIdx.x; i < kWaves * kBins; i += kThreads) (&wh[0][0])[i] = 0;
  __syncthreads();
  unsigned long long z = 0;
  for (int v = b.v0 + threadIdx.x; v < b.v1; v += kThreads) {
    const float s = __fdiv_rn(b.x[v], T);
    const uint32_t k = key32(s);
    if (k < kmin) continue;
    const unsigned long long m = MASS ? mass_of(s, mx) : 1ull;
    if (zsum) z += m;
    if ((k & mask) == prefix) atomicAdd(&wh[wave][(k >> shift) & (uint32_t)(nb - 1)], m);
  }
  __syncthreads();
  for (int t = threadIdx.x; t < nb; t += kThreads) {
    unsigned long long h = 0;
    for (int q = 0; q < kWaves; q++) h += wh[q][t];
    if (h) atomicAdd(&w->hist[t], h);
  }
  if (zsum) {
    z = block_reduce_u64(z, [](unsigned long long p, unsigned long long q) { return p + q; });
    if (threadIdx.x == 0 && z) atomicAdd(&w->z, z);
  }
  if (!last_block(w)) return;

  // The last workgroup: suffix sums S[d] = sum of bins >= d, then the digit d,
  // the largest in [1, nb) with (mass above +) S[d] >= what is sought, else 0
  // (S is non-increasing, so d is the count of such d).
  for (int t = threadIdx.x; t < nb; t += kThreads) hs[t] = load_u64(&w->hist[t]);
  if (threadIdx.x == 0) ndig = 0;
  __syncthreads();
  for (int off = 1; off < nb; off <<= 1) {
    unsigned long long add[kBins / kThreads];
#pragma unroll
    for (int i = 0; i < kBins / kThreads; i++) {
      const int t = threadIdx.x + i * kThreads;
      add[i] = t < nb && t + off < nb ? hs[t + off] : 0ull;
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < kBins / kThreads; i++) {
      const int t = threadIdx.x + i * kThreads;
      if (t < nb) hs[t] += add[i];
    }
    __syncthreads();
  }
  unsigned long long target = 0;
  if (MASS) {
    if (zsum) {
      target = (unsigned long long)((double)a.sp.top_p * (double)load_u64(&w->z));
      if (target < 1) target = 1;
    } else {
      target = load_u64(&w->target);
    }
  }
  // top-k: `need` is the rank still sought (k at pass 0); top-p: the mass above the prefix
  const unsigned long long need = pass == 0 ? (MASS ? 0ull : (unsigned long long)a.sp.top_k) : load_u64(&w->need);
  for (int t = threadIdx.x; t < nb; t += kThreads) {
    const bool ok = t >= 1 && (MASS ? need + hs[t] >= target : hs[t] >= need);
    const unsigned long long bal = __ballot(ok);
    if ((threadIdx.x & 63) == 0 && bal) atomicAdd(&ndig, (unsigned int)__popcll(bal));
    w->hist[t] = 0;  // ready for the next pass
  }
  __syncthreads();
  const uint32_t d = ndig;
  if (threadIdx.x == 0) {
    const unsigned long long above = (int)d < nb - 1 ? hs[d + 1] : 0ull;
    const uint32_t np = prefix | (d << shift);
    if (zsum) w->target = target;
    if (pass < kPasses - 1) {
      w->prefix = np;
      w->mask = mask | ((uint32_t)(nb - 1) << shift);
      w->need = MASS ? need + above : need - above;
    } else {
      if (MASS) w->pmin = np;
      else w->kmin = np;
      w->prefix = 0;
      w->mask = 0;
      w->need = 0;
    }
    w->ticket = 0;
  }
}

// The draw (GREEDY: the first index of the maximum logit); the last workgroup
// writes the token and clears the row's work for the next call.
template <bool GREEDY>
__global__ void __launch_bounds__(kThreads) k_draw(Args a) {
  Block b;
  if (!setup(a, b)) return;
  SampleWork* w = b.w;
  const float T = a.sp.temperature;
  const uint32_t kmin = load_u32(&w->kmin), pmin = load_u32(&w->pmin);
  const uint32_t keep = kmin > pmin ? kmin : pmin;
  const uint64_t base = GREEDY ? 0 : draw_base(a.sp.seed, b.counter);
  unsigned long long best = 0;
  for (int v = b.v0 + threadIdx.x; v < b.v1; v += kThreads) {
    uint32_t k;
    if (GREEDY) {
      k = key32(b.x[v]);
    } else {
      if (key32(__fdiv_rn(b.x[v], T)) < keep) continue;
      k = gumbel_key(b.x[v], T, base, v);
    }
    const unsigned long long key = ((unsigned long long)k << 32) | (0xffffffffu - (uint32_t)v);
    best = key > best ? key : best;
  }
  best = block_reduce_u64(best, [](unsigned long long p, unsigned long long q) { return p > q ? p : q; });
  if (threadIdx.x == 0) atomicMax(&w->best, best);
  if (!last_block(w)) return;
  if (threadIdx.x == 0) {
    const int tok = (int)(0xffffffffu - (uint32_t)load_u64(&w->best));
    if (a.st) {
      DecodeState* st = a.st;
      st->tok = tok;
      if (a.log) a.log[st->step - 1] = tok;
      st->done = (st->eos >= 0 && tok == st->eos) ? 1u : 0u;
    } else {
      a.out[b.row] = tok;
    }
    w->z = w->target = w->need = w->best = 0;
    w->maxkey = w->prefix = w->mask = w->kmin = w->pmin = 0;
    w->ticket = 0;
  }
}

// Workgroups per row: about 128 workgroups in all, at least 8 per row.
int groups_for(int rows) {
  int g = 128;
  while (g > 8 && g * rows > 128) g >>= 1;
  return g;
}

int launch(const Args& a, int rows, hipStream_t stream) {
  const dim3 grid(groups_for(rows), rows), block(kThreads);
  const SampleParams& sp = a.sp;
  if (!(sp.temperature > 0.f)) {
    hipLaunchKernelGGL(k_draw<true>, grid, block, 0, stream, a);
  } else {
    const bool topk = sp.top_k > 0 && sp.top_k < a.V;
    const bool topp = sp.top_p > 0.f && sp.top_p < 1.f;
    if (topp && !a.st) hipLaunchKernelGGL(k_max, grid, block, 0, stream, a);
    if (topk)
      for (int p = 0; p < sample::kPasses; p++) hipLaunchKernelGGL(k_hist<false>, grid, block, 0, stream, a, p);
    if (topp)
      for (int p = 0; p < sample::kPasses; p++) hipLaunchKernelGGL(k_hist<true>, grid, block, 0, stream, a, p);
    hipLaunchKernelGGL(k_draw<false>, grid, block, 0, stream, a);
  }
  return hipGetLastError() == hipSuccess ? QMK_OK : QMK_ERR_HIP;
}

// Work of qmk_sample_rows per (device, stream), kSampleRowsMax rows, kept until
// the process ends: calls on one stream are ordered, so they may share it;
// calls on different streams may overlap, so they do not.
std::mutex g_mu;
std::map<std::pair<int, hipStream_t>, SampleWork*> g_work;

int stream_work(hipStream_t stream, SampleWork** out) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return QMK_ERR_HIP;
  std::lock_guard<std::mutex> lk(g_mu);
  auto it = g_work.find({dev, stream});
  if (it == g_work.end()) {
    SampleWork* w = nullptr;
    if (alloc_sample_work(&w, kSampleRowsMax) != QMK_OK) return QMK_ERR_HIP;
    it = g_work.emplace(std::make_pair(dev, stream), w).first;
  }
  *out = it->second;
  return QMK_OK;
}

}  // namespace sample

int alloc_sample_work(SampleWork** out, int rows) {
  const size_t bytes = (size_t)rows * sizeof(SampleWork);
  if (hipMalloc(out, bytes) != hipSuccess) return QMK_ERR_HIP;
  if (hipMemset(*out, 0, bytes) != hipSuccess) {
    (void)hipFree(*out);
    *out = nullptr;
    return QMK_ERR_HIP;
  }
  return QMK_OK;
}

int launch_sample_state(const float* logits, int vocab, const SampleParams& sp, DecodeState* st, int* log,
                        SampleWork* work, hipStream_t stream) {
  sample::Args a{logits, vocab, sp, nullptr, nullptr, st, log, work};
  return sample::launch(a, 1, stream);
}

}  // namespace qmk

using namespace qmk;

extern "C" int qmk_sample_rows(const float* logits, int rows, int vocab, float temperature, int top_k, float top_p,
                               unsigned long long seed, const long long* counters, int* out_tokens,
                               hipStream_t stream) {
  if (!logits || !counters || !out_tokens || rows < 1 || rows > 65535 || vocab < 1) return QMK_ERR_ARG;
  if (!(top_p == top_p) || !(temperature == temperature)) return QMK_ERR_ARG;  // NaN
  const SampleParams sp{temperature, top_k, top_p, (uint64_t)seed};
  SampleWork* work = nullptr;
  int s = sample::stream_work(stream, &work);
  if (s != QMK_OK) return s;
  for (int r0 = 0; r0 < rows && s == QMK_OK; r0 += kSampleRowsMax) {
    const int n = rows - r0 < kSampleRowsMax ? rows - r0 : kSampleRowsMax;
    sample::Args a{logits + (size_t)r0 * vocab, vocab, sp, counters + r0, out_tokens + r0, nullptr, nullptr, work};
    s = sample::launch(a, n, stream);
  }
  return s;
}
