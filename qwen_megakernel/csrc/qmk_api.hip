// Host side of libqwen_megakernel_amd.so: the C ABI declared in
// include/qwen_megakernel.h.
//
// The reference keeps barrier counters, flags and pinned ints in file-static
// singletons allocated on first use with unchecked cudaMalloc
// (csrc/kernel.cu:1446-1473), so two decoders on two streams corrupt each
// other.  Here each (device, stream) pair owns a DecodeState plus exchange
// buffers, created on first use and checked.  Launches on one stream are
// ordered by the stream.  Launches of the decode kernel on different streams
// of one device are ordered by the library (DeviceOrder below): the kernel
// needs all 256 workgroups resident at once, one per CU, and its workgroups
// wait on each other, so two overlapping instances could each hold part of
// the CUs and wait for workgroups that cannot start.

#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cstring>
#include <map>
#include <mutex>
#include <utility>
#include <vector>

#include "../../include/qwen_megakernel.h"
#include "qmk_batch_decode.h"
#include "qmk_decode_kernel.h"
#include "qmk_phase_bench.h"
#include "qmk_sample.h"

namespace qmk {
namespace {

using Model = Qwen3_0_6B;  // the reference's model; the shape the reference launchers serve
using Dm = Dims<Model>;
// One exchange area per stream serves every model.
constexpr uint32_t kXWords = Dims<Qwen3_0_6B>::X_WORDS > Dims<Qwen3_1_7B>::X_WORDS ? Dims<Qwen3_0_6B>::X_WORDS
                                                                                    : Dims<Qwen3_1_7B>::X_WORDS;

// The batched persistent kernel's exchange area (one per stream, allocated on
// its first use) serves every (model, batch size) it runs.
template <int B>
constexpr uint32_t bx_words_for() {
  return BDims<Qwen3_0_6B, B>::X_WORDS > BDims<Qwen3_1_7B, B>::X_WORDS ? BDims<Qwen3_0_6B, B>::X_WORDS
                                                                       : BDims<Qwen3_1_7B, B>::X_WORDS;
}
constexpr uint32_t kBXWords = bx_words_for<4>() > bx_words_for<3>()
                                  ? (bx_words_for<4>() > bx_words_for<2>() ? bx_words_for<4>() : bx_words_for<2>())
                                  : (bx_words_for<3>() > bx_words_for<2>() ? bx_words_for<3>() : bx_words_for<2>());

thread_local int t_status = QMK_OK;

// Scratch of the allocation-free entry point (qmk_decode_model_noalloc): one
// DecodeState header followed by one exchange area sized for the larger of the
// two models' layouts, 979,200 bytes.  Each GPU holds its own copy until the
// process ends.  Host code never uses this name as an address: qmk_init()
// takes the device address of the current device's copy with
// hipGetSymbolAddress and keeps it in that device's DevInfo.
constexpr size_t kScratchBytes = sizeof(DecodeState) + (size_t)kXWords * 4;
static __device__ __align__(256) uint32_t scratch[kScratchBytes / 4];

// generate: persistent launches recorded once into a HIP graph and replayed
// in groups of this many steps (the rest launched directly)
constexpr int kGraphSteps = 32;

struct DevInfo;

struct Ctx {
  int device = -1;
  DevInfo* dev = nullptr;
  uint32_t ticks_per_s = 100000000u;  // the device's wall-clock rate (the default wait bound is one second)
  int last_model = -1;                // model of the last launch on this stream's exchange area
  DecodeState* st = nullptr;
  uint32_t* x = nullptr;
  uint32_t* host_err = nullptr;
  int xcd_local = 0;
  uint32_t timeout = kTimeoutDefault;
  uint64_t* trace = nullptr;
  // persistent-mode token log (int[kMaxSeqLen]); the kernel always writes here, so the recorded
  // launch arguments do not depend on the caller's output tensor
  int* log = nullptr;
  bool use_graphs = true;
  hipStream_t cap = nullptr;      // private stream the graph is recorded on
  struct Graph {
    hipGraphExec_t exec = nullptr;
    KArgs args{};
    int model = -1;
    bool sampled = false;
    SampleParams sp{};
  } graphs[3];                    // by attention form (form_of): short, long, deep
  float* logits = nullptr;        // sampled generate: the step's logits (float[vocab])
  SampleWork* swork = nullptr;    // sampled generate: the sampler's work between its launches
  // batched persistent kernel: its own state header (epoch, error bits) and exchange area
  DecodeState* bst = nullptr;
  uint32_t* bx = nullptr;
  int last_bkind = -1;            // model * 8 + batch of the last batched launch on this stream
};

struct DevInfo {
  bool checked = false;  // set only once the checks ran to completion (a HIP failure leaves it unset)
  bool ok = false;
  int xcd_local = 0;
  uint32_t ticks_per_s = 100000000u;
  // cross-stream ordering of decode launches on this device
  std::mutex order_mu;
  hipEvent_t order_evt = nullptr;      // recorded after every group once order_multi is set
  hipStream_t order_stream = nullptr;  // the stream of the last decode launch group
  bool order_valid = false;
  bool order_multi = false;            // a second stream has launched on this device
  uint32_t* scratch = nullptr;         // this device's copy of `scratch` (set by qmk_init)
  uint32_t noalloc_timeout = 0;        // wait bound of qmk_decode_model_noalloc (0: one second)
  bool batch_ok = false;               // every batched persistent kernel fits one workgroup per CU
  // device copies of the layer tables the batched persistent kernel was called with (device_table)
  struct Table {
    std::vector<LayerPtrs> host;
    LayerPtrs* dev = nullptr;
  };
  std::mutex table_mu;
  std::vector<Table> tables;
};

constexpr size_t kMaxTables = 64;  // distinct batched layer tables kept per device

std::mutex g_mu;
std::map<std::pair<int, hipStream_t>, Ctx*> g_ctx;
std::map<int, DevInfo> g_dev;

// XCD probe results (one per workgroup), read back once per device; a static
// array, so the device check allocates no device memory.
__device__ int g_xcd_probe[kNumWG];

__global__ void xcd_probe_kernel(int* ok) {
  if (threadIdx.x == 0) {
    unsigned v;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(v));
    ok[blockIdx.x] = ((v & 0xfu) == (blockIdx.x & 7u)) ? 1 : 0;
  }
}

// Building blocks of the decode kernel on one wave, for unit tests:
// out[0,n) = bf16 rounding of in, out[n,2n) = softmax exp of in, then for the
// first 64 inputs (one per lane): sum over the four 16-lane rows, the two
// values of the row-pair swap and the two values of the half-wave swap.
__global__ void selftest_kernel(const float* in, float* out, int n) {
  const int lane = threadIdx.x;
  for (int i = lane; i < n; i += 64) {
    out[i] = bf16r(in[i]);
    out[n + i] = exp_acc(in[i]);
  }
  const float v = in[lane];
  float a, b;
  out[2 * n + lane] = rows_sum4(v);
  swap16(v, a, b);
  out[2 * n + 64 + lane] = a;
  out[2 * n + 128 + lane] = b;
  swap32(v, a, b);
  out[2 * n + 192 + lane] = a;
  out[2 * n + 256 + lane] = b;
}

__global__ void set_step_kernel(DecodeState* st, int pos, int tok, int eos) {
  st->pos = pos;
  st->tok = tok;
  st->step = 0;
  st->eos = eos;
  st->done = 0;
  st->ran = 0;
}

int fail(int s) {
  t_status = s;
  return s;
}

// Checks the current device: gfx950-class with >= 256 CUs, the decode kernel
// fits one workgroup per CU, and whether workgroup b runs on XCD b%8.  The
// result is kept only when every HIP call succeeded, so a transient failure
// leaves the device unchecked and the next call checks again.  The probe runs
// on a private stream (not the null stream, which another stream's graph
// capture would forbid).  Called with g_mu held.
int check_device(int dev, DevInfo** out) {
  DevInfo& di = g_dev[dev];
  *out = &di;
  if (di.checked) return di.ok ? QMK_OK : QMK_ERR_DEVICE;
  hipDeviceProp_t prop;
  if (hipGetDeviceProperties(&prop, dev) != hipSuccess) return QMK_ERR_HIP;
  int occ = 0, occ17 = 0;
  int occl = 0, occl17 = 0, occd = 0, occd17 = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, reinterpret_cast<const void*>(decode_kernel<Qwen3_0_6B, false>), kBlock,
                                                   0) != hipSuccess ||
      hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ17, reinterpret_cast<const void*>(decode_kernel<Qwen3_1_7B, false>), kBlock,
                                                   0) != hipSuccess ||
      hipOccupancyMaxActiveBlocksPerMultiprocessor(
          &occl, reinterpret_cast<const void*>(decode_kernel<Qwen3_0_6B, false, true>), kBlock, 0) != hipSuccess ||
      hipOccupancyMaxActiveBlocksPerMultiprocessor(
          &occl17, reinterpret_cast<const void*>(decode_kernel<Qwen3_1_7B, false, true>), kBlock, 0) != hipSuccess ||
      hipOccupancyMaxActiveBlocksPerMultiprocessor(
          &occd, reinterpret_cast<const void*>(decode_kernel_deep<Qwen3_0_6B, false>), kBlock, 0) != hipSuccess ||
      hipOccupancyMaxActiveBlocksPerMultiprocessor(
          &occd17, reinterpret_cast<const void*>(decode_kernel_deep<Qwen3_1_7B, false>), kBlock, 0) != hipSuccess)
    return QMK_ERR_HIP;
  if (prop.multiProcessorCount < kNumWG || occ < 1 || occ17 < 1 || occl < 1 || occl17 < 1 || occd < 1 ||
      occd17 < 1) {
    di.checked = true;
    di.ok = false;
    return QMK_ERR_DEVICE;
  }
  // the batched persistent kernels: without room for one workgroup per CU, qmk_decode_batch keeps
  // its multi-launch path
  bool batch_ok = true;
  {
    const std::pair<const void*, int> bk[] = {
        {reinterpret_cast<const void*>(batch_decode_kernel<Qwen3_0_6B, 2>), batch_block<2>()},
        {reinterpret_cast<const void*>(batch_decode_kernel<Qwen3_0_6B, 3>), batch_block<3>()},
        {reinterpret_cast<const void*>(batch_decode_kernel<Qwen3_0_6B, 4>), batch_block<4>()},
        {reinterpret_cast<const void*>(batch_decode_kernel<Qwen3_1_7B, 2>), batch_block<2>()},
        {reinterpret_cast<const void*>(batch_decode_kernel<Qwen3_1_7B, 3>), batch_block<3>()},
        {reinterpret_cast<const void*>(batch_decode_kernel<Qwen3_1_7B, 4>), batch_block<4>()}};
    for (const auto& k : bk) {
      int ob = 0;
      if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&ob, k.first, k.second, 0) != hipSuccess) return QMK_ERR_HIP;
      batch_ok = batch_ok && ob >= 1;
    }
  }
  uint32_t ticks = 100000000u;
  int khz = 0;
  if (hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, dev) == hipSuccess && khz > 0)
    ticks = (uint32_t)khz * 1000u;
  hipStream_t ps = nullptr;
  if (hipStreamCreateWithFlags(&ps, hipStreamNonBlocking) != hipSuccess) return QMK_ERR_HIP;
  int* d_ok = nullptr;
  int h_ok[kNumWG];
  bool good = hipGetSymbolAddress(reinterpret_cast<void**>(&d_ok), HIP_SYMBOL(g_xcd_probe)) == hipSuccess;
  if (good) {
    hipLaunchKernelGGL(xcd_probe_kernel, dim3(kNumWG), dim3(64), 0, ps, d_ok);
    good = hipGetLastError() == hipSuccess &&
           hipMemcpyAsync(h_ok, d_ok, sizeof(h_ok), hipMemcpyDeviceToHost, ps) == hipSuccess &&
           hipStreamSynchronize(ps) == hipSuccess;
  }
  (void)hipStreamDestroy(ps);
  if (!good) return QMK_ERR_HIP;
  if (!di.order_evt && hipEventCreateWithFlags(&di.order_evt, hipEventDisableTiming) != hipSuccess) return QMK_ERR_HIP;
  int all = 1;
  for (int i = 0; i < kNumWG; i++) all &= h_ok[i];
  di.xcd_local = all;
  di.batch_ok = batch_ok;
  di.ticks_per_s = ticks;
  di.ok = true;
  di.checked = true;
  return QMK_OK;
}

// Orders one group of decode launches on `stream` after the previous group on
// the same device, whatever stream that was on.  While a device sees one
// stream nothing is added (a marker after every launch costs 4 us between
// back-to-back kernels, measured).  When a second stream first launches, the
// device is synchronised once, and from then on an event is recorded after
// every group, on the stream that group used, and a group on another stream
// waits on it.  The lock keeps the check, the wait, the launches and the
// record of one group together against other host threads.  A stream under
// graph capture is left alone (the graph's owner orders its replays).
class DeviceOrder {
 public:
  DeviceOrder(DevInfo* di, hipStream_t stream) : di_(di), stream_(stream), lk_(di->order_mu) {
    capturing_ = capturing(stream);
    if (capturing_) return;
    if (di_->order_valid && di_->order_stream != stream) {
      if (!di_->order_multi) {
        ok_ = hipDeviceSynchronize() == hipSuccess;
        di_->order_multi = true;
      } else {
        ok_ = hipStreamWaitEvent(stream, di_->order_evt, 0) == hipSuccess;
      }
    }
    di_->order_stream = stream;
    di_->order_valid = true;
  }
  bool ok() const { return ok_; }
  // call once the group's launches are enqueued
  int finish() {
    if (capturing_ || !di_->order_multi) return QMK_OK;
    return hipEventRecord(di_->order_evt, stream_) == hipSuccess ? QMK_OK : QMK_ERR_HIP;
  }

 private:
  static bool capturing(hipStream_t s) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(s, &cs) != hipSuccess) {
      (void)hipGetLastError();
      return false;
    }
    return cs != hipStreamCaptureStatusNone;
  }
  DevInfo* di_;
  hipStream_t stream_;
  std::lock_guard<std::mutex> lk_;
  bool capturing_ = false;
  bool ok_ = true;
};

// Zeroes a stream's exchange words and restarts its tags (epoch 0), keeping
// the error word: run when the stream switches models, whose exchange layouts
// differ, so no word left by the other layout is ever read as current.
__global__ void clear_exchange_kernel(DecodeState* st, uint32_t* x, uint32_t n) {
  for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) x[i] = 0u;
  if (blockIdx.x == 0 && threadIdx.x == 0) st->epoch = 0u;
}

// Start of every qmk_decode_model_noalloc call, one workgroup: on the first
// call of a process (zeroed scratch) or when the model differs from the last
// call's, zero the exchange words and restart the tags; after a failed call
// (error bits set), move the tags past every tag that call could have written.
// Then clear the error bits, so one failure does not block later calls.
__global__ void noalloc_prepare_kernel(DecodeState* st, uint32_t* x, uint32_t n, uint32_t model_tag) {
  __shared__ int mode;
  if (threadIdx.x == 0) mode = st->reserved[0] != model_tag ? 2 : (st->err != 0 ? 1 : 0);
  __syncthreads();
  if (mode == 2)
    for (uint32_t i = threadIdx.x; i < n; i += blockDim.x) x[i] = 0u;
  if (threadIdx.x == 0) {
    if (mode == 2) {
      st->epoch = 0u;
      st->reserved[0] = model_tag;
    } else if (mode == 1) {
      st->epoch += 2u * 256u;  // a launch advances the tags by at most 9 * 28 + 1
    }
    st->err = 0u;
    st->done = 0u;
  }
}

int prepare_model(Ctx* ctx, int model, hipStream_t stream) {
  if (ctx->last_model == model) return QMK_OK;
  if (ctx->last_model >= 0) {
    hipLaunchKernelGGL(clear_exchange_kernel, dim3(kNumWG), dim3(256), 0, stream, ctx->st, ctx->x, kXWords);
    if (hipGetLastError() != hipSuccess) return QMK_ERR_HIP;
  }
  ctx->last_model = model;
  return QMK_OK;
}

int get_ctx(hipStream_t stream, Ctx** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess) return QMK_ERR_HIP;
  std::lock_guard<std::mutex> lk(g_mu);
  auto key = std::make_pair(dev, stream);
  auto it = g_ctx.find(key);
  if (it != g_ctx.end()) {
    *out = it->second;
    return QMK_OK;
  }
  DevInfo* di = nullptr;
  int s = check_device(dev, &di);
  if (s != QMK_OK) return s;
  Ctx* c = new Ctx();
  c->device = dev;
  c->dev = di;
  c->xcd_local = di->xcd_local;
  c->ticks_per_s = di->ticks_per_s;
  c->timeout = di->ticks_per_s;  // 1 second
  const size_t bytes = sizeof(DecodeState) + (size_t)kXWords * 4;
  void* mem = nullptr;
  if (hipMalloc(&mem, bytes) != hipSuccess) {
    delete c;
    return QMK_ERR_HIP;
  }
  if (hipMemset(mem, 0, bytes) != hipSuccess || hipHostMalloc(&c->host_err, sizeof(uint32_t), hipHostMallocDefault) != hipSuccess) {
    (void)hipFree(mem);
    delete c;
    return QMK_ERR_HIP;
  }
  *c->host_err = 0;
  if (hipMalloc(&c->log, (size_t)kMaxSeqLen * sizeof(int)) != hipSuccess) {
    (void)hipFree(mem);
    (void)hipHostFree(c->host_err);
    delete c;
    return QMK_ERR_HIP;
  }
  c->st = reinterpret_cast<DecodeState*>(mem);
  c->x = reinterpret_cast<uint32_t*>(reinterpret_cast<char*>(mem) + sizeof(DecodeState));
  g_ctx[key] = c;
  *out = c;
  return QMK_OK;
}

struct Common {
  int model;  // QMK_MODEL_*
  const void* embed;
  const LDGLayerWeights* layers;
  const void* final_norm;
  const void* lm_head;
  const void* cos_t;
  const void* sin_t;
  void* k_cache;
  void* v_cache;
  void* hidden_out;
  void* normalized_out;
  int num_layers;
  int max_seq_len;
  float attn_scale;
};

int validate(const Common& c) {
  if (!c.embed || !c.layers || !c.final_norm || !c.lm_head || !c.cos_t || !c.sin_t || !c.k_cache || !c.v_cache)
    return QMK_ERR_ARG;
  for (const void* p : {c.embed, (const void*)c.layers, c.final_norm, c.lm_head, c.cos_t, c.sin_t,
                        (const void*)c.k_cache, (const void*)c.v_cache})
    if (!aligned16(p)) return QMK_ERR_ARG;
  if (c.model != QMK_MODEL_QWEN3_0_6B && c.model != QMK_MODEL_QWEN3_1_7B) return QMK_ERR_ARG;
  if (c.num_layers < 1 || c.num_layers > 28 || c.max_seq_len < 1 || c.max_seq_len > kMaxSeqLen) return QMK_ERR_ARG;
  if (!(c.attn_scale > 0.f)) return QMK_ERR_ARG;
  return QMK_OK;
}

KArgs make_args(const Common& c, Ctx* ctx) {
  KArgs a{};
  a.embed = static_cast<const uint16_t*>(c.embed);
  a.layers = reinterpret_cast<const LayerPtrs*>(c.layers);
  a.final_norm = static_cast<const uint16_t*>(c.final_norm);
  a.lm_head = static_cast<const uint16_t*>(c.lm_head);
  a.cos_t = static_cast<const uint16_t*>(c.cos_t);
  a.sin_t = static_cast<const uint16_t*>(c.sin_t);
  a.k_cache = static_cast<uint16_t*>(c.k_cache);
  a.v_cache = static_cast<uint16_t*>(c.v_cache);
  a.hidden_out = static_cast<uint16_t*>(c.hidden_out);
  a.normalized_out = static_cast<float*>(c.normalized_out);
  a.st = ctx->st;
  a.x = ctx->x;
  a.host_err = ctx->host_err;
  a.num_layers = c.num_layers;
  a.max_seq_len = c.max_seq_len;
  a.attn_scale = c.attn_scale;
  a.rms_eps = 1e-6f;
  a.timeout = ctx->timeout;
  a.xcd_local = ctx->xcd_local;
  a.trace = ctx->trace;
  return a;
}

// The attention form of a step at context `ctx` (positions 0..ctx-1): 0 up to kLongContext,
// 1 up to kDeepContext, 2 beyond.
int form_of(long long ctx) { return ctx > kDeepContext ? 2 : ctx > kLongContext ? 1 : 0; }

template <class M>
void launch_model(const KArgs& a, int form, hipStream_t stream) {
  const bool t = a.temperature > 0.f;
  const dim3 g(kNumWG), k(kBlock);
  if (form == 2) {
    if (t) hipLaunchKernelGGL((decode_kernel_deep<M, true>), g, k, 0, stream, a);
    else hipLaunchKernelGGL((decode_kernel_deep<M, false>), g, k, 0, stream, a);
  } else if (form == 1) {
    if (t) hipLaunchKernelGGL((decode_kernel<M, true, true>), g, k, 0, stream, a);
    else hipLaunchKernelGGL((decode_kernel<M, false, true>), g, k, 0, stream, a);
  } else {
    if (t) hipLaunchKernelGGL((decode_kernel<M, true, false>), g, k, 0, stream, a);
    else hipLaunchKernelGGL((decode_kernel<M, false, false>), g, k, 0, stream, a);
  }
}

// One decode launch in attention form `form` (form_of the step's context).
int launch(const KArgs& a, int model, int form, hipStream_t stream) {
  if (model == QMK_MODEL_QWEN3_1_7B) launch_model<Qwen3_1_7B>(a, form, stream);
  else launch_model<Qwen3_0_6B>(a, form, stream);
  return hipGetLastError() == hipSuccess ? QMK_OK : QMK_ERR_HIP;
}

int poisoned(Ctx* ctx) { return (*ctx->host_err != 0) ? QMK_ERR_POISONED : QMK_OK; }

int decode_impl(const Common& c, int token, int position, int* out_token, float* logits, hipStream_t stream,
                bool persistent) {
  int s = validate(c);
  if (s != QMK_OK) return fail(s);
  if (position < 0 || position >= c.max_seq_len) return fail(QMK_ERR_POSITION);
  if (token < 0 || token >= Dm::V) return fail(QMK_ERR_ARG);
  Ctx* ctx = nullptr;
  if ((s = get_ctx(stream, &ctx)) != QMK_OK) return fail(s);
  if ((s = poisoned(ctx)) != QMK_OK) return fail(s);
  KArgs a = make_args(c, ctx);
  a.out_token = out_token;
  a.logits = logits;
  DeviceOrder order(ctx->dev, stream);
  if (!order.ok()) return fail(QMK_ERR_HIP);
  if ((s = prepare_model(ctx, c.model, stream)) != QMK_OK) return fail(s);
  if (persistent) {
    hipLaunchKernelGGL(set_step_kernel, dim3(1), dim3(1), 0, stream, ctx->st, position, token, -1);
    a.position = -1;
  } else {
    a.position = position;
    a.token = token;
  }
  s = launch(a, c.model, form_of(position + 1), stream);
  const int so = order.finish();
  return fail(s != QMK_OK ? s : so);
}

// One step of the generate loop: the decode launch, and with sampling the
// sampler that replaces its greedy token.
int launch_step(const KArgs& a, int model, const SampleParams* sp, SampleWork* sw, int form,
                hipStream_t stream) {
  int s = launch(a, model, form, stream);
  if (s == QMK_OK && sp) s = launch_sample_state(a.logits, Dims<Qwen3_0_6B>::V, *sp, a.st, a.out_log, sw, stream);
  return s;
}

// The instantiated graph of kGraphSteps steps with arguments `a` (and `sp`) in
// one attention form, recorded again when the arguments, the model or the
// sampling change.
int graph_for(Ctx* ctx, const KArgs& a, int model, const SampleParams* sp, int form, hipGraphExec_t* out) {
  const bool sampled = sp != nullptr;
  Ctx::Graph& gr = ctx->graphs[form];
  if (gr.exec && gr.model == model && std::memcmp(&gr.args, &a, sizeof(KArgs)) == 0 && gr.sampled == sampled &&
      (!sampled || std::memcmp(&gr.sp, sp, sizeof(SampleParams)) == 0)) {
    *out = gr.exec;
    return QMK_OK;
  }
  if (gr.exec) {
    (void)hipGraphExecDestroy(gr.exec);
    gr.exec = nullptr;
  }
  if (!ctx->cap && hipStreamCreateWithFlags(&ctx->cap, hipStreamNonBlocking) != hipSuccess) return QMK_ERR_HIP;
  if (hipStreamBeginCapture(ctx->cap, hipStreamCaptureModeThreadLocal) != hipSuccess) return QMK_ERR_HIP;
  int s = QMK_OK;
  for (int i = 0; i < kGraphSteps && s == QMK_OK; i++) s = launch_step(a, model, sp, ctx->swork, form, ctx->cap);
  hipGraph_t g = nullptr;
  const hipError_t e = hipStreamEndCapture(ctx->cap, &g);
  if (s != QMK_OK || e != hipSuccess || !g) {
    if (g) (void)hipGraphDestroy(g);
    return QMK_ERR_HIP;
  }
  hipGraphExec_t ex = nullptr;
  const hipError_t ie = hipGraphInstantiate(&ex, g, nullptr, nullptr, 0);
  (void)hipGraphDestroy(g);
  if (ie != hipSuccess) return QMK_ERR_HIP;
  gr.exec = ex;
  gr.args = a;
  gr.model = model;
  gr.sampled = sampled;
  if (sampled) gr.sp = *sp;
  *out = ex;
  return QMK_OK;
}

// The launches of generate_impl, in order on `stream`.
int generate_steps(Ctx* ctx, const Common& c, const KArgs& a, int first_token_id, int num_steps, int eos,
                   int* output_log, int start_position, hipStream_t stream, const SampleParams* sp) {
  int s = QMK_OK;
  hipLaunchKernelGGL(set_step_kernel, dim3(1), dim3(1), 0, stream, ctx->st, start_position, first_token_id,
                     eos < 0 ? -1 : eos);
  // Step i runs at context start_position + i + 1, in the attention form of that context
  // (form_of); each run of steps in one form replays that form's graph, with direct launches for
  // the remainder.
  for (int done = 0; done < num_steps;) {
    const long long ctx0 = (long long)start_position + done + 1;
    const int form = form_of(ctx0);
    int run = num_steps - done;
    if (form == 0) run = (int)std::min<long long>(run, kLongContext - ctx0 + 1);
    if (form == 1) run = (int)std::min<long long>(run, kDeepContext - ctx0 + 1);
    hipGraphExec_t g = nullptr;
    if (ctx->use_graphs && run >= kGraphSteps && graph_for(ctx, a, c.model, sp, form, &g) == QMK_OK) {
      for (; run >= kGraphSteps; run -= kGraphSteps, done += kGraphSteps)
        if (hipGraphLaunch(g, stream) != hipSuccess) return QMK_ERR_HIP;
    }
    for (; run > 0; run--, done++)
      if ((s = launch_step(a, c.model, sp, ctx->swork, form, stream)) != QMK_OK) return s;
  }
  if (hipMemcpyAsync(output_log, ctx->log, (size_t)num_steps * sizeof(int), hipMemcpyDeviceToDevice, stream) !=
      hipSuccess)
    return QMK_ERR_HIP;
  return QMK_OK;
}

// num_steps persistent launches from (start_position, first_token_id); the
// log is copied into output_log at the end.  eos >= 0: stop token.
int generate_impl(const Common& c, int first_token_id, int num_steps, int eos, int* output_log, int start_position,
                  hipStream_t stream, const SampleParams* sp = nullptr) {
  int s = validate(c);
  if (s != QMK_OK) return fail(s);
  if (num_steps < 0 || !output_log) return fail(QMK_ERR_ARG);
  if (num_steps == 0) return fail(QMK_OK);
  // every step must stay inside the cache: the last one runs at start+num_steps-1
  if (start_position < 0 || (long long)start_position + num_steps > (long long)c.max_seq_len)
    return fail(QMK_ERR_POSITION);
  if (first_token_id < 0 || first_token_id >= Dm::V || eos >= Dm::V) return fail(QMK_ERR_ARG);
  Ctx* ctx = nullptr;
  if ((s = get_ctx(stream, &ctx)) != QMK_OK) return fail(s);
  if ((s = poisoned(ctx)) != QMK_OK) return fail(s);
  KArgs a = make_args(c, ctx);
  a.position = -1;
  a.out_log = ctx->log;
  if (sp && sp->temperature > 0.f && sp->top_k <= 0 && !(sp->top_p > 0.f && sp->top_p < 1.f)) {
    // temperature only: the draw is the decode kernel's own LM-head argmax over perturbed scores
    a.temperature = sp->temperature;
    a.seed = sp->seed;
    sp = nullptr;
  }
  if (sp) {
    if (!ctx->logits && hipMalloc(&ctx->logits, (size_t)Dm::V * sizeof(float)) != hipSuccess) return fail(QMK_ERR_HIP);
    if (!ctx->swork && alloc_sample_work(&ctx->swork, 1) != QMK_OK) return fail(QMK_ERR_HIP);
    a.logits = ctx->logits;
  }
  DeviceOrder order(ctx->dev, stream);
  if (!order.ok()) return fail(QMK_ERR_HIP);
  if ((s = prepare_model(ctx, c.model, stream)) != QMK_OK) return fail(s);
  s = generate_steps(ctx, c, a, first_token_id, num_steps, eos, output_log, start_position, stream, sp);
  const int so = order.finish();
  return fail(s != QMK_OK ? s : so);
}

// ---------------------------------------------------------------- batched persistent step

std::atomic<int> g_batch_persistent{1};  // qmk_set_batch_persistent

template <class M>
int launch_batch(int batch, const BArgs& a, hipStream_t stream) {
  switch (batch) {
    case 2: hipLaunchKernelGGL((batch_decode_kernel<M, 2>), dim3(kNumWG), dim3(batch_block<2>()), 0, stream, a); break;
    case 3: hipLaunchKernelGGL((batch_decode_kernel<M, 3>), dim3(kNumWG), dim3(batch_block<3>()), 0, stream, a); break;
    default: hipLaunchKernelGGL((batch_decode_kernel<M, 4>), dim3(kNumWG), dim3(batch_block<4>()), 0, stream, a); break;
  }
  return hipGetLastError() == hipSuccess ? QMK_OK : QMK_ERR_HIP;
}

// The device copy of a batched step's layer table (num_layers entries): uploaded once per distinct
// table with a synchronous copy into a new buffer, which no kernel reads yet, and kept until the
// process ends.  QMK_ERR_DEVICE (the caller takes the multi-launch path) where no copy can be made
// now: on a stream under capture, or with kMaxTables tables already kept.
int device_table(DevInfo* di, const LDGLayerWeights* host, int num_layers, hipStream_t stream,
                 const LayerPtrs** out) {
  static_assert(sizeof(LayerPtrs) == sizeof(LDGLayerWeights), "layer table layout");
  const size_t bytes = (size_t)num_layers * sizeof(LayerPtrs);
  std::lock_guard<std::mutex> lk(di->table_mu);
  for (const DevInfo::Table& t : di->tables)
    if ((int)t.host.size() == num_layers && std::memcmp(t.host.data(), host, bytes) == 0) {
      *out = t.dev;
      return QMK_OK;
    }
  if (di->tables.size() >= kMaxTables) return QMK_ERR_DEVICE;
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(stream, &cs) != hipSuccess) return QMK_ERR_HIP;
  if (cs != hipStreamCaptureStatusNone) return QMK_ERR_DEVICE;
  DevInfo::Table t;
  t.host.resize((size_t)num_layers);
  std::memcpy(t.host.data(), host, bytes);
  if (hipMalloc(&t.dev, bytes) != hipSuccess) return QMK_ERR_HIP;
  if (hipMemcpy(t.dev, t.host.data(), bytes, hipMemcpyHostToDevice) != hipSuccess) {
    (void)hipFree(t.dev);
    return QMK_ERR_HIP;
  }
  *out = t.dev;
  di->tables.push_back(std::move(t));
  return QMK_OK;
}

bool ranges_overlap(const void* a, size_t an, const void* b, size_t bn) {
  const char* pa = static_cast<const char*>(a);
  const char* pb = static_cast<const char*>(b);
  return pa < pb + bn && pb < pa + an;
}

int batch_persistent_impl(int model, int batch, const int* tokens, const int* positions, int* out_tokens,
                          float* logits_out, const void* embed_weight, const LDGLayerWeights* layer_weights_host,
                          const void* final_norm_weight, const void* lm_head_weight, const void* cos_table,
                          const void* sin_table, void* k_cache, void* v_cache, long long seq_stride, int num_layers,
                          int max_seq_len, int max_context, float attn_scale, hipStream_t stream) {
  if (model != QMK_MODEL_QWEN3_0_6B && model != QMK_MODEL_QWEN3_1_7B) return QMK_ERR_ARG;
  if (batch < kBatchMin || batch > kBatchMax || !tokens || !positions || !out_tokens || !embed_weight ||
      !layer_weights_host || !final_norm_weight || !lm_head_weight || !cos_table || !sin_table || !k_cache ||
      !v_cache || num_layers < 1 || num_layers > kMaxLayers || max_seq_len < 1 || max_seq_len > kMaxSeqLen ||
      max_context < 1 || max_context > max_seq_len || max_context > kBatchMaxContext || !(attn_scale > 0.f))
    return QMK_ERR_ARG;
  if (seq_stride < (long long)num_layers * Dm::NKV * max_seq_len * Dm::D || seq_stride % 8 != 0) return QMK_ERR_ARG;
  for (const void* q : {embed_weight, final_norm_weight, lm_head_weight, cos_table, sin_table, (const void*)k_cache,
                        (const void*)v_cache})
    if (!aligned16(q)) return QMK_ERR_ARG;
  // out_tokens is written (-1) at the start of the step, before every workgroup has read tokens
  if (ranges_overlap(tokens, batch * sizeof(int), out_tokens, batch * sizeof(int)) ||
      ranges_overlap(positions, batch * sizeof(int), out_tokens, batch * sizeof(int)))
    return QMK_ERR_ARG;
  BArgs a{};
  for (int L = 0; L < num_layers; L++) {
    const LDGLayerWeights& w = layer_weights_host[L];
    const void* p[11] = {w.input_layernorm_weight, w.q_proj_weight, w.k_proj_weight, w.v_proj_weight,
                         w.q_norm_weight, w.k_norm_weight, w.o_proj_weight, w.post_attn_layernorm_weight,
                         w.gate_proj_weight, w.up_proj_weight, w.down_proj_weight};
    for (const void* q : p)
      if (!q || !aligned16(q)) return QMK_ERR_ARG;
  }
  Ctx* ctx = nullptr;
  int s = get_ctx(stream, &ctx);
  if (s != QMK_OK) return s;
  if (!ctx->dev->batch_ok) return QMK_ERR_DEVICE;
  if ((s = poisoned(ctx)) != QMK_OK) return s;
  if ((s = device_table(ctx->dev, layer_weights_host, num_layers, stream, &a.layers)) != QMK_OK) return s;
  if (!ctx->bx) {
    const size_t bytes = sizeof(DecodeState) + (size_t)kBXWords * 4;
    void* mem = nullptr;
    if (hipMalloc(&mem, bytes) != hipSuccess) return QMK_ERR_HIP;
    if (hipMemset(mem, 0, bytes) != hipSuccess) {
      (void)hipFree(mem);
      return QMK_ERR_HIP;
    }
    ctx->bst = reinterpret_cast<DecodeState*>(mem);
    ctx->bx = reinterpret_cast<uint32_t*>(reinterpret_cast<char*>(mem) + sizeof(DecodeState));
  }
  a.embed = static_cast<const uint16_t*>(embed_weight);
  a.final_norm = static_cast<const uint16_t*>(final_norm_weight);
  a.lm_head = static_cast<const uint16_t*>(lm_head_weight);
  a.cos_t = static_cast<const uint16_t*>(cos_table);
  a.sin_t = static_cast<const uint16_t*>(sin_table);
  a.k_cache = static_cast<uint16_t*>(k_cache);
  a.v_cache = static_cast<uint16_t*>(v_cache);
  a.seq_stride = seq_stride;
  a.tokens = tokens;
  a.positions = positions;
  a.out_tokens = out_tokens;
  a.logits = logits_out;
  a.st = ctx->bst;
  a.x = ctx->bx;
  a.host_err = ctx->host_err;
  a.trace = ctx->trace;
  a.num_layers = num_layers;
  a.max_seq_len = max_seq_len;
  a.max_context = max_context;
  a.attn_scale = attn_scale;
  a.rms_eps = 1e-6f;
  a.timeout = ctx->timeout;
  a.xcd_local = ctx->xcd_local;
  DeviceOrder order(ctx->dev, stream);
  if (!order.ok()) return QMK_ERR_HIP;
  const int kind = model * 8 + batch;
  if (ctx->last_bkind >= 0 && ctx->last_bkind != kind) {
    // another layout's words must never be read as current: zero them and restart the tags
    hipLaunchKernelGGL(clear_exchange_kernel, dim3(kNumWG), dim3(256), 0, stream, ctx->bst, ctx->bx, kBXWords);
    if (hipGetLastError() != hipSuccess) return QMK_ERR_HIP;
  }
  ctx->last_bkind = kind;
  s = model == QMK_MODEL_QWEN3_1_7B ? launch_batch<Qwen3_1_7B>(batch, a, stream)
                                    : launch_batch<Qwen3_0_6B>(batch, a, stream);
  const int so = order.finish();
  return s != QMK_OK ? s : so;
}

size_t phase_copy_elems(int phase) {
  switch (phase) {
    case kPhaseQKV: return (size_t)(Dm::QS + 2 * Dm::NKV * Dm::D) * Dm::H;
    case kPhaseO: return (size_t)Dm::H * Dm::QS;
    case kPhaseGateUp: return (size_t)2 * Dm::I * Dm::H;
    case kPhaseDown: return (size_t)Dm::H * Dm::I;
    case kPhaseLmHead: return (size_t)Dm::V * Dm::H;
    default: return 0;
  }
}

template <int P>
void launch_phase(const PhaseArgs& pa, hipStream_t stream) {
  hipLaunchKernelGGL((phase_kernel<Model, P>), dim3(kNumWG), dim3(kBlock), 0, stream, pa);
}

}  // namespace
}  // namespace qmk

using namespace qmk;

extern "C" {

void launch_ldg_decode_direct(int input_token_id, int* output_token_id, const void* embed_weight,
                              const LDGLayerWeights* layer_weights, const void* final_norm_weight,
                              const void* lm_head_weight, const void* cos_table, const void* sin_table, void* k_cache,
                              void* v_cache, void* hidden_buffer, void* g_activations, void* g_residual, void* g_q,
                              void* g_k, void* g_v, void* g_attn_out, void* g_mlp_intermediate, void* g_normalized,
                              void* block_max_vals, void* block_max_idxs, int num_layers, int position,
                              int max_seq_len, float attn_scale, hipStream_t stream) {
  (void)g_activations; (void)g_residual; (void)g_q; (void)g_k; (void)g_v; (void)g_attn_out;
  (void)g_mlp_intermediate; (void)block_max_vals; (void)block_max_idxs;
  Common c{QMK_MODEL_QWEN3_0_6B, embed_weight, layer_weights, final_norm_weight, lm_head_weight, cos_table, sin_table, k_cache, v_cache,
           hidden_buffer, g_normalized, num_layers, max_seq_len, attn_scale};
  decode_impl(c, input_token_id, position, output_token_id, nullptr, stream, false);
}

void launch_ldg_decode_persistent(int input_token_id, int* output_token_id, const void* embed_weight,
                                  const LDGLayerWeights* layer_weights, const void* final_norm_weight,
                                  const void* lm_head_weight, const void* cos_table, const void* sin_table,
                                  void* k_cache, void* v_cache, void* hidden_buffer, void* g_activations,
                                  void* g_residual, void* g_q, void* g_k, void* g_v, void* g_attn_out,
                                  void* g_mlp_intermediate, void* g_normalized, void* block_max_vals,
                                  void* block_max_idxs, int num_layers, int position, int cache_len,
                                  int max_seq_len, float attn_scale, hipStream_t stream) {
  (void)g_activations; (void)g_residual; (void)g_q; (void)g_k; (void)g_v; (void)g_attn_out;
  (void)g_mlp_intermediate; (void)block_max_vals; (void)block_max_idxs;
  if (cache_len != position + 1) {
    fail(QMK_ERR_ARG);
    return;
  }
  Common c{QMK_MODEL_QWEN3_0_6B, embed_weight, layer_weights, final_norm_weight, lm_head_weight, cos_table, sin_table, k_cache, v_cache,
           hidden_buffer, g_normalized, num_layers, max_seq_len, attn_scale};
  decode_impl(c, input_token_id, position, output_token_id, nullptr, stream, true);
}

void launch_ldg_generate_nosync(int first_token_id, int num_steps, const void* embed_weight,
                                const LDGLayerWeights* layer_weights, const void* final_norm_weight,
                                const void* lm_head_weight, const void* cos_table, const void* sin_table,
                                void* k_cache, void* v_cache, void* hidden_buffer, void* g_activations,
                                void* g_residual, void* g_q, void* g_k, void* g_v, void* g_attn_out,
                                void* g_mlp_intermediate, void* g_normalized, void* block_max_vals,
                                void* block_max_idxs, int* output_log, int num_layers, int start_position,
                                int max_seq_len, float attn_scale, hipStream_t stream) {
  (void)g_activations; (void)g_residual; (void)g_q; (void)g_k; (void)g_v; (void)g_attn_out;
  (void)g_mlp_intermediate; (void)block_max_vals; (void)block_max_idxs;
  qmk_generate_model(QMK_MODEL_QWEN3_0_6B, first_token_id, num_steps, embed_weight, layer_weights, final_norm_weight,
                     lm_head_weight, cos_table, sin_table, k_cache, v_cache, hidden_buffer, g_normalized, output_log,
                     num_layers, start_position, max_seq_len, attn_scale, stream);
}

int qmk_generate_model(int model, int first_token_id, int num_steps, const void* embed_weight,
                       const LDGLayerWeights* layer_weights, const void* final_norm_weight, const void* lm_head_weight,
                       const void* cos_table, const void* sin_table, void* k_cache, void* v_cache,
                       void* hidden_buffer, void* g_normalized, int* output_log, int num_layers, int start_position,
                       int max_seq_len, float attn_scale, hipStream_t stream) {
  Common c{model, embed_weight, layer_weights, final_norm_weight, lm_head_weight, cos_table, sin_table, k_cache, v_cache,
           hidden_buffer, g_normalized, num_layers, max_seq_len, attn_scale};
  return generate_impl(c, first_token_id, num_steps, -1, output_log, start_position, stream);
}

int qmk_generate_eos(int model, int first_token_id, int num_steps, int eos_token_id, const void* embed_weight,
                     const LDGLayerWeights* layer_weights, const void* final_norm_weight, const void* lm_head_weight,
                     const void* cos_table, const void* sin_table, void* k_cache, void* v_cache, void* hidden_buffer,
                     void* g_normalized, int* output_log, int num_layers, int start_position, int max_seq_len,
                     float attn_scale, hipStream_t stream) {
  if (eos_token_id < 0) return fail(QMK_ERR_ARG);
  Common c{model, embed_weight, layer_weights, final_norm_weight, lm_head_weight, cos_table, sin_table, k_cache, v_cache,
           hidden_buffer, g_normalized, num_layers, max_seq_len, attn_scale};
  return generate_impl(c, first_token_id, num_steps, eos_token_id, output_log, start_position, stream);
}

int qmk_generate_sample(int model, int first_token_id, int num_steps, int eos_token_id, float temperature, int top_k,
                        float top_p, unsigned long long seed, const void* embed_weight,
                        const LDGLayerWeights* layer_weights, const void* final_norm_weight,
                        const void* lm_head_weight, const void* cos_table, const void* sin_table, void* k_cache,
                        void* v_cache, void* hidden_buffer, void* g_normalized, int* output_log, int num_layers,
                        int start_position, int max_seq_len, float attn_scale, hipStream_t stream) {
  if (!(temperature == temperature) || !(top_p == top_p)) return fail(QMK_ERR_ARG);
  Common c{model, embed_weight, layer_weights, final_norm_weight, lm_head_weight, cos_table, sin_table, k_cache, v_cache,
           hidden_buffer, g_normalized, num_layers, max_seq_len, attn_scale};
  const SampleParams sp{temperature, top_k, top_p, (uint64_t)seed};
  return generate_impl(c, first_token_id, num_steps, eos_token_id < 0 ? -1 : eos_token_id, output_log,
                       start_position, stream, &sp);
}

int qmk_set_graph_launch(hipStream_t stream, int enable) {
  Ctx* ctx = nullptr;
  const int s = get_ctx(stream, &ctx);
  if (s != QMK_OK) return fail(s);
  ctx->use_graphs = enable != 0;
  return fail(QMK_OK);
}

int qmk_decode_model(int model, int input_token_id, int* output_token_id, float* logits_out,
                     const void* embed_weight, const LDGLayerWeights* layer_weights, const void* final_norm_weight,
                     const void* lm_head_weight, const void* cos_table, const void* sin_table, void* k_cache,
                     void* v_cache, void* hidden_buffer, void* g_normalized, int num_layers, int position,
                     int max_seq_len, float attn_scale, hipStream_t stream) {
  Common c{model, embed_weight, layer_weights, final_norm_weight, lm_head_weight, cos_table, sin_table, k_cache, v_cache,
           hidden_buffer, g_normalized, num_layers, max_seq_len, attn_scale};
  return decode_impl(c, input_token_id, position, output_token_id, logits_out, stream, false);
}

int qmk_decode_logits(int input_token_id, int* output_token_id, float* logits_out, const void* embed_weight,
                      const LDGLayerWeights* layer_weights, const void* final_norm_weight, const void* lm_head_weight,
                      const void* cos_table, const void* sin_table, void* k_cache, void* v_cache, void* hidden_buffer,
                      void* g_normalized, int num_layers, int position, int max_seq_len, float attn_scale,
                      hipStream_t stream) {
  Common c{QMK_MODEL_QWEN3_0_6B, embed_weight, layer_weights, final_norm_weight, lm_head_weight, cos_table, sin_table, k_cache, v_cache,
           hidden_buffer, g_normalized, num_layers, max_seq_len, attn_scale};
  return decode_impl(c, input_token_id, position, output_token_id, logits_out, stream, false);
}

int qmk_init(void) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess) return fail(QMK_ERR_HIP);
  std::lock_guard<std::mutex> lk(g_mu);
  DevInfo* di = nullptr;
  const int s = check_device(dev, &di);
  if (s != QMK_OK) return fail(s);
  if (!di->scratch) {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) return fail(QMK_ERR_HIP);
    di->scratch = static_cast<uint32_t*>(p);
  }
  return fail(QMK_OK);
}

int qmk_decode_model_noalloc(int model, int input_token_id, int* output_token_id, float* logits_out,
                             const void* embed_weight, const LDGLayerWeights* layer_weights,
                             const void* final_norm_weight, const void* lm_head_weight, const void* cos_table,
                             const void* sin_table, void* k_cache, void* v_cache, void* hidden_buffer,
                             void* g_normalized, int num_layers, int position, int max_seq_len, float attn_scale,
                             hipStream_t stream) {
  // the scratch holds one exchange area for at most kMaxLayers layers of either model and caches of
  // at most kMaxSeqLen positions (the kernel's own limits)
  if (num_layers > kMaxLayers || max_seq_len > kMaxSeqLen) return fail(QMK_ERR_SIZE);
  Common c{model, embed_weight, layer_weights, final_norm_weight, lm_head_weight, cos_table, sin_table, k_cache, v_cache,
           hidden_buffer, g_normalized, num_layers, max_seq_len, attn_scale};
  int s = validate(c);
  if (s != QMK_OK) return fail(s);
  if (position < 0 || position >= c.max_seq_len) return fail(QMK_ERR_POSITION);
  if (input_token_id < 0 || input_token_id >= Dm::V) return fail(QMK_ERR_ARG);
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess) return fail(QMK_ERR_HIP);
  DevInfo* di = nullptr;
  uint32_t timeout = 0;
  {
    std::lock_guard<std::mutex> lk(g_mu);
    auto it = g_dev.find(dev);
    if (it != g_dev.end() && it->second.ok && it->second.scratch) {
      di = &it->second;
      timeout = di->noalloc_timeout ? di->noalloc_timeout : di->ticks_per_s;
    }
  }
  if (!di) return fail(QMK_ERR_INIT);
  Ctx view;  // the kernel arguments' view of the scratch; nothing is allocated
  view.st = reinterpret_cast<DecodeState*>(di->scratch);
  view.x = di->scratch + sizeof(DecodeState) / 4;
  view.timeout = timeout;
  view.xcd_local = di->xcd_local;
  KArgs a = make_args(c, &view);
  a.out_token = output_token_id;
  a.logits = logits_out;
  a.position = position;
  a.token = input_token_id;
  DeviceOrder order(di, stream);
  if (!order.ok()) return fail(QMK_ERR_HIP);
  hipLaunchKernelGGL(noalloc_prepare_kernel, dim3(1), dim3(256), 0, stream, view.st, view.x, kXWords,
                     (uint32_t)model + 1u);
  s = hipGetLastError() == hipSuccess ? launch(a, model, form_of(position + 1), stream) : QMK_ERR_HIP;
  const int so = order.finish();
  return fail(s != QMK_OK ? s : so);
}

namespace {
// the current device's entry once qmk_init has set its scratch up, else null
DevInfo* noalloc_device() {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess) return nullptr;
  std::lock_guard<std::mutex> lk(g_mu);
  auto it = g_dev.find(dev);
  return (it != g_dev.end() && it->second.ok && it->second.scratch) ? &it->second : nullptr;
}
}  // namespace

int qmk_noalloc_set_wait_limit(uint32_t ticks) {
  DevInfo* di = noalloc_device();
  if (!di) return fail(QMK_ERR_INIT);
  std::lock_guard<std::mutex> lk(g_mu);
  di->noalloc_timeout = ticks;
  return fail(QMK_OK);
}

uint32_t qmk_noalloc_device_error(hipStream_t stream) {
  DevInfo* di = noalloc_device();
  if (!di) return 0xffffffffu;
  if (hipStreamSynchronize(stream) != hipSuccess) return 0xffffffffu;
  // the state header sits at the start of the scratch; one word straight into a local
  uint32_t v = 0;
  if (hipMemcpy(&v, &reinterpret_cast<DecodeState*>(di->scratch)->err, sizeof(v), hipMemcpyDeviceToHost) !=
      hipSuccess)
    return 0xffffffffu;
  return v;
}

int qmk_last_status(void) { return t_status; }

const char* qmk_status_string(int status) {
  switch (status) {
    case QMK_OK: return "ok";
    case QMK_ERR_ARG: return "invalid argument";
    case QMK_ERR_POSITION: return "position outside [0, max_seq_len)";
    case QMK_ERR_DEVICE: return "device unsuitable: needs a gfx950 GPU with 256 CUs";
    case QMK_ERR_HIP: return "HIP runtime call failed";
    case QMK_ERR_POISONED: return "an earlier launch on this stream failed on the device; call qmk_reset";
    case QMK_ERR_INIT: return "qmk_init() has not been called on this device";
    case QMK_ERR_SIZE:
      return "input beyond the allocation-free entry point's limits (num_layers <= 28, max_seq_len <= 65536)";
    default: return "unknown status";
  }
}

uint32_t qmk_device_error(hipStream_t stream) {
  Ctx* ctx = nullptr;
  if (get_ctx(stream, &ctx) != QMK_OK) return 0xffffffffu;
  if (hipStreamSynchronize(stream) != hipSuccess) return 0xffffffffu;
  uint32_t v = 0, vb = 0;
  if (hipMemcpy(&v, &ctx->st->err, sizeof(v), hipMemcpyDeviceToHost) != hipSuccess) return 0xffffffffu;
  if (ctx->bst && hipMemcpy(&vb, &ctx->bst->err, sizeof(vb), hipMemcpyDeviceToHost) != hipSuccess) return 0xffffffffu;
  return v | vb | *ctx->host_err;
}

int qmk_reset(hipStream_t stream) {
  Ctx* ctx = nullptr;
  int s = get_ctx(stream, &ctx);
  if (s != QMK_OK) return fail(s);
  if (hipStreamSynchronize(stream) != hipSuccess) return fail(QMK_ERR_HIP);
  const size_t bytes = sizeof(DecodeState) + (size_t)kXWords * 4;
  if (hipMemset(ctx->st, 0, bytes) != hipSuccess) return fail(QMK_ERR_HIP);
  if (ctx->bst && hipMemset(ctx->bst, 0, sizeof(DecodeState) + (size_t)kBXWords * 4) != hipSuccess)
    return fail(QMK_ERR_HIP);
  *ctx->host_err = 0;
  return fail(QMK_OK);
}

int qmk_set_wait_limit(hipStream_t stream, uint32_t ticks) {
  Ctx* ctx = nullptr;
  int s = get_ctx(stream, &ctx);
  if (s != QMK_OK) return fail(s);
  if (ticks == 0) ticks = ctx->ticks_per_s;
  ctx->timeout = ticks;
  return fail(QMK_OK);
}

int qmk_set_trace(hipStream_t stream, uint64_t* buf, size_t entries) {
  Ctx* ctx = nullptr;
  int s = get_ctx(stream, &ctx);
  if (s != QMK_OK) return fail(s);
  if (buf && entries < (size_t)qmk_trace_entries(28)) return fail(QMK_ERR_ARG);
  ctx->trace = buf;
  return fail(QMK_OK);
}

size_t qmk_trace_entries(int num_layers) {
  return (size_t)(num_layers * (kTracePoints + kComputePoints) + 3) * kNumWG;
}

int qmk_selftest_blocks(const float* in, float* out, int n, hipStream_t stream) {
  if (!in || !out || n < 64) return fail(QMK_ERR_ARG);
  hipLaunchKernelGGL(selftest_kernel, dim3(1), dim3(64), 0, stream, in, out, n);
  return fail(hipGetLastError() == hipSuccess ? QMK_OK : QMK_ERR_HIP);
}

size_t qmk_phase_copy_elems(int phase) { return phase_copy_elems(phase); }

int qmk_phase_bench(int phase, const void* weights, int n_copies, const void* norm_weight, const void* act, void* out,
                    hipStream_t stream) {
  if (phase_copy_elems(phase) == 0 || !weights || n_copies < 1 || !act || !out || (phase == kPhaseQKV && !norm_weight))
    return fail(QMK_ERR_ARG);
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess) return fail(QMK_ERR_HIP);
  {
    std::lock_guard<std::mutex> lk(g_mu);
    DevInfo* di = nullptr;
    const int s = check_device(dev, &di);
    if (s != QMK_OK) return fail(s);
  }
  PhaseArgs pa{static_cast<const uint16_t*>(weights), phase_copy_elems(phase), n_copies,
               static_cast<const uint16_t*>(norm_weight), static_cast<const uint16_t*>(act), out, 1e-6f};
  switch (phase) {
    case kPhaseQKV: launch_phase<kPhaseQKV>(pa, stream); break;
    case kPhaseO: launch_phase<kPhaseO>(pa, stream); break;
    case kPhaseGateUp: launch_phase<kPhaseGateUp>(pa, stream); break;
    case kPhaseDown: launch_phase<kPhaseDown>(pa, stream); break;
    default: launch_phase<kPhaseLmHead>(pa, stream); break;
  }
  return fail(hipGetLastError() == hipSuccess ? QMK_OK : QMK_ERR_HIP);
}

void qmk_launch_geometry(int* workgroups, int* threads) {
  if (workgroups) *workgroups = kNumWG;
  if (threads) *threads = kBlock;
}

int qmk_decode_batch_persistent(int model, int batch, const int* tokens, const int* positions, int* out_tokens,
                                float* logits_out, const void* embed_weight, const LDGLayerWeights* layer_weights_host,
                                const void* final_norm_weight, const void* lm_head_weight, const void* cos_table,
                                const void* sin_table, void* k_cache, void* v_cache, long long seq_stride,
                                int num_layers, int max_seq_len, int max_context, float attn_scale,
                                hipStream_t stream) {
  return fail(batch_persistent_impl(model, batch, tokens, positions, out_tokens, logits_out, embed_weight,
                                    layer_weights_host, final_norm_weight, lm_head_weight, cos_table, sin_table,
                                    k_cache, v_cache, seq_stride, num_layers, max_seq_len, max_context, attn_scale,
                                    stream));
}

int qmk_set_batch_persistent(int enable) {
  g_batch_persistent.store(enable != 0);
  return QMK_OK;
}

int qmk_batch_persistent_enabled(void) { return g_batch_persistent.load(); }

}  // extern "C"
