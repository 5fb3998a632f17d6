// Qwen3 batch-1 bf16 decode step for MI355X (gfx950): one persistent kernel
// launch per token (28 decoder layers, final norm, tied LM head and argmax).
//
// Replaces the reference's ldg_decode_kernel_direct / _persistent +
// ldg_lm_head_fused + ldg_update_step (reference csrc/kernel.cu:1189-1440).
// The reference splits the work over 128 blocks of 16 warps that meet at
// global atomic barriers (csrc/kernel.cu:94-119).  Here 256 workgroups run,
// one per CU; workgroup b sits on XCD x = b % 8 with rank r = b / 8 inside
// it, and the eight XCDs split each layer the way eight GPUs would under
// tensor parallelism, so that almost every hand-off stays inside one XCD's L2:
//
//   XCD x owns KV head x and its query heads 2x, 2x+1 (QKV rows, attention),
//   the matching 256 input columns of o_proj, and the m slice
//   [384x, 384x+384) (gate/up rows and the matching 384 input columns of
//   down_proj).  o_proj and down_proj therefore produce per-XCD partial sums,
//   which are reduced across XCDs: rank r of every XCD owns hidden rows
//   [32r, 32r+32), sums the eight partials of those rows and applies the
//   residual add.
//
// Activations move between workgroups as tagged words (qmk_device.h).  Per
// layer (k = exchange index inside the layer):
//
//   k  exchange   producers -> consumers                scope
//   0  qkv        32 WGs of XCD x -> same 32 WGs         XCD-local
//   1  ml         softmax (max, sum) per WG and head     XCD-local
//   2  acc        P@V partial sums per WG and head       XCD-local
//   3  attn       attention output of heads 2x, 2x+1     XCD-local
//   4  o          o_proj partials, rows 32r..32r+31      across XCDs (8 -> 8)
//   5  h2         h' = h + o_proj(attn)                  XCD-local
//   6  m          silu(gate) * up, slice of XCD x        XCD-local
//   7  d          down_proj partials, rows 32r..32r+31   across XCDs (8 -> 8)
//   8  h          h'' = h' + down(m)                     XCD-local
//
// Numerics follow HF Qwen3's bf16 eager path, op for op: every output is
// rounded to bf16 where HF rounds it (norm outputs, projections, q/k norm,
// RoPE products and sum, attention scores and their scaling, softmax
// probabilities, attention output, residual adds, SiLU and its product,
// logits); dot products accumulate in fp32.  Attention is split over the 32
// workgroups of an XCD and takes HF's two passes in every form: the
// workgroups' (max, sum) pairs are merged first, so that the probabilities
// are normalised with the global max and sum and rounded to bf16 before P@V.
//
// Each workgroup has 9 waves.  Wave 0 ("control") moves activations: it polls
// exchanges, applies norms / RoPE / residuals / SiLU, publishes results and
// fills LDS.  Waves 1..8 ("compute") hold each phase's weight slice in VGPRs,
// requested one layer before use, so HBM streams while the control wave
// waits on exchanges; the control wave never has weight loads outstanding,
// so its polls are not queued behind them.

#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "qmk_device.h"
#include "qmk_sample.h"
#include "qmk_state.h"

namespace qmk {

struct Qwen3_0_6B {
  static constexpr int H = 1024, I = 3072, NQ = 16, NKV = 8, D = 128, V = 151936;
};

struct Qwen3_1_7B {
  static constexpr int H = 2048, I = 6144, NQ = 16, NKV = 8, D = 128, V = 151936;
};

constexpr int kMaxSeqLen = 65536;                          // longest cache the kernel accepts
constexpr int kChunkMax = kMaxSeqLen / kGroupSize;         // attention positions per workgroup
constexpr int kTracePoints = 13;                           // control-wave stamps per layer
constexpr int kComputePoints = 12;                         // compute-wave stamps per layer (start/end of 6 phases)
constexpr int kMaxLayers = 28;
constexpr int kKvU = 2;        // attention: each wave covers 4 positions (16-lane rows) x kKvU per batch
constexpr int kKvStages = 4;   // K/V batches in flight per wave (LDS ring)
constexpr int kLongContext = 2048;  // contexts above this run decode_kernel<M, S, true>
constexpr int kDeepContext = 12288; // contexts above this run decode_kernel_deep<M, S>
// Short-context Qwen3-0.6B, two-pass form: this layer's gate/up slice is requested at barrier c
// (it drains during the scores and the (max, sum) exchange) and its o_proj slice at barrier e
// (during P@V).  Same-box A/B at context 1024: both at c 1,999 tok/s, both at e 2,010, gate/up at c
// and o_proj at e 2,062.  A pause of 0.25-1 us between the down_proj partials' publish and the next
// layer's K/V and QKV-row requests measured 2,064 / 2,065 / 2,044 against 2,061.
constexpr bool kGateUpAtC = true, kOprojAtC = false;

template <class M>
struct Dims {
  static constexpr int H = M::H, I = M::I, NQ = M::NQ, NKV = M::NKV, D = M::D, V = M::V;
  static constexpr int QS = NQ * D;             // attention output width
  static constexpr int GQ = NQ / NKV;           // query heads per KV head
  static constexpr int RG = (GQ + 2) * D;       // q+k+v rows of one KV-head group
  static constexpr int RQ_WG = RG / kGroupSize; // QKV rows per workgroup
  static constexpr int RQ_W = RQ_WG / kComputeWaves;
  static constexpr int LH = H / 512;            // 16-byte chunks per lane for a K=H row
  static constexpr int OC = GQ * D;             // o_proj input columns per XCD
  static constexpr int MS = I / kGroups;        // m slice per XCD
  static constexpr int M_WG = MS / kGroupSize;  // m values per workgroup
  static constexpr int GU_W = 2 * M_WG / kComputeWaves;  // gate/up rows per wave
  static constexpr int ROWS_WG = H / kGroupSize;          // reduce-scatter rows per workgroup
  static constexpr int ROWS_W = ROWS_WG / kComputeWaves;  // o/down rows per wave
  static constexpr int OP = ROWS_W / 4;         // o/down passes per wave (four rows, one per 16-lane slot)
  static constexpr int LO = OC / 8 / 16;        // o_proj chunks per lane (16 lanes per row)
  static constexpr int LD = MS / 8 / 16;        // down_proj chunks per lane
  static constexpr int LM_RPW = (V + kNumWG - 1) / kNumWG;
  static constexpr int LM_U = 8 / LH;           // LM-head rows per wave per batch (two batches in flight)
  static constexpr int NX = 9;                  // exchanges per layer
  static constexpr int OUT = 2 * M_WG > 64 ? 2 * M_WG : 64;  // per-workgroup results handed to the control wave
  // Weight prefetch.  When a workgroup's share of a layer fits the compute
  // waves' registers (Qwen3-0.6B: 120 KB per workgroup), every phase's slice is
  // requested one layer ahead into its own registers.  Otherwise (Qwen3-1.7B:
  // 384 KB per workgroup) each phase's slice is requested at the end of the
  // compute phase before it, into a buffer the QKV, gate/up and down phases
  // share (o_proj keeps its own, being loaded before attention).
  static constexpr bool kStream = H > 1024;
  static constexpr int NBUF = (RQ_W * LH > GU_W * LH ? RQ_W * LH : GU_W * LH) > OP * LD
                                  ? (RQ_W * LH > GU_W * LH ? RQ_W * LH : GU_W * LH)
                                  : OP * LD;
  // exchange layout (words)
  static constexpr uint32_t X_QKV = 0;                                        // [xcd][RG]
  static constexpr uint32_t X_ML = X_QKV + kGroups * RG;                      // [xcd][rank][GQ*4]
  static constexpr uint32_t X_ACC = X_ML + kGroups * kGroupSize * GQ * 4;     // [xcd][rank][GQ*D*2]
  static constexpr uint32_t X_ATTN = X_ACC + kGroups * kGroupSize * GQ * D * 2;  // [xcd][OC]
  static constexpr uint32_t X_O = X_ATTN + kGroups * OC;                      // [xcd][rank][ROWS_WG*2]
  static constexpr uint32_t X_H2 = X_O + kGroups * kGroupSize * ROWS_WG * 2;  // [xcd][H]
  static constexpr uint32_t X_M = X_H2 + kGroups * H;                         // [xcd][MS]
  static constexpr uint32_t X_D = X_M + kGroups * MS;                         // [xcd][rank][ROWS_WG*2]
  static constexpr uint32_t X_H = X_D + kGroups * kGroupSize * ROWS_WG * 2;   // [xcd][H]
  static constexpr uint32_t X_KEY = X_H + kGroups * H;                        // [wg][4]
  static constexpr uint32_t X_WORDS = X_KEY + kNumWG * 4;

  static_assert(RG % kGroupSize == 0 && RQ_WG % kComputeWaves == 0, "QKV split");
  static_assert((GQ * D) % RQ_WG == 0 && D % RQ_WG == 0 && RQ_WG % 4 == 0, "QKV block inside one projection");
  static_assert(H % 512 == 0, "K=H rows in 512-element wave loads");
  static_assert(OC % 128 == 0 && MS % 128 == 0, "o/down slices in 16-lane row segments");
  static_assert(ROWS_W % 4 == 0, "o/down: passes of four rows, one per 16-lane slot");
  static_assert(8 % LH == 0, "LM-head batch");
  static_assert(64 % (ROWS_WG / 2) == 0 || (ROWS_WG / 2) % 64 == 0, "reduce-scatter lane mapping");
  static_assert(2 * M_WG == GU_W * kComputeWaves && M_WG % 4 == 0, "gate/up split");
  static_assert(GQ * (D / 8) == kGroupSize, "combine: one (head, 8-dim block) per workgroup");
  static_assert(ROWS_WG % 16 == 0, "reduce-scatter: 16 lanes x 2 rows");
  static_assert(X_WORDS % 4 == 0, "alignment");
};

struct LayerPtrs {  // same order as the reference's LDGLayerWeights (csrc/torch_bindings.cpp:21-33)
  const uint16_t* in_ln;
  const uint16_t* wq;
  const uint16_t* wk;
  const uint16_t* wv;
  const uint16_t* q_norm;
  const uint16_t* k_norm;
  const uint16_t* wo;
  const uint16_t* post_ln;
  const uint16_t* wg;
  const uint16_t* wu;
  const uint16_t* wd;
};

struct KArgs {
  const uint16_t* embed;
  const LayerPtrs* layers;
  const uint16_t* final_norm;
  const uint16_t* lm_head;
  const uint16_t* cos_t;
  const uint16_t* sin_t;
  uint16_t* k_cache;
  uint16_t* v_cache;
  uint16_t* hidden_out;    // optional bf16 [H]: final hidden state
  float* normalized_out;   // optional f32 [H]: final-norm output
  int* out_token;          // optional
  float* logits;           // optional f32 [V]: bf16-valued logits
  int* out_log;            // optional: generated-token log (persistent mode)
  DecodeState* st;
  uint32_t* x;             // exchange words
  uint32_t* host_err;      // optional host-visible error word
  uint64_t* trace;         // optional: wall-clock stamps [layer*13 + point][workgroup], then 3 final points
  int num_layers;
  int max_seq_len;
  int position;            // < 0: read position/token/step from the state
  int token;
  float attn_scale;
  float rms_eps;
  float temperature;       // > 0: the step's token is a Gumbel-max draw from softmax(logits / temperature)
  uint64_t seed;           //      with the random numbers of (seed, position); 0: greedy
  uint32_t timeout;
  int xcd_local;           // 1: XCD-local exchanges stay in the XCD's L2
};

__device__ __forceinline__ float rcp_sqrt_torch(float v) {
  // torch CPU rsqrt = 1 / sqrt(x), each correctly rounded
  return __fdiv_rn(1.0f, __fsqrt_rn(v));
}

// A pointer read from LDS lands in VGPRs; all lanes hold the same value, so
// move it to SGPRs for scalar address arithmetic.
template <class T>
__device__ __forceinline__ T* uniform_ptr(T* p) {
  const uint64_t v = reinterpret_cast<uint64_t>(p);
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
  return reinterpret_cast<T*>(((uint64_t)hi << 32) | lo);
}

__device__ __forceinline__ float f32_from_words(uint32_t hi_word, uint32_t lo_word) {
  return __uint_as_float((hi_word & 0xffff0000u) | (lo_word >> 16));
}

template <class M>
struct Smem {
  using Dm = Dims<M>;
  float x[Dm::H];                    // layer input (residual), bf16 values
  float h2[Dm::H];                   // post-attention hidden
  uint16_t n[Dm::H];                 // normalised activation (bf16)
  uint16_t attn[Dm::OC];             // attention output of this XCD's heads
  uint16_t m[Dm::MS];                // this XCD's m slice
  float qkv[Dm::RG];
  uint16_t q[Dm::GQ * Dm::D];
  uint16_t k[Dm::D];
  uint16_t v[Dm::D];
  float sc[Dm::GQ][kChunkMax];       // this workgroup's attention scores (bf16 values)
  u32x4 kv[kKvStages][kComputeWaves][kKvU][kWave];  // K/V batches, written by the loads themselves (LDS DMA)
  float wml[kComputeWaves][Dm::GQ][2];
  float wacc[kComputeWaves][Dm::GQ][Dm::D];
  float ml[Dm::GQ][2];               // global softmax max and sum per head
  float out[Dm::OUT];
  uint64_t best[kComputeWaves];
  LayerPtrs layers[kMaxLayers];      // copy of the packed pointer table, read once per launch
  int abort_flag;
  int stop_flag;                     // persistent mode: the stop token was emitted by an earlier launch
};

// The long-context kernel's LDS: the same object with per-wave score and
// probability arrays appended (one object, so the compiler can tell that reads
// of the other fields never alias the K/V ring's in-flight DMA).  They are
// indexed by the wave's entry i = 8 batch + 4 u + slot, so the one-position-
// per-lane passes touch consecutive words; indexed by position, a wave's
// positions (4 wave + slot + 32 u + 64 batch) would fall on four banks.
constexpr int kWaveEntries = 8 * (kChunkMax / (32 * kKvU));  // entries of one wave's batches
constexpr int kHeadStride = kWaveEntries + 8;                 // head 1 starts eight banks after head 0
template <class M>
struct SmemLong : Smem<M> {
  float sw[kComputeWaves][2 * kHeadStride];  // scores of head h at [wave][h * kHeadStride + i] (bf16 values)
  uint32_t pw[kComputeWaves][kWaveEntries];  // bf16 probabilities, head 1 << 16 | head 0
};

struct Step {
  uint32_t epoch;
  int pos, tok, step, C, nl;
  int chunk, p_begin, p_end, n_act;  // this workgroup's attention positions
  bool persistent;
};

// ------------------------------------------------------------- control wave

template <class M>
struct Ctl {
  using Dm = Dims<M>;
  const KArgs& a;
  Smem<M>& s;
  int lane;

  __device__ Ctl(const KArgs& a_, Smem<M>& s_, int lane_) : a(a_), s(s_), lane(lane_) {}

  __device__ void fail(uint32_t bits) {
    atomicOr(&a.st->err, bits);
    if (a.host_err) __hip_atomic_store(a.host_err, bits, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    s.abort_flag = 1;
  }

  // Waits until the NCH 16-byte chunks named by off(i) (word offsets into the
  // exchange area, i < NCH) all carry ``tag``; calls sink(i, chunk) once per
  // chunk as it arrives.  A round is one 16-byte load per lane for every 64
  // chunks (NC loads).  A CU returns vector-memory data in order, so every poll
  // load in flight delays the next one and the compute waves' loads behind it:
  // rounds of one load, and of two loads in the Qwen3-0.6B kernel, keep two
  // rounds in flight (a chunk that lands while one is out is seen by the next
  // half a round trip later), larger rounds keep one.  Measured on the decode
  // step: two rounds everywhere 1,866 tok/s, one everywhere 1,890, two for
  // one-load rounds only 1,899; three or four rounds 1,688 / 1,567.  With the
  // control wave's element work cut (same-box A/B, context 1024): two rounds
  // for rounds of up to two loads 2,118-2,120 against 2,115, up to three
  // 2,104, up to four 2,056; Qwen3-1.7B (whose one two-load gather is the qkv
  // exchange, polled behind the o_proj slice requested before it) 1,103
  // against 1,111 with two rounds for it, so it keeps one.
  template <int NCH, class Off, class F>
  __device__ bool gather(uint32_t tag, Off&& off, F&& sink) {
    constexpr int NC = (NCH + 63) / 64;
    static_assert(NC <= 16, "gather size");
    if (s.abort_flag) return false;  // an earlier wait of this workgroup expired: go to the next barrier
    auto rs = make_rsrc(a.x, 0x7fffffffu);
    uint32_t o[NC];
    uint32_t pend = 0;
#pragma unroll
    for (int j = 0; j < NC; j++) {
      const int i = j * 64 + lane;
      o[j] = i < NCH ? off(i) * 4u : 0u;
      if (i < NCH) pend |= 1u << j;
    }
    // Every round issues all NC loads so the wait for the oldest round is a
    // static vmcnt((R - 1) * NC); chunks already received are pointed past the end of the
    // buffer descriptor, which makes their loads return 0 without memory traffic.
    constexpr uint32_t kOOB = 0xfffffff0u;
    constexpr int R = (NC == 1 || (NC == 2 && !Dm::kStream)) ? 2 : 1;  // rounds in flight
    u32x4 v[R][NC];
#pragma unroll
    for (int k = 0; k < R - 1; k++)
#pragma unroll
      for (int j = 0; j < NC; j++) v[k][j] = poll16(rs, (pend & (1u << j)) ? o[j] : kOOB);
    const uint64_t t0 = wall_clock64();
    while (true) {
      // round k is waited for (static vmcnt((R - 1) * NC)) after the next one is issued
#pragma unroll
      for (int k = 0; k < R; k++) {
#pragma unroll
        for (int j = 0; j < NC; j++) v[(k + R - 1) % R][j] = poll16(rs, (pend & (1u << j)) ? o[j] : kOOB);
#pragma unroll
        for (int j = 0; j < NC; j++)
          if ((pend & (1u << j)) && chunk_ok(v[k][j], tag)) {
            sink(j * 64 + lane, v[k][j]);
            pend &= ~(1u << j);
          }
        if (!__any(pend != 0)) return true;
      }
      if (wall_clock64() - t0 > a.timeout) {
        fail(kErrTimeout);
        return false;
      }
    }
    return true;
  }

  // Contiguous NW words at word offset ``base``.
  template <int NW, class F>
  __device__ bool gather_range(uint32_t base, uint32_t tag, F&& sink) {
    static_assert(NW % 4 == 0, "whole chunks");
    return gather<NW / 4>(tag, [&](int i) { return base + 4u * (uint32_t)i; }, sink);
  }

  // gather sinks: chunk ci (four bf16 payloads) to fp32 dst[4ci..4ci+3], or to bf16 dst[4ci..]
  static __device__ auto to_f32(float* dst) {
    return [dst](int ci, u32x4 v) {
      float* d = dst + 4 * ci;
      d[0] = bf16_to_f32(v.x >> 16); d[1] = bf16_to_f32(v.y >> 16);
      d[2] = bf16_to_f32(v.z >> 16); d[3] = bf16_to_f32(v.w >> 16);
    };
  }
  static __device__ auto to_bf16(uint16_t* dst) {
    return [dst](int ci, u32x4 v) {
      uint32_t* d = reinterpret_cast<uint32_t*>(dst) + 2 * ci;
      d[0] = (v.x >> 16) | (v.y & 0xffff0000u);
      d[1] = (v.z >> 16) | (v.w & 0xffff0000u);
    };
  }

  __device__ void put(bool local, uint32_t w, u32x4 d) {
    if (local && a.xcd_local) put4<false>(a.x, w, d);
    else put4<true>(a.x, w, d);
  }

  __device__ void put_bf16x4(bool local, uint32_t w, float v0, float v1, float v2, float v3, uint32_t tag) {
    u32x4 d;
    d.x = word(f32_to_bf16(v0), tag);
    d.y = word(f32_to_bf16(v1), tag);
    d.z = word(f32_to_bf16(v2), tag);
    d.w = word(f32_to_bf16(v3), tag);
    put(local, w, d);
  }

  __device__ void put_f32x2(bool local, uint32_t w, float v0, float v1, uint32_t tag) {
    const uint32_t b0 = __float_as_uint(v0), b1 = __float_as_uint(v1);
    u32x4 d;
    d.x = (b0 & 0xffff0000u) | tag;
    d.y = (b0 << 16) | tag;
    d.z = (b1 & 0xffff0000u) | tag;
    d.w = (b1 << 16) | tag;
    put(local, w, d);
  }

  // Norm weights are requested before the control wave starts polling, so
  // their latency overlaps the wait instead of following it.
  struct NormW {
    uint32_t w[Dm::H / 128];  // bf16 pairs lane + 64*i
  };
  __device__ NormW load_norm(const uint16_t* w) {
    NormW r;
    const uint32_t* w2 = reinterpret_cast<const uint32_t*>(w);
#pragma unroll
    for (int i = 0; i < Dm::H / 128; i++) r.w[i] = ld32(w2 + lane + 64 * i);
    return r;
  }

  // RMSNorm of ``src`` (fp32 holding bf16 values) with bf16 weight -> s.n:
  // bf16(w * bf16(x * rsqrt(mean(x^2) + eps)))  (HF Qwen3RMSNorm).
  __device__ void rmsnorm(const float* src, const NormW& nw) {
    constexpr int P = Dm::H / 128;  // element pairs per lane
    float2 xv[P];
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < P; i++) {
      xv[i] = reinterpret_cast<const float2*>(src)[lane + 64 * i];
      ss += xv[i].x * xv[i].x + xv[i].y * xv[i].y;
    }
    ss = wave_sum(ss);
    // the mean: H is a power of two, so the product with 1/H is the correctly rounded quotient
    static_assert((Dm::H & (Dm::H - 1)) == 0, "H a power of two");
    const float rstd = rcp_sqrt_torch(ss * (1.0f / Dm::H) + a.rms_eps);
    // two elements per conversion: bf16(x * rstd), then bf16(w * that)
#pragma unroll
    for (int i = 0; i < P; i++) {
      const int pi = lane + 64 * i;
      const uint32_t wp = nw.w[i];
      const uint32_t xn = pack_bf16x2(xv[i].x * rstd, xv[i].y * rstd);
      reinterpret_cast<uint32_t*>(s.n)[pi] = pack_bf16x2(lo_bf16(wp) * lo_bf16(xn), hi_bf16(wp) * hi_bf16(xn));
    }
  }

  // Per-head RMSNorm weight and RoPE row values for elements lane, lane + 64.
  struct HeadW {
    float w0, w1, c0, c1, s0, s1;
  };
  __device__ HeadW load_head(const uint16_t* w, const uint16_t* cosr, const uint16_t* sinr) {
    HeadW h;
    h.w0 = bf16_to_f32(ldu16(w + lane));
    h.w1 = bf16_to_f32(ldu16(w + lane + 64));
    h.c0 = bf16_to_f32(ldu16(cosr + lane));
    h.c1 = bf16_to_f32(ldu16(cosr + lane + 64));
    h.s0 = bf16_to_f32(ldu16(sinr + lane));
    h.s1 = bf16_to_f32(ldu16(sinr + lane + 64));
    return h;
  }

  // Per-head RMSNorm + rotate-half RoPE of the GQ q heads and the k head held in s.qkv, into s.q
  // and s.k.  Each head's sum of squares is reduced on its own; the correctly rounded 1/sqrt of
  // head h's mean is evaluated in lane h, once for all heads, and read back with readlane.
  __device__ void qk_norm_rope(const HeadW& hq, const HeadW& hk) {
    constexpr int NH = Dm::GQ + 1;
    static_assert((Dm::D & (Dm::D - 1)) == 0, "head_dim a power of two");
    float x0[NH], x1[NH], v = 0.f;
#pragma unroll
    for (int h = 0; h < NH; h++) {
      x0[h] = s.qkv[h * Dm::D + lane];
      x1[h] = s.qkv[h * Dm::D + lane + 64];
      const float ss = wave_sum(x0[h] * x0[h] + x1[h] * x1[h]);
      v = lane == h ? ss : v;
    }
    const float rl = rcp_sqrt_torch(v * (1.0f / Dm::D) + a.rms_eps);
#pragma unroll
    for (int h = 0; h < NH; h++) {
      const float rstd = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(rl), h));
      head_rope(x0[h], x1[h], rstd, h < Dm::GQ ? hq : hk, h < Dm::GQ ? s.q + h * Dm::D : s.k);
    }
  }

  __device__ void head_rope(float x0, float x1, float rstd, const HeadW& hw, uint16_t* dst) {
    // the lane's two elements share each bf16 conversion
    const uint32_t xn = pack_bf16x2(x0 * rstd, x1 * rstd);
    const uint32_t nn = pack_bf16x2(hw.w0 * lo_bf16(xn), hw.w1 * hi_bf16(xn));
    const float n0 = lo_bf16(nn), n1 = hi_bf16(nn);
    // x*cos + rotate_half(x)*sin with rotate_half(x) = (-x[64:], x[:64]), each product rounded
    const uint32_t pc = pack_bf16x2(n0 * hw.c0, n1 * hw.c1);
    const uint32_t ps = pack_bf16x2(-n1 * hw.s0, n0 * hw.s1);
    const uint32_t y = pack_bf16x2(lo_bf16(pc) + lo_bf16(ps), hi_bf16(pc) + hi_bf16(ps));
    dst[lane] = (uint16_t)(y & 0xffffu);
    dst[lane + 64] = (uint16_t)(y >> 16);
  }

  // Reduce-scatter across XCDs: sums the eight XCD partials of this rank's
  // ROWS_WG hidden rows (fixed order), adds the residual ``res`` and rounds
  // like HF: bf16(res + bf16(sum)).  Publishes the rows into this XCD's copy
  // of ``x_dst``.  Returns false on timeout.
  __device__ bool reduce_rows(uint32_t x_src, uint32_t src_tag, const float* res, uint32_t x_dst, uint32_t dst_tag,
                              int xcd, int r) {
    constexpr int R = Dm::ROWS_WG;       // rows per rank, 2 per chunk
    constexpr int CPX = R / 2;           // chunks per source XCD
    constexpr int NSL = kGroups * CPX / 64;  // chunks per lane
    static_assert(CPX <= 64 && 64 % CPX == 0, "a source XCD's chunks within one 64-chunk slot");
    float sum0 = 0.f, sum1 = 0.f;
    // chunk i: source XCD i / CPX, rows 2*(i % CPX) .. +1; lane l receives chunks l + 64*slot
    float part0[NSL], part1[NSL];
    const bool ok = gather<kGroups * CPX>(
        src_tag, [&](int i) { return x_src + (uint32_t)(((i / CPX) * kGroupSize + r) * R * 2 + (i % CPX) * 4); },
        [&](int i, u32x4 v) {
          const int slot = i / 64;
          part0[slot] = f32_from_words(v.x, v.y);
          part1[slot] = f32_from_words(v.z, v.w);
        });
    if (!ok) return false;
    // lane l < CPX sums row pair l over the sources in order 0..7, each fetched
    // from the lane that received it, (src * CPX) % 64 lanes ahead, by row swaps
    float p0[kGroups], p1[kGroups];
#pragma unroll
    for (int src = 0; src < kGroups; src++) {
      const int sl = (src * CPX) / 64;
      switch ((src * CPX) % 64) {
        case 0: p0[src] = part0[sl]; p1[src] = part1[sl]; break;
        case 16: p0[src] = lane_ahead<16>(part0[sl]); p1[src] = lane_ahead<16>(part1[sl]); break;
        case 32: p0[src] = lane_ahead<32>(part0[sl]); p1[src] = lane_ahead<32>(part1[sl]); break;
        default: p0[src] = lane_ahead<48>(part0[sl]); p1[src] = lane_ahead<48>(part1[sl]); break;
      }
    }
#pragma unroll
    for (int src = 0; src < kGroups; src++) {
      sum0 += p0[src];
      sum1 += p1[src];
    }
    if (lane < CPX) {
      const int row = R * r + 2 * lane;
      const uint32_t sb = pack_bf16x2(sum0, sum1);
      const uint32_t hb = pack_bf16x2(res[row] + lo_bf16(sb), res[row + 1] + hi_bf16(sb));
      const uint32_t hb0 = hb & 0xffffu, hb1 = hb >> 16;
      // two words per lane: pairs of lanes form one 16-byte store
      const uint32_t ob0 = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)hb0, 0xB1, 0xf, 0xf, false);  // lane ^ 1
      const uint32_t ob1 = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)hb1, 0xB1, 0xf, 0xf, false);
      if ((lane & 1) == 0) {
        u32x4 d;
        d.x = word(hb0, dst_tag);
        d.y = word(hb1, dst_tag);
        d.z = word(ob0, dst_tag);
        d.w = word(ob1, dst_tag);
        put(true, x_dst + (uint32_t)(xcd * Dm::H + row), d);
      }
    }
    return true;
  }
};

// ------------------------------------------------------------- compute waves

template <int NL>
__device__ __forceinline__ void load_row(u32x4 (&dst)[NL], const uint16_t* row, int k0, int lane) {
#pragma unroll
  for (int j = 0; j < NL; j++) dst[j] = ld_stream(row + k0 + 512 * j + 8 * lane);
}

template <int NL>
__device__ __forceinline__ void load_act(u32x4 (&dst)[NL], const uint16_t* act, int k0, int lane) {
#pragma unroll
  for (int j = 0; j < NL; j++) dst[j] = *reinterpret_cast<const u32x4*>(act + k0 + 512 * j + 8 * lane);
}

template <int NL>
__device__ __forceinline__ float row_dot(const u32x4 (&w)[NL], const u32x4 (&x)[NL]) {
  float acc = 0.f;
#pragma unroll
  for (int j = 0; j < NL; j++) acc = dot8(w[j], x[j], acc);
  return wave_sum(acc);
}

// Four rows per wave, one per 16-lane slot: lane (slot, t) reads chunks
// t, t+16, .. of its row's NL*16-chunk segment.
template <int NL>
__device__ __forceinline__ void load_seg(u32x4 (&dst)[NL], const uint16_t* row_seg, int t16) {
#pragma unroll
  for (int j = 0; j < NL; j++) dst[j] = ld_stream(row_seg + 8 * (t16 + 16 * j));
}

template <int NL>
__device__ __forceinline__ float seg_dot(const u32x4 (&w)[NL], const uint16_t* act, int t16) {
  float acc = 0.f;
#pragma unroll
  for (int j = 0; j < NL; j++) acc = dot8(w[j], *reinterpret_cast<const u32x4*>(act + 8 * (t16 + 16 * j)), acc);
  return row16_sum(acc);
}

// The same on register slices addressed from a base pointer with constant
// offsets (fully unrolled, so they stay in registers).
template <int NL>
__device__ __forceinline__ void load_row_p(u32x4* dst, const uint16_t* row, int lane) {
#pragma unroll
  for (int j = 0; j < NL; j++) dst[j] = ld_stream(row + 512 * j + 8 * lane);
}

template <int NL>
__device__ __forceinline__ float row_dot_p(const u32x4* w, const u32x4 (&x)[NL]) {
  float acc = 0.f;
#pragma unroll
  for (int j = 0; j < NL; j++) acc = dot8(w[j], x[j], acc);
  return wave_sum(acc);
}

template <int NL>
__device__ __forceinline__ void load_seg_p(u32x4* dst, const uint16_t* row_seg, int t16) {
#pragma unroll
  for (int j = 0; j < NL; j++) dst[j] = ld_stream(row_seg + 8 * (t16 + 16 * j));
}

template <int NL>
__device__ __forceinline__ float seg_dot_p(const u32x4* w, const uint16_t* act, int t16) {
  float acc = 0.f;
#pragma unroll
  for (int j = 0; j < NL; j++) acc = dot8(w[j], *reinterpret_cast<const u32x4*>(act + 8 * (t16 + 16 * j)), acc);
  return row16_sum(acc);
}

template <class M>
__device__ __forceinline__ const uint16_t* qkv_row(const LayerPtrs& w, int g, int vr) {
  using Dm = Dims<M>;
  if (vr < Dm::GQ * Dm::D) return w.wq + (size_t)(g * Dm::GQ * Dm::D + vr) * Dm::H;
  vr -= Dm::GQ * Dm::D;
  if (vr < Dm::D) return w.wk + (size_t)(g * Dm::D + vr) * Dm::H;
  vr -= Dm::D;
  return w.wv + (size_t)(g * Dm::D + vr) * Dm::H;
}

__device__ __forceinline__ uint32_t orderable16(uint32_t h) { return (h & 0x8000u) ? (~h & 0xffffu) : (h | 0x8000u); }

// ------------------------------------------------------------- the kernel
//
// Barrier schedule (both roles execute the same s_barrier sequence, 9 per
// layer; each role has its own loop so that the compute waves' weight
// registers and the control wave's poll buffers never share live ranges).
// Where a compute phase's result goes straight to other workgroups (QKV rows,
// o_proj and down_proj partials) the compute waves publish it themselves and
// no barrier follows the phase: the control wave starts polling right away.
//
//   per layer   control wave                          compute waves
//   ..a         h (or embedding row) -> RMSNorm        .
//   a..c        qkv exchange, q/k norm, RoPE, KV write QKV rows -> publish; K prefetch
//   c..d        .                                      scores, local (max, sum)
//   d..e        (max, sum) exchange -> global max/sum  V prefetch
//   e..f        .                                      probabilities, P@V
//   f..g        acc exchange, combine, attn exchange   .
//   g..i        o reduce-scatter, h' exchange, norm    o_proj partial rows -> publish
//   i..j        .                                      gate/up rows
//   j..k        m exchange                             .
//   k..a'       d reduce-scatter, h'' publish          down_proj partial rows -> publish
//   final       gather h, final norm | LM-head rows | argmax keys, WG 0 picks the token

#define QMK_SYNC()            \
  do {                        \
    __syncthreads();          \
    if (s.abort_flag) return; \
  } while (0)

// The step's end, control wave: gather the last layer's output h (exchange words at x_h, this XCD's
// copy), final RMSNorm into LDS for the compute waves' LM-head rows (barrier final a), then (after
// barrier final b) publish this workgroup's best (logit, row) key at x_key; workgroup 0 gathers the
// 256 keys, writes the token and advances the stream state.
template <class M>
__device__ __forceinline__ void final_control(Ctl<M>& ctl, const KArgs& a, Smem<M>& s, const Step& p, int b, int lane,
                                              uint32_t x_h, uint32_t x_key) {
  using Dm = Dims<M>;
  const int xcd = b & (kGroups - 1);
  auto stamp = [&](int point) {
    if (a.trace && lane == 0) a.trace[(size_t)point * kNumWG + b] = wall_clock64();
  };
  const auto nw_final = ctl.load_norm(a.final_norm);
  if (ctl.template gather_range<Dm::H>(x_h + xcd * Dm::H, make_tag(p.epoch, (uint32_t)((p.nl - 1) * Dm::NX + 8)),
                                              Ctl<M>::to_f32(s.x))) {
    ctl.rmsnorm(s.x, nw_final);
    if (b == 0) {
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      for (int i = lane; i < Dm::H; i += 64) {
        if (a.hidden_out) a.hidden_out[i] = (uint16_t)f32_to_bf16(s.x[i]);
        if (a.normalized_out) a.normalized_out[i] = bf16_to_f32(s.n[i]);
      }
    }
  }
  stamp(p.nl * kTracePoints + 0);
  QMK_SYNC();  // final a
  QMK_SYNC();  // final b
  stamp(p.nl * kTracePoints + 1);
  const uint32_t tk = make_tag(p.epoch, (uint32_t)(p.nl * Dm::NX));
  if (lane == 0) {
    uint64_t best = 0;
#pragma unroll
    for (int cc = 0; cc < kComputeWaves; cc++) best = s.best[cc] > best ? s.best[cc] : best;
    const uint32_t idx = 0xffffffffu - (uint32_t)best;
    const uint32_t score32 = (uint32_t)(best >> 32);
    u32x4 d;
    d.x = word(score32 >> 16, tk);
    d.y = word(idx & 0xffffu, tk);
    d.z = word(idx >> 16, tk);
    d.w = word(score32 & 0xffffu, tk);
    put4<true>(a.x, x_key + 4 * b, d);
  }
  if (b == 0) {
    uint64_t best = 0;
    const bool ok = ctl.template gather_range<kNumWG * 4>(x_key, tk, [&](int ci, u32x4 v) {
      const uint32_t idx = (v.y >> 16) | (v.z & 0xffff0000u);
      const uint32_t score32 = (v.x & 0xffff0000u) | (v.w >> 16);
      const uint64_t key = ((uint64_t)score32 << 32) | (uint64_t)(0xffffffffu - idx);
      best = key > best ? key : best;
    });
    stamp(p.nl * kTracePoints + 2);
    if (ok) {
      best = wave_max_u64_all(best);
      const int token = (int)(0xffffffffu - (uint32_t)best);
      if (lane == 0) {
        DecodeState* st = a.st;
        if (a.out_token) *a.out_token = token;
        if (p.persistent) {
          if (a.out_log) a.out_log[p.step] = token;
          st->tok = token;
          st->pos = p.pos + 1;
          st->step = p.step + 1;
          st->ran = 1;
          if (token == st->eos) st->done = 1;
        }
        st->epoch = p.epoch + (uint32_t)(p.nl * Dm::NX + 1);
      }
    }
  }
}

template <class M>
__device__ __forceinline__ void control_path(const KArgs& a, Smem<M>& s, const Step& p, int b, int lane) {
  using Dm = Dims<M>;
  const int xcd = b & (kGroups - 1), r = b >> 3;
  Ctl<M> ctl(a, s, lane);
  auto tag_of = [&](int layer, int k) { return make_tag(p.epoch, (uint32_t)(layer * Dm::NX + k)); };
  auto stamp = [&](int point) {
    if (a.trace && lane == 0) a.trace[(size_t)point * kNumWG + b] = wall_clock64();
  };
  const size_t kv_layer_stride = (size_t)Dm::NKV * a.max_seq_len * Dm::D;
  auto to_f32 = [](float* dst) { return Ctl<M>::to_f32(dst); };
  auto to_bf16 = [](uint16_t* dst) { return Ctl<M>::to_bf16(dst); };

  for (int L = 0; L < p.nl; L++) {
    const LayerPtrs& w = s.layers[L];
    const int tp = L * kTracePoints;
    stamp(tp + 0);
    // ------------------------------------------------------------ ..a
    const auto nw_in = ctl.load_norm(w.in_ln);
    if (L == 0) {
      const uint16_t* e = a.embed + (size_t)p.tok * Dm::H;
#pragma unroll
      for (int j = 0; j < Dm::LH; j++) {
        const u32x4 v = ld16(e + 512 * j + 8 * lane);
        float* d = s.x + 512 * j + 8 * lane;
        d[0] = lo_bf16(v.x); d[1] = hi_bf16(v.x); d[2] = lo_bf16(v.y); d[3] = hi_bf16(v.y);
        d[4] = lo_bf16(v.z); d[5] = hi_bf16(v.z); d[6] = lo_bf16(v.w); d[7] = hi_bf16(v.w);
      }
      ctl.rmsnorm(s.x, nw_in);
    } else if (ctl.template gather_range<Dm::H>(Dm::X_H + xcd * Dm::H, tag_of(L - 1, 8), to_f32(s.x))) {
      ctl.rmsnorm(s.x, nw_in);
    }
    stamp(tp + 1);
    QMK_SYNC();  // a
    stamp(tp + 2);
    // ------------------------------------------------------------ a..c  qkv (the compute waves publish their rows)
    {
      const uint32_t t = tag_of(L, 0);
      const uint16_t* cosr = a.cos_t + (size_t)p.pos * Dm::D;
      const uint16_t* sinr = a.sin_t + (size_t)p.pos * Dm::D;
      const auto hq = ctl.load_head(w.q_norm, cosr, sinr);
      const auto hk = ctl.load_head(w.k_norm, cosr, sinr);
      if (ctl.template gather_range<Dm::RG>(Dm::X_QKV + xcd * Dm::RG, t, to_f32(s.qkv))) {
        ctl.qk_norm_rope(hq, hk);
        const float v0 = s.qkv[(Dm::GQ + 1) * Dm::D + lane], v1 = s.qkv[(Dm::GQ + 1) * Dm::D + lane + 64];
        s.v[lane] = (uint16_t)f32_to_bf16(v0);
        s.v[lane + 64] = (uint16_t)f32_to_bf16(v1);
        if (r == 0) {
          const size_t o = L * kv_layer_stride + ((size_t)xcd * a.max_seq_len + p.pos) * Dm::D;
          a.k_cache[o + lane] = s.k[lane];
          a.k_cache[o + lane + 64] = s.k[lane + 64];
          a.v_cache[o + lane] = (uint16_t)f32_to_bf16(v0);
          a.v_cache[o + lane + 64] = (uint16_t)f32_to_bf16(v1);
        }
      }
    }
    stamp(tp + 3);
    QMK_SYNC();  // c
    QMK_SYNC();  // d
    stamp(tp + 4);
    // ------------------------------------------------------------ d..e  softmax max and sum
    {
      const uint32_t t = tag_of(L, 1);
      // lanes 0..GQ-1: merge the eight wave (max, sum) pairs of head h = lane
      float mx = -INFINITY, sm = 0.f;
      if (lane < Dm::GQ) {
#pragma unroll
        for (int c = 0; c < kComputeWaves; c++) mx = fmaxf(mx, s.wml[c][lane][0]);
#pragma unroll
        for (int c = 0; c < kComputeWaves; c++) {
          const float mc = s.wml[c][lane][0];
          sm += mc == -INFINITY ? 0.f : s.wml[c][lane][1] * exp_acc(mc - mx);
        }
      }
      if (lane < Dm::GQ) ctl.put_f32x2(true, Dm::X_ML + (xcd * kGroupSize + r) * Dm::GQ * 4 + 4 * lane, mx, sm, t);
      // gather every active workgroup's pairs: chunk i = (rank i / GQ, head i % GQ)
      float pm[2] = {-INFINITY, -INFINITY}, pl[2] = {0.f, 0.f};
      const bool ok = ctl.template gather<kGroupSize * Dm::GQ>(
          t, [&](int i) { return Dm::X_ML + (uint32_t)((xcd * kGroupSize + i / Dm::GQ) * Dm::GQ * 4 + 4 * (i % Dm::GQ)); },
          [&](int i, u32x4 v) {
            pm[i / 64] = f32_from_words(v.x, v.y);
            pl[i / 64] = f32_from_words(v.z, v.w);
          });
      if (ok) {
        // lane l holds chunks l and l+64 (64 chunks: only the first): head = l % GQ
        static_assert(kGroupSize * Dm::GQ <= 64, "one chunk per lane");
        const int h = lane % Dm::GQ;
        const bool act = (lane / Dm::GQ) < p.n_act;
        float m0 = act ? pm[0] : -INFINITY;
        static_assert(Dm::GQ == 2, "lane classes of two");
        const float gm = class2_max(m0);
        const float lsum = class2_sum((act && m0 != -INFINITY) ? pl[0] * exp_acc(m0 - gm) : 0.f);
        if (lane < Dm::GQ) {
          s.ml[h][0] = gm;
          s.ml[h][1] = lsum;
        }
      }
    }
    stamp(tp + 5);
    QMK_SYNC();  // e
    QMK_SYNC();  // f
    stamp(tp + 6);
    // ------------------------------------------------------------ f..g  P@V partials, combine, attn
    {
      const uint32_t t = tag_of(L, 2);
      // this workgroup's P@V partial: lane holds dims 2*lane, 2*lane+1 of each head
#pragma unroll
      for (int h = 0; h < Dm::GQ; h++) {
        float a0 = 0.f, a1 = 0.f;
#pragma unroll
        for (int c = 0; c < kComputeWaves; c++) {
          a0 += s.wacc[c][h][2 * lane];
          a1 += s.wacc[c][h][2 * lane + 1];
        }
        ctl.put_f32x2(true, Dm::X_ACC + (uint32_t)((xcd * kGroupSize + r) * Dm::GQ * Dm::D * 2 + h * Dm::D * 2 + 4 * lane),
                      a0, a1, t);
      }
      // combine: this workgroup owns head hh, dims 8kb..8kb+7.  Chunk i = (rank i/4,
      // dims 8kb+2(i%4), +1); lane l receives chunks l and l+64 (ranks l/4 and l/4+16).
      const int hh = r / (Dm::D / 8), kb = r % (Dm::D / 8);
      static_assert(kGroupSize * 4 == 128, "two chunks per lane");
      float v0[2] = {0.f, 0.f}, v1[2] = {0.f, 0.f};
      const bool ok2 = ctl.template gather<kGroupSize * 4>(
          t,
          [&](int i) {
            return Dm::X_ACC + (uint32_t)((xcd * kGroupSize + i / 4) * Dm::GQ * Dm::D * 2 + hh * Dm::D * 2 +
                                          (8 * kb + 2 * (i % 4)) * 2);
          },
          [&](int i, u32x4 v) {
            const bool act = (i / 4) < p.n_act;
            v0[(i / 64) & 1] = act ? f32_from_words(v.x, v.y) : 0.f;
            v1[(i / 64) & 1] = act ? f32_from_words(v.z, v.w) : 0.f;
          });
      if (ok2) {
        float s0 = v0[0] + v0[1], s1 = v1[0] + v1[1];  // ranks l/4 and l/4 + 16
        // sum over the 16 lanes of each class l % 4: row_ror:12 and row_ror:8 inside each 16-lane row
        // (lanes 0..3 read lanes 4..7, then 8..11), then the row swaps.  Lane l < 4 then holds the
        // sum over all ranks of dims 8kb+2l, +1, added as the xor butterfly adds it:
        // (v_l + v_l+4) + (v_l+8 + v_l+12), then with row 1's, then with rows 2-3's.
        s0 = dpp_add<0x12C>(s0);
        s1 = dpp_add<0x12C>(s1);
        s0 = dpp_add<0x128>(s0);
        s1 = dpp_add<0x128>(s1);
        s0 = rows_sum4(s0);
        s1 = rows_sum4(s1);
        // lanes 0 and 1 publish dims 8kb..8kb+3 (from lanes 0, 1) and 8kb+4..8kb+7 (lanes 2, 3)
        const float d2 = dpp_mov<0x88>(s0), d3 = dpp_mov<0x88>(s1);  // quad_perm [0,2,0,2]
        const float d4 = dpp_mov<0xDD>(s0), d5 = dpp_mov<0xDD>(s1);  // quad_perm [1,3,1,3]
        if (lane < 2)
          ctl.put_bf16x4(true, Dm::X_ATTN + (uint32_t)(xcd * Dm::OC + hh * Dm::D + 8 * kb + 4 * lane), d2, d3, d4, d5,
                         tag_of(L, 3));
        ctl.template gather_range<Dm::OC>(Dm::X_ATTN + xcd * Dm::OC, tag_of(L, 3), to_bf16(s.attn));
      }
    }
    stamp(tp + 7);
    QMK_SYNC();  // g
    stamp(tp + 8);
    // ------------------------------------------------------------ g..i  o reduce-scatter (the compute waves publish
    //                                                                    the partials), h', norm
    {
      const auto nw_post = ctl.load_norm(w.post_ln);
      if (ctl.reduce_rows(Dm::X_O, tag_of(L, 4), s.x, Dm::X_H2, tag_of(L, 5), xcd, r) &&
          ctl.template gather_range<Dm::H>(Dm::X_H2 + xcd * Dm::H, tag_of(L, 5), to_f32(s.h2)))
        ctl.rmsnorm(s.h2, nw_post);
    }
    stamp(tp + 9);
    QMK_SYNC();  // i
    QMK_SYNC();  // j
    stamp(tp + 10);
    // ------------------------------------------------------------ j..k  m
    {
      // one m value per lane; lane 4j publishes values 4j..4j+3, taken from its quad by DPP
      static_assert(Dm::M_WG % 4 == 0 && Dm::M_WG <= 64, "m values in whole quads of one wave");
      float mv = 0.f;
      if (lane < Dm::M_WG) {
        const float gt = s.out[lane];
        const float up = s.out[Dm::M_WG + lane];
        mv = bf16r(bf16r(__fdiv_rn(gt, 1.0f + expf(-gt))) * up);
      }
      const float m1 = quad_lane<1>(mv), m2 = quad_lane<2>(mv), m3 = quad_lane<3>(mv);
      if (lane < Dm::M_WG && (lane & 3) == 0)
        ctl.put_bf16x4(true, Dm::X_M + (uint32_t)(xcd * Dm::MS + Dm::M_WG * r + lane), mv, m1, m2, m3, tag_of(L, 6));
      ctl.template gather_range<Dm::MS>(Dm::X_M + xcd * Dm::MS, tag_of(L, 6), to_bf16(s.m));
    }
    stamp(tp + 11);
    QMK_SYNC();  // k
    stamp(tp + 12);
    // ------------------------------------------------------------ k..a'  d reduce-scatter (the compute waves publish
    //                                                                     the partials), h''
    ctl.reduce_rows(Dm::X_D, tag_of(L, 7), s.h2, Dm::X_H, tag_of(L, 8), xcd, r);
  }

  // ------------------------------------------------------------------ final
  final_control<M>(ctl, a, s, p, b, lane, Dm::X_H, Dm::X_KEY);
}

// The step's end, compute waves: LM-head rows of this workgroup (594 per workgroup, every eighth to
// each wave) against the final-normed activation, keeping the best 64-bit key (barriers final a
// and final b, matching final_control).
template <class M, bool SAMPLED>
__device__ __forceinline__ void final_compute(const KArgs& a, Smem<M>& s, const Step& p, int b, int c, int lane) {
  using Dm = Dims<M>;
  {
    u32x4 act[Dm::LH];  // the final-normed activation, loaded after barrier final a
    const int row0 = b * Dm::LM_RPW;
    const int nrows = min(Dm::V - row0, Dm::LM_RPW);
    const int nmine = (nrows - c + kComputeWaves - 1) / kComputeWaves;
    uint64_t best = 0;
    u32x4 bufA[Dm::LM_U][Dm::LH], bufB[Dm::LM_U][Dm::LH];
    auto row_of = [&](int i) { return row0 + c + kComputeWaves * i; };
    auto load_batch = [&](u32x4 (&buf)[Dm::LM_U][Dm::LH], int i0) {
#pragma unroll
      for (int u = 0; u < Dm::LM_U; u++) {
        const int i = min(i0 + u, nmine - 1);
        load_row(buf[u], a.lm_head + (size_t)row_of(i) * Dm::H, 0, lane);
      }
    };
    // key = score32 << 32 | ~row: score32 = orderable bf16 logit << 16 (greedy, the first index of
    // the maximum) or the order-preserving key of logit / T + Gumbel noise (a draw)
    const uint64_t base = SAMPLED ? draw_base(a.seed, (uint64_t)p.pos) : 0;
    auto do_batch = [&](u32x4 (&buf)[Dm::LM_U][Dm::LH], int i0) {
#pragma unroll
      for (int u = 0; u < Dm::LM_U; u++) {
        const float v = row_dot(buf[u], act);
        if (i0 + u < nmine) {
          const int row = row_of(i0 + u);
          const uint32_t hb = f32_to_bf16(v);
          uint32_t score32;
          if constexpr (SAMPLED) score32 = gumbel_key(bf16_to_f32(hb), a.temperature, base, row);
          else score32 = orderable16(hb) << 16;
          const uint64_t key = ((uint64_t)score32 << 32) | (uint64_t)(0xffffffffu - (uint32_t)row);
          best = key > best ? key : best;
          if (a.logits && lane == 0) a.logits[row] = bf16_to_f32(hb);
        }
      }
    };
    // the first batch of rows needs no activation: requested before barrier final a, it streams
    // while the control wave gathers h and applies the final norm
    load_batch(bufA, 0);
    QMK_SYNC();  // final a
    load_act(act, s.n, 0, lane);
    for (int i = 0; i < nmine; i += 2 * Dm::LM_U) {
      load_batch(bufB, i + Dm::LM_U);
      do_batch(bufA, i);
      if (i + 2 * Dm::LM_U < nmine) load_batch(bufA, i + 2 * Dm::LM_U);
      do_batch(bufB, i + Dm::LM_U);
    }
    if (lane == 0) s.best[c] = best;
  }
  QMK_SYNC();  // final b
}

// LONG: the long-context attention form; sw and pw are this wave's rows of
// SmemLong::sw and SmemLong::pw, unused otherwise.  DEEP (with LONG): the ring's
// first K batches are all requested before barrier c and its first V batches at
// barrier d, so that a wave streaming many batches starts both passes with the
// ring full.
template <class M, bool SAMPLED, bool LONG, bool DEEP = false>
__device__ __forceinline__ void compute_path(const KArgs& a, Smem<M>& s, const Step& p, int b, int c, int lane,
                                             [[maybe_unused]] float* sw, [[maybe_unused]] uint32_t* pw) {
  using Dm = Dims<M>;
  const int xcd = b & (kGroups - 1), r = b >> 3;
  const int slot = lane >> 4, t16 = lane & 15;
  const size_t kv_layer_stride = (size_t)Dm::NKV * a.max_seq_len * Dm::D;

  // Weight registers (see Dims::kStream): one layer ahead in per-phase
  // registers, or one phase ahead in a buffer shared by QKV, gate/up and down.
  constexpr bool ST = Dm::kStream;
  u32x4 w_q[ST ? 1 : Dm::RQ_W * Dm::LH];
  u32x4 w_gu[ST ? 1 : Dm::GU_W * Dm::LH];
  u32x4 w_d[ST ? 1 : Dm::OP * Dm::LD];
  u32x4 w_buf[ST ? Dm::NBUF : 1];
  u32x4 w_o[Dm::OP * Dm::LO];
  u32x4* const wq = ST ? w_buf : w_q;
  u32x4* const wgu = ST ? w_buf : w_gu;
  u32x4* const wd = ST ? w_buf : w_d;

  // o_proj / down_proj: rows ROWS_WG*r + ROWS_W*c + 4*pass + slot, this XCD's input columns
  auto rs_row = [&](int pass) { return Dm::ROWS_WG * r + Dm::ROWS_W * c + 4 * pass + slot; };
  const bool gu_up = c >= kComputeWaves / 2;
  const int gu_i = (gu_up ? c - kComputeWaves / 2 : c) * Dm::GU_W;          // within this workgroup's m values
  const int gu_m0 = Dm::MS * xcd + Dm::M_WG * r + gu_i;                     // global m index
  const int gu_out = (gu_up ? Dm::M_WG : 0) + gu_i;

  auto prefetch_qkv = [&](int layer) {
    LayerPtrs w;
    w.wq = uniform_ptr(s.layers[layer].wq);
    w.wk = uniform_ptr(s.layers[layer].wk);
    w.wv = uniform_ptr(s.layers[layer].wv);
#pragma unroll
    for (int i = 0; i < Dm::RQ_W; i++)
      load_row_p<Dm::LH>(wq + i * Dm::LH, qkv_row<M>(w, xcd, Dm::RQ_WG * r + Dm::RQ_W * c + i), lane);
  };
  // hot: read the final-norm weights (one H-wide row that every workgroup reads anyway) in place
  // of the row, for a request that only keeps the load count of every path equal
  auto prefetch_qkv_row = [&](int layer, int i, bool hot = false) {
    LayerPtrs w;
    w.wq = uniform_ptr(s.layers[layer].wq);
    w.wk = uniform_ptr(s.layers[layer].wk);
    w.wv = uniform_ptr(s.layers[layer].wv);
    const uint16_t* row = qkv_row<M>(w, xcd, Dm::RQ_WG * r + Dm::RQ_W * c + i);
    load_row_p<Dm::LH>(wq + i * Dm::LH, hot ? a.final_norm : row, lane);
  };
  auto prefetch_o = [&](int layer) {
    const uint16_t* wo_base = uniform_ptr(s.layers[layer].wo);
#pragma unroll
    for (int op = 0; op < Dm::OP; op++)
      load_seg_p<Dm::LO>(w_o + op * Dm::LO, wo_base + (size_t)rs_row(op) * Dm::QS + Dm::OC * xcd, t16);
  };
  auto prefetch_gu = [&](int layer) {
    const uint16_t* base = uniform_ptr(gu_up ? s.layers[layer].wu : s.layers[layer].wg);
#pragma unroll
    for (int i = 0; i < Dm::GU_W; i++) load_row_p<Dm::LH>(wgu + i * Dm::LH, base + (size_t)(gu_m0 + i) * Dm::H, lane);
  };
  auto prefetch_dn = [&](int layer) {
    const uint16_t* wd_base = uniform_ptr(s.layers[layer].wd);
#pragma unroll
    for (int op = 0; op < Dm::OP; op++)
      load_seg_p<Dm::LD>(wd + op * Dm::LD, wd_base + (size_t)rs_row(op) * Dm::I + Dm::MS * xcd, t16);
  };

  // EARLY (short-context form with every slice in its own registers): attention
  // runs HF's two passes, scores and the wave's (max, sum) in c..d, P@V in e..f
  // (the control wave merges the (max, sum) pairs in d..e and combines the P@V
  // partials in f..g).  A CU returns vector-memory data in order, so every
  // request is placed where the control wave's polls do not follow it closely:
  // this layer's gate/up and o_proj slices at barrier c and its down slice at i
  // (the two windows in which the control wave does not poll), and the next
  // layer's K, V and QKV rows right after the down_proj partials, where they
  // land while the control wave reduces down_proj and gathers h.  Measured
  // placements at context 1024 (direct launches) in earlier forms of this
  // kernel: with the QKV rows at i, 1,996-2,005 tok/s; QKV row 0 and gate/up
  // at c, o_proj, down and QKV row 1 at i 1,974-1,983; gate/up and both QKV
  // rows at c 1,955; the V rows requested before barrier c with the K rows
  // 1,943.  Those of this form are given where each request is issued.
  constexpr bool EARLY = !ST && !LONG;
  // EARLY: this layer's gate/up (GU_C) and o_proj (O_C) slices requested at barrier c, else at e
  constexpr bool GU_C = kGateUpAtC;
  constexpr bool O_C = kOprojAtC;
  static_assert(!EARLY || kLongContext / kGroupSize <= 32 * kKvU, "EARLY: at most one K/V batch per wave");
  prefetch_qkv(0);
  if (!ST && !EARLY) {
    prefetch_o(0);
    prefetch_gu(0);
    prefetch_dn(0);
  }

  // compute wave 0 stamps the start and end of each of its phases
  uint64_t* ctrace = a.trace ? a.trace + (size_t)(a.num_layers * kTracePoints + 3) * kNumWG : nullptr;
  auto cstamp = [&](int L, int k) {
    if (ctrace && c == 0 && lane == 0) ctrace[(size_t)(L * kComputePoints + k) * kNumWG + b] = wall_clock64();
  };
  constexpr int U = kKvU;
  auto base0_of = [&](int wave_c) { return p.p_begin + 4 * wave_c; };  // first position of a wave's batches
  for (int L = 0; L < p.nl; L++) {
    const uint16_t* kc = a.k_cache + L * kv_layer_stride + (size_t)xcd * a.max_seq_len * Dm::D;
    const uint16_t* vc = a.v_cache + L * kv_layer_stride + (size_t)xcd * a.max_seq_len * Dm::D;
    // the layer whose slices are requested one layer ahead; the last layer requests its own again
    // (L2-warm, unused), so every path issues the same loads and the compiler's counted waits
    // hold for all layers
    [[maybe_unused]] const int L_next = L + 1 < p.nl ? L + 1 : L;
    // K/V batches go straight from HBM into this wave's slots of an LDS ring
    // (kKvStages batches in flight) and are read back with the same lane
    // layout: lane (slot, t16) holds dims 8*t16..+7 of position base + 32u + slot.
    const int nb = base0_of(c) < p.p_end ? (p.p_end - base0_of(c) + 32 * U - 1) / (32 * U) : 0;  // batches of this wave
    // row0: every position loads row 0 (a request that only keeps the load count of every path equal)
    auto kv_issue_at = [&](const uint16_t* base, int j, int stage, bool row0 = false) {
      const int bpos = base0_of(c) + 32 * U * j;
#pragma unroll
      for (int u = 0; u < U; u++) {
        const int pp = bpos + 32 * u + slot;
        // positions outside this workgroup's range (and pos, whose K/V come from
        // LDS) load row 0, which every cache has; their values are never used
        const int pl = (!row0 && pp < p.p_end && pp != p.pos) ? pp : 0;
        __builtin_amdgcn_global_load_lds(as_global<void>(base + (size_t)pl * Dm::D + 8 * t16),
                                         (__attribute__((address_space(3))) void*)&s.kv[stage][c][u][0], 16, 0, 0);
      }
    };
    auto kv_issue = [&](const uint16_t* base, int j) { kv_issue_at(base, j, j % kKvStages); };
    // wait until batch j has landed: the batches issued after it may stay in flight
    auto kv_wait = [&](int j, int newer) { wait_vmcnt(U * min(kKvStages - 1, nb - 1 - j) + newer); };
    auto kv_refill = [&](const uint16_t* base, int j) {
      if (j + kKvStages < nb) {
        __builtin_amdgcn_s_waitcnt(kWaitLgkm0);  // this wave's reads of the slot are done
        kv_issue(base, j + kKvStages);
      }
    };
    QMK_SYNC();  // a
    cstamp(L, 0);
    {
      // rows RQ_W*c, +1 of this workgroup's RQ_WG q/k/v rows, published as two words
      static_assert(Dm::RQ_W == 2, "one 8-byte store per wave");
      u32x4 act[Dm::LH];
      load_act(act, s.n, 0, lane);
      const float v0 = row_dot_p<Dm::LH>(wq, act);
      const float v1 = row_dot_p<Dm::LH>(wq + Dm::LH, act);
      if (lane == 0) {
        const uint32_t t = make_tag(p.epoch, (uint32_t)(L * Dm::NX + 0));
        put2(a.x, Dm::X_QKV + xcd * Dm::RG + Dm::RQ_WG * r + Dm::RQ_W * c, word(f32_to_bf16(v0), t),
             word(f32_to_bf16(v1), t), !a.xcd_local);
      }
    }
    if (ST) prefetch_o(L);  // o_proj slice, kept through attention
    const int base0 = base0_of(c);
    cstamp(L, 1);
    // Keys of the positions before pos are in the cache already.  Batch 0 is
    // requested while the control wave exchanges q/k/v (the barrier below
    // waits for it, as it waits for every LDS write); the rest of the ring
    // fills after the barrier, behind the first batch's compute.  (Requested
    // right after barrier a instead, batch 0 measured slower: 1,946 against
    // 1,960 tok/s.)
    if constexpr (DEEP) {
      for (int j = 0; j < min(nb, kKvStages); j++) kv_issue(kc, j);
    } else if constexpr (EARLY) {
      if (nb > 0 && L == 0) kv_issue(kc, 0);  // later layers' K rows were requested after down_proj
    } else {
      if (nb > 0) kv_issue(kc, 0);
    }
    if constexpr (EARLY) {
      QMK_SYNC();  // c
      cstamp(L, 2);
      // Layer 0's V rows into ring stage 1 (its K rows are in stage 0); later layers' K and V
      // rows were requested after the previous layer's down_proj, and barrier a waited for them.
      // Then this layer's gate/up and o_proj slices.  The control wave does not poll between
      // barriers c and f, so nothing queues behind them.  (A wave without positions loads row 0
      // too: requests on every path keep the compiler's counted waits exact.)  While the V rows
      // were requested here for every layer, computing the scores before requesting the slices
      // was faster (2,136 against 2,118 tok/s over contexts 129..1152); with the K and V rows in
      // LDS at barrier c the two orders measure the same (2,178-2,180 either way; 2,155-2,156
      // against 2,152 at context 1024 with the slices first).
      if (L == 0) kv_issue_at(vc, 0, 1);
      if constexpr (GU_C) prefetch_gu(L);
      if constexpr (O_C) prefetch_o(L);
      // weight loads issued after the V rows
      constexpr int kLoadsC = (GU_C ? Dm::GU_W * Dm::LH : 0) + (O_C ? Dm::OP * Dm::LO : 0);
      // ---------------------------------------------- attention over this wave's positions
      // Lane (slot, t16) holds dims 8*t16..+7 of position base0 + 32u + slot.  Scores as HF
      // rounds them, kept in registers between the two passes.
      float m_w[Dm::GQ], l_w[Dm::GQ], acc[Dm::GQ][8];
#pragma unroll
      for (int h = 0; h < Dm::GQ; h++) {
        m_w[h] = -INFINITY;
        l_w[h] = 0.f;
#pragma unroll
        for (int i = 0; i < 8; i++) acc[h][i] = 0.f;
      }
      float sc[U][Dm::GQ];  // this lane's row's scores (-inf past the range)
      if (nb > 0) {
        u32x4 qv[Dm::GQ];
#pragma unroll
        for (int h = 0; h < Dm::GQ; h++) qv[h] = *reinterpret_cast<const u32x4*>(s.q + h * Dm::D + 8 * t16);
        const u32x4 k_now = *reinterpret_cast<const u32x4*>(s.k + 8 * t16);
#pragma unroll
        for (int u = 0; u < U; u++) {
          const int pp = base0 + 32 * u + slot;
          // the K rows landed before barrier c (it waits for every LDS write)
          const u32x4 kx = pp == p.pos ? k_now : s.kv[0][c][u][lane];
#pragma unroll
          for (int h = 0; h < Dm::GQ; h++) {
            const float x = bf16r(bf16r(row16_sum(dot8(kx, qv[h], 0.f))) * a.attn_scale);
            sc[u][h] = pp < p.p_end ? x : -INFINITY;
            m_w[h] = fmaxf(m_w[h], sc[u][h]);
          }
        }
#pragma unroll
        for (int h = 0; h < Dm::GQ; h++) {  // wave maximum over the four 16-lane rows
          float x, y;
          swap16(m_w[h], x, y);
          m_w[h] = fmaxf(x, y);
          swap32(m_w[h], x, y);
          m_w[h] = fmaxf(x, y);
        }
      }
      // the V rows have landed (layer 0's were requested at c; the others before barrier a); the
      // weight slices may stay in flight.  Waiting here, before any barrier, also tells the
      // compiler that no LDS DMA is outstanding at the barriers that follow.
      wait_vmcnt_upto<kLoadsC>();
      // HF's two passes: the wave's (max, sum of exp(s - max)) to the control wave, which merges the
      // workgroups' pairs across the XCD (barriers d..e); then bf16(exp(s - M) / L) times V.
      if (nb > 0) {
#pragma unroll
        for (int u = 0; u < U; u++) {
          const int pp = base0 + 32 * u + slot;
#pragma unroll
          for (int h = 0; h < Dm::GQ; h++) l_w[h] += pp < p.p_end ? exp_acc(sc[u][h] - m_w[h]) : 0.f;
        }
      }
#pragma unroll
      for (int h = 0; h < Dm::GQ; h++) {
        l_w[h] = rows_sum4(l_w[h]);  // the rows hold different positions, the lanes of a row the same one
        if (lane == 0) {
          s.wml[c][h][0] = m_w[h];
          s.wml[c][h][1] = l_w[h];
        }
      }
      cstamp(L, 3);
      QMK_SYNC();  // d
      QMK_SYNC();  // e
      if constexpr (!GU_C) prefetch_gu(L);
      if constexpr (!O_C) prefetch_o(L);
      cstamp(L, 4);
      if (nb > 0) {
        float gm[Dm::GQ], ginv[Dm::GQ];
#pragma unroll
        for (int h = 0; h < Dm::GQ; h++) {
          gm[h] = s.ml[h][0];
          ginv[h] = __fdiv_rn(1.0f, s.ml[h][1]);
        }
        const u32x4 v_now = *reinterpret_cast<const u32x4*>(s.v + 8 * t16);
#pragma unroll
        for (int u = 0; u < U; u++) {
          const int pp = base0 + 32 * u + slot;
          const u32x4 vx = pp == p.pos ? v_now : s.kv[1][c][u][lane];
          const float vf[8] = {lo_bf16(vx.x), hi_bf16(vx.x), lo_bf16(vx.y), hi_bf16(vx.y),
                               lo_bf16(vx.z), hi_bf16(vx.z), lo_bf16(vx.w), hi_bf16(vx.w)};
#pragma unroll
          for (int h = 0; h < Dm::GQ; h++) {
            // HF: softmax in fp32, probabilities rounded to bf16 before P@V; positions past the
            // range (they load row 0) take probability 0 and their values are not used
            const float pr = pp < p.p_end ? bf16r(exp_acc(sc[u][h] - gm[h]) * ginv[h]) : 0.f;
#pragma unroll
            for (int i = 0; i < 8; i++) acc[h][i] += pp < p.p_end ? pr * vf[i] : 0.f;
          }
        }
      }
#pragma unroll
      for (int h = 0; h < Dm::GQ; h++) {
#pragma unroll
        for (int i = 0; i < 8; i++) acc[h][i] = rows_sum4(acc[h][i]);
        if (lane < 16) {
#pragma unroll
          for (int i = 0; i < 8; i++) s.wacc[c][h][8 * t16 + i] = acc[h][i];
        }
      }
    } else {
      QMK_SYNC();  // c
      if constexpr (!DEEP)
        for (int j = 1; j < min(nb, kKvStages); j++) kv_issue(kc, j);
      cstamp(L, 2);
      // ------------------------------------------------ scores and local (max, sum)
      // position of entry i of this wave's batches (i = 8 batch + 4 u + slot)
      [[maybe_unused]] auto wave_pos = [&](int i) { return base0 + 32 * U * (i >> 3) + 32 * ((i >> 2) & 1) + (i & 3); };
      if constexpr (LONG) {
        // A batch gives each 16-lane row two positions (u = 0, 1) and two heads: four
        // partial dot products per lane, summed over the row in one transposed
        // reduction, after which lane t16 < 4 of the row owns the score of
        // (u = t16 & 1, head = (t16 >> 1) & 1) and alone scales, stores and maxes it.
        // The softmax terms are then computed once per position, one position per
        // lane, instead of once per lane of its row.
        static_assert(Dm::GQ == 2 && U == 2, "four (position, head) scores per lane and batch");
        const int own_u = t16 & 1, own_h = (t16 >> 1) & 1;
        const bool owner = t16 < 4;
        {
          u32x4 qv[Dm::GQ];
    #pragma unroll
          for (int h = 0; h < Dm::GQ; h++) qv[h] = *reinterpret_cast<const u32x4*>(s.q + h * Dm::D + 8 * t16);
          const u32x4 k_now = *reinterpret_cast<const u32x4*>(s.k + 8 * t16);
          // Scores of this wave's positions (to LDS) and their maximum; the keys of
          // the next batch are requested before the current batch is used.
          float mloc = -INFINITY;  // owners: the maximum of head own_h over their positions
          for (int j = 0; j < nb; j++) {
            const int base = base0 + 32 * U * j;
            kv_wait(j, 0);
            const int pp0 = base + slot, pp1 = base + 32 + slot;
            const u32x4 k0 = pp0 == p.pos ? k_now : s.kv[j % kKvStages][c][0][lane];
            const u32x4 k1 = pp1 == p.pos ? k_now : s.kv[j % kKvStages][c][1][lane];
            const float x = row16_sum_t4(dot8(k0, qv[0], 0.f), dot8(k0, qv[1], 0.f), dot8(k1, qv[0], 0.f),
                                         dot8(k1, qv[1], 0.f), t16);
            const float sc = bf16r(bf16r(x) * a.attn_scale);
            const int pp = own_u ? pp1 : pp0;
            if (owner && pp < p.p_end) {
              sw[own_h * kHeadStride + 8 * j + 4 * own_u + slot] = sc;
              mloc = fmaxf(mloc, sc);
            }
            kv_refill(kc, j);
          }
          // Every K batch has landed (the last wait was vmcnt(0)); saying so here
          // lets the compiler drop the vmcnt(0) it would otherwise put before the
          // next workgroup barriers, which would also wait for weight prefetches.
          wait_vmcnt(0);
          // wave maximum per head: lanes 0, 1 of each row hold head 0, lanes 2, 3 head 1
          {
            float x, y;
            mloc = fmaxf(mloc, dpp_get<0xB1>(mloc));
            swap16(mloc, x, y);
            mloc = fmaxf(x, y);
            swap32(mloc, x, y);
            mloc = fmaxf(x, y);
          }
          const float wm[2] = {__int_as_float(__builtin_amdgcn_readlane(__float_as_int(mloc), 0)),
                               __int_as_float(__builtin_amdgcn_readlane(__float_as_int(mloc), 2))};
          __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
          __builtin_amdgcn_wave_barrier();
          __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
          // sum of exp(s - max), one position per lane
          float lsum[Dm::GQ] = {0.f, 0.f};
          for (int i = lane; i < 8 * nb; i += kWave) {
            const int pp = wave_pos(i);
            if (pp < p.p_end) {
    #pragma unroll
              for (int h = 0; h < Dm::GQ; h++) lsum[h] += exp_acc(sw[h * kHeadStride + i] - wm[h]);
            }
          }
    #pragma unroll
          for (int h = 0; h < Dm::GQ; h++) {
            lsum[h] = wave_total(lsum[h]);
            if (lane == 0) {
              s.wml[c][h][0] = wm[h];
              s.wml[c][h][1] = lsum[h];
            }
          }
        }
      } else {
        {
          u32x4 qv[Dm::GQ];
    #pragma unroll
          for (int h = 0; h < Dm::GQ; h++) qv[h] = *reinterpret_cast<const u32x4*>(s.q + h * Dm::D + 8 * t16);
          const u32x4 k_now = *reinterpret_cast<const u32x4*>(s.k + 8 * t16);
          // Scores of this wave's positions (to LDS) and their maximum; the keys of
          // the next batch are requested before the current batch is used.
          float mloc[Dm::GQ];
    #pragma unroll
          for (int h = 0; h < Dm::GQ; h++) mloc[h] = -INFINITY;
          for (int j = 0; j < nb; j++) {
            const int base = base0 + 32 * U * j;
            kv_wait(j, 0);
    #pragma unroll
            for (int u = 0; u < U; u++) {
              if (base + 32 * u >= p.p_end) break;  // the rest of the batch is past this workgroup's range
              const int pp = base + 32 * u + slot;
              const u32x4 kx = pp == p.pos ? k_now : s.kv[j % kKvStages][c][u][lane];
    #pragma unroll
              for (int h = 0; h < Dm::GQ; h++) {
                float sc = row16_sum(dot8(kx, qv[h], 0.f));
                sc = bf16r(bf16r(sc) * a.attn_scale);
                if (pp < p.p_end) {
                  if (t16 == 0) s.sc[h][pp - p.p_begin] = sc;
                  mloc[h] = fmaxf(mloc[h], sc);
                }
              }
            }
            kv_refill(kc, j);
          }
          // Every K batch has landed (the last wait was vmcnt(0)); saying so here
          // lets the compiler drop the vmcnt(0) it would otherwise put before the
          // next workgroup barriers, which would also wait for weight prefetches.
          wait_vmcnt(0);
          // wave maximum over the four 16-lane rows, then the sum of exp(s - max)
          // with one exponential per position
    #pragma unroll
          for (int h = 0; h < Dm::GQ; h++) {
            float x, y;
            swap16(mloc[h], x, y);
            mloc[h] = fmaxf(x, y);
            swap32(mloc[h], x, y);
            mloc[h] = fmaxf(x, y);
          }
          __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
          __builtin_amdgcn_wave_barrier();
          __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
          float lsum[Dm::GQ];
    #pragma unroll
          for (int h = 0; h < Dm::GQ; h++) lsum[h] = 0.f;
          for (int j = 0; j < nb; j++) {
            const int base = base0 + 32 * U * j;
    #pragma unroll
            for (int u = 0; u < U; u++) {
              const int pp = base + 32 * u + slot;
              if (pp < p.p_end) {
    #pragma unroll
                for (int h = 0; h < Dm::GQ; h++) lsum[h] += exp_acc(s.sc[h][pp - p.p_begin] - mloc[h]);
              }
            }
          }
    #pragma unroll
          for (int h = 0; h < Dm::GQ; h++) {
            lsum[h] = rows_sum4(lsum[h]);  // rows hold different positions; lanes of a row the same one
            if (lane == 0) {
              s.wml[c][h][0] = mloc[h];
              s.wml[c][h][1] = lsum[h];
            }
          }
        }
      }
      cstamp(L, 3);
      QMK_SYNC();  // d
      if constexpr (DEEP) {
        // the V batches stream while the control wave exchanges (max, sum)
        for (int j = 0; j < min(nb, kKvStages); j++) kv_issue(vc, j);
        QMK_SYNC();  // e
      } else {
        if (nb > 0) kv_issue(vc, 0);
        QMK_SYNC();  // e
        for (int j = 1; j < min(nb, kKvStages); j++) kv_issue(vc, j);
      }
      cstamp(L, 4);
      // ------------------------------------------------ probabilities and P@V
      if constexpr (LONG)
      {
        const u32x4 v_now = *reinterpret_cast<const u32x4*>(s.v + 8 * t16);
        float gm[Dm::GQ], ginv[Dm::GQ];
  #pragma unroll
        for (int h = 0; h < Dm::GQ; h++) {
          gm[h] = s.ml[h][0];
          ginv[h] = __fdiv_rn(1.0f, s.ml[h][1]);
        }
        // HF: softmax in fp32, probabilities rounded to bf16 before P@V; one
        // position per lane, both heads' bf16 bits in one word
        for (int i = lane; i < 8 * nb; i += kWave) {
          const int pp = wave_pos(i);
          if (pp < p.p_end) {
            const uint32_t p0 = f32_to_bf16(exp_acc(sw[i] - gm[0]) * ginv[0]);
            const uint32_t p1 = f32_to_bf16(exp_acc(sw[kHeadStride + i] - gm[1]) * ginv[1]);
            pw[i] = p1 << 16 | p0;
          }
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        float acc[Dm::GQ][8];
  #pragma unroll
        for (int h = 0; h < Dm::GQ; h++)
  #pragma unroll
          for (int i = 0; i < 8; i++) acc[h][i] = 0.f;
        for (int j = 0; j < nb; j++) {
          const int base = base0 + 32 * U * j;
          kv_wait(j, 0);
          // the row's two positions are paired in bf16x2 operands: probabilities
          // (head h of both) and values (one dimension of both), so one dot2
          // accumulates two positions; a position past the range has probability 0
          const int pp0 = base + slot, pp1 = base + 32 + slot;
          // positions past the range loaded cache row 0, which the caller may not have written: their
          // values are replaced by 0, so that a NaN there cannot reach the sum through 0 * NaN
          const u32x4 zero = {0u, 0u, 0u, 0u};
          const u32x4 v0 = pp0 == p.pos ? v_now : pp0 < p.p_end ? s.kv[j % kKvStages][c][0][lane] : zero;
          const u32x4 v1 = pp1 == p.pos ? v_now : pp1 < p.p_end ? s.kv[j % kKvStages][c][1][lane] : zero;
          const uint32_t w0 = pp0 < p.p_end ? pw[8 * j + slot] : 0u;
          const uint32_t w1 = pp1 < p.p_end ? pw[8 * j + 4 + slot] : 0u;
          const bf16x2 pr[2] = {as_bf2(__builtin_amdgcn_perm(w1, w0, 0x05040100u)),
                                as_bf2(__builtin_amdgcn_perm(w1, w0, 0x07060302u))};
          const uint32_t va[4] = {v0.x, v0.y, v0.z, v0.w}, vb[4] = {v1.x, v1.y, v1.z, v1.w};
  #pragma unroll
          for (int k = 0; k < 4; k++) {
            const bf16x2 lo = as_bf2(__builtin_amdgcn_perm(vb[k], va[k], 0x05040100u));  // dim 2k
            const bf16x2 hi = as_bf2(__builtin_amdgcn_perm(vb[k], va[k], 0x07060302u));  // dim 2k+1
  #pragma unroll
            for (int h = 0; h < Dm::GQ; h++) {
              acc[h][2 * k] = __builtin_amdgcn_fdot2_f32_bf16(pr[h], lo, acc[h][2 * k], false);
              acc[h][2 * k + 1] = __builtin_amdgcn_fdot2_f32_bf16(pr[h], hi, acc[h][2 * k + 1], false);
            }
          }
          kv_refill(vc, j);
        }
        wait_vmcnt(0);  // every V batch has landed (see above)
        // sum the wave's four slots; lanes 0..15 then hold dims 8*t16..+7
  #pragma unroll
        for (int h = 0; h < Dm::GQ; h++) {
  #pragma unroll
          for (int i = 0; i < 8; i++) acc[h][i] = rows_sum4(acc[h][i]);
          if (lane < 16) {
  #pragma unroll
            for (int i = 0; i < 8; i++) s.wacc[c][h][8 * t16 + i] = acc[h][i];
          }
        }
      }
      else
      {
        const u32x4 v_now = *reinterpret_cast<const u32x4*>(s.v + 8 * t16);
        float gm[Dm::GQ], ginv[Dm::GQ];
  #pragma unroll
        for (int h = 0; h < Dm::GQ; h++) {
          gm[h] = s.ml[h][0];
          ginv[h] = __fdiv_rn(1.0f, s.ml[h][1]);
        }
        float acc[Dm::GQ][8];
  #pragma unroll
        for (int h = 0; h < Dm::GQ; h++)
  #pragma unroll
          for (int i = 0; i < 8; i++) acc[h][i] = 0.f;
        for (int j = 0; j < nb; j++) {
          const int base = base0 + 32 * U * j;
          kv_wait(j, 0);
  #pragma unroll
          for (int u = 0; u < U; u++) {
            if (base + 32 * u >= p.p_end) break;
            const int pp = base + 32 * u + slot;
            if (pp < p.p_end) {
              const u32x4 vx = pp == p.pos ? v_now : s.kv[j % kKvStages][c][u][lane];
              const float vf[8] = {lo_bf16(vx.x), hi_bf16(vx.x), lo_bf16(vx.y), hi_bf16(vx.y),
                                   lo_bf16(vx.z), hi_bf16(vx.z), lo_bf16(vx.w), hi_bf16(vx.w)};
  #pragma unroll
              for (int h = 0; h < Dm::GQ; h++) {
                // HF: softmax in fp32, probabilities rounded to bf16 before P@V
                const float pr = bf16r(exp_acc(s.sc[h][pp - p.p_begin] - gm[h]) * ginv[h]);
  #pragma unroll
                for (int i = 0; i < 8; i++) acc[h][i] += pr * vf[i];
              }
            }
          }
          kv_refill(vc, j);
        }
        wait_vmcnt(0);  // every V batch has landed
        // sum the wave's four slots; lanes 0..15 then hold dims 8*t16..+7
  #pragma unroll
        for (int h = 0; h < Dm::GQ; h++) {
  #pragma unroll
          for (int i = 0; i < 8; i++) acc[h][i] = rows_sum4(acc[h][i]);
          if (lane < 16) {
  #pragma unroll
            for (int i = 0; i < 8; i++) s.wacc[c][h][8 * t16 + i] = acc[h][i];
          }
        }
      }
      if (!ST && !EARLY && L + 1 < p.nl) prefetch_qkv(L + 1);
    }
    cstamp(L, 5);
    QMK_SYNC();  // f
    QMK_SYNC();  // g
    cstamp(L, 6);
#pragma unroll
    for (int op = 0; op < Dm::OP; op++) {
      // o_proj partial of row ROWS_W*c + 4*op + slot of this workgroup's rows, to every XCD's reducer
      const float v = seg_dot_p<Dm::LO>(w_o + op * Dm::LO, s.attn, t16);
      if (t16 == 0) {
        const uint32_t t = make_tag(p.epoch, (uint32_t)(L * Dm::NX + 4));
        put2(a.x, Dm::X_O + (uint32_t)((xcd * kGroupSize + r) * Dm::ROWS_WG + Dm::ROWS_W * c + 4 * op + slot) * 2,
             f32_hi_word(v, t), f32_lo_word(v, t), true);
      }
    }
    if (ST) prefetch_gu(L);
    else if (!EARLY && L + 1 < p.nl) prefetch_o(L + 1);
    cstamp(L, 7);
    QMK_SYNC();  // i
    cstamp(L, 8);
    // EARLY: this layer's down slice, then the gate/up rows (the next layer's QKV rows follow the
    // down_proj partials, with its K and V rows)
    if constexpr (EARLY) prefetch_dn(L);
    {
      u32x4 act[Dm::LH];
      load_act(act, s.n, 0, lane);
#pragma unroll
      for (int i = 0; i < Dm::GU_W; i++) {
        const float v = row_dot_p<Dm::LH>(wgu + i * Dm::LH, act);
        if (lane == 0) s.out[gu_out + i] = bf16r(v);
      }
    }
    if (ST) prefetch_dn(L);
    else if (!EARLY && L + 1 < p.nl) prefetch_gu(L + 1);
    cstamp(L, 9);
    QMK_SYNC();  // j
    QMK_SYNC();  // k
    cstamp(L, 10);
#pragma unroll
    for (int op = 0; op < Dm::OP; op++) {
      const float v = seg_dot_p<Dm::LD>(wd + op * Dm::LD, s.m, t16);
      if (t16 == 0) {
        const uint32_t t = make_tag(p.epoch, (uint32_t)(L * Dm::NX + 7));
        put2(a.x, Dm::X_D + (uint32_t)((xcd * kGroupSize + r) * Dm::ROWS_WG + Dm::ROWS_W * c + 4 * op + slot) * 2,
             f32_hi_word(v, t), f32_lo_word(v, t), true);
      }
    }
    if (ST) {
      if (L + 1 < p.nl) prefetch_qkv(L + 1);
    } else if (!EARLY && L + 1 < p.nl) {
      prefetch_dn(L + 1);
    }
    if constexpr (EARLY) {
      // The next layer's K and V rows into ring stages 0 and 1, free since this layer's
      // attention, then its QKV rows: they land while the control wave reduces down_proj and
      // gathers h (barrier a waits for them), so neither the qkv exchange's polls nor the
      // attention window wait behind the K and V rows, and the m exchange's polls no longer wait
      // behind the QKV rows.  Same-box A/B at context 1024: K and V requested in the layer's own
      // windows (K before barrier c, V after it) 2,125 tok/s; K here 2,140; K and V here
      // 2,151-2,152; the QKV rows here too instead of between the gate/up dot products 2,153
      // (over contexts 129..1152: 2,177 -> 2,184).  The last layer issues the same requests, so
      // that every path issues the same loads and the compiler's counted waits stay exact, but
      // they read one row that every workgroup of the XCD shares (row 0 of this layer's K and V
      // rows of the XCD's head, the final-norm weights): L2 hits instead of a second HBM read of
      // its own rows.
      const bool last = L + 1 == p.nl;
      if (nb > 0) kv_issue_at(a.k_cache + L_next * kv_layer_stride + (size_t)xcd * a.max_seq_len * Dm::D, 0, 0, last);
      kv_issue_at(a.v_cache + L_next * kv_layer_stride + (size_t)xcd * a.max_seq_len * Dm::D, 0, 1, last);
      prefetch_qkv_row(L_next, 0, last);
      prefetch_qkv_row(L_next, 1, last);
    }
    cstamp(L, 11);
  }

  final_compute<M, SAMPLED>(a, s, p, b, c, lane);
}

// SAMPLED: the LM-head keys are Gumbel-perturbed (temperature sampling, KArgs::temperature > 0);
// a separate instantiation so the greedy kernel carries none of it.
// LONG: the attention form for contexts beyond kLongContext (each score and
// softmax term computed once per position, P@V on bf16 pairs).  Both forms are
// exact for every context; the host picks by the step's context, because the
// long form, compiled into the same kernel, slows the short-context exchanges.
template <class M, bool SAMPLED, bool LONG, bool DEEP, class S>
__device__ __forceinline__ void decode_body(const KArgs& a, S& s) {
  using Dm = Dims<M>;
  const int b = blockIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // uniform: scalar branches on the role
  const int lane = threadIdx.x & 63;

  DecodeState* st = a.st;
  {
    // copy the per-layer pointer table (num_layers x 11 pointers) into LDS
    const int n = min(a.num_layers, kMaxLayers) * (int)(sizeof(LayerPtrs) / sizeof(void*));
    const uint64_t* src = reinterpret_cast<const uint64_t*>(a.layers);
    uint64_t* dst = reinterpret_cast<uint64_t*>(s.layers);
    for (int i = threadIdx.x; i < n; i += kBlock) dst[i] = src[i];
  }
  if (threadIdx.x == 0) {
    // One thread reads the state's error word so the whole workgroup takes the
    // same decision; a non-zero value (an earlier launch failed) makes this
    // launch a no-op until the state is reset.
    s.abort_flag = __hip_atomic_load(&st->err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0;
    // A step that fails on the device leaves -1 here, never a stale token.
    if (b == 0 && a.out_token) *a.out_token = -1;
    // `done` is written only by workgroup 0 at the end of a launch, after every workgroup of that
    // launch has read it, so all workgroups of one launch see the same value.
    s.stop_flag = (a.position < 0 && st->done != 0) ? 1 : 0;
  }
  __syncthreads();
  if (s.abort_flag) return;
  if (s.stop_flag) {
    // after the stop token: no position, cache or exchange is touched; the log gets the stop token
    // (HF pads finished sequences with pad_token_id = eos_token_id)
    if (b == 0 && threadIdx.x == 0) {
      const int step = st->step;
      if (a.out_log) a.out_log[step] = st->eos;
      st->step = step + 1;
      st->ran = 0;
    }
    return;
  }
  Step p;
  p.epoch = st->epoch;
  p.persistent = a.position < 0;
  p.pos = p.persistent ? st->pos : a.position;
  p.tok = p.persistent ? st->tok : a.token;
  p.step = p.persistent ? st->step : 0;
  p.nl = a.num_layers;
  p.C = p.pos + 1;
  if (p.pos < 0 || p.pos >= a.max_seq_len || p.tok < 0 || p.tok >= Dm::V) {
    if (b == 0 && threadIdx.x == 0) {
      const uint32_t bits = (p.pos < 0 || p.pos >= a.max_seq_len) ? kErrPosition : kErrToken;
      atomicOr(&st->err, bits);
      if (a.host_err) __hip_atomic_store(a.host_err, bits, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    }
    return;
  }
  p.chunk = (p.C + kGroupSize - 1) / kGroupSize;
  const int r = b >> 3;
  p.p_begin = min(p.C, r * p.chunk);
  p.p_end = min(p.C, p.p_begin + p.chunk);
  p.n_act = (p.C + p.chunk - 1) / p.chunk;
  if (wave == 0) {
    control_path<M>(a, s, p, b, lane);
  } else if constexpr (LONG) {
    compute_path<M, SAMPLED, true, DEEP>(a, s, p, b, wave - 1, lane, s.sw[wave - 1], s.pw[wave - 1]);
  } else {
    compute_path<M, SAMPLED, false>(a, s, p, b, wave - 1, lane, nullptr, nullptr);
  }
}

template <class M, bool SAMPLED = false, bool LONG = false>
__global__ void __launch_bounds__(kBlock, 1) decode_kernel(KArgs a) {
  __shared__ std::conditional_t<LONG, SmemLong<M>, Smem<M>> s;
  decode_body<M, SAMPLED, LONG, false>(a, s);
}

// The long form for contexts beyond kDeepContext, where each wave streams more K/V batches than
// the ring holds: both passes start with the ring full (DEEP).  Below that context, the ring's
// extra requests delay the q/k/v and (max, sum) exchanges by more than they save.
template <class M, bool SAMPLED = false>
__global__ void __launch_bounds__(kBlock, 1) decode_kernel_deep(KArgs a) {
  __shared__ SmemLong<M> s;
  decode_body<M, SAMPLED, true, true>(a, s);
}

#undef QMK_SYNC

}  // namespace qmk
