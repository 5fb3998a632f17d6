// Batched decode step for MI355X (gfx950) as one persistent kernel: B
// sequences (2 <= B <= 4), one token each, through every layer, the final
// norm, the LM head and argmax in a single launch.
//
// It is the decode kernel of qmk_decode_kernel.h with B rows per weight read:
// the same 256 workgroups x 9 waves, the same XCD tensor-parallel split (XCD x
// owns KV head x, its query heads, 256 o_proj input columns and the m slice
// [MS x, MS x + MS)), the same tagged-word exchanges (each carries the B
// sequences' payloads under one tag, so a sequence costs no extra round trip)
// and the same HF rounding points.  The compute waves stream each phase's
// weight slice once, one phase ahead, into registers and dot it against the B
// activation rows in LDS; weights are read once per step for the whole batch.
// Attention runs per sequence (each has its own context and cache) over the
// 32 workgroups of an XCD in HF's two passes: scores and a (max, sum)
// exchange, then probabilities rounded to bf16 before P@V, as HF rounds them.
// One LDS ring stage per sequence holds its K rows, then its V rows.
// Contexts up to kBatchMaxContext positions give each wave at most one K/V
// batch per sequence.  Each sequence has its own control wave, so the
// per-sequence exchanges, norms and merges of a step run side by side.
//
// It replaces the seven launches per layer of the fused batched step
// (qmk_batch.hip) for these shapes; the reference decodes one sequence
// (qwen_megakernel/model.py:111-250), so there is no reference counterpart.
//
//   k  exchange   producers -> consumers                  scope
//   0  qkv        32 WGs of XCD x -> same 32 WGs           XCD-local  [xcd][b][RG]
//   1  ml         softmax (max, sum) per WG and head       XCD-local  [xcd][rank][b][GQ*4]
//   2  acc        P@V partials per WG and head             XCD-local  [xcd][rank][b][GQ*D*2]
//   3  attn       attention output of heads 2x, 2x+1       XCD-local  [xcd][b][OC]
//   4  o          o_proj partials, rows of rank r          across     [xcd][rank][b][ROWS_WG*2]
//   5  h2         h' = h + o_proj(attn)                    XCD-local  [xcd][b][H]
//   6  m          silu(gate) * up, slice of XCD x          XCD-local  [xcd][b][MS]
//   7  d          down_proj partials                       across     [xcd][rank][b][ROWS_WG*2]
//   8  h          h'' = h' + down(m)                       XCD-local  [xcd][b][H]
//   (the tags advance by Dims::NX = 9 per layer, as in the decode kernel)

#pragma once

#include "qmk_decode_kernel.h"

namespace qmk {

constexpr int kBatchMin = 2, kBatchMax = 4;
constexpr int kBatchMaxContext = kGroupSize * 32 * kKvU;  // 2048: one K/V batch per wave and sequence
constexpr uint32_t kNoChunk = 0xffffffffu;

template <class M, int B>
struct BDims {
  using D1 = Dims<M>;
  static constexpr int H = D1::H, I = D1::I, GQ = D1::GQ, D = D1::D, V = D1::V, QS = D1::QS, NKV = D1::NKV;
  static constexpr int RG = D1::RG, RQ_WG = D1::RQ_WG, RQ_W = D1::RQ_W, LH = D1::LH, OC = D1::OC, MS = D1::MS;
  static constexpr int M_WG = D1::M_WG, GU_W = D1::GU_W, ROWS_WG = D1::ROWS_WG, ROWS_W = D1::ROWS_W;
  static constexpr int OP = D1::OP, LO = D1::LO, LD = D1::LD, LM_RPW = D1::LM_RPW, NX = D1::NX;
  static constexpr int NBUF = D1::NBUF;     // the shared weight buffer of the QKV, gate/up and down phases
  static constexpr int LMU = 2;  // LM-head rows per wave per batch (two batches in flight)
  static constexpr int CPX = ROWS_WG / 2;   // reduce-scatter: chunks per source XCD and sequence
  // exchange layout (words)
  static constexpr uint32_t X_QKV = 0;
  static constexpr uint32_t X_ML = X_QKV + kGroups * B * RG;
  static constexpr uint32_t X_ACC = X_ML + kGroups * kGroupSize * B * GQ * 4;
  static constexpr uint32_t X_ATTN = X_ACC + kGroups * kGroupSize * B * GQ * D * 2;
  static constexpr uint32_t X_O = X_ATTN + kGroups * B * OC;
  static constexpr uint32_t X_H2 = X_O + kGroups * kGroupSize * B * ROWS_WG * 2;
  static constexpr uint32_t X_M = X_H2 + kGroups * B * H;
  static constexpr uint32_t X_D = X_M + kGroups * B * MS;
  static constexpr uint32_t X_H = X_D + kGroups * kGroupSize * B * ROWS_WG * 2;
  static constexpr uint32_t X_KEY = X_H + kGroups * B * H;
  static constexpr uint32_t X_WORDS = X_KEY + kNumWG * B * 4;

  static_assert(B >= kBatchMin && B <= kBatchMax, "batch size");
  static_assert(RQ_W * B <= 8 && LMU * B <= 8, "QKV and LM-head dots reduced eight at a time");
  static_assert((kGroups * CPX * B) % 64 == 0 && kGroups * CPX * B <= 16 * 64 && (kGroups * CPX) % 64 == 0,
                "reduce-scatter: whole 64-chunk slots per sequence, at most 16 loads per lane");
  static_assert(kGroupSize * 4 == 128, "combine: two acc chunks per lane and sequence");
  static_assert(X_WORDS % 4 == 0, "alignment");
};

// Kernel arguments.  The layer table is a device copy (num_layers x 88 bytes) that the host library
// uploads once per distinct table, as the decode kernel's is; the kernel copies it into LDS.
struct BArgs {
  const LayerPtrs* layers;
  const uint16_t* embed;
  const uint16_t* final_norm;
  const uint16_t* lm_head;
  const uint16_t* cos_t;
  const uint16_t* sin_t;
  uint16_t* k_cache;       // sequence b's cache at k_cache + b * seq_stride: [layer][8][max_seq_len][128]
  uint16_t* v_cache;
  long long seq_stride;    // elements
  const int* tokens;       // [B] device
  const int* positions;    // [B] device
  int* out_tokens;         // [B] device: next greedy token, -1 for an invalid row
  float* logits;           // optional [B][V]
  DecodeState* st;         // epoch and error bits of this stream's batched kernel
  uint32_t* x;             // exchange words
  uint32_t* host_err;
  uint64_t* trace;         // optional: the decode kernel's stamp layout (control points, then compute points)
  int num_layers;
  int max_seq_len;
  int max_context;         // every valid position is below it (<= kBatchMaxContext)
  float attn_scale;
  float rms_eps;
  uint32_t timeout;
  int xcd_local;
};

template <class M, int B>
struct BSmem {
  using Dm = BDims<M, B>;
  uint16_t n[B][Dm::H];              // gathered hidden rows, normalised in place (bf16)
  float res[B][Dm::ROWS_WG];         // this rank's residual rows: h, then h'
  float qkv[B][Dm::RG];
  uint16_t q[B][Dm::GQ * Dm::D];
  uint16_t k[B][Dm::D];
  uint16_t v[B][Dm::D];
  uint16_t attn[B][Dm::OC];
  uint16_t m[B][Dm::MS];
  u32x4 kv[kKvStages][kComputeWaves][kKvU][kWave];  // K/V rows (LDS DMA)
  float wml[kComputeWaves][B][Dm::GQ][2];
  float ml[B][Dm::GQ][2];            // global softmax max and sum per sequence and head
  float wacc[kComputeWaves][B][Dm::GQ][Dm::D];
  float out[B][2 * Dm::M_WG];
  uint64_t best[kComputeWaves][B];
  LayerPtrs layers[kMaxLayers];
  int abort_flag;
  // attention hand-offs inside the workgroup, per sequence, counting up through the launch (so no
  // reset is needed): compute waves that published their (max, sum) (8 per layer), layers whose
  // global (max, sum) is in ml (set by the sequence's control wave), compute waves that published
  // their P@V partial (8 per layer)
  int sig_scores[B];
  int sig_ml[B];
  int sig_pv[B];
  int sig_attn[B];  // layers whose attention output is in attn (set by the sequence's control wave)
  int sig_n2[B];    // layers whose post-attention normed row is in n (set by the control wave)
  int sig_gu[B];    // compute waves that wrote the sequence's gate/up outputs to out (8 per layer)
  int sig_m[B];     // layers whose SiLU(gate)*up row is in m (set by the control wave)
};

// In-workgroup signals between waves through LDS.  A wave's LDS operations complete in order, so
// waiting for lgkmcnt(0) before the signal makes every LDS write the wave issued before it visible
// to a wave that has seen the signal.  They are written as inline assembly: as LDS atomics the
// compiler would put a vmcnt(0) before each of them (it cannot tell them from the K/V ring that
// the wave's LDS-DMA loads are filling), which would stall the wave on every K/V batch in flight.
__device__ __forceinline__ uint32_t lds_addr(const int* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) int*)p;
}
__device__ __forceinline__ void lds_signal_add(int* p) {
  asm volatile("s_waitcnt lgkmcnt(0)\n\tds_add_u32 %0, %1" ::"v"(lds_addr(p)), "v"(1) : "memory");
}
__device__ __forceinline__ void lds_signal_set(int* p, int v) {
  asm volatile("s_waitcnt lgkmcnt(0)\n\tds_write_b32 %0, %1" ::"v"(lds_addr(p)), "v"(v) : "memory");
}
// A 16-byte LDS store the compiler does not hold back behind the K/V ring's loads (see above); a
// later lds_signal_add orders it before the signal.
__device__ __forceinline__ void lds_store16(float* p, float4 v) {
  typedef float f32x4 __attribute__((ext_vector_type(4)));
  const f32x4 x = {v.x, v.y, v.z, v.w};
  asm volatile("ds_write_b128 %0, %1" ::"v"((uint32_t)(uintptr_t)(__attribute__((address_space(3))) float*)p), "v"(x)
               : "memory");
}
__device__ __forceinline__ int lds_read_now(const int* p) {
  int v;
  asm volatile("ds_read_b32 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=v"(v) : "v"(lds_addr(p)) : "memory");
  return __builtin_amdgcn_readfirstlane(v);
}
// Waits until *p >= v.  Returns false when the workgroup has aborted or the wait exceeded
// ``timeout`` ticks of the wall clock (the caller then records the failure).
__device__ __forceinline__ bool lds_wait_ge(int* p, int v, int* abort_flag, uint32_t timeout) {
  const uint64_t t0 = wall_clock64();
  while (lds_read_now(p) < v) {
    if (lds_read_now(abort_flag)) return false;
    if (wall_clock64() - t0 > timeout) return false;
    __builtin_amdgcn_s_sleep(1);
  }
  return true;
}

template <int B>
struct BStep {
  uint32_t epoch;
  int nl;
  int pos[B], tok[B];
  bool valid[B];
  int p_begin[B], p_end[B], n_act[B];  // this workgroup's attention positions per sequence
};

// ------------------------------------------------------------- control wave

template <class M, int B>
struct BCtl {
  using Dm = BDims<M, B>;
  const BArgs& a;
  BSmem<M, B>& s;
  int lane;

  __device__ BCtl(const BArgs& a_, BSmem<M, B>& s_, int lane_) : a(a_), s(s_), lane(lane_) {}

  __device__ void fail(uint32_t bits) {
    atomicOr(&a.st->err, bits);
    if (a.host_err) __hip_atomic_store(a.host_err, bits, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    s.abort_flag = 1;
  }

  // Waits until every chunk named by off(j) (the word offset of this lane's
  // 16-byte chunk in load slot j < NC, or kNoChunk) carries ``tag``; calls
  // sink(j, chunk) once per chunk as it arrives.  The poll rules of the decode
  // kernel's gather: rounds of one load keep two rounds in flight, larger
  // rounds one; received chunks are pointed past the buffer descriptor.
  template <int NC, class Off, class F>
  __device__ bool gather(uint32_t tag, Off&& off, F&& sink) {
    static_assert(NC >= 1 && NC <= 16, "gather size");
    auto rs = make_rsrc(a.x, 0x7fffffffu);
    uint32_t o[NC];
    uint32_t pend = 0;
#pragma unroll
    for (int j = 0; j < NC; j++) {
      const uint32_t w = off(j);
      o[j] = w == kNoChunk ? 0u : w * 4u;
      if (w != kNoChunk) pend |= 1u << j;
    }
    constexpr uint32_t kOOB = 0xfffffff0u;
    constexpr int R = NC == 1 ? 2 : 1;
    u32x4 v[R][NC];
#pragma unroll
    for (int k = 0; k < R - 1; k++)
#pragma unroll
      for (int j = 0; j < NC; j++) v[k][j] = poll16(rs, (pend & (1u << j)) ? o[j] : kOOB);
    const uint64_t t0 = wall_clock64();
    while (true) {
#pragma unroll
      for (int k = 0; k < R; k++) {
#pragma unroll
        for (int j = 0; j < NC; j++) v[(k + R - 1) % R][j] = poll16(rs, (pend & (1u << j)) ? o[j] : kOOB);
#pragma unroll
        for (int j = 0; j < NC; j++)
          if ((pend & (1u << j)) && chunk_ok(v[k][j], tag)) {
            sink(j, v[k][j]);
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

  // HF Qwen3RMSNorm of the bf16 row in place: bf16(w * bf16(x * rsqrt(mean(x^2) + eps))),
  // the sum of squares in the decode kernel's order
  __device__ void rmsnorm_inplace(uint16_t* row, const NormW& nw) {
    constexpr int P = Dm::H / 128;
    uint32_t* r2 = reinterpret_cast<uint32_t*>(row);
    float2 xv[P];
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < P; i++) {
      const uint32_t u = r2[lane + 64 * i];
      xv[i] = make_float2(lo_bf16(u), hi_bf16(u));
      ss += xv[i].x * xv[i].x + xv[i].y * xv[i].y;
    }
    ss = wave_sum(ss);
    // the mean: H is a power of two, so the product with 1/H is the correctly rounded quotient
    static_assert((Dm::H & (Dm::H - 1)) == 0, "H a power of two");
    const float rstd = rcp_sqrt_torch(ss * (1.0f / Dm::H) + a.rms_eps);
    // two elements per conversion: bf16(x * rstd), then bf16(w * that)
#pragma unroll
    for (int i = 0; i < P; i++) {
      const uint32_t wp = nw.w[i];
      const uint32_t xn = pack_bf16x2(xv[i].x * rstd, xv[i].y * rstd);
      r2[lane + 64 * i] = pack_bf16x2(lo_bf16(wp) * lo_bf16(xn), hi_bf16(wp) * hi_bf16(xn));
    }
  }

  // Per-head RMSNorm + rotate-half RoPE (elements lane, lane + 64) of the GQ q heads and the k
  // head at qkv, into q and k.  Each head's sum of squares is reduced on its own; the correctly
  // rounded 1/sqrt of head h's mean is evaluated in lane h, once for all heads, and read back.
  __device__ void qk_norm_rope(const float* qkv, float qw0, float qw1, float kw0, float kw1, float c0, float c1,
                               float s0, float s1, uint16_t* q, uint16_t* k) {
    constexpr int NH = Dm::GQ + 1;
    static_assert((Dm::D & (Dm::D - 1)) == 0, "head_dim a power of two");
    float x0[NH], x1[NH], v = 0.f;
#pragma unroll
    for (int h = 0; h < NH; h++) {
      x0[h] = qkv[h * Dm::D + lane];
      x1[h] = qkv[h * Dm::D + lane + 64];
      const float ss = wave_sum(x0[h] * x0[h] + x1[h] * x1[h]);
      v = lane == h ? ss : v;
    }
    const float rl = rcp_sqrt_torch(v * (1.0f / Dm::D) + a.rms_eps);
#pragma unroll
    for (int h = 0; h < NH; h++) {
      const float rstd = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(rl), h));
      const bool isq = h < Dm::GQ;
      uint16_t* dst = isq ? q + h * Dm::D : k;
      // the lane's two elements share each bf16 conversion
      const uint32_t xn = pack_bf16x2(x0[h] * rstd, x1[h] * rstd);
      const uint32_t nn = pack_bf16x2((isq ? qw0 : kw0) * lo_bf16(xn), (isq ? qw1 : kw1) * hi_bf16(xn));
      const float n0 = lo_bf16(nn), n1 = hi_bf16(nn);
      // x*cos + rotate_half(x)*sin with rotate_half(x) = (-x[64:], x[:64]), each product rounded
      const uint32_t pc = pack_bf16x2(n0 * c0, n1 * c1);
      const uint32_t ps = pack_bf16x2(-n1 * s0, n0 * s1);
      const uint32_t y = pack_bf16x2(lo_bf16(pc) + lo_bf16(ps), hi_bf16(pc) + hi_bf16(ps));
      dst[lane] = (uint16_t)(y & 0xffffu);
      dst[lane + 64] = (uint16_t)(y >> 16);
    }
  }

  // Reduce-scatter across XCDs for sequence sb: sums the eight XCD partials of
  // this rank's ROWS_WG rows (fixed order), adds the residual s.res[sb] and
  // rounds like HF, bf16(res + bf16(sum)); keeps the result as the next
  // residual and publishes the rows into this XCD's copy of x_dst.
  __device__ bool reduce_rows(uint32_t x_src, uint32_t src_tag, uint32_t x_dst, uint32_t dst_tag, int xcd, int r,
                              int sb) {
    constexpr int R = Dm::ROWS_WG, CPX = Dm::CPX;
    constexpr int NSL = kGroups * CPX / 64;  // load slots
    float part0[NSL], part1[NSL];
    // chunk k = 64 j + lane: source XCD k / CPX, row pair k % CPX
    const bool ok = gather<NSL>(
        src_tag,
        [&](int j) {
          const int k = j * 64 + lane;
          return x_src + (uint32_t)((((k / CPX) * kGroupSize + r) * B + sb) * R * 2 + (k % CPX) * 4);
        },
        [&](int j, u32x4 v) {
          part0[j] = f32_from_words(v.x, v.y);
          part1[j] = f32_from_words(v.z, v.w);
        });
    if (!ok) return false;
    // lane l < CPX sums row pair l over the sources in order 0..7, each fetched from the lane that
    // received it, (src * CPX) % 64 lanes ahead, by row swaps
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
    float sum0 = 0.f, sum1 = 0.f;
#pragma unroll
    for (int src = 0; src < kGroups; src++) {
      sum0 += p0[src];
      sum1 += p1[src];
    }
    uint32_t hb0 = 0, hb1 = 0;
    if (lane < CPX) {
      const uint32_t sbits = pack_bf16x2(sum0, sum1);
      const uint32_t hb = pack_bf16x2(s.res[sb][2 * lane] + lo_bf16(sbits), s.res[sb][2 * lane + 1] + hi_bf16(sbits));
      s.res[sb][2 * lane] = lo_bf16(hb);
      s.res[sb][2 * lane + 1] = hi_bf16(hb);
      hb0 = hb & 0xffffu;
      hb1 = hb >> 16;
    }
    const uint32_t ob0 = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)hb0, 0xB1, 0xf, 0xf, false);  // lane ^ 1
    const uint32_t ob1 = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)hb1, 0xB1, 0xf, 0xf, false);
    if (lane < CPX && (lane & 1) == 0) {
      u32x4 d;
      d.x = word(hb0, dst_tag);
      d.y = word(hb1, dst_tag);
      d.z = word(ob0, dst_tag);
      d.w = word(ob1, dst_tag);
      put(true, x_dst + (uint32_t)((xcd * B + sb) * Dm::H + R * r + 2 * lane), d);
    }
    return true;
  }

  // Sequence sb's NW-word vector at base + sb * NW: sink(ci, chunk) for chunk ci < NW / 4.
  template <int NW, class F>
  __device__ bool gather_seq(uint32_t base, int sb, uint32_t tag, F&& sink) {
    static_assert(NW % 4 == 0, "whole chunks");
    constexpr int NCH = NW / 4, NCS = (NCH + 63) / 64;
    return gather<NCS>(
        tag,
        [&](int j) {
          const int ci = j * 64 + lane;
          return ci < NCH ? base + (uint32_t)(sb * NW + 4 * ci) : kNoChunk;
        },
        [&](int j, u32x4 v) { sink(j * 64 + lane, v); });
  }
};

#define QMK_BSYNC()           \
  do {                        \
    __syncthreads();          \
    if (s.abort_flag) return; \
  } while (0)

// Barrier schedule per layer (every wave): a, c, d, e, f, g, i, j, k; then final a, final b.
// Control wave b (b < B) moves sequence b's activations; the compute waves serve all sequences.
//
//   per layer   control wave b                            compute waves
//   ..a         h rows of sequence b -> RMSNorm            .
//   a..c        qkv exchange, q/k norm, RoPE, KV append    QKV rows -> publish; o_proj slice; K rows of seq 0
//   c..d        .                                          scores and the wave's (max, sum) per sequence
//   d..e        (max, sum) exchange -> global max, sum     V rows requested
//   e..f        .                                          probabilities, P@V per sequence
//   f..g        acc exchange, combine, attn exchange       .
//   g..i        o reduce-scatter, h' exchange, norm        o_proj partials -> publish; gate/up slice
//   i..j        .                                          gate/up rows; down slice
//   j..k        m exchange                                 .
//   k..a'       d reduce-scatter, h'' publish              down partials -> publish; next QKV slice
template <class M, int B>
__device__ __forceinline__ void batch_control(const BArgs& a, BSmem<M, B>& s, const BStep<B>& p, int wg, int sb,
                                              int lane) {
  using Dm = BDims<M, B>;
  const int xcd = wg & (kGroups - 1), r = wg >> 3;
  BCtl<M, B> ctl(a, s, lane);
  auto tag_of = [&](int layer, int k) { return make_tag(p.epoch, (uint32_t)(layer * Dm::NX + k)); };
  auto stamp = [&](int point) {
    if (a.trace && sb == 0 && lane == 0) a.trace[(size_t)point * kNumWG + wg] = wall_clock64();
  };
  // this wave's sequence (uniform selects, no indexed register arrays)
  int pos = 0, tok = 0, n_act = 0;
  bool valid = false;
#pragma unroll
  for (int b = 0; b < B; b++)
    if (b == sb) {
      pos = p.pos[b];
      tok = p.tok[b];
      n_act = p.n_act[b];
      valid = p.valid[b];
    }
  const size_t kv_layer_stride = (size_t)Dm::NKV * a.max_seq_len * Dm::D;
  uint16_t* const n = s.n[sb];
  auto to_n = [&](int ci, u32x4 v) {
    uint32_t* d = reinterpret_cast<uint32_t*>(n) + 2 * ci;
    d[0] = (v.x >> 16) | (v.y & 0xffff0000u);
    d[1] = (v.z >> 16) | (v.w & 0xffff0000u);
  };

  for (int L = 0; L < p.nl; L++) {
    // The lane index is made opaque once per layer, so the addresses derived from it are
    // recomputed where they are used instead of being hoisted out of the layer loop and spilled.
    asm volatile("" : "+v"(lane));
    ctl.lane = lane;
    const LayerPtrs& w = s.layers[L];
    const int tp = L * kTracePoints;
    stamp(tp + 0);
    // ------------------------------------------------------------ ..a  h row, RMSNorm
    {
      const auto nw_in = ctl.load_norm(w.in_ln);
      bool ok = true;
      if (L == 0) {
        const uint16_t* e = a.embed + (size_t)tok * Dm::H;
#pragma unroll
        for (int j = 0; j < Dm::LH; j++)
          *reinterpret_cast<u32x4*>(n + 512 * j + 8 * lane) = ld16(e + 512 * j + 8 * lane);
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        // the residual rows this rank reduces
        for (int i = lane; i < Dm::ROWS_WG; i += kWave) s.res[sb][i] = bf16_to_f32(n[Dm::ROWS_WG * r + i]);
      } else {
        ok = ctl.template gather_seq<Dm::H>(Dm::X_H + xcd * B * Dm::H, sb, tag_of(L - 1, 8), to_n);
      }
      if (ok) ctl.rmsnorm_inplace(n, nw_in);
    }
    stamp(tp + 1);
    QMK_BSYNC();  // a
    stamp(tp + 2);
    // ------------------------------------------------------------ a..c  qkv (the compute waves publish their rows)
    {
      const float qw0 = bf16_to_f32(ldu16(w.q_norm + lane)), qw1 = bf16_to_f32(ldu16(w.q_norm + lane + 64));
      const float kw0 = bf16_to_f32(ldu16(w.k_norm + lane)), kw1 = bf16_to_f32(ldu16(w.k_norm + lane + 64));
      const uint16_t* cosr = a.cos_t + (size_t)pos * Dm::D;
      const uint16_t* sinr = a.sin_t + (size_t)pos * Dm::D;
      const float c0 = bf16_to_f32(ldu16(cosr + lane)), c1 = bf16_to_f32(ldu16(cosr + lane + 64));
      const float s0 = bf16_to_f32(ldu16(sinr + lane)), s1 = bf16_to_f32(ldu16(sinr + lane + 64));
      float* const qkv = s.qkv[sb];
      const bool ok = ctl.template gather_seq<Dm::RG>(Dm::X_QKV + xcd * B * Dm::RG, sb, tag_of(L, 0),
                                                       [&](int ci, u32x4 v) {
                                                         float* d = qkv + 4 * ci;
                                                         d[0] = bf16_to_f32(v.x >> 16);
                                                         d[1] = bf16_to_f32(v.y >> 16);
                                                         d[2] = bf16_to_f32(v.z >> 16);
                                                         d[3] = bf16_to_f32(v.w >> 16);
                                                       });
      if (ok) {
        ctl.qk_norm_rope(qkv, qw0, qw1, kw0, kw1, c0, c1, s0, s1, s.q[sb], s.k[sb]);
        const float v0 = qkv[(Dm::GQ + 1) * Dm::D + lane], v1 = qkv[(Dm::GQ + 1) * Dm::D + lane + 64];
        s.v[sb][lane] = (uint16_t)f32_to_bf16(v0);
        s.v[sb][lane + 64] = (uint16_t)f32_to_bf16(v1);
        if (r == 0 && valid) {
          const size_t o = (size_t)sb * a.seq_stride + L * kv_layer_stride + ((size_t)xcd * a.max_seq_len + pos) * Dm::D;
          a.k_cache[o + lane] = s.k[sb][lane];
          a.k_cache[o + lane + 64] = s.k[sb][lane + 64];
          a.v_cache[o + lane] = (uint16_t)f32_to_bf16(v0);
          a.v_cache[o + lane + 64] = (uint16_t)f32_to_bf16(v1);
        }
      }
    }
    stamp(tp + 3);
    QMK_BSYNC();  // c
    // the compute waves' (max, sum) of this sequence (they score the sequences in order, so the
    // exchange of an early sequence overlaps the scores of the later ones)
    if (!lds_wait_ge(&s.sig_scores[sb], kComputeWaves * (L + 1), &s.abort_flag, a.timeout)) ctl.fail(kErrTimeout);
    stamp(tp + 4);
    // ------------------------------------------------------------ softmax max and sum
    {
      const uint32_t t = tag_of(L, 1);
      // lanes 0..GQ-1 merge the eight waves' (max, sum) of head h = lane and publish them
      if (lane < Dm::GQ) {
        float mx = -INFINITY, sm = 0.f;
#pragma unroll
        for (int c = 0; c < kComputeWaves; c++) mx = fmaxf(mx, s.wml[c][sb][lane][0]);
#pragma unroll
        for (int c = 0; c < kComputeWaves; c++) {
          const float mc = s.wml[c][sb][lane][0];
          sm += mc == -INFINITY ? 0.f : s.wml[c][sb][lane][1] * exp_acc(mc - mx);
        }
        ctl.put_f32x2(true, Dm::X_ML + (uint32_t)(((xcd * kGroupSize + r) * B + sb) * Dm::GQ * 4 + 4 * lane), mx, sm,
                      t);
      }
      // lane l receives (rank l / GQ, head l % GQ); ranks past the active range hold no positions
      static_assert(kGroupSize * Dm::GQ == 64, "one chunk per lane");
      float pm = -INFINITY, pl = 0.f;
      const bool ok = ctl.template gather<1>(
          t,
          [&](int) {
            return Dm::X_ML + (uint32_t)(((xcd * kGroupSize + lane / Dm::GQ) * B + sb) * Dm::GQ * 4 + 4 * (lane % Dm::GQ));
          },
          [&](int, u32x4 v) {
            const bool act = lane / Dm::GQ < n_act;
            pm = act ? f32_from_words(v.x, v.y) : -INFINITY;
            pl = act ? f32_from_words(v.z, v.w) : 0.f;
          });
      if (ok) {
        static_assert(Dm::GQ == 2, "lane classes of two");
        const float gm = class2_max(pm);
        const float lsum = class2_sum(pm == -INFINITY ? 0.f : pl * exp_acc(pm - gm));
        if (lane < Dm::GQ) {
          s.ml[sb][lane][0] = gm;
          s.ml[sb][lane][1] = lsum;
        }
      }
      // set even after a failed exchange, so no compute wave waits for it (the abort flag is set)
      if (lane == 0) lds_signal_set(&s.sig_ml[sb], L + 1);
    }
    stamp(tp + 5);
    if (!lds_wait_ge(&s.sig_pv[sb], kComputeWaves * (L + 1), &s.abort_flag, a.timeout)) ctl.fail(kErrTimeout);
    stamp(tp + 6);
    // ------------------------------------------------------------ f..g  P@V partials, combine, attn
    {
      const uint32_t t = tag_of(L, 2);
      const uint32_t slot = (uint32_t)((xcd * kGroupSize + r) * B + sb);
      // this workgroup's P@V partial (the waves' in a fixed order); lane holds dims 2 lane, 2 lane + 1
#pragma unroll
      for (int h = 0; h < Dm::GQ; h++) {
        float a0 = 0.f, a1 = 0.f;
#pragma unroll
        for (int c = 0; c < kComputeWaves; c++) {
          a0 += s.wacc[c][sb][h][2 * lane];
          a1 += s.wacc[c][sb][h][2 * lane + 1];
        }
        ctl.put_f32x2(true, Dm::X_ACC + slot * Dm::GQ * Dm::D * 2 + h * Dm::D * 2 + 4 * lane, a0, a1, t);
      }
      // combine: this workgroup owns head hh, dims 8kb..8kb+7.  Slot j: acc chunk (rank
      // 16 j + lane / 4, dims 8kb + 2(lane%4), +1).
      const int hh = r / (Dm::D / 8), kb = r % (Dm::D / 8);
      float v0[2] = {0.f, 0.f}, v1[2] = {0.f, 0.f};
      const bool ok2 = ctl.template gather<2>(
          t,
          [&](int j) {
            const int rank = j * 16 + lane / 4;
            return Dm::X_ACC + (uint32_t)(((xcd * kGroupSize + rank) * B + sb) * Dm::GQ * Dm::D * 2 + hh * Dm::D * 2 +
                                          (8 * kb + 2 * (lane % 4)) * 2);
          },
          [&](int j, u32x4 v) {
            const bool act = j * 16 + lane / 4 < n_act;
            v0[j] = act ? f32_from_words(v.x, v.y) : 0.f;
            v1[j] = act ? f32_from_words(v.z, v.w) : 0.f;
          });
      if (ok2) {
        float x0 = v0[0] + v0[1];
        float x1 = v1[0] + v1[1];
        // sum over the 16 lanes of each class lane % 4: row_ror:12 and row_ror:8 inside each 16-lane
        // row (lanes 0..3 read lanes 4..7, then 8..11), then the row swaps; lane l < 4 then holds the
        // sum over all ranks of dims 8kb + 2l, +1, in the xor butterfly's order
        x0 = rows_sum4(dpp_add<0x128>(dpp_add<0x12C>(x0)));
        x1 = rows_sum4(dpp_add<0x128>(dpp_add<0x12C>(x1)));
        // lanes 0 and 1 publish dims 8kb..8kb+3 (from lanes 0, 1) and 8kb+4..8kb+7 (lanes 2, 3)
        const float d2 = dpp_mov<0x88>(x0), d3 = dpp_mov<0x88>(x1);  // quad_perm [0,2,0,2]
        const float d4 = dpp_mov<0xDD>(x0), d5 = dpp_mov<0xDD>(x1);  // quad_perm [1,3,1,3]
        if (lane < 2)
          ctl.put_bf16x4(true, Dm::X_ATTN + (uint32_t)((xcd * B + sb) * Dm::OC + hh * Dm::D + 8 * kb + 4 * lane), d2,
                         d3, d4, d5, tag_of(L, 3));
        uint16_t* const at = s.attn[sb];
        ctl.template gather_seq<Dm::OC>(Dm::X_ATTN + xcd * B * Dm::OC, sb, tag_of(L, 3), [&](int ci, u32x4 v) {
          uint32_t* d = reinterpret_cast<uint32_t*>(at) + 2 * ci;
          d[0] = (v.x >> 16) | (v.y & 0xffff0000u);
          d[1] = (v.z >> 16) | (v.w & 0xffff0000u);
        });
      }
    }
    // set even after a failed exchange, so no compute wave waits for it (the abort flag is set)
    if (lane == 0) lds_signal_set(&s.sig_attn[sb], L + 1);
    stamp(tp + 7);
    stamp(tp + 8);
    // ------------------------------------------------------------ g..i  o reduce-scatter, h', norm
    {
      const auto nw_post = ctl.load_norm(w.post_ln);
      if (ctl.reduce_rows(Dm::X_O, tag_of(L, 4), Dm::X_H2, tag_of(L, 5), xcd, r, sb) &&
          ctl.template gather_seq<Dm::H>(Dm::X_H2 + xcd * B * Dm::H, sb, tag_of(L, 5), to_n))
        ctl.rmsnorm_inplace(n, nw_post);
      // set even after a failed exchange, so no compute wave waits for it (the abort flag is set)
      if (lane == 0) lds_signal_set(&s.sig_n2[sb], L + 1);
    }
    stamp(tp + 9);
    // the sequence's gate/up outputs (the compute waves take the sequences in pairs)
    if (!lds_wait_ge(&s.sig_gu[sb], kComputeWaves * (L + 1), &s.abort_flag, a.timeout)) ctl.fail(kErrTimeout);
    stamp(tp + 10);
    // ------------------------------------------------------------ j..k  m
    {
      // one m value per lane; lane 4j publishes values 4j..4j+3, taken from its quad by DPP
      static_assert(Dm::M_WG % 4 == 0 && Dm::M_WG <= 64, "m values in whole quads of one wave");
      float mv = 0.f;
      if (lane < Dm::M_WG) {
        const float gt = s.out[sb][lane];
        const float up = s.out[sb][Dm::M_WG + lane];
        mv = bf16r(bf16r(__fdiv_rn(gt, 1.0f + expf(-gt))) * up);
      }
      const float m1 = quad_lane<1>(mv), m2 = quad_lane<2>(mv), m3 = quad_lane<3>(mv);
      if (lane < Dm::M_WG && (lane & 3) == 0)
        ctl.put_bf16x4(true, Dm::X_M + (uint32_t)((xcd * B + sb) * Dm::MS + Dm::M_WG * r + lane), mv, m1, m2, m3,
                       tag_of(L, 6));
      uint16_t* const mm = s.m[sb];
      ctl.template gather_seq<Dm::MS>(Dm::X_M + xcd * B * Dm::MS, sb, tag_of(L, 6), [&](int ci, u32x4 v) {
        uint32_t* d = reinterpret_cast<uint32_t*>(mm) + 2 * ci;
        d[0] = (v.x >> 16) | (v.y & 0xffff0000u);
        d[1] = (v.z >> 16) | (v.w & 0xffff0000u);
      });
      // set even after a failed exchange, so no compute wave waits for it (the abort flag is set)
      if (lane == 0) lds_signal_set(&s.sig_m[sb], L + 1);
    }
    stamp(tp + 11);
    stamp(tp + 12);
    // ------------------------------------------------------------ k..a'  d reduce-scatter, h''
    ctl.reduce_rows(Dm::X_D, tag_of(L, 7), Dm::X_H, tag_of(L, 8), xcd, r, sb);
  }

  // ------------------------------------------------------------------ final
  {
    const auto nw_final = ctl.load_norm(a.final_norm);
    if (ctl.template gather_seq<Dm::H>(Dm::X_H + xcd * B * Dm::H, sb, tag_of(p.nl - 1, 8), to_n))
      ctl.rmsnorm_inplace(n, nw_final);
  }
  stamp(p.nl * kTracePoints + 0);
  QMK_BSYNC();  // final a
  QMK_BSYNC();  // final b
  stamp(p.nl * kTracePoints + 1);
  const uint32_t tk = make_tag(p.epoch, (uint32_t)(p.nl * Dm::NX));
  if (lane == 0) {
    uint64_t best = 0;
#pragma unroll
    for (int cc = 0; cc < kComputeWaves; cc++) best = s.best[cc][sb] > best ? s.best[cc][sb] : best;
    const uint32_t idx = 0xffffffffu - (uint32_t)best;
    const uint32_t score32 = (uint32_t)(best >> 32);
    u32x4 d;
    d.x = word(score32 >> 16, tk);
    d.y = word(idx & 0xffffu, tk);
    d.z = word(idx >> 16, tk);
    d.w = word(score32 & 0xffffu, tk);
    put4<true>(a.x, Dm::X_KEY + 4 * (wg * B + sb), d);
  }
  if (wg == 0) {
    // sequence sb's key of workgroup 64 j + lane
    uint64_t best = 0;
    const bool ok = ctl.template gather<kNumWG / 64>(
        tk, [&](int j) { return Dm::X_KEY + 4u * (uint32_t)((64 * j + lane) * B + sb); },
        [&](int j, u32x4 v) {
          const uint32_t idx = (v.y >> 16) | (v.z & 0xffff0000u);
          const uint32_t score32 = (v.x & 0xffff0000u) | (v.w >> 16);
          const uint64_t key = ((uint64_t)score32 << 32) | (uint64_t)(0xffffffffu - idx);
          best = key > best ? key : best;
        });
    stamp(p.nl * kTracePoints + 2);
    if (ok) {
      best = wave_max_u64(best);
      if (lane == 0) {
        a.out_tokens[sb] = valid ? (int)(0xffffffffu - (uint32_t)best) : -1;
        // the tags of the next launch; it starts after every wave of this one has finished
        if (sb == 0) a.st->epoch = p.epoch + (uint32_t)(p.nl * Dm::NX + 1);
      }
    }
  }
}

template <class M, int B>
__device__ __forceinline__ void batch_compute(const BArgs& a, BSmem<M, B>& s, const BStep<B>& p, int wg, int c,
                                              int lane) {
  using Dm = BDims<M, B>;
  const int xcd = wg & (kGroups - 1), r = wg >> 3;
  const size_t kv_layer_stride = (size_t)Dm::NKV * a.max_seq_len * Dm::D;
  constexpr int U = kKvU;

  u32x4 w_buf[Dm::NBUF];         // QKV, gate/up and down slices, one phase ahead
  u32x4 w_o[Dm::OP * Dm::LO];    // o_proj slice, requested after QKV and kept through attention

  // the lambdas read ``lane`` itself, which is laundered per layer, so their lane-derived addresses
  // are not hoisted out of the layer loop
  auto rs_row = [&](int pass) { return Dm::ROWS_WG * r + Dm::ROWS_W * c + 4 * pass + (lane >> 4); };
  const bool gu_up = c >= kComputeWaves / 2;
  const int gu_i = (gu_up ? c - kComputeWaves / 2 : c) * Dm::GU_W;
  const int gu_m0 = Dm::MS * xcd + Dm::M_WG * r + gu_i;
  const int gu_out = (gu_up ? Dm::M_WG : 0) + gu_i;

  auto prefetch_qkv = [&](int layer) {
    LayerPtrs w;
    w.wq = uniform_ptr(s.layers[layer].wq);
    w.wk = uniform_ptr(s.layers[layer].wk);
    w.wv = uniform_ptr(s.layers[layer].wv);
#pragma unroll
    for (int i = 0; i < Dm::RQ_W; i++)
      load_row_p<Dm::LH>(w_buf + i * Dm::LH, qkv_row<M>(w, xcd, Dm::RQ_WG * r + Dm::RQ_W * c + i), lane);
  };
  auto prefetch_o = [&](int layer) {
    const uint16_t* wo_base = uniform_ptr(s.layers[layer].wo);
#pragma unroll
    for (int op = 0; op < Dm::OP; op++)
      load_seg_p<Dm::LO>(w_o + op * Dm::LO, wo_base + (size_t)rs_row(op) * Dm::QS + Dm::OC * xcd, lane & 15);
  };
  auto prefetch_gu = [&](int layer, int i0, int i1) {
    const uint16_t* base = uniform_ptr(gu_up ? s.layers[layer].wu : s.layers[layer].wg);
#pragma unroll
    for (int i = i0; i < i1; i++)
      load_row_p<Dm::LH>(w_buf + i * Dm::LH, base + (size_t)(gu_m0 + i) * Dm::H, lane);
  };
  auto prefetch_dn = [&](int layer) {
    const uint16_t* wd_base = uniform_ptr(s.layers[layer].wd);
#pragma unroll
    for (int op = 0; op < Dm::OP; op++)
      load_seg_p<Dm::LD>(w_buf + op * Dm::LD, wd_base + (size_t)rs_row(op) * Dm::I + Dm::MS * xcd, lane & 15);
  };

  uint64_t* ctrace = a.trace ? a.trace + (size_t)(a.num_layers * kTracePoints + 3) * kNumWG : nullptr;
  auto cstamp = [&](int L, int k) {
    if (ctrace && c == 0 && lane == 0) ctrace[(size_t)(L * kComputePoints + k) * kNumWG + wg] = wall_clock64();
  };
  prefetch_qkv(0);
  for (int L = 0; L < p.nl; L++) {
    asm volatile("" : "+v"(lane));  // addresses derived from the lane are recomputed per layer, not hoisted
    const int slot = lane >> 4, t16 = lane & 15;
    auto cache_of = [&](uint16_t* base, int b) {
      return base + (size_t)b * a.seq_stride + L * kv_layer_stride + (size_t)xcd * a.max_seq_len * Dm::D;
    };
    // Sequence b's K (then V) rows go to ring stage b.  Lane (slot, t16) holds dims 8*t16..+7 of
    // position p_begin + 4c + 32u + slot; positions outside this workgroup's range (and pos, whose
    // K/V come from LDS) load row 0, never used.
    auto issue_kv = [&](int b, bool vrows) {
      const uint16_t* base = cache_of(vrows ? a.v_cache : a.k_cache, b);
      const int base0 = p.p_begin[b] + 4 * c;
#pragma unroll
      for (int u = 0; u < U; u++) {
        const int pp = base0 + 32 * u + slot;
        const int pl = (pp < p.p_end[b] && pp != p.pos[b]) ? pp : 0;
        __builtin_amdgcn_global_load_lds(as_global<void>(base + (size_t)pl * Dm::D + 8 * t16),
                                         (__attribute__((address_space(3))) void*)&s.kv[b][c][u][0], 16, 0, 0);
      }
    };
    QMK_BSYNC();  // a
    cstamp(L, 0);
    {
      // value k = RQ_W b + row; lanes 8k.. receive its sum, lane 8k publishes it
      float v8[8];
#pragma unroll
      for (int k = 0; k < 8; k++) v8[k] = 0.f;
#pragma unroll
      for (int b = 0; b < B; b++) {
        u32x4 act[Dm::LH];
        load_act(act, s.n[b], 0, lane);
#pragma unroll
        for (int i = 0; i < Dm::RQ_W; i++) v8[Dm::RQ_W * b + i] = row_part<Dm::LH>(w_buf + i * Dm::LH, act);
      }
      const float tot = wave_sum8(v8, lane);
      const int k = lane >> 3;
      if ((lane & 7) == 0 && k < Dm::RQ_W * B) {
        const uint32_t t = make_tag(p.epoch, (uint32_t)(L * Dm::NX + 0));
        put1(a.x, Dm::X_QKV + (xcd * B + k / Dm::RQ_W) * Dm::RG + Dm::RQ_WG * r + Dm::RQ_W * c + k % Dm::RQ_W,
             word(f32_to_bf16(tot), t), !a.xcd_local);
      }
    }
    prefetch_o(L);
    issue_kv(0, false);  // sequence 0's keys stream while the control waves exchange q/k/v
    cstamp(L, 1);
    QMK_BSYNC();  // c
    cstamp(L, 2);
    // ---------------------------------------------- attention, HF's two passes
    // Pass 1 (c..d): this wave's scores per sequence, kept in registers, and the wave's softmax
    // (max, sum); the control waves merge them over the XCD's workgroups (d..e) while the V rows
    // land in the ring.  Pass 2 (e..f): probabilities bf16(exp(s - M) / L), rounded where HF
    // rounds them, times the V rows.
    static_assert(B <= kKvStages, "one ring stage per sequence");
#pragma unroll
    for (int b = 1; b < B; b++) issue_kv(b, false);
    float sc[B][U][Dm::GQ];
#pragma unroll
    for (int b = 0; b < B; b++) {
      // sequence b's keys; the later sequences' keys and the earlier sequences' V rows, issued
      // after them, may stay in flight
      wait_vmcnt(U * (B - 1));
      const int base0 = p.p_begin[b] + 4 * c;
      float m_w[Dm::GQ], l_w[Dm::GQ];
#pragma unroll
      for (int h = 0; h < Dm::GQ; h++) {
        m_w[h] = -INFINITY;
        l_w[h] = 0.f;
      }
      if (base0 < p.p_end[b]) {
        u32x4 qv[Dm::GQ];
#pragma unroll
        for (int h = 0; h < Dm::GQ; h++) qv[h] = *reinterpret_cast<const u32x4*>(s.q[b] + h * Dm::D + 8 * t16);
        const u32x4 k_now = *reinterpret_cast<const u32x4*>(s.k[b] + 8 * t16);
#pragma unroll
        for (int u = 0; u < U; u++) {
          // a row group past the workgroup's range (u = 1 for every wave at contexts up to 1024)
          // is skipped with a wave-uniform branch
          if (base0 + 32 * u >= p.p_end[b]) {
#pragma unroll
            for (int h = 0; h < Dm::GQ; h++) sc[b][u][h] = -INFINITY;
            continue;
          }
          const int pp = base0 + 32 * u + slot;
          const u32x4 kx = pp == p.pos[b] ? k_now : s.kv[b][c][u][lane];
#pragma unroll
          for (int h = 0; h < Dm::GQ; h++) {
            const float x = bf16r(bf16r(row16_sum(dot8(kx, qv[h], 0.f))) * a.attn_scale);
            sc[b][u][h] = pp < p.p_end[b] ? x : -INFINITY;
            m_w[h] = fmaxf(m_w[h], sc[b][u][h]);
          }
        }
#pragma unroll
        for (int h = 0; h < Dm::GQ; h++) {
          float x, y;
          swap16(m_w[h], x, y);
          m_w[h] = fmaxf(x, y);
          swap32(m_w[h], x, y);
          m_w[h] = fmaxf(x, y);
#pragma unroll
          for (int u = 0; u < U; u++)
            if (base0 + 32 * u + slot < p.p_end[b]) l_w[h] += exp_acc(sc[b][u][h] - m_w[h]);
          l_w[h] = rows_sum4(l_w[h]);  // rows hold different positions, a row's lanes the same one
        }
      } else {
#pragma unroll
        for (int u = 0; u < U; u++)
#pragma unroll
          for (int h = 0; h < Dm::GQ; h++) sc[b][u][h] = -INFINITY;
      }
      if (lane == 0) {
#pragma unroll
        for (int h = 0; h < Dm::GQ; h++) {
          s.wml[c][b][h][0] = m_w[h];
          s.wml[c][b][h][1] = l_w[h];
        }
        lds_signal_add(&s.sig_scores[b]);
      }
      // sequence b's V rows replace its keys in this wave's slots of ring stage b (this wave's
      // reads of them are done: the signal waited for them, and lgkmcnt(0) covers every lane)
      __builtin_amdgcn_s_waitcnt(kWaitLgkm0);
      issue_kv(b, true);
    }
    cstamp(L, 3);
    auto fail_here = [&]() {
      atomicOr(&a.st->err, kErrTimeout);
      if (a.host_err) __hip_atomic_store(a.host_err, kErrTimeout, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
      s.abort_flag = 1;
    };
#pragma unroll
    for (int b = 0; b < B; b++) {
      // the sequence's global (max, sum), then its V rows (the later sequences' may stay in flight)
      if (!lds_wait_ge(&s.sig_ml[b], L + 1, &s.abort_flag, a.timeout) && !lds_read_now(&s.abort_flag)) fail_here();
      if (b == 0) cstamp(L, 4);
      wait_vmcnt(U * (B - b - 1));
      const int base0 = p.p_begin[b] + 4 * c;
      float acc[Dm::GQ][8];
#pragma unroll
      for (int h = 0; h < Dm::GQ; h++)
#pragma unroll
        for (int i = 0; i < 8; i++) acc[h][i] = 0.f;
      if (base0 < p.p_end[b]) {
        const u32x4 v_now = *reinterpret_cast<const u32x4*>(s.v[b] + 8 * t16);
        float gm[Dm::GQ], ginv[Dm::GQ];
#pragma unroll
        for (int h = 0; h < Dm::GQ; h++) {
          gm[h] = s.ml[b][h][0];
          ginv[h] = __fdiv_rn(1.0f, s.ml[b][h][1]);
        }
#pragma unroll
        for (int u = 0; u < U; u++) {
          if (base0 + 32 * u >= p.p_end[b]) continue;  // wave-uniform, as in pass 1
          const int pp = base0 + 32 * u + slot;
          const u32x4 vx = pp == p.pos[b] ? v_now : s.kv[b][c][u][lane];
          const float vf[8] = {lo_bf16(vx.x), hi_bf16(vx.x), lo_bf16(vx.y), hi_bf16(vx.y),
                               lo_bf16(vx.z), hi_bf16(vx.z), lo_bf16(vx.w), hi_bf16(vx.w)};
#pragma unroll
          for (int h = 0; h < Dm::GQ; h++) {
            // HF: softmax in fp32, probabilities rounded to bf16 before P@V; positions past the
            // range (which load row 0) get probability 0
            const float pr = pp < p.p_end[b] ? bf16r(exp_acc(sc[b][u][h] - gm[h]) * ginv[h]) : 0.f;
            // a position past the range (it loaded cache row 0, which the caller may not have written)
            // leaves the sum untouched, so that a NaN there cannot enter it through 0 * NaN
#pragma unroll
            for (int i = 0; i < 8; i++) acc[h][i] = pp < p.p_end[b] ? __builtin_fmaf(pr, vf[i], acc[h][i]) : acc[h][i];
          }
        }
      }
      // the wave's four 16-lane rows summed for all 16 values at once: a half-wave swap halves
      // the values each lane carries, a row-pair swap halves them again; lane (t16, row) then
      // holds values 4 (row & 1) + j of head row >> 1, dims 8 t16 + 4 (row & 1) + j
      static_assert(Dm::GQ == 2, "16 accumulators per lane");
      float w8[8];
#pragma unroll
      for (int j = 0; j < 8; j++) {
        const auto r2 = __builtin_amdgcn_permlane32_swap(__float_as_uint(acc[0][j]), __float_as_uint(acc[1][j]),
                                                         false, false);
        w8[j] = __uint_as_float(r2[0]) + __uint_as_float(r2[1]);  // lanes 0-31: head 0, 32-63: head 1
      }
      float4 z;
      float* zf = reinterpret_cast<float*>(&z);
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const auto r2 = __builtin_amdgcn_permlane16_swap(__float_as_uint(w8[j]), __float_as_uint(w8[j + 4]), false,
                                                         false);
        zf[j] = __uint_as_float(r2[0]) + __uint_as_float(r2[1]);  // even rows: dims j, odd rows: dims j + 4
      }
      lds_store16(&s.wacc[c][b][lane >> 5][8 * t16 + 4 * ((lane >> 4) & 1)], z);
      if (lane == 0) lds_signal_add(&s.sig_pv[b]);
    }
    // every K/V item has landed (the last wait was vmcnt(0)); saying so lets the compiler drop the
    // vmcnt(0) it would otherwise put before the next workgroup barrier
    wait_vmcnt(0);
    // half of the gate/up slice now, half after o_proj: the first half drains during the
    // attention-output exchanges, and the polls of the o reduce-scatter queue behind only the second
    prefetch_gu(L, 0, Dm::GU_W / 2);
    cstamp(L, 5);
    // o_proj partials, each sequence's as soon as its attention output is in LDS: its chunks are
    // read from LDS once and serve every row pass
#pragma unroll
    for (int b = 0; b < B; b++) {
      if (!lds_wait_ge(&s.sig_attn[b], L + 1, &s.abort_flag, a.timeout) && !lds_read_now(&s.abort_flag)) fail_here();
      if (b == 0) cstamp(L, 6);
      u32x4 xa[Dm::LO];
#pragma unroll
      for (int j = 0; j < Dm::LO; j++) xa[j] = *reinterpret_cast<const u32x4*>(s.attn[b] + 8 * (t16 + 16 * j));
#pragma unroll
      for (int op = 0; op < Dm::OP; op++) {
        const float v = row16_sum(row_part<Dm::LO>(w_o + op * Dm::LO, xa));
        if (t16 == 0) {
          const uint32_t t = make_tag(p.epoch, (uint32_t)(L * Dm::NX + 4));
          put2(a.x, Dm::X_O + (uint32_t)(((xcd * kGroupSize + r) * B + b) * Dm::ROWS_WG + Dm::ROWS_W * c + 4 * op + slot) * 2,
               f32_hi_word(v, t), f32_lo_word(v, t), true);
        }
      }
    }
    prefetch_gu(L, Dm::GU_W / 2, Dm::GU_W);
    cstamp(L, 7);
    {
      // Sequences in passes of SB, their activation rows read from LDS once and held in registers;
      // the partial dots of a pass are summed eight at a time: value k of group g is row
      // RPG g + k / SB of sequence b0 + k % SB.
      constexpr int SB = B > 2 ? 2 : B;
      constexpr int RPG = 8 / SB;
      constexpr int NG = (Dm::GU_W + RPG - 1) / RPG;
#pragma unroll
      for (int b0 = 0; b0 < B; b0 += SB) {
        // the pass's post-attention normed rows
#pragma unroll
        for (int j = 0; j < SB; j++)
          if (b0 + j < B && !lds_wait_ge(&s.sig_n2[b0 + j], L + 1, &s.abort_flag, a.timeout) &&
              !lds_read_now(&s.abort_flag))
            fail_here();
        if (b0 == 0) cstamp(L, 8);
        u32x4 act[SB][Dm::LH];
#pragma unroll
        for (int j = 0; j < SB; j++)
          if (b0 + j < B) load_act(act[j], s.n[b0 + j], 0, lane);
#pragma unroll
        for (int g = 0; g < NG; g++) {
          float v8[8];
#pragma unroll
          for (int k = 0; k < 8; k++) v8[k] = 0.f;
#pragma unroll
          for (int q = 0; q < RPG; q++)
#pragma unroll
            for (int j = 0; j < SB; j++)
              if (RPG * g + q < Dm::GU_W && b0 + j < B)
                v8[SB * q + j] = row_part<Dm::LH>(w_buf + (RPG * g + q) * Dm::LH, act[j]);
          const float tot = wave_sum8(v8, lane);
          const int k = lane >> 3, row = RPG * g + k / SB, bj = b0 + k % SB;
          if ((lane & 7) == 0 && k < RPG * SB && row < Dm::GU_W && bj < B) s.out[bj][gu_out + row] = bf16r(tot);
        }
        if (lane == 0) {
#pragma unroll
          for (int j = 0; j < SB; j++)
            if (b0 + j < B) lds_signal_add(&s.sig_gu[b0 + j]);
        }
      }
    }
    prefetch_dn(L);
    cstamp(L, 9);
    // down_proj partials, each sequence's as soon as its m row is in LDS
#pragma unroll
    for (int b = 0; b < B; b++) {
      if (!lds_wait_ge(&s.sig_m[b], L + 1, &s.abort_flag, a.timeout) && !lds_read_now(&s.abort_flag)) fail_here();
      if (b == 0) cstamp(L, 10);
      u32x4 xm[Dm::LD];
#pragma unroll
      for (int j = 0; j < Dm::LD; j++) xm[j] = *reinterpret_cast<const u32x4*>(s.m[b] + 8 * (t16 + 16 * j));
#pragma unroll
      for (int op = 0; op < Dm::OP; op++) {
        const float v = row16_sum(row_part<Dm::LD>(w_buf + op * Dm::LD, xm));
        if (t16 == 0) {
          const uint32_t t = make_tag(p.epoch, (uint32_t)(L * Dm::NX + 7));
          put2(a.x, Dm::X_D + (uint32_t)(((xcd * kGroupSize + r) * B + b) * Dm::ROWS_WG + Dm::ROWS_W * c + 4 * op + slot) * 2,
               f32_hi_word(v, t), f32_lo_word(v, t), true);
        }
      }
    }
    if (L + 1 < p.nl) prefetch_qkv(L + 1);
    cstamp(L, 11);
  }

  // ------------------------------------------------------------ LM head
  {
    constexpr int LMU = Dm::LMU;
    u32x4 act[B][Dm::LH];  // the final-normed rows, loaded after barrier final a
    const int row0 = wg * Dm::LM_RPW;
    const int nrows = min(Dm::V - row0, Dm::LM_RPW);
    const int nmine = (nrows - c + kComputeWaves - 1) / kComputeWaves;
    // lanes 8k.. hold value k = B u + b of every batch (row u of the batch, sequence b) after the
    // eight-way reduction; each lane keeps the best key of its value
    const int kv = lane >> 3;
    const int kb = kv % B;
    const bool kval = kv < LMU * B;
    uint64_t best = 0;
    u32x4 bufA[LMU][Dm::LH], bufB[LMU][Dm::LH];
    auto row_of = [&](int i) { return row0 + c + kComputeWaves * i; };
    auto load_batch = [&](u32x4 (&buf)[LMU][Dm::LH], int i0) {
#pragma unroll
      for (int u = 0; u < LMU; u++) {
        const int i = min(i0 + u, nmine - 1);
        load_row(buf[u], a.lm_head + (size_t)row_of(i) * Dm::H, 0, lane);
      }
    };
    auto do_batch = [&](u32x4 (&buf)[LMU][Dm::LH], int i0) {
      float v8[8];
#pragma unroll
      for (int k = 0; k < 8; k++) v8[k] = 0.f;
#pragma unroll
      for (int u = 0; u < LMU; u++)
#pragma unroll
        for (int b = 0; b < B; b++) v8[B * u + b] = row_part<Dm::LH>(buf[u], act[b]);
      const float tot = wave_sum8(v8, lane);
      const int iu = i0 + kv / B;
      if (kval && iu < nmine) {
        const int row = row_of(iu);
        const uint32_t hb = f32_to_bf16(tot);
        const uint64_t key = ((uint64_t)(orderable16(hb) << 16) << 32) | (uint64_t)(0xffffffffu - (uint32_t)row);
        best = key > best ? key : best;
        if (a.logits && (lane & 7) == 0) a.logits[(size_t)kb * Dm::V + row] = bf16_to_f32(hb);
      }
    };
    load_batch(bufA, 0);
    QMK_BSYNC();  // final a
#pragma unroll
    for (int b = 0; b < B; b++) load_act(act[b], s.n[b], 0, lane);
    for (int i = 0; i < nmine; i += 2 * LMU) {
      load_batch(bufB, i + LMU);
      do_batch(bufA, i);
      if (i + 2 * LMU < nmine) load_batch(bufA, i + 2 * LMU);
      do_batch(bufB, i + LMU);
    }
#pragma unroll
    for (int b = 0; b < B; b++) {
      const uint64_t kb_best = wave_max_u64(kval && kb == b ? best : 0);
      if (lane == 0) s.best[c][b] = kb_best;
    }
  }
  QMK_BSYNC();  // final b
}

template <int B>
constexpr int batch_block() { return (B + kComputeWaves) * kWave; }

template <class M, int B>
__global__ void __launch_bounds__(batch_block<B>(), 1) batch_decode_kernel(BArgs a) {
  using Dm = BDims<M, B>;
  __shared__ BSmem<M, B> s;
  const int wg = blockIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  // a step that fails (or is skipped after an earlier failure) leaves -1, never a stale token
  if (wg == 0 && (int)threadIdx.x < B) a.out_tokens[threadIdx.x] = -1;
  {
    const int n = min(a.num_layers, kMaxLayers) * (int)(sizeof(LayerPtrs) / sizeof(void*));
    const uint64_t* src = reinterpret_cast<const uint64_t*>(a.layers);
    uint64_t* dst = reinterpret_cast<uint64_t*>(s.layers);
    for (int i = threadIdx.x; i < n; i += batch_block<B>()) dst[i] = src[i];
  }
  if (threadIdx.x == 0) s.abort_flag = __hip_atomic_load(&a.st->err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0;
  if ((int)threadIdx.x < B) {
    s.sig_scores[threadIdx.x] = 0;
    s.sig_ml[threadIdx.x] = 0;
    s.sig_pv[threadIdx.x] = 0;
    s.sig_attn[threadIdx.x] = 0;
    s.sig_n2[threadIdx.x] = 0;
    s.sig_gu[threadIdx.x] = 0;
    s.sig_m[threadIdx.x] = 0;
  }
  __syncthreads();
  if (s.abort_flag) return;
  BStep<B> p;
  p.epoch = a.st->epoch;
  p.nl = a.num_layers;
  const int r = wg >> 3;
#pragma unroll
  for (int b = 0; b < B; b++) {
    const int tok = a.tokens[b], pos = a.positions[b];
    // an invalid row (token outside the vocabulary, position outside [0, max_context)) runs as
    // token 0 at position 0 without touching its cache, and emits -1
    p.valid[b] = tok >= 0 && tok < Dm::V && pos >= 0 && pos < a.max_context;
    p.tok[b] = p.valid[b] ? tok : 0;
    p.pos[b] = p.valid[b] ? pos : 0;
    const int C = p.pos[b] + 1;
    const int chunk = (C + kGroupSize - 1) / kGroupSize;
    p.p_begin[b] = min(C, r * chunk);
    p.p_end[b] = min(C, p.p_begin[b] + chunk);
    p.n_act[b] = (C + chunk - 1) / chunk;
  }
  if (wave < B) batch_control<M, B>(a, s, p, wg, wave, lane);
  else batch_compute<M, B>(a, s, p, wg, wave - B, lane);
}

#undef QMK_BSYNC

}  // namespace qmk
