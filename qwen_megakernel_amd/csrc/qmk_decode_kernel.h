// Qwen3 batch-1 bf16 decode step for MI355X (gfx950): one persistent kernel
// launch per token (28 decoder layers, final norm, tied LM head and argmax).
//
// Replaces the reference's ldg_decode_kernel_direct / _persistent +
// ldg_lm_head_fused + ldg_update_step (reference csrc/kernel.cu:1189-1440).
// The reference splits the work over 128 blocks of 16 warps that meet at
// global atomic barriers (csrc/kernel.cu:94-119); here 256 workgroups (one per
// CU, so b % 8 is the XCD) hand activations to each other through tagged words
// (qmk_device.h), with no barrier anywhere:
//
//   phase   producers -> consumers           exchange (words)
//   QKV     256 WGs   -> the 32 WGs of an XCD  q/k/v of one KV-head group (512)
//   ATT     32 WGs    -> same 32 WGs           split-K softmax partials
//   COMB    32 WGs    -> all                   attention output (2048)
//   O       all       -> all                   h' = h + o_proj(attn) (1024)
//   GU      all       -> all                   m = silu(gate) * up (3072)
//   DOWN    all       -> all                   h'' = h' + down(m) (1024)
//   LMHEAD  all       -> WG 0                  (logit, index) argmax keys
//
// Numerics follow HF Qwen3's bf16 eager path: every op output is rounded to
// bf16 where HF rounds it (norm outputs, projections, q/k norm, RoPE products
// and sum, attention scores and output, residual adds, SiLU and its product,
// logits); dot products accumulate in fp32.  One deliberate difference: the
// softmax probabilities are not rounded to bf16 before the PV product (the
// split-K combine rescales unnormalised partials).
//
// Each workgroup has 9 waves.  Wave 0 ("control") moves activations: it polls
// exchanges, applies norms/RoPE/residuals/SiLU, publishes results and fills
// LDS.  Waves 1..8 ("compute") hold the current and next layer's weight
// slices in VGPRs: each phase's weights are requested one layer before they
// are used, so HBM streams while the control waves wait on exchanges.  The
// control wave never has weight loads outstanding, so its polls are not
// ordered behind them.

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "qmk_device.h"
#include "qmk_state.h"

namespace qmk {

struct Qwen3_0_6B {
  static constexpr int H = 1024, I = 3072, NQ = 16, NKV = 8, D = 128, V = 151936;
};

template <class M>
struct Dims {
  static constexpr int H = M::H, I = M::I, NQ = M::NQ, NKV = M::NKV, D = M::D, V = M::V;
  static constexpr int QS = NQ * D;             // attention output width
  static constexpr int GQ = NQ / NKV;           // query heads per KV head
  static constexpr int RG = (GQ + 2) * D;       // q+k+v rows of one KV-head group
  static constexpr int RQ_WG = RG / kGroupSize; // QKV rows per workgroup
  static constexpr int RQ_W = RQ_WG / kComputeWaves;
  static constexpr int LH = H / 512;            // 16-byte chunks per lane for a K=H row
  static constexpr int O_ROWS = H / kNumWG;
  static constexpr int O_WPR = kComputeWaves / O_ROWS;   // waves per O row
  static constexpr int LO = (QS / 512) / O_WPR;
  static constexpr int M_WG = I / kNumWG;
  static constexpr int GU_W = 2 * M_WG / kComputeWaves;  // gate/up rows per wave
  static constexpr int D_ROWS = H / kNumWG;
  static constexpr int D_WPR = kComputeWaves / D_ROWS;
  static constexpr int LD = (I / 512) / D_WPR;
  static constexpr int LM_RPW = (V + kNumWG - 1) / kNumWG;
  static constexpr int LM_U = 4;                         // LM-head rows per batch per wave
  static constexpr int N_X_PER_LAYER = 6;
  // exchange layout (words)
  static constexpr int PART_HEAD = 4 + 2 * D;          // m, l (2 words each) + acc
  static constexpr int PART_WG = GQ * PART_HEAD;
  static constexpr uint32_t X_QKV = 0;
  static constexpr uint32_t X_PART = X_QKV + kGroups * RG;
  static constexpr uint32_t X_ATTN = X_PART + kGroups * kGroupSize * PART_WG;
  static constexpr uint32_t X_H2 = X_ATTN + QS;
  static constexpr uint32_t X_M = X_H2 + H;
  static constexpr uint32_t X_H = X_M + I;
  static constexpr uint32_t X_KEY = X_H + H;
  static constexpr uint32_t X_WORDS = X_KEY + kNumWG * 4;

  static_assert(RG % kGroupSize == 0 && RQ_WG % kComputeWaves == 0, "QKV split");
  static_assert(RQ_WG % 4 == 0 && (GQ * D) % RQ_WG == 0 && D % RQ_WG == 0, "QKV block inside one projection");
  static_assert(H % 512 == 0 && QS % 512 == 0 && I % 512 == 0, "row chunks");
  static_assert(O_ROWS * O_WPR == kComputeWaves && D_ROWS * D_WPR == kComputeWaves, "row split");
  static_assert(2 * M_WG == GU_W * kComputeWaves && M_WG % 4 == 0, "gate/up split");
  static_assert(GQ * (D / 8) == kGroupSize, "combine: one (head, 8-dim block) per group member");
  static_assert(H % 256 == 0 && QS % 256 == 0 && I % 256 == 0 && RG % 256 == 0, "gather granularity");
  static_assert(O_ROWS == 4 && D_ROWS == 4, "publish of four residual rows per workgroup");
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
  uint32_t timeout;
  int xcd_local;           // 1: XCD-local exchanges stay in the XCD's L2
};

__device__ __forceinline__ float rcp_sqrt_torch(float v) {
  // torch CPU rsqrt = 1 / sqrt(x), each correctly rounded
  return __fdiv_rn(1.0f, __fsqrt_rn(v));
}

template <class M>
struct Smem {
  using Dm = Dims<M>;
  float x[Dm::H];                    // layer input (residual), bf16 values
  float h2[Dm::H];                   // post-attention hidden
  uint16_t n[Dm::H];                 // normalised activation (bf16)
  uint16_t attn[Dm::QS];
  uint16_t m[Dm::I];
  float qkv[Dm::RG];
  uint16_t q[Dm::GQ * Dm::D];
  uint16_t k[Dm::D];
  uint16_t v[Dm::D];
  float wp[kComputeWaves][Dm::GQ][Dm::D + 2];
  uint32_t comb[kGroupSize][20];
  float out[32];
  uint64_t best[kComputeWaves];
  int abort_flag;
};

// ------------------------------------------------------------- control wave

template <class M>
struct Ctl {
  using Dm = Dims<M>;
  const KArgs& a;
  Smem<M>& s;
  int lane;
  uint32_t epoch;

  __device__ Ctl(const KArgs& a_, Smem<M>& s_, int lane_, uint32_t epoch_) : a(a_), s(s_), lane(lane_), epoch(epoch_) {}

  __device__ void fail(uint32_t bits) {
    atomicOr(&a.st->err, bits);
    if (a.host_err) __hip_atomic_store(a.host_err, bits, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    s.abort_flag = 1;
  }

  // Wait until the NW words at ``buf`` all carry ``tag``; hand each 16-byte
  // chunk (chunk index, 4 words) to ``sink``.
  template <int NW, class F>
  __device__ bool gather(const uint32_t* buf, uint32_t tag, F&& sink) {
    constexpr int NC = NW / 256;
    static_assert(NW % 256 == 0 && NC <= 32, "gather size");
    auto rs = make_rsrc(buf, NW * 4);
    u32x4 v[NC];
    uint32_t pend = NC == 32 ? 0xffffffffu : ((1u << NC) - 1u);
    const uint64_t t0 = wall_clock64();
    while (true) {
#pragma unroll
      for (int j = 0; j < NC; j++)
        if (pend & (1u << j)) v[j] = poll16(rs, (uint32_t)(j * 64 + lane) * 16u);
#pragma unroll
      for (int j = 0; j < NC; j++)
        if ((pend & (1u << j)) && chunk_ok(v[j], tag)) pend &= ~(1u << j);
      if (!__any(pend != 0)) break;
      if (wall_clock64() - t0 > a.timeout) { fail(kErrTimeout); return false; }
    }
#pragma unroll
    for (int j = 0; j < NC; j++) sink(j * 64 + lane, v[j]);
    return true;
  }

  template <bool DEVICE>
  __device__ void publish4(uint32_t w, float v0, float v1, float v2, float v3, uint32_t tag) {
    u32x4 d;
    d.x = word(f32_to_bf16(v0), tag);
    d.y = word(f32_to_bf16(v1), tag);
    d.z = word(f32_to_bf16(v2), tag);
    d.w = word(f32_to_bf16(v3), tag);
    put4<DEVICE>(a.x, w, d);
  }

  // RMSNorm of ``src`` (fp32 holding bf16 values) with bf16 weight -> s.n:
  // bf16(w * bf16(x * rsqrt(mean(x^2) + eps)))  (HF Qwen3RMSNorm).
  __device__ void rmsnorm(const float* src, const uint16_t* w) {
    constexpr int P = Dm::H / 128;  // element pairs per lane
    float2 xv[P];
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < P; i++) {
      xv[i] = reinterpret_cast<const float2*>(src)[lane + 64 * i];
      ss += xv[i].x * xv[i].x + xv[i].y * xv[i].y;
    }
    ss = wave_sum(ss);
    const float rstd = rcp_sqrt_torch(__fdiv_rn(ss, (float)Dm::H) + a.rms_eps);
    const uint32_t* w2 = reinterpret_cast<const uint32_t*>(w);
#pragma unroll
    for (int i = 0; i < P; i++) {
      const int pi = lane + 64 * i;
      const uint32_t wp = w2[pi];
      const float n0 = bf16r(lo_bf16(wp) * bf16r(xv[i].x * rstd));
      const float n1 = bf16r(hi_bf16(wp) * bf16r(xv[i].y * rstd));
      reinterpret_cast<uint32_t*>(s.n)[pi] = f32_to_bf16(n0) | (f32_to_bf16(n1) << 16);
    }
  }

  // Per-head RMSNorm + rotate-half RoPE of one 128-wide head held in s.qkv.
  __device__ void head_norm_rope(int src_off, const uint16_t* w, const uint16_t* cosr, const uint16_t* sinr,
                                 uint16_t* dst) {
    const float x0 = s.qkv[src_off + lane], x1 = s.qkv[src_off + lane + 64];
    const float ss = wave_sum(x0 * x0 + x1 * x1);
    const float rstd = rcp_sqrt_torch(__fdiv_rn(ss, (float)Dm::D) + a.rms_eps);
    const float n0 = bf16r(bf16_to_f32(w[lane]) * bf16r(x0 * rstd));
    const float n1 = bf16r(bf16_to_f32(w[lane + 64]) * bf16r(x1 * rstd));
    const float c0 = bf16_to_f32(cosr[lane]), c1 = bf16_to_f32(cosr[lane + 64]);
    const float s0 = bf16_to_f32(sinr[lane]), s1 = bf16_to_f32(sinr[lane + 64]);
    // q*cos + rotate_half(q)*sin with rotate_half(q) = (-q[64:], q[:64])
    const float y0 = bf16r(bf16r(n0 * c0) + bf16r(-n1 * s0));
    const float y1 = bf16r(bf16r(n1 * c1) + bf16r(n0 * s1));
    dst[lane] = (uint16_t)f32_to_bf16(y0);
    dst[lane + 64] = (uint16_t)f32_to_bf16(y1);
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
// Barrier schedule (both roles execute the same s_barrier sequence; each role
// has its own loop so that the compute waves' weight registers and the
// control wave's poll buffers never share live ranges):
//
//   per layer   control wave                        compute waves
//   a           h (or embedding row) -> norm         .
//   a..b        .                                    QKV rows
//   b..c        publish qkv, gather qkv, qk-norm,    .
//               RoPE, KV-cache append
//   c..d        .                                    split-K attention
//   d..e        publish partial, combine, gather o   .
//   e..f        .                                    O rows
//   f..g        publish h', gather h', norm          .
//   g..h        .                                    gate/up rows
//   h..i        publish m, gather m                  .
//   i..j        .                                    down rows
//   j..a'       publish h''                          .
//   k           gather h, final norm                 .
//   k..l        .                                    LM-head rows
//   l..         argmax keys, WG 0 picks the token    .

constexpr int kTracePoints = 13;  // wall-clock stamps per layer (see the schedule above)

struct Step {
  uint32_t epoch;
  int pos, tok, step, C, nl;
  bool persistent;
};

#define QMK_SYNC()            \
  do {                        \
    __syncthreads();          \
    if (s.abort_flag) return; \
  } while (0)

template <class M>
__device__ __forceinline__ void control_path(const KArgs& a, Smem<M>& s, const Step& p, int b, int lane) {
  using Dm = Dims<M>;
  const int g = b & (kGroups - 1), r = b >> 3;
  Ctl<M> ctl(a, s, lane, p.epoch);
  auto tag_of = [&](int layer, int k) { return make_tag(p.epoch, (uint32_t)(layer * Dm::N_X_PER_LAYER + k)); };
  const size_t kv_layer_stride = (size_t)Dm::NKV * a.max_seq_len * Dm::D;
  auto to_f32 = [&](float* dst) {
    return [dst](int ci, u32x4 v) {
      float* d = dst + 4 * ci;
      d[0] = bf16_to_f32(v.x >> 16); d[1] = bf16_to_f32(v.y >> 16);
      d[2] = bf16_to_f32(v.z >> 16); d[3] = bf16_to_f32(v.w >> 16);
    };
  };
  auto to_bf16 = [&](uint16_t* dst) {
    return [dst](int ci, u32x4 v) {
      uint32_t* d = reinterpret_cast<uint32_t*>(dst) + 2 * ci;
      d[0] = (v.x >> 16) | (v.y & 0xffff0000u);
      d[1] = (v.z >> 16) | (v.w & 0xffff0000u);
    };
  };

  auto stamp = [&](int point) {
    if (a.trace && lane == 0) a.trace[(size_t)point * kNumWG + b] = wall_clock64();
  };
  for (int L = 0; L < p.nl; L++) {
    const LayerPtrs& w = a.layers[L];
    const int tp = L * kTracePoints;
    stamp(tp + 0);
    // ---------------------------------------------------------------- a
    if (L == 0) {
      const uint16_t* e = a.embed + (size_t)p.tok * Dm::H;
#pragma unroll
      for (int j = 0; j < Dm::LH; j++) {
        const u32x4 v = ld16(e + 512 * j + 8 * lane);
        float* d = s.x + 512 * j + 8 * lane;
        d[0] = lo_bf16(v.x); d[1] = hi_bf16(v.x); d[2] = lo_bf16(v.y); d[3] = hi_bf16(v.y);
        d[4] = lo_bf16(v.z); d[5] = hi_bf16(v.z); d[6] = lo_bf16(v.w); d[7] = hi_bf16(v.w);
      }
      ctl.rmsnorm(s.x, w.in_ln);
    } else if (ctl.template gather<Dm::H>(a.x + Dm::X_H, tag_of(L - 1, 5), to_f32(s.x))) {
      ctl.rmsnorm(s.x, w.in_ln);
    }
    stamp(tp + 1);
    QMK_SYNC();  // a
    QMK_SYNC();  // b
    stamp(tp + 2);
    {
      const uint32_t t = tag_of(L, 0);
      if (lane < Dm::RQ_WG / 4) {
        const float* o = s.out + 4 * lane;
        const uint32_t wi = Dm::X_QKV + g * Dm::RG + Dm::RQ_WG * r + 4 * lane;
        if (a.xcd_local) ctl.template publish4<false>(wi, o[0], o[1], o[2], o[3], t);
        else ctl.template publish4<true>(wi, o[0], o[1], o[2], o[3], t);
      }
      if (ctl.template gather<Dm::RG>(a.x + Dm::X_QKV + g * Dm::RG, t, to_f32(s.qkv))) {
        const uint16_t* cosr = a.cos_t + (size_t)p.pos * Dm::D;
        const uint16_t* sinr = a.sin_t + (size_t)p.pos * Dm::D;
#pragma unroll
        for (int h = 0; h < Dm::GQ; h++) ctl.head_norm_rope(h * Dm::D, w.q_norm, cosr, sinr, s.q + h * Dm::D);
        ctl.head_norm_rope(Dm::GQ * Dm::D, w.k_norm, cosr, sinr, s.k);
        const float v0 = s.qkv[(Dm::GQ + 1) * Dm::D + lane], v1 = s.qkv[(Dm::GQ + 1) * Dm::D + lane + 64];
        s.v[lane] = (uint16_t)f32_to_bf16(v0);
        s.v[lane + 64] = (uint16_t)f32_to_bf16(v1);
        if (r == 0) {
          const size_t o = L * kv_layer_stride + ((size_t)g * a.max_seq_len + p.pos) * Dm::D;
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
    {
      // workgroup partial = merge of the eight wave partials, then publish
      const uint32_t t = tag_of(L, 1);
#pragma unroll
      for (int h = 0; h < Dm::GQ; h++) {
        float mw[kComputeWaves];
        float mx = -INFINITY;
#pragma unroll
        for (int cc = 0; cc < kComputeWaves; cc++) { mw[cc] = s.wp[cc][h][0]; mx = fmaxf(mx, mw[cc]); }
        float lsum = 0.f, a0 = 0.f, a1 = 0.f;
#pragma unroll
        for (int cc = 0; cc < kComputeWaves; cc++) {
          const float f = mw[cc] == -INFINITY ? 0.f : __expf(mw[cc] - mx);
          lsum += s.wp[cc][h][1] * f;
          a0 += s.wp[cc][h][2 + 2 * lane] * f;
          a1 += s.wp[cc][h][3 + 2 * lane] * f;
        }
        const uint32_t base = Dm::X_PART + (uint32_t)((g * kGroupSize + r) * Dm::PART_WG + h * Dm::PART_HEAD);
        u32x4 d;
        const uint32_t ba0 = __float_as_uint(a0), ba1 = __float_as_uint(a1);
        d.x = word(ba0 >> 16, t); d.y = word(ba0 & 0xffffu, t); d.z = word(ba1 >> 16, t); d.w = word(ba1 & 0xffffu, t);
        if (a.xcd_local) put4<false>(a.x, base + 4 + 4 * lane, d); else put4<true>(a.x, base + 4 + 4 * lane, d);
        if (lane == 0) {
          const uint32_t bm = __float_as_uint(mx), bl = __float_as_uint(lsum);
          d.x = word(bm >> 16, t); d.y = word(bm & 0xffffu, t); d.z = word(bl >> 16, t); d.w = word(bl & 0xffffu, t);
          if (a.xcd_local) put4<false>(a.x, base, d); else put4<true>(a.x, base, d);
        }
      }
      stamp(tp + 5);
      // combine: this workgroup owns (head hh, dims 8kb..8kb+7) of its group
      const int hh = r / (Dm::D / 8), kb = r % (Dm::D / 8);
      const uint32_t pbase = Dm::X_PART + (uint32_t)(g * kGroupSize * Dm::PART_WG + hh * Dm::PART_HEAD);
      auto rs = make_rsrc(a.x, 0x7fffffffu);
      constexpr int NCH = kGroupSize * 5;  // (m,l) chunk + four acc chunks per partial
      constexpr int PER = (NCH + 63) / 64;
      u32x4 v[PER];
      uint32_t off[PER];
      uint32_t pend = 0;
#pragma unroll
      for (int i = 0; i < PER; i++) {
        const int ci = lane + 64 * i;
        const int j = ci / 5, q = ci % 5;
        off[i] = pbase + (uint32_t)(j * Dm::PART_WG) + (q == 0 ? 0u : (uint32_t)(4 + 16 * kb + 4 * (q - 1)));
        if (ci < NCH) pend |= 1u << i;
      }
      const uint64_t t0 = wall_clock64();
      bool ok = true;
      while (true) {
#pragma unroll
        for (int i = 0; i < PER; i++)
          if (pend & (1u << i)) v[i] = poll16(rs, off[i] * 4u);
#pragma unroll
        for (int i = 0; i < PER; i++)
          if ((pend & (1u << i)) && chunk_ok(v[i], t)) pend &= ~(1u << i);
        if (!__any(pend != 0)) break;
        if (wall_clock64() - t0 > a.timeout) { ctl.fail(kErrTimeout); ok = false; break; }
      }
      stamp(tp + 6);
      if (ok) {
#pragma unroll
        for (int i = 0; i < PER; i++) {
          const int ci = lane + 64 * i;
          if (ci < NCH) {
            const int j = ci / 5, q = ci % 5;
            s.comb[j][4 * q + 0] = v[i].x >> 16;
            s.comb[j][4 * q + 1] = v[i].y >> 16;
            s.comb[j][4 * q + 2] = v[i].z >> 16;
            s.comb[j][4 * q + 3] = v[i].w >> 16;
          }
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        if (lane < 2) {
          float mx = -INFINITY;
          for (int j = 0; j < kGroupSize; j++) mx = fmaxf(mx, __uint_as_float((s.comb[j][0] << 16) | s.comb[j][1]));
          float lsum = 0.f, o[4] = {0.f, 0.f, 0.f, 0.f};
          for (int j = 0; j < kGroupSize; j++) {
            const float mj = __uint_as_float((s.comb[j][0] << 16) | s.comb[j][1]);
            const float f = mj == -INFINITY ? 0.f : __expf(mj - mx);
            lsum += __uint_as_float((s.comb[j][2] << 16) | s.comb[j][3]) * f;
#pragma unroll
            for (int d = 0; d < 4; d++) {
              const int dd = 4 * lane + d;
              o[d] += __uint_as_float((s.comb[j][4 + 2 * dd] << 16) | s.comb[j][5 + 2 * dd]) * f;
            }
          }
          const uint32_t wi = Dm::X_ATTN + (uint32_t)((g * Dm::GQ + hh) * Dm::D + 8 * kb + 4 * lane);
          ctl.template publish4<true>(wi, __fdiv_rn(o[0], lsum), __fdiv_rn(o[1], lsum), __fdiv_rn(o[2], lsum),
                                      __fdiv_rn(o[3], lsum), tag_of(L, 2));
        }
        ctl.template gather<Dm::QS>(a.x + Dm::X_ATTN, tag_of(L, 2), to_bf16(s.attn));
      }
    }
    stamp(tp + 7);
    QMK_SYNC();  // e
    QMK_SYNC();  // f
    stamp(tp + 8);
    if (lane == 0) {
      float hv[4];
#pragma unroll
      for (int i = 0; i < 4; i++) {
        float o = 0.f;
#pragma unroll
        for (int q = 0; q < Dm::O_WPR; q++) o += s.out[i * Dm::O_WPR + q];
        hv[i] = bf16r(s.x[Dm::O_ROWS * b + i] + bf16r(o));
      }
      ctl.template publish4<true>(Dm::X_H2 + Dm::O_ROWS * b, hv[0], hv[1], hv[2], hv[3], tag_of(L, 3));
    }
    if (ctl.template gather<Dm::H>(a.x + Dm::X_H2, tag_of(L, 3), to_f32(s.h2))) ctl.rmsnorm(s.h2, w.post_ln);
    stamp(tp + 9);
    QMK_SYNC();  // g
    QMK_SYNC();  // h
    stamp(tp + 10);
    if (lane < Dm::M_WG / 4) {
      float mv[4];
#pragma unroll
      for (int q = 0; q < 4; q++) {
        const float gt = s.out[4 * lane + q];
        const float up = s.out[Dm::M_WG + 4 * lane + q];
        const float sg = bf16r(__fdiv_rn(gt, 1.0f + expf(-gt)));
        mv[q] = bf16r(sg * up);
      }
      ctl.template publish4<true>(Dm::X_M + Dm::M_WG * b + 4 * lane, mv[0], mv[1], mv[2], mv[3], tag_of(L, 4));
    }
    ctl.template gather<Dm::I>(a.x + Dm::X_M, tag_of(L, 4), to_bf16(s.m));
    stamp(tp + 11);
    QMK_SYNC();  // i
    QMK_SYNC();  // j
    stamp(tp + 12);
    if (lane == 0) {
      float hv[4];
#pragma unroll
      for (int i = 0; i < 4; i++) {
        float d = 0.f;
#pragma unroll
        for (int q = 0; q < Dm::D_WPR; q++) d += s.out[i * Dm::D_WPR + q];
        hv[i] = bf16r(s.h2[Dm::D_ROWS * b + i] + bf16r(d));
      }
      ctl.template publish4<true>(Dm::X_H + Dm::D_ROWS * b, hv[0], hv[1], hv[2], hv[3], tag_of(L, 5));
    }
  }

  // ------------------------------------------------------------------ k
  if (ctl.template gather<Dm::H>(a.x + Dm::X_H, tag_of(p.nl - 1, 5), to_f32(s.x))) {
    ctl.rmsnorm(s.x, a.final_norm);
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
  QMK_SYNC();  // k
  QMK_SYNC();  // l
  stamp(p.nl * kTracePoints + 1);
  const uint32_t tk = make_tag(p.epoch, (uint32_t)(p.nl * Dm::N_X_PER_LAYER));
  if (lane == 0) {
    uint64_t best = 0;
#pragma unroll
    for (int cc = 0; cc < kComputeWaves; cc++) best = s.best[cc] > best ? s.best[cc] : best;
    const uint32_t idx = 0xffffffffu - (uint32_t)best;
    u32x4 d;
    d.x = word((uint32_t)(best >> 32) & 0xffffu, tk);
    d.y = word(idx & 0xffffu, tk);
    d.z = word(idx >> 16, tk);
    d.w = word(0, tk);
    put4<true>(a.x, Dm::X_KEY + 4 * b, d);
  }
  if (b == 0) {
    uint64_t best = 0;
    const bool ok = ctl.template gather<kNumWG * 4>(a.x + Dm::X_KEY, tk, [&](int ci, u32x4 v) {
      const uint32_t idx = (v.y >> 16) | (v.z & 0xffff0000u);
      const uint64_t key = ((uint64_t)(v.x >> 16) << 32) | (uint64_t)(0xffffffffu - idx);
      best = key > best ? key : best;
    });
    stamp(p.nl * kTracePoints + 2);
    if (ok) {
      best = wave_max_u64(best);
      const int token = (int)(0xffffffffu - (uint32_t)best);
      if (lane == 0) {
        DecodeState* st = a.st;
        if (a.out_token) *a.out_token = token;
        if (p.persistent) {
          if (a.out_log) a.out_log[p.step] = token;
          st->tok = token;
          st->pos = p.pos + 1;
          st->step = p.step + 1;
        }
        st->epoch = p.epoch + (uint32_t)(p.nl * Dm::N_X_PER_LAYER + 1);
      }
    }
  }
}

template <class M>
__device__ __forceinline__ void compute_path(const KArgs& a, Smem<M>& s, const Step& p, int b, int c, int lane) {
  using Dm = Dims<M>;
  const int g = b & (kGroups - 1), r = b >> 3;
  const size_t kv_layer_stride = (size_t)Dm::NKV * a.max_seq_len * Dm::D;

  // Weight registers, requested one layer ahead.
  u32x4 wq[Dm::RQ_W][Dm::LH];
  u32x4 wo[Dm::LO];
  u32x4 wgu[Dm::GU_W][Dm::LH];
  u32x4 wd[Dm::LD];

  const int o_row = Dm::O_ROWS * b + c / Dm::O_WPR;
  const int o_k0 = (c % Dm::O_WPR) * (Dm::QS / Dm::O_WPR);
  const int d_row = Dm::D_ROWS * b + c / Dm::D_WPR;
  const int d_k0 = (c % Dm::D_WPR) * (Dm::I / Dm::D_WPR);
  const bool gu_up = c >= kComputeWaves / 2;
  const int gu_m0 = Dm::M_WG * b + (gu_up ? c - kComputeWaves / 2 : c) * Dm::GU_W;
  const int gu_out = (gu_up ? Dm::M_WG : 0) + (gu_up ? c - kComputeWaves / 2 : c) * Dm::GU_W;

  auto prefetch_qkv = [&](int layer) {
    const LayerPtrs& w = a.layers[layer];
#pragma unroll
    for (int i = 0; i < Dm::RQ_W; i++) load_row(wq[i], qkv_row<M>(w, g, Dm::RQ_WG * r + Dm::RQ_W * c + i), 0, lane);
  };
  auto prefetch_o = [&](int layer) { load_row(wo, a.layers[layer].wo + (size_t)o_row * Dm::QS, o_k0, lane); };
  auto prefetch_gu = [&](int layer) {
    const uint16_t* base = gu_up ? a.layers[layer].wu : a.layers[layer].wg;
#pragma unroll
    for (int i = 0; i < Dm::GU_W; i++) load_row(wgu[i], base + (size_t)(gu_m0 + i) * Dm::H, 0, lane);
  };
  auto prefetch_dn = [&](int layer) { load_row(wd, a.layers[layer].wd + (size_t)d_row * Dm::I, d_k0, lane); };

  prefetch_qkv(0);
  prefetch_o(0);
  prefetch_gu(0);
  prefetch_dn(0);

  const int chunk = (p.C + kGroupSize - 1) / kGroupSize;
  const int p_begin = min(p.C, r * chunk);
  const int p_end = min(p.C, p_begin + chunk);
  const int slot = lane >> 4, t16 = lane & 15;

  for (int L = 0; L < p.nl; L++) {
    const uint16_t* kc = a.k_cache + L * kv_layer_stride + (size_t)g * a.max_seq_len * Dm::D;
    const uint16_t* vc = a.v_cache + L * kv_layer_stride + (size_t)g * a.max_seq_len * Dm::D;
    QMK_SYNC();  // a
    {
      u32x4 act[Dm::LH];
      load_act(act, s.n, 0, lane);
#pragma unroll
      for (int i = 0; i < Dm::RQ_W; i++) {
        const float v = row_dot(wq[i], act);
        if (lane == 0) s.out[Dm::RQ_W * c + i] = bf16r(v);
      }
    }
    QMK_SYNC();  // b
    QMK_SYNC();  // c
    {
      u32x4 qv[Dm::GQ];
#pragma unroll
      for (int h = 0; h < Dm::GQ; h++) qv[h] = *reinterpret_cast<const u32x4*>(s.q + h * Dm::D + 8 * t16);
      const u32x4 k_now = *reinterpret_cast<const u32x4*>(s.k + 8 * t16);
      const u32x4 v_now = *reinterpret_cast<const u32x4*>(s.v + 8 * t16);
      float mrun[Dm::GQ], lrun[Dm::GQ], acc[Dm::GQ][8];
#pragma unroll
      for (int h = 0; h < Dm::GQ; h++) {
        mrun[h] = -INFINITY;
        lrun[h] = 0.f;
#pragma unroll
        for (int i = 0; i < 8; i++) acc[h][i] = 0.f;
      }
      constexpr int U = 2;  // each wave covers 4 positions (one per 16-lane slot) per step, U steps per batch
      for (int base = p_begin + 4 * c; base < p_end; base += 32 * U) {
        u32x4 kk[U], vv[U];
        bool valid[U];
#pragma unroll
        for (int u = 0; u < U; u++) {
          const int pp = base + 32 * u + slot;
          valid[u] = pp < p_end;
          const int pl = (valid[u] && pp != p.pos) ? pp : p_begin;
          kk[u] = ld16(kc + (size_t)pl * Dm::D + 8 * t16);
          vv[u] = ld16(vc + (size_t)pl * Dm::D + 8 * t16);
        }
#pragma unroll
        for (int u = 0; u < U; u++) {
          const int pp = base + 32 * u + slot;
          const u32x4 kx = pp == p.pos ? k_now : kk[u];
          const u32x4 vx = pp == p.pos ? v_now : vv[u];
#pragma unroll
          for (int h = 0; h < Dm::GQ; h++) {
            float sc = row16_sum(dot8(kx, qv[h], 0.f));
            sc = bf16r(bf16r(sc) * a.attn_scale);
            if (valid[u]) {
              const float mn = fmaxf(mrun[h], sc);
              const float corr = __expf(mrun[h] - mn);
              const float pe = __expf(sc - mn);
              lrun[h] = lrun[h] * corr + pe;
              acc[h][0] = acc[h][0] * corr + pe * lo_bf16(vx.x);
              acc[h][1] = acc[h][1] * corr + pe * hi_bf16(vx.x);
              acc[h][2] = acc[h][2] * corr + pe * lo_bf16(vx.y);
              acc[h][3] = acc[h][3] * corr + pe * hi_bf16(vx.y);
              acc[h][4] = acc[h][4] * corr + pe * lo_bf16(vx.z);
              acc[h][5] = acc[h][5] * corr + pe * hi_bf16(vx.z);
              acc[h][6] = acc[h][6] * corr + pe * lo_bf16(vx.w);
              acc[h][7] = acc[h][7] * corr + pe * hi_bf16(vx.w);
              mrun[h] = mn;
            }
          }
        }
      }
      // merge the wave's four position slots
#pragma unroll
      for (int h = 0; h < Dm::GQ; h++) {
#pragma unroll
        for (int o = 16; o <= 32; o <<= 1) {
          const float mo = __shfl_xor(mrun[h], o);
          const float lo = __shfl_xor(lrun[h], o);
          const float mn = fmaxf(mrun[h], mo);
          const float f1 = mrun[h] == -INFINITY ? 0.f : __expf(mrun[h] - mn);
          const float f2 = mo == -INFINITY ? 0.f : __expf(mo - mn);
          lrun[h] = lrun[h] * f1 + lo * f2;
#pragma unroll
          for (int i = 0; i < 8; i++) {
            const float ao = __shfl_xor(acc[h][i], o);
            acc[h][i] = acc[h][i] * f1 + ao * f2;
          }
          mrun[h] = mn;
        }
        if (lane < 16) {
#pragma unroll
          for (int i = 0; i < 8; i++) s.wp[c][h][2 + 8 * t16 + i] = acc[h][i];
          if (lane == 0) {
            s.wp[c][h][0] = mrun[h];
            s.wp[c][h][1] = lrun[h];
          }
        }
      }
    }
    if (L + 1 < p.nl) prefetch_qkv(L + 1);
    QMK_SYNC();  // d
    QMK_SYNC();  // e
    {
      u32x4 act[Dm::LO];
      load_act(act, s.attn, o_k0, lane);
      const float v = row_dot(wo, act);
      if (lane == 0) s.out[c] = v;
    }
    if (L + 1 < p.nl) prefetch_o(L + 1);
    QMK_SYNC();  // f
    QMK_SYNC();  // g
    {
      u32x4 act[Dm::LH];
      load_act(act, s.n, 0, lane);
#pragma unroll
      for (int i = 0; i < Dm::GU_W; i++) {
        const float v = row_dot(wgu[i], act);
        if (lane == 0) s.out[gu_out + i] = bf16r(v);
      }
    }
    if (L + 1 < p.nl) prefetch_gu(L + 1);
    QMK_SYNC();  // h
    QMK_SYNC();  // i
    {
      u32x4 act[Dm::LD];
      load_act(act, s.m, d_k0, lane);
      const float v = row_dot(wd, act);
      if (lane == 0) s.out[c] = v;
    }
    if (L + 1 < p.nl) prefetch_dn(L + 1);
    QMK_SYNC();  // j
  }

  QMK_SYNC();  // k
  {
    u32x4 act[Dm::LH];
    load_act(act, s.n, 0, lane);
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
    auto do_batch = [&](u32x4 (&buf)[Dm::LM_U][Dm::LH], int i0) {
#pragma unroll
      for (int u = 0; u < Dm::LM_U; u++) {
        const float v = row_dot(buf[u], act);
        if (i0 + u < nmine) {
          const int row = row_of(i0 + u);
          const uint32_t hb = f32_to_bf16(v);
          const uint64_t key = ((uint64_t)orderable16(hb) << 32) | (uint64_t)(0xffffffffu - (uint32_t)row);
          best = key > best ? key : best;
          if (a.logits && lane == 0) a.logits[row] = bf16_to_f32(hb);
        }
      }
    };
    load_batch(bufA, 0);
    for (int i = 0; i < nmine; i += 2 * Dm::LM_U) {
      load_batch(bufB, i + Dm::LM_U);
      do_batch(bufA, i);
      if (i + 2 * Dm::LM_U < nmine) load_batch(bufA, i + 2 * Dm::LM_U);
      do_batch(bufB, i + Dm::LM_U);
    }
    if (lane == 0) s.best[c] = best;
  }
  QMK_SYNC();  // l
}

template <class M>
__global__ void __launch_bounds__(kBlock, 1) decode_kernel(KArgs a) {
  using Dm = Dims<M>;
  __shared__ Smem<M> s;
  const int b = blockIdx.x;
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;

  DecodeState* st = a.st;
  if (threadIdx.x == 0) {
    // One thread reads the state's error word so the whole workgroup takes the
    // same decision; a non-zero value (an earlier launch failed) makes this
    // launch a no-op until the state is reset.
    s.abort_flag = __hip_atomic_load(&st->err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0;
    // A step that fails on the device leaves -1 here, never a stale token.
    if (b == 0 && a.out_token) *a.out_token = -1;
  }
  __syncthreads();
  if (s.abort_flag) return;
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
  if (wave == 0)
    control_path<M>(a, s, p, b, lane);
  else
    compute_path<M>(a, s, p, b, wave - 1, lane);
}

#undef QMK_SYNC

}  // namespace qmk
