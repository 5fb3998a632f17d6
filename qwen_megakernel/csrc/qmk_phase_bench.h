// Per-phase weight-streaming kernels: each GEMV phase of the decode step run
// on its own, over a rotating set of distinct weight copies, so that its HBM
// streaming rate can be measured without the exchanges that bound the full
// step.  Every phase uses the decode kernel's own work split and load width,
// with register prefetch one copy ahead (two for the small o/down slices; the
// decode kernel requests each phase's weights one layer ahead); a workgroup
// walks through all copies without waiting for the others, because the input
// activation is fixed.
//
// Phases and layouts (bf16, row-major [out][in], one copy after another):
//   QKV      RMSNorm(x) then q/k/v rows [4096][1024] (q 0..2047, k 2048..3071,
//            v 3072..4095); out bf16[4096]
//   O        [1024][2048]; out f32[8][1024]: the per-XCD partial sums over the
//            XCD's 256 input columns, as the decode kernel produces them
//   GATE_UP  gate [3072][1024] then up [3072][1024]; out bf16[3072] =
//            bf16(bf16(silu(g)) * u)
//   DOWN     [1024][3072]; out f32[8][1024] per-XCD partials over 384 columns
//   LM_HEAD  [151936][1024]; out u64[256][8]: per-wave best key
//            (orderable bf16 logit << 32 | ~row); the largest is the argmax
// Only the last copy's results remain in ``out``; every copy is computed.
#pragma once

#include "qmk_decode_kernel.h"

namespace qmk {

enum PhaseId : int { kPhaseQKV = 0, kPhaseO = 1, kPhaseGateUp = 2, kPhaseDown = 3, kPhaseLmHead = 4 };

struct PhaseArgs {
  const uint16_t* w;       // copy 0
  size_t copy_elems;       // bf16 elements per copy
  int n_copies;
  const uint16_t* norm_w;  // QKV: RMSNorm weight [H]
  const uint16_t* act;     // input vector (bf16)
  void* out;
  float rms_eps;
};

template <class M>
struct PhaseSmem {
  using Dm = Dims<M>;
  uint16_t act[Dm::I > Dm::QS ? Dm::I : Dm::QS];
  float gu[2][2 * Dm::M_WG];
};

template <class M, int PHASE>
__global__ void __launch_bounds__(kBlock, 1) phase_kernel(PhaseArgs a) {
  using Dm = Dims<M>;
  __shared__ PhaseSmem<M> s;
  const int b = blockIdx.x, wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int xcd = b & (kGroups - 1), r = b >> 3;
  const int slot = lane >> 4, t16 = lane & 15;

  // ---- input vector into LDS (RMSNorm for QKV, as the decode kernel's control wave does)
  constexpr int NIN = PHASE == kPhaseO ? Dm::QS : PHASE == kPhaseDown ? Dm::I : Dm::H;
  if (wave == 0) {
    if (PHASE == kPhaseQKV) {
      constexpr int P = Dm::H / 128;
      float2 xv[P];
      float ss = 0.f;
#pragma unroll
      for (int i = 0; i < P; i++) {
        const uint32_t u = ld32(reinterpret_cast<const uint32_t*>(a.act) + lane + 64 * i);
        xv[i] = make_float2(lo_bf16(u), hi_bf16(u));
        ss += xv[i].x * xv[i].x + xv[i].y * xv[i].y;
      }
      ss = wave_sum(ss);
      const float rstd = rcp_sqrt_torch(__fdiv_rn(ss, (float)Dm::H) + a.rms_eps);
#pragma unroll
      for (int i = 0; i < P; i++) {
        const uint32_t wp = ld32(reinterpret_cast<const uint32_t*>(a.norm_w) + lane + 64 * i);
        const float n0 = bf16r(lo_bf16(wp) * bf16r(xv[i].x * rstd));
        const float n1 = bf16r(hi_bf16(wp) * bf16r(xv[i].y * rstd));
        reinterpret_cast<uint32_t*>(s.act)[lane + 64 * i] = f32_to_bf16(n0) | (f32_to_bf16(n1) << 16);
      }
    } else {
      for (int i = lane; i < NIN / 8; i += 64) reinterpret_cast<u32x4*>(s.act)[i] = ld16(a.act + 8 * i);
    }
  }
  __syncthreads();

  const int nc = a.n_copies;
  auto copy_base = [&](int k) { return a.w + (size_t)k * a.copy_elems; };

  if (PHASE == kPhaseGateUp) {
    // waves 1..4 gate rows, 5..8 up rows (3 each), wave 0 forms silu(g) * u
    const int c = wave - 1;
    const bool up = c >= kComputeWaves / 2;
    const int gi = (up ? c - kComputeWaves / 2 : c) * Dm::GU_W;
    const int m0 = Dm::MS * xcd + Dm::M_WG * r + gi;
    u32x4 w[Dm::GU_W][Dm::LH];
    auto load = [&](int k) {
      const uint16_t* base = copy_base(k) + (up ? (size_t)Dm::I * Dm::H : 0);
#pragma unroll
      for (int i = 0; i < Dm::GU_W; i++) load_row(w[i], base + (size_t)(m0 + i) * Dm::H, 0, lane);
    };
    if (wave > 0) load(0);
    for (int k = 0; k < nc; k++) {
      if (wave > 0) {
        u32x4 act[Dm::LH];
        load_act(act, s.act, 0, lane);
        float v[Dm::GU_W];
#pragma unroll
        for (int i = 0; i < Dm::GU_W; i++) v[i] = row_dot(w[i], act);
        if (k + 1 < nc) load(k + 1);
        if (lane == 0) {
#pragma unroll
          for (int i = 0; i < Dm::GU_W; i++) s.gu[k & 1][(up ? Dm::M_WG : 0) + gi + i] = bf16r(v[i]);
        }
      }
      __syncthreads();
      if (wave == 0 && lane < Dm::M_WG) {
        const float g = s.gu[k & 1][lane], u = s.gu[k & 1][Dm::M_WG + lane];
        const float sg = bf16r(__fdiv_rn(g, 1.0f + expf(-g)));
        reinterpret_cast<uint16_t*>(a.out)[Dm::MS * xcd + Dm::M_WG * r + lane] = (uint16_t)f32_to_bf16(bf16r(sg * u));
      }
    }
    return;
  }

  if (wave == 0) return;
  const int c = wave - 1;

  if (PHASE == kPhaseQKV) {
    u32x4 w[Dm::RQ_W][Dm::LH];
    auto load = [&](int k) {
      LayerPtrs lp;
      lp.wq = copy_base(k);
      lp.wk = lp.wq + (size_t)Dm::QS * Dm::H;
      lp.wv = lp.wk + (size_t)Dm::NKV * Dm::D * Dm::H;
#pragma unroll
      for (int i = 0; i < Dm::RQ_W; i++) load_row(w[i], qkv_row<M>(lp, xcd, Dm::RQ_WG * r + Dm::RQ_W * c + i), 0, lane);
    };
    load(0);
    for (int k = 0; k < nc; k++) {
      u32x4 act[Dm::LH];
      load_act(act, s.act, 0, lane);
      float v[Dm::RQ_W];
#pragma unroll
      for (int i = 0; i < Dm::RQ_W; i++) v[i] = row_dot(w[i], act);
      if (k + 1 < nc) load(k + 1);
      if (lane == 0) {
#pragma unroll
        for (int i = 0; i < Dm::RQ_W; i++) {
          // global row index of vr = RQ_WG*r + RQ_W*c + i within KV group xcd
          const int vr = Dm::RQ_WG * r + Dm::RQ_W * c + i;
          int row;
          if (vr < Dm::GQ * Dm::D) row = xcd * Dm::GQ * Dm::D + vr;
          else if (vr < (Dm::GQ + 1) * Dm::D) row = Dm::QS + xcd * Dm::D + (vr - Dm::GQ * Dm::D);
          else row = Dm::QS + Dm::NKV * Dm::D + xcd * Dm::D + (vr - (Dm::GQ + 1) * Dm::D);
          reinterpret_cast<uint16_t*>(a.out)[row] = (uint16_t)f32_to_bf16(v[i]);
        }
      }
    }
  } else if (PHASE == kPhaseO || PHASE == kPhaseDown) {
    constexpr int K = PHASE == kPhaseO ? Dm::QS : Dm::I;     // row length
    constexpr int SEG = PHASE == kPhaseO ? Dm::OC : Dm::MS;  // this XCD's columns
    constexpr int NL = PHASE == kPhaseO ? Dm::LO : Dm::LD;
    const int row = Dm::ROWS_WG * r + Dm::ROWS_W * c + slot;
    // these slices are small (16-24 KB per CU), so two copies are kept in flight
    u32x4 w0[NL], w1[NL];
    auto load = [&](u32x4 (&w)[NL], int k) { load_seg(w, copy_base(k) + (size_t)row * K + SEG * xcd, t16); };
    auto step = [&](u32x4 (&w)[NL], int k) {
      const float v = seg_dot(w, s.act + SEG * xcd, t16);
      if (k + 2 < nc) load(w, k + 2);
      if (t16 == 0) reinterpret_cast<float*>(a.out)[xcd * Dm::H + row] = v;
    };
    load(w0, 0);
    if (nc > 1) load(w1, 1);
    for (int k = 0; k < nc; k += 2) {
      step(w0, k);
      if (k + 1 < nc) step(w1, k + 1);
    }
  } else if (PHASE == kPhaseLmHead) {
    u32x4 act[Dm::LH];
    load_act(act, s.act, 0, lane);
    const int row0 = b * Dm::LM_RPW;
    const int nrows = min(Dm::V - row0, Dm::LM_RPW);
    const int nmine = (nrows - c + kComputeWaves - 1) / kComputeWaves;
    constexpr int NB = (Dm::LM_RPW + kComputeWaves * Dm::LM_U - 1) / (kComputeWaves * Dm::LM_U);  // batches per copy
    const int total = NB * nc;
    u32x4 bufA[Dm::LM_U][Dm::LH], bufB[Dm::LM_U][Dm::LH];
    uint64_t best = 0;
    auto load_batch = [&](u32x4 (&buf)[Dm::LM_U][Dm::LH], int g) {
      const uint16_t* base = copy_base(g / NB);
      const int i0 = (g % NB) * Dm::LM_U;
#pragma unroll
      for (int u = 0; u < Dm::LM_U; u++) {
        const int i = max(0, min(i0 + u, nmine - 1));
        load_row(buf[u], base + (size_t)(row0 + c + kComputeWaves * i) * Dm::H, 0, lane);
      }
    };
    auto do_batch = [&](u32x4 (&buf)[Dm::LM_U][Dm::LH], int g) {
      const int i0 = (g % NB) * Dm::LM_U;
      if (i0 == 0) best = 0;
#pragma unroll
      for (int u = 0; u < Dm::LM_U; u++) {
        const float v = row_dot(buf[u], act);
        if (i0 + u < nmine) {
          const uint32_t rrow = (uint32_t)(row0 + c + kComputeWaves * (i0 + u));
          const uint64_t key = ((uint64_t)orderable16(f32_to_bf16(v)) << 32) | (uint64_t)(0xffffffffu - rrow);
          best = key > best ? key : best;
        }
      }
      if ((g % NB) == NB - 1 && lane == 0) reinterpret_cast<uint64_t*>(a.out)[b * kComputeWaves + c] = best;
    };
    load_batch(bufA, 0);
    for (int g = 0; g < total; g += 2) {
      if (g + 1 < total) load_batch(bufB, g + 1);
      do_batch(bufA, g);
      if (g + 2 < total) load_batch(bufA, g + 2);
      if (g + 1 < total) do_batch(bufB, g + 1);
    }
  }
}

}  // namespace qmk
