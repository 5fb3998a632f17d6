// Device-side building blocks of the gfx950 decode kernel: bf16 rounding,
// wave64 reductions, weight streaming, and the tagged-word exchange that
// replaces grid barriers.
//
// Exchange protocol.  Every value that crosses workgroups travels as a 32-bit
// word (payload16 << 16 | tag16).  The tag is derived from a per-launch epoch
// and the exchange's index within the launch, and is never 0, so zeroed memory
// and data left over from any earlier exchange are never mistaken for the
// current one.  A consumer polls the words themselves and re-reads only the
// 16-byte chunks whose tags are stale; one exchange therefore costs one
// store-to-load latency instead of a barrier round trip, and only 4-byte
// single-copy atomicity is relied upon.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>
#include <utility>

namespace qmk {

typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));  // MFMA 16x16x32 bf16 operand
typedef float f32x4 __attribute__((ext_vector_type(4)));    // MFMA 16x16 accumulator

constexpr int kWave = 64;
constexpr int kNumWG = 256;       // one workgroup per CU of an MI355X
constexpr int kComputeWaves = 8;  // waves 1..8 stream weights; wave 0 moves activations
constexpr int kBlock = (kComputeWaves + 1) * kWave;
constexpr int kGroups = 8;        // workgroup b runs on XCD b % 8
constexpr int kGroupSize = kNumWG / kGroups;

// The kernels read weights, tables, caches and activations with 16-byte vector loads (and LDS DMA),
// so every such pointer must be 16-byte aligned (torch allocations are); the entry points check it.
inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// ---------------------------------------------------------------- bf16

__device__ __forceinline__ float bf16_to_f32(uint32_t h) { return __uint_as_float(h << 16); }

// fp32 -> bf16 bits, round to nearest even (gfx950 v_cvt_pk_bf16_f32), as
// c10::BFloat16 does for every non-NaN value; tests/test_gpu_blocks.py checks
// it against torch on ties, subnormals and infinities.
__device__ __forceinline__ uint32_t f32_to_bf16(float f) {
  const __bf16 h = (__bf16)f;
  return (uint32_t)__builtin_bit_cast(unsigned short, h);
}

// Value of ``f`` rounded to bf16, as fp32.
__device__ __forceinline__ float bf16r(float f) { return bf16_to_f32(f32_to_bf16(f)); }

// Two fp32 values rounded to bf16 as f32_to_bf16 rounds them, in one v_cvt_pk_bf16_f32 (the
// scalar form converts one value per instruction): ``lo`` in bits [15:0], ``hi`` in [31:16].
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  typedef float f32x2 __attribute__((ext_vector_type(2)));
  const f32x2 v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
}

__device__ __forceinline__ float lo_bf16(uint32_t packed) { return __uint_as_float(packed << 16); }
__device__ __forceinline__ float hi_bf16(uint32_t packed) { return __uint_as_float(packed & 0xffff0000u); }

__device__ __forceinline__ bf16x2 as_bf2(uint32_t u) { return __builtin_bit_cast(bf16x2, u); }

// acc + dot(w[0..7], x[0..7]) for eight bf16 pairs held as two 16-byte chunks.
__device__ __forceinline__ float dot8(u32x4 w, u32x4 x, float acc) {
  uint32_t w0 = w.x, w1 = w.y, w2 = w.z, w3 = w.w;
  uint32_t x0 = x.x, x1 = x.y, x2 = x.z, x3 = x.w;
  acc = __builtin_amdgcn_fdot2_f32_bf16(as_bf2(w0), as_bf2(x0), acc, false);
  acc = __builtin_amdgcn_fdot2_f32_bf16(as_bf2(w1), as_bf2(x1), acc, false);
  acc = __builtin_amdgcn_fdot2_f32_bf16(as_bf2(w2), as_bf2(x2), acc, false);
  acc = __builtin_amdgcn_fdot2_f32_bf16(as_bf2(w3), as_bf2(x3), acc, false);
  return acc;
}

// exp(x) for the softmax: 2^(x*log2(e)) with the product split into a rounded
// high part and its exact low remainder (Cody-Waite style), so that the
// argument error stays within an ulp for any |x|; the hardware exp2 covers the
// rest.  exp_finite takes finite x (it gives NaN for -inf); exp_acc clamps the
// argument at -128 first, whose exp underflows to 0, so -inf (an empty softmax
// row, a masked score) gives 0.  For every finite x the two give the same value
// (below -128 both give 0).
__device__ __forceinline__ float exp_finite(float x) {
  constexpr float kL2eHi = 1.44269502162933349609375f;   // log2(e) rounded to fp32
  constexpr float kL2eLo = 1.925963033500011e-08f;        // log2(e) - kL2eHi
  constexpr float kLn2 = 0.693147180559945309f;
  const float hi = x * kL2eHi;
  const float lo = __builtin_fmaf(x, kL2eHi, -hi) + x * kL2eLo;  // |lo| < 2^-16: 2^lo = 1 + lo*ln2
  const float e = __builtin_amdgcn_exp2f(hi);
  return __builtin_fmaf(e * lo, kLn2, e);
}

__device__ __forceinline__ float exp_acc(float x) { return exp_finite(fmaxf(x, -128.0f)); }

// Exchange a value with the lane 16 (sum over rows 2k, 2k+1) or 32 lanes away
// (sum over the two wave halves) through the gfx950 permlane swaps, which run
// on the VALU instead of the LDS crossbar.  Return {own row's value, partner's}
// in an order that is the same for both partners (so symmetric merges agree).
__device__ __forceinline__ void swap16(float v, float& a, float& b) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  a = __uint_as_float(r[0]);
  b = __uint_as_float(r[1]);
}
__device__ __forceinline__ void swap32(float v, float& a, float& b) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  a = __uint_as_float(r[0]);
  b = __uint_as_float(r[1]);
}
// Value of lane l + OFF (OFF = 16, 32 or 48), by the row swaps above.  Valid in the lanes whose
// source stays in the wave: row 0 for OFF = 48, rows 0 and 1 for OFF = 32, rows 0 and 2 for 16.
template <int OFF>
__device__ __forceinline__ float lane_ahead(float v) {
  static_assert(OFF == 16 || OFF == 32 || OFF == 48, "a whole number of rows");
  float a, b;
  if constexpr (OFF == 16) {
    swap16(v, a, b);  // rows 0 and 2 receive rows 1 and 3 in b
  } else {
    swap32(v, a, b);  // rows 0 and 1 receive rows 2 and 3 in b
    if constexpr (OFF == 48) swap16(b, a, b);  // row 0 receives row 1 of that: row 3
  }
  return b;
}
__device__ __forceinline__ float rows_sum4(float v) {  // sum over the four 16-lane rows, in every lane
  float a, b;
  swap16(v, a, b);
  v = a + b;
  swap32(v, a, b);
  return a + b;
}

// ------------------------------------------------------------ reductions

template <int CTRL>
__device__ __forceinline__ float dpp_add(float v) {
  int s = __builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false);
  return v + __int_as_float(s);
}

// Value of lane 4*(lane/4) + Q (the lane's quad member Q), by DPP quad_perm.
template <int Q>
__device__ __forceinline__ float quad_lane(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), Q * 0x55, 0xf, 0xf, false));
}

// Any DPP lane move (CTRL: quad_perm 0x00-0xFF; row_ror:n 0x120 + n, by which lane i of each
// 16-lane row reads lane (i - n) mod 16, so row_ror:12 reads lane i + 4 for i < 12).
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}

// Sum over each row of 16 lanes; every lane of the row receives the row sum.
__device__ __forceinline__ float row16_sum(float v) {
  v = dpp_add<0xB1>(v);   // quad_perm [1,0,3,2]
  v = dpp_add<0x4E>(v);   // quad_perm [2,3,0,1]
  v = dpp_add<0x141>(v);  // row_half_mirror
  v = dpp_add<0x140>(v);  // row_mirror
  return v;
}

template <int CTRL>
__device__ __forceinline__ float dpp_get(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}

// Four row sums at once, transposed: every lane contributes v[u][h] for
// u, h in {0, 1}, and lane t16 of each 16-lane row receives the row sum of
// v[t16 & 1][(t16 >> 1) & 1].  Two quad exchanges halve the values carried
// (each lane keeps the half its index selects and adds its partner's copy of
// it), then rotations by 4 and 8 lanes add the four quads.  The last steps
// associate differently in different lanes, so only one lane per value
// (t16 < 4) should be read when bit-identical copies matter.
__device__ __forceinline__ float row16_sum_t4(float v00, float v01, float v10, float v11, int t16) {
  const bool b0 = (t16 & 1) != 0, b1 = (t16 & 2) != 0;
  const float k0 = b0 ? v10 : v00, k1 = b0 ? v11 : v01;  // kept: u = bit 0
  const float s0 = b0 ? v00 : v10, s1 = b0 ? v01 : v11;  // the partner's u
  const float n0 = k0 + dpp_get<0xB1>(s0);               // quad_perm [1,0,3,2]
  const float n1 = k1 + dpp_get<0xB1>(s1);
  float r = (b1 ? n1 : n0) + dpp_get<0x4E>(b1 ? n0 : n1);  // quad_perm [2,3,0,1]; kept: h = bit 1
  r += dpp_get<0x124>(r);                                // row_ror:4
  r += dpp_get<0x128>(r);                                // row_ror:8
  return r;
}

// Maximum and sum over the lanes of each class lane % 2 (lanes 2 apart), as the xor butterfly over
// distances 2, 4, .., 32 forms them, in lanes 0..3: DPP quad_perm [2,3,0,1], then row_ror:12 and
// row_ror:8 (lanes 0..3 read lanes 4..7, then 8..11, as the xor by 4 and by 8 would), then the row
// swaps.  Every lane of the wave must be active.
__device__ __forceinline__ float class2_max(float v) {
  v = fmaxf(v, dpp_mov<0x4E>(v));
  v = fmaxf(v, dpp_mov<0x12C>(v));
  v = fmaxf(v, dpp_mov<0x128>(v));
  float a, b;
  swap16(v, a, b);
  v = fmaxf(a, b);
  swap32(v, a, b);
  return fmaxf(a, b);
}
__device__ __forceinline__ float class2_sum(float v) {
  v = dpp_add<0x4E>(v);
  v = dpp_add<0x12C>(v);
  v = dpp_add<0x128>(v);
  return rows_sum4(v);
}

// Sum over the wave, the same value in every lane.
__device__ __forceinline__ float wave_total(float v) { return rows_sum4(row16_sum(v)); }

// Sum over the wave; uniform result.
__device__ __forceinline__ float wave_sum(float v) {
  v = row16_sum(v);
  float a = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
  float b = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
  float c = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
  float d = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
  return (a + b) + (c + d);
}

__device__ __forceinline__ float wave_max(float v) {
  for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
  return v;
}

__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
  for (int o = 32; o >= 1; o >>= 1) {
    uint64_t w = __shfl_xor(v, o);
    v = w > v ? w : v;
  }
  return v;
}

// The same maxima by DPP (quads, then rotations inside each 16-lane row) and the row swaps, on
// the VALU instead of the LDS crossbar.  Every lane of the wave must be active.
__device__ __forceinline__ float wave_max_all(float v) {
  v = fmaxf(v, dpp_mov<0xB1>(v));   // quad_perm [1,0,3,2]
  v = fmaxf(v, dpp_mov<0x4E>(v));   // quad_perm [2,3,0,1]
  v = fmaxf(v, dpp_mov<0x12C>(v));  // row_ror:12
  v = fmaxf(v, dpp_mov<0x128>(v));  // row_ror:8
  float a, b;
  swap16(v, a, b);
  v = fmaxf(a, b);
  swap32(v, a, b);
  return fmaxf(a, b);
}

__device__ __forceinline__ uint64_t wave_max_u64_all(uint64_t v) {
  auto take = [&v](uint32_t lo, uint32_t hi) {
    const uint64_t w = ((uint64_t)hi << 32) | lo;
    v = w > v ? w : v;
  };
  auto dpp = [](uint64_t x, auto ctrl) {
    return std::pair<uint32_t, uint32_t>(
        (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)x, decltype(ctrl)::value, 0xf, 0xf, false),
        (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)(x >> 32), decltype(ctrl)::value, 0xf, 0xf, false));
  };
  {
    const auto p = dpp(v, std::integral_constant<int, 0xB1>());
    take(p.first, p.second);
  }
  {
    const auto p = dpp(v, std::integral_constant<int, 0x4E>());
    take(p.first, p.second);
  }
  {
    const auto p = dpp(v, std::integral_constant<int, 0x124>());
    take(p.first, p.second);
  }
  {
    const auto p = dpp(v, std::integral_constant<int, 0x128>());
    take(p.first, p.second);
  }
  {
    const auto lo = __builtin_amdgcn_permlane16_swap((uint32_t)v, (uint32_t)v, false, false);
    const auto hi = __builtin_amdgcn_permlane16_swap((uint32_t)(v >> 32), (uint32_t)(v >> 32), false, false);
    take(lo[0], hi[0]);
    take(lo[1], hi[1]);
  }
  {
    const auto lo = __builtin_amdgcn_permlane32_swap((uint32_t)v, (uint32_t)v, false, false);
    const auto hi = __builtin_amdgcn_permlane32_swap((uint32_t)(v >> 32), (uint32_t)(v >> 32), false, false);
    take(lo[0], hi[0]);
    take(lo[1], hi[1]);
  }
  return v;
}

// ------------------------------------------------------------ memory

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), 0, bytes, 0x00020000);
}

// Global-memory loads.  Pointers that reach the kernel through the LDS copy of
// the layer table are generic, and a generic load compiles to a FLAT
// instruction, which also counts in lgkmcnt; the s_waitcnt lgkmcnt(0) of every
// workgroup barrier would then wait for all weight prefetches in flight.  The
// address-space cast makes these VMEM-only (global_load), so only the
// instructions that consume the data wait for it.
template <class T>
using gptr = const __attribute__((address_space(1))) T*;

template <class T>
__device__ __forceinline__ gptr<T> as_global(const void* p) {
  return (gptr<T>)(p);
}

// Streaming 16-byte weight load (non-temporal: weights are read once per token).
__device__ __forceinline__ u32x4 ld_stream(const void* p) { return __builtin_nontemporal_load(as_global<u32x4>(p)); }

__device__ __forceinline__ u32x4 ld16(const void* p) { return *as_global<u32x4>(p); }
__device__ __forceinline__ uint32_t ld32(const void* p) { return *as_global<uint32_t>(p); }
__device__ __forceinline__ uint32_t ldu16(const void* p) { return *as_global<uint16_t>(p); }

// s_waitcnt immediates (gfx9 encoding: vmcnt [3:0] + [15:14], expcnt [6:4],
// lgkmcnt [11:8]); a field at its maximum does not wait.
constexpr int kWaitLgkm0 = 0xF | (0x3 << 14) | (0x7 << 4);  // lgkmcnt(0) only

// Waits until at most n vector-memory operations of this wave are outstanding
// (n <= 12; larger n waits for 12, which is safe, only later than needed).
__device__ __forceinline__ void wait_vmcnt(int n) {
  constexpr int kKeep = (0x7 << 4) | (0xF << 8);
  switch (n) {
    case 0: __builtin_amdgcn_s_waitcnt(0 | kKeep); break;
    case 1: __builtin_amdgcn_s_waitcnt(1 | kKeep); break;
    case 2: __builtin_amdgcn_s_waitcnt(2 | kKeep); break;
    case 3: __builtin_amdgcn_s_waitcnt(3 | kKeep); break;
    case 4: __builtin_amdgcn_s_waitcnt(4 | kKeep); break;
    case 5: __builtin_amdgcn_s_waitcnt(5 | kKeep); break;
    case 6: __builtin_amdgcn_s_waitcnt(6 | kKeep); break;
    case 7: __builtin_amdgcn_s_waitcnt(7 | kKeep); break;
    case 8: __builtin_amdgcn_s_waitcnt(8 | kKeep); break;
    case 9: __builtin_amdgcn_s_waitcnt(9 | kKeep); break;
    case 10: __builtin_amdgcn_s_waitcnt(10 | kKeep); break;
    case 11: __builtin_amdgcn_s_waitcnt(11 | kKeep); break;
    default: __builtin_amdgcn_s_waitcnt(12 | kKeep); break;
  }
  asm volatile("" ::: "memory");  // LDS written by the completed loads is read only after this point
}

// The same for a compile-time count up to 63 (the whole vmcnt range).
template <int N>
__device__ __forceinline__ void wait_vmcnt_upto() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
  asm volatile("" ::: "memory");
}

// ------------------------------------------------------- tagged exchange

constexpr uint32_t kTimeoutDefault = 100u * 1000u * 1000u;  // 1 s of the 100 MHz wall clock

// Error bits written to the state word (and mirrored to the host word).
enum : uint32_t {
  kErrTimeout = 1u,
  kErrPosition = 2u,
  kErrToken = 4u,
  kErrPoisoned = 8u,
};

__device__ __forceinline__ uint32_t make_tag(uint32_t epoch, uint32_t k) { return ((epoch + k) % 65535u) + 1u; }

__device__ __forceinline__ uint32_t word(uint32_t payload16, uint32_t tag) { return (payload16 << 16) | tag; }

__device__ __forceinline__ bool chunk_ok(u32x4 v, uint32_t tag) {
  return ((v.x & 0xffffu) == tag) & ((v.y & 0xffffu) == tag) & ((v.z & 0xffffu) == tag) & ((v.w & 0xffffu) == tag);
}

// Store four words (16 bytes) at word index ``w``.  XCD-visible stores write
// through to the device-coherent level; XCD-local ones stay in this XCD's L2,
// which is where the same-XCD consumers' device-scope loads find them.
template <bool DEVICE>
__device__ __forceinline__ void put4(uint32_t* buf, uint32_t w, u32x4 v) {
  auto rs = make_rsrc(buf, 0x7fffffffu);
  if (DEVICE)
    __builtin_amdgcn_raw_buffer_store_b128(v, rs, w * 4u, 0, 0x10 /* sc1 */);
  else
    __builtin_amdgcn_raw_buffer_store_b128(v, rs, w * 4u, 0, 0);
}

// Two words (8 bytes) at word index ``w`` (even), same scopes as put4.
__device__ __forceinline__ void put2(uint32_t* buf, uint32_t w, uint32_t w0, uint32_t w1, bool device) {
  typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
  auto rs = make_rsrc(buf, 0x7fffffffu);
  u32x2 v;
  v.x = w0;
  v.y = w1;
  if (device)
    __builtin_amdgcn_raw_buffer_store_b64(v, rs, w * 4u, 0, 0x10 /* sc1 */);
  else
    __builtin_amdgcn_raw_buffer_store_b64(v, rs, w * 4u, 0, 0);
}

// An fp32 value as two tagged words: high 16 bits first, then the low 16 bits.
__device__ __forceinline__ uint32_t f32_hi_word(float v, uint32_t tag) { return (__float_as_uint(v) & 0xffff0000u) | tag; }
__device__ __forceinline__ uint32_t f32_lo_word(float v, uint32_t tag) { return (__float_as_uint(v) << 16) | tag; }

__device__ __forceinline__ void put1_device(uint32_t* p, uint32_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Eight sums over the wave at once: lanes 8k..8k+7 receive the sum over all 64
// lanes of v[k].  Each step halves the values a lane carries and adds its
// partner's copy of the ones it keeps: the half-wave swap (lanes l, l ^ 32) and
// the row-pair swap (l, l ^ 16) on the gfx950 permlane swaps, a rotation by 8
// inside each 16-lane row (l, l ^ 8) on DPP; three DPP adds then sum each group
// of eight lanes.  About 20 instructions for eight sums, against about 90 for
// eight separate wave reductions.
__device__ __forceinline__ float wave_sum8(const float (&v)[8], int lane) {
  float w[4];
#pragma unroll
  for (int j = 0; j < 4; j++) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v[j]), __float_as_uint(v[j + 4]), false, false);
    w[j] = __uint_as_float(r[0]) + __uint_as_float(r[1]);  // lanes 0-31: v[j], lanes 32-63: v[j + 4]
  }
  float z[2];
#pragma unroll
  for (int j = 0; j < 2; j++) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(w[j]), __float_as_uint(w[j + 2]), false, false);
    z[j] = __uint_as_float(r[0]) + __uint_as_float(r[1]);  // even rows: w[j], odd rows: w[j + 2]
  }
  const bool hi = (lane & 8) != 0;
  float x = (hi ? z[1] : z[0]) + dpp_get<0x128>(hi ? z[0] : z[1]);  // row_ror:8, i.e. lane ^ 8
  x = dpp_add<0xB1>(x);   // quad_perm [1,0,3,2]
  x = dpp_add<0x4E>(x);   // quad_perm [2,3,0,1]
  x = dpp_add<0x141>(x);  // row_half_mirror: the other quad of the eight lanes
  return x;
}

// This lane's share of a row's dot product (NL 16-byte chunks of weights and activations).
template <int NL>
__device__ __forceinline__ float row_part(const u32x4* w, const u32x4 (&x)[NL]) {
  float acc = 0.f;
#pragma unroll
  for (int j = 0; j < NL; j++) acc = dot8(w[j], x[j], acc);
  return acc;
}

// One 4-byte word at word index ``w``, same scopes as put4.
__device__ __forceinline__ void put1(uint32_t* buf, uint32_t w, uint32_t v, bool device) {
  auto rs = make_rsrc(buf, 0x7fffffffu);
  if (device)
    __builtin_amdgcn_raw_buffer_store_b32(v, rs, w * 4u, 0, 0x10 /* sc1 */);
  else
    __builtin_amdgcn_raw_buffer_store_b32(v, rs, w * 4u, 0, 0);
}

__device__ __forceinline__ u32x4 poll16(__amdgpu_buffer_rsrc_t rs, uint32_t byte_off) {
  return __builtin_amdgcn_raw_buffer_load_b128(rs, byte_off, 0, 0x10 /* sc1: miss the non-coherent caches */);
}

}  // namespace qmk
