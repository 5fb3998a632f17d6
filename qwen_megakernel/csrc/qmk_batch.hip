// Batched forward of T tokens through Qwen3 on gfx950: prompt prefill (T
// tokens of one sequence at consecutive positions) and batched decode (one
// token of each of B sequences, each at its own position), or any mix.
// Unlike the per-token decode kernel, the work here has T rows per weight
// read, so the projections run as MFMA GEMMs (v_mfma_f32_16x16x32_bf16) and a
// layer is a short sequence of kernels on the caller's stream instead of one
// persistent launch.  Numerics follow HF Qwen3's bf16 eager path op for op, as
// the decode kernel does: every projection is an fp32 sum rounded once to
// bf16; norms, RoPE, softmax probabilities, residual adds and SiLU*up round
// where HF rounds.
//
// The reference prefills one token per step() (qwen_megakernel/model.py:210-211)
// and decodes one sequence; the batched forward is an addition.
//
// Per layer (kernels in launch order):
//   gemm_tiled(qkv)    -> qkv_finish (split-K sum, q/k RMSNorm + RoPE, K/V append;
//                         in the GEMM's epilogue when K is not split)
//   attention          (one kernel per (token, KV head) for many tokens; a
//                       context-split pair + merge for few tokens)
//   gemm_tiled(o)      -> residual_norm (residual add, post-attention RMSNorm)
//   gemm_tiled(g|u)    -> gate_up_finish (SiLU(g) * u; in the GEMM's epilogue when K
//                         is not split)
//   gemm_tiled(down)   -> residual_norm (residual add, next layer's input RMSNorm
//                                        or the final norm)
// then lm_head_gemm over the emitted rows (bf16 logits, per-tile argmax keys)
// -> keys_reduce (per-row argmax).

#include <hip/hip_runtime.h>

#include <algorithm>

#include "../../include/qwen_megakernel.h"
#include "qmk_batch_decode.h"
#include "qmk_decode_kernel.h"

namespace qmk {
namespace batch {


constexpr int kD = 128, kNQ = 16, kNKV = 8, kQS = kNQ * kD, kNQKV = (kNQ + 2 * kNKV) * kD;
constexpr int kAttnChunk = 2048;  // one-kernel attention: scores of this many positions per LDS pass
constexpr int kQT = 64, kKB = 64, kKPad = kD + 8, kVPad = kKB + 8;  // MFMA prefill attention tiles
constexpr int kMfmaAttnTokens = 320;   // prompts of this many tokens run attention_mfma
constexpr int kMfmaAttnContext = 256;  // so do fewer tokens over this many positions of context
constexpr int kMaxAttnChunks = 16;    // attention_mfma over key chunks: tiles x chunks at most
constexpr int kSplitChunk = 64;   // split attention: positions per workgroup
constexpr int kSplitBelow = 32;   // fewer tokens than this use the split attention ...
constexpr int kSplitContext = 128;  // ... over more than this many positions of context
constexpr int kMaxSplit = 16;     // K splits of one GEMM (their partials are summed in a fixed order)
constexpr int kMaxEmit = 256;

static_assert(Qwen3_0_6B::D == kD && Qwen3_0_6B::NQ == kNQ && Qwen3_0_6B::NKV == kNKV, "head layout");
static_assert(Qwen3_1_7B::D == kD && Qwen3_1_7B::NQ == kNQ && Qwen3_1_7B::NKV == kNKV, "head layout");

// Per-token metadata, checked once (prep_tokens).  An invalid token (id outside
// the vocabulary, sequence or position out of range) reads embedding row 0,
// writes nothing into any cache and emits -1.
struct Tok {
  int token, seq, pos, valid;
};

struct Cache {
  uint16_t* k;
  uint16_t* v;
  long long seq_stride;  // elements from one sequence's [L][NKV][S][D] block to the next
  int max_seq_len;
};

__device__ __forceinline__ bf16x8 ld_bf16x8(const uint16_t* p) { return __builtin_bit_cast(bf16x8, ld16(p)); }
__device__ __forceinline__ bf16x8 ld_bf16x8_stream(const uint16_t* p) {
  return __builtin_bit_cast(bf16x8, ld_stream(p));
}

__device__ __forceinline__ size_t cache_base(const Cache& c, const Tok& tk, int L, int g) {
  return (size_t)tk.seq * c.seq_stride + ((size_t)L * kNKV + g) * c.max_seq_len * kD;
}

// Sum over the block (256 threads) of one value per head; `red` is [2][4].
__device__ __forceinline__ void block_sum2(float (&v)[2], float (*red)[4]) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  v[0] = wave_sum(v[0]);
  v[1] = wave_sum(v[1]);
  __syncthreads();
  if (lane == 0) {
    red[0][wave] = v[0];
    red[1][wave] = v[1];
  }
  __syncthreads();
#pragma unroll
  for (int h = 0; h < 2; h++) v[h] = (red[h][0] + red[h][1]) + (red[h][2] + red[h][3]);
}

__device__ __forceinline__ void block_max2(float (&v)[2], float (*red)[4]) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  v[0] = wave_max(v[0]);
  v[1] = wave_max(v[1]);
  __syncthreads();
  if (lane == 0) {
    red[0][wave] = v[0];
    red[1][wave] = v[1];
  }
  __syncthreads();
#pragma unroll
  for (int h = 0; h < 2; h++) v[h] = fmaxf(fmaxf(red[h][0], red[h][1]), fmaxf(red[h][2], red[h][3]));
}

// ---------------------------------------------------------------- tokens

__global__ void __launch_bounds__(256) prep_tokens(const int* __restrict__ tokens, const int* __restrict__ seqs,
                                                   const int* __restrict__ pos, int T, const int* __restrict__ emit,
                                                   int R, int num_seqs, int max_context, int vocab,
                                                   Tok* __restrict__ tok, int* __restrict__ erow) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i < T) {
    const int id = tokens[i], sq = seqs ? seqs[i] : i, p = pos[i];
    const bool ok = id >= 0 && id < vocab && sq >= 0 && sq < num_seqs && p >= 0 && p < max_context;
    tok[i] = Tok{ok ? id : 0, ok ? sq : 0, ok ? p : 0, ok ? 1 : 0};
  }
  if (i < R) {
    const int e = emit ? emit[i] : i;
    erow[i] = (e >= 0 && e < T) ? e : -1;
  }
}

// X[t] = embed[token[t]]
__global__ void __launch_bounds__(256) embed_rows(const uint16_t* __restrict__ embed, const Tok* __restrict__ tok,
                                                  int H, uint16_t* __restrict__ X) {
  const int t = blockIdx.x;
  const uint16_t* e = embed + (size_t)tok[t].token * H;
  for (int i = threadIdx.x; i < H / 8; i += 256) reinterpret_cast<u32x4*>(X + (size_t)t * H)[i] = ld16(e + 8 * i);
}

// ---------------------------------------------------------------- GEMM
//
// W rows come from up to three row-major [rows][K] matrices laid end to end
// (q, k, v; or gate, up).  The GEMMs run on 16x16x32 bf16 MFMAs, whose
// operand layouts (checked by qmk_selftest_mfma) are: lane l supplies
// A[l%16][8*(l/16) .. +7] and B[8*(l/16) .. +7][l%16], i.e. 16 contiguous bytes
// of an X row and of a W row; it receives C[4*(l/16) + i][l%16], i = 0..3.
struct Seg {
  const uint16_t* w[3];
  int rows[3];
};

__device__ __forceinline__ const uint16_t* seg_row(const Seg& s, int n, int K) {
  if (n < s.rows[0]) return s.w[0] + (size_t)n * K;
  n -= s.rows[0];
  if (n < s.rows[1]) return s.w[1] + (size_t)n * K;
  n -= s.rows[1];
  return s.w[2] + (size_t)n * K;
}

// The work after the q/k/v projection for one (token, head) of the 32 q/k/v heads, one wave,
// lane l holding the head's bf16-rounded projections x0 = column l, x1 = column l + 64: q:
// RMSNorm over head_dim + RoPE -> Q;  k: the same -> K cache at the token's position;  v: -> V
// cache.  (modeling_qwen3.py:252-253, 168)
struct QkvOut {
  const Tok* tok;
  int L;
  const uint16_t* q_norm;
  const uint16_t* k_norm;
  const uint16_t* cos_t;
  const uint16_t* sin_t;
  Cache c;
  float eps;
  uint16_t* Q;
};

__device__ __forceinline__ void qkv_head(const QkvOut& o, int t, int h, int lane, float x0, float x1) {
  const Tok tk = o.tok[t];
  if (h >= kNQ + kNKV) {
    if (tk.valid) {
      uint16_t* dst = o.c.v + cache_base(o.c, tk, o.L, h - kNQ - kNKV) + (size_t)tk.pos * kD;
      dst[lane] = (uint16_t)f32_to_bf16(x0);
      dst[lane + 64] = (uint16_t)f32_to_bf16(x1);
    }
    return;
  }
  const bool is_q = h < kNQ;
  if (!is_q && !tk.valid) return;
  const uint16_t* nw = is_q ? o.q_norm : o.k_norm;
  const uint16_t* cr = o.cos_t + (size_t)tk.pos * kD;
  const uint16_t* sr = o.sin_t + (size_t)tk.pos * kD;
  const float ss = wave_sum(x0 * x0 + x1 * x1);
  const float rstd = rcp_sqrt_torch(__fdiv_rn(ss, (float)kD) + o.eps);
  const float n0 = bf16r(bf16_to_f32(ldu16(nw + lane)) * bf16r(x0 * rstd));
  const float n1 = bf16r(bf16_to_f32(ldu16(nw + lane + 64)) * bf16r(x1 * rstd));
  const float c0 = bf16_to_f32(ldu16(cr + lane)), c1 = bf16_to_f32(ldu16(cr + lane + 64));
  const float s0 = bf16_to_f32(ldu16(sr + lane)), s1 = bf16_to_f32(ldu16(sr + lane + 64));
  // x*cos + rotate_half(x)*sin, rotate_half(x) = (-x[64:], x[:64])
  const float y0 = bf16r(bf16r(n0 * c0) + bf16r(-n1 * s0));
  const float y1 = bf16r(bf16r(n1 * c1) + bf16r(n0 * s1));
  uint16_t* dst =
      is_q ? o.Q + (size_t)t * kQS + h * kD : o.c.k + cache_base(o.c, tk, o.L, h - kNQ) + (size_t)tk.pos * kD;
  dst[lane] = (uint16_t)f32_to_bf16(y0);
  dst[lane + 64] = (uint16_t)f32_to_bf16(y1);
}

// qkv_head for the 128 rows x 128 columns of one head held in LDS (bf16), rows t0.. (those
// below T): wave w takes rows 32w..32w+31, four at a time, 16 lanes per row; lane c of a row
// holds columns 4c..4c+3 and their RoPE partners 64+4c..64+4c+3.  The sum of squares runs over
// the row's 16 lanes.  Everything the rows read from global memory besides the tile (their token
// records, then their cos/sin entries, and the head-norm weights) is requested up front by
// qkv_rows_fetch, before the tile goes through LDS, so the eight row groups do not each wait for
// two dependent loads.
struct QkvRowsIn {
  Tok tk[8];
  uint2 cl[8], ch[8], sl[8], sh[8];
  float nw[8];
};

__device__ __forceinline__ void qkv_rows_fetch(const QkvOut& o, int t0, int T, int h, int w, int lane, QkvRowsIn& in) {
  const int c = lane & 15, sub = lane >> 4;
  const bool is_v = h >= kNQ + kNKV, is_q = h < kNQ;
#pragma unroll
  for (int it = 0; it < 8; it++) {
    const int t = t0 + 32 * w + 4 * it + sub;
    in.tk[it] = o.tok[t < T ? t : t0];
  }
  if (is_v) return;
  const uint16_t* wp = is_q ? o.q_norm : o.k_norm;
#pragma unroll
  for (int e = 0; e < 4; e++) {
    in.nw[e] = bf16_to_f32(ldu16(wp + 4 * c + e));
    in.nw[4 + e] = bf16_to_f32(ldu16(wp + 64 + 4 * c + e));
  }
#pragma unroll
  for (int it = 0; it < 8; it++) {
    const size_t pb = (size_t)in.tk[it].pos * kD;
    in.cl[it] = *reinterpret_cast<const uint2*>(o.cos_t + pb + 4 * c);
    in.ch[it] = *reinterpret_cast<const uint2*>(o.cos_t + pb + 64 + 4 * c);
    in.sl[it] = *reinterpret_cast<const uint2*>(o.sin_t + pb + 4 * c);
    in.sh[it] = *reinterpret_cast<const uint2*>(o.sin_t + pb + 64 + 4 * c);
  }
}

__device__ __forceinline__ void qkv_tile_rows(const QkvOut& o, const uint16_t (*Xh)[128], int t0, int T, int h, int w,
                                              int lane, const QkvRowsIn& in) {
  const int c = lane & 15, sub = lane >> 4;
  const bool is_v = h >= kNQ + kNKV, is_q = h < kNQ;
#pragma unroll
  for (int it = 0; it < 8; it++) {
    const int row = 32 * w + 4 * it + sub, t = t0 + row;
    if (t0 + 32 * w + 4 * it >= T) break;  // uniform: no row of this group is below T
    const bool live = t < T;
    const Tok tk = in.tk[it];
    const uint2 lo = *reinterpret_cast<const uint2*>(&Xh[row][4 * c]);
    const uint2 hi = *reinterpret_cast<const uint2*>(&Xh[row][64 + 4 * c]);
    float x[8] = {lo_bf16(lo.x), hi_bf16(lo.x), lo_bf16(lo.y), hi_bf16(lo.y),
                  lo_bf16(hi.x), hi_bf16(hi.x), lo_bf16(hi.y), hi_bf16(hi.y)};
    if (is_v) {
      if (live && tk.valid) {
        uint16_t* dst = o.c.v + cache_base(o.c, tk, o.L, h - kNQ - kNKV) + (size_t)tk.pos * kD;
        *reinterpret_cast<uint2*>(dst + 4 * c) = lo;
        *reinterpret_cast<uint2*>(dst + 64 + 4 * c) = hi;
      }
      continue;
    }
    float ss = 0.f;
#pragma unroll
    for (int e = 0; e < 8; e++) ss += x[e] * x[e];
#pragma unroll
    for (int m = 1; m < 16; m <<= 1) ss += __shfl_xor(ss, m);  // within the row's 16 lanes
    const float rstd = rcp_sqrt_torch(__fdiv_rn(ss, (float)kD) + o.eps);
    float n[8];
#pragma unroll
    for (int e = 0; e < 8; e++) n[e] = bf16r(in.nw[e] * bf16r(x[e] * rstd));
    const uint2 cl = in.cl[it], ch = in.ch[it], sl = in.sl[it], sh = in.sh[it];
    const float cs[8] = {lo_bf16(cl.x), hi_bf16(cl.x), lo_bf16(cl.y), hi_bf16(cl.y),
                         lo_bf16(ch.x), hi_bf16(ch.x), lo_bf16(ch.y), hi_bf16(ch.y)};
    const float sn[8] = {lo_bf16(sl.x), hi_bf16(sl.x), lo_bf16(sl.y), hi_bf16(sl.y),
                         lo_bf16(sh.x), hi_bf16(sh.x), lo_bf16(sh.y), hi_bf16(sh.y)};
    // x*cos + rotate_half(x)*sin, rotate_half(x) = (-x[64:], x[:64])
    float y[8];
#pragma unroll
    for (int e = 0; e < 4; e++) {
      y[e] = bf16r(bf16r(n[e] * cs[e]) + bf16r(-n[4 + e] * sn[e]));
      y[4 + e] = bf16r(bf16r(n[4 + e] * cs[4 + e]) + bf16r(n[e] * sn[4 + e]));
    }
    if (!live || (!is_q && !tk.valid)) continue;
    uint16_t* dst =
        is_q ? o.Q + (size_t)t * kQS + h * kD : o.c.k + cache_base(o.c, tk, o.L, h - kNQ) + (size_t)tk.pos * kD;
    *reinterpret_cast<uint2*>(dst + 4 * c) = make_uint2(pack_bf16x2(y[0], y[1]), pack_bf16x2(y[2], y[3]));
    *reinterpret_cast<uint2*>(dst + 64 + 4 * c) = make_uint2(pack_bf16x2(y[4], y[5]), pack_bf16x2(y[6], y[7]));
  }
}

// SiLU(g) * u as HF rounds it: bf16(bf16(silu(g)) * u), g and u bf16 (modeling_qwen3.py:82)
__device__ __forceinline__ float silu_mul(float g, float u) {
  const float sg = bf16r(__fdiv_rn(g, 1.0f + expf(-g)));
  return bf16r(sg * u);
}

// What gemm_tiled does with its sums: kEpiPart writes them to part (any K split); with the K
// range unsplit, kEpiQkv (128-column tiles = one q/k/v head each) runs the head's norm, RoPE and
// K/V append (qkv_head) and kEpiGateUp (tile columns 0..63 the gate rows m0..m0+63, 64..127
// the up rows of the same m) writes bf16(bf16(silu(g)) * u) to M, so neither the fp32 sums nor
// a finishing kernel touch memory.
enum { kEpiPart = 0, kEpiQkv = 1, kEpiGateUp = 2 };

struct GateUpOut {
  uint16_t* M;
  int I;
};

// Large T (prompt prefill): an LDS-tiled MFMA GEMM, part[z][t][n] = the sum
// over K split z of X[t][k] W[n][k].  Workgroup tile 128 rows x TN columns
// (TN = 128, or 64 for narrow N so that more workgroups run), BK = 64; wave w
// computes rows 64*(w&1)..+63 x columns (TN/2)*(w>>1)..+TN/2-1 as 4 x TN/32
// MFMA tiles.  Both operands go from global memory straight into LDS (LDS DMA,
// 16 bytes per lane) through two stages: step s+1's requests are issued right
// after the barrier that opens step s, so they land during step s's MFMAs.
// A stage row is 64 bf16, eight 16-byte chunks; chunk c of row r sits at
// position c ^ (r & 7), so the lanes that read one chunk of 8 consecutive rows
// touch every LDS bank once.  Two workgroups per CU (64 KB of LDS each).
// Measured at 2048 tokens against the same tiles staged through registers
// with padded rows: q/k/v 27.5 -> 22.4 us, gate/up 41.3 -> 32.5, o 19.4 ->
// 17.4, down 24.7 -> 22.9 (bit-identical sums: the K order is unchanged).
constexpr int kTM = 128, kTK = 64;

// 16 bytes per lane from global memory straight into LDS: lane i's bytes land at lds + 16 i (lds
// is the same for every lane of the wave)
__device__ __forceinline__ void dma16(const void* src, void* lds) {
  __builtin_amdgcn_global_load_lds(as_global<void>(src), (__attribute__((address_space(3))) void*)lds, 16, 0, 0);
}

template <int TN, int EPI = kEpiPart>
__global__ void __launch_bounds__(256, 2) gemm_tiled(const uint16_t* __restrict__ X, int T, int K, Seg seg, int N,
                                                     int ksplit, float* __restrict__ part, QkvOut qo, GateUpOut go) {
  static_assert(TN == 64 || TN == 128, "tile width");
  static_assert(EPI == kEpiPart || TN == 128, "fused epilogues take 128-column tiles");
  constexpr int WJ = TN / 32;  // 16-column MFMA tiles per wave (a wave covers TN / 2 columns)
  constexpr int ABytes = kTM * kTK * 2, BBytes = TN * kTK * 2, StB = ABytes + BBytes;
  constexpr int NA = ABytes / 4096, NB = BBytes / 4096;  // 1 KB DMA blocks (8 rows) per wave and stage
  __shared__ __align__(1024) unsigned char sm[2 * StB];
  const int n0 = blockIdx.x * TN, t0 = blockIdx.y * kTM;
  // K split z of ksplit (blockIdx.z): columns [kz, kz + K / ksplit); partial sums to part[z]
  const int kz = blockIdx.z * (K / ksplit);
  part += (size_t)blockIdx.z * T * N;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int wm = w & 1, wn = w >> 1;
  // DMA block q of wave w holds rows 8 (NA w + q) .. +7 of A (of B: NB); lane l fills position
  // l % 8 of row l / 8 of the block, i.e. it requests chunk (l % 8) ^ (row & 7) of that row
  const uint16_t* asrc[NA];
  const uint16_t* bsrc[NB];
#pragma unroll
  for (int q = 0; q < NA; q++) {
    const int row = 8 * (NA * w + q) + (lane >> 3), c = (lane & 7) ^ (row & 7);
    asrc[q] = X + (size_t)min(t0 + row, T - 1) * K + kz + 8 * c;
  }
#pragma unroll
  for (int q = 0; q < NB; q++) {
    const int row = 8 * (NB * w + q) + (lane >> 3), c = (lane & 7) ^ (row & 7);
    if constexpr (EPI == kEpiGateUp)  // tile columns 0..63: gate rows m0.., 64..127: up rows m0..
      bsrc[q] = seg.w[row >> 6] + (size_t)(n0 / 2 + (row & 63)) * K + kz + 8 * c;
    else
      bsrc[q] = seg_row(seg, n0 + row, K) + kz + 8 * c;
  }
  auto issue = [&](int st) {
    const int k = st * kTK;
    unsigned char* base = sm + (st & 1) * StB;
#pragma unroll
    for (int q = 0; q < NA; q++) dma16(asrc[q] + k, base + 1024 * (NA * w + q));
#pragma unroll
    for (int q = 0; q < NB; q++) dma16(bsrc[q] + k, base + ABytes + 1024 * (NB * w + q));
  };
  f32x4 acc[4][WJ];
#pragma unroll
  for (int i = 0; i < 4; i++)
#pragma unroll
    for (int j = 0; j < WJ; j++) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  const int l16 = lane & 15, lq = lane >> 4;
  const int steps = K / ksplit / kTK;
  issue(0);
  for (int st = 0; st < steps; st++) {
    wait_vmcnt(0);    // this wave's requests of step st have landed
    __syncthreads();  // every wave's have, and step st - 1's stage is read
    if (st + 1 < steps) issue(st + 1);
    const unsigned char* base = sm + (st & 1) * StB;
#pragma unroll
    for (int kc = 0; kc < kTK / 8; kc += 4) {  // 32 K per MFMA: chunks kc..kc+3, lane chunk kc + lq
      bf16x8 a[4], b[WJ];
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int row = 64 * wm + 16 * i + l16;
        a[i] = *reinterpret_cast<const bf16x8*>(base + row * (kTK * 2) + 16 * ((kc + lq) ^ (row & 7)));
      }
#pragma unroll
      for (int j = 0; j < WJ; j++) {
        const int row = (TN / 2) * wn + 16 * j + l16;
        b[j] = *reinterpret_cast<const bf16x8*>(base + ABytes + row * (kTK * 2) + 16 * ((kc + lq) ^ (row & 7)));
      }
#pragma unroll
      for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < WJ; j++) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[i], b[j], acc[i][j], 0, 0, 0);
    }
  }
  if constexpr (EPI == kEpiPart) {
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
      for (int j = 0; j < WJ; j++) {
        const int n = n0 + (TN / 2) * wn + 16 * j + l16;
#pragma unroll
        for (int r = 0; r < 4; r++) {
          const int t = t0 + 64 * wm + 16 * i + 4 * (lane >> 4) + r;
          if (t < T) part[(size_t)t * N + n] = acc[i][j][r];
        }
      }
  } else if constexpr (EPI == kEpiQkv) {
    // the tile's 128 rows x 128 columns (one head), bf16-rounded, through LDS: then wave w takes
    // rows 32w..32w+31 one at a time, lane l columns l and l + 64
    static_assert(sizeof(sm) >= kTM * 128 * 2, "the head tile fits the operand stages");
    auto Xh = reinterpret_cast<uint16_t(*)[128]>(sm);
    QkvRowsIn in;
    qkv_rows_fetch(qo, t0, T, blockIdx.x, w, lane, in);
    __syncthreads();  // every wave's last operand reads are done
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
      for (int j = 0; j < WJ; j++)
#pragma unroll
        for (int r = 0; r < 4; r++)
          Xh[64 * wm + 16 * i + 4 * (lane >> 4) + r][64 * wn + 16 * j + l16] = (uint16_t)f32_to_bf16(acc[i][j][r]);
    __syncthreads();
    qkv_tile_rows(qo, Xh, t0, T, blockIdx.x, w, lane, in);
  } else {
    // the tile's gate and up projections, bf16-rounded, through LDS: G[row][c], U[row][c] for
    // m = m0 + c; then each thread takes 8 consecutive m of one row at a time and stores them
    // as one 16-byte chunk
    static_assert(sizeof(sm) >= 2 * kTM * 64 * 2, "the gate and up tiles fit the operand stages");
    auto G = reinterpret_cast<uint16_t(*)[64]>(sm);
    auto U = G + kTM;
    __syncthreads();  // every wave's last operand reads are done
    auto GU = wn == 0 ? G : U;
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
      for (int j = 0; j < WJ; j++)
#pragma unroll
        for (int r = 0; r < 4; r++)
          GU[64 * wm + 16 * i + 4 * (lane >> 4) + r][16 * j + l16] = (uint16_t)f32_to_bf16(acc[i][j][r]);
    __syncthreads();
    const int m0 = n0 / 2, row = threadIdx.x >> 1, t = t0 + row;
    if (t < T) {
#pragma unroll
      for (int q = 0; q < 4; q++) {
        const int c0 = 32 * (threadIdx.x & 1) + 8 * q;
        const u32x4 g8 = *reinterpret_cast<const u32x4*>(&G[row][c0]);
        const u32x4 u8 = *reinterpret_cast<const u32x4*>(&U[row][c0]);
        const uint32_t gw[4] = {g8.x, g8.y, g8.z, g8.w}, uw[4] = {u8.x, u8.y, u8.z, u8.w};
        uint32_t mw[4];
#pragma unroll
        for (int e = 0; e < 4; e++)
          mw[e] = pack_bf16x2(silu_mul(lo_bf16(gw[e]), lo_bf16(uw[e])), silu_mul(hi_bf16(gw[e]), hi_bf16(uw[e])));
        *reinterpret_cast<u32x4*>(go.M + (size_t)t * go.I + m0 + c0) = u32x4{mw[0], mw[1], mw[2], mw[3]};
      }
    }
  }
}

// Sum of the K-split partials of element (t, n), in split order.  All loads
// are issued before the first add.
__device__ __forceinline__ float sum_splits(const float* part, int ksplit, int T, int N, int t, int n) {
  const size_t stride = (size_t)T * N, idx = (size_t)t * N + n;
  float v[kMaxSplit];
#pragma unroll
  for (int s = 0; s < kMaxSplit; s++) v[s] = s < ksplit ? part[s * stride + idx] : 0.f;
  float y = v[0];
#pragma unroll
  for (int s = 1; s < kMaxSplit; s++)
    if (s < ksplit) y += v[s];
  return y;
}

// ---------------------------------------------------------------- row kernels

// One workgroup of 256 threads per token, J = H / 256 consecutive elements per
// thread (16-byte partial loads, 8- or 16-byte bf16 loads and stores).
// x = X[t] (+ bf16(sum of the split partials, in split order) when `part` is
// given, written back: HF's bf16 residual add);
// N[t] = bf16(w * bf16(x * rsqrt(mean(x^2) + eps))) (Qwen3RMSNorm).
// (At 2048 tokens, 4 splits: 12.2 us with one element per thread of 1024.)
template <int H>
__global__ void __launch_bounds__(256) residual_norm(const float* __restrict__ part, int ksplit, int T,
                                                     uint16_t* __restrict__ X, const uint16_t* __restrict__ w,
                                                     float eps, uint16_t* __restrict__ Nout) {
  constexpr int J = H / 256, JW = J / 2, JV = J / 4;  // elements, bf16 pairs, float4s per thread
  static_assert(J == 4 || J == 8, "four or eight elements per thread");
  typedef unsigned words_t __attribute__((ext_vector_type(JW)));
  __shared__ float red[4];
  const int t = blockIdx.x, wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int i0 = J * threadIdx.x;
  words_t* const xp = reinterpret_cast<words_t*>(X + (size_t)t * H + i0);
  const words_t xw = *xp;
  float y[J];
#pragma unroll
  for (int e = 0; e < JW; e++) {
    y[2 * e] = lo_bf16(xw[e]);
    y[2 * e + 1] = hi_bf16(xw[e]);
  }
  if (part) {
    const size_t stride = (size_t)T * H;
    const float* p0 = part + (size_t)t * H + i0;
    float sum[J];
    // the splits in groups of G: every load of a group is issued before its adds.  Groups of
    // four for few splits (2048 tokens, 4 splits: 8.0 us, against 8.9 with groups of 16), of 16
    // float4 registers for many (128 tokens, 16 splits: 3.8 us, against 4.3 with groups of 4)
    auto add_splits = [&](auto g) {
      constexpr int G = decltype(g)::value;
      for (int s0 = 0; s0 < ksplit; s0 += G) {
        f32x4 v[G][JV];
#pragma unroll
        for (int q = 0; q < G; q++)
          if (s0 + q < ksplit) {
#pragma unroll
            for (int c = 0; c < JV; c++) v[q][c] = *reinterpret_cast<const f32x4*>(p0 + (s0 + q) * stride + 4 * c);
          }
#pragma unroll
        for (int q = 0; q < G; q++)
          if (s0 + q < ksplit) {
#pragma unroll
            for (int j = 0; j < J; j++) sum[j] = s0 + q == 0 ? v[q][j / 4][j % 4] : sum[j] + v[q][j / 4][j % 4];
          }
      }
    };
    if (ksplit <= 4) add_splits(std::integral_constant<int, 4>{});
    else add_splits(std::integral_constant<int, 16 / JV>{});
    words_t out;
#pragma unroll
    for (int e = 0; e < JW; e++) {
      y[2 * e] = bf16r(y[2 * e] + bf16r(sum[2 * e]));
      y[2 * e + 1] = bf16r(y[2 * e + 1] + bf16r(sum[2 * e + 1]));
      out[e] = pack_bf16x2(y[2 * e], y[2 * e + 1]);
    }
    *xp = out;
  }
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < J; j++) ss += y[j] * y[j];
  ss = wave_sum(ss);
  if (lane == 0) red[wave] = ss;
  __syncthreads();
  ss = (red[0] + red[1]) + (red[2] + red[3]);
  const float rstd = rcp_sqrt_torch(__fdiv_rn(ss, (float)H) + eps);
  const words_t ww = *reinterpret_cast<const words_t*>(w + i0);
  words_t out;
#pragma unroll
  for (int e = 0; e < JW; e++)
    out[e] = pack_bf16x2(bf16r(lo_bf16(ww[e]) * bf16r(y[2 * e] * rstd)), bf16r(hi_bf16(ww[e]) * bf16r(y[2 * e + 1] * rstd)));
  *reinterpret_cast<words_t*>(Nout + (size_t)t * H + i0) = out;
}

// One wave per (token, head) of the 32 q/k/v heads.  Sums the split partials
// and rounds (the bf16 projections), then q: RMSNorm over head_dim + RoPE ->
// Q;  k: the same -> K cache at the token's position;  v: -> V cache.
// (modeling_qwen3.py:252-253, 168)
__global__ void __launch_bounds__(64) qkv_finish(const float* __restrict__ part, int ksplit, int T, QkvOut o) {
  const int t = blockIdx.x, h = blockIdx.y, lane = threadIdx.x;
  const float x0 = bf16r(sum_splits(part, ksplit, T, kNQKV, t, h * kD + lane));
  const float x1 = bf16r(sum_splits(part, ksplit, T, kNQKV, t, h * kD + lane + 64));
  qkv_head(o, t, h, lane, x0, x1);
}

// M[t][n] = bf16(bf16(silu(g)) * u); g and u are columns n and I + n of the
// gate/up product (modeling_qwen3.py:82).
__global__ void __launch_bounds__(256) gate_up_finish(const float* __restrict__ part, int ksplit, int T, int I,
                                                      uint16_t* __restrict__ M) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= (size_t)T * I) return;
  const int t = (int)(i / I), n = (int)(i % I);
  const float g = bf16r(sum_splits(part, ksplit, T, 2 * I, t, n));
  const float u = bf16r(sum_splits(part, ksplit, T, 2 * I, t, I + n));
  M[i] = (uint16_t)f32_to_bf16(silu_mul(g, u));
}

// ---------------------------------------------------------------- attention
//
// Eager GQA attention of token t over positions 0..pos of its sequence, for
// the two query heads of KV head g (modeling_qwen3.py:185-203): scores
// bf16(bf16(q.k) * scale), softmax in fp32 with the global max, probabilities
// rounded to bf16, P@V summed in fp32 and rounded to bf16.

// Scores of positions [c0, cend) into sc[h][p - c0]; running max in m.
// Each 16-lane row takes one position (16 lanes x 8 dims); a wave four.
__device__ __forceinline__ void score_chunk(const uint16_t* kc, const u32x4 (&qv)[2], float scale, int c0, int cend,
                                            float* sc0, float* sc1, float (&m)[2]) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, slot = lane >> 4, t16 = lane & 15;
  for (int p = c0 + wave * 4 + slot; p < cend; p += 16) {
    const u32x4 kx = ld16(kc + (size_t)p * kD + 8 * t16);
    const float s0 = bf16r(bf16r(row16_sum(dot8(kx, qv[0], 0.f))) * scale);
    const float s1 = bf16r(bf16r(row16_sum(dot8(kx, qv[1], 0.f))) * scale);
    if (t16 == 0) {
      sc0[p - c0] = s0;
      sc1[p - c0] = s1;
    }
    m[0] = fmaxf(m[0], s0);
    m[1] = fmaxf(m[1], s1);
  }
}

// Probability-weighted V rows [0, n) of the chunk, dims 2*lane..+1 of both
// heads, wave w taking rows w, w+4, ...
__device__ __forceinline__ void pv_chunk(const uint16_t* vc, const float* p0, const float* p1, int n,
                                         float (&acc)[2][2]) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
#pragma unroll 4
  for (int i = wave; i < n; i += 4) {
    const uint32_t v2 = ld32(vc + (size_t)i * kD + 2 * lane);
    const float va = lo_bf16(v2), vb = hi_bf16(v2);
    const float pa = p0[i], pb = p1[i];
    acc[0][0] += pa * va;
    acc[0][1] += pa * vb;
    acc[1][0] += pb * va;
    acc[1][1] += pb * vb;
  }
}

// Sum of the four waves' P@V partials (fixed order); thread (h = tid/128, d = tid%128).
__device__ __forceinline__ float pv_merge_waves(const float (&acc)[2][2], float (*pv)[2][kD]) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  __syncthreads();
#pragma unroll
  for (int h = 0; h < 2; h++) {
    pv[wave][h][2 * lane] = acc[h][0];
    pv[wave][h][2 * lane + 1] = acc[h][1];
  }
  __syncthreads();
  const int h = threadIdx.x >> 7, d = threadIdx.x & 127;
  return ((pv[0][h][d] + pv[1][h][d]) + pv[2][h][d]) + pv[3][h][d];
}

// attention_rows' work for token t and KV head g (both query heads)
__device__ __forceinline__ void attention_row(const uint16_t* __restrict__ Q, const Tok tk, int t, int g, int t16,
                                              int L, const Cache& c, float scale, uint16_t* __restrict__ out,
                                              float (*sc)[kAttnChunk], float (*red)[4], float (*pv)[2][kD]) {
  uint16_t* dst = out + (size_t)t * kQS + 2 * g * kD;  // both heads: 256 contiguous values
  if (!tk.valid) {
    dst[threadIdx.x] = 0;
    return;
  }
  const int C = tk.pos + 1;
  const size_t base = cache_base(c, tk, L, g);
  const uint16_t* kc = c.k + base;
  const uint16_t* vc = c.v + base;
  u32x4 qv[2];
#pragma unroll
  for (int h = 0; h < 2; h++) qv[h] = ld16(Q + (size_t)t * kQS + (2 * g + h) * kD + 8 * t16);
  const int nch = (C + kAttnChunk - 1) / kAttnChunk;
  float M[2] = {-INFINITY, -INFINITY};
  for (int ch = 0; ch < nch; ch++)
    score_chunk(kc, qv, scale, ch * kAttnChunk, min(C, (ch + 1) * kAttnChunk), sc[0], sc[1], M);
  block_max2(M, red);
  float S[2] = {0.f, 0.f};
  float dummy[2];
  for (int ch = 0; ch < nch; ch++) {
    const int c0 = ch * kAttnChunk, n = min(C - c0, kAttnChunk);
    if (nch > 1) {
      __syncthreads();
      score_chunk(kc, qv, scale, c0, c0 + n, sc[0], sc[1], dummy);
      __syncthreads();
    }
    for (int i = threadIdx.x; i < n; i += 256) {
      S[0] += exp_acc(sc[0][i] - M[0]);
      S[1] += exp_acc(sc[1][i] - M[1]);
    }
  }
  block_sum2(S, red);
  const float inv0 = __fdiv_rn(1.0f, S[0]), inv1 = __fdiv_rn(1.0f, S[1]);
  float acc[2][2] = {{0.f, 0.f}, {0.f, 0.f}};
  for (int ch = 0; ch < nch; ch++) {
    const int c0 = ch * kAttnChunk, n = min(C - c0, kAttnChunk);
    __syncthreads();
    if (nch > 1) {
      score_chunk(kc, qv, scale, c0, c0 + n, sc[0], sc[1], dummy);
      __syncthreads();
    }
    for (int i = threadIdx.x; i < n; i += 256) {
      sc[0][i] = bf16r(exp_acc(sc[0][i] - M[0]) * inv0);
      sc[1][i] = bf16r(exp_acc(sc[1][i] - M[1]) * inv1);
    }
    __syncthreads();
    pv_chunk(vc + (size_t)c0 * kD, sc[0], sc[1], n, acc);
  }
  dst[threadIdx.x] = (uint16_t)f32_to_bf16(pv_merge_waves(acc, pv));
}

// One workgroup per (token, KV head), for many tokens (token t = blockIdx.x,
// blockIdx.x + gridDim.x, ...; a grid narrower than T when attention_mfma ran,
// so that the workgroups of the tiles it covered cost little: at 2048 tokens
// a full grid of such exits took 4.9 us).  Contexts longer than kAttnChunk are
// processed in chunks, recomputing the scores in each of the three passes
// (max, sum, P@V) instead of keeping them.
__global__ void __launch_bounds__(256) attention_rows(const uint16_t* __restrict__ Q, const Tok* __restrict__ tok,
                                                      int T, int L, Cache c, float scale, uint16_t* __restrict__ out,
                                                      const int* __restrict__ redo) {
  __shared__ float sc[2][kAttnChunk];
  __shared__ float red[2][4];
  __shared__ float pv[4][2][kD];
  const int g = blockIdx.y, t16 = threadIdx.x & 15;
  for (int t = blockIdx.x; t < T; t += gridDim.x) {
    if (redo && redo[t / kQT] == 0) continue;  // attention_mfma covered this token's tile
    __syncthreads();  // the previous token's reads of the shared arrays are done
    attention_row(Q, tok[t], t, g, t16, L, c, scale, out, sc, red, pv);
  }
}

// Prompt prefill attention on MFMA.  Tiles of kQT consecutive tokens; one
// workgroup of 8 waves per (pair of tiles, query head h): tiles i and nt-1-i
// (the middle tile alone when nt is odd), one after the other, so that every
// workgroup's causal work is about the same (the last tile alone has twice
// the average).  For a tile whose tokens are one sequence at consecutive
// positions (every prompt prefill) the tile's 64 query rows share each block
// of kKB cached keys and values, staged through LDS.  Two passes over the keys,
// as HF's eager softmax: pass 1 gives each row's max M and sum L of exp(s - M)
// (online per lane over the blocks, then across lanes and the two waves of a
// row group); pass 2 recomputes the scores, rounds the probabilities
// bf16(exp(s - M) / L) and multiplies them with V on MFMA.  Scores are
// bf16(bf16(q.k) * scale), as in attention_rows.  A tile that is not one such
// run (several sequences, an invalid token) is marked in redo[tile] and left to
// attention_rows.
//
// MFMA 16x16x32 bf16 layout: lane l supplies A[l%16][8(l/16)..+7] and
// B[8(l/16)..+7][l%16] and receives C[4(l/16)+i][l%16].  Wave w owns query rows
// 16(w/2)..+15 of the tile and keys 32(w%2)..+31 of every block (two waves per
// row group, each with half of the keys).  Scores are computed transposed (A =
// 16 keys' K rows, B = the rows' q), so lane (l16, lg) holds row l16's scores of
// keys 16n + 4lg + i, i = 0..3: every lane carries one query row.  P@V takes A =
// those probabilities straight from the registers: the 8 k-slots 8lg..8lg+7 of
// a 32-key step are keys 4lg..4lg+3 and 16+4lg..16+4lg+3 of the wave's half
// block, and V is stored transposed in LDS in that slot order (B = V^T rows,
// 16 contiguous bytes per lane).  The two waves of a row group add their P@V
// partials through LDS at the end (in a fixed order).
constexpr int kAttnWaves = 8;

// LDS slot of key q (0..kKB-1) of a block in the transposed V: the order in
// which a wave's P@V k-slots take its keys (see above)
__device__ __forceinline__ int attn_v_slot(int q) {
  const int half = q >> 5, r = q & 31;
  return 32 * half + 8 * ((r & 15) >> 2) + 4 * (r >> 4) + (r & 3);
}

// Modes: kAttnFull (kernel attention_mfma) runs both passes over a tile's whole context (pairs of
// tiles per workgroup, as above).  For few tiles over a long context the keys are split into chunks
// of ck blocks, one workgroup per (tile, chunk, query head): kAttnPass1 (attention_mfma_pass1)
// writes each row's (max, sum) of its chunk to ml; kAttnPass2 (attention_mfma_pass2) takes every
// chunk's (max, sum) of its rows (in chunk order) for the global max M and sum L, and writes its
// chunk's P@V partial (fp32) to part; attention_mfma_merge adds the partials in chunk order.
// Workgroups of chunks past a tile's last key do nothing.
enum AttnMode : int { kAttnFull = 0, kAttnPass1 = 1, kAttnPass2 = 2 };

// Index of (tile, head, chunk)'s row block in the split passes' ml and part buffers
__device__ __forceinline__ size_t attn_chunk_row(int tile, int h, int nch, int chunk, int row) {
  return (((size_t)tile * kNQ + h) * nch + chunk) * kQT + row;
}

template <int MODE>
__device__ __forceinline__ void attention_mfma_body(const uint16_t* __restrict__ Q, const Tok* __restrict__ tok, int T,
                                                    int L, Cache c, float scale, uint16_t* __restrict__ out,
                                                    int* __restrict__ redo, int nch, int ck, float2* __restrict__ ml,
                                                    float* __restrict__ part) {
  constexpr int NT = kAttnWaves * 64;
  static_assert(kQT == 64 && kKB == 64 && kAttnWaves == 8, "4 row groups of 16 x 2 key halves of 32");
  // K block [kKB][kKPad] and transposed V [kD][kVPad]; after the passes the same bytes hold the
  // odd waves' P@V partials [4 row groups][16 rows][kD] fp32 for the even waves to add
  constexpr int kKBytes = kKB * kKPad * 2, kVBytes = kD * kVPad * 2, kRedBytes = 4 * 16 * kD * 4;
  static_assert(kKBytes + kVBytes >= kRedBytes, "the partials fit in the K/V buffers");
  __shared__ __align__(16) unsigned char smem[kKBytes + kVBytes];
  __shared__ int s_ok[2];
  auto Ks = reinterpret_cast<uint16_t(*)[kKPad]>(smem);
  auto Vt = reinterpret_cast<uint16_t(*)[kVPad]>(smem + kKBytes);
  auto Vw = reinterpret_cast<uint32_t(*)[kVPad / 2]>(smem + kKBytes);  // the same rows as 32-bit words
  auto red = reinterpret_cast<float(*)[16][kD]>(smem);
  __shared__ float s_ml[4][2][16][2];  // (max, sum) per row group, key half and row
  const int nt = (T + kQT - 1) / kQT;
  const int h = blockIdx.y, g = h >> 1;
  // the wave index made uniform, so that branches on the wave's rows and keys are scalar
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63, l16 = lane & 15,
            lg = lane >> 4;
  const int rg = w >> 1, kh = w & 1;  // rows 16rg..16rg+15, keys 32kh..32kh+31 of each block
  // kAttnFull: the pair (i, nt - 1 - i); the split passes: tile blockIdx.x / nch, chunk blockIdx.x % nch
  const int tiles[2] = {MODE == kAttnFull ? (int)blockIdx.x : (int)blockIdx.x / nch,
                        MODE == kAttnFull ? nt - 1 - (int)blockIdx.x : (int)blockIdx.x / nch};
  const int chunk = MODE == kAttnFull ? 0 : (int)blockIdx.x % nch;
  const int ntile = tiles[1] == tiles[0] ? 1 : 2;
  // which of the pair's tiles are one sequence at consecutive positions
  if (threadIdx.x < 2) s_ok[threadIdx.x] = 1;
  __syncthreads();
  for (int u = 0; u < ntile; u++) {
    const int t0 = tiles[u] * kQT, nrows = min(kQT, T - t0);
    if ((int)threadIdx.x < nrows) {
      const Tok first = tok[t0], tk = tok[t0 + threadIdx.x];
      if (!tk.valid || tk.seq != first.seq || tk.pos != first.pos + (int)threadIdx.x) s_ok[u] = 0;
    }
  }
  __syncthreads();
  if (MODE != kAttnPass2 && h == 0 && chunk == 0 && threadIdx.x < (unsigned)ntile)
    redo[tiles[threadIdx.x]] = s_ok[threadIdx.x] ? 0 : 1;

  for (int u = 0; u < ntile; u++) {
    if (!s_ok[u]) continue;  // uniform over the workgroup
    const int t0 = tiles[u] * kQT, nrows = min(kQT, T - t0);
    const Tok first = tok[t0];
    const int pos0 = __builtin_amdgcn_readfirstlane(first.pos), pmax = pos0 + nrows - 1;
    const size_t base = cache_base(c, first, L, g);
    const uint16_t* kc = c.k + base;
    const uint16_t* vc = c.v + base;
    // B operands: this lane's query row (rows past the tile's tokens repeat its last one)
    const int tq = t0 + min(16 * rg + l16, nrows - 1);
    bf16x8 qb[4];
#pragma unroll
    for (int kk = 0; kk < 4; kk++) qb[kk] = ld_bf16x8(Q + (size_t)tq * kQS + h * kD + 32 * kk + 8 * lg);
    const int rpos = pos0 + 16 * rg + l16;      // this lane's row position
    const int wave_first = pos0 + 16 * rg;      // the wave's smallest row position
    const int wave_last = pos0 + 16 * rg + 15;  // the wave's largest row position
    const int nkb = (pmax + kKB) / kKB;         // blocks covering positions 0..pmax
    // this workgroup's blocks: all of them, or its chunk's (none past the tile's last key)
    const int kb0 = MODE == kAttnFull ? 0 : chunk * ck, kb1 = MODE == kAttnFull ? nkb : min(kb0 + ck, nkb);
    if (kb0 >= kb1) continue;  // uniform over the workgroup
    // Block kb: positions kb*kKB + pr; rows past pmax load row pmax (masked below).  Each
    // thread carries kCh 16-byte chunks of K (and of V): block kb+1 is requested into registers
    // before block kb's MFMAs, so its memory latency overlaps them, and written to LDS after
    // the next barrier.
    constexpr int kCh = kKB * (kD / 8) / NT;
    // two register sets: block kb + 2 is requested right after block kb is written to LDS, so a
    // request has two blocks of compute to land
    u32x4 rk[2][kCh], rv[2][kCh];
    auto load_k = [&](int set, int kb) {
#pragma unroll
      for (int j = 0; j < kCh; j++) {
        const int ci = threadIdx.x + NT * j, pr = ci >> 4, col = (ci & 15) * 8;
        rk[set][j] = ld16(kc + (size_t)min(kb * kKB + pr, pmax) * kD + col);
      }
    };
    // V: this thread carries keys 2va and 2va+1 of the block, dims 8vc..8vc+7 (a wave's lanes
    // cover four dim chunks of 16 key pairs), so each transposed LDS word takes both keys' values
    static_assert(kCh == 2, "one key pair per thread");
    const int va = (lane >> 2) + 16 * (w & 1), vcol = 8 * ((lane & 3) + 4 * (w >> 1));
    auto load_v = [&](int set, int kb) {
#pragma unroll
      for (int j = 0; j < 2; j++) rv[set][j] = ld16(vc + (size_t)min(kb * kKB + 2 * va + j, pmax) * kD + vcol);
    };
    auto put_k = [&](int set) {
#pragma unroll
      for (int j = 0; j < kCh; j++) {
        const int ci = threadIdx.x + NT * j, pr = ci >> 4, col = (ci & 15) * 8;
        *reinterpret_cast<u32x4*>(&Ks[pr][col]) = rk[set][j];
      }
    };
    auto put_v = [&](int set) {  // transposed, keys in P@V slot order: Vt[dim][slot]; keys 2va, 2va+1
                                 // take adjacent slots, so each dim is one 32-bit word
      const int sw = attn_v_slot(2 * va) >> 1;
      const u32x4 a0 = rv[set][0], a1 = rv[set][1];
      const uint32_t k0[4] = {a0.x, a0.y, a0.z, a0.w}, k1[4] = {a1.x, a1.y, a1.z, a1.w};
#pragma unroll
      for (int e = 0; e < 4; e++) {
        Vw[vcol + 2 * e][sw] = (k0[e] & 0xffffu) | (k1[e] << 16);
        Vw[vcol + 2 * e + 1][sw] = (k0[e] >> 16) | (k1[e] & 0xffff0000u);
      }
    };
    // raw q.k of row l16 with keys kb*kKB + 32kh + 16n + 4lg + i
    auto tile_scores = [&](int n) {
      f32x4 sc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kk = 0; kk < 4; kk++)
        sc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
            *reinterpret_cast<const bf16x8*>(&Ks[32 * kh + 16 * n + l16][32 * kk + 8 * lg]), qb[kk], sc, 0, 0, 0);
      return sc;
    };
    // the four scores bf16(bf16(q.k) * scale), two roundings per conversion; no branch per
    // element (the callers mask by select), so the four chains interleave
    auto scaled = [&](const f32x4& sc, float (&x)[4]) {
      const uint32_t r01 = pack_bf16x2(sc[0], sc[1]), r23 = pack_bf16x2(sc[2], sc[3]);
      const uint32_t s01 = pack_bf16x2(lo_bf16(r01) * scale, hi_bf16(r01) * scale);
      const uint32_t s23 = pack_bf16x2(lo_bf16(r23) * scale, hi_bf16(r23) * scale);
      x[0] = lo_bf16(s01);
      x[1] = hi_bf16(s01);
      x[2] = lo_bf16(s23);
      x[3] = hi_bf16(s23);
    };
    // ---- pass 1: per lane, online max and sum of exp over its positions (one exp per score,
    // one rescale per block)
    float m = -INFINITY, ls = 0.f;
    auto pass1 = [&](int kb) {
      const int kbase = kb * kKB + 32 * kh;
      if (kbase > wave_last) return;  // every key of the wave's half block follows its rows
      // MASKED: the half block reaches the causal diagonal of the wave's rows (the last one or two
      // blocks of a tile); every earlier key precedes every row, so neither the mask nor the
      // clamp of exp_acc is needed (exp_finite gives the same values for finite arguments)
      auto block = [&](auto masked) {
        constexpr bool MASKED = decltype(masked)::value;
        float x[2][4];
        float mb = -INFINITY;
#pragma unroll
        for (int n = 0; n < 2; n++) {
          const f32x4 sc = !MASKED || kbase + 16 * n <= wave_last ? tile_scores(n) : f32x4{0.f, 0.f, 0.f, 0.f};
          scaled(sc, x[n]);
#pragma unroll
          for (int i = 0; i < 4; i++) {
            if constexpr (MASKED) x[n][i] = kbase + 16 * n + 4 * lg + i <= rpos ? x[n][i] : -INFINITY;
            mb = fmaxf(mb, x[n][i]);
          }
        }
        // no branch: while every key so far is masked for this lane's row (mn = -inf) the terms
        // are taken against 0, and exp_acc turns -inf into 0, so ls stays 0
        const float mn = fmaxf(m, mb);
        const float ref = MASKED && mn == -INFINITY ? 0.f : mn;
        float e = 0.f;
#pragma unroll
        for (int n = 0; n < 2; n++)
#pragma unroll
          for (int i = 0; i < 4; i++) e += MASKED ? exp_acc(x[n][i] - ref) : exp_finite(x[n][i] - ref);
        ls = ls * exp_acc(m - ref) + e;
        m = mn;
      };
      if (kbase + 31 <= wave_first) block(std::false_type{});
      else block(std::true_type{});
    };
    float gm, ginv;
    if constexpr (MODE != kAttnPass2) {
      // blocks past the last one are requested too (clamped rows, never used), so that every path
      // issues the same loads and the compiler's counted waits stay exact
      load_k(0, kb0);
      load_k(1, kb0 + 1);
      for (int kb = kb0; kb < kb1; kb += 2) {
        __syncthreads();  // the previous block's reads are done
        put_k(0);
        __syncthreads();
        load_k(0, kb + 2);
        pass1(kb);
        if (kb + 1 >= kb1) break;
        __syncthreads();
        put_k(1);
        __syncthreads();
        load_k(1, kb + 3);
        pass1(kb + 1);
      }
      // row l16's (max, sum): over the 4 lanes of equal l16, then the row group's two waves (the
      // even wave's pair first in every wave, so both waves hold the same M and 1/L)
      {
        float mx = m;
        mx = fmaxf(mx, __shfl_xor(mx, 16));
        mx = fmaxf(mx, __shfl_xor(mx, 32));
        float sm = m == -INFINITY ? 0.f : ls * exp_acc(m - mx);
        sm += __shfl_xor(sm, 16);
        sm += __shfl_xor(sm, 32);
        if (lg == 0) {
          s_ml[rg][kh][l16][0] = mx;
          s_ml[rg][kh][l16][1] = sm;
        }
      }
      __syncthreads();
      const float m0 = s_ml[rg][0][l16][0], l0 = s_ml[rg][0][l16][1];
      const float m1 = s_ml[rg][1][l16][0], l1 = s_ml[rg][1][l16][1];
      gm = fmaxf(m0, m1);
      const float sm = (m0 == -INFINITY ? 0.f : l0 * exp_acc(m0 - gm)) + (m1 == -INFINITY ? 0.f : l1 * exp_acc(m1 - gm));
      if constexpr (MODE == kAttnPass1) {
        // the chunk's (max, sum) of row 16rg + l16 (-inf, 0 when every key of the chunk follows it)
        if (kh == 0 && lg == 0) ml[attn_chunk_row(tiles[u], h, nch, chunk, 16 * rg + l16)] = make_float2(gm, sm);
        continue;
      }
      ginv = __fdiv_rn(1.0f, sm);
    } else {
      // the row's global (max, sum) from its chunks' (chunk 0 holds key 0, so the sum is > 0), the
      // sum in chunk order.  Every chunk's pairs of the tile's rows go to LDS first (over the K/V
      // buffers, unused until the barrier that opens pass 2's first block), in one round of loads.
      const int nc = (nkb + ck - 1) / ck, row = 16 * rg + l16;
      float2* const s_cml = reinterpret_cast<float2*>(smem);  // [nc][kQT]
      static_assert(kMaxAttnChunks * kQT * sizeof(float2) <= kKBytes + kVBytes, "the chunks' pairs fit in LDS");
      for (int i = threadIdx.x; i < nc * kQT; i += NT) s_cml[i] = ml[attn_chunk_row(tiles[u], h, nch, i / kQT, i % kQT)];
      __syncthreads();
      float mx = -INFINITY;
      for (int q = 0; q < nc; q++) mx = fmaxf(mx, s_cml[q * kQT + row].x);
      float sm = 0.f;
      for (int q = 0; q < nc; q++) {
        const float2 e = s_cml[q * kQT + row];
        sm += e.x == -INFINITY ? 0.f : e.y * exp_acc(e.x - mx);
      }
      gm = mx;
      ginv = __fdiv_rn(1.0f, sm);
    }
    // ---- pass 2: probabilities (bf16, as HF rounds them) times V
    f32x4 acc[8];
#pragma unroll
    for (int j = 0; j < 8; j++) acc[j] = f32x4{0.f, 0.f, 0.f, 0.f};
    auto pass2 = [&](int kb) {
      const int kbase = kb * kKB + 32 * kh;
      if (kbase > wave_last) return;
      // A operand: k-slot 4n + i of this lane is key kbase + 16n + 4lg + i of row l16
      uint32_t pw[4];
      auto probs = [&](auto masked) {  // MASKED as in pass 1
        constexpr bool MASKED = decltype(masked)::value;
#pragma unroll
        for (int n = 0; n < 2; n++) {
          // a 16-key tile wholly past the wave's rows is masked for every row: no MFMA for it
          const f32x4 sc = !MASKED || kbase + 16 * n <= wave_last ? tile_scores(n) : f32x4{0.f, 0.f, 0.f, 0.f};
          float x[4], pr[4];
          scaled(sc, x);
#pragma unroll
          for (int i = 0; i < 4; i++) {
            // the probability bf16(exp(s - M) / L) (rounded once, by the packing below); masked
            // keys, whose terms may be anything, take 0
            if constexpr (MASKED) pr[i] = kbase + 16 * n + 4 * lg + i <= rpos ? exp_acc(x[i] - gm) * ginv : 0.f;
            else pr[i] = exp_finite(x[i] - gm) * ginv;
          }
          pw[2 * n] = pack_bf16x2(pr[0], pr[1]);
          pw[2 * n + 1] = pack_bf16x2(pr[2], pr[3]);
        }
      };
      if (kbase + 31 <= wave_first) probs(std::false_type{});
      else probs(std::true_type{});
      const bf16x8 pa = __builtin_bit_cast(bf16x8, u32x4{pw[0], pw[1], pw[2], pw[3]});
#pragma unroll
      for (int j = 0; j < 8; j++)
        acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
            pa, *reinterpret_cast<const bf16x8*>(&Vt[16 * j + l16][32 * kh + 8 * lg]), acc[j], 0, 0, 0);
    };
    load_k(0, kb0);
    load_v(0, kb0);
    load_k(1, kb0 + 1);
    load_v(1, kb0 + 1);
    for (int kb = kb0; kb < kb1; kb += 2) {
      __syncthreads();
      put_k(0);
      put_v(0);
      __syncthreads();
      load_k(0, kb + 2);
      load_v(0, kb + 2);
      pass2(kb);
      if (kb + 1 >= kb1) break;
      __syncthreads();
      put_k(1);
      put_v(1);
      __syncthreads();
      load_k(1, kb + 3);
      load_v(1, kb + 3);
      pass2(kb + 1);
    }
    // the row group's two partials: the odd wave's through LDS (over the K/V buffers), added to
    // the even wave's
    __syncthreads();
    if (kh == 1) {
#pragma unroll
      for (int j = 0; j < 8; j++)
#pragma unroll
        for (int i = 0; i < 4; i++) red[rg][4 * lg + i][16 * j + l16] = acc[j][i];
    }
    __syncthreads();
    if (kh == 0) {
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int r = 16 * rg + 4 * lg + i;
        if (r < nrows) {
          if constexpr (MODE == kAttnFull) {
            uint16_t* dst = out + (size_t)(t0 + r) * kQS + h * kD;
#pragma unroll
            for (int j = 0; j < 8; j++)
              dst[16 * j + l16] = (uint16_t)f32_to_bf16(acc[j][i] + red[rg][4 * lg + i][16 * j + l16]);
          } else {  // this chunk's fp32 partial of the row
            float* dst = part + attn_chunk_row(tiles[u], h, nch, chunk, r) * kD;
#pragma unroll
            for (int j = 0; j < 8; j++) dst[16 * j + l16] = acc[j][i] + red[rg][4 * lg + i][16 * j + l16];
          }
        }
      }
    }
  }
}

#define QMK_ATTN_ARGS                                                                                      \
  const uint16_t *__restrict__ Q, const Tok *__restrict__ tok, int T, int L, Cache c, float scale,                 \
      uint16_t *__restrict__ out, int *__restrict__ redo, int nch, int ck, float2 *__restrict__ ml,                 \
      float *__restrict__ part
// The pairs, the first pass over key chunks and the second.  (Held to 128 registers, for two
// workgroups of the second pass per CU, it spilled 18 and ran slower: 32 tokens after 7,000
// positions 2.57-2.63 against 2.39-2.44 ms per prefill.)
__global__ void __launch_bounds__(kAttnWaves * 64) attention_mfma(QMK_ATTN_ARGS) {
  attention_mfma_body<kAttnFull>(Q, tok, T, L, c, scale, out, redo, nch, ck, ml, part);
}
__global__ void __launch_bounds__(kAttnWaves * 64) attention_mfma_pass1(QMK_ATTN_ARGS) {
  attention_mfma_body<kAttnPass1>(Q, tok, T, L, c, scale, out, redo, nch, ck, ml, part);
}
__global__ void __launch_bounds__(kAttnWaves * 64) attention_mfma_pass2(QMK_ATTN_ARGS) {
  attention_mfma_body<kAttnPass2>(Q, tok, T, L, c, scale, out, redo, nch, ck, ml, part);
}
#undef QMK_ATTN_ARGS

// The split passes' output: each row of a tile attention_mfma covered (redo 0) is the sum of its
// chunks' partials in chunk order, rounded to bf16.  One workgroup of kD threads per (token, query
// head).
__global__ void __launch_bounds__(kD) attention_mfma_merge(const Tok* __restrict__ tok, int T, int nch, int ck,
                                                          const float* __restrict__ part,
                                                          const int* __restrict__ redo, uint16_t* __restrict__ out) {
  const int t = blockIdx.x, h = blockIdx.y, d = threadIdx.x;
  const int tile = t / kQT, t0 = tile * kQT, nrows = min(kQT, T - t0);
  if (redo[tile]) return;
  const int pmax = tok[t0].pos + nrows - 1;
  const int nc = ((pmax + kKB) / kKB + ck - 1) / ck;
  // eight chunks' loads in flight at a time, added in chunk order
  float y = 0.f;
  for (int q0 = 0; q0 < nc; q0 += 8) {
    float v[8];
#pragma unroll
    for (int j = 0; j < 8; j++) v[j] = q0 + j < nc ? part[attn_chunk_row(tile, h, nch, q0 + j, t - t0) * kD + d] : 0.f;
#pragma unroll
    for (int j = 0; j < 8; j++)
      if (q0 + j < nc) y += v[j];
  }
  out[(size_t)t * kQS + h * kD + d] = (uint16_t)f32_to_bf16(y);
}

// Few tokens: the context of each (token, KV head) is split over workgroups of
// kSplitChunk positions.  attn_split_scores writes the chunk's scores and its
// (max m_j, sum l_j of exp(s - m_j)) per head; attn_split_pv takes the global
// max M and the sum S = sum_j l_j * exp(m_j - M) (fixed order, identical in
// every workgroup of the token), forms the probabilities and a partial P@V;
// attn_split_merge adds the partials in chunk order.
__global__ void __launch_bounds__(256) attn_split_scores(const uint16_t* __restrict__ Q, const Tok* __restrict__ tok,
                                                         int L, Cache c, float scale, int nch,
                                                         float* __restrict__ scores, float2* __restrict__ ml) {
  __shared__ float sc[2][kSplitChunk];
  __shared__ float red[2][4];
  const int t = blockIdx.x, g = blockIdx.y, j = blockIdx.z, t16 = threadIdx.x & 15;
  const Tok tk = tok[t];
  const int C = tk.valid ? tk.pos + 1 : 0;
  const int c0 = j * kSplitChunk;
  if (c0 >= C) return;
  const int n = min(C - c0, kSplitChunk);
  const size_t base = cache_base(c, tk, L, g);
  u32x4 qv[2];
#pragma unroll
  for (int h = 0; h < 2; h++) qv[h] = ld16(Q + (size_t)t * kQS + (2 * g + h) * kD + 8 * t16);
  float m[2] = {-INFINITY, -INFINITY};
  score_chunk(c.k + base, qv, scale, c0, c0 + n, sc[0], sc[1], m);
  block_max2(m, red);
  float l[2] = {0.f, 0.f};
  const size_t ncap = (size_t)nch * kSplitChunk;
  for (int i = threadIdx.x; i < n; i += 256) {
#pragma unroll
    for (int h = 0; h < 2; h++) {
      const float s = sc[h][i];
      scores[((size_t)t * kNQ + 2 * g + h) * ncap + c0 + i] = s;
      l[h] += exp_acc(s - m[h]);
    }
  }
  block_sum2(l, red);
  if (threadIdx.x < 2)
    ml[((size_t)t * kNQ + 2 * g + threadIdx.x) * nch + j] = make_float2(m[threadIdx.x], l[threadIdx.x]);
}

__global__ void __launch_bounds__(256) attn_split_pv(const Tok* __restrict__ tok, int L, Cache c, int nch,
                                                     const float* __restrict__ scores, const float2* __restrict__ ml,
                                                     float* __restrict__ pvp) {
  __shared__ float pr[2][kSplitChunk];
  __shared__ float pv[4][2][kD];
  const int t = blockIdx.x, g = blockIdx.y, j = blockIdx.z;
  const Tok tk = tok[t];
  const int C = tk.valid ? tk.pos + 1 : 0;
  const int c0 = j * kSplitChunk;
  if (c0 >= C) return;
  const int n = min(C - c0, kSplitChunk), used = (C + kSplitChunk - 1) / kSplitChunk;
  const size_t ncap = (size_t)nch * kSplitChunk;
  float M[2], inv[2];
#pragma unroll
  for (int h = 0; h < 2; h++) {
    const float2* mlh = ml + ((size_t)t * kNQ + 2 * g + h) * nch;
    float mx = -INFINITY;
    for (int q = 0; q < used; q++) mx = fmaxf(mx, mlh[q].x);
    float s = 0.f;
    for (int q = 0; q < used; q++) s += mlh[q].y * exp_acc(mlh[q].x - mx);
    M[h] = mx;
    inv[h] = __fdiv_rn(1.0f, s);
  }
  for (int i = threadIdx.x; i < n; i += 256) {
#pragma unroll
    for (int h = 0; h < 2; h++)
      pr[h][i] = bf16r(exp_acc(scores[((size_t)t * kNQ + 2 * g + h) * ncap + c0 + i] - M[h]) * inv[h]);
  }
  __syncthreads();
  float acc[2][2] = {{0.f, 0.f}, {0.f, 0.f}};
  pv_chunk(c.v + cache_base(c, tk, L, g) + (size_t)c0 * kD, pr[0], pr[1], n, acc);
  const float y = pv_merge_waves(acc, pv);
  pvp[(((size_t)t * nch + j) * kNQ + 2 * g) * kD + threadIdx.x] = y;
}

// out[t][i] = bf16(sum over the token's chunks of the partial P@V), i over
// the 16 x 128 head outputs; grid (token, 8 slices of 256).
__global__ void __launch_bounds__(256) attn_split_merge(const Tok* __restrict__ tok, int nch,
                                                        const float* __restrict__ pvp, uint16_t* __restrict__ out) {
  const int t = blockIdx.x, i = blockIdx.y * 256 + threadIdx.x;
  const Tok tk = tok[t];
  const int C = tk.valid ? tk.pos + 1 : 0;
  const int used = (C + kSplitChunk - 1) / kSplitChunk;
  const float* src = pvp + (size_t)t * nch * kQS + i;
  float y = 0.f;
#pragma unroll 8
  for (int q = 0; q < used; q++) y += src[(size_t)q * kQS];
  out[(size_t)t * kQS + i] = (uint16_t)f32_to_bf16(y);
}

// ---------------------------------------------------------------- LM head
//
// The LM head runs as lm_head_gemm (the GEMM above over the full K, one wave
// per 16-row x 64-column tile) whose epilogue rounds each logit to bf16,
// optionally writes its fp32 copy, and keeps, per row and tile, the largest
// key (orderable bf16 logit << 32 | ~index): the first index of the maximum,
// HF's greedy argmax.  keys_reduce then takes each row's largest key over the
// tiles; no atomics, so the result is independent of scheduling.

__device__ __forceinline__ unsigned long long key_max(unsigned long long a, unsigned long long b) { return a > b ? a : b; }

__global__ void __launch_bounds__(256) lm_head_gemm(const uint16_t* __restrict__ X, const int* __restrict__ rows,
                                                    int R, const uint16_t* __restrict__ W, int K, int V,
                                                    unsigned long long* __restrict__ keys_part,
                                                    float* __restrict__ logits) {
  constexpr int NB = 4;
  const int nblk = gridDim.x;
  const int b = blockIdx.x;
  const int lb = (nblk % kGroups == 0) ? (b % kGroups) * (nblk / kGroups) + b / kGroups : b;
  const int wave = lb * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int mtiles = (R + 15) / 16, ntiles = V / (16 * NB);
  const int mt = wave % mtiles, nt = wave / mtiles;
  if (nt >= ntiles) return;
  const int kq = 8 * (lane >> 4);
  const int xr = max(rows[min(mt * 16 + (lane & 15), R - 1)], 0);
  const uint16_t* xa = X + (size_t)xr * K + kq;
  const uint16_t* wb[NB];
#pragma unroll
  for (int j = 0; j < NB; j++) wb[j] = W + (size_t)(nt * 16 * NB + 16 * j + (lane & 15)) * K + kq;
  f32x4 acc[NB];
#pragma unroll
  for (int j = 0; j < NB; j++) acc[j] = f32x4{0.f, 0.f, 0.f, 0.f};
  bf16x8 a0 = ld_bf16x8(xa), a1 = ld_bf16x8(xa + 32), b0[NB], b1[NB];
#pragma unroll
  for (int j = 0; j < NB; j++) {
    b0[j] = ld_bf16x8_stream(wb[j]);
    b1[j] = ld_bf16x8_stream(wb[j] + 32);
  }
  for (int k = 0; k < K; k += 64) {
    bf16x8 na0, na1, nb0[NB], nb1[NB];
    const bool more = k + 64 < K;
    if (more) {
      na0 = ld_bf16x8(xa + k + 64);
      na1 = ld_bf16x8(xa + k + 96);
#pragma unroll
      for (int j = 0; j < NB; j++) {
        nb0[j] = ld_bf16x8_stream(wb[j] + k + 64);
        nb1[j] = ld_bf16x8_stream(wb[j] + k + 96);
      }
    }
#pragma unroll
    for (int j = 0; j < NB; j++) {
      acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a0, b0[j], acc[j], 0, 0, 0);
      acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1, b1[j], acc[j], 0, 0, 0);
    }
    if (more) {
      a0 = na0;
      a1 = na1;
#pragma unroll
      for (int j = 0; j < NB; j++) {
        b0[j] = nb0[j];
        b1[j] = nb1[j];
      }
    }
  }
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const int t = mt * 16 + 4 * (lane >> 4) + i;
    unsigned long long best = 0;
#pragma unroll
    for (int j = 0; j < NB; j++) {
      const int n = nt * 16 * NB + 16 * j + (lane & 15);
      const uint32_t hb = f32_to_bf16(acc[j][i]);
      if (logits && t < R) logits[(size_t)t * V + n] = bf16_to_f32(hb);
      best = key_max(best, ((unsigned long long)orderable16(hb) << 32) | (unsigned long long)(0xffffffffu - (uint32_t)n));
    }
    // max over the 16 lanes that hold row t
#pragma unroll
    for (int o = 1; o < 16; o <<= 1) best = key_max(best, __shfl_xor(best, o));
    if ((lane & 15) == 0 && t < R) keys_part[(size_t)t * ntiles + nt] = best;
  }
}

// LM head for at most 16 emitted rows, streamed by a persistent grid: 256
// workgroups of 8 waves; wave g takes the 16-column vocabulary tiles g, g+2048,
// ... (4 or 5 each, so every CU streams within 8% of the mean), walking them as
// one sequence of 64-K steps with kLmDepth steps of weights in flight across
// tile boundaries.  The emitted rows sit in LDS.  Each wave keeps its best key
// per row; keys_reduce takes the best over the 2048 waves.
constexpr int kLmWaves = 8, kLmBlocks = 256, kLmDepth = 4;

__global__ void __launch_bounds__(kLmWaves * 64) lm_head_stream(const uint16_t* __restrict__ X,
                                                                const int* __restrict__ rows, int R,
                                                                const uint16_t* __restrict__ W, int K, int V,
                                                                unsigned long long* __restrict__ keys_part,
                                                                float* __restrict__ logits) {
  extern __shared__ __align__(16) uint16_t xl[];  // [R][K]
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  for (int i = threadIdx.x; i < R * K / 8; i += kLmWaves * 64) {
    const int r = (i * 8) / K, k = (i * 8) % K;
    *reinterpret_cast<u32x4*>(xl + r * K + k) = ld16(X + (size_t)max(rows[r], 0) * K + k);
  }
  const int nw = gridDim.x * kLmWaves, gw = blockIdx.x * kLmWaves + wave;
  const int ntiles = V / 16, KS = K / 64;
  const int mine = gw < ntiles ? (ntiles - gw + nw - 1) / nw : 0;
  const int nsteps = mine * KS;
  const int kq = 8 * (lane >> 4);
  const int row = min(lane & 15, R - 1);
  auto wptr = [&](int step) {
    return W + (size_t)((gw + (step / KS) * nw) * 16 + (lane & 15)) * K + kq + (step % KS) * 64;
  };
  bf16x8 buf[kLmDepth][2];
#pragma unroll
  for (int u = 0; u < kLmDepth; u++)
    if (u < nsteps) {
      buf[u][0] = ld_bf16x8_stream(wptr(u));
      buf[u][1] = ld_bf16x8_stream(wptr(u) + 32);
    }
  __syncthreads();
  unsigned long long best[4] = {0, 0, 0, 0};
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  for (int s0 = 0; s0 < nsteps; s0 += kLmDepth) {
#pragma unroll
    for (int u = 0; u < kLmDepth; u++) {
      const int step = s0 + u;
      if (step < nsteps) {
        const int k = (step % KS) * 64;
        const bf16x8 a0 = *reinterpret_cast<const bf16x8*>(xl + row * K + kq + k);
        const bf16x8 a1 = *reinterpret_cast<const bf16x8*>(xl + row * K + kq + k + 32);
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a0, buf[u][0], acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1, buf[u][1], acc, 0, 0, 0);
        if (step + kLmDepth < nsteps) {
          buf[u][0] = ld_bf16x8_stream(wptr(step + kLmDepth));
          buf[u][1] = ld_bf16x8_stream(wptr(step + kLmDepth) + 32);
        }
        if (step % KS == KS - 1) {  // the tile is complete
          const int n = (gw + (step / KS) * nw) * 16 + (lane & 15);
#pragma unroll
          for (int i = 0; i < 4; i++) {
            const int t = 4 * (lane >> 4) + i;
            const uint32_t hb = f32_to_bf16(acc[i]);
            if (logits && t < R) logits[(size_t)t * V + n] = bf16_to_f32(hb);
            best[i] = key_max(best[i], ((unsigned long long)orderable16(hb) << 32) |
                                           (unsigned long long)(0xffffffffu - (uint32_t)n));
          }
          acc = f32x4{0.f, 0.f, 0.f, 0.f};
        }
      }
    }
  }
#pragma unroll
  for (int i = 0; i < 4; i++) {
    unsigned long long b = best[i];
#pragma unroll
    for (int o = 1; o < 16; o <<= 1) b = key_max(b, __shfl_xor(b, o));
    const int t = 4 * (lane >> 4) + i;
    if ((lane & 15) == 0 && t < R) keys_part[(size_t)t * nw + gw] = b;
  }
}

// out[r] = token of row r's largest key over the LM head's tiles (-1 for an
// invalid emit row or token).  One workgroup per row.
__global__ void __launch_bounds__(256) keys_reduce(const unsigned long long* __restrict__ keys_part, int ntiles,
                                                   const int* __restrict__ erow, const Tok* __restrict__ tok,
                                                   int* __restrict__ out) {
  __shared__ unsigned long long red[4];
  const int r = blockIdx.x, wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  unsigned long long best = 0;
  for (int i = threadIdx.x; i < ntiles; i += 256) best = key_max(best, keys_part[(size_t)r * ntiles + i]);
  best = wave_max_u64(best);
  if (lane == 0) red[wave] = best;
  __syncthreads();
  if (threadIdx.x == 0) {
    best = key_max(key_max(red[0], red[1]), key_max(red[2], red[3]));
    const int e = erow[r];
    out[r] = (e >= 0 && tok[e].valid) ? (int)(0xffffffffu - (uint32_t)best) : -1;
  }
}

// LM head for at most 4 emitted rows with each vocabulary row read whole: one wave instruction
// loads 1 KB of one row (lm_head_stream's MFMA operands take 64 bytes of each of 16 rows per
// instruction, which streams the head at about 5.3 TB/s against about 7 for whole rows).  The same
// persistent grid: wave gw takes vocabulary rows gw, gw + 2048, ..., four rows of weights in
// flight; each lane holds the emitted rows' matching 16-byte chunks in registers and adds its share
// of every dot product with v_dot2; wave_sum8 then finishes eight (vocabulary row, emitted row)
// sums at once, and the lanes that receive them round the logits and keep the best keys.  Keys
// per (emitted row, wave) as lm_head_stream's, for keys_reduce.
template <int R, int K>
__global__ void __launch_bounds__(kLmWaves * 64) lm_head_rows(const uint16_t* __restrict__ X,
                                                              const int* __restrict__ rows, int nrow,
                                                              const uint16_t* __restrict__ W, int V,
                                                              unsigned long long* __restrict__ keys_part,
                                                              float* __restrict__ logits) {
  static_assert(R >= 1 && R <= 4 && K % 512 == 0, "up to four rows, whole 512-element segments");
  constexpr int NS = K / 512;        // 16-byte chunks per lane of one vocabulary row
  constexpr int G = R == 3 ? 2 : 8 / R;  // vocabulary rows per eight-sum reduction
  constexpr int D = 4;               // vocabulary rows in flight (eight: 52.0 against 49.6 us, one 1024-wide row)
  const int lane = threadIdx.x & 63;
  const int nw = gridDim.x * kLmWaves, gw = blockIdx.x * kLmWaves + (threadIdx.x >> 6);
  const int mine = gw < V ? (V - gw + nw - 1) / nw : 0;  // this wave's vocabulary rows
  // the emitted rows' chunks (row r: elements 512 s + 8 lane .. +7 of segment s); rows past nrow
  // repeat the last one and are never written
  u32x4 x[R][NS];
#pragma unroll
  for (int r = 0; r < R; r++) {
    const uint16_t* xr = X + (size_t)max(rows[min(r, nrow - 1)], 0) * K;
#pragma unroll
    for (int sg = 0; sg < NS; sg++) x[r][sg] = ld16(xr + 512 * sg + 8 * lane);
  }
  auto wrow = [&](int i) { return W + (size_t)(gw + nw * min(i, mine - 1)) * K + 8 * lane; };
  u32x4 buf[D][NS];
#pragma unroll
  for (int u = 0; u < D; u++)
#pragma unroll
    for (int sg = 0; sg < NS; sg++) buf[u][sg] = ld_stream(wrow(u) + 512 * sg);
  unsigned long long best = 0;  // lanes 8k: the best key of emitted row k % R
  float v[8];
#pragma unroll
  for (int k = 0; k < 8; k++) v[k] = 0.f;
  // rows past `mine` read the wave's last row again (every path issues the same loads) and are
  // left out of the keys
  for (int i0 = 0; i0 < mine; i0 += 8) {
#pragma unroll
    for (int u = 0; u < 8; u++) {
      const int i = i0 + u, g = u % G;
#pragma unroll
      for (int r = 0; r < R; r++) {
        float acc = 0.f;
#pragma unroll
        for (int sg = 0; sg < NS; sg++) acc = dot8(buf[u % D][sg], x[r][sg], acc);
        v[g * R + r] = acc;
      }
#pragma unroll
      for (int sg = 0; sg < NS; sg++) buf[u % D][sg] = ld_stream(wrow(i + D) + 512 * sg);
      if (g == G - 1) {
        const float sum = wave_sum8(v, lane);  // lanes 8k..8k+7: slot k = (row g', emitted row r)
        const int k = lane >> 3, gk = k / R, rk = k % R;
        const int n = gw + nw * (i - (G - 1) + gk);
        if ((lane & 7) == 0 && k < G * R && i - (G - 1) + gk < mine && rk < nrow) {
          const uint32_t hb = f32_to_bf16(sum);
          if (logits) logits[(size_t)rk * V + n] = bf16_to_f32(hb);
          best = key_max(best, ((unsigned long long)orderable16(hb) << 32) | (unsigned long long)(0xffffffffu - (uint32_t)n));
        }
      }
    }
  }
  // each emitted row's best over its lanes (8k with k % R = r)
#pragma unroll
  for (int r = 0; r < R; r++) {
    unsigned long long b = ((lane & 7) == 0 && (lane >> 3) % R == r && (lane >> 3) < G * R) ? best : 0ull;
    b = wave_max_u64(b);
    if (lane == 0 && r < nrow) keys_part[(size_t)r * nw + gw] = b;
  }
}

// ---------------------------------------------------------------- decode step, few sequences
//
// One token per sequence, at most 16 sequences (one MFMA row tile), contexts
// up to kFusedCtx: seven launches per layer instead of eleven.
//
//   gemm_rows<NORM>(q,k,v)   input RMSNorm in the prologue, bf16 q|k|v out
//   attention_split          q/k head norm + RoPE, K/V append, scores and each
//                            position split's (max, sum) over all CUs;
//                            attention_pv the probabilities (HF's rounding) times
//                            V per split; attention_merge adds the splits
//   gemm_rows(o)             epilogue: residual add into the hidden rows
//   gemm_rows<NORM>(g|u)     post-attention RMSNorm in the prologue, SiLU(g)*u out
//   gemm_rows(down)          epilogue: residual add
//
// gemm_rows: one workgroup of 16 waves per 16*NB-column tile; wave w takes
// K/16 of the K range (the MFMA operand layout above) and the
// 16 partial tiles are summed in LDS in wave order, so every column is one
// fp32 sum rounded once, with no partials in memory and no finish kernel.

constexpr int kRowWaves = 16;
constexpr int kMaxRowsH = 2048;   // largest hidden size a NORM prologue stages in LDS
constexpr int kFusedCtx = 4096;   // longest context of the fused decode attention
constexpr int kAttnRounds = 4;    // fused attention: 64-position rounds of K or V loads in flight per wave

enum RowEpi : int { kEpiStore = 0, kEpiResidual = 1, kEpiSiluMul = 2 };

// Row of W feeding column `col` of tile `tile` (NC columns): kEpiSiluMul takes
// gate rows in columns 0..NC/2-1 and the up rows of the same NC/2 outputs in
// columns NC/2..NC-1; otherwise the seg rows in order.
template <int EPI, int NC>
__device__ __forceinline__ const uint16_t* tile_row(const Seg& seg, int tile, int col, int K) {
  if (EPI == kEpiSiluMul) return seg.w[col / (NC / 2)] + (size_t)(tile * (NC / 2) + col % (NC / 2)) * K;
  return seg_row(seg, tile * NC + col, K);
}

// Dynamic LDS of gemm_rows: the normalised input rows (NORM), then the NW
// partial tiles, then the per-wave sums of squares.
template <int NB, int NW, bool NORM>
constexpr size_t rows_lds(int T, int K) {
  return (NORM ? (size_t)((T * K * 2 + 15) / 16 * 16) : 0) + (size_t)NW * 16 * 16 * NB * 4 + (size_t)NW * 16 * 4 + 64;
}

// HALF: 8 output columns per tile (the MFMA's columns 8-15 repeat rows 0-7,
// whose loads the same instruction already makes), twice the workgroups of an
// N / 16 grid for the narrow o and down projections.
template <int NB, int EPI, bool NORM, int NW, int ITERS, int MAXT, bool HALF = false>
__global__ void __launch_bounds__(NW * 64) gemm_rows(const uint16_t* __restrict__ X, const uint16_t* __restrict__ norm_w,
                                                     float eps, int T, int K, Seg seg, uint16_t* __restrict__ Y,
                                                     int ldy) {
  constexpr int NC = 16 * NB;
  constexpr int NO = HALF ? 8 : NC;  // output columns per tile
  static_assert(!HALF || (NB == 1 && EPI != kEpiSiluMul), "half tiles: one 16-column MFMA tile, plain rows");
  extern __shared__ __align__(16) unsigned char smem[];
  uint16_t* xs = reinterpret_cast<uint16_t*>(smem);
  const size_t xs_bytes = NORM ? (size_t)((T * K * 2 + 15) / 16 * 16) : 0;
  float (*red)[16][NC] = reinterpret_cast<float (*)[16][NC]>(smem + xs_bytes);
  float (*ssr)[16] = reinterpret_cast<float (*)[16]>(smem + xs_bytes + (size_t)NW * 16 * NC * 4);
  float* rstd_s = reinterpret_cast<float*>(smem + xs_bytes + (size_t)NW * 16 * NC * 4 + (size_t)NW * 16 * 4);
  const int tile = blockIdx.x;
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int kq = 8 * (lane >> 4);
  const int k0 = w * (64 * ITERS);
  const int row = min(lane & 15, T - 1);
  // NORM: the T input rows in 16-byte chunks (chunk c = thread + NT * q covers row 8c / K) and
  // their norm weights are requested first, then the wave's whole weight slice, so that waiting
  // for the rows (vector memory returns in order) never waits for the weights
  constexpr int NT = NW * 64, MAXQ = NORM ? (MAXT * kMaxRowsH / 8 + NT - 1) / NT : 1;  // T <= MAXT
  const int nchunks = T * K / 8;
  u32x4 xr[MAXQ], wr[MAXQ];
  if (NORM) {
#pragma unroll
    for (int q = 0; q < MAXQ; q++) {
      const int c = threadIdx.x + NT * q;
      if (c < nchunks) {
        xr[q] = ld16(X + (size_t)c * 8);
        wr[q] = ld16(norm_w + (c * 8) % K);
      }
    }
  }
  bf16x8 b[ITERS][2][NB];
#pragma unroll
  for (int j = 0; j < NB; j++) {
    const uint16_t* wrow = (HALF ? tile_row<EPI, NO>(seg, tile, lane & 7, K)
                                 : tile_row<EPI, NC>(seg, tile, 16 * j + (lane & 15), K)) + kq + k0;
#pragma unroll
    for (int it = 0; it < ITERS; it++) {
      b[it][0][j] = ld_bf16x8_stream(wrow + 64 * it);
      b[it][1][j] = ld_bf16x8_stream(wrow + 64 * it + 32);
    }
  }
  if (NORM) {
    // RMSNorm of the rows into LDS, bf16(w * bf16(x * rstd)) as HF.  A wave's 64 chunks of one q
    // lie in one row (K / 8 is a multiple of 64), so each wave sum belongs to one row.
    float (*ssq)[NW] = reinterpret_cast<float (*)[NW]>(&ssr[0][0]);  // [MAXQ][NW] <= [16][NW]
#pragma unroll
    for (int q = 0; q < MAXQ; q++) {
      const int c0 = w * 64 + NT * q;  // the wave's first chunk of this q
      if (c0 < nchunks) {
        float part = 0.f;
        const u32x4 v = xr[q];
        const uint32_t u4[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int e = 0; e < 4; e++) {
          const float lo = lo_bf16(u4[e]), hi = hi_bf16(u4[e]);
          part += lo * lo + hi * hi;
        }
        part = wave_sum(part);
        if (lane == 0) ssq[q][w] = part;
      }
    }
    __syncthreads();
    if ((int)threadIdx.x < T) {
      // row t's wave sums, in (q, wave) order
      float ss = 0.f;
      for (int q = 0; q < MAXQ; q++)
        for (int ww = 0; ww < NW; ww++) {
          const int c0 = ww * 64 + NT * q;
          if (c0 < nchunks && (c0 * 8) / K == (int)threadIdx.x) ss += ssq[q][ww];
        }
      rstd_s[threadIdx.x] = rcp_sqrt_torch(__fdiv_rn(ss, (float)K) + eps);
    }
    __syncthreads();
#pragma unroll
    for (int q = 0; q < MAXQ; q++) {
      const int c = threadIdx.x + NT * q;
      if (c < nchunks) {
        const float r = rstd_s[(c * 8) / K];
        const uint32_t xv[4] = {xr[q].x, xr[q].y, xr[q].z, xr[q].w};
        const uint32_t wv[4] = {wr[q].x, wr[q].y, wr[q].z, wr[q].w};
        uint32_t o[4];
#pragma unroll
        for (int e = 0; e < 4; e++) {
          const float n0 = bf16r(lo_bf16(wv[e]) * bf16r(lo_bf16(xv[e]) * r));
          const float n1 = bf16r(hi_bf16(wv[e]) * bf16r(hi_bf16(xv[e]) * r));
          o[e] = f32_to_bf16(n0) | (f32_to_bf16(n1) << 16);
        }
        *reinterpret_cast<u32x4*>(xs + (size_t)c * 8) = u32x4{o[0], o[1], o[2], o[3]};
      }
    }
    __syncthreads();
  }
  auto load_a = [&](int k) -> bf16x8 {
    if (NORM) return *reinterpret_cast<const bf16x8*>(xs + row * K + kq + k);
    return ld_bf16x8(X + (size_t)row * K + kq + k);
  };
  bf16x8 a[ITERS][2];
#pragma unroll
  for (int it = 0; it < ITERS; it++) {
    a[it][0] = load_a(k0 + 64 * it);
    a[it][1] = load_a(k0 + 64 * it + 32);
  }
  f32x4 acc[NB];
#pragma unroll
  for (int j = 0; j < NB; j++) acc[j] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int it = 0; it < ITERS; it++)
#pragma unroll
    for (int j = 0; j < NB; j++) {
      acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[it][0], b[it][0][j], acc[j], 0, 0, 0);
      acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[it][1], b[it][1][j], acc[j], 0, 0, 0);
    }
#pragma unroll
  for (int j = 0; j < NB; j++)
#pragma unroll
    for (int i = 0; i < 4; i++) red[w][4 * (lane >> 4) + i][16 * j + (lane & 15)] = acc[j][i];
  __syncthreads();
  const int t = threadIdx.x / NO, c = threadIdx.x % NO;
  if (t >= T || t >= 16) return;
  auto col_sum = [&](int cc) {
    float y = 0.f;
#pragma unroll
    for (int q = 0; q < NW; q++) y += red[q][t][cc];  // wave order
    return y;
  };
  if (EPI == kEpiSiluMul) {
    if (c >= NC / 2) return;
    const float g = bf16r(col_sum(c)), u = bf16r(col_sum(c + NC / 2));
    const float sg = bf16r(__fdiv_rn(g, 1.0f + expf(-g)));
    Y[(size_t)t * ldy + tile * (NC / 2) + c] = (uint16_t)f32_to_bf16(bf16r(sg * u));
    return;
  }
  const float y = bf16r(col_sum(c));
  uint16_t* dst = Y + (size_t)t * ldy + tile * NO + c;
  if (EPI == kEpiResidual) *dst = (uint16_t)f32_to_bf16(bf16r(bf16_to_f32(*dst) + y));
  else *dst = (uint16_t)f32_to_bf16(y);
}

// Decode-step attention, split over positions: S workgroups of kSplitWaves
// waves per (sequence's token, KV head), S * T * 8 >= 256, so that every CU
// streams K/V (one workgroup per (token, KV head) left 224 of 256 CUs idle at
// four sequences), in HF's two passes over three launches:
// - attention_split requests the token's q/k/v head values, norm weights and
//   RoPE row, then every K row of its positions [pb, pe) (a CU returns loads in
//   order, so the small loads come first); forms the q heads 2g, 2g+1 and k head
//   g (head RMSNorm + RoPE, as HF), and split 0 appends the token's K/V at its
//   position (the token's own K is used from LDS, so no workgroup of this launch
//   reads that cache row); scores its positions as HF rounds them, stores them
//   (fp32) and writes the split's (max m, sum l of exp(s - m)) per head;
// - attention_pv merges the S (m, l) pairs into the global (M, L) in split order
//   (the same in every workgroup of the token), forms the probabilities
//   bf16(exp(s - M) * (1 / L)) as HF rounds them, and multiplies them with the V
//   rows of its positions: a partial P@V per split;
// - attention_merge adds the S partials in split order and rounds to bf16.
// Valid only when no other token of the launch writes this sequence's cache
// (one token per sequence).
constexpr int kSplitWaves = 4;    // waves per workgroup
constexpr int kSplitRounds = 8;   // 16-position rounds of K (or V) rows in flight per wave
constexpr int kMaxAttnSplit = 32;

struct AttnPart {
  float acc[2][kD];  // P@V of heads 2g, 2g+1 over the split's positions (probabilities normalised)
  float m[2], l[2];  // the split's maximum score and sum of exp(s - m)
};

// position splits per (token, KV head) for T tokens
int attn_splits(int T) { return std::min(kMaxAttnSplit, std::max(1, 256 / (kNKV * T))); }

// scores[(t * kNQ + head) * cap + p] of token t's positions p: written by attention_split, read
// by attention_pv
__global__ void __launch_bounds__(kSplitWaves * 64) attention_split(
    const uint16_t* __restrict__ QKV, const Tok* __restrict__ tok, int L, const uint16_t* q_norm,
    const uint16_t* k_norm, const uint16_t* cos_t, const uint16_t* sin_t, Cache c, float eps, float scale,
    AttnPart* __restrict__ part, float* __restrict__ scores, int cap, uint16_t* __restrict__ out) {
  __shared__ uint16_t qs[2][kD], kn[kD];
  __shared__ float wm[kSplitWaves][2], wl[kSplitWaves][2];
  const int t = blockIdx.x, g = blockIdx.y, sp = blockIdx.z, S = gridDim.z;
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63, slot = lane >> 4, t16 = lane & 15;
  const Tok tk = tok[t];
  if (!tk.valid) {
    if (sp == 0 && threadIdx.x < 2 * kD) out[(size_t)t * kQS + 2 * g * kD + threadIdx.x] = 0;
    return;
  }
  const int pos = tk.pos, C = pos + 1;
  const int chunk = (C + S - 1) / S;
  const int pb = min(C, sp * chunk), pe = min(C, pb + chunk);
  const size_t base = cache_base(c, tk, L, g);
  const uint16_t* kc = c.k + base;
  // waves 0, 1: q heads 2g, 2g+1; wave 2: k head g; wave 3: v head g
  const int h = w < 2 ? 2 * g + w : (w == 2 ? kNQ + g : kNQ + kNKV + g);
  const uint16_t* src = QKV + (size_t)t * kNQKV + h * kD;
  const uint16_t* nw = w < 2 ? q_norm : k_norm;
  const uint32_t x0b = ldu16(src + lane), x1b = ldu16(src + lane + 64);
  const uint32_t w0b = ldu16(nw + lane), w1b = ldu16(nw + lane + 64);
  const uint16_t* cr = cos_t + (size_t)pos * kD;
  const uint16_t* sr = sin_t + (size_t)pos * kD;
  const uint32_t c0b = ldu16(cr + lane), c1b = ldu16(cr + lane + 64);
  const uint32_t s0b = ldu16(sr + lane), s1b = ldu16(sr + lane + 64);
  // lane (slot, t16) of wave w takes dims 8*t16..+7 of position p0 + 16r + 4w + slot in round r;
  // positions outside [pb, pe) and pos itself load row 0 (every cache has it) and are masked
  u32x4 kx[kSplitRounds];
  auto issue = [&](int p0) {
#pragma unroll
    for (int r = 0; r < kSplitRounds; r++) {
      const int p = p0 + 16 * r + 4 * w + slot;
      kx[r] = ld16(kc + (size_t)((p < pe && p != pos) ? p : 0) * kD + 8 * t16);
    }
  };
  issue(pb);
  {
    const float x0 = bf16_to_f32(x0b), x1 = bf16_to_f32(x1b);
    if (w == 3) {
      if (sp == 0) {
        c.v[base + (size_t)pos * kD + lane] = (uint16_t)x0b;
        c.v[base + (size_t)pos * kD + lane + 64] = (uint16_t)x1b;
      }
    } else {
      const float ss = wave_sum(x0 * x0 + x1 * x1);
      const float rstd = rcp_sqrt_torch(__fdiv_rn(ss, (float)kD) + eps);
      const float n0 = bf16r(bf16_to_f32(w0b) * bf16r(x0 * rstd));
      const float n1 = bf16r(bf16_to_f32(w1b) * bf16r(x1 * rstd));
      const float c0 = bf16_to_f32(c0b), c1 = bf16_to_f32(c1b), s0 = bf16_to_f32(s0b), s1 = bf16_to_f32(s1b);
      const uint16_t y0 = (uint16_t)f32_to_bf16(bf16r(bf16r(n0 * c0) + bf16r(-n1 * s0)));
      const uint16_t y1 = (uint16_t)f32_to_bf16(bf16r(bf16r(n1 * c1) + bf16r(n0 * s1)));
      if (w < 2) {
        qs[w][lane] = y0;
        qs[w][lane + 64] = y1;
      } else {
        kn[lane] = y0;
        kn[lane + 64] = y1;
        if (sp == 0) {
          c.k[base + (size_t)pos * kD + lane] = y0;
          c.k[base + (size_t)pos * kD + lane + 64] = y1;
        }
      }
    }
  }
  __syncthreads();
  u32x4 qv[2];
#pragma unroll
  for (int hh = 0; hh < 2; hh++) qv[hh] = *reinterpret_cast<const u32x4*>(&qs[hh][8 * t16]);
  const u32x4 k_now = *reinterpret_cast<const u32x4*>(&kn[8 * t16]);
  float* const sc_out = scores + ((size_t)t * kNQ + 2 * g) * cap;
  float m[2] = {-INFINITY, -INFINITY}, l[2] = {0.f, 0.f};
  for (int p0 = pb; p0 < pe; p0 += 16 * kSplitRounds) {
    if (p0 != pb) issue(p0);  // positions beyond the first 16 * kSplitRounds of the split
    float sc[kSplitRounds][2], bm[2] = {-INFINITY, -INFINITY};
#pragma unroll
    for (int r = 0; r < kSplitRounds; r++) {
      const int p = p0 + 16 * r + 4 * w + slot;
      const u32x4 kr = p == pos ? k_now : kx[r];
#pragma unroll
      for (int hh = 0; hh < 2; hh++) {
        const float x = bf16r(bf16r(row16_sum(dot8(kr, qv[hh], 0.f))) * scale);
        sc[r][hh] = p < pe ? x : -INFINITY;
        bm[hh] = fmaxf(bm[hh], sc[r][hh]);
        if (t16 == 0 && p < pe) sc_out[(size_t)hh * cap + p] = x;
      }
    }
#pragma unroll
    for (int hh = 0; hh < 2; hh++) {
      float a, b;
      swap16(bm[hh], a, b);
      bm[hh] = fmaxf(a, b);
      swap32(bm[hh], a, b);
      bm[hh] = fmaxf(a, b);
      // rescale the running sum to the new maximum
      const float mn = fmaxf(m[hh], bm[hh]);
      l[hh] *= m[hh] == -INFINITY ? 0.f : exp_acc(m[hh] - mn);
      m[hh] = mn;
    }
#pragma unroll
    for (int r = 0; r < kSplitRounds; r++)
#pragma unroll
      for (int hh = 0; hh < 2; hh++) l[hh] += sc[r][hh] == -INFINITY ? 0.f : exp_acc(sc[r][hh] - m[hh]);
  }
  // the wave's four rows summed (every lane of a row holds the same terms; lane 0 speaks for them)
#pragma unroll
  for (int hh = 0; hh < 2; hh++) {
    l[hh] = rows_sum4(l[hh]);
    if (lane == 0) {
      wm[w][hh] = m[hh];
      wl[w][hh] = l[hh];
    }
  }
  __syncthreads();
  // this workgroup's (max, sum): the waves rescaled to its maximum, in wave order
  AttnPart* pt = part + ((size_t)t * kNKV + g) * S;
  if (threadIdx.x < 2) {
    const int hh = threadIdx.x;
    float mx = -INFINITY;
#pragma unroll
    for (int q = 0; q < kSplitWaves; q++) mx = fmaxf(mx, wm[q][hh]);
    float ls = 0.f;
#pragma unroll
    for (int q = 0; q < kSplitWaves; q++) ls += wm[q][hh] == -INFINITY ? 0.f : wl[q][hh] * exp_acc(wm[q][hh] - mx);
    pt[sp].m[hh] = mx;
    pt[sp].l[hh] = ls;
  }
}

// The second pass of a split: the global (max, sum) of (token t, KV head g) from its S splits' pairs
// in split order, the probabilities bf16(exp(s - M) * (1 / L)) of the split's positions (HF rounds
// them to bf16), and their product with V: AttnPart::acc of this split.
__global__ void __launch_bounds__(kSplitWaves * 64) attention_pv(const Tok* __restrict__ tok, int L, Cache c,
                                                                 AttnPart* __restrict__ part,
                                                                 const float* __restrict__ scores, int cap) {
  __shared__ float wacc[kSplitWaves][2][kD];
  const int t = blockIdx.x, g = blockIdx.y, sp = blockIdx.z, S = gridDim.z;
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63, slot = lane >> 4, t16 = lane & 15;
  const Tok tk = tok[t];
  if (!tk.valid) return;  // attention_split wrote the zeros
  const int C = tk.pos + 1;
  const int chunk = (C + S - 1) / S;
  const int pb = min(C, sp * chunk), pe = min(C, pb + chunk);
  const uint16_t* vc = c.v + cache_base(c, tk, L, g);
  // lane (slot, t16) of wave w takes dims 8*t16..+7 of position p0 + 16r + 4w + slot in round r;
  // positions outside [pb, pe) load row 0 and are masked
  u32x4 vx[kSplitRounds];
  auto issue = [&](int p0) {
#pragma unroll
    for (int r = 0; r < kSplitRounds; r++) {
      const int p = p0 + 16 * r + 4 * w + slot;
      vx[r] = ld16(vc + (size_t)(p < pe ? p : 0) * kD + 8 * t16);
    }
  };
  issue(pb);
  AttnPart* pt = part + ((size_t)t * kNKV + g) * S;
  float M[2], inv[2];
#pragma unroll
  for (int hh = 0; hh < 2; hh++) {
    float mx = -INFINITY;
    for (int q = 0; q < S; q++) mx = fmaxf(mx, pt[q].m[hh]);
    float ls = 0.f;
    for (int q = 0; q < S; q++) {
      const float mq = pt[q].m[hh];
      ls += mq == -INFINITY ? 0.f : pt[q].l[hh] * exp_acc(mq - mx);
    }
    M[hh] = mx;
    inv[hh] = __fdiv_rn(1.0f, ls);
  }
  const float* sc_in = scores + ((size_t)t * kNQ + 2 * g) * cap;
  float acc[2][8];
#pragma unroll
  for (int hh = 0; hh < 2; hh++)
#pragma unroll
    for (int i = 0; i < 8; i++) acc[hh][i] = 0.f;
  for (int p0 = pb; p0 < pe; p0 += 16 * kSplitRounds) {
    if (p0 != pb) issue(p0);
#pragma unroll
    for (int r = 0; r < kSplitRounds; r++) {
      const int p = p0 + 16 * r + 4 * w + slot;
      const u32x4 vr = vx[r];
      const float vf[8] = {lo_bf16(vr.x), hi_bf16(vr.x), lo_bf16(vr.y), hi_bf16(vr.y),
                           lo_bf16(vr.z), hi_bf16(vr.z), lo_bf16(vr.w), hi_bf16(vr.w)};
#pragma unroll
      for (int hh = 0; hh < 2; hh++) {
        const float pr = p < pe ? bf16r(exp_acc(sc_in[(size_t)hh * cap + p] - M[hh]) * inv[hh]) : 0.f;
        // a masked position (it loaded cache row 0, which the caller may not have written) leaves the
        // sum untouched, so that a NaN there cannot enter it through 0 * NaN
#pragma unroll
        for (int i = 0; i < 8; i++) acc[hh][i] = p < pe ? __builtin_fmaf(pr, vf[i], acc[hh][i]) : acc[hh][i];
      }
    }
  }
  // the wave's four rows summed; lanes 0..15 hold dims 8*t16..+7
#pragma unroll
  for (int hh = 0; hh < 2; hh++) {
#pragma unroll
    for (int i = 0; i < 8; i++) acc[hh][i] = rows_sum4(acc[hh][i]);
    if (lane < 16) {
#pragma unroll
      for (int i = 0; i < 8; i++) wacc[w][hh][8 * t16 + i] = acc[hh][i];
    }
  }
  __syncthreads();
  // this split's partial: the waves' in wave order
  {
    const int hh = threadIdx.x >> 7, d = threadIdx.x & 127;  // 256 threads: both heads' dims
    float a = 0.f;
#pragma unroll
    for (int q = 0; q < kSplitWaves; q++) a += wacc[q][hh][d];
    pt[sp].acc[hh][d] = a;
  }
}

// The attention output of (token t, KV head g): its S partials added in split order.  256 threads:
// thread i takes head 2g + i / 128, dim i % 128.
__global__ void __launch_bounds__(256) attention_merge(const Tok* __restrict__ tok, int S,
                                                       const AttnPart* __restrict__ part, uint16_t* __restrict__ out) {
  const int t = blockIdx.x, g = blockIdx.y;
  if (!tok[t].valid) return;  // attention_split wrote the zeros
  const AttnPart* pt = part + ((size_t)t * kNKV + g) * S;
  uint16_t* dst = out + (size_t)t * kQS + 2 * g * kD;
  const int hh = threadIdx.x >> 7, d = threadIdx.x & 127;
  float y = 0.f;
  for (int q = 0; q < S; q++) y += pt[q].acc[hh][d];
  dst[threadIdx.x] = (uint16_t)f32_to_bf16(y);
}

// ---------------------------------------------------------------- self-test

// C[16][16] = A[16][32] . B[16][32]^T through one MFMA with the operand
// layouts the GEMMs assume.
__global__ void mfma_selftest(const uint16_t* A, const uint16_t* B, float* C) {
  const int lane = threadIdx.x, kq = 8 * (lane >> 4);
  const bf16x8 a = ld_bf16x8(A + (lane & 15) * 32 + kq);
  const bf16x8 b = ld_bf16x8(B + (lane & 15) * 32 + kq);
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, acc, 0, 0, 0);
#pragma unroll
  for (int i = 0; i < 4; i++) C[(4 * (lane >> 4) + i) * 16 + (lane & 15)] = acc[i];
}

// ---------------------------------------------------------------- host side

struct Gemm {
  int ksplit, tn;  // K splits, tile width (128 or 64 columns)
};

// Every projection of both models takes the LDS-tiled GEMM at any token count: N a multiple of the
// 128-column tile and K a multiple of four 64-wide steps.  (A register-staged MFMA GEMM, one wave
// per 16-row tile, ran below 96 tokens before; the tiled kernel on a 128-row tile whose rows past
// T repeat the last one was faster at every count measured: 4 tokens 1.55 -> 1.34 ms per 0.6B
// prefill, 64 tokens 2.09 -> 1.55, 80 tokens 2.43 -> 1.65.)
template <class M>
constexpr bool tiled_shapes() {
  using Dm = Dims<M>;
  constexpr int kStep4 = 4 * kTK;
  return kNQKV % 128 == 0 && Dm::H % 128 == 0 && (2 * Dm::I) % 128 == 0 && Dm::H % kStep4 == 0 &&
         kQS % kStep4 == 0 && Dm::I % kStep4 == 0;
}
static_assert(tiled_shapes<Qwen3_0_6B>() && tiled_shapes<Qwen3_1_7B>(), "projection shapes of the tiled GEMM");

// 128-column tiles: K split (at most 8 ways, >= 4 steps of 64 each) until about 512 workgroups
// run, two per CU.
int tiled_splits(int T, int N, int K) {
  const long long tiles = (long long)((T + kTM - 1) / kTM) * (N / 128);
  int ks = 1;
  while (tiles * ks < 512 && ks < 8 && K % (ks * 2 * 4 * kTK) == 0) ks *= 2;
  return ks;
}

// 64-column tiles, for problems whose 128-column plan leaves CUs idle (narrow N at a few hundred
// rows or fewer): K split (at most 16 ways, >= 2 steps of 64 each) until 256 workgroups run (512
// for at most 16 rows, whose partials are small: 4-token prefill 1.245 -> 1.20 ms, 16 tokens 1.266
// -> 1.245; at 64 tokens 512 was slower, 1.535 -> 1.585), while the fp32 partials
// (ksplit * T * N * 4 bytes) stay within twice the weight bytes (N * K * 2).
int narrow_splits(int T, int N, int K) {
  const long long tiles = (long long)((T + kTM - 1) / kTM) * (N / 64), target = T <= 16 ? 512 : 256;
  int ks = 1;
  while (tiles * ks < target && ks * 2 <= kMaxSplit && K % (ks * 2 * kTK) == 0 && K / (ks * 2) >= 2 * kTK &&
         (long long)ks * 2 * T * 4 <= 2LL * K * 2)
    ks *= 2;
  return ks;
}

Gemm plan_gemm(int T, int N, int K) {
  const int ks = tiled_splits(T, N, K);
  const long long wgs = (long long)((T + kTM - 1) / kTM) * (N / 128) * ks;
  if (wgs >= 256) return {ks, 128};
  const int ks64 = narrow_splits(T, N, K);
  if ((long long)((T + kTM - 1) / kTM) * (N / 64) * ks64 > wgs) return {ks64, 64};
  return {ks, 128};
}

// The q/k/v and gate/up GEMMs with their finishing work in the epilogue (kEpiQkv, kEpiGateUp)
// when the plan can leave K unsplit: at least kFuseMinWG 128-column tiles (q/k/v: that many per
// 1024 of K).  Then no fp32 sums go to memory and no finishing kernel runs; *ks_out = 0 says so.
// Otherwise the sums go to part and *ks_out is the split count for the finishing kernel.  With
// half the CUs given a tile, the unsplit GEMM plus its epilogue still beats the split one plus the
// finishing kernel (prefill ms, against a bound of one tile per CU: 0.6B 384 tokens 2.84-2.90 ->
// 2.67-2.74, 512 3.25-3.34 -> 3.01-3.10, 640 3.80-3.88 -> 3.30-3.36, 896 4.08-4.19 -> 3.79-3.88;
// 1.7B 256 tokens 3.47-3.57 -> 3.31-3.38, gate/up on 192 tiles); with a quarter it loses (0.6B
// 256 tokens 2.39-2.45 -> 2.62-2.65, q/k/v on 64 tiles and gate/up on 96), and so does the 1.7B
// q/k/v, whose K of 2048 doubles each tile's work, on 128 and 160 tiles (512 tokens 4.06-4.15
// -> 4.38-4.49, 640 5.10-5.20 -> 5.27-5.37).
constexpr int kFuseMinWG = 128;

void launch_gemm(const uint16_t* X, int T, int K, const Seg& seg, int N, float* part, hipStream_t s, int* ks_out,
                 int epi = kEpiPart, const QkvOut* qo = nullptr, const GateUpOut* go = nullptr) {
  const QkvOut q0 = qo ? *qo : QkvOut{};
  const GateUpOut g0 = go ? *go : GateUpOut{};
  const long long fuse_min = epi == kEpiQkv ? (long long)kFuseMinWG * std::max(1, K / 1024) : kFuseMinWG;
  if (epi != kEpiPart && (long long)((T + kTM - 1) / kTM) * (N / 128) >= fuse_min) {
    const dim3 grid(N / 128, (T + kTM - 1) / kTM, 1);
    if (epi == kEpiQkv)
      hipLaunchKernelGGL((gemm_tiled<128, kEpiQkv>), grid, dim3(256), 0, s, X, T, K, seg, N, 1, part, q0, g0);
    else
      hipLaunchKernelGGL((gemm_tiled<128, kEpiGateUp>), grid, dim3(256), 0, s, X, T, K, seg, N, 1, part, q0, g0);
    *ks_out = 0;
    return;
  }
  const Gemm g = plan_gemm(T, N, K);
  const dim3 grid(N / g.tn, (T + kTM - 1) / kTM, g.ksplit);
  if (g.tn == 128)
    hipLaunchKernelGGL((gemm_tiled<128, kEpiPart>), grid, dim3(256), 0, s, X, T, K, seg, N, g.ksplit, part, q0, g0);
  else
    hipLaunchKernelGGL((gemm_tiled<64, kEpiPart>), grid, dim3(256), 0, s, X, T, K, seg, N, g.ksplit, part, q0, g0);
  *ks_out = g.ksplit;
}

size_t part_floats(int T, int N, int K) { return (size_t)plan_gemm(T, N, K).ksplit * T * N; }

int split_chunks(int max_context) { return (max_context + kSplitChunk - 1) / kSplitChunk; }

// The context-split attention (three launches, each token's context over workgroups of 64
// positions) for few tokens over a longer context; the row kernel (one launch) for few tokens over
// a short one.  Qwen3-0.6B prefills, split against rows, same box: from position 0, 1 token 1.31 /
// 1.21 ms and 31 tokens 1.45 / 1.35; from 96, 1.41 / 1.39; from 192, 1.46 / 1.56; from 500, 1.45 /
// 2.14.  Its work grows with tokens x context, attention_mfma's with the context alone (a 64-token
// tile costs the same for 1 token as for 64), so a prompt of one sequence takes attention_mfma
// from about 6144 tokens x positions (split against attention_mfma with its keys in chunks: 8
// tokens after 600 positions 1.55 / 1.62 ms; 2 after 1500 1.61 / 1.64, 8 after 1500 1.83 / 1.68;
// 1 after 4000 2.01 / 2.07, 2 after 4000 2.12 / 2.08; 1 after 7000 2.60 / 2.38; 31 after 7000
// 17.96 / 2.42).  A batched decode step (one token per sequence, whose tiles hold several
// sequences and would fall back to the row kernel) keeps the split form.
constexpr int kSplitWork = 6144;
bool split_attention(int T, int max_context, bool one_per_seq) {
  return T < kSplitBelow && max_context > kSplitContext && (one_per_seq || (long long)T * max_context < kSplitWork);
}

// attention_mfma pays off from about 320 tokens or 256 positions of context (below that the row
// kernel's per-token reads are cheaper than its passes).  Measured 0.6B prefills, row kernel
// against attention_mfma: 256 tokens 2.55 / 2.62 ms, 384 tokens 3.37 / 3.18, 512 tokens 4.23 /
// 3.67, 768 tokens 5.85 / 4.45; with its keys in chunks (below), after 400 positions: 32 tokens
// 2.01 / 1.78, 256 tokens 3.57 / 2.45; after 950: 64 tokens 3.06 / 1.99.
bool mfma_attention(int T, int max_context, bool one_per_seq) {
  return !split_attention(T, max_context, one_per_seq) && (T >= kMfmaAttnTokens || max_context >= kMfmaAttnContext);
}

// attention_mfma's keys in chunks of ck blocks (nch > 1: the split passes) when its tile pairs would
// leave CUs idle and either the context before the prompt is at least as long as the prompt (a
// prompt of few tiles over a long context, e.g. a new turn appended to a long conversation, where
// each pair's workgroup would walk the whole context alone: Qwen3-0.6B, pairs against chunks, 128
// tokens after 7000 positions 13.9 / 2.8 ms, 32 tokens after 4000 4.82 / 1.90) or the prompt has
// at most 8 tiles (from position 0: 384 tokens 2.87-2.90 / 2.82-2.83, 512 tokens 3.32-3.36 /
// 3.24; with more tiles from position 0 the pairs balance the causal work as well: 768 tokens
// 3.70-3.74 / 3.75-3.76, 1024 tokens 3.97-4.00 / 3.99).
// Up to 8 tiles, at most kMaxAttnChunks tile chunks, at least two blocks each: 256 workgroups, so
// the second pass (one workgroup per CU) runs in one round (at most 32: 32 tokens after 7,000
// positions 2.39-2.44 against 2.02-2.07 ms per prefill; at most 8: 2.34-2.38).  More tiles take up
// to 4 x kMaxAttnChunks tile chunks, two or more rounds, rather than one chunk each (1024 tokens
// after 4000 positions 10.76 -> 7.56 ms, after 6000 14.05 -> 9.17).  The fp32 partials (32 KB per
// tile chunk and head) stay within 32 MB.
struct AttnSplit {
  int nch, ck;
};
AttnSplit attn_mfma_split(int T, int max_context) {
  const int nt = (T + kQT - 1) / kQT, nkb = (max_context + kKB - 1) / kKB;
  if ((nt + 1) / 2 * kNQ >= kNumWG || (max_context < 2 * T && nt > 8)) return {1, nkb};
  const int nch = std::min((nt <= 8 ? kMaxAttnChunks : 4 * kMaxAttnChunks) / nt, nkb / 2);
  if (nch < 2) return {1, nkb};
  const int ck = (nkb + nch - 1) / nch;
  return {(nkb + ck - 1) / ck, ck};
}

struct Layout {
  size_t tok, erow, keys, x, n, q, att, m, qkv, apart, part, scores, ml, pv, redo, mml, mpart, total;
};

constexpr int kLmTiles(int V) { return V / 64; }

// The decode step of few sequences (one token each) takes the fused path.
bool fused_decode(int T, int max_context) { return T <= 16 && max_context <= kFusedCtx; }

template <class M>
Layout layout(int T, int R, int max_context, bool one_per_seq = false) {
  using Dm = Dims<M>;
  auto al = [](size_t b) { return (b + 255) & ~(size_t)255; };
  Layout l{};
  size_t off = 0;
  auto take = [&](size_t& field, size_t bytes) {
    field = off;
    off += al(bytes);
  };
  take(l.tok, (size_t)T * sizeof(Tok));
  take(l.erow, (size_t)R * 4);
  take(l.keys, (size_t)R * std::max(kLmTiles(Dm::V), kLmBlocks * kLmWaves) * 8);
  take(l.x, (size_t)T * Dm::H * 2);
  take(l.n, (size_t)T * Dm::H * 2);
  take(l.q, (size_t)T * kQS * 2);
  take(l.att, (size_t)T * kQS * 2);
  take(l.m, (size_t)T * Dm::I * 2);
  if (one_per_seq && fused_decode(T, max_context)) {
    take(l.qkv, (size_t)T * kNQKV * 2);
    take(l.apart, (size_t)T * kNKV * attn_splits(T) * sizeof(AttnPart));
    take(l.scores, (size_t)T * kNQ * max_context * 4);
    l.total = off;
    return l;
  }
  size_t pf = part_floats(T, kNQKV, Dm::H);
  pf = std::max(pf, part_floats(T, Dm::H, kQS));
  pf = std::max(pf, part_floats(T, 2 * Dm::I, Dm::H));
  pf = std::max(pf, part_floats(T, Dm::H, Dm::I));
  take(l.part, pf * 4);
  // the buffers of every attention form the forward may pick for these sizes (one token per
  // sequence or not: the workspace size query does not say)
  if (split_attention(T, max_context, true)) {
    const int nch = split_chunks(max_context);
    take(l.scores, (size_t)T * kNQ * nch * kSplitChunk * 4);
    take(l.ml, (size_t)T * kNQ * nch * 8);
    take(l.pv, (size_t)T * nch * kQS * 4);
  }
  take(l.redo, (size_t)((T + kQT - 1) / kQT) * 4);
  const AttnSplit sp = attn_mfma_split(T, max_context);
  if (mfma_attention(T, max_context, false) && sp.nch > 1) {  // attention_mfma's chunks: (max, sum), partials
    const size_t rows = (size_t)((T + kQT - 1) / kQT) * kNQ * sp.nch * kQT;
    take(l.mml, rows * sizeof(float2));
    take(l.mpart, rows * kD * 4);
  }
  l.total = off;
  return l;
}

struct Args {
  int T, R, num_seqs, max_context;
  bool one_per_seq;  // token t is sequence t's only token (batched decode step)
  const int *tokens, *seqs, *pos, *emit;
  int* out_tokens;
  float* logits;
  const uint16_t *embed, *final_norm, *lm_head, *cos_t, *sin_t;
  const LDGLayerWeights* layers;  // host array
  Cache cache;
  int num_layers;
  float attn_scale;
  char* ws;
};

// LM head + argmax of R emitted rows: the streamed persistent form for R <= 16,
// the tiled GEMM above that.
template <class M>
void launch_lm_head(const uint16_t* N, const int* erow, int R, const uint16_t* W, unsigned long long* keys,
                    float* logits, const Tok* tok, int* out, hipStream_t s) {
  using Dm = Dims<M>;
  if (R <= 4) {
    const dim3 grid(kLmBlocks), block(kLmWaves * 64);
    switch (R) {
      case 1: hipLaunchKernelGGL((lm_head_rows<1, Dm::H>), grid, block, 0, s, N, erow, R, W, Dm::V, keys, logits); break;
      case 2: hipLaunchKernelGGL((lm_head_rows<2, Dm::H>), grid, block, 0, s, N, erow, R, W, Dm::V, keys, logits); break;
      case 3: hipLaunchKernelGGL((lm_head_rows<3, Dm::H>), grid, block, 0, s, N, erow, R, W, Dm::V, keys, logits); break;
      default: hipLaunchKernelGGL((lm_head_rows<4, Dm::H>), grid, block, 0, s, N, erow, R, W, Dm::V, keys, logits); break;
    }
    hipLaunchKernelGGL(keys_reduce, dim3(R), dim3(256), 0, s, keys, kLmBlocks * kLmWaves, erow, tok, out);
    return;
  }
  if (R <= 16) {
    const size_t lds = (size_t)R * Dm::H * 2;
    hipLaunchKernelGGL(lm_head_stream, dim3(kLmBlocks), dim3(kLmWaves * 64), lds, s, N, erow, R, W, Dm::H, Dm::V,
                       keys, logits);
    hipLaunchKernelGGL(keys_reduce, dim3(R), dim3(256), 0, s, keys, kLmBlocks * kLmWaves, erow, tok, out);
    return;
  }
  const int lm_waves = ((R + 15) / 16) * kLmTiles(Dm::V);
  hipLaunchKernelGGL(lm_head_gemm, dim3((lm_waves + 3) / 4), dim3(256), 0, s, N, erow, R, W, Dm::H, Dm::V, keys,
                     logits);
  hipLaunchKernelGGL(keys_reduce, dim3(R), dim3(256), 0, s, keys, kLmTiles(Dm::V), erow, tok, out);
}

// gemm_rows over `tiles` 16-column tiles (NB = 1), NW waves each taking
// K / NW = 64 * ITERS of the K range; ITERS picked from K.
template <int EPI, bool NORM, int NW, int ITERS, int MAXT, bool HALF>
void launch_rows_t(int tiles, const uint16_t* X, const uint16_t* nw, float eps, int T, int K, const Seg& seg,
                   uint16_t* Y, int ldy, hipStream_t s) {
  const size_t lds = rows_lds<1, NW, NORM>(T, K);
  if (lds > 64 * 1024) {
    // 16 normalised rows of 2048: above the default dynamic LDS limit (gfx950 has 160 KB per CU)
    static bool raised = false;
    if (!raised)
      raised = hipFuncSetAttribute(reinterpret_cast<const void*>(gemm_rows<1, EPI, NORM, NW, ITERS, MAXT, HALF>),
                                   hipFuncAttributeMaxDynamicSharedMemorySize, 96 * 1024) == hipSuccess;
  }
  hipLaunchKernelGGL((gemm_rows<1, EPI, NORM, NW, ITERS, MAXT, HALF>), dim3(tiles), dim3(NW * 64), lds, s, X, nw, eps, T,
                     K, seg, Y, ldy);
}

// NORM kernels stage the rows in registers sized for T <= 4 (the common batch) or T <= 16.
template <int EPI, bool NORM, int NW, int ITERS, bool HALF>
void launch_rows_it(int tiles, const uint16_t* X, const uint16_t* nw, float eps, int T, int K, const Seg& seg,
                    uint16_t* Y, int ldy, hipStream_t s) {
  if (!NORM || T <= 4) launch_rows_t<EPI, NORM, NW, ITERS, 4, HALF>(tiles, X, nw, eps, T, K, seg, Y, ldy, s);
  else launch_rows_t<EPI, NORM, NW, ITERS, 16, HALF>(tiles, X, nw, eps, T, K, seg, Y, ldy, s);
}

// `tiles` tiles of 16 output columns, or of 8 (HALF)
template <int EPI, bool NORM, int NW, bool HALF = false>
void launch_rows(int tiles, const uint16_t* X, const uint16_t* nw, float eps, int T, int K, const Seg& seg,
                 uint16_t* Y, int ldy, hipStream_t s) {
  switch (K / (64 * NW)) {
    case 1: launch_rows_it<EPI, NORM, NW, 1, HALF>(tiles, X, nw, eps, T, K, seg, Y, ldy, s); break;
    case 2: launch_rows_it<EPI, NORM, NW, 2, HALF>(tiles, X, nw, eps, T, K, seg, Y, ldy, s); break;
    case 3: launch_rows_it<EPI, NORM, NW, 3, HALF>(tiles, X, nw, eps, T, K, seg, Y, ldy, s); break;
    case 4: launch_rows_it<EPI, NORM, NW, 4, HALF>(tiles, X, nw, eps, T, K, seg, Y, ldy, s); break;
    default: launch_rows_it<EPI, NORM, NW, 6, HALF>(tiles, X, nw, eps, T, K, seg, Y, ldy, s); break;
  }
}

template <class M>
int forward_fused(const Args& a, hipStream_t s) {
  using Dm = Dims<M>;
  const int T = a.T, R = a.R;
  const Layout l = layout<M>(T, R, a.max_context, true);
  Tok* tok = reinterpret_cast<Tok*>(a.ws + l.tok);
  int* erow = reinterpret_cast<int*>(a.ws + l.erow);
  auto* keys = reinterpret_cast<unsigned long long*>(a.ws + l.keys);
  uint16_t* X = reinterpret_cast<uint16_t*>(a.ws + l.x);
  uint16_t* N = reinterpret_cast<uint16_t*>(a.ws + l.n);
  uint16_t* ATT = reinterpret_cast<uint16_t*>(a.ws + l.att);
  uint16_t* MM = reinterpret_cast<uint16_t*>(a.ws + l.m);
  uint16_t* QKV = reinterpret_cast<uint16_t*>(a.ws + l.qkv);
  const float eps = 1e-6f;
  auto u16 = [](const void* p) { return static_cast<const uint16_t*>(p); };
  // every K is split into 16 (8 for gate/up) slices of 64 * {1, 2, 3, 4, 6}
  static_assert(Dm::H == 1024 || Dm::H == 2048, "K splits of the hidden size");
  static_assert(Dm::I == 3072 || Dm::I == 6144, "K splits of the MLP size");
  static_assert(kQS == 2048 && Dm::H <= kMaxRowsH, "K splits of the attention output");
  AttnPart* apart = reinterpret_cast<AttnPart*>(a.ws + l.apart);
  float* ascores = reinterpret_cast<float*>(a.ws + l.scores);
  const int nsplit = attn_splits(T);
  hipLaunchKernelGGL(prep_tokens, dim3((std::max(T, R) + 255) / 256), dim3(256), 0, s, a.tokens, a.seqs, a.pos, T,
                     a.emit, R, a.num_seqs, a.max_context, Dm::V, tok, erow);
  hipLaunchKernelGGL(embed_rows, dim3(T), dim3(256), 0, s, a.embed, tok, Dm::H, X);
  for (int L = 0; L < a.num_layers; L++) {
    const LDGLayerWeights& w = a.layers[L];
    const Seg qkv{{u16(w.q_proj_weight), u16(w.k_proj_weight), u16(w.v_proj_weight)}, {kQS, kNKV * kD, kNKV * kD}};
    launch_rows<kEpiStore, true, 16>(kNQKV / 16, X, u16(w.input_layernorm_weight), eps, T, Dm::H, qkv, QKV, kNQKV, s);
    hipLaunchKernelGGL(attention_split, dim3(T, kNKV, nsplit), dim3(kSplitWaves * 64), 0, s, QKV, tok, L,
                       u16(w.q_norm_weight), u16(w.k_norm_weight), a.cos_t, a.sin_t, a.cache, eps, a.attn_scale,
                       apart, ascores, a.max_context, ATT);
    hipLaunchKernelGGL(attention_pv, dim3(T, kNKV, nsplit), dim3(kSplitWaves * 64), 0, s, tok, L, a.cache, apart,
                       ascores, a.max_context);
    hipLaunchKernelGGL(attention_merge, dim3(T, kNKV), dim3(256), 0, s, tok, nsplit, apart, ATT);
    const Seg o{{u16(w.o_proj_weight), nullptr, nullptr}, {Dm::H, 0, 0}};
    launch_rows<kEpiResidual, false, 16, true>(Dm::H / 8, ATT, nullptr, eps, T, kQS, o, X, Dm::H, s);
    const Seg gu{{u16(w.gate_proj_weight), u16(w.up_proj_weight), nullptr}, {Dm::I, Dm::I, 0}};
    launch_rows<kEpiSiluMul, true, 8>(Dm::I / 8, X, u16(w.post_attn_layernorm_weight), eps, T, Dm::H, gu, MM, Dm::I,
                                      s);
    const Seg dn{{u16(w.down_proj_weight), nullptr, nullptr}, {Dm::H, 0, 0}};
    launch_rows<kEpiResidual, false, 16, true>(Dm::H / 8, MM, nullptr, eps, T, Dm::I, dn, X, Dm::H, s);
  }
  hipLaunchKernelGGL((residual_norm<Dm::H>), dim3(T), dim3(256), 0, s, nullptr, 0, T, X, a.final_norm, eps, N);
  launch_lm_head<M>(N, erow, R, a.lm_head, keys, a.logits, tok, a.out_tokens, s);
  return hipGetLastError() == hipSuccess ? QMK_OK : QMK_ERR_HIP;
}

template <class M>
int forward(const Args& a, hipStream_t s) {
  using Dm = Dims<M>;
  const int T = a.T, R = a.R;
  if (a.one_per_seq && fused_decode(T, a.max_context)) return forward_fused<M>(a, s);
  const Layout l = layout<M>(T, R, a.max_context);
  Tok* tok = reinterpret_cast<Tok*>(a.ws + l.tok);
  int* erow = reinterpret_cast<int*>(a.ws + l.erow);
  auto* keys = reinterpret_cast<unsigned long long*>(a.ws + l.keys);
  uint16_t* X = reinterpret_cast<uint16_t*>(a.ws + l.x);
  uint16_t* N = reinterpret_cast<uint16_t*>(a.ws + l.n);
  uint16_t* Qb = reinterpret_cast<uint16_t*>(a.ws + l.q);
  uint16_t* ATT = reinterpret_cast<uint16_t*>(a.ws + l.att);
  uint16_t* MM = reinterpret_cast<uint16_t*>(a.ws + l.m);
  float* part = reinterpret_cast<float*>(a.ws + l.part);
  const float eps = 1e-6f;
  const bool split = split_attention(T, a.max_context, a.one_per_seq);
  const int nch = split ? split_chunks(a.max_context) : 0;
  const bool mfma_attn = mfma_attention(T, a.max_context, a.one_per_seq);
  const AttnSplit asp = attn_mfma_split(T, a.max_context);
  auto blocks = [](size_t n) { return dim3((unsigned)((n + 255) / 256)); };
  auto u16 = [](const void* p) { return static_cast<const uint16_t*>(p); };
  int ks = 1;

  hipLaunchKernelGGL(prep_tokens, blocks(std::max(T, R)), dim3(256), 0, s, a.tokens, a.seqs, a.pos, T, a.emit, R,
                     a.num_seqs, a.max_context, Dm::V, tok, erow);
  hipLaunchKernelGGL(embed_rows, dim3(T), dim3(256), 0, s, a.embed, tok, Dm::H, X);
  hipLaunchKernelGGL((residual_norm<Dm::H>), dim3(T), dim3(256), 0, s, nullptr, 0, T, X,
                     u16(a.layers[0].input_layernorm_weight), eps, N);
  for (int L = 0; L < a.num_layers; L++) {
    const LDGLayerWeights& w = a.layers[L];
    const Seg qkv{{u16(w.q_proj_weight), u16(w.k_proj_weight), u16(w.v_proj_weight)}, {kQS, kNKV * kD, kNKV * kD}};
    const QkvOut qo{tok, L, u16(w.q_norm_weight), u16(w.k_norm_weight), a.cos_t, a.sin_t, a.cache, eps, Qb};
    launch_gemm(N, T, Dm::H, qkv, kNQKV, part, s, &ks, kEpiQkv, &qo);
    if (ks) hipLaunchKernelGGL(qkv_finish, dim3(T, kNQ + 2 * kNKV), dim3(64), 0, s, part, ks, T, qo);
    if (split) {
      float* scores = reinterpret_cast<float*>(a.ws + l.scores);
      float2* ml = reinterpret_cast<float2*>(a.ws + l.ml);
      float* pvp = reinterpret_cast<float*>(a.ws + l.pv);
      hipLaunchKernelGGL(attn_split_scores, dim3(T, kNKV, nch), dim3(256), 0, s, Qb, tok, L, a.cache, a.attn_scale,
                         nch, scores, ml);
      hipLaunchKernelGGL(attn_split_pv, dim3(T, kNKV, nch), dim3(256), 0, s, tok, L, a.cache, nch, scores, ml, pvp);
      hipLaunchKernelGGL(attn_split_merge, dim3(T, kQS / 256), dim3(256), 0, s, tok, nch, pvp, ATT);
    } else {
      if (mfma_attn) {
        // tiles of one sequence's consecutive tokens on MFMA; any other tile row by row
        int* redo = reinterpret_cast<int*>(a.ws + l.redo);
        const int ntiles = (T + kQT - 1) / kQT;
        if (asp.nch > 1) {
          float2* aml = reinterpret_cast<float2*>(a.ws + l.mml);
          float* apart = reinterpret_cast<float*>(a.ws + l.mpart);
          const dim3 grid(ntiles * asp.nch, kNQ);
          hipLaunchKernelGGL(attention_mfma_pass1, grid, dim3(kAttnWaves * 64), 0, s, Qb, tok, T, L, a.cache,
                             a.attn_scale, ATT, redo, asp.nch, asp.ck, aml, apart);
          hipLaunchKernelGGL(attention_mfma_pass2, grid, dim3(kAttnWaves * 64), 0, s, Qb, tok, T, L, a.cache,
                             a.attn_scale, ATT, redo, asp.nch, asp.ck, aml, apart);
          hipLaunchKernelGGL(attention_mfma_merge, dim3(T, kNQ), dim3(kD), 0, s, tok, T, asp.nch, asp.ck, apart, redo,
                             ATT);
        } else {
          hipLaunchKernelGGL(attention_mfma, dim3((ntiles + 1) / 2, kNQ), dim3(kAttnWaves * 64), 0, s, Qb,
                             tok, T, L, a.cache, a.attn_scale, ATT, redo, 1, 0, nullptr, nullptr);
        }
        // the tiles attention_mfma left (redo) row by row: 256 x 8 workgroups loop over the tokens
        hipLaunchKernelGGL(attention_rows, dim3(std::min(T, 256), kNKV), dim3(256), 0, s, Qb, tok, T, L, a.cache,
                           a.attn_scale, ATT, redo);
      } else {
        hipLaunchKernelGGL(attention_rows, dim3(T, kNKV), dim3(256), 0, s, Qb, tok, T, L, a.cache, a.attn_scale, ATT,
                           nullptr);
      }
    }
    const Seg o{{u16(w.o_proj_weight), nullptr, nullptr}, {Dm::H, 0, 0}};
    launch_gemm(ATT, T, kQS, o, Dm::H, part, s, &ks);
    hipLaunchKernelGGL((residual_norm<Dm::H>), dim3(T), dim3(256), 0, s, part, ks, T, X,
                       u16(w.post_attn_layernorm_weight), eps, N);
    const Seg gu{{u16(w.gate_proj_weight), u16(w.up_proj_weight), nullptr}, {Dm::I, Dm::I, 0}};
    const GateUpOut go{MM, Dm::I};
    launch_gemm(N, T, Dm::H, gu, 2 * Dm::I, part, s, &ks, kEpiGateUp, nullptr, &go);
    if (ks) hipLaunchKernelGGL(gate_up_finish, blocks((size_t)T * Dm::I), dim3(256), 0, s, part, ks, T, Dm::I, MM);
    const Seg dn{{u16(w.down_proj_weight), nullptr, nullptr}, {Dm::H, 0, 0}};
    launch_gemm(MM, T, Dm::I, dn, Dm::H, part, s, &ks);
    const uint16_t* next_norm = L + 1 < a.num_layers ? u16(a.layers[L + 1].input_layernorm_weight) : a.final_norm;
    hipLaunchKernelGGL((residual_norm<Dm::H>), dim3(T), dim3(256), 0, s, part, ks, T, X, next_norm, eps, N);
  }
  launch_lm_head<M>(N, erow, R, a.lm_head, keys, a.logits, tok, a.out_tokens, s);
  return hipGetLastError() == hipSuccess ? QMK_OK : QMK_ERR_HIP;
}

}  // namespace batch
}  // namespace qmk

using namespace qmk;

extern "C" {

size_t qmk_forward_workspace_bytes(int model, int num_tokens, int num_emit, int max_context) {
  if (num_tokens < 1 || num_emit < 1 || num_emit > batch::kMaxEmit || max_context < 1) return 0;
  if (model == QMK_MODEL_QWEN3_1_7B) return batch::layout<Qwen3_1_7B>(num_tokens, num_emit, max_context).total;
  if (model == QMK_MODEL_QWEN3_0_6B) return batch::layout<Qwen3_0_6B>(num_tokens, num_emit, max_context).total;
  return 0;
}

int qmk_forward_tokens(int model, int num_tokens, const int* tokens, const int* seq_ids, const int* positions,
                       int num_emit, const int* emit_rows, int* out_tokens, float* logits_out,
                       const void* embed_weight, const LDGLayerWeights* layer_weights_host,
                       const void* final_norm_weight, const void* lm_head_weight, const void* cos_table,
                       const void* sin_table, void* k_cache, void* v_cache, int num_seqs, long long seq_stride,
                       int num_layers, int max_seq_len, int max_context, float attn_scale, void* workspace,
                       size_t workspace_bytes, hipStream_t stream) {
  if (model != QMK_MODEL_QWEN3_0_6B && model != QMK_MODEL_QWEN3_1_7B) return QMK_ERR_ARG;
  if (num_tokens < 1 || num_emit < 1 || num_emit > batch::kMaxEmit || !tokens || !seq_ids || !positions ||
      !emit_rows || !out_tokens || !embed_weight || !layer_weights_host || !final_norm_weight || !lm_head_weight ||
      !cos_table || !sin_table || !k_cache || !v_cache || !workspace || num_seqs < 1 || num_layers < 1 ||
      num_layers > kMaxLayers || max_seq_len < 1 || max_context < 1 || max_context > max_seq_len ||
      !(attn_scale > 0.f))
    return QMK_ERR_ARG;
  const long long kv_per_seq = (long long)num_layers * batch::kNKV * max_seq_len * batch::kD;
  if (num_seqs > 1 && (seq_stride < kv_per_seq || seq_stride % 8 != 0)) return QMK_ERR_ARG;
  for (const void* q : {embed_weight, final_norm_weight, lm_head_weight, cos_table, sin_table, (const void*)k_cache,
                        (const void*)v_cache, (const void*)workspace})
    if (!aligned16(q)) return QMK_ERR_ARG;
  for (int L = 0; L < num_layers; L++) {
    const LDGLayerWeights& w = layer_weights_host[L];
    const void* p[11] = {w.input_layernorm_weight, w.q_proj_weight, w.k_proj_weight, w.v_proj_weight,
                         w.q_norm_weight, w.k_norm_weight, w.o_proj_weight, w.post_attn_layernorm_weight,
                         w.gate_proj_weight, w.up_proj_weight, w.down_proj_weight};
    for (const void* q : p)
      if (!q || !aligned16(q)) return QMK_ERR_ARG;
  }
  if (workspace_bytes < qmk_forward_workspace_bytes(model, num_tokens, num_emit, max_context)) return QMK_ERR_ARG;
  batch::Args a{};
  a.T = num_tokens;
  a.R = num_emit;
  a.num_seqs = num_seqs;
  a.max_context = max_context;
  a.tokens = tokens;
  a.seqs = seq_ids;
  a.pos = positions;
  a.emit = emit_rows;
  a.out_tokens = out_tokens;
  a.logits = logits_out;
  a.embed = static_cast<const uint16_t*>(embed_weight);
  a.final_norm = static_cast<const uint16_t*>(final_norm_weight);
  a.lm_head = static_cast<const uint16_t*>(lm_head_weight);
  a.cos_t = static_cast<const uint16_t*>(cos_table);
  a.sin_t = static_cast<const uint16_t*>(sin_table);
  a.layers = layer_weights_host;
  a.cache = batch::Cache{static_cast<uint16_t*>(k_cache), static_cast<uint16_t*>(v_cache),
                         num_seqs > 1 ? seq_stride : 0, max_seq_len};
  a.num_layers = num_layers;
  a.attn_scale = attn_scale;
  a.ws = static_cast<char*>(workspace);
  return model == QMK_MODEL_QWEN3_1_7B ? batch::forward<Qwen3_1_7B>(a, stream) : batch::forward<Qwen3_0_6B>(a, stream);
}

size_t qmk_decode_batch_workspace_bytes(int model, int batch, int max_context) {
  if (batch < 1 || batch > batch::kMaxEmit || max_context < 1) return 0;
  if (model == QMK_MODEL_QWEN3_1_7B) return batch::layout<Qwen3_1_7B>(batch, batch, max_context, true).total;
  if (model == QMK_MODEL_QWEN3_0_6B) return batch::layout<Qwen3_0_6B>(batch, batch, max_context, true).total;
  return 0;
}

int qmk_decode_batch(int model, int batch, const int* tokens, const int* positions, int* out_tokens,
                     float* logits_out, const void* embed_weight, const LDGLayerWeights* layer_weights_host,
                     const void* final_norm_weight, const void* lm_head_weight, const void* cos_table,
                     const void* sin_table, void* k_cache, void* v_cache, long long seq_stride, int num_layers,
                     int max_seq_len, int max_context, float attn_scale, void* workspace, size_t workspace_bytes,
                     hipStream_t stream) {
  if (model != QMK_MODEL_QWEN3_0_6B && model != QMK_MODEL_QWEN3_1_7B) return QMK_ERR_ARG;
  if (batch < 1 || batch > batch::kMaxEmit || !tokens || !positions || !out_tokens || !embed_weight ||
      !layer_weights_host || !final_norm_weight || !lm_head_weight || !cos_table || !sin_table || !k_cache ||
      !v_cache || !workspace || num_layers < 1 || num_layers > kMaxLayers || max_seq_len < 1 || max_context < 1 ||
      max_context > max_seq_len || !(attn_scale > 0.f))
    return QMK_ERR_ARG;
  const long long kv_per_seq = (long long)num_layers * batch::kNKV * max_seq_len * batch::kD;
  if (batch > 1 && (seq_stride < kv_per_seq || seq_stride % 8 != 0)) return QMK_ERR_ARG;
  for (const void* q : {embed_weight, final_norm_weight, lm_head_weight, cos_table, sin_table, (const void*)k_cache,
                        (const void*)v_cache, (const void*)workspace})
    if (!aligned16(q)) return QMK_ERR_ARG;
  for (int L = 0; L < num_layers; L++) {
    const LDGLayerWeights& w = layer_weights_host[L];
    const void* p[11] = {w.input_layernorm_weight, w.q_proj_weight, w.k_proj_weight, w.v_proj_weight,
                         w.q_norm_weight, w.k_norm_weight, w.o_proj_weight, w.post_attn_layernorm_weight,
                         w.gate_proj_weight, w.up_proj_weight, w.down_proj_weight};
    for (const void* q : p)
      if (!q || !aligned16(q)) return QMK_ERR_ARG;
  }
  // The persistent kernel writes out_tokens (-1) before every workgroup has read tokens and
  // positions, so a call whose out_tokens overlaps them takes the multi-launch path, which reads
  // them first.
  const auto overlaps = [&](const void* p) {
    const char* a = static_cast<const char*>(p);
    const char* o = reinterpret_cast<const char*>(out_tokens);
    return a < o + batch * sizeof(int) && o < a + batch * sizeof(int);
  };
  if (qmk_batch_persistent_enabled() && batch >= kBatchMin && batch <= kBatchMax && max_context <= kBatchMaxContext &&
      !overlaps(tokens) && !overlaps(positions)) {
    const int s = qmk_decode_batch_persistent(model, batch, tokens, positions, out_tokens, logits_out, embed_weight,
                                              layer_weights_host, final_norm_weight, lm_head_weight, cos_table,
                                              sin_table, k_cache, v_cache, seq_stride, num_layers, max_seq_len,
                                              max_context, attn_scale, stream);
    if (s != QMK_ERR_DEVICE) return s;
  }
  if (workspace_bytes < qmk_decode_batch_workspace_bytes(model, batch, max_context)) return QMK_ERR_ARG;
  batch::Args a{};
  a.T = batch;
  a.R = batch;
  a.num_seqs = batch;
  a.max_context = max_context;
  a.one_per_seq = true;
  a.tokens = tokens;
  a.seqs = nullptr;
  a.pos = positions;
  a.emit = nullptr;
  a.out_tokens = out_tokens;
  a.logits = logits_out;
  a.embed = static_cast<const uint16_t*>(embed_weight);
  a.final_norm = static_cast<const uint16_t*>(final_norm_weight);
  a.lm_head = static_cast<const uint16_t*>(lm_head_weight);
  a.cos_t = static_cast<const uint16_t*>(cos_table);
  a.sin_t = static_cast<const uint16_t*>(sin_table);
  a.layers = layer_weights_host;
  a.cache = batch::Cache{static_cast<uint16_t*>(k_cache), static_cast<uint16_t*>(v_cache), batch > 1 ? seq_stride : 0,
                         max_seq_len};
  a.num_layers = num_layers;
  a.attn_scale = attn_scale;
  a.ws = static_cast<char*>(workspace);
  return model == QMK_MODEL_QWEN3_1_7B ? batch::forward<Qwen3_1_7B>(a, stream) : batch::forward<Qwen3_0_6B>(a, stream);
}

int qmk_selftest_mfma(const void* a, const void* b, float* c, hipStream_t stream) {
  if (!a || !b || !c) return QMK_ERR_ARG;
  hipLaunchKernelGGL(batch::mfma_selftest, dim3(1), dim3(64), 0, stream, static_cast<const uint16_t*>(a),
                     static_cast<const uint16_t*>(b), c);
  return hipGetLastError() == hipSuccess ? QMK_OK : QMK_ERR_HIP;
}

}  // extern "C"
