// Block e4m3 quantizer of the attention's upstream gradient dO, the input
// contract of the full-FP8 attention backward
// (ops/flydsl/hstu_do_fp8.py:16-38 the contract, :42-86 the kernel,
// :95-121 the wrapper quantize_do_e4m3_blk).
//
// One power-of-two scale per (sequence, head, token group).  The groups are
// the MX K-block groups of the backward's token-contracting MFMAs: inside
// each 64-token tile of a sequence, tokens p with p % 16 in [0, 8) form one
// group and [8, 16) the other (32 tokens each).  Per group
//   e = floor(log2(448 / amax)) from the fp32 bits of amax, clamped to
//       [-60, 60]; 60 for a subnormal amax, 0 for an all-zero group;
//   dO8 = e4m3(dO * 2^e),  E8[token, head] = 127 - e (the E8M0 byte of 2^-e).
// HBM-bound: 2 bytes read, 1 written per element.  A block takes one 64-token
// tile of one sequence (all heads); each thread holds its 8-element pieces of
// the tile in registers between the max and the conversion.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "hstu_common.h"
#include "hstu_mi355x.h"

using namespace hstu;

namespace {

constexpr int kTile = 64;  // tokens per block

// floor(log2(448 / a)) for a normal fp32 a > 0: a = 1.f * 2^E', and
// 448 / a = (1.75 / 1.f) * 2^(8 - E'), so e = 8 - E' when 1.f <= 1.75
// (mantissa bits <= 0x600000) and 7 - E' otherwise; then a * 2^e lies in
// (224, 448].  The fp32 bits give it exactly (a float log2 is off by one at
// powers of two).
__device__ __forceinline__ int group_exp(float a) {
  const uint32_t bits = __builtin_bit_cast(uint32_t, a);
  const int E = (int)((bits >> 23) & 0xffu);
  int e = (bits & 0x7fffffu) <= 0x600000u ? 135 - E : 134 - E;
  e = min(max(e, -60), 60);
  if (E == 0) e = 60;  // subnormal amax
  return a == 0.f ? 0 : e;
}

// max over the G (8 or 16) consecutive lanes of a 16-lane DPP row
template <int G>
__device__ __forceinline__ float group_max(float v) {
  auto mx = [](float x, float y) { return __builtin_fmaxf(x, y); };
  v = mx(v, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0xB1, 0xf, 0xf, false)));
  v = mx(v, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x4E, 0xf, 0xf, false)));
  v = mx(v, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x141, 0xf, 0xf, false)));
  if constexpr (G == 16)
    v = mx(v, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x140, 0xf, 0xf, false)));
  return v;
}

// HD = H * D elements per token row (128 .. 512), D = 64 or 128; F32 input
// rows are fp32, else bf16.  A tile is 64 tokens (p0 .. p0 + 63 of the
// sequence at st, length L) by HT heads (h0 .. h0 + HT - 1), for a 256-thread
// block.  8-element pieces: PPR per token row of the tile, each thread owns
// piece column c = tid % PPR (so one head) of tokens tid / PPR + i * 256 / PPR;
// amax_lds: the block's [HT][2] group maxima.
template <int HD, int D, int HT, bool F32>
__device__ __forceinline__ void do_tile(const uint8_t* __restrict__ x, int64_t x_rs, int64_t st, int L, int p0,
                                        int h0, uint8_t* __restrict__ y, uint8_t* __restrict__ e8,
                                        uint32_t (&amax_lds)[HT][2]) {
  constexpr int H = HD / D, PPR = HT * D / 8, TPI = 256 / PPR, NP = kTile / TPI, LPH = D / 8;
  constexpr int ES = F32 ? 4 : 2;
  static_assert(256 % PPR == 0 && kTile % TPI == 0 && (LPH == 8 || LPH == 16), "piece layout");
  const int tid = threadIdx.x;
  if (tid < 2 * HT) amax_lds[tid >> 1][tid & 1] = 0u;
  const int c = tid % PPR, tok0 = tid / PPR, h = c / LPH;
  // all loads first; rows past the sequence are zero (they take no part in the max)
  constexpr int KW = F32 ? 2 : 1;  // 16-byte loads per piece
  u32x4 raw[NP * KW];
#pragma unroll
  for (int i = 0; i < NP; ++i) {
    const int tok = tok0 + i * TPI;
    const uint8_t* src = x + ((st + p0 + tok) * x_rs + (int64_t)h0 * D + (int64_t)c * 8) * ES;
    const bool ok = p0 + tok < L;
#pragma unroll
    for (int k = 0; k < KW; ++k) raw[i * KW + k] = ok ? *(const u32x4*)(src + 16 * k) : u32x4{0u, 0u, 0u, 0u};
  }
  // element e (0..7) of piece i, fp32
  auto elem = [&](int i, int e) -> float {
    if constexpr (F32) {
      // through a scalar: a bit_cast of an ext-vector element lvalue reads element 0
      const uint32_t u = raw[i * 2 + e / 4][e % 4];
      return __builtin_bit_cast(float, u);
    } else {
      const uint32_t w = raw[i][e / 2];
      return __builtin_bit_cast(float, (e % 2) ? (w & 0xffff0000u) : (w << 16));
    }
  };
  float a0 = 0.f, a1 = 0.f;  // per-lane max |x| of group 0 / 1 tokens
#pragma unroll
  for (int i = 0; i < NP; ++i) {
    const int tok = tok0 + i * TPI;
    float m = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) m = __builtin_fmaxf(m, __builtin_fabsf(elem(i, e)));
    if ((tok & 15) < 8) a0 = __builtin_fmaxf(a0, m);
    else a1 = __builtin_fmaxf(a1, m);
  }
  a0 = group_max<LPH>(a0);
  a1 = group_max<LPH>(a1);
  __syncthreads();  // the amax slots are zeroed
  if (c % LPH == 0) {
    // non-negative floats order as their bit patterns
    atomicMax(&amax_lds[h][0], __builtin_bit_cast(uint32_t, a0));
    atomicMax(&amax_lds[h][1], __builtin_bit_cast(uint32_t, a1));
  }
  __syncthreads();
  const int e0 = group_exp(__builtin_bit_cast(float, amax_lds[h][0]));
  const int e1 = group_exp(__builtin_bit_cast(float, amax_lds[h][1]));
  // 2^e exactly, from the exponent field
  const float s0 = __builtin_bit_cast(float, (uint32_t)(e0 + 127) << 23);
  const float s1 = __builtin_bit_cast(float, (uint32_t)(e1 + 127) << 23);
#pragma unroll
  for (int i = 0; i < NP; ++i) {
    const int tok = tok0 + i * TPI;
    if (p0 + tok >= L) continue;
    const float s = (tok & 15) < 8 ? s0 : s1;
    float f[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) f[e] = __builtin_fminf(__builtin_fmaxf(elem(i, e) * s, -448.f), 448.f);
    int lo = __builtin_amdgcn_cvt_pk_fp8_f32(f[0], f[1], 0, false);
    lo = __builtin_amdgcn_cvt_pk_fp8_f32(f[2], f[3], lo, true);
    int hi = __builtin_amdgcn_cvt_pk_fp8_f32(f[4], f[5], 0, false);
    hi = __builtin_amdgcn_cvt_pk_fp8_f32(f[6], f[7], hi, true);
    *(u32x2*)(y + (st + p0 + tok) * HD + h0 * D + c * 8) = u32x2{(uint32_t)lo, (uint32_t)hi};
  }
  // E8 bytes: one per (token, head) of the tile
  for (int k = tid; k < kTile * HT; k += 256) {
    const int tok = k / HT, hh = k - tok * HT;
    if (p0 + tok >= L) continue;
    const float a = __builtin_bit_cast(float, amax_lds[hh][(tok & 15) < 8 ? 0 : 1]);
    e8[(st + p0 + tok) * H + h0 + hh] = (uint8_t)(127 - group_exp(a));
  }
}

// Block (b, t) of the B x ntiles grid: tile t of sequence b, if it has tokens.
template <int HD, int D, bool F32>
__global__ void __launch_bounds__(256) do_blk_kernel(const uint8_t* __restrict__ x, int64_t x_rs,
                                                      const int64_t* __restrict__ seq_offsets, int ntiles,
                                                      uint8_t* __restrict__ y, uint8_t* __restrict__ e8) {
  __shared__ uint32_t amax_lds[HD / D][2];
  const int b = blockIdx.x / ntiles, t = blockIdx.x - b * ntiles;
  const int64_t st = seq_offsets[b];
  const int L = (int)(seq_offsets[b + 1] - st);
  if (t * kTile >= L) return;
  do_tile<HD, D, HD / D, F32>(x, x_rs, st, L, t * kTile, 0, y, e8, amax_lds);
}

// The same token tiles, only those that hold tokens, split by head and walked
// by a persistent grid: each block first builds the tile prefix of the
// sequences in LDS (tiles of sequence b = ceil(min(L_b, 64 ntiles) / 64)),
// then takes (tile, head) items blockIdx.x, blockIdx.x + gridDim.x, ... (the
// H heads of a token tile are consecutive items), finding each tile's
// sequence by binary search.  Blocks therefore start their next item's loads
// while others still store, no block is spent on the padding of short
// sequences, and items of one head (16 KiB of bf16 at D = 128) balance the
// grid's last round better than whole token tiles.  B <= kPersistMaxB.
constexpr int kPersistMaxB = 4096;
template <int HD, int D, bool F32>
__global__ void __launch_bounds__(256) do_blk_persistent(const uint8_t* __restrict__ x, int64_t x_rs,
                                                          const int64_t* __restrict__ seq_offsets, int B,
                                                          int ntiles, uint8_t* __restrict__ y,
                                                          uint8_t* __restrict__ e8) {
  constexpr int H = HD / D;
  __shared__ uint32_t amax_lds[1][2];
  __shared__ int pre[kPersistMaxB + 1];
  __shared__ int part[256];
  const int tid = threadIdx.x;
  const int64_t cap = (int64_t)ntiles * kTile;
  auto tiles = [&](int b) {
    const int64_t L = min(seq_offsets[b + 1] - seq_offsets[b], cap);
    return (int)((max(L, (int64_t)0) + kTile - 1) / kTile);
  };
  // exclusive prefix: thread tid sums sequences [tid per, tid per + per)
  const int per = (B + 255) / 256, b0 = tid * per;
  int sum = 0;
  for (int i = 0; i < per; ++i)
    if (b0 + i < B) sum += tiles(b0 + i);
  part[tid] = sum;
  __syncthreads();
  for (int off = 1; off < 256; off <<= 1) {
    const int add = tid >= off ? part[tid - off] : 0;
    __syncthreads();
    part[tid] += add;
    __syncthreads();
  }
  int run = tid ? part[tid - 1] : 0;
  for (int i = 0; i < per; ++i) {
    if (b0 + i < B) {
      pre[b0 + i] = run;
      run += tiles(b0 + i);
    }
  }
  if (tid == 255) pre[B] = part[255];
  __syncthreads();
  const int total = pre[B] * H;
  for (int item = blockIdx.x; item < total; item += gridDim.x) {
    const int tile = item / H, hh = item - tile * H;
    // the last b with pre[b] <= tile (sequences without tiles share their
    // successor's prefix and are skipped by taking the last)
    int lo = 0, hi = B - 1;
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (pre[mid] <= tile) lo = mid;
      else hi = mid - 1;
    }
    const int64_t st = seq_offsets[lo];
    const int L = (int)(seq_offsets[lo + 1] - st);
    do_tile<HD, D, 1, F32>(x, x_rs, st, L, (tile - pre[lo]) * kTile, hh, y, e8, amax_lds);
    __syncthreads();  // the tile's E8 reads of amax_lds are done before the next tile resets it
  }
}

// Persistent grid: sixteen blocks per CU (measured at config 3: 47.9 us
// against 53 us with 2048 blocks and 49.2 us with 8192), never more than the
// B x ntiles x H items there can be.
constexpr int kPersistBlocks = 4096;
template <int HD, int D>
void launch_blk(bool f32, int B, int ntiles, const void* x, int64_t rs, const int64_t* offs, void* y, void* e8,
                hipStream_t s) {
  const int64_t all = (int64_t)B * ntiles;
  if (B <= kPersistMaxB) {
    const int grid = (int)std::min<int64_t>(all * (HD / D), kPersistBlocks);
    if (f32)
      hipLaunchKernelGGL((do_blk_persistent<HD, D, true>), dim3(grid), dim3(256), 0, s, (const uint8_t*)x, rs, offs,
                         B, ntiles, (uint8_t*)y, (uint8_t*)e8);
    else
      hipLaunchKernelGGL((do_blk_persistent<HD, D, false>), dim3(grid), dim3(256), 0, s, (const uint8_t*)x, rs, offs,
                         B, ntiles, (uint8_t*)y, (uint8_t*)e8);
    return;
  }
  if (f32)
    hipLaunchKernelGGL((do_blk_kernel<HD, D, true>), dim3((unsigned)all), dim3(256), 0, s, (const uint8_t*)x, rs, offs,
                       ntiles, (uint8_t*)y, (uint8_t*)e8);
  else
    hipLaunchKernelGGL((do_blk_kernel<HD, D, false>), dim3((unsigned)all), dim3(256), 0, s, (const uint8_t*)x, rs,
                       offs, ntiles, (uint8_t*)y, (uint8_t*)e8);
}

// dO8 * 2^(E8 - 127) -> bf16, 8 elements of one (token, head) per thread.
// Exact: an e4m3 value (3 mantissa bits) times 2^-e, |e| <= 60, is a bf16.
__global__ void __launch_bounds__(256) do_dequant_kernel(const uint8_t* __restrict__ y,
                                                         const uint8_t* __restrict__ e8, int64_t chunks, int H,
                                                         int D, uint16_t* __restrict__ out, int64_t out_rs) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= chunks) return;
  const int cpr = H * D / 8;                  // 8-element chunks per token row
  const int64_t t = i / cpr;
  const int c = (int)(i - t * cpr), h = c * 8 / D;
  const u32x2 w = *(const u32x2*)(y + (t * H * D + (int64_t)c * 8));
  const float s = __builtin_bit_cast(float, (uint32_t)e8[t * H + h] << 23);  // 2^(E8 - 127)
  uint32_t o[4];
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const f32x2 lo = __builtin_amdgcn_cvt_pk_f32_fp8((int)w[k], false);
    const f32x2 hi = __builtin_amdgcn_cvt_pk_f32_fp8((int)w[k], true);
    o[2 * k] = pack_bf16(lo[0] * s, lo[1] * s);
    o[2 * k + 1] = pack_bf16(hi[0] * s, hi[1] * s);
  }
  *(u32x4*)(out + t * out_rs + (int64_t)c * 8) = u32x4{o[0], o[1], o[2], o[3]};
}

}  // namespace

extern "C" int hstu_dequantize_do_e4m3_blk(const void* dout_e4m3, const void* e8, int64_t T, int H, int D,
                                           void* out, int64_t out_row_stride, hipStream_t stream) {
  if (T < 0 || H <= 0 || D <= 0 || (T > 0 && (!dout_e4m3 || !e8 || !out)) || out_row_stride < (int64_t)H * D)
    return HSTU_E_BAD_ARG;
  if (D % 8 || (uintptr_t)dout_e4m3 % 8 || (uintptr_t)out % 16 || out_row_stride % 8) return HSTU_E_UNSUPPORTED;
  const int64_t chunks = T * (int64_t)H * D / 8;
  if (chunks == 0) return 0;
  if ((chunks + 255) / 256 >= ((int64_t)1 << 31)) return HSTU_E_UNSUPPORTED;
  hipLaunchKernelGGL(do_dequant_kernel, dim3((unsigned)((chunks + 255) / 256)), dim3(256), 0, stream,
                     (const uint8_t*)dout_e4m3, (const uint8_t*)e8, chunks, H, D, (uint16_t*)out, out_row_stride);
  return (int)hipGetLastError();
}

extern "C" int hstu_quantize_do_e4m3_blk(int dtype, const void* dout, int64_t dout_row_stride,
                                         const int64_t* seq_offsets, int B, int H, int D, int max_seq_len,
                                         void* dout_e4m3, void* e8, hipStream_t stream) {
  if (dtype != HSTU_DTYPE_BF16 && dtype != HSTU_DTYPE_FP32) return HSTU_E_BAD_ARG;
  if (B < 0 || H <= 0 || D <= 0 || max_seq_len <= 0 || dout == nullptr || seq_offsets == nullptr ||
      dout_e4m3 == nullptr || e8 == nullptr || dout_row_stride < (int64_t)H * D)
    return HSTU_E_BAD_ARG;
  const int HD = H * D;
  if ((D != 64 && D != 128) || (HD != 128 && HD != 256 && HD != 512)) return HSTU_E_UNSUPPORTED;
  const int es = dtype == HSTU_DTYPE_FP32 ? 4 : 2;
  if ((uintptr_t)dout % 16 || (dout_row_stride * es) % 16 || (uintptr_t)dout_e4m3 % 8) return HSTU_E_UNSUPPORTED;
  if (B == 0) return 0;
  const int ntiles = (max_seq_len + kTile - 1) / kTile;
  if ((int64_t)B * ntiles >= (int64_t)1 << 31) return HSTU_E_UNSUPPORTED;
  const bool f32 = dtype == HSTU_DTYPE_FP32;
  if (D == 128 && HD == 512) launch_blk<512, 128>(f32, B, ntiles, dout, dout_row_stride, seq_offsets, dout_e4m3, e8, stream);
  else if (D == 128 && HD == 256) launch_blk<256, 128>(f32, B, ntiles, dout, dout_row_stride, seq_offsets, dout_e4m3, e8, stream);
  else if (D == 128) launch_blk<128, 128>(f32, B, ntiles, dout, dout_row_stride, seq_offsets, dout_e4m3, e8, stream);
  else if (HD == 512) launch_blk<512, 64>(f32, B, ntiles, dout, dout_row_stride, seq_offsets, dout_e4m3, e8, stream);
  else if (HD == 256) launch_blk<256, 64>(f32, B, ntiles, dout, dout_row_stride, seq_offsets, dout_e4m3, e8, stream);
  else launch_blk<128, 64>(f32, B, ntiles, dout, dout_row_stride, seq_offsets, dout_e4m3, e8, stream);
  return (int)hipGetLastError();
}
