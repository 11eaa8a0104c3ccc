// Row-wise LayerNorm kernels around the HSTU attention (gfx950):
//   * the output block's LN * U * dropout with the [u | x | y] concat
//     (ops/pytorch/pt_hstu_linear.py:23-82; the separated-mask Triton path,
//     ops/triton/triton_hstu_linear.py:529-700 forward, :1566-1760 backward);
//   * its dropout mask: Philox4x32-10 keep bits packed one bit per
//     concatenated block (triton_hstu_linear.py:331-375, 428-470, 2542-2600);
//   * the weighted LayerNorm with e4m3 output that feeds the UVQK GEMM
//     (ops/triton/triton_layer_norm.py:1668-1740; the same kernel without u).
// Every kernel reads and writes each row once: HBM-bound.  A wave owns a row
// (D / 64 consecutive elements per lane: one 16-byte bf16 access per lane for
// D = 512); mean and variance are exact two-pass sums over the wave.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <mutex>
#include <type_traits>

#include "hstu_common.h"
#include "hstu_mi355x.h"

using namespace hstu;

namespace {

enum Act { kActNone = 0, kActSilu = 1, kActSigmoid = 2 };

constexpr int kFwdRows = 8;       // rows per forward block: one mask16 Philox group
// Backward grid: rows are strided over the waves.  With u (the output block,
// ~11 KB of traffic per row) one block per CU measured best; the plain
// LayerNorm backward (6 KB per row, fewer registers) needs 4 per CU to cover
// the memory latency.
constexpr int kBwdBlocksU = 256, kBwdBlocksMax = 1024;

// ------------------------------------------------------------------ Philox
// Philox4x32-10 (Salmon, Moraes, Dror, Shaw, SC'11) on counter (c0, 0, 0, 0)
// and key (k0, k1): Triton's tl.randint4x(seed, offset) with k = seed's low and
// high words.  Integer only, so the bits are exact.
__device__ __forceinline__ void philox4x32_10(uint32_t c0, uint32_t k0, uint32_t k1, uint32_t (&r)[4]) {
  uint32_t c1 = 0, c2 = 0, c3 = 0;
#pragma unroll
  for (int i = 0; i < 10; ++i) {
    const uint64_t pa = (uint64_t)c0 * 0xD2511F53u;
    const uint64_t pb = (uint64_t)c2 * 0xCD9E8D57u;
    // three-input xors in one v_bitop3 each (truth table 0x96 = a ^ b ^ c)
    const uint32_t n0 = __builtin_amdgcn_bitop3_b32((uint32_t)(pb >> 32), c1, k0, 0x96);
    const uint32_t n2 = __builtin_amdgcn_bitop3_b32((uint32_t)(pa >> 32), c3, k1, 0x96);
    c1 = (uint32_t)pb;
    c3 = (uint32_t)pa;
    c0 = n0;
    c2 = n2;
    k0 += 0x9E3779B9u;
    k1 += 0xBB67AE85u;
  }
  r[0] = c0;
  r[1] = c1;
  r[2] = c2;
  r[3] = c3;
}

struct MaskSpec {
  int num_masks;  // 1 + concat_u + concat_x: bit 0 = y, then x, then u
  int mask16;     // 1: one decision per 16-bit half (8 rows per Philox group)
  int thr;        // mask16: smallest kept half; else largest dropped x ^ (x >> 31)
  int block_d;    // Philox offset stride per mask (next power of two of D)
  uint32_t k0, k1;
};

// Keep bits of rows 8g .. 8g+7 at column col.
//   mask16: one group of 8 rows; word i's low half decides row i, its high
//           half row i + 4 (triton_hstu_linear.py:428-470);
//   else:   two groups of 4 rows (4g .. 4g+3 from group 2g, the next four from
//           group 2g + 1), word i decides row i of its group (:331-375).
// Counter of mask j in group p: p * num_masks * block_d + j * block_d + col
// (32-bit wrap, like the reference's int32 arithmetic).
__device__ __forceinline__ void mask_bits8(const MaskSpec& m, uint32_t g, int col, uint32_t (&bits)[8]) {
#pragma unroll
  for (int r = 0; r < 8; ++r) bits[r] = 0;
  const uint32_t stride = (uint32_t)(m.num_masks * m.block_d);
  if (m.mask16) {
    for (int j = 0; j < m.num_masks; ++j) {
      uint32_t w[4];
      philox4x32_10(g * stride + (uint32_t)(j * m.block_d + col), m.k0, m.k1, w);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        bits[i] |= ((int)(w[i] & 0xffffu) >= m.thr ? 1u : 0u) << j;
        bits[i + 4] |= ((int)(w[i] >> 16) >= m.thr ? 1u : 0u) << j;
      }
    }
  } else {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      for (int j = 0; j < m.num_masks; ++j) {
        uint32_t w[4];
        philox4x32_10((2 * g + h) * stride + (uint32_t)(j * m.block_d + col), m.k0, m.k1, w);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int x = (int)w[i];
          bits[4 * h + i] |= ((x ^ (x >> 31)) > m.thr ? 1u : 0u) << j;
        }
      }
    }
  }
}

// ------------------------------------------------------------------ helpers
// v + DPP-moved v (lanes the control leaves unwritten add 0)
template <int CTRL, int ROW_MASK = 0xf, int BANK_MASK = 0xf>
__device__ __forceinline__ float dpp_add(float v) {
  const int m = __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, ROW_MASK, BANK_MASK, true);
  return v + __builtin_bit_cast(float, m);
}
// Sum over the wave, returned as a wave-uniform (scalar) value: prefix sums
// inside each 16-lane row (row_shr 1, 2, 4, 8), then the row totals carried
// by row_bcast 15 / 31; lane 63 ends with the total.
__device__ __forceinline__ float wave_sum(float v) {
  v = dpp_add<0x111>(v);
  v = dpp_add<0x112>(v);
  v = dpp_add<0x114>(v);
  v = dpp_add<0x118>(v);
  v = dpp_add<0x142, 0xa>(v);
  v = dpp_add<0x143, 0xc>(v);
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}
__device__ __forceinline__ float sigmoidf(float x) {
  return __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(-kLog2e * x));
}
__device__ __forceinline__ float bf16f(uint32_t b16) { return __builtin_bit_cast(float, b16 << 16); }

// EPT consecutive bf16 (EPT = 4 or 8: one 8- or 16-byte access), loaded raw
// and unpacked separately so that a load can be issued well before its use.
template <int EPT>
using RawT = typename std::conditional<EPT == 8, u32x4, u32x2>::type;
template <int EPT>
using MaskRawT = typename std::conditional<EPT == 8, u32x2, uint32_t __attribute__((ext_vector_type(1)))>::type;
template <int EPT>
__device__ __forceinline__ RawT<EPT> load_raw(const uint16_t* src) {
  return *(const RawT<EPT>*)src;
}
template <int EPT>
__device__ __forceinline__ void unpack_bf16(const RawT<EPT>& w, float (&v)[EPT]) {
#pragma unroll
  for (int i = 0; i < EPT / 2; ++i) {
    v[2 * i] = bf16f(w[i] & 0xffffu);
    v[2 * i + 1] = bf16f(w[i] >> 16);
  }
}
template <int EPT>
__device__ __forceinline__ void load_bf16(const uint16_t* src, float (&v)[EPT]) {
  unpack_bf16<EPT>(load_raw<EPT>(src), v);
}
template <int EPT>
__device__ __forceinline__ void store_bf16(uint16_t* dst, const float (&v)[EPT]) {
  if constexpr (EPT == 8)
    *(u32x4*)dst = u32x4{pack_bf16(v[0], v[1]), pack_bf16(v[2], v[3]), pack_bf16(v[4], v[5]), pack_bf16(v[6], v[7])};
  else
    *(u32x2*)dst = u32x2{pack_bf16(v[0], v[1]), pack_bf16(v[2], v[3])};
}
// e4m3(clamp(v * inv, +-448)), round to nearest even
template <int EPT>
__device__ __forceinline__ void store_e4m3(uint8_t* dst, const float (&v)[EPT], float inv) {
  uint32_t w[EPT / 4];
#pragma unroll
  for (int i = 0; i < EPT / 4; ++i) {
    float c[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) c[r] = __builtin_fminf(__builtin_fmaxf(v[4 * i + r] * inv, -448.f), 448.f);
    int x = __builtin_amdgcn_cvt_pk_fp8_f32(c[0], c[1], 0, false);
    x = __builtin_amdgcn_cvt_pk_fp8_f32(c[2], c[3], x, true);
    w[i] = (uint32_t)x;
  }
  if constexpr (EPT == 8) *(u32x2*)dst = u32x2{w[0], w[1]};
  else *(uint32_t*)dst = w[0];
}
template <int EPT>
__device__ __forceinline__ void load_bytes(const uint8_t* src, uint32_t (&b)[EPT]) {
  uint32_t w[EPT / 4];
  if constexpr (EPT == 8) {
    const u32x2 v = *(const u32x2*)src;
    w[0] = v[0];
    w[1] = v[1];
  } else {
    w[0] = *(const uint32_t*)src;
  }
#pragma unroll
  for (int i = 0; i < EPT; ++i) b[i] = (w[i / 4] >> (8 * (i % 4))) & 0xffu;
}
template <int EPT>
__device__ __forceinline__ void store_bytes(uint8_t* dst, const uint32_t (&b)[EPT]) {
  uint32_t w[EPT / 4] = {};
#pragma unroll
  for (int i = 0; i < EPT; ++i) w[i / 4] |= b[i] << (8 * (i % 4));
  if constexpr (EPT == 8) *(u32x2*)dst = u32x2{w[0], w[1]};
  else *(uint32_t*)dst = w[0];
}

// ------------------------------------------------------------------ forward
// Element i of a LayerNorm parameter vector, fp32 or bf16 (converted exactly).
__device__ __forceinline__ float ln_param(const void* v, int i, int bf16) {
  return bf16 ? __builtin_bit_cast(float, (uint32_t)((const uint16_t*)v)[i] << 16) : ((const float*)v)[i];
}
// A lane's EPT consecutive weight and bias values from column c0, fp32 or
// bf16 (a kernel-uniform branch; vector loads, 16-byte aligned vectors).
template <int EPT>
__device__ __forceinline__ void ln_params(const void* w, const void* b, int bf16, int c0, float (&wv)[EPT],
                                          float (&bv)[EPT]) {
  static_assert(EPT == 4 || EPT == 8, "4 or 8 columns a lane");
  if (bf16) {
    uint32_t x[EPT / 2], y[EPT / 2];
    if constexpr (EPT == 8) {
      const u32x4 p = *(const u32x4*)((const uint16_t*)w + c0), q = *(const u32x4*)((const uint16_t*)b + c0);
#pragma unroll
      for (int i = 0; i < 4; ++i) x[i] = p[i], y[i] = q[i];
    } else {
      const u32x2 p = *(const u32x2*)((const uint16_t*)w + c0), q = *(const u32x2*)((const uint16_t*)b + c0);
#pragma unroll
      for (int i = 0; i < 2; ++i) x[i] = p[i], y[i] = q[i];
    }
#pragma unroll
    for (int i = 0; i < EPT / 2; ++i) {
      wv[2 * i] = __builtin_bit_cast(float, x[i] << 16);
      wv[2 * i + 1] = __builtin_bit_cast(float, x[i] & 0xffff0000u);
      bv[2 * i] = __builtin_bit_cast(float, y[i] << 16);
      bv[2 * i + 1] = __builtin_bit_cast(float, y[i] & 0xffff0000u);
    }
  } else {
#pragma unroll
    for (int i = 0; i < EPT / 4; ++i) {
      const f32x4 p = *(const f32x4*)((const float*)w + c0 + 4 * i), q = *(const f32x4*)((const float*)b + c0 + 4 * i);
#pragma unroll
      for (int j = 0; j < 4; ++j) wv[4 * i + j] = p[j], bv[4 * i + j] = q[j];
    }
  }
}

struct FwdArgs {
  const uint16_t* x;
  int64_t ldx;
  const uint16_t* u;  // null: weighted LayerNorm only
  int64_t ldu;
  const void* w;  // LayerNorm weight and bias, fp32 or bf16 (w_bf16)
  const void* b;
  int w_bf16;
  float eps, inv_d;
  int rows;
  int silu_u, concat_u, concat_x;
  float drop_scale;  // fp32(1 / fp32(1 - ratio))
  MaskSpec ms;
  uint8_t* mask;
  int64_t ldm;
  void* y;
  int64_t ldy;
  float inv_scale;
  const float* out_scale;  // device scale (nullable): e4m3 output uses 1 / out_scale[0]
  float* mean;
  float* rstd;
};

constexpr int kNoU = 3;  // activation slot of the plain weighted LayerNorm

// 0x00 / 0xff per byte of a mask word (4 elements): keep bit `bit` of each.
__device__ __forceinline__ uint32_t byte_keep(uint32_t mw, uint32_t bit) {
  const uint32_t t = (mw >> (31 - __builtin_clz(bit))) & 0x01010101u;
  uint32_t t8 = t << 8;
  asm volatile("" : "+v"(t8));  // keeps t * 255 as shift and subtract (not a quarter-rate multiply)
  return t8 - t;
}

// One D-wide output block: e4m3(clamp(v * scale)) or bf16(v * scale), the
// dropped elements zeroed in the packed words (bytes of mask word `mw`).
template <int EPT, bool DROP, bool E4M3>
__device__ __forceinline__ void store_block(void* dst, const float (&v)[EPT], float scale, const uint32_t (&mw)[EPT / 4],
                                            uint32_t bit) {
  if constexpr (E4M3) {
    uint32_t w[EPT / 4];
#pragma unroll
    for (int q = 0; q < EPT / 4; ++q) {
      float c[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) c[r] = __builtin_amdgcn_fmed3f(v[4 * q + r] * scale, -448.f, 448.f);
      int x = __builtin_amdgcn_cvt_pk_fp8_f32(c[0], c[1], 0, false);
      x = __builtin_amdgcn_cvt_pk_fp8_f32(c[2], c[3], x, true);
      w[q] = (uint32_t)x;
      if constexpr (DROP) w[q] &= byte_keep(mw[q], bit);
    }
    if constexpr (EPT == 8) *(u32x2*)dst = u32x2{w[0], w[1]};
    else *(uint32_t*)dst = w[0];
  } else {
    uint32_t w[EPT / 2];
#pragma unroll
    for (int q = 0; q < EPT / 2; ++q) {
      w[q] = DROP ? pack_bf16(v[2 * q] * scale, v[2 * q + 1] * scale) : pack_bf16(v[2 * q], v[2 * q + 1]);
    }
    if constexpr (DROP) {
#pragma unroll
      for (int q = 0; q < EPT / 4; ++q) {
        const uint32_t bm = byte_keep(mw[q], bit);
        w[2 * q] &= __builtin_amdgcn_perm(bm, bm, 0x01010000u);      // bytes 0,0,1,1 -> two halves
        w[2 * q + 1] &= __builtin_amdgcn_perm(bm, bm, 0x03030202u);  // bytes 2,2,3,3
      }
    }
    if constexpr (EPT == 8) *(u32x4*)dst = u32x4{w[0], w[1], w[2], w[3]};
    else *(u32x2*)dst = u32x2{w[0], w[1]};
  }
}

// A block owns rows 8*blockIdx.x .. +7.  Its waves issue their two rows' loads
// first; with dropout the 256 threads then build the 8 rows' mask bytes in LDS
// (one Philox call per (mask, column) for mask16) while those loads are in
// flight; then wave w normalises rows w and w + 4.
// ACT: kActNone / kActSilu / kActSigmoid, or kNoU (no u: weighted LayerNorm).
template <int EPT, int ACT, bool DROP, bool E4M3>
__global__ void __launch_bounds__(kThreads) ln_mul_fwd_kernel(FwdArgs a) {
  constexpr int D = 64 * EPT;
  constexpr bool HU = ACT != kNoU;
  __shared__ __attribute__((aligned(16))) uint8_t lmask[DROP ? kFwdRows * D : 16];
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int c0 = lane * EPT;
  // rows past the end re-read the last row and store nothing
  RawT<EPT> xr[2], ur[2];
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const int64_t row = min((int64_t)blockIdx.x * kFwdRows + wave + 4 * k, (int64_t)a.rows - 1);
    xr[k] = load_raw<EPT>(a.x + row * a.ldx + c0);
    if constexpr (HU) ur[k] = load_raw<EPT>(a.u + row * a.ldu + c0);
  }
  float w[EPT], bb[EPT];
  ln_params<EPT>(a.w, a.b, a.w_bf16, c0, w, bb);
  if constexpr (DROP) {
    for (int col = threadIdx.x; col < D; col += kThreads) {
      uint32_t bits[8];
      mask_bits8(a.ms, blockIdx.x, col, bits);
#pragma unroll
      for (int r = 0; r < 8; ++r) lmask[r * D + col] = (uint8_t)bits[r];
    }
    __syncthreads();
  }
  const bool cu = HU && a.concat_u;
  const uint32_t bit_x = a.concat_x ? 2u : 0u, bit_u = cu ? (a.concat_x ? 4u : 2u) : 0u;
  float inv_scale = a.inv_scale;
  if (E4M3 && a.out_scale != nullptr) inv_scale = 1.0f / a.out_scale[0];
  const float scale = E4M3 ? (DROP ? a.drop_scale * inv_scale : inv_scale) : a.drop_scale;
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const int rl = wave + 4 * k;
    const int64_t row = (int64_t)blockIdx.x * kFwdRows + rl;
    if (row >= a.rows) break;
    float x[EPT], u[EPT];
    unpack_bf16<EPT>(xr[k], x);
    if constexpr (HU) unpack_bf16<EPT>(ur[k], u);
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < EPT; ++i) s += x[i];
    const float mean = wave_sum(s) * a.inv_d;
    float xm[EPT], q = 0.f;
#pragma unroll
    for (int i = 0; i < EPT; ++i) {
      xm[i] = x[i] - mean;
      q += xm[i] * xm[i];
    }
    const float rstd = __builtin_amdgcn_rsqf(wave_sum(q) * a.inv_d + a.eps);
    if (lane == 0) {
      a.mean[row] = mean;
      a.rstd[row] = rstd;
    }
    float z[EPT], uo[EPT];
#pragma unroll
    for (int i = 0; i < EPT; ++i) {
      z[i] = (xm[i] * rstd) * w[i] + bb[i];
      if constexpr (HU) {
        const float sg = sigmoidf(u[i]);
        const float silu = u[i] * sg;
        z[i] *= ACT == kActSilu ? silu : ACT == kActSigmoid ? sg : u[i];
        uo[i] = a.silu_u ? silu : u[i];
      }
    }
    uint32_t mw[EPT / 4];
    if constexpr (DROP) {
      const uint8_t* lm = lmask + rl * D + c0;
      if constexpr (EPT == 8) {
        const u32x2 t = *(const u32x2*)lm;
        mw[0] = t[0];
        mw[1] = t[1];
        *(u32x2*)(a.mask + row * a.ldm + c0) = t;
      } else {
        mw[0] = *(const uint32_t*)lm;
        *(uint32_t*)(a.mask + row * a.ldm + c0) = mw[0];
      }
    }
    uint8_t* yr = (uint8_t*)a.y + row * a.ldy * (E4M3 ? 1 : 2);
    constexpr int esz = E4M3 ? 1 : 2;
    int col = 0;
    if (cu) store_block<EPT, DROP, E4M3>(yr + ((col++) * D + c0) * esz, uo, scale, mw, bit_u);
    if (a.concat_x) store_block<EPT, DROP, E4M3>(yr + ((col++) * D + c0) * esz, x, scale, mw, bit_x);
    store_block<EPT, DROP, E4M3>(yr + (col * D + c0) * esz, z, scale, mw, 1u);
  }
}

// Standalone mask (the reference's _create_dropout_mask): 8 rows per block.
__global__ void __launch_bounds__(kThreads) dropout_mask_kernel(MaskSpec ms, int rows, int D, uint8_t* mask,
                                                                int64_t ldm) {
  for (int col = threadIdx.x; col < D; col += kThreads) {
    uint32_t bits[8];
    mask_bits8(ms, blockIdx.x, col, bits);
#pragma unroll
    for (int r = 0; r < 8; ++r) {
      const int64_t row = (int64_t)blockIdx.x * 8 + r;
      if (row < rows) mask[row * ldm + col] = (uint8_t)bits[r];
    }
  }
}

// ------------------------------------------------------------------ backward
struct BwdArgs {
  const uint16_t* dy;  // [rows, ncols * D], the forward's column order
  int64_t lddy;
  const uint16_t* x;
  int64_t ldx;
  const uint16_t* u;
  int64_t ldu;
  const void* w;  // LayerNorm weight and bias, fp32 or bf16 (w_bf16)
  const void* b;
  int w_bf16;
  const float* mean;
  const float* rstd;
  float inv_d;
  int rows;
  int silu_u, concat_u, concat_x;
  const uint8_t* mask;  // null: no dropout
  int64_t ldm;
  float drop_scale;
  uint16_t* dx;
  int64_t lddx;
  uint16_t* du;
  int64_t lddu;
  uint16_t* y;  // recomputed bf16 forward output (null: not wanted)
  int64_t ldy;
  const uint16_t* dres;  // bf16 gradient added to dx (null: none; never with concat_x)
  int64_t lddres;
  float* partial;  // [gridDim.x, 2, D]: per-block dweight, dbias sums
};

// v * s where bit `pos` of mask word mw is set, else +0 (sign-extended 1-bit
// field as an and-mask on the product's bits).
__device__ __forceinline__ float keep_scaled(float v, float s, uint32_t mw, uint32_t pos) {
  const uint32_t m = (uint32_t)__builtin_amdgcn_sbfe((int)mw, pos, 1);
  return __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, v * s) & m);
}

// Raw inputs of one row for a lane's EPT columns c0 .. c0 + EPT - 1.
template <int EPT>
struct LnBwdRowIn {
  RawT<EPT> x, gy, gx, gu, u;
  MaskRawT<EPT> m;
  float mean, rstd;
};

// The per-row backward of LN * U * dropout for a lane's EPT columns: du, the
// recomputed y (Y), dx, and the lane's dweight / dbias sums.  Shared by the
// standalone backward and the out-projection-fused one, so that both compute
// a row with the same operations in the same order.
template <int EPT, int ACT, bool DROP, bool Y>
__device__ __forceinline__ void ln_bwd_row(const BwdArgs& a, int64_t row, int c0, const LnBwdRowIn<EPT>& in,
                                           const float (&w)[EPT], const float (&bb)[EPT], float (&dw)[EPT],
                                           float (&db)[EPT]) {
  constexpr int D = 64 * EPT;
  constexpr bool HU = ACT != kNoU;
  const bool cu = HU && a.concat_u, cx = a.concat_x;
  const int col_u = 0, col_x = cu ? 1 : 0, col_z = (cu ? 1 : 0) + (cx ? 1 : 0);
  const uint32_t pos_x = 1, pos_u = cx ? 2 : 1;  // bit of x / u in a mask byte
  const float mean = in.mean, rstd = in.rstd;
  float x[EPT], gy[EPT], gx[EPT], gu[EPT], u[EPT];
  unpack_bf16<EPT>(in.x, x);
  unpack_bf16<EPT>(in.gy, gy);
  unpack_bf16<EPT>(in.gx, gx);
  unpack_bf16<EPT>(in.gu, gu);
  if constexpr (HU) unpack_bf16<EPT>(in.u, u);
  uint32_t mw[EPT / 4];
  if constexpr (DROP) {
#pragma unroll
    for (int q = 0; q < EPT / 4; ++q) mw[q] = in.m[q];
#pragma unroll
    for (int i = 0; i < EPT; ++i) {
      const uint32_t b0 = 8 * (i % 4);
      gy[i] = keep_scaled(gy[i], a.drop_scale, mw[i / 4], b0);
      gx[i] = keep_scaled(gx[i], a.drop_scale, mw[i / 4], b0 + pos_x);
      gu[i] = keep_scaled(gu[i], a.drop_scale, mw[i / 4], b0 + pos_u);
    }
  }
  // du and the recomputed y first, so that u, ln and m(u) die before the
  // row reductions; xh, g and gx stay live for dx.
  float xh[EPT], g[EPT], s1 = 0.f, s2 = 0.f;
#pragma unroll
  for (int i = 0; i < EPT; ++i) {
    xh[i] = (x[i] - mean) * rstd;
    const float ln = xh[i] * w[i] + bb[i];
    float mul = 1.f;
    if constexpr (HU) {
      const float sg = sigmoidf(u[i]);
      const float silu = u[i] * sg;
      const float dsilu = sg + silu * (1.f - sg);
      float dm;
      if constexpr (ACT == kActSilu) {
        mul = silu;
        dm = dsilu;
      } else if constexpr (ACT == kActSigmoid) {
        mul = sg;
        dm = sg * (1.f - sg);
      } else {
        mul = u[i];
        dm = 1.f;
      }
      gu[i] = gy[i] * ln * dm + (a.silu_u ? gu[i] * dsilu : gu[i]);
      if (a.silu_u) u[i] = silu;  // the concatenated u, for the recomputed y
    }
    g[i] = gy[i] * mul;  // gradient at ln
    gy[i] = ln * mul;    // y before dropout (gy is dead from here)
  }
  if constexpr (HU) store_bf16<EPT>(a.du + row * a.lddu + c0, gu);
  if constexpr (Y) {
    if constexpr (DROP) {
#pragma unroll
      for (int i = 0; i < EPT; ++i) {
        const uint32_t b0 = 8 * (i % 4);
        gy[i] = keep_scaled(gy[i], a.drop_scale, mw[i / 4], b0);
        x[i] = keep_scaled(x[i], a.drop_scale, mw[i / 4], b0 + pos_x);
        if constexpr (HU) u[i] = keep_scaled(u[i], a.drop_scale, mw[i / 4], b0 + pos_u);
      }
    }
    uint16_t* yr = a.y + row * a.ldy + c0;
    if (cu) store_bf16<EPT>(yr + col_u * D, u);
    if (cx) store_bf16<EPT>(yr + col_x * D, x);
    store_bf16<EPT>(yr + col_z * D, gy);
  }
#pragma unroll
  for (int i = 0; i < EPT; ++i) {
    const float wg = w[i] * g[i];
    s1 += xh[i] * wg;
    s2 += wg;
    dw[i] += g[i] * xh[i];
    db[i] += g[i];
  }
  const float c1 = wave_sum(s1) * a.inv_d, c2 = wave_sum(s2) * a.inv_d;
  float dx[EPT];
#pragma unroll
  for (int i = 0; i < EPT; ++i) dx[i] = gx[i] + (w[i] * g[i] - (xh[i] * c1 + c2)) * rstd;
  store_bf16<EPT>(a.dx + row * a.lddx + c0, dx);
}

// Wave i handles rows i, i + nwaves, ... in order; each block then sums its
// four waves' dweight / dbias in a fixed order, so the result is deterministic.
// ACT: kActNone / kActSilu / kActSigmoid, or kNoU (no u: weighted LayerNorm).
template <int EPT, int ACT, bool DROP, bool Y>
__global__ void __launch_bounds__(kThreads) ln_mul_bwd_kernel(BwdArgs a) {
  constexpr int D = 64 * EPT;
  constexpr bool HU = ACT != kNoU;
  __shared__ float red[4][2][D];
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int nw = gridDim.x * 4;
  const int c0 = lane * EPT;
  float w[EPT], bb[EPT], dw[EPT], db[EPT];
  ln_params<EPT>(a.w, a.b, a.w_bf16, c0, w, bb);
#pragma unroll
  for (int i = 0; i < EPT; ++i) dw[i] = db[i] = 0.f;
  const bool cu = HU && a.concat_u, cx = a.concat_x;
  const int col_u = 0, col_x = cu ? 1 : 0, col_z = (cu ? 1 : 0) + (cx ? 1 : 0);
  // Software pipeline: the next row's loads are in flight while this row is
  // computed (rows are independent).
  auto fetch = [&](int64_t row, LnBwdRowIn<EPT>& r) {
    const uint16_t* dyr = a.dy + row * a.lddy + c0;
    r.x = load_raw<EPT>(a.x + row * a.ldx + c0);
    r.gy = load_raw<EPT>(dyr + col_z * D);
    // without an x block, a residual branch's gradient takes gx's place: dx = gx + the LN backward
    r.gx = cx ? load_raw<EPT>(dyr + col_x * D) : a.dres ? load_raw<EPT>(a.dres + row * a.lddres + c0) : RawT<EPT>{};
    r.gu = cu ? load_raw<EPT>(dyr + col_u * D) : RawT<EPT>{};
    if constexpr (HU) r.u = load_raw<EPT>(a.u + row * a.ldu + c0);
    if constexpr (DROP) r.m = *(const MaskRawT<EPT>*)(a.mask + row * a.ldm + c0);
    r.mean = a.mean[row];
    r.rstd = a.rstd[row];
  };
  int64_t row = (int64_t)blockIdx.x * 4 + wave;
  LnBwdRowIn<EPT> cur;
  if (row < a.rows) fetch(row, cur);
  for (; row < a.rows; row += nw) {
    LnBwdRowIn<EPT> nxt;
    if (row + nw < a.rows) fetch(row + nw, nxt);
    ln_bwd_row<EPT, ACT, DROP, Y>(a, row, c0, cur, w, bb, dw, db);
    cur = nxt;
  }
#pragma unroll
  for (int i = 0; i < EPT; ++i) {
    red[wave][0][c0 + i] = dw[i];
    red[wave][1][c0 + i] = db[i];
  }
  __syncthreads();
  float* dst = a.partial + (int64_t)blockIdx.x * 2 * D;
  for (int c = threadIdx.x; c < 2 * D; c += kThreads) {
    const int k = c / D, cc = c - k * D;
    dst[c] = ((red[0][k][cc] + red[1][k][cc]) + red[2][k][cc]) + red[3][k][cc];
  }
}

// dweight / dbias: the column sums of the [nblocks, 2D] partial rows (dweight
// columns, then dbias), in a fixed order.  Block x owns 64 columns; thread
// (q, c) of 16 x 64 sums rows q + 16 k into accumulator k % 8 (eight loads in
// flight per thread), adds its eight accumulators pairwise, and the 16 row
// groups are added in a fixed tree.
constexpr int kRedThreads = 1024;
__global__ void __launch_bounds__(kRedThreads) ln_reduce_partials(const float* partial, int nblocks, int D,
                                                                  float* dweight, float* dbias) {
  __shared__ float part[16][64];
  const int cl = threadIdx.x & 63, q = threadIdx.x >> 6;
  const int c = blockIdx.x * 64 + cl;  // column of the [2, D] partial row
  const int64_t ld = 2 * (int64_t)D;
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  if (c < 2 * D) {
    int bk = q;
    for (; bk + 7 * 16 < nblocks; bk += 8 * 16) {
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[j] += partial[(int64_t)(bk + 16 * j) * ld + c];
    }
#pragma unroll
    for (int j = 0; j < 8; ++j)
      if (bk + 16 * j < nblocks) acc[j] += partial[(int64_t)(bk + 16 * j) * ld + c];
  }
  part[q][cl] = ((acc[0] + acc[1]) + (acc[2] + acc[3])) + ((acc[4] + acc[5]) + (acc[6] + acc[7]));
  __syncthreads();
#pragma unroll
  for (int w = 8; w > 0; w >>= 1) {
    if (q < w) part[q][cl] += part[q + w][cl];
    __syncthreads();
  }
  if (q == 0 && c < 2 * D) {
    const float t = part[0][cl];
    if (c < D) dweight[c] = t;
    else dbias[c - D] = t;
  }
}

// ------------------------------------------------- fused out-projection backward
// The output projection's FP8 dgrad fused with the LN * U * dropout backward
// (the reference's DLRM_HSTU_FP8_BWD_OUTPROJ_LNMD_FUSED kernel,
// ops/hip/l11_outproj_lnmd.cu:1-6): dy = bf16(g8 . w8^T * (s_g s_w) + 0),
// [rows, 1536] = the [u' | x | y] gradient, exactly as the e5m2 dgrad GEMM
// computes it (same MFMA, operand bytes, k order and epilogue), but it never
// leaves the chip: the LN backward consumes it row by row.
//
// One persistent workgroup per CU (8 waves) walks blocks of 64 rows.  GEMM
// phase: the block's e5m2 rows sit in LDS (64 x 512 bytes, 544-byte pitch);
// wave w owns columns 32 w .. 32 w + 31 of each of the six 256-column tiles
// for all 64 rows, and loads its W fragments straight from L2 into registers
// two (tile, k-step) chunks ahead -- no W staging, so the phase has no
// barrier.  After a tile's fourth k-step the wave's 32 results per lane are
// rounded to bf16 and kept packed (96 registers for the six tiles).
// Consumer phase: two groups of 32 rows; every wave writes its columns of the
// group into an LDS row buffer (3088-byte pitch), then runs four of its rows
// through ln_bwd_row (the standalone backward's row code), the x / u / mask
// loads of its next two rows in flight.
struct OutBwdArgs {
  BwdArgs ln;        // dy, y unused
  const uint8_t* g8;  // e5m2 [rows, 512]
  int64_t ldg;        // bytes
  const uint8_t* w8;  // e4m3 [1536, 512]
  int64_t ldw;        // bytes
  const float* g_scale;
  const float* w_scale;
  int nblk;
};
constexpr int kObThreads = 512, kObRows = 64, kObN = 1536, kObK = 512, kObD = 512, kObTileN = 256;
constexpr int kObApitch = kObK + 32;      // 544: conflict-free b128 fragment reads
constexpr int kObRpitch = 2 * kObN + 16;  // 3088
constexpr int kObGroup = 32;              // rows per consumer group
constexpr int kObA = kObRows * kObApitch;                       // 34816
constexpr int kObLnOff = kObA + kObGroup * kObRpitch;           // LN weight, bias: fp32 [2][512]
constexpr int kObSumOff = kObLnOff + 2 * kObD * 4;              // the workgroup's dweight, dbias sums
constexpr int kObLds = kObSumOff + 2 * kObD * 4;                // 141824
constexpr int kObTiles = kObN / kObTileN, kObSteps = kObK / 128, kObChunks = kObTiles * kObSteps;  // 6, 4, 24
constexpr int kObGrid = 256;

template <int ACT, bool DROP>
__global__ void __launch_bounds__(kObThreads, 1) outproj_ln_bwd_kernel(OutBwdArgs p) {
  constexpr int EPT = 8;
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  uint8_t* const al = smem;
  uint8_t* const rl = smem + kObA;
  float* const lnwb = (float*)(smem + kObLnOff);
  float* const wsum = (float*)(smem + kObSumOff);
  const BwdArgs& a = p.ln;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, li = lane & 15, g = lane >> 4;
  lnwb[tid] = ln_param(a.w, tid, a.w_bf16);
  lnwb[kObD + tid] = ln_param(a.b, tid, a.w_bf16);  // published by the first block's prologue barrier
  wsum[tid] = wsum[kObD + tid] = 0.f;  // thread t alone adds to entries t and 512 + t
  const int c0 = lane * EPT;
  const float scale = p.g_scale[0] * p.w_scale[0];
  const uint32_t ldw = (uint32_t)p.ldw, ldg = (uint32_t)p.ldg;
  const BufRsrc wr = make_rsrc(p.w8, (kObN - 1) * ldw + kObK);
  // W fragment (tile nt, k-step kk, column sub-tile cf): row 256 nt + 32 wave
  // + 16 cf + li, bytes 128 kk + 16 g and + 64 (the chunk part in soffset)
  const uint32_t w_voff = (uint32_t)(32 * wave + li) * ldw + 16 * g;
  auto load_w = [&](int c, i32x8 (&f)[2]) {
    const uint32_t soff = (uint32_t)((c >> 2) * kObTileN) * ldw + 128 * (c & 3);
#pragma unroll
    for (int cf = 0; cf < 2; ++cf) {
      const uint32_t v = w_voff + (uint32_t)(16 * cf) * ldw;
      f[cf] = cat8(buf_ld128(wr, v, soff), buf_ld128(wr, v + 64, soff));
    }
  };

  // the consumer's global inputs of one row (dy comes from LDS)
  auto fetch = [&](int64_t row, LnBwdRowIn<EPT>& r) {
    r.x = load_raw<EPT>(a.x + row * a.ldx + c0);
    r.u = load_raw<EPT>(a.u + row * a.ldu + c0);
    if constexpr (DROP) r.m = *(const MaskRawT<EPT>*)(a.mask + row * a.ldm + c0);
    r.mean = a.mean[row];
    r.rstd = a.rstd[row];
  };

  const int a_rd = li * kObApitch + 16 * g;
  for (int blk = blockIdx.x; blk < p.nblk; blk += gridDim.x) {
    const int64_t m0 = (int64_t)blk * kObRows;
    const int mrows = (int)min((int64_t)kObRows, (int64_t)a.rows - m0);
    i32x8 wf[2][2];
    {
      // the block's e5m2 rows (rows past the end read as zero); W chunks 0, 1
      const BufRsrc ar = make_rsrc(p.g8 + m0 * p.ldg, (uint32_t)(mrows - 1) * ldg + kObK);
      u32x4 ast[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int e = tid + kObThreads * i;
        ast[i] = buf_ld128(ar, (uint32_t)(e >> 5) * ldg + 16 * (e & 31), 0);
      }
      load_w(0, wf[0]);
      load_w(1, wf[1]);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int e = tid + kObThreads * i;
        *(u32x4*)(al + (e >> 5) * kObApitch + 16 * (e & 31)) = ast[i];
      }
    }
    __syncthreads();
    uint32_t dyp[kObTiles][2][4][2];  // [tile][column sub-tile][row sub-tile][pair]
    f32x4 acc[2][4];
#pragma unroll
    for (int c = 0; c < kObChunks; ++c) {
      const int nt = c >> 2, kk = c & 3;
      if (kk == 0) {
#pragma unroll
        for (int cf = 0; cf < 2; ++cf)
#pragma unroll
          for (int rf = 0; rf < 4; ++rf) acc[cf][rf] = zero4();
      }
#pragma unroll
      for (int rf = 0; rf < 4; ++rf) {
        const uint8_t* r = al + a_rd + rf * 16 * kObApitch + kk * 128;
        const i32x8 bop = cat8(lds_ld128(r), lds_ld128(r + 64));
#pragma unroll
        for (int cf = 0; cf < 2; ++cf)
          acc[cf][rf] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(wf[c & 1][cf], bop, acc[cf][rf], 0, 1, 0, 0,
                                                                        0, 0);
      }
      if (c + 2 < kObChunks) load_w(c + 2, wf[c & 1]);
      if (kk == 3) {
        // lane: row 16 rf + li, columns 256 nt + 32 wave + 16 cf + 4 g .. + 3
#pragma unroll
        for (int cf = 0; cf < 2; ++cf)
#pragma unroll
          for (int rf = 0; rf < 4; ++rf) {
            float v[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) v[r] = acc[cf][rf][r] * scale + 0.f;
            dyp[nt][cf][rf][0] = pack_bf16(v[0], v[1]);
            dyp[nt][cf][rf][1] = pack_bf16(v[2], v[3]);
          }
      }
      // no scheduling across chunks: hoisted reads and MFMAs of later chunks
      // would keep several chunks' operands live
      __builtin_amdgcn_sched_barrier(0);
    }

    // consumer: group G = rows 32 G .. 32 G + 31 of the block (row sub-tiles
    // 2 G, 2 G + 1); wave w then takes rows w, w + 8, w + 16, w + 24 of it,
    // two rows' loads in flight
    float dw[EPT], db[EPT];
#pragma unroll
    for (int i = 0; i < EPT; ++i) dw[i] = db[i] = 0.f;
    auto put = [&](int G) {
      uint8_t* dst = rl + li * kObRpitch + 2 * (32 * wave + 4 * g);
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int nt = 0; nt < kObTiles; ++nt)
#pragma unroll
          for (int cf = 0; cf < 2; ++cf)
            *(u32x2*)(dst + 16 * h * kObRpitch + 2 * (nt * kObTileN + 16 * cf)) =
                u32x2{dyp[nt][cf][2 * G + h][0], dyp[nt][cf][2 * G + h][1]};
    };
#pragma unroll 1
    for (int G = 0; G < 2; ++G) {
      LnBwdRowIn<EPT> in[2];
#pragma unroll
      for (int k = 0; k < 2; ++k) {
        const int rr = kObGroup * G + 8 * k + wave;
        if (rr < mrows) fetch(m0 + rr, in[k]);
      }
      if (G == 0) put(0);
      else put(1);
      __syncthreads();
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int rr = kObGroup * G + 8 * k + wave;
        LnBwdRowIn<EPT>& cur = in[k & 1];
        if (rr < mrows) {
          const uint8_t* src = rl + (8 * k + wave) * kObRpitch + 16 * lane;
          cur.gu = *(const u32x4*)src;
          cur.gx = *(const u32x4*)(src + 2 * kObD);
          cur.gy = *(const u32x4*)(src + 4 * kObD);
          // the LN weight and bias, read per row so that they hold no
          // registers across the phases
          float w[EPT], bb[EPT];
          const f32x4 w0 = *(const f32x4*)(lnwb + c0), w1 = *(const f32x4*)(lnwb + c0 + 4);
          const f32x4 b0 = *(const f32x4*)(lnwb + kObD + c0), b1 = *(const f32x4*)(lnwb + kObD + c0 + 4);
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            w[i] = w0[i];
            w[i + 4] = w1[i];
            bb[i] = b0[i];
            bb[i + 4] = b1[i];
          }
          ln_bwd_row<EPT, ACT, DROP, false>(a, m0 + rr, c0, cur, w, bb, dw, db);
        }
        if (k + 2 < 4 && rr + 16 < mrows) fetch(m0 + rr + 16, cur);
      }
      __syncthreads();
    }
    // the block's dweight / dbias: its 8 waves summed in a fixed order (the
    // A tile's LDS is free until the next block's prologue), added to the
    // workgroup's sums
    float* red = (float*)smem;  // [8][2][512]
#pragma unroll
    for (int i = 0; i < EPT; ++i) {
      red[(wave * 2 + 0) * kObD + c0 + i] = dw[i];
      red[(wave * 2 + 1) * kObD + c0 + i] = db[i];
    }
    __syncthreads();
    for (int c = tid; c < 2 * kObD; c += kObThreads) {
      const int k = c / kObD, cc = c - k * kObD;
      float t = red[k * kObD + cc];
#pragma unroll
      for (int v = 1; v < 8; ++v) t += red[(v * 2 + k) * kObD + cc];
      wsum[c] += t;
    }
    __syncthreads();
  }
  // the workgroup's sums over its blocks (in block order)
  float* dst = a.partial + (int64_t)blockIdx.x * 2 * kObD;
  for (int c = tid; c < 2 * kObD; c += kObThreads) dst[c] = wsum[c];
}

// ------------------------------------------------------------------ host
bool aligned(const void* p, int a) { return ((uintptr_t)p % a) == 0; }

int ncols_of(const void* u, int concat_u, int concat_x) {
  return (u != nullptr && concat_u ? 1 : 0) + (concat_x ? 1 : 0) + 1;
}

// Keep threshold of the 32-bit mask, from the fp32 test Triton's
// uint_to_uniform_float(x) > ratio makes (triton_hstu_linear.py:2335-2355):
// the largest x' = x ^ (x >> 31) in [-1, 2^31 - 1] that is dropped.
int keep_above(float ratio) {
  const float scale = 4.6566127342e-10f;
  auto keep = [&](int64_t v) { return (float)v * scale > ratio; };
  int64_t lo = 0, hi = (int64_t)1 << 31;
  while (lo < hi) {
    const int64_t mid = (lo + hi) / 2;
    if (keep(mid)) hi = mid;
    else lo = mid + 1;
  }
  return (int)(lo - 1);
}

MaskSpec mask_spec(int D, int num_masks, bool mask16, float ratio, uint64_t seed) {
  MaskSpec m{};
  m.num_masks = num_masks;
  m.mask16 = mask16;
  if (mask16) {  // P(drop) = round(ratio * 65536) / 65536, ties to even (:2542-2544)
    const double t = std::nearbyint((double)ratio * 65536.0);
    m.thr = (int)(t < 0 ? 0 : t > 65536 ? 65536 : t);
  } else {
    m.thr = keep_above(ratio);
  }
  int bd = 1;
  while (bd < D) bd <<= 1;
  m.block_d = bd;
  m.k0 = (uint32_t)(seed & 0xffffffffu);
  m.k1 = (uint32_t)(seed >> 32);
  return m;
}

// rows >= 0 and a D some kernel instantiation serves
bool d_served(int D) { return D == 512 || D == 256; }

template <int EPT, int ACT>
void launch_fwd_act(bool drop, bool e4m3, const FwdArgs& a, hipStream_t st) {
  const dim3 g((a.rows + kFwdRows - 1) / kFwdRows), b(kThreads);
  if (drop && e4m3) hipLaunchKernelGGL((ln_mul_fwd_kernel<EPT, ACT, true, true>), g, b, 0, st, a);
  else if (drop) hipLaunchKernelGGL((ln_mul_fwd_kernel<EPT, ACT, true, false>), g, b, 0, st, a);
  else if (e4m3) hipLaunchKernelGGL((ln_mul_fwd_kernel<EPT, ACT, false, true>), g, b, 0, st, a);
  else hipLaunchKernelGGL((ln_mul_fwd_kernel<EPT, ACT, false, false>), g, b, 0, st, a);
}
template <int EPT>
void launch_fwd_ept(int act, bool drop, bool e4m3, const FwdArgs& a, hipStream_t st) {
  switch (act) {
    case kActNone: launch_fwd_act<EPT, kActNone>(drop, e4m3, a, st); break;
    case kActSilu: launch_fwd_act<EPT, kActSilu>(drop, e4m3, a, st); break;
    case kActSigmoid: launch_fwd_act<EPT, kActSigmoid>(drop, e4m3, a, st); break;
    default: launch_fwd_act<EPT, kNoU>(drop, e4m3, a, st); break;
  }
}
void launch_fwd(int D, int act, bool drop, bool e4m3, const FwdArgs& a, hipStream_t st) {
  if (D == 512) launch_fwd_ept<8>(act, drop, e4m3, a, st);
  else launch_fwd_ept<4>(act, drop, e4m3, a, st);
}

template <int EPT, int ACT>
void launch_bwd_act(bool drop, bool y, const BwdArgs& a, hipStream_t st) {
  const dim3 g(ACT == kNoU ? kBwdBlocksMax : kBwdBlocksU), b(kThreads);
  if (drop && y) hipLaunchKernelGGL((ln_mul_bwd_kernel<EPT, ACT, true, true>), g, b, 0, st, a);
  else if (drop) hipLaunchKernelGGL((ln_mul_bwd_kernel<EPT, ACT, true, false>), g, b, 0, st, a);
  else if (y) hipLaunchKernelGGL((ln_mul_bwd_kernel<EPT, ACT, false, true>), g, b, 0, st, a);
  else hipLaunchKernelGGL((ln_mul_bwd_kernel<EPT, ACT, false, false>), g, b, 0, st, a);
}
template <int EPT>
void launch_bwd_ept(int act, bool drop, bool y, const BwdArgs& a, hipStream_t st) {
  switch (act) {
    case kActNone: launch_bwd_act<EPT, kActNone>(drop, y, a, st); break;
    case kActSilu: launch_bwd_act<EPT, kActSilu>(drop, y, a, st); break;
    case kActSigmoid: launch_bwd_act<EPT, kActSigmoid>(drop, y, a, st); break;
    default: launch_bwd_act<EPT, kNoU>(drop, y, a, st); break;
  }
}
void launch_bwd(int D, int act, bool drop, bool y, const BwdArgs& a, hipStream_t st) {
  if (D == 512) launch_bwd_ept<8>(act, drop, y, a, st);
  else launch_bwd_ept<4>(act, drop, y, a, st);
}

}  // namespace

extern "C" int hstu_dropout_mask(int rows, int D, int num_masks, int mask16, float dropout_ratio, uint64_t seed,
                                 void* mask, int64_t ldm, hipStream_t stream) {
  if (rows < 0 || D <= 0 || num_masks < 1 || num_masks > 3 || mask == nullptr || ldm < D ||
      !(dropout_ratio >= 0.f && dropout_ratio <= 1.f))
    return HSTU_E_BAD_ARG;
  if (!d_served(D)) return HSTU_E_UNSUPPORTED;
  if (rows == 0) return 0;
  const MaskSpec ms = mask_spec(D, num_masks, mask16 != 0, dropout_ratio, seed);
  hipLaunchKernelGGL(dropout_mask_kernel, dim3((rows + 7) / 8), dim3(kThreads), 0, stream, ms, rows, D,
                     (uint8_t*)mask, ldm);
  return (int)hipGetLastError();
}

// LayerNorm weight / bias: fp32, or bf16 read as is (the parameters' own
// dtype, so a caller needs no conversion per call).
static bool param_dtype_ok(int t) { return t == HSTU_DTYPE_FP32 || t == HSTU_DTYPE_BF16; }
// the kernels read a lane's parameters as 16-byte vectors (8 bytes for bf16 at D = 256)
static bool params_aligned(const void* w, const void* b) { return aligned(w, 16) && aligned(b, 16); }

extern "C" int hstu_ln_mul_fwd(const void* x, int64_t ldx, const void* u, int64_t ldu, const void* weight,
                               const void* bias, int param_dtype, float eps, int rows, int D, int mul_u_act, int silu_u,
                               int concat_u, int concat_x, int training, float dropout_ratio, uint64_t seed,
                               int mask16, void* mask, int64_t ldm, void* y, int64_t ldy, int out_dtype,
                               float inv_scale, const float* out_scale, float* mean, float* rstd,
                               hipStream_t stream) {
  if (rows < 0 || D <= 0 || x == nullptr || ldx < D || (u != nullptr && ldu < D) || weight == nullptr ||
      bias == nullptr || mean == nullptr || rstd == nullptr || y == nullptr || mul_u_act < 0 || mul_u_act > 2 ||
      !(dropout_ratio >= 0.f && dropout_ratio <= 1.f) || !param_dtype_ok(param_dtype))
    return HSTU_E_BAD_ARG;
  if (out_dtype != HSTU_DTYPE_BF16 && out_dtype != HSTU_DTYPE_FP8_E4M3) return HSTU_E_BAD_ARG;
  const int ncols = ncols_of(u, concat_u, concat_x);
  if (ldy < (int64_t)ncols * D) return HSTU_E_BAD_ARG;
  if (!d_served(D)) return HSTU_E_UNSUPPORTED;
  const bool dropout = training && dropout_ratio > 0.f;
  if (dropout && (mask == nullptr || ldm < D)) return HSTU_E_BAD_ARG;
  const int ept = D / 64;
  const int ysz = out_dtype == HSTU_DTYPE_BF16 ? 2 : 1;
  if (!aligned(x, 2 * ept) || ldx % ept || (u != nullptr && (!aligned(u, 2 * ept) || ldu % ept)) ||
      !aligned(y, ysz * ept) || ldy % ept || (dropout && (!aligned(mask, ept) || ldm % ept)) ||
      !params_aligned(weight, bias))
    return HSTU_E_UNSUPPORTED;
  if (rows == 0) return 0;
  FwdArgs a{};
  a.x = (const uint16_t*)x;
  a.ldx = ldx;
  a.u = (const uint16_t*)u;
  a.ldu = ldu;
  a.w = weight;
  a.b = bias;
  a.w_bf16 = param_dtype == HSTU_DTYPE_BF16;
  a.eps = eps;
  a.inv_d = 1.f / (float)D;
  a.rows = rows;
  a.silu_u = silu_u;
  a.concat_u = concat_u;
  a.concat_x = concat_x;
  a.drop_scale = dropout ? 1.f / (1.f - dropout_ratio) : 1.f;
  a.ms = mask_spec(D, ncols, mask16 != 0, dropout_ratio, seed);
  a.mask = (uint8_t*)mask;
  a.ldm = ldm;
  a.y = y;
  a.ldy = ldy;
  a.inv_scale = inv_scale;
  a.out_scale = out_scale;
  a.mean = mean;
  a.rstd = rstd;
  launch_fwd(D, u == nullptr ? kNoU : mul_u_act, dropout, out_dtype == HSTU_DTYPE_FP8_E4M3, a, stream);
  return (int)hipGetLastError();
}

extern "C" int64_t hstu_ln_mul_bwd_workspace_bytes(int rows, int D) {
  if (rows < 0 || !d_served(D)) return -1;
  return (int64_t)kBwdBlocksMax * 2 * D * 4;
}

extern "C" int hstu_ln_mul_bwd(const void* dy, int64_t lddy, const void* x, int64_t ldx, const void* u,
                               int64_t ldu, const void* weight, const void* bias, int param_dtype, const float* mean,
                               const float* rstd, int rows, int D, int mul_u_act, int silu_u, int concat_u,
                               int concat_x, float dropout_ratio, const void* mask, int64_t ldm, void* dx,
                               int64_t lddx, void* du, int64_t lddu, void* y, int64_t ldy, const void* dres,
                               int64_t lddres, float* dweight, float* dbias, void* workspace,
                               int64_t workspace_bytes, hipStream_t stream) {
  if (rows < 0 || D <= 0 || dy == nullptr || x == nullptr || ldx < D || dx == nullptr || lddx < D ||
      (u != nullptr && (ldu < D || du == nullptr || lddu < D)) || weight == nullptr || bias == nullptr ||
      mean == nullptr || rstd == nullptr || dweight == nullptr || dbias == nullptr || mul_u_act < 0 ||
      mul_u_act > 2 || (mask != nullptr && (ldm < D || !(dropout_ratio >= 0.f && dropout_ratio <= 1.f))) ||
      !param_dtype_ok(param_dtype))
    return HSTU_E_BAD_ARG;
  const int ncols = ncols_of(u, concat_u, concat_x);
  if (lddy < (int64_t)ncols * D || (y != nullptr && ldy < (int64_t)ncols * D)) return HSTU_E_BAD_ARG;
  if (dres != nullptr && (concat_x || mask != nullptr || lddres < D)) return HSTU_E_BAD_ARG;
  if (!d_served(D)) return HSTU_E_UNSUPPORTED;
  if (workspace == nullptr || workspace_bytes < hstu_ln_mul_bwd_workspace_bytes(rows, D)) return HSTU_E_BAD_ARG;
  const int ept = D / 64;
  auto ok = [&](const void* p, int64_t ld, int esz) { return aligned(p, esz * ept) && ld % ept == 0; };
  if (!ok(dy, lddy, 2) || !ok(x, ldx, 2) || !ok(dx, lddx, 2) ||
      (u != nullptr && (!ok(u, ldu, 2) || !ok(du, lddu, 2))) || (y != nullptr && !ok(y, ldy, 2)) ||
      (mask != nullptr && !ok(mask, ldm, 1)) || (dres != nullptr && !ok(dres, lddres, 2)) ||
      !params_aligned(weight, bias))
    return HSTU_E_UNSUPPORTED;
  BwdArgs a{};
  a.dy = (const uint16_t*)dy;
  a.lddy = lddy;
  a.x = (const uint16_t*)x;
  a.ldx = ldx;
  a.u = (const uint16_t*)u;
  a.ldu = ldu;
  a.w = weight;
  a.b = bias;
  a.w_bf16 = param_dtype == HSTU_DTYPE_BF16;
  a.mean = mean;
  a.rstd = rstd;
  a.inv_d = 1.f / (float)D;
  a.rows = rows;
  a.silu_u = silu_u;
  a.concat_u = concat_u;
  a.concat_x = concat_x;
  a.mask = (const uint8_t*)mask;
  a.ldm = ldm;
  a.drop_scale = 1.f / (1.f - dropout_ratio);
  a.dx = (uint16_t*)dx;
  a.lddx = lddx;
  a.du = (uint16_t*)du;
  a.lddu = lddu;
  a.y = (uint16_t*)y;
  a.ldy = ldy;
  a.dres = (const uint16_t*)dres;
  a.lddres = lddres;
  a.partial = (float*)workspace;
  launch_bwd(D, u == nullptr ? kNoU : mul_u_act, mask != nullptr, y != nullptr, a, stream);
  hipLaunchKernelGGL(ln_reduce_partials, dim3((2 * D + 63) / 64), dim3(kRedThreads), 0, stream, a.partial,
                     u == nullptr ? kBwdBlocksMax : kBwdBlocksU, D, dweight, dbias);
  return (int)hipGetLastError();
}

extern "C" int64_t hstu_outproj_ln_bwd_workspace_bytes(int rows) {
  if (rows < 0) return -1;
  return (int64_t)kObGrid * 2 * kObD * 4;
}

extern "C" int hstu_outproj_ln_bwd(const void* g8, int64_t ldg, const float* g_scale, const void* w8, int64_t ldw,
                                   const float* w_scale, const void* x, int64_t ldx, const void* u, int64_t ldu,
                                   const void* weight, const void* bias, int param_dtype, const float* mean,
                                   const float* rstd, int rows, int D, int mul_u_act, int silu_u, float dropout_ratio,
                                   const void* mask,
                                   int64_t ldm, void* dx, int64_t lddx, void* du, int64_t lddu, float* dweight,
                                   float* dbias, void* workspace, int64_t workspace_bytes, hipStream_t stream) {
  if (rows < 0 || g8 == nullptr || w8 == nullptr || g_scale == nullptr || w_scale == nullptr || x == nullptr ||
      u == nullptr || dx == nullptr || du == nullptr || weight == nullptr || bias == nullptr || mean == nullptr ||
      rstd == nullptr || dweight == nullptr || dbias == nullptr || mul_u_act < 0 || mul_u_act > 2 ||
      ldg < kObK || ldw < kObK || ldx < D || ldu < D || lddx < D || lddu < D ||
      (mask != nullptr && (ldm < D || !(dropout_ratio >= 0.f && dropout_ratio <= 1.f))) ||
      !param_dtype_ok(param_dtype))
    return HSTU_E_BAD_ARG;
  if (D != kObD) return HSTU_E_UNSUPPORTED;
  if (workspace == nullptr || workspace_bytes < hstu_outproj_ln_bwd_workspace_bytes(rows)) return HSTU_E_BAD_ARG;
  auto al16 = [](const void* p, int64_t ld, int esz) { return aligned(p, 16) && (ld * esz) % 16 == 0; };
  if (!al16(g8, ldg, 1) || !al16(w8, ldw, 1) || !al16(x, ldx, 2) || !al16(u, ldu, 2) || !al16(dx, lddx, 2) ||
      !al16(du, lddu, 2) || (mask != nullptr && (!aligned(mask, 8) || ldm % 8 != 0)))
    return HSTU_E_UNSUPPORTED;
  if ((int64_t)(kObN - 1) * ldw + kObK > 0xffffffffLL || (int64_t)(kObRows - 1) * ldg + kObK > 0xffffffffLL)
    return HSTU_E_UNSUPPORTED;
  if (rows == 0) {
    // no rows: zero weight gradients, like the standalone backward
    hipLaunchKernelGGL(ln_reduce_partials, dim3((2 * D + 63) / 64), dim3(kRedThreads), 0, stream,
                       (const float*)workspace, 0, D, dweight, dbias);
    return (int)hipGetLastError();
  }
  OutBwdArgs p{};
  BwdArgs& a = p.ln;
  a.x = (const uint16_t*)x;
  a.ldx = ldx;
  a.u = (const uint16_t*)u;
  a.ldu = ldu;
  a.w = weight;
  a.b = bias;
  a.w_bf16 = param_dtype == HSTU_DTYPE_BF16;
  a.mean = mean;
  a.rstd = rstd;
  a.inv_d = 1.f / (float)D;
  a.rows = rows;
  a.silu_u = silu_u;
  a.concat_u = 1;
  a.concat_x = 1;
  a.mask = (const uint8_t*)mask;
  a.ldm = ldm;
  a.drop_scale = 1.f / (1.f - dropout_ratio);
  a.dx = (uint16_t*)dx;
  a.lddx = lddx;
  a.du = (uint16_t*)du;
  a.lddu = lddu;
  a.partial = (float*)workspace;
  p.g8 = (const uint8_t*)g8;
  p.ldg = ldg;
  p.w8 = (const uint8_t*)w8;
  p.ldw = ldw;
  p.g_scale = g_scale;
  p.w_scale = w_scale;
  p.nblk = (int)(((int64_t)rows + kObRows - 1) / kObRows);
  const int grid = std::min(p.nblk, kObGrid);
  const void* fn;
  const bool drop = mask != nullptr;
  switch (mul_u_act) {
    case kActNone: fn = drop ? (const void*)outproj_ln_bwd_kernel<kActNone, true> : (const void*)outproj_ln_bwd_kernel<kActNone, false>; break;
    case kActSilu: fn = drop ? (const void*)outproj_ln_bwd_kernel<kActSilu, true> : (const void*)outproj_ln_bwd_kernel<kActSilu, false>; break;
    default: fn = drop ? (const void*)outproj_ln_bwd_kernel<kActSigmoid, true> : (const void*)outproj_ln_bwd_kernel<kActSigmoid, false>; break;
  }
  static std::once_flag once[6];
  static hipError_t set_err[6];
  const int slot = 2 * mul_u_act + (drop ? 1 : 0);
  std::call_once(once[slot], [&] { set_err[slot] = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, kObLds); });
  if (set_err[slot] != hipSuccess) return (int)set_err[slot];
  void* args[] = {&p};
  hipError_t e = hipLaunchKernel(fn, dim3(grid), dim3(kObThreads), args, (size_t)kObLds, stream);
  if (e != hipSuccess) return (int)e;
  hipLaunchKernelGGL(ln_reduce_partials, dim3((2 * D + 63) / 64), dim3(kRedThreads), 0, stream, a.partial, grid, D,
                     dweight, dbias);
  return (int)hipGetLastError();
}
