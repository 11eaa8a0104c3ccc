// Weight gradients over the token axis of the HSTU layer's projections,
//   C[n1][n2] = sa * sb * sum_t A[t][n1] * B[t][n2],
// from row-major operands that hold one token per row: x^T dz of the UVQK
// projection (A = LN(x) [T, 512], B = d(uvqk) [T, 2048]) and y^T dout of the
// output projection (A = y [T, 1536], B = dout [T, 512]), for MI355X (gfx950).
// Reference behaviour followed (paths relative to
// recommendation_v4/hstu/generative_recommenders/):
//   bf16 wgrad dw = x^T dz         ops/triton/triton_addmm.py:1737-1750
//   output-projection wgrad        ops/triton/triton_hstu_linear.py (torch.mm(y.t(), dout))
//   split-K over tokens, fixed-    ops/triton/fp8_wgrad.py:27-160 (fp8_wgrad: fp32
//   order second pass                partials [SPLIT, N1, N2], reduce, then the scales)
//
// Design: the output is small (0.75-1 M elements) and the contraction long
// (T ~ 162 K tokens), so the tokens are split over workgroups: tiles x split
// ~ one workgroup per CU.  A workgroup owns a 256 (n1) x 256 (n2) tile of one
// token range; 8 waves as 4 (n1) x 2 (n2) of 64 x 128.  Each k-step of 32
// tokens stages both operands' 32 x 512-byte tile rows in LDS as they lie in
// memory (token rows, 544-byte pitch), and the MFMA operands come out of LDS
// with the transposed read ds_read_b64_tr_b16, which turns a token-major tile
// into k(token)-contiguous fragments: lane group g gets tokens {4g..4g+3,
// 16+4g..16+4g+3} of column li in both operands, so the contraction sees the
// same token order on both sides.  The MFMA (v_mfma_f32_16x16x32_bf16) runs
// with B as its A operand, so a lane's result is 4 consecutive n2 of one n1
// row.  Global loads for step k+1 are issued into registers before step k's
// MFMAs and written to the other LDS buffer after them (one barrier per
// step).  Workgroups are numbered so that the tiles of one token range run on
// one XCD and share its L2.  With split > 1 every workgroup writes an fp32
// partial tile; a second kernel sums the splits in a fixed order, applies
// sa * sb and writes bf16 or fp32 (bitwise reproducible, no atomics).
// Optionally (bf16) the workgroups of the first n1 tile also sum B's columns
// from the registers they stage (the projection's bias gradient), so the
// layer needs no separate pass over d(uvqk) for it.
// The fp8 form (e4m3 A, e4m3 or e5m2 B: the reference's fp8_wgrad operands)
// takes 128-token steps of 256-byte rows through the same LDS budget, reads
// its fragments with ds_read_b64_tr_b8 (four 8-token reads per 32-byte
// fragment) and runs v_mfma_f32_16x16x128_f8f6f4 with the operands' formats.

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>
#include <mutex>
#include <vector>

#include "hstu_common.h"
#include "hstu_mi355x.h"

namespace {
using namespace hstu;

constexpr int kWThreads = 512;  // 8 waves
constexpr int kBN1 = 256, kBN2 = 256;  // output tile
constexpr int kCus = 256;

// Per operand format: bf16 steps of 64 tokens (512-byte tile rows, 544-byte
// pitch) or fp8 steps of 128 tokens (256-byte rows, 272-byte pitch).  Both
// stage 64 KiB per step and take 136 KiB of LDS for two steps.
template <bool F8>
struct WCfg {
  static constexpr int KT = F8 ? 128 : 64;           // tokens per k-step
  static constexpr int ES = F8 ? 1 : 2;              // bytes per element
  static constexpr int ROW = kBN1 * ES;              // tile row bytes
  static constexpr int PITCH = ROW + (F8 ? 16 : 32);  // conflict-free transposed reads
  static constexpr int TILE = KT * PITCH;
  static constexpr int STAGE = 2 * TILE;             // A tile then B tile
  static constexpr int LDS = 2 * STAGE;
  static constexpr int CPR = ROW / 16;               // 16-byte chunks per tile row
  static constexpr int Q = KT * CPR / kWThreads;     // staged chunks per thread per operand
};
constexpr int kWLds = WCfg<false>::LDS;
static_assert(WCfg<true>::LDS == kWLds, "one LDS size");


struct WgradParams {
  const uint8_t* A;
  const uint8_t* B;
  int64_t lda, ldb;  // bytes
  int64_t T;
  int64_t tps;  // tokens per split, a multiple of kKT
  int N1, N2;
  int split, tiles_n2, tiles;
  float* ws;     // [split][N1][N2] fp32 partials when split > 1
  float* cs_ws;  // [split][N2] column-sum partials when split > 1
  float* colsum; // fp32 [N2]: sum over the tokens of B, or null (bf16 only)
  void* out;
  int64_t ldo;  // elements
  int out_f32;
  const float* sa;
  const float* sb;
};

// F8: A and B fp8 with MFMA formats FA / FB (0 e4m3, 1 e5m2); else bf16.
template <bool F8, int FA, int FB>
__global__ void __launch_bounds__(kWThreads, 1) wgrad_kernel(WgradParams p) {
  using C = WCfg<F8>;
  constexpr int kKT = C::KT, kWPitch = C::PITCH, kWTile = C::TILE, kWStage = C::STAGE, kQ = C::Q;
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  // XCD-contiguous numbering: workgroup b runs on XCD b % 8; consecutive idx
  // (one token range, all its tiles) land on one XCD.
  const int total = p.tiles * p.split;
  const int per_xcd = (total + 7) / 8;
  const int idx = (int)(blockIdx.x % 8) * per_xcd + (int)(blockIdx.x / 8);
  if (idx >= total) return;
  const int s = idx / p.tiles, tile = idx - s * p.tiles;
  const int t1 = tile / p.tiles_n2, t2 = tile - t1 * p.tiles_n2;
  const int n10 = t1 * kBN1, n20 = t2 * kBN2;
  const int64_t tb = (int64_t)s * p.tps;
  const int64_t te = min(tb + p.tps, p.T);
  const int nk = (int)((te - tb + kKT - 1) / kKT);

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, li = lane & 15, g = lane >> 4;
  const int w1 = (wave >> 1) * 64, w2 = (wave & 1) * 128;

  // Token rows tb .. te-1 of the tile's column band; rows past te (the next
  // split's, or past T) read as zero.
  const uint32_t lda = (uint32_t)p.lda, ldb = (uint32_t)p.ldb;
  const BufRsrc ar = make_rsrc(p.A + tb * p.lda + n10 * C::ES, (uint32_t)((te - tb - 1) * p.lda + C::ROW));
  const BufRsrc br = make_rsrc(p.B + tb * p.ldb + n20 * C::ES, (uint32_t)((te - tb - 1) * p.ldb + C::ROW));
  // staging: chunk c = tid + 512 q (q < kQ) of a kKT-row tile
  uint32_t va[kQ], vb[kQ], lo[kQ];
#pragma unroll
  for (int q = 0; q < kQ; ++q) {
    const int c = tid + kWThreads * q, row = c / C::CPR, col = c % C::CPR;
    va[q] = row * lda + col * 16;
    vb[q] = row * ldb + col * 16;
    lo[q] = row * kWPitch + col * 16;
  }
  u32x4 ra[kQ], rb[kQ];
  auto load = [&](int kk) {
    const uint32_t sa_off = (uint32_t)kk * kKT * lda, sb_off = (uint32_t)kk * kKT * ldb;
#pragma unroll
    for (int q = 0; q < kQ; ++q) {
      ra[q] = buf_ld128(ar, va[q], sa_off);
      rb[q] = buf_ld128(br, vb[q], sb_off);
    }
  };
  // column sums of B (the bias gradient of the layer's projection), taken
  // from the staged registers by the workgroups of the first n1 tile: a
  // thread's chunks all sit at byte column 16 (tid % 32) of the tile
  const bool do_cs = !F8 && p.colsum != nullptr && t1 == 0;
  float cs[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  auto store = [&](uint8_t* st) {
#pragma unroll
    for (int q = 0; q < kQ; ++q) {
      *(u32x4*)(st + lo[q]) = ra[q];
      *(u32x4*)(st + kWTile + lo[q]) = rb[q];
    }
    if (do_cs) {
#pragma unroll
      for (int q = 0; q < kQ; ++q)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const uint32_t w = rb[q][e];
          cs[2 * e] += __builtin_bit_cast(float, w << 16);
          cs[2 * e + 1] += __builtin_bit_cast(float, w & 0xffff0000u);
        }
    }
  };

  f32x4 acc[8][4];  // [n2 block][n1 block], lane: n1 = 16i + li, n2 = 16j + 4g .. +3
#pragma unroll
  for (int j = 0; j < 8; ++j)
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[j][i] = zero4();

  if (nk > 0) {
    load(0);
    store(smem);
  }
  __syncthreads();
  // transposed-read start.  bf16: row 4g + li/4, 4-column group li % 4.
  // fp8: token row 8g + li/2 (plus 32 per read), 8-column half li % 2.
  const int tr = F8 ? (8 * g + (li >> 1)) * kWPitch + (li & 1) * 8 : (4 * g + (li >> 2)) * kWPitch + (li & 3) * 8;
  const int a_rd = tr + w1 * C::ES, b_rd = kWTile + tr + w2 * C::ES;
  for (int kk = 0; kk < nk; ++kk) {
    const uint8_t* buf = smem + (kk & 1) * kWStage;
    if (kk + 1 < nk) load(kk + 1);
    if constexpr (F8) {
      // one 128-token MFMA step: lane (li, g) holds tokens 32r + 8g .. +7 of
      // its column in bytes 8r .. 8r+7 (r = 0..3), the same in both operands
      auto frag = [&](const uint8_t* q0) {
        const u32x2 r0 = lds_tr8(q0), r1 = lds_tr8(q0 + 32 * kWPitch);
        const u32x2 r2 = lds_tr8(q0 + 64 * kWPitch), r3 = lds_tr8(q0 + 96 * kWPitch);
        i32x8 f;
        f[0] = (int)r0[0]; f[1] = (int)r0[1]; f[2] = (int)r1[0]; f[3] = (int)r1[1];
        f[4] = (int)r2[0]; f[5] = (int)r2[1]; f[6] = (int)r3[0]; f[7] = (int)r3[1];
        return f;
      };
      i32x8 af[4], bfr[8];
#pragma unroll
      for (int i = 0; i < 4; ++i) af[i] = frag(buf + a_rd + 16 * i);
#pragma unroll
      for (int j = 0; j < 8; ++j) bfr[j] = frag(buf + b_rd + 16 * j);
#pragma unroll
      for (int j = 0; j < 8; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          acc[j][i] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(bfr[j], af[i], acc[j][i], FB, FA, 0, 0, 0, 0);
    } else {
#pragma unroll
    for (int h = 0; h < kKT / 32; ++h) {
      const uint8_t* hb = buf + h * 32 * kWPitch;
      u32x4 af[4], bfr[8];
#pragma unroll
      for (int i = 0; i < 4; ++i)
        af[i] = cat_tr(lds_tr16(hb + a_rd + 32 * i), lds_tr16(hb + a_rd + 32 * i + 16 * kWPitch));
#pragma unroll
      for (int j = 0; j < 8; ++j)
        bfr[j] = cat_tr(lds_tr16(hb + b_rd + 32 * j), lds_tr16(hb + b_rd + 32 * j + 16 * kWPitch));
#pragma unroll
      for (int j = 0; j < 8; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[j][i] = mfma_bf16(bfr[j], af[i], acc[j][i]);
    }
    }
    if (kk + 1 < nk) store(smem + ((kk + 1) & 1) * kWStage);
    __syncthreads();
  }

  if (do_cs) {
    // fold the 16 row slots (tid / 32) of each column in LDS, in a fixed order
    float* red = (float*)smem;
#pragma unroll
    for (int e = 0; e < 8; ++e) red[(tid >> 5) * 256 + (tid & 31) * 8 + e] = cs[e];
    __syncthreads();
    if (tid < 256) {
      float t = 0.f;
#pragma unroll
      for (int k = 0; k < 16; ++k) t += red[k * 256 + tid];
      if (p.split > 1) p.cs_ws[(int64_t)s * p.N2 + n20 + tid] = t;
      else p.colsum[n20 + tid] = t;
    }
  }
  if (p.split > 1) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int n1 = n10 + w1 + 16 * i + li;
      float* row = p.ws + ((int64_t)s * p.N1 + n1) * p.N2 + n20 + w2 + 4 * g;
#pragma unroll
      for (int j = 0; j < 8; ++j) *(f32x4*)(row + 16 * j) = acc[j][i];
    }
    return;
  }
  const float sc = (p.sa ? p.sa[0] : 1.f) * (p.sb ? p.sb[0] : 1.f);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int n1 = n10 + w1 + 16 * i + li;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int n2 = n20 + w2 + 16 * j + 4 * g;
      const f32x4 v = acc[j][i] * sc;
      if (p.out_f32) *(f32x4*)((float*)p.out + (int64_t)n1 * p.ldo + n2) = v;
      else *(u32x2*)((uint16_t*)p.out + (int64_t)n1 * p.ldo + n2) = u32x2{pack_bf16(v[0], v[1]), pack_bf16(v[2], v[3])};
    }
  }
}

// out[n1][n2] = sa * sb * sum_{s < split} ws[s][n1][n2], summed in split order;
// 4 consecutive n2 per thread; the threads past N1 * N2 / 4 do the same for
// the column sums (colsum[n2] = sum_s cs_ws[s][n2], unscaled).  split == 0
// writes zeros (no tokens).
__global__ void __launch_bounds__(256) wgrad_reduce_kernel(const float* __restrict__ ws, int split, int N1, int N2,
                                                           const float* __restrict__ sa,
                                                           const float* __restrict__ sb, void* __restrict__ out,
                                                           int64_t ldo, int out_f32, const float* __restrict__ cs_ws,
                                                           float* __restrict__ colsum) {
  const int64_t e = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
  const int64_t numel = (int64_t)N1 * N2;
  if (e >= numel) {
    const int64_t c = e - numel;
    if (colsum == nullptr || c >= N2) return;
    f32x4 t = zero4();
    for (int s = 0; s < split; ++s) t += *(const f32x4*)(cs_ws + (int64_t)s * N2 + c);
    *(f32x4*)(colsum + c) = t;
    return;
  }
  f32x4 acc = zero4();
  for (int s = 0; s < split; ++s) acc += *(const f32x4*)(ws + s * numel + e);
  acc *= (sa ? sa[0] : 1.f) * (sb ? sb[0] : 1.f);
  const int64_t n1 = e / N2, n2 = e - n1 * N2;
  if (out_f32) *(f32x4*)((float*)out + n1 * ldo + n2) = acc;
  else *(u32x2*)((uint16_t*)out + n1 * ldo + n2) = u32x2{pack_bf16(acc[0], acc[1]), pack_bf16(acc[2], acc[3])};
}

hipError_t set_wgrad_lds(const void* fn) {
  static std::mutex mu;
  static std::vector<const void*> done;
  std::lock_guard<std::mutex> lock(mu);
  for (const void* d : done)
    if (d == fn) return hipSuccess;
  hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, kWLds);
  if (e == hipSuccess) done.push_back(fn);
  return e;
}

// tokens per split for a requested split (<= 0: about one workgroup per CU,
// at least 4 k-steps per split), and the split that results
constexpr int kPlanKT = 128;  // token ranges are multiples of both formats' k-steps
void plan(int64_t T, int N1, int N2, int split, int64_t* tps, int* eff) {
  const int tiles = (N1 / kBN1) * (N2 / kBN2);
  if (split <= 0) split = (int)std::max<int64_t>(1, std::min<int64_t>(kCus / std::max(tiles, 1), (T + 127) / 128));
  if (T <= 0) {
    *tps = kPlanKT;
    *eff = 0;
    return;
  }
  const int64_t per = (T + split - 1) / split;
  *tps = (per + kPlanKT - 1) / kPlanKT * kPlanKT;
  *eff = (int)((T + *tps - 1) / *tps);
}

}  // namespace

extern "C" int hstu_wgrad_split(int64_t T, int N1, int N2, int split) {
  if (T < 0 || N1 <= 0 || N2 <= 0 || N1 % kBN1 || N2 % kBN2) return -1;
  int64_t tps;
  int eff;
  plan(T, N1, N2, split, &tps, &eff);
  return eff;
}

extern "C" int64_t hstu_wgrad_workspace_bytes(int64_t T, int N1, int N2, int split) {
  const int eff = hstu_wgrad_split(T, N1, N2, split);
  if (eff < 0) return -1;
  return eff > 1 ? (int64_t)eff * (N1 + 1) * N2 * 4 : 0;  // product and column-sum partials
}

extern "C" int hstu_wgrad(int a_dtype, const void* A, int64_t lda, int b_dtype, const void* B, int64_t ldb, int64_t T,
                          int N1, int N2, const float* scale_a, const float* scale_b, void* out, int64_t ldo,
                          int out_dtype, float* colsum_b, int split, void* workspace, int64_t workspace_bytes,
                          hipStream_t stream) {
  if (T < 0 || N1 <= 0 || N2 <= 0 || !out || (T > 0 && (!A || !B)) || lda < N1 || ldb < N2 || ldo < N2 ||
      (out_dtype != HSTU_DTYPE_BF16 && out_dtype != HSTU_DTYPE_FP32))
    return HSTU_E_BAD_ARG;
  const bool bf16 = a_dtype == HSTU_DTYPE_BF16 && b_dtype == HSTU_DTYPE_BF16;
  const bool f8 = a_dtype == HSTU_DTYPE_FP8_E4M3 && (b_dtype == HSTU_DTYPE_FP8_E4M3 || b_dtype == HSTU_DTYPE_FP8_E5M2);
  if (!bf16 && !f8) return HSTU_E_UNSUPPORTED;
  const int es = bf16 ? 2 : 1;
  if (colsum_b && (!bf16 || (uintptr_t)colsum_b % 16)) return HSTU_E_UNSUPPORTED;
  if (N1 % kBN1 || N2 % kBN2 || (lda * es) % 16 || (ldb * es) % 16 || ((uintptr_t)A | (uintptr_t)B) % 16 ||
      (uintptr_t)out % (out_dtype == HSTU_DTYPE_FP32 ? 16 : 8) || ldo % 4)
    return HSTU_E_UNSUPPORTED;
  int64_t tps;
  int eff;
  plan(T, N1, N2, split, &tps, &eff);
  const int64_t need = eff > 1 ? (int64_t)eff * (N1 + 1) * N2 * 4 : 0;
  if (workspace_bytes < need || (need > 0 && !workspace)) return HSTU_E_BAD_ARG;
  // one split's rows must stay within 32-bit buffer offsets
  if ((tps + kPlanKT) * std::max(lda, ldb) * es >= ((int64_t)1 << 32)) return HSTU_E_UNSUPPORTED;
  const int tiles = (N1 / kBN1) * (N2 / kBN2);
  const int out_f32 = out_dtype == HSTU_DTYPE_FP32;
  if (eff > 0) {
    WgradParams p{};
    p.A = (const uint8_t*)A;
    p.B = (const uint8_t*)B;
    p.lda = lda * es;
    p.ldb = ldb * es;
    p.T = T;
    p.tps = tps;
    p.N1 = N1;
    p.N2 = N2;
    p.split = eff;
    p.tiles_n2 = N2 / kBN2;
    p.tiles = tiles;
    p.ws = (float*)workspace;
    p.cs_ws = eff > 1 ? (float*)workspace + (int64_t)eff * N1 * N2 : nullptr;
    p.colsum = colsum_b;
    p.out = out;
    p.ldo = ldo;
    p.out_f32 = out_f32;
    p.sa = scale_a;
    p.sb = scale_b;
    const int64_t total = (int64_t)tiles * eff;
    if (total >= ((int64_t)1 << 31)) return HSTU_E_UNSUPPORTED;
    const int grid = (int)((total + 7) / 8 * 8);
    const void* kern = bf16 ? (const void*)wgrad_kernel<false, 0, 0>
                       : b_dtype == HSTU_DTYPE_FP8_E5M2 ? (const void*)wgrad_kernel<true, 0, 1>
                                                         : (const void*)wgrad_kernel<true, 0, 0>;
    hipError_t e = set_wgrad_lds(kern);
    if (e != hipSuccess) return (int)e;
    void* args[] = {&p};
    e = hipLaunchKernel(kern, dim3(grid), dim3(kWThreads), args, (size_t)kWLds, stream);
    if (e != hipSuccess) return (int)e;
  }
  if (eff != 1) {
    const int64_t threads = (int64_t)N1 * N2 / 4 + (colsum_b ? N2 / 4 : 0);
    const float* cs_ws = eff > 1 ? (const float*)workspace + (int64_t)eff * N1 * N2 : nullptr;
    hipLaunchKernelGGL(wgrad_reduce_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, stream,
                       (const float*)workspace, eff, N1, N2, scale_a, scale_b, out, ldo, out_f32, cs_ws, colsum_b);
  }
  return (int)hipGetLastError();
}
