// FP8 (OCP e4m3) projection GEMMs and the e4m3 quantizer of the HSTU layer,
// for MI355X (gfx950).
//
//   C[m][n] = epilogue( sum_k A[m][k] * W[n][k] )
//   epilogue: v = acc * sa(m) * sw(n) [+ bias[n]]; silu(v) for n in [silu_begin,
//             silu_end) (the U slice); [+ residual[m][n]]; store bf16, or e4m3 of
//             clamp(v / out_scale, +-448).
//
// A is [M, K] row-major e4m3 -- or e5m2, for the backward's gradient operand --
// (per-tensor or per-row scale), W is [N, K] row-major e4m3 (the transposed
// weight, per-tensor or per-column scale).
// Reference behaviour followed (paths relative to
// recommendation_v4/hstu/generative_recommenders/):
//   UVQK / VQK projection  ops/triton/triton_hstu_preprocess_and_attention.py:1257-1289
//   K=512 e4m3-output GEMM ops/hip/k512_fp8_gemm.cu:13-17 (acc*(sa*sb) + bias, sat448, e4m3)
//   K=1536 out-projection  ops/hip/k1536_fp8_addmm.cu:10-18 (bf16(acc*s + C))
//   SiLU on U only         ops/hstu_compute.py:140
//   quantizer              ops/triton/triton_fp8.py:396-413, 760-781 (scale = amax/448)
//   FP8 backward dgrad     ops/triton/bwd_fp8.py:1347-1395 (e5m2 dY x e4m3 W^T, per-tensor scales)
//   one-pass cast + amax   ops/triton/bwd_fp8.py:194-217, 827-866
//   cast + amax + colsum   ops/triton/bwd_fp8.py:378-434, 608-692 (quantize_amax_colsum)
//
// Design: workgroup tile 128 (M) x 128 (N), 4 waves as 2 x 2 of 64 x 64.  The
// MFMA (v_mfma_f32_16x16x128_f8f6f4) is issued operand-swapped, W rows as the
// A operand and A rows as the B operand, so a lane's C fragment holds 4
// consecutive output columns of one row (8-byte bf16 / 4-byte e4m3 stores).
// K steps of 128 stream through a 2-stage LDS ring of direct global->LDS
// loads (80 KiB per workgroup, two workgroups per CU so one's epilogue and
// loads overlap the other's MFMAs).  Rows are padded to 160 bytes and lane
// group g holds the 16-byte k-chunks g and g+4 of a row in both operands,
// which keeps the operand reads free of bank conflicts.  Tiles are numbered
// so that each XCD runs a contiguous range and the N tiles of one A row panel
// run back to back on the same XCD (A panel reuse in that XCD's L2).

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>
#include <mutex>
#include <type_traits>
#include <vector>

#include "hstu_common.h"
#include "hstu_mi355x.h"

namespace {
using namespace hstu;

struct GemmParams {
  const uint8_t* A;
  const uint8_t* W;
  int64_t lda, ldw;  // bytes
  const float* a_scale;
  const float* w_scale;
  int a_mode, w_mode;  // 0: per-tensor scalar, 1: per-row (A) / per-column (W)
  const uint16_t* bias;  // bf16 [N] or null
  const uint16_t* resid;  // bf16 [M, N] or null
  int64_t ldr;            // elements
  void* C;
  int64_t ldc;  // elements
  const float* out_scale;  // e4m3 output only
  int M, N, K;
  int silu_begin, silu_end;
  int tiles_m, tiles_n;
};

#ifndef HSTU_GEMM_REGSTAGE
#define HSTU_GEMM_REGSTAGE 1
#endif
#ifndef HSTU_GEMM_WIDE
#define HSTU_GEMM_WIDE 1
#endif
#ifndef HSTU_GEMM_DUO
#define HSTU_GEMM_DUO 1
#endif
constexpr int kBM = 128, kBN = 128, kBK = 128;
constexpr int kPitch = kBK + 32;  // 160: conflict-free operand reads
using GTile = DirectTile<128, kBK, kPitch>;  // 20 load instructions, 5 per wave
constexpr int kTileBytes = GTile::BYTES;     // 20 KiB
constexpr int kStage = 2 * kTileBytes;       // W tile then A tile
constexpr int kGemmLds = 2 * kStage;         // 80 KiB
constexpr int kCnt = 2 * GTile::PER_WAVE;    // load instructions per wave per stage

// One operand's k-step tile (128 rows x 128 bytes) staged global -> registers
// -> LDS: four 16-byte chunks per thread.  Loads issued a whole k-step ahead
// land while the MFMAs run; only the LDS store waits for them.
struct RegTile {
  u32x4 r[4];
  __device__ __forceinline__ void load(BufRsrc rs, uint32_t ld, uint32_t soff) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int c = threadIdx.x + kThreads * i, row = c >> 3, col = c & 7;
      r[i] = buf_ld128(rs, (uint32_t)row * ld + col * 16, soff);
    }
  }
  __device__ __forceinline__ void store(uint8_t* tile) const {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int c = threadIdx.x + kThreads * i, row = c >> 3, col = c & 7;
      *(u32x4*)(tile + row * kPitch + col * 16) = r[i];
    }
  }
};

__device__ __forceinline__ float bf16_to_f32(uint16_t b) { return __builtin_bit_cast(float, (uint32_t)b << 16); }

// Operand formats of the tile kernel: A and W e4m3; A e5m2 (the MFMA's B
// operand format 1, bf8) against e4m3 W; or A and W bf16, unscaled (a k-step
// of 128 bytes is then 64 elements, two v_mfma_f32_16x16x32_bf16 per operand
// pair: chunk g of a lane is elements 8g .. 8g+7 of the first 32, chunk g+4
// the same of the second 32).
enum GemmFmt { kE4M3 = 0, kE5M2A = 1, kBF16 = 2 };

// acc * s + b rounded after the multiply and after the add (no FMA), the
// e4m3-output epilogue's order (k512_fp8_gemm.cu:13-17: "MUL THEN ADD").
__device__ __forceinline__ float mul_then_add(float acc, float s, float b) {
#pragma clang fp contract(off)
  return acc * s + b;
}

template <bool E4M3_OUT, bool RESID, int FMT>
__global__ void __launch_bounds__(kThreads, 2) fp8_gemm_kernel(GemmParams p) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  // XCD-contiguous tile order: workgroup i runs on XCD i % 8.
  const int total = p.tiles_m * p.tiles_n;
  const int per_xcd = (total + 7) / 8;
  const int idx = (int)(blockIdx.x % 8) * per_xcd + (int)(blockIdx.x / 8);
  if (idx >= total) return;
  const int mt = idx / p.tiles_n, nt = idx - mt * p.tiles_n;
  const int m0 = mt * kBM, n0 = nt * kBN;

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, li = lane & 15, g = lane >> 4;
  const int wn = (wave & 1) * 64, wm = (wave >> 1) * 64;  // wave's n / m offsets in the tile

  const int mrows = min(kBM, p.M - m0);
  const BufRsrc arsrc = make_rsrc(p.A + (int64_t)m0 * p.lda, (uint32_t)((mrows - 1) * p.lda + p.K));
  const BufRsrc wrsrc = make_rsrc(p.W + (int64_t)n0 * p.ldw, (uint32_t)((kBN - 1) * p.ldw + p.K));
  GTile at, wt;
  at.init((uint32_t)p.lda);
  wt.init((uint32_t)p.ldw);
  const int nk = p.K / kBK;

  f32x4 acc[4][4];  // [n sub-tile][m sub-tile] of C^T
#pragma unroll
  for (int a = 0; a < 4; ++a)
#pragma unroll
    for (int b = 0; b < 4; ++b) acc[a][b] = zero4();

  // Epilogue operands, loaded now so their latency hides under the k-loop:
  // lane holds C[m = m0+wm+16ms+li][n = n0+wn+16ns+4g .. +3].
  float sa[4];
  f32x4 sw[4];
  u32x2 bias[4];
#pragma unroll
  for (int ms = 0; ms < 4; ++ms) {
    const int m = min(m0 + wm + 16 * ms + li, p.M - 1);
    sa[ms] = FMT == kBF16 ? 1.f : p.a_mode ? p.a_scale[m] : p.a_scale[0];
  }
#pragma unroll
  for (int ns = 0; ns < 4; ++ns) {
    const int n = n0 + wn + 16 * ns + 4 * g;
    if (FMT == kBF16) sw[ns] = f32x4{1.f, 1.f, 1.f, 1.f};
    else if (p.w_mode) sw[ns] = *(const f32x4*)(p.w_scale + n);
    else sw[ns] = f32x4{p.w_scale[0], p.w_scale[0], p.w_scale[0], p.w_scale[0]};
    bias[ns] = p.bias ? *(const u32x2*)(p.bias + n) : u32x2{0u, 0u};
  }

#if HSTU_GEMM_REGSTAGE
  RegTile wreg, areg;
  wreg.load(wrsrc, (uint32_t)p.ldw, 0);
  areg.load(arsrc, (uint32_t)p.lda, 0);
  wreg.store(smem);
  areg.store(smem + kTileBytes);
  __syncthreads();
#else
  wt.load(wrsrc, 0, smem);
  at.load(arsrc, 0, smem + kTileBytes);
  wait_vm();
  __syncthreads();
#endif

  // lane group g holds 16-byte k-chunks g and g+4 of a row
  const int w_rd = (wn + li) * kPitch + 16 * g;
  const int a_rd = kTileBytes + (wm + li) * kPitch + 16 * g;
  for (int kk = 0; kk < nk; ++kk) {
    const uint8_t* buf = smem + (kk & 1) * kStage;
    if (kk + 1 < nk) {
#if HSTU_GEMM_REGSTAGE
      wreg.load(wrsrc, (uint32_t)p.ldw, (kk + 1) * kBK);
      areg.load(arsrc, (uint32_t)p.lda, (kk + 1) * kBK);
#else
      uint8_t* nb = smem + ((kk + 1) & 1) * kStage;
      wt.load(wrsrc, (kk + 1) * kBK, nb);
      at.load(arsrc, (kk + 1) * kBK, nb + kTileBytes);
#endif
    }
    i32x8 bop[4];
#pragma unroll
    for (int ms = 0; ms < 4; ++ms) {
      const uint8_t* r = buf + a_rd + ms * 16 * kPitch;
      bop[ms] = cat8(lds_ld128(r), lds_ld128(r + 64));
    }
#pragma unroll
    for (int ns = 0; ns < 4; ++ns) {
      const uint8_t* r = buf + w_rd + ns * 16 * kPitch;
      const i32x8 aop = cat8(lds_ld128(r), lds_ld128(r + 64));
#pragma unroll
      for (int ms = 0; ms < 4; ++ms) {
        if constexpr (FMT == kE5M2A) {  // W rows e4m3 (format 0), A rows e5m2 (format 1)
          acc[ns][ms] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(aop, bop[ms], acc[ns][ms], 0, 1, 0, 0, 0, 0);
        } else if constexpr (FMT == kBF16) {
          const u32x4 alo = {(uint32_t)aop[0], (uint32_t)aop[1], (uint32_t)aop[2], (uint32_t)aop[3]};
          const u32x4 ahi = {(uint32_t)aop[4], (uint32_t)aop[5], (uint32_t)aop[6], (uint32_t)aop[7]};
          const u32x4 blo = {(uint32_t)bop[ms][0], (uint32_t)bop[ms][1], (uint32_t)bop[ms][2], (uint32_t)bop[ms][3]};
          const u32x4 bhi = {(uint32_t)bop[ms][4], (uint32_t)bop[ms][5], (uint32_t)bop[ms][6], (uint32_t)bop[ms][7]};
          acc[ns][ms] = mfma_bf16(ahi, bhi, mfma_bf16(alo, blo, acc[ns][ms]));
        } else {
          acc[ns][ms] = mfma_fp8(aop, bop[ms], acc[ns][ms]);
        }
      }
    }
#if HSTU_GEMM_REGSTAGE
    if (kk + 1 < nk) {
      uint8_t* nb = smem + ((kk + 1) & 1) * kStage;
      wreg.store(nb);
      areg.store(nb + kTileBytes);
    }
    __syncthreads();
#else
    wait_vm();
    __syncthreads();
#endif
  }

  // ---- epilogue: lane holds C[m = m0+wm+16ms+li][n = n0+wn+16ns+4g .. +3]
  const float out_s = E4M3_OUT ? p.out_scale[0] : 1.f;
#pragma unroll
  for (int ms = 0; ms < 4; ++ms) {
    const int m = m0 + wm + 16 * ms + li;
    if (m >= p.M) continue;
#pragma unroll
    for (int ns = 0; ns < 4; ++ns) {
      const int n = n0 + wn + 16 * ns + 4 * g;
      float v[4];
      {
        const u32x2 b = p.bias ? bias[ns] : u32x2{0u, 0u};
        const float bb[4] = {bf16_to_f32(b[0] & 0xffff), bf16_to_f32(b[0] >> 16), bf16_to_f32(b[1] & 0xffff),
                             bf16_to_f32(b[1] >> 16)};
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float sc = sa[ms] * sw[ns][r];
          v[r] = E4M3_OUT ? mul_then_add(acc[ns][ms][r], sc, bb[r]) : acc[ns][ms][r] * sc + bb[r];
        }
      }
      if (n < p.silu_end && n + 4 > p.silu_begin) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          if (n + r >= p.silu_begin && n + r < p.silu_end)
            v[r] = v[r] * __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(-kLog2e * v[r]));
        }
      }
      if constexpr (RESID) {
        const u32x2 c = *(const u32x2*)(p.resid + (int64_t)m * p.ldr + n);
        v[0] += bf16_to_f32(c[0] & 0xffff);
        v[1] += bf16_to_f32(c[0] >> 16);
        v[2] += bf16_to_f32(c[1] & 0xffff);
        v[3] += bf16_to_f32(c[1] >> 16);
      }
      if constexpr (E4M3_OUT) {
        float c[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) c[r] = __builtin_fminf(__builtin_fmaxf(v[r] / out_s, -448.f), 448.f);
        int w = __builtin_amdgcn_cvt_pk_fp8_f32(c[0], c[1], 0, false);
        w = __builtin_amdgcn_cvt_pk_fp8_f32(c[2], c[3], w, true);
        *(uint32_t*)((uint8_t*)p.C + (int64_t)m * p.ldc + n) = (uint32_t)w;
      } else {
        *(u32x2*)((uint16_t*)p.C + (int64_t)m * p.ldc + n) = u32x2{pack_bf16(v[0], v[1]), pack_bf16(v[2], v[3])};
      }
    }
  }
}

// W-stationary persistent form for K <= 512 (the UVQK / VQK projections and
// the K = 512 dgrad).  With K = 512 a 128 x 128 tile is only four k-steps, so
// the tile-per-workgroup kernel above spends most of its time waiting for each
// step's loads.  Here one workgroup per CU keeps its N tile's whole W panel
// (128 x K bytes) in LDS and walks a stream of M tiles (m tile s, s + streams,
// ...); the next tile's A rows are loaded into registers while the current
// tile's MFMAs and epilogue run, so a memory round trip hides behind a whole
// tile (two tiles ahead measured no faster).  8 waves as 4 (m) x 2 (n) of 32 x 64; the same operand-swapped MFMA,
// 16-byte k-chunks {g, g+4} per lane group and epilogue as above (no residual).
// With 8 | workgroups and tiles_n | workgroups / 8, the N tiles of one M
// stream run on one XCD and share its L2 for the A rows.
constexpr int kWsThreads = 512;
constexpr int kWsMaxK = 512;
constexpr int kWsPitch = kWsMaxK + 32;  // 544 = 32 mod 64: conflict-free b128 reads
constexpr int kWsPanel = 128 * kWsPitch;
constexpr int kWsLds = 2 * kWsPanel;    // W panel, A tile: 136 KiB
constexpr int kWsCus = 256;

// NK = K / 128 k-steps (compile time, so the k-loop unrolls).  The output
// leaves through LDS: after the tile's MFMAs each wave writes its 32 x 64
// sub-tile into a private slice of the (then free) A buffer and stores it back
// as whole 128-byte (bf16) or 64-byte (e4m3) row segments.
constexpr int kWsSlicePitch = 144;  // 128-byte rows + 16
template <bool E4M3_OUT, bool A_BF8, int NK>
__global__ void __launch_bounds__(kWsThreads, 1) fp8_gemm_ws_kernel(GemmParams p, int streams) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  uint8_t* const wl = smem;
  uint8_t* const al = smem + kWsPanel;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, li = lane & 15, g = lane >> 4;
  const int wm = (wave >> 1) * 32, wn = (wave & 1) * 64;
  int nt, s;
  const int per_xcd = (int)gridDim.x / 8;
  if ((int)gridDim.x % 8 == 0 && per_xcd % p.tiles_n == 0) {
    const int xcd = (int)blockIdx.x % 8, slot = (int)blockIdx.x / 8;
    nt = slot % p.tiles_n;
    s = xcd * (per_xcd / p.tiles_n) + slot / p.tiles_n;
  } else {
    nt = (int)blockIdx.x % p.tiles_n;
    s = (int)blockIdx.x / p.tiles_n;
  }
  const int n0 = nt * kBN;
  const int K = p.K, cpr = K / 16, qn = 128 * cpr / kWsThreads;  // staged chunks per thread (<= 8)

  // staging slots: chunk c = tid + 512 q of a 128-row x K-byte operand tile
  uint32_t lo[8], vw[8], va[8];
#pragma unroll
  for (int q = 0; q < 8; ++q) {
    const int c = tid + kWsThreads * q, row = c / cpr, col = c - (c / cpr) * cpr;
    lo[q] = row * kWsPitch + col * 16;
    vw[q] = row * (uint32_t)p.ldw + col * 16;
    va[q] = row * (uint32_t)p.lda + col * 16;
  }
  u32x4 st[8];
  {
    const BufRsrc wr = make_rsrc(p.W + (int64_t)n0 * p.ldw, (uint32_t)(127 * p.ldw + K));
#pragma unroll
    for (int q = 0; q < 8; ++q)
      if (q < qn) st[q] = buf_ld128(wr, vw[q], 0);
#pragma unroll
    for (int q = 0; q < 8; ++q)
      if (q < qn) *(u32x4*)(wl + lo[q]) = st[q];
  }
  auto load_a = [&](int mt) {
    const int m0 = mt * kBM, mrows = min(kBM, p.M - m0);
    const BufRsrc ar = make_rsrc(p.A + (int64_t)m0 * p.lda, (uint32_t)((mrows - 1) * p.lda + K));
#pragma unroll
    for (int q = 0; q < 8; ++q)
      if (q < qn) st[q] = buf_ld128(ar, va[q], 0);
  };
  auto store_a = [&]() {
#pragma unroll
    for (int q = 0; q < 8; ++q)
      if (q < qn) *(u32x4*)(al + lo[q]) = st[q];
  };

  // per-workgroup epilogue constants: lane's columns n0 + wn + 16 ns + 4 g .. +3
  f32x4 swv[4], bv[4];
  bool silu_any[4];
#pragma unroll
  for (int ns = 0; ns < 4; ++ns) {
    const int n = n0 + wn + 16 * ns + 4 * g;
    if (p.w_mode) swv[ns] = *(const f32x4*)(p.w_scale + n);
    else swv[ns] = f32x4{p.w_scale[0], p.w_scale[0], p.w_scale[0], p.w_scale[0]};
    if (p.bias) {
      const u32x2 b = *(const u32x2*)(p.bias + n);
      bv[ns] = f32x4{bf16_to_f32(b[0] & 0xffff), bf16_to_f32(b[0] >> 16), bf16_to_f32(b[1] & 0xffff),
                     bf16_to_f32(b[1] >> 16)};
    } else {
      bv[ns] = zero4();
    }
    silu_any[ns] = n < p.silu_end && n + 4 > p.silu_begin;
  }
  const float out_s = E4M3_OUT ? p.out_scale[0] : 1.f;

  int mt = s;
  if (mt < p.tiles_m) {
    load_a(mt);
    store_a();
  }
  __syncthreads();
  const int w_rd = (wn + li) * kWsPitch + 16 * g;
  const int a_rd = (wm + li) * kWsPitch + 16 * g;
  uint8_t* const slice = al + wave * 32 * kWsSlicePitch;
  for (; mt < p.tiles_m; mt += streams) {
    const int nxt = mt + streams;
    if (nxt < p.tiles_m) load_a(nxt);
    const int m0 = mt * kBM;
    float sa[2];
#pragma unroll
    for (int ms = 0; ms < 2; ++ms) {
      const int m = min(m0 + wm + 16 * ms + li, p.M - 1);
      sa[ms] = p.a_mode ? p.a_scale[m] : p.a_scale[0];
    }
    f32x4 acc[4][2];
#pragma unroll
    for (int a = 0; a < 4; ++a) acc[a][0] = acc[a][1] = zero4();
#pragma unroll
    for (int kk = 0; kk < NK; ++kk) {
      i32x8 bop[2];
#pragma unroll
      for (int ms = 0; ms < 2; ++ms) {
        const uint8_t* r = al + a_rd + ms * 16 * kWsPitch + kk * kBK;
        bop[ms] = cat8(lds_ld128(r), lds_ld128(r + 64));
      }
#pragma unroll
      for (int ns = 0; ns < 4; ++ns) {
        const uint8_t* r = wl + w_rd + ns * 16 * kWsPitch + kk * kBK;
        const i32x8 aop = cat8(lds_ld128(r), lds_ld128(r + 64));
#pragma unroll
        for (int ms = 0; ms < 2; ++ms) {
          if constexpr (A_BF8)
            acc[ns][ms] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(aop, bop[ms], acc[ns][ms], 0, 1, 0, 0, 0, 0);
          else
            acc[ns][ms] = mfma_fp8(aop, bop[ms], acc[ns][ms]);
        }
      }
    }
    __syncthreads();  // every wave is done with this tile's A rows: the slices are free
    // epilogue: lane holds C[m = m0 + wm + 16 ms + li][n = n0 + wn + 16 ns + 4 g .. +3];
    // slice row r = 16 ms + li, byte column (16 ns + 4 g) * element size
#pragma unroll
    for (int ms = 0; ms < 2; ++ms) {
      const int m = m0 + wm + 16 * ms + li;
#pragma unroll
      for (int ns = 0; ns < 4; ++ns) {
        const int n = n0 + wn + 16 * ns + 4 * g;
        float v[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float sc = sa[ms] * swv[ns][r];
          v[r] = E4M3_OUT ? mul_then_add(acc[ns][ms][r], sc, bv[ns][r]) : acc[ns][ms][r] * sc + bv[ns][r];
        }
        if (silu_any[ns]) {
#pragma unroll
          for (int r = 0; r < 4; ++r)
            if (n + r >= p.silu_begin && n + r < p.silu_end)
              v[r] = v[r] * __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(-kLog2e * v[r]));
        }
        if constexpr (E4M3_OUT) {
          float c[4];
#pragma unroll
          for (int r = 0; r < 4; ++r) c[r] = __builtin_fminf(__builtin_fmaxf(v[r] / out_s, -448.f), 448.f);
          int w = __builtin_amdgcn_cvt_pk_fp8_f32(c[0], c[1], 0, false);
          w = __builtin_amdgcn_cvt_pk_fp8_f32(c[2], c[3], w, true);
          *(uint32_t*)(slice + (16 * ms + li) * kWsSlicePitch + (16 * ns + 4 * g)) = (uint32_t)w;
        } else {
          *(u32x2*)(slice + (16 * ms + li) * kWsSlicePitch + (16 * ns + 4 * g) * 2) =
              u32x2{pack_bf16(v[0], v[1]), pack_bf16(v[2], v[3])};
        }
        (void)m;
      }
    }
    // the wave's own slice back as whole row segments (lane order: row-major 16-byte chunks)
    {
      constexpr int ES = E4M3_OUT ? 1 : 2, CPRW = 64 * ES / 16;  // chunks per 64-column row
#pragma unroll
      for (int i = 0; i < 32 * CPRW / 64; ++i) {
        const int c = lane + 64 * i, r = c / CPRW, cc = c - r * CPRW;
        const u32x4 d = *(const u32x4*)(slice + r * kWsSlicePitch + cc * 16);
        const int m = m0 + wm + r;
        if (m < p.M) *(u32x4*)((uint8_t*)p.C + ((int64_t)m * p.ldc + n0 + wn) * ES + cc * 16) = d;
      }
    }
    __syncthreads();  // every wave has read its slice back
    if (nxt < p.tiles_m) store_a();
    __syncthreads();
  }
}

// Persistent producer/consumer form, for N % 256 == 0, K % 256 == 0 and a
// 64-column aligned SiLU range (every FP8 projection of the layer).  At
// K = 512 the output dominates the HBM traffic, so the kernel is built to
// keep the stores streaming under the MFMAs (the epilogue's VALU work itself
// still runs between k-steps: its 128 accumulators per lane leave no
// registers for a second tile).  On gfx9 a wave's loads and stores share one in-order counter
// (vmcnt): a wave that stores a tile's output and then waits for a later
// load waits for those stores to drain first.  So the waves that store never
// load from global memory:
//  * one workgroup per CU, 5 waves: a loader wave and 4 MFMA waves.  The
//    loader only issues global -> LDS loads (buffer_load ... lds) into a
//    3-stage ring, two k-steps ahead, and stages each tile's column scales,
//    bias and row scales.  The MFMA waves only read LDS, issue MFMAs and run
//    the epilogue; their stores are never waited for.  One s_barrier per
//    k-step: the loader arrives once the step's loads have landed, the MFMA
//    waves once they have read the previous stage.
//  * workgroup tile 128 (M) x 256 (N); MFMA wave w owns all 128 rows and the
//    64 columns [64 w, 64 w + 64): per 128-byte k-step 12 operand reads (24
//    ds_read_b128) feed 32 v_mfma_f32_16x16x128_f8f6f4, issued
//    operand-swapped (W rows as the A operand) so a lane's accumulators are
//    output columns of one row.
//  * W rows are placed in LDS in a permuted order (free: it is the source
//    offset of each lane's load) so that the 16 accumulators a lane holds for
//    one output row are whole 16-byte stores: bf16 columns 8 g .. 8 g + 7 and
//    32 + 8 g .. 32 + 8 g + 7 of the wave's 64 (one store instruction writes
//    64 contiguous bytes of each of 16 rows), e4m3 columns 16 g .. 16 g + 15.
//  * XCD x walks the tile range [x * per_xcd, (x + 1) * per_xcd), numbered
//    M-panel-major, so the N tiles of one A panel run close in time on one
//    XCD and share its L2.
// An LDS operand tile is R rows x 128 bytes with the 16-byte chunk c of row r
// at position c ^ swz(r), swz(r) = ((r >> 1) & 7) ^ (((r >> 5) & 1) << 2): a
// ds_read_b128 of 16 consecutive rows (one chunk each) hits 16 distinct bank
// groups (measured conflict-free; (r & 7) ^ ((r >> 3) & 1) is not).  swz is
// constant under r -> r + 64 and flips bit 2 under r -> r + 32, so the
// operand rows 16 i + li read chunk g at (g ^ ((li >> 1) & 7)) ^ 4 ((i >> 1) & 1):
// for odd i >> 1 the chunks g and g + 4 trade places.
constexpr int kWideBN = 256;
constexpr int kPcThreads = 320;  // 4 MFMA waves + the loader
constexpr int kPcStages = 3;
constexpr int kPcA = 128 * 128;          // A item: 128 rows x 128 bytes
constexpr int kPcStage = kPcA + 256 * 128;  // + W item: 256 rows x 128 bytes = 48 KiB

__device__ __forceinline__ int wide_swz(int r) { return ((r >> 1) & 7) ^ (((r >> 5) & 1) << 2); }

// Column (within the wave's 64) of accumulator element e = 4 ns + r of lane
// group g.
template <bool E4M3_OUT>
__device__ __forceinline__ int wide_col(int g, int e) {
  if constexpr (E4M3_OUT) return 16 * g + e;
  else return e < 8 ? 8 * g + e : 32 + 8 * g + (e - 8);
}

// v / s rounded to fp32 exactly as the division, from y = 1 / s (correctly
// rounded): q0 = v y, r = v - q0 s (exact with the FMA), q = q0 + r y
// (Markstein's correction, Handbook of Floating-Point Arithmetic sec. 4.7).
// Non-finite q0 (v infinite or NaN, or v y overflowing) is kept as is.
__device__ __forceinline__ float div_by(float v, float s, float y) {
  const float q0 = v * y;
  const float q = __builtin_fmaf(__builtin_fmaf(-q0, s, v), y, q0);
  return __builtin_fabsf(q0) < __builtin_huge_valf() ? q : q0;
}

// Barriers without a memory fence (a fence would make the MFMA waves wait
// for their own stores): the MFMA waves wait for their LDS reads only, the
// loader for its loads up to the last VM outstanding ones.
__device__ __forceinline__ void pc_barrier_lds() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }
template <int VM>
__device__ __forceinline__ void pc_barrier_vm() {
  static_assert(VM == 0 || VM == 48, "loader wait counts");
  if constexpr (VM == 48) asm volatile("s_waitcnt vmcnt(48) lgkmcnt(0)\n\ts_barrier" ::: "memory");
  else asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

template <bool E4M3_OUT, bool RESID, bool A_BF8>
__global__ void __launch_bounds__(kPcThreads, 1) fp8_gemm_pc_kernel(GemmParams p, int per_xcd) {
  __shared__ __attribute__((aligned(1024))) uint8_t stage[kPcStages][kPcStage];
  // the current tile's column scales, bias and row scales
  __shared__ __attribute__((aligned(16))) float col_sw[kWideBN];
  __shared__ __attribute__((aligned(16))) uint16_t col_b[kWideBN];
  __shared__ __attribute__((aligned(16))) float row_sa[kBM];
  const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int xcd = (int)blockIdx.x & 7, gx = (int)gridDim.x >> 3;
  const int total = p.tiles_m * p.tiles_n;
  const int t0 = xcd * per_xcd + ((int)blockIdx.x >> 3);
  const int t_end = min((xcd + 1) * per_xcd, total);
  const int ntiles = t0 < t_end ? (t_end - t0 + gx - 1) / gx : 0;
  const int nk = p.K >> 7;  // even, >= 2
  const int S = ntiles * nk;  // k-steps of this workgroup
  if (S == 0) return;

  if (wave == 4) {
    // ---------------- loader: LDS slot q = 64 i + lane of an item is row
    // q >> 3, position q & 7, which holds chunk (q & 7) ^ swz(row)
    uint32_t av[16], wv[32];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int q = 64 * i + lane, r = q >> 3;
      av[i] = (uint32_t)r * (uint32_t)p.lda + (((q & 7) ^ wide_swz(r)) * 16);
    }
#pragma unroll
    for (int i = 0; i < 32; ++i) {
      const int q = 64 * i + lane, j = q >> 3, jj = j & 15;
      const int col = 64 * (j >> 6) + wide_col<E4M3_OUT>(jj >> 2, 4 * ((j >> 4) & 3) + (jj & 3));
      wv[i] = (uint32_t)col * (uint32_t)p.ldw + (((q & 7) ^ wide_swz(j)) * 16);
    }
    const BufRsrc wrs = make_rsrc(p.W, (uint32_t)((int64_t)(p.N - 1) * p.ldw + p.K));
    auto issue = [&](int s) {
      const int t = t0 + (s / nk) * gx, kk = s - (s / nk) * nk;
      const int mt = t / p.tiles_n, nt = t - mt * p.tiles_n;
      const int m0 = mt * kBM, mrows = min(kBM, p.M - m0);
      // rows past M read as zero (the range check covers the vector offset)
      const BufRsrc ars = make_rsrc(p.A + (int64_t)m0 * p.lda, (uint32_t)((mrows - 1) * p.lda + p.K));
      uint8_t* st = stage[s % kPcStages];
#pragma unroll
      for (int i = 0; i < 16; ++i) buf_to_lds<16>(ars, st + 1024 * i, av[i], kk * 128);
      const uint32_t wso = (uint32_t)(nt * kWideBN) * (uint32_t)p.ldw + kk * 128;
#pragma unroll
      for (int i = 0; i < 32; ++i) buf_to_lds<16>(wrs, st + kPcA + 1024 * i, wv[i], wso);
    };
    issue(0);
    if (S > 1) {
      issue(1);
      pc_barrier_vm<48>();
    } else {
      pc_barrier_vm<0>();
    }
    // The tile's constants, also as LDS loads (the loader's only memory
    // operations are LDS loads, so its waits count them exactly): column
    // scales (replicated for a per-tensor scale), bias (zero without one) and
    // row scales, read in the tile's epilogue, after barrier s + 1.
    const BufRsrc swr = make_rsrc(p.w_scale, p.w_mode ? (uint32_t)p.N * 4u : 4u);
    const BufRsrc bsr = make_rsrc(p.bias, p.bias ? (uint32_t)p.N * 2u : 0u);
    const BufRsrc sar = make_rsrc(p.a_scale, p.a_mode ? (uint32_t)p.M * 4u : 4u);
    for (int s = 0; s < S; ++s) {
      // after barrier s: step s is readable, the stage of step s - 1 is free
      const int tile_i = s / nk, kk = s - tile_i * nk;
      if (kk == 0) {
        const int t = t0 + tile_i * gx, mt = t / p.tiles_n, nt = t - mt * p.tiles_n;
        const int n0 = nt * kWideBN, m0 = mt * kBM;
#pragma unroll
        for (int i = 0; i < 4; ++i)
          buf_to_lds<4>(swr, (uint8_t*)col_sw + 256 * i, p.w_mode ? (uint32_t)(n0 + 64 * i + lane) * 4u : 0u, 0);
#pragma unroll
        for (int i = 0; i < 2; ++i) buf_to_lds<4>(bsr, (uint8_t*)col_b + 256 * i, (uint32_t)(n0 + 128 * i + 2 * lane) * 2u, 0);
#pragma unroll
        for (int i = 0; i < 2; ++i)
          buf_to_lds<4>(sar, (uint8_t*)row_sa + 256 * i, p.a_mode ? (uint32_t)min(m0 + 64 * i + lane, p.M - 1) * 4u : 0u, 0);
      }
      if (s + 2 < S) {
        issue(s + 2);
        pc_barrier_vm<48>();  // all but step s + 2's loads: step s + 1 and the constants
      } else if (s + 1 < S) {
        pc_barrier_vm<0>();
      }
    }
    return;
  }

  // ---------------- MFMA waves
  const int li = lane & 15, g = lane >> 4;
  // chunks g and g + 4 of operand row li (rows 16 i + li with (i >> 1) even;
  // odd: the two trade places)
  const uint32_t a_rd0 = li * 128 + ((g ^ wide_swz(li)) * 16);
  const uint32_t a_rd1 = li * 128 + (((g + 4) ^ wide_swz(li)) * 16);
  const uint32_t w_rd0 = kPcA + 64 * wave * 128 + a_rd0, w_rd1 = kPcA + 64 * wave * 128 + a_rd1;

  f32x4 acc[8][4];
  // epilogue: lane holds C[m0 + 16 ms + li][n0 + 64 wave + wide_col(g, e)],
  // e = 4 ns + r: the runs c0 + (0..7) (e < 8) and c1 + (0..7) (e >= 8).
  // Stores (and residual loads) go through buffer resources bounded at the
  // tile's valid rows: rows past M are dropped by the range check.
  auto epilogue = [&](int m0, int n0) {
    constexpr int ES = E4M3_OUT ? 1 : 2;
    const int vrows = min(kBM, p.M - m0);
    const BufRsrc crs = make_rsrc((uint8_t*)p.C + (int64_t)m0 * p.ldc * ES, (uint32_t)(vrows * p.ldc * ES));
    const BufRsrc rrs = make_rsrc(RESID ? (const void*)(p.resid + (int64_t)m0 * p.ldr) : p.C,
                                  RESID ? (uint32_t)(vrows * p.ldr * 2) : 0u);
    const float os = E4M3_OUT ? p.out_scale[0] : 1.f;
    const float oy = E4M3_OUT ? 1.f / os : 1.f;
    const int cl0 = 64 * wave + (E4M3_OUT ? 16 * g : 8 * g);
    const int cl1 = cl0 + (E4M3_OUT ? 8 : 32);
    // SiLU on the wave's 64 columns or on none of them: the host takes this
    // form only for a 64-column aligned [silu_begin, silu_end) (the U slice)
    const int wc0 = n0 + 64 * wave;
    const bool silu = wc0 >= p.silu_begin && wc0 < p.silu_end;
#pragma unroll
    for (int ms = 0; ms < 8; ++ms) {
      const int r = 16 * ms + li;  // row within the tile
      const float sa = row_sa[r];
      float v[16];
#pragma unroll
      for (int run = 0; run < 2; ++run) {
        const int cl = run ? cl1 : cl0, c = n0 + cl;
        const f32x4 x0 = *(const f32x4*)(col_sw + cl), x1 = *(const f32x4*)(col_sw + cl + 4);
        const u32x4 b = *(const u32x4*)(col_b + cl);
        const float sw[8] = {x0[0], x0[1], x0[2], x0[3], x1[0], x1[1], x1[2], x1[3]};
        float* o = v + 8 * run;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float bb = bf16_to_f32(e & 1 ? (uint16_t)(b[e >> 1] >> 16) : (uint16_t)(b[e >> 1] & 0xffff));
          const float a = acc[ms][2 * run + (e >> 2)][e & 3];
          o[e] = E4M3_OUT ? mul_then_add(a, sa * sw[e], bb) : a * (sa * sw[e]) + bb;
        }
        if (silu) {
#pragma unroll
          for (int e = 0; e < 8; ++e) o[e] = o[e] * __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(-kLog2e * o[e]));
        }
        if constexpr (RESID) {
          const u32x4 rv = buf_ld128(rrs, (uint32_t)(r * p.ldr + c) * 2, 0);
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            o[2 * j] += bf16_to_f32(rv[j] & 0xffff);
            o[2 * j + 1] += bf16_to_f32(rv[j] >> 16);
          }
        }
        if constexpr (!E4M3_OUT) {
          __builtin_amdgcn_raw_buffer_store_b128(
              u32x4{pack_bf16(o[0], o[1]), pack_bf16(o[2], o[3]), pack_bf16(o[4], o[5]), pack_bf16(o[6], o[7])}, crs,
              (uint32_t)(r * p.ldc + c) * 2, 0, 0);
        }
      }
      if constexpr (E4M3_OUT) {  // the lane's 16 columns are contiguous: one 16-byte store
        uint32_t w[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          float q[4];
#pragma unroll
          for (int k = 0; k < 4; ++k)
            q[k] = __builtin_fminf(__builtin_fmaxf(os == 1.f ? v[4 * j + k] : div_by(v[4 * j + k], os, oy), -448.f),
                                   448.f);
          w[j] = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(q[2], q[3], __builtin_amdgcn_cvt_pk_fp8_f32(q[0], q[1], 0, false),
                                                           true);
        }
        __builtin_amdgcn_raw_buffer_store_b128(u32x4{w[0], w[1], w[2], w[3]}, crs, (uint32_t)(r * p.ldc + n0 + cl0), 0, 0);
      }
    }
  };

  for (int s = 0; s < S; ++s) {
    const int tile_i = s / nk, kk = s - tile_i * nk;
    pc_barrier_lds();  // step s has landed; every wave is done with step s - 1
    if (kk == 0) {
#pragma unroll
      for (int ms = 0; ms < 8; ++ms)
#pragma unroll
        for (int ns = 0; ns < 4; ++ns) acc[ms][ns] = zero4();
    }
    const uint8_t* st = stage[s % kPcStages];
    i32x8 w[4];
#pragma unroll
    for (int ns = 0; ns < 4; ++ns) {
      const uint32_t lo = ns & 2 ? w_rd1 : w_rd0, hi = ns & 2 ? w_rd0 : w_rd1;
      w[ns] = cat8(lds_ld128(st + lo + 2048 * ns), lds_ld128(st + hi + 2048 * ns));
    }
#pragma unroll
    for (int ms = 0; ms < 8; ++ms) {
      const uint32_t lo = ms & 2 ? a_rd1 : a_rd0, hi = ms & 2 ? a_rd0 : a_rd1;
      const i32x8 b = cat8(lds_ld128(st + lo + 2048 * ms), lds_ld128(st + hi + 2048 * ms));
#pragma unroll
      for (int ns = 0; ns < 4; ++ns) {
        if constexpr (A_BF8)  // W e4m3 (format 0), A e5m2 (format 1)
          acc[ms][ns] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(w[ns], b, acc[ms][ns], 0, 1, 0, 0, 0, 0);
        else
          acc[ms][ns] = mfma_fp8(w[ns], b, acc[ms][ns]);
      }
    }
    if (kk == nk - 1) {
      const int t = t0 + tile_i * gx, mt = t / p.tiles_n;
      epilogue(mt * kBM, (t - mt * p.tiles_n) * kWideBN);
    }
  }
}

// ---------------------------------------------------------------- two-workgroup form
// The producer/consumer form runs each tile's epilogue after its last k-step
// with one MFMA wave per SIMD, so the SIMD's MFMA pipe idles for the
// epilogue's length (at K = 512 about as long as the k-steps).  This form
// keeps the tile (128 x 256), the operand layout and the epilogue, and puts two
// workgroups on each CU instead, so one workgroup's epilogue runs while the
// other's MFMAs do:
//  * one tile per workgroup, 4 waves (wave w owns all 128 rows and the 64
//    columns [64 w, 64 w + 64)), at most 128 accumulators + 96 operand
//    registers: two waves per SIMD.
//  * 80 KiB of LDS: a ring of 5 slots of 16 KiB.  Each k-step has three
//    items, A (128 rows x 128 bytes), W0 (the tile's W rows 0-127, read by
//    waves 0 and 1) and W1 (rows 128-255, waves 2 and 3); item i lives in
//    slot i mod 5.  The prologue issues items 0-4; k-step s issues items
//    3 s + 5 .. 3 s + 7 once every wave has read its own three, so A and W0
//    go two k-steps ahead and W1 (an L2 hit: all tiles share W) one.
//  * every wave issues a quarter of each item (4 LDS DMAs of 1 KiB).  The
//    DMAs are inline assembly, invisible to the compiler (which would
//    otherwise wait for all of them before every LDS read); their waits are
//    the explicit vmcnt below, exact because nothing else of the wave's
//    vector memory operations is outstanding in the k-loop.
//  * the epilogue's constants (the lane's column scales and bias, its rows'
//    scales) are loaded to registers at the last k-step, once no DMA is left.
constexpr int kDuoThreads = 256;
constexpr int kDuoItem = 128 * 128;  // 16 KiB
constexpr int kDuoSlots = 5;         // 80 KiB: two workgroups per CU

typedef int i32x4 __attribute__((ext_vector_type(4)));
// make_rsrc's descriptor as four scalar registers, for inline assembly
__device__ __forceinline__ i32x4 rsrc_sgprs(const void* base, uint32_t bytes) {
  const uint64_t a = (uint64_t)(uintptr_t)base;
  i32x4 r;
  r[0] = __builtin_amdgcn_readfirstlane((int)(uint32_t)a);
  r[1] = __builtin_amdgcn_readfirstlane((int)((uint32_t)(a >> 32) & 0xffffu));  // stride 0
  r[2] = __builtin_amdgcn_readfirstlane((int)bytes);
  r[3] = 0x00020000;
  return r;
}
// 4 x 16 bytes per lane from the buffer to LDS: load j writes lds + 1024 j +
// 16 lane, from voffset v[j] + soff.  M0 is saved and restored.
__device__ __forceinline__ void duo_dma4(uint32_t lds, const uint32_t (&v)[4], i32x4 r, uint32_t soff) {
  uint32_t saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %1\n\ts_nop 0\n\tbuffer_load_dwordx4 %2, %6, %7 offen lds\n\t"
      "s_add_u32 m0, m0, 0x400\n\ts_nop 0\n\tbuffer_load_dwordx4 %3, %6, %7 offen lds\n\t"
      "s_add_u32 m0, m0, 0x400\n\ts_nop 0\n\tbuffer_load_dwordx4 %4, %6, %7 offen lds\n\t"
      "s_add_u32 m0, m0, 0x400\n\ts_nop 0\n\tbuffer_load_dwordx4 %5, %6, %7 offen lds\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(saved)
      : "s"(lds), "v"(v[0]), "v"(v[1]), "v"(v[2]), "v"(v[3]), "s"(r), "s"(soff)
      : "memory", "scc");
}
// At most VM of this wave's vector-memory operations outstanding and its LDS
// operations done, then s_barrier.
template <int VM>
__device__ __forceinline__ void duo_barrier() {
  asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(VM) : "memory");
}

template <bool E4M3_OUT, bool RESID, bool A_BF8>
__global__ void __launch_bounds__(kDuoThreads, 2) fp8_gemm_duo_kernel(GemmParams p, int per_xcd) {
  __shared__ __attribute__((aligned(1024))) uint8_t ring[kDuoSlots][kDuoItem];
  const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  // XCD x runs the tile range [x per_xcd, (x + 1) per_xcd), M-panel-major:
  // the N tiles of one A panel run close in time and share the XCD's L2
  const int xcd = (int)blockIdx.x & 7;
  const int t = xcd * per_xcd + ((int)blockIdx.x >> 3);
  if (t >= min((xcd + 1) * per_xcd, p.tiles_m * p.tiles_n)) return;
  const int mt = t / p.tiles_n, nt = t - mt * p.tiles_n;
  const int m0 = mt * kBM, n0 = nt * kWideBN, mrows = min(kBM, p.M - m0);
  const int nk = p.K >> 7;

  // DMA sources of this wave's chunks 4 wave + j of an item: LDS slot
  // q = 64 i + lane is row q >> 3, position q & 7, which holds chunk
  // (q & 7) ^ swz(row); W item h row r is the tile's W row 128 h + r, placed
  // in the permuted column order (swz is the same for r and 128 + r)
  uint32_t av[4], wv[2][4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int q = 64 * (4 * wave + j) + lane, r = q >> 3;
    const uint32_t pos = (uint32_t)(((q & 7) ^ wide_swz(r)) * 16);
    av[j] = (uint32_t)r * (uint32_t)p.lda + pos;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int jr = 128 * h + r, jj = jr & 15;
      const int col = 64 * (jr >> 6) + wide_col<E4M3_OUT>(jj >> 2, 4 * ((jr >> 4) & 3) + (jj & 3));
      wv[h][j] = (uint32_t)col * (uint32_t)p.ldw + pos;
    }
  }
  // rows past M read as zero (the range check covers the vector offset)
  const i32x4 ars = rsrc_sgprs(p.A + (int64_t)m0 * p.lda, (uint32_t)((mrows - 1) * p.lda + p.K));
  const i32x4 wrs = rsrc_sgprs(p.W + (int64_t)n0 * p.ldw, (uint32_t)((kWideBN - 1) * p.ldw + p.K));
  const uint32_t ring0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) const uint8_t*)&ring[0][0];
  const int nitems = 3 * nk;
  auto issue = [&](int it) {  // item it: k-step it / 3; 0 A, 1 W0, 2 W1
    const int s = it / 3, kind = it - 3 * s;
    const uint32_t dst = __builtin_amdgcn_readfirstlane(ring0 + (uint32_t)((it % kDuoSlots) * kDuoItem + 4096 * wave));
    if (kind == 0) duo_dma4(dst, av, ars, (uint32_t)(s * 128));
    else duo_dma4(dst, wv[kind - 1], wrs, (uint32_t)(s * 128));
  };
  for (int it = 0; it < min(5, nitems); ++it) issue(it);

  const int li = lane & 15, g = lane >> 4;
  // chunks g and g + 4 of operand row li (rows 16 i + li with (i >> 1) even;
  // odd: the two trade places)
  const uint32_t a_rd0 = li * 128 + ((g ^ wide_swz(li)) * 16);
  const uint32_t a_rd1 = li * 128 + (((g + 4) ^ wide_swz(li)) * 16);
  const uint32_t w_off = 64 * (wave & 1) * 128;

  // epilogue constants of the lane's 16 columns (runs c0 + 0..7, c1 + 0..7)
  // and 8 rows (16 ms + li)
  const int cl0 = 64 * wave + (E4M3_OUT ? 16 * g : 8 * g);
  const int cl1 = cl0 + (E4M3_OUT ? 8 : 32);
  f32x4 swv[4];
  u32x4 bv[2];
  float sav[8];
  auto load_consts = [&]() {
    const BufRsrc swr = make_rsrc(p.w_scale, (uint32_t)p.N * 4u);
    const BufRsrc bsr = make_rsrc(p.bias, p.bias ? (uint32_t)p.N * 2u : 0u);
    if (p.w_mode) {
#pragma unroll
      for (int run = 0; run < 2; ++run) {
        const uint32_t c = (uint32_t)(n0 + (run ? cl1 : cl0));
        swv[2 * run] = __builtin_bit_cast(f32x4, buf_ld128(swr, c * 4u, 0));
        swv[2 * run + 1] = __builtin_bit_cast(f32x4, buf_ld128(swr, c * 4u + 16u, 0));
      }
    } else {
      const float s0 = p.w_scale[0];
#pragma unroll
      for (int i = 0; i < 4; ++i) swv[i] = f32x4{s0, s0, s0, s0};
    }
#pragma unroll
    for (int run = 0; run < 2; ++run) bv[run] = buf_ld128(bsr, (uint32_t)(n0 + (run ? cl1 : cl0)) * 2u, 0);
    if (p.a_mode) {
      const BufRsrc sar = make_rsrc(p.a_scale, (uint32_t)p.M * 4u);
#pragma unroll
      for (int ms = 0; ms < 8; ++ms) sav[ms] = buf_ldf(sar, (uint32_t)min(m0 + 16 * ms + li, p.M - 1) * 4u, 0);
    } else {
      const float s0 = p.a_scale[0];
#pragma unroll
      for (int ms = 0; ms < 8; ++ms) sav[ms] = s0;
    }
  };

  f32x4 acc[8][4];
  auto mfma_rows = [&](const i32x8 (&w)[4], const i32x8 (&a)[4], int ms0, bool first) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int ns = 0; ns < 4; ++ns) {
        const f32x4 c = first ? zero4() : acc[ms0 + i][ns];
        if constexpr (A_BF8)  // W e4m3 (format 0), A e5m2 (format 1)
          acc[ms0 + i][ns] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(w[ns], a[i], c, 0, 1, 0, 0, 0, 0);
        else
          acc[ms0 + i][ns] = mfma_fp8(w[ns], a[i], c);
      }
  };
  auto read_a = [&](const uint8_t* st, int ms0, i32x8 (&a)[4]) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int ms = ms0 + i;
      const uint32_t lo = ms & 2 ? a_rd1 : a_rd0, hi = ms & 2 ? a_rd0 : a_rd1;
      a[i] = cat8(lds_ld128(st + lo + 2048 * ms), lds_ld128(st + hi + 2048 * ms));
    }
  };
  // one k-step (FIRST: accumulators start at zero; LAST: no items left to
  // issue, the epilogue constants are loaded instead)
  auto kstep = [&](int s, auto first_c, auto last_c) {
    constexpr bool FIRST = decltype(first_c)::value, LAST = decltype(last_c)::value;
    // this wave's items of step s have landed (issued after them: items
    // 3 s + 3, 3 s + 4, if step s + 1 exists), then every wave's
    if constexpr (LAST) duo_barrier<0>();
    else duo_barrier<8>();
    const uint8_t* sa_ = ring[(3 * s) % kDuoSlots];
    const uint8_t* sw_ = ring[(3 * s + 1 + (wave >> 1)) % kDuoSlots] + w_off;
    i32x8 w[4], a0[4], a1[4];
#pragma unroll
    for (int ns = 0; ns < 4; ++ns) {
      const uint32_t lo = ns & 2 ? a_rd1 : a_rd0, hi = ns & 2 ? a_rd0 : a_rd1;
      w[ns] = cat8(lds_ld128(sw_ + lo + 2048 * ns), lds_ld128(sw_ + hi + 2048 * ns));
    }
    read_a(sa_, 0, a0);
    mfma_rows(w, a0, 0, FIRST);
    read_a(sa_, 4, a1);
    duo_barrier<0>();  // every wave has read step s: its three slots are free
    if constexpr (LAST) {
      load_consts();
    } else {
#pragma unroll
      for (int k = 5; k < 8; ++k)
        if (3 * s + k < nitems) issue(3 * s + k);
    }
    mfma_rows(w, a1, 4, FIRST);
  };
  kstep(0, std::true_type{}, std::false_type{});
  for (int s = 1; s < nk - 1; ++s) kstep(s, std::false_type{}, std::false_type{});
  kstep(nk - 1, std::false_type{}, std::true_type{});

  // epilogue: lane holds C[m0 + 16 ms + li][n0 + 64 wave + wide_col(g, e)],
  // e = 4 ns + r: the runs c0 + (0..7) (e < 8) and c1 + (0..7) (e >= 8).
  // Stores (and residual loads) go through buffer resources bounded at the
  // tile's valid rows: rows past M are dropped by the range check.
  constexpr int ES = E4M3_OUT ? 1 : 2;
  const BufRsrc crs = make_rsrc((uint8_t*)p.C + (int64_t)m0 * p.ldc * ES, (uint32_t)(mrows * p.ldc * ES));
  const BufRsrc rrs = make_rsrc(RESID ? (const void*)(p.resid + (int64_t)m0 * p.ldr) : p.C,
                                RESID ? (uint32_t)(mrows * p.ldr * 2) : 0u);
  const float os = E4M3_OUT ? p.out_scale[0] : 1.f;
  const float oy = E4M3_OUT ? 1.f / os : 1.f;
  const int wc0 = n0 + 64 * wave;
  const bool silu = wc0 >= p.silu_begin && wc0 < p.silu_end;
#pragma unroll
  for (int ms = 0; ms < 8; ++ms) {
    const int r = 16 * ms + li;
    float v[16];
#pragma unroll
    for (int run = 0; run < 2; ++run) {
      const int c = n0 + (run ? cl1 : cl0);
      const f32x4 x0 = swv[2 * run], x1 = swv[2 * run + 1];
      const u32x4 b = bv[run];
      const float sw[8] = {x0[0], x0[1], x0[2], x0[3], x1[0], x1[1], x1[2], x1[3]};
      float* o = v + 8 * run;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float bb = bf16_to_f32(e & 1 ? (uint16_t)(b[e >> 1] >> 16) : (uint16_t)(b[e >> 1] & 0xffff));
        const float a = acc[ms][2 * run + (e >> 2)][e & 3];
        o[e] = E4M3_OUT ? mul_then_add(a, sav[ms] * sw[e], bb) : a * (sav[ms] * sw[e]) + bb;
      }
      if (silu) {
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] = o[e] * __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(-kLog2e * o[e]));
      }
      if constexpr (RESID) {
        const u32x4 rv = buf_ld128(rrs, (uint32_t)(r * p.ldr + c) * 2, 0);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          o[2 * j] += bf16_to_f32(rv[j] & 0xffff);
          o[2 * j + 1] += bf16_to_f32(rv[j] >> 16);
        }
      }
      if constexpr (!E4M3_OUT) {
        __builtin_amdgcn_raw_buffer_store_b128(
            u32x4{pack_bf16(o[0], o[1]), pack_bf16(o[2], o[3]), pack_bf16(o[4], o[5]), pack_bf16(o[6], o[7])}, crs,
            (uint32_t)(r * p.ldc + c) * 2, 0, 0);
      }
    }
    if constexpr (E4M3_OUT) {  // the lane's 16 columns are contiguous: one 16-byte store
      uint32_t w[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        float q[4];
#pragma unroll
        for (int k = 0; k < 4; ++k)
          q[k] = __builtin_fminf(__builtin_fmaxf(os == 1.f ? v[4 * j + k] : div_by(v[4 * j + k], os, oy), -448.f),
                                 448.f);
        w[j] = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(q[2], q[3], __builtin_amdgcn_cvt_pk_fp8_f32(q[0], q[1], 0, false),
                                                         true);
      }
      __builtin_amdgcn_raw_buffer_store_b128(u32x4{w[0], w[1], w[2], w[3]}, crs, (uint32_t)(r * p.ldc + n0 + cl0), 0, 0);
    }
  }
}

// Per-group e4m3 quantization of bf16 rows: scale = amax/448 over each group
// of `group` consecutive elements (1/448 for an all-zero group), out =
// e4m3(clamp(x / scale, +-448)).  One wave per (row, group); group <= 4096 and
// a multiple of 8.  With a given per-tensor scale (scale_in != null) no amax
// is taken.
__global__ void quantize_e4m3_kernel(const uint16_t* x, int64_t ldx, int rows, int cols, int group,
                                     const float* scale_in, uint8_t* out, int64_t ldo, float* scale_out) {
  const int groups_per_row = cols / group;
  const int gid = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (gid >= rows * groups_per_row) return;
  const int lane = threadIdx.x & 63;
  const int row = gid / groups_per_row, gc = (gid - row * groups_per_row) * group;
  const uint16_t* src = x + (int64_t)row * ldx + gc;
  // each lane handles 8-element chunks lane, lane+64, ...
  float amax = 0.f;
  constexpr int kMaxCh = 8;  // 8-element chunks per lane (group <= 8 * 8 * 64)
  u32x4 chunk[kMaxCh];
  const int nch = group / 8;
#pragma unroll
  for (int c = 0; c < kMaxCh; ++c) {
    const int ch = lane + 64 * c;
    chunk[c] = u32x4{0u, 0u, 0u, 0u};
    if (ch < nch) chunk[c] = *(const u32x4*)(src + ch * 8);
    if (!scale_in) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        amax = __builtin_fmaxf(amax, __builtin_fabsf(bf16_to_f32(chunk[c][e] & 0xffff)));
        amax = __builtin_fmaxf(amax, __builtin_fabsf(bf16_to_f32(chunk[c][e] >> 16)));
      }
    }
  }
  float scale;
  if (scale_in) {
    scale = scale_in[0];
  } else {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) amax = __builtin_fmaxf(amax, __shfl_xor(amax, off));
    scale = amax > 0.f ? amax / 448.f : 1.f / 448.f;
    if (lane == 0) scale_out[gid] = scale;
  }
  uint8_t* dst = out + (int64_t)row * ldo + gc;
#pragma unroll
  for (int c = 0; c < kMaxCh; ++c) {
    const int ch = lane + 64 * c;
    if (ch >= nch) continue;
    float f[8];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      // true division, as the reference quantizer computes value / scale
      f[2 * e] = __builtin_fminf(__builtin_fmaxf(bf16_to_f32(chunk[c][e] & 0xffff) / scale, -448.f), 448.f);
      f[2 * e + 1] = __builtin_fminf(__builtin_fmaxf(bf16_to_f32(chunk[c][e] >> 16) / scale, -448.f), 448.f);
    }
    int lo = __builtin_amdgcn_cvt_pk_fp8_f32(f[0], f[1], 0, false);
    lo = __builtin_amdgcn_cvt_pk_fp8_f32(f[2], f[3], lo, true);
    int hi = __builtin_amdgcn_cvt_pk_fp8_f32(f[4], f[5], 0, false);
    hi = __builtin_amdgcn_cvt_pk_fp8_f32(f[6], f[7], hi, true);
    *(u32x2*)(dst + ch * 8) = u32x2{(uint32_t)lo, (uint32_t)hi};
  }
}

// One-pass FP8 cast with the amax of the input: out = fp8(clamp(x * inv_scale,
// +-limit)) (e4m3 or e5m2, RNE) over n contiguous elements, and per 8192-element
// block the max |x| (before scaling) into partial[block].  A thread casts 32
// consecutive elements: 4 (bf16) or 8 (fp32) 16-byte loads, two 16-byte stores.
constexpr int kCastBlock = 8192;
template <bool IN_F32, bool OUT_BF8>
__global__ void __launch_bounds__(256) cast_fp8_amax_kernel(const uint8_t* __restrict__ x, int64_t n,
                                                            const float* __restrict__ inv_scale, float limit,
                                                            uint8_t* __restrict__ out, float* __restrict__ partial) {
  constexpr int ES = IN_F32 ? 4 : 2, NL = 32 * ES / 16;
  __shared__ float red[4];
  const int tid = threadIdx.x;
  const int64_t e0 = (int64_t)blockIdx.x * kCastBlock + (int64_t)tid * 32;
  u32x4 w[NL];
#pragma unroll
  for (int i = 0; i < NL; ++i) {
    const int64_t e = e0 + i * (16 / ES);
    w[i] = e < n ? *(const u32x4*)(x + e * ES) : u32x4{0u, 0u, 0u, 0u};
  }
  const float s = inv_scale[0];
  float amax = 0.f, v[32];
#pragma unroll
  for (int i = 0; i < NL; ++i) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t u = w[i][j];
      if constexpr (IN_F32) {
        v[4 * i + j] = __builtin_bit_cast(float, u);
      } else {
        v[8 * i + 2 * j] = __builtin_bit_cast(float, u << 16);
        v[8 * i + 2 * j + 1] = __builtin_bit_cast(float, u & 0xffff0000u);
      }
    }
  }
#pragma unroll
  for (int k = 0; k < 32; ++k) amax = __builtin_fmaxf(amax, __builtin_fabsf(v[k]));
  if (e0 < n) {
    uint32_t o[8];
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      float c[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) c[r] = __builtin_fminf(__builtin_fmaxf(v[4 * q + r] * s, -limit), limit);
      int t;
      if constexpr (OUT_BF8) {
        t = __builtin_amdgcn_cvt_pk_bf8_f32(c[0], c[1], 0, false);
        t = __builtin_amdgcn_cvt_pk_bf8_f32(c[2], c[3], t, true);
      } else {
        t = __builtin_amdgcn_cvt_pk_fp8_f32(c[0], c[1], 0, false);
        t = __builtin_amdgcn_cvt_pk_fp8_f32(c[2], c[3], t, true);
      }
      o[q] = (uint32_t)t;
    }
    // n % 32 == 0, so a thread's 32 elements are all in range or all out
    *(u32x4*)(out + e0) = u32x4{o[0], o[1], o[2], o[3]};
    *(u32x4*)(out + e0 + 16) = u32x4{o[4], o[5], o[6], o[7]};
  }
  // block max: wave reduction, then four waves through LDS
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) amax = __builtin_fmaxf(amax, __shfl_xor(amax, off));
  if ((tid & 63) == 0) red[tid >> 6] = amax;
  __syncthreads();
  if (tid == 0) partial[blockIdx.x] = __builtin_fmaxf(__builtin_fmaxf(red[0], red[1]), __builtin_fmaxf(red[2], red[3]));
}

// max(a, b) that returns NaN when either is NaN (torch.maximum / amax).
__device__ __forceinline__ float max_nan(float a, float b) { return a != a ? a : (b != b || b > a ? b : a); }

// The 32 elements a thread of the 8192-element cast blocks handles, as fp32.
// Vector elements go through a scalar before __builtin_bit_cast: bit-casting
// an ext-vector element lvalue reads element 0 whatever the index.
template <bool IN_F32>
__device__ __forceinline__ void load32(const uint8_t* __restrict__ x, int64_t n, int64_t e0, float (&v)[32]) {
  constexpr int ES = IN_F32 ? 4 : 2, NL = 32 * ES / 16;
  u32x4 w[NL];
#pragma unroll
  for (int i = 0; i < NL; ++i) {
    const int64_t e = e0 + i * (16 / ES);
    w[i] = e < n ? *(const u32x4*)(x + e * ES) : u32x4{0u, 0u, 0u, 0u};
  }
#pragma unroll
  for (int i = 0; i < NL; ++i) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t u = w[i][j];
      if constexpr (IN_F32) {
        v[4 * i + j] = __builtin_bit_cast(float, u);
      } else {
        v[8 * i + 2 * j] = __builtin_bit_cast(float, u << 16);
        v[8 * i + 2 * j + 1] = __builtin_bit_cast(float, u & 0xffff0000u);
      }
    }
  }
}

// Unit-margin e4m3 quantization of a whole tensor (the dgrad's weight):
// scale = max(amax |x|, 1e-30) * fp32(1 / 448) (torch divides a tensor by a
// host scalar as a product with the scalar's fp32 reciprocal), out =
// e4m3(clamp(x * (1 / scale), +-448)) with 1 / scale correctly rounded (its
// reciprocal kernel).  Pass 1: per 8192-element block the max |x| (NaN
// propagates, as torch.amax) into partial[block].
template <bool IN_F32>
__global__ void __launch_bounds__(256) absmax_partials_kernel(const uint8_t* __restrict__ x, int64_t n,
                                                              float* __restrict__ partial) {
  __shared__ float red[4];
  const int tid = threadIdx.x;
  float v[32];
  load32<IN_F32>(x, n, (int64_t)blockIdx.x * kCastBlock + (int64_t)tid * 32, v);
  float m = 0.f;
#pragma unroll
  for (int k = 0; k < 32; ++k) m = max_nan(m, __builtin_fabsf(v[k]));
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) m = max_nan(m, __shfl_xor(m, off));
  if ((tid & 63) == 0) red[tid >> 6] = m;
  __syncthreads();
  if (tid == 0) partial[blockIdx.x] = max_nan(max_nan(red[0], red[1]), max_nan(red[2], red[3]));
}
// Pass 2: every block folds the partials in the same way, derives the scale
// and casts its 8192 elements; block 0 writes the scale.
template <bool IN_F32>
__global__ void __launch_bounds__(256) cast_unit_e4m3_kernel(const uint8_t* __restrict__ x, int64_t n,
                                                             const float* __restrict__ partial, int parts,
                                                             uint8_t* __restrict__ out, float* __restrict__ scale_out) {
  __shared__ float inv_sh;
  const int tid = threadIdx.x;
  if (tid < 64) {
    float m = 0.f;
    for (int i = tid; i < parts; i += 64) m = max_nan(m, partial[i]);
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) m = max_nan(m, __shfl_xor(m, off));
    if (tid == 0) {
      const float c = m != m ? m : __builtin_fmaxf(m, 1.0e-30f);
      const float scale = c * (1.0f / 448.0f);
      inv_sh = 1.0f / scale;
      if (blockIdx.x == 0) scale_out[0] = scale;
    }
  }
  __syncthreads();
  const float s = inv_sh;
  const int64_t e0 = (int64_t)blockIdx.x * kCastBlock + (int64_t)tid * 32;
  if (e0 >= n) return;
  float v[32];
  load32<IN_F32>(x, n, e0, v);
  uint32_t o[8];
#pragma unroll
  for (int q = 0; q < 8; ++q) {
    float c[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) c[r] = __builtin_fminf(__builtin_fmaxf(v[4 * q + r] * s, -448.f), 448.f);
    int t = __builtin_amdgcn_cvt_pk_fp8_f32(c[0], c[1], 0, false);
    t = __builtin_amdgcn_cvt_pk_fp8_f32(c[2], c[3], t, true);
    o[q] = (uint32_t)t;
  }
  *(u32x4*)(out + e0) = u32x4{o[0], o[1], o[2], o[3]};
  *(u32x4*)(out + e0 + 16) = u32x4{o[4], o[5], o[6], o[7]};
}

// One call's update of a delayed-scale site, state = [scale, 1 / scale,
// window peak, overflowed calls]: a = max of the call's amax values (NaN
// propagates); when live, count the call if a > scale * limit; peak =
// max(peak, a); snapshot (nullable) <- the scale the call was cast with;
// when rolling, scale = max(peak, 1e-30) * factor, 1 / scale, peak = 0.
// One block of 256 threads (a cast of config 3's gradients leaves ~10 000
// partials); the arithmetic is the host policy's, operation for operation.
constexpr int kSiteThreads = 1024;
__global__ void __launch_bounds__(kSiteThreads) site_update_kernel(const float* __restrict__ vals, int count,
                                                                   float* __restrict__ st, float limit, int live,
                                                                   int roll, float factor,
                                                                   float* __restrict__ snapshot) {
  __shared__ float red[kSiteThreads / 64];
  const int tid = threadIdx.x;
  // four loads in flight per thread (max_nan is order-free)
  float m = 0.f, m1 = 0.f, m2 = 0.f, m3 = 0.f;
  int i = tid;
  for (; i + 3 * kSiteThreads < count; i += 4 * kSiteThreads) {
    m = max_nan(m, vals[i]);
    m1 = max_nan(m1, vals[i + kSiteThreads]);
    m2 = max_nan(m2, vals[i + 2 * kSiteThreads]);
    m3 = max_nan(m3, vals[i + 3 * kSiteThreads]);
  }
  for (; i < count; i += kSiteThreads) m = max_nan(m, vals[i]);
  m = max_nan(max_nan(m, m1), max_nan(m2, m3));
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) m = max_nan(m, __shfl_xor(m, off));
  if ((tid & 63) == 0) red[tid >> 6] = m;
  __syncthreads();
  if (tid != 0) return;
#pragma unroll
  for (int w = 1; w < kSiteThreads / 64; ++w) m = max_nan(m, red[w]);
  const float scale = st[0];
  if (live) st[3] = st[3] + (m > scale * limit ? 1.f : 0.f);
  const float peak = max_nan(st[2], m);
  st[2] = peak;
  if (snapshot != nullptr) snapshot[0] = scale;
  if (roll) {
    const float c = peak != peak ? peak : __builtin_fmaxf(peak, 1.0e-30f);
    const float s = c * factor;
    st[0] = s;
    st[1] = 1.0f / s;
    st[2] = 0.f;
  }
}

// One read of a row-major bf16 gradient [rows, cols] -> its FP8 copy
// [rows_out, cols] (fp8(clamp(x * inv_scale, +-limit)), rows >= rows zero),
// the max |x| and the fp32 column sums of the unquantized input (the bias
// gradient).  A block owns kCsRows rows x 256 columns: 32 threads x 8 columns
// across a row, 8 rows at a time, kCsUnroll row loads in flight per thread.
// Each thread keeps its 8 column sums in registers; the block folds its 8 row
// slots through LDS once, into part_col[stripe][cols].  Blocks are numbered
// column block fastest, so the blocks in flight read whole rows.
constexpr int kCsRows = 512, kCsCols = 256, kCsUnroll = 8;

template <bool OUT_BF8>
__global__ void __launch_bounds__(256) cast_fp8_amax_colsum_kernel(
    const uint16_t* __restrict__ x, int64_t ldx, int64_t rows, int64_t rows_out, int cols, int ncb,
    const float* __restrict__ inv_scale, float limit, uint8_t* __restrict__ out, float* __restrict__ part_col,
    float* __restrict__ part_amax) {
  __shared__ float red[8][kCsCols];
  __shared__ float wmax[4];
  const int tid = threadIdx.x, c = tid & 31, r = tid >> 5;
  const int cb = (int)(blockIdx.x % (unsigned)ncb);
  const int64_t stripe = blockIdx.x / (unsigned)ncb;
  const int col = cb * kCsCols + c * 8;
  const int64_t row0 = stripe * kCsRows;
  const float s = inv_scale[0];
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  float amax = 0.f;
  for (int it = 0; it < kCsRows / 8; it += kCsUnroll) {
    if (row0 + it * 8 >= rows_out) break;  // block-uniform
    u32x4 w[kCsUnroll];
#pragma unroll
    for (int u = 0; u < kCsUnroll; ++u) {
      const int64_t row = row0 + (it + u) * 8 + r;
      w[u] = row < rows ? *(const u32x4*)(x + row * ldx + col) : u32x4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int u = 0; u < kCsUnroll; ++u) {
      const int64_t row = row0 + (it + u) * 8 + r;
      float v[8];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t b = w[u][j];
        v[2 * j] = __builtin_bit_cast(float, b << 16);
        v[2 * j + 1] = __builtin_bit_cast(float, b & 0xffff0000u);
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        acc[e] += v[e];
        amax = __builtin_fmaxf(amax, __builtin_fabsf(v[e]));
      }
      if (row < rows_out) {
        float q[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) q[e] = __builtin_fminf(__builtin_fmaxf(v[e] * s, -limit), limit);
        int lo, hi;
        if constexpr (OUT_BF8) {
          lo = __builtin_amdgcn_cvt_pk_bf8_f32(q[0], q[1], 0, false);
          lo = __builtin_amdgcn_cvt_pk_bf8_f32(q[2], q[3], lo, true);
          hi = __builtin_amdgcn_cvt_pk_bf8_f32(q[4], q[5], 0, false);
          hi = __builtin_amdgcn_cvt_pk_bf8_f32(q[6], q[7], hi, true);
        } else {
          lo = __builtin_amdgcn_cvt_pk_fp8_f32(q[0], q[1], 0, false);
          lo = __builtin_amdgcn_cvt_pk_fp8_f32(q[2], q[3], lo, true);
          hi = __builtin_amdgcn_cvt_pk_fp8_f32(q[4], q[5], 0, false);
          hi = __builtin_amdgcn_cvt_pk_fp8_f32(q[6], q[7], hi, true);
        }
        *(u32x2*)(out + row * cols + col) = u32x2{(uint32_t)lo, (uint32_t)hi};
      }
    }
  }
  // stripes that start past the input store no partials (padding only)
  if (row0 >= rows) return;  // block-uniform
#pragma unroll
  for (int e = 0; e < 8; ++e) red[r][c * 8 + e] = acc[e];
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) amax = __builtin_fmaxf(amax, __shfl_xor(amax, off));
  if ((tid & 63) == 0) wmax[tid >> 6] = amax;
  __syncthreads();
  float t = 0.f;
#pragma unroll
  for (int k = 0; k < 8; ++k) t += red[k][tid];
  part_col[stripe * cols + cb * kCsCols + tid] = t;
  if (tid == 0)
    part_amax[stripe * ncb + cb] = __builtin_fmaxf(__builtin_fmaxf(wmax[0], wmax[1]), __builtin_fmaxf(wmax[2], wmax[3]));
}

// colsum[col] = sum over stripes of part_col[stripe][col] (32 columns x 8
// stripe lanes per block, folded in a fixed order), and in the last block
// amax[0] = max of the amax partials.
__global__ void __launch_bounds__(256) colsum_finish_kernel(const float* __restrict__ part_col, int64_t nstripes,
                                                            int cols, float* __restrict__ colsum,
                                                            const float* __restrict__ part_amax, int64_t namax,
                                                            float* __restrict__ amax_out) {
  __shared__ float red[8][32];
  const int tid = threadIdx.x;
  if ((int)blockIdx.x < cols / 32) {
    const int c = tid & 31, g = tid >> 5, col = blockIdx.x * 32 + c;
    // stripes g + 8 k into accumulator k % 8: eight loads in flight
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    int64_t i = g;
    for (; i + 7 * 8 < nstripes; i += 8 * 8) {
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[j] += part_col[(i + 8 * j) * cols + col];
    }
#pragma unroll
    for (int j = 0; j < 8; ++j)
      if (i + 8 * j < nstripes) acc[j] += part_col[(i + 8 * j) * cols + col];
    red[g][c] = ((acc[0] + acc[1]) + (acc[2] + acc[3])) + ((acc[4] + acc[5]) + (acc[6] + acc[7]));
    __syncthreads();
    if (g == 0) {
      float t = 0.f;
#pragma unroll
      for (int k = 0; k < 8; ++k) t += red[k][c];
      colsum[col] = t;
    }
  } else {
    float m = 0.f, m1 = 0.f, m2 = 0.f, m3 = 0.f;
    int64_t i = tid;
    for (; i + 3 * 256 < namax; i += 4 * 256) {
      m = __builtin_fmaxf(m, part_amax[i]);
      m1 = __builtin_fmaxf(m1, part_amax[i + 256]);
      m2 = __builtin_fmaxf(m2, part_amax[i + 512]);
      m3 = __builtin_fmaxf(m3, part_amax[i + 768]);
    }
    for (; i < namax; i += 256) m = __builtin_fmaxf(m, part_amax[i]);
    m = __builtin_fmaxf(__builtin_fmaxf(m, m1), __builtin_fmaxf(m2, m3));
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) m = __builtin_fmaxf(m, __shfl_xor(m, off));
    if ((tid & 63) == 0) red[0][tid >> 6] = m;
    __syncthreads();
    if (tid == 0) amax_out[0] = __builtin_fmaxf(__builtin_fmaxf(red[0][0], red[0][1]), __builtin_fmaxf(red[0][2], red[0][3]));
  }
}

inline int64_t cs_align(int64_t n) { return (n + 255) / 256 * 256; }

template <bool E, bool B>
const void* ws_kernel_nk(int nk) {
  switch (nk) {
    case 1: return (const void*)fp8_gemm_ws_kernel<E, B, 1>;
    case 2: return (const void*)fp8_gemm_ws_kernel<E, B, 2>;
    case 3: return (const void*)fp8_gemm_ws_kernel<E, B, 3>;
    default: return (const void*)fp8_gemm_ws_kernel<E, B, 4>;
  }
}
// form 0: bf16 out, 1: e4m3 out, 2: e5m2 A with bf16 out
const void* ws_kernel(int form, int nk) {
  return form == 2 ? ws_kernel_nk<false, true>(nk) : form == 1 ? ws_kernel_nk<true, false>(nk)
                                                               : ws_kernel_nk<false, false>(nk);
}

hipError_t set_gemm_lds_size(const void* fn, int bytes) {
  static std::mutex mu;
  static std::vector<const void*> done;
  std::lock_guard<std::mutex> lock(mu);
  for (const void* d : done)
    if (d == fn) return hipSuccess;
  hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
  if (e == hipSuccess) done.push_back(fn);
  return e;
}

// compute units of the current device (cached per device)
int device_cus() {
  static std::mutex mu;
  static std::vector<int> cus;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0) return 256;
  std::lock_guard<std::mutex> lock(mu);
  if ((int)cus.size() <= dev) cus.resize(dev + 1, 0);
  if (cus[dev] == 0) {
    int n = 0;
    cus[dev] = hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0 ? n : 256;
  }
  return cus[dev];
}

hipError_t set_gemm_lds(const void* fn) {
  static std::mutex mu;
  static std::vector<const void*> done;
  std::lock_guard<std::mutex> lock(mu);
  for (const void* d : done)
    if (d == fn) return hipSuccess;
  hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, kGemmLds);
  if (e == hipSuccess) done.push_back(fn);
  return e;
}

}  // namespace

extern "C" int hstu_fp8_gemm(int a_dtype, const void* A, int64_t lda, const void* W, int64_t ldw,
                             const float* a_scale, int a_scale_mode, const float* w_scale, int w_scale_mode,
                             const void* bias, const void* residual, int64_t ldr, void* C, int64_t ldc,
                             int out_dtype, const float* out_scale, int M, int N, int K, int silu_begin,
                             int silu_end, hipStream_t stream) {
  if (a_dtype != HSTU_DTYPE_FP8_E4M3 && a_dtype != HSTU_DTYPE_FP8_E5M2) return HSTU_E_BAD_ARG;
  if (M < 0 || N <= 0 || K <= 0 || N % kBN != 0 || K % kBK != 0 || !A || !W || !C || !a_scale || !w_scale)
    return HSTU_E_BAD_ARG;
  if (lda < K || ldw < K || lda % 16 != 0 || ldw % 16 != 0 || ((uintptr_t)A | (uintptr_t)W) % 16 != 0)
    return HSTU_E_UNSUPPORTED;
  if (ldc < N || (residual && ldr < N) || (out_dtype != HSTU_DTYPE_BF16 && out_dtype != HSTU_DTYPE_FP8_E4M3) ||
      (out_dtype == HSTU_DTYPE_FP8_E4M3 && !out_scale))
    return HSTU_E_BAD_ARG;
  if ((int64_t)(kBM - 1) * lda + K > 0xffffffffLL || (int64_t)(kBN - 1) * ldw + K > 0xffffffffLL)
    return HSTU_E_UNSUPPORTED;
  if (M == 0) return 0;
  GemmParams p{};
  p.A = (const uint8_t*)A;
  p.W = (const uint8_t*)W;
  p.lda = lda;
  p.ldw = ldw;
  p.a_scale = a_scale;
  p.w_scale = w_scale;
  p.a_mode = a_scale_mode != 0;
  p.w_mode = w_scale_mode != 0;
  p.bias = (const uint16_t*)bias;
  p.resid = (const uint16_t*)residual;
  p.ldr = ldr;
  p.C = C;
  p.ldc = ldc;
  p.out_scale = out_scale;
  p.M = M;
  p.N = N;
  p.K = K;
  p.silu_begin = silu_begin;
  p.silu_end = silu_end;
  p.tiles_m = (M + kBM - 1) / kBM;
  // producer/consumer form: N % 256, K % 256, 16-byte aligned epilogue rows
  const bool out8 = out_dtype == HSTU_DTYPE_FP8_E4M3;
  const bool wide_ok =
      HSTU_GEMM_WIDE && N % kWideBN == 0 && K % 256 == 0 && (uintptr_t)C % 16 == 0 && ldc % (out8 ? 16 : 8) == 0 &&
      (uintptr_t)bias % 4 == 0 && (silu_begin >= silu_end || (silu_begin % 64 == 0 && silu_end % 64 == 0)) &&
      (int64_t)kBM * ldc * (out8 ? 1 : 2) <= 0xffffffffLL && (int64_t)kBM * ldr * 2 <= 0xffffffffLL &&
      (int64_t)M * 4 <= 0xffffffffLL &&
      (!residual || ((uintptr_t)residual % 16 == 0 && ldr % 8 == 0)) && (int64_t)(N - 1) * ldw + K <= 0xffffffffLL &&
      (a_dtype == HSTU_DTYPE_FP8_E4M3 || (!out8 && !residual));
  if (wide_ok) {
    p.tiles_n = N / kWideBN;
    const int total = p.tiles_m * p.tiles_n;
    const int per_xcd = (total + 7) / 8;
    const int gx = std::max(1, std::min(device_cus() / 8, per_xcd));  // one workgroup per CU
    int parg = per_xcd;
    void* args[] = {&p, &parg};
    // two-workgroup form, except at N = 512 without a residual (the [M, 512]
    // projections and the K = 2048 dgrad), where the producer/consumer form
    // measured faster (0.112 against 0.118 ms at M = 262 144, K = 512)
    if (HSTU_GEMM_DUO && (N > 512 || residual)) {
      void (*dk)(GemmParams, int);
      if (a_dtype == HSTU_DTYPE_FP8_E5M2) dk = fp8_gemm_duo_kernel<false, false, true>;
      else if (out8) dk = residual ? fp8_gemm_duo_kernel<true, true, false> : fp8_gemm_duo_kernel<true, false, false>;
      else dk = residual ? fp8_gemm_duo_kernel<false, true, false> : fp8_gemm_duo_kernel<false, false, false>;
      return (int)hipLaunchKernel((const void*)dk, dim3(8 * per_xcd), dim3(kDuoThreads), args, 0, stream);
    }
    void (*kern)(GemmParams, int);
    if (a_dtype == HSTU_DTYPE_FP8_E5M2) kern = fp8_gemm_pc_kernel<false, false, true>;
    else if (out8) kern = residual ? fp8_gemm_pc_kernel<true, true, false> : fp8_gemm_pc_kernel<true, false, false>;
    else kern = residual ? fp8_gemm_pc_kernel<false, true, false> : fp8_gemm_pc_kernel<false, false, false>;
    return (int)hipLaunchKernel((const void*)kern, dim3(8 * gx), dim3(kPcThreads), args, 0, stream);
  }
  p.tiles_n = N / kBN;
  // W-stationary persistent form: about one workgroup per CU, streams of M
  // tiles; its output leaves in 16-byte row segments (else the tile kernel)
  const bool ws_rows = (uintptr_t)C % 16 == 0 && (out_dtype == HSTU_DTYPE_FP8_E4M3 ? ldc % 16 == 0 : ldc % 8 == 0);
  if (K <= kWsMaxK && !residual && p.tiles_n <= kWsCus && ws_rows) {
    const int streams = std::max(1, std::min(kWsCus / p.tiles_n, p.tiles_m));
    if (a_dtype == HSTU_DTYPE_FP8_E5M2 && out_dtype != HSTU_DTYPE_BF16) return HSTU_E_UNSUPPORTED;  // dgrad form
    const int form = a_dtype == HSTU_DTYPE_FP8_E5M2 ? 2 : out_dtype == HSTU_DTYPE_FP8_E4M3 ? 1 : 0;
    const void* wk = ws_kernel(form, K / kBK);
    hipError_t e = set_gemm_lds_size(wk, kWsLds);
    if (e != hipSuccess) return (int)e;
    int sarg = streams;
    void* args[] = {&p, &sarg};
    return (int)hipLaunchKernel(wk, dim3(streams * p.tiles_n), dim3(kWsThreads), args, (size_t)kWsLds, stream);
  }
  const int total = p.tiles_m * p.tiles_n;
  const int grid = (total + 7) / 8 * 8;
  void (*kern)(GemmParams);
  if (a_dtype == HSTU_DTYPE_FP8_E5M2) {
    if (out_dtype != HSTU_DTYPE_BF16 || residual) return HSTU_E_UNSUPPORTED;  // the dgrad form only
    kern = fp8_gemm_kernel<false, false, kE5M2A>;
  } else if (out_dtype == HSTU_DTYPE_FP8_E4M3) {
    kern = residual ? fp8_gemm_kernel<true, true, kE4M3> : fp8_gemm_kernel<true, false, kE4M3>;
  } else {
    kern = residual ? fp8_gemm_kernel<false, true, kE4M3> : fp8_gemm_kernel<false, false, kE4M3>;
  }
  hipError_t e = set_gemm_lds((const void*)kern);
  if (e != hipSuccess) return (int)e;
  void* args[] = {&p};
  return (int)hipLaunchKernel((const void*)kern, dim3(grid), dim3(kThreads), args, (size_t)kGemmLds, stream);
}

extern "C" int hstu_bf16_gemm(const void* A, int64_t lda, const void* W, int64_t ldw, const void* bias,
                              const void* residual, int64_t ldr, void* C, int64_t ldc, int M, int N, int K,
                              int silu_begin, int silu_end, hipStream_t stream) {
  // the tile kernel on bf16 rows: k counted in bytes (128-byte k-steps)
  if (M < 0 || N <= 0 || K <= 0 || N % kBN != 0 || (2 * K) % kBK != 0 || !A || !W || !C) return HSTU_E_BAD_ARG;
  if (lda < K || ldw < K || ldc < N || (residual && ldr < N)) return HSTU_E_BAD_ARG;
  if (lda % 8 != 0 || ldw % 8 != 0 || ldc % 4 != 0 || (residual && ldr % 4 != 0) ||
      ((uintptr_t)A | (uintptr_t)W) % 16 != 0 || (uintptr_t)C % 8 != 0 || (uintptr_t)residual % 8 != 0 ||
      (uintptr_t)bias % 8 != 0)
    return HSTU_E_UNSUPPORTED;
  if ((int64_t)(kBM - 1) * 2 * lda + 2 * K > 0xffffffffLL || (int64_t)(kBN - 1) * 2 * ldw + 2 * K > 0xffffffffLL)
    return HSTU_E_UNSUPPORTED;
  if (M == 0) return 0;
  GemmParams p{};
  p.A = (const uint8_t*)A;
  p.W = (const uint8_t*)W;
  p.lda = 2 * lda;
  p.ldw = 2 * ldw;
  p.bias = (const uint16_t*)bias;
  p.resid = (const uint16_t*)residual;
  p.ldr = ldr;
  p.C = C;
  p.ldc = ldc;
  p.M = M;
  p.N = N;
  p.K = 2 * K;
  p.silu_begin = silu_begin;
  p.silu_end = silu_end;
  p.tiles_m = (M + kBM - 1) / kBM;
  p.tiles_n = N / kBN;
  void (*kern)(GemmParams) = residual ? fp8_gemm_kernel<false, true, kBF16> : fp8_gemm_kernel<false, false, kBF16>;
  hipError_t e = set_gemm_lds((const void*)kern);
  if (e != hipSuccess) return (int)e;
  const int grid = (p.tiles_m * p.tiles_n + 7) / 8 * 8;
  void* args[] = {&p};
  return (int)hipLaunchKernel((const void*)kern, dim3(grid), dim3(kThreads), args, (size_t)kGemmLds, stream);
}

extern "C" int hstu_fp8_gemm_rowcol(const void* A, int64_t lda, const void* W, int64_t ldw, const float* a_scale,
                                    int a_scale_mode, const float* w_scale, int w_scale_mode, const void* bias,
                                    const void* residual, int64_t ldr, void* C, int64_t ldc, int out_dtype,
                                    const float* out_scale, int M, int N, int K, int silu_begin, int silu_end,
                                    hipStream_t stream) {
  return hstu_fp8_gemm(HSTU_DTYPE_FP8_E4M3, A, lda, W, ldw, a_scale, a_scale_mode, w_scale, w_scale_mode, bias,
                       residual, ldr, C, ldc, out_dtype, out_scale, M, N, K, silu_begin, silu_end, stream);
}

extern "C" int hstu_quantize_e4m3_rows(const void* x, int64_t ldx, int rows, int cols, int group,
                                       const float* scale_in, void* out, int64_t ldo, float* scale_out,
                                       hipStream_t stream) {
  if (rows < 0 || cols <= 0 || group <= 0 || cols % group != 0 || group % 8 != 0 || group > 4096 || !x || !out ||
      ldx < cols || ldo < cols || ldx % 8 != 0 || ldo % 8 != 0 || (!scale_in && !scale_out))
    return HSTU_E_BAD_ARG;
  if (((uintptr_t)x % 16) != 0 || ((uintptr_t)out % 8) != 0) return HSTU_E_UNSUPPORTED;
  if (rows == 0) return 0;
  const int64_t groups = (int64_t)rows * (cols / group);
  const int grid = (int)((groups + 3) / 4);
  hipLaunchKernelGGL(quantize_e4m3_kernel, dim3(grid), dim3(256), 0, stream, (const uint16_t*)x, ldx, rows, cols,
                     group, scale_in, (uint8_t*)out, ldo, scale_out);
  return (int)hipGetLastError();
}

extern "C" int64_t hstu_cast_fp8_amax_partials(int64_t n) { return n < 0 ? -1 : (n + kCastBlock - 1) / kCastBlock; }

extern "C" int hstu_cast_fp8_amax(int in_dtype, const void* x, int64_t n, const float* inv_scale, int out_dtype,
                                  float limit, void* out, float* partial_amax, int64_t partial_count,
                                  hipStream_t stream) {
  if ((in_dtype != HSTU_DTYPE_BF16 && in_dtype != HSTU_DTYPE_FP32) ||
      (out_dtype != HSTU_DTYPE_FP8_E4M3 && out_dtype != HSTU_DTYPE_FP8_E5M2) || n < 0 || !x || !inv_scale || !out ||
      !partial_amax || !(limit > 0.f))
    return HSTU_E_BAD_ARG;
  if (partial_count < hstu_cast_fp8_amax_partials(n)) return HSTU_E_BAD_ARG;
  if (n % 32 != 0 || (uintptr_t)x % 16 || (uintptr_t)out % 16) return HSTU_E_UNSUPPORTED;
  if (n == 0) return 0;
  const int64_t grid = hstu_cast_fp8_amax_partials(n);
  if (grid >= ((int64_t)1 << 31)) return HSTU_E_UNSUPPORTED;
  const bool f32 = in_dtype == HSTU_DTYPE_FP32, bf8 = out_dtype == HSTU_DTYPE_FP8_E5M2;
  auto* xp = (const uint8_t*)x;
  auto* op = (uint8_t*)out;
  if (f32 && bf8) hipLaunchKernelGGL((cast_fp8_amax_kernel<true, true>), dim3(grid), dim3(256), 0, stream, xp, n, inv_scale, limit, op, partial_amax);
  else if (f32) hipLaunchKernelGGL((cast_fp8_amax_kernel<true, false>), dim3(grid), dim3(256), 0, stream, xp, n, inv_scale, limit, op, partial_amax);
  else if (bf8) hipLaunchKernelGGL((cast_fp8_amax_kernel<false, true>), dim3(grid), dim3(256), 0, stream, xp, n, inv_scale, limit, op, partial_amax);
  else hipLaunchKernelGGL((cast_fp8_amax_kernel<false, false>), dim3(grid), dim3(256), 0, stream, xp, n, inv_scale, limit, op, partial_amax);
  return (int)hipGetLastError();
}

extern "C" int hstu_quantize_e4m3_unit(int in_dtype, const void* x, int64_t n, void* out, float* scale_out,
                                       float* partial, int64_t partial_count, hipStream_t stream) {
  if ((in_dtype != HSTU_DTYPE_BF16 && in_dtype != HSTU_DTYPE_FP32) || n <= 0 || !x || !out || !scale_out ||
      !partial)
    return HSTU_E_BAD_ARG;
  const int64_t grid = hstu_cast_fp8_amax_partials(n);
  if (partial_count < grid) return HSTU_E_BAD_ARG;
  if (n % 32 != 0 || (uintptr_t)x % 16 || (uintptr_t)out % 16 || grid >= ((int64_t)1 << 31)) return HSTU_E_UNSUPPORTED;
  auto* xp = (const uint8_t*)x;
  auto* op = (uint8_t*)out;
  if (in_dtype == HSTU_DTYPE_FP32) {
    hipLaunchKernelGGL(absmax_partials_kernel<true>, dim3(grid), dim3(256), 0, stream, xp, n, partial);
    hipLaunchKernelGGL(cast_unit_e4m3_kernel<true>, dim3(grid), dim3(256), 0, stream, xp, n, partial, (int)grid, op,
                       scale_out);
  } else {
    hipLaunchKernelGGL(absmax_partials_kernel<false>, dim3(grid), dim3(256), 0, stream, xp, n, partial);
    hipLaunchKernelGGL(cast_unit_e4m3_kernel<false>, dim3(grid), dim3(256), 0, stream, xp, n, partial, (int)grid, op,
                       scale_out);
  }
  return (int)hipGetLastError();
}

extern "C" int hstu_fp8_site_update(const float* amax_values, int count, float* state, float limit, int live,
                                    int roll, float factor, float* snapshot, hipStream_t stream) {
  if (!amax_values || count <= 0 || !state || !(limit > 0.f)) return HSTU_E_BAD_ARG;
  hipLaunchKernelGGL(site_update_kernel, dim3(1), dim3(kSiteThreads), 0, stream, amax_values, count, state, limit, live, roll,
                     factor, snapshot);
  return (int)hipGetLastError();
}

extern "C" int64_t hstu_cast_fp8_amax_colsum_workspace_bytes(int64_t rows, int64_t cols) {
  if (rows < 0 || cols <= 0 || cols % kCsCols != 0) return -1;
  const int64_t stripes = (rows + kCsRows - 1) / kCsRows;
  return cs_align(stripes * cols * 4) + cs_align(stripes * (cols / kCsCols) * 4);
}

extern "C" int hstu_cast_fp8_amax_colsum(const void* x, int64_t ldx, int64_t rows, int64_t cols,
                                         const float* inv_scale, int out_dtype, float limit, void* out,
                                         int64_t rows_out, float* colsum, float* amax, void* workspace,
                                         int64_t workspace_bytes, hipStream_t stream) {
  if ((out_dtype != HSTU_DTYPE_FP8_E4M3 && out_dtype != HSTU_DTYPE_FP8_E5M2) || rows < 0 || rows_out < rows ||
      cols <= 0 || ldx < cols || !inv_scale || !colsum || !amax || !(limit > 0.f) || (rows > 0 && !x) ||
      (rows_out > 0 && !out))
    return HSTU_E_BAD_ARG;
  if (cols % kCsCols != 0 || cols > (1 << 30) || ldx % 8 != 0 || (uintptr_t)x % 16 || (uintptr_t)out % 8)
    return HSTU_E_UNSUPPORTED;
  const int64_t need = hstu_cast_fp8_amax_colsum_workspace_bytes(rows, cols);
  if (workspace_bytes < need || (need > 0 && !workspace)) return HSTU_E_BAD_ARG;
  const int ncb = (int)(cols / kCsCols);
  const int64_t stripes = (rows + kCsRows - 1) / kCsRows;
  const int64_t launch = std::max(stripes, (rows_out + kCsRows - 1) / kCsRows) * ncb;
  if (launch >= ((int64_t)1 << 31)) return HSTU_E_UNSUPPORTED;
  float* part_col = (float*)workspace;
  float* part_amax = (float*)((uint8_t*)workspace + cs_align(stripes * cols * 4));
  if (launch > 0) {
    if (out_dtype == HSTU_DTYPE_FP8_E5M2)
      hipLaunchKernelGGL((cast_fp8_amax_colsum_kernel<true>), dim3((unsigned)launch), dim3(256), 0, stream,
                         (const uint16_t*)x, ldx, rows, rows_out, (int)cols, ncb, inv_scale, limit, (uint8_t*)out,
                         part_col, part_amax);
    else
      hipLaunchKernelGGL((cast_fp8_amax_colsum_kernel<false>), dim3((unsigned)launch), dim3(256), 0, stream,
                         (const uint16_t*)x, ldx, rows, rows_out, (int)cols, ncb, inv_scale, limit, (uint8_t*)out,
                         part_col, part_amax);
  }
  hipLaunchKernelGGL(colsum_finish_kernel, dim3((unsigned)(cols / 32 + 1)), dim3(256), 0, stream, part_col, stripes,
                     (int)cols, colsum, part_amax, stripes * ncb, amax);
  return (int)hipGetLastError();
}
