// Delta-q ("cached" / targets-only) HSTU attention on gfx950: the last DS
// positions of each sequence, given as compact query rows, against the whole
// sequence's keys and values.
//   forward:  ops/pytorch/pt_hstu_attention.py:191-251 (pytorch_cached_hstu_mha),
//             launched by triton_cached_hstu_mha (ops/triton/triton_hstu_attention.py:3710-3866);
//   backward: _hstu_attn_delta_bwd (triton_hstu_attention.py:3033-3163) and its op
//             triton_hstu_attention_delta_bwd (:3413-3480).
//
// SiLU attention has no softmax normalisation: out_i = sum_j silu(s_ij)/N v_j
// splits over key chunks into partial sums that add up in any grouping.  A
// block takes one (query row, head, 256-key chunk) in the forward and one
// (sequence, head, chunk) in the backward; per-chunk fp32 partials go to a
// workspace and a second kernel sums them in chunk order (deterministic).
// With one query per sequence each key is read once and the work is
// HBM-bound: a group of lanes shares a K/V row, one 16-byte piece each, for
// both the dot products (summed across the group with DPP) and the D-wide
// outputs.
#include <hip/hip_runtime.h>

#include "hstu_common.h"
#include "hstu_mi355x.h"

using namespace hstu;

namespace {

constexpr int kChunk = 256;  // keys per block
constexpr int kMaxDsBwd = 4;  // delta rows per sequence served by the backward

struct DeltaParams {
  const uint8_t* q;  // [B*DS, H, D] (bf16, or e4m3 when q_e4m3)
  int q_e4m3;
  const uint8_t* k;  // [T, H, D]
  const uint8_t* v;
  const uint16_t* dout;  // [B*DS, H, D] bf16 (backward)
  int64_t q_rs, k_rs, v_rs, do_rs;  // row strides, elements
  float alpha, q_scale, k_scale, v_scale, inv_n;
  const int64_t* seq_offsets;
  int B, H, N, DS;
  const int* num_targets;
  int max_attn_len, contextual_seq_len;
  float* part;  // [rows * H, nchunk, D] fp32 partial sums
  int nchunk;
  uint16_t* out;  // forward output [B*DS, H, D]
  int64_t out_rs;
  uint16_t* dq;  // backward outputs
  uint16_t* dk;
  uint16_t* dv;
  int64_t dq_rs, dk_rs, dv_rs;
};

__device__ __forceinline__ float bf16f_(uint32_t b) { return __builtin_bit_cast(float, b << 16); }
__device__ __forceinline__ float bf16_round(float x) { return bf16f_(to_bf16(x)); }

// 8 consecutive q elements starting at element offset `off` (bf16: one
// 16-byte load; e4m3: 8 bytes in the low half), raw.  Issued ahead of the K/V
// loads and converted later, so the wait for them does not wait for K/V.
__device__ __forceinline__ u32x4 load_q8(const DeltaParams& p, int64_t off) {
  if (p.q_e4m3) {
    const u32x2 t = *(const u32x2*)(p.q + off);
    return u32x4{t[0], t[1], 0u, 0u};
  }
  return *(const u32x4*)(p.q + 2 * off);
}
// fp32 values of a load_q8 piece (e4m3 times `scale`).
__device__ __forceinline__ void cvt_q8(const DeltaParams& p, const u32x4& w, float scale, float* f) {
  if (p.q_e4m3) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const f32x2 lo = __builtin_amdgcn_cvt_pk_f32_fp8((int)w[i], false);
      const f32x2 hi = __builtin_amdgcn_cvt_pk_f32_fp8((int)w[i], true);
      f[4 * i] = lo[0] * scale;
      f[4 * i + 1] = lo[1] * scale;
      f[4 * i + 2] = hi[0] * scale;
      f[4 * i + 3] = hi[1] * scale;
    }
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f[2 * i] = __builtin_bit_cast(float, w[i] << 16);
      f[2 * i + 1] = __builtin_bit_cast(float, w[i] & 0xffff0000u);
    }
  }
}

struct DeltaSeq {
  int64_t start;
  int len, L, b;  // len: the jagged length; L = min(len, N)
};
__device__ __forceinline__ DeltaSeq delta_seq(const DeltaParams& p, int b) {
  DeltaSeq s;
  s.b = b;
  s.start = p.seq_offsets[b];
  s.len = (int)(p.seq_offsets[b + 1] - s.start);
  s.L = min(s.len, p.N);
  return s;
}
__device__ __forceinline__ MaskCtx delta_mask(const DeltaParams& p, const DeltaSeq& s) {
  MaskCtx m;
  m.L = s.L;
  m.targets = p.num_targets != nullptr;
  m.nt = m.targets ? p.num_targets[s.b] : 0;
  m.ctx = p.contextual_seq_len;
  m.max_attn = p.max_attn_len;
  return m;
}

// ------------------------------------------------------------------ layout
// LPR lanes share a K/V row, each taking one 16-byte piece (EPL elements), so
// a wave's load instruction covers RPW whole rows; the 256 threads cover RPB
// rows per round and a 256-key chunk in ROUNDS rounds.  A lane keeps the same
// rows for the scores and for the D-wide outputs, and issues all its K / V
// loads before the first use.
template <int D, bool FP8>
struct RowMap {
  static constexpr int ES = FP8 ? 1 : 2;
  static constexpr int LPR = D * ES / 16;
  static constexpr int EPL = 16 / ES;
  static constexpr int RPW = 64 / LPR;
  static constexpr int RPB = 4 * RPW;
  static constexpr int ROUNDS = kChunk / RPB;
};

template <int CTRL>
__device__ __forceinline__ float dpp_sum(float v) {
  return v + __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xf, 0xf, false));
}
// Sum over the LPR lanes of a row group (LPR = 4, 8 or 16): xor 1, xor 2
// (quad_perm), then the half-row / row mirrors pair the quads / halves.
template <int LPR>
__device__ __forceinline__ float group_sum(float v) {
  v = dpp_sum<0xB1>(v);  // quad_perm [1, 0, 3, 2]
  v = dpp_sum<0x4E>(v);  // quad_perm [2, 3, 0, 1]
  if constexpr (LPR >= 8) v = dpp_sum<0x141>(v);  // row_half_mirror
  if constexpr (LPR >= 16) v = dpp_sum<0x140>(v);  // row_mirror
  return v;
}

// EPL elements of a 16-byte piece, fp32, times `scale`; with ROUND the
// products are rounded to bf16 (the reference's k_real / v_real).
template <bool FP8, bool ROUND>
__device__ __forceinline__ void unpack16(const u32x4& w, float scale, float (&f)[FP8 ? 16 : 8]) {
  if constexpr (FP8) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const f32x2 lo = __builtin_amdgcn_cvt_pk_f32_fp8((int)w[i], false);
      const f32x2 hi = __builtin_amdgcn_cvt_pk_f32_fp8((int)w[i], true);
      f[4 * i] = lo[0] * scale;
      f[4 * i + 1] = lo[1] * scale;
      f[4 * i + 2] = hi[0] * scale;
      f[4 * i + 3] = hi[1] * scale;
    }
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f[2 * i] = bf16f_(w[i] & 0xffffu) * scale;
      f[2 * i + 1] = bf16f_(w[i] >> 16) * scale;
    }
  }
  if constexpr (ROUND) {
#pragma unroll
    for (int e = 0; e < (FP8 ? 16 : 8); ++e) f[e] = bf16_round(f[e]);
  }
}

// ------------------------------------------------------------------ bf16 pairs
// e4m3 and bf16 values are exact in bf16, and products of two bf16 values are
// exact in fp32, so v_dot2_f32_bf16 on bf16 pairs gives the exact products
// of the fp32 formulation with fp32 sums, at half the instructions.
__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, a), __builtin_bit_cast(bf16x2, b), c, false);
}
// bytes 0-1 (HI false) or 2-3 (HI true) of an e4m3 word as a bf16 pair (exact)
template <bool HI>
__device__ __forceinline__ uint32_t fp8_pair(uint32_t w) {
  return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8((int)w, 1.f, HI));
}
// A load_q8 piece as 4 bf16 pairs (elements 2i, 2i + 1 in word i).
__device__ __forceinline__ void q8_pairs(const DeltaParams& p, const u32x4& w, uint32_t* o) {
  if (p.q_e4m3) {
    o[0] = fp8_pair<false>(w[0]);
    o[1] = fp8_pair<true>(w[0]);
    o[2] = fp8_pair<false>(w[1]);
    o[3] = fp8_pair<true>(w[1]);
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) o[i] = w[i];
  }
}

// ------------------------------------------------------------------ forward
// 1-D grid over (head, chunk, delta row), head fastest: the heads of a chunk
// run side by side, so the concurrent blocks read adjacent pieces of the same
// [H, D] rows rather than one head's strided slice.  Scores from the inputs
// as stored: e4m3 products accumulate exactly in fp32 and the scale product
// multiplies the dot; silu / N rounded to bf16, V dequantized and rounded to
// bf16 -- the reference's FP8 forward rounding order
// (triton_hstu_attention.py:503-522).  Rounds go in pairs: the two keys' bf16
// weights and V values (same d) form the bf16 pairs of one dot2 per element.
template <int D, bool FP8>
__global__ void __launch_bounds__(kThreads) delta_fwd_kernel(DeltaParams p) {
  using M = RowMap<D, FP8>;
  constexpr int EPL = M::EPL;
  static_assert(M::ROUNDS % 2 == 0, "rounds go in pairs");
  __shared__ float red[M::RPB * D];
  const int tid = threadIdx.x, h = blockIdx.x % p.H, hc = blockIdx.x / p.H;
  const int chunk = hc % p.nchunk, row = hc / p.nchunk;
  const int b = row / p.DS, r = row - b * p.DS;
  const DeltaSeq sq = delta_seq(p, b);
  const int j0 = chunk * kChunk;
  if (j0 >= sq.L) return;
  const int i = sq.L - p.DS + r;  // the query's position in its sequence
  const int wave = tid >> 6, lane = tid & 63;
  const int slot = wave * M::RPW + lane / M::LPR, e0 = (lane % M::LPR) * EPL;
  const int jn = min(kChunk, sq.L - j0);
  u32x4 qw[EPL / 8];
#pragma unroll
  for (int c = 0; c < EPL / 8; ++c) qw[c] = load_q8(p, row * p.q_rs + (int64_t)h * D + e0 + 8 * c);
  u32x4 kr[M::ROUNDS], vr[M::ROUNDS];
#pragma unroll
  for (int t = 0; t < M::ROUNDS; ++t) {
    const int64_t j = sq.start + j0 + min(t * M::RPB + slot, jn - 1);
    kr[t] = *(const u32x4*)(p.k + (j * p.k_rs + (int64_t)h * D + e0) * M::ES);
    vr[t] = *(const u32x4*)(p.v + (j * p.v_rs + (int64_t)h * D + e0) * M::ES);
  }
  uint32_t qb[EPL / 2];
#pragma unroll
  for (int c = 0; c < EPL / 8; ++c) q8_pairs(p, qw[c], qb + 4 * c);
  const MaskCtx mc = delta_mask(p, sq);
  const float xs = p.alpha * p.q_scale * p.k_scale;
  float acc[EPL] = {};
#pragma unroll
  for (int t = 0; t < M::ROUNDS; t += 2) {
    uint32_t wb[2];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const u32x4 k = kr[t + u];
      float part = 0.f;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        if constexpr (FP8) {
          part = dot2(fp8_pair<false>(k[c]), qb[2 * c], part);
          part = dot2(fp8_pair<true>(k[c]), qb[2 * c + 1], part);
        } else {
          part = dot2(k[c], qb[c], part);
        }
      }
      const float x = group_sum<M::LPR>(part) * xs;
      const int jj = (t + u) * M::RPB + slot;
      float w = 0.f;
      if (jj < jn && i >= 0 && valid_generic(i, j0 + jj, mc))
        w = x * __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(-kLog2e * x)) * p.inv_n;
      wb[u] = to_bf16(w);
    }
    const uint32_t wp = wb[0] | (wb[1] << 16);
    if constexpr (FP8) {
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const f32x2 a0 = __builtin_amdgcn_cvt_pk_f32_fp8((int)vr[t][c], false);
        const f32x2 a1 = __builtin_amdgcn_cvt_pk_f32_fp8((int)vr[t][c], true);
        const f32x2 b0 = __builtin_amdgcn_cvt_pk_f32_fp8((int)vr[t + 1][c], false);
        const f32x2 b1 = __builtin_amdgcn_cvt_pk_f32_fp8((int)vr[t + 1][c], true);
        const float vs = p.v_scale;
        acc[4 * c] = dot2(pack_bf16(a0[0] * vs, b0[0] * vs), wp, acc[4 * c]);
        acc[4 * c + 1] = dot2(pack_bf16(a0[1] * vs, b0[1] * vs), wp, acc[4 * c + 1]);
        acc[4 * c + 2] = dot2(pack_bf16(a1[0] * vs, b1[0] * vs), wp, acc[4 * c + 2]);
        acc[4 * c + 3] = dot2(pack_bf16(a1[1] * vs, b1[1] * vs), wp, acc[4 * c + 3]);
      }
    } else {
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        // (v_t[2c], v_t+1[2c]) and (v_t[2c+1], v_t+1[2c+1])
        acc[2 * c] = dot2(__builtin_amdgcn_perm(vr[t + 1][c], vr[t][c], 0x05040100u), wp, acc[2 * c]);
        acc[2 * c + 1] = dot2(__builtin_amdgcn_perm(vr[t + 1][c], vr[t][c], 0x07060302u), wp, acc[2 * c + 1]);
      }
    }
  }
#pragma unroll
  for (int e = 0; e < EPL; ++e) red[slot * D + e0 + e] = acc[e];
  __syncthreads();
  if (tid < D) {
    float t = 0.f;
    for (int g = 0; g < M::RPB; ++g) t += red[g * D + tid];
    p.part[(((int64_t)row * p.H + h) * p.nchunk + chunk) * D + tid] = t;
  }
}

// out[row, h, :] = sum of the chunk partials in chunk order (rows whose
// sequence is shorter than DS get zeros).
template <int D>
__global__ void delta_fwd_finalize(DeltaParams p) {
  const int row = blockIdx.x, h = blockIdx.y, d = threadIdx.x;
  if (d >= D) return;
  const int b = row / p.DS, r = row - b * p.DS;
  const DeltaSeq sq = delta_seq(p, b);
  float t = 0.f;
  if (sq.L - p.DS + r >= 0) {
    const int nc = (sq.L + kChunk - 1) / kChunk;
    const float* src = p.part + (((int64_t)row * p.H + h) * p.nchunk) * D + d;
    for (int c = 0; c < nc; ++c) t += src[(int64_t)c * D];
  }
  p.out[(int64_t)row * p.out_rs + (int64_t)h * D + d] = to_bf16(t);
}

// ------------------------------------------------------------------ backward
// A K or V piece of one key as bf16 pairs along d, dequantized and rounded:
// (x.to(fp32) * scale).to(bf16) per element; bf16 inputs (scale 1) are their
// own words.
template <bool FP8>
__device__ __forceinline__ void real_pairs(const u32x4& w, float scale, uint32_t (&o)[FP8 ? 8 : 4]) {
  if constexpr (FP8) {
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const f32x2 lo = __builtin_amdgcn_cvt_pk_f32_fp8((int)w[c], false);
      const f32x2 hi = __builtin_amdgcn_cvt_pk_f32_fp8((int)w[c], true);
      o[2 * c] = pack_bf16(lo[0] * scale, lo[1] * scale);
      o[2 * c + 1] = pack_bf16(hi[0] * scale, hi[1] * scale);
    }
  } else {
#pragma unroll
    for (int c = 0; c < 4; ++c) o[c] = w[c];
  }
}
__device__ __forceinline__ float bf_lo(uint32_t w) { return __builtin_bit_cast(float, w << 16); }
__device__ __forceinline__ float bf_hi(uint32_t w) { return __builtin_bit_cast(float, w & 0xffff0000u); }

// 1-D grid over (head, chunk, sequence), head fastest as in the forward; the
// block handles the sequence's DS query rows (DS = 1..4, a template argument
// so the row loops unroll without conditions).  As in the reference backward
// (triton_hstu_attention.py:3033-3163), K and V are dequantized and rounded
// to bf16 (k_real, v_real) and silu / dS are rounded to bf16 before they
// scale dO / q / k_real:
//   dv_j = sum_r silu_rj/N dO_r,  dk_j = alpha sum_r dS_rj q_r,
//   dq_r = alpha sum_j dS_rj k_real_j,  dS = (dO_r . v_j) sig (1 + x (1 - sig)) / N.
// Every product above has bf16 operands (q and dO are bf16 or e4m3), so the
// sums run as v_dot2_f32_bf16 over bf16 pairs: along d for the dots, across
// row pairs for dk / dv, across key pairs (two rounds) for dq.  A lane keeps
// its K / V pieces in registers from the scores to dk, dv, dq.
template <int D, bool FP8, int DS>
__global__ void __launch_bounds__(kThreads) delta_bwd_kernel(DeltaParams p) {
  using M = RowMap<D, FP8>;
  constexpr int EPL = M::EPL, WPL = EPL / 2;  // elements / bf16-pair words per lane piece
  constexpr int RP = DS / 2;                  // row pairs
  static_assert(M::ROUNDS % 2 == 0, "rounds go in pairs");
  __shared__ uint32_t qd2[DS][D / 2], dod2[DS][D / 2];  // q, dO rows as bf16 pairs along d
  __shared__ uint32_t qr2[RP > 0 ? RP : 1][D], dor2[RP > 0 ? RP : 1][D];  // rows (2rp, 2rp + 1) paired per d
  __shared__ float red[M::RPB * D];
  const int tid = threadIdx.x, h = blockIdx.x % p.H, hc = blockIdx.x / p.H;
  const int chunk = hc % p.nchunk, b = hc / p.nchunk;
  const DeltaSeq sq = delta_seq(p, b);
  const int j0 = chunk * kChunk;
  if (j0 >= sq.len) return;
  const int wave = tid >> 6, lane = tid & 63;
  const int slot = wave * M::RPW + lane / M::LPR, e0 = (lane % M::LPR) * EPL;
  const int jn = min(kChunk, sq.len - j0);  // rows to write
  const int jl = min(kChunk, sq.L - j0);    // rows with attention (the rest get zero gradients)
  // q and dO of the DS rows: 8-element pieces, one per thread of the first
  // DS * D / 8 (<= 64), loaded ahead of K / V
  constexpr int kPieces = DS * D / 8;
  static_assert(kPieces <= kThreads, "one q / dO piece per thread");
  const int pr = tid / (D / 8), pd = (tid % (D / 8)) * 8;
  const int64_t prow = (int64_t)b * DS + pr;
  u32x4 qw{}, dw{};
  if (tid < kPieces) {
    qw = load_q8(p, prow * p.q_rs + (int64_t)h * D + pd);
    dw = *(const u32x4*)(p.dout + prow * p.do_rs + (int64_t)h * D + pd);
  }
  u32x4 kr[M::ROUNDS], vr[M::ROUNDS];
#pragma unroll
  for (int t = 0; t < M::ROUNDS; ++t) {
    const int64_t j = sq.start + j0 + min(t * M::RPB + slot, jn - 1);
    kr[t] = *(const u32x4*)(p.k + (j * p.k_rs + (int64_t)h * D + e0) * M::ES);
    vr[t] = *(const u32x4*)(p.v + (j * p.v_rs + (int64_t)h * D + e0) * M::ES);
  }
  if (tid < kPieces) {
    uint32_t qp[4];
    q8_pairs(p, qw, qp);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      qd2[pr][pd / 2 + i] = qp[i];
      dod2[pr][pd / 2 + i] = dw[i];
    }
  }
  __syncthreads();
  if constexpr (RP > 0) {
    for (int x = tid; x < RP * D; x += kThreads) {
      const int rp = x / D, d = x - rp * D;
      const uint32_t q0 = qd2[2 * rp][d / 2], q1 = qd2[2 * rp + 1][d / 2];
      const uint32_t o0 = dod2[2 * rp][d / 2], o1 = dod2[2 * rp + 1][d / 2];
      qr2[rp][d] = (d & 1) ? ((q0 >> 16) | (q1 & 0xffff0000u)) : ((q0 & 0xffffu) | (q1 << 16));
      dor2[rp][d] = (d & 1) ? ((o0 >> 16) | (o1 & 0xffff0000u)) : ((o0 & 0xffffu) | (o1 << 16));
    }
    __syncthreads();
  }
  const MaskCtx mc = delta_mask(p, sq);
  const float xs = p.alpha * p.q_scale, ka = p.alpha * p.q_scale;
  float dqa[DS][EPL] = {};
#pragma unroll
  for (int t = 0; t < M::ROUNDS; t += 2) {
    uint32_t kp[2][WPL], dsb[2][DS];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int jj = (t + u) * M::RPB + slot;
      uint32_t vp[WPL];
      real_pairs<FP8>(kr[t + u], p.k_scale, kp[u]);
      real_pairs<FP8>(vr[t + u], p.v_scale, vp);
      float w[DS], ds[DS];
#pragma unroll
      for (int r = 0; r < DS; ++r) {
        float sp = 0.f, dpp = 0.f;
#pragma unroll
        for (int c = 0; c < WPL; ++c) {
          sp = dot2(kp[u][c], qd2[r][e0 / 2 + c], sp);
          dpp = dot2(vp[c], dod2[r][e0 / 2 + c], dpp);
        }
        const float x = group_sum<M::LPR>(sp) * xs;
        const float dpv = group_sum<M::LPR>(dpp);
        const int i = sq.L - DS + r;
        w[r] = ds[r] = 0.f;
        if (jj < jl && i >= 0 && valid_generic(i, j0 + jj, mc)) {
          const float sg = __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(-kLog2e * x));
          w[r] = bf16_round(x * sg * p.inv_n);
          ds[r] = bf16_round(dpv * sg * (1.f + x * (1.f - sg)) * p.inv_n);
        }
        dsb[u][r] = __builtin_bit_cast(uint32_t, ds[r]) >> 16;
      }
      float dk[EPL], dv[EPL];
      if constexpr (RP == 0) {
#pragma unroll
        for (int e = 0; e < EPL; ++e) dk[e] = dv[e] = 0.f;
      } else {
#pragma unroll
        for (int e = 0; e < EPL; ++e) dk[e] = dv[e] = 0.f;
#pragma unroll
        for (int rp = 0; rp < RP; ++rp) {
          const uint32_t wp = (__builtin_bit_cast(uint32_t, w[2 * rp]) >> 16) |
                              (__builtin_bit_cast(uint32_t, w[2 * rp + 1]) & 0xffff0000u);
          const uint32_t sp2 = dsb[u][2 * rp] | (dsb[u][2 * rp + 1] << 16);
#pragma unroll
          for (int e = 0; e < EPL; ++e) {
            dv[e] = dot2(dor2[rp][e0 + e], wp, dv[e]);
            dk[e] = dot2(qr2[rp][e0 + e], sp2, dk[e]);
          }
        }
      }
      if constexpr (DS & 1) {  // the unpaired last row
#pragma unroll
        for (int c = 0; c < WPL; ++c) {
          const uint32_t qq = qd2[DS - 1][e0 / 2 + c], oo = dod2[DS - 1][e0 / 2 + c];
          dk[2 * c] = __builtin_fmaf(ds[DS - 1], bf_lo(qq), dk[2 * c]);
          dk[2 * c + 1] = __builtin_fmaf(ds[DS - 1], bf_hi(qq), dk[2 * c + 1]);
          dv[2 * c] = __builtin_fmaf(w[DS - 1], bf_lo(oo), dv[2 * c]);
          dv[2 * c + 1] = __builtin_fmaf(w[DS - 1], bf_hi(oo), dv[2 * c + 1]);
        }
      }
      if (jj < jn) {
        const int64_t jr = sq.start + j0 + jj;
        uint16_t* dkr = p.dk + jr * p.dk_rs + (int64_t)h * D + e0;
        uint16_t* dvr = p.dv + jr * p.dv_rs + (int64_t)h * D + e0;
#pragma unroll
        for (int c = 0; c < EPL / 8; ++c) {
          *(u32x4*)(dkr + 8 * c) = u32x4{pack_bf16(dk[8 * c] * ka, dk[8 * c + 1] * ka),
                                         pack_bf16(dk[8 * c + 2] * ka, dk[8 * c + 3] * ka),
                                         pack_bf16(dk[8 * c + 4] * ka, dk[8 * c + 5] * ka),
                                         pack_bf16(dk[8 * c + 6] * ka, dk[8 * c + 7] * ka)};
          *(u32x4*)(dvr + 8 * c) = u32x4{pack_bf16(dv[8 * c], dv[8 * c + 1]), pack_bf16(dv[8 * c + 2], dv[8 * c + 3]),
                                         pack_bf16(dv[8 * c + 4], dv[8 * c + 5]),
                                         pack_bf16(dv[8 * c + 6], dv[8 * c + 7])};
        }
      }
    }
    // dq over the key pair: (k_real_t[e], k_real_t+1[e]) against (dS_t, dS_t+1)
#pragma unroll
    for (int r = 0; r < DS; ++r) {
      const uint32_t sp2 = dsb[0][r] | (dsb[1][r] << 16);
#pragma unroll
      for (int c = 0; c < WPL; ++c) {
        dqa[r][2 * c] = dot2(__builtin_amdgcn_perm(kp[1][c], kp[0][c], 0x05040100u), sp2, dqa[r][2 * c]);
        dqa[r][2 * c + 1] = dot2(__builtin_amdgcn_perm(kp[1][c], kp[0][c], 0x07060302u), sp2, dqa[r][2 * c + 1]);
      }
    }
    // keep each round pair's unpacked K / V inside it (bounds the registers)
    __builtin_amdgcn_sched_barrier(0);
  }
  // the last chunk block also zeroes the rows of a sequence longer than its
  // chunks reach (rows past N have no attention)
  if (chunk == p.nchunk - 1) {
    for (int j = j0 + kChunk + slot; j < sq.len; j += M::RPB) {
#pragma unroll
      for (int c = 0; c < EPL / 8; ++c) {
        *(u32x4*)(p.dk + (sq.start + j) * p.dk_rs + (int64_t)h * D + e0 + 8 * c) = u32x4{0u, 0u, 0u, 0u};
        *(u32x4*)(p.dv + (sq.start + j) * p.dv_rs + (int64_t)h * D + e0 + 8 * c) = u32x4{0u, 0u, 0u, 0u};
      }
    }
  }
#pragma unroll
  for (int r = 0; r < DS; ++r) {
    __syncthreads();
#pragma unroll
    for (int e = 0; e < EPL; ++e) red[slot * D + e0 + e] = dqa[r][e];
    __syncthreads();
    if (tid < D) {
      float t = 0.f;
      for (int g = 0; g < M::RPB; ++g) t += red[g * D + tid];
      p.part[((((int64_t)b * DS + r) * p.H + h) * p.nchunk + chunk) * D + tid] = t;
    }
  }
}

// dq[row, h, :] = alpha * sum of the chunk partials in chunk order.
template <int D>
__global__ void delta_bwd_finalize(DeltaParams p) {
  const int row = blockIdx.x, h = blockIdx.y, d = threadIdx.x;
  if (d >= D) return;
  const int b = row / p.DS;
  const DeltaSeq sq = delta_seq(p, b);
  const int nc = (sq.len + kChunk - 1) / kChunk;
  const float* src = p.part + (((int64_t)row * p.H + h) * p.nchunk) * D + d;
  float t = 0.f;
  for (int c = 0; c < nc; ++c) t += src[(int64_t)c * D];
  p.dq[(int64_t)row * p.dq_rs + (int64_t)h * D + d] = to_bf16(t * p.alpha);
}

bool aligned(const void* ptr, int a) { return ((uintptr_t)ptr % a) == 0; }

template <int D, bool FP8>
void launch_bwd(int ds, dim3 grid, const DeltaParams& p, hipStream_t st) {
  static_assert(kMaxDsBwd == 4, "one kernel per delta size");
  switch (ds) {
    case 1: hipLaunchKernelGGL((delta_bwd_kernel<D, FP8, 1>), grid, dim3(kThreads), 0, st, p); break;
    case 2: hipLaunchKernelGGL((delta_bwd_kernel<D, FP8, 2>), grid, dim3(kThreads), 0, st, p); break;
    case 3: hipLaunchKernelGGL((delta_bwd_kernel<D, FP8, 3>), grid, dim3(kThreads), 0, st, p); break;
    default: hipLaunchKernelGGL((delta_bwd_kernel<D, FP8, 4>), grid, dim3(kThreads), 0, st, p); break;
  }
}

int nchunks(int N) { return (N + kChunk - 1) / kChunk; }

}  // namespace

extern "C" int64_t hstu_delta_attn_workspace_bytes(int B, int H, int D, int N, int delta_size) {
  if (B < 0 || H <= 0 || D <= 0 || N <= 0 || delta_size <= 0) return -1;
  return (int64_t)B * delta_size * H * nchunks(N) * D * 4;
}

namespace {
int delta_common_check(int dtype, int q_dtype, int B, int H, int D, int N, int DS, const void* q, const void* k,
                       const void* v, int64_t q_rs, int64_t k_rs, int64_t v_rs, const int64_t* seq_offsets,
                       void* ws, int64_t ws_bytes) {
  if (dtype != HSTU_DTYPE_BF16 && dtype != HSTU_DTYPE_FP8_E4M3) return HSTU_E_BAD_ARG;
  if (q_dtype != HSTU_DTYPE_BF16 && q_dtype != HSTU_DTYPE_FP8_E4M3) return HSTU_E_BAD_ARG;
  if (B < 0 || H <= 0 || N <= 0 || DS <= 0 || q == nullptr || k == nullptr || v == nullptr || seq_offsets == nullptr)
    return HSTU_E_BAD_ARG;
  if (q_rs < (int64_t)H * D || k_rs < (int64_t)H * D || v_rs < (int64_t)H * D) return HSTU_E_BAD_ARG;
  if (D != 64 && D != 128) return HSTU_E_UNSUPPORTED;
  const int es = dtype == HSTU_DTYPE_BF16 ? 2 : 1, qes = q_dtype == HSTU_DTYPE_BF16 ? 2 : 1;
  // the row pieces of q, k and v are read with 8- and 16-byte vector loads
  if (!aligned(k, 16) || !aligned(v, 16) || !aligned(q, 16) || (k_rs * es) % 16 || (v_rs * es) % 16 ||
      (q_rs * qes) % 16)
    return HSTU_E_UNSUPPORTED;
  if (ws == nullptr || ws_bytes < hstu_delta_attn_workspace_bytes(B, H, D, N, DS)) return HSTU_E_BAD_ARG;
  // one block per (head, chunk, row) in a 1-D grid; the finalize grid's y is H
  if ((int64_t)H * nchunks(N) * B * DS >= (int64_t)1 << 24 || H > 65535) return HSTU_E_UNSUPPORTED;
  return 0;
}
}  // namespace

extern "C" int hstu_delta_attn_fwd(int dtype, int q_dtype, const void* q, const void* k, const void* v, int64_t q_rs, int64_t k_rs,
                                   int64_t v_rs, float q_scale, float k_scale, float v_scale,
                                   const int64_t* seq_offsets, int B, int H, int D, int N, int delta_size,
                                   float alpha, const int* num_targets, int max_attn_len, int contextual_seq_len,
                                   void* out, int64_t out_rs, void* workspace, int64_t workspace_bytes,
                                   hipStream_t stream) {
  int st = delta_common_check(dtype, q_dtype, B, H, D, N, delta_size, q, k, v, q_rs, k_rs, v_rs, seq_offsets,
                              workspace, workspace_bytes);
  if (st) return st;
  if (out == nullptr || out_rs < (int64_t)H * D) return HSTU_E_BAD_ARG;
  if (B == 0) return 0;
  DeltaParams p{};
  p.q = (const uint8_t*)q;
  p.k = (const uint8_t*)k;
  p.v = (const uint8_t*)v;
  p.q_rs = q_rs;
  p.k_rs = k_rs;
  p.v_rs = v_rs;
  const bool fp8 = dtype == HSTU_DTYPE_FP8_E4M3;
  p.q_e4m3 = q_dtype == HSTU_DTYPE_FP8_E4M3;
  p.alpha = alpha;
  p.q_scale = p.q_e4m3 ? q_scale : 1.f;
  p.k_scale = fp8 ? k_scale : 1.f;
  p.v_scale = fp8 ? v_scale : 1.f;
  p.inv_n = 1.f / (float)N;
  p.seq_offsets = seq_offsets;
  p.B = B;
  p.H = H;
  p.N = N;
  p.DS = delta_size;
  p.num_targets = num_targets;
  p.max_attn_len = max_attn_len;
  p.contextual_seq_len = contextual_seq_len;
  p.part = (float*)workspace;
  p.nchunk = nchunks(N);
  p.out = (uint16_t*)out;
  p.out_rs = out_rs;
  const dim3 grid((uint32_t)((int64_t)H * p.nchunk * B * delta_size)), fin(B * delta_size, H);
  if (D == 128) {
    if (fp8) hipLaunchKernelGGL((delta_fwd_kernel<128, true>), grid, dim3(kThreads), 0, stream, p);
    else hipLaunchKernelGGL((delta_fwd_kernel<128, false>), grid, dim3(kThreads), 0, stream, p);
    hipLaunchKernelGGL(delta_fwd_finalize<128>, fin, dim3(128), 0, stream, p);
  } else {
    if (fp8) hipLaunchKernelGGL((delta_fwd_kernel<64, true>), grid, dim3(kThreads), 0, stream, p);
    else hipLaunchKernelGGL((delta_fwd_kernel<64, false>), grid, dim3(kThreads), 0, stream, p);
    hipLaunchKernelGGL(delta_fwd_finalize<64>, fin, dim3(64), 0, stream, p);
  }
  return (int)hipGetLastError();
}

extern "C" int hstu_delta_attn_bwd(int dtype, int q_dtype, const void* dout, int64_t do_rs, const void* q, const void* k,
                                   const void* v, int64_t q_rs, int64_t k_rs, int64_t v_rs, float q_scale,
                                   float k_scale, float v_scale, const int64_t* seq_offsets, int B, int H, int D,
                                   int N, int delta_size, float alpha, const int* num_targets, int max_attn_len,
                                   int contextual_seq_len, void* dq, void* dk, void* dv, int64_t dq_rs, int64_t dk_rs,
                                   int64_t dv_rs, void* workspace, int64_t workspace_bytes, hipStream_t stream) {
  int st = delta_common_check(dtype, q_dtype, B, H, D, N, delta_size, q, k, v, q_rs, k_rs, v_rs, seq_offsets,
                              workspace, workspace_bytes);
  if (st) return st;
  if (dout == nullptr || dq == nullptr || dk == nullptr || dv == nullptr || do_rs < (int64_t)H * D ||
      dq_rs < (int64_t)H * D || dk_rs < (int64_t)H * D || dv_rs < (int64_t)H * D)
    return HSTU_E_BAD_ARG;
  if (delta_size > kMaxDsBwd) return HSTU_E_UNSUPPORTED;
  if (!aligned(dk, 16) || !aligned(dv, 16) || !aligned(dout, 16) || dk_rs % 8 || dv_rs % 8 || do_rs % 8)
    return HSTU_E_UNSUPPORTED;
  if (B == 0) return 0;
  DeltaParams p{};
  p.q = (const uint8_t*)q;
  p.k = (const uint8_t*)k;
  p.v = (const uint8_t*)v;
  p.dout = (const uint16_t*)dout;
  p.q_rs = q_rs;
  p.k_rs = k_rs;
  p.v_rs = v_rs;
  p.do_rs = do_rs;
  const bool fp8 = dtype == HSTU_DTYPE_FP8_E4M3;
  p.q_e4m3 = q_dtype == HSTU_DTYPE_FP8_E4M3;
  p.alpha = alpha;
  p.q_scale = p.q_e4m3 ? q_scale : 1.f;
  p.k_scale = fp8 ? k_scale : 1.f;
  p.v_scale = fp8 ? v_scale : 1.f;
  p.inv_n = 1.f / (float)N;
  p.seq_offsets = seq_offsets;
  p.B = B;
  p.H = H;
  p.N = N;
  p.DS = delta_size;
  p.num_targets = num_targets;
  p.max_attn_len = max_attn_len;
  p.contextual_seq_len = contextual_seq_len;
  p.part = (float*)workspace;
  p.nchunk = nchunks(N);
  p.dq = (uint16_t*)dq;
  p.dk = (uint16_t*)dk;
  p.dv = (uint16_t*)dv;
  p.dq_rs = dq_rs;
  p.dk_rs = dk_rs;
  p.dv_rs = dv_rs;
  const dim3 grid((uint32_t)((int64_t)H * p.nchunk * B)), fin(B * delta_size, H);
  if (D == 128) {
    if (fp8) launch_bwd<128, true>(delta_size, grid, p, stream);
    else launch_bwd<128, false>(delta_size, grid, p, stream);
    hipLaunchKernelGGL(delta_bwd_finalize<128>, fin, dim3(128), 0, stream, p);
  } else {
    if (fp8) launch_bwd<64, true>(delta_size, grid, p, stream);
    else launch_bwd<64, false>(delta_size, grid, p, stream);
    hipLaunchKernelGGL(delta_bwd_finalize<64>, fin, dim3(64), 0, stream, p);
  }
  return (int)hipGetLastError();
}
