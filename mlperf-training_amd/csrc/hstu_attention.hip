// HSTU jagged causal SiLU attention for MI355X (gfx950, CDNA4).
//
//   out_i = sum_{valid j <= i} silu(alpha * q_i.k_j [+ bias(i-j)]) / N * v_j
//
// Forward and backward over jagged [T, H, D] tensors addressed through int64
// seq_offsets, no padding.  bf16 inputs use v_mfma_f32_16x16x32_bf16 for both
// contractions; e4m3 (OCP) inputs use v_mfma_f32_16x16x128_f8f6f4 for Q.K^T
// with per-(token, head) fp32 scales applied as a rank-1 factor on the score
// tile, and bf16 MFMA for P.V with V dequantized while it is staged into LDS
// (the reference's FP8 forward does the same: P and V go to bf16,
// ops/triton/triton_hstu_attention.py:503-520).
//
// Reference behaviour followed (paths relative to
// recommendation_v4/hstu/generative_recommenders/):
//   forward tile math   ops/triton/triton_hstu_attention.py:415-522
//   n-loop / diagonal   ops/triton/triton_hstu_attention.py:584-911
//   backward tile math  ops/triton/triton_hstu_attention.py:2090-2212, 2500
//   mask                ops/pytorch/pt_hstu_attention.py:32-84
//
// Design (per kernel, one workgroup = 4 waves of 64 lanes):
//   * every MFMA is 16x16; a lane's C fragment holds rows 4*(lane/16)+r,
//     column lane%16.  Scores are computed transposed (S^T = K.Q^T) where the
//     next contraction runs over keys, so the C fragment of S^T is already
//     the A operand of P.V: no shuffles between the two GEMMs.
//   * an operand whose contraction index runs along rows in memory (V for
//     P.V, dO / Q for dV / dK, K for dQ) is staged into LDS transposed, in a
//     key order ("sigma") that makes each lane's eight keys contiguous, so the
//     B operand is one ds_read_b128.  LDS row pitches are padded by 16 bytes,
//     which makes the 16-lane row reads of every operand conflict-free.
//   * SiLU uses the hardware exp2 / rcp: with t = -x*log2(e),
//     silu(x) = -ln2 * t / (1 + 2^t); the -ln2/N factor is applied once to
//     the fp32 accumulator instead of per score.
//   * tiles strictly below the diagonal skip the mask; tiles strictly above
//     it are never visited (per wave), so causal work is ~P pairs, not N^2.
//   * global -> register prefetch of tile t+1 overlaps the MFMAs of tile t;
//     LDS is double buffered with one barrier per tile.
//   * grids are 1-D with the heaviest blocks first (longest key range); the
//     (sequence, head) index is rotated per block level so that the 8 XCDs
//     (workgroup i runs on XCD i % 8) get equal shares of long sequences.
//   * dq/dk/dv are written exactly once (two kernels: dK/dV with the key block
//     outer, dQ with the query block outer); no atomics, deterministic.

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <climits>
#include <mutex>
#include <type_traits>
#include <vector>

#include "hstu_common.h"
#include "hstu_mi355x.h"

namespace {
using namespace hstu;

// ---------------------------------------------------------------- tile movers
// Each mover is split into load() (global -> registers, issued before the
// MFMAs of the current tile) and store() (registers -> LDS, after them).
// Rows at or beyond `nrows` are zero-filled.

// ROWS x D elements of ES bytes, copied as-is; LDS pitch D*ES + 16.
template <int ROWS, int D, int ES>
struct CopyTile {
  static constexpr int CPR = D * ES / 16;
  static constexpr int N = ROWS * CPR / kThreads;
  static constexpr int PITCH = D * ES + 16;
  static_assert(N >= 1 && ROWS * CPR % kThreads == 0, "tile/thread mismatch");
  u32x4 r[N];
  __device__ __forceinline__ void load(const uint8_t* base, int64_t rs_bytes, int row0, int nrows) {
#pragma unroll
    for (int i = 0; i < N; ++i) {
      const int item = threadIdx.x + kThreads * i, row = item / CPR, ch = item % CPR;
      r[i] = u32x4{0u, 0u, 0u, 0u};
      if (row0 + row < nrows) r[i] = *(const u32x4*)(base + (int64_t)(row0 + row) * rs_bytes + ch * 16);
    }
  }
  __device__ __forceinline__ void store(uint8_t* lds) const {
#pragma unroll
    for (int i = 0; i < N; ++i) {
      const int item = threadIdx.x + kThreads * i, row = item / CPR, ch = item % CPR;
      *(u32x4*)(lds + row * PITCH + ch * 16) = r[i];
    }
  }
};

// ROWS x D e4m3 rows -> bf16 rows (times the row's scale); LDS pitch 2D + 16.
template <int ROWS, int D>
struct DeqTile {
  static constexpr int CPR = D / 16;
  static constexpr int N = ROWS * CPR / kThreads;
  static constexpr int PITCH = D * 2 + 16;
  static_assert(N >= 1 && ROWS * CPR % kThreads == 0, "tile/thread mismatch");
  u32x4 r[N];
  float s[N];
  __device__ __forceinline__ void load(const uint8_t* base, int64_t rs_bytes, const float* sbase,
                                       int64_t srs, int row0, int nrows) {
#pragma unroll
    for (int i = 0; i < N; ++i) {
      const int item = threadIdx.x + kThreads * i, row = item / CPR, ch = item % CPR;
      r[i] = u32x4{0u, 0u, 0u, 0u};
      s[i] = 0.f;
      if (row0 + row < nrows) {
        r[i] = *(const u32x4*)(base + (int64_t)(row0 + row) * rs_bytes + ch * 16);
        s[i] = sbase[(int64_t)(row0 + row) * srs];
      }
    }
  }
  __device__ __forceinline__ void store(uint8_t* lds) const {
#pragma unroll
    for (int i = 0; i < N; ++i) {
      const int item = threadIdx.x + kThreads * i, row = item / CPR, ch = item % CPR;
      u32x2 a = fp8x4_to_bf16x4(r[i][0], s[i]), b = fp8x4_to_bf16x4(r[i][1], s[i]);
      u32x2 c = fp8x4_to_bf16x4(r[i][2], s[i]), d = fp8x4_to_bf16x4(r[i][3], s[i]);
      uint8_t* dst = lds + row * PITCH + ch * 32;
      *(u32x4*)dst = u32x4{a[0], a[1], b[0], b[1]};
      *(u32x4*)(dst + 16) = u32x4{c[0], c[1], d[0], d[1]};
    }
  }
};

// ROWS x D rows (bf16, or e4m3 times the row's scale) -> transposed bf16
// [D][ROWS] in sigma key order; LDS pitch 2*ROWS + 16.  One item = 4 rows x
// 8 columns, transposed in registers into 8 runs of 4 keys (ds_write_b64).
template <int ROWS, int D, bool FP8>
struct TransTile {
  static constexpr int ITEMS = (ROWS / 4) * (D / 8);
  static constexpr int PITCH = ROWS * 2 + 16;
  static_assert(ITEMS <= kThreads, "one item per thread");
  u32x4 r[4];   // bf16: 8 values per row; fp8: r[kk][0..1] holds 8 bytes
  float s[4];
  __device__ __forceinline__ void load(const uint8_t* base, int64_t rs_bytes, const float* sbase,
                                       int64_t srs, int row0, int nrows) {
    const int item = threadIdx.x;
    const int a = item % (ROWS / 4), c8 = item / (ROWS / 4);
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      r[kk] = u32x4{0u, 0u, 0u, 0u};
      s[kk] = 0.f;
      const int row = row0 + 4 * a + kk;
      if (item < ITEMS && row < nrows) {
        const uint8_t* src = base + (int64_t)row * rs_bytes;
        if constexpr (FP8) {
          u32x2 w = *(const u32x2*)(src + c8 * 8);
          r[kk][0] = w[0];
          r[kk][1] = w[1];
          s[kk] = sbase[(int64_t)row * srs];
        } else {
          r[kk] = *(const u32x4*)(src + c8 * 16);
        }
      }
    }
  }
  __device__ __forceinline__ void store(uint8_t* lds) const {
    const int item = threadIdx.x;
    if (item >= ITEMS) return;
    const int a = item % (ROWS / 4), c8 = item / (ROWS / 4);
    u32x4 w[4];
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      if constexpr (FP8) {
        u32x2 lo = fp8x4_to_bf16x4(r[kk][0], s[kk]);
        u32x2 hi = fp8x4_to_bf16x4(r[kk][1], s[kk]);
        w[kk] = u32x4{lo[0], lo[1], hi[0], hi[1]};
      } else {
        w[kk] = r[kk];
      }
    }
    uint8_t* col = lds + sigma(4 * a) * 2;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      // column pair (2e, 2e+1) of the 8-column chunk
      u32x2 ev = {(w[0][e] & 0xffffu) | (w[1][e] << 16), (w[2][e] & 0xffffu) | (w[3][e] << 16)};
      u32x2 od = {(w[0][e] >> 16) | (w[1][e] & 0xffff0000u), (w[2][e] >> 16) | (w[3][e] & 0xffff0000u)};
      *(u32x2*)(col + (8 * c8 + 2 * e) * PITCH) = ev;
      *(u32x2*)(col + (8 * c8 + 2 * e + 1) * PITCH) = od;
    }
  }
};

// ROWS per-row fp32 scales -> LDS (zero beyond nrows).
template <int ROWS>
struct ScaleTile {
  float s;
  __device__ __forceinline__ void load(const float* sbase, int64_t srs, int row0, int nrows) {
    s = 0.f;
    if (threadIdx.x < ROWS && row0 + (int)threadIdx.x < nrows) s = sbase[(int64_t)(row0 + threadIdx.x) * srs];
  }
  __device__ __forceinline__ void store(uint8_t* lds) const {
    if (threadIdx.x < ROWS) ((float*)lds)[threadIdx.x] = s;
  }
};


// ---------------------------------------------------------------- params
// Bias gradient: every dQ block (sequence, head, 128-query block) writes its
// own row of partial sums to the workspace; kDbiasChunks fixed-order partial
// sums of the rows, then their fixed-order sum, give dbias (no atomics).
constexpr int kDbiasChunks = 64;

// Length of one head's row of the pre-clamped bias table (build_bias_ext):
// entry off + N + 127 holds the bias of relative offset off, for every off a
// forward or dK/dV tile window can ask for.
__host__ __device__ inline int bias_ext_len(int N) { return 2 * N + 256; }

struct AttnParams {
  const uint8_t* q;
  const uint8_t* k;
  const uint8_t* v;
  const uint8_t* dout;
  int64_t q_rs, k_rs, v_rs, do_rs;  // row strides, elements
  const float* q_scale;
  const float* k_scale;
  const float* v_scale;
  int64_t s_rs, s_hs;
  const int64_t* seq_offsets;
  const int32_t* num_targets;
  uint16_t* out;  // forward output
  uint16_t* dq;
  uint16_t* dk;
  uint16_t* dv;
  int64_t o_rs, dq_rs, dk_rs, dv_rs;
  int B, H, N;
  float alpha, inv_n;
  int max_attn_len, contextual_seq_len;
  const float* bias;  // [H, 2*bias_R - 1] or null
  int bias_R;
  float* dbias;       // bias gradient, same shape (backward)
  const float* bias_ext;  // workspace: pre-clamped, pre-scaled bias rows [H, 2N+192]
  const uint8_t* q16;     // workspace: bf16 copy of e4m3 q, [T, H, D]
  float* dbias_part;      // workspace: one bias-gradient row per dQ block [blocks, H, dbias_w]
  const int64_t* dq_base;  // workspace: per-sequence exclusive prefix of 128-query blocks [B + 1]
  int dbias_w;            // floats per row: offsets 0 .. R-1 (causal), -(R-1) .. R-1 (generic masks)
  const int* sched_items;  // block schedule (schedule_block): [8][sched_cap] (sequence*H + head)
  const int* sched_start;  // [8][sched_cap + 1] first block position of each item on its XCD
  const int* sched_count;  // [8] items per XCD
  int sched_cap;
  int blocks_per_seq;  // ceil(N / 128)
  uint8_t* ds_ws;           // workspace: bf16 dS tiles written by dK/dV, read by dQ (causal masks)
  const int64_t* ds_base;   // workspace: per-sequence exclusive prefix of ds_tiles(L) [B + 1]
  // full-FP8 backward (hstu_attn_bwd_fp8)
  const uint8_t* do8;       // e4m3 dO [T, H, D], row stride do_rs bytes
  const uint8_t* e8;        // [T, H]: 127 - e of each token's dO group (dO8 = e4m3(dO * 2^e))
  const unsigned* f8max;    // workspace: kScaleParts partial maxima (float bits) of q_scale, k_scale
  float p8_scale;           // e4m3 P = silu / N * p8_scale (a power of two times N-relative)
  float ds8_scale;          // e4m3 dS = dS' * (scale normaliser) * ds8_scale
  // FP8 P.V forward (hstu_attn_fwd_fp8_pv)
  float pv_c;               // 2^-3 f32(2^3 / s): the sigmoid denominator factor of P' s
  float pv_out;             // f32(1 / s): undoes the P scale on the output
};

// ---------------------------------------------------------------- bias gradient rows
// A dQ block keeps one LDS histogram of dbias_w floats per wave.  A wave adds
// into its own histogram only, in program order, and the 64 lanes of one
// add hit distinct offsets, so every sum has one fixed order.  At the end
// the block adds its waves' histograms in wave order and stores the row of
// its slot (dq_base[b] + block) * H + h.

// The 64 lanes' sum, as lane 0 holds it after a fixed butterfly.
__device__ __forceinline__ float wave_sum_fixed(float x) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) x += __shfl_xor(x, off);
  return x;
}

// Adds a wave's per-lane clamped-offset sums into its histogram entry `at`
// (lane 0 after the fixed-order lane sum); call with the whole wave.
__device__ __forceinline__ void hist_add_clamped(float* hist_w, int at, float v, int lane) {
  const float s = wave_sum_fixed(v);
  if (lane == 0) hist_w[at] += s;
}

// Waits for every wave, then writes this block's row: the sum of the NW
// wave histograms (hist, NW x W floats) in wave order.
template <int NW>
__device__ __forceinline__ void dbias_store_row(const AttnParams& p, const float* hist, int b, int blk, int h) {
  __syncthreads();
  const int W = p.dbias_w;
  float* dst = p.dbias_part + ((p.dq_base[b] + blk) * p.H + h) * (int64_t)W;
  for (int i = threadIdx.x; i < W; i += NW * 64) {
    float v = hist[i];
#pragma unroll
    for (int w = 1; w < NW; ++w) v += hist[w * W + i];
    dst[i] = v;
  }
}

struct SeqCtx {
  int64_t start;
  int L, b, h, blk;
};
// Workgroup -> (sequence, head, 128-row block), from the schedule that
// schedule_block wrote: workgroup i runs on XCD x = i % 8 and takes the
// (i / 8)-th block of that XCD's list.  heavy_last: the block with the most
// key tiles is the last one of its sequence (forward, dQ) rather than the
// first (dK/dV); each item's blocks run heaviest first.  False = no work.
// With half != nullptr two workgroups share each block (i = 16 k + 8 h + x:
// half h of the k-th block), on the same XCD one after the other.
__device__ __forceinline__ bool seq_ctx(const AttnParams& p, bool heavy_last, SeqCtx& c, int* half = nullptr) {
  const int x = blockIdx.x & 7, k = half ? blockIdx.x >> 4 : blockIdx.x >> 3;
  if (half) *half = (blockIdx.x >> 3) & 1;
  const int n = p.sched_count[x];
  const int* st = p.sched_start + x * (p.sched_cap + 1);
  if (k >= st[n]) return false;
  int lo = 0, hi = n - 1;  // the last item whose first block is <= k
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (st[mid] <= k) lo = mid;
    else hi = mid - 1;
  }
  const int bh = p.sched_items[x * p.sched_cap + lo];
  const int m = k - st[lo];
  c.b = bh / p.H;
  c.h = bh - c.b * p.H;
  c.start = p.seq_offsets[c.b];
  c.L = min((int)(p.seq_offsets[c.b + 1] - c.start), p.N);
  const int nb = (c.L + 127) / 128;
  c.blk = heavy_last ? nb - 1 - m : m;
  return true;
}
// dS tiles.  For the causal mask the dK/dV kernel computes dS for key block
// kb (128 keys) against query tiles qt = 4 kb .. ceil(L/32) - 1 (32 queries);
// it stores each such (kb, qt) tile, bf16, for the dQ kernel to contract
// with K instead of recomputing S, dP and the SiLU derivative.  Tiles of one
// (sequence, head) are consecutive in kb-major order, so tile (kb, qt) is at
// kb * QT - 2 kb^2 - 2 kb + qt, and a sequence has ds_tiles(L) of them.
// Inside a tile (8 KiB): [wave w][key sub-tile kt][lane] 16-byte packs, the
// A operand of dK/dV's dK MFMA: keys 32 w + 16 kt + li, queries
// {4g .. 4g+3, 16+4g .. 16+4g+3} of the tile (times the query's e4m3 scale).
constexpr int kDsTileBytes = 8192;
__host__ __device__ inline int64_t ds_tiles(int64_t L) {
  const int64_t nb = (L + 127) / 128, qt = (L + 31) / 32;
  return nb * qt - 2 * nb * nb + 2 * nb;
}
__device__ __forceinline__ uint8_t* ds_tile(const AttnParams& p, const SeqCtx& c, int kb, int qt) {
  const int64_t QT = (c.L + 31) / 32;
  const int64_t idx = p.ds_base[c.b] * p.H + (int64_t)c.h * ds_tiles(c.L) + (int64_t)kb * QT -
                      2 * (int64_t)kb * kb - 2 * (int64_t)kb + qt;
  return p.ds_ws + idx * kDsTileBytes;
}

__device__ __forceinline__ MaskCtx mask_ctx(const AttnParams& p, const SeqCtx& c) {
  MaskCtx m;
  m.L = c.L;
  m.targets = p.num_targets != nullptr;
  m.nt = m.targets ? p.num_targets[c.b] : 0;
  m.ctx = p.contextual_seq_len;
  m.max_attn = p.max_attn_len;
  return m;
}

// =====================================================================
// Forward.  Block = 128 query rows (32 per wave), key tiles of 64.
// =====================================================================
// s_waitcnt vmcnt(N) with expcnt / lgkmcnt left at their maxima (gfx9 encoding).
template <int N>
__device__ __forceinline__ void wait_vm_le() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// Unpadded 128-byte e4m3 tile rows: data chunk c (bytes 16c .. 16c + 15) of
// row r sits at 16-byte slot c ^ swz128(r).  A ds_read_b128 of 16 consecutive
// rows (one chunk each) then hits 16 distinct bank groups, as do the
// transposed reads of row groups 8 and 32 apart; swz128 is constant under
// r -> r + 16.
__host__ __device__ constexpr int swz128(int r) { return ((r >> 1) & 7) ^ (((r >> 5) & 1) << 2); }

template <int D, bool FP8>
struct FwdCfg {
  static constexpr int BM = 128, BN = 64, KT = BN / 16, DT = D / 16, KS = D / 32;
  static constexpr int ES = FP8 ? 1 : 2;
  // bf16 rows at a pitch of row bytes + 32 (== 32 mod 64) for the 16-row
  // ds_read_b128 operand reads and the ds_read_b64_tr_b16 V reads; the e4m3
  // K tile uses unpadded swizzled rows (swz128) inside the same region.
  static constexpr int KP = D * ES + 32;
  static constexpr int VP = D * 2 + 32;
  static constexpr int K_OFF = 0;
  static constexpr int V_OFF = K_OFF + BN * KP;
  static constexpr int SC_OFF = V_OFF + BN * VP;              // e4m3: (sk, sv) per key
  static constexpr int BIAS_OFF = SC_OFF + (FP8 ? BN * 8 : 0);  // BM + BN bias values
  static constexpr int BUF = BIAS_OFF + (BM + BN) * 4;
  static constexpr int LDS = 2 * BUF;
  static constexpr int K_CPR = D * ES / 16;                 // 16-byte chunks per K row
  static constexpr int K_N = BN * K_CPR / kThreads;         // K chunks per thread
  // V source pieces per row: 16 bytes (bf16), or 8 e4m3 bytes that become one
  // 16-byte bf16 store, so that 16 lanes write one whole LDS row (256 bytes)
  // and a store instruction's passes hit distinct banks
  static constexpr int V_CPR = FP8 ? D / 8 : D * ES / 16;
  static constexpr int V_N = BN * V_CPR / kThreads;
};

// Registers of one staged K/V tile (global -> registers -> LDS).
template <int D, bool FP8>
struct FwdStage {
  using C = FwdCfg<D, FP8>;
  u32x4 k[C::K_N];
  std::conditional_t<FP8, u32x2, u32x4> v[C::V_N];
  float sc;    // e4m3: sk (threads 0..63) or sv (threads 64..127) of one key
  float bias;  // threads 0..BM+BN-2: one bias value of the tile's offset band
};

template <int D, bool FP8, bool GENERIC, bool BIAS>
__global__ void __launch_bounds__(kThreads, 2) hstu_fwd_kernel(AttnParams p) {
  using C = FwdCfg<D, FP8>;
  static_assert(!FP8 || D == 128, "e4m3 path is specialised for D = 128");
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];

  SeqCtx sc;
  if (!seq_ctx(p, /*heavy_last=*/true, sc)) return;
  const int L = sc.L, h = sc.h;
  const int m0 = sc.blk * C::BM;
  if (m0 >= L) return;
  const MaskCtx mc = mask_ctx(p, sc);

  const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63, li = lane & 15,
            g = lane >> 4;
  const int mw0 = m0 + wave * 32;
  const bool wave_active = mw0 < L;

  const uint32_t krs = (uint32_t)(p.k_rs * C::ES), vrs = (uint32_t)(p.v_rs * C::ES);
  const int64_t qrs = p.q_rs * C::ES;
  const uint8_t* qb = p.q + (sc.start * p.q_rs + (int64_t)h * D) * C::ES;
  // Buffer resources over this (sequence, head): rows >= L read as zero.
  const BufRsrc krsrc = make_rsrc(p.k + (sc.start * p.k_rs + (int64_t)h * D) * C::ES,
                                  (uint32_t)(L > 0 ? (L - 1) * krs + D * C::ES : 0));
  const BufRsrc vrsrc = make_rsrc(p.v + (sc.start * p.v_rs + (int64_t)h * D) * C::ES,
                                  (uint32_t)(L > 0 ? (L - 1) * vrs + D * C::ES : 0));
  const uint32_t s_step = FP8 ? (uint32_t)(p.s_rs * 4) : 0u;
  const uint32_t sbytes = FP8 ? (uint32_t)(p.s_rs ? L * p.s_rs * 4 : 4) : 0u;
  const BufRsrc sk_rsrc = make_rsrc(FP8 ? p.k_scale + sc.start * p.s_rs + h * p.s_hs : nullptr, sbytes);
  const BufRsrc sv_rsrc = make_rsrc(FP8 ? p.v_scale + sc.start * p.s_rs + h * p.s_hs : nullptr, sbytes);
  const float* biasb = BIAS ? p.bias + (int64_t)h * (2 * p.bias_R - 1) : nullptr;
  const int R1 = p.bias_R - 1;

  // per-thread constant staging offsets
  uint32_t k_voff[C::K_N], k_loff[C::K_N], v_voff[C::V_N], v_loff[C::V_N];
#pragma unroll
  for (int i = 0; i < C::K_N; ++i) {
    const int item = tid + kThreads * i, row = item / C::K_CPR, ch = item % C::K_CPR;
    k_voff[i] = row * krs + ch * 16;
    k_loff[i] = FP8 ? C::K_OFF + row * 128 + 16 * (ch ^ swz128(row)) : C::K_OFF + row * C::KP + ch * 16;
  }
#pragma unroll
  for (int i = 0; i < C::V_N; ++i) {
    const int item = tid + kThreads * i, row = item / C::V_CPR, ch = item % C::V_CPR;
    v_voff[i] = row * vrs + ch * (FP8 ? 8 : 16);
    v_loff[i] = C::V_OFF + row * C::VP + ch * 16;
  }

  // Q fragments (B operand of S^T = K.Q^T): lane holds query mw0+16qt+li.
  u32x4 qf[2][C::KS];
  i32x8 qf8[2];
  float cq[2];
#pragma unroll
  for (int qt = 0; qt < 2; ++qt) {
    const int row = mw0 + qt * 16 + li;
    const bool ok = row < L;
    const uint8_t* src = qb + (int64_t)row * qrs;
    cq[qt] = -p.alpha * kLog2e;
    if constexpr (FP8) {
      u32x4 lo = {0u, 0u, 0u, 0u}, hi = {0u, 0u, 0u, 0u};
      float s = 0.f;
      if (ok) {
        lo = *(const u32x4*)(src + 16 * g);
        hi = *(const u32x4*)(src + 64 + 16 * g);
        s = p.q_scale[(sc.start + row) * p.s_rs + h * p.s_hs];
      }
      qf8[qt] = cat8(lo, hi);
      cq[qt] *= s;
    } else {
#pragma unroll
      for (int st = 0; st < C::KS; ++st) {
        qf[qt][st] = u32x4{0u, 0u, 0u, 0u};
        if (ok) qf[qt][st] = *(const u32x4*)(src + (32 * st + 8 * g) * 2);
      }
    }
  }

  f32x4 o[2][C::DT];
#pragma unroll
  for (int qt = 0; qt < 2; ++qt)
#pragma unroll
    for (int dt = 0; dt < C::DT; ++dt) o[qt][dt] = zero4();

  int n_end = min(m0 + C::BM, L);
  if (GENERIC && m0 < p.contextual_seq_len) n_end = L;
  const int ntiles = (n_end + C::BN - 1) / C::BN;

  FwdStage<D, FP8> stg;
  auto load = [&](int n0) {
#pragma unroll
    for (int i = 0; i < C::K_N; ++i) stg.k[i] = buf_ld128(krsrc, k_voff[i], n0 * krs);
#pragma unroll
    for (int i = 0; i < C::V_N; ++i) {
      if constexpr (FP8) stg.v[i] = buf_ld64(vrsrc, v_voff[i], n0 * vrs);
      else stg.v[i] = buf_ld128(vrsrc, v_voff[i], n0 * vrs);
    }
    if constexpr (FP8) {
      // wave 0: the tile's key scales, wave 1: its value scales
      if (wave == 0) {
        stg.sc = buf_ldf(sk_rsrc, (uint32_t)lane * s_step, n0 * s_step);
      } else if (wave == 1) {
        stg.sc = buf_ldf(sv_rsrc, (uint32_t)lane * s_step, n0 * s_step);
      }
    }
    if constexpr (BIAS) {
      // offsets i-j of this tile span [m0-n0-(BN-1), m0-n0+BM-1]; scaled at
      // the LDS store, so that nothing waits for the loads before the tile's math
      if (tid < C::BM + C::BN - 1) {
        const int off = m0 - n0 - (C::BN - 1) + tid;
        stg.bias = biasb[min(max(off, -R1), R1) + R1];
      }
    }
  };
  auto store = [&](uint8_t* buf) {
#pragma unroll
    for (int i = 0; i < C::K_N; ++i) *(u32x4*)(buf + k_loff[i]) = stg.k[i];
#pragma unroll
    for (int i = 0; i < C::V_N; ++i) {
      if constexpr (FP8) {
        // exact e4m3 -> bf16 (scale 1); the per-key V scale is folded into P
        const u32x2 w = stg.v[i];
        u32x4 b;
#pragma unroll
        for (int e = 0; e < 2; ++e) {
          b[2 * e] = cvt_fp8x2_bf16<false>(w[e]);
          b[2 * e + 1] = cvt_fp8x2_bf16<true>(w[e]);
        }
        *(u32x4*)(buf + v_loff[i]) = b;
      } else {
        *(u32x4*)(buf + v_loff[i]) = stg.v[i];
      }
    }
    if constexpr (FP8) {
      // (sk, 1 / sv) per key: 1 / sv enters the sigmoid's denominator; a zero
      // scale (rows past L, all-zero rows) has V = 0, so any finite factor does
      float v = stg.sc;
      if (tid >= 64) v = v > 0.f ? 1.0f / v : 1.0f;
      if (tid < 128) ((float*)(buf + C::SC_OFF))[(tid & 63) * 2 + (tid >> 6)] = v;
    }
    if constexpr (BIAS) {
      if (tid < C::BM + C::BN - 1) ((float*)(buf + C::BIAS_OFF))[tid] = stg.bias * -kLog2e;
    }
  };

  // Per-lane LDS addresses (tile-invariant).
  // e4m3: lane group g holds the 16-byte k-chunks g and g+4 of a row (the
  // same order in both MFMA operands), so each b128 read is conflict-free.
  const int k_rd = C::K_OFF + li * C::KP + 16 * g;
  // e4m3 (swizzled rows 16 kt + li): chunks g and g + 4 at slots g ^ swz128 and that ^ 4,
  // swz128(16 kt + li) = (li >> 1) ^ 4 (kt >> 1)
  const int ka0 = C::K_OFF + li * 128 + 16 * (g ^ (li >> 1)), ka1 = ka0 ^ 64;
  // tr16: lane j of group g addresses row 4g + j/4 (+16 for the second half), column 4*(j%4)
  const int v_rd = C::V_OFF + (4 * g + (li >> 2)) * C::VP + (li & 3) * 8;
  // bias index of element (qt, kt, r) = bias_rd + 16*(qt-kt) - r
  const int bias_rd = 32 * wave + (C::BN - 1) + li - 4 * g;

  load(0);
  store(smem);
  __syncthreads();

  for (int t = 0; t < ntiles; ++t) {
    const int n0 = t * C::BN;
    const uint8_t* buf = smem + (t & 1) * C::BUF;
    if (t + 1 < ntiles) load(n0 + C::BN);

    if (wave_active && (GENERIC || n0 <= mw0 + 31)) {
      // ---- S^T = K . Q^T : s[kt][qt], keys n0+16kt+4g+r, query mw0+16qt+li
      f32x4 s[C::KT][2];
#pragma unroll
      for (int kt = 0; kt < C::KT; ++kt) {
        const uint8_t* krow = buf + k_rd + kt * 16 * C::KP;
        if constexpr (FP8) {
          const uint8_t* kb = buf + kt * 16 * 128;
          i32x8 a = cat8(lds_ld128(kb + (kt < 2 ? ka0 : ka1)), lds_ld128(kb + (kt < 2 ? ka1 : ka0)));
          s[kt][0] = mfma_fp8(a, qf8[0], zero4());
          s[kt][1] = mfma_fp8(a, qf8[1], zero4());
        } else {
          s[kt][0] = zero4();
          s[kt][1] = zero4();
#pragma unroll
          for (int st = 0; st < C::KS; ++st) {
            u32x4 a = lds_ld128(krow + st * 64);
            s[kt][0] = mfma_bf16(a, qf[0][st], s[kt][0]);
            s[kt][1] = mfma_bf16(a, qf[1][st], s[kt][1]);
          }
        }
      }
      // ---- SiLU epilogue on the accumulators, packed into P (A operand)
      const bool need_mask = GENERIC || (n0 + C::BN - 1 > mw0);
      // whole tile in the clamped bias region: one constant
      const bool bias_const = BIAS && (m0 - n0 - (C::BN - 1) >= R1);
      const float* bias_lds = (const float*)(buf + C::BIAS_OFF);
      u32x4 pa[2][C::BN / 32];
      auto epilogue = [&](auto masked_tag, auto bconst_tag) {
        constexpr bool MASKED = decltype(masked_tag)::value;
        constexpr bool BCONST = decltype(bconst_tag)::value;
        const float bconst = (BIAS && BCONST) ? bias_lds[0] : 0.f;
#pragma unroll
        for (int kt = 0; kt < C::KT; ++kt) {
          f32x4 skv = {1.f, 1.f, 1.f, 1.f}, svv = {1.f, 1.f, 1.f, 1.f};
          if constexpr (FP8) {
            const float* scp = (const float*)(buf + C::SC_OFF) + (kt * 16 + 4 * g) * 2;
            f32x4 a = *(const f32x4*)scp, b = *(const f32x4*)(scp + 4);
            skv = f32x4{a[0], a[2], b[0], b[2]};
            svv = f32x4{a[1], a[3], b[1], b[3]};
          }
#pragma unroll
          for (int qt = 0; qt < 2; ++qt) {
            float pv[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              float b = 0.f;
              if constexpr (BIAS) b = BCONST ? bconst : bias_lds[bias_rd + 16 * (qt - kt) - r];
              const float t = scaled_score<FP8, BIAS>(s[kt][qt][r], cq[qt], skv[r], b);
              // e4m3: t sigmoid sv = t / (2^t / sv + 1 / sv), svv holding 1 / sv
              float val;
              if constexpr (FP8) val = t * __builtin_amdgcn_rcpf(__builtin_fmaf(__builtin_amdgcn_exp2f(t), svv[r], svv[r]));
              else val = t * sig_of_t(t);
              if constexpr (MASKED) {
                const int i = mw0 + qt * 16 + li, j = n0 + kt * 16 + 4 * g + r;
                const bool ok = GENERIC ? valid_generic(i, j, mc) : (j <= i);
                val = ok ? val : 0.f;
              }
              pv[r] = val;
            }
            pa[qt][kt >> 1][(kt & 1) * 2 + 0] = pack_bf16(pv[0], pv[1]);
            pa[qt][kt >> 1][(kt & 1) * 2 + 1] = pack_bf16(pv[2], pv[3]);
          }
        }
      };
      if (need_mask) {
        if (bias_const) epilogue(std::true_type{}, std::true_type{});
        else epilogue(std::true_type{}, std::false_type{});
      } else {
        if (bias_const) epilogue(std::false_type{}, std::true_type{});
        else epilogue(std::false_type{}, std::false_type{});
      }
      // ---- O += P . V  (V rows read transposed by ds_read_b64_tr_b16); the
      // raised wave priority lets this wave's MFMAs issue ahead of the other
      // workgroup's epilogue VALU work on the same SIMD
      __builtin_amdgcn_s_setprio(1);
#pragma unroll
      for (int c = 0; c < C::BN / 32; ++c) {
#pragma unroll
        for (int dt = 0; dt < C::DT; ++dt) {
          const uint8_t* vp = buf + v_rd + c * 32 * C::VP + dt * 32;
          u32x4 bv = cat_tr(lds_tr16(vp), lds_tr16(vp + 16 * C::VP));
          o[0][dt] = mfma_bf16(pa[0][c], bv, o[0][dt]);
          o[1][dt] = mfma_bf16(pa[1][c], bv, o[1][dt]);
        }
      }
      __builtin_amdgcn_s_setprio(0);
    }

    if (t + 1 < ntiles) store(smem + ((t + 1) & 1) * C::BUF);
    __syncthreads();
  }

  if (!wave_active) return;
  const float fin = -kLn2 * p.inv_n;
#pragma unroll
  for (int qt = 0; qt < 2; ++qt) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int row = mw0 + qt * 16 + 4 * g + r;
      if (row < L) {
        uint16_t* dst = p.out + (sc.start + row) * p.o_rs + (int64_t)h * D + li;
#pragma unroll
        for (int dt = 0; dt < C::DT; ++dt) dst[dt * 16] = to_bf16(o[qt][dt][r] * fin);
      }
    }
  }
}

// =====================================================================
// FP8 P.V forward (hstu_attn_fwd_fp8_pv): the reference's production
// forward contract DLRM_HSTU_FP8_FWD_PV=1 (ops/flydsl/hstu_flydsl_mha.py:
// 2199-2330; the gin default, dlrm_v4/train/gin/yambda_5b.gin:3293-3319).
// The SiLU output is rounded to e4m3 with a static scale s before P.V:
//   P' = -log2(e) silu(x)    (the exp2-domain SiLU: x' = -log2(e) x,
//                             P' = x' / (1 + 2^x'))
//   P8 = e4m3_sat(P' s r_k), out = sum_k P8 v8_k 2^E(k) (-ln2 / (s N)) [s_v]
// V stays raw e4m3 and P.V is an e4m3 MFMA.  With one per-tensor V scale
// (the reference's qkv_scale) r_k = 1 and s_v rides on the output.  With
// per-(token, head) V scales r_k = s_v(k) 2^-E(k), E(k) the frexp exponent
// of the largest V scale among the 32 keys of the tile that share k's bit 4,
// and 2^E(k) returns as the E8M0 block scale of the P.V MFMA.
//
// Block = 128 queries, 4 waves of 32; key tiles of 64.  All products are
// 32x32x64 e4m3 MFMAs.  S = Q.K^T leaves a lane one key (column) and 16
// queries, so the per-key scales and the sigmoid factor are lane scalars and
// the 16 per-query factors stay in registers for the whole loop.  The e4m3 P
// goes through a per-wave LDS region as P^T [key][query] (4-byte stores)
// and comes back transposed (ds_read_b64_tr_b8) as the A operand of
// O = P.V, with lane group g holding keys 32 g .. 32 g + 31; V's B operand
// reads the same keys from the V tile, also transposed.  The S products of
// the next 32-key sub-tile are issued before each sub-tile's epilogue, so the
// matrix cores work through them while the wave runs the SiLU.
// =====================================================================
// The largest x over the 32 lanes of the wave that share bit 4 of the lane
// index: DPP within each 16-lane row (lane ^ 1, ^ 2, then the mirrors that
// pair quads and half-rows), then rows r and r + 2 through permlane32_swap.
// All VALU: no LDS round trip.
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float max_lanes_same_bit4(float x) {
  x = fmaxf(x, dpp_f32<0xB1>(x));   // quad_perm [1, 0, 3, 2]: lane ^ 1
  x = fmaxf(x, dpp_f32<0x4E>(x));   // quad_perm [2, 3, 0, 1]: lane ^ 2
  x = fmaxf(x, dpp_f32<0x141>(x));  // row_half_mirror: the other quad of 8
  x = fmaxf(x, dpp_f32<0x140>(x));  // row_mirror: the other half of 16
  const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_int(x), __float_as_int(x), false, false);
  return fmaxf(x, __int_as_float((threadIdx.x & 32) ? sw[0] : sw[1]));
}

struct Pv8Cfg {
  static constexpr int BM = 128, BN = 64;
  // K ring of 3 tiles (tile t + 2 is staged while t and t + 1 are read),
  // V ring of 2; 64 rows of 128 e4m3 bytes each, unpadded: chunk c of K row
  // r at 16-byte slot c ^ swz128(r), of V row r at c ^ v_swz(r)
  static constexpr int KT = BN * 128;
  static constexpr int K_OFF = 0;
  static constexpr int VS_OFF = 3 * KT;
  // V stage: V rows, then the BM + BN - 1 bias values of the tile in four
  // copies, copy c shifted by c floats (copy_c[y] = window[y - c]), so that
  // every lane reads its runs of four with 16-byte aligned ds_read_b128s from
  // the copy that aligns them.  The copies start at dwords 0, 204, 412, 620
  // (0, 12, 28, 44 mod 64): the 16 lanes of a read pass, four of each copy,
  // then cover the 64 banks once.
  static constexpr int V_REL = 0, BIAS_REL = BN * 128;
  __host__ __device__ static constexpr int bias_copy(int c) { return c == 0 ? 0 : c == 1 ? 204 : c == 2 ? 412 : 620; }
  static constexpr int VSTAGE = BIAS_REL + (620 + 200) * 4;
  static constexpr int P_OFF = VS_OFF + 2 * VSTAGE;  // per wave: P^T, 64 keys x 32 queries
  // the block's table: two E8M0 bytes (as ints) per key tile, then c_k per key
  static constexpr int TAB_OFF = P_OFF + 4 * BN * 32;
  static int lds(int N) {
    const int nt = (N + BN - 1) / BN;
    return TAB_OFF + 8 * nt + 4 * BN * nt;
  }
  static_assert(VSTAGE % 16 == 0, "stage alignment");
  __host__ __device__ static constexpr int v_swz(int r) { return r & 6; }
};

template <bool BIAS>
__global__ void __launch_bounds__(kThreads, 2) hstu_fwd_pv8_kernel(AttnParams p) {
  using C = Pv8Cfg;
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  SeqCtx sc;
  if (!seq_ctx(p, /*heavy_last=*/true, sc)) return;
  const int L = sc.L, h = sc.h;
  const int m0 = sc.blk * C::BM;
  if (m0 >= L) return;
  const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int l32 = lane & 31, hg = lane >> 5, j16 = lane & 15, hi16 = (lane >> 4) & 1;
  const int mw0 = m0 + 32 * wave;
  const bool per_tensor = p.s_rs == 0;

  const uint32_t krs = (uint32_t)p.k_rs, vrs = (uint32_t)p.v_rs;
  const BufRsrc krsrc = make_rsrc(p.k + sc.start * p.k_rs + (int64_t)h * 128, L > 0 ? (L - 1) * krs + 128 : 0u);
  const BufRsrc vrsrc = make_rsrc(p.v + sc.start * p.v_rs + (int64_t)h * 128, L > 0 ? (L - 1) * vrs + 128 : 0u);
  const uint32_t s_step = (uint32_t)(p.s_rs * 4);
  const uint32_t sbytes = (uint32_t)(p.s_rs ? L * p.s_rs * 4 : 4);
  const BufRsrc sk_rsrc = make_rsrc(p.k_scale + sc.start * p.s_rs + h * p.s_hs, sbytes);
  const BufRsrc sv_rsrc = make_rsrc(p.v_scale + sc.start * p.s_rs + h * p.s_hs, sbytes);
  const float* biasb = BIAS ? p.bias + (int64_t)h * (2 * p.bias_R - 1) : nullptr;
  const int R1 = p.bias_R - 1;

  // K/V staging by LDS DMA: wave w's load i writes the 1 KiB of rows
  // 8 w + 32 i .. + 7 of the tile; lane l lands in slot l % 8 of row
  // 8 w + 32 i + l / 8 and so loads the data chunk that slot holds,
  // (l % 8) ^ swizzle(row)
  uint32_t k_voff[2], v_voff[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int row = 8 * wave + 32 * i + (lane >> 3), slot = lane & 7;
    k_voff[i] = row * krs + 16 * (slot ^ swz128(row));
    v_voff[i] = row * vrs + 16 * (slot ^ C::v_swz(row));
  }

  // Q (A operand of S): query mw0 + l32, bytes 64 kk + 32 hg .. + 31 of its row
  i32x8 qa[2];
  // -alpha log2(e) s_q of query mw0 + l32 in the half-wave hg = b, 0 in the
  // other: the A operand of the outer product that scales key sub-tile b
  float cqa[2];
  {
    const int row = mw0 + l32;
    const bool ok = row < L;
    const uint8_t* src = p.q + (sc.start + row) * p.q_rs + (int64_t)h * 128 + 32 * hg;
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      u32x4 lo = {0u, 0u, 0u, 0u}, hi = {0u, 0u, 0u, 0u};
      if (ok) {
        lo = *(const u32x4*)(src + 64 * kk);
        hi = *(const u32x4*)(src + 64 * kk + 16);
      }
      qa[kk] = cat8(lo, hi);
    }
    const float cq = ok ? -p.alpha * kLog2e * p.q_scale[(sc.start + row) * p.s_rs + h * p.s_hs] : 0.f;
    cqa[0] = hg ? 0.f : cq;
    cqa[1] = hg ? cq : 0.f;
  }

  f32x16 o[4];
#pragma unroll
  for (int db = 0; db < 4; ++db)
#pragma unroll
    for (int r = 0; r < 16; ++r) o[db][r] = 0.f;

  const int n_end = min(m0 + C::BM, L);
  const int ntiles = (n_end + C::BN - 1) / C::BN;
  // tiles this wave computes: key tile t is needed while 64 t <= mw0 + 31
  const int wtiles = mw0 < L ? min(ntiles, (mw0 + 31) / C::BN + 1) : 0;
  // the block's table of E8M0 bytes (two per key tile) and per-key c_k
  int* const e8t = (int*)(smem + C::TAB_OFF);
  float* const ckt = (float*)(smem + C::TAB_OFF + 8 * ((p.N + C::BN - 1) / C::BN));

  float st_bias = 0.f;
  auto load_k = [&](int n0, uint8_t* kbuf) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < 2; ++i) buf_to_lds<16>(krsrc, kbuf + (8 * wave + 32 * i) * 128, k_voff[i], n0 * krs);
  };
  // key scales of the tile at n0, lane = key (every wave loads its own)
  auto load_sk = [&](int n0) __attribute__((always_inline)) {
    return buf_ldf(sk_rsrc, (uint32_t)lane * s_step, n0 * s_step);
  };
  auto load_v = [&](int n0, uint8_t* vbuf) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < 2; ++i)
      buf_to_lds<16>(vrsrc, vbuf + C::V_REL + (8 * wave + 32 * i) * 128, v_voff[i], n0 * vrs);
    if constexpr (BIAS) {
      // offsets i - j of the tile span [m0 - n0 - (BN - 1), m0 - n0 + BM - 1]
      // (threads tid < BM + BN - 1 store theirs)
      const int off = m0 - n0 - (C::BN - 1) + tid;
      st_bias = biasb[min(max(off, -R1), R1) + R1];
    }
  };
  // the V stage's bias window
  auto store_v = [&](uint8_t* vbuf) __attribute__((always_inline)) {
    if constexpr (BIAS) {
      if (tid < C::BM + C::BN - 1) {
        float* w = (float*)(vbuf + C::BIAS_REL);
        const float x = st_bias * -kLog2e;
#pragma unroll
        for (int c = 0; c < 4; ++c) w[C::bias_copy(c) + tid + c] = x;
      }
    }
  };
  auto kbuf = [&](int t) { return smem + C::K_OFF + (t % 3) * C::KT; };
  auto vbuf = [&](int t) { return smem + C::VS_OFF + (t & 1) * C::VSTAGE; };
  // the K stage of tile t as a wave-uniform byte offset: one add per read address
  auto kstage = [&](int t) { return (uint32_t)__builtin_amdgcn_readfirstlane((t % 3) * C::KT); };

  // K (B operand of S) reads: key 32 b + l32, chunks 4 kk + 2 hg + e at slots
  // (4 kk + 2 hg + e) ^ swz128(32 b + l32) = ((2 hg + e) ^ swz128(l32)) ^ 4 (kk ^ b)
  const int x0 = swz128(l32);
  const int ka0 = l32 * 128 + 16 * ((2 * hg) ^ x0), ka1 = l32 * 128 + 16 * ((2 * hg + 1) ^ x0);
  const int kx0 = ka0 ^ 64, kx1 = ka1 ^ 64;
  // S of key sub-tile b (32 keys) of a K tile: lane key 32 b + l32, register j
  // query 8 (j / 4) + 4 hg + j % 4
  // (the operands k[0], k[1] pair with qa[0], qa[1])
  auto k_read = [&](uint32_t kst, int b, i32x8 (&k)[2]) __attribute__((always_inline)) {
    const uint8_t* kb = smem + C::K_OFF + kst + 4096 * b;
    k[0] = cat8(lds_ld128(kb + (b ? kx0 : ka0)), lds_ld128(kb + (b ? kx1 : ka1)));
    k[1] = cat8(lds_ld128(kb + (b ? ka0 : kx0)), lds_ld128(kb + (b ? ka1 : kx1)));
  };
  auto s_mfma = [&](uint32_t kst, int b) __attribute__((always_inline)) {
    i32x8 k[2];
    k_read(kst, b, k);
    f32x16 z;
#pragma unroll
    for (int r = 0; r < 16; ++r) z[r] = 0.f;
    return mfma32_fp8(qa[1], k[1], mfma32_fp8(qa[0], k[0], z));
  };
  // P^T: key row 32 b + l32 (32 bytes); byte 16 hg + 4 i + r holds query
  // 8 i + 4 hg + r, so a lane stores its 16 bytes at once, in 16-byte chunk
  // hg ^ ((row >> 2) & 1): a store's 8-lane passes (8 rows) then cover all
  // 32 banks, and so do the transposed reads' 16-lane passes
  uint8_t* const pw = smem + C::P_OFF + 2048 * wave;
  const int pst = l32 * 32 + 16 * (hg ^ ((l32 >> 2) & 1));
  // bias index of (key sub-tile b, register j): bias_lo + 32 (1 - b) + 8 (j / 4) + j % 4
  const int bias_lo = 32 * wave + 4 * hg - l32 + (C::BN - 1) - 32;
  // SiLU epilogue of one key sub-tile into P^T (e4m3); scl holds the score
  // scales c_q s_k of the sub-tile's elements (the outer product).  hook(g),
  // g = 0..2, issues one of the caller's MFMAs; the scheduling groups at the
  // end place them one at a time between pieces of this wave's VALU work
  // instead of back to back (a wave does not issue past an MFMA that waits
  // for the matrix core)
  // the lane's 16 bias values (the window holds clamped values, so tiles
  // past the bias range read their constant) and c_k of key sub-tile b,
  // read ahead of the epilogue that uses them
  // the lane's runs start at window index bias_lo + 32 (1 - b) + 8 i, which
  // is 3 - l32 mod 4: copy (l32 + 1) & 3 holds them 16-byte aligned
  const int bias_c = (l32 + 1) & 3;
  const int bias_at = 4 * (C::bias_copy(bias_c) + bias_lo + bias_c);
  auto load_bias = [&](const uint8_t* vb, int n0, int b, float (&bj)[16], float& ck) __attribute__((always_inline)) {
    // the lane's base as an opaque LDS address, so that its four reads share
    // one base register and differ in the instructions' offsets
    uint32_t baddr =
        (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) uint8_t*)(vb + C::BIAS_REL) + bias_at;
    if constexpr (BIAS) asm volatile("" : "+v"(baddr));
    const __attribute__((address_space(3))) f32x4* bias_lane =
        (const __attribute__((address_space(3))) f32x4*)(uintptr_t)(baddr + 128 * (1 - b));
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const f32x4 v = BIAS ? bias_lane[2 * i] : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int r = 0; r < 4; ++r) bj[4 * i + r] = v[r];
    }
    ck = ckt[n0 + 32 * b + l32];
  };
  auto epilogue = [&](const f32x16& s, const f32x16& scl, int b, int n0, const float (&bj)[16], float ck,
                      auto masked_tag, auto&& hook) __attribute__((always_inline)) {
    constexpr bool MASKED = decltype(masked_tag)::value;
    const int key = n0 + 32 * b + l32;
    u32x4 pk;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if (i > 0) hook(i - 1);
      float pv[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int j = 4 * i + r;
        float x;
        if constexpr (BIAS) x = __builtin_fmaf(s[j], scl[j], bj[j]);
        else x = s[j] * scl[j];
        // P' s r_k = x / ((2^x + 1) / (s r_k)), c_k = 1 / (s r_k)
        float v = x * __builtin_amdgcn_rcpf(__builtin_fmaf(__builtin_amdgcn_exp2f(x), ck, ck));
        if constexpr (MASKED) v = key <= mw0 + 8 * i + 4 * hg + r ? v : 0.f;
        pv[r] = v;
      }
      pk[i] = pack_fp8x4(pv[0], pv[1], pv[2], pv[3]);
    }
    *(u32x4*)(pw + pst + 1024 * b) = pk;
#pragma unroll
    for (int g = 0; g < 3; ++g) {
      __builtin_amdgcn_sched_group_barrier(0x402, 24, 0);  // VALU incl. transcendental
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // one MFMA
    }
  };
  auto run_epilogue = [&](const f32x16& s, const f32x16& scl, int b, int n0, const float (&bj)[16], float ck,
                          auto&& hook) __attribute__((always_inline)) {
    if (n0 + 32 * b + 31 > mw0) epilogue(s, scl, b, n0, bj, ck, std::true_type{}, hook);
    else epilogue(s, scl, b, n0, bj, ck, std::false_type{}, hook);
  };
  // P (A operand of P.V) reads, u = 0..3: key rows 32 hg + 8 u + j16 / 2,
  // byte column 16 hi16 + 8 (j16 & 1), in chunk hi16 ^ (j16 >> 3); lane l32
  // of the operand then holds query 8 ((l32 & 15) >> 2) + 4 (l32 >> 4) + (l32 & 3)
  int pld[4];
#pragma unroll
  for (int u = 0; u < 4; ++u)
    pld[u] = (32 * hg + 8 * u + (j16 >> 1)) * 32 + 16 * (hi16 ^ (j16 >> 3)) + 8 * (j16 & 1);
  // V (B operand of P.V) reads for d block db: key rows 32 hg + 8 u + j16 / 2,
  // chunk 2 db + hi16 at slot (2 db + hi16) ^ v_swz(row) (v_swz(row) = (j16 >> 1) & 6)
  const int vsw = (j16 >> 1) & 6;
  int vld[4];
#pragma unroll
  for (int db = 0; db < 4; ++db)
    vld[db] = C::V_REL + (32 * hg + (j16 >> 1)) * 128 + 16 * ((2 * db + hi16) ^ vsw) + 8 * (j16 & 1);

  // per-key factors c_k = 1 / (s r_k), r_k = s_v 2^-E over the key's group
  // (the keys of its 64-key tile with the same bit 4), and the group's
  // E8M0 byte 127 + E, for all of the block's key tiles: wave w takes tiles
  // w, w + 4, .. (lane = key), four value-scale loads at a time
  for (int T0 = wave; T0 < ntiles; T0 += 16) {
    float svs[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) svs[u] = buf_ldf(sv_rsrc, (uint32_t)lane * s_step, (uint32_t)(64 * (T0 + 4 * u)) * s_step);
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int T = T0 + 4 * u;
      if (T >= ntiles) break;
      const float sv = svs[u];
      float c = p.pv_c;
      int e8 = 127;
      if (!per_tensor) {
        const float m = max_lanes_same_bit4(sv);
        int e = 0;
        if (m > 0.f) (void)frexpf(m, &e);
        e8 = 127 + e;
        if (sv > 0.f) c = ldexpf(p.pv_c * __builtin_amdgcn_rcpf(sv), e);
      }
      ckt[64 * T + lane] = c;
      if ((lane & 47) == 0) e8t[2 * T + (lane >> 4)] = e8;
    }
  }

  // prologue: K tiles 0 and 1, V tile 0, S of sub-tile (0, 0)
  fp8_saturate_mode(true);
  float sk_cur = load_sk(0), sk_next = 0.f;
  load_k(0, kbuf(0));
  load_v(0, vbuf(0));
  load_k(C::BN, kbuf(1));
  store_v(vbuf(0));
  lds_dma_wait();
  __syncthreads();
  f32x16 s0, s1, sc0, sc1;
  if (wtiles > 0) {
    s0 = s_mfma(kstage(0), 0);
    sc0 = mfma32_outer(cqa[0], sk_cur);
  }

  // tile t: S(t, 1) and the score scales of sub-tile (t, 1) run on the
  // matrix cores during the epilogue of (t, 0), S(t + 1, 0) and its scales
  // during that of (t, 1); K is staged two tiles ahead, V one (the DMA into
  // a stage starts a barrier after the stage's last reads).  The key
  // scales of tile t + 1 are loaded first, so that waiting for them does not
  // wait for the K/V loads; every load is issued on every tile (past the
  // sequence the buffer range check returns zeros into a stage nobody reads,
  // the bias index is clamped), so the wait counts the compiler derives are
  // exact instead of falling back to waiting for all loads
  for (int t = 0; t < ntiles; ++t) {
    const int n0 = t * C::BN;
    sk_next = load_sk(n0 + C::BN);
    __builtin_amdgcn_sched_barrier(0);  // issued before the tile loads
    load_k(n0 + 2 * C::BN, kbuf(t + 2));
    load_v(n0 + C::BN, vbuf(t + 1));
    const uint8_t* vb = vbuf(t);
    if (t < wtiles) {
      // S(t, 1) and its scales during the epilogue of (t, 0); S(t + 1, 0)
      // and its scales during that of (t, 1) (computed, unused, past the
      // wave's last tile: the K stage and the key scales are in bounds)
      i32x8 kr[2];
      k_read(kstage(t), 1, kr);
      // both sub-tiles' bias values and c_k now: sub-tile 1's arrive during
      // the epilogue of sub-tile 0
      float bj0[16], bj1[16], ck0, ck1;
      load_bias(vb, n0, 0, bj0, ck0);
      load_bias(vb, n0, 1, bj1, ck1);
      run_epilogue(s0, sc0, 0, n0, bj0, ck0, [&](int g) __attribute__((always_inline)) {
        if (g == 0) {
          f32x16 z;
#pragma unroll
          for (int r = 0; r < 16; ++r) z[r] = 0.f;
          s1 = mfma32_fp8(qa[0], kr[0], z);
        } else if (g == 1) {
          s1 = mfma32_fp8(qa[1], kr[1], s1);
        } else {
          sc1 = mfma32_outer(cqa[1], sk_cur);
        }
      });
      k_read(kstage(t + 1), 0, kr);
      run_epilogue(s1, sc1, 1, n0, bj1, ck1, [&](int g) __attribute__((always_inline)) {
        if (g == 0) {
          f32x16 z;
#pragma unroll
          for (int r = 0; r < 16; ++r) z[r] = 0.f;
          s0 = mfma32_fp8(qa[0], kr[0], z);
        } else if (g == 1) {
          s0 = mfma32_fp8(qa[1], kr[1], s0);
        } else {
          sc0 = mfma32_outer(cqa[0], sk_next);
        }
      });
      // the wave's own P^T stores precede its transposed reads (LDS keeps a
      // wave's operations in order); this only stops the compiler reordering
      asm volatile("" ::: "memory");
      i32x8 pa;
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const u32x2 w = lds_tr8(pw + pld[u]);
        pa[2 * u] = (int)w[0];
        pa[2 * u + 1] = (int)w[1];
      }
      const int e8v = e8t[2 * t + hg];
      // ---- O += P.V, V's group scales as the B operand's E8M0
#pragma unroll
      for (int db = 0; db < 4; ++db) {
        i32x8 bv;
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const u32x2 w = lds_tr8(vb + vld[db] + 1024 * u);
          bv[2 * u] = (int)w[0];
          bv[2 * u + 1] = (int)w[1];
        }
        o[db] = mfma32_fp8_scaled(pa, bv, o[db], 127, e8v);
      }
    }
    store_v(vbuf(t + 1));
    sk_cur = sk_next;
    // this wave's LDS DMA of tiles t + 1 (V) and t + 2 (K) has landed; the
    // barrier publishes all four waves'
    lds_dma_wait();
    __syncthreads();
  }
  fp8_saturate_mode(false);

  if (mw0 >= L) return;
  float fin = -kLn2 * p.inv_n * p.pv_out;
  if (per_tensor) fin *= p.v_scale[0];
  // lane: d = 32 db + l32, register j: operand row 8 i + 4 hg + r (i = j / 4,
  // r = j % 4), which is query 16 (i & 1) + 8 hg + 4 (i >> 1) + r (the P^T byte order)
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    const int i = j >> 2;
    const int row = mw0 + 16 * (i & 1) + 8 * hg + 4 * (i >> 1) + (j & 3);
    if (row < L) {
      uint16_t* dst = p.out + (sc.start + row) * p.o_rs + (int64_t)h * 128 + l32;
#pragma unroll
      for (int db = 0; db < 4; ++db) dst[32 * db] = to_bf16(o[db][j] * fin);
    }
  }
}

// =====================================================================
// Backward.  Both kernels stage their per-tile operands as bf16 rows (e4m3
// inputs are converted exactly, scale 1, while staging; the per-row scales
// are applied in the epilogue), so one LDS copy of a tile serves as an A
// operand (row reads, ds_read_b128) and as a B operand (ds_read_b64_tr_b16).
// A row pitch of 2D+32 bytes (== 32 mod 64) keeps both read patterns free
// of bank conflicts.
// =====================================================================
template <int D>
struct BwdPitch {
  static constexpr int P = D * 2 + 32;
};

// ROWS x D input rows (bf16, or e4m3 converted exactly) -> bf16 LDS rows.
template <int ROWS, int D, bool FP8>
struct RowStage {
  static constexpr int ES = FP8 ? 1 : 2;
  static constexpr int CPR = D * ES / 16;  // 16-byte source chunks per row
  static constexpr int ITEMS = ROWS * CPR;
  static constexpr int N = (ITEMS + kThreads - 1) / kThreads;
  u32x4 r[N];
  uint32_t voff[N], loff[N];
  __device__ __forceinline__ void init(uint32_t rs_bytes, int lds_off) {
#pragma unroll
    for (int i = 0; i < N; ++i) {
      const int item = threadIdx.x + kThreads * i, row = item / CPR, ch = item % CPR;
      voff[i] = row * rs_bytes + ch * 16;
      loff[i] = lds_off + row * BwdPitch<D>::P + ch * 16 * (FP8 ? 2 : 1);
    }
  }
  __device__ __forceinline__ void load(BufRsrc rs, uint32_t soff) {
#pragma unroll
    for (int i = 0; i < N; ++i) {
      if (ITEMS % kThreads == 0 || threadIdx.x + kThreads * i < ITEMS) r[i] = buf_ld128(rs, voff[i], soff);
    }
  }
  __device__ __forceinline__ void store(uint8_t* buf) const {
#pragma unroll
    for (int i = 0; i < N; ++i) {
      if (!(ITEMS % kThreads == 0 || threadIdx.x + kThreads * i < ITEMS)) continue;
      if constexpr (FP8) {
        const u32x4 w = r[i];
        u32x4 lo, hi;
#pragma unroll
        for (int e = 0; e < 2; ++e) {
          lo[2 * e] = cvt_fp8x2_bf16<false>(w[e]);
          lo[2 * e + 1] = cvt_fp8x2_bf16<true>(w[e]);
          hi[2 * e] = cvt_fp8x2_bf16<false>(w[e + 2]);
          hi[2 * e + 1] = cvt_fp8x2_bf16<true>(w[e + 2]);
        }
        *(u32x4*)(buf + loff[i]) = lo;
        *(u32x4*)(buf + loff[i] + 16) = hi;
      } else {
        *(u32x4*)(buf + loff[i]) = r[i];
      }
    }
  }
};

// Fragment of 16 rows x D as the B operand of a 16x16x32 bf16 MFMA whose
// contraction runs over d: lane (li, g) gets row `row`, columns 32st+8g..+7.
// e4m3 rows are converted exactly; `scale` multiplies every element (only
// used where the rounding of the scaled value to bf16 is acceptable).
template <int D, bool FP8>
__device__ __forceinline__ void load_row_frag(u32x4 (&f)[D / 32], const uint8_t* base, int64_t rs_bytes, int row,
                                              bool ok, int g, float scale) {
#pragma unroll
  for (int st = 0; st < D / 32; ++st) {
    f[st] = u32x4{0u, 0u, 0u, 0u};
    if (!ok) continue;
    if constexpr (FP8) {
      const u32x2 w = *(const u32x2*)(base + (int64_t)row * rs_bytes + 32 * st + 8 * g);
      const u32x2 a = fp8x4_to_bf16x4(w[0], scale), b = fp8x4_to_bf16x4(w[1], scale);
      f[st] = u32x4{a[0], a[1], b[0], b[1]};
    } else {
      f[st] = *(const u32x4*)(base + (int64_t)row * rs_bytes + (32 * st + 8 * g) * 2);
    }
  }
}

// ---------------------------------------------------------------------
// dQ (and the bias gradient).  Block = 128 queries (32 per wave), key tiles
// of 64.  S^T = K.Q^T, dP^T = V.dO^T (C fragments: key 4g+r, query li),
// dS = dP*sig*(1 + x(1-sig)), dQ += dS.K.
// ---------------------------------------------------------------------
template <int D>
struct DqCfg {
  static constexpr int BM = 128, BN = 64, KT = BN / 16, DT = D / 16, KS = D / 32;
  static constexpr int P = BwdPitch<D>::P;
  static constexpr int K_OFF = 0;
  static constexpr int V_OFF = K_OFF + BN * P;
  static constexpr int SC_OFF = V_OFF + BN * P;  // (sk, sv) per key
  static constexpr int BIAS_OFF = SC_OFF + BN * 8;
  static constexpr int BUF = BIAS_OFF + (BM + BN) * 4;
  static constexpr int HIST_OFF = 2 * BUF;  // bias-gradient histograms, 2R - 1 floats per wave
  static int lds(bool bias, int R) { return HIST_OFF + (bias ? 4 * (2 * R - 1) * 4 : 0); }
};

// ---------------------------------------------------------------------------
// Diagonal (relative-offset) sums of score gradients, for the bias gradient.
//
// A 16x16 MFMA result fragment holds element (row 4g+r, col li) in lane
// 16g+li, register r; its diagonal index is li - 4g - r in [-15, 15].  Four
// fragments of a 32x32 sub-tile, shifted by 16*S (S = -1, 0, +1), cover the
// 63 diagonals -31..31.  diag_accumulate folds a fragment into four
// per-lane partial sums a[k], where lane (g, p) of a[k] holds diagonal
// p - 4g + 16(1-k); diag_reduce then gives each lane of the wave the whole
// sum of one diagonal, p + 16(1-g), so that one conflict-free LDS add per
// lane replaces 16 atomics that collide four ways.
// ---------------------------------------------------------------------------

// Row-local (16-lane) DPP move; a lane whose source is outside its row reads 0.
template <int CTRL>
__device__ __forceinline__ float dpp_row(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL, 0xF, 0xF, true));
}

// folds a fragment into the bucket pair (hi, lo) = diagonals p - 4g, p - 4g - 16
__device__ __forceinline__ void diag_accumulate_to(float& hi, float& lo, const float (&v)[4]) {
  // lane p takes column p + r of register r (row_shl:r): diagonal p - 4g
  hi += v[0];
  hi += dpp_row<0x101>(v[1]);
  hi += dpp_row<0x102>(v[2]);
  hi += dpp_row<0x103>(v[3]);
  // ... and column p + r - 16 (row_shr:16-r): diagonal p - 4g - 16
  lo += dpp_row<0x11F>(v[1]);
  lo += dpp_row<0x11E>(v[2]);
  lo += dpp_row<0x11D>(v[3]);
}
// diag_accumulate_to of the products x[r] c[r], one FMA per term (the DPP
// move fused into v_fmac_f32, which the compiler does not do by itself); c[r]
// is the factor of the lane the DPP reads for x[r], lane (p + r) mod 16.  A
// DPP source written by a VALU instruction needs two wait states first: the
// s_nop 0 and the plain FMA give them to x[1..3], and the closing s_nop 1
// gives them to a DPP read of hi or lo that follows (the compiler's hazard
// check does not look into inline assembly).
__device__ __forceinline__ void diag_fma_to(float& hi, float& lo, const float (&x)[4], const float (&c)[4]) {
  asm("s_nop 0\n\t"
      "v_fmac_f32 %0, %2, %6\n\t"
      "v_fmac_f32_dpp %0, %3, %7 row_shl:1 row_mask:0xf bank_mask:0xf bound_ctrl:1\n\t"
      "v_fmac_f32_dpp %0, %4, %8 row_shl:2 row_mask:0xf bank_mask:0xf bound_ctrl:1\n\t"
      "v_fmac_f32_dpp %0, %5, %9 row_shl:3 row_mask:0xf bank_mask:0xf bound_ctrl:1\n\t"
      "v_fmac_f32_dpp %1, %3, %7 row_shr:15 row_mask:0xf bank_mask:0xf bound_ctrl:1\n\t"
      "v_fmac_f32_dpp %1, %4, %8 row_shr:14 row_mask:0xf bank_mask:0xf bound_ctrl:1\n\t"
      "v_fmac_f32_dpp %1, %5, %9 row_shr:13 row_mask:0xf bank_mask:0xf bound_ctrl:1\n\t"
      "s_nop 1"
      : "+v"(hi), "+v"(lo)
      : "v"(x[0]), "v"(x[1]), "v"(x[2]), "v"(x[3]), "v"(c[0]), "v"(c[1]), "v"(c[2]), "v"(c[3]));
}
// lane p of each 16-lane row <- lane (p + R) mod 16 (row_ror by 16 - R)
template <int R>
__device__ __forceinline__ float row_rot(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0x120 + 16 - R, 0xF, 0xF,
                                                               false));
}
template <int S>
__device__ __forceinline__ void diag_accumulate(float (&a)[4], const float (&v)[4]) {
  diag_accumulate_to(a[1 - S], a[2 - S], v);
}

template <int CTRL, int ROWS>
__device__ __forceinline__ float dpp_rows(float old, float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, old),
                                                               __builtin_bit_cast(int, x), CTRL, ROWS, 0xF, false));
}
// lane (g, p) of row g <- lane (g, (p + 4 g) mod 16): row_ror by 16 - 4 g on rows 1..3
__device__ __forceinline__ float skew_undo(float x) {
  float y = dpp_rows<0x12C, 0x2>(x, x);
  y = dpp_rows<0x128, 0x4>(y, x);
  return dpp_rows<0x124, 0x8>(y, x);
}
__device__ __forceinline__ float lane_xor32(float x) {
  const auto s = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(int, x), __builtin_bit_cast(int, x), false, false);
  return __builtin_bit_cast(float, (threadIdx.x & 32) ? s[0] : s[1]);
}
__device__ __forceinline__ float lane_xor16(float x) {
  const auto s = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(int, x), __builtin_bit_cast(int, x), false, false);
  return __builtin_bit_cast(float, (threadIdx.x & 16) ? s[0] : s[1]);
}

// Reduce-scatter over the four rows of unskewed buckets b0..b3 (lane p of
// every row holds the same diagonal of a bucket): lane 16g+p gets the sum over
// the rows of bucket g at p.  DPP and permlane swaps only: no LDS round trip.
__device__ __forceinline__ float diag_scatter(float b0, float b1, float b2, float b3, int lane) {
  const bool upper = lane >= 32, odd = ((lane >> 4) & 1) != 0;
  float ka = upper ? b2 : b0, kb = upper ? b3 : b1;
  const float sa = upper ? b0 : b2, sb = upper ? b1 : b3;
  ka += lane_xor32(sa);
  kb += lane_xor32(sb);
  return (odd ? kb : ka) + lane_xor16(odd ? ka : kb);
}

// Sum over the wave of diagonal p + 16(1-g) for lane 16g+p (g = 3, p = 0 is
// diagonal -32, always 0).
__device__ __forceinline__ float diag_reduce(const float (&a)[4], int lane) {
  const int g = lane >> 4, p = lane & 15;
  // undo the 4g skew: lane (g, p) reads lane (g, p + 4g mod 16); wrapped
  // reads land one bucket (16 diagonals) lower
  const bool wrap = p + 4 * g >= 16;
  const float g0 = skew_undo(a[0]), g1 = skew_undo(a[1]), g2 = skew_undo(a[2]), g3 = skew_undo(a[3]);
  return diag_scatter(wrap ? 0.f : g0, wrap ? g0 : g1, wrap ? g1 : g2, wrap ? g2 : g3, lane);
}

template <int D, bool FP8, bool GENERIC, bool BIAS>
__global__ void __launch_bounds__(kThreads, 2) hstu_bwd_dq_kernel(AttnParams p) {
  using C = DqCfg<D>;
  constexpr int ES = FP8 ? 1 : 2;
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];

  SeqCtx sc;
  if (!seq_ctx(p, /*heavy_last=*/true, sc)) return;
  const int L = sc.L, h = sc.h;
  const int m0 = sc.blk * C::BM;
  if (m0 >= L) return;
  const MaskCtx mc = mask_ctx(p, sc);

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, li = lane & 15, g = lane >> 4;
  const int mw0 = m0 + wave * 32;
  const bool wave_active = mw0 < L;

  const uint32_t krs = (uint32_t)(p.k_rs * ES), vrs = (uint32_t)(p.v_rs * ES);
  const BufRsrc krsrc = make_rsrc(p.k + (sc.start * p.k_rs + (int64_t)h * D) * ES,
                                  (uint32_t)(L > 0 ? (L - 1) * krs + D * ES : 0));
  const BufRsrc vrsrc = make_rsrc(p.v + (sc.start * p.v_rs + (int64_t)h * D) * ES,
                                  (uint32_t)(L > 0 ? (L - 1) * vrs + D * ES : 0));
  const uint32_t s_step = FP8 ? (uint32_t)(p.s_rs * 4) : 0u;
  const uint32_t sbytes = FP8 ? (uint32_t)(p.s_rs ? L * p.s_rs * 4 : 4) : 0u;
  const BufRsrc sk_rsrc = make_rsrc(FP8 ? p.k_scale + sc.start * p.s_rs + h * p.s_hs : nullptr, sbytes);
  const BufRsrc sv_rsrc = make_rsrc(FP8 ? p.v_scale + sc.start * p.s_rs + h * p.s_hs : nullptr, sbytes);
  const float* biasb = BIAS ? p.bias + (int64_t)h * (2 * p.bias_R - 1) : nullptr;
  const int R1 = p.bias_R - 1;
  // the wave's bias-gradient histogram: offset o at entry o + R - 1, o = -(R-1) .. R-1
  float* hist0 = (float*)(smem + C::HIST_OFF);
  float* hist = hist0 + wave * (2 * p.bias_R - 1);
  if constexpr (BIAS) {
    for (int i = tid; i < 4 * (2 * p.bias_R - 1); i += kThreads) hist0[i] = 0.f;
  }

  // Q and dO fragments (B operands): lane holds query mw0+16qt+li.
  u32x4 qf[2][C::KS], dof[2][C::KS];
  float cq[2];
  {
    const uint8_t* qb = p.q + (sc.start * p.q_rs + (int64_t)h * D) * ES;
    const uint8_t* dob = p.dout + (sc.start * p.do_rs + (int64_t)h * D) * 2;
#pragma unroll
    for (int qt = 0; qt < 2; ++qt) {
      const int row = mw0 + qt * 16 + li;
      const bool ok = row < L;
      load_row_frag<D, FP8>(qf[qt], qb, p.q_rs * ES, row, ok, g, 1.f);
      load_row_frag<D, false>(dof[qt], dob, p.do_rs * 2, row, ok, g, 1.f);
      cq[qt] = -p.alpha * kLog2e;
      if constexpr (FP8) cq[qt] *= ok ? p.q_scale[(sc.start + row) * p.s_rs + h * p.s_hs] : 0.f;
    }
  }

  f32x4 acc[2][C::DT];
#pragma unroll
  for (int qt = 0; qt < 2; ++qt)
#pragma unroll
    for (int dt = 0; dt < C::DT; ++dt) acc[qt][dt] = zero4();

  int n_end = min(m0 + C::BM, L);
  if (GENERIC && m0 < p.contextual_seq_len) n_end = L;
  const int ntiles = (n_end + C::BN - 1) / C::BN;

  RowStage<C::BN, D, FP8> k_st, v_st;
  k_st.init(krs, C::K_OFF);
  v_st.init(vrs, C::V_OFF);
  float sc_v = 0.f, bias_v = 0.f;
  auto load = [&](int n0) {
    k_st.load(krsrc, n0 * krs);
    v_st.load(vrsrc, n0 * vrs);
    if constexpr (FP8) {
      if (tid < 64) sc_v = buf_ldf(sk_rsrc, (uint32_t)tid * s_step, n0 * s_step);
      else if (tid < 128) sc_v = buf_ldf(sv_rsrc, (uint32_t)(tid - 64) * s_step, n0 * s_step);
    }
    if constexpr (BIAS) {
      if (tid < C::BM + C::BN - 1) {
        const int off = m0 - n0 - (C::BN - 1) + tid;
        bias_v = biasb[min(max(off, -R1), R1) + R1] * -kLog2e;
      }
    }
  };
  auto store = [&](uint8_t* buf) {
    k_st.store(buf);
    v_st.store(buf);
    if constexpr (FP8) {
      if (tid < 128) ((float*)(buf + C::SC_OFF))[(tid & 63) * 2 + (tid >> 6)] = sc_v;
    }
    if constexpr (BIAS) {
      if (tid < C::BM + C::BN - 1) ((float*)(buf + C::BIAS_OFF))[tid] = bias_v;
    }
  };

  const int k_rd = C::K_OFF + li * C::P + 16 * g;
  const int v_rd = C::V_OFF + li * C::P + 16 * g;
  const int kt_rd = C::K_OFF + (4 * g + (li >> 2)) * C::P + (li & 3) * 8;  // tr16
  const int bias_rd = 32 * wave + (C::BN - 1) + li - 4 * g;
  float dclamp = 0.f, dclampn = 0.f;  // bias gradient of elements in the clamped regions (+, -)

  load(0);
  store(smem);
  __syncthreads();

  for (int t = 0; t < ntiles; ++t) {
    const int n0 = t * C::BN;
    const uint8_t* buf = smem + (t & 1) * C::BUF;
    if (t + 1 < ntiles) load(n0 + C::BN);

    if (wave_active && (GENERIC || n0 <= mw0 + 31)) {
      const bool need_mask = GENERIC || (n0 + C::BN - 1 > mw0);
      const bool bias_const = BIAS && (m0 - n0 - (C::BN - 1) >= R1);
      const float* bias_lds = (const float*)(buf + C::BIAS_OFF);
      // Two halves of 32 keys each (key sub-tiles 2c, 2c+1), to keep the
      // score registers of one half live at a time.
#pragma unroll
      for (int c = 0; c < C::BN / 32; ++c) {
        if (!GENERIC && n0 + 32 * c > mw0 + 31) break;  // half entirely above the diagonal
        f32x4 s[2][2], dp[2][2];
#pragma unroll
        for (int h2 = 0; h2 < 2; ++h2) {
          const int kt = 2 * c + h2;
          s[h2][0] = s[h2][1] = dp[h2][0] = dp[h2][1] = zero4();
#pragma unroll
          for (int st = 0; st < C::KS; ++st) {
            const u32x4 a = lds_ld128(buf + k_rd + kt * 16 * C::P + st * 64);
            s[h2][0] = mfma_bf16(a, qf[0][st], s[h2][0]);
            s[h2][1] = mfma_bf16(a, qf[1][st], s[h2][1]);
            const u32x4 b = lds_ld128(buf + v_rd + kt * 16 * C::P + st * 64);
            dp[h2][0] = mfma_bf16(b, dof[0][st], dp[h2][0]);
            dp[h2][1] = mfma_bf16(b, dof[1][st], dp[h2][1]);
          }
        }
        u32x4 dsa[2];
        auto epilogue = [&](auto masked_tag, auto bconst_tag) {
          constexpr bool MASKED = decltype(masked_tag)::value;
          constexpr bool BCONST = decltype(bconst_tag)::value;
          const float bconst = (BIAS && BCONST) ? bias_lds[0] : 0.f;
          float dacc[4] = {0.f, 0.f, 0.f, 0.f};  // diagonal partial sums (bias gradient)
#pragma unroll
          for (int h2 = 0; h2 < 2; ++h2) {
            const int kt = 2 * c + h2;
            f32x4 skv = {1.f, 1.f, 1.f, 1.f}, svv = {1.f, 1.f, 1.f, 1.f};
            if constexpr (FP8) {
              const float* scp = (const float*)(buf + C::SC_OFF) + (kt * 16 + 4 * g) * 2;
              const f32x4 a = *(const f32x4*)scp, b = *(const f32x4*)(scp + 4);
              skv = f32x4{a[0], a[2], b[0], b[2]};
              svv = f32x4{a[1], a[3], b[1], b[3]};
            }
#pragma unroll
            for (int qt = 0; qt < 2; ++qt) {
              float dsv[4], dsr[4];
#pragma unroll
              for (int r = 0; r < 4; ++r) {
                float b = 0.f;
                if constexpr (BIAS) b = BCONST ? bconst : bias_lds[bias_rd + 16 * (qt - kt) - r];
                const float t = scaled_score<FP8, BIAS>(s[h2][qt][r], cq[qt], skv[r], b);
                float ds = dsilu_dp(t, FP8 ? dp[h2][qt][r] * svv[r] : dp[h2][qt][r]);
                if constexpr (MASKED) {
                  const int i = mw0 + qt * 16 + li, j = n0 + kt * 16 + 4 * g + r;
                  const bool ok = GENERIC ? valid_generic(i, j, mc) : (j <= i);
                  ds = ok ? ds : 0.f;
                }
                if constexpr (BIAS) {
                  if constexpr (BCONST) dclamp += ds;
                  else dsr[r] = ds;
                }
                if constexpr (FP8) ds *= skv[r];
                dsv[r] = ds;
              }
              if constexpr (BIAS && !BCONST) {
                if (qt == h2) diag_accumulate<0>(dacc, dsr);
                else if (qt > h2) diag_accumulate<1>(dacc, dsr);
                else diag_accumulate<-1>(dacc, dsr);
              }
              dsa[qt][h2 * 2 + 0] = pack_bf16(dsv[0], dsv[1]);
              dsa[qt][h2 * 2 + 1] = pack_bf16(dsv[2], dsv[3]);
            }
          }
          if constexpr (BIAS && !BCONST) {
            // this lane's diagonal of the 32x32 sub-tile, as a relative offset i - j
            const float dv = diag_reduce(dacc, lane);
            const int off = (mw0 - n0 - 32 * c) + li + 16 - 16 * g;
            if (off >= R1) dclamp += dv;
            else if (off > -R1) atomicAdd(&hist[off + R1], dv);
            else dclampn += dv;
          }
        };
        if (need_mask) {
          if (bias_const) epilogue(std::true_type{}, std::true_type{});
          else epilogue(std::true_type{}, std::false_type{});
        } else {
          if (bias_const) epilogue(std::false_type{}, std::true_type{});
          else epilogue(std::false_type{}, std::false_type{});
        }
        // ---- dQ += dS . K  (K rows read transposed)
#pragma unroll
        for (int dt = 0; dt < C::DT; ++dt) {
          const uint8_t* kp = buf + kt_rd + c * 32 * C::P + dt * 32;
          const u32x4 bk = cat_tr(lds_tr16(kp), lds_tr16(kp + 16 * C::P));
          acc[0][dt] = mfma_bf16(dsa[0], bk, acc[0][dt]);
          acc[1][dt] = mfma_bf16(dsa[1], bk, acc[1][dt]);
        }
      }
    }

    if (t + 1 < ntiles) store(smem + ((t + 1) & 1) * C::BUF);
    __syncthreads();
  }

  if constexpr (BIAS) {
    hist_add_clamped(hist, 2 * R1, dclamp, lane);
    hist_add_clamped(hist, 0, dclampn, lane);
    dbias_store_row<4>(p, hist0, sc.b, sc.blk, h);
  }

  if (!wave_active) return;
  const float fin = p.alpha * p.inv_n;
#pragma unroll
  for (int qt = 0; qt < 2; ++qt) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int row = mw0 + qt * 16 + 4 * g + r;
      if (row < L) {
        uint16_t* dst = p.dq + (sc.start + row) * p.dq_rs + (int64_t)h * D + li;
#pragma unroll
        for (int dt = 0; dt < C::DT; ++dt) dst[dt * 16] = to_bf16(acc[qt][dt][r] * fin);
      }
    }
  }
}

// ---------------------------------------------------------------------
// dQ from the stored dS tiles (causal masks).  Block = 128 queries (one
// 32-query tile per wave), key steps of 64.  No recompute: the block stages
// K (bf16; e4m3 rows times their key scale, rounded to bf16), each wave
// stages its own dS tile rows, and both are read transposed so that
// dQ^T = K^T . dS^T comes out of 16x16x32 bf16 MFMAs with a lane holding
// four consecutive d of one query (8-byte stores).  The bias gradient is
// taken from the dS values the wave holds in registers (C-fragment layout:
// query 4g+r, key li), as the recomputing dQ kernel does.
// ---------------------------------------------------------------------
template <int D>
struct DqWsCfg {
  static constexpr int BM = 128, BNK = 64, DT = D / 16;
  static constexpr int P = BwdPitch<D>::P;  // K rows [key][d], bf16
  static constexpr int PS = 96;             // dS rows [key][32 queries], bf16 (64 B + pad, conflict-free tr reads)
  static constexpr int K_OFF = 0;
  static constexpr int DS_OFF = K_OFF + BNK * P;
  static constexpr int DS_WAVE = BNK * PS;
  static constexpr int HIST_OFF = DS_OFF + 4 * DS_WAVE;  // bias-gradient histograms, R floats per wave
  static int lds(bool bias, int R) { return HIST_OFF + (bias ? 4 * R * 4 : 0); }
};

template <int D, bool FP8, bool BIAS>
__global__ void __launch_bounds__(kThreads, 2) hstu_bwd_dq_ws_kernel(AttnParams p) {
  using C = DqWsCfg<D>;
  constexpr int ES = FP8 ? 1 : 2;
  constexpr int KCH = D * ES / 16;                 // 16-byte K chunks per row
  constexpr int KIT = C::BNK * KCH / kThreads;     // K chunks per thread per step
  static_assert(C::BNK * KCH % kThreads == 0, "K staging");
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];

  SeqCtx sc;
  if (!seq_ctx(p, /*heavy_last=*/true, sc)) return;
  const int L = sc.L, h = sc.h;
  const int m0 = sc.blk * C::BM;
  if (m0 >= L) return;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, li = lane & 15, g = lane >> 4;
  const int qw0 = m0 + wave * 32;  // the wave's query tile
  const bool wave_active = qw0 < L;
  const int qt = qw0 / 32;
  const int n_end = min(m0 + C::BM, L);
  const int nsteps = (n_end + C::BNK - 1) / C::BNK;

  const uint32_t krs = (uint32_t)(p.k_rs * ES);
  const BufRsrc krsrc = make_rsrc(p.k + (sc.start * p.k_rs + (int64_t)h * D) * ES,
                                  (uint32_t)(L > 0 ? (L - 1) * krs + D * ES : 0));
  const int R1 = p.bias_R - 1;
  // the wave's bias-gradient histogram, offsets 0 .. R - 1
  float* hist0 = (float*)(smem + C::HIST_OFF);
  float* hist = hist0 + wave * p.bias_R;
  if constexpr (BIAS) {
    for (int i = tid; i < 4 * p.bias_R; i += kThreads) hist0[i] = 0.f;
  }
  // 1 / q_scale of the lane's queries: for the dQ store (query qs*16 + li) and
  // for the bias gradient (queries qs*16 + 4g + r of the dS fragments)
  float inv_st[2] = {1.f, 1.f}, inv_db[2][4];
#pragma unroll
  for (int qs = 0; qs < 2; ++qs)
#pragma unroll
    for (int r = 0; r < 4; ++r) inv_db[qs][r] = 1.f;
  if constexpr (FP8) {
    auto qsc = [&](int row) {
      return row < L ? 1.f / p.q_scale[(sc.start + row) * p.s_rs + h * p.s_hs] : 1.f;
    };
#pragma unroll
    for (int qs = 0; qs < 2; ++qs) {
      inv_st[qs] = qsc(qw0 + 16 * qs + li);
#pragma unroll
      for (int r = 0; r < 4; ++r) inv_db[qs][r] = qsc(qw0 + 16 * qs + 4 * g + r);
    }
  }

  f32x4 acc[C::DT][2];
#pragma unroll
  for (int dt = 0; dt < C::DT; ++dt) acc[dt][0] = acc[dt][1] = zero4();

  // staged registers of one step: K chunks (+ key scales) and this wave's 4 dS packs
  u32x4 kraw[KIT];
  float ksc[KIT];
  u32x4 dsp[4] = {u32x4{0u, 0u, 0u, 0u}, u32x4{0u, 0u, 0u, 0u}, u32x4{0u, 0u, 0u, 0u}, u32x4{0u, 0u, 0u, 0u}};
  auto load = [&](int step) {
    const int k0 = step * C::BNK;
#pragma unroll
    for (int i = 0; i < KIT; ++i) {
      const int item = tid + kThreads * i, row = item / KCH, ch = item % KCH;
      kraw[i] = buf_ld128(krsrc, (uint32_t)(row * krs + ch * 16), (uint32_t)(k0 * krs));
      if constexpr (FP8) ksc[i] = k0 + row < L ? p.k_scale[(sc.start + k0 + row) * p.s_rs + h * p.s_hs] : 0.f;
    }
    if (wave_active) {
      const int kb = step >> 1, c = step & 1;
      const uint8_t* t = ds_tile(p, sc, kb, qt) + ((2 * c) * 2 * 64 + lane) * 16;
#pragma unroll
      for (int j = 0; j < 4; ++j) dsp[j] = *(const u32x4*)(t + j * 64 * 16);  // (w' = 2c + j/2, kt = j%2)
    }
  };
  auto store = [&]() {
#pragma unroll
    for (int i = 0; i < KIT; ++i) {
      const int item = tid + kThreads * i, row = item / KCH, ch = item % KCH;
      uint8_t* dst = smem + C::K_OFF + row * C::P + ch * 16 * (FP8 ? 2 : 1);
      if constexpr (FP8) {
        const u32x4 w = kraw[i];
        const u32x2 a = fp8x4_to_bf16x4(w[0], ksc[i]), b = fp8x4_to_bf16x4(w[1], ksc[i]);
        const u32x2 c = fp8x4_to_bf16x4(w[2], ksc[i]), d = fp8x4_to_bf16x4(w[3], ksc[i]);
        *(u32x4*)dst = u32x4{a[0], a[1], b[0], b[1]};
        *(u32x4*)(dst + 16) = u32x4{c[0], c[1], d[0], d[1]};
      } else {
        *(u32x4*)dst = kraw[i];
      }
    }
    // the wave's dS rows: key 32 (j/2) + 16 (j%2) + li, queries 4g..4g+3 and 16+4g..16+4g+3
    uint8_t* db = smem + C::DS_OFF + wave * C::DS_WAVE;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      uint8_t* row = db + (32 * (j >> 1) + 16 * (j & 1) + li) * C::PS;
      *(u32x2*)(row + 8 * g) = u32x2{dsp[j][0], dsp[j][1]};
      *(u32x2*)(row + 32 + 8 * g) = u32x2{dsp[j][2], dsp[j][3]};
    }
  };

  // transposed reads (ds_read_b64_tr_b16): lane (li, g) starts at row 4g + li/4, byte (li%4)*8
  const int trk = (4 * g + (li >> 2)) * C::P + (li & 3) * 8;   // K tile
  const int trs = (4 * g + (li >> 2)) * C::PS + (li & 3) * 8;  // dS rows
  float dclamp = 0.f;
  // the bias gradient's carried buckets (see the step body) and the
  // reduce-scatter of four unskewed buckets w .. w + 3: lane (g, li) sums
  // offset xw - li + 16 g, xw = base0 + 16 w
  float cr_m3 = 0.f, cr_m2 = 0.f, cr_g = 0.f;
  int base_last = INT_MIN;
  const bool bwrap = li + 4 * g >= 16;
  auto bias_flush = [&](float t0, float t1, float t2, float t3, int xw) {
    const float dv = diag_scatter(t0, t1, t2, t3, lane);
    const int off = xw + 16 * g - li;
    if (off >= R1) dclamp += dv;
    else if (off >= 0) atomicAdd(&hist[off], dv);
  };

  load(0);
  store();
  __syncthreads();
  for (int step = 0; step < nsteps; ++step) {
    const int k0 = step * C::BNK;
    u32x4 cur[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) cur[j] = dsp[j];
    if (step + 1 < nsteps) load(step + 1);
    if (wave_active && k0 <= qw0 + 31) {
      if constexpr (BIAS) {
        // bias gradient from the held dS, as per-lane diagonal sums in
        // buckets of 16 offsets: bucket v (bk[v + 3], v = -3..2) holds in lane
        // (g, li) the offset i - j = base0 + 16 v - (li - 4 g), base0 = qw0 -
        // k0; the 32 x 32 sub-tile of keys k0 + 32 wl .. folds into buckets
        // -2 wl - 1 .. -2 wl + 2.  Unskewed, bucket w holds base0 + 16 w - li.
        // The next step's buckets 1, 2 are this step's -3, -2, so a step
        // completes the offsets base0 - 15 .. base0 + 48 (unskewed buckets
        // 0..3, bucket 3 the previous step's -1) and carries -3, -2 and
        // unskewed -1.
        const int base0 = qw0 - k0;
        auto piece = [&](int wl, int qs, int kt, float (&v)[4]) {
          const u32x4 w = cur[2 * wl + kt];
          v[0] = __builtin_bit_cast(float, w[2 * qs] << 16) * inv_db[qs][0];
          v[1] = __builtin_bit_cast(float, w[2 * qs] & 0xffff0000u) * inv_db[qs][1];
          v[2] = __builtin_bit_cast(float, w[2 * qs + 1] << 16) * inv_db[qs][2];
          v[3] = __builtin_bit_cast(float, w[2 * qs + 1] & 0xffff0000u) * inv_db[qs][3];
        };
        if (base0 - 63 >= R1) {  // every offset clamps
#pragma unroll
          for (int wl = 0; wl < 2; ++wl)
#pragma unroll
            for (int qs = 0; qs < 2; ++qs)
#pragma unroll
              for (int kt = 0; kt < 2; ++kt) {
                float v[4];
                piece(wl, qs, kt, v);
                dclamp += (v[0] + v[1]) + (v[2] + v[3]);
              }
          cr_m3 = cr_m2 = cr_g = 0.f;
        } else {
          float bk[6] = {0.f, 0.f, 0.f, 0.f, cr_m3, cr_m2};
#pragma unroll
          for (int wl = 0; wl < 2; ++wl) {
            // rows = queries (16 qs + 4g + r), cols = keys (16 kt + li): shift kt - qs
            float v00[4], v11[4], v01[4], v10[4];
            piece(wl, 0, 0, v00);
            piece(wl, 1, 1, v11);
            piece(wl, 0, 1, v01);
            piece(wl, 1, 0, v10);
            const int o = 3 - 2 * wl;  // bucket index of v = -2 wl
            diag_accumulate_to(bk[o], bk[o + 1], v00);
            diag_accumulate_to(bk[o], bk[o + 1], v11);
            diag_accumulate_to(bk[o - 1], bk[o], v01);
            diag_accumulate_to(bk[o + 1], bk[o + 2], v10);
          }
          float gu[5];  // unskewed bucket w = -1..3 (gu[w + 1])
#pragma unroll
          for (int w = 0; w < 4; ++w) gu[w] = skew_undo(bk[w + 2]);
          gu[4] = cr_g;
          float t[4];  // bucket w = 0..3 (wrapped lanes read bucket w - 1)
#pragma unroll
          for (int w = 0; w < 4; ++w) t[w] = bwrap ? gu[w] : gu[w + 1];
          bias_flush(t[0], t[1], t[2], t[3], base0);
          cr_m3 = bk[0];
          cr_m2 = bk[1];
          cr_g = gu[0];
        }
        base_last = base0;
      }
      const uint8_t* kb = smem + C::K_OFF;
      const uint8_t* dsb = smem + C::DS_OFF + wave * C::DS_WAVE;
#pragma unroll
      for (int c2 = 0; c2 < 2; ++c2) {
        if (k0 + 32 * c2 > qw0 + 31) break;  // keys entirely after the wave's queries
        u32x4 bq[2];
#pragma unroll
        for (int qs = 0; qs < 2; ++qs) {
          const uint8_t* q = dsb + trs + c2 * 32 * C::PS + qs * 32;
          bq[qs] = cat_tr(lds_tr16(q), lds_tr16(q + 16 * C::PS));
        }
#pragma unroll
        for (int dt = 0; dt < C::DT; ++dt) {
          const uint8_t* kp = kb + trk + c2 * 32 * C::P + dt * 32;
          const u32x4 ak = cat_tr(lds_tr16(kp), lds_tr16(kp + 16 * C::P));
          acc[dt][0] = mfma_bf16(ak, bq[0], acc[dt][0]);
          acc[dt][1] = mfma_bf16(ak, bq[1], acc[dt][1]);
        }
      }
    }
    __syncthreads();
    if (step + 1 < nsteps) {
      store();
      __syncthreads();
    }
  }

  if constexpr (BIAS) {
    // the carried buckets: unskewed 1, 2, 3 of a step past the wave's last
    // (its buckets -3..0 are empty), offsets down to that step's base0 - 63
    if (wave_active && base_last != INT_MIN && base_last - 64 + 48 >= 0) {
      const float g1 = skew_undo(cr_m3), g2 = skew_undo(cr_m2);
      bias_flush(0.f, bwrap ? 0.f : g1, bwrap ? g1 : g2, bwrap ? g2 : cr_g, base_last - 64);
    }
    hist_add_clamped(hist, R1, dclamp, lane);
    dbias_store_row<4>(p, hist0, sc.b, sc.blk, h);
  }

  if (!wave_active) return;
  const float fin = p.alpha * p.inv_n;
#pragma unroll
  for (int qs = 0; qs < 2; ++qs) {
    const int row = qw0 + 16 * qs + li;
    if (row >= L) continue;
    const float f = fin * inv_st[qs];
    uint16_t* dst = p.dq + (sc.start + row) * p.dq_rs + (int64_t)h * D + 4 * g;
#pragma unroll
    for (int dt = 0; dt < C::DT; ++dt)
      *(u32x2*)(dst + dt * 16) = u32x2{pack_bf16(acc[dt][qs][0] * f, acc[dt][qs][1] * f),
                                       pack_bf16(acc[dt][qs][2] * f, acc[dt][qs][3] * f)};
  }
}

// ---------------------------------------------------------------------
// dK / dV.  Block = 128 keys (32 per wave), query tiles of 32.
//   S = Q.K^T, dP = dO.V^T (C fragments: query 4g+r, key li)
//   dV += P^T.dO, dK += dS^T.Q
// A query tile is too little work to hide a global load behind, so tiles
// stream through a 3-stage LDS ring fed only by direct global->LDS loads
// (bf16 Q -- for e4m3 inputs an exact bf16 copy made by a prepass --, dO,
// the per-query scales and the bias band), with the same number of load
// instructions per wave per tile so that one vmcnt bound covers a tile.
// ---------------------------------------------------------------------
template <int D, bool FP8, bool BIAS>
struct DkvCfg {
  static constexpr int BN = 128, BMQ = 32, QS = BMQ / 16, DT = D / 16, KS = D / 32;
  static constexpr int NSTAGE = 3;
  static constexpr int P = BwdPitch<D>::P;
  using DTile = DirectTile<BMQ, D * 2, P>;
  static constexpr int TILE = DTile::BYTES;
  // e4m3 inputs: the raw q rows as well, A operand of the e4m3 S MFMA
  static constexpr int P8 = D + 32;
  using Q8Tile = DirectTile<BMQ, D, P8>;
  static constexpr int Q_OFF = 0;
  static constexpr int Q8_OFF = Q_OFF + TILE;
  static constexpr int DO_OFF = Q8_OFF + (FP8 ? Q8Tile::BYTES : 0);
  static constexpr int SQ_OFF = DO_OFF + TILE;   // 64 floats (one 4-byte load instruction)
  static constexpr int BIAS_OFF = SQ_OFF + 256;  // 192 floats (three)
  static constexpr int DUMMY_OFF = BIAS_OFF + 768;
  static constexpr int STAGE = DUMMY_OFF + 1024;
  static constexpr int N_Q = DTile::NINSTR, N_Q8 = FP8 ? Q8Tile::NINSTR : 0, N_DO = DTile::NINSTR;
  static constexpr int N_SQ = FP8 ? 1 : 0, N_BIAS = BIAS ? 3 : 0;
  static constexpr int N_REAL = N_Q + N_Q8 + N_DO + N_SQ + N_BIAS;
  static constexpr int CNT = (N_REAL + 3) / 4;  // load instructions per wave per tile
  static constexpr int LDS = NSTAGE * STAGE;
};


template <int D, bool FP8, bool GENERIC, bool BIAS>
__global__ void __launch_bounds__(kThreads, 2) hstu_bwd_dkdv_kernel(AttnParams p) {
  using C = DkvCfg<D, FP8, BIAS>;
  constexpr int ES = FP8 ? 1 : 2;
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];

  SeqCtx sc;
  if (!seq_ctx(p, /*heavy_last=*/false, sc)) return;
  const int L = sc.L, h = sc.h;
  const int n0 = sc.blk * C::BN;
  if (n0 >= L) return;
  const MaskCtx mc = mask_ctx(p, sc);

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, li = lane & 15, g = lane >> 4;
  const int kw0 = n0 + wave * 32;
  const bool wave_active = kw0 < L;

  // bf16 Q rows: the input itself, or the prepass's copy of the e4m3 input.
  const uint8_t* q16 = FP8 ? p.q16 + (sc.start * p.H + h) * (int64_t)D * 2
                           : p.q + (sc.start * p.q_rs + (int64_t)h * D) * 2;
  const uint32_t qrs = FP8 ? (uint32_t)(p.H * D * 2) : (uint32_t)(p.q_rs * 2);
  const uint32_t dors = (uint32_t)(p.do_rs * 2);
  const BufRsrc qrsrc = make_rsrc(q16, (uint32_t)(L > 0 ? (L - 1) * qrs + D * 2 : 0));
  const BufRsrc dorsrc = make_rsrc(p.dout + (sc.start * p.do_rs + (int64_t)h * D) * 2,
                                   (uint32_t)(L > 0 ? (L - 1) * dors + D * 2 : 0));
  const uint32_t q8rs = (uint32_t)p.q_rs;  // e4m3 q rows, bytes
  const BufRsrc q8rsrc = make_rsrc(FP8 ? p.q + sc.start * p.q_rs + (int64_t)h * D : nullptr,
                                   FP8 ? (uint32_t)(L > 0 ? (L - 1) * q8rs + D : 0) : 0u);
  const uint32_t s_step = FP8 ? (uint32_t)(p.s_rs * 4) : 0u;
  const BufRsrc sq_rsrc = make_rsrc(FP8 ? p.q_scale + sc.start * p.s_rs + h * p.s_hs : nullptr,
                                    FP8 ? (uint32_t)(p.s_rs ? L * p.s_rs * 4 : 4) : 0u);
  // pre-clamped, pre-scaled bias table: entry off + N + 127 holds the bias of offset off
  const int ext_len = bias_ext_len(p.N);
  const BufRsrc b_rsrc = make_rsrc(BIAS ? p.bias_ext + (int64_t)h * ext_len : nullptr,
                                   BIAS ? (uint32_t)(ext_len * 4) : 0u);

  // K and V fragments (B operands): lane holds key kw0+16kt+li.  V is
  // dequantized (scale applied) once here; K's scale goes into ck.
  // e4m3 K stays raw (B operand of the e4m3 MFMA: lane group g holds the
  // 16-byte k-chunks g and g+4 of its key row, as the Q8 tile reads below).
  u32x4 kf[2][C::KS], vf[2][C::KS];
  i32x8 kf8[2];
  float ck[2];
  {
    const uint8_t* kb = p.k + (sc.start * p.k_rs + (int64_t)h * D) * ES;
    const uint8_t* vb = p.v + (sc.start * p.v_rs + (int64_t)h * D) * ES;
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) {
      const int row = kw0 + kt * 16 + li;
      const bool ok = row < L;
      float sv = 1.f;
      ck[kt] = -p.alpha * kLog2e;
      if constexpr (FP8) {
        sv = ok ? p.v_scale[(sc.start + row) * p.s_rs + h * p.s_hs] : 0.f;
        ck[kt] *= ok ? p.k_scale[(sc.start + row) * p.s_rs + h * p.s_hs] : 0.f;
        u32x4 lo = {0u, 0u, 0u, 0u}, hi = {0u, 0u, 0u, 0u};
        if (ok) {
          lo = *(const u32x4*)(kb + (int64_t)row * p.k_rs + 16 * g);
          hi = *(const u32x4*)(kb + (int64_t)row * p.k_rs + 64 + 16 * g);
        }
        kf8[kt] = cat8(lo, hi);
      } else {
        load_row_frag<D, false>(kf[kt], kb, p.k_rs * 2, row, ok, g, 1.f);
      }
      load_row_frag<D, FP8>(vf[kt], vb, p.v_rs * ES, row, ok, g, sv);
    }
  }

  f32x4 dk[2][C::DT], dv[2][C::DT];
#pragma unroll
  for (int kt = 0; kt < 2; ++kt)
#pragma unroll
    for (int dt = 0; dt < C::DT; ++dt) dk[kt][dt] = dv[kt][dt] = zero4();

  const int m_begin = GENERIC ? 0 : n0;
  const int ntiles = (L - m_begin + C::BMQ - 1) / C::BMQ;

  // Per-lane global offset of load instruction i of a tile of padded rows
  // (cpr 16-byte slots per LDS row, dcpr of them data); recomputed at each
  // issue rather than held in registers.
  auto tile_voff = [&](int i, int cpr, int dcpr, uint32_t rs) -> uint32_t {
    const int c = i * 64 + lane;
    int row = c / cpr, col = c % cpr;
    if (col >= dcpr) col -= dcpr;
    row = row < C::BMQ ? row : C::BMQ - 1;
    return row * rs + col * 16;
  };
  // One load instruction; the slot (which tile piece it moves) is a
  // compile-time constant, so each wave's issue sequence is straight-line.
  // Slots: [bf16 Q][e4m3 Q][dO][q scales][bias band][dummies].
  constexpr int S_Q8 = C::N_Q, S_DO = S_Q8 + C::N_Q8, S_SQ = S_DO + C::N_DO, S_BIAS = S_SQ + C::N_SQ;
  // The per-lane voffset of each of this wave's load slots (slot wave + 4j)
  // depends only on (slot, lane): computed once, the tile base goes into the
  // scalar offset at each issue.
  uint32_t voffc[C::CNT];
#pragma unroll
  for (int jj = 0; jj < C::CNT; ++jj) {
    const int slot = wave + 4 * jj;
    uint32_t v;
    if (slot < S_Q8) v = tile_voff(slot, C::P / 16, D * 2 / 16, qrs);
    else if (slot < S_DO) v = tile_voff(slot - S_Q8, C::P8 / 16, D / 16, q8rs);
    else if (slot < S_SQ) v = tile_voff(slot - S_DO, C::P / 16, D * 2 / 16, dors);
    else if (FP8 && slot == S_SQ) v = (uint32_t)min(lane, C::BMQ - 1) * s_step;
    else if (BIAS && slot < C::N_REAL) v = ((slot - S_BIAS) * 64 + lane) * 4;
    else v = lane * 16;
    voffc[jj] = v;
  }
  auto issue_slot = [&](auto slot_c, auto j_c, int m0, uint8_t* stage) {
#if defined(__HIP_DEVICE_COMPILE__)
    typedef __attribute__((address_space(3))) void lds_t;
    constexpr int slot = decltype(slot_c)::value;
    const uint32_t vo = voffc[decltype(j_c)::value];
    if constexpr (slot < S_Q8) {
      __builtin_amdgcn_raw_ptr_buffer_load_lds(qrsrc, (lds_t*)(stage + C::Q_OFF + slot * 1024), 16, vo, m0 * qrs, 0,
                                               0);
    } else if constexpr (slot < S_DO) {
      __builtin_amdgcn_raw_ptr_buffer_load_lds(q8rsrc, (lds_t*)(stage + C::Q8_OFF + (slot - S_Q8) * 1024), 16, vo,
                                               m0 * q8rs, 0, 0);
    } else if constexpr (slot < S_SQ) {
      __builtin_amdgcn_raw_ptr_buffer_load_lds(dorsrc, (lds_t*)(stage + C::DO_OFF + (slot - S_DO) * 1024), 16, vo,
                                               m0 * dors, 0, 0);
    } else if constexpr (FP8 && slot == S_SQ) {
      __builtin_amdgcn_raw_ptr_buffer_load_lds(sq_rsrc, (lds_t*)(stage + C::SQ_OFF), 4, vo, m0 * s_step, 0, 0);
    } else if constexpr (BIAS && slot < C::N_REAL) {
      constexpr int b = slot - S_BIAS;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(b_rsrc, (lds_t*)(stage + C::BIAS_OFF + b * 256), 4, vo,
                                               (uint32_t)(m0 - n0 + p.N) * 4u, 0, 0);
    } else {
      __builtin_amdgcn_raw_ptr_buffer_load_lds(qrsrc, (lds_t*)(stage + C::DUMMY_OFF), 16, vo, 0, 0, 0);
    }
#else
    (void)m0;
    (void)stage;
#endif
  };
  auto issue = [&](int m0, uint8_t* stage) {
    auto run = [&](auto wave_c) {
      constexpr int W = decltype(wave_c)::value;
      static_for<C::CNT>([&](auto j) {
        issue_slot(std::integral_constant<int, W + 4 * decltype(j)::value>{}, j, m0, stage);
      });
    };
    const int w = __builtin_amdgcn_readfirstlane(wave);
    if (w == 0) run(std::integral_constant<int, 0>{});
    else if (w == 1) run(std::integral_constant<int, 1>{});
    else if (w == 2) run(std::integral_constant<int, 2>{});
    else run(std::integral_constant<int, 3>{});
  };

  const int q_rd = C::Q_OFF + li * C::P + 16 * g;
  const int q8_rd = C::Q8_OFF + li * C::P8 + 16 * g;
  const int do_rd = C::DO_OFF + li * C::P + 16 * g;
  const int tr_rd = (4 * g + (li >> 2)) * C::P + (li & 3) * 8;  // tr16, relative to a tile
  // bias index of element (qs, kt, r) = bias_rd + 16*(qs-kt) + r
  const int bias_rd = (C::BN - 1) - 32 * wave + 4 * g - li;
  const int R1 = p.bias_R - 1;

#pragma unroll
  for (int st = 0; st < C::NSTAGE - 1; ++st) issue(m_begin + st * C::BMQ, smem + st * C::STAGE);
  wait_vm_le<(C::NSTAGE - 2) * C::CNT>();
  __syncthreads();

  int cur = 0;  // stage holding the current tile

  // One query tile; MASKED / BCONST select the epilogue at compile time so
  // each loop below has a single code path (two paths in one loop push the
  // register allocation past the 256 VGPRs of two waves per SIMD).
  auto tile_body = [&](int t, auto masked_tag, auto bconst_tag) {
    constexpr bool MASKED = decltype(masked_tag)::value;
    constexpr bool BCONST = decltype(bconst_tag)::value;
    const int m0 = m_begin + t * C::BMQ;
    const uint8_t* buf = smem + cur * C::STAGE;
    {
      int nxt = cur + C::NSTAGE - 1;
      nxt = nxt >= C::NSTAGE ? nxt - C::NSTAGE : nxt;
      issue(m0 + (C::NSTAGE - 1) * C::BMQ, smem + nxt * C::STAGE);
    }

    u32x4 ds_out[2] = {u32x4{0u, 0u, 0u, 0u}, u32x4{0u, 0u, 0u, 0u}};  // this tile's dS for the dQ kernel
    if (wave_active && (GENERIC || m0 + C::BMQ - 1 >= kw0)) {
      f32x4 s[C::QS][2], dp[C::QS][2];
#pragma unroll
      for (int qs = 0; qs < C::QS; ++qs) {
        s[qs][0] = s[qs][1] = dp[qs][0] = dp[qs][1] = zero4();
        if constexpr (FP8) {
          // e4m3 q.k products are exact in the fp32 accumulator, as in the bf16 form
          const uint8_t* a8 = buf + q8_rd + qs * 16 * C::P8;
          const i32x8 a = cat8(lds_ld128(a8), lds_ld128(a8 + 64));
          s[qs][0] = mfma_fp8(a, kf8[0], s[qs][0]);
          s[qs][1] = mfma_fp8(a, kf8[1], s[qs][1]);
        }
#pragma unroll
        for (int st = 0; st < C::KS; ++st) {
          if constexpr (!FP8) {
            const u32x4 a = lds_ld128(buf + q_rd + qs * 16 * C::P + st * 64);
            s[qs][0] = mfma_bf16(a, kf[0][st], s[qs][0]);
            s[qs][1] = mfma_bf16(a, kf[1][st], s[qs][1]);
          }
          const u32x4 b = lds_ld128(buf + do_rd + qs * 16 * C::P + st * 64);
          dp[qs][0] = mfma_bf16(b, vf[0][st], dp[qs][0]);
          dp[qs][1] = mfma_bf16(b, vf[1][st], dp[qs][1]);
        }
      }
      const float* bias_lds = (const float*)(buf + C::BIAS_OFF);
      const float bconst = (BIAS && BCONST) ? bias_lds[0] : 0.f;
      u32x4 pa[2], dsa[2];
#pragma unroll
      for (int qs = 0; qs < C::QS; ++qs) {
        f32x4 sqv = {1.f, 1.f, 1.f, 1.f};
        if constexpr (FP8) sqv = lds_ldf4(buf + C::SQ_OFF + (qs * 16 + 4 * g) * 4);
#pragma unroll
        for (int kt = 0; kt < 2; ++kt) {
          float pv[4], dsv[4];
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            float b = 0.f;
            if constexpr (BIAS) b = BCONST ? bconst : bias_lds[bias_rd + 16 * (qs - kt) + r];
            const float t = scaled_score<FP8, BIAS>(s[qs][kt][r], ck[kt], sqv[r], b);
            const float sg = sig_of_t(t);
            float pval = t * sg;
            float dval = dp[qs][kt][r] * dsilu_factor(sg, pval);
            if constexpr (FP8) dval *= sqv[r];
            if constexpr (MASKED) {
              const int i = m0 + qs * 16 + 4 * g + r, j = kw0 + kt * 16 + li;
              const bool ok = GENERIC ? valid_generic(i, j, mc) : (j <= i);
              pval = ok ? pval : 0.f;
              dval = ok ? dval : 0.f;
            }
            pv[r] = pval;
            dsv[r] = dval;
          }
          pa[kt][qs * 2 + 0] = pack_bf16(pv[0], pv[1]);
          pa[kt][qs * 2 + 1] = pack_bf16(pv[2], pv[3]);
          dsa[kt][qs * 2 + 0] = pack_bf16(dsv[0], dsv[1]);
          dsa[kt][qs * 2 + 1] = pack_bf16(dsv[2], dsv[3]);
        }
      }
      if constexpr (!GENERIC) {
        ds_out[0] = dsa[0];
        ds_out[1] = dsa[1];
      }
      // ---- dV += P^T . dO, dK += dS^T . Q  (dO and Q rows read transposed,
      // one d-step ahead of their MFMAs)
      auto tr_pair = [&](int off) {
        return cat_tr(lds_tr16(buf + off + tr_rd), lds_tr16(buf + off + tr_rd + 16 * C::P));
      };
      u32x4 nbdo = tr_pair(C::DO_OFF), nbq = tr_pair(C::Q_OFF);
#pragma unroll
      for (int dt = 0; dt < C::DT; ++dt) {
        const u32x4 bdo = nbdo, bq = nbq;
        if (dt + 1 < C::DT) {
          nbdo = tr_pair(C::DO_OFF + (dt + 1) * 32);
          nbq = tr_pair(C::Q_OFF + (dt + 1) * 32);
        }
        dv[0][dt] = mfma_bf16(pa[0], bdo, dv[0][dt]);
        dv[1][dt] = mfma_bf16(pa[1], bdo, dv[1][dt]);
        dk[0][dt] = mfma_bf16(dsa[0], bq, dk[0][dt]);
        dk[1][dt] = mfma_bf16(dsa[1], bq, dk[1][dt]);
      }
    }

    wait_vm_le<(C::NSTAGE - 2) * C::CNT>();
    __syncthreads();
    cur = cur + 1 == C::NSTAGE ? 0 : cur + 1;
    if constexpr (!GENERIC) {
      // after the wait, so these stores are the newest vector-memory
      // operations and the next tile's vmcnt bound covers its loads first
      // (a later placement measured slower); streaming stores, since the dQ
      // kernel reads the tiles long after
      uint8_t* dst = ds_tile(p, sc, sc.blk, m0 / C::BMQ) + ((wave * 2) * 64 + lane) * 16;
      __builtin_nontemporal_store(ds_out[0], (u32x4*)dst);
      __builtin_nontemporal_store(ds_out[1], (u32x4*)(dst + 64 * 16));
    }
  };

  // Tiles [0, t_mask) touch the diagonal of some wave's keys (queries below
  // n0 + BN - 1); tiles from t_const on have every offset i-j >= R-1 and so a
  // constant bias.
  const int t_mask = GENERIC ? ntiles : min(ntiles, (C::BN - 1 + C::BMQ - 1) / C::BMQ);
  int t_const = ntiles;
  if (BIAS && !GENERIC) t_const = max(t_mask, min(ntiles, (R1 + C::BN - 1 + C::BMQ - 1) / C::BMQ));
  int t = 0;
  for (; t < t_mask; ++t) tile_body(t, std::true_type{}, std::false_type{});
  for (; t < t_const; ++t) tile_body(t, std::false_type{}, std::false_type{});
  if constexpr (BIAS) {
    for (; t < ntiles; ++t) tile_body(t, std::false_type{}, std::true_type{});
  }

  if (!wave_active) return;
  const float fin_v = -kLn2 * p.inv_n;
  const float fin_k = p.alpha * p.inv_n;
#pragma unroll
  for (int kt = 0; kt < 2; ++kt) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int row = kw0 + kt * 16 + 4 * g + r;
      if (row < L) {
        uint16_t* dstk = p.dk + (sc.start + row) * p.dk_rs + (int64_t)h * D + li;
        uint16_t* dstv = p.dv + (sc.start + row) * p.dv_rs + (int64_t)h * D + li;
#pragma unroll
        for (int dt = 0; dt < C::DT; ++dt) {
          dstk[dt * 16] = to_bf16(dk[kt][dt][r] * fin_k);
          dstv[dt * 16] = to_bf16(dv[kt][dt][r] * fin_v);
        }
      }
    }
  }
}

// =====================================================================
// Full-FP8 backward (hstu_attn_bwd_fp8): e4m3 q, k, v and an e4m3 dO with
// one power-of-two scale per (sequence, head, 32-token group) -- the input
// contract of the reference's production backward (quantize_do_e4m3_blk,
// ops/flydsl/hstu_do_fp8.py:16-38; ops/flydsl/hstu_flydsl_mha.py:1330-1394).
// All five products are v_mfma_scale_f32_16x16x128_f8f6f4:
//   S = Q.K^T, dP = dO8.V^T          e4m3 x e4m3, dP kept in dO8's scaled domain
//   dV^T = dO8^T . P8                P8 = e4m3(silu / N * 2^(c+3)), c = ceil(log2 N);
//                                    the dO group scales 2^-e ride the MFMA's
//                                    E8M0 operand of the dO side
//   dK^T = Q8^T . dS8k               dS8k = e4m3(dS' s_q 2^-Eq 2^(c-3)), E8M0 = dO group
//   dQ^T = K8^T . dS8q^T             dS8q = e4m3(dS' s_k 2^-Ek 2^(c-3)), stored e4m3
// where dS' = s_v dP silu'(x) / N (the dO scale still applied), 2^-Eq / 2^-Ek
// the power-of-two normalisers of the largest q / k scale, and the P and dS
// pre-scales the reference's N-relative ones (hstu_flydsl_mha.py:1351-1370).
//
// K-slot layout.  A 16x16x128 e4m3 operand lane (row, group g) holds K
// indices 16g..16g+15 and 64+16g..+15, and K-block b (32 indices) takes its
// E8M0 scale from lane group b.  In the dK/dV kernel the contraction index is
// the query of a 128-query tile; the S fragment gives lane group g the
// queries 16qs + 4g + r (qs = 0..7).  Two permlane16 swaps per 64 queries
// turn those into runs of eight -- group 0: queries {0-7, 16-23}, 1: {32-39,
// 48-55}, 2: {8-15, 24-31}, 3: {40-47, 56-63} (+64 for the high half) -- so
// K-block b holds exactly the 32 tokens of one dO group (p / 64, (p % 16) / 8),
// and the other operand reads the same tokens with ds_read_b64_tr_b8.
// =====================================================================
struct F8Bwd {
  // dK/dV: a 128-key block is two workgroups of 4 waves (64 keys), 16 keys
  // a wave; three such workgroups share a CU (one LDS stage each, at most 168
  // VGPRs), so the three waves of a SIMD belong to different workgroups and
  // do not meet at the same barriers: while one workgroup waits for its next
  // tile's loads, the others compute
  static constexpr int NT = 256;
  static constexpr int BN = 128, BM = 128;  // keys per block, queries per tile
  // dK/dV stage: Q and dO tiles of 128-byte e4m3 rows, unpadded (LDS DMA
  // writes 1 KiB runs), data chunk c (bytes 16c .. 16c + 15) of row r at
  // 16-byte slot c ^ kv_swz(r).  The swizzle spreads the 16 rows of a
  // ds_read_b128 and the row groups 8 and 32 apart of a ds_read_b64_tr_b8
  // over distinct banks; it is constant under r -> r + 16 (bits 1-3 and 5).
  __host__ __device__ static constexpr int kv_swz(int r) { return swz128(r); }
  static constexpr int Q_OFF = 0;
  static constexpr int DO_OFF = Q_OFF + BM * 128;
  static constexpr int SQ_OFF = DO_OFF + BM * 128;  // 128 fp32 query scales
  static constexpr int B_OFF = SQ_OFF + BM * 4;     // 256 fp32: pre-scaled bias of offsets m0-n0-127 ..
  static constexpr int STAGE = B_OFF + 256 * 4;
  static constexpr int LDS = STAGE;
  static constexpr int TILE = BN * BM;  // one stored e4m3 dS tile (16 KiB)
  // dQ: K tile [key][d] and dS tile [key][query] (queries permuted so that
  // a stored piece is one 16-byte chunk), unpadded 128-byte rows, data chunk
  // c of row r at slot c ^ q_swz(r).  16-byte stores go 8 lanes per pass
  // with banks repeating every 128 bytes: the dS stores (8 aligned rows, one
  // chunk each) and the K stores (one row's 8 chunks) hit distinct banks.
  // The transposed 8-byte reads go 32 lanes per pass over 256 bytes of banks
  // (rows 8 g + (li >> 1) + 32 m, two lane groups g): 16 aligned rows, two
  // lanes a row, are spread when the slots of the even rows, and of the odd
  // rows, differ (bit 3 of the row flips the slot's bit 0).
  __host__ __device__ static constexpr int q_swz(int r) { return (r & 7) ^ ((r >> 3) & 1); }
  static constexpr int QK_OFF = 0;
  static constexpr int QDS_OFF = QK_OFF + BN * 128;
  static constexpr int QHIST_OFF = QDS_OFF + BN * 128;
  static int dq_lds(bool bias, int R) { return QHIST_OFF + (bias ? 4 * R * 4 : 0); }  // a histogram per wave
};

// Stored dS tiles: for key block kb and query tile qt >= kb of a sequence
// with nq = ceil(L / 128) tiles, (sequence, head) items hold nq (nq + 1) / 2
// tiles, kb-major.  Inside a tile: [wave w][half hf][lane][16 bytes], the
// 4 dwords qs = 0..3 of lane (li, g) being keys 16 w + li, queries
// 64 hf + 16 qs + 4 g + (0..3).
__host__ __device__ inline int64_t f8_tiles(int64_t L) {
  const int64_t nq = (L + 127) / 128;
  return nq * (nq + 1) / 2;
}
__device__ __forceinline__ uint8_t* f8_tile(const AttnParams& p, const SeqCtx& c, int kb, int qt) {
  const int64_t nq = (c.L + 127) / 128;
  const int64_t idx = p.ds_base[c.b] * p.H + (int64_t)c.h * f8_tiles(c.L) + (int64_t)kb * nq -
                      (int64_t)kb * (kb - 1) / 2 + (qt - kb);
  return p.ds_ws + idx * F8Bwd::TILE;
}

// The largest scale of array `which` (0: q, 1: k) from the kScaleParts
// partial maxima the set-up launch left (non-negative floats order as their
// bits); every lane of the wave must be active.
constexpr int kScaleParts = 64;
__device__ __forceinline__ unsigned f8_max_scale(const unsigned* parts, int which) {
  static_assert(kScaleParts == 64, "one partial per lane");
  unsigned m = parts[2 * (threadIdx.x & 63) + which];
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) m = max(m, (unsigned)__shfl_xor((int)m, off));
  return __builtin_amdgcn_readfirstlane(m);
}
// 2^-E with E the frexp exponent of the largest scale: s * 2^-E in (0, 1).
__device__ __forceinline__ float f8_norm(unsigned bits) {
  int e = 0;
  (void)frexpf(__uint_as_float(bits), &e);
  return ldexpf(1.0f, -e);
}

__device__ __forceinline__ uint32_t buf_ldu8(BufRsrc r, uint32_t voff) {
  return (uint32_t)__builtin_amdgcn_raw_buffer_load_b8(r, voff, 0, 0);
}

// Scale modes: kScalesPerToken ([T, H] scales), kScalesPerTensor (one scale
// per tensor: the query scale, and so the score's exp2 factor and dS8k's
// factor, is a per-block constant and no query scales are staged),
// kScalesShared (one scale tensor for q, k and v, the reference's qkv_scale:
// also the dK and dQ casts of dS are the same bytes, so each score is cast
// twice (P8, dS8) instead of three times).
enum ScaleMode { kScalesPerToken = 0, kScalesPerTensor = 1, kScalesShared = 2 };

template <bool BIAS, int SM>
__global__ void __launch_bounds__(F8Bwd::NT, 3) hstu_bwd_f8_dkdv_kernel(AttnParams p) {
  constexpr bool PT = SM != kScalesPerToken;
  using C = F8Bwd;
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  SeqCtx sc;
  int half = 0;
  if (!seq_ctx(p, /*heavy_last=*/false, sc, &half)) return;
  const int L = sc.L, h = sc.h;
  const int n0 = sc.blk * C::BN;
  if (n0 >= L) return;
  const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63, li = lane & 15,
            g = lane >> 4;
  const int wv = 4 * half + wave;  // the wave's 16 keys within the 128-key block
  const int kw0 = n0 + 16 * wv;
  const int key = kw0 + li;
  const bool key_ok = key < L;

  // buffer resources over this (sequence, head): rows >= L read as zero
  const uint32_t qrs = (uint32_t)p.q_rs, dors = (uint32_t)p.do_rs;
  const BufRsrc q_rsrc = make_rsrc(p.q + sc.start * p.q_rs + (int64_t)h * 128, L > 0 ? (L - 1) * qrs + 128 : 0u);
  const BufRsrc do_rsrc = make_rsrc(p.do8 + sc.start * p.do_rs + (int64_t)h * 128, L > 0 ? (L - 1) * dors + 128 : 0u);
  const uint32_t s_step = (uint32_t)(p.s_rs * 4);
  const BufRsrc sq_rsrc = make_rsrc(p.q_scale + sc.start * p.s_rs + h * p.s_hs, (uint32_t)(p.s_rs ? L * p.s_rs * 4 : 4));
  const BufRsrc e8_rsrc = make_rsrc(p.e8 + sc.start * p.H + h, (uint32_t)(L * p.H));
  const int ext_len = bias_ext_len(p.N);
  const BufRsrc b_rsrc = make_rsrc(BIAS ? p.bias_ext + (int64_t)h * ext_len : nullptr, BIAS ? (uint32_t)(ext_len * 4) : 0u);

  // this lane's key: e4m3 K and V rows (B operands of S and dP), its scales
  i32x8 kf8 = {0, 0, 0, 0, 0, 0, 0, 0}, vf8 = {0, 0, 0, 0, 0, 0, 0, 0};
  float sk = 0.f, sv = 0.f;
  if (key_ok) {
    const uint8_t* kr = p.k + (sc.start + key) * p.k_rs + (int64_t)h * 128;
    const uint8_t* vr = p.v + (sc.start + key) * p.v_rs + (int64_t)h * 128;
    kf8 = cat8(*(const u32x4*)(kr + 16 * g), *(const u32x4*)(kr + 64 + 16 * g));
    vf8 = cat8(*(const u32x4*)(vr + 16 * g), *(const u32x4*)(vr + 64 + 16 * g));
    sk = p.k_scale[(sc.start + key) * p.s_rs + h * p.s_hs];
    sv = p.v_scale[(sc.start + key) * p.s_rs + h * p.s_hs];
  }
  const float nq = f8_norm(f8_max_scale(p.f8max, 0)), nk = f8_norm(f8_max_scale(p.f8max, 1));
  // P8 = e4m3(t sigma kp) is computed as t sigma' with sigma' = kp sigma =
  // 1 / ((1 + 2^t) / kp); then silu'(x) kp = fma(P, fma(sigma', ln2 / kp, -ln2), sigma'),
  // and the 1 / kp goes into the dS factors
  const float kp = -kLn2 * p.p8_scale * p.inv_n;
  const float ikp = 1.0f / kp, ln2_kp = kLn2 * ikp;
  const float ck = -p.alpha * kLog2e * sk;                    // times s_q: exp2 argument factor
  const float an = sv * nq * p.ds8_scale * p.inv_n * ikp;     // times s_q: dS8k factor
  const float bn = sv * sk * nk * p.ds8_scale * p.inv_n * ikp;  // dS8q factor (with PT also dS8k's)
  // one query scale: the exp2 argument and dS8k factors are constants
  const float sq_pt = PT ? p.q_scale[0] : 0.f;
  const float ck_pt = PT ? ck * sq_pt : 0.f, an_pt = PT ? an * sq_pt : 0.f;

  f32x4 dvt[8], dkt[8];
#pragma unroll
  for (int dt = 0; dt < 8; ++dt) dvt[dt] = dkt[dt] = zero4();

  // one 128-query tile in the workgroup's one stage, loaded by LDS DMA after
  // the previous tile's barrier (the other two workgroups of the CU compute
  // meanwhile): wave w takes rows
  // 8 w + 32 i + (lane >> 3), i = 0..3, of Q and dO (lane slot lane & 7
  // holds data chunk (lane & 7) ^ kv_swz(row), which depends on i through
  // bit 5 of the row), waves 0-1 the 128 query scales, wave w bias values
  // 64 w .. 64 w + 63
  const int lrow = 8 * wave + (lane >> 3);
  uint32_t q_voff[2], d_voff[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const uint32_t chunk = 16u * (uint32_t)((lane & 7) ^ C::kv_swz(lrow + 32 * j));
    q_voff[j] = lrow * qrs + chunk;
    d_voff[j] = lrow * dors + chunk;
  }
  // E8M0 byte of the dO group K-block g covers: token m0 + 64 (g >> 1) + 8 (g & 1),
  // loaded with its tile (complete at the tile's wait)
  const uint32_t e8_tok = 64 * (g >> 1) + 8 * (g & 1);
  int sc_next = 0;
  auto load = [&](int m0, uint8_t* st) {
    sc_next = (int)buf_ldu8(e8_rsrc, (uint32_t)(m0 + (int)e8_tok) * (uint32_t)p.H);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      buf_to_lds<16>(q_rsrc, st + C::Q_OFF + (8 * wave + 32 * i) * 128, q_voff[i & 1], (uint32_t)(m0 + 32 * i) * qrs);
      buf_to_lds<16>(do_rsrc, st + C::DO_OFF + (8 * wave + 32 * i) * 128, d_voff[i & 1],
                     (uint32_t)(m0 + 32 * i) * dors);
    }
    if (!PT && wave < 2)
      buf_to_lds<4>(sq_rsrc, st + C::SQ_OFF + 256 * wave, (uint32_t)lane * s_step, (uint32_t)(m0 + 64 * wave) * s_step);
    if (BIAS) {
      buf_to_lds<4>(b_rsrc, st + C::B_OFF + 256 * wave, (uint32_t)(64 * wave + lane) * 4u,
                    (uint32_t)(m0 - n0 + p.N) * 4u);
    }
  };

  // S / dP A operands: row 64 hf + 16 qs + li, data chunks g and g + 4 at
  // slots g ^ kv_swz(row) and that ^ 4, kv_swz(row) = (li >> 1) ^ 4 (qs >> 1)
  const int ab0 = li * 128 + 16 * (g ^ (li >> 1)), ab1 = ab0 ^ 64;
  // transposed (tr_b8) operand reads: lane group g takes the tokens
  // base(g) + {0, 16} (low half) and + {64, 80} (high half), 8 each; the
  // swizzle of its rows is that of base(g) + li / 2
  const int tr_row = 32 * (g & 1) + 8 * (g >> 1) + (li >> 1);
  const int tr_base = tr_row * 128 + 8 * (li & 1), tr_x = 16 * C::kv_swz(tr_row);
  auto tr_frag = [&](const uint8_t* tile, int dt) {
    const uint8_t* t = tile + tr_base + ((16 * dt) ^ tr_x);
    const u32x2 r0 = lds_tr8(t), r1 = lds_tr8(t + 16 * 128);
    const u32x2 r2 = lds_tr8(t + 64 * 128), r3 = lds_tr8(t + 80 * 128);
    i32x8 f;  // read order: tokens +0..7, +16..23, +64..71, +80..87
    f[0] = (int)r0[0]; f[1] = (int)r0[1]; f[2] = (int)r1[0]; f[3] = (int)r1[1];
    f[4] = (int)r2[0]; f[5] = (int)r2[1]; f[6] = (int)r3[0]; f[7] = (int)r3[1];
    return f;
  };
  const int R1 = p.bias_R - 1;
  const int bias_lane = 127 + 4 * g - 16 * wv - li;  // + 64 hf + 16 qs + r
  const int ntiles = (L - n0 + C::BM - 1) / C::BM;

  // this block's stored dS tiles (query tiles blk, blk + 1, .. are consecutive)
  uint8_t* const ds_dst = f8_tile(p, sc, sc.blk, sc.blk) + (size_t)((wv * 2) * 64 + lane) * 16;
  fp8_saturate_mode(true);
  load(n0, smem);
  lds_dma_wait();
  __syncthreads();

  auto tile_body = [&](int t, auto masked_tag, auto bconst_tag) {
    constexpr bool MASKED = decltype(masked_tag)::value;
    constexpr bool BCONST = decltype(bconst_tag)::value;
    const int m0 = n0 + t * C::BM;
    if (t > 0) {  // after the previous tile's barrier every wave is done with the stage
      load(m0, smem);
      wait_vm_le<0>();
      __syncthreads();
    }
    const uint8_t* buf = smem;
    const int sc_e = sc_next;
    uint8_t* dst = ds_dst + (size_t)t * C::TILE;
    const float* bias_lds = (const float*)(buf + C::B_OFF);
    // the lane's bias values through one opaque LDS base register: the 32
    // reads of a tile then differ only in the instructions' offsets (with a
    // plain pointer the compiler kept 16 addresses live across tiles and
    // spilled them at 168 VGPRs)
    uint32_t bbase = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) uint8_t*)(buf + C::B_OFF) +
                     4u * (uint32_t)bias_lane;
    if constexpr (BIAS) asm volatile("" : "+v"(bbase));
    const __attribute__((address_space(3))) float* blane = (const __attribute__((address_space(3))) float*)(uintptr_t)bbase;
    const float bconst = (BIAS && BCONST) ? bias_lds[0] : 0.f;
    uint32_t pd[8], dk8[8];
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
      f32x4 s[4], dp[4];
#pragma unroll
      for (int qs = 0; qs < 4; ++qs) {
        const int rb = (64 * hf + 16 * qs) * 128;
        const int lo = rb + (qs < 2 ? ab0 : ab1), hi = rb + (qs < 2 ? ab1 : ab0);
        const i32x8 aq = cat8(lds_ld128(buf + C::Q_OFF + lo), lds_ld128(buf + C::Q_OFF + hi));
        const i32x8 ad = cat8(lds_ld128(buf + C::DO_OFF + lo), lds_ld128(buf + C::DO_OFF + hi));
        s[qs] = mfma_fp8(aq, kf8, zero4());
        dp[qs] = mfma_fp8(ad, vf8, zero4());
      }
      uint32_t dq8[4];
#pragma unroll
      for (int qs = 0; qs < 4; ++qs) {
        const f32x4 sq4 = PT ? f32x4{0.f, 0.f, 0.f, 0.f} : lds_ldf4(buf + C::SQ_OFF + (64 * hf + 16 * qs + 4 * g) * 4);
        float pv[4], dkv[4], dqv[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          float tt = PT ? s[qs][r] * ck_pt : s[qs][r] * (ck * sq4[r]);
          if constexpr (BIAS) tt += BCONST ? bconst : blane[64 * hf + 16 * qs + r];
          const float sgk = __builtin_amdgcn_rcpf(__builtin_fmaf(__builtin_amdgcn_exp2f(tt), ikp, ikp));
          float pval = tt * sgk;
          float dsv = dp[qs][r] * __builtin_fmaf(pval, __builtin_fmaf(sgk, ln2_kp, -kLn2), sgk);
          if constexpr (MASKED) {
            const bool ok = 64 * hf + 16 * qs + 4 * g + r >= 16 * wv + li;
            pval = ok ? pval : 0.f;
            dsv = ok ? dsv : 0.f;
          }
          // saturated to +-448 by the conversion (MODE.FP16_OVFL)
          pv[r] = pval;
          dqv[r] = dsv * bn;
          // shared scale: an s_q = bn (s_q = s_k, the same normaliser)
          dkv[r] = SM == kScalesShared ? dqv[r] : dsv * (PT ? an_pt : an * sq4[r]);
        }
        pd[4 * hf + qs] = pack_fp8x4(pv[0], pv[1], pv[2], pv[3]);
        dq8[qs] = pack_fp8x4(dqv[0], dqv[1], dqv[2], dqv[3]);
        dk8[4 * hf + qs] = SM == kScalesShared ? dq8[qs] : pack_fp8x4(dkv[0], dkv[1], dkv[2], dkv[3]);
      }
      __builtin_amdgcn_sched_barrier(0);  // bounds the live ranges at 168 VGPRs
      // the dQ kernel's operand, streamed out (read once, much later)
      __builtin_nontemporal_store(u32x4{dq8[0], dq8[1], dq8[2], dq8[3]}, (u32x4*)(dst + hf * 64 * 16));
      // runs of eight queries per lane group (groups 0<->1 and 2<->3 trade qs 2,3 for qs 0,1)
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const auto a = __builtin_amdgcn_permlane16_swap(pd[4 * hf + j], pd[4 * hf + j + 2], false, false);
        pd[4 * hf + j] = a[0];
        pd[4 * hf + j + 2] = a[1];
        const auto b = __builtin_amdgcn_permlane16_swap(dk8[4 * hf + j], dk8[4 * hf + j + 2], false, false);
        dk8[4 * hf + j] = b[0];
        dk8[4 * hf + j + 2] = b[1];
      }
    }
    __builtin_amdgcn_sched_barrier(0);  // phase B's operand reads stay in phase B
    // after the swaps pd[4 hf + j] holds queries base(g) + 64 hf + {0, 16, 4, 20}[j] + 0..3:
    // B operand dwords in the A fragment's token order (+0..3, 4..7, 16..19, 20..23)
    i32x8 bp, bk;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int src = (j & 4) | ((j & 1) << 1) | ((j >> 1) & 1);  // 0 2 1 3 4 6 5 7
      bp[j] = (int)pd[src];
      bk[j] = (int)dk8[src];
    }
    // dV^T += dO8^T . P8 (dO group scales on the dO side), dK^T += Q8^T . dS8k
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
      const i32x8 ado = tr_frag(buf + C::DO_OFF, dt);
      dvt[dt] = mfma_fp8_scaled(ado, bp, dvt[dt], sc_e, 127);
      const i32x8 aq = tr_frag(buf + C::Q_OFF, dt);
      dkt[dt] = mfma_fp8_scaled(aq, bk, dkt[dt], 127, sc_e);
    }
    // operand reads one step ahead of their MFMAs: {8 tr reads}, 7 x {2 MFMAs, 8 tr reads}, {2 MFMAs}
    __builtin_amdgcn_sched_group_barrier(0x100, 8, 0);
#pragma unroll
    for (int i = 0; i < 7; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 8, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
    __syncthreads();  // every wave is done with the stage
  };

  // tile 0 holds the diagonal; tiles whose smallest offset m0 - n0 - 127 is
  // >= R - 1 see one clamped bias value
  int t_const = ntiles;
  if (BIAS) t_const = max(1, min(ntiles, (R1 + 127 + C::BM - 1) / C::BM));
  tile_body(0, std::true_type{}, std::false_type{});
  int t = 1;
  for (; t < t_const; ++t) tile_body(t, std::false_type{}, std::false_type{});
  if constexpr (BIAS) {
    for (; t < ntiles; ++t) tile_body(t, std::false_type{}, std::true_type{});
  }

  fp8_saturate_mode(false);
  if (!key_ok) return;
  // lane (key, g) holds d = 16 dt + 4 g + r of its key
  const float fin_v = 1.0f / p.p8_scale;
  const float fin_k = p.alpha / (nq * p.ds8_scale);
  uint16_t* dkr = p.dk + (sc.start + key) * p.dk_rs + (int64_t)h * 128 + 4 * g;
  uint16_t* dvr = p.dv + (sc.start + key) * p.dv_rs + (int64_t)h * 128 + 4 * g;
#pragma unroll
  for (int dt = 0; dt < 8; ++dt) {
    *(u32x2*)(dkr + 16 * dt) = u32x2{pack_bf16(dkt[dt][0] * fin_k, dkt[dt][1] * fin_k),
                                     pack_bf16(dkt[dt][2] * fin_k, dkt[dt][3] * fin_k)};
    *(u32x2*)(dvr + 16 * dt) = u32x2{pack_bf16(dvt[dt][0] * fin_v, dvt[dt][1] * fin_v),
                                     pack_bf16(dvt[dt][2] * fin_v, dvt[dt][3] * fin_v)};
  }
}

// dQ from the stored e4m3 dS tiles (and the bias gradient from the same
// bytes).  Block = one 128-query tile qt of a (sequence, head); it walks the
// key blocks kb = 0..qt.  Per step the K tile [key][d] and the dS tile
// [key][query] are staged in LDS; dQ^T = K8^T . dS8q^T with both operands
// read transposed (ds_read_b64_tr_b8), so a lane ends with 4 consecutive d
// of one query.
template <bool BIAS>
__global__ void __launch_bounds__(kThreads, 2) hstu_bwd_f8_dq_kernel(AttnParams p) {
  using C = F8Bwd;
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  SeqCtx sc;
  if (!seq_ctx(p, /*heavy_last=*/true, sc)) return;
  const int L = sc.L, h = sc.h;
  const int qt = sc.blk;
  const int m0 = qt * C::BM;
  if (m0 >= L) return;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, li = lane & 15, g = lane >> 4;
  const uint32_t krs = (uint32_t)p.k_rs;
  const BufRsrc k_rsrc = make_rsrc(p.k + sc.start * p.k_rs + (int64_t)h * 128, L > 0 ? (L - 1) * krs + 128 : 0u);
  const BufRsrc e8_rsrc = make_rsrc(p.e8 + sc.start * p.H + h, (uint32_t)(L * p.H));
  const uint32_t s_step = (uint32_t)(p.s_rs * 4);
  const BufRsrc sk_rsrc = make_rsrc(p.k_scale + sc.start * p.s_rs + h * p.s_hs, (uint32_t)(p.s_rs ? L * p.s_rs * 4 : 4));
  const float nk = f8_norm(f8_max_scale(p.f8max, 1));
  const float unscale = 1.0f / (nk * p.ds8_scale);
  const int R1 = p.bias_R - 1;
  // the wave's bias-gradient histogram, offsets 0 .. R - 1
  float* hist0 = (float*)(smem + C::QHIST_OFF);
  float* hist = hist0 + wave * p.bias_R;
  if constexpr (BIAS) {
    for (int i = tid; i < 4 * p.bias_R; i += kThreads) hist0[i] = 0.f;
  }
  // bias gradient: the E8 byte of the dO group of this lane's query rows in
  // half hf as an f32 exponent field, the scale operand of the scaled e4m3
  // conversion (which multiplies by 2^(field - 127), exactly the group scale)
  float grp[2] = {1.f, 1.f};
  if constexpr (BIAS) {
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
      const uint32_t b = buf_ldu8(e8_rsrc, (uint32_t)(m0 + 64 * hf + 8 * (g >> 1)) * (uint32_t)p.H);
      grp[hf] = __builtin_bit_cast(float, b << 23);
    }
  }

  f32x4 acc[8][2];
#pragma unroll
  for (int dt = 0; dt < 8; ++dt) acc[dt][0] = acc[dt][1] = zero4();

  // staged registers of one key block: 4 K chunks, this lane's 4 dS pieces
  // (waves 2 wave, 2 wave + 1 of the dK/dV kernel, halves 0, 1) and, for the
  // bias gradient, 1 / s_k of its two keys
  u32x4 kc[4], dsp[4];
  float isk[2] = {0.f, 0.f};
  auto load = [&](int kb) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int c = tid + kThreads * i, row = c >> 3, ch = c & 7;
      kc[i] = buf_ld128(k_rsrc, row * krs + 16 * ch, (uint32_t)(kb * C::BN) * krs);
    }
    const uint8_t* tile = f8_tile(p, sc, kb, qt);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int w = 2 * wave + (j >> 1), hf = j & 1;
      dsp[j] = *(const u32x4*)(tile + (size_t)((w * 2 + hf) * 64 + lane) * 16);
    }
    if constexpr (BIAS) {
      // raw s_k; inverted when the step's operands are stored, so that
      // nothing waits for these loads before the current step's math
#pragma unroll
      for (int j = 0; j < 2; ++j)
        isk[j] = buf_ldf(sk_rsrc, (uint32_t)(16 * (2 * wave + j) + li) * s_step, (uint32_t)(kb * C::BN) * s_step);
    }
  };
  auto store = [&]() {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int c = tid + kThreads * i, row = c >> 3, ch = c & 7;
      *(u32x4*)(smem + C::QK_OFF + row * 128 + 16 * (ch ^ C::q_swz(row))) = kc[i];
    }
    // a piece holds queries 64 hf + 16 qs + 4 g + (0..3), qs = 0..3: it goes
    // whole into 16-byte chunk 4 hf + g of its key row (query-permuted rows)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int w = 2 * wave + (j >> 1), hf = j & 1;
      const int r = 16 * w + li;
      *(u32x4*)(smem + C::QDS_OFF + r * 128 + 16 * ((4 * hf + g) ^ C::q_swz(r))) = dsp[j];
    }
  };
  float dclamp = 0.f;
  // bias gradient of the staged step, as per-lane diagonal sums in buckets
  // of 16 offsets.  Bucket v (bk[v + 1], v = -1..8) holds in lane (g, li) the
  // offset i - j = base0 + 16 v - (li - 4 g), base0 = m0 - kb BN - 32 wave
  // (i - j of this wave's first query and key); the 32 x 32 sub-tile of
  // query rows 32 s .. 32 s + 31 (s = 2 hf + qp) folds into buckets
  // 2 s - 1 .. 2 s + 2.  Unskewed, bucket w holds base0 + 16 w - li in every
  // row.  The next step's buckets 7, 8 are this step's -1, 0, so a step
  // completes the offsets base0 + 17 .. base0 + 144 (unskewed buckets 2..9,
  // bucket 9 the previous step's 1) and carries buckets -1, 0 and unskewed 1.
  float cr_m1 = 0.f, cr_0 = 0.f, cr_g1 = 0.f;
  const bool wrap = li + 4 * g >= 16;
  // unskewed buckets t0..t3 = w, w + 1, w + 2, w + 3: lane (g, li) sums
  // offset xw - li + 16 g, xw = base0 + 16 w
  auto flush = [&](float t0, float t1, float t2, float t3, int xw) {
    const float dv = diag_scatter(t0, t1, t2, t3, lane);
    const int off = xw + 16 * g - li;
    if (off >= R1) dclamp += dv;
    else if (off >= 0) atomicAdd(&hist[off], dv);
  };
  // the 16 scores of sub-tile s, query sub-tile a, key sub-tile kt, times
  // their dO group scale (exact: a power of two), not yet times 1 / s_k
  auto piece = [&](const u32x4 (&pcs)[4], int s, int a, int kt, float (&v)[4]) {
    const int hf = s >> 1, qp = s & 1;
    const uint32_t w = pcs[2 * kt + hf][2 * qp + a];
    const f32x2 lo = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(w, grp[hf], false);
    const f32x2 hi = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(w, grp[hf], true);
    v[0] = lo[0];
    v[1] = lo[1];
    v[2] = hi[0];
    v[3] = hi[1];
  };
  auto bias_grad = [&](int kb, const u32x4 (&pcs)[4], const float (&iskv)[2]) {
    const int base0 = m0 - kb * C::BN - 32 * wave;
    if (base0 - 31 >= R1) {  // every offset clamps
#pragma unroll
      for (int s = 0; s < 4; ++s)
#pragma unroll
        for (int a = 0; a < 2; ++a)
#pragma unroll
          for (int kt = 0; kt < 2; ++kt) {
            float v[4];
            piece(pcs, s, a, kt, v);
            dclamp = __builtin_fmaf((v[0] + v[1]) + (v[2] + v[3]), iskv[kt], dclamp);
          }
      cr_m1 = cr_0 = cr_g1 = 0.f;
      return;
    }
    float bk[10];
#pragma unroll
    for (int i = 0; i < 8; ++i) bk[i] = 0.f;
    bk[8] = cr_m1;
    bk[9] = cr_0;
    // 1 / s_k of the key that lane (p + r) mod 16 holds, per key sub-tile
    float ck[2][4];
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) {
      ck[kt][0] = iskv[kt];
      ck[kt][1] = row_rot<1>(iskv[kt]);
      ck[kt][2] = row_rot<2>(iskv[kt]);
      ck[kt][3] = row_rot<3>(iskv[kt]);
    }
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      // rows = queries (16 a + 4 g + r), cols = keys (16 kt + li): shift kt - a
      float v00[4], v11[4], v01[4], v10[4];
      piece(pcs, s, 0, 0, v00);
      piece(pcs, s, 1, 1, v11);
      piece(pcs, s, 0, 1, v01);
      piece(pcs, s, 1, 0, v10);
      diag_fma_to(bk[2 * s + 1], bk[2 * s + 2], v00, ck[0]);
      diag_fma_to(bk[2 * s + 1], bk[2 * s + 2], v11, ck[1]);
      diag_fma_to(bk[2 * s], bk[2 * s + 1], v01, ck[1]);
      diag_fma_to(bk[2 * s + 2], bk[2 * s + 3], v10, ck[0]);
    }
    float gu[10];  // unskewed bucket w = 1..9
#pragma unroll
    for (int w = 1; w < 9; ++w) gu[w] = skew_undo(bk[w + 1]);
    gu[9] = cr_g1;
    float t[10];  // bucket w: offsets base0 + 16 w - li (wrapped lanes read bucket w - 1)
#pragma unroll
    for (int w = 2; w < 10; ++w) t[w] = wrap ? gu[w - 1] : gu[w];
    flush(t[2], t[3], t[4], t[5], base0 + 32);
    flush(t[6], t[7], t[8], t[9], base0 + 96);
    cr_m1 = bk[0];
    cr_0 = bk[1];
    cr_g1 = gu[1];
  };

  // operand reads: dS^T columns (byte 16 chunk + li of the permuted rows:
  // query 64 (chunk >> 2) + 4 (chunk & 3) + 16 (li >> 2) + (li & 3)) and K^T
  // rows (d = 16 chunk + li) over the keys 8 g + 32 m .. + 7, m = 0..3 (the
  // contraction order is the same for both operands)
  const int tr_row = 8 * g + (li >> 1);
  const int trk = tr_row * 128 + 8 * (li & 1), trx = 16 * C::q_swz(tr_row);
  auto frag = [&](const uint8_t* tile, int chunk) {
    const uint8_t* t = tile + trk + ((16 * chunk) ^ trx);
    const u32x2 r0 = lds_tr8(t), r1 = lds_tr8(t + 32 * 128);
    const u32x2 r2 = lds_tr8(t + 64 * 128), r3 = lds_tr8(t + 96 * 128);
    i32x8 f;
    f[0] = (int)r0[0]; f[1] = (int)r0[1]; f[2] = (int)r1[0]; f[3] = (int)r1[1];
    f[4] = (int)r2[0]; f[5] = (int)r2[1]; f[6] = (int)r3[0]; f[7] = (int)r3[1];
    return f;
  };

  const int nsteps = qt + 1;
  load(0);
  store();
  __syncthreads();
  for (int kb = 0; kb < nsteps; ++kb) {
    u32x4 cur[4];
    float cur_isk[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) cur_isk[j] = isk[j] > 0.f ? unscale / isk[j] : 0.f;
#pragma unroll
    for (int j = 0; j < 4; ++j) cur[j] = dsp[j];
    if (kb + 1 < nsteps) load(kb + 1);
    i32x8 bq[2];
#pragma unroll
    for (int qs = 0; qs < 2; ++qs) bq[qs] = frag(smem + C::QDS_OFF, 2 * wave + qs);
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
      const i32x8 ak = frag(smem + C::QK_OFF, dt);
      acc[dt][0] = mfma_fp8(ak, bq[0], acc[dt][0]);
      acc[dt][1] = mfma_fp8(ak, bq[1], acc[dt][1]);
    }
    if constexpr (BIAS) bias_grad(kb, cur, cur_isk);
    __syncthreads();
    if (kb + 1 < nsteps) {
      store();
      __syncthreads();
    }
  }

  if constexpr (BIAS) {
    // the carried buckets: unskewed 7, 8, 9 of a step past the last (its
    // buckets 1..6 are empty), offsets down to the last step's base0 - 47
    const int base_v = m0 - nsteps * C::BN - 32 * wave;
    if (base_v + 144 >= 0) {
      const float g7 = skew_undo(cr_m1), g8 = skew_undo(cr_0);
      flush(0.f, wrap ? 0.f : g7, wrap ? g7 : g8, wrap ? g8 : cr_g1, base_v + 96);
    }
    hist_add_clamped(hist, R1, dclamp, lane);
    dbias_store_row<4>(p, hist0, sc.b, qt, h);
  }
  // dQ_i = alpha 2^-e(i) / (nk ds8_scale) . acc
  const float fin = p.alpha * unscale;
#pragma unroll
  for (int qs = 0; qs < 2; ++qs) {
    const int chunk = 2 * wave + qs;
    const int row = m0 + 64 * (chunk >> 2) + 4 * (chunk & 3) + 16 * (li >> 2) + (li & 3);
    if (row >= L) continue;
    const uint32_t b = buf_ldu8(e8_rsrc, (uint32_t)row * (uint32_t)p.H);
    const float f = fin * ldexpf(1.0f, (int)b - 127);
    uint16_t* dst = p.dq + (sc.start + row) * p.dq_rs + (int64_t)h * 128 + 4 * g;
#pragma unroll
    for (int dt = 0; dt < 8; ++dt)
      *(u32x2*)(dst + 16 * dt) = u32x2{pack_bf16(acc[dt][qs][0] * f, acc[dt][qs][1] * f),
                                       pack_bf16(acc[dt][qs][2] * f, acc[dt][qs][3] * f)};
  }
}

// out[b] = sum over sequences b' < b of count(b), out[B] = the total, by
// one 1024-thread block; part: 1024 int64 of shared memory.
template <class F>
__device__ void seq_exclusive_scan(int B, F count, int64_t* part, int64_t* out) {
  const int tid = threadIdx.x, per = (B + 1023) / 1024, b0 = tid * per;
  int64_t sum = 0;
  for (int i = 0; i < per; ++i)
    if (b0 + i < B) sum += count(b0 + i);
  part[tid] = sum;
  __syncthreads();
  for (int off = 1; off < 1024; off <<= 1) {
    const int64_t add = tid >= off ? part[tid - off] : 0;
    __syncthreads();
    part[tid] += add;
    __syncthreads();
  }
  int64_t run = tid ? part[tid - 1] : 0;
  for (int i = 0; i < per; ++i) {
    if (b0 + i < B) {
      out[b0 + i] = run;
      run += count(b0 + i);
    }
  }
  if (tid == 1023) out[B] = part[1023];
  __syncthreads();
}

// 128-query dQ blocks of a sequence: ceil(min(length, N) / 128).
__device__ __forceinline__ int64_t dq_blocks(const int64_t* seq_offsets, int b, int N) {
  return (min(seq_offsets[b + 1] - seq_offsets[b], (int64_t)N) + 127) / 128;
}

// base[b] = sum over sequences b' < b of f8_tiles(min(length, N)); base[B] =
// the total; dq_base the same prefix of 128-query blocks (the bias-gradient
// rows).
__device__ void f8_tile_prefix(const int64_t* seq_offsets, int B, int N, int64_t* base, int64_t* dq_base) {
  __shared__ int64_t part[1024];
  seq_exclusive_scan(B, [&](int b) { return f8_tiles(min(seq_offsets[b + 1] - seq_offsets[b], (int64_t)N)); },
                     part, base);
  seq_exclusive_scan(B, [&](int b) { return dq_blocks(seq_offsets, b, N); }, part, dq_base);
}

// Partial maxima of |q_scale| and |k_scale| over [T, H] (or the scalar):
// block bx of kScaleParts 1024-thread blocks writes parts[2 bx], [2 bx + 1]
// (float bits) over tokens bx * 1024 + tid, stepping by kScaleParts * 1024.
__device__ void f8_scale_part(const float* qs, const float* ks, int64_t ntok, int H, int64_t srs, int64_t shs,
                              unsigned* parts, int bx) {
  __shared__ float red[2][16];
  float mq = 0.f, mk = 0.f;
  for (int64_t t = bx * (int64_t)blockDim.x + threadIdx.x; t < ntok; t += (int64_t)kScaleParts * blockDim.x) {
    for (int hh = 0; hh < H; ++hh) {
      const int64_t o = t * srs + hh * shs;
      mq = fmaxf(mq, fabsf(qs[o]));
      mk = fmaxf(mk, fabsf(ks[o]));
    }
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    mq = fmaxf(mq, __shfl_xor(mq, off));
    mk = fmaxf(mk, __shfl_xor(mk, off));
  }
  const int wv = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    red[0][wv] = mq;
    red[1][wv] = mk;
  }
  __syncthreads();
  if (threadIdx.x < 2) {
    float m = 0.f;
    for (int w = 0; w < (int)(blockDim.x >> 6); ++w) m = fmaxf(m, red[threadIdx.x][w]);
    parts[2 * bx + threadIdx.x] = __float_as_uint(m);
  }
}

// e4m3 q rows -> exact bf16 copy [T, H, D] for the dK/dV kernel (scale 1).
__global__ void convert_q8_bf16(const uint8_t* q8, int64_t q_rs, const int64_t* seq_offsets, int B, int H, int D,
                                uint16_t* q16) {
  const int64_t T = seq_offsets[B];
  const int cpr = H * D / 16;  // 16-element chunks per token
  const int64_t n = T * cpr;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t t = i / cpr;
    const int c = (int)(i - t * cpr);
    const u32x4 w = *(const u32x4*)(q8 + t * q_rs + c * 16);
    u32x4 lo, hi;
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      lo[2 * e] = cvt_fp8x2_bf16<false>(w[e]);
      lo[2 * e + 1] = cvt_fp8x2_bf16<true>(w[e]);
      hi[2 * e] = cvt_fp8x2_bf16<false>(w[e + 2]);
      hi[2 * e + 1] = cvt_fp8x2_bf16<true>(w[e + 2]);
    }
    u32x4* dst = (u32x4*)(q16 + t * (int64_t)H * D + c * 16);
    dst[0] = lo;
    dst[1] = hi;
  }
}

// bias table [H, 2R-1] -> [H, bias_ext_len(N)] with entry off+N+127 =
// bias(clamp(off)) * -log2(e): block bx of nbx of head h
__device__ void build_bias_ext(const float* bias, int R, int N, float* ext, int h, int bx, int nbx) {
  const int len = bias_ext_len(N);
  const int R1 = R - 1;
  for (int i = bx * blockDim.x + threadIdx.x; i < len; i += nbx * blockDim.x) {
    const int off = i - N - 127;
    ext[(int64_t)h * len + i] = bias[(int64_t)h * (2 * R - 1) + min(max(off, -R1), R1) + R1] * -kLog2e;
  }
}

// ---------------------------------------------------------------------------
// Block schedule.  Workgroups are dispatched to the 8 XCDs round-robin
// (workgroup i -> XCD i % 8), and each XCD has its own L2.  The schedule
// gives every XCD whole (sequence, head) items, so the 128-row blocks of one
// item run on one XCD at about the same time and re-read that item's K/V
// (forward, dQ) or Q/dO (dK/dV) tiles from that XCD's L2 instead of from
// HBM.  Items are ranked by block count (descending; counting sort, ties in
// any order) and dealt in snake order 0..7,7..0,..., which keeps the per-XCD
// work of a sorted list within one item of even; on an XCD they run in rank
// order, heaviest first.  One workgroup of 1024 threads; O(B*H) work.
// Output (ints): items[8][cap], start[8][cap+1] (exclusive block-count
// prefix per XCD, start[x][n_x] = the XCD's total), count[8]; scratch nb[B],
// rank[B].
// ---------------------------------------------------------------------------
constexpr int kSchedBins = 1024;  // block counts >= 1023 share the last bin (order only)

__host__ __device__ inline int sched_cap(int B, int H) { return (B * H + 7) / 8; }
inline int64_t sched_ints(int B, int H) {
  const int64_t cap = sched_cap(B, H);
  return 8 * cap + 8 * (cap + 1) + 8 + 2 * (int64_t)B;
}

__device__ void schedule_block(const int64_t* seq_offsets, int B, int H, int N, int* ws) {
  const int cap = sched_cap(B, H);
  int* items = ws;
  int* start = items + 8 * cap;
  int* count = start + 8 * (cap + 1);
  int* nbv = count + 8;
  int* rank = nbv + B;
  __shared__ int bins[kSchedBins];
  __shared__ int scan[kSchedBins];
  const int tid = threadIdx.x;  // blockDim.x == kSchedBins
  bins[tid] = 0;
  __syncthreads();
  for (int b = tid; b < B; b += kSchedBins) {
    const int64_t L = min(seq_offsets[b + 1] - seq_offsets[b], (int64_t)N);
    const int nb = (int)((max(L, (int64_t)0) + 127) / 128);
    nbv[b] = nb;
    atomicAdd(&bins[min(nb, kSchedBins - 1)], 1);
  }
  __syncthreads();
  // exclusive prefix in descending bin order: first rank of bin v = sum of bins above v
  const int v = kSchedBins - 1 - tid;
  const int mine = bins[v];
  scan[tid] = mine;
  __syncthreads();
  for (int off = 1; off < kSchedBins; off <<= 1) {
    const int add = tid >= off ? scan[tid - off] : 0;
    __syncthreads();
    scan[tid] += add;
    __syncthreads();
  }
  bins[v] = scan[tid] - mine;
  __syncthreads();
  for (int b = tid; b < B; b += kSchedBins) rank[b] = atomicAdd(&bins[min(nbv[b], kSchedBins - 1)], 1);
  __syncthreads();
  // item r = rank*H + head -> XCD by snake order, dense index j on that XCD
  for (int b = tid; b < B; b += kSchedBins) {
    const int nb = nbv[b];
    for (int h = 0; h < H; ++h) {
      const int r = rank[b] * H + h, q = r & 15;
      const int x = q < 8 ? q : 15 - q;
      const int j = (r >> 4) * 2 + (q >= 8 ? 1 : 0);
      items[x * cap + j] = b * H + h;
      start[x * (cap + 1) + j] = nb;
    }
  }
  __syncthreads();
  // per XCD (one wave each): exclusive scan of the block counts
  const int wave = tid >> 6, lane = tid & 63;
  if (wave < 8) {
    const int x = wave, BH = B * H, full = BH >> 4, rem = BH & 15;
    const int n = 2 * full + (x < rem ? 1 : 0) + (15 - x < rem ? 1 : 0);
    int* st = start + x * (cap + 1);
    int carry = 0;
    for (int j0 = 0; j0 < n; j0 += 64) {
      const int j = j0 + lane;
      const int c = j < n ? st[j] : 0;
      int incl = c;
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const int y = __shfl_up(incl, o);
        if (lane >= o) incl += y;
      }
      if (j < n) st[j] = carry + incl - c;
      carry += __shfl(incl, 63);
    }
    if (lane == 0) {
      st[n] = carry;
      count[x] = n;
    }
  }
}

// Point p at the block schedule in ws (sched_ints(B, H) ints).
void use_schedule(AttnParams& p, int B, int H, int* ws) {
  p.sched_cap = sched_cap(B, H);
  p.sched_items = ws;
  p.sched_start = ws + 8 * p.sched_cap;
  p.sched_count = p.sched_start + 8 * (p.sched_cap + 1);
}
// grid covering every XCD's longest possible list
int sched_grid(int B, int H, int N) { return 8 * sched_cap(B, H) * ((N + 127) / 128); }

int64_t align256(int64_t b) { return (b + 255) / 256 * 256; }
int64_t bias_ext_bytes(int H, int N) { return align256((int64_t)H * bias_ext_len(N) * 4); }
// Bias-gradient rows: one per dQ block and head, at most ceil(T/128) + B
// blocks per head, of up to 2R - 1 floats; then the chunk sums.
int64_t dbias_rows_bytes(int64_t T, int B, int H, int R) {
  return align256(((T + 127) / 128 + B) * H * (int64_t)(2 * R - 1) * 4);
}
int64_t dbias_chunks_bytes(int H, int R) { return align256((int64_t)kDbiasChunks * H * (2 * R - 1) * 4); }
int64_t sched_bytes(int B, int H) { return align256(sched_ints(B, H) * 4); }
// Forward workspace: the block schedule.
int64_t fwd_workspace_bytes(int B, int H) { return sched_bytes(B, H); }
// Backward workspace: [block schedule][pre-clamped bias rows][bf16 copy of
// e4m3 q][bias-gradient rows][their chunk sums][dQ block prefix][dS tile
// prefix][dS tiles]; byte offsets of each part.  The dS tiles are sized by a bound that needs no lengths:
// ds_tiles(L) <= 2 nb (nb + 1) with nb = ceil(L / 128) <= ceil(N / 128), so
// the sum over sequences is at most 2 (ceil(N/128) + 1) (ceil(T/128) + B).
struct BwdWs {
  int64_t sched, bias_ext, q16, part, chunks, dq_base, ds_base, ds, total;
};
int64_t ds_tiles_bound(int64_t T, int B, int N) { return 2 * ((N + 127) / 128 + 1) * ((T + 127) / 128 + B); }
BwdWs bwd_ws(int dtype, int64_t T, int B, int H, int D, int N, int R) {
  BwdWs w;
  int64_t o = 0;
  w.sched = o;
  o += sched_bytes(B, H);
  w.bias_ext = o;
  if (R > 0) o += bias_ext_bytes(H, N);
  w.q16 = o;
  if (dtype == HSTU_DTYPE_FP8_E4M3) o += align256(T * H * D * 2);
  w.part = o;
  if (R > 0) o += dbias_rows_bytes(T, B, H, R);
  w.chunks = o;
  if (R > 0) o += dbias_chunks_bytes(H, R);
  w.dq_base = o;
  o += align256(((int64_t)B + 1) * 8);
  w.ds_base = o;
  o += align256(((int64_t)B + 1) * 8);
  w.ds = o;
  o += ds_tiles_bound(T, B, N) * H * kDsTileBytes;
  w.total = o;
  return w;
}


// base[b] = sum over sequences b' < b of ds_tiles(min(length, N)); base[B] =
// the total; dq_base (if not null) the same prefix of 128-query blocks.
__global__ void __launch_bounds__(1024) ds_tile_prefix(const int64_t* seq_offsets, int B, int N, int64_t* base,
                                                       int64_t* dq_base) {
  __shared__ int64_t part[1024];
  seq_exclusive_scan(B, [&](int b) { return ds_tiles(min(seq_offsets[b + 1] - seq_offsets[b], (int64_t)N)); },
                     part, base);
  if (dq_base != nullptr) seq_exclusive_scan(B, [&](int b) { return dq_blocks(seq_offsets, b, N); }, part, dq_base);
}

// dq_base alone (the recomputing dQ kernel's bias-gradient rows).
__global__ void __launch_bounds__(1024) dq_block_prefix(const int64_t* seq_offsets, int B, int N, int64_t* dq_base) {
  __shared__ int64_t part[1024];
  seq_exclusive_scan(B, [&](int b) { return dq_blocks(seq_offsets, b, N); }, part, dq_base);
}

// Chunk c of head h's bias-gradient rows: the sum of rows c * per ..
// min((c + 1) * per, n) - 1 in a fixed order, n = dq_base[B] rows per head.
__global__ void dbias_chunk_sum(const float* rows, const int64_t* dq_base, int B, int H, int W, float* chunks) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x, h = blockIdx.y, c = blockIdx.z;
  if (i >= W) return;
  const int64_t n = dq_base[B], per = (n + kDbiasChunks - 1) / kDbiasChunks;
  const int64_t r0 = c * per, r1 = min(n, r0 + per);
  // row r0 + 8 j + k into accumulator k (eight loads in flight), then a fixed tree
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  int64_t r = r0;
  for (; r + 8 <= r1; r += 8) {
#pragma unroll
    for (int k = 0; k < 8; ++k) acc[k] += rows[((r + k) * H + h) * W + i];
  }
#pragma unroll
  for (int k = 0; k < 7; ++k)
    if (r + k < r1) acc[k] += rows[((r + k) * H + h) * W + i];
  const float s = ((acc[0] + acc[1]) + (acc[2] + acc[3])) + ((acc[4] + acc[5]) + (acc[6] + acc[7]));
  chunks[((int64_t)c * H + h) * W + i] = s;
}

// dbias [H, 2R - 1] = scale * the chunks summed in a fixed order.  A row of W
// floats holds the offsets R - W .. R - 1; dbias entries below are zero.
__global__ void dbias_finish(const float* chunks, int H, int W, int R, float scale, float* dbias) {
  const int j = blockIdx.x * blockDim.x + threadIdx.x, h = blockIdx.y, n = 2 * R - 1;
  if (j >= n) return;
  const int i = j - (n - W);
  // chunk c into accumulator c % 8 (eight loads in flight), then a fixed tree
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  if (i >= 0) {
    static_assert(kDbiasChunks % 8 == 0, "whole groups of eight chunks");
    for (int c = 0; c < kDbiasChunks; c += 8) {
#pragma unroll
      for (int k = 0; k < 8; ++k) acc[k] += chunks[((int64_t)(c + k) * H + h) * W + i];
    }
  }
  const float s = ((acc[0] + acc[1]) + (acc[2] + acc[3])) + ((acc[4] + acc[5]) + (acc[6] + acc[7]));
  dbias[(int64_t)h * n + j] = s * scale;
}

// The bias gradient from the dQ blocks' rows (p.dbias_part, p.dq_base,
// p.dbias_w): chunk sums, then dbias, both in a fixed order.
hipError_t dbias_reduce(const AttnParams& p, float* chunks, float scale, float* dbias, hipStream_t stream) {
  const int W = p.dbias_w;
  hipLaunchKernelGGL(dbias_chunk_sum, dim3((W + 255) / 256, p.H, kDbiasChunks), dim3(256), 0, stream,
                     p.dbias_part, p.dq_base, p.B, p.H, W, chunks);
  hipLaunchKernelGGL(dbias_finish, dim3((2 * p.bias_R - 1 + 255) / 256, p.H), dim3(256), 0, stream, chunks, p.H, W,
                     p.bias_R, scale, dbias);
  return hipGetLastError();
}

// Rows of a sequence beyond max_seq_len are not computed by the kernels (the
// reference's padded path drops them, so their output is zero); zero them so
// every output element is written.  Exits at once when every L <= N.
// Block bx of nbx of sequence s.
__device__ void zero_rows_beyond_n(const int64_t* seq_offsets, int N, int width, uint16_t* a, int64_t a_rs,
                                   uint16_t* b, int64_t b_rs, uint16_t* c, int64_t c_rs, int s, int bx, int nbx) {
  const int64_t start = seq_offsets[s];
  const int L = (int)(seq_offsets[s + 1] - start);
  for (int row = N + bx; row < L; row += nbx) {
    for (int col = threadIdx.x; col < width; col += blockDim.x) {
      a[(start + row) * a_rs + col] = 0;
      if (b) b[(start + row) * b_rs + col] = 0;
      if (c) c[(start + row) * c_rs + col] = 0;
    }
  }
}

// The small set-up work of an attention call in one launch of 1024-thread
// blocks, by block role (each block takes one role, so every barrier inside
// a role is block-uniform): the block schedule (one block, if sched); the FP8
// backward's tile and dQ-block prefixes (one block) and the partial maxima of
// its q and k scales (kScaleParts blocks), if tile_base; the pre-clamped bias rows (bias_bx blocks per head,
// if bias_ext); rows past N zeroed in up to three outputs (kPrepZero blocks
// per sequence, if z[0]).  The roles touch disjoint memory.
constexpr int kPrepZero = 4;
struct PrepArgs {
  const int64_t* seq_offsets;
  int B, H, N;
  int* sched;  // null: no schedule block
  int64_t* tile_base;
  int64_t* dq_base;
  unsigned* f8max;  // tile_base null: no prefix and no scale blocks
  const float* qs;
  const float* ks;
  int64_t ntok;
  int sH;
  int64_t srs, shs;
  const float* bias;
  float* bias_ext;  // null: no bias blocks
  int R, bias_bx;
  int width;
  uint16_t* z[3];  // z[0] null: no zeroing blocks
  int64_t zrs[3];
};
int prep_blocks(const PrepArgs& a) {
  return (a.sched ? 1 : 0) + (a.tile_base ? 1 + kScaleParts : 0) + (a.bias_ext ? a.H * a.bias_bx : 0) +
         (a.z[0] ? kPrepZero * a.B : 0);
}
__global__ void __launch_bounds__(1024) attn_prep(PrepArgs a) {
  int blk = (int)blockIdx.x;
  if (a.sched) {
    if (blk == 0) {
      schedule_block(a.seq_offsets, a.B, a.H, a.N, a.sched);
      return;
    }
    blk -= 1;
  }
  if (a.tile_base) {
    if (blk == 0) {
      f8_tile_prefix(a.seq_offsets, a.B, a.N, a.tile_base, a.dq_base);
      return;
    }
    if (blk <= kScaleParts) {
      f8_scale_part(a.qs, a.ks, a.ntok, a.sH, a.srs, a.shs, a.f8max, blk - 1);
      return;
    }
    blk -= 1 + kScaleParts;
  }
  if (a.bias_ext) {
    const int nb = a.H * a.bias_bx;
    if (blk < nb) {
      build_bias_ext(a.bias, a.R, a.N, a.bias_ext, blk / a.bias_bx, blk % a.bias_bx, a.bias_bx);
      return;
    }
    blk -= nb;
  }
  if (a.z[0] && blk < kPrepZero * a.B)
    zero_rows_beyond_n(a.seq_offsets, a.N, a.width, a.z[0], a.zrs[0], a.z[1], a.zrs[1], a.z[2], a.zrs[2],
                       blk / kPrepZero, blk % kPrepZero, kPrepZero);
}
hipError_t launch_prep(const PrepArgs& a, hipStream_t stream) {
  const int n = prep_blocks(a);
  if (n > 0) hipLaunchKernelGGL(attn_prep, dim3(n), dim3(1024), 0, stream, a);
  return hipGetLastError();
}
PrepArgs prep_args(const int64_t* seq_offsets, int B, int H, int N) {
  PrepArgs a{};
  a.seq_offsets = seq_offsets;
  a.B = B;
  a.H = H;
  a.N = N;
  return a;
}

// ---------------------------------------------------------------- launch
constexpr int kMaxLdsBytes = 160 * 1024;  // LDS of one gfx950 CU

// Raise each kernel's dynamic-LDS limit to the CU's 160 KiB once; the actual
// allocation is the launch's size (the forward uses ~72 KiB, so two
// workgroups share a CU).
hipError_t ensure_lds(const void* fn) {
  static std::mutex mu;
  static std::vector<const void*> done;
  std::lock_guard<std::mutex> lock(mu);
  for (const void* d : done)
    if (d == fn) return hipSuccess;
  hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, kMaxLdsBytes);
  if (e == hipSuccess) done.push_back(fn);
  return e;
}

hipError_t launch(void (*kernel)(AttnParams), int lds, int grid, AttnParams p, hipStream_t stream,
                  int threads = kThreads) {
  if (lds > kMaxLdsBytes) return hipErrorInvalidValue;
  // a kernel with static LDS only (lds == 0) needs no dynamic limit; raising
  // it to the whole CU would exceed what its static part leaves
  if (lds > 0) {
    hipError_t e = ensure_lds((const void*)kernel);
    if (e != hipSuccess) return e;
  }
  void* args[] = {&p};
  return hipLaunchKernel((const void*)kernel, dim3(grid), dim3(threads), args, (size_t)lds, stream);
}

bool check_common(int dtype, int H, int D, int B, int N, int64_t rs_q, int64_t rs_k, int64_t rs_v,
                  const float* qs, const float* ks, const float* vs, int bias_R, const float* bias) {
  if (dtype != HSTU_DTYPE_BF16 && dtype != HSTU_DTYPE_FP8_E4M3) return false;
  if (B < 0 || H <= 0 || N <= 0) return false;
  if (rs_q < (int64_t)H * D || rs_k < (int64_t)H * D || rs_v < (int64_t)H * D) return false;
  if (dtype == HSTU_DTYPE_FP8_E4M3 && (!qs || !ks || !vs)) return false;
  if (bias != nullptr && bias_R < 1) return false;
  return true;
}

int row_alignment_ok(int dtype, int64_t rs, const void* ptr) {
  // 16-byte vector loads need every row (and the head offset) 16-byte aligned.
  const int es = dtype == HSTU_DTYPE_BF16 ? 2 : 1;
  return ((rs * es) % 16 == 0) && (((uintptr_t)ptr) % 16 == 0);
}

}  // namespace

extern "C" const char* hstu_version(void) {
  return "hstu-mi355x 0.1 (gfx950: bf16 16x16x32 / e4m3 16x16x128 MFMA)";
}

namespace {
// Argument checks shared by both forward entry points (0 = launchable).
int fwd_check(int dtype, const void* q, const void* k, const void* v, int64_t q_row_stride, int64_t k_row_stride,
              int64_t v_row_stride, const float* q_scale, const float* k_scale, const float* v_scale, int B, int H,
              int D, int max_seq_len, const float* attn_bias, int bias_R, int64_t total_tokens) {
  if (!check_common(dtype, H, D, B, max_seq_len, q_row_stride, k_row_stride, v_row_stride, q_scale, k_scale,
                    v_scale, bias_R, attn_bias) ||
      total_tokens < 0)
    return HSTU_E_BAD_ARG;
  if (!(D == 128 || (D == 64 && dtype == HSTU_DTYPE_BF16))) return HSTU_E_UNSUPPORTED;
  if (!row_alignment_ok(dtype, q_row_stride, q) || !row_alignment_ok(dtype, k_row_stride, k) ||
      !row_alignment_ok(dtype, v_row_stride, v))
    return HSTU_E_UNSUPPORTED;
  return 0;
}

// The forward launches; `sched_ws` holds sched_ints(B, H) ints of device memory.
int fwd_launch(int dtype, const void* q, const void* k, const void* v, int64_t q_row_stride, int64_t k_row_stride,
               int64_t v_row_stride, const float* q_scale, const float* k_scale, const float* v_scale,
               int64_t scale_row_stride, int64_t scale_head_stride, const int64_t* seq_offsets, int B, int H, int D,
               int max_seq_len, float alpha, const int32_t* num_targets, int max_attn_len, int contextual_seq_len,
               const float* attn_bias, int bias_R, void* out, int64_t out_row_stride, int* sched_ws,
               hipStream_t stream, float pv_scale = 0.f) {
  AttnParams p{};
  p.q = (const uint8_t*)q;
  p.k = (const uint8_t*)k;
  p.v = (const uint8_t*)v;
  p.q_rs = q_row_stride;
  p.k_rs = k_row_stride;
  p.v_rs = v_row_stride;
  p.q_scale = q_scale;
  p.k_scale = k_scale;
  p.v_scale = v_scale;
  p.s_rs = scale_row_stride;
  p.s_hs = scale_head_stride;
  p.seq_offsets = seq_offsets;
  p.num_targets = num_targets;
  p.out = (uint16_t*)out;
  p.o_rs = out_row_stride;
  p.B = B;
  p.H = H;
  p.N = max_seq_len;
  p.alpha = alpha;
  p.inv_n = 1.0f / (float)max_seq_len;
  p.max_attn_len = max_attn_len;
  p.contextual_seq_len = contextual_seq_len;
  const bool generic = num_targets != nullptr || max_attn_len > 0 || contextual_seq_len > 0;
  p.blocks_per_seq = (max_seq_len + 127) / 128;
  const int grid = sched_grid(B, H, max_seq_len);
  p.bias = attn_bias;
  p.bias_R = bias_R;
  // the block schedule, and the rows past max_seq_len zeroed, in one launch
  PrepArgs pa = prep_args(seq_offsets, B, H, max_seq_len);
  pa.sched = sched_ws;
  pa.width = H * D;
  pa.z[0] = p.out;
  pa.zrs[0] = p.o_rs;
  hipError_t e = launch_prep(pa, stream);
  if (e != hipSuccess) return (int)e;
  use_schedule(p, B, H, sched_ws);
#define HSTU_FWD(DD, F8, G, BB) launch(hstu_fwd_kernel<DD, F8, G, BB>, FwdCfg<DD, F8>::LDS, grid, p, stream)
#define HSTU_FWD_B(DD, F8, G) (has_bias ? HSTU_FWD(DD, F8, G, true) : HSTU_FWD(DD, F8, G, false))
  const bool has_bias = attn_bias != nullptr;
  if (pv_scale > 0.f) {
    // FP8 P.V: P8 = e4m3(P' s); pv_c = 2^-3 f32(2^3 / s) is f32(1 / s) up to
    // its last bit, and makes P' s the product the reference's cast divides
    // by 2^-3 (hstu_fwd.py pv_s)
    p.pv_c = (float)(8.0f / pv_scale) * 0.125f;
    p.pv_out = 1.0f / pv_scale;
    e = has_bias ? launch(hstu_fwd_pv8_kernel<true>, Pv8Cfg::lds(max_seq_len), grid, p, stream)
                 : launch(hstu_fwd_pv8_kernel<false>, Pv8Cfg::lds(max_seq_len), grid, p, stream);
  } else if (dtype == HSTU_DTYPE_FP8_E4M3) {
    e = generic ? HSTU_FWD_B(128, true, true) : HSTU_FWD_B(128, true, false);
  } else if (D == 128) {
    e = generic ? HSTU_FWD_B(128, false, true) : HSTU_FWD_B(128, false, false);
  } else {
    e = generic ? HSTU_FWD_B(64, false, true) : HSTU_FWD_B(64, false, false);
  }
#undef HSTU_FWD_B
#undef HSTU_FWD
  if (e != hipSuccess) return (int)e;
  return (int)hipGetLastError();
}
}  // namespace

extern "C" int hstu_attn_fwd(int dtype, const void* q, const void* k, const void* v, int64_t q_row_stride,
                             int64_t k_row_stride, int64_t v_row_stride, const float* q_scale,
                             const float* k_scale, const float* v_scale, int64_t scale_row_stride,
                             int64_t scale_head_stride, const int64_t* seq_offsets, int B, int H, int D,
                             int max_seq_len, float alpha, const int32_t* num_targets, int max_attn_len,
                             int contextual_seq_len, const float* attn_bias, int bias_R, void* out,
                             int64_t out_row_stride, void* workspace, int64_t workspace_bytes,
                             int64_t total_tokens, hipStream_t stream) {
  const int c = fwd_check(dtype, q, k, v, q_row_stride, k_row_stride, v_row_stride, q_scale, k_scale, v_scale, B, H,
                          D, max_seq_len, attn_bias, bias_R, total_tokens);
  if (c != 0) return c;
  if (B == 0) return 0;
  if (workspace == nullptr || workspace_bytes < fwd_workspace_bytes(B, H)) return HSTU_E_BAD_ARG;
  return fwd_launch(dtype, q, k, v, q_row_stride, k_row_stride, v_row_stride, q_scale, k_scale, v_scale,
                    scale_row_stride, scale_head_stride, seq_offsets, B, H, D, max_seq_len, alpha, num_targets,
                    max_attn_len, contextual_seq_len, attn_bias, bias_R, out, out_row_stride, (int*)workspace,
                    stream);
}

extern "C" int hstu_attn_fwd_fp8_pv_max_seq_len(void) {
  int n = 64;
  while (Pv8Cfg::lds(n + 64) <= kMaxLdsBytes) n += 64;
  return n;
}

extern "C" int hstu_attn_fwd_fp8_pv(const void* q, const void* k, const void* v, int64_t q_row_stride,
                                    int64_t k_row_stride, int64_t v_row_stride, const float* q_scale,
                                    const float* k_scale, const float* v_scale, int64_t scale_row_stride,
                                    int64_t scale_head_stride, const int64_t* seq_offsets, int B, int H, int D,
                                    int max_seq_len, float alpha, const int32_t* num_targets, int max_attn_len,
                                    int contextual_seq_len, const float* attn_bias, int bias_R, float pv_scale,
                                    void* out, int64_t out_row_stride, void* workspace, int64_t workspace_bytes,
                                    int64_t total_tokens, hipStream_t stream) {
  const int c = fwd_check(HSTU_DTYPE_FP8_E4M3, q, k, v, q_row_stride, k_row_stride, v_row_stride, q_scale, k_scale,
                          v_scale, B, H, D, max_seq_len, attn_bias, bias_R, total_tokens);
  if (c != 0) return c;
  if (!(pv_scale > 0.f) || !(pv_scale < 448.f)) return HSTU_E_BAD_ARG;
  // the causal mask only (the reference arms FP8 P.V on its causal config)
  if (num_targets != nullptr || max_attn_len > 0 || contextual_seq_len > 0) return HSTU_E_UNSUPPORTED;
  // the block's per-key table grows with N: refused before any launch past
  // the CU's 160 KiB of LDS
  if (max_seq_len > hstu_attn_fwd_fp8_pv_max_seq_len()) return HSTU_E_UNSUPPORTED;
  if (B == 0) return 0;
  if (workspace == nullptr || workspace_bytes < fwd_workspace_bytes(B, H)) return HSTU_E_BAD_ARG;
  return fwd_launch(HSTU_DTYPE_FP8_E4M3, q, k, v, q_row_stride, k_row_stride, v_row_stride, q_scale, k_scale,
                    v_scale, scale_row_stride, scale_head_stride, seq_offsets, B, H, D, max_seq_len, alpha, nullptr, 0,
                    0, attn_bias, bias_R, out, out_row_stride, (int*)workspace, stream, pv_scale);
}

// ---------------------------------------------------------------------------
// Allocation-free forward.  The block schedule goes to `scratch`, a
// file-scope device array of HSTU_ATTN_FWD_NOALLOC_SCRATCH_BYTES that every
// GPU the library runs on holds until the process ends.  Host code never
// passes the array's name to a kernel (on the host it is only a stand-in):
// the device address comes from hipGetSymbolAddress, looked up once per
// device on the first call made with that device current, and kept per
// device.  Every call on a GPU shares that GPU's array; the schedule kernel
// writes every entry the attention kernel then reads, so nothing needs
// clearing, and calls that overlap on one GPU (other streams) race.
// ---------------------------------------------------------------------------
static_assert(HSTU_ATTN_FWD_NOALLOC_SCRATCH_BYTES % 256 == 0, "scratch size");
static __device__ __align__(256) uint8_t scratch[HSTU_ATTN_FWD_NOALLOC_SCRATCH_BYTES];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_addr[kMaxDevices] = {};

// The current device's address of `scratch` (looked up on first use).
hipError_t scratch_address(void** addr) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_addr[dev] == nullptr) {
    void* a = nullptr;
    e = hipGetSymbolAddress(&a, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    if (a == nullptr) return hipErrorInvalidSymbol;
    g_scratch_addr[dev] = a;
  }
  *addr = g_scratch_addr[dev];
  return hipSuccess;
}
}  // namespace

extern "C" int hstu_attn_fwd_noalloc(int dtype, const void* q, const void* k, const void* v, int64_t q_row_stride,
                                     int64_t k_row_stride, int64_t v_row_stride, const float* q_scale,
                                     const float* k_scale, const float* v_scale, int64_t scale_row_stride,
                                     int64_t scale_head_stride, const int64_t* seq_offsets, int B, int H, int D,
                                     int max_seq_len, float alpha, const int32_t* num_targets, int max_attn_len,
                                     int contextual_seq_len, const float* attn_bias, int bias_R, void* out,
                                     int64_t out_row_stride, int64_t total_tokens, hipStream_t stream) {
  const int c = fwd_check(dtype, q, k, v, q_row_stride, k_row_stride, v_row_stride, q_scale, k_scale, v_scale, B, H,
                          D, max_seq_len, attn_bias, bias_R, total_tokens);
  if (c != 0) return c;
  if (B == 0) return 0;
  if (fwd_workspace_bytes(B, H) > HSTU_ATTN_FWD_NOALLOC_SCRATCH_BYTES) return HSTU_E_SCRATCH_TOO_SMALL;
  void* ws = nullptr;
  const hipError_t e = scratch_address(&ws);
  if (e != hipSuccess) return (int)e;
  return fwd_launch(dtype, q, k, v, q_row_stride, k_row_stride, v_row_stride, q_scale, k_scale, v_scale,
                    scale_row_stride, scale_head_stride, seq_offsets, B, H, D, max_seq_len, alpha, num_targets,
                    max_attn_len, contextual_seq_len, attn_bias, bias_R, out, out_row_stride, (int*)ws, stream);
}

namespace {
enum BwdParts { kBwdDkdv = 1, kBwdDq = 2, kBwdAll = 3 };

int attn_bwd_impl(int parts, int dtype, const void* dout, int64_t dout_row_stride, const void* q, const void* k,
                  const void* v, int64_t q_row_stride, int64_t k_row_stride, int64_t v_row_stride,
                  const float* q_scale, const float* k_scale, const float* v_scale, int64_t scale_row_stride,
                  int64_t scale_head_stride, const int64_t* seq_offsets, int B, int H, int D, int max_seq_len,
                  float alpha, const int32_t* num_targets, int max_attn_len, int contextual_seq_len,
                  const float* attn_bias, int bias_R, void* dq, void* dk, void* dv, int64_t dq_row_stride,
                  int64_t dk_row_stride, int64_t dv_row_stride, float* dbias, void* workspace,
                  int64_t workspace_bytes, int64_t total_tokens, hipStream_t stream) {
  if (!check_common(dtype, H, D, B, max_seq_len, q_row_stride, k_row_stride, v_row_stride, q_scale, k_scale,
                    v_scale, bias_R, attn_bias) ||
      (dbias != nullptr && attn_bias == nullptr))
    return HSTU_E_BAD_ARG;
  if (!(D == 128 || (D == 64 && dtype == HSTU_DTYPE_BF16))) return HSTU_E_UNSUPPORTED;
  if (!row_alignment_ok(dtype, q_row_stride, q) || !row_alignment_ok(dtype, k_row_stride, k) ||
      !row_alignment_ok(dtype, v_row_stride, v) || !row_alignment_ok(HSTU_DTYPE_BF16, dout_row_stride, dout))
    return HSTU_E_UNSUPPORTED;
  if (((parts & kBwdDq) && (dq == nullptr || dq_row_stride < (int64_t)H * D)) ||
      ((parts & kBwdDkdv) && (dk == nullptr || dv == nullptr || dk_row_stride < (int64_t)H * D ||
                              dv_row_stride < (int64_t)H * D)))
    return HSTU_E_BAD_ARG;
  if (B == 0) return 0;
  AttnParams p{};
  p.q = (const uint8_t*)q;
  p.k = (const uint8_t*)k;
  p.v = (const uint8_t*)v;
  p.dout = (const uint8_t*)dout;
  p.q_rs = q_row_stride;
  p.k_rs = k_row_stride;
  p.v_rs = v_row_stride;
  p.do_rs = dout_row_stride;
  p.q_scale = q_scale;
  p.k_scale = k_scale;
  p.v_scale = v_scale;
  p.s_rs = scale_row_stride;
  p.s_hs = scale_head_stride;
  p.seq_offsets = seq_offsets;
  p.num_targets = num_targets;
  p.dq = (uint16_t*)dq;
  p.dk = (uint16_t*)dk;
  p.dv = (uint16_t*)dv;
  p.dq_rs = dq_row_stride;
  p.dk_rs = dk_row_stride;
  p.dv_rs = dv_row_stride;
  p.B = B;
  p.H = H;
  p.N = max_seq_len;
  p.alpha = alpha;
  p.inv_n = 1.0f / (float)max_seq_len;
  p.max_attn_len = max_attn_len;
  p.contextual_seq_len = contextual_seq_len;
  p.blocks_per_seq = (max_seq_len + 127) / 128;
  const bool generic = num_targets != nullptr || max_attn_len > 0 || contextual_seq_len > 0;
  const int grid = sched_grid(B, H, max_seq_len);
  p.bias = attn_bias;
  p.bias_R = bias_R;
  p.dbias = dbias;
  const bool has_bias = attn_bias != nullptr;
  hipError_t e;
  const BwdWs wl = bwd_ws(dtype, total_tokens, B, H, D, max_seq_len, has_bias ? bias_R : 0);
  if (total_tokens < 0 || workspace_bytes < wl.total || workspace == nullptr) return HSTU_E_BAD_ARG;
  // the dQ kernels' per-wave bias-gradient histograms must fit the CU's LDS
  if (has_bias && (parts & kBwdDq)) {
    const int lds = generic ? (D == 128 ? DqCfg<128>::lds(true, bias_R) : DqCfg<64>::lds(true, bias_R))
                            : (D == 128 ? DqWsCfg<128>::lds(true, bias_R) : DqWsCfg<64>::lds(true, bias_R));
    if (lds > kMaxLdsBytes) return HSTU_E_UNSUPPORTED;
  }
  uint8_t* ws = (uint8_t*)workspace;
  // the block schedule, the pre-clamped bias rows (dK/dV) and the rows past
  // max_seq_len of this half's outputs zeroed, in one launch
  PrepArgs pa = prep_args(seq_offsets, B, H, max_seq_len);
  pa.sched = (int*)(ws + wl.sched);
  if ((parts & kBwdDkdv) && has_bias) {
    pa.bias = attn_bias;
    pa.R = bias_R;
    pa.bias_ext = (float*)(ws + wl.bias_ext);
    pa.bias_bx = (bias_ext_len(max_seq_len) + 1023) / 1024;
  }
  pa.width = H * D;
  pa.z[0] = (parts & kBwdDq) ? p.dq : p.dk;
  pa.zrs[0] = (parts & kBwdDq) ? p.dq_rs : p.dk_rs;
  pa.z[1] = (parts & kBwdDkdv) ? p.dk : (uint16_t*)nullptr;
  pa.zrs[1] = p.dk_rs;
  pa.z[2] = (parts & kBwdDkdv) ? p.dv : (uint16_t*)nullptr;
  pa.zrs[2] = p.dv_rs;
  e = launch_prep(pa, stream);
  if (e != hipSuccess) return (int)e;
  use_schedule(p, B, H, (int*)(ws + wl.sched));
  if (!generic) {
    // dS tiles pass from the dK/dV kernel to the dQ kernel through the workspace
    p.ds_base = (const int64_t*)(ws + wl.ds_base);
    p.ds_ws = ws + wl.ds;
    hipLaunchKernelGGL(ds_tile_prefix, dim3(1), dim3(1024), 0, stream, seq_offsets, B, max_seq_len,
                       (int64_t*)(ws + wl.ds_base), has_bias ? (int64_t*)(ws + wl.dq_base) : (int64_t*)nullptr);
  }
  if (parts & kBwdDkdv) {
    if (has_bias) p.bias_ext = (const float*)(ws + wl.bias_ext);
    if (dtype == HSTU_DTYPE_FP8_E4M3) {
      p.q16 = ws + wl.q16;
      hipLaunchKernelGGL(convert_q8_bf16, dim3(1024), dim3(256), 0, stream, (const uint8_t*)q, q_row_stride,
                         seq_offsets, B, H, D, (uint16_t*)p.q16);
    }
    // dK / dV: 128-key blocks, longest query range first.
#define HSTU_DKV(DD, F8, G, BB) launch(hstu_bwd_dkdv_kernel<DD, F8, G, BB>, DkvCfg<DD, F8, BB>::LDS, grid, p, stream)
#define HSTU_DKV_B(DD, F8, G) (has_bias ? HSTU_DKV(DD, F8, G, true) : HSTU_DKV(DD, F8, G, false))
    if (dtype == HSTU_DTYPE_FP8_E4M3) {
      e = generic ? HSTU_DKV_B(128, true, true) : HSTU_DKV_B(128, true, false);
    } else if (D == 128) {
      e = generic ? HSTU_DKV_B(128, false, true) : HSTU_DKV_B(128, false, false);
    } else {
      e = generic ? HSTU_DKV_B(64, false, true) : HSTU_DKV_B(64, false, false);
    }
#undef HSTU_DKV_B
#undef HSTU_DKV
    if (e != hipSuccess) return (int)e;
  }
  if (parts & kBwdDq) {
    if (has_bias) {
      // one bias-gradient row per dQ block: offsets 0 .. R-1, or -(R-1) .. R-1
      // for the masks that admit keys after the query
      p.dbias_part = (float*)(ws + wl.part);
      p.dq_base = (const int64_t*)(ws + wl.dq_base);
      p.dbias_w = generic ? 2 * bias_R - 1 : bias_R;
      if (generic)
        hipLaunchKernelGGL(dq_block_prefix, dim3(1), dim3(1024), 0, stream, seq_offsets, B, max_seq_len,
                           (int64_t*)(ws + wl.dq_base));
    }
    // dQ (+ bias gradient): 128-query blocks, longest key range first.  With
    // the causal mask, from the dS tiles the dK/dV kernel stored.
    if (!generic) {
#define HSTU_DQW(DD, F8, BB) launch(hstu_bwd_dq_ws_kernel<DD, F8, BB>, DqWsCfg<DD>::lds(BB, bias_R), grid, p, stream)
      if (dtype == HSTU_DTYPE_FP8_E4M3) e = has_bias ? HSTU_DQW(128, true, true) : HSTU_DQW(128, true, false);
      else if (D == 128) e = has_bias ? HSTU_DQW(128, false, true) : HSTU_DQW(128, false, false);
      else e = has_bias ? HSTU_DQW(64, false, true) : HSTU_DQW(64, false, false);
#undef HSTU_DQW
    } else {
    const int lds = DqCfg<128>::lds(has_bias, bias_R);
    const int lds64 = DqCfg<64>::lds(has_bias, bias_R);
#define HSTU_DQ(DD, F8, G, BB) launch(hstu_bwd_dq_kernel<DD, F8, G, BB>, DD == 128 ? lds : lds64, grid, p, stream)
#define HSTU_DQ_B(DD, F8, G) (has_bias ? HSTU_DQ(DD, F8, G, true) : HSTU_DQ(DD, F8, G, false))
    if (dtype == HSTU_DTYPE_FP8_E4M3) {
      e = generic ? HSTU_DQ_B(128, true, true) : HSTU_DQ_B(128, true, false);
    } else if (D == 128) {
      e = generic ? HSTU_DQ_B(128, false, true) : HSTU_DQ_B(128, false, false);
    } else {
      e = generic ? HSTU_DQ_B(64, false, true) : HSTU_DQ_B(64, false, false);
    }
#undef HSTU_DQ_B
#undef HSTU_DQ
    }
    if (e != hipSuccess) return (int)e;
    if (has_bias && dbias != nullptr) {
      e = dbias_reduce(p, (float*)(ws + wl.chunks), p.inv_n, dbias, stream);
      if (e != hipSuccess) return (int)e;
    }
  }
  return (int)hipGetLastError();
}
}  // namespace

#define HSTU_BWD_ARGS                                                                                        \
  dtype, dout, dout_row_stride, q, k, v, q_row_stride, k_row_stride, v_row_stride, q_scale, k_scale, v_scale, \
      scale_row_stride, scale_head_stride, seq_offsets, B, H, D, max_seq_len, alpha, num_targets,             \
      max_attn_len, contextual_seq_len, attn_bias, bias_R, dq, dk, dv, dq_row_stride, dk_row_stride,          \
      dv_row_stride, dbias, workspace, workspace_bytes, total_tokens, stream
#define HSTU_BWD_PARAMS                                                                                        \
  int dtype, const void *dout, int64_t dout_row_stride, const void *q, const void *k, const void *v,           \
      int64_t q_row_stride, int64_t k_row_stride, int64_t v_row_stride, const float *q_scale,                 \
      const float *k_scale, const float *v_scale, int64_t scale_row_stride, int64_t scale_head_stride,        \
      const int64_t *seq_offsets, int B, int H, int D, int max_seq_len, float alpha,                          \
      const int32_t *num_targets, int max_attn_len, int contextual_seq_len, const float *attn_bias,           \
      int bias_R, void *dq, void *dk, void *dv, int64_t dq_row_stride, int64_t dk_row_stride,                 \
      int64_t dv_row_stride, float *dbias, void *workspace, int64_t workspace_bytes, int64_t total_tokens,        \
      hipStream_t stream

extern "C" int64_t hstu_attn_bwd_workspace_bytes(int dtype, int64_t total_tokens, int B, int H, int D,
                                                 int max_seq_len, int bias_R) {
  if (B < 0 || H <= 0 || total_tokens < 0) return -1;
  return bwd_ws(dtype, total_tokens, B, H, D, max_seq_len, bias_R).total;
}

extern "C" int64_t hstu_attn_fwd_workspace_bytes(int dtype, int64_t total_tokens, int B, int H, int D,
                                                 int max_seq_len) {
  (void)dtype;
  (void)D;
  if (B < 0 || H <= 0 || total_tokens < 0 || max_seq_len < 0) return -1;
  return fwd_workspace_bytes(B, H);
}
extern "C" int hstu_attn_bwd(HSTU_BWD_PARAMS) { return attn_bwd_impl(kBwdAll, HSTU_BWD_ARGS); }
extern "C" int hstu_attn_bwd_dkdv(HSTU_BWD_PARAMS) { return attn_bwd_impl(kBwdDkdv, HSTU_BWD_ARGS); }
extern "C" int hstu_attn_bwd_dq(HSTU_BWD_PARAMS) { return attn_bwd_impl(kBwdDq, HSTU_BWD_ARGS); }

// ---------------------------------------------------------------------------
// Full-FP8 backward entry point.
// ---------------------------------------------------------------------------
namespace {
// Workspace: [block schedule][pre-clamped bias rows][partial bias gradients]
// [scale maxima][dS tile prefix][e4m3 dS tiles].  The tiles are sized by a
// bound that needs no lengths: sum_b nq_b (nq_b + 1) / 2 <= (nq_max + 1) / 2 *
// (ceil(T / 128) + B), nq_max = ceil(N / 128).
struct F8Ws {
  int64_t sched, bias_ext, part, chunks, dq_base, maxv, base, tiles, total;
};
int64_t f8_tiles_bound(int64_t T, int B, int N) {
  const int64_t nq = (N + 127) / 128;
  return ((nq + 1) * ((T + 127) / 128 + B) + 1) / 2;
}
F8Ws f8_ws(int64_t T, int B, int H, int N, int R) {
  F8Ws w;
  int64_t o = 0;
  w.sched = o;
  o += sched_bytes(B, H);
  w.bias_ext = o;
  if (R > 0) o += bias_ext_bytes(H, N);
  w.part = o;
  if (R > 0) o += dbias_rows_bytes(T, B, H, R);
  w.chunks = o;
  if (R > 0) o += dbias_chunks_bytes(H, R);
  w.dq_base = o;
  o += align256(((int64_t)B + 1) * 8);
  w.maxv = o;
  o += align256(kScaleParts * 2 * 4);
  w.base = o;
  o += align256(((int64_t)B + 1) * 8);
  w.tiles = o;
  o += f8_tiles_bound(T, B, N) * H * F8Bwd::TILE;
  w.total = o;
  return w;
}
int ceil_log2(int n) {
  int c = 0;
  while ((1 << c) < n) ++c;
  return c;
}
}  // namespace

extern "C" int64_t hstu_attn_bwd_fp8_workspace_bytes(int64_t total_tokens, int B, int H, int D, int max_seq_len,
                                                     int bias_R) {
  if (B < 0 || H <= 0 || D != 128 || total_tokens < 0 || max_seq_len <= 0 || bias_R < 0) return -1;
  return f8_ws(total_tokens, B, H, max_seq_len, bias_R).total;
}

namespace {
int attn_bwd_fp8_impl(int parts, const void* dout8, const void* dout_e8, int64_t dout_row_stride, const void* q,
                      const void* k, const void* v, int64_t q_row_stride, int64_t k_row_stride,
                      int64_t v_row_stride, const float* q_scale, const float* k_scale, const float* v_scale,
                      int64_t scale_row_stride, int64_t scale_head_stride, const int64_t* seq_offsets, int B,
                      int H, int D, int max_seq_len, float alpha, int p8_scale_log2, int ds8_scale_log2,
                      const float* attn_bias, int bias_R, void* dq,
                      void* dk, void* dv, int64_t dq_row_stride, int64_t dk_row_stride, int64_t dv_row_stride,
                      float* dbias, void* workspace, int64_t workspace_bytes, int64_t total_tokens,
                      hipStream_t stream) {
  if (!check_common(HSTU_DTYPE_FP8_E4M3, H, D, B, max_seq_len, q_row_stride, k_row_stride, v_row_stride, q_scale,
                    k_scale, v_scale, bias_R, attn_bias) ||
      (dbias != nullptr && attn_bias == nullptr) || dout8 == nullptr || dout_e8 == nullptr ||
      dout_row_stride < (int64_t)H * D || total_tokens < 0 ||
      ((parts & kBwdDq) && (dq == nullptr || dq_row_stride < (int64_t)H * D)) ||
      ((parts & kBwdDkdv) && (dk == nullptr || dv == nullptr || dk_row_stride < (int64_t)H * D ||
                              dv_row_stride < (int64_t)H * D)))
    return HSTU_E_BAD_ARG;
  if (D != 128) return HSTU_E_UNSUPPORTED;
  if (!row_alignment_ok(HSTU_DTYPE_FP8_E4M3, q_row_stride, q) || !row_alignment_ok(HSTU_DTYPE_FP8_E4M3, k_row_stride, k) ||
      !row_alignment_ok(HSTU_DTYPE_FP8_E4M3, v_row_stride, v) ||
      !row_alignment_ok(HSTU_DTYPE_FP8_E4M3, dout_row_stride, dout8) ||
      ((parts & kBwdDq) && !row_alignment_ok(HSTU_DTYPE_BF16, dq_row_stride, dq)) ||
      ((parts & kBwdDkdv) && (!row_alignment_ok(HSTU_DTYPE_BF16, dk_row_stride, dk) ||
                              !row_alignment_ok(HSTU_DTYPE_BF16, dv_row_stride, dv))))
    return HSTU_E_UNSUPPORTED;
  // silu * N >= -0.279 is clamped from above only, exact while the P
  // pre-scale stays <= 2^(ceil(log2 N) + 9) (hstu_flydsl_mha.py:1371-1374)
  if (p8_scale_log2 < -64 || p8_scale_log2 > 64 || ds8_scale_log2 < -64 || ds8_scale_log2 > 64 ||
      p8_scale_log2 > ceil_log2(max_seq_len < 2 ? 2 : max_seq_len) + 9)
    return HSTU_E_BAD_ARG;
  // the dQ kernel's per-wave bias-gradient histograms must fit the CU's LDS
  if (attn_bias != nullptr && F8Bwd::dq_lds(true, bias_R) > kMaxLdsBytes) return HSTU_E_UNSUPPORTED;
  if (B == 0) return 0;
  const bool has_bias = attn_bias != nullptr;
  const F8Ws wl = f8_ws(total_tokens, B, H, max_seq_len, has_bias ? bias_R : 0);
  if (workspace == nullptr || workspace_bytes < wl.total) return HSTU_E_BAD_ARG;
  uint8_t* ws = (uint8_t*)workspace;
  AttnParams p{};
  p.q = (const uint8_t*)q;
  p.k = (const uint8_t*)k;
  p.v = (const uint8_t*)v;
  p.do8 = (const uint8_t*)dout8;
  p.e8 = (const uint8_t*)dout_e8;
  p.q_rs = q_row_stride;
  p.k_rs = k_row_stride;
  p.v_rs = v_row_stride;
  p.do_rs = dout_row_stride;
  p.q_scale = q_scale;
  p.k_scale = k_scale;
  p.v_scale = v_scale;
  p.s_rs = scale_row_stride;
  p.s_hs = scale_head_stride;
  p.seq_offsets = seq_offsets;
  p.dq = (uint16_t*)dq;
  p.dk = (uint16_t*)dk;
  p.dv = (uint16_t*)dv;
  p.dq_rs = dq_row_stride;
  p.dk_rs = dk_row_stride;
  p.dv_rs = dv_row_stride;
  p.B = B;
  p.H = H;
  p.N = max_seq_len;
  p.alpha = alpha;
  p.inv_n = 1.0f / (float)max_seq_len;
  p.bias = attn_bias;
  p.bias_R = bias_R;
  p.dbias = dbias;
  // power-of-two pre-scales of the e4m3 P and dS (hstu_flydsl_mha.py:1351-1370:
  // 2^(ceil(log2 N) + K), K = 3 and -3 by default, -5 for dS in production)
  p.p8_scale = ldexpf(1.0f, p8_scale_log2);
  p.ds8_scale = ldexpf(1.0f, ds8_scale_log2);
  p.f8max = (const unsigned*)(ws + wl.maxv);
  p.ds_base = (const int64_t*)(ws + wl.base);
  p.ds_ws = ws + wl.tiles;
  const int grid = sched_grid(B, H, max_seq_len);
  // One launch for the set-up: with the dK/dV half, the block schedule, the
  // tile and dQ-block prefixes (and the scale-maximum reset) and the
  // pre-clamped bias rows, all read by both halves (the dQ half, which runs
  // after it on the same workspace, builds none of them); and the rows past
  // max_seq_len of this half's outputs zeroed.
  PrepArgs pa = prep_args(seq_offsets, B, H, max_seq_len);
  if (parts & kBwdDkdv) {
    pa.sched = (int*)(ws + wl.sched);
    pa.tile_base = (int64_t*)(ws + wl.base);
    pa.dq_base = (int64_t*)(ws + wl.dq_base);
    pa.f8max = (unsigned*)(ws + wl.maxv);
    const bool per_token = scale_row_stride || scale_head_stride;
    pa.qs = q_scale;
    pa.ks = k_scale;
    pa.ntok = per_token ? total_tokens : 1;
    pa.sH = per_token ? H : 1;
    pa.srs = scale_row_stride;
    pa.shs = scale_head_stride;
    if (has_bias) {
      pa.bias = attn_bias;
      pa.R = bias_R;
      pa.bias_ext = (float*)(ws + wl.bias_ext);
      pa.bias_bx = (bias_ext_len(max_seq_len) + 1023) / 1024;
    }
  }
  pa.width = H * D;
  pa.z[0] = (parts & kBwdDq) ? p.dq : p.dk;
  pa.zrs[0] = (parts & kBwdDq) ? p.dq_rs : p.dk_rs;
  pa.z[1] = (parts & kBwdDkdv) ? p.dk : (uint16_t*)nullptr;
  pa.zrs[1] = p.dk_rs;
  pa.z[2] = (parts & kBwdDkdv) ? p.dv : (uint16_t*)nullptr;
  pa.zrs[2] = p.dv_rs;
  hipError_t e = launch_prep(pa, stream);
  if (e != hipSuccess) return (int)e;
  use_schedule(p, B, H, (int*)(ws + wl.sched));
  if (parts & kBwdDkdv) {
    const bool per_token = scale_row_stride || scale_head_stride;
    if (has_bias) p.bias_ext = (const float*)(ws + wl.bias_ext);
    // one scale tensor for q and k (the same device address): the shared mode
    const int sm = per_token ? kScalesPerToken : (q_scale == k_scale ? kScalesShared : kScalesPerTensor);
#define HSTU_F8_DKDV(BB, SS) launch(hstu_bwd_f8_dkdv_kernel<BB, SS>, F8Bwd::LDS, 2 * grid, p, stream, F8Bwd::NT)
#define HSTU_F8_DKDV_B(SS) (has_bias ? HSTU_F8_DKDV(true, SS) : HSTU_F8_DKDV(false, SS))
    e = sm == kScalesPerToken ? HSTU_F8_DKDV_B(kScalesPerToken)
                              : (sm == kScalesShared ? HSTU_F8_DKDV_B(kScalesShared) : HSTU_F8_DKDV_B(kScalesPerTensor));
#undef HSTU_F8_DKDV_B
#undef HSTU_F8_DKDV
    if (e != hipSuccess) return (int)e;
  }
  if (parts & kBwdDq) {
    if (has_bias) {
      p.dbias_part = (float*)(ws + wl.part);
      p.dq_base = (const int64_t*)(ws + wl.dq_base);
      p.dbias_w = bias_R;
    }
    e = has_bias ? launch(hstu_bwd_f8_dq_kernel<true>, F8Bwd::dq_lds(true, bias_R), grid, p, stream)
                 : launch(hstu_bwd_f8_dq_kernel<false>, F8Bwd::dq_lds(false, 0), grid, p, stream);
    if (e != hipSuccess) return (int)e;
    if (has_bias && dbias != nullptr) {
      e = dbias_reduce(p, (float*)(ws + wl.chunks), 1.0f, dbias, stream);
      if (e != hipSuccess) return (int)e;
    }
  }
  return (int)hipGetLastError();
}
}  // namespace

#define HSTU_BWD_FP8_PARAMS                                                                                       \
  const void *dout8, const void *dout_e8, int64_t dout_row_stride, const void *q, const void *k, const void *v,  \
      int64_t q_row_stride, int64_t k_row_stride, int64_t v_row_stride, const float *q_scale,                    \
      const float *k_scale, const float *v_scale, int64_t scale_row_stride, int64_t scale_head_stride,           \
      const int64_t *seq_offsets, int B, int H, int D, int max_seq_len, float alpha, int p8_scale_log2,          \
      int ds8_scale_log2, const float *attn_bias, int bias_R, void *dq, void *dk, void *dv,                      \
      int64_t dq_row_stride, int64_t dk_row_stride,                                                              \
      int64_t dv_row_stride, float *dbias, void *workspace, int64_t workspace_bytes, int64_t total_tokens,       \
      hipStream_t stream
#define HSTU_BWD_FP8_ARGS                                                                                        \
  dout8, dout_e8, dout_row_stride, q, k, v, q_row_stride, k_row_stride, v_row_stride, q_scale, k_scale, v_scale, \
      scale_row_stride, scale_head_stride, seq_offsets, B, H, D, max_seq_len, alpha, p8_scale_log2,             \
      ds8_scale_log2, attn_bias, bias_R, dq, dk,                                                                 \
      dv, dq_row_stride, dk_row_stride, dv_row_stride, dbias, workspace, workspace_bytes, total_tokens, stream
extern "C" int hstu_attn_bwd_fp8(HSTU_BWD_FP8_PARAMS) { return attn_bwd_fp8_impl(kBwdAll, HSTU_BWD_FP8_ARGS); }
extern "C" int hstu_attn_bwd_fp8_dkdv(HSTU_BWD_FP8_PARAMS) { return attn_bwd_fp8_impl(kBwdDkdv, HSTU_BWD_FP8_ARGS); }
extern "C" int hstu_attn_bwd_fp8_dq(HSTU_BWD_FP8_PARAMS) { return attn_bwd_fp8_impl(kBwdDq, HSTU_BWD_FP8_ARGS); }
