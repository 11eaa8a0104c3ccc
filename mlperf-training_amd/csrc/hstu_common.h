// Shared gfx950 device primitives of the HSTU kernels (MFMA wrappers, buffer
// resources, transposed LDS reads, direct global->LDS tile loads).
#ifndef HSTU_COMMON_H_
#define HSTU_COMMON_H_

#include <hip/hip_runtime.h>
#include <utility>
#include <stdint.h>

namespace hstu {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
constexpr int kThreads = 256;

// ---------------------------------------------------------------- primitives
__device__ __forceinline__ f32x4 mfma_bf16(u32x4 a, u32x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                 __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}
// e4m3 x e4m3, K = 128, no block scaling (scale operands 0 select the plain
// v_mfma_f32_16x16x128_f8f6f4).
__device__ __forceinline__ f32x4 mfma_fp8(i32x8 a, i32x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 0, 0, 0, 0, 0, 0);
}
// e4m3 x e4m3, 32x32x64.  Lane l: row (A) / column (B) l % 32, K group
// l / 32 (32 bytes); byte j of group g pairs with byte j of group g of the
// other operand.  The accumulator: lane l, register r holds row
// 8 (r / 4) + 4 (l / 32) + r % 4, column l % 32 (probed on gfx950).
__device__ __forceinline__ f32x16 mfma32_fp8(i32x8 a, i32x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c, 0, 0, 0, 0, 0, 0);
}
// The same with E8M0 block scales: bytes 16 b .. 16 b + 15 of both K groups
// of row (column) i are scaled by 2^(byte - 127) of lane 32 b + i's sa (sb)
// (probed on gfx950).
__device__ __forceinline__ f32x16 mfma32_fp8_scaled(i32x8 a, i32x8 b, f32x16 c, int sa, int sb) {
  return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c, 0, 0, 0, sa, 0, sb);
}
// Outer product on the matrix cores (32x32x2 fp32 MFMA): element (i, j) is
// A(i, 0) B(0, j) + A(i, 1) B(1, j), lane l supplying A(l % 32, l / 32) as a
// and B(l / 32, l % 32) as b; it lands in register r of lane l with
// i = 8 (r / 4) + 4 (l / 32) + r % 4, j = l % 32.  A half-wave passing a = 0
// leaves the other half-wave's product, the correctly rounded fp32 product,
// bitwise equal to v_mul_f32 (probed on gfx950, 4.2e6 products).
__device__ __forceinline__ f32x16 mfma32_outer(float a, float b) {
  f32x16 z;
#pragma unroll
  for (int r = 0; r < 16; ++r) z[r] = 0.f;
  return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, z, 0, 0, 0);
}
__device__ __forceinline__ uint32_t pack_bf16(float lo, float hi) {
  f32x2 v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
}
__device__ __forceinline__ uint16_t to_bf16(float x) {
  return __builtin_bit_cast(uint16_t, (__bf16)x);
}
__device__ __forceinline__ u32x4 lds_ld128(const uint8_t* p) { return *(const u32x4*)p; }
__device__ __forceinline__ f32x4 lds_ldf4(const uint8_t* p) { return *(const f32x4*)p; }
__device__ __forceinline__ i32x8 cat8(u32x4 lo, u32x4 hi) {
  i32x8 r;
  r[0] = lo[0]; r[1] = lo[1]; r[2] = lo[2]; r[3] = lo[3];
  r[4] = hi[0]; r[5] = hi[1]; r[6] = hi[2]; r[7] = hi[3];
  return r;
}
__device__ __forceinline__ f32x4 zero4() { return f32x4{0.f, 0.f, 0.f, 0.f}; }

// Raw buffer access: 32-bit offsets from a per-(sequence, head) base, with
// hardware zero-fill beyond `bytes` (rows past the sequence end).
typedef __amdgpu_buffer_rsrc_t BufRsrc;
__device__ __forceinline__ BufRsrc make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ u32x4 buf_ld128(BufRsrc r, uint32_t voff, uint32_t soff) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0);
}
__device__ __forceinline__ u32x2 buf_ld64(BufRsrc r, uint32_t voff, uint32_t soff) {
  return __builtin_amdgcn_raw_buffer_load_b64(r, voff, soff, 0);
}
__device__ __forceinline__ float buf_ldf(BufRsrc r, uint32_t voff, uint32_t soff) {
  return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, 0));
}

// Buffer loads straight into LDS (gfx950 buffer_load_dword{,x4} ... lds):
// lane l of the wave writes its BYTES bytes at lds + BYTES * l (`lds` must be
// wave-uniform: it goes through M0); offsets past the range are written as
// zero.  The write lands asynchronously: wait with lds_dma_wait() before a
// barrier that publishes it.
template <int BYTES>
__device__ __forceinline__ void buf_to_lds(BufRsrc r, uint8_t* lds, uint32_t voff, uint32_t soff) {
  static_assert(BYTES == 4 || BYTES == 16, "LDS DMA of 4 or 16 bytes per lane");
  auto* l = (__attribute__((address_space(3))) void*)lds;
  if constexpr (BYTES == 16) __builtin_amdgcn_raw_ptr_buffer_load_lds(r, l, 16, voff, soff, 0, 0);
  else __builtin_amdgcn_raw_ptr_buffer_load_lds(r, l, 4, voff, soff, 0, 0);
}
// s_waitcnt vmcnt(0) (expcnt, lgkmcnt left at their maxima 7, 15) as a real
// instruction, so the compiler's own wait insertion counts it
__device__ __forceinline__ void lds_dma_wait() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// Transposed LDS read (gfx950 ds_read_b64_tr_b16).  Within each 16-lane
// group, lane j supplies the address of 4 consecutive bf16 M[j][0..3]; lane i
// receives M[4r + i/4][i%4] for r = 0..3.  With lane j pointing at row
// base + j/4, column 4*(j%4) of a row-major tile, lane i gets rows
// base..base+3 of column i: the B operand of an MFMA whose contraction runs
// along the rows.
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ u32x2 lds_tr16(const uint8_t* p) {
  typedef __attribute__((address_space(3))) bf16x4 lds_bf16x4;
  const lds_bf16x4* lp = (const lds_bf16x4*)(__attribute__((address_space(3))) const uint8_t*)(p);
  return __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)lp));
}
__device__ __forceinline__ u32x4 cat_tr(u32x2 a, u32x2 b) { return u32x4{a[0], a[1], b[0], b[1]}; }

// ds_read_b64_tr_b8: within a 16-lane group, lane i receives byte i % 8 of
// the 8-byte chunks addressed by lanes 2r + i / 8, r = 0..7.  With lane j
// addressing token row t0 + j / 2 at byte column c0 + 8 (j % 2), lane i gets
// column c0 + i of tokens t0 .. t0 + 7, one token per byte.
__device__ __forceinline__ u32x2 lds_tr8(const uint8_t* p) {
  typedef int v2i __attribute__((ext_vector_type(2)));
  typedef __attribute__((address_space(3))) v2i lds_v2i;
  const lds_v2i* lp = (const lds_v2i*)(__attribute__((address_space(3))) const uint8_t*)(p);
  return __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_v2i*)lp));
}

// e4m3 x e4m3, K = 128, with E8M0 block scales: the K-block b (K indices
// 32b .. 32b+31) of row i of A is scaled by 2^(byte - 127) of lane 16b + i's
// sa, and of column j of B by lane 16b + j's sb (byte 0 of each).  A lane
// (row i, group g) supplies K indices 16g .. 16g+15 (bytes 0-15) and
// 64 + 16g .. 64 + 16g + 15 (bytes 16-31), so block b covers the low halves
// of groups 2b, 2b+1 (b < 2) or the high halves of groups 2b-4, 2b-3.
__device__ __forceinline__ f32x4 mfma_fp8_scaled(i32x8 a, i32x8 b, f32x4 c, int sa, int sb) {
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 0, 0, 0, sa, 0, sb);
}

// MODE.FP16_OVFL (MODE bit 23) of the wave.  Set, v_cvt_pk_fp8_f32 turns
// every finite input beyond the e4m3 range into +-448 instead of NaN -- the
// same byte as a clamp to +-448 followed by the conversion (probed on gfx950
// over in-range, boundary, 1e30 and 3.39e38 inputs; +-inf and NaN still give
// NaN) -- so a kernel whose values are finite can drop its clamps.  It also
// makes v_cvt_pk_bf16_f32 return +-bf16 max instead of +-inf above that
// range, so kernels clear it before their bf16 outputs.
__device__ __forceinline__ void fp8_saturate_mode(bool on) {
  if (on) asm volatile("s_setreg_imm32_b32 hwreg(HW_REG_MODE, 23, 1), 1\n\ts_nop 7\n\ts_nop 7" ::: "memory");
  else asm volatile("s_setreg_imm32_b32 hwreg(HW_REG_MODE, 23, 1), 0\n\ts_nop 7\n\ts_nop 7" ::: "memory");
}

// Four floats -> four e4m3 bytes (RNE).  By default the conversion does not
// saturate (out-of-range values become NaN): callers clamp to +-448 first or
// run under fp8_saturate_mode(true).
__device__ __forceinline__ uint32_t pack_fp8x4(float a, float b, float c, float d) {
  // the first conversion writes the low half and keeps the high half of its
  // old operand, which the second one overwrites: a's own register will do
  // (no copy when a dies here)
  int w = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, __builtin_bit_cast(int, a), false);
  return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(c, d, w, true);
}

// two e4m3 bytes (low or high half of w) -> two bf16, exact (scale 1.0)
template <bool HI>
__device__ __forceinline__ uint32_t cvt_fp8x2_bf16(uint32_t w) {
  return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8((int)w, 1.0f, HI));
}

// t = -x*log2(e)  ->  t * sigmoid(x) = t / (1 + 2^t)   (== -silu(x)/ln2)
__device__ __forceinline__ float sig_of_t(float t) {
  return __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(t));
}

// Exponent argument t = -x*log2(e) of a score: raw MFMA dot product s times
// the row factor c1 (-alpha*log2(e), times one operand's e4m3 scale) and the
// other operand's scale c2 (e4m3 only), plus the pre-scaled bias b.
template <bool FP8, bool BIAS>
__device__ __forceinline__ float scaled_score(float s, float c1, float c2, float b) {
  const float a = s * c1;
  if constexpr (FP8 && BIAS) return __builtin_fmaf(a, c2, b);
  else if constexpr (FP8) return a * c2;
  else if constexpr (BIAS) return a + b;
  else return a;
}

// silu'(x) in terms of sg = sigmoid(x) and p = t * sg, where t = -x*log2(e):
//   silu'(x) = sg + x*sg*(1 - sg) = sg + p*(ln2*sg - ln2)   (x*sg = -ln2 * p)
__device__ __forceinline__ float dsilu_factor(float sg, float p) {
  return __builtin_fmaf(p, __builtin_fmaf(sg, kLn2, -kLn2), sg);
}
// dS before the 1/N factor: dP * silu'(x), from t = -x*log2(e).
__device__ __forceinline__ float dsilu_dp(float t, float dp) {
  const float sg = sig_of_t(t);
  return dp * dsilu_factor(sg, t * sg);
}

// 4 e4m3 bytes of a word -> 4 floats scaled by s, as 2 packed bf16 words.
__device__ __forceinline__ u32x2 fp8x4_to_bf16x4(uint32_t w, float s) {
  f32x2 lo = __builtin_amdgcn_cvt_pk_f32_fp8((int)w, false);
  f32x2 hi = __builtin_amdgcn_cvt_pk_f32_fp8((int)w, true);
  return u32x2{pack_bf16(lo[0] * s, lo[1] * s), pack_bf16(hi[0] * s, hi[1] * s)};
}

// Key order inside a transposed LDS tile.  The S^T C fragment of key
// sub-tiles 2c and 2c+1 gives lane group g the keys {32c+4g+r, 32c+16+4g+r};
// storing key 32c+16h+4g+r at column 32c+8g+4h+r makes those eight keys one
// contiguous 16-byte run, in register order.
__device__ __forceinline__ int sigma(int kk) {
  return (kk & ~31) | (((kk >> 2) & 3) << 3) | (((kk >> 4) & 1) << 2) | (kk & 3);
}


// Global -> LDS tile copy without registers (buffer_load_dwordx4 ... lds).
// One wave instruction writes 64 consecutive 16-byte LDS slots, so the tile's
// padded rows are laid out as PITCH/16 slots per row and lane l of
// instruction i fills slot 64i+l: a data slot loads its (row, chunk), a pad
// slot reloads a data chunk of the same row (never read).  Rows beyond the
// buffer's end read as zero.  Completion is tracked by vmcnt: wait_vm() then a
// barrier before the tile is read.
template <int ROWS, int ROW_BYTES, int PITCH>
struct DirectTile {
  static_assert(PITCH % 16 == 0 && ROW_BYTES % 16 == 0 && PITCH - ROW_BYTES <= ROW_BYTES, "layout");
  static constexpr int CPR = PITCH / 16, DATA_CPR = ROW_BYTES / 16;
  static constexpr int NINSTR = (ROWS * CPR + 63) / 64;
  static constexpr int BYTES = NINSTR * 1024;  // LDS footprint, >= ROWS * PITCH
  static constexpr int PER_WAVE = (NINSTR + kThreads / 64 - 1) / (kThreads / 64);
  uint32_t voff[PER_WAVE];
  __device__ __forceinline__ void init(uint32_t rs_bytes) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
#pragma unroll
    for (int j = 0; j < PER_WAVE; ++j) {
      const int c = (wave + 4 * j) * 64 + lane;
      int row = c / CPR, col = c - (c / CPR) * CPR;
      if (col >= DATA_CPR) col -= DATA_CPR;
      row = row < ROWS ? row : ROWS - 1;
      voff[j] = row * rs_bytes + col * 16;
    }
  }
  __device__ __forceinline__ void load(BufRsrc rs, uint32_t soff, uint8_t* tile) const {
    // Device pass only: the host pass cannot form the LDS address-space
    // pointer, and a failed host instantiation would drop the kernel's
    // launch stub.
#if defined(__HIP_DEVICE_COMPILE__)
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
#pragma unroll
    for (int j = 0; j < PER_WAVE; ++j) {
      const int i = wave + 4 * j;
      if (i < NINSTR)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (__attribute__((address_space(3))) void*)(tile + i * 1024), 16,
                                                 voff[j], soff, 0, 0);
    }
#else
    (void)rs;
    (void)soff;
    (void)tile;
#endif
  }
};
// f(std::integral_constant<int, 0>{}) ... f(std::integral_constant<int, N-1>{})
template <int N, typename F, int... I>
__device__ __forceinline__ void static_for_impl(F&& f, std::integer_sequence<int, I...>) {
  (f(std::integral_constant<int, I>{}), ...);
}
template <int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  static_for_impl<N>(f, std::make_integer_sequence<int, N>{});
}

// ---------------------------------------------------------------- mask
struct MaskCtx {
  int L, nt, ctx, max_attn;
  bool targets;
};
// _get_valid_attn_mask (ops/pytorch/pt_hstu_attention.py:32-84), per element.
__device__ __forceinline__ bool valid_generic(int i, int j, const MaskCtx& m) {
  int max_ids = m.L, ii = i, jj = j;
  if (m.ctx > 0) {
    ii = max(i - m.ctx + 1, 0);
    jj = max(j - m.ctx + 1, 0);
    max_ids = m.L - m.ctx + 1;
  }
  if (m.targets) {
    max_ids -= m.nt;
    ii = min(ii, max_ids);
    jj = min(jj, max_ids);
  }
  const int dist = ii - jj;
  bool v = (i == j) || (dist > 0);
  if (m.max_attn > 0) v = v && (dist <= m.max_attn);
  if (m.ctx > 0) v = v || (ii == 0 && jj < max_ids);
  return v && j < m.L && i < m.L;
}

// vmcnt(0); expcnt and lgkmcnt left at their maxima.
__device__ __forceinline__ void wait_vm() { __builtin_amdgcn_s_waitcnt(0x0F70); }


}  // namespace hstu

#endif  // HSTU_COMMON_H_
