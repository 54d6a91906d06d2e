// Device helpers shared by the attention kernels of libloom_infer_hip.so
// (gfx950): BF16 storage conversions, 16-byte and range-limited raw buffer
// loads of NHD K/V rows, and wave-level primitives.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace loom_dev {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// half::bf16::from_f32: round to nearest even; a NaN keeps its sign and top
// payload bits with the quiet bit set ((bits >> 16) | 0x40).  gfx950's
// v_cvt_pk_bf16_f32 gives exactly these bits for every one of the 2^32 FP32
// inputs (checked exhaustively on MI355X against the integer form
// ((bits + 0x7fff + ((bits >> 16) & 1)) >> 16, NaN as above)); the integer
// form compiles to a branch per element, which costs more than the stores
// it feeds in the latency-bound kernels.
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t bf16x2_pack(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){lo, hi}, bf16x2_t));
}
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  return __builtin_bit_cast(uint16_t, (__bf16)f);
}

__device__ __forceinline__ u32x4 load16(const uint16_t *p) {
  return *reinterpret_cast<const u32x4 *>(p);
}

// K/V pages are read exactly once per kv-head: nontemporal loads keep them
// from displacing reusable lines in L2/MALL (measured on MI355X: a plain
// streaming read tops out near 6.2 TB/s, a nontemporal one near 6.9 TB/s).
#ifndef LOOM_DECODE_NT_K
#define LOOM_DECODE_NT_K 1
#endif
#ifndef LOOM_DECODE_NT_V
#define LOOM_DECODE_NT_V 1
#endif
// Raw buffer loads of one page's rows for one kv-head.  The resource covers
// exactly the valid rows of the page (none for a prefetch past the wave's last
// page), so rows beyond it return zero without touching memory: the pipeline's
// look-ahead and the tail of a request's last page cost no HBM traffic.
// Cache policy bit 1 is NT on gfx950.
template <bool NT>
__device__ __forceinline__ u32x4 load16_rows(__amdgpu_buffer_rsrc_t r, int byte_offset) {
  return __builtin_bit_cast(
      u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, byte_offset, 0, NT ? 2 : 0));
}

// `row_elems`: elements between consecutive token rows of one kv-head
// (Hkv * 128 in NHD storage, 128 in HND pages).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t page_rows_rsrc(const uint16_t *base,
                                                                int valid_rows, int row_elems) {
  // gfx9 word 3: 32-bit data format, no swizzle; stride 0 (raw addressing)
  const int bytes = valid_rows > 0 ? ((valid_rows - 1) * row_elems + 128) * 2 : 0;
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t *>(base), 0, bytes, 0x00020000);
}

// 16 bytes per lane from a buffer straight into LDS: lane i's bytes land at
// lds + 16 i (the LDS address is the same for every lane; offsets outside the
// buffer's range read as zeros).  Completion is counted by vmcnt and is NOT
// tracked by the compiler: the caller waits (wait_vmcnt) before the barrier
// that publishes the data.  (Issued as inline assembly so that the compiler
// does not wait for these loads before every later LDS access or barrier: it
// cannot tell the ring slot being filled from the one being read.)
// M0 (the LDS base of the load) is written here and declared clobbered; the
// kernels that use this keep nothing else in M0 (they use no LDS-DMA
// builtins or indexed register moves), so the compiler's note that it does
// not preserve reserved registers around the statement does not apply.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void lds_load16(__amdgpu_buffer_rsrc_t r, void *lds, int byte_offset) {
  const uint32_t m0 =
      __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(__attribute__((address_space(3))) void *)lds);
  asm volatile("s_mov_b32 m0, %1\n\tbuffer_load_dwordx4 %0, %2, 0 offen lds" ::"v"(byte_offset),
               "s"(m0), "s"(r)
               : "m0", "memory");
}
// The same with the LDS byte address given directly (wave-uniform), so a
// caller that keeps one LDS base address needs no generic-to-LDS pointer
// conversion per load.
__device__ __forceinline__ void lds_load16_at(__amdgpu_buffer_rsrc_t r, uint32_t lds_addr,
                                              int byte_offset) {
  const uint32_t m0 = __builtin_amdgcn_readfirstlane(lds_addr);
  asm volatile("s_mov_b32 m0, %1\n\tbuffer_load_dwordx4 %0, %2, 0 offen lds" ::"v"(byte_offset),
               "s"(m0), "s"(r)
               : "m0", "memory");
}
#pragma clang diagnostic pop

// Transposing 8-byte LDS read (ds_read_b64_tr_b16): within each 16 lanes,
// lane i receives element i % 4 of the four 16-bit elements addressed by
// lane 4k + i / 4, for k = 0..3.
__device__ __forceinline__ u32x2 lds_read_tr16(const void *lds) {
  typedef short s16x4 __attribute__((ext_vector_type(4)));
  typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
  const s16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4 *)(lds));
  return __builtin_bit_cast(u32x2, v);
}

// Transposing 8-byte LDS read of bytes (ds_read_b64_tr_b8): within each 16
// lanes, lane i receives as byte k (k = 0..7) byte i % 8 of the 8 bytes lane
// 2k + i / 8 addresses.
__device__ __forceinline__ u32x2 lds_read_tr8(const void *lds) {
  typedef int s32x2 __attribute__((ext_vector_type(2)));
  typedef __attribute__((address_space(3))) s32x2 lds_s32x2;
  const s32x2 v = __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_s32x2 *)(lds));
  return __builtin_bit_cast(u32x2, v);
}

// Waits until at most N vector memory loads of this wave are outstanding
// (lgkm and export counters not waited on).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 16, "vmcnt field");
  __builtin_amdgcn_s_waitcnt((0xF << 8) | (0x7 << 4) | N);
}

// 8-byte raw buffer load (FP8 rows: 8 elements per lane).
template <bool NT>
__device__ __forceinline__ u32x2 load8_rows(__amdgpu_buffer_rsrc_t r, int byte_offset) {
  return __builtin_bit_cast(
      u32x2, __builtin_amdgcn_raw_buffer_load_b64(r, byte_offset, 0, NT ? 2 : 0));
}

// FP8 E4M3 (OCP) storage.  Every E4M3 value is exact in BF16 (3 mantissa bits,
// exponents 2^-9 .. 2^8), so the decode conversion is lossless.
__device__ __forceinline__ u32x4 fp8x8_to_bf16x8(u32x2 w) {
  // gfx950's two-element E4M3 -> BF16 conversion with scale 1 (exact: every
  // E4M3 value is a BF16 value); half the instructions of widening through
  // FP32 and repacking.
  u32x4 o;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    o[2 * h] = __builtin_bit_cast(uint32_t,
                                  __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8((int)w[h], 1.0f, false));
    o[2 * h + 1] = __builtin_bit_cast(
        uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8((int)w[h], 1.0f, true));
  }
  return o;
}

// FP32 -> E4M3: finite values saturate to +-448, round to nearest even (the
// subnormal grid is m * 2^-9), NaN -> 0x7F.
__device__ __forceinline__ uint32_t fp8_e4m3_from_f32(float x) {
  const uint32_t u = __float_as_uint(x);
  const uint32_t s = (u >> 24) & 0x80u;
  const uint32_t au = u & 0x7fffffffu;
  if (au > 0x7f800000u) return 0x7Fu;
  const float a = __uint_as_float(au);
  if (a >= 448.0f) return s | 0x7Eu;
  if (a < 0.015625f) return s | (uint32_t)__builtin_rintf(a * 512.0f);
  int exp = (int)(au >> 23) - 127;
  uint32_t top = (au >> 20) & 7u;
  const uint32_t rem = au & 0xFFFFFu;
  top += (rem > 0x80000u || (rem == 0x80000u && (top & 1u))) ? 1u : 0u;
  if (top == 8u) {
    top = 0u;
    ++exp;
  }
  const uint32_t code = min((uint32_t)((exp + 7) << 3) | top, 0x7Eu);
  return s | code;
}

// OR of `p` over a workgroup of W waves with one barrier (HIP's
// __syncthreads_or takes three and an LDS atomic): each wave publishes its
// ballot in slots[wave].  `slots` belongs to one call site, and that site must
// not run twice without a barrier in between (a fast wave would overwrite a
// word that a slow one has yet to read).
template <int W>
__device__ __forceinline__ bool block_or(bool p, uint32_t (&slots)[W]) {
  const uint32_t any_lane = __builtin_amdgcn_ballot_w64(p) != 0 ? 1u : 0u;
  if ((threadIdx.x & 63) == 0) slots[threadIdx.x >> 6] = any_lane;
  __syncthreads();
  uint32_t any = 0;
#pragma unroll
  for (int i = 0; i < W; ++i) any |= slots[i];
  return any != 0;
}

__device__ __forceinline__ bf16x8 as_bf16x8(u32x4 v) { return __builtin_bit_cast(bf16x8, v); }

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

__device__ __forceinline__ void wave_lds_fence() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Wave-uniform values the compiler cannot prove uniform (loaded through the
// vector path): pin them to SGPRs.
__device__ __forceinline__ int uni(int x) { return __builtin_amdgcn_readfirstlane(x); }
__device__ __forceinline__ int64_t uni64(int64_t x) {
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)x);
  const int32_t hi = __builtin_amdgcn_readfirstlane((int)(x >> 32));
  return ((int64_t)hi << 32) | lo;
}

__device__ __forceinline__ int64_t shfl_up64(int64_t x, int o) {
  const int lo = __shfl_up((int)(uint32_t)x, o, 64);
  const int hi = __shfl_up((int)(x >> 32), o, 64);
  return ((int64_t)hi << 32) | (uint32_t)lo;
}

// Sum / max of an int over the wave (butterfly: every lane gets the result).
__device__ __forceinline__ int wave_sum_i32(int x) {
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) x += __shfl_xor(x, o, 64);
  return x;
}
__device__ __forceinline__ int wave_max_i32(int x) {
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) x = max(x, __shfl_xor(x, o, 64));
  return x;
}

__device__ __forceinline__ int64_t wave_incl_scan64(int64_t x, int lane) {
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int64_t y = shfl_up64(x, o);
    if (lane >= o) x += y;
  }
  return x;
}

typedef short s16x4 __attribute__((ext_vector_type(4)));

// Upper 16 bits of two floats packed into one register (lo <- a, hi <- b).
__device__ __forceinline__ uint32_t pack_hi16(uint32_t a, uint32_t b) {
  return __builtin_amdgcn_perm(b, a, 0x07060302u);
}
__device__ __forceinline__ uint32_t pack_lo16(uint32_t a, uint32_t b) {
  return __builtin_amdgcn_perm(b, a, 0x05040100u);
}
__device__ __forceinline__ s16x4 as_s16x4(uint32_t lo, uint32_t hi) {
  return __builtin_bit_cast(s16x4, u32x2{lo, hi});
}

// Max / sum over the four 16-lane rows of a wave (the lanes l, l^16, l^32,
// l^48 share a query column): v_permlane16_swap / v_permlane32_swap, no LDS.
__device__ __forceinline__ float quad_max(float x) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  x = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
// IEEE 754-2019 maximum (a NaN operand gives NaN): unlike fmaxf it needs no
// quieting of its inputs, and gfx950 takes three operands per instruction.
__device__ __forceinline__ float fmax_nan(float a, float b) {
  return __builtin_elementwise_maximum(a, b);
}
__device__ __forceinline__ float quad_max_nan(float x) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  x = fmax_nan(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  return fmax_nan(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ __forceinline__ float quad_sum(float x) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  x = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// Two 16-bit halves packed into bf16x8 operands: four registers, low halves
// first.
__device__ __forceinline__ bf16x8 as_bf16x8(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
  return __builtin_bit_cast(bf16x8, u32x4{a, b, c, d});
}

}  // namespace loom_dev
