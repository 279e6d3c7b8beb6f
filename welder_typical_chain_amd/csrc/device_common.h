// device_common.h -- device-side helpers shared by the gfx950 chain kernels
// (fused_matmul_softmax.hip, rowblock_softmax.hip, wide_tile.hip): vector types, buffer
// descriptors and loads, direct-to-LDS loads with hand-counted waits, the
// LDS transpose read, output packing and wave reductions.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "tile_layout.h"

namespace wtc {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
constexpr uint32_t kOutOfRange = 0x80000000u;  // buffer offset that reads 0
// cache-policy operand of the buffer builtins on gfx950: the nt bit
constexpr int kCachePolicyNT = 2;
// The split path's first pass stores exp2(y - tile max) (in [0, 1]) for
// the rescale pass to scale in place: in the output type, except that a
// bf16 output keeps them in f16 (the same 2 bytes, 2^-11 instead of 2^-8
// rounding), so that the output is rounded to bf16 only once, by the
// rescale pass.  Those f16 values are stored times 2^15 (exact), so that
// exponentials down to 2^-29 keep f16's full precision and only those
// below 2^-39 flush to zero; the rescale factor carries the 2^-15 back.
constexpr int split_store_dt(int out_dt) { return out_dt == DT_BF16 ? DT_F16 : out_dt; }
constexpr float split_store_scale(int out_dt) { return out_dt == DT_BF16 ? 32768.0f : 1.0f; }
template <int OUT_DT> struct OutTraits;
template <> struct OutTraits<DT_F32> { static constexpr int SZ = 4; };
template <> struct OutTraits<DT_F16> { static constexpr int SZ = 2; };
template <> struct OutTraits<DT_BF16> { static constexpr int SZ = 2; };
__device__ inline __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                           0x00020000);
}
__device__ inline u32x4 bload16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0));
}
__device__ inline u32x2 bload8(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(r, (int)off, 0, 0));
}

typedef int i32x4 __attribute__((ext_vector_type(4)));
#define WTC_LDS __attribute__((address_space(3)))

// Raw buffer descriptor: base, stride 0, num_records = bytes, gfx9 dword3.
__device__ inline i32x4 raw_rsrc(const void* base, uint32_t bytes) {
  const uint64_t a = reinterpret_cast<uint64_t>(base);
  i32x4 r;
  r[0] = (int)(uint32_t)a;
  r[1] = (int)((uint32_t)(a >> 32) & 0xFFFFu);
  r[2] = (int)bytes;
  r[3] = 0x00020000;
  return r;
}

// 16 bytes per lane into LDS at lds_base + 16*lane.  The descriptor and the
// LDS base are wave-uniform; readfirstlane states that to the compiler so
// the "s" operands always get scalar registers (free when they already are).
__device__ inline void dma16(i32x4 rsrc, uint32_t voff, uint32_t lds_base) {
  i32x4 r;
#pragma unroll
  for (int i = 0; i < 4; ++i) r[i] = __builtin_amdgcn_readfirstlane(rsrc[i]);
  const uint32_t m = __builtin_amdgcn_readfirstlane(lds_base);
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
               :
               : "s"(m), "v"(voff), "s"(r)
               : "memory", "m0");
}

// Wait until at most N of this wave's direct-to-LDS loads are in flight and
// its LDS reads are done, then meet the other waves.
template <int N>
__device__ inline void wait_loads_barrier() {
  asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" : : "n"(N) : "memory");
}

typedef __fp16 h4 __attribute__((__vector_size__(4 * sizeof(__fp16))));

typedef int i32x2 __attribute__((ext_vector_type(2)));
// ds_read_b64_tr_b8: see tile_layout.h (btr8_k / btr8_n) for the lane mapping.
__device__ inline u32x2 tr8_read(const uint8_t* p) {
  return __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr8_b64_v2i32((WTC_LDS i32x2*)(p)));
}

__device__ inline u32x2 tr_read(const uint8_t* p) {
  const h4 v = __builtin_amdgcn_ds_read_tr16_b64_v4f16((WTC_LDS h4*)(p));
  return __builtin_bit_cast(u32x2, v);
}

// -------------------------------------------------------------------------
// Output conversion: four f32 -> two 32-bit words of f16 / bf16 (RNE).  A
// two-element vector conversion selects gfx950's packed converts
// (v_cvt_pk_f16_f32 / v_cvt_pk_bf16_f32: one instruction per word instead
// of two converts and an or); the whole vector is bit cast, never an element.
// -------------------------------------------------------------------------
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
template <int OUT_DT> __device__ inline void pack4(const f32x4& x, uint32_t* w0, uint32_t* w1);
template <> __device__ inline void pack4<DT_F16>(const f32x4& x, uint32_t* w0, uint32_t* w1) {
  const f16x2 lo = __builtin_convertvector(f32x2{x[0], x[1]}, f16x2);
  const f16x2 hi = __builtin_convertvector(f32x2{x[2], x[3]}, f16x2);
  *w0 = __builtin_bit_cast(uint32_t, lo);
  *w1 = __builtin_bit_cast(uint32_t, hi);
}
template <> __device__ inline void pack4<DT_BF16>(const f32x4& x, uint32_t* w0, uint32_t* w1) {
  const bf16x2 lo = __builtin_convertvector(f32x2{x[0], x[1]}, bf16x2);
  const bf16x2 hi = __builtin_convertvector(f32x2{x[2], x[3]}, bf16x2);
  *w0 = __builtin_bit_cast(uint32_t, lo);
  *w1 = __builtin_bit_cast(uint32_t, hi);
}

// Four f32 values times f -> two words of the output type.  f16: scalar
// conversions of the products, which the compiler fuses into v_fma_mixlo_f16
// (one rounding of the exact product to f16, where a f32 multiply followed
// by a packed convert would round twice); bf16: packed converts of the
// products.
template <int OUT_DT> __device__ inline void pack4_product(const f32x4& x, float f, uint32_t* w0, uint32_t* w1);
template <> __device__ inline void pack4_product<DT_F16>(const f32x4& x, float f, uint32_t* w0, uint32_t* w1) {
  const float x0 = x[0] * f, x1 = x[1] * f, x2 = x[2] * f, x3 = x[3] * f;
  *w0 = (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)x0) |
        ((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)x1) << 16);
  *w1 = (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)x2) |
        ((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)x3) << 16);
}
template <> __device__ inline void pack4_product<DT_BF16>(const f32x4& x, float f, uint32_t* w0, uint32_t* w1) {
  pack4<DT_BF16>(x * f, w0, w1);
}

__device__ inline float wave_xor32_max(float x) { return fmaxf(x, __shfl_xor(x, 32)); }

// Value of lane quad_perm(CTRL) of this lane's quad (DPP quad permute, no LDS
// round trip): 0xB1 swaps lanes 0<->1 and 2<->3 (xor 1), 0x4E swaps the
// pairs (xor 2).  Every lane of the wave must be active.
template <int CTRL>
__device__ inline float dpp_quad(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), CTRL, 0xF, 0xF, true));
}
__device__ inline float wave_xor32_sum(float x) { return x + __shfl_xor(x, 32); }

// The same reductions with the lane 32 apart in registers: v_permlane32_swap
// of x with itself leaves x[l % 32] in word 0 and x[l % 32 + 32] in word 1
// of every lane l, so both halves combine the pair in the same operand
// order (bit-identical results) without an LDS round trip.  The words are
// copied to scalars before the bit cast.
__device__ inline void xor32_pair(float x, float* lo, float* hi) {
  const uint32_t u = __builtin_bit_cast(uint32_t, x);
  const auto q = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  const uint32_t a = q[0], b = q[1];
  *lo = __builtin_bit_cast(float, a);
  *hi = __builtin_bit_cast(float, b);
}
__device__ inline float xor32_max(float x) {
  float a, b;
  xor32_pair(x, &a, &b);
  return fmaxf(a, b);
}
__device__ inline float xor32_min(float x) {
  float a, b;
  xor32_pair(x, &a, &b);
  return fminf(a, b);
}
__device__ inline float xor32_sum(float x) {
  float a, b;
  xor32_pair(x, &a, &b);
  return a + b;
}

// 64-bit relaxed atomic access at agent scope for the split path's per-tile
// row statistics (max, sumexp): one store, so a reader never sees half of it.
__device__ inline void store_stat(float2* p, float m, float s) {
  const uint64_t u = (uint64_t)__builtin_bit_cast(uint32_t, m) |
                     ((uint64_t)__builtin_bit_cast(uint32_t, s) << 32);
  __hip_atomic_store(reinterpret_cast<uint64_t*>(p), u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace wtc
