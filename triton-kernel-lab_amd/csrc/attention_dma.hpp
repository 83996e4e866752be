// Device helpers shared by the buffer->LDS DMA attention kernels (attention_fwd.hip,
// attention_bwd.hip): MFMA wrappers on raw 32-bit fragments, accumulator packing,
// explicit wait counters, and LDS reads as inline asm (the compiler would wait for
// every outstanding LDS DMA before each compiler-visible LDS read).
#pragma once
#include "tk_common.hpp"

namespace tk_attn {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x2 __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) void lds_void;

constexpr float kNegInf = -INFINITY;
template <typename T>
struct Mma;
template <>
struct Mma<_Float16> {
  static __device__ __forceinline__ f32x16 run(i32x4 a, i32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
};
template <>
struct Mma<__bf16> {
  static __device__ __forceinline__ f32x16 run(i32x4 a, i32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
};

// Registers 8g .. 8g+7 of an accumulator rounded (RNE) to T: an MFMA operand.
template <typename T>
__device__ __forceinline__ i32x4 acc_frag(const f32x16& acc, int g) {
  const f32x8 v = {acc[g * 8 + 0], acc[g * 8 + 1], acc[g * 8 + 2], acc[g * 8 + 3],
                   acc[g * 8 + 4], acc[g * 8 + 5], acc[g * 8 + 6], acc[g * 8 + 7]};
  if constexpr (__is_same(T, __bf16))
    return __builtin_bit_cast(i32x4, __builtin_convertvector(v, bf16x8));
  else
    return __builtin_bit_cast(i32x4, __builtin_convertvector(v, f16x8));
}

template <typename T>
__device__ __forceinline__ uint32_t pack2(float lo, float hi) {
  const uint16_t a = __builtin_bit_cast(uint16_t, tk::from_f32<T>(lo));
  const uint16_t b = __builtin_bit_cast(uint16_t, tk::from_f32<T>(hi));
  return uint32_t(a) | (uint32_t(b) << 16);
}

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
  // s_waitcnt fields: vmcnt[3:0], expcnt[6:4] (7 = no wait), lgkmcnt[11:8] (15 = no
  // wait), vmcnt[5:4] at [15:14].
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

template <int N>
__device__ __forceinline__ void wait_lgkm() {
  asm volatile("s_waitcnt lgkmcnt(%0)" ::"i"(N) : "memory");
}

// Keeps every use of an LDS-read result below the preceding wait (volatile asm
// statements stay in program order; this one redefines the value).
__device__ __forceinline__ void pin(i32x4& f) { asm volatile("" : "+v"(f)); }

// Barrier without __syncthreads()'s fence, which would wait for every outstanding DMA.
__device__ __forceinline__ void barrier_no_fence() { asm volatile("s_barrier" ::: "memory"); }

template <int OFF>
__device__ __forceinline__ i32x4 lds_read_b128(uint32_t addr) {
  i32x4 r;
  asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(r) : "v"(addr), "i"(OFF));
  return r;
}

template <int OFF>
__device__ __forceinline__ i32x2 lds_read_tr16(uint32_t addr) {
  i32x2 r;
  asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(r) : "v"(addr), "i"(OFF));
  return r;
}

// V^T fragment for 16 keys starting at row ROW0 of the stage's V tile: rows ROW0 .. +3
// (k-index 0..3 of this lane half) and ROW0 + 8 .. +11 (k-index 4..7).
template <int ROW0, int RB>
__device__ __forceinline__ i32x4 read_v(uint32_t addr) {
  const i32x2 a = lds_read_tr16<ROW0 * RB>(addr);
  const i32x2 b = lds_read_tr16<(ROW0 + 8) * RB>(addr);
  return i32x4{a[0], a[1], b[0], b[1]};
}

// Lane maximum over itself and lane ^ 32 (the swap returns both values, in either order).
__device__ __forceinline__ float max_with_partner(float x) {
  const auto pr = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x),
                                                   false, false);
  return fmaxf(__uint_as_float(pr[0]), __uint_as_float(pr[1]));
}

__device__ __forceinline__ float sum_with_partner(float x) {
  const auto pr = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x),
                                                   false, false);
  return __uint_as_float(pr[0]) + __uint_as_float(pr[1]);
}

}  // namespace tk_attn
