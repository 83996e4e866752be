// Row-per-group building blocks shared by the softmax and RMSNorm kernels.
//
// A row of `cols` elements is owned by a group of RT threads (RT = 64: one
// wave; RT = 256 or 1024: several waves meeting in LDS). Each thread holds
// VALS elements of the row in registers, as VALS/VEC vectors of VEC
// contiguous elements: vector i of thread `lane` covers columns
// [(i*RT + lane)*VEC, +VEC). With VEC = 16/sizeof(T) every access is one
// 128-bit load or store and a wave touches 1 KiB of contiguous row per
// vector index; VEC = 1 is the fallback for rows whose base or stride is not
// 16-byte aligned or whose width is not a multiple of VEC.
#pragma once

#include "tk_common.hpp"

namespace tk {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef int i32x4 __attribute__((ext_vector_type(4)));

// Cache-policy bits of gfx950 buffer loads and stores (the aux operand: sc0 = 1,
// nt = 2, sc1 = 16). Rows streamed once are loaded non-temporally so they do not
// displace reusable lines in L2 and the 256 MiB last-level cache; measured on the
// residual-RMSNorm step (bf16 16384 x 4096), non-temporal loads plus these store
// policies took the forward from 5.2 to 5.8 TB/s and the backward stage 1 from 4.9
// to 5.3 TB/s run alone, and the forward+backward step from 4.6 to 5.3 TB/s.
constexpr int kCpolDefault = 0;
constexpr int kCpolStream = 2;  // nt
constexpr int kCpolSc1 = 16;    // sc1

template <typename T, int VEC, int RT, int VALS>
__device__ __forceinline__ void load_row(const T* __restrict__ row, int cols, int lane, float* v,
                                         float fill) {
  constexpr int ITEMS = VALS / VEC;
#pragma unroll
  for (int i = 0; i < ITEMS; ++i) {
    const int c = (i * RT + lane) * VEC;
    if (c < cols) {
      load_vec<T, VEC>(row + c, v + i * VEC);
    } else {
#pragma unroll
      for (int j = 0; j < VEC; ++j) v[i * VEC + j] = fill;
    }
  }
}

template <typename T, int VEC, int RT, int VALS>
__device__ __forceinline__ void store_row(T* __restrict__ row, int cols, int lane, const float* v) {
  constexpr int ITEMS = VALS / VEC;
#pragma unroll
  for (int i = 0; i < ITEMS; ++i) {
    const int c = (i * RT + lane) * VEC;
    if (c < cols) store_vec<T, VEC>(row + c, v + i * VEC);
  }
}

// Branch-free 16-byte row access through a buffer resource spanning the row, with
// cache policy CPOL; columns at or past `cols` load as `fill` and are not stored.
// `row` must be wave-uniform (see RawRow::load_buf).
template <typename T, int VEC, int RT, int VALS, int CPOL>
__device__ __forceinline__ void load_row_buf(const T* row, int cols, int lane, float* v,
                                             float fill) {
  static_assert(VEC * sizeof(T) == 16, "16-byte vectors only");
  constexpr int ITEMS = VALS / VEC;
  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<T*>(row), (short)0, uint32_t(cols) * uint32_t(sizeof(T)), 0x00020000);
#pragma unroll
  for (int i = 0; i < ITEMS; ++i) {
    const int c = (i * RT + lane) * VEC;
    const Vec<T, VEC> r = __builtin_bit_cast(
        Vec<T, VEC>, __builtin_amdgcn_raw_buffer_load_b128(rs, uint32_t(c * int(sizeof(T))), 0, CPOL));
#pragma unroll
    for (int j = 0; j < VEC; ++j) v[i * VEC + j] = c < cols ? to_f32(r.v[j]) : fill;
  }
}

template <typename T, int VEC, int RT, int VALS, int CPOL>
__device__ __forceinline__ void store_row_buf(T* row, int cols, int lane, const float* v) {
  static_assert(VEC * sizeof(T) == 16, "16-byte vectors only");
  constexpr int ITEMS = VALS / VEC;
  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
      row, (short)0, uint32_t(cols) * uint32_t(sizeof(T)), 0x00020000);
#pragma unroll
  for (int i = 0; i < ITEMS; ++i) {
    const int c = (i * RT + lane) * VEC;
    Vec<T, VEC> r;
#pragma unroll
    for (int j = 0; j < VEC; ++j) r.v[j] = from_f32<T>(v[i * VEC + j]);
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(i32x4, r), rs,
                                           uint32_t(c * int(sizeof(T))), 0, CPOL);
  }
}

// Column of element e (0 <= e < VALS) held by thread `lane`.
template <int VEC, int RT>
__device__ __forceinline__ int row_column(int e, int lane) {
  return ((e / VEC) * RT + lane) * VEC + (e % VEC);
}

// Bits of one storage element <-> float32.
template <typename T>
__device__ __forceinline__ float bits_to_f32(uint32_t b);
template <>
__device__ __forceinline__ float bits_to_f32<float>(uint32_t b) { return __uint_as_float(b); }
template <>
__device__ __forceinline__ float bits_to_f32<__bf16>(uint32_t b) { return __uint_as_float(b << 16); }
template <>
__device__ __forceinline__ float bits_to_f32<_Float16>(uint32_t b) {
  return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(b)));
}
template <typename T>
__device__ __forceinline__ uint32_t f32_to_bits(float f) {
  if constexpr (sizeof(T) == 4) {
    return __float_as_uint(f);
  } else {
    return __builtin_bit_cast(uint16_t, from_f32<T>(f));
  }
}

// A row held in registers as packed storage words (no float copy): 16-bit
// rows take half the registers of their float32 values. Element e of thread
// `lane` is column row_column<VEC, RT>(e, lane).
template <typename T, int VEC, int RT, int VALS>
struct RawRow {
  static constexpr int ITEMS = VALS / VEC;
  static constexpr int PER_WORD = 4 / int(sizeof(T));  // elements per 32-bit word
  static constexpr int WORDS_PER_VEC = (VEC + PER_WORD - 1) / PER_WORD;
  uint32_t w[ITEMS * WORDS_PER_VEC];

  __device__ __forceinline__ void load(const T* __restrict__ row, int cols, int lane) {
#pragma unroll
    for (int i = 0; i < ITEMS; ++i) {
      const int c = (i * RT + lane) * VEC;
      uint32_t* dst = w + i * WORDS_PER_VEC;
      if constexpr (VEC * sizeof(T) == 16) {
        const uint4 u = c < cols ? *reinterpret_cast<const uint4*>(row + c) : make_uint4(0, 0, 0, 0);
        dst[0] = u.x;
        dst[1] = u.y;
        dst[2] = u.z;
        dst[3] = u.w;
      } else {
        static_assert(VEC == 1, "scalar fallback");
        dst[0] = c < cols ? f32_to_bits<T>(to_f32(row[c])) : 0u;
      }
    }
  }
  // Branch-free 16-byte variants through a buffer resource whose extent is the row
  // (columns past `cols` read as zero and are not written), with cache policy CPOL
  // (kCpol*). `row` must be the same for every lane of a wave: a divergent base
  // makes the compiler wrap each access in a readfirstlane loop.
  template <int CPOL>
  __device__ __forceinline__ void load_buf(const T* row, int cols, int lane) {
    static_assert(VEC * sizeof(T) == 16, "16-byte vectors only");
    const __amdgpu_buffer_rsrc_t rs = row_rsrc(row, cols);
#pragma unroll
    for (int i = 0; i < ITEMS; ++i) {
      const u32x4 u = __builtin_bit_cast(
          u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, byte_offset(i, lane), 0, CPOL));
#pragma unroll
      for (int j = 0; j < 4; ++j) w[i * 4 + j] = u[j];
    }
  }
  template <int CPOL>
  __device__ __forceinline__ void store_buf(T* row, int cols, int lane) const {
    static_assert(VEC * sizeof(T) == 16, "16-byte vectors only");
    const __amdgpu_buffer_rsrc_t rs = row_rsrc(row, cols);
#pragma unroll
    for (int i = 0; i < ITEMS; ++i) {
      const u32x4 u = {w[i * 4 + 0], w[i * 4 + 1], w[i * 4 + 2], w[i * 4 + 3]};
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(i32x4, u), rs, byte_offset(i, lane),
                                             0, CPOL);
    }
  }
  __device__ __forceinline__ static __amdgpu_buffer_rsrc_t row_rsrc(const T* row, int cols) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<T*>(row), (short)0,
                                             uint32_t(cols) * uint32_t(sizeof(T)), 0x00020000);
  }
  __device__ __forceinline__ static uint32_t byte_offset(int i, int lane) {
    return uint32_t((i * RT + lane) * VEC * int(sizeof(T)));
  }

  __device__ __forceinline__ void store(T* __restrict__ row, int cols, int lane) const {
#pragma unroll
    for (int i = 0; i < ITEMS; ++i) {
      const int c = (i * RT + lane) * VEC;
      if (c >= cols) continue;
      const uint32_t* src = w + i * WORDS_PER_VEC;
      if constexpr (VEC * sizeof(T) == 16) {
        *reinterpret_cast<uint4*>(row + c) = make_uint4(src[0], src[1], src[2], src[3]);
      } else {
        row[c] = from_f32<T>(bits_to_f32<T>(src[0]));
      }
    }
  }
  __device__ __forceinline__ uint32_t bits(int e) const {
    if constexpr (VEC == 1 || PER_WORD == 1) {
      return w[e];
    } else {
      const uint32_t word = w[e / PER_WORD];
      return (e & 1) ? (word >> 16) : (word & 0xffffu);
    }
  }
  __device__ __forceinline__ float get(int e) const { return bits_to_f32<T>(bits(e)); }
  __device__ __forceinline__ void set(int e, float f) {
    const uint32_t b = f32_to_bits<T>(f);
    if constexpr (VEC == 1 || PER_WORD == 1) {
      w[e] = b;
    } else {
      uint32_t& word = w[e / PER_WORD];
      word = (e & 1) ? ((word & 0xffffu) | (b << 16)) : ((word & 0xffff0000u) | b);
    }
  }
};

// Launch shape for a row width: RT threads per row, VALS elements per thread.
struct RowShape {
  int rt;
  int vals;
};

// Smallest thread group (64, 256 or 1024 threads) that covers `cols` with at
// most `max_vals` register-resident elements per thread (VALS in {16, 32, 64}).
// Returns false when the row is wider than 1024 * max_vals.
inline bool pick_row_shape(int64_t cols, RowShape* shape, int max_vals = 64) {
  static const int kThreads[] = {64, 256, 1024};
  static const int kVals[] = {16, 32, 64};
  for (int rt : kThreads) {
    for (int vals : kVals) {
      if (vals <= max_vals && cols <= int64_t(rt) * vals) {
        *shape = {rt, vals};
        return true;
      }
    }
  }
  return false;
}

}  // namespace tk

// Expands `__VA_ARGS__` with constexpr RT and VALS bound to `shape`.
#define TK_DISPATCH_ROW_SHAPE(shape, ...)                                \
  switch ((shape).rt * 100 + (shape).vals) {                             \
    case 6416: { constexpr int RT = 64, VALS = 16; __VA_ARGS__; break; }      \
    case 6432: { constexpr int RT = 64, VALS = 32; __VA_ARGS__; break; }      \
    case 6464: { constexpr int RT = 64, VALS = 64; __VA_ARGS__; break; }      \
    case 25616: { constexpr int RT = 256, VALS = 16; __VA_ARGS__; break; }    \
    case 25632: { constexpr int RT = 256, VALS = 32; __VA_ARGS__; break; }    \
    case 25664: { constexpr int RT = 256, VALS = 64; __VA_ARGS__; break; }    \
    case 102416: { constexpr int RT = 1024, VALS = 16; __VA_ARGS__; break; }  \
    case 102432: { constexpr int RT = 1024, VALS = 32; __VA_ARGS__; break; }  \
    case 102464: { constexpr int RT = 1024, VALS = 64; __VA_ARGS__; break; }  \
    default: return tk::fail("internal: no row kernel for shape %d/%d", (shape).rt, (shape).vals); \
  }

