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

// Column of element e (0 <= e < VALS) held by thread `lane`.
template <int VEC, int RT>
__device__ __forceinline__ int row_column(int e, int lane) {
  return ((e / VEC) * RT + lane) * VEC + (e % VEC);
}

// Launch shape for a row width: RT threads per row, VALS elements per thread.
struct RowShape {
  int rt;
  int vals;
};

// Smallest group that covers `cols` with at most 64 register-resident
// elements per thread: one wave up to 64*64 columns, 256 threads up to
// 16384, 1024 threads up to 65536. Returns false when the row is wider.
inline bool pick_row_shape(int64_t cols, RowShape* shape) {
  static const int kThreads[] = {64, 256, 1024};
  for (int rt : kThreads) {
    if (cols <= int64_t(rt) * 16) {
      *shape = {rt, 16};
      return true;
    }
    if (cols <= int64_t(rt) * 64) {
      *shape = {rt, 64};
      return true;
    }
  }
  return false;
}

}  // namespace tk

// Expands `__VA_ARGS__` with constexpr RT and VALS bound to `shape`.
#define TK_DISPATCH_ROW_SHAPE(shape, ...)                                \
  switch ((shape).rt * 100 + (shape).vals) {                             \
    case 6416: { constexpr int RT = 64, VALS = 16; __VA_ARGS__; break; }      \
    case 6464: { constexpr int RT = 64, VALS = 64; __VA_ARGS__; break; }      \
    case 25616: { constexpr int RT = 256, VALS = 16; __VA_ARGS__; break; }    \
    case 25664: { constexpr int RT = 256, VALS = 64; __VA_ARGS__; break; }    \
    case 102416: { constexpr int RT = 1024, VALS = 16; __VA_ARGS__; break; }  \
    case 102464: { constexpr int RT = 1024, VALS = 64; __VA_ARGS__; break; }  \
    default: return tk::fail("internal: no row kernel for shape %d/%d", (shape).rt, (shape).vals); \
  }

