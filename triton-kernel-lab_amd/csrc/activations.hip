// Pointwise kernels outside the transformer hot path that complete the
// registry: strided vector add, and ReLU / exact GELU / SiLU / tanh with their
// derivatives (src/tklab/kernels/vector_add.py:17-34,
// src/tklab/kernels/activations.py:60-136). Float32 math, one rounding to the
// storage dtype per output, products rounded separately.
#include "tk_common.hpp"

#pragma clang fp contract(off)

namespace {

constexpr int kBlock = 256;

enum Activation { kRelu = 0, kGelu = 1, kSilu = 2, kTanh = 3 };

using tk::stable_sigmoid;

template <int ACT>
__device__ __forceinline__ float act_value(float x) {
  if constexpr (ACT == kRelu) return fmaxf(x, 0.f);
  if constexpr (ACT == kGelu) return 0.5f * x * (1.0f + erff(x * 0.7071067811865476f));
  if constexpr (ACT == kSilu) return x * stable_sigmoid(x);
  return 2.0f * stable_sigmoid(2.0f * x) - 1.0f;  // tanh through the sigmoid identity
}

template <int ACT>
__device__ __forceinline__ float act_grad(float x) {
  if constexpr (ACT == kRelu) return x > 0.f ? 1.0f : 0.0f;
  if constexpr (ACT == kGelu) {
    const float cdf = 0.5f * (1.0f + erff(x * 0.7071067811865476f));
    const float pdf = 0.3989422804014327f * expf(-0.5f * x * x);
    return cdf + x * pdf;
  }
  if constexpr (ACT == kSilu) {
    const float s = stable_sigmoid(x);
    return s * (1.0f + x * (1.0f - s));
  }
  const float t = 2.0f * stable_sigmoid(2.0f * x) - 1.0f;
  return 1.0f - t * t;
}

inline unsigned grid_for(int64_t chunks) {
  int64_t blocks = tk::cdiv(chunks, kBlock);
  if (blocks > 256 * 64) blocks = 256 * 64;
  return static_cast<unsigned>(blocks);
}

template <typename T>
__global__ __launch_bounds__(kBlock) void vector_add_kernel(const T* __restrict__ x,
                                                            const T* __restrict__ y,
                                                            T* __restrict__ out, int64_t n,
                                                            int64_t xs, int64_t ys, int64_t os) {
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x; i < n;
       i += static_cast<int64_t>(gridDim.x) * kBlock)
    out[i * os] = tk::from_f32<T>(tk::to_f32(x[i * xs]) + tk::to_f32(y[i * ys]));
}

template <typename T, int VEC>
__global__ __launch_bounds__(kBlock) void vector_add_vec_kernel(const T* __restrict__ x,
                                                                const T* __restrict__ y,
                                                                T* __restrict__ out, int64_t chunks) {
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x; i < chunks;
       i += static_cast<int64_t>(gridDim.x) * kBlock) {
    float a[VEC], b[VEC];
    tk::load_vec<T, VEC>(x + i * VEC, a);
    tk::load_vec<T, VEC>(y + i * VEC, b);
#pragma unroll
    for (int j = 0; j < VEC; ++j) a[j] += b[j];
    tk::store_vec<T, VEC>(out + i * VEC, a);
  }
}

template <typename T, int VEC, int ACT>
__global__ __launch_bounds__(kBlock) void act_fwd_kernel(const T* __restrict__ x, T* __restrict__ y,
                                                         int chunks, tk::FastDiv per_row,
                                                         int64_t xs, int64_t ys) {
  for (int i = blockIdx.x * kBlock + threadIdx.x; i < chunks; i += gridDim.x * kBlock) {
    const int row = per_row.div(i);
    const int c = (i - row * static_cast<int>(per_row.d)) * VEC;
    float v[VEC];
    tk::load_vec<T, VEC>(x + row * xs + c, v);
#pragma unroll
    for (int j = 0; j < VEC; ++j) v[j] = act_value<ACT>(v[j]);
    tk::store_vec<T, VEC>(y + row * ys + c, v);
  }
}

template <typename T, int VEC, int ACT>
__global__ __launch_bounds__(kBlock) void act_bwd_kernel(const T* __restrict__ dy,
                                                         const T* __restrict__ x,
                                                         T* __restrict__ dx, int chunks,
                                                         tk::FastDiv per_row, int64_t dys,
                                                         int64_t xs, int64_t dxs) {
  for (int i = blockIdx.x * kBlock + threadIdx.x; i < chunks; i += gridDim.x * kBlock) {
    const int row = per_row.div(i);
    const int c = (i - row * static_cast<int>(per_row.d)) * VEC;
    float g[VEC], v[VEC];
    tk::load_vec<T, VEC>(dy + row * dys + c, g);
    tk::load_vec<T, VEC>(x + row * xs + c, v);
#pragma unroll
    for (int j = 0; j < VEC; ++j) g[j] = g[j] * act_grad<ACT>(v[j]);
    tk::store_vec<T, VEC>(dx + row * dxs + c, g);
  }
}

bool rows_vector_ok(int dtype, int64_t cols, std::initializer_list<const void*> ptrs,
                    std::initializer_list<int64_t> strides) {
  const int es = tk::elem_size(dtype);
  if (cols % (16 / es) != 0) return false;
  for (const void* p : ptrs)
    if (!tk::aligned16(p)) return false;
  for (int64_t s : strides)
    if ((s * es) % 16 != 0) return false;
  return true;
}

}  // namespace

#define TK_DISPATCH_ACT(kind, ACT, ...)                                        \
  switch (kind) {                                                              \
    case kRelu: { constexpr int ACT = kRelu; __VA_ARGS__; break; }             \
    case kGelu: { constexpr int ACT = kGelu; __VA_ARGS__; break; }             \
    case kSilu: { constexpr int ACT = kSilu; __VA_ARGS__; break; }             \
    case kTanh: { constexpr int ACT = kTanh; __VA_ARGS__; break; }             \
    default: return tk::fail("activation: unknown kind %d", kind);             \
  }

extern "C" int tk_vector_add(int dtype, const void* x, const void* y, void* out, int64_t n,
                             int64_t x_stride, int64_t y_stride, int64_t out_stride,
                             void* stream) {
  if (!tk::valid_dtype(dtype)) return tk::fail("vector_add: unsupported dtype code %d", dtype);
  if (x == nullptr || y == nullptr || out == nullptr) return tk::fail("vector_add: null pointer");
  if (n <= 0) return tk::fail("vector_add: empty problem");
  if (!tk::row_strides_ok(n, 1, {x_stride, y_stride, out_stride}))
    return tk::fail("vector_add: strides must be non-negative and keep rows in range");
  hipStream_t s = tk::as_stream(stream);
  const int vec = 16 / tk::elem_size(dtype);
  const bool vok = x_stride == 1 && y_stride == 1 && out_stride == 1 && n % vec == 0 &&
                   tk::aligned16(x) && tk::aligned16(y) && tk::aligned16(out);
  TK_DISPATCH_DTYPE(dtype, T,
    if (vok) {
      constexpr int VEC = 16 / int(sizeof(T));
      hipLaunchKernelGGL((vector_add_vec_kernel<T, VEC>), dim3(grid_for(n / VEC)), dim3(kBlock), 0,
                         s, (const T*)x, (const T*)y, (T*)out, n / VEC);
    } else {
      hipLaunchKernelGGL((vector_add_kernel<T>), dim3(grid_for(n)), dim3(kBlock), 0, s,
                         (const T*)x, (const T*)y, (T*)out, n, x_stride, y_stride, out_stride);
    });
  return tk::check_launch("vector_add");
}

extern "C" int tk_activation_fwd(int dtype, int kind, const void* x, void* y, int64_t rows,
                                 int64_t cols, int64_t x_row_stride, int64_t y_row_stride,
                                 void* stream) {
  if (!tk::valid_dtype(dtype)) return tk::fail("activation_fwd: unsupported dtype code %d", dtype);
  if (x == nullptr || y == nullptr) return tk::fail("activation_fwd: null pointer");
  if (rows <= 0 || cols <= 0) return tk::fail("activation_fwd: empty problem");
  if (!tk::row_strides_ok(rows, cols, {x_row_stride, y_row_stride}))
    return tk::fail("activation_fwd: strides must be non-negative and keep rows in range");
  if (x_row_stride == cols && y_row_stride == cols) {
    cols = tk::folded_extent(rows, cols);
    rows = 1;
    if (cols < 0) return tk::fail("activation_fwd: problem too large");
  }
  const bool vok = rows_vector_ok(dtype, cols, {x, y}, {x_row_stride, y_row_stride});
  const int64_t vec = vok ? 16 / tk::elem_size(dtype) : 1;
  int64_t chunks;
  if (__builtin_mul_overflow(rows, cols / vec, &chunks) || chunks > INT32_MAX - 64 * kBlock * 256)
    return tk::fail("activation_fwd: problem too large");
  const tk::FastDiv div(static_cast<uint32_t>(cols / vec));
  hipStream_t s = tk::as_stream(stream);
  TK_DISPATCH_DTYPE(dtype, T,
    TK_DISPATCH_VEC(T, vok,
      TK_DISPATCH_ACT(kind, ACT,
        hipLaunchKernelGGL((act_fwd_kernel<T, VEC, ACT>), dim3(grid_for(chunks)), dim3(kBlock), 0,
                           s, (const T*)x, (T*)y, (int)chunks, div, x_row_stride, y_row_stride))));
  return tk::check_launch("activation_fwd");
}

extern "C" int tk_activation_bwd(int dtype, int kind, const void* dy, const void* x, void* dx,
                                 int64_t rows, int64_t cols, int64_t dy_row_stride,
                                 int64_t x_row_stride, int64_t dx_row_stride, void* stream) {
  if (!tk::valid_dtype(dtype)) return tk::fail("activation_bwd: unsupported dtype code %d", dtype);
  if (dy == nullptr || x == nullptr || dx == nullptr) return tk::fail("activation_bwd: null pointer");
  if (rows <= 0 || cols <= 0) return tk::fail("activation_bwd: empty problem");
  if (!tk::row_strides_ok(rows, cols, {dy_row_stride, x_row_stride, dx_row_stride}))
    return tk::fail("activation_bwd: strides must be non-negative and keep rows in range");
  if (dy_row_stride == cols && x_row_stride == cols && dx_row_stride == cols) {
    cols = tk::folded_extent(rows, cols);
    rows = 1;
    if (cols < 0) return tk::fail("activation_bwd: problem too large");
  }
  const bool vok =
      rows_vector_ok(dtype, cols, {dy, x, dx}, {dy_row_stride, x_row_stride, dx_row_stride});
  const int64_t vec = vok ? 16 / tk::elem_size(dtype) : 1;
  int64_t chunks;
  if (__builtin_mul_overflow(rows, cols / vec, &chunks) || chunks > INT32_MAX - 64 * kBlock * 256)
    return tk::fail("activation_bwd: problem too large");
  const tk::FastDiv div(static_cast<uint32_t>(cols / vec));
  hipStream_t s = tk::as_stream(stream);
  TK_DISPATCH_DTYPE(dtype, T,
    TK_DISPATCH_VEC(T, vok,
      TK_DISPATCH_ACT(kind, ACT,
        hipLaunchKernelGGL((act_bwd_kernel<T, VEC, ACT>), dim3(grid_for(chunks)), dim3(kBlock), 0,
                           s, (const T*)dy, (const T*)x, (T*)dx, (int)chunks, div, dy_row_stride,
                           x_row_stride, dx_row_stride))));
  return tk::check_launch("activation_bwd");
}
