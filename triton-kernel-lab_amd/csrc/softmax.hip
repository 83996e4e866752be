// Row-wise softmax, one row per thread group, the whole row in registers.
//
// Math follows the reference kernel (src/tklab/kernels/fused_softmax.py:32-39):
// float32 values, masked tail = -inf, shifted = x - rowmax, numerator = exp (here the
// hardware exp2 of shifted * log2(e)), y = numerator / rowsum (here numerator * (1/rowsum)),
// stored in the input dtype.
// One HBM read and one HBM write per element.
#include <algorithm>
#include <cstdlib>

#include "rows.hpp"

namespace {

// max, exponentials (tk::hw_exp, the hardware exp2 of x log2(e)), sum and scaling of one row
// held in registers, in place.
template <int RT, int VALS>
__device__ __forceinline__ void softmax_row(float* v, float* scratch) {
  float m = v[0];
#pragma unroll
  for (int e = 1; e < VALS; ++e) m = fmaxf(m, v[e]);
  m = tk::group_allreduce<RT>(m, tk::MaxOp{}, scratch);
  float s = 0.f;
#pragma unroll
  for (int e = 0; e < VALS; ++e) {
    v[e] = tk::hw_exp(v[e] - m);
    s += v[e];
  }
  s = tk::group_allreduce<RT>(s, tk::SumOp{}, scratch);
  const float inv = 1.0f / s;
#pragma unroll
  for (int e = 0; e < VALS; ++e) v[e] *= inv;
}

// P rows per thread group (P = 2 only for single-wave rows): every row's loads are issued
// first, so the exponentials and stores of a row overlap the loads of the next. On f32
// 4096 x 4096 (one wave per row, all waves resident in one round) one row per wave ran
// 26.8-27.2 us with libm's expf and 25.6 us with hw_exp; two rows per wave with hw_exp
// 23.2-23.6 us; three or four rows per wave through two register buffers 27-29 us (too
// few waves per SIMD). One row group per workgroup (a single wave for rows of up to 4096
// columns): 23.5-23.7 us against 23.9-24.0 us with four single-wave groups per workgroup.
template <typename T, int VEC, int RT, int VALS, int P>
__global__ __launch_bounds__(RT) void softmax_fwd_kernel(
    const T* __restrict__ x, T* __restrict__ y, int rows, int cols, int64_t x_stride,
    int64_t y_stride) {
  static_assert(P == 1 || RT == 64, "several rows per group only for single-wave rows");
  __shared__ float scratch[RT / 64];
  const int lane = threadIdx.x % RT;
  // Rows of 16-byte vectors are streamed once: non-temporal buffer loads and stores
  // (f32 4096 x 4096 went from 4.9 to 5.9 TB/s). The row index is wave-uniform and
  // readfirstlane lets the compiler keep each row's buffer resource scalar.
  constexpr bool kBuf = VEC * sizeof(T) == 16;
  const int row0 = __builtin_amdgcn_readfirstlane(static_cast<int>(blockIdx.x) * P);
  if (row0 >= rows) return;  // the whole workgroup: row0 is uniform

  float v[P][VALS];
#pragma unroll
  for (int p = 0; p < P; ++p) {
    // A group past the last row reloads that row and does not store it.
    const int64_t r = min(row0 + p, rows - 1);
    if constexpr (kBuf)
      tk::load_row_buf<T, VEC, RT, VALS, tk::kCpolStream>(x + r * x_stride, cols, lane, v[p],
                                                           -INFINITY);
    else
      tk::load_row<T, VEC, RT, VALS>(x + r * x_stride, cols, lane, v[p], -INFINITY);
  }
#pragma unroll
  for (int p = 0; p < P; ++p) {
    softmax_row<RT, VALS>(v[p], scratch);
    const int64_t r = row0 + p;
    if (r >= rows) break;
    if constexpr (kBuf)
      tk::store_row_buf<T, VEC, RT, VALS, tk::kCpolStream>(y + r * y_stride, cols, lane, v[p]);
    else
      tk::store_row<T, VEC, RT, VALS>(y + r * y_stride, cols, lane, v[p]);
  }
}

// ------------------------------------------------------------------ online softmax
//
// Rows of any width (beyond the single-pass register budget): each row is split
// into chunks of kOnlineChunk columns, one 256-thread workgroup per chunk.
//   partial: chunk max m_c and s_c = sum exp(x - m_c) over the chunk (one read).
//   apply:   M = max_c m_c, S = sum_c s_c * exp(m_c - M), both folded in a fixed
//            order by every workgroup of the row; then y = exp(x - M) * (1 / S)
//            (a second read of the chunk, one write).
// As two launches (rows wider than kSingleReadChunks chunks) HBM traffic is two reads and
// one write per element; narrower rows take the single-read kernel below, which computes
// the same partials and the same fold in one launch. The workspace holds two floats per
// chunk (one 64-bit word in the single-read kernel). The exponentials are tk::hw_exp (the
// hardware exp2 of x log2(e)): with libm's expf the two passes over f32 64 x 1048576 took
// 0.135 ms, with hw_exp 0.126 ms.

constexpr int kOnlineThreads = 256;
constexpr int kOnlineVals = 64;
constexpr int kOnlineChunk = kOnlineThreads * kOnlineVals;  // 16384 columns

// The first read keeps the default cache policy (a chunk may still be in the
// last-level cache when the second pass reads it); the second read is the last use.
template <typename T, int VEC, int CPOL>
__device__ __forceinline__ void load_chunk(const T* p, int n, int lane, float* v) {
  if constexpr (VEC * sizeof(T) == 16)
    tk::load_row_buf<T, VEC, kOnlineThreads, kOnlineVals, CPOL>(p, n, lane, v, -INFINITY);
  else
    tk::load_row<T, VEC, kOnlineThreads, kOnlineVals>(p, n, lane, v, -INFINITY);
}

template <typename T, int VEC>
__global__ __launch_bounds__(kOnlineThreads) void softmax_online_partial_kernel(
    const T* __restrict__ x, float* __restrict__ partials, int cols, int chunks,
    int64_t x_stride) {
  __shared__ float scratch[kOnlineThreads / 64];
  const int row = blockIdx.x / chunks;
  const int chunk = blockIdx.x - row * chunks;
  const int c0 = chunk * kOnlineChunk;
  const int n = min(kOnlineChunk, cols - c0);
  float v[kOnlineVals];
  load_chunk<T, VEC, tk::kCpolDefault>(x + row * x_stride + c0, n, threadIdx.x, v);
  float m = v[0];
#pragma unroll
  for (int e = 1; e < kOnlineVals; ++e) m = fmaxf(m, v[e]);
  m = tk::group_allreduce<kOnlineThreads>(m, tk::MaxOp{}, scratch);
  float s = 0.f;
  if (m != -INFINITY) {
#pragma unroll
    for (int e = 0; e < kOnlineVals; ++e) s += tk::hw_exp(v[e] - m);
  }
  s = tk::group_allreduce<kOnlineThreads>(s, tk::SumOp{}, scratch);
  if (threadIdx.x == 0) {
    float* out = partials + 2 * static_cast<int64_t>(blockIdx.x);
    out[0] = m;
    out[1] = s;
  }
}

template <typename T, int VEC>
__global__ __launch_bounds__(kOnlineThreads) void softmax_online_apply_kernel(
    const T* __restrict__ x, T* __restrict__ y, const float* __restrict__ partials, int cols,
    int chunks, int64_t x_stride, int64_t y_stride) {
  __shared__ float scratch[kOnlineThreads / 64];
  const int row = blockIdx.x / chunks;
  const int chunk = blockIdx.x - row * chunks;
  const int c0 = chunk * kOnlineChunk;
  const int n = min(kOnlineChunk, cols - c0);
  float v[kOnlineVals];
  load_chunk<T, VEC, tk::kCpolStream>(x + row * x_stride + c0, n, threadIdx.x, v);
  // Row statistics from the chunk partials, in a fixed order (identical in every
  // workgroup of the row).
  const float* pr = partials + 2 * static_cast<int64_t>(row) * chunks;
  float m = -INFINITY;
  for (int j = threadIdx.x; j < chunks; j += kOnlineThreads) m = fmaxf(m, pr[2 * j]);
  m = tk::group_allreduce<kOnlineThreads>(m, tk::MaxOp{}, scratch);
  float s = 0.f;
  for (int j = threadIdx.x; j < chunks; j += kOnlineThreads) {
    const float mj = pr[2 * j];
    if (mj != -INFINITY) s += pr[2 * j + 1] * tk::hw_exp(mj - m);
  }
  s = tk::group_allreduce<kOnlineThreads>(s, tk::SumOp{}, scratch);
  const float inv = 1.0f / s;
#pragma unroll
  for (int e = 0; e < kOnlineVals; ++e) v[e] = tk::hw_exp(v[e] - m) * inv;
  T* yr = y + row * y_stride + c0;
  if constexpr (VEC * sizeof(T) == 16)
    tk::store_row_buf<T, VEC, kOnlineThreads, kOnlineVals, tk::kCpolStream>(yr, n, threadIdx.x,
                                                                             v);
  else
    tk::store_row<T, VEC, kOnlineThreads, kOnlineVals>(yr, n, threadIdx.x, v);
}

// ------------------------------------------------------------------ single-read online softmax
//
// For rows of at most kSingleReadChunks chunks, one launch reads x once: each workgroup keeps
// its chunk in registers, publishes the chunk's (max, sum of exp) and waits until every
// chunk of its row has published, then folds the row's partials exactly as the apply pass
// does and writes its chunk. HBM traffic is one read and one write per element.
//
// Workgroup b handles chunk b % chunks of row b / chunks, so a row's chunks are consecutive
// workgroups. The dispatcher starts each XCD's workgroups in index order, so every workgroup of
// the lowest unfinished row has started (or can start) before any later workgroup holds its
// slot: no row waits on a workgroup that cannot start while one row's chunks (at most
// kSingleReadChunks workgroups) fit on the device. The wait is bounded all the same: after
// `polls` polls a workgroup computes every chunk's partial of its row from x itself, with the
// same arithmetic and thread mapping, and folds those, so the result is bitwise the same on
// either path and no workgroup waits without end. (A ticket counter handing out chunks in
// start order, which needs no assumption about dispatch order, ran f32 64 x 1048576 in
// 0.121 ms against 0.103 ms: one contended atomic before every workgroup's loads.)
//
// Partials are published and polled as device-scope atomic 64-bit words, so the exchange does
// not depend on which XCD's L2 holds a line and needs no cache write-back or invalidate: with a
// release increment of a per-row counter (an L2 write-back per workgroup) and acquire polls the
// same problem ran 0.55-0.58 ms. A word is never zero once published (a finite maximum has a
// sum >= 1, its own term being exp2(0) = 1; -inf and NaN have non-zero bits), so the call
// clears the words first (online_clear_kernel) and a zero word is an unpublished chunk.

constexpr int kSingleReadChunks = 64;  // rows up to 1 048 576 columns
constexpr int kSpinPolls = 1 << 15;    // polls (a ~64-cycle sleep each) before the fallback

// A chunk's max and sum of exp(v - max) over the workgroup (the partial kernel's arithmetic).
__device__ __forceinline__ void chunk_partial(const float* v, float* scratch, float& m, float& s) {
  m = v[0];
#pragma unroll
  for (int e = 1; e < kOnlineVals; ++e) m = fmaxf(m, v[e]);
  m = tk::group_allreduce<kOnlineThreads>(m, tk::MaxOp{}, scratch);
  s = 0.f;
  if (m != -INFINITY) {
#pragma unroll
    for (int e = 0; e < kOnlineVals; ++e) s += tk::hw_exp(v[e] - m);
  }
  s = tk::group_allreduce<kOnlineThreads>(s, tk::SumOp{}, scratch);
}

// chunk_partial of the chunk at p (n valid columns) without holding it in registers: the
// same values in the same order (element e of the thread is column
// ((e / VEC) * 256 + thread) * VEC + e % VEC), read twice, one vector at a time. Used only
// when the bounded wait expires, so it trades reads for registers.
template <typename T, int VEC>
__device__ __forceinline__ void chunk_partial_streamed(const T* p, int n, float* scratch,
                                                       float& m, float& s) {
  constexpr int ITEMS = kOnlineVals / VEC;
  auto item = [&](int i, float* f) {
    const int c = (i * kOnlineThreads + static_cast<int>(threadIdx.x)) * VEC;
    if (c < n) {
      tk::load_vec<T, VEC>(p + c, f);
    } else {
#pragma unroll
      for (int k = 0; k < VEC; ++k) f[k] = -INFINITY;
    }
  };
  float f[VEC];
  item(0, f);
  m = f[0];
#pragma unroll
  for (int k = 1; k < VEC; ++k) m = fmaxf(m, f[k]);
#pragma unroll 1
  for (int i = 1; i < ITEMS; ++i) {
    item(i, f);
#pragma unroll
    for (int k = 0; k < VEC; ++k) m = fmaxf(m, f[k]);
  }
  m = tk::group_allreduce<kOnlineThreads>(m, tk::MaxOp{}, scratch);
  s = 0.f;
  if (m != -INFINITY) {
#pragma unroll 1
    for (int i = 0; i < ITEMS; ++i) {
      item(i, f);
#pragma unroll
      for (int k = 0; k < VEC; ++k) s += tk::hw_exp(f[k] - m);
    }
  }
  s = tk::group_allreduce<kOnlineThreads>(s, tk::SumOp{}, scratch);
}

// Row statistics from the chunk partials (m_j, s_j) held by threads j < chunks (the apply
// kernel's fold: the same thread mapping and reduction order).
__device__ __forceinline__ void fold_partials(float mj, float sj, int chunks, float* scratch,
                                              float& m, float& s) {
  const bool mine = static_cast<int>(threadIdx.x) < chunks;
  m = tk::group_allreduce<kOnlineThreads>(mine ? mj : -INFINITY, tk::MaxOp{}, scratch);
  const float term = mine && mj != -INFINITY ? sj * tk::hw_exp(mj - m) : 0.f;
  s = tk::group_allreduce<kOnlineThreads>(term, tk::SumOp{}, scratch);
}

// Zeroes the partial words of a single-read call (a kernel rather than a memset, so the call
// can be captured in a graph).
__global__ __launch_bounds__(256) void online_clear_kernel(uint64_t* __restrict__ words, int n) {
  for (int64_t i = blockIdx.x * 256 + threadIdx.x; i < n; i += int64_t(gridDim.x) * 256)
    words[i] = 0;
}

// Five waves per SIMD (96 registers) where the chunk fits without spills (float32 and bfloat16
// 16-byte vectors: f32 64 x 1048576 0.1022 vs 0.1033 ms at four).
template <typename T, int VEC>
__global__ __launch_bounds__(kOnlineThreads)
__attribute__((amdgpu_waves_per_eu(VEC == 1 ? 3 : __is_same(T, _Float16) ? 4 : 5))) void
softmax_online_single_read_kernel(
    const T* __restrict__ x, T* __restrict__ y, float* __restrict__ partials,
    int cols, int chunks, int64_t x_stride, int64_t y_stride, int polls) {
  __shared__ float scratch[kOnlineThreads / 64];
  __shared__ float fallback[2 * kSingleReadChunks];
  const int row = static_cast<int>(blockIdx.x) / chunks;
  const int chunk = static_cast<int>(blockIdx.x) - row * chunks;
  const T* xr = x + row * x_stride;
  float v[kOnlineVals];
  {
    const int c0 = chunk * kOnlineChunk;
    load_chunk<T, VEC, tk::kCpolStream>(xr + c0, min(kOnlineChunk, cols - c0), threadIdx.x, v);
  }
  float m, s;
  chunk_partial(v, scratch, m, s);
  // The chunk's partial is published as one 64-bit word (max bits low, sum bits high); thread
  // j < chunks polls chunk j's word until it is non-zero.
  uint64_t* pr = reinterpret_cast<uint64_t*>(partials) + static_cast<int64_t>(row) * chunks;
  if (threadIdx.x == 0) {
    const uint64_t word = uint64_t(__float_as_uint(m)) | (uint64_t(__float_as_uint(s)) << 32);
    __hip_atomic_store(pr + chunk, word, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  bool have = true;
  uint64_t word = 0;
  if (static_cast<int>(threadIdx.x) < chunks) {
    have = false;
    for (int poll = 0; poll < polls; ++poll) {
      word = __hip_atomic_load(pr + threadIdx.x, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (word != 0) {
        have = true;
        break;
      }
      __builtin_amdgcn_s_sleep(1);
    }
  }
  float mj = -INFINITY, sj = 0.f;
  if (__syncthreads_and(have)) {
    if (static_cast<int>(threadIdx.x) < chunks) {
      mj = __uint_as_float(static_cast<uint32_t>(word));
      sj = __uint_as_float(static_cast<uint32_t>(word >> 32));
    }
  } else {
    // Bounded wait expired: every chunk's partial of this row from x (this chunk stays in v).
    for (int j = 0; j < chunks; ++j) {
      const int c0 = j * kOnlineChunk;
      float mk, sk;
      chunk_partial_streamed<T, VEC>(xr + c0, min(kOnlineChunk, cols - c0), scratch, mk, sk);
      if (threadIdx.x == 0) {
        fallback[2 * j] = mk;
        fallback[2 * j + 1] = sk;
      }
    }
    __syncthreads();
    if (static_cast<int>(threadIdx.x) < chunks) {
      mj = fallback[2 * threadIdx.x];
      sj = fallback[2 * threadIdx.x + 1];
    }
  }
  float row_m, row_s;
  fold_partials(mj, sj, chunks, scratch, row_m, row_s);
  const float inv = 1.0f / row_s;
#pragma unroll
  for (int e = 0; e < kOnlineVals; ++e) v[e] = tk::hw_exp(v[e] - row_m) * inv;
  const int c0 = chunk * kOnlineChunk;
  const int n = min(kOnlineChunk, cols - c0);
  T* yr = y + row * y_stride + c0;
  if constexpr (VEC * sizeof(T) == 16)
    tk::store_row_buf<T, VEC, kOnlineThreads, kOnlineVals, tk::kCpolStream>(yr, n, threadIdx.x, v);
  else
    tk::store_row<T, VEC, kOnlineThreads, kOnlineVals>(yr, n, threadIdx.x, v);
}

}  // namespace

extern "C" int tk_softmax_online_fwd(int dtype, const void* x, void* y, float* partials,
                                     int64_t rows, int64_t cols, int64_t x_row_stride,
                                     int64_t y_row_stride, void* stream) {
  if (!tk::valid_dtype(dtype)) return tk::fail("online softmax: unsupported dtype code %d", dtype);
  if (x == nullptr || y == nullptr || partials == nullptr)
    return tk::fail("online softmax: null pointer");
  if ((reinterpret_cast<uintptr_t>(partials) & 7) != 0)
    return tk::fail("online softmax: workspace must be 8-byte aligned");
  if (rows <= 0 || cols <= 0) return tk::fail("online softmax: empty problem");
  if (!tk::row_strides_ok(rows, cols, {x_row_stride, y_row_stride}))
    return tk::fail("online softmax: strides must be non-negative and keep rows in range");
  if (cols > INT32_MAX) return tk::fail("online softmax: more than 2^31-1 columns");
  const int64_t chunks = tk::cdiv(cols, kOnlineChunk);
  if (rows * chunks > INT32_MAX) return tk::fail("online softmax: too many chunks");
  const int es = tk::elem_size(dtype);
  const int vec = 16 / es;
  const bool vector_ok = tk::aligned16(x) && tk::aligned16(y) && cols % vec == 0 &&
                         (x_row_stride * es) % 16 == 0 && (y_row_stride * es) % 16 == 0;
  const dim3 grid(static_cast<unsigned>(rows * chunks));
  const dim3 block(kOnlineThreads);
  hipStream_t s = tk::as_stream(stream);
  if (chunks <= kSingleReadChunks) {
    // One read of x. The environment variable TKLAB_ONLINE_SOFTMAX_POLLS lowers the bound on
    // the wait (0: every workgroup takes the fallback), so tests can check that both paths
    // give the same bits.
    int polls = kSpinPolls;
    if (const char* env = std::getenv("TKLAB_ONLINE_SOFTMAX_POLLS"))
      polls = std::min(std::max(std::atoi(env), 0), kSpinPolls);
    const int words = static_cast<int>(rows * chunks);
    const unsigned clear_blocks = static_cast<unsigned>(std::min<int64_t>(tk::cdiv(words, 256), 1024));
    hipLaunchKernelGGL(online_clear_kernel, dim3(clear_blocks), dim3(256), 0, s,
                       reinterpret_cast<uint64_t*>(partials), words);
    TK_DISPATCH_DTYPE(dtype, T,
      TK_DISPATCH_VEC(T, vector_ok,
        hipLaunchKernelGGL((softmax_online_single_read_kernel<T, VEC>), grid, block, 0, s,
                           static_cast<const T*>(x), static_cast<T*>(y), partials, (int)cols,
                           (int)chunks, x_row_stride, y_row_stride, polls)));
    return tk::check_launch("online softmax");
  }
  TK_DISPATCH_DTYPE(dtype, T,
    TK_DISPATCH_VEC(T, vector_ok,
      hipLaunchKernelGGL((softmax_online_partial_kernel<T, VEC>), grid, block, 0, s,
                         static_cast<const T*>(x), partials, (int)cols, (int)chunks,
                         x_row_stride);
      hipLaunchKernelGGL((softmax_online_apply_kernel<T, VEC>), grid, block, 0, s,
                         static_cast<const T*>(x), static_cast<T*>(y), partials, (int)cols,
                         (int)chunks, x_row_stride, y_row_stride)));
  return tk::check_launch("online softmax");
}

extern "C" int tk_softmax_fwd(int dtype, const void* x, void* y, int64_t rows, int64_t cols,
                              int64_t x_row_stride, int64_t y_row_stride, void* stream) {
  if (!tk::valid_dtype(dtype)) return tk::fail("softmax: unsupported dtype code %d", dtype);
  if (x == nullptr || y == nullptr) return tk::fail("softmax: null pointer");
  if (rows <= 0 || cols <= 0) return tk::fail("softmax: empty problem");
  if (!tk::row_strides_ok(rows, cols, {x_row_stride, y_row_stride}))
    return tk::fail("softmax: strides must be non-negative and keep rows in range");
  if (rows > INT32_MAX) return tk::fail("softmax: too many rows");
  tk::RowShape shape;
  if (cols > 65536 || !tk::pick_row_shape(cols, &shape))
    return tk::fail("softmax: %lld columns exceed the 65536-column single-pass limit",
                    (long long)cols);
  const int es = tk::elem_size(dtype);
  const int vec = 16 / es;
  const bool vector_ok = tk::aligned16(x) && tk::aligned16(y) && cols % vec == 0 &&
                         (x_row_stride * es) % 16 == 0 && (y_row_stride * es) % 16 == 0;
  // Two single-wave rows per wave once that still leaves two waves per SIMD (4096 rows).
  const bool pair = shape.rt == 64 && rows >= 4096;
  const dim3 grid(static_cast<unsigned>(tk::cdiv(rows, pair ? 2 : 1)));
  const dim3 block(shape.rt);
  hipStream_t s = tk::as_stream(stream);
  TK_DISPATCH_DTYPE(dtype, T,
    TK_DISPATCH_VEC(T, vector_ok,
      TK_DISPATCH_ROW_SHAPE(shape,
        constexpr int P2 = RT == 64 ? 2 : 1;
        if (pair)
          hipLaunchKernelGGL((softmax_fwd_kernel<T, VEC, RT, VALS, P2>), grid, block, 0, s,
                             static_cast<const T*>(x), static_cast<T*>(y), (int)rows, (int)cols,
                             x_row_stride, y_row_stride);
        else
          hipLaunchKernelGGL((softmax_fwd_kernel<T, VEC, RT, VALS, 1>), grid, block, 0, s,
                             static_cast<const T*>(x), static_cast<T*>(y), (int)rows, (int)cols,
                             x_row_stride, y_row_stride))));
  return tk::check_launch("softmax");
}
