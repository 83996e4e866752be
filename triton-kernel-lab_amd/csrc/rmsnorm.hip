// RMSNorm (optionally with a fused residual add): forward, and the two-stage
// deterministic backward.
//
// Forward math (src/tklab/kernels/rms_norm.py:61-78 and
// src/tklab/kernels/residual_rms_norm.py:52-82): s = x (+ residual, rounded to
// the storage dtype), rstd = 1/sqrt(sum(s*s)/n + eps), y = s * rstd * w.
//
// Backward math (src/tklab/kernels/rms_norm.py:105-133): x_hat = x*rstd,
// g = w*dy, dx = rstd*(g - x_hat*sum(g*x_hat)/n) (+ incoming_dx),
// dweight = sum over rows of dy*x_hat.
//
// The reference accumulates dweight partials under a global spin lock in an
// order that depends on scheduling. Here each workgroup is one group: it owns the
// rows row % group_count == g (the reference's lock grouping, rms_norm.py:134) and
// takes them in increasing order, keeps its column partials in registers (a thread
// always holds the same columns), folds its row slots together in LDS in a fixed
// order and writes partial_dw[g] once. Stage 2 sums the partial
// rows in a fixed order. Both stages are bitwise reproducible.
#include <atomic>

#include "rows.hpp"

#pragma clang fp contract(off)

namespace {

constexpr int kNormBlock = 256;

template <typename T, int VEC, int RT, int VALS>
__global__ __launch_bounds__(RT >= kNormBlock ? RT : kNormBlock) void rmsnorm_fwd_kernel(
    const T* __restrict__ x, const T* __restrict__ residual, const T* __restrict__ weight,
    T* __restrict__ residual_sum, T* __restrict__ y, float* __restrict__ rstd_out, int rows,
    int cols, int64_t x_stride, int64_t r_stride, int64_t s_stride, int64_t y_stride, float eps) {
  constexpr int SLOTS = RT >= kNormBlock ? 1 : kNormBlock / RT;
  using Row = tk::RawRow<T, VEC, RT, VALS>;
  __shared__ float scratch[RT / 64];
  // 16-byte rows go through buffer accesses with per-stream cache policies: the
  // inputs are streamed (non-temporal), the outputs stored with sc1.
  constexpr bool kBuf = VEC * sizeof(T) == 16;
  const int lane = threadIdx.x % RT;
  // A wave's threads share one row (RT >= 64); readfirstlane makes that visible to
  // the compiler, so the row's buffer resource lives in scalar registers.
  const int row = __builtin_amdgcn_readfirstlane(blockIdx.x * SLOTS + threadIdx.x / RT);
  if (row >= rows) return;  // SLOTS > 1 only for barrier-free single-wave rows

  // s is kept in the storage type: with a residual it is rounded there anyway.
  Row sv;
  if constexpr (kBuf)
    sv.template load_buf<tk::kCpolStream>(x + row * x_stride, cols, lane);
  else
    sv.load(x + row * x_stride, cols, lane);
  if (residual != nullptr) {
    Row rv;
    if constexpr (kBuf)
      rv.template load_buf<tk::kCpolStream>(residual + row * r_stride, cols, lane);
    else
      rv.load(residual + row * r_stride, cols, lane);
#pragma unroll
    for (int e = 0; e < VALS; ++e) sv.set(e, sv.get(e) + rv.get(e));
    if (residual_sum != nullptr) {
      if constexpr (kBuf)
        sv.template store_buf<tk::kCpolSc1>(residual_sum + row * s_stride, cols, lane);
      else
        sv.store(residual_sum + row * s_stride, cols, lane);
    }
  }

  float ss = 0.f;
#pragma unroll
  for (int e = 0; e < VALS; ++e) ss += sv.get(e) * sv.get(e);
  ss = tk::group_allreduce<RT>(ss, tk::SumOp{}, scratch);
  const float rstd = 1.0f / sqrtf(ss / static_cast<float>(cols) + eps);

  // Statistics mode (y null): only s and rstd are produced, for a consumer that applies
  // rstd and the weight itself (the row-scaled GEMM).
  if (y != nullptr) {
    Row wv;
    wv.load(weight, cols, lane);
#pragma unroll
    for (int e = 0; e < VALS; ++e) wv.set(e, sv.get(e) * rstd * wv.get(e));
    if constexpr (kBuf)
      wv.template store_buf<tk::kCpolSc1>(y + row * y_stride, cols, lane);
    else
      wv.store(y + row * y_stride, cols, lane);
  }
  if (rstd_out != nullptr && lane == 0) rstd_out[row] = rstd;
}

// Row tensors of the backward stage 1 and their row strides.
template <typename T>
struct RowPtrs {
  const T* x;
  const T* dy;
  const T* inc;
  T* dx;
  int64_t xs, dys, incs, dxs;
};

// One row's x, dy, incoming gradient and rstd, held in registers.
template <typename Row>
struct RowSet {
  Row x, dy, inc;
  float r;
};

template <typename T, typename Row>
__device__ __forceinline__ void load_rowset(RowSet<Row>& s, const RowPtrs<T>& p, int64_t row,
                                            int cols, int lane, const float* rstd) {
  s.x.load(p.x + row * p.xs, cols, lane);
  s.dy.load(p.dy + row * p.dys, cols, lane);
  if (p.inc != nullptr) s.inc.load(p.inc + row * p.incs, cols, lane);
  s.r = rstd[row];
}

// Branch-free, non-temporal row loads for 16-byte vectors (RawRow::load_buf: columns
// at or past `cols` read as zero, so cols = 0 loads nothing from memory). Without
// branches the compiler can count the loads still in flight exactly and wait only for
// the row it uses.
template <typename T, typename Row>
__device__ __forceinline__ void load_rowset_buf(RowSet<Row>& s, const RowPtrs<T>& p, int64_t row,
                                                int cols, int lane, const float* rstd) {
  s.x.template load_buf<tk::kCpolStream>(p.x + row * p.xs, cols, lane);
  s.dy.template load_buf<tk::kCpolStream>(p.dy + row * p.dys, cols, lane);
  if (p.inc != nullptr) s.inc.template load_buf<tk::kCpolStream>(p.inc + row * p.incs, cols, lane);
  s.r = rstd[row];
}

// dx of one row and its dweight contribution: x_hat = x*rstd, g = w*dy,
// dx = rstd*(g - x_hat*mean(g*x_hat)) (+ incoming), acc += dy*x_hat. Every thread of the
// row group calls it (group_allreduce holds block barriers for multi-wave rows).
template <typename T, int VEC, int RT, int VALS, bool ACC_LDS, typename Row>
__device__ __forceinline__ void stage1_row(RowSet<Row>& s, const Row& wv, const RowPtrs<T>& p,
                                           int64_t row, int cols, int lane, float* acc,
                                           float* fold, float* scratch) {
  float dot = 0.f;
#pragma unroll
  for (int e = 0; e < VALS; ++e) {
    const float x_hat = s.x.get(e) * s.r;
    const float d = s.dy.get(e);
    if constexpr (ACC_LDS)
      fold[tk::row_column<VEC, RT>(e, lane)] += d * x_hat;
    else
      acc[e] += d * x_hat;
    dot += (wv.get(e) * d) * x_hat;
  }
  dot = tk::group_allreduce<RT>(dot, tk::SumOp{}, scratch);
  const float mean = dot / static_cast<float>(cols);
#pragma unroll
  for (int e = 0; e < VALS; ++e) {
    const float x_hat = s.x.get(e) * s.r;
    const float g = wv.get(e) * s.dy.get(e);
    float v = s.r * (g - x_hat * mean);
    if (p.inc != nullptr) v += s.inc.get(e);
    s.x.set(e, v);
  }
  if constexpr (VEC * sizeof(T) == 16)
    s.x.template store_buf<tk::kCpolStream>(p.dx + row * p.dxs, cols, lane);
  else
    s.x.store(p.dx + row * p.dxs, cols, lane);
}

// Threads per workgroup of the backward stage 1: four single-wave row slots,
// or one multi-wave row group.
template <int RT>
constexpr int bwd_block() { return RT == 64 ? 256 : RT; }

template <typename T, int VEC, int RT, int VALS>
__global__ __launch_bounds__(bwd_block<RT>()) void rmsnorm_bwd_stage1_kernel(
    T* __restrict__ dx, const T* __restrict__ dy, const T* __restrict__ incoming,
    float* __restrict__ partial, const T* __restrict__ x, const T* __restrict__ weight,
    const float* __restrict__ rstd, int32_t* __restrict__ counts, int rows, int cols,
    int64_t x_stride, int64_t dy_stride, int64_t inc_stride, int64_t dx_stride) {
  constexpr int SLOTS = bwd_block<RT>() / RT;
  constexpr int WIDTH = RT * VALS;  // columns one row slot covers
  using Row = tk::RawRow<T, VEC, RT, VALS>;
  // dweight partials: registers, except for the widest launched rows (1024 threads
  // x 32 values, beyond the 128 registers a 1024-thread workgroup allows), whose
  // single slot keeps them in 128 KiB of LDS; each address belongs to one thread.
  // (1024 x 64 is never launched: rows are limited to 65536 bytes.)
  constexpr bool ACC_LDS = SLOTS == 1 && RT == 1024 && VALS == 32;
  // Slot partials are folded through LDS once, at the end (single-wave slots only).
  __shared__ float fold[SLOTS > 1 || ACC_LDS ? WIDTH : 1];
  __shared__ float scratch[RT / 64];

  const int group = blockIdx.x;
  // A slot is one wave or a whole workgroup, so it is wave-uniform (and so are the row
  // addresses and buffer descriptors derived from it).
  const int slot = __builtin_amdgcn_readfirstlane(threadIdx.x / RT);
  const int lane = threadIdx.x % RT;
  // Rows of this group: row = group + k * G for k = 0, 1, ... (G = gridDim.x, the row % G
  // grouping of the lock-based original), so at any time the groups stream a window of
  // about G neighbouring rows of each tensor; slot s takes the rows k = s mod SLOTS.
  const int G = gridDim.x;
  const int group_rows = group < rows ? (rows - 1 - group) / G + 1 : 0;
  auto row_of = [&](int k) { return static_cast<int64_t>(group) + static_cast<int64_t>(k) * G; };

  // dweight partials of this thread's columns, accumulated over its rows in order.
  float acc[ACC_LDS ? 1 : VALS];
#pragma unroll
  for (int e = 0; e < VALS; ++e) {
    if constexpr (ACC_LDS)
      fold[tk::row_column<VEC, RT>(e, lane)] = 0.f;
    else
      acc[e] = 0.f;
  }

  // The weight row is loaded once, before any row: a load issued after the prefetches
  // would make its wait (in-order vmcnt) wait for them too.
  Row wv;
  wv.load(weight, cols, lane);
  const RowPtrs<T> ptr{x, dy, incoming, dx, x_stride, dy_stride, inc_stride, dx_stride};
  if (group_rows == 0) {
    // A group past the last row owns no rows (the entry points launch min(G, rows)
    // groups, so none does); it would only write a zero partial row.
  } else if constexpr (RT < 1024 && VEC * sizeof(T) == 16) {
    // Software pipeline, unrolled by three so the three row buffers rotate roles
    // without register copies (a copy would wait for the load still in flight): the
    // loads of the next two rows of this slot overlap the current row's reduction.
    // Loads are issued unconditionally, so the wait before each row counts exactly the
    // two younger rows' loads; past the group's last row they use a zero-length buffer
    // (the last row's address, zero extent), which returns zeros without memory traffic.
    RowSet<Row> ra, rb, rc;
    const int last = max(group_rows - 1, 0);
    auto rowk = [&](int k) { return row_of(min(k, last)); };
    auto extent = [&](int k) { return k < group_rows ? cols : 0; };
    const int k0 = slot;
    load_rowset_buf<T>(ra, ptr, rowk(k0), extent(k0), lane, rstd);
    load_rowset_buf<T>(rb, ptr, rowk(k0 + SLOTS), extent(k0 + SLOTS), lane, rstd);
    for (int k = k0; k < group_rows; k += 3 * SLOTS) {
      load_rowset_buf<T>(rc, ptr, rowk(k + 2 * SLOTS), extent(k + 2 * SLOTS), lane, rstd);
      stage1_row<T, VEC, RT, VALS, ACC_LDS>(ra, wv, ptr, row_of(k), cols, lane, acc, fold, scratch);
      if (k + SLOTS >= group_rows) break;
      load_rowset_buf<T>(ra, ptr, rowk(k + 3 * SLOTS), extent(k + 3 * SLOTS), lane, rstd);
      stage1_row<T, VEC, RT, VALS, ACC_LDS>(rb, wv, ptr, row_of(k + SLOTS), cols, lane, acc, fold,
                                            scratch);
      if (k + 2 * SLOTS >= group_rows) break;
      load_rowset_buf<T>(rb, ptr, rowk(k + 4 * SLOTS), extent(k + 4 * SLOTS), lane, rstd);
      stage1_row<T, VEC, RT, VALS, ACC_LDS>(rc, wv, ptr, row_of(k + 2 * SLOTS), cols, lane, acc,
                                            fold, scratch);
    }
  } else {
    // 1024-thread workgroups (at most 128 registers) and the unaligned scalar path:
    // one row at a time.
    RowSet<Row> ra;
    for (int k = slot; k < group_rows; k += SLOTS) {
      load_rowset<T>(ra, ptr, row_of(k), cols, lane, rstd);
      stage1_row<T, VEC, RT, VALS, ACC_LDS>(ra, wv, ptr, row_of(k), cols, lane, acc, fold, scratch);
    }
  }

  float* out = partial + static_cast<int64_t>(group) * cols;
  if constexpr (SLOTS == 1) {
#pragma unroll
    for (int e = 0; e < VALS; ++e) {
      const int c = tk::row_column<VEC, RT>(e, lane);
      if (c < cols) out[c] = ACC_LDS ? fold[c] : acc[e];
    }
  } else {
    // ((slot 0 + slot 1) + slot 2) + ...: one slot at a time, in slot order.
    for (int s2 = 0; s2 < SLOTS; ++s2) {
      if (slot == s2) {
#pragma unroll
        for (int e = 0; e < VALS; ++e) {
          const int c = tk::row_column<VEC, RT>(e, lane);
          if (c < cols) fold[c] = s2 == 0 ? acc[e] : fold[c] + acc[e];
        }
      }
      __syncthreads();
    }
    for (int c = threadIdx.x; c < cols; c += bwd_block<RT>()) out[c] = fold[c];
  }
  if (counts != nullptr && threadIdx.x == 0) counts[group] = 1;
}

constexpr int kStage2Cols = 32;    // columns per workgroup: 128-byte row segments
constexpr int kStage2Slices = 32;  // interleaved partial-row slices per column
constexpr int kStage2Threads = kStage2Cols * kStage2Slices;

// dw[c] = sum over g of partial[g][c]. Thread (slice s, column c) sums the rows
// g = s, s + 32, s + 64, ... in increasing order; the 32 slice sums are then added
// in slice order. Narrow column blocks give cols / 32 workgroups, enough to keep
// many partial rows in flight.
template <typename T>
__global__ __launch_bounds__(kStage2Threads) void rmsnorm_bwd_stage2_kernel(
    const float* __restrict__ partial, T* __restrict__ dw, int group_count, int cols) {
  __shared__ float slices[kStage2Slices][kStage2Cols];
  const int col = threadIdx.x % kStage2Cols;
  const int slice = threadIdx.x / kStage2Cols;
  const int c = blockIdx.x * kStage2Cols + col;
  float s = 0.f;
  if (c < cols) {
#pragma unroll 16
    for (int g = slice; g < group_count; g += kStage2Slices)
      s += partial[static_cast<int64_t>(g) * cols + c];
  }
  slices[slice][col] = s;
  __syncthreads();
  if (slice == 0 && c < cols) {
    float t = slices[0][col];
#pragma unroll
    for (int i = 1; i < kStage2Slices; ++i) t += slices[i][col];
    dw[c] = tk::from_f32<T>(t);
  }
}

bool rows_vector_ok(int dtype, int64_t cols, std::initializer_list<const void*> ptrs,
                    std::initializer_list<int64_t> strides) {
  const int es = tk::elem_size(dtype);
  if (cols % (16 / es) != 0) return false;
  for (const void* p : ptrs)
    if (p != nullptr && !tk::aligned16(p)) return false;
  for (int64_t s : strides)
    if ((s * es) % 16 != 0) return false;
  return true;
}

int check_rows(const char* what, int dtype, int64_t rows, int64_t cols, bool vector_ok,
               tk::RowShape* shape) {
  if (!tk::valid_dtype(dtype)) return tk::fail("%s: unsupported dtype code %d", what, dtype);
  if (rows <= 0 || cols <= 0) return tk::fail("%s: empty problem", what);
  if (rows > INT32_MAX) return tk::fail("%s: too many rows", what);
  // At most 32 registers per row tensor per thread: 64 packed 16-bit values,
  // 32 float32 values, or 32 unpacked values on the unaligned scalar path.
  const int max_vals = vector_ok ? 128 / tk::elem_size(dtype) : 32;
  if (cols * tk::elem_size(dtype) > 65536 || !tk::pick_row_shape(cols, shape, max_vals))
    return tk::fail("%s: feature row exceeds the 65536-byte fused limit", what);
  return 0;
}

}  // namespace

extern "C" int tk_rmsnorm_fwd(int dtype, const void* x, const void* residual, const void* weight,
                              void* residual_sum, void* y, float* rstd, int64_t rows, int64_t cols,
                              int64_t x_row_stride, int64_t residual_row_stride,
                              int64_t residual_sum_row_stride, int64_t y_row_stride, float eps,
                              void* stream) {
  if (x == nullptr || (y != nullptr && weight == nullptr) || (y == nullptr && rstd == nullptr))
    return tk::fail("rmsnorm_fwd: null pointer");
  if (!tk::row_strides_ok(rows, cols,
                          {x_row_stride, residual ? residual_row_stride : 0,
                           residual_sum ? residual_sum_row_stride : 0, y ? y_row_stride : 0}))
    return tk::fail("rmsnorm_fwd: strides must be non-negative and keep rows in range");
  if (!(eps > 0.f)) return tk::fail("rmsnorm_fwd: eps must be finite and positive");
  const bool vector_ok = tk::valid_dtype(dtype) && rows_vector_ok(
      dtype, cols, {x, residual, weight, residual_sum, y},
      {x_row_stride, residual ? residual_row_stride : 0, residual_sum ? residual_sum_row_stride : 0,
       y_row_stride});
  tk::RowShape shape;
  if (check_rows("rmsnorm_fwd", dtype, rows, cols, vector_ok, &shape)) return 1;
  // At most 16 values per thread where the row allows (several waves per row): on the
  // bf16 16384 x 4096 residual forward one wave per row (64 values per thread) ran 93 us,
  // four waves per row 88 us. Rows wider than 1024 x 16 keep the wider shape.
  tk::pick_row_shape(cols, &shape, 16);
  const int slots = shape.rt >= kNormBlock ? 1 : kNormBlock / shape.rt;
  const dim3 grid(static_cast<unsigned>(tk::cdiv(rows, slots)));
  const dim3 block(shape.rt >= kNormBlock ? shape.rt : kNormBlock);
  hipStream_t s = tk::as_stream(stream);
  TK_DISPATCH_DTYPE(dtype, T,
    TK_DISPATCH_VEC(T, vector_ok,
      TK_DISPATCH_ROW_SHAPE(shape,
        hipLaunchKernelGGL((rmsnorm_fwd_kernel<T, VEC, RT, VALS>), grid, block, 0, s,
                           static_cast<const T*>(x), static_cast<const T*>(residual),
                           static_cast<const T*>(weight), static_cast<T*>(residual_sum),
                           static_cast<T*>(y), rstd, (int)rows, (int)cols, x_row_stride,
                           residual_row_stride, residual_sum_row_stride, y_row_stride, eps))));
  return tk::check_launch("rmsnorm_fwd");
}

extern "C" int tk_rmsnorm_bwd_stage1(int dtype, void* dx, const void* dy, const void* incoming_dx,
                                     float* partial_dw, const void* x, const void* weight,
                                     const float* rstd, int32_t* locks, int64_t rows, int64_t cols,
                                     int64_t x_row_stride, int64_t dy_row_stride,
                                     int64_t incoming_dx_row_stride, int64_t dx_row_stride,
                                     int64_t group_size, void* stream) {
  if (dx == nullptr || dy == nullptr || partial_dw == nullptr || x == nullptr ||
      weight == nullptr || rstd == nullptr || locks == nullptr)
    return tk::fail("rmsnorm_bwd_stage1: null pointer");
  if (!tk::row_strides_ok(rows, cols,
                          {x_row_stride, dy_row_stride,
                           incoming_dx ? incoming_dx_row_stride : 0, dx_row_stride}))
    return tk::fail("rmsnorm_bwd_stage1: strides must be non-negative and keep rows in range");
  if (group_size <= 0 || group_size > INT32_MAX)
    return tk::fail("rmsnorm_bwd_stage1: group_size must be positive");
  const int64_t group_count = group_size < rows ? group_size : rows;
  const bool vector_ok = tk::valid_dtype(dtype) && rows_vector_ok(
      dtype, cols, {dx, dy, incoming_dx, x, weight},
      {x_row_stride, dy_row_stride, incoming_dx ? incoming_dx_row_stride : 0, dx_row_stride});
  tk::RowShape shape;
  if (check_rows("rmsnorm_bwd_stage1", dtype, rows, cols, vector_ok, &shape)) return 1;
  // Stage 1 holds three rows of three tensors plus the dweight partials per thread: at
  // most 64 bytes of each row tensor per thread (32 packed 16-bit or 16 float32 values)
  // keeps that in registers without spilling.
  tk::pick_row_shape(cols, &shape, 64 / tk::elem_size(dtype));
  const dim3 grid(static_cast<unsigned>(group_count));
  hipStream_t s = tk::as_stream(stream);
  int32_t* counts = locks + group_size;
  TK_DISPATCH_DTYPE(dtype, T,
    TK_DISPATCH_VEC(T, vector_ok,
      TK_DISPATCH_ROW_SHAPE(shape,
        hipLaunchKernelGGL((rmsnorm_bwd_stage1_kernel<T, VEC, RT, VALS>), grid,
                           dim3(bwd_block<RT>()), 0, s, static_cast<T*>(dx),
                           static_cast<const T*>(dy), static_cast<const T*>(incoming_dx),
                           partial_dw, static_cast<const T*>(x), static_cast<const T*>(weight),
                           rstd, counts, (int)rows, (int)cols, x_row_stride, dy_row_stride,
                           incoming_dx_row_stride, dx_row_stride))));
  return tk::check_launch("rmsnorm_bwd_stage1");
}

extern "C" int tk_rmsnorm_bwd_stage2(int dtype, const float* partial_dw, void* dw,
                                     int64_t group_count, int64_t cols, void* stream) {
  if (!tk::valid_dtype(dtype)) return tk::fail("rmsnorm_bwd_stage2: unsupported dtype code %d", dtype);
  if (partial_dw == nullptr || dw == nullptr) return tk::fail("rmsnorm_bwd_stage2: null pointer");
  if (group_count <= 0 || cols <= 0 || group_count > INT32_MAX || cols > INT32_MAX ||
      group_count * cols > INT32_MAX)
    return tk::fail("rmsnorm_bwd_stage2: bad partial shape");
  const dim3 grid(static_cast<unsigned>(tk::cdiv(cols, kStage2Cols)));
  hipStream_t s = tk::as_stream(stream);
  TK_DISPATCH_DTYPE(dtype, T,
    hipLaunchKernelGGL((rmsnorm_bwd_stage2_kernel<T>), grid, dim3(kStage2Threads), 0, s,
                       partial_dw, static_cast<T*>(dw), (int)group_count, (int)cols));
  return tk::check_launch("rmsnorm_bwd_stage2");
}

// ----------------------------------------------------------------------------------------------
// Backward without allocation: the dweight partial rows live in a library-owned device array.

namespace {

// Float32 dweight partial rows of tk_rmsnorm_bwd_noalloc: group_count x cols floats at most
// (16 MiB). Each GPU holds its own copy for the life of the process. In host code the name is
// only a stand-in: kernels receive the device address from hipGetSymbolAddress.
constexpr int64_t kNoallocScratchFloats = TK_RMSNORM_NOALLOC_SCRATCH_BYTES / 4;
__device__ __align__(256) float scratch[kNoallocScratchFloats];

constexpr int kMaxDevices = 64;
std::atomic<float*> g_scratch_address[kMaxDevices];

// Device address of the current device's `scratch`, looked up once per device (the lookup is
// idempotent, so two threads racing on the first call store the same address).
int scratch_address(const char* what, hipStream_t stream, float** out) {
  int device = 0;
  hipError_t err = hipGetDevice(&device);
  if (err != hipSuccess) return tk::fail("%s: hipGetDevice failed: %s", what, hipGetErrorString(err));
  if (device < 0 || device >= kMaxDevices)
    return tk::fail("%s: device ordinal %d out of range", what, device);
  if (stream != nullptr) {
    hipDevice_t stream_device = 0;
    err = hipStreamGetDevice(stream, &stream_device);
    if (err != hipSuccess)
      return tk::fail("%s: hipStreamGetDevice failed: %s", what, hipGetErrorString(err));
    if (stream_device != device)
      return tk::fail("%s: the stream belongs to device %d, the current device is %d", what,
                      static_cast<int>(stream_device), device);
  }
  float* address = g_scratch_address[device].load(std::memory_order_acquire);
  if (address == nullptr) {
    void* symbol = nullptr;
    err = hipGetSymbolAddress(&symbol, HIP_SYMBOL(scratch));
    if (err != hipSuccess || symbol == nullptr)
      return tk::fail("%s: hipGetSymbolAddress(scratch) failed: %s", what, hipGetErrorString(err));
    address = static_cast<float*>(symbol);
    g_scratch_address[device].store(address, std::memory_order_release);
  }
  *out = address;
  return 0;
}

}  // namespace

extern "C" int tk_rmsnorm_bwd_noalloc(int dtype, void* dx, void* dw, const void* dy,
                                      const void* incoming_dx, const void* x, const void* weight,
                                      const float* rstd, int64_t rows, int64_t cols,
                                      int64_t x_row_stride, int64_t dy_row_stride,
                                      int64_t incoming_dx_row_stride, int64_t dx_row_stride,
                                      int64_t group_size, void* stream) {
  if (dx == nullptr || dw == nullptr || dy == nullptr || x == nullptr || weight == nullptr ||
      rstd == nullptr)
    return tk::fail("rmsnorm_bwd_noalloc: null pointer");
  if (!tk::row_strides_ok(rows, cols,
                          {x_row_stride, dy_row_stride,
                           incoming_dx ? incoming_dx_row_stride : 0, dx_row_stride}))
    return tk::fail("rmsnorm_bwd_noalloc: strides must be non-negative and keep rows in range");
  if (group_size <= 0 || group_size > INT32_MAX)
    return tk::fail("rmsnorm_bwd_noalloc: group_size must be positive");
  if (rows <= 0 || cols <= 0) return tk::fail("rmsnorm_bwd_noalloc: empty problem");
  const int64_t group_count = group_size < rows ? group_size : rows;
  if (cols > kNoallocScratchFloats || group_count > kNoallocScratchFloats / cols)
    return tk::fail("rmsnorm_bwd_noalloc: %lld partial rows of %lld columns need %lld bytes of "
                    "scratch, above the %lld-byte maximum (use fewer groups)",
                    static_cast<long long>(group_count), static_cast<long long>(cols),
                    static_cast<long long>(group_count * cols * 4),
                    static_cast<long long>(TK_RMSNORM_NOALLOC_SCRATCH_BYTES));
  const bool vector_ok = tk::valid_dtype(dtype) && rows_vector_ok(
      dtype, cols, {dx, dy, incoming_dx, x, weight},
      {x_row_stride, dy_row_stride, incoming_dx ? incoming_dx_row_stride : 0, dx_row_stride});
  tk::RowShape shape;
  if (check_rows("rmsnorm_bwd_noalloc", dtype, rows, cols, vector_ok, &shape)) return 1;
  tk::pick_row_shape(cols, &shape, 64 / tk::elem_size(dtype));
  hipStream_t s = tk::as_stream(stream);
  float* partial = nullptr;
  if (scratch_address("rmsnorm_bwd_noalloc", s, &partial)) return 1;
  // Stage 1 writes every one of the group_count = min(group_size, rows) partial rows, so
  // the array needs no clearing; stage 2 reads exactly those rows.
  TK_DISPATCH_DTYPE(dtype, T,
    TK_DISPATCH_VEC(T, vector_ok,
      TK_DISPATCH_ROW_SHAPE(shape,
        hipLaunchKernelGGL((rmsnorm_bwd_stage1_kernel<T, VEC, RT, VALS>),
                           dim3(static_cast<unsigned>(group_count)), dim3(bwd_block<RT>()), 0, s,
                           static_cast<T*>(dx), static_cast<const T*>(dy),
                           static_cast<const T*>(incoming_dx), partial, static_cast<const T*>(x),
                           static_cast<const T*>(weight), rstd, nullptr, (int)rows, (int)cols,
                           x_row_stride, dy_row_stride, incoming_dx_row_stride,
                           dx_row_stride))));
  if (tk::check_launch("rmsnorm_bwd_noalloc (stage 1)")) return 1;
  TK_DISPATCH_DTYPE(dtype, T,
    hipLaunchKernelGGL((rmsnorm_bwd_stage2_kernel<T>),
                       dim3(static_cast<unsigned>(tk::cdiv(cols, kStage2Cols))),
                       dim3(kStage2Threads), 0, s, partial, static_cast<T*>(dw), (int)group_count,
                       (int)cols));
  return tk::check_launch("rmsnorm_bwd_noalloc (stage 2)");
}
