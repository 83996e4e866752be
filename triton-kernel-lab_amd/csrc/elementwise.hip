// Elementwise kernels: SwiGLU forward/backward, rotate-half RoPE forward/backward, and
// row scaling (folding a normalization weight into a projection).
//
// A chunk is VEC contiguous elements (VEC = 16/sizeof(T): one 128-bit access per
// tensor). A workgroup pass takes kUnroll * kBlock consecutive chunks; each thread
// issues the loads of its kUnroll chunks before any arithmetic, so every wave keeps
// a contiguous 4 KiB run per tensor in flight (one chunk per thread, or chunks far
// apart, leave HBM well short of its bandwidth). Row strides are honoured, so row-sliced views need no copy; the
// row of a chunk comes from a multiply-shift division by chunks_per_row. Tensors
// touched once are loaded and stored non-temporally; the RoPE cos/sin tables use
// plain loads, since a broadcast table (row stride 0) is reused by every row.
//
// Floating-point contraction is disabled so each product and sum is rounded
// separately, the same way PyTorch's pointwise ops evaluate these formulas.
#include "tk_common.hpp"

#pragma clang fp contract(off)

namespace {

constexpr int kBlock = 256;
// The RoPE kernels run one wave per workgroup: bf16 [4,32,4096,128] forward 67.3-67.5 ->
// 65.8-65.9 us and backward 66.9-67.3 -> 65.4-65.5 us against four waves; the SwiGLU
// backward ran 3 % slower that way (382-384 -> 394-395 us), so SwiGLU keeps four.
constexpr int kRopeBlock = 64;

using tk::stable_sigmoid;

constexpr int kUnroll = 4;
// RoPE: two chunks per thread and pass (one-wave workgroups): forward 66.2-66.5 -> 65.8-66.0
// us, backward 65.5-65.9 -> 65.1-65.3 us; SwiGLU runs best at four (two: 222 -> 226 us
// forward, eight: 239 us).
constexpr int kRopeUnroll = 2;
// One workgroup per pass of kUnroll * kBlock chunks up to 2^18 passes (beyond that the loop
// strides): on SwiGLU bf16 16384 x 14336 a grid of 8192 workgroups walking the passes
// grid-stride ran 231 / 395 us (forward / backward), one workgroup per pass 218 / 379 us.
constexpr int64_t kMaxBlocks = int64_t(1) << 18;

struct Grid1D {
  unsigned blocks;
};

inline Grid1D chunk_grid(int64_t chunks, int block = kBlock, int unroll = kUnroll) {
  int64_t blocks = tk::cdiv(chunks, int64_t(block) * unroll);
  if (blocks > kMaxBlocks) blocks = kMaxBlocks;
  return {static_cast<unsigned>(blocks)};
}

// Chunk i of a row-major problem: its row and the first element's column.
struct ChunkPos {
  int row, col;
};

template <int VEC>
__device__ __forceinline__ ChunkPos chunk_pos(uint32_t i, const tk::FastDiv& per_row) {
  const uint32_t row = per_row.div(i);
  return {static_cast<int>(row), static_cast<int>(i - row * per_row.d) * VEC};
}

// ------------------------------------------------------------------ SwiGLU

// y = value * gate * sigmoid(gate)  (src/tklab/kernels/swiglu.py:44-58)
template <typename T, int VEC>
__global__ __launch_bounds__(kBlock) void swiglu_fwd_kernel(
    const T* __restrict__ value, const T* __restrict__ gate, T* __restrict__ y, uint32_t chunks,
    tk::FastDiv per_row, int64_t vs, int64_t gs, int64_t ys) {
  // A workgroup pass covers kUnroll * kBlock consecutive chunks (one 4 KiB run per
  // wave and tensor), then the grid strides on.
  const uint32_t stride = gridDim.x * kBlock * kUnroll;
  for (uint32_t i0 = blockIdx.x * kBlock * kUnroll + threadIdx.x; i0 < chunks; i0 += stride) {
    float v[kUnroll][VEC], g[kUnroll][VEC];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const uint32_t i = i0 + u * kBlock;
      if (i >= chunks) break;
      const ChunkPos p = chunk_pos<VEC>(i, per_row);
      tk::load_vec_stream<T, VEC>(value + p.row * vs + p.col, v[u]);
      tk::load_vec_stream<T, VEC>(gate + p.row * gs + p.col, g[u]);
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const uint32_t i = i0 + u * kBlock;
      if (i >= chunks) break;
      const ChunkPos p = chunk_pos<VEC>(i, per_row);
#pragma unroll
      for (int j = 0; j < VEC; ++j) v[u][j] = v[u][j] * g[u][j] * stable_sigmoid(g[u][j]);
      tk::store_vec_stream<T, VEC>(y + p.row * ys + p.col, v[u]);
    }
  }
}

// dvalue = dy * silu(g); dgate = dy * value * sigmoid(g) * (1 + g * (1 - sigmoid(g)))
// (src/tklab/kernels/swiglu.py:82-108)
template <typename T, int VEC>
__global__ __launch_bounds__(kBlock) void swiglu_bwd_kernel(
    const T* __restrict__ dy, const T* __restrict__ value, const T* __restrict__ gate,
    T* __restrict__ dvalue, T* __restrict__ dgate, uint32_t chunks, tk::FastDiv per_row, int64_t dys,
    int64_t vs, int64_t gs, int64_t dvs, int64_t dgs) {
  // A workgroup pass covers kUnroll * kBlock consecutive chunks (one 4 KiB run per
  // wave and tensor), then the grid strides on.
  const uint32_t stride = gridDim.x * kBlock * kUnroll;
  for (uint32_t i0 = blockIdx.x * kBlock * kUnroll + threadIdx.x; i0 < chunks; i0 += stride) {
    float d[kUnroll][VEC], v[kUnroll][VEC], g[kUnroll][VEC];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const uint32_t i = i0 + u * kBlock;
      if (i >= chunks) break;
      const ChunkPos p = chunk_pos<VEC>(i, per_row);
      tk::load_vec_stream<T, VEC>(dy + p.row * dys + p.col, d[u]);
      tk::load_vec_stream<T, VEC>(value + p.row * vs + p.col, v[u]);
      tk::load_vec_stream<T, VEC>(gate + p.row * gs + p.col, g[u]);
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const uint32_t i = i0 + u * kBlock;
      if (i >= chunks) break;
      const ChunkPos p = chunk_pos<VEC>(i, per_row);
      float dv[VEC], dg[VEC];
#pragma unroll
      for (int j = 0; j < VEC; ++j) {
        const float sg = stable_sigmoid(g[u][j]);
        const float silu = g[u][j] * sg;
        const float dsilu = sg * (1.0f + g[u][j] * (1.0f - sg));
        dv[j] = d[u][j] * silu;
        dg[j] = d[u][j] * v[u][j] * dsilu;
      }
      tk::store_vec_stream<T, VEC>(dvalue + p.row * dvs + p.col, dv);
      tk::store_vec_stream<T, VEC>(dgate + p.row * dgs + p.col, dg);
    }
  }
}

// ------------------------------------------------------------------ RoPE

// y1 = x1*cos - x2*sin; y2 = x2*cos + x1*sin  (src/tklab/kernels/rope.py:44-73)
// kPositions: the tables are indexed by position, table row = row mod `positions.d`
// (rows of [batch, heads, seq, D] with positions 0 .. seq-1); otherwise by row.
template <bool kPositions>
__device__ __forceinline__ int table_row(int row, const tk::FastDiv& positions) {
  if constexpr (kPositions)
    return row - static_cast<int>(positions.div(row)) * static_cast<int>(positions.d);
  else
    return row;
}

// Table loads: non-temporal when the tables hold one row per x row (kStreamTables, each table
// row read once), plain when rows share them (a broadcast or position-indexed table).
template <typename T, int VEC, bool kStream>
__device__ __forceinline__ void load_table(const T* p, float* f) {
  if constexpr (kStream)
    tk::load_vec_stream<T, VEC>(p, f);
  else
    tk::load_vec<T, VEC>(p, f);
}

template <typename T, int VEC, bool kPositions = false, bool kStreamTables = false>
__global__ __launch_bounds__(kRopeBlock) void rope_fwd_kernel(
    const T* __restrict__ x, const T* __restrict__ cosv, const T* __restrict__ sinv,
    T* __restrict__ y, uint32_t chunks, tk::FastDiv per_row, int half, int64_t xs, int64_t cs,
    int64_t ss, int64_t ys, tk::FastDiv positions = tk::FastDiv()) {
  // A workgroup (one wave) pass covers kRopeUnroll * kRopeBlock consecutive chunks (a 2 KiB
  // run per tensor), then the grid strides on.
  constexpr uint32_t kPass = kRopeBlock * kRopeUnroll;
  const uint32_t stride = gridDim.x * kPass;
  for (uint32_t i0 = blockIdx.x * kPass + threadIdx.x; i0 < chunks; i0 += stride) {
    float x1[kRopeUnroll][VEC], x2[kRopeUnroll][VEC];
    float co[kRopeUnroll][VEC], si[kRopeUnroll][VEC];
#pragma unroll
    for (int u = 0; u < kRopeUnroll; ++u) {
      const uint32_t i = i0 + u * kRopeBlock;
      if (i >= chunks) break;
      const ChunkPos p = chunk_pos<VEC>(i, per_row);
      const T* xr = x + p.row * xs;
      const int tr = table_row<kPositions>(p.row, positions);
      tk::load_vec_stream<T, VEC>(xr + p.col, x1[u]);
      tk::load_vec_stream<T, VEC>(xr + half + p.col, x2[u]);
      load_table<T, VEC, kStreamTables>(cosv + tr * cs + p.col, co[u]);
      load_table<T, VEC, kStreamTables>(sinv + tr * ss + p.col, si[u]);
    }
#pragma unroll
    for (int u = 0; u < kRopeUnroll; ++u) {
      const uint32_t i = i0 + u * kRopeBlock;
      if (i >= chunks) break;
      const ChunkPos p = chunk_pos<VEC>(i, per_row);
      float y1[VEC], y2[VEC];
#pragma unroll
      for (int j = 0; j < VEC; ++j) {
        y1[j] = x1[u][j] * co[u][j] - x2[u][j] * si[u][j];
        y2[j] = x2[u][j] * co[u][j] + x1[u][j] * si[u][j];
      }
      T* yr = y + p.row * ys;
      tk::store_vec_stream<T, VEC>(yr + p.col, y1);
      tk::store_vec_stream<T, VEC>(yr + half + p.col, y2);
    }
  }
}

// dx1 = dy1*cos + dy2*sin; dx2 = dy2*cos - dy1*sin;
// dcos = dy1*x1 + dy2*x2; dsin = -dy1*x2 + dy2*x1  (src/tklab/kernels/rope.py:102-160)
template <typename T, int VEC, bool kPositions = false, bool kStreamTables = false>
__global__ __launch_bounds__(kRopeBlock) void rope_bwd_kernel(
    const T* __restrict__ dy, const T* __restrict__ x, const T* __restrict__ cosv,
    const T* __restrict__ sinv, T* __restrict__ dx, T* __restrict__ dcos, T* __restrict__ dsin,
    uint32_t chunks, tk::FastDiv per_row, int half, int64_t dys, int64_t xs, int64_t cs, int64_t ss,
    int64_t dxs, int64_t dcs, int64_t dss, tk::FastDiv positions = tk::FastDiv()) {
  const bool need_x = dcos != nullptr || dsin != nullptr;
  // A workgroup (one wave) pass covers kRopeUnroll * kRopeBlock consecutive chunks (a 2 KiB
  // run per tensor), then the grid strides on.
  constexpr uint32_t kPass = kRopeBlock * kRopeUnroll;
  const uint32_t stride = gridDim.x * kPass;
  for (uint32_t i0 = blockIdx.x * kPass + threadIdx.x; i0 < chunks; i0 += stride) {
    float d1[kRopeUnroll][VEC], d2[kRopeUnroll][VEC];
    float co[kRopeUnroll][VEC], si[kRopeUnroll][VEC];
#pragma unroll
    for (int u = 0; u < kRopeUnroll; ++u) {
      const uint32_t i = i0 + u * kRopeBlock;
      if (i >= chunks) break;
      const ChunkPos p = chunk_pos<VEC>(i, per_row);
      const T* dyr = dy + p.row * dys;
      const int tr = table_row<kPositions>(p.row, positions);
      tk::load_vec_stream<T, VEC>(dyr + p.col, d1[u]);
      tk::load_vec_stream<T, VEC>(dyr + half + p.col, d2[u]);
      load_table<T, VEC, kStreamTables>(cosv + tr * cs + p.col, co[u]);
      load_table<T, VEC, kStreamTables>(sinv + tr * ss + p.col, si[u]);
    }
#pragma unroll
    for (int u = 0; u < kRopeUnroll; ++u) {
      const uint32_t i = i0 + u * kRopeBlock;
      if (i >= chunks) break;
      const ChunkPos p = chunk_pos<VEC>(i, per_row);
      float o1[VEC], o2[VEC];
#pragma unroll
      for (int j = 0; j < VEC; ++j) {
        o1[j] = d1[u][j] * co[u][j] + d2[u][j] * si[u][j];
        o2[j] = d2[u][j] * co[u][j] - d1[u][j] * si[u][j];
      }
      T* dxr = dx + p.row * dxs;
      tk::store_vec_stream<T, VEC>(dxr + p.col, o1);
      tk::store_vec_stream<T, VEC>(dxr + half + p.col, o2);
      if (need_x) {
        float x1[VEC], x2[VEC];
        const T* xr = x + p.row * xs;
        tk::load_vec_stream<T, VEC>(xr + p.col, x1);
        tk::load_vec_stream<T, VEC>(xr + half + p.col, x2);
        if (dcos != nullptr) {
#pragma unroll
          for (int j = 0; j < VEC; ++j) o1[j] = d1[u][j] * x1[j] + d2[u][j] * x2[j];
          tk::store_vec_stream<T, VEC>(dcos + p.row * dcs + p.col, o1);
        }
        if (dsin != nullptr) {
#pragma unroll
          for (int j = 0; j < VEC; ++j) o2[j] = -d1[u][j] * x2[j] + d2[u][j] * x1[j];
          tk::store_vec_stream<T, VEC>(dsin + p.row * dss + p.col, o2);
        }
      }
    }
  }
}

// ------------------------------------------------------------------ row scaling

// y[r, c] = x[r, c] * scale[r], one float32 product rounded to T: folds a normalization
// weight into the rows of the projection that follows it (W'[k, :] = w[k] * W[k, :]).
template <typename T, int VEC>
__global__ __launch_bounds__(kBlock) void scale_rows_kernel(
    const T* __restrict__ x, const T* __restrict__ scale, T* __restrict__ y, uint32_t chunks,
    tk::FastDiv per_row, int64_t xs, int64_t ys) {
  const uint32_t stride = gridDim.x * kBlock * kUnroll;
  for (uint32_t i0 = blockIdx.x * kBlock * kUnroll + threadIdx.x; i0 < chunks; i0 += stride) {
    float v[kUnroll][VEC], sc[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const uint32_t i = i0 + u * kBlock;
      if (i >= chunks) break;
      const ChunkPos p = chunk_pos<VEC>(i, per_row);
      tk::load_vec_stream<T, VEC>(x + p.row * xs + p.col, v[u]);
      sc[u] = tk::to_f32(scale[p.row]);
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const uint32_t i = i0 + u * kBlock;
      if (i >= chunks) break;
      const ChunkPos p = chunk_pos<VEC>(i, per_row);
#pragma unroll
      for (int j = 0; j < VEC; ++j) v[u][j] = v[u][j] * sc[u];
      tk::store_vec_stream<T, VEC>(y + p.row * ys + p.col, v[u]);
    }
  }
}

bool vector_ok(int dtype, int64_t width, std::initializer_list<const void*> ptrs,
               std::initializer_list<int64_t> strides) {
  const int es = tk::elem_size(dtype);
  if (width % (16 / es) != 0) return false;
  for (const void* p : ptrs)
    if (p != nullptr && !tk::aligned16(p)) return false;
  for (int64_t s : strides)
    if ((s * es) % 16 != 0) return false;
  return true;
}

int check_problem(const char* what, int dtype, int64_t rows, int64_t width, int vec,
                  int64_t* chunks_per_row, int64_t* chunks) {
  if (!tk::valid_dtype(dtype)) return tk::fail("%s: unsupported dtype code %d", what, dtype);
  if (rows <= 0 || width <= 0) return tk::fail("%s: empty problem", what);
  *chunks_per_row = width / vec;
  if (__builtin_mul_overflow(rows, *chunks_per_row, chunks))
    return tk::fail("%s: problem too large", what);
  // Chunk indices are unsigned 32-bit: below INT32_MAX plus one grid stride (at most
  // kUnroll * kMaxBlocks * kBlock = 2^28), so any int32-addressable problem fits.
  static_assert(int64_t(INT32_MAX) + kUnroll * kMaxBlocks * kBlock <= int64_t(UINT32_MAX),
                "grid stride overflows the 32-bit chunk index");
  if (*chunks > INT32_MAX) return tk::fail("%s: problem too large", what);
  return 0;
}

}  // namespace

extern "C" int tk_swiglu_fwd(int dtype, const void* value, const void* gate, void* y, int64_t rows,
                             int64_t cols, int64_t value_row_stride, int64_t gate_row_stride,
                             int64_t y_row_stride, void* stream) {
  if (value == nullptr || gate == nullptr || y == nullptr) return tk::fail("swiglu_fwd: null pointer");
  if (!tk::row_strides_ok(rows, cols, {value_row_stride, gate_row_stride, y_row_stride}))
    return tk::fail("swiglu_fwd: strides must be non-negative and keep rows in range");
  // A fully contiguous problem is one long row: no per-chunk division work.
  if (rows > 0 && cols > 0 && value_row_stride == cols && gate_row_stride == cols &&
      y_row_stride == cols) {
    cols = tk::folded_extent(rows, cols);
    rows = 1;
    if (cols < 0) return tk::fail("swiglu_fwd: problem too large");
  }
  const bool vok = tk::valid_dtype(dtype) &&
                   vector_ok(dtype, cols, {value, gate, y},
                             {value_row_stride, gate_row_stride, y_row_stride});
  const int vec = vok ? 16 / tk::elem_size(dtype) : 1;
  int64_t per_row, chunks;
  if (check_problem("swiglu_fwd", dtype, rows, cols, vec, &per_row, &chunks)) return 1;
  const tk::FastDiv div(static_cast<uint32_t>(per_row));
  const Grid1D g = chunk_grid(chunks);
  hipStream_t s = tk::as_stream(stream);
  TK_DISPATCH_DTYPE(dtype, T,
    TK_DISPATCH_VEC(T, vok,
      hipLaunchKernelGGL((swiglu_fwd_kernel<T, VEC>), dim3(g.blocks), dim3(kBlock), 0, s,
                         static_cast<const T*>(value), static_cast<const T*>(gate),
                         static_cast<T*>(y), (int)chunks, div, value_row_stride,
                         gate_row_stride, y_row_stride)));
  return tk::check_launch("swiglu_fwd");
}

extern "C" int tk_swiglu_bwd(int dtype, const void* dy, const void* value, const void* gate,
                             void* dvalue, void* dgate, int64_t rows, int64_t cols,
                             int64_t dy_row_stride, int64_t value_row_stride,
                             int64_t gate_row_stride, int64_t dvalue_row_stride,
                             int64_t dgate_row_stride, void* stream) {
  if (dy == nullptr || value == nullptr || gate == nullptr || dvalue == nullptr || dgate == nullptr)
    return tk::fail("swiglu_bwd: null pointer");
  if (!tk::row_strides_ok(rows, cols,
                          {dy_row_stride, value_row_stride, gate_row_stride, dvalue_row_stride,
                           dgate_row_stride}))
    return tk::fail("swiglu_bwd: strides must be non-negative and keep rows in range");
  if (rows > 0 && cols > 0 && dy_row_stride == cols && value_row_stride == cols &&
      gate_row_stride == cols && dvalue_row_stride == cols && dgate_row_stride == cols) {
    cols = tk::folded_extent(rows, cols);
    rows = 1;
    if (cols < 0) return tk::fail("swiglu_bwd: problem too large");
  }
  const bool vok = tk::valid_dtype(dtype) &&
                   vector_ok(dtype, cols, {dy, value, gate, dvalue, dgate},
                             {dy_row_stride, value_row_stride, gate_row_stride,
                              dvalue_row_stride, dgate_row_stride});
  const int vec = vok ? 16 / tk::elem_size(dtype) : 1;
  int64_t per_row, chunks;
  if (check_problem("swiglu_bwd", dtype, rows, cols, vec, &per_row, &chunks)) return 1;
  const tk::FastDiv div(static_cast<uint32_t>(per_row));
  const Grid1D g = chunk_grid(chunks);
  hipStream_t s = tk::as_stream(stream);
  TK_DISPATCH_DTYPE(dtype, T,
    TK_DISPATCH_VEC(T, vok,
      hipLaunchKernelGGL((swiglu_bwd_kernel<T, VEC>), dim3(g.blocks), dim3(kBlock), 0, s,
                         static_cast<const T*>(dy), static_cast<const T*>(value),
                         static_cast<const T*>(gate), static_cast<T*>(dvalue),
                         static_cast<T*>(dgate), (int)chunks, div, dy_row_stride,
                         value_row_stride, gate_row_stride, dvalue_row_stride,
                         dgate_row_stride)));
  return tk::check_launch("swiglu_bwd");
}

extern "C" int tk_rope_fwd(int dtype, const void* x, const void* cos, const void* sin, void* y,
                           int64_t rows, int64_t half_dim, int64_t x_row_stride,
                           int64_t cos_row_stride, int64_t sin_row_stride, int64_t y_row_stride,
                           void* stream) {
  if (x == nullptr || cos == nullptr || sin == nullptr || y == nullptr)
    return tk::fail("rope_fwd: null pointer");
  if (!tk::row_strides_ok(rows, 2 * half_dim,
                          {x_row_stride, cos_row_stride, sin_row_stride, y_row_stride}))
    return tk::fail("rope_fwd: strides must be non-negative and keep rows in range");
  // The second half starts half_dim elements in, so half_dim joins the strides.
  const bool vok = tk::valid_dtype(dtype) &&
                   vector_ok(dtype, half_dim, {x, cos, sin, y},
                             {x_row_stride, cos_row_stride, sin_row_stride, y_row_stride});
  const int vec = vok ? 16 / tk::elem_size(dtype) : 1;
  int64_t per_row, chunks;
  if (check_problem("rope_fwd", dtype, rows, half_dim, vec, &per_row, &chunks)) return 1;
  const tk::FastDiv div(static_cast<uint32_t>(per_row));
  const Grid1D g = chunk_grid(chunks, kRopeBlock, kRopeUnroll);
  hipStream_t s = tk::as_stream(stream);
  const bool stream_tables = cos_row_stride != 0 && sin_row_stride != 0;
  TK_DISPATCH_DTYPE(dtype, T,
    TK_DISPATCH_VEC(T, vok,
      if (stream_tables)
        hipLaunchKernelGGL((rope_fwd_kernel<T, VEC, false, true>), dim3(g.blocks), dim3(kRopeBlock),
                           0, s, static_cast<const T*>(x), static_cast<const T*>(cos),
                           static_cast<const T*>(sin), static_cast<T*>(y), (int)chunks, div,
                           (int)half_dim, x_row_stride, cos_row_stride, sin_row_stride,
                           y_row_stride);
      else
        hipLaunchKernelGGL((rope_fwd_kernel<T, VEC>), dim3(g.blocks), dim3(kRopeBlock), 0, s,
                           static_cast<const T*>(x), static_cast<const T*>(cos),
                           static_cast<const T*>(sin), static_cast<T*>(y), (int)chunks, div,
                           (int)half_dim, x_row_stride, cos_row_stride, sin_row_stride,
                           y_row_stride)));
  return tk::check_launch("rope_fwd");
}

extern "C" int tk_rope_bwd(int dtype, const void* dy, const void* x, const void* cos,
                           const void* sin, void* dx, void* dcos, void* dsin, int64_t rows,
                           int64_t half_dim, int64_t dy_row_stride, int64_t x_row_stride,
                           int64_t cos_row_stride, int64_t sin_row_stride, int64_t dx_row_stride,
                           int64_t dcos_row_stride, int64_t dsin_row_stride, void* stream) {
  if (dy == nullptr || cos == nullptr || sin == nullptr || dx == nullptr)
    return tk::fail("rope_bwd: null pointer");
  const bool need_x = dcos != nullptr || dsin != nullptr;
  if (need_x && x == nullptr) return tk::fail("rope_bwd: x is required for dcos/dsin");
  if (!tk::row_strides_ok(rows, 2 * half_dim,
                          {dy_row_stride, need_x ? x_row_stride : 0, cos_row_stride,
                           sin_row_stride, dx_row_stride, dcos ? dcos_row_stride : 0,
                           dsin ? dsin_row_stride : 0}))
    return tk::fail("rope_bwd: strides must be non-negative and keep rows in range");
  const bool vok =
      tk::valid_dtype(dtype) &&
      vector_ok(dtype, half_dim, {dy, need_x ? x : nullptr, cos, sin, dx, dcos, dsin},
                {dy_row_stride, need_x ? x_row_stride : 0, cos_row_stride, sin_row_stride,
                 dx_row_stride, dcos ? dcos_row_stride : 0, dsin ? dsin_row_stride : 0});
  const int vec = vok ? 16 / tk::elem_size(dtype) : 1;
  int64_t per_row, chunks;
  if (check_problem("rope_bwd", dtype, rows, half_dim, vec, &per_row, &chunks)) return 1;
  const tk::FastDiv div(static_cast<uint32_t>(per_row));
  const Grid1D g = chunk_grid(chunks, kRopeBlock, kRopeUnroll);
  hipStream_t s = tk::as_stream(stream);
  const bool stream_tables = cos_row_stride != 0 && sin_row_stride != 0;
  TK_DISPATCH_DTYPE(dtype, T,
    TK_DISPATCH_VEC(T, vok,
      if (stream_tables)
        hipLaunchKernelGGL((rope_bwd_kernel<T, VEC, false, true>), dim3(g.blocks), dim3(kRopeBlock),
                           0, s, static_cast<const T*>(dy), static_cast<const T*>(x),
                           static_cast<const T*>(cos), static_cast<const T*>(sin),
                           static_cast<T*>(dx), static_cast<T*>(dcos), static_cast<T*>(dsin),
                           (int)chunks, div, (int)half_dim, dy_row_stride, x_row_stride,
                           cos_row_stride, sin_row_stride, dx_row_stride, dcos_row_stride,
                           dsin_row_stride);
      else
        hipLaunchKernelGGL((rope_bwd_kernel<T, VEC>), dim3(g.blocks), dim3(kRopeBlock), 0, s,
                           static_cast<const T*>(dy), static_cast<const T*>(x),
                           static_cast<const T*>(cos), static_cast<const T*>(sin),
                           static_cast<T*>(dx), static_cast<T*>(dcos), static_cast<T*>(dsin),
                           (int)chunks, div, (int)half_dim, dy_row_stride, x_row_stride,
                           cos_row_stride, sin_row_stride, dx_row_stride, dcos_row_stride,
                           dsin_row_stride)));
  return tk::check_launch("rope_bwd");
}

extern "C" int tk_scale_rows(int dtype, const void* x, const void* scale, void* y, int64_t rows,
                             int64_t cols, int64_t x_row_stride, int64_t y_row_stride,
                             void* stream) {
  if (x == nullptr || scale == nullptr || y == nullptr) return tk::fail("scale_rows: null pointer");
  if (!tk::row_strides_ok(rows, cols, {x_row_stride, y_row_stride}))
    return tk::fail("scale_rows: strides must be non-negative and keep rows in range");
  const bool vok = tk::valid_dtype(dtype) &&
                   vector_ok(dtype, cols, {x, y}, {x_row_stride, y_row_stride});
  const int vec = vok ? 16 / tk::elem_size(dtype) : 1;
  int64_t per_row, chunks;
  if (check_problem("scale_rows", dtype, rows, cols, vec, &per_row, &chunks)) return 1;
  const tk::FastDiv div(static_cast<uint32_t>(per_row));
  const Grid1D g = chunk_grid(chunks);
  hipStream_t s = tk::as_stream(stream);
  TK_DISPATCH_DTYPE(dtype, T,
    TK_DISPATCH_VEC(T, vok,
      hipLaunchKernelGGL((scale_rows_kernel<T, VEC>), dim3(g.blocks), dim3(kBlock), 0, s,
                         static_cast<const T*>(x), static_cast<const T*>(scale),
                         static_cast<T*>(y), (int)chunks, div, x_row_stride, y_row_stride)));
  return tk::check_launch("scale_rows");
}

// RoPE over rows of [batch, heads, seq, D] (row stride x_row_stride / y_row_stride)
// with position-indexed tables cos/sin [>= seq][D/2]: row r uses table row r mod seq.
// Forward (inverse = false) or the input gradient (inverse = true: RoPE with -sin).
extern "C" int tk_rope_positions(int dtype, const void* x, const void* cos, const void* sin,
                                 void* y, int64_t rows, int64_t seq, int64_t half_dim,
                                 int64_t x_row_stride, int64_t table_row_stride,
                                 int64_t y_row_stride, int inverse, void* stream) {
  if (x == nullptr || cos == nullptr || sin == nullptr || y == nullptr)
    return tk::fail("rope_positions: null pointer");
  if (!tk::row_strides_ok(rows, 2 * half_dim, {x_row_stride, table_row_stride, y_row_stride}))
    return tk::fail("rope_positions: strides must be non-negative and keep rows in range");
  if (seq <= 0 || seq > rows || rows % seq != 0)
    return tk::fail("rope_positions: rows must be a positive multiple of seq");
  const bool vok = tk::valid_dtype(dtype) &&
                   vector_ok(dtype, half_dim, {x, cos, sin, y},
                             {x_row_stride, table_row_stride, y_row_stride});
  const int vec = vok ? 16 / tk::elem_size(dtype) : 1;
  int64_t per_row, chunks;
  if (check_problem("rope_positions", dtype, rows, half_dim, vec, &per_row, &chunks)) return 1;
  const tk::FastDiv div(static_cast<uint32_t>(per_row));
  const tk::FastDiv positions(static_cast<uint32_t>(seq));
  const Grid1D g = chunk_grid(chunks, kRopeBlock, kRopeUnroll);
  hipStream_t s = tk::as_stream(stream);
  if (inverse) {
    TK_DISPATCH_DTYPE(dtype, T,
      TK_DISPATCH_VEC(T, vok,
        hipLaunchKernelGGL((rope_bwd_kernel<T, VEC, true>), dim3(g.blocks), dim3(kRopeBlock), 0, s,
                           static_cast<const T*>(x), static_cast<const T*>(nullptr),
                           static_cast<const T*>(cos), static_cast<const T*>(sin),
                           static_cast<T*>(y), static_cast<T*>(nullptr),
                           static_cast<T*>(nullptr), (int)chunks, div, (int)half_dim,
                           x_row_stride, 0, table_row_stride, table_row_stride, y_row_stride, 0,
                           0, positions)));
  } else {
    TK_DISPATCH_DTYPE(dtype, T,
      TK_DISPATCH_VEC(T, vok,
        hipLaunchKernelGGL((rope_fwd_kernel<T, VEC, true>), dim3(g.blocks), dim3(kRopeBlock), 0, s,
                           static_cast<const T*>(x), static_cast<const T*>(cos),
                           static_cast<const T*>(sin), static_cast<T*>(y), (int)chunks, div,
                           (int)half_dim, x_row_stride, table_row_stride, table_row_stride,
                           y_row_stride, positions)));
  }
  return tk::check_launch("rope_positions");
}
