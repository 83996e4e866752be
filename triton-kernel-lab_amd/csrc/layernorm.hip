// LayerNorm forward and deterministic two-stage backward (registry kernel
// outside the transformer hot path; src/tklab/kernels/layer_norm.py:37-174
// defines the math). Same structure as the RMSNorm kernels in rmsnorm.hip:
// packed rows in registers, one group per workgroup owning rows
// r % group_size == g, float32 partials folded in a fixed order, no locks.
//   forward:  mean = sum(x)/n, c = x - mean, rstd = 1/sqrt(sum(c*c)/n + eps),
//             y = c * rstd * w + b
//   backward: x_hat = (x - mean) * rstd, g = w * dy,
//             dx = rstd * (g - sum(g)/n - x_hat * sum(g*x_hat)/n),
//             dw = sum_rows dy * x_hat, db = sum_rows dy
#include "rows.hpp"

#pragma clang fp contract(off)

namespace {

constexpr int kBlock = 256;

template <typename T, int VEC, int RT, int VALS>
__global__ __launch_bounds__(RT >= kBlock ? RT : kBlock) void layernorm_fwd_kernel(
    const T* __restrict__ x, const T* __restrict__ weight, const T* __restrict__ bias,
    T* __restrict__ y, float* __restrict__ mean_out, float* __restrict__ rstd_out, int rows,
    int cols, int64_t x_stride, int64_t y_stride, float eps) {
  constexpr int SLOTS = RT >= kBlock ? 1 : kBlock / RT;
  using Row = tk::RawRow<T, VEC, RT, VALS>;
  __shared__ float scratch[RT / 64];
  const int lane = threadIdx.x % RT;
  const int row = blockIdx.x * SLOTS + threadIdx.x / RT;
  if (row >= rows) return;  // SLOTS > 1 only for barrier-free single-wave rows

  Row xv;
  xv.load(x + row * x_stride, cols, lane);
  float sum = 0.f;
#pragma unroll
  for (int e = 0; e < VALS; ++e) sum += xv.get(e);
  sum = tk::group_allreduce<RT>(sum, tk::SumOp{}, scratch);
  const float mean = sum / static_cast<float>(cols);
  float var = 0.f;
#pragma unroll
  for (int e = 0; e < VALS; ++e) {
    const float c = tk::row_column<VEC, RT>(e, lane) < cols ? xv.get(e) - mean : 0.f;
    var += c * c;
  }
  var = tk::group_allreduce<RT>(var, tk::SumOp{}, scratch);
  const float rstd = 1.0f / sqrtf(var / static_cast<float>(cols) + eps);
  Row wv, bv;
  wv.load(weight, cols, lane);
  bv.load(bias, cols, lane);
#pragma unroll
  for (int e = 0; e < VALS; ++e) xv.set(e, (xv.get(e) - mean) * rstd * wv.get(e) + bv.get(e));
  xv.store(y + row * y_stride, cols, lane);
  if (lane == 0) {
    if (mean_out != nullptr) mean_out[row] = mean;
    if (rstd_out != nullptr) rstd_out[row] = rstd;
  }
}

template <int RT>
constexpr int bwd_block() { return RT == 64 ? 256 : RT; }

template <typename T, int VEC, int RT, int VALS>
__global__ __launch_bounds__(bwd_block<RT>()) void layernorm_bwd_stage1_kernel(
    T* __restrict__ dx, const T* __restrict__ dy, float* __restrict__ partial_dw,
    float* __restrict__ partial_db, const T* __restrict__ x, const T* __restrict__ weight,
    const float* __restrict__ mean, const float* __restrict__ rstd, int32_t* __restrict__ counts,
    int rows, int cols, int64_t x_stride, int64_t dy_stride, int64_t dx_stride, int group_size) {
  constexpr int SLOTS = bwd_block<RT>() / RT;
  constexpr int WIDTH = RT * VALS;
  constexpr bool ACC_LDS = 2 * SLOTS * WIDTH * 4 <= 131072;
  using Row = tk::RawRow<T, VEC, RT, VALS>;
  __shared__ float acc_lds[ACC_LDS ? 2 * SLOTS * WIDTH : 1];
  __shared__ float scratch[RT / 64];

  const int group = blockIdx.x;
  const int slot = threadIdx.x / RT;
  const int lane = threadIdx.x % RT;
  const int group_rows = (rows - 1 - group) / group_size + 1;
  const int iters = (group_rows + SLOTS - 1) / SLOTS;

  float acc_w[ACC_LDS ? 1 : VALS], acc_b[ACC_LDS ? 1 : VALS];
  float* lw = acc_lds + slot * WIDTH;
  float* lb = acc_lds + (SLOTS + slot) * WIDTH;
#pragma unroll
  for (int e = 0; e < VALS; ++e) {
    if constexpr (ACC_LDS) {
      lw[tk::row_column<VEC, RT>(e, lane)] = 0.f;
      lb[tk::row_column<VEC, RT>(e, lane)] = 0.f;
    } else {
      acc_w[e] = acc_b[e] = 0.f;
    }
  }

  for (int it = 0; it < iters; ++it) {
    const int k = it * SLOTS + slot;
    const bool valid = k < group_rows;
    const int64_t row = static_cast<int64_t>(group) + static_cast<int64_t>(k) * group_size;
    Row xv, dv, wv;
    float mu = 0.f, r = 0.f;
    if (valid) {
      xv.load(x + row * x_stride, cols, lane);
      dv.load(dy + row * dy_stride, cols, lane);
      mu = mean[row];
      r = rstd[row];
    } else {
      xv.load(x, 0, lane);
      dv.load(dy, 0, lane);
    }
    wv.load(weight, cols, lane);
    float s1 = 0.f, s2 = 0.f;
#pragma unroll
    for (int e = 0; e < VALS; ++e) {
      const bool in = tk::row_column<VEC, RT>(e, lane) < cols;
      const float x_hat = in ? (xv.get(e) - mu) * r : 0.f;
      const float d = dv.get(e);
      const float g = wv.get(e) * d;
      if constexpr (ACC_LDS) {
        lw[tk::row_column<VEC, RT>(e, lane)] += d * x_hat;
        lb[tk::row_column<VEC, RT>(e, lane)] += d;
      } else {
        acc_w[e] += d * x_hat;
        acc_b[e] += d;
      }
      s1 += g;
      s2 += g * x_hat;
    }
    s1 = tk::group_allreduce<RT>(s1, tk::SumOp{}, scratch);
    s2 = tk::group_allreduce<RT>(s2, tk::SumOp{}, scratch);
    const float m1 = s1 / static_cast<float>(cols);
    const float m2 = s2 / static_cast<float>(cols);
    if (valid) {
#pragma unroll
      for (int e = 0; e < VALS; ++e) {
        const float x_hat = (xv.get(e) - mu) * r;
        const float g = wv.get(e) * dv.get(e);
        xv.set(e, r * (g - m1 - x_hat * m2));
      }
      xv.store(dx + row * dx_stride, cols, lane);
    }
  }

  float* ow = partial_dw + static_cast<int64_t>(group) * cols;
  float* ob = partial_db + static_cast<int64_t>(group) * cols;
  if constexpr (!ACC_LDS) {
#pragma unroll
    for (int e = 0; e < VALS; ++e) {
      const int c = tk::row_column<VEC, RT>(e, lane);
      if (c < cols) {
        ow[c] = acc_w[e];
        ob[c] = acc_b[e];
      }
    }
  } else {
    __syncthreads();
    for (int c = threadIdx.x; c < cols; c += bwd_block<RT>()) {
      float tw = acc_lds[c], tb = acc_lds[SLOTS * WIDTH + c];
#pragma unroll
      for (int s2 = 1; s2 < SLOTS; ++s2) {
        tw += acc_lds[s2 * WIDTH + c];
        tb += acc_lds[(SLOTS + s2) * WIDTH + c];
      }
      ow[c] = tw;
      ob[c] = tb;
    }
  }
  if (threadIdx.x == 0) counts[group] = 1;
}

template <typename T>
__global__ __launch_bounds__(256) void layernorm_bwd_stage2_kernel(
    const float* __restrict__ pw, const float* __restrict__ pb, T* __restrict__ dw,
    T* __restrict__ db, int group_count, int cols) {
  const int c = blockIdx.x * 256 + threadIdx.x;
  if (c >= cols) return;
  float sw = 0.f, sb = 0.f;
  for (int g = 0; g < group_count; ++g) {
    sw += pw[static_cast<int64_t>(g) * cols + c];
    sb += pb[static_cast<int64_t>(g) * cols + c];
  }
  dw[c] = tk::from_f32<T>(sw);
  db[c] = tk::from_f32<T>(sb);
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
  const int max_vals = vector_ok ? 128 / tk::elem_size(dtype) : 32;
  if (cols * tk::elem_size(dtype) > 65536 || !tk::pick_row_shape(cols, shape, max_vals))
    return tk::fail("%s: feature row exceeds the 65536-byte fused limit", what);
  return 0;
}

}  // namespace

extern "C" int tk_layernorm_fwd(int dtype, const void* x, const void* weight, const void* bias,
                                void* y, float* mean, float* rstd, int64_t rows, int64_t cols,
                                int64_t x_row_stride, int64_t y_row_stride, float eps,
                                void* stream) {
  if (x == nullptr || weight == nullptr || bias == nullptr || y == nullptr)
    return tk::fail("layernorm_fwd: null pointer");
  if (!tk::row_strides_ok(rows, cols, {x_row_stride, y_row_stride}))
    return tk::fail("layernorm_fwd: strides must be non-negative and keep rows in range");
  if (!(eps > 0.f)) return tk::fail("layernorm_fwd: eps must be finite and positive");
  const bool vok = tk::valid_dtype(dtype) &&
                   rows_vector_ok(dtype, cols, {x, weight, bias, y}, {x_row_stride, y_row_stride});
  tk::RowShape shape;
  if (check_rows("layernorm_fwd", dtype, rows, cols, vok, &shape)) return 1;
  const int slots = shape.rt >= kBlock ? 1 : kBlock / shape.rt;
  const dim3 grid(static_cast<unsigned>(tk::cdiv(rows, slots)));
  const dim3 block(shape.rt >= kBlock ? shape.rt : kBlock);
  hipStream_t s = tk::as_stream(stream);
  TK_DISPATCH_DTYPE(dtype, T,
    TK_DISPATCH_VEC(T, vok,
      TK_DISPATCH_ROW_SHAPE(shape,
        hipLaunchKernelGGL((layernorm_fwd_kernel<T, VEC, RT, VALS>), grid, block, 0, s,
                           (const T*)x, (const T*)weight, (const T*)bias, (T*)y, mean, rstd,
                           (int)rows, (int)cols, x_row_stride, y_row_stride, eps))));
  return tk::check_launch("layernorm_fwd");
}

extern "C" int tk_layernorm_bwd_stage1(int dtype, void* dx, const void* dy, float* partial_dw,
                                       float* partial_db, const void* x, const void* weight,
                                       const float* mean, const float* rstd, int32_t* locks,
                                       int64_t rows, int64_t cols, int64_t x_row_stride,
                                       int64_t dy_row_stride, int64_t dx_row_stride,
                                       int64_t group_size, void* stream) {
  if (!dx || !dy || !partial_dw || !partial_db || !x || !weight || !mean || !rstd || !locks)
    return tk::fail("layernorm_bwd_stage1: null pointer");
  if (!tk::row_strides_ok(rows, cols, {x_row_stride, dy_row_stride, dx_row_stride}))
    return tk::fail("layernorm_bwd_stage1: strides must be non-negative and keep rows in range");
  if (group_size <= 0 || group_size > INT32_MAX)
    return tk::fail("layernorm_bwd_stage1: group_size must be positive");
  const bool vok = tk::valid_dtype(dtype) &&
                   rows_vector_ok(dtype, cols, {dx, dy, x, weight},
                                  {x_row_stride, dy_row_stride, dx_row_stride});
  tk::RowShape shape;
  if (check_rows("layernorm_bwd_stage1", dtype, rows, cols, vok, &shape)) return 1;
  const int64_t group_count = group_size < rows ? group_size : rows;
  hipStream_t s = tk::as_stream(stream);
  TK_DISPATCH_DTYPE(dtype, T,
    TK_DISPATCH_VEC(T, vok,
      TK_DISPATCH_ROW_SHAPE(shape,
        hipLaunchKernelGGL((layernorm_bwd_stage1_kernel<T, VEC, RT, VALS>),
                           dim3(static_cast<unsigned>(group_count)), dim3(bwd_block<RT>()), 0, s,
                           (T*)dx, (const T*)dy, partial_dw, partial_db, (const T*)x,
                           (const T*)weight, mean, rstd, locks + group_size, (int)rows, (int)cols,
                           x_row_stride, dy_row_stride, dx_row_stride, (int)group_size))));
  return tk::check_launch("layernorm_bwd_stage1");
}

extern "C" int tk_layernorm_bwd_stage2(int dtype, const float* partial_dw, const float* partial_db,
                                       void* dw, void* db, int64_t group_count, int64_t cols,
                                       void* stream) {
  if (!tk::valid_dtype(dtype)) return tk::fail("layernorm_bwd_stage2: unsupported dtype code %d", dtype);
  if (!partial_dw || !partial_db || !dw || !db) return tk::fail("layernorm_bwd_stage2: null pointer");
  if (group_count <= 0 || cols <= 0 || group_count > INT32_MAX || cols > INT32_MAX ||
      group_count * cols > INT32_MAX)
    return tk::fail("layernorm_bwd_stage2: bad partial shape");
  hipStream_t s = tk::as_stream(stream);
  TK_DISPATCH_DTYPE(dtype, T,
    hipLaunchKernelGGL((layernorm_bwd_stage2_kernel<T>), dim3((unsigned)tk::cdiv(cols, 256)),
                       dim3(256), 0, s, partial_dw, partial_db, (T*)dw, (T*)db, (int)group_count,
                       (int)cols));
  return tk::check_launch("layernorm_bwd_stage2");
}
