// Calibration kernels: the measured roofs the hot-path kernels are priced
// against, beside the published peaks.
//
//   tk_roof_copy  — device-to-device copy at the HBM streaming limit: 16-byte
//                   non-temporal accesses, each thread issuing the loads of kUnroll
//                   chunks of a contiguous 4 KiB-per-wave run before its stores (the
//                   access shape and cache policy of the elementwise kernels).
//   tk_roof_stream — R reads and W writes per chunk position (R:W of 1:0, 0:1, 1:1, 2:1,
//                   3:1, 2:2, 3:2), one 8 or 16 KiB tile of every array per workgroup,
//                   stores non-temporal or sc1: the HBM roof is the best of these mixes, since
//                   reads and writes turn the HBM bus around differently and the kernels
//                   here run several mixes.
//   tk_roof_mfma  — dense v_mfma_f32_16x16x32_{f16,bf16} issue with no memory
//                   traffic: each wave keeps 2 * kChains independent 16x16 float32
//                   accumulators so back-to-back MFMAs never wait on one
//                   another, and writes one float per wave at the end so none of
//                   the work can be removed. 16x16x32 rather than 32x32x16: with
//                   random operands the clock is power-limited, and the 16x16
//                   shape sustains ~7% more FLOP/s (1.90 vs 1.78 PFLOP/s bf16).
//
// Neither has a counterpart in the reference; they exist so that achieved
// GB/s and TFLOP/s can be stated as fractions of what this GPU sustains at the
// clocks it runs at under load, not only of the published peaks.
#include "tk_common.hpp"

namespace {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef int i32x4 __attribute__((ext_vector_type(4)));

// ------------------------------------------------------------------ copy

constexpr int kCopyBlock = 256;
constexpr int kCopyUnroll = 4;
constexpr int64_t kCopyMaxBlocks = 8192;

__global__ __launch_bounds__(kCopyBlock) void roof_copy_kernel(const i32x4* __restrict__ src,
                                                               i32x4* __restrict__ dst,
                                                               int64_t chunks) {
  constexpr int64_t kPass = int64_t(kCopyBlock) * kCopyUnroll;
  for (int64_t base = int64_t(blockIdx.x) * kPass; base < chunks;
       base += int64_t(gridDim.x) * kPass) {
    const int64_t i0 = base + threadIdx.x;
    i32x4 v[kCopyUnroll];
#pragma unroll
    for (int u = 0; u < kCopyUnroll; ++u) {
      const int64_t i = i0 + int64_t(u) * kCopyBlock;
      if (i < chunks) v[u] = __builtin_nontemporal_load(src + i);
    }
#pragma unroll
    for (int u = 0; u < kCopyUnroll; ++u) {
      const int64_t i = i0 + int64_t(u) * kCopyBlock;
      if (i < chunks) __builtin_nontemporal_store(v[u], dst + i);
    }
  }
}

// R arrays of `chunks` 16-byte chunks read, W arrays written; written chunk i is
// {i, 0, 0, 0} xor the chunks read at position i. The arrays are cut into tiles of 256 * U
// chunks (4 U KiB per array); workgroup b takes tiles b, b + G, ... (G = gridDim.x: one
// tile per workgroup when the grid covers the arrays, else a grid-stride walk), read with
// non-temporal buffer loads and written with cache policy CPOL; the buffer extent ends at the array's
// end, so a partial last tile loads zeros past it and drops those stores. With W == 0
// the xor of everything a thread read is stored only when it equals `sentinel`, which
// never happens for the calibration data but keeps every load live.
template <int R, int W, int CPOL, int U>
__global__ __launch_bounds__(kCopyBlock) void roof_stream_kernel(const i32x4* __restrict__ src,
                                                                 i32x4* __restrict__ dst,
                                                                 int64_t chunks, int sentinel) {
  constexpr int64_t kTile = int64_t(kCopyBlock) * U;
  i32x4 sink = i32x4{0, 0, 0, 0};
  for (int64_t base = int64_t(blockIdx.x) * kTile; base < chunks;
       base += int64_t(gridDim.x) * kTile) {
    const int64_t left = chunks - base;
    const uint32_t extent = uint32_t((left < kTile ? left : kTile) * 16);
    i32x4 v[U];
#pragma unroll
    for (int u = 0; u < U; ++u)
      v[u] = i32x4{int(base + u * kCopyBlock + threadIdx.x), 0, 0, 0};
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
          const_cast<i32x4*>(src + int64_t(r) * chunks + base), (short)0, extent, 0x00020000);
#pragma unroll
      for (int u = 0; u < U; ++u)
        v[u] ^= __builtin_bit_cast(
            i32x4, __builtin_amdgcn_raw_buffer_load_b128(
                       rs, uint32_t((u * kCopyBlock + threadIdx.x) * 16), 0, 2));
    }
    if constexpr (W == 0) {
#pragma unroll
      for (int u = 0; u < U; ++u) sink ^= v[u];
    } else {
#pragma unroll
      for (int w = 0; w < W; ++w) {
        const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
            dst + int64_t(w) * chunks + base, (short)0, extent, 0x00020000);
#pragma unroll
        for (int u = 0; u < U; ++u)
          __builtin_amdgcn_raw_buffer_store_b128(
              v[u], rs, uint32_t((u * kCopyBlock + threadIdx.x) * 16), 0, CPOL);
      }
    }
  }
  if constexpr (W == 0) {
    if (sink[0] == sentinel && sink[1] == sentinel && sink[2] == sentinel && sink[3] == sentinel)
      dst[blockIdx.x * kCopyBlock + threadIdx.x] = sink;
  }
}

// ------------------------------------------------------------------ MFMA

constexpr int kMfmaBlock = 256;  // four waves, one per SIMD
constexpr int kChains = 8;       // independent accumulators per wave

template <typename T>
struct RoofMma;
template <>
struct RoofMma<_Float16> {
  __device__ __forceinline__ static f32x4 run(i32x4 a, i32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
};
template <>
struct RoofMma<__bf16> {
  __device__ __forceinline__ static f32x4 run(i32x4 a, i32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
};

template <typename T>
__global__ __launch_bounds__(kMfmaBlock) void roof_mfma_kernel(float* __restrict__ out,
                                                               int iters) {
  const int wave = (blockIdx.x * kMfmaBlock + threadIdx.x) >> 6;
  const int lane = threadIdx.x & 63;
  // Operands with random sign and mantissa bits (magnitudes in [0.5, 1) for f16,
  // [2^-8, 2^-7) for bf16), a different pair for every chain, so the multiplier
  // inputs toggle the way real data does; constant operands draw less power and
  // let the clock run higher than any GEMM can.
  i32x4 a[kChains], b[kChains];
  uint32_t h = 0x9E3779B9u * static_cast<uint32_t>(wave * 64 + lane + 1);
  auto next = [&h]() {  // xorshift32
    h ^= h << 13;
    h ^= h >> 17;
    h ^= h << 5;
    return static_cast<int>((h & 0x83FF83FFu) | 0x38003800u);
  };
#pragma unroll
  for (int c = 0; c < kChains; ++c) {
    a[c] = i32x4{next(), next(), next(), next()};
    b[c] = i32x4{next(), next(), next(), next()};
  }
  // One iteration is 2 * kChains MFMAs of 16 x 16 x 32 (kChains * 32768 FLOP).
  f32x4 acc[2 * kChains];
#pragma unroll
  for (int c = 0; c < 2 * kChains; ++c) acc[c] = f32x4{};
  // kChains iterations per trip, so that every operand index is static.
  for (int it = 0; it < iters; it += kChains) {
#pragma unroll
    for (int r = 0; r < kChains; ++r)
#pragma unroll
      for (int c = 0; c < 2 * kChains; ++c)
        acc[c] = RoofMma<T>::run(a[c & (kChains - 1)], b[(c + r) & (kChains - 1)], acc[c]);
  }
  float s = 0.f;
#pragma unroll
  for (int c = 0; c < 2 * kChains; ++c)
#pragma unroll
    for (int r = 0; r < 4; ++r) s += acc[c][r];
  if (lane == 0) out[wave] = s;
}

}  // namespace

extern "C" int tk_roof_copy(const void* src, void* dst, int64_t bytes, void* stream) {
  if (bytes < 0 || bytes % 16 != 0)
    return tk::fail("tk_roof_copy: bytes must be a non-negative multiple of 16 (got %lld)",
                    static_cast<long long>(bytes));
  if (bytes == 0) return 0;
  if (src == nullptr || dst == nullptr || !tk::aligned16(src) || !tk::aligned16(dst))
    return tk::fail("tk_roof_copy: src and dst must be non-null and 16-byte aligned");
  const int64_t chunks = bytes / 16;
  int64_t blocks = tk::cdiv(chunks, int64_t(kCopyBlock) * kCopyUnroll);
  if (blocks > kCopyMaxBlocks) blocks = kCopyMaxBlocks;
  hipLaunchKernelGGL(roof_copy_kernel, dim3(static_cast<unsigned>(blocks)), dim3(kCopyBlock), 0,
                     tk::as_stream(stream), static_cast<const i32x4*>(src),
                     static_cast<i32x4*>(dst), chunks);
  return tk::check_launch("tk_roof_copy");
}

extern "C" int tk_roof_stream(const void* src, void* dst, int64_t bytes, int reads, int writes,
                              int store_policy, int tile_kib, int64_t max_workgroups,
                              void* stream) {
  if (bytes <= 0 || bytes % 16 != 0)
    return tk::fail("tk_roof_stream: bytes must be a positive multiple of 16 (got %lld)",
                    static_cast<long long>(bytes));
  if (src == nullptr || dst == nullptr || !tk::aligned16(src) || !tk::aligned16(dst))
    return tk::fail("tk_roof_stream: src and dst must be non-null and 16-byte aligned");
  if (store_policy != 0 && store_policy != 1)
    return tk::fail("tk_roof_stream: store_policy must be 0 (non-temporal) or 1 (sc1), got %d",
                    store_policy);
  if (tile_kib != 8 && tile_kib != 16)
    return tk::fail("tk_roof_stream: tile_kib must be 8 or 16, got %d", tile_kib);
  const int64_t chunks = bytes / 16;
  if (max_workgroups < 0 || max_workgroups > INT32_MAX)
    return tk::fail("tk_roof_stream: max_workgroups must be 0 (one per tile) or positive");
  int64_t blocks = tk::cdiv(chunks, int64_t(kCopyBlock) * (tile_kib / 4));
  if (max_workgroups > 0 && blocks > max_workgroups) blocks = max_workgroups;
  if (blocks > INT32_MAX) return tk::fail("tk_roof_stream: too many bytes");
  // With no writes the sink store may touch one chunk per thread of the grid.
  if (writes == 0 && blocks * kCopyBlock > chunks)
    return tk::fail("tk_roof_stream: a read-only run needs at least %lld bytes",
                    static_cast<long long>(blocks * kCopyBlock * 16));
  const dim3 grid(static_cast<unsigned>(blocks));
  hipStream_t s = tk::as_stream(stream);
  const i32x4* in = static_cast<const i32x4*>(src);
  i32x4* out = static_cast<i32x4*>(dst);
  const int sentinel = 0x5A5A5A5A;
#define TK_ROOF_STREAM_LAUNCH(R, W, CPOL, U)                                                    \
  hipLaunchKernelGGL((roof_stream_kernel<R, W, CPOL, U>), grid, dim3(kCopyBlock), 0, s, in, out, \
                     chunks, sentinel)
#define TK_ROOF_STREAM(R, W)                                                                    \
  if (reads == R && writes == W) {                                                              \
    if (tile_kib == 16) {                                                                       \
      if (store_policy == 0) TK_ROOF_STREAM_LAUNCH(R, W, 2, 4);                                 \
      else TK_ROOF_STREAM_LAUNCH(R, W, 16, 4);                                                  \
    } else {                                                                                    \
      if (store_policy == 0) TK_ROOF_STREAM_LAUNCH(R, W, 2, 2);                                 \
      else TK_ROOF_STREAM_LAUNCH(R, W, 16, 2);                                                  \
    }                                                                                           \
    return tk::check_launch("tk_roof_stream");                                                 \
  }
  TK_ROOF_STREAM(1, 0)
  TK_ROOF_STREAM(0, 1)
  TK_ROOF_STREAM(1, 1)
  TK_ROOF_STREAM(2, 1)
  TK_ROOF_STREAM(3, 1)
  TK_ROOF_STREAM(2, 2)
  TK_ROOF_STREAM(3, 2)
#undef TK_ROOF_STREAM
#undef TK_ROOF_STREAM_LAUNCH
  return tk::fail("tk_roof_stream: unsupported mix %d reads : %d writes", reads, writes);
}

extern "C" int tk_roof_mfma(int dtype, float* out, int64_t waves, int64_t iters, void* stream) {
  if (dtype != TK_DTYPE_F16 && dtype != TK_DTYPE_BF16)
    return tk::fail("tk_roof_mfma: dtype must be TK_DTYPE_F16 or TK_DTYPE_BF16");
  if (waves <= 0 || waves % (kMfmaBlock / 64) != 0 || waves > (int64_t(1) << 24))
    return tk::fail("tk_roof_mfma: waves must be a positive multiple of %d up to 2^24 (got %lld)",
                    kMfmaBlock / 64, static_cast<long long>(waves));
  if (iters <= 0 || iters % kChains != 0 || iters > (int64_t(1) << 30))
    return tk::fail("tk_roof_mfma: iters must be a positive multiple of %d up to 2^30 (got %lld)",
                    kChains, static_cast<long long>(iters));
  if (out == nullptr) return tk::fail("tk_roof_mfma: out is null");
  const dim3 grid(static_cast<unsigned>(waves / (kMfmaBlock / 64)));
  if (dtype == TK_DTYPE_F16)
    hipLaunchKernelGGL(roof_mfma_kernel<_Float16>, grid, dim3(kMfmaBlock), 0,
                       tk::as_stream(stream), out, static_cast<int>(iters));
  else
    hipLaunchKernelGGL(roof_mfma_kernel<__bf16>, grid, dim3(kMfmaBlock), 0,
                       tk::as_stream(stream), out, static_cast<int>(iters));
  return tk::check_launch("tk_roof_mfma");
}
