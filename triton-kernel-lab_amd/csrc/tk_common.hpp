// Shared device and host helpers for the gfx950 kernels of libtklab_hip.so.
//
// Storage types are float, _Float16 and __bf16; all arithmetic is float32.
// Conversions to the 16-bit types round to nearest even (the hardware
// v_cvt instructions), which is also how PyTorch rounds.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <initializer_list>

#include "tklab_hip.h"

namespace tk {

// ---------------------------------------------------------------- host side

// Record a failure message for tk_last_error() and return 1.
int fail(const char* fmt, ...) __attribute__((format(printf, 1, 2)));

// After a launch: turn a pending HIP error into a failure.
int check_launch(const char* what);

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

inline int elem_size(int dtype) { return dtype == TK_DTYPE_F32 ? 4 : 2; }

inline bool valid_dtype(int dtype) {
  return dtype == TK_DTYPE_F32 || dtype == TK_DTYPE_F16 || dtype == TK_DTYPE_BF16;
}

// (d1 - 1) * s1 + (d2 - 1) * s2, the element offset of a 2-D operand's last element, in
// 128-bit arithmetic so no stride or size makes it wrap.
inline __int128 extent(int64_t d1, int64_t s1, int64_t d2, int64_t s2) {
  return static_cast<__int128>(d1 - 1) * s1 + static_cast<__int128>(d2 - 1) * s2;
}

// Row strides are element counts >= 0 (0 repeats one row, as broadcast tables do; no
// kernel here addresses rows before a tensor's base pointer), and the last row of a
// `rows` x `cols` operand ends below 2^52 elements past its base, so no row offset the
// kernels form in 64-bit arithmetic can wrap. Sizes are checked separately.
inline bool row_strides_ok(int64_t rows, int64_t cols, std::initializer_list<int64_t> strides) {
  for (int64_t s : strides)
    if (s < 0 || extent(rows, s, cols, 1) >= (static_cast<__int128>(1) << 52)) return false;
  return true;
}

// rows * cols of a row-major problem folded into one long row, or -1 when either is not
// positive or the product leaves int64.
inline int64_t folded_extent(int64_t rows, int64_t cols) {
  int64_t n;
  if (rows <= 0 || cols <= 0 || __builtin_mul_overflow(rows, cols, &n)) return -1;
  return n;
}

// ---------------------------------------------------------------- conversions

__device__ __forceinline__ float to_f32(float v) { return v; }
__device__ __forceinline__ float to_f32(_Float16 v) { return static_cast<float>(v); }
__device__ __forceinline__ float to_f32(__bf16 v) { return static_cast<float>(v); }

template <typename T>
__device__ __forceinline__ T from_f32(float v) { return static_cast<T>(v); }

// float16 results are rounded to float32 first, as the reference computes in float32
// and then casts. Without the opaque step the backend folds a preceding float32
// multiply into the conversion (v_fma_mixlo_f16 rounds the exact product once), which
// differs from float32-then-float16 rounding when the float32 product is a float16 tie.
template <>
__device__ __forceinline__ _Float16 from_f32<_Float16>(float v) {
  asm("" : "+v"(v));
  return static_cast<_Float16>(v);
}

// Round a float32 value to T and back (T = float is the identity).
template <typename T>
__device__ __forceinline__ float round_to(float v) { return to_f32(from_f32<T>(v)); }

// e^x as exp2(x * log2(e)) on the hardware exponential (v_exp_f32, 1 ulp), the way
// Triton lowers tl.exp: libm's expf adds a range reduction of ~12 more VALU instructions
// per element. -inf gives 0, NaN stays NaN.
__device__ __forceinline__ float hw_exp(float x) {
  return __builtin_amdgcn_exp2f(x * 1.44269504088896341f);
}

// sigmoid from exp(-|z|), branch-stable for any z
// (src/tklab/kernels/_elementwise_math.py:12-18). Shared by the SwiGLU kernels and
// the fused GEMM + SwiGLU epilogue so both evaluate it with the same instructions.
// The exponential is the hardware one, exp2(-|z| * log2(e)) (v_exp_f32), and the quotient
// a hardware reciprocal (v_rcp_f32, 1 ulp), the way Triton lowers the reference's tl.exp
// and `/`: the libm-accurate expf plus an IEEE division took ~20 VALU instructions per
// element, which made the SwiGLU forward (6 bytes of HBM traffic per element) VALU-bound.
__device__ __forceinline__ float stable_sigmoid(float z) {
  const float e = __builtin_amdgcn_exp2f(-fabsf(z) * 1.44269504088896341f);
  const float r = __builtin_amdgcn_rcpf(1.0f + e);
  return z >= 0.f ? r : e * r;
}

// ---------------------------------------------------------------- vector IO

template <typename T, int N>
struct alignas(sizeof(T) * N) Vec {
  T v[N];
};

// Load N consecutive elements starting at p into f[0..N). For N*sizeof(T) == 16
// the pointer must be 16-byte aligned; the load is one 128-bit access.
template <typename T, int N>
__device__ __forceinline__ void load_vec(const T* p, float* f) {
  Vec<T, N> r = *reinterpret_cast<const Vec<T, N>*>(p);
#pragma unroll
  for (int j = 0; j < N; ++j) f[j] = to_f32(r.v[j]);
}

template <typename T, int N>
__device__ __forceinline__ void store_vec(T* p, const float* f) {
  Vec<T, N> r;
#pragma unroll
  for (int j = 0; j < N; ++j) r.v[j] = from_f32<T>(f[j]);
  *reinterpret_cast<Vec<T, N>*>(p) = r;
}

// Non-temporal variants for data touched once (`global_load/store … nt`): streamed
// tensors then do not displace reusable lines from L2 and the last-level cache.
// Measured on the SwiGLU and RoPE benchmark shapes: 5-12% more HBM throughput.
// Vectors narrower than 16 bytes use the plain forms.
template <typename T, int N>
__device__ __forceinline__ void load_vec_stream(const T* p, float* f) {
  if constexpr (N * sizeof(T) == 16) {
    typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));
    const Vec<T, N> r = __builtin_bit_cast(
        Vec<T, N>, __builtin_nontemporal_load(reinterpret_cast<const u32x4v*>(p)));
#pragma unroll
    for (int j = 0; j < N; ++j) f[j] = to_f32(r.v[j]);
  } else {
    load_vec<T, N>(p, f);
  }
}

template <typename T, int N>
__device__ __forceinline__ void store_vec_stream(T* p, const float* f) {
  if constexpr (N * sizeof(T) == 16) {
    typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));
    Vec<T, N> r;
#pragma unroll
    for (int j = 0; j < N; ++j) r.v[j] = from_f32<T>(f[j]);
    __builtin_nontemporal_store(__builtin_bit_cast(u32x4v, r), reinterpret_cast<u32x4v*>(p));
  } else {
    store_vec<T, N>(p, f);
  }
}

// ---------------------------------------------------------------- wave64 reductions
//
// Butterfly all-reduce: xor 1 and xor 2 with DPP quad permutes, then the
// 8-lane half-mirror and 16-lane mirror (after the quad steps every lane of a
// quad holds the quad's value, so mirroring pairs distinct quads), xor 16 with
// ds_swizzle, and the two 32-lane halves combined through readlane. Every
// lane ends with the full result.

template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}

constexpr int kDppQuadXor1 = 0xB1;     // quad_perm [1,0,3,2]
constexpr int kDppQuadXor2 = 0x4E;     // quad_perm [2,3,0,1]
constexpr int kDppRowHalfMirror = 0x141;
constexpr int kDppRowMirror = 0x140;
constexpr int kSwizzleXor16 = 0x401F;  // bit mode: and 0x1F, or 0, xor 0x10

struct SumOp {
  __device__ __forceinline__ float operator()(float a, float b) const { return a + b; }
};
struct MaxOp {
  __device__ __forceinline__ float operator()(float a, float b) const { return fmaxf(a, b); }
};

template <typename Op>
__device__ __forceinline__ float wave_allreduce(float v, Op op) {
  v = op(v, dpp_f32<kDppQuadXor1>(v));
  v = op(v, dpp_f32<kDppQuadXor2>(v));
  v = op(v, dpp_f32<kDppRowHalfMirror>(v));
  v = op(v, dpp_f32<kDppRowMirror>(v));
  v = op(v, __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), kSwizzleXor16)));
  const float lo = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
  const float hi = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
  return op(lo, hi);
}

// All-reduce over a group of RT threads (RT a multiple of 64). For RT > 64 the
// per-wave results meet in `scratch` (RT/64 floats of LDS); the call contains
// two block barriers, so every thread of the block must reach it.
// Workgroup barrier that orders LDS only: this wave's LDS operations complete,
// then s_barrier. Unlike __syncthreads() it does not wait for outstanding global
// loads, so rows prefetched before it stay in flight.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

template <int RT, typename Op>
__device__ __forceinline__ float group_allreduce(float v, Op op, float* scratch) {
  v = wave_allreduce(v, op);
  if constexpr (RT > 64) {
    constexpr int W = RT / 64;
    const int wave = (threadIdx.x % RT) / 64;
    if ((threadIdx.x & 63) == 0) scratch[wave] = v;
    lds_barrier();
    float r = scratch[0];
#pragma unroll
    for (int w = 1; w < W; ++w) r = op(r, scratch[w]);
    lds_barrier();  // every wave has read scratch before it is reused
    v = r;
  }
  return v;
}

// ---------------------------------------------------------------- integer division

// Division by a runtime constant d >= 1 for 0 <= n < 2^31 (round-up multiply
// and shift, Granlund & Montgomery 1994).
struct FastDiv {
  uint32_t d, m, s;
  FastDiv() = default;
  explicit FastDiv(uint32_t divisor) : d(divisor), m(0), s(0) {
    while ((1u << s) < d) ++s;
    m = static_cast<uint32_t>(((uint64_t(1) << 32) * ((uint64_t(1) << s) - d)) / d + 1);
  }
  __device__ __forceinline__ uint32_t div(uint32_t n) const {
    const uint64_t t = __umulhi(n, m);
    return static_cast<uint32_t>((t + n) >> s);
  }
};

}  // namespace tk

// Dispatch on a runtime dtype code to a templated functor call.
#define TK_DISPATCH_DTYPE(dtype, T, ...)                      \
  switch (dtype) {                                            \
    case TK_DTYPE_F32: {                                      \
      using T = float;                                        \
      __VA_ARGS__;                                            \
      break;                                                  \
    }                                                         \
    case TK_DTYPE_F16: {                                      \
      using T = _Float16;                                     \
      __VA_ARGS__;                                            \
      break;                                                  \
    }                                                         \
    case TK_DTYPE_BF16: {                                     \
      using T = __bf16;                                       \
      __VA_ARGS__;                                            \
      break;                                                  \
    }                                                         \
    default:                                                  \
      return tk::fail("unsupported dtype code %d", (int)dtype); \
  }

// Expands `__VA_ARGS__` with constexpr VEC = 16/sizeof(T) when `vector_ok`, else 1.
#define TK_DISPATCH_VEC(T, vector_ok, ...)                         \
  if (vector_ok) {                                                 \
    constexpr int VEC = 16 / int(sizeof(T));                       \
    __VA_ARGS__;                                                   \
  } else {                                                         \
    constexpr int VEC = 1;                                         \
    __VA_ARGS__;                                                   \
  }
