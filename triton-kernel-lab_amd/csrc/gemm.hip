// GEMM C = A * B on CDNA4 MFMA: f16/bf16 inputs, float32 accumulation,
// f16/bf16 output (src/tklab/kernels/matmul.py:72-164 computes the same
// product; here the tiling is MI355X's own).
//
// tk_gemm sends row-major operands with K % 32 == 0 to the buffer->LDS DMA kernel
// in gemm_dma.hip. This file's register-staged kernel takes everything else:
// arbitrary strides (transposed views), K tails, unaligned rows.
//
// Block tile 256 x 256, K step 64, 256 threads = 4 wave64s in a 2 x 2 grid;
// each wave owns a 128 x 128 sub-tile as 4 x 4 MFMA tiles of
// v_mfma_f32_32x32x16 (256 float32 accumulators per lane, one wave per SIMD).
//
// LDS holds both operands K-contiguous, [256 rows][64 k] per operand, two
// buffers (128 KiB): a row is 8 chunks of 16 bytes (8 elements) and chunk c
// of row r is stored at chunk c ^ swz(r), so that the MFMA operand reads
// (8 consecutive rows, same chunk) and the tile writes both hit 8 distinct
// 16-byte bank groups.
//   A rows are m: swz = m % 8. A 16-byte global load is 8 consecutive k of
//   one row and goes to LDS unchanged.
//   B is stored transposed (rows are n): each thread loads an 8 k x 8 n block
//   (eight 16-byte loads from eight k rows), transposes it in registers, and
//   writes eight 16-byte chunks; swz = (n % 8) ^ ((n / 8) % 8).
// MFMA operand layout (32x32x16): lane l supplies row l % 32 of A (resp.
// column l % 32 of B) at k = 8*(l / 32) .. +7; accumulator register r of lane
// l is D[8*(r/4) + 4*(l/32) + r%4][l % 32].
//
// Tile order: workgroup w runs on XCD w % 8; tiles are renumbered so each XCD
// works through a contiguous range, walked in groups of 4 M-tiles so
// concurrently running tiles share A and B panels in that XCD's L2.
#include "gemm.hpp"
#include "tk_common.hpp"

namespace {

constexpr int BM = 256, BN = 256, BK = 64;
constexpr int kThreads = 256;
constexpr int kGroupM = 4;
constexpr int kXcds = 8;

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

template <typename T>
struct Mfma;
template <>
struct Mfma<_Float16> {
  using Frag = f16x8;
  static __device__ __forceinline__ f32x16 run(Frag a, Frag b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
};
template <>
struct Mfma<__bf16> {
  using Frag = bf16x8;
  static __device__ __forceinline__ f32x16 run(Frag a, Frag b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
};

__device__ __forceinline__ int swz_a(int m) { return m & 7; }
__device__ __forceinline__ int swz_b(int n) { return (n & 7) ^ ((n >> 3) & 7); }

// One operand tile in LDS: 256 rows x 64 halves, 32 KiB.
constexpr int kTileHalves = 256 * 64;

struct Problem {
  int m, n, k;
  int64_t sam, sak, sbk, sbn, scm, scn;
  int tiles_m, tiles_n;
};

// Registers holding the next K tile: A chunks (8 x 16 B) and the B block (8 x 16 B).
struct Staged {
  uint4 a[8];
  uint4 b[8];
};

template <typename T>
__device__ __forceinline__ uint16_t bits_of(T v) {
  return __builtin_bit_cast(uint16_t, v);
}

// Global -> registers for the K tile starting at k0.
// FAST: unit-stride rows, 16-byte aligned rows, K and N multiples of 8.
// Otherwise every element is loaded on its own with full strides and bounds.
template <typename T, bool FAST>
__device__ __forceinline__ void load_tile(const T* __restrict__ A, const T* __restrict__ B,
                                          const Problem& p, int m0, int n0, int k0, Staged& s) {
  const int t = threadIdx.x;
#pragma unroll
  for (int c = 0; c < 8; ++c) {
    const int idx = c * kThreads + t;
    const int row = idx >> 3, chunk = idx & 7;
    const int m = m0 + row, k = k0 + chunk * 8;
    if constexpr (FAST) {
      if (m < p.m && k < p.k)
        s.a[c] = *reinterpret_cast<const uint4*>(A + m * p.sam + k);
      else
        s.a[c] = make_uint4(0, 0, 0, 0);
    } else {
      uint16_t h[8];
#pragma unroll
      for (int e = 0; e < 8; ++e)
        h[e] = (m < p.m && k + e < p.k) ? bits_of(A[m * p.sam + (k + e) * p.sak]) : uint16_t(0);
      s.a[c] = make_uint4(h[0] | (uint32_t(h[1]) << 16), h[2] | (uint32_t(h[3]) << 16),
                          h[4] | (uint32_t(h[5]) << 16), h[6] | (uint32_t(h[7]) << 16));
    }
  }
  const int nc = t & 31, kb = t >> 5;
  const int n = n0 + nc * 8;
#pragma unroll
  for (int r = 0; r < 8; ++r) {
    const int k = k0 + kb * 8 + r;
    if constexpr (FAST) {
      if (k < p.k && n < p.n)
        s.b[r] = *reinterpret_cast<const uint4*>(B + k * p.sbk + n);
      else
        s.b[r] = make_uint4(0, 0, 0, 0);
    } else {
      uint16_t h[8];
#pragma unroll
      for (int e = 0; e < 8; ++e)
        h[e] = (k < p.k && n + e < p.n) ? bits_of(B[k * p.sbk + (n + e) * p.sbn]) : uint16_t(0);
      s.b[r] = make_uint4(h[0] | (uint32_t(h[1]) << 16), h[2] | (uint32_t(h[3]) << 16),
                          h[4] | (uint32_t(h[5]) << 16), h[6] | (uint32_t(h[7]) << 16));
    }
  }
}

__device__ __forceinline__ uint32_t word(const uint4& v, int i) {
  return i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w;
}

// Registers -> LDS buffer. B's 8 x 8 block is transposed on the way:
// out[e] holds column n + e for k = kb*8 .. kb*8+7.
__device__ __forceinline__ void store_tile(uint16_t* __restrict__ lds_a,
                                           uint16_t* __restrict__ lds_b, const Staged& s) {
  const int t = threadIdx.x;
#pragma unroll
  for (int c = 0; c < 8; ++c) {
    const int idx = c * kThreads + t;
    const int row = idx >> 3, chunk = idx & 7;
    *reinterpret_cast<uint4*>(lds_a + row * 64 + ((chunk ^ swz_a(row)) << 3)) = s.a[c];
  }
  const int nc = t & 31, kb = t >> 5;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    uint32_t w[4];
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      const uint32_t lo = word(s.b[2 * d], e >> 1);
      const uint32_t hi = word(s.b[2 * d + 1], e >> 1);
      w[d] = (e & 1) ? ((lo >> 16) | (hi & 0xffff0000u)) : ((lo & 0xffffu) | (hi << 16));
    }
    const int n = nc * 8 + e;
    *reinterpret_cast<uint4*>(lds_b + n * 64 + ((kb ^ swz_b(n)) << 3)) =
        make_uint4(w[0], w[1], w[2], w[3]);
  }
}

template <typename T, bool FAST>
__global__ __attribute__((amdgpu_flat_work_group_size(kThreads, kThreads),
                          amdgpu_waves_per_eu(1, 1))) void
gemm_kernel(const T* __restrict__ A, const T* __restrict__ B, T* __restrict__ C, Problem p) {
  using Frag = typename Mfma<T>::Frag;
  __shared__ __attribute__((aligned(16))) uint16_t lds[2][2][kTileHalves];

  // ---- tile order: XCD-contiguous ranges, grouped along M.
  const int total = p.tiles_m * p.tiles_n;
  int w = blockIdx.x;
  if (total % kXcds == 0) w = (w % kXcds) * (total / kXcds) + w / kXcds;
  const int per_group = kGroupM * p.tiles_n;
  const int group = w / per_group;
  const int first_m = group * kGroupM;
  const int group_m = min(p.tiles_m - first_m, kGroupM);
  const int tile_m = first_m + (w % per_group) % group_m;
  const int tile_n = (w % per_group) / group_m;
  const int m0 = tile_m * BM, n0 = tile_n * BN;

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int wm = (wave >> 1) * 128, wn = (wave & 1) * 128;

  f32x16 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  const int k_tiles = (p.k + BK - 1) / BK;
  Staged st;
  load_tile<T, FAST>(A, B, p, m0, n0, 0, st);
  store_tile(lds[0][0], lds[0][1], st);
  __syncthreads();

  const int lrow = lane & 31, lhalf = lane >> 5;
  for (int kt = 0; kt < k_tiles; ++kt) {
    const int buf = kt & 1;
    const bool more = kt + 1 < k_tiles;
    if (more) load_tile<T, FAST>(A, B, p, m0, n0, (kt + 1) * BK, st);

    const uint16_t* la = lds[buf][0];
    const uint16_t* lb = lds[buf][1];
#pragma unroll
    for (int kk = 0; kk < BK / 16; ++kk) {
      const int chunk = kk * 2 + lhalf;
      Frag af[4], bf[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int m = wm + i * 32 + lrow;
        af[i] = *reinterpret_cast<const Frag*>(la + m * 64 + ((chunk ^ swz_a(m)) << 3));
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int n = wn + j * 32 + lrow;
        bf[j] = *reinterpret_cast<const Frag*>(lb + n * 64 + ((chunk ^ swz_b(n)) << 3));
      }
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = Mfma<T>::run(af[i], bf[j], acc[i][j]);
    }

    if (more) store_tile(lds[buf ^ 1][0], lds[buf ^ 1][1], st);
    __syncthreads();
  }

  // ---- epilogue: D[8*(r/4) + 4*(l/32) + r%4][l%32] of each 32 x 32 tile.
#pragma unroll
  for (int i = 0; i < 4; ++i) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int n = n0 + wn + j * 32 + lrow;
      if (n >= p.n) continue;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int m = m0 + wm + i * 32 + (r >> 2) * 8 + lhalf * 4 + (r & 3);
        if (m < p.m) C[m * p.scm + n * p.scn] = tk::from_f32<T>(acc[i][j][r]);
      }
    }
  }
}

}  // namespace

extern "C" int tk_gemm(int dtype, const void* a, const void* b, void* c, int64_t m, int64_t n,
                       int64_t k, int64_t stride_am, int64_t stride_ak, int64_t stride_bk,
                       int64_t stride_bn, int64_t stride_cm, int64_t stride_cn, int acc_fp16,
                       void* stream) {
  (void)acc_fp16;  // MFMA accumulates f16/bf16 products in float32 only.
  if (dtype != TK_DTYPE_F16 && dtype != TK_DTYPE_BF16)
    return tk::fail("gemm: dtype must be float16 or bfloat16");
  if (a == nullptr || b == nullptr || c == nullptr) return tk::fail("gemm: null pointer");
  if (m <= 0 || n <= 0 || k <= 0) return tk::fail("gemm: empty problem");
  if (stride_am <= 0 || stride_ak <= 0 || stride_bk <= 0 || stride_bn <= 0 || stride_cm <= 0 ||
      stride_cn <= 0)
    return tk::fail("gemm: strides must be positive");
  // 32-bit element offsets inside the kernel.
  const int64_t lim = INT32_MAX;
  if (m > lim || n > lim || k > lim || tk::extent(m, stride_am, k, stride_ak) > lim ||
      tk::extent(k, stride_bk, n, stride_bn) > lim || tk::extent(m, stride_cm, n, stride_cn) > lim)
    return tk::fail("gemm: operand exceeds the int32 offset range");
  const int64_t tiles_m = tk::cdiv(m, BM), tiles_n = tk::cdiv(n, BN);
  if (tiles_m * tiles_n > INT32_MAX) return tk::fail("gemm: too many tiles");
  Problem p{(int)m, (int)n, (int)k, stride_am, stride_ak, stride_bk, stride_bn,
            stride_cm, stride_cn, (int)tiles_m, (int)tiles_n};
  hipStream_t s = tk::as_stream(stream);
  if (tk::gemm_dma_applies(a, b, m, n, k, stride_am, stride_ak, stride_bk, stride_bn)) {
    tk::gemm_dma_launch(dtype, a, b, c, m, n, k, stride_am, stride_bk, stride_cm, stride_cn, s);
    return tk::check_launch("gemm");
  }
  const bool fast = stride_ak == 1 && stride_bn == 1 && k % 8 == 0 && n % 8 == 0 &&
                    stride_am % 8 == 0 && stride_bk % 8 == 0 && tk::aligned16(a) &&
                    tk::aligned16(b);
  const dim3 grid(static_cast<unsigned>(tiles_m * tiles_n));
  if (dtype == TK_DTYPE_F16) {
    using T = _Float16;
    if (fast)
      hipLaunchKernelGGL((gemm_kernel<T, true>), grid, dim3(kThreads), 0, s,
                         static_cast<const T*>(a), static_cast<const T*>(b), static_cast<T*>(c), p);
    else
      hipLaunchKernelGGL((gemm_kernel<T, false>), grid, dim3(kThreads), 0, s,
                         static_cast<const T*>(a), static_cast<const T*>(b), static_cast<T*>(c), p);
  } else {
    using T = __bf16;
    if (fast)
      hipLaunchKernelGGL((gemm_kernel<T, true>), grid, dim3(kThreads), 0, s,
                         static_cast<const T*>(a), static_cast<const T*>(b), static_cast<T*>(c), p);
    else
      hipLaunchKernelGGL((gemm_kernel<T, false>), grid, dim3(kThreads), 0, s,
                         static_cast<const T*>(a), static_cast<const T*>(b), static_cast<T*>(c), p);
  }
  return tk::check_launch("gemm");
}

extern "C" int tk_gemm_swiglu(int dtype, const void* a, const void* b_gate, const void* b_up,
                              void* y, int64_t m, int64_t n, int64_t k, int64_t stride_am,
                              int64_t stride_ak, int64_t stride_gk, int64_t stride_gn,
                              int64_t stride_uk, int64_t stride_un, int64_t stride_ym,
                              int64_t stride_yn, void* stream) {
  if (dtype != TK_DTYPE_F16 && dtype != TK_DTYPE_BF16)
    return tk::fail("gemm_swiglu: dtype must be float16 or bfloat16");
  if (a == nullptr || b_gate == nullptr || b_up == nullptr || y == nullptr)
    return tk::fail("gemm_swiglu: null pointer");
  if (m <= 0 || n <= 0 || k <= 0) return tk::fail("gemm_swiglu: empty problem");
  if (stride_ym <= 0 || stride_yn <= 0) return tk::fail("gemm_swiglu: strides must be positive");
  const int64_t lim = INT32_MAX;
  if (m > lim || n > lim || k > lim || tk::extent(m, stride_ym, n, stride_yn) > lim)
    return tk::fail("gemm_swiglu: operand exceeds the int32 offset range");
  if (!tk::gemm_dma_applies(a, b_gate, m, n, k, stride_am, stride_ak, stride_gk, stride_gn) ||
      !tk::gemm_dma_applies(a, b_up, m, n, k, stride_am, stride_ak, stride_uk, stride_un))
    return tk::fail("gemm_swiglu: needs unit inner strides, 16-byte aligned rows, k %% 32 == 0, "
                    "n %% 8 == 0 and operands below 2 GiB");
  if (tk::cdiv(m, BM) * tk::cdiv(n, 128) > INT32_MAX) return tk::fail("gemm_swiglu: too many tiles");
  tk::gemm_swiglu_dma_launch(dtype, a, b_gate, b_up, y, m, n, k, stride_am, stride_gk, stride_uk,
                             stride_ym, stride_yn, tk::as_stream(stream));
  return tk::check_launch("gemm_swiglu");
}

extern "C" int tk_gemm_rowscale(int dtype, const void* a, const void* b, const float* row_scale,
                                void* c, int64_t m, int64_t n, int64_t k, int64_t stride_am,
                                int64_t stride_ak, int64_t stride_bk, int64_t stride_bn,
                                int64_t stride_cm, int64_t stride_cn, void* stream) {
  if (dtype != TK_DTYPE_F16 && dtype != TK_DTYPE_BF16)
    return tk::fail("gemm_rowscale: dtype must be float16 or bfloat16");
  if (a == nullptr || b == nullptr || row_scale == nullptr || c == nullptr)
    return tk::fail("gemm_rowscale: null pointer");
  if (m <= 0 || n <= 0 || k <= 0) return tk::fail("gemm_rowscale: empty problem");
  if (stride_cm <= 0 || stride_cn <= 0) return tk::fail("gemm_rowscale: strides must be positive");
  const int64_t lim = INT32_MAX;
  if (m > lim || n > lim || k > lim || tk::extent(m, stride_cm, n, stride_cn) > lim)
    return tk::fail("gemm_rowscale: operand exceeds the int32 offset range");
  if (!tk::gemm_dma_applies(a, b, m, n, k, stride_am, stride_ak, stride_bk, stride_bn))
    return tk::fail("gemm_rowscale: needs unit inner strides, 16-byte aligned rows, k %% 32 == 0, "
                    "n %% 8 == 0 and operands below 2 GiB");
  if (tk::cdiv(m, BM) * tk::cdiv(n, BN) > INT32_MAX) return tk::fail("gemm_rowscale: too many tiles");
  tk::gemm_dma_launch(dtype, a, b, c, m, n, k, stride_am, stride_bk, stride_cm, stride_cn,
                      tk::as_stream(stream), row_scale);
  return tk::check_launch("gemm_rowscale");
}
