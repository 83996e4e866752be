// GEMM C = A * B for row-major f16/bf16 A [M, K] and B [K, N] (unit inner stride),
// float32 accumulation: the fast path behind tk_gemm (src/tklab/kernels/matmul.py:72-164
// computes the same product with a Triton tile loop).
//
// Block tile 256 x 256, K step 32, 512 threads = 8 wave64s in a 2 (M) x 4 (N) grid, two
// waves per SIMD; each wave owns 128 x 64 of C as 8 x 4 tiles of v_mfma_f32_16x16x32
// (128 accumulators). With two waves per SIMD, one wave's LDS reads, DMA issue and
// barrier waits are covered by the other wave's MFMAs. 16x16x32 rather than 32x32x16:
// the clock is power-limited under dense MFMA load, and the 16x16 shape sustains more
// FLOP/s (MFMA-only with random operands 1.90 vs 1.78 PFLOP/s bf16; this GEMM 1.39 vs
// 1.29 PFLOP/s at 8192^3 with the same tiles and LDS traffic). The MFMAs compute C^T
// tiles (the B fragment as the first operand), so a lane's four accumulator registers
// are four consecutive columns of one row and leave as one 8-byte store.
//
// Operands reach LDS by buffer->LDS DMA (buffer_load_dwordx4 ... lds): no VGPR staging.
// LDS is a ring of kStages stages of 32 KiB (A tile then B tile); K tile t+kAhead is
// issued while tile t is multiplied, kAhead = kStages - 2, so the stage being refilled
// was last read two tiles ago and one barrier per K tile orders every reuse. The
// barrier sits between the wave's row tiles 0-3 and 4-7: rows 0-3 run while rows 4-7
// of the same K tile are read and tile t + kAhead is issued; rows 4-7 run while the
// next tile's rows 0-3 and B fragments (a second register set) are read.
//
// Stage layout (bytes), chosen so every LDS read phase touches 64 distinct banks:
//   A: 256 rows x 64 B; the 16-byte chunk c (k = 8c .. 8c+7) of row r sits at chunk
//      c ^ a_swz(r), a_swz(r) = bit 0 of r | bit 2 of r << 1. A fragment (16 rows, lane
//      group g taking k = 8g .. 8g+7) is one ds_read_b128. Measured on gfx950, an
//      isolated stream of these reads sustains 256 B/clock/CU with this swizzle and
//      155 B/clock/CU (four bank-conflict cycles per read) with c ^ ((r >> 2) & 3)
//      or with none.
//   B: 32 k-rows x 512 B, row-major in n; the 32-byte granule g (n = 16g .. 16g+15) of
//      k-row k sits at granule g ^ (2 * (k & 3) + ((k >> 3) & 1)). Fragments are read
//      with ds_read_b64_tr_b16, which transposes 4 k x 16 n blocks into the MFMA B
//      layout: two reads give one lane its 8 consecutive k of one column. One read phase
//      (32 lanes) covers two lane groups on k-rows 8 apart; the (k >> 3) term puts their
//      8 granules on distinct banks.
// A DMA instruction moves 64 lanes x 16 B into 1 KiB of contiguous LDS at M0, so the
// swizzle is applied on the global side: each lane fetches the chunk that belongs at its
// LDS slot.
//
// The compiler inserts vmcnt(0) before any LDS read that may alias an LDS DMA, which
// would drain the prefetch ring every step; fragment reads are therefore inline asm
// ordered by explicit s_waitcnt, with the MFMA/LDS/DMA interleave pinned by
// sched_barrier.
//
// Tile order: workgroup w runs on XCD w % 8; tiles are renumbered so each XCD walks a
// contiguous range in groups of 4 M-tiles, sharing A and B panels in that XCD's L2.
//
// Row-scaled variant (kRowScale): C[m, :] = round(s[m] * acc),
// one float32 multiply before the rounding. With s = rstd of a normalization whose
// weight is folded into B, this is the normalized GEMM rms_norm(a) * B' without the
// normalized activations ever being written.
//
// SwiGLU variant (kSwiGLU): Y = swiglu(value = A*B_up, gate = A*B_gate) for two weights
// [K, N]. A block computes 256 x 128 of Y from a 256-column B tile holding the gate
// columns n0..n0+127 then the same up columns, laid out in LDS as two 128-column blocks
// (256-byte k-rows, same granule swizzle: still 64 distinct banks per read phase), so
// every B DMA instruction reads one weight. Wave (wm, wq) takes gate columns 32wq ..
// 32wq+31 as its N tiles 0, 1 and the same up columns as N tiles 2, 3, and
// the epilogue rounds both to the storage type (as the unfused GEMMs store them) and
// writes value * gate * sigmoid(gate): the two M x N intermediates never reach HBM and
// the result is bitwise that of the two GEMMs followed by the SwiGLU kernel.
#include "gemm.hpp"
#include "tk_common.hpp"

// No floating-point contraction in this file: the SwiGLU epilogue must round
// value * gate * sigmoid(gate) to float32 and then to the storage type, as the SwiGLU
// kernel and the reference do (a fused multiply-convert would round once).
#pragma clang fp contract(off)

namespace {

constexpr int BM = 256, BN = 256, BK = 32;
constexpr int kThreads = 512;  // 8 waves
constexpr int kStages = 5;
constexpr int kAhead = kStages - 2;
constexpr int kGroupM = 4;
constexpr int kXcds = 8;
constexpr int kOperandBytes = 256 * BK * 2;  // 16 KiB per operand per stage
constexpr int kStageBytes = 2 * kOperandBytes;
constexpr uint32_t kOob = 0x80000000u;  // past every buffer's num_records: reads as zero

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x2 __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) void lds_void;


struct Problem {
  int m, n, k;
  int lda, ldb, ldb2;  // ldb2: the up weight's k stride (SwiGLU variant)
  int64_t scm, scn;
  int tiles_m, tiles_n;
  uint32_t a_bytes, b_bytes, b2_bytes;
  const float* row_scale;  // kRowScale: C[m, :] = round(row_scale[m] * acc)
};

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
  // s_waitcnt fields: vmcnt[3:0], expcnt[6:4] (7 = no wait), lgkmcnt[11:8] (15 = no wait),
  // vmcnt[5:4] at [15:14].
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

// Workgroup barrier without the release/acquire fence __syncthreads() carries: the
// fence would wait for every outstanding DMA, while each caller has already waited
// for exactly the tile it is about to read.
__device__ __forceinline__ void barrier_no_fence() { asm volatile("s_barrier" ::: "memory"); }

__device__ __forceinline__ void sched_fence() { __builtin_amdgcn_sched_barrier(0); }

template <int OFF>
__device__ __forceinline__ i32x4 lds_read_b128(uint32_t addr) {
  i32x4 r;
  asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(r) : "v"(addr), "i"(OFF));
  return r;
}

template <int OFF>
__device__ __forceinline__ i32x2 lds_read_tr16(uint32_t addr) {
  i32x2 r;
  asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(r) : "v"(addr), "i"(OFF));
  return r;
}

// Y = value * gate * sigmoid(gate) on values already rounded to T, in the SwiGLU
// kernel's operation order (contraction off: each product rounded separately).
template <typename T>
__device__ __forceinline__ T swiglu_out(float gate_acc, float up_acc) {
  const float g = tk::round_to<T>(gate_acc);
  const float v = tk::round_to<T>(up_acc);
  return tk::from_f32<T>(v * g * tk::stable_sigmoid(g));
}

// v_mfma_f32_16x16x32: A lane l holds row l % 16, k = 8 (l / 16) .. +7; B lane l holds
// column l % 16, the same k; D lane l holds column l % 16, rows 4 (l / 16) .. +3.
typedef float f32x4 __attribute__((ext_vector_type(4)));

template <typename T>
struct Mfma;
template <>
struct Mfma<_Float16> {
  static __device__ __forceinline__ f32x4 run(i32x4 a, i32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
};
template <>
struct Mfma<__bf16> {
  static __device__ __forceinline__ f32x4 run(i32x4 a, i32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
};

// A row swizzle: 16-byte chunk c of row r sits at c ^ a_swz(r).
__device__ __forceinline__ int a_swz(int r) { return (r & 1) | ((r >> 1) & 2); }

// B k-row swizzle: 32-byte granule g of k-row k sits at g ^ b_swz(k). A 16x16x32 B
// fragment read phase covers two 16-lane groups reading k-rows 8 apart, so the swizzle
// carries bit 3 of k besides the (k & 3) term that separates the 4 rows of one read.
__device__ __forceinline__ int b_swz(int k) { return 2 * (k & 3) + ((k >> 3) & 1); }

// A fragment of row tile I (16 rows = 1 KiB of the stage).
template <int I>
__device__ __forceinline__ i32x4 read_a(uint32_t addr) {
  return lds_read_b128<I * 1024>(addr);
}

// B fragment: k-rows +0..3 and +4..7 of this lane group (ROWB bytes per k-row).
template <int ROWB>
__device__ __forceinline__ i32x4 read_b(uint32_t addr) {
  const i32x2 lo = lds_read_tr16<kOperandBytes>(addr);
  const i32x2 hi = lds_read_tr16<kOperandBytes + 4 * ROWB>(addr);
  return i32x4{lo[0], lo[1], hi[0], hi[1]};
}

template <int N>
__device__ __forceinline__ void wait_lgkm_pin(i32x4 (&f)[N]) {
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
  for (int i = 0; i < N; ++i) asm volatile("" : "+v"(f[i]));
}

template <typename T, bool kSwiGLU, bool kRowScale>
__global__ __attribute__((amdgpu_flat_work_group_size(kThreads, kThreads),
                          amdgpu_waves_per_eu(2, 2))) void
gemm_dma_kernel(const T* __restrict__ A, const T* __restrict__ B, const T* __restrict__ B2,
                  T* __restrict__ C, Problem p) {
  constexpr int kTileN = kSwiGLU ? 128 : BN;
  constexpr int kRowB = kSwiGLU ? 256 : 512;
  __shared__ __attribute__((aligned(1024))) char lds[kStages * kStageBytes];

  const int total = p.tiles_m * p.tiles_n;
  int w = blockIdx.x;
  if (total % kXcds == 0) w = (w % kXcds) * (total / kXcds) + w / kXcds;
  const int per_group = kGroupM * p.tiles_n;
  const int first_m = (w / per_group) * kGroupM;
  const int group_m = min(p.tiles_m - first_m, kGroupM);
  const int tile_m = first_m + (w % per_group) % group_m;
  const int tile_n = (w % per_group) / group_m;
  const int m0 = tile_m * BM, n0 = tile_n * kTileN;

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = (wave >> 2) * 128, wn = (wave & 3) * 64;
  const int l16 = lane & 15, lg = lane >> 4;
  const __amdgpu_buffer_rsrc_t ra =
      __builtin_amdgcn_make_buffer_rsrc((void*)A, (short)0, p.a_bytes, 0x00020000);
  const bool up_half = kSwiGLU && wave >= 4;
  const __amdgpu_buffer_rsrc_t rb =
      up_half ? __builtin_amdgcn_make_buffer_rsrc((void*)B2, (short)0, p.b2_bytes, 0x00020000)
              : __builtin_amdgcn_make_buffer_rsrc((void*)B, (short)0, p.b_bytes, 0x00020000);
  const int ldb = up_half ? p.ldb2 : p.ldb;
  const uint32_t lds_base = (uint32_t)(uintptr_t)(lds_void*)lds;

  uint32_t a_src[2], b_src[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int r = (wave * 2 + i) * 16 + (lane >> 2);
    const int c = (lane & 3) ^ a_swz(r);
    a_src[i] = (m0 + r < p.m) ? uint32_t((m0 + r) * p.lda + c * 8) * 2u : kOob;
    if constexpr (kSwiGLU) {
      const int L = wave * 2 + i;
      const int kr = 4 * (L & 7) + (lane >> 4);
      const int slot = lane & 15;
      const int chunk = (((slot >> 1) ^ b_swz(kr)) << 1) | (slot & 1);
      b_src[i] = (n0 + chunk * 8 < p.n) ? uint32_t(kr * ldb + n0 + chunk * 8) * 2u : kOob;
    } else {
      const int kr = (wave * 2 + i) * 2 + (lane >> 5);
      const int slot = lane & 31;
      const int chunk = (((slot >> 1) ^ b_swz(kr)) << 1) | (slot & 1);
      b_src[i] = (n0 + chunk * 8 < p.n) ? uint32_t(kr * ldb + n0 + chunk * 8) * 2u : kOob;
    }
  }
  const uint32_t b_tile_bytes = uint32_t(BK * ldb) * 2u;
  const int kt = p.k / BK;

  float row_scale = 0.f;
  if constexpr (kRowScale)
    if (threadIdx.x < BM) row_scale = p.row_scale[min(m0 + (int)threadIdx.x, p.m - 1)];

  auto dma = [&](int x, int tile, int slot) {
    tile = min(tile, kt - 1);
    char* stage = lds + slot * kStageBytes;
    if (x < 2)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, (lds_void*)(stage + (wave * 2 + x) * 1024), 16,
                                               a_src[x], tile * (BK * 2), 0, 0);
    else
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          rb, (lds_void*)(stage + kOperandBytes + (wave * 2 + x - 2) * 1024), 16, b_src[x - 2],
          tile * b_tile_bytes, 0, 0);
  };

  // A: row wm + l16 (+16 per row tile), chunk lg swizzled (a_swz reads only the row's
  // low four bits, the same for every row tile). B: k-rows 8 lg + (l16 >> 2) (+4), columns of N tile j starting
  // at 4 (l16 & 3).
  const uint32_t a_addr = (wm + l16) * 64 + ((lg ^ a_swz(l16)) * 16);
  uint32_t b_addr[4];
  {
    const int jj = l16 >> 2, q = l16 & 3;
    const int kr = 8 * lg + jj;
    const int sw = b_swz(kr);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if constexpr (kSwiGLU) {
        // N tiles 0, 1: gate columns 32 (wave & 3) + 16 j; tiles 2, 3: the same up columns.
        const int g = 2 * (wave & 3) + (j & 1);
        b_addr[j] = (j >> 1) * 8192 + kr * 256 + ((g ^ sw) * 32) + q * 8;
      } else {
        const int g = wn / 16 + j;
        b_addr[j] = kr * 512 + ((g ^ sw) * 32) + q * 8;
      }
    }
  }

  f32x4 acc[8][4];
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

#pragma unroll
  for (int t = 0; t < kAhead; ++t)
#pragma unroll
    for (int x = 0; x < 4; ++x) dma(x, t, t);
  wait_vmcnt<(kAhead - 1) * 4>();
  barrier_no_fence();

  i32x4 a_lo[4], a_hi[4], b0[4], b1[4];
  a_lo[0] = read_a<0>(lds_base + a_addr);
  a_lo[1] = read_a<1>(lds_base + a_addr);
  a_lo[2] = read_a<2>(lds_base + a_addr);
  a_lo[3] = read_a<3>(lds_base + a_addr);
#pragma unroll
  for (int j = 0; j < 4; ++j) b0[j] = read_b<kRowB>(lds_base + b_addr[j]);

  // One K tile; B is this tile's B fragments, Bn receives the next tile's.
  auto step = [&](int t, int stage, int fill, i32x4 (&Bc)[4], i32x4 (&Bn)[4]) {
    const uint32_t base = lds_base + stage * kStageBytes;
    const int next = stage + 1 == kStages ? 0 : stage + 1;
    const uint32_t next_base = lds_base + next * kStageBytes;
    wait_lgkm_pin(a_lo);
    wait_lgkm_pin(Bc);
    sched_fence();
    // Rows 0-3; read rows 4-7 of this tile, issue tile t + kAhead.
#pragma unroll
    for (int x = 0; x < 16; ++x) {
      const int i = x >> 2, j = x & 3;
      acc[i][j] = Mfma<T>::run(Bc[j], a_lo[i], acc[i][j]);
      sched_fence();
      if (j == 0) {
        if (i == 0) a_hi[0] = read_a<4>(base + a_addr);
        if (i == 1) a_hi[1] = read_a<5>(base + a_addr);
        if (i == 2) a_hi[2] = read_a<6>(base + a_addr);
        if (i == 3) a_hi[3] = read_a<7>(base + a_addr);
      }
      if (j == 2) dma(i, t + kAhead, fill);
      sched_fence();
    }
    wait_vmcnt<(kAhead - 1) * 4>();
    barrier_no_fence();
    wait_lgkm_pin(a_hi);
    sched_fence();
    // Rows 4-7; read rows 0-3 and B of tile t+1.
#pragma unroll
    for (int x = 0; x < 16; ++x) {
      const int i = x >> 2, j = x & 3;
      acc[4 + i][j] = Mfma<T>::run(Bc[j], a_hi[i], acc[4 + i][j]);
      sched_fence();
      if (j == 0) {
        if (i == 0) a_lo[0] = read_a<0>(next_base + a_addr);
        if (i == 1) a_lo[1] = read_a<1>(next_base + a_addr);
        if (i == 2) a_lo[2] = read_a<2>(next_base + a_addr);
        if (i == 3) a_lo[3] = read_a<3>(next_base + a_addr);
      }
      if (j == 2) Bn[i] = read_b<kRowB>(next_base + b_addr[i]);
      sched_fence();
    }
  };

  int stage = 0, fill = kAhead;
  auto advance = [&]() {
    stage = stage + 1 == kStages ? 0 : stage + 1;
    fill = fill + 1 == kStages ? 0 : fill + 1;
  };
  int t = 0;
  for (; t + 1 < kt; t += 2) {
    step(t, stage, fill, b0, b1);
    advance();
    step(t + 1, stage, fill, b1, b0);
    advance();
  }
  if (t < kt) step(t, stage, fill, b0, b1);
  wait_vmcnt<0>();
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");

  // acc[i][j] holds C^T: register r of lane l is C[m][n] with m = m0 + wm + 16 i + l % 16 and
  // n = n0 + (N tile j's first column) + 4 (l / 16) + r, so a lane stores 4 consecutive
  // columns of one row: one 8-byte store when C rows are contiguous and 8-byte aligned.
  const bool vec = p.scn == 1 && (p.scm & 3) == 0 && (reinterpret_cast<uintptr_t>(C) & 7) == 0;
  auto store4 = [&](int m, int n, const float (&v)[4]) {
    if (m >= p.m || n >= p.n) return;
    T* dst = C + m * p.scm + n * p.scn;
    if (vec) {  // p.n % 8 == 0, so n .. n+3 are in range
      const uint32_t lo = uint32_t(__builtin_bit_cast(uint16_t, tk::from_f32<T>(v[0]))) |
                          (uint32_t(__builtin_bit_cast(uint16_t, tk::from_f32<T>(v[1]))) << 16);
      const uint32_t hi = uint32_t(__builtin_bit_cast(uint16_t, tk::from_f32<T>(v[2]))) |
                          (uint32_t(__builtin_bit_cast(uint16_t, tk::from_f32<T>(v[3]))) << 16);
      *reinterpret_cast<uint2*>(dst) = uint2{lo, hi};
    } else {
#pragma unroll
      for (int r = 0; r < 4; ++r)
        if (n + r < p.n) dst[r * p.scn] = tk::from_f32<T>(v[r]);
    }
  };
  if constexpr (kSwiGLU) {
#pragma unroll
    for (int jj = 0; jj < 2; ++jj) {
      const int n = n0 + (wave & 3) * 32 + jj * 16 + lg * 4;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int m = m0 + wm + i * 16 + l16;
        float v[4];
#pragma unroll
        for (int r = 0; r < 4; ++r)
          v[r] = static_cast<float>(swiglu_out<T>(acc[i][jj][r], acc[i][jj + 2][r]));
        store4(m, n, v);
      }
    }
  } else {
    const float* scales = reinterpret_cast<const float*>(lds);
    if constexpr (kRowScale) {
      __syncthreads();
      if (threadIdx.x < BM) reinterpret_cast<float*>(lds)[threadIdx.x] = row_scale;
      __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int m = m0 + wm + i * 16 + l16;
      const float sc = kRowScale ? scales[wm + i * 16 + l16] : 1.f;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int n = n0 + wn + j * 16 + lg * 4;
        float v[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) v[r] = kRowScale ? acc[i][j][r] * sc : acc[i][j][r];
        store4(m, n, v);
      }
    }
  }
}


}  // namespace

namespace tk {

bool gemm_dma_applies(const void* a, const void* b, int64_t m, int64_t n, int64_t k,
                      int64_t stride_am, int64_t stride_ak, int64_t stride_bk,
                      int64_t stride_bn) {
  // Buffer offsets are 32-bit with kOob (2^31) reserved as "outside".
  const int64_t a_bytes = ((m - 1) * stride_am + k) * 2;
  const int64_t b_bytes = ((k - 1) * stride_bk + n) * 2;
  return stride_ak == 1 && stride_bn == 1 && k % BK == 0 && n % 8 == 0 && stride_am % 8 == 0 &&
         stride_bk % 8 == 0 && aligned16(a) && aligned16(b) && a_bytes < int64_t(kOob) &&
         b_bytes < int64_t(kOob);
}

void gemm_dma_launch(int dtype, const void* a, const void* b, void* c, int64_t m, int64_t n,
                     int64_t k, int64_t stride_am, int64_t stride_bk, int64_t stride_cm,
                     int64_t stride_cn, hipStream_t stream, const float* row_scale) {
  const uint32_t b_bytes = (uint32_t)(((k - 1) * stride_bk + n) * 2);
  Problem p{(int)m,
            (int)n,
            (int)k,
            (int)stride_am,
            (int)stride_bk,
            (int)stride_bk,
            stride_cm,
            stride_cn,
            (int)cdiv(m, BM),
            (int)cdiv(n, BN),
            (uint32_t)(((m - 1) * stride_am + k) * 2),
            b_bytes,
            b_bytes,
            row_scale};
  const dim3 grid(static_cast<unsigned>(p.tiles_m * p.tiles_n));
  if (dtype == TK_DTYPE_F16) {
    using T = _Float16;
    if (row_scale != nullptr)
      hipLaunchKernelGGL((gemm_dma_kernel<T, false, true>), grid, dim3(kThreads), 0, stream,
                         static_cast<const T*>(a), static_cast<const T*>(b),
                         static_cast<const T*>(b), static_cast<T*>(c), p);
    else
      hipLaunchKernelGGL((gemm_dma_kernel<T, false, false>), grid, dim3(kThreads), 0, stream,
                         static_cast<const T*>(a), static_cast<const T*>(b),
                         static_cast<const T*>(b), static_cast<T*>(c), p);
  } else {
    using T = __bf16;
    if (row_scale != nullptr)
      hipLaunchKernelGGL((gemm_dma_kernel<T, false, true>), grid, dim3(kThreads), 0, stream,
                         static_cast<const T*>(a), static_cast<const T*>(b),
                         static_cast<const T*>(b), static_cast<T*>(c), p);
    else
      hipLaunchKernelGGL((gemm_dma_kernel<T, false, false>), grid, dim3(kThreads), 0, stream,
                         static_cast<const T*>(a), static_cast<const T*>(b),
                         static_cast<const T*>(b), static_cast<T*>(c), p);
  }
}

void gemm_swiglu_dma_launch(int dtype, const void* a, const void* b_gate, const void* b_up,
                            void* y, int64_t m, int64_t n, int64_t k, int64_t stride_am,
                            int64_t stride_gk, int64_t stride_uk, int64_t stride_ym,
                            int64_t stride_yn, hipStream_t stream) {
  Problem p{(int)m,
            (int)n,
            (int)k,
            (int)stride_am,
            (int)stride_gk,
            (int)stride_uk,
            stride_ym,
            stride_yn,
            (int)cdiv(m, BM),
            (int)cdiv(n, 128),
            (uint32_t)(((m - 1) * stride_am + k) * 2),
            (uint32_t)(((k - 1) * stride_gk + n) * 2),
            (uint32_t)(((k - 1) * stride_uk + n) * 2),
            nullptr};
  const dim3 grid(static_cast<unsigned>(p.tiles_m * p.tiles_n));
  if (dtype == TK_DTYPE_F16)
    hipLaunchKernelGGL((gemm_dma_kernel<_Float16, true, false>), grid, dim3(kThreads), 0, stream,
                       static_cast<const _Float16*>(a), static_cast<const _Float16*>(b_gate),
                       static_cast<const _Float16*>(b_up), static_cast<_Float16*>(y), p);
  else
    hipLaunchKernelGGL((gemm_dma_kernel<__bf16, true, false>), grid, dim3(kThreads), 0, stream,
                       static_cast<const __bf16*>(a), static_cast<const __bf16*>(b_gate),
                       static_cast<const __bf16*>(b_up), static_cast<__bf16*>(y), p);
}

}  // namespace tk
