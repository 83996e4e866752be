// GEMM C = A * B for row-major f16/bf16 A [M, K] and B [K, N] (unit inner stride),
// float32 accumulation: the fast path behind tk_gemm (src/tklab/kernels/matmul.py:72-164
// computes the same product with a Triton tile loop).
//
// Block tile 256 x 256, K step 32, 512 threads = 8 wave64s in a 2 (M) x 4 (N) grid, two
// waves per SIMD; each wave owns 128 x 64 of C as 4 x 2 tiles of v_mfma_f32_32x32x16
// (128 accumulators). With two waves per SIMD, one wave's LDS reads, DMA issue and
// barrier waits are covered by the other wave's MFMAs.
//
// Operands reach LDS by buffer->LDS DMA (buffer_load_dwordx4 ... lds): no VGPR staging.
// LDS is a ring of kStages stages of 32 KiB (A tile then B tile); K tile t+kAhead is
// issued while tile t is multiplied, kAhead = kStages - 2, so the stage being refilled
// was last read two tiles ago and one barrier per K tile orders every reuse.
//
// Stage layout (bytes), chosen so every LDS read phase touches 64 distinct banks:
//   A: 256 rows x 64 B; the 16-byte chunk c (k = 8c .. 8c+7) of row r sits at chunk
//      c ^ ((r >> 2) & 3). Fragment reads are ds_read_b128 (16 lanes per phase).
//   B: 32 k-rows x 512 B, row-major in n; the 32-byte granule g (n = 16g .. 16g+15) of
//      k-row k sits at granule g ^ (2 * (k & 3)). Fragments are read with
//      ds_read_b64_tr_b16 (32 lanes per phase), which transposes 4 k x 16 n blocks into
//      the MFMA B layout: two reads give one lane its 8 consecutive k of one column.
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
// (256-byte k-rows, 32-byte granule g of k-row k at g ^ (2 * (k & 3)): still 64 distinct
// banks per read phase), so every B DMA instruction reads one weight. Wave (wm, wq)
// takes gate columns 32wq.. as its N tile 0 and the same up columns as N tile 1, and
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
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x2 __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) void lds_void;

template <typename T>
struct Mfma;
template <>
struct Mfma<_Float16> {
  static __device__ __forceinline__ f32x16 run(i32x4 a, i32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
};
template <>
struct Mfma<__bf16> {
  static __device__ __forceinline__ f32x16 run(i32x4 a, i32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
};

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

// A fragment of row block i (32 rows = 2 KiB) with i folded into the immediate offset.
__device__ __forceinline__ i32x4 read_a(int i, uint32_t addr) {
  switch (i) {
    case 0: return lds_read_b128<0>(addr);
    case 1: return lds_read_b128<2048>(addr);
    case 2: return lds_read_b128<4096>(addr);
    default: return lds_read_b128<6144>(addr);
  }
}

// B fragment for k half KK (16 k-rows of ROWB bytes): k-rows +0..3 and +4..7 of this
// lane group.
template <int KK, int ROWB>
__device__ __forceinline__ i32x4 read_b(uint32_t addr) {
  const i32x2 lo = lds_read_tr16<kOperandBytes + KK * 16 * ROWB>(addr);
  const i32x2 hi = lds_read_tr16<kOperandBytes + KK * 16 * ROWB + 4 * ROWB>(addr);
  return i32x4{lo[0], lo[1], hi[0], hi[1]};
}

struct Frags {
  i32x4 a[4], b[2];
};

// Waits for this wave's LDS reads; the fragments are in/out operands so no use of them
// can be scheduled above the wait.
__device__ __forceinline__ void wait_lgkm(Frags& f) {
  asm volatile("s_waitcnt lgkmcnt(0)"
               : "+v"(f.a[0]), "+v"(f.a[1]), "+v"(f.a[2]), "+v"(f.a[3]), "+v"(f.b[0]),
                 "+v"(f.b[1]));
}

// Y = value * gate * sigmoid(gate) on values already rounded to T, in the SwiGLU
// kernel's operation order (contraction off: each product rounded separately).
template <typename T>
__device__ __forceinline__ T swiglu_out(float gate_acc, float up_acc) {
  const float g = tk::round_to<T>(gate_acc);
  const float v = tk::round_to<T>(up_acc);
  return tk::from_f32<T>(v * g * tk::stable_sigmoid(g));
}

template <typename T, bool kSwiGLU, bool kRowScale>
__global__ __attribute__((amdgpu_flat_work_group_size(kThreads, kThreads),
                          amdgpu_waves_per_eu(2, 2))) void
gemm_dma_kernel(const T* __restrict__ A, const T* __restrict__ B, const T* __restrict__ B2,
                T* __restrict__ C, Problem p) {
  constexpr int kTileN = kSwiGLU ? 128 : BN;  // output columns per block
  constexpr int kRowB = kSwiGLU ? 256 : 512;  // bytes per B k-row in LDS
  __shared__ __attribute__((aligned(1024))) char lds[kStages * kStageBytes];

  const int total = p.tiles_m * p.tiles_n;
  int w = blockIdx.x;
  if (total % kXcds == 0) w = (w % kXcds) * (total / kXcds) + w / kXcds;
  const int per_group = kGroupM * p.tiles_n;  // p.tiles_n counts kTileN-column tiles
  const int first_m = (w / per_group) * kGroupM;
  const int group_m = min(p.tiles_m - first_m, kGroupM);
  const int tile_m = first_m + (w % per_group) % group_m;
  const int tile_n = (w % per_group) / group_m;
  const int m0 = tile_m * BM, n0 = tile_n * kTileN;

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = (wave >> 2) * 128, wn = (wave & 3) * 64;
  const int lrow = lane & 31;
  const int lhalf = lane >> 5;
  const __amdgpu_buffer_rsrc_t ra =
      __builtin_amdgcn_make_buffer_rsrc((void*)A, (short)0, p.a_bytes, 0x00020000);
  // SwiGLU: waves 0-3 fill the gate block, waves 4-7 the up block.
  const bool up_half = kSwiGLU && wave >= 4;
  const __amdgpu_buffer_rsrc_t rb =
      up_half ? __builtin_amdgcn_make_buffer_rsrc((void*)B2, (short)0, p.b2_bytes, 0x00020000)
              : __builtin_amdgcn_make_buffer_rsrc((void*)B, (short)0, p.b_bytes, 0x00020000);
  const int ldb = up_half ? p.ldb2 : p.ldb;
  const uint32_t lds_base = (uint32_t)(uintptr_t)(lds_void*)lds;

  // DMA sources for K tile 0 (bytes). Wave w fills A rows 32w .. 32w+31 (2 loads of 16
  // rows) and B k-rows 4w .. 4w+3 (2 loads of 2 k-rows). Rows past M and columns past N
  // read as zero; K is a multiple of BK on this path.
  uint32_t a_src[2], b_src[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int r = (wave * 2 + i) * 16 + (lane >> 2);
    const int c = (lane & 3) ^ ((r >> 2) & 3);
    a_src[i] = (m0 + r < p.m) ? uint32_t((m0 + r) * p.lda + c * 8) * 2u : kOob;
    if constexpr (kSwiGLU) {
      // Load L = 2*wave + i: block L / 8 (gate, up), k-rows 4*(L % 8) .. +3 of 256 B.
      const int L = wave * 2 + i;
      const int kr = 4 * (L & 7) + (lane >> 4);
      const int slot = lane & 15;
      const int chunk = (((slot >> 1) ^ (2 * (kr & 3))) << 1) | (slot & 1);
      b_src[i] = (n0 + chunk * 8 < p.n) ? uint32_t(kr * ldb + n0 + chunk * 8) * 2u : kOob;
    } else {
      const int kr = (wave * 2 + i) * 2 + (lane >> 5);
      const int slot = lane & 31;
      const int chunk = (((slot >> 1) ^ (2 * (kr & 3))) << 1) | (slot & 1);
      b_src[i] = (n0 + chunk * 8 < p.n) ? uint32_t(kr * ldb + n0 + chunk * 8) * 2u : kOob;
    }
  }
  const uint32_t b_tile_bytes = uint32_t(BK * ldb) * 2u;
  const int kt = p.k / BK;

  // Row-scaled variant: thread t < 256 fetches the scale of tile row t (rows past M
  // clamp to row M - 1 and are never stored) before the first DMA, so the load has
  // landed long before the epilogue; one register through the main loop.
  float row_scale = 0.f;
  if constexpr (kRowScale)
    if (threadIdx.x < BM) row_scale = p.row_scale[min(m0 + (int)threadIdx.x, p.m - 1)];

  // DMA x (0..3: two A loads, two B loads) of K tile `tile` into ring slot `slot`. Tiles past the end reload the
  // last tile into a slot that is never read again, so every step issues the same number
  // of loads and the vmcnt arithmetic stays constant.
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

  // Lane read addresses inside a stage: A row wm + lrow, chunk (2*kk + lhalf) swizzled;
  // B k-row 8*(g>>1) + jj (+16*kk, +4), columns wn + 32j + 16*(g&1) + 4q.
  uint32_t a_addr[2], b_addr[2];
  {
    const int sa = (lrow >> 2) & 3;
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) a_addr[kk] = (wm + lrow) * 64 + (((kk * 2 + lhalf) ^ sa) * 16);
    const int g = lane >> 4, jj = (lane & 15) >> 2, q = lane & 3;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      if constexpr (kSwiGLU) {
        // N tile j is block j (gate, up), columns 32 * (wave & 3) ..
        const int n = (wave & 3) * 32 + (g & 1) * 16 + 4 * q;
        b_addr[j] = j * 8192 +
                    (((g >> 1) * 8 + jj) * 128 + (((n >> 4) ^ (2 * jj)) * 16) + (n & 15)) * 2;
      } else {
        const int n = wn + j * 32 + (g & 1) * 16 + 4 * q;
        b_addr[j] = (((g >> 1) * 8 + jj) * 256 + (((n >> 4) ^ (2 * jj)) * 16) + (n & 15)) * 2;
      }
    }
  }

  f32x16 acc[4][2];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

#pragma unroll
  for (int t = 0; t < kAhead; ++t)
#pragma unroll
    for (int x = 0; x < 4; ++x) dma(x, t, t);
  wait_vmcnt<(kAhead - 1) * 4>();
  barrier_no_fence();

  Frags f0, f1;
#pragma unroll
  for (int i = 0; i < 4; ++i) f0.a[i] = read_a(i, lds_base + a_addr[0]);
#pragma unroll
  for (int j = 0; j < 2; ++j) f0.b[j] = read_b<0, kRowB>(lds_base + b_addr[j]);

  int stage = 0, fill = kAhead;
  for (int t = 0; t < kt; ++t) {
    const uint32_t base = lds_base + stage * kStageBytes;
    const int next = stage + 1 == kStages ? 0 : stage + 1;
    const uint32_t next_base = lds_base + next * kStageBytes;

    // First k half of tile t; meanwhile read the second half and issue tile t + kAhead.
    wait_lgkm(f0);
    sched_fence();
#pragma unroll
    for (int x = 0; x < 8; ++x) {
      acc[x >> 1][x & 1] = Mfma<T>::run(f0.a[x >> 1], f0.b[x & 1], acc[x >> 1][x & 1]);
      sched_fence();
      if (x < 4) {
        f1.a[x] = read_a(x, base + a_addr[1]);
      } else if (x < 6) {
        if (x == 4) f1.b[0] = read_b<1, kRowB>(base + b_addr[0]);
        else f1.b[1] = read_b<1, kRowB>(base + b_addr[1]);
      }
      if (x >= 4) dma(x - 4, t + kAhead, fill);
      sched_fence();
    }

    // Tile t+1 has landed for this wave once only the later tiles' loads are pending;
    // the barrier makes every wave's share visible (and retires all reads of tile t-1).
    wait_vmcnt<(kAhead - 1) * 4>();
    barrier_no_fence();

    // Second k half of tile t; meanwhile read the first half of tile t+1.
    wait_lgkm(f1);
    sched_fence();
#pragma unroll
    for (int x = 0; x < 8; ++x) {
      acc[x >> 1][x & 1] = Mfma<T>::run(f1.a[x >> 1], f1.b[x & 1], acc[x >> 1][x & 1]);
      sched_fence();
      if (x < 4) {
        f0.a[x] = read_a(x, next_base + a_addr[0]);
      } else if (x < 6) {
        if (x == 4) f0.b[0] = read_b<0, kRowB>(next_base + b_addr[0]);
        else f0.b[1] = read_b<0, kRowB>(next_base + b_addr[1]);
      }
      sched_fence();
    }
    stage = next;
    fill = fill + 1 == kStages ? 0 : fill + 1;
  }
  // No DMA may still be writing when the workgroup's LDS is released.
  wait_vmcnt<0>();
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");

  if constexpr (kSwiGLU) {
    const int n = n0 + (wave & 3) * 32 + lrow;
    if (n < p.n) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int m = m0 + wm + i * 32 + (r >> 2) * 8 + lhalf * 4 + (r & 3);
          if (m < p.m) C[m * p.scm + n * p.scn] = swiglu_out<T>(acc[i][0][r], acc[i][1][r]);
        }
      }
    }
  } else {
    // Row-scaled variant: the tile's 256 scales go through the (now idle) LDS, thread t
    // writing the one it fetched at entry; a lane then reads its rows in groups of 4.
    const float* scales = reinterpret_cast<const float*>(lds);
    if constexpr (kRowScale) {
      __syncthreads();  // every wave is done reading the last K tile
      if (threadIdx.x < BM) reinterpret_cast<float*>(lds)[threadIdx.x] = row_scale;
      __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float sc[16];
      if constexpr (kRowScale) {
#pragma unroll
        for (int g4 = 0; g4 < 4; ++g4) {
          const float4 q = *reinterpret_cast<const float4*>(scales + wm + i * 32 + g4 * 8 + lhalf * 4);
          sc[g4 * 4 + 0] = q.x;
          sc[g4 * 4 + 1] = q.y;
          sc[g4 * 4 + 2] = q.z;
          sc[g4 * 4 + 3] = q.w;
        }
      }
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int n = n0 + wn + j * 32 + lrow;
        if (n >= p.n) continue;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int m = m0 + wm + i * 32 + (r >> 2) * 8 + lhalf * 4 + (r & 3);
          const float v = kRowScale ? acc[i][j][r] * sc[r] : acc[i][j][r];
          if (m < p.m) C[m * p.scm + n * p.scn] = tk::from_f32<T>(v);
        }
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
