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
// are four consecutive columns of one row (8 bytes once rounded). The epilogue stages the
// rounded tile in the idle rings and writes whole rows from there.
//
// Operands reach LDS by buffer->LDS DMA (buffer_load_dwordx4 ... lds): no VGPR staging.
// A and B have rings of their own: A in 64-wide K tiles (three stages of 256 rows x 128 B),
// B in 32-wide K tiles (four stages of 32 k-rows x 512 B), 160 KiB in all. Each DMA request
// then covers a whole 128-byte line: with 32-wide A tiles every A row was a 64-byte half
// line, and the vector memory path (texture data unit 95 % busy, two thirds of it waiting
// on L1, L1 waiting on L2 two thirds of the time) moved a third more requests than bytes
// needed. The loop runs 32-wide steps with one barrier each, placed between the wave's
// row tiles 0-3 and 4-7: rows 0-3 run while rows 4-7 of the same step are read and the
// step's DMA is issued; rows 4-7 run while the next step's rows 0-3 and B fragments (a
// second register set) are read.
//
// Stage layout (bytes), chosen so every LDS read phase touches 64 distinct banks:
//   A: 256 rows x 128 B; the 16-byte chunk c (k = 8c .. 8c+7 of the 64-wide tile) of row r
//      sits at chunk c ^ a_swz(r), a_swz(r) = (r >> 1) & 7. A fragment (16 rows, lane
//      group g taking k = 8g .. 8g+7 of the step's 32-wide half) is one ds_read_b128.
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
constexpr int kGroupM = 4;
constexpr int kXcds = 8;
// A ring: kAStages stages of one 64-wide K tile (256 rows x 128 B); B ring: kBStages stages
// of one 32-wide K tile (32 k-rows x 512 B). 96 + 64 KiB: all of the CU's LDS.
constexpr int kAStages = 3, kBStages = 4;
constexpr int kABytes = 256 * 64 * 2;        // 32 KiB per A stage
constexpr int kOperandBytes = 256 * BK * 2;  // 16 KiB per B stage
constexpr int kBRing = kAStages * kABytes;   // B ring offset
constexpr int kLdsBytes = kBRing + kBStages * kOperandBytes;
constexpr uint32_t kOob = 0x80000000u;  // past every buffer's num_records: reads as zero
// Epilogue: the C tile is staged in the ring's LDS (at most 256 rows of 528 bytes), the row
// scales of the row-scaled variant after it.
constexpr int kScaleOff = 256 * 528;
static_assert(kScaleOff + 256 * 4 <= kLdsBytes, "row scales past the LDS block");

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

// A row swizzle (128-byte rows): 16-byte chunk c of row r sits at c ^ a_swz(r). A fragment
// read phase takes one chunk of 16 consecutive rows: even and odd rows fall in opposite
// halves of a 256-byte bank row, and (r >> 1) & 7 puts the 8 rows of each half on distinct
// 16-byte slots.
__device__ __forceinline__ int a_swz(int r) { return (r >> 1) & 7; }

// B k-row swizzle: 32-byte granule g of k-row k sits at g ^ b_swz(k). A 16x16x32 B
// fragment read phase covers two 16-lane groups reading k-rows 8 apart, so the swizzle
// carries bit 3 of k besides the (k & 3) term that separates the 4 rows of one read.
__device__ __forceinline__ int b_swz(int k) { return 2 * (k & 3) + ((k >> 3) & 1); }

// A fragment of row tile I (16 rows = 2 KiB of the stage).
template <int I>
__device__ __forceinline__ i32x4 read_a(uint32_t addr) {
  return lds_read_b128<I * 2048>(addr);
}

// B fragment: k-rows +0..3 and +4..7 of this lane group (ROWB bytes per k-row).
template <int ROWB>
__device__ __forceinline__ i32x4 read_b(uint32_t addr) {
  const i32x2 lo = lds_read_tr16<0>(addr);
  const i32x2 hi = lds_read_tr16<4 * ROWB>(addr);
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
  __shared__ __attribute__((aligned(1024))) char lds[kLdsBytes];

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

  // A DMA x (0..3) of a 64-wide K tile: rows 8 (4 wave + x) .. +7, eight lanes per 128-byte
  // row; each lane fetches the chunk that belongs at its LDS slot.
  // a_last: the same sources for the last 64-wide tile when only its first 32 columns lie
  // inside K (kt odd): lanes whose chunk falls in the second half read nothing. The tile's
  // offset travels in soffset, which the buffer range check does not cover, so without
  // this the last row of A would be read up to 64 bytes past its end.
  uint32_t a_src[4], a_last[4], b_src[2];
#pragma unroll
  for (int x = 0; x < 4; ++x) {
    const int r = (wave * 4 + x) * 8 + (lane >> 3);
    const int c = (lane & 7) ^ a_swz(r);
    a_src[x] = (m0 + r < p.m) ? uint32_t((m0 + r) * p.lda + c * 8) * 2u : kOob;
    a_last[x] = c < 4 ? a_src[x] : kOob;
  }
#pragma unroll
  for (int i = 0; i < 2; ++i) {
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
  const int kt = p.k / BK;      // 32-wide K tiles
  const int kt64 = (kt + 1) / 2;  // 64-wide A tiles (the last one half used when kt is odd)

  float row_scale = 0.f;
  if constexpr (kRowScale)
    if (threadIdx.x < BM) row_scale = p.row_scale[min(m0 + (int)threadIdx.x, p.m - 1)];

  // Tiles past the end reload the last one into a stage that is never read, keeping every
  // step's DMA count constant.
  const int half_tile = (kt & 1) ? kt64 - 1 : kt64;  // index of a half-used A tile, if any
  auto dma_a = [&](int x, int tile, int slot) {
    tile = min(tile, kt64 - 1);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(
        ra, (lds_void*)(lds + slot * kABytes + (wave * 4 + x) * 1024), 16,
        tile == half_tile ? a_last[x] : a_src[x], tile * 128, 0, 0);
  };
  auto dma_b = [&](int x, int tile, int slot) {
    tile = min(tile, kt - 1);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(
        rb, (lds_void*)(lds + kBRing + slot * kOperandBytes + (wave * 2 + x) * 1024), 16,
        b_src[x], tile * b_tile_bytes, 0, 0);
  };

  // A: row wm + l16 (+16 per row tile), chunk lg (first 32-wide half of the 64-wide tile)
  // or 4 + lg (second half), swizzled (a_swz reads only the row's low four bits, the same
  // for every row tile). B: k-rows 8 lg + (l16 >> 2) (+4), columns of N tile j starting at
  // 4 (l16 & 3).
  const uint32_t a_addr0 = (wm + l16) * 128 + ((lg ^ a_swz(l16)) * 16);
  const uint32_t a_addr1 = (wm + l16) * 128 + (((4 + lg) ^ a_swz(l16)) * 16);
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

  // DMA schedule. 32-wide step t issues B tile t + 3 (two instructions per wave) into B
  // stage (t + 3) % 4 and, when t is odd, the 64-wide A tile (t + 3) / 2 (four per wave)
  // into A stage ((t + 3) / 2) % 3. A stage reuse: A tile v's last fragments (rows 4-7 of
  // step 2v + 1) are read in the first half of step 2v + 1 and waited for after that step's
  // barrier, so every wave is done with them at the barrier of step 2v + 2; tile v + 3
  // refills the stage from step 2v + 3 on. B stage reuse: B tile t's fragments are read in
  // the second half of step t - 1 and waited for at the start of step t; tile t + 4 refills
  // the stage in step t + 1. Step t's barrier needs 32-wide tile t + 1 landed, issued in
  // step t - 2 or earlier, so each wave waits until at most the 8 instructions of steps
  // t - 1 and t are in flight. The prologue is steps -3 .. -1 of the same schedule.
  dma_a(0, 0, 0); dma_a(1, 0, 0); dma_a(2, 0, 0); dma_a(3, 0, 0);
  dma_b(0, 0, 0); dma_b(1, 0, 0);
  dma_b(0, 1, 1); dma_b(1, 1, 1);
  dma_a(0, 1, 1); dma_a(1, 1, 1); dma_a(2, 1, 1); dma_a(3, 1, 1);
  dma_b(0, 2, 2); dma_b(1, 2, 2);
  wait_vmcnt<8>();
  barrier_no_fence();

  i32x4 a_lo[4], a_hi[4], b0[4], b1[4];
  a_lo[0] = read_a<0>(lds_base + a_addr0);
  a_lo[1] = read_a<1>(lds_base + a_addr0);
  a_lo[2] = read_a<2>(lds_base + a_addr0);
  a_lo[3] = read_a<3>(lds_base + a_addr0);
#pragma unroll
  for (int j = 0; j < 4; ++j) b0[j] = read_b<kRowB>(lds_base + kBRing + b_addr[j]);

  // One 32-wide step t (half H of the 64-wide A tile in A stage sa; B stage sb). Bc holds
  // this step's B fragments, Bn receives the next step's. The next step reads A stage
  // sa_next (the same stage when H == 0) and B stage sb_next.
  auto step = [&](auto half, int t, int sa, int sa_next, int sb, int sb_next, i32x4 (&Bc)[4],
                  i32x4 (&Bn)[4]) {
    constexpr int H = decltype(half)::value;
    const uint32_t a_cur = lds_base + sa * kABytes + (H ? a_addr1 : a_addr0);
    const uint32_t a_next = lds_base + sa_next * kABytes + (H ? a_addr0 : a_addr1);
    const uint32_t b_next = lds_base + kBRing + sb_next * kOperandBytes;
    // Refill targets: B stage (t + 3) % 4 == (sb + 3) % 4, A stage of tile (t + 3) / 2.
    const int fill_b = sb == 0 ? 3 : sb - 1;
    const int fill_a = sa == 0 ? 2 : sa - 1;
    wait_lgkm_pin(a_lo);
    wait_lgkm_pin(Bc);
    sched_fence();
    // Rows 0-3; read rows 4-7 of this step, issue the DMA.
#pragma unroll
    for (int x = 0; x < 16; ++x) {
      const int i = x >> 2, j = x & 3;
      acc[i][j] = Mfma<T>::run(Bc[j], a_lo[i], acc[i][j]);
      sched_fence();
      if (j == 0) {
        if (i == 0) a_hi[0] = read_a<4>(a_cur);
        if (i == 1) a_hi[1] = read_a<5>(a_cur);
        if (i == 2) a_hi[2] = read_a<6>(a_cur);
        if (i == 3) a_hi[3] = read_a<7>(a_cur);
      }
      if (H == 1 && j == 1) dma_a(i, (t + 3) >> 1, fill_a);
      if (j == 3 && (i & 1) == 0) dma_b(i >> 1, t + 3, fill_b);
      sched_fence();
    }
    wait_vmcnt<8>();
    barrier_no_fence();
    wait_lgkm_pin(a_hi);
    sched_fence();
    // Rows 4-7; read rows 0-3 and B of step t + 1.
#pragma unroll
    for (int x = 0; x < 16; ++x) {
      const int i = x >> 2, j = x & 3;
      acc[4 + i][j] = Mfma<T>::run(Bc[j], a_hi[i], acc[4 + i][j]);
      sched_fence();
      if (j == 0) {
        if (i == 0) a_lo[0] = read_a<0>(a_next);
        if (i == 1) a_lo[1] = read_a<1>(a_next);
        if (i == 2) a_lo[2] = read_a<2>(a_next);
        if (i == 3) a_lo[3] = read_a<3>(a_next);
      }
      if (j == 2) Bn[i] = read_b<kRowB>(b_next + b_addr[i]);
      sched_fence();
    }
  };

  // 64-wide A tile u: steps 2u (B stage sb) and 2u + 1 (sb + 1), A stage sa.
  int sa = 0, sb = 0;
  for (int u = 0; 2 * u < kt; ++u) {
    const int sa_next = sa == kAStages - 1 ? 0 : sa + 1;
    step(std::integral_constant<int, 0>{}, 2 * u, sa, sa, sb, sb + 1, b0, b1);
    if (2 * u + 1 < kt)
      step(std::integral_constant<int, 1>{}, 2 * u + 1, sa, sa_next, sb + 1,
           sb + 2 == kBStages ? 0 : sb + 2, b1, b0);
    sa = sa_next;
    sb = sb + 2 == kBStages ? 0 : sb + 2;
  }
  wait_vmcnt<0>();
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");

  // acc[i][j] holds C^T: register r of lane l is C[m][n] with m = m0 + wm + 16 i + l % 16 and
  // n = n0 + (N tile j's first column) + 4 (l / 16) + r: four consecutive columns of one row.
  // The rings are idle once every wave is here, so when C rows are 16-byte aligned the block
  // stages its rounded tile in LDS and writes it back as whole rows, 16 bytes per lane, with
  // non-temporal stores of full 128-byte lines; otherwise each lane stores its four columns.
  // Staged, the epilogue of fp16 4096^3 took ~4 instead of ~8 us of a ~108 us launch (a
  // timing-only copy without stores ran 102 us): 4096^3 108.1 -> 104.3 us, 8192^3 784 ->
  // 773 us, the row-scaled 16384x6144x4096 GEMM 675 -> 645 us. Staged with default-policy
  // stores: 105.1, 773 and 654 us. Per-lane non-temporal stores write 32-byte segments of
  // four lines and were 5-14 % slower than default-policy ones.
  __syncthreads();
  const float* scales = reinterpret_cast<const float*>(lds + kScaleOff);
  if constexpr (kRowScale) {
    if (threadIdx.x < BM) reinterpret_cast<float*>(lds + kScaleOff)[threadIdx.x] = row_scale;
    __syncthreads();
  }
  // The tile's outputs as (row within the tile, column within the tile, four values).
  auto for_each_out = [&](auto&& emit) {
    if constexpr (kSwiGLU) {
#pragma unroll
      for (int jj = 0; jj < 2; ++jj) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          float v[4];
#pragma unroll
          for (int r = 0; r < 4; ++r)
            v[r] = static_cast<float>(swiglu_out<T>(acc[i][jj][r], acc[i][jj + 2][r]));
          emit(wm + i * 16 + l16, (wave & 3) * 32 + jj * 16 + lg * 4, v);
        }
      }
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float sc = kRowScale ? scales[wm + i * 16 + l16] : 1.f;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          float v[4];
#pragma unroll
          for (int r = 0; r < 4; ++r) v[r] = kRowScale ? acc[i][j][r] * sc : acc[i][j][r];
          emit(wm + i * 16 + l16, wn + j * 16 + lg * 4, v);
        }
      }
    }
  };
  auto pack4 = [](const float (&v)[4]) {
    const uint32_t lo = uint32_t(__builtin_bit_cast(uint16_t, tk::from_f32<T>(v[0]))) |
                        (uint32_t(__builtin_bit_cast(uint16_t, tk::from_f32<T>(v[1]))) << 16);
    const uint32_t hi = uint32_t(__builtin_bit_cast(uint16_t, tk::from_f32<T>(v[2]))) |
                        (uint32_t(__builtin_bit_cast(uint16_t, tk::from_f32<T>(v[3]))) << 16);
    return uint2{lo, hi};
  };
  const bool rows16 =
      p.scn == 1 && (p.scm & 7) == 0 && (reinterpret_cast<uintptr_t>(C) & 15) == 0;
  if (rows16) {
    // Stage rows of kTileN values at a stride of kTileN * 2 + 16 bytes (4 dwords past a
    // multiple of the 64 banks), so the 16 rows x 2 lane groups of an 8-byte write phase hit
    // distinct banks; then kTileN / 8 lanes per row copy 16 bytes each (p.n % 8 == 0, so a
    // 16-byte group is wholly inside or outside N).
    constexpr int kStride = kTileN * 2 + 16;
    static_assert(BM * kStride <= kScaleOff, "staged tile overlaps the row scales");
    for_each_out([&](int r, int c, const float (&v)[4]) {
      *reinterpret_cast<uint2*>(lds + r * kStride + c * 2) = pack4(v);
    });
    __syncthreads();
    constexpr int kLanesPerRow = kTileN / 8;
    constexpr int kRowsPerPass = kThreads / kLanesPerRow;
    const int cr = threadIdx.x / kLanesPerRow, cc = (threadIdx.x % kLanesPerRow) * 8;
#pragma unroll 4
    for (int pass = 0; pass < BM / kRowsPerPass; ++pass) {
      const int r = pass * kRowsPerPass + cr;
      const i32x4 v = *reinterpret_cast<const i32x4*>(lds + r * kStride + cc * 2);
      if (m0 + r < p.m && n0 + cc < p.n)
        __builtin_nontemporal_store(v, reinterpret_cast<i32x4*>(C + (m0 + r) * p.scm + n0 + cc));
    }
    return;
  }
  const bool vec = p.scn == 1 && (p.scm & 3) == 0 && (reinterpret_cast<uintptr_t>(C) & 7) == 0;
  for_each_out([&](int r, int c, const float (&v)[4]) {
    const int m = m0 + r, n = n0 + c;
    if (m >= p.m || n >= p.n) return;
    T* dst = C + m * p.scm + n * p.scn;
    if (vec) {  // p.n % 8 == 0, so n .. n+3 are in range
      *reinterpret_cast<uint2*>(dst) = pack4(v);
    } else {
#pragma unroll
      for (int q = 0; q < 4; ++q)
        if (n + q < p.n) dst[q * p.scn] = tk::from_f32<T>(v[q]);
    }
  });
}


}  // namespace

namespace tk {

bool gemm_dma_applies(const void* a, const void* b, int64_t m, int64_t n, int64_t k,
                      int64_t stride_am, int64_t stride_ak, int64_t stride_bk,
                      int64_t stride_bn) {
  // Buffer offsets are 32-bit with kOob (2^31) reserved as "outside"; row strides are
  // positive (the offsets are unsigned).
  if (m <= 0 || n <= 0 || k <= 0 || stride_am <= 0 || stride_bk <= 0) return false;
  const __int128 a_bytes = (extent(m, stride_am, 1, 0) + k) * 2;
  const __int128 b_bytes = (extent(k, stride_bk, 1, 0) + n) * 2;
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
