// Flash attention forward for head_dim 64/128 (f16/bf16) on CDNA4 MFMA: the path behind
// tk_attn_fwd (src/tklab/kernels/flash_attention.py:124-264 is the Triton kernel it
// replaces: base-2 online softmax on scores * scale * log2(e) in _attention_inner
// (:55-121), O = acc / l and log-sum-exp m + log2(l) (:248-264)).
//
// Workgroup: 256 queries, 8 wave64s of 32 queries (two 16-query tiles), two waves per SIMD.
// Key/value blocks of 64 (four 16-key tiles). All products are v_mfma_f32_16x16x32.
//
// Per wave and key block j:
//   S^T = K Q^T     4 key tiles x 2 query tiles over D/32 k-steps: lane l holds query
//                   16 qt + l % 16 and keys 16 kt + 4 (l / 16) + {0..3}, so a query's
//                   maximum and sum span the four lanes l % 16 + 16 {0..3} (permlane32 and
//                   permlane16 swaps).
//   softmax         masked only on diagonal / ragged blocks. The reference maximum only
//                   moves when a block's maximum exceeds it by more than 2^8 (exponentials
//                   stay <= 256), so O is rescaled in a few blocks rather than most, and
//                   the cross-lane maximum is only formed when some lane's own maximum
//                   would move it.
//   O^T += V^T P^T  D/16 feature tiles x 2 query tiles over two 32-key steps; P^T comes
//                   straight from the S^T registers (key tiles 2s and 2s + 1 give k-index
//                   0..3 and 4..7 of lane group l / 16), and V^T fragments are read with
//                   ds_read_b64_tr_b16 from row-major V rows in exactly that key order.
// Q fragments stay in registers for the whole key loop.
//
// Ping-pong: the barrier-separated phases alternate an MFMA phase M(j) (O^T += V_{j-1}^T
// P_{j-1}^T, then S^T_j) and a softmax phase V(j); the two waves of each SIMD (found from
// the hardware SIMD id) run opposite phases, so one wave's exponentials overlap the other's
// MFMAs. Each phase's register results are pinned before its barrier so the compiler
// cannot sink them into the next phase.
//
// K and V blocks reach LDS by buffer->LDS DMA (no VGPR staging) into a 4-stage ring; block
// j is read in phases 2j .. 2j+3 and its stage is refilled from phase 2j+4 on: each wave
// issues its share of block m + 2 spread over the read units of its MFMA phase of block m
// (issued as one burst after a barrier, the DMA instructions held the issuing waves ~300
// cycles per block; causal D128 1.91 -> 1.83 ms). LDS layouts keep every read phase on 64
// distinct banks:
//   K [64 keys][D]: 16-byte chunk c of row r at slot c ^ kswz(r) (ds_read_b128, 16 lanes
//                   per phase read one chunk of 16 rows);
//   V [64 keys][D]: 32-byte granule g of row r at granule g ^ vswz(r) (ds_read_b64_tr_b16,
//                   32 lanes per phase read one granule of 8 rows).
// The DMA writes 1 KiB contiguous per instruction, so the swizzle is applied on the global
// side (each lane fetches the chunk that belongs in its LDS slot). LDS reads are inline
// asm ordered by explicit waits: the compiler would otherwise wait for every outstanding
// DMA before each read.
#include "attention.hpp"
#include "attention_dma.hpp"

namespace {

using namespace tk_attn;

constexpr int kThreads = 512;
constexpr float kLazyRescale = 8.f;

struct Shape {
  int heads, seq;  // seq: the sequence length (varlen: the longest sequence)
  int group;  // query heads per KV head: K/V of head h are those of KV head h / group
  // Variable-length batches (null for equal lengths): sequence b is the rows
  // cu[b] .. cu[b+1] of a packed [total][head][dim] layout (the batch strides are 0),
  // and the LSE is [head][total].
  const int32_t* cu;
  int total, batch;
  int64_t q[3], k[3], v[3], o[3];  // batch, head, sequence strides (elements)
  float scale_log2;
  int q_blocks, tiles;
  uint32_t k_bytes, v_bytes;  // per-head buffer extents
  // RoPE applied to Q in the prologue (null: none): position-indexed tables [pos][D/2]
  // of T with row stride rope_stride; query i uses row i.
  const void* rope_cos;
  const void* rope_sin;
  int64_t rope_stride;
};

// Arguments of the forward kernel, passed as its only parameter (read through kernel_args
// in its tile loop).
template <typename T>
struct FwdArgs {
  const T* Q;
  const T* K;
  const T* V;
  T* O;
  float* lse;
  Shape s;
};

// Rotate-half RoPE of one 16-byte Q fragment pair: x1 holds features f .. f+7 and x2
// features f + D/2 .. f + D/2 + 7 (f < D/2); c and s hold cos/sin of f .. f+7. The
// arithmetic is the RoPE kernel's: products rounded separately (no contraction), then
// each result rounded to T, so the rotated Q is bitwise the one tk_rope_fwd stores.
template <typename T>
__device__ __forceinline__ void rope_fragment(i32x4& x1, i32x4& x2, i32x4 c, i32x4 s) {
#pragma clang fp contract(off)
  typedef T t8 __attribute__((ext_vector_type(8)));
  const t8 a = __builtin_bit_cast(t8, x1), b = __builtin_bit_cast(t8, x2);
  const t8 cv = __builtin_bit_cast(t8, c), sv = __builtin_bit_cast(t8, s);
  t8 y1, y2;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float xa = static_cast<float>(a[e]), xb = static_cast<float>(b[e]);
    const float ce = static_cast<float>(cv[e]), se = static_cast<float>(sv[e]);
    y1[e] = tk::from_f32<T>(xa * ce - xb * se);
    y2[e] = tk::from_f32<T>(xb * ce + xa * se);
  }
  x1 = __builtin_bit_cast(i32x4, y1);
  x2 = __builtin_bit_cast(i32x4, y2);
}

template <int D>
struct Geo {
  static constexpr int BM = 256, BN = 64, WAVES = 8, QW = 32;
  static constexpr int KS = D / 32;             // k-steps of S^T (32 features each)
  static constexpr int KH = KS / 2;             // k-steps per half of the feature range
  static constexpr int FT = D / 16;             // 16-feature tiles of O^T
  static constexpr int RB = D * 2;              // bytes per K/V row
  static constexpr int OPB = BN * RB;           // bytes per operand per stage
  static constexpr int STB = 2 * OPB;           // stage: K tile then V tile
  static constexpr int STAGES = 4;
  static constexpr int ROWS_PER_DMA = 1024 / RB;
  static constexpr int DMA_PER_OP = OPB / 1024 / WAVES;  // per wave, per operand
  static constexpr int DMA_PER_BLOCK = 2 * DMA_PER_OP;
  static constexpr int SLOTS = RB / 16;         // 16-byte slots per row
  // K: 16-byte chunk c of row r at slot c ^ kswz(r). A read phase (16 lanes) takes one
  // chunk of 16 consecutive rows.
  static __device__ __forceinline__ int kswz(int r) { return D == 128 ? (r & 15) : ((r >> 1) & 7); }
  // V: 32-byte granule g of row r at granule g ^ vswz(r). A transposed read phase (32
  // lanes) takes one granule of 8 consecutive rows.
  static __device__ __forceinline__ int vswz(int r) { return D == 128 ? (r & 7) : ((r >> 1) & 3); }
  // O staging: 16-byte granule q of staged row r at q ^ oswz(r). An 8-byte write phase (16
  // rows x 2 lane groups) and a 16-byte read phase then fall on distinct banks.
  static __device__ __forceinline__ int oswz(int r) { return D == 128 ? (r & 15) : ((r >> 1) & 7); }
};

// DMA of key/value block `blk` into its ring stage (clamped to `last`: blocks past the end
// reload the last one into a stage that is never read, keeping the per-phase load count
// constant).
template <int D>
__device__ __forceinline__ void dma_block(__amdgpu_buffer_rsrc_t rk, __amdgpu_buffer_rsrc_t rv,
                                          char* lds, const uint32_t* k_src,
                                          const uint32_t* v_src, int blk, int last,
                                          uint32_t k_blk, uint32_t v_blk, int wave) {
  using G = Geo<D>;
  char* stage = lds + (blk % G::STAGES) * G::STB;
  blk = min(blk, last);
#pragma unroll
  for (int x = 0; x < G::DMA_PER_OP; ++x) {
    const int id = wave * G::DMA_PER_OP + x;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rk, (lds_void*)(stage + id * 1024), 16, k_src[x],
                                             blk * k_blk, 0, 0);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rv, (lds_void*)(stage + G::OPB + id * 1024), 16,
                                             v_src[x], blk * v_blk, 0, 0);
  }
}

// DMA instruction i (0 .. DMA_PER_BLOCK - 1) of this wave's share of block `blk`: K chunks
// first, then V.
template <int D>
__device__ __forceinline__ void dma_one(__amdgpu_buffer_rsrc_t rk, __amdgpu_buffer_rsrc_t rv,
                                        char* lds, const uint32_t* k_src, const uint32_t* v_src,
                                        int blk, int last, uint32_t k_blk, uint32_t v_blk,
                                        int wave, int i) {
  using G = Geo<D>;
  char* stage = lds + (blk % G::STAGES) * G::STB;
  blk = min(blk, last);
  const int x = i % G::DMA_PER_OP;
  const int id = wave * G::DMA_PER_OP + x;
  if (i < G::DMA_PER_OP)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rk, (lds_void*)(stage + id * 1024), 16, k_src[x],
                                             blk * k_blk, 0, 0);
  else
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rv, (lds_void*)(stage + G::OPB + id * 1024), 16,
                                             v_src[x], blk * v_blk, 0, 0);
}

// The MFMA phase as a pipeline of read units of four LDS instructions each: V units
// (u < NV) hold 32-key step s = u / (FT/2) of feature tiles 2p and 2p+1 (p = u % (FT/2)),
// K units (u >= NV) k-step kk = u - NV of the four key tiles. Unit u's MFMAs run while
// units u+1 .. u+DEPTH-1 are in flight.
template <int D>
struct Units {
  static constexpr int FP = Geo<D>::FT / 2;  // feature-tile pairs per 32-key step
  static constexpr int NV = 2 * FP;          // V units of a block
  // Units in flight, and V units issued at the end of the softmax phase (at most 15 LDS
  // reads may be in flight before a wave's issue stalls). head_dim 64 keeps fewer in
  // flight to stay within 128 registers.
  static constexpr int DEPTH = D == 64 ? 3 : 4;
  static constexpr int PREFETCH = D == 64 ? 2 : 3;
};

// Issues V unit u of the V tile at vb into vu[u].
template <int D>
__device__ __forceinline__ void read_v_unit(i32x4 (&vu)[Units<D>::NV][2], uint32_t vb,
                                            const uint32_t (&va)[Geo<D>::FT], int u) {
  constexpr int FP = Units<D>::FP, RB = Geo<D>::RB;
  const int s = u / FP, p = u % FP;
#pragma unroll
  for (int i = 0; i < 2; ++i)
    vu[u][i] = s == 0 ? read_v16<0, RB>(vb + va[2 * p + i]) : read_v16<32, RB>(vb + va[2 * p + i]);
}

// The MFMA phase of one wave: O^T += V_{j-1}^T P^T from the previous softmax phase's pf
// (DO_PV; P^T is dead before S^T is produced), then S^T(j) = K_j Q^T into st (DO_S).
// kb / vb: LDS addresses of the K tile of block j and the V tile of block j-1. With DO_PV
// the first PREFETCH V units were issued by the preceding softmax phase.
template <typename T, int D, bool DO_S, bool DO_PV, typename Hook>
__device__ __forceinline__ void mfma_phase(Hook&& hook, uint32_t kb, uint32_t vb, const uint32_t (&ka)[Geo<D>::KS],
                                           const uint32_t (&va)[Geo<D>::FT],
                                           const i32x4 (&qf)[2][Geo<D>::KS], f32x4 (&st)[2][4],
                                           const i32x4 (&pf)[2][2], f32x4 (&acc)[Geo<D>::FT][2],
                                           i32x4 (&vu)[Units<D>::NV][2]) {
  using G = Geo<D>;
  constexpr int KS = G::KS, RB = G::RB, FP = Units<D>::FP;
  constexpr int NV = DO_PV ? Units<D>::NV : 0, NU = NV + (DO_S ? KS : 0);
  constexpr int DEPTH = Units<D>::DEPTH;
  constexpr int PRE = DO_PV ? Units<D>::PREFETCH : 0;  // units issued before the phase
  static_assert(!DO_PV || Units<D>::NV >= PRE, "the prefetched units are V units");
  i32x4 kf[KS][4];
  auto issue = [&](int u) {
    if (u < NV) {
      read_v_unit<D>(vu, vb, va, u);
    } else {
      const int kk = u - NV;
      const uint32_t a = kb + ka[kk];
      kf[kk][0] = lds_read_b128<0>(a);
      kf[kk][1] = lds_read_b128<16 * RB>(a);
      kf[kk][2] = lds_read_b128<32 * RB>(a);
      kf[kk][3] = lds_read_b128<48 * RB>(a);
    }
  };
#pragma unroll
  for (int u = PRE; u < DEPTH && u < NU; ++u) issue(u);
  sched_fence();
#pragma unroll
  for (int u = 0; u < NU; ++u) {
    // Units u+1 .. min(u+DEPTH, NU)-1 may still be in flight (four instructions each).
    const int after = (u + DEPTH < NU ? u + DEPTH : NU) - (u + 1);
    if (after >= 3)
      wait_lgkm<12>();
    else if (after == 2)
      wait_lgkm<8>();
    else if (after == 1)
      wait_lgkm<4>();
    else
      wait_lgkm<0>();
    if (u < NV) {
      const int s = u / FP, p = u % FP;
      pin(vu[u][0]);
      pin(vu[u][1]);
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int qt = 0; qt < 2; ++qt)
          acc[2 * p + i][qt] = Mma16<T>::run(vu[u][i], pf[qt][s], acc[2 * p + i][qt]);
    } else {
      const int kk = u - NV;
#pragma unroll
      for (int kt = 0; kt < 4; ++kt) pin(kf[kk][kt]);
#pragma unroll
      for (int kt = 0; kt < 4; ++kt)
#pragma unroll
        for (int qt = 0; qt < 2; ++qt)
          st[qt][kt] = Mma16<T>::run(kf[kk][kt], qf[qt][kk],
                                     kk == 0 ? f32x4{0.f, 0.f, 0.f, 0.f} : st[qt][kt]);
    }
    if (u + DEPTH < NU) issue(u + DEPTH);
    hook(u, NU);
    sched_fence();
  }
}

// head_dim 64 uses 64 KiB of LDS per workgroup: held to 128 registers, two workgroups
// share a CU (four waves per SIMD).
// Equal lengths at head_dim 128: one workgroup per causal pair of query blocks
// (paired_tile). Not at head_dim 64: at 128 registers the two-block loop spills inside the
// key loop (causal B4 H32 N8192 1.22 -> 1.42 ms).
template <int D>
constexpr bool kPaired = D == 128;

template <typename T, int D, bool CAUSAL>
__global__ __attribute__((amdgpu_flat_work_group_size(kThreads, kThreads),
                          amdgpu_waves_per_eu(D == 64 ? 4 : 2))) void
attn_fwd_dma_kernel(FwdArgs<T> kernel_arg) {
  using G = Geo<D>;
  constexpr int BM = G::BM, BN = G::BN, KS = G::KS, FT = G::FT, RB = G::RB, OPB = G::OPB,
                STB = G::STB, STAGES = G::STAGES, DPB = G::DMA_PER_BLOCK;
  __shared__ __attribute__((aligned(1024))) char lds[STAGES * STB];
  // O staging: 16 rows of D values per wave (one query tile at a time), 32 KiB at head_dim
  // 128 and 16 KiB at 64, so the ring and the staging fill the CU's 160 KiB (one workgroup
  // at 128, two at 64). Until the first epilogue it holds each wave's SIMD id.
  __shared__ __attribute__((aligned(16))) char ostage[G::WAVES * 16 * RB];

  const int wave0 = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint32_t lds_base = (uint32_t)(uintptr_t)(lds_void*)lds;
  // Ping-pong partner: the two waves that share a SIMD (hardware SIMD id from HW_ID) take
  // opposite phases; grp is the wave's rank (0 or 1) among them.
  int grp = 0;
  {
    int* simd_of = reinterpret_cast<int*>(ostage);
    if ((threadIdx.x & 63) == 0) simd_of[wave0] = simd_id();
    __syncthreads();
#pragma unroll
    for (int w = 0; w < G::WAVES; ++w)
      grp += (w < wave0 && simd_of[w] == simd_of[wave0]) ? 1 : 0;
    grp = __builtin_amdgcn_readfirstlane(grp) & 1;
  }

  // Causal, equal lengths, head_dim 128: the two query blocks paired_tile deals this
  // workgroup (blocks i and QB-1-i of one head). Otherwise one query block per workgroup;
  // varlen: the heavy-first schedule over every sequence's query blocks (level = query
  // block), heads interleaved over the XCDs.
  for (int it = 0; (kPaired<D> && CAUSAL) || it == 0; ++it) {
    const FwdArgs<T>& args = kernel_args<FwdArgs<T>>();
    const Shape& s = args.s;
    const T* __restrict__ Q = args.Q;
    const T* __restrict__ K = args.K;
    const T* __restrict__ V = args.V;
    int b, h, qb, start = 0, N = s.seq;
    uint32_t k_bytes = s.k_bytes, v_bytes = s.v_bytes;
    if (s.cu != nullptr) {
      if (it > 0) break;
      h = varlen_head(blockIdx.x, s.heads);
      VarlenTile vt;
      if (!varlen_tile(s.cu, s.batch, s.total, s.seq, BM, blockIdx.x / s.heads, vt)) break;
      b = vt.b;
      qb = vt.level;
      const VarlenRows rows = varlen_rows(s.cu, b, s.total, s.seq);
      start = rows.start;
      N = rows.n;
      if (qb * BM >= N) break;  // uniform: the whole workgroup leaves
      k_bytes = uint32_t(((N - 1) * s.k[2] + D) * 2);
      v_bytes = uint32_t(((N - 1) * s.v[2] + D) * 2);
    } else if constexpr (kPaired<D> && CAUSAL) {
      int bh, rank;
      if (!paired_tile(it, s.tiles / s.q_blocks, s.q_blocks, bh, rank)) break;
      qb = s.q_blocks - 1 - rank;
      b = bh / s.heads;
      h = bh % s.heads;
    } else {
      // One tile per workgroup: XCD-contiguous ranges so a head's blocks share one L2;
      // causal: the heaviest (last) query block of a head first.
      if (it > 0) break;
      int w = blockIdx.x;
      if (s.tiles % 8 == 0) w = (w % 8) * (s.tiles / 8) + w / 8;
      const int bh = w / s.q_blocks;
      qb = CAUSAL ? s.q_blocks - 1 - w % s.q_blocks : w % s.q_blocks;
      b = bh / s.heads;
      h = bh % s.heads;
    }
    // After the first tile: every wave has left the previous tile (its last LDS reads
    // are not followed by a barrier) before this tile's DMA refills the ring.
    if (it > 0) barrier_no_fence();
    // The lane and wave indices pass through an empty asm once per tile, so the addresses
    // derived from them are formed inside the tile rather than hoisted and held across the
    // loop.
    int lane = threadIdx.x & 63;
    int wave = wave0;
    if constexpr (kPaired<D> && CAUSAL) asm volatile("" : "+v"(lane), "+s"(wave));
    const int c = lane & 15, g = lane >> 4;
    const int kvh = h / s.group;
    const T* Qh = Q + b * s.q[0] + h * s.q[1] + int64_t(start) * s.q[2];
    const T* Kh = K + b * s.k[0] + kvh * s.k[1] + int64_t(start) * s.k[2];
    const T* Vh = V + b * s.v[0] + kvh * s.v[1] + int64_t(start) * s.v[2];

    const int q0 = qb * BM;
    const int wq0 = q0 + wave * G::QW;

    const __amdgpu_buffer_rsrc_t rk =
        __builtin_amdgcn_make_buffer_rsrc((void*)Kh, (short)0, k_bytes, 0x00020000);
    const __amdgpu_buffer_rsrc_t rv =
        __builtin_amdgcn_make_buffer_rsrc((void*)Vh, (short)0, v_bytes, 0x00020000);

    // DMA sources (bytes from the head's base, block-relative row). Rows past the sequence
    // end are past the buffer extent and read as zero.
    uint32_t k_src[G::DMA_PER_OP], v_src[G::DMA_PER_OP];
#pragma unroll
    for (int x = 0; x < G::DMA_PER_OP; ++x) {
      const int id = wave * G::DMA_PER_OP + x;
      const int row = id * G::ROWS_PER_DMA + lane / G::SLOTS;
      const int slot = lane % G::SLOTS;
      k_src[x] = uint32_t(row * s.k[2] + (slot ^ G::kswz(row)) * 8) * 2u;
      const int granule = (slot >> 1) ^ G::vswz(row);
      v_src[x] = uint32_t(row * s.v[2] + granule * 16 + (slot & 1) * 8) * 2u;
    }
    const int kv_end = CAUSAL ? min(N, q0 + BM) : N;
    const int kv_blocks = (kv_end + BN - 1) / BN;
    const int last = kv_blocks - 1;
    const uint32_t k_blk = uint32_t(BN * s.k[2]) * 2u, v_blk = uint32_t(BN * s.v[2]) * 2u;
    // The first STAGES - 1 blocks are fetched before anything else.
#pragma unroll
    for (int blk = 0; blk < STAGES - 1; ++blk)
      dma_block<D>(rk, rv, lds, k_src, v_src, blk, last, k_blk, v_blk, wave);

    // Q fragments (B operand of S^T): query tile qt holds query wq0 + 16 qt + c, k-step kk
    // features 32 kk + 8 g .. +7.
    i32x4 qf[2][KS];
#pragma unroll
    for (int qt = 0; qt < 2; ++qt) {
      const int query = wq0 + 16 * qt + c;
#pragma unroll
      for (int kk = 0; kk < KS; ++kk)
        qf[qt][kk] = query < N
                         ? *reinterpret_cast<const i32x4*>(Qh + query * s.q[2] + kk * 32 + g * 8)
                         : i32x4{0, 0, 0, 0};
    }
    // RoPE: fragments kk and kk + KS/2 hold features 32 kk + 8 g .. +7 and the same + D/2,
    // so the rotate-half pairs sit in one lane. Queries past the end keep zero tables (their
    // Q is 0).
    if (s.rope_cos != nullptr) {
#pragma unroll
      for (int qt = 0; qt < 2; ++qt) {
        const int query = wq0 + 16 * qt + c;
        const int64_t at = int64_t(query) * s.rope_stride + g * 8;
        const T* cr = static_cast<const T*>(s.rope_cos) + at;
        const T* sr = static_cast<const T*>(s.rope_sin) + at;
#pragma unroll
        for (int kk = 0; kk < KS / 2; ++kk) {
          const i32x4 cv = query < N ? *reinterpret_cast<const i32x4*>(cr + kk * 32) : i32x4{0, 0, 0, 0};
          const i32x4 sv = query < N ? *reinterpret_cast<const i32x4*>(sr + kk * 32) : i32x4{0, 0, 0, 0};
          rope_fragment<T>(qf[qt][kk], qf[qt][kk + KS / 2], cv, sv);
        }
      }
    }
    // Lane read addresses inside a stage: K row c of key tile kt (+16 kt rows), chunk
    // 4 kk + g; V rows 4 g + j (+32 per key step, +16 for k-index 4..7), features
    // 16 ft + 4 q .. +3, with j = c / 4, q = c % 4.
    uint32_t ka[KS], va[FT];
#pragma unroll
    for (int kk = 0; kk < KS; ++kk) ka[kk] = c * RB + (((4 * kk + g) ^ G::kswz(c)) * 16);
    {
      const int row = 4 * g + (c >> 2), q = c & 3;
#pragma unroll
      for (int ft = 0; ft < FT; ++ft) va[ft] = OPB + row * RB + ((ft ^ G::vswz(row)) * 32) + q * 8;
    }

    // O^T accumulators: acc[ft][qt] register r is feature 16 ft + 4 g + r of query
    // wq0 + 16 qt + c. st[qt][kt] register r: score of key n0 + 16 kt + 4 g + r.
    f32x4 acc[FT][2], st[2][4];
    i32x4 pf[2][2], vu[Units<D>::NV][2];
#pragma unroll
    for (int ft = 0; ft < FT; ++ft)
#pragma unroll
      for (int qt = 0; qt < 2; ++qt) acc[ft][qt] = f32x4{0.f, 0.f, 0.f, 0.f};
    float m_run[2] = {kNegInf, kNegInf}, l_part[2] = {0.f, 0.f};
    const float sl2 = s.scale_log2;

    // Block 0 landed.
    wait_lgkm<0>();
    wait_vmcnt<(STAGES - 2) * DPB>();
    barrier_no_fence();
    // Ping-pong: the two waves that share a SIMD take opposite phases. The workgroup runs
    // phases t = 0, 1, ... separated by barriers; a wave alternates an MFMA phase M(j)
    // (S^T of block j, O^T += V^T P^T of block j-1) and a softmax phase V(j), the second
    // wave of each SIMD one phase behind the first, so one wave's exponentials run while
    // the other's MFMAs occupy the matrix pipe. Block j is read in phases 2j .. 2j+3; at
    // the start of phase 2m (m >= 1) its stage's next block m + STAGES - 2 is fetched,
    // and block m must have landed before phase 2m begins.
    const int phases = 2 * kv_blocks + 2;
    int t = 0;
    // Block m + STAGES - 2 (m >= 1) is fetched during this wave's MFMA phase of block m
    // (phase 2m + grp), its DMA_PER_BLOCK instructions spread over the phase's read units;
    // after the wave's last MFMA phase, at the start of phase 2m + grp (tail mode). Block m+1
    // was issued by every wave before the end of phase 2m + 1 (grp 0 in phase 2m - 2, grp 1
    // in 2m - 1), so the wait at the end of each odd phase, which leaves one block's
    // instructions in flight, still covers it.
    bool tail = false;
    int tail_m = 0;
    auto end_phase = [&]() {
      if (t & 1) wait_vmcnt<(STAGES - 3) * DPB>();
      barrier_no_fence();
      ++t;
      if (tail && tail_m <= kv_blocks && t == 2 * tail_m + grp) {
        dma_block<D>(rk, rv, lds, k_src, v_src, tail_m + STAGES - 2, last, k_blk, v_blk, wave);
        ++tail_m;
      }
    };
    // Hook of the MFMA phase of block m: after unit u of nu, the DMA instructions whose
    // share of the phase ends there (DMA_PER_BLOCK of them over the nu units).
    auto dma_hook = [&](int m) {
      return [&, m](int u, int nu) {
        const int a = (u * DPB) / nu, b2 = ((u + 1) * DPB) / nu;
        if (b2 != a)
          dma_one<D>(rk, rv, lds, k_src, v_src, m + STAGES - 2, last, k_blk, v_blk, wave, b2 - 1);
      };
    };
    auto no_hook = [](int, int) {};
    auto kbase = [&](int j) { return lds_base + (j % STAGES) * STB; };

    // Softmax phase of block j: P = exp2(S * scale * log2(e) - m) into pf, the running
    // statistics updated. The reference maximum m_run only moves when the block's maximum
    // exceeds it by more than kLazyRescale (log2 units): exponentials stay
    // <= 2^kLazyRescale, and O and l are rescaled in few blocks instead of whenever one of
    // the wave's 32 maxima grows. O = acc / l and the log-sum-exp m_run + log2(l) do not
    // depend on which reference is used.
    auto softmax_phase = [&](int j) {
      const int n0 = j * BN;
      const bool need_mask = n0 + BN > N || (CAUSAL && n0 + BN - 1 > wq0);
      if (__builtin_expect(need_mask, 0)) {
#pragma unroll
        for (int qt = 0; qt < 2; ++qt)
#pragma unroll
          for (int kt = 0; kt < 4; ++kt) {
            const int k0 = n0 + 16 * kt + 4 * g;  // the lane's first key of this tile
            int lim = N - 1 - k0;                 // last valid offset from k0
            if (CAUSAL) lim = min(lim, wq0 + 16 * qt + c - k0);
#pragma unroll
            for (int r = 0; r < 4; ++r)
              if (r > lim) st[qt][kt][r] = kNegInf;
          }
      }
      if constexpr (D == 128) {
        // Exponentials against the current reference first. A lane whose 16 exponentials of a
        // query sum to at most 2^kLazyRescale has none above it, so when no lane of the wave
        // exceeds that sum no reference moves and no maximum is needed. Otherwise the column
        // maxima are formed from the scores, which are still intact, and the queries whose
        // reference moves are recomputed.
        f32x4 p[2][4];
        float sum[2];
        auto exps = [&](int qt) {
          const float neg = -m_run[qt];
    #pragma unroll
          for (int kt = 0; kt < 4; ++kt)
    #pragma unroll
            for (int r = 0; r < 4; ++r)
              p[qt][kt][r] = __builtin_amdgcn_exp2f(__builtin_fmaf(st[qt][kt][r], sl2, neg));
          float s0 = p[qt][0][0];
    #pragma unroll
          for (int i = 1; i < 16; ++i) s0 += p[qt][i / 4][i % 4];
          sum[qt] = s0;
        };
        exps(0);
        exps(1);
        constexpr float kLazyLimit = 256.f;  // 2^kLazyRescale
        if (__builtin_expect(
                __builtin_amdgcn_ballot_w64(!(sum[0] <= kLazyLimit) || !(sum[1] <= kLazyLimit)) != 0,
                0)) {
    #pragma unroll
          for (int qt = 0; qt < 2; ++qt) {
            float mx = kNegInf;
    #pragma unroll
            for (int kt = 0; kt < 4; ++kt)
    #pragma unroll
              for (int r = 0; r < 4; ++r) mx = fmaxf(mx, st[qt][kt][r]);
            const float bm = max_over_column(mx) * sl2;
            const bool move = bm > m_run[qt] + kLazyRescale;
            if (__builtin_amdgcn_ballot_w64(move)) {
              const float m_new = move ? bm : m_run[qt];
              const float alpha = move ? __builtin_amdgcn_exp2f(m_run[qt] - m_new) : 1.f;
              l_part[qt] *= alpha;
    #pragma unroll
              for (int ft = 0; ft < FT; ++ft) acc[ft][qt] *= alpha;
              m_run[qt] = m_new;
              exps(qt);
            }
          }
        }
    #pragma unroll
        for (int qt = 0; qt < 2; ++qt) {
          l_part[qt] += sum[qt];
          pf[qt][0] = acc_frag2<T>(p[qt][0], p[qt][1]);
          pf[qt][1] = acc_frag2<T>(p[qt][2], p[qt][3]);
        }
      } else {
        // head_dim 64 (128 registers): the exponentials overwrite the scores, so the maximum
        // comes first. A column's maximum exceeds the threshold only if one of its four
        // lanes' does: the cross-lane reduction runs only when some lane of the wave sees
        // such a maximum.
        float mx[2], m_new[2];
        bool move[2];
#pragma unroll
        for (int qt = 0; qt < 2; ++qt) {
          mx[qt] = kNegInf;
#pragma unroll
          for (int kt = 0; kt < 4; ++kt)
#pragma unroll
            for (int r = 0; r < 4; ++r) mx[qt] = fmaxf(mx[qt], st[qt][kt][r]);
          move[qt] = mx[qt] * sl2 > m_run[qt] + kLazyRescale;
          m_new[qt] = m_run[qt];
        }
        if (__builtin_expect(__builtin_amdgcn_ballot_w64(move[0] || move[1]) != 0, 0)) {
#pragma unroll
          for (int qt = 0; qt < 2; ++qt) {
            const float bm = max_over_column(mx[qt]) * sl2;
            move[qt] = bm > m_run[qt] + kLazyRescale;
            m_new[qt] = move[qt] ? bm : m_run[qt];
          }
        }
#pragma unroll
        for (int qt = 0; qt < 2; ++qt) {
          const float neg = -m_new[qt];
          float sum = 0.f;
#pragma unroll
          for (int kt = 0; kt < 4; ++kt)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              const float pv = __builtin_amdgcn_exp2f(__builtin_fmaf(st[qt][kt][r], sl2, neg));
              st[qt][kt][r] = pv;
              sum += pv;
            }
          if (__builtin_amdgcn_ballot_w64(move[qt])) {
            const float alpha = move[qt] ? __builtin_amdgcn_exp2f(m_run[qt] - m_new[qt]) : 1.f;
            l_part[qt] *= alpha;
#pragma unroll
            for (int ft = 0; ft < FT; ++ft) acc[ft][qt] *= alpha;
          }
          l_part[qt] += sum;
          m_run[qt] = m_new[qt];
          pf[qt][0] = acc_frag2<T>(st[qt][0], st[qt][1]);
          pf[qt][1] = acc_frag2<T>(st[qt][2], st[qt][3]);
        }
      }
    };

    // This wave multiplies a prefix of the workgroup's blocks (causal: those starting at or
    // before its last query); every wave takes part in every phase's barrier and loads.
    const int n = CAUSAL ? min(kv_blocks, (wq0 + G::QW - 1) / BN + 1) : kv_blocks;
    // The loop is entered after M(0) and leaves before V(n-1) (with the softmax phase first
    // in the body the compiler keeps one copy of the O accumulators across the back edge).
    // A phase's results are pinned before its closing barrier: the barrier orders memory
    // only, and the compiler would otherwise sink register work (the exponentials, the
    // MFMA chains) into the next phase, where it runs beside the partner wave's same kind
    // of work.
    auto pin_mfma = [&]() {
#pragma unroll
      for (int qt = 0; qt < 2; ++qt)
#pragma unroll
        for (int kt = 0; kt < 4; ++kt) pin(st[qt][kt]);
#pragma unroll
      for (int ft = 0; ft < FT; ++ft)
#pragma unroll
        for (int qt = 0; qt < 2; ++qt) pin(acc[ft][qt]);
    };
    // The softmax phase ends by issuing the first PREFETCH V units of the next MFMA phase
    // (block j's V tile has landed since phase 2j).
    auto pin_softmax = [&](int j) {
#pragma unroll
      for (int qt = 0; qt < 2; ++qt) {
        pin(pf[qt][0]);
        pin(pf[qt][1]);
        asm volatile("" : "+v"(l_part[qt]), "+v"(m_run[qt]));
      }
#pragma unroll
      for (int u = 0; u < Units<D>::PREFETCH; ++u) read_v_unit<D>(vu, kbase(j), va, u);
    };
    if (grp) end_phase();
    mfma_phase<T, D, true, false>(no_hook, kbase(0), 0, ka, va, qf, st, pf, acc, vu);
    pin_mfma();
    end_phase();
    for (int j = 1; j < n; ++j) {
      softmax_phase(j - 1);
      pin_softmax(j - 1);
      end_phase();
      mfma_phase<T, D, true, true>(dma_hook(j), kbase(j), kbase(j - 1), ka, va, qf, st, pf, acc, vu);
      pin_mfma();
      end_phase();
    }
    softmax_phase(n - 1);
    pin_softmax(n - 1);
    end_phase();
    mfma_phase<T, D, false, true>(dma_hook(n), 0, kbase(n - 1), ka, va, qf, st, pf, acc, vu);
    tail = true;
    tail_m = n + 1;
    while (t < phases - 1) end_phase();
    // No DMA may still be writing when the workgroup's LDS is released.
    wait_vmcnt<0>();

    // O = O^T / l: acc[ft][qt] register r is feature 16 ft + 4 g + r of query
    // wq0 + 16 qt + c, 8 bytes once rounded. Each query tile goes through the wave's own
    // staging rows and leaves as whole rows, 16 bytes per lane and full 128-byte lines, with
    // non-temporal stores (the per-lane 8-byte stores wrote 32-byte pieces of lines); the
    // entry points accept only 16-byte aligned tensors and strides that are multiples of 8
    // elements, so every O row is 16-byte aligned. The staging rows belong to one wave: no
    // barrier. The output pointer, strides and lane indices are formed here afresh rather
    // than held across the key loop (at head_dim 64 that spilled registers).
    const FwdArgs<T>& ea = kernel_args<FwdArgs<T>>();
    int el = threadIdx.x & 63;
    asm volatile("" : "+v"(el));
    const int ec = el & 15, eg = el >> 4;
    const int64_t o_row = ea.s.o[2];
    T* const Oe = ea.O + b * ea.s.o[0] + h * ea.s.o[1] + int64_t(start) * o_row;
    char* const orows = ostage + wave * (16 * RB);
#pragma unroll
    for (int qt = 0; qt < 2; ++qt) {
      const float l = sum_over_column(l_part[qt]);
      const float inv = 1.0f / l;
#pragma unroll
      for (int ft = 0; ft < FT; ++ft) {
        uint2 u;
        u.x = pack2<T>(acc[ft][qt][0] * inv, acc[ft][qt][1] * inv);
        u.y = pack2<T>(acc[ft][qt][2] * inv, acc[ft][qt][3] * inv);
        *reinterpret_cast<uint2*>(orows + ec * RB + (((2 * ft + (eg >> 1)) ^ G::oswz(ec)) * 16) +
                                  (eg & 1) * 8) = u;
      }
      constexpr int LPR = RB / 16, RPI = 64 / LPR;  // lanes per row, rows per instruction
#pragma unroll
      for (int p = 0; p < 16 / RPI; ++p) {
        const int r = p * RPI + el / LPR, q = el % LPR;
        const i32x4 v = *reinterpret_cast<const i32x4*>(orows + r * RB + ((q ^ G::oswz(r)) * 16));
        const int row_query = wq0 + 16 * qt + r;
        if (row_query < N)
          __builtin_nontemporal_store(v, reinterpret_cast<i32x4*>(Oe + row_query * o_row + q * 8));
      }
      const int query = wq0 + 16 * qt + ec;
      if (query < N && ea.lse != nullptr && eg == 0) {
        const int64_t at = ea.s.cu != nullptr ? int64_t(h) * ea.s.total + start + query
                                              : (int64_t(b) * ea.s.heads + h) * N + query;
        ea.lse[at] = m_run[qt] + __log2f(l);
      }
    }
  }  // tiles
}

// Causal head_dim 128, equal lengths: `items` workgroups (paired_items); otherwise one
// workgroup per query block.
template <typename T, int D>
void launch(bool causal, int64_t items, hipStream_t st, const void* q, const void* k,
            const void* v, void* o, float* lse, const Shape& s) {
  const int64_t n = kPaired<D> && causal && s.cu == nullptr ? items : int64_t(s.tiles);
  const dim3 grid(static_cast<unsigned>(n));
  const FwdArgs<T> a{(const T*)q, (const T*)k, (const T*)v, (T*)o, lse, s};
  if (causal)
    hipLaunchKernelGGL((attn_fwd_dma_kernel<T, D, true>), grid, dim3(kThreads), 0, st, a);
  else
    hipLaunchKernelGGL((attn_fwd_dma_kernel<T, D, false>), grid, dim3(kThreads), 0, st, a);
}

int64_t head_extent_bytes(int64_t seq, int64_t head_dim, int64_t seq_stride) {
  return ((seq - 1) * seq_stride + head_dim) * 2;
}

}  // namespace

namespace tk {

bool attn_fwd_dma_applies(int64_t seq, int64_t head_dim, const int64_t* k_strides,
                          const int64_t* v_strides) {
  // Buffer offsets are 32-bit: each head's K and V rows must span less than 2 GiB.
  const int64_t lim = int64_t(1) << 31;
  return head_extent_bytes(seq, head_dim, k_strides[2]) < lim &&
         head_extent_bytes(seq, head_dim, v_strides[2]) < lim;
}

void attn_fwd_dma_launch(int dtype, const void* q, const void* k, const void* v, void* o,
                         float* lse, int64_t batch, int64_t heads, int64_t kv_heads, int64_t seq,
                         int64_t head_dim, const int64_t* q_strides, const int64_t* k_strides,
                         const int64_t* v_strides, const int64_t* o_strides, float sm_scale,
                         bool causal, hipStream_t stream, const int32_t* cu_seqlens,
                         int64_t total, const void* rope_cos, const void* rope_sin,
                         int64_t rope_stride) {
  Shape s{};
  s.rope_cos = rope_cos;
  s.rope_sin = rope_sin;
  s.rope_stride = rope_stride;
  s.heads = (int)heads;
  s.seq = (int)seq;
  s.group = (int)(heads / kv_heads);
  s.cu = cu_seqlens;
  s.total = (int)total;
  for (int i = 0; i < 3; ++i) {
    s.q[i] = q_strides[i];
    s.k[i] = k_strides[i];
    s.v[i] = v_strides[i];
    s.o[i] = o_strides[i];
  }
  s.scale_log2 = sm_scale * 1.4426950408889634f;
  s.batch = (int)batch;
  s.q_blocks = (int)cdiv(seq, 256);
  s.tiles = cu_seqlens != nullptr ? (int)(varlen_tiles(batch, total, seq, 256) * heads)
                                  : (int)(s.q_blocks * batch * heads);
  s.k_bytes = (uint32_t)head_extent_bytes(seq, head_dim, k_strides[2]);
  s.v_bytes = (uint32_t)head_extent_bytes(seq, head_dim, v_strides[2]);
  const int64_t items = cu_seqlens == nullptr ? paired_items(batch * heads, s.q_blocks)
                                              : int64_t(s.tiles);
  if (dtype == TK_DTYPE_F16) {
    if (head_dim == 64) launch<_Float16, 64>(causal, items, stream, q, k, v, o, lse, s);
    else launch<_Float16, 128>(causal, items, stream, q, k, v, o, lse, s);
  } else {
    if (head_dim == 64) launch<__bf16, 64>(causal, items, stream, q, k, v, o, lse, s);
    else launch<__bf16, 128>(causal, items, stream, q, k, v, o, lse, s);
  }
}

}  // namespace tk
