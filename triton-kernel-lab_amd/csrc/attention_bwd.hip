// Flash attention recompute backward for head_dim 64/128 (f16/bf16) on CDNA4 MFMA: the
// dK/dV pass behind tk_attn_bwd_dkdv (src/tklab/kernels/flash_attention.py:383-491:
// P = exp2(S * scale * log2(e) - lse), dS = P (dP - delta), dV = P^T dO, dK = scale dS^T Q;
// each output is written by exactly one workgroup, so the pass is deterministic). The dQ
// pass is attention_bwd_dq.hip.
//
// head_dim 128, attn_bwd_dkdv_pp_kernel. Workgroup: 128 keys, 8 wave64s in 4
// producer/consumer pairs of 32 keys (waves w and w + 4, which share a SIMD), streaming the
// query blocks of 64; all products are v_mfma_f32_16x16x32. Per pair and query block:
//   producer  S = Q K^T, dP = dO V^T (Q / dO rows as A operands, ds_read_b128; K and V
//             fragments in registers), then P = exp2(S c - lse), dS = P (dP - delta),
//             written to LDS as the consumer's B-operand fragments (lane = key);
//   consumer  dV^T += dO^T P, dK^T += Q^T dS with dO^T / Q^T read transposed
//             (ds_read_b64_tr_b16) from the same tiles, accumulators in registers.
// Barrier-separated phases: producer MFMA (block v) | producer elementwise (v) | ...; the
// consumer reads block v - 1's exchange fragments at the start of the producer's MFMA
// phase v and runs its MFMAs for v - 1 beside the producer's elementwise phase (non-causal:
// its first 2 of 16 read units already beside the producer's MFMAs), so the exponentials of
// one wave run beside the other wave's MFMAs. Each wave holds only half of the state (K/V
// and S/dP, or the dK/dV accumulators), and one 8 KiB exchange buffer per pair suffices.
// Q/dO tiles reach LDS by buffer->LDS DMA into a ring (block v is read in phases 2v - 1 ..
// 2v+3); tiles read both ways store the 16-byte chunk c of row r at slot c ^ swz(r), which
// keeps the 16-row ds_read_b128 phases and the transposed phases on distinct banks.
//
// head_dim 64, attn_bwd_dkdv_dma_kernel: a workgroup owns 128 keys (4 wave64s x 32, one
// wave per SIMD) and walks the query blocks of 64. It is held to 256 registers, so two
// workgroups share a CU and each SIMD has a second wave to cover the first one's LDS and
// MFMA latencies (at head_dim 64 the pair kernel's elementwise phase, the same work as at
// 128, outlasts the consumer's halved MFMA phase). K and V fragments stay in registers.
// Per query block each wave computes S = Q K^T and dP = dO V^T (32x32x16 MFMAs,
// accumulator lane = one key, so P and dS feed the next MFMAs as B operands straight from
// registers), then dV^T += dO^T P and dK^T += Q^T dS with dO^T / Q^T read transposed from
// the same row-major tiles that S and dP read with ds_read_b128. Tiles reach LDS by
// buffer->LDS DMA into a 3-stage ring, two blocks ahead, one barrier per block.
#include "attention.hpp"
#include "attention_dma.hpp"

namespace {

using namespace tk_attn;

constexpr int kThreads = 512;   // producer/consumer kernel (head_dim 128)
constexpr int kThreads1 = 256;  // one-wave-per-SIMD kernel (head_dim 64)

struct BwdShape {
  int heads, seq;       // query heads
  int group;            // query heads per KV head (1: multi-head attention)
  int64_t st[3];        // batch, head, sequence strides of q, dO, dQ
  int64_t kst[3];       // batch, head, sequence strides of k, v, dK, dV
  float scale, scale_log2;
  int blocks_per_head;  // 128-row blocks per head
  int tiles, kv_tiles;  // dQ grid (query heads), dK/dV grid (KV heads)
  uint32_t head_bytes;     // extent of one query head's rows
  uint32_t kv_head_bytes;  // extent of one KV head's rows
  // Variable-length batches (null for equal lengths): sequence b is rows cu[b] ..
  // cu[b+1] of packed [total][head][dim] tensors (batch strides 0; seq is the longest
  // length), and lse / delta are [head][total].
  const int32_t* cu;
  int total, batch;
};

// Sequence b of a batch: its first row and length, and the buffer extents of one of
// its query-side / KV-side heads. Varlen lengths are clamped into [0, total] and to
// seq, so no lengths table can address rows outside the packed tensors.
struct SeqSpan {
  int start, n;
  uint32_t q_bytes, kv_bytes;
};

template <int D>
__device__ __forceinline__ SeqSpan seq_span(const BwdShape& s, int b) {
  if (s.cu == nullptr) return {0, s.seq, s.head_bytes, s.kv_head_bytes};
  const VarlenRows r = varlen_rows(s.cu, b, s.total, s.seq);
  return {r.start, r.n, uint32_t(((r.n - 1) * s.st[2] + D) * 2),
          uint32_t(((r.n - 1) * s.kst[2] + D) * 2)};
}

template <int D>
struct BwdGeo {
  static constexpr int WAVES = 4, LW = 32;     // rows (keys or queries) per wave
  static constexpr int BW = WAVES * LW;        // rows per workgroup: 128
  static constexpr int BB = 64;                // rows per streamed block
  static constexpr int KS = D / 16, DT = D / 32;
  static constexpr int RB = D * 2;             // bytes per row
  static constexpr int TILE = BB * RB;         // bytes per streamed tile
  static constexpr int STAGES = 3;
  static constexpr int ROWS_PER_DMA = 1024 / RB;
  static constexpr int DMA_PER_TILE = TILE / 1024 / WAVES;  // per wave
  static constexpr int SLOTS = RB / 16;        // 16-byte slots per row
  // Layout for tiles read only with ds_read_b128 (16 rows, one chunk per phase).
  static __device__ __forceinline__ int row_swz(int r) {
    return D == 128 ? (r & 15) : ((r >> 1) & 7);
  }
  // Layout for tiles also read with ds_read_b64_tr_b16 (4 rows x 4 chunks per phase).
  static __device__ __forceinline__ int dual_swz(int r) {
    return D == 128 ? (((r & 3) << 2) | ((r >> 2) & 3))
                    : ((((r >> 1) & 1) << 2) | ((r >> 2) & 3));
  }
};

// Source offset (bytes, tile-relative row) of DMA `x` of this wave for a [64][D] tile
// stored with swizzle `swz`.
template <int D, bool DUAL>
__device__ __forceinline__ uint32_t tile_src(int wave, int x, int lane, int64_t row_stride) {
  using G = BwdGeo<D>;
  const int id = wave * G::DMA_PER_TILE + x;
  const int row = id * G::ROWS_PER_DMA + lane / G::SLOTS;
  const int slot = lane % G::SLOTS;
  const int chunk = slot ^ (DUAL ? G::dual_swz(row) : G::row_swz(row));
  return uint32_t(row * row_stride + chunk * 8) * 2u;
}

// Lane address (bytes, inside a tile) of the A-operand fragment for a 32-row tile read
// with ds_read_b128: row lane % 32, chunk 2 kk + lane / 32.
template <int D, bool DUAL>
__device__ __forceinline__ uint32_t frag_addr(int lane, int kk) {
  using G = BwdGeo<D>;
  const int row = lane & 31;
  const int swz = DUAL ? G::dual_swz(row) : G::row_swz(row);
  return row * G::RB + (((2 * kk + (lane >> 5)) ^ swz) * 16);
}

// Lane address of a transposed read (ds_read_b64_tr_b16) of feature tile dt: rows
// 4 hi + j + half8 (k-index 0..3 for half8 = 0, 4..7 for half8 = 8; +16 per 16-row
// step), features 32 dt + 16 g + 4 q. The dual swizzle uses row bits 0..3, so the
// two row groups get their own addresses; only the step (row bits 4..5) is folded
// into the instruction's immediate offset.
template <int D>
__device__ __forceinline__ uint32_t tr_addr(int lane, int dt, int half8) {
  using G = BwdGeo<D>;
  const int g = (lane >> 4) & 1, j = (lane & 15) >> 2, q = lane & 3, hi = lane >> 5;
  const int row = 4 * hi + j + half8;
  const int chunk = 2 * (2 * dt + g) + (q >> 1);
  return row * G::RB + ((chunk ^ G::dual_swz(row)) * 16) + (q & 1) * 8;
}

// Transposed fragment of the 16 rows starting at ROW0 (a multiple of 16) of the tile
// OFF bytes past the lane addresses.
template <int ROW0, int RB, int OFF>
__device__ __forceinline__ i32x4 read_tr(uint32_t addr0, uint32_t addr8) {
  const i32x2 a = lds_read_tr16<OFF + ROW0 * RB>(addr0);
  const i32x2 b = lds_read_tr16<OFF + ROW0 * RB>(addr8);
  return i32x4{a[0], a[1], b[0], b[1]};
}

template <int RB, int OFF = 0>
__device__ __forceinline__ i32x4 read_tr_step(int step, uint32_t addr0, uint32_t addr8) {
  switch (step) {
    case 0: return read_tr<0, RB, OFF>(addr0, addr8);
    case 1: return read_tr<16, RB, OFF>(addr0, addr8);
    case 2: return read_tr<32, RB, OFF>(addr0, addr8);
    default: return read_tr<48, RB, OFF>(addr0, addr8);
  }
}

// Row fragment (ds_read_b128) of row tile `mt` (32 rows = 32 * RB bytes) of the tile
// OFF bytes past the lane address.
template <int RB, int OFF = 0>
__device__ __forceinline__ i32x4 read_row(int mt, uint32_t addr) {
  return mt == 0 ? lds_read_b128<OFF>(addr) : lds_read_b128<OFF + 32 * RB>(addr);
}


// DMA of one [64][D] tile of each of two tensors (rsrc a -> stage, rsrc b -> stage + TILE):
// this wave's DMA_PER_TILE loads of each, `blk_off` bytes into the head.
template <int D>
__device__ __forceinline__ void dma_tiles(__amdgpu_buffer_rsrc_t ra, __amdgpu_buffer_rsrc_t rb,
                                          char* stage, const uint32_t* a_src,
                                          const uint32_t* b_src, uint32_t blk_off, int wave) {
  using G = BwdGeo<D>;
#pragma unroll
  for (int x = 0; x < G::DMA_PER_TILE; ++x) {
    const int id = wave * G::DMA_PER_TILE + x;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, (lds_void*)(stage + id * 1024), 16, a_src[x],
                                             blk_off, 0, 0);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rb, (lds_void*)(stage + G::TILE + id * 1024), 16,
                                             b_src[x], blk_off, 0, 0);
  }
}

// DMA of 32 statistics floats (lanes 0..31, 4 bytes each) to `dst`.
__device__ __forceinline__ void dma_stats(__amdgpu_buffer_rsrc_t rs, char* dst, uint32_t src,
                                          uint32_t blk_off, int lane) {
  if (lane < 32) __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void*)dst, 4, src, blk_off, 0, 0);
}

__device__ __forceinline__ int acc_row(int r, int hi) { return ((r >> 2) << 3) + (hi << 2) + (r & 3); }



// Row operands of one 32-query sub-block of the dK/dV pass: Q and dO fragments
// (ds_read_b128, features 16 kk + 8 hi .. +7 of query lane % 32) and the lse / delta of
// the 16 queries this lane's accumulator registers hold (4 groups of 4 consecutive).
struct SubRows {
  i32x4 q[8], o[8];
  i32x4 lse[4], dlt[4];
};

template <int D>
__device__ __forceinline__ void read_sub_rows(SubRows& r, int mt, const uint32_t* qa,
                                              uint32_t sa) {
  constexpr int KS = D / 16, RB = D * 2, TILE = 64 * RB;
#pragma unroll
  for (int kk = 0; kk < KS; ++kk) {
    r.q[kk] = read_row<RB>(mt, qa[kk]);
    r.o[kk] = read_row<RB, TILE>(mt, qa[kk]);
  }
  // Statistics of query group g of tile mt start at float 32 mt + 8 g (+ 4 hi, in sa, which
  // already points at the stage's statistics); delta follows lse after 64 floats.
  if (mt == 0) {
    r.lse[0] = lds_read_b128<0>(sa);   r.dlt[0] = lds_read_b128<256>(sa);
    r.lse[1] = lds_read_b128<32>(sa);  r.dlt[1] = lds_read_b128<288>(sa);
    r.lse[2] = lds_read_b128<64>(sa);  r.dlt[2] = lds_read_b128<320>(sa);
    r.lse[3] = lds_read_b128<96>(sa);  r.dlt[3] = lds_read_b128<352>(sa);
  } else {
    r.lse[0] = lds_read_b128<128>(sa); r.dlt[0] = lds_read_b128<384>(sa);
    r.lse[1] = lds_read_b128<160>(sa); r.dlt[1] = lds_read_b128<416>(sa);
    r.lse[2] = lds_read_b128<192>(sa); r.dlt[2] = lds_read_b128<448>(sa);
    r.lse[3] = lds_read_b128<224>(sa); r.dlt[3] = lds_read_b128<480>(sa);
  }
}

template <int D>
__device__ __forceinline__ void pin_sub_rows(SubRows& r) {
#pragma unroll
  for (int kk = 0; kk < D / 16; ++kk) {
    pin(r.q[kk]);
    pin(r.o[kk]);
  }
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    pin(r.lse[g]);
    pin(r.dlt[g]);
  }
}

// ---------------------------------------------------------------- dK / dV

// Equal lengths: one workgroup per causal pair of key blocks (paired_tile) in the head_dim
// 64 kernel (causal B4 H32 N8192 2.13-2.23 -> 2.11-2.16 ms). The head_dim 128 kernel keeps
// one key block per workgroup: there a two-block loop spilled 97 registers around the key
// block's stream (3.86 -> 4.10 ms).
template <int D>
constexpr bool kPairedKv = D == 64;

template <typename T, int D, bool CAUSAL>
__global__ __attribute__((amdgpu_flat_work_group_size(kThreads1, kThreads1),
                          amdgpu_waves_per_eu(D == 64 ? 2 : 1, D == 64 ? 2 : 1))) void
attn_bwd_dkdv_dma_kernel(const T* __restrict__ Q, const T* __restrict__ K,
                         const T* __restrict__ V, const T* __restrict__ dO, T* __restrict__ dK,
                         T* __restrict__ dV, const float* __restrict__ lse,
                         const float* __restrict__ delta, BwdShape s) {
  using G = BwdGeo<D>;
  constexpr int BB = G::BB, KS = G::KS, DT = G::DT, RB = G::RB, TILE = G::TILE;
  constexpr int STAT = 2 * BB * 4;             // lse[64] then delta[64]
  constexpr int STB = 2 * TILE + STAT;          // stage: Q, dO, statistics
  constexpr int NDMA = 2 * G::DMA_PER_TILE + 1; // per wave per block
  __shared__ __attribute__((aligned(1024))) char lds[G::STAGES * STB];
  // dK / dV staging: the wave's 32 key rows of one of them at a time (16 KiB per workgroup;
  // two workgroups still share a CU at head_dim 64).
  __shared__ __attribute__((aligned(16))) char kvstage[G::WAVES * G::LW * RB];

  // Workgroup -> (batch, KV head, key blocks). The KV head's `group` query heads are
  // streamed one after another as one sequence of query blocks (virtual block J: head
  // J / nblk), so dK and dV sum over the group in a fixed order with a single writer.
  // Equal lengths: the key blocks paired_tile deals this workgroup (causal: blocks i and
  // NB-1-i of one KV head). Varlen: one key block per workgroup, the heavy-first schedule
  // over every sequence's key blocks (level = blocks after this one, so causal's longest
  // query ranges start first), KV heads interleaved over the XCDs.
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int kv_heads = s.heads / s.group;
  for (int it = 0; (kPairedKv<D> && CAUSAL) || it == 0; ++it) {
    int b, kvh, kblk;
    if (s.cu != nullptr) {
      if (it > 0) break;
      kvh = varlen_head(blockIdx.x, kv_heads);
      VarlenTile vt;
      if (!varlen_tile(s.cu, s.batch, s.total, s.seq, G::BW, blockIdx.x / kv_heads, vt)) break;
      b = vt.b;
      const int nb = (varlen_rows(s.cu, b, s.total, s.seq).n + G::BW - 1) / G::BW;
      kblk = nb - 1 - vt.level;
    } else if constexpr (kPairedKv<D> && CAUSAL) {
      int bkv;
      if (!paired_tile(it, s.kv_tiles / s.blocks_per_head, s.blocks_per_head, bkv, kblk))
        break;
      b = bkv / kv_heads;
      kvh = bkv % kv_heads;
    } else {
      int w = blockIdx.x;
      if (s.kv_tiles % 8 == 0) w = (w % 8) * (s.kv_tiles / 8) + w / 8;
      const int bkv = w / s.blocks_per_head;
      kblk = w % s.blocks_per_head;
      b = bkv / kv_heads;
      kvh = bkv % kv_heads;
    }
    // After the first key block: every wave has left the previous block (its last LDS
    // reads are not followed by a barrier) before this block's DMA refills the ring.
    if (it > 0) barrier_no_fence();
    const SeqSpan sp = seq_span<D>(s, b);
    const int N = sp.n;
    const int64_t sn = s.st[2], kn = s.kst[2];
    const int64_t kvbase = b * s.kst[0] + kvh * s.kst[1] + int64_t(sp.start) * kn;
    const int64_t qbase = b * s.st[0] + int64_t(kvh) * s.group * s.st[1] + int64_t(sp.start) * sn;
    // Statistics of the group's first query head; head g of the group is g heads later.
    const int64_t stat_head = s.cu != nullptr ? s.total : N;
    const int64_t stat0 = s.cu != nullptr
                              ? int64_t(kvh) * s.group * s.total + sp.start
                              : (int64_t(b) * s.heads + int64_t(kvh) * s.group) * N;

    // The lane index passes through an empty asm once per key block, so the per-lane
    // addresses derived from it are formed inside the block rather than held across the loop.
    int lane = threadIdx.x & 63;
    if constexpr (kPairedKv<D> && CAUSAL) asm volatile("" : "+v"(lane));
    const int l32 = lane & 31, hi = lane >> 5;
    const int kb0 = kblk * G::BW;
    if (kb0 >= N) break;  // varlen: past this sequence's end (uniform)
    const int wk0 = kb0 + wave * G::LW;
    const int key = wk0 + l32;  // this lane's key (column of S and dP)

    // K and V fragments of this wave's keys (B operands of S = Q K^T and dP = dO V^T).
    i32x4 kf[KS], vf[KS];
#pragma unroll
    for (int kk = 0; kk < KS; ++kk) {
      const int64_t off = kvbase + int64_t(key) * kn + kk * 16 + hi * 8;
      kf[kk] = key < N ? *reinterpret_cast<const i32x4*>(K + off) : i32x4{0, 0, 0, 0};
      vf[kk] = key < N ? *reinterpret_cast<const i32x4*>(V + off) : i32x4{0, 0, 0, 0};
    }

    // Query-side sources of the group's first head; head g adds g head strides. Each
    // head gets its own buffer extent, so rows past the sequence end read as zero.
    const T* q_head0 = Q + qbase;
    const T* do_head0 = dO + qbase;
    const float* stat_head0 = (wave < 2 ? lse : delta) + stat0;
    const uint32_t lds_base = (uint32_t)(uintptr_t)(lds_void*)lds;

    uint32_t q_src[G::DMA_PER_TILE];
#pragma unroll
    for (int x = 0; x < G::DMA_PER_TILE; ++x) q_src[x] = tile_src<D, true>(wave, x, lane, sn);
    const uint32_t st_src = uint32_t((wave & 1) * 32 + l32) * 4u;
    const uint32_t blk_bytes = uint32_t(BB * sn) * 2u;

    const int first = CAUSAL ? kb0 / BB : 0;  // first query block with a query >= kb0
    const int nblk = (N + BB - 1) / BB - first;

    // DMA of the next block in stream order (head dg of the group, relative block dj) into
    // stage ST; past the end the last block is reloaded. Blocks are fetched strictly in
    // order, so a cursor replaces a division, and the head's buffer resources are rebuilt
    // only when the cursor moves to the next head.
    int dg = 0, dj = 0;
    __amdgpu_buffer_rsrc_t rq = __builtin_amdgcn_make_buffer_rsrc((void*)q_head0, (short)0,
                                                                  sp.q_bytes, 0x00020000);
    __amdgpu_buffer_rsrc_t rdo = __builtin_amdgcn_make_buffer_rsrc((void*)do_head0, (short)0,
                                                                   sp.q_bytes, 0x00020000);
    __amdgpu_buffer_rsrc_t rst = __builtin_amdgcn_make_buffer_rsrc(
        (void*)stat_head0, (short)0, uint32_t(N) * 4u, 0x00020000);
  #define TK_BWD_DKDV_DMA(ST)                                                                 \
    {                                                                                         \
      const int qb_ = first + (dg >= s.group ? nblk - 1 : dj);                                \
      dma_tiles<D>(rq, rdo, lds + (ST) * STB, q_src, q_src, qb_ * blk_bytes, wave);           \
      dma_stats(rst, lds + (ST) * STB + 2 * TILE + wave * 128, st_src, qb_ * BB * 4, lane);   \
      if (dg < s.group && ++dj == nblk) {                                                     \
        dj = 0;                                                                               \
        if (++dg < s.group) {                                                                 \
          const int64_t h_ = int64_t(dg) * s.st[1];                                           \
          rq = __builtin_amdgcn_make_buffer_rsrc((void*)(q_head0 + h_), (short)0,             \
                                                 sp.q_bytes, 0x00020000);                     \
          rdo = __builtin_amdgcn_make_buffer_rsrc((void*)(do_head0 + h_), (short)0,           \
                                                  sp.q_bytes, 0x00020000);                    \
          rst = __builtin_amdgcn_make_buffer_rsrc((void*)(stat_head0 + dg * stat_head),       \
                                                  (short)0, uint32_t(N) * 4u, 0x00020000);    \
        }                                                                                     \
      }                                                                                       \
    }

    f32x16 acc_dv[DT], acc_dk[DT];
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc_dv[dt][r] = acc_dk[dt][r] = 0.f;

    uint32_t qa[KS], ta0[DT], ta8[DT];
#pragma unroll
    for (int kk = 0; kk < KS; ++kk) qa[kk] = frag_addr<D, true>(lane, kk);
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
      ta0[dt] = tr_addr<D>(lane, dt, 0);
      ta8[dt] = tr_addr<D>(lane, dt, 8);
    }
    const uint32_t sa = (hi * 4) * 4;  // statistics: query offset 4 hi within each group of 8
    const float sl2 = s.scale_log2;

    TK_BWD_DKDV_DMA(0)
    TK_BWD_DKDV_DMA(1)
    int stage = 0, fill = 2;
    // Causal: this wave's blocks start at the first one holding a query >= its first key.
    const int wave_first = CAUSAL ? min(nblk, (wk0 / BB) - first) : 0;
    for (int g = 0; g < s.group; ++g) {
    int j = 0;
    for (; j < wave_first; ++j) {
      wait_vmcnt<NDMA>();
      barrier_no_fence();
      TK_BWD_DKDV_DMA(fill)
      stage = stage + 1 == G::STAGES ? 0 : stage + 1;
      fill = fill + 1 == G::STAGES ? 0 : fill + 1;
    }
    for (; j < nblk; ++j) {
      wait_vmcnt<NDMA>();
      barrier_no_fence();
      TK_BWD_DKDV_DMA(fill)
      const int q0 = (first + j) * BB;
      // Lane addresses for this stage; the dO tile and the 16-row steps are immediates.
      const uint32_t sbase = lds_base + stage * STB;
      uint32_t qs_a[KS], t0[DT], t8[DT];
#pragma unroll
      for (int kk = 0; kk < KS; ++kk) qs_a[kk] = sbase + qa[kk];
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        t0[dt] = sbase + ta0[dt];
        t8[dt] = sbase + ta8[dt];
      }
      const uint32_t st_a = sbase + 2 * TILE + sa;
      const bool need_mask = CAUSAL && q0 < wk0 + G::LW - 1;

      // Two sub-blocks of 32 queries (query tile mt); each sub-block's transposed reads are
      // issued before its softmax arithmetic.
#pragma unroll
      for (int mt = 0; mt < 2; ++mt) {
        SubRows rows;
        read_sub_rows<D>(rows, mt, qs_a, st_a);
        wait_lgkm<0>();
        pin_sub_rows<D>(rows);
        // S = Q K^T and dP = dO V^T for 32 queries x this wave's 32 keys.
        f32x16 sc, dp;
        {
          const f32x16 z = {};
#pragma unroll
          for (int kk = 0; kk < KS; ++kk) {
            sc = Mma<T>::run(rows.q[kk], kf[kk], kk == 0 ? z : sc);
            dp = Mma<T>::run(rows.o[kk], vf[kk], kk == 0 ? z : dp);
          }
        }
        i32x4 to[2][DT], tq[2][DT];
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
          for (int dt = 0; dt < DT; ++dt) {
            to[i][dt] = read_tr_step<RB, TILE>(2 * mt + i, t0[dt], t8[dt]);
            tq[i][dt] = read_tr_step<RB>(2 * mt + i, t0[dt], t8[dt]);
          }
        // Causal: keys after a query get S = -inf (exp2 -> 0); only diagonal blocks.
        if (__builtin_expect(need_mask, 0)) {
          const int lim = q0 + mt * 32 + 4 * hi - key;  // key <= query  <=>  offset >= -lim
#pragma unroll
          for (int r = 0; r < 16; ++r)
            if (acc_row(r, 0) + lim < 0) sc[r] = kNegInf;
        }
        // P = exp2(S c - lse), dS = P (dP - delta); register r holds query
        // q0 + 32 mt + 8 (r / 4) + 4 hi + r % 4.
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const float l = __int_as_float(rows.lse[r >> 2][r & 3]);
          const float dl = __int_as_float(rows.dlt[r >> 2][r & 3]);
          const float pv = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[r], sl2, -l));
          sc[r] = pv;
          dp[r] = pv * (dp[r] - dl);
        }
        const i32x4 pf[2] = {acc_frag<T>(sc, 0), acc_frag<T>(sc, 1)};
        const i32x4 df[2] = {acc_frag<T>(dp, 0), acc_frag<T>(dp, 1)};
        wait_lgkm<0>();
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
          for (int dt = 0; dt < DT; ++dt) {
            pin(to[i][dt]);
            pin(tq[i][dt]);
          }
        // dV^T += dO^T P and dK^T += Q^T dS.
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
          for (int dt = 0; dt < DT; ++dt) {
            acc_dv[dt] = Mma<T>::run(to[i][dt], pf[i], acc_dv[dt]);
            acc_dk[dt] = Mma<T>::run(tq[i][dt], df[i], acc_dk[dt]);
          }
      }
      stage = stage + 1 == G::STAGES ? 0 : stage + 1;
      fill = fill + 1 == G::STAGES ? 0 : fill + 1;
    }
    }
  #undef TK_BWD_DKDV_DMA
    wait_vmcnt<0>();

    // dK = scale (dK^T)^T, dV = (dV^T)^T: register r of tile dt is feature
    // 32 dt + 8 (r / 4) + 4 hi + r % 4 of this lane's key, 8 bytes once rounded (16-byte
    // granule 4 dt + r / 4 of the row, half hi). Each of dK and dV goes through the wave's
    // staging rows (granule q of row r at q ^ row_swz(r)) and leaves as whole rows, 16 bytes
    // per lane, non-temporal full 128-byte lines (per-lane stores wrote 16 bytes to each of
    // 32 rows per instruction); the entry points accept only 16-byte aligned tensors and
    // strides that are multiples of 8 elements, so every row is 16-byte aligned.
    char* const krows = kvstage + wave * (G::LW * RB);
    auto emit = [&](T* dst, const f32x16 (&acc)[DT], float scale) {
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int g4 = 0; g4 < 4; ++g4) {
          uint2 u;
          u.x = pack2<T>(acc[dt][g4 * 4 + 0] * scale, acc[dt][g4 * 4 + 1] * scale);
          u.y = pack2<T>(acc[dt][g4 * 4 + 2] * scale, acc[dt][g4 * 4 + 3] * scale);
          *reinterpret_cast<uint2*>(krows + l32 * RB + (((4 * dt + g4) ^ G::row_swz(l32)) * 16) +
                                    hi * 8) = u;
        }
      constexpr int LPR = RB / 16, RPI = 64 / LPR;  // lanes per row, rows per instruction
#pragma unroll
      for (int p = 0; p < G::LW / RPI; ++p) {
        const int r = p * RPI + lane / LPR, q = lane % LPR;
        const i32x4 v = *reinterpret_cast<const i32x4*>(krows + r * RB + ((q ^ G::row_swz(r)) * 16));
        if (wk0 + r < N)
          __builtin_nontemporal_store(
              v, reinterpret_cast<i32x4*>(dst + kvbase + int64_t(wk0 + r) * kn + q * 8));
      }
    };
    emit(dK, acc_dk, s.scale);
    emit(dV, acc_dv, 1.0f);
  }  // key blocks
}

template <int D>
struct KvGeo {
  static constexpr int PAIRS = 4, LK = 32;       // wave pairs, keys per pair
  static constexpr int BW = PAIRS * LK;          // keys per workgroup: 128
  static constexpr int BB = 64;                  // queries per streamed block
  static constexpr int KS = D / 32;              // k-steps of S and dP
  static constexpr int FT = D / 16;              // 16-feature tiles of dK^T / dV^T
  static constexpr int FP = FT / 2;
  static constexpr int RB = D * 2;               // bytes per row
  static constexpr int OPB = BB * RB;            // bytes per operand tile
  static constexpr int STAT = 2 * BB * 4;        // lse[64] then delta[64]
  static constexpr int STB = 2 * OPB + STAT;     // stage: Q, dO, statistics
  static constexpr int STAGES = D == 128 ? 3 : 4;
  static constexpr int XB = 8 * 1024;            // exchange bytes per pair: 8 fragments
  static constexpr int LDS = STAGES * STB + PAIRS * XB;
  static constexpr int ROWS_PER_DMA = 1024 / RB;
  static constexpr int DMA_PER_OP = OPB / 1024 / 8;
  static constexpr int DMA_PER_BLOCK = 2 * DMA_PER_OP + 1;  // Q, dO, statistics
  static constexpr int SLOTS = RB / 16;
  // Read units (four LDS instructions each). Producer: KS Q-row units then KS dO-row
  // units (query tiles 0..3 of one k-step). Consumer: 2 FP transposed-dO units (32-query
  // step s = v / FP, feature tiles 2p, 2p + 1), then 2 FP transposed-Q units. DEPTH units
  // are in flight; the first PREFETCH units of an MFMA phase are issued at the end of the
  // wave's preceding phase.
  static constexpr int NA = 2 * KS, NB = 4 * FP;
  static constexpr int DEPTH_A = 3, PREFETCH_A = 2, DEPTH_B = 3;
  // Without causal masking the consumer runs units 0 .. SPLIT_B - 1 of a block beside the
  // producer's MFMAs and the rest beside the producer's elementwise phase (non-causal D128
  // 1.995 -> 1.934 ms); causal runs all of them beside the elementwise phase (3.77 vs 3.85
  // ms split), whose diagonal blocks carry the masking.
  static constexpr int SPLIT_B = 2;
  // Tiles read both as rows (ds_read_b128: 16 rows of one chunk) and transposed
  // (ds_read_b64_tr_b16: 8 rows x 32 bytes per 32-lane phase). The transposed phases need
  // bits 1..3 of the swizzle distinct over rows 0..7 and over rows 8..15; for the row reads
  // gfx950's bank mapping was measured rather than derived: with these swizzles a stream of
  // either read sustains 236-256 B/clock/CU, while the swizzle ((r & 7) << 1) | r3 (a
  // bijection on 16 rows) held the row reads to 155 B/clock/CU.
  static __device__ __forceinline__ int swz(int r) {
    return D == 128 ? (((r >> 3) & 1) | ((r & 3) << 1) | ((((r >> 2) ^ (r >> 3)) & 1) << 3))
                    : (r & 7);
  }
};

// Two transposed reads of 16 rows each, OFF and OFF + 16 rows past the lane address: a
// 32-query A operand in the query order of an operand built from two 16x16 accumulators.
template <int OFF, int RB>
__device__ __forceinline__ i32x4 read_t16(uint32_t addr) {
  const i32x2 a = lds_read_tr16<OFF>(addr);
  const i32x2 b = lds_read_tr16<OFF + 16 * RB>(addr);
  return i32x4{a[0], a[1], b[0], b[1]};
}

__device__ __forceinline__ void lds_write_b128(uint32_t addr, i32x4 v) {
  asm volatile("ds_write_b128 %0, %1" ::"v"(addr), "v"(v) : "memory");
}

// Stream of query blocks, in order: the KV head's `group` query heads one after another,
// blocks first .. first + nblk - 1 of each; past the end the last block is reloaded.
// Blocks are fetched strictly in order, so a cursor replaces a division, and the head's
// buffer resources are rebuilt only when the cursor moves to the next head.
template <typename T>
struct QStream {
  const T* q0;
  const T* o0;
  const float* st0;     // lse (waves 0-3) or delta (waves 4-7) of the group's first head
  int64_t head, st_head;  // element strides between the group's heads
  uint32_t q_bytes, st_bytes, blk_bytes;
  int group, nblk, first;
  int dg, dj, fill;  // cursor
};

// Buffer resources of the cursor's head (Q, dO, statistics).
template <typename T>
__device__ __forceinline__ void qstream_open(const QStream<T>& c, __amdgpu_buffer_rsrc_t& rq,
                                             __amdgpu_buffer_rsrc_t& rdo,
                                             __amdgpu_buffer_rsrc_t& rst) {
  rq = __builtin_amdgcn_make_buffer_rsrc((void*)(c.q0 + c.dg * c.head), (short)0, c.q_bytes,
                                         0x00020000);
  rdo = __builtin_amdgcn_make_buffer_rsrc((void*)(c.o0 + c.dg * c.head), (short)0, c.q_bytes,
                                          0x00020000);
  rst = __builtin_amdgcn_make_buffer_rsrc((void*)(c.st0 + c.dg * c.st_head), (short)0,
                                          c.st_bytes, 0x00020000);
}

// DMA of the next block of the stream into its stage: this wave's DMA_PER_OP loads of the
// Q and dO tiles and 16 statistics floats (wave w: lse rows 16 w .. (waves 0-3), delta
// rows 16 (w - 4) .. (waves 4-7)).
template <typename T, int D>
__device__ __forceinline__ void qstream_dma(QStream<T>& c, __amdgpu_buffer_rsrc_t& rq,
                                            __amdgpu_buffer_rsrc_t& rdo,
                                            __amdgpu_buffer_rsrc_t& rst, char* lds,
                                            const uint32_t* src, uint32_t st_src, int wave,
                                            int lane) {
  using G = KvGeo<D>;
  char* stage = lds + c.fill * G::STB;
  const uint32_t off = uint32_t(c.first + (c.dg >= c.group ? c.nblk - 1 : c.dj)) * c.blk_bytes;
#pragma unroll
  for (int x = 0; x < G::DMA_PER_OP; ++x) {
    const int id = wave * G::DMA_PER_OP + x;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rq, (lds_void*)(stage + id * 1024), 16, src[x], off,
                                             0, 0);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rdo, (lds_void*)(stage + G::OPB + id * 1024), 16,
                                             src[x], off, 0, 0);
  }
  const uint32_t st_off =
      uint32_t(c.first + (c.dg >= c.group ? c.nblk - 1 : c.dj)) * uint32_t(G::BB * 4);
  if (lane < 16)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rst, (lds_void*)(stage + 2 * G::OPB + wave * 64), 4,
                                             st_src, st_off, 0, 0);
  c.fill = c.fill + 1 == G::STAGES ? 0 : c.fill + 1;
  if (c.dg < c.group && ++c.dj == c.nblk) {
    c.dj = 0;
    if (++c.dg < c.group) qstream_open(c, rq, rdo, rst);
  }
}

// Producer read unit u (Q rows for u < KS, else dO rows; k-step u % KS, query tiles
// 0..3 at +16 rows each) of the stage at sb.
template <int D>
__device__ __forceinline__ void producer_unit(i32x4 (&rf)[KvGeo<D>::NA][4], uint32_t sb,
                                              const uint32_t (&qa)[KvGeo<D>::KS], int u) {
  constexpr int KS = KvGeo<D>::KS, RB = KvGeo<D>::RB, OPB = KvGeo<D>::OPB;
  const uint32_t a = sb + qa[u % KS];
  if (u < KS) {
    rf[u][0] = lds_read_b128<0>(a);
    rf[u][1] = lds_read_b128<16 * RB>(a);
    rf[u][2] = lds_read_b128<32 * RB>(a);
    rf[u][3] = lds_read_b128<48 * RB>(a);
  } else {
    rf[u][0] = lds_read_b128<OPB>(a);
    rf[u][1] = lds_read_b128<OPB + 16 * RB>(a);
    rf[u][2] = lds_read_b128<OPB + 32 * RB>(a);
    rf[u][3] = lds_read_b128<OPB + 48 * RB>(a);
  }
}

// Producer MFMA phase: S = Q K^T and dP = dO V^T for the block's 64 queries and the pair's
// 32 keys (st / dp [qt][kt] register r: query 16 qt + 4 g + r, key 16 kt + c). Its first
// PREFETCH_A units were issued by the preceding phase.
template <typename T, int D>
__device__ __forceinline__ void producer_mfma(uint32_t sb, const uint32_t (&qa)[KvGeo<D>::KS],
                                              const i32x4 (&kf)[2][KvGeo<D>::KS],
                                              const i32x4 (&vf)[2][KvGeo<D>::KS],
                                              f32x4 (&st)[4][2], f32x4 (&dp)[4][2],
                                              i32x4 (&rf)[KvGeo<D>::NA][4]) {
  using G = KvGeo<D>;
  constexpr int KS = G::KS, NU = G::NA, DEPTH = G::DEPTH_A, PRE = G::PREFETCH_A;
#pragma unroll
  for (int u = PRE; u < DEPTH && u < NU; ++u) producer_unit<D>(rf, sb, qa, u);
  sched_fence();
#pragma unroll
  for (int u = 0; u < NU; ++u) {
    const int after = (u + DEPTH < NU ? u + DEPTH : NU) - (u + 1);
    if (after >= 2)
      wait_lgkm<8>();
    else if (after == 1)
      wait_lgkm<4>();
    else
      wait_lgkm<0>();
#pragma unroll
    for (int qt = 0; qt < 4; ++qt) pin(rf[u][qt]);
    const int kk = u % KS;
    const f32x4 z = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int qt = 0; qt < 4; ++qt)
#pragma unroll
      for (int kt = 0; kt < 2; ++kt) {
        if (u < KS)
          st[qt][kt] = Mma16<T>::run(rf[u][qt], kf[kt][kk], kk == 0 ? z : st[qt][kt]);
        else
          dp[qt][kt] = Mma16<T>::run(rf[u][qt], vf[kt][kk], kk == 0 ? z : dp[qt][kt]);
      }
    if (u + DEPTH < NU) producer_unit<D>(rf, sb, qa, u + DEPTH);
    sched_fence();
  }
}

// Consumer read unit u (transposed dO for u < 2 FP, else transposed Q) of the stage at sb.
template <int D>
__device__ __forceinline__ void consumer_unit(i32x4 (&tu)[KvGeo<D>::NB][2], uint32_t sb,
                                              const uint32_t (&ta)[KvGeo<D>::FT], int u) {
  using G = KvGeo<D>;
  constexpr int FP = G::FP, RB = G::RB, OPB = G::OPB;
  const int v = u < 2 * FP ? u : u - 2 * FP;
  const int s = v / FP, p = v % FP;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const uint32_t a = sb + ta[2 * p + i];
    if (u < 2 * FP)
      tu[u][i] = s == 0 ? read_t16<OPB, RB>(a) : read_t16<OPB + 32 * RB, RB>(a);
    else
      tu[u][i] = s == 0 ? read_t16<0, RB>(a) : read_t16<32 * RB, RB>(a);
  }
}

// Consumer MFMAs of one block: dV^T += dO^T P and dK^T += Q^T dS over the block's 64
// queries (adv / adk [ft][kt] register r: feature 16 ft + 4 g + r, key 16 kt + c). The first
// DEPTH_B units were issued by the caller; after unit SPLIT - 1 (before the first, for
// SPLIT = 0) the accumulators are pinned and `mid` (the phase barrier) runs, the reads in
// flight continuing across it.
template <typename T, int D, int SPLIT, typename F>
__device__ __forceinline__ void consumer_mfma(uint32_t sb, const uint32_t (&ta)[KvGeo<D>::FT],
                                              const i32x4 (&pf)[2][2], const i32x4 (&df)[2][2],
                                              f32x4 (&adv)[KvGeo<D>::FT][2],
                                              f32x4 (&adk)[KvGeo<D>::FT][2],
                                              i32x4 (&tu)[KvGeo<D>::NB][2], F&& mid) {
  using G = KvGeo<D>;
  constexpr int FP = G::FP, FT = G::FT, NU = G::NB, DEPTH = G::DEPTH_B;
  if constexpr (SPLIT == 0) {
    mid();
    sched_fence();
  }
#pragma unroll
  for (int u = 0; u < NU; ++u) {
    const int after = (u + DEPTH < NU ? u + DEPTH : NU) - (u + 1);
    if (after >= 3)
      wait_lgkm<12>();
    else if (after == 2)
      wait_lgkm<8>();
    else if (after == 1)
      wait_lgkm<4>();
    else
      wait_lgkm<0>();
    pin(tu[u][0]);
    pin(tu[u][1]);
    const int v = u < 2 * FP ? u : u - 2 * FP;
    const int s = v / FP, p = v % FP;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int kt = 0; kt < 2; ++kt) {
        if (u < 2 * FP)
          adv[2 * p + i][kt] = Mma16<T>::run(tu[u][i], pf[s][kt], adv[2 * p + i][kt]);
        else
          adk[2 * p + i][kt] = Mma16<T>::run(tu[u][i], df[s][kt], adk[2 * p + i][kt]);
      }
    if (u + DEPTH < NU) consumer_unit<D>(tu, sb, ta, u + DEPTH);
    sched_fence();
    if (u == SPLIT - 1) {
#pragma unroll
      for (int ft = 0; ft < FT; ++ft)
#pragma unroll
        for (int kt = 0; kt < 2; ++kt) {
          pin(adv[ft][kt]);
          pin(adk[ft][kt]);
        }
      mid();
      sched_fence();
    }
  }
}

// ---------------------------------------------------------------- dK / dV

template <typename T, int D, bool CAUSAL>
__global__ __attribute__((amdgpu_flat_work_group_size(kThreads, kThreads),
                          amdgpu_waves_per_eu(2))) void
attn_bwd_dkdv_pp_kernel(const T* __restrict__ Q, const T* __restrict__ K,
                        const T* __restrict__ V, const T* __restrict__ dO, T* __restrict__ dK,
                        T* __restrict__ dV, const float* __restrict__ lse,
                        const float* __restrict__ delta, BwdShape s) {
  using G = KvGeo<D>;
  constexpr int BB = G::BB, KS = G::KS, FT = G::FT, RB = G::RB, STB = G::STB;
  constexpr int STAGES = G::STAGES, DPB = G::DMA_PER_BLOCK;
  __shared__ __attribute__((aligned(1024))) char lds[G::LDS];

  // Workgroup -> (batch, KV head, key block). The KV head's `group` query heads are
  // streamed one after another as one sequence of query blocks, so dK and dV sum over
  // the group in a fixed order with a single writer. Key block 0 (the most causal work)
  // comes first. Varlen: the heavy-first schedule over every sequence's key blocks
  // (level = blocks after this one), KV heads interleaved over the XCDs.
  const int kv_heads = s.heads / s.group;
  int b, kvh, kblk;
  if (s.cu != nullptr) {
    kvh = varlen_head(blockIdx.x, kv_heads);
    VarlenTile vt;
    if (!varlen_tile(s.cu, s.batch, s.total, s.seq, G::BW, blockIdx.x / kv_heads, vt)) return;
    b = vt.b;
    const int nb = (varlen_rows(s.cu, b, s.total, s.seq).n + G::BW - 1) / G::BW;
    kblk = nb - 1 - vt.level;
  } else {
    int w = blockIdx.x;
    if (s.kv_tiles % 8 == 0) w = (w % 8) * (s.kv_tiles / 8) + w / 8;
    const int bkv = w / s.blocks_per_head;
    kblk = w % s.blocks_per_head;
    b = bkv / kv_heads;
    kvh = bkv % kv_heads;
  }
  const SeqSpan sp = seq_span<D>(s, b);
  const int N = sp.n;
  const int64_t sn = s.st[2], kn = s.kst[2];
  const int64_t kvbase = b * s.kst[0] + kvh * s.kst[1] + int64_t(sp.start) * kn;
  const int64_t qbase = b * s.st[0] + int64_t(kvh) * s.group * s.st[1] + int64_t(sp.start) * sn;
  // Statistics of the group's first query head; head g of the group is g heads later.
  const int64_t stat_head = s.cu != nullptr ? s.total : N;
  const int64_t stat0 = s.cu != nullptr
                            ? int64_t(kvh) * s.group * s.total + sp.start
                            : (int64_t(b) * s.heads + int64_t(kvh) * s.group) * N;

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int c = lane & 15, g = lane >> 4;
  const int kb0 = kblk * G::BW;
  if (kb0 >= N) return;  // varlen: past this sequence's end (uniform)
  // Wave w < 4 produces P and dS for keys pk0 .. pk0 + 31; wave w + 4 consumes them.
  const bool producer = wave < G::PAIRS;
  const int pair = producer ? wave : wave - G::PAIRS;
  const int pk0 = kb0 + pair * G::LK;

  const int first = CAUSAL ? kb0 / BB : 0;  // first query block with a query >= kb0
  const int nblk = (N + BB - 1) / BB - first;
  const int nv = s.group * nblk;            // blocks in the stream

  QStream<T> qs;
  qs.q0 = Q + qbase;
  qs.o0 = dO + qbase;
  qs.st0 = (wave < 4 ? lse : delta) + stat0;
  qs.head = s.st[1];
  qs.st_head = stat_head;
  qs.q_bytes = sp.q_bytes;
  qs.st_bytes = uint32_t(N) * 4u;
  qs.blk_bytes = uint32_t(BB * sn) * 2u;
  qs.group = s.group;
  qs.nblk = nblk;
  qs.first = first;
  qs.dg = qs.dj = qs.fill = 0;
  __amdgpu_buffer_rsrc_t rq, rdo, rst;
  qstream_open(qs, rq, rdo, rst);
  uint32_t src[G::DMA_PER_OP];
#pragma unroll
  for (int x = 0; x < G::DMA_PER_OP; ++x) {
    const int id = wave * G::DMA_PER_OP + x;
    const int row = id * G::ROWS_PER_DMA + lane / G::SLOTS;
    const int slot = lane % G::SLOTS;
    src[x] = uint32_t(row * sn + (slot ^ G::swz(row)) * 8) * 2u;
  }
  const uint32_t st_src = uint32_t((wave & 3) * 16 + lane) * 4u;
#pragma unroll
  for (int i = 0; i < STAGES - 1; ++i)
    qstream_dma<T, D>(qs, rq, rdo, rst, lds, src, st_src, wave, lane);

  const uint32_t lds_base = (uint32_t)(uintptr_t)(lds_void*)lds;
  const uint32_t xb = lds_base + STAGES * STB + pair * G::XB + lane * 16;
  const float sl2 = s.scale_log2;
  int t = 0;
  // Block v is DMA'd at the start of phase 2v - 2 (STAGES - 2) blocks ahead and waited
  // for at the end of phase 2v - 2, so the producer can prefetch its first units at the
  // end of phase 2v - 1.
  auto end_phase = [&]() {
    if (!(t & 1)) wait_vmcnt<(STAGES - 3) * DPB>();
    barrier_no_fence();
    ++t;
    if (!(t & 1)) qstream_dma<T, D>(qs, rq, rdo, rst, lds, src, st_src, wave, lane);
  };
  // Causal: a block whose last query precedes the pair's first key contributes nothing.
  auto active = [&](int j) { return !CAUSAL || (first + j) * BB + BB - 1 >= pk0; };

  wait_vmcnt<(STAGES - 2) * DPB>();
  barrier_no_fence();

  if (producer) {
    // K and V fragments (B operands): key tile kt holds key pk0 + 16 kt + c, k-step kk
    // features 32 kk + 8 g .. +7.
    i32x4 kf[2][KS], vf[2][KS];
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) {
      const int key = pk0 + 16 * kt + c;
#pragma unroll
      for (int kk = 0; kk < KS; ++kk) {
        const int64_t off = kvbase + int64_t(key) * kn + kk * 32 + g * 8;
        kf[kt][kk] = key < N ? *reinterpret_cast<const i32x4*>(K + off) : i32x4{0, 0, 0, 0};
        vf[kt][kk] = key < N ? *reinterpret_cast<const i32x4*>(V + off) : i32x4{0, 0, 0, 0};
      }
    }
    // Row reads: row c of query tile qt (+16 qt rows, an immediate), chunk 4 kk + g.
    uint32_t qa[KS];
#pragma unroll
    for (int kk = 0; kk < KS; ++kk) qa[kk] = c * RB + (((4 * kk + g) ^ G::swz(c)) * 16);
    const uint32_t sa = 2 * G::OPB + 16 * g;  // statistics of queries 16 qt + 4 g .. +3
    i32x4 rf[G::NA][4];
    if (active(0)) {
#pragma unroll
      for (int u = 0; u < G::PREFETCH_A; ++u) producer_unit<D>(rf, lds_base, qa, u);
    }
    int stage = 0, j = 0;
    for (int v = 0; v < nv; ++v) {
      const bool act = active(j);
      const int jn = j + 1 == nblk ? 0 : j + 1;
      const int sn = stage + 1 == STAGES ? 0 : stage + 1;
      const uint32_t sb = lds_base + stage * STB;
      f32x4 st[4][2], dp[4][2];
      i32x4 lq[4], dq[4];
      if (act) {
        producer_mfma<T, D>(sb, qa, kf, vf, st, dp, rf);
        // lse / delta of the lane's 16 queries, waited for in the next phase.
        lq[0] = lds_read_b128<0>(sb + sa);
        lq[1] = lds_read_b128<64>(sb + sa);
        lq[2] = lds_read_b128<128>(sb + sa);
        lq[3] = lds_read_b128<192>(sb + sa);
        dq[0] = lds_read_b128<256>(sb + sa);
        dq[1] = lds_read_b128<320>(sb + sa);
        dq[2] = lds_read_b128<384>(sb + sa);
        dq[3] = lds_read_b128<448>(sb + sa);
        // Results pinned before the barrier (it orders memory only; the compiler would
        // sink register work into the next phase).
#pragma unroll
        for (int qt = 0; qt < 4; ++qt)
#pragma unroll
          for (int kt = 0; kt < 2; ++kt) {
            pin(st[qt][kt]);
            pin(dp[qt][kt]);
          }
      }
      end_phase();
      if (act) {
        wait_lgkm<0>();
#pragma unroll
        for (int qt = 0; qt < 4; ++qt) {
          pin(lq[qt]);
          pin(dq[qt]);
        }
        // P = exp2(S c - lse), dS = P (dP - delta); keys after the query are masked
        // (causal diagonal blocks only).
        const int q0 = (first + j) * BB;
        if (CAUSAL && q0 < pk0 + G::LK - 1) {
#pragma unroll
          for (int qt = 0; qt < 4; ++qt)
#pragma unroll
            for (int kt = 0; kt < 2; ++kt) {
              const int lim = q0 + 16 * qt + 4 * g - (pk0 + 16 * kt + c);
#pragma unroll
              for (int r = 0; r < 4; ++r)
                if (r + lim < 0) st[qt][kt][r] = kNegInf;
            }
        }
#pragma unroll
        for (int qt = 0; qt < 4; ++qt)
#pragma unroll
          for (int kt = 0; kt < 2; ++kt)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              const float l = __int_as_float(lq[qt][r]), dl = __int_as_float(dq[qt][r]);
              const float p = __builtin_amdgcn_exp2f(__builtin_fmaf(st[qt][kt][r], sl2, -l));
              st[qt][kt][r] = p;
              dp[qt][kt][r] = p * (dp[qt][kt][r] - dl);
            }
        // Fragments of the consumer's B operands: 32-query step s (query tiles 2s, 2s + 1),
        // key tile kt; P at 1 KiB * (2 s + kt), dS 4 KiB further.
#pragma unroll
        for (int s2 = 0; s2 < 2; ++s2)
#pragma unroll
          for (int kt = 0; kt < 2; ++kt) {
            lds_write_b128(xb + (2 * s2 + kt) * 1024,
                           acc_frag2<T>(st[2 * s2][kt], st[2 * s2 + 1][kt]));
            lds_write_b128(xb + 4096 + (2 * s2 + kt) * 1024,
                           acc_frag2<T>(dp[2 * s2][kt], dp[2 * s2 + 1][kt]));
          }
        wait_lgkm<0>();
      }
      // First units of the next block's MFMA phase (its tile landed by the end of the
      // previous phase).
      if (v + 1 < nv && active(jn)) {
#pragma unroll
        for (int u = 0; u < G::PREFETCH_A; ++u)
          producer_unit<D>(rf, lds_base + sn * STB, qa, u);
      }
      end_phase();
      stage = sn;
      j = jn;
    }
    end_phase();
  } else {
    // Transposed reads: row 4 g + c / 4 (+16 for k-index 4..7, +32 per 32-query step),
    // features 16 ft + 4 (c % 4) .. +3: chunk 2 ft + (c % 4) / 2, half (c % 4) % 2.
    uint32_t ta[FT];
    {
      const int row = 4 * g + (c >> 2), q = c & 3;
#pragma unroll
      for (int ft = 0; ft < FT; ++ft)
        ta[ft] = row * RB + (((2 * ft + (q >> 1)) ^ G::swz(row)) * 16) + (q & 1) * 8;
    }
    f32x4 adv[FT][2], adk[FT][2];
#pragma unroll
    for (int ft = 0; ft < FT; ++ft)
#pragma unroll
      for (int kt = 0; kt < 2; ++kt) adv[ft][kt] = adk[ft][kt] = f32x4{0.f, 0.f, 0.f, 0.f};
    i32x4 tu[G::NB][2];
    end_phase();
    end_phase();
    // Causal: the pair's blocks of each head start at the first one holding a query >= its
    // first key; the blocks before it only keep the phase count.
    const int jact = CAUSAL ? min(nblk, max(0, pk0 / BB - first)) : 0;
    int stage = 0, v = 0;
    for (int dg = 0; dg < s.group; ++dg) {
      for (int j = 0; j < jact; ++j, ++v) {
        end_phase();
        if (v + 1 < nv) end_phase();
        stage = stage + 1 == STAGES ? 0 : stage + 1;
      }
      for (int j = jact; j < nblk; ++j, ++v) {
        const uint32_t sb = lds_base + stage * STB;
        // The producer's fragments of block v, then the first transposed units; the
        // exchange reads have completed once only those units are outstanding.
        i32x4 pf[2][2], df[2][2];
#pragma unroll
        for (int s2 = 0; s2 < 2; ++s2)
#pragma unroll
          for (int kt = 0; kt < 2; ++kt) {
            pf[s2][kt] = lds_read_b128<0>(xb + (2 * s2 + kt) * 1024);
            df[s2][kt] = lds_read_b128<4096>(xb + (2 * s2 + kt) * 1024);
          }
#pragma unroll
        for (int u = 0; u < G::DEPTH_B; ++u) consumer_unit<D>(tu, sb, ta, u);
        wait_lgkm<4 * G::DEPTH_B>();
#pragma unroll
        for (int s2 = 0; s2 < 2; ++s2)
#pragma unroll
          for (int kt = 0; kt < 2; ++kt) {
            pin(pf[s2][kt]);
            pin(df[s2][kt]);
          }
        consumer_mfma<T, D, CAUSAL ? 0 : G::SPLIT_B>(sb, ta, pf, df, adv, adk, tu, end_phase);
#pragma unroll
        for (int ft = 0; ft < FT; ++ft)
#pragma unroll
          for (int kt = 0; kt < 2; ++kt) {
            pin(adv[ft][kt]);
            pin(adk[ft][kt]);
          }
        if (v + 1 < nv) end_phase();
        stage = stage + 1 == STAGES ? 0 : stage + 1;
      }
    }
    wait_vmcnt<0>();
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    // dK = scale (dK^T)^T, dV = (dV^T)^T: register r of adk / adv [ft][kt] is feature
    // 16 ft + 4 g + r of key pk0 + 16 kt + c, 8 bytes once rounded. Each key tile goes
    // through the pair's exchange buffer (the producer has written its last fragments and
    // this wave has read them): dK rows then dV rows, 16-byte granule q of row r at
    // q ^ (r & 15), read back as whole rows and stored 16 bytes per lane as non-temporal full
    // 128-byte lines; the entry points accept only 16-byte aligned tensors and strides that
    // are multiples of 8 elements, so every row is 16-byte aligned. Lane indices are formed
    // afresh here.
    int el = threadIdx.x & 63;
    asm volatile("" : "+v"(el));
    const int ec = el & 15, eg = el >> 4;
    T* const dKh = dK + kvbase;
    T* const dVh = dV + kvbase;
    char* const xrows = lds + STAGES * STB + pair * G::XB;
    static_assert(2 * 16 * RB <= G::XB, "two 16-key tiles of rows per exchange buffer");
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) {
#pragma unroll
      for (int ft = 0; ft < FT; ++ft) {
        const int at = ec * RB + (((2 * ft + (eg >> 1)) ^ ec) * 16) + (eg & 1) * 8;
        uint2 u;
        u.x = pack2<T>(adk[ft][kt][0] * s.scale, adk[ft][kt][1] * s.scale);
        u.y = pack2<T>(adk[ft][kt][2] * s.scale, adk[ft][kt][3] * s.scale);
        *reinterpret_cast<uint2*>(xrows + at) = u;
        u.x = pack2<T>(adv[ft][kt][0], adv[ft][kt][1]);
        u.y = pack2<T>(adv[ft][kt][2], adv[ft][kt][3]);
        *reinterpret_cast<uint2*>(xrows + 16 * RB + at) = u;
      }
      constexpr int LPR = RB / 16, RPI = 64 / LPR;  // lanes per row, rows per instruction
#pragma unroll
      for (int p = 0; p < 16 / RPI; ++p) {
        const int r = p * RPI + el / LPR, q = el % LPR;
        const int from = r * RB + ((q ^ r) * 16);
        const i32x4 vk = *reinterpret_cast<const i32x4*>(xrows + from);
        const i32x4 vv = *reinterpret_cast<const i32x4*>(xrows + 16 * RB + from);
        const int row_key = pk0 + 16 * kt + r;
        if (row_key < N) {
          const int64_t to = int64_t(row_key) * kn + q * 8;
          __builtin_nontemporal_store(vk, reinterpret_cast<i32x4*>(dKh + to));
          __builtin_nontemporal_store(vv, reinterpret_cast<i32x4*>(dVh + to));
        }
      }
    }
    return;
  }
  wait_vmcnt<0>();
}

BwdShape make_shape(int64_t batch, int64_t heads, int64_t kv_heads, int64_t seq,
                    int64_t head_dim, const int64_t* q_strides, const int64_t* kv_strides,
                    float sm_scale, const int32_t* cu_seqlens, int64_t total) {
  BwdShape s{};
  s.cu = cu_seqlens;
  s.total = (int)total;
  s.heads = (int)heads;
  s.seq = (int)seq;
  s.group = (int)(heads / kv_heads);
  for (int i = 0; i < 3; ++i) {
    s.st[i] = q_strides[i];
    s.kst[i] = kv_strides[i];
  }
  s.scale = sm_scale;
  s.scale_log2 = sm_scale * 1.4426950408889634f;
  s.batch = (int)batch;
  s.blocks_per_head = (int)tk::cdiv(seq, 128);
  const int64_t per_head = cu_seqlens != nullptr ? varlen_tiles(batch, total, seq, 128)
                                                 : s.blocks_per_head * batch;
  s.tiles = (int)(per_head * heads);
  s.kv_tiles = (int)(per_head * kv_heads);
  s.head_bytes = (uint32_t)(((seq - 1) * q_strides[2] + head_dim) * 2);
  s.kv_head_bytes = (uint32_t)(((seq - 1) * kv_strides[2] + head_dim) * 2);
  return s;
}

// head_dim 128: the producer/consumer kernel; head_dim 64: the one-wave-per-SIMD kernel,
// whose two workgroups per CU overlap one workgroup's exponentials with the other's
// MFMAs (at head_dim 64 a producer's elementwise phase, the same work as at 128, outlasts
// the consumer's halved MFMA phase).
// Causal head_dim 64 (kPairedKv), equal lengths: paired_items workgroups; otherwise one
// workgroup per key block.
template <typename T>
void launch_dkdv(int64_t head_dim, bool causal, hipStream_t stream, const void* q,
                 const void* k, const void* v, const void* dout, void* dk, void* dv,
                 const float* lse, const float* delta, const BwdShape& s) {
  const bool paired = s.cu == nullptr && causal && head_dim == 64 && kPairedKv<64>;
  const int64_t n = paired ? paired_items(s.kv_tiles / s.blocks_per_head, s.blocks_per_head)
                           : int64_t(s.kv_tiles);
  const dim3 grid(static_cast<unsigned>(n));
  if (head_dim == 64) {
    if (causal)
      hipLaunchKernelGGL((attn_bwd_dkdv_dma_kernel<T, 64, true>), grid, dim3(kThreads1), 0,
                         stream, (const T*)q, (const T*)k, (const T*)v, (const T*)dout, (T*)dk,
                         (T*)dv, lse, delta, s);
    else
      hipLaunchKernelGGL((attn_bwd_dkdv_dma_kernel<T, 64, false>), grid, dim3(kThreads1), 0,
                         stream, (const T*)q, (const T*)k, (const T*)v, (const T*)dout, (T*)dk,
                         (T*)dv, lse, delta, s);
  } else {
    if (causal)
      hipLaunchKernelGGL((attn_bwd_dkdv_pp_kernel<T, 128, true>), grid, dim3(kThreads), 0,
                         stream, (const T*)q, (const T*)k, (const T*)v, (const T*)dout, (T*)dk,
                         (T*)dv, lse, delta, s);
    else
      hipLaunchKernelGGL((attn_bwd_dkdv_pp_kernel<T, 128, false>), grid, dim3(kThreads), 0,
                         stream, (const T*)q, (const T*)k, (const T*)v, (const T*)dout, (T*)dk,
                         (T*)dv, lse, delta, s);
  }
}

}  // namespace

namespace tk {

bool attn_bwd_dma_applies(int64_t seq, int64_t head_dim, const int64_t* q_strides,
                          const int64_t* kv_strides) {
  // 32-bit buffer offsets: one head's rows must span less than 2 GiB.
  const int64_t lim = int64_t(1) << 31;
  return ((seq - 1) * q_strides[2] + head_dim) * 2 < lim &&
         ((seq - 1) * kv_strides[2] + head_dim) * 2 < lim;
}

void attn_bwd_dkdv_dma_launch(int dtype, const void* q, const void* k, const void* v,
                              const void* dout, void* dk, void* dv, const float* lse,
                              const float* delta, int64_t batch, int64_t heads,
                              int64_t kv_heads, int64_t seq, int64_t head_dim,
                              const int64_t* q_strides, const int64_t* kv_strides,
                              float sm_scale, bool causal, hipStream_t stream,
                              const int32_t* cu_seqlens, int64_t total) {
  const BwdShape s = make_shape(batch, heads, kv_heads, seq, head_dim, q_strides, kv_strides,
                                sm_scale, cu_seqlens, total);
  if (dtype == TK_DTYPE_F16)
    launch_dkdv<_Float16>(head_dim, causal, stream, q, k, v, dout, dk, dv, lse, delta, s);
  else
    launch_dkdv<__bf16>(head_dim, causal, stream, q, k, v, dout, dk, dv, lse, delta, s);
}

}  // namespace tk
