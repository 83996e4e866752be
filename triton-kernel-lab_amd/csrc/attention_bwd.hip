// Flash attention recompute backward for head_dim 64/128 (f16/bf16) on CDNA4 MFMA: the
// dK/dV pass behind tk_attn_bwd_dkdv (src/tklab/kernels/flash_attention.py:383-491:
// P = exp2(S * scale * log2(e) - lse), dS = P (dP - delta), dV = P^T dO, dK = scale dS^T Q;
// each output is written by exactly one workgroup, so the pass is deterministic). The dQ
// pass is attention_bwd_dq.hip.
//
// dK/dV pass: a workgroup owns 128 keys (4 wave64s x 32, one wave per SIMD) and walks the
// query blocks of 64. With head_dim 64 the kernel is held to 256 registers (it fits
// without spills), so two workgroups share a CU and each SIMD has a second wave to cover
// the first one's LDS and MFMA latencies (+13-16% over one wave per SIMD); head_dim 128
// needs ~400 registers and ~98 KiB of LDS, one workgroup per CU. K and V fragments stay in
// registers. Per query block each wave computes S = Q K^T and dP = dO V^T (accumulator
// lane = one key, so P and dS feed the next MFMAs as B operands straight from registers),
// then dV^T += dO^T P and dK^T += Q^T dS with dO^T / Q^T read transposed
// (ds_read_b64_tr_b16) from the same row-major tiles that S and dP read with ds_read_b128.
//
// Tiles reach LDS by buffer->LDS DMA into a 3-stage ring, two blocks ahead, one barrier
// per block. Tiles read both ways (Q, dO) store the 16-byte chunk c of row r at slot
// c ^ dual_swz(r), which keeps both the 16-row ds_read_b128 phases and the 4-row x
// 64-byte transposed phases on 64 distinct banks.
#include "attention.hpp"
#include "attention_dma.hpp"

namespace {

using namespace tk_attn;

constexpr int kThreads = 256;  // 4 waves, one per SIMD of the CU

template <int N>
__device__ __forceinline__ void wait_lgkm_n() {
  asm volatile("s_waitcnt lgkmcnt(%0)" ::"i"(N) : "memory");
}

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

template <typename T, int D, bool CAUSAL>
__global__ __attribute__((amdgpu_flat_work_group_size(kThreads, kThreads),
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

  // Workgroup -> (batch, KV head, key block). The KV head's `group` query heads are
  // streamed one after another as one sequence of query blocks (virtual block J: head
  // J / nblk), so dK and dV sum over the group in a fixed order with a single writer.
  // Varlen: the heavy-first schedule over every sequence's key blocks (level = blocks
  // after this one, so causal's longest query ranges start first), KV heads interleaved
  // over the XCDs.
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
  const int l32 = lane & 31, hi = lane >> 5;
  const int kb0 = kblk * G::BW;
  if (kb0 >= N) return;  // varlen: past this sequence's end (uniform)
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
      wait_lgkm_n<0>();
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
      wait_lgkm_n<0>();
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
  // 32 dt + 8 (r / 4) + 4 hi + r % 4 of this lane's key.
  if (key < N) {
    T* dkr = dK + kvbase + int64_t(key) * kn;
    T* dvr = dV + kvbase + int64_t(key) * kn;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int g4 = 0; g4 < 4; ++g4) {
        const int d = dt * 32 + g4 * 8 + hi * 4;
        uint2 u;
        u.x = pack2<T>(acc_dk[dt][g4 * 4 + 0] * s.scale, acc_dk[dt][g4 * 4 + 1] * s.scale);
        u.y = pack2<T>(acc_dk[dt][g4 * 4 + 2] * s.scale, acc_dk[dt][g4 * 4 + 3] * s.scale);
        *reinterpret_cast<uint2*>(dkr + d) = u;
        u.x = pack2<T>(acc_dv[dt][g4 * 4 + 0], acc_dv[dt][g4 * 4 + 1]);
        u.y = pack2<T>(acc_dv[dt][g4 * 4 + 2], acc_dv[dt][g4 * 4 + 3]);
        *reinterpret_cast<uint2*>(dvr + d) = u;
      }
  }
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

#define TK_BWD_LAUNCH(TILES, KERNEL, ...)                                                   \
  do {                                                                                      \
    const dim3 grid(static_cast<unsigned>(TILES));                                         \
    if (dtype == TK_DTYPE_F16) {                                                            \
      using T = _Float16;                                                                   \
      if (head_dim == 64) {                                                                 \
        if (causal) hipLaunchKernelGGL((KERNEL<T, 64, true>), grid, dim3(kThreads), 0, stream, __VA_ARGS__); \
        else hipLaunchKernelGGL((KERNEL<T, 64, false>), grid, dim3(kThreads), 0, stream, __VA_ARGS__);      \
      } else {                                                                              \
        if (causal) hipLaunchKernelGGL((KERNEL<T, 128, true>), grid, dim3(kThreads), 0, stream, __VA_ARGS__); \
        else hipLaunchKernelGGL((KERNEL<T, 128, false>), grid, dim3(kThreads), 0, stream, __VA_ARGS__);      \
      }                                                                                     \
    } else {                                                                                \
      using T = __bf16;                                                                     \
      if (head_dim == 64) {                                                                 \
        if (causal) hipLaunchKernelGGL((KERNEL<T, 64, true>), grid, dim3(kThreads), 0, stream, __VA_ARGS__); \
        else hipLaunchKernelGGL((KERNEL<T, 64, false>), grid, dim3(kThreads), 0, stream, __VA_ARGS__);      \
      } else {                                                                              \
        if (causal) hipLaunchKernelGGL((KERNEL<T, 128, true>), grid, dim3(kThreads), 0, stream, __VA_ARGS__); \
        else hipLaunchKernelGGL((KERNEL<T, 128, false>), grid, dim3(kThreads), 0, stream, __VA_ARGS__);      \
      }                                                                                     \
    }                                                                                       \
  } while (0)

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
  TK_BWD_LAUNCH(s.kv_tiles, attn_bwd_dkdv_dma_kernel, (const T*)q, (const T*)k, (const T*)v,
                (const T*)dout, (T*)dk, (T*)dv, lse, delta, s);
}

}  // namespace tk
