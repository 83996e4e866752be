// Flash attention backward, dQ pass, for head_dim 64/128 (f16/bf16) on CDNA4 MFMA: the
// path behind tk_attn_bwd_dq (src/tklab/kernels/flash_attention.py:493-533 is the Triton
// kernel it replaces: P = exp2(S * scale * log2(e) - lse), dS = P (dP - delta),
// dQ = scale dS K; every dQ row is written by exactly one workgroup, so the pass is
// deterministic).
//
// Workgroup: 256 queries, 8 wave64s of 32 queries (two 16-query tiles), two waves per SIMD;
// key/value blocks of 64 (four 16-key tiles); all products are v_mfma_f32_16x16x32.
// Per wave and key block j:
//   S^T  = K Q^T     K rows as A operands (ds_read_b128), Q fragments in registers;
//   dP^T = V dO^T    V rows as A operands, dO fragments in registers (head_dim 64: the
//                    accumulators seeded with -delta, so they hold dP^T - delta);
//   P = exp2(S^T c - lse), dS^T = P (dP^T - delta): lane l holds query 16 qt + l % 16, so
//                    lse and delta are one value per lane and query tile;
//   dQ^T += K^T dS^T K^T fragments read transposed (ds_read_b64_tr_b16) from the same K
//                    tile, in the key order of the dS^T operand (key tiles 2s, 2s + 1).
// The K tile is read both ways, so its 16-byte chunk c of row r sits at c ^ kswz(r), a
// permutation that keeps 16 consecutive rows of one chunk (row reads) and 8 consecutive
// rows of one 32-byte granule (transposed reads) on distinct banks.
//
// Ping-pong, as in the forward: barrier-separated phases alternate an MFMA phase M(j)
// (dQ^T += K_{j-1}^T dS_{j-1}^T, then S^T_j and dP^T_j) and an elementwise phase V(j)
// (P, dS); the two waves of each SIMD run opposite phases. K/V blocks reach LDS by
// buffer->LDS DMA into a 4-stage ring (block j is read in phases 2j .. 2j+3); each wave
// issues its share of block m + 2 spread over the read units of its MFMA phase of block m,
// not as a burst after a barrier (causal D128 2.65 -> 2.60 ms).
#include "attention.hpp"
#include "attention_dma.hpp"

namespace {

using namespace tk_attn;

constexpr int kThreads = 512;

struct DqShape {
  int heads, seq;
  int group;  // query heads per KV head
  // Variable-length batches (null for equal lengths): sequence b is rows cu[b] ..
  // cu[b+1] of packed [total][head][dim] tensors (batch strides 0); lse / delta are
  // [head][total].
  const int32_t* cu;
  int total, batch;
  int64_t q[3], kv[3];  // batch, head, sequence strides of q / dO / dQ and of k / v
  float scale, scale_log2;
  int q_blocks, tiles;
  uint32_t kv_bytes;  // extent of one KV head's rows
};

template <int D>
struct DqGeo {
  static constexpr int BM = 256, BN = 64, WAVES = 8, QW = 32;
  static constexpr int KS = D / 32;             // k-steps of S^T / dP^T
  // dP^T accumulators seeded with -delta, one VALU subtraction per score fewer in the
  // elementwise phase: head_dim 64 (VALU-bound, 180 registers); at head_dim 128 the kernel
  // holds 256 registers and the seed's earlier-live accumulators spill.
  static constexpr bool SEED = D == 64;
  static constexpr int FT = D / 16;             // 16-feature tiles of dQ^T
  static constexpr int FP = FT / 2;             // feature-tile pairs per 32-key step
  static constexpr int RB = D * 2;              // bytes per K/V row
  static constexpr int OPB = BN * RB;           // bytes per operand per stage
  static constexpr int STB = 2 * OPB;           // stage: K tile then V tile
  static constexpr int STAGES = 4;
  static constexpr int ROWS_PER_DMA = 1024 / RB;
  static constexpr int DMA_PER_OP = OPB / 1024 / WAVES;
  static constexpr int DMA_PER_BLOCK = 2 * DMA_PER_OP;
  static constexpr int SLOTS = RB / 16;
  // dQ staging: 16-byte granule q of staged row r at q ^ oswz(r), so an 8-byte write phase
  // (16 rows x 2 lane groups) and a 16-byte read phase fall on distinct banks.
  static __device__ __forceinline__ int oswz(int r) { return D == 128 ? (r & 15) : ((r >> 1) & 7); }
  // Read units of the MFMA phase (four LDS instructions each): NT transposed-K units
  // (32-key step s = u / FP, feature tiles 2p, 2p + 1), then KS K-row units, then KS V-row
  // units. DEPTH units are in flight (head_dim 128 holds two to stay within 256
  // registers); PREFETCH transposed units are issued at the end of the elementwise phase.
  static constexpr int NT = 2 * FP;
  static constexpr int DEPTH = D == 128 ? 2 : 3, PREFETCH = 2;
  // Tiles read both as rows (ds_read_b128: 16 rows of one chunk) and transposed
  // (ds_read_b64_tr_b16: 8 rows x 32 bytes per 32-lane phase). The transposed phases need
  // bits 1..3 of the swizzle distinct over rows 0..7 and over rows 8..15; for the row reads
  // gfx950's bank mapping was measured rather than derived: with these swizzles a stream of
  // either read sustains 236-256 B/clock/CU, while the swizzle ((r & 7) << 1) | r3 (a
  // bijection on 16 rows) held the row reads to 155 B/clock/CU.
  static __device__ __forceinline__ int kswz(int r) {
    return D == 128 ? (((r >> 3) & 1) | ((r & 3) << 1) | ((((r >> 2) ^ (r >> 3)) & 1) << 3))
                    : (r & 7);
  }
  // V (rows only): 16 consecutive rows of one chunk on distinct banks.
  static __device__ __forceinline__ int vswz(int r) { return D == 128 ? (r & 15) : ((r >> 1) & 7); }
};

template <int D>
__device__ __forceinline__ void dq_dma_block(__amdgpu_buffer_rsrc_t rk, __amdgpu_buffer_rsrc_t rv,
                                             char* lds, const uint32_t* k_src,
                                             const uint32_t* v_src, int blk, int last,
                                             uint32_t blk_bytes, int wave) {
  using G = DqGeo<D>;
  char* stage = lds + (blk % G::STAGES) * G::STB;
  blk = min(blk, last);
#pragma unroll
  for (int x = 0; x < G::DMA_PER_OP; ++x) {
    const int id = wave * G::DMA_PER_OP + x;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rk, (lds_void*)(stage + id * 1024), 16, k_src[x],
                                             blk * blk_bytes, 0, 0);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rv, (lds_void*)(stage + G::OPB + id * 1024), 16,
                                             v_src[x], blk * blk_bytes, 0, 0);
  }
}

// DMA instruction i (0 .. DMA_PER_BLOCK - 1) of this wave's share of block `blk`: K chunks
// first, then V.
template <int D>
__device__ __forceinline__ void dq_dma_one(__amdgpu_buffer_rsrc_t rk, __amdgpu_buffer_rsrc_t rv,
                                           char* lds, const uint32_t* k_src,
                                           const uint32_t* v_src, int blk, int last,
                                           uint32_t blk_bytes, int wave, int i) {
  using G = DqGeo<D>;
  char* stage = lds + (blk % G::STAGES) * G::STB;
  blk = min(blk, last);
  const int x = i % G::DMA_PER_OP;
  const int id = wave * G::DMA_PER_OP + x;
  if (i < G::DMA_PER_OP)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rk, (lds_void*)(stage + id * 1024), 16, k_src[x],
                                             blk * blk_bytes, 0, 0);
  else
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rv, (lds_void*)(stage + G::OPB + id * 1024), 16,
                                             v_src[x], blk * blk_bytes, 0, 0);
}

// Transposed-K unit u of the K tile at kb into tu[u].
template <int D>
__device__ __forceinline__ void read_t_unit(i32x4 (&tu)[DqGeo<D>::NT][2], uint32_t kb,
                                            const uint32_t (&ta)[DqGeo<D>::FT], int u) {
  constexpr int FP = DqGeo<D>::FP, RB = DqGeo<D>::RB;
  const int s = u / FP, p = u % FP;
#pragma unroll
  for (int i = 0; i < 2; ++i)
    tu[u][i] = s == 0 ? read_v16<0, RB>(kb + ta[2 * p + i]) : read_v16<32, RB>(kb + ta[2 * p + i]);
}

// The MFMA phase of one wave: dQ^T += K_{j-1}^T dS^T from the previous elementwise phase
// (DO_DQ; its first PREFETCH units were issued by that phase), then S^T(j) = K_j Q^T and
// dP^T(j) = V_j dO^T (DO_S), with DqGeo::SEED starting from -delta of the lane's query
// (nd), so the elementwise phase forms dS = P (dP - delta) with one multiply. kb / tb:
// LDS addresses of block j's stage and block j-1's.
template <typename T, int D, bool DO_S, bool DO_DQ, typename Hook>
__device__ __forceinline__ void dq_mfma_phase(Hook&& hook, uint32_t kb, uint32_t tb,
                                              const uint32_t (&ka)[DqGeo<D>::KS],
                                              const uint32_t (&va)[DqGeo<D>::KS],
                                              const uint32_t (&ta)[DqGeo<D>::FT],
                                              const i32x4 (&qf)[2][DqGeo<D>::KS],
                                              const i32x4 (&of)[2][DqGeo<D>::KS],
                                              f32x4 (&st)[2][4], f32x4 (&dp)[2][4],
                                              const float (&nd)[2],
                                              const i32x4 (&df)[2][2],
                                              f32x4 (&acc)[DqGeo<D>::FT][2],
                                              i32x4 (&tu)[DqGeo<D>::NT][2]) {
  using G = DqGeo<D>;
  constexpr int KS = G::KS, RB = G::RB, FP = G::FP, OPB = G::OPB;
  constexpr int NT = DO_DQ ? G::NT : 0, NU = NT + (DO_S ? 2 * KS : 0);
  constexpr int DEPTH = G::DEPTH, PRE = DO_DQ ? G::PREFETCH : 0;
  i32x4 rf[2 * KS][4];  // K-row units then V-row units
  auto issue = [&](int u) {
    if (u < NT) {
      read_t_unit<D>(tu, tb, ta, u);
    } else {
      const int r = u - NT;  // r < KS: K rows, k-step r; else V rows, k-step r - KS
      const uint32_t a = r < KS ? kb + ka[r] : kb + OPB + va[r - KS];
      rf[r][0] = lds_read_b128<0>(a);
      rf[r][1] = lds_read_b128<16 * RB>(a);
      rf[r][2] = lds_read_b128<32 * RB>(a);
      rf[r][3] = lds_read_b128<48 * RB>(a);
    }
  };
#pragma unroll
  for (int u = PRE; u < DEPTH && u < NU; ++u) issue(u);
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
    if (u < NT) {
      const int s = u / FP, p = u % FP;
      pin(tu[u][0]);
      pin(tu[u][1]);
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int qt = 0; qt < 2; ++qt)
          acc[2 * p + i][qt] = Mma16<T>::run(tu[u][i], df[qt][s], acc[2 * p + i][qt]);
    } else {
      const int r = u - NT;
#pragma unroll
      for (int kt = 0; kt < 4; ++kt) pin(rf[r][kt]);
      if (r < KS) {
#pragma unroll
        for (int kt = 0; kt < 4; ++kt)
#pragma unroll
          for (int qt = 0; qt < 2; ++qt)
            st[qt][kt] = Mma16<T>::run(rf[r][kt], qf[qt][r],
                                       r == 0 ? f32x4{0.f, 0.f, 0.f, 0.f} : st[qt][kt]);
      } else {
        const int kk = r - KS;
        // k-step 0 starts from -delta (SEED) or zero.
#pragma unroll
        for (int kt = 0; kt < 4; ++kt)
#pragma unroll
          for (int qt = 0; qt < 2; ++qt) {
            const f32x4 c0 =
                G::SEED ? f32x4{nd[qt], nd[qt], nd[qt], nd[qt]} : f32x4{0.f, 0.f, 0.f, 0.f};
            dp[qt][kt] = Mma16<T>::run(rf[r][kt], of[qt][kk], kk == 0 ? c0 : dp[qt][kt]);
          }
      }
    }
    if (u + DEPTH < NU) issue(u + DEPTH);
    hook(u, NU);
    sched_fence();
  }
}

template <typename T, int D, bool CAUSAL>
__global__ __attribute__((amdgpu_flat_work_group_size(kThreads, kThreads),
                          amdgpu_waves_per_eu(2))) void
attn_bwd_dq_pp_kernel(const T* __restrict__ Q, const T* __restrict__ K, const T* __restrict__ V,
                      const T* __restrict__ dO, T* __restrict__ dQ, const float* __restrict__ lse,
                      const float* __restrict__ delta, DqShape s) {
  using G = DqGeo<D>;
  constexpr int BM = G::BM, BN = G::BN, KS = G::KS, FT = G::FT, RB = G::RB, STB = G::STB, STAGES = G::STAGES, DPB = G::DMA_PER_BLOCK;
  __shared__ __attribute__((aligned(1024))) char lds[STAGES * STB];
  // dQ staging: 16 rows of D values per wave (one query tile at a time); 32 KiB at head_dim
  // 128, so the ring and the staging fill the CU's 160 KiB. Until the epilogue it holds
  // each wave's SIMD id.
  __shared__ __attribute__((aligned(16))) char qstage[G::WAVES * 16 * RB];
  int* const simd_of = reinterpret_cast<int*>(qstage);

  // Workgroup -> (batch*head, query block), as in the forward: XCD-contiguous ranges,
  // causal heaviest-first; varlen: the heavy-first schedule, heads over the XCDs.
  int b, h, qb, start = 0, N = s.seq;
  uint32_t kv_bytes = s.kv_bytes;
  if (s.cu != nullptr) {
    h = varlen_head(blockIdx.x, s.heads);
    VarlenTile vt;
    if (!varlen_tile(s.cu, s.batch, s.total, s.seq, BM, blockIdx.x / s.heads, vt)) return;
    b = vt.b;
    qb = vt.level;
    const VarlenRows rows = varlen_rows(s.cu, b, s.total, s.seq);
    start = rows.start;
    N = rows.n;
    if (qb * BM >= N) return;  // uniform: the whole workgroup leaves
    kv_bytes = uint32_t(((N - 1) * s.kv[2] + D) * 2);
  } else {
    int w = blockIdx.x;
    if (s.tiles % 8 == 0) w = (w % 8) * (s.tiles / 8) + w / 8;
    const int bh = w / s.q_blocks;
    qb = CAUSAL ? s.q_blocks - 1 - w % s.q_blocks : w % s.q_blocks;
    b = bh / s.heads;
    h = bh % s.heads;
  }
  const int64_t qbase = b * s.q[0] + h * s.q[1] + int64_t(start) * s.q[2];
  const int64_t kvbase = b * s.kv[0] + (h / s.group) * s.kv[1] + int64_t(start) * s.kv[2];
  const int64_t stat = s.cu != nullptr ? int64_t(h) * s.total + start
                                       : (int64_t(b) * s.heads + h) * N;

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int c = lane & 15, g = lane >> 4;
  const int q0 = qb * BM;
  const int wq0 = q0 + wave * G::QW;
  if (lane == 0) simd_of[wave] = simd_id();

  const __amdgpu_buffer_rsrc_t rk =
      __builtin_amdgcn_make_buffer_rsrc((void*)(K + kvbase), (short)0, kv_bytes, 0x00020000);
  const __amdgpu_buffer_rsrc_t rv =
      __builtin_amdgcn_make_buffer_rsrc((void*)(V + kvbase), (short)0, kv_bytes, 0x00020000);
  const uint32_t lds_base = (uint32_t)(uintptr_t)(lds_void*)lds;
  uint32_t k_src[G::DMA_PER_OP], v_src[G::DMA_PER_OP];
#pragma unroll
  for (int x = 0; x < G::DMA_PER_OP; ++x) {
    const int id = wave * G::DMA_PER_OP + x;
    const int row = id * G::ROWS_PER_DMA + lane / G::SLOTS;
    const int slot = lane % G::SLOTS;
    k_src[x] = uint32_t(row * s.kv[2] + (slot ^ G::kswz(row)) * 8) * 2u;
    v_src[x] = uint32_t(row * s.kv[2] + (slot ^ G::vswz(row)) * 8) * 2u;
  }
  const int kv_end = CAUSAL ? min(N, q0 + BM) : N;
  const int kv_blocks = (kv_end + BN - 1) / BN;
  const int last = kv_blocks - 1;
  const uint32_t blk_bytes = uint32_t(BN * s.kv[2]) * 2u;
#pragma unroll
  for (int blk = 0; blk < STAGES - 1; ++blk)
    dq_dma_block<D>(rk, rv, lds, k_src, v_src, blk, last, blk_bytes, wave);

  // Q and dO fragments (B operands): query tile qt holds query wq0 + 16 qt + c, k-step kk
  // features 32 kk + 8 g .. +7; lse and delta of the same queries.
  i32x4 qf[2][KS], of[2][KS];
  float lse_q[2];
  float nd[2];  // -delta of the query: the dP^T accumulators' initial value
#pragma unroll
  for (int qt = 0; qt < 2; ++qt) {
    const int query = wq0 + 16 * qt + c;
    const bool in = query < N;
#pragma unroll
    for (int kk = 0; kk < KS; ++kk) {
      const int64_t off = qbase + int64_t(query) * s.q[2] + kk * 32 + g * 8;
      qf[qt][kk] = in ? *reinterpret_cast<const i32x4*>(Q + off) : i32x4{0, 0, 0, 0};
      of[qt][kk] = in ? *reinterpret_cast<const i32x4*>(dO + off) : i32x4{0, 0, 0, 0};
    }
    lse_q[qt] = in ? lse[stat + query] : 0.f;
    nd[qt] = in ? -delta[stat + query] : 0.f;
  }

  // Lane read addresses inside a stage: K / V row c of key tile kt (+16 kt rows), chunk
  // 4 kk + g; transposed K: row 4 g + c / 4 (+32 per key step, +16 for k-index 4..7),
  // features 16 ft + 4 (c % 4) .. +3, i.e. chunk 2 ft + (c % 4) / 2, half (c % 4) % 2.
  uint32_t ka[KS], va[KS], ta[FT];
#pragma unroll
  for (int kk = 0; kk < KS; ++kk) {
    ka[kk] = c * RB + (((4 * kk + g) ^ G::kswz(c)) * 16);
    va[kk] = c * RB + (((4 * kk + g) ^ G::vswz(c)) * 16);
  }
  {
    const int row = 4 * g + (c >> 2), q = c & 3;
#pragma unroll
    for (int ft = 0; ft < FT; ++ft)
      ta[ft] = row * RB + (((2 * ft + (q >> 1)) ^ G::kswz(row)) * 16) + (q & 1) * 8;
  }

  // dQ^T accumulators: acc[ft][qt] register r is feature 16 ft + 4 g + r of query
  // wq0 + 16 qt + c. st / dp [qt][kt] register r: key n0 + 16 kt + 4 g + r.
  f32x4 acc[FT][2], st[2][4], dp[2][4];
  i32x4 df[2][2], tu[G::NT][2];
#pragma unroll
  for (int ft = 0; ft < FT; ++ft)
#pragma unroll
    for (int qt = 0; qt < 2; ++qt) acc[ft][qt] = f32x4{0.f, 0.f, 0.f, 0.f};
  const float sl2 = s.scale_log2;

  wait_lgkm<0>();
  wait_vmcnt<(STAGES - 2) * DPB>();
  barrier_no_fence();
  int grp = 0;
#pragma unroll
  for (int w = 0; w < G::WAVES; ++w) grp += (w < wave && simd_of[w] == simd_of[wave]) ? 1 : 0;
  grp = __builtin_amdgcn_readfirstlane(grp) & 1;
  const int phases = 2 * kv_blocks + 2;
  int t = 0;
  // Block m + STAGES - 2 (m >= 1) is fetched during this wave's MFMA phase of block m
  // (phase 2m + grp), its DMA_PER_BLOCK instructions spread over the phase's read units;
  // after the wave's last MFMA phase, at the start of phase 2m + grp (tail mode). Block m+1
  // was issued by every wave before the end of phase 2m + 1, so the wait at the end of
  // each odd phase, which leaves one block's instructions in flight, still covers it.
  bool tail = false;
  int tail_m = 0;
  auto end_phase = [&]() {
    if (t & 1) wait_vmcnt<(STAGES - 3) * DPB>();
    barrier_no_fence();
    ++t;
    if (tail && tail_m <= kv_blocks && t == 2 * tail_m + grp) {
      dq_dma_block<D>(rk, rv, lds, k_src, v_src, tail_m + STAGES - 2, last, blk_bytes, wave);
      ++tail_m;
    }
  };
  // Hook of the MFMA phase of block m: after unit u of nu, the DMA instructions whose share
  // of the phase ends there (DMA_PER_BLOCK of them over the nu units).
  auto dma_hook = [&](int m) {
    return [&, m](int u, int nu) {
      const int a = (u * DPB) / nu, b2 = ((u + 1) * DPB) / nu;
      if (b2 != a)
        dq_dma_one<D>(rk, rv, lds, k_src, v_src, m + STAGES - 2, last, blk_bytes, wave, b2 - 1);
    };
  };
  auto no_hook = [](int, int) {};
  auto kbase = [&](int j) { return lds_base + (j % STAGES) * STB; };

  // Elementwise phase of block j: P = exp2(S^T c - lse), dS^T = P (dP^T - delta) into df;
  // keys past the end or after the query are masked (diagonal and ragged blocks only).
  auto dS_phase = [&](int j) {
    const int n0 = j * BN;
    const bool need_mask = n0 + BN > N || (CAUSAL && n0 + BN - 1 > wq0);
    if (__builtin_expect(need_mask, 0)) {
#pragma unroll
      for (int qt = 0; qt < 2; ++qt)
#pragma unroll
        for (int kt = 0; kt < 4; ++kt) {
          const int k0 = n0 + 16 * kt + 4 * g;
          int lim = N - 1 - k0;
          if (CAUSAL) lim = min(lim, wq0 + 16 * qt + c - k0);
#pragma unroll
          for (int r = 0; r < 4; ++r)
            if (r > lim) st[qt][kt][r] = kNegInf;
        }
    }
#pragma unroll
    for (int qt = 0; qt < 2; ++qt) {
      const float nl = -lse_q[qt];
#pragma unroll
      for (int kt = 0; kt < 4; ++kt)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float p = __builtin_amdgcn_exp2f(__builtin_fmaf(st[qt][kt][r], sl2, nl));
          // Seeded accumulators already hold dP - delta; nd is -delta.
          dp[qt][kt][r] = G::SEED ? p * dp[qt][kt][r] : p * (dp[qt][kt][r] + nd[qt]);
        }
      df[qt][0] = acc_frag2<T>(dp[qt][0], dp[qt][1]);
      df[qt][1] = acc_frag2<T>(dp[qt][2], dp[qt][3]);
    }
  };
  // Each phase's register results are pinned before its closing barrier (the barrier
  // orders memory only; the compiler would sink register work into the next phase).
  auto pin_mfma = [&]() {
#pragma unroll
    for (int qt = 0; qt < 2; ++qt)
#pragma unroll
      for (int kt = 0; kt < 4; ++kt) {
        pin(st[qt][kt]);
        pin(dp[qt][kt]);
      }
#pragma unroll
    for (int ft = 0; ft < FT; ++ft)
#pragma unroll
      for (int qt = 0; qt < 2; ++qt) pin(acc[ft][qt]);
  };
  // The elementwise phase ends by issuing the first transposed-K units of the next MFMA
  // phase (block j's K tile has landed since phase 2j).
  auto pin_dS = [&](int j) {
#pragma unroll
    for (int qt = 0; qt < 2; ++qt) {
      pin(df[qt][0]);
      pin(df[qt][1]);
    }
#pragma unroll
    for (int u = 0; u < G::PREFETCH; ++u) read_t_unit<D>(tu, kbase(j), ta, u);
  };

  const int n = CAUSAL ? min(kv_blocks, (wq0 + G::QW - 1) / BN + 1) : kv_blocks;
  if (grp) end_phase();
  dq_mfma_phase<T, D, true, false>(no_hook, kbase(0), 0, ka, va, ta, qf, of, st, dp, nd, df, acc,
                                   tu);
  pin_mfma();
  end_phase();
  for (int j = 1; j < n; ++j) {
    dS_phase(j - 1);
    pin_dS(j - 1);
    end_phase();
    dq_mfma_phase<T, D, true, true>(dma_hook(j), kbase(j), kbase(j - 1), ka, va, ta, qf, of, st, dp,
                                    nd, df, acc, tu);
    pin_mfma();
    end_phase();
  }
  dS_phase(n - 1);
  pin_dS(n - 1);
  end_phase();
  dq_mfma_phase<T, D, false, true>(dma_hook(n), 0, kbase(n - 1), ka, va, ta, qf, of, st, dp, nd,
                                   df, acc, tu);
  tail = true;
  tail_m = n + 1;
  while (t < phases - 1) end_phase();
  wait_vmcnt<0>();

  // dQ = scale (dQ^T)^T: acc[ft][qt] register r is feature 16 ft + 4 g + r of query
  // wq0 + 16 qt + c, 8 bytes once rounded. Each query tile goes through the wave's own
  // staging rows (every wave has read the SIMD ids long before) and leaves as whole rows,
  // 16 bytes per lane and full 128-byte lines, with non-temporal stores; the entry points
  // accept only 16-byte aligned tensors and strides that are multiples of 8 elements, so
  // every dQ row is 16-byte aligned. Lane indices are formed afresh rather than held across
  // the key loop.
  int el = threadIdx.x & 63;
  asm volatile("" : "+v"(el));
  const int ec = el & 15, eg = el >> 4;
  T* const dQh = dQ + qbase;
  char* const qrows = qstage + wave * (16 * RB);
#pragma unroll
  for (int qt = 0; qt < 2; ++qt) {
#pragma unroll
    for (int ft = 0; ft < FT; ++ft) {
      uint2 u;
      u.x = pack2<T>(acc[ft][qt][0] * s.scale, acc[ft][qt][1] * s.scale);
      u.y = pack2<T>(acc[ft][qt][2] * s.scale, acc[ft][qt][3] * s.scale);
      *reinterpret_cast<uint2*>(qrows + ec * RB + (((2 * ft + (eg >> 1)) ^ G::oswz(ec)) * 16) +
                                (eg & 1) * 8) = u;
    }
    constexpr int LPR = RB / 16, RPI = 64 / LPR;  // lanes per row, rows per instruction
#pragma unroll
    for (int p = 0; p < 16 / RPI; ++p) {
      const int r = p * RPI + el / LPR, q = el % LPR;
      const i32x4 v = *reinterpret_cast<const i32x4*>(qrows + r * RB + ((q ^ G::oswz(r)) * 16));
      const int row_query = wq0 + 16 * qt + r;
      if (row_query < N)
        __builtin_nontemporal_store(
            v, reinterpret_cast<i32x4*>(dQh + int64_t(row_query) * s.q[2] + q * 8));
    }
  }
}

template <typename T, int D>
void launch(bool causal, dim3 grid, hipStream_t st, const void* q, const void* k, const void* v,
            const void* dout, void* dq, const float* lse, const float* delta, const DqShape& s) {
  if (causal)
    hipLaunchKernelGGL((attn_bwd_dq_pp_kernel<T, D, true>), grid, dim3(kThreads), 0, st,
                       (const T*)q, (const T*)k, (const T*)v, (const T*)dout, (T*)dq, lse, delta, s);
  else
    hipLaunchKernelGGL((attn_bwd_dq_pp_kernel<T, D, false>), grid, dim3(kThreads), 0, st,
                       (const T*)q, (const T*)k, (const T*)v, (const T*)dout, (T*)dq, lse, delta, s);
}

}  // namespace

namespace tk {

void attn_bwd_dq_dma_launch(int dtype, const void* q, const void* k, const void* v,
                           const void* dout, void* dq, const float* lse, const float* delta,
                           int64_t batch, int64_t heads, int64_t kv_heads, int64_t seq,
                           int64_t head_dim, const int64_t* q_strides, const int64_t* kv_strides,
                           float sm_scale, bool causal, hipStream_t stream,
                           const int32_t* cu_seqlens, int64_t total) {
  DqShape s{};
  s.heads = (int)heads;
  s.seq = (int)seq;
  s.group = (int)(heads / kv_heads);
  s.cu = cu_seqlens;
  s.total = (int)total;
  s.batch = (int)batch;
  for (int i = 0; i < 3; ++i) {
    s.q[i] = q_strides[i];
    s.kv[i] = kv_strides[i];
  }
  s.scale = sm_scale;
  s.scale_log2 = sm_scale * 1.4426950408889634f;
  s.q_blocks = (int)cdiv(seq, 256);
  s.tiles = cu_seqlens != nullptr ? (int)(varlen_tiles(batch, total, seq, 256) * heads)
                                  : (int)(s.q_blocks * batch * heads);
  s.kv_bytes = (uint32_t)(((seq - 1) * kv_strides[2] + head_dim) * 2);
  const dim3 grid(static_cast<unsigned>(s.tiles));
  if (dtype == TK_DTYPE_F16) {
    if (head_dim == 64) launch<_Float16, 64>(causal, grid, stream, q, k, v, dout, dq, lse, delta, s);
    else launch<_Float16, 128>(causal, grid, stream, q, k, v, dout, dq, lse, delta, s);
  } else {
    if (head_dim == 64) launch<__bf16, 64>(causal, grid, stream, q, k, v, dout, dq, lse, delta, s);
    else launch<__bf16, 128>(causal, grid, stream, q, k, v, dout, dq, lse, delta, s);
  }
}

}  // namespace tk
