// Flash attention forward for head_dim 64/128 (f16/bf16) on CDNA4 MFMA: the path behind
// tk_attn_fwd (src/tklab/kernels/flash_attention.py:124-264 is the Triton kernel it
// replaces: base-2 online softmax on scores * scale * log2(e) in _attention_inner
// (:55-121), O = acc / l and log-sum-exp m + log2(l) (:248-264)).
//
// Workgroup: 256 queries, 8 wave64s of 32 queries, two waves per SIMD, so one wave's
// softmax (VALU, transcendental) runs while the other wave's MFMAs occupy the matrix
// pipe. Key/value blocks of 64.
//
// Per wave and key block:
//   S^T = K Q^T   2 key tiles (32 x 32) over D/16 k-steps: an accumulator lane owns one
//                 query (column lane % 32) and 16 keys of each tile; the partner lane
//                 lane ^ 32 holds the other keys, so row max/sum need one permlane32 swap.
//   softmax       masked only on diagonal / ragged blocks; the O rescale is skipped when
//                 no row max of the wave moved (alpha == 1 exactly).
//   O^T += V^T P^T  D/32 feature tiles over 4 steps of 16 keys; P^T comes straight from
//                 the S^T registers (registers 8g..8g+7 of a lane hold keys
//                 16g + 4 hi + {0..3} and 16g + 8 + 4 hi + {0..3}), and V^T fragments
//                 are read with ds_read_b64_tr_b16 from row-major V using exactly those
//                 two 4-key row groups, so no data permutation is needed anywhere.
// Q fragments stay in registers for the whole key loop.
//
// K and V blocks reach LDS by buffer->LDS DMA (no VGPR staging) into a 3-stage ring,
// two blocks ahead; one barrier per block orders every reuse. LDS layouts keep every read
// phase on 64 distinct banks:
//   K [64 keys][D]: 16-byte chunk c of row r at slot c ^ kswz(r) (ds_read_b128, 16 lanes
//                   per phase read 16 rows of one chunk);
//   V [64 keys][D]: 32-byte granule g of row r at granule g ^ vswz(r) (ds_read_b64_tr_b16,
//                   32 lanes per phase read 4 rows x 2 granules).
// The DMA writes 1 KiB contiguous per instruction, so the swizzle is applied on the global
// side (each lane fetches the chunk that belongs in its LDS slot). LDS reads are inline
// asm ordered by explicit waits: the compiler would otherwise wait for every outstanding
// DMA before each read.
#include "attention.hpp"
#include "attention_dma.hpp"

namespace {

using namespace tk_attn;

constexpr int kThreads = 512;

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
  static constexpr int KS = D / 16, DT = D / 32;
  static constexpr int RB = D * 2;              // bytes per K/V row
  static constexpr int OPB = BN * RB;           // bytes per operand per stage
  static constexpr int STB = 2 * OPB;           // stage: K tile then V tile
  static constexpr int STAGES = 3;
  static constexpr int ROWS_PER_DMA = 1024 / RB;
  static constexpr int DMA_PER_OP = OPB / 1024 / WAVES;  // per wave, per operand
  static constexpr int DMA_PER_BLOCK = 2 * DMA_PER_OP;
  static constexpr int SLOTS = RB / 16;         // 16-byte slots per row
  static __device__ __forceinline__ int kswz(int r) { return D == 128 ? (r & 15) : ((r >> 1) & 7); }
  static __device__ __forceinline__ int vswz(int r) { return D == 128 ? 2 * (r & 3) : 2 * ((r >> 1) & 1); }
};

// DMA of key/value block `blk` (clamped to `last`: blocks past the end reload the last
// one into a stage that is never read, keeping the per-block load count constant).
template <int D>
__device__ __forceinline__ void dma_block(__amdgpu_buffer_rsrc_t rk, __amdgpu_buffer_rsrc_t rv,
                                          char* stage, const uint32_t* k_src,
                                          const uint32_t* v_src, int blk, int last,
                                          uint32_t k_blk, uint32_t v_blk, int wave) {
  using G = Geo<D>;
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

template <typename T, int D, bool CAUSAL>
__global__ __attribute__((amdgpu_flat_work_group_size(kThreads, kThreads))) void
attn_fwd_dma_kernel(const T* __restrict__ Q, const T* __restrict__ K, const T* __restrict__ V,
                    T* __restrict__ O, float* __restrict__ lse, Shape s) {
  using G = Geo<D>;
  constexpr int BM = G::BM, BN = G::BN, KS = G::KS, DT = G::DT, RB = G::RB, OPB = G::OPB,
                STB = G::STB, STAGES = G::STAGES;
  __shared__ __attribute__((aligned(1024))) char lds[STAGES * STB];

  // Workgroup -> (batch*head, query block). Equal lengths: XCD-contiguous ranges so a
  // head's blocks share one L2; causal: the heaviest (last) query block of a head first.
  // Varlen: the heavy-first schedule over every sequence's query blocks (level = query
  // block), heads interleaved over the XCDs.
  int b, h, qb, start = 0, N = s.seq;
  uint32_t k_bytes = s.k_bytes, v_bytes = s.v_bytes;
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
    k_bytes = uint32_t(((N - 1) * s.k[2] + D) * 2);
    v_bytes = uint32_t(((N - 1) * s.v[2] + D) * 2);
  } else {
    int w = blockIdx.x;
    if (s.tiles % 8 == 0) w = (w % 8) * (s.tiles / 8) + w / 8;
    const int bh = w / s.q_blocks;
    qb = CAUSAL ? s.q_blocks - 1 - w % s.q_blocks : w % s.q_blocks;
    b = bh / s.heads;
    h = bh % s.heads;
  }
  const int kvh = h / s.group;
  const T* Qh = Q + b * s.q[0] + h * s.q[1] + int64_t(start) * s.q[2];
  const T* Kh = K + b * s.k[0] + kvh * s.k[1] + int64_t(start) * s.k[2];
  const T* Vh = V + b * s.v[0] + kvh * s.v[1] + int64_t(start) * s.v[2];
  T* Oh = O + b * s.o[0] + h * s.o[1] + int64_t(start) * s.o[2];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int l32 = lane & 31, hi = lane >> 5;
  const int q0 = qb * BM;
  const int wq0 = q0 + wave * G::QW;

  const __amdgpu_buffer_rsrc_t rk =
      __builtin_amdgcn_make_buffer_rsrc((void*)Kh, (short)0, k_bytes, 0x00020000);
  const __amdgpu_buffer_rsrc_t rv =
      __builtin_amdgcn_make_buffer_rsrc((void*)Vh, (short)0, v_bytes, 0x00020000);
  const uint32_t lds_base = (uint32_t)(uintptr_t)(lds_void*)lds;

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
  const uint32_t k_blk = uint32_t(BN * s.k[2]) * 2u, v_blk = uint32_t(BN * s.v[2]) * 2u;

  // Q fragments (B operand of S^T): query wq0 + l32, features 16 kk + 8 hi .. +7.
  i32x4 qf[KS];
  {
    const int query = wq0 + l32;
#pragma unroll
    for (int kk = 0; kk < KS; ++kk)
      qf[kk] = query < N ? *reinterpret_cast<const i32x4*>(Qh + query * s.q[2] + kk * 16 + hi * 8)
                         : i32x4{0, 0, 0, 0};
  }
  // RoPE tables of this lane's query, loaded with Q; the rotation waits until the first
  // K/V blocks' DMA has been issued.
  const bool rope = s.rope_cos != nullptr && wq0 + l32 < N;
  i32x4 rc[KS / 2], rsn[KS / 2];
  if (rope) {
    const int64_t at = int64_t(wq0 + l32) * s.rope_stride + hi * 8;
    const T* cr = static_cast<const T*>(s.rope_cos) + at;
    const T* sr = static_cast<const T*>(s.rope_sin) + at;
#pragma unroll
    for (int kk = 0; kk < KS / 2; ++kk) {
      rc[kk] = *reinterpret_cast<const i32x4*>(cr + kk * 16);
      rsn[kk] = *reinterpret_cast<const i32x4*>(sr + kk * 16);
    }
  }
  // Lane read addresses inside a stage: K row l32 (+32 for the second key tile), chunk
  // 2 kk + hi; V rows 4 hi + j (+16 per key step, +8 for k-index 4..7), features
  // 32 dt + 16 g + 4 q .. +3.
  uint32_t ka[KS], va[DT];
#pragma unroll
  for (int kk = 0; kk < KS; ++kk) ka[kk] = l32 * RB + (((2 * kk + hi) ^ G::kswz(l32)) * 16);
  {
    const int g = (lane >> 4) & 1, j = (lane & 15) >> 2, q = lane & 3;
    const int row = 4 * hi + j;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
      va[dt] = OPB + row * RB + (((2 * dt + g) ^ G::vswz(row)) * 32) + q * 8;
  }

  f32x16 acc[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[dt][r] = 0.f;
  float m_run = kNegInf, l_part = 0.f;
  const float sl2 = s.scale_log2;

  dma_block<D>(rk, rv, lds, k_src, v_src, 0, kv_blocks - 1, k_blk, v_blk, wave);
  dma_block<D>(rk, rv, lds + STB, k_src, v_src, 1, kv_blocks - 1, k_blk, v_blk, wave);
  // Fragments kk and kk + KS/2 hold features 16 kk + 8 hi .. +7 and the same + D/2: the
  // rotate-half pairs sit in one lane.
  if (rope) {
#pragma unroll
    for (int kk = 0; kk < KS / 2; ++kk) rope_fragment<T>(qf[kk], qf[kk + KS / 2], rc[kk], rsn[kk]);
  }
  int stage = 0, fill = 2;
  // This wave multiplies a prefix of the workgroup's blocks (causal: those starting at or
  // before its last query) and only helps to load the rest.
  const int wave_blocks = CAUSAL ? min(kv_blocks, (wq0 + G::QW - 1) / BN + 1) : kv_blocks;
  int j = 0;
  for (; j < wave_blocks; ++j) {
    // Block j has landed once only block j+1's loads are pending; the barrier makes every
    // wave's share visible and retires all reads of block j-1, whose stage is refilled.
    wait_vmcnt<G::DMA_PER_BLOCK>();
    barrier_no_fence();
    dma_block<D>(rk, rv, lds + fill * STB, k_src, v_src, j + 2, kv_blocks - 1, k_blk, v_blk,
                 wave);
    const int n0 = j * BN;
    const uint32_t base = lds_base + stage * STB;

    // S^T = K Q^T; the second half of the feature range is read during the first's MFMAs.
    i32x4 kf[2][2][KS / 2];
#pragma unroll
    for (int half = 0; half < 2; ++half)
#pragma unroll
      for (int i = 0; i < KS / 2; ++i) {
        kf[half][0][i] = lds_read_b128<0>(base + ka[half * (KS / 2) + i]);
        kf[half][1][i] = lds_read_b128<32 * RB>(base + ka[half * (KS / 2) + i]);
      }
    f32x16 st[2];
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      if (half == 0)
        wait_lgkm<KS>();  // the KS reads of the second half may still be in flight
      else
        wait_lgkm<0>();
#pragma unroll
      for (int i = 0; i < KS / 2; ++i) {
        pin(kf[half][0][i]);
        pin(kf[half][1][i]);
      }
#pragma unroll
      for (int i = 0; i < KS / 2; ++i) {
        const int kk = half * (KS / 2) + i;
        if (kk == 0) {
          const f32x16 z = {};
          st[0] = Mma<T>::run(kf[0][0][0], qf[0], z);
          st[1] = Mma<T>::run(kf[0][1][0], qf[0], z);
        } else {
          st[0] = Mma<T>::run(kf[half][0][i], qf[kk], st[0]);
          st[1] = Mma<T>::run(kf[half][1][i], qf[kk], st[1]);
        }
      }
    }

    // Online softmax for query wq0 + l32. Register r of key tile nt holds key
    // n0 + 32 nt + 4 hi + 8 (r / 4) + r % 4.
    const int query = wq0 + l32;
    const bool need_mask = n0 + BN > N || (CAUSAL && n0 + BN - 1 > wq0);
    if (__builtin_expect(need_mask, 0)) {
#pragma unroll
      for (int nt = 0; nt < 2; ++nt) {
        int lim = N - 1 - (n0 + nt * 32 + 4 * hi);  // last valid offset from the lane's first key
        if (CAUSAL) lim = min(lim, query - (n0 + nt * 32 + 4 * hi));
#pragma unroll
        for (int r = 0; r < 16; ++r)
          if (((r >> 2) << 3) + (r & 3) > lim) st[nt][r] = kNegInf;
      }
    }
    float mx = kNegInf;
#pragma unroll
    for (int nt = 0; nt < 2; ++nt)
#pragma unroll
      for (int r = 0; r < 16; ++r) mx = fmaxf(mx, st[nt][r]);
    mx = max_with_partner(mx);
    const float m_new = fmaxf(m_run, mx * sl2);

    // First two 16-key steps of V^T, read while the exponentials run.
    i32x4 vf[2][DT];
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
      vf[0][dt] = read_v<0, RB>(base + va[dt]);
      vf[1][dt] = read_v<16, RB>(base + va[dt]);
    }
    const float neg = -m_new;
    float sum = 0.f;
#pragma unroll
    for (int nt = 0; nt < 2; ++nt)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float p = __builtin_amdgcn_exp2f(__builtin_fmaf(st[nt][r], sl2, neg));
        st[nt][r] = p;
        sum += p;
      }
    const float alpha = m_new == kNegInf ? 1.f : __builtin_amdgcn_exp2f(m_run - m_new);
    l_part = l_part * alpha + sum;
    if (__builtin_amdgcn_ballot_w64(alpha != 1.f)) {
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[dt][r] *= alpha;
    }
    m_run = m_new;
    const i32x4 pf[4] = {acc_frag<T>(st[0], 0), acc_frag<T>(st[0], 1), acc_frag<T>(st[1], 0),
                         acc_frag<T>(st[1], 1)};

    // O^T += V^T P^T; the last two key steps are read during the first two's MFMAs.
    wait_lgkm<0>();
#pragma unroll
    for (int g = 0; g < 2; ++g)
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) pin(vf[g][dt]);
    i32x4 vf2[2][DT];
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
      vf2[0][dt] = read_v<32, RB>(base + va[dt]);
      vf2[1][dt] = read_v<48, RB>(base + va[dt]);
    }
#pragma unroll
    for (int g = 0; g < 2; ++g)
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) acc[dt] = Mma<T>::run(vf[g][dt], pf[g], acc[dt]);
    wait_lgkm<0>();
#pragma unroll
    for (int g = 0; g < 2; ++g)
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) pin(vf2[g][dt]);
#pragma unroll
    for (int g = 0; g < 2; ++g)
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) acc[dt] = Mma<T>::run(vf2[g][dt], pf[2 + g], acc[dt]);

    stage = stage + 1 == STAGES ? 0 : stage + 1;
    fill = fill + 1 == STAGES ? 0 : fill + 1;
  }
  for (; j < kv_blocks; ++j) {
    wait_vmcnt<G::DMA_PER_BLOCK>();
    barrier_no_fence();
    dma_block<D>(rk, rv, lds + fill * STB, k_src, v_src, j + 2, kv_blocks - 1, k_blk, v_blk,
                 wave);
    fill = fill + 1 == STAGES ? 0 : fill + 1;
  }
  // No DMA may still be writing when the workgroup's LDS is released.
  wait_vmcnt<0>();

  // O = O^T / l: register r of tile dt is feature 32 dt + 8 (r / 4) + 4 hi + r % 4.
  const float l = sum_with_partner(l_part);
  const float inv = 1.0f / l;
  const int query = wq0 + l32;
  if (query < N) {
    T* orow = Oh + query * s.o[2];
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int g4 = 0; g4 < 4; ++g4) {
        const int d = dt * 32 + g4 * 8 + hi * 4;
        uint2 u;
        u.x = pack2<T>(acc[dt][g4 * 4 + 0] * inv, acc[dt][g4 * 4 + 1] * inv);
        u.y = pack2<T>(acc[dt][g4 * 4 + 2] * inv, acc[dt][g4 * 4 + 3] * inv);
        *reinterpret_cast<uint2*>(orow + d) = u;
      }
    if (lse != nullptr && hi == 0) {
      const int64_t at = s.cu != nullptr ? int64_t(h) * s.total + start + query
                                         : (int64_t(b) * s.heads + h) * N + query;
      lse[at] = m_run + __log2f(l);
    }
  }
}

template <typename T, int D>
void launch(bool causal, dim3 grid, hipStream_t st, const void* q, const void* k, const void* v,
            void* o, float* lse, const Shape& s) {
  if (causal)
    hipLaunchKernelGGL((attn_fwd_dma_kernel<T, D, true>), grid, dim3(kThreads), 0, st,
                       (const T*)q, (const T*)k, (const T*)v, (T*)o, lse, s);
  else
    hipLaunchKernelGGL((attn_fwd_dma_kernel<T, D, false>), grid, dim3(kThreads), 0, st,
                       (const T*)q, (const T*)k, (const T*)v, (T*)o, lse, s);
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
  const dim3 grid(static_cast<unsigned>(s.tiles));
  if (dtype == TK_DTYPE_F16) {
    if (head_dim == 64) launch<_Float16, 64>(causal, grid, stream, q, k, v, o, lse, s);
    else launch<_Float16, 128>(causal, grid, stream, q, k, v, o, lse, s);
  } else {
    if (head_dim == 64) launch<__bf16, 64>(causal, grid, stream, q, k, v, o, lse, s);
    else launch<__bf16, 128>(causal, grid, stream, q, k, v, o, lse, s);
  }
}

}  // namespace tk
