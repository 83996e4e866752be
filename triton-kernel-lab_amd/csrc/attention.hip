// Flash attention forward and recompute backward on CDNA4 MFMA
// (v_mfma_f32_32x32x16_{f16,bf16}), head_dim D in {64, 128}.
//
// Reference semantics (src/tklab/kernels/flash_attention.py): base-2 online
// softmax on scores * scale * log2(e) (:90-117), O = acc / l, base-2
// log-sum-exp m + log2(l) (:248-264); backward = delta preprocess (:383-395),
// a dK/dV pass over query blocks (:437-466) and a dQ pass over key blocks
// (:512-533), each output written by exactly one workgroup.
//
// Layout choices (all MI355X-specific):
//  * The forward and dQ passes compute S^T = K Q^T, so an accumulator lane owns
//    one query (column l % 32) and 16 keys per 32 x 32 tile; a query's row max
//    and row sum need one exchange with lane l ^ 32 only. The dK/dV pass
//    computes S = Q K^T so a lane owns one key.
//  * MFMA operands must be K-contiguous per lane. Where the contraction runs
//    over the sequence (P V, dS K, P^T dO, dS^T Q), the sequence-major operand
//    is staged TRANSPOSED in LDS ([D][64 positions]) and its 64 sequence indices
//    are permuted within each group of 16 (swap of index bits 2 and 3) so that
//    the 8 indices one accumulator lane holds in registers g*8..g*8+7 are 8
//    consecutive positions: the probability tile then feeds the next MFMA
//    straight from registers.
//  * Row-major LDS tiles ([64][D]) and transposed tiles ([D][64]) store 16-byte
//    chunk c of row r at chunk c ^ (r % 8): 8 consecutive rows read by one
//    operand load hit 8 distinct bank groups.
#include "attention.hpp"
#include "tk_common.hpp"

namespace {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kThreads = 256;
constexpr float kNegInf = -INFINITY;

template <typename T>
struct Mma;
template <>
struct Mma<_Float16> {
  using Frag = f16x8;
  static __device__ __forceinline__ f32x16 run(Frag a, Frag b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
};
template <>
struct Mma<__bf16> {
  using Frag = bf16x8;
  static __device__ __forceinline__ f32x16 run(Frag a, Frag b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
};

__device__ __forceinline__ f32x16 zero16() {
  f32x16 z;
#pragma unroll
  for (int i = 0; i < 16; ++i) z[i] = 0.f;
  return z;
}

// Swap of bits 2 and 3: sequence index <-> position inside a 16-group (an involution).
__device__ __forceinline__ int perm16(int i) {
  return (i & ~15) | (i & 3) | (((i >> 3) & 1) << 2) | (((i >> 2) & 1) << 3);
}

// Accumulator register r of lane `lane` in a 32 x 32 tile sits at row
// 8*(r/4) + 4*(lane/32) + r%4 and column lane % 32.
__device__ __forceinline__ int acc_row(int r, int lane) {
  return ((r >> 2) << 3) + ((lane >> 5) << 2) + (r & 3);
}

template <typename T>
__device__ __forceinline__ uint32_t pack2(float lo, float hi) {
  const uint16_t a = __builtin_bit_cast(uint16_t, tk::from_f32<T>(lo));
  const uint16_t b = __builtin_bit_cast(uint16_t, tk::from_f32<T>(hi));
  return uint32_t(a) | (uint32_t(b) << 16);
}

// Registers g*8 .. g*8+7 of an accumulator, rounded to T, as an MFMA operand.
template <typename T>
__device__ __forceinline__ typename Mma<T>::Frag acc_frag(const f32x16& acc, int g) {
  uint4 u;
  u.x = pack2<T>(acc[g * 8 + 0], acc[g * 8 + 1]);
  u.y = pack2<T>(acc[g * 8 + 2], acc[g * 8 + 3]);
  u.z = pack2<T>(acc[g * 8 + 4], acc[g * 8 + 5]);
  u.w = pack2<T>(acc[g * 8 + 6], acc[g * 8 + 7]);
  return __builtin_bit_cast(typename Mma<T>::Frag, u);
}

__device__ __forceinline__ uint32_t word(const uint4& v, int i) {
  return i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w;
}

__device__ __forceinline__ uint16_t half_of(const uint4& v, int e) {
  const uint32_t w = word(v, e >> 1);
  return static_cast<uint16_t>((e & 1) ? (w >> 16) : (w & 0xffffu));
}

// ---------------------------------------------------------------- LDS tiles
//
// A tile covers 64 sequence indices x D features. Row tiles are [64][D]
// (feature-contiguous); transposed tiles are [D][64] (position-contiguous).

template <int D>
struct RowTile {
  static constexpr int kPerThread = 64 * D / 8 / kThreads;  // 16-byte chunks per thread
  uint4 r[kPerThread];

  template <typename T>
  __device__ __forceinline__ void load(const T* __restrict__ base, int64_t stride, int row0,
                                       int rows) {
#pragma unroll
    for (int c = 0; c < kPerThread; ++c) {
      const int idx = c * kThreads + threadIdx.x;
      const int row = idx / (D / 8), ch = idx % (D / 8);
      r[c] = (row0 + row < rows)
                 ? *reinterpret_cast<const uint4*>(base + (row0 + row) * stride + ch * 8)
                 : make_uint4(0, 0, 0, 0);
    }
  }
  __device__ __forceinline__ void store(uint16_t* __restrict__ lds) const {
#pragma unroll
    for (int c = 0; c < kPerThread; ++c) {
      const int idx = c * kThreads + threadIdx.x;
      const int row = idx / (D / 8), ch = idx % (D / 8);
      *reinterpret_cast<uint4*>(lds + row * D + ((ch ^ (row & 7)) << 3)) = r[c];
    }
  }
};

template <int D>
struct TransTile {
  static constexpr int kPerThread = D / 32;        // sequence positions per thread
  static constexpr int kThreadsPerBlock = 256 / D;  // threads sharing one 8 x 8 block
  uint4 r[kPerThread];

  template <typename T>
  __device__ __forceinline__ void load(const T* __restrict__ base, int64_t stride, int row0,
                                       int rows) {
    const int blk = threadIdx.x / kThreadsPerBlock, part = threadIdx.x % kThreadsPerBlock;
    const int c = blk & 7, db = blk >> 3;
#pragma unroll
    for (int i = 0; i < kPerThread; ++i) {
      const int seq = perm16(c * 8 + part * kPerThread + i);
      r[i] = (row0 + seq < rows)
                 ? *reinterpret_cast<const uint4*>(base + (row0 + seq) * stride + db * 8)
                 : make_uint4(0, 0, 0, 0);
    }
  }
  __device__ __forceinline__ void store(uint16_t* __restrict__ lds) const {
    const int blk = threadIdx.x / kThreadsPerBlock, part = threadIdx.x % kThreadsPerBlock;
    const int c = blk & 7, db = blk >> 3;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int d = db * 8 + e;
      uint16_t* dst = lds + d * 64 + ((c ^ (d & 7)) << 3) + part * kPerThread;
      if constexpr (kPerThread == 4) {
        const uint32_t w0 = uint32_t(half_of(r[0], e)) | (uint32_t(half_of(r[1], e)) << 16);
        const uint32_t w1 = uint32_t(half_of(r[2], e)) | (uint32_t(half_of(r[3], e)) << 16);
        *reinterpret_cast<uint2*>(dst) = make_uint2(w0, w1);
      } else {
        *reinterpret_cast<uint32_t*>(dst) =
            uint32_t(half_of(r[0], e)) | (uint32_t(half_of(r[1], e)) << 16);
      }
    }
  }
};

// Operand fragment from a row tile: row `row`, 16-byte chunk `chunk`.
template <typename T, int D>
__device__ __forceinline__ typename Mma<T>::Frag row_frag(const uint16_t* lds, int row, int chunk) {
  return *reinterpret_cast<const typename Mma<T>::Frag*>(lds + row * D + ((chunk ^ (row & 7)) << 3));
}

// Operand fragment from a transposed tile: feature row `d`, position chunk `chunk`.
template <typename T>
__device__ __forceinline__ typename Mma<T>::Frag trans_frag(const uint16_t* lds, int d, int chunk) {
  return *reinterpret_cast<const typename Mma<T>::Frag*>(lds + d * 64 + ((chunk ^ (d & 7)) << 3));
}

// Fragment straight from global memory (row `row` of a [rows][D] matrix).
template <typename T>
__device__ __forceinline__ typename Mma<T>::Frag global_frag(const T* base, int64_t stride, int row,
                                                             int rows, int col) {
  uint4 u = row < rows ? *reinterpret_cast<const uint4*>(base + row * stride + col)
                       : make_uint4(0, 0, 0, 0);
  return __builtin_bit_cast(typename Mma<T>::Frag, u);
}

struct Shape {
  int heads, seq;
  int64_t q[3], k[3], v[3], o[3];  // batch, head, seq strides
  float scale, scale_log2;
  int q_blocks, tiles;
};

// Workgroup -> (batch*head, query block): XCD-contiguous tile ranges (a head's
// query blocks run on one XCD and share its L2); for causal masks the
// heaviest (last) query block of a head first.
template <bool CAUSAL>
__device__ __forceinline__ void tile_of(const Shape& s, int& bh, int& qb) {
  int w = blockIdx.x;
  if (s.tiles % 8 == 0) w = (w % 8) * (s.tiles / 8) + w / 8;
  bh = w / s.q_blocks;
  qb = w % s.q_blocks;
  if (CAUSAL) qb = s.q_blocks - 1 - qb;
}

// ---------------------------------------------------------------- forward
//
// Register-staged forward, used only when a head's K or V rows span 2 GiB or more
// (the DMA forward in attention_fwd.hip addresses them with 32-bit offsets).
// Workgroup: 256 queries (4 waves x 64); key blocks of 64.
// Per wave and key block: S^T (2 key tiles x 2 query tiles) over D/16 steps,
// softmax, O^T (D/32 feature tiles x 2 query tiles) += V^T P^T over 4 steps.

template <typename T, int D, bool CAUSAL>
__global__ __attribute__((amdgpu_flat_work_group_size(kThreads, kThreads),
                          amdgpu_waves_per_eu(1, 1))) void
attn_fwd_kernel(const T* __restrict__ Q, const T* __restrict__ K, const T* __restrict__ V,
                T* __restrict__ O, float* __restrict__ lse, Shape s) {
  using Frag = typename Mma<T>::Frag;
  constexpr int BM = 256, BN = 64, DT = D / 32, KS = D / 16;
  __shared__ __attribute__((aligned(16))) uint16_t k_lds[2][64 * D];
  __shared__ __attribute__((aligned(16))) uint16_t v_lds[2][64 * D];

  int bh, qb;
  tile_of<CAUSAL>(s, bh, qb);
  const int b = bh / s.heads, h = bh % s.heads;
  const T* Qh = Q + b * s.q[0] + h * s.q[1];
  const T* Kh = K + b * s.k[0] + h * s.k[1];
  const T* Vh = V + b * s.v[0] + h * s.v[1];
  T* Oh = O + b * s.o[0] + h * s.o[1];
  const int N = s.seq;

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int l32 = lane & 31, hi = lane >> 5;
  const int q0 = qb * BM;
  const int wq0 = q0 + wave * 64;  // this wave's first query

  Frag qf[2][KS];
#pragma unroll
  for (int mt = 0; mt < 2; ++mt)
#pragma unroll
    for (int kk = 0; kk < KS; ++kk)
      qf[mt][kk] = global_frag<T>(Qh, s.q[2], wq0 + mt * 32 + l32, N, kk * 16 + hi * 8);

  f32x16 acc_o[DT][2];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) acc_o[dt][0] = acc_o[dt][1] = zero16();
  float m_run[2] = {kNegInf, kNegInf};
  float l_part[2] = {0.f, 0.f};

  const int kv_end = CAUSAL ? min(N, q0 + BM) : N;
  const int kv_blocks = (kv_end + BN - 1) / BN;

  RowTile<D> kst;
  TransTile<D> vst;
  kst.load(Kh, s.k[2], 0, N);
  vst.load(Vh, s.v[2], 0, N);
  kst.store(k_lds[0]);
  vst.store(v_lds[0]);
  __syncthreads();

  for (int j = 0; j < kv_blocks; ++j) {
    const int buf = j & 1;
    const int n0 = j * BN;
    const bool more = j + 1 < kv_blocks;
    if (more) {
      kst.load(Kh, s.k[2], n0 + BN, N);
      vst.load(Vh, s.v[2], n0 + BN, N);
    }
    // A wave whose queries all precede the block's first key has nothing to add.
    const bool active = !CAUSAL || n0 <= wq0 + 63;
    if (active) {
      const uint16_t* kl = k_lds[buf];
      const uint16_t* vl = v_lds[buf];
      f32x16 st[2][2];
#pragma unroll
      for (int nt = 0; nt < 2; ++nt) st[nt][0] = st[nt][1] = zero16();
#pragma unroll
      for (int kk = 0; kk < KS; ++kk) {
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) {
          const Frag kf = row_frag<T, D>(kl, nt * 32 + l32, kk * 2 + hi);
          st[nt][0] = Mma<T>::run(kf, qf[0][kk], st[nt][0]);
          st[nt][1] = Mma<T>::run(kf, qf[1][kk], st[nt][1]);
        }
      }
      const bool need_mask = n0 + BN > N || (CAUSAL && n0 + BN - 1 > wq0);
#pragma unroll
      for (int mt = 0; mt < 2; ++mt) {
        const int query = wq0 + mt * 32 + l32;
        float mx = kNegInf;
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) {
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            float x = st[nt][mt][r] * s.scale_log2;
            if (need_mask) {
              const int key = n0 + nt * 32 + acc_row(r, lane);
              if (key >= N || (CAUSAL && key > query)) x = kNegInf;
            }
            st[nt][mt][r] = x;
            mx = fmaxf(mx, x);
          }
        }
        mx = fmaxf(mx, __shfl_xor(mx, 32));
        const float m_new = fmaxf(m_run[mt], mx);
        const float alpha = __builtin_amdgcn_exp2f(m_run[mt] - m_new);
        m_run[mt] = m_new;
        float sum = 0.f;
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) {
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const float p = __builtin_amdgcn_exp2f(st[nt][mt][r] - m_new);
            st[nt][mt][r] = p;
            sum += p;
          }
        }
        l_part[mt] = l_part[mt] * alpha + sum;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
#pragma unroll
          for (int r = 0; r < 16; ++r) acc_o[dt][mt][r] *= alpha;
      }
      // O^T += V^T P^T: 2 key tiles x 2 steps of 16 keys.
#pragma unroll
      for (int nt = 0; nt < 2; ++nt) {
#pragma unroll
        for (int g = 0; g < 2; ++g) {
          const Frag p0 = acc_frag<T>(st[nt][0], g);
          const Frag p1 = acc_frag<T>(st[nt][1], g);
#pragma unroll
          for (int dt = 0; dt < DT; ++dt) {
            const Frag vf = trans_frag<T>(vl, dt * 32 + l32, nt * 4 + g * 2 + hi);
            acc_o[dt][0] = Mma<T>::run(vf, p0, acc_o[dt][0]);
            acc_o[dt][1] = Mma<T>::run(vf, p1, acc_o[dt][1]);
          }
        }
      }
    }
    if (more) {
      kst.store(k_lds[buf ^ 1]);
      vst.store(v_lds[buf ^ 1]);
    }
    __syncthreads();
  }

  // Epilogue: O = O^T / l, written as 4 consecutive features per store.
#pragma unroll
  for (int mt = 0; mt < 2; ++mt) {
    const float l = l_part[mt] + __shfl_xor(l_part[mt], 32);
    const float inv = 1.0f / l;
    const int query = wq0 + mt * 32 + l32;
    if (query < N) {
      T* orow = Oh + query * s.o[2];
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
#pragma unroll
        for (int g4 = 0; g4 < 4; ++g4) {
          const int d = dt * 32 + g4 * 8 + hi * 4;
          uint2 u;
          u.x = pack2<T>(acc_o[dt][mt][g4 * 4 + 0] * inv, acc_o[dt][mt][g4 * 4 + 1] * inv);
          u.y = pack2<T>(acc_o[dt][mt][g4 * 4 + 2] * inv, acc_o[dt][mt][g4 * 4 + 3] * inv);
          *reinterpret_cast<uint2*>(orow + d) = u;
        }
      }
      if (lse != nullptr && hi == 0) lse[static_cast<int64_t>(bh) * N + query] = m_run[mt] + __log2f(l);
    }
  }
}

// ---------------------------------------------------------------- backward: delta

// delta[row] = sum_d O[row][d] * dO[row][d]; D/8 lanes per row, 16 bytes each. A workgroup
// takes kPreUnroll passes of kThreads / (D/8) consecutive rows; each thread loads its pieces
// of kPreUnroll rows before any arithmetic, and the row -> (batch, head, position) split is
// a multiply-shift division (one row per thread with 64-bit divisions: B4 H32 N8192 D128
// in 93.6 instead of 89.4 us). O and dO are read once, non-temporally (B4 H32 N8192 D128
// 89.5 -> 82.3 us, D64 48.9 -> 43.4 us); eight rows per thread instead of four ran 97 us.
constexpr int kPreUnroll = 4;

template <typename T, int D>
__global__ __launch_bounds__(kThreads) void attn_bwd_preprocess_kernel(
    const T* __restrict__ O, const T* __restrict__ dO, float* __restrict__ delta,
    tk::FastDiv seq_div, tk::FastDiv head_div, int64_t sb, int64_t sh, int64_t sn, int rows) {
  constexpr int LPR = D / 8;            // lanes per row
  constexpr int RPP = kThreads / LPR;   // rows per pass
  const int part = threadIdx.x % LPR;
  const int r0 = blockIdx.x * (RPP * kPreUnroll) + threadIdx.x / LPR;
  float o[kPreUnroll][8], g[kPreUnroll][8];
#pragma unroll
  for (int u = 0; u < kPreUnroll; ++u) {
    const int row = r0 + u * RPP;
    if (row < rows) {
      const int bh = static_cast<int>(seq_div.div(static_cast<uint32_t>(row)));
      const int i = row - bh * static_cast<int>(seq_div.d);
      const int b = static_cast<int>(head_div.div(static_cast<uint32_t>(bh)));
      const int h = bh - b * static_cast<int>(head_div.d);
      const int64_t off = b * sb + h * sh + i * sn + part * 8;
      tk::load_vec_stream<T, 8>(O + off, o[u]);
      tk::load_vec_stream<T, 8>(dO + off, g[u]);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) o[u][e] = g[u][e] = 0.f;
    }
  }
#pragma unroll
  for (int u = 0; u < kPreUnroll; ++u) {
    float acc = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) acc += o[u][e] * g[u][e];
#pragma unroll
    for (int w = LPR / 2; w >= 1; w >>= 1) acc += __shfl_xor(acc, w);
    const int row = r0 + u * RPP;
    if (row < rows && part == 0) delta[row] = acc;
  }
}

// ---------------------------------------------------------------- backward: dQ
//
// Workgroup: 128 queries (4 waves x 32); key blocks of 64.
// Per wave and key block: S^T = K Q^T and dP^T = V dO^T (2 key tiles each),
// P^T = exp2(S^T*c - lse), dS^T = P^T (dP^T - delta), dQ^T += K^T dS^T.

template <typename T, int D, bool CAUSAL>
__global__ __attribute__((amdgpu_flat_work_group_size(kThreads, kThreads),
                          amdgpu_waves_per_eu(1, 2))) void
attn_bwd_dq_kernel(const T* __restrict__ Q, const T* __restrict__ K, const T* __restrict__ V,
                   const T* __restrict__ dO, T* __restrict__ dQ, const float* __restrict__ lse,
                   const float* __restrict__ delta, Shape s) {
  using Frag = typename Mma<T>::Frag;
  constexpr int BM = 128, BN = 64, DT = D / 32, KS = D / 16;
  __shared__ __attribute__((aligned(16))) uint16_t k_lds[2][64 * D];
  __shared__ __attribute__((aligned(16))) uint16_t kt_lds[2][64 * D];
  __shared__ __attribute__((aligned(16))) uint16_t v_lds[2][64 * D];

  int bh, qb;
  tile_of<CAUSAL>(s, bh, qb);
  const int b = bh / s.heads, h = bh % s.heads;
  const int64_t base = b * s.q[0] + h * s.q[1];  // one stride set for all tensors
  const T* Qh = Q + base;
  const T* Kh = K + base;
  const T* Vh = V + base;
  const T* dOh = dO + base;
  T* dQh = dQ + base;
  const int64_t sn = s.q[2];
  const int N = s.seq;

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int l32 = lane & 31, hi = lane >> 5;
  const int q0 = qb * BM;
  const int query = q0 + wave * 32 + l32;
  const int wq0 = q0 + wave * 32;

  Frag qf[KS], df[KS];
#pragma unroll
  for (int kk = 0; kk < KS; ++kk) {
    qf[kk] = global_frag<T>(Qh, sn, query, N, kk * 16 + hi * 8);
    df[kk] = global_frag<T>(dOh, sn, query, N, kk * 16 + hi * 8);
  }
  const float lse_q = query < N ? lse[static_cast<int64_t>(bh) * N + query] : 0.f;
  const float delta_q = query < N ? delta[static_cast<int64_t>(bh) * N + query] : 0.f;

  f32x16 acc_dq[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) acc_dq[dt] = zero16();

  const int kv_end = CAUSAL ? min(N, q0 + BM) : N;
  const int kv_blocks = (kv_end + BN - 1) / BN;

  RowTile<D> kst, vst;
  TransTile<D> ktst;
  kst.load(Kh, sn, 0, N);
  ktst.load(Kh, sn, 0, N);
  vst.load(Vh, sn, 0, N);
  kst.store(k_lds[0]);
  ktst.store(kt_lds[0]);
  vst.store(v_lds[0]);
  __syncthreads();

  for (int j = 0; j < kv_blocks; ++j) {
    const int buf = j & 1;
    const int n0 = j * BN;
    const bool more = j + 1 < kv_blocks;
    if (more) {
      kst.load(Kh, sn, n0 + BN, N);
      ktst.load(Kh, sn, n0 + BN, N);
      vst.load(Vh, sn, n0 + BN, N);
    }
    const bool active = !CAUSAL || n0 <= wq0 + 31;
    if (active) {
      f32x16 st[2], dp[2];
      st[0] = st[1] = dp[0] = dp[1] = zero16();
#pragma unroll
      for (int kk = 0; kk < KS; ++kk) {
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) {
          st[nt] = Mma<T>::run(row_frag<T, D>(k_lds[buf], nt * 32 + l32, kk * 2 + hi), qf[kk], st[nt]);
          dp[nt] = Mma<T>::run(row_frag<T, D>(v_lds[buf], nt * 32 + l32, kk * 2 + hi), df[kk], dp[nt]);
        }
      }
#pragma unroll
      for (int nt = 0; nt < 2; ++nt) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int key = n0 + nt * 32 + acc_row(r, lane);
          float p = __builtin_amdgcn_exp2f(st[nt][r] * s.scale_log2 - lse_q);
          if (key >= N || query >= N || (CAUSAL && key > query)) p = 0.f;
          st[nt][r] = p * (dp[nt][r] - delta_q);  // dS^T
        }
      }
#pragma unroll
      for (int nt = 0; nt < 2; ++nt) {
#pragma unroll
        for (int g = 0; g < 2; ++g) {
          const Frag dsf = acc_frag<T>(st[nt], g);
#pragma unroll
          for (int dt = 0; dt < DT; ++dt)
            acc_dq[dt] = Mma<T>::run(trans_frag<T>(kt_lds[buf], dt * 32 + l32, nt * 4 + g * 2 + hi),
                                     dsf, acc_dq[dt]);
        }
      }
    }
    if (more) {
      kst.store(k_lds[buf ^ 1]);
      ktst.store(kt_lds[buf ^ 1]);
      vst.store(v_lds[buf ^ 1]);
    }
    __syncthreads();
  }

  if (query < N) {
    T* row = dQh + query * sn;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
#pragma unroll
      for (int g4 = 0; g4 < 4; ++g4) {
        const int d = dt * 32 + g4 * 8 + hi * 4;
        uint2 u;
        u.x = pack2<T>(acc_dq[dt][g4 * 4 + 0] * s.scale, acc_dq[dt][g4 * 4 + 1] * s.scale);
        u.y = pack2<T>(acc_dq[dt][g4 * 4 + 2] * s.scale, acc_dq[dt][g4 * 4 + 3] * s.scale);
        *reinterpret_cast<uint2*>(row + d) = u;
      }
    }
  }
}

// ---------------------------------------------------------------- backward: dK, dV
//
// Workgroup: 128 keys (4 waves x 32); query blocks of 64.
// Per wave and query block: S = Q K^T and dP = dO V^T (2 query tiles each;
// an accumulator lane owns one key), P = exp2(S*c - lse), dS = P (dP - delta),
// dV^T-tiles += P^T dO and dK-tiles += dS^T Q with dO and Q staged transposed.
// Accumulators dV[dt], dK[dt] hold D[key row][feature column].

template <typename T, int D, bool CAUSAL>
__global__ __attribute__((amdgpu_flat_work_group_size(kThreads, kThreads),
                          amdgpu_waves_per_eu(1, 1))) void
attn_bwd_dkdv_kernel(const T* __restrict__ Q, const T* __restrict__ K, const T* __restrict__ V,
                     const T* __restrict__ dO, T* __restrict__ dK, T* __restrict__ dV,
                     const float* __restrict__ lse, const float* __restrict__ delta, Shape s) {
  using Frag = typename Mma<T>::Frag;
  constexpr int BNK = 128, BMQ = 64, DT = D / 32, KS = D / 16;
  __shared__ __attribute__((aligned(16))) uint16_t q_lds[2][64 * D];
  __shared__ __attribute__((aligned(16))) uint16_t qt_lds[2][64 * D];
  __shared__ __attribute__((aligned(16))) uint16_t do_lds[2][64 * D];
  __shared__ __attribute__((aligned(16))) uint16_t dot_lds[2][64 * D];
  __shared__ float stat_lds[2][2][64];  // [buf][lse | delta][query]

  int bh, kb;
  {
    int w = blockIdx.x;
    if (s.tiles % 8 == 0) w = (w % 8) * (s.tiles / 8) + w / 8;
    bh = w / s.q_blocks;  // q_blocks holds the number of key blocks here
    kb = w % s.q_blocks;
  }
  const int b = bh / s.heads, h = bh % s.heads;
  const int64_t base = b * s.q[0] + h * s.q[1];
  const T* Qh = Q + base;
  const T* Kh = K + base;
  const T* Vh = V + base;
  const T* dOh = dO + base;
  const int64_t sn = s.q[2];
  const int N = s.seq;
  const float* lse_h = lse + static_cast<int64_t>(bh) * N;
  const float* delta_h = delta + static_cast<int64_t>(bh) * N;

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int l32 = lane & 31, hi = lane >> 5;
  const int k0 = kb * BNK;
  const int key = k0 + wave * 32 + l32;
  const int wk0 = k0 + wave * 32;

  Frag kf[KS], vf[KS];
#pragma unroll
  for (int kk = 0; kk < KS; ++kk) {
    kf[kk] = global_frag<T>(Kh, sn, key, N, kk * 16 + hi * 8);
    vf[kk] = global_frag<T>(Vh, sn, key, N, kk * 16 + hi * 8);
  }
  f32x16 acc_dk[DT], acc_dv[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) acc_dk[dt] = acc_dv[dt] = zero16();

  const int q_first = CAUSAL ? (k0 / BMQ) : 0;
  const int q_blocks = (N + BMQ - 1) / BMQ;

  RowTile<D> qst, dost;
  TransTile<D> qtst, dotst;
  float stat = 0.f;
  auto stage = [&](int qblk) {
    const int m0 = qblk * BMQ;
    qst.load(Qh, sn, m0, N);
    qtst.load(Qh, sn, m0, N);
    dost.load(dOh, sn, m0, N);
    dotst.load(dOh, sn, m0, N);
    if (threadIdx.x < 128) {
      const int i = m0 + (threadIdx.x & 63);
      const float* src = threadIdx.x < 64 ? lse_h : delta_h;
      stat = i < N ? src[i] : 0.f;
    }
  };
  auto commit = [&](int buf) {
    qst.store(q_lds[buf]);
    qtst.store(qt_lds[buf]);
    dost.store(do_lds[buf]);
    dotst.store(dot_lds[buf]);
    if (threadIdx.x < 128) stat_lds[buf][threadIdx.x >> 6][threadIdx.x & 63] = stat;
  };

  if (q_first < q_blocks) {
    stage(q_first);
    commit(0);
  }
  __syncthreads();

  for (int qi = q_first; qi < q_blocks; ++qi) {
    const int buf = (qi - q_first) & 1;
    const int m0 = qi * BMQ;
    const bool more = qi + 1 < q_blocks;
    if (more) stage(qi + 1);
    const bool active = !CAUSAL || m0 + BMQ - 1 >= wk0;
    if (active) {
      f32x16 sc[2], dp[2];
      sc[0] = sc[1] = dp[0] = dp[1] = zero16();
#pragma unroll
      for (int kk = 0; kk < KS; ++kk) {
#pragma unroll
        for (int mt = 0; mt < 2; ++mt) {
          sc[mt] = Mma<T>::run(row_frag<T, D>(q_lds[buf], mt * 32 + l32, kk * 2 + hi), kf[kk], sc[mt]);
          dp[mt] = Mma<T>::run(row_frag<T, D>(do_lds[buf], mt * 32 + l32, kk * 2 + hi), vf[kk], dp[mt]);
        }
      }
      // S = Q K^T: rows are queries, the lane's column is `key`.
#pragma unroll
      for (int mt = 0; mt < 2; ++mt) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int ql = mt * 32 + acc_row(r, lane);
          const int q = m0 + ql;
          float p = __builtin_amdgcn_exp2f(sc[mt][r] * s.scale_log2 - stat_lds[buf][0][ql]);
          if (q >= N || key >= N || (CAUSAL && key > q)) p = 0.f;
          sc[mt][r] = p;
          dp[mt][r] = p * (dp[mt][r] - stat_lds[buf][1][ql]);
        }
      }
      // dV[key][d] += sum_q P[q][key] dO[q][d];  dK[key][d] += sum_q dS[q][key] Q[q][d].
#pragma unroll
      for (int mt = 0; mt < 2; ++mt) {
#pragma unroll
        for (int g = 0; g < 2; ++g) {
          const Frag pf = acc_frag<T>(sc[mt], g);
          const Frag dsf = acc_frag<T>(dp[mt], g);
#pragma unroll
          for (int dt = 0; dt < DT; ++dt) {
            const int chunk = mt * 4 + g * 2 + hi;
            acc_dv[dt] = Mma<T>::run(pf, trans_frag<T>(dot_lds[buf], dt * 32 + l32, chunk), acc_dv[dt]);
            acc_dk[dt] = Mma<T>::run(dsf, trans_frag<T>(qt_lds[buf], dt * 32 + l32, chunk), acc_dk[dt]);
          }
        }
      }
    }
    if (more) commit(buf ^ 1);
    __syncthreads();
  }

  // Accumulator [key row][feature column]: lane l holds feature dt*32 + l%32
  // for keys wk0 + acc_row(r, l).
  T* dKh = dK + base;
  T* dVh = dV + base;
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) {
    const int d = dt * 32 + l32;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int kr = wk0 + acc_row(r, lane);
      if (kr < N) {
        dKh[kr * sn + d] = tk::from_f32<T>(acc_dk[dt][r] * s.scale);
        dVh[kr * sn + d] = tk::from_f32<T>(acc_dv[dt][r]);
      }
    }
  }
}

// ---------------------------------------------------------------- host side

int check_common(const char* what, int dtype, int64_t batch, int64_t heads, int64_t seq,
                 int64_t head_dim) {
  if (dtype != TK_DTYPE_F16 && dtype != TK_DTYPE_BF16)
    return tk::fail("%s: dtype must be float16 or bfloat16", what);
  if (head_dim != 64 && head_dim != 128) return tk::fail("%s: head_dim must be 64 or 128", what);
  if (batch <= 0 || heads <= 0 || seq <= 0) return tk::fail("%s: empty problem", what);
  if (batch * heads > INT32_MAX / 2 || seq > INT32_MAX / 2)
    return tk::fail("%s: problem too large", what);
  return 0;
}

bool strides_ok(const int64_t* st, int64_t batch, int64_t heads, int64_t seq, int64_t d) {
  for (int i = 0; i < 3; ++i)
    if (st[i] <= 0 || st[i] % 8 != 0) return false;
  // 128-bit sum: no stride or size makes it wrap.
  return tk::extent(batch, st[0], heads, st[1]) + tk::extent(seq, st[2], d, 1) <= INT32_MAX;
}

}  // namespace

#define TK_ATTN_DISPATCH(dtype, head_dim, causal, KERNEL, grid, ...)                    \
  do {                                                                                  \
    hipStream_t st_ = tk::as_stream(stream);                                            \
    if (dtype == TK_DTYPE_F16) {                                                        \
      using T = _Float16;                                                               \
      if (head_dim == 64) {                                                             \
        if (causal) hipLaunchKernelGGL((KERNEL<T, 64, true>), grid, dim3(kThreads), 0, st_, __VA_ARGS__); \
        else hipLaunchKernelGGL((KERNEL<T, 64, false>), grid, dim3(kThreads), 0, st_, __VA_ARGS__);      \
      } else {                                                                          \
        if (causal) hipLaunchKernelGGL((KERNEL<T, 128, true>), grid, dim3(kThreads), 0, st_, __VA_ARGS__); \
        else hipLaunchKernelGGL((KERNEL<T, 128, false>), grid, dim3(kThreads), 0, st_, __VA_ARGS__);      \
      }                                                                                 \
    } else {                                                                            \
      using T = __bf16;                                                                 \
      if (head_dim == 64) {                                                             \
        if (causal) hipLaunchKernelGGL((KERNEL<T, 64, true>), grid, dim3(kThreads), 0, st_, __VA_ARGS__); \
        else hipLaunchKernelGGL((KERNEL<T, 64, false>), grid, dim3(kThreads), 0, st_, __VA_ARGS__);      \
      } else {                                                                          \
        if (causal) hipLaunchKernelGGL((KERNEL<T, 128, true>), grid, dim3(kThreads), 0, st_, __VA_ARGS__); \
        else hipLaunchKernelGGL((KERNEL<T, 128, false>), grid, dim3(kThreads), 0, st_, __VA_ARGS__);      \
      }                                                                                 \
    }                                                                                   \
  } while (0)

extern "C" int tk_attn_fwd(int dtype, const void* q, const void* k, const void* v, void* o,
                           float* lse, int64_t batch, int64_t heads, int64_t seq,
                           int64_t head_dim, const int64_t* q_strides, const int64_t* k_strides,
                           const int64_t* v_strides, const int64_t* o_strides, float sm_scale,
                           int causal, void* stream) {
  if (check_common("attn_fwd", dtype, batch, heads, seq, head_dim)) return 1;
  if (!q || !k || !v || !o || !q_strides || !k_strides || !v_strides || !o_strides)
    return tk::fail("attn_fwd: null pointer");
  if (!strides_ok(q_strides, batch, heads, seq, head_dim) ||
      !strides_ok(k_strides, batch, heads, seq, head_dim) ||
      !strides_ok(v_strides, batch, heads, seq, head_dim) ||
      !strides_ok(o_strides, batch, heads, seq, head_dim))
    return tk::fail("attn_fwd: strides must be positive multiples of 8 within int32 range");
  if (!tk::aligned16(q) || !tk::aligned16(k) || !tk::aligned16(v) || !tk::aligned16(o))
    return tk::fail("attn_fwd: tensors must be 16-byte aligned");
  if (tk::attn_fwd_dma_applies(seq, head_dim, k_strides, v_strides)) {
    tk::attn_fwd_dma_launch(dtype, q, k, v, o, lse, batch, heads, heads, seq, head_dim,
                            q_strides, k_strides, v_strides, o_strides, sm_scale, causal != 0,
                            tk::as_stream(stream));
    return tk::check_launch("attn_fwd");
  }
  Shape s{};
  s.heads = (int)heads;
  s.seq = (int)seq;
  for (int i = 0; i < 3; ++i) {
    s.q[i] = q_strides[i];
    s.k[i] = k_strides[i];
    s.v[i] = v_strides[i];
    s.o[i] = o_strides[i];
  }
  s.scale = sm_scale;
  s.scale_log2 = sm_scale * 1.4426950408889634f;
  s.q_blocks = (int)tk::cdiv(seq, 256);
  s.tiles = (int)(s.q_blocks * batch * heads);
  const dim3 grid(static_cast<unsigned>(s.tiles));
  TK_ATTN_DISPATCH(dtype, head_dim, causal, attn_fwd_kernel, grid, static_cast<const T*>(q),
                   static_cast<const T*>(k), static_cast<const T*>(v), static_cast<T*>(o), lse, s);
  return tk::check_launch("attn_fwd");
}

extern "C" int tk_attn_bwd_preprocess(int dtype, const void* o, const void* dout, float* delta,
                                      int64_t batch, int64_t heads, int64_t seq,
                                      int64_t head_dim, const int64_t* strides, void* stream) {
  if (check_common("attn_bwd_preprocess", dtype, batch, heads, seq, head_dim)) return 1;
  if (!o || !dout || !delta || !strides) return tk::fail("attn_bwd_preprocess: null pointer");
  if (!strides_ok(strides, batch, heads, seq, head_dim))
    return tk::fail("attn_bwd_preprocess: strides must be positive multiples of 8 within int32 "
                    "range");
  if (!tk::aligned16(o) || !tk::aligned16(dout))
    return tk::fail("attn_bwd_preprocess: tensors must be 16-byte aligned");
  const int64_t rows = batch * heads * seq;
  if (rows > INT32_MAX / 2) return tk::fail("attn_bwd_preprocess: too many rows");
  const int64_t rows_per_block = kThreads / (head_dim / 8) * kPreUnroll;
  const int64_t blocks = tk::cdiv(rows, rows_per_block);
  const tk::FastDiv seq_div(static_cast<uint32_t>(seq)), head_div(static_cast<uint32_t>(heads));
  hipStream_t st = tk::as_stream(stream);
  if (dtype == TK_DTYPE_F16) {
    using T = _Float16;
    if (head_dim == 64)
      hipLaunchKernelGGL((attn_bwd_preprocess_kernel<T, 64>), dim3(blocks), dim3(kThreads), 0, st,
                         (const T*)o, (const T*)dout, delta, seq_div, head_div, strides[0],
                         strides[1], strides[2], (int)rows);
    else
      hipLaunchKernelGGL((attn_bwd_preprocess_kernel<T, 128>), dim3(blocks), dim3(kThreads), 0, st,
                         (const T*)o, (const T*)dout, delta, seq_div, head_div, strides[0],
                         strides[1], strides[2], (int)rows);
  } else {
    using T = __bf16;
    if (head_dim == 64)
      hipLaunchKernelGGL((attn_bwd_preprocess_kernel<T, 64>), dim3(blocks), dim3(kThreads), 0, st,
                         (const T*)o, (const T*)dout, delta, seq_div, head_div, strides[0],
                         strides[1], strides[2], (int)rows);
    else
      hipLaunchKernelGGL((attn_bwd_preprocess_kernel<T, 128>), dim3(blocks), dim3(kThreads), 0, st,
                         (const T*)o, (const T*)dout, delta, seq_div, head_div, strides[0],
                         strides[1], strides[2], (int)rows);
  }
  return tk::check_launch("attn_bwd_preprocess");
}

namespace {
int bwd_shape(const char* what, int dtype, const void* const* ptrs, int nptr, int64_t batch,
              int64_t heads, int64_t seq, int64_t head_dim, const int64_t* strides, float sm_scale,
              int rows_per_block, Shape* s) {
  if (check_common(what, dtype, batch, heads, seq, head_dim)) return 1;
  if (!strides) return tk::fail("%s: null pointer", what);
  for (int i = 0; i < nptr; ++i) {
    if (!ptrs[i]) return tk::fail("%s: null pointer", what);
    if (!tk::aligned16(ptrs[i])) return tk::fail("%s: tensors must be 16-byte aligned", what);
  }
  if (!strides_ok(strides, batch, heads, seq, head_dim))
    return tk::fail("%s: strides must be positive multiples of 8 within int32 range", what);
  *s = Shape{};
  s->heads = (int)heads;
  s->seq = (int)seq;
  for (int i = 0; i < 3; ++i) s->q[i] = s->k[i] = s->v[i] = s->o[i] = strides[i];
  s->scale = sm_scale;
  s->scale_log2 = sm_scale * 1.4426950408889634f;
  s->q_blocks = (int)tk::cdiv(seq, rows_per_block);
  s->tiles = (int)(s->q_blocks * batch * heads);
  return 0;
}
}  // namespace

extern "C" int tk_attn_bwd_dkdv(int dtype, const void* q, const void* k, const void* v,
                                const void* dout, void* dk, void* dv, const float* lse,
                                const float* delta, int64_t batch, int64_t heads, int64_t seq,
                                int64_t head_dim, const int64_t* strides, float sm_scale,
                                int causal, void* stream) {
  const void* ptrs[] = {q, k, v, dout, dk, dv, lse, delta};
  Shape s;
  if (bwd_shape("attn_bwd_dkdv", dtype, ptrs, 8, batch, heads, seq, head_dim, strides, sm_scale,
                128, &s))
    return 1;
  if (tk::attn_bwd_dma_applies(seq, head_dim, strides, strides)) {
    tk::attn_bwd_dkdv_dma_launch(dtype, q, k, v, dout, dk, dv, lse, delta, batch, heads, heads,
                                 seq, head_dim, strides, strides, sm_scale, causal != 0,
                                 tk::as_stream(stream));
    return tk::check_launch("attn_bwd_dkdv");
  }
  const dim3 grid(static_cast<unsigned>(s.tiles));
  TK_ATTN_DISPATCH(dtype, head_dim, causal, attn_bwd_dkdv_kernel, grid, (const T*)q, (const T*)k,
                   (const T*)v, (const T*)dout, (T*)dk, (T*)dv, lse, delta, s);
  return tk::check_launch("attn_bwd_dkdv");
}

extern "C" int tk_attn_bwd_dq(int dtype, const void* q, const void* k, const void* v,
                              const void* dout, void* dq, const float* lse, const float* delta,
                              int64_t batch, int64_t heads, int64_t seq, int64_t head_dim,
                              const int64_t* strides, float sm_scale, int causal, void* stream) {
  const void* ptrs[] = {q, k, v, dout, dq, lse, delta};
  Shape s;
  if (bwd_shape("attn_bwd_dq", dtype, ptrs, 7, batch, heads, seq, head_dim, strides, sm_scale, 128,
                &s))
    return 1;
  if (tk::attn_bwd_dma_applies(seq, head_dim, strides, strides)) {
    tk::attn_bwd_dq_dma_launch(dtype, q, k, v, dout, dq, lse, delta, batch, heads, heads, seq,
                               head_dim, strides, strides, sm_scale, causal != 0,
                               tk::as_stream(stream));
    return tk::check_launch("attn_bwd_dq");
  }
  const dim3 grid(static_cast<unsigned>(s.tiles));
  TK_ATTN_DISPATCH(dtype, head_dim, causal, attn_bwd_dq_kernel, grid, (const T*)q, (const T*)k,
                   (const T*)v, (const T*)dout, (T*)dq, lse, delta, s);
  return tk::check_launch("attn_bwd_dq");
}

// ---------------------------------------------------------------- grouped-query attention
//
// Query head h attends with K/V head h / (heads / kv_heads). Same kernels as the
// multi-head entry points (which are the kv_heads == heads case); the dK/dV pass sums a
// KV head's query heads in a fixed order, so the backward stays deterministic. Needs the
// buffer->LDS kernels (each head's rows below 2 GiB).

namespace {
int gqa_check(const char* what, int dtype, const void* const* ptrs, int nptr, int64_t batch,
              int64_t heads, int64_t kv_heads, int64_t seq, int64_t head_dim,
              const int64_t* const* strides, const bool* kv_side, int nstr) {
  if (check_common(what, dtype, batch, heads, seq, head_dim)) return 1;
  if (kv_heads <= 0 || heads % kv_heads != 0)
    return tk::fail("%s: heads must be a positive multiple of kv_heads", what);
  for (int i = 0; i < nptr; ++i) {
    if (!ptrs[i]) return tk::fail("%s: null pointer", what);
    if (!tk::aligned16(ptrs[i])) return tk::fail("%s: tensors must be 16-byte aligned", what);
  }
  for (int i = 0; i < nstr; ++i) {
    if (!strides[i]) return tk::fail("%s: null pointer", what);
    if (!strides_ok(strides[i], batch, kv_side[i] ? kv_heads : heads, seq, head_dim))
      return tk::fail("%s: strides must be positive multiples of 8 within int32 range", what);
  }
  return 0;
}
}  // namespace

extern "C" int tk_attn_fwd_gqa(int dtype, const void* q, const void* k, const void* v, void* o,
                               float* lse, int64_t batch, int64_t heads, int64_t kv_heads,
                               int64_t seq, int64_t head_dim, const int64_t* q_strides,
                               const int64_t* k_strides, const int64_t* v_strides,
                               const int64_t* o_strides, float sm_scale, int causal,
                               void* stream) {
  const void* ptrs[] = {q, k, v, o};
  const int64_t* st[] = {q_strides, k_strides, v_strides, o_strides};
  const bool kv[] = {false, true, true, false};
  if (gqa_check("attn_fwd_gqa", dtype, ptrs, 4, batch, heads, kv_heads, seq, head_dim, st, kv, 4))
    return 1;
  if (!tk::attn_fwd_dma_applies(seq, head_dim, k_strides, v_strides))
    return tk::fail("attn_fwd_gqa: each head's rows must span less than 2 GiB");
  tk::attn_fwd_dma_launch(dtype, q, k, v, o, lse, batch, heads, kv_heads, seq, head_dim,
                          q_strides, k_strides, v_strides, o_strides, sm_scale, causal != 0,
                          tk::as_stream(stream));
  return tk::check_launch("attn_fwd_gqa");
}

extern "C" int tk_attn_fwd_rope(int dtype, const void* q, const void* k, const void* v, void* o,
                                float* lse, const void* rope_cos, const void* rope_sin,
                                int64_t table_rows, int64_t table_row_stride, void* k_rot,
                                int64_t batch, int64_t heads, int64_t kv_heads, int64_t seq,
                                int64_t head_dim, const int64_t* q_strides,
                                const int64_t* k_strides, const int64_t* v_strides,
                                const int64_t* o_strides, float sm_scale, int causal,
                                void* stream) {
  const void* ptrs[] = {q, k, v, o, rope_cos, rope_sin, k_rot};
  const int64_t* st[] = {q_strides, k_strides, v_strides, o_strides};
  const bool kv[] = {false, true, true, false};
  if (gqa_check("attn_fwd_rope", dtype, ptrs, 7, batch, heads, kv_heads, seq, head_dim, st, kv, 4))
    return 1;
  if (table_rows < seq) return tk::fail("attn_fwd_rope: the tables need a row per position");
  if (table_row_stride < head_dim / 2 || table_row_stride > INT32_MAX ||
      (table_row_stride * 2) % 16 != 0 || !tk::aligned16(rope_cos) || !tk::aligned16(rope_sin))
    return tk::fail("attn_fwd_rope: table rows must be 16-byte aligned, strides below 2^31");
  if (k_strides[1] != seq * k_strides[2] || k_strides[0] != kv_heads * k_strides[1])
    return tk::fail("attn_fwd_rope: K must be [batch][kv_heads][seq] rows of one row stride");
  // K is rotated once into the workspace: every query block re-reads each K block, so a
  // rotation inside the attention loop would be repeated once per query block.
  const int64_t rot_strides[3] = {kv_heads * seq * head_dim, seq * head_dim, head_dim};
  if (!tk::attn_fwd_dma_applies(seq, head_dim, rot_strides, v_strides))
    return tk::fail("attn_fwd_rope: each head's rows must span less than 2 GiB");
  if (tk_rope_positions(dtype, k, rope_cos, rope_sin, k_rot, batch * kv_heads * seq, seq,
                        head_dim / 2, k_strides[2], table_row_stride, head_dim, 0, stream))
    return 1;
  tk::attn_fwd_dma_launch(dtype, q, k_rot, v, o, lse, batch, heads, kv_heads, seq, head_dim,
                          q_strides, rot_strides, v_strides, o_strides, sm_scale, causal != 0,
                          tk::as_stream(stream), nullptr, 0, rope_cos, rope_sin,
                          table_row_stride);
  return tk::check_launch("attn_fwd_rope");
}

extern "C" int tk_attn_bwd_dkdv_gqa(int dtype, const void* q, const void* k, const void* v,
                                    const void* dout, void* dk, void* dv, const float* lse,
                                    const float* delta, int64_t batch, int64_t heads,
                                    int64_t kv_heads, int64_t seq, int64_t head_dim,
                                    const int64_t* q_strides, const int64_t* kv_strides,
                                    float sm_scale, int causal, void* stream) {
  const void* ptrs[] = {q, k, v, dout, dk, dv, lse, delta};
  const int64_t* st[] = {q_strides, kv_strides};
  const bool kv[] = {false, true};
  if (gqa_check("attn_bwd_dkdv_gqa", dtype, ptrs, 8, batch, heads, kv_heads, seq, head_dim, st,
                kv, 2))
    return 1;
  if (!tk::attn_bwd_dma_applies(seq, head_dim, q_strides, kv_strides))
    return tk::fail("attn_bwd_dkdv_gqa: each head's rows must span less than 2 GiB");
  tk::attn_bwd_dkdv_dma_launch(dtype, q, k, v, dout, dk, dv, lse, delta, batch, heads, kv_heads,
                               seq, head_dim, q_strides, kv_strides, sm_scale, causal != 0,
                               tk::as_stream(stream));
  return tk::check_launch("attn_bwd_dkdv_gqa");
}

extern "C" int tk_attn_bwd_dq_gqa(int dtype, const void* q, const void* k, const void* v,
                                  const void* dout, void* dq, const float* lse,
                                  const float* delta, int64_t batch, int64_t heads,
                                  int64_t kv_heads, int64_t seq, int64_t head_dim,
                                  const int64_t* q_strides, const int64_t* kv_strides,
                                  float sm_scale, int causal, void* stream) {
  const void* ptrs[] = {q, k, v, dout, dq, lse, delta};
  const int64_t* st[] = {q_strides, kv_strides};
  const bool kv[] = {false, true};
  if (gqa_check("attn_bwd_dq_gqa", dtype, ptrs, 7, batch, heads, kv_heads, seq, head_dim, st, kv,
                2))
    return 1;
  if (!tk::attn_bwd_dma_applies(seq, head_dim, q_strides, kv_strides))
    return tk::fail("attn_bwd_dq_gqa: each head's rows must span less than 2 GiB");
  tk::attn_bwd_dq_dma_launch(dtype, q, k, v, dout, dq, lse, delta, batch, heads, kv_heads, seq,
                             head_dim, q_strides, kv_strides, sm_scale, causal != 0,
                             tk::as_stream(stream));
  return tk::check_launch("attn_bwd_dq_gqa");
}

// ---------------------------------------------------------------- variable-length batches
//
// Packed [total][heads][head_dim] tensors with int32 cu_seqlens[batch + 1]: sequence b is
// rows cu_seqlens[b] .. cu_seqlens[b+1]. Strides are {token, head} in elements. The kernels
// clamp every sequence into [0, total] and to max_seqlen, so a malformed lengths table
// cannot address memory outside the tensors. LSE and delta are float32 [heads][total]
// (tk_attn_bwd_preprocess with batch 1, seq total and strides {total * token, head, token}
// computes delta in that layout).

namespace {
int varlen_check(const char* what, int dtype, const void* const* ptrs, int nptr,
                 const int32_t* cu, int64_t batch, int64_t heads, int64_t kv_heads,
                 int64_t max_seqlen, int64_t total, int64_t head_dim,
                 const int64_t* const* strides, const bool* kv_side, int nstr) {
  if (check_common(what, dtype, batch, heads, max_seqlen, head_dim)) return 1;
  if (cu == nullptr) return tk::fail("%s: null pointer", what);
  if (kv_heads <= 0 || heads % kv_heads != 0)
    return tk::fail("%s: heads must be a positive multiple of kv_heads", what);
  if (total <= 0 || total > INT32_MAX || max_seqlen > total)
    return tk::fail("%s: total must be positive and at least max_seqlen", what);
  for (int i = 0; i < nptr; ++i) {
    if (!ptrs[i]) return tk::fail("%s: null pointer", what);
    if (!tk::aligned16(ptrs[i])) return tk::fail("%s: tensors must be 16-byte aligned", what);
  }
  for (int i = 0; i < nstr; ++i) {
    const int64_t* st = strides[i];
    if (!st) return tk::fail("%s: null pointer", what);
    const int64_t h = kv_side[i] ? kv_heads : heads;
    if (st[0] <= 0 || st[1] <= 0 || st[0] % 8 || st[1] % 8 ||
        tk::extent(total, st[0], h, st[1]) + head_dim - 1 > INT32_MAX)
      return tk::fail("%s: strides must be positive multiples of 8 within int32 range", what);
    // Each head's rows go through one 32-bit buffer range.
    if (((total - 1) * st[0] + head_dim) * 2 >= (int64_t(1) << 31))
      return tk::fail("%s: each head's rows must span less than 2 GiB", what);
  }
  return 0;
}

// {token, head} -> the kernels' {batch, head, sequence} strides (batch stride 0).
struct Strides3 {
  int64_t v[3];
};
Strides3 packed(const int64_t* st) { return {{0, st[1], st[0]}}; }
}  // namespace

extern "C" int tk_attn_fwd_varlen(int dtype, const void* q, const void* k, const void* v,
                                  void* o, float* lse, const int32_t* cu_seqlens, int64_t batch,
                                  int64_t heads, int64_t kv_heads, int64_t max_seqlen,
                                  int64_t total, int64_t head_dim, const int64_t* q_strides,
                                  const int64_t* kv_strides, const int64_t* o_strides,
                                  float sm_scale, int causal, void* stream) {
  const void* ptrs[] = {q, k, v, o};
  const int64_t* st[] = {q_strides, kv_strides, o_strides};
  const bool kv[] = {false, true, false};
  if (varlen_check("attn_fwd_varlen", dtype, ptrs, 4, cu_seqlens, batch, heads, kv_heads,
                   max_seqlen, total, head_dim, st, kv, 3))
    return 1;
  const Strides3 qs = packed(q_strides), ks = packed(kv_strides), os = packed(o_strides);
  tk::attn_fwd_dma_launch(dtype, q, k, v, o, lse, batch, heads, kv_heads, max_seqlen, head_dim,
                          qs.v, ks.v, ks.v, os.v, sm_scale, causal != 0, tk::as_stream(stream),
                          cu_seqlens, total);
  return tk::check_launch("attn_fwd_varlen");
}

extern "C" int tk_attn_bwd_dkdv_varlen(int dtype, const void* q, const void* k, const void* v,
                                       const void* dout, void* dk, void* dv, const float* lse,
                                       const float* delta, const int32_t* cu_seqlens,
                                       int64_t batch, int64_t heads, int64_t kv_heads,
                                       int64_t max_seqlen, int64_t total, int64_t head_dim,
                                       const int64_t* q_strides, const int64_t* kv_strides,
                                       float sm_scale, int causal, void* stream) {
  const void* ptrs[] = {q, k, v, dout, dk, dv, lse, delta};
  const int64_t* st[] = {q_strides, kv_strides};
  const bool kv[] = {false, true};
  if (varlen_check("attn_bwd_dkdv_varlen", dtype, ptrs, 8, cu_seqlens, batch, heads, kv_heads,
                   max_seqlen, total, head_dim, st, kv, 2))
    return 1;
  const Strides3 qs = packed(q_strides), ks = packed(kv_strides);
  tk::attn_bwd_dkdv_dma_launch(dtype, q, k, v, dout, dk, dv, lse, delta, batch, heads, kv_heads,
                               max_seqlen, head_dim, qs.v, ks.v, sm_scale, causal != 0,
                               tk::as_stream(stream), cu_seqlens, total);
  return tk::check_launch("attn_bwd_dkdv_varlen");
}

extern "C" int tk_attn_bwd_dq_varlen(int dtype, const void* q, const void* k, const void* v,
                                     const void* dout, void* dq, const float* lse,
                                     const float* delta, const int32_t* cu_seqlens,
                                     int64_t batch, int64_t heads, int64_t kv_heads,
                                     int64_t max_seqlen, int64_t total, int64_t head_dim,
                                     const int64_t* q_strides, const int64_t* kv_strides,
                                     float sm_scale, int causal, void* stream) {
  const void* ptrs[] = {q, k, v, dout, dq, lse, delta};
  const int64_t* st[] = {q_strides, kv_strides};
  const bool kv[] = {false, true};
  if (varlen_check("attn_bwd_dq_varlen", dtype, ptrs, 7, cu_seqlens, batch, heads, kv_heads,
                   max_seqlen, total, head_dim, st, kv, 2))
    return 1;
  const Strides3 qs = packed(q_strides), ks = packed(kv_strides);
  tk::attn_bwd_dq_dma_launch(dtype, q, k, v, dout, dq, lse, delta, batch, heads, kv_heads,
                             max_seqlen, head_dim, qs.v, ks.v, sm_scale, causal != 0,
                             tk::as_stream(stream), cu_seqlens, total);
  return tk::check_launch("attn_bwd_dq_varlen");
}

