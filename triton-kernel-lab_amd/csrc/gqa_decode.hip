// Grouped-query attention decode: one query token per sequence and head, a KV
// cache per KV head shared by G = q_heads / kv_heads query heads
// (kv_head(h) = h / G), variable context lengths per sequence.
//
// The reference has no such kernel; its research note fixes the workload and the
// mapping (docs/research/gqa_decode_model.md, "Canonical decode workload",
// "Semantic GQA mapping"), and the arithmetic is its attention forward applied to
// one query row (src/tklab/kernels/flash_attention.py:90-117, 248-264): scores
// scaled by scale*log2(e), p = exp2(s - m), P rounded to the storage dtype before
// the PV product, O = acc / l, base-2 LSE = m + log2(l).
//
// Split kernel: one wave per (batch, kv head, split of split_len keys), both
// products on MFMA (v_mfma_f32_16x16x32), so the VALU work per key does not grow
// with G and the kernel stays HBM-bound:
//   S^T (16 keys x 16 heads) = K (16 keys x 32 dims) . Q^T, Q^T held in registers with
//     heads >= G zero. Lane l then holds head l%16's scores for keys 4*(l/16)..+3 of
//     the tile; a head's row maximum is a max over the lane's values and lanes ^16, ^32.
//   O^T (16 dims x 16 heads) += V^T (16 dims x 32 keys) . P^T, P^T straight from the
//     score registers (two tiles give a lane 8 keys, the MFMA k-order), V^T read with
//     ds_read_b64_tr_b16.
//   K and V reach LDS by non-temporal buffer->LDS DMA into a ring of 32-key tiles (4
//     stages at head_dim 128, 8 at 64: 64 KiB, so two waves share a CU), 3 (7) tiles
//     ahead. Rows past the split's end lie outside the tile's buffer range and arrive as
//     zeros. Measured on one box (B32 Hq32 Hkv8 L8192 D128): the earlier kernel (tiles
//     loaded into registers one tile ahead, 4 waves per CU) 0.195-0.201 ms; this ring with
//     default-policy loads 0.193-0.200 ms at any depth from 1 to 3 tiles ahead (2-4 waves
//     per CU), also with tiles dealt cyclically over a head's waves; with non-temporal
//     loads 0.168-0.172 ms at every depth. The bound was the cache policy, not the bytes
//     in flight or the access order.
// Combine kernel: one workgroup per (batch, query head) folds the splits in a
// fixed order (independent of timing) and writes O and the LSE. With one split per
// (batch, KV head) the split wave writes O = o / l and the LSE itself and the combine is not
// launched.
#include "attention_dma.hpp"
#include "tk_common.hpp"

namespace {

constexpr int kWave = 64;
constexpr float kLog2e = 1.4426950408889634f;

struct DecodeShape {
  int batch, q_heads, kv_heads, max_len, split_len, splits;
  int64_t qb, qh, kb, kh, kl, vb, vh, vl, ob, oh;
  float scale_log2;
};

// Floats per (batch, head, split) partial row: D output sums, then m and l; the
// stride keeps every row 16-byte aligned.
template <int D>
constexpr int partial_stride() {
  return D + 4;
}

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef int i32x4v __attribute__((ext_vector_type(4)));
typedef float f32x4v __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8v __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8v __attribute__((ext_vector_type(8)));

template <typename T>
__device__ __forceinline__ f32x4v mma16(i32x4v a, i32x4v b, f32x4v c) {
  if constexpr (__is_same(T, __bf16))
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8v, a),
                                                   __builtin_bit_cast(bf16x8v, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8v, a),
                                                  __builtin_bit_cast(f16x8v, b), c, 0, 0, 0);
}

// Two floats rounded to T and packed (element 0 in the low half).
template <typename T>
__device__ __forceinline__ int pack2(float lo, float hi) {
  if constexpr (__is_same(T, __bf16)) {
    const uint32_t a = __builtin_bit_cast(uint16_t, static_cast<__bf16>(lo));
    const uint32_t b = __builtin_bit_cast(uint16_t, static_cast<__bf16>(hi));
    return static_cast<int>(a | (b << 16));
  } else {
    const uint32_t a = __builtin_bit_cast(uint16_t, tk::from_f32<_Float16>(lo));
    const uint32_t b = __builtin_bit_cast(uint16_t, tk::from_f32<_Float16>(hi));
    return static_cast<int>(a | (b << 16));
  }
}

__device__ __forceinline__ i32x4v load16(const void* p) {
  return *reinterpret_cast<const i32x4v*>(p);
}

constexpr int kTileKeys = 32;  // keys per iteration: two 16-key MFMA tiles
constexpr uint32_t kOob = 0x80000000u;  // past every buffer's range: reads as zero
// Cache policy of the K/V loads: non-temporal (`nt`). Each key is read once; with the
// default policy the same kernel streamed at 5.5 TB/s, non-temporal at 6.4 TB/s (B32 Hq32
// Hkv8 L8192 D128, same box).
constexpr int kNonTemporal = 2;

// LDS ring of the split kernel: NS stages, each a 32-key tile of K followed by the same
// keys of V, rows of D elements stored whole (DMA writes 1 KiB of contiguous LDS per
// instruction, so the layout is a swizzle, not padding).
template <int D>
struct Ring {
  static constexpr int RB = D * 2;             // bytes per row
  static constexpr int TILE = kTileKeys * RB;  // bytes per tensor tile
  static constexpr int STAGE = 2 * TILE;
  static constexpr int NS = D == 128 ? 4 : 8;  // 64 KiB
  static constexpr int IPT = TILE / 1024;      // DMA instructions per tensor tile
  static constexpr int RPI = 1024 / RB;        // rows per DMA instruction
  static constexpr int CPR = RB / 16;          // 16-byte chunks per row
  static constexpr int QTILE = 16 * RB;        // Q^T tile: 16 heads
  // vmcnt is 6 bits: at most 63 DMA instructions may be outstanding.
  static_assert((NS - 1) * 2 * IPT < 64, "ring deeper than the vmcnt counter");
  // K: 16-byte chunk c of row r at slot c ^ kswz(r). A ds_read_b128 phase (16 lanes)
  // takes one chunk of 16 consecutive rows, on 16 distinct bank groups.
  static __device__ __forceinline__ int kswz(int r) { return D == 128 ? (r & 15) : ((r >> 1) & 7); }
  // V: 32-byte granule g of row r at granule g ^ vswz(r). A transposed read phase (32
  // lanes) takes one granule of 8 consecutive rows, on 8 distinct granule positions.
  static __device__ __forceinline__ int vswz(int r) { return D == 128 ? (r & 7) : ((r >> 1) & 3); }
};

// A wave-uniform address, asserted to the compiler (each half through readfirstlane), so
// buffer descriptors built from it stay in scalar registers.
__device__ __forceinline__ void* uniform_ptr(const void* p) {
  const uint64_t a = reinterpret_cast<uintptr_t>(p);
  const uint32_t lo = __builtin_amdgcn_readfirstlane(uint32_t(a));
  const uint32_t hi = __builtin_amdgcn_readfirstlane(uint32_t(a >> 32));
  return reinterpret_cast<void*>((uint64_t(hi) << 32) | lo);
}

// DMA of the 32-key tile starting at key0 of K and V into ring stage `stage`. The buffer
// ranges end at the split's last key, so rows past it (and whole tiles past the end,
// issued to keep the wait counts static) read as zero without a memory access.
template <typename T, int D>
__device__ __forceinline__ void ring_dma(char* ring, const T* kbase, const T* vbase,
                                         int64_t kl, int64_t vl, int key0, int k1, int stage,
                                         const uint32_t* koff, const uint32_t* voff) {
  using R = Ring<D>;
  const int rows = min(max(k1 - key0, 0), kTileKeys);
  const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc(
      uniform_ptr(kbase + int64_t(key0) * kl), (short)0,
      __builtin_amdgcn_readfirstlane(uint32_t(rows * kl * 2)), 0x00020000);
  const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc(
      uniform_ptr(vbase + int64_t(key0) * vl), (short)0,
      __builtin_amdgcn_readfirstlane(uint32_t(rows * vl * 2)), 0x00020000);
  char* dst = ring + stage * R::STAGE;
#pragma unroll
  for (int i = 0; i < R::IPT; ++i)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rk, (tk_attn::lds_void*)(dst + i * 1024), 16,
                                             koff[i], 0, 0, kNonTemporal);
#pragma unroll
  for (int i = 0; i < R::IPT; ++i)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rv, (tk_attn::lds_void*)(dst + R::TILE + i * 1024),
                                             16, voff[i], 0, 0, kNonTemporal);
}

template <typename T, int D, int G>
__global__ __launch_bounds__(kWave) void gqa_decode_split_kernel(
    const T* __restrict__ q, const T* __restrict__ k, const T* __restrict__ v,
    const int32_t* __restrict__ seqlens, float* __restrict__ partials, T* __restrict__ o_out,
    float* __restrict__ lse_out, DecodeShape s) {
  using R = Ring<D>;
  using tk_attn::i32x2;
  using tk_attn::lds_read_b128;
  using tk_attn::lds_read_tr16;
  using tk_attn::pin;
  constexpr int DC = D / 32;     // 32-dim chunks (QK k-steps)
  constexpr int OC = D / 16;     // 16-dim output chunks (PV MFMAs)
  constexpr int NS = R::NS, IPT = R::IPT, RB = R::RB;
  // The ring, then the Q tile: heads kvh G .. +15 (rows past G zero) x D, K's swizzle.
  __shared__ __attribute__((aligned(1024))) char ring[NS * R::STAGE + R::QTILE];

  const int split = blockIdx.x;
  const int kvh = blockIdx.y;
  const int b = blockIdx.z;
  // Wave-uniform (readfirstlane): the tile's buffer ranges derive from it and must be
  // scalar, or the compiler wraps each DMA in a loop over the distinct lane values.
  int len = seqlens != nullptr ? __builtin_amdgcn_readfirstlane(seqlens[b]) : s.max_len;
  len = min(max(len, 0), s.max_len);
  const int k0 = split * s.split_len;
  // One split per (batch, KV head): this wave normalizes and writes O and the LSE itself
  // (the combine pass is not launched). An empty sequence gives O = 0 and LSE = -inf, as
  // the combine pass would.
  const bool direct = s.splits == 1;
  if (k0 >= len) {
    if (direct) {
      for (int i = threadIdx.x; i < G * (D / 8); i += kWave) {
        const int h = kvh * G + i / (D / 8);
        *reinterpret_cast<uint4*>(o_out + b * s.ob + h * s.oh + (i % (D / 8)) * 8) =
            uint4{0u, 0u, 0u, 0u};
        if (lse_out != nullptr && i % (D / 8) == 0)
          lse_out[static_cast<int64_t>(b) * s.q_heads + h] = -INFINITY;
      }
    }
    return;  // the combine kernel reads only splits below len
  }
  const int k1 = min(k0 + s.split_len, len);
  const int ntiles = (k1 - k0 + kTileKeys - 1) / kTileKeys;
  auto tile_key = [&](int j) { return k0 + j * kTileKeys; };

  const int lane = threadIdx.x;
  const int row16 = lane & 15;   // key of a K fragment / head of a score or output lane
  const int quad = lane >> 4;    // k-group of an MFMA operand / row group of a result

  const T* kbase = k + b * s.kb + kvh * s.kh;
  const T* vbase = v + b * s.vb + kvh * s.vh;
  // DMA sources: instruction i of a tile covers rows RPI i .. +RPI-1; this lane fetches the
  // chunk that belongs at its LDS slot.
  uint32_t koff[IPT], voff[IPT];
#pragma unroll
  for (int i = 0; i < IPT; ++i) {
    const int row = i * R::RPI + lane / R::CPR;
    const int slot = lane % R::CPR;
    koff[i] = uint32_t(row * s.kl * 2) + uint32_t((slot ^ R::kswz(row)) * 16);
    const int chunk = (((slot >> 1) ^ R::vswz(row)) << 1) | (slot & 1);
    voff[i] = uint32_t(row * s.vl * 2) + uint32_t(chunk * 16);
  }
  // Q^T tile first, by DMA like K and V, so every load of the kernel is counted by the
  // explicit waits (a register load of Q made the compiler wait for the whole prologue).
  {
    const __amdgpu_buffer_rsrc_t rq = __builtin_amdgcn_make_buffer_rsrc(
        uniform_ptr(q + b * s.qb + int64_t(kvh) * G * s.qh), (short)0,
        __builtin_amdgcn_readfirstlane(uint32_t((G - 1) * s.qh * 2 + D * 2)), 0x00020000);
#pragma unroll
    for (int i = 0; i < R::QTILE / 1024; ++i) {
      const int head = i * R::RPI + lane / R::CPR;
      const int slot = lane % R::CPR;
      const uint32_t off = head < G ? uint32_t(head * s.qh * 2) + uint32_t((slot ^ R::kswz(head)) * 16)
                                    : kOob;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          rq, (tk_attn::lds_void*)(ring + NS * R::STAGE + i * 1024), 16, off, 0, 0, 0);
    }
  }
#pragma unroll
  for (int t = 0; t < NS - 1; ++t)
    ring_dma<T, D>(ring, kbase, vbase, s.kl, s.vl, tile_key(t), k1, t, koff, voff);

  // LDS lane addresses. K fragment (tile t2 at +16 t2 rows, an immediate): row row16,
  // chunk 4c + quad. V^T (ds_read_b64_tr_b16: in each 16-lane group, lane 4j + cc reads
  // row j of a 4 x 16 block, columns 4cc .. +3): rows 4 quad + (row16 >> 2) (+16 for the
  // second 16 keys), dims 16c + 4 (row16 & 3) .. +3.
  const uint32_t ring_base = (uint32_t)(uintptr_t)(tk_attn::lds_void*)ring;
  uint32_t ka[DC], va[OC];
#pragma unroll
  for (int c = 0; c < DC; ++c) ka[c] = row16 * RB + (((4 * c + quad) ^ R::kswz(row16)) * 16);
  {
    const int trow = 4 * quad + (row16 >> 2);
#pragma unroll
    for (int c = 0; c < OC; ++c)
      va[c] = R::TILE + trow * RB + ((c ^ R::vswz(trow)) * 32) + 8 * (row16 & 3);
  }

  // Q^T fragments: head row16 (zero past G), dims 32c + 8*quad .. +7.
  i32x4v qf[DC];
  tk_attn::wait_vmcnt<(NS - 1) * 2 * IPT>();
#pragma unroll
  for (int c = 0; c < DC; ++c) qf[c] = lds_read_b128<0>(ring_base + NS * R::STAGE + ka[c]);
  tk_attn::wait_lgkm<0>();
#pragma unroll
  for (int c = 0; c < DC; ++c) pin(qf[c]);

  f32x4v o[OC];
#pragma unroll
  for (int c = 0; c < OC; ++c) o[c] = f32x4v{0.f, 0.f, 0.f, 0.f};
  float m = -INFINITY;  // reference maximum of head row16 (identical in its 4 lanes)
  float l = 0.f;        // this lane's share of head row16's sum

  for (int it = 0; it < ntiles; ++it) {
    // Tile it has landed once at most the NS - 2 younger tiles' loads are outstanding; the
    // stage read in the previous iteration (its reads have returned) takes tile it + NS - 1.
    tk_attn::wait_vmcnt<(NS - 2) * 2 * IPT>();
    ring_dma<T, D>(ring, kbase, vbase, s.kl, s.vl, tile_key(it + NS - 1), k1,
                   (it + NS - 1) % NS, koff, voff);
    __builtin_amdgcn_sched_barrier(0);
    const uint32_t sb = ring_base + (it % NS) * R::STAGE;
    const int key0 = tile_key(it);

    i32x4v kc[2][DC];
#pragma unroll
    for (int c = 0; c < DC; ++c) {
      kc[0][c] = lds_read_b128<0>(sb + ka[c]);
      kc[1][c] = lds_read_b128<16 * RB>(sb + ka[c]);
    }
    tk_attn::wait_lgkm<0>();
#pragma unroll
    for (int c = 0; c < DC; ++c) {
      pin(kc[0][c]);
      pin(kc[1][c]);
    }
    // Scores, scaled to base 2: sc[t][r] is key key0 + 16t + 4*quad + r.
    float sc[2][4];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      f32x4v acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int c = 0; c < DC; ++c) acc = mma16<T>(kc[t][c], qf[c], acc);
#pragma unroll
      for (int r = 0; r < 4; ++r)
        sc[t][r] = key0 + 16 * t + 4 * quad + r < k1 ? acc[r] * s.scale_log2 : -INFINITY;
    }
    // V^T fragments, read while the softmax runs, in batches of at most 4 output chunks
    // (8 reads: lgkmcnt counts at most 15 outstanding LDS instructions).
    constexpr int HB = OC < 4 ? OC : 4;
    i32x2 lo[OC], hi[OC];
#pragma unroll
    for (int c = 0; c < HB; ++c) {
      lo[c] = lds_read_tr16<0>(sb + va[c]);
      hi[c] = lds_read_tr16<16 * RB>(sb + va[c]);
    }
    // Lazy rescale: the reference maximum m moves only when the tile's maximum exceeds it
    // by more than 8 (base-2 units), so p <= 2^8 and o, l are rescaled in a few tiles
    // instead of nearly every one; O = o / l and LSE = m + log2(l) do not depend on m.
    float bmax = sc[0][0];
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int r = 0; r < 4; ++r) bmax = fmaxf(bmax, sc[t][r]);
    bmax = tk_attn::max_over_column(bmax);  // finite: the tile's first key is live
    const bool grow = bmax > m + 8.f;
    if (__builtin_amdgcn_ballot_w64(grow) != 0) {  // wave-uniform: a scalar branch
      const float mnew = grow ? bmax : m;
      float alpha = __builtin_amdgcn_exp2f(m - mnew);  // 1 if kept, 0 on the first tile
      // Defined inside the branch, so the multiplies below cannot be hoisted out of it.
      asm volatile("" : "+v"(alpha));
      m = mnew;
      l *= alpha;
#pragma unroll
      for (int c = 0; c < OC; ++c) o[c] *= alpha;
    }
    float psum = 0.f;
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        sc[t][r] = __builtin_amdgcn_exp2f(sc[t][r] - m);
        psum += sc[t][r];
      }
    l += psum;
    // P^T operand: head row16, k-order (tile 0 keys 4*quad..+3, tile 1 keys 4*quad..+3).
    const i32x4v pf = {pack2<T>(sc[0][0], sc[0][1]), pack2<T>(sc[0][2], sc[0][3]),
                       pack2<T>(sc[1][0], sc[1][1]), pack2<T>(sc[1][2], sc[1][3])};
#pragma unroll
    for (int c0 = 0; c0 < OC; c0 += HB) {
      tk_attn::wait_lgkm<0>();
#pragma unroll
      for (int c = c0; c < c0 + HB; ++c) asm volatile("" : "+v"(lo[c]), "+v"(hi[c]));
      if (c0 + HB < OC) {
#pragma unroll
        for (int c = c0 + HB; c < c0 + 2 * HB; ++c) {
          lo[c] = lds_read_tr16<0>(sb + va[c]);
          hi[c] = lds_read_tr16<16 * RB>(sb + va[c]);
        }
      }
#pragma unroll
      for (int c = c0; c < c0 + HB; ++c)
        o[c] = mma16<T>(i32x4v{lo[c][0], lo[c][1], hi[c][0], hi[c][1]}, pf, o[c]);
    }
  }
  // The tiles issued past the end still write (zeros) into this wave's LDS.
  tk_attn::wait_vmcnt<0>();

  // A head's sum is spread over its 4 lanes (row16, +16, +32, +48).
  l += __shfl_xor(l, 16);
  l += __shfl_xor(l, 32);
  if (direct) {
    // The combine pass's arithmetic for a single split: O = o / l, LSE = m + log2(l).
    if (row16 < G) {
      const int h = kvh * G + row16;
      T* orow = o_out + b * s.ob + h * s.oh;
#pragma unroll
      for (int c = 0; c < OC; ++c) {
        T* dst = orow + 16 * c + 4 * quad;
#pragma unroll
        for (int r = 0; r < 4; ++r) dst[r] = tk::from_f32<T>(o[c][r] / l);
      }
      if (lse_out != nullptr && quad == 0)
        lse_out[static_cast<int64_t>(b) * s.q_heads + h] = m + log2f(l);
    }
    return;
  }
  if (row16 < G) {
    const int h = kvh * G + row16;
    float* out = partials + ((static_cast<int64_t>(b) * s.q_heads + h) * s.splits + split) *
                                partial_stride<D>();
    // o[c][r] is dim 16c + 4*quad + r of head row16.
#pragma unroll
    for (int c = 0; c < OC; ++c)
      *reinterpret_cast<float4*>(out + 16 * c + 4 * quad) =
          make_float4(o[c][0], o[c][1], o[c][2], o[c][3]);
    if (quad == 0) {
      out[D] = m;
      out[D + 1] = l;
    }
  }
}

constexpr int kCombineThreads = 256;

// One workgroup per (batch, query head). Thread t owns column t % D of the split
// slice t / D (R = 256 / D slices, splits i = slice, slice + R, ...); the slices
// are folded in order through LDS, so the result does not depend on timing.
template <typename T, int D>
__global__ __launch_bounds__(kCombineThreads) void gqa_decode_combine_kernel(
    const int32_t* __restrict__ seqlens, const float* __restrict__ partials, T* __restrict__ o,
    float* __restrict__ lse, DecodeShape s) {
  constexpr int PS = partial_stride<D>();
  constexpr int R = kCombineThreads / D;
  __shared__ float red[kCombineThreads / 64];
  __shared__ float acc_s[R][D];
  __shared__ float sum_s[R];
  const int h = blockIdx.x;
  const int b = blockIdx.y;
  const int t = threadIdx.x;
  int len = seqlens != nullptr ? seqlens[b] : s.max_len;
  len = min(max(len, 0), s.max_len);
  const int nsplit = (len + s.split_len - 1) / s.split_len;
  const float* pr = partials + (static_cast<int64_t>(b) * s.q_heads + h) * s.splits * PS;
  const int d = t % D;
  const int slice = t / D;
  float mx = -INFINITY, acc = 0.f, lsum = 0.f;
  if (nsplit <= R) {
    // At most one split per slice: its m, l and column d are loaded together, before the
    // maximum is formed (one round trip to memory instead of two); the same folds as below.
    float mi = -INFINITY, li = 0.f, oi = 0.f;
    if (slice < nsplit) {
      mi = pr[slice * PS + D];
      li = pr[slice * PS + D + 1];
      oi = pr[slice * PS + d];
    }
    mx = tk::group_allreduce<kCombineThreads>(mi, tk::MaxOp{}, red);
    if (mx != -INFINITY && slice < nsplit) {
      const float w = __builtin_amdgcn_exp2f(mi - mx);
      lsum = 0.f + li * w;
      acc = 0.f + oi * w;
    }
  } else {
    for (int i = t; i < nsplit; i += kCombineThreads) mx = fmaxf(mx, pr[i * PS + D]);
    mx = tk::group_allreduce<kCombineThreads>(mx, tk::MaxOp{}, red);
    if (mx != -INFINITY) {
      for (int i = slice; i < nsplit; i += R) {
        const float w = __builtin_amdgcn_exp2f(pr[i * PS + D] - mx);
        lsum += pr[i * PS + D + 1] * w;
        acc += pr[i * PS + d] * w;
      }
    }
  }
  acc_s[slice][d] = acc;
  if (d == 0) sum_s[slice] = lsum;
  tk::lds_barrier();
  if (t < D) {
    float a = acc_s[0][t], ls = sum_s[0];
#pragma unroll
    for (int r = 1; r < R; ++r) {
      a += acc_s[r][t];
      ls += sum_s[r];
    }
    o[b * s.ob + h * s.oh + t] = tk::from_f32<T>(ls > 0.f ? a / ls : 0.f);
    if (lse != nullptr && t == 0)
      lse[static_cast<int64_t>(b) * s.q_heads + h] = ls > 0.f ? mx + log2f(ls) : -INFINITY;
  }
}

template <typename T, int D, int G>
void launch_decode(const T* q, const T* k, const T* v, T* o, float* lse, float* partials,
                   const int32_t* seqlens, const DecodeShape& s, hipStream_t stream) {
  hipLaunchKernelGGL((gqa_decode_split_kernel<T, D, G>),
                     dim3(s.splits, s.kv_heads, s.batch), dim3(kWave), 0, stream, q, k, v,
                     seqlens, partials, o, lse, s);
  if (s.splits > 1)
    hipLaunchKernelGGL((gqa_decode_combine_kernel<T, D>), dim3(s.q_heads, s.batch),
                       dim3(kCombineThreads), 0, stream, seqlens, partials, o, lse, s);
}

template <typename T, int D>
int dispatch_group(int group, const T* q, const T* k, const T* v, T* o, float* lse,
                   float* partials, const int32_t* seqlens, const DecodeShape& s,
                   hipStream_t stream) {
  switch (group) {
    case 1: launch_decode<T, D, 1>(q, k, v, o, lse, partials, seqlens, s, stream); break;
    case 2: launch_decode<T, D, 2>(q, k, v, o, lse, partials, seqlens, s, stream); break;
    case 4: launch_decode<T, D, 4>(q, k, v, o, lse, partials, seqlens, s, stream); break;
    case 8: launch_decode<T, D, 8>(q, k, v, o, lse, partials, seqlens, s, stream); break;
    default: return tk::fail("gqa decode: q_heads / kv_heads must be 1, 2, 4 or 8 (got %d)", group);
  }
  return 0;
}

}  // namespace

extern "C" int tk_gqa_decode(int dtype, const void* q, const void* k, const void* v, void* o,
                             float* lse, float* partials, const int32_t* seqlens, int64_t batch,
                             int64_t q_heads, int64_t kv_heads, int64_t max_len, int64_t head_dim,
                             int64_t split_len, const int64_t* q_strides,
                             const int64_t* k_strides, const int64_t* v_strides,
                             const int64_t* o_strides, float scale, void* stream) {
  if (dtype != TK_DTYPE_F16 && dtype != TK_DTYPE_BF16)
    return tk::fail("gqa decode: dtype must be float16 or bfloat16");
  if (q == nullptr || k == nullptr || v == nullptr || o == nullptr || partials == nullptr ||
      q_strides == nullptr || k_strides == nullptr || v_strides == nullptr ||
      o_strides == nullptr)
    return tk::fail("gqa decode: null pointer");
  if (batch <= 0 || q_heads <= 0 || kv_heads <= 0 || max_len <= 0)
    return tk::fail("gqa decode: empty problem");
  if (head_dim != 64 && head_dim != 128) return tk::fail("gqa decode: head_dim must be 64 or 128");
  if (q_heads % kv_heads != 0) return tk::fail("gqa decode: q_heads must be a multiple of kv_heads");
  if (batch > 65535 || kv_heads > 65535 || q_heads > 65535 || max_len > INT32_MAX)
    return tk::fail("gqa decode: problem too large");
  if (split_len <= 0 || split_len % 64 != 0)
    return tk::fail("gqa decode: split_len must be a positive multiple of 64");
  const int64_t splits = tk::cdiv(max_len, split_len);
  if (splits > INT32_MAX / 2) return tk::fail("gqa decode: too many splits");
  // Every row access is one 16-byte load: aligned bases and row strides.
  for (const void* p : {q, k, v, static_cast<const void*>(o)})
    if (!tk::aligned16(p)) return tk::fail("gqa decode: tensors must be 16-byte aligned");
  const int64_t strides[] = {q_strides[0], q_strides[1], k_strides[0], k_strides[1], k_strides[2],
                             v_strides[0], v_strides[1], v_strides[2], o_strides[0], o_strides[1]};
  for (int64_t st : strides)
    if (st < 0 || (st * 2) % 16 != 0)
      return tk::fail("gqa decode: strides must be non-negative multiples of 8 elements");
  // The DMA tiles address rows through 32-bit buffer offsets (32 rows, or G heads, apart).
  for (int64_t st : {q_strides[1], k_strides[2], v_strides[2]})
    if (st >= (int64_t(1) << 24))
      return tk::fail("gqa decode: head and key strides must be below 2^24 elements");
  DecodeShape s;
  s.batch = static_cast<int>(batch);
  s.q_heads = static_cast<int>(q_heads);
  s.kv_heads = static_cast<int>(kv_heads);
  s.max_len = static_cast<int>(max_len);
  s.split_len = static_cast<int>(split_len);
  s.splits = static_cast<int>(splits);
  s.qb = q_strides[0];
  s.qh = q_strides[1];
  s.kb = k_strides[0];
  s.kh = k_strides[1];
  s.kl = k_strides[2];
  s.vb = v_strides[0];
  s.vh = v_strides[1];
  s.vl = v_strides[2];
  s.ob = o_strides[0];
  s.oh = o_strides[1];
  s.scale_log2 = scale * kLog2e;
  const int group = static_cast<int>(q_heads / kv_heads);
  hipStream_t st = tk::as_stream(stream);
  int rc;
  if (dtype == TK_DTYPE_BF16) {
    rc = head_dim == 128
             ? dispatch_group<__bf16, 128>(group, static_cast<const __bf16*>(q),
                                           static_cast<const __bf16*>(k),
                                           static_cast<const __bf16*>(v), static_cast<__bf16*>(o),
                                           lse, partials, seqlens, s, st)
             : dispatch_group<__bf16, 64>(group, static_cast<const __bf16*>(q),
                                          static_cast<const __bf16*>(k),
                                          static_cast<const __bf16*>(v), static_cast<__bf16*>(o),
                                          lse, partials, seqlens, s, st);
  } else {
    rc = head_dim == 128
             ? dispatch_group<_Float16, 128>(group, static_cast<const _Float16*>(q),
                                             static_cast<const _Float16*>(k),
                                             static_cast<const _Float16*>(v),
                                             static_cast<_Float16*>(o), lse, partials, seqlens, s,
                                             st)
             : dispatch_group<_Float16, 64>(group, static_cast<const _Float16*>(q),
                                            static_cast<const _Float16*>(k),
                                            static_cast<const _Float16*>(v),
                                            static_cast<_Float16*>(o), lse, partials, seqlens, s,
                                            st);
  }
  if (rc != 0) return rc;
  return tk::check_launch("gqa decode");
}
