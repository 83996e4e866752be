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
//   S^T (16 keys x 16 heads) = K (16 keys x 32 dims) . Q^T, K fragments loaded
//     from HBM straight into registers (lane l: key l%16, dims 8*(l/16)..+7 of a
//     32-dim chunk), Q^T held in registers with heads >= G zero. Lane l then holds
//     head l%16's scores for keys 4*(l/16)..+3 of the tile; a head's row maximum
//     is a max over the lane's values and lanes ^16, ^32.
//   O^T (16 dims x 16 heads) += V^T (16 dims x 32 keys) . P^T, P^T straight from
//     the score registers (two tiles give a lane 8 keys, the MFMA k-order), V^T
//     read from a per-wave LDS copy of the 32-key V tile with ds_read_b64_tr_b16
//     (rows padded so each 32-lane phase hits 32 distinct banks).
//   Loads of the next 32 keys are issued before the current ones are used.
// Combine kernel: one workgroup per (batch, query head) folds the splits in a
// fixed order (independent of timing) and writes O and the LSE.
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

// Elements per LDS row of the V tile: D plus 16 (32 bytes) of padding, so the rows
// one 32-lane ds_read_b64_tr_b16 phase reads fall on 32 distinct banks.
template <int D>
constexpr int vt_row() {
  return D + 16;
}

constexpr int kTileKeys = 32;  // keys per iteration: two 16-key MFMA tiles

template <typename T, int D, int G>
__global__ __launch_bounds__(kWave) void gqa_decode_split_kernel(
    const T* __restrict__ q, const T* __restrict__ k, const T* __restrict__ v,
    const int32_t* __restrict__ seqlens, float* __restrict__ partials, DecodeShape s) {
  constexpr int DC = D / 32;     // 32-dim chunks (QK k-steps)
  constexpr int OC = D / 16;     // 16-dim output chunks (PV MFMAs)
  constexpr int VCH = kTileKeys * D / 8 / kWave;  // 16-byte V chunks per lane per tile
  constexpr int VRC = D / 8;     // 16-byte chunks per V row
  constexpr int VR = vt_row<D>();
  __shared__ __attribute__((aligned(16))) T vt[kTileKeys * VR];

  const int split = blockIdx.x;
  const int kvh = blockIdx.y;
  const int b = blockIdx.z;
  int len = seqlens != nullptr ? seqlens[b] : s.max_len;
  len = min(max(len, 0), s.max_len);
  const int k0 = split * s.split_len;
  if (k0 >= len) return;  // the combine kernel reads only splits below len
  const int k1 = min(k0 + s.split_len, len);

  const int lane = threadIdx.x;
  const int row16 = lane & 15;   // key of a K fragment / head of a score or output lane
  const int quad = lane >> 4;    // k-group of an MFMA operand / row group of a result

  // Q^T fragments: head row16 (zero past G), dims 32c + 8*quad .. +7.
  i32x4v qf[DC];
#pragma unroll
  for (int c = 0; c < DC; ++c) {
    qf[c] = i32x4v{0, 0, 0, 0};
    if (row16 < G) qf[c] = load16(q + b * s.qb + (kvh * G + row16) * s.qh + 32 * c + 8 * quad);
  }
  const T* kbase = k + b * s.kb + kvh * s.kh;
  const T* vbase = v + b * s.vb + kvh * s.vh;

  // Loads of one 32-key tile: K fragments (tile t, chunk c) and V 16-byte chunks.
  i32x4v kf[2][DC], vf[VCH];
  auto load_tile = [&](int key0) {
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const int key = key0 + 16 * t + row16;
#pragma unroll
      for (int c = 0; c < DC; ++c)
        kf[t][c] = key < k1 ? load16(kbase + static_cast<int64_t>(key) * s.kl + 32 * c + 8 * quad)
                            : i32x4v{0, 0, 0, 0};
    }
#pragma unroll
    for (int i = 0; i < VCH; ++i) {
      const int id = i * kWave + lane;
      const int key = key0 + id / VRC;
      vf[i] = key < k1 ? load16(vbase + static_cast<int64_t>(key) * s.vl + 8 * (id % VRC))
                       : i32x4v{0, 0, 0, 0};
    }
  };

  f32x4v o[OC];
#pragma unroll
  for (int c = 0; c < OC; ++c) o[c] = f32x4v{0.f, 0.f, 0.f, 0.f};
  float m = -INFINITY;  // running maximum of head row16 (identical in its 4 lanes)
  float l = 0.f;        // this lane's share of head row16's sum

  load_tile(k0);
  for (int key0 = k0; key0 < k1; key0 += kTileKeys) {
    i32x4v kc[2][DC], vc[VCH];
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int c = 0; c < DC; ++c) kc[t][c] = kf[t][c];
#pragma unroll
    for (int i = 0; i < VCH; ++i) vc[i] = vf[i];
    if (key0 + kTileKeys < k1) load_tile(key0 + kTileKeys);

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
    float bmax = sc[0][0];
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int r = 0; r < 4; ++r) bmax = fmaxf(bmax, sc[t][r]);
    bmax = fmaxf(bmax, __shfl_xor(bmax, 16));
    bmax = fmaxf(bmax, __shfl_xor(bmax, 32));
    const float mnew = fmaxf(m, bmax);  // finite: the tile's first key is live
    const float alpha = __builtin_amdgcn_exp2f(m - mnew);
    m = mnew;
    float p[2][4];
    float psum = 0.f;
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        p[t][r] = __builtin_amdgcn_exp2f(sc[t][r] - mnew);
        psum += p[t][r];
      }
    l = l * alpha + psum;
    // P^T operand: head row16, k-order (tile 0 keys 4*quad..+3, tile 1 keys 4*quad..+3).
    const i32x4v pf = {pack2<T>(p[0][0], p[0][1]), pack2<T>(p[0][2], p[0][3]),
                       pack2<T>(p[1][0], p[1][1]), pack2<T>(p[1][2], p[1][3])};

    // V tile to LDS (row-major, padded rows), then V^T fragments by transposed reads.
#pragma unroll
    for (int i = 0; i < VCH; ++i) {
      const int id = i * kWave + lane;
      *reinterpret_cast<i32x4v*>(vt + (id / VRC) * VR + 8 * (id % VRC)) = vc[i];
    }
    // ds_read_b64_tr_b16: in each 16-lane group, lane 4j + c addresses row j and
    // columns 4c..4c+3 of a 4 x 16 block; lane i receives column i of the 4 rows.
    const int trow = 4 * quad + (row16 >> 2);
    const int tcol = 4 * (row16 & 3);
#pragma unroll
    for (int c = 0; c < OC; ++c) {
      o[c] *= alpha;
      typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
      const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
          (lds_s16x4*)(vt + trow * VR + 16 * c + tcol));
      const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
          (lds_s16x4*)(vt + (16 + trow) * VR + 16 * c + tcol));
      const i32x4v vtf = {__builtin_bit_cast(int, short2{lo[0], lo[1]}),
                          __builtin_bit_cast(int, short2{lo[2], lo[3]}),
                          __builtin_bit_cast(int, short2{hi[0], hi[1]}),
                          __builtin_bit_cast(int, short2{hi[2], hi[3]})};
      o[c] = mma16<T>(vtf, pf, o[c]);
    }
  }

  // A head's sum is spread over its 4 lanes (row16, +16, +32, +48).
  l += __shfl_xor(l, 16);
  l += __shfl_xor(l, 32);
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
  float mx = -INFINITY;
  for (int i = t; i < nsplit; i += kCombineThreads) mx = fmaxf(mx, pr[i * PS + D]);
  mx = tk::group_allreduce<kCombineThreads>(mx, tk::MaxOp{}, red);
  const int d = t % D;
  const int slice = t / D;
  float acc = 0.f, lsum = 0.f;
  if (mx != -INFINITY) {
    for (int i = slice; i < nsplit; i += R) {
      const float w = __builtin_amdgcn_exp2f(pr[i * PS + D] - mx);
      lsum += pr[i * PS + D + 1] * w;
      acc += pr[i * PS + d] * w;
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
                     seqlens, partials, s);
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
