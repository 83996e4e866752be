// Device helpers shared by the buffer->LDS DMA attention kernels (attention_fwd.hip,
// attention_bwd.hip): MFMA wrappers on raw 32-bit fragments, accumulator packing,
// explicit wait counters, and LDS reads as inline asm (the compiler would wait for
// every outstanding LDS DMA before each compiler-visible LDS read).
#pragma once
#include "tk_common.hpp"

namespace tk_attn {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x2 __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) void lds_void;

constexpr float kNegInf = -INFINITY;
template <typename T>
struct Mma;
template <>
struct Mma<_Float16> {
  static __device__ __forceinline__ f32x16 run(i32x4 a, i32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
};
template <>
struct Mma<__bf16> {
  static __device__ __forceinline__ f32x16 run(i32x4 a, i32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
};

// v_mfma_f32_16x16x32: A lane l holds row l % 16, k = 8 (l / 16) .. +7; B lane l holds
// column l % 16, the same k; D lane l holds column l % 16, rows 4 (l / 16) .. +3.
template <typename T>
struct Mma16;
template <>
struct Mma16<_Float16> {
  static __device__ __forceinline__ f32x4 run(i32x4 a, i32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
};
template <>
struct Mma16<__bf16> {
  static __device__ __forceinline__ f32x4 run(i32x4 a, i32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
};

// Two 16x16 accumulators (4 registers each) rounded (RNE) to T: one MFMA operand whose
// k-indices 0..3 are lo's registers and 4..7 hi's.
template <typename T>
__device__ __forceinline__ i32x4 acc_frag2(const f32x4& lo, const f32x4& hi) {
  const f32x8 v = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
  if constexpr (__is_same(T, __bf16))
    return __builtin_bit_cast(i32x4, __builtin_convertvector(v, bf16x8));
  else
    return __builtin_bit_cast(i32x4, __builtin_convertvector(v, f16x8));
}

// Registers 8g .. 8g+7 of an accumulator rounded (RNE) to T: an MFMA operand.
template <typename T>
__device__ __forceinline__ i32x4 acc_frag(const f32x16& acc, int g) {
  const f32x8 v = {acc[g * 8 + 0], acc[g * 8 + 1], acc[g * 8 + 2], acc[g * 8 + 3],
                   acc[g * 8 + 4], acc[g * 8 + 5], acc[g * 8 + 6], acc[g * 8 + 7]};
  if constexpr (__is_same(T, __bf16))
    return __builtin_bit_cast(i32x4, __builtin_convertvector(v, bf16x8));
  else
    return __builtin_bit_cast(i32x4, __builtin_convertvector(v, f16x8));
}

template <typename T>
__device__ __forceinline__ uint32_t pack2(float lo, float hi) {
  const uint16_t a = __builtin_bit_cast(uint16_t, tk::from_f32<T>(lo));
  const uint16_t b = __builtin_bit_cast(uint16_t, tk::from_f32<T>(hi));
  return uint32_t(a) | (uint32_t(b) << 16);
}

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
  // s_waitcnt fields: vmcnt[3:0], expcnt[6:4] (7 = no wait), lgkmcnt[11:8] (15 = no
  // wait), vmcnt[5:4] at [15:14].
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

template <int N>
__device__ __forceinline__ void wait_lgkm() {
  asm volatile("s_waitcnt lgkmcnt(%0)" ::"i"(N) : "memory");
}

// Keeps every use of an LDS-read result below the preceding wait (volatile asm
// statements stay in program order; this one redefines the value).
__device__ __forceinline__ void pin(i32x4& f) { asm volatile("" : "+v"(f)); }
__device__ __forceinline__ void pin(f32x4& f) { asm volatile("" : "+v"(f)); }

// Barrier without __syncthreads()'s fence, which would wait for every outstanding DMA.
__device__ __forceinline__ void barrier_no_fence() { asm volatile("s_barrier" ::: "memory"); }

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

// Transposed fragment of a 32-key step starting at row ROW0 of a row-major [keys][D] tile:
// rows ROW0 + 4g .. +3 (k-index 0..3 of lane group g = lane / 16) and ROW0 + 16 + 4g .. +3
// (k-index 4..7), the key order of an operand built from two 16x16 accumulators (key
// tiles 2s and 2s + 1). The lane supplies the address of row ROW0 + 4g + (lane % 16) / 4,
// features 4 (lane % 4) .. +3 of its 16-feature tile.
template <int ROW0, int RB>
__device__ __forceinline__ i32x4 read_v16(uint32_t addr) {
  const i32x2 a = lds_read_tr16<ROW0 * RB>(addr);
  const i32x2 b = lds_read_tr16<(ROW0 + 16) * RB>(addr);
  return i32x4{a[0], a[1], b[0], b[1]};
}

__device__ __forceinline__ void sched_fence() { __builtin_amdgcn_sched_barrier(0); }

// SIMD of the executing wave (HW_ID bits 5:4).
__device__ __forceinline__ int simd_id() {
  return __builtin_amdgcn_s_getreg((1 << 11) | (4 << 6) | 4);
}

// Lane maximum over itself and lane ^ 32 (the swap returns both values, in either order).
__device__ __forceinline__ float max_with_partner(float x) {
  const auto pr = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x),
                                                   false, false);
  return fmaxf(__uint_as_float(pr[0]), __uint_as_float(pr[1]));
}

__device__ __forceinline__ float sum_with_partner(float x) {
  const auto pr = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x),
                                                   false, false);
  return __uint_as_float(pr[0]) + __uint_as_float(pr[1]);
}

// Maximum / sum over the four lanes l % 16 + 16 {0..3} (a 16x16 accumulator column):
// a permlane32 swap pairs l with l ^ 32, a permlane16 swap then l with l ^ 16. Both
// swaps return the lane's own and its partner's value (in either order), so every lane
// of a column ends with the same result.
__device__ __forceinline__ float max_over_column(float x) {
  x = max_with_partner(x);
  const auto pr = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x),
                                                   false, false);
  return fmaxf(__uint_as_float(pr[0]), __uint_as_float(pr[1]));
}

__device__ __forceinline__ float sum_over_column(float x) {
  x = sum_with_partner(x);
  const auto pr = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x),
                                                   false, false);
  return __uint_as_float(pr[0]) + __uint_as_float(pr[1]);
}

// ---- Variable-length batches ---------------------------------------------------------
// Sequence b is rows cu[b] .. cu[b+1] of the packed tensors. Both offsets are clamped
// into [0, total] (the end also to >= the start) and the length to seq, so no lengths
// table can address rows outside the packed tensors.
struct VarlenRows {
  int start, n;
};
__device__ __forceinline__ VarlenRows varlen_rows(const int32_t* cu, int b, int total, int seq) {
  const int start = min(max(cu[b], 0), total);
  return {start, min(min(max(cu[b + 1], start), total) - start, seq)};
}

// Sum over the wave of v in [0, 2^bits): one ballot per bit, so the result is scalar.
__device__ __forceinline__ int wave_sum_bits(int v, int bits) {
  int sum = 0;
  for (int k = 0; k < bits; ++k) sum += __popcll(__ballot((v >> k) & 1)) << k;
  return sum;
}

// Heavy-first tile schedule of a variable-length batch, shared by every head. Sequence
// b has nb_b = ceil(n_b / blk) blocks and contributes one tile to each level
// 0 .. nb_b - 1; tiles are numbered from the top level down and by sequence within a
// level, so tile 0 is the last block of the longest sequence and every sequence's
// heaviest tiles start before any lighter ones. Tiles at levels >= j number
// C(j) = sum_b max(0, nb_b - j): tile t is at the largest level j with C(j) > t
// (binary search over the levels), and is the (t - C(j+1))-th sequence with
// nb_b > j. The first 64 sequences' block counts stay in a register; longer batches
// reload the offsets on each pass. The caller makes t wave-uniform; the results are
// scalar. Returns false when t is past the last tile.
struct VarlenTile {
  int b, level;
};
__device__ __forceinline__ bool varlen_tile(const int32_t* cu, int batch, int total, int seq,
                                            int blk, int t, VarlenTile& out) {
  const int lane = threadIdx.x & 63;
  const int levels = (seq + blk - 1) / blk;
  const int bits = 32 - __builtin_clz(unsigned(levels));  // max(0, nb - j) <= levels
  auto blocks = [&](int b) {
    return b < batch ? (varlen_rows(cu, b, total, seq).n + blk - 1) / blk : 0;
  };
  const int nb0 = blocks(lane);
  auto chunk = [&](int b0) { return b0 == 0 ? nb0 : blocks(b0 + lane); };
  auto tiles_from = [&](int j) {
    int c = 0;
    for (int b0 = 0; b0 < batch; b0 += 64) c += wave_sum_bits(max(chunk(b0) - j, 0), bits);
    return c;
  };
  if (t >= tiles_from(0)) return false;
  int lo = 0, hi = levels, c_hi = 0;  // C(lo) > t >= C(hi) == c_hi
  while (hi - lo > 1) {
    const int mid = (lo + hi) >> 1;
    const int c = tiles_from(mid);
    if (c > t) {
      lo = mid;
    } else {
      hi = mid;
      c_hi = c;
    }
  }
  int r = t - c_hi;  // rank among the sequences with more than lo blocks
  for (int b0 = 0; b0 < batch; b0 += 64) {
    const bool has = chunk(b0) > lo;
    const uint64_t m = __ballot(has);
    const int c = __popcll(m);
    if (r < c) {
      const int below =
          __builtin_amdgcn_mbcnt_hi(uint32_t(m >> 32), __builtin_amdgcn_mbcnt_lo(uint32_t(m), 0));
      out.b = b0 + __builtin_ctzll(__ballot(has && below == r));
      out.level = lo;
      return true;
    }
    r -= c;
  }
  return false;
}

// Workgroups of a variable-length launch: w = tile * heads + i. Consecutive workgroups
// take the heads of one tile, which the hardware deals round-robin over the 8 XCDs, so
// every XCD gets an equal share of each level. With heads % 8 == 0, slot i maps to head
// (i % 8) * (heads / 8) + i / 8: XCD x then holds heads x*heads/8 .. (x+1)*heads/8 - 1,
// and a grouped-query group's heads share one L2.
__device__ __forceinline__ int varlen_head(int w, int heads) {
  const int i = w % heads;
  return heads % 8 == 0 ? (i % 8) * (heads / 8) + i / 8 : i;
}

// Upper bound on the tiles of a variable-length batch: sum_b ceil(n_b / blk) is below
// total / blk + batch for offsets that partition [0, total], and at most batch * levels.
inline int64_t varlen_tiles(int64_t batch, int64_t total, int64_t seq, int64_t blk) {
  const int64_t by_total = (total + blk - 1) / blk + batch;
  const int64_t by_seq = batch * ((seq + blk - 1) / blk);
  return by_total < by_seq ? by_total : by_seq;
}

// A kernel's argument block, read afresh: `Args` is the kernel's only parameter, so it
// starts the kernarg segment. The segment pointer passes through an empty asm at each
// call, so a loop that calls this once per iteration loads the arguments where each
// iteration uses them instead of hoisting the loads out of the loop and holding every
// field in scalar registers across it (which made persistent loops spill).
template <typename Args>
__device__ __forceinline__ const Args& kernel_args() {
  typedef const __attribute__((address_space(4))) char kernarg_char;
  kernarg_char* p = (kernarg_char*)__builtin_amdgcn_kernarg_segment_ptr();
  asm volatile("" : "+s"(p));
  return *(const Args*)p;
}

// Block `it` (0, 1) of this workgroup in a causal launch that deals blocks in pairs: the
// grid has one workgroup per pair (paired_items), ranks i and units-1-i of one head (rank 0
// is a head's heaviest block under causal masking), so every pair carries the same work.
// Returns (head, rank), or false when the workgroup is done. With heads and the grid both
// multiples of 8, workgroup w runs on XCD w % 8 and takes a pair of that XCD's eighth of
// the heads (a head's K/V or Q/dO blocks then stay in one L2), head-major. Equal durations
// keep the hardware dispatcher from stalling: it hands workgroups to the XCDs in a fixed
// round-robin order and waits on an XCD whose next CU is still busy, so with one causal
// block per workgroup a CU sat idle ~11.5 us on average between blocks (non-causal:
// 2.8 us). Pairs ran the causal D128 forward 1.80 -> 1.75 ms on one box and 1.86 -> 1.81 ms
// on another; persistent workgroups (one per CU slot, walking their pairs) 1.82 ms there.
__device__ __forceinline__ bool paired_tile(int& it, int heads, int units, int& head,
                                            int& rank) {
  int j = blockIdx.x, gx = gridDim.x, h0 = 0, hn = heads;
  if (heads % 8 == 0 && gridDim.x % 8 == 0) {
    j = blockIdx.x / 8;
    gx = gridDim.x / 8;
    hn = heads / 8;
    h0 = (blockIdx.x % 8) * hn;
  }
  const int ph = (units + 1) / 2;  // pairs per head
  for (;;) {
    const int p = j + (it >> 1) * gx;
    if (p >= hn * ph) return false;
    const int i = p % ph;
    head = h0 + p / ph;
    if ((it & 1) == 0) {
      rank = i;
      return true;
    }
    if (i != units - 1 - i) {
      rank = units - 1 - i;
      return true;
    }
    ++it;  // odd unit count: the middle rank has no partner
  }
}

// Workgroups of a paired launch over `heads` heads of `units` blocks (paired_tile).
inline int64_t paired_items(int64_t heads, int64_t units) { return heads * ((units + 1) / 2); }

}  // namespace tk_attn
