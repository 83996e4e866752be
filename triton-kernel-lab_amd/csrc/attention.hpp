// Internal interface between the attention entry points (attention.hip) and the
// buffer->LDS DMA kernels (attention_fwd.hip, attention_bwd.hip, attention_bwd_dq.hip). `kv_heads` divides
// `heads`: query head h reads K/V head h / (heads / kv_heads) (kv_heads == heads is
// multi-head attention). With `cu_seqlens` (int32[batch + 1]) the batch is variable-length:
// sequence b is rows cu_seqlens[b] .. cu_seqlens[b + 1] of a packed [total][head][dim]
// layout (batch strides 0, `seq` the longest length) and LSE / delta are [head][total].
// With rope tables (forward only) Q is rotated (rotate-half RoPE, tables [pos][D/2]
// indexed by query position) as it is loaded.
#pragma once
#include <hip/hip_runtime.h>
#include <cstdint>

namespace tk {

// True when each head's K and V rows span less than 2 GiB (32-bit buffer offsets).
// The caller has already checked dtype, head_dim and 16-byte row alignment.
bool attn_fwd_dma_applies(int64_t seq, int64_t head_dim, const int64_t* k_strides,
                          const int64_t* v_strides);

void attn_fwd_dma_launch(int dtype, const void* q, const void* k, const void* v, void* o,
                         float* lse, int64_t batch, int64_t heads, int64_t kv_heads, int64_t seq,
                         int64_t head_dim, const int64_t* q_strides, const int64_t* k_strides,
                         const int64_t* v_strides, const int64_t* o_strides, float sm_scale,
                         bool causal, hipStream_t stream, const int32_t* cu_seqlens = nullptr,
                         int64_t total = 0, const void* rope_cos = nullptr,
                         const void* rope_sin = nullptr, int64_t rope_stride = 0);

// True when one query head's rows (layout of q, dO, dQ) and one KV head's rows (layout
// of k, v, dK, dV) each span less than 2 GiB. The caller has already checked dtype,
// head_dim and 16-byte row alignment.
bool attn_bwd_dma_applies(int64_t seq, int64_t head_dim, const int64_t* q_strides,
                          const int64_t* kv_strides);

// dK, dV per KV head, summed over its query heads in a fixed order (single writer).
void attn_bwd_dkdv_dma_launch(int dtype, const void* q, const void* k, const void* v,
                              const void* dout, void* dk, void* dv, const float* lse,
                              const float* delta, int64_t batch, int64_t heads,
                              int64_t kv_heads, int64_t seq, int64_t head_dim,
                              const int64_t* q_strides, const int64_t* kv_strides,
                              float sm_scale, bool causal, hipStream_t stream,
                              const int32_t* cu_seqlens = nullptr, int64_t total = 0);

// dQ per query head (attention_bwd_dq.hip); each row has a single writer.
void attn_bwd_dq_dma_launch(int dtype, const void* q, const void* k, const void* v,
                            const void* dout, void* dq, const float* lse, const float* delta,
                            int64_t batch, int64_t heads, int64_t kv_heads, int64_t seq,
                            int64_t head_dim, const int64_t* q_strides,
                            const int64_t* kv_strides, float sm_scale, bool causal,
                            hipStream_t stream, const int32_t* cu_seqlens = nullptr,
                            int64_t total = 0);

}  // namespace tk
