// Internal interface between the GEMM entry point (gemm.hip) and its buffer->LDS DMA
// fast path (gemm_dma.hip).
#pragma once
#include <hip/hip_runtime.h>
#include <cstdint>

namespace tk {

// True when the DMA kernel handles this problem: row-major f16/bf16 operands with unit
// inner strides, 16-byte aligned rows, K a multiple of 32 and byte extents below 2 GiB.
bool gemm_dma_applies(const void* a, const void* b, int64_t m, int64_t n, int64_t k,
                      int64_t stride_am, int64_t stride_ak, int64_t stride_bk, int64_t stride_bn);

// Enqueues the DMA kernel; arguments are checked by the caller. With `row_scale`
// (float32[m]) row m of C is round(row_scale[m] * acc).
void gemm_dma_launch(int dtype, const void* a, const void* b, void* c, int64_t m, int64_t n,
                     int64_t k, int64_t stride_am, int64_t stride_bk, int64_t stride_cm,
                     int64_t stride_cn, hipStream_t stream, const float* row_scale = nullptr);

// Enqueues the SwiGLU-fused DMA kernel: y = swiglu(value = a * b_up, gate = a * b_gate),
// both weights [K, N] row-major; each must satisfy gemm_dma_applies with `a`.
void gemm_swiglu_dma_launch(int dtype, const void* a, const void* b_gate, const void* b_up,
                            void* y, int64_t m, int64_t n, int64_t k, int64_t stride_am,
                            int64_t stride_gk, int64_t stride_uk, int64_t stride_ym,
                            int64_t stride_yn, hipStream_t stream);

}  // namespace tk
