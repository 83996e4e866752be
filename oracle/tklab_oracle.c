/*
 * tklab_oracle.c — CPU restatement of triton-kernel-lab's transformer-layer
 * kernels. TEST INFRASTRUCTURE ONLY: the checker that tests/, the smoke test
 * and bench.py's cpu_baseline leg compare the HIP kernels against. Nothing in
 * the product (the tklab package, libtklab_hip.so) links or calls it.
 *
 * Conventions
 *   - Every tensor is a contiguous float32 array holding values that are
 *     exactly representable in the storage dtype `dt` (0 = float32,
 *     1 = float16, 2 = bfloat16); the caller converts.
 *   - Arithmetic is float32 in the reference kernel's operation order, except
 *     that long sums (row reductions, dot products) accumulate in double so
 *     the oracle is at least as accurate as any summation order the device
 *     may use. Where the reference stores or casts to the storage dtype
 *     (outputs, the residual sum, attention's P and dS operands) the oracle
 *     rounds to nearest-even in `dt` at the same point.
 *   - Each function cites the reference lines it restates.
 *
 * Pinning: tests/test_oracle.py checks every function here against PyTorch
 * library routines (softmax, F.rms_norm, F.silu, matmul, SDPA, autograd) and
 * closed forms (constant rows, identity matrices, norm preservation, the
 * inverse-rotation identity, single-key attention, the base-2 LSE closed form);
 * or_gqa_decode reduces to the last row of causal or_attn_fwd, to repeated KV
 * heads and to truncated caches, and matches PyTorch's SDPA.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define OR_F32 0
#define OR_F16 1
#define OR_BF16 2

static const double kLog2e = 1.4426950408889634;

static uint32_t f2u(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return u;
}
static float u2f(uint32_t u) {
  float f;
  memcpy(&f, &u, 4);
  return f;
}

/* Round-to-nearest-even of a float32 value to bfloat16 (8-bit mantissa). */
static float round_bf16(float f) {
  uint32_t u = f2u(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return f; /* NaN */
  u += 0x7fffu + ((u >> 16) & 1u);
  return u2f(u & 0xffff0000u);
}

/* Round-to-nearest-even of a float32 value to IEEE binary16. */
static float round_f16(float f) {
  const uint32_t u = f2u(f);
  const uint32_t a = u & 0x7fffffffu;
  if (a >= 0x7f800000u) return f;                /* Inf / NaN */
  if (a < 0x38800000u) {                         /* below 2^-14: subnormal quantum 2^-24 */
    return rintf(f * 16777216.0f) / 16777216.0f; /* exact scaling; rintf rounds to even */
  }
  uint32_t r = a + 0x0fffu + ((a >> 13) & 1u); /* drop 13 mantissa bits, nearest-even */
  r &= ~0x1fffu;
  if (r >= 0x47800000u) r = 0x7f800000u; /* >= 65520 rounds past 65504 */
  return u2f(r | (u & 0x80000000u));
}

float or_round(float f, int dt) {
  if (dt == OR_F16) return round_f16(f);
  if (dt == OR_BF16) return round_bf16(f);
  return f;
}

void or_round_array(float* x, int64_t n, int dt) {
  for (int64_t i = 0; i < n; ++i) x[i] = or_round(x[i], dt);
}

/* ------------------------------------------------------------------ softmax
 * src/tklab/kernels/fused_softmax.py:32-39: float32 row, shifted = x - max,
 * numerator = exp(shifted), y = numerator / sum, stored in the input dtype. */
void or_softmax(const float* x, float* y, int64_t rows, int64_t cols, int dt) {
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; ++r) {
    const float* xr = x + r * cols;
    float* yr = y + r * cols;
    float m = xr[0];
    for (int64_t c = 1; c < cols; ++c) m = fmaxf(m, xr[c]);
    double sum = 0.0;
    for (int64_t c = 0; c < cols; ++c) {
      yr[c] = expf(xr[c] - m);
      sum += yr[c];
    }
    const float s = (float)sum;
    for (int64_t c = 0; c < cols; ++c) yr[c] = or_round(yr[c] / s, dt);
  }
}

/* ------------------------------------------------------------------ RMSNorm
 * Forward: src/tklab/kernels/rms_norm.py:61-78 and
 * src/tklab/kernels/residual_rms_norm.py:52-82.
 *   s = x (+ residual, rounded to dt), mean_sq = sum(s*s)/n,
 *   rstd = 1/sqrt(mean_sq + eps), y = s * rstd * w (rounded to dt).
 * `residual`, `sum_out` and `rstd_out` may be NULL. */
void or_rmsnorm_fwd(const float* x, const float* residual, const float* w, float* sum_out,
                    float* y, float* rstd_out, int64_t rows, int64_t cols, float eps, int dt) {
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; ++r) {
    const float* xr = x + r * cols;
    float* yr = y + r * cols;
    double ss = 0.0;
    for (int64_t c = 0; c < cols; ++c) {
      float s = xr[c];
      if (residual) s = or_round(s + residual[r * cols + c], dt);
      if (sum_out) sum_out[r * cols + c] = s;
      yr[c] = s; /* stash s; overwritten below */
      ss += (double)s * s;
    }
    const float mean_sq = (float)(ss / (double)cols);
    const float rstd = 1.0f / sqrtf(mean_sq + eps);
    for (int64_t c = 0; c < cols; ++c) yr[c] = or_round(yr[c] * rstd * w[c], dt);
    if (rstd_out) rstd_out[r] = rstd;
  }
}

/* Backward: src/tklab/kernels/rms_norm.py:105-133 (stage 1) and 153-173 (stage 2).
 *   x_hat = x*rstd, g = w*dy, dx = rstd*(g - x_hat*sum(g*x_hat)/n) (+ incoming),
 *   dw = sum over rows of dy*x_hat. dx and dw are rounded to dt. `incoming`
 *   may be NULL. `dw_acc` is scratch of `cols` doubles. */
void or_rmsnorm_bwd(const float* dy, const float* x, const float* w, const float* rstd,
                    const float* incoming, float* dx, float* dw, double* dw_acc, int64_t rows,
                    int64_t cols, int dt) {
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; ++r) {
    const float rs = rstd[r];
    double dot = 0.0;
    for (int64_t c = 0; c < cols; ++c) {
      const float x_hat = x[r * cols + c] * rs;
      const float g = w[c] * dy[r * cols + c];
      dot += (double)g * x_hat;
    }
    const float mean = (float)(dot / (double)cols);
    for (int64_t c = 0; c < cols; ++c) {
      const float x_hat = x[r * cols + c] * rs;
      const float g = w[c] * dy[r * cols + c];
      float d = rs * (g - x_hat * mean);
      if (incoming) d += incoming[r * cols + c];
      dx[r * cols + c] = or_round(d, dt);
    }
  }
  for (int64_t c = 0; c < cols; ++c) dw_acc[c] = 0.0;
  for (int64_t r = 0; r < rows; ++r) {
    const float rs = rstd[r];
    for (int64_t c = 0; c < cols; ++c) dw_acc[c] += (double)(dy[r * cols + c] * (x[r * cols + c] * rs));
  }
  for (int64_t c = 0; c < cols; ++c) dw[c] = or_round((float)dw_acc[c], dt);
}

/* ------------------------------------------------------------------ SwiGLU
 * Stable sigmoid: src/tklab/kernels/_elementwise_math.py:12-18.
 * Forward src/tklab/kernels/swiglu.py:44-58: y = value * gate * sigmoid(gate).
 * Backward swiglu.py:82-108: dvalue = dy*silu, dgate = dy*value*silu'. */
static float stable_sigmoid(float z) {
  const float e = expf(-fabsf(z));
  const float d = 1.0f + e;
  return z >= 0.0f ? 1.0f / d : e / d;
}

void or_swiglu_fwd(const float* value, const float* gate, float* y, int64_t n, int dt) {
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < n; ++i) {
    const float g = gate[i];
    y[i] = or_round(value[i] * g * stable_sigmoid(g), dt);
  }
}

void or_swiglu_bwd(const float* dy, const float* value, const float* gate, float* dvalue,
                   float* dgate, int64_t n, int dt) {
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < n; ++i) {
    const float g = gate[i];
    const float s = stable_sigmoid(g);
    const float silu = g * s;
    const float dsilu = s * (1.0f + g * (1.0f - s));
    dvalue[i] = or_round(dy[i] * silu, dt);
    dgate[i] = or_round(dy[i] * value[i] * dsilu, dt);
  }
}

/* ------------------------------------------------------------------ RoPE
 * Forward src/tklab/kernels/rope.py:44-73: y1 = x1*c - x2*s, y2 = x2*c + x1*s.
 * Backward rope.py:102-160: dx1 = dy1*c + dy2*s, dx2 = dy2*c - dy1*s,
 * dcos = dy1*x1 + dy2*x2, dsin = -dy1*x2 + dy2*x1 (dcos/dsin may be NULL). */
void or_rope_fwd(const float* x, const float* cs, const float* sn, float* y, int64_t rows,
                 int64_t half, int dt) {
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; ++r) {
    for (int64_t c = 0; c < half; ++c) {
      const float x1 = x[r * 2 * half + c], x2 = x[r * 2 * half + half + c];
      const float co = cs[r * half + c], si = sn[r * half + c];
      y[r * 2 * half + c] = or_round(x1 * co - x2 * si, dt);
      y[r * 2 * half + half + c] = or_round(x2 * co + x1 * si, dt);
    }
  }
}

void or_rope_bwd(const float* dy, const float* x, const float* cs, const float* sn, float* dx,
                 float* dcos, float* dsin, int64_t rows, int64_t half, int dt) {
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; ++r) {
    for (int64_t c = 0; c < half; ++c) {
      const float d1 = dy[r * 2 * half + c], d2 = dy[r * 2 * half + half + c];
      const float x1 = x[r * 2 * half + c], x2 = x[r * 2 * half + half + c];
      const float co = cs[r * half + c], si = sn[r * half + c];
      dx[r * 2 * half + c] = or_round(d1 * co + d2 * si, dt);
      dx[r * 2 * half + half + c] = or_round(d2 * co - d1 * si, dt);
      if (dcos) dcos[r * half + c] = or_round(d1 * x1 + d2 * x2, dt);
      if (dsin) dsin[r * half + c] = or_round(-d1 * x2 + d2 * x1, dt);
    }
  }
}

/* ------------------------------------------------------------------ GEMM
 * src/tklab/kernels/matmul.py:130-154: C = A*B accumulated (here in double,
 * the reference in float32), cast to the output dtype at the end. */
void or_gemm(const float* a, const float* b, float* c, int64_t m, int64_t n, int64_t k, int dt) {
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < m; ++i) {
    double* acc = (double*)calloc((size_t)n, sizeof(double));
    for (int64_t p = 0; p < k; ++p) {
      const double av = a[i * k + p];
      const float* br = b + p * n;
      for (int64_t j = 0; j < n; ++j) acc[j] += av * br[j];
    }
    for (int64_t j = 0; j < n; ++j) c[i * n + j] = or_round((float)acc[j], dt);
    free(acc);
  }
}

/* ------------------------------------------------------------------ attention
 * Forward, src/tklab/kernels/flash_attention.py:90-117 and 248-264, per
 * (head, query row i), evaluated with the exact row maximum instead of the
 * running one:
 *   s_j = (q_i . k_j) * scale * log2(e) (masked to -inf for j > i if causal),
 *   m = max_j s_j, p_j = exp2(s_j - m), l = sum_j p_j,
 *   o_i = sum_j round_dt(p_j) v_j / l (rounded to dt), lse_i = m + log2(l).
 * q/k/v/o are [heads][seq][d]; lse is [heads][seq] (may be NULL). */
void or_attn_fwd(const float* q, const float* k, const float* v, float* o, float* lse,
                 int64_t heads, int64_t seq, int64_t d, float scale, int causal, int dt) {
  const float scale_log2 = (float)(scale * kLog2e);
#pragma omp parallel for collapse(2) schedule(dynamic, 4)
  for (int64_t h = 0; h < heads; ++h) {
    for (int64_t i = 0; i < seq; ++i) {
      const float* qi = q + (h * seq + i) * d;
      const float* kh = k + h * seq * d;
      const float* vh = v + h * seq * d;
      const int64_t nk = causal ? i + 1 : seq;
      float* s = (float*)__builtin_alloca(sizeof(float) * (size_t)nk);
      double* acc = (double*)__builtin_alloca(sizeof(double) * (size_t)d);
      float m = -INFINITY;
      for (int64_t j = 0; j < nk; ++j) {
        double dot = 0.0;
        for (int64_t t = 0; t < d; ++t) dot += (double)qi[t] * kh[j * d + t];
        s[j] = (float)dot * scale_log2;
        m = fmaxf(m, s[j]);
      }
      double l = 0.0;
      for (int64_t t = 0; t < d; ++t) acc[t] = 0.0;
      for (int64_t j = 0; j < nk; ++j) {
        const float p = exp2f(s[j] - m);
        l += p;
        const double pr = or_round(p, dt);
        for (int64_t t = 0; t < d; ++t) acc[t] += pr * vh[j * d + t];
      }
      float* oi = o + (h * seq + i) * d;
      for (int64_t t = 0; t < d; ++t) oi[t] = or_round((float)(acc[t] / l), dt);
      if (lse) lse[h * seq + i] = m + log2f((float)l);
    }
  }
}

/* Grouped-query attention decode: for each (batch b, query head h) one query
 * row q[b][h] attends to the first n_b = clamp(lens[b], 0, L) rows of the KV
 * head kv = h / (q_heads / kv_heads) (docs/research/gqa_decode_model.md,
 * "Semantic GQA mapping"), with exactly the arithmetic of or_attn_fwd for one
 * row (flash_attention.py:90-117, 248-264). n_b = 0 gives o = 0, lse = -inf.
 * q, o: [batch][q_heads][d]; k, v: [batch][kv_heads][L][d]; lens may be NULL
 * (n_b = L); lse: [batch][q_heads] (may be NULL). */
void or_gqa_decode(const float* q, const float* k, const float* v, const int32_t* lens, float* o,
                   float* lse, int64_t batch, int64_t q_heads, int64_t kv_heads, int64_t len,
                   int64_t d, float scale, int dt) {
  const float scale_log2 = (float)(scale * kLog2e);
  const int64_t group = q_heads / kv_heads;
#pragma omp parallel for collapse(2) schedule(dynamic, 4)
  for (int64_t b = 0; b < batch; ++b) {
    for (int64_t h = 0; h < q_heads; ++h) {
      int64_t nk = lens ? lens[b] : len;
      if (nk < 0) nk = 0;
      if (nk > len) nk = len;
      const float* qi = q + (b * q_heads + h) * d;
      const float* kh = k + (b * kv_heads + h / group) * len * d;
      const float* vh = v + (b * kv_heads + h / group) * len * d;
      float* oi = o + (b * q_heads + h) * d;
      if (nk == 0) {
        for (int64_t t = 0; t < d; ++t) oi[t] = 0.0f;
        if (lse) lse[b * q_heads + h] = -INFINITY;
        continue;
      }
      float* s = (float*)malloc(sizeof(float) * (size_t)nk);
      double* acc = (double*)malloc(sizeof(double) * (size_t)d);
      float m = -INFINITY;
      for (int64_t j = 0; j < nk; ++j) {
        double dot = 0.0;
        for (int64_t t = 0; t < d; ++t) dot += (double)qi[t] * kh[j * d + t];
        s[j] = (float)dot * scale_log2;
        m = fmaxf(m, s[j]);
      }
      double l = 0.0;
      for (int64_t t = 0; t < d; ++t) acc[t] = 0.0;
      for (int64_t j = 0; j < nk; ++j) {
        const float p = exp2f(s[j] - m);
        l += p;
        const double pr = or_round(p, dt);
        for (int64_t t = 0; t < d; ++t) acc[t] += pr * vh[j * d + t];
      }
      for (int64_t t = 0; t < d; ++t) oi[t] = or_round((float)(acc[t] / l), dt);
      if (lse) lse[b * q_heads + h] = m + log2f((float)l);
      free(s);
      free(acc);
    }
  }
}

/* Backward, src/tklab/kernels/flash_attention.py:383-395 (delta from the
 * stored O), 437-466 (dK, dV) and 512-533 (dQ):
 *   P_ij = exp2(s_ij - lse_i) (0 where masked), dV_j = sum_i round(P_ij) dO_i,
 *   dP_ij = dO_i . V_j, dS_ij = P_ij (dP_ij - delta_i),
 *   dK_j = scale * sum_i round(dS_ij) Q_i, dQ_i = scale * sum_j round(dS_ij) K_j.
 * `ds` is scratch of heads*seq*seq floats (0 where masked). */
void or_attn_bwd(const float* q, const float* k, const float* v, const float* o, const float* dout,
                 const float* lse, float* dq, float* dk, float* dv, float* ds, int64_t heads,
                 int64_t seq, int64_t d, float scale, int causal, int dt) {
  const float scale_log2 = (float)(scale * kLog2e);
#pragma omp parallel for schedule(dynamic, 1)
  for (int64_t h = 0; h < heads; ++h) {
    const float* qh = q + h * seq * d;
    const float* kh = k + h * seq * d;
    const float* vh = v + h * seq * d;
    const float* oh = o + h * seq * d;
    const float* doh = dout + h * seq * d;
    float* dsh = ds + h * seq * seq;
    float* dvh = dv + h * seq * d;
    double* accv = (double*)calloc((size_t)(seq * d), sizeof(double));
    for (int64_t i = 0; i < seq; ++i) {
      double delta = 0.0;
      for (int64_t t = 0; t < d; ++t) delta += (double)oh[i * d + t] * doh[i * d + t];
      const float di = (float)delta;
      for (int64_t j = 0; j < seq; ++j) {
        if (causal && j > i) {
          dsh[i * seq + j] = 0.0f;
          continue;
        }
        double dot = 0.0, dp = 0.0;
        for (int64_t t = 0; t < d; ++t) {
          dot += (double)qh[i * d + t] * kh[j * d + t];
          dp += (double)doh[i * d + t] * vh[j * d + t];
        }
        const float p = exp2f((float)dot * scale_log2 - lse[h * seq + i]);
        const double pr = or_round(p, dt);
        for (int64_t t = 0; t < d; ++t) accv[j * d + t] += pr * doh[i * d + t];
        dsh[i * seq + j] = p * ((float)dp - di);
      }
    }
    for (int64_t t = 0; t < seq * d; ++t) dvh[t] = or_round((float)accv[t], dt);
    free(accv);
    /* dQ_i = scale * sum_j round(dS_ij) K_j */
    for (int64_t i = 0; i < seq; ++i) {
      for (int64_t t = 0; t < d; ++t) {
        double acc = 0.0;
        for (int64_t j = 0; j < seq; ++j) acc += (double)or_round(dsh[i * seq + j], dt) * kh[j * d + t];
        dq[(h * seq + i) * d + t] = or_round((float)acc * scale, dt);
      }
    }
    /* dK_j = scale * sum_i round(dS_ij) Q_i */
    for (int64_t j = 0; j < seq; ++j) {
      for (int64_t t = 0; t < d; ++t) {
        double acc = 0.0;
        for (int64_t i = 0; i < seq; ++i) acc += (double)or_round(dsh[i * seq + j], dt) * qh[i * d + t];
        dk[(h * seq + j) * d + t] = or_round((float)acc * scale, dt);
      }
    }
  }
}
