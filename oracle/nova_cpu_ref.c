/*
 * nova_cpu_ref -- CPU oracle for the Nova GPU matmul / reduction path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file restates, in plain C, what Nova's CPU
 * pipeline `nova-opt-pipeline` (lib/Pipeline/Pipeline.cpp:61-187) computes
 * for the hot ops.  Only tests/, __graft_entry__.smoke() and the bench's
 * cpu_baseline leg load it, and only as the checker or as the timed CPU
 * baseline.  The product path (libnova_hip) never calls into it.
 *
 * The reference cannot be built here (it needs MLIR/LLVM 21.1.6 at
 * a832a5222e489298337fbb5876f8dcaf072c5cca; no MLIR is installed and there
 * is no network), so oracle/_ref stays empty and this restatement is pinned
 * by the reference's own known-answer test (test/wrapper.c:94-100), closed
 * forms, invariants and f64 brute force (tests/test_oracle.py).
 *
 * Arithmetic conventions that follow from the reference pipeline:
 *   - no fast-math flags anywhere and MathUpliftToFMA (Pipeline.cpp:145) only
 *     fires on `contract` ops, which Nova never emits: every mulf/addf is a
 *     separately rounded f32 operation.  Build with -ffp-contract=off.
 *   - the CPU pipeline is single threaded (affine-parallelize produces
 *     scf.parallel, lowered to sequential loops, Pipeline.cpp:135, 165):
 *     every reduction runs sequentially in index order.
 *   - math.exp / math.log / math.tanh are libm calls; math.rsqrt lowers to
 *     1 / sqrt (ConvertMathToLLVM, Pipeline.cpp:173).
 *
 * dtype codes: 0 = f32, 1 = bf16 (uint16 bits), 2 = f16 (uint16 bits).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* ---- dtype adapters (NovaCastOpLowering, NovaToLinalgGeneric.cpp:37-85):
 *      widening is arith.extf (exact), narrowing arith.truncf (RNE).   ---- */

float nova_ref_bf16_to_f32(uint16_t h) {
  uint32_t u = (uint32_t)h << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

uint16_t nova_ref_f32_to_bf16(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

float nova_ref_f16_to_f32(uint16_t h) {
  uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  uint32_t e = (h >> 10) & 0x1fu;
  uint32_t m = h & 0x3ffu;
  uint32_t u;
  if (e == 0) {
    if (m == 0) {
      u = sign;
    } else { /* subnormal: normalise */
      int sh = 0;
      while (!(m & 0x400u)) { m <<= 1; ++sh; }
      m &= 0x3ffu;
      u = sign | ((uint32_t)(127 - 15 - sh + 1) << 23) | (m << 13);
    }
  } else if (e == 31) {
    u = sign | 0x7f800000u | (m << 13);
  } else {
    u = sign | ((e + 127 - 15) << 23) | (m << 13);
  }
  float f;
  memcpy(&f, &u, 4);
  return f;
}

uint16_t nova_ref_f32_to_f16(float f) {
  uint32_t x;
  memcpy(&x, &f, 4);
  uint32_t sign = (x >> 16) & 0x8000u;
  uint32_t ax = x & 0x7fffffffu;
  if (ax > 0x7f800000u) return (uint16_t)(sign | 0x7e00u);
  if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);
  if (ax < 0x38800000u) {
    if (ax < 0x33000000u) return (uint16_t)sign;
    uint32_t e = ax >> 23;
    uint32_t m = (ax & 0x7fffffu) | 0x800000u;
    uint32_t shift = 126 - e;
    uint32_t r = m >> shift;
    uint32_t rem = m & ((1u << shift) - 1);
    uint32_t half = 1u << (shift - 1);
    if (rem > half || (rem == half && (r & 1))) r++;
    return (uint16_t)(sign | r);
  }
  uint32_t r = ax - 0x38000000u;
  uint32_t lsb = (r >> 13) & 1u;
  r += 0xfffu + lsb;
  return (uint16_t)(sign | (r >> 13));
}

static inline float load_as_f32(const void *p, int dt, int64_t i) {
  if (dt == 0) return ((const float *)p)[i];
  if (dt == 1) return nova_ref_bf16_to_f32(((const uint16_t *)p)[i]);
  return nova_ref_f16_to_f32(((const uint16_t *)p)[i]);
}

static inline void store_from_f32(void *p, int dt, int64_t i, float v) {
  if (dt == 0) ((float *)p)[i] = v;
  else if (dt == 1) ((uint16_t *)p)[i] = nova_ref_f32_to_bf16(v);
  else ((uint16_t *)p)[i] = nova_ref_f32_to_f16(v);
}

/* Round-trip a value through the output dtype (what the reference returns). */
static inline float round_to(int dt, float v) {
  if (dt == 1) return nova_ref_bf16_to_f32(nova_ref_f32_to_bf16(v));
  if (dt == 2) return nova_ref_f16_to_f32(nova_ref_f32_to_f16(v));
  return v;
}

/* ---- GELU, tanh form (NovaGeluForwardPattern, NovaToLinalgGeneric.cpp:
 *      1277-1337, op order of :1310-1331, f32 constants).              ---- */
float nova_ref_gelu_f32(float x) {
  const float c0 = 4.471500e-02f;
  const float k = 0.7978845608028654f;
  float x2 = x * x;
  float x3 = x2 * x;
  float cubic = c0 * x3;
  float inner = x + cubic;
  float scaled = k * inner;
  float t = tanhf(scaled);
  float one_pt = 1.0f + t;
  float half_x = 0.5f * x;
  return half_x * one_pt;
}

void nova_ref_gelu_array(const float *x, float *y, int64_t n) {
  for (int64_t i = 0; i < n; ++i) y[i] = nova_ref_gelu_f32(x[i]);
}

/* ---- One output element of the contraction.
 * linalg.matmul / linalg.batch_matmul body (NovaToLinalg.cpp:1040, 1045):
 *   C += extf(A) * extf(B) in the output (f32) type, k ascending, starting
 *   from the zero fill (NovaToLinalg.cpp:971) or, after FuseMatmulBias
 *   (FuseMatmulBias.cpp:95-199, accumulator init at :184-188), from bias[j].
 * nova.linear: input . weight + bias (NovaToLinalgGeneric.cpp:1623-1822),
 * followed here by the optional nova.gelu and the final nova.cast.      ---- */
static inline float dot_elem(const void *A, int adt, int64_t a0, int64_t sak,
                             const void *B, int bdt, int64_t b0, int64_t sbk,
                             int64_t K, float init) {
  float acc = init;
  for (int64_t k = 0; k < K; ++k) {
    float a = load_as_f32(A, adt, a0 + k * sak);
    float b = load_as_f32(B, bdt, b0 + k * sbk);
    float p = a * b;
    acc = acc + p;
  }
  return acc;
}

/*
 * Dense or strided GEMM over a batch, loop nest (b, i, j, k) with k
 * innermost, as linalg->affine lowering emits it (Pipeline.cpp:130).
 * Strides are in elements.  C is dense [batch, M, N] of dtype cdt.
 * epilogue: 0 = none, 1 = bias (accumulator init), 2 = bias then GELU,
 *           3 = GELU without bias.
 */
int nova_ref_gemm(const void *A, int adt, int64_t sab, int64_t sam, int64_t sak,
                  const void *B, int bdt, int64_t sbb, int64_t sbk, int64_t sbn,
                  const void *bias, int biasdt, int epilogue, void *C, int cdt,
                  int64_t batch, int64_t M, int64_t N, int64_t K) {
  if (!A || !B || !C || batch < 0 || M < 0 || N < 0 || K < 0) return -1;
  if ((epilogue == 1 || epilogue == 2) && !bias) return -1;
  for (int64_t b = 0; b < batch; ++b)
    for (int64_t i = 0; i < M; ++i)
      for (int64_t j = 0; j < N; ++j) {
        float init = 0.0f;
        if (epilogue == 1 || epilogue == 2) init = load_as_f32(bias, biasdt, j);
        float v = dot_elem(A, adt, b * sab + i * sam, sak, B, bdt,
                           b * sbb + j * sbn, sbk, K, init);
        if (epilogue == 2 || epilogue == 3) v = nova_ref_gelu_f32(v);
        store_from_f32(C, cdt, (b * M + i) * N + j, v);
      }
  return 0;
}

/*
 * linalg.matmul / batch_matmul with a bf16 or f16 outs operand (cdt == adt ==
 * bdt): the named op's body C += A * B is evaluated in the outs type, so the
 * product and each partial sum are rounded to it (cast_signed of a same-type
 * operand is the operand itself).  NovaMatmulOpLowering creates this form
 * for an f16 x f16 nova.matmul, whose inferred result type is f16
 * (NovaToLinalg.cpp:1027-1049, NovaOps.cpp:1198), and nova.linear for
 * narrow operands (NovaToLinalgGeneric.cpp:1623-1822), whose bias then
 * initialises the accumulator (FuseMatmulBias.cpp:184-188; epilogue 1, bias
 * of dtype cdt).  x86 has no bf16 / f16 arithmetic, so LLVM evaluates each
 * operation in f32 and rounds it back; that is what this does.
 */
int nova_ref_gemm_acc_out(const void *A, const void *B, int64_t sab, int64_t sam, int64_t sak,
                          int64_t sbb, int64_t sbk, int64_t sbn, const void *bias,
                          int epilogue, void *C, int cdt, int64_t batch, int64_t M,
                          int64_t N, int64_t K) {
  if (!A || !B || !C || batch < 0 || M < 0 || N < 0 || K < 0) return -1;
  if (cdt != 1 && cdt != 2) return -1;
  if (epilogue != 0 && epilogue != 1) return -1;
  if (epilogue == 1 && !bias) return -1;
  for (int64_t b = 0; b < batch; ++b)
    for (int64_t i = 0; i < M; ++i)
      for (int64_t j = 0; j < N; ++j) {
        float acc = epilogue == 1 ? load_as_f32(bias, cdt, j) : 0.0f;
        for (int64_t k = 0; k < K; ++k) {
          float a = load_as_f32(A, cdt, b * sab + i * sam + k * sak);
          float w = load_as_f32(B, cdt, b * sbb + k * sbk + j * sbn);
          float p = round_to(cdt, a * w);
          acc = round_to(cdt, acc + p);
        }
        store_from_f32(C, cdt, (b * M + i) * N + j, acc);
      }
  return 0;
}

/*
 * linalg.matmul / linalg.batch_matmul whose outs holds data (a function
 * argument, as in test/pipeline-tests/02_matmul_aligned.mlir:15-19): the
 * named op's body C += A * B runs from each element's value in C, k
 * ascending (the loop nest of nova_ref_gemm; NovaMatmulOpLowering's own
 * linalg ops start from a zero fill instead, NovaToLinalg.cpp:1031-1049).
 * C is dense [batch, M, N], read as the initial value and overwritten.
 * cdt 0 (f32): operands extended to f32 (adt, bdt any float type), f32
 * products and sums.  cdt 1 / 2 (bf16 / f16, == adt == bdt): every product
 * and partial sum rounded to cdt, as in nova_ref_gemm_acc_out.
 */
int nova_ref_gemm_accumulate(const void *A, int adt, int64_t sab, int64_t sam, int64_t sak,
                             const void *B, int bdt, int64_t sbb, int64_t sbk, int64_t sbn,
                             void *C, int cdt, int64_t batch, int64_t M, int64_t N, int64_t K) {
  if (!A || !B || !C || batch < 0 || M < 0 || N < 0 || K < 0) return -1;
  if (cdt != 0 && (cdt != adt || cdt != bdt || (cdt != 1 && cdt != 2))) return -1;
  for (int64_t b = 0; b < batch; ++b)
    for (int64_t i = 0; i < M; ++i)
      for (int64_t j = 0; j < N; ++j) {
        const int64_t c = (b * M + i) * N + j;
        float v;
        if (cdt == 0) {
          v = dot_elem(A, adt, b * sab + i * sam, sak, B, bdt, b * sbb + j * sbn, sbk, K,
                       load_as_f32(C, 0, c));
        } else {
          float acc = load_as_f32(C, cdt, c);
          for (int64_t k = 0; k < K; ++k) {
            float a = load_as_f32(A, cdt, b * sab + i * sam + k * sak);
            float w = load_as_f32(B, cdt, b * sbb + k * sbk + j * sbn);
            float p = round_to(cdt, a * w);
            acc = round_to(cdt, acc + p);
          }
          v = acc;
        }
        store_from_f32(C, cdt, c, v);
      }
  return 0;
}

/*
 * Same arithmetic as nova_ref_gemm for a list of output coordinates
 * idx[3*t + {0,1,2}] = (b, i, j).  out[t] receives the value the reference
 * would store, widened back to f32 (so bf16/f16 outputs are already rounded).
 */
int nova_ref_gemm_sampled(const void *A, int adt, int64_t sab, int64_t sam,
                          int64_t sak, const void *B, int bdt, int64_t sbb,
                          int64_t sbk, int64_t sbn, const void *bias,
                          int biasdt, int epilogue, int cdt, int64_t K,
                          const int64_t *idx, int64_t count, float *out) {
  if (!A || !B || !idx || !out || count < 0 || K < 0) return -1;
  if ((epilogue == 1 || epilogue == 2) && !bias) return -1;
  for (int64_t t = 0; t < count; ++t) {
    int64_t b = idx[3 * t], i = idx[3 * t + 1], j = idx[3 * t + 2];
    float init = 0.0f;
    if (epilogue == 1 || epilogue == 2) init = load_as_f32(bias, biasdt, j);
    float v = dot_elem(A, adt, b * sab + i * sam, sak, B, bdt,
                       b * sbb + j * sbn, sbk, K, init);
    if (epilogue == 2 || epilogue == 3) v = nova_ref_gelu_f32(v);
    out[t] = round_to(cdt, v);
  }
  return 0;
}

/*
 * LayerNorm over the last dim (NovaLayerNormPattern,
 * NovaToLinalgGeneric.cpp:1997-2126):
 *   S = sum x, Q = sum x*x      (one sequential pass, :2064-2077)
 *   mean = S*invD; var = Q*invD - mean*mean; rstd = rsqrt(var + eps)
 *   y = ((x - mean) * rstd) * gamma + beta            (:2101-2113)
 * invD = 1.0f / (float)D (:2026).  Results (y, S, rstd) (:2123).
 * The op hard-codes eps = 1e-5 (:2025); eps is a parameter here so the
 * boundary can carry it, and callers pass 1e-5.
 */
int nova_ref_layer_norm_f32(const float *x, const float *gamma,
                            const float *beta, float *y, float *mean_sum,
                            float *rstd_out, int64_t rows, int64_t D,
                            float eps) {
  if (!x || !gamma || !beta || !y || rows < 0 || D <= 0) return -1;
  const float invD = 1.0f / (float)D;
  for (int64_t r = 0; r < rows; ++r) {
    const float *xr = x + r * D;
    float s = 0.0f, q = 0.0f;
    for (int64_t d = 0; d < D; ++d) {
      s = xr[d] + s;
      float sq = xr[d] * xr[d];
      q = sq + q;
    }
    float mean = s * invD;
    float sq_mean = q * invD;
    float mean_sq = mean * mean;
    float var = sq_mean - mean_sq;
    float var_eps = var + eps;
    float rstd = 1.0f / sqrtf(var_eps);
    float *yr = y + r * D;
    for (int64_t d = 0; d < D; ++d) {
      float diff = xr[d] - mean;
      float norm = diff * rstd;
      float scaled = norm * gamma[d];
      yr[d] = scaled + beta[d];
    }
    if (mean_sum) mean_sum[r] = s;
    if (rstd_out) rstd_out[r] = rstd;
  }
  return 0;
}

/*
 * Full MEAN over a 1-D vector (lowerFullReduceMeanToSCF,
 * NovaToLinalg.cpp:1974-2126): 64 blocks (:2003) each sum a contiguous chunk
 * of ceil(n/64) elements sequentially (end clamped to n), then the 64
 * partials are summed sequentially and divided by (float)n.
 */
float nova_ref_mean_f32(const float *v, int64_t n) {
  const int64_t blocks = 64;
  const int64_t per = (n + blocks - 1) / blocks;
  float partial[64];
  for (int64_t b = 0; b < blocks; ++b) {
    int64_t start = b * per;
    int64_t end = start + per;
    if (end > n) end = n;
    float s = 0.0f;
    for (int64_t i = start; i < end; ++i) s = s + v[i];
    partial[b] = s;
  }
  float total = 0.0f;
  for (int64_t b = 0; b < blocks; ++b) total = total + partial[b];
  return total / (float)n;
}

/*
 * Softmax cross-entropy (NovaSceForwardLowering,
 * NovaToLinalgGeneric.cpp:801-1010):
 *   mx  = max_c x                                   (maximumf, -inf init)
 *   sum = sum_c exp(x - mx)                         (sequential)
 *   lse = log(max(sum, 1e-7))                       (:881)
 *   softmax = exp(x - mx) / max(sum, 1e-7)
 *   loss_r  = lse - (x[label] - mx)                 (gather at :964)
 *   loss    = MEAN_r loss_r                         (:992, 64-chunk mean)
 * Labels are i32 here (the lowering zero-extends narrower ints first).
 * A label outside [0, C) has no defined value in the reference (the gather
 * reads out of bounds); the oracle returns -2 for it.
 */
int nova_ref_sce_f32(const float *logits, const int32_t *labels, int64_t rows,
                     int64_t C, float *softmax, float *loss_rows,
                     float *loss) {
  if (!logits || !labels || rows <= 0 || C <= 0) return -1;
  float *lr = loss_rows;
  float *tmp = NULL;
  if (!lr) {
    tmp = (float *)malloc((size_t)rows * sizeof(float));
    if (!tmp) return -1;
    lr = tmp;
  }
  const float eps = 1.0e-7f;
  for (int64_t r = 0; r < rows; ++r) {
    const float *xr = logits + r * C;
    float mx = -INFINITY;
    for (int64_t c = 0; c < C; ++c) {
      float v = xr[c];
      mx = (v != v || mx != mx) ? NAN : (v > mx ? v : mx);
    }
    float sum = 0.0f;
    for (int64_t c = 0; c < C; ++c) {
      float sh = xr[c] - mx;
      sum = sum + expf(sh);
    }
    float safe = sum > eps ? sum : eps;
    if (sum != sum) safe = sum;
    float lse = logf(safe);
    if (softmax) {
      float *sr = softmax + r * C;
      for (int64_t c = 0; c < C; ++c) sr[c] = expf(xr[c] - mx) / safe;
    }
    int32_t t = labels[r];
    if (t < 0 || (int64_t)t >= C) {
      free(tmp);
      return -2;
    }
    float shifted = xr[t] - mx;
    lr[r] = lse - shifted;
  }
  if (loss) *loss = nova_ref_mean_f32(lr, rows);
  free(tmp);
  return 0;
}

/*
 * Softmax cross-entropy backward (NovaSceBackwardLowering,
 * NovaToLinalgGeneric.cpp:1012-1137) for rank 2 with the class dim last:
 *   diff = softmax with -1.0 scatter-added at (r, label_r)      (:1102-1113)
 *   grad = diff * invN, invN = 1.0 / N formed in double and rounded to f32
 *          by getFloatAttr (:1121-1125), N = product of the non-class dims
 *          = rows (:1054-1063), one f32 multiply per element (:1127-1128).
 * Elements off the label are softmax * invN (scatter_add leaves them as is).
 * A label outside [0, C) has no defined result in the reference (the
 * scatter index leaves the row); the oracle returns -2 for it.
 */
int nova_ref_sce_backward_f32(const float *softmax, const int32_t *labels,
                              int64_t rows, int64_t C, float *grad) {
  if (!softmax || !labels || !grad || rows <= 0 || C <= 0) return -1;
  const float invN = (float)(1.0 / (double)rows);
  for (int64_t r = 0; r < rows; ++r) {
    const int32_t t = labels[r];
    if (t < 0 || (int64_t)t >= C) return -2;
    const float *sr = softmax + r * C;
    float *gr = grad + r * C;
    for (int64_t c = 0; c < C; ++c) {
      float d = sr[c];
      if (c == t) d = d + -1.0f;
      gr[c] = d * invN;
    }
  }
  return 0;
}

/*
 * LayerNorm backward (NovaLayerNormBackwardPattern,
 * NovaToLinalgGeneric.cpp:2128-2371): given gy, x, gamma and the forward's
 * saved (mean_sum S, rstd), with invD = 1.0f / (float)D (:2159):
 *   gyGamma = gy * gamma; mean = S * invD; xHat = (x - mean) * rstd
 *   s1 = sum_d gyGamma, s2 = sum_d gyGamma * xHat   (sequential over d,
 *                                                    :2236-2258)
 *   dx = ((gyGamma - s1*invD) - xHat * (s2*invD)) * rstd        (:2264-2288)
 *   dgamma[d] = sum_r gy * xHat, dbeta[d] = sum_r gy  (sequential over rows,
 *                                                    :2345-2366)
 * Any of dx, dgamma, dbeta may be NULL.
 */
int nova_ref_layer_norm_backward_f32(const float *gy, const float *x,
                                     const float *gamma, const float *mean_sum,
                                     const float *rstd, float *dx,
                                     float *dgamma, float *dbeta, int64_t rows,
                                     int64_t D) {
  if (!gy || !x || !gamma || !mean_sum || !rstd || rows < 0 || D <= 0) return -1;
  const float invD = 1.0f / (float)D;
  if (dx) {
    for (int64_t r = 0; r < rows; ++r) {
      const float *gr = gy + r * D, *xr = x + r * D;
      const float mean = mean_sum[r] * invD;
      const float rs = rstd[r];
      float s1 = 0.0f, s2 = 0.0f;
      for (int64_t d = 0; d < D; ++d) {
        float gg = gr[d] * gamma[d];
        float diff = xr[d] - mean;
        float xh = diff * rs;
        float ggx = gg * xh;
        s1 = gg + s1;
        s2 = ggx + s2;
      }
      const float ms1 = s1 * invD, ms2 = s2 * invD;
      float *dr = dx + r * D;
      for (int64_t d = 0; d < D; ++d) {
        float gg = gr[d] * gamma[d];
        float diff = xr[d] - mean;
        float xh = diff * rs;
        float t1 = gg - ms1;
        float t2 = xh * ms2;
        float t3 = t1 - t2;
        dr[d] = t3 * rs;
      }
    }
  }
  if (dgamma || dbeta) {
    /* Row-outer traversal with one accumulator per column: each column
     * still sums its rows in order (the reference's loop nest), only the
     * memory walk is row-major. */
    float *ag = (float *)calloc((size_t)D, sizeof(float));
    float *ab = (float *)calloc((size_t)D, sizeof(float));
    if (!ag || !ab) {
      free(ag);
      free(ab);
      return -1;
    }
    for (int64_t r = 0; r < rows; ++r) {
      const float mean = mean_sum[r] * invD;
      const float rs = rstd[r];
      for (int64_t d = 0; d < D; ++d) {
        float diff = x[r * D + d] - mean;
        float xh = diff * rs;
        float gxh = gy[r * D + d] * xh;
        ag[d] = ag[d] + gxh;
        ab[d] = ab[d] + gy[r * D + d];
      }
    }
    if (dgamma) memcpy(dgamma, ag, (size_t)D * sizeof(float));
    if (dbeta) memcpy(dbeta, ab, (size_t)D * sizeof(float));
    free(ag);
    free(ab);
  }
  return 0;
}

/*
 * Column sums out[c] = sum_r in[r, c], sequential over rows in the
 * accumulator's f32 (the grad_bias reduction of NovaLinearBackwardPattern,
 * NovaToLinalgGeneric.cpp:1970-1989, body in + acc at :1861-1865).  `in` is [rows, cols]
 * of dtype dt with row stride ld (elements).
 */
int nova_ref_col_sum(const void *in, int dt, int64_t rows, int64_t cols,
                     int64_t ld, float *out) {
  if (!in || !out || rows < 0 || cols < 0) return -1;
  /* Row-outer walk, one accumulator per column, rows in order. */
  for (int64_t c = 0; c < cols; ++c) out[c] = 0.0f;
  for (int64_t r = 0; r < rows; ++r)
    for (int64_t c = 0; c < cols; ++c) out[c] = load_as_f32(in, dt, r * ld + c) + out[c];
  return 0;
}

/* ==== Program glue: the ops a whole training step needs around the hot
 *      ops (the reference's GPT step ltest/test.mlir uses each one).  ==== */

/* Index element: narrow integers zero-extended (arith.extui,
 * NovaToLinalgGeneric.cpp:2434-2449 for gather, NovaToLinalg.cpp:1240-1244
 * for scatter_add), i32 / i64 as signed indices.
 * idx_dt: 3 = i32, 4 = i64, 5 = i16. */
static int64_t load_index(const void *idx, int dt, int64_t i) {
  if (dt == 5) return (int64_t)((const uint16_t *)idx)[i];
  if (dt == 3) return (int64_t)((const int32_t *)idx)[i];
  return ((const int64_t *)idx)[i];
}

/* nova.add / sub / mul / div (Nova_BinaryOp, NovaOps.td:600-700): one
 * IEEE f32 operation per element over operands already broadcast to the
 * result shape (dense, n elements).  op: 0 add, 1 sub, 2 mul, 3 div. */
int nova_ref_binary_f32(const float *a, const float *b, float *c, int64_t n, int op) {
  if (!a || !b || !c || n < 0 || op < 0 || op > 3) return -1;
  for (int64_t i = 0; i < n; ++i) {
    const float x = a[i], y = b[i];
    c[i] = op == 0 ? x + y : op == 1 ? x - y : op == 2 ? x * y : x / y;
  }
  return 0;
}

/* nova.gelu_backward (NovaGeluBackwardPattern, NovaToLinalgGeneric.cpp:
 * 1339-1425), the generic body of :1383-1420 in its operation order:
 * x2 = x*x; x3 = x2*x; cubic = 0.044715*x3; inner = x + cubic;
 * gx = 0.797884583*inner; poly = 1 + x2*0.134145; dgx = poly*0.797884583;
 * t = tanh(gx); term1 = 0.5*(1 + t); term2 = 0.5*(x*(dgx*(1 - t*t)));
 * result = grad_out * (term1 + term2). */
float nova_ref_gelu_backward_f32(float go, float x) {
  const float k = 0.797884583f;
  float x2 = x * x;
  float x3 = x2 * x;
  float cubic = 4.471500e-02f * x3;
  float inner = x + cubic;
  float gx = k * inner;
  float xsq_c = x2 * 0.134145f;
  float poly = 1.0f + xsq_c;
  float dgx = poly * k;
  float t = tanhf(gx);
  float t2 = t * t;
  float one_pt = 1.0f + t;
  float term1 = 0.5f * one_pt;
  float om = 1.0f - t2;
  float t2a = dgx * om;
  float t2b = x * t2a;
  float term2 = 0.5f * t2b;
  float dg = term1 + term2;
  return go * dg;
}

void nova_ref_gelu_backward_array(const float *go, const float *x, float *out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = nova_ref_gelu_backward_f32(go[i], x[i]);
}

/* nova.gather along axis 0 (NovaGatherOpLowering, NovaToLinalgGeneric.cpp:
 * 2372-2471): out[i, :] = table[idx[i], :].  The reference's tensor.extract
 * of an index outside [0, V) is undefined; this restatement (and the GPU
 * kernel) gives a NaN row. */
int nova_ref_gather_f32(const float *table, int64_t V, int64_t D, const void *idx, int idx_dt,
                        int64_t n, float *out) {
  if (!table || !idx || !out || V < 0 || D < 0 || n < 0) return -1;
  for (int64_t i = 0; i < n; ++i) {
    const int64_t r = load_index(idx, idx_dt, i);
    for (int64_t c = 0; c < D; ++c)
      out[i * D + c] = (r >= 0 && r < V) ? table[r * D + c] : NAN;
  }
  return 0;
}

/* nova.scatter_add along axis 0 (NovaScatterAddOpLowering, NovaToLinalg.cpp:
 * 1086-1290), in place on out (the op's input): out[idx[i], :] += src[i, :]
 * for i ascending (the CPU pipeline runs the forall sequentially); indices
 * outside [0, V) are skipped (the scf.if of :1262-1276). */
int nova_ref_scatter_add_f32(float *out, int64_t V, int64_t D, const void *idx, int idx_dt,
                             int64_t n, const float *src) {
  if (!out || !idx || !src || V < 0 || D < 0 || n < 0) return -1;
  for (int64_t i = 0; i < n; ++i) {
    const int64_t r = load_index(idx, idx_dt, i);
    if (r < 0 || r >= V) continue;
    for (int64_t c = 0; c < D; ++c) out[r * D + c] = out[r * D + c] + src[i * D + c];
  }
  return 0;
}

/* nova.reduce<sum> over one dimension (Nova_ReduceOp, NovaOps.td:191-230):
 * x as [outer, n, inner], out[o, i] = sum_j x[o, j, i], j ascending from
 * 0.0f (a sequential linalg.reduce on the CPU pipeline). */
int nova_ref_reduce_sum_f32(const float *x, int64_t outer, int64_t n, int64_t inner,
                            float *out) {
  if (!x || !out || outer < 0 || n < 0 || inner < 0) return -1;
  for (int64_t o = 0; o < outer; ++o)
    for (int64_t i = 0; i < inner; ++i) {
      float acc = 0.0f;
      for (int64_t j = 0; j < n; ++j) acc = acc + x[(o * n + j) * inner + i];
      out[o * inner + i] = acc;
    }
  return 0;
}

/* Labels / indices to i32: zero-extension of narrow integers (the label
 * widening of NovaSceForwardLowering, NovaToLinalgGeneric.cpp:801-1010),
 * truncation of i64. */
int nova_ref_index_to_i32(const void *idx, int idx_dt, int64_t n, int32_t *out) {
  if (!idx || !out || n < 0) return -1;
  for (int64_t i = 0; i < n; ++i) out[i] = (int32_t)load_index(idx, idx_dt, i);
  return 0;
}
