/*
 * oracle.c -- CPU restatement of mlx-bun's quantized-inference hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker that the HIP library is
 * compared against.  Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it; the product path never routes through it.
 *
 * Every function cites the reference code whose semantics it restates
 * (paths relative to the mlx-bun repository).  The arithmetic itself lives in
 * MLX (mlx 0.31.2 / mlx-c 0.6.0, not vendored in the reference); where MLX's
 * published algorithm fixes a detail the reference does not show, the comment
 * says so.
 *
 * Numeric conventions:
 *   - T is the activation dtype: float16 (mlx_dtype 9), bfloat16 (12) or
 *     float32 (10).  T tensors cross this interface as raw 16-bit patterns
 *     (uint16) for f16/bf16 and as float for f32.
 *   - "fp32 reference" functions accumulate in double and return double, so
 *     they are at least as accurate as an fp32-accumulating implementation.
 *   - "_t" restatements reproduce the reference's rounding points (every MLX
 *     op on a T array rounds its result to T).
 *
 * Parity pins: tests/test_oracle_golden.py (reference golden vectors) and
 * tests/test_oracle_math.py (closed forms, invariants, independent numpy).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define DT_F16 9
#define DT_F32 10
#define DT_BF16 12

/* ------------------------------------------------------------------ dtypes */

static inline float bits_to_f32(uint32_t u) {
  float f;
  memcpy(&f, &u, 4);
  return f;
}
static inline uint32_t f32_to_bits(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return u;
}

static float bf16_to_f32(uint16_t h) { return bits_to_f32(((uint32_t)h) << 16); }

/* round-to-nearest-even, NaN preserved as quiet NaN */
static uint16_t f32_to_bf16(float f) {
  uint32_t u = f32_to_bits(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40);
  uint32_t lsb = (u >> 16) & 1u;
  u += 0x7fffu + lsb;
  return (uint16_t)(u >> 16);
}

static float f16_to_f32(uint16_t h) {
  uint32_t sign = (uint32_t)(h >> 15) << 31;
  uint32_t exp = (h >> 10) & 0x1f;
  uint32_t man = h & 0x3ff;
  if (exp == 0) {
    if (man == 0) return bits_to_f32(sign);
    /* subnormal: value = man * 2^-24 */
    float v = (float)man * 5.9604644775390625e-8f;
    return sign ? -v : v;
  }
  if (exp == 31) return bits_to_f32(sign | 0x7f800000u | (man << 13));
  return bits_to_f32(sign | ((exp + 112) << 23) | (man << 13));
}

/* round-to-nearest-even conversion float -> binary16 */
static uint16_t f32_to_f16(float f) {
  uint32_t u = f32_to_bits(f);
  uint32_t sign = (u >> 16) & 0x8000u;
  uint32_t a = u & 0x7fffffffu;
  if (a > 0x7f800000u) return (uint16_t)(sign | 0x7e00u);
  if (a >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* rounds to inf */
  if (a < 0x38800000u) {                                     /* subnormal/zero */
    /* value / 2^-24, rounded to nearest even integer */
    float v = bits_to_f32(a) * 16777216.0f;
    float r = nearbyintf(v); /* default rounding mode: nearest-even */
    return (uint16_t)(sign | (uint32_t)r);
  }
  uint32_t exp = ((a >> 23) - 112) << 10;
  uint32_t man = (a >> 13) & 0x3ffu;
  uint32_t rest = a & 0x1fffu;
  uint32_t h = exp | man;
  if (rest > 0x1000u || (rest == 0x1000u && (h & 1u))) h += 1; /* may carry into exp */
  return (uint16_t)(sign | h);
}

static float t_load(const void* p, int64_t i, int dtype) {
  if (dtype == DT_F32) return ((const float*)p)[i];
  uint16_t h = ((const uint16_t*)p)[i];
  return dtype == DT_BF16 ? bf16_to_f32(h) : f16_to_f32(h);
}

static void t_store(void* p, int64_t i, int dtype, float v) {
  if (dtype == DT_F32) {
    ((float*)p)[i] = v;
    return;
  }
  ((uint16_t*)p)[i] = dtype == DT_BF16 ? f32_to_bf16(v) : f32_to_f16(v);
}

/* round a float to the nearest T value (the result of any MLX op on T) */
static float t_round(float v, int dtype) {
  if (dtype == DT_F32) return v;
  if (dtype == DT_BF16) return bf16_to_f32(f32_to_bf16(v));
  return f16_to_f32(f32_to_f16(v));
}

static int dtype_ok(int dtype) { return dtype == DT_F16 || dtype == DT_BF16 || dtype == DT_F32; }
static int bits_ok(int bits) { return bits == 2 || bits == 4 || bits == 8; }

/* most negative finite T: the fill value quantizedSdpaUnfused uses for masked
 * scores (FINFO_MIN, src/model/gemma4-base.ts:1263-1267) */
static float finfo_min(int dtype) {
  if (dtype == DT_F16) return -65504.0f;
  if (dtype == DT_BF16) return -3.3895313892515355e38f;
  return -3.4028234663852886e38f;
}

void oracle_to_t(const float* in, int64_t n, int dtype, void* out) {
  for (int64_t i = 0; i < n; i++) t_store(out, i, dtype, in[i]);
}

void oracle_from_t(const void* in, int64_t n, int dtype, float* out) {
  for (int64_t i = 0; i < n; i++) out[i] = t_load(in, i, dtype);
}

/* --------------------------------------------------------------- quantize */

/*
 * mx.quantize(w, group_size, bits, mode="affine") as called by ops.quantize
 * (src/mlx/ops.ts:615-641) for every KV-cache append
 * (src/model/gemma4-base.ts:479-480, :1075-1076) and cache conversion
 * (:395-404, :892-903).
 *
 * Per group of `gs` consecutive elements along the last axis, in fp32:
 *   scale = max((max - min) / (2^bits - 1), 1e-7)
 *   side  = |min| > |max|;  scale = side ? scale : -scale;  edge = side ? min : max
 *   q0 = round(edge / scale)
 *   if q0 != 0: scale = edge / q0, bias = edge   else bias = 0
 *   code = clamp(round((w - bias) / scale), 0, 2^bits - 1)   (unrounded fp32 scale/bias)
 *   stored scale/bias = T(scale), T(bias)  (round-to-nearest-even)
 * `round` is round-half-away-from-zero: that is what reproduces every word of
 * goldens/rotating-kvq.bin (the reference's only quantize golden, produced by
 * scripts/regen-rotating-kvq-goldens.ts:51-72).  Codes pack little-endian:
 * element j of a uint32 occupies bits [j*bits, (j+1)*bits).
 * min/max are the true group extrema.
 */
int oracle_quantize(const float* w, int64_t rows, int64_t dim, int gs, int bits, int dtype,
                    uint32_t* packed, void* scales, void* biases) {
  if (!dtype_ok(dtype) || !bits_ok(bits) || gs <= 0 || dim % gs || gs % (32 / bits)) return 1;
  const float n_bins = (float)((1 << bits) - 1);
  const int per_word = 32 / bits;
  const int64_t groups = dim / gs;
  for (int64_t r = 0; r < rows; r++) {
    for (int64_t g = 0; g < groups; g++) {
      const float* x = w + r * dim + g * gs;
      float mn = x[0], mx = x[0];
      for (int i = 1; i < gs; i++) {
        mn = fminf(mn, x[i]);
        mx = fmaxf(mx, x[i]);
      }
      float scale = fmaxf((mx - mn) / n_bins, 1e-7f);
      int side = fabsf(mn) > fabsf(mx);
      scale = side ? scale : -scale;
      float edge = side ? mn : mx;
      float q0 = roundf(edge / scale);
      float bias = 0.0f;
      if (q0 != 0.0f) {
        scale = edge / q0;
        bias = edge;
      }
      t_store(scales, r * groups + g, dtype, scale);
      t_store(biases, r * groups + g, dtype, bias);
      for (int wi = 0; wi < gs / per_word; wi++) {
        uint32_t word = 0;
        for (int j = 0; j < per_word; j++) {
          float c = roundf((x[wi * per_word + j] - bias) / scale);
          c = fminf(fmaxf(c, 0.0f), n_bins);
          word |= ((uint32_t)c) << (j * bits);
        }
        packed[(r * dim + g * gs) / per_word + wi] = word;
      }
    }
  }
  return 0;
}

static inline uint32_t code_at(const uint32_t* row_words, int64_t d, int bits) {
  const int per_word = 32 / bits;
  uint32_t w = row_words[d / per_word];
  return (w >> ((d % per_word) * bits)) & ((1u << bits) - 1u);
}

/*
 * mx.dequantize (src/mlx/ops.ts:212-225): w = scale * code + bias per group
 * as one fused multiply-add in fp32, rounded once to T.  For T in {f16, bf16}
 * scale*code is exact in fp32, so fused and unfused evaluation agree; for
 * fp32 the fused form is what MLX's `scale * q + bias` compiles to.
 * Output is the T value widened to float.
 */
int oracle_dequantize(const uint32_t* packed, const void* scales, const void* biases, int dtype,
                      int64_t rows, int64_t dim, int gs, int bits, float* out) {
  if (!dtype_ok(dtype) || !bits_ok(bits) || dim % gs) return 1;
  const int64_t groups = dim / gs;
  const int64_t words = dim * bits / 32;
  for (int64_t r = 0; r < rows; r++) {
    for (int64_t d = 0; d < dim; d++) {
      float s = t_load(scales, r * groups + d / gs, dtype);
      float b = t_load(biases, r * groups + d / gs, dtype);
      float c = (float)code_at(packed + r * words, d, bits);
      out[r * dim + d] = t_round(fmaf(s, c, b), dtype);
    }
  }
  return 0;
}

/* exact dequantized value (double) of element d of a quantized row */
static inline double deq_exact(const uint32_t* row_words, const void* scales, const void* biases,
                               int64_t srow, int64_t d, int gs, int bits, int dtype, int64_t groups) {
  double s = t_load(scales, srow * groups + d / gs, dtype);
  double b = t_load(biases, srow * groups + d / gs, dtype);
  return s * (double)code_at(row_words, d, bits) + b;
}

/* ----------------------------------------------------------- quantized mm */

/*
 * mx.quantized_matmul (src/mlx/ops.ts:171-184, :760-775), fp32 reference.
 * x: [batch, M, K] float (T values); W batch wb = b / (batch / w_batch).
 * transpose=1: W [N, K] quantized along K, y = x @ deq(W)^T   (QuantizedLinear,
 *              src/model/gemma4-base.ts:120-158)
 * transpose=0: W [K, N] quantized along N, y = x @ deq(W)     (the P.V product
 *              of quantizedSdpaUnfused, :1332)
 * y: [batch, M, N] double.
 */
int oracle_qmm(const float* x, int64_t batch, int64_t M, int64_t K, const uint32_t* w,
               const void* scales, const void* biases, int dtype, int64_t w_batch, int64_t N,
               int gs, int bits, int transpose, double* y) {
  if (!dtype_ok(dtype) || !bits_ok(bits) || w_batch <= 0 || batch % w_batch) return 1;
  const int64_t rep = batch / w_batch;
  if (transpose) {
    if (K % gs) return 1;
    const int64_t groups = K / gs, words = K * bits / 32;
    double* wrow = (double*)malloc(sizeof(double) * K);
    for (int64_t b = 0; b < batch; b++) {
      const int64_t wb = b / rep;
      for (int64_t n = 0; n < N; n++) {
        const int64_t srow = wb * N + n;
        for (int64_t k = 0; k < K; k++)
          wrow[k] = deq_exact(w + srow * words, scales, biases, srow, k, gs, bits, dtype, groups);
        for (int64_t m = 0; m < M; m++) {
          const float* xr = x + (b * M + m) * K;
          double acc = 0.0;
          for (int64_t k = 0; k < K; k++) acc += (double)xr[k] * wrow[k];
          y[(b * M + m) * N + n] = acc;
        }
      }
    }
    free(wrow);
  } else {
    if (N % gs) return 1;
    const int64_t groups = N / gs, words = N * bits / 32;
    for (int64_t b = 0; b < batch; b++) {
      const int64_t wb = b / rep;
      for (int64_t m = 0; m < M; m++) {
        double* yr = y + (b * M + m) * N;
        for (int64_t n = 0; n < N; n++) yr[n] = 0.0;
        for (int64_t k = 0; k < K; k++) {
          const int64_t srow = wb * K + k;
          double xv = x[(b * M + m) * K + k];
          for (int64_t n = 0; n < N; n++)
            yr[n] += xv * deq_exact(w + srow * words, scales, biases, srow, n, gs, bits, dtype, groups);
        }
      }
    }
  }
  return 0;
}

/* ------------------------------------------------------------------- sdpa */

/*
 * Key-slot geometry shared by every SDPA entry point.
 *
 * The cache holds `cap` slots per (batch row, kv head).  Row b attends
 * `valid` logical positions j = 0..valid-1 (oldest first):
 *   valid = valid_len ? min(valid_len[b], cap) : n_kv
 *   slot(j) = ring_off ? (ring_off[b] - valid + j) mod cap : j
 * ring_off is the ring write index (the slot the next token goes to), so the
 * valid slots are the `valid` most recently written ones.  This restates the
 * rotating caches' fetch (RotatingQuantizedKVCache #activeSlices,
 * src/model/gemma4-base.ts:1096-1106) and the batched ring's per-row window
 * (buildBatchedRotatingMask, src/model/batched-rotating.ts:40-75, where every
 * row shares one ring index and left padding shortens `valid`).
 * Query row i of Lq sits at logical position valid - Lq + i (bottom-right
 * alignment, createCausalMask src/model/gemma4-base.ts:1595-1615):
 *   causal: j <= pos;  window > 0: pos < j + window.
 */
typedef struct {
  int B, Hq, Hkv, Lq, D;
  int64_t cap, n_kv;
  const int32_t* valid_len;
  const int32_t* ring_off;
  int causal, window;
  int gs, bits, dtype;
} geom_t;

static int64_t row_valid(const geom_t* g, int b) {
  if (!g->valid_len) return g->n_kv;
  int64_t v = g->valid_len[b];
  if (v < 0) v = 0;
  return v < g->cap ? v : g->cap;
}

static int64_t row_slot(const geom_t* g, int b, int64_t valid, int64_t j) {
  if (!g->ring_off) return j;
  int64_t s = ((int64_t)g->ring_off[b] - valid + j) % g->cap;
  return s < 0 ? s + g->cap : s;
}

static int allowed(const geom_t* g, int64_t valid, int i, int64_t j) {
  int64_t pos = valid - g->Lq + i;
  if (g->causal && j > pos) return 0;
  if (g->window > 0 && !(pos < j + g->window)) return 0;
  return 1;
}

/* q' = T(q * T(scale)); quantizedSdpaUnfused skips the multiply when scale==1
 * (src/model/gemma4-base.ts:1284-1286, weak-scalar rule src/mlx/ops.ts:47-60) */
static void scale_queries(const float* q, int64_t n, float scale, int dtype, float* out) {
  if (scale == 1.0f) {
    memcpy(out, q, sizeof(float) * n);
    return;
  }
  float st = t_round(scale, dtype);
  for (int64_t i = 0; i < n; i++) out[i] = t_round(q[i] * st, dtype);
}

static int geom_check(const geom_t* g) {
  if (!dtype_ok(g->dtype) || !bits_ok(g->bits) || g->D % g->gs || g->Hkv <= 0 || g->Hq % g->Hkv)
    return 1;
  if (g->Lq <= 0 || g->cap <= 0 || (!g->valid_len && (g->n_kv < 0 || g->n_kv > g->cap))) return 1;
  return 0;
}

/*
 * fp32 reference of quantizedSdpa (src/model/gemma4-base.ts:1560-1578):
 * softmax(q' . deq(K)^T + mask) . deq(V) with double accumulation, GQA by
 * q head h -> kv head h / (Hq / Hkv) (the [B,Hkv,nRep,L,D] reshape of :1290).
 * q: [B,Hq,Lq,D] float T-values; out: [B,Hq,Lq,D] double.  Rows with no
 * allowed key produce zeros.
 */
int oracle_sdpa(const float* q, int dtype, int B, int Hq, int Hkv, int Lq, int D,
                const uint32_t* kp, const void* ks, const void* kb, const uint32_t* vp,
                const void* vs, const void* vb, int64_t cap, int64_t n_kv,
                const int32_t* valid_len, const int32_t* ring_off, int causal, int window,
                float scale, int gs, int bits, double* out) {
  geom_t g = {B, Hq, Hkv, Lq, D, cap, n_kv, valid_len, ring_off, causal, window, gs, bits, dtype};
  if (geom_check(&g)) return 1;
  const int nrep = Hq / Hkv;
  const int64_t words = (int64_t)D * bits / 32, groups = D / gs;
  const int64_t qn = (int64_t)B * Hq * Lq * D;
  float* qs = (float*)malloc(sizeof(float) * qn);
  scale_queries(q, qn, scale, dtype, qs);
  int64_t maxv = 0;
  for (int b = 0; b < B; b++) {
    int64_t v = row_valid(&g, b);
    if (v > maxv) maxv = v;
  }
#pragma omp parallel
  {
    double* sc = (double*)malloc(sizeof(double) * (maxv > 0 ? maxv : 1));
    double* kd = (double*)malloc(sizeof(double) * D);
    double* acc = (double*)malloc(sizeof(double) * D);
#pragma omp for collapse(2) schedule(dynamic)
    for (int b = 0; b < B; b++) {
      for (int h = 0; h < Hq; h++) {
        const int kvh = h / nrep;
        const int64_t valid = row_valid(&g, b);
        const int64_t base = ((int64_t)b * Hkv + kvh) * cap;
        for (int i = 0; i < Lq; i++) {
          const float* qr = qs + (((int64_t)b * Hq + h) * Lq + i) * D;
          double m = -INFINITY;
          for (int64_t j = 0; j < valid; j++) {
            if (!allowed(&g, valid, i, j)) {
              sc[j] = -INFINITY;
              continue;
            }
            const int64_t row = base + row_slot(&g, b, valid, j);
            double s = 0.0;
            for (int d = 0; d < D; d++)
              s += (double)qr[d] * deq_exact(kp + row * words, ks, kb, row, d, gs, bits, dtype, groups);
            sc[j] = s;
            if (s > m) m = s;
          }
          for (int d = 0; d < D; d++) acc[d] = 0.0;
          double l = 0.0;
          if (m > -INFINITY) {
            for (int64_t j = 0; j < valid; j++) {
              if (sc[j] == -INFINITY) continue;
              double p = exp(sc[j] - m);
              l += p;
              const int64_t row = base + row_slot(&g, b, valid, j);
              for (int d = 0; d < D; d++)
                kd[d] = deq_exact(vp + row * words, vs, vb, row, d, gs, bits, dtype, groups);
              for (int d = 0; d < D; d++) acc[d] += p * kd[d];
            }
          }
          double* o = out + (((int64_t)b * Hq + h) * Lq + i) * D;
          for (int d = 0; d < D; d++) o[d] = l > 0.0 ? acc[d] / l : 0.0;
        }
      }
    }
    free(sc);
    free(kd);
    free(acc);
  }
  free(qs);
  return 0;
}

/* MLX quantized_matmul result for one (query, key) dot: fp32-dequantized
 * operands, wide accumulation, rounded to T */
static float qdot_t(const float* qr, const uint32_t* words_row, const void* s, const void* bsc,
                    int64_t row, int D, int gs, int bits, int dtype, int64_t groups) {
  double acc = 0.0;
  for (int d = 0; d < D; d++) acc += (double)qr[d] * deq_exact(words_row, s, bsc, row, d, gs, bits, dtype, groups);
  return t_round((float)acc, dtype);
}

/*
 * quantizedSdpaUnfused with the reference's rounding points
 * (src/model/gemma4-base.ts:1273-1340): scores = T(qmm(q', K)),
 * masked -> FINFO_MIN[T], probs = T(softmax_fp32(scores)) (precise softmax),
 * out = T(qmm(probs, V)).  Output: T values widened to float.
 */
int oracle_sdpa_unfused_t(const float* q, int dtype, int B, int Hq, int Hkv, int Lq, int D,
                          const uint32_t* kp, const void* ks, const void* kb, const uint32_t* vp,
                          const void* vs, const void* vb, int64_t cap, int64_t n_kv,
                          const int32_t* valid_len, const int32_t* ring_off, int causal, int window,
                          float scale, int gs, int bits, float* out) {
  geom_t g = {B, Hq, Hkv, Lq, D, cap, n_kv, valid_len, ring_off, causal, window, gs, bits, dtype};
  if (geom_check(&g)) return 1;
  const int nrep = Hq / Hkv;
  const int64_t words = (int64_t)D * bits / 32, groups = D / gs;
  const int64_t qn = (int64_t)B * Hq * Lq * D;
  float* qs = (float*)malloc(sizeof(float) * qn);
  scale_queries(q, qn, scale, dtype, qs);
  int64_t maxv = 1;
  for (int b = 0; b < B; b++) {
    int64_t v = row_valid(&g, b);
    if (v > maxv) maxv = v;
  }
  const float fill = finfo_min(dtype);
#pragma omp parallel
  {
    float* sc = (float*)malloc(sizeof(float) * maxv);
    double* acc = (double*)malloc(sizeof(double) * D);
#pragma omp for collapse(2) schedule(dynamic)
    for (int b = 0; b < B; b++) {
      for (int h = 0; h < Hq; h++) {
        const int kvh = h / nrep;
        const int64_t valid = row_valid(&g, b);
        const int64_t base = ((int64_t)b * Hkv + kvh) * cap;
        for (int i = 0; i < Lq; i++) {
          const float* qr = qs + (((int64_t)b * Hq + h) * Lq + i) * D;
          float m = -INFINITY;
          for (int64_t j = 0; j < valid; j++) {
            const int64_t row = base + row_slot(&g, b, valid, j);
            float s = qdot_t(qr, kp + row * words, ks, kb, row, D, gs, bits, dtype, groups);
            if (!allowed(&g, valid, i, j)) s = fill;
            sc[j] = s;
            if (s > m) m = s;
          }
          float l = 0.0f;
          for (int64_t j = 0; j < valid; j++) {
            sc[j] = expf(sc[j] - m);
            l += sc[j];
          }
          for (int64_t j = 0; j < valid; j++) sc[j] = t_round(sc[j] / l, dtype);
          for (int d = 0; d < D; d++) acc[d] = 0.0;
          for (int64_t j = 0; j < valid; j++) {
            const int64_t row = base + row_slot(&g, b, valid, j);
            for (int d = 0; d < D; d++)
              acc[d] += (double)sc[j] * deq_exact(vp + row * words, vs, vb, row, d, gs, bits, dtype, groups);
          }
          float* o = out + (((int64_t)b * Hq + h) * Lq + i) * D;
          for (int d = 0; d < D; d++) o[d] = t_round((float)acc[d], dtype);
        }
      }
    }
    free(sc);
    free(acc);
  }
  free(qs);
  return 0;
}

/*
 * quantizedSdpaTiled with the reference's rounding points
 * (src/model/gemma4-base.ts:1356-1521): FlashAttention-2 over 512-column key
 * chunks (FUSED_N_CHUNK, :1345) with the running max / sum / output kept as T
 * arrays, every elementwise op rounding to T.  Logical key order (no ring
 * geometry beyond slot mapping).  Output: T values widened to float.
 */
int oracle_sdpa_tiled_t(const float* q, int dtype, int B, int Hq, int Hkv, int Lq, int D,
                        const uint32_t* kp, const void* ks, const void* kb, const uint32_t* vp,
                        const void* vs, const void* vb, int64_t cap, int64_t n_kv,
                        const int32_t* valid_len, const int32_t* ring_off, int causal, int window,
                        float scale, int gs, int bits, int n_chunk, float* out) {
  geom_t g = {B, Hq, Hkv, Lq, D, cap, n_kv, valid_len, ring_off, causal, window, gs, bits, dtype};
  if (geom_check(&g) || n_chunk <= 0) return 1;
  const int nrep = Hq / Hkv;
  const int64_t words = (int64_t)D * bits / 32, groups = D / gs;
  const int64_t qn = (int64_t)B * Hq * Lq * D;
  float* qs = (float*)malloc(sizeof(float) * qn);
  scale_queries(q, qn, scale, dtype, qs);
  const float fill = finfo_min(dtype);
#define TR(x) t_round((x), dtype)
#pragma omp parallel
  {
    float* sc = (float*)malloc(sizeof(float) * n_chunk);
    float* oacc = (float*)malloc(sizeof(float) * D);
    double* dacc = (double*)malloc(sizeof(double) * D);
#pragma omp for collapse(2) schedule(dynamic)
    for (int b = 0; b < B; b++) {
      for (int h = 0; h < Hq; h++) {
        const int kvh = h / nrep;
        const int64_t valid = row_valid(&g, b);
        const int64_t base = ((int64_t)b * Hkv + kvh) * cap;
        for (int i = 0; i < Lq; i++) {
          const float* qr = qs + (((int64_t)b * Hq + h) * Lq + i) * D;
          float rowmax = 0.0f, rowsum = 0.0f;
          int first = 1;
          for (int64_t n0 = 0; n0 < valid; n0 += n_chunk) {
            int64_t n1 = n0 + n_chunk < valid ? n0 + n_chunk : valid;
            float cmax = -INFINITY;
            for (int64_t j = n0; j < n1; j++) {
              const int64_t row = base + row_slot(&g, b, valid, j);
              float s = qdot_t(qr, kp + row * words, ks, kb, row, D, gs, bits, dtype, groups);
              if (!allowed(&g, valid, i, j)) s = fill;
              sc[j - n0] = s;
              if (s > cmax) cmax = s;
            }
            float newmax = first ? cmax : (rowmax > cmax ? rowmax : cmax);
            float factor = first ? 0.0f : TR(expf(TR(rowmax - newmax)));
            double esum = 0.0;
            for (int64_t j = n0; j < n1; j++) {
              sc[j - n0] = TR(expf(TR(sc[j - n0] - newmax)));
              esum += sc[j - n0];
            }
            for (int d = 0; d < D; d++) dacc[d] = 0.0;
            for (int64_t j = n0; j < n1; j++) {
              const int64_t row = base + row_slot(&g, b, valid, j);
              for (int d = 0; d < D; d++)
                dacc[d] += (double)sc[j - n0] * deq_exact(vp + row * words, vs, vb, row, d, gs, bits, dtype, groups);
            }
            if (first) {
              rowsum = TR((float)esum);
              for (int d = 0; d < D; d++) oacc[d] = TR((float)dacc[d]);
              first = 0;
            } else {
              rowsum = TR(TR(factor * rowsum) + TR((float)esum));
              for (int d = 0; d < D; d++) oacc[d] = TR(TR(oacc[d] * factor) + TR((float)dacc[d]));
            }
            rowmax = newmax;
          }
          float* o = out + (((int64_t)b * Hq + h) * Lq + i) * D;
          for (int d = 0; d < D; d++) o[d] = valid > 0 ? TR(oacc[d] / rowsum) : 0.0f;
        }
      }
    }
    free(sc);
    free(oacc);
    free(dacc);
  }
#undef TR
  free(qs);
  return 0;
}
