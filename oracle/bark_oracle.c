/*
 * CPU oracle for the Conformer encoder hot path — TEST INFRASTRUCTURE ONLY.
 * See bark_oracle.h for the contract. Built with -ffp-contract=off so that the
 * only fused multiply-adds are the explicit ones the reference also fuses
 * (its AVX2 GEMM micro-kernel); every other `a*b + c` rounds twice, as Rust
 * does. Only tests/, smoke() and bench.py's cpu_baseline leg load this.
 */
#include "bark_oracle.h"

#include <immintrin.h>
#include <math.h>
#include <omp.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#define HIDDEN 1024
#define HEADS 8
#define HDIM 128
#define FFN 4096
#define PANEL 16
#define MR 6
#define BQ 256
#define TM 192
#define TN 128

static inline int div_ceil(int a, int b) { return (a + b - 1) / b; }
static inline int pad128(int n) { return (n + 127) & ~127; }

/* ------------------------------------------------------------------------- */
/* f32 <-> f16 / bf16.  f32->f16 is IEEE round-to-nearest-even with subnormals,
 * the behaviour of half::f16::from_f32 used by src/raw.rs:130-133. */
uint16_t bo_f32_to_f16(float v) {
  uint32_t x;
  memcpy(&x, &v, 4);
  uint32_t sign = (x >> 16) & 0x8000u;
  uint32_t ax = x & 0x7fffffffu;
  if (ax >= 0x7f800000u) { /* inf / nan */
    if (ax == 0x7f800000u) return (uint16_t)(sign | 0x7c00u);
    return (uint16_t)(sign | 0x7e00u | ((ax >> 13) & 0x3ffu));
  }
  if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* rounds to >= 65520 */
  int32_t exp = (int32_t)(ax >> 23) - 127;
  uint32_t mant = ax & 0x7fffffu;
  if (exp >= -14) { /* normal f16 */
    uint32_t h = ((uint32_t)(exp + 15) << 10) | (mant >> 13);
    uint32_t rem = mant & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h += 1u; /* carry may bump exp */
    return (uint16_t)(sign | h);
  }
  if (exp < -25) return (uint16_t)sign; /* below half the smallest subnormal */
  /* subnormal: value = m * 2^-24 */
  mant |= 0x800000u;
  int shift = 13 + (-14 - exp); /* mantissa bits dropped */
  uint32_t h = mant >> shift;
  uint32_t rem = mant & ((1u << shift) - 1u);
  uint32_t halfway = 1u << (shift - 1);
  if (rem > halfway || (rem == halfway && (h & 1u))) h += 1u;
  return (uint16_t)(sign | h);
}

float bo_f16_to_f32(uint16_t h) {
  uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
  uint32_t exp = (h >> 10) & 0x1fu;
  uint32_t mant = h & 0x3ffu;
  uint32_t x;
  if (exp == 0) {
    if (mant == 0) {
      x = sign;
    } else { /* subnormal: normalise */
      int e = -1;
      do {
        e++;
        mant <<= 1;
      } while ((mant & 0x400u) == 0);
      mant &= 0x3ffu;
      x = sign | ((uint32_t)(127 - 15 - e) << 23) | (mant << 13);
    }
  } else if (exp == 31) {
    x = sign | 0x7f800000u | (mant << 13);
  } else {
    x = sign | ((exp - 15 + 127) << 23) | (mant << 13);
  }
  float f;
  memcpy(&f, &x, 4);
  return f;
}

uint16_t bo_f32_to_bf16(float v) {
  uint32_t x;
  memcpy(&x, &v, 4);
  if ((x & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((x >> 16) | 0x40u);
  uint32_t lsb = (x >> 16) & 1u;
  x += 0x7fffu + lsb;
  return (uint16_t)(x >> 16);
}

/* src/raw.rs:118-120 */
float bo_bf16_to_f32(uint16_t b) {
  uint32_t x = ((uint32_t)b & 0x8000u) << 16 | (((uint32_t)b & 0x7fffu) << 16);
  float f;
  memcpy(&f, &x, 4);
  return f;
}

static inline float round_to_f16(float v) { return bo_f16_to_f32(bo_f32_to_f16(v)); }

void bo_round_f16_array(const float *in, float *out, size_t n) {
#pragma omp parallel for schedule(static) if (n > 65536)
  for (size_t i = 0; i < n; ++i) out[i] = round_to_f16(in[i]);
}

void bo_f32_to_f16_array(const float *in, uint16_t *out, size_t n) {
#pragma omp parallel for schedule(static) if (n > 65536)
  for (size_t i = 0; i < n; ++i) out[i] = bo_f32_to_f16(in[i]);
}

/* ------------------------------------------------------------------------- */
/* src/bark.rs:597-611: 0 -> 0, 1..=k -> +lev[c-1], above -> -lev[c-k-1], and a
 * magnitude past the k stored levels reads as 0 (then negated: -0.0). */
float bo_expand(uint32_t code, uint32_t k, const uint16_t *levels) {
  if (code == 0) return 0.0f;
  uint32_t mag;
  int negative;
  if (code <= k) {
    mag = code - 1;
    negative = 0;
  } else {
    mag = code - k - 1;
    negative = 1;
  }
  float value = mag < k ? bo_f16_to_f32(levels[mag]) : 0.0f;
  return negative ? -value : value;
}

/* src/bark.rs:379-391 (read() of a Levels2 entry) */
void bo_lowbit_expand(const uint32_t *codes, const uint16_t *levels, uint32_t k,
                      int64_t rows, int64_t cols, float *out) {
  int64_t ld = (cols + 7) / 8;
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; ++r)
    for (int64_t c = 0; c < cols; ++c) {
      uint32_t w = codes[r * ld + c / 8];
      uint32_t code = (w >> (4 * (c % 8))) & 0xfu;
      out[r * cols + c] = bo_expand(code, k, levels + r * 4);
    }
}

void bo_lut4_expand(const uint8_t *codes, const uint16_t *lut16, int64_t rows,
                    int64_t cols, float *out) {
  int64_t ld = (cols + 1) / 2;
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; ++r)
    for (int64_t c = 0; c < cols; ++c) {
      uint8_t b = codes[r * ld + c / 2];
      uint32_t code = (c & 1) ? (uint32_t)(b >> 4) : (uint32_t)(b & 0xfu);
      out[r * cols + c] = bo_f16_to_f32(lut16[r * 16 + code]);
    }
}

/* ------------------------------------------------------------------------- */
/* src/encoder.rs:228-245: row pi holds pos = T-1-pi; [2i] = sin, [2i+1] = cos of
 * pos * 1/10000^(2i/1024), all in f32 with the platform libm. */
void bo_pos_embed(int t, float *out) {
  int p = 2 * t - 1;
  float inv_freq[HIDDEN / 2];
  for (int i = 0; i < HIDDEN / 2; ++i)
    inv_freq[i] = 1.0f / powf(10000.0f, (2.0f * (float)i) / (float)HIDDEN);
#pragma omp parallel for schedule(static) if (p > 64)
  for (int pi = 0; pi < p; ++pi) {
    float pos = (float)((p - 1) / 2 - pi);
    float *row = out + (size_t)pi * HIDDEN;
    for (int i = 0; i < HIDDEN / 2; ++i) {
      float f = pos * inv_freq[i];
      row[2 * i] = sinf(f);
      row[2 * i + 1] = cosf(f);
    }
  }
}

/* ------------------------------------------------------------------------- */
/* Packed weight panels [panel][k][16] (src/cpu/gemm.rs:27-210). f16 storage is
 * numerically identical to f32 storage of f16-rounded values. */
struct bo_packw {
  int n, k, half;
  float *data;
  uint16_t *data16;
};

bo_packw *bo_pack_rows(const float *w, int n, int k, int half) {
  bo_packw *p = (bo_packw *)calloc(1, sizeof(bo_packw));
  p->n = n;
  p->k = k;
  p->half = half;
  int panels = div_ceil(n, PANEL);
  size_t sz = (size_t)panels * k * PANEL;
  if (half)
    p->data16 = (uint16_t *)aligned_alloc(64, ((sz * 2 + 63) / 64) * 64);
  else
    p->data = (float *)aligned_alloc(64, ((sz * 4 + 63) / 64) * 64);
#pragma omp parallel for schedule(static)
  for (int pn = 0; pn < panels; ++pn) {
    for (int kk = 0; kk < k; ++kk) {
      size_t base = ((size_t)pn * k + kk) * PANEL;
      for (int j = 0; j < PANEL; ++j) {
        int row = pn * PANEL + j;
        float v = row < n ? w[(size_t)row * k + kk] : 0.0f;
        if (half)
          p->data16[base + j] = bo_f32_to_f16(v);
        else
          p->data[base + j] = v;
      }
    }
  }
  return p;
}

/* (n rows of length k) taken from a (k, n) matrix with row stride ld
 * (refill_cols, src/cpu/gemm.rs:169-202), optional f16 rounding of values. */
static void pack_cols(bo_packw *p, const float *src, int ld, int n, int k, int round16) {
  p->n = n;
  p->k = k;
  p->half = 0;
  int panels = div_ceil(n, PANEL);
  size_t sz = (size_t)panels * k * PANEL;
  free(p->data);
  p->data = (float *)aligned_alloc(64, ((sz * 4 + 63) / 64) * 64);
  for (int pn = 0; pn < panels; ++pn)
    for (int kk = 0; kk < k; ++kk) {
      size_t base = ((size_t)pn * k + kk) * PANEL;
      for (int j = 0; j < PANEL; ++j) {
        int col = pn * PANEL + j;
        float v = col < n ? src[(size_t)kk * ld + col] : 0.0f;
        p->data[base + j] = round16 ? round_to_f16(v) : v;
      }
    }
}

/* refill_rows (src/cpu/gemm.rs:107-136) into an existing f32 pack */
static void pack_rows_f32(bo_packw *p, const float *w, int n, int k) {
  p->n = n;
  p->k = k;
  p->half = 0;
  int panels = div_ceil(n, PANEL);
  size_t sz = (size_t)panels * k * PANEL;
  free(p->data);
  p->data = (float *)aligned_alloc(64, ((sz * 4 + 63) / 64) * 64);
  for (int pn = 0; pn < panels; ++pn)
    for (int kk = 0; kk < k; ++kk) {
      size_t base = ((size_t)pn * k + kk) * PANEL;
      for (int j = 0; j < PANEL; ++j) {
        int row = pn * PANEL + j;
        p->data[base + j] = row < n ? w[(size_t)row * k + kk] : 0.0f;
      }
    }
}

void bo_packw_free(bo_packw *w) {
  if (!w) return;
  free(w->data);
  free(w->data16);
  free(w);
}

/* One 6x16 micro tile: acc = fma(a[r][kk], w[kk][j], acc) for kk in k0..k1,
 * the reference's per-element FMA chain (src/cpu/gemm.rs:654-671). */
__attribute__((target("avx2,fma,f16c"))) static void micro6(
    const float *a, int lda, const bo_packw *w, int panel, int k0, int k1, float *buf) {
  __m256 acc[MR][2];
  for (int r = 0; r < MR; ++r) acc[r][0] = acc[r][1] = _mm256_setzero_ps();
  size_t pbase = (size_t)panel * w->k * PANEL;
  if (w->half) {
    const uint16_t *wp = w->data16 + pbase;
    for (int kk = k0; kk < k1; ++kk) {
      const uint16_t *wpk = wp + (size_t)kk * PANEL;
      __m256 w0 = _mm256_cvtph_ps(_mm_loadu_si128((const __m128i *)wpk));
      __m256 w1 = _mm256_cvtph_ps(_mm_loadu_si128((const __m128i *)(wpk + 8)));
#pragma GCC unroll 6
      for (int r = 0; r < MR; ++r) {
        __m256 av = _mm256_broadcast_ss(a + (size_t)r * lda + kk);
        acc[r][0] = _mm256_fmadd_ps(av, w0, acc[r][0]);
        acc[r][1] = _mm256_fmadd_ps(av, w1, acc[r][1]);
      }
    }
  } else {
    const float *wp = w->data + pbase;
    for (int kk = k0; kk < k1; ++kk) {
      const float *wpk = wp + (size_t)kk * PANEL;
      __m256 w0 = _mm256_loadu_ps(wpk);
      __m256 w1 = _mm256_loadu_ps(wpk + 8);
#pragma GCC unroll 6
      for (int r = 0; r < MR; ++r) {
        __m256 av = _mm256_broadcast_ss(a + (size_t)r * lda + kk);
        acc[r][0] = _mm256_fmadd_ps(av, w0, acc[r][0]);
        acc[r][1] = _mm256_fmadd_ps(av, w1, acc[r][1]);
      }
    }
  }
  for (int r = 0; r < MR; ++r) {
    _mm256_storeu_ps(buf + r * PANEL, acc[r][0]);
    _mm256_storeu_ps(buf + r * PANEL + 8, acc[r][1]);
  }
}

/* C rows [0,rows) x panel columns [n0, n0+ncols) over k0..k1; a short final row
 * tile is zero-padded to MR rows (extra rows are computed and dropped). */
static void tile(const float *a, int lda, const bo_packw *w, int n0, int ncols, float *c,
                 int ldc, int rows, int k0, int k1) {
  int first = n0 / PANEL;
  int panels = div_ceil(ncols, PANEL);
  float buf[MR * PANEL];
  float *pad = NULL;
  for (int row = 0; row < rows; row += MR) {
    int tr = rows - row < MR ? rows - row : MR;
    const float *ap = a + (size_t)row * lda;
    int alda = lda;
    if (tr < MR) {
      if (!pad) pad = (float *)calloc((size_t)MR * lda, sizeof(float));
      memset(pad, 0, (size_t)MR * lda * sizeof(float));
      for (int r = 0; r < tr; ++r)
        memcpy(pad + (size_t)r * lda + k0, ap + (size_t)r * lda + k0,
               (size_t)(k1 - k0) * sizeof(float));
      ap = pad;
    }
    for (int p = 0; p < panels; ++p) {
      int cols = ncols - p * PANEL < PANEL ? ncols - p * PANEL : PANEL;
      micro6(ap, alda, w, first + p, k0, k1, buf);
      for (int r = 0; r < tr; ++r)
        memcpy(c + (size_t)(row + r) * ldc + p * PANEL, buf + r * PANEL,
               (size_t)cols * sizeof(float));
    }
  }
  free(pad);
}

static int mr_floor(int v) {
  int r = v / MR * MR;
  return r > MR ? r : MR;
}
static int panel_floor(int v) {
  int r = v / PANEL * PANEL;
  return r > PANEL ? r : PANEL;
}

/* src/cpu/gemm.rs:220-311: C[0..m, n0..n0+ncols] = A[m,k] . W[n0.., k]^T.
 * The 2-D task split only schedules work; each element's value is its FMA
 * chain, so results do not depend on `threads`. */
void bo_gemm(const float *a, const bo_packw *w, float *c, int m, int n0, int ncols,
             int threads) {
  int k = w->k;
  if (m == 0 || ncols == 0 || k == 0) return;
  if (n0 % PANEL != 0 || n0 + ncols > w->n) {
    fprintf(stderr, "bo_gemm: bad column range\n");
    abort();
  }
  if (threads < 1) threads = 1;
  int tm = mr_floor(TM < (m > MR ? m : MR) ? TM : (m > MR ? m : MR));
  int tn = panel_floor(TN < ncols ? TN : ncols);
  for (;;) {
    if (div_ceil(m, tm) * div_ceil(ncols, tn) >= threads * 2) break;
    int can_m = tm > MR, can_n = tn > PANEL;
    if (!can_m && !can_n) break;
    if ((can_m && tm >= tn) || !can_n)
      tm = mr_floor((tm / 2) > MR ? tm / 2 : MR);
    else
      tn = panel_floor(tn / 2);
  }
  int mt = div_ceil(m, tm), nt = div_ceil(ncols, tn);
#pragma omp parallel for schedule(dynamic) num_threads(threads)
  for (int task = 0; task < mt * nt; ++task) {
    int mi = task / nt, ni = task % nt;
    int m0 = mi * tm, rows = m - m0 < tm ? m - m0 : tm;
    int tn0 = n0 + ni * tn, cols = ncols - ni * tn < tn ? ncols - ni * tn : tn;
    tile(a + (size_t)m0 * k, k, w, tn0, cols, c + (size_t)m0 * ncols + (tn0 - n0), ncols,
         rows, 0, k);
  }
}

/* src/cpu/gemm.rs:348-415 with the worker count explicit: k is cut into
 * `workers` chunks, each an FMA chain from 0; partials summed in worker order. */
void bo_gemm_split_k(const float *a, const bo_packw *w, float *c, int m, int n0,
                     int ncols, int workers_param, int threads) {
  int k = w->k;
  int workers = workers_param < div_ceil(k, 64) ? workers_param : div_ceil(k, 64);
  if (workers < 1) workers = 1;
  if (workers <= 1) {
    bo_gemm(a, w, c, m, n0, ncols, threads);
    return;
  }
  int chunk = div_ceil(k, workers);
  float *parts = (float *)calloc((size_t)workers * m * ncols, sizeof(float));
#pragma omp parallel for schedule(dynamic) num_threads(threads)
  for (int wi = 0; wi < workers; ++wi) {
    int k0 = wi * chunk;
    int k1 = k0 + chunk < k ? k0 + chunk : k;
    if (k0 >= k1) continue;
    tile(a, k, w, n0, ncols, parts + (size_t)wi * m * ncols, ncols, m, k0, k1);
  }
  for (int i = 0; i < m * ncols; ++i) {
    float acc = 0.0f;
    for (int wi = 0; wi < workers; ++wi) acc += parts[(size_t)wi * m * ncols + i];
    c[i] = acc;
  }
  free(parts);
}

void bo_gemm_fma_chain(const float *a, const float *w, float *c, int m, int n, int k) {
#pragma omp parallel for schedule(static)
  for (int r = 0; r < m; ++r)
    for (int j = 0; j < n; ++j) {
      float acc = 0.0f;
      for (int kk = 0; kk < k; ++kk)
        acc = fmaf(a[(size_t)r * k + kk], w[(size_t)j * k + kk], acc);
      c[(size_t)r * n + j] = acc;
    }
}

void bo_gemm_naive_f64(const float *a, const float *w, double *c, int m, int n, int k) {
#pragma omp parallel for schedule(static)
  for (int r = 0; r < m; ++r)
    for (int j = 0; j < n; ++j) {
      double acc = 0.0;
      for (int kk = 0; kk < k; ++kk)
        acc += (double)a[(size_t)r * k + kk] * (double)w[(size_t)j * k + kk];
      c[(size_t)r * n + j] = acc;
    }
}

/* ------------------------------------------------------------------------- */
/* src/cpu/ops.rs:15-56 — 256 lanes of (e0+e2)+(e1+e3), tree 128..1. */
void bo_layer_norm(const float *src, float *dst, const float *w, const float *b,
                   int rows, int dim) {
#pragma omp parallel for schedule(static) if (rows >= 8)
  for (int r = 0; r < rows; ++r) {
    const float *x = src + (size_t)r * dim;
    float *y = dst + (size_t)r * dim;
    float rs[256], rq[256];
    for (int lane = 0; lane < 256; ++lane) {
      float e0 = x[lane], e1 = x[lane + 256], e2 = x[lane + 512], e3 = x[lane + 768];
      rs[lane] = (e0 + e2) + (e1 + e3);
      rq[lane] = (e0 * e0 + e2 * e2) + (e1 * e1 + e3 * e3);
    }
    for (int s = 128; s > 0; s >>= 1)
      for (int i = 0; i < s; ++i) {
        rs[i] += rs[i + s];
        rq[i] += rq[i + s];
      }
    float inv_n = 1.0f / (float)dim;
    float mean = rs[0] * inv_n;
    float var = rq[0] * inv_n - mean * mean;
    float inv_std = 1.0f / sqrtf(var + 1e-5f);
    for (int i = 0; i < dim; ++i) y[i] = (x[i] - mean) * inv_std * w[i] + b[i];
  }
}

/* src/cpu/ops.rs:59-70 */
void bo_silu(float *x, size_t n) {
#pragma omp parallel for schedule(static) if (n >= 4096)
  for (size_t i = 0; i < n; ++i) x[i] = x[i] / (1.0f + expf(-x[i]));
}

/* src/cpu/ops.rs:74-95 */
void bo_glu(const float *src, float *dst, int rows, int c) {
#pragma omp parallel for schedule(static) if (rows >= 8)
  for (int r = 0; r < rows; ++r)
    for (int i = 0; i < c; ++i) {
      float a = src[(size_t)r * c * 2 + i];
      float bb = src[(size_t)r * c * 2 + c + i];
      dst[(size_t)r * c + i] = a / (1.0f + expf(-bb));
    }
}

/* src/cpu/ops.rs:98-111 */
void bo_add_scaled(float *a, const float *b, float scale, size_t n) {
#pragma omp parallel for schedule(static) if (n >= 8192)
  for (size_t i = 0; i < n; ++i) a[i] += scale * b[i];
}

/* src/cpu/ops.rs:114-125 */
void bo_add_bias(float *x, const float *bias, int rows, int dim) {
#pragma omp parallel for schedule(static) if (rows >= 8)
  for (int r = 0; r < rows; ++r)
    for (int i = 0; i < dim; ++i) x[(size_t)r * dim + i] += bias[i];
}

/* src/cpu/ops.rs:133-189 */
void bo_rel_softmax_rows(float *probs, const float *bd, int win, int rows, int t, int q0,
                         int j0, float scale) {
#pragma omp parallel for schedule(static) if (rows >= 8)
  for (int qi = 0; qi < rows; ++qi) {
    int shift = t - 1 - (q0 + qi) - j0;
    const float *brow = bd + (size_t)qi * win;
    float *prow = probs + (size_t)qi * t;
    float m = -INFINITY;
    for (int k = 0; k < t; ++k) {
      float s = scale * (prow[k] + brow[shift + k]);
      prow[k] = s;
      if (s > m) m = s;
    }
    float part[256];
    for (int lane = 0; lane < 256; ++lane) {
      float acc = 0.0f;
      for (int j = lane; j < t; j += 256) {
        float e = expf(prow[j] - m);
        prow[j] = e;
        acc += e;
      }
      part[lane] = acc;
    }
    for (int s = 128; s > 0; s >>= 1)
      for (int i = 0; i < s; ++i) part[i] += part[i + s];
    float sum = part[0];
    for (int k = 0; k < t; ++k) prow[k] /= sum;
  }
}

/* src/cpu/ops.rs:195-233 — taps i=0..8 at t+i-4, zero outside [0, rows). */
void bo_dwconv_bn_silu(const float *src, const float *dw, const float *bn_a,
                       const float *bn_b, float *dst, int rows, int dim) {
#pragma omp parallel for schedule(static) if (rows >= 8)
  for (int t = 0; t < rows; ++t)
    for (int c = 0; c < dim; ++c) {
      float acc = 0.0f;
      for (int i = 0; i < 9; ++i) {
        int tt = t + i - 4;
        if (tt < 0 || tt >= rows) continue;
        acc += src[(size_t)tt * dim + c] * dw[c * 9 + i];
      }
      float y = acc * bn_a[c] + bn_b[c];
      dst[(size_t)t * dim + c] = y / (1.0f + expf(-y));
    }
}

/* src/cpu/ops.rs:238-279 */
static void pack_attention_inputs(const float *qkv, int rows, const float *bu,
                                  const float *bv, float *qu, float *qv, float *kh,
                                  float *vh) {
#pragma omp parallel for schedule(static) if (rows >= 8)
  for (int i = 0; i < HEADS * rows; ++i) {
    int h = i / rows, q = i % rows;
    for (int j = 0; j < HDIM; ++j) {
      int b = h * HDIM + j;
      const float *row = qkv + (size_t)q * 3072;
      qu[(size_t)i * HDIM + j] = row[b] + bu[b];
      qv[(size_t)i * HDIM + j] = row[b] + bv[b];
      kh[(size_t)i * HDIM + j] = round_to_f16(row[1024 + b]);
      vh[(size_t)i * HDIM + j] = round_to_f16(row[2048 + b]);
    }
  }
}

/* ------------------------------------------------------------------------- */
/* Weights held by name (src/cpu/mod.rs:47-152). */
enum {
  L_Q, L_K, L_V, L_RELK, L_O, L_FF1A, L_FF1B, L_FF2A, L_FF2B, L_PW1, L_PW2, L_DW,
  L_BN_W, L_BN_B, L_BN_M, L_BN_V, L_BU, L_BV,
  L_LN0W, L_LN0B, L_LN1W, L_LN1B, L_LN2W, L_LN2B, L_LN3W, L_LN3B, L_LN4W, L_LN4B,
  L_COUNT
};
static const char *LAYER_NAMES[L_COUNT] = {
    "self_attn.q_proj.weight", "self_attn.k_proj.weight", "self_attn.v_proj.weight",
    "self_attn.relative_k_proj.weight", "self_attn.o_proj.weight",
    "feed_forward1.linear1.weight", "feed_forward1.linear2.weight",
    "feed_forward2.linear1.weight", "feed_forward2.linear2.weight",
    "conv.pointwise_conv1.weight", "conv.pointwise_conv2.weight",
    "conv.depthwise_conv.weight", "conv.norm.weight", "conv.norm.bias",
    "conv.norm.running_mean", "conv.norm.running_var", "self_attn.bias_u",
    "self_attn.bias_v", "norm_feed_forward1.weight", "norm_feed_forward1.bias",
    "norm_self_att.weight", "norm_self_att.bias", "norm_conv.weight", "norm_conv.bias",
    "norm_feed_forward2.weight", "norm_feed_forward2.bias", "norm_out.weight",
    "norm_out.bias"};
static const int64_t LAYER_SIZES[L_COUNT] = {
    1024 * 1024, 1024 * 1024, 1024 * 1024, 1024 * 1024, 1024 * 1024, 4096 * 1024,
    1024 * 4096, 4096 * 1024, 1024 * 4096, 2048 * 1024, 1024 * 1024, 1024 * 9,
    1024, 1024, 1024, 1024, 1024, 1024, 1024, 1024, 1024, 1024, 1024, 1024, 1024, 1024,
    1024, 1024};

typedef struct {
  float *raw[L_COUNT];
  bo_packw *qkv, *o, *ff1a, *ff1b, *ff2a, *ff2b, *pw1, *pw2;
  float *relk; /* f16-rounded (1024, 1024), the A operand of the relK GEMM */
  float *dw;   /* f16-rounded (1024, 9) */
  float bn_a[HIDDEN], bn_b[HIDDEN];
} bo_layer;

struct bo_encoder {
  int n_layers;
  float *sub_w_raw, *sub_b, *proj_w_raw, *proj_b;
  bo_packw *sub_w, *proj_w;
  bo_layer *layers;
  int finalized;
};

bo_encoder *bo_encoder_new(int n_layers) {
  if (n_layers < 1 || n_layers > 24) return NULL;
  bo_encoder *e = (bo_encoder *)calloc(1, sizeof(bo_encoder));
  e->n_layers = n_layers;
  e->layers = (bo_layer *)calloc((size_t)n_layers, sizeof(bo_layer));
  return e;
}

void bo_encoder_free(bo_encoder *e) {
  if (!e) return;
  free(e->sub_w_raw);
  free(e->sub_b);
  free(e->proj_w_raw);
  free(e->proj_b);
  bo_packw_free(e->sub_w);
  bo_packw_free(e->proj_w);
  for (int l = 0; l < e->n_layers; ++l) {
    bo_layer *L = &e->layers[l];
    for (int i = 0; i < L_COUNT; ++i) free(L->raw[i]);
    bo_packw_free(L->qkv);
    bo_packw_free(L->o);
    bo_packw_free(L->ff1a);
    bo_packw_free(L->ff1b);
    bo_packw_free(L->ff2a);
    bo_packw_free(L->ff2b);
    bo_packw_free(L->pw1);
    bo_packw_free(L->pw2);
    free(L->relk);
    free(L->dw);
  }
  free(e->layers);
  free(e);
}

static float *dup_f32(const float *v, int64_t n) {
  float *p = (float *)malloc((size_t)n * sizeof(float));
  memcpy(p, v, (size_t)n * sizeof(float));
  return p;
}

static int set_slot(float **slot, const float *v, int64_t n, int64_t want) {
  if (n != want) return -1;
  free(*slot);
  *slot = dup_f32(v, n);
  return 0;
}

int bo_encoder_set(bo_encoder *e, const char *name, const float *v, int64_t n) {
  if (!strcmp(name, "encoder.subsampling.linear.weight"))
    return set_slot(&e->sub_w_raw, v, n, 1024 * 4096);
  if (!strcmp(name, "encoder.subsampling.linear.bias")) return set_slot(&e->sub_b, v, n, 1024);
  if (!strcmp(name, "encoder_projector.weight"))
    return set_slot(&e->proj_w_raw, v, n, 640 * 1024);
  if (!strcmp(name, "encoder_projector.bias")) return set_slot(&e->proj_b, v, n, 640);
  const char *pre = "encoder.layers.";
  size_t pl = strlen(pre);
  if (strncmp(name, pre, pl)) return -1;
  char *end = NULL;
  long l = strtol(name + pl, &end, 10);
  if (!end || *end != '.' || l < 0 || l >= e->n_layers) return -1;
  const char *suffix = end + 1;
  for (int i = 0; i < L_COUNT; ++i)
    if (!strcmp(suffix, LAYER_NAMES[i]))
      return set_slot(&e->layers[l].raw[i], v, n, LAYER_SIZES[i]);
  return -1;
}

/* f16v (src/cpu/mod.rs:35-37) then pack_rows (f16 panels, src/cpu/gemm.rs:64-70) */
static bo_packw *pack_f16v(const float *w, int n, int k) {
  float *r = (float *)malloc((size_t)n * k * sizeof(float));
  bo_round_f16_array(w, r, (size_t)n * k);
  bo_packw *p = bo_pack_rows(r, n, k, 1);
  free(r);
  return p;
}

int bo_encoder_finalize(bo_encoder *e) {
  if (!e->sub_w_raw || !e->sub_b || !e->proj_w_raw || !e->proj_b) return -1;
  for (int l = 0; l < e->n_layers; ++l)
    for (int i = 0; i < L_COUNT; ++i)
      if (!e->layers[l].raw[i]) return -2 - l;
  e->sub_w = pack_f16v(e->sub_w_raw, 1024, 4096);
  e->proj_w = pack_f16v(e->proj_w_raw, 640, 1024);
  for (int l = 0; l < e->n_layers; ++l) {
    bo_layer *L = &e->layers[l];
    float *cat = (float *)malloc((size_t)3072 * 1024 * sizeof(float));
    memcpy(cat, L->raw[L_Q], (size_t)1024 * 1024 * 4);
    memcpy(cat + 1024 * 1024, L->raw[L_K], (size_t)1024 * 1024 * 4);
    memcpy(cat + 2 * 1024 * 1024, L->raw[L_V], (size_t)1024 * 1024 * 4);
    L->qkv = pack_f16v(cat, 3072, 1024);
    free(cat);
    L->relk = (float *)malloc((size_t)1024 * 1024 * 4);
    bo_round_f16_array(L->raw[L_RELK], L->relk, (size_t)1024 * 1024);
    L->o = pack_f16v(L->raw[L_O], 1024, 1024);
    L->ff1a = pack_f16v(L->raw[L_FF1A], 4096, 1024);
    L->ff1b = pack_f16v(L->raw[L_FF1B], 1024, 4096);
    L->ff2a = pack_f16v(L->raw[L_FF2A], 4096, 1024);
    L->ff2b = pack_f16v(L->raw[L_FF2B], 1024, 4096);
    L->pw1 = pack_f16v(L->raw[L_PW1], 2048, 1024);
    L->pw2 = pack_f16v(L->raw[L_PW2], 1024, 1024);
    L->dw = (float *)malloc((size_t)1024 * 9 * 4);
    bo_round_f16_array(L->raw[L_DW], L->dw, (size_t)1024 * 9);
    for (int c = 0; c < HIDDEN; ++c) { /* src/cpu/mod.rs:113-119 */
      float a = L->raw[L_BN_W][c] / sqrtf(L->raw[L_BN_V][c] + 1e-5f);
      L->bn_a[c] = a;
      L->bn_b[c] = L->raw[L_BN_B][c] - L->raw[L_BN_M][c] * a;
    }
  }
  e->finalized = 1;
  return 0;
}

typedef struct {
  int t, pp;
  float *normed, *ffb, *tmp, *tmp2, *qkv, *qu, *qv, *kh, *vh, *relk_t, *attnout, *cb1,
      *cb2, *probs, *bd, *attn_h;
  bo_packw kh_pack[HEADS], vh_pack[HEADS], rkh_pack[HEADS];
  bo_packw *pos;
} scratch_t;

static void scratch_init(scratch_t *s, int t) {
  memset(s, 0, sizeof(*s));
  s->t = t;
  s->pp = pad128(2 * t - 1);
  size_t T = (size_t)t;
  s->normed = (float *)calloc(T * HIDDEN, 4);
  s->ffb = (float *)calloc(T * FFN, 4);
  s->tmp = (float *)calloc(T * HIDDEN, 4);
  s->tmp2 = (float *)calloc(T * HIDDEN, 4);
  s->qkv = (float *)calloc(T * 3072, 4);
  s->qu = (float *)calloc(HEADS * T * HDIM, 4);
  s->qv = (float *)calloc(HEADS * T * HDIM, 4);
  s->kh = (float *)calloc(HEADS * T * HDIM, 4);
  s->vh = (float *)calloc(HEADS * T * HDIM, 4);
  s->relk_t = (float *)calloc((size_t)HIDDEN * s->pp, 4);
  s->attnout = (float *)calloc(T * HIDDEN, 4);
  s->cb1 = (float *)calloc(T * 2048, 4);
  s->cb2 = (float *)calloc(T * HIDDEN, 4);
  s->probs = (float *)calloc((size_t)BQ * T, 4);
  s->bd = (float *)calloc((size_t)BQ * (T + BQ + 2 * PANEL), 4);
  s->attn_h = (float *)calloc((size_t)BQ * HDIM, 4);
  /* position table padded to pp rows and packed as f32 (src/cpu/mod.rs:158-161) */
  float *pos_pad = (float *)calloc((size_t)s->pp * HIDDEN, 4);
  bo_pos_embed(t, pos_pad);
  s->pos = bo_pack_rows(pos_pad, s->pp, HIDDEN, 0);
  free(pos_pad);
}

static void scratch_free(scratch_t *s) {
  free(s->normed); free(s->ffb); free(s->tmp); free(s->tmp2); free(s->qkv);
  free(s->qu); free(s->qv); free(s->kh); free(s->vh); free(s->relk_t);
  free(s->attnout); free(s->cb1); free(s->cb2); free(s->probs); free(s->bd);
  free(s->attn_h);
  for (int h = 0; h < HEADS; ++h) {
    free(s->kh_pack[h].data);
    free(s->vh_pack[h].data);
    free(s->rkh_pack[h].data);
  }
  bo_packw_free(s->pos);
}

/* src/cpu/layer.rs:157-327 — FF1, attention, conv, FF2, norm_out into normed. */
static void layer_forward(const bo_layer *L, float *x, scratch_t *s, int threads,
                          int av_workers) {
  int t = s->t, pp = s->pp;
  float scale = powf((float)HDIM, -0.5f);
  float **raw = (float **)L->raw;
  size_t tH = (size_t)t * HIDDEN;

  /* FF1: h += 0.5 * ff2(silu(ff1(ln1(h)))) */
  bo_layer_norm(x, s->normed, raw[L_LN0W], raw[L_LN0B], t, HIDDEN);
  bo_gemm(s->normed, L->ff1a, s->ffb, t, 0, 4096, threads);
  bo_silu(s->ffb, (size_t)t * 4096);
  bo_gemm(s->ffb, L->ff1b, s->tmp, t, 0, HIDDEN, threads);
  bo_add_scaled(x, s->tmp, 0.5f, tH);

  /* attention */
  bo_layer_norm(x, s->normed, raw[L_LN1W], raw[L_LN1B], t, HIDDEN);
  bo_gemm(s->normed, L->qkv, s->qkv, t, 0, 3072, threads);
  pack_attention_inputs(s->qkv, t, raw[L_BU], raw[L_BV], s->qu, s->qv, s->kh, s->vh);
  for (int h = 0; h < HEADS; ++h) {
    /* k: (n = t, k = 128) rows; v: (k = t, n = 128) from a (t,128) matrix */
    pack_rows_f32(&s->kh_pack[h], s->kh + (size_t)h * t * HDIM, t, HDIM);
    pack_cols(&s->vh_pack[h], s->vh + (size_t)h * t * HDIM, HDIM, HDIM, t, 0);
  }
  /* relk_t[d][p] = relk[d] . pos[p], rounded through f16 when packed */
  bo_gemm(L->relk, s->pos, s->relk_t, HIDDEN, 0, pp, threads);
  for (int h = 0; h < HEADS; ++h)
    pack_cols(&s->rkh_pack[h], s->relk_t + (size_t)h * HDIM * pp, pp, pp, HDIM, 1);

  for (int q0 = 0; q0 < t;) {
    int rows = t - q0 < BQ ? t - q0 : BQ;
    int jmin = t - 1 - (q0 + rows - 1);
    int jmax = 2 * t - 2 - q0 < pp - 1 ? 2 * t - 2 - q0 : pp - 1;
    int j0 = (jmin / PANEL) * PANEL;
    int j1 = (jmax + PANEL) / PANEL * PANEL;
    if (j1 > pp) j1 = pp;
    int win = j1 - j0;
    for (int h = 0; h < HEADS; ++h) {
      bo_gemm(s->qu + (size_t)h * t * HDIM + (size_t)q0 * HDIM, &s->kh_pack[h], s->probs,
              rows, 0, t, threads);
      bo_gemm(s->qv + (size_t)h * t * HDIM + (size_t)q0 * HDIM, &s->rkh_pack[h], s->bd,
              rows, j0, win, threads);
      bo_rel_softmax_rows(s->probs, s->bd, win, rows, t, q0, j0, scale);
      bo_gemm_split_k(s->probs, &s->vh_pack[h], s->attn_h, rows, 0, HDIM, av_workers,
                      threads);
      for (int qi = 0; qi < rows; ++qi)
        memcpy(s->attnout + (size_t)(q0 + qi) * HIDDEN + h * HDIM,
               s->attn_h + (size_t)qi * HDIM, HDIM * sizeof(float));
    }
    q0 += rows;
  }
  bo_gemm(s->attnout, L->o, s->tmp, t, 0, HIDDEN, threads);
  bo_add_scaled(x, s->tmp, 1.0f, tH);

  /* conv module */
  bo_layer_norm(x, s->normed, raw[L_LN2W], raw[L_LN2B], t, HIDDEN);
  bo_gemm(s->normed, L->pw1, s->cb1, t, 0, 2048, threads);
  bo_glu(s->cb1, s->cb2, t, HIDDEN);
  bo_dwconv_bn_silu(s->cb2, L->dw, L->bn_a, L->bn_b, s->tmp, t, HIDDEN);
  bo_gemm(s->tmp, L->pw2, s->tmp2, t, 0, HIDDEN, threads);
  bo_add_scaled(x, s->tmp2, 1.0f, tH);

  /* FF2 */
  bo_layer_norm(x, s->normed, raw[L_LN3W], raw[L_LN3B], t, HIDDEN);
  bo_gemm(s->normed, L->ff2a, s->ffb, t, 0, 4096, threads);
  bo_silu(s->ffb, (size_t)t * 4096);
  bo_gemm(s->ffb, L->ff2b, s->tmp, t, 0, HIDDEN, threads);
  bo_add_scaled(x, s->tmp, 0.5f, tH);

  /* norm_out into the scratch; the caller decides whether x takes it */
  bo_layer_norm(x, s->normed, raw[L_LN4W], raw[L_LN4B], t, HIDDEN);
}

int bo_encoder_encode(bo_encoder *e, const float *sub, int t, int layers, float *out,
                      int threads, int av_workers) {
  if (!e->finalized || t < 1) return -1;
  omp_set_num_threads(threads);
  scratch_t s;
  scratch_init(&s, t);
  float *x = (float *)calloc((size_t)t * HIDDEN, 4);
  bo_gemm(sub, e->sub_w, x, t, 0, HIDDEN, threads);
  bo_add_bias(x, e->sub_b, t, HIDDEN);
  int upto = layers < e->n_layers ? layers : e->n_layers;
  for (int i = 0; i < upto; ++i) {
    layer_forward(&e->layers[i], x, &s, threads, av_workers);
    if (i + 1 < upto || upto == e->n_layers)
      memcpy(x, s.normed, (size_t)t * HIDDEN * sizeof(float));
  }
  if (upto == e->n_layers) {
    bo_gemm(x, e->proj_w, out, t, 0, 640, threads);
    bo_add_bias(out, e->proj_b, t, 640);
  } else {
    memcpy(out, x, (size_t)t * HIDDEN * sizeof(float));
  }
  free(x);
  scratch_free(&s);
  return 0;
}

int bo_encoder_encode_dump(bo_encoder *e, const float *sub, int t, float *dumps,
                           float *pooler, int threads, int av_workers) {
  if (!e->finalized || t < 1) return -1;
  omp_set_num_threads(threads);
  scratch_t s;
  scratch_init(&s, t);
  float *x = (float *)calloc((size_t)t * HIDDEN, 4);
  bo_gemm(sub, e->sub_w, x, t, 0, HIDDEN, threads);
  bo_add_bias(x, e->sub_b, t, HIDDEN);
  for (int i = 0; i < e->n_layers; ++i) {
    layer_forward(&e->layers[i], x, &s, threads, av_workers);
    memcpy(dumps + (size_t)i * t * HIDDEN, x, (size_t)t * HIDDEN * sizeof(float));
    memcpy(x, s.normed, (size_t)t * HIDDEN * sizeof(float));
  }
  bo_gemm(x, e->proj_w, pooler, t, 0, 640, threads);
  bo_add_bias(pooler, e->proj_b, t, 640);
  free(x);
  scratch_free(&s);
  return 0;
}

int bo_encoder_block(bo_encoder *e, int layer, float *x, int t, int apply_norm_out,
                     int threads, int av_workers) {
  if (!e->finalized || layer < 0 || layer >= e->n_layers || t < 1) return -1;
  omp_set_num_threads(threads);
  scratch_t s;
  scratch_init(&s, t);
  layer_forward(&e->layers[layer], x, &s, threads, av_workers);
  if (apply_norm_out) memcpy(x, s.normed, (size_t)t * HIDDEN * sizeof(float));
  scratch_free(&s);
  return 0;
}

/* ------------------------------------------------------------------------- */
/* src/sub.rs:11-13 */
int bo_conv_len(int l) { return (l + 2 - 3) / 2 + 1; }

#define SUBC 256

/* src/sub.rs:288-300 */
static void mask_time(float *x, int t, int m, int vlen) {
  if (vlen >= t) return;
#pragma omp parallel for schedule(static)
  for (int c = 0; c < SUBC; ++c)
    for (int i = vlen; i < t; ++i)
      for (int j = 0; j < m; ++j) x[(size_t)c * t * m + (size_t)i * m + j] = 0.0f;
}

/* src/sub.rs:174-203: s = b; s += w*x over (ki,kj) with out-of-range taps skipped */
static float *dw_conv(const float *x, const float *w, const float *b, int t_in, int m_in) {
  int t_out = bo_conv_len(t_in), m_out = bo_conv_len(m_in);
  float *out = (float *)calloc((size_t)SUBC * t_out * m_out, 4);
#pragma omp parallel for schedule(static)
  for (int c = 0; c < SUBC; ++c)
    for (int i = 0; i < t_out; ++i)
      for (int j = 0; j < m_out; ++j) {
        float s = b[c];
        for (int ki = 0; ki < 3; ++ki) {
          int ii = 2 * i + ki - 1;
          if (ii < 0 || ii >= t_in) continue;
          for (int kj = 0; kj < 3; ++kj) {
            int jj = 2 * j + kj - 1;
            if (jj < 0 || jj >= m_in) continue;
            s += w[c * 9 + ki * 3 + kj] * x[(size_t)c * t_in * m_in + (size_t)ii * m_in + jj];
          }
        }
        out[(size_t)c * t_out * m_out + (size_t)i * m_out + j] = s;
      }
  return out;
}

/* src/sub.rs:208-257: out[co][p] = relu(sum_ci w[co][ci]*x[ci][p] (mul+add,
 * ascending ci, zero weights skipped) + b[co]) */
static float *pw_conv(const float *x, const float *w, const float *b, int t, int m) {
  size_t p = (size_t)t * m;
  float *out = (float *)calloc((size_t)SUBC * p, 4);
#pragma omp parallel for schedule(static)
  for (int co = 0; co < SUBC; ++co) {
    float *orow = out + (size_t)co * p;
    for (int ci = 0; ci < SUBC; ++ci) {
      float wv = w[co * SUBC + ci];
      if (wv != 0.0f) {
        const float *xrow = x + (size_t)ci * p;
        for (size_t q = 0; q < p; ++q) orow[q] = orow[q] + wv * xrow[q];
      }
    }
    float bv = b[co];
    for (size_t q = 0; q < p; ++q) {
      float v = orow[q] + bv;
      orow[q] = v > 0.0f ? v : 0.0f;
    }
  }
  return out;
}

/* src/sub.rs:107-286 */
int bo_subsample(const float *l0w, const float *l0b, const float *l2w, const float *l2b,
                 const float *l3w, const float *l3b, const float *l5w, const float *l5b,
                 const float *l6w, const float *l6b, const float *mel, int f, int n_valid,
                 float *out, int threads) {
  if (f < 1) return -1;
  omp_set_num_threads(threads);
  const int m0 = 128;
  int f1 = bo_conv_len(f), m1 = bo_conv_len(m0);
  size_t p1 = (size_t)f1 * m1;
  float *x = (float *)malloc((size_t)SUBC * p1 * 4);
  /* conv1: out = b; out += w[tap] * x_tap for taps 0..8 (mul then add) */
#pragma omp parallel for schedule(static)
  for (int co = 0; co < SUBC; ++co) {
    float *o = x + (size_t)co * p1;
    for (size_t pix = 0; pix < p1; ++pix) {
      int i = (int)(pix / m1), j = (int)(pix % m1);
      float acc = l0b[co];
      for (int tp = 0; tp < 9; ++tp) {
        int ki = tp / 3, kj = tp % 3;
        int ii = 2 * i + ki, jj = 2 * j + kj;
        float v = 0.0f;
        if (ii > 0 && ii <= 2 * f && jj > 0 && jj <= 2 * m0) {
          int si = ii - 1, sj = jj - 1;
          if (si < f && sj < m0) v = mel[(size_t)si * m0 + sj];
        }
        acc = acc + l0w[co * 9 + tp] * v;
      }
      o[pix] = acc > 0.0f ? acc : 0.0f;
    }
  }
  int vlen = bo_conv_len(n_valid > 1 ? n_valid : 1);
  mask_time(x, f1, m1, vlen < f1 ? vlen : f1);
  float *x2 = dw_conv(x, l2w, l2b, f1, m1);
  free(x);
  int len = bo_conv_len(f1), mlen = bo_conv_len(m1);
  vlen = bo_conv_len(vlen);
  mask_time(x2, len, mlen, vlen < len ? vlen : len);
  float *x3 = pw_conv(x2, l3w, l3b, len, mlen);
  free(x2);
  float *x4 = dw_conv(x3, l5w, l5b, len, mlen);
  free(x3);
  len = bo_conv_len(len);
  mlen = bo_conv_len(mlen);
  vlen = bo_conv_len(vlen);
  mask_time(x4, len, mlen, vlen < len ? vlen : len);
  float *x5 = pw_conv(x4, l6w, l6b, len, mlen);
  free(x4);
  int t = len;
  for (int c = 0; c < SUBC; ++c)
    for (int i = 0; i < t; ++i)
      for (int j = 0; j < mlen; ++j)
        out[(size_t)i * SUBC * mlen + (size_t)c * mlen + j] =
            x5[(size_t)c * t * mlen + (size_t)i * mlen + j];
  free(x5);
  return t;
}
