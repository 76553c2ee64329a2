/*
 * nibble_oracle.c -- CPU restatement of the reference's W4A16 format and its
 * dequantise-then-matmul path.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the shipped library links, loads or
 * calls this file.  It is the checker that tests/, __graft_entry__.smoke() and
 * the cpu_baseline leg of bench.py compare the HIP kernels against.
 *
 * Every function names the reference lines it restates (paths relative to the
 * arvindcr4/nibblegemm tree):
 *
 *   nibble_oracle_pack            python/nibblegemm/quant.py:164-182
 *   nibble_oracle_unpack          python/nibblegemm/quant.py:185-196
 *   nibble_oracle_quantize_rtn    python/nibblegemm/quant.py:127-161 (clip_search=False)
 *   nibble_oracle_dequantize      python/nibblegemm/quant.py:199-204
 *   nibble_oracle_matmul_f32      python/nibblegemm/quant.py:207-215
 *   nibble_oracle_matmul_f64      (brute-force double-precision check, no counterpart)
 *   nibble_oracle_f32_to_f16 /
 *   nibble_oracle_f16_to_f32      IEEE-754 binary16 round-to-nearest-even, the
 *                                 conversion torch's .to(torch.float16) performs
 *
 * Format (quant.py:8-54): W is [K, N] consumed as Y = X @ W.  Groups of G rows
 * along K share one fp16 scale per column.  Symmetric INT4 stored biased as
 * q + 8 in [0, 15].  Eight nibbles along K share one 32-bit word,
 * qweight[K/8, N]; logical offset k within the word lives in nibble slot
 * SLOT_FOR_K[k] = {0, 4, 1, 5, 2, 6, 3, 7} (even k in slots 0..3, odd k in
 * slots 4..7).
 *
 * Pinning (how each function is checked against something other than itself)
 * is listed in tests/test_oracle.py.
 */
#include <math.h>
#include <stdlib.h>
#include <stdint.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

static const int kSlotForK[8] = {0, 4, 1, 5, 2, 6, 3, 7};

/* ------------------------------------------------------------------------- */
/* binary16 <-> binary32                                                      */
/* ------------------------------------------------------------------------- */
static inline uint32_t f32_bits(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return u;
}

static inline float bits_f32(uint32_t u) {
  float f;
  memcpy(&f, &u, 4);
  return f;
}

/* Exact widening: every binary16 value is representable in binary32. */
float nibble_oracle_f16_to_f32(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  const uint32_t exp = (h >> 10) & 0x1fu;
  const uint32_t man = h & 0x3ffu;
  if (exp == 0x1fu) return bits_f32(sign | 0x7f800000u | (man << 13)); /* inf / nan */
  if (exp == 0) {
    /* zero or subnormal: man * 2^-24, exact in binary32 */
    const float v = ldexpf((float)man, -24);
    return sign ? -v : v;
  }
  return bits_f32(sign | ((exp + 112u) << 23) | (man << 13));
}

/* Round-to-nearest, ties-to-even narrowing, with overflow to inf and gradual
 * underflow into binary16 subnormals. */
uint16_t nibble_oracle_f32_to_f16(float f) {
  const uint32_t x = f32_bits(f);
  const uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
  const uint32_t ax = x & 0x7fffffffu;

  if (ax >= 0x7f800000u) /* inf or nan (quiet the nan, keep a payload bit) */
    return (uint16_t)(sign | (ax > 0x7f800000u ? 0x7e00u : 0x7c00u));

  const int e = (int)(ax >> 23) - 127; /* unbiased binary32 exponent */
  if (e >= 16) return (uint16_t)(sign | 0x7c00u);

  uint32_t full = (ax & 0x7fffffu) | 0x800000u; /* 24-bit significand */
  int shift;                                    /* bits dropped from `full` */
  uint32_t exp_field;
  if (e >= -14) { /* normal binary16 */
    shift = 13;
    exp_field = (uint32_t)(e + 15);
  } else { /* subnormal binary16 (or rounds to zero) */
    if (ax == 0) return sign;
    shift = 13 + (-14 - e);
    if (shift > 25) return sign; /* below half of the smallest subnormal */
    exp_field = 0;
  }
  uint32_t kept = full >> shift;
  const uint32_t rem = full & ((1u << shift) - 1u);
  const uint32_t half = 1u << (shift - 1);
  if (exp_field) kept &= 0x3ffu; /* drop the implicit bit for normals */
  uint32_t out = (exp_field << 10) | kept;
  if (rem > half || (rem == half && (kept & 1u))) out += 1u; /* carries into exp */
  return (uint16_t)(sign | out);
}

void nibble_oracle_f32_to_f16_array(const float* in, uint16_t* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = nibble_oracle_f32_to_f16(in[i]);
}

void nibble_oracle_f16_to_f32_array(const uint16_t* in, float* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = nibble_oracle_f16_to_f32(in[i]);
}

/* ------------------------------------------------------------------------- */
/* pack / unpack  (quant.py:164-196)                                          */
/* ------------------------------------------------------------------------- */

/* qu: uint8 [K, N] in [0, 15] -> packed uint32 [K/8, N].
 * Returns 0, or -1 if K % 8 != 0, or -2 if a value exceeds 15
 * (the reference raises ValueError for both, quant.py:172-175). */
int nibble_oracle_pack(const uint8_t* qu, int64_t K, int64_t N, uint32_t* packed) {
  if (K % 8) return -1;
  for (int64_t i = 0; i < K * N; ++i)
    if (qu[i] > 15) return -2;
  for (int64_t r = 0; r < K / 8; ++r) {
    for (int64_t n = 0; n < N; ++n) {
      uint32_t w = 0;
      for (int k = 0; k < 8; ++k) w |= (uint32_t)(qu[(r * 8 + k) * N + n] & 0xFu) << (4 * kSlotForK[k]);
      packed[r * N + n] = w;
    }
  }
  return 0;
}

/* packed uint32 [rows, N] -> uint8 [rows*8, N] */
void nibble_oracle_unpack(const uint32_t* packed, int64_t rows, int64_t N, uint8_t* qu) {
  for (int64_t r = 0; r < rows; ++r)
    for (int k = 0; k < 8; ++k)
      for (int64_t n = 0; n < N; ++n)
        qu[(r * 8 + k) * N + n] = (uint8_t)((packed[r * N + n] >> (4 * kSlotForK[k])) & 0xFu);
}

/* ------------------------------------------------------------------------- */
/* RTN quantiser  (quant.py:127-161, default clip_search=False)               */
/* ------------------------------------------------------------------------- */

/* W fp32 [K, N] -> qu uint8 [K, N] in [0,15], scales_f32 fp32 [K/G, N] (the
 * un-rounded scales the reference divides by) and scales_f16 [K/G, N].
 * scale = max(max|w| / 7, 1e-8); q = clamp(round_half_even(w / scale), -8, 7).
 * Returns -1 if K % G or G % 8 is non-zero (quant.py:138-141). */
int nibble_oracle_quantize_rtn(const float* W, int64_t K, int64_t N, int64_t G, uint8_t* qu,
                               float* scales_f32, uint16_t* scales_f16) {
  if (G <= 0 || K % G || G % 8) return -1;
  const float floor_scale = 1e-8f;
  for (int64_t g = 0; g < K / G; ++g) {
    for (int64_t n = 0; n < N; ++n) {
      float amax = 0.0f;
      for (int64_t k = g * G; k < (g + 1) * G; ++k) {
        const float a = fabsf(W[k * N + n]);
        if (a > amax) amax = a;
      }
      float s = amax / 7.0f;
      if (s < floor_scale) s = floor_scale;
      scales_f32[g * N + n] = s;
      scales_f16[g * N + n] = nibble_oracle_f32_to_f16(s);
      for (int64_t k = g * G; k < (g + 1) * G; ++k) {
        float q = nearbyintf(W[k * N + n] / s); /* FE_TONEAREST: ties to even */
        if (q < -8.0f) q = -8.0f;
        if (q > 7.0f) q = 7.0f;
        qu[k * N + n] = (uint8_t)((int)q + 8);
      }
    }
  }
  return 0;
}

/* ------------------------------------------------------------------------- */
/* dequantize  (quant.py:199-204)                                             */
/* ------------------------------------------------------------------------- */

/* out fp16 [K, N] = f16( (nibble - 8) * f32(scale) ).  The product of a 4-bit
 * integer and an 11-bit significand is exact in binary32, so this is one RNE
 * rounding of the exact real product. */
void nibble_oracle_dequantize(const uint32_t* packed, const uint16_t* scales, int64_t K, int64_t N,
                              int64_t G, uint16_t* out) {
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < K / 8; ++r) {
    for (int k = 0; k < 8; ++k) {
      const int64_t kk = r * 8 + k;
      const uint16_t* srow = scales + (kk / G) * N;
      uint16_t* orow = out + kk * N;
      for (int64_t n = 0; n < N; ++n) {
        const int nib = (int)((packed[r * N + n] >> (4 * kSlotForK[k])) & 0xFu);
        orow[n] = nibble_oracle_f32_to_f16((float)(nib - 8) * nibble_oracle_f16_to_f32(srow[n]));
      }
    }
  }
}

/* ------------------------------------------------------------------------- */
/* reference matmul  (quant.py:207-215)                                       */
/* ------------------------------------------------------------------------- */

/* Y fp16 [M, N] = f16( X_f32 @ W_f32 ), X fp16 [M, K], W fp16 [K, N] (the
 * dequantized weight).  Accumulation in binary32, k ascending: every output
 * is acc = acc + x[k] * w[k] (a rounded product, then a rounded sum; this
 * file is built with -ffp-contract=off) for k = 0 .. K - 1.
 *
 * As the reference converts the whole weight to binary32 once
 * (dequantize(qw).float()), so does this: W and X are widened first, then
 * blocks of 8 rows x 256 columns accumulate together (the per-output order
 * is unchanged, so is every bit).  Below 4 rows widening the whole weight
 * costs more than it saves: the rows are done one by one. */
static void matmul_f32_rows(const uint16_t* X, const uint16_t* W, int64_t M, int64_t K, int64_t N,
                            uint16_t* Y, float* Yf32);

void nibble_oracle_matmul_f32(const uint16_t* X, const uint16_t* W, int64_t M, int64_t K, int64_t N,
                              uint16_t* Y, float* Yf32) {
  enum { MB = 8, NB = 256 };
  if (M < 4) {
    matmul_f32_rows(X, W, M, K, N, Y, Yf32);
    return;
  }
  float* w32 = (float*)malloc((size_t)(K * N > 0 ? K * N : 1) * sizeof(float));
  float* x32 = (float*)malloc((size_t)(M * K > 0 ? M * K : 1) * sizeof(float));
  if (w32 == NULL || x32 == NULL) {
    free(w32);
    free(x32);
    matmul_f32_rows(X, W, M, K, N, Y, Yf32);
    return;
  }
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < K * N; ++i) w32[i] = nibble_oracle_f16_to_f32(W[i]);
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < M * K; ++i) x32[i] = nibble_oracle_f16_to_f32(X[i]);
#pragma omp parallel for collapse(2) schedule(static)
  for (int64_t mb = 0; mb < M; mb += MB) {
    for (int64_t nb = 0; nb < N; nb += NB) {
      float acc[MB][NB];
      const int64_t rows = (mb + MB < M) ? MB : M - mb;
      const int64_t cols = (nb + NB < N) ? NB : N - nb;
      for (int64_t r = 0; r < rows; ++r)
        for (int64_t c = 0; c < cols; ++c) acc[r][c] = 0.0f;
      for (int64_t k = 0; k < K; ++k) {
        const float* wrow = w32 + k * N + nb;
        for (int64_t r = 0; r < rows; ++r) {
          const float x = x32[(mb + r) * K + k];
          float* a = acc[r];
#pragma omp simd
          for (int64_t c = 0; c < cols; ++c) a[c] = a[c] + x * wrow[c];
        }
      }
      for (int64_t r = 0; r < rows; ++r)
        for (int64_t c = 0; c < cols; ++c) {
          const int64_t o = (mb + r) * N + nb + c;
          if (Yf32) Yf32[o] = acc[r][c];
          Y[o] = nibble_oracle_f32_to_f16(acc[r][c]);
        }
    }
  }
  free(w32);
  free(x32);
}

/* The same product without the widened copies (used when they cannot be
 * allocated): one row at a time, each weight widened as it is read. */
static void matmul_f32_rows(const uint16_t* X, const uint16_t* W, int64_t M, int64_t K, int64_t N,
                            uint16_t* Y, float* Yf32) {
  const int64_t NB = 256;
#pragma omp parallel for collapse(2) schedule(static)
  for (int64_t m = 0; m < M; ++m) {
    for (int64_t nb = 0; nb < N; nb += NB) {
      float acc[256];
      const int64_t ne = (nb + NB < N) ? nb + NB : N;
      for (int64_t n = nb; n < ne; ++n) acc[n - nb] = 0.0f;
      for (int64_t k = 0; k < K; ++k) {
        const float x = nibble_oracle_f16_to_f32(X[m * K + k]);
        const uint16_t* wrow = W + k * N;
        for (int64_t n = nb; n < ne; ++n) acc[n - nb] += x * nibble_oracle_f16_to_f32(wrow[n]);
      }
      for (int64_t n = nb; n < ne; ++n) {
        if (Yf32) Yf32[m * N + n] = acc[n - nb];
        Y[m * N + n] = nibble_oracle_f32_to_f16(acc[n - nb]);
      }
    }
  }
}

/* Same product in binary64 (no fp16 output rounding): the brute-force value the
 * fp32 paths are measured against. */
void nibble_oracle_matmul_f64(const uint16_t* X, const uint16_t* W, int64_t M, int64_t K, int64_t N,
                              double* Y) {
#pragma omp parallel for collapse(2) schedule(static)
  for (int64_t m = 0; m < M; ++m) {
    for (int64_t n = 0; n < N; ++n) {
      double acc = 0.0;
      for (int64_t k = 0; k < K; ++k)
        acc += (double)nibble_oracle_f16_to_f32(X[m * K + k]) * (double)nibble_oracle_f16_to_f32(W[k * N + n]);
      Y[m * N + n] = acc;
    }
  }
}

int nibble_oracle_max_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

void nibble_oracle_set_threads(int n) {
#ifdef _OPENMP
  if (n > 0) omp_set_num_threads(n);
#else
  (void)n;
#endif
}
