/*
 * w4a16_oracle.c - CPU restatement of the reference's W4A16 ("ARC") decode-linear math.
 *
 * TEST INFRASTRUCTURE ONLY. This file is the checker the parity tests, smoke() and bench.py's
 * cpu_baseline leg compare the HIP library against. Nothing in the product links or calls it.
 *
 * Each function cites the reference code it restates (paths relative to the reference checkout):
 *   fko_dequant            csrc/kernels/decode_quant_linear/arc_w4a16.cu:160-181 (dequant_w4a16_kernel)
 *                          and src/fast_kernels/benchmarking/decode_linear_w4a16.py:184-190
 *   fko_pack_packets       arc_w4a16.cu:87-122 (pack_arc_packets_kernel)
 *   fko_dequant_packets    arc_w4a16.cu:183-220 (dequant_arc_packets_kernel)
 *   fko_group_sums         arc_w4a16.cu:124-158 (compute_arc_group_sums_kernel)
 *   fko_gemv               decode_linear_w4a16.py:177-192 (_explicit_reference_output):
 *                          fp32 weights alpha*q + beta, matmul, cast to the activation dtype
 *   fko_gemv_f32           the same with fp32 accumulation, as the reference computes it (the
 *                          CPU baseline bench.py times)
 *   fko_reduce_partials    arc_w4a16.cu:388-402
 * Conversions (fko_f32_to_f16_bits, fko_f32_to_bf16_bits) are IEEE round-to-nearest-even,
 * written from the format definitions.
 *
 * Deliberate difference from the reference: fko_gemv accumulates the fp32 products in double,
 * so it is a tighter oracle than the reference's fp32 matmul; only the final cast rounds.
 */
#include <math.h>
#include <stddef.h>
#include <stdint.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

#define FKO_TILE 128

static float bits_to_f32(uint32_t u) {
  float f;
  memcpy(&f, &u, sizeof(f));
  return f;
}

static uint32_t f32_to_bits(float f) {
  uint32_t u;
  memcpy(&u, &f, sizeof(u));
  return u;
}

/* IEEE binary16 -> binary32 (exact). */
float fko_f16_bits_to_f32(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  const uint32_t exp = (h >> 10) & 0x1fu;
  const uint32_t man = h & 0x3ffu;
  if (exp == 0) {
    /* zero or subnormal: man * 2^-24 */
    const float v = (float)man * 5.9604644775390625e-08f;
    return (sign != 0) ? -v : v;
  }
  if (exp == 0x1f) {
    return bits_to_f32(sign | 0x7f800000u | (man << 13));
  }
  return bits_to_f32(sign | ((exp + 112u) << 23) | (man << 13));
}

/* IEEE binary32 -> binary16, round to nearest, ties to even; overflow -> inf; NaN stays NaN. */
uint16_t fko_f32_to_f16_bits(float f) {
  const uint32_t u = f32_to_bits(f);
  const uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
  const uint32_t abs = u & 0x7fffffffu;
  if (abs >= 0x7f800000u) {
    return (uint16_t)(sign | 0x7c00u | (abs > 0x7f800000u ? 0x200u : 0u));
  }
  const int32_t exp = (int32_t)(abs >> 23) - 127;
  uint32_t man = (abs & 0x7fffffu) | 0x800000u; /* 24-bit significand */
  if (exp > 15) {
    return (uint16_t)(sign | 0x7c00u);
  }
  int shift;           /* bits to drop from the 24-bit significand */
  uint32_t biased_exp; /* binary16 exponent field before rounding */
  if (exp >= -14) {
    shift = 13;
    biased_exp = (uint32_t)(exp + 15);
  } else {
    /* subnormal binary16: value = m * 2^-24 */
    shift = 13 + (-14 - exp);
    biased_exp = 0;
    if (shift > 24) {
      return sign; /* below half of the smallest subnormal: rounds to zero */
    }
  }
  const uint32_t kept = man >> shift;
  const uint32_t rem = man & ((1u << shift) - 1u);
  const uint32_t half = 1u << (shift - 1);
  uint32_t r = kept;
  if (rem > half || (rem == half && (kept & 1u))) {
    r += 1u;
  }
  uint32_t out;
  if (biased_exp == 0) {
    out = r; /* may carry into the smallest normal, which is the correct encoding */
  } else {
    /* r holds the implicit bit at bit 10; a carry to bit 11 bumps the exponent */
    out = (biased_exp << 10) + (r - 0x400u);
    if (out >= 0x7c00u) {
      out = 0x7c00u;
    }
  }
  return (uint16_t)(sign | out);
}

float fko_bf16_bits_to_f32(uint16_t b) { return bits_to_f32((uint32_t)b << 16); }

uint16_t fko_f32_to_bf16_bits(float f) {
  const uint32_t u = f32_to_bits(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) {
    return (uint16_t)((u >> 16) | 0x40u);
  }
  const uint32_t lsb = (u >> 16) & 1u;
  return (uint16_t)((u + 0x7fffu + lsb) >> 16);
}

static inline float act_to_f32(uint16_t v, int act_bf16) {
  return act_bf16 ? fko_bf16_bits_to_f32(v) : fko_f16_bits_to_f32(v);
}

static inline uint16_t f32_to_act(float v, int act_bf16) {
  return act_bf16 ? fko_f32_to_bf16_bits(v) : fko_f32_to_f16_bits(v);
}

/* Code k of row n: low nibble of byte k/2 for even k, high nibble for odd k. */
static inline uint32_t code_at(const uint8_t* q_row, int k) {
  const uint8_t b = q_row[k >> 1];
  return (k & 1) ? (uint32_t)(b >> 4) : (uint32_t)(b & 0x0fu);
}

/* fp32 weight value alpha*q + beta: product then sum, each rounded to fp32 (exact for the
 * quantisation recipes in use). Built with -ffp-contract=off so the two roundings stay. */
static inline float weight_f32(float alpha, float beta, uint32_t q) {
  const float prod = alpha * (float)q;
  return prod + beta;
}

/* W[n,k] = half_rn(alpha*q + beta). */
void fko_dequant(const uint8_t* q, const uint16_t* alpha, const uint16_t* beta, uint16_t* out,
                 int n, int k, int group_size) {
  const int ng = k / group_size;
#pragma omp parallel for schedule(static)
  for (int r = 0; r < n; ++r) {
    const uint8_t* q_row = q + (size_t)r * (size_t)(k / 2);
    for (int c = 0; c < k; ++c) {
      const int g = c / group_size;
      const float a = fko_f16_bits_to_f32(alpha[(size_t)r * ng + g]);
      const float b = fko_f16_bits_to_f32(beta[(size_t)r * ng + g]);
      out[(size_t)r * k + c] = fko_f32_to_f16_bits(weight_f32(a, b, code_at(q_row, c)));
    }
  }
}

size_t fko_packet_stride_bytes(int group_size) {
  return (size_t)FKO_TILE * (size_t)(group_size / 2) + 2u * FKO_TILE * 2u;
}

/* Packet (tile t, group g) at row t*NG + g: code word w of column c at byte (w*128 + c)*4,
 * then alpha[128], then beta[128]. */
void fko_pack_packets(const uint8_t* q, const uint16_t* alpha, const uint16_t* beta,
                      uint8_t* packets, int n, int k, int group_size) {
  const int ng = k / group_size;
  const int words = group_size / 8;
  const size_t stride = fko_packet_stride_bytes(group_size);
  const size_t qb = (size_t)FKO_TILE * (size_t)(group_size / 2);
  for (int t = 0; t < n / FKO_TILE; ++t) {
    for (int g = 0; g < ng; ++g) {
      uint8_t* packet = packets + ((size_t)t * ng + g) * stride;
      for (int c = 0; c < FKO_TILE; ++c) {
        const size_t row = (size_t)t * FKO_TILE + c;
        const uint8_t* src = q + row * (size_t)(k / 2) + (size_t)g * (group_size / 2);
        for (int w = 0; w < words; ++w) {
          memcpy(packet + ((size_t)w * FKO_TILE + c) * 4u, src + (size_t)w * 4u, 4);
        }
        memcpy(packet + qb + (size_t)c * 2u, &alpha[row * ng + g], 2);
        memcpy(packet + qb + FKO_TILE * 2u + (size_t)c * 2u, &beta[row * ng + g], 2);
      }
    }
  }
}

void fko_dequant_packets(const uint8_t* packets, uint16_t* out, int n, int k, int group_size) {
  const int ng = k / group_size;
  const size_t stride = fko_packet_stride_bytes(group_size);
  const size_t qb = (size_t)FKO_TILE * (size_t)(group_size / 2);
#pragma omp parallel for schedule(static)
  for (int r = 0; r < n; ++r) {
    const int t = r / FKO_TILE;
    const int c = r % FKO_TILE;
    for (int col = 0; col < k; ++col) {
      const int g = col / group_size;
      const int within = col % group_size;
      const uint8_t* packet = packets + ((size_t)t * ng + g) * stride;
      uint32_t word;
      memcpy(&word, packet + ((size_t)(within / 8) * FKO_TILE + c) * 4u, 4);
      const uint32_t code = (word >> (4 * (within % 8))) & 0xfu;
      uint16_t a16, b16;
      memcpy(&a16, packet + qb + (size_t)c * 2u, 2);
      memcpy(&b16, packet + qb + FKO_TILE * 2u + (size_t)c * 2u, 2);
      out[(size_t)r * k + col] = fko_f32_to_f16_bits(
          weight_f32(fko_f16_bits_to_f32(a16), fko_f16_bits_to_f32(b16), code));
    }
  }
}

/* sums[b, g] = sum of the group's activations, accumulated in double, rounded once to fp32. */
void fko_group_sums(const uint16_t* x, float* sums, int batch, int k, int group_size,
                    int act_bf16) {
  const int ng = k / group_size;
  for (int b = 0; b < batch; ++b) {
    for (int g = 0; g < ng; ++g) {
      double s = 0.0;
      for (int i = 0; i < group_size; ++i) {
        s += (double)act_to_f32(x[(size_t)b * k + (size_t)g * group_size + i], act_bf16);
      }
      sums[(size_t)b * ng + g] = (float)s;
    }
  }
}

/* y[m, n] = cast( sum_k (alpha*q + beta)[n,k] (fp32) * x[m,k] ), double accumulation. With
 * out_f32 != NULL the unrounded sums are also returned (for error analysis in tests). */
void fko_gemv(const uint16_t* x, const uint8_t* q, const uint16_t* alpha, const uint16_t* beta,
              uint16_t* out, float* out_f32, int batch, int n, int k, int group_size,
              int act_bf16) {
  const int ng = k / group_size;
#pragma omp parallel
  {
    float xf[16384];
    /* Rows of x are converted once per block of K to keep the inner loop on floats. */
#pragma omp for schedule(static)
    for (int r = 0; r < n; ++r) {
      const uint8_t* q_row = q + (size_t)r * (size_t)(k / 2);
      for (int m = 0; m < batch; ++m) {
        double acc = 0.0;
        for (int k0 = 0; k0 < k; k0 += 16384) {
          const int kc = (k - k0) < 16384 ? (k - k0) : 16384;
          for (int i = 0; i < kc; ++i) {
            xf[i] = act_to_f32(x[(size_t)m * k + k0 + i], act_bf16);
          }
          for (int g0 = k0; g0 < k0 + kc; g0 += group_size) {
            const int g = g0 / group_size;
            const float a = fko_f16_bits_to_f32(alpha[(size_t)r * ng + g]);
            const float b = fko_f16_bits_to_f32(beta[(size_t)r * ng + g]);
            for (int i = 0; i < group_size; ++i) {
              const float w = weight_f32(a, b, code_at(q_row, g0 + i));
              acc += (double)w * (double)xf[g0 + i - k0];
            }
          }
        }
        out[(size_t)m * n + r] = f32_to_act((float)acc, act_bf16);
        if (out_f32 != NULL) {
          out_f32[(size_t)m * n + r] = (float)acc;
        }
      }
    }
  }
}

/* fko_gemv with the reference's own arithmetic (decode_linear_w4a16.py:177-192: fp32 weights,
 * fp32 matmul): the products accumulate in float, in k order, then one cast. The CPU baseline that
 * bench.py times; the parity tests use fko_gemv. */
void fko_gemv_f32(const uint16_t* x, const uint8_t* q, const uint16_t* alpha, const uint16_t* beta,
                  uint16_t* out, int batch, int n, int k, int group_size, int act_bf16) {
  const int ng = k / group_size;
#pragma omp parallel
  {
    float xf[16384];
#pragma omp for schedule(static)
    for (int r = 0; r < n; ++r) {
      const uint8_t* q_row = q + (size_t)r * (size_t)(k / 2);
      for (int m = 0; m < batch; ++m) {
        float acc = 0.0f;
        for (int k0 = 0; k0 < k; k0 += 16384) {
          const int kc = (k - k0) < 16384 ? (k - k0) : 16384;
          for (int i = 0; i < kc; ++i) {
            xf[i] = act_to_f32(x[(size_t)m * k + k0 + i], act_bf16);
          }
          for (int g0 = k0; g0 < k0 + kc; g0 += group_size) {
            const int g = g0 / group_size;
            const float a = fko_f16_bits_to_f32(alpha[(size_t)r * ng + g]);
            const float b = fko_f16_bits_to_f32(beta[(size_t)r * ng + g]);
            for (int i = 0; i < group_size; ++i) {
              acc += weight_f32(a, b, code_at(q_row, g0 + i)) * xf[g0 + i - k0];
            }
          }
        }
        out[(size_t)m * n + r] = f32_to_act(acc, act_bf16);
      }
    }
  }
}

/* out[i] = half_rn(sum_s partials[s, i]), slices added in order, fp32. */
void fko_reduce_partials(const float* partials, uint16_t* out, int batch, int n, int splits) {
  const size_t total = (size_t)batch * n;
  for (size_t i = 0; i < total; ++i) {
    float v = 0.0f;
    for (int s = 0; s < splits; ++s) {
      v += partials[(size_t)s * total + i];
    }
    out[i] = fko_f32_to_f16_bits(v);
  }
}

int fko_max_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

void fko_set_threads(int threads) {
#ifdef _OPENMP
  if (threads > 0) {
    omp_set_num_threads(threads);
  }
#else
  (void)threads;
#endif
}
