/* Host restatement of the division used by the GEMV RMSNorm prologue
 * (chomik-grad_amd/csrc/k_gemv.hip, quotient()): q = x * inv, then one Newton
 * correction with the exact residual fma(-q, d, x), sign taken from x.  It is
 * compared with IEEE x / d after rounding both to the storage type:
 *   fp16: every finite fp16 x over every normal fp16 d;
 *   bf16: every bf16 x with |x| in [2^-100, 2^100] or zero, over every bf16 d
 *         in [2^-9, 2^64] (the domain the kernel admits);
 * with inv = RN(1/d) moved by -2..+2 ulp.  argv[1] = stride over divisors
 * (1 = exhaustive); argv[2] = "plain" drops the Newton correction (a planted
 * mistake the comparison must catch).  Prints the mismatch count per format;
 * exit status 1 on any mismatch. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

static float half_to_float(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  const int exp = (h >> 10) & 0x1f;
  const uint32_t man = h & 0x3ffu;
  if (exp == 0) return sign ? -ldexpf((float)man, -24) : ldexpf((float)man, -24);
  return u2f(sign | (uint32_t)(exp - 15 + 127) << 23 | man << 13);
}

/* float -> fp16 bits, round to nearest even (finite inputs; overflow -> inf) */
static uint16_t float_to_half(float f) {
  const uint32_t u = f2u(f);
  const uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
  const float a = fabsf(f);
  if (isnan(f)) return sign | 0x7e00u;
  if (a >= 65520.0f) return sign | 0x7c00u;
  if (a < 0x1p-14f) { /* subnormal range: quantum 2^-24 */
    const float q = nearbyintf(a * 0x1p24f); /* default rounding mode is RNE */
    return sign | (uint16_t)q;
  }
  int e;
  const float m = frexpf(a, &e); /* a = m * 2^e, m in [0.5, 1) */
  const float scaled = nearbyintf(m * 2048.0f); /* 11 significant bits */
  uint32_t bits = (uint32_t)scaled;
  int exp = e - 1 + 15;
  if (bits == 2048) { bits = 1024; exp += 1; }
  if (exp >= 31) return sign | 0x7c00u;
  return sign | (uint16_t)(exp << 10) | (uint16_t)(bits - 1024);
}

static uint16_t float_to_bf16(float f) {
  uint32_t u = f2u(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

static int plain = 0;

static float quotient(float x, float d, float inv) {
  const float q = x * inv;
  if (plain) return q;
  return copysignf(fmaf(fmaf(-q, d, x), inv, q), x);
}

int main(int argc, char** argv) {
  const int stride = argc > 1 ? atoi(argv[1]) : 1;
  plain = argc > 2 && strcmp(argv[2], "plain") == 0;
  long long bad_total = 0;
  for (int fmt = 0; fmt < 2; ++fmt) {
    long long cases = 0, bad = 0;
    for (uint32_t db = 0; db < 0x8000u; db += (uint32_t)stride) {
      float d;
      if (fmt == 0) {
        if ((db & 0x7c00u) == 0 || (db & 0x7c00u) == 0x7c00u) continue;
        d = half_to_float((uint16_t)db);
      } else {
        if ((db & 0x7f80u) == 0 || (db & 0x7f80u) == 0x7f80u) continue;
        d = u2f(db << 16);
        if (d < 0x1p-9f || d > 0x1p64f) continue;
      }
      const float inv0 = 1.0f / d;
      for (int k = -2; k <= 2; ++k) {
        const float inv = u2f(f2u(inv0) + (uint32_t)k);
        for (uint32_t xb = 0; xb < 0x10000u; ++xb) {
          float x;
          if (fmt == 0) {
            if ((xb & 0x7c00u) == 0x7c00u) continue;
            x = half_to_float((uint16_t)xb);
          } else {
            if ((xb & 0x7f80u) == 0x7f80u) continue;
            x = u2f(xb << 16);
            const float ax = fabsf(x);
            if (!(ax == 0.0f || (ax >= 0x1p-100f && ax <= 0x1p100f))) continue;
          }
          const float ref = x / d, q = quotient(x, d, inv);
          const int differ = fmt == 0 ? float_to_half(ref) != float_to_half(q)
                                      : float_to_bf16(ref) != float_to_bf16(q);
          bad += differ;
          ++cases;
        }
      }
    }
    printf("%s cases %lld mismatches %lld\n", fmt == 0 ? "fp16" : "bf16", cases, bad);
    bad_total += bad;
  }
  return bad_total ? 1 : 0;
}
