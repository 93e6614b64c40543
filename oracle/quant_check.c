/*
 * quant_check.c -- TEST INFRASTRUCTURE (checker only, never shipped or timed).
 *
 * Host restatement of the FP8 quantizer of the append kernels
 * (pipeswift_amd/csrc/psk_common.h: make_qscale, QuantConv) and sweeps that
 * compare its bytes with those of the IEEE fp32 quotient path, which is what
 * the reference's quantization computes: x.float() / scale, clamp to +-448,
 * then float8_e4m3fn (reference: pipeswift/utils/fp8_kv.py:75-77 at scale 1,
 * pipeswift/utils/triton_kernels/reshape_and_cache.py:66-77).
 *
 * The kernel sequence, for a per-tensor scale s (the same in every lane):
 *   r    = RN(1 / |s|)                         once per wave
 *   fast = 2^-80 <= |s| < 2^100
 *   fast:  a = |x|;  y = RN(a * r);  e = fma(-y, |s|, a);  m = fma(e, r, y)
 *   else:  m = |x| / |s|                         (IEEE division)
 *   byte = e4m3fn_rne(min(m, 448)) | (sign(x) ^ sign(s))
 *          (min: the kernel's unsigned min on the bits of m >= +0 or NaN,
 *           the same as IEEE minNum there: NaN and +inf -> 448)
 *   NaN quotient (fast: the bits of y read as unsigned exceed +inf's, i.e.
 *   y is NaN, which with r finite and positive is exactly x NaN; else: m is
 *   NaN) -> policy byte:
 *          0xFE (clamp_min, the reference's Triton clamp) or 0x7F | sign(x) (torch)
 * The IEEE path: q = x / s; NaN -> the same policy byte; else
 *   byte = e4m3fn_rne(clamp(q, -448, 448)).
 * The GPU code runs with f32 denormals preserved (IEEE mode); x86 SSE arithmetic
 * without FTZ/DAZ is the same IEEE binary32 arithmetic, and fmaf is the fused
 * multiply-add with one rounding, as v_fma_f32.  Build without -ffast-math.
 *
 * Exported for ctypes (tests/test_quant_division.py):
 *   qc_e4m3(x, n, out)                   E4M3FN RNE bytes of clamp(x), NaN -> 0x7F|sign
 *   qc_quantize(x, n, s, policy, out)    the kernel's bytes for one scale
 *   qc_sweep_all(kind, amax_kind, variant, out, bad)  every 16-bit input
 *        pattern (bf16 or f16) x every scale RN(a / 448) for a over all finite
 *        positive 16-bit patterns of amax_kind
 *   qc_sweep_random(seed, n, mode, variant, out, bad)  sampled fp32 inputs and
 *        scales
 * Sweep counters out[0..4]: cases, fast-path cases, clamped-magnitude
 * mismatches (min(m, 448) against |clamp(x / s)| bit for bit, where the IEEE
 * quotient is not NaN), byte mismatches (both NaN policies), and magnitude
 * mismatches where |clamp(x / s)| is not below 2^-20.  Magnitudes below 2^-20
 * convert to a signed zero in E4M3 (its smallest subnormal is 2^-9), so there
 * only the sign has to agree; the kernel's sequence may leave such a quotient
 * inexact when |x| < 2^-100.
 * bad[0..2]: the first byte-mismatching (x bits, s bits, kernel magnitude bits),
 * or the first magnitude mismatch when no byte differs.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

static inline uint32_t fbits(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return u;
}
static inline float bitsf(uint32_t u) {
  float f;
  memcpy(&f, &u, 4);
  return f;
}

/* E4M3FN (bias 7, max 448, no infinities) of a value already clamped to
 * [-448, 448], round to nearest even; NaN -> 0x7F | sign. */
static inline uint8_t e4m3_of_clamped(float v) {
  const uint32_t u = fbits(v);
  const uint8_t sign = (uint8_t)((u >> 24) & 0x80u);
  if (isnan(v)) return (uint8_t)(sign | 0x7Fu);
  const float a = fabsf(v);
  if (a < 0x1p-6f) {
    /* subnormal range: multiples of 2^-9, RNE by the current rounding mode;
     * 8 * 2^-9 rounds up to the smallest normal, whose code is 0x08 */
    const int m = (int)nearbyintf(a * 512.0f);
    return (uint8_t)(sign | (uint8_t)m);
  }
  uint32_t au = fbits(a);
  au += 0x7FFFFu + ((au >> 20) & 1u); /* RNE to 3 mantissa bits */
  const int e = (int)(au >> 23) - 127;
  const uint32_t m3 = (au >> 20) & 7u;
  return (uint8_t)(sign | (uint8_t)(((e + 7) << 3) | (int)m3));
}

static inline float med3_448(float q) { return q < -448.0f ? -448.0f : (q > 448.0f ? 448.0f : q); }

static inline uint8_t sign_of(float x) { return (uint8_t)((fbits(x) >> 24) & 0x80u); }

static inline uint8_t nan_byte(float x, int policy) { return policy == 0 ? (uint8_t)0xFE : (uint8_t)(0x7Fu | sign_of(x)); }

typedef struct {
  float s, r;   /* |scale| and RN(1 / |scale|) */
  int fast;
  uint8_t neg;  /* 0x80 for a negative scale: flips every output sign */
  float raw;    /* the scale as given */
} qscale;

static inline qscale make_qscale(float s) {
  qscale q;
  q.raw = s;
  q.s = fabsf(s);
  q.r = 1.0f / q.s;
  q.fast = q.s >= 0x1p-80f && q.s < 0x1p100f;
  q.neg = signbit(s) ? 0x80 : 0;
  return q;
}

/* variant 0 is the kernel's sequence.  The others are planted mistakes for
 * the tests to show that the sweeps detect them: 1 drops the FMA correction
 * (the magnitude is RN(|x| * RN(1/s))), 2 drops the range gate (every scale
 * takes the reciprocal path). */
static int g_variant = 0;

/* The kernel's byte; *mag = min(m, 448), the value the converter receives. */
static inline uint8_t kernel_byte(float x, const qscale* q, int policy, float* mag) {
  float m;
  int nanq;
  if (q->fast || g_variant == 2) {
    const float a = fabsf(x);
    const float y = a * q->r;
    if (g_variant == 1) {
      m = y;
    } else {
      const float e = fmaf(-y, q->s, a);
      m = fmaf(e, q->r, y);
    }
    nanq = fbits(y) > 0x7F800000u;
  } else {
    m = fabsf(x) / q->s;
    nanq = isnan(m);
  }
  *mag = fminf(m, 448.0f);
  if (nanq) return nan_byte(x, policy);
  return (uint8_t)(e4m3_of_clamped(*mag) | (sign_of(x) ^ q->neg));
}

/* The IEEE quotient path's byte; *mag = |clamp(x / s)| or NaN. */
static inline uint8_t ieee_byte(float x, float s, int policy, float* mag) {
  const float qv = x / s;
  if (isnan(qv)) {
    *mag = NAN;
    return nan_byte(x, policy);
  }
  const float c = med3_448(qv);
  *mag = fabsf(c);
  return e4m3_of_clamped(c);
}

void qc_e4m3(const float* x, int64_t n, uint8_t* out) {
  for (int64_t i = 0; i < n; ++i) out[i] = isnan(x[i]) ? nan_byte(x[i], 1) : e4m3_of_clamped(med3_448(x[i]));
}

void qc_quantize(const float* x, int64_t n, float s, int policy, uint8_t* out) {
  g_variant = 0;
  const qscale q = make_qscale(s);
  float mag;
  for (int64_t i = 0; i < n; ++i) out[i] = kernel_byte(x[i], &q, policy, &mag);
}

static float half_to_float(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  const uint32_t e = (h >> 10) & 0x1Fu, m = h & 0x3FFu;
  if (e == 0x1F) return bitsf(sign | 0x7F800000u | (m << 13));
  if (e == 0) {
    const float f = (float)m * 0x1p-24f;
    return sign ? -f : f;
  }
  return bitsf(sign | ((e + 112u) << 23) | (m << 13));
}

static float pattern_to_float(int kind, uint32_t p) {
  return kind == 0 ? bitsf(p << 16) : half_to_float((uint16_t)p);
}

typedef struct {
  int64_t cases, fast, mag_bad, byte_bad, big_bad;
  uint32_t bad[3];
  int have_bad, have_byte_bad;
} tally;

static inline void check_one(float x, const qscale* q, tally* t) {
  t->cases++;
  t->fast += q->fast;
  int byte_bad = 0, mag_bad = 0;
  float km = 0.0f, rm = 0.0f;
  for (int policy = 0; policy < 2; ++policy) {
    const uint8_t kb = kernel_byte(x, q, policy, &km);
    const uint8_t rb = ieee_byte(x, q->raw, policy, &rm);
    byte_bad |= kb != rb;
  }
  if (!isnan(rm) && fbits(km) != fbits(rm)) {
    mag_bad = 1;
    t->mag_bad++;
    if (!(rm < 0x1p-20f)) t->big_bad++;
  }
  if (byte_bad) t->byte_bad++;
  if ((byte_bad && !t->have_byte_bad) || (mag_bad && !t->have_bad)) {
    t->bad[0] = fbits(x);
    t->bad[1] = fbits(q->s);
    t->bad[2] = fbits(km);
    t->have_bad = 1;
    t->have_byte_bad |= byte_bad;
  }
}

static void merge(tally* dst, const tally* src) {
  dst->cases += src->cases;
  dst->fast += src->fast;
  dst->mag_bad += src->mag_bad;
  dst->byte_bad += src->byte_bad;
  dst->big_bad += src->big_bad;
  if ((src->have_byte_bad && !dst->have_byte_bad) || (src->have_bad && !dst->have_bad)) {
    memcpy(dst->bad, src->bad, sizeof(dst->bad));
    dst->have_bad = 1;
    dst->have_byte_bad |= src->have_byte_bad;
  }
}

static void emit(const tally* t, int64_t* out, uint32_t* bad) {
  out[0] = t->cases;
  out[1] = t->fast;
  out[2] = t->mag_bad;
  out[3] = t->byte_bad;
  out[4] = t->big_bad;
  if (bad) memcpy(bad, t->bad, sizeof(t->bad));
}

/* Every input pattern of `kind` (0 bf16, 1 f16; all 65536, NaNs and
 * infinities included) against the scale RN(a / 448) of every finite positive
 * pattern a of `amax_kind` -- the per-tensor scale the amax kernel produces. */
void qc_sweep_all(int kind, int amax_kind, int variant, int64_t* out, uint32_t* bad) {
  g_variant = variant;
  static float xs[65536];
  for (uint32_t p = 0; p < 65536u; ++p) xs[p] = pattern_to_float(kind, p);
  const uint32_t amax_hi = amax_kind == 0 ? 0x7F80u : 0x7C00u; /* first non-finite pattern */
  tally total;
  memset(&total, 0, sizeof(total));
#pragma omp parallel
  {
    tally t;
    memset(&t, 0, sizeof(t));
#pragma omp for schedule(dynamic, 64)
    for (int64_t a = 1; a < (int64_t)amax_hi; ++a) {
      const float amax = pattern_to_float(amax_kind, (uint32_t)a);
      const qscale q = make_qscale(amax / 448.0f);
      for (uint32_t p = 0; p < 65536u; ++p) check_one(xs[p], &q, &t);
    }
#pragma omp critical
    merge(&total, &t);
  }
  emit(&total, out, bad);
}

static inline uint64_t splitmix(uint64_t* st) {
  uint64_t z = (*st += 0x9E3779B97F4A7C15ull);
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

static float finite_f32(uint64_t r) {
  uint32_t u = (uint32_t)r;
  if ((u & 0x7F800000u) == 0x7F800000u) u &= 0xBFFFFFFFu; /* fold inf/NaN into finite values */
  return bitsf(u);
}

/* Sampled fp32 cases, n per call, split over threads by index (deterministic).
 *   mode 0: x a random finite fp32 pattern, s = RN(|a| / 448) for a random finite fp32 a
 *   mode 1: adversarial, quotients whose significand lies within 2^-10 of 2 (where
 *           RN(x * RN(1/s)) can miss x/s by more than an ulp): s random in the fast
 *           range, x = RN(q * s) for such a q
 *   mode 2: x random in [-2^20, 2^20] magnitude range, s a random fp32 in [2^-80, 2^100)
 *   mode 3: s near the gate (2^-80 and 2^100, a few ulps either side), x random finite */
void qc_sweep_random(uint64_t seed, int64_t n, int mode, int variant, int64_t* out, uint32_t* bad) {
  g_variant = variant;
  tally total;
  memset(&total, 0, sizeof(total));
#pragma omp parallel
  {
    tally t;
    memset(&t, 0, sizeof(t));
#pragma omp for schedule(static)
    for (int64_t i = 0; i < n; ++i) {
      uint64_t st = seed ^ ((uint64_t)i * 0xD6E8FEB86659FD93ull);
      const uint64_t r0 = splitmix(&st), r1 = splitmix(&st), r2 = splitmix(&st);
      float x, s;
      if (mode == 0) {
        x = finite_f32(r0);
        s = fabsf(finite_f32(r1)) / 448.0f;
      } else if (mode == 1) {
        const int se = (int)(r0 % 170u) - 75; /* s in [2^-75, 2^95) */
        s = ldexpf(1.0f + (float)(r1 & 0x7FFFFFu) * 0x1p-23f, se);
        const float qsig = 2.0f - (float)((r1 >> 23) & 0x3FFFu) * 0x1p-24f; /* (2 - 2^-10, 2] */
        const int qe = (int)(r2 % 40u) - 20;
        const float q = ldexpf(qsig, qe) * ((r2 >> 40) & 1u ? -1.0f : 1.0f);
        x = q * s;
        if (!isfinite(x)) x = 1.0f;
      } else if (mode == 2) {
        const int xe = (int)(r0 % 40u) - 20;
        x = ldexpf(1.0f + (float)(r0 >> 40 & 0x7FFFFFu) * 0x1p-23f, xe) * ((r0 >> 63) ? -1.0f : 1.0f);
        const int se = (int)(r1 % 180u) - 80;
        s = ldexpf(1.0f + (float)(r1 >> 40 & 0x7FFFFFu) * 0x1p-23f, se);
      } else {
        const int k = (int)(r1 % 64u) - 32;
        const float edge = (r1 >> 32) & 1u ? 0x1p-80f : 0x1p100f;
        s = bitsf((uint32_t)((int64_t)fbits(edge) + k));
        x = finite_f32(r0);
      }
      if (!(s > 0.0f) || !isfinite(s)) s = 1.0f;
      const qscale q = make_qscale(s);
      check_one(x, &q, &t);
      (void)r2;
    }
#pragma omp critical
    merge(&total, &t);
  }
  emit(&total, out, bad);
}
