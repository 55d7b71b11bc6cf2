/* CPU restatement of the C1 and C2 programs for bench.py's cpu_baseline leg:
 * the numpy oracle's algorithm (oracle/ops.py c1_rowsum, c2_reference), in C
 * over host threads (rows split evenly), so the reported CPU figure uses every
 * host core. Test infrastructure: only tests/, smoke() and bench.py's
 * cpu_baseline load it; the plugin never does.
 *
 *   C2 (reference: api.cc:4046-4170 argmax pair rule, api.cc:3982-4044 f16
 *   reductions): per row of bf16 logits, the NaN-propagating maximum and the
 *   lowest index holding it (the first NaN when the row has one); the row
 *   cast to f16 (round to nearest even) and its sum (accumulated in double,
 *   rounded to f32 then f16, as c2_reference), max and min (f16 compares:
 *   NaN propagates).
 *   C1 (reference program_build.zig:10-207 elementwise chain + reduce_sum):
 *   sum over a row of tanh(x*y + 0.5)*x - max(y, 0), in double from the f32
 *   inputs (finite), rounded once to f32.
 *
 * Pinned by tests/test_oracle_c.py: the f16 conversion against numpy for all
 * 65,536 bf16 values, and both programs against the numpy oracle.
 */
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <string.h>

static float bf16_to_f32(uint16_t b) {
  uint32_t u = (uint32_t)b << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

static uint16_t f32_to_bf16_rne(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu)) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

/* IEEE binary32 -> binary16, round to nearest, ties to even. */
uint16_t pjrtx_oracle_f32_to_f16(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  const uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
  const uint32_t exp = (u >> 23) & 0xffu;
  uint32_t man = u & 0x7fffffu;
  if (exp == 0xffu) return (uint16_t)(sign | 0x7c00u | (man ? 0x200u | (man >> 13) : 0u)); /* inf / quiet NaN */
  const int e = (int)exp - 127 + 15; /* biased f16 exponent */
  if (e >= 31) return (uint16_t)(sign | 0x7c00u);
  if (e <= 0) {
    /* subnormal f16 (or zero): value = man' * 2^-24 */
    if (e < -10) return sign; /* below half the smallest subnormal */
    man |= 0x800000u;         /* implicit bit */
    const int shift = 14 - e; /* 24-bit significand -> units of 2^-24 */
    uint32_t q = man >> shift;
    const uint32_t rem = man & ((1u << shift) - 1u), half = 1u << (shift - 1);
    if (rem > half || (rem == half && (q & 1u))) ++q;
    return (uint16_t)(sign | q); /* q may carry into the smallest normal: still correct */
  }
  uint32_t q = ((uint32_t)e << 10) | (man >> 13);
  const uint32_t rem = man & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) ++q; /* a carry may reach infinity: correct */
  return (uint16_t)(sign | q);
}

float pjrtx_oracle_f16_to_f32(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  const uint32_t exp = (h >> 10) & 0x1fu, man = h & 0x3ffu;
  uint32_t u;
  if (exp == 0x1fu) {
    u = sign | 0x7f800000u | (man << 13);
  } else if (exp == 0) {
    float f = (float)man * 5.9604644775390625e-08f; /* man * 2^-24, exact */
    return sign ? -f : f;
  } else {
    u = sign | ((exp - 15 + 127) << 23) | (man << 13);
  }
  float f;
  memcpy(&f, &u, 4);
  return f;
}

typedef struct {
  const void* a;
  const void* b;
  int64_t cols, r0, r1;
  void* o0;
  void* o1;
  void* o2;
  void* o3;
  void* o4;
} Job;

/* The f16 value (as a float) of a bf16 value: bf16's 8-bit significand fits
 * f16's 11 bits, so only magnitudes below f16's normal range (rounded to the
 * 2^-24 grid) and above its largest finite value change; both go through the
 * exact conversion. */
static float bf16_as_f16(float v) {
  const float a = fabsf(v);
  if (a >= 6.103515625e-05f && a <= 65504.f) return v;
  return pjrtx_oracle_f16_to_f32(pjrtx_oracle_f32_to_f16(v));
}

enum { kChunk = 2048 };

static void* c2_rows(void* arg) {
  const Job* j = (const Job*)arg;
  const uint16_t* x = (const uint16_t*)j->a;
  for (int64_t r = j->r0; r < j->r1; ++r) {
    const uint16_t* row = x + r * j->cols;
    float best = -INFINITY;
    int32_t bi = 0;
    int nan_at = -1;
    double sum = 0.0;
    float mx = -INFINITY, mn = INFINITY;
    for (int64_t c0 = 0; c0 < j->cols; c0 += kChunk) {
      const int64_t c1 = c0 + kChunk < j->cols ? c0 + kChunk : j->cols;
      /* chunk maximum and minimum (NaN-free lanes), then the search */
      float cmx = -INFINITY, cmn = INFINITY;
      int cnan = 0;
      double csum = 0.0;
      for (int64_t i = c0; i < c1; ++i) {
        const float v = bf16_to_f32(row[i]);
        cnan |= v != v;
        cmx = v > cmx ? v : cmx;
        cmn = v < cmn ? v : cmn;
        csum += (double)bf16_as_f16(v);
      }
      sum += csum;
      if (cnan && nan_at < 0) {
        for (int64_t i = c0; i < c1; ++i)
          if (bf16_to_f32(row[i]) != bf16_to_f32(row[i])) {
            nan_at = (int)i;
            break;
          }
      }
      if (nan_at < 0 && cmx > best) { /* ties keep the lowest index: strictly greater */
        for (int64_t i = c0; i < c1; ++i)
          if (bf16_to_f32(row[i]) == cmx) {
            bi = (int32_t)i;
            break;
          }
        best = cmx;
      }
      mx = cmx > mx ? cmx : mx;
      mn = cmn < mn ? cmn : mn;
    }
    if (nan_at >= 0) {
      bi = nan_at;
      best = bf16_to_f32(row[nan_at]);
    }
    ((uint16_t*)j->o0)[r] = f32_to_bf16_rne(best);
    ((int32_t*)j->o1)[r] = bi;
    ((uint16_t*)j->o2)[r] = pjrtx_oracle_f32_to_f16((float)sum);
    /* f16 rounding is monotonic: the f16 max / min are the rounded bf16 ones */
    ((uint16_t*)j->o3)[r] = nan_at >= 0 ? 0x7e00u : pjrtx_oracle_f32_to_f16(mx);
    ((uint16_t*)j->o4)[r] = nan_at >= 0 ? 0x7e00u : pjrtx_oracle_f32_to_f16(mn);
  }
  return 0;
}

/* One row of C1 (oracle/c/c1_row.c: a tanh the compiler can vectorize). */
double pjrtx_oracle_c1_row(const float* xr, const float* yr, int64_t cols);

static void* c1_rows(void* arg) {
  const Job* j = (const Job*)arg;
  const float* x = (const float*)j->a;
  const float* y = (const float*)j->b;
  for (int64_t r = j->r0; r < j->r1; ++r)
    ((float*)j->o0)[r] = (float)pjrtx_oracle_c1_row(x + r * j->cols, y + r * j->cols, j->cols);
  return 0;
}

enum { kMaxThreads = 256 };

static int run_rows(void* (*fn)(void*), Job proto, int64_t rows, int threads) {
  if (threads < 1) threads = 1;
  if (threads > kMaxThreads) threads = kMaxThreads;
  if (threads > rows) threads = (int)(rows > 0 ? rows : 1);
  pthread_t tid[kMaxThreads];
  Job jobs[kMaxThreads];
  for (int t = 0; t < threads; ++t) {
    jobs[t] = proto;
    jobs[t].r0 = rows * t / threads;
    jobs[t].r1 = rows * (t + 1) / threads;
    if (t == 0) continue;
    if (pthread_create(&tid[t], 0, fn, &jobs[t]) != 0) { /* run it here instead */
      fn(&jobs[t]);
      tid[t] = 0;
    }
  }
  fn(&jobs[0]);
  for (int t = 1; t < threads; ++t)
    if (tid[t]) pthread_join(tid[t], 0);
  return threads;
}

/* Returns the number of threads used. */
int pjrtx_oracle_c2(const uint16_t* logits_bf16, int64_t rows, int64_t cols, uint16_t* max_bf16, int32_t* argmax,
                    uint16_t* sum_f16, uint16_t* max_f16, uint16_t* min_f16, int threads) {
  Job p = {logits_bf16, 0, cols, 0, 0, max_bf16, argmax, sum_f16, max_f16, min_f16};
  return run_rows(c2_rows, p, rows, threads);
}

int pjrtx_oracle_c1(const float* x, const float* y, int64_t rows, int64_t cols, float* out, int threads) {
  Job p = {x, y, cols, 0, 0, out, 0, 0, 0, 0};
  return run_rows(c1_rows, p, rows, threads);
}

/* Every bf16 bit pattern converted to f16 (the test's exhaustive pin). */
void pjrtx_oracle_bf16_to_f16_table(uint16_t* out65536) {
  for (uint32_t b = 0; b < 65536u; ++b) out65536[b] = pjrtx_oracle_f32_to_f16(bf16_to_f32((uint16_t)b));
}
