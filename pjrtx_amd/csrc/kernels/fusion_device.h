// Device-side building blocks for the per-fusion-group kernels that the
// planner generates at PJRT compile time (compiled with hiprtc for gfx950).
//
// The generated kernel for a fusion group is this header plus one
// expression body: the hand-written parts here are the memory access
// (16-byte vector loads/stores), the XLA element semantics of every
// StableHLO elementwise op, and the 64-lane wavefront + LDS reductions.
// It replaces the reference's generated MSL helpers
// (reference: src/backend/mlx_metal/executable_metal_graph_map_rules.zig:41-234,
// executable_metal_graph_reduction.zig:57-323).
//
// Element policy: f16/bf16 values are carried in float registers and rounded
// back to their type after every op whose result has that type, which keeps
// the per-op rounding of a bf16/f16 program.
#pragma once

typedef unsigned char uint8_t;
typedef signed char int8_t;
typedef unsigned short uint16_t;
typedef short int16_t;
typedef unsigned int uint32_t;
typedef int int32_t;
typedef unsigned long long uint64_t;
typedef long long int64_t;

#define PJRTX_DEV static __device__ __forceinline__

// ---------------------------------------------------------------- conversions

PJRTX_DEV float bf16_to_f32(uint16_t b) { return __builtin_bit_cast(float, (uint32_t)b << 16); }

PJRTX_DEV uint16_t f32_to_bf16(float f) {
  uint32_t u = __builtin_bit_cast(uint32_t, f);
  if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu)) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

PJRTX_DEV float round_bf16(float f) { return bf16_to_f32(f32_to_bf16(f)); }

PJRTX_DEV float f16_to_f32(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }
PJRTX_DEV uint16_t f32_to_f16(float f) { return __builtin_bit_cast(uint16_t, (_Float16)f); }
PJRTX_DEV float round_f16(float f) { return (float)(_Float16)f; }
// acc + x for an x holding an f16 value: one mixed-precision FMA, x * 1.0 +
// acc with the f16 operand widened exactly and one f32 rounding, which is
// the f32 add's result bit for bit in one instruction instead of two.
PJRTX_DEV float add_f16v(float acc, float x) {
  const _Float16 h = (_Float16)x;
  float r;
  asm("v_fma_mix_f32 %0, %1, 1.0, %2 op_sel_hi:[1,0,0]" : "=v"(r) : "v"(h), "v"(acc));
  return r;
}
// acc + x + y for x, y holding f16 values (or f32 values to be rounded to
// f16): one packed round-to-nearest convert (v_cvt_pk_f16_f32) and one
// v_dot2 with the pair (1, 1), x * 1 + y * 1 + acc accumulated in f32. Two
// instructions per pair instead of four; the pair is added as one step, so
// the sum's rounding differs from two sequential f32 adds (an f32 sum of
// f16 values either way).
PJRTX_DEV float add2_f16v(float acc, float x, float y) {
  typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
  typedef float f2_t __attribute__((ext_vector_type(2)));
  const h2_t h = __builtin_convertvector((f2_t){x, y}, h2_t);
  return __builtin_amdgcn_fdot2(h, (h2_t){(_Float16)1, (_Float16)1}, acc, false);
}

// stablehlo.reduce_precision on the bits of a float with E exponent and Mn
// mantissa bits: the mantissa rounds to m bits (to nearest, ties to even;
// a carry moves into the exponent), then exponents beyond e bits' range go
// to +-inf (overflow) or +-0 (underflow, which includes the source's
// subnormals when e < E). A NaN input stays that NaN when m > 0.
template <typename U, int E, int Mn>
PJRTX_DEV U rp_bits(U u, int e, int m) {
  constexpr int W = 1 + E + Mn;
  const U sign = (U)((U)1 << (W - 1));
  const U expm = (U)((((U)1 << E) - 1) << Mn);
  const U manm = (U)(((U)1 << Mn) - 1);
  const bool nan = (U)(u & expm) == expm && (U)(u & manm) != 0;
  const U x = u;
  if (m < Mn) {
    const int sh = Mn - m;
    const U last = (U)((U)1 << sh);
    const U bias = (U)((last >> 1) - 1 + ((u & last) >> sh));
    u = (U)((U)(u + bias) & (U)~(U)(last - 1));
  }
  if (e < E) {
    const U b = (U)(((U)1 << (E - 1)) - 1);
    const U rb = (U)(((U)1 << (e - 1)) - 1);
    const U xe = (U)(u & expm);
    const bool over = xe > (U)((U)(b + rb) << Mn);
    const bool under = xe <= (U)((U)(b - rb) << Mn);
    const U sz = (U)(u & sign);
    u = over ? (U)(sz | expm) : (under ? sz : u);
  }
  return (m > 0 && nan) ? x : u;
}
PJRTX_DEV float rp_f32(float x, int e, int m) {
  return __builtin_bit_cast(float, rp_bits<uint32_t, 8, 23>(__builtin_bit_cast(uint32_t, x), e, m));
}
PJRTX_DEV double rp_f64(double x, int e, int m) {
  return __builtin_bit_cast(double, rp_bits<uint64_t, 11, 52>(__builtin_bit_cast(uint64_t, x), e, m));
}
// 16-bit types arrive as the float of their value (exact).
PJRTX_DEV float rp_bf16(float x, int e, int m) {
  return bf16_to_f32(rp_bits<uint16_t, 8, 7>((uint16_t)(__builtin_bit_cast(uint32_t, x) >> 16), e, m));
}
PJRTX_DEV float rp_f16(float x, int e, int m) { return f16_to_f32(rp_bits<uint16_t, 5, 10>(f32_to_f16(x), e, m)); }

// Storage <-> compute for each element kind.
PJRTX_DEV float ld_f32(const float* p, uint32_t i) { return p[i]; }
PJRTX_DEV float ld_bf16(const uint16_t* p, uint32_t i) { return bf16_to_f32(p[i]); }
PJRTX_DEV float ld_f16(const uint16_t* p, uint32_t i) { return f16_to_f32(p[i]); }

// ------------------------------------------------------------ vector accesses
// Loads N consecutive storage elements starting at `base` (multiple of N).
// `full` is false only for the last partial vector of a tensor, which is read
// element by element up to `n`.

template <typename S, int N>
struct VecBytes {
  static constexpr int kBytes = (int)sizeof(S) * N;
};

// 16-byte loads; NT selects the non-temporal (`nt`) form, the hint for data
// read once: on gfx950 such loads stream faster and do not displace what the
// memory-side cache (MALL) holds for other buffers.
typedef uint32_t pjrtx_v4 __attribute__((ext_vector_type(4)));
template <bool NT = false>
PJRTX_DEV pjrtx_v4 ld16(const void* p) {
  if constexpr (NT) return __builtin_nontemporal_load(reinterpret_cast<const pjrtx_v4*>(p));
  else return *reinterpret_cast<const pjrtx_v4*>(p);
}

template <typename S, int N, bool NT = false>
PJRTX_DEV void ldv(S (&dst)[N], const S* __restrict__ src, uint32_t base, uint32_t n, bool full) {
  if (full) {
    constexpr int kBytes = (int)sizeof(S) * N;
    if constexpr (kBytes % 16 == 0) {
      typedef uint32_t v4 __attribute__((ext_vector_type(4)));
#pragma unroll
      for (int c = 0; c < kBytes / 16; ++c) {
        v4 v = ld16<NT>(reinterpret_cast<const char*>(src + base) + 16 * c);
        *reinterpret_cast<v4*>(reinterpret_cast<char*>(dst) + 16 * c) = v;
      }
    } else if constexpr (kBytes == 8) {
      typedef uint32_t v2 __attribute__((ext_vector_type(2)));
      *reinterpret_cast<v2*>(dst) = *reinterpret_cast<const v2*>(src + base);
    } else if constexpr (kBytes == 4) {
      *reinterpret_cast<uint32_t*>(dst) = *reinterpret_cast<const uint32_t*>(src + base);
    } else {
#pragma unroll
      for (int j = 0; j < N; ++j) dst[j] = src[base + j];
    }
  } else {
#pragma unroll
    for (int j = 0; j < N; ++j) dst[j] = (base + j < n) ? src[base + j] : src[n - 1];
  }
}

// Keeps the registers of a load live to this point (an empty asm reading
// them), so that a load whose other uses sit inside a branch is still issued
// with the loads before it instead of being moved into that branch.
template <typename S, int N>
PJRTX_DEV void keep_live(const S (&a)[N]) {
  if constexpr (sizeof(a) % 4 == 0) {
#pragma unroll
    for (int i = 0; i < (int)(sizeof(a) / 4); ++i) {
      uint32_t w;
      __builtin_memcpy(&w, reinterpret_cast<const char*>(a) + 4 * i, 4);
      asm volatile("" ::"v"(w));
    }
  } else {
#pragma unroll
    for (int i = 0; i < N; ++i) {
      uint32_t w = 0;
      __builtin_memcpy(&w, &a[i], sizeof(S) < 4 ? sizeof(S) : 4);
      asm volatile("" ::"v"(w));
    }
  }
}

template <typename S, int N>
PJRTX_DEV void stv(S* __restrict__ dst, uint32_t base, const S (&src)[N], uint32_t n, bool full) {
  if (full) {
    constexpr int kBytes = (int)sizeof(S) * N;
    if constexpr (kBytes % 16 == 0) {
      typedef uint32_t v4 __attribute__((ext_vector_type(4)));
#pragma unroll
      for (int c = 0; c < kBytes / 16; ++c) {
        *reinterpret_cast<v4*>(reinterpret_cast<char*>(dst + base) + 16 * c) =
            *reinterpret_cast<const v4*>(reinterpret_cast<const char*>(src) + 16 * c);
      }
    } else if constexpr (kBytes == 8) {
      typedef uint32_t v2 __attribute__((ext_vector_type(2)));
      *reinterpret_cast<v2*>(dst + base) = *reinterpret_cast<const v2*>(src);
    } else if constexpr (kBytes == 4) {
      *reinterpret_cast<uint32_t*>(dst + base) = *reinterpret_cast<const uint32_t*>(src);
    } else {
#pragma unroll
      for (int j = 0; j < N; ++j) dst[base + j] = src[j];
    }
  } else {
#pragma unroll
    for (int j = 0; j < N; ++j)
      if (base + j < n) dst[base + j] = src[j];
  }
}

// -------------------------------------------------- XLA elementwise semantics

PJRTX_DEV bool isnan_f(float x) { return x != x; }
PJRTX_DEV bool isnan_d(double x) { return x != x; }

// maximum/minimum propagate NaN (XLA semantics), unlike fmaxf/fminf.
PJRTX_DEV float max_f(float a, float b) { return (isnan_f(a) || a >= b) ? a : b; }
PJRTX_DEV float min_f(float a, float b) { return (isnan_f(a) || a <= b) ? a : b; }
PJRTX_DEV double max_d(double a, double b) { return (isnan_d(a) || a >= b) ? a : b; }
PJRTX_DEV double min_d(double a, double b) { return (isnan_d(a) || a <= b) ? a : b; }
template <typename T> PJRTX_DEV T max_i(T a, T b) { return a > b ? a : b; }
template <typename T> PJRTX_DEV T min_i(T a, T b) { return a < b ? a : b; }

PJRTX_DEV float sign_f(float x) { return isnan_f(x) ? x : (x > 0.f ? 1.f : (x < 0.f ? -1.f : x)); }
PJRTX_DEV double sign_d(double x) { return isnan_d(x) ? x : (x > 0.0 ? 1.0 : (x < 0.0 ? -1.0 : x)); }
template <typename T> PJRTX_DEV T sign_i(T x) { return (T)((x > 0) - (x < 0)); }

PJRTX_DEV float logistic_f(float x) { return 1.0f / (1.0f + __expf(-x)); }
PJRTX_DEV float rsqrt_f(float x) { return 1.0f / sqrtf(x); }
PJRTX_DEV float is_finite_f(float x) { return __builtin_isfinite(x); }

// Integer division / remainder with XLA's defined results for x/0 and
// INT_MIN/-1 (x/0 = -1, x%0 = x, INT_MIN/-1 = INT_MIN, INT_MIN%-1 = 0).
template <typename T> PJRTX_DEV T div_s(T a, T b) {
  if (b == 0) return (T)-1;
  if (b == (T)-1 && a == (T)((T)1 << (sizeof(T) * 8 - 1))) return a;
  return a / b;
}
template <typename T> PJRTX_DEV T rem_s(T a, T b) {
  if (b == 0) return a;
  if (b == (T)-1) return 0;
  return a % b;
}
template <typename T> PJRTX_DEV T div_u(T a, T b) { return b == 0 ? (T)~(T)0 : a / b; }
template <typename T> PJRTX_DEV T rem_u(T a, T b) { return b == 0 ? a : a % b; }

// Shifts: amounts >= bit width give 0 (left/logical) or the sign fill.
template <typename T, typename U> PJRTX_DEV T shl(T a, T b) {
  return ((U)b >= sizeof(T) * 8) ? (T)0 : (T)((U)a << (U)b);
}
template <typename T, typename U> PJRTX_DEV T shr_logical(T a, T b) {
  return ((U)b >= sizeof(T) * 8) ? (T)0 : (T)((U)a >> (U)b);
}
template <typename T, typename U> PJRTX_DEV T shr_arith(T a, T b) {
  const U bits = sizeof(T) * 8;
  return ((U)b >= bits) ? (T)(a < 0 ? -1 : 0) : (T)(a >> b);
}

template <typename T> PJRTX_DEV T ipow(T base, T exp) {
  if (exp < 0) return (base == 1) ? (T)1 : (base == (T)-1 ? ((exp & 1) ? (T)-1 : (T)1) : (T)0);
  T r = 1;
  while (exp) {
    if (exp & 1) r *= base;
    base *= base;
    exp >>= 1;
  }
  return r;
}

// float -> integer converts saturate and map NaN to 0 (XLA semantics).
template <typename T> PJRTX_DEV T f2i(float x, float lo, float hi) {
  if (isnan_f(x)) return (T)0;
  if (x <= lo) return (T)lo;
  if (x >= hi) return (T)hi;
  return (T)x;
}
PJRTX_DEV int32_t f2i32(float x) {
  if (isnan_f(x)) return 0;
  if (x <= -2147483648.0f) return (-2147483647 - 1);
  if (x >= 2147483648.0f) return 2147483647;
  return (int32_t)x;
}
PJRTX_DEV uint32_t f2u32(float x) {
  if (isnan_f(x) || x <= 0.0f) return 0u;
  if (x >= 4294967296.0f) return 4294967295u;
  return (uint32_t)x;
}
PJRTX_DEV int64_t f2i64(float x) {
  if (isnan_f(x)) return 0;
  if (x <= -9223372036854775808.0f) return (-9223372036854775807LL - 1);
  if (x >= 9223372036854775808.0f) return 9223372036854775807LL;
  return (int64_t)x;
}

// Float total order key (for TOTALORDER comparisons).
// Negative floats get their magnitude bits flipped so that signed integer
// order equals -NaN < -inf < ... < -0 < +0 < ... < +inf < +NaN.
PJRTX_DEV int32_t total_order_key(float x) {
  int32_t i = __builtin_bit_cast(int32_t, x);
  return i < 0 ? (i ^ 0x7fffffff) : i;
}

// ------------------------------------------------------------ argmax order
// (value, index) pairs ordered so that NaN wins over any number, larger
// values win, and ties go to the lower index. This is the order JAX's argmax
// comparator defines; it is total on distinct indices, so any combine tree
// gives the same winner.
template <typename I>
PJRTX_DEV bool argmax_better(float va, I ia, float vb, I ib) {
  const bool na = isnan_f(va), nb = isnan_f(vb);
  if (na != nb) return na;
  if (!na && va != vb) return va > vb;
  return ia < ib;
}
template <typename I>
PJRTX_DEV bool argmin_better(float va, I ia, float vb, I ib) {
  const bool na = isnan_f(va), nb = isnan_f(vb);
  if (na != nb) return na;
  if (!na && va != vb) return va < vb;
  return ia < ib;
}

// In-order forms used while one thread walks its elements by increasing
// index: the newcomer x (higher index) replaces the accumulator only if it
// is strictly better, or is the first NaN. Same winner as argmax_better for
// that order, at a fraction of the instructions.
PJRTX_DEV bool argmax_take(float x, float acc) { return x > acc || (isnan_f(x) && !isnan_f(acc)); }
PJRTX_DEV bool argmin_take(float x, float acc) { return x < acc || (isnan_f(x) && !isnan_f(acc)); }
// NaN-propagating running max/min (an accumulator that saw NaN stays NaN).
// Reduction max/min: IEEE 754-2019 maximum/minimum (NaN propagates, -0 <
// +0), so the result does not depend on the order partials are combined in.
// gfx950 folds two new values per v_maximum3_f32 / v_minimum3_f32.
PJRTX_DEV float max_r(float a, float b) { return __builtin_elementwise_maximum(a, b); }
PJRTX_DEV float min_r(float a, float b) { return __builtin_elementwise_minimum(a, b); }
PJRTX_DEV float max_seq(float acc, float x) { return max_r(acc, x); }
PJRTX_DEV float min_seq(float acc, float x) { return min_r(acc, x); }

// ------------------------------------------------------------ decode GEMV
typedef uint32_t gv_u32x4 __attribute__((ext_vector_type(4)));
// Decode weights are read once per token, more of them than the MALL holds:
// non-temporal loads by default (the C5 decode step: 2370 -> 2580 tokens/s).
template <bool NT = true>
PJRTX_DEV gv_u32x4 gv_load16(const uint16_t* p) { return ld16<NT>(p); }
// acc[e] += x * w[e] for the eight 16-bit weights of one 16-byte piece, in
// element order (bf16: the high half of each 32-bit word is the odd element).
template <bool kF16>
PJRTX_DEV void gv_fma8(float* acc, float x, const gv_u32x4& w) {
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const uint32_t u = w[q];
    float lo, hi;
    if constexpr (kF16) {
      lo = f16_to_f32((uint16_t)(u & 0xffffu));
      hi = f16_to_f32((uint16_t)(u >> 16));
    } else {
      lo = __builtin_bit_cast(float, u << 16);
      hi = __builtin_bit_cast(float, u & 0xffff0000u);
    }
    acc[2 * q] = __builtin_fmaf(x, lo, acc[2 * q]);
    acc[2 * q + 1] = __builtin_fmaf(x, hi, acc[2 * q + 1]);
  }
}
// X element k of a decode GEMV whose input is a split decode attention's
// partials (floats [head][split][m, l, D unnormalized values]; l = -1 marks
// a split past the row's last allowed key): gv_attn_load requests the
// element's m, l and value of every split (so a kernel can issue its weight
// loads before waiting for them); gv_attn_fold merges the splits in split
// order with the attention kernel's own merge arithmetic (max of m; weights
// exp(m - max); sums of l and of the values times the weights; one
// division) and rounds to the 16-bit input type.
template <int NS, int D>
PJRTX_DEV void gv_attn_load(const float* __restrict__ part, uint32_t k, float (&ms)[NS], float (&ls)[NS],
                            float (&vs)[NS]) {
  const float* pr = part + (size_t)(k / D) * NS * (D + 2);
  const uint32_t d = k % D;
#pragma unroll
  for (int u = 0; u < NS; ++u) {
    ms[u] = pr[u * (D + 2)];
    ls[u] = pr[u * (D + 2) + 1];
    vs[u] = pr[u * (D + 2) + 2 + d];
  }
}
template <int NS, bool kF16>
PJRTX_DEV float gv_attn_fold(const float (&ms)[NS], const float (&ls)[NS], const float (&vs)[NS]) {
  float mall = -__builtin_inff();
#pragma unroll
  for (int u = 0; u < NS; ++u)
    if (ls[u] != -1.f) mall = fmaxf(mall, ms[u]);
  const float mref = mall == -__builtin_inff() ? 0.f : mall;
  float lsum = 0.f, acc = 0.f;
#pragma unroll
  for (int u = 0; u < NS; ++u) {
    if (ls[u] != -1.f) {
      const float f = expf(ms[u] - mref);
      lsum += ls[u] * f;
      acc += vs[u] * f;
    }
  }
  return kF16 ? round_f16(acc / lsum) : round_bf16(acc / lsum);
}
template <int NS, int D, bool kF16>
PJRTX_DEV float gv_attn_merge(const float* __restrict__ part, uint32_t k) {
  float ms[NS], ls[NS], vs[NS];
  gv_attn_load<NS, D>(part, k, ms, ls, vs);
  return gv_attn_fold<NS, kF16>(ms, ls, vs);
}

// ------------------------------------------------------ wavefront reductions
// 64-lane wavefronts: xor-butterfly over lane offsets 32..1. Every lane ends
// with the same value, combined in a fixed order (deterministic).

template <typename T>
PJRTX_DEV T wave_shfl_xor(T v, int mask) {
  if constexpr (sizeof(T) == 8) {
    uint64_t u = __builtin_bit_cast(uint64_t, v);
    uint32_t lo = (uint32_t)u, hi = (uint32_t)(u >> 32);
    lo = (uint32_t)__shfl_xor((int)lo, mask, 64);
    hi = (uint32_t)__shfl_xor((int)hi, mask, 64);
    return __builtin_bit_cast(T, ((uint64_t)hi << 32) | lo);
  } else if constexpr (sizeof(T) == 4) {
    return __builtin_bit_cast(T, __shfl_xor(__builtin_bit_cast(int, v), mask, 64));
  } else {
    return (T)__shfl_xor((int)v, mask, 64);
  }
}

// DPP lane exchanges within rows of 16 lanes (no LDS round trip): xor 1
// and xor 2 as quad permutations, then the half-row and row mirrors, which
// pair each lane with the other half of its 8- (16-) lane group; once the
// earlier steps made those halves uniform that is the xor 4 (xor 8) partner.
// After the four steps every row of 16 lanes holds one value; lane_value
// reads a row's value from a lane (0, 16, 32, 48) into a uniform register.
constexpr int kDppXor1 = 0xB1, kDppXor2 = 0x4E, kDppHalfMirror = 0x141, kDppMirror = 0x140;

template <int kCtrl, typename T>
PJRTX_DEV T dpp_move(T v) {
  if constexpr (sizeof(T) == 8) {
    const uint64_t u = __builtin_bit_cast(uint64_t, v);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)u, kCtrl, 0xf, 0xf, false);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)(u >> 32), kCtrl, 0xf, 0xf, false);
    return __builtin_bit_cast(T, ((uint64_t)hi << 32) | lo);
  } else if constexpr (sizeof(T) == 4) {
    return __builtin_bit_cast(T, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), kCtrl, 0xf, 0xf, false));
  } else {
    return (T)__builtin_amdgcn_update_dpp(0, (int)v, kCtrl, 0xf, 0xf, false);
  }
}

template <typename T>
PJRTX_DEV T lane_value(T v, int lane) {
  if constexpr (sizeof(T) == 8) {
    const uint64_t u = __builtin_bit_cast(uint64_t, v);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)u, lane);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(u >> 32), lane);
    return __builtin_bit_cast(T, ((uint64_t)hi << 32) | lo);
  } else if constexpr (sizeof(T) == 4) {
    return __builtin_bit_cast(T, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
  } else {
    return (T)__builtin_amdgcn_readlane((int)v, lane);
  }
}

// `v` of the lowest lane whose `mine` is true, in every lane (some lane's
// `mine` must be true).
PJRTX_DEV float wave_value_at(float v, bool mine) {
  const unsigned long long own = __ballot(mine);
  return __shfl(v, __ffsll(own) - 1, 64);
}
