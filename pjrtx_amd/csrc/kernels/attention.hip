// Fused attention for gfx950: softmax(scale * Q.K^T, masked) . V in one
// kernel, the score matrix never leaving the chip.
//
//  * attn_tiles (bf16 / f16, head dim 64 or 128): a workgroup owns 128
//    queries of one (batch, head), 32 per wave, and walks the allowed keys in
//    blocks of 64 staged through LDS (K row-major, V transposed). Each wave
//    computes S^T = K.Q^T on v_mfma_f32_16x16x32 so that a lane holds 16
//    scores of ONE query: the row max and sum are a 16-value in-lane fold
//    plus two xor shuffles. The exponentials, rounded to the input type, are
//    the B operand of O^T += V^T.P^T directly from registers (the V^T tile
//    stores keys in the order a lane holds them), and the running output is
//    rescaled per lane by its own query's factor. Q stays in registers for
//    the whole walk. Workgroups take the heaviest (latest) query tiles first;
//    when B*H is a multiple of 8, one head's query tiles run on one XCD so
//    its K and V are served from that XCD's L2.
//  * attn_pipe (head dim 128, the default for it): the same work split with
//    K and V loaded straight into LDS, V^T fragments from transposing LDS
//    reads and a leaner softmax (see its comment below).
//  * attn_rows (any element type, head dim <= 512): one workgroup per query
//    row, its 4 waves splitting the keys in blocks of 64 (one key per lane
//    for the scores, then lanes across the head dim for P.V), combined at the
//    end in wave order. Decode (one query) and f32 take this kernel.
//
// Both use the online-softmax recurrence (running max m, sum l, output
// rescaled by exp(m_old - m_new)); a row with no allowed key yields 0/0 =
// NaN as the unfused softmax does.
//
// Replaces the reference's scaled-dot-product-attention custom call
// (reference: src/backend/mlx_metal/api.cc:4928-5062, which calls
// mlx::core::fast::scaled_dot_product_attention with the boolean mask of
// api.cc:937-950) and, through the planner's rewrite, its unfused
// dot_general / softmax / dot_general path (api.cc:3349-3498, 3982-4044).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <type_traits>

#include "common.h"
#include "kernels/attention.h"

namespace pjrtx {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint16_t f32_to_bf16_rne(float f) {
  uint32_t u = __builtin_bit_cast(uint32_t, f);
  if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu)) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}
__device__ __forceinline__ float bf16_to_f32(uint16_t b) { return __builtin_bit_cast(float, (uint32_t)b << 16); }
__device__ __forceinline__ uint16_t f32_to_f16(float f) { return __builtin_bit_cast(uint16_t, (_Float16)f); }
__device__ __forceinline__ float f16_to_f32(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }

template <bool kF16>
__device__ __forceinline__ uint16_t from_f32(float x) {
  if constexpr (kF16) return f32_to_f16(x);
  else return f32_to_bf16_rne(x);
}
template <bool kF16>
__device__ __forceinline__ float to_f32(uint16_t x) {
  if constexpr (kF16) return f16_to_f32(x);
  else return bf16_to_f32(x);
}

typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

// Two floats rounded (to nearest even) and packed as 16-bit values, low
// half first: one v_cvt_pk_* on gfx950.
template <bool kF16>
__device__ __forceinline__ uint32_t pack2(float a, float b) {
  if constexpr (kF16) return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{a, b}, f16x2));
  else return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{a, b}, bf16x2));
}
template <bool kF16>
__device__ __forceinline__ float round16(float x) {
  if constexpr (kF16) return (float)(_Float16)x;
  else return (float)(__bf16)x;
}

template <bool kF16>
__device__ __forceinline__ f32x4 mfma16(const u32x4& a, const u32x4& b, const f32x4& c) {
  if constexpr (kF16)
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0, 0,
                                                   0);
}

__device__ __forceinline__ int64_t read_offset(const AttnParams& p) {
  int64_t off = 0;
  if (p.offset_ptr) {
    switch (p.offset_bytes) {
      case 8: off += *static_cast<const int64_t*>(p.offset_ptr); break;
      case 4:
        off += p.offset_signed ? (int64_t)*static_cast<const int32_t*>(p.offset_ptr)
                               : (int64_t)*static_cast<const uint32_t*>(p.offset_ptr);
        break;
      case 2:
        off += p.offset_signed ? (int64_t)*static_cast<const int16_t*>(p.offset_ptr)
                               : (int64_t)*static_cast<const uint16_t*>(p.offset_ptr);
        break;
      default:
        off += p.offset_signed ? (int64_t)*static_cast<const int8_t*>(p.offset_ptr)
                               : (int64_t)*static_cast<const uint8_t*>(p.offset_ptr);
        break;
    }
    if (p.offset_as_s32) off = (int64_t)(int32_t)(uint32_t)(uint64_t)off;
  }
  return off + p.offset;
}

// Last allowed key of query q, clamped to [-1, Skv - 1].
__device__ __forceinline__ int key_limit(const AttnParams& p, int64_t off, int64_t q) {
  const int64_t lim = p.causal ? (int64_t)p.q_coef * q + off : (int64_t)p.Skv - 1;
  return (int)std::max<int64_t>(-1, std::min<int64_t>(lim, (int64_t)p.Skv - 1));
}

// ---------------------------------------------------------------- tiles

constexpr int FQ = 128;  // queries per workgroup (32 per wave)
constexpr int FK = 64;   // keys per block

// K tile [FK][D]: 16-byte chunk `ch` of key row `row`, XOR-swizzled so the
// 16 rows a fragment read touches fall in distinct banks.
template <int D>
__device__ __forceinline__ int kswz(int row, int ch) {
  if constexpr (D == 128) return row * 128 + ((ch ^ (row & 15)) << 3);
  else return row * 64 + ((ch ^ ((row >> 1) & 7)) << 3);
}
// V^T tile [D][FK] (64 key positions per head-dim row), same swizzle idea.
__device__ __forceinline__ int vswz(int row, int ch) { return row * 64 + ((ch ^ ((row >> 1) & 7)) << 3); }
// Position of block key j in a V^T row. Lane group g of a wave holds, for a
// 32-key step, keys 4g..4g+3 and 16+4g..16+4g+3 of its S^T tiles; placing
// them at positions 8g..8g+7 makes the lane's P values a contiguous B
// fragment.
__device__ __forceinline__ int vpos(int key) {
  return (key & 32) | (((key & 15) >> 2) << 3) | (((key >> 4) & 1) << 2) | (key & 3);
}

template <bool kF16, int D, bool kRound>
__global__ void __launch_bounds__(256, 2) attn_tiles(AttnParams p, const uint16_t* __restrict__ Q,
                                                     const uint16_t* __restrict__ K, const uint16_t* __restrict__ V,
                                                     uint16_t* __restrict__ O) {
  constexpr int NCH = D / 8;   // 16-byte chunks per row
  constexpr int NDS = D / 32;  // MFMA k-steps over the head dim
  constexpr int NDT = D / 16;  // 16-wide output tiles over the head dim
  constexpr int KPT = D / 32;  // K chunks per thread; V keys per thread
  __shared__ __attribute__((aligned(16))) uint16_t Ks[FK * D];
  __shared__ __attribute__((aligned(16))) uint16_t Vt[D * FK];

  const int nq = (p.Sq + FQ - 1) / FQ;
  const int BH = p.B * p.Hq;
  const int bid = blockIdx.x;
  int bh, qtile;
  if (BH % 8 == 0) {
    const int x = bid & 7, n = bid >> 3;
    bh = (n / nq) * 8 + x;
    qtile = nq - 1 - n % nq;
  } else {
    bh = bid % BH;
    qtile = nq - 1 - bid / BH;
  }
  const int b = bh / p.Hq, h = bh - b * p.Hq;
  const int hk = h / (p.Hq / p.Hkv);
  const int q0 = qtile * FQ;
  const uint16_t* Qp = Q + (int64_t)b * p.q_b + (int64_t)h * p.q_h;
  const uint16_t* Kp = K + (int64_t)b * p.k_b + (int64_t)hk * p.k_h;
  const uint16_t* Vp = V + (int64_t)b * p.v_b + (int64_t)hk * p.v_h;
  uint16_t* Op = O + (int64_t)b * p.o_b + (int64_t)h * p.o_h;

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int g = lane >> 4, c16 = lane & 15;
  const u32x4 zero = {0u, 0u, 0u, 0u};

  // Q fragments: the B operand of S^T = K.Q^T (lane: query c16 of the
  // 16-query tile, head dims 32*ds + 8*g .. +8).
  u32x4 qf[2][NDS];
  int lim[2];
  const int64_t off = read_offset(p);
#pragma unroll
  for (int qt = 0; qt < 2; ++qt) {
    const int q = q0 + wave * 32 + qt * 16 + c16;
#pragma unroll
    for (int ds = 0; ds < NDS; ++ds)
      qf[qt][ds] = q < p.Sq ? *reinterpret_cast<const u32x4*>(Qp + (int64_t)q * p.q_s + ds * 32 + g * 8) : zero;
    lim[qt] = key_limit(p, off, q);
  }
  // Keys the workgroup needs, and the prefix that needs no mask.
  const int kend = key_limit(p, off, std::min(q0 + FQ, p.Sq) - 1) + 1;
  const int free_end = key_limit(p, off, q0) + 1;  // q_coef >= 0: the first query has the lowest limit
  const int nblocks = (kend + FK - 1) / FK;

  const float c2 = p.scale * 1.44269504088896340736f;  // scale * log2(e)
  float m[2] = {-INFINITY, -INFINITY}, l[2] = {0.f, 0.f};
  f32x4 oacc[NDT][2];
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt) oacc[dt][0] = oacc[dt][1] = f32x4{0.f, 0.f, 0.f, 0.f};

  u32x4 kreg[KPT], vreg[KPT];
  const int vdc = tid % NCH, vkg = tid / NCH;  // V: head-dim chunk, key group of KPT keys
  auto gload = [&](int kb) {
#pragma unroll
    for (int j = 0; j < KPT; ++j) {
      const int c = tid + 256 * j;
      const int key = kb * FK + c / NCH;
      kreg[j] = key < p.Skv ? *reinterpret_cast<const u32x4*>(Kp + (int64_t)key * p.k_s + (c % NCH) * 8) : zero;
    }
#pragma unroll
    for (int r = 0; r < KPT; ++r) {
      const int key = kb * FK + vkg * KPT + r;
      vreg[r] = key < p.Skv ? *reinterpret_cast<const u32x4*>(Vp + (int64_t)key * p.v_s + vdc * 8) : zero;
    }
  };
  auto lstore = [&]() {
#pragma unroll
    for (int j = 0; j < KPT; ++j) {
      const int c = tid + 256 * j;
      *reinterpret_cast<u32x4*>(&Ks[kswz<D>(c / NCH, c % NCH)]) = kreg[j];
    }
    const int pos = vpos(vkg * KPT);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      uint32_t e[KPT];
#pragma unroll
      for (int r = 0; r < KPT; ++r) e[r] = (vreg[r][i >> 1] >> (16 * (i & 1))) & 0xffffu;
      const int at = vswz(vdc * 8 + i, pos >> 3) + (pos & 7);
      if constexpr (KPT == 4) {
        *reinterpret_cast<u32x2*>(&Vt[at]) = u32x2{e[0] | (e[1] << 16), e[2] | (e[3] << 16)};
      } else {
        *reinterpret_cast<uint32_t*>(&Vt[at]) = e[0] | (e[1] << 16);
      }
    }
  };

  if (nblocks > 0) {
    gload(0);
    lstore();
  }
  __syncthreads();
  for (int kb = 0; kb < nblocks; ++kb) {
    if (kb + 1 < nblocks) gload(kb + 1);
    // S^T[key][query] for the wave's 32 queries and the block's 64 keys.
    f32x4 sacc[4][2];
#pragma unroll
    for (int kt = 0; kt < 4; ++kt) sacc[kt][0] = sacc[kt][1] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ds = 0; ds < NDS; ++ds) {
#pragma unroll
      for (int kt = 0; kt < 4; ++kt) {
        const u32x4 a = *reinterpret_cast<const u32x4*>(&Ks[kswz<D>(kt * 16 + c16, ds * 4 + g)]);
        sacc[kt][0] = mfma16<kF16>(a, qf[0][ds], sacc[kt][0]);
        sacc[kt][1] = mfma16<kF16>(a, qf[1][ds], sacc[kt][1]);
      }
    }
    const bool need_mask = kb * FK + FK > free_end;
    u32x4 pf[2][2];
#pragma unroll
    for (int qt = 0; qt < 2; ++qt) {
      // Max on the unscaled scores (scale > 0), exponentials as
      // exp2(s * scale * log2(e) - m * scale * log2(e)): one FMA and one
      // v_exp_f32 per score.
      float s[4][4];
      float mx = -INFINITY;
#pragma unroll
      for (int kt = 0; kt < 4; ++kt)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          float x = sacc[kt][qt][r];
          if constexpr (kRound) x = round16<kF16>(x);
          if (need_mask && kb * FK + kt * 16 + g * 4 + r > lim[qt]) x = -INFINITY;
          s[kt][r] = x;
          mx = fmaxf(mx, x);
        }
      mx = fmaxf(mx, __shfl_xor(mx, 16));
      mx = fmaxf(mx, __shfl_xor(mx, 32));
      const float mnew = fmaxf(m[qt], mx);
      const float mc = (mnew == -INFINITY ? 0.f : mnew) * c2;
      const float alpha = __builtin_amdgcn_exp2f(m[qt] * c2 - mc);  // 0 while m is -inf, 1 when m is unchanged
      float ps = 0.f;
#pragma unroll
      for (int kt = 0; kt < 4; ++kt)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          s[kt][r] = __builtin_amdgcn_exp2f(fmaf(s[kt][r], c2, -mc));
          ps += s[kt][r];
        }
      ps += __shfl_xor(ps, 16);
      ps += __shfl_xor(ps, 32);
      l[qt] = l[qt] * alpha + ps;
      m[qt] = mnew;
      if (!__all(alpha == 1.f)) {
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt) oacc[dt][qt] *= alpha;
      }
#pragma unroll
      for (int st = 0; st < 2; ++st)
        pf[qt][st] = u32x4{pack2<kF16>(s[2 * st][0], s[2 * st][1]), pack2<kF16>(s[2 * st][2], s[2 * st][3]),
                           pack2<kF16>(s[2 * st + 1][0], s[2 * st + 1][1]),
                           pack2<kF16>(s[2 * st + 1][2], s[2 * st + 1][3])};
    }
    // O^T[d][query] += V^T[d][key] . P^T[key][query]
#pragma unroll
    for (int st = 0; st < 2; ++st) {
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt) {
        const u32x4 a = *reinterpret_cast<const u32x4*>(&Vt[vswz(dt * 16 + c16, st * 4 + g)]);
        oacc[dt][0] = mfma16<kF16>(a, pf[0][st], oacc[dt][0]);
        oacc[dt][1] = mfma16<kF16>(a, pf[1][st], oacc[dt][1]);
      }
    }
    __syncthreads();
    if (kb + 1 < nblocks) lstore();
    __syncthreads();
  }

  // Lane: query c16 of tile qt, head dims 16*dt + 4*g .. +4.
#pragma unroll
  for (int qt = 0; qt < 2; ++qt) {
    const int q = q0 + wave * 32 + qt * 16 + c16;
    if (q >= p.Sq) continue;
    uint16_t* orow = Op + (int64_t)q * p.o_s;
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) {
      const f32x4 o = oacc[dt][qt];
      *reinterpret_cast<u32x2*>(orow + dt * 16 + g * 4) =
          u32x2{pack2<kF16>(o[0] / l[qt], o[1] / l[qt]), pack2<kF16>(o[2] / l[qt], o[3] / l[qt])};
    }
  }
}

// ------------------------------------------------------ DMA tiles
// attn_pipe (head dim 128): the tile kernel's work split (128 queries per
// workgroup, 32 per wave, 64-key blocks, S^T = K.Q^T so a lane holds 16
// scores of one query) with the memory and the VALU work laid out for
// gfx950:
//  * K and V blocks go from global memory straight into LDS (buffer loads
//    with the LDS destination, 16 bytes a lane), two LDS stages each, one
//    barrier per block; no register staging.
//  * V stays row-major in LDS; the V^T fragments of O^T += V^T.P^T come from
//    transposing LDS reads (ds_read_b64_tr_b16: lane j of a 16-lane group
//    gets element j & 3 of the rows that lanes 4e + (j >> 2) address, e =
//    0..3), so one read gives 4 consecutive keys of one head-dim column.
//  * Softmax VALU kept small: NaN-propagating max3 (no operand
//    canonicalization), the max taken on the unrounded scores (rounding is
//    monotone), one packed convert per two scores for the rounding, the row
//    sums from the P.V MFMAs (a row of ones beside V^T), and the running max
//    raised only when it grows by more than 2^8 in the exponential, so most
//    blocks skip the output rescale.
// LDS: K stage [64 keys][128] with 16-byte chunk c of row r at c ^ (r & 15)
// (the 16 rows of a fragment read fall in distinct banks); V stage [64][128]
// with chunk c of row r at c ^ 2 (r & 7) (the 8 rows a half-wave of
// transposing reads touches fall in distinct banks). The buffer loads place
// lane L's 16 bytes at slot L of the wave's 1 KB, so the swizzle is applied
// on the global side: the lane filling slot (r, s) fetches chunk s ^ f(r).
typedef __attribute__((address_space(3))) void* attn_lds_ptr;
typedef short attn_v4i16 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) attn_v4i16 attn_lds_v4i16;

constexpr int PK = 64;          // keys per block
constexpr int PSTAGE = PK * 128;  // elements per K or V stage

__device__ __forceinline__ int pk_swz(int row, int ch) { return row * 128 + ((ch ^ (row & 15)) << 3); }
__device__ __forceinline__ int pv_swz(int row, int ch) { return row * 128 + ((ch ^ ((row & 7) << 1)) << 3); }
constexpr int attn_vmcnt0() { return (7 << 4) | (15 << 8); }  // s_waitcnt vmcnt(0) alone

template <bool kF16, bool kRound>
__global__ void __launch_bounds__(256, 2) attn_pipe(AttnParams p, const uint16_t* __restrict__ Q,
                                                    const uint16_t* __restrict__ K, const uint16_t* __restrict__ V,
                                                    uint16_t* __restrict__ O, int order, int pair, int prio) {
  constexpr int D = 128, NDS = 4, NDT = 8;
  __shared__ __attribute__((aligned(16))) uint16_t Ks[2 * PSTAGE];
  __shared__ __attribute__((aligned(16))) uint16_t Vs[2 * PSTAGE];

  const int nq = (p.Sq + FQ - 1) / FQ;
  // pair: a workgroup takes query tiles nq-1-j and j (the heaviest with the
  // lightest), so every workgroup has the same number of key blocks.
  const int nslots = pair ? (nq + 1) / 2 : nq;
  const int BH = p.B * p.Hq;
  const int bid = blockIdx.x;
  int bh, slot;
  if (BH % 8 == 0) {
    // One (batch, head)'s query tiles on one XCD (its K and V from that
    // XCD's L2). order 0: a head's tiles in a row, latest first; order g > 0:
    // heads in groups of g per XCD, each group's tiles latest first across
    // its heads, so the heaviest tiles of the last group start early and
    // light ones end the launch.
    const int x = bid & 7, n = bid >> 3;
    if (order > 0) {
      const int hx = BH / 8;
      const int gsz = std::min(order, hx);
      const int span = gsz * nslots;
      const int grp = n / span, w = n - grp * span;
      const int gfirst = grp * gsz, gcount = std::min(gsz, hx - gfirst);
      slot = w / gcount;
      bh = (gfirst + w % gcount) * 8 + x;
    } else {
      bh = (n / nslots) * 8 + x;
      slot = n % nslots;
    }
  } else {
    bh = bid % BH;
    slot = bid / BH;
  }
  const int tile0 = nq - 1 - slot;
  const int tile1 = pair && slot < tile0 ? slot : -1;
  const int b = bh / p.Hq, h = bh - b * p.Hq;
  const int hk = h / (p.Hq / p.Hkv);
  const uint16_t* Qp = Q + (int64_t)b * p.q_b + (int64_t)h * p.q_h;
  const uint16_t* Kp = K + (int64_t)b * p.k_b + (int64_t)hk * p.k_h;
  const uint16_t* Vp = V + (int64_t)b * p.v_b + (int64_t)hk * p.v_h;
  uint16_t* Op = O + (int64_t)b * p.o_b + (int64_t)h * p.o_h;
  for (int ti = 0; ti < 2; ++ti) {
  const int qtile = ti == 0 ? tile0 : tile1;
  if (qtile < 0) break;
  if (ti > 0) __syncthreads();  // the first tile's last LDS reads are done
  const int q0 = qtile * FQ;

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int g = lane >> 4, c16 = lane & 15;
  const u32x4 zero = {0u, 0u, 0u, 0u};

  u32x4 qf[2][NDS];
  int lim[2];
  const int64_t off = read_offset(p);
#pragma unroll
  for (int qt = 0; qt < 2; ++qt) {
    const int q = q0 + wave * 32 + qt * 16 + c16;
#pragma unroll
    for (int ds = 0; ds < NDS; ++ds)
      qf[qt][ds] = q < p.Sq ? *reinterpret_cast<const u32x4*>(Qp + (int64_t)q * p.q_s + ds * 32 + g * 8) : zero;
    lim[qt] = key_limit(p, off, q);
  }
  const int kend = key_limit(p, off, std::min(q0 + FQ, p.Sq) - 1) + 1;
  const int free_end = key_limit(p, off, q0) + 1;
  const int nblocks = (kend + PK - 1) / PK;

  // Buffer resources over this head's keys: rows past Skv read as zero.
  const uint32_t k_bytes = (uint32_t)(((int64_t)(p.Skv - 1) * p.k_s + D) * 2);
  const uint32_t v_bytes = (uint32_t)(((int64_t)(p.Skv - 1) * p.v_s + D) * 2);
  const __amdgpu_buffer_rsrc_t krs =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(Kp), 0, p.Skv > 0 ? (int)k_bytes : 0, 0x00020000);
  const __amdgpu_buffer_rsrc_t vrs =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(Vp), 0, p.Skv > 0 ? (int)v_bytes : 0, 0x00020000);
  // Wave w fills rows 16w .. 16w+15 of a stage, four rows per load; the
  // lane part of each load's offset is fixed, the block part is scalar.
  const int wave_u = __builtin_amdgcn_readfirstlane(wave);
  const int lrow = lane >> 4, lslot = lane & 15;
  uint32_t koff[4], voff[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int row = wave_u * 16 + i * 4 + lrow;
    koff[i] = (uint32_t)(((int64_t)row * p.k_s + ((lslot ^ (row & 15)) * 8)) * 2);
    voff[i] = (uint32_t)(((int64_t)row * p.v_s + ((lslot ^ ((row & 7) << 1)) * 8)) * 2);
  }
  auto dma_k = [&](int kb, int stage) {
    const uint32_t sblk = (uint32_t)((int64_t)kb * PK * p.k_s * 2);
#pragma unroll
    for (int i = 0; i < 4; ++i)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(krs, (attn_lds_ptr)(Ks + stage * PSTAGE + (wave_u * 16 + i * 4) * 128),
                                               16, koff[i], sblk, 0, 0);
  };
  auto dma_v = [&](int kb, int stage) {
    const uint32_t sblk = (uint32_t)((int64_t)kb * PK * p.v_s * 2);
#pragma unroll
    for (int i = 0; i < 4; ++i)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(vrs, (attn_lds_ptr)(Vs + stage * PSTAGE + (wave_u * 16 + i * 4) * 128),
                                               16, voff[i], sblk, 0, 0);
  };

  const float c2 = p.scale * 1.44269504088896340736f;
  float m[2] = {-INFINITY, -INFINITY};
  f32x4 oacc[NDT][2];
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt) oacc[dt][0] = oacc[dt][1] = f32x4{0.f, 0.f, 0.f, 0.f};
  // Row sums: O^T rows of an all-ones V^T tile (every element of a lane's
  // accumulator holds its query's sum).
  f32x4 lacc[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
  const uint32_t one2 = kF16 ? 0x3c003c00u : 0x3f803f80u;
  const u32x4 ones = {one2, one2, one2, one2};

  // S^T[key][query] of block kb for the wave's 32 queries, from K stage `stage`.
  auto scores = [&](int stage, f32x4 (&sacc)[4][2]) {
    const uint16_t* ks = Ks + stage * PSTAGE;
#pragma unroll
    for (int kt = 0; kt < 4; ++kt) sacc[kt][0] = sacc[kt][1] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ds = 0; ds < NDS; ++ds) {
#pragma unroll
      for (int kt = 0; kt < 4; ++kt) {
        const u32x4 a = *reinterpret_cast<const u32x4*>(&ks[pk_swz(kt * 16 + c16, ds * 4 + g)]);
        sacc[kt][0] = mfma16<kF16>(a, qf[0][ds], sacc[kt][0]);
        sacc[kt][1] = mfma16<kF16>(a, qf[1][ds], sacc[kt][1]);
      }
    }
  };
  // Softmax of block kb's scores into P^T fragments; running max, sum and
  // output rescale.
  // Keys past a query's limit: only blocks that reach past the first
  // query's limit have any (a branch of its own, so unmasked blocks pay
  // nothing per score).
  auto mask = [&](int kb, f32x4 (&sacc)[4][2]) {
    if (kb * PK + PK <= free_end) return;
#pragma unroll
    for (int qt = 0; qt < 2; ++qt)
#pragma unroll
      for (int kt = 0; kt < 4; ++kt)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (kb * PK + kt * 16 + g * 4 + r > lim[qt]) sacc[kt][qt][r] = -INFINITY;
  };
  // Running max: raised only when a block's max exceeds it by more than
  // 2^8 in the exponential (then the output and sum are rescaled), so the
  // exponentials stay below 2^8 and most blocks skip the rescale. The row
  // sums come from the P.V products (a row of ones beside V), so the softmax
  // itself is max, round, exponential and pack.
  auto softmax = [&](int kb, f32x4 (&sacc)[4][2], u32x4 (&pf)[2][2]) {
    (void)kb;
    float alpha[2];
#pragma unroll
    for (int qt = 0; qt < 2; ++qt) {
      float s[4][4];
#pragma unroll
      for (int kt = 0; kt < 4; ++kt)
#pragma unroll
        for (int r = 0; r < 4; ++r) s[kt][r] = sacc[kt][qt][r];
      float mx = -INFINITY;
#pragma unroll
      for (int kt = 0; kt < 4; ++kt)
        mx = __builtin_elementwise_maximum(
            mx, __builtin_elementwise_maximum(__builtin_elementwise_maximum(s[kt][0], s[kt][1]),
                                              __builtin_elementwise_maximum(s[kt][2], s[kt][3])));
      mx = __builtin_elementwise_maximum(mx, __shfl_xor(mx, 16));
      mx = __builtin_elementwise_maximum(mx, __shfl_xor(mx, 32));
      if constexpr (kRound) mx = round16<kF16>(mx);
      const bool raise = mx * c2 > m[qt] * c2 + 8.f;
      const float mnew = raise ? mx : m[qt];
      const float mc = (mnew == -INFINITY ? 0.f : mnew) * c2;
      alpha[qt] = __builtin_amdgcn_exp2f(m[qt] * c2 - mc);
      m[qt] = mnew;
#pragma unroll
      for (int kt = 0; kt < 4; ++kt)
#pragma unroll
        for (int r = 0; r < 4; r += 2) {
          float x0 = s[kt][r], x1 = s[kt][r + 1];
          if constexpr (kRound) {
            const uint32_t pk = pack2<kF16>(x0, x1);
            if constexpr (kF16) {
              x0 = (float)__builtin_bit_cast(_Float16, (uint16_t)(pk & 0xffffu));
              x1 = (float)__builtin_bit_cast(_Float16, (uint16_t)(pk >> 16));
            } else {
              x0 = __builtin_bit_cast(float, pk << 16);
              x1 = __builtin_bit_cast(float, pk & 0xffff0000u);
            }
          }
          s[kt][r] = __builtin_amdgcn_exp2f(fmaf(x0, c2, -mc));
          s[kt][r + 1] = __builtin_amdgcn_exp2f(fmaf(x1, c2, -mc));
        }
#pragma unroll
      for (int st = 0; st < 2; ++st)
        pf[qt][st] = u32x4{pack2<kF16>(s[2 * st][0], s[2 * st][1]), pack2<kF16>(s[2 * st][2], s[2 * st][3]),
                           pack2<kF16>(s[2 * st + 1][0], s[2 * st + 1][1]),
                           pack2<kF16>(s[2 * st + 1][2], s[2 * st + 1][3])};
    }
    if (!__all(alpha[0] == 1.f && alpha[1] == 1.f)) {
#pragma unroll
      for (int qt = 0; qt < 2; ++qt) {
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt) oacc[dt][qt] *= alpha[qt];
        lacc[qt][0] *= alpha[qt];
      }
    }
  };
  // O^T[d][query] += V^T[d][key] . P^T[key][query] from V stage `stage`.
  auto pv = [&](int stage, const u32x4 (&pf)[2][2]) {
    const uint16_t* vs = Vs + stage * PSTAGE;
    const int i = lane & 15;
#pragma unroll
    for (int st = 0; st < 2; ++st) {
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt) {
        const int r0 = st * 32 + 4 * g + (i >> 2), r1 = r0 + 16;
        const int ch = 2 * dt + ((i & 3) >> 1), sub = 4 * (i & 1);
        const attn_v4i16 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (attn_lds_v4i16*)((__attribute__((address_space(3))) uint16_t*)(vs + pv_swz(r0, ch) + sub)));
        const attn_v4i16 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (attn_lds_v4i16*)((__attribute__((address_space(3))) uint16_t*)(vs + pv_swz(r1, ch) + sub)));
        const u32x2 l2 = __builtin_bit_cast(u32x2, lo), h2 = __builtin_bit_cast(u32x2, hi);
        const u32x4 a = u32x4{l2[0], l2[1], h2[0], h2[1]};
        oacc[dt][0] = mfma16<kF16>(a, pf[0][st], oacc[dt][0]);
        oacc[dt][1] = mfma16<kF16>(a, pf[1][st], oacc[dt][1]);
      }
      lacc[0] = mfma16<kF16>(ones, pf[0][st], lacc[0]);
      lacc[1] = mfma16<kF16>(ones, pf[1][st], lacc[1]);
    }
  };

  f32x4 sA[4][2];
  u32x4 pf[2][2];
  // Block kb from stage kb & 1 while block kb + 1 loads into the other
  // (read in the step before); two workgroups per CU overlap one's MFMAs
  // with the other's softmax. A wave whose 32 queries allow none of a
  // block's keys (the diagonal blocks past its last query) only takes part
  // in the loads and barriers.
  const int wave_last = key_limit(p, off, std::min(q0 + wave * 32 + 31, p.Sq - 1));
  if (nblocks > 0) {
    dma_k(0, 0);
    dma_v(0, 0);
  }
  for (int kb = 0; kb < nblocks; ++kb) {
    __builtin_amdgcn_s_waitcnt(attn_vmcnt0());
    __syncthreads();
    if (kb + 1 < nblocks) {
      dma_k(kb + 1, (kb + 1) & 1);
      dma_v(kb + 1, (kb + 1) & 1);
    }
    if (kb * PK > wave_last) continue;
    // With `prio`, the matrix-core phases run at raised wave priority: on a
    // SIMD whose other wave is in its softmax, the MFMAs issue first
    // (environment: PJRTX_ATTN_PRIO=0 disables; 360-365 vs 368-370 us on
    // [8,32,2048,128] causal bf16).
    if (prio) __builtin_amdgcn_s_setprio(1);
    scores(kb & 1, sA);
    if (prio) __builtin_amdgcn_s_setprio(0);
    mask(kb, sA);
    softmax(kb, sA, pf);
    if (prio) __builtin_amdgcn_s_setprio(1);
    pv(kb & 1, pf);
    if (prio) __builtin_amdgcn_s_setprio(0);
  }

#pragma unroll
  for (int qt = 0; qt < 2; ++qt) {
    const int q = q0 + wave * 32 + qt * 16 + c16;
    if (q >= p.Sq) continue;
    uint16_t* orow = Op + (int64_t)q * p.o_s;
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) {
      const f32x4 o = oacc[dt][qt];
      const float lq = lacc[qt][0];
      *reinterpret_cast<u32x2*>(orow + dt * 16 + g * 4) =
          u32x2{pack2<kF16>(o[0] / lq, o[1] / lq), pack2<kF16>(o[2] / lq, o[3] / lq)};
    }
  }
  }
}

// ----------------------------------------------------------------- rows

template <typename T>
struct Elem;
template <>
struct Elem<float> {
  __device__ static float get(float x) { return x; }
  __device__ static float put(float x) { return x; }
};
template <>
struct Elem<uint16_t> {  // bf16
  __device__ static float get(uint16_t x) { return bf16_to_f32(x); }
  __device__ static uint16_t put(float x) { return f32_to_bf16_rne(x); }
};
template <>
struct Elem<_Float16> {
  __device__ static float get(_Float16 x) { return (float)x; }
  __device__ static _Float16 put(float x) { return (_Float16)x; }
};

// Head dims [lane*DPL, lane*DPL + DPL) belong to the lane in the P.V pass.
template <typename T, int DPL>
__global__ void __launch_bounds__(256) attn_rows(AttnParams p, const T* __restrict__ Q, const T* __restrict__ K,
                                                 const T* __restrict__ V, T* __restrict__ O) {
  constexpr int DMAX = 64 * DPL;
  __shared__ float qs[DMAX];
  __shared__ float wm[4], wl[4];
  __shared__ float wo[4][DMAX];
  const int row = blockIdx.x;
  const int q = row % p.Sq;
  const int bh = row / p.Sq;
  const int b = bh / p.Hq, h = bh - b * p.Hq;
  const int hk = h / (p.Hq / p.Hkv);
  const T* Kp = K + (int64_t)b * p.k_b + (int64_t)hk * p.k_h;
  const T* Vp = V + (int64_t)b * p.v_b + (int64_t)hk * p.v_h;
  const T* qrow = Q + (int64_t)b * p.q_b + (int64_t)h * p.q_h + (int64_t)q * p.q_s;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int D = p.D;
  for (int d = tid; d < D; d += 256) qs[d] = Elem<T>::get(qrow[d]);
  __syncthreads();
  const int nkeys = key_limit(p, read_offset(p), q) + 1;
  const int nb = (nkeys + 63) / 64;
  float m = -INFINITY, l = 0.f, o[DPL];
#pragma unroll
  for (int c = 0; c < DPL; ++c) o[c] = 0.f;
  for (int kb = wave; kb < nb; kb += 4) {
    const int key = kb * 64 + lane;
    float s = -INFINITY;
    if (key < nkeys) {
      const T* kr = Kp + (int64_t)key * p.k_s;
      float acc = 0.f;
      for (int d = 0; d < D; ++d) acc += qs[d] * Elem<T>::get(kr[d]);
      if (p.round_scores) acc = Elem<T>::get(Elem<T>::put(acc));
      s = acc * p.scale;
    }
    float mx = s;
#pragma unroll
    for (int k = 32; k >= 1; k >>= 1) mx = fmaxf(mx, __shfl_xor(mx, k));
    const float mnew = fmaxf(m, mx);
    const float mref = mnew == -INFINITY ? 0.f : mnew;
    const float alpha = expf(m - mref);
    const float pe = expf(s - mref);
    float ps = pe;
#pragma unroll
    for (int k = 32; k >= 1; k >>= 1) ps += __shfl_xor(ps, k);
    l = l * alpha + ps;
    m = mnew;
#pragma unroll
    for (int c = 0; c < DPL; ++c) o[c] *= alpha;
    const int last = nkeys - 1;
#pragma unroll 8
    for (int j = 0; j < 64; ++j) {
      const float pj = __shfl(pe, j);
      const T* vr = Vp + (int64_t)std::min(kb * 64 + j, last) * p.v_s + lane * DPL;
#pragma unroll
      for (int c = 0; c < DPL; ++c)
        if (lane * DPL + c < D) o[c] += pj * Elem<T>::get(vr[c]);
    }
  }
  if (lane == 0) {
    wm[wave] = m;
    wl[wave] = l;
  }
#pragma unroll
  for (int c = 0; c < DPL; ++c) wo[wave][lane * DPL + c] = o[c];
  __syncthreads();
  if (wave != 0) return;
  const float mall = fmaxf(fmaxf(wm[0], wm[1]), fmaxf(wm[2], wm[3]));
  const float mref = mall == -INFINITY ? 0.f : mall;
  float f[4], lsum = 0.f;
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    f[w] = expf(wm[w] - mref);
    lsum += wl[w] * f[w];
  }
  T* orow = O + (int64_t)b * p.o_b + (int64_t)h * p.o_h + (int64_t)q * p.o_s;
#pragma unroll
  for (int c = 0; c < DPL; ++c) {
    const int d = lane * DPL + c;
    if (d >= D) continue;
    float acc = 0.f;
#pragma unroll
    for (int w = 0; w < 4; ++w) acc += wo[w][d] * f[w];
    orow[d] = Elem<T>::put(acc / lsum);
  }
}

// --------------------------------------------------------------- decode

// Few queries per (batch, head): the keys of each query row are split into
// chunks of `keys_per_split` (a multiple of 64), one workgroup per (row,
// chunk), so a decode step launches rows x splits workgroups. A workgroup
// walks its chunk 64 keys per pass with both loads in flight at once: for
// the scores 4 lanes share a key (each a quarter of its K row, folded by two
// xor shuffles), for P.V a lane owns one 16-byte head-dim piece of a group of
// keys (each V row read as one coalesced span). Each wave scores a quarter
// of a pass's keys and its P.V lanes read the same keys, so it runs an
// online softmax of its own (max and sum by xor shuffles, P handed to the
// P.V lanes by shuffles) with no barrier between passes; after the last
// pass the four waves' (max, sum, output) meet through LDS, the key groups
// of P.V folded in group order, each scaled by its wave's exp(m_w - max).
// Splits past the row's last allowed key exit at once.
//
// One split: the workgroup writes the row. Otherwise each split writes
// (m, l, unnormalized O) to `part`; in fused mode (workgroup b runs on XCD
// b % 8 and the row's splits were placed on one XCD) the split counts its
// arrival on the row's L2 counter once its stores are acknowledged by that
// L2, and the last to arrive merges the splits in split order (reading past
// its L1) and puts the counter back to zero; without it attn_combine, launched
// next, merges them the same way. The merge order is fixed, so the result
// does not depend on which split arrives last.
//
// Partials mode (`mode` kDecodePartials): `part` is the step's output. Every
// split writes its (m, l, unnormalized O), one split included, and the
// splits past the row's last allowed key write l = -1 (a sum of exponentials
// is never negative) and exit, so the reader (a decode GEMV staging its
// input) merges the splits whose l is not -1, in split order, with the same
// arithmetic as merge_splits.
constexpr int DK = 64;
constexpr int kDecodeCombine = 0, kDecodeFused = 1, kDecodePartials = 2;
constexpr int kCounterStride = 32;  // uint32 per arrival counter: one 128-byte line each

template <typename T>
__device__ __forceinline__ int active_splits(const AttnParams& p, int q, int keys_per_split) {
  const int nkeys = key_limit(p, read_offset(p), q) + 1;
  return nkeys <= 0 ? 1 : (nkeys + keys_per_split - 1) / keys_per_split;
}

// Merges splits 0..nact-1 (nact <= 64) of a row's partials `pr` (per split:
// m, l, then D unnormalized outputs) into out[d] for d < D, by the block's
// first D threads (D <= blockDim.x). The splits' (m, l) go through LDS first,
// one load per thread; each output then folds its splits in split order,
// eight loads in flight at a time. kCoherent: loads that skip this CU's L1
// (other workgroups of this XCD wrote the partials).
template <bool kCoherent, typename T>
__device__ __forceinline__ void merge_splits(const float* pr, int nact, int D, T* out, float* msh, float* lsh) {
  auto ld = [](const float* a) {
    if constexpr (kCoherent) return __hip_atomic_load(a, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    else return *a;
  };
  const int tid = threadIdx.x;
  if (nact <= 16) {
    // Up to 16 splits: every (m, l, value) of the thread's column requested
    // at once (clamped, unconditional loads: one L2 round trip instead of
    // three), then the same fold in split order as below, so the same bits.
    if (tid >= D) return;
    float ms[16], ls[16], vs[16];
#pragma unroll
    for (int u = 0; u < 16; ++u) {
      const int64_t sp = (int64_t)(u < nact ? u : nact - 1) * (D + 2);
      ms[u] = ld(pr + sp);
      ls[u] = ld(pr + sp + 1);
      vs[u] = ld(pr + sp + 2 + tid);
    }
    float mall = -INFINITY;
#pragma unroll
    for (int u = 0; u < 16; ++u)
      if (u < nact) mall = fmaxf(mall, ms[u]);
    const float mref = mall == -INFINITY ? 0.f : mall;
    float lsum = 0.f, acc = 0.f;
#pragma unroll
    for (int u = 0; u < 16; ++u) {
      if (u < nact) {
        const float f = expf(ms[u] - mref);
        lsum += ls[u] * f;
        acc += vs[u] * f;
      }
    }
    out[tid] = Elem<T>::put(acc / lsum);
    return;
  }
  if (tid < nact) {
    msh[tid] = ld(pr + (int64_t)tid * (D + 2));
    lsh[tid] = ld(pr + (int64_t)tid * (D + 2) + 1);
  }
  __syncthreads();
  if (tid >= D) return;
  float mall = -INFINITY;
  for (int s = 0; s < nact; ++s) mall = fmaxf(mall, msh[s]);
  const float mref = mall == -INFINITY ? 0.f : mall;
  float lsum = 0.f, acc = 0.f;
  for (int s0 = 0; s0 < nact; s0 += 8) {
    float v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) v[u] = s0 + u < nact ? ld(pr + (int64_t)(s0 + u) * (D + 2) + 2 + tid) : 0.f;
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      if (s0 + u < nact) {
        const float f = expf(msh[s0 + u] - mref);
        lsum += lsh[s0 + u] * f;
        acc += v[u] * f;
      }
    }
  }
  out[tid] = Elem<T>::put(acc / lsum);
}

template <typename T, int NCH, int DKT>
__global__ void __launch_bounds__(256) attn_decode(AttnParams p, const T* __restrict__ Q, const T* __restrict__ K,
                                                   const T* __restrict__ V, T* __restrict__ O, float* __restrict__ part,
                                                   int keys_per_split, int nsplit, uint32_t* __restrict__ counters,
                                                   int mode) {
  constexpr int EPC = 16 / sizeof(T);  // elements per 16-byte piece
  constexpr int D = NCH * EPC;
  constexpr int LPK = 256 / DKT;       // lanes per key in the scores (4 for 64-key passes, 8 for 32)
  static_assert(NCH % LPK == 0 || DKT == 64, "a K row splits evenly over a key's lanes");
  constexpr int CPT = NCH >= LPK ? NCH / LPK : 1;  // pieces of a K row per lane
  constexpr int G = 256 / NCH;         // key groups in P.V
  constexpr int KG = DKT / G;          // keys per group
  static_assert(KG >= 1, "at least one key per P.V group");
  __shared__ float wred[2][4];
  __shared__ float ow[G][D];
  __shared__ float msh[64], lsh[64];
  __shared__ uint32_t last_s;
  const int rows = p.B * p.Hq * p.Sq;
  // The row's splits share b % 8 (one XCD): row = (b % 8) + 8 * ((b / 8) / nsplit).
  const int xcd = blockIdx.x & 7, jj = blockIdx.x >> 3;
  const int row = xcd + 8 * (jj / nsplit);
  const int split = jj % nsplit;
  if (row >= rows) return;
  const int q = row % p.Sq;
  const int bh = row / p.Sq;
  const int b = bh / p.Hq, h = bh - b * p.Hq;
  const int hk = h / (p.Hq / p.Hkv);
  const T* Kp = K + (int64_t)b * p.k_b + (int64_t)hk * p.k_h;
  const T* Vp = V + (int64_t)b * p.v_b + (int64_t)hk * p.v_h;
  const T* Qp = Q + (int64_t)b * p.q_b + (int64_t)h * p.q_h + (int64_t)q * p.q_s;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int quarter = tid % LPK, kslot = tid / LPK;  // scores: key slot, share of the row
  const int c = tid % NCH, g = tid / NCH;             // P.V: head-dim piece, key group
  const int k0 = split * keys_per_split;
  // The query and the split's first pass of K and V rows are requested
  // before the position is read (it only decides which keys count): one
  // memory round trip for all of them. Rows are clamped to the cache; keys
  // past the allowed ones are masked below whatever those rows hold.
  u32x4 qraw[CPT];
#pragma unroll
  for (int i = 0; i < CPT; ++i) qraw[i] = *reinterpret_cast<const u32x4*>(Qp + (quarter * CPT + i) * EPC);
  u32x4 kv0[CPT], vv0[KG];
  const int slast = p.Skv > 0 ? p.Skv - 1 : 0;
  if (p.Skv > 0) {
    const int kst = std::min(k0 + kslot, slast);
#pragma unroll
    for (int i = 0; i < CPT; ++i)
      kv0[i] = *reinterpret_cast<const u32x4*>(Kp + (int64_t)kst * p.k_s + (quarter * CPT + i) * EPC);
#pragma unroll
    for (int i = 0; i < KG; ++i) {
      const int kk = std::min(k0 + g * KG + i, slast);
      vv0[i] = *reinterpret_cast<const u32x4*>(Vp + (int64_t)kk * p.v_s + c * EPC);
    }
  }
  const int nkeys = key_limit(p, read_offset(p), q) + 1;
  const int nact = nkeys <= 0 ? 1 : (nkeys + keys_per_split - 1) / keys_per_split;
  if (split >= nact) {
    if (mode == kDecodePartials && tid == 0) part[((int64_t)row * nsplit + split) * (D + 2) + 1] = -1.f;
    return;
  }
  float qv[CPT * EPC];
#pragma unroll
  for (int i = 0; i < CPT; ++i) {
    const T* e8 = reinterpret_cast<const T*>(&qraw[i]);
#pragma unroll
    for (int e = 0; e < EPC; ++e) qv[i * EPC + e] = Elem<T>::get(e8[e]);
  }
  const int k1 = std::min(nkeys, k0 + keys_per_split);
  // Wave w scores keys w DKT/4 .. (w+1) DKT/4 - 1 of every pass, and its P.V
  // lanes read exactly those keys' V rows (group g's keys start at g KG, and
  // a wave's groups start at w DKT/4), so each wave keeps an online softmax
  // of its own (max, sum and output over its keys) and the passes need no
  // barrier: P moves from the scoring lanes to the P.V lanes by shuffles.
  // The four waves' states meet once, after the last pass.
  const int wk0 = wave * (DKT / 4);
  float m = -INFINITY, l = 0.f, o[EPC];
#pragma unroll
  for (int e = 0; e < EPC; ++e) o[e] = 0.f;
  for (int kb = k0; kb < k1; kb += DKT) {
    const int key = kb + kslot;
    u32x4 kv[CPT], vv[KG];
    if (kb == k0) {
#pragma unroll
      for (int i = 0; i < CPT; ++i) kv[i] = kv0[i];
#pragma unroll
      for (int i = 0; i < KG; ++i) vv[i] = vv0[i];
    } else {
      // later passes (splits of more than one pass): K and V requested
      // together, rows past k1 read the last allowed row
      const int kcl = std::min(key, k1 - 1);
#pragma unroll
      for (int i = 0; i < CPT; ++i)
        kv[i] = *reinterpret_cast<const u32x4*>(Kp + (int64_t)kcl * p.k_s + (quarter * CPT + i) * EPC);
#pragma unroll
      for (int i = 0; i < KG; ++i) {
        const int kk = std::min(kb + g * KG + i, k1 - 1);
        vv[i] = *reinterpret_cast<const u32x4*>(Vp + (int64_t)kk * p.v_s + c * EPC);
      }
    }
    float acc = 0.f;
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      const T* e8 = reinterpret_cast<const T*>(&kv[i]);
#pragma unroll
      for (int e = 0; e < EPC; ++e) acc += qv[i * EPC + e] * Elem<T>::get(e8[e]);
    }
#pragma unroll
    for (int k = 1; k < LPK; k <<= 1) acc += __shfl_xor(acc, k);
    if (p.round_scores) acc = Elem<T>::get(Elem<T>::put(acc));
    const float sc = key < k1 ? acc * p.scale : -INFINITY;
    // the wave's max and sum over its keys (xor butterflies over the key
    // bits of the lane index: every lane ends with them)
    float mx = sc;
#pragma unroll
    for (int k = 32; k >= LPK; k >>= 1) mx = fmaxf(mx, __shfl_xor(mx, k));
    const float mnew = fmaxf(m, mx);
    const float mref = mnew == -INFINITY ? 0.f : mnew;
    const float alpha = expf(m - mref);
    const float pe = expf(sc - mref);
    float sum = quarter == 0 ? pe : 0.f;
#pragma unroll
    for (int k = 32; k >= LPK; k >>= 1) sum += __shfl_xor(sum, k);
    l = l * alpha + sum;
    m = mnew;
#pragma unroll
    for (int e = 0; e < EPC; ++e) o[e] *= alpha;
#pragma unroll
    for (int i = 0; i < KG; ++i) {
      // a key past k1 adds nothing (its row may hold anything); its
      // exponential sits in lane (key - wk0) LPK of this wave
      const int kk = g * KG + i;
      const bool in = kb + kk < k1;
      const float pj = __shfl(pe, (kk - wk0) * LPK);
      const T* e8 = reinterpret_cast<const T*>(&vv[i]);
#pragma unroll
      for (int e = 0; e < EPC; ++e) o[e] += in ? pj * Elem<T>::get(e8[e]) : 0.f;
    }
  }
  // The waves meet: each wave's (l, O) scaled by exp(m_w - max m_w).
#pragma unroll
  for (int e = 0; e < EPC; ++e) ow[g][c * EPC + e] = o[e];
  if (lane == 0) {
    wred[0][wave] = m;
    wred[1][wave] = l;
  }
  __syncthreads();
  float fw[4];
  {
    const float mall = fmaxf(fmaxf(wred[0][0], wred[0][1]), fmaxf(wred[0][2], wred[0][3]));
    const float mr = mall == -INFINITY ? 0.f : mall;
#pragma unroll
    for (int w = 0; w < 4; ++w) fw[w] = expf(wred[0][w] - mr);
    l = ((wred[1][0] * fw[0] + wred[1][1] * fw[1]) + wred[1][2] * fw[2]) + wred[1][3] * fw[3];
    m = mall;
  }
  float acc = 0.f;
  if (tid < D) {
#pragma unroll
    for (int gg = 0; gg < G; ++gg) acc += ow[gg][tid] * fw[gg / (G / 4)];
  }
  T* orow = O + (int64_t)b * p.o_b + (int64_t)h * p.o_h + (int64_t)q * p.o_s;
  if (nact == 1 && mode != kDecodePartials) {
    if (tid < D) orow[tid] = Elem<T>::put(acc / l);
    return;
  }
  float* pr = part + (int64_t)row * nsplit * (D + 2);
  if (tid < D) pr[(int64_t)split * (D + 2) + 2 + tid] = acc;
  if (tid == 0) {
    pr[(int64_t)split * (D + 2)] = m;
    pr[(int64_t)split * (D + 2) + 1] = l;
  }
  if (mode != kDecodeFused) return;
  __builtin_amdgcn_s_waitcnt(0);  // this wave's partial stores are in the L2
  __syncthreads();
  if (tid == 0) {
    uint32_t* ctr = counters + (int64_t)row * kCounterStride;
    const uint32_t last = __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                          (uint32_t)(nact - 1);
    if (last) __hip_atomic_store(ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    last_s = last;
  }
  __syncthreads();
  if (!last_s) return;
  merge_splits<true>(pr, nact, D, orow, msh, lsh);
}

template <typename T>
__global__ void __launch_bounds__(512) attn_combine(AttnParams p, const float* __restrict__ part, int nsplit,
                                                    int keys_per_split, T* __restrict__ O) {
  const int row = blockIdx.x;
  const int q = row % p.Sq;
  const int bh = row / p.Sq;
  const int b = bh / p.Hq, h = bh - b * p.Hq;
  const int nact = active_splits<T>(p, q, keys_per_split);
  if (nact == 1) return;  // the split kernel wrote the row
  __shared__ float msh[64], lsh[64];
  const float* pr = part + (int64_t)row * nsplit * (p.D + 2);
  merge_splits<false>(pr, nact, p.D, O + (int64_t)b * p.o_b + (int64_t)h * p.o_h + (int64_t)q * p.o_s, msh, lsh);
}

template <typename T>
bool decode_fits(const AttnParams& p) {
  constexpr int EPC = 16 / sizeof(T);
  if (p.D % EPC != 0) return false;
  const int nch = p.D / EPC;
  if (nch != 4 && nch != 8 && nch != 16 && nch != 32) return false;
  for (int64_t st : {p.q_b, p.q_h, p.q_s, p.k_b, p.k_h, p.k_s, p.v_b, p.v_h, p.v_s})
    if (st % EPC != 0) return false;
  return true;
}

template <typename T>
void launch_decode(hipStream_t s, const AttnParams& p, const T* q, const T* k, const T* v, T* o, float* part,
                   int nsplit, int keys_per_split, uint32_t* counters, int mode) {
  constexpr int EPC = 16 / sizeof(T);
  const int64_t rows = static_cast<int64_t>(p.B) * p.Hq * p.Sq;
  const dim3 grid(static_cast<uint32_t>(8 * ((rows + 7) / 8) * nsplit)), block(256);
  // 32-key passes for splits that are not whole 64-key passes (K rows of at
  // least 8 pieces, so a key's 8 lanes each take whole pieces).
  const bool half = keys_per_split % DK != 0;
#define PJRTX_DEC(NC, DKT) \
  hipLaunchKernelGGL((attn_decode<T, NC, DKT>), grid, block, 0, s, p, q, k, v, o, part, keys_per_split, nsplit, counters, mode)
  switch (p.D / EPC) {
    case 4: PJRTX_DEC(4, 64); break;
    case 8: if (half) PJRTX_DEC(8, 32); else PJRTX_DEC(8, 64); break;
    case 16: if (half) PJRTX_DEC(16, 32); else PJRTX_DEC(16, 64); break;
    default: if (half) PJRTX_DEC(32, 32); else PJRTX_DEC(32, 64); break;
  }
#undef PJRTX_DEC
  if (nsplit > 1 && mode == kDecodeCombine)
    hipLaunchKernelGGL((attn_combine<T>), dim3(static_cast<uint32_t>(rows)), dim3(std::max(64, p.D)), 0, s, p, part,
                       nsplit, keys_per_split, o);
}

template <typename T>
void launch_rows(hipStream_t s, const AttnParams& p, const void* Q, const void* K, const void* V, void* out) {
  const dim3 grid(static_cast<uint32_t>(static_cast<int64_t>(p.B) * p.Hq * p.Sq)), block(256);
  const T* q = static_cast<const T*>(Q);
  const T* k = static_cast<const T*>(K);
  const T* v = static_cast<const T*>(V);
  T* o = static_cast<T*>(out);
  if (p.D <= 64) hipLaunchKernelGGL((attn_rows<T, 1>), grid, block, 0, s, p, q, k, v, o);
  else if (p.D <= 128) hipLaunchKernelGGL((attn_rows<T, 2>), grid, block, 0, s, p, q, k, v, o);
  else if (p.D <= 256) hipLaunchKernelGGL((attn_rows<T, 4>), grid, block, 0, s, p, q, k, v, o);
  else hipLaunchKernelGGL((attn_rows<T, 8>), grid, block, 0, s, p, q, k, v, o);
}

}  // namespace

bool attention_uses_tiles(const AttnParams& p, DType t) {
  if (t != DType::kBF16 && t != DType::kF16) return false;
  if (!(p.scale > 0.f)) return false;  // the tile kernel takes the row max before scaling
  if (p.D != 64 && p.D != 128) return false;
  if (p.Sq < 16) return false;
  for (int64_t st : {p.q_b, p.q_h, p.q_s, p.k_b, p.k_h, p.k_s, p.v_b, p.v_h, p.v_s})
    if (st % 8 != 0) return false;
  for (int64_t st : {p.o_b, p.o_h, p.o_s})
    if (st % 4 != 0) return false;
  return true;
}

AttnPath attention_path(const AttnParams& p, DType t, int* nsplit, int* keys_per_split) {
  *nsplit = 1;
  *keys_per_split = 0;
  if (attention_uses_tiles(p, t)) return AttnPath::kTiles;
  const bool fits = t == DType::kF32 ? decode_fits<float>(p) : t == DType::kBF16 ? decode_fits<uint16_t>(p)
                    : t == DType::kF16 ? decode_fits<_Float16>(p) : false;
  if (!fits) return AttnPath::kRows;
  // Splits of whole 64-key passes (32-key ones with
  // PJRTX_ATTN_DECODE_KEYS=32, head dims of 8 pieces or more; slower on the
  // decode workload, where each workgroup's fixed cost dominates): enough
  // splits for about PJRTX_ATTN_DECODE_WGS (512) workgroups over the rows,
  // at most 64 per row.
  const int64_t rows = static_cast<int64_t>(p.B) * p.Hq * p.Sq;
  const int64_t epc = t == DType::kF32 ? 4 : 8;
  const int unit = p.D / epc >= 8 && env_int("PJRTX_ATTN_DECODE_KEYS", 64) == 32 ? 32 : DK;
  const int64_t target = std::max<int64_t>(1, env_int("PJRTX_ATTN_DECODE_WGS", 512));
  const int passes = std::max(1, (p.Skv + unit - 1) / unit);
  const int want = static_cast<int>(std::max<int64_t>(1, std::min<int64_t>(64, (target + rows - 1) / rows)));
  const int n = std::min(passes, want);
  const int per = (passes + n - 1) / n;
  *keys_per_split = per * unit;
  *nsplit = (p.Skv + *keys_per_split - 1) / *keys_per_split;
  if (*nsplit < 1) *nsplit = 1;
  return AttnPath::kDecode;
}

size_t attention_scratch_bytes(const AttnParams& p, DType t) {
  int nsplit = 1, per = 0;
  if (attention_path(p, t, &nsplit, &per) != AttnPath::kDecode || nsplit == 1) return 0;
  return static_cast<size_t>(p.B) * p.Hq * p.Sq * nsplit * (p.D + 2) * sizeof(float);
}

void launch_attention(hipStream_t s, const AttnParams& p, DType t, const void* Q, const void* K, const void* V,
                      void* out, float* scratch, uint32_t* counters, bool xcd_local, bool partials_out) {
  PJRTX_CHECK(p.B >= 1 && p.Hq >= 1 && p.Hkv >= 1 && p.Hq % p.Hkv == 0 && p.D >= 1 && p.Sq >= 0 && p.Skv >= 0,
              Code::kInvalidArgument, "attention: bad shape");
  PJRTX_CHECK(p.D <= 512, Code::kUnimplemented, "attention: head dim above 512");
  PJRTX_CHECK(p.causal == 0 || p.q_coef == 0 || p.q_coef == 1, Code::kInternal, "attention: mask slope must be 0 or 1");
  if (p.Sq == 0) return;
  int nsplit = 1, per = 0;
  const AttnPath path = attention_path(p, t, &nsplit, &per);
  if (path == AttnPath::kDecode) {
    PJRTX_CHECK(static_cast<int64_t>(p.B) * p.Hq * p.Sq < (int64_t(1) << 31), Code::kUnimplemented,
                "attention: too many query rows");
    PJRTX_CHECK(!partials_out || nsplit > 1, Code::kInternal, "attention: partials output without key splits");
    if (partials_out) scratch = static_cast<float*>(out);
    PJRTX_CHECK(nsplit == 1 || scratch != nullptr, Code::kInternal, "attention: split decode needs scratch");
    const int64_t rows = static_cast<int64_t>(p.B) * p.Hq * p.Sq;
    const int mode = partials_out ? kDecodePartials
                      : xcd_local && counters != nullptr && rows <= kAttnCounterRows ? kDecodeFused
                                                                                      : kDecodeCombine;
    if (t == DType::kF32)
      launch_decode<float>(s, p, static_cast<const float*>(Q), static_cast<const float*>(K),
                           static_cast<const float*>(V), static_cast<float*>(out), scratch, nsplit, per, counters, mode);
    else if (t == DType::kBF16)
      launch_decode<uint16_t>(s, p, static_cast<const uint16_t*>(Q), static_cast<const uint16_t*>(K),
                              static_cast<const uint16_t*>(V), static_cast<uint16_t*>(out), scratch, nsplit, per,
                              counters, mode);
    else
      launch_decode<_Float16>(s, p, static_cast<const _Float16*>(Q), static_cast<const _Float16*>(K),
                              static_cast<const _Float16*>(V), static_cast<_Float16*>(out), scratch, nsplit, per,
                              counters, mode);
  } else if (path == AttnPath::kTiles) {
    const int64_t grid = static_cast<int64_t>(p.B) * p.Hq * ((p.Sq + FQ - 1) / FQ);
    PJRTX_CHECK(grid < (int64_t(1) << 31), Code::kUnimplemented, "attention: too many query tiles");
    const bool f16 = t == DType::kF16;
    const uint16_t* q = static_cast<const uint16_t*>(Q);
    const uint16_t* k = static_cast<const uint16_t*>(K);
    const uint16_t* v = static_cast<const uint16_t*>(V);
    uint16_t* o = static_cast<uint16_t*>(out);
    const dim3 g(static_cast<uint32_t>(grid)), block(256);
#define PJRTX_ATTN(F16, DIM, RND) hipLaunchKernelGGL((attn_tiles<F16, DIM, RND>), g, block, 0, s, p, q, k, v, o)
    const int order = static_cast<int>(env_int("PJRTX_ATTN_ORDER", 8));
    const int pair = p.causal && env_int("PJRTX_ATTN_PAIR", 1) != 0 ? 1 : 0;
    const dim3 gp(static_cast<uint32_t>(static_cast<int64_t>(p.B) * p.Hq *
                                        (pair ? ((p.Sq + FQ - 1) / FQ + 1) / 2 : (p.Sq + FQ - 1) / FQ)));
    const int prio = static_cast<int>(env_int("PJRTX_ATTN_PRIO", 1));
#define PJRTX_PIPE(F16, RND) hipLaunchKernelGGL((attn_pipe<F16, RND>), gp, block, 0, s, p, q, k, v, o, order, pair, prio)
    const bool rnd = p.round_scores != 0;
    // The DMA kernel addresses K and V through 32-bit buffer offsets;
    // PJRTX_ATTN_PIPE=0 keeps the register-staged tile kernel.
    const bool dma = p.D == 128 && env_int("PJRTX_ATTN_PIPE", 1) != 0 &&
                     ((int64_t)std::max(p.Skv, 1) + PK) * std::max(p.k_s, p.v_s) * 2 < (int64_t(1) << 31);
    if (dma && f16 && rnd) PJRTX_PIPE(true, true);
    else if (dma && f16) PJRTX_PIPE(true, false);
    else if (dma && rnd) PJRTX_PIPE(false, true);
    else if (dma) PJRTX_PIPE(false, false);
    else if (p.D == 128 && f16 && rnd) PJRTX_ATTN(true, 128, true);
    else if (p.D == 128 && f16) PJRTX_ATTN(true, 128, false);
    else if (p.D == 128 && rnd) PJRTX_ATTN(false, 128, true);
    else if (p.D == 128) PJRTX_ATTN(false, 128, false);
    else if (f16 && rnd) PJRTX_ATTN(true, 64, true);
    else if (f16) PJRTX_ATTN(true, 64, false);
    else if (rnd) PJRTX_ATTN(false, 64, true);
    else PJRTX_ATTN(false, 64, false);
#undef PJRTX_ATTN
#undef PJRTX_PIPE
  } else {
    PJRTX_CHECK(static_cast<int64_t>(p.B) * p.Hq * p.Sq < (int64_t(1) << 31), Code::kUnimplemented,
                "attention: too many query rows");
    switch (t) {
      case DType::kF32: launch_rows<float>(s, p, Q, K, V, out); break;
      case DType::kBF16: launch_rows<uint16_t>(s, p, Q, K, V, out); break;
      case DType::kF16: launch_rows<_Float16>(s, p, Q, K, V, out); break;
      default: fail(Code::kUnimplemented, "attention: element type must be f32, bf16 or f16");
    }
  }
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) fail(Code::kInternal, strformat("attention launch failed: %s", hipGetErrorString(e)));
}

}  // namespace pjrtx
