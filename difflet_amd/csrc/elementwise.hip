// Bandwidth-bound kernels of the DiT block: LayerNorm + adaLN modulation, RMSNorm, fused
// per-head q/k RMSNorm + rotary embedding, rotary embedding alone, GELU-tanh, gate/residual,
// the small-M GEMV of the modulation linears, and the sinusoidal timestep embedding.
//
// Layout: activations are token-major rows ([rows, dim], innermost contiguous). One wavefront
// owns one row, so every statistic is a wavefront reduction with no LDS and no barrier, and
// each lane moves 16-byte vectors (8 bf16) so HBM traffic is fully coalesced.
#include <type_traits>

#include "common.hpp"
#include <float.h>

namespace dlt {

// ------------------------------------------------------------------ vector load/store of 8
template <typename T> struct V8;
template <> struct V8<bf16> {
  static __device__ __forceinline__ void load(const bf16* p, float* v) {
    u32x4 r = *reinterpret_cast<const u32x4*>(p);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[2 * i] = bf16bits_to_f32(r[i] & 0xffffu);
      v[2 * i + 1] = bf16bits_to_f32(r[i] >> 16);
    }
  }
  static __device__ __forceinline__ void store(bf16* p, const float* v) {
    u32x4 r;
#pragma unroll
    for (int i = 0; i < 4; ++i) r[i] = pack_bf16x2(v[2 * i], v[2 * i + 1]);
    *reinterpret_cast<u32x4*>(p) = r;
  }
};
template <> struct V8<f16> {
  static __device__ __forceinline__ void load(const f16* p, float* v) {
    typedef _Float16 h8 __attribute__((ext_vector_type(8)));
    h8 r = *reinterpret_cast<const h8*>(p);
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = (float)r[i];
  }
  static __device__ __forceinline__ void store(f16* p, const float* v) {
    typedef _Float16 h8 __attribute__((ext_vector_type(8)));
    h8 r;
#pragma unroll
    for (int i = 0; i < 8; ++i) r[i] = (_Float16)v[i];
    *reinterpret_cast<h8*>(p) = r;
  }
};
template <> struct V8<float> {
  static __device__ __forceinline__ void load(const float* p, float* v) {
    f32x4 a = *reinterpret_cast<const f32x4*>(p);
    f32x4 b = *reinterpret_cast<const f32x4*>(p + 4);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[i] = a[i];
      v[4 + i] = b[i];
    }
  }
  static __device__ __forceinline__ void store(float* p, const float* v) {
    f32x4 a, b;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      a[i] = v[i];
      b[i] = v[4 + i];
    }
    *reinterpret_cast<f32x4*>(p) = a;
    *reinterpret_cast<f32x4*>(p + 4) = b;
  }
};

// Raw 16-byte (fp32: 32-byte) loads converted in a separate step, so a load inside a branch has
// no use there and the compiler need not wait for it before the branch ends.
template <typename T> struct Raw8 {
  u32x4 r;
  static __device__ __forceinline__ Raw8 load(const T* p) {
    return Raw8{*reinterpret_cast<const u32x4*>(p)};
  }
  static __device__ __forceinline__ Raw8 zero() { return Raw8{u32x4{0u, 0u, 0u, 0u}}; }
  __device__ __forceinline__ void cvt(float* v) const {
    if constexpr (std::is_same<T, bf16>::value) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        v[2 * i] = bf16bits_to_f32(r[i] & 0xffffu);
        v[2 * i + 1] = bf16bits_to_f32(r[i] >> 16);
      }
    } else {
      typedef _Float16 h8 __attribute__((ext_vector_type(8)));
      const h8 h = __builtin_bit_cast(h8, r);
#pragma unroll
      for (int i = 0; i < 8; ++i) v[i] = (float)h[i];
    }
  }
};
template <> struct Raw8<float> {
  f32x4 a, b;
  static __device__ __forceinline__ Raw8 load(const float* p) {
    return Raw8{*reinterpret_cast<const f32x4*>(p), *reinterpret_cast<const f32x4*>(p + 4)};
  }
  static __device__ __forceinline__ Raw8 zero() { return Raw8{f32x4{}, f32x4{}}; }
  __device__ __forceinline__ void cvt(float* v) const {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[i] = a[i];
      v[4 + i] = b[i];
    }
  }
};

// ------------------------------------------------------------------ LayerNorm + modulation
// NV = 16-byte vectors per lane; dim <= 64 * 8 * NV and dim % 8 == 0. One wavefront per row:
// chunk j of a lane is elements (lane + 64 j) * 8 .. + 8 of the row.
template <typename TX, typename TM, int NV, bool FULL>
struct LnRow {
  // 16-bit modulation vectors are held like the row; fp32 ones (8 registers per chunk each)
  // are read where they are used, from L1 / L2 (every row of a batch shares them)
  static constexpr bool HOLD = sizeof(TM) == 2;
  Raw8<TX> x[NV];
  Raw8<TM> m[HOLD ? NV : 1], a[HOLD ? NV : 1];
  const TM* mp;
  const TM* ap;
  int lane_, dim_;
  float mean, rstd, madd;

  // Every load of the row and of both modulation vectors is issued before the first use, from
  // an in-bounds address (chunks past dim re-read chunk 0 and are excluded after): a load
  // guarded by c < dim next to its use makes the compiler wait for each chunk in turn. The
  // row stays in registers as loaded (16-bit words), so a wave needs few registers and many
  // rows are in flight per compute unit. A missing modulation vector reads as zeros, and the
  // output is LN(x) * (m + madd) + a with madd = 1 for one_plus or no mul vector.
  __device__ __forceinline__ void load(const TX* __restrict__ xr, int dim, const TM* mb,
                                       const TM* ab, int one_plus, float eps, int lane) {
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      const int c = (lane + 64 * j) * 8;
      x[j] = Raw8<TX>::load(xr + (FULL || c < dim ? c : 0));
    }
    mp = mb;
    ap = ab;
    lane_ = lane;
    dim_ = dim;
    if constexpr (HOLD) {
#pragma unroll
      for (int j = 0; j < NV; ++j) {
        const int c = (lane + 64 * j) * 8;
        m[j] = mb ? Raw8<TM>::load(mb + (FULL || c < dim ? c : 0)) : Raw8<TM>::zero();
        a[j] = ab ? Raw8<TM>::load(ab + (FULL || c < dim ? c : 0)) : Raw8<TM>::zero();
      }
    }
    madd = (one_plus || !mb) ? 1.0f : 0.0f;
    float s = 0.f;
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      if (FULL || (lane + 64 * j) * 8 < dim) {
        float v[8];
        x[j].cvt(v);
#pragma unroll
        for (int i = 0; i < 8; ++i) s += v[i];
      }
    }
    mean = wave_sum(s) / (float)dim;
    float q = 0.f;
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      if (FULL || (lane + 64 * j) * 8 < dim) {
        float v[8];
        x[j].cvt(v);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const float d = v[i] - mean;
          q += d * d;
        }
      }
    }
    rstd = 1.0f / __builtin_sqrtf(wave_sum(q) / (float)dim + eps);
  }

  // modulated output of chunk j (elements (lane + 64 j) * 8 .. + 8)
  __device__ __forceinline__ void out(int j, float (&o)[8]) const {
    float v[8], m8[8], a8[8];
    x[j].cvt(v);
    if constexpr (HOLD) {
      m[j].cvt(m8);
      a[j].cvt(a8);
    } else {  // (chunks past dim re-read chunk 0; their outputs are not stored)
      const int c0 = (lane_ + 64 * j) * 8, c = FULL || c0 < dim_ ? c0 : 0;
      (mp ? Raw8<TM>::load(mp + c) : Raw8<TM>::zero()).cvt(m8);
      (ap ? Raw8<TM>::load(ap + c) : Raw8<TM>::zero()).cvt(a8);
    }
    const float nm = -mean * rstd;
#pragma unroll
    for (int i = 0; i < 8; ++i)
      o[i] = __builtin_fmaf(__builtin_fmaf(v[i], rstd, nm), m8[i] + madd, a8[i]);
  }
};

// One wavefront per row; rows of batch b use mul / add + b * mod_stride (split > 0: rows below
// split are batch 0, the rest batch 1).
template <typename TX, typename TY, typename TM, int NV, bool FULL>
__global__ __launch_bounds__(256) void layernorm_modulate_kernel(
    const TX* __restrict__ x, int64_t ldx, TY* __restrict__ y, int64_t ldy, int64_t rows,
    int dim, const TM* __restrict__ mul, const TM* __restrict__ add, int64_t mod_stride,
    int64_t rows_per_batch, int64_t split, int one_plus, float eps) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int64_t b = split > 0 ? (row >= split ? 1 : 0) : row / rows_per_batch;
  LnRow<TX, TM, NV, FULL> r;
  r.load(x + row * ldx, dim, mul ? mul + b * mod_stride : nullptr,
         add ? add + b * mod_stride : nullptr, one_plus, eps, lane);
  TY* yr = y + row * ldy;
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int c = (lane + 64 * j) * 8;
    if (FULL || c < dim) {
      float o[8];
      r.out(j, o);
      V8<TY>::store(yr + c, o);
    }
  }
}

// layernorm_modulate rounded to bf16, then quantized per row to e4m3 (absmax / 448 scale): the
// output equals quantize_fp8_rowwise of layernorm_modulate's bf16 result. The rounded row is kept
// packed in registers between the absmax and the encoding.
template <typename TX, typename TM, int NV, bool FULL>
__global__ __launch_bounds__(256) void layernorm_modulate_fp8_kernel(
    const TX* __restrict__ x, int64_t ldx, uint8_t* __restrict__ q, int64_t ldq,
    float* __restrict__ scale, int64_t rows, int dim, const TM* __restrict__ mul,
    const TM* __restrict__ add, int64_t mod_stride, int64_t rows_per_batch, int64_t split,
    int one_plus, float eps) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int64_t b = split > 0 ? (row >= split ? 1 : 0) : row / rows_per_batch;
  LnRow<TX, TM, NV, FULL> r;
  r.load(x + row * ldx, dim, mul ? mul + b * mod_stride : nullptr,
         add ? add + b * mod_stride : nullptr, one_plus, eps, lane);
  u32x4 ob[NV];  // the bf16-rounded output, packed
  float amax = 0.f;
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    float o[8];
    r.out(j, o);
#pragma unroll
    for (int i = 0; i < 4; ++i) ob[j][i] = pack_bf16x2(o[2 * i], o[2 * i + 1]);
    if (FULL || (lane + 64 * j) * 8 < dim) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        amax = __builtin_fmaxf(amax, __builtin_fmaxf(__builtin_fabsf(bf16bits_to_f32(ob[j][i] & 0xffffu)),
                                                     __builtin_fabsf(bf16bits_to_f32(ob[j][i] >> 16))));
    }
  }
  amax = wave_max(amax);
  const float inv = rowwise_inv(amax);
  if (lane == 0) scale[row] = rowwise_scale(amax);
  uint8_t* qr = q + row * ldq;
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int c = (lane + 64 * j) * 8;
    if (FULL || c < dim) {
      float o[8];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        o[2 * i] = bf16bits_to_f32(ob[j][i] & 0xffffu);
        o[2 * i + 1] = bf16bits_to_f32(ob[j][i] >> 16);
      }
      *reinterpret_cast<u32x2*>(qr + c) = encode8_rowwise(o, inv);
    }
  }
}

// layernorm_modulate rounded to bf16, then quantized to MXFP8 in the GEMM's swizzled layout:
// the output equals quantize_mxfp8(swizzled) of layernorm_modulate's bf16 result, codes and
// E8M0 scales. dim is a multiple of 512 (whole swizzle tiles), so chunk j of lane L (columns
// (L + 64 j) * 8 .. + 8) is run L / 16 of block L % 16 of tile j: the four runs of a block sit in
// lanes b, b + 16, b + 32, b + 48 of one register, and the block's exponent maximum is two
// cross-lane steps. The codes go to the wave's LDS row at their swizzled bytes ((8 b + r) * 4 +
// run for element r of a run), then out to HBM in whole 16-byte pieces; the scales likewise.
template <typename TX, typename TM, int NV>
__global__ __launch_bounds__(256) void layernorm_modulate_mx_kernel(
    const TX* __restrict__ x, int64_t ldx, uint8_t* __restrict__ q, int64_t ldq,
    uint8_t* __restrict__ scale, int64_t ld_scale, int64_t rows, int dim,
    const TM* __restrict__ mul, const TM* __restrict__ add, int64_t mod_stride,
    int64_t rows_per_batch, int64_t split, int one_plus, float eps) {
  constexpr int ROW = NV * 512;  // codes of one row (dim == ROW)
  __shared__ __attribute__((aligned(16))) uint8_t stage[4][ROW + ROW / 32];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int64_t row = (int64_t)blockIdx.x * 4 + w;
  if (row >= rows) return;  // whole waves: the LDS rows are per wave, no barrier is needed
  const int64_t b = split > 0 ? (row >= split ? 1 : 0) : row / rows_per_batch;
  LnRow<TX, TM, NV, true> r;
  r.load(x + row * ldx, dim, mul ? mul + b * mod_stride : nullptr,
         add ? add + b * mod_stride : nullptr, one_plus, eps, lane);
  uint8_t* st = stage[w];
  const int run = lane >> 4, blk = lane & 15;
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    float o[8];
    r.out(j, o);
#pragma unroll
    for (int i = 0; i < 4; ++i) {  // the bf16 output, as layernorm_modulate stores it
      const uint32_t p = pack_bf16x2(o[2 * i], o[2 * i + 1]);
      o[2 * i] = bf16bits_to_f32(p & 0xffffu);
      o[2 * i + 1] = bf16bits_to_f32(p >> 16);
    }
    uint32_t emax = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t e = (__builtin_bit_cast(uint32_t, o[i]) >> 23) & 0xffu;
      emax = e > emax ? e : emax;
    }
    emax = max(emax, (uint32_t)__shfl_xor((int)emax, 16, kWave));
    emax = max(emax, (uint32_t)__shfl_xor((int)emax, 32, kWave));
    const int su = (int)emax - 7 < 0 ? 0 : (int)emax - 7;  // clamp(e_max - 7, 0, 255)
    const float m = __builtin_bit_cast(float, (uint32_t)(254 - su) << 23);  // 2^(127 - su)
    float c[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) c[i] = clamp448(__fmul_rn(o[i], m));
    const uint32_t lo = e4m3x4(c[0], c[1], c[2], c[3]), hi = e4m3x4(c[4], c[5], c[6], c[7]);
    uint8_t* tile = st + j * 512 + blk * 32 + run;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      tile[4 * i] = (uint8_t)(lo >> (8 * i));
      tile[4 * (4 + i)] = (uint8_t)(hi >> (8 * i));
    }
    if (run == 0) st[ROW + j * 16 + blk] = (uint8_t)su;
  }
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  uint8_t* qr = q + row * ldq;
#pragma unroll
  for (int i = lane; i < ROW / 16; i += 64)
    *reinterpret_cast<u32x4*>(qr + 16 * i) = *reinterpret_cast<const u32x4*>(st + 16 * i);
  if (lane < ROW / 512)
    *reinterpret_cast<u32x4*>(scale + row * ld_scale + 16 * lane) =
        *reinterpret_cast<const u32x4*>(st + ROW + 16 * lane);
}

// ------------------------------------------------------------------ RMSNorm (fp32 law)
template <typename T, typename TW, int NV>
__global__ __launch_bounds__(256) void rms_norm_kernel(const T* __restrict__ x, int64_t ldx,
                                                       T* __restrict__ y, int64_t ldy,
                                                       int64_t rows, int dim,
                                                       const TW* __restrict__ w, float eps) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const T* xr = x + row * ldx;
  float v[NV][8];
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int c = (lane + 64 * j) * 8;
    if (c < dim) {
      V8<T>::load(xr + c, v[j]);
#pragma unroll
      for (int i = 0; i < 8; ++i) s += v[j][i] * v[j][i];
    }
  }
  const float r = 1.0f / __builtin_sqrtf(wave_sum(s) / (float)dim + eps);
  T* yr = y + row * ldy;
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int c = (lane + 64 * j) * 8;
    if (c < dim) {
      float w8[8], o[8];
      if (w) {
        V8<TW>::load(w + c, w8);
      } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) w8[i] = 1.f;
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) o[i] = v[j][i] * r * w8[i];
      V8<T>::store(yr + c, o);
    }
  }
}

// ------------------------------------------------------------------ rotary helpers
// Rotates 8 consecutive head-dim elements starting at dim index d0 (even) in place.
// law 0 (fp32 interleaved, apply_rotary_emb_fp32): out[2i] = x[2i] c[2i] - x[2i+1] s[2i],
//                                                  out[2i+1] = x[2i+1] c[2i+1] + x[2i] s[2i+1]
// law 1 (stride-2, apply_rotary_emb): out[2i] = x[2i] c[2i] - x[2i+1] s[2i+1],
//                                     out[2i+1] = x[2i] s[2i+1] + x[2i+1] c[2i]
__device__ __forceinline__ void rope8(float* v, const float* cs, const float* sn, int law) {
  float c[8], s[8];
  *reinterpret_cast<f32x4*>(c) = *reinterpret_cast<const f32x4*>(cs);
  *reinterpret_cast<f32x4*>(c + 4) = *reinterpret_cast<const f32x4*>(cs + 4);
  *reinterpret_cast<f32x4*>(s) = *reinterpret_cast<const f32x4*>(sn);
  *reinterpret_cast<f32x4*>(s + 4) = *reinterpret_cast<const f32x4*>(sn + 4);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float a = v[2 * i], b = v[2 * i + 1];
    if (law == 0) {
      v[2 * i] = a * c[2 * i] - b * s[2 * i];
      v[2 * i + 1] = b * c[2 * i + 1] + a * s[2 * i + 1];
    } else {
      v[2 * i] = a * c[2 * i] - b * s[2 * i + 1];
      v[2 * i + 1] = a * s[2 * i + 1] + b * c[2 * i];
    }
  }
}

// ------------------------------------------------------------------ q/k RMSNorm across heads
// do_norm 2 with head_dim 128 and rows of NV * 512 values (Wan: 40 heads = 5120): one wavefront
// per row holds q and k as loaded (every load issued before the first use), one reduction
// each, then scales each 8-value chunk by rsqrt(mean + eps) and the norm weights, rotates it
// and stores it in place. (Chunk c of a lane: values (lane + 64 c) * 8 .. + 8.)
template <typename T, typename TW, int NV>
__global__ __launch_bounds__(256) void qk_rms_rows_kernel(
    T* __restrict__ buf, int64_t ld, int64_t rows, int64_t q_off, int64_t k_off,
    const TW* __restrict__ wq, const TW* __restrict__ wk, int64_t split,
    const TW* __restrict__ wq2, const TW* __restrict__ wk2, float eps,
    const float* __restrict__ cosb, const float* __restrict__ sinb, int64_t rope_rows,
    int law) {
  constexpr int HD = 128;
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const bool has[2] = {q_off >= 0, k_off >= 0};
  T* const base[2] = {buf + row * ld + (has[0] ? q_off : 0), buf + row * ld + (has[1] ? k_off : 0)};
  Raw8<T> x[2][NV];
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int j = 0; j < NV; ++j) x[t][j] = Raw8<T>::load(base[t] + (lane + 64 * j) * 8);
  float ss[2] = {0.f, 0.f};
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      float v[8];
      x[t][j].cvt(v);
#pragma unroll
      for (int i = 0; i < 8; ++i) ss[t] += v[i] * v[i];
    }
  ss[0] = wave_sum(ss[0]);
  ss[1] = wave_sum(ss[1]);
  const bool second = split > 0 && row >= split;  // rows past split: the second weights
  // every chunk of a lane sits at the same place in its head ((lane + 64 c) * 8 mod 128 =
  // lane * 8 mod 128), so the row's cos / sin values are loaded once for all of them
  float cs[8], sn[8];
  if (cosb) {
    const int64_t tr = (row % rope_rows) * HD + (lane * 8) % HD;
    *reinterpret_cast<f32x4*>(cs) = *reinterpret_cast<const f32x4*>(cosb + tr);
    *reinterpret_cast<f32x4*>(cs + 4) = *reinterpret_cast<const f32x4*>(cosb + tr + 4);
    *reinterpret_cast<f32x4*>(sn) = *reinterpret_cast<const f32x4*>(sinb + tr);
    *reinterpret_cast<f32x4*>(sn + 4) = *reinterpret_cast<const f32x4*>(sinb + tr + 4);
  }
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    if (!has[t]) continue;
    const float r = 1.0f / __builtin_sqrtf(ss[t] / (float)(NV * 512) + eps);
    const TW* w = t == 0 ? (second ? wq2 : wq) : (second ? wk2 : wk);
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      const int c = (lane + 64 * j) * 8;
      float v[8], w8[8];
      x[t][j].cvt(v);
      if (w) {
        Raw8<TW>::load(w + c).cvt(w8);
      } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) w8[i] = 1.f;
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) v[i] = v[i] * r * w8[i];
      if (cosb) rope8(v, cs, sn, law);
      V8<T>::store(base[t] + c, v);
    }
  }
}

// ------------------------------------------------------------------ q/k RMSNorm + RoPE
// One wavefront per row; LPH = lanes per head (head_dim / 8); a wave covers 64 / LPH heads
// per step. do_norm 1: per-head RMS, reduced over the LPH lanes of one head with xor shuffles,
// weight [head_dim]. do_norm 2: one RMS over all heads of the tensor (a first pass over the
// row, one wave reduction), weight [heads * head_dim].
template <typename T, typename TW, int LPH>
__global__ __launch_bounds__(256) void qk_norm_rope_kernel(
    T* __restrict__ buf, int64_t ld, int64_t rows, int heads, int64_t q_off, int64_t k_off,
    int do_norm, const TW* __restrict__ wq, const TW* __restrict__ wk, int64_t split,
    const TW* __restrict__ wq2, const TW* __restrict__ wk2, float eps,
    const float* __restrict__ cosb, const float* __restrict__ sinb, int64_t rope_rows,
    int law) {
  constexpr int HD = LPH * 8;
  constexpr int HPS = 64 / LPH;  // heads per step
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int sub = lane % LPH;  // which 8-wide slice of the head
  const int hl = lane / LPH;   // which head of the step
  const int d0 = sub * 8;
  const float* cr = cosb ? cosb + (row % rope_rows) * HD + d0 : nullptr;
  const float* sr = sinb ? sinb + (row % rope_rows) * HD + d0 : nullptr;
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const int64_t off = t == 0 ? q_off : k_off;
    if (off < 0) continue;
    const bool second = split > 0 && row >= split;  // rows past split: the second weights
    const TW* w = t == 0 ? (second ? wq2 : wq) : (second ? wk2 : wk);
    T* base = buf + row * ld + off;
    float r_row = 1.f;
    if (do_norm == 2) {
      float s = 0.f;
      for (int h0 = 0; h0 < heads; h0 += HPS) {
        const int h = h0 + hl;
        if (h < heads) {
          float v[8];
          V8<T>::load(base + (int64_t)h * HD + d0, v);
#pragma unroll
          for (int i = 0; i < 8; ++i) s += v[i] * v[i];
        }
      }
      r_row = 1.0f / __builtin_sqrtf(wave_sum(s) / (float)(heads * HD) + eps);
    }
    for (int h0 = 0; h0 < heads; h0 += HPS) {
      const int h = h0 + hl;
      if (h < heads) {
        T* p = base + (int64_t)h * HD + d0;
        float v[8];
        V8<T>::load(p, v);
        if (do_norm) {
          float r = r_row;
          if (do_norm == 1) {
            float s = 0.f;
#pragma unroll
            for (int i = 0; i < 8; ++i) s += v[i] * v[i];
#pragma unroll
            for (int o = LPH / 2; o > 0; o >>= 1) s += __shfl_xor(s, o, 64);
            r = 1.0f / __builtin_sqrtf(s / (float)HD + eps);
          }
          float w8[8];
          if (w) {
            V8<TW>::load(w + (do_norm == 2 ? (int64_t)h * HD : 0) + d0, w8);
          } else {
#pragma unroll
            for (int i = 0; i < 8; ++i) w8[i] = 1.f;
          }
#pragma unroll
          for (int i = 0; i < 8; ++i) v[i] = v[i] * r * w8[i];
        }
        if (cr) rope8(v, cr, sr, law);
        V8<T>::store(p, v);
      }
    }
  }
}

// The per-head forms (do_norm 0 / 1) with one wavefront per (row, q or k, group of 64 / LPH
// heads): a head's norm needs only its own LPH lanes, so the row's head groups run in parallel
// instead of one after another behind each load's latency.
template <typename T, typename TW, int LPH>
__global__ __launch_bounds__(256) void qk_norm_rope_heads_kernel(
    T* __restrict__ buf, int64_t ld, int64_t rows, int heads, int64_t q_off, int64_t k_off,
    int do_norm, const TW* __restrict__ wq, const TW* __restrict__ wk, int64_t split,
    const TW* __restrict__ wq2, const TW* __restrict__ wk2, float eps,
    const float* __restrict__ cosb, const float* __restrict__ sinb, int64_t rope_rows,
    int law) {
  constexpr int HD = LPH * 8;
  constexpr int HPS = 64 / LPH;  // heads per wavefront
  const int lane = threadIdx.x & 63;
  const int steps = (heads + HPS - 1) / HPS;
  const int64_t task = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int64_t rt = task / steps;
  const int step = (int)(task - rt * steps);
  const int64_t row = rt >> 1;
  const int t = (int)(rt & 1);
  if (row >= rows) return;
  const int64_t off = t == 0 ? q_off : k_off;
  const int h = step * HPS + lane / LPH;
  if (off < 0 || h >= heads) return;
  const int d0 = (lane % LPH) * 8;
  const bool second = split > 0 && row >= split;  // rows past split: the second weights
  const TW* w = t == 0 ? (second ? wq2 : wq) : (second ? wk2 : wk);
  T* p = buf + row * ld + off + (int64_t)h * HD + d0;
  float v[8];
  V8<T>::load(p, v);
  if (do_norm) {
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) s += v[i] * v[i];
#pragma unroll
    for (int o = LPH / 2; o > 0; o >>= 1) s += __shfl_xor(s, o, 64);
    const float r = 1.0f / __builtin_sqrtf(s / (float)HD + eps);
    float w8[8];
    if (w) {
      V8<TW>::load(w + d0, w8);
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) w8[i] = 1.f;
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = v[i] * r * w8[i];
  }
  if (cosb) {
    const int64_t rr = row % rope_rows;
    rope8(v, cosb + rr * HD + d0, sinb + rr * HD + d0, law);
  }
  V8<T>::store(p, v);
}

// ------------------------------------------------------------------ RoPE, out of place
template <typename T, int LPH>
__global__ __launch_bounds__(256) void rope_kernel(const T* __restrict__ x, T* __restrict__ y,
                                                   int64_t outer, int64_t seq,
                                                   int64_t xos, int64_t xss, int64_t yos,
                                                   int64_t yss, const float* __restrict__ cosb,
                                                   const float* __restrict__ sinb,
                                                   int64_t rope_rows, int law) {
  constexpr int HD = LPH * 8;
  constexpr int RPW = 64 / LPH;  // rows per wave
  const int lane = threadIdx.x & 63;
  const int64_t total = outer * seq;
  const int64_t r = ((int64_t)blockIdx.x * 4 + (threadIdx.x >> 6)) * RPW + lane / LPH;
  if (r >= total) return;
  const int64_t o = r / seq, s = r % seq;
  const int d0 = (lane % LPH) * 8;
  float v[8];
  V8<T>::load(x + o * xos + s * xss + d0, v);
  rope8(v, cosb + (s % rope_rows) * HD + d0, sinb + (s % rope_rows) * HD + d0, law);
  V8<T>::store(y + o * yos + s * yss + d0, v);
}

// ------------------------------------------------------------------ GELU-tanh
template <typename T>
__global__ __launch_bounds__(256) void gelu_kernel(const T* __restrict__ x, T* __restrict__ y,
                                                   int64_t n) {
  const int64_t nv = n / 8;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < nv;
       i += (int64_t)gridDim.x * 256) {
    float v[8];
    V8<T>::load(x + i * 8, v);
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = gelu_tanh(v[j]);
    V8<T>::store(y + i * 8, v);
  }
  for (int64_t i = nv * 8 + (int64_t)blockIdx.x * 256 + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * 256)
    Elt<T>::store(y + i, gelu_tanh(Elt<T>::load(x + i)));
}

// ------------------------------------------------------------------ gated GELU
// y[r, c] = gelu_tanh(x[r, c]) * x[r, f + c]: the T5 / UMT5 gated FFN's act(wi_0 h) * wi_1 h,
// both projections computed by one GEMM into the two halves of x's rows.
template <typename T>
__global__ __launch_bounds__(256) void gated_gelu_kernel(const T* __restrict__ x, int64_t ldx,
                                                         T* __restrict__ y, int64_t ldy,
                                                         int64_t rows, int64_t f) {
  const int64_t nvr = f / 8;
  const int64_t nv = rows * nvr;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < nv;
       i += (int64_t)gridDim.x * 256) {
    const int64_t r = i / nvr, c = (i % nvr) * 8;
    float g[8], l[8];
    V8<T>::load(x + r * ldx + c, g);
    V8<T>::load(x + r * ldx + f + c, l);
#pragma unroll
    for (int j = 0; j < 8; ++j) g[j] = gelu_tanh(g[j]) * l[j];
    V8<T>::store(y + r * ldy + c, g);
  }
}

// ------------------------------------------------------------------ embedding rows
// out[i, :] = table[ids[i], :] as raw 16-byte pieces (any element type); an id outside
// [0, table_rows) gives a zero row instead of a read past the table.
__global__ __launch_bounds__(256) void embedding_kernel(const int64_t* __restrict__ ids,
                                                        int64_t n, const uint8_t* __restrict__ table,
                                                        int64_t table_rows, int64_t ldt,
                                                        uint8_t* __restrict__ out, int64_t ldo,
                                                        int64_t row_bytes) {
  const int64_t nvr = row_bytes / 16;
  const int64_t nv = n * nvr;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < nv;
       i += (int64_t)gridDim.x * 256) {
    const int64_t r = i / nvr, c = (i % nvr) * 16;
    const int64_t id = ids[r];
    u32x4 v = {0u, 0u, 0u, 0u};
    if (id >= 0 && id < table_rows) v = *reinterpret_cast<const u32x4*>(table + id * ldt + c);
    *reinterpret_cast<u32x4*>(out + r * ldo + c) = v;
  }
}

// ------------------------------------------------------------------ relative position bias
// out[b, h, q, k] = table[bucket[k - q + seq_q - 1], h] (fp32), or the lowest float where
// key k of batch element b is padding (key_keep[b, k] == 0): the T5 bias plus the additive
// padding mask. A bucket outside [0, num_buckets) gives NaN rather than a read past the table.
template <typename TT>
__global__ __launch_bounds__(256) void relative_bias_kernel(
    const int32_t* __restrict__ bucket, int num_buckets, const TT* __restrict__ table,
    int64_t heads, int64_t batch, int64_t seq_q, int64_t seq_k,
    const uint8_t* __restrict__ keep, int64_t keep_stride, float* __restrict__ out) {
  const int64_t total = batch * heads * seq_q * seq_k;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * 256) {
    const int64_t k = i % seq_k;
    const int64_t q = (i / seq_k) % seq_q;
    const int64_t bh = i / (seq_k * seq_q);
    const int64_t h = bh % heads, b = bh / heads;
    float v;
    if (keep && keep[b * keep_stride + k] == 0) {
      v = -FLT_MAX;
    } else {
      const int bk = bucket[k - q + seq_q - 1];
      v = (bk >= 0 && bk < num_buckets) ? Elt<TT>::load(table + (int64_t)bk * heads + h)
                                        : __builtin_nanf("");
    }
    out[i] = v;
  }
}

// ------------------------------------------------------------------ gate * x + residual
template <typename T, typename TG>
__global__ __launch_bounds__(256) void gate_residual_kernel(
    const T* __restrict__ res, const T* __restrict__ x, const TG* __restrict__ gate,
    T* __restrict__ y, int64_t rows, int64_t dim, int64_t gate_stride, int64_t rpb) {
  const int64_t nvr = dim / 8;
  const int64_t nv = rows * nvr;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < nv;
       i += (int64_t)gridDim.x * 256) {
    const int64_t r = i / nvr, c = (i % nvr) * 8;
    float a[8], b[8], g[8];
    V8<T>::load(res + r * dim + c, a);
    V8<T>::load(x + r * dim + c, b);
    V8<TG>::load(gate + (r / rpb) * gate_stride + c, g);
#pragma unroll
    for (int j = 0; j < 8; ++j) a[j] = a[j] + g[j] * b[j];
    V8<T>::store(y + r * dim + c, a);
  }
}

// ------------------------------------------------------------------ small-M GEMV
// One wavefront per output column n; the activated input rows sit in LDS as fp32 (rounded to
// the input dtype first, as the reference's `silu(emb)` tensor is). W is read once, 16 bytes
// per lane per step, so the kernel runs at HBM speed. M is a compile-time bound on the rows;
// rows m..M-1 of the LDS stage are zero and never stored.
template <typename T, int M>
__global__ __launch_bounds__(256) void gemv_kernel(const T* __restrict__ x, int m, int k,
                                                   int64_t ldx, const bf16* __restrict__ w,
                                                   int64_t ldw, int64_t n,
                                                   const T* __restrict__ bias,
                                                   T* __restrict__ y, int64_t ldy, int act) {
  extern __shared__ float xs[];  // [M][k]
  for (int i = threadIdx.x; i < M * k; i += 256) {
    const int r = i / k, kk = i - r * k;
    float v = 0.f;
    if (r < m) {
      v = Elt<T>::load(x + r * ldx + kk);
      if (act == 1) {
        T t;
        Elt<T>::store(&t, silu(v));
        v = Elt<T>::load(&t);
      }
    }
    xs[i] = v;
  }
  __syncthreads();
  const int lane = threadIdx.x & 63;
  // Two columns per wave and 3072-wide groups of six 1 KB loads per column, unguarded: twelve
  // loads in flight per wave before the first multiply; the k % 3072 tail is guarded.
  constexpr int U = 6, CP = 2;
  const int kfull = k - k % (U * 512);
  const int64_t step = (int64_t)gridDim.x * 4 * CP;
  for (int64_t c0 = ((int64_t)blockIdx.x * 4 + (threadIdx.x >> 6)) * CP; c0 < n; c0 += step) {
    const bf16* wr[CP];
#pragma unroll
    for (int p = 0; p < CP; ++p) wr[p] = w + (c0 + p < n ? c0 + p : n - 1) * ldw + lane * 8;
    float acc[CP][M];
#pragma unroll
    for (int p = 0; p < CP; ++p)
#pragma unroll
      for (int r = 0; r < M; ++r) acc[p][r] = 0.f;
    auto fma8 = [&](const u32x4& wv, int c, float* a) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float w0 = bf16bits_to_f32(wv[i] & 0xffffu);
        const float w1 = bf16bits_to_f32(wv[i] >> 16);
#pragma unroll
        for (int r = 0; r < M; ++r)
          a[r] += w0 * xs[r * k + c + 2 * i] + w1 * xs[r * k + c + 2 * i + 1];
      }
    };
    for (int g = 0; g < kfull; g += U * 512) {
      u32x4 wv[CP][U];
#pragma unroll
      for (int p = 0; p < CP; ++p)
#pragma unroll
        for (int u = 0; u < U; ++u)
          wv[p][u] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(wr[p] + g + u * 512));
#pragma unroll
      for (int p = 0; p < CP; ++p)
#pragma unroll
        for (int u = 0; u < U; ++u) fma8(wv[p][u], g + u * 512 + lane * 8, acc[p]);
    }
    for (int c = kfull; c + lane * 8 < k; c += 512) {
#pragma unroll
      for (int p = 0; p < CP; ++p)
        fma8(*reinterpret_cast<const u32x4*>(wr[p] + c), c + lane * 8, acc[p]);
    }
#pragma unroll
    for (int p = 0; p < CP; ++p) {
#pragma unroll
      for (int r = 0; r < M; ++r) {
        const float t = wave_sum(acc[p][r]);
        if (lane == 0 && r < m && c0 + p < n) {
          const float bv = bias ? Elt<T>::load(bias + c0 + p) : 0.f;
          Elt<T>::store(y + r * ldy + c0 + p, t + bv);
        }
      }
    }
  }
}

// ------------------------------------------------------------------ timestep embedding
template <typename T>
__global__ void timestep_embedding_kernel(const float* __restrict__ t, T* __restrict__ y,
                                          int64_t m, int dim, int flip, float shift,
                                          float scale, float neg_log_period) {
  const int half = dim / 2;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < m * dim;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = i / dim;
    const int c = (int)(i % dim);
    float v = 0.f;
    if (c < 2 * half) {
      const int j = c < half ? c : c - half;
      // exponent = -ln(max_period) * j / (half - shift) in fp32, emb = exp(exponent), as torch
      const float e = (neg_log_period * (float)j) / ((float)half - shift);
      const float arg = scale * (t[r] * expf(e));
      const bool first = c < half;
      // unflipped order is [sin, cos]; flip_sin_to_cos swaps the halves
      const bool is_sin = flip ? !first : first;
      v = is_sin ? sinf(arg) : cosf(arg);
    }
    Elt<T>::store(y + i, v);
  }
}

}  // namespace dlt

using namespace dlt;

// ======================================================================== dispatch helpers
#define DLT_DISPATCH_FLOAT(dt, T, ...)                                          \
  switch (dt) {                                                                \
    case DIFFLET_BF16: { typedef bf16 T; __VA_ARGS__; break; }                 \
    case DIFFLET_F16: { typedef f16 T; __VA_ARGS__; break; }                   \
    case DIFFLET_F32: { typedef float T; __VA_ARGS__; break; }                 \
    default: dlt_set_error("unsupported dtype %d", (int)(dt)); return DIFFLET_EINVAL; \
  }

static bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

template <typename TX, typename TY, typename TM>
static int launch_ln(const void* x, int64_t ldx, void* y, int64_t ldy, int64_t rows,
                     int64_t dim, const void* mul, const void* add, int64_t mod_stride,
                     int64_t rpb, int64_t split, int one_plus, float eps, hipStream_t s) {
  const int nv = (int)((dim + 511) / 512);
  dim3 grid((unsigned)((rows + 3) / 4)), block(256);
#define DLT_LN1(NV, FULL)                                                                     \
  hipLaunchKernelGGL((layernorm_modulate_kernel<TX, TY, TM, NV, FULL>), grid, block, 0, s,  \
                     (const TX*)x, ldx, (TY*)y, ldy, rows, (int)dim, (const TM*)mul,         \
                     (const TM*)add, mod_stride, rpb, split, one_plus, eps)
#define DLT_LN(NV)                          \
  do {                                      \
    if (dim == 512 * (NV)) DLT_LN1(NV, true); \
    else DLT_LN1(NV, false);                \
  } while (0)
  if (nv <= 2) DLT_LN(2);
  else if (nv <= 4) DLT_LN(4);
  else if (nv <= 6) DLT_LN(6);
  else if (nv <= 8) DLT_LN(8);
  else if (nv <= 10) DLT_LN(10);
  else if (nv <= 16) DLT_LN(16);
  else { dlt_set_error("layernorm: dim %lld exceeds 8192", (long long)dim); return DIFFLET_EUNSUPPORTED; }
#undef DLT_LN
#undef DLT_LN1
  return dlt_check_launch("layernorm_modulate");
}

extern "C" int difflet_rocm_layernorm_modulate(const void* x, int64_t ldx, void* y,
                                               int64_t ldy, int dtype, int out_dtype,
                                               int64_t rows, int64_t dim, const void* mul,
                                               const void* add, int mod_dtype,
                                               int64_t mod_stride, int64_t rows_per_batch,
                                               int64_t split, int one_plus, float eps,
                                               difflet_stream_t stream) {
  DLT_REQUIRE(x && y, DIFFLET_EINVAL, "layernorm: null pointer");
  DLT_REQUIRE(split >= 0, DIFFLET_EINVAL, "layernorm: split must be >= 0");
  DLT_REQUIRE(rows >= 0 && dim > 0 && dim % 8 == 0, DIFFLET_EINVAL,
              "layernorm: dim %lld must be a positive multiple of 8", (long long)dim);
  DLT_REQUIRE(ldx % 8 == 0 && ldy % 8 == 0 && (mod_stride % 8 == 0 || (!mul && !add)),
              DIFFLET_EINVAL, "layernorm: strides must be multiples of 8 elements");
  DLT_REQUIRE(aligned16(x) && aligned16(y) && (!mul || aligned16(mul)) &&
                  (!add || aligned16(add)),
              DIFFLET_EINVAL, "layernorm: pointers must be 16-byte aligned");
  if (rows == 0) return DIFFLET_OK;
  if (rows_per_batch <= 0) rows_per_batch = rows;
  hipStream_t s = (hipStream_t)stream;
  DLT_DISPATCH_FLOAT(dtype, TX,
    DLT_DISPATCH_FLOAT(out_dtype, TY,
      DLT_DISPATCH_FLOAT(mod_dtype, TM,
        return launch_ln<TX, TY, TM>(x, ldx, y, ldy, rows, dim, mul, add, mod_stride,
                                     rows_per_batch, split, one_plus, eps, s))));
  return DIFFLET_OK;
}

template <typename TX, typename TM>
static int launch_ln_fp8(const void* x, int64_t ldx, uint8_t* q, int64_t ldq, float* scale,
                         int64_t rows, int64_t dim, const void* mul, const void* add,
                         int64_t mod_stride, int64_t rpb, int64_t split, int one_plus,
                         float eps, hipStream_t s) {
  const int nv = (int)((dim + 511) / 512);
  dim3 grid((unsigned)((rows + 3) / 4)), block(256);
#define DLT_LNQ1(NV, FULL)                                                                    \
  hipLaunchKernelGGL((layernorm_modulate_fp8_kernel<TX, TM, NV, FULL>), grid, block, 0, s,  \
                     (const TX*)x, ldx, q, ldq, scale, rows, (int)dim, (const TM*)mul,        \
                     (const TM*)add, mod_stride, rpb, split, one_plus, eps)
#define DLT_LNQ(NV)                          \
  do {                                       \
    if (dim == 512 * (NV)) DLT_LNQ1(NV, true); \
    else DLT_LNQ1(NV, false);                \
  } while (0)
  if (nv <= 2) DLT_LNQ(2);
  else if (nv <= 4) DLT_LNQ(4);
  else if (nv <= 6) DLT_LNQ(6);
  else if (nv <= 8) DLT_LNQ(8);
  else if (nv <= 10) DLT_LNQ(10);
  else if (nv <= 16) DLT_LNQ(16);
  else { dlt_set_error("layernorm_modulate_fp8: dim %lld exceeds 8192", (long long)dim); return DIFFLET_EUNSUPPORTED; }
#undef DLT_LNQ
#undef DLT_LNQ1
  return dlt_check_launch("layernorm_modulate_fp8");
}

extern "C" int difflet_rocm_layernorm_modulate_fp8(const void* x, int64_t ldx, uint8_t* q,
                                                   int64_t ldq, float* scale, int dtype,
                                                   int64_t rows, int64_t dim, const void* mul,
                                                   const void* add, int mod_dtype,
                                                   int64_t mod_stride, int64_t rows_per_batch,
                                                   int64_t split, int one_plus, float eps,
                                                   difflet_stream_t stream) {
  DLT_REQUIRE(x && q && scale, DIFFLET_EINVAL, "layernorm_modulate_fp8: null pointer");
  DLT_REQUIRE(split >= 0, DIFFLET_EINVAL, "layernorm_modulate_fp8: split must be >= 0");
  DLT_REQUIRE(rows >= 0 && dim > 0 && dim % 8 == 0, DIFFLET_EINVAL,
              "layernorm_modulate_fp8: dim %lld must be a positive multiple of 8",
              (long long)dim);
  DLT_REQUIRE(ldx % 8 == 0 && ldq % 8 == 0 && (mod_stride % 8 == 0 || (!mul && !add)),
              DIFFLET_EINVAL, "layernorm_modulate_fp8: strides must be multiples of 8 elements");
  DLT_REQUIRE(aligned16(x) && ((uintptr_t)q & 7) == 0 && (!mul || aligned16(mul)) &&
                  (!add || aligned16(add)),
              DIFFLET_EINVAL, "layernorm_modulate_fp8: misaligned pointers");
  if (rows == 0) return DIFFLET_OK;
  if (rows_per_batch <= 0) rows_per_batch = rows;
  hipStream_t s = (hipStream_t)stream;
  DLT_DISPATCH_FLOAT(dtype, TX,
    DLT_DISPATCH_FLOAT(mod_dtype, TM,
      return launch_ln_fp8<TX, TM>(x, ldx, q, ldq, scale, rows, dim, mul, add, mod_stride,
                                   rows_per_batch, split, one_plus, eps, s)));
  return DIFFLET_OK;
}

template <typename TM>
static int launch_ln_mx(const void* x, int64_t ldx, uint8_t* q, int64_t ldq, uint8_t* scale,
                        int64_t ld_scale, int64_t rows, int64_t dim, const void* mul,
                        const void* add, int64_t mod_stride, int64_t rpb, int64_t split,
                        int one_plus, float eps, hipStream_t s) {
  dim3 grid((unsigned)((rows + 3) / 4)), block(256);
#define DLT_LNMX(NV)                                                                          \
  case NV:                                                                                     \
    hipLaunchKernelGGL((layernorm_modulate_mx_kernel<bf16, TM, NV>), grid, block, 0, s,       \
                       (const bf16*)x, ldx, q, ldq, scale, ld_scale, rows, (int)dim,          \
                       (const TM*)mul, (const TM*)add, mod_stride, rpb, split, one_plus, eps); \
    break;
  switch ((int)(dim / 512)) {
    DLT_LNMX(1) DLT_LNMX(2) DLT_LNMX(3) DLT_LNMX(4) DLT_LNMX(5) DLT_LNMX(6) DLT_LNMX(7)
    DLT_LNMX(8) DLT_LNMX(9) DLT_LNMX(10) DLT_LNMX(11) DLT_LNMX(12) DLT_LNMX(13) DLT_LNMX(14)
    DLT_LNMX(15) DLT_LNMX(16)
    default:
      dlt_set_error("layernorm_modulate_mx: dim %lld exceeds 8192", (long long)dim);
      return DIFFLET_EUNSUPPORTED;
  }
#undef DLT_LNMX
  return dlt_check_launch("layernorm_modulate_mx");
}

extern "C" int difflet_rocm_layernorm_modulate_mx(const void* x, int64_t ldx, uint8_t* q,
                                                  int64_t ldq, uint8_t* scale, int64_t ld_scale,
                                                  int dtype, int64_t rows, int64_t dim,
                                                  const void* mul, const void* add,
                                                  int mod_dtype, int64_t mod_stride,
                                                  int64_t rows_per_batch, int64_t split,
                                                  int one_plus, float eps,
                                                  difflet_stream_t stream) {
  DLT_REQUIRE(x && q && scale, DIFFLET_EINVAL, "layernorm_modulate_mx: null pointer");
  DLT_REQUIRE(dtype == DIFFLET_BF16, DIFFLET_EUNSUPPORTED,
              "layernorm_modulate_mx: x must be bf16");
  DLT_REQUIRE(mod_dtype == DIFFLET_BF16 || mod_dtype == DIFFLET_F32, DIFFLET_EUNSUPPORTED,
              "layernorm_modulate_mx: modulation vectors must be bf16 or fp32");
  DLT_REQUIRE(split >= 0, DIFFLET_EINVAL, "layernorm_modulate_mx: split must be >= 0");
  DLT_REQUIRE(rows >= 0 && dim > 0 && dim % 512 == 0, DIFFLET_EINVAL,
              "layernorm_modulate_mx: dim %lld must be a positive multiple of 512 (whole "
              "swizzle tiles)", (long long)dim);
  DLT_REQUIRE(ldx % 8 == 0 && ldq % 16 == 0 && ld_scale % 16 == 0 &&
                  (mod_stride % 8 == 0 || (!mul && !add)),
              DIFFLET_EINVAL,
              "layernorm_modulate_mx: ldx and mod_stride must be multiples of 8 elements, "
              "ldq and ld_scale multiples of 16 bytes");
  DLT_REQUIRE(aligned16(x) && aligned16(q) && aligned16(scale) && (!mul || aligned16(mul)) &&
                  (!add || aligned16(add)),
              DIFFLET_EINVAL, "layernorm_modulate_mx: pointers must be 16-byte aligned");
  if (rows == 0) return DIFFLET_OK;
  if (rows_per_batch <= 0) rows_per_batch = rows;
  hipStream_t s = (hipStream_t)stream;
  if (mod_dtype == DIFFLET_BF16)
    return launch_ln_mx<bf16>(x, ldx, q, ldq, scale, ld_scale, rows, dim, mul, add, mod_stride,
                              rows_per_batch, split, one_plus, eps, s);
  return launch_ln_mx<float>(x, ldx, q, ldq, scale, ld_scale, rows, dim, mul, add, mod_stride,
                             rows_per_batch, split, one_plus, eps, s);
}

template <typename T, typename TW>
static int launch_rms(const void* x, int64_t ldx, void* y, int64_t ldy, int64_t rows,
                      int64_t dim, const void* w, float eps, hipStream_t s) {
  const int nv = (int)((dim + 511) / 512);
  dim3 grid((unsigned)((rows + 3) / 4)), block(256);
#define DLT_RMS(NV)                                                                         \
  hipLaunchKernelGGL((rms_norm_kernel<T, TW, NV>), grid, block, 0, s, (const T*)x, ldx,     \
                     (T*)y, ldy, rows, (int)dim, (const TW*)w, eps)
  if (nv <= 1) DLT_RMS(1);
  else if (nv <= 2) DLT_RMS(2);
  else if (nv <= 4) DLT_RMS(4);
  else if (nv <= 8) DLT_RMS(8);
  else if (nv <= 10) DLT_RMS(10);
  else if (nv <= 16) DLT_RMS(16);
  else { dlt_set_error("rms_norm: dim %lld exceeds 8192", (long long)dim); return DIFFLET_EUNSUPPORTED; }
#undef DLT_RMS
  return dlt_check_launch("rms_norm");
}

extern "C" int difflet_rocm_rms_norm(const void* x, int64_t ldx, void* y, int64_t ldy,
                                     int dtype, int64_t rows, int64_t dim, const void* weight,
                                     int wdtype, float eps, difflet_stream_t stream) {
  DLT_REQUIRE(x && y, DIFFLET_EINVAL, "rms_norm: null pointer");
  DLT_REQUIRE(rows >= 0 && dim > 0 && dim % 8 == 0 && ldx % 8 == 0 && ldy % 8 == 0,
              DIFFLET_EINVAL, "rms_norm: dim and strides must be multiples of 8");
  DLT_REQUIRE(aligned16(x) && aligned16(y) && (!weight || aligned16(weight)), DIFFLET_EINVAL,
              "rms_norm: pointers must be 16-byte aligned");
  if (rows == 0) return DIFFLET_OK;
  hipStream_t s = (hipStream_t)stream;
  DLT_DISPATCH_FLOAT(dtype, T,
    DLT_DISPATCH_FLOAT(wdtype, TW,
      return launch_rms<T, TW>(x, ldx, y, ldy, rows, dim, weight, eps, s)));
  return DIFFLET_OK;
}

template <typename T, typename TW>
static int launch_qk(void* buf, int64_t ld, int64_t rows, int64_t heads, int64_t hd,
                     int64_t q_off, int64_t k_off, int do_norm, const void* wq,
                     const void* wk, int64_t split, const void* wq2, const void* wk2,
                     float eps, const float* c, const float* sn, int64_t rope_rows, int law,
                     hipStream_t s) {
  dim3 grid((unsigned)((rows + 3) / 4)), block(256);
#define DLT_QKR(NV)                                                                          \
  hipLaunchKernelGGL((qk_rms_rows_kernel<T, TW, NV>), grid, block, 0, s, (T*)buf, ld, rows,   \
                     q_off, k_off, (const TW*)wq, (const TW*)wk, split, (const TW*)wq2,       \
                     (const TW*)wk2, eps, c, sn, rope_rows, law)
  if (do_norm == 2 && hd == 128) {  // across heads: whole rows in registers when they fit
    switch (heads * 128) {
      case 2048: DLT_QKR(4); return dlt_check_launch("qk_norm_rope");
      case 3072: DLT_QKR(6); return dlt_check_launch("qk_norm_rope");
      case 4096: DLT_QKR(8); return dlt_check_launch("qk_norm_rope");
      case 5120: DLT_QKR(10); return dlt_check_launch("qk_norm_rope");
      case 6144: DLT_QKR(12); return dlt_check_launch("qk_norm_rope");
      default: break;
    }
  }
#undef DLT_QKR
#define DLT_QK(LPH)                                                                        \
  if (do_norm != 2) {                                                                      \
    const int64_t tasks = rows * 2 * ((heads + 64 / (LPH) - 1) / (64 / (LPH)));            \
    hipLaunchKernelGGL((qk_norm_rope_heads_kernel<T, TW, LPH>), dim3((unsigned)((tasks + 3) / 4)), \
                       block, 0, s, (T*)buf, ld, rows, (int)heads, q_off, k_off, do_norm,  \
                       (const TW*)wq, (const TW*)wk, split, (const TW*)wq2, (const TW*)wk2, \
                       eps, c, sn, rope_rows, law);                                        \
  } else                                                                                   \
  hipLaunchKernelGGL((qk_norm_rope_kernel<T, TW, LPH>), grid, block, 0, s, (T*)buf, ld,    \
                     rows, (int)heads, q_off, k_off, do_norm, (const TW*)wq,                \
                     (const TW*)wk, split, (const TW*)wq2, (const TW*)wk2, eps, c, sn,       \
                     rope_rows, law)
  switch (hd) {
    case 32: DLT_QK(4); break;
    case 64: DLT_QK(8); break;
    case 128: DLT_QK(16); break;
    case 256: DLT_QK(32); break;
    default: dlt_set_error("qk_norm_rope: head_dim %lld not in {32,64,128,256}", (long long)hd);
      return DIFFLET_EUNSUPPORTED;
  }
#undef DLT_QK
  return dlt_check_launch("qk_norm_rope");
}

extern "C" int difflet_rocm_qk_norm_rope(void* buf, int64_t ld, int dtype, int64_t rows,
                                         int64_t heads, int64_t head_dim, int64_t q_off,
                                         int64_t k_off, int do_norm, const void* wq,
                                         const void* wk, int64_t split, const void* wq2,
                                         const void* wk2, int wdtype, float eps,
                                         const float* cos, const float* sin,
                                         int64_t rope_rows, int law,
                                         difflet_stream_t stream) {
  DLT_REQUIRE(buf, DIFFLET_EINVAL, "qk_norm_rope: null buffer");
  DLT_REQUIRE(rows >= 0 && heads > 0 && ld % 8 == 0 && (q_off < 0 || q_off % 8 == 0) &&
                  (k_off < 0 || k_off % 8 == 0),
              DIFFLET_EINVAL, "qk_norm_rope: strides and offsets must be multiples of 8");
  DLT_REQUIRE(!cos == !sin, DIFFLET_EINVAL, "qk_norm_rope: cos and sin go together");
  DLT_REQUIRE(!cos || rope_rows > 0, DIFFLET_EINVAL, "qk_norm_rope: rope_rows must be > 0");
  DLT_REQUIRE(law == 0 || law == 1, DIFFLET_EINVAL, "qk_norm_rope: law must be 0 or 1");
  DLT_REQUIRE(do_norm >= 0 && do_norm <= 2, DIFFLET_EINVAL, "qk_norm_rope: do_norm must be 0, 1 or 2");
  DLT_REQUIRE(split >= 0, DIFFLET_EINVAL, "qk_norm_rope: split must be >= 0");
  if (split == 0 || split >= rows) {  // one segment: the second weights are not read
    split = 0;
    wq2 = wq;
    wk2 = wk;
  }
  DLT_REQUIRE(aligned16(buf) && (!cos || (aligned16(cos) && aligned16(sin))), DIFFLET_EINVAL,
              "qk_norm_rope: pointers must be 16-byte aligned");
  if (rows == 0) return DIFFLET_OK;
  hipStream_t s = (hipStream_t)stream;
  DLT_DISPATCH_FLOAT(dtype, T,
    DLT_DISPATCH_FLOAT(wdtype, TW,
      return launch_qk<T, TW>(buf, ld, rows, heads, head_dim, q_off, k_off, do_norm, wq, wk,
                              split, wq2, wk2, eps, cos, sin, rope_rows, law, s)));
  return DIFFLET_OK;
}

template <typename T>
static int launch_rope(const void* x, void* y, int64_t outer, int64_t seq, int64_t head_dim,
                       int64_t xos, int64_t xss, int64_t yos, int64_t yss, const float* cos,
                       const float* sin, int64_t rope_rows, int law, hipStream_t s) {
  const int64_t total = outer * seq;
  int lph;
  switch (head_dim) {
    case 32: lph = 4; break;
    case 64: lph = 8; break;
    case 128: lph = 16; break;
    case 256: lph = 32; break;
    default:
      dlt_set_error("rope: head_dim %lld not in {32,64,128,256}", (long long)head_dim);
      return DIFFLET_EUNSUPPORTED;
  }
  const int64_t rows_per_block = 4 * (64 / lph);
  dim3 grid((unsigned)((total + rows_per_block - 1) / rows_per_block)), block(256);
#define DLT_ROPE(LPH)                                                                         \
  hipLaunchKernelGGL((rope_kernel<T, LPH>), grid, block, 0, s, (const T*)x, (T*)y, outer, seq, \
                     xos, xss, yos, yss, cos, sin, rope_rows, law)
  if (lph == 4) DLT_ROPE(4);
  else if (lph == 8) DLT_ROPE(8);
  else if (lph == 16) DLT_ROPE(16);
  else DLT_ROPE(32);
#undef DLT_ROPE
  return dlt_check_launch("rope");
}

extern "C" int difflet_rocm_rope(const void* x, void* y, int dtype, int64_t outer,
                                 int64_t seq, int64_t head_dim, int64_t xos, int64_t xss,
                                 int64_t yos, int64_t yss, const float* cos, const float* sin,
                                 int64_t rope_rows, int law, difflet_stream_t stream) {
  DLT_REQUIRE(x && y && cos && sin, DIFFLET_EINVAL, "rope: null pointer");
  DLT_REQUIRE(outer >= 0 && seq >= 0 && rope_rows > 0 && (law == 0 || law == 1),
              DIFFLET_EINVAL, "rope: bad shape or law");
  DLT_REQUIRE(xos % 8 == 0 && xss % 8 == 0 && yos % 8 == 0 && yss % 8 == 0 && aligned16(x) &&
                  aligned16(y) && aligned16(cos) && aligned16(sin),
              DIFFLET_EINVAL, "rope: strides must be multiples of 8 and pointers aligned");
  if (outer * seq == 0) return DIFFLET_OK;
  hipStream_t s = (hipStream_t)stream;
  DLT_DISPATCH_FLOAT(dtype, T,
    return launch_rope<T>(x, y, outer, seq, head_dim, xos, xss, yos, yss, cos, sin, rope_rows,
                          law, s));
  return DIFFLET_OK;
}

extern "C" int difflet_rocm_gelu_tanh(const void* x, void* y, int dtype, int64_t n,
                                      difflet_stream_t stream) {
  DLT_REQUIRE(x && y && n >= 0, DIFFLET_EINVAL, "gelu: bad arguments");
  DLT_REQUIRE(aligned16(x) && aligned16(y), DIFFLET_EINVAL, "gelu: pointers must be aligned");
  if (n == 0) return DIFFLET_OK;
  hipStream_t s = (hipStream_t)stream;
  int64_t blocks = (n / 8 + 255) / 256;
  if (blocks < 1) blocks = 1;
  if (blocks > 65536) blocks = 65536;
  DLT_DISPATCH_FLOAT(dtype, T,
    hipLaunchKernelGGL((gelu_kernel<T>), dim3((unsigned)blocks), dim3(256), 0, s,
                       (const T*)x, (T*)y, n));
  return dlt_check_launch("gelu_tanh");
}

extern "C" int difflet_rocm_gate_residual(const void* residual, const void* x,
                                          const void* gate, void* y, int dtype,
                                          int gate_dtype, int64_t rows, int64_t dim,
                                          int64_t gate_stride, int64_t rows_per_batch,
                                          difflet_stream_t stream) {
  DLT_REQUIRE(residual && x && gate && y, DIFFLET_EINVAL, "gate_residual: null pointer");
  DLT_REQUIRE(dim % 8 == 0 && gate_stride % 8 == 0 && aligned16(residual) && aligned16(x) &&
                  aligned16(gate) && aligned16(y),
              DIFFLET_EINVAL, "gate_residual: dim must be a multiple of 8, pointers aligned");
  if (rows * dim == 0) return DIFFLET_OK;
  if (rows_per_batch <= 0) rows_per_batch = rows;
  hipStream_t s = (hipStream_t)stream;
  int64_t blocks = (rows * dim / 8 + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  DLT_DISPATCH_FLOAT(dtype, T,
    DLT_DISPATCH_FLOAT(gate_dtype, TG,
      hipLaunchKernelGGL((gate_residual_kernel<T, TG>), dim3((unsigned)blocks), dim3(256), 0,
                         s, (const T*)residual, (const T*)x, (const TG*)gate, (T*)y, rows,
                         dim, gate_stride, rows_per_batch)));
  return dlt_check_launch("gate_residual");
}

extern "C" int difflet_rocm_gated_gelu(const void* x, int64_t ldx, void* y, int64_t ldy,
                                       int dtype, int64_t rows, int64_t f,
                                       difflet_stream_t stream) {
  DLT_REQUIRE(x && y && rows >= 0 && f > 0, DIFFLET_EINVAL, "gated_gelu: bad arguments");
  DLT_REQUIRE(f % 8 == 0 && ldx % 8 == 0 && ldy % 8 == 0 && ldx >= 2 * f && ldy >= f &&
                  aligned16(x) && aligned16(y),
              DIFFLET_EINVAL,
              "gated_gelu: f and the row strides must be multiples of 8 (ldx >= 2 f, ldy >= f), "
              "pointers 16-byte aligned");
  if (rows == 0) return DIFFLET_OK;
  int64_t blocks = (rows * f / 8 + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  DLT_DISPATCH_FLOAT(dtype, T,
    hipLaunchKernelGGL((gated_gelu_kernel<T>), dim3((unsigned)blocks), dim3(256), 0,
                       (hipStream_t)stream, (const T*)x, ldx, (T*)y, ldy, rows, f));
  return dlt_check_launch("gated_gelu");
}

extern "C" int difflet_rocm_embedding(const int64_t* ids, int64_t n, const void* table,
                                      int64_t table_rows, int64_t ldt_bytes, void* out,
                                      int64_t ldo_bytes, int64_t row_bytes,
                                      difflet_stream_t stream) {
  DLT_REQUIRE(n >= 0 && table_rows > 0 && row_bytes > 0, DIFFLET_EINVAL,
              "embedding: bad sizes");
  if (n == 0) return DIFFLET_OK;
  DLT_REQUIRE(ids && table && out, DIFFLET_EINVAL, "embedding: null pointer");
  DLT_REQUIRE(row_bytes % 16 == 0 && ldt_bytes % 16 == 0 && ldo_bytes % 16 == 0 &&
                  ldt_bytes >= row_bytes && ldo_bytes >= row_bytes && aligned16(table) &&
                  aligned16(out),
              DIFFLET_EINVAL, "embedding: rows must be 16-byte multiples and aligned");
  int64_t blocks = (n * (row_bytes / 16) + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  hipLaunchKernelGGL(embedding_kernel, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream,
                     ids, n, (const uint8_t*)table, table_rows, ldt_bytes, (uint8_t*)out,
                     ldo_bytes, row_bytes);
  return dlt_check_launch("embedding");
}

extern "C" int difflet_rocm_relative_bias(const int32_t* buckets, int num_buckets,
                                          const void* table, int table_dtype, int64_t heads,
                                          int64_t batch, int64_t seq_q, int64_t seq_k,
                                          const uint8_t* key_keep, int64_t keep_stride,
                                          float* out, difflet_stream_t stream) {
  DLT_REQUIRE(num_buckets > 0 && heads > 0 && batch >= 0 && seq_q >= 0 && seq_k >= 0,
              DIFFLET_EINVAL, "relative_bias: bad sizes");
  const int64_t total = batch * heads * seq_q * seq_k;
  if (total == 0) return DIFFLET_OK;
  DLT_REQUIRE(buckets && table && out, DIFFLET_EINVAL, "relative_bias: null pointer");
  DLT_REQUIRE(!key_keep || keep_stride >= seq_k, DIFFLET_EINVAL,
              "relative_bias: keep_stride shorter than seq_k");
  int64_t blocks = (total + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  DLT_DISPATCH_FLOAT(table_dtype, TT,
    hipLaunchKernelGGL((relative_bias_kernel<TT>), dim3((unsigned)blocks), dim3(256), 0,
                       (hipStream_t)stream, buckets, num_buckets, (const TT*)table, heads, batch,
                       seq_q, seq_k, key_keep, keep_stride, out));
  return dlt_check_launch("relative_bias");
}

template <typename T>
static int launch_gemv(const void* x, int64_t m, int mb, int64_t k, int64_t ldx, const void* w,
                       int64_t ldw, int64_t n, const void* bias, void* y, int64_t ldy, int act,
                       hipStream_t s) {
  int64_t blocks = (n + 7) / 8;
  if (blocks > 8192) blocks = 8192;
  const size_t lds = (size_t)(mb * k * 4);
#define DLT_GEMV(M)                                                                          \
  hipLaunchKernelGGL((gemv_kernel<T, M>), dim3((unsigned)blocks), dim3(256), lds, s,         \
                     (const T*)x, (int)m, (int)k, ldx, (const bf16*)w, ldw, n, (const T*)bias,     \
                     (T*)y, ldy, act)
  switch (mb) {
    case 1: DLT_GEMV(1); break;
    case 2: DLT_GEMV(2); break;
    case 4: DLT_GEMV(4); break;
    default: DLT_GEMV(8); break;
  }
#undef DLT_GEMV
  return dlt_check_launch("gemv");
}

extern "C" int difflet_rocm_gemv(const void* x, int dtype, int64_t m, int64_t k, int64_t ldx,
                                 const void* w, int64_t ldw, int64_t n, const void* bias,
                                 void* y, int64_t ldy, int act, difflet_stream_t stream) {
  DLT_REQUIRE(x && w && y, DIFFLET_EINVAL, "gemv: null pointer");
  DLT_REQUIRE(m >= 1 && m <= 8, DIFFLET_EUNSUPPORTED, "gemv: m = %lld not in [1, 8]",
              (long long)m);
  DLT_REQUIRE(k > 0 && k % 8 == 0 && ldw % 8 == 0 && ldw >= k && aligned16(w), DIFFLET_EINVAL,
              "gemv: k and ldw must be multiples of 8, ldw >= k and w 16-byte aligned");
  const int mb = m <= 1 ? 1 : m <= 2 ? 2 : m <= 4 ? 4 : 8;
  DLT_REQUIRE(mb * k * 4 <= 64 * 1024, DIFFLET_EUNSUPPORTED,
              "gemv: m * k = %lld exceeds the 16384-element LDS stage", (long long)(mb * k));
  DLT_REQUIRE(act == 0 || act == 1, DIFFLET_EINVAL, "gemv: act must be 0 or 1");
  if (n == 0) return DIFFLET_OK;
  hipStream_t s = (hipStream_t)stream;
  DLT_DISPATCH_FLOAT(dtype, T,
    return launch_gemv<T>(x, m, mb, k, ldx, w, ldw, n, bias, y, ldy, act, s));
  return DIFFLET_OK;
}

extern "C" int difflet_rocm_timestep_embedding(const float* t, void* y, int dtype, int64_t m,
                                               int64_t dim, int flip_sin_to_cos,
                                               float downscale_freq_shift, float scale,
                                               float max_period, difflet_stream_t stream) {
  DLT_REQUIRE(t && y && m >= 0 && dim > 0, DIFFLET_EINVAL, "timestep_embedding: bad args");
  if (m == 0) return DIFFLET_OK;
  hipStream_t s = (hipStream_t)stream;
  const int64_t total = m * dim;
  DLT_DISPATCH_FLOAT(dtype, T,
    hipLaunchKernelGGL((timestep_embedding_kernel<T>),
                       dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, t, (T*)y, m,
                       (int)dim, flip_sin_to_cos, downscale_freq_shift, scale,
                       (float)(-log((double)max_period))));
  return dlt_check_launch("timestep_embedding");
}
