// Shared device helpers for the gfx950 (CDNA4) kernels of the DiT denoise step.
//
// Everything here is written for 64-lane wavefronts. Types are the compiler's native vector
// types so MFMA builtins take them directly.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/difflet_rocm.h"

namespace dlt {

typedef __bf16 bf16;
typedef _Float16 f16;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kWave = 64;

// ------------------------------------------------------------------ bf16 conversions
// Round-to-nearest-even fp32 -> bf16 on the bit pattern (NaN kept quiet), the same rounding
// torch uses for `.to(torch.bfloat16)`.
// fp32 -> bf16 rounding to nearest even, NaN quieted to (bits >> 16) | 0x40: gfx950's
// v_cvt_pk_bf16_f32, which equals u += 0x7fff + ((u >> 16) & 1), u >> 16 (NaN: the quieted top
// half) on all 2^32 fp32 bit patterns in both halves of the pair (checked exhaustively on the
// GPU), in one instruction per two values instead of five per value. a goes in the low half.
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  typedef float f32x2_t __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t){a, b}, bf16x2_t));
}
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  return (uint16_t)(pack_bf16x2(f, 0.0f) & 0xffffu);
}
__device__ __forceinline__ bf16 f32_to_bf16(float f) {
  return __builtin_bit_cast(bf16, f32_to_bf16_bits(f));
}
__device__ __forceinline__ float bf16_to_f32(bf16 h) {
  return __builtin_bit_cast(float, ((uint32_t)__builtin_bit_cast(uint16_t, h)) << 16);
}
__device__ __forceinline__ float bf16bits_to_f32(uint32_t bits16) {
  return __builtin_bit_cast(float, bits16 << 16);
}

// Element loaders/storers for the activation dtypes the kernels accept.
template <typename T> struct Elt;
template <> struct Elt<bf16> {
  static __device__ __forceinline__ float load(const bf16* p) { return bf16_to_f32(*p); }
  static __device__ __forceinline__ void store(bf16* p, float v) { *p = f32_to_bf16(v); }
};
template <> struct Elt<f16> {
  static __device__ __forceinline__ float load(const f16* p) { return (float)*p; }
  static __device__ __forceinline__ void store(f16* p, float v) { *p = (f16)v; }
};
template <> struct Elt<float> {
  static __device__ __forceinline__ float load(const float* p) { return *p; }
  static __device__ __forceinline__ void store(float* p, float v) { *p = v; }
};

// ------------------------------------------------------------------ fp8 e4m3fn encode
// Round-to-nearest-even fp32 -> OCP float8_e4m3fn code. The caller clamps to [-448, 448]
// first (both quantizer laws do), so no input reaches the NaN code except NaN itself.
// Written on the integer bit pattern so CPU and GPU agree bit for bit.
__device__ __forceinline__ uint32_t f32_to_e4m3fn(float x) {
  uint32_t u = __builtin_bit_cast(uint32_t, x);
  uint32_t sign = (u >> 24) & 0x80u;
  uint32_t a = u & 0x7fffffffu;
  if (a > 0x7f800000u) return sign | 0x7fu;          // NaN
  if (a >= 0x43e00000u) return sign | 0x7eu;         // >= 448: saturate (inputs are clamped)
  if (a < 0x3c800000u) {                             // below 2^-6: subnormal grid of 2^-9
    float m = __builtin_rintf(__builtin_bit_cast(float, a) * 512.0f);
    return sign | (uint32_t)m;                       // 8 rounds up into the smallest normal
  }
  uint32_t r = (a + 0x7ffffu + ((a >> 20) & 1u)) >> 20;  // RNE on the 3 kept mantissa bits
  return sign | (r - (120u << 3));                   // rebias 127 -> 7
}

__device__ __forceinline__ float clamp448(float v) {
  return __builtin_fminf(__builtin_fmaxf(v, -448.0f), 448.0f);
}

// The per-row fp8 law's row constants: a = max(amax, 2^-112) keeps 448 / a finite for all-zero
// rows; scale = a / 448 and inv = 448 / a are IEEE fp32 divides.
__device__ __forceinline__ float rowwise_inv(float amax) {
  return __fdiv_rn(448.0f, __builtin_fmaxf(amax, 1.925929944387236e-34f));
}
__device__ __forceinline__ float rowwise_scale(float amax) {
  return __fdiv_rn(__builtin_fmaxf(amax, 1.925929944387236e-34f), 448.0f);
}
// Four e4m3fn codes (a in the low byte) of values already clamped to [-448, 448], rounded to
// nearest even by the hardware conversion (v_cvt_pk_fp8_f32 writes two codes into the selected
// half of its destination). Its codes equal f32_to_e4m3fn's for every fp32 input in
// [-448, 448], both signs (checked exhaustively on gfx950).
__device__ __forceinline__ uint32_t e4m3x4(float a, float b, float c, float d) {
  int w = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
  w = __builtin_amdgcn_cvt_pk_fp8_f32(c, d, w, true);
  return (uint32_t)w;
}

// Eight codes e4m3(clamp(v * inv)), little-endian in two dwords.
__device__ __forceinline__ u32x2 encode8_rowwise(const float* v, float inv) {
  float c[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) c[i] = clamp448(__fmul_rn(v[i], inv));
  return u32x2{e4m3x4(c[0], c[1], c[2], c[3]), e4m3x4(c[4], c[5], c[6], c[7])};
}

// ------------------------------------------------------------------ wave reductions
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, kWave));
  return v;
}

// Block-wide sum over `nwaves` waves through a small LDS scratch (one slot per wave).
template <int NWAVES>
__device__ __forceinline__ float block_sum(float v, float* red) {
  v = wave_sum(v);
  const int lane = threadIdx.x & (kWave - 1), w = threadIdx.x / kWave;
  if (NWAVES == 1) return v;
  __syncthreads();
  if (lane == 0) red[w] = v;
  __syncthreads();
  float t = 0.f;
#pragma unroll
  for (int i = 0; i < NWAVES; ++i) t += red[i];
  return t;
}
template <int NWAVES>
__device__ __forceinline__ float block_max(float v, float* red) {
  v = wave_max(v);
  const int lane = threadIdx.x & (kWave - 1), w = threadIdx.x / kWave;
  if (NWAVES == 1) return v;
  __syncthreads();
  if (lane == 0) red[w] = v;
  __syncthreads();
  float t = red[0];
#pragma unroll
  for (int i = 1; i < NWAVES; ++i) t = fmaxf(t, red[i]);
  return t;
}

// ------------------------------------------------------------------ math
// GELU with the tanh approximation, 0.5 x (1 + tanh(sqrt(2/pi) (x + 0.044715 x^3))), with tanh
// written through exp: tanh(u) = 1 - 2 / (exp(2u) + 1), which saturates cleanly at +-1.
// 0.5 x (1 + tanh(u)), u = sqrt(2/pi) (x + 0.044715 x^3), written as x sigmoid(2u) =
// x / (1 + 2^(x (c0 + c1 x^2))) with c0 = -2 sqrt(2/pi) log2(e), c1 = 0.044715 c0: the same
// function in five VALU operations and two transcendentals. Large negative x gives 2^+inf = inf
// and x * 0; large positive x gives x.
__device__ __forceinline__ float gelu_tanh(float x) {
  constexpr float c0 = -2.302208198144325f;  // -2 * 0.7978845608028654 * 1.4426950408889634
  constexpr float c1 = c0 * 0.044715f;
  const float e = __builtin_amdgcn_exp2f(x * __builtin_fmaf(x * x, c1, c0));
  return x * __builtin_amdgcn_rcpf(1.0f + e);
}
__device__ __forceinline__ float silu(float x) { return x / (1.0f + __expf(-x)); }

// Sum over each row of 16 lanes, result in all 16, by DPP lane moves (no LDS round trip):
// quad_perm [1,0,3,2] and [2,3,0,1] give each lane its quad's sum, row_half_mirror (lane i of
// 8 takes lane 7 - i) adds the neighbouring quad, row_mirror (i takes 15 - i) the other half.
template <int CTRL>
__device__ __forceinline__ float dpp_move(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float sum16_dpp(float v) {
  v += dpp_move<0xB1>(v);   // quad_perm [1, 0, 3, 2]
  v += dpp_move<0x4E>(v);   // quad_perm [2, 3, 0, 1]
  v += dpp_move<0x141>(v);  // row_half_mirror
  v += dpp_move<0x140>(v);  // row_mirror
  return v;
}

// ------------------------------------------------------------------ buffer resources
// Raw buffer loads: an out-of-range offset reads zero, which is how GEMM and attention tiles
// handle ragged M / N / sequence edges without branches.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                           0x00020000);
}
__device__ __forceinline__ u32x4 buf_load16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}
__device__ __forceinline__ u32x2 buf_load8(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0));
}

// Where a causal convolution's im2col rows come from (the frames of difflet_rocm_conv_causal),
// for the kernels that gather them instead of reading materialized rows: output pixel r =
// (t, y, x) of an ho x wo frame, column k = tap (dt, ky, kx) x C + c, read from buffer frame b =
// t + dt + fbase (zero when b < 0) at element (b >> lfpb) fstride + (b & (2^lfpb - 1)) sub +
// ((y + ky - half) >> up) w + ((x + kx - half) >> up)) ld + c, zero outside the frame.
struct ConvGeo {
  int64_t fstride, sub, ld;  // elements
  int lfpb, fbase;
  int w, ho, wo, up, half, ks;
  uint32_t po, po_m, wo_m, cin, cin_m;  // divisors and their magic numbers (conv_magic)
  int ktot;                             // kt ks^2 C
};

// q = n / d, r = n % d for n < 2^32, m = conv_magic(d): the high word of n m is floor(n / d) or
// one less (n (2^32 mod d) / (d 2^32) < 1), which one compare fixes.
__device__ __forceinline__ uint32_t conv_udiv(uint32_t n, uint32_t d, uint32_t m, uint32_t& r) {
  uint32_t q = __umulhi(n, m);
  r = n - q * d;
  if (r >= d) {
    ++q;
    r -= d;
  }
  return q;
}
inline uint32_t conv_magic(uint32_t d) {
  const uint64_t m = (1ULL << 32) / d;
  return m > 0xffffffffULL ? 0xffffffffu : (uint32_t)m;
}
// tap -> (dt, ky, kx) for ks in {1, 3} (tap = (dt ks + ky) ks + kx; exact for tap < 27)
__device__ __forceinline__ void conv_tap(int tap, int ks, int& dt, int& ky, int& kx) {
  dt = tap, ky = 0, kx = 0;
  if (ks == 3) {
    dt = (tap * 57) >> 9;
    const int rr = tap - 9 * dt;
    ky = (rr * 11) >> 5;
    kx = rr - 3 * ky;
  }
}

// The fp32 convolution on the fp32 matrix-core GEMM with its A rows gathered (gemm_f32.hip).
int launch_conv_f32(const float* x, const ConvGeo& g, int64_t rows, const float* w, int64_t n,
                    int64_t kpad, const float* bias, const float* res, int64_t ldr, float* out,
                    int64_t ldo, hipStream_t s);

}  // namespace dlt

// Error plumbing shared by every entry point: a status code plus a message readable through
// difflet_rocm_last_error().
void dlt_set_error(const char* fmt, ...);
int dlt_check_launch(const char* what);

#define DLT_REQUIRE(cond, code, ...)   \
  do {                                 \
    if (!(cond)) {                     \
      dlt_set_error(__VA_ARGS__);      \
      return (code);                   \
    }                                  \
  } while (0)
