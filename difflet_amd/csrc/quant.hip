// Activation / weight quantizers to fp8 e4m3fn, bit-exact with the CPU laws.
//
// Per-row (per-token activations, per-output-channel weights): one wavefront per row, a pass
// for the absmax and a pass that writes codes (the second pass re-reads the row from L2).
//
// MXFP8 (difflet/quant/mx.py:46-108): one thread per 32-element block. A block is 32 consecutive
// positions of the swizzle order; inside a K tile of width `tile` (512, or the remainder) with
// sub = tile / 4, swizzled position r * 4 + j is logical k = k0 + j * sub + r, so block b of the
// tile is the four runs k0 + j * sub + 8 b + [0, 8), j = 0..3: four 16-byte loads of bf16.
#include "common.hpp"

namespace dlt {

template <typename T> struct Load8;
template <> struct Load8<bf16> {
  static __device__ __forceinline__ void f(const bf16* p, float* v) {
    u32x4 r = *reinterpret_cast<const u32x4*>(p);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[2 * i] = bf16bits_to_f32(r[i] & 0xffffu);
      v[2 * i + 1] = bf16bits_to_f32(r[i] >> 16);
    }
  }
};
template <> struct Load8<f16> {
  static __device__ __forceinline__ void f(const f16* p, float* v) {
    typedef _Float16 h8 __attribute__((ext_vector_type(8)));
    h8 r = *reinterpret_cast<const h8*>(p);
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = (float)r[i];
  }
};
template <> struct Load8<float> {
  static __device__ __forceinline__ void f(const float* p, float* v) {
    f32x4 a = *reinterpret_cast<const f32x4*>(p);
    f32x4 b = *reinterpret_cast<const f32x4*>(p + 4);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[i] = a[i];
      v[4 + i] = b[i];
    }
  }
};

__device__ __forceinline__ float clamp448(float v) {
  return __builtin_fminf(__builtin_fmaxf(v, -448.0f), 448.0f);
}

// ------------------------------------------------------------------ per-row
template <typename T>
__global__ __launch_bounds__(256) void quant_rowwise_kernel(const T* __restrict__ x,
                                                            int64_t rows, int64_t cols,
                                                            int64_t ldx, uint8_t* __restrict__ q,
                                                            int64_t ldq,
                                                            float* __restrict__ scale) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const T* xr = x + row * ldx;
  float amax = 0.f;
  for (int64_t c = lane * 8; c < cols; c += 512) {
    float v[8];
    Load8<T>::f(xr + c, v);
#pragma unroll
    for (int i = 0; i < 8; ++i) amax = __builtin_fmaxf(amax, __builtin_fabsf(v[i]));
  }
  amax = wave_max(amax);
  const float a = __builtin_fmaxf(amax, 1.925929944387236e-34f);  // 2^-112: 448 / a stays finite
  const float inv = __fdiv_rn(448.0f, a);
  if (lane == 0) scale[row] = __fdiv_rn(a, 448.0f);
  uint8_t* qr = q + row * ldq;
  for (int64_t c = lane * 8; c < cols; c += 512) {
    float v[8];
    Load8<T>::f(xr + c, v);
    u32x2 o = {0u, 0u};
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t code = f32_to_e4m3fn(clamp448(__fmul_rn(v[i], inv)));
      o[i >> 2] |= code << (8 * (i & 3));
    }
    *reinterpret_cast<u32x2*>(qr + c) = o;
  }
}

// ------------------------------------------------------------------ MXFP8
template <typename T>
__global__ __launch_bounds__(256) void quant_mx_kernel(const T* __restrict__ x, int64_t rows,
                                                       int64_t cols, int64_t ldx,
                                                       uint8_t* __restrict__ q, int64_t ldq,
                                                       uint8_t* __restrict__ scale, int64_t lds,
                                                       int swizzled_out) {
  const int64_t nblk = cols / 32;
  const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (gid >= rows * nblk) return;
  const int64_t row = gid / nblk;
  const int64_t blk = gid % nblk;  // block index along the swizzle order
  const int64_t full = cols / 512;
  int64_t k0, sub, b;
  if (blk < full * 16) {
    k0 = (blk / 16) * 512;
    sub = 128;
    b = blk % 16;
  } else {
    k0 = full * 512;
    sub = (cols - k0) / 4;
    b = blk - full * 16;
  }
  const T* xr = x + row * ldx;
  float v[4][8];
  uint32_t emax = 0;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    Load8<T>::f(xr + k0 + j * sub + 8 * b, v[j]);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t e = (__builtin_bit_cast(uint32_t, v[j][i]) >> 23) & 0xffu;
      emax = e > emax ? e : emax;
    }
  }
  const int su = (int)emax - 7 < 0 ? 0 : (int)emax - 7;  // clamp(e_max - 7, 0, 255)
  scale[row * lds + blk] = (uint8_t)su;
  // x / 2^(su - 127) == x * 2^(127 - su): both exact powers of two, same rounding
  const float mul = __builtin_bit_cast(float, (uint32_t)(254 - su) << 23);
  uint8_t codes[4][8];
#pragma unroll
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int i = 0; i < 8; ++i)
      codes[j][i] = (uint8_t)f32_to_e4m3fn(clamp448(__fmul_rn(v[j][i], mul)));
  uint8_t* qr = q + row * ldq;
  if (swizzled_out) {
    // swizzled position (8 b + r) * 4 + j holds logical run j, element r
    u32x4 o0, o1;
#pragma unroll
    for (int r = 0; r < 4; ++r)
      o0[r] = codes[0][r] | (codes[1][r] << 8) | (codes[2][r] << 16) | ((uint32_t)codes[3][r] << 24);
#pragma unroll
    for (int r = 0; r < 4; ++r)
      o1[r] = codes[0][4 + r] | (codes[1][4 + r] << 8) | (codes[2][4 + r] << 16) |
              ((uint32_t)codes[3][4 + r] << 24);
    *reinterpret_cast<u32x4*>(qr + k0 + 32 * b) = o0;
    *reinterpret_cast<u32x4*>(qr + k0 + 32 * b + 16) = o1;
  } else {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      u32x2 o;
      o[0] = codes[j][0] | (codes[j][1] << 8) | (codes[j][2] << 16) | ((uint32_t)codes[j][3] << 24);
      o[1] = codes[j][4] | (codes[j][5] << 8) | (codes[j][6] << 16) | ((uint32_t)codes[j][7] << 24);
      *reinterpret_cast<u32x2*>(qr + k0 + j * sub + 8 * b) = o;
    }
  }
}

}  // namespace dlt

using namespace dlt;

extern "C" int difflet_rocm_quantize_fp8_rowwise(const void* x, int dtype, int64_t rows,
                                                 int64_t cols, int64_t ldx, uint8_t* q,
                                                 int64_t ldq, float* scale,
                                                 difflet_stream_t stream) {
  DLT_REQUIRE(x && q && scale, DIFFLET_EINVAL, "quantize_fp8_rowwise: null pointer");
  DLT_REQUIRE(rows >= 0 && cols > 0 && cols % 8 == 0 && ldx % 8 == 0 && ldq % 8 == 0,
              DIFFLET_EINVAL, "quantize_fp8_rowwise: cols and strides must be multiples of 8");
  DLT_REQUIRE(((uintptr_t)x & 15) == 0 && ((uintptr_t)q & 7) == 0, DIFFLET_EINVAL,
              "quantize_fp8_rowwise: misaligned pointers");
  if (rows == 0) return DIFFLET_OK;
  hipStream_t s = (hipStream_t)stream;
  dim3 grid((unsigned)((rows + 3) / 4)), block(256);
  switch (dtype) {
    case DIFFLET_BF16:
      hipLaunchKernelGGL((quant_rowwise_kernel<bf16>), grid, block, 0, s, (const bf16*)x, rows,
                         cols, ldx, q, ldq, scale);
      break;
    case DIFFLET_F16:
      hipLaunchKernelGGL((quant_rowwise_kernel<f16>), grid, block, 0, s, (const f16*)x, rows,
                         cols, ldx, q, ldq, scale);
      break;
    case DIFFLET_F32:
      hipLaunchKernelGGL((quant_rowwise_kernel<float>), grid, block, 0, s, (const float*)x,
                         rows, cols, ldx, q, ldq, scale);
      break;
    default:
      dlt_set_error("quantize_fp8_rowwise: unsupported dtype %d", dtype);
      return DIFFLET_EINVAL;
  }
  return dlt_check_launch("quantize_fp8_rowwise");
}

extern "C" int difflet_rocm_quantize_mxfp8(const void* x, int dtype, int64_t rows, int64_t cols,
                                           int64_t ldx, uint8_t* q, int64_t ldq,
                                           uint8_t* scale, int64_t lds, int swizzled_out,
                                           difflet_stream_t stream) {
  DLT_REQUIRE(x && q && scale, DIFFLET_EINVAL, "quantize_mxfp8: null pointer");
  DLT_REQUIRE(rows >= 0 && cols > 0 && cols % 128 == 0, DIFFLET_EINVAL,
              "quantize_mxfp8: K=%lld must be a multiple of 128 for the MX layout",
              (long long)cols);
  DLT_REQUIRE(ldx % 8 == 0 && ldq % 16 == 0 && lds >= cols / 32, DIFFLET_EINVAL,
              "quantize_mxfp8: bad strides");
  DLT_REQUIRE(((uintptr_t)x & 15) == 0 && ((uintptr_t)q & 15) == 0, DIFFLET_EINVAL,
              "quantize_mxfp8: misaligned pointers");
  if (rows == 0) return DIFFLET_OK;
  hipStream_t s = (hipStream_t)stream;
  const int64_t threads = rows * (cols / 32);
  dim3 grid((unsigned)((threads + 255) / 256)), block(256);
  switch (dtype) {
    case DIFFLET_BF16:
      hipLaunchKernelGGL((quant_mx_kernel<bf16>), grid, block, 0, s, (const bf16*)x, rows,
                         cols, ldx, q, ldq, scale, lds, swizzled_out);
      break;
    case DIFFLET_F16:
      hipLaunchKernelGGL((quant_mx_kernel<f16>), grid, block, 0, s, (const f16*)x, rows, cols,
                         ldx, q, ldq, scale, lds, swizzled_out);
      break;
    case DIFFLET_F32:
      hipLaunchKernelGGL((quant_mx_kernel<float>), grid, block, 0, s, (const float*)x, rows,
                         cols, ldx, q, ldq, scale, lds, swizzled_out);
      break;
    default:
      dlt_set_error("quantize_mxfp8: unsupported dtype %d", dtype);
      return DIFFLET_EINVAL;
  }
  return dlt_check_launch("quantize_mxfp8");
}
