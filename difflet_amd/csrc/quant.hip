// Activation / weight quantizers to fp8 e4m3fn, bit-exact with the CPU laws.
//
// Per-row (per-token activations, per-output-channel weights): 16-bit rows up to 16384 wide run
// one workgroup per row holding the row in registers (one read of the row); wider or fp32 rows
// run one wavefront per row in two passes (absmax, then codes).
//
// MXFP8 (difflet/quant/mx.py:46-108): one thread per 32-element block. A block is 32 consecutive
// positions of the swizzle order; inside a K tile of width `tile` (512, or the remainder) with
// sub = tile / 4, swizzled position r * 4 + j is logical k = k0 + j * sub + r, so block b of the
// tile is the four runs k0 + j * sub + 8 b + [0, 8), j = 0..3: four 16-byte loads of bf16.
#include <type_traits>

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

// Eight 16-bit values held in a 16-byte register vector, to fp32.
template <typename T> __device__ __forceinline__ void decode8(u32x4 r, float* v);
template <> __device__ __forceinline__ void decode8<bf16>(u32x4 r, float* v) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    v[2 * i] = bf16bits_to_f32(r[i] & 0xffffu);
    v[2 * i + 1] = bf16bits_to_f32(r[i] >> 16);
  }
}
template <> __device__ __forceinline__ void decode8<f16>(u32x4 r, float* v) {
  typedef _Float16 h8 __attribute__((ext_vector_type(8)));
  const h8 h = __builtin_bit_cast(h8, r);
#pragma unroll
  for (int i = 0; i < 8; ++i) v[i] = (float)h[i];
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
  const float inv = rowwise_inv(amax);
  if (lane == 0) scale[row] = rowwise_scale(amax);
  uint8_t* qr = q + row * ldq;
  for (int64_t c = lane * 8; c < cols; c += 512) {
    float v[8];
    Load8<T>::f(xr + c, v);
    *reinterpret_cast<u32x2*>(qr + c) = encode8_rowwise(v, inv);
  }
}

// Single pass for 16-bit rows up to 2048 NCH elements: one workgroup per row, each thread keeps
// its NCH chunks of 8 as raw 16-byte vectors, so the row is read from memory once. GELU (bf16
// rows): columns >= act_col_start (a multiple of 8) first become gelu_tanh(x) rounded to bf16,
// the values a GELU epilogue would have stored, and are quantized as such.
template <typename T, int NCH, bool GELU = false>
__global__ __launch_bounds__(256) void quant_rowwise_wg_kernel(const T* __restrict__ x,
                                                               int64_t cols, int64_t ldx,
                                                               uint8_t* __restrict__ q,
                                                               int64_t ldq,
                                                               float* __restrict__ scale,
                                                               int64_t act_col_start = 0) {
  __shared__ float red[4];
  const int64_t row = blockIdx.x;
  const int tid = threadIdx.x;
  const T* xr = x + row * ldx;
  u32x4 raw[NCH];
  float amax = 0.f;
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    const int64_t col = ((int64_t)c * 256 + tid) * 8;
    raw[c] = col < cols ? *reinterpret_cast<const u32x4*>(xr + col) : u32x4{0u, 0u, 0u, 0u};
  }
  if constexpr (GELU) {
    static_assert(std::is_same<T, bf16>::value, "the GELU quantizer takes bf16 rows");
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      const int64_t col = ((int64_t)c * 256 + tid) * 8;
      if (col >= act_col_start && col < cols) {
        float v[8];
        decode8<T>(raw[c], v);
#pragma unroll
        for (int i = 0; i < 4; ++i) raw[c][i] = pack_bf16x2(gelu_tanh(v[2 * i]), gelu_tanh(v[2 * i + 1]));
      }
    }
  }
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    float v[8];
    decode8<T>(raw[c], v);
#pragma unroll
    for (int i = 0; i < 8; ++i) amax = __builtin_fmaxf(amax, __builtin_fabsf(v[i]));
  }
  amax = block_max<4>(amax, red);
  const float inv = rowwise_inv(amax);
  if (tid == 0) scale[row] = rowwise_scale(amax);
  uint8_t* qr = q + row * ldq;
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    const int64_t col = ((int64_t)c * 256 + tid) * 8;
    if (col < cols) {
      float v[8];
      decode8<T>(raw[c], v);
      *reinterpret_cast<u32x2*>(qr + col) = encode8_rowwise(v, inv);
    }
  }
}

template <typename T>
static void launch_rowwise(const void* x, int64_t rows, int64_t cols, int64_t ldx, uint8_t* q,
                           int64_t ldq, float* scale, hipStream_t s) {
  const int64_t nch = (cols + 2047) / 2048;
  const dim3 wg_grid((unsigned)rows), block(256);
#define DLT_QWG(N)                                                                           \
  hipLaunchKernelGGL((quant_rowwise_wg_kernel<T, N>), wg_grid, block, 0, s, (const T*)x, cols, \
                     ldx, q, ldq, scale)
  if (nch <= 1) DLT_QWG(1);
  else if (nch <= 2) DLT_QWG(2);
  else if (nch <= 4) DLT_QWG(4);
  else if (nch <= 6) DLT_QWG(6);
  else if (nch <= 8) DLT_QWG(8);
  else
    hipLaunchKernelGGL((quant_rowwise_kernel<T>), dim3((unsigned)((rows + 3) / 4)), block, 0, s,
                       (const T*)x, rows, cols, ldx, q, ldq, scale);
#undef DLT_QWG
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
  float c[4][8];  // clamped scaled values, encoded by e4m3x4 (round to nearest even)
#pragma unroll
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int i = 0; i < 8; ++i) c[j][i] = clamp448(__fmul_rn(v[j][i], mul));
  uint8_t* qr = q + row * ldq;
  if (swizzled_out) {
    // swizzled position (8 b + r) * 4 + j holds logical run j, element r
    u32x4 o0, o1;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      o0[r] = e4m3x4(c[0][r], c[1][r], c[2][r], c[3][r]);
      o1[r] = e4m3x4(c[0][4 + r], c[1][4 + r], c[2][4 + r], c[3][4 + r]);
    }
    *reinterpret_cast<u32x4*>(qr + k0 + 32 * b) = o0;
    *reinterpret_cast<u32x4*>(qr + k0 + 32 * b + 16) = o1;
  } else {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const u32x2 o = {e4m3x4(c[j][0], c[j][1], c[j][2], c[j][3]),
                       e4m3x4(c[j][4], c[j][5], c[j][6], c[j][7])};
      *reinterpret_cast<u32x2*>(qr + k0 + j * sub + 8 * b) = o;
    }
  }
}

}  // namespace dlt

using namespace dlt;

extern "C" int difflet_rocm_quantize_fp8_rowwise_gelu(const void* x, int dtype, int64_t rows,
                                                      int64_t cols, int64_t ldx, uint8_t* q,
                                                      int64_t ldq, float* scale,
                                                      int64_t act_col_start,
                                                      difflet_stream_t stream) {
  DLT_REQUIRE(x && q && scale, DIFFLET_EINVAL, "quantize_fp8_rowwise_gelu: null pointer");
  DLT_REQUIRE(dtype == DIFFLET_BF16, DIFFLET_EUNSUPPORTED,
              "quantize_fp8_rowwise_gelu: rows must be bf16");
  DLT_REQUIRE(rows >= 0 && cols > 0 && cols % 8 == 0 && cols <= 16384 && ldx % 8 == 0 &&
                  ldq % 8 == 0 && act_col_start >= 0 && act_col_start % 8 == 0,
              DIFFLET_EINVAL,
              "quantize_fp8_rowwise_gelu: cols (at most 16384), strides and act_col_start must "
              "be multiples of 8");
  DLT_REQUIRE(((uintptr_t)x & 15) == 0 && ((uintptr_t)q & 7) == 0, DIFFLET_EINVAL,
              "quantize_fp8_rowwise_gelu: misaligned pointers");
  if (rows == 0) return DIFFLET_OK;
  hipStream_t s = (hipStream_t)stream;
  const int64_t nch = (cols + 2047) / 2048;
  const dim3 grid((unsigned)rows), block(256);
#define DLT_QWGG(N)                                                                            \
  hipLaunchKernelGGL((quant_rowwise_wg_kernel<bf16, N, true>), grid, block, 0, s,              \
                     (const bf16*)x, cols, ldx, q, ldq, scale, act_col_start)
  if (nch <= 1) DLT_QWGG(1);
  else if (nch <= 2) DLT_QWGG(2);
  else if (nch <= 4) DLT_QWGG(4);
  else if (nch <= 6) DLT_QWGG(6);
  else DLT_QWGG(8);
#undef DLT_QWGG
  return dlt_check_launch("quantize_fp8_rowwise_gelu");
}

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
      launch_rowwise<bf16>(x, rows, cols, ldx, q, ldq, scale, s);
      break;
    case DIFFLET_F16:
      launch_rowwise<f16>(x, rows, cols, ldx, q, ldq, scale, s);
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
