// fp32 GEMM on the matrix cores: C = A W^T (+ bias) (+ residual), every operand fp32.
//
// The linears of a model loaded in fp32 (the T5 / UMT5 text encoders' fp32 option, whose
// reference runs F.linear in fp32: difflet/backends/cpu/ops_impl/linear.py:9-41) run here.
// v_mfma_f32_32x32x2f32 takes one fp32 value of each operand per lane and K step: lane l gives
// row l % 32 of its operand at K index l / 32. A K stage of 32 is cut the same way for both
// operands, lane half h taking K indices h * 16 .. h * 16 + 15 in turn (a fixed bijection of
// the stage's 32 indices onto the 16 MFMA steps x 2 halves), so each lane reads its 16 values
// of a row with four 16-byte LDS reads.
//
// The same kernel runs the fp32 causal convolutions of the VAE decoders as implicit GEMMs: the A
// loader gathers each row's 4-float runs from the frames (difflet_rocm_conv_causal).
//
// Workgroup tile 64 (M) x 128 (N), 4 waves of 32 x 64 (two 32 x 32 MFMA tiles); A and W stages
// of 32 floats per row in LDS, double-buffered (55 KB: two workgroups per compute unit), the
// next stage loaded into registers while the current one is multiplied. As in the bf16 GEMM the
// weight fragment is the MFMA's first operand, so a lane's accumulators hold one row m of C and
// four runs of 4 consecutive columns: the epilogue reads bias / residual and stores C in 16-byte
// pieces. Rows and columns past M / N read zero and are not stored.

#include <hip/hip_runtime.h>

#include <stdint.h>

#include "common.hpp"
#include "difflet_rocm.h"

namespace dlt {

constexpr int F32_BM = 64, F32_BN = 128, F32_BK = 32;
constexpr int F32_LDS_STRIDE = F32_BK + 4;  // floats per LDS row: 16-byte pad against conflicts

struct GemmF32Args {
  const float* a;  // [m][lda], or (CONV) the frames the rows are gathered from by g
  ConvGeo g;
  const float* w;
  const float* bias;
  const float* res;
  float* c;
  int64_t lda, ldw, ldr, ldc;
  int64_t m, n, k;
  int tiles_m, tiles, xcd_chunk;
};

// CONV: A is the im2col rows of a causal convolution, gathered from the frames (p.a) by p.g
template <bool CONV>
__global__ __launch_bounds__(256, 2) void gemm_f32_kernel(const GemmF32Args p) {
  __shared__ __attribute__((aligned(16))) float sa[2][F32_BM * F32_LDS_STRIDE];
  __shared__ __attribute__((aligned(16))) float sw[2][F32_BN * F32_LDS_STRIDE];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  // workgroups are dealt to the 8 XCDs in turn; when the count divides evenly, consecutive
  // tiles (which share a W tile) are given to workgroups on one XCD, so its L2 serves them
  int t = blockIdx.x;
  if (p.xcd_chunk > 0) t = (blockIdx.x & 7) * p.xcd_chunk + (blockIdx.x >> 3);
  const int64_t m0 = (int64_t)(t % p.tiles_m) * F32_BM, n0 = (int64_t)(t / p.tiles_m) * F32_BN;

  // global -> registers: A 64 x 32 floats (2 x 16 bytes per thread), W 128 x 32 (4 x 16 bytes);
  // thread i of a 256-wide pass takes row i / 8, floats (i % 8) * 4 .. + 4
  f32x4 ra[2], rw[4];
  const int lr = tid >> 3, lc = (tid & 7) * 4;
  // CONV: the output pixel (frame, y, x) of this thread's two A rows (y far outside past m)
  int rt[2] = {0, 0}, ry[2] = {0, 0}, rx[2] = {0, 0};
  if constexpr (CONV) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int64_t m = m0 + lr + 32 * j;
      uint32_t pp, xx;
      const uint32_t t = conv_udiv((uint32_t)m, p.g.po, p.g.po_m, pp);
      const uint32_t y = conv_udiv(pp, (uint32_t)p.g.wo, p.g.wo_m, xx);
      rt[j] = (int)t;
      ry[j] = m < p.m ? (int)y : -(1 << 24);
      rx[j] = (int)xx;
    }
  }
  auto load = [&](int64_t k0) {
    const int64_t kk = k0 + lc;
    const bool kok = kk < p.k;  // K % 4 == 0: a run of 4 is all in or all out
    if constexpr (CONV) {  // the run is channels c .. c + 3 of one tap (C % 4 == 0)
      uint32_t c;
      const int tap = (int)conv_udiv((uint32_t)kk, p.g.cin, p.g.cin_m, c);
      int dt, ky, kx;
      conv_tap(tap, p.g.ks, dt, ky, kx);
      const bool col = kk < p.g.ktot;
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int f = rt[j] + dt + p.g.fbase;
        const int yy = ry[j] + ky - p.g.half, xs = rx[j] + kx - p.g.half;
        const bool ok = col && f >= 0 && (uint32_t)yy < (uint32_t)p.g.ho &&
                        (uint32_t)xs < (uint32_t)p.g.wo;
        const int64_t off = (int64_t)(f >> p.g.lfpb) * p.g.fstride +
                            (int64_t)(f & ((1 << p.g.lfpb) - 1)) * p.g.sub +
                            ((int64_t)(yy >> p.g.up) * p.g.w + (xs >> p.g.up)) * p.g.ld + c;
        ra[j] = ok ? *reinterpret_cast<const f32x4*>(p.a + off) : f32x4{0.f, 0.f, 0.f, 0.f};
      }
    } else {
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int64_t m = m0 + lr + 32 * j;
        ra[j] = (kok && m < p.m) ? *reinterpret_cast<const f32x4*>(p.a + m * p.lda + kk)
                                 : f32x4{0.f, 0.f, 0.f, 0.f};
      }
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t n = n0 + lr + 32 * j;
      rw[j] = (kok && n < p.n) ? *reinterpret_cast<const f32x4*>(p.w + n * p.ldw + kk)
                               : f32x4{0.f, 0.f, 0.f, 0.f};
    }
  };
  auto store = [&](int buf) {
#pragma unroll
    for (int j = 0; j < 2; ++j)
      *reinterpret_cast<f32x4*>(&sa[buf][(lr + 32 * j) * F32_LDS_STRIDE + lc]) = ra[j];
#pragma unroll
    for (int j = 0; j < 4; ++j)
      *reinterpret_cast<f32x4*>(&sw[buf][(lr + 32 * j) * F32_LDS_STRIDE + lc]) = rw[j];
  };

  f32x16 acc[2];
#pragma unroll
  for (int j = 0; j < 2; ++j)
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[j][i] = 0.f;
  const int fr = lane & 31, fh = lane >> 5;
  const int nk = (int)((p.k + F32_BK - 1) / F32_BK);
  load(0);
  store(0);
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    const int buf = kt & 1;
    if (kt + 1 < nk) load((int64_t)(kt + 1) * F32_BK);
    float af[16], wf[2][16];
    const float* ap = &sa[buf][(wm * 32 + fr) * F32_LDS_STRIDE + fh * 16];
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const f32x4 x = *reinterpret_cast<const f32x4*>(ap + 4 * v);
#pragma unroll
      for (int e = 0; e < 4; ++e) af[4 * v + e] = x[e];
    }
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const float* wp = &sw[buf][(wn * 64 + j * 32 + fr) * F32_LDS_STRIDE + fh * 16];
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const f32x4 x = *reinterpret_cast<const f32x4*>(wp + 4 * v);
#pragma unroll
        for (int e = 0; e < 4; ++e) wf[j][4 * v + e] = x[e];
      }
    }
#pragma unroll
    for (int s = 0; s < 16; ++s)
#pragma unroll
      for (int j = 0; j < 2; ++j)
        acc[j] = __builtin_amdgcn_mfma_f32_32x32x2f32(wf[j][s], af[s], acc[j], 0, 0, 0);
    // the other buffer was last read before the previous barrier: safe to refill
    if (kt + 1 < nk) store(buf ^ 1);
    __syncthreads();
  }

  // epilogue: lane l holds row m = l % 32 of the wave's rows; register 4 q + e of tile j is
  // column n0 + wn * 64 + j * 32 + q * 8 + 4 (l / 32) + e (N % 4 == 0: runs of 4 are whole)
  const int64_t m = m0 + wm * 32 + fr;
  if (m >= p.m) return;
#pragma unroll
  for (int j = 0; j < 2; ++j)
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int64_t n = n0 + wn * 64 + j * 32 + q * 8 + fh * 4;
      if (n >= p.n) continue;
      f32x4 v = {acc[j][4 * q], acc[j][4 * q + 1], acc[j][4 * q + 2], acc[j][4 * q + 3]};
      if (p.bias) {
        const f32x4 b = *reinterpret_cast<const f32x4*>(p.bias + n);
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] += b[e];
      }
      if (p.res) {
        const f32x4 r = *reinterpret_cast<const f32x4*>(p.res + m * p.ldr + n);
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = r[e] + v[e];
      }
      *reinterpret_cast<f32x4*>(p.c + m * p.ldc + n) = v;
    }
}

}  // namespace dlt

using namespace dlt;

extern "C" int difflet_rocm_gemm_f32(const float* a, int64_t lda, const float* w, int64_t ldw,
                                     const float* bias, const float* residual, int64_t ldr,
                                     float* c, int64_t ldc, int64_t m, int64_t n, int64_t k,
                                     difflet_stream_t stream) {
  DLT_REQUIRE(m >= 0 && n > 0 && k > 0, DIFFLET_EINVAL,
              "gemm_f32: need m >= 0 and positive n, k (m=%lld n=%lld k=%lld)", (long long)m,
              (long long)n, (long long)k);
  if (m == 0) return DIFFLET_OK;
  DLT_REQUIRE(a && w && c, DIFFLET_EINVAL, "gemm_f32: null pointer");
  DLT_REQUIRE(k % 4 == 0 && n % 4 == 0, DIFFLET_EINVAL,
              "gemm_f32: k and n must be multiples of 4 (k=%lld n=%lld)", (long long)k,
              (long long)n);
  DLT_REQUIRE(lda >= k && ldw >= k && ldc >= n && (!residual || ldr >= n), DIFFLET_EINVAL,
              "gemm_f32: leading dimensions shorter than the rows");
  DLT_REQUIRE(lda % 4 == 0 && ldw % 4 == 0 && ldc % 4 == 0 && (!residual || ldr % 4 == 0),
              DIFFLET_EINVAL, "gemm_f32: leading dimensions must be multiples of 4");
  const void* ps[5] = {a, w, c, bias, residual};
  for (int i = 0; i < 5; ++i)
    DLT_REQUIRE(((uintptr_t)ps[i] & 15) == 0, DIFFLET_EINVAL,
                "gemm_f32: pointers must be 16-byte aligned");
  const int64_t tiles_m = (m + F32_BM - 1) / F32_BM, tiles_n = (n + F32_BN - 1) / F32_BN;
  DLT_REQUIRE(tiles_m * tiles_n < (1LL << 31), DIFFLET_EUNSUPPORTED, "gemm_f32: too many tiles");
  GemmF32Args args{};
  args.a = a;
  args.w = w;
  args.bias = bias;
  args.res = residual;
  args.c = c;
  args.lda = lda;
  args.ldw = ldw;
  args.ldr = ldr;
  args.ldc = ldc;
  args.m = m;
  args.n = n;
  args.k = k;
  args.tiles_m = (int)tiles_m;
  args.tiles = (int)(tiles_m * tiles_n);
  args.xcd_chunk = args.tiles % 8 == 0 ? args.tiles / 8 : 0;
  hipLaunchKernelGGL((gemm_f32_kernel<false>), dim3((unsigned)args.tiles), dim3(256), 0,
                     (hipStream_t)stream, args);
  return dlt_check_launch("gemm_f32");
}

namespace dlt {

// The implicit-GEMM form of the fp32 convolution (difflet_rocm_conv_causal with dtype F32): the
// same tiles and K order as the fp32 GEMM of the im2col rows, so the same results bit for bit.
int launch_conv_f32(const float* x, const ConvGeo& g, int64_t rows, const float* w, int64_t n,
                    int64_t kpad, const float* bias, const float* res, int64_t ldr, float* out,
                    int64_t ldo, hipStream_t s) {
  const int64_t tiles_m = (rows + F32_BM - 1) / F32_BM, tiles_n = (n + F32_BN - 1) / F32_BN;
  GemmF32Args args{};
  args.a = x;
  args.g = g;
  args.w = w;
  args.bias = bias;
  args.res = res;
  args.c = out;
  args.lda = 0;
  args.ldw = kpad;
  args.ldr = ldr;
  args.ldc = ldo;
  args.m = rows;
  args.n = n;
  args.k = kpad;
  args.tiles_m = (int)tiles_m;
  args.tiles = (int)(tiles_m * tiles_n);
  args.xcd_chunk = args.tiles % 8 == 0 ? args.tiles / 8 : 0;
  hipLaunchKernelGGL((gemm_f32_kernel<true>), dim3((unsigned)args.tiles), dim3(256), 0, s, args);
  return dlt_check_launch("conv_causal");
}

}  // namespace dlt
