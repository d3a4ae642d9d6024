// Kernels of the VAE decoder (diffusers' 2D Decoder as the reference builds it for FLUX:
// difflet/models/flux/vae/modeling_vae.py:107-117, difflet/backends/neuron/flux/vae.py:25-36):
// GroupNorm over channels-last activations, the im2col gather of a 3x3 convolution (with the
// nearest 2x upsampling of Upsample2D folded into its addressing), and the row softmax of the
// mid-block attention. The convolutions and linears themselves run on the GEMMs.
//
// Activations are channels-last: [batch][pixels][channels], pixels row-major (y * W + x).
//
// GroupNorm runs in three passes over the activation: per-chunk, per-channel sums (of x, then of
// (x - mean)^2), each merged per (batch, group) in double precision, then the normalization
// with the affine weights (and SiLU) applied elementwise. Two passes for the variance keep it
// free of the E[x^2] - E[x]^2 cancellation; both statistics are the population ones of
// F.group_norm.

#include <hip/hip_runtime.h>

#include <float.h>
#include <stdint.h>

#include "common.hpp"
#include "difflet_rocm.h"

namespace dlt {

// 8 consecutive values as fp32, from bf16 (16 bytes) or fp32 (32 bytes)
template <typename T> struct Vec8;
template <> struct Vec8<bf16> {
  static __device__ __forceinline__ void load(const bf16* p, float* v) {
    const u32x4 r = *reinterpret_cast<const u32x4*>(p);
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
template <> struct Vec8<float> {
  static __device__ __forceinline__ void load(const float* p, float* v) {
    const f32x4 a = *reinterpret_cast<const f32x4*>(p), b = *reinterpret_cast<const f32x4*>(p + 4);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[i] = a[i];
      v[4 + i] = b[i];
    }
  }
  static __device__ __forceinline__ void store(float* p, const float* v) {
    *reinterpret_cast<f32x4*>(p) = f32x4{v[0], v[1], v[2], v[3]};
    *reinterpret_cast<f32x4*>(p + 4) = f32x4{v[4], v[5], v[6], v[7]};
  }
};

// ---- GroupNorm pass 1 / 2: per-channel sums over a chunk of pixels. Thread t handles channels
// 8 (t % tpp) .. + 8 of pixel t / tpp of each pass (tpp = C / 8 threads per pixel); the
// workgroup's threads that share channels are summed through LDS. mean == nullptr: sums of x;
// else sums of (x - mean[b][group])^2. partial: [batch][chunks][C].
template <typename T>
__global__ __launch_bounds__(256) void gn_stats_kernel(const T* __restrict__ x, int64_t pixels,
                                                       int channels, int groups, int64_t chunk,
                                                       const float* __restrict__ mean,
                                                       float* __restrict__ partial) {
  __shared__ float red[256][9];
  const int tid = threadIdx.x, tpp = channels / 8, ppass = 256 / tpp;
  const int b = blockIdx.y, ck = blockIdx.x;
  const int cv = tid % tpp, pr = tid / tpp;
  const bool active = pr < ppass;
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  float mu[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  const int cpg = channels / groups;
  if (mean && active)
#pragma unroll
    for (int i = 0; i < 8; ++i) mu[i] = mean[b * groups + (cv * 8 + i) / cpg];
  const int64_t p0 = ck * chunk, p1 = min(p0 + chunk, pixels);
  const T* xb = x + (int64_t)b * pixels * channels;
  if (active)
    for (int64_t p = p0 + pr; p < p1; p += ppass) {
      float v[8];
      Vec8<T>::load(xb + p * channels + cv * 8, v);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float d = v[i] - mu[i];
        acc[i] += mean ? d * d : v[i];
      }
    }
#pragma unroll
  for (int i = 0; i < 8; ++i) red[tid][i] = active ? acc[i] : 0.f;
  __syncthreads();
  if (tid < tpp) {
    float s[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int r = 0; r < ppass; ++r)
#pragma unroll
      for (int i = 0; i < 8; ++i) s[i] += red[r * tpp + tid][i];
    float* out = partial + ((int64_t)b * gridDim.x + ck) * channels + tid * 8;
#pragma unroll
    for (int i = 0; i < 8; ++i) out[i] = s[i];
  }
}

// One workgroup per (batch, group): the chunks' partial sums of the group's channels merged in
// double (each thread strides over (chunk, channel) pairs, then a tree through LDS). mode 0: the
// mean; mode 1: rstd = 1 / sqrt(var + eps) from the sums of squared deviations.
__global__ __launch_bounds__(256) void gn_reduce_kernel(const float* __restrict__ partial,
                                                        int batch, int chunks, int channels,
                                                        int groups, int64_t pixels, int mode,
                                                        float eps, float* __restrict__ out) {
  __shared__ double red[256];
  const int i = blockIdx.x;  // b * groups + g
  const int b = i / groups, gi = i % groups, cpg = channels / groups;
  double s = 0.0;
  for (int e = threadIdx.x; e < chunks * cpg; e += 256) {
    const int c = e / cpg, k = e % cpg;
    s += (double)partial[((int64_t)b * chunks + c) * channels + gi * cpg + k];
  }
  red[threadIdx.x] = s;
  __syncthreads();
  for (int w = 128; w > 0; w >>= 1) {
    if ((int)threadIdx.x < w) red[threadIdx.x] += red[threadIdx.x + w];
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    const double n = (double)pixels * (double)cpg;
    out[i] = mode == 0 ? (float)(red[0] / n) : (float)(1.0 / __builtin_sqrt(red[0] / n + (double)eps));
  }
}

// y = (x - mean) * rstd * weight + bias, then SiLU when act == 1. Thread t of a workgroup keeps
// channels 8 (t % nv) .. + 8 (nv = C / 8 vectors per pixel) for all its pixels, with the scale
// rstd * weight and shift bias - mean * scale of its 8 channels computed once; blockIdx.y is the
// batch element.
template <typename T>
__global__ __launch_bounds__(256) void gn_apply_kernel(const T* __restrict__ x, T* __restrict__ y,
                                                       int64_t pixels, int channels, int groups,
                                                       const float* __restrict__ mean,
                                                       const float* __restrict__ rstd,
                                                       const float* __restrict__ w,
                                                       const float* __restrict__ bias, int act) {
  const int nv = channels / 8, ppb = 256 / nv;  // pixels per workgroup pass
  const int cv = threadIdx.x % nv, pr = threadIdx.x / nv;
  if (pr >= ppb) return;
  const int b = blockIdx.y, cpg = channels / groups;
  float sc[8], sh[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    const int c = cv * 8 + k, gi = b * groups + c / cpg;
    sc[k] = rstd[gi] * (w ? w[c] : 1.f);
    sh[k] = (bias ? bias[c] : 0.f) - mean[gi] * sc[k];
  }
  const int64_t base = (int64_t)b * pixels * channels + cv * 8;
  for (int64_t p = (int64_t)blockIdx.x * ppb + pr; p < pixels; p += (int64_t)gridDim.x * ppb) {
    float v[8];
    Vec8<T>::load(x + base + p * channels, v);
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      float o = __builtin_fmaf(v[k], sc[k], sh[k]);
      if (act == 1) o = o / (1.0f + __expf(-o));
      v[k] = o;
    }
    Vec8<T>::store(y + base + p * channels, v);
  }
}

// ---- softmax over rows of fp32 scores: p = exp(s * scale - max) / sum, written in T. One
// workgroup per row.
template <typename T>
__global__ __launch_bounds__(256) void softmax_rows_kernel(const float* __restrict__ s,
                                                           int64_t lds, T* __restrict__ p,
                                                           int64_t ldp, int64_t cols,
                                                           float scale) {
  __shared__ float red[4];
  const float* row = s + (int64_t)blockIdx.x * lds;
  T* prow = p + (int64_t)blockIdx.x * ldp;
  // rows of 16-byte runs when both strides and bases allow (the scores of the decoders); the
  // rest of a row, or every element otherwise, one at a time
  const bool vec = (lds & 3) == 0 && ((uintptr_t)s & 15) == 0 && (ldp & 3) == 0 &&
                   ((uintptr_t)p & (4 * sizeof(T) - 1)) == 0;
  const int64_t nv = vec ? cols >> 2 : 0;
  // one read for both statistics: each thread's running max and its sum of exp(x - max),
  // rescaled when the max moves; then the block's max and the sums rescaled to it
  float m = -INFINITY, sum = 0.f;
  for (int64_t v = threadIdx.x; v < nv; v += 256) {
    const f32x4 x = *reinterpret_cast<const f32x4*>(row + 4 * v);
    const float a = x[0] * scale, b = x[1] * scale, c = x[2] * scale, d = x[3] * scale;
    const float nm = fmaxf(m, fmaxf(fmaxf(a, b), fmaxf(c, d)));
    sum = sum * __expf(m - nm) + __expf(a - nm) + __expf(b - nm) + __expf(c - nm) +
          __expf(d - nm);
    m = nm;
  }
  for (int64_t c = 4 * nv + threadIdx.x; c < cols; c += 256) {
    const float x = row[c] * scale;
    const float nm = fmaxf(m, x);
    sum = sum * __expf(m - nm) + __expf(x - nm);
    m = nm;
  }
  const float mx = block_max<4>(m, red);
  sum = block_sum<4>(m == -INFINITY ? 0.f : sum * __expf(m - mx), red);
  const float inv = 1.0f / sum;
  for (int64_t v = threadIdx.x; v < nv; v += 256) {
    const f32x4 x = *reinterpret_cast<const f32x4*>(row + 4 * v);
    float o[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) o[e] = __expf(x[e] * scale - mx) * inv;
    if constexpr (sizeof(T) == 2) {
      const u32x2 w = {pack_bf16x2(o[0], o[1]), pack_bf16x2(o[2], o[3])};
      *reinterpret_cast<u32x2*>(prow + 4 * v) = w;
    } else {
      *reinterpret_cast<f32x4*>(prow + 4 * v) = f32x4{o[0], o[1], o[2], o[3]};
    }
  }
  for (int64_t c = 4 * nv + threadIdx.x; c < cols; c += 256)
    Elt<T>::store(prow + c, __expf(row[c] * scale - mx) * inv);
}

// ---- Wan's 3D causal VAE decoder (difflet/models/wan/vae/modeling_vae.py).
//
// Frames are channels-last too: frame f of a chunk is [pixels][channels] at a frame address
// base(f) = (f / fpb) * fstride + (f % fpb) * sub with pixel stride ld. fpb = 2 reads the time
// convolution's [t][pixels][2C] output as the frames it interleaves (frame 2t = channels
// [0, C) of frame t, frame 2t + 1 = channels [C, 2C)) without a copy.

// ---- im2col of a convolution over channels-last frames: a causal (kt, ks, ks) kernel, kt and
// ks in {1, 3}, spatial padding ks / 2 and temporal padding kt - 1 frames in front (kt = 1,
// ks = 3: a 3x3 Conv2d per frame). For output frame t of the chunk and output pixel (y, x),
// tap (dt, ky, kx) reads frame t + dt - (kt - 1) at pixel (y + ky - ks / 2, x + kx - ks / 2),
// zero outside the frame; a frame before the chunk (-2 or -1) comes from the two-frame cache
// [2][pixels][C] of the convolution's input (zeros when cache is null). Row r of out holds
// output row row0 + r = t * Ho * Wo + y * Wo + x; columns ((dt * ks + ky) * ks + kx) * C + c,
// zero from kt ks^2 C to kpad. up == 1 doubles each frame by nearest neighbour first.
//
// A gather bound by its stores (a row of K columns from K / C source pixels). Each workgroup
// first tabulates its columns' (tap, channel) in LDS, one entry per 16-byte chunk; then each
// wave takes one output row at a time (its frame and pixel computed once per row) and its lanes
// copy consecutive 16-byte chunks, so every store instruction writes 1 KB in one piece.
constexpr int IM2COL_MAX_TAB = 8192;  // chunks with data per row (LDS: 32 KB)
template <typename T>
__global__ __launch_bounds__(256) void im2col_rows_kernel(
    const T* __restrict__ x, int64_t fstride, int fpb, int64_t sub, int64_t ld,
    const T* __restrict__ cache, int h, int w, int channels, int kt, int ks, int up,
    int64_t row0, int64_t rows, T* __restrict__ out, int64_t ldo, int kpad) {
  constexpr int EV = 16 / sizeof(T);
  extern __shared__ uint32_t tab[];
  const int ho = h << up, wo = w << up;
  const int64_t po = (int64_t)ho * wo, pin = (int64_t)h * w;
  const int half = ks >> 1;
  const int nk = kt * ks * ks * channels / EV;  // chunks with data
  const int nv = kpad / EV;                     // chunks per output row
  for (int j = threadIdx.x; j < nk; j += 256) {
    const int col = j * EV, tap = col / channels, c = col - tap * channels;
    const int dt = tap / (ks * ks), rem = tap - dt * ks * ks, ky = rem / ks, kx = rem - ky * ks;
    tab[j] = ((uint32_t)dt << 28) | ((uint32_t)ky << 24) | ((uint32_t)kx << 20) | (uint32_t)c;
  }
  __syncthreads();
  const int lane = threadIdx.x & 63;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  for (int64_t r = (int64_t)blockIdx.x * 4 + wv; r < rows; r += (int64_t)gridDim.x * 4) {
    const int64_t R = row0 + r;
    const int t = (int)(R / po);
    const int p = (int)(R - (int64_t)t * po);
    const int oy = p / wo, ox = p - oy * wo;
    T* dst = out + r * ldo;
    for (int j = lane; j < nv; j += 64) {
      u32x4 v = {0u, 0u, 0u, 0u};
      if (j < nk) {
        const uint32_t e = tab[j];
        const int dt = (int)(e >> 28), ky = (int)(e >> 24) & 15, kx = (int)(e >> 20) & 15;
        const int c = (int)(e & 0xfffffu);
        const int f = t + dt - (kt - 1);
        const int yy = oy + ky - half, xs = ox + kx - half;
        if (yy >= 0 && yy < ho && xs >= 0 && xs < wo) {
          const int64_t pix = (int64_t)(yy >> up) * w + (xs >> up);
          const T* src = nullptr;
          if (f >= 0)
            src = x + (int64_t)(f / fpb) * fstride + (int64_t)(f % fpb) * sub + pix * ld + c;
          else if (cache)
            src = cache + ((int64_t)(f + 2) * pin + pix) * channels + c;
          if (src) v = *reinterpret_cast<const u32x4*>(src);
        }
      }
      *reinterpret_cast<u32x4*>(dst + j * EV) = v;
    }
  }
}

// WanRMSNorm over the channels of each pixel, then SiLU when act == 1 (modeling_vae.py:154-160):
// y = x * sqrt(C) / max(||x||_2, eps) * gamma, in fp32, rounded once. LPR lanes share a pixel
// row, each holding NV vectors of 8 channels (channels <= 8 * LPR * NV); a lane group takes RB
// rows at a time, their loads issued together, and each lane holds its gamma values throughout.
template <typename T, int LPR, int NV, int RB>
__global__ __launch_bounds__(256) void rms_channels_kernel(const T* __restrict__ x, int64_t ldx,
                                                           T* __restrict__ y, int64_t ldy,
                                                           int64_t rows, int channels,
                                                           const float* __restrict__ gamma,
                                                           float eps, int act) {
  const int lane = threadIdx.x % LPR;
  const int nvec = channels / 8;
  const float root = __builtin_sqrtf((float)channels);
  float g[NV][8];
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int vi = lane + j * LPR;
#pragma unroll
    for (int k = 0; k < 8; ++k) g[j][k] = vi < nvec ? gamma[vi * 8 + k] : 0.f;
  }
  const int64_t stride = (int64_t)gridDim.x * (256 / LPR);
  for (int64_t row0 = ((int64_t)blockIdx.x * 256 + threadIdx.x) / LPR; row0 < rows;
       row0 += stride * RB) {
    float v[RB][NV][8];
    float ss[RB];
#pragma unroll
    for (int r = 0; r < RB; ++r) {
      const int64_t row = row0 + r * stride;
      ss[r] = 0.f;
#pragma unroll
      for (int j = 0; j < NV; ++j) {
        const int vi = lane + j * LPR;
        if (row < rows && vi < nvec) Vec8<T>::load(x + row * ldx + vi * 8, v[r][j]);
      }
    }
#pragma unroll
    for (int r = 0; r < RB; ++r) {
      const int64_t row = row0 + r * stride;
#pragma unroll
      for (int j = 0; j < NV; ++j) {
        const int vi = lane + j * LPR;
        if (row < rows && vi < nvec) {
#pragma unroll
          for (int k = 0; k < 8; ++k) ss[r] = __builtin_fmaf(v[r][j][k], v[r][j][k], ss[r]);
        }
      }
#pragma unroll
      for (int o = LPR / 2; o > 0; o >>= 1) ss[r] += __shfl_xor(ss[r], o, LPR);
    }
#pragma unroll
    for (int r = 0; r < RB; ++r) {
      const int64_t row = row0 + r * stride;
      const float scale = root / fmaxf(__builtin_sqrtf(ss[r]), eps);
#pragma unroll
      for (int j = 0; j < NV; ++j) {
        const int vi = lane + j * LPR;
        if (row < rows && vi < nvec) {
#pragma unroll
          for (int k = 0; k < 8; ++k) {
            float o = v[r][j][k] * scale * g[j][k];
            // SiLU with the hardware reciprocal (1 ulp) in place of the IEEE divide, which
            // costs more than the rest of the row's arithmetic
            if (act == 1) o = o * __builtin_amdgcn_rcpf(1.0f + __expf(-o));
            v[r][j][k] = o;
          }
          Vec8<T>::store(y + row * ldy + vi * 8, v[r][j]);
        }
      }
    }
  }
}

// Channels-last rows [n][ld] (the first `channels` columns used) -> channel-first planes
// out[c][n], each value clamped to [lo, hi]: one thread per row.
template <typename T>
__global__ __launch_bounds__(256) void rows_to_planes_kernel(const T* __restrict__ x, int64_t ld,
                                                             int64_t n, int channels,
                                                             T* __restrict__ out, float lo,
                                                             float hi) {
  for (int64_t q = (int64_t)blockIdx.x * 256 + threadIdx.x; q < n;
       q += (int64_t)gridDim.x * 256)
    for (int c = 0; c < channels; ++c) {
      const float v = Elt<T>::load(x + q * ld + c);  // NaN passes, as torch.clamp keeps it
      Elt<T>::store(out + (int64_t)c * n + q, v < lo ? lo : (v > hi ? hi : v));
    }
}

}  // namespace dlt

using namespace dlt;

#define DLT_DISPATCH_BF16_F32(dt, T, ...)                                          \
  switch (dt) {                                                                    \
    case DIFFLET_BF16: { typedef bf16 T; __VA_ARGS__; break; }                     \
    case DIFFLET_F32: { typedef float T; __VA_ARGS__; break; }                     \
    default: dlt_set_error("unsupported dtype %d (bf16 or fp32)", (int)(dt));       \
      return DIFFLET_EUNSUPPORTED;                                                 \
  }

static bool vae_aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

// chunking of the GroupNorm statistics: at most 512 chunks per image, each a multiple of the
// pixels one pass of 256 threads covers
static int64_t gn_chunk(int64_t pixels, int channels) {
  const int64_t ppass = 256 / (channels / 8);
  int64_t chunk = (pixels + 511) / 512;
  chunk = (chunk + ppass - 1) / ppass * ppass;
  return chunk < ppass ? ppass : chunk;
}

extern "C" int64_t difflet_rocm_group_norm_workspace_bytes(int64_t batch, int64_t pixels,
                                                           int64_t channels, int64_t groups) {
  if (batch <= 0 || pixels <= 0 || channels <= 0 || groups <= 0) return 0;
  const int64_t chunks = (pixels + gn_chunk(pixels, (int)channels) - 1) / gn_chunk(pixels, (int)channels);
  return (batch * chunks * channels + 2 * batch * groups) * 4;
}

extern "C" int difflet_rocm_group_norm(const void* x, void* y, int dtype, int64_t batch,
                                       int64_t pixels, int64_t channels, int64_t groups,
                                       const float* weight, const float* bias, float eps, int act,
                                       void* workspace, int64_t workspace_bytes,
                                       difflet_stream_t stream) {
  DLT_REQUIRE(batch >= 0 && pixels >= 0 && groups > 0 && channels > 0, DIFFLET_EINVAL,
              "group_norm: bad sizes");
  DLT_REQUIRE(channels % groups == 0 && channels % 8 == 0 && channels <= 2048, DIFFLET_EINVAL,
              "group_norm: channels (%lld) must be a multiple of 8 and of groups (%lld), <= 2048",
              (long long)channels, (long long)groups);
  DLT_REQUIRE(act == 0 || act == 1, DIFFLET_EINVAL, "group_norm: act must be 0 or 1");
  if (batch * pixels == 0) return DIFFLET_OK;
  DLT_REQUIRE(x && y && workspace, DIFFLET_EINVAL, "group_norm: null pointer");
  DLT_REQUIRE(vae_aligned16(x) && vae_aligned16(y) && vae_aligned16(workspace), DIFFLET_EINVAL,
              "group_norm: pointers must be 16-byte aligned");
  DLT_REQUIRE(batch < 65536, DIFFLET_EUNSUPPORTED, "group_norm: batch too large");
  const int64_t need = difflet_rocm_group_norm_workspace_bytes(batch, pixels, channels, groups);
  DLT_REQUIRE(workspace_bytes >= need, DIFFLET_EINVAL,
              "group_norm: workspace of %lld bytes, need %lld", (long long)workspace_bytes,
              (long long)need);
  const int64_t chunk = gn_chunk(pixels, (int)channels);
  const int chunks = (int)((pixels + chunk - 1) / chunk);
  float* partial = reinterpret_cast<float*>(workspace);
  float* mean = partial + batch * chunks * channels;
  float* rstd = mean + batch * groups;
  hipStream_t s = (hipStream_t)stream;
  const dim3 sgrid((unsigned)chunks, (unsigned)batch);
  const unsigned rblocks = (unsigned)(batch * groups);
  const int64_t ppb = 256 / (channels / 8);
  int64_t ablocks = (pixels + ppb - 1) / ppb;
  if (ablocks > 4096) ablocks = 4096;
  const dim3 agrid((unsigned)ablocks, (unsigned)batch);
  DLT_DISPATCH_BF16_F32(dtype, T,
    hipLaunchKernelGGL((gn_stats_kernel<T>), sgrid, dim3(256), 0, s, (const T*)x, pixels,
                       (int)channels, (int)groups, chunk, (const float*)nullptr, partial);
    hipLaunchKernelGGL(gn_reduce_kernel, dim3(rblocks), dim3(256), 0, s, partial, (int)batch,
                       chunks, (int)channels, (int)groups, pixels, 0, eps, mean);
    hipLaunchKernelGGL((gn_stats_kernel<T>), sgrid, dim3(256), 0, s, (const T*)x, pixels,
                       (int)channels, (int)groups, chunk, (const float*)mean, partial);
    hipLaunchKernelGGL(gn_reduce_kernel, dim3(rblocks), dim3(256), 0, s, partial, (int)batch,
                       chunks, (int)channels, (int)groups, pixels, 1, eps, rstd);
    hipLaunchKernelGGL((gn_apply_kernel<T>), agrid, dim3(256), 0, s, (const T*)x, (T*)y, pixels,
                       (int)channels, (int)groups, mean, rstd, weight, bias, act));
  return dlt_check_launch("group_norm");
}

extern "C" int difflet_rocm_im2col3x3(const void* x, int dtype, int64_t height, int64_t width,
                                      int64_t channels, int upsample, int64_t row0, int64_t rows,
                                      void* out, int64_t ldo, int64_t kpad,
                                      difflet_stream_t stream) {
  DLT_REQUIRE(height > 0 && width > 0 && channels > 0 && (upsample == 0 || upsample == 1),
              DIFFLET_EINVAL, "im2col3x3: bad sizes");
  DLT_REQUIRE(x && out, DIFFLET_EINVAL, "im2col3x3: null pointer");
  const int ev = dtype == DIFFLET_F32 ? 4 : 8;
  DLT_REQUIRE(channels % ev == 0 && kpad % ev == 0 && kpad >= 9 * channels && ldo >= kpad &&
                  ldo % ev == 0 && vae_aligned16(x) && vae_aligned16(out),
              DIFFLET_EINVAL,
              "im2col3x3: channels, kpad and ldo must be multiples of %d (16 bytes), kpad >= 9 C, "
              "pointers aligned", ev);
  const int64_t ho = height << upsample, wo = width << upsample;
  DLT_REQUIRE(ho * wo < (1LL << 31) && 9 * channels < (1LL << 30), DIFFLET_EUNSUPPORTED,
              "im2col3x3: image too large");
  DLT_REQUIRE(row0 >= 0 && rows >= 0 && row0 + rows <= ho * wo, DIFFLET_EINVAL,
              "im2col3x3: rows [%lld, %lld) outside the %lld output pixels", (long long)row0,
              (long long)(row0 + rows), (long long)(ho * wo));
  if (rows == 0) return DIFFLET_OK;
  DLT_REQUIRE(9 * channels / ev <= IM2COL_MAX_TAB, DIFFLET_EUNSUPPORTED,
              "im2col3x3: too many channels");
  int64_t blocks = (rows + 3) / 4;
  if (blocks > 65536) blocks = 65536;
  const size_t tab_bytes = (size_t)(9 * channels / ev) * 4;
  DLT_DISPATCH_BF16_F32(dtype, T,
    hipLaunchKernelGGL((im2col_rows_kernel<T>), dim3((unsigned)blocks), dim3(256), tab_bytes,
                       (hipStream_t)stream, (const T*)x, (int64_t)0, 1, (int64_t)0, channels,
                       (const T*)nullptr, (int)height, (int)width, (int)channels, 1, 3, upsample,
                       row0, rows, (T*)out, ldo, (int)kpad));
  return dlt_check_launch("im2col3x3");
}

extern "C" int difflet_rocm_softmax_rows(const float* s, int64_t lds, void* p, int64_t ldp,
                                         int dtype, int64_t rows, int64_t cols, float scale,
                                         difflet_stream_t stream) {
  DLT_REQUIRE(rows >= 0 && cols > 0 && lds >= cols && ldp >= cols, DIFFLET_EINVAL,
              "softmax_rows: bad sizes");
  if (rows == 0) return DIFFLET_OK;
  DLT_REQUIRE(s && p, DIFFLET_EINVAL, "softmax_rows: null pointer");
  DLT_REQUIRE(rows < (1LL << 31), DIFFLET_EUNSUPPORTED, "softmax_rows: too many rows");
  DLT_DISPATCH_BF16_F32(dtype, T,
    hipLaunchKernelGGL((softmax_rows_kernel<T>), dim3((unsigned)rows), dim3(256), 0,
                       (hipStream_t)stream, s, lds, (T*)p, ldp, cols, scale));
  return dlt_check_launch("softmax_rows");
}

extern "C" int difflet_rocm_im2col_causal(const void* x, int64_t frame_stride,
                                          int64_t frames_per_block, int64_t sub_stride,
                                          int64_t pixel_stride, const void* cache, int dtype,
                                          int64_t height, int64_t width, int64_t channels,
                                          int64_t kt, int64_t ks, int upsample, int64_t row0,
                                          int64_t rows, void* out, int64_t ldo, int64_t kpad,
                                          difflet_stream_t stream) {
  DLT_REQUIRE(height > 0 && width > 0 && channels > 0 && (upsample == 0 || upsample == 1) &&
                  (kt == 1 || kt == 3) && (ks == 1 || ks == 3) &&
                  (frames_per_block == 1 || frames_per_block == 2),
              DIFFLET_EINVAL, "im2col_causal: bad sizes or taps (kt, ks in {1, 3})");
  DLT_REQUIRE(x && out, DIFFLET_EINVAL, "im2col_causal: null pointer");
  const int ev = dtype == DIFFLET_F32 ? 4 : 8;
  const int64_t k = kt * ks * ks * channels;
  DLT_REQUIRE(channels % ev == 0 && kpad % ev == 0 && kpad >= k && ldo >= kpad && ldo % ev == 0 &&
                  pixel_stride >= channels && pixel_stride % ev == 0 && sub_stride % ev == 0 &&
                  frame_stride % ev == 0 && vae_aligned16(x) && vae_aligned16(out) &&
                  (!cache || vae_aligned16(cache)),
              DIFFLET_EINVAL,
              "im2col_causal: channels, strides, kpad and ldo must be multiples of %d (16 bytes), "
              "kpad >= kt ks^2 C, pointers aligned", ev);
  const int64_t ho = height << upsample, wo = width << upsample;
  DLT_REQUIRE(ho * wo < (1LL << 31) && k < (1LL << 30), DIFFLET_EUNSUPPORTED,
              "im2col_causal: frame too large");
  DLT_REQUIRE(row0 >= 0 && rows >= 0 && (row0 + rows) / (ho * wo) < (1LL << 31), DIFFLET_EINVAL,
              "im2col_causal: bad row range");
  if (rows == 0) return DIFFLET_OK;
  DLT_REQUIRE(k / ev <= IM2COL_MAX_TAB, DIFFLET_EUNSUPPORTED, "im2col_causal: too many columns");
  int64_t blocks = (rows + 3) / 4;
  if (blocks > 65536) blocks = 65536;
  const size_t tab_bytes = (size_t)(k / ev) * 4;
  DLT_DISPATCH_BF16_F32(dtype, T,
    hipLaunchKernelGGL((im2col_rows_kernel<T>), dim3((unsigned)blocks), dim3(256), tab_bytes,
                       (hipStream_t)stream, (const T*)x, frame_stride, (int)frames_per_block,
                       sub_stride, pixel_stride, (const T*)cache, (int)height, (int)width,
                       (int)channels, (int)kt, (int)ks, upsample, row0, rows, (T*)out, ldo,
                       (int)kpad));
  return dlt_check_launch("im2col_causal");
}

template <typename T, int LPR, int NV, int RB>
static void launch_rms_channels(const void* x, int64_t ldx, void* y, int64_t ldy, int64_t rows,
                                int channels, const float* gamma, float eps, int act,
                                hipStream_t s) {
  int64_t blocks = (rows * LPR + 256 * RB - 1) / (256 * RB);
  if (blocks > 16384) blocks = 16384;
  hipLaunchKernelGGL((rms_channels_kernel<T, LPR, NV, RB>), dim3((unsigned)blocks), dim3(256), 0,
                     s, (const T*)x, ldx, (T*)y, ldy, rows, channels, gamma, eps, act);
}

extern "C" int difflet_rocm_rms_norm_channels(const void* x, int64_t ldx, void* y, int64_t ldy,
                                              int dtype, int64_t rows, int64_t channels,
                                              const float* gamma, float eps, int act,
                                              difflet_stream_t stream) {
  DLT_REQUIRE(rows >= 0 && channels > 0 && channels % 8 == 0 && channels <= 2048 &&
                  ldx >= channels && ldy >= channels && (act == 0 || act == 1) && eps > 0.f,
              DIFFLET_EINVAL,
              "rms_norm_channels: channels (%lld) must be a multiple of 8, <= 2048, "
              "row strides >= channels, act 0 or 1, eps > 0", (long long)channels);
  if (rows == 0) return DIFFLET_OK;
  DLT_REQUIRE(x && y && gamma, DIFFLET_EINVAL, "rms_norm_channels: null pointer");
  const int ev = dtype == DIFFLET_F32 ? 4 : 8;
  DLT_REQUIRE(ldx % ev == 0 && ldy % ev == 0 && vae_aligned16(x) && vae_aligned16(y),
              DIFFLET_EINVAL, "rms_norm_channels: rows must be 16-byte aligned");
  hipStream_t s = (hipStream_t)stream;
  const int nvec = (int)(channels / 8);
  DLT_DISPATCH_BF16_F32(dtype, T,
    if (nvec <= 16) launch_rms_channels<T, 16, 1, 4>(x, ldx, y, ldy, rows, (int)channels, gamma, eps, act, s);
    else if (nvec <= 32) launch_rms_channels<T, 32, 1, 4>(x, ldx, y, ldy, rows, (int)channels, gamma, eps, act, s);
    else if (nvec <= 64) launch_rms_channels<T, 64, 1, 4>(x, ldx, y, ldy, rows, (int)channels, gamma, eps, act, s);
    else launch_rms_channels<T, 64, 4, 1>(x, ldx, y, ldy, rows, (int)channels, gamma, eps, act, s));
  return dlt_check_launch("rms_norm_channels");
}

extern "C" int difflet_rocm_rows_to_planes(const void* x, int64_t ld, int dtype, int64_t n,
                                           int64_t channels, void* out, float lo, float hi,
                                           difflet_stream_t stream) {
  DLT_REQUIRE(n >= 0 && channels > 0 && ld >= channels && lo <= hi, DIFFLET_EINVAL,
              "rows_to_planes: bad sizes");
  if (n == 0) return DIFFLET_OK;
  DLT_REQUIRE(x && out, DIFFLET_EINVAL, "rows_to_planes: null pointer");
  int64_t blocks = (n + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  DLT_DISPATCH_BF16_F32(dtype, T,
    hipLaunchKernelGGL((rows_to_planes_kernel<T>), dim3((unsigned)blocks), dim3(256), 0,
                       (hipStream_t)stream, (const T*)x, ld, n, (int)channels, (T*)out, lo, hi));
  return dlt_check_launch("rows_to_planes");
}
