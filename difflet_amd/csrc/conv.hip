// The VAE decoders' convolutions as implicit GEMMs on the bf16 matrix cores: the GEMM of the
// im2col rows with the packed weight, where each K stage gathers its 64 columns of the im2col
// rows straight from the channels-last frames into the LDS, so the rows (9 C or 27 C columns per
// output pixel) are never written to memory. fp32 convolutions take the fp32 GEMM with the same
// gather in its register-staged loader (launch_conv_f32, gemm_f32.hip).
//
// The convolution is WanCausalConv3d (difflet/models/wan/vae/modeling_vae.py:95-134: kernel
// (kt, ks, ks), kt - 1 frames of zero or cached padding in front, ks / 2 pixels around), the
// resampler's per-frame nn.Conv2d(3, padding=1) after a nearest 2x upsampling (:163-226), and
// with kt = 1 on one frame the FLUX decoder's 3x3 convolutions. Column k of an output pixel's row
// is tap (dt, ky, kx) = k / C and channel k % C, taps in (dt, ky, kx) order, the weight's layout
// [Cout][kt][ks][ks][C] (zero past kt ks^2 C).
//
// Tiles: 8 waves, WMW along the output pixels and 8 / WMW along the output channels, each wave 64
// pixels x 32 NJ channels (2 x NJ MFMA 32x32x16 tiles). Cout <= 96 runs one channel tile of
// 32 NJ with 512 pixels (the 96-channel full-resolution stage: no MFMA column wasted); wider
// convolutions run 256 x 192 or 256 x 128 tiles. A stage is 64 K elements (128 bytes) of every
// row, staged by direct-to-LDS buffer loads in two LDS slots, 8 rows x 128 B per load
// instruction, chunk c of row r at c ^ swz8(r) as in the GEMM kernel. Each lane's 16-byte chunk
// of an A row is 8 channels of one tap of one pixel (C is a multiple of 8), so its address is the
// pixel's shifted position in its frame: out-of-frame taps, padding columns and rows past the
// end take an offset past the buffer, which the load's range check turns into zeros.

#include "common.hpp"

namespace dlt {
namespace {

__device__ __forceinline__ int swz8(int row) { return (row & 7) ^ ((row >> 3) & 1); }
__device__ __forceinline__ int lds_off8(int row, int chunk) {
  return row * 128 + ((chunk ^ swz8(row)) << 4);
}

}  // namespace

struct ConvArgs {
  const uint8_t* x;  // the input frames, x_bytes long
  const uint8_t* w;  // [n][kpad] bf16
  const bf16* bias;  // [n] or null
  const bf16* res;   // [rows][ldr] or null
  bf16* out;         // [rows][ldo]
  uint32_t x_bytes;
  uint32_t rows;                 // output pixels: frames x ho x wo
  uint32_t fstride_b, sub_b, ld_b;  // frame-block, sub-frame and pixel strides of x, bytes
  int lfpb;                      // log2 of frames per block
  int fbase;                     // buffer frame of output frame t's tap dt: t + dt + fbase
  int w_in, ho, wo, up, half, ks, kt;
  uint32_t po, po_m, wo_m;       // pixels per output frame; magic numbers of po and wo
  uint32_t cin, cin_m;
  int ktot, nk;                  // kt ks^2 C; K stages (kpad / 64)
  int n;                         // output channels (weight rows)
  uint32_t ldw_b;                // weight row bytes
  int64_t ldr, ldo;
  int tiles_n, tiles;  // channel tiles across; workgroups (tiles x ksplit)
  int ksplit;          // K ranges per tile: > 1 writes fp32 partial sums to ws
  float* ws;           // [ksplit][rows][n]
};

constexpr uint32_t kOutside = 0x80000000u;  // an offset past every buffer (x_bytes < 2^31)

// LIN: no upsampling, so a tap moves every pixel by the same offset: each A row keeps its
// pixel's byte offset and a bit per tap that is inside the frames, and a load is that offset
// plus the chunk's tap offset when the bit is set (4 VALU operations instead of about 15)
template <int WMW, int NJ, bool LIN>
__global__ __launch_bounds__(512, 1) void conv_igemm_kernel(const ConvArgs a) {
  constexpr int WNW = 8 / WMW;
  constexpr int BM = 64 * WMW, BN = 32 * NJ * WNW;
  constexpr int SA = BM / 64;  // A slabs (8 rows x 128 B) per wave and stage
  constexpr int SW = BN / 8;   // W slabs per stage, wave w taking w, w + 8, ...
  constexpr int NWJ = (SW + 7) / 8;
  constexpr int SLOT = (BM + BN) * 128;
  static_assert(SA % 2 == 0 && SA <= 8 && NWJ <= 3 && NJ <= 3 && 2 * SLOT <= 160 * 1024,
                "tile does not fit the LDS");
  __shared__ __attribute__((aligned(16))) uint8_t lds[2 * SLOT];
  typedef __attribute__((address_space(3))) void lds_void;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave % WMW, wn = wave / WMW;

  // workgroups go round-robin over the 8 XCDs: give each XCD a contiguous run of tiles, so the
  // pixels it convolves at once (and their neighbours the taps read) share its L2
  int tile;
  {
    const int bid = blockIdx.x, per = a.tiles >> 3, rem = a.tiles & 7, xc = bid & 7, i = bid >> 3;
    tile = xc < rem ? xc * (per + 1) + i : rem * (per + 1) + (xc - rem) * per + i;
  }
  // a tile's K stages [kbeg, kend): all of them, or range `piece` of ksplit
  const int piece = tile % a.ksplit;
  tile /= a.ksplit;
  const int kbeg = piece * a.nk / a.ksplit, kend = (piece + 1) * a.nk / a.ksplit;
  const int tm = tile / a.tiles_n, tn = tile - tm * a.tiles_n;
  const uint32_t m0 = (uint32_t)tm * BM;
  const int n0 = tn * BN;

  const __amdgpu_buffer_rsrc_t rx = make_rsrc(a.x, a.x_bytes);
  const __amdgpu_buffer_rsrc_t rw =
      make_rsrc(a.w + (int64_t)n0 * a.ldw_b, (uint32_t)(a.n - n0) * a.ldw_b);

  // A load i of this lane fills row (wave SA + i) 8 + lane / 8 of the stage, physical chunk
  // lane % 8, i.e. logical chunk lc0 ^ (i & 1): its output pixel (frame, y, x), y far outside
  // the frame past the last row
  const int lc0 = (lane & 7) ^ (lane >> 3);
  // arrays whose elements reach target builtins are sized for the largest tile, not by SA, NWJ
  // or NJ: with a template-dependent size the host pass drops the kernel's launch stub
  int rt[8], ry[8], rxp[8];  // LIN: rt = the pixel's byte offset at tap (0, half, half),
                             // ry = the bits of the taps inside the frames
#pragma unroll
  for (int i = 0; i < SA; ++i) {
    const uint32_t R = m0 + (uint32_t)((wave * SA + i) * 8 + (lane >> 3));
    uint32_t p, xx;
    const uint32_t t = conv_udiv(R, a.po, a.po_m, p);
    const uint32_t y = conv_udiv(p, (uint32_t)a.wo, a.wo_m, xx);
    const bool in = R < a.rows;
    if constexpr (LIN) {
      // the taps (dt, ky, kx) inside: rows y + ky - half and columns x + kx - half of the
      // frame, buffer frames t + dt + fbase >= 0; bit (dt ks + ky) ks + kx
      const int b = (int)t + a.fbase;
      uint32_t cols = 0, rows = 0, frames = 0;
#pragma unroll
      for (int q = 0; q < 3; ++q) {
        const int d = q - a.half;
        cols |= (q < a.ks && (uint32_t)((int)xx + d) < (uint32_t)a.wo) ? 1u << q : 0u;
        rows |= (q < a.ks && (uint32_t)((int)y + d) < (uint32_t)a.ho) ? 1u << q : 0u;
        frames |= (q < a.kt && b + q >= 0) ? 1u << q : 0u;
      }
      uint32_t plane = 0;  // the ks x ks taps of one frame
#pragma unroll
      for (int q = 0; q < 3; ++q) plane |= (rows >> q & 1u) ? cols << (q * a.ks) : 0u;
      uint32_t m = 0;
#pragma unroll
      for (int q = 0; q < 3; ++q) m |= (frames >> q & 1u) ? plane << (q * a.ks * a.ks) : 0u;
      // modulo 2^32 (b < 0 before a causal convolution's first frames, t past the last row):
      // every offset a set bit selects is in range
      rt[i] = (int)((uint32_t)(b >> a.lfpb) * a.fstride_b +
                    (uint32_t)(b & ((1 << a.lfpb) - 1)) * a.sub_b +
                    (y * (uint32_t)a.w_in + xx) * a.ld_b);
      ry[i] = in ? (int)m : 0;
      rxp[i] = 0;
    } else {
      rt[i] = (int)t;
      ry[i] = in ? (int)y : -(1 << 24);
      rxp[i] = (int)xx;
    }
  }
  uint32_t w_off[3];
#pragma unroll
  for (int j = 0; j < NWJ; ++j) {
    const int s = wave + 8 * j;
    const int r = s * 8 + (lane >> 3);
    w_off[j] = (uint32_t)r * a.ldw_b + (uint32_t)(((lane & 7) ^ swz8(r)) << 4);
  }

  // column chunk lc of stage kt: its tap as a frame offset and a pixel shift, and its channel
  // byte offset (padding columns: a shift that leaves every frame)
  // (LIN: fo = the tap's bit, 31 past the real columns; cb = its byte offset with the channel's)
  struct Tap {
    int fo, dy, dx;
    uint32_t cb;
  };
  auto tap_of = [&](int kt, int lc) {
    const uint32_t kk = (uint32_t)(kt * 64 + lc * 8);
    uint32_t c;
    const int tap = (int)conv_udiv(kk, a.cin, a.cin_m, c);
    int dt, ky, kx;
    conv_tap(tap, a.ks, dt, ky, kx);
    Tap o;
    if constexpr (LIN) {
      o.fo = (int)kk < a.ktot ? tap : 31;
      o.dy = o.dx = 0;
      o.cb = (uint32_t)(dt >> a.lfpb) * a.fstride_b +
             (uint32_t)((ky - a.half) * a.w_in + (kx - a.half)) * a.ld_b + c * 2;
    } else {
      o.fo = dt + a.fbase;
      o.dy = (int)kk < a.ktot ? ky - a.half : -(1 << 24);
      o.dx = kx - a.half;
      o.cb = c * 2;
    }
    return o;
  };
  auto a_off = [&](int i, const Tap& tp) {
    if constexpr (LIN)
      return ((uint32_t)ry[i] >> tp.fo & 1u) ? (uint32_t)rt[i] + tp.cb : kOutside;
    const int f = rt[i] + tp.fo, yy = ry[i] + tp.dy, xs = rxp[i] + tp.dx;
    const bool ok = (uint32_t)yy < (uint32_t)a.ho && (uint32_t)xs < (uint32_t)a.wo && f >= 0;
    const uint32_t pix = (uint32_t)(yy >> a.up) * (uint32_t)a.w_in + (uint32_t)(xs >> a.up);
    const uint32_t off = (uint32_t)(f >> a.lfpb) * a.fstride_b +
                         (uint32_t)(f & ((1 << a.lfpb) - 1)) * a.sub_b + pix * a.ld_b + tp.cb;
    return ok ? off : kOutside;
  };
  // part p (of 2) of stage kt's loads into slot st: A loads [p SA / 2, (p + 1) SA / 2), and with
  // part 1 this wave's W slabs
  Tap tp0, tp1;
  auto issue_part = [&](int kt, int st, int p) {
    uint8_t* sl = lds + st * SLOT;
    if (p == 0) {
      tp0 = tap_of(kt, lc0);
      tp1 = tap_of(kt, lc0 ^ 1);
    }
#pragma unroll
    for (int i = p * SA / 2; i < (p + 1) * SA / 2; ++i) {
      // a named offset: with the call inside the builtin's arguments the host pass drops the
      // launch stub
      const uint32_t off = a_off(i, (i & 1) ? tp1 : tp0);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rx, (lds_void*)(sl + (wave * SA + i) * 1024), 16,
                                               off, 0, 0, 0);
    }
    if (p == 1) {
#pragma unroll
      for (int j = 0; j < NWJ; ++j)
        if (wave + 8 * j < SW)
          __builtin_amdgcn_raw_ptr_buffer_load_lds(
              rw, (lds_void*)(sl + BM * 128 + (wave + 8 * j) * 1024), 16, w_off[j],
              (uint32_t)kt * 128, 0, 0);
    }
  };

  f32x16 acc[2][3];  // columns j < NJ used (fixed sizes: see rt above)
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < NJ; ++j) acc[i][j] = f32x16{};

  const int frow = lane & 31, fhalf = lane >> 5;
  i32x4 fa[2], fw[2][3];
  auto read_a = [&](int st, int ks, int i) {
    const uint8_t* sA = lds + st * SLOT;
    fa[i] = *reinterpret_cast<const i32x4*>(sA + lds_off8(wm * 64 + i * 32 + frow, 2 * ks + fhalf));
  };
  auto read_w = [&](int st, int ks, int set) {
    const uint8_t* sW = lds + st * SLOT + BM * 128;
#pragma unroll
    for (int j = 0; j < NJ; ++j)
      fw[set][j] = *reinterpret_cast<const i32x4*>(
          sW + lds_off8(wn * 32 * NJ + j * 32 + frow, 2 * ks + fhalf));
  };
  // D[channel][pixel]: the weight fragment is the first operand, as in the GEMM kernel, so the
  // products and their order match the im2col GEMM's
  auto mma_tile = [&](int set, int i) {
#pragma unroll
    for (int j = 0; j < NJ; ++j)
      acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, fw[set][j]),
                                                          __builtin_bit_cast(bf16x8, fa[i]),
                                                          acc[i][j], 0, 0, 0);
  };

  // Stage 0 lands before the loop; stage kt + 1 is in flight while stage kt computes. Before the
  // last K step of stage kt every wave waits for its loads (stage kt + 1's, the only ones in
  // flight) and its LDS reads, and one barrier publishes stage kt + 1 and frees slot kt & 1 for
  // stage kt + 2, whose loads go out with the last K step's MFMAs.
  issue_part(kbeg, 0, 0);
  issue_part(kbeg, 0, 1);
  __builtin_amdgcn_s_waitcnt(0x0070);  // vmcnt(0) lgkmcnt(0)
  __syncthreads();
  if (kend - kbeg > 1) {
    issue_part(kbeg + 1, 1, 0);
    issue_part(kbeg + 1, 1, 1);
  }
  read_w(0, 0, 0);
  read_a(0, 0, 0);
  read_a(0, 0, 1);
  for (int kt = kbeg; kt < kend; ++kt) {
    const int st = (kt - kbeg) & 1;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      const int set = ks & 1;
      const bool last = ks == 3;
      const int nst = last ? (st ^ 1) : st, nks = last ? 0 : ks + 1;
      const bool loads = last && kt + 2 < kend;
      if (last) {
        __builtin_amdgcn_s_waitcnt(0x0070);
        asm volatile("s_barrier" ::: "memory");
      }
      read_w(nst, nks, set ^ 1);
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        mma_tile(set, i);
        read_a(nst, nks, i);
        if (loads) issue_part(kt + 2, st, i);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  }

  // ---- epilogue: lane holds pixel m0 + wm 64 + 32 i + (lane & 31) and, per group g, the four
  // channels 8 g + 4 (lane >> 5) .. + 3 of each 32-channel tile: + bias (+ residual), rounded once
  // (a K range: the fp32 partial sums, which conv_split_reduce_kernel adds up)
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const uint32_t R = m0 + (uint32_t)(wm * 64 + i * 32 + frow);
    if (R >= a.rows) continue;
    if (a.ksplit > 1) {
#pragma unroll
      for (int j = 0; j < NJ; ++j)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int c = n0 + wn * 32 * NJ + j * 32 + g * 8 + fhalf * 4;
          if (c >= a.n) continue;
          const f32x4 v = {acc[i][j][g * 4], acc[i][j][g * 4 + 1], acc[i][j][g * 4 + 2],
                           acc[i][j][g * 4 + 3]};
          *reinterpret_cast<f32x4*>(a.ws + ((int64_t)piece * a.rows + R) * a.n + c) = v;
        }
      continue;
    }
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int c = n0 + wn * 32 * NJ + j * 32 + g * 8 + fhalf * 4;
        if (c >= a.n) continue;
        float v[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) v[q] = acc[i][j][g * 4 + q];
        if (a.bias) {
          const u32x2 b = *reinterpret_cast<const u32x2*>(a.bias + c);
          v[0] += bf16bits_to_f32(b[0] & 0xffffu);
          v[1] += bf16bits_to_f32(b[0] >> 16);
          v[2] += bf16bits_to_f32(b[1] & 0xffffu);
          v[3] += bf16bits_to_f32(b[1] >> 16);
        }
        if (a.res) {
          const u32x2 r = *reinterpret_cast<const u32x2*>(a.res + (int64_t)R * a.ldr + c);
          v[0] += bf16bits_to_f32(r[0] & 0xffffu);
          v[1] += bf16bits_to_f32(r[0] >> 16);
          v[2] += bf16bits_to_f32(r[1] & 0xffffu);
          v[3] += bf16bits_to_f32(r[1] >> 16);
        }
        const u32x2 o = {pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
        *reinterpret_cast<u32x2*>(a.out + (int64_t)R * a.ldo + c) = o;
      }
    }
  }
}

// out[r][c..c+3] = sum over the K ranges in order of ws[p][r][c..c+3] + bias (+ residual),
// rounded once: one thread per 4 channels of a row
__global__ __launch_bounds__(256) void conv_split_reduce_kernel(const float* __restrict__ ws,
                                                                int ksplit, uint32_t rows, int n,
                                                                const bf16* __restrict__ bias,
                                                                const bf16* res, int64_t ldr,
                                                                bf16* out, int64_t ldo) {
  const int ng = n >> 2;
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= (int64_t)rows * ng) return;
  const int64_t r = i / ng;
  const int c = (int)(i - r * ng) * 4;
  f32x4 v = *reinterpret_cast<const f32x4*>(ws + r * n + c);
  for (int p = 1; p < ksplit; ++p)
    v += *reinterpret_cast<const f32x4*>(ws + ((int64_t)p * rows + r) * n + c);
  float o[4] = {v[0], v[1], v[2], v[3]};
  if (bias) {
    const u32x2 b = *reinterpret_cast<const u32x2*>(bias + c);
    o[0] += bf16bits_to_f32(b[0] & 0xffffu);
    o[1] += bf16bits_to_f32(b[0] >> 16);
    o[2] += bf16bits_to_f32(b[1] & 0xffffu);
    o[3] += bf16bits_to_f32(b[1] >> 16);
  }
  if (res) {
    const u32x2 q = *reinterpret_cast<const u32x2*>(res + r * ldr + c);
    o[0] += bf16bits_to_f32(q[0] & 0xffffu);
    o[1] += bf16bits_to_f32(q[0] >> 16);
    o[2] += bf16bits_to_f32(q[1] & 0xffffu);
    o[3] += bf16bits_to_f32(q[1] >> 16);
  }
  const u32x2 w = {pack_bf16x2(o[0], o[1]), pack_bf16x2(o[2], o[3])};
  *reinterpret_cast<u32x2*>(out + r * ldo + c) = w;
}

namespace {

// The tile for n output channels, as (WMW, NJ): the widest that wastes little, 512 x 32 NJ up to
// 96 channels, 256 x 128 up to 128, then 256 x 192 unless rounding up to 192 adds over an eighth
// (256 channels: two 256 x 128).
void conv_tile(int64_t n, int& wmw, int& nj) {
  if (n <= 96) {
    wmw = 8;
    nj = (int)((n + 31) / 32);
  } else if (n <= 128 || (n + 191) / 192 * 192 * 8 > 9 * n) {
    wmw = 4;
    nj = 2;
  } else {
    wmw = 4;
    nj = 3;
  }
}

// Compute units of the current device (0 without one: then nothing is split).
int conv_device_cus() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  if (cached[dev] == 0) {
    int v = 0;
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
      return 0;
    cached[dev] = v;
  }
  return cached[dev];
}

struct ConvPlan {
  int wmw, nj, tiles_n, ksplit;
  int64_t tiles;  // whole tiles
};

// A launch of under half a wave of tiles (the 60 x 104 latent-resolution convolutions: 50
// tiles, K = 10368) cuts each tile's K stages into up to 8 ranges of at least 8 stages, so about
// one wave of workgroups runs; the ranges' fp32 partial sums meet in a second kernel.
ConvPlan conv_plan(int64_t rows, int64_t n, int64_t kpad, int cus) {
  ConvPlan p;
  conv_tile(n, p.wmw, p.nj);
  const int bm = 64 * p.wmw, bn = 32 * p.nj * (8 / p.wmw);
  p.tiles_n = (int)((n + bn - 1) / bn);
  p.tiles = (rows + bm - 1) / bm * p.tiles_n;
  p.ksplit = 1;
  const int64_t nk = kpad / 64;
  if (p.tiles > 0 && 2 * p.tiles < cus) {
    int64_t k = cus / p.tiles;
    if (k > 8) k = 8;
    if (k > nk / 8) k = nk / 8;
    if (k > 1) p.ksplit = (int)k;
  }
  return p;
}

int64_t conv_ws_bytes(const ConvPlan& p, int64_t rows, int64_t n) {
  return p.ksplit > 1 ? (int64_t)p.ksplit * rows * n * 4 : 0;
}

bool aligned(const void* p, uintptr_t a) { return ((uintptr_t)p & (a - 1)) == 0; }

}  // namespace
}  // namespace dlt

using namespace dlt;

extern "C" int difflet_rocm_conv_causal(const void* x, int64_t x_elems, int64_t frame_stride,
                                        int64_t frames_per_block, int64_t sub_stride,
                                        int64_t pixel_stride, int64_t lead_frames, int dtype,
                                        int64_t height, int64_t width, int64_t channels,
                                        int64_t kt, int64_t ks, int upsample, int64_t frames,
                                        const void* w, int64_t n, int64_t kpad, const void* bias,
                                        const void* residual, int64_t ldr, void* out,
                                        int64_t ldo, void* workspace, int64_t workspace_bytes,
                                        difflet_stream_t stream) {
  DLT_REQUIRE(dtype == DIFFLET_BF16 || dtype == DIFFLET_F32, DIFFLET_EUNSUPPORTED,
              "conv_causal: bf16 or fp32");
  DLT_REQUIRE(height > 0 && width > 0 && channels > 0 && frames >= 0 && n > 0 &&
                  (upsample == 0 || upsample == 1) && (kt == 1 || kt == 3) &&
                  (ks == 1 || ks == 3) && (frames_per_block == 1 || frames_per_block == 2) &&
                  lead_frames >= 0 && lead_frames <= 2,
              DIFFLET_EINVAL, "conv_causal: bad sizes or taps (kt, ks in {1, 3})");
  DLT_REQUIRE(x && w && out, DIFFLET_EINVAL, "conv_causal: null pointer");
  const bool f32 = dtype == DIFFLET_F32;
  const int ev = f32 ? 4 : 8, kq = f32 ? 4 : 64;  // elements per 16 bytes; the K stage multiple
  const int64_t k = kt * ks * ks * channels;
  DLT_REQUIRE(channels % ev == 0 && pixel_stride >= channels && pixel_stride % ev == 0 &&
                  sub_stride % ev == 0 && frame_stride % ev == 0 && kpad % kq == 0 && kpad >= k &&
                  n % 4 == 0 && ldo >= n && ldo % 4 == 0 &&
                  (!residual || (ldr >= n && ldr % 4 == 0 && aligned(residual, 2 * ev))) &&
                  (!bias || aligned(bias, 2 * ev)) && aligned(x, 16) && aligned(w, 16) &&
                  aligned(out, 2 * ev),
              DIFFLET_EINVAL,
              "conv_causal: channels and strides multiples of 16 bytes, kpad a multiple of %d "
              ">= kt ks^2 C, n, ldo, ldr multiples of 4, pointers aligned (x, w: 16 bytes; "
              "bias, residual, out: 4 elements)", kq);
  const int64_t ho = height << upsample, wo = width << upsample, po = ho * wo;
  const int64_t rows = frames * po;
  DLT_REQUIRE(rows < (1LL << 31) && k < (1LL << 24) &&
                  (f32 || (x_elems * 2 < (1LL << 31) && n * kpad * 2 < (1LL << 32))),
              DIFFLET_EUNSUPPORTED,
              "conv_causal: the output must hold under 2^31 pixels (bf16: the frames span under "
              "2 GiB)");
  if (rows == 0) return DIFFLET_OK;
  {  // every frame the taps read lies inside x
    const int64_t last = frames - 1 + lead_frames;
    const int64_t end = (last / frames_per_block) * frame_stride +
                        (last % frames_per_block) * sub_stride +
                        (height * width - 1) * pixel_stride + channels;
    DLT_REQUIRE(end <= x_elems, DIFFLET_EINVAL,
                "conv_causal: frames 0..%lld of the input overrun x (%lld elements)",
                (long long)last, (long long)x_elems);
  }
  hipStream_t s = (hipStream_t)stream;
  if (f32) {
    ConvGeo g;
    g.fstride = frame_stride;
    g.sub = sub_stride;
    g.ld = pixel_stride;
    g.lfpb = frames_per_block == 2 ? 1 : 0;
    g.fbase = (int)(lead_frames - (kt - 1));
    g.w = (int)width;
    g.ho = (int)ho;
    g.wo = (int)wo;
    g.up = upsample;
    g.half = (int)(ks / 2);
    g.ks = (int)ks;
    g.po = (uint32_t)po;
    g.po_m = conv_magic((uint32_t)po);
    g.wo_m = conv_magic((uint32_t)wo);
    g.cin = (uint32_t)channels;
    g.cin_m = conv_magic((uint32_t)channels);
    g.ktot = (int)k;
    return launch_conv_f32((const float*)x, g, rows, (const float*)w, n, kpad,
                           (const float*)bias, (const float*)residual, ldr, (float*)out, ldo, s);
  }
  ConvArgs a;
  a.x = (const uint8_t*)x;
  a.w = (const uint8_t*)w;
  a.bias = (const bf16*)bias;
  a.res = (const bf16*)residual;
  a.out = (bf16*)out;
  a.x_bytes = (uint32_t)(x_elems * 2);
  a.rows = (uint32_t)rows;
  a.fstride_b = (uint32_t)(frame_stride * 2);
  a.sub_b = (uint32_t)(sub_stride * 2);
  a.ld_b = (uint32_t)(pixel_stride * 2);
  a.lfpb = frames_per_block == 2 ? 1 : 0;
  a.fbase = (int)(lead_frames - (kt - 1));
  a.w_in = (int)width;
  a.ho = (int)ho;
  a.wo = (int)wo;
  a.up = upsample;
  a.half = (int)(ks / 2);
  a.ks = (int)ks;
  a.kt = (int)kt;
  a.po = (uint32_t)po;
  a.po_m = conv_magic((uint32_t)po);
  a.wo_m = conv_magic((uint32_t)wo);
  a.cin = (uint32_t)channels;
  a.cin_m = conv_magic((uint32_t)channels);
  a.ktot = (int)k;
  a.nk = (int)(kpad / 64);
  a.n = (int)n;
  a.ldw_b = (uint32_t)(kpad * 2);
  a.ldr = ldr;
  a.ldo = ldo;
  ConvPlan plan = conv_plan(rows, n, kpad, conv_device_cus());
  if (conv_ws_bytes(plan, rows, n) > workspace_bytes || !aligned(workspace, 16)) plan.ksplit = 1;
  a.tiles_n = plan.tiles_n;
  a.ksplit = plan.ksplit;
  a.ws = (float*)workspace;
  a.tiles = (int)(plan.tiles * plan.ksplit);
  const dim3 grid((unsigned)a.tiles), block(512);
  // taps at fixed pixel offsets unless the frames are upsampled (or read as interleaved pairs
  // by a kernel that spans frames)
  const bool lin = upsample == 0 && (frames_per_block == 1 || kt == 1);
#define DLT_CONV_LAUNCH(W, J)                                                      \
  do {                                                                             \
    if (lin)                                                                       \
      hipLaunchKernelGGL((conv_igemm_kernel<W, J, true>), grid, block, 0, s, a);  \
    else                                                                           \
      hipLaunchKernelGGL((conv_igemm_kernel<W, J, false>), grid, block, 0, s, a); \
  } while (0)
  if (plan.wmw == 8 && plan.nj == 1)
    DLT_CONV_LAUNCH(8, 1);
  else if (plan.wmw == 8 && plan.nj == 2)
    DLT_CONV_LAUNCH(8, 2);
  else if (plan.wmw == 8)
    DLT_CONV_LAUNCH(8, 3);
  else if (plan.nj == 2)
    DLT_CONV_LAUNCH(4, 2);
  else
    DLT_CONV_LAUNCH(4, 3);
#undef DLT_CONV_LAUNCH
  if (plan.ksplit > 1) {
    const int64_t items = rows * (n / 4);
    hipLaunchKernelGGL(conv_split_reduce_kernel, dim3((unsigned)((items + 255) / 256)), dim3(256),
                       0, s, (const float*)workspace, plan.ksplit, (uint32_t)rows, (int)n,
                       (const bf16*)bias, (const bf16*)residual, ldr, (bf16*)out, ldo);
  }
  return dlt_check_launch("conv_causal");
}

extern "C" int64_t difflet_rocm_conv_causal_workspace_bytes(int64_t rows, int64_t n,
                                                            int64_t kpad) {
  if (rows <= 0 || n <= 0 || kpad <= 0) return 0;
  return conv_ws_bytes(conv_plan(rows, n, kpad, conv_device_cus()), rows, n);
}
