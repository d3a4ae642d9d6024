// GEMMs of the DiT block on CDNA4 matrix cores: C = epilogue(A W^T + bias).
//
// A [M, K] and W [N, K] are both K-contiguous (activations and nn.Linear weights as stored).
// One kernel skeleton serves three element types:
//   bf16  : v_mfma_f32_32x32x16_bf16, 64 K-elements (128 bytes) per K tile;
//   fp8   : v_mfma_f32_32x32x64_f8f6f4 (e4m3), 128 K-elements per K tile, per-row scales of A
//           and W applied in the epilogue (acc * sa[m] * sw[n]);
//   mxfp8 : v_mfma_scale_f32_32x32x64_f8f6f4 with one E8M0 scale per 32-element block of a
//           row (the block split over the two lane groups, see the K loop), 128 K per K tile.
// A K tile is therefore always 128 bytes per row, and the LDS geometry is shared.
//
// Tiling: a 256-thread workgroup (4 wavefronts in a 2 x 2 grid) owns a 256 x 256 tile of C;
// each wavefront owns 128 x 128 = 4 x 4 MFMA tiles of 32 x 32, 256 fp32 accumulators per lane.
// The MFMA's first operand is the W tile and its second the A tile, so accumulator lane l holds
// row m = l % 32 and registers run along n in groups of 4 consecutive columns: the epilogue
// reads bias / gate / residual and writes C in 8-byte pieces.
//
// LDS: two stages of (A tile + W tile) = 2 x 64 KB. A row of a K tile is 8 chunks of 16 bytes;
// chunk c of row r lives at chunk c ^ (r & 7), so the 8 lanes an ds_read_b128 serves together
// (8 consecutive rows, one chunk) hit 8 different bank groups. Global loads are raw buffer
// loads: rows past M (or N) read as zero, so ragged edges need no branches.
//
// Tile order: workgroup ids are spread round-robin over the 8 XCDs, each with its own L2. The id
// is remapped so each XCD gets a contiguous run of tiles, and tiles run in groups of 8 tile rows
// so the W and A panels of neighbouring tiles stay L2-resident.
#include "common.hpp"

namespace dlt {

constexpr int BM = 256, BN = 256, KT_BYTES = 128, NTHREADS = 256;
constexpr int MAX_PROBLEMS = 4;
constexpr int GROUP_M = 8;

enum class Elem { BF16, FP8, MX };

struct GemmProblemDev {
  const uint8_t* a;
  const uint8_t* w;
  uint8_t* c;
  const bf16* bias;
  const bf16* gate;
  const bf16* res;
  const void* a_scale;
  const void* w_scale;
  int64_t lda, ldw, ldc, ldr, gate_stride;  // element strides (A / W in elements of Elem)
  int64_t m, rows_per_batch;
  int tiles_m, tile_start;
};

struct GemmArgs {
  GemmProblemDev p[MAX_PROBLEMS];
  int nprob, total_tiles, tiles_n;
  int n, k;
  int act_col_start;
};

template <Elem E> struct ElemTraits;
template <> struct ElemTraits<Elem::BF16> { static constexpr int KT = 64, BYTES = 2; };
template <> struct ElemTraits<Elem::FP8> { static constexpr int KT = 128, BYTES = 1; };
template <> struct ElemTraits<Elem::MX> { static constexpr int KT = 128, BYTES = 1; };

__device__ __forceinline__ int lds_off(int row, int chunk) {
  return row * KT_BYTES + ((chunk ^ (row & 7)) << 4);
}

template <Elem E, int EPI>
__global__ __launch_bounds__(NTHREADS, 1) void gemm_kernel(const GemmArgs args) {
  constexpr int KT = ElemTraits<E>::KT;
  constexpr int EB = ElemTraits<E>::BYTES;
  __shared__ __attribute__((aligned(16))) uint8_t smem[2][2][BM * KT_BYTES];  // [stage][A|W]

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;

  // ---- tile assignment: XCD-contiguous runs, then grouped raster
  int bid = blockIdx.x;
  const int T = args.total_tiles;
  if ((T & 7) == 0) bid = (bid & 7) * (T >> 3) + (bid >> 3);
  int p = 0;
#pragma unroll
  for (int i = 1; i < MAX_PROBLEMS; ++i)
    if (i < args.nprob && bid >= args.p[i].tile_start) p = i;
  const GemmProblemDev& P = args.p[p];
  int t = bid - P.tile_start;
  const int tn_count = args.tiles_n;
  const int group_size = GROUP_M * tn_count;
  const int g = t / group_size;
  const int first_m = g * GROUP_M;
  const int gm = min(P.tiles_m - first_m, GROUP_M);
  const int tm = first_m + (t % group_size) % gm;
  const int tn = (t % group_size) / gm;
  const int64_t m0 = (int64_t)tm * BM;
  const int64_t n0 = (int64_t)tn * BN;
  const int M = (int)P.m, N = args.n, K = args.k;

  // ---- buffer resources: this tile's A rows and W rows (out-of-range rows read zero)
  const int64_t a_row_bytes = P.lda * EB, w_row_bytes = P.ldw * EB;
  const int64_t a_valid = (int64_t)(M - m0) * a_row_bytes;
  const int64_t w_valid = (int64_t)(N - n0) * w_row_bytes;
  const __amdgpu_buffer_rsrc_t ra =
      make_rsrc(P.a + m0 * a_row_bytes, (uint32_t)min(a_valid, (int64_t)0xffffffff));
  const __amdgpu_buffer_rsrc_t rw =
      make_rsrc(P.w + n0 * w_row_bytes, (uint32_t)min(w_valid, (int64_t)0xffffffff));

  // thread t stages chunks (row = t/8 + 32 i, chunk = t % 8), i = 0..7, of both tiles
  const int srow = tid >> 3, schunk = tid & 7;
  u32x4 ga[8], gw[8];
  auto load_global = [&](int kt) {
    const uint32_t kb = (uint32_t)kt * KT_BYTES + schunk * 16;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int r = srow + 32 * i;
      ga[i] = buf_load16(ra, (uint32_t)(r * a_row_bytes) + kb);
      gw[i] = buf_load16(rw, (uint32_t)(r * w_row_bytes) + kb);
    }
  };
  auto store_lds = [&](int st) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int r = srow + 32 * i;
      *reinterpret_cast<u32x4*>(&smem[st][0][lds_off(r, schunk)]) = ga[i];
      *reinterpret_cast<u32x4*>(&smem[st][1][lds_off(r, schunk)]) = gw[i];
    }
  };

  // ---- MX scales: one dword per row per K tile holds the tile's 4 block scales
  const int ksb = K / 32;  // scale row stride (blocks per row)
  uint32_t sa_w[4], sw_w[4];
  auto load_scales = [&](int kt) {
    if constexpr (E == Elem::MX) {
      const uint8_t* as = (const uint8_t*)P.a_scale;
      const uint8_t* ws = (const uint8_t*)P.w_scale;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int64_t mr = m0 + wm * 128 + i * 32 + (lane & 31);
        const int64_t nr = n0 + wn * 128 + i * 32 + (lane & 31);
        sa_w[i] = mr < M ? *reinterpret_cast<const uint32_t*>(as + mr * ksb + kt * 4) : 0u;
        sw_w[i] = nr < N ? *reinterpret_cast<const uint32_t*>(ws + nr * ksb + kt * 4) : 0u;
      }
    }
  };

  f32x16 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x16{};

  const int nkt = K / KT;
  load_global(0);
  load_scales(0);
  store_lds(0);
  __syncthreads();

  const int frow = lane & 31;  // fragment row within a 32-row MFMA tile
  const int fhalf = lane >> 5;
  for (int kt = 0; kt < nkt; ++kt) {
    const int st = kt & 1;
    uint32_t cur_sa[4], cur_sw[4];
    if constexpr (E == Elem::MX) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        cur_sa[i] = sa_w[i];
        cur_sw[i] = sw_w[i];
      }
    }
    if (kt + 1 < nkt) {
      load_global(kt + 1);
      load_scales(kt + 1);
    }
    const uint8_t* sA = smem[st][0];
    const uint8_t* sW = smem[st][1];
    if constexpr (E == Elem::BF16) {
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {  // 16 K per step
        const int chunk = ks * 2 + fhalf;
        bf16x8 fa[4], fw[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          fa[i] = *reinterpret_cast<const bf16x8*>(sA + lds_off(wm * 128 + i * 32 + frow, chunk));
          fw[i] = *reinterpret_cast<const bf16x8*>(sW + lds_off(wn * 128 + i * 32 + frow, chunk));
        }
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int j = 0; j < 4; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fw[j], fa[i], acc[i][j], 0, 0, 0);
      }
    } else {
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        // 64 K per step = two 32-K blocks b0 | b1 (chunks 4ks..4ks+1 | 4ks+2..4ks+3). The
        // f8f6f4 MFMA takes K in lane-group halves: bytes 0-15 of both lane groups are one
        // 32-K block (scaled by the group-0 lane's scale), bytes 16-31 the other (scaled by the
        // group-1 lane's). So group g holds chunk g of b0 and chunk g of b1, and its scale is
        // that of block 2 ks + g.
        const int chunk = ks * 4 + fhalf;
        i32x8 fa[4], fw[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int ra_ = wm * 128 + i * 32 + frow, rw_ = wn * 128 + i * 32 + frow;
          const i32x4 a0 = *reinterpret_cast<const i32x4*>(sA + lds_off(ra_, chunk));
          const i32x4 a1 = *reinterpret_cast<const i32x4*>(sA + lds_off(ra_, chunk + 2));
          const i32x4 w0 = *reinterpret_cast<const i32x4*>(sW + lds_off(rw_, chunk));
          const i32x4 w1 = *reinterpret_cast<const i32x4*>(sW + lds_off(rw_, chunk + 2));
          fa[i] = i32x8{a0[0], a0[1], a0[2], a0[3], a1[0], a1[1], a1[2], a1[3]};
          fw[i] = i32x8{w0[0], w0[1], w0[2], w0[3], w1[0], w1[1], w1[2], w1[3]};
        }
        if constexpr (E == Elem::FP8) {
#pragma unroll
          for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j)
              acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(
                  fw[j], fa[i], acc[i][j], 0, 0, 0, 0, 0, 0);
        } else {
          const int sh = (ks * 2 + fhalf) * 8;  // block 2 ks + g within the tile's 4
#pragma unroll
          for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j)
              acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(
                  fw[j], fa[i], acc[i][j], 0, 0, 0, (int)((cur_sw[j] >> sh) & 0xffu), 0,
                  (int)((cur_sa[i] >> sh) & 0xffu));
        }
      }
    }
    if (kt + 1 < nkt) store_lds(st ^ 1);
    __syncthreads();
  }

  // ---- epilogue: lane l holds row m = l % 32 of each MFMA tile, columns in runs of 4
  const int act_start = args.act_col_start;
  const float* ws = reinterpret_cast<const float*>(P.w_scale);
  const bf16* bias = P.bias;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int64_t m = m0 + wm * 128 + i * 32 + frow;
    const bool mok = m < M;
    const int64_t mc = mok ? m : 0;  // clamped row for address formation
    float sa = 1.f;
    if constexpr (E == Elem::FP8) sa = mok ? reinterpret_cast<const float*>(P.a_scale)[mc] : 0.f;
    const int64_t bidx = mc / P.rows_per_batch;
    bf16* crow = reinterpret_cast<bf16*>(P.c) + mc * P.ldc;
    const bf16* rrow = EPI == DIFFLET_EPI_GATE_RESIDUAL ? P.res + mc * P.ldr : nullptr;
    const bf16* grow = EPI == DIFFLET_EPI_GATE_RESIDUAL ? P.gate + bidx * P.gate_stride : nullptr;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int64_t n = n0 + wn * 128 + j * 32 + q * 8 + fhalf * 4;
        float v[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = acc[i][j][q * 4 + e];
        if (mok && n < N) {  // N % 4 == 0, so a run of 4 is all in or all out
          {
            float sw4[4] = {1.f, 1.f, 1.f, 1.f}, bb[4] = {0.f, 0.f, 0.f, 0.f};
            if constexpr (E == Elem::FP8) {
              const f32x4 t4 = *reinterpret_cast<const f32x4*>(ws + n);
#pragma unroll
              for (int e = 0; e < 4; ++e) sw4[e] = t4[e];
            }
            if (bias) {
              const u32x2 t = *reinterpret_cast<const u32x2*>(bias + n);
              bb[0] = bf16bits_to_f32(t[0] & 0xffffu);
              bb[1] = bf16bits_to_f32(t[0] >> 16);
              bb[2] = bf16bits_to_f32(t[1] & 0xffffu);
              bb[3] = bf16bits_to_f32(t[1] >> 16);
            }
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              if constexpr (E == Elem::FP8) v[e] = v[e] * (sa * sw4[e]);
              v[e] += bb[e];
            }
            if constexpr (EPI == DIFFLET_EPI_GELU) {
#pragma unroll
              for (int e = 0; e < 4; ++e)
                if (n + e >= act_start) v[e] = gelu_tanh(v[e]);
            } else if constexpr (EPI == DIFFLET_EPI_GATE_RESIDUAL) {
              const u32x2 rt = *reinterpret_cast<const u32x2*>(rrow + n);
              const u32x2 gt = *reinterpret_cast<const u32x2*>(grow + n);
              v[0] = bf16bits_to_f32(rt[0] & 0xffffu) + bf16bits_to_f32(gt[0] & 0xffffu) * v[0];
              v[1] = bf16bits_to_f32(rt[0] >> 16) + bf16bits_to_f32(gt[0] >> 16) * v[1];
              v[2] = bf16bits_to_f32(rt[1] & 0xffffu) + bf16bits_to_f32(gt[1] & 0xffffu) * v[2];
              v[3] = bf16bits_to_f32(rt[1] >> 16) + bf16bits_to_f32(gt[1] >> 16) * v[3];
            }
            u32x2 o;
            o[0] = pack_bf16x2(v[0], v[1]);
            o[1] = pack_bf16x2(v[2], v[3]);
            *reinterpret_cast<u32x2*>(crow + n) = o;
          }
        }
      }
    }
  }
}

template <Elem E>
static int gemm_launch(const char* name, int nproblems, const difflet_gemm_problem* problems,
                       int64_t n, int64_t k, int epilogue, int64_t act_col_start,
                       hipStream_t stream) {
  constexpr int KT = ElemTraits<E>::KT;
  constexpr int EB = ElemTraits<E>::BYTES;
  DLT_REQUIRE(problems && nproblems >= 1 && nproblems <= MAX_PROBLEMS, DIFFLET_EINVAL,
              "%s: nproblems must be in [1, %d]", name, MAX_PROBLEMS);
  DLT_REQUIRE(n > 0 && k > 0 && k % KT == 0, DIFFLET_EINVAL,
              "%s: k = %lld must be a positive multiple of %d", name, (long long)k, KT);
  DLT_REQUIRE(n < (1LL << 30) && k < (1LL << 30), DIFFLET_EINVAL, "%s: n or k too large", name);
  DLT_REQUIRE(n % 4 == 0, DIFFLET_EINVAL, "%s: n = %lld must be a multiple of 4", name,
              (long long)n);
  DLT_REQUIRE(epilogue >= DIFFLET_EPI_NONE && epilogue <= DIFFLET_EPI_GATE_RESIDUAL,
              DIFFLET_EINVAL, "%s: unknown epilogue %d", name, epilogue);
  GemmArgs args = {};
  args.nprob = nproblems;
  args.n = (int)n;
  args.k = (int)k;
  args.tiles_n = (int)((n + BN - 1) / BN);
  args.act_col_start = (int)(act_col_start < 0 ? 0 : act_col_start);
  int64_t tiles = 0;
  for (int i = 0; i < nproblems; ++i) {
    const difflet_gemm_problem& q = problems[i];
    DLT_REQUIRE(q.m >= 0 && q.m < (1LL << 30), DIFFLET_EINVAL, "%s: bad m", name);
    DLT_REQUIRE(q.a && q.w && q.c, DIFFLET_EINVAL, "%s: null operand in problem %d", name, i);
    DLT_REQUIRE(q.lda >= k && q.ldw >= k && q.ldc >= n, DIFFLET_EINVAL,
                "%s: leading dimensions smaller than the matrix in problem %d", name, i);
    DLT_REQUIRE((q.lda * EB) % 16 == 0 && (q.ldw * EB) % 16 == 0 && q.ldc % 4 == 0 &&
                    ((uintptr_t)q.a & 15) == 0 && ((uintptr_t)q.w & 15) == 0 &&
                    ((uintptr_t)q.c & 7) == 0,
                DIFFLET_EINVAL, "%s: operands must be 16-byte aligned row by row", name);
    DLT_REQUIRE((int64_t)q.m * q.lda * EB < (1LL << 32) && n * q.ldw * EB < (1LL << 32),
                DIFFLET_EUNSUPPORTED, "%s: an operand exceeds 4 GiB", name);
    if (epilogue == DIFFLET_EPI_GATE_RESIDUAL) {
      DLT_REQUIRE(q.gate && q.residual && q.ldr >= n, DIFFLET_EINVAL,
                  "%s: gate/residual epilogue needs gate and residual", name);
      DLT_REQUIRE(q.ldr % 4 == 0 && q.gate_stride % 4 == 0 && ((uintptr_t)q.gate & 7) == 0 &&
                      ((uintptr_t)q.residual & 7) == 0,
                  DIFFLET_EINVAL, "%s: gate/residual rows must be 8-byte aligned", name);
    }
    DLT_REQUIRE(((uintptr_t)q.bias & 7) == 0, DIFFLET_EINVAL, "%s: bias must be 8-byte aligned",
                name);
    if (E == Elem::FP8)
      DLT_REQUIRE(((uintptr_t)q.w_scale & 15) == 0, DIFFLET_EINVAL,
                  "%s: w_scale must be 16-byte aligned", name);
    if (E == Elem::MX)
      DLT_REQUIRE(((uintptr_t)q.a_scale & 3) == 0 && ((uintptr_t)q.w_scale & 3) == 0,
                  DIFFLET_EINVAL, "%s: scale rows must be 4-byte aligned", name);
    if (E == Elem::FP8 || E == Elem::MX)
      DLT_REQUIRE(q.a_scale && q.w_scale, DIFFLET_EINVAL, "%s: scales are required", name);
    GemmProblemDev& d = args.p[i];
    d.a = (const uint8_t*)q.a;
    d.w = (const uint8_t*)q.w;
    d.c = (uint8_t*)q.c;
    d.bias = (const bf16*)q.bias;
    d.gate = (const bf16*)q.gate;
    d.res = (const bf16*)q.residual;
    d.a_scale = q.a_scale;
    d.w_scale = q.w_scale;
    d.lda = q.lda;
    d.ldw = q.ldw;
    d.ldc = q.ldc;
    d.ldr = q.ldr;
    d.gate_stride = q.gate_stride;
    d.m = q.m;
    d.rows_per_batch = q.rows_per_batch > 0 ? q.rows_per_batch : (q.m > 0 ? q.m : 1);
    d.tiles_m = (int)((q.m + BM - 1) / BM);
    d.tile_start = (int)tiles;
    tiles += (int64_t)d.tiles_m * args.tiles_n;
  }
  for (int i = nproblems; i < MAX_PROBLEMS; ++i) args.p[i].tile_start = 1 << 30;
  if (tiles == 0) return DIFFLET_OK;
  DLT_REQUIRE(tiles < (1LL << 30), DIFFLET_EUNSUPPORTED, "%s: too many tiles", name);
  args.total_tiles = (int)tiles;
  dim3 grid((unsigned)tiles), block(NTHREADS);
  switch (epilogue) {
    case DIFFLET_EPI_NONE:
      hipLaunchKernelGGL((gemm_kernel<E, DIFFLET_EPI_NONE>), grid, block, 0, stream, args);
      break;
    case DIFFLET_EPI_GELU:
      hipLaunchKernelGGL((gemm_kernel<E, DIFFLET_EPI_GELU>), grid, block, 0, stream, args);
      break;
    default:
      hipLaunchKernelGGL((gemm_kernel<E, DIFFLET_EPI_GATE_RESIDUAL>), grid, block, 0, stream,
                         args);
      break;
  }
  return dlt_check_launch(name);
}

}  // namespace dlt

using namespace dlt;

extern "C" int difflet_rocm_gemm_bf16(int nproblems, const difflet_gemm_problem* problems,
                                      int64_t n, int64_t k, int epilogue,
                                      int64_t act_col_start, difflet_stream_t stream) {
  return gemm_launch<Elem::BF16>("gemm_bf16", nproblems, problems, n, k, epilogue,
                                 act_col_start, (hipStream_t)stream);
}

extern "C" int difflet_rocm_gemm_fp8_rowwise(int nproblems, const difflet_gemm_problem* problems,
                                             int64_t n, int64_t k, int epilogue,
                                             int64_t act_col_start, difflet_stream_t stream) {
  return gemm_launch<Elem::FP8>("gemm_fp8_rowwise", nproblems, problems, n, k, epilogue,
                                act_col_start, (hipStream_t)stream);
}

extern "C" int difflet_rocm_gemm_mxfp8(int nproblems, const difflet_gemm_problem* problems,
                                       int64_t n, int64_t k, int epilogue, int64_t act_col_start,
                                       difflet_stream_t stream) {
  return gemm_launch<Elem::MX>("gemm_mxfp8", nproblems, problems, n, k, epilogue,
                               act_col_start, (hipStream_t)stream);
}
