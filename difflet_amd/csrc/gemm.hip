// GEMMs of the DiT block on CDNA4 matrix cores: C = epilogue(A W^T + bias).
//
// A [M, K] and W [N, K] are both K-contiguous (activations and nn.Linear weights as stored).
// One kernel skeleton serves three element types:
//   bf16  : v_mfma_f32_32x32x16_bf16, 64 K-elements (128 bytes) per K stage, 4 MFMA K steps;
//   fp8   : v_mfma_f32_32x32x64_f8f6f4 (e4m3), 128 K-elements per K stage, 2 K steps, per-row
//           scales of A and W applied in the epilogue (acc * sa[m] * sw[n]);
//   mxfp8 : v_mfma_scale_f32_32x32x64_f8f6f4 with one E8M0 scale per 32-element block of a
//           row (the block split over the two lane groups, see the K loop), 128 K per K stage.
// A K stage is therefore always 128 bytes per row, and the LDS geometry is shared.
//
// Tiling: a workgroup owns a 256 x 256 tile of C: 8 wavefronts in a 2 x 4 grid, each 128 x 64 =
// 4 x 2 MFMA tiles of 32 x 32 (128 fp32 accumulators per lane), two per SIMD, so one
// wavefront's MFMAs cover the other's LDS waits. Launches whose last wave of tiles would be
// poorly filled cut tiles along K over the compute units (the split schedule below).
// The MFMA's first operand is the W tile and its second the A tile, so accumulator lane l holds
// row m = l % 32 and registers run along n in groups of 4 consecutive columns: the epilogue
// reads bias / gate / residual and writes C in 8-byte pieces.
//
// LDS: two stage slots of (A tile + W tile) = 2 x 64 KB, filled by direct-to-LDS buffer loads
// (no register round trip) that each move 8 whole 128-byte rows; MXFP8 adds a 24 KB ring of
// E8M0 scale blocks. Rows are XOR-swizzled in 16-byte chunks (swz8 below) so fragment reads are
// free of bank conflicts. Global loads are raw buffer loads: rows past M (or N) read as zero, so
// ragged edges need no branches.
//
// K loop: one barrier per stage, placed before the stage's last K step: the fragments of the
// next K step are read while the current one's MFMAs run, and the next stage's loads go out
// with the last K step, a quarter per A tile, so each stage has a whole stage to land.
//
// Tile order: workgroup ids are spread round-robin over the 8 XCDs, each with its own L2. The id
// is remapped so each XCD gets a contiguous run of tiles, and tiles run in groups of 8 tile rows
// so the W and A panels of neighbouring tiles stay L2-resident.
#include <algorithm>
#include <type_traits>
#include <vector>

#include "common.hpp"

namespace dlt {

constexpr int BM = 256, BN = 256;
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
  const bf16* nq;     // fused q/k norm: RMSNorm weights of q and k heads (NULL: 1)
  const bf16* nk;
  int64_t rope_row0;  // RoPE table row of row 0
  uint8_t* cs;        // EPI_GELU_MX: E8M0 scales of C, row stride ldcs
  int64_t ldcs;
};

// Split schedule. Tiles [0, dp) run one per workgroup. The other S < cus tiles (the last,
// poorly filled wave) are cut along K, in units of `gran` K stages (nu units per tile), over
// the nx = 8 XCDs as a whole: workgroups are dealt to the XCDs round-robin, so split workgroup
// s runs on XCD c = s % 8 as its member r = s / 8 of g = cus / 8. The S tiles form
// ng = ceil(S / g) groups of g consecutive tiles; XCD c takes the contiguous range
// [lo(c), lo(c + 1)) of the ng * nu (group, unit) pairs, lo(c) = c * ng * nu / 8, and its
// member r runs tile (group * g + r) of every group in it (nothing where that is past S). The g
// workgroups of an XCD thus walk K in lockstep over g neighbouring tiles, as whole tiles do, and
// share each K slice of their A and W panels through the XCD's L2; a range spans at most two
// groups (ng <= 8). A tile cut between XCDs c0 .. c1 is finished by the last contributor to
// arrive: each other one stores its fp32 accumulators in its workspace slot and counts itself in
// the tile's counter; the last adds the slots in XCD order (a fixed order: the result does not
// depend on who arrives last) and runs the epilogue. Nobody waits.
struct SkPlan {
  int dp;      // data-parallel tiles (workgroups 0 .. dp - 1)
  int groups;  // split workgroups after them (0: no split part; else nx * g)
  int nu;      // units per tile: K stages in granules of `gran` (the last may be shorter)
  int gran;    // K stages per unit (MX: 4, one block of E8M0 scales per row)
  int S;       // cut tiles
  int g;       // tiles per group = workgroups per XCD
  int nx;      // XCDs
  int64_t units;  // ng * nu
};
__host__ __device__ inline int64_t sk_lo(const SkPlan& p, int c) {
  return (int64_t)c * p.units / p.nx;
}
// the XCD whose range holds (group, unit) pair x (0 <= x < units)
__host__ __device__ inline int sk_owner(const SkPlan& p, int64_t x) {
  return (int)(((x + 1) * p.nx - 1) / p.units);
}
// workspace slot of member r of XCD c for its piece of group gi: two per workgroup, 0 for the
// first group of c's range, 1 for the second
__host__ __device__ inline int sk_slot(const SkPlan& p, int c, int r, int gi) {
  return 2 * (c * p.g + r) + (sk_lo(p, c) >= (int64_t)gi * p.nu ? 0 : 1);
}
constexpr int64_t SK_CTR_BYTES = 16384;        // one int counter per split tile
constexpr int SK_MAX_TILES = (int)(SK_CTR_BYTES / 4);
constexpr int64_t SK_SLOT_BYTES = 256 * 256 * 4;  // fp32 accumulators of one 256 x 256 tile
constexpr int SK_MIN_STAGES = 8;               // shortest K range worth a workgroup
constexpr int SK_MIN_SAVED_STAGES = 24;         // shortest cut off the busiest K walk (below)

struct GemmArgs {
  GemmProblemDev p[MAX_PROBLEMS];
  int nprob, total_tiles, tiles_n;
  int n, k;
  int act_col_start;
  SkPlan sk;
  uint8_t* ws;  // split workspace: counters, then 2 slots per split workgroup
  // fused q/k RMSNorm + RoPE on output columns [q_col, q_col + qk_cols) and [k_col, ..)
  // (qk_cols 0: off; all multiples of 256, so a tile lies wholly inside or outside)
  int qk_cols, q_col, k_col, rope_law;
  float qk_eps;
  const float* rope_cos;
  const float* rope_sin;
};

// KT: K elements per stage, KTB its bytes per row, NSLOT the stages the LDS ring holds. WN:
// wavefronts along N (two along M). Every type runs 8 wavefronts of 128 x 64 (measured against 4
// of 128 x 128: +10-20 % for fp8, +0-6 % for bf16, and 128 accumulators leave room for the
// split-tile code without spills). bf16 and fp8 stage 128 bytes of each row (two slots of
// 64 KB): a direct-to-LDS load then fetches 8 rows x 128 B, one whole line per row, which moves
// data from L2 into LDS 1.5x faster than 16 rows x 64 B (measured on FLUX's shapes: the loads
// alone of fp8 W1 take 123 against 193 us). MXFP8 stages the same 128 bytes (128 codes) per row;
// its E8M0 scales (4 bytes per row and stage) take a separate 24 KB ring.
template <Elem E> struct ElemTraits;
template <> struct ElemTraits<Elem::BF16> {
  static constexpr int KT = 64, BYTES = 2, WN = 4, KTB = 128, NSLOT = 2;
};
template <> struct ElemTraits<Elem::FP8> {
  static constexpr int KT = 128, BYTES = 1, WN = 4, KTB = 128, NSLOT = 2;
};
template <> struct ElemTraits<Elem::MX> {
  static constexpr int KT = 128, BYTES = 1, WN = 4, KTB = 128, NSLOT = 2;
};


// Workgroup barrier without the LDS drain __syncthreads implies. At each use the only LDS reads
// still in flight are of the stage being computed, which no load of this iteration overwrites;
// the memory clobber keeps the compiler from moving LDS accesses across it.
__device__ __forceinline__ void stage_barrier() { asm volatile("s_barrier" ::: "memory"); }

// A 128-byte stage row is 8 chunks of 16; chunk c of row r sits at c ^ swz8(r), swz8(r) =
// (r & 7) ^ ((r >> 3) & 1). A fragment read takes one logical chunk of 32 consecutive rows: any 8
// aligned consecutive rows land in 8 distinct 16-byte bank groups (an LDS serving 8 lanes over
// 32 banks per cycle), and any 16 aligned consecutive rows in 16 distinct ones of the 256-byte
// period (16 lanes over 64 banks): even and odd rows each see all 8 chunk positions.
__device__ __forceinline__ int swz8(int row) { return (row & 7) ^ ((row >> 3) & 1); }
__device__ __forceinline__ int lds_off8(int row, int chunk) {
  return row * 128 + ((chunk ^ swz8(row)) << 4);
}

// Scaled f8f6f4 MFMA whose E8M0 scales are byte oa of sw (first operand) and byte ob of sa
// (second). The byte selects are instruction fields: callers pass values that are constant
// after unrolling, and the switches fold away.
template <int OA>
__device__ __forceinline__ f32x16 mfma_mx_b(const i32x8& w, const i32x8& a, const f32x16& c,
                                            uint32_t sw, int ob, uint32_t sa) {
  switch (ob) {
    case 0: return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(w, a, c, 0, 0, OA, (int)sw, 0, (int)sa);
    case 1: return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(w, a, c, 0, 0, OA, (int)sw, 1, (int)sa);
    case 2: return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(w, a, c, 0, 0, OA, (int)sw, 2, (int)sa);
    default: return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(w, a, c, 0, 0, OA, (int)sw, 3, (int)sa);
  }
}
__device__ __forceinline__ f32x16 mfma_mx(const i32x8& w, const i32x8& a, const f32x16& c,
                                          int oa, uint32_t sw, int ob, uint32_t sa) {
  switch (oa) {
    case 0: return mfma_mx_b<0>(w, a, c, sw, ob, sa);
    case 1: return mfma_mx_b<1>(w, a, c, sw, ob, sa);
    case 2: return mfma_mx_b<2>(w, a, c, sw, ob, sa);
    default: return mfma_mx_b<3>(w, a, c, sw, ob, sa);
  }
}

// WN = ElemTraits<E>::WN wavefronts along N, 2 along M: 128 WN threads.
// SPLIT: the launch uses the split schedule (workgroups may own several tiles or parts of
// them). Whole-tile launches (SPLIT false, the DiT steps) hold no state across tiles, so the
// K loop's addressing and the epilogue do not compete for registers with a tile loop.
template <Elem E, int EPI, int WN, bool QK, bool SPLIT>
__global__ __launch_bounds__(128 * WN, 1) void gemm_kernel(const GemmArgs args) {
  constexpr int KT = ElemTraits<E>::KT;
  constexpr int EB = ElemTraits<E>::BYTES;
  constexpr int KTB = ElemTraits<E>::KTB, NSLOT = ElemTraits<E>::NSLOT;
  constexpr int WN_WAVES = WN, NWAVES = 2 * WN;
  constexpr int WTN = BN / WN_WAVES, TJ = WTN / 32;  // wave tile 128 x WTN: 4 x TJ MFMA tiles
  constexpr int SLABS = 2 * BM * KTB / 1024 / NWAVES;  // 1 KB LDS slabs one wave loads per stage
  // LDS: the stage ring [slot][A|W] (128 KB) and (MX) the E8M0 scales of 8 stages (16 bytes) per
  // row, a ring of 3 such blocks [slot][A|W][row]. One LDS variable: with two, the compiler
  // gives their accesses alias scopes and then drains all loads (vmcnt(0)) before each LDS read
  // that follows a direct-to-LDS load.
  constexpr int RING_BYTES = NSLOT * 2 * BM * KTB;
  constexpr int SC_BYTES = E == Elem::MX ? 3 * 2 * BM * 16 : 0;
  static_assert(RING_BYTES == 128 * 1024, "the epilogues stage a 256 x 256 bf16 tile in the ring");
  __shared__ __attribute__((aligned(16))) uint8_t lds[RING_BYTES + SC_BYTES];
  auto& smem = *reinterpret_cast<uint8_t(*)[NSLOT][2][BM * KTB]>(lds);
  auto& smem_sc = *reinterpret_cast<uint32_t(*)[3][2][BM][4]>(lds + RING_BYTES);

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  // wave-uniform, held in a scalar register: LDS-DMA destinations (M0) are then scalar math
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / WN_WAVES, wn = wave % WN_WAVES;

  // ---- work: one whole tile (data-parallel part), or a range of (group, K unit) pairs
  const SkPlan& plan = args.sk;
  const int nk = args.k / KT, nu = plan.nu;
  int bid = blockIdx.x;
  [[maybe_unused]] int c_self = -1, r_self = 0;  // split workgroups: XCD and member
  int64_t u_lo = 0, u_hi = 1;                     // one piece, or pairs [u_lo, u_hi)
  if (!SPLIT || bid < plan.dp) {                  // XCD-contiguous runs of tiles
    if ((plan.dp & 7) == 0) bid = (bid & 7) * (plan.dp >> 3) + (bid >> 3);
  } else {
    c_self = (bid - plan.dp) % plan.nx;
    r_self = (bid - plan.dp) / plan.nx;
    u_lo = sk_lo(plan, c_self);
    u_hi = sk_lo(plan, c_self + 1);
  }
  // the split-tile flag lives in the LDS ring, idle when it is used (one LDS variable, above)
  [[maybe_unused]] volatile int& sk_flag = *reinterpret_cast<volatile int*>(lds);

  for (int64_t u = u_lo; u < u_hi;) {
  int tt, ub, ue;  // tile, and the units [ub, ue) of it that run here
  if (!SPLIT || c_self < 0) {
    tt = bid, ub = 0, ue = nu;
    u = u_hi;
  } else {
    const int gi = (int)(u / nu);
    const int64_t g0 = (int64_t)gi * nu;
    ub = (int)(u - g0);
    ue = (int)(min(u_hi, g0 + nu) - g0);
    if (u != u_lo) __syncthreads();  // the previous piece's last LDS reads are done
    u = g0 + ue;
    const int tl = gi * plan.g + r_self;
    if (tl >= plan.S) continue;  // past the last cut tile: nothing to run in this group
    tt = plan.dp + tl;
  }
  // its K stages [kbeg, kend) run here; the loop below counts them from 0
  const int kbeg = ub * plan.gran, kend = min(ue * plan.gran, nk), nkt = kend - kbeg;

  // ---- tile -> problem, grouped raster
  int p = 0;
#pragma unroll
  for (int i = 1; i < MAX_PROBLEMS; ++i)
    if (i < args.nprob && tt >= args.p[i].tile_start) p = i;
  const GemmProblemDev& P = args.p[p];
  int t = tt - P.tile_start;
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

  // Direct-to-LDS staging: a stage of one operand is 256 rows x 128 bytes = 32 KB = 32 slabs of
  // 1 KB; wave w fills slabs 4 w .. 4 w + 3. Lane l of load i writes slot p = (4 w + i) * 64 + l,
  // i.e. row p / 8, physical chunk p % 8, so it loads logical chunk (p % 8) ^ swz8(row) of that
  // row. Per-lane offsets are fixed; the stage's K offset goes in soffset.
  typedef __attribute__((address_space(3))) void lds_void;
  constexpr int SA = SLABS / 2;  // slabs of each operand per wave
  // Arrays handed to target builtins are sized for the largest geometry (4), not by SA / TJ:
  // with a template-dependent size the host pass drops the kernel's launch stub unreported.
  uint32_t a_off[4], w_off[4];
#pragma unroll
  for (int i = 0; i < SA; ++i) {
    const int p = (wave * SA + i) * 64 + lane;
    const int r = p >> 3, ch = (p & 7) ^ swz8(r);  // 8 rows x 8 chunks per slab
    a_off[i] = (uint32_t)(r * a_row_bytes) + ch * 16;
    w_off[i] = (uint32_t)(r * w_row_bytes) + ch * 16;
  }
  // MX scales: block q = the 16 scale bytes of stages 4 q .. 4 q + 3 of every row (K-blocks
  // 16 q .. 16 q + 15; stage s's 4 bytes are word s % 4), in ring slot q % 3. Block q + 1 is
  // loaded in 8 parts of 64 rows (A rows for parts 0-3, W rows for 4-7) while the stages of
  // block q are issued: with stage s, waves 2 (s % 4) and 2 (s % 4) + 1 load the parts of their
  // own number. The loads of stage s land by the barrier that publishes stage s, two stages
  // before block q + 1's first stage 4 q + 4 at the latest, and slot (q + 1) % 3 was last read
  // by block q - 2, whose stages end before stage 4 q, the first to carry block q + 1. The whole offset goes in
  // the per-lane offset so the resource's range check covers it: bytes past the scale array
  // (rows past M / N, a last block shorter than 16 bytes) read zero.
  const int ksb = K / 32;  // scale row stride (blocks per row)
  __amdgpu_buffer_rsrc_t rsa = rw, rsw = rw;
  if constexpr (E == Elem::MX) {
    rsa = make_rsrc((const uint8_t*)P.a_scale + m0 * ksb, (uint32_t)((M - m0) * ksb));
    rsw = make_rsrc((const uint8_t*)P.w_scale + n0 * ksb, (uint32_t)((N - n0) * ksb));
  }
  auto issue_scales = [&](int blk, int p) {  // MX: part p of scale block blk (of the range)
    const uint32_t row = (p & 3) * 64 + lane;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(p < 4 ? rsa : rsw,
                                             (lds_void*)&smem_sc[blk % 3][p >> 2][(p & 3) * 64][0],
                                             16, row * ksb + ((kbeg >> 2) + blk) * 16, 0, 0, 0);
  };
  // part `part` (of 4) of stage kt's loads: a quarter of this wave's slabs, A slabs first (MX:
  // with part 0, waves 2 (kt % 4) and 2 (kt % 4) + 1 also load their parts of the next scale
  // block)
  auto issue_part = [&](int kt, int st, int part) {
    const uint32_t kb = (uint32_t)(kbeg + kt) * KTB;  // kt counts from the range start
#pragma unroll
    for (int s = part * SLABS / 4; s < (part + 1) * SLABS / 4; ++s) {
      if (s < SA)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            ra, (lds_void*)&smem[st][0][(wave * SA + s) * 1024], 16, a_off[s], kb, 0, 0);
      else
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            rw, (lds_void*)&smem[st][1][(wave * SA + s - SA) * 1024], 16, w_off[s - SA], kb, 0, 0);
    }
    if constexpr (E == Elem::MX) {
      if (part == 0 && (wave >> 1) == (kt & 3)) issue_scales((kt >> 2) + 1, wave);
    }
  };
  auto issue_stage = [&](int kt, int st) {
#pragma unroll
    for (int i = 0; i < 4; ++i) issue_part(kt, st, i);
  };
  // vector-memory instructions one stage issues per wave (for s_waitcnt vmcnt). A stage that
  // also carries an MX scale part issues one more, which only makes a wait conservative: the
  // waits allow the loads of the stages issued after the awaited one to stay in flight, and
  // those are at least LOADS_PER_STAGE per stage.
  constexpr int LOADS_PER_STAGE = SLABS;

  f32x16 acc[4][4];  // columns j < TJ used
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < TJ; ++j) acc[i][j] = f32x16{};

  const int frow = lane & 31;  // fragment row within a 32-row MFMA tile
  const int fhalf = lane >> 5;

  static_assert(KTB == 128 && NSLOT == 2, "the K loop runs 128-byte stages in two slots");
  {
    // ---- 128-byte stages in two LDS slots. A stage is NKS MFMA K steps (bf16 4 of 16 elements,
    // fp8 and MX 2 of 64); fragments of the next K step are read while the current one's
    // MFMAs run (two register sets). Before the last K step of stage kt every wave waits for its
    // loads of stage kt + 1 (the only ones in flight) and for its own reads of this stage, and
    // one barrier then publishes stage kt + 1 and frees this slot; the loads of stage kt + 2
    // into it go out with the last K step's MFMAs, so each stage has a whole stage to land.
    constexpr int NKS = E == Elem::BF16 ? 4 : 2;
    constexpr int NA = E == Elem::BF16 ? 1 : 2;  // 16-byte LDS reads per fragment
    // A fragments roll: tile i's fragment of the next K step is read into its registers right
    // after tile i's MFMAs of this step issue; W fragments alternate between two sets. With 128
    // accumulators that keeps a wave within 256 registers (two whole sets spill).
    // MX: K step ks of a stage is K-blocks 2 ks (lane group 0's chunks) and 2 ks + 1 (group 1's),
    // each lane passing its row's scale of its group's block: byte 2 ks + fhalf of the stage's
    // scale word. The scales roll with the fragments they belong to, packed one byte per tile
    // (the MFMA's scale byte select picks the tile's): A tile i in byte i of sa, W tile j of set
    // s in byte j of sw[s]. Eight separate registers push the loop past 256 and spill.
    i32x4 fa[4][2], fw[2][4][2];  // [tile][part]; fw[set][tile j < TJ][part]
    [[maybe_unused]] uint32_t sa = 0, sw[2] = {0, 0};
    auto scale_of = [&](int op, int r, int skt, int ks) {  // MX: operand op's scale for row r
      return (uint32_t)(reinterpret_cast<const uint8_t*>(&smem_sc[(skt >> 2) % 3][op][r][skt & 3]) +
                        fhalf)[2 * ks];
    };
    // fragments of K step ks of stage skt (counted from the range start), in ring slot st
    auto read_a = [&](int st, int skt, int ks, int i) {
      const uint8_t* sA = smem[st][0];
      const int r = wm * 128 + i * 32 + frow;
#pragma unroll
      for (int h = 0; h < NA; ++h)
        fa[i][h] = *reinterpret_cast<const i32x4*>(sA + lds_off8(r, 2 * NA * ks + 2 * h + fhalf));
      if constexpr (E == Elem::MX)
        sa = (sa & ~(0xffu << (8 * i))) | (scale_of(0, r, skt, ks) << (8 * i));
    };
    auto read_w = [&](int st, int skt, int ks, int set) {
      const uint8_t* sW = smem[st][1];
      if constexpr (E == Elem::MX) sw[set] = 0;
#pragma unroll
      for (int j = 0; j < TJ; ++j) {
        const int r = wn * WTN + j * 32 + frow;
#pragma unroll
        for (int h = 0; h < NA; ++h)
          fw[set][j][h] =
              *reinterpret_cast<const i32x4*>(sW + lds_off8(r, 2 * NA * ks + 2 * h + fhalf));
        if constexpr (E == Elem::MX) sw[set] |= scale_of(1, r, skt, ks) << (8 * j);
      }
    };
    auto mma_tile = [&](int set, int i) {
#pragma unroll
      for (int j = 0; j < TJ; ++j) {
        if constexpr (E == Elem::BF16) {
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
              __builtin_bit_cast(bf16x8, fw[set][j][0]), __builtin_bit_cast(bf16x8, fa[i][0]),
              acc[i][j], 0, 0, 0);
        } else {
          const i32x8 w8 = {fw[set][j][0][0], fw[set][j][0][1], fw[set][j][0][2], fw[set][j][0][3],
                            fw[set][j][1][0], fw[set][j][1][1], fw[set][j][1][2], fw[set][j][1][3]};
          const i32x8 a8 = {fa[i][0][0], fa[i][0][1], fa[i][0][2], fa[i][0][3],
                            fa[i][1][0], fa[i][1][1], fa[i][1][2], fa[i][1][3]};
          if constexpr (E == Elem::FP8)
            acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(w8, a8, acc[i][j], 0, 0,
                                                                        0, 0, 0, 0);
          else
          {
            acc[i][j] = mfma_mx(w8, a8, acc[i][j], j, sw[set], i, sa);
            // pinned here: left free, the scaled MFMAs sink below the next step's fragment
            // reads, whose registers then all live at once and spill
            asm volatile("" : "+v"(acc[i][j]));
          }
        }
      }
    };
    if constexpr (E == Elem::MX) {  // scale block 0, one part per wave, ahead of stage 0
#pragma unroll
      for (int p = wave; p < 8; p += NWAVES) issue_scales(0, p);
    }
    issue_stage(0, 0);
    if (nkt > 1) {
      issue_stage(1, 1);
      constexpr int c = LOADS_PER_STAGE;  // stage 0 landed, stage 1 may be in flight
      __builtin_amdgcn_s_waitcnt(0x0f70 | (c & 15) | ((c >> 4) << 14));
    } else {
      __builtin_amdgcn_s_waitcnt(0x0f70);
    }
    __syncthreads();
    read_w(0, 0, 0, 0);
#pragma unroll
    for (int i = 0; i < 4; ++i) read_a(0, 0, 0, i);
    for (int kt = 0; kt < nkt; ++kt) {
      const int st = kt & 1;
#pragma unroll
      for (int ks = 0; ks < NKS; ++ks) {
        const int set = ks & 1;
        const bool last = ks == NKS - 1;
        // the next K step: of this stage, or the first of stage kt + 1 (past the range's last
        // stage it reads stale LDS that nothing uses)
        const int nst = last ? (st ^ 1) : st, nkt_s = last ? kt + 1 : kt, nks = last ? 0 : ks + 1;
        const bool loads = last && kt + 2 < nkt;
        if (last) {
          // stage kt + 1 has landed (only its loads are in flight) and this wave's reads of
          // slot st are done; the barrier publishes the one and frees the other
          __builtin_amdgcn_s_waitcnt(0x0070);  // vmcnt(0) lgkmcnt(0)
          stage_barrier();
        }
        read_w(nst, nkt_s, nks, set ^ 1);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          mma_tile(set, i);
          read_a(nst, nkt_s, nks, i);
          if (loads) issue_part(kt + 2, st, i);
          __builtin_amdgcn_sched_barrier(0);
        }
      }
    }
  }

  // ---- a tile cut between XCDs c0 .. c1: the last contributor to arrive finishes it.
  // Partial sums move through the workspace with device-scope (sc1) loads and stores, which
  // the L2 of another XCD cannot serve stale; a store is complete (vmcnt) before its workgroup
  // counts itself, so a count read at device scope orders them without cache-wide fences.
  if constexpr (SPLIT) if (kbeg != 0 || kend != nk) {
    const int tl = tt - plan.dp;  // tile index within the split part
    const int gi = tl / plan.g;    // its group
    const int64_t x0 = (int64_t)gi * nu;
    const int c0 = sk_owner(plan, x0), c1 = sk_owner(plan, x0 + nu - 1);
    const int nc = c1 - c0 + 1;
    int* ctr = reinterpret_cast<int*>(args.ws) + tl;
    const __amdgpu_buffer_rsrc_t rs =
        make_rsrc(args.ws + SK_CTR_BYTES, (uint32_t)(2 * plan.groups * SK_SLOT_BYTES));
    constexpr int SC1 = 16;  // cache policy: device scope
    // lane-major slot layout: each store / load instruction moves 1 KB contiguous; only the
    // lane's 16 bytes vary across the wave, the rest is a scalar offset
    const uint32_t vo = (uint32_t)lane * 16;
    auto soff = [&](int c, int i, int j, int q) {
      return (uint32_t)(sk_slot(plan, c, r_self, gi) * SK_SLOT_BYTES) +
             (uint32_t)(((wave * (4 * TJ) + i * TJ + j) * 4 + q) * 1024);
    };
    // With two contributors (a + b == b + a) or as the first one, this workgroup's own
    // accumulators can stay in registers and still be summed in contributor order
    const bool own_in_regs = nc == 2 || c_self == c0;
    bool last = false;
    __syncthreads();  // every wave's loads into the ring have landed (the flag is in slot 0)
    if (own_in_regs) {
      if (tid == 0)
        sk_flag = __hip_atomic_load(ctr, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == nc - 1;
      __syncthreads();
      last = sk_flag;
      __syncthreads();
    }
    if (!last) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < TJ; ++j)
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const f32x4 v = {acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2],
                             acc[i][j][4 * q + 3]};
            __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), rs, vo,
                                                   soff(c_self, i, j, q), SC1);
          }
      __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0): the stores are complete
      __syncthreads();
      if (tid == 0)
        sk_flag = __hip_atomic_fetch_add(ctr, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                  nc - 1;
      __syncthreads();
      last = sk_flag;
    }
    if (!last) continue;  // another contributor finishes the tile
    if (!own_in_regs) {  // the own part is in its slot too: sum every slot from zero
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < TJ; ++j) acc[i][j] = f32x16{};
    }
    for (int c = c0; c <= c1; ++c) {
      if (own_in_regs && c == c_self) continue;
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < TJ; ++j) {
          // one MFMA tile's 16 values at a time: the accumulators already fill the registers
          // (cast whole vectors: hipcc lowers a bit_cast of one vector element to a load of
          // element 0)
          f32x4 v[4];
#pragma unroll
          for (int q = 0; q < 4; ++q)
            v[q] = __builtin_bit_cast(
                f32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, vo, soff(c, i, j, q), SC1));
#pragma unroll
          for (int q = 0; q < 4; ++q)
#pragma unroll
            for (int e = 0; e < 4; ++e) acc[i][j][4 * q + e] += v[q][e];
          __builtin_amdgcn_sched_barrier(0);
        }
    }
    if (tid == 0) __hip_atomic_store(ctr, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }

  // ---- epilogue: lane l holds row m = l % 32 of each MFMA tile; register 4 q + e of tile
  // (i, j) is column n = n0 + wn * WTN + j * 32 + q * 8 + 4 g + e (N % 4 == 0, so a run of 4
  // is all in or all out). Column vectors (bias, gate, W scales) are read once for the whole
  // tile, and each row block's residual is read before any of its stores: the residual may
  // alias C, so loads left between stores would each wait out a full memory latency.
  if constexpr (EPI == DIFFLET_EPI_F32) {
    // fp32 C = acc (+ bias), straight from the accumulators: 16 bytes per lane and register
    // group (the scores of the VAE decoders' mid-block attention, which a softmax reads next)
    float* C = reinterpret_cast<float*>(P.c);
#pragma unroll
    for (int j = 0; j < TJ; ++j)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int64_t n = n0 + wn * WTN + j * 32 + q * 8 + fhalf * 4;
        if (n >= N) continue;
        float b[4] = {0.f, 0.f, 0.f, 0.f};
        if (P.bias) {
          const u32x2 bv = *reinterpret_cast<const u32x2*>(reinterpret_cast<const bf16*>(P.bias) + n);
          b[0] = bf16bits_to_f32(bv[0] & 0xffffu);
          b[1] = bf16bits_to_f32(bv[0] >> 16);
          b[2] = bf16bits_to_f32(bv[1] & 0xffffu);
          b[3] = bf16bits_to_f32(bv[1] >> 16);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int64_t m = m0 + wm * 128 + i * 32 + frow;
          if (m >= M) continue;
          const f32x4 v = {acc[i][j][4 * q] + b[0], acc[i][j][4 * q + 1] + b[1],
                           acc[i][j][4 * q + 2] + b[2], acc[i][j][4 * q + 3] + b[3]};
          *reinterpret_cast<f32x4*>(C + m * P.ldc + n) = v;
        }
      }
    continue;  // the next piece (split workgroups), or the end of the loop
  }
  const float* ws = reinterpret_cast<const float*>(P.w_scale);
  // fused q/k RMSNorm + RoPE: this tile's 256 columns are two heads of q or of k; a head's 128
  // columns are the 64 of waves wn = 2 h and 2 h + 1, whose per-row sums of squares meet in LDS
  bool qk_tile = false;
  if constexpr (QK)
    qk_tile = (n0 >= args.q_col && n0 < (int64_t)args.q_col + args.qk_cols) ||
              (n0 >= args.k_col && n0 < (int64_t)args.k_col + args.qk_cols);
  if constexpr (EPI != DIFFLET_EPI_GATE_RESIDUAL) {
    // Plain and GELU tiles go out through the idle LDS ring: each wave writes its values (the
    // same fp32 math and bf16 rounding as a direct store) as [256 rows][32 chunks of 16 bytes],
    // chunk c of row r at c ^ (r & 31); then each half-wave stores one row of the tile, 16 bytes
    // per lane, 512 contiguous bytes. Stored straight from the accumulators, a wave instruction
    // covers 32 rows x 16 bytes, and the plain and GELU epilogues took 25-30 % of the fp8 GEMMs.
    uint8_t* tile = lds;
    const float* wsc = reinterpret_cast<const float*>(P.w_scale);
    // the 4 row scales (fp8) for the whole tile; a W tile's column vectors while it is stored
    float sa[4] = {1.f, 1.f, 1.f, 1.f};
    if constexpr (E == Elem::FP8)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int64_t m = m0 + wm * 128 + i * 32 + frow;
        sa[i] = m < M ? reinterpret_cast<const float*>(P.a_scale)[m] : 0.f;
      }
    __syncthreads();  // every wave's last fragment reads of the ring are done
    // GELU on columns >= act_col_start: a tile lies wholly on one side (uniform branch) or
    // straddles it (per-column select, no branch)
    auto stage = [&](auto gelu_mode) {
      constexpr int G = decltype(gelu_mode)::value;  // 0 none, 1 every column, 2 per column
#pragma unroll
      for (int j = 0; j < TJ; ++j) {
        u32x2 bv[4];
        f32x4 wv[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int64_t n = n0 + wn * WTN + j * 32 + q * 8 + fhalf * 4;
          const bool nok = n < N;
          bv[q] = (P.bias && nok) ? *reinterpret_cast<const u32x2*>(P.bias + n) : u32x2{0u, 0u};
          if constexpr (E == Elem::FP8)
            wv[q] = nok ? *reinterpret_cast<const f32x4*>(wsc + n) : f32x4{};
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int r = wm * 128 + i * 32 + frow;  // tile row
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const int cl = wn * WTN + j * 32 + q * 8 + fhalf * 4;  // tile column of the 4 values
            float v[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              v[e] = acc[i][j][q * 4 + e];
              if constexpr (E == Elem::FP8) v[e] = v[e] * (sa[i] * wv[q][e]);
              v[e] += bf16bits_to_f32(e & 1 ? bv[q][e >> 1] >> 16 : bv[q][e >> 1] & 0xffffu);
              if constexpr (G == 1) v[e] = gelu_tanh(v[e]);
              if constexpr (G == 2) {
                const float g = gelu_tanh(v[e]);
                v[e] = n0 + cl + e >= args.act_col_start ? g : v[e];
              }
            }
            const u32x2 o = {pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
            *reinterpret_cast<u32x2*>(tile + r * 512 + (((cl >> 3) ^ (r & 31)) << 4) + (cl & 7) * 2) = o;
          }
        }
      }
    };
    if constexpr (EPI == DIFFLET_EPI_GELU) {
      if (n0 >= args.act_col_start) stage(std::integral_constant<int, 1>{});
      else if (n0 + BN > args.act_col_start) stage(std::integral_constant<int, 2>{});
      else stage(std::integral_constant<int, 0>{});
    } else if constexpr (EPI == DIFFLET_EPI_GELU_MX) {
      stage(std::integral_constant<int, 1>{});
    } else {
      stage(std::integral_constant<int, 0>{});
    }
    __syncthreads();
    if constexpr (QK) if (qk_tile) {
      // fused q/k RMSNorm + RoPE: this tile's 256 columns are two heads of q or of k (the
      // staged values are the plain GEMM's bf16 output); each half-wave takes one row, 16 lanes
      // per 128-column head reduce its sum of squares with xor shuffles, scale by
      // rsqrt(mean + eps) and the norm weights, rotate and store 16 bytes per lane
      const bf16* nw = (n0 >= args.q_col && n0 < (int64_t)args.q_col + args.qk_cols) ? P.nq : P.nk;
      {
        const int ch = lane & 31, half = lane >> 5;  // 16-byte chunk of the row, which row of two
        const int d = (ch & 15) * 8;                 // column within the head
        const u32x4 wraw = nw ? *reinterpret_cast<const u32x4*>(nw + d)
                              : u32x4{0x3f803f80u, 0x3f803f80u, 0x3f803f80u, 0x3f803f80u};
        // each half-wave takes rows wave * 2 + half + 16 t; batches of RB rows issue all their
        // LDS and RoPE-table loads before any arithmetic (one latency per batch, not per row;
        // the accumulators are dead here, so the registers are free)
        constexpr int RB = 4, SLOTS = BM / (2 * NWAVES);
        const bool law0 = args.rope_law == 0;
#pragma unroll 1
        for (int t0 = 0; t0 < SLOTS; t0 += RB) {
          u32x4 raw[RB];
          f32x4 c[RB][2], sn[RB][2];
#pragma unroll
          for (int b = 0; b < RB; ++b) {
            const int r = wave * 2 + half + (t0 + b) * 2 * NWAVES;
            const int64_t mc = min(m0 + r, (int64_t)M - 1);  // rows past M read a valid table row
            raw[b] = *reinterpret_cast<const u32x4*>(tile + r * 512 + ((ch ^ (r & 31)) << 4));
            const int64_t rr = P.rope_row0 + mc;
            const float* cp = args.rope_cos + rr * 128 + d;
            const float* sp = args.rope_sin + rr * 128 + d;
            c[b][0] = *reinterpret_cast<const f32x4*>(cp);
            c[b][1] = *reinterpret_cast<const f32x4*>(cp + 4);
            sn[b][0] = *reinterpret_cast<const f32x4*>(sp);
            sn[b][1] = *reinterpret_cast<const f32x4*>(sp + 4);
          }
#pragma unroll
          for (int b = 0; b < RB; ++b) {
            const int r = wave * 2 + half + (t0 + b) * 2 * NWAVES;
            const int64_t m = m0 + r;
            float v[8];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              v[2 * e] = bf16bits_to_f32(raw[b][e] & 0xffffu);
              v[2 * e + 1] = bf16bits_to_f32(raw[b][e] >> 16);
            }
            float ss = 0.f;
#pragma unroll
            for (int e = 0; e < 8; ++e) ss += v[e] * v[e];
            ss = sum16_dpp(ss);  // 16 lanes hold one head of one row
            const float rs = __builtin_amdgcn_rsqf(ss * (1.0f / 128.0f) + args.qk_eps);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              v[2 * e] = v[2 * e] * rs * bf16bits_to_f32(wraw[e] & 0xffffu);
              v[2 * e + 1] = v[2 * e + 1] * rs * bf16bits_to_f32(wraw[e] >> 16);
            }
            const float* cf = reinterpret_cast<const float*>(&c[b][0]);
            const float* sf = reinterpret_cast<const float*>(&sn[b][0]);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const float a0 = v[2 * e], b0 = v[2 * e + 1];
              if (law0) {
                v[2 * e] = a0 * cf[2 * e] - b0 * sf[2 * e];
                v[2 * e + 1] = b0 * cf[2 * e + 1] + a0 * sf[2 * e + 1];
              } else {
                v[2 * e] = a0 * cf[2 * e] - b0 * sf[2 * e + 1];
                v[2 * e + 1] = a0 * sf[2 * e + 1] + b0 * cf[2 * e];
              }
            }
            if (m < M) {
              u32x4 st;
#pragma unroll
              for (int e = 0; e < 4; ++e) st[e] = pack_bf16x2(v[2 * e], v[2 * e + 1]);
              *reinterpret_cast<u32x4*>(reinterpret_cast<bf16*>(P.c) + m * P.ldc + n0 + ch * 8) = st;
            }
          }
        }
      }
      continue;  // this tile is stored
    }
    if constexpr (EPI == DIFFLET_EPI_GELU_MX) {
      // the staged bf16 GELU output quantized to MXFP8 in blocks of 32 consecutive columns:
      // each half-wave takes one row, lanes 4 b .. 4 b + 3 hold block b's 32 values (8 each);
      // their exponent maximum meets over two xor shuffles inside the quad, then each lane
      // stores its 8 codes and the block's first lane its E8M0 scale (N % 32 == 0: a block is
      // wholly in or out, and the quad takes one branch)
      const int ch = lane & 31, half = lane >> 5;
      const int64_t n = n0 + ch * 8;
      for (int r = wave * 2 + half; r < BM; r += 2 * NWAVES) {
        const int64_t m = m0 + r;
        if (m >= M) break;  // rows only grow
        if (n >= N) continue;
        const u32x4 raw = *reinterpret_cast<const u32x4*>(tile + r * 512 + ((ch ^ (r & 31)) << 4));
        float v[8];
        uint32_t emax = 0;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          v[2 * e] = bf16bits_to_f32(raw[e] & 0xffffu);
          v[2 * e + 1] = bf16bits_to_f32(raw[e] >> 16);
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const uint32_t x = (__builtin_bit_cast(uint32_t, v[e]) >> 23) & 0xffu;
          emax = x > emax ? x : emax;
        }
        emax = max(emax, (uint32_t)__shfl_xor((int)emax, 1, 64));
        emax = max(emax, (uint32_t)__shfl_xor((int)emax, 2, 64));
        const int su = (int)emax - 7 < 0 ? 0 : (int)emax - 7;  // clamp(e_max - 7, 0, 255)
        const float mul = __builtin_bit_cast(float, (uint32_t)(254 - su) << 23);  // 2^(127 - su)
        float c[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) c[e] = clamp448(__fmul_rn(v[e], mul));
        *reinterpret_cast<u32x2*>(P.c + m * P.ldc + n) =
            u32x2{e4m3x4(c[0], c[1], c[2], c[3]), e4m3x4(c[4], c[5], c[6], c[7])};
        if ((ch & 3) == 0) P.cs[m * P.ldcs + (n >> 5)] = (uint8_t)su;
      }
      continue;  // this tile is stored
    }
    const int ch = lane & 31, half = lane >> 5;  // 16-byte chunk of the row, which row of two
    const int64_t n = n0 + ch * 8;
    // 16-byte stores need 16-byte aligned rows; otherwise two 8-byte halves (N % 4 == 0)
    const bool wide = (((uintptr_t)P.c & 15) == 0) && (P.ldc % 8 == 0);
    for (int r = wave * 2 + half; r < BM; r += 2 * NWAVES) {
      const int64_t m = m0 + r;
      if (m >= M) break;  // rows only grow
      if (n >= N) continue;
      const u32x4 raw = *reinterpret_cast<const u32x4*>(tile + r * 512 + ((ch ^ (r & 31)) << 4));
      bf16* dst = reinterpret_cast<bf16*>(P.c) + m * P.ldc + n;
      if (wide && n + 8 <= N) {
        *reinterpret_cast<u32x4*>(dst) = raw;
      } else {
        *reinterpret_cast<u32x2*>(dst) = u32x2{raw[0], raw[1]};
        if (n + 4 < N) *reinterpret_cast<u32x2*>(dst + 4) = u32x2{raw[2], raw[3]};
      }
    }
    continue;  // this tile is stored
  }
  if constexpr (SPLIT) {
    // the split schedule's kernels (whose cut-tile state stays live) store straight from the
    // accumulators: staged through the ring they spilled 140-250 bytes per lane
    const bf16* bias = P.bias;
    u32x2 bias_v[4][4], gate_v[4][4];  // [j < TJ][q]
    f32x4 ws_v[4][4];
  #pragma unroll
    for (int j = 0; j < TJ; ++j)
  #pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int64_t n = n0 + wn * WTN + j * 32 + q * 8 + fhalf * 4;
        const bool nok = n < N;
        bias_v[j][q] = (bias && nok) ? *reinterpret_cast<const u32x2*>(bias + n) : u32x2{0u, 0u};
        if constexpr (E == Elem::FP8)
          ws_v[j][q] = nok ? *reinterpret_cast<const f32x4*>(ws + n) : f32x4{};
        if constexpr (EPI == DIFFLET_EPI_GATE_RESIDUAL) {
          // one gate row per batch element: a wave's 128 rows lie in one batch element, since
          // the host requires rows_per_batch % 128 == 0 when a problem holds several. A wave whose
          // rows all lie past M stores nothing; its row is clamped to M - 1 so the gate read stays
          // within the ceil(M / rows_per_batch) rows the gate holds.
          const int64_t b0 = min(m0 + wm * 128, (int64_t)M - 1) / P.rows_per_batch;
          gate_v[j][q] = nok ? *reinterpret_cast<const u32x2*>(P.gate + b0 * P.gate_stride + n)
                             : u32x2{0u, 0u};
        }
      }
  #pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t m = m0 + wm * 128 + i * 32 + frow;
      const bool mok = m < M;
      const int64_t mc = mok ? m : 0;  // clamped row for address formation
      float sa = 1.f;
      if constexpr (E == Elem::FP8) sa = mok ? reinterpret_cast<const float*>(P.a_scale)[mc] : 0.f;
      bf16* crow = reinterpret_cast<bf16*>(P.c) + mc * P.ldc;
      u32x2 res_v[4][4];
      if constexpr (EPI == DIFFLET_EPI_GATE_RESIDUAL) {
        const bf16* rrow = P.res + mc * P.ldr;
  #pragma unroll
        for (int j = 0; j < TJ; ++j)
  #pragma unroll
          for (int q = 0; q < 4; ++q) {
            const int64_t n = n0 + wn * WTN + j * 32 + q * 8 + fhalf * 4;
            res_v[j][q] = (mok && n < N) ? *reinterpret_cast<const u32x2*>(rrow + n) : u32x2{0u, 0u};
          }
      }
  #pragma unroll
      for (int j = 0; j < TJ; ++j)
  #pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int64_t n = n0 + wn * WTN + j * 32 + q * 8 + fhalf * 4;
          float v[4];
  #pragma unroll
          for (int e = 0; e < 4; ++e) {
            v[e] = acc[i][j][q * 4 + e];
            if constexpr (E == Elem::FP8) v[e] = v[e] * (sa * ws_v[j][q][e]);
            v[e] += bf16bits_to_f32(e & 1 ? bias_v[j][q][e >> 1] >> 16
                                          : bias_v[j][q][e >> 1] & 0xffffu);
          }
          {
  #pragma unroll
            for (int e = 0; e < 4; ++e) {
              const uint32_t rw_ = res_v[j][q][e >> 1], gw_ = gate_v[j][q][e >> 1];
              v[e] = bf16bits_to_f32(e & 1 ? rw_ >> 16 : rw_ & 0xffffu) +
                     bf16bits_to_f32(e & 1 ? gw_ >> 16 : gw_ & 0xffffu) * v[e];
            }
          }
          if (mok && n < N) {
            u32x2 o;
            o[0] = pack_bf16x2(v[0], v[1]);
            o[1] = pack_bf16x2(v[2], v[3]);
            *reinterpret_cast<u32x2*>(crow + n) = o;
          }
        }
    }
    continue;  // this tile is stored
  }
  // ---- gate * (acc + bias) + residual (EPI_GATE_RESIDUAL) through the LDS ring, one row half
  // (128 rows) at a time: the fp32 values of a 128 x 256 half tile fill the 128 KB ring. The 4
  // waves of row half p write y = acc (* a_scale * w_scale) + bias in fp32 as [128 rows][64
  // chunks of 16 bytes], chunk c of row r at c ^ (r & 63) (conflict-free both ways), then each
  // of their half-waves takes 16 rows of the half, reads 8 columns per lane and stores 16 bytes
  // per lane, 512 contiguous bytes per row; the other half's waves wait (their accumulators
  // stay live, the writers' are dead once staged, which leaves registers for the residual
  // rows). The math is the direct store's: fp32 y, fp32 res + gate * y, one bf16 rounding. A
  // half-wave loads its residual rows before it stores any of them (the residual may alias C;
  // each row is read and written by the same half-wave), the first RB of them before the
  // staging so that their latency overlaps it. Stored straight from the accumulators (as the split
  // schedule's kernels still do), each wave instruction touches 32 rows x 8 bytes; staged, the
  // epilogue costs 3-16 us less per launch at 4608 x 3072.
  {
    float* yt = reinterpret_cast<float*>(lds);
    const int ch = lane & 31, half = lane >> 5;  // 8-column chunk of a row, which row of two
    const int64_t n = n0 + ch * 8;
    const bool nin = n < N, nfull = n + 8 <= N;  // N % 4 == 0: a chunk is full or half full
    const bool wide_c = (((uintptr_t)P.c & 15) == 0) && (P.ldc % 8 == 0);
    const bool wide_r = (((uintptr_t)P.res & 15) == 0) && (P.ldr % 8 == 0);
    constexpr int RPH = 128 / (2 * WN_WAVES), RB = 4;  // rows per half-wave of the half
    const int hr = wn * 2 + half;                         // this half-wave's first row
    const int64_t mh = m0 + wm * 128;                     // first row of this wave's half
    auto load8 = [&](const bf16* src, bool wide) {  // 8 bf16 (4 when only half the chunk is in)
      if (wide && nfull) return *reinterpret_cast<const u32x4*>(src);
      u32x4 v = {0u, 0u, 0u, 0u};
      const u32x2 lo = *reinterpret_cast<const u32x2*>(src);
      v[0] = lo[0];
      v[1] = lo[1];
      if (nfull) {
        const u32x2 hi = *reinterpret_cast<const u32x2*>(src + 4);
        v[2] = hi[0];
        v[3] = hi[1];
      }
      return v;
    };
    auto load_res = [&](int t) {  // residual row t of this half-wave (t < RPH)
      const int64_t m = mh + hr + t * 2 * WN_WAVES;
      return (m < M && nin) ? load8(P.res + m * P.ldr + n, wide_r) : u32x4{0u, 0u, 0u, 0u};
    };
    auto stage = [&]() {
#pragma unroll
      for (int j = 0; j < TJ; ++j) {
        u32x2 bv[4];
        f32x4 wv[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int64_t nc = n0 + wn * WTN + j * 32 + q * 8 + fhalf * 4;
          const bool nok = nc < N;
          bv[q] = (P.bias && nok) ? *reinterpret_cast<const u32x2*>(P.bias + nc) : u32x2{0u, 0u};
          if constexpr (E == Elem::FP8)
            wv[q] = nok ? *reinterpret_cast<const f32x4*>(reinterpret_cast<const float*>(P.w_scale) + nc)
                        : f32x4{};
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int r = i * 32 + frow;  // row within the half
          float sa = 1.f;
          if constexpr (E == Elem::FP8)
            sa = mh + r < M ? reinterpret_cast<const float*>(P.a_scale)[mh + r] : 0.f;
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const int cl = wn * WTN + j * 32 + q * 8 + fhalf * 4;  // tile column of the 4 values
            f32x4 y;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              float v = acc[i][j][q * 4 + e];
              if constexpr (E == Elem::FP8) v = v * (sa * wv[q][e]);
              y[e] = v + bf16bits_to_f32(e & 1 ? bv[q][e >> 1] >> 16 : bv[q][e >> 1] & 0xffffu);
            }
            *reinterpret_cast<f32x4*>(yt + r * 256 + (((cl >> 2) ^ (r & 63)) << 2)) = y;
          }
        }
      }
    };
    // rows in batches of RB, the next batch's residual loads issued before this batch's math
    // (the first batch's before the staging)
    u32x4 cur[RB];
#pragma unroll
    for (int t = 0; t < RB; ++t) cur[t] = load_res(t);
    auto emit = [&]() {
      // one gate row per batch element: 128 rows lie in one (rows_per_batch % 128 == 0 when a
      // problem holds several); a half past M stores nothing and reads row M - 1's gate
      const int64_t b0 = min(mh, (int64_t)M - 1) / P.rows_per_batch;
      const u32x4 gv = nin ? load8(P.gate + b0 * P.gate_stride + n, false) : u32x4{0u, 0u, 0u, 0u};
#pragma unroll 1
      for (int t0 = 0; t0 < RPH; t0 += RB) {
        u32x4 nxt[RB];
        if (t0 + RB < RPH) {
#pragma unroll
          for (int t = 0; t < RB; ++t) nxt[t] = load_res(t0 + RB + t);
        }
#pragma unroll
        for (int t = 0; t < RB; ++t) {
          const int r = hr + (t0 + t) * 2 * WN_WAVES;  // row within the half
          const int64_t m = mh + r;
          if (m >= M || !nin) continue;
          const f32x4 y0 = *reinterpret_cast<const f32x4*>(yt + r * 256 + (((2 * ch) ^ (r & 63)) << 2));
          const f32x4 y1 = *reinterpret_cast<const f32x4*>(yt + r * 256 + (((2 * ch + 1) ^ (r & 63)) << 2));
          float v[8];
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const float y = e < 4 ? y0[e] : y1[e - 4];
            const uint32_t rw_ = cur[t][e >> 1], gw_ = gv[e >> 1];
            v[e] = bf16bits_to_f32(e & 1 ? rw_ >> 16 : rw_ & 0xffffu) +
                   bf16bits_to_f32(e & 1 ? gw_ >> 16 : gw_ & 0xffffu) * y;
          }
          u32x4 o;
#pragma unroll
          for (int e = 0; e < 4; ++e) o[e] = pack_bf16x2(v[2 * e], v[2 * e + 1]);
          bf16* dst = reinterpret_cast<bf16*>(P.c) + m * P.ldc + n;
          if (wide_c && nfull) {
            *reinterpret_cast<u32x4*>(dst) = o;
          } else {
            *reinterpret_cast<u32x2*>(dst) = u32x2{o[0], o[1]};
            if (nfull) *reinterpret_cast<u32x2*>(dst + 4) = u32x2{o[2], o[3]};
          }
        }
#pragma unroll
        for (int t = 0; t < RB; ++t) cur[t] = nxt[t];
      }
    };
    // the same four barriers on both sides: ring free, half 0 staged, half 0 read, half 1 staged
    if (wm == 0) {
      __syncthreads();
      stage();
      __syncthreads();
      emit();
      __syncthreads();
      __syncthreads();
    } else {
      __syncthreads();
      __syncthreads();
      __syncthreads();
      stage();
      __syncthreads();
      emit();
    }
  }
  }  // tiles of this workgroup
}

// Compute units of the current device (one GEMM workgroup fits a CU: its LDS use is > 80 KB).
static int device_cus() {
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

static int64_t sk_workspace_bytes(int groups) {
  return SK_CTR_BYTES + 2 * (int64_t)groups * SK_SLOT_BYTES;
}

// The schedule of T tiles of nk K stages (cut in units of `gran` stages) on `cus` compute
// units. Whole tiles while the last wave of workgroups would still be >= 92 % full; otherwise
// the full waves run whole tiles and the S tiles of the last one are cut over the XCDs (see
// SkPlan), when each XCD's range is at least SK_MIN_STAGES stages and the cut takes a quarter
// off the launch's K walk (waves * nu units on the busiest workgroup), and at least
// SK_MIN_SAVED_STAGES stages. The cut tiles' partial sums go through memory: 256 KB out and
// back per cut, all CUs at once, which at ~6 TB/s costs about as much as 10-20 % of a
// 3072-deep tile, whatever the K walk saves. On MI355X that pays on Qwen-Image's 336-tile
// launches (FF2 MXFP8 365 -> 316 us, bf16 576 -> 483 us; 60 and 30 stages saved) and Wan's
// 80-tile bf16 text k/v projection (93 -> 87 us, 40 saved), and loses on FLUX's 216-, 648-
// and 864-tile ones (out projection bf16 87 -> 101 us, FF1 fp8 169 -> 198 us) and on the MXFP8
// twin of that k/v projection (49 -> 66 us, 20 saved), which these rules leave whole.
static SkPlan sk_plan(int T, int nk, int gran, int cus, int64_t ws_bytes) {
  const int nu = (nk + gran - 1) / gran;
  SkPlan pl = {T, 0, nu, gran, 0, 0, 0, 0};
  constexpr int NX = 8;
  if (cus <= 0 || T <= 0 || cus % NX != 0) return pl;
  const int waves = (T + cus - 1) / cus;
  if ((double)T >= 0.92 * (double)waves * cus) return pl;
  const int dp = (T / cus) * cus, S = T - dp, g = cus / NX;  // 0 < S < 0.92 cus
  const int ng = (S + g - 1) / g;
  const int64_t units = (int64_t)ng * nu;
  const int64_t span = (units + NX - 1) / NX;
  if (S > SK_MAX_TILES || ws_bytes < sk_workspace_bytes(cus) ||
      units / NX < std::max(1, SK_MIN_STAGES / gran) ||
      4 * (nu - span) < (int64_t)waves * nu || (nu - span) * gran < SK_MIN_SAVED_STAGES)
    return pl;
  pl.dp = dp;
  pl.groups = cus;
  pl.S = S;
  pl.g = g;
  pl.nx = NX;
  pl.units = units;
  return pl;
}

template <Elem E>
static int gemm_launch(const char* name, int nproblems, const difflet_gemm_problem* problems,
                       int64_t n, int64_t k, int epilogue, int64_t act_col_start,
                       void* workspace, int64_t workspace_bytes, const difflet_gemm_qk* qk,
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
  DLT_REQUIRE(epilogue >= DIFFLET_EPI_NONE && epilogue <= DIFFLET_EPI_F32,
              DIFFLET_EINVAL, "%s: unknown epilogue %d", name, epilogue);
  const bool f32_out = epilogue == DIFFLET_EPI_F32;
  DLT_REQUIRE(!f32_out || (E == Elem::BF16 && !qk), DIFFLET_EUNSUPPORTED,
              "%s: the fp32-output epilogue runs on the bf16 GEMM without the q/k norm", name);
  if (f32_out) workspace = nullptr;  // whole tiles
  const bool mx_out = epilogue == DIFFLET_EPI_GELU_MX;
  DLT_REQUIRE(!mx_out || E == Elem::MX, DIFFLET_EUNSUPPORTED,
              "%s: the GELU -> MXFP8 epilogue runs on the MXFP8 GEMM only", name);
  DLT_REQUIRE(!mx_out || (n % 32 == 0 && act_col_start == 0 && !qk), DIFFLET_EINVAL,
              "%s: the GELU -> MXFP8 epilogue needs n %% 32 == 0, act_col_start 0 and no "
              "fused q/k norm", name);
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
                    ((uintptr_t)q.c & (f32_out ? 15 : 7)) == 0,
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
    if (mx_out)
      DLT_REQUIRE(q.c_scale && q.ldc % 8 == 0 && q.ld_c_scale >= n / 32,
                  DIFFLET_EINVAL,
                  "%s: the GELU -> MXFP8 epilogue needs c_scale [m, n / 32] and ldc %% 8 == 0 "
                  "in problem %d", name, i);
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
    DLT_REQUIRE(epilogue != DIFFLET_EPI_GATE_RESIDUAL || d.rows_per_batch >= q.m ||
                    d.rows_per_batch % 128 == 0,
                DIFFLET_EUNSUPPORTED,
                "%s: with several batches per problem, rows_per_batch must be a multiple of 128",
                name);
    d.nq = (const bf16*)q.norm_q;
    d.nk = (const bf16*)q.norm_k;
    d.rope_row0 = q.rope_row0;
    d.cs = (uint8_t*)q.c_scale;
    d.ldcs = q.ld_c_scale;
    DLT_REQUIRE(!qk || (q.rope_row0 >= 0 && ((uintptr_t)q.norm_q & 7) == 0 &&
                        ((uintptr_t)q.norm_k & 7) == 0),
                DIFFLET_EINVAL, "%s: q/k norm weights must be 8-byte aligned, rope_row0 >= 0",
                name);
    d.tiles_m = (int)((q.m + BM - 1) / BM);
    d.tile_start = (int)tiles;
    tiles += (int64_t)d.tiles_m * args.tiles_n;
  }
  for (int i = nproblems; i < MAX_PROBLEMS; ++i) args.p[i].tile_start = 1 << 30;
  if (tiles == 0) return DIFFLET_OK;
  DLT_REQUIRE(tiles < (1LL << 30), DIFFLET_EUNSUPPORTED, "%s: too many tiles", name);
  args.total_tiles = (int)tiles;
  DLT_REQUIRE(workspace_bytes >= 0 && (workspace == nullptr || ((uintptr_t)workspace & 255) == 0),
              DIFFLET_EINVAL, "%s: workspace must be 256-byte aligned", name);
  if (qk) {
    const bool q_on = qk->q_col >= 0, k_on = qk->k_col >= 0;
    DLT_REQUIRE(epilogue != DIFFLET_EPI_GATE_RESIDUAL, DIFFLET_EUNSUPPORTED,
                "%s: the q/k norm epilogue combines with EPI_NONE or EPI_GELU only", name);
    DLT_REQUIRE(qk->cols > 0 && qk->cols % 256 == 0 && (q_on || k_on) &&
                    (!q_on || (qk->q_col % 256 == 0 && qk->q_col + qk->cols <= n)) &&
                    (!k_on || (qk->k_col % 256 == 0 && qk->k_col + qk->cols <= n)) &&
                    (!q_on || !k_on || qk->q_col + qk->cols <= qk->k_col ||
                     qk->k_col + qk->cols <= qk->q_col),
                DIFFLET_EINVAL,
                "%s: q/k columns must be disjoint ranges of n starting and ending at multiples "
                "of 256", name);
    DLT_REQUIRE(epilogue != DIFFLET_EPI_GELU ||
                    ((!q_on || qk->q_col + qk->cols <= act_col_start) &&
                     (!k_on || qk->k_col + qk->cols <= act_col_start)),
                DIFFLET_EINVAL, "%s: q/k columns must lie below act_col_start", name);
    for (int i = 0; i < nproblems; ++i)
      DLT_REQUIRE(problems[i].rope_row0 + problems[i].m <= qk->rows, DIFFLET_EINVAL,
                  "%s: problem %d reads RoPE rows up to %lld of a %lld-row table", name, i,
                  (long long)(problems[i].rope_row0 + problems[i].m), (long long)qk->rows);
    DLT_REQUIRE(qk->cos && qk->sin && ((uintptr_t)qk->cos & 15) == 0 &&
                    ((uintptr_t)qk->sin & 15) == 0 && (qk->law == 0 || qk->law == 1),
                DIFFLET_EINVAL, "%s: RoPE tables (16-byte aligned) and law 0 or 1 required",
                name);
    args.qk_cols = (int)qk->cols;
    args.q_col = q_on ? (int)qk->q_col : -(1 << 30);
    args.k_col = k_on ? (int)qk->k_col : -(1 << 30);
    args.rope_law = qk->law;
    args.qk_eps = qk->eps;
    args.rope_cos = qk->cos;
    args.rope_sin = qk->sin;
  }
  args.sk = sk_plan((int)tiles, (int)(k / KT), E == Elem::MX ? 4 : 1,
                    workspace ? device_cus() : 0, workspace ? workspace_bytes : 0);
  args.ws = (uint8_t*)workspace;
  constexpr int NT = ElemTraits<E>::WN;
  dim3 grid((unsigned)(args.sk.dp + args.sk.groups)), block(128 * NT);
  const bool split = args.sk.groups > 0;
  auto go = [&](auto epi, auto fused) {
    constexpr int EP = decltype(epi)::value;
    constexpr bool Q = decltype(fused)::value;
    if (split)
      hipLaunchKernelGGL((gemm_kernel<E, EP, NT, Q, true>), grid, block, 0, stream, args);
    else
      hipLaunchKernelGGL((gemm_kernel<E, EP, NT, Q, false>), grid, block, 0, stream, args);
  };
  using std::integral_constant;
  switch (epilogue * 2 + (qk ? 1 : 0)) {
    case 2 * DIFFLET_EPI_NONE:
      go(integral_constant<int, DIFFLET_EPI_NONE>{}, std::false_type{});
      break;
    case 2 * DIFFLET_EPI_NONE + 1:
      go(integral_constant<int, DIFFLET_EPI_NONE>{}, std::true_type{});
      break;
    case 2 * DIFFLET_EPI_GELU:
      go(integral_constant<int, DIFFLET_EPI_GELU>{}, std::false_type{});
      break;
    case 2 * DIFFLET_EPI_GELU + 1:
      go(integral_constant<int, DIFFLET_EPI_GELU>{}, std::true_type{});
      break;
    case 2 * DIFFLET_EPI_GELU_MX:
      if constexpr (E == Elem::MX)
        go(integral_constant<int, DIFFLET_EPI_GELU_MX>{}, std::false_type{});
      break;
    case 2 * DIFFLET_EPI_F32:
      if constexpr (E == Elem::BF16)
        go(integral_constant<int, DIFFLET_EPI_F32>{}, std::false_type{});
      break;
    default:
      go(integral_constant<int, DIFFLET_EPI_GATE_RESIDUAL>{}, std::false_type{});
      break;
  }
  return dlt_check_launch(name);
}

}  // namespace dlt

using namespace dlt;

extern "C" int64_t difflet_rocm_gemm_workspace_bytes(void) {
  const int cus = device_cus();
  return cus > 0 ? sk_workspace_bytes(cus) : 0;
}

extern "C" int difflet_rocm_gemm_bf16(int nproblems, const difflet_gemm_problem* problems,
                                      int64_t n, int64_t k, int epilogue,
                                      int64_t act_col_start, void* workspace,
                                      int64_t workspace_bytes, const difflet_gemm_qk* qk,
                                      difflet_stream_t stream) {
  return gemm_launch<Elem::BF16>("gemm_bf16", nproblems, problems, n, k, epilogue,
                                 act_col_start, workspace, workspace_bytes, qk,
                                 (hipStream_t)stream);
}

extern "C" int difflet_rocm_gemm_fp8_rowwise(int nproblems, const difflet_gemm_problem* problems,
                                             int64_t n, int64_t k, int epilogue,
                                             int64_t act_col_start, void* workspace,
                                             int64_t workspace_bytes, const difflet_gemm_qk* qk,
                                      difflet_stream_t stream) {
  return gemm_launch<Elem::FP8>("gemm_fp8_rowwise", nproblems, problems, n, k, epilogue,
                                act_col_start, workspace, workspace_bytes, qk,
                                 (hipStream_t)stream);
}

extern "C" int difflet_rocm_gemm_mxfp8(int nproblems, const difflet_gemm_problem* problems,
                                       int64_t n, int64_t k, int epilogue, int64_t act_col_start,
                                       void* workspace, int64_t workspace_bytes,
                                       const difflet_gemm_qk* qk, difflet_stream_t stream) {
  return gemm_launch<Elem::MX>("gemm_mxfp8", nproblems, problems, n, k, epilogue,
                               act_col_start, workspace, workspace_bytes, qk,
                                 (hipStream_t)stream);
}

// Host walk of the split schedule the kernels follow (same functions): every (tile, K stage)
// runs on exactly one workgroup, each cut tile's contributors are the XCDs the kernels sum, and
// no two pieces share a workspace slot. Returns 0, or the first violated check's number;
// dp / groups receive the plan.
extern "C" int difflet_rocm_gemm_schedule_check(int tiles, int k_stages, int gran, int cus,
                                                int64_t workspace_bytes, int* dp, int* groups) {
  if (tiles <= 0 || k_stages <= 0 || gran <= 0 || cus <= 0) return 1;
  const SkPlan pl = sk_plan(tiles, k_stages, gran, cus, workspace_bytes);
  if (dp) *dp = pl.dp;
  if (groups) *groups = pl.groups;
  if (pl.groups == 0) return pl.dp == tiles ? 0 : 2;
  const int S = pl.S;
  if (pl.dp % cus != 0 || pl.dp + S != tiles || pl.groups != pl.nx * pl.g || pl.groups > cus ||
      pl.units != (int64_t)((S + pl.g - 1) / pl.g) * pl.nu || pl.units > (int64_t)pl.nx * pl.nu)
    return 3;
  if (SK_CTR_BYTES + 2 * (int64_t)pl.groups * SK_SLOT_BYTES > workspace_bytes ||
      S > SK_MAX_TILES)
    return 4;
  std::vector<int> covered((size_t)S * k_stages, 0);  // per (tile, K stage)
  std::vector<int> slot_tile(2 * (size_t)pl.groups, -1);
  for (int s = 0; s < pl.groups; ++s) {  // the kernel's walk
    const int c = s % pl.nx, r = s / pl.nx;
    const int64_t lo = sk_lo(pl, c), hi = sk_lo(pl, c + 1);
    if (hi - lo < std::max(1, SK_MIN_STAGES / gran)) return 5;
    for (int64_t u = lo; u < hi;) {
      const int gi = (int)(u / pl.nu);
      const int64_t g0 = (int64_t)gi * pl.nu;
      const int ub = (int)(u - g0), ue = (int)(std::min(hi, g0 + pl.nu) - g0);
      u = g0 + ue;
      const int tl = gi * pl.g + r;
      if (tl >= S) continue;
      const int kbeg = ub * gran, kend = std::min(ue * gran, k_stages);
      if (kbeg >= kend) return 6;
      for (int k = kbeg; k < kend; ++k) covered[(size_t)tl * k_stages + k] += 1;
      const int c0 = sk_owner(pl, g0), c1 = sk_owner(pl, g0 + pl.nu - 1);
      if (c < c0 || c > c1) return 7;
      if ((kbeg != 0 || kend != k_stages) != (c0 != c1)) return 8;
      if (c0 != c1) {  // a cut tile: this piece's slot
        const int slot = sk_slot(pl, c, r, gi);
        if (slot != 2 * (c * pl.g + r) && slot != 2 * (c * pl.g + r) + 1) return 9;
        if (slot_tile[slot] != -1) return 10;
        slot_tile[slot] = tl;
      }
    }
  }
  for (int v : covered)
    if (v != 1) return 11;
  for (int gi = 0; gi * pl.g < S; ++gi) {  // the owners per the formula hold the group's pairs
    const int64_t x0 = (int64_t)gi * pl.nu, x1 = x0 + pl.nu;
    const int c0 = sk_owner(pl, x0), c1 = sk_owner(pl, x1 - 1);
    if (sk_lo(pl, c0) > x0 || sk_lo(pl, c1 + 1) < x1) return 12;
    if (c0 < c1 && sk_lo(pl, c0 + 1) <= x0) return 13;
  }
  return 0;
}
