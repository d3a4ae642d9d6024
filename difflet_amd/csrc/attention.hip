// Flash attention forward for the DiT's joint / self / cross attention on CDNA4 matrix cores.
//
// out = softmax(q k^T * scale [+ mask]) v with head_dim 128, bf16 or fp16 inputs, fp32 softmax
// statistics and accumulation, one pass over K/V (online softmax), O(S) memory.
//
// Work split: a 256-thread workgroup (4 wavefronts) owns 128 query rows of one (batch, head);
// each wavefront owns 32 of them. K/V stream through LDS in tiles of 64 keys, double-buffered.
// Unmasked attention over more than 1024 keys runs the ping-pong variant (attn_pp_kernel,
// below): 8 wavefronts, 256 queries, two groups alternating MFMA and softmax phases.
//
// Operand roles. Scores are computed transposed, S^T = K Q^T (MFMA 32x32x16, first operand a K
// fragment, second a Q fragment held in registers for the whole kernel), so accumulator lane l
// holds query l % 32 and its registers run over keys. Every softmax statistic of a query then
// lives in two lanes (l and l ^ 32): row max and row sum need one cross-lane exchange, and the
// rescale of the output accumulator is a per-lane multiply. The output is also accumulated
// transposed, O^T += V^T P^T: the P^T operand is the lane's own probabilities (the 8 keys a
// lane holds for a 16-key MFMA step are {4g..4g+3, 8+4g..8+4g+3}, g = l / 32, and the V^T
// operand is read in that same key order), so P never leaves registers.
//
// LDS: K tile row-major [64 keys][128 dims] with a 272-byte row pitch (256 + 16): the K fragment
// reads of 8 or 16 lanes (consecutive keys, one 16-byte chunk) land in distinct bank groups, and
// every fragment address is the lane's base plus an immediate. V tile stored transposed
// [128 dims][64 keys] with a 144-byte row pitch and the key quads of each 16-key group in the
// order 0, 2, 1, 3 (vt_quad_pos): a lane's 8 keys of an MFMA step are one 16-byte read, and the
// reads of 16 lanes (16 dims) cover all banks. Both are written from registers (V transposed in the
// write), one barrier per K/V tile.
//
// VALU budget: the softmax costs about as many instruction cycles as the MFMAs, so the fast
// (unmasked) path folds the scale into one FMA ahead of exp2 (p = exp2(s c - m), the running
// max kept in scaled units, c > 0), checks the key bound only on the last tile, and rescales
// the output only when some lane's running max moved (wave-uniform branch).
//
// Masking follows the reference: masked scores become the lowest finite float (so a fully
// masked row averages V, as softmax over equal finfo.min scores does); keys past seq_k do not
// exist and take -inf.
#include <mutex>
#include <vector>
#include <type_traits>

#include "common.hpp"
#include <float.h>

namespace dlt {

constexpr int HD = 128;
constexpr int BLOCK_M = 128;
constexpr int BLOCK_N = 64;
constexpr int VT_PITCH = BLOCK_N * 2 + 16;  // bytes per V^T row
constexpr int K_PITCH = HD * 2 + 16;         // bytes per K row
constexpr float LOG2E = 1.4426950408889634f;

// The split schedule of one launch (below); groups == 0: one query tile per workgroup.
struct AttPlan {
  int groups;     // workgroups, one per compute unit (a multiple of 8)
  int dp;         // query tiles run whole, a multiple of groups
  int w;          // workgroups per lockstep set of the cut part (divides groups / 8)
  int sets;       // groups / w
  int64_t units;  // (group of w cut tiles, key tile) units: ceil(S / w) * key tiles
};

struct AttnArgs {
  const uint8_t* q;
  const uint8_t* k;
  const uint8_t* v;
  uint8_t* o;
  int64_t qs[3], ks[3], vs[3], os[3];  // element strides: batch, head, seq
  int heads, seq_q, seq_k;
  int q_tiles, total;
  float scale_log2;
  int causal;
  const void* mask;
  int mask_dtype;
  int64_t ms[4];
  const int32_t* bmin;
  const int32_t* bmax;
  int64_t bs[3];
  // split schedule of the ping-pong kernel (sp.groups == 0: one query tile per workgroup)
  AttPlan sp;
  uint8_t* ws;
};

// One additive-mask entry (fp32, bf16 or fp16) at element offset mo.
__device__ inline float load_mask(const AttnArgs& a, int64_t mo) {
  if (a.mask_dtype == DIFFLET_F32) return reinterpret_cast<const float*>(a.mask)[mo];
  if (a.mask_dtype == DIFFLET_BF16) return bf16_to_f32(reinterpret_cast<const bf16*>(a.mask)[mo]);
  return (float)reinterpret_cast<const f16*>(a.mask)[mo];
}

// score + mask * unit (unit converts the mask to the score's units). A finite fill such as
// finfo.min stays finite, as the reference's score + mask does in fp32: a sum that overflows
// from a finite mask value is clamped to the lowest float, so a row whose every key carries the
// fill averages v instead of dividing zero by zero. A -inf mask entry stays -inf.
__device__ inline float add_mask(float x, float add, float unit) {
  const float y = __builtin_fmaf(add, unit, x);
  return (y == -INFINITY && add != -INFINITY) ? -FLT_MAX : y;
}

// Split schedule of the ping-pong kernel, for launches whose last wave of workgroups would leave
// many compute units idle: one workgroup per compute unit. The launch's T query tiles (each of
// nt key tiles) run in two parts, each workgroup running its cut part first:
//  - whole tiles: dp = floor(T / groups) * groups tiles, round r giving workgroup (XCD x,
//    member j) tile r * groups + x * (groups / 8) + j, so the 32 workgroups of an XCD run 32
//    neighbouring query tiles (one or two heads) and walk their keys in lockstep through the
//    XCD's L2;
//  - cut tiles: the S = T - dp others, in groups of w tiles, as (group, key tile) units. The
//    workgroups form `sets` = groups / w lockstep sets of w (an XCD holds groups / 8 / w of
//    them, set s = x * (groups / 8 / w) + j / w, member j % w); set s takes the contiguous unit
//    range [lo(s), lo(s + 1)), and its member m runs tile dp + group * w + m over each unit of
//    the range, so the w workgroups of a set read the same keys of the same few heads at the
//    same time. w is chosen among the divisors of groups / 8 to balance the sets' ranges.
// A query tile cut between sets s0 .. s1 is finished by the last of them to arrive: every
// contributor stores its unnormalized output, running max and running sum to a workspace slot
// and counts itself in the tile's counter; the last one merges the slots in set order (a fixed
// order: the result does not depend on which one arrives last), normalizes and writes the
// output. A set's range cuts at most two groups (its first and its last), hence two slots per
// workgroup.
constexpr int64_t ATT_CTR_BYTES = 16384;                  // one int counter per query tile
constexpr int ATT_MAX_TILES = (int)(ATT_CTR_BYTES / 4);
constexpr int64_t ATT_SLOT_OUT = 8 * 16 * 1024;           // fp32 output: 8 waves x 16 KB
constexpr int64_t ATT_SLOT_BYTES = ATT_SLOT_OUT + 8 * 64 * 8;  // + (max, sum) per lane
__host__ __device__ inline int64_t att_lo(const AttPlan& p, int s) {
  return (int64_t)s * p.units / p.sets;
}
__host__ __device__ inline int att_owner(const AttPlan& p, int64_t x) {  // set holding unit x
  return (int)(((x + 1) * p.sets - 1) / p.units);
}
// slot of set s's part of a tile of the group starting at unit x0 (its first or last cut group)
__host__ __device__ inline int att_slot(const AttPlan& p, int s, int member, int64_t x0) {
  return 2 * (s * p.w + member) + (att_lo(p, s) >= x0 ? 0 : 1);
}

template <typename T> struct MfmaT;
template <> struct MfmaT<bf16> {
  typedef bf16x8 frag;
  // lazy-rescale limit of the ping-pong softmax: every P below it is a finite 16-bit operand
  static constexpr float kLazyLimit = 0x1p20f;
  static __device__ __forceinline__ f32x16 mma(frag a, frag b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ uint32_t pack2(float a, float b) {
    bf16x2 v = {(bf16)a, (bf16)b};
    return __builtin_bit_cast(uint32_t, v);
  }
};
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
template <> struct MfmaT<f16> {
  typedef f16x8 frag;
  static constexpr float kLazyLimit = 0x1p15f;  // fp16's largest finite value is 65504
  static __device__ __forceinline__ f32x16 mma(frag a, frag b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ uint32_t pack2(float a, float b) {
    f16x2 v = {(_Float16)a, (_Float16)b};
    return __builtin_bit_cast(uint32_t, v);
  }
};

__device__ __forceinline__ int k_off(int row, int chunk) { return row * K_PITCH + (chunk << 4); }

// Position of key quad q (keys 4q .. 4q + 3 of a tile) in a V^T row: inside each 16-key group the
// middle quads swap, so the 8 keys a lane group feeds one 16-key MFMA step, {4g .. 4g + 3,
// 8 + 4g .. 8 + 4g + 3}, sit side by side and load as one 16-byte read.
__device__ __forceinline__ int vt_quad_pos(int q) {
  const int r = q & 3;
  return (q & ~3) | (r == 1 ? 2 : r == 2 ? 1 : r);
}

// Ping-pong kernel LDS: K and V tiles both row-major [64 keys][128 dims], filled by direct-to-LDS
// buffer loads (the DMA writes each instruction's 64 lanes x 16 bytes to 1 KB of consecutive
// 16-byte slots, so the layouts are slot maps with padding, not swizzles). K rows take 17 slots
// (272 bytes, the same as k_off): a b128 fragment read of 16 consecutive keys at one chunk hits
// 16 distinct bank groups. V rows take 20 slots (320 bytes) and are read through
// ds_read_b64_tr_b16, which transposes within each 16-lane group: lane j of the group supplies
// the address of 4 dims of key row j / 4, and lane i receives dim i of the 4 rows. A V^T operand
// (8 keys of one dim per lane) is two such reads; their 32 lanes touch 4 rows x 8 chunks, at
// bank groups 4 row + chunk (mod 16), all distinct.
constexpr int PK_SLOTS = 17, PV_SLOTS = 20;
constexpr int PK_BYTES = BLOCK_N * PK_SLOTS * 16, PV_BYTES = BLOCK_N * PV_SLOTS * 16;
static_assert(PK_SLOTS * 16 == K_PITCH, "K fragment reads use k_off");
typedef short v4i16 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void lds_void_t;
typedef __attribute__((address_space(3))) v4i16 lds_v4i16_t;
typedef int i32x4_t __attribute__((ext_vector_type(4)));

// One direct-to-LDS load: 16 bytes per lane at byte offset voff of buffer r into LDS bytes
// [lds_addr + 16 lane, + 16). Written as inline assembly so that the compiler does not track it:
// the builtin makes it wait for every such load before the next LDS read of any address (it
// cannot tell the tile being filled from the ones being read), which put each tile's whole
// load latency in front of the next phase's fragment reads. The kernel waits for these loads
// itself (vmcnt(0) before the barrier that publishes a tile); the compiler's own waits for the
// loads it does track only grow stricter with untracked loads in flight.
// r: the buffer resource's four words (rsrc_words).
__device__ __forceinline__ void dma16(i32x4_t r, const uint8_t* lds_ptr, uint32_t voff) {
  const uint32_t la = (uint32_t)reinterpret_cast<uintptr_t>((lds_void_t*)lds_ptr);
  // s_nop 4: five wait states for a resource word a VALU instruction (v_readlane) may have just
  // written; s_nop 0: one between the M0 write and the load that reads it
  asm volatile("s_nop 4\n\ts_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
               :
               : "s"(la), "v"(voff), "s"(r)
               : "memory", "m0");
}
// The words of make_rsrc's resource: base address, stride 0, `bytes` records, the same flags.
__device__ __forceinline__ i32x4_t rsrc_words(const void* base, uint32_t bytes) {
  const uint64_t a = reinterpret_cast<uint64_t>(base);
  return i32x4_t{(int)(uint32_t)a, (int)(uint32_t)((a >> 32) & 0xffffu), (int)bytes, 0x00020000};
}

// max / sum of x over lanes l and l ^ 32 (the two lanes holding one query's statistics).
// v_permlane32_swap exchanges the upper half of its first operand with the lower half of its
// second: given x twice, the two results hold {x, x of lane l ^ 32} in every lane, so their max
// or sum is the pair's. A VALU instruction, unlike ds_bpermute, so it neither uses the LDS nor
// waits on it.
__device__ __forceinline__ float pair_max(float x) {
  const uint32_t u = __builtin_bit_cast(uint32_t, x);
  const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  return fmaxf(__builtin_bit_cast(float, (uint32_t)r[0]), __builtin_bit_cast(float, (uint32_t)r[1]));
}
__device__ __forceinline__ float pair_sum(float x) {
  const uint32_t u = __builtin_bit_cast(uint32_t, x);
  const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  return __builtin_bit_cast(float, (uint32_t)r[0]) + __builtin_bit_cast(float, (uint32_t)r[1]);
}

// D: head dim, 128 or 64 (T5 / UMT5 encoders). The K tile's row pitch is D * 2 + 16 bytes.
template <typename T, bool MASKED, int D>
__global__ __launch_bounds__(256, 2) void attn_fwd_kernel(const AttnArgs a) {
  typedef typename MfmaT<T>::frag frag;
  constexpr int KP = D * 2 + 16;      // K row pitch
  constexpr int NC = D / 16;          // Q fragments (16 dims each)
  constexpr int NDT = D / 32;         // 32-dim output tiles
  constexpr int KCH = D / 8;          // 16-byte chunks per K row
  __shared__ __attribute__((aligned(16))) uint8_t sk[2][BLOCK_N * KP];
  __shared__ __attribute__((aligned(16))) uint8_t sv[2][D * VT_PITCH];
  auto kofs = [](int row, int chunk) { return row * KP + (chunk << 4); };

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int col = lane & 31, g = lane >> 5;

  // XCD-aware order: each XCD (ids round-robin over 8) gets a contiguous run of tiles, i.e.
  // whole heads, so one head's K/V stays in one L2.
  int bid = blockIdx.x;
  if ((a.total & 7) == 0) bid = (bid & 7) * (a.total >> 3) + (bid >> 3);
  const int bh = bid / a.q_tiles;
  const int qt = bid % a.q_tiles;
  const int b = bh / a.heads, h = bh % a.heads;
  const int q0 = qt * BLOCK_M + wave * 32;
  const int my_q = q0 + col;

  const uint8_t* qp = a.q + (b * a.qs[0] + h * a.qs[1]) * 2;
  const uint8_t* kp = a.k + (b * a.ks[0] + h * a.ks[1]) * 2;
  const uint8_t* vp = a.v + (b * a.vs[0] + h * a.vs[1]) * 2;
  const int64_t qrow = a.qs[2] * 2, krow = a.ks[2] * 2, vrow = a.vs[2] * 2;

  // ---- Q fragments (second MFMA operand): lane holds q row my_q, dims 16c + 8g .. +8
  frag qf[NC];
  {
    const __amdgpu_buffer_rsrc_t rq =
        make_rsrc(qp, (uint32_t)min((int64_t)a.seq_q * qrow, (int64_t)0xffffffff));
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      // rows past seq_q lie past the resource's range and read zero
      qf[c] = __builtin_bit_cast(frag, buf_load16(rq, (uint32_t)(my_q * qrow) + (c * 16 + g * 8) * 2));
    }
  }

  const __amdgpu_buffer_rsrc_t rk =
      make_rsrc(kp, (uint32_t)min((int64_t)a.seq_k * krow, (int64_t)0xffffffff));
  const __amdgpu_buffer_rsrc_t rv =
      make_rsrc(vp, (uint32_t)min((int64_t)a.seq_k * vrow, (int64_t)0xffffffff));

  // staging: K rows (t / KCH + (256 / KCH) i), chunk t % KCH; V keys 4 (t % 16) + i, dims
  // 8 (t / 16) .. +8 (threads past the head's D / 8 dim groups move no V)
  constexpr int KRI = 256 / KCH, NKI = BLOCK_N / KRI;  // K rows per pass, passes
  const int kr = tid / KCH, kc = tid % KCH;
  const int vkg = tid & 15, vdg = tid >> 4;
  const bool v_on = vdg < D / 8;
  const int vt_pos = vt_quad_pos(vkg) * 8;  // byte offset of this thread's key quad in a V^T row
  u32x4 gk[NKI], gv[4];
  auto load_tile = [&](int j0) {
#pragma unroll
    for (int i = 0; i < NKI; ++i) {
      const int key = j0 + kr + KRI * i;
      gk[i] = buf_load16(rk, (uint32_t)(key * krow) + kc * 16);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int vkey = j0 + vkg * 4 + i;
      gv[i] = v_on ? buf_load16(rv, (uint32_t)(vkey * vrow) + vdg * 16) : u32x4{0u, 0u, 0u, 0u};
    }
  };
  auto store_tile = [&](int st) {
#pragma unroll
    for (int i = 0; i < NKI; ++i)
      *reinterpret_cast<u32x4*>(&sk[st][kofs(kr + KRI * i, kc)]) = gk[i];
    if (!v_on) return;
    // transpose: for each of the 8 dims, the 4 keys' 16-bit values side by side
#pragma unroll
    for (int d = 0; d < 8; ++d) {
      const int w = d >> 1, sh = (d & 1) * 16;
      const uint32_t k0 = (gv[0][w] >> sh) & 0xffffu, k1 = (gv[1][w] >> sh) & 0xffffu;
      const uint32_t k2 = (gv[2][w] >> sh) & 0xffffu, k3 = (gv[3][w] >> sh) & 0xffffu;
      u32x2 pk;
      pk[0] = k0 | (k1 << 16);
      pk[1] = k2 | (k3 << 16);
      *reinterpret_cast<u32x2*>(&sv[st][(vdg * 8 + d) * VT_PITCH + vt_pos]) = pk;
    }
  };

  f32x16 acc[NDT];
#pragma unroll
  for (int i = 0; i < NDT; ++i) acc[i] = f32x16{};
  float m_run = -INFINITY, l_run = 0.f;

  int bmin = 0, bmax = a.seq_k;
  if (MASKED && a.bmin && my_q < a.seq_q) {
    bmin = a.bmin[b * a.bs[0] + h * a.bs[1] + (int64_t)my_q * a.bs[2]];
    bmax = a.bmax[b * a.bs[0] + h * a.bs[1] + (int64_t)my_q * a.bs[2]];
  }

  const int ntiles = (a.seq_k + BLOCK_N - 1) / BLOCK_N;
  load_tile(0);
  store_tile(0);
  __syncthreads();

  for (int jt = 0; jt < ntiles; ++jt) {
    const int st = jt & 1;
    const int j0 = jt * BLOCK_N;
    if (jt + 1 < ntiles) load_tile(j0 + BLOCK_N);

    // ---- S^T = K Q^T for 2 x 32 keys
    f32x16 s[2];
#pragma unroll
    for (int kt2 = 0; kt2 < 2; ++kt2) {
      s[kt2] = f32x16{};
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        const frag kf =
            *reinterpret_cast<const frag*>(&sk[st][kofs(kt2 * 32 + col, c * 2 + g)]);
        s[kt2] = MfmaT<T>::mma(kf, qf[c], s[kt2]);
      }
    }

    // ---- scale, mask, online softmax (this lane: query my_q, 32 of the tile's keys)
    // Scores stay raw in the fast path (p = exp2(s * cmul - m)); the masked path scales them
    // first (cmul = 1) so additive masks and finfo.min fills work in scaled units.
    float cmul = a.scale_log2;
    if (MASKED) {
      cmul = 1.0f;
#pragma unroll
      for (int kt2 = 0; kt2 < 2; ++kt2)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int key = j0 + kt2 * 32 + (v >> 2) * 8 + g * 4 + (v & 3);
          float x = s[kt2][v] * a.scale_log2;
          bool masked = key < bmin || key >= bmax || (a.causal && key > my_q);
          if (a.mask && !masked && key < a.seq_k && my_q < a.seq_q) {
            const int64_t mo = b * a.ms[0] + h * a.ms[1] + (int64_t)my_q * a.ms[2] +
                               (int64_t)key * a.ms[3];
            if (a.mask_dtype == DIFFLET_BOOL) {
              masked = reinterpret_cast<const uint8_t*>(a.mask)[mo] == 0;
            } else {
              x = add_mask(x, load_mask(a, mo), LOG2E);
            }
          }
          s[kt2][v] = masked ? -FLT_MAX : x;
        }
    }
    if (j0 + BLOCK_N > a.seq_k) {  // last tile: keys past seq_k do not exist
#pragma unroll
      for (int kt2 = 0; kt2 < 2; ++kt2)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int key = j0 + kt2 * 32 + (v >> 2) * 8 + g * 4 + (v & 3);
          if (key >= a.seq_k) s[kt2][v] = -INFINITY;
        }
    }
    float mx = -INFINITY;
#pragma unroll
    for (int kt2 = 0; kt2 < 2; ++kt2)
#pragma unroll
      for (int v = 0; v < 16; ++v) mx = fmaxf(mx, s[kt2][v]);
    mx = pair_max(mx);
    const float m_new = fmaxf(m_run, mx * cmul);
    const float m_use = m_new == -INFINITY ? 0.f : m_new;
    const float alpha = __builtin_amdgcn_exp2f(m_run - m_use);
    m_run = m_new;
    float ls = 0.f;
    uint32_t pp[2][8];  // P as packed 16-bit pairs, in register order
#pragma unroll
    for (int kt2 = 0; kt2 < 2; ++kt2)
#pragma unroll
      for (int v = 0; v < 16; v += 2) {
        const float p0 = __builtin_amdgcn_exp2f(__builtin_fmaf(s[kt2][v], cmul, -m_use));
        const float p1 = __builtin_amdgcn_exp2f(__builtin_fmaf(s[kt2][v + 1], cmul, -m_use));
        ls += p0 + p1;
        pp[kt2][v >> 1] = MfmaT<T>::pack2(p0, p1);
      }
    l_run = l_run * alpha + ls;
    if (__any(alpha != 1.0f)) {  // the running max moved for some query of this wave
#pragma unroll
      for (int i = 0; i < NDT; ++i)
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[i][v] *= alpha;
    }

    // ---- O^T += V^T P^T, 16 keys per MFMA: keys base + {4g..4g+3, 8+4g..8+4g+3}
#pragma unroll
    for (int kt2 = 0; kt2 < 2; ++kt2)
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        const int base = kt2 * 32 + hh * 16;
        u32x4 pb;
#pragma unroll
        for (int u = 0; u < 4; ++u) pb[u] = pp[kt2][hh * 4 + u];
        const frag pf = __builtin_bit_cast(frag, pb);
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt) {
          const frag vf = *reinterpret_cast<const frag*>(
              &sv[st][(dt * 32 + col) * VT_PITCH + (base + g * 8) * 2]);
          acc[dt] = MfmaT<T>::mma(vf, pf, acc[dt]);
        }
      }

    if (jt + 1 < ntiles) store_tile(st ^ 1);
    __syncthreads();
  }

  // ---- normalize and write: lane holds query my_q, dims dt*32 + (v/4)*8 + 4g + v%4
  const float l_tot = pair_sum(l_run);
  const float inv = 1.0f / l_tot;
  if (my_q < a.seq_q) {
    T* op = reinterpret_cast<T*>(a.o) + b * a.os[0] + h * a.os[1] + (int64_t)my_q * a.os[2];
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        u32x2 w;
        w[0] = MfmaT<T>::pack2(acc[dt][q4 * 4 + 0] * inv, acc[dt][q4 * 4 + 1] * inv);
        w[1] = MfmaT<T>::pack2(acc[dt][q4 * 4 + 2] * inv, acc[dt][q4 * 4 + 3] * inv);
        *reinterpret_cast<u32x2*>(op + dt * 32 + q4 * 8 + g * 4) = w;
      }
  }
}

// Unmasked fast path: ping-pong between two wavefront groups. A 512-thread workgroup owns 256
// queries; waves 0-3 (group A) and 4-7 (group B) each own 128, 32 per wave, and wave w shares
// its SIMD with wave w ^ 4. Time is cut into phases separated by workgroup barriers; in every
// phase one group runs MFMAs (the previous tile's P V and the next tile's scores) while the
// other runs the softmax of its current tile on the VALU, then they swap, so each SIMD's matrix
// core and VALU work on different waves at once. B trails A by one phase:
//   phase 2j:     A: softmax(j), stores V(j), loads V(j + 1)  |  B: P V(j - 1), scores(j + 0)
//   phase 2j + 1: A: P V(j), scores(j + 1)                    |  B: softmax(j), stores K(j + 2),
//                                                                loads K(j + 3)
// K(j) lives in sk[j & 1] (read in phases 2j - 1 and 2j, refilled in 2j + 1), V(j) in sv[j & 1]
// (written in 2j, read in 2j + 1 and 2j + 2). The MFMA group raises its wave priority so the
// SIMD issues its MFMAs first whenever the matrix core frees up.
// Workgroup barrier between ping-pong phases: this wave's LDS reads and writes are done
// (lgkmcnt(0)), then s_barrier. Unlike __syncthreads it does not wait for the global loads in
// flight: those feed the LDS only two phases later, and waiting here exposed their latency.
__device__ __forceinline__ void phase_barrier() {
  __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0), vmcnt / expcnt untouched
  asm volatile("s_barrier" ::: "memory");
}
// The same after this wave's direct-to-LDS loads have landed but for the last VM issued (they
// complete in order): the barrier then publishes the tile the earlier ones filled.
template <int VM>
__device__ __forceinline__ void vm_phase_barrier() {
  static_assert(VM >= 0 && VM < 16, "vmcnt field");
  __builtin_amdgcn_s_waitcnt(0x0070 | VM);  // vmcnt(VM) lgkmcnt(0)
  asm volatile("s_barrier" ::: "memory");
}

template <typename T>
__global__ __launch_bounds__(512, 1) void attn_pp_kernel(const AttnArgs a) {
  typedef typename MfmaT<T>::frag frag;
  // one LDS variable (two K tiles, two V tiles, the split flag): with several, the compiler gives
  // their accesses alias scopes and waits for every direct-to-LDS load before each LDS read
  __shared__ __attribute__((aligned(16))) uint8_t lds[3 * PK_BYTES + 3 * PV_BYTES + 16];
  auto sk = [&](int st) { return lds + st * PK_BYTES; };
  auto sv = [&](int st) { return lds + 3 * PK_BYTES + st * PV_BYTES; };
  volatile int& last_flag = *reinterpret_cast<volatile int*>(lds + 3 * PK_BYTES + 3 * PV_BYTES);

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const bool grp_a = wave < 4;
  const int gt = tid & 255;  // thread index within the group
  const int col = lane & 31, g = lane >> 5;

  const int ntiles = (a.seq_k + BLOCK_N - 1) / BLOCK_N;
  // work: one query tile, or (split schedule) the units of this workgroup's lockstep set in the
  // cut part, then its whole tiles (cut parts first: their merges then overlap the whole tiles
  // of other workgroups instead of all landing at the end; 1-2.5 % faster at 24 x 4608 and
  // 24 x 7145 keys)
  const AttPlan& sp = a.sp;
  int bid = blockIdx.x, set = 0, member = 0, nwhole = 1;
  int64_t u = 0, u_hi = 0;
  if (sp.groups) {
    const int xcd = bid & 7, j = bid >> 3, per = sp.groups >> 3;  // dealt round-robin
    set = xcd * (per / sp.w) + j / sp.w;
    member = j % sp.w;
    bid = xcd * per + j;  // position within a round of whole tiles
    nwhole = sp.dp / sp.groups;
    u = att_lo(sp, set);
    u_hi = att_lo(sp, set + 1);
  } else if ((gridDim.x & 7) == 0) {  // XCD-contiguous runs of query tiles (heads share an L2)
    bid = (bid & 7) * (gridDim.x >> 3) + (bid >> 3);
  }
  bool ran = false;
  int cut = 0;  // cut parts walked so far
  for (int piece = 0;; ++piece) {
  int item, t0 = 0, nt = ntiles;  // key tiles [t0, t0 + nt) run here
  int64_t x0 = 0;                 // a cut tile's group: its first unit
  if (u >= u_hi) {
    const int whole = piece - cut;  // whole tiles run so far
    if (whole >= nwhole) break;
    item = sp.groups ? whole * sp.groups + bid : bid;
  } else {
    const int gi = (int)(u / ntiles);
    x0 = (int64_t)gi * ntiles;
    t0 = (int)(u - x0);
    nt = (int)min((int64_t)(ntiles - t0), u_hi - u);
    u += nt;
    ++cut;
    item = sp.dp + gi * sp.w + member;
    if (item >= a.total) continue;  // the last group has fewer than w tiles
  }
  if (ran) __syncthreads();  // the previous query tile's LDS reads are done
  ran = true;
  const int bh = item / a.q_tiles;
  const int qt = item % a.q_tiles;
  const int b = bh / a.heads, h = bh % a.heads;
  const int my_q = qt * (2 * BLOCK_M) + wave * 32 + col;

  const uint8_t* qp = a.q + (b * a.qs[0] + h * a.qs[1]) * 2;
  const uint8_t* kp = a.k + (b * a.ks[0] + h * a.ks[1]) * 2;
  const uint8_t* vp = a.v + (b * a.vs[0] + h * a.vs[1]) * 2;
  const int64_t qrow = a.qs[2] * 2, krow = a.ks[2] * 2, vrow = a.vs[2] * 2;

  frag qf[8];  // Q fragments (second MFMA operand): row my_q, dims 16c + 8g .. +8
  // Loaded after the prologue's tile loads and waited for with them (vmcnt(0)): the compiler
  // tracks these loads but not the tile loads, and a wait for them still pending at the loop
  // would sit in the loop body, where the hardware counter also holds the tile loads in flight.
  auto load_q = [&]() {
    const __amdgpu_buffer_rsrc_t rq =
        make_rsrc(qp, (uint32_t)min((int64_t)a.seq_q * qrow, (int64_t)0xffffffff));
#pragma unroll
    for (int c = 0; c < 8; ++c)
      qf[c] = __builtin_bit_cast(frag, buf_load16(rq, (uint32_t)(my_q * qrow) + (c * 16 + g * 8) * 2));
    __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0)
  };
  const i32x4_t rk = rsrc_words(kp, (uint32_t)min((int64_t)a.seq_k * krow, (int64_t)0xffffffff));
  const i32x4_t rv = rsrc_words(vp, (uint32_t)min((int64_t)a.seq_k * vrow, (int64_t)0xffffffff));

  // staging by direct-to-LDS loads, 4 waves per tile: group B loads K, group A loads V. A tile
  // of P slots per row is P instructions of 1 KB; wave wb of the group issues instructions
  // n = wb + 4 i. Lane l of instruction n fills slot 64 n + l = (row, slot-in-row); the pad slots
  // load the row's last chunk again (never read). Rows past seq_k load row seq_k - 1 (real,
  // finite data: its keys are masked to -inf and its P is 0), so no LDS row is left stale. The
  // whole offset goes in the per-lane offset, which the buffer's range check covers (the host
  // keeps seq_k + 128 rows within 4 GiB).
  const int wb = wave & 3;
  const int pslots = grp_a ? PV_SLOTS : PK_SLOTS;
  const uint32_t row_bytes = (uint32_t)(grp_a ? vrow : krow);
  uint32_t rc[5];  // (row << 16) | byte offset in the row
#pragma unroll
  for (int i = 0; i < 5; ++i) {
    const int sl = (wb + 4 * i) * 64 + lane;
    rc[i] = ((uint32_t)(sl / pslots) << 16) | (uint32_t)(min(sl % pslots, 15) * 16);
  }
  auto dma_voff = [&](int j0, int i) {
    const uint32_t row = (uint32_t)min(j0 + (int)(rc[i] >> 16), a.seq_k - 1);
    return row * row_bytes + (rc[i] & 0xffffu);
  };
  auto dma_k = [&](int j0, int st) {
#pragma unroll
    for (int i = 0; i < 5; ++i)
      if (wb + 4 * i < PK_SLOTS)
        dma16(rk, sk(st) + (wb + 4 * i) * 1024, dma_voff(j0, i));
  };
  auto dma_v = [&](int j0, int st) {
#pragma unroll
    for (int i = 0; i < 5; ++i)
      dma16(rv, sv(st) + (wb + 4 * i) * 1024, dma_voff(j0, i));
  };
  // V^T fragment reads: lane l of 16-lane group G supplies key row 4 g + (l >> 2) % 4 of the
  // 8-key half and dims 32 dt + 16 (G % 2) + 4 (l % 4); it receives dim 32 dt + l % 32 of keys
  // {4g .. 4g + 3} (first read) and {8 + 4g .. 8 + 4g + 3} (second), the order of its P values
  const uint32_t vl = (uint32_t)((4 * g + ((lane >> 2) & 3)) * (PV_SLOTS * 16) +
                                 32 * ((lane >> 4) & 1) + 8 * (lane & 3));

  f32x16 acc[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) acc[i] = f32x16{};
  f32x16 s[2];          // scores of the tile being softmaxed next
  uint32_t pp[2][8] = {};  // P of the tile being multiplied next, packed 16-bit pairs
  float m_run = -INFINITY, l_run = 0.f;
  const float cmul = a.scale_log2;

  // One MFMA phase: O^T += V^T P^T of the tile in sv(vst), 16 MFMAs (steps 0-15: 16-key block
  // gi = step / 4, output dims 32 dt, dt = step % 4, two transposing 8-byte reads each), then
  // S^T = K Q^T of the tile in sk(kst), 16 MFMAs (steps 16-31: two d-chunks for both 32-key
  // blocks per group of four, one 16-byte read each), so consecutive MFMAs are independent.
  // Fragment reads run ahead of their MFMAs: 6 steps in the P V part (12 reads in flight: the
  // LDS counter holds 15), 12 steps in the scores part; sched_barrier keeps the compiler from
  // pulling each read down next to its MFMA, where every MFMA would wait out an LDS latency.
  auto mfma_phase = [&](int vst, int kst) {
    frag fr[16];  // ring: step t's fragment in fr[t % 16] (at most 13 steps in flight)
    auto issue = [&](int t) {
      if (t < 16) {
        const int gi = t >> 2, dt = t & 3;
        const int base = (gi >> 1) * 32 + (gi & 1) * 16;
        const uint8_t* p = sv(vst) + vl + base * (PV_SLOTS * 16) + dt * 64;
        const v4i16 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16_t*)p);
        const v4i16 hi =
            __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16_t*)(p + 8 * (PV_SLOTS * 16)));
        const u32x2 l2 = __builtin_bit_cast(u32x2, lo), h2 = __builtin_bit_cast(u32x2, hi);
        fr[t & 15] = __builtin_bit_cast(frag, u32x4{l2[0], l2[1], h2[0], h2[1]});
      } else {
        const int u = (t - 16) & 3, kt2 = u & 1, c = 2 * ((t - 16) >> 2) + (u >> 1);
        fr[t & 15] = *reinterpret_cast<const frag*>(sk(kst) + k_off(kt2 * 32 + col, c * 2 + g));
      }
    };
    auto run = [&](int t) {
      if (t < 16) {
        const int gi = t >> 2, dt = t & 3, kt2 = gi >> 1, hh = gi & 1;
        const u32x4 pb = {pp[kt2][hh * 4], pp[kt2][hh * 4 + 1], pp[kt2][hh * 4 + 2],
                          pp[kt2][hh * 4 + 3]};
        acc[dt] = MfmaT<T>::mma(fr[t & 15], __builtin_bit_cast(frag, pb), acc[dt]);
      } else {
        const int u = (t - 16) & 3, kt2 = u & 1, c = 2 * ((t - 16) >> 2) + (u >> 1);
        s[kt2] = MfmaT<T>::mma(fr[t & 15], qf[c], c == 0 ? f32x16{} : s[kt2]);
      }
    };
    constexpr auto upto = [](int t) { return t < 16 ? t + 6 : (t + 12 < 31 ? t + 12 : 31); };
#pragma unroll
    for (int t = 0; t <= upto(0); ++t) issue(t);
#pragma unroll
    for (int t = 0; t < 32; ++t) {
      if (t > 0) {
#pragma unroll
        for (int n = upto(t - 1) + 1; n <= upto(t); ++n) issue(n);
      }
      __builtin_amdgcn_sched_barrier(0);
      run(t);
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  auto scores_only = [&](int st) {  // the prologue's S^T = K Q^T of tile 0
#pragma unroll
    for (int kt2 = 0; kt2 < 2; ++kt2) {
      s[kt2] = f32x16{};
#pragma unroll
      for (int c = 0; c < 8; ++c) {
        const frag kf = *reinterpret_cast<const frag*>(sk(st) + k_off(kt2 * 32 + col, c * 2 + g));
        s[kt2] = MfmaT<T>::mma(kf, qf[c], s[kt2]);
      }
    }
  };
  auto softmax = [&](int j0) {  // online softmax of s (keys j0 ..), P into pp
    if (j0 + BLOCK_N > a.seq_k) {  // last tile: keys past seq_k do not exist
#pragma unroll
      for (int kt2 = 0; kt2 < 2; ++kt2)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int key = j0 + kt2 * 32 + (v >> 2) * 8 + g * 4 + (v & 3);
          if (key >= a.seq_k) s[kt2][v] = -INFINITY;
        }
    }
    // Lazy rescaling without a max on the common path: the exponentials are taken relative to
    // the reference m_run (scaled units; m_run never exceeds the running max, so the largest
    // score seen so far has p >= 1 and the sums cannot vanish). Only when some lane's sum
    // reaches the type's limit (2^20 for bf16, 2^15 for fp16: a score more than 20 or 15 above
    // m_run, the first tile, where m_run is -inf and the sums are inf or NaN, or a large jump)
    // does the wave find the tile's max, move m_run to it, rescale O and l and take the
    // exponentials again. Every P then stays below the limit: exact in the fp32 sums and finite
    // in the 16-bit P operand (bf16 reaches 3.4e38, fp16 only 65504; the relative precision of
    // either does not depend on the magnitude). The result is the same softmax: O and l share
    // the reference m_run, which the final normalization and the split merge divide out.
    auto exps = [&](float m_use) {  // P relative to m_use, and the lane's sum of it
      float ls = 0.f;
#pragma unroll
      for (int kt2 = 0; kt2 < 2; ++kt2)
#pragma unroll
        for (int v = 0; v < 16; v += 2) {
          const float p0 = __builtin_amdgcn_exp2f(__builtin_fmaf(s[kt2][v], cmul, -m_use));
          const float p1 = __builtin_amdgcn_exp2f(__builtin_fmaf(s[kt2][v + 1], cmul, -m_use));
          ls += p0 + p1;
          pp[kt2][v >> 1] = MfmaT<T>::pack2(p0, p1);
        }
      return ls;
    };
    float ls = exps(m_run);
    if (__any(!(ls < MfmaT<T>::kLazyLimit))) {
      float mx = -INFINITY;
#pragma unroll
      for (int kt2 = 0; kt2 < 2; ++kt2)
#pragma unroll
        for (int v = 0; v < 16; ++v) mx = fmaxf(mx, s[kt2][v]);
      mx = pair_max(mx);
      const float m_new = fmaxf(m_run, mx * cmul);
      const float alpha = m_new == -INFINITY ? 1.f : __builtin_amdgcn_exp2f(m_run - m_new);
      m_run = m_new;
      l_run *= alpha;
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[i][v] *= alpha;
      ls = exps(m_run == -INFINITY ? 0.f : m_run);
    }
    l_run += ls;
    // P is computed here, in the softmax phase: without the pins the compiler sinks the
    // exponentials past the rescale branch into the next MFMA phase, where P is first read,
    // and the MFMA wave then runs the softmax itself
#pragma unroll
    for (int kt2 = 0; kt2 < 2; ++kt2)
#pragma unroll
      for (int i = 0; i < 8; ++i) asm volatile("" : "+v"(pp[kt2][i]));
  };

  // The two groups run separate loops with the same barrier sequence (2 + 2 nt barriers), so
  // each loop's registers are allocated for that group alone. Key tiles t0 .. t0 + nt - 1, in a
  // ring of three K and three V buffers (tile j in buffer j mod 3). Loads in flight: K(j + 3) from
  // B's softmax phase 2j + 1 to the barrier ending phase 2j + 4 (A's scores(j + 3) are phase
  // 2j + 5); V(j + 2) from A's MFMA phase 2j + 1 to the barrier ending phase 2j + 4 (A's
  // P V(j + 2) is phase 2j + 5). Each lands in the buffer whose last readers finished in phase
  // 2j. Every iteration issues its loads, past the last tile too (their rows clamp to the last
  // key, in bounds, and nobody reads them), so each barrier waits with one fixed vmcnt that lets
  // the newest tile's loads (4 or 5 instructions per wave) stay in flight.
  const int k0 = t0 * BLOCK_N;
  if (grp_a) {
    dma_v(k0, 0);
    dma_v(k0 + BLOCK_N, 1);
    load_q();
    phase_barrier();  // prologue: B has K(t0) in LDS
    scores_only(0);
    phase_barrier();
    // ring buffers of tiles j, j + 1, j + 2 (rotated, not j % 3: a division the compiler
    // keeps in vector registers)
    int r0 = 0, r1 = 1, r2 = 2;
    for (int jt = 0; jt < nt; ++jt) {
      const int j0 = k0 + jt * BLOCK_N;
      softmax(j0);             // phase 2j
      vm_phase_barrier<5>();  // V(j) landed, V(j + 1) may be in flight
      dma_v(j0 + 2 * BLOCK_N, r2);
      __builtin_amdgcn_s_setprio(1);  // phase 2j + 1 (past the last tile the scores read
      mfma_phase(r0, r1);             // an unused K buffer and go unused)
      __builtin_amdgcn_s_setprio(0);
      phase_barrier();
      const int r = r0;
      r0 = r1, r1 = r2, r2 = r;
    }
  } else {
    dma_k(k0, 0);
    dma_k(k0 + BLOCK_N, 1);
    dma_k(k0 + 2 * BLOCK_N, 2);
    // sv(2) is read as "tile -1" by the first P V (with P = 0): zeros, not stale LDS that
    // could hold NaN patterns
    for (int i = gt; i < PV_BYTES / 16; i += 256)
      *reinterpret_cast<u32x4*>(sv(2) + i * 16) = u32x4{0u, 0u, 0u, 0u};
    load_q();               // with K(t0 .. t0 + 2) landed
    phase_barrier();
    phase_barrier();        // A scores tile 0
    int rp = 2, r0 = 0, r1 = 1;  // ring buffers of tiles j - 1, j, j + 1
    for (int jt = 0; jt < nt; ++jt) {
      const int j0 = k0 + jt * BLOCK_N;
      __builtin_amdgcn_s_setprio(1);  // phase 2j (the first P V is of "tile -1": P = 0)
      mfma_phase(rp, r0);
      __builtin_amdgcn_s_setprio(0);
      vm_phase_barrier<4>();  // K(j + 1) landed, K(j + 2) may be in flight
      softmax(j0);            // phase 2j + 1
      dma_k(j0 + 3 * BLOCK_N, r0);
      phase_barrier();
      const int r = rp;
      rp = r0, r0 = r1, r1 = r;
    }
    mfma_phase(rp, r0);  // phase 2n: the last P V (scores unused)
  }
  __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0): no load into the LDS outlives the tile

  if (nt != ntiles) {
    // a query tile cut between split workgroups: store this part (device-scope sc1 stores,
    // complete before the count, so the last contributor's device-scope loads see them)
    const int c0 = att_owner(sp, x0), c1 = att_owner(sp, x0 + ntiles - 1);
    const __amdgpu_buffer_rsrc_t rs =
        make_rsrc(a.ws + ATT_CTR_BYTES, (uint32_t)(2 * sp.groups * ATT_SLOT_BYTES));
    constexpr int SC1 = 16;
    auto slot = [&](int c) { return (uint32_t)(att_slot(sp, c, member, x0) * ATT_SLOT_BYTES); };
    const uint32_t vo = (uint32_t)lane * 16, mo = (uint32_t)(ATT_SLOT_OUT + (wave * 64 + lane) * 8);
    {
      const uint32_t so = slot(set);
#pragma unroll
      for (int dt = 0; dt < 4; ++dt)
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4) {
          const f32x4 v = {acc[dt][q4 * 4], acc[dt][q4 * 4 + 1], acc[dt][q4 * 4 + 2],
                           acc[dt][q4 * 4 + 3]};
          __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), rs, vo,
                                                 so + (uint32_t)((wave * 16 + dt * 4 + q4) * 1024),
                                                 SC1);
        }
      const u32x2 ml = {__builtin_bit_cast(uint32_t, m_run), __builtin_bit_cast(uint32_t, l_run)};
      __builtin_amdgcn_raw_buffer_store_b64(ml, rs, mo, so, SC1);
    }
    __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0): the stores are complete
    __syncthreads();
    int* ctr = reinterpret_cast<int*>(a.ws) + item;
    if (tid == 0)
      last_flag = __hip_atomic_fetch_add(ctr, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == c1 - c0;
    __syncthreads();
    if (!last_flag) continue;  // another contributor finishes this query tile
    // merge the parts in contributor order: running max, then the rescaled sums
    // (loaded vectors are cast whole: hipcc lowers a bit_cast of one vector element to a read
    // of element 0)
    typedef float f32x2_t __attribute__((ext_vector_type(2)));
    float m_all = -INFINITY;
    for (int c = c0; c <= c1; ++c) {
      const f32x2_t ml =
          __builtin_bit_cast(f32x2_t, __builtin_amdgcn_raw_buffer_load_b64(rs, mo, slot(c), SC1));
      m_all = fmaxf(m_all, ml[0]);
    }
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) acc[dt] = f32x16{};
    l_run = 0.f;
    for (int c = c0; c <= c1; ++c) {
      const uint32_t so = slot(c);
      const f32x2_t ml =
          __builtin_bit_cast(f32x2_t, __builtin_amdgcn_raw_buffer_load_b64(rs, mo, so, SC1));
      const float f = ml[0] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(ml[0] - m_all);
      l_run += f * ml[1];
#pragma unroll
      for (int dt = 0; dt < 4; ++dt) {
        f32x4 v[4];
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4)
          v[q4] = __builtin_bit_cast(
              f32x4, __builtin_amdgcn_raw_buffer_load_b128(
                         rs, vo, so + (uint32_t)((wave * 16 + dt * 4 + q4) * 1024), SC1));
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4)
#pragma unroll
          for (int e = 0; e < 4; ++e) acc[dt][q4 * 4 + e] += f * v[q4][e];
      }
    }
    if (tid == 0) __hip_atomic_store(ctr, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }

  const float inv = 1.0f / pair_sum(l_run);
  if (my_q < a.seq_q) {
    T* op = reinterpret_cast<T*>(a.o) + b * a.os[0] + h * a.os[1] + (int64_t)my_q * a.os[2];
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        u32x2 w;
        w[0] = MfmaT<T>::pack2(acc[dt][q4 * 4 + 0] * inv, acc[dt][q4 * 4 + 1] * inv);
        w[1] = MfmaT<T>::pack2(acc[dt][q4 * 4 + 2] * inv, acc[dt][q4 * 4 + 3] * inv);
        *reinterpret_cast<u32x2*>(op + dt * 32 + q4 * 8 + g * 4) = w;
      }
  }
  }  // query tiles of this workgroup
}

}  // namespace dlt

using namespace dlt;

// Compute units of the current device (one ping-pong workgroup fills a CU's LDS share).
static int att_device_cus() {
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

static int64_t att_workspace_bytes(int groups) {
  return ATT_CTR_BYTES + 2 * (int64_t)groups * ATT_SLOT_BYTES;
}

// The split schedule of T query tiles of nt key tiles on `cus` compute units: none (one query
// tile per workgroup) while the last wave of workgroups would be at least 90 % full; else full
// rounds of whole tiles and the remaining S tiles cut in lockstep sets of w workgroups, w the
// divisor of cus / 8 that gives the sets the fewest key tiles each (the larger on a tie: fewer
// heads per XCD at once), keeping at least one unit per set.
static AttPlan att_plan(int64_t T, int nt, int cus, int64_t ws_bytes) {
  AttPlan p = {0, 0, 0, 0, 0};
  if (cus <= 0 || cus % 8 != 0 || nt <= 0 || T <= cus || T > ATT_MAX_TILES ||
      ws_bytes < att_workspace_bytes(cus))
    return p;
  const int64_t S = T % cus;
  if (S == 0 || S * 10 >= (int64_t)cus * 9) return p;
  const int per = cus / 8;
  int64_t best = -1;
  for (int w = per; w >= 1; --w) {
    if (per % w != 0) continue;
    const int sets = cus / w;
    const int64_t units = (S + w - 1) / w * nt;
    if (units < sets) continue;
    const int64_t steps = (units + sets - 1) / sets;
    if (best < 0 || steps < best) {
      best = steps;
      p.w = w;
      p.sets = sets;
      p.units = units;
    }
  }
  if (best < 0) return p;
  p.groups = cus;
  p.dp = (int)(T - S);
  return p;
}

// Host walk of the split schedule the kernel follows (same functions): every (query tile, key
// tile) runs on exactly one workgroup, each cut tile's contributors are the sets the kernel
// counts, and no two parts share a workspace slot. Returns 0, or the first violated check's
// number; dp and w receive the plan (0 and 0: no split).
extern "C" int difflet_rocm_attention_schedule_check(int64_t tiles, int key_tiles, int cus,
                                                     int64_t workspace_bytes, int* dp, int* w) {
  if (tiles <= 0 || key_tiles <= 0 || cus <= 0) return 1;
  const AttPlan p = att_plan(tiles, key_tiles, cus, workspace_bytes);
  if (dp) *dp = p.dp;
  if (w) *w = p.w;
  if (p.groups == 0) return 0;
  const int per = p.groups / 8;
  if (p.groups != cus || p.dp % cus != 0 || p.dp >= tiles || per % p.w != 0 ||
      p.sets * p.w != p.groups || p.units != (tiles - p.dp + p.w - 1) / p.w * key_tiles ||
      p.units < p.sets)
    return 2;
  std::vector<int> covered((size_t)tiles * key_tiles, 0);
  std::vector<int64_t> slot_tile(2 * (size_t)p.groups, -1);
  std::vector<int> set_seen(p.sets, 0);
  for (int b = 0; b < p.groups; ++b) {  // the kernel's walk, workgroup b
    const int xcd = b & 7, j = b >> 3;
    const int set = xcd * (per / p.w) + j / p.w, member = j % p.w, pos = xcd * per + j;
    set_seen[set] += 1;
    for (int r = 0; r < p.dp / p.groups; ++r) {
      const int64_t item = (int64_t)r * p.groups + pos;
      for (int k = 0; k < key_tiles; ++k) covered[(size_t)item * key_tiles + k] += 1;
    }
    const int64_t lo = att_lo(p, set), hi = att_lo(p, set + 1);
    if (hi <= lo) return 3;
    for (int64_t u = lo; u < hi;) {
      const int gi = (int)(u / key_tiles);
      const int64_t x0 = (int64_t)gi * key_tiles;
      const int t0 = (int)(u - x0);
      const int nt = (int)std::min((int64_t)(key_tiles - t0), hi - u);
      u += nt;
      const int64_t item = p.dp + (int64_t)gi * p.w + member;
      if (item >= tiles) continue;
      for (int k = t0; k < t0 + nt; ++k) covered[(size_t)item * key_tiles + k] += 1;
      const int c0 = att_owner(p, x0), c1 = att_owner(p, x0 + key_tiles - 1);
      if (set < c0 || set > c1) return 4;
      if ((nt != key_tiles) != (c0 != c1)) return 5;
      if (nt != key_tiles) {
        const int sl = att_slot(p, set, member, x0);
        if (sl != 2 * (set * p.w + member) && sl != 2 * (set * p.w + member) + 1) return 6;
        if (slot_tile[sl] != -1) return 7;
        slot_tile[sl] = item;
      }
    }
  }
  for (int v : set_seen)
    if (v != p.w) return 8;
  for (int v : covered)
    if (v != 1) return 9;
  for (int64_t gi = 0; p.dp + gi * p.w < tiles; ++gi) {  // every set in c0 .. c1 holds units
    const int64_t x0 = gi * key_tiles;                   // of the group
    const int c0 = att_owner(p, x0), c1 = att_owner(p, x0 + key_tiles - 1);
    if (att_lo(p, c0) > x0 || att_lo(p, c1 + 1) < x0 + key_tiles) return 10;
    for (int c = c0; c <= c1; ++c)
      if (att_lo(p, c + 1) <= x0 || att_lo(p, c) >= x0 + key_tiles) return 11;
  }
  return 0;
}

extern "C" int64_t difflet_rocm_attention_workspace_bytes(void) {
  const int cus = att_device_cus();
  return cus > 0 ? att_workspace_bytes(cus) : 0;
}

// ---- fp32 inputs (models run in fp32, as the reference's CPU op computes them): scores,
// softmax and P V in fp32 on the VALU, one query per lane, 256 queries per workgroup (64 when
// 256 would leave most compute units idle). K and V tiles of 32 keys go through LDS and are read
// by every lane at the same address (broadcast).
// Online softmax per lane over each tile; masks, bounds, causal and scale as the MFMA kernels.
constexpr int F32_TILE = 32;
template <int D, int NQ>  // NQ: queries (threads) per workgroup, 64 or 256
__global__ __launch_bounds__(NQ, 1) void attn_f32_kernel(const AttnArgs a) {
  __shared__ __attribute__((aligned(16))) float skk[F32_TILE][D];
  __shared__ __attribute__((aligned(16))) float svv[F32_TILE][D];
  const int tid = threadIdx.x;
  const int bh = blockIdx.x / a.q_tiles, qt = blockIdx.x % a.q_tiles;
  const int b = bh / a.heads, h = bh % a.heads;
  const int my_q = qt * NQ + tid;
  const bool qok = my_q < a.seq_q;
  const float* qp = reinterpret_cast<const float*>(a.q) + b * a.qs[0] + h * a.qs[1];
  const float* kp = reinterpret_cast<const float*>(a.k) + b * a.ks[0] + h * a.ks[1];
  const float* vp = reinterpret_cast<const float*>(a.v) + b * a.vs[0] + h * a.vs[1];
  float q[D], o[D];
#pragma unroll
  for (int d = 0; d < D; d += 4) {
    const f32x4 x = qok ? *reinterpret_cast<const f32x4*>(qp + (int64_t)my_q * a.qs[2] + d)
                        : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      q[d + e] = x[e];
      o[d + e] = 0.f;
    }
  }
  int bmin = 0, bmax = a.seq_k;
  if (a.bmin && qok) {
    bmin = a.bmin[b * a.bs[0] + h * a.bs[1] + (int64_t)my_q * a.bs[2]];
    bmax = a.bmax[b * a.bs[0] + h * a.bs[1] + (int64_t)my_q * a.bs[2]];
  }
  const float scale = a.scale_log2 / LOG2E;
  float m_run = -INFINITY, l_run = 0.f;
  for (int j0 = 0; j0 < a.seq_k; j0 += F32_TILE) {
    __syncthreads();  // the previous tile's reads are done
    for (int i = tid; i < F32_TILE * D / 4; i += NQ) {
      const int key = j0 + i / (D / 4), d = (i % (D / 4)) * 4;
      f32x4 kv = {0.f, 0.f, 0.f, 0.f}, vv = {0.f, 0.f, 0.f, 0.f};
      if (key < a.seq_k) {
        kv = *reinterpret_cast<const f32x4*>(kp + (int64_t)key * a.ks[2] + d);
        vv = *reinterpret_cast<const f32x4*>(vp + (int64_t)key * a.vs[2] + d);
      }
      *reinterpret_cast<f32x4*>(&skk[i / (D / 4)][d]) = kv;
      *reinterpret_cast<f32x4*>(&svv[i / (D / 4)][d]) = vv;
    }
    __syncthreads();
    float sc[F32_TILE];
    float mx = -INFINITY;
#pragma unroll 4
    for (int j = 0; j < F32_TILE; ++j) {
      const int key = j0 + j;
      float dot = 0.f;
#pragma unroll
      for (int d = 0; d < D; ++d) dot += q[d] * skk[j][d];
      float x = dot * scale;
      bool masked = key < bmin || key >= bmax || (a.causal && key > my_q);
      if (a.mask && !masked && key < a.seq_k && qok) {
        const int64_t mo = b * a.ms[0] + h * a.ms[1] + (int64_t)my_q * a.ms[2] +
                           (int64_t)key * a.ms[3];
        if (a.mask_dtype == DIFFLET_BOOL) masked = reinterpret_cast<const uint8_t*>(a.mask)[mo] == 0;
        else x = add_mask(x, load_mask(a, mo), 1.0f);
      }
      x = masked ? -FLT_MAX : x;
      if (key >= a.seq_k) x = -INFINITY;  // keys past seq_k do not exist
      sc[j] = x;
      mx = fmaxf(mx, x);
    }
    const float m_new = fmaxf(m_run, mx);
    const float m_use = m_new == -INFINITY ? 0.f : m_new;
    const float alpha = __expf(m_run - m_use);
    m_run = m_new;
    l_run *= alpha;
#pragma unroll
    for (int d = 0; d < D; ++d) o[d] *= alpha;
#pragma unroll 4
    for (int j = 0; j < F32_TILE; ++j) {
      const float p = __expf(sc[j] - m_use);
      l_run += p;
#pragma unroll
      for (int d = 0; d < D; ++d) o[d] += p * svv[j][d];
    }
  }
  if (qok) {
    float* op = reinterpret_cast<float*>(a.o) + b * a.os[0] + h * a.os[1] + (int64_t)my_q * a.os[2];
    const float inv = 1.0f / l_run;
#pragma unroll
    for (int d = 0; d < D; d += 4)
      *reinterpret_cast<f32x4*>(op + d) = f32x4{o[d] * inv, o[d + 1] * inv, o[d + 2] * inv, o[d + 3] * inv};
  }
}

// Counters of the split schedule back to zero before a launch that uses them (a fill kernel,
// not a memset node, so the pair can be captured into a graph).
__global__ void att_zero_counters(int* __restrict__ ctr, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) ctr[i] = 0;
}

// The body of both attention entry points. clear_counters: zero the workspace's counters on
// the stream before a split-schedule launch (the caller-owned workspace is zeroed once by its
// owner and left zeroed by the kernels; the library's own scratch is cleared every time).
static int attention_impl(const char* name, const void* q, const void* k, const void* v,
                          void* o, int dtype, int64_t batch, int64_t heads, int64_t seq_q,
                          int64_t seq_k, int64_t head_dim, const int64_t* q_strides,
                          const int64_t* k_strides, const int64_t* v_strides,
                          const int64_t* o_strides, float scale, int causal, const void* mask,
                          int mask_dtype, const int64_t* mask_strides, const int32_t* bound_min,
                          const int32_t* bound_max, const int64_t* bound_strides,
                          void* workspace, int64_t workspace_bytes, bool clear_counters,
                          difflet_stream_t stream) {
  DLT_REQUIRE(q && k && v && o && q_strides && k_strides && v_strides && o_strides,
              DIFFLET_EINVAL, "attention: null pointer");
  DLT_REQUIRE(dtype == DIFFLET_BF16 || dtype == DIFFLET_F16 || dtype == DIFFLET_F32,
              DIFFLET_EUNSUPPORTED, "attention: dtype %d unsupported (bf16, fp16, fp32)", dtype);
  DLT_REQUIRE(head_dim == HD || head_dim == 64, DIFFLET_EUNSUPPORTED,
              "attention: head_dim %lld unsupported (128 or 64)", (long long)head_dim);
  DLT_REQUIRE(batch >= 0 && heads >= 0 && seq_q >= 0 && seq_k >= 0, DIFFLET_EINVAL,
              "attention: negative size");
  DLT_REQUIRE(seq_q < (1 << 24) && seq_k < (1 << 24) && batch * heads < (1 << 24),
              DIFFLET_EUNSUPPORTED, "attention: sizes too large");
  DLT_REQUIRE(!bound_min == !bound_max, DIFFLET_EINVAL,
              "attention: bound_min and bound_max must both be provided");
  DLT_REQUIRE(!(bound_min && mask), DIFFLET_EINVAL,
              "attention: attention_mask and bounds are mutually exclusive");
  DLT_REQUIRE(!bound_min || bound_strides, DIFFLET_EINVAL, "attention: bound strides missing");
  DLT_REQUIRE(!mask || (mask_strides && (mask_dtype == DIFFLET_BOOL || mask_dtype == DIFFLET_F32 ||
                                         mask_dtype == DIFFLET_BF16 || mask_dtype == DIFFLET_F16)),
              DIFFLET_EINVAL, "attention: bad mask");
  const int64_t* ss[4] = {q_strides, k_strides, v_strides, o_strides};
  const void* ps[4] = {q, k, v, o};
  const int64_t elem_align = dtype == DIFFLET_F32 ? 4 : 8;  // elements per 16 bytes
  for (int i = 0; i < 4; ++i) {
    DLT_REQUIRE(ss[i][2] % elem_align == 0 && ss[i][1] % elem_align == 0 &&
                    ss[i][0] % elem_align == 0 && ((uintptr_t)ps[i] & 15) == 0,
                DIFFLET_EINVAL, "attention: rows must be 16-byte aligned");
  }
  // queries up to one workgroup tile (256) and keys up to two K/V tiles past the end are
  // addressed (and read as zero through the buffer range check), so those byte offsets must
  // fit 32 bits (the fp32 kernel uses 64-bit addresses)
  DLT_REQUIRE(dtype == DIFFLET_F32 || (seq_q + 256) * q_strides[2] * 2 < (1LL << 32) &&
                  (seq_k + 128) * k_strides[2] * 2 < (1LL << 32) &&
                  (seq_k + 128) * v_strides[2] * 2 < (1LL << 32),
              DIFFLET_EUNSUPPORTED, "attention: one head's sequence exceeds 4 GiB");
  if (batch * heads * seq_q == 0) return DIFFLET_OK;
  DLT_REQUIRE(seq_k > 0, DIFFLET_EUNSUPPORTED, "attention: seq_k must be positive");

  AttnArgs args = {};
  args.q = (const uint8_t*)q;
  args.k = (const uint8_t*)k;
  args.v = (const uint8_t*)v;
  args.o = (uint8_t*)o;
  for (int i = 0; i < 3; ++i) {
    args.qs[i] = q_strides[i];
    args.ks[i] = k_strides[i];
    args.vs[i] = v_strides[i];
    args.os[i] = o_strides[i];
  }
  args.heads = (int)heads;
  args.seq_q = (int)seq_q;
  args.seq_k = (int)seq_k;
  // the fast paths need scale > 0 (scores stay raw and are scaled inside exp2); the ping-pong
  // kernel pays a few tiles of pipeline fill, so short key sequences (cross-attention to text)
  // run the single-group kernel
  const bool masked = causal || mask || bound_min || !(scale > 0.0f);
  const bool pingpong = head_dim == HD && !masked && seq_k > 1024;
  const int qblock = pingpong ? 2 * BLOCK_M : BLOCK_M;  // queries per workgroup
  args.q_tiles = (int)((seq_q + qblock - 1) / qblock);
  const int64_t total = (int64_t)args.q_tiles * batch * heads;
  DLT_REQUIRE(total < (1LL << 31), DIFFLET_EUNSUPPORTED, "attention: too many tiles");
  args.total = (int)total;
  args.scale_log2 = scale * LOG2E;
  args.causal = causal;
  args.mask = mask;
  args.mask_dtype = mask_dtype;
  if (mask)
    for (int i = 0; i < 4; ++i) args.ms[i] = mask_strides[i];
  args.bmin = bound_min;
  args.bmax = bound_max;
  if (bound_min)
    for (int i = 0; i < 3; ++i) args.bs[i] = bound_strides[i];
  hipStream_t s = (hipStream_t)stream;
  if (dtype == DIFFLET_F32) {
    const int cus = att_device_cus();
    const bool narrow = (int64_t)((seq_q + 255) / 256) * batch * heads < 2 * (cus > 0 ? cus : 256);
    const int nq = narrow ? 64 : 256;
    args.q_tiles = (int)((seq_q + nq - 1) / nq);
    const int64_t t32 = (int64_t)args.q_tiles * batch * heads;
    DLT_REQUIRE(t32 < (1LL << 31), DIFFLET_EUNSUPPORTED, "%s: too many tiles", name);
    args.total = (int)t32;
    const dim3 g32((unsigned)t32);
    if (head_dim == 64 && narrow) hipLaunchKernelGGL((attn_f32_kernel<64, 64>), g32, dim3(64), 0, s, args);
    else if (head_dim == 64) hipLaunchKernelGGL((attn_f32_kernel<64, 256>), g32, dim3(256), 0, s, args);
    else if (narrow) hipLaunchKernelGGL((attn_f32_kernel<128, 64>), g32, dim3(64), 0, s, args);
    else hipLaunchKernelGGL((attn_f32_kernel<128, 256>), g32, dim3(256), 0, s, args);
    return dlt_check_launch(name);
  }
  dim3 grid((unsigned)total);
  if (pingpong && workspace) {
    // split schedule when the last wave of workgroups would leave > 10 % of the CUs idle
    const int cus = att_device_cus();
    args.sp = att_plan(total, (int)((seq_k + BLOCK_N - 1) / BLOCK_N), cus, workspace_bytes);
    if (args.sp.groups) {
      args.ws = (uint8_t*)workspace;
      grid = dim3((unsigned)cus);
      if (clear_counters) {
        const int n = (int)total;  // one counter per query tile
        hipLaunchKernelGGL(att_zero_counters, dim3((unsigned)((n + 255) / 256)), dim3(256), 0,
                           s, reinterpret_cast<int*>(workspace), n);
        const int st = dlt_check_launch(name);
        if (st != DIFFLET_OK) return st;
      }
    }
  }
  auto fwd = [&](auto t, auto d) {
    using TT = decltype(t);
    constexpr int DD = decltype(d)::value;
    if (masked) hipLaunchKernelGGL((attn_fwd_kernel<TT, true, DD>), grid, dim3(256), 0, s, args);
    else hipLaunchKernelGGL((attn_fwd_kernel<TT, false, DD>), grid, dim3(256), 0, s, args);
  };
  using D64 = std::integral_constant<int, 64>;
  using D128 = std::integral_constant<int, 128>;
  if (dtype == DIFFLET_BF16) {
    if (pingpong) hipLaunchKernelGGL((attn_pp_kernel<bf16>), grid, dim3(512), 0, s, args);
    else if (head_dim == 64) fwd(bf16{}, D64{});
    else fwd(bf16{}, D128{});
  } else {
    if (pingpong) hipLaunchKernelGGL((attn_pp_kernel<f16>), grid, dim3(512), 0, s, args);
    else if (head_dim == 64) fwd(f16{}, D64{});
    else fwd(f16{}, D128{});
  }
  return dlt_check_launch(name);
}

extern "C" int difflet_rocm_attention(const void* q, const void* k, const void* v, void* o,
                                      int dtype, int64_t batch, int64_t heads, int64_t seq_q,
                                      int64_t seq_k, int64_t head_dim, const int64_t* q_strides,
                                      const int64_t* k_strides, const int64_t* v_strides,
                                      const int64_t* o_strides, float scale, int causal,
                                      const void* mask, int mask_dtype,
                                      const int64_t* mask_strides, const int32_t* bound_min,
                                      const int32_t* bound_max, const int64_t* bound_strides,
                                      void* workspace, int64_t workspace_bytes,
                                      difflet_stream_t stream) {
  return attention_impl("attention", q, k, v, o, dtype, batch, heads, seq_q, seq_k, head_dim,
                        q_strides, k_strides, v_strides, o_strides, scale, causal, mask,
                        mask_dtype, mask_strides, bound_min, bound_max, bound_strides, workspace,
                        workspace_bytes, false, stream);
}

// ---- attention that allocates nothing: the split schedule's workspace is this file's static
// device array. Each device holds its own copy (69.2 MB, for up to 256 compute units) from
// module load until the process ends; every call on a device shares it, so calls that overlap
// in time on one device race (one stream, or calls ordered by events, is safe).
constexpr int ATT_SCRATCH_GROUPS = 256;
constexpr int64_t ATT_SCRATCH_BYTES = ATT_CTR_BYTES + 2 * (int64_t)ATT_SCRATCH_GROUPS * ATT_SLOT_BYTES;
static __device__ __align__(256) uint8_t scratch[ATT_SCRATCH_BYTES];

// The device address of `scratch` on the current device, looked up once per device with that
// device current (in host code the array's name is not a device address).
static void* att_scratch_ptr(int* err) {
  static std::mutex mu;
  static void* ptrs[64] = {nullptr};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) {
    *err = 1;
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(mu);
  if (ptrs[dev] == nullptr) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr) {
      dlt_set_error("attention_noalloc: hipGetSymbolAddress of the scratch array failed on "
                    "device %d: %s", dev, hipGetErrorString(e));
      *err = 2;
      return nullptr;
    }
    ptrs[dev] = p;
  }
  return ptrs[dev];
}

extern "C" int difflet_rocm_attention_noalloc(const void* q, const void* k, const void* v,
                                              void* o, int dtype, int64_t batch, int64_t heads,
                                              int64_t seq_q, int64_t seq_k, int64_t head_dim,
                                              const int64_t* q_strides, const int64_t* k_strides,
                                              const int64_t* v_strides, const int64_t* o_strides,
                                              float scale, int causal, const void* mask,
                                              int mask_dtype, const int64_t* mask_strides,
                                              const int32_t* bound_min, const int32_t* bound_max,
                                              const int64_t* bound_strides,
                                              difflet_stream_t stream) {
  const int cus = att_device_cus();
  DLT_REQUIRE(cus > 0, DIFFLET_ELAUNCH, "attention_noalloc: no device");
  DLT_REQUIRE(cus <= ATT_SCRATCH_GROUPS, DIFFLET_EUNSUPPORTED,
              "attention_noalloc: the device has %d compute units; the static scratch holds the "
              "split schedule of at most %d (%lld bytes)", cus, ATT_SCRATCH_GROUPS,
              (long long)ATT_SCRATCH_BYTES);
  int err = 0;
  void* ws = att_scratch_ptr(&err);
  if (err == 1) {
    dlt_set_error("attention_noalloc: no current device");
    return DIFFLET_ELAUNCH;
  }
  if (err) return DIFFLET_ELAUNCH;
  return attention_impl("attention_noalloc", q, k, v, o, dtype, batch, heads, seq_q, seq_k,
                        head_dim, q_strides, k_strides, v_strides, o_strides, scale, causal,
                        mask, mask_dtype, mask_strides, bound_min, bound_max, bound_strides, ws,
                        att_workspace_bytes(cus), true, stream);
}
