/*
 * difflet_rocm.h -- the C ABI of the MI355X (gfx950) DiT denoise-step kernels.
 *
 * One shared library, libdifflet_rocm.so, exports these entry points. They are what the
 * `rocm` backend of Difflet's backend-neutral op surface binds (through ctypes, from
 * difflet_amd/backends/rocm/ops_impl/ *.py and difflet_amd/quant/), in place of the torch
 * calls the CUDA backend makes. Each declaration names the reference interface it replaces.
 *
 * Conventions shared by every entry point:
 *   - Pointers are device pointers the caller allocated; no entry point allocates, frees or
 *     synchronizes. Work is enqueued on `stream` (a hipStream_t; NULL is the null stream).
 *   - Shapes and strides are int64 element counts. The innermost dimension is contiguous.
 *   - Return value: DIFFLET_OK (0) or an error code; difflet_rocm_last_error() then holds a
 *     message (thread-local).
 *   - Inference only: there are no backward entry points.
 */
#ifndef DIFFLET_ROCM_H
#define DIFFLET_ROCM_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void* difflet_stream_t;

enum difflet_dtype {
  DIFFLET_F32 = 0,
  DIFFLET_BF16 = 1,
  DIFFLET_F16 = 2,
  DIFFLET_U8 = 3,   /* raw bytes: fp8 e4m3fn codes, E8M0 scales */
  DIFFLET_BOOL = 4, /* one byte per element, nonzero = attend */
  DIFFLET_I32 = 5
};

enum difflet_status {
  DIFFLET_OK = 0,
  DIFFLET_EINVAL = 1,       /* bad shape, stride, pointer or dtype */
  DIFFLET_EUNSUPPORTED = 2, /* a valid request this build does not implement */
  DIFFLET_ELAUNCH = 3       /* the HIP runtime refused the launch */
};

/* Library identity and error reporting. */
const char* difflet_rocm_last_error(void);
const char* difflet_rocm_version(void);
int difflet_rocm_abi_version(void);
/* Number of gfx950 devices the library can launch on (0 when none). */
int difflet_rocm_device_count(void);

/* ------------------------------------------------------------------------------------------
 * Attention.
 * Replaces difflet/backends/cuda/ops_impl/attention.py:41-86 (`attention` / `_sdpa`); the
 * semantics are the CPU oracle's, difflet/backends/cpu/ops_impl/attention.py:8-48:
 *   out = softmax(q k^T * scale [+ mask]) v, softmax in fp32, output in v's dtype.
 * q: [batch, heads, seq_q, head_dim] addressed by strides {b, h, s}; k, v: [.., seq_k, ..];
 * o: like q. head_dim 64 or 128; dtype BF16 or F16 (matrix-core kernels) or F32 (a VALU
 * kernel, one query per lane).
 * causal: key j > query i is masked. mask: optional, [batch, heads, seq_q, seq_k] through
 * strides (0 broadcasts); BOOL (nonzero attends) or F32/BF16/F16 additive. bound_min /
 * bound_max: optional int32 [batch, heads, seq_q] through strides; keys in [min, max) attend
 * (difflet/backends/cpu/ops_impl/attention.py:24-35). Masked scores take the dtype's lowest
 * finite value, so a fully masked row averages v exactly as the reference does.
 * workspace / workspace_bytes: optional device memory for the split schedule of unmasked
 * attention over more than 1024 keys. When the launch's 256-query tiles would leave the last
 * wave of workgroups under 90 % full, one workgroup per compute unit runs the last round's
 * query tiles cut along the keys over lockstep sets of workgroups (the workgroups of a set read
 * the same key tiles together), then the full rounds of whole tiles; query tiles cut
 * between sets are merged, in a fixed order, by the last contributor (a deterministic result;
 * the summation order differs from the unsplit one by fp32 rounding). With workspace NULL or too small every query tile runs whole.
 * The workspace must be zero-filled once when allocated (the kernels leave it zeroed), and
 * launches that may overlap in time must not share one.
 * ---------------------------------------------------------------------------------------- */
int difflet_rocm_attention(const void* q, const void* k, const void* v, void* o, int dtype,
                           int64_t batch, int64_t heads, int64_t seq_q, int64_t seq_k,
                           int64_t head_dim, const int64_t* q_strides, const int64_t* k_strides,
                           const int64_t* v_strides, const int64_t* o_strides, float scale,
                           int causal, const void* mask, int mask_dtype,
                           const int64_t* mask_strides, const int32_t* bound_min,
                           const int32_t* bound_max, const int64_t* bound_strides,
                           void* workspace, int64_t workspace_bytes, difflet_stream_t stream);

/* Bytes of attention workspace the split schedule needs on the current device: 16 KiB of
 * counters + 2 x 132 KiB per compute unit (0 without a device). No counterpart in the
 * reference, whose attention calls torch's SDPA (difflet/backends/cuda/ops_impl/attention.py:41-86). */
int64_t difflet_rocm_attention_workspace_bytes(void);

/* Host-side check of the attention's split schedule for `tiles` query tiles of `key_tiles` key
 * tiles on `cus` compute units with `workspace_bytes` of workspace: each (query tile, key tile)
 * runs on exactly one workgroup, and cut tiles are merged from the right contributors and
 * slots. Returns 0 or the number of the failed check; *dp / *w receive the whole-tile count and
 * the workgroups per lockstep set (0 and 0: no split). Runs on the CPU only (for tests). */
int difflet_rocm_attention_schedule_check(int64_t tiles, int key_tiles, int cus,
                                          int64_t workspace_bytes, int* dp, int* w);

/* difflet_rocm_attention with no workspace argument, allocating nothing: no counterpart in the
 * reference. It is for callers that cannot allocate device memory (code under HIP graph
 * capture, serving loops, harnesses that forbid hipMalloc). Same arguments, semantics and
 * results as difflet_rocm_attention given a workspace (the same kernels and schedule). The
 * split schedule's workspace is instead a static device array of the library: 69.2 MB per
 * device (16 KiB of counters + 2 x 132 KiB for each of up to 256 compute units), held from
 * module load until the process ends; a device with more compute units is refused
 * (DIFFLET_EUNSUPPORTED). Its address is looked up on a device's first call, so make that
 * first call outside capture. The counters are cleared on the stream by a small fill kernel
 * before each split launch. Every call on one device shares the array: calls that may overlap
 * in time on one device (different streams without ordering) race. */
int difflet_rocm_attention_noalloc(const void* q, const void* k, const void* v, void* o,
                                   int dtype, int64_t batch, int64_t heads, int64_t seq_q,
                                   int64_t seq_k, int64_t head_dim, const int64_t* q_strides,
                                   const int64_t* k_strides, const int64_t* v_strides,
                                   const int64_t* o_strides, float scale, int causal,
                                   const void* mask, int mask_dtype, const int64_t* mask_strides,
                                   const int32_t* bound_min, const int32_t* bound_max,
                                   const int64_t* bound_strides, difflet_stream_t stream);

/* ------------------------------------------------------------------------------------------
 * GEMM with fused epilogues: for each problem p, C_p = epilogue(A_p W_p^T + bias_p).
 * Replaces F.linear in difflet/backends/_torch_megatron/linear.py:120-126,189-202 (and the
 * CPU twins difflet/backends/cpu/ops_impl/linear.py:9-41), plus the elementwise tails the
 * FLUX blocks apply to linear outputs: GELU-tanh (difflet/layers/activations.py:59-65),
 * gate * (x + bias) + residual (difflet/models/flux/modeling_flux.py:720-731,840-866).
 * All problems of one call share n, k and the epilogue; each has its own A, W, C, M.
 * ---------------------------------------------------------------------------------------- */
enum difflet_epilogue {
  DIFFLET_EPI_NONE = 0,           /* C = acc + bias */
  DIFFLET_EPI_GELU = 1,           /* C = gelu_tanh(acc + bias) for columns >= act_col_start */
  DIFFLET_EPI_GATE_RESIDUAL = 2,  /* C = residual + gate[batch] * (acc + bias) */
  /* MXFP8 GEMM only: y = gelu_tanh(acc + bias) on every column, rounded to bf16, then
   * quantized to MXFP8 in blocks of 32 consecutive columns (the block law of
   * difflet/quant/mx.py:85-108): C receives the e4m3 codes (one byte per element, row stride
   * ldc bytes) and c_scale the E8M0 scales [m, n / 32] (row stride ld_c_scale bytes). With W's
   * rows (and the bias) in the swizzle order of difflet/quant/mx.py:65-76 over n, C and c_scale
   * are difflet_rocm_quantize_mxfp8 (swizzled) of the bf16 GELU output in logical order: the
   * next MXFP8 GEMM's A operand (a feed-forward's hidden activation), written once. n % 32 == 0,
   * act_col_start 0, no fused q/k norm; ldc and ld_c_scale multiples of 8. The reference's
   * device MX linear quantizes its activations inside the matmul kernel
   * (difflet/backends/neuron/ops_impl/fp8_kernels.py:46-58). */
  DIFFLET_EPI_GELU_MX = 3,
  /* bf16 GEMM only: C = acc + bias stored as fp32 (C [m, n] fp32, row stride ldc floats, 16-byte
   * aligned), no fused q/k norm, never split: the fp32 scores of the VAE decoders' mid-block
   * attention (one head of all channels, 384 or 512 wide, which the flash kernels do not
   * take), whose reference (SDPA in the model dtype) keeps them in fp32 before the softmax. */
  DIFFLET_EPI_F32 = 4
};

typedef struct difflet_gemm_problem {
  const void* a;        /* [m, k], row stride lda (bf16, or e4m3 codes for the fp8 GEMMs) */
  int64_t lda;
  const void* w;        /* [n, k], row stride ldw */
  int64_t ldw;
  void* c;              /* [m, n] bf16, row stride ldc */
  int64_t ldc;
  const void* bias;     /* [n] bf16 or NULL */
  const void* gate;     /* GATE_RESIDUAL: [batches, n] bf16, batch stride gate_stride */
  int64_t gate_stride;
  const void* residual; /* GATE_RESIDUAL: [m, n] bf16, row stride ldr (may alias c) */
  int64_t ldr;
  const void* a_scale;  /* fp8 GEMMs: per-row scales of A (see each entry point) */
  const void* w_scale;  /* fp8 GEMMs: per-column (per-row of W) scales */
  int64_t m;
  int64_t rows_per_batch; /* rows of A per batch element, for gate indexing (>= m for one) */
  const void* norm_q;   /* fused q/k norm (difflet_gemm_qk): [128] bf16 RMSNorm weights of q */
  const void* norm_k;   /*   and of k for this problem's rows (NULL: weight 1) */
  int64_t rope_row0;    /*   RoPE table row of this problem's row 0 */
  void* c_scale;        /* EPI_GELU_MX: E8M0 scales of C [m, n / 32], row stride ld_c_scale */
  int64_t ld_c_scale;
} difflet_gemm_problem;

/* Optional fused q/k RMSNorm + RoPE epilogue (EPI_NONE or EPI_GELU), for attention
 * projections whose output holds q and k heads of 128 columns: in columns [q_col, q_col + cols)
 * and [k_col, k_col + cols) each head's 128 values of a row are rounded to bf16 (the plain
 * GEMM's output), scaled by rsqrt(mean of squares + eps) and the problem's norm weights, rotated
 * by the fp32 tables cos / sin [rows, 128] at row rope_row0 + m (law 0: interleaved pairs with
 * per-element angles, 1: the reference's stride-2 form) and stored as bf16: the result of the
 * GEMM followed by difflet_rocm_qk_norm_rope (do_norm 1), up to fp32 summation order. q_col,
 * k_col and cols are multiples of 256 (q_col or k_col -1 skips that part); with EPI_GELU the
 * columns lie below act_col_start. Replaces the pair linear + norm_q/norm_k + apply_rotary_emb
 * of the reference's attention processors (difflet/models/flux/modeling_flux.py:616-949). */
typedef struct difflet_gemm_qk {
  int64_t q_col, k_col, cols;
  const float* cos;
  const float* sin;
  int law;
  float eps;
  int64_t rows;  /* rows of cos / sin: every problem needs rope_row0 + m <= rows */
} difflet_gemm_qk;

/* Workspace of the GEMMs below (all three take the same one). With a workspace, a launch whose
 * output tiles would leave the last wave of workgroups less than 92 % full runs its full waves
 * as whole tiles and cuts the last wave's tiles along K over the 8 XCDs: in groups of 32 tiles,
 * each XCD takes a contiguous range of (group, K unit) pairs and its 32 workgroups walk the
 * same K units of 32 neighbouring tiles together (whole-tile L2 sharing is kept). The cut is
 * made only when it takes a quarter and at least 24 K stages off the launch's K walk
 * (Qwen-Image's 336-tile projections qualify; FLUX's 216-tile ones, which would save an
 * eighth, stay whole, and so does an MXFP8 projection of 512 rows at K = 4096). The workgroup
 * finishing a cut tile adds the fp32 partial sums of the others in a fixed order, so results
 * are deterministic for a given device. With workspace NULL (or too small) every tile runs
 * whole on one workgroup. The workspace must be zero-filled once when allocated; the GEMMs
 * leave it zeroed. Launches that may overlap in time (different streams) must not share one.
 * Returns the bytes needed on the current device: 16 KiB of counters + 2 x 256 KiB per compute
 * unit. No counterpart in the reference, whose linears call the vendor BLAS
 * (torch.nn.functional.linear, difflet/backends/cpu/ops_impl/linear.py:9-41). */
int64_t difflet_rocm_gemm_workspace_bytes(void);

/* bf16 x bf16 -> fp32 accumulate -> bf16. k % 64 == 0. */
int difflet_rocm_gemm_bf16(int nproblems, const difflet_gemm_problem* problems, int64_t n,
                           int64_t k, int epilogue, int64_t act_col_start, void* workspace,
                           int64_t workspace_bytes, const difflet_gemm_qk* qk,
                           difflet_stream_t stream);

/* fp8 e4m3 x e4m3 with per-row scales: acc * a_scale[m] * w_scale[n] (both fp32), then the
 * epilogue. a_scale / w_scale come from difflet_rocm_quantize_fp8_rowwise. k % 128 == 0.
 * New format, no reference counterpart (the reference's only fp8 recipe is MXFP8,
 * difflet/quant/spec.py:22-33); it is the per-channel x per-token linear of the FLUX fp8 step. */
int difflet_rocm_gemm_fp8_rowwise(int nproblems, const difflet_gemm_problem* problems,
                                  int64_t n, int64_t k, int epilogue, int64_t act_col_start,
                                  void* workspace, int64_t workspace_bytes,
                                  const difflet_gemm_qk* qk, difflet_stream_t stream);

/* MXFP8: e4m3 codes in swizzled K order with one E8M0 scale (uint8) per 32 values along K,
 * a_scale [m, k/32] and w_scale [n, k/32] (row strides k/32). Replaces the nkilib
 * `matmul_mxfp8` call of difflet/backends/neuron/ops_impl/fp8_kernels.py:30-71,101-125 and
 * computes what difflet/quant/fake_linear.py:56-61 (FakeQuantMXLinear.forward) computes.
 * k % 128 == 0. */
int difflet_rocm_gemm_mxfp8(int nproblems, const difflet_gemm_problem* problems, int64_t n,
                            int64_t k, int epilogue, int64_t act_col_start, void* workspace,
                            int64_t workspace_bytes, const difflet_gemm_qk* qk,
                            difflet_stream_t stream);

/* Host-side check of the split schedule the GEMMs use for `tiles` output tiles of `k_stages`
 * K stages, cut in units of `gran` stages (1; 4 for MXFP8), on `cus` compute units with
 * `workspace_bytes` of workspace: each (tile, stage) runs on exactly one workgroup, and cut
 * tiles are summed from the right contributors and slots. Returns 0 or the number of the failed
 * check; *dp / *groups receive the whole-tile count and the number of split workgroups. Runs on
 * the CPU only (for tests). */
int difflet_rocm_gemm_schedule_check(int tiles, int k_stages, int gran, int cus,
                                     int64_t workspace_bytes, int* dp, int* groups);

/* ------------------------------------------------------------------------------------------
 * Quantizers (bit-exact with the CPU laws).
 * ---------------------------------------------------------------------------------------- */
/* Per-row e4m3: amax = max|x|, a = max(amax, 2^-112), scale = a / 448, inv = 448 / a,
 * q = e4m3_rne(clamp(x * inv, -448, 448)) (IEEE fp32 ops). scale: fp32 [rows]. Used for
 * per-token activations and per-output-channel weights. No reference counterpart (see
 * difflet_rocm_gemm_fp8_rowwise). */
int difflet_rocm_quantize_fp8_rowwise(const void* x, int dtype, int64_t rows, int64_t cols,
                                      int64_t ldx, uint8_t* q, int64_t ldq, float* scale,
                                      difflet_stream_t stream);

/* difflet_rocm_quantize_fp8_rowwise of y, where y = x on columns below act_col_start and
 * y = bf16(gelu_tanh(x)) from act_col_start on (difflet/layers/activations.py:59-65): the GELU
 * of an MLP's bf16 pre-activation applied where the per-token fp8 activation is quantized, so the
 * producing GEMM stores the pre-activation with a plain epilogue. x bf16, cols <= 16384,
 * act_col_start a multiple of 8. Part of this library's per-token fp8 law (no reference
 * counterpart, like difflet_rocm_quantize_fp8_rowwise). */
int difflet_rocm_quantize_fp8_rowwise_gelu(const void* x, int dtype, int64_t rows, int64_t cols,
                                           int64_t ldx, uint8_t* q, int64_t ldq, float* scale,
                                           int64_t act_col_start, difflet_stream_t stream);

/* MXFP8 block law of difflet/quant/mx.py:46-108 (`swizzle_perm`, `_block_scales`,
 * `quantize_mx`): blocks are consecutive 32 values in swizzle order, scale_u8 =
 * clamp(max exponent field - 7, 0, 255), q = e4m3_rne(clamp(x / 2^(scale_u8 - 127), +-448)).
 * swizzled_out = 0 stores codes in logical K order (the reference's storage); 1 stores them in
 * swizzle order, the operand order difflet_rocm_gemm_mxfp8 reads. scale: uint8 [rows, cols/32]
 * row stride lds. cols % 128 == 0. */
int difflet_rocm_quantize_mxfp8(const void* x, int dtype, int64_t rows, int64_t cols,
                                int64_t ldx, uint8_t* q, int64_t ldq, uint8_t* scale,
                                int64_t lds, int swizzled_out, difflet_stream_t stream);

/* ------------------------------------------------------------------------------------------
 * Normalization and modulation.
 * ---------------------------------------------------------------------------------------- */
/* LayerNorm over the last dim (fp32 statistics, biased variance) then an affine:
 *   one_plus = 1: y = LN(x) * (1 + mul[b]) + add[b]   (adaLN: difflet/layers/normalization.py
 *                 :81-84,141-147,185-190; Wan difflet/models/wan/modeling_wan.py:741-763)
 *   one_plus = 0: y = LN(x) * mul + add               (nn.LayerNorm, difflet/backends/cpu/
 *                 ops_impl/norm.py:9); mul / add may be NULL (no affine).
 * mul / add: [batches, dim] of mod_dtype with batch stride mod_stride, batch = row /
 * rows_per_batch; or, with split > 0, two segments: rows < split use mul / add and rows >=
 * split use mul + mod_stride / add + mod_stride (mod_stride may be negative), e.g. the text and
 * image rows of a joint block in one launch with their own modulation vectors. */
int difflet_rocm_layernorm_modulate(const void* x, int64_t ldx, void* y, int64_t ldy,
                                    int dtype, int out_dtype, int64_t rows, int64_t dim,
                                    const void* mul, const void* add, int mod_dtype,
                                    int64_t mod_stride, int64_t rows_per_batch, int64_t split,
                                    int one_plus, float eps, difflet_stream_t stream);

/* difflet_rocm_layernorm_modulate with bf16 output followed by difflet_rocm_quantize_fp8_rowwise,
 * in one pass and bit-identical with that pair: the modulated row is rounded to bf16, then
 * q[row] = e4m3(clamp(y * 448 / a)), scale[row] = a / 448, a = max(max|y|, 2^-112). It feeds
 * the per-token fp8 linears that follow an adaLN (the q/k/v and MLP-in projections of
 * difflet/models/flux/modeling_flux.py:840-866; the per-row fp8 format is this library's). */
int difflet_rocm_layernorm_modulate_fp8(const void* x, int64_t ldx, uint8_t* q, int64_t ldq,
                                        float* scale, int dtype, int64_t rows, int64_t dim,
                                        const void* mul, const void* add, int mod_dtype,
                                        int64_t mod_stride, int64_t rows_per_batch,
                                        int64_t split, int one_plus, float eps,
                                        difflet_stream_t stream);

/* difflet_rocm_layernorm_modulate's output rounded to bf16 and quantized to MXFP8 in one pass,
 * in the layout the MXFP8 GEMM reads: the result equals difflet_rocm_quantize_mxfp8 (swizzled)
 * of the bf16 LayerNorm + modulation output, bit for bit: codes q [rows, dim] in swizzle order
 * (row stride ldq bytes) and E8M0 scales [rows, dim / 32] (row stride ld_scale bytes), the block
 * law of difflet/quant/mx.py:85-108. It feeds the MXFP8 linears that follow an adaLN (the
 * q/k/v and MLP-in projections of difflet/models/qwen_image/modeling_qwen.py:241-281, Wan's
 * cross-attention q and FFN-in, difflet/models/wan/modeling_wan.py:735-763), which quantize
 * their activations per call (difflet/backends/neuron/ops_impl/fp8_kernels.py:46-58).
 * x bf16; mul / add bf16 or fp32; dim a multiple of 512 (whole swizzle tiles), at most 8192;
 * ldq and ld_scale multiples of 16; every pointer 16-byte aligned. */
int difflet_rocm_layernorm_modulate_mx(const void* x, int64_t ldx, uint8_t* q, int64_t ldq,
                                       uint8_t* scale, int64_t ld_scale, int dtype, int64_t rows,
                                       int64_t dim, const void* mul, const void* add,
                                       int mod_dtype, int64_t mod_stride, int64_t rows_per_batch,
                                       int64_t split, int one_plus, float eps,
                                       difflet_stream_t stream);

/* RMSNorm with fp32 statistics, normalisation and affine and one cast back to dtype: the
 * law of rms_norm_fp32 (difflet/backends/_torch_megatron/norm.py:35-45) and of the CUDA
 * backend's RMSNorm (difflet/backends/cuda/ops_impl/norm.py:24-44). weight may be NULL. */
int difflet_rocm_rms_norm(const void* x, int64_t ldx, void* y, int64_t ldy, int dtype,
                          int64_t rows, int64_t dim, const void* weight, int wdtype, float eps,
                          difflet_stream_t stream);

/* Fused q/k RMSNorm + rotary embedding, in place, on rows of a projection buffer: for each
 * row r and head h, x = buf[r * ld + off + h * head_dim .. +head_dim] for off in (q_off, k_off)
 * (an offset < 0 skips that tensor), x <- rope(rmsnorm_fp32(x) * w) with
 *   do_norm 0: no norm; 1: the RMS of each head, w [head_dim] (FLUX / Qwen-Image per-head
 *   q/k norm); 2: one RMS over all heads * head_dim values of the row, w [heads * head_dim]
 *   (Wan's rms_norm_across_heads, difflet/models/wan/modeling_wan.py:564-578 via
 *   difflet/backends/_torch_megatron/norm.py:35-45), and the rotary law
 *   law 0: difflet/backends/_torch_megatron/embeddings.py:24-33 (apply_rotary_emb_fp32,
 *          interleaved pairs, fp32, cast back);
 *   law 1: difflet/backends/cpu/ops_impl/embeddings.py:6-14 (apply_rotary_emb: cos of the
 *          even, sin of the odd table entries).
 * Replaces the norm_q/norm_k + apply_rotary_emb sequence of difflet/models/flux/
 * modeling_flux.py:1249-1252,1289-1294,1407-1411. cos / sin: fp32 [rope_rows, head_dim], row
 * index r % rope_rows; NULL skips the rotation. wq / wk NULL: unit weights. With
 * 0 < split < rows, rows >= split use the weights wq2 / wk2 (the image rows of a joint block
 * whose text rows come first). */
int difflet_rocm_qk_norm_rope(void* buf, int64_t ld, int dtype, int64_t rows, int64_t heads,
                              int64_t head_dim, int64_t q_off, int64_t k_off, int do_norm,
                              const void* wq, const void* wk, int64_t split, const void* wq2,
                              const void* wk2, int wdtype, float eps, const float* cos,
                              const float* sin, int64_t rope_rows, int law,
                              difflet_stream_t stream);

/* Rotary embedding out of place on a strided [batch*heads, seq, head_dim] tensor with tables
 * [seq, head_dim] (row index s % rope_rows); laws as above. Replaces apply_rotary_emb /
 * apply_rotary_emb_fp32 of the op surface (difflet/ops/embeddings.py:12-25). */
int difflet_rocm_rope(const void* x, void* y, int dtype, int64_t outer, int64_t seq,
                      int64_t head_dim, int64_t x_outer_stride, int64_t x_seq_stride,
                      int64_t y_outer_stride, int64_t y_seq_stride, const float* cos,
                      const float* sin, int64_t rope_rows, int law, difflet_stream_t stream);

/* ------------------------------------------------------------------------------------------
 * Elementwise and small-M kernels.
 * ---------------------------------------------------------------------------------------- */
/* y = gelu_tanh(x), n elements (difflet/layers/activations.py:59-65). */
int difflet_rocm_gelu_tanh(const void* x, void* y, int dtype, int64_t n, difflet_stream_t stream);

/* y[r, :] = residual[r, :] + gate[b, :] * x[r, :] (fp32 math, one rounding), [rows, dim]
 * (the gate/residual tails of difflet/models/flux/modeling_flux.py:840-866). */
int difflet_rocm_gate_residual(const void* residual, const void* x, const void* gate, void* y,
                               int dtype, int gate_dtype, int64_t rows, int64_t dim,
                               int64_t gate_stride, int64_t rows_per_batch,
                               difflet_stream_t stream);

/* y[i, n] = sum_k act(x[i, k]) w[n, k] + bias[n] for m <= 8 rows: the adaLN modulation
 * linears `linear(silu(emb))` of difflet/layers/normalization.py:81,141,187 and the timestep
 * MLPs, HBM-bound on W. act: 0 none, 1 SiLU. x, bias, y: dtype; w: bf16 [n, k] row stride ldw. */
int difflet_rocm_gemv(const void* x, int dtype, int64_t m, int64_t k, int64_t ldx,
                      const void* w, int64_t ldw, int64_t n, const void* bias, void* y,
                      int64_t ldy, int act, difflet_stream_t stream);

/* Sinusoidal timestep embedding of difflet/layers/embeddings.py:422-473
 * (get_timestep_embedding): t fp32 [m] -> y [m, dim] in dtype. */
int difflet_rocm_timestep_embedding(const float* t, void* y, int dtype, int64_t m,
                                    int64_t dim, int flip_sin_to_cos, float downscale_freq_shift,
                                    float scale, float max_period, difflet_stream_t stream);

/* ------------------------------------------------------------------------------------------
 * Text encoders (T5-XXL for FLUX, UMT5-XXL for Wan): the steps before the denoise loop.
 * ---------------------------------------------------------------------------------------- */
/* C[m, :n] = A[m, :k] W[:n, :k]^T (+ bias[n]) (+ residual[m, n]), every operand fp32, on the
 * fp32 matrix cores: the linears of a model loaded in fp32, which the reference runs as
 * F.linear (ColumnParallelLinear / RowParallelLinear, difflet/backends/cpu/ops_impl/
 * linear.py:9-41; the T5 FFN keeps `wo` in fp32: difflet/models/flux/t5/modeling_t5.py:139-149).
 * k and n multiples of 4, leading dimensions multiples of 4, pointers 16-byte aligned; residual
 * may alias c. */
int difflet_rocm_gemm_f32(const float* a, int64_t lda, const float* w, int64_t ldw,
                          const float* bias, const float* residual, int64_t ldr, float* c,
                          int64_t ldc, int64_t m, int64_t n, int64_t k, difflet_stream_t stream);

/* y[r, c] = gelu_tanh(x[r, c]) * x[r, f + c] for c < f: the gated FFN's act(wi_0(h)) * wi_1(h)
 * with gelu_new (difflet/models/flux/t5/modeling_t5.py:133-136,
 * difflet/models/wan/umt5/modeling_umt5.py:125-128), both projections in one [rows, 2 f]
 * buffer. f, ldx and ldy multiples of 8. */
int difflet_rocm_gated_gelu(const void* x, int64_t ldx, void* y, int64_t ldy, int dtype,
                            int64_t rows, int64_t f, difflet_stream_t stream);

/* out[i, :] = table[ids[i], :] for n int64 ids, rows of row_bytes bytes (any element type);
 * strides in bytes. ParallelEmbedding at tp = 1 (F.embedding: difflet/backends/cpu/ops_impl/
 * linear.py:44-53). The reference raises on an id outside [0, table_rows); the caller checks
 * the ids, and the kernel writes a zero row for such an id rather than reading past the table. */
int difflet_rocm_embedding(const int64_t* ids, int64_t n, const void* table, int64_t table_rows,
                           int64_t ldt_bytes, void* out, int64_t ldo_bytes, int64_t row_bytes,
                           difflet_stream_t stream);

/* The T5 relative position bias with the key padding folded in, fp32 [batch, heads, seq_q,
 * seq_k]: out[b, h, q, k] = table[buckets[k - q + seq_q - 1], h] (table [num_buckets, heads]
 * in table_dtype), or the lowest finite float where key_keep[b, k] == 0 (key_keep null: no
 * padding). buckets[j] is the bucket of relative position j - (seq_q - 1) (compute_bias and
 * _relative_position_bucket: difflet/models/flux/t5/modeling_t5.py:200-269,
 * difflet/models/wan/umt5/modeling_umt5.py:196-242; the padding mask of modeling_umt5.py:
 * 354-358). A bucket outside [0, num_buckets) gives NaN. */
int difflet_rocm_relative_bias(const int32_t* buckets, int num_buckets, const void* table,
                               int table_dtype, int64_t heads, int64_t batch, int64_t seq_q,
                               int64_t seq_k, const uint8_t* key_keep, int64_t keep_stride,
                               float* out, difflet_stream_t stream);

/* ------------------------------------------------------------------------------------------
 * VAE decoder (FLUX's: diffusers' 2D Decoder, difflet/models/flux/vae/modeling_vae.py:107-117,
 * difflet/backends/neuron/flux/vae.py:25-36). Channels-last activations [batch][pixels][C].
 * ---------------------------------------------------------------------------------------- */
/* Bytes of workspace difflet_rocm_group_norm needs for these sizes. */
int64_t difflet_rocm_group_norm_workspace_bytes(int64_t batch, int64_t pixels, int64_t channels,
                                                int64_t groups);

/* GroupNorm over channels-last x (bf16 or fp32): per (batch, group) mean and population
 * variance in fp32 / double, y = (x - mean) / sqrt(var + eps) * weight + bias (fp32 vectors,
 * either may be null), then SiLU when act == 1. PatchedGroupNorm / nn.GroupNorm + SiLU of the
 * decoder's resnets and output (modeling_vae.py:39-68: F.group_norm in fp32). channels a
 * multiple of 8 and of groups, <= 2048; y may alias x. */
int difflet_rocm_group_norm(const void* x, void* y, int dtype, int64_t batch, int64_t pixels,
                            int64_t channels, int64_t groups, const float* weight,
                            const float* bias, float eps, int act, void* workspace,
                            int64_t workspace_bytes, difflet_stream_t stream);

/* im2col of a 3x3, padding 1 convolution over one channels-last image [height][width][C]
 * (bf16 or fp32), for output pixels row0 .. row0 + rows - 1: out [rows][ldo], row r = the 9
 * taps' C channels (tap 3 ky + kx) around output pixel row0 + r = (y, x), zero outside the
 * image, columns 9 C .. kpad zero. upsample == 1 first doubles the image by nearest neighbour
 * (Upsample2D's interpolate before its conv), so Ho = 2 height. The GEMM of out with the weight
 * [Cout][ky][kx][C] is that range of the convolution (nn.Conv2d(k=3, padding=1)). */
int difflet_rocm_im2col3x3(const void* x, int dtype, int64_t height, int64_t width,
                           int64_t channels, int upsample, int64_t row0, int64_t rows, void* out,
                           int64_t ldo, int64_t kpad, difflet_stream_t stream);

/* p[r, :] = softmax(s[r, :] * scale) for fp32 scores, p in dtype (bf16 or fp32): the mid-block
 * attention's upcast softmax (one head of 512 channels, whose head width the flash kernels do
 * not take). */
int difflet_rocm_softmax_rows(const float* s, int64_t lds, void* p, int64_t ldp, int dtype,
                              int64_t rows, int64_t cols, float scale, difflet_stream_t stream);

/* ------------------------------------------------------------------------------------------
 * Wan's 3D causal VAE decoder (WanVAEDecoderModel, difflet/models/wan/vae/modeling_vae.py:509-560;
 * the same decoder serves Qwen-Image's one latent frame). Frames channels-last, decoded one
 * latent frame (chunk) at a time, each causal convolution keeping the last two frames of its
 * input as the next chunk's cache (modeling_vae.py:121-134, 225-268).
 * ---------------------------------------------------------------------------------------- */
/* im2col of a causal (kt, ks, ks) convolution, kt and ks in {1, 3} (WanCausalConv3d with
 * padding (kt - 1, ks / 2, ks / 2) front-only in time, modeling_vae.py:95-134; ks = 3, kt = 1 is
 * the resampler's nn.Conv2d(3, padding=1) per frame, with upsample == 1 its nearest 2x first,
 * :163-226). Chunk frame f lies at x + (f / frames_per_block) * frame_stride + (f %
 * frames_per_block) * sub_stride, pixel stride pixel_stride (elements); frames_per_block 2 reads
 * the time convolution's [t][pixels][2C] output as its interleaved frames 2t, 2t + 1
 * (modeling_vae.py:219-221). Frames -2 and -1 come from cache [2][height * width][channels]
 * (zeros when cache is null: the first chunk's zero padding). out [rows][ldo]: row r is output
 * row row0 + r = (frame, y, x) of the chunk at the output resolution, columns ((dt ks + ky) ks +
 * kx) C + c, zero from kt ks^2 C to kpad; the GEMM with the weight [Cout][kt][ks][ks][C] is that
 * range of the convolution. channels, strides, kpad, ldo multiples of 16 bytes. */
int difflet_rocm_im2col_causal(const void* x, int64_t frame_stride, int64_t frames_per_block,
                               int64_t sub_stride, int64_t pixel_stride, const void* cache,
                               int dtype, int64_t height, int64_t width, int64_t channels,
                               int64_t kt, int64_t ks, int upsample, int64_t row0, int64_t rows,
                               void* out, int64_t ldo, int64_t kpad, difflet_stream_t stream);

/* The causal convolution whose rows difflet_rocm_im2col_causal writes, times its packed weight,
 * as one implicit GEMM (the rows are gathered stage by stage, never written): out[r][o] =
 * bias[o] + sum_k row_r[k] w[o][k] (+ residual[r][o]) for the frames * Ho * Wo output pixels r
 * of the chunk and o < n, rounded once. bf16 runs on the bf16 matrix cores (the rows gathered
 * into the LDS), fp32 on the fp32 GEMM (difflet_rocm_gemm_f32's tiles); the products and their
 * order are those of the im2col rows' GEMM of the dtype (bf16: difflet_rocm_gemm, whole tiles),
 * so the two agree bit for bit, unless the workspace (difflet_rocm_conv_causal_workspace_bytes; null
 * and 0 always run whole tiles) lets a small convolution cut its K stages. It replaces
 * WanCausalConv3d.forward and the resampler's Conv2d (modeling_vae.py:121-134, 163-226) in the
 * Wan decoder's bf16 path, and with kt = 1 and one frame the FLUX decoder's 3x3 convolutions
 * (diffusers' Decoder, difflet/models/flux/vae/modeling_vae.py:107-117). Calls on one stream
 * may share a workspace; calls that overlap may not. Chunk frame f (f >= -2) lies
 * at buffer frame b = f + lead_frames of x (x_elems elements): at x + (b / frames_per_block) *
 * frame_stride + (b % frames_per_block) * sub_stride, pixel stride pixel_stride; b < 0 reads
 * zero. A causal convolution passes its two-frame cache as buffer frames 0 and 1 (lead_frames
 * 2); lead_frames 0 with kt = 3 is the first chunk's zero padding. w [n][kpad], the weight
 * [Cout][kt][ks][ks][C] zero-padded to kpad (a multiple of 64 for bf16, 4 for fp32) columns
 * and n (a multiple of 4) rows; bias [n] or null; residual [rows][ldr] or null, may equal out
 * [rows][ldo]; all of x's dtype. Channels and strides multiples of 16 bytes; bf16 frames span
 * under 2 GiB. */
int difflet_rocm_conv_causal(const void* x, int64_t x_elems, int64_t frame_stride,
                             int64_t frames_per_block, int64_t sub_stride, int64_t pixel_stride,
                             int64_t lead_frames, int dtype, int64_t height, int64_t width,
                             int64_t channels, int64_t kt, int64_t ks, int upsample,
                             int64_t frames, const void* w, int64_t n, int64_t kpad,
                             const void* bias, const void* residual, int64_t ldr, void* out,
                             int64_t ldo, void* workspace, int64_t workspace_bytes,
                             difflet_stream_t stream);

/* Workspace bytes difflet_rocm_conv_causal uses (bf16) for rows = frames * Ho * Wo output
 * pixels, n weight rows and kpad columns on the current device: nonzero when the convolution is too
 * small to fill the compute units (under half a wave of tiles) and its K stages are then cut
 * into ranges whose fp32 partial sums are added in order by a second kernel (the result then
 * differs from the whole-tile GEMM's by fp32 summation order). A smaller workspace runs whole
 * tiles. */
int64_t difflet_rocm_conv_causal_workspace_bytes(int64_t rows, int64_t n, int64_t kpad);

/* WanRMSNorm over the channels of each row (pixel), then SiLU when act == 1
 * (modeling_vae.py:137-160, F.normalize in fp32): y = x sqrt(C) / max(||x||_2, eps) * gamma
 * (fp32 gamma [C]), bf16 or fp32 rows of stride ldx / ldy; channels a multiple of 8, <= 2048; y
 * may alias x. */
int difflet_rocm_rms_norm_channels(const void* x, int64_t ldx, void* y, int64_t ldy, int dtype,
                                   int64_t rows, int64_t channels, const float* gamma, float eps,
                                   int act, difflet_stream_t stream);

/* out[c][q] = clamp(x[q][c], lo, hi) for q < n, c < channels (x rows of stride ld): the
 * decoder's channels-last output as the [C][frames * pixels] planes of a [B, C, T, H, W] video,
 * with the final clamp to [-1, 1] (modeling_vae.py:557). */
int difflet_rocm_rows_to_planes(const void* x, int64_t ld, int dtype, int64_t n,
                                int64_t channels, void* out, float lo, float hi,
                                difflet_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* DIFFLET_ROCM_H */
