/*
 * libqlora_gfx950 — C-ABI of the MI355X (gfx950) QLoRA training-step kernel set.
 *
 * Each entry point replaces one Triton kernel (or torch GEMM call site) of the reference's
 * `solution/` package together with its host-side launch; the reference file:line it
 * replaces is cited on each declaration. The Python façades in `hackathon_amd/` keep the
 * reference's function signatures and call these through ctypes.
 *
 * Conventions
 *   - All tensor arguments are raw DEVICE pointers; sizes and strides are in ELEMENTS.
 *   - `stream` is a hipStream_t (NULL = the legacy null stream). Every call only enqueues
 *     work on `stream`; nothing synchronises the host, nothing allocates device memory.
 *   - Return value: QL_OK (0) on success; a negative QL_E* code for a rejected argument
 *     (nothing was launched); a positive hipError_t code if the launch itself failed.
 *     No entry point throws across the ABI.
 *   - dtype tags: QL_F32 / QL_F16 / QL_BF16 (storage of fp16/bf16 is IEEE binary16 /
 *     bfloat16 bits). All arithmetic is fp32; every store to a 16-bit type is RNE.
 */
#ifndef QLORA_GFX950_H
#define QLORA_GFX950_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { QL_F32 = 0, QL_F16 = 1, QL_BF16 = 2 };

enum {
  QL_OK = 0,
  QL_EINVAL = -1, /* null pointer, negative size, unsupported blocksize/flag */
  QL_EDTYPE = -2, /* dtype tag or dtype combination not supported */
  QL_EALIGN = -3, /* pointer/stride alignment a kernel requires is not met */
  QL_ESHAPE = -4  /* inconsistent sizes */
};

typedef void* ql_stream_t; /* hipStream_t */

/* Library identification and error text. qlora_abi_version() is 3 for the signatures in this
 * file (version 1 had no `slots` argument in the qlora_lora_down / qlora_lora_wgrad family;
 * version 2 wrote qlora_lora_pack_group's bt as [16, N] instead of [16 count, N]). */
int qlora_abi_version(void);
const char* qlora_strerror(int status);

/*
 * NF4 dequantisation with optional double-quantised absmax.
 * Replaces: solution/nf4.py:25-49 (nf4_dequant_kernel) + solution/nf4.py:71-92
 * (dequantize_nf4's unpacking of QuantState and launch).
 *
 *   packed   uint8[n_weights/2]; byte i holds weight 2i in its HIGH nibble and weight
 *            2i+1 in its LOW nibble (solution/nf4.py:30,45-47).
 *   nested=1 absmax is uint8[ceil(n/blocksize)] codes; the block scale is
 *              s = code2[absmax[blk]] * absmax2[blk / blocksize2] ; s = s + offset
 *            with two separate fp32 roundings (no FMA contraction).
 *   nested=0 absmax is float32[ceil(n/blocksize)] and s = absmax[blk].
 *   out[j] = round_to(out_dtype, nf4_table[nibble_j] * s),  blk = j / blocksize.
 * n_weights must be even; blocksize (and blocksize2 when nested) even and >= 2.
 * out_dtype: QL_BF16, QL_F16 or QL_F32.
 */
int qlora_nf4_dequant(const uint8_t* packed, int64_t n_weights, const void* absmax, int nested,
                      const float* code2, const float* absmax2, float offset, int blocksize,
                      int blocksize2, const float* nf4_table, void* out, int out_dtype,
                      ql_stream_t stream);

/*
 * NF4 quantisation with optional double-quantised absmax: the format qlora_nf4_dequant reads.
 *   per block of `blocksize` weights: absmax = max |w|; code = nearest NF4 level (nf4_code,
 *   16 sorted fp32) of w * (1/absmax), ties to the lower level; packed two per byte, high
 *   nibble first.  nested = 0: absmax (fp32 [nblocks]) is written as is.
 *   nested = 1: offset = mean(absmax) accumulated in fp64, rounded to fp32 (*offset); absmax
 *   (uint8 [nblocks]) = nearest code2 level (256 sorted fp32) of (absmax - offset) / absmax2,
 *   with absmax2 (fp32 [ceil(nblocks/256)]) the max |absmax - offset| of each 256-block
 *   (blocksize2 must be 256). Workspace: qlora_nf4_quantize_workspace_size bytes, 16-B aligned.
 * n even, blocksize even; w_dtype QL_F32 / QL_F16 / QL_BF16.
 * Replaces: bitsandbytes' quantize_4bit(..., compress_statistics=True) that produces the
 * QuantState solution/nf4.py:73-86 reads (solution/test_kernels.py:41-52).
 */
int64_t qlora_nf4_quantize_workspace_size(int64_t n, int blocksize, int nested);
int qlora_nf4_quantize(const void* w, int w_dtype, int64_t n, int blocksize, int nested,
                       int blocksize2, const float* nf4_code, const float* code2, uint8_t* packed,
                       void* absmax, float* absmax2, float* offset, void* workspace,
                       int64_t workspace_bytes, ql_stream_t stream);

/*
 * RMSNorm forward over rows of length n_cols (frozen weight).
 * Replaces: solution/rmsnorm.py:24-39 (rmsnorm_fwd_kernel) + :64-78 (launch).
 *   rstd[r] = 1 / sqrt(sum(x^2)/n_cols + eps)                  (fp32)
 *   y = w * round_{x_dtype}(x * rstd)   (rounding only when x is 16-bit), stored as y_dtype.
 * Strides are row strides; the last dimension must be unit-stride.
 */
int qlora_rmsnorm_fwd(const void* x, int x_dtype, int64_t x_row_stride, const void* w,
                      int w_dtype, void* y, int y_dtype, int64_t y_row_stride, float* rstd,
                      int64_t n_rows, int64_t n_cols, float eps, ql_stream_t stream);

/*
 * RMSNorm backward (no weight gradient: the weight is frozen).
 * Replaces: solution/rmsnorm.py:42-55 (rmsnorm_bwd_kernel) + :81-90 (launch).
 *   g = dy * w;  dx = rstd * (g - x * rstd^2 * mean(g * x)), stored as dx_dtype.
 */
int qlora_rmsnorm_bwd(const void* dy, int dy_dtype, int64_t dy_row_stride, const void* x,
                      int x_dtype, int64_t x_row_stride, const void* w, int w_dtype,
                      const float* rstd, void* dx, int dx_dtype, int64_t dx_row_stride,
                      int64_t n_rows, int64_t n_cols, ql_stream_t stream);

/*
 * RMSNorm of a residual sum: h = x + d rounded to x's dtype (written to h), then the
 * qlora_rmsnorm_fwd of h (y, rstd). x, d and h share x_dtype; y_dtype = promote(x, w).
 * Rows must hold a multiple of 8 elements (at most 8192), start 16-B aligned, w 16-B aligned
 * (QL_ESHAPE / QL_EALIGN otherwise).
 * Replaces: `residual + hidden_states` followed by the post-attention Qwen2RMSNorm in
 * Qwen2DecoderLayer.forward (transformers/models/qwen2/modeling_qwen2.py:280-291), the
 * decoder layer around the reference's RMSNorm patch (solution/rmsnorm.py:99-115).
 */
int qlora_add_rmsnorm_fwd(const void* x, const void* d, int x_dtype, int64_t x_row_stride,
                          int64_t d_row_stride, const void* w, int w_dtype, void* h,
                          int64_t h_row_stride, void* y, int y_dtype, int64_t y_row_stride,
                          float* rstd, int64_t n_rows, int64_t n_cols, float eps,
                          ql_stream_t stream);

/*
 * qlora_rmsnorm_bwd plus the gradient of the normalised row's other use (the residual
 * stream): dx = rmsnorm_bwd(dy) + dres, summed in fp32 and rounded once to x's dtype (dres
 * and dx have x's dtype). Same row requirements as qlora_add_rmsnorm_fwd.
 * Replaces: the RMSNorm backward of solution/rmsnorm.py:42-55 and the gradient add autograd
 * performs where Qwen2DecoderLayer's residual stream forks.
 */
int qlora_rmsnorm_bwd_residual(const void* dy, int dy_dtype, int64_t dy_row_stride,
                               const void* x, int x_dtype, int64_t x_row_stride, const void* w,
                               int w_dtype, const float* rstd, const void* dres,
                               int64_t dres_row_stride, void* dx, int64_t dx_row_stride,
                               int64_t n_rows, int64_t n_cols, ql_stream_t stream);

/*
 * Rotary embedding of q and k in one launch, forward or backward (transpose).
 * Replaces: solution/rope.py:24-62 (rope_qk_kernel) + :65-75 (_launch).
 * q/k/q_out/k_out are (B, H, S, D) tensors given by strides {b, h, s} (last dim unit
 * stride); cos/sin are (B or broadcast, S, D) with strides {cs_b, cs_s} (cs_b may be 0).
 * With halves (x1,x2), (c1,c2), (s1,s2):
 *   forward : o1 = x1*c1 - x2*s1 ;  o2 = x2*c2 + x1*s2
 *   backward: d1 = g1*c1 + g2*s2 ;  d2 = g2*c2 - g1*s1
 * in_dtype is the dtype of q and k; out_dtype of q_out and k_out; cs_dtype of cos/sin.
 * D must be even.
 */
int qlora_rope_qk(const void* q, const void* k, void* q_out, void* k_out, const void* cos,
                  const void* sin, int in_dtype, int cs_dtype, int out_dtype, int64_t B,
                  int64_t S, int64_t HQ, int64_t HK, int64_t D, const int64_t* q_strides,
                  const int64_t* k_strides, const int64_t* qo_strides, const int64_t* ko_strides,
                  int64_t cs_stride_b, int64_t cs_stride_s, int backward, ql_stream_t stream);

/*
 * SwiGLU forward: out = silu(gate) * up, computed in fp32, all tensors contiguous, one dtype.
 * Replaces: solution/swiglu.py:15-22 (example_swiglu_fwd_kernel) + :44-51.
 */
int qlora_swiglu_fwd(const void* gate, const void* up, void* out, int dtype, int64_t n,
                     ql_stream_t stream);

/*
 * SwiGLU backward: dup = g*gate*sig ; dgate = g*up*sig*(1 + gate*(1 - sig)), sig = sigmoid(gate).
 * Replaces: solution/swiglu.py:25-37 (example_swiglu_bwd_kernel) + :54-61.
 */
int qlora_swiglu_bwd(const void* grad, const void* gate, const void* up, void* dgate, void* dup,
                     int dtype, int64_t n, ql_stream_t stream);

/*
 * The same two operations on [rows, cols] operands with their own row strides (element
 * leading dimensions), e.g. gate and up as the two column halves of one fused gate|up
 * projection output and dgate / dup written into the halves of one gradient buffer.
 * cols % 8 == 0; every pointer 16-B aligned and every leading dimension 16-B granular
 * (QL_EALIGN otherwise); the math is exactly that of the contiguous forms.
 * Replaces: solution/swiglu.py:44-61 when gate and up are views of one buffer.
 */
int qlora_swiglu_fwd_rows(const void* gate, int64_t ldg, const void* up, int64_t ldu, void* out,
                          int64_t ldo, int64_t rows, int64_t cols, int dtype, ql_stream_t stream);
int qlora_swiglu_bwd_rows(const void* grad, int64_t ldgr, const void* gate, int64_t ldg,
                          const void* up, int64_t ldu, void* dgate, int64_t lddg, void* dup,
                          int64_t lddu, int64_t rows, int64_t cols, int dtype,
                          ql_stream_t stream);

/*
 * LoRA input dropout + scale + cast, rows of n_cols.
 * Replaces: solution/lora.py:29-46 (lora_dropout_scale_kernel) + :74-81 (_dropout_scale).
 *   p > 0 : keep = U(seed, row*n_cols + col) > p ;  out = keep ? in*scale : 0
 *   p <= 0: out = in * scale
 * U is Philox4x32-10 (counter = {flat index as uint32, 0, 0, 0}, key = {seed lo, seed hi}),
 * word 0 folded to non-negative int32 and multiplied by 4.6566127342e-10f: the uniform
 * that Triton's tl.rand(seed, int32 offset) returns.
 */
int qlora_lora_dropout_scale(const void* in, int in_dtype, int64_t in_row_stride, void* out,
                             int out_dtype, int64_t out_row_stride, int64_t n_rows,
                             int64_t n_cols, uint64_t seed, float p, float scale,
                             ql_stream_t stream);

/*
 * LoRA scaled add: out = base + lo * scaling in fp32, stored as out_dtype.
 * Replaces: solution/lora.py:49-60 (lora_scaled_add_kernel) + :96-106 (ScaledAdd.forward).
 */
int qlora_lora_scaled_add(const void* base, int base_dtype, int64_t base_row_stride,
                          const void* lo, int lo_dtype, int64_t lo_row_stride, void* out,
                          int out_dtype, int64_t out_row_stride, int64_t n_rows, int64_t n_cols,
                          float scaling, ql_stream_t stream);

/*
 * LoRA dropout forward that also keeps the mask: out = in * keep * scale (the bits of
 * qlora_lora_dropout_scale with p > 0, the same Philox uniform), and the keep bits in 8 x 8
 * blocks: rows 8 R .. 8 R + 7 take bits_group_stride bytes from R * bits_group_stride, and in
 * them byte 8 (c / 8) + row % 8 holds keep(row, c .. c + 7), bit j for column c + j
 * (c % 8 == 0). An 8 x 8 block is one 8-byte word; ceil(n_rows / 8) * bits_group_stride bytes
 * in all (the bytes of rows past n_rows in the last group are not written). in and out share
 * dtype QL_BF16 or QL_F16; n_cols % 8 == 0, bits_group_stride >= n_cols and a multiple of 8,
 * 16-B aligned rows (QL_ESHAPE / QL_EALIGN otherwise); 0 < p < 1 (QL_EINVAL otherwise).
 * Replaces: solution/lora.py:29-46 + :84-89 (DropoutCast.forward) for the fused 4-bit LoRA
 * layer, whose backward reads the bits instead of regenerating the mask (:90-93).
 */
int qlora_lora_dropout_scale_bits(const void* in, int64_t in_row_stride, void* out,
                                  int64_t out_row_stride, uint8_t* bits,
                                  int64_t bits_group_stride, int64_t n_rows, int64_t n_cols,
                                  int dtype, uint64_t seed, float p, float scale,
                                  ql_stream_t stream);

/*
 * The integer form of the dropout test, host only (no GPU call): with x the Philox word folded
 * to [0, 2^31) (x < 0 -> -x-1), the uniform (float)x * 4.6566127342e-10f is > p exactly when
 * x >= qlora_dropout_keep_threshold(p) (2^31: nothing is kept; NaN p keeps nothing). The
 * dropout kernels compare against this value instead of forming the uniform.
 * No counterpart in the reference (solution/lora.py:41-44 forms the float uniform); exported so
 * that the equivalence can be checked without a GPU.
 */
uint32_t qlora_dropout_keep_threshold(float p);

/*
 * The adapter's input gradient through the dropout, added to the base layer's:
 *   dx[m][k] += keep(m, k) ? scale * sum_{r<16} du[m][r] * A[r][k] : 0
 * du = s g B [M, >= 16], A [16, K] (rank 16), dx [M, K], all dtype (QL_BF16 / QL_F16); keep from
 * qlora_lora_dropout_scale_bits' bits (its layout, bits_group_stride >= K and a multiple of 8).
 * The rank-16 products run on the matrix cores (16-bit operands, fp32 sums), dx is rounded
 * once. K % 8 == 0 and 16-B aligned rows (QL_ESHAPE / QL_EALIGN otherwise).
 * Replaces: solution/lora.py:90-93 (DropoutCast.backward) applied to lora_A's input gradient
 * (the autograd of :172), and autograd's sum with the base layer's gradient.
 */
int qlora_lora_up_masked_add(void* dx, int64_t dx_row_stride, const void* du,
                             int64_t du_row_stride, const void* A, int64_t a_row_stride,
                             const uint8_t* bits, int64_t bits_group_stride, int64_t M, int64_t K,
                             int dtype, float scale, ql_stream_t stream);

/*
 * The same for the 1 <= slots <= 4 adapters of a group that read one input (q/k/v, gate/up),
 * each with its own mask, in one pass over dx:
 *   dx[m][k] += scale * sum_{g < slots, keep_g(m, k)} sum_{r<16} du[m][16 g + r] * A[16 g + r][k]
 * du [M, >= 16 slots] (adapter g in columns 16 g ..), A [16 slots, K] (adapter g in rows 16 g ..),
 * bits: a host array of `slots` device pointers, adapter g's bits (the layout above) at
 * bits[g], all with bits_group_stride. The kept adapters' sums are added in fp32 in slot order and dx is
 * rounded once (so slots = 1 is qlora_lora_up_masked_add, bit for bit). QL_EINVAL for slots
 * outside 1 .. 4 or a null pointer; shapes and alignment as above.
 * Replaces: solution/lora.py:90-93 (DropoutCast.backward) of each adapter of the group, applied
 * to its lora_A input gradient (the autograd of :172), and autograd's sums of those gradients
 * with each other and the base layers'.
 */
int qlora_lora_up_masked_add_slots(void* dx, int64_t dx_row_stride, const void* du,
                                   int64_t du_row_stride, const void* A, int64_t a_row_stride,
                                   const uint8_t* const* bits, int64_t bits_group_stride, int slots,
                                   int64_t M, int64_t K, int dtype, float scale,
                                   ql_stream_t stream);

/*
 * LoRA dropout fused with the adapters' down-projections, for 1 <= slots <= 4 adapters that
 * read one input x [M, K] (K % 64 == 0), each with its own seed (host array seeds[slots]):
 *   xd[g]   = x * keep_g * scale      in dtype, as qlora_lora_dropout_scale_bits(seeds[g]) writes it
 *   bits[g] = keep_g                  layout of qlora_lora_dropout_scale_bits
 *   u[m][16 g + c] = sum_k xd[g][m][k] * A[16 g + c][k]   fp32 sums, rounded once to dtype
 * with u's columns 16 slots .. u_cols-1 set to zero and, when u_t is not null, u_t [16 slots,
 * >= M] = its transpose. xd (may be null: the dropped inputs are then not stored) and bits are
 * host arrays of `slots` device pointers sharing xd_row_stride / bits_group_stride. dtype
 * QL_BF16 / QL_F16 for x, A, xd, u; 16-B aligned x, A and xd rows (QL_EALIGN); 0 < p < 1 and a
 * null pointer QL_EINVAL; shapes QL_ESHAPE. A
 * workspace of qlora_lora_dropout_down_workspace_size bytes (16-B aligned) lets the K range
 * split over workgroups (fp32 partials summed in split order); without it the call runs
 * unsplit, with the same xd and bits and u summed in another order.
 * Replaces: solution/lora.py:29-46 + :84-89 (DropoutCast.forward) of each adapter of the group
 * and the lora_A nn.Linear applied to its output (:172), in one pass over x.
 */
int64_t qlora_lora_dropout_down_workspace_size(int64_t M, int64_t K, int slots);
int qlora_lora_dropout_down(const void* x, int64_t x_row_stride, const void* A,
                            int64_t a_row_stride, int64_t M, int64_t K, int slots, int dtype,
                            const uint64_t* seeds, float p, float scale, void* const* xd,
                            int64_t xd_row_stride, uint8_t* const* bits, int64_t bits_group_stride,
                            void* u, int64_t u_row_stride, int u_cols, void* u_t,
                            int64_t u_t_row_stride, void* workspace, int64_t workspace_bytes,
                            ql_stream_t stream);

/*
 * Measurement only (no counterpart in the reference; nothing in the step calls it): the
 * matrix-core rate under layers of the NT GEMM's pipeline. One workgroup of 4 waves per CU (one
 * wave per SIMD, as the GEMM runs) issues the GEMM's 4 x 4 grid of v_mfma_f32_32x32x16 on the
 * data of `operands` (16 x 64 uint4, dtype QL_BF16 / QL_F16, 16-B aligned):
 * workgroups * 4 * iters * 32 * 32768 FLOP. mode 0: fragments in registers; mode 1: every
 * fragment read from LDS; mode 2: also the K loop's two 64 KiB stages with one barrier and 16
 * direct-to-LDS loads of 1 KiB per wave per 64-k step, from `source` (2 MiB, 16-B aligned,
 * ignored by modes 0 and 1); mode 3: mode 2 with those loads staged through registers. out (>= 256 * workgroups floats) receives a sum of each lane's
 * accumulators. QL_EINVAL for iters <= 0, workgroups outside 1 .. 65535, another mode or a
 * missing source.
 */
int qlora_mfma_probe(const void* operands, int dtype, int mode, int64_t iters, int workgroups,
                     float* out, const void* source, ql_stream_t stream);

/*
 * Per-row cross-entropy statistics over a chunk of logits, optionally overwriting the
 * logits IN PLACE with the gradient.
 * Replaces: solution/fused_ce.py:42-96 (ce_row_kernel) + :99-109 (ce_rows) and
 *           solution/cross_entropy.py:48-90 (fused_ce_kernel).
 *   lse = log(sum exp z); entropy = lse - sum(softmax*z); argmax = first index of the max.
 *   A row is labelled when target >= 0 (ignore_mode 0, fused_ce.py:50) or
 *   target != -100 (ignore_mode 1, cross_entropy.py:54).
 *   loss = labelled ? lse - z[target] : 0
 *   correct (int32, may be NULL) = labelled && argmax == target
 *   pred (int64, may be NULL) = argmax
 *   write_grad: z <- (softmax - onehot(target)) * (labelled ? grad_scale : 0)
 * logits dtype: QL_F16, QL_BF16 or QL_F32; target is int64[n_rows].
 */
int qlora_ce_rows(void* logits, int logits_dtype, int64_t row_stride, int64_t n_rows,
                  int64_t vocab, const int64_t* target, float* loss, float* entropy,
                  int32_t* correct, int64_t* pred, int ignore_mode, int write_grad,
                  float grad_scale, ql_stream_t stream);

/*
 * qlora_ce_rows with grad_scale read from device memory (one fp32; may be NULL when
 * write_grad is 0). Replaces the same code as qlora_ce_rows: the reference computes
 * GRAD_GAIN / float(denominator) on the host (solution/cross_entropy.py:105-106), which
 * waits for the GPU when the denominator is a count still on the device. With the scale
 * formed on the device the host never waits; the values are the same.
 */
int qlora_ce_rows_scale_ptr(void* logits, int logits_dtype, int64_t row_stride,
                            int64_t n_rows, int64_t vocab, const int64_t* target, float* loss,
                            float* entropy, int32_t* correct, int64_t* pred, int ignore_mode,
                            int write_grad, const float* grad_scale, ql_stream_t stream);

/*
 * Dense GEMM on bf16/fp16 matrix cores (fp32 accumulation):
 *   C[M,N] = alpha * sum_k A[m,k] * B[n,k]  + beta * C[M,N]  + bias[n]
 * a_km = 0: A is [M,K] with row stride lda (k contiguous); a_km = 1: A is stored [K,M].
 * b_kn = 0: B is [N,K] with row stride ldb (k contiguous); b_kn = 1: B is stored [K,N].
 * in_dtype (A, B and bias): QL_BF16 or QL_F16. c_dtype: any. bias may be NULL; beta = 0
 * never reads C. Any M, N, K and leading dimensions are accepted (ld >= row length, else
 * QL_ESHAPE; element-aligned pointers, else QL_EALIGN); the fast path wants 16-B aligned
 * k-contiguous rows (ld % 8 == 0) and 8-B aligned K-outer rows (ld % 4 == 0).
 * Replaces the torch GEMM call sites of the path: F.linear / torch.matmul in
 * solution/nf4.py:102,111; the LoRA A/B nn.Linear of solution/lora.py:172; the chunk GEMMs
 * of solution/cross_entropy.py:117,123 and solution/fused_ce.py:135,143.
 */
int qlora_gemm(int a_km, int b_kn, int64_t M, int64_t N, int64_t K, const void* A, int64_t lda,
               const void* B, int64_t ldb, int in_dtype, void* C, int64_t ldc, int c_dtype,
               const void* bias, float alpha, float beta, ql_stream_t stream);

/*
 * Bytes of workspace qlora_gemm_ws uses for split-K on this problem (0 = it runs unsplit).
 * Split-K is chosen when the output has too few 256 x 256 tiles to fill the GPU and K is
 * long: the dz @ W of a logits chunk (K = vocabulary) and skinny outputs. Only plain
 * k-contiguous operands (a_km = b_kn = 0, K % 64 == 0) are split.
 * Replaces: the cuBLAS split-K heuristics behind torch.mm in solution/cross_entropy.py:123
 * and solution/fused_ce.py:143.
 */
int64_t qlora_gemm_workspace_size(int a_km, int b_kn, int64_t M, int64_t N, int64_t K);

/*
 * qlora_gemm with a caller-owned device workspace (16-B aligned) for split-K. With less
 * workspace than qlora_gemm_workspace_size reports, it runs unsplit. Partials are summed in
 * split order, so results do not depend on scheduling.
 * Replaces: the same torch GEMM call sites as qlora_gemm.
 */
int qlora_gemm_ws(int a_km, int b_kn, int64_t M, int64_t N, int64_t K, const void* A,
                  int64_t lda, const void* B, int64_t ldb, int in_dtype, void* C, int64_t ldc,
                  int c_dtype, const void* bias, float alpha, float beta, void* workspace,
                  int64_t workspace_bytes, ql_stream_t stream);

/*
 * NF4 dequantisation into the TRANSPOSED layout: out_t[k * ld_out + n] = W[n][k] for the
 * weight W [rows, cols] that qlora_nf4_dequant would produce row-major; bit-identical
 * values. The backward of the 4-bit linear (solution/nf4.py:110-111, grad_x = dY @ W) then
 * runs as a k-contiguous GEMM against W^T.
 * Replaces: solution/nf4.py:25-49 + :110 (the re-dequantisation in NF4Linear.backward).
 * Requires cols % 128 == 0, rows % 8 == 0, ld_out % 8 == 0, blocksize a power of two >= 16
 * (blocksize2 a power of two when nested), packed and out_t 16-B aligned (else
 * QL_ESHAPE / QL_EINVAL / QL_EALIGN); out_dtype QL_BF16 or QL_F16.
 */
int qlora_nf4_dequant_t(const uint8_t* packed, int64_t rows, int64_t cols, const void* absmax,
                        int nested, const float* code2, const float* absmax2, float offset,
                        int blocksize, int blocksize2, const float* nf4_table, void* out_t,
                        int64_t ld_out, int out_dtype, ql_stream_t stream);

/*
 * Several NF4 weights dequantised in ONE launch: the projections that read the same input
 * (q/k/v, gate/up). Each entry describes one weight W_i [rows, cols] with the arguments of
 * qlora_nf4_dequant (n_weights = rows * cols; absmax, code2, absmax2, offset, blocksize,
 * blocksize2) and its own output `out`; `nested` and `out_dtype` are shared. Results are
 * bit-identical to one qlora_nf4_dequant call per entry.
 * Replaces: solution/nf4.py:71-92 (dequantize_nf4) called once per projection; the
 * grouping itself has no reference counterpart.
 * 1 <= count <= 4. Every entry needs rows * cols % 8 == 0, blocksize a power of two >= 8
 * (blocksize2 a power of two when nested), packed 4-B and out 16-B aligned (else QL_ESHAPE /
 * QL_EINVAL / QL_EALIGN); weights outside these rules go through qlora_nf4_dequant. The
 * outputs must not overlap one another.
 */
typedef struct ql_nf4_weight {
  const uint8_t* packed;
  int64_t rows;
  int64_t cols;
  const void* absmax;
  const float* code2;
  const float* absmax2;
  float offset;
  int blocksize;
  int blocksize2;
  void* out;
} ql_nf4_weight;
int qlora_nf4_dequant_group(const ql_nf4_weight* weights, int count, int nested,
                            const float* nf4_table, int out_dtype, ql_stream_t stream);

/*
 * The transposed form of qlora_nf4_dequant_group: entry i writes W_i^T with the layout of
 * qlora_nf4_dequant_t, out_i[k * ld_out + n] = W_i[n][k], where out_i is normally the
 * column block of a shared [cols, ld_out] buffer (out_t + first output column of W_i), as
 * the backward of the fused projections wants dY_cat @ W_cat. Bit-identical to one
 * qlora_nf4_dequant_t call per entry. Each entry follows qlora_nf4_dequant_t's rules (cols %
 * 128 == 0, rows % 8 == 0, ld_out >= rows, blocksize a power of two >= 16, 16-B aligned
 * packed and out); ld_out % 8 == 0; out_dtype QL_BF16 or QL_F16; 1 <= count <= 4; the
 * column blocks must not overlap.
 * Replaces: solution/nf4.py:110 (the backward's re-dequantisation) once per projection.
 */
int qlora_nf4_dequant_t_group(const ql_nf4_weight* weights, int count, int nested,
                              const float* nf4_table, int64_t ld_out, int out_dtype,
                              ql_stream_t stream);

/*
 * 16-bit transpose: out[c * ld_out + r] = in[r * ld_in + c] for r < rows, c < cols.
 * Lays out k-contiguous operands: the frozen lm_head weight for dz @ W
 * (solution/cross_entropy.py:123, solution/fused_ce.py:143) and the LoRA factors.
 */
int qlora_transpose16(const void* in, int64_t rows, int64_t cols, int64_t ld_in, void* out,
                      int64_t ld_out, ql_stream_t stream);

/*
 * NT GEMM over two concatenated K segments (bf16/fp16 operands, fp32 accumulation):
 *   C[M,N] = alpha * (A[M,K] B[N,K]^T + A2[M,K2] B2[N,K2]^T) (+ bias[n])
 * K and K2 multiples of 64, one of them at most 128 (QL_ESHAPE otherwise); all four operands
 * k-contiguous, 16-B aligned, leading dimensions multiples of 8. The short segment is summed
 * first. With the rank-16 LoRA factors zero-padded to 64 columns this is the whole
 * 4-bit LoRA linear in one GEMM: y = x W^T + u (s B)^T with u = x A^T (forward) and
 * dx = g (W^T)^T + du A^T-padded (backward).
 * Replaces: solution/nf4.py:102,111 (F.linear / matmul on the dequantised weight) together
 * with solution/lora.py:49-60,172 (the adapter GEMMs and the fp32 scaled add).
 * Workspace (16-B aligned) enables split-K; see qlora_gemm_nt_cat_workspace_size.
 */
int64_t qlora_gemm_nt_cat_workspace_size(int64_t M, int64_t N, int64_t K);
int qlora_gemm_nt_cat(int64_t M, int64_t N, int64_t K, const void* A, int64_t lda, const void* B,
                      int64_t ldb, int64_t K2, const void* A2, int64_t lda2, const void* B2,
                      int64_t ldb2, int in_dtype, void* C, int64_t ldc, int c_dtype,
                      const void* bias, float alpha, void* workspace, int64_t workspace_bytes,
                      ql_stream_t stream);

/*
 * qlora_gemm_nt_cat (no bias, alpha 1) with a residual added to the output in the GEMM's
 * store: C = R + (A B^T + A2 B2^T), the product rounded to c_dtype and the sum rounded again,
 * so C equals qlora_gemm_nt_cat followed by `R + C` bit for bit. R [M, N] in c_dtype (bf16 or
 * fp16; QL_EDTYPE for fp32), 16-B aligned, ld_residual >= N a multiple of 8 (QL_EALIGN
 * otherwise); R must not overlap C (QL_EINVAL).
 * Replaces: the decoder layer's final `residual + mlp(x)` (transformers
 * modeling_qwen2.py:297, the Qwen2 layer the reference's patched modules run in) taken into
 * the down projection's GEMM (solution/nf4.py:102 with solution/lora.py:172).
 */
int qlora_gemm_nt_cat_residual(int64_t M, int64_t N, int64_t K, const void* A, int64_t lda,
                               const void* B, int64_t ldb, int64_t K2, const void* A2,
                               int64_t lda2, const void* B2, int64_t ldb2, int in_dtype, void* C,
                               int64_t ldc, int c_dtype, const void* residual,
                               int64_t ld_residual, void* workspace, int64_t workspace_bytes,
                               ql_stream_t stream);

/*
 * The 4-bit base GEMM with its NF4 weight dequantised inside the GEMM, on the way into LDS:
 *   C[M,N] = alpha * (A[M,K] W[N,K]^T + A2[M,K2] B2[N,K2]^T) (+ bias[n]),  C in in_dtype,
 * where W is the weight qlora_nf4_dequant produces from (packed, absmax, nested, code2,
 * absmax2, offset, blocksize, blocksize2, nf4_table) for n_weights = N * K, rounded to
 * in_dtype: the products see exactly those 16-bit values, so C equals qlora_gemm_nt_cat on
 * the dequantised W bit for bit. W's packed bytes are read once per 256-row tile of A instead
 * of writing and re-reading a dense 16-bit copy.
 * K % 64 == 0; blocksize a power of two >= 64 dividing K (blocksize2 a power of two when
 * nested); K2 % 64 == 0 and K2 <= 128 (the rank-16 LoRA segment, zero-padded to 64 columns,
 * as in qlora_gemm_nt_cat); A, packed 16-B aligned, lda >= K a multiple of 8; A2/B2 as in
 * qlora_gemm_nt_cat; in_dtype QL_BF16 or QL_F16. Workspace (16-B aligned,
 * qlora_gemm_nf4_workspace_size bytes) enables split-K for outputs with few 256 x 256 tiles.
 * Replaces: solution/nf4.py:101-102 (dequantize_nf4 + F.linear in NF4Linear.forward) together
 * with solution/lora.py:49-60,172 (the adapter GEMMs and the scaled add).
 */
int64_t qlora_gemm_nf4_workspace_size(int64_t M, int64_t N, int64_t K);
int qlora_gemm_nf4(int64_t M, int64_t N, int64_t K, const void* A, int64_t lda,
                   const uint8_t* packed, const void* absmax, int nested, const float* code2,
                   const float* absmax2, float offset, int blocksize, int blocksize2,
                   const float* nf4_table, int64_t K2, const void* A2, int64_t lda2,
                   const void* B2, int64_t ldb2, int in_dtype, void* C, int64_t ldc,
                   const void* bias, float alpha, void* workspace, int64_t workspace_bytes,
                   ql_stream_t stream);

/*
 * LoRA down-projection (rank 16) for `slots` = G adapters (1 <= G <= 4) that share X:
 *   out[m, c] = alpha * sum_k X[m,k] Y[c,k]  for c < 16 G   (Y [16 G, K]: adapter g in rows
 *                                                            16 g .. 16 g + 15)
 *   out[m, c] = 0  for 16 G <= c < out_cols   (the zero padding the GEMM segment above reads).
 * u = x A^T in forward (Y = A [16, in], or the A of q/k/v stacked); du = s * g B in backward
 * (Y = B^T [16, out]). When out_t is not NULL the 16 G columns are also written transposed,
 * out_t[c * ldt + m] (ldt >= M, in_dtype): the token-contiguous operand qlora_lora_wgrad
 * takes. K % 32 == 0; X, Y 16-B aligned with ldx, ldy multiples of 8, ldx, ldy >= K,
 * 32 * ldx < 2^31 (128 * ldx < 2^31 when G = 1, K >= 8192 and M >= 1024: those calls stream
 * X in 64-row blocks) and 32 * G * ldy < 2^31, else QL_EINVAL; in_dtype QL_BF16/QL_F16; out_dtype
 * QL_BF16/QL_F16/QL_F32. Streams X from HBM once for all G adapters.
 * Replaces: solution/lora.py:172 (lora_A(x)) and its autograd backward through lora_B.
 */
int64_t qlora_lora_down_workspace_size(int64_t M, int64_t K, int slots);
int qlora_lora_down(const void* X, int64_t ldx, const void* Y, int64_t ldy, int64_t M, int64_t K,
                    int slots, int in_dtype, void* out, int64_t ldo, int out_cols, int out_dtype,
                    float alpha, void* out_t, int64_t ldt, void* workspace,
                    int64_t workspace_bytes, ql_stream_t stream);

/*
 * LoRA weight gradient (rank 16) for `slots` = G adapters that share Q, a reduction over the
 * token rows:
 *   out[n, c] = alpha * sum_m Q[m, n] * PT[c, m]     (fp32 [N, 16 G], c < 16 G; stored
 *                                                     [16 G, N] when out_transposed = 1)
 * dB = s * g^T u (PT = u^T, Q = g); dA^T = x^T du (PT = du^T stacked over the adapters that
 * read x, Q = x); PT is the transposed output of qlora_lora_down. N % 8 == 0; Q 16-B aligned
 * with ldq a multiple of 8, N <= ldq, 64 * ldq < 2^31; PT [16 G, ldpt >= M] 16-B aligned with
 * ldpt a multiple of 8, 32 * G * ldpt < 2^31; out 16-B aligned.
 * Replaces: the autograd weight gradients of solution/lora.py:172 (lora_A / lora_B).
 */
int64_t qlora_lora_wgrad_workspace_size(int64_t M, int64_t N, int slots);
int qlora_lora_wgrad(const void* PT, int64_t ldpt, const void* Q, int64_t ldq, int64_t M, int64_t N,
                     int slots, int in_dtype, float* out, int out_transposed, float alpha,
                     void* workspace, int64_t workspace_bytes, ql_stream_t stream);

/*
 * The lora_A gradients of 1 <= slots <= 4 adapters whose inputs are their own dropout masks of
 * one input Q [M, N] (N % 8 == 0), in one pass over Q:
 *   out[16 g + c][n] = alpha * sum_m PT[16 g + c][m] * xd_g[m][n]     fp32 [16 slots, N]
 *   xd_g[m][n] = keep_g(m, n) ? (Q[m][n] * scale rounded to dtype) : 0
 * i.e. qlora_lora_wgrad (transposed output) over each adapter's dropped input as
 * qlora_lora_dropout_scale_bits / qlora_lora_dropout_down form it, without storing it. bits: a
 * host array of `slots` device pointers to keep bits in the layout of
 * qlora_lora_dropout_scale_bits (8-B aligned; bits_group_stride >= N, a multiple of 8). PT, Q,
 * dtype, alignment and the workspace (qlora_lora_wgrad_workspace_size) as qlora_lora_wgrad;
 * the sums run in the same order, so each adapter's result equals qlora_lora_wgrad over its
 * stored dropped input bit for bit.
 * Replaces: the autograd of solution/lora.py:172 for lora_A (du^T xd) on DropoutCast's output
 * (:84-93), for the adapters of a group at once.
 */
int qlora_lora_wgrad_masked(const void* PT, int64_t ldpt, const void* Q, int64_t ldq, int64_t M,
                            int64_t N, int slots, int dtype, const uint8_t* const* bits,
                            int64_t bits_group_stride, float scale, float* out, float alpha,
                            void* workspace, int64_t workspace_bytes, ql_stream_t stream);

/*
 * The lora_B weight gradients of `slots` = G adapters whose outputs are concatenated (the
 * q/k/v projections), from one multi-slot pass over the concatenated output gradient:
 *   out[n, c] = alphas[q] * sum_m Q[m, n] * PT[16 q + c, m]    for off_q <= n < off_{q+1}
 * (fp32 [N, 16]: adapter q's dB = s_q g_q^T u_q in rows off_q .. off_{q+1} - 1). col_offsets
 * (host, G + 1 values: 0 = off_0 <= .. <= off_G = N) and alphas (host, G) are read at the
 * call. The other slots' products over a column are computed and discarded. Same Q / PT
 * requirements as qlora_lora_wgrad; out and the workspace (qlora_lora_wgrad_diag_workspace_size
 * bytes, required) 16-B aligned. Deterministic: the partial sums are added in a fixed order.
 * Replaces: the autograd lora_B gradients of solution/lora.py:172 for projections fused into
 * one GEMM (no reference counterpart for the fused layout itself).
 */
int64_t qlora_lora_wgrad_diag_workspace_size(int64_t M, int64_t N, int slots);
int qlora_lora_wgrad_diag(const void* PT, int64_t ldpt, const void* Q, int64_t ldq, int64_t M,
                          int64_t N, int slots, int in_dtype, const int64_t* col_offsets,
                          const float* alphas, float* out, void* workspace,
                          int64_t workspace_bytes, ql_stream_t stream);

/*
 * qlora_lora_wgrad without a workspace argument, for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving or training loops, C hosts without an
 * allocator). No counterpart in the reference. Same arguments, results and rules as
 * qlora_lora_wgrad, bit for bit: the split partials go to a 16 MiB array inside the library,
 * one per GPU, held until the process ends. A call whose split partials need more than
 * 16 MiB (qlora_lora_wgrad_workspace_size > 16 MiB: e.g. 4 slots, N > 16384, M >= 4096) returns
 * QL_ESHAPE and launches nothing. All calls on one GPU share its array: calls that overlap on
 * that GPU (different streams or threads) race and must be ordered by the caller. The call
 * allocates nothing (no hipMalloc, no library allocation).
 */
int qlora_lora_wgrad_noalloc(const void* PT, int64_t ldpt, const void* Q, int64_t ldq, int64_t M,
                             int64_t N, int slots, int in_dtype, float* out, int out_transposed,
                             float alpha, ql_stream_t stream);

/*
 * SwiGLU backward fused with the gate and up adapters' down-projections of its gradients
 * (a LoRA MLP whose gate/up outputs are the two halves gate, up [rows, cols]):
 *   dgate, dup = exactly as qlora_swiglu_bwd_rows (stored, row-strided)
 *   du[m, c]      = alpha_gate * sum_k dgate[m, k] * bt_gate[c, k]    c < 16
 *   du[m, 16 + c] = alpha_up   * sum_k dup[m, k]   * bt_up[c, k]
 *   du[m, c] = 0 for 32 <= c < out_cols; du_t (optional, [32, ldt >= rows]) = du[:, :32]^T.
 * bt_gate / bt_up are the adapters' B^T [16, cols] (ld ldbt). The gradients are multiplied
 * from an on-chip copy of each tile, so the two down-projections do not read them back from
 * HBM.
 * cols % 32 == 0; every matrix 16-B aligned with a leading dimension that is a multiple of 8,
 * at least cols, and below 2^24; dtype QL_BF16 or QL_F16 (du and du_t in it too). Not in
 * place: the byte ranges dgate and dup span must not meet those of grad, gate or up
 * (QL_EINVAL otherwise).
 * Replaces: solution/swiglu.py:25-37 (the SwiGLU backward) and the lora_B autograd backward
 * of solution/lora.py:172 for the gate and up projections.
 */
int64_t qlora_swiglu_bwd_lora_down_workspace_size(int64_t rows, int64_t cols);
int qlora_swiglu_bwd_lora_down(const void* grad, int64_t ldgr, const void* gate, int64_t ldg,
                               const void* up, int64_t ldu, void* dgate, int64_t lddg, void* dup,
                               int64_t lddu, int64_t rows, int64_t cols, const void* bt_gate,
                               const void* bt_up, int64_t ldbt, float alpha_gate, float alpha_up,
                               int dtype, void* du, int64_t ldo, int out_cols, void* du_t,
                               int64_t ldt, void* workspace, int64_t workspace_bytes,
                               ql_stream_t stream);

/*
 * qlora_swiglu_bwd_lora_down plus both adapters' lora_B gradients in the same pass:
 *   dgate, dup, du, du_t = as qlora_swiglu_bwd_lora_down (du summed in another order: within
 *                          fp32 rounding of it, not bit for bit)
 *   db_gate[k, c] = beta_gate * sum_m dgate[m, k] * ut_gate[c, m]    fp32 [cols, 16]
 *   db_up[k, c]   = beta_up   * sum_m dup[m, k]   * ut_up[c, m]
 * ut_gate / ut_up [16, rows] (ld ldut >= rows, a multiple of 8) are the adapters'
 * down-projections of the forward input, transposed (u^T of y = base + s B (A x)), so
 * db = s (dY)^T u is the lora_B gradient. With ud_t and da_down (both or neither), also the
 * lora_A gradient of the adapter of the layer that reads h = silu(gate) * up (the down
 * projection of a LoRA MLP), h recomputed on chip with the forward's bits:
 *   da_down[c, k] = beta_down * sum_m ud_t[c, m] * h[m, k]             fp32 [16, cols]
 * where ud_t [16, rows] (ld ldut) is that adapter's du^T (du = s dY B). Each workgroup owns
 * 256 columns and a range of rows, keeps the tile's gradients (and h) on chip for every
 * product and writes fp32 partials: nothing is read back from HBM. The workspace (16-B
 * aligned, at least qlora_swiglu_bwd_lora_workspace_size(rows, cols, with_da) bytes) is
 * required (QL_EINVAL without it); db_gate, db_up and da_down are 16-B aligned. Other rules as
 * qlora_swiglu_bwd_lora_down.
 * Replaces: solution/swiglu.py:25-37 (the SwiGLU backward) and the lora_B autograd backward
 * of solution/lora.py:172 for the gate and up projections (both the down-projection of the
 * output gradient and the weight gradient of B), and the lora_A weight gradient of the down
 * projection's adapter (the same line's autograd, du^T h).
 */
int64_t qlora_swiglu_bwd_lora_workspace_size(int64_t rows, int64_t cols, int with_da);
int qlora_swiglu_bwd_lora(const void* grad, int64_t ldgr, const void* gate, int64_t ldg,
                          const void* up, int64_t ldu, void* dgate, int64_t lddg, void* dup,
                          int64_t lddu, int64_t rows, int64_t cols, const void* bt_gate,
                          const void* bt_up, int64_t ldbt, const void* ut_gate,
                          const void* ut_up, int64_t ldut, float alpha_gate, float alpha_up,
                          float beta_gate, float beta_up, int dtype, void* du, int64_t ldo,
                          int out_cols, void* du_t, int64_t ldt, float* db_gate, float* db_up,
                          const void* ud_t, float beta_down, float* da_down, void* workspace,
                          int64_t workspace_bytes, ql_stream_t stream);

/*
 * qlora_swiglu_bwd_lora with the down projection's adapter under LoRA dropout: ud_t and da_down
 * are required, and h recomputed on chip is that adapter's dropped input, keep(m, k) * (h[m, k]
 * * scale rounded to dtype), keep from the bits qlora_swiglu_fwd_lora_down_dropout stored
 * (0 < p < 1; bits 8-B aligned, bits_group_stride >= cols and a multiple of 8):
 *   da_down[c, k] = beta_down * sum_m ud_t[c, m] * keep(m, k) * (h[m, k] * scale)
 * With du_add (may be NULL), the gradient the SwiGLU backward differentiates is first
 *   grad[m, k] + scale * keep(m, k) * sum_r du_add[m, r] * a_add[r, k]      (r < 16)
 * rounded to dtype: the down adapter's input gradient through its dropout mask, what
 * qlora_lora_up_masked_add adds to grad in place (the same bits), taken on chip instead; grad
 * itself is not written. du_add [rows, >= 16] (8-B aligned, ld_du_add % 4 == 0), a_add
 * [16, cols] (ld_a_add >= cols) in dtype.
 * Replaces: as qlora_swiglu_bwd_lora, with the lora_A gradient of the down projection taken on
 * DropoutCast's output (solution/lora.py:84-93,172) and, with du_add, DropoutCast.backward on
 * that adapter's input gradient summed into grad (solution/lora.py:90-93).
 */
int qlora_swiglu_bwd_lora_dropout(const void* grad, int64_t ldgr, const void* gate, int64_t ldg,
                                  const void* up, int64_t ldu, void* dgate, int64_t lddg,
                                  void* dup, int64_t lddu, int64_t rows, int64_t cols,
                                  const void* bt_gate, const void* bt_up, int64_t ldbt,
                                  const void* ut_gate, const void* ut_up, int64_t ldut,
                                  float alpha_gate, float alpha_up, float beta_gate,
                                  float beta_up, int dtype, void* du, int64_t ldo, int out_cols,
                                  void* du_t, int64_t ldt, float* db_gate, float* db_up,
                                  const void* ud_t, float beta_down, float* da_down,
                                  const uint8_t* bits, int64_t bits_group_stride, float p,
                                  float scale, const void* du_add, int64_t ld_du_add,
                                  const void* a_add, int64_t ld_a_add, void* workspace,
                                  int64_t workspace_bytes, ql_stream_t stream);

/*
 * SwiGLU forward fused with the down-projection of its output by the adapter of the layer
 * that reads it (the down projection of a LoRA MLP):
 *   h = silu(gate) * up                  the bits of qlora_swiglu_fwd_rows (row-strided)
 *   u[m, c] = alpha * sum_k h[m, k] * a[c, k]     c < 16, a = that adapter's A [16, cols]
 *   u[m, c] = 0 for 16 <= c < out_cols;  u_t (optional, [16, ldt >= rows]) = u[:, :16]^T.
 * The products use an on-chip copy of each tile of h, so h is not read back from HBM.
 * Workspace (16-B aligned) enables a split over the columns; see the size query. cols % 32 ==
 * 0; every matrix 16-B aligned with a leading dimension that is a multiple of 8, at least
 * cols, and below 2^24; dtype QL_BF16 or QL_F16 (u and u_t in it too). Not in place: h must
 * not meet gate or up (QL_EINVAL otherwise).
 * Replaces: solution/swiglu.py:15-22 (the SwiGLU forward) together with the first adapter
 * GEMM of solution/lora.py:172 (lora_A(x)) for the down projection.
 */
int64_t qlora_swiglu_fwd_lora_down_workspace_size(int64_t rows, int64_t cols);
int qlora_swiglu_fwd_lora_down(const void* gate, int64_t ldg, const void* up, int64_t ldu,
                               void* h, int64_t ldh, int64_t rows, int64_t cols, const void* a,
                               int64_t lda, float alpha, int dtype, void* u, int64_t ldo,
                               int out_cols, void* u_t, int64_t ldt, void* workspace,
                               int64_t workspace_bytes, ql_stream_t stream);

/*
 * The same with LoRA dropout on h for the down projection's adapter (seed, 0 < p < 1, scale =
 * 1 / (1 - p); the workspace size query above covers this form): h is stored as above, the
 * adapter's keep mask of it (the Philox test of
 * qlora_lora_dropout_scale_bits at flat index m * cols + k) goes to bits in that entry's 8 x 8
 * block layout (8-B aligned, bits_group_stride >= cols and a multiple of 8), and
 *   u[m, c] = alpha * sum_k keep(m, k) * (h[m, k] * scale rounded to dtype) * a[c, k].
 * Replaces: solution/swiglu.py:15-22 together with DropoutCast.forward (solution/lora.py:29-46,
 * 84-89) on its output and lora_A of the down projection (:172).
 */
int qlora_swiglu_fwd_lora_down_dropout(const void* gate, int64_t ldg, const void* up,
                                       int64_t ldu, void* h, int64_t ldh, int64_t rows,
                                       int64_t cols, const void* a, int64_t lda, float alpha,
                                       int dtype, void* u, int64_t ldo, int out_cols, void* u_t,
                                       int64_t ldt, uint64_t seed, float p, float scale,
                                       uint8_t* bits, int64_t bits_group_stride,
                                       void* workspace, int64_t workspace_bytes,
                                       ql_stream_t stream);

/*
 * The compute-dtype operands of one rank-16 adapter, from its fp32 factors A [16, K] and
 * B [N, 16], in one launch (K % 8 == 0, pad >= 16):
 *   a16 [16, K] = A;  at_pad [K, pad] = A^T | 0;  bs_pad [N, pad] = scaling * B | 0;
 *   bt [16, N] = B^T;          out_dtype QL_BF16 or QL_F16, round to nearest even.
 * Replaces: the casts of the adapter weights to the autocast dtype inside the nn.Linear
 * calls of solution/lora.py:172 (and the layouts the fused GEMM segments need).
 */
int qlora_lora_pack(const float* A, const float* B, int64_t K, int64_t N, float scaling,
                    int out_dtype, void* a16, void* at_pad, void* bs_pad, void* bt, int pad,
                    ql_stream_t stream);

/*
 * The operands of up to four rank-16 adapters that read the same input (the q/k/v or gate/up
 * projections of a layer), packed for one GEMM per direction over the concatenated outputs.
 * factors[g] (host array, count <= 4, count * 16 <= pad): A [16, K] and B [n_g, 16] fp32,
 * scaling s_g; N = sum n_g, off_g = n_0 + .. + n_{g-1}:
 *   a16 [16 count, K]: rows 16g .. 16g+15 = A_g;
 *   at_pad [K, pad]:   columns 16g .. 16g+15 = A_g^T, the rest 0;
 *   bs_pad [N, pad]:   row off_g + n: columns 16g .. 16g+15 = s_g B_g[n], the rest 0;
 *   bt [16 count, N]:  block-diagonal: rows 16g .. 16g+15, columns off_g .. off_g + n_g - 1
 *                      = B_g^T, every other entry 0 (so qlora_lora_down with `slots` = count
 *                      over all N columns gives each adapter's du = g_g B_g in slot g).
 * out_dtype QL_BF16 or QL_F16, round to nearest even; K % 8 == 0.
 * Replaces: the per-projection casts of solution/lora.py:172 for projections fused into one
 * GEMM (no reference counterpart for the fused layout itself).
 */
typedef struct ql_lora_factor {
  const float* A;
  const float* B;
  int64_t n;
  float scaling;
} ql_lora_factor;
int qlora_lora_pack_group(const ql_lora_factor* factors, int count, int64_t K, int out_dtype,
                          void* a16, void* at_pad, void* bs_pad, void* bt, int pad,
                          ql_stream_t stream);

/*
 * Many qlora_lora_pack_group calls in one launch: every adapter group of a model packed at
 * once (the 112 per-projection packs of a 28-layer step become one launch).
 * `jobs` is an array of `njobs` descriptors in DEVICE memory (the library reads it on the
 * GPU only, so it cannot check it: the caller guarantees 1 <= count <= 4, pad >= 16 count,
 * K % 8 == 0, A/B pointers as for qlora_lora_pack_group, and outputs 16-B aligned and
 * disjoint). Job j writes its four outputs at out_base + its byte offsets, with the values
 * qlora_lora_pack_group writes. `max_items` is the largest job's work-item count,
 * (K + N) (pad / 8) + N + 2 count K with N = sum n; it sizes the grid.
 * Replaces: the per-projection casts of solution/lora.py:172 (no reference counterpart for
 * packing several layers at once).
 */
typedef struct ql_lora_pack_job {
  const float* A[4];   /* lora_A weights [16, K], fp32 row-major; unused slots ignored */
  const float* B[4];   /* lora_B weights [n_g, 16], fp32 row-major */
  int64_t n[4];        /* output features of each adapter */
  float scaling[4];
  int64_t K;           /* input features, shared by the group */
  int64_t a16;         /* byte offsets from out_base: a16 [16 count, K] */
  int64_t at_pad;      /* [K, pad] */
  int64_t bs_pad;      /* [N, pad] */
  int64_t bt;          /* [16 count, N] */
  int32_t count;       /* adapters in the group, 1..4 */
  int32_t reserved;
} ql_lora_pack_job;
int qlora_lora_pack_jobs(const ql_lora_pack_job* jobs, int njobs, int64_t max_items,
                         void* out_base, int out_dtype, int pad, ql_stream_t stream);

/*
 * Causal flash attention forward with grouped-query heads (HQ % HK == 0), head_dim 128:
 *   o[b, hq, s, :] = sum_t softmax_t(scale * q[b,hq,s,:] . k[b,hk,t,:], t <= s) v[b,hk,t,:]
 *   lse[b, hq, s] = log sum_{t <= s} exp(scale * q . k)    (fp32 [B, HQ, S]; may be NULL)
 * with hk = hq / (HQ / HK). Tensors are (B, H, S, D) described by element strides {b, h, s}
 * (last dim contiguous; every stride a multiple of 8, pointers 16-B aligned); dtype QL_BF16 or
 * QL_F16; fp32 softmax and accumulation.
 * Replaces: torch.nn.functional.scaled_dot_product_attention(..., is_causal=True) as
 * Qwen2Attention calls it through transformers' SDPA integration
 * (transformers/models/qwen2/modeling_qwen2.py:216-229); not patched by the reference.
 */
int qlora_attn_fwd(const void* q, const void* k, const void* v, void* o, float* lse, int dtype,
                   int64_t B, int64_t HQ, int64_t HK, int64_t S, int64_t D,
                   const int64_t* q_strides, const int64_t* k_strides, const int64_t* v_strides,
                   const int64_t* o_strides, float scale, ql_stream_t stream);

/*
 * Causal flash attention backward (same shapes, layouts and dtype as qlora_attn_fwd):
 *   given q, k, v, the forward output o, its gradient d_o and the forward's lse,
 *   dq = scale * dS k,  dk = scale * dS^T q (summed over the query heads of each kv head),
 *   dv = P^T d_o (summed likewise), with P = exp(scale q k^T - lse) causal and
 *   dS = P * (d_o v^T - rowsum(d_o * o)).
 * d_o uses o's strides; dk and dv share dkv_strides. dq, dk and dv are written, not added to.
 * The workspace (qlora_attn_bwd_workspace_size bytes, 16-B aligned) holds rowsum(d_o * o) and,
 * when HQ > HK, the per-query-head fp32 dk and dv that are summed over each kv head's group.
 * Deterministic: every output element is reduced in a fixed order.
 * Replaces: the autograd backward of the SDPA call that qlora_attn_fwd replaces.
 */
int64_t qlora_attn_bwd_workspace_size(int64_t B, int64_t HQ, int64_t HK, int64_t S);
int qlora_attn_bwd(const void* q, const void* k, const void* v, const void* o, const void* d_o,
                   const float* lse, void* dq, void* dk, void* dv, int dtype, int64_t B,
                   int64_t HQ, int64_t HK, int64_t S, int64_t D, const int64_t* q_strides,
                   const int64_t* k_strides, const int64_t* v_strides, const int64_t* o_strides,
                   const int64_t* dq_strides, const int64_t* dkv_strides, float scale,
                   void* workspace, int64_t workspace_bytes, ql_stream_t stream);

/*
 * AdamW (torch.optim.AdamW semantics: decoupled weight decay, bias-corrected moments, no
 * amsgrad) over many fp32 tensors in one launch. `table` is a DEVICE array of n_tensors
 * descriptors; tensor t covers chunks [first_chunk, first_chunk + ceil(numel / C)) of the
 * launch, C = qlora_adamw_chunk_elems(), the tensors in order and without gaps, n_chunks the
 * total. The scalars are the values torch computes in double for this step, rounded to fp32:
 *   decay = 1 - lr * weight_decay, one_minus_beta1 = 1 - beta1, one_minus_beta2 = 1 - beta2,
 *   step_size = lr / (1 - beta1^step), bias_correction2_sqrt = sqrt(1 - beta2^step).
 * Per element: p *= decay; m = lerp(m, g, 1 - beta1); v = v beta2 + (1 - beta2) g g;
 *   p += -step_size * m / (sqrt(v) / bias_correction2_sqrt + eps).
 * Replaces: the optimizer of the reference's training step (the trainer's torch AdamW over the
 * LoRA parameters); the reference has no kernel for it.
 */
typedef struct ql_adamw_tensor {
  float* param;
  const float* grad;
  float* exp_avg;
  float* exp_avg_sq;
  int64_t numel;
  int64_t first_chunk;
} ql_adamw_tensor;
int64_t qlora_adamw_chunk_elems(void);
int qlora_adamw_fp32(const ql_adamw_tensor* table, int n_tensors, int64_t n_chunks, float decay,
                     float beta2, float one_minus_beta1, float one_minus_beta2, float step_size,
                     float bias_correction2_sqrt, float eps, ql_stream_t stream);

#ifdef __cplusplus
} /* extern "C" */
#endif

#endif /* QLORA_GFX950_H */
