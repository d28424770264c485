/*
 * h3k -- MI355X (gfx950) kernels of the W4A8 ConvRot quantised-linear path, behind a plain C ABI.
 *
 * Conventions
 *   - Every pointer argument is a device pointer owned by the caller unless stated otherwise.
 *   - `stream` is a hipStream_t passed as void*; all work is stream-ordered, no entry point synchronises.
 *   - Return 0 on success, a negative H3K_E* code on failure; h3k_last_error() then names the problem
 *     (thread-local, valid until the next failing call on the same thread).
 *   - Strides (ld*) are in ELEMENTS of the pointed-to type (bytes for int8 data).
 *   - Nothing allocates device memory: scratch is a caller workspace sized by the matching *_workspace call.
 *
 * Numerics follow the reference's portable torch backend, quant_mode "ck" (default) or "eager".
 */
#ifndef H3K_H
#define H3K_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* element type codes */
#define H3K_BF16 0
#define H3K_F16 1
#define H3K_F32 2
#define H3K_FP8E4M3 3 /* OCP E4M3FN bytes (scales only) */

/* quant modes */
#define H3K_MODE_CK 0    /* absmax of the unrounded fp32 rotation; epilogue (acc*xs)*s_ch */
#define H3K_MODE_EAGER 1 /* absmax of the dtype-rounded rotation; epilogue acc*(xs*s_ch) */

/* error codes */
#define H3K_OK 0
#define H3K_EINVAL -1   /* bad shape / dtype / alignment / option */
#define H3K_ELAUNCH -2  /* a HIP runtime call or kernel launch failed */
#define H3K_ESPACE -3   /* workspace too small */

/* ABI version (bumped on any signature change or addition). */
int h3k_version(void);

/* Message of the last failure on this thread ("" if none). */
const char* h3k_last_error(void);

/*
 * Block-Hadamard rotation + per-token int8 quantisation.
 * Replaces h3turbo/h3/qlinear.py:295-303 (quantize_activation) and :267-292 (_quantize_rows).
 *   x   [rows, k] of x_dtype (H3K_BF16 | H3K_F16 | H3K_F32), row stride ldx elements
 *   rot rotation block, a power of 4 in [4, 1024] dividing k
 *   q   int8 [rows, k] out, row stride ldq bytes;  xs float32 [rows] out (the per-row scale)
 */
int h3k_rotate_quant(const void* x, int x_dtype, int64_t rows, int64_t k, int64_t ldx, int rot, int mode,
                     int8_t* q, int64_t ldq, float* xs, void* stream);

/*
 * Block-Hadamard rotation only: y = round_to_dtype(fp32(x @ H)) per `rot` block, y has x's dtype.
 * Replaces h3turbo/h3/qlinear.py:118-132 (rotate) for bf16/f16/f32 inputs.
 */
int h3k_rotate(const void* x, int x_dtype, int64_t rows, int64_t k, int64_t ldx, int rot, void* y, int64_t ldy,
               void* stream);

/*
 * int4 codebook indices -> exact int8 grid: clamp(rint(codebook[nib] * s_rel[n, k/group]), -127, 127).
 * Replaces h3turbo/h3/qlinear.py:194-204 (decode_int8_grid) and :157-191 (_pair_lut/_decode_rows).
 *   q      packed [n, k/2] bytes, low nibble = even k, row stride ldq bytes (8-byte aligned)
 *   s_rel  [n, k/group] of s_dtype (H3K_FP8E4M3 | H3K_F16 | H3K_BF16 | H3K_F32), row stride lds elements
 *   codebook float32 [16] (device)
 *   w8     int8 [n, k] out, row stride ldw bytes (16-byte aligned)
 */
int h3k_decode_w4(const void* q, int64_t ldq, const void* s_rel, int s_dtype, int64_t lds, const float* codebook,
                  int64_t n, int64_t k, int group, int8_t* w8, int64_t ldw, void* stream);

/*
 * int8 x int8 -> int32 GEMM (TN: both operands K-contiguous) on int8 MFMA with the fused epilogue
 *   ck   : out = round(f32(f32(acc) * xs[m]) * s_ch[n])
 *   eager: out = round(f32(acc) * f32(xs[m] * s_ch[n]))
 *   bias : out = round(f32(out) + f32(bias[n]))  (bias already in out_dtype; NULL for none)
 * Replaces h3turbo/h3/qlinear.py:236-254 (_int8_mm) and :396-405 (_TorchRunner._a8 epilogue).
 *   a [m, k] int8 (lda bytes), w8 [n, k] int8 (ldw bytes), out [m, n] of out_dtype (ldo elements)
 *   acc_out optional int32 [m, n] (ld n) copy of the exact accumulators (NULL to skip)
 */
int h3k_gemm_a8w8(const int8_t* a, int64_t lda, const float* xs, const int8_t* w8, int64_t ldw, const float* s_ch,
                  const void* bias, int64_t m, int64_t n, int64_t k, int mode, void* out, int out_dtype, int64_t ldo,
                  int32_t* acc_out, void* stream);

/*
 * The packed int8 weight grid of the large-shape GEMM: K-steps t of 64 bytes by blocks b of 32 weight rows (n padded
 * with zero rows to a multiple of 256; NBP = padded n / 32), block (t, b) at byte (t * NBP + b) * 2048 as two 1 KiB
 * MFMA operand fragments in which lane l holds row 32b + (l & 31), bytes 64t + 32(l >> 5) + 16h .. + 16 (h = 0, 1).
 * Same levels as the row-major grid of h3k_decode_w4, another order.  k must be a multiple of 64.
 */
int64_t h3k_w8_packed_bytes(int64_t n, int64_t k); /* size of the packed grid, -1 for a bad shape */

/*
 * int4 codebook indices -> the packed int8 grid (same levels as h3k_decode_w4).
 * Replaces h3turbo/h3/qlinear.py:194-204 (decode_int8_grid) where the grid feeds the large-shape GEMM.
 *   q packed [n, k/2] (ldq bytes, 16-byte aligned, ldq a multiple of 16); s_rel, codebook as for h3k_decode_w4;
 *   w8p h3k_w8_packed_bytes(n, k) bytes, 16-byte aligned
 */
int h3k_decode_w4_packed(const void* q, int64_t ldq, const void* s_rel, int s_dtype, int64_t lds, const float* codebook,
                         int64_t n, int64_t k, int group, int8_t* w8p, void* stream);

/* Row-major int8 grid [n, k] (ldw bytes, 16-byte aligned) -> the packed grid.  A layout change, no reference
 * counterpart: for callers holding a decoded grid. */
int h3k_pack_w8(const int8_t* w8, int64_t ldw, int64_t n, int64_t k, int8_t* w8p, void* stream);

/* 1 when h3k_gemm_a8w8_packed serves an m x n x k GEMM (k a multiple of 256, at least 512; more than 512 rows and
 * enough 256 x 256 output tiles to fill the chip, and by the launch's cost model no slower than the row-major
 * pipeline), else 0: the route the W4A8 linear takes. */
int h3k_gemm_packed_serves(int64_t m, int64_t n, int64_t k);

/*
 * h3k_gemm_a8w8 over the packed weight grid, for the shapes h3k_gemm_packed_serves accepts: the weight fragments
 * go from L2 straight into registers, only the activations are staged through LDS.  Same contract and bit-identical
 * results as h3k_gemm_a8w8.
 * Replaces h3turbo/h3/qlinear.py:236-254 (_int8_mm) and :396-405 (_TorchRunner._a8 epilogue).
 *   a [m, k] int8 (lda bytes, 16-byte aligned, (m-1)*lda + k < 2^32), xs/s_ch/bias 16-byte aligned
 */
int h3k_gemm_a8w8_packed(const int8_t* a, int64_t lda, const float* xs, const int8_t* w8p, const float* s_ch,
                         const void* bias, int64_t m, int64_t n, int64_t k, int mode, void* out, int out_dtype,
                         int64_t ldo, int32_t* acc_out, void* stream);

/*
 * Bytes of the split-tail workspace h3k_gemm_a8w8_packed_ws uses for an m x n x k GEMM, 0 when it runs whole tiles
 * only.  The split: when the last round of 256 x 256 tiles would leave CUs idle and the cost model of the launch says
 * it pays, those tiles are cut along K into pieces (one per idle CU) whose int32 partial sums a fix-up kernel adds
 * (exact) before the epilogue.
 */
int64_t h3k_gemm_packed_split_bytes(int64_t m, int64_t n, int64_t k);

/*
 * h3k_gemm_a8w8_packed without the accumulator dump, for any shape the packed kernel runs (k a multiple of 256, at
 * least 512, m >= 4, n a multiple of 4), taking the split tail for 16-bit outputs when the workspace holds
 * h3k_gemm_packed_split_bytes(m, n, k) bytes (256-byte aligned); with a smaller workspace (or none), whole tiles.
 * Results are bit-identical either way.
 * Replaces h3turbo/h3/qlinear.py:236-254 (_int8_mm) and :396-405 (_TorchRunner._a8 epilogue).
 */
int h3k_gemm_a8w8_packed_ws(const int8_t* a, int64_t lda, const float* xs, const int8_t* w8p, const float* s_ch,
                            const void* bias, int64_t m, int64_t n, int64_t k, int mode, void* out, int out_dtype,
                            int64_t ldo, void* workspace, size_t workspace_bytes, void* stream);

/*
 * W4A8 GEMM for few token rows (m <= 128): the int4 weight is decoded in registers into the int8 MFMA operands,
 * so the int8 grid is never written; exact int32 accumulators and the epilogue of h3k_gemm_a8w8.
 * Replaces, fused, h3turbo/h3/qlinear.py:157-204 (decode_int8_grid), :236-254 (_int8_mm) and :396-405 (_a8
 * epilogue) for the calls with few rows.
 *   a [m, k] int8 (lda bytes, 16-byte aligned), xs [m] float32
 *   q packed [n, k/2] (ldq bytes, 16-byte aligned), s_rel [n, k/group] of s_dtype (lds elements), codebook [16]
 *   group 16, 32 or a multiple of 64; k a multiple of 64
 *   workspace: int32 scratch of h3k_gemm_w4a8_workspace(m, n, k) bytes (16-byte aligned; NULL when that is 0),
 *   used when the call splits K; contents on entry are ignored
 *   acc_out optional int32 [m, n] copy of the exact accumulators (NULL to skip)
 */
int64_t h3k_gemm_w4a8_workspace(int64_t m, int64_t n, int64_t k);
int h3k_gemm_w4a8(const int8_t* a, int64_t lda, const float* xs, const void* q, int64_t ldq, const void* s_rel,
                  int s_dtype, int64_t lds, const float* codebook, int group, const float* s_ch, const void* bias,
                  int64_t m, int64_t n, int64_t k, int mode, void* out, int out_dtype, int64_t ldo, int32_t* workspace,
                  int32_t* acc_out, void* stream);

/*
 * The whole W4A8 ConvRot linear: rotate+quantise x, decode the weight, GEMM + epilogue.  m <= 32 with k a multiple
 * of 64: the fused few-row GEMM, no decode pass; shapes h3k_gemm_packed_serves accepts: the packed grid and its
 * GEMM; otherwise the row-major grid and h3k_gemm_a8w8.
 * Fills the slot of comfy_kitchen's w4a8_int8_linear call, h3turbo/h3/qlinear.py:427-429 (_run_ck).
 * workspace: device scratch of h3k_w4a8_linear_workspace(m, n, k) bytes, 256-byte aligned.  That size includes
 * the packed GEMM's split tail where it is taken; a workspace without it (the activations, their scales and the
 * weight grid only) is accepted and runs whole tiles.
 */
size_t h3k_w4a8_linear_workspace(int64_t m, int64_t n, int64_t k);
int h3k_w4a8_linear(const void* x, int x_dtype, int64_t m, int64_t k, int64_t ldx, const void* q, int64_t ldq,
                    const void* s_rel, int s_dtype, int64_t lds, const float* s_ch, const float* codebook, int64_t n,
                    int group, int rot, const void* bias, int mode, void* out, int out_dtype, int64_t ldo,
                    void* workspace, size_t workspace_bytes, void* stream);

/*
 * h3k_w4a8_linear without a workspace, for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  No counterpart in the reference.  The scratch is a
 * static device array of 128 MiB per GPU, held until the process ends; calls whose h3k_w4a8_linear_workspace(m, n, k)
 * exceeds it fail with H3K_ESPACE (split the rows).  Nothing is allocated or freed.  Every call on a GPU uses that
 * GPU's one array: calls that overlap on one GPU (two streams, two threads) race and must be ordered by the caller.
 */
int h3k_w4a8_linear_noalloc(const void* x, int x_dtype, int64_t m, int64_t k, int64_t ldx, const void* q, int64_t ldq,
                            const void* s_rel, int s_dtype, int64_t lds, const float* s_ch, const float* codebook,
                            int64_t n, int group, int rot, const void* bias, int mode, void* out, int out_dtype,
                            int64_t ldo, void* stream);

/*
 * h3k_rotate_quant of an activation applied as the input is read, in one pass:
 *   act 1 (swiglu): x rows are [gate | up] (2k wide); the quantised input is silu(gate) * up, each op rounded to
 *                   the activation dtype -- replaces qlinear.py:376-379 (_swiglu) + :295-303 (quantize_activation)
 *                   for fc2's input (input_act="swiglu", qlinear.py:494-501)
 *   act 2 (gelu_tanh): the quantised input is gelu(x, tanh approximation) rounded to the activation dtype (the
 *                   config-4 GELU block's fc2 input; no reference counterpart, the reference block is SwiGLU)
 * bf16/f16 x, rotation 256, k a multiple of 256 up to 32768; 16-byte aligned rows.
 * The first bf16 gelu_tanh call on a device fills a 128 KiB table of the GELU of every bf16 value on the given
 * stream and synchronises that stream once; a first call on a stream under graph capture evaluates the formula in
 * the kernel instead (the same values).
 */
int h3k_rotate_quant_act(const void* x, int x_dtype, int64_t rows, int64_t k, int64_t ldx, int act, int rot, int mode,
                         int8_t* q, int64_t ldq, float* xs, void* stream);

/*
 * Per-head RMSNorm + split-half rotary embedding of q and k, in place, bf16.
 * Replaces h3turbo/h3/layout.py:329-355 (norm_rope_, impl "torch": the numerics of comfy_kitchen's fused
 * rms_rope_split_half_ called at :339, which the reference reproduces with rms_norm_fused_order, :309-326).
 *   q, k     bf16 [tokens, heads, head_dim] with heads contiguous; ldq / ldk = elements between tokens
 *   head_dim a multiple of 32 in [32, 256]; half = rotary pairs (2 * half <= head_dim)
 *   wq, wk   fp32 [head_dim] norm weights; cos, sin fp32 [tokens, half], row stride ldcs; eps in fp32
 */
int h3k_qk_norm_rope(void* q, int64_t ldq, void* k, int64_t ldk, int64_t tokens, int heads, int head_dim,
                     const float* wq, const float* wk, const float* cos, const float* sin, int64_t ldcs, int half,
                     float eps, void* stream);

/*
 * The block's attention prologue in one pass: per token and head, read the q, k and v head rows of the qkv
 * projection output, apply h3k_qk_norm_rope's per-head RMSNorm + split-half rotation to q and k (the same
 * arithmetic in the same order: bit-identical results), and write q, k, v head-major for the attention kernel.
 * Replaces h3turbo/h3/model.py:196-214 (_attention: the qkv split, norm_rope_ at layout.py:329-355, and the
 * [S, heads, D] -> [1, heads, S, D] layout the SDPA call at model.py:215-226 consumes).
 *   qkv        bf16 [tokens, 3 * heads * head_dim] = (q | k | v), row stride ldqkv elements
 *   head_dim   32, 64, 128 or 256; half, wq, wk, cos, sin, ldcs, eps as for h3k_qk_norm_rope
 *   q/k/v_out  bf16 [heads, tokens, head_dim]: element (h, t, d) at out[h * head_stride + t * head_dim + d]
 */
int h3k_qkv_split_norm_rope(const void* qkv, int64_t ldqkv, int64_t tokens, int heads, int head_dim, const float* wq,
                            const float* wk, const float* cos, const float* sin, int64_t ldcs, int half, float eps,
                            void* q_out, void* k_out, void* v_out, int64_t head_stride, void* stream);

/*
 * h3k_rotate_quant over head-major rows: row r of the [rows, k] activation is the concatenation over heads h of
 * x[h * head_stride + r * ldx + 0 .. head_dim-1] (the attention output [heads, tokens, head_dim] read as
 * [tokens, heads * head_dim] without a transpose copy).  Same numerics and outputs as h3k_rotate_quant.
 * Replaces the transpose + reshape of the attention output before the out projection
 * (h3turbo/h3/model.py:226-228) together with the out projection's quantize_activation (qlinear.py:295-303).
 *   bf16/f16 activations, rot = 256, head_dim a power of two >= 16 dividing k; x, q 16-byte aligned
 */
int h3k_rotate_quant_heads(const void* x, int x_dtype, int64_t rows, int64_t k, int64_t ldx, int head_dim,
                           int64_t head_stride, int rot, int mode, int8_t* q, int64_t ldq, float* xs, void* stream);

/*
 * RMSNorm + AdaLN modulation of the residual stream in one pass, bf16:
 *   n = bf16(x * rsqrt(mean(x^2) + eps) * w)  (fp32 math)    h = bf16(bf16(n * bf16(1 + scale[m])) + shift[m])
 * with m = row_of_token[t] (NULL: row 0).  Replaces h3turbo/h3/model.py:64-65 (_rms) followed by :106-109
 * (_scale_shift_), as _block applies them before the qkv and fc1 projections (:234-242).
 *   x, h       bf16 [rows, k], row strides ldx / ldh; k a multiple of 8, at most 8192
 *   w          [k] norm weight; shift, scale [R, k] modulation rows, row stride ldm; all three of vec_dtype,
 *              H3K_BF16, or H3K_F32 (rounded to bf16 in the kernel as .to(torch.bfloat16) would, no copy needed)
 *   all pointers 16-byte aligned, strides multiples of 8 elements
 */
int h3k_rms_modulate(const void* x, int64_t ldx, int64_t rows, int64_t k, const void* w, const void* shift,
                     const void* scale, int64_t ldm, const int32_t* row_of_token, float eps, void* h, int64_t ldh,
                     int vec_dtype, void* stream);

/*
 * W4A8 linear with unquantised activations ("a16"): out = round_out(fp32(y * s_ch) + bias), y = xr @ levels^T with
 * fp32 accumulation, xr the rotated activation in bf16 or f16 (a_dtype), levels the decoded int8 grid [n, k]
 * (h3k_decode_w4, row stride ldw).  Replaces _TorchRunner._a16's GEMM, h3turbo/h3/qlinear.py:407-424
 * (torch.mm(xr, levels^T, out_dtype=fp32) on tensor cores, then * s_ch, + bias).  The levels are exact in the
 * 16-bit dtype, so this is the 16-bit MFMA on (xr, levels).  bias is fp32 [n] or NULL.  k a multiple of 16; xr and
 * level rows 16-byte aligned.
 */
int h3k_gemm_a16(const void* a, int a_dtype, int64_t lda, const int8_t* w8, int64_t ldw, const float* s_ch,
                 const float* bias, int64_t m, int64_t n, int64_t k, void* out, int out_dtype, int64_t ldo,
                 void* stream);

/*
 * The DiT block's gated residual add, in place, bf16: x[t] += y[t] * gate[row_of_token[t]] per token row t, as one
 * pass.  Replaces the per-segment x[a:b].addcmul_(y[a:b], gate[row].to(x.dtype)) of _gate_,
 * h3turbo/h3/model.py:112-115.  gate is bf16 or fp32 (gate_dtype H3K_BF16 | H3K_F32; fp32 is rounded to bf16 in
 * the kernel, as .to(x.dtype)), one row of k per modulation row (stride ldg);
 * row_of_token is int32 [rows].  Each element is bf16(fp32(x + y * gate)): the bf16 product is exact in fp32, so
 * this equals torch's addcmul on bf16 tensors.  k a multiple of 8, rows and strides 16-byte aligned.
 */
int h3k_gated_add(void* x, int64_t ldx, const void* y, int64_t ldy, const void* gate, int64_t ldg,
                  const int32_t* row_of_token, int64_t rows, int64_t k, int gate_dtype, void* stream);

/*
 * h3k_gated_add followed by h3k_rms_modulate of the updated rows, in one pass over x: x[t] += y[t] * gate[m], then
 * h[t] = the RMSNorm + modulation of the new x[t] (weights w, shift[m], scale[m]), m = row_of_token[t].  Replaces
 * the attention branch's _gate_ (h3turbo/h3/model.py:112-115) and the _rms + _scale_shift_ before fc1 (:64-65,
 * :106-109) as _block runs them back to back (:234-242); bit-identical to the two entry points in sequence.
 * Arguments and alignment as for those two (gate, w, shift and scale all of vec_dtype); row_of_token must not
 * be NULL; h must not overlap x or y.
 */
int h3k_gated_add_rms_modulate(void* x, int64_t ldx, const void* y, int64_t ldy, const void* gate, int64_t ldg,
                               int64_t rows, int64_t k, const void* w, const void* shift, const void* scale,
                               int64_t ldm, const int32_t* row_of_token, float eps, void* h, int64_t ldh,
                               int vec_dtype, void* stream);

/*
 * Host -> device copy of one weight block on the streaming engine's copy stream (hipMemcpyAsync).
 * Replaces the slot copy of h3turbo/h3/stream.py:346-354 (_issue: slot.buf.copy_(src, non_blocking)).
 * src is host memory (page-locked for an asynchronous copy), dst device memory.
 */
int h3k_copy_h2d_async(void* dst, const void* src, size_t nbytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* H3K_H */
