/*
 * kat.h -- C ABI of the MI355X (gfx950) rational-attention kernel library
 * (libkat.so).
 *
 * Each entry point replaces one Triton launch of the reference
 * `kernels` package (SkyeGunasekaran/fastAlgebraicTransformer); the file:line
 * of the launch it replaces is given beside it. The reference's Python API
 * (autograd Functions and functional wrappers) sits above this ABI unchanged.
 *
 * Conventions (all entry points):
 *   - Device pointers are raw HIP device addresses; sizes and leading
 *     dimensions ("ld_*") and strides are in ELEMENTS, not bytes.
 *   - `stream` is a hipStream_t passed as void* (NULL = the null stream).
 *     Work is enqueued asynchronously; nothing synchronises the host.
 *   - No entry point allocates device memory. Scratch comes from the caller
 *     through a workspace pointer whose size the matching *_workspace_size()
 *     function returns.
 *   - Return 0 (KAT_OK) on success; otherwise a kat_status code, with a
 *     human-readable message in kat_last_error() (per host thread).
 *   - Every entry point is stateless and reentrant; concurrent calls on
 *     different streams are independent.
 *   - Arithmetic runs in fp32 (fp64 for KAT_F64 tensors) on inputs upcast
 *     from `dtype`; outputs are stored in `dtype`, statistics (L, mu) in fp32.
 */
#ifndef KAT_H_
#define KAT_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum kat_dtype {
  KAT_F32 = 0,
  KAT_BF16 = 1,
  KAT_F16 = 2,
  KAT_F64 = 3
} kat_dtype;

typedef enum kat_status {
  KAT_OK = 0,
  KAT_EINVAL = 1,       /* bad argument (null pointer, negative size, bad stride) */
  KAT_EUNSUPPORTED = 2, /* valid but unsupported combination (dtype, head dim) */
  KAT_EHIP = 3          /* HIP runtime error at launch */
} kat_status;

/* Library version (major*10000 + minor*100 + patch). */
int kat_version(void);

/* Message of the last failed call on this host thread ("" if none). */
const char* kat_last_error(void);

/* ------------------------------------------------------------------------
 * rational softmax over the last dim: p = sigma(x)^4 / (sum sigma(x)^4 + eps)
 * Replaces rational_softmax_fwd_kernel[(n_rows,)](...) at fused_ops.py:450-456
 * (kernel fused_ops.py:52-106). x, p: [n_rows, n_cols] with row strides.
 * ---------------------------------------------------------------------- */
int kat_rsoftmax_fwd(const void* x, void* p, int64_t n_rows, int64_t n_cols,
                     int64_t ld_x, int64_t ld_p, float eps, int dtype, void* stream);

/* dx = p * g * (dy - <dy, p>), g = 2 / ((|x|+1)^2 (sigma(x) + eps)).
 * Replaces rational_softmax_bwd_kernel[(n_rows,)](...) at fused_ops.py:479-485
 * (kernel fused_ops.py:113-189). */
int kat_rsoftmax_bwd(const void* dy, const void* x, const void* p, void* dx,
                     int64_t n_rows, int64_t n_cols, int64_t ld_dy, int64_t ld_x,
                     int64_t ld_p, int64_t ld_dx, float eps, int dtype, void* stream);

/* ------------------------------------------------------------------------
 * rational SwiGLU: out = gate * sigma(gate) * value (elementwise).
 * Replaces swiglu_fwd_kernel[(n_rows,)](...) at fused_ops.py:506-511
 * (kernel fused_ops.py:196-229). Row strides let gate/value be the two halves
 * of one packed [rows, 2F] buffer without copies.
 * ---------------------------------------------------------------------- */
int kat_rswiglu_fwd(const void* gate, const void* value, void* out, int64_t n_rows,
                    int64_t n_cols, int64_t ld_gate, int64_t ld_value, int64_t ld_out,
                    int dtype, void* stream);

/* dgate = dy * value * (sigma + gate * sigma'), dvalue = dy * gate * sigma.
 * Replaces swiglu_bwd_kernel[(n_rows,)](...) at fused_ops.py:532-537
 * (kernel fused_ops.py:236-288). */
int kat_rswiglu_bwd(const void* dy, const void* gate, const void* value, void* dgate,
                    void* dvalue, int64_t n_rows, int64_t n_cols, int64_t ld_dy,
                    int64_t ld_gate, int64_t ld_value, int64_t ld_dgate, int64_t ld_dvalue,
                    int dtype, void* stream);

/* ------------------------------------------------------------------------
 * mean-error norm: mu = mean|x| (stored fp32, without eps),
 * y = x / (mu + eps) * w.  w: [n_cols] of dtype_w (KAT_F32 or == dtype).
 * Replaces mean_error_norm_fwd_kernel[(n_rows,)](...) at fused_ops.py:558-564
 * (kernel fused_ops.py:295-342).
 * ---------------------------------------------------------------------- */
int kat_men_fwd(const void* x, const void* w, void* y, float* mu, int64_t n_rows,
                int64_t n_cols, int64_t ld_x, int64_t ld_y, float eps, int dtype,
                int dtype_w, void* stream);

/* Workspace bytes kat_men_bwd needs for (n_rows, n_cols, dtype). */
size_t kat_men_bwd_workspace_size(int64_t n_rows, int64_t n_cols, int dtype);

/* dx = dy*w/mu' - sign(x) * (sum(dy*y)/n) / mu',  mu' = mu + eps, sign(0) = 0;
 * dw = sum_rows dy * x / mu'  (fp32; fp64 when dtype is KAT_F64), reduced
 * deterministically. Replaces mean_error_norm_bwd_kernel[(n_rows,)](...) at
 * fused_ops.py:585-591 (kernel fused_ops.py:349-423) together with the torch
 * grad_weight reduction at fused_ops.py:593-597. */
int kat_men_bwd(const void* dy, const void* x, const void* w, const float* mu, void* dx,
                void* dw, void* workspace, size_t workspace_bytes, int64_t n_rows,
                int64_t n_cols, int64_t ld_dy, int64_t ld_x, int64_t ld_dx, float eps,
                int dtype, int dtype_w, void* stream);

/* Residual add fused with the norm:
 *   h = x + r   (rounded to `dtype` as torch's promoted add rounds it)
 *   y = h / (mean|h| + eps) * w,  mu = mean|h|
 * x, h have `dtype`; r has `dtype_r` and y `dtype_y`, each `dtype`, or
 * KAT_BF16 / KAT_F16 when dtype is KAT_F32 (an autocast branch added to an
 * fp32 residual stream; a y read by an autocast matmul, rounded once as its
 * cast would). h, y and mu equal the add followed by kat_men_fwd (and the
 * cast) bit for bit. Replaces the pre-norm block's `x = x + branch(...)` and
 * the norm that reads it (algebraic_model.py:150-151 -> fused_ops.py:558-564).
 * h must not overlap x or r. */
int kat_add_men_fwd(const void* x, const void* r, const void* w, void* h, void* y, float* mu,
                    int64_t n_rows, int64_t n_cols, int64_t ld_x, int64_t ld_r, int64_t ld_h,
                    int64_t ld_y, float eps, int dtype, int dtype_r, int dtype_y, int dtype_w,
                    void* stream);

/* Backward of kat_add_men_fwd. dh is the gradient reaching h through the
 * residual stream (dtype), dy the gradient of y (dtype_y):
 *   dx = round(norm_bwd(dy, h)) + dh   (as autograd sums h's two gradients)
 *   dr = dx cast to dtype_r (skipped when dr is NULL)
 *   dw = sum_rows dy * h / (mu + eps)
 * Workspace: kat_men_bwd_workspace_size(n_rows, n_cols, dtype). Replaces the
 * backward launch at fused_ops.py:585-597 together with autograd's sum of
 * h's gradients and the cast of the branch gradient
 * (algebraic_model.py:150-151). */
int kat_add_men_bwd(const void* dy, const void* dh, const void* h, const void* w, const float* mu,
                    void* dx, void* dr, void* dw, void* workspace, size_t workspace_bytes,
                    int64_t n_rows, int64_t n_cols, int64_t ld_dy, int64_t ld_dh, int64_t ld_h,
                    int64_t ld_dx, int64_t ld_dr, float eps, int dtype, int dtype_r, int dtype_y,
                    int dtype_w, void* stream);

/* ------------------------------------------------------------------------
 * rational attention, layout [B, H, T, D] with arbitrary (b, h, t) strides and
 * unit d-stride. Always causal, as the reference (the `causal` flag is
 * accepted and ignored, forward.py:273 / backward.py:282); the _masked entry
 * points further down add a padding mask and a non-causal mode.
 *   s_ij = scale * <q_i, k_j> - slope_h * (i - j)   (j <= i)
 *   f_ij = sigma(s_ij)^4,  L_i = sum_j f_ij  (fp32, stored without eps)
 *   o_i  = sum_j f_ij v_j / (L_i + eps)
 * strides: 12 int64 = (b, h, t) strides of q, k, v, out, in that order.
 * l_strides: 3 int64 = (b, h, t) strides of L. slopes: fp32 [H].
 * Replaces the host wrapper + rational_attention_fwd_kernel[(B,H,T)] launch at
 * forward.py:267-319 (kernel forward.py:49-159). dtype KAT_BF16/KAT_F16 use
 * the MFMA kernels (D a multiple of 8 up to 256, 16-byte aligned rows; a D
 * between the layout widths 32, 64, 128 and 256 runs in the kernels of the
 * next width, the columns past D read as zeros and not stored); KAT_F32 with
 * D a multiple of 4 up to 256 and 16-byte aligned rows uses the fp32 MFMA
 * kernel (v_mfma_f32_16x16x4_f32: fp32 products and sums); KAT_F64 and the
 * other calls (D <= 1024; larger D returns KAT_EUNSUPPORTED) use the tiled
 * kernels, in fp32 arithmetic (fp64 for KAT_F64; the reference computes in
 * fp32 for every dtype, forward.py:103, and stores in the input dtype, :155).
 * L is fp32 for every dtype.
 * ---------------------------------------------------------------------- */
int kat_attn_fwd(const void* q, const void* k, const void* v, void* out, float* L,
                 const float* slopes, int64_t B, int64_t H, int64_t T, int64_t D,
                 const int64_t* strides, const int64_t* l_strides, float scale, float eps,
                 int causal, int dtype, void* stream);

/* Workspace bytes kat_attn_bwd needs (causal, as every kat_attn_bwd call).
 * On the MFMA path it holds, besides per-row and per-tile values and an fp16
 * copy of Q (O(B*H*T*D) bytes), the fp16 dS tiles of the causal half of each
 * head's T x T scores in 64 x 64 tiles, ~T^2 bytes per head: at most a cap of
 * 4 GiB of them (KAT_ATTN_DS_CAP_BYTES in the environment sets another cap)
 * for as many heads as fit. A head whose tiles exceed the cap runs in bands
 * of its keys (multiples of 512 keys, each band's tiles within the cap, dQ
 * summed in fp32 over the bands in a fixed order; results are bit-identical
 * to one band), plus T*D*4 bytes for those sums, so the workspace stays
 * within cap + O(B*H*T*D) bytes at every T up to the T at which one band of
 * 512 keys alone exceeds the cap (T ~ 2^23 at 4 GiB). The tiled path (fp32,
 * fp64, other head dims) needs 2 B*H*T values of the accumulation type. */
size_t kat_attn_bwd_workspace_size(int64_t B, int64_t H, int64_t T, int64_t D, int dtype);

/* Gradients of kat_attn_fwd:
 *   Delta_i = <dO_i, O_i>,  p = f / (L + eps),  g = 2 / ((|s|+1)^2 (sigma + eps))
 *   dS = p g (<dO_i, v_j> - Delta_i),  dq = scale dS K,  dk = scale dS^T Q,
 *   dv = P^T dO.
 * strides: 24 int64 = (b, h, t) strides of q, k, v, out, dout, dq, dk, dv.
 * Replaces the host wrapper + the dq and dkv launches at backward.py:273-341
 * (kernels backward.py:62-158 and 165-266). Deterministic. The MFMA and tiled
 * paths split the calls as kat_attn_fwd's (MFMA: KAT_BF16 / KAT_F16 with D a
 * multiple of 8 up to 256, KAT_F32 with D a multiple of 4 up to 256, 16-byte
 * aligned rows; the fp32 backward recomputes S and dP with fp32 products and
 * the reference's g, and needs only the tiled path's workspace). On the
 * bf16 / fp16 MFMA path
 * dS is computed once (by the dK/dV kernel, which stores it for dQ), and it
 * and the copies of Q and K its products take enter the MFMA in fp16, each
 * with a power-of-two scale chosen from the data (per 64-row tile for Q, per
 * 32 keys for K, per 64-query tile from a bound on |dS| for dS) and undone
 * exactly: the gradients are exactly equivariant under power-of-two scalings
 * of q, k, v and dout, and per-tile maxima of |q| and |k| in [2^-46, 2^55]
 * are covered. The dS bounds assume (out, L) are the forward's outputs for
 * (q, k, v), as the reference's derivation does. */
int kat_attn_bwd(const void* q, const void* k, const void* v, const void* out,
                 const float* L, const void* dout, void* dq, void* dk, void* dv,
                 const float* slopes, void* workspace, size_t workspace_bytes, int64_t B,
                 int64_t H, int64_t T, int64_t D, const int64_t* strides,
                 const int64_t* l_strides, float scale, float eps, int causal, int dtype,
                 void* stream);

/* Attention with a key padding mask and an optional non-causal mode; no
 * counterpart launch in the reference, whose kernels ignore both (forward.py:273,
 * backward.py:282) while its model's CPU path applies the padding mask
 * (algebraic_model.py:112-136, mask == 0 drops a key, :129-131).
 *   key_mask: uint8 [B, T], element (b, j) at key_mask[b * mask_stride_b + j];
 *             key j of batch b is attended iff it is nonzero. NULL: every key.
 *   causal:   nonzero -> keys j <= i (as kat_attn_fwd); 0 -> every key, with
 *             ALiBi -slope * |i - j| (the CPU path's form, :118-121).
 * A dropped key contributes nothing (the CPU path's -1e4 fill leaves
 * sigma(-1e4)^4 ~ 6e-18 per key); a query with no visible key gets L = 0,
 * o = 0, dq = 0, and dropped keys get dk = dv = 0. Other arguments, layouts
 * as kat_attn_fwd / kat_attn_bwd; the backward's workspace size comes from
 * kat_attn_bwd_masked_workspace_size. */
int kat_attn_fwd_masked(const void* q, const void* k, const void* v, void* out, float* L,
                        const float* slopes, const uint8_t* key_mask, int64_t mask_stride_b,
                        int64_t B, int64_t H, int64_t T, int64_t D, const int64_t* strides,
                        const int64_t* l_strides, float scale, float eps, int causal, int dtype,
                        void* stream);
/* Workspace bytes kat_attn_bwd_masked needs for the given mode: as
 * kat_attn_bwd_workspace_size for causal != 0; for causal == 0 the dS tiles
 * cover all of each head's T x T scores (~2 T^2 bytes per head), under the
 * same cap and banding. No counterpart in the reference (its kernels have no
 * non-causal mode). */
size_t kat_attn_bwd_masked_workspace_size(int64_t B, int64_t H, int64_t T, int64_t D, int dtype,
                                          int causal);
int kat_attn_bwd_masked(const void* q, const void* k, const void* v, const void* out,
                        const float* L, const void* dout, void* dq, void* dk, void* dv,
                        const float* slopes, const uint8_t* key_mask, int64_t mask_stride_b,
                        void* workspace, size_t workspace_bytes, int64_t B, int64_t H, int64_t T,
                        int64_t D, const int64_t* strides, const int64_t* l_strides, float scale,
                        float eps, int causal, int dtype, void* stream);

/* ----------------------------------------------------------------------
 * Decode: one query per (batch, head) against a KV cache -- the last row of
 * the causal attention that the reference's generate() recomputes over the
 * whole prefix for every new token (algebraic_model.py:239-265 ->
 * forward.py:267-319). With n = lengths[b] (or T when lengths is NULL; values
 * are clamped to [0, T]) cached keys and the query at position i = n - 1:
 *   s_j = scale <q, k_j> - slope_h (i - j),  f_j = sigma(s_j)^4   (j < n)
 *   L = sum_j f_j (fp32, without eps),  out = sum_j f_j v_j / (L + eps)
 * q, out: [B, H, D] with (b, h) strides; k, v: [B, H, T, D] caches with
 * (b, h, t) strides (any layout, e.g. token-major [B, T, H, D]); unit
 * d-stride and 16-byte aligned rows. strides: 10 int64 = q (b, h), k (b, h, t),
 * v (b, h, t), out (b, h). L: [B*H] fp32 or NULL. dtype KAT_F32 (D a
 * multiple of 4 up to 128), KAT_BF16 / KAT_F16 (D a multiple of 8 up to 256).
 * Keys are split into chunks across work-groups and the partial sums added in
 * a fixed order (deterministic); the workspace holds the partials. */
size_t kat_attn_decode_workspace_size(int64_t B, int64_t H, int64_t T, int64_t D, int dtype);
int kat_attn_decode(const void* q, const void* k, const void* v, void* out, float* L,
                    const float* slopes, const int32_t* lengths, void* workspace,
                    size_t workspace_bytes, int64_t B, int64_t H, int64_t T, int64_t D,
                    const int64_t* strides, float scale, float eps, int dtype, void* stream);

/* Allocation-free variant of kat_attn_decode. No counterpart in the
 * reference; it is for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * Same arguments, semantics and results as kat_attn_decode (bit for bit), but
 * the split-KV partials live in a fixed device array of the library,
 * KAT_DECODE_SCRATCH_BYTES per GPU, held until the process ends, instead of
 * a caller's workspace. Calls whose partials (B*H*splits*(D+1) floats, with
 * splits as kat_attn_decode picks them; kat_attn_decode_workspace_size gives
 * the byte count) exceed the array fail with KAT_EUNSUPPORTED. The call
 * allocates nothing; the first call on a device looks up the array's device
 * address (hipGetSymbolAddress) once and keeps it for the process, so the
 * entry point must not be used on a device after hipDeviceReset (which
 * invalidates that address). Every call on one GPU shares that
 * GPU's array: calls that overlap in time on one GPU (different streams or
 * host threads) race; calls ordered on one stream do not. */
#define KAT_DECODE_SCRATCH_BYTES ((size_t)8 << 20)
int kat_attn_decode_noalloc(const void* q, const void* k, const void* v, void* out, float* L,
                            const float* slopes, const int32_t* lengths, int64_t B, int64_t H,
                            int64_t T, int64_t D, const int64_t* strides, float scale, float eps,
                            int dtype, void* stream);

/* ----------------------------------------------------------------------
 * Measurement helper (no counterpart in the reference; used by bench.py to
 * report a measured MFMA rate beside the spec peak). `blocks` x 256 threads
 * each run `iters` rounds of 16 independent v_mfma_f32_16x16x32_bf16 chains
 * and write one float per thread to `out` (blocks * 256 floats). *flops
 * receives the flops the launch executes.
 * ---------------------------------------------------------------------- */
int kat_probe_mfma_bf16(float* out, int blocks, int iters, double* flops, void* stream);

/* The same loop on random bf16 operands (eight operand pairs per lane, uniform
 * in [-1, 1), taken in turn) with two waves per SIMD: `blocks` x 512 threads,
 * `out` receives blocks * 512 floats. Data that toggles like real operands
 * draws more power than the low-entropy operands above, and the sustained rate
 * is what the chip's power management allows (no counterpart in the
 * reference; bench.py reports it beside the spec peak). */
int kat_probe_mfma_bf16_random(float* out, int blocks, int iters, double* flops, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* KAT_H_ */
