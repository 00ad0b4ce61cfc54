/*
 * pom_amd — C ABI of the MI355X (gfx950) Polynomial Mixer kernels.
 *
 * Plain pointers and sizes only; every device pointer refers to memory on the
 * device that is current on the calling thread, and every launch is enqueued on
 * `stream` (a hipStream_t passed as void*; NULL = the null stream).  No entry
 * point synchronises, allocates or frees.  Results are deterministic: all
 * reductions are fixed-order (no floating-point atomics).
 *
 * Return value: POM_OK (0) or an error code; pom_last_error() describes the
 * last failure on the calling thread.  Invalid arguments are rejected before
 * anything is launched.
 *
 * Workspace: entry points that reduce across workgroups take a device
 * workspace of at least the size the matching *_workspace_size() reports,
 * 256-byte aligned.  Its contents need no initialisation and are scratch
 * between calls; calls that may run at the same time (different streams)
 * must not share one.  The size depends only on the shape arguments of the
 * size query, so one buffer sized for the largest shape serves every call.
 *
 * Layouts (element strides; the last axis is always contiguous):
 *   x, grad_x, y_s, sh ...  (B, N, C) views  -> pom_view {data, stride_b, stride_n}
 *   coeff, grad_coeff       (P, K) fp32 row-major
 *   aggregate outputs       (B, G, P) contiguous in the element type, G = N / frame_len
 *   mask, count             (B, N) fp32 weights (1 = keep), (B,) fp32
 */
#ifndef POM_AMD_H
#define POM_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define POM_AMD_ABI_VERSION 10
#define POM_MAX_DEGREE 16

typedef enum { POM_DTYPE_F32 = 0, POM_DTYPE_BF16 = 1, POM_DTYPE_F16 = 2 } pom_dtype;
typedef enum { POM_ROPE_NONE = 0, POM_ROPE_1D = 1, POM_ROPE_2D = 2 } pom_rope_kind;
typedef enum {
  POM_OK = 0,
  POM_ERR_INVALID = 1,      /* bad shape, stride, pointer or argument   */
  POM_ERR_UNSUPPORTED = 2,  /* valid but outside what the kernels cover */
  POM_ERR_WORKSPACE = 3,    /* workspace missing or too small           */
  POM_ERR_DEVICE = 4        /* the HIP runtime reported an error        */
} pom_status;

/* A (B, N, C) view with unit stride on the last axis. Strides in elements. */
typedef struct pom_view {
  void* data;
  int64_t stride_b;
  int64_t stride_n;
} pom_view;

/* Optional channel-major ("transposed") copy of a (B, N, C) output: element
 * (b, n, c) at data[c * stride_c + b * stride_b + n], in elements.  The
 * backward's weight-gradient GEMMs reduce over tokens and take operands that
 * are contiguous along them; the kernels that produce sh and dY write this
 * copy in the same pass.  Built for 16-bit types with 16-byte lanes (every
 * channel count a multiple of 8 and 16-byte-aligned views); other requests
 * return POM_ERR_UNSUPPORTED before anything is launched.  NULL: none. */
typedef struct pom_tview {
  void* data;
  int64_t stride_c;
  int64_t stride_b;
} pom_tview;

/* Rotary tables (fp32) and integer token positions.
 *   1-D: cos0/sin0 (rows0, P/2), pos[n * pos_stride]           (pom/pom_rope.py:93-117, :152-180)
 *   2-D: cos0/sin0 rows (rows0, P/4), cos1/sin1 columns (rows1, P/4),
 *        pos[n * pos_stride + 0] = row, pos[n * pos_stride + 1] = column
 *                                                               (pom/pom_rope.py:120-149, :183-235)
 * A position p in [-rows, 0) selects table row p + rows, as torch's indexing
 * of the tables does; positions outside [-rows, rows) are clamped to the
 * table (the reference raises on them; the Python host rejects them where it
 * can check without a device sync). */
typedef struct pom_rope {
  int kind;                 /* pom_rope_kind */
  const float* cos0;
  const float* sin0;
  const float* cos1;
  const float* sin1;
  int64_t table_stride;
  int64_t rows0;
  int64_t rows1;
  const int64_t* pos;
  int64_t pos_stride;
} pom_rope;

int pom_abi_version(void);
const char* pom_last_error(void);

/* ------------------------------------------------------------------------
 * Aggregation: h = act(x), p = sum_{j<K} coeff[:, j] h^(j+1), aggregated over
 * tokens.  Modes, selected by the arguments:
 *   mean         mask == NULL, frame_len == N, rope == NULL/NONE
 *                replaces poly_agg_mean_triton            (pom/pom_triton.py:383-403)
 *   masked mean  mask != NULL (frame_len == N): sum m*p / sum m, an all-zero
 *                row gives 0; tokens with m == 0 are never read
 *                replaces poly_agg_masked_triton          (pom/pom_triton_masked.py:402-428)
 *   frame-causal 1 < frame_len < N: output row f = running mean of the
 *                frame means of frames 0..f, evaluated with the element-type
 *                rounding of every step of PoM.state_forward
 *                (pom/pom.py:252-259), so it equals a state_forward loop
 *                over the frames bit for bit, and full_mask_mixer with a
 *                block-causal 3-D mask (pom/pom.py:41-45) up to that rounding
 *   token-causal frame_len == 1 (N > 1): output row n = mean of tokens 0..n
 *                (chunked scan) — replaces poly_agg_causal_triton
 *                (pom/pom_triton_causal.py:400-423) and, with 1-D RoPE,
 *                poly_agg_rope_causal_triton (pom/pom_triton_rope.py:1020-1053);
 *                grad_out must then be contiguous (B, N, P)
 *   state carry  carry != NULL: (B, P) previous 'h' in the element type and
 *                n_past previous calls; frame 0 continues that recurrence
 *   RoPE         rope->kind 1-D / 2-D: each token's p is rotated before it is
 *                aggregated — replaces poly_agg_rope_mean_triton
 *                (pom/pom_triton_rope.py:985-1017) and the 2-D PyTorch route
 *                (pom/pom_rope.py:511-515)
 * ------------------------------------------------------------------------ */
size_t pom_agg_workspace_size(int dtype, int64_t B, int64_t N, int64_t P, int K,
                              int64_t frame_len, int rope_kind, int backward);

/* Forward.  out: (B, N/frame_len, P) contiguous in dtype.  count_out: (B,)
 * fp32 sum of the mask weights (masked mode; required there).
 * coeff: (P, K) contiguous in param_dtype (a pom_dtype; the coefficient
 * parameter's own type, so no conversion is needed around the call). */
int pom_agg_fwd(int dtype, int param_dtype, int64_t B, int64_t N, int64_t P, int K,
                const pom_view* x, const void* coeff,
                const float* mask, int64_t mask_stride_b, int64_t mask_stride_n,
                int64_t frame_len, const void* carry, int64_t n_past,
                const pom_rope* rope,
                void* out, float* count_out,
                void* workspace, size_t workspace_bytes, void* stream);

/* Allocation-free variant of pom_agg_fwd: the same arguments and results,
 * without the workspace.  No counterpart in the reference: it is for callers
 * that cannot allocate (code under HIP graph capture, serving loops,
 * harnesses that forbid hipMalloc).  Its scratch is a static device array of
 * POM_NOALLOC_SCRATCH_BYTES per GPU, held from the first call on that GPU
 * until the process ends; shapes whose pom_agg_workspace_size (forward) is
 * larger are rejected with POM_ERR_WORKSPACE before anything is launched.
 * The call allocates and frees nothing.  Every call on one GPU shares that
 * GPU's scratch, so calls that may overlap on one GPU (different streams)
 * race; serialise them, or use pom_agg_fwd with a workspace each. */
#define POM_NOALLOC_SCRATCH_BYTES ((size_t)16 << 20)
int pom_agg_fwd_noalloc(int dtype, int param_dtype, int64_t B, int64_t N, int64_t P, int K,
                        const pom_view* x, const void* coeff,
                        const float* mask, int64_t mask_stride_b, int64_t mask_stride_n,
                        int64_t frame_len, const void* carry, int64_t n_past,
                        const pom_rope* rope,
                        void* out, float* count_out, void* stream);

/* Backward.  grad_out: (B, N/frame_len, P) fp32.  count: (B,) fp32 from the
 * forward (masked mode).  grad_x: view written for every token (0 where the
 * mask is 0); may alias a slice of a larger buffer (e.g. the h-half of dY).
 * grad_x_t: channel-major copy of grad_x, or NULL (not in token-causal mode).
 * grad_coeff: (P, K) in param_dtype, overwritten.  The gradient of `carry` is
 * n_past * sum_f grad_out[f] / (n_past + f + 1) and is left to the caller. */
int pom_agg_bwd(int dtype, int param_dtype, int64_t B, int64_t N, int64_t P, int K,
                const pom_view* x, const void* coeff,
                const float* mask, int64_t mask_stride_b, int64_t mask_stride_n,
                const float* count,
                int64_t frame_len, int64_t n_past,
                const pom_rope* rope,
                const float* grad_out, const pom_view* grad_x, const pom_tview* grad_x_t,
                void* grad_coeff,
                void* workspace, size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------
 * Gating (pom/pom.py:207, :103-122; query-side RoPE pom/pom_rope.py:522):
 *   sh = R(pos) hardsigmoid(y_s + bias) * hagg[b, n / (N / groups)]
 * hagg: (B, groups, P) contiguous in the element type (the aggregation's
 * output; groups == N gives one row per token).  bias: (P,) in param_dtype
 * (the bias parameter's own type) or NULL.
 * ------------------------------------------------------------------------ */
size_t pom_gate_workspace_size(int dtype, int64_t B, int64_t N, int64_t P, int64_t groups,
                               int rope_kind);

/* sh_t: channel-major copy of sh, or NULL. */
int pom_gate_fwd(int dtype, int param_dtype, int64_t B, int64_t N, int64_t P,
                 const pom_view* ys, const void* bias, const void* hagg, int64_t groups,
                 const pom_rope* rope, const pom_view* sh, const pom_tview* sh_t, void* stream);

/* Backward.  grad_ys: view (e.g. the s-half of dY) receiving dL/dy_s;
 * grad_ys_t: its channel-major copy, or NULL.
 * grad_hagg: (B, groups, P) fp32, 16-byte aligned.  grad_bias: (P,) in
 * param_dtype or NULL. */
int pom_gate_bwd(int dtype, int param_dtype, int64_t B, int64_t N, int64_t P,
                 const pom_view* ys, const void* bias, const void* hagg, int64_t groups,
                 const pom_rope* rope, const pom_view* grad_sh, const pom_view* grad_ys,
                 const pom_tview* grad_ys_t, float* grad_hagg, void* grad_bias,
                 void* workspace, size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------
 * Per-head gating, n_sel_heads = H > 1 (pom/pom.py:118-122 with the gate of
 * pom/pom.py:207 and the query-side RoPE of pom/pom_rope.py:417-437, :522):
 *   sh[b, n, c] = R(pos) hardsigmoid(y_s + bias)[b, n, c / (P / H)]
 *                 * hagg[b, n / (N / groups), c]
 * y_s: (B, N, H) view; bias: (H,) in param_dtype or NULL.  RoPE acts on the
 * H gate channels: tables of width >= H/2 (1-D) or >= H/4 (2-D), i.e. the
 * reference's full-width tables taken every head_dim / 2 (1-D) or head_dim
 * (2-D) columns.  hagg: (B, groups, P) contiguous in the element type.
 * ------------------------------------------------------------------------ */
size_t pom_gate_heads_workspace_size(int dtype, int64_t B, int64_t N, int64_t P, int64_t H,
                                     int64_t groups);

/* sh_t: channel-major copy of sh, or NULL (16-bit types; built for P % 8 == 0
 * and N % 8 == 0 with 16-byte-aligned operands, else POM_ERR_UNSUPPORTED). */
int pom_gate_heads_fwd(int dtype, int param_dtype, int64_t B, int64_t N, int64_t P, int64_t H,
                       const pom_view* ys, const void* bias, const void* hagg, int64_t groups,
                       const pom_rope* rope, const pom_view* sh, const pom_tview* sh_t, void* stream);

/* Backward.  grad_ys: (B, N, H) view receiving dL/dy_s.  grad_hagg:
 * (B, groups, P) fp32.  grad_bias: (H,) in param_dtype or NULL. */
int pom_gate_heads_bwd(int dtype, int param_dtype, int64_t B, int64_t N, int64_t P, int64_t H,
                       const pom_view* ys, const void* bias, const void* hagg, int64_t groups,
                       const pom_rope* rope, const pom_view* grad_sh, const pom_view* grad_ys,
                       float* grad_hagg, void* grad_bias,
                       void* workspace, size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------
 * Per-token polynomial features (pom/pom.py:83-88), the operand of the
 * dense (B, M, N) mask route (full_mask_mixer, pom/pom.py:41-45, whose mixing
 * is a batched GEMM left to the GEMM library):
 *   out[b, n, c] = sum_{j<K} coeff[c, j] act(x[b, n, c])^(j+1)
 * coeff: (P, K) in param_dtype; x, out, grad views (B, N, P).
 * ------------------------------------------------------------------------ */
size_t pom_features_workspace_size(int dtype, int64_t B, int64_t N, int64_t P, int K);

int pom_features_fwd(int dtype, int param_dtype, int64_t B, int64_t N, int64_t P, int K,
                     const pom_view* x, const void* coeff, const pom_view* out, void* stream);

/* Backward: grad_x = grad_out * p'(h) * act'(x); grad_coeff (P, K) in
 * param_dtype = sum over tokens of grad_out * h^(j+1). */
int pom_features_bwd(int dtype, int param_dtype, int64_t B, int64_t N, int64_t P, int K,
                     const pom_view* x, const void* coeff, const pom_view* grad_out,
                     const pom_view* grad_x, void* grad_coeff,
                     void* workspace, size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------
 * Operand layout
 * ------------------------------------------------------------------------ */

/* dst (cols x rows, row stride ld_dst) = src^T (rows x cols, row stride
 * ld_src), in elements of dtype.  Out of place, on `stream`.
 * No counterpart in the reference (which leaves operand layout to its GEMM
 * library): the fused layer uses it to give its projection GEMMs operands
 * that are contiguous along the reduction dimension (token-contiguous x^T,
 * g^T, sh^T, dY^T for the weight gradients; transposed weights for the data
 * gradients).  16-byte-aligned operands with strides a multiple of 16 bytes
 * take the vector path. */
int pom_transpose(int dtype, int64_t rows, int64_t cols, const void* src, int64_t ld_src,
                  void* dst, int64_t ld_dst, void* stream);

/* ------------------------------------------------------------------------
 * Projection GEMM (matrix cores)
 * ------------------------------------------------------------------------ */

/* C (M x N, row stride ldc) = A B with bf16 operands and fp32 accumulation,
 * on `stream`.  Replaces the bf16 nn.Linear products of the projections,
 * pom/pom.py:187-191 (qc_proj, ag_proj), :205-207 (the fused [h | s]
 * projection) and :231 (the output projection), and their autograd
 * backward (data and weight gradients).  Each operand is read in either
 * row-major layout, so no product needs a transposed copy:
 *   a_layout POM_GEMM_K_CONTIG : A(m, k) = A[m * lda + k]
 *            POM_GEMM_MN_CONTIG: A(m, k) = A[k * lda + m]
 *   b_layout POM_GEMM_K_CONTIG : B(k, n) = B[n * ldb + k]   (an nn.Linear weight, y = x W^T)
 *            POM_GEMM_MN_CONTIG: B(k, n) = B[k * ldb + n]
 * out_dtype: POM_DTYPE_BF16 (round to nearest even) or POM_DTYPE_F32.
 * Requirements (else POM_ERR_UNSUPPORTED): M, N multiples of 8 (a tile
 * that does not divide them leaves a partial last tile, whose rows and
 * columns past M / N are not stored), K a multiple of 64, operands and
 * leading dimensions 16-byte aligned.  tile < 0 and splits <= 0 choose both from the shape
 * (pom_gemm_plan).  splits > 1 divides K into that many contiguous parts
 * whose fp32 partials are summed in a fixed order (deterministic), using
 * pom_gemm_workspace_size() bytes of workspace.  splits == POM_GEMM_STREAM_K
 * shares the tiles' 64-steps evenly among 256 workgroups (one per CU), so a
 * workgroup's range may cover parts of two tiles; the fp32 tile partials are
 * summed in a fixed order too (needs tiles x K / 64 >= 256). */
typedef enum { POM_GEMM_K_CONTIG = 0, POM_GEMM_MN_CONTIG = 1 } pom_gemm_layout;
#define POM_GEMM_STREAM_K 256
#define POM_GEMM_TILES 6   /* tile ids: 256x256, 256x192, 192x256, 256x128, 128x256, 128x128 (BM x BN) */

/* The tile and split count pom_gemm uses for this shape and these layouts
 * when asked to choose (a measured table for the baseline configurations'
 * weight gradients, else a cost model); returns POM_ERR_UNSUPPORTED if M or
 * N is not a multiple of 8.  pom_gemm_workspace_size with tile < 0 reports the
 * largest need of the four layouts' plans. */
int pom_gemm_plan(int64_t M, int64_t N, int64_t K, int a_layout, int b_layout, int* tile, int* splits);
size_t pom_gemm_workspace_size(int64_t M, int64_t N, int64_t K, int tile, int splits);
int pom_gemm(int a_layout, int b_layout, int64_t M, int64_t N, int64_t K, const void* A, int64_t lda,
             const void* B, int64_t ldb, int out_dtype, void* C, int64_t ldc, int tile, int splits,
             void* workspace, size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------
 * Library GEMMs of the fused layer (rocBLAS / hipBLASLt, by solution index)
 * ------------------------------------------------------------------------ */

/* C (n x m, row stride ldc) = A B^T for bf16 A (m x k, row stride lda) and
 * B (n x k, row stride ldb), fp32 accumulation -- BLAS's column-major
 * C = A^T B with transa = T, transb = N -- on `stream`, with the library
 * solution registered for exactly this (m, n, k, lda, ldb, ldc).  This is the
 * form of every projection product of the fused layer when its operands are
 * contiguous along the reduction (pom/pom.py:187-191, :205-207, :231 and
 * their backward).  No counterpart in the reference, which calls its GEMMs
 * through torch: these entry points let the layer's launch sequence run in
 * C++ with the kernels torch's offline-tuned selection table names
 * (pom_amd/tuned/gemm_gfx950.csv), registered by the caller.  Unregistered
 * shapes are refused (POM_ERR_UNSUPPORTED); there is no heuristic fallback.
 * hipBLASLt solutions may need workspace (POM_ERR_WORKSPACE when short). */
typedef enum { POM_BLAS_ROCBLAS = 1, POM_BLAS_HIPBLASLT = 2 } pom_blas_lib;

int pom_blas_set_solution(int64_t m, int64_t n, int64_t k, int64_t lda, int64_t ldb, int64_t ldc, int lib,
                          int index);
/* 1 when a solution is registered for the shape, else 0. */
int pom_blas_has_solution(int64_t m, int64_t n, int64_t k, int64_t lda, int64_t ldb, int64_t ldc);
int pom_blas_gemm(int64_t m, int64_t n, int64_t k, const void* A, int64_t lda, const void* B, int64_t ldb, void* C,
                  int64_t ldc, void* workspace, size_t workspace_bytes, void* stream);
/* The file of the loaded rocBLAS (POM_BLAS_ROCBLAS) or hipBLASLt library
 * these calls go to: solution indices are those of that build. */
const char* pom_blas_library(int lib);

/* ------------------------------------------------------------------------
 * The fused layer, one call per direction (pom/pom.py:216-231 with
 * _get_h_s :204-207 and pom() :125-135; RoPE pom/pom_rope.py:476-526):
 *   forward : Y = x Wq^T (T x W) -> hagg = aggregate(Y[:, :P]) ->
 *             sh = gate(Y[:, P:P+S], hagg) -> out = sh Wa^T (+ b_ag)
 *   backward: dsh = g Wa; dW_ag = g^T sh; db_ag = sum_t g; dY[:, P:P+S],
 *             dL/dhagg from the gate; dY[:, :P], dcoeff from the
 *             aggregation; dx = dY Wq; dW_qc = dY^T x
 * for bf16 activations and weights, T = B * N tokens.  No counterpart in
 * the reference (whose layer is a chain of torch calls): it replaces the
 * Python operator's launch sequence so that an eager step spends no host
 * time between launches.  Every projection runs through pom_blas_gemm and
 * each weight gradient on pom_gemm when a tile divides it, else through
 * pom_blas_gemm on the token-contiguous copies xt, sht, gt, dyt (which must
 * then be given); a library product whose shape has no registered solution
 * makes the call return POM_ERR_UNSUPPORTED before anything is launched.  The aggregation (mask, frames,
 * carry, RoPE) and gating (full width or per head) options are those of
 * pom_agg_* and pom_gate[_heads]_*.  All launches go to `stream`; the
 * workspace holds pom_layer_workspace_size() bytes.
 * ------------------------------------------------------------------------ */
typedef struct pom_layer_args {
  int64_t B, N, D, P;
  int64_t S;              /* gate width: P, or heads when heads > 1 */
  int64_t W;              /* row width of Y and dY, >= P + S (padding columns zero in Wq) */
  int64_t heads;          /* > 1: per-head gate */
  int K;                  /* polynomial degree */
  int param_dtype;        /* se_bias, coeff and their gradients */
  int bias_ag_dtype;      /* b_ag */
  int64_t frame_len, n_past;
  const void* wq;         /* (W, D) bf16 */
  const void* wq_t;       /* (D, W) bf16, backward with dx */
  const void* wa;         /* (D, P) bf16 */
  const void* wa_t;       /* (P, D) bf16, backward */
  const void* se_bias;    /* (S,) or NULL */
  const void* coeff;      /* (P, K) */
  const void* b_ag;       /* (D,) or NULL */
  const float* mask;      /* (B, N) fp32 weights or NULL */
  int64_t mask_stride_b, mask_stride_n;
  const void* carry;      /* (B, P) bf16 running mean or NULL */
  const pom_rope* rope_h; /* aggregation side, or NULL */
  const pom_rope* rope_s; /* gate side, or NULL */
  /* activations (forward outputs, backward inputs) */
  const void* x;          /* (T, D) */
  void* xt;               /* (D, T) or NULL */
  void* y;                /* (T, W) */
  void* hagg;             /* (B, N / frame_len, P) */
  float* count;           /* (B,) when masked */
  void* sh;               /* (T, P) */
  void* sht;              /* (P, T) or NULL */
  void* out;              /* (T, D), forward */
  /* backward */
  const void* g;          /* (T, D) upstream gradient */
  void* gt;               /* (D, T) scratch or NULL */
  void* dsh;              /* (T, P) scratch */
  void* dy;               /* (T, W) scratch */
  void* dyt;              /* (W, T) scratch or NULL */
  void* dx;               /* (T, D) or NULL: not wanted */
  void* dwq;              /* (W, D) in dwq_dtype, or NULL */
  int dwq_dtype;
  void* dwa;              /* (D, P) in dwa_dtype, or NULL */
  int dwa_dtype;
  void* dse_bias;         /* (S,) in param_dtype, or NULL */
  void* dcoeff;           /* (P, K) in param_dtype */
  float* db_ag;           /* (D,) fp32, or NULL */
  float* dh;              /* (B, N / frame_len, P) fp32: dL/dhagg */
  const float* grad_hagg; /* (B, N / frame_len, P) fp32 added to dh, or NULL */
  void* workspace;
  size_t workspace_bytes;
} pom_layer_args;

/* sizeof(pom_layer_args), for bindings to check their copy of the layout */
size_t pom_layer_args_size(void);
size_t pom_layer_workspace_size(const pom_layer_args* args, int backward);
int pom_layer_fwd(const pom_layer_args* args, void* stream);
int pom_layer_bwd(const pom_layer_args* args, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* POM_AMD_H */
