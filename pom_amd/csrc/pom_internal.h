// Internal launch descriptors shared by the kernel files and the C-ABI layer.
// Nothing here is part of the public interface (include/pom_amd.h is).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace pom {

enum DType { DT_F32 = 0, DT_BF16 = 1, DT_F16 = 2 };

enum Mode {
  MODE_PLAIN = 0, MODE_MASKED = 1, MODE_ROPE1D = 2, MODE_ROPE2D = 3,
  MODE_ROPE1D_MASKED = 4, MODE_ROPE2D_MASKED = 5   // RoPE with (B, N) mask weights (aggregation only)
};

// Channel layout of a mode (PLAIN, ROPE1D or ROPE2D) and whether it weights
// tokens by a mask.
__host__ __device__ constexpr int mode_layout(int m) {
  return m == MODE_MASKED ? MODE_PLAIN : m == MODE_ROPE1D_MASKED ? MODE_ROPE1D : m == MODE_ROPE2D_MASKED ? MODE_ROPE2D : m;
}
__host__ __device__ constexpr bool mode_masked(int m) {
  return m == MODE_MASKED || m == MODE_ROPE1D_MASKED || m == MODE_ROPE2D_MASKED;
}

// RoPE cos/sin tables (fp32, row stride `stride`) and integer positions.
// 1-D: table 0 = (S, P/2), pos[n * pos_sn].
// 2-D: table 0 = rows (H, P/4), table 1 = columns (W, P/4),
//      pos[n * pos_sn + 0] = row, pos[n * pos_sn + 1] = column.
struct RopeTables {
  const float* cos0 = nullptr;
  const float* sin0 = nullptr;
  const float* cos1 = nullptr;
  const float* sin1 = nullptr;
  int64_t stride = 0;
  int64_t rows0 = 0, rows1 = 0;
  const int64_t* pos = nullptr;
  int64_t pos_sn = 0;
};

// Streaming geometry shared by every token-parallel kernel.
//
// Channels are cut into "units": a channel (plain modes) or a rotation pair
// (RoPE modes).  A lane owns `cpt` consecutive units (one 16-byte load of
// bf16 per half), 2^lpr_log2 lanes cover one token row of a slab, and a
// 256-thread workgroup streams the rows [rbeg, rend) of one chunk.
// Tokens are grouped in F frames of L tokens; a frame is cut into cpf chunks
// of at most RC rows, so no chunk straddles two frames.
struct Geom {
  int cpt = 8;
  int lpr_log2 = 3;
  int64_t nvec = 0;     // vector columns = units / cpt
  int64_t nslabs = 0;   // ceil(nvec / 2^lpr_log2)
  int64_t L = 0;        // frame length in tokens
  int64_t F = 1;        // frame count (N = F * L)
  int64_t RC = 0;       // rows per chunk
  int64_t cpf = 1;      // chunks per frame = ceil(L / RC)
  int64_t nch = 1;      // chunks per batch row = F * cpf
  int half = 0;         // RoPE: one lane per half of a rotation pair (units = channels)
  int nb = 1;           // batch rows per workgroup (divides B; > 1 only with `half`)
};

// A parameter vector (coefficients, gate bias) or its gradient, in the
// parameter's own dtype: kernels read and write it directly, so a 16-bit
// model needs no conversion launches around the layer.
struct ParamIn {
  const void* ptr = nullptr;
  int dt = DT_F32;
};
struct ParamOut {
  void* ptr = nullptr;
  int dt = DT_F32;
};

// Optional channel-major ("transposed") copy of a (B, N, P) output:
// element (b, n, c) at data[c * ld + b * sb + n].  data == nullptr: none.
struct TrOut {
  void* data = nullptr;
  int64_t ld = 0, sb = 0;
};

struct AggParams {
  int dtype = DT_BF16;
  int mode = MODE_PLAIN;
  int K = 2;                      // polynomial degree
  Geom g;

  int64_t B = 0, N = 0, P = 0;
  const void* x = nullptr;        // (B, N, P) view, unit channel stride
  int64_t sxb = 0, sxn = 0;
  ParamIn coeff;                  // (P, K)

  const float* mask = nullptr;    // (B, N) weights (masked mode)
  int64_t msb = 0, msn = 0;

  RopeTables rope;

  const void* carry = nullptr;    // (B, P) previous running mean, element type, or null
  int64_t n_past = 0;

  // forward
  void* out = nullptr;            // (B, F, P) element type
  float* count_out = nullptr;     // (B,) masked: sum of the mask weights
  int direct = 0;                 // the chunk kernel writes `out` itself (nch == 1, F == 1, no carry)

  // backward
  const float* go = nullptr;      // (B, F, P) fp32 upstream gradient
  const float* count_in = nullptr;
  const float* wf = nullptr;      // (B, F, P) fp32 per-frame token weights (F > 1)
  void* gx = nullptr;             // (B, N, P) view, unit channel stride
  int64_t sgb = 0, sgn = 0;
  TrOut gxt;                      // channel-major copy of gx, or none
  ParamOut gc;                    // (P, K)

  // workspace
  float* part = nullptr;          // forward (B, nch, P) sums | backward (B, nch, K, P)
  float* pcnt = nullptr;          // (B, nch) masked forward: partial counts
};

// Forward: chunk kernel (+ finalize unless direct).  Backward: per-frame
// weights (F > 1), chunk kernel, coefficient-gradient finalize.
// T is float, __hip_bfloat16 or __half; instantiated in kernels_<type>.hip.
template <typename T> hipError_t agg_fwd_t(const AggParams& p, hipStream_t st);
template <typename T> hipError_t agg_bwd_t(const AggParams& p, hipStream_t st);

// Token-causal (prefix mean per token) aggregation as a chunked scan.
struct ScanParams {
  int dtype = DT_BF16;
  int mode = MODE_PLAIN;          // PLAIN / ROPE1D / ROPE2D
  int K = 2;
  int cpt = 8;
  int64_t nvec = 0;               // vector columns
  int64_t B = 0, N = 0, P = 0;
  int64_t RC = 0, nch = 0;        // rows per chunk, chunks per row

  const void* x = nullptr;
  int64_t sxb = 0, sxn = 0;
  ParamIn coeff;
  RopeTables rope;

  void* out = nullptr;            // (B, N, P) element type, contiguous
  const float* go = nullptr;      // (B, N, P) fp32 contiguous upstream gradient
  void* gx = nullptr;
  int64_t sgb = 0, sgn = 0;
  ParamOut gc;

  float* csum = nullptr;          // (B, nch, P) chunk sums
  float* part = nullptr;          // (B, nch, K, P) backward coefficient partials
};

template <typename T> hipError_t scan_fwd_t(const ScanParams& p, hipStream_t st);
template <typename T> hipError_t scan_bwd_t(const ScanParams& p, hipStream_t st);

// Gating: sh = rot(hardsigmoid(y_s + bias)) * hagg[group(token)]
struct GateParams {
  int dtype = DT_BF16;
  int mode = MODE_PLAIN;          // PLAIN / ROPE1D / ROPE2D
  Geom g;                         // frames = hagg groups; F == N means one group per token

  int64_t B = 0, N = 0, P = 0;
  const void* ys = nullptr;       // (B, N, P) gate pre-activation view
  int64_t ysb = 0, ysn = 0;
  ParamIn bias;                   // (P,); ptr null: no bias
  const void* hagg = nullptr;     // (B, G, P) element type
  RopeTables rope;

  void* sh = nullptr;             // (B, N, P) output view (forward)
  int64_t shb = 0, shn = 0;
  TrOut sht;                      // channel-major copy of sh, or none

  const void* dsh = nullptr;      // (B, N, P) upstream gradient view (backward)
  int64_t dsb = 0, dsn = 0;
  void* dys = nullptr;            // (B, N, P) gradient of y_s (backward)
  int64_t dyb = 0, dyn = 0;
  TrOut dyst;                     // channel-major copy of dys, or none
  float* dhagg = nullptr;         // (B, G, P) fp32
  ParamOut dbias;                 // (P,); ptr null: not wanted

  float* part_h = nullptr;        // (B, nch, P)
  float* part_b = nullptr;        // (B, nch, P)
};

// per_token: hagg holds one row per token (token-causal aggregation).
template <typename T> hipError_t gate_fwd_t(const GateParams& p, int per_token, hipStream_t st);
template <typename T> hipError_t gate_bwd_t(const GateParams& p, int per_token, hipStream_t st);

// Per-token polynomial features p = poly(act(x)) and their backward (the
// dense-mask route's operand).  One thread per V-channel chunk and chunk of
// RC token rows.
struct FeatParams {
  int dtype = DT_BF16;
  int K = 2;
  int V = 1;
  int64_t B = 0, N = 0, P = 0;
  int64_t RC = 1, nch = 1;
  const void* x = nullptr;        // (B, N, P) view
  int64_t sxb = 0, sxn = 0;
  ParamIn coeff;                  // (P, K)
  void* out = nullptr;            // (B, N, P) view (forward)
  int64_t sob = 0, son = 0;
  const void* go = nullptr;       // (B, N, P) upstream gradient view (backward)
  int64_t sgob = 0, sgon = 0;
  void* gx = nullptr;             // (B, N, P) view
  int64_t sgxb = 0, sgxn = 0;
  ParamOut gc;                    // (P, K)
  float* part = nullptr;          // (B, nch, K, P)
};

template <typename T> hipError_t features_fwd_t(const FeatParams& p, hipStream_t st);
template <typename T> hipError_t features_bwd_t(const FeatParams& p, hipStream_t st);

// Per-head gating (n_sel_heads = H > 1): sh[b,n,c] = rot(hardsigmoid(y_s + bias))[h] * hagg[b, n / L, c],
// h = c / hd, P = H * hd.
// lanes per token row of the per-head forward row walk (8 channels each)
constexpr int kFwdRowLanes = 32;

struct HeadsParams {
  int dtype = DT_BF16;
  int mode = MODE_PLAIN;          // PLAIN / ROPE1D / ROPE2D over the H gate channels
  int V = 1;                      // elements per thread chunk; divides hd
  int64_t B = 0, N = 0, P = 0, H = 0, hd = 0;
  int64_t L = 0, G = 1;           // tokens per hagg group, groups (N = G * L)

  const void* ys = nullptr;       // (B, N, H) gate pre-activation view
  int64_t ysb = 0, ysn = 0;
  ParamIn bias;                   // (H,); ptr null: no bias
  const void* hagg = nullptr;     // (B, G, P) element type, contiguous
  RopeTables rope;                // tables over the H channels: 1-D (S, H/2), 2-D (rows, H/4)

  void* sh = nullptr;             // (B, N, P) output view (forward)
  int64_t shb = 0, shn = 0;

  const void* dsh = nullptr;      // (B, N, P) upstream gradient view (backward)
  int64_t dsb = 0, dsn = 0;
  void* dys = nullptr;            // (B, N, H) gradient of y_s
  int64_t dyb = 0, dyn = 0;
  float* dhagg = nullptr;         // (B, G, P) fp32
  ParamOut dbias;                 // (H,); ptr null: not wanted

  TrOut sht;                      // channel-major copy of sh (tile path, 16-bit), or none
  int64_t fwd_rows = 0;           // > 0: forward row walk (heads_fwd_rows), token rows per workgroup

  // general path
  int64_t tok_wgs = 1;            // workgroups of the token-row kernel (= bias partial rows)
  int64_t RC = 1, cpf = 1, nch = 1;   // aggregate-gradient chunks: cpf chunks of RC rows per group
  float* sgate = nullptr;         // (B, N, H) fp32 rotated gate values
  float* part_b = nullptr;        // (tok_wgs, H)
  float* part_h = nullptr;        // (B, nch, P) | tile path: (B, ntt, P) per-walk partials

  // tile path (64 tokens x 64 channels per workgroup)
  int tile = 0;
  int tpw = 1;                    // token tiles per backward workgroup (a walk stays inside one group)
  int64_t ntt = 1;                // backward walks per batch row = cdiv(N, 64 * tpw)
  int64_t nhm = 1;                // heads a channel tile can touch (dot-partial stride)
  float* dpart = nullptr;         // (B * N, channel tiles, nhm) per-head dot partials
  float* dzbuf = nullptr;         // (cdiv(B * N, 16), H) fp32 dz sums per 16-token group
                                  // | row path: (B * ntt, H) per walk

  // row path (backward): a workgroup walks wt tokens of one batch row over all
  // P channels; ntt = cdiv(N, wt) walks per row, part_h (B, ntt, P)
  int rows = 0;
  int64_t wt = 0;
};

// LDS of the token-row backward kernel: per wave, cpr chunk dots and two
// H-vectors.
inline size_t heads_token_smem_bytes(int64_t cpr, int64_t H) { return sizeof(float) * 4 * (size_t)(cpr + 2 * H); }

// Row-walk backward of per-head gating: tokens per step, threads per
// workgroup (one per 8-channel chunk and at least one per (step token, head)
// slot, whole 64-lane waves) and LDS bytes (double-buffered dot products).
constexpr int kHeadsRowU = 8;
inline int heads_rows_threads(int64_t P, int64_t H) {
  const int64_t need = P / 8 > kHeadsRowU * H ? P / 8 : kHeadsRowU * H;
  return (int)((need + 63) / 64 * 64);
}
inline size_t heads_rows_smem(int64_t P, int64_t H) {
  const int64_t a = 2 * kHeadsRowU * (P / 8), c = kHeadsRowU * H;
  return sizeof(float) * (size_t)(a > c ? a : c);
}

template <typename T> hipError_t heads_fwd_t(const HeadsParams& p, hipStream_t st);
template <typename T> hipError_t heads_bwd_t(const HeadsParams& p, hipStream_t st);

// dst (C x R, row stride ldd) = src^T (R x C, row stride lds); elements of elem_bytes (2 or 4).
hipError_t transpose_t(int elem_bytes, const void* src, int64_t lds, void* dst, int64_t ldd, int64_t R, int64_t C,
                       hipStream_t st);

// Sets the calling thread's pom_last_error() message and returns `code`.
int set_error(int code, const char* msg);

}  // namespace pom
