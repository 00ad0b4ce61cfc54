// Internal launch descriptors shared by the kernel files and the C-ABI layer.
// Nothing here is part of the public interface (include/pom_amd.h is).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace pom {

enum DType { DT_F32 = 0, DT_BF16 = 1, DT_F16 = 2 };

enum Mode { MODE_PLAIN = 0, MODE_MASKED = 1, MODE_ROPE1D = 2, MODE_ROPE2D = 3 };

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

struct AggParams {
  int dtype = DT_BF16;
  int mode = MODE_PLAIN;
  int cpt = 8;          // channels per lane (vector width)
  int lpr_log2 = 6;     // log2(lanes per token row)
  int K = 2;            // polynomial degree

  int64_t B = 0, N = 0, P = 0;
  const void* x = nullptr;        // (B, N, P) view, unit channel stride
  int64_t sxb = 0, sxn = 0;
  const float* coeff = nullptr;   // (P, K)

  const float* mask = nullptr;    // (B, N) weights (masked mode)
  int64_t msb = 0, msn = 0;

  int64_t L = 0, NF = 1;          // frame length and frame count (N = L * NF)
  int64_t RC = 0, nchunks = 0, cpf = 0;   // rows per chunk, chunks per row, chunks per frame
  int64_t nvec = 0, nslabs = 0;   // lane vector columns, channel slabs

  RopeTables rope;

  const void* carry = nullptr;    // state carry (B, P) in the element type, or null
  int64_t n_past = 0;
  int round_carry = 1;            // round H to the element type after every frame

  // forward outputs
  void* out = nullptr;            // (B, NF, P) element type
  float* count_out = nullptr;     // (B,) masked: sum of weights

  // backward inputs / outputs
  const float* go = nullptr;      // (B, NF, P) fp32 upstream gradient
  const float* count_in = nullptr;
  void* gx = nullptr;             // (B, N, P) view, unit channel stride
  int64_t sgb = 0, sgn = 0;
  float* gc = nullptr;            // (P, K) fp32

  // workspace
  float* partial = nullptr;
  float* fmean = nullptr;
  int* cnt1 = nullptr;
  int* cnt2 = nullptr;
};

hipError_t launch_agg(const AggParams& p, bool bwd, hipStream_t st);

// Gating: sh = rot(hardsigmoid(y_s + bias)) * hagg[group(token)]
struct GateParams {
  int dtype = DT_BF16;
  int mode = MODE_PLAIN;          // PLAIN / ROPE1D / ROPE2D
  int cpt = 8;
  int lpr_log2 = 6;

  int64_t B = 0, N = 0, P = 0;
  const void* ys = nullptr;       // (B, N, P) gate pre-activation view
  int64_t ysb = 0, ysn = 0;
  const float* bias = nullptr;    // (P,) or null
  const float* hagg = nullptr;    // (B, G, P) fp32
  int64_t G = 1, Lg = 0;          // groups and tokens per group (N = G * Lg)
  RopeTables rope;

  int64_t RC = 0, nchunks = 0, cpg = 0;   // rows per chunk, chunks per row, chunks per group
  int64_t nvec = 0, nslabs = 0;

  void* sh = nullptr;             // (B, N, P) output view (forward)
  int64_t shb = 0, shn = 0;

  const void* dsh = nullptr;      // (B, N, P) upstream gradient view (backward)
  int64_t dsb = 0, dsn = 0;
  void* dys = nullptr;            // (B, N, P) gradient of y_s (backward)
  int64_t dyb = 0, dyn = 0;
  float* dhagg = nullptr;         // (B, G, P) fp32
  float* dbias = nullptr;         // (P,) fp32 or null

  float* part_h = nullptr;        // (B * nchunks, P)
  float* part_b = nullptr;        // (B * nchunks, P)
  float* part_bb = nullptr;       // (B, P)
  int* cnt_h = nullptr;           // (B * G * nslabs)
  int* cnt_b1 = nullptr;          // (B * nslabs)
  int* cnt_b2 = nullptr;          // (nslabs)
};

hipError_t launch_gate(const GateParams& p, bool bwd, hipStream_t st);

}  // namespace pom
