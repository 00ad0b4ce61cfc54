// C ABI of the PoM kernels: argument validation, launch geometry and
// workspace carving.  See include/pom_amd.h for the contract.
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <string>

#include "../../include/pom_amd.h"
#include "pom_internal.h"

namespace {

thread_local std::string g_err;

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_err = buf;
  return code;
}

int hip_status(hipError_t e, const char* what) {
  if (e == hipSuccess) return POM_OK;
  return fail(POM_ERR_DEVICE, "%s: %s", what, hipGetErrorString(e));
}

int elem_bytes(int dtype) { return dtype == POM_DTYPE_F32 ? 4 : 2; }

bool aligned(const void* p, int64_t bytes) {
  return (reinterpret_cast<uintptr_t>(p) % (uintptr_t)bytes) == 0;
}

int64_t pow2_divisor(int64_t v, int64_t cap) {
  int64_t d = 1;
  while (d < cap && v % (d * 2) == 0) d *= 2;
  return d;
}

int64_t next_pow2(int64_t v) {
  int64_t d = 1;
  while (d < v) d *= 2;
  return d;
}

int ilog2(int64_t v) {
  int l = 0;
  while ((int64_t(1) << l) < v) ++l;
  return l;
}

constexpr int64_t kTargetWorkgroups = 2048;   // 8 per CU on 256 CUs
constexpr int64_t kMinChunkRows = 64;

// Geometry shared by all streaming kernels.
struct Geom {
  int cpt = 1;
  int lpr_log2 = 0;
  int64_t nvec = 0, nslabs = 0;
  int64_t RC = 0;
};

// Lanes per token row: a power of two covering the vector columns without
// idle lanes when possible.
void choose_lanes(Geom& g) {
  int64_t lpr;
  if (g.nvec >= 64) {
    lpr = pow2_divisor(g.nvec, 64);
    if (lpr < 16) lpr = 64;   // ragged width: accept idle lanes in the last slab
  } else {
    lpr = next_pow2(g.nvec);
  }
  g.lpr_log2 = ilog2(lpr);
  g.nslabs = (g.nvec + lpr - 1) / lpr;
}

// Rows per chunk: a power of two dividing `seg` (the frame/group length),
// halved until B * chunks * slabs reaches the target.  It depends only on
// (seg, B, slabs), so a single-frame call (state_forward) and a multi-frame
// call over frames of the same length reduce every frame identically.
int64_t choose_rc(int64_t seg, int64_t B, int64_t nslabs) {
  int64_t rc = seg;
  while (rc % 2 == 0 && rc / 2 >= kMinChunkRows && B * (seg / rc) * nslabs < kTargetWorkgroups) rc /= 2;
  if (rc > 4096 && rc % 2 == 0) {
    // keep chunks short enough that the fixed-order reduction stays balanced
    while (rc > 4096 && rc % 2 == 0) rc /= 2;
  }
  return rc;
}

// Largest vector width (channels per lane) that every pointer, stride and
// channel count admits, capped by a register budget of `reg_cap` values.
int choose_cpt(int dtype, int64_t units, bool rope, int K, int reg_cap,
               std::initializer_list<const void*> ptrs, std::initializer_list<int64_t> strides) {
  const int eb = elem_bytes(dtype);
  int cpt = 16 / eb;
  int km = K <= 2 ? 2 : K <= 4 ? 4 : K <= 8 ? 8 : 16;
  while (cpt > 1) {
    bool ok = units % cpt == 0 && (rope ? 2 : 1) * cpt * km <= reg_cap;
    for (const void* p : ptrs) ok = ok && (p == nullptr || aligned(p, (int64_t)cpt * eb));
    for (int64_t s : strides) ok = ok && (s % cpt == 0);
    if (ok) break;
    cpt /= 2;
  }
  return cpt;
}

struct Carve {
  char* base;
  size_t cap, off;
  template <typename T>
  T* take(int64_t count) {
    off = (off + 255) & ~size_t(255);
    T* p = reinterpret_cast<T*>(base + off);
    off += sizeof(T) * (size_t)count;
    return p;
  }
};

int check_view(const pom_view* v, const char* name) {
  if (!v || !v->data) return fail(POM_ERR_INVALID, "%s: null view", name);
  if (v->stride_b < 0 || v->stride_n < 0) return fail(POM_ERR_INVALID, "%s: negative stride", name);
  return POM_OK;
}

int check_rope(const pom_rope* r, int64_t P, pom::RopeTables& t, int& mode) {
  mode = pom::MODE_PLAIN;
  if (!r || r->kind == POM_ROPE_NONE) return POM_OK;
  if (r->kind != POM_ROPE_1D && r->kind != POM_ROPE_2D) return fail(POM_ERR_INVALID, "rope: bad kind %d", r->kind);
  if (!r->cos0 || !r->sin0 || !r->pos) return fail(POM_ERR_INVALID, "rope: null table or positions");
  if (r->rows0 <= 0) return fail(POM_ERR_INVALID, "rope: empty table");
  if (r->kind == POM_ROPE_1D) {
    if (P % 2) return fail(POM_ERR_INVALID, "rope 1-D: channel count %lld must be even", (long long)P);
    if (r->table_stride < P / 2) return fail(POM_ERR_INVALID, "rope 1-D: table narrower than P/2");
    mode = pom::MODE_ROPE1D;
  } else {
    if (P % 4) return fail(POM_ERR_INVALID, "rope 2-D: channel count %lld must be divisible by 4", (long long)P);
    if (!r->cos1 || !r->sin1 || r->rows1 <= 0) return fail(POM_ERR_INVALID, "rope 2-D: null column table");
    if (r->table_stride < P / 4) return fail(POM_ERR_INVALID, "rope 2-D: table narrower than P/4");
    mode = pom::MODE_ROPE2D;
  }
  t.cos0 = r->cos0; t.sin0 = r->sin0; t.cos1 = r->cos1; t.sin1 = r->sin1;
  t.stride = r->table_stride; t.rows0 = r->rows0; t.rows1 = r->rows1;
  t.pos = r->pos; t.pos_sn = r->pos_stride;
  return POM_OK;
}

// Shared set-up of the aggregation entry points.
int setup_agg(pom::AggParams& p, int dtype, int64_t B, int64_t N, int64_t P, int K, const pom_view* x,
              const float* coeff, const float* mask, int64_t msb, int64_t msn, int64_t frame_len,
              const pom_rope* rope, bool bwd, const pom_view* gx) {
  if (dtype != POM_DTYPE_F32 && dtype != POM_DTYPE_BF16 && dtype != POM_DTYPE_F16)
    return fail(POM_ERR_INVALID, "unknown dtype %d", dtype);
  if (B <= 0 || N <= 0 || P <= 0) return fail(POM_ERR_INVALID, "empty shape B=%lld N=%lld P=%lld",
                                              (long long)B, (long long)N, (long long)P);
  if (K < 1 || K > POM_MAX_DEGREE) return fail(POM_ERR_UNSUPPORTED, "degree %d outside [1, %d]", K, POM_MAX_DEGREE);
  if (int r = check_view(x, "x")) return r;
  if (!coeff) return fail(POM_ERR_INVALID, "coeff is null");
  if (frame_len <= 0 || N % frame_len) return fail(POM_ERR_INVALID, "frame_len %lld must divide N=%lld",
                                                  (long long)frame_len, (long long)N);
  int rmode;
  if (int r = check_rope(rope, P, p.rope, rmode)) return r;
  if (mask) {
    if (rmode != pom::MODE_PLAIN) return fail(POM_ERR_UNSUPPORTED, "masked aggregation with RoPE");
    if (frame_len != N) return fail(POM_ERR_UNSUPPORTED, "masked aggregation with frames");
    p.mode = pom::MODE_MASKED;
  } else {
    p.mode = rmode;
  }
  p.dtype = dtype; p.K = K; p.B = B; p.N = N; p.P = P;
  p.x = x->data; p.sxb = x->stride_b; p.sxn = x->stride_n;
  p.coeff = coeff;
  p.mask = mask; p.msb = msb; p.msn = msn;
  p.L = frame_len; p.NF = N / frame_len;
  p.round_carry = frame_len > 1;

  const bool is_rope = p.mode == pom::MODE_ROPE1D || p.mode == pom::MODE_ROPE2D;
  const int64_t units = p.mode == pom::MODE_ROPE2D ? P / 4 : (p.mode == pom::MODE_ROPE1D ? P / 2 : P);
  Geom g;
  const void* gxp = (bwd && gx) ? gx->data : nullptr;
  const int64_t sgb = (bwd && gx) ? gx->stride_b : 0, sgn = (bwd && gx) ? gx->stride_n : 0;
  g.cpt = choose_cpt(dtype, units, is_rope, K, 32, {x->data, gxp},
                     {x->stride_b, x->stride_n, sgb, sgn});
  if (is_rope) {
    // fp32 tables are read CPT at a time: the table stride and base must admit it
    while (g.cpt > 1 && (p.rope.stride % g.cpt || !aligned(p.rope.cos0, 4 * g.cpt) ||
                         !aligned(p.rope.sin0, 4 * g.cpt) ||
                         (p.rope.cos1 && !aligned(p.rope.cos1, 4 * g.cpt)) ||
                         (p.rope.sin1 && !aligned(p.rope.sin1, 4 * g.cpt))))
      g.cpt /= 2;
  }
  g.nvec = (is_rope ? P / 2 : P) / g.cpt;
  choose_lanes(g);
  g.RC = choose_rc(frame_len, B, g.nslabs);
  p.cpt = g.cpt; p.lpr_log2 = g.lpr_log2; p.nvec = g.nvec; p.nslabs = g.nslabs;
  p.RC = g.RC; p.nchunks = N / g.RC; p.cpf = frame_len / g.RC;
  if (B * p.nchunks * p.nslabs > 0x7fffffffLL) return fail(POM_ERR_UNSUPPORTED, "grid too large");
  return POM_OK;
}

// Upper bound of the chunk count for a segment length: choose_rc never goes
// below min(seg, kMinChunkRows) rows, so the workspace size does not depend on
// the vector width the pointers and strides of a particular call admit.
int64_t max_chunks(int64_t N, int64_t seg) {
  const int64_t rc_min = seg < kMinChunkRows ? seg : kMinChunkRows;
  return (N + rc_min - 1) / rc_min;
}

size_t agg_ws_bytes(const pom::AggParams& p, bool bwd) {
  const int64_t nc = max_chunks(p.N, p.L);
  size_t f = bwd ? (size_t)(p.B * nc * p.K * p.P + p.B * p.K * p.P + 1024)
                 : (size_t)(p.B * nc * p.P + p.B * p.NF * p.P + 1024);
  return POM_COUNTER_BYTES + f * sizeof(float) + 4096;
}

size_t agg_counters(const pom::AggParams& p, bool bwd) {
  return bwd ? (size_t)(p.B * p.nslabs + p.nslabs) : (size_t)(p.B * p.NF * p.nslabs + p.B * p.nslabs);
}

int carve_agg(pom::AggParams& p, bool bwd, void* ws, size_t ws_bytes) {
  const size_t need = agg_ws_bytes(p, bwd);
  if (!ws) return fail(POM_ERR_WORKSPACE, "workspace is null (need %zu bytes)", need);
  if (ws_bytes < need) return fail(POM_ERR_WORKSPACE, "workspace %zu bytes, need %zu", ws_bytes, need);
  if (agg_counters(p, bwd) * sizeof(int) > POM_COUNTER_BYTES)
    return fail(POM_ERR_UNSUPPORTED, "too many frames/slabs for the counter area");
  Carve c{static_cast<char*>(ws), ws_bytes, 0};
  p.cnt1 = c.take<int>(bwd ? p.B * p.nslabs : p.B * p.NF * p.nslabs);
  p.cnt2 = c.take<int>(bwd ? p.nslabs : p.B * p.nslabs);
  c.off = POM_COUNTER_BYTES;
  p.partial = c.take<float>(bwd ? p.B * p.nchunks * p.K * p.P : p.B * p.nchunks * p.P);
  p.fmean = c.take<float>(bwd ? p.B * p.K * p.P : p.B * p.NF * p.P);
  return POM_OK;
}

int setup_gate(pom::GateParams& p, int dtype, int64_t B, int64_t N, int64_t P, const pom_view* ys,
               const float* hagg, int64_t groups, const pom_rope* rope,
               std::initializer_list<const pom_view*> views) {
  if (dtype != POM_DTYPE_F32 && dtype != POM_DTYPE_BF16 && dtype != POM_DTYPE_F16)
    return fail(POM_ERR_INVALID, "unknown dtype %d", dtype);
  if (B <= 0 || N <= 0 || P <= 0) return fail(POM_ERR_INVALID, "empty shape");
  if (int r = check_view(ys, "y_s")) return r;
  for (const pom_view* v : views)
    if (int r = check_view(v, "gate view")) return r;
  if (!hagg) return fail(POM_ERR_INVALID, "hagg is null");
  if (groups <= 0 || N % groups) return fail(POM_ERR_INVALID, "groups %lld must divide N=%lld",
                                            (long long)groups, (long long)N);
  if (int r = check_rope(rope, P, p.rope, p.mode)) return r;
  p.dtype = dtype; p.B = B; p.N = N; p.P = P;
  p.ys = ys->data; p.ysb = ys->stride_b; p.ysn = ys->stride_n;
  p.hagg = hagg; p.G = groups; p.Lg = N / groups;
  const bool is_rope = p.mode != pom::MODE_PLAIN;
  const int64_t units = p.mode == pom::MODE_ROPE2D ? P / 4 : (is_rope ? P / 2 : P);
  Geom g;
  const void* ptrs[4] = {ys->data, nullptr, nullptr, nullptr};
  int64_t strides[8] = {ys->stride_b, ys->stride_n, 0, 0, 0, 0, 0, 0};
  int i = 1, j = 2;
  for (const pom_view* v : views) {
    if (i < 4) ptrs[i++] = v->data;
    if (j < 8) { strides[j++] = v->stride_b; strides[j++] = v->stride_n; }
  }
  g.cpt = choose_cpt(dtype, units, false, 1, 64, {ptrs[0], ptrs[1], ptrs[2], ptrs[3]},
                     {strides[0], strides[1], strides[2], strides[3], strides[4], strides[5], strides[6], strides[7]});
  if (is_rope) {
    while (g.cpt > 1 && (p.rope.stride % g.cpt || !aligned(p.rope.cos0, 4 * g.cpt) ||
                         !aligned(p.rope.sin0, 4 * g.cpt) ||
                         (p.rope.cos1 && !aligned(p.rope.cos1, 4 * g.cpt)) ||
                         (p.rope.sin1 && !aligned(p.rope.sin1, 4 * g.cpt))))
      g.cpt /= 2;
  }
  // hagg / bias are fp32 and read CPT at a time
  while (g.cpt > 1 && (P % g.cpt)) g.cpt /= 2;
  g.nvec = (is_rope ? P / 2 : P) / g.cpt;
  choose_lanes(g);
  // Per-token groups (Lg == 1) take any chunk length; otherwise chunks stay
  // inside one group.
  g.RC = p.Lg == 1 ? choose_rc(N, B, g.nslabs) : choose_rc(p.Lg, B, g.nslabs);
  p.cpt = g.cpt; p.lpr_log2 = g.lpr_log2; p.nvec = g.nvec; p.nslabs = g.nslabs;
  p.RC = g.RC; p.nchunks = N / g.RC; p.cpg = p.Lg >= g.RC ? p.Lg / g.RC : 0;
  if (B * p.nchunks * p.nslabs > 0x7fffffffLL) return fail(POM_ERR_UNSUPPORTED, "grid too large");
  return POM_OK;
}

size_t gate_ws_bytes(const pom::GateParams& p) {
  const int64_t nc = max_chunks(p.N, p.Lg == 1 ? p.N : p.Lg);
  return POM_COUNTER_BYTES + sizeof(float) * (size_t)(2 * p.B * nc * p.P + p.B * p.P + 1024) + 4096;
}

}  // namespace

extern "C" {

int pom_abi_version(void) { return POM_AMD_ABI_VERSION; }

const char* pom_last_error(void) { return g_err.c_str(); }

size_t pom_agg_workspace_size(int dtype, int64_t B, int64_t N, int64_t P, int K, int64_t frame_len,
                              int rope_kind, int backward) {
  pom::AggParams p;
  pom_view x{reinterpret_cast<void*>(256), 0, 0};
  // strides do not change the workspace size; use the contiguous layout
  x.stride_n = P; x.stride_b = N * P;
  float dummy_t[4];
  int64_t dummy_pos[2];
  pom_rope r{rope_kind, dummy_t, dummy_t, dummy_t, dummy_t, P, 1, 1, dummy_pos, 1};
  if (rope_kind == POM_ROPE_1D) r.table_stride = P / 2;
  if (rope_kind == POM_ROPE_2D) r.table_stride = P / 4;
  const float* coeff = dummy_t;
  if (setup_agg(p, dtype, B, N, P, K, &x, coeff, nullptr, 0, 0, frame_len,
                rope_kind == POM_ROPE_NONE ? nullptr : &r, backward != 0, &x) != POM_OK)
    return 0;
  return agg_ws_bytes(p, backward != 0);
}

int pom_agg_fwd(int dtype, int64_t B, int64_t N, int64_t P, int K, const pom_view* x, const float* coeff,
                const float* mask, int64_t mask_stride_b, int64_t mask_stride_n, int64_t frame_len,
                const void* carry, int64_t n_past, const pom_rope* rope, void* out, float* count_out,
                void* workspace, size_t workspace_bytes, void* stream) {
  pom::AggParams p;
  if (int r = setup_agg(p, dtype, B, N, P, K, x, coeff, mask, mask_stride_b, mask_stride_n, frame_len, rope,
                        false, nullptr))
    return r;
  if (!out) return fail(POM_ERR_INVALID, "out is null");
  if (carry && n_past < 1) return fail(POM_ERR_INVALID, "carry given with n_past=%lld", (long long)n_past);
  p.carry = carry; p.n_past = carry ? n_past : 0;
  p.out = out; p.count_out = count_out;
  if (int r = carve_agg(p, false, workspace, workspace_bytes)) return r;
  return hip_status(pom::launch_agg(p, false, static_cast<hipStream_t>(stream)), "pom_agg_fwd launch");
}

int pom_agg_bwd(int dtype, int64_t B, int64_t N, int64_t P, int K, const pom_view* x, const float* coeff,
                const float* mask, int64_t mask_stride_b, int64_t mask_stride_n, const float* count,
                int64_t frame_len, int64_t n_past, const pom_rope* rope, const float* grad_out,
                const pom_view* grad_x, float* grad_coeff, void* workspace, size_t workspace_bytes,
                void* stream) {
  pom::AggParams p;
  if (int r = check_view(grad_x, "grad_x")) return r;
  if (int r = setup_agg(p, dtype, B, N, P, K, x, coeff, mask, mask_stride_b, mask_stride_n, frame_len, rope,
                        true, grad_x))
    return r;
  if (!grad_out || !grad_coeff) return fail(POM_ERR_INVALID, "grad_out / grad_coeff is null");
  if (mask && !count) return fail(POM_ERR_INVALID, "masked backward needs the forward's count");
  if (n_past < 0) return fail(POM_ERR_INVALID, "negative n_past");
  p.n_past = n_past;
  p.go = grad_out; p.count_in = count;
  p.gx = grad_x->data; p.sgb = grad_x->stride_b; p.sgn = grad_x->stride_n;
  p.gc = grad_coeff;
  if (int r = carve_agg(p, true, workspace, workspace_bytes)) return r;
  return hip_status(pom::launch_agg(p, true, static_cast<hipStream_t>(stream)), "pom_agg_bwd launch");
}

size_t pom_gate_workspace_size(int dtype, int64_t B, int64_t N, int64_t P, int64_t groups, int rope_kind) {
  pom::GateParams p;
  pom_view v{reinterpret_cast<void*>(256), N * P, P};
  float dummy_t[4];
  int64_t dummy_pos[2];
  pom_rope r{rope_kind, dummy_t, dummy_t, dummy_t, dummy_t, P, 1, 1, dummy_pos, 1};
  if (rope_kind == POM_ROPE_1D) r.table_stride = P / 2;
  if (rope_kind == POM_ROPE_2D) r.table_stride = P / 4;
  if (setup_gate(p, dtype, B, N, P, &v, dummy_t, groups, rope_kind == POM_ROPE_NONE ? nullptr : &r,
                 {&v, &v}) != POM_OK)
    return 0;
  return gate_ws_bytes(p);
}

int pom_gate_fwd(int dtype, int64_t B, int64_t N, int64_t P, const pom_view* ys, const float* bias,
                 const float* hagg, int64_t groups, const pom_rope* rope, const pom_view* sh, void* stream) {
  pom::GateParams p;
  if (int r = check_view(sh, "sh")) return r;
  if (int r = setup_gate(p, dtype, B, N, P, ys, hagg, groups, rope, {sh})) return r;
  p.bias = bias;
  p.sh = sh->data; p.shb = sh->stride_b; p.shn = sh->stride_n;
  return hip_status(pom::launch_gate(p, false, static_cast<hipStream_t>(stream)), "pom_gate_fwd launch");
}

int pom_gate_bwd(int dtype, int64_t B, int64_t N, int64_t P, const pom_view* ys, const float* bias,
                 const float* hagg, int64_t groups, const pom_rope* rope, const pom_view* grad_sh,
                 const pom_view* grad_ys, float* grad_hagg, float* grad_bias, void* workspace,
                 size_t workspace_bytes, void* stream) {
  pom::GateParams p;
  if (int r = check_view(grad_sh, "grad_sh")) return r;
  if (int r = check_view(grad_ys, "grad_ys")) return r;
  if (int r = setup_gate(p, dtype, B, N, P, ys, hagg, groups, rope, {grad_sh, grad_ys})) return r;
  if (!grad_hagg) return fail(POM_ERR_INVALID, "grad_hagg is null");
  p.bias = bias;
  p.dsh = grad_sh->data; p.dsb = grad_sh->stride_b; p.dsn = grad_sh->stride_n;
  p.dys = grad_ys->data; p.dyb = grad_ys->stride_b; p.dyn = grad_ys->stride_n;
  p.dhagg = grad_hagg; p.dbias = grad_bias;
  const size_t need = gate_ws_bytes(p);
  if (!workspace || workspace_bytes < need)
    return fail(POM_ERR_WORKSPACE, "gate workspace %zu bytes, need %zu", workspace_bytes, need);
  const bool row_groups = p.Lg < p.RC;   // per-token groups need no group counters
  const size_t counters = (size_t)((row_groups ? 0 : p.B * p.G * p.nslabs) + p.B * p.nslabs + p.nslabs);
  if (counters * sizeof(int) > POM_COUNTER_BYTES)
    return fail(POM_ERR_UNSUPPORTED, "too many groups for the counter area");
  Carve c{static_cast<char*>(workspace), workspace_bytes, 0};
  p.cnt_h = c.take<int>(row_groups ? 0 : p.B * p.G * p.nslabs);
  p.cnt_b1 = c.take<int>(p.B * p.nslabs);
  p.cnt_b2 = c.take<int>(p.nslabs);
  c.off = POM_COUNTER_BYTES;
  p.part_h = c.take<float>(p.B * p.nchunks * p.P);
  p.part_b = c.take<float>(p.B * p.nchunks * p.P);
  p.part_bb = c.take<float>(p.B * p.P);
  return hip_status(pom::launch_gate(p, true, static_cast<hipStream_t>(stream)), "pom_gate_bwd launch");
}

}  // extern "C"
