// C ABI of the PoM kernels: argument validation, launch geometry, workspace
// carving and dtype dispatch.  See include/pom_amd.h for the contract.
#include <hip/hip_runtime.h>
#include <hip/hip_bf16.h>
#include <hip/hip_fp16.h>

#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <initializer_list>
#include <mutex>
#include <string>

#include "../../include/pom_amd.h"
#include "gemm.h"
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

bool aligned(const void* p, int64_t bytes) { return (reinterpret_cast<uintptr_t>(p) % (uintptr_t)bytes) == 0; }

int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

int ilog2_ceil(int64_t v) {
  int l = 0;
  while ((int64_t(1) << l) < v) ++l;
  return l;
}

// Tunables (read once): lanes per token row, target workgroup count and the
// shortest chunk worth its own workgroup.
struct Tune {
  int lpr_log2 = 3;        // 8 lanes x 16 bytes = 128-byte row segments
  int64_t target_wg = 1024;      // per-head general path, polynomial features
  int64_t gate_target_wg = 2048; // full-width gating kernels (all frames; RoPE lanes count twice)
  int64_t agg_target_wg = 512;   // aggregation: one chunk per row when B * slabs reaches it
  int64_t min_rows = 128;
  int64_t scan_target_wg = 2048;
  int heads_rows = 1;              // per-head backward: row walk where it applies
  int64_t heads_rows_target = 512; // per-head row walk: workgroups wanted
  Tune() {
    if (const char* s = getenv("POM_AMD_LPR_LOG2")) lpr_log2 = atoi(s);
    if (const char* s = getenv("POM_AMD_TARGET_WG")) target_wg = atoll(s);
    if (const char* s = getenv("POM_AMD_GATE_TARGET_WG")) gate_target_wg = atoll(s);
    if (const char* s = getenv("POM_AMD_AGG_TARGET_WG")) agg_target_wg = atoll(s);
    if (const char* s = getenv("POM_AMD_MIN_ROWS")) min_rows = atoll(s);
    if (const char* s = getenv("POM_AMD_SCAN_TARGET_WG")) scan_target_wg = atoll(s);
    if (const char* s = getenv("POM_AMD_HEADS_ROWS")) heads_rows = atoi(s);
    if (const char* s = getenv("POM_AMD_HEADS_ROWS_TARGET")) heads_rows_target = atoll(s);
    if (lpr_log2 < 0 || lpr_log2 > 6) lpr_log2 = 3;
    if (target_wg < 1) target_wg = 1024;
    if (gate_target_wg < 1) gate_target_wg = 2048;
    if (agg_target_wg < 1) agg_target_wg = 512;
    if (min_rows < 1) min_rows = 128;
    if (scan_target_wg < 1) scan_target_wg = 2048;
    if (heads_rows_target < 1) heads_rows_target = 512;
  }
};
const Tune& tune() {
  static const Tune t;
  return t;
}

// Largest vector width (units per lane) that every pointer, stride and unit
// count admits: 16-byte accesses when possible.
int choose_cpt(int dtype, int64_t units, std::initializer_list<const void*> ptrs,
               std::initializer_list<int64_t> strides, const pom::RopeTables* rope) {
  const int eb = elem_bytes(dtype);
  int cpt = 16 / eb;
  while (cpt > 1) {
    bool ok = units % cpt == 0;
    for (const void* p : ptrs) ok = ok && (p == nullptr || aligned(p, (int64_t)cpt * eb));
    for (int64_t s : strides) ok = ok && (s % cpt == 0);
    if (rope && rope->cos0) {
      // fp32 tables are read cpt at a time
      ok = ok && rope->stride % cpt == 0 && aligned(rope->cos0, 4 * cpt) && aligned(rope->sin0, 4 * cpt) &&
           (!rope->cos1 || aligned(rope->cos1, 4 * cpt)) && (!rope->sin1 || aligned(rope->sin1, 4 * cpt));
    }
    if (ok) break;
    cpt /= 2;
  }
  return cpt;
}

// Slabs for `nvec` vector columns.
void choose_slabs(pom::Geom& g) {
  int lb = tune().lpr_log2;
  const int need = ilog2_ceil(g.nvec);
  if (need < lb) lb = need;
  g.lpr_log2 = lb;
  g.nslabs = cdiv(g.nvec, int64_t(1) << lb);
}

// Chunks: frames of L rows cut into cpf chunks, doubling cpf until one
// frame's grid reaches the target or chunks would drop below min_rows.  The
// choice ignores the frame count on purpose: a frame is then summed in the
// same order whether it arrives alone (PoM.state_forward) or among others.
void choose_chunks(pom::Geom& g, int64_t B, int64_t target) {
  int64_t cpf = 1;
  while (B * cpf * g.nslabs < target && cdiv(g.L, 2 * cpf) >= tune().min_rows) cpf *= 2;
  g.RC = cdiv(g.L, cpf);
  g.cpf = cdiv(g.L, g.RC);
  g.nch = g.F * g.cpf;
}

// Gating-kernel chunks.  The gate forward is elementwise and only the
// backward's dhagg / dbias sums follow the chunking, so unlike the
// aggregation's, the count may depend on the frames: the workgroups of all
// frames together are held near the target.  A RoPE lane carries both
// halves of its pairs, so RoPE modes aim at half as many workgroups.
void choose_gate_chunks(pom::Geom& g, int64_t B, bool rope) {
  const int64_t target = rope ? tune().gate_target_wg / 2 : tune().gate_target_wg;
  int64_t cpf = 1;
  while (B * g.F * cpf * g.nslabs < target && cdiv(g.L, 2 * cpf) >= tune().min_rows) cpf *= 2;
  g.RC = cdiv(g.L, cpf);
  g.cpf = cdiv(g.L, g.RC);
  g.nch = g.F * g.cpf;
}

// Upper bound of the chunk count of choose_chunks for any slab count.
int64_t max_chunks(int64_t F, int64_t L) {
  int64_t cpf = 1;
  while (cdiv(L, 2 * cpf) >= tune().min_rows) cpf *= 2;
  return F * cdiv(L, cdiv(L, cpf));
}

// Scan chunks (token-causal): about scan_target_wg workgroups, >= 16 rows each.
void scan_chunks(int64_t B, int64_t N, int64_t nvec, int64_t& RC, int64_t& nch) {
  const int64_t cols = cdiv(nvec, 256);
  int64_t want = cdiv(tune().scan_target_wg, B * cols);
  if (want < 1) want = 1;
  RC = cdiv(N, want);
  if (RC < 16) RC = 16;
  if (RC > N) RC = N;
  nch = cdiv(N, RC);
}

int64_t scan_max_chunks(int64_t N) { return cdiv(N, N < 16 ? N : 16); }

struct Carve {
  char* base;
  size_t off;
  template <typename T>
  T* take(int64_t count) {
    off = (off + 255) & ~size_t(255);
    T* p = reinterpret_cast<T*>(base + off);
    off += sizeof(T) * (size_t)count;
    return p;
  }
};

size_t carve_bytes(std::initializer_list<int64_t> floats) {
  size_t off = 0;
  for (int64_t n : floats) off = ((off + 255) & ~size_t(255)) + sizeof(float) * (size_t)n;
  return off + 256;
}

int check_view(const pom_view* v, const char* name) {
  if (!v || !v->data) return fail(POM_ERR_INVALID, "%s: null view", name);
  if (v->stride_b < 0 || v->stride_n < 0) return fail(POM_ERR_INVALID, "%s: negative stride", name);
  return POM_OK;
}

int check_dtype(int dtype) {
  if (dtype != POM_DTYPE_F32 && dtype != POM_DTYPE_BF16 && dtype != POM_DTYPE_F16)
    return fail(POM_ERR_INVALID, "unknown dtype %d", dtype);
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

bool is_rope(int mode) {
  return pom::mode_layout(mode) == pom::MODE_ROPE1D || pom::mode_layout(mode) == pom::MODE_ROPE2D;
}

// Units (channels or rotation pairs) a lane vector covers.
int64_t unit_count(int mode, int64_t P) { return is_rope(mode) ? P / 2 : P; }

template <typename F>
hipError_t by_dtype(int dtype, F&& fn) {
  switch (dtype) {
    case POM_DTYPE_F32: return fn(float{});
    case POM_DTYPE_BF16: return fn(__hip_bfloat16{});
    case POM_DTYPE_F16: return fn(__half{});
    default: return hipErrorInvalidValue;
  }
}

// Shared validation and geometry of the aggregation entry points.
int setup_agg(pom::AggParams& p, int dtype, int param_dtype, int64_t B, int64_t N, int64_t P, int K,
              const pom_view* x, const void* coeff, const float* mask, int64_t msb, int64_t msn,
              int64_t frame_len, const pom_rope* rope, const pom_view* gx) {
  if (int r = check_dtype(dtype)) return r;
  if (check_dtype(param_dtype)) return fail(POM_ERR_INVALID, "bad param_dtype %d", param_dtype);
  if (B <= 0 || N <= 0 || P <= 0)
    return fail(POM_ERR_INVALID, "empty shape B=%lld N=%lld P=%lld", (long long)B, (long long)N, (long long)P);
  if (K < 1 || K > POM_MAX_DEGREE) return fail(POM_ERR_UNSUPPORTED, "degree %d outside [1, %d]", K, POM_MAX_DEGREE);
  if (int r = check_view(x, "x")) return r;
  if (!coeff) return fail(POM_ERR_INVALID, "coeff is null");
  if (frame_len <= 0 || N % frame_len)
    return fail(POM_ERR_INVALID, "frame_len %lld must divide N=%lld", (long long)frame_len, (long long)N);
  int rmode;
  if (int r = check_rope(rope, P, p.rope, rmode)) return r;
  if (mask) {
    if (frame_len != N) return fail(POM_ERR_UNSUPPORTED, "masked aggregation with frames");
    p.mode = rmode == pom::MODE_ROPE1D ? pom::MODE_ROPE1D_MASKED
           : rmode == pom::MODE_ROPE2D ? pom::MODE_ROPE2D_MASKED : pom::MODE_MASKED;
  } else {
    p.mode = rmode;
  }
  p.dtype = dtype; p.K = K; p.B = B; p.N = N; p.P = P;
  p.x = x->data; p.sxb = x->stride_b; p.sxn = x->stride_n;
  p.coeff = {coeff, param_dtype};
  p.mask = mask; p.msb = msb; p.msn = msn;
  const void* gxp = gx ? gx->data : nullptr;
  const int64_t sgb = gx ? gx->stride_b : 0, sgn = gx ? gx->stride_n : 0;
  const int64_t units = unit_count(p.mode, P);
  p.g.cpt = choose_cpt(dtype, pom::mode_layout(p.mode) == pom::MODE_ROPE2D ? P / 4 : units, {x->data, gxp},
                       {x->stride_b, x->stride_n, sgb, sgn}, is_rope(p.mode) ? &p.rope : nullptr);
  p.g.nvec = units / p.g.cpt;
  choose_slabs(p.g);
  if (frame_len == 1 && N > 1) {
    p.g.L = N;   // token-causal: the scan sets its own chunking (setup_scan)
    p.g.F = 1;
  } else {
    p.g.L = frame_len;
    p.g.F = N / frame_len;
  }
  choose_chunks(p.g, B, tune().agg_target_wg);
  if (p.g.nslabs > 0x7fffffffLL || p.g.nch > 65535 || B > 65535)
    return fail(POM_ERR_UNSUPPORTED, "grid too large (slabs %lld, chunks %lld, B %lld)", (long long)p.g.nslabs,
                (long long)p.g.nch, (long long)B);
  return POM_OK;
}

// Token-causal scan geometry on top of setup_agg (which saw frame_len == 1).
void setup_scan(const pom::AggParams& a, pom::ScanParams& s) {
  s.dtype = a.dtype; s.mode = a.mode; s.K = a.K; s.cpt = a.g.cpt; s.nvec = a.g.nvec;
  s.B = a.B; s.N = a.N; s.P = a.P;
  scan_chunks(a.B, a.N, a.g.nvec, s.RC, s.nch);
  s.x = a.x; s.sxb = a.sxb; s.sxn = a.sxn; s.coeff = a.coeff; s.rope = a.rope;
}

size_t agg_ws_bytes(int64_t B, int64_t N, int64_t P, int K, int64_t frame_len, bool bwd) {
  if (frame_len == 1 && N > 1) {
    const int64_t nc = scan_max_chunks(N);
    return bwd ? carve_bytes({B * nc * P, B * nc * K * P}) : carve_bytes({B * nc * P});
  }
  const int64_t F = N / frame_len;
  const int64_t nc = max_chunks(F, frame_len);
  return bwd ? carve_bytes({B * nc * K * P, B * F * P}) : carve_bytes({B * nc * P, B * nc});
}

// Channel-major copy requested by `tv` (or none): validated against the
// geometry chosen for the launch.
int set_tview(pom::TrOut& t, const pom_tview* tv, int dtype, int cpt, int64_t B, int64_t N, const char* name) {
  if (!tv) return POM_OK;
  if (!tv->data) return fail(POM_ERR_INVALID, "%s: data is null", name);
  if (dtype == POM_DTYPE_F32 || cpt != 8)
    return fail(POM_ERR_UNSUPPORTED, "%s: the channel-major copy needs 16-bit elements and 16-byte lanes", name);
  if (!aligned(tv->data, 2)) return fail(POM_ERR_INVALID, "%s: data must be element-aligned", name);
  if (tv->stride_b < N || tv->stride_c < (B - 1) * tv->stride_b + N)
    return fail(POM_ERR_INVALID, "%s: strides (c %lld, b %lld) overlap for B=%lld N=%lld", name,
                (long long)tv->stride_c, (long long)tv->stride_b, (long long)B, (long long)N);
  t.data = tv->data;
  t.ld = tv->stride_c;
  t.sb = tv->stride_b;
  return POM_OK;
}

int need_ws(void* ws, size_t have, size_t need) {
  if (!ws) return fail(POM_ERR_WORKSPACE, "workspace is null (need %zu bytes)", need);
  if (have < need) return fail(POM_ERR_WORKSPACE, "workspace %zu bytes, need %zu", have, need);
  if (!aligned(ws, 256)) return fail(POM_ERR_WORKSPACE, "workspace must be 256-byte aligned");
  return POM_OK;
}

int setup_gate(pom::GateParams& p, int& per_token, int dtype, int64_t B, int64_t N, int64_t P,
               const pom_view* ys, const void* hagg, int64_t groups, const pom_rope* rope,
               std::initializer_list<const pom_view*> views) {
  if (int r = check_dtype(dtype)) return r;
  if (B <= 0 || N <= 0 || P <= 0) return fail(POM_ERR_INVALID, "empty shape");
  if (int r = check_view(ys, "y_s")) return r;
  for (const pom_view* v : views)
    if (int r = check_view(v, "gate view")) return r;
  if (!hagg) return fail(POM_ERR_INVALID, "hagg is null");
  if (groups <= 0 || N % groups)
    return fail(POM_ERR_INVALID, "groups %lld must divide N=%lld", (long long)groups, (long long)N);
  if (int r = check_rope(rope, P, p.rope, p.mode)) return r;
  p.dtype = dtype; p.B = B; p.N = N; p.P = P;
  p.ys = ys->data; p.ysb = ys->stride_b; p.ysn = ys->stride_n;
  p.hagg = hagg;
  per_token = (groups == N && N > 1) ? 1 : 0;
  const int64_t units = unit_count(p.mode, P);
  const void* ptrs[3] = {nullptr, nullptr, nullptr};
  int64_t strides[6] = {0, 0, 0, 0, 0, 0};
  int i = 0;
  for (const pom_view* v : views) {
    if (i < 3) { ptrs[i] = v->data; strides[2 * i] = v->stride_b; strides[2 * i + 1] = v->stride_n; }
    ++i;
  }
  p.g.cpt = choose_cpt(dtype, p.mode == pom::MODE_ROPE2D ? P / 4 : units, {ys->data, hagg, ptrs[0], ptrs[1], ptrs[2]},
                       {ys->stride_b, ys->stride_n, strides[0], strides[1], strides[2], strides[3], strides[4],
                        strides[5]},
                       is_rope(p.mode) ? &p.rope : nullptr);
  // fp32 partial and dhagg rows are written cpt at a time: P must admit it
  while (p.g.cpt > 1 && P % p.g.cpt) p.g.cpt /= 2;
  p.g.nvec = units / p.g.cpt;
  choose_slabs(p.g);
  if (per_token || groups == 1) {
    p.g.F = 1;
    p.g.L = N;
  } else {
    p.g.F = groups;
    p.g.L = N / groups;
  }
  choose_gate_chunks(p.g, B, is_rope(p.mode));
  if (p.g.nch > 65535 || B > 65535) return fail(POM_ERR_UNSUPPORTED, "grid too large");
  return POM_OK;
}

size_t gate_ws_bytes(int64_t B, int64_t N, int64_t P, int64_t groups) {
  const bool per_token = groups == N && N > 1;
  const int64_t F = (per_token || groups == 1) ? 1 : groups;
  const int64_t nc = max_chunks(F, N / F);
  return carve_bytes({B * nc * P, B * nc * P});
}

// Per-head gating geometry: chunk width V, token-kernel grid, aggregate-
// gradient chunks.  Depends on the shape only (the workspace size query
// repeats it without pointers), except V, which also follows alignment.
struct HeadsGeom {
  int64_t tok_wgs = 1, RC = 1, cpf = 1, nch = 1, L = 1, G = 1;
};

HeadsGeom heads_geom(int64_t B, int64_t N, int64_t P, int64_t groups, int V) {
  HeadsGeom g;
  const int64_t ntok = B * N;
  g.tok_wgs = cdiv(ntok, 4);
  if (g.tok_wgs > 1024) g.tok_wgs = 1024;
  g.G = groups;
  g.L = N / groups;
  const int64_t cols = cdiv(P / V, 256);
  int64_t cpf = 1;
  while (B * cols * g.G * cpf < tune().target_wg && cdiv(g.L, 2 * cpf) >= 16) cpf *= 2;
  g.RC = cdiv(g.L, cpf);
  g.cpf = cdiv(g.L, g.RC);
  g.nch = g.G * g.cpf;
  return g;
}

// Tile path geometry: 64-token x 64-channel workgroups.
constexpr int64_t kHeadTile = 64;

int64_t heads_nhm(int64_t P, int64_t H) {
  const int64_t hd = P / H, n = (kHeadTile - 1) / (hd > 0 ? hd : 1) + 2;
  return n < H ? n : H;
}

// Token tiles per backward workgroup: 4 when every walk stays inside one group
// (single-token groups, or groups a multiple of 4 tiles long), else 1.
int heads_tpw(int64_t N, int64_t L) {
  (void)N;
  return (L == 1 || L % (4 * kHeadTile) == 0) ? 4 : 1;
}

// Row-walk backward: tokens per walk, the largest of 256 .. 8 that gives the
// target workgroup count (walks stay inside one hagg group); 0 when the row
// walk does not apply (single-token groups, head_dim not a multiple of 8, a
// row wider than one workgroup, or more heads than its reduction slots).
int64_t heads_rows_wt(int64_t B, int64_t N, int64_t P, int64_t H, int64_t groups) {
  if (!tune().heads_rows || groups <= 0 || N % groups) return 0;
  const int64_t L = N / groups;
  if (L == 1 || P % 8 || P % H || (P / H) % 8) return 0;
  if (pom::heads_rows_threads(P, H) > 1024 || pom::heads_rows_smem(P, H) > 64 * 1024) return 0;
  if (B > 65535) return 0;
  int64_t pick = 0;
  for (int64_t wt : {256, 128, 64, 32, 16, 8}) {
    if (groups > 1 && L % wt) continue;
    pick = wt;
    if (B * cdiv(N, wt) >= tune().heads_rows_target) break;
  }
  return pick;
}

size_t heads_ws_bytes(int64_t B, int64_t N, int64_t P, int64_t H, int64_t groups) {
  int64_t nch = 1, tok_wgs = 1;
  for (int V : {1, 2, 4, 8}) {   // every chunk width the call may choose
    const HeadsGeom g = heads_geom(B, N, P, groups, V);
    if (g.nch > nch) nch = g.nch;
    tok_wgs = g.tok_wgs;
  }
  const size_t general = carve_bytes({B * N * H, tok_wgs * H, B * nch * P});
  const int64_t nct = cdiv(P, kHeadTile), ntt = cdiv(N, kHeadTile);
  const size_t tile = carve_bytes({B * N * nct * heads_nhm(P, H), B * ntt * P, B * N * H});
  size_t best = general > tile ? general : tile;
  if (const int64_t wt = heads_rows_wt(B, N, P, H, groups)) {
    const int64_t nw = cdiv(N, wt);
    const size_t rows = carve_bytes({B * nw * P, B * nw * H});
    if (rows > best) best = rows;
  }
  return best;
}

int setup_heads(pom::HeadsParams& p, int dtype, int param_dtype, int64_t B, int64_t N, int64_t P, int64_t H,
                const pom_view* ys, const void* bias, const void* hagg, int64_t groups, const pom_rope* rope,
                std::initializer_list<const pom_view*> views) {
  if (int r = check_dtype(dtype)) return r;
  if (check_dtype(param_dtype)) return fail(POM_ERR_INVALID, "bad param_dtype %d", param_dtype);
  if (B <= 0 || N <= 0 || P <= 0) return fail(POM_ERR_INVALID, "empty shape");
  if (H <= 0 || P % H)
    return fail(POM_ERR_INVALID, "head count %lld must divide P=%lld", (long long)H, (long long)P);
  if (int r = check_view(ys, "y_s")) return r;
  for (const pom_view* v : views)
    if (int r = check_view(v, "gate view")) return r;
  if (!hagg) return fail(POM_ERR_INVALID, "hagg is null");
  if (groups <= 0 || N % groups)
    return fail(POM_ERR_INVALID, "groups %lld must divide N=%lld", (long long)groups, (long long)N);
  if (int r = check_rope(rope, H, p.rope, p.mode)) return r;
  p.dtype = dtype; p.B = B; p.N = N; p.P = P; p.H = H; p.hd = P / H;
  p.ys = ys->data; p.ysb = ys->stride_b; p.ysn = ys->stride_n;
  p.bias = {bias, param_dtype};
  p.hagg = hagg;
  // chunk width: the widest (<= 16 bytes) that divides head_dim and that every
  // vector operand's base and strides admit
  const int eb = elem_bytes(dtype);
  int V = 16 / eb;
  while (V > 1) {
    bool ok = p.hd % V == 0 && aligned(hagg, (int64_t)V * eb);
    for (const pom_view* v : views)
      ok = ok && aligned(v->data, (int64_t)V * eb) && v->stride_b % V == 0 && v->stride_n % V == 0;
    if (ok) break;
    V /= 2;
  }
  p.V = V;
  if (pom::heads_token_smem_bytes(P / V, H) > 64 * 1024)
    return fail(POM_ERR_UNSUPPORTED, "per-head gating: P/V + 2H = %lld too large for the row kernel",
                (long long)(P / V + 2 * H));
  const HeadsGeom g = heads_geom(B, N, P, groups, V);
  p.tok_wgs = g.tok_wgs; p.RC = g.RC; p.cpf = g.cpf; p.nch = g.nch; p.L = g.L; p.G = g.G;
  if (p.nch > 65535 || B > 65535) return fail(POM_ERR_UNSUPPORTED, "grid too large");
  // tile path: 8-element vectors on every P-wide operand, tiles inside one group
  bool tile = P % 8 == 0 && (p.L == 1 || p.L % kHeadTile == 0) && aligned(hagg, 16) &&
              cdiv(N, kHeadTile) <= 65535 && H <= 256 &&   // dz tile: kHeadTile x H floats of LDS
              P / H >= 8;                                   // a tile touches at most 9 heads
  for (const pom_view* v : views)
    tile = tile && aligned(v->data, 16) && v->stride_b % 8 == 0 && v->stride_n % 8 == 0;
  p.tile = tile ? 1 : 0;
  p.tpw = heads_tpw(N, p.L);
  p.ntt = cdiv(N, kHeadTile * p.tpw);
  p.nhm = heads_nhm(P, H);
  return POM_OK;
}

// Polynomial-feature geometry: chunk width V (<= 16 bytes, aligned, and at
// most 32 / KM so the per-thread coefficient and gradient arrays stay in
// registers) and token chunks.
int features_km(int K) { return K <= 4 ? K : (K <= 8 ? 8 : 16); }

void features_chunks(int64_t B, int64_t N, int64_t P, int V, int64_t& RC, int64_t& nch) {
  const int64_t cols = cdiv(P / V, 256);
  int64_t cpf = 1;
  while (B * cols * cpf < tune().target_wg && cdiv(N, 2 * cpf) >= 16) cpf *= 2;
  RC = cdiv(N, cpf);
  nch = cdiv(N, RC);
}

size_t features_ws_bytes(int64_t B, int64_t N, int64_t P, int K) {
  int64_t nch = 1;
  for (int V : {1, 2, 4, 8}) {
    int64_t rc, n;
    features_chunks(B, N, P, V, rc, n);
    if (n > nch) nch = n;
  }
  return carve_bytes({B * nch * (int64_t)K * P});
}

int setup_features(pom::FeatParams& p, int dtype, int param_dtype, int64_t B, int64_t N, int64_t P, int K,
                   const pom_view* x, const void* coeff, std::initializer_list<const pom_view*> views) {
  if (int r = check_dtype(dtype)) return r;
  if (check_dtype(param_dtype)) return fail(POM_ERR_INVALID, "bad param_dtype %d", param_dtype);
  if (B <= 0 || N <= 0 || P <= 0) return fail(POM_ERR_INVALID, "empty shape");
  if (K < 1 || K > POM_MAX_DEGREE) return fail(POM_ERR_UNSUPPORTED, "degree %d outside [1, %d]", K, POM_MAX_DEGREE);
  if (int r = check_view(x, "x")) return r;
  for (const pom_view* v : views)
    if (int r = check_view(v, "features view")) return r;
  if (!coeff) return fail(POM_ERR_INVALID, "coeff is null");
  p.dtype = dtype; p.K = K; p.B = B; p.N = N; p.P = P;
  p.x = x->data; p.sxb = x->stride_b; p.sxn = x->stride_n;
  p.coeff = {coeff, param_dtype};
  const int eb = elem_bytes(dtype);
  int V = 16 / eb;
  const int vmax = 32 / features_km(K) > 0 ? 32 / features_km(K) : 1;
  while (V > vmax) V /= 2;
  while (V > 1) {
    bool ok = P % V == 0 && aligned(x->data, (int64_t)V * eb) && x->stride_b % V == 0 && x->stride_n % V == 0;
    for (const pom_view* v : views)
      ok = ok && aligned(v->data, (int64_t)V * eb) && v->stride_b % V == 0 && v->stride_n % V == 0;
    if (ok) break;
    V /= 2;
  }
  p.V = V;
  features_chunks(B, N, P, V, p.RC, p.nch);
  if (p.nch > 65535 || B > 65535) return fail(POM_ERR_UNSUPPORTED, "grid too large");
  return POM_OK;
}

}  // namespace

// Device scratch of pom_agg_fwd_noalloc: one copy per GPU, allocated when the
// code object is loaded on that GPU and held until the process ends.  In host
// code the name is only a handle; the device address comes from
// hipGetSymbolAddress, once per device, and only that address is ever passed
// to a kernel.
static __device__ __align__(256) unsigned char scratch[POM_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxScratchDevices] = {};

// Device address of `scratch` on the current device (looked up on the first
// call per device, with that device current).
int scratch_for_current_device(void** out) {
  int dev = -1;
  if (hipError_t e = hipGetDevice(&dev); e != hipSuccess) return hip_status(e, "hipGetDevice");
  if (dev < 0 || dev >= kMaxScratchDevices)
    return fail(POM_ERR_UNSUPPORTED, "device index %d is beyond the %d the static scratch tracks", dev,
                kMaxScratchDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    if (hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)); e != hipSuccess)
      return hip_status(e, "hipGetSymbolAddress(scratch)");
    if (!p) return fail(POM_ERR_DEVICE, "hipGetSymbolAddress(scratch) returned null");
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return POM_OK;
}

}  // namespace

namespace pom {
// The calling thread's pom_last_error() message, for the other C ABI files.
int set_error(int code, const char* msg) {
  g_err = msg;
  return code;
}
}  // namespace pom

extern "C" {

int pom_abi_version(void) { return POM_AMD_ABI_VERSION; }

const char* pom_last_error(void) { return g_err.c_str(); }

size_t pom_agg_workspace_size(int dtype, int64_t B, int64_t N, int64_t P, int K, int64_t frame_len, int rope_kind,
                              int backward) {
  if (check_dtype(dtype) || B <= 0 || N <= 0 || P <= 0 || K < 1 || K > POM_MAX_DEGREE || frame_len <= 0 ||
      N % frame_len || rope_kind < POM_ROPE_NONE || rope_kind > POM_ROPE_2D)
    return 0;
  return agg_ws_bytes(B, N, P, K, frame_len, backward != 0);
}

int pom_agg_fwd(int dtype, int param_dtype, int64_t B, int64_t N, int64_t P, int K, const pom_view* x,
                const void* coeff,
                const float* mask, int64_t mask_stride_b, int64_t mask_stride_n, int64_t frame_len,
                const void* carry, int64_t n_past, const pom_rope* rope, void* out, float* count_out,
                void* workspace, size_t workspace_bytes, void* stream) {
  pom::AggParams p;
  if (int r = setup_agg(p, dtype, param_dtype, B, N, P, K, x, coeff, mask, mask_stride_b, mask_stride_n, frame_len, rope,
                        nullptr))
    return r;
  if (!out) return fail(POM_ERR_INVALID, "out is null");
  if (carry && n_past < 1) return fail(POM_ERR_INVALID, "carry given with n_past=%lld", (long long)n_past);
  if (mask && !count_out) return fail(POM_ERR_INVALID, "masked forward needs count_out");
  if (carry && frame_len == 1 && N > 1) return fail(POM_ERR_UNSUPPORTED, "carry with token-causal aggregation");
  p.carry = carry;
  p.n_past = carry ? n_past : 0;
  p.out = out;
  p.count_out = count_out;
  const hipStream_t st = static_cast<hipStream_t>(stream);
  if (int r = need_ws(workspace, workspace_bytes, agg_ws_bytes(B, N, P, K, frame_len, false))) return r;
  Carve c{static_cast<char*>(workspace), 0};
  if (frame_len == 1 && N > 1) {
    pom::ScanParams s;
    setup_scan(p, s);
    s.out = out;
    s.csum = c.take<float>(B * s.nch * P);
    return hip_status(by_dtype(dtype, [&](auto t) { return pom::scan_fwd_t<decltype(t)>(s, st); }),
                      "pom_agg_fwd (token-causal) launch");
  }
  p.direct = (p.g.nch == 1 && p.g.F == 1 && !carry) ? 1 : 0;
  p.part = c.take<float>(B * p.g.nch * P);
  p.pcnt = c.take<float>(B * p.g.nch);
  return hip_status(by_dtype(dtype, [&](auto t) { return pom::agg_fwd_t<decltype(t)>(p, st); }),
                    "pom_agg_fwd launch");
}

int pom_agg_fwd_noalloc(int dtype, int param_dtype, int64_t B, int64_t N, int64_t P, int K, const pom_view* x,
                        const void* coeff, const float* mask, int64_t mask_stride_b, int64_t mask_stride_n,
                        int64_t frame_len, const void* carry, int64_t n_past, const pom_rope* rope, void* out,
                        float* count_out, void* stream) {
  // The scratch size is checked from the shape alone, before anything else.
  // An invalid shape reports 0 here and is rejected by pom_agg_fwd's checks.
  const size_t need = pom_agg_workspace_size(dtype, B, N, P, K, frame_len, rope ? rope->kind : POM_ROPE_NONE, 0);
  if (need > POM_NOALLOC_SCRATCH_BYTES)
    return fail(POM_ERR_WORKSPACE,
                "pom_agg_fwd_noalloc: this shape needs %zu bytes of scratch, more than the %zu of the static "
                "scratch; call pom_agg_fwd with a workspace instead",
                need, (size_t)POM_NOALLOC_SCRATCH_BYTES);
  void* ws = nullptr;
  if (int r = scratch_for_current_device(&ws)) return r;
  return pom_agg_fwd(dtype, param_dtype, B, N, P, K, x, coeff, mask, mask_stride_b, mask_stride_n, frame_len, carry,
                     n_past, rope, out, count_out, ws, POM_NOALLOC_SCRATCH_BYTES, stream);
}

int pom_agg_bwd(int dtype, int param_dtype, int64_t B, int64_t N, int64_t P, int K, const pom_view* x,
                const void* coeff,
                const float* mask, int64_t mask_stride_b, int64_t mask_stride_n, const float* count,
                int64_t frame_len, int64_t n_past, const pom_rope* rope, const float* grad_out,
                const pom_view* grad_x, const pom_tview* grad_x_t, void* grad_coeff, void* workspace,
                size_t workspace_bytes, void* stream) {
  pom::AggParams p;
  if (int r = check_view(grad_x, "grad_x")) return r;
  if (int r = setup_agg(p, dtype, param_dtype, B, N, P, K, x, coeff, mask, mask_stride_b, mask_stride_n, frame_len, rope,
                        grad_x))
    return r;
  if (!grad_out || !grad_coeff) return fail(POM_ERR_INVALID, "grad_out / grad_coeff is null");
  if (mask && !count) return fail(POM_ERR_INVALID, "masked backward needs the forward's count");
  if (n_past < 0) return fail(POM_ERR_INVALID, "negative n_past");
  if (n_past > 0 && frame_len == 1 && N > 1) return fail(POM_ERR_UNSUPPORTED, "carry with token-causal aggregation");
  if (grad_x_t && frame_len == 1 && N > 1)
    return fail(POM_ERR_UNSUPPORTED, "grad_x_t with token-causal aggregation");
  if (grad_x_t && mask && is_rope(p.mode))
    return fail(POM_ERR_UNSUPPORTED, "grad_x_t with masked RoPE aggregation");
  if (int r = set_tview(p.gxt, grad_x_t, dtype, p.g.cpt, B, N, "grad_x_t")) return r;
  const hipStream_t st = static_cast<hipStream_t>(stream);
  if (int r = need_ws(workspace, workspace_bytes, agg_ws_bytes(B, N, P, K, frame_len, true))) return r;
  Carve c{static_cast<char*>(workspace), 0};
  if (frame_len == 1 && N > 1) {
    pom::ScanParams s;
    setup_scan(p, s);
    s.go = grad_out;
    s.gx = grad_x->data; s.sgb = grad_x->stride_b; s.sgn = grad_x->stride_n;
    s.gc = {grad_coeff, param_dtype};
    s.csum = c.take<float>(B * s.nch * P);
    s.part = c.take<float>(B * s.nch * K * P);
    return hip_status(by_dtype(dtype, [&](auto t) { return pom::scan_bwd_t<decltype(t)>(s, st); }),
                      "pom_agg_bwd (token-causal) launch");
  }
  if (is_rope(p.mode) && !grad_x_t) {
    // one lane per half of a rotation pair (the units become channels), and
    // with 16- or 8-byte lanes up to four batch rows per workgroup sharing
    // each table lookup
    p.g.half = 1;
    p.g.nb = (mask || p.g.cpt < 4) ? 1 : (B % 4 == 0 ? 4 : (B % 2 == 0 ? 2 : 1));
    p.g.nvec *= 2;
    choose_slabs(p.g);
    choose_chunks(p.g, B / p.g.nb, tune().agg_target_wg);
    if (p.g.nslabs > 0x7fffffffLL || p.g.nch > 65535)
      return fail(POM_ERR_UNSUPPORTED, "grid too large (slabs %lld, chunks %lld)", (long long)p.g.nslabs,
                  (long long)p.g.nch);
  }
  p.n_past = n_past;
  p.go = grad_out;
  p.count_in = count;
  p.gx = grad_x->data; p.sgb = grad_x->stride_b; p.sgn = grad_x->stride_n;
  p.gc = {grad_coeff, param_dtype};
  p.part = c.take<float>(B * p.g.nch * K * P);
  float* wf = c.take<float>(B * p.g.F * P);
  p.wf = p.g.F > 1 ? wf : nullptr;
  return hip_status(by_dtype(dtype, [&](auto t) { return pom::agg_bwd_t<decltype(t)>(p, st); }),
                    "pom_agg_bwd launch");
}

size_t pom_gate_workspace_size(int dtype, int64_t B, int64_t N, int64_t P, int64_t groups, int rope_kind) {
  if (check_dtype(dtype) || B <= 0 || N <= 0 || P <= 0 || groups <= 0 || N % groups ||
      rope_kind < POM_ROPE_NONE || rope_kind > POM_ROPE_2D)
    return 0;
  return gate_ws_bytes(B, N, P, groups);
}

int pom_gate_fwd(int dtype, int param_dtype, int64_t B, int64_t N, int64_t P, const pom_view* ys,
                 const void* bias, const void* hagg, int64_t groups, const pom_rope* rope, const pom_view* sh,
                 const pom_tview* sh_t, void* stream) {
  pom::GateParams p;
  int per_token = 0;
  if (int r = check_view(sh, "sh")) return r;
  if (int r = setup_gate(p, per_token, dtype, B, N, P, ys, hagg, groups, rope, {sh})) return r;
  if (int r = set_tview(p.sht, sh_t, dtype, p.g.cpt, B, N, "sh_t")) return r;
  if (check_dtype(param_dtype)) return fail(POM_ERR_INVALID, "bad param_dtype %d", param_dtype);
  p.bias = {bias, param_dtype};
  p.sh = sh->data; p.shb = sh->stride_b; p.shn = sh->stride_n;
  const hipStream_t st = static_cast<hipStream_t>(stream);
  return hip_status(by_dtype(dtype, [&](auto t) { return pom::gate_fwd_t<decltype(t)>(p, per_token, st); }),
                    "pom_gate_fwd launch");
}

int pom_gate_bwd(int dtype, int param_dtype, int64_t B, int64_t N, int64_t P, const pom_view* ys,
                 const void* bias, const void* hagg, int64_t groups, const pom_rope* rope,
                 const pom_view* grad_sh, const pom_view* grad_ys, const pom_tview* grad_ys_t, float* grad_hagg,
                 void* grad_bias,
                 void* workspace, size_t workspace_bytes, void* stream) {
  pom::GateParams p;
  int per_token = 0;
  if (int r = check_view(grad_sh, "grad_sh")) return r;
  if (int r = check_view(grad_ys, "grad_ys")) return r;
  if (int r = setup_gate(p, per_token, dtype, B, N, P, ys, hagg, groups, rope, {grad_sh, grad_ys})) return r;
  if (!grad_hagg) return fail(POM_ERR_INVALID, "grad_hagg is null");
  if (!aligned(grad_hagg, 4 * p.g.cpt)) return fail(POM_ERR_INVALID, "grad_hagg must be 16-byte aligned");
  if (int r = set_tview(p.dyst, grad_ys_t, dtype, p.g.cpt, B, N, "grad_ys_t")) return r;
  if (check_dtype(param_dtype)) return fail(POM_ERR_INVALID, "bad param_dtype %d", param_dtype);
  p.bias = {bias, param_dtype};
  p.dsh = grad_sh->data; p.dsb = grad_sh->stride_b; p.dsn = grad_sh->stride_n;
  p.dys = grad_ys->data; p.dyb = grad_ys->stride_b; p.dyn = grad_ys->stride_n;
  p.dhagg = grad_hagg;
  p.dbias = {grad_bias, param_dtype};
  if (int r = need_ws(workspace, workspace_bytes, gate_ws_bytes(B, N, P, groups))) return r;
  Carve c{static_cast<char*>(workspace), 0};
  p.part_h = c.take<float>(B * p.g.nch * P);
  p.part_b = c.take<float>(B * p.g.nch * P);
  const hipStream_t st = static_cast<hipStream_t>(stream);
  return hip_status(by_dtype(dtype, [&](auto t) { return pom::gate_bwd_t<decltype(t)>(p, per_token, st); }),
                    "pom_gate_bwd launch");
}

size_t pom_gate_heads_workspace_size(int dtype, int64_t B, int64_t N, int64_t P, int64_t H, int64_t groups) {
  if (check_dtype(dtype) || B <= 0 || N <= 0 || P <= 0 || H <= 0 || P % H || groups <= 0 || N % groups) return 0;
  return heads_ws_bytes(B, N, P, H, groups);
}

int pom_gate_heads_fwd(int dtype, int param_dtype, int64_t B, int64_t N, int64_t P, int64_t H,
                       const pom_view* ys, const void* bias, const void* hagg, int64_t groups,
                       const pom_rope* rope, const pom_view* sh, const pom_tview* sh_t, void* stream) {
  pom::HeadsParams p;
  if (int r = check_view(sh, "sh")) return r;
  if (int r = setup_heads(p, dtype, param_dtype, B, N, P, H, ys, bias, hagg, groups, rope, {sh})) return r;
  if (sh_t) {
    // written by the tile kernel in 16-byte token runs
    const bool ok = p.tile && N % 8 == 0 && aligned(sh_t->data, 16) && sh_t->stride_c % 8 == 0 &&
                    sh_t->stride_b % 8 == 0;
    if (int r = set_tview(p.sht, sh_t, dtype, ok ? 8 : 1, B, N, "sh_t")) return r;
  }
  p.sh = sh->data; p.shb = sh->stride_b; p.shn = sh->stride_n;
  // row walk: the plain gate without the channel-major copy, 8-channel chunks
  // inside one head and one hagg row per batch row, 16-byte sh rows and hagg;
  // about heads_rows_target x 4 workgroups of whole 8-row steps
  if (tune().heads_rows && !sh_t && p.mode == pom::MODE_PLAIN && P % 8 == 0 && p.hd % 8 == 0 && p.G == 1 &&
      aligned(hagg, 16) && aligned(sh->data, 16) && sh->stride_b % 8 == 0 && sh->stride_n % 8 == 0) {
    const int64_t cols = cdiv(P / 8, pom::kFwdRowLanes);
    const int64_t want = cdiv(tune().heads_rows_target * 4, B * cols);
    p.fwd_rows = cdiv(cdiv(N, want > 0 ? want : 1), 8) * 8;
    if (cdiv(N, p.fwd_rows) > 65535) p.fwd_rows = cdiv(cdiv(N, 65535), 8) * 8;
  }
  const hipStream_t st = static_cast<hipStream_t>(stream);
  return hip_status(by_dtype(dtype, [&](auto t) { return pom::heads_fwd_t<decltype(t)>(p, st); }),
                    "pom_gate_heads_fwd launch");
}

int pom_gate_heads_bwd(int dtype, int param_dtype, int64_t B, int64_t N, int64_t P, int64_t H,
                       const pom_view* ys, const void* bias, const void* hagg, int64_t groups,
                       const pom_rope* rope, const pom_view* grad_sh, const pom_view* grad_ys,
                       float* grad_hagg, void* grad_bias,
                       void* workspace, size_t workspace_bytes, void* stream) {
  pom::HeadsParams p;
  if (int r = check_view(grad_sh, "grad_sh")) return r;
  if (int r = check_view(grad_ys, "grad_ys")) return r;
  if (int r = setup_heads(p, dtype, param_dtype, B, N, P, H, ys, bias, hagg, groups, rope, {grad_sh})) return r;
  if (!grad_hagg) return fail(POM_ERR_INVALID, "grad_hagg is null");
  if (!aligned(grad_hagg, 4)) return fail(POM_ERR_INVALID, "grad_hagg must be 4-byte aligned");
  p.dsh = grad_sh->data; p.dsb = grad_sh->stride_b; p.dsn = grad_sh->stride_n;
  p.dys = grad_ys->data; p.dyb = grad_ys->stride_b; p.dyn = grad_ys->stride_n;
  p.dhagg = grad_hagg;
  p.dbias = {grad_bias, param_dtype};
  if (p.tile && !aligned(grad_hagg, 16)) p.tile = 0;   // per-token rows are stored 8 floats at a time
  if (int r = need_ws(workspace, workspace_bytes, heads_ws_bytes(B, N, P, H, groups))) return r;
  // row walk: 16-byte chunks of dsh and hagg (the tile path's operand conditions)
  const int64_t wt = heads_rows_wt(B, N, P, H, groups);
  if (wt > 0 && aligned(hagg, 16) && aligned(grad_sh->data, 16) && grad_sh->stride_b % 8 == 0 &&
      grad_sh->stride_n % 8 == 0) {
    p.rows = 1;
    p.wt = wt;
    p.ntt = cdiv(N, wt);
  }
  Carve c{static_cast<char*>(workspace), 0};
  if (p.rows) {
    p.part_h = c.take<float>(B * p.ntt * P);
    p.dzbuf = c.take<float>(B * p.ntt * H);
  } else if (p.tile) {
    p.dpart = c.take<float>(B * N * cdiv(P, kHeadTile) * p.nhm);
    p.part_h = c.take<float>(B * p.ntt * P);
    p.dzbuf = c.take<float>(B * N * H);
  } else {
    p.sgate = c.take<float>(B * N * H);
    p.part_b = c.take<float>(p.tok_wgs * H);
    p.part_h = c.take<float>(B * p.nch * P);
  }
  const hipStream_t st = static_cast<hipStream_t>(stream);
  return hip_status(by_dtype(dtype, [&](auto t) { return pom::heads_bwd_t<decltype(t)>(p, st); }),
                    "pom_gate_heads_bwd launch");
}

size_t pom_features_workspace_size(int dtype, int64_t B, int64_t N, int64_t P, int K) {
  if (check_dtype(dtype) || B <= 0 || N <= 0 || P <= 0 || K < 1 || K > POM_MAX_DEGREE) return 0;
  return features_ws_bytes(B, N, P, K);
}

int pom_features_fwd(int dtype, int param_dtype, int64_t B, int64_t N, int64_t P, int K,
                     const pom_view* x, const void* coeff, const pom_view* out, void* stream) {
  pom::FeatParams p;
  if (int r = check_view(out, "out")) return r;
  if (int r = setup_features(p, dtype, param_dtype, B, N, P, K, x, coeff, {out})) return r;
  p.out = out->data; p.sob = out->stride_b; p.son = out->stride_n;
  const hipStream_t st = static_cast<hipStream_t>(stream);
  return hip_status(by_dtype(dtype, [&](auto t) { return pom::features_fwd_t<decltype(t)>(p, st); }),
                    "pom_features_fwd launch");
}

int pom_features_bwd(int dtype, int param_dtype, int64_t B, int64_t N, int64_t P, int K,
                     const pom_view* x, const void* coeff, const pom_view* grad_out,
                     const pom_view* grad_x, void* grad_coeff,
                     void* workspace, size_t workspace_bytes, void* stream) {
  pom::FeatParams p;
  if (int r = check_view(grad_out, "grad_out")) return r;
  if (int r = check_view(grad_x, "grad_x")) return r;
  if (int r = setup_features(p, dtype, param_dtype, B, N, P, K, x, coeff, {grad_out, grad_x})) return r;
  if (!grad_coeff) return fail(POM_ERR_INVALID, "grad_coeff is null");
  p.go = grad_out->data; p.sgob = grad_out->stride_b; p.sgon = grad_out->stride_n;
  p.gx = grad_x->data; p.sgxb = grad_x->stride_b; p.sgxn = grad_x->stride_n;
  p.gc = {grad_coeff, param_dtype};
  if (int r = need_ws(workspace, workspace_bytes, features_ws_bytes(B, N, P, K))) return r;
  Carve c{static_cast<char*>(workspace), 0};
  p.part = c.take<float>(B * p.nch * (int64_t)K * P);
  const hipStream_t st = static_cast<hipStream_t>(stream);
  return hip_status(by_dtype(dtype, [&](auto t) { return pom::features_bwd_t<decltype(t)>(p, st); }),
                    "pom_features_bwd launch");
}

int pom_transpose(int dtype, int64_t rows, int64_t cols, const void* src, int64_t ld_src, void* dst,
                  int64_t ld_dst, void* stream) {
  if (int r = check_dtype(dtype)) return r;
  if (rows < 0 || cols < 0) return fail(POM_ERR_INVALID, "rows (%lld) and cols (%lld) must be >= 0",
                                        (long long)rows, (long long)cols);
  if (rows == 0 || cols == 0) return POM_OK;
  if (!src || !dst) return fail(POM_ERR_INVALID, "src and dst must be non-null");
  if (ld_src < cols) return fail(POM_ERR_INVALID, "ld_src (%lld) < cols (%lld)", (long long)ld_src, (long long)cols);
  if (ld_dst < rows) return fail(POM_ERR_INVALID, "ld_dst (%lld) < rows (%lld)", (long long)ld_dst, (long long)rows);
  const int eb = elem_bytes(dtype);
  if (!aligned(src, eb) || !aligned(dst, eb)) return fail(POM_ERR_INVALID, "src and dst must be element-aligned");
  const hipStream_t st = static_cast<hipStream_t>(stream);
  return hip_status(pom::transpose_t(eb, src, ld_src, dst, ld_dst, rows, cols, st), "pom_transpose launch");
}

}  // extern "C"

// ---------------------------------------------------------------------------
// Projection GEMM
// ---------------------------------------------------------------------------

namespace {

constexpr int kGemmMaxSplits = 8;

struct GemmCost {
  double us = 1e30;
  int tile = -1, splits = 1;
};

// Modelled time of one (tile, splits) choice: whole rounds of 256 workgroups
// (one per CU) of the per-workgroup time, plus the fixed-order reduction of
// the fp32 partials when split.  Smaller tiles run the matrix cores less
// efficiently (more LDS and L2 traffic per flop); a partial edge tile costs a
// whole one.
double gemm_model_us(int64_t M, int64_t N, int64_t K, int tile, int splits) {
  int bm, bn;
  pom::gemm_tile_dims(tile, &bm, &bn);
  static const double tile_rate[pom::GEMM_TILE_COUNT] = {1.0, 0.97, 0.97, 0.88, 0.88, 0.7};
  const int64_t units = cdiv(M, bm) * cdiv(N, bn) * splits;
  const int64_t rounds = cdiv(units, 256);
  const double cu_flops = 4.0 * 1024 * 2.1e9 * 0.7 * tile_rate[tile];   // per CU per second
  const double wg_us = 2.0 * bm * bn * ((double)K / splits) / cu_flops * 1e6
                       + 1.5 + (double)bm * bn * (splits > 1 ? 4 : 2) / 120e9 * 1e6;
  double us = rounds * wg_us;
  if (splits > 1) us += 3.0 + ((double)splits * 4 + 2) * M * N / 4.5e12 * 1e6;
  return us;
}

// Every tile takes any M, N that are multiples of 8 (the kernel masks the
// partial edge tiles); 8-element groups keep the reductions' vector accesses
// inside a row.  POM_AMD_GEMM_PARTIAL_TILES=0 (read once) admits only tiles
// that divide M and N.
bool gemm_tile_fits(int64_t M, int64_t N, int tile) {
  static const bool partial = [] {
    const char* e = getenv("POM_AMD_GEMM_PARTIAL_TILES");
    return !(e && e[0] == '0');
  }();
  if (tile < 0 || tile >= pom::GEMM_TILE_COUNT || M % 8 || N % 8) return false;
  if (partial) return true;
  int bm, bn;
  pom::gemm_tile_dims(tile, &bm, &bn);
  return M % bm == 0 && N % bn == 0;
}

size_t gemm_ws_bytes(int64_t M, int64_t N, int tile, int splits) {
  if (splits == pom::GEMM_STREAM_K) {
    int bm, bn;
    pom::gemm_tile_dims(tile, &bm, &bn);
    return pom::gemm_streamk_ws_bytes(M, N, bm, bn);
  }
  return splits > 1 ? (size_t)splits * (size_t)M * (size_t)N * 4 : 0;
}

// stream-K needs at least one 64-step per workgroup
bool gemm_streamk_fits(int64_t M, int64_t N, int64_t K, int tile) {
  int bm, bn;
  pom::gemm_tile_dims(tile, &bm, &bn);
  return cdiv(M, bm) * cdiv(N, bn) * (K / 64) >= pom::kStreamKGroups;
}

// Measured best (tile, splits) for the weight-gradient products of the baseline configurations
// (M/N-contiguous operands; MI355X, isolated runs over every tile and 1-8 splits, then stream-K
// against that choice inside the layer's backward, same box, alternating).  Stream-K's workgroups
// start at different k offsets, so the CUs of one XCD no longer read the same operand slices
// together, and the L2 reuse of the lockstep split-K grid is lost.  In the layer that costs more
// than the idle CUs it fills everywhere but config 4's dW_qc (882-887 us against 908-912); e.g.
// config 5's dW_qc 677-681 against 609-612, config 2 isolated 236 against 202.
// dW_ag runs on pom_layer_bwd's second stream beside the data-gradient chain, where fewer splits than the
// isolated best leave compute units to that chain and write fewer fp32 partials.  Its split counts were chosen
// inside the layer's backward (same box, three alternating rounds).  Config 2: 2 splits, 0.930-0.932 ms per step
// against 0.942-0.945 with 4 (0.681-0.683 against 0.707-0.715 with 16 gate heads; 1 split 0.99).  Config 3: 4
// against 8, 2.331-2.337 against 2.358-2.361.  Config 4: 2 against 4, 4.604-4.615 against 4.649-4.666.  Config
// 5: 2 against 7, 2.605-2.614 against 2.627-2.636 (4 and 3 were mixed).  Config 2's other shapes measured slower
// (3 splits, the 256 x 192 tile with 2, the 128 x 128 tile unsplit).
// sk_tile >= 0: stream-K on that tile, unless POM_AMD_GEMM_STREAMK=0 asks for (tile, splits).
struct GemmTuned {
  int64_t M, N, K;
  int a_layout, b_layout, tile, splits, sk_tile;
};
const GemmTuned kGemmTuned[] = {
    {1152, 2304, 16384, 1, 1, 2, 2, -1},  // config 2: dW_ag = g^T sh
    {4608, 1152, 16384, 1, 1, 1, 2, -1},  // config 2: dW_qc = dY^T x
    {2368, 1152, 16384, 1, 1, 1, 4, -1},  // config 2 with 16 gate heads: dW_qc (10 row tiles, the last partial)
    {1024, 2048, 65536, 1, 1, 0, 4, -1},  // config 3
    {4096, 1024, 65536, 1, 1, 0, 4, -1},
    {1024, 4096, 65536, 1, 1, 0, 2, -1},  // config 4
    {8192, 1024, 65536, 1, 1, 0, 4, 0},
    {1536, 3072, 32768, 1, 1, 0, 2, -1},  // config 5
    {6144, 1536, 32768, 1, 1, 0, 3, -1},
};

bool streamk_allowed() {
  static const bool on = [] {
    const char* e = getenv("POM_AMD_GEMM_STREAMK");
    return !(e && e[0] == '0');
  }();
  return on;
}

// POM_AMD_GEMM_FORCE="tile,splits" pins the choice (tile sweeps); then the measured table; then the
// cost model.
GemmCost gemm_choose(int64_t M, int64_t N, int64_t K, int a_layout, int b_layout) {
  GemmCost best;
  static const char* force = getenv("POM_AMD_GEMM_FORCE");
  if (force) {
    int t = -1, sp = 1;
    if (sscanf(force, "%d,%d", &t, &sp) == 2 && t >= 0 && t < pom::GEMM_TILE_COUNT && gemm_tile_fits(M, N, t) &&
        ((sp >= 1 && sp <= kGemmMaxSplits && K / 64 >= sp) ||
         (sp == pom::GEMM_STREAM_K && gemm_streamk_fits(M, N, K, t)))) {
      best.tile = t;
      best.splits = sp;
      best.us = 0;
      return best;
    }
  }
  for (const GemmTuned& e : kGemmTuned) {
    if (e.M == M && e.N == N && e.K == K && e.a_layout == a_layout && e.b_layout == b_layout) {
      const bool sk = e.sk_tile >= 0 && streamk_allowed();
      best.tile = sk ? e.sk_tile : e.tile;
      best.splits = sk ? pom::GEMM_STREAM_K : e.splits;
      best.us = 0;
      return best;
    }
  }
  for (int t = 0; t < pom::GEMM_TILE_COUNT; ++t) {
    if (!gemm_tile_fits(M, N, t)) continue;
    for (int sp = 1; sp <= kGemmMaxSplits; ++sp) {
      if (K / 64 < 8 * sp) break;
      const double us = gemm_model_us(M, N, K, t, sp);
      if (us < best.us) best = {us, t, sp};
    }
  }
  return best;
}

}  // namespace

extern "C" {

int pom_gemm_plan(int64_t M, int64_t N, int64_t K, int a_layout, int b_layout, int* tile, int* splits) {
  if (M <= 0 || N <= 0 || K <= 0 || K % 64) return fail(POM_ERR_UNSUPPORTED, "gemm: K (%lld) must be a positive multiple of 64", (long long)K);
  const GemmCost c = gemm_choose(M, N, K, a_layout, b_layout);
  if (c.tile < 0)
    return fail(POM_ERR_UNSUPPORTED, "gemm: M=%lld and N=%lld must be multiples of 8", (long long)M, (long long)N);
  if (tile) *tile = c.tile;
  if (splits) *splits = c.splits;
  return POM_OK;
}

size_t pom_gemm_workspace_size(int64_t M, int64_t N, int64_t K, int tile, int splits) {
  if (tile < 0 || splits <= 0) {   // the largest need over both layouts' plans
    size_t need = 0;
    for (int al = 0; al < 2; ++al)
      for (int bl = 0; bl < 2; ++bl) {
        int t = -1, sp = 1;
        if (pom_gemm_plan(M, N, K, al, bl, &t, &sp) != POM_OK) return 0;
        const size_t b = gemm_ws_bytes(M, N, t, splits <= 0 ? sp : splits);
        need = b > need ? b : need;
      }
    return need;
  }
  if (tile >= pom::GEMM_TILE_COUNT) return 0;
  return gemm_ws_bytes(M, N, tile, splits);
}

int pom_gemm(int a_layout, int b_layout, int64_t M, int64_t N, int64_t K, const void* A, int64_t lda,
             const void* B, int64_t ldb, int out_dtype, void* C, int64_t ldc, int tile, int splits,
             void* workspace, size_t workspace_bytes, void* stream) {
  if ((a_layout != POM_GEMM_K_CONTIG && a_layout != POM_GEMM_MN_CONTIG) ||
      (b_layout != POM_GEMM_K_CONTIG && b_layout != POM_GEMM_MN_CONTIG))
    return fail(POM_ERR_INVALID, "gemm: layouts must be POM_GEMM_K_CONTIG or POM_GEMM_MN_CONTIG");
  if (out_dtype != POM_DTYPE_BF16 && out_dtype != POM_DTYPE_F32)
    return fail(POM_ERR_UNSUPPORTED, "gemm: out_dtype must be bf16 or f32");
  if (M < 0 || N < 0 || K < 0) return fail(POM_ERR_INVALID, "gemm: negative size");
  if (M == 0 || N == 0) return POM_OK;
  if (K == 0 || K % 64) return fail(POM_ERR_UNSUPPORTED, "gemm: K (%lld) must be a positive multiple of 64", (long long)K);
  if (!A || !B || !C) return fail(POM_ERR_INVALID, "gemm: null operand");
  const bool amn = a_layout == POM_GEMM_MN_CONTIG, bmn = b_layout == POM_GEMM_MN_CONTIG;
  if (lda < (amn ? M : K) || ldb < (bmn ? N : K) || ldc < N)
    return fail(POM_ERR_INVALID, "gemm: leading dimension too small (lda %lld, ldb %lld, ldc %lld)", (long long)lda,
                (long long)ldb, (long long)ldc);
  if (!aligned(A, 16) || !aligned(B, 16) || !aligned(C, 16) || lda % 8 || ldb % 8 ||
      ldc % (out_dtype == POM_DTYPE_F32 ? 4 : 8))
    return fail(POM_ERR_UNSUPPORTED, "gemm: operands and leading dimensions must be 16-byte aligned");
  if (tile < 0 || splits <= 0) {
    const GemmCost c = gemm_choose(M, N, K, a_layout, b_layout);
    if (tile < 0) tile = c.tile;
    if (splits <= 0) splits = c.splits;
  }
  if (tile < 0 || tile >= pom::GEMM_TILE_COUNT || !gemm_tile_fits(M, N, tile))
    return fail(POM_ERR_UNSUPPORTED, "gemm: tile %d with M=%lld, N=%lld (tile ids 0-5; M and N multiples of 8)", tile,
                (long long)M, (long long)N);
  if (splits == pom::GEMM_STREAM_K) {
    if (!gemm_streamk_fits(M, N, K, tile))
      return fail(POM_ERR_UNSUPPORTED, "gemm: stream-K needs tiles x K / 64 >= %d", pom::kStreamKGroups);
  } else if (splits > kGemmMaxSplits || splits > K / 64) {
    return fail(POM_ERR_UNSUPPORTED, "gemm: splits (%d) must be <= %d and <= K / 64, or POM_GEMM_STREAM_K", splits,
                kGemmMaxSplits);
  }
  if (M * N > ((int64_t)1 << 31) || M > INT32_MAX || N > INT32_MAX || K / 64 > INT32_MAX)
    return fail(POM_ERR_UNSUPPORTED, "gemm: output too large");
  const size_t need = gemm_ws_bytes(M, N, tile, splits);
  if (need && (!workspace || workspace_bytes < need || !aligned(workspace, 16)))
    return fail(POM_ERR_WORKSPACE, "gemm: workspace of %zu bytes (16-byte aligned) needed, got %zu", need,
                workspace ? workspace_bytes : (size_t)0);
  pom::GemmProblem p;
  p.A = A;
  p.B = B;
  p.C = C;
  p.workspace = workspace;
  p.lda = lda;
  p.ldb = ldb;
  p.ldc = ldc;
  p.M = M;
  p.N = N;
  p.K = K;
  p.a_mn = amn;
  p.b_mn = bmn;
  p.out_f32 = out_dtype == POM_DTYPE_F32;
  p.tile = tile;
  p.splits = splits;
  return hip_status(pom::gemm_bf16(p, static_cast<hipStream_t>(stream)), "pom_gemm launch");
}

}  // extern "C"
