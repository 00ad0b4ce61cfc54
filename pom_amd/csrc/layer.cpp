// Library GEMMs of the layer's projections, called from C++ (pom_blas_*).
//
// Every projection product of the fused layer has both operands contiguous
// along the reduction dimension: A (m, k) and B (n, k) row-major with unit k
// stride, and writes C (n, m) row-major.  In BLAS's column-major terms that is
// C = op(A) op(B) with op(A) = A^T (transa = T), op(B) = B (transb = N).
//
// The kernel for each shape comes from the offline-tuned table that also
// drives torch's GEMMs (pom_amd/tuned/gemm_gfx950.csv, read by torch's
// TunableOp): a rocBLAS or a hipBLASLt solution index, registered here by the
// Python layer (pom_blas_set_solution).  The calls below are the ones
// TunableOp makes for such an entry -- bf16 operands and output, fp32 compute
// and scale, alpha = 1, beta = 0, C also the output -- so a product run here
// and the same product run through torch.mm execute the same kernel.  A shape
// without an entry is refused (POM_ERR_UNSUPPORTED): there is no heuristic
// fallback, so the caller knows which kernel runs.
//
// The library instances are the ones the process has loaded: with torch
// imported first these are torch's own copies, whose solution indices the
// table records (pom_blas_library reports the file each symbol resolves to).
#include <hip/hip_runtime.h>
#include <hipblaslt/hipblaslt-ext.hpp>
#include <hipblaslt/hipblaslt.h>
#include <rocblas/rocblas.h>

#include <dlfcn.h>

#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <unordered_map>
#include <vector>

#include "../../include/pom_amd.h"
#include "pom_internal.h"

namespace {

constexpr int kMaxDevices = 64;

struct Shape {
  int64_t m, n, k, lda, ldb, ldc;
  bool operator==(const Shape& o) const {
    return m == o.m && n == o.n && k == o.k && lda == o.lda && ldb == o.ldb && ldc == o.ldc;
  }
};
struct ShapeHash {
  size_t operator()(const Shape& s) const {
    size_t h = 1469598103934665603ull;
    for (int64_t v : {s.m, s.n, s.k, s.lda, s.ldb, s.ldc}) h = (h ^ (size_t)v) * 1099511628211ull;
    return h;
  }
};

struct Solution {
  int lib;     // POM_BLAS_ROCBLAS or POM_BLAS_HIPBLASLT
  int index;   // the library's solution index
};

// hipBLASLt descriptors and algorithm of one registered shape on one device
struct LtPlan {
  hipblasLtMatmulDesc_t desc = nullptr;
  hipblasLtMatrixLayout_t a = nullptr, b = nullptr, c = nullptr;
  hipblasLtMatmulAlgo_t algo{};
  size_t workspace = 0;
};

struct DeviceBlas {
  rocblas_handle rb = nullptr;
  hipblasLtHandle_t lt = nullptr;
  std::unordered_map<Shape, LtPlan, ShapeHash> plans;
};

std::mutex g_mu;   // the table and the per-device handles (a handle's stream is set per call)
std::unordered_map<Shape, Solution, ShapeHash> g_table;
DeviceBlas g_dev[kMaxDevices];

int err(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int err(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  return pom::set_error(code, buf);
}

int current_device(int& dev) {
  if (hipGetDevice(&dev) != hipSuccess) return err(POM_ERR_DEVICE, "pom_blas: no current device");
  if (dev < 0 || dev >= kMaxDevices) return err(POM_ERR_UNSUPPORTED, "pom_blas: device %d", dev);
  return POM_OK;
}

// hipBLASLt plan for shape s: descriptors as TunableOp builds them and the
// algorithm of solution `index`, checked against the problem.
int make_lt_plan(DeviceBlas& d, const Shape& s, int index, LtPlan& p) {
  if (!d.lt && hipblasLtCreate(&d.lt) != HIPBLAS_STATUS_SUCCESS)
    return err(POM_ERR_DEVICE, "pom_blas: hipblasLtCreate failed");
  const hipblasOperation_t ta = HIPBLAS_OP_T, tb = HIPBLAS_OP_N;
  if (hipblasLtMatmulDescCreate(&p.desc, HIPBLAS_COMPUTE_32F, HIP_R_32F) != HIPBLAS_STATUS_SUCCESS ||
      hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSA, &ta, sizeof(ta)) != HIPBLAS_STATUS_SUCCESS ||
      hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSB, &tb, sizeof(tb)) != HIPBLAS_STATUS_SUCCESS ||
      hipblasLtMatrixLayoutCreate(&p.a, HIP_R_16BF, s.k, s.m, s.lda) != HIPBLAS_STATUS_SUCCESS ||
      hipblasLtMatrixLayoutCreate(&p.b, HIP_R_16BF, s.k, s.n, s.ldb) != HIPBLAS_STATUS_SUCCESS ||
      hipblasLtMatrixLayoutCreate(&p.c, HIP_R_16BF, s.m, s.n, s.ldc) != HIPBLAS_STATUS_SUCCESS)
    return err(POM_ERR_DEVICE, "pom_blas: hipBLASLt descriptor creation failed");
  std::vector<int> idx{index};
  std::vector<hipblasLtMatmulHeuristicResult_t> res;
  if (hipblaslt_ext::getAlgosFromIndex(d.lt, idx, res) != HIPBLAS_STATUS_SUCCESS || res.empty())
    return err(POM_ERR_UNSUPPORTED, "pom_blas: hipBLASLt has no solution %d", index);
  p.algo = res[0].algo;
  const float alpha = 1.0f, beta = 0.0f;
  if (hipblaslt_ext::matmulIsAlgoSupported(d.lt, p.desc, &alpha, p.a, p.b, &beta, p.c, p.c, p.algo, p.workspace) !=
      HIPBLAS_STATUS_SUCCESS)
    return err(POM_ERR_UNSUPPORTED, "pom_blas: hipBLASLt solution %d does not support m=%lld n=%lld k=%lld", index,
               (long long)s.m, (long long)s.n, (long long)s.k);
  return POM_OK;
}

void free_lt_plan(LtPlan& p) {
  if (p.a) hipblasLtMatrixLayoutDestroy(p.a);
  if (p.b) hipblasLtMatrixLayoutDestroy(p.b);
  if (p.c) hipblasLtMatrixLayoutDestroy(p.c);
  if (p.desc) hipblasLtMatmulDescDestroy(p.desc);
  p = LtPlan{};
}

// The file a loaded symbol resolves to, or "" when none does.
const char* symbol_file(const void* sym) {
  Dl_info info;
  if (sym && dladdr(sym, &info) && info.dli_fname) return info.dli_fname;
  return "";
}

}  // namespace

namespace pom {

// C (n, m), row stride ldc = A (m, k) . B (n, k)^T, bf16, with the registered
// solution of this shape; on `st`.
int blas_gemm_tn(int64_t m, int64_t n, int64_t k, const void* A, int64_t lda, const void* B, int64_t ldb, void* C,
                 int64_t ldc, void* workspace, size_t workspace_bytes, hipStream_t st) {
  const Shape s{m, n, k, lda, ldb, ldc};
  std::lock_guard<std::mutex> lock(g_mu);
  auto it = g_table.find(s);
  if (it == g_table.end())
    return err(POM_ERR_UNSUPPORTED,
               "pom_blas: no solution registered for m=%lld n=%lld k=%lld lda=%lld ldb=%lld ldc=%lld",
               (long long)m, (long long)n, (long long)k, (long long)lda, (long long)ldb, (long long)ldc);
  int dev;
  if (int r = current_device(dev)) return r;
  DeviceBlas& d = g_dev[dev];
  const float alpha = 1.0f, beta = 0.0f;
  if (it->second.lib == POM_BLAS_ROCBLAS) {
    if (!d.rb && rocblas_create_handle(&d.rb) != rocblas_status_success)
      return err(POM_ERR_DEVICE, "pom_blas: rocblas_create_handle failed");
    if (rocblas_set_stream(d.rb, st) != rocblas_status_success)
      return err(POM_ERR_DEVICE, "pom_blas: rocblas_set_stream failed");
    const rocblas_status r = rocblas_gemm_ex(
        d.rb, rocblas_operation_transpose, rocblas_operation_none, (rocblas_int)m, (rocblas_int)n, (rocblas_int)k,
        &alpha, A, rocblas_datatype_bf16_r, (rocblas_int)lda, B, rocblas_datatype_bf16_r, (rocblas_int)ldb, &beta, C,
        rocblas_datatype_bf16_r, (rocblas_int)ldc, C, rocblas_datatype_bf16_r, (rocblas_int)ldc,
        rocblas_datatype_f32_r, rocblas_gemm_algo_solution_index, it->second.index, rocblas_gemm_flags_none);
    if (r != rocblas_status_success)
      return err(POM_ERR_DEVICE, "pom_blas: rocblas_gemm_ex (solution %d) failed with status %d", it->second.index,
                 (int)r);
    return POM_OK;
  }
  auto pit = d.plans.find(s);
  if (pit == d.plans.end()) {
    LtPlan p;
    if (int r = make_lt_plan(d, s, it->second.index, p)) {
      free_lt_plan(p);
      return r;
    }
    pit = d.plans.emplace(s, p).first;
  }
  const LtPlan& p = pit->second;
  if (p.workspace > workspace_bytes || (p.workspace && !workspace))
    return err(POM_ERR_WORKSPACE, "pom_blas: hipBLASLt solution %d needs %zu bytes of workspace, got %zu",
               it->second.index, p.workspace, workspace_bytes);
  if (hipblasLtMatmul(d.lt, p.desc, &alpha, A, p.a, B, p.b, &beta, C, p.c, C, p.c, &p.algo, workspace,
                      workspace_bytes, st) != HIPBLAS_STATUS_SUCCESS)
    return err(POM_ERR_DEVICE, "pom_blas: hipblasLtMatmul (solution %d) failed", it->second.index);
  return POM_OK;
}

}  // namespace pom

extern "C" {

int pom_blas_set_solution(int64_t m, int64_t n, int64_t k, int64_t lda, int64_t ldb, int64_t ldc, int lib,
                          int index) {
  if (m <= 0 || n <= 0 || k <= 0 || lda < k || ldb < k || ldc < m)
    return err(POM_ERR_INVALID, "pom_blas_set_solution: bad shape m=%lld n=%lld k=%lld lda=%lld ldb=%lld ldc=%lld",
               (long long)m, (long long)n, (long long)k, (long long)lda, (long long)ldb, (long long)ldc);
  if (lib != POM_BLAS_ROCBLAS && lib != POM_BLAS_HIPBLASLT)
    return err(POM_ERR_INVALID, "pom_blas_set_solution: unknown library %d", lib);
  if (m > 0x7fffffff || n > 0x7fffffff || k > 0x7fffffff || lda > 0x7fffffff || ldb > 0x7fffffff ||
      ldc > 0x7fffffff)
    return err(POM_ERR_UNSUPPORTED, "pom_blas_set_solution: dimensions beyond 32 bits");
  const Shape s{m, n, k, lda, ldb, ldc};
  std::lock_guard<std::mutex> lock(g_mu);
  g_table[s] = Solution{lib, index};
  for (DeviceBlas& d : g_dev) {   // a re-registered shape rebuilds its hipBLASLt plan
    auto it = d.plans.find(s);
    if (it != d.plans.end()) {
      free_lt_plan(it->second);
      d.plans.erase(it);
    }
  }
  return POM_OK;
}

int pom_blas_has_solution(int64_t m, int64_t n, int64_t k, int64_t lda, int64_t ldb, int64_t ldc) {
  std::lock_guard<std::mutex> lock(g_mu);
  return g_table.count(Shape{m, n, k, lda, ldb, ldc}) ? 1 : 0;
}

int pom_blas_gemm(int64_t m, int64_t n, int64_t k, const void* A, int64_t lda, const void* B, int64_t ldb, void* C,
                  int64_t ldc, void* workspace, size_t workspace_bytes, void* stream) {
  if (!A || !B || !C) return err(POM_ERR_INVALID, "pom_blas_gemm: null operand");
  return pom::blas_gemm_tn(m, n, k, A, lda, B, ldb, C, ldc, workspace, workspace_bytes,
                           static_cast<hipStream_t>(stream));
}

const char* pom_blas_library(int lib) {
  if (lib == POM_BLAS_ROCBLAS) return symbol_file(reinterpret_cast<const void*>(&rocblas_gemm_ex));
  if (lib == POM_BLAS_HIPBLASLT) return symbol_file(reinterpret_cast<const void*>(&hipblasLtMatmul));
  return "";
}

}  // extern "C"

// ===========================================================================
// The fused layer's launch sequence (pom_layer_fwd / pom_layer_bwd)
//
// The order and the operands are those of the Python operator's bf16
// training path (pom_amd/ops.py _PoMLayer): each projection on
// K-contiguous operands through pom_blas_gemm (the kernel the tuned table
// names), each weight gradient on pom_gemm when a tile divides it (else on
// the library with token-contiguous copies made by the transpose kernel),
// and the aggregation and gating through their own entry points.  Every
// launch goes to one stream, so one workspace serves each step in turn.
// ===========================================================================
#include <hip/hip_bf16.h>
#include <hip/hip_fp16.h>

namespace {

constexpr size_t kBlasWorkspace = size_t(64) << 20;   // hipBLASLt solutions' workspace
constexpr int kThreadsL = 256;

__device__ __forceinline__ float load_param(const void* p, int dt, int64_t i) {
  if (dt == POM_DTYPE_BF16) return __bfloat162float(static_cast<const __hip_bfloat16*>(p)[i]);
  if (dt == POM_DTYPE_F16) return __half2float(static_cast<const __half*>(p)[i]);
  return static_cast<const float*>(p)[i];
}

// out[r, c] = bf16(out[r, c] + bf16(bias[c])): torch's out + b_ag.to(bf16)
__global__ void __launch_bounds__(kThreadsL) add_bias_rows(__hip_bfloat16* out, int64_t rows, int64_t cols,
                                                           const void* bias, int bdt) {
  const int64_t n = rows * cols;
  for (int64_t i = (int64_t)blockIdx.x * kThreadsL + threadIdx.x; i < n; i += (int64_t)gridDim.x * kThreadsL) {
    const int64_t c = i % cols;
    const float b = __bfloat162float(__float2bfloat16(load_param(bias, bdt, c)));
    out[i] = __float2bfloat16(__bfloat162float(out[i]) + b);
  }
}

// part[chunk, c] = sum over rows [chunk * rc, ...) of g[r, c] in fp32, rows in order
__global__ void __launch_bounds__(kThreadsL) col_sum_part(const __hip_bfloat16* g, int64_t rows, int64_t cols,
                                                          int64_t rc, float* part) {
  const int64_t c = (int64_t)blockIdx.x * kThreadsL + threadIdx.x;
  if (c >= cols) return;
  const int64_t r0 = (int64_t)blockIdx.y * rc;
  const int64_t r1 = r0 + rc < rows ? r0 + rc : rows;
  float s = 0.0f;
  for (int64_t r = r0; r < r1; ++r) s += __bfloat162float(g[r * cols + c]);
  part[blockIdx.y * cols + c] = s;
}

// out[c] = sum over chunks of part[chunk, c], chunks in order
__global__ void __launch_bounds__(kThreadsL) col_sum_final(const float* part, int64_t nchunks, int64_t cols,
                                                           float* out) {
  const int64_t c = (int64_t)blockIdx.x * kThreadsL + threadIdx.x;
  if (c >= cols) return;
  float s = 0.0f;
  for (int64_t k = 0; k < nchunks; ++k) s += part[k * cols + c];
  out[c] = s;
}

// a[i] += b[i] (fp32)
__global__ void __launch_bounds__(kThreadsL) add_f32(float* a, const float* b, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * kThreadsL + threadIdx.x; i < n; i += (int64_t)gridDim.x * kThreadsL)
    a[i] += b[i];
}

// y[r, c0 .. c0 + w) = 0 for every row (row stride ld)
__global__ void __launch_bounds__(kThreadsL) zero_cols(__hip_bfloat16* y, int64_t rows, int64_t ld, int64_t c0,
                                                       int64_t w) {
  const int64_t n = rows * w;
  for (int64_t i = (int64_t)blockIdx.x * kThreadsL + threadIdx.x; i < n; i += (int64_t)gridDim.x * kThreadsL)
    y[(i / w) * ld + c0 + i % w] = __float2bfloat16(0.0f);
}

dim3 grid_for(int64_t n) {
  int64_t b = (n + kThreadsL - 1) / kThreadsL;
  return dim3((unsigned)(b < 65536 ? (b > 0 ? b : 1) : 65536));
}

int launched(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return err(POM_ERR_DEVICE, "pom_layer: %s launch: %s", what, hipGetErrorString(e));
  return POM_OK;
}

// the weight gradient C (M x N) = A^T B over T tokens, A (T x M) and B (T x N)
// token-major: pom_gemm's plan when a tile divides (M, N)
bool wgrad_fits(int64_t M, int64_t N, int64_t T) {
  int tile = -1, splits = 0;
  return pom_gemm_plan(M, N, T, POM_GEMM_MN_CONTIG, POM_GEMM_MN_CONTIG, &tile, &splits) == POM_OK;
}

size_t wgrad_ws(int64_t M, int64_t N, int64_t T) {
  int tile = -1, splits = 0;
  if (pom_gemm_plan(M, N, T, POM_GEMM_MN_CONTIG, POM_GEMM_MN_CONTIG, &tile, &splits) != POM_OK) return 0;
  return pom_gemm_workspace_size(M, N, T, tile, splits);
}

int64_t groups_of(const pom_layer_args* a) { return a->N / a->frame_len; }

size_t align256(size_t v) { return (v + 255) / 256 * 256; }

// Workspace regions, used by launches that may run at the same time on two
// streams: [library GEMMs | dW_ag split partials | dW_qc split partials |
// aggregation / gating / bias-gradient partials].
struct Regions {
  size_t wa_off = 0, wq_off = 0, rest_off = 0, total = 0;
};

// POM_AMD_LAYER_OVERLAP (read at every backward call, a few hundred ns): bit 1
// runs dW_qc on a second stream beside dx (both only read dY), bit 2 runs dW_ag
// there beside the data-gradient chain (it only reads g and sh); 0: one
// stream.  Default 2 (dW_ag beside the chain: C2 -2.4 %, c2h -3 %, C3-C5 the
// same or better).  A stream being captured into a graph keeps one stream.
int overlap_mode(hipStream_t st) {
  const char* s = getenv("POM_AMD_LAYER_OVERLAP");
  const int mode = s ? atoi(s) & 3 : 2;
  if (!mode) return 0;
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(st, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone) return 0;
  return mode;
}

// a second stream (default priority) and two events per device, made once
// The second stream of a device and its two events, shared by every caller on that device.  A stream wait binds to
// the event's latest record when the wait is issued, so each record + wait pair runs under `mu`: another thread
// re-recording the event between the two would otherwise make this caller wait for that thread's stream instead.
struct Side {
  hipStream_t stream = nullptr;
  hipEvent_t fork = nullptr, join = nullptr;
  std::mutex mu;
};
std::mutex g_side_mu;
Side g_side[kMaxDevices];

int side_of(Side*& out) {
  int dev;
  if (int r = current_device(dev)) return r;
  std::lock_guard<std::mutex> lock(g_side_mu);
  Side& s = g_side[dev];
  if (!s.stream) {   // published only when the stream and both events exist
    hipStream_t stream = nullptr;
    hipEvent_t fork = nullptr, join = nullptr;
    if (hipStreamCreateWithFlags(&stream, hipStreamNonBlocking) != hipSuccess ||
        hipEventCreateWithFlags(&fork, hipEventDisableTiming) != hipSuccess ||
        hipEventCreateWithFlags(&join, hipEventDisableTiming) != hipSuccess) {
      if (join) (void)hipEventDestroy(join);
      if (fork) (void)hipEventDestroy(fork);
      if (stream) (void)hipStreamDestroy(stream);
      return err(POM_ERR_DEVICE, "pom_layer: second stream creation failed");
    }
    s.fork = fork;
    s.join = join;
    s.stream = stream;
  }
  out = &s;
  return POM_OK;
}

// `to` waits for everything enqueued on `from` so far (ev is one of sd's events)
int wait_for(Side* sd, hipStream_t to, hipStream_t from, hipEvent_t ev) {
  std::lock_guard<std::mutex> lock(sd->mu);
  if (hipEventRecord(ev, from) != hipSuccess || hipStreamWaitEvent(to, ev, 0) != hipSuccess)
    return err(POM_ERR_DEVICE, "pom_layer: stream ordering failed");
  return POM_OK;
}

// every library product of the direction has a registered solution (checked
// before anything is launched)
int check_solutions(const pom_layer_args* a, bool backward) {
  const int64_t D = a->D, P = a->P, W = a->W, T = a->B * a->N;
  struct S6 { int64_t m, n, k; const char* what; bool used; };
  const S6 list[] = {
      {W, T, D, "qc_proj", !backward},
      {D, T, P, "ag_proj", !backward},
      {P, T, D, "ag_proj data gradient", backward},
      {D, T, W, "qc_proj data gradient", backward && a->dx != nullptr},
      {P, D, T, "ag_proj weight gradient", backward && a->dwa != nullptr && !wgrad_fits(D, P, T)},
      {D, W, T, "qc_proj weight gradient", backward && a->dwq != nullptr && !wgrad_fits(W, D, T)},
  };
  for (const S6& s : list)
    if (s.used && !pom_blas_has_solution(s.m, s.n, s.k, s.k, s.k, s.m))
      return err(POM_ERR_UNSUPPORTED, "pom_layer: no library solution registered for the %s (m=%lld n=%lld k=%lld)",
                 s.what, (long long)s.m, (long long)s.n, (long long)s.k);
  return POM_OK;
}

int rope_kind(const pom_rope* r) { return r ? r->kind : POM_ROPE_NONE; }

int check_args(const pom_layer_args* a) {
  if (!a) return err(POM_ERR_INVALID, "pom_layer: null arguments");
  if (a->B <= 0 || a->N <= 0 || a->D <= 0 || a->P <= 0 || a->S <= 0 || a->W < a->P + a->S || a->K < 1)
    return err(POM_ERR_INVALID, "pom_layer: bad shape B=%lld N=%lld D=%lld P=%lld S=%lld W=%lld K=%d",
               (long long)a->B, (long long)a->N, (long long)a->D, (long long)a->P, (long long)a->S,
               (long long)a->W, a->K);
  if (a->heads > 1 ? a->S != a->heads : a->S != a->P)
    return err(POM_ERR_INVALID, "pom_layer: gate width %lld for heads %lld", (long long)a->S, (long long)a->heads);
  if (a->frame_len <= 0 || a->N % a->frame_len) return err(POM_ERR_INVALID, "pom_layer: frame_len must divide N");
  if (!a->wq || !a->wa || !a->coeff || !a->y || !a->hagg)
    return err(POM_ERR_INVALID, "pom_layer: null weight, coefficient or activation");
  return POM_OK;
}

Regions layer_regions(const pom_layer_args* a, int backward) {
  const int64_t T = a->B * a->N, G = groups_of(a);
  size_t wa = 0, wq = 0, rest = 0;
  auto upd = [](size_t& m, size_t v) { m = v > m ? v : m; };
  upd(rest, pom_agg_workspace_size(POM_DTYPE_BF16, a->B, a->N, a->P, a->K, a->frame_len, rope_kind(a->rope_h),
                                   backward));
  if (a->heads > 1) upd(rest, pom_gate_heads_workspace_size(POM_DTYPE_BF16, a->B, a->N, a->P, a->heads, G));
  else upd(rest, pom_gate_workspace_size(POM_DTYPE_BF16, a->B, a->N, a->P, G, rope_kind(a->rope_s)));
  if (backward) {
    wa = wgrad_ws(a->D, a->P, T);
    wq = wgrad_ws(a->W, a->D, T);
    upd(rest, (size_t)((T + 31) / 32) * (size_t)a->D * sizeof(float));   // bias-gradient partials
  }
  Regions r;
  r.wa_off = kBlasWorkspace;
  r.wq_off = r.wa_off + align256(wa);
  r.rest_off = r.wq_off + align256(wq);
  r.total = r.rest_off + align256(rest > 0 ? rest : 256);
  return r;
}

}  // namespace

extern "C" {

size_t pom_layer_args_size(void) { return sizeof(pom_layer_args); }

size_t pom_layer_workspace_size(const pom_layer_args* a, int backward) {
  if (check_args(a)) return 0;
  return layer_regions(a, backward).total;
}

int pom_layer_fwd(const pom_layer_args* a, void* stream) {
  if (int r = check_args(a)) return r;
  if (!a->x || !a->sh || !a->out) return err(POM_ERR_INVALID, "pom_layer_fwd: null x, sh or out");
  if (int r = check_solutions(a, false)) return r;
  const hipStream_t st = static_cast<hipStream_t>(stream);
  const int64_t B = a->B, N = a->N, D = a->D, P = a->P, W = a->W, T = B * N, G = groups_of(a);
  const Regions rg = layer_regions(a, 0);
  if (!a->workspace || a->workspace_bytes < rg.total)
    return err(POM_ERR_WORKSPACE, "pom_layer_fwd: workspace of %zu bytes, need %zu", a->workspace_bytes, rg.total);
  void* ws = a->workspace;   // library GEMMs
  const size_t wsb = kBlasWorkspace;
  void* wr = static_cast<char*>(a->workspace) + rg.rest_off;   // aggregation and gating
  const size_t wrb = a->workspace_bytes - rg.rest_off;
  auto* y = static_cast<__hip_bfloat16*>(a->y);
  if (a->xt)
    if (int r = pom_transpose(POM_DTYPE_BF16, T, D, a->x, D, a->xt, T, stream)) return r;
  if (int r = pom::blas_gemm_tn(W, T, D, a->wq, D, a->x, D, a->y, W, ws, wsb, st)) return r;   // Y = x Wq^T
  const pom_view hv{a->y, N * W, W}, sv{y + P, N * W, W}, shv{a->sh, N * P, P};
  if (int r = pom_agg_fwd(POM_DTYPE_BF16, a->param_dtype, B, N, P, a->K, &hv, a->coeff, a->mask, a->mask_stride_b,
                          a->mask_stride_n, a->frame_len, a->carry, a->n_past, a->rope_h, a->hagg, a->count, wr,
                          wrb, stream))
    return r;
  const pom_tview tv{a->sht, T, N};
  const pom_tview* shtv = a->sht ? &tv : nullptr;
  if (a->heads > 1) {
    int r = pom_gate_heads_fwd(POM_DTYPE_BF16, a->param_dtype, B, N, P, a->heads, &sv, a->se_bias, a->hagg, G,
                               a->rope_s, &shv, shtv, stream);
    if (r == POM_ERR_UNSUPPORTED && shtv) {   // no fused copy for this shape: transpose after
      r = pom_gate_heads_fwd(POM_DTYPE_BF16, a->param_dtype, B, N, P, a->heads, &sv, a->se_bias, a->hagg, G,
                             a->rope_s, &shv, nullptr, stream);
      if (!r) r = pom_transpose(POM_DTYPE_BF16, T, P, a->sh, P, a->sht, T, stream);
    }
    if (r) return r;
  } else {
    int r = pom_gate_fwd(POM_DTYPE_BF16, a->param_dtype, B, N, P, &sv, a->se_bias, a->hagg, G, a->rope_s, &shv,
                         shtv, stream);
    if (r == POM_ERR_UNSUPPORTED && shtv) {
      r = pom_gate_fwd(POM_DTYPE_BF16, a->param_dtype, B, N, P, &sv, a->se_bias, a->hagg, G, a->rope_s, &shv,
                       nullptr, stream);
      if (!r) r = pom_transpose(POM_DTYPE_BF16, T, P, a->sh, P, a->sht, T, stream);
    }
    if (r) return r;
  }
  if (int r = pom::blas_gemm_tn(D, T, P, a->wa, P, a->sh, P, a->out, D, ws, wsb, st)) return r;   // out = sh Wa^T
  if (a->b_ag) {
    hipLaunchKernelGGL(add_bias_rows, grid_for(T * D), dim3(kThreadsL), 0, st, static_cast<__hip_bfloat16*>(a->out),
                       T, D, a->b_ag, a->bias_ag_dtype);
    if (int r = launched("bias")) return r;
  }
  return POM_OK;
}

int pom_layer_bwd(const pom_layer_args* a, void* stream) {
  if (int r = check_args(a)) return r;
  if (!a->g || !a->dsh || !a->dy || !a->dcoeff || !a->dh)
    return err(POM_ERR_INVALID, "pom_layer_bwd: null g, dsh, dy, dcoeff or dh");
  if (int r = check_solutions(a, true)) return r;
  const hipStream_t st = static_cast<hipStream_t>(stream);
  const int64_t B = a->B, N = a->N, D = a->D, P = a->P, S = a->S, W = a->W, T = B * N, G = groups_of(a);
  const Regions rg = layer_regions(a, 1);
  if (!a->workspace || a->workspace_bytes < rg.total)
    return err(POM_ERR_WORKSPACE, "pom_layer_bwd: workspace of %zu bytes, need %zu", a->workspace_bytes, rg.total);
  void* ws = a->workspace;   // library GEMMs
  const size_t wsb = kBlasWorkspace;
  void* wga = static_cast<char*>(a->workspace) + rg.wa_off;   // pom_gemm split partials of dW_ag
  const size_t wgab = rg.wq_off - rg.wa_off;
  void* wgq = static_cast<char*>(a->workspace) + rg.wq_off;   // and of dW_qc
  const size_t wgqb = rg.rest_off - rg.wq_off;
  void* wr = static_cast<char*>(a->workspace) + rg.rest_off;   // streaming kernels' partials
  const size_t wrb = a->workspace_bytes - rg.rest_off;
  // the weight gradients that may run on the second stream (pom_gemm only)
  const int ov = overlap_mode(st);
  const bool side_wa = (ov & 2) && a->dwa && wgrad_fits(D, P, T);
  const bool side_wq = (ov & 1) && a->dwq && wgrad_fits(W, D, T);
  Side* sd = nullptr;
  if (side_wa || side_wq)
    if (int r = side_of(sd)) return r;
  // once work is forked to the second stream, every return joins it back
  struct Join {
    Side* sd = nullptr;
    hipStream_t st;
    bool armed = false;
    ~Join() {
      if (armed) (void)wait_for(sd, st, sd->stream, sd->join);
    }
  } join{sd, st};
  auto* y = static_cast<__hip_bfloat16*>(a->y);
  auto* dy = static_cast<__hip_bfloat16*>(a->dy);
  if (!a->wa_t) return err(POM_ERR_INVALID, "pom_layer_bwd: null wa_t");
  // dW_ag = g^T sh, on the second stream beside the data-gradient chain
  if (side_wa) {
    if (int r = wait_for(sd, sd->stream, st, sd->fork)) return r;
    join.armed = true;
    if (int r = pom_gemm(POM_GEMM_MN_CONTIG, POM_GEMM_MN_CONTIG, D, P, T, a->g, D, a->sh, P, a->dwa_dtype, a->dwa, P,
                         -1, 0, wga, wgab, sd->stream))
      return r;
  }
  // dsh = g Wa
  if (int r = pom::blas_gemm_tn(P, T, D, a->wa_t, D, a->g, D, a->dsh, P, ws, wsb, st)) return r;
  // dW_ag = g^T sh
  if (a->dwa && !side_wa) {
    if (wgrad_fits(D, P, T)) {
      if (int r = pom_gemm(POM_GEMM_MN_CONTIG, POM_GEMM_MN_CONTIG, D, P, T, a->g, D, a->sh, P, a->dwa_dtype, a->dwa,
                           P, -1, 0, wga, wgab, stream))
        return r;
    } else {
      if (!a->gt || !a->sht || a->dwa_dtype != POM_DTYPE_BF16)
        return err(POM_ERR_INVALID, "pom_layer_bwd: dW_ag off pom_gemm needs gt, sht and a bf16 output");
      if (int r = pom_transpose(POM_DTYPE_BF16, T, D, a->g, D, a->gt, T, stream)) return r;
      if (int r = pom::blas_gemm_tn(P, D, T, a->sht, T, a->gt, T, a->dwa, P, ws, wsb, st)) return r;
    }
  }
  // db_ag = sum over tokens of g, in fp32
  if (a->db_ag) {
    const int64_t rc = 32, nch = (T + rc - 1) / rc;
    float* part = static_cast<float*>(wr);
    const dim3 gp((unsigned)((D + kThreadsL - 1) / kThreadsL), (unsigned)nch);
    hipLaunchKernelGGL(col_sum_part, gp, dim3(kThreadsL), 0, st, static_cast<const __hip_bfloat16*>(a->g), T, D, rc,
                       part);
    hipLaunchKernelGGL(col_sum_final, dim3((unsigned)((D + kThreadsL - 1) / kThreadsL)), dim3(kThreadsL), 0, st,
                       part, nch, D, a->db_ag);
    if (int r = launched("bias gradient")) return r;
  }
  if (W > P + S) {   // the padding columns of dY meet W_qc's zero rows in dx = dY W_qc
    hipLaunchKernelGGL(zero_cols, grid_for(T * (W - P - S)), dim3(kThreadsL), 0, st, dy, T, W, P + S, W - P - S);
    if (int r = launched("padding")) return r;
  }
  const pom_view sv{y + P, N * W, W}, dshv{a->dsh, N * P, P}, dysv{dy + P, N * W, W};
  if (a->heads > 1) {
    if (int r = pom_gate_heads_bwd(POM_DTYPE_BF16, a->param_dtype, B, N, P, a->heads, &sv, a->se_bias, a->hagg, G,
                                   a->rope_s, &dshv, &dysv, a->dh, a->dse_bias, wr, wrb, stream))
      return r;
    if (a->dyt)   // the gate rows of dY^T (with the padding rows)
      if (int r = pom_transpose(POM_DTYPE_BF16, T, W - P, dy + P, W, static_cast<__hip_bfloat16*>(a->dyt) + P * T, T,
                                stream))
        return r;
  } else {
    const pom_tview tv{a->dyt ? static_cast<__hip_bfloat16*>(a->dyt) + P * T : nullptr, T, N};
    int r = pom_gate_bwd(POM_DTYPE_BF16, a->param_dtype, B, N, P, &sv, a->se_bias, a->hagg, G, a->rope_s, &dshv,
                         &dysv, a->dyt ? &tv : nullptr, a->dh, a->dse_bias, wr, wrb, stream);
    if (r == POM_ERR_UNSUPPORTED && a->dyt) {
      r = pom_gate_bwd(POM_DTYPE_BF16, a->param_dtype, B, N, P, &sv, a->se_bias, a->hagg, G, a->rope_s, &dshv,
                       &dysv, nullptr, a->dh, a->dse_bias, wr, wrb, stream);
      if (!r) r = pom_transpose(POM_DTYPE_BF16, T, S, dy + P, W, static_cast<__hip_bfloat16*>(a->dyt) + P * T, T,
                                stream);
    }
    if (r) return r;
  }
  if (a->grad_hagg) {
    hipLaunchKernelGGL(add_f32, grid_for(B * G * P), dim3(kThreadsL), 0, st, a->dh, a->grad_hagg, B * G * P);
    if (int r = launched("aggregate gradient")) return r;
  }
  {
    const pom_view hv{a->y, N * W, W}, dhv{a->dy, N * W, W};
    const pom_tview tv{a->dyt, T, N};
    int r = pom_agg_bwd(POM_DTYPE_BF16, a->param_dtype, B, N, P, a->K, &hv, a->coeff, a->mask, a->mask_stride_b,
                        a->mask_stride_n, a->count, a->frame_len, a->n_past, a->rope_h, a->dh, &dhv,
                        a->dyt ? &tv : nullptr, a->dcoeff, wr, wrb, stream);
    if (r == POM_ERR_UNSUPPORTED && a->dyt) {
      r = pom_agg_bwd(POM_DTYPE_BF16, a->param_dtype, B, N, P, a->K, &hv, a->coeff, a->mask, a->mask_stride_b,
                      a->mask_stride_n, a->count, a->frame_len, a->n_past, a->rope_h, a->dh, &dhv, nullptr,
                      a->dcoeff, wr, wrb, stream);
      if (!r) r = pom_transpose(POM_DTYPE_BF16, T, P, a->dy, W, a->dyt, T, stream);
    }
    if (r) return r;
  }
  // dW_qc = dY^T x on the second stream beside dx (both only read dY)
  if (side_wq) {
    if (int r = wait_for(sd, sd->stream, st, sd->fork)) return r;
    join.armed = true;
    if (int r = pom_gemm(POM_GEMM_MN_CONTIG, POM_GEMM_MN_CONTIG, W, D, T, a->dy, W, a->x, D, a->dwq_dtype, a->dwq, D,
                         -1, 0, wgq, wgqb, sd->stream))
      return r;
  }
  // dx = dY Wq
  if (a->dx) {
    if (!a->wq_t) return err(POM_ERR_INVALID, "pom_layer_bwd: null wq_t");
    if (int r = pom::blas_gemm_tn(D, T, W, a->wq_t, W, a->dy, W, a->dx, D, ws, wsb, st)) return r;
  }
  // dW_qc = dY^T x
  if (a->dwq && !side_wq) {
    if (wgrad_fits(W, D, T)) {
      if (int r = pom_gemm(POM_GEMM_MN_CONTIG, POM_GEMM_MN_CONTIG, W, D, T, a->dy, W, a->x, D, a->dwq_dtype, a->dwq,
                           D, -1, 0, wgq, wgqb, stream))
        return r;
    } else {
      if (!a->xt || !a->dyt || a->dwq_dtype != POM_DTYPE_BF16)
        return err(POM_ERR_INVALID, "pom_layer_bwd: dW_qc off pom_gemm needs xt, dyt and a bf16 output");
      if (int r = pom::blas_gemm_tn(D, W, T, a->xt, T, a->dyt, T, a->dwq, D, ws, wsb, st)) return r;
    }
  }
  if (join.armed) {   // the caller's stream sees the second stream's work done
    join.armed = false;
    if (int r = wait_for(sd, st, sd->stream, sd->join)) return r;
  }
  return POM_OK;
}

}  // extern "C"
