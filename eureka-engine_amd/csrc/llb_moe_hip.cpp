// llb_moe_hip.cpp -- the C ABI (include/llb_moe_hip.h): the backend contract on HIP and the
// per-layer launch sequence of the MoE FFN.
#include "../../include/llb_moe_hip.h"

#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <atomic>

#include "moe_kernels.h"

int launch_gauss(uint64_t seed, uint64_t stream, uint64_t i0, uint64_t n, float sigma, float* out, hipStream_t st);
int launch_gen_rows(uint32_t fm, uint64_t seed, uint64_t stream, uint64_t r0, uint64_t nr, uint32_t cols, float sigma,
                    uint8_t* out, hipStream_t st);
int moe_q8_forward(const llb_moe_layer* L, uint32_t T, const float* h2, const float* x1, float* y, const uint32_t* ids,
                   const float* wt, const float* sgo, const TopkArgs* tk, uint8_t* sc, hipStream_t st);
size_t moe_q8_scratch(const llb_moe_layer* L, uint32_t T);
void moe_q8_set_gemm(bool on);
bool moe_q8_gemm_enabled();
int launch_q8_1(const float* x, uint32_t n, int8_t* q, float2* ds, hipStream_t st);
int launch_spin(uint32_t us, hipStream_t st);
int launch_zero(void* p, uint64_t n, hipStream_t st);

static thread_local char g_err[512];
static hipStream_t g_stream = nullptr;

static int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof g_err, fmt, ap);
  va_end(ap);
  return code;
}
static int hip_ok(hipError_t e, const char* what) {
  if (e == hipSuccess) return 0;
  return fail(LLB_HIP_EDEVICE, "%s: %s", what, hipGetErrorString(e));
}
// for the library's other host files: set the error text, read the stream
int llb_fail_msg(int code, const char* msg) { return fail(code, "%s", msg); }
hipStream_t llb_cur_stream() { return g_stream; }
// a launch's error (bad configuration, no device) is what hipGetLastError reports right after it
static int launched(int rc, const char* what) {
  if (rc != 0) return fail(LLB_HIP_EINVAL, "%s: no kernel for this format / shape", what);
  return hip_ok(hipGetLastError(), what);
}

// optional per-stage timing: an event pair around each stage of a forward, read after a sync
static const char* g_stage_name[ST_NSTAGE] = {"route", "topk", "gate_up", "down", "q8_1"};
static bool g_timing = false;
static bool g_capturing = false;
struct StageEv {
  hipEvent_t a[64], b[64];
  int n;
  double us;
  long cnt;
};
static StageEv g_ev[ST_NSTAGE];
// one-kernel stages are armed here and timed by the GPU around that kernel (LAUNCH_K);
// ST_Q8X (several kernels) records stream events around them
static int g_armed = -1, g_fired = -1;
void stage_begin(int s) {
  if (!g_timing || g_capturing) return;
  StageEv& e = g_ev[s];
  if (e.n >= 64) return;
  if (!e.a[e.n]) { (void)hipEventCreate(&e.a[e.n]); (void)hipEventCreate(&e.b[e.n]); }
  if (s == ST_Q8X) (void)hipEventRecord(e.a[e.n], g_stream);
  else g_armed = s;
}
bool stage_armed(hipEvent_t* a, hipEvent_t* b) {
  if (g_armed < 0) return false;
  StageEv& e = g_ev[g_armed];
  *a = e.a[e.n];
  *b = e.b[e.n];
  g_fired = g_armed;
  g_armed = -1;
  return true;
}
void stage_end(int s) {
  if (!g_timing || g_capturing) return;
  StageEv& e = g_ev[s];
  if (e.n >= 64) return;
  if (s == ST_Q8X) {
    (void)hipEventRecord(e.b[e.n], g_stream);
    e.n++;
  } else if (g_fired == s) {
    e.n++;
  }
  g_armed = g_fired = -1;
}
static void stage_collect() {
  for (int s = 0; s < ST_NSTAGE; s++) {
    StageEv& e = g_ev[s];
    for (int i = 0; i < e.n; i++) {
      float ms = 0;
      hipError_t r = hipEventSynchronize(e.b[i]);
      if (r == hipSuccess) r = hipEventElapsedTime(&ms, e.a[i], e.b[i]);
      if (r == hipSuccess) {
        e.us += 1000.0 * ms;
        e.cnt++;
      } else {
        hip_ok(r, "stage timing");
      }
    }
    e.n = 0;
  }
}

template <class T> static T* dp(llb_dptr p) { return reinterpret_cast<T*>((uintptr_t)p); }

uint64_t llb_row_bytes(uint32_t fm, uint32_t cols);
// stream residency (llb_moe_gguf.cpp): the token's k experts into the staging slots; *slots = their ids
int stream_stage(const llb_moe_layer* L, const uint32_t* d_ids, const uint32_t** slots);
static uint64_t row_bytes(uint32_t fm, uint32_t cols) { return llb_row_bytes(fm, cols); }
uint64_t llb_row_bytes(uint32_t fm, uint32_t cols) {
  switch (fm) {
    case LLB_FM_F32: return (uint64_t)cols * 4;
    case LLB_FM_Q8_0: return (uint64_t)cols / 32 * 34;
    case LLB_FM_Q4_K: return (uint64_t)cols / 256 * 144;
    case LLB_FM_Q6_K: return (uint64_t)cols / 256 * 210;
    case LLB_FM_Q5_K: return (uint64_t)cols / 256 * 176;
  }
  return 0;
}
static bool expert_fm(uint32_t f) {
  return f == LLB_FM_Q8_0 || f == LLB_FM_Q4_K || f == LLB_FM_Q6_K || f == LLB_FM_Q5_K;
}
// llb_cdepth (host/llb_host.c:52-58) and llb_tuned (:64-76) for the formats this path takes
static uint32_t cdepth(uint32_t cols) {
  uint32_t d = 0;
  while ((1u << d) < cols) d++;
  return d - 2;
}
static bool tuned(uint32_t fm, uint32_t cols) {
  uint32_t d = cdepth(cols), cg = cols / 4;
  if (fm == LLB_FM_F32) return d >= 9 && d <= 12;
  if (fm == LLB_FM_Q4_K || fm == LLB_FM_Q6_K) return (cg % 256 == 0 && d >= 8 && d <= 13) || (d >= 9 && d <= 11);
  if (fm == LLB_FM_Q5_K) return cg % 256 == 0 && d >= 8 && d <= 13;
  return false;
}

extern "C" {

const char* llb_hip_last_error(void) { return g_err; }

int llb_hip_init(int device) {
  g_err[0] = 0;
  const int rc = hip_ok(hipSetDevice(device), "hipSetDevice");
  return rc ? rc : noalloc_setup(device);
}
int llb_hip_set_stream(void* s) {
  g_stream = (hipStream_t)s;
  return 0;
}
llb_dptr llb_hip_alloc_zero(size_t bytes) {
  void* p = nullptr;
  if (hip_ok(hipMalloc(&p, bytes ? bytes : 4), "hipMalloc") != 0) return 0;
  if (hip_ok(hipMemset(p, 0, bytes ? bytes : 4), "hipMemset") != 0) {
    (void)hipFree(p);
    return 0;
  }
  return (llb_dptr)(uintptr_t)p;
}
int llb_hip_free(llb_dptr p) { return hip_ok(hipFree(dp<void>(p)), "hipFree"); }
// a fill kernel, not hipMemsetAsync: inside a graph capture it is recorded as a kernel node (the
// reference's CUDA twin leaves its capture instead, host/llb_backend_cuda.h:193-196)
int llb_hip_zero(llb_dptr p, size_t bytes) {
  if (bytes && !p) return fail(LLB_HIP_EINVAL, "llb_zero: null buffer");
  return launched(launch_zero(dp<void>(p), bytes, g_stream), "llb_zero");
}
int llb_hip_copy(llb_dptr d, llb_dptr s, size_t bytes) {
  return hip_ok(hipMemcpyAsync(dp<void>(d), dp<void>(s), bytes, hipMemcpyDeviceToDevice, g_stream), "llb_copy");
}
int llb_hip_write(llb_dptr d, const void* h, size_t bytes) {
  int rc = hip_ok(hipMemcpyAsync(dp<void>(d), h, bytes, hipMemcpyHostToDevice, g_stream), "llb_write");
  return rc ? rc : hip_ok(hipStreamSynchronize(g_stream), "llb_write");
}
int llb_hip_read(void* h, llb_dptr p, size_t bytes) {
  int rc = hip_ok(hipMemcpyAsync(h, dp<void>(p), bytes, hipMemcpyDeviceToHost, g_stream), "llb_read");
  return rc ? rc : hip_ok(hipStreamSynchronize(g_stream), "llb_read");
}
int llb_hip_sync(void) { return hip_ok(hipStreamSynchronize(g_stream), "llb_sync"); }

// kernel by name and LLB_LAUNCH (host/llb_backend.h:11-24; the CUDA twin's cuModuleGetFunction and
// cuLaunchKernel, host/llb_backend_cuda.h:7-11,82-99): a code object loaded once, its kernels looked up
// by name, launched gx * gy groups of bx threads with sm bytes of dynamic LDS on the library's stream,
// each argument the address of a host variable holding its value (the values are copied at the call)
int llb_hip_module_load(const char* path, uint64_t* module) {
  if (!path || !module) return fail(LLB_HIP_EINVAL, "module_load: null argument");
  hipModule_t m = nullptr;
  int rc = hip_ok(hipModuleLoad(&m, path), "hipModuleLoad");
  if (rc) return rc;
  *module = (uint64_t)(uintptr_t)m;
  return 0;
}
int llb_hip_module_function(uint64_t module, const char* name, void** fn) {
  if (!module || !name || !fn) return fail(LLB_HIP_EINVAL, "module_function: null argument");
  hipFunction_t f = nullptr;
  int rc = hip_ok(hipModuleGetFunction(&f, (hipModule_t)(uintptr_t)module, name), "hipModuleGetFunction");
  if (rc) return fail(rc, "module_function: no kernel named %s", name);
  *fn = (void*)f;
  return 0;
}
int llb_hip_launch(void* fn, uint32_t gx, uint32_t gy, uint32_t bx, uint32_t sm, void** args, uint32_t na) {
  return llb_hip_launch3(fn, gx, gy, 1, bx, sm, args, na);
}
// the same with a z grid (the fast prefill's grouped launches, host/llb_pf.h:284-285)
int llb_hip_launch3(void* fn, uint32_t gx, uint32_t gy, uint32_t gz, uint32_t bx, uint32_t sm, void** args,
                    uint32_t na) {
  if (!fn) return fail(LLB_HIP_EINVAL, "launch: null kernel");
  if (!gx || !gy || !gz || !bx || bx > 1024)
    return fail(LLB_HIP_EINVAL, "launch: grid %u x %u x %u of %u threads", gx, gy, gz, bx);
  if (sm > 160 * 1024) return fail(LLB_HIP_EINVAL, "launch: %u bytes of LDS (at most 160 KiB)", sm);
  if (na && !args) return fail(LLB_HIP_EINVAL, "launch: %u arguments but no argument array", na);
  for (uint32_t i = 0; i < na; i++)
    if (!args[i]) return fail(LLB_HIP_EINVAL, "launch: argument %u is a null address", i);
  return hip_ok(hipModuleLaunchKernel((hipFunction_t)fn, gx, gy, gz, bx, 1, 1, sm, g_stream, na ? args : nullptr,
                                      nullptr),
                "hipModuleLaunchKernel");
}
// host memory the device reads and writes in place (cuMemHostAlloc(DEVICEMAP | PORTABLE) +
// cuMemHostGetDevicePointer, host/llb_host.c:446-489): pinned, mapped, and its device address
int llb_hip_host_alloc(size_t bytes, void** host, llb_dptr* dev) {
  if (!host || !dev) return fail(LLB_HIP_EINVAL, "host_alloc: null argument");
  void* h = nullptr;
  int rc = hip_ok(hipHostMalloc(&h, bytes ? bytes : 4, hipHostMallocMapped | hipHostMallocPortable), "hipHostMalloc");
  if (rc) return rc;
  void* d = nullptr;
  if ((rc = hip_ok(hipHostGetDevicePointer(&d, h, 0), "hipHostGetDevicePointer"))) {
    (void)hipHostFree(h);
    return rc;
  }
  *host = h;
  *dev = (llb_dptr)(uintptr_t)d;
  return 0;
}
int llb_hip_host_free(void* host) { return host ? hip_ok(hipHostFree(host), "hipHostFree") : 0; }
// host bytes into device memory in stream order, no wait (cuMemcpyHtoDAsync, host/llb_host.c:691-693): the
// host buffer must stay as it is until the copy has run (pinned memory for a copy that overlaps)
int llb_hip_copy_h2d_async(llb_dptr d, const void* h, size_t bytes) {
  if (bytes && (!d || !h)) return fail(LLB_HIP_EINVAL, "copy_h2d_async: null buffer");
  return hip_ok(hipMemcpyAsync(dp<void>(d), h, bytes, hipMemcpyHostToDevice, g_stream), "copy_h2d_async");
}

// graph record / replay (llb_graph_begin / llb_graph_end, host/llb_backend_cuda.h:125-184): the
// launches between begin and end are captured from the library's stream (a capture needs a
// non-null stream: the library makes its own when none is set) and replayed as one graph
static hipStream_t g_own = nullptr;
int llb_hip_graph_begin(void) {
  if (g_capturing) return fail(LLB_HIP_EINVAL, "graph_begin: already capturing");
  if (!g_stream) {
    if (!g_own) {
      int rc = hip_ok(hipStreamCreateWithFlags(&g_own, hipStreamNonBlocking), "hipStreamCreate");
      if (rc) return rc;
    }
    g_stream = g_own;
  }
  int rc = hip_ok(hipStreamBeginCapture(g_stream, hipStreamCaptureModeThreadLocal), "hipStreamBeginCapture");
  if (rc == 0) g_capturing = true;
  return rc;
}
int llb_hip_graph_end(uint64_t* handle) {
  if (!g_capturing) return fail(LLB_HIP_EINVAL, "graph_end: not capturing");
  g_capturing = false;
  hipGraph_t g = nullptr;
  int rc = hip_ok(hipStreamEndCapture(g_stream, &g), "hipStreamEndCapture");
  if (rc) return rc;
  hipGraphExec_t x = nullptr;
  rc = hip_ok(hipGraphInstantiate(&x, g, nullptr, nullptr, 0), "hipGraphInstantiate");
  (void)hipGraphDestroy(g);
  if (rc) return rc;
  *handle = (uint64_t)(uintptr_t)x;
  return 0;
}
int llb_hip_graph_launch(uint64_t handle) {
  return hip_ok(hipGraphLaunch((hipGraphExec_t)(uintptr_t)handle, g_stream), "hipGraphLaunch");
}
// a kernel that keeps the stream busy for `us` microseconds of wall clock (s_memrealtime, 100 MHz),
// so that launches queued behind it run back to back: the stage timings then measure kernels, not
// the host's launch rate. Bounded: it exits at its deadline whatever happens.
int llb_hip_spin(uint32_t us) {
  if (us > 100000) return fail(LLB_HIP_EINVAL, "spin: at most 100 ms");
  return launched(launch_spin(us, g_stream), "spin");
}
int llb_hip_graph_free(uint64_t handle) {
  return hip_ok(hipGraphExecDestroy((hipGraphExec_t)(uintptr_t)handle), "hipGraphExecDestroy");
}
int llb_hip_mem_info(size_t* f, size_t* t) { return hip_ok(hipMemGetInfo(f, t), "hipMemGetInfo"); }

// ---------------------------------------------------------------- layer checks and scratch

static int check_layer(const llb_moe_layer* L, int tier) {
  if (!L) return fail(LLB_HIP_EINVAL, "null layer");
  const uint32_t fg = L->fx & 15, fu = L->fx >> 4 & 15, fd = L->fx >> 8 & 15, fz = L->fx >> 12 & 1;
  if (!L->dm || L->dm % 256 || !L->ef || L->ef % 256) return fail(LLB_HIP_EINVAL, "dm and ef must be multiples of 256");
  if (!L->ne || L->ne > 1024 || !L->nk || L->nk > L->ne || L->nk > 63)
    return fail(LLB_HIP_EINVAL, "need 1 <= nk <= min(ne, 63), ne <= 1024");
  if (!expert_fm(fg) || !expert_fm(fu) || !expert_fm(fd)) return fail(LLB_HIP_EINVAL, "expert formats: Q8_0, Q4_K, Q5_K, Q6_K");
  if (fz && fu != fg) return fail(LLB_HIP_EINVAL, "fused gate+up needs one format");
  if (tier == LLB_MOE_EXACT && fg != fu) return fail(LLB_HIP_EINVAL, "exact tier: gate and up in one format");
  if (!L->router || !L->G || !L->D || (!fz && !L->U)) return fail(LLB_HIP_EINVAL, "null weights");
  const uint32_t d = cdepth(L->dm);
  if (!tuned(LLB_FM_F32, L->dm) || d > 11) return fail(LLB_HIP_EINVAL, "router: dm in 1025..8192 (the engine tree)");
  if (L->sf) {
    if (L->sf % 256 || !L->shgate || !L->SG || !L->SU || !L->SD) return fail(LLB_HIP_EINVAL, "shared expert: sf % 256, weights");
    if (L->fsg != L->fsu || !tuned(L->fsg, L->dm) || L->fsg == LLB_FM_Q8_0 || !expert_fm(L->fsg))
      return fail(LLB_HIP_EINVAL, "shared gate/up: one K-quant format on a tuned width");
    if (tuned(L->fsd, L->sf) || L->fsd == LLB_FM_Q8_0 || !expert_fm(L->fsd))
      return fail(LLB_HIP_EINVAL, "shared down: a K-quant on llb_gemv_any's order (untuned width)");
  }
  if (64 / (L->nk + (L->sf ? 1 : 0)) < 1) return fail(LLB_HIP_EINVAL, "nk too large");
  return 0;
}

static size_t al(size_t n) { return (n + 255) & ~(size_t)255; }

struct ExactScratch {
  size_t lg, gsu, sa, sgo, act, ctr, total;
};
static ExactScratch exact_layout(const llb_moe_layer* L, uint32_t T) {
  ExactScratch s;
  size_t o = 0;
  s.lg = o; o += al((size_t)T * (L->ne + 1) * 4);
  s.gsu = o; o += al((size_t)T * 2 * L->sf * 4 + 4);
  s.sa = o; o += al((size_t)T * L->sf * 4 + 4);
  s.sgo = o; o += al((size_t)T * 4);
  s.act = o; o += al((size_t)T * L->nk * L->ef * 4);
  s.ctr = o; o += al(8 * 4);
  s.total = o;
  return s;
}

struct GemmScratch {
  size_t x16, off, xmap, inv, gcnt, act, out, spill, sact, shd, total;
};
static GemmScratch gemm_layout(const llb_moe_layer* L, uint32_t T) {
  GemmScratch g;
  const size_t n = (size_t)T * L->nk;
  size_t o = 0;
  g.x16 = o; o += al((size_t)T * L->dm * 2);
  g.off = o; o += al(((size_t)L->ne + 1) * 4);
  g.xmap = o; o += al(n * 4);
  g.inv = o; o += al(n * 4);
  g.gcnt = o; o += al(group_cnt_bytes((uint32_t)n, L->ne));
  g.act = o; o += al(n * L->ef * 2);
  g.out = o; o += al(n * L->dm * 2);
  g.spill = o; o += al(n * L->dm * 4);  // f32 down outputs past f16's range (touched only there)
  g.sact = o; o += al((size_t)T * L->sf * 2 + 4);
  g.shd = o; o += al((size_t)T * L->dm * 4);
  g.total = o;
  return g;
}

size_t llb_moe_hip_scratch_bytes(const llb_moe_layer* L, uint32_t T, int tier) {
  if (!L || !T) return 0;
  const size_t a = exact_layout(L, T).total;
  if (tier == LLB_MOE_Q8) return a + moe_q8_scratch(L, T);
  if (tier == LLB_MOE_F16) return a + gemm_layout(L, T).total;
  return a;
}

// router + shared gate logit + shared gate / up (the tree rows), then top-k and sa
// the router / shared rows launch, then top-k -- or, with defer, top-k's arguments for a later
// launch that routes in-kernel
// the input step riding on the router launch (llb_moe_hip_forward_norm): x, z, w, eps in; x1, h2 out
struct NormIn {
  const float *x, *z, *w;
  float eps;
  float *x1, *h2;
};
static int route(const llb_moe_layer* L, uint32_t T, const float* h2, uint32_t* ids, float* wt, uint8_t* sc,
                 const ExactScratch& s, bool shared_rows = true, TopkArgs* defer = nullptr,
                 const NormIn* nin = nullptr, bool dec = false) {
  float* lg = (float*)(sc + s.lg);
  float* gsu = (float*)(sc + s.gsu);
  TreeArgs a{};
  a.cols = L->dm;
  a.x = h2;
  a.T = T;
  a.xstride = L->dm;
  a.tch = 16;
  const uint32_t ns = 1u << (cdepth(L->dm) - 9);
  a.seg[0] = TreeSeg{dp<uint8_t>(L->router), LLB_FM_F32, (uint64_t)L->dm * 4, L->ne, lg, L->ne + 1,
                     dp<float>(L->router_bias)};
  a.seg[1] = TreeSeg{dp<uint8_t>(L->shgate), LLB_FM_F32, (uint64_t)L->dm * 4, L->sf ? 1u : 0u, lg + L->ne, L->ne + 1,
                     nullptr};
  a.seg[2] = TreeSeg{dp<uint8_t>(L->SG), L->fsg, row_bytes(L->fsg, L->dm), L->sf, gsu, 2 * L->sf, nullptr};
  a.seg[3] = TreeSeg{dp<uint8_t>(L->SU), L->fsu, row_bytes(L->fsu, L->dm), L->sf, gsu + L->sf, 2 * L->sf, nullptr};
  a.nseg = shared_rows ? 4 : 2;
  if (nin) {
    a.x = nin->x;
    a.nz = nin->z;
    a.nw = nin->w;
    a.eps = nin->eps;
    a.x1o = nin->x1;
    a.h2o = nin->h2;
  }
  int rc;
  stage_begin(ST_ROUTE);
#ifdef MOE_DEC_STAMPS
  a.stamps = g_dec_stamps;
#endif
  if (dec) rc = launched(launch_router(a, 1u << (cdepth(L->dm) - 6), g_stream), "router");
  else rc = launched(launch_tree_rows(a, ns, g_stream), "router + shared gate / up");
  if (rc) return rc;
  stage_end(ST_ROUTE);
  TopkArgs k{};
  k.lg = lg;
  k.lstride = L->ne + 1;
  k.ne = L->ne;
  k.nk = L->nk;
  k.has_sg = L->sf ? 1 : 0;
  k.sf = L->sf;
  k.ids = ids;
  k.wt = wt;
  k.sgo = (float*)(sc + s.sgo);
  if (defer) {
    *defer = k;
    return 0;
  }
  stage_begin(ST_TOPK);
  rc = launched(launch_topk(k, T, g_stream), "topk");
  stage_end(ST_TOPK);
  return rc;
}

static int fused_forward(const llb_moe_layer* L, uint32_t T, const float* h2, const float* x1, float* y, uint32_t* ids,
                         float* wt, uint8_t* sc, const ExactScratch& s);

// A second stream for work that overlaps the routed experts' GEMMs (the shared expert's), one per
// device, default priority, with a fork / join event pair. fork: the side stream waits for everything
// queued on the library's stream so far; join: the library's stream waits for the side stream. Both are
// event edges, so a graph capture records them (the side stream joins the capture and is joined back).
struct Side {
  hipStream_t s = nullptr;
  hipEvent_t fork = nullptr, join = nullptr;
};
static Side g_side[64];
static int side_get(Side** out) {
  int d = 0;
  int rc = hip_ok(hipGetDevice(&d), "hipGetDevice");
  if (rc) return rc;
  if (d < 0 || d >= 64) return fail(LLB_HIP_EINVAL, "device %d: at most 64 devices", d);
  Side& x = g_side[d];
  if (!x.s) {
    if ((rc = hip_ok(hipStreamCreateWithFlags(&x.s, hipStreamNonBlocking), "side hipStreamCreate"))) return rc;
    if ((rc = hip_ok(hipEventCreateWithFlags(&x.fork, hipEventDisableTiming), "side hipEventCreate"))) return rc;
    if ((rc = hip_ok(hipEventCreateWithFlags(&x.join, hipEventDisableTiming), "side hipEventCreate"))) return rc;
  }
  *out = &x;
  return 0;
}

// the grouped-GEMM tier: exact routing, the dispatch permutation, expert GEMMs on MFMA, combine
static int gemm_forward(const llb_moe_layer* L, uint32_t T, const float* h2, const float* x1, float* y, uint32_t* ids,
                        float* wt, uint8_t* sc, const ExactScratch& s, const NormIn* nin) {
  const uint32_t fg = L->fx & 15, fu = L->fx >> 4 & 15, fd = L->fx >> 8 & 15, fz = L->fx >> 12 & 1;
  if (fg != fu) return fail(LLB_HIP_EINVAL, "f16 tier: gate and up in one format");
  if (L->sf && L->fsg != L->fsu) return fail(LLB_HIP_EINVAL, "f16 tier: shared gate and up in one format");
  if (L->dm % 256 || L->ef % 128 || L->sf % 128 || L->ne > 1024)
    return fail(LLB_HIP_EINVAL, "f16 tier: dm a multiple of 256, ef and sf of 128, at most 1024 experts");
  const GemmScratch gs = gemm_layout(L, T);
  uint8_t* gb = sc + s.total;
  int rc;
  if ((rc = route(L, T, h2, ids, wt, sc, s, false, nullptr, nin))) return rc;
  const uint32_t n = T * L->nk;
  uint32_t* off = (uint32_t*)(gb + gs.off);
  uint32_t* xmap = (uint32_t*)(gb + gs.xmap);
  uint32_t* inv = (uint32_t*)(gb + gs.inv);
  _Float16* x16 = (_Float16*)(gb + gs.x16);
  stage_begin(ST_Q8X);
  if ((rc = launched(launch_group(ids, n, L->nk, L->ne, off, xmap, inv, h2, x16, (uint64_t)T * L->dm, g_stream,
                                  (uint32_t*)(gb + gs.gcnt)),
                     "group + f16 activations")))
    return rc;
  stage_end(ST_Q8X);
  // the shared expert (dense over the T tokens) needs only x16: on the side stream, overlapping the
  // routed GEMMs, which leave most of the chip idle at a few hundred tokens
  const float* shd = nullptr;
  Side* side = nullptr;
  if (L->sf) {
    if ((rc = side_get(&side))) return rc;
    if ((rc = hip_ok(hipEventRecord(side->fork, g_stream), "fork hipEventRecord"))) return rc;
    if ((rc = hip_ok(hipStreamWaitEvent(side->s, side->fork, 0), "fork hipStreamWaitEvent"))) return rc;
    const uint32_t mt = (T + gemm_bm() - 1) / gemm_bm();
    GemmArgs sg{};
    sg.W0 = dp<uint8_t>(L->SG);
    sg.W1 = dp<uint8_t>(L->SU);
    sg.rb = row_bytes(L->fsg, L->dm);
    sg.K = L->dm;
    sg.N = L->sf;
    sg.M = T;
    sg.A = x16;
    sg.arows = T;
    sg.out = gb + gs.sact;
    if (L->PSG && L->PSU) {
      sg.P0 = dp<uint8_t>(L->PSG);
      sg.P1 = dp<uint8_t>(L->PSU);
    }
    if ((rc = launched(launch_moe_gemm(sg, L->fsg, 0, mt, side->s), "shared gate/up GEMM"))) return rc;
    GemmArgs sd{};
    sd.W0 = dp<uint8_t>(L->SD);
    sd.rb = row_bytes(L->fsd, L->sf);
    sd.K = L->sf;
    sd.N = L->dm;
    sd.M = T;
    sd.A = (const _Float16*)(gb + gs.sact);
    sd.arows = T;
    sd.out = gb + gs.shd;
    sd.P0 = L->PSD ? dp<uint8_t>(L->PSD) : nullptr;
    if ((rc = launched(launch_moe_gemm(sd, L->fsd, 1, mt, side->s), "shared down GEMM"))) return rc;
    if ((rc = hip_ok(hipEventRecord(side->join, side->s), "join hipEventRecord"))) return rc;
    shd = (const float*)(gb + gs.shd);
  }
  const uint64_t rbg = row_bytes(fg, L->dm), rbd = row_bytes(fd, L->ef);
  const uint32_t maxt = n / gemm_bm() + L->ne + 1;  // >= sum over experts of ceil(M_e / BM)
  GemmArgs g{};
  g.W0 = dp<uint8_t>(L->G);
  g.W1 = fz ? g.W0 + (uint64_t)L->ef * rbg : dp<uint8_t>(L->U);
  g.es = (uint64_t)(fz ? 2 : 1) * L->ef * rbg;
  g.rb = rbg;
  g.K = L->dm;
  g.N = L->ef;
  g.A = x16;
  g.arows = T;
  g.xmap = xmap;
  g.off = off;
  g.ne = L->ne;
  g.out = gb + gs.act;
  if (L->PG && L->PU) {
    g.P0 = dp<uint8_t>(L->PG);
    g.P1 = dp<uint8_t>(L->PU);
    g.pes = pack_bytes(fg, L->ef, L->dm);
  }
  stage_begin(ST_GU);
  if ((rc = launched(launch_moe_gemm(g, fg, 0, maxt, g_stream), "expert gate/up GEMM"))) return rc;
  stage_end(ST_GU);
  GemmArgs d = g;
  d.W0 = dp<uint8_t>(L->D);
  d.W1 = nullptr;
  d.es = (uint64_t)L->dm * rbd;
  d.rb = rbd;
  d.K = L->ef;
  d.N = L->dm;
  d.A = (const _Float16*)(gb + gs.act);
  d.arows = n;
  d.xmap = nullptr;
  d.out = gb + gs.out;
  d.o16 = 1;
  d.spill = (float*)(gb + gs.spill);
  d.P0 = L->PD ? dp<uint8_t>(L->PD) : nullptr;
  d.P1 = nullptr;
  d.pes = pack_bytes(fd, L->dm, L->ef);
  stage_begin(ST_DN);
  if ((rc = launched(launch_moe_gemm(d, fd, 1, maxt, g_stream), "expert down GEMM"))) return rc;
  stage_end(ST_DN);
  if (side && (rc = hip_ok(hipStreamWaitEvent(g_stream, side->join, 0), "join hipStreamWaitEvent"))) return rc;
  return launched(launch_combine((const _Float16*)(gb + gs.out), (const float*)(gb + gs.spill), inv, wt, L->nk, shd, (const float*)(sc + s.sgo), x1, y,
                                 L->dm, T, g_stream),
                  "combine");
}

// packed stacks: G, U, D, then SG, SU, SD, each at a 256-byte boundary
static size_t al256(size_t v) { return (v + 255) & ~(size_t)255; }
struct PackPlan {
  uint32_t fm[6], R[6], K[6], ne[6];
  llb_dptr W[6];
  uint64_t es[6];
  size_t off[6], bytes;
};
static bool pack_plan(const llb_moe_layer* L, PackPlan& p) {
  const uint32_t fg = L->fx & 15, fu = L->fx >> 4 & 15, fd = L->fx >> 8 & 15, fz = L->fx >> 12 & 1;
  if (fg != fu || L->dm % 256 || L->ef % 128 || L->sf % 128 || (L->sf && L->fsg != L->fsu)) return false;
  const uint64_t rbg = row_bytes(fg, L->dm);
  const uint32_t fm[6] = {fg, fu, fd, L->fsg, L->fsu, L->fsd};
  const uint32_t R[6] = {L->ef, L->ef, L->dm, L->sf, L->sf, L->dm}, K[6] = {L->dm, L->dm, L->ef, L->dm, L->dm, L->sf};
  const llb_dptr W[6] = {L->G, fz ? L->G + L->ef * rbg : L->U, L->D, L->SG, L->SU, L->SD};
  p.bytes = 0;
  for (int i = 0; i < 6; i++) {
    const bool sh = i >= 3;
    p.fm[i] = fm[i];
    p.R[i] = R[i];
    p.K[i] = K[i];
    p.ne[i] = sh ? (L->sf ? 1 : 0) : L->ne;
    p.W[i] = W[i];
    p.es[i] = (uint64_t)(i < 2 && fz ? 2 : 1) * R[i] * row_bytes(fm[i], K[i]);
    p.off[i] = p.bytes;
    if (!p.ne[i]) continue;
    const uint64_t b = pack_bytes(fm[i], R[i], K[i]);
    if (!b) return false;
    p.bytes = al256(p.bytes + b * p.ne[i]);
  }
  return true;
}
size_t llb_moe_hip_pack_bytes(const llb_moe_layer* L) {
  PackPlan p;
  return L && pack_plan(L, p) ? p.bytes : 0;
}
int llb_moe_hip_pack(llb_moe_layer* L, llb_dptr buf, size_t bytes) {
  PackPlan p;
  if (!L || !buf) return fail(LLB_HIP_EINVAL, "pack: null layer or buffer");
  if (!pack_plan(L, p)) return fail(LLB_HIP_EINVAL, "pack: the f16 tier cannot take this layer");
  if (bytes < p.bytes) return fail(LLB_HIP_EINVAL, "pack: buffer smaller than llb_moe_hip_pack_bytes");
  int rc;
  for (int i = 0; i < 6; i++) {
    if (!p.ne[i]) continue;
    if ((rc = launched(launch_pack(p.fm[i], dp<uint8_t>(p.W[i]), p.es[i], row_bytes(p.fm[i], p.K[i]), p.R[i], p.K[i],
                                   p.ne[i], dp<uint8_t>(buf + p.off[i]), g_stream),
                       "pack")))
      return rc;
  }
  L->PG = buf + p.off[0];
  L->PU = buf + p.off[1];
  L->PD = buf + p.off[2];
  L->PSG = L->sf ? buf + p.off[3] : 0;
  L->PSU = L->sf ? buf + p.off[4] : 0;
  L->PSD = L->sf ? buf + p.off[5] : 0;
  return 0;
}

// the fused one-launch layer (exact tier, small T). It hung the GPU twice and the cause is not
// shown, so it stays off: asking for it is refused; 0 (the four-launch path) is accepted.
static int g_fused = 0;
// the one-token decode's top-k variant (topk_block4 when set); off until it has run on a GPU
static std::atomic<int> g_lean_topk{0};
static int g_ncu = 0;
int llb_moe_hip_set_fused(int on) {
  if (on)
    return fail(LLB_HIP_EINVAL,
                "set_fused: the fused one-launch layer is disabled (it hung the GPU twice; cause not shown)");
  g_fused = 0;
  return 0;
}
int llb_moe_hip_set_q8_gemm(int on) {
  moe_q8_set_gemm(on != 0);
  return 0;
}
int llb_moe_hip_q8_gemm(void) { return moe_q8_gemm_enabled() ? 1 : 0; }
int llb_moe_hip_set_lean_topk(int on) {
  g_lean_topk.store(on ? 1 : 0);
  return 0;
}
int llb_moe_hip_lean_topk(void) { return g_lean_topk.load(); }
int llb_moe_hip_set_group_scan(int on) {
  moe_set_group_scan(on != 0);
  return 0;
}
int llb_moe_hip_group_scan(void) { return moe_group_scan_enabled() ? 1 : 0; }
size_t llb_moe_hip_group_scratch_bytes(uint32_t n, uint32_t ne) {
  return std::max((size_t)(ne + 1) * 4, group_cnt_bytes(n, ne));
}
int llb_moe_hip_status(llb_dptr scratch, const llb_moe_layer* L, uint32_t T) {
  if (!scratch || !L || !T) return fail(LLB_HIP_EINVAL, "status: null argument");
  const ExactScratch s = exact_layout(L, T);
  uint32_t e = 0;
  int rc = hip_ok(hipMemcpyAsync(&e, dp<uint8_t>(scratch) + s.ctr + 5 * 4, 4, hipMemcpyDeviceToHost, g_stream), "status");
  if (!rc) rc = hip_ok(hipStreamSynchronize(g_stream), "status");
  if (rc) return rc;
  if (e) {
    uint32_t z = 0;
    (void)hipMemcpy(dp<uint8_t>(scratch) + s.ctr + 5 * 4, &z, 4, hipMemcpyHostToDevice);
    return fail(LLB_HIP_EDEVICE, "fused layer: a phase wait timed out (results of that launch are not valid)");
  }
  return 0;
}

static int forward_impl(const llb_moe_layer* L, uint32_t T, llb_dptr h2, llb_dptr x1, llb_dptr y, llb_dptr ids,
                        llb_dptr wt, llb_dptr scratch, size_t scratch_bytes, int tier, const NormIn* nin);

int llb_moe_hip_forward(const llb_moe_layer* L, uint32_t T, llb_dptr h2, llb_dptr x1, llb_dptr y, llb_dptr ids,
                        llb_dptr wt, llb_dptr scratch, size_t scratch_bytes, int tier) {
  return forward_impl(L, T, h2, x1, y, ids, wt, scratch, scratch_bytes, tier, nullptr);
}

int llb_moe_hip_forward_norm(const llb_moe_layer* L, uint32_t T, llb_dptr x, llb_dptr z, llb_dptr w, float eps,
                             llb_dptr x1, llb_dptr h2, llb_dptr y, llb_dptr ids, llb_dptr wt, llb_dptr scratch,
                             size_t scratch_bytes, int tier) {
  if (!L) return fail(LLB_HIP_EINVAL, "null layer");
  if (!x || !z || !w || !x1 || !h2) return fail(LLB_HIP_EINVAL, "forward_norm: null input-step buffer");
  if (T == 0) return 0;
  // the router launch carries the input step for T < 16 (its one-token-a-block kernel), outside the
  // fused persistent path; otherwise llb_rmsnorm_add's own launch first -- the same bits either way
  const bool ride = T < 16 && L->dm % 4 == 0 && L->dm <= 16384 &&
                    !(tier == LLB_MOE_EXACT && g_fused && T <= 8);
  if (!ride) {
    int rc = llb_moe_hip_rmsnorm_add(x, z, w, eps, T, L->dm, x1, h2);
    return rc ? rc : llb_moe_hip_forward(L, T, h2, x1, y, ids, wt, scratch, scratch_bytes, tier);
  }
  const NormIn nin{dp<float>(x), dp<float>(z), dp<float>(w), eps, dp<float>(x1), dp<float>(h2)};
  return forward_impl(L, T, h2, x1, y, ids, wt, scratch, scratch_bytes, tier, &nin);
}

// the one-token decode layer of the exact tier (moe_decode.hip): router; top-k + gate / up + SwiGLU
// (with the shared expert's gate / up rows); down + combine + residual. It takes dm = 2048, one
// format for gate and up, at most 16 down tasks (nk + the shared expert), expert widths that are
// multiples of 128, and 16-aligned stacks.
static bool dec_ok(const llb_moe_layer* L) {
  const uint32_t fg = L->fx & 15, fu = L->fx >> 4 & 15, fz = L->fx >> 12 & 1;
  const uint64_t rbg = row_bytes(fg, L->dm);
  const uint64_t U = fz ? L->G + (uint64_t)L->ef * rbg : L->U;
  auto a16 = [](uint64_t p) { return p % 16 == 0; };
  if (L->dm != 2048 || fg != fu || L->nk + (L->sf ? 1 : 0) > 16 || L->ef % 128 || L->ef > 4096) return false;
  // the gate / up launch spreads the shared expert's features over its blocks, at most 15 a block
  if (L->sf > 15 * (L->nk * L->ef / 16)) return false;
  if (!a16(L->G) || !a16(U) || !a16(L->D) || !a16(L->router)) return false;
  if (L->sf && (L->sf % 128 || L->sf > 4096 || !a16(L->SG) || !a16(L->SU) || !a16(L->SD) || !a16(L->shgate)))
    return false;
  return true;
}
// the q8 tier's decode layer on the same kernels needs its down launch to take the layer (it has no
// general fallback of the same numerics)
static bool dec_q8_ok(const llb_moe_layer* L) {
  const uint32_t fd = L->fx >> 8 & 15;
  return dec_ok(L) && dn_dec_lds(L->nk, L->ef, L->sf, row_bytes(fd, L->ef), L->sf ? row_bytes(L->fsd, L->sf) : 0,
                                 L->dm, L->sf != 0, true, nullptr, nullptr) != 0;
}
static int decode_forward(const llb_moe_layer* L, const float* h2, const float* x1, float* y, uint32_t* ids,
                          float* wt, uint8_t* sc, const ExactScratch& s, const NormIn* nin, bool q8) {
  const uint32_t fg = L->fx & 15, fd = L->fx >> 8 & 15, fz = L->fx >> 12 & 1;
  TopkArgs tk{};
  int rc = route(L, 1, h2, ids, wt, sc, s, false, &tk, nin, true);
  if (rc) return rc;
  const uint64_t rbg = row_bytes(fg, L->dm);
  DecGuArgs g{};
  g.G = dp<uint8_t>(L->G);
  g.U = fz ? g.G + (uint64_t)L->ef * rbg : dp<uint8_t>(L->U);
  g.es = (uint64_t)(fz ? 2 : 1) * L->ef * rbg;
  g.SG = L->sf ? dp<uint8_t>(L->SG) : nullptr;
  g.SU = L->sf ? dp<uint8_t>(L->SU) : nullptr;
  g.dm = L->dm;
  g.ef = L->ef;
  g.nk = L->nk;
  g.sf = L->sf;
  g.h2 = h2;
  g.act = (float*)(sc + s.act);
  g.gsu = (float*)(sc + s.gsu);
  g.sa = (float*)(sc + s.sa);
  g.tk = tk;
  g.D = dp<uint8_t>(L->D);
  g.rbd = row_bytes(fd, L->ef);
  g.SD = L->sf ? dp<uint8_t>(L->SD) : nullptr;
  g.rbs = L->sf ? row_bytes(L->fsd, L->sf) : 0;
  g.ndb = (L->dm + 7) / 8;
  g.lean = g_lean_topk.load() ? 1u : 0u;
#ifdef MOE_DEC_STAMPS
  g.stamps = g_dec_stamps;
#endif
  stage_begin(ST_GU);
  if ((rc = launched(launch_gu_dec(g, fg, L->sf ? L->fsg : 0, q8, g_stream), "top-k + expert gate/up (decode)")))
    return rc;
  stage_end(ST_GU);
  DecDnArgs d{};
  d.D = dp<uint8_t>(L->D);
  d.rbd = row_bytes(fd, L->ef);
  d.SD = L->sf ? dp<uint8_t>(L->SD) : nullptr;
  d.rbs = L->sf ? row_bytes(L->fsd, L->sf) : 0;
  d.dm = L->dm;
  d.ef = L->ef;
  d.nk = L->nk;
  d.sf = L->sf;
  d.act = g.act;
  d.sa = g.sa;
  d.ids = ids;
  d.wt = wt;
  d.sgo = tk.sgo;
  d.x1 = x1;
  d.y = y;
#ifdef MOE_DEC_STAMPS
  d.stamps = g_dec_stamps;
#endif
  stage_begin(ST_DN);
  int lr = launch_dn_dec(d, fd, L->sf ? L->fsd : 0, q8, g_stream);
  if (lr && !q8) {  // more down tasks or wider rows than its LDS holds: the general down kernel, same inputs
    DnArgs o{};
    o.D = d.D;
    o.rbd = d.rbd;
    o.SD = d.SD;
    o.rbs = d.rbs;
    o.dm = d.dm;
    o.ef = d.ef;
    o.nk = d.nk;
    o.sf = d.sf;
    o.rw = dn_rows(L->nk, L->ef, L->sf);
    o.act = d.act;
    o.gsu = g.gsu;
    o.ids = ids;
    o.wt = wt;
    o.sgo = d.sgo;
    o.x1 = x1;
    o.y = y;
    lr = launch_dn_exact(o, fd, L->sf ? L->fsd : 0, 1, g_stream);
  }
  rc = launched(lr, "expert down + combine (decode)");
  stage_end(ST_DN);
  return rc;
}

static int forward_impl(const llb_moe_layer* L, uint32_t T, llb_dptr h2, llb_dptr x1, llb_dptr y, llb_dptr ids,
                        llb_dptr wt, llb_dptr scratch, size_t scratch_bytes, int tier, const NormIn* nin) {
  int rc = check_layer(L, tier);
  if (rc) return rc;
  if (T == 0) return 0;
  if (!h2 || !y || !ids || !wt || !scratch) return fail(LLB_HIP_EINVAL, "null buffer");
  if (tier != LLB_MOE_EXACT && tier != LLB_MOE_Q8 && tier != LLB_MOE_F16) return fail(LLB_HIP_EINVAL, "unknown tier %d", tier);
  if (scratch_bytes < llb_moe_hip_scratch_bytes(L, T, tier))
    return fail(LLB_HIP_ESCRATCH, "scratch %zu < %zu bytes", scratch_bytes, llb_moe_hip_scratch_bytes(L, T, tier));
  uint8_t* sc = dp<uint8_t>(scratch);
  const ExactScratch s = exact_layout(L, T);
  const uint32_t fg = L->fx & 15, fu = L->fx >> 4 & 15, fd = L->fx >> 8 & 15, fz = L->fx >> 12 & 1;
  const uint32_t nsp = 1u << (cdepth(L->dm) - 9), fs = L->sf ? L->fsd : 0;
  if (tier == LLB_MOE_EXACT && g_fused && T <= 8 && fg == fu && fused_supported(fg, fd, fs, nsp))
    return fused_forward(L, T, dp<float>(h2), dp<float>(x1), dp<float>(y), dp<uint32_t>(ids), dp<float>(wt), sc, s);
  if (tier == LLB_MOE_F16)
    return gemm_forward(L, T, dp<float>(h2), dp<float>(x1), dp<float>(y), dp<uint32_t>(ids), dp<float>(wt), sc, s, nin);
  // one token: the exact tier routes inside its gate / up launch (one launch fewer a layer; every
  // block recomputes the token's routing, which only pays off for a single token)
  // stream residency (the k chosen experts copied in per token): exact tier, one token, eager
  const bool streamed = L->res == LLB_MOE_RES_STREAM;
  if (streamed && (tier != LLB_MOE_EXACT || T != 1 || g_capturing))
    return fail(LLB_HIP_EINVAL, "stream residency: the exact tier, one token, outside graph capture");
  // one token on the decode kernels: the exact tier, and the q8 tier (the same launches with q8_1
  // activations and integer dots)
  if (T == 1 && !streamed && ((tier == LLB_MOE_EXACT && dec_ok(L)) || (tier == LLB_MOE_Q8 && dec_q8_ok(L))))
    return decode_forward(L, dp<float>(h2), dp<float>(x1), dp<float>(y), dp<uint32_t>(ids), dp<float>(wt), sc, s, nin,
                          tier == LLB_MOE_Q8);
  TopkArgs tk{};
  const bool fuse_topk = (tier == LLB_MOE_Q8 || fg == fu) && T == 1 && !streamed;
  // the q8 tier computes the shared gate / up rows in its own gate / up launch (int8 dots)
  if ((rc = route(L, T, dp<float>(h2), dp<uint32_t>(ids), dp<float>(wt), sc, s, tier != LLB_MOE_Q8,
                  fuse_topk ? &tk : nullptr, nin)))
    return rc;
  const uint64_t rbg = row_bytes(fg, L->dm), rbu = row_bytes(fu, L->dm);
  const uint64_t esg = (uint64_t)(fz ? 2 : 1) * L->ef * rbg;
  const uint8_t* G = dp<uint8_t>(L->G);
  const uint8_t* U = fz ? G + (uint64_t)L->ef * rbg : dp<uint8_t>(L->U);
  if (tier == LLB_MOE_Q8) {
    rc = moe_q8_forward(L, T, dp<float>(h2), dp<float>(x1), dp<float>(y), dp<uint32_t>(ids), dp<float>(wt),
                        (const float*)(sc + s.sgo), fuse_topk ? &tk : nullptr, sc + s.total, g_stream);
    return launched(rc, "q8 tier");
  }
  GuArgs g{};
  g.G = G;
  g.U = U;
  // the expert stride: fused stacks hold gate and up rows per expert (llb_host.c:636)
  g.rbg = rbg;
  g.rbu = rbu;
  g.dm = L->dm;
  g.ef = L->ef;
  g.nk = L->nk;
  g.h2 = dp<float>(h2);
  g.ids = dp<uint32_t>(ids);
  g.act = (float*)(sc + s.act);
  g.es = esg;
  if (streamed) {  // G / U / D are the staging slots, the experts' ids the slot numbers
    const uint32_t* slots = nullptr;
    if ((rc = stream_stage(L, dp<uint32_t>(ids), &slots))) return rc;
    g.ids = slots;
  }
  stage_begin(ST_GU);
  rc = fuse_topk ? launch_gu_topk(g, tk, fg, fu, T * L->nk, g_stream) : launch_gu_exact(g, fg, fu, T * L->nk, g_stream);
  if ((rc = launched(rc, fuse_topk ? "top-k + expert gate/up" : "expert gate/up"))) return rc;
  stage_end(ST_GU);
  DnArgs d{};
  d.D = dp<uint8_t>(L->D);
  d.rbd = row_bytes(fd, L->ef);
  d.SD = dp<uint8_t>(L->SD);
  d.rbs = L->sf ? row_bytes(L->fsd, L->sf) : 0;
  d.dm = L->dm;
  d.ef = L->ef;
  d.nk = L->nk;
  d.sf = L->sf;
  d.rw = dn_rows(L->nk, L->ef, L->sf);
  d.act = g.act;
  d.gsu = (float*)(sc + s.gsu);
  d.ids = g.ids;
  d.wt = dp<float>(wt);
  d.sgo = (float*)(sc + s.sgo);
  d.x1 = dp<float>(x1);
  d.y = dp<float>(y);
  stage_begin(ST_DN);
  rc = launched(launch_dn_exact(d, fd, L->sf ? L->fsd : 0, T, g_stream), "expert down + combine");
  stage_end(ST_DN);
  if (!rc && streamed) rc = stream_done();
  return rc;
}

// the fused layer: the same four stages' argument blocks, one persistent launch
static int fused_forward(const llb_moe_layer* L, uint32_t T, const float* h2, const float* x1, float* y, uint32_t* ids,
                         float* wt, uint8_t* sc, const ExactScratch& s) {
  const uint32_t fg = L->fx & 15, fd = L->fx >> 8 & 15, fz = L->fx >> 12 & 1;
  const uint64_t rbg = row_bytes(fg, L->dm);
  FusedArgs f{};
  float* lg = (float*)(sc + s.lg);
  float* gsu = (float*)(sc + s.gsu);
  f.tr.cols = L->dm;
  f.tr.x = h2;
  f.tr.T = T;
  f.tr.xstride = L->dm;
  f.tr.tch = 1;
  f.tr.seg[0] = TreeSeg{dp<uint8_t>(L->router), LLB_FM_F32, (uint64_t)L->dm * 4, L->ne, lg, L->ne + 1,
                       dp<float>(L->router_bias)};
  f.tr.seg[1] = TreeSeg{dp<uint8_t>(L->shgate), LLB_FM_F32, (uint64_t)L->dm * 4, L->sf ? 1u : 0u, lg + L->ne, L->ne + 1,
                       nullptr};
  f.tr.seg[2] = TreeSeg{dp<uint8_t>(L->SG), L->fsg, row_bytes(L->fsg, L->dm), L->sf, gsu, 2 * L->sf, nullptr};
  f.tr.seg[3] = TreeSeg{dp<uint8_t>(L->SU), L->fsu, row_bytes(L->fsu, L->dm), L->sf, gsu + L->sf, 2 * L->sf, nullptr};
  f.tr.nseg = 4;
  const uint32_t rows = L->ne + (L->sf ? 1 + 2 * L->sf : 0);
  f.tk = TopkArgs{lg, L->ne + 1, L->ne, L->nk, L->sf ? 1u : 0u, L->sf, ids, wt, (float*)(sc + s.sgo)};
  f.gu.G = dp<uint8_t>(L->G);
  f.gu.U = fz ? f.gu.G + (uint64_t)L->ef * rbg : dp<uint8_t>(L->U);
  f.gu.rbg = rbg;
  f.gu.rbu = row_bytes(L->fx >> 4 & 15, L->dm);
  f.gu.es = (uint64_t)(fz ? 2 : 1) * L->ef * rbg;
  f.gu.dm = L->dm;
  f.gu.ef = L->ef;
  f.gu.nk = L->nk;
  f.gu.h2 = h2;
  f.gu.ids = ids;
  f.gu.act = (float*)(sc + s.act);
  f.dn.D = dp<uint8_t>(L->D);
  f.dn.rbd = row_bytes(fd, L->ef);
  f.dn.SD = dp<uint8_t>(L->SD);
  f.dn.rbs = L->sf ? row_bytes(L->fsd, L->sf) : 0;
  f.dn.dm = L->dm;
  f.dn.ef = L->ef;
  f.dn.nk = L->nk;
  f.dn.sf = L->sf;
  f.dn.rw = dn_rows(L->nk, L->ef, L->sf);
  f.dn.act = f.gu.act;
  f.dn.gsu = gsu;
  f.dn.ids = ids;
  f.dn.wt = wt;
  f.dn.sgo = (float*)(sc + s.sgo);
  f.dn.x1 = x1;
  f.dn.y = y;
  f.T = T;
  const uint32_t rpi = 4 * tree_rows_per_wave(1u << (cdepth(L->dm) - 9));  // 4 waves an item
  f.rpt = (rows + rpi - 1) / rpi;
  f.nR = T * f.rpt;
  f.np = 4;
  f.nG = T * L->nk * L->ef / f.np;
  f.dpt = (L->dm + f.dn.rw - 1) / f.dn.rw;
  f.nD = T * f.dpt;
  f.spin = 20000000u;  // 0.2 s
  f.ctr = (uint32_t*)(sc + s.ctr);
  if (!g_ncu) {
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
      n = 256;
    g_ncu = n;
  }
  const uint32_t items = f.nR + T + f.nG + f.nD;
  const uint32_t grid = items < (uint32_t)g_ncu * 4 ? items : (uint32_t)g_ncu * 4;
  stage_begin(ST_GU);
  int rc = launched(launch_fused(f, fg, fd, L->sf ? L->fsd : 0, 1u << (cdepth(L->dm) - 9), grid, g_stream), "fused layer");
  stage_end(ST_GU);
  return rc;
}

// per-stage timing (diagnostics and the benchmark's per-kernel roofline): on = 1 starts a fresh
// tally; read returns the mean microseconds of each stage and the stage names
int llb_moe_hip_timing(int on) {
  g_timing = on != 0;
  for (int s = 0; s < ST_NSTAGE; s++) { g_ev[s].n = 0; g_ev[s].us = 0; g_ev[s].cnt = 0; }
  return 0;
}
int llb_moe_hip_timing_read(double* mean_us, long* counts, int n) {
  stage_collect();
  for (int s = 0; s < ST_NSTAGE && s < n; s++) {
    mean_us[s] = g_ev[s].cnt ? g_ev[s].us / g_ev[s].cnt : 0.0;
    counts[s] = g_ev[s].cnt;
  }
  return ST_NSTAGE;
}
const char* llb_moe_hip_stage_name(int s) { return s >= 0 && s < ST_NSTAGE ? g_stage_name[s] : ""; }

// ---------------------------------------------------------------- kernel-level entry points

int llb_moe_hip_topk(llb_dptr lg, uint32_t lstride, uint32_t T, uint32_t ne, uint32_t nk, uint32_t has_sg,
                     llb_dptr ids, llb_dptr wt, llb_dptr sgo) {
  if (!ne || ne > 1024 || !nk || nk > ne || nk > 64 || lstride < ne + (has_sg ? 1 : 0))
    return fail(LLB_HIP_EINVAL, "topk: need 1 <= nk <= min(ne, 64), ne <= 1024");
  TopkArgs k{};
  k.lg = dp<float>(lg);
  k.lstride = lstride;
  k.ne = ne;
  k.nk = nk;
  k.has_sg = has_sg;
  k.ids = dp<uint32_t>(ids);
  k.wt = dp<float>(wt);
  k.sgo = dp<float>(sgo);
  return launched(launch_topk(k, T, g_stream), "topk");
}

int llb_moe_hip_group(llb_dptr ids, uint32_t n, uint32_t nk, uint32_t ne, llb_dptr off, llb_dptr xmap, llb_dptr inv,
                      llb_dptr scratch, size_t scratch_bytes) {
  if (!ne || !nk || n % nk) return fail(LLB_HIP_EINVAL, "group: n must be a multiple of nk");
  // (the per-expert scans need no scratch; (ne + 1) * 4 bytes has always been asked)
  const size_t need = moe_group_scan_enabled() ? llb_moe_hip_group_scratch_bytes(n, ne) : (size_t)(ne + 1) * 4;
  if (scratch_bytes < need) return fail(LLB_HIP_ESCRATCH, "group: scratch < %zu bytes", need);
  return launched(launch_group(dp<uint32_t>(ids), n, nk, ne, dp<uint32_t>(off), dp<uint32_t>(xmap), dp<uint32_t>(inv),
                               nullptr, nullptr, 0, g_stream, dp<uint32_t>(scratch)),
                  "group");
}

int llb_moe_hip_rmsnorm_add(llb_dptr x, llb_dptr z, llb_dptr w, float eps, uint32_t T, uint32_t n, llb_dptr x1,
                            llb_dptr h2) {
  if (!x || !z || !w || !h2) return fail(LLB_HIP_EINVAL, "rmsnorm_add: null operand");
  if (n == 0 || n > 16384 || T == 0 || (n > 512 && n % 4))
    return fail(LLB_HIP_EINVAL, "rmsnorm_add: 1 <= n <= 16384, n % 4 == 0 past 512, T >= 1");
  return launched(launch_rmsnorm_add(dp<float>(x), dp<float>(z), dp<float>(w), eps, T, n, dp<float>(x1), dp<float>(h2),
                                     g_stream),
                  "rmsnorm_add");
}

int llb_moe_hip_q8_1(llb_dptr x, uint32_t n, llb_dptr q, llb_dptr ds) {
  if (n % 32) return fail(LLB_HIP_EINVAL, "q8_1: n % 32 != 0");
  return launched(launch_q8_1(dp<float>(x), n, dp<int8_t>(q), dp<float2>(ds), g_stream), "q8_1");
}

int llb_moe_hip_exp(llb_dptr x, uint64_t n, llb_dptr y) {
  if (n && (!x || !y)) return fail(LLB_HIP_EINVAL, "exp: null buffer");
  return launched(launch_exp(dp<float>(x), dp<float>(y), n, g_stream), "exp");
}

int llb_moe_hip_dequant(uint32_t fm, llb_dptr W, uint32_t rows, uint32_t cols, llb_dptr out) {
  if (!row_bytes(fm, cols) || cols % 32 || (fm != LLB_FM_F32 && fm != LLB_FM_Q8_0 && cols % 256))
    return fail(LLB_HIP_EINVAL, "dequant: bad format / width");
  return launched(launch_dequant(fm, dp<uint8_t>(W), row_bytes(fm, cols), rows, cols, dp<float>(out), g_stream), "dequant");
}

int llb_moe_hip_gen_gauss(uint64_t seed, uint64_t stream, uint64_t i0, uint64_t n, float sigma, llb_dptr out) {
  return launched(launch_gauss(seed, stream, i0, n, sigma, dp<float>(out), g_stream), "gen_gauss");
}
int llb_moe_hip_gen_rows(uint32_t fm, uint64_t seed, uint64_t stream, uint64_t r0, uint64_t nr, uint32_t cols,
                         float sigma, llb_dptr out) {
  if (!row_bytes(fm, cols)) return fail(LLB_HIP_EINVAL, "gen_rows: bad format");
  return launched(launch_gen_rows(fm, seed, stream, r0, nr, cols, sigma, dp<uint8_t>(out), g_stream), "gen_rows");
}

}  // extern "C"
