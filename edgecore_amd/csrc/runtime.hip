// Host runtime of libedgecore_hip.so: the C ABI of include/edgecore.h.
//
// One GPU per process (device 0 or $EDGECORE_DEVICE), one non-blocking HIP
// stream at the default priority.  gpt2_load reads the .ecm file once, packs
// every tensor into one HBM arena (Qwen2 q/k/v back to back so one GEMV
// produces all three), builds the RoPE table on the host with the same libm
// calls as the reference and allocates the fp16 KV cache and workspaces.
// A forward call copies tokens/positions/slots in, enqueues the layer kernels
// and copies logits (or greedy ids) out.
#include "edgecore.h"
#include "ec_kernels.h"

#include <hip/hip_runtime.h>

#include <errno.h>
#include <fcntl.h>
#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

using namespace ec;

// ---------------------------------------------------------------------------
// errors, device, stream
// ---------------------------------------------------------------------------

static thread_local char g_err[512];
static int g_inited = 0;
static int g_device = 0;
static hipStream_t g_stream = nullptr;
// a prefill reads each layer's weights into the memory-side cache on a
// second stream while that layer's attention runs (EDGECORE_TOUCH=0: off)
static hipStream_t g_side = nullptr;
static hipEvent_t g_touch_ev[4] = {};
static unsigned g_touch_i = 0;
static unsigned *g_touch_sink = nullptr;  // this GPU's copy of touch_sink (below)
static bool g_touch = true;
// the persistent decode step: a plain launch of one block per CU (no
// cooperative-launch barriers: ~30 us less per step) until a step reports a
// timed-out wait (a block that never became resident), then cooperative
// launches from there on, the failed step redone (EDGECORE_STEP_COOP=1:
// cooperative from the start).  EDGECORE_STEP_TEST_FAIL=1 makes the first
// plain step report a timeout (tests of the switch).
static bool g_step_coop = false;
static bool g_step_test_fail = false;
// EDGECORE_TAIL_TEST_FAIL=1 makes the first forward through the batched
// layer tail report a timed-out wait (tests of the fallback to the GEMVs)
static bool g_tail_test_fail = false;
static int g_touch_blocks = 8;  // one per XCD; a multiple of 8 (EDGECORE_TOUCH_BLOCKS)
constexpr int kTouchMinRows = 1024;  // prompts at least this long
static hipDeviceProp_t g_prop;
static int g_max_lds = 65536;
// replay the single-token greedy step as a HIP graph (EDGECORE_GRAPHS=0 turns it off)
static bool g_use_graphs = true;
// int8 linears with kGemmMinM rows or more on the matrix cores
// (EDGECORE_MFMA=0: the vector GEMV for every M)
static bool g_use_mfma = true;

static int set_err(int code, const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof g_err, fmt, ap);
  va_end(ap);
  return code;
}

#define EC_HIP(call)                                                                        \
  do {                                                                                      \
    hipError_t e_ = (call);                                                                 \
    if (e_ != hipSuccess)                                                                   \
      return set_err(-3, "%s failed: %s (%s:%d)", #call, hipGetErrorString(e_), __FILE__,   \
                     __LINE__);                                                             \
  } while (0)

extern "C" const char *ec_last_error(void) { return g_err; }

extern "C" size_t ec_gpt2_sizeof(void) { return sizeof(GPT2); }

// Scratch of ec_topk_dev_noalloc: a file-scope device array, one copy per
// GPU for the life of the process (kNoAllocScratch bytes).  Host code never
// uses the array's name as an address: ec_init resolves this GPU's copy with
// hipGetSymbolAddress and keeps the pointer (g_scratch_dev[device]).
constexpr size_t kNoAllocScratch = (size_t)4 << 20;
constexpr int kMaxDevices = 64;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratch];
static void *g_scratch_dev[kMaxDevices] = {};
// The weight-touch kernel's sink word (it stores a value no load can be
// proven dead against), also a file-scope device array: the library's set-up
// allocates nothing, so a first call into ec_topk_dev_noalloc allocates
// nothing either.
static __device__ __align__(256) unsigned touch_sink[64];

// Every device and pinned-host allocation of the library goes through these
// helpers, which count them (ec_alloc_count).
static long g_allocs = 0;
template <class T>
static hipError_t dev_malloc(T **p, size_t bytes) {
  __atomic_add_fetch(&g_allocs, 1, __ATOMIC_RELAXED);
  return hipMalloc((void **)p, bytes);
}
template <class T>
static hipError_t host_malloc(T **p, size_t bytes, unsigned flags) {
  __atomic_add_fetch(&g_allocs, 1, __ATOMIC_RELAXED);
  return hipHostMalloc((void **)p, bytes, flags);
}
extern "C" long ec_alloc_count(void) { return __atomic_load_n(&g_allocs, __ATOMIC_RELAXED); }

// Device selection, properties, settings and the device arrays' addresses:
// everything the library's set-up does that neither allocates nor creates a
// stream or an event (ec_topk_dev_noalloc needs no more).
static int g_dev_inited = 0;
static int init_device(void) {
  if (g_dev_inited) return 0;
  const char *d = getenv("EDGECORE_DEVICE");
  g_device = d ? atoi(d) : 0;
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess || n <= 0)
    return set_err(-2, "no HIP device available");
  if (g_device < 0 || g_device >= n)
    return set_err(-2, "EDGECORE_DEVICE=%d out of range (%d devices)", g_device, n);
  EC_HIP(hipSetDevice(g_device));
  EC_HIP(hipGetDeviceProperties(&g_prop, g_device));
  int lds = 0;
  if (hipDeviceGetAttribute(&lds, hipDeviceAttributeMaxSharedMemoryPerBlock, g_device) == hipSuccess &&
      lds > 0)
    g_max_lds = lds;
  const char *tch = getenv("EDGECORE_TOUCH");
  g_touch = !(tch && !strcmp(tch, "0"));
  const char *sc = getenv("EDGECORE_STEP_COOP");
  g_step_coop = sc && !strcmp(sc, "1");
  const char *sf = getenv("EDGECORE_STEP_TEST_FAIL");
  g_step_test_fail = sf && !strcmp(sf, "1");
  const char *tf = getenv("EDGECORE_TAIL_TEST_FAIL");
  g_tail_test_fail = tf && !strcmp(tf, "1");
  const char *tb = getenv("EDGECORE_TOUCH_BLOCKS");
  if (tb && atoi(tb) >= 8) g_touch_blocks = atoi(tb) / 8 * 8;
  const char *gr = getenv("EDGECORE_GRAPHS");
  g_use_graphs = !(gr && !strcmp(gr, "0"));
  const char *mf = getenv("EDGECORE_MFMA");
  g_use_mfma = !(mf && !strcmp(mf, "0"));
  gemv_set_max_blocks(8 * g_prop.multiProcessorCount);
  gemv_set_max_lds(g_max_lds);
  if (g_device < kMaxDevices) {
    void *p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) == hipSuccess) g_scratch_dev[g_device] = p;
    else (void)hipGetLastError();  // ec_topk_dev_noalloc reports it
  }
  EC_HIP(hipGetSymbolAddress((void **)&g_touch_sink, HIP_SYMBOL(touch_sink)));
  g_dev_inited = 1;
  return 0;
}

extern "C" int ec_init(void) {
  if (g_inited) return 0;
  const int r = init_device();
  if (r) return r;
  EC_HIP(hipStreamCreateWithFlags(&g_stream, hipStreamNonBlocking));
  EC_HIP(hipStreamCreateWithFlags(&g_side, hipStreamNonBlocking));
  for (hipEvent_t &ev : g_touch_ev) EC_HIP(hipEventCreateWithFlags(&ev, hipEventDisableTiming));
  g_inited = 1;
  return 0;
}

#define EC_INIT()                      \
  do {                                 \
    int r_ = ec_init();                \
    if (r_) return r_;                 \
  } while (0)

extern "C" void *ec_stream(void) {
  if (ec_init()) return nullptr;
  return (void *)g_stream;
}

extern "C" int ec_sync(void) {
  EC_INIT();
  EC_HIP(hipStreamSynchronize(g_stream));
  return 0;
}

extern "C" int ec_device_info(char *buf, int len) {
  EC_INIT();
  int n = snprintf(buf, (size_t)len,
                   "{\"device\": %d, \"name\": \"%s\", \"arch\": \"%s\", \"cus\": %d, "
                   "\"hbm_bytes\": %zu, \"max_lds_per_block\": %d, \"clock_khz\": %d}",
                   g_device, g_prop.name, g_prop.gcnArchName, g_prop.multiProcessorCount,
                   (size_t)g_prop.totalGlobalMem, g_max_lds, g_prop.clockRate);
  return n;
}

extern "C" void *ec_dev_alloc(size_t bytes) {
  if (ec_init()) return nullptr;
  void *p = nullptr;
  if (dev_malloc(&p, bytes ? bytes : 1) != hipSuccess) {
    set_err(-3, "hipMalloc(%zu) failed", bytes);
    return nullptr;
  }
  return p;
}

extern "C" int ec_dev_free(void *p) {
  EC_INIT();
  if (p) EC_HIP(hipFree(p));
  return 0;
}

extern "C" int ec_memcpy_h2d(void *dst, const void *src, size_t bytes) {
  EC_INIT();
  EC_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, g_stream));
  EC_HIP(hipStreamSynchronize(g_stream));
  return 0;
}

extern "C" int ec_memcpy_d2h(void *dst, const void *src, size_t bytes) {
  EC_INIT();
  EC_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, g_stream));
  EC_HIP(hipStreamSynchronize(g_stream));
  return 0;
}

extern "C" int ec_memset_dev(void *dst, int value, size_t bytes) {
  EC_INIT();
  EC_HIP(hipMemsetAsync(dst, value, bytes, g_stream));
  EC_HIP(hipStreamSynchronize(g_stream));
  return 0;
}

// ---------------------------------------------------------------------------
// per-kernel timing
// ---------------------------------------------------------------------------

struct ProfRec {
  const char *fam;
  int ev;  // index of the first of two pooled events
  double bytes;
};
struct ProfAgg {
  const char *fam;
  int n;
  double us, bytes;
};
// The event pool is bounded: when it is full, the stream is synchronized, the
// pending records are folded into per-family totals and the events reused, so
// a profiled run of any length holds at most kProfEvents events.
constexpr size_t kProfEvents = 4096;
static bool g_prof_on = false;
static std::string g_prof_filter;
static std::vector<hipEvent_t> g_ev_pool;
static size_t g_ev_used = 0;
static std::vector<ProfRec> g_prof;
static std::vector<ProfAgg> g_prof_agg;

// fold every pending record into g_prof_agg (the stream must be idle)
static int prof_harvest() {
  for (const ProfRec &r : g_prof) {
    float ms = 0.0f;
    EC_HIP(hipEventElapsedTime(&ms, g_ev_pool[r.ev], g_ev_pool[r.ev + 1]));
    size_t i = 0;
    for (; i < g_prof_agg.size(); i++)
      if (!strcmp(g_prof_agg[i].fam, r.fam)) break;
    if (i == g_prof_agg.size()) g_prof_agg.push_back({r.fam, 0, 0.0, 0.0});
    g_prof_agg[i].n++;
    g_prof_agg[i].us += ms * 1000.0;
    g_prof_agg[i].bytes += r.bytes;
  }
  g_prof.clear();
  g_ev_used = 0;
  return 0;
}

static void prof_release_events() {
  for (hipEvent_t e : g_ev_pool) (void)hipEventDestroy(e);
  g_ev_pool.clear();
  g_ev_used = 0;
}

static int prof_begin(const char *fam, double bytes) {
  if (!g_prof_on) return -1;
  if (!g_prof_filter.empty() && strcmp(fam, g_prof_filter.c_str()) != 0) return -1;
  if (g_ev_used + 2 > kProfEvents) {
    // pool full: wait for the recorded launches and reuse their events
    if (hipStreamSynchronize(g_stream) != hipSuccess || prof_harvest() != 0) return -1;
  }
  while (g_ev_pool.size() < g_ev_used + 2) {
    hipEvent_t e;
    if (hipEventCreate(&e) != hipSuccess) return -1;
    g_ev_pool.push_back(e);
  }
  const int ev = (int)g_ev_used;
  g_ev_used += 2;
  g_launch_ev[0] = g_ev_pool[ev];
  g_launch_ev[1] = g_ev_pool[ev + 1];
  g_prof.push_back({fam, ev, bytes});
  return (int)g_prof.size() - 1;
}

// the launch inside the EC_LAUNCH call consumed the events; if it did not
// launch (an error path), the record is dropped
static void prof_end(int rec) {
  if (rec < 0) return;
  if (g_launch_ev[0]) {
    g_launch_ev[0] = g_launch_ev[1] = nullptr;
    g_prof.pop_back();
    g_ev_used -= 2;
  }
}

extern "C" int ec_prof_start(const char *filter) {
  EC_INIT();
  g_prof_filter = filter ? filter : "";
  g_prof.clear();
  g_prof_agg.clear();
  g_ev_used = 0;
  g_prof_on = true;
  return 0;
}

extern "C" int ec_prof_stop(char *buf, int len) {
  EC_INIT();
  g_prof_on = false;
  EC_HIP(hipStreamSynchronize(g_stream));
  const int hr = prof_harvest();
  prof_release_events();
  if (hr) return hr;
  std::string s = "[";
  for (size_t i = 0; i < g_prof_agg.size(); i++) {
    const ProfAgg &g = g_prof_agg[i];
    char tmp[512];
    const double avg = g.us / g.n, bpl = g.bytes / g.n;
    snprintf(tmp, sizeof tmp,
             "%s{\"kernel\": \"%s\", \"launches\": %d, \"total_us\": %.3f, \"avg_us\": %.4f, "
             "\"bytes_per_launch\": %.0f, \"gbps\": %.2f}",
             i ? ", " : "", g.fam, g.n, g.us, avg, bpl, avg > 0 ? bpl / (avg * 1e3) : 0.0);
    s += tmp;
  }
  s += "]";
  g_prof_agg.clear();
  if ((int)s.size() + 1 > len) return set_err(-1, "ec_prof_stop: buffer too small (%zu)", s.size() + 1);
  memcpy(buf, s.c_str(), s.size() + 1);
  return (int)s.size();
}

#define EC_LAUNCH(fam, bytes, call)                                                        \
  do {                                                                                     \
    const int p_ = prof_begin(fam, (double)(bytes));                                      \
    const hipError_t e_ = (call);                                                          \
    prof_end(p_);                                                                          \
    if (e_ != hipSuccess) return set_err(-3, "%s launch failed: %s", fam, hipGetErrorString(e_)); \
  } while (0)

// ---------------------------------------------------------------------------
// kernel ABI
// ---------------------------------------------------------------------------

// algorithmic bytes of one GEMV launch: weights (twice for gate+up), weight
// scales and bias, the activation rows read, the output rows written (read
// too for a residual add)
static double gemv_bytes(int wt, int pro, int epi, int M, int K, int N, bool scales, bool bias) {
  const double wb = wt == WT_I8 ? 1.0 : 2.0, mats = epi == EPI_SWIGLU ? 2.0 : 1.0;
  double b = mats * ((double)N * K * wb + (scales ? 4.0 * N : 0.0)) + (bias ? 4.0 * N : 0.0);
  b += (double)M * K * (pro == PRO_I8 ? 1.0 : 4.0);
  b += 4.0 * M * N * ((epi == EPI_RESID || epi == EPI_BIAS_RESID) ? 2.0 : 1.0);
  return b;
}

// the fused vector kernel when the shape allows it, else the generic kernel
static hipError_t gemv_any(const GemvArgs &a, int wt, int epi, int pro, hipStream_t s) {
  if (gemv_vector_ok(a, wt, pro)) return gemv(a, wt, epi, pro, s);
  return gemv_generic(a, wt, epi, s);
}

extern "C" int ec_gemm_int8_dev(float *C, const int8_t *A, const float *a_scale, const int8_t *B,
                                const float *b_scale, const float *bias, int M, int K, int N) {
  EC_INIT();
  if (M < 0 || N < 0 || K < 0) return set_err(-1, "gemm_int8: negative shape M=%d K=%d N=%d", M, K, N);
  if (M == 0 || N == 0) return 0;
  if (!C || !a_scale || (K > 0 && (!A || !B))) return set_err(-1, "gemm_int8: null pointer");
  GemvArgs a{A, K, a_scale, nullptr, nullptr, 0.0, B, nullptr, b_scale, nullptr, bias, C, N, M, K, N, nullptr};
  const double bytes = gemv_bytes(WT_I8, PRO_I8, EPI_STORE, M, K, N, b_scale, bias);
  if (g_use_mfma && M >= kGemmMinM && gemm_i8_ok(a, EPI_STORE)) {
    if (M <= 32) {
      EC_LAUNCH("gemm_i8", bytes, gemm_i8_skinny(a, EPI_STORE, 0, g_stream));
    } else {
      EC_LAUNCH("gemm_i8", bytes, gemm_i8(a, EPI_STORE, g_stream));
    }
    return 0;
  }
  EC_LAUNCH("gemv_i8", bytes, gemv_any(a, WT_I8, EPI_STORE, PRO_I8, g_stream));
  return 0;
}

// int8 matrix-core GEMM with a fused epilogue and a chosen row tile, on
// device buffers: the forward's prefill linears, callable alone for checks
extern "C" int ec_gemm_int8_epi_dev(int epi, int bm, float *C, const int8_t *A, const float *a_scale,
                                    const int8_t *B, const float *b_scale, const int8_t *B2,
                                    const float *b2_scale, const float *bias, int M, int K, int N) {
  EC_INIT();
  if (M < 1 || N < 1 || K < 16 || K % 16)
    return set_err(-1, "ec_gemm_int8_epi_dev: shape M=%d K=%d N=%d (K a multiple of 16)", M, K, N);
  if (epi != EPI_STORE && epi != EPI_RESID && epi != EPI_GELU && epi != EPI_SWIGLU)
    return set_err(-1, "ec_gemm_int8_epi_dev: epilogue %d (0 store, 1 residual, 2 GELU, 3 SwiGLU)", epi);
  if (bm != 0 && bm != 16 && bm != 32 && bm != 64 && bm != 128)
    return set_err(-1, "ec_gemm_int8_epi_dev: row tile %d", bm);
  if (bm == 16 && M > 32) return set_err(-1, "ec_gemm_int8_epi_dev: the skinny kernel (bm 16) takes M <= 32, not %d", M);
  if (!C || !A || !a_scale || !B || (epi == EPI_SWIGLU && !B2)) return set_err(-1, "ec_gemm_int8_epi_dev: null pointer");
  GemvArgs a{A, K, a_scale, nullptr, nullptr, 0.0, B, B2, b_scale, b2_scale, epi == EPI_SWIGLU ? nullptr : bias,
             C, N, M, K, N, nullptr};
  if (!gemm_i8_ok(a, epi)) return set_err(-1, "ec_gemm_int8_epi_dev: unaligned operands");
  if (bm == 16) {
    EC_LAUNCH("gemm_i8", 0.0, gemm_i8_skinny(a, epi, 0, g_stream));
    return 0;
  }
  EC_LAUNCH("gemm_i8", 0.0, gemm_i8_tile(a, epi, bm, g_stream));
  return 0;
}

// 16-bit parts of the kernel-ABI 16-bit GEMMs' activation rows, grown on demand
static uint16_t *g_w16_parts = nullptr;
static float *g_w16_rs = nullptr;
static size_t g_w16_halves = 0, g_w16_rows = 0;

static int w16_workspace(int M, int ldp) {
  const size_t halves = (size_t)M * 3 * ldp;
  if (halves > g_w16_halves) {
    EC_HIP(hipStreamSynchronize(g_stream));
    if (g_w16_parts) EC_HIP(hipFree(g_w16_parts));
    g_w16_parts = nullptr;
    g_w16_halves = 0;
    EC_HIP(dev_malloc(&g_w16_parts, halves * sizeof(uint16_t)));
    g_w16_halves = halves;
  }
  if ((size_t)M > g_w16_rows) {
    EC_HIP(hipStreamSynchronize(g_stream));
    if (g_w16_rs) EC_HIP(hipFree(g_w16_rs));
    g_w16_rs = nullptr;
    g_w16_rows = 0;
    EC_HIP(dev_malloc(&g_w16_rs, (size_t)M * sizeof(float)));
    g_w16_rows = M;
  }
  return 0;
}

static int gemm_w16_dev(float *C, const float *A, const uint16_t *B, int M, int K, int N, bool bf16) {
  EC_INIT();
  if (M < 0 || N < 0 || K < 0) return set_err(-1, "gemm: negative shape M=%d K=%d N=%d", M, K, N);
  if (M == 0 || N == 0) return 0;
  if (!C || (K > 0 && (!A || !B))) return set_err(-1, "gemm: null pointer");
  const int wt = bf16 ? WT_BF16 : WT_F16;
  GemvArgs a{A, K, nullptr, nullptr, nullptr, 0.0, B, nullptr, nullptr, nullptr, nullptr, C, N, M, K, N, nullptr};
  const double bytes = gemv_bytes(wt, PRO_F32, EPI_STORE, M, K, N, false, false);
  if (g_use_mfma && M >= kGemmMinM && gemm_w16_ok(a, wt, EPI_STORE)) {
    const int ldp = (K + 7) & ~7;
    int r;
    if ((r = w16_workspace(M, ldp))) return r;
    EC_LAUNCH("gemm_w16", bytes, gemm_w16(a, wt, EPI_STORE, g_w16_parts, ldp, g_w16_rs, g_stream));
    return 0;
  }
  EC_LAUNCH("gemv_w16", bytes, gemv_any(a, wt, EPI_STORE, PRO_F32, g_stream));
  return 0;
}

// 16-bit-weight matrix-core GEMM with a fused epilogue and a chosen row tile,
// on device buffers: the forward's 16-bit prefill linears, callable alone for
// checks.  wt 1 fp16 / 2 bf16; epi as ec_gemm_int8_epi_dev plus 4-6 (bias
// store / residual / GELU).
extern "C" int ec_gemm_w16_epi_dev(int wt, int epi, int bm, float *C, const float *A, const uint16_t *B,
                                   const uint16_t *B2, const float *bias, int M, int K, int N) {
  EC_INIT();
  if (wt != WT_F16 && wt != WT_BF16) return set_err(-1, "ec_gemm_w16_epi_dev: weight type %d (1 fp16, 2 bf16)", wt);
  if (M < 1 || N < 1 || K < 8 || K % 8)
    return set_err(-1, "ec_gemm_w16_epi_dev: shape M=%d K=%d N=%d (K a multiple of 8)", M, K, N);
  if (epi < EPI_STORE || epi > EPI_BIAS_GELU) return set_err(-1, "ec_gemm_w16_epi_dev: epilogue %d", epi);
  if (bm != 0 && bm != 16 && bm != 32 && bm != 64 && bm != 128)
    return set_err(-1, "ec_gemm_w16_epi_dev: row tile %d", bm);
  if (bm == 16 && M > 32) return set_err(-1, "ec_gemm_w16_epi_dev: the skinny kernel (bm 16) takes M <= 32, not %d", M);
  if (!C || !A || !B || (epi == EPI_SWIGLU && !B2)) return set_err(-1, "ec_gemm_w16_epi_dev: null pointer");
  GemvArgs a{A, K, nullptr, nullptr, nullptr, 0.0, B, B2, nullptr, nullptr, bias, C, N, M, K, N, nullptr};
  if (!gemm_w16_ok(a, wt, epi)) return set_err(-1, "ec_gemm_w16_epi_dev: unaligned operands");
  const int ldp = (K + 7) & ~7;
  int r;
  if ((r = w16_workspace(M, ldp))) return r;
  EC_LAUNCH("gemm_w16", 0.0, gemm_w16_tile(a, wt, epi, bm, g_w16_parts, ldp, g_w16_rs, g_stream));
  return 0;
}

extern "C" int ec_gemm_fp16_fp32_dev(float *C, const float *A, const uint16_t *B, int M, int K, int N) {
  return gemm_w16_dev(C, A, B, M, K, N, false);
}

extern "C" int ec_gemm_bf16_fp32_dev(float *C, const float *A, const uint16_t *B, int M, int K, int N) {
  return gemm_w16_dev(C, A, B, M, K, N, true);
}

extern "C" int ec_quantize_rows_dev(const float *in, int M, int K, int8_t *q, float *s) {
  EC_INIT();
  if (M < 0 || K < 0) return set_err(-1, "quantize_rows: negative shape");
  if (M == 0) return 0;
  if (!in || !q || !s) return set_err(-1, "quantize_rows: null pointer");
  EC_LAUNCH("quant", 5.0 * M * K + 4.0 * M, quant_rows(in, K, M, K, q, K, s, g_stream));
  return 0;
}

extern "C" int ec_device_math(int op, const void *in, void *out, size_t n) {
  EC_INIT();
  if (!in || !out) return set_err(-1, "ec_device_math: null pointer");
  if (n == 0) return 0;
  EC_LAUNCH(op == MATH_COPY ? "copy" : "math", 8.0 * n, device_math(op, in, out, n, g_stream));
  EC_HIP(hipStreamSynchronize(g_stream));
  return 0;
}

// grow-only device staging for the host-pointer ABI
struct Staging {
  void *p = nullptr;
  size_t n = 0;
};
static Staging g_st[6];

static int stage(int i, size_t bytes, void **out) {
  if (g_st[i].n < bytes) {
    if (g_st[i].p) EC_HIP(hipFree(g_st[i].p));
    g_st[i].p = nullptr;
    g_st[i].n = 0;
    EC_HIP(dev_malloc(&g_st[i].p, bytes));
    g_st[i].n = bytes;
  }
  *out = g_st[i].p;
  return 0;
}

static void abi_die(const char *fn) {
  fprintf(stderr, "%s: %s\n", fn, g_err);
  exit(1);
}

static int gemm_int8_host(float *C, const int8_t *A, const float *a_scale, const int8_t *B,
                          const float *b_scale, const float *bias, int M, int K, int N) {
  EC_INIT();
  if (M <= 0 || N <= 0) return 0;
  if (K < 0) K = 0;
  void *dA, *das, *dB, *dbs = nullptr, *dbias = nullptr, *dC;
  int r;
  if ((r = stage(0, (size_t)M * K + 16, &dA)) || (r = stage(1, (size_t)M * 4, &das)) ||
      (r = stage(2, (size_t)N * K + 16, &dB)) || (r = stage(4, (size_t)M * N * 4, &dC)))
    return r;
  if (K) EC_HIP(hipMemcpyAsync(dA, A, (size_t)M * K, hipMemcpyHostToDevice, g_stream));
  EC_HIP(hipMemcpyAsync(das, a_scale, (size_t)M * 4, hipMemcpyHostToDevice, g_stream));
  if (K) EC_HIP(hipMemcpyAsync(dB, B, (size_t)N * K, hipMemcpyHostToDevice, g_stream));
  if (b_scale || bias) {
    if ((r = stage(3, (size_t)N * 8, &dbs))) return r;
    if (b_scale) EC_HIP(hipMemcpyAsync(dbs, b_scale, (size_t)N * 4, hipMemcpyHostToDevice, g_stream));
    dbias = (char *)dbs + (size_t)N * 4;
    if (bias) EC_HIP(hipMemcpyAsync(dbias, bias, (size_t)N * 4, hipMemcpyHostToDevice, g_stream));
  }
  if ((r = ec_gemm_int8_dev((float *)dC, (const int8_t *)dA, (const float *)das, (const int8_t *)dB,
                            b_scale ? (const float *)dbs : nullptr,
                            bias ? (const float *)dbias : nullptr, M, K, N)))
    return r;
  EC_HIP(hipMemcpyAsync(C, dC, (size_t)M * N * 4, hipMemcpyDeviceToHost, g_stream));
  EC_HIP(hipStreamSynchronize(g_stream));
  return 0;
}

static int gemm_w16_host(float *C, const float *A, const uint16_t *B, int M, int K, int N, bool bf16) {
  EC_INIT();
  if (M <= 0 || N <= 0) return 0;
  if (K < 0) K = 0;
  void *dA, *dB, *dC;
  int r;
  if ((r = stage(0, (size_t)M * K * 4 + 16, &dA)) || (r = stage(2, (size_t)N * K * 2 + 16, &dB)) ||
      (r = stage(4, (size_t)M * N * 4, &dC)))
    return r;
  if (K) {
    EC_HIP(hipMemcpyAsync(dA, A, (size_t)M * K * 4, hipMemcpyHostToDevice, g_stream));
    EC_HIP(hipMemcpyAsync(dB, B, (size_t)N * K * 2, hipMemcpyHostToDevice, g_stream));
  }
  if ((r = gemm_w16_dev((float *)dC, (const float *)dA, (const uint16_t *)dB, M, K, N, bf16))) return r;
  EC_HIP(hipMemcpyAsync(C, dC, (size_t)M * N * 4, hipMemcpyDeviceToHost, g_stream));
  EC_HIP(hipStreamSynchronize(g_stream));
  return 0;
}

extern "C" void gemm_int8(float *C, const int8_t *A, const float *a_scale, const int8_t *B,
                          const float *b_scale, const float *bias, int M, int K, int N) {
  if (gemm_int8_host(C, A, a_scale, B, b_scale, bias, M, K, N)) abi_die("gemm_int8");
}

extern "C" void gemm_fp16_fp32(float *C, const float *A, const uint16_t *B, int M, int K, int N) {
  if (gemm_w16_host(C, A, B, M, K, N, false)) abi_die("gemm_fp16_fp32");
}

extern "C" void gemm_bf16_fp32(float *C, const float *A, const uint16_t *B, int M, int K, int N) {
  if (gemm_w16_host(C, A, B, M, K, N, true)) abi_die("gemm_bf16_fp32");
}

// ---------------------------------------------------------------------------
// model
// ---------------------------------------------------------------------------

struct LayerDev {
  const float *ln1_g, *ln1_b, *ln2_g, *ln2_b;
  const void *wqkv;
  const float *sqkv, *bqkv;
  const void *wo;
  const float *so, *bo;
  const void *wg, *wu;
  const float *sg, *su;
  const void *wfc;
  const float *sfc, *bfc;
  const void *wd;
  const float *sd, *bd;
};

struct DevModel {
  char *arena = nullptr;
  size_t arena_bytes = 0;
  std::vector<LayerDev> L;
  double2 *rope = nullptr;
  int half = 0;
  int eff_ctx = 0, mmax = 0, lm_rows = 0;
  int qkv_ld = 0, aq_ld = 0, F = 0;
  int *d_tok = nullptr, *d_pos = nullptr, *d_slot = nullptr, *d_amax = nullptr;
  int *h_stage = nullptr;  // pinned: tokens | positions | slots
  float *x = nullptr, *h = nullptr, *qkv = nullptr, *att = nullptr, *ff = nullptr;
  int8_t *aq = nullptr;
  float *as = nullptr;
  // 16-bit parts of fp32 activation rows for the 16-bit-weight matrix-core
  // GEMM ([rows * 3][ah_ld] halves) and their row scales
  uint16_t *ah = nullptr;
  int ah_ld = 0, ah_rows = 0;
  float *ahs = nullptr;
  float *logits = nullptr;
  float *att_sc = nullptr;  // decode attention scores [batch_cap][H][eff_ctx] (long contexts)
  // Batched decode (16-32 tokens) with the activation quantization of the o
  // and down projections inside their skinny GEMMs (EDGECORE_FUSEQ=0 at load
  // turns it off): partial row maxima of the attention output [32][4 H] and
  // of the FFN activation [32][ceil(F / 16)], written by the attention and
  // gate/up (fc) launches
  bool fuse_quant = false;
  bool ff_pmax = false;  // the last gate/up (fc) launch wrote pmax_ff
  float *pmax_att = nullptr, *pmax_ff = nullptr;
  int np_att = 0, np_ff = 0;
  uint16_t *kc = nullptr, *vc = nullptr;
  size_t kv_layer = 0;  // elements per layer of one cache
  const uint16_t *lm = nullptr;
  unsigned long long *cand = nullptr;  // LM-head argmax candidates [lm_rows][gemv blocks]
  int ncand = 0;
  // single-token greedy decode step captured as one HIP graph (see forward_impl)
  hipGraphExec_t step_graph = nullptr;
  int step_bucket = 0;  // the graph's attention LDS covers positions < step_bucket
  // chained greedy decode (ec_generate_greedy): steps whose token comes from
  // the previous step's argmax on the device; ids collected in d_gen
  // [0]: one step, [1]: kChainBurst steps in a row (one launch's overhead
  // for all of them), each for one 512-position bucket
  hipGraphExec_t chain_graph[2] = {nullptr, nullptr};
  int chain_bucket[2] = {0, 0};
  bool chaining = false;  // set while a chained step is enqueued or captured
  int *d_gen = nullptr;
  // the 100 MHz clock before the first chained step ([0]) and at the end of
  // each (argmax) step k ([k + 1]), [eff_ctx + 1]
  unsigned long long *d_gen_t = nullptr;
  int *h_amax = nullptr;  // pinned: the graphs' argmax outputs (batch_cap ids)
  // greedy decode steps of M tokens in distinct slots (kernel-per-op path),
  // one HIP graph per (M, 512-position bucket), oldest replaced first
  struct DecodeGraph {
    int M, bucket;
    hipGraphExec_t exec;
  };
  std::vector<DecodeGraph> dec_graphs;
  // device top-k for sampled decoding: chunk candidates, NaN flags, results
  unsigned long long *tk_cand = nullptr;  // [lm_rows][topk_chunks(V)][kTopkMax + 1]
  unsigned char *tk_nan = nullptr;        // [lm_rows][topk_chunks(V)]
  float *tk_vals = nullptr;               // [lm_rows][kTopkMax + 1]
  int *tk_idx = nullptr, *tk_status = nullptr;
  int last_lm_rows = 0;  // rows of the LM-head chunk the last forward left in `logits`
  // persistent decode step (decode_step.hip), for int8 Qwen2 models of its shape
  bool step_ok = false;
  // 0: the int8 Qwen2 step (decode_step.hip), 1: the fp16 GPT-2 step
  // (decode_step_gpt2.hip)
  int step_kind = 0;
  StepLayer *d_layers = nullptr;  // device copy of the layers' pointers
  Step16Layer *d_layers16 = nullptr;
  unsigned long long *xch = nullptr;  // tagged exchange words
  float *ffv = nullptr;               // the step's FFN words, two halves of [L][F]
  size_t ffv_words = 0;
  size_t xch_bytes = 0;
  // one-token step I/O, device and pinned host: [0] token, [1] position,
  // [2] slot, [3] tag (copied in, 16 bytes); [4] a wait timed out, [5] the
  // greedy id (copied out, 8 bytes)
  int *d_step_io = nullptr, *h_step_io = nullptr;
  unsigned step_tag = 0;          // last tag used
  bool step_nograph = false;      // capturing the step failed once: launch it directly
  unsigned long long *d_trace = nullptr;  // EDGECORE_STEP_TRACE=1: phase timestamps of the last step
  // batched decode's layer tail (decode_tail.hip), int8 Qwen2 of its shapes
  bool tail_ok = false;
  unsigned long long *tail_xch = nullptr;  // its exchange words
  int *d_tail_io = nullptr;  // [0] launch tag, [1] blocks finished, [2] a wait timed out
  int *h_tail_err = nullptr;  // pinned copy of [2] after each forward that used it
};

// host outputs of a forward that selects the top-k logits of its LM-head rows
struct TopkReq {
  int top_k;
  float *vals;
  int *idx;
  int *status;
};

namespace {

struct Place {
  const EcmTensor *t;
  size_t off;
};

struct Loader {
  GPT2 *g;
  const char *base;
  EcmTensor *tens;
  int n;
  std::vector<Place> places;
  size_t cursor = 0;
  char err[256] = {0};

  const EcmTensor *find(const char *name) const {
    for (int i = 0; i < n; i++)
      if (!strcmp(tens[i].name, name)) return &tens[i];
    return nullptr;
  }
  // reserve an aligned arena slot (or, with `glue`, the bytes right after the
  // previous tensor) and return its offset; -1 on a size mismatch
  long place(const EcmTensor *t, size_t want_bytes, int want_dtype, bool glue = false) {
    if (!t) return -1;
    if (t->bytes != want_bytes || (want_dtype >= 0 && t->dtype != want_dtype)) {
      snprintf(err, sizeof err, "ecm: tensor %s has %zu bytes of dtype %d, expected %zu of dtype %d",
               t->name, t->bytes, t->dtype, want_bytes, want_dtype);
      return -2;
    }
    if (!glue) cursor = (cursor + 255) & ~(size_t)255;
    places.push_back({t, cursor});
    const size_t off = cursor;
    cursor += t->bytes;
    return (long)off;
  }
};

}  // namespace

static void free_dev(DevModel *d) {
  if (!d) return;
  void *ps[] = {d->arena, d->rope, d->d_tok, d->d_pos, d->d_slot, d->d_amax, d->x, d->h, d->qkv,
                d->att, d->ff, d->aq, d->as, d->ah, d->ahs, d->att_sc, d->logits, d->kc, d->vc, d->cand, d->tk_cand,
                d->tk_nan, d->tk_vals, d->tk_idx, d->tk_status, d->d_layers, d->d_layers16, d->xch, d->ffv,
                d->d_step_io, d->d_trace,
                d->d_gen, d->d_gen_t, d->pmax_att, d->pmax_ff, d->tail_xch, d->d_tail_io};
  for (void *p : ps)
    if (p) (void)hipFree(p);
  if (d->h_stage) (void)hipHostFree(d->h_stage);
  if (d->h_amax) (void)hipHostFree(d->h_amax);
  if (d->h_step_io) (void)hipHostFree(d->h_step_io);
  if (d->h_tail_err) (void)hipHostFree(d->h_tail_err);
  if (d->step_graph) (void)hipGraphExecDestroy(d->step_graph);
  for (hipGraphExec_t ge : d->chain_graph)
    if (ge) (void)hipGraphExecDestroy(ge);
  for (auto &dg : d->dec_graphs) (void)hipGraphExecDestroy(dg.exec);
  d->dec_graphs.clear();
  delete d;
}

// The device state of each loaded model, keyed by the address of its GPT2
// struct: the struct itself keeps the reference's layout (src/edgecore.h:
// 170-234) field for field, so a caller compiled against that header passes a
// struct of the same size.  A GPT2 must therefore not be moved or copied
// between gpt2_load and gpt2_free (the reference's callers never do).
static std::mutex g_models_mu;
static std::unordered_map<const GPT2 *, DevModel *> g_models;

static DevModel *dev_of(const GPT2 *g) {
  if (!g) return nullptr;
  std::lock_guard<std::mutex> lk(g_models_mu);
  auto it = g_models.find(g);
  return it == g_models.end() ? nullptr : it->second;
}

static void dev_attach(const GPT2 *g, DevModel *d) {
  std::lock_guard<std::mutex> lk(g_models_mu);
  g_models[g] = d;
}

static DevModel *dev_detach(const GPT2 *g) {
  std::lock_guard<std::mutex> lk(g_models_mu);
  auto it = g_models.find(g);
  if (it == g_models.end()) return nullptr;
  DevModel *d = it->second;
  g_models.erase(it);
  return d;
}

// The persistent decode step's shape (decode_step.hip): int8 Qwen2 with
// d_model 896, head_dim 64, up to 8 query heads per KV group (4 blocks per
// head on one XCD of 32 CUs), up to 8 KV groups, FFN <= 5120 in 16-byte rows,
// on a device with 256 CUs and cooperative launch.  EDGECORE_STEP=0 turns it
// off (the forward then runs a kernel per operation).
// The persistent step's exchange state back to "nothing written": the tagged
// words to tag 0, both FFN halves to kStepFfEmpty (not inside a capture).
static hipError_t step_clear(DevModel *d, hipStream_t s) {
  hipError_t e = hipMemsetAsync(d->xch, 0, d->xch_bytes, s);
  if (e == hipSuccess && d->ffv) e = hipMemsetD32Async((hipDeviceptr_t)d->ffv, (int)kStepFfEmpty, d->ffv_words, s);
  return e;
}

// The persistent step that applies to a model: 0 the int8 Qwen2 step, 1 the
// fp16 GPT-2 step, -1 none (a kernel per operation).
static int step_shape_kind(const GPT2 *g, const DevModel *d) {
  const char *env = getenv("EDGECORE_STEP");
  if (env && !strcmp(env, "0")) return -1;
  int coop = 0;
  if (hipDeviceGetAttribute(&coop, hipDeviceAttributeCooperativeLaunch, g_device) != hipSuccess || !coop) return -1;
  if (g_prop.multiProcessorCount != kStepBlocks) return -1;
  const int H = g->n_head, KVH = g->n_kv_head, E = g->n_embd, F = d->F;
  if (g->arch == ARCH_QWEN2 && g->precision == 0 && E == 896 && g->head_dim == 64 && KVH >= 1 && KVH <= 8 &&
      H % KVH == 0 && (H / KVH) * kStepSlices <= kStepBlocks / 8 && F % 16 == 0 && F <= 5120 &&
      H * kStepSlices + E / 16 + (F + 63) / 64 < kStepBlocks)
    return 0;
  if (g->arch != ARCH_QWEN2 && g->precision == 1 && E == kStep16E && g->head_dim == 64 && H == E / 64 &&
      KVH == H && F == kStep16F && g->wpe && g->sliding_window == 0)
    return 1;
  return -1;
}

// The batched decode's layer tail (decode_tail.hip) applies to int8 Qwen2
// models of its shapes on a device with kStepBlocks CUs and cooperative
// launch.  EDGECORE_TAIL=0 turns it off (the batched decode then runs a GEMV
// per linear).
static bool tail_shape_ok(const GPT2 *g, const DevModel *d) {
  const char *env = getenv("EDGECORE_TAIL");
  if (env && !strcmp(env, "0")) return false;
  int coop = 0;
  if (hipDeviceGetAttribute(&coop, hipDeviceAttributeCooperativeLaunch, g_device) != hipSuccess || !coop) return false;
  if (g_prop.multiProcessorCount != kStepBlocks) return false;
  return g->arch == ARCH_QWEN2 && g->precision == 0 &&
         batch_tail_shape_ok(g->n_embd, d->F, g->n_embd + 2 * g->n_kv_embd);
}

static int load_impl(GPT2 *g, const char *path, int batch_cap, int max_ctx) {
  memset(g, 0, sizeof *g);
  g->batch_cap = batch_cap < 1 ? 1 : batch_cap;
  g->max_ctx = max_ctx > 0 ? max_ctx : 0;
  g->eps = 1e-5;
  EC_INIT();

  const int fd = open(path, O_RDONLY);
  if (fd < 0) return set_err(-1, "open model %s: %s", path, strerror(errno));
  struct stat st;
  if (fstat(fd, &st) != 0 || st.st_size <= 0) {
    close(fd);
    return set_err(-1, "model %s is empty", path);
  }
  void *map = mmap(nullptr, (size_t)st.st_size, PROT_READ, MAP_PRIVATE, fd, 0);
  close(fd);
  if (map == MAP_FAILED) return set_err(-1, "mmap model: %s", strerror(errno));
  g->file_data = map;
  g->file_size = (size_t)st.st_size;
  g->file_mapped = 1;

  std::vector<EcmTensor> tens(4096);
  const int n = ecm_parse(map, g->file_size, tens.data(), (int)tens.size(), g);
  if (n < 0) return set_err(-1, "ecm: cannot parse %s", path);
  for (int i = 0; i < n; i++)
    if (tens[i].offset + tens[i].bytes > g->file_size)
      return set_err(-1, "ecm: tensor %s extends past the end of the file (truncated?)", tens[i].name);

  Loader ld{g, (const char *)map, tens.data(), n};
  const bool qwen = g->arch == ARCH_QWEN2;
  const EcmTensor *t0 = ld.find(qwen ? "blocks.0.q.w" : "blocks.0.attn.w");
  if (!ld.find("wte") || !ld.find("ln_f.g")) return set_err(-1, "ecm: missing core tensors (wte, ln_f.g)");
  if (!t0) return set_err(-1, "ecm: missing %s", qwen ? "blocks.0.q.w" : "blocks.0.attn.w");
  if (t0->dtype == 1) g->precision = 1;
  else if (t0->dtype == 2) g->precision = 0;
  else if (t0->dtype == 4) g->precision = 2;
  else return set_err(-1, "ecm: unexpected linear weight dtype");

  const int E = g->n_embd, H = g->n_head, V = g->vocab, Lc = g->n_layer;
  if (E <= 0 || H <= 0 || V <= 0 || Lc <= 0 || g->n_ctx <= 0 || E % H)
    return set_err(-1, "ecm: bad shape meta (n_embd %d, n_head %d, vocab %d, n_layer %d, n_ctx %d)", E, H,
                   V, Lc, g->n_ctx);
  if (qwen) {  // set_qwen2_defaults, src/gpt2.c:149-159
    if (g->n_kv_head <= 0) g->n_kv_head = g->n_head;
    g->head_dim = E / H;
    g->n_kv_embd = g->n_kv_head * g->head_dim;
    if (g->intermediate <= 0) g->intermediate = 4 * E;
    if (g->rope_theta <= 0) g->rope_theta = 10000.0;
    if (g->yarn_orig_max <= 0) g->yarn_orig_max = g->n_ctx;
    if (g->yarn_factor <= 0) g->yarn_factor = 1.0;
    if (g->yarn_attention_factor <= 0) g->yarn_attention_factor = 1.0;
  } else {
    g->n_kv_embd = E;
    g->n_kv_head = H;
    g->intermediate = 4 * E;
    g->head_dim = E / H;
  }
  const int kv = g->n_kv_embd, F = g->intermediate, hd = g->head_dim;
  const int wdt = g->precision == 0 ? 2 : g->precision == 1 ? 1 : 4;  // linear weight dtype
  const int edt = g->precision == 2 ? 4 : 1;                          // embedding dtype
  const size_t wb = g->precision == 0 ? 1 : 2;
  const int eff = gpt2_eff_ctx(g);

  DevModel *d = new DevModel();
  free_dev(dev_detach(g));
  dev_attach(g, d);
  d->eff_ctx = eff;
  d->F = F;
  d->L.resize(Lc);

  long o_wte = ld.place(ld.find("wte"), (size_t)V * E * 2, edt), o_wpe = -1, o_lm = -1;
  long o_lnf = ld.place(ld.find("ln_f.g"), (size_t)E * 4, 0), o_lnfb = -1;
  if (!qwen) {
    if (!ld.find("wpe") || !ld.find("ln_f.b")) return set_err(-1, "ecm: missing wpe / ln_f.b");
    o_wpe = ld.place(ld.find("wpe"), (size_t)g->n_ctx * E * 2, edt);
    o_lnfb = ld.place(ld.find("ln_f.b"), (size_t)E * 4, 0);
  } else {
    const EcmTensor *lmh = ld.find("lm_head.w");
    if (lmh && !g->tie_word_embeddings) o_lm = ld.place(lmh, (size_t)V * E * 2, edt);
    if (g->tie_word_embeddings || !lmh) g->tie_word_embeddings = 1;
  }
  if (o_wte < 0 || o_lnf < 0 || (!qwen && (o_wpe < 0 || o_lnfb < 0)) || o_lm == -2)
    return set_err(-1, "%s", ld.err[0] ? ld.err : "ecm: bad core tensor");

  struct LOff {
    long ln1, ln1b, ln2, ln2b, w[7], s[7], b[7];
  };
  std::vector<LOff> lo(Lc);
  char nm[256];
  for (int l = 0; l < Lc; l++) {
    LOff &o = lo[l];
    for (int i = 0; i < 7; i++) o.w[i] = o.s[i] = o.b[i] = -1;
    auto vec = [&](const char *suf, bool need) -> long {
      snprintf(nm, sizeof nm, "blocks.%d.%s", l, suf);
      const EcmTensor *t = ld.find(nm);
      if (!t) return need ? -3 : -1;
      return ld.place(t, (size_t)E * 4, 0);
    };
    o.ln1 = vec("ln_1.g", true);
    o.ln2 = vec("ln_2.g", true);
    o.ln1b = qwen ? -1 : vec("ln_1.b", true);
    o.ln2b = qwen ? -1 : vec("ln_2.b", true);
    if (o.ln1 < 0 || o.ln2 < 0 || (!qwen && (o.ln1b < 0 || o.ln2b < 0)))
      return set_err(-1, "%s", ld.err[0] ? ld.err : "ecm: missing layer norm tensors");
    // linear list: name, out, in; qwen q/k/v are glued back to back
    const char *qn[7] = {"q", "k", "v", "o", "gate", "up", "down"};
    const int qo[7] = {E, kv, kv, E, F, F, E}, qi[7] = {E, E, E, E, E, E, F};
    const char *gn[4] = {"attn", "proj", "fc", "fc2"};
    const int go[4] = {3 * E, E, 4 * E, E}, gi[4] = {E, E, E, 4 * E};
    const int cnt = qwen ? 7 : 4;
    for (int i = 0; i < cnt; i++) {
      const char *suf = qwen ? qn[i] : gn[i];
      const int out = qwen ? qo[i] : go[i], in = qwen ? qi[i] : gi[i];
      snprintf(nm, sizeof nm, "blocks.%d.%s.w", l, suf);
      o.w[i] = ld.place(ld.find(nm), (size_t)out * in * wb, wdt, qwen && (i == 1 || i == 2));
      if (o.w[i] < 0) return set_err(-1, "%s", ld.err[0] ? ld.err : "ecm: missing linear weight");
    }
    if (g->precision == 0) {
      for (int i = 0; i < cnt; i++) {
        const char *suf = qwen ? qn[i] : gn[i];
        const int out = qwen ? qo[i] : go[i];
        snprintf(nm, sizeof nm, "blocks.%d.%s.s", l, suf);
        o.s[i] = ld.place(ld.find(nm), (size_t)out * 4, 0, qwen && (i == 1 || i == 2));
        if (o.s[i] < 0) return set_err(-1, "%s", ld.err[0] ? ld.err : "ecm: missing int8 scale");
      }
    }
    if (!qwen) {  // GPT-2 linears carry biases (src/gpt2.c:289-305); Qwen2 biases are ignored
      for (int i = 0; i < 4; i++) {
        snprintf(nm, sizeof nm, "blocks.%d.%s.b", l, gn[i]);
        o.b[i] = ld.place(ld.find(nm), (size_t)go[i] * 4, 0);
        if (o.b[i] < 0) return set_err(-1, "%s", ld.err[0] ? ld.err : "ecm: missing bias");
      }
    }
  }
  const EcmTensor *tv = ld.find("tokenizer.vocab"), *tm = ld.find("tokenizer.merges");
  if (!tv || !tm) return set_err(-1, "ecm: tokenizer blobs missing");
  if (tokenizer_load(&g->tok, ld.base + tv->offset, tv->bytes, ld.base + tm->offset, tm->bytes, V,
                     qwen ? 1 : 0) != 0)
    return set_err(-1, "ecm: tokenizer blobs unreadable");

  // upload the arena
  d->arena_bytes = (ld.cursor + 255) & ~(size_t)255;
  EC_HIP(dev_malloc(&d->arena, d->arena_bytes));
  for (const Place &p : ld.places)
    EC_HIP(hipMemcpy(d->arena + p.off, ld.base + p.t->offset, p.t->bytes, hipMemcpyHostToDevice));
  char *A = d->arena;
  auto F32 = [&](long off) -> const float * { return off >= 0 ? (const float *)(A + off) : nullptr; };
  g->wte = (const uint16_t *)(A + o_wte);
  g->wpe = o_wpe >= 0 ? (const uint16_t *)(A + o_wpe) : nullptr;
  g->lm_head = o_lm >= 0 ? (const uint16_t *)(A + o_lm) : nullptr;
  g->lnf_g = F32(o_lnf);
  g->lnf_b = F32(o_lnfb);
  d->lm = g->lm_head ? g->lm_head : g->wte;
  g->lw = (struct LayerW *)calloc((size_t)Lc, sizeof *g->lw);
  for (int l = 0; l < Lc; l++) {
    const LOff &o = lo[l];
    struct LayerW *W = &g->lw[l];
    LayerDev &D = d->L[l];
    W->ln1_g = D.ln1_g = F32(o.ln1);
    W->ln1_b = D.ln1_b = F32(o.ln1b);
    W->ln2_g = D.ln2_g = F32(o.ln2);
    W->ln2_b = D.ln2_b = F32(o.ln2b);
    if (qwen) {
      const void *w[7];
      for (int i = 0; i < 7; i++) w[i] = A + o.w[i];
      W->q_w = w[0]; W->k_w = w[1]; W->v_w = w[2]; W->o_w = w[3];
      W->gate_w = w[4]; W->up_w = w[5]; W->down_w = w[6];
      W->q_s = F32(o.s[0]); W->k_s = F32(o.s[1]); W->v_s = F32(o.s[2]); W->o_s = F32(o.s[3]);
      W->gate_s = F32(o.s[4]); W->up_s = F32(o.s[5]); W->down_s = F32(o.s[6]);
      D.wqkv = w[0]; D.sqkv = W->q_s; D.bqkv = nullptr;
      D.wo = w[3]; D.so = W->o_s; D.bo = nullptr;
      D.wg = w[4]; D.sg = W->gate_s; D.wu = w[5]; D.su = W->up_s;
      D.wd = w[6]; D.sd = W->down_s; D.bd = nullptr;
    } else {
      W->attn_w = A + o.w[0]; W->proj_w = A + o.w[1]; W->fc_w = A + o.w[2]; W->fc2_w = A + o.w[3];
      W->attn_s = F32(o.s[0]); W->proj_s = F32(o.s[1]); W->fc_s = F32(o.s[2]); W->fc2_s = F32(o.s[3]);
      W->attn_b = F32(o.b[0]); W->proj_b = F32(o.b[1]); W->fc_b = F32(o.b[2]); W->fc2_b = F32(o.b[3]);
      D.wqkv = W->attn_w; D.sqkv = W->attn_s; D.bqkv = W->attn_b;
      D.wo = W->proj_w; D.so = W->proj_s; D.bo = W->proj_b;
      D.wfc = W->fc_w; D.sfc = W->fc_s; D.bfc = W->fc_b;
      D.wd = W->fc2_w; D.sd = W->fc2_s; D.bd = W->fc2_b;
    }
  }

  // RoPE table: the reference's qwen_inv_freq / qwen_rope_cos_sin
  // (src/gpt2.c:608-654) evaluated once per position with the same libm calls
  if (qwen) {
    int half = hd / 2;
    if (half > 512) half = 512;
    d->half = half;
    std::vector<double> invf(half);
    const int dim = 2 * half;
    const double inv_base = 1.0 / g->rope_theta;
    for (int i = 0; i < half; i++) invf[i] = pow(inv_base, (double)(2 * i) / (double)dim);
    if (g->rope_type == ROPE_YARN) {
      const double pi2 = 6.28318530717958647692, logbase = log(g->rope_theta);
      double lo_ = floor((double)dim * log(g->yarn_orig_max / (32.0 * pi2)) / (2.0 * logbase));
      double hi_ = ceil((double)dim * log(g->yarn_orig_max / (1.0 * pi2)) / (2.0 * logbase));
      if (lo_ < 0.0) lo_ = 0.0;
      if (hi_ > (double)(dim - 1)) hi_ = (double)(dim - 1);
      double span = hi_ - lo_;
      if (span < 1.0) span = 1.0;
      for (int i = 0; i < half; i++) {
        double ramp = ((double)i - lo_) / span;
        if (ramp < 0.0) ramp = 0.0;
        if (ramp > 1.0) ramp = 1.0;
        const double extrap = invf[i], interp = invf[i] / g->yarn_factor;
        invf[i] = interp * ramp + extrap * (1.0 - ramp);
      }
    }
    std::vector<double2> tab((size_t)eff * half);
    const double scale = g->yarn_attention_factor;
    for (int p = 0; p < eff; p++)
      for (int i = 0; i < half; i++) {
        const double f = (double)p * invf[i];
        tab[(size_t)p * half + i] = make_double2(cos(f) * scale, sin(f) * scale);
      }
    EC_HIP(dev_malloc(&d->rope, tab.size() * sizeof(double2)));
    EC_HIP(hipMemcpy(d->rope, tab.data(), tab.size() * sizeof(double2), hipMemcpyHostToDevice));
  }

  // KV cache [L][B][eff_ctx][kv] fp16, zeroed
  d->kv_layer = (size_t)g->batch_cap * eff * kv;
  const size_t kvb = d->kv_layer * Lc * sizeof(uint16_t);
  EC_HIP(dev_malloc(&d->kc, kvb));
  EC_HIP(dev_malloc(&d->vc, kvb));
  EC_HIP(hipMemset(d->kc, 0, kvb));
  EC_HIP(hipMemset(d->vc, 0, kvb));
  g->k_cache = d->kc;
  g->v_cache = d->vc;

  // workspaces for M up to max(eff_ctx, batch_cap) (src/gpt2.c:319-348)
  const int mmax = eff > g->batch_cap ? eff : g->batch_cap;
  d->mmax = mmax;
  d->qkv_ld = qwen ? E + 2 * kv : 3 * E;
  const int qmax = E > F ? E : F;
  d->aq_ld = (qmax + 15) & ~15;
  d->lm_rows = mmax < 64 ? mmax : 64;
  if (d->lm_rows < g->batch_cap) d->lm_rows = g->batch_cap;
  EC_HIP(dev_malloc(&d->x, (size_t)mmax * E * 4));
  EC_HIP(dev_malloc(&d->h, (size_t)mmax * E * 4));
  EC_HIP(dev_malloc(&d->qkv, (size_t)mmax * d->qkv_ld * 4));
  EC_HIP(dev_malloc(&d->att, (size_t)mmax * E * 4));
  EC_HIP(dev_malloc(&d->ff, (size_t)mmax * F * 4));
  EC_HIP(dev_malloc(&d->aq, (size_t)mmax * d->aq_ld));
  EC_HIP(dev_malloc(&d->as, (size_t)mmax * 4));
  {
    // 16-bit linears: every row of every layer; int8 models: the LM head's rows
    const bool w16 = g->precision != 0;
    d->ah_rows = w16 ? mmax : d->lm_rows;
    d->ah_ld = ((w16 ? qmax : E) + 7) & ~7;
    EC_HIP(dev_malloc(&d->ah, (size_t)d->ah_rows * 3 * d->ah_ld * sizeof(uint16_t)));
    EC_HIP(dev_malloc(&d->ahs, (size_t)d->ah_rows * 4));
  }
  EC_HIP(dev_malloc(&d->att_sc, (size_t)g->batch_cap * g->n_head * eff * sizeof(float)));
  {
    const char *fq = getenv("EDGECORE_FUSEQ");
    d->fuse_quant = g->precision == 0 && !(fq && !strcmp(fq, "0"));
    d->np_att = 4 * g->n_head;
    d->np_ff = (F + 15) / 16;
    // partials a launch never writes stay 0, which no row maximum goes below
    EC_HIP(dev_malloc(&d->pmax_att, (size_t)32 * d->np_att * sizeof(float)));
    EC_HIP(dev_malloc(&d->pmax_ff, (size_t)32 * d->np_ff * sizeof(float)));
    EC_HIP(hipMemset(d->pmax_att, 0, (size_t)32 * d->np_att * sizeof(float)));
    EC_HIP(hipMemset(d->pmax_ff, 0, (size_t)32 * d->np_ff * sizeof(float)));
  }
  EC_HIP(dev_malloc(&d->logits, (size_t)d->lm_rows * V * 4));
  EC_HIP(dev_malloc(&d->d_tok, (size_t)mmax * 4));
  EC_HIP(dev_malloc(&d->d_pos, (size_t)mmax * 4));
  EC_HIP(dev_malloc(&d->d_slot, (size_t)mmax * 4));
  EC_HIP(dev_malloc(&d->d_amax, (size_t)mmax * 4));
  EC_HIP(host_malloc((void **)&d->h_stage, ((size_t)mmax * 3 + 1) * 4, hipHostMallocDefault));
  EC_HIP(host_malloc((void **)&d->h_amax, (size_t)(g->batch_cap > 4 ? g->batch_cap : 4) * sizeof(int),
                       hipHostMallocDefault));
  d->ncand = gemv_max_blocks();
  EC_HIP(dev_malloc(&d->cand, (size_t)d->lm_rows * d->ncand * sizeof(unsigned long long)));
  {
    const size_t nb = (size_t)topk_chunks(V), n = kTopkMax + 1;
    EC_HIP(dev_malloc(&d->tk_cand, (size_t)d->lm_rows * nb * n * sizeof(unsigned long long)));
    EC_HIP(dev_malloc(&d->tk_nan, (size_t)d->lm_rows * nb));
    EC_HIP(dev_malloc(&d->tk_vals, (size_t)d->lm_rows * n * sizeof(float)));
    EC_HIP(dev_malloc(&d->tk_idx, (size_t)d->lm_rows * n * sizeof(int)));
    EC_HIP(dev_malloc(&d->tk_status, (size_t)d->lm_rows * sizeof(int)));
  }
  if (tail_shape_ok(g, d)) {
    const int E = g->n_embd;
    const size_t words = batch_tail_xch_words(E);
    EC_HIP(dev_malloc(&d->tail_xch, words * sizeof(unsigned long long)));
    EC_HIP(hipMemset(d->tail_xch, 0, words * sizeof(unsigned long long)));
    EC_HIP(dev_malloc(&d->d_tail_io, 8 * sizeof(int)));
    const int io0[8] = {1, 0, 0, 0, 0, 0, 0, 0};  // tag 1: the cleared words (tag 0) never match
    EC_HIP(hipMemcpy(d->d_tail_io, io0, sizeof io0, hipMemcpyHostToDevice));
    EC_HIP(host_malloc((void **)&d->h_tail_err, sizeof(int), hipHostMallocDefault));
    *d->h_tail_err = 0;
    d->tail_ok = true;
  }
  int kind = step_shape_kind(g, d);
  if (kind == 1) {  // the GPT-2 step adds every bias
    for (int l = 0; l < Lc; l++) {
      const LayerDev &W = d->L[l];
      if (!W.ln1_b || !W.ln2_b || !W.bqkv || !W.bo || !W.bfc || !W.bd) kind = -1;
    }
  }
  if (kind >= 0) {
    d->step_kind = kind;
    if (kind == 0) {
      std::vector<StepLayer> sl(Lc);
      for (int l = 0; l < Lc; l++) {
        const LayerDev &W = d->L[l];
        sl[l] = StepLayer{W.ln1_g, W.ln2_g, (const int8_t *)W.wqkv, W.sqkv, (const int8_t *)W.wo, W.so,
                          (const int8_t *)W.wg, (const int8_t *)W.wu, W.sg, W.su, (const int8_t *)W.wd, W.sd};
      }
      EC_HIP(dev_malloc(&d->d_layers, sl.size() * sizeof(StepLayer)));
      EC_HIP(hipMemcpy(d->d_layers, sl.data(), sl.size() * sizeof(StepLayer), hipMemcpyHostToDevice));
      d->xch_bytes = (size_t)Lc * 3 * (size_t)E * sizeof(unsigned long long);
      EC_HIP(dev_malloc(&d->xch, d->xch_bytes));
      d->ffv_words = (size_t)2 * Lc * F;
      EC_HIP(dev_malloc(&d->ffv, d->ffv_words * sizeof(float)));
    } else {
      std::vector<Step16Layer> sl(Lc);
      for (int l = 0; l < Lc; l++) {
        const LayerDev &W = d->L[l];
        sl[l] = Step16Layer{W.ln1_g, W.ln1_b, W.ln2_g, W.ln2_b, (const uint16_t *)W.wqkv, W.bqkv,
                            (const uint16_t *)W.wo, W.bo, (const uint16_t *)W.wfc, W.bfc, (const uint16_t *)W.wd, W.bd};
      }
      EC_HIP(dev_malloc(&d->d_layers16, sl.size() * sizeof(Step16Layer)));
      EC_HIP(hipMemcpy(d->d_layers16, sl.data(), sl.size() * sizeof(Step16Layer), hipMemcpyHostToDevice));
      d->xch_bytes = (size_t)Lc * kStep16Words * sizeof(unsigned long long);
      EC_HIP(dev_malloc(&d->xch, d->xch_bytes));
      d->ffv_words = (size_t)2 * Lc * F;
      EC_HIP(dev_malloc(&d->ffv, d->ffv_words * sizeof(float)));
    }
    EC_HIP(step_clear(d, nullptr));
    EC_HIP(hipDeviceSynchronize());
    EC_HIP(dev_malloc(&d->d_step_io, 8 * sizeof(int)));
    EC_HIP(hipMemset(d->d_step_io, 0, 8 * sizeof(int)));
    EC_HIP(host_malloc((void **)&d->h_step_io, 8 * sizeof(int), hipHostMallocDefault));
    memset(d->h_step_io, 0, 8 * sizeof(int));
    EC_HIP(dev_malloc(&d->d_gen, (size_t)d->eff_ctx * sizeof(int)));
    EC_HIP(dev_malloc(&d->d_gen_t, (size_t)(d->eff_ctx + 1) * sizeof(unsigned long long)));
    const char *tr = getenv("EDGECORE_STEP_TRACE");
    if (tr && !strcmp(tr, "1")) {
      const size_t tb = (size_t)kStepBlocks * Lc * kStepEvents * sizeof(unsigned long long);
      EC_HIP(dev_malloc(&d->d_trace, tb));
      EC_HIP(hipMemset(d->d_trace, 0, tb));
    }
    d->step_ok = true;
  }
  g->ws_x = d->x;
  g->ws_tmp = d->h;
  g->ws_qkv = d->qkv;
  g->ws_attn = d->att;
  g->ws_scores = nullptr;  // attention scores live in LDS
  g->ws_q = d->aq;
  g->ws_qs = d->as;
  g->ws_q_cols = (size_t)d->aq_ld;

  munmap(g->file_data, g->file_size);
  g->file_data = nullptr;
  g->file_size = 0;
  g->file_mapped = 0;
  return 0;
}

extern "C" int gpt2_load(GPT2 *g, const char *path, int batch_cap, int max_ctx) {
  const int r = load_impl(g, path, batch_cap, max_ctx);
  if (r) {
    fprintf(stderr, "%s\n", g_err);
    gpt2_free(g);
    return -1;
  }
  return 0;
}

extern "C" void gpt2_free(GPT2 *g) {
  if (!g) return;
  tokenizer_free(&g->tok);
  free(g->lw);
  free_dev(dev_detach(g));
  if (g->file_data && g->file_mapped) munmap(g->file_data, g->file_size);
  memset(g, 0, sizeof *g);
}

extern "C" int gpt2_kv_reset(GPT2 *g) {
  EC_INIT();
  DevModel *d = dev_of(g);
  if (!d) return set_err(-1, "gpt2_kv_reset: model not loaded");
  const size_t b = d->kv_layer * g->n_layer * sizeof(uint16_t);
  EC_HIP(hipMemsetAsync(d->kc, 0, b, g_stream));
  EC_HIP(hipMemsetAsync(d->vc, 0, b, g_stream));
  EC_HIP(hipStreamSynchronize(g_stream));
  return 0;
}

// One linear layer: the fused GEMV when the shape allows it; otherwise the
// prologue runs as its own kernel (norm / quantize into the aq or h
// workspace) and the generic kernel does the product.
// profiler family of a linear that runs on the matrix-core GEMM: "gemv_X" -> "gemm_X"
static const char *gemm_family(const char *fam) {
  static const char *const names[][2] = {{"gemv_qkv", "gemm_qkv"},       {"gemv_o", "gemm_o"},
                                         {"gemv_gateup", "gemm_gateup"}, {"gemv_fc", "gemm_fc"},
                                         {"gemv_down", "gemm_down"},     {"gemv_lmhead", "gemm_lmhead"}};
  for (const auto &n : names)
    if (!strcmp(fam, n[0])) return n[1];
  return "gemm_i8";
}

static int linear(GPT2 *g, DevModel *d, const char *fam, GemvArgs a, int wt, int epi, int pro, hipStream_t s) {
  const double bytes = gemv_bytes(wt, pro, epi, a.M, a.K, a.N, a.ws != nullptr, a.bias != nullptr);
  if (wt == WT_I8 && g_use_mfma && a.M >= kGemmMinM) {
    // batched decode: the quantization inside the skinny GEMM, from the
    // producer's partial row maxima
    if (pro == PRO_QUANT && a.pmax && (a.pmax != d->pmax_ff || d->ff_pmax) && gemm_i8_skinny_q_ok(a, epi)) {
      EC_LAUNCH(gemm_family(fam), bytes, gemm_i8_skinny_q(a, epi, s));
      return 0;
    }
    // many rows: the norm / quantization as its own pass into int8 rows, then
    // the matrix-core GEMM
    GemvArgs q = a;
    if (pro != PRO_I8) {
      q.A = d->aq;
      q.lda = d->aq_ld;
      q.as = d->as;
    }
    if (gemm_i8_ok(q, epi)) {
      const float *A = (const float *)a.A;
      if (pro == PRO_QUANT) {
        EC_LAUNCH("quant", 5.0 * a.M * a.K, quant_rows(A, a.lda, a.M, a.K, d->aq, d->aq_ld, d->as, s));
      } else if (pro == PRO_RMS || pro == PRO_LN) {
        EC_LAUNCH("norm_quant", 5.0 * a.M * a.K,
                  norm_rows(A, a.M, a.K, a.gamma, a.beta, g->eps, nullptr, 0, d->aq, d->aq_ld, d->as, s));
      }
      if (a.M <= 32) {
        EC_LAUNCH(gemm_family(fam), bytes, gemm_i8_skinny(q, epi, 0, s));
        if (a.pmax_out == d->pmax_ff) d->ff_pmax = a.pmax_out != nullptr;
      } else {
        EC_LAUNCH(gemm_family(fam), bytes, gemm_i8(q, epi, s));
        if (a.pmax_out == d->pmax_ff) d->ff_pmax = false;
      }
      return 0;
    }
  }
  if (wt != WT_I8 && g_use_mfma && a.M >= kGemmMinM && a.M <= d->ah_rows && a.K <= d->ah_ld &&
      gemm_w16_ok(a, wt, epi)) {
    // many rows, 16-bit weights: the norm as its own pass into fp32 rows, then
    // the matrix-core GEMM (which splits the rows into 16-bit parts first)
    GemvArgs q = a;
    if (pro == PRO_RMS || pro == PRO_LN) {
      EC_LAUNCH("norm", 8.0 * a.M * a.K,
                norm_rows((const float *)a.A, a.M, a.K, a.gamma, a.beta, g->eps, d->h, a.K, nullptr, 0, nullptr, s));
      q.A = d->h;
      q.lda = a.K;
    }
    EC_LAUNCH("split16", 4.0 * a.M * a.K * (1.0 + w16_parts(wt) / 2.0),
              split_rows16(q, wt, d->ah, d->ah_ld, d->ahs, s));
    EC_LAUNCH(gemm_family(fam), bytes, gemm_w16_parts(q, wt, epi, 0, d->ah, d->ah_ld, d->ahs, s));
    return 0;
  }
  if (a.pmax_out == d->pmax_ff) d->ff_pmax = false;  // the paths below leave the partial maxima unwritten
  if (gemv_vector_ok(a, wt, pro)) {
    EC_LAUNCH(fam, bytes, gemv(a, wt, epi, pro, s));
    return 0;
  }
  const float *A = (const float *)a.A;
  if (pro == PRO_QUANT) {
    EC_LAUNCH("quant", 5.0 * a.M * a.K, quant_rows(A, a.lda, a.M, a.K, d->aq, d->aq_ld, d->as, s));
  } else if ((pro == PRO_RMS || pro == PRO_LN) && wt == WT_I8) {
    EC_LAUNCH("norm_quant", 5.0 * a.M * a.K,
              norm_rows(A, a.M, a.K, a.gamma, a.beta, g->eps, nullptr, 0, d->aq, d->aq_ld, d->as, s));
  } else if (pro == PRO_RMS || pro == PRO_LN) {
    EC_LAUNCH("norm", 8.0 * a.M * a.K, norm_rows(A, a.M, a.K, a.gamma, a.beta, g->eps, d->h, a.K, nullptr, 0, nullptr, s));
  }
  if (wt == WT_I8 && pro != PRO_I8) {
    a.A = d->aq;
    a.lda = d->aq_ld;
    a.as = d->as;
  } else if (pro == PRO_RMS || pro == PRO_LN) {
    a.A = d->h;
    a.lda = a.K;
  }
  EC_LAUNCH(fam, bytes, gemv_generic(a, wt, epi, s));
  return 0;
}

// positions per attention product tile for launches with positions < max_npos
// (multiple of 4); below 4 the device LDS cannot hold the scores
static int attn_vtile(int max_npos, int hd, int kv) {
  const size_t lds_fixed = attention_lds_bytes(max_npos, hd, 0);
  if (lds_fixed >= (size_t)g_max_lds) return 0;
  const size_t room = ((size_t)g_max_lds - lds_fixed) / ((size_t)attn_pitch(hd, kv) * sizeof(float));
  const size_t cap = (size_t)attention_max_vtile(hd, kv);
  int vtile = (int)(room < cap ? room : cap) & ~3;
  if (vtile > ((max_npos + 3) & ~3)) vtile = (max_npos + 3) & ~3;
  return vtile;
}

// Enqueue one forward on stream s: the copy of the staged tokens / positions
// / slots, every kernel, and the copies of logits and argmax ids into the
// given host buffers (either may be null).  max_npos bounds pos + 1 over the
// batch and sizes the attention LDS; distinct: no two tokens share a slot
// (RoPE and the KV append then run inside attention); abytes: algorithmic
// attention bytes, for the profiler only.
// LDS the persistent step reserves outside the dynamic area (its static arrays)
constexpr size_t kStepStaticLds = 4096;

// the attention area of the step's dynamic LDS (the attention kernel's
// layout, with room for the prefetched V tile), rounded to 16 bytes; the
// attention blocks' row and codes follow it
static size_t step_attn_area(int max_npos, int vtile, int kv) {
  const size_t a = attention_lds_bytes(max_npos, 64, vtile);
  const size_t prod = (3 * 64 + (size_t)((max_npos + 3) & ~3)) * sizeof(float);
  const size_t v = prod + step_vtile_off(vtile, kv) + (size_t)vtile * 32;
  return ((a > v ? a : v) + 15) & ~(size_t)15;
}

// LDS the int8 Qwen2 step uses past the attention area: the attention
// blocks' norm row and codes
static size_t step_row_bytes(const GPT2 *g, const DevModel *d) {
  (void)d;
  return step_norm_bytes(g->n_embd);
}

// the attention product tile of the persistent step for max_npos positions
// (attn_vtile with the step's static LDS and the attention blocks' rows set
// aside, and room for the V tile)
static int step_vtile(const GPT2 *g, const DevModel *d, int max_npos) {
  if (d->step_kind == 1) return max_npos <= kStep16MaxPos ? 4 : 0;  // no LDS tile: any value >= 4 means it fits
  const int kv = g->n_kv_embd;
  const size_t budget = (size_t)g_max_lds - kStepStaticLds - step_row_bytes(g, d);
  const size_t lds_fixed = attention_lds_bytes(max_npos, 64, 0);
  if (lds_fixed >= budget) return 0;
  const size_t room = (budget - lds_fixed) / ((size_t)attn_pitch(64, 0) * sizeof(float));
  const size_t cap = (size_t)attention_max_vtile(64, 128);
  int vtile = (int)(room < cap ? room : cap) & ~3;
  if (vtile > ((max_npos + 3) & ~3)) vtile = (max_npos + 3) & ~3;
  while (vtile >= 4 && step_attn_area(max_npos, vtile, kv) > budget) vtile -= 4;
  return vtile;
}

static size_t step_lds(const GPT2 *g, const DevModel *d, int max_npos, int vtile) {
  if (d->step_kind == 1) return decode_step_gpt2_scratch_bytes();  // its attention keeps K / V in registers
  const size_t a = step_attn_area(max_npos, vtile, g->n_kv_embd) + step_row_bytes(g, d),
               b = d->step_kind == 1 ? decode_step_gpt2_scratch_bytes() : decode_step_scratch_bytes(g->n_embd, d->F);
  return a > b ? a : b;
}

// algorithmic bytes of one persistent step: every layer's weights and row
// scales (int8) or biases (fp16) once, plus the K/V rows its attention reads
static double step_bytes(const GPT2 *g, const DevModel *d, int npos) {
  const double E = g->n_embd, F = d->F, kv = g->n_kv_embd;
  if (d->step_kind == 1) {
    const double w = 3 * E * E + E * E + 2 * F * E, b = 3 * E + E + F + E + 4 * E;
    return g->n_layer * (2 * w + 4 * b + (double)npos * kv * 4);
  }
  const double rows = (E + 2 * kv) + E + 2 * F + E;
  const double w = E * (E + 2 * kv) + E * E + 2 * F * E + F * E;
  return g->n_layer * (w + 4 * rows + (double)npos * kv * 4);
}

// The layers of a one-token forward as one persistent launch (decode_step.hip);
// x after the last layer lands in d->x.
static int enqueue_step(GPT2 *g, DevModel *d, int max_npos, hipStream_t s) {
  const int vtile = step_vtile(g, d, max_npos);
  if (vtile < 4) return set_err(-1, "decode step: position %d does not fit the LDS", max_npos - 1);
  if (!d->chaining)  // a chained step's inputs were written by the previous step
    EC_HIP(hipMemcpyAsync(d->d_step_io, d->h_step_io, 4 * sizeof(int), hipMemcpyHostToDevice, s));
  int *io = d->d_step_io;
  AttnArgs aa{};
  aa.kc = d->kc;
  aa.vc = d->vc;
  aa.kc_w = d->kc;
  aa.vc_w = d->vc;
  aa.pos = io + 1;
  aa.slot = io + 2;
  aa.H = g->n_head;
  aa.KVH = g->n_kv_head;
  aa.hd = 64;
  aa.kv = g->n_kv_embd;
  aa.C = d->eff_ctx;
  aa.window = g->sliding_window;
  aa.inv_hd = 1.0 / sqrt(64.0);
  aa.M = 1;
  aa.max_npos = max_npos;
  aa.vtile = vtile;
  aa.fuse_kv = 1;
  aa.cs = g->arch == ARCH_QWEN2 ? d->rope : nullptr;  // GPT-2: no rotation
  aa.half = d->half;
  const size_t lds = step_lds(g, d, max_npos, vtile);
  // decode_step is a cooperative launch (not through klaunch): its profiler
  // events are recorded on the stream around it
  const int p_ = prof_begin("decode_step", step_bytes(g, d, max_npos));
  hipEvent_t e0 = g_launch_ev[0], e1 = g_launch_ev[1];
  g_launch_ev[0] = g_launch_ev[1] = nullptr;
  if (e0) EC_HIP(hipEventRecord(e0, s));
  hipError_t e;
  if (d->step_kind == 1) {
    const Step16Args sa{d->d_layers16, g->wte, g->wpe, g->n_layer, g->eps, d->kv_layer, io,
                        reinterpret_cast<const unsigned *>(io + 3), d->xch, d->x, io + 4, d->d_trace, d->ffv, aa};
    e = decode_step_gpt2(sa, lds, g_step_coop, s);
  } else {
    const StepArgs sa{d->d_layers, g->wte, g->n_layer, g->n_embd, g->n_head, g->n_kv_head, d->F, g->eps,
                      d->kv_layer, io, reinterpret_cast<const unsigned *>(io + 3), d->xch, d->x, io + 4, d->d_trace,
                      aa, (int)(step_attn_area(max_npos, vtile, g->n_kv_embd) / sizeof(float)), d->ffv};
    e = decode_step(sa, lds, g_step_coop, s);
  }
  if (e0 && e == hipSuccess) EC_HIP(hipEventRecord(e1, s));
  if (e != hipSuccess) {
    if (p_ >= 0) {
      g_prof.pop_back();
      g_ev_used -= 2;
    }
    return set_err(-3, "decode_step launch failed: %s", hipGetErrorString(e));
  }
  return 0;
}

// The batched layer tail applies: up to kTailMaxM tokens, each in its own
// slot (the attention appends each token's k / v itself), not a prefill
static bool use_tail(const DevModel *d, int M, bool run, bool distinct) {
  return d->tail_ok && !run && distinct && M <= kTailMaxM;
}

// After a forward through the layer tail: 1 if one of its waits timed out (a
// block that never became resident) -- the flag is cleared, the tail turned
// off and the captured graphs dropped, and the forward is to be redone
// through the separate kernels; -1 if clearing failed; 0 otherwise
static int tail_timed_out(DevModel *d) {
  bool fail = *d->h_tail_err != 0;
  if (g_tail_test_fail) {
    g_tail_test_fail = false;
    fail = true;
  }
  if (!fail) return 0;
  *d->h_tail_err = 0;
  if (hipMemset(d->d_tail_io + 2, 0, sizeof(int)) != hipSuccess || hipDeviceSynchronize() != hipSuccess) return -1;
  d->tail_ok = false;
  for (auto &dg : d->dec_graphs) (void)hipGraphExecDestroy(dg.exec);
  d->dec_graphs.clear();
  fprintf(stderr, "edgecore: a batched layer tail's blocks were not all resident; separate kernels from now on\n");
  return 1;
}

static int enqueue_forward(GPT2 *g, DevModel *d, int M, int lm_from, bool distinct, bool run, int max_npos,
                           double abytes, float *logits, int *argmax, const TopkReq *tk, hipStream_t s,
                           bool step = false) {
  const int E = g->n_embd, H = g->n_head, V = g->vocab, kv = g->n_kv_embd, hd = g->head_dim;
  const bool qwen = g->arch == ARCH_QWEN2, i8 = g->precision == 0, bf16 = g->precision == 2;
  const int wt = i8 ? WT_I8 : (bf16 ? WT_BF16 : WT_F16);
  const int pro_norm = qwen ? PRO_RMS : PRO_LN;
  const int vtile = attn_vtile(max_npos, hd, kv);
  if (vtile < 4)
    return set_err(-1, "position %d needs more LDS for attention scores than the device has (%d bytes)",
                   max_npos - 1, g_max_lds);
  const int *st = d->h_stage;
  if (!step) {
    EC_HIP(hipMemcpyAsync(d->d_tok, st, (size_t)M * 4, hipMemcpyHostToDevice, s));
    EC_HIP(hipMemcpyAsync(d->d_pos, st + d->mmax, (size_t)M * 4, hipMemcpyHostToDevice, s));
    EC_HIP(hipMemcpyAsync(d->d_slot, st + 2 * d->mmax, (size_t)M * 4, hipMemcpyHostToDevice, s));
  }

  int r;
  if (step && (r = enqueue_step(g, d, max_npos, s))) return r;
  if (!step)
    EC_LAUNCH("embed", (double)M * E * (g->wpe ? 8 : 6),
              embed(g->wte, g->wpe, bf16, d->d_tok, d->d_pos, M, E, d->x, s));

  const int F = d->F, ldq = d->qkv_ld;
  const int nqkv = qwen ? E + 2 * kv : 3 * E;
  // batched decode of 16-32 tokens: o and down quantize inside their GEMMs
  const bool fq = d->fuse_quant && i8 && g_use_mfma && !run && M >= kGemmMinM && M <= 32;
  // a decode of up to 4 tokens: each layer's o, MLP and the next layer's
  // q|k|v in one launch (decode_tail.hip)
  const bool tail = !step && use_tail(d, M, run, distinct);
  bool touched = false;
  for (int l = 0; l < (step ? 0 : g->n_layer); l++) {
    const LayerDev &W = d->L[l];
    uint16_t *kcl = d->kc + d->kv_layer * l, *vcl = d->vc + d->kv_layer * l;
    // norm -> q|k|v projection (GPT-2 bias: inside the int8 epilogue, a bias pass for 16-bit);
    // after the first layer the layer tail has computed it
    if (!tail || l == 0) {
      GemvArgs a{d->x, E, nullptr, W.ln1_g, W.ln1_b, g->eps, W.wqkv, nullptr, W.sqkv, nullptr, W.bqkv,
                 d->qkv, ldq, M, E, nqkv, nullptr};
      const int epi = (!i8 && W.bqkv) ? EPI_BIAS : EPI_STORE;
      if ((r = linear(g, d, "gemv_qkv", a, wt, epi, pro_norm, s))) return r;
    }
    float *kq = d->qkv + E, *vq = d->qkv + E + (qwen ? kv : E);
    if (!distinct) {  // RoPE (Qwen2) + fp16 KV append
      KvArgs ka{d->qkv, kq, vq, ldq, ldq, H, g->n_kv_head, hd, kv, qwen ? d->rope : nullptr, d->half,
                d->d_pos, d->d_slot, kcl, vcl, d->eff_ctx, M};
      EC_LAUNCH("rope_kv", (double)M * (qwen ? (E + kv) * 8 + kv * 8 : kv * 12), rope_kv_append(ka, s));
    }
    AttnArgs aa{d->qkv, ldq, kcl, vcl, d->att, E, d->d_pos, d->d_slot, H, g->n_kv_head, hd, kv,
                d->eff_ctx, qwen ? g->sliding_window : 0, 1.0 / sqrt((double)hd), M, max_npos, vtile,
                distinct ? 1 : 0, kq, vq, ldq, (distinct && qwen) ? d->rope : nullptr, d->half, kcl, vcl};
    if (!run && M <= g->batch_cap) {  // long decode contexts: scores pass, then softmax / sums
      aa.scores = d->att_sc;
      aa.sc_ld = d->eff_ctx;
    }
    if (fq) {
      aa.pmax = d->pmax_att;
      aa.np = d->np_att;
    }
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    if (g_touch && run && M >= kTouchMinRows && hipStreamIsCapturing(s, &cap) == hipSuccess &&
        cap == hipStreamCaptureStatusNone) {
      // this layer's o / MLP weights and the next layer's q|k|v rows into
      // the memory-side cache while the attention runs
      const size_t eb = i8 ? 1 : 2;
      TouchArgs ta{};
      ta.sink = g_touch_sink;
      auto add = [&](const void *w, int rows, int cols) {
        if (w && ta.n_ranges < kTouchRanges && (cols * eb) % 16 == 0) {
          ta.p[ta.n_ranges] = (const uint4 *)w;
          ta.rows[ta.n_ranges] = rows;
          ta.row16[ta.n_ranges++] = (int)(cols * eb / 16);
        }
      };
      add(W.wo, E, E);
      if (qwen) {
        add(W.wg, F, E);
        add(W.wu, F, E);
      } else {
        add(W.wfc, F, E);
      }
      add(W.wd, E, F);
      if (l + 1 < g->n_layer) add(d->L[l + 1].wqkv, nqkv, E);
      hipEvent_t ev = g_touch_ev[g_touch_i++ & 3];
      EC_HIP(hipEventRecord(ev, s));
      EC_HIP(hipStreamWaitEvent(g_side, ev, 0));
      EC_HIP(touch_ranges(ta, g_touch_blocks, g_side));
      touched = true;
    }
    if (run && attention_prefill_ok(aa, g_max_lds)) {
      EC_LAUNCH("attention_prefill", abytes, attention_prefill(aa, g_max_lds, s));
    } else if (attention_split_ok(aa)) {
      EC_LAUNCH("attention_scores", abytes / 2, attention_scores(aa, s));
      EC_LAUNCH("attention", abytes / 2, attention_after_scores(aa, s));
    } else {
      EC_LAUNCH("attention", abytes, attention(aa, s));
    }
    if (tail) {
      const bool nx = l + 1 < g->n_layer;
      const LayerDev &Wn = d->L[nx ? l + 1 : l];
      const BatchTailArgs ta{(const int8_t *)W.wo, W.so, W.bo, W.ln2_g, (const int8_t *)W.wg, (const int8_t *)W.wu,
                             W.sg, W.su, (const int8_t *)W.wd, W.sd, W.bd, nx ? Wn.ln1_g : nullptr,
                             nx ? (const int8_t *)Wn.wqkv : nullptr, nx ? Wn.sqkv : nullptr, nx ? Wn.bqkv : nullptr,
                             d->att, d->x, d->qkv, ldq, M, E, F, nqkv, g->eps, d->tail_xch,
                             reinterpret_cast<unsigned *>(d->d_tail_io), reinterpret_cast<unsigned *>(d->d_tail_io + 1),
                             d->d_tail_io + 2};
      const double tb = (double)E * E + 3.0 * F * E + (nx ? (double)nqkv * E : 0.0) + 8.0 * M * E;
      EC_LAUNCH("decode_tail", tb, batch_tail(ta, g_step_coop, s));
      continue;
    }
    // output projection + residual
    {
      GemvArgs a{d->att, E, nullptr, nullptr, nullptr, 0.0, W.wo, nullptr, W.so, nullptr, W.bo, d->x, E, M, E, E,
                 nullptr};
      if (fq) {
        a.pmax = d->pmax_att;
        a.np = d->np_att;
      }
      const int epi = i8 ? EPI_RESID : (W.bo ? EPI_BIAS_RESID : EPI_RESID);
      if ((r = linear(g, d, "gemv_o", a, wt, epi, i8 ? PRO_QUANT : PRO_F32, s))) return r;
    }
    // MLP up: SwiGLU gate/up (Qwen2) or fc + GELU (GPT-2), norm fused
    if (qwen) {
      GemvArgs a{d->x, E, nullptr, W.ln2_g, nullptr, g->eps, W.wg, W.wu, W.sg, W.su, nullptr, d->ff, F, M, E, F,
                 nullptr};
      if (fq) {
        a.pmax_out = d->pmax_ff;
        a.np_out = d->np_ff;
      }
      if ((r = linear(g, d, "gemv_gateup", a, wt, EPI_SWIGLU, PRO_RMS, s))) return r;
    } else {
      GemvArgs a{d->x, E, nullptr, W.ln2_g, W.ln2_b, g->eps, W.wfc, nullptr, W.sfc, nullptr, W.bfc, d->ff, F, M,
                 E, F, nullptr};
      if (fq) {
        a.pmax_out = d->pmax_ff;
        a.np_out = d->np_ff;
      }
      if ((r = linear(g, d, "gemv_fc", a, wt, i8 ? EPI_GELU : EPI_BIAS_GELU, PRO_LN, s))) return r;
    }
    // MLP down + residual
    {
      GemvArgs a{d->ff, F, nullptr, nullptr, nullptr, 0.0, W.wd, nullptr, W.sd, nullptr, W.bd, d->x, E, M, F, E,
                 nullptr};
      if (fq) {
        a.pmax = d->pmax_ff;
        a.np = d->np_ff;
      }
      const int epi = i8 ? EPI_RESID : (W.bd ? EPI_BIAS_RESID : EPI_RESID);
      if ((r = linear(g, d, "gemv_down", a, wt, epi, i8 ? PRO_QUANT : PRO_F32, s))) return r;
    }
  }
  if (tail) EC_HIP(hipMemcpyAsync(d->h_tail_err, d->d_tail_io + 2, sizeof(int), hipMemcpyDeviceToHost, s));
  if (touched) {  // the side stream's reads end before anything after this forward
    hipEvent_t ev = g_touch_ev[g_touch_i++ & 3];
    EC_HIP(hipEventRecord(ev, g_side));
    EC_HIP(hipStreamWaitEvent(s, ev, 0));
  }
  // final norm fused into the LM head (always fp16/bf16, src/gpt2.c:576-580 / 799-804);
  // greedy ids from per-block argmax candidates
  const int lwt = bf16 ? WT_BF16 : WT_F16;
  int *amax_dev = step ? d->d_step_io + 5 : d->d_amax;  // a step's id goes out with its error flag
  bool advanced = false;  // a chained step's inputs were advanced by the argmax launch
  for (int r0 = lm_from; r0 < M; r0 += d->lm_rows) {
    const int rows = M - r0 < d->lm_rows ? M - r0 : d->lm_rows;
    GemvArgs a{d->x + (size_t)r0 * E, E, nullptr, g->lnf_g, g->lnf_b, g->eps, d->lm, nullptr, nullptr, nullptr,
               nullptr, d->logits, V, rows, E, V, nullptr};
    // the matrix-core GEMM (many rows: the weights stream once) leaves the
    // argmax to argmax_rows; the fused GEMV keeps per-block candidates
    const bool mfma = g_use_mfma && rows >= kGemmMinM && rows <= d->ah_rows && E <= d->ah_ld &&
                      gemm_w16_ok(a, lwt, EPI_STORE);
    const bool fused = !mfma && gemv_vector_ok(a, lwt, pro_norm);
    if (argmax && fused) a.cand = d->cand;
    if ((r = linear(g, d, "gemv_lmhead", a, lwt, EPI_STORE, pro_norm, s))) return r;
    if (argmax) {
      if (fused) {
        // a chained step advances its inputs in the same launch
        const bool adv = step && d->chaining;
        EC_LAUNCH("argmax", 8.0 * rows * gemv_grid_x(a, lwt, EPI_STORE),
                  argmax_finalize(d->cand, gemv_grid_x(a, lwt, EPI_STORE), d->logits, V, rows,
                                  amax_dev + (r0 - lm_from), s, adv ? d->d_step_io : nullptr,
                                  adv ? d->d_gen : nullptr, adv ? d->d_gen_t : nullptr));
        if (adv) advanced = true;
      } else {
        int nc = 0;
        EC_LAUNCH("argmax_chunks", 4.0 * rows * V, argmax_chunks(d->logits, rows, V, d->cand, d->ncand, &nc, s));
        EC_LAUNCH("argmax", 8.0 * rows * nc,
                  argmax_finalize(d->cand, nc, d->logits, V, rows, amax_dev + (r0 - lm_from), s));
      }
    }
    if (logits)
      EC_HIP(hipMemcpyAsync(logits + (size_t)(r0 - lm_from) * V, d->logits, (size_t)rows * V * 4,
                            hipMemcpyDeviceToHost, s));
    if (tk) {
      const int n = tk->top_k + 1, ro = r0 - lm_from;
      EC_LAUNCH("topk_select", 4.0 * rows * V,
                topk_select(d->logits, rows, V, V, tk->top_k, d->tk_cand, d->tk_nan, s));
      EC_LAUNCH("topk_merge", 8.0 * rows * topk_chunks(V) * n,
                topk_merge(d->tk_cand, d->tk_nan, rows, V, tk->top_k, d->tk_vals, d->tk_idx, d->tk_status, s));
      EC_HIP(hipMemcpyAsync(tk->vals + (size_t)ro * n, d->tk_vals, (size_t)rows * n * 4, hipMemcpyDeviceToHost, s));
      EC_HIP(hipMemcpyAsync(tk->idx + (size_t)ro * n, d->tk_idx, (size_t)rows * n * 4, hipMemcpyDeviceToHost, s));
      EC_HIP(hipMemcpyAsync(tk->status + ro, d->tk_status, (size_t)rows * 4, hipMemcpyDeviceToHost, s));
    }
    d->last_lm_rows = rows;
  }
  if (step && d->chaining) {  // nothing goes to the host: the next step reads its inputs on the device
    if (!advanced) EC_HIP(step_advance(d->d_step_io, d->d_gen, s, d->d_gen_t));
  } else if (step) {
    EC_HIP(hipMemcpyAsync(d->h_step_io + 4, d->d_step_io + 4, 2 * sizeof(int), hipMemcpyDeviceToHost, s));
  }
  else if (argmax && lm_from < M)
    EC_HIP(hipMemcpyAsync(argmax, d->d_amax, (size_t)(M - lm_from) * 4, hipMemcpyDeviceToHost, s));
  return 0;
}

// After a step whose waits timed out: clear the flag; if the step ran as a
// plain launch, switch to cooperative launches (captured graphs dropped) and
// return 1 (redo the step), else 0 (a real failure)
static int step_timed_out(DevModel *d) {
  int *io = d->h_step_io;
  io[4] = 0;
  if (hipMemset(d->d_step_io + 4, 0, sizeof(int)) != hipSuccess) return 0;
  // the redo must not find FFN words of the abandoned launch
  if (step_clear(d, nullptr) != hipSuccess || hipDeviceSynchronize() != hipSuccess) return 0;
  if (g_step_coop) return 0;
  g_step_coop = true;
  if (d->step_graph) (void)hipGraphExecDestroy(d->step_graph);
  for (int i = 0; i < 2; i++) {
    if (d->chain_graph[i]) (void)hipGraphExecDestroy(d->chain_graph[i]);
    d->chain_graph[i] = nullptr;
    d->chain_bucket[i] = 0;
  }
  d->step_graph = nullptr;
  d->step_bucket = 0;
  fprintf(stderr, "edgecore: a decode step's blocks were not all resident; cooperative launches from now on\n");
  return 1;
}

// chained greedy steps per graph launch when they fit one bucket
constexpr int kChainBurst = 16;

// the host-side stand-in for a timed-out plain step (EDGECORE_STEP_TEST_FAIL=1)
static bool step_test_fail() {
  if (!g_step_test_fail || g_step_coop) return false;
  g_step_test_fail = false;
  return true;
}

static int forward_impl(GPT2 *g, const int *tokens, const int *positions, const int *seqs, int M,
                        int lm_from, float *logits, int *argmax, const TopkReq *tk = nullptr) {
  EC_INIT();
  DevModel *d = dev_of(g);
  if (!d) return set_err(-1, "model not loaded");
  if (M < 1 || M > d->mmax) return set_err(-1, "M=%d outside [1, %d]", M, d->mmax);
  if (lm_from < 0 || lm_from > M) return set_err(-1, "lm_from=%d outside [0, %d]", lm_from, M);
  if (!tokens || !positions) return set_err(-1, "null tokens/positions");
  const int E = g->n_embd, V = g->vocab, kv = g->n_kv_embd, hd = g->head_dim;
  int *st = d->h_stage;
  int max_npos = 0;
  for (int m = 0; m < M; m++) {
    if (tokens[m] < 0 || tokens[m] >= V) return set_err(-1, "token %d at row %d outside [0, %d)", tokens[m], m, V);
    if (positions[m] < 0 || positions[m] >= d->eff_ctx)
      return set_err(-1, "position %d at row %d outside [0, %d)", positions[m], m, d->eff_ctx);
    int slot = seqs ? seqs[m] : m;
    if (slot < 0) return set_err(-1, "negative slot %d at row %d", slot, m);
    if (slot >= g->batch_cap) slot = g->batch_cap - 1;  // src/gpt2.c:512-513
    st[m] = tokens[m];
    st[d->mmax + m] = positions[m];
    st[2 * d->mmax + m] = slot;
    if (positions[m] + 1 > max_npos) max_npos = positions[m] + 1;
  }
  if (hd > 256) return set_err(-1, "head_dim %d above 256 is not supported", hd);
  if (attn_vtile(max_npos, hd, kv) < 4)
    return set_err(-1, "position %d needs more LDS for attention scores than the device has (%d bytes)",
                   max_npos - 1, g_max_lds);
  // RoPE and the KV append run inside attention when no token of the batch
  // reads another token's slot (decode); otherwise as their own kernel first
  bool distinct = true;
  for (int m = 0; m < M && distinct; m++)
    for (int j = 0; j < m; j++)
      if (st[2 * d->mmax + j] == st[2 * d->mmax + m]) {
        distinct = false;
        break;
      }
  // one slot's run of consecutive positions (a prefill): the prefill attention
  bool run = M > 1;
  for (int m = 1; m < M && run; m++)
    run = st[2 * d->mmax + m] == st[2 * d->mmax] && st[d->mmax + m] == st[d->mmax] + m;
  double abytes = 0;
  for (int m = 0; m < M; m++) abytes += (double)(positions[m] + 1) * kv * 4 + 8.0 * E;
  hipStream_t s = g_stream;

  // The single-token greedy step (the decode loop) runs as one HIP graph: the
  // staging copies, every kernel and the copy of the argmax id, captured once
  // per 512-position bucket (the attention LDS is sized for the bucket; the
  // kernels read position and slot from device memory).  The host writes the
  // token / position / slot into the pinned stage before each replay.
  int bucket = (max_npos + 511) / 512 * 512;
  if (bucket > d->eff_ctx) bucket = d->eff_ctx;
  if (tk && !topk_ok(V, tk->top_k))
    return set_err(-1, "top_k=%d outside (0, %d) or above %d", tk->top_k, V, kTopkMax);
  const bool step = M == 1 && lm_from == 0 && d->step_ok && step_vtile(g, d, max_npos) >= 4;
  if (step) {
    // one token through the persistent step: its inputs and the step's tag
    // into the pinned I/O block, then -- for a greedy step without logits --
    // a HIP graph of the copy in, the step, the LM head, the argmax and the
    // copy out, captured once per 512-position bucket (the attention LDS is
    // sized for the bucket; the kernels read token, position and slot from
    // device memory); otherwise the same launches directly
    int *io = d->h_step_io;
    io[0] = st[0];
    io[1] = st[d->mmax];
    io[2] = st[2 * d->mmax];
    if (++d->step_tag == 0) {  // after 2^32 steps: clear the words of the old tags
      EC_HIP(step_clear(d, s));
      d->step_tag = 1;
    }
    io[3] = (int)d->step_tag;
    io[4] = io[5] = 0;
    bool graph = argmax && !logits && !tk && !g_prof_on && g_use_graphs && !d->step_nograph &&
                 step_vtile(g, d, bucket) >= 4;
    if (graph && (!d->step_graph || d->step_bucket != bucket)) {
      if (d->step_graph) {
        EC_HIP(hipGraphExecDestroy(d->step_graph));
        d->step_graph = nullptr;
      }
      // a runtime that cannot capture the cooperative launch leaves the
      // step to direct launches from then on
      hipGraph_t gr = nullptr;
      hipError_t e = hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal);
      int r = 0;
      if (e == hipSuccess) {
        r = enqueue_forward(g, d, 1, 0, true, false, bucket, abytes, nullptr, argmax, nullptr, s, true);
        e = hipStreamEndCapture(s, &gr);
      }
      if (e == hipSuccess && r == 0) e = hipGraphInstantiate(&d->step_graph, gr, nullptr, nullptr, 0);
      if (gr) (void)hipGraphDestroy(gr);
      if (e != hipSuccess || r != 0) {
        fprintf(stderr, "edgecore: the decode step could not be captured as a HIP graph (%s); launching it "
                "directly\n", r ? g_err : hipGetErrorString(e));
        (void)hipGetLastError();
        d->step_graph = nullptr;
        d->step_nograph = true;
        graph = false;
        g_err[0] = 0;
      } else {
        d->step_bucket = bucket;
      }
    }
    if (graph) {
      EC_HIP(hipGraphLaunch(d->step_graph, s));
    } else {
      const int r = enqueue_forward(g, d, M, lm_from, distinct, run, max_npos, abytes, logits, argmax, tk, s, true);
      if (r) return r;
    }
    EC_HIP(hipStreamSynchronize(s));
    if (io[4] || step_test_fail()) {
      if (step_timed_out(d)) return forward_impl(g, tokens, positions, seqs, M, lm_from, logits, argmax, tk);
      return set_err(-3, "decode step: a block's wait for another's results timed out (results discarded)");
    }
    if (argmax) argmax[0] = io[5];
    return 0;
  }
  // a greedy decode step of M tokens, each in its own slot: one HIP graph per
  // (M, bucket) of the staging copies, every kernel and the copy of the M
  // argmax ids into pinned memory
  if (lm_from == 0 && argmax && !logits && !tk && !g_prof_on && g_use_graphs && distinct && !run &&
      M <= g->batch_cap && attn_vtile(bucket, hd, kv) >= 4) {
    hipGraphExec_t ex = nullptr;
    for (const auto &dg : d->dec_graphs)
      if (dg.M == M && dg.bucket == bucket) ex = dg.exec;
    if (!ex) {
      constexpr size_t kMaxGraphs = 8;
      if (d->dec_graphs.size() >= kMaxGraphs) {
        EC_HIP(hipGraphExecDestroy(d->dec_graphs.front().exec));
        d->dec_graphs.erase(d->dec_graphs.begin());
      }
      EC_HIP(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal));
      const int r = enqueue_forward(g, d, M, 0, true, false, bucket, abytes, nullptr, d->h_amax, nullptr, s);
      hipGraph_t graph = nullptr;
      const hipError_t e = hipStreamEndCapture(s, &graph);
      if (r) {
        if (graph) (void)hipGraphDestroy(graph);
        return r;
      }
      EC_HIP(e);
      const hipError_t ei = hipGraphInstantiate(&ex, graph, nullptr, nullptr, 0);
      (void)hipGraphDestroy(graph);
      EC_HIP(ei);
      d->dec_graphs.push_back({M, bucket, ex});
    }
    EC_HIP(hipGraphLaunch(ex, s));
    EC_HIP(hipStreamSynchronize(s));
    if (use_tail(d, M, run, distinct)) {
      const int tr = tail_timed_out(d);
      if (tr > 0) return forward_impl(g, tokens, positions, seqs, M, lm_from, logits, argmax, tk);
      if (tr < 0) return set_err(-3, "batched decode: clearing a timed-out layer tail failed");
    }
    memcpy(argmax, d->h_amax, (size_t)M * sizeof(int));
    return 0;
  }
  const bool tail = use_tail(d, M, run, distinct);
  const int r = enqueue_forward(g, d, M, lm_from, distinct, run, max_npos, abytes, logits, argmax, tk, s);
  if (r) return r;
  EC_HIP(hipStreamSynchronize(s));
  if (tail) {
    const int tr = tail_timed_out(d);
    if (tr > 0) return forward_impl(g, tokens, positions, seqs, M, lm_from, logits, argmax, tk);
    if (tr < 0) return set_err(-3, "batched decode: clearing a timed-out layer tail failed");
  }
  return 0;
}

extern "C" int gpt2_forward_ex(GPT2 *g, const int *tokens, const int *positions, const int *seqs, int M,
                               int lm_from, float *logits, int *argmax) {
  return forward_impl(g, tokens, positions, seqs, M, lm_from, logits, argmax);
}

extern "C" int gpt2_forward_topk(GPT2 *g, const int *tokens, const int *positions, const int *seqs, int M,
                                 int lm_from, int top_k, float *vals, int *idx, int *status) {
  if (lm_from < M && (!vals || !idx || !status)) return set_err(-1, "gpt2_forward_topk: null output");
  const TopkReq tk{top_k, vals, idx, status};
  return forward_impl(g, tokens, positions, seqs, M, lm_from, nullptr, nullptr, &tk);
}

extern "C" int ec_topk_max(void) { return kTopkMax; }

extern "C" int ec_step_trace(GPT2 *g, unsigned long long *out, size_t n) {
  EC_INIT();
  DevModel *d = dev_of(g);
  if (!d) return set_err(-1, "model not loaded");
  if (!d->d_trace) return set_err(-1, "ec_step_trace: load the model with EDGECORE_STEP_TRACE=1");
  const size_t need = (size_t)kStepBlocks * g->n_layer * kStepEvents;
  if (!out || n < need) return set_err(-1, "ec_step_trace: %zu words needed", need);
  EC_HIP(hipMemcpy(out, d->d_trace, need * sizeof(unsigned long long), hipMemcpyDeviceToHost));
  return (int)need;
}

extern "C" int ec_last_logits(GPT2 *g, int row, float *out) {
  EC_INIT();
  DevModel *d = dev_of(g);
  if (!d) return set_err(-1, "model not loaded");
  if (!out || row < 0 || row >= d->last_lm_rows)
    return set_err(-1, "ec_last_logits: row %d outside the last LM-head chunk (%d rows)", row, d->last_lm_rows);
  EC_HIP(hipMemcpyAsync(out, d->logits + (size_t)row * g->vocab, (size_t)g->vocab * 4, hipMemcpyDeviceToHost,
                        g_stream));
  EC_HIP(hipStreamSynchronize(g_stream));
  return 0;
}

extern "C" int ec_topk_dev(const float *logits, int rows, int vocab, int ld, int top_k, float *vals, int *idx,
                           int *status) {
  EC_INIT();
  if (rows < 0 || ld < vocab) return set_err(-1, "ec_topk_dev: rows=%d ld=%d vocab=%d", rows, ld, vocab);
  if (rows == 0) return 0;
  if (!topk_ok(vocab, top_k))
    return set_err(-1, "ec_topk_dev: top_k=%d outside (0, %d) or above %d", top_k, vocab, kTopkMax);
  if (!logits || !vals || !idx || !status) return set_err(-1, "ec_topk_dev: null pointer");
  const int nb = topk_chunks(vocab), n = top_k + 1;
  unsigned long long *cand = nullptr;
  unsigned char *nanf = nullptr;
  float *dv = nullptr;
  int *di = nullptr, *ds = nullptr;
  hipError_t e = dev_malloc(&cand, (size_t)rows * nb * n * sizeof(unsigned long long));
  if (e == hipSuccess) e = dev_malloc(&nanf, (size_t)rows * nb);
  if (e == hipSuccess) e = dev_malloc(&dv, (size_t)rows * n * 4);
  if (e == hipSuccess) e = dev_malloc(&di, (size_t)rows * n * 4);
  if (e == hipSuccess) e = dev_malloc(&ds, (size_t)rows * 4);
  if (e == hipSuccess) e = topk_select(logits, rows, vocab, ld, top_k, cand, nanf, g_stream);
  if (e == hipSuccess) e = topk_merge(cand, nanf, rows, vocab, top_k, dv, di, ds, g_stream);
  if (e == hipSuccess) e = hipMemcpyAsync(vals, dv, (size_t)rows * n * 4, hipMemcpyDeviceToHost, g_stream);
  if (e == hipSuccess) e = hipMemcpyAsync(idx, di, (size_t)rows * n * 4, hipMemcpyDeviceToHost, g_stream);
  if (e == hipSuccess) e = hipMemcpyAsync(status, ds, (size_t)rows * 4, hipMemcpyDeviceToHost, g_stream);
  if (e == hipSuccess) e = hipStreamSynchronize(g_stream);
  for (void *p : {(void *)cand, (void *)nanf, (void *)dv, (void *)di, (void *)ds})
    if (p) (void)hipFree(p);
  if (e != hipSuccess) return set_err(-3, "ec_topk_dev: %s", hipGetErrorString(e));
  return 0;
}

// ec_topk_dev with its scratch in the library's device array instead of
// allocations: candidates [rows][chunks][top_k + 1], NaN flags, and the
// results staged for the copies to the host, each region 256-byte aligned.
// Every scratch byte the kernels read is written first by them in the same
// call, so nothing needs clearing.  Calls overlapping on one GPU share the
// array and race.
extern "C" int ec_topk_dev_noalloc(const float *logits, int rows, int vocab, int ld, int top_k, float *vals,
                                   int *idx, int *status) {
  // the device set-up only: no allocation, stream or event; the library's
  // stream once some other call has created it, else the null stream
  {
    const int r0 = init_device();
    if (r0) return r0;
  }
  hipStream_t s = g_inited ? g_stream : nullptr;
  if (rows < 0 || ld < vocab) return set_err(-1, "ec_topk_dev_noalloc: rows=%d ld=%d vocab=%d", rows, ld, vocab);
  if (rows == 0) return 0;
  if (!topk_ok(vocab, top_k))
    return set_err(-1, "ec_topk_dev_noalloc: top_k=%d outside (0, %d) or above %d", top_k, vocab, kTopkMax);
  if (!logits || !vals || !idx || !status) return set_err(-1, "ec_topk_dev_noalloc: null pointer");
  char *base = g_device < kMaxDevices ? (char *)g_scratch_dev[g_device] : nullptr;
  if (!base) return set_err(-3, "ec_topk_dev_noalloc: the device scratch array is unavailable");
  const int nb = topk_chunks(vocab), n = top_k + 1;
  auto up = [](size_t b) { return (b + 255) & ~(size_t)255; };
  const size_t o_nan = up((size_t)rows * nb * n * sizeof(unsigned long long));
  const size_t o_v = o_nan + up((size_t)rows * nb), o_i = o_v + up((size_t)rows * n * 4);
  const size_t o_s = o_i + up((size_t)rows * n * 4), need = o_s + up((size_t)rows * 4);
  if (need > kNoAllocScratch)
    return set_err(-1, "ec_topk_dev_noalloc: %d rows of vocab %d at top_k %d need %zu bytes of scratch, above "
                   "its %zu", rows, vocab, top_k, need, kNoAllocScratch);
  unsigned long long *cand = (unsigned long long *)base;
  unsigned char *nanf = (unsigned char *)(base + o_nan);
  float *dv = (float *)(base + o_v);
  int *di = (int *)(base + o_i), *ds = (int *)(base + o_s);
  hipError_t e = topk_select(logits, rows, vocab, ld, top_k, cand, nanf, s);
  if (e == hipSuccess) e = topk_merge(cand, nanf, rows, vocab, top_k, dv, di, ds, s);
  if (e == hipSuccess) e = hipMemcpyAsync(vals, dv, (size_t)rows * n * 4, hipMemcpyDeviceToHost, s);
  if (e == hipSuccess) e = hipMemcpyAsync(idx, di, (size_t)rows * n * 4, hipMemcpyDeviceToHost, s);
  if (e == hipSuccess) e = hipMemcpyAsync(status, ds, (size_t)rows * 4, hipMemcpyDeviceToHost, s);
  if (e == hipSuccess) e = hipStreamSynchronize(s);
  if (e != hipSuccess) return set_err(-3, "ec_topk_dev_noalloc: %s", hipGetErrorString(e));
  return 0;
}

// Greedy decode of n tokens in one slot: `token` at position `pos` gives
// out[0], out[0] at pos + 1 gives out[1], and so on -- the ids of n greedy
// gpt2_forward_ex steps.  With the persistent step the steps are chained on
// the device: each step's argmax id becomes the next step's token (and the
// position and tag advance) in a one-thread kernel, so the host launches the
// n steps back to back and reads the ids once; one HIP graph per 512-position
// bucket.  Otherwise (no persistent step for this model, or the profiler on)
// one forward per token.
extern "C" int ec_generate_greedy_timed(GPT2 *g, int token, int pos, int slot, int n, int *out, double *step_ms) {
  EC_INIT();
  DevModel *d = dev_of(g);
  if (!d) return set_err(-1, "model not loaded");
  if (!out || n < 1) return set_err(-1, "ec_generate_greedy: n=%d (at least 1) and an output array", n);
  if (token < 0 || token >= g->vocab) return set_err(-1, "ec_generate_greedy: token %d outside [0, %d)", token, g->vocab);
  if (pos < 0 || n > d->eff_ctx - pos)
    return set_err(-1, "ec_generate_greedy: positions %d..%d outside [0, %d)", pos, pos + n - 1, d->eff_ctx);
  if (slot < 0) return set_err(-1, "ec_generate_greedy: negative slot %d", slot);
  if (slot >= g->batch_cap) slot = g->batch_cap - 1;  // as the forward (src/gpt2.c:512-513)
  if (!d->step_ok || g_prof_on || step_vtile(g, d, pos + n) < 4) {
    int t = token;
    for (int k = 0; k < n; k++) {
      const int p = pos + k;
      const double t0 = now_sec();
      const int r = forward_impl(g, &t, &p, &slot, 1, 0, nullptr, &out[k]);
      if (r) return r;
      if (step_ms) step_ms[k] = (now_sec() - t0) * 1e3;
      t = out[k];
    }
    return 0;
  }
  hipStream_t s = g_stream;
  if (d->step_tag > 0xFFFFFFFFu - (unsigned)n - 1u) {  // the tags below must not wrap: clear the old ones
    EC_HIP(step_clear(d, s));
    d->step_tag = 0;
  }
  int *io = d->h_step_io;
  io[0] = token;
  io[1] = pos;
  io[2] = slot;
  io[3] = (int)(d->step_tag + 1u);
  io[4] = io[5] = io[6] = 0;
  // An error after the first step was enqueued leaves steps with the tags
  // step_tag + 1.. possibly run (wholly or in part): their words carry tags
  // that the next call would use again.  Wait for what was enqueued, clear
  // every exchange word and FFN half, and start the tags over.
  auto abandon = [&](int r) {
    (void)hipStreamSynchronize(s);
    if (step_clear(d, s) == hipSuccess) (void)hipStreamSynchronize(s);
    (void)hipGetLastError();
    d->step_tag = 0;
    return r;
  };
  EC_HIP(hipMemcpyAsync(d->d_step_io, io, 7 * sizeof(int), hipMemcpyHostToDevice, s));
  if (step_ms) EC_HIP(chain_stamp(d->d_gen_t, s));
  for (int k = 0; k < n;) {
    const int max_npos = pos + k + 1;
    int bucket = (max_npos + 511) / 512 * 512;
    if (bucket > d->eff_ctx) bucket = d->eff_ctx;
    // kChainBurst steps in one graph when their positions stay in the bucket
    const int len = (n - k >= kChainBurst && bucket - (pos + k) >= kChainBurst) ? kChainBurst : 1;
    const int gi = len == 1 ? 0 : 1;
    bool graph = g_use_graphs && !d->step_nograph && step_vtile(g, d, bucket) >= 4;
    if (graph && (!d->chain_graph[gi] || d->chain_bucket[gi] != bucket)) {
      if (d->chain_graph[gi]) {
        const hipError_t ed = hipGraphExecDestroy(d->chain_graph[gi]);
        d->chain_graph[gi] = nullptr;
        if (ed != hipSuccess)
          return abandon(set_err(-3, "ec_generate_greedy: hipGraphExecDestroy: %s", hipGetErrorString(ed)));
      }
      hipGraph_t gr = nullptr;
      hipError_t e = hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal);
      int r = 0;
      if (e == hipSuccess) {
        d->chaining = true;
        for (int j = 0; j < len && r == 0; j++)
          r = enqueue_forward(g, d, 1, 0, true, false, bucket, 0.0, nullptr, io + 5, nullptr, s, true);
        d->chaining = false;
        e = hipStreamEndCapture(s, &gr);
      }
      if (e == hipSuccess && r == 0) e = hipGraphInstantiate(&d->chain_graph[gi], gr, nullptr, nullptr, 0);
      if (gr) (void)hipGraphDestroy(gr);
      if (e != hipSuccess || r != 0) {
        (void)hipGetLastError();
        g_err[0] = 0;
        d->chain_graph[gi] = nullptr;
        graph = false;
      } else {
        d->chain_bucket[gi] = bucket;
      }
    }
    int r = 0;
    if (graph) {
      const hipError_t e = hipGraphLaunch(d->chain_graph[gi], s);
      if (e != hipSuccess) r = set_err(-3, "ec_generate_greedy: graph launch: %s", hipGetErrorString(e));
      k += len;
    } else {
      d->chaining = true;
      r = enqueue_forward(g, d, 1, 0, true, false, max_npos, 0.0, nullptr, io + 5, nullptr, s, true);
      d->chaining = false;
      k += 1;
    }
    if (r) return abandon(r);
  }
  d->step_tag += (unsigned)n;
  hipError_t e = hipMemcpyAsync(io + 4, d->d_step_io + 4, sizeof(int), hipMemcpyDeviceToHost, s);
  if (e == hipSuccess) e = hipMemcpyAsync(out, d->d_gen, (size_t)n * sizeof(int), hipMemcpyDeviceToHost, s);
  std::vector<unsigned long long> stamps(step_ms ? (size_t)n + 1 : 0);
  if (step_ms && e == hipSuccess)
    e = hipMemcpyAsync(stamps.data(), d->d_gen_t, (size_t)(n + 1) * sizeof(unsigned long long),
                       hipMemcpyDeviceToHost, s);
  if (e == hipSuccess) e = hipStreamSynchronize(s);
  if (e != hipSuccess) return abandon(set_err(-3, "ec_generate_greedy: %s", hipGetErrorString(e)));
  // s_memrealtime counts a constant 100 MHz clock: 1e5 ticks per ms
  for (int k = 0; step_ms && k < n; k++) step_ms[k] = (double)(stamps[k + 1] - stamps[k]) * 1e-5;
  if (io[4] || step_test_fail()) {
    if (step_timed_out(d)) return ec_generate_greedy_timed(g, token, pos, slot, n, out, step_ms);
    return set_err(-3, "ec_generate_greedy: a block's wait for another's results timed out (ids discarded)");
  }
  return 0;
}

extern "C" int ec_generate_greedy(GPT2 *g, int token, int pos, int slot, int n, int *out) {
  return ec_generate_greedy_timed(g, token, pos, slot, n, out, nullptr);
}

extern "C" int ec_attention_dev(const float *q, int ldq, const uint16_t *kc, const uint16_t *vc, int nslots, int C,
                                int H, int KVH, int hd, const int *pos, const int *slot, int M, int window, float *out,
                                int ldo, int path) {
  EC_INIT();
  if (!q || !kc || !vc || !pos || !slot || !out) return set_err(-1, "ec_attention_dev: null pointer");
  if (M < 1 || nslots < 1 || C < 1 || H < 1 || KVH < 1 || H % KVH || hd < 1 || ldq < H * hd || ldo < H * hd ||
      window < 0 || path < 0 || path > 2)
    return set_err(-1, "ec_attention_dev: M=%d slots=%d C=%d H=%d KVH=%d hd=%d ldq=%d ldo=%d window=%d path=%d", M,
                   nslots, C, H, KVH, hd, ldq, ldo, window, path);
  int max_npos = 0;
  for (int m = 0; m < M; m++) {
    if (pos[m] < 0 || pos[m] >= C || slot[m] < 0 || slot[m] >= nslots)
      return set_err(-1, "ec_attention_dev: token %d has position %d / slot %d outside [0, %d) / [0, %d)", m, pos[m],
                     slot[m], C, nslots);
    if (path == 0 && (slot[m] != slot[0] || pos[m] != pos[0] + m))
      return set_err(-1, "ec_attention_dev: path 0 takes one slot's consecutive positions (token %d)", m);
    if (pos[m] + 1 > max_npos) max_npos = pos[m] + 1;
  }
  const int kv = KVH * hd;
  const int vtile = attn_vtile(max_npos, hd, kv);
  if (vtile < 4) return set_err(-1, "ec_attention_dev: position %d needs more LDS than the device has", max_npos - 1);
  int *dps = nullptr;
  float *dsc = nullptr;
  hipError_t e = dev_malloc(&dps, (size_t)2 * M * sizeof(int));
  if (e == hipSuccess && path == 2) e = dev_malloc(&dsc, (size_t)M * H * C * sizeof(float));
  if (e == hipSuccess) e = hipMemcpyAsync(dps, pos, (size_t)M * sizeof(int), hipMemcpyHostToDevice, g_stream);
  if (e == hipSuccess) e = hipMemcpyAsync(dps + M, slot, (size_t)M * sizeof(int), hipMemcpyHostToDevice, g_stream);
  AttnArgs aa{q, ldq, kc, vc, out, ldo, dps, dps + M, H, KVH, hd, kv, C, window, 1.0 / sqrt((double)hd), M, max_npos,
              vtile, 0, nullptr, nullptr, 0, nullptr, 0, nullptr, nullptr, 0};
  aa.scores = dsc;
  aa.sc_ld = C;
  bool shape_ok = true;
  if (e == hipSuccess) {
    if (path == 0) {
      shape_ok = attention_prefill_ok(aa, g_max_lds);
      if (shape_ok) e = attention_prefill(aa, g_max_lds, g_stream);
    } else {
      e = attention(aa, g_stream);
    }
  }
  if (e == hipSuccess) e = hipStreamSynchronize(g_stream);
  if (dps) (void)hipFree(dps);
  if (dsc) (void)hipFree(dsc);
  if (!shape_ok) return set_err(-1, "ec_attention_dev: the prefill kernel does not take head_dim %d / %d positions", hd,
                                max_npos);
  if (e != hipSuccess) return set_err(-3, "ec_attention_dev: %s", hipGetErrorString(e));
  return 0;
}

extern "C" void gpt2_forward(GPT2 *g, const int *tokens, const int *positions, const int *seqs, int M,
                             float *logits) {
  if (forward_impl(g, tokens, positions, seqs, M, 0, logits, nullptr)) {
    fprintf(stderr, "gpt2_forward: %s\n", g_err);
    exit(1);
  }
}

extern "C" void qwen2_forward(GPT2 *g, const int *tokens, const int *positions, const int *seqs, int M,
                              float *logits) {
  if (g->arch != ARCH_QWEN2) {
    fprintf(stderr, "qwen2_forward: model is not a qwen2 model\n");
    exit(1);
  }
  gpt2_forward(g, tokens, positions, seqs, M, logits);
}

// Releases what the library holds outside models: its two streams and their
// events, the timing events, and the staging and part buffers of the
// host-pointer GEMM entry points.  Every model must have been freed
// (gpt2_free) first.  A later call sets the library up again.  The driver
// calls it before it exits, so that nothing of the library's is left for the
// HIP runtime's own teardown.
extern "C" int ec_release(void) {
  if (!g_inited) return 0;
  {
    std::lock_guard<std::mutex> lk(g_models_mu);
    if (!g_models.empty()) return set_err(-1, "ec_release: %zu models still loaded", g_models.size());
  }
  EC_HIP(hipStreamSynchronize(g_stream));
  EC_HIP(hipStreamSynchronize(g_side));
  prof_release_events();
  g_prof.clear();
  g_prof_agg.clear();
  g_prof_on = false;
  for (Staging &st : g_st) {
    if (st.p) EC_HIP(hipFree(st.p));
    st = Staging{};
  }
  if (g_w16_parts) EC_HIP(hipFree(g_w16_parts));
  if (g_w16_rs) EC_HIP(hipFree(g_w16_rs));
  g_w16_parts = nullptr;
  g_w16_rs = nullptr;
  g_w16_halves = g_w16_rows = 0;
  for (hipEvent_t &ev : g_touch_ev) {
    if (ev) EC_HIP(hipEventDestroy(ev));
    ev = nullptr;
  }
  EC_HIP(hipStreamDestroy(g_side));
  EC_HIP(hipStreamDestroy(g_stream));
  g_side = g_stream = nullptr;
  g_inited = 0;
  return 0;
}
