// ptk_kernels.hip -- gfx950 (MI355X) kernels of the PrimeTTS conv hot path, and the thin C-ABI
// layer (ptk.h) through which the C host code reaches them.
//
// Wide Conv1d / ConvTranspose1d run as one implicit GEMM on the fp32 matrix cores
// (v_mfma_f32_32x32x2_f32, or v_mfma_f32_16x16x4_f32 for 16-row tiles when one batch item's grid
// is too small to fill the chip): GEMM rows are output channels (convT: phase rows r*C4 + co, the
// reference's packed phase layout), columns are output positions, the reduction runs over
// (tap, input channel).  im2col never exists: each wave stages a window of input columns per
// channel chunk in LDS and reads it K times at the K tap shifts.  The four waves of a workgroup
// (eight for the 8-way split of single problems that leave one wave per SIMD) split the input
// channels and reduce through LDS in a fixed order (deterministic), then the
// epilogue (bias, LeakyReLU/ReLU/scalar ops, residual / branch-sum tensor adds, division) is
// applied on the accumulator values right before the single store.
#include <hip/hip_runtime.h>

#include <atomic>
#include <mutex>

#include <type_traits>

#include <limits.h>
#include <math.h>
#include <stdint.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "ptk.h"

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// ------------------------------------------------------------------------------ error handling
static thread_local char g_err[512];

static void set_err(const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof g_err, fmt, ap);
  va_end(ap);
}

#define HCHK(x)                                                                  \
  do {                                                                           \
    hipError_t e_ = (x);                                                         \
    if (e_ != hipSuccess) {                                                      \
      set_err("%s failed: %s (%s:%d)", #x, hipGetErrorString(e_), __FILE__, __LINE__); \
      return -1;                                                                 \
    }                                                                            \
  } while (0)

extern "C" const char *ptk_last_error(void) { return g_err; }

// ------------------------------------------------------------------------------ static scratch
// Device memory for callers that cannot allocate any (ptd_decode_noalloc): one array per GPU,
// loaded with the code object and held until the process ends.  On the host, `scratch` is only a
// stand-in for the symbol; host code uses the device address hipGetSymbolAddress gives for the
// current device (each GPU has its own copy at its own address), kept per device below.  Every
// user of a GPU shares that GPU's array: work that overlaps in time on one GPU races on it.
static __device__ __align__(256) unsigned char scratch[PTK_STATIC_SCRATCH_BYTES];
#define PTK_SCRATCH_MAX_DEVICES 64
static std::mutex g_scratch_lock;
static void *g_scratch_ptr[PTK_SCRATCH_MAX_DEVICES];
// Users of one GPU's scratch are ordered on that GPU: each waits for the work of the one before
// (an event recorded after it), whatever stream either ran on.  The event is made at set-up with
// the address; g_scratch_use[dev] is held from the wait until the record, so two host threads
// cannot both wait on the same predecessor.
static hipEvent_t g_scratch_done[PTK_SCRATCH_MAX_DEVICES];
static bool g_scratch_recorded[PTK_SCRATCH_MAX_DEVICES];
static std::mutex g_scratch_use[PTK_SCRATCH_MAX_DEVICES];

static int scratch_device(int *dev) {
  HCHK(hipGetDevice(dev));
  if (*dev < 0 || *dev >= PTK_SCRATCH_MAX_DEVICES) {
    set_err("static scratch: device %d out of range", *dev);
    return -1;
  }
  return 0;
}

// resolve (once per device, with that device current) the current device's copy of `scratch`
// and make its ordering event
static int scratch_resolve(void **out) {
  int dev = -1;
  if (scratch_device(&dev)) return -1;
  std::lock_guard<std::mutex> lk(g_scratch_lock);
  if (!g_scratch_ptr[dev]) {
    void *p = nullptr;
    HCHK(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    if (!p) {
      set_err("static scratch: hipGetSymbolAddress gave NULL on device %d", dev);
      return -1;
    }
    if (!g_scratch_done[dev]) HCHK(hipEventCreateWithFlags(&g_scratch_done[dev], hipEventDisableTiming));
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return 0;
}

extern "C" int ptk_static_scratch(void **p, size_t *bytes) {
  *p = nullptr;
  *bytes = 0;
  if (scratch_resolve(p)) return -1;
  *bytes = PTK_STATIC_SCRATCH_BYTES;
  return 0;
}

static int stream_capturing(hipStream_t st, bool *on) {
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  HCHK(hipStreamIsCapturing(st, &cs));
  *on = cs != hipStreamCaptureStatusNone;
  return 0;
}

extern "C" int ptk_scratch_acquire(void *s, int *dev_out) {
  int dev = -1;
  void *p;
  *dev_out = -1;
  if (scratch_resolve(&p) || scratch_device(&dev)) return -1;
  g_scratch_use[dev].lock();
  *dev_out = dev;
  bool cap = false;
  hipError_t e = hipSuccess;
  if (stream_capturing((hipStream_t) s, &cap) == 0) {
    if (!cap && g_scratch_recorded[dev]) e = hipStreamWaitEvent((hipStream_t) s, g_scratch_done[dev], 0);
    if (e == hipSuccess) return 0;
    set_err("hipStreamWaitEvent on the static scratch's event failed: %s", hipGetErrorString(e));
  }
  g_scratch_use[dev].unlock();
  *dev_out = -1;
  return -1;
}

extern "C" int ptk_scratch_release(void *s, int dev, int recorded_work) {
  if (dev < 0 || dev >= PTK_SCRATCH_MAX_DEVICES) return -1;
  bool cap = false;
  int rc = stream_capturing((hipStream_t) s, &cap);
  if (rc == 0 && recorded_work && !cap) {
    const hipError_t e = hipEventRecord(g_scratch_done[dev], (hipStream_t) s);
    if (e == hipSuccess) {
      g_scratch_recorded[dev] = true;
    } else {
      set_err("hipEventRecord on the static scratch's event failed: %s", hipGetErrorString(e));
      rc = -1;
    }
  }
  g_scratch_use[dev].unlock();
  return rc;
}

// ------------------------------------------------------------------------------ runtime wrappers
// Device 0 for the calling thread.  The device count is queried once per process; the current
// device is per-thread HIP state, so every thread that creates a context selects it itself (the
// reference brings contexts up from one thread per stream, concurrently).
extern "C" int ptk_init(void) {
  static std::once_flag once;
  static hipError_t count_err = hipSuccess;
  static int ndev = 0;
  std::call_once(once, [] { count_err = hipGetDeviceCount(&ndev); });
  HCHK(count_err);
  if (ndev < 1) {
    set_err("no HIP device");
    return -1;
  }
  thread_local bool selected = false;
  if (!selected) {
    HCHK(hipSetDevice(0));
    selected = true;
    // PT_V21_SYNC, the reference's scheduling mode for host waits (pt_v21_cuda.cu:758-764): 0 spin,
    // 1 blocking, 2 yield (ROCm treats blocking as yield).  Unset: HIP's own choice.  Set once per
    // process, on the first thread to select the device; on a device already active in this
    // process (another library made it so) HIP refuses the change, which is ignored here as the
    // reference ignores it.
    static std::once_flag sync_once;
    std::call_once(sync_once, [] {
      const char *e = getenv("PT_V21_SYNC");
      if (!e) return;
      const int mode = atoi(e);
      const unsigned fl = mode == 0 ? hipDeviceScheduleSpin
                        : mode == 1 ? hipDeviceScheduleBlockingSync
                        : mode == 2 ? hipDeviceScheduleYield : 0u;
      if (fl && hipSetDeviceFlags(fl) != hipSuccess) (void) hipGetLastError();
    });
    // set-up of the static scratch's address for this device, outside any later stream capture;
    // a failure here is reported by the entry point that needs it (which retries), not by init
    void *p;
    if (scratch_resolve(&p)) g_err[0] = 0;
  }
  return 0;
}
extern "C" int ptk_stream_create(void **s) {
  hipStream_t st;
  HCHK(hipStreamCreateWithFlags(&st, hipStreamNonBlocking));
  *s = (void *) st;
  return 0;
}
extern "C" int ptk_stream_destroy(void *s) {
  HCHK(hipStreamDestroy((hipStream_t) s));
  return 0;
}
// A bounded single-workgroup kernel of dependent ALU work: no memory reads, no waits, one store
// per lane.  Two launches on one hardware queue run one after the other, on two queues at once,
// which is how the servers time the queue placement of their streams.
// (a device symbol the host could read, so the loop and its store are not removed as dead code)
__device__ float ptk_calib_sink[64];
__global__ void __launch_bounds__(64) calib_kernel(int iters, float seed) {
  float v = seed + (float) threadIdx.x;
  for (int i = 0; i < iters; i++) v = v * 0.999f + 0.5f;
  ptk_calib_sink[threadIdx.x] = v;
}
extern "C" int ptk_calib_launch(int iters, void *s) {
  if (iters < 1 || iters > (1 << 22)) {
    set_err("ptk_calib_launch: %d iterations outside [1, 2^22]", iters);
    return -1;
  }
  hipLaunchKernelGGL(calib_kernel, dim3(1), dim3(64), 0, (hipStream_t) s, iters, 1.0f);
  HCHK(hipGetLastError());
  return 0;
}
extern "C" int ptk_stream_sync(void *s) {
  HCHK(hipStreamSynchronize((hipStream_t) s));
  return 0;
}
extern "C" int ptk_stream_query(void *s) {
  hipError_t e = hipStreamQuery((hipStream_t) s);
  if (e == hipSuccess) return 1;
  if (e == hipErrorNotReady) return 0;
  set_err("hipStreamQuery: %s", hipGetErrorString(e));
  return -1;
}
// Failure injection for tests of the error paths: after `skip` more device allocations succeed,
// the next `n` fail as if the device were out of memory (process-wide; nothing reaches the
// device).  n = 0 switches it off.
static std::mutex g_inject_lock;
static int g_inject_skip, g_inject_fail;
extern "C" void ptk_fail_allocs(int skip, int n) {
  std::lock_guard<std::mutex> lk(g_inject_lock);
  g_inject_skip = skip > 0 ? skip : 0;
  g_inject_fail = n > 0 ? n : 0;
}
static bool inject_alloc_failure() {
  std::lock_guard<std::mutex> lk(g_inject_lock);
  if (g_inject_fail <= 0) return false;
  if (g_inject_skip > 0) {
    g_inject_skip--;
    return false;
  }
  g_inject_fail--;
  return true;
}
extern "C" int ptk_malloc(void **p, size_t bytes) {
  if (inject_alloc_failure()) {
    *p = nullptr;
    set_err("hipMalloc(%zu bytes) failed: injected allocation failure", bytes);
    return -1;
  }
  HCHK(hipMalloc(p, bytes ? bytes : 1));
  return 0;
}
extern "C" int ptk_free(void *p) {
  if (p) HCHK(hipFree(p));
  return 0;
}
extern "C" int ptk_h2d_async(void *dst, const void *src, size_t bytes, void *s) {
  if (bytes) HCHK(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, (hipStream_t) s));
  return 0;
}
extern "C" int ptk_d2h_async(void *dst, const void *src, size_t bytes, void *s) {
  if (bytes) HCHK(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, (hipStream_t) s));
  return 0;
}
extern "C" int ptk_d2d_async(void *dst, const void *src, size_t bytes, void *s) {
  if (bytes) HCHK(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, (hipStream_t) s));
  return 0;
}
extern "C" int ptk_fill_async(void *dst, int byte, size_t bytes, void *s) {
  HCHK(hipMemsetAsync(dst, byte, bytes, (hipStream_t) s));
  return 0;
}
extern "C" int ptk_d2d_2d_async(void *dst, size_t dpitch, const void *src, size_t spitch,
                                size_t wb, size_t h, void *s) {
  if (wb && h)
    HCHK(hipMemcpy2DAsync(dst, dpitch, src, spitch, wb, h, hipMemcpyDeviceToDevice, (hipStream_t) s));
  return 0;
}
extern "C" int ptk_d2h_2d_async(void *dst, size_t dpitch, const void *src, size_t spitch,
                                size_t wb, size_t h, void *s) {
  if (wb && h)
    HCHK(hipMemcpy2DAsync(dst, dpitch, src, spitch, wb, h, hipMemcpyDeviceToHost, (hipStream_t) s));
  return 0;
}
extern "C" int ptk_h2d_2d_async(void *dst, size_t dpitch, const void *src, size_t spitch,
                                size_t wb, size_t h, void *s) {
  if (wb && h)
    HCHK(hipMemcpy2DAsync(dst, dpitch, src, spitch, wb, h, hipMemcpyHostToDevice, (hipStream_t) s));
  return 0;
}
extern "C" int ptk_event_create(void **e) {
  hipEvent_t ev;
  HCHK(hipEventCreate(&ev));
  *e = (void *) ev;
  return 0;
}
extern "C" int ptk_event_destroy(void *e) {
  HCHK(hipEventDestroy((hipEvent_t) e));
  return 0;
}
extern "C" int ptk_event_record(void *e, void *s) {
  HCHK(hipEventRecord((hipEvent_t) e, (hipStream_t) s));
  return 0;
}
extern "C" int ptk_stream_wait_event(void *s, void *e) {
  HCHK(hipStreamWaitEvent((hipStream_t) s, (hipEvent_t) e, 0));
  return 0;
}
extern "C" int ptk_event_elapsed_ms(float *ms, void *e0, void *e1) {
  HCHK(hipEventElapsedTime(ms, (hipEvent_t) e0, (hipEvent_t) e1));
  return 0;
}
extern "C" int ptk_event_sync(void *e) {
  HCHK(hipEventSynchronize((hipEvent_t) e));
  return 0;
}
extern "C" int ptk_device_sync(void) {
  HCHK(hipDeviceSynchronize());
  return 0;
}
extern "C" int ptk_capture_begin(void *s) {
  HCHK(hipStreamBeginCapture((hipStream_t) s, hipStreamCaptureModeThreadLocal));
  return 0;
}
extern "C" int ptk_capture_end(void *s, void **exec) {
  hipGraph_t g = nullptr;
  HCHK(hipStreamEndCapture((hipStream_t) s, &g));
  if (!exec) {
    if (g) (void) hipGraphDestroy(g);
    return 0;
  }
  hipGraphExec_t e = nullptr;
  const hipError_t err = hipGraphInstantiate(&e, g, nullptr, nullptr, 0);
  (void) hipGraphDestroy(g);
  HCHK(err);
  *exec = (void *) e;
  return 0;
}
extern "C" int ptk_graph_launch(void *exec, void *s) {
  HCHK(hipGraphLaunch((hipGraphExec_t) exec, (hipStream_t) s));
  return 0;
}
extern "C" int ptk_graph_destroy(void *exec) {
  if (exec) HCHK(hipGraphExecDestroy((hipGraphExec_t) exec));
  return 0;
}

// ------------------------------------------------------------------------------ weight relayout
// Packed [M/4][K][cin][4] (the reference's conv layout; a convT's phase rows are just more rows)
// -> MFMA operand layout [Mp/32][K][cinp/8][64][4].  For a row block mb, tap k and a chunk of 8
// input channels, lane l = 32*h + r of a wave holds the four floats
//     W[mb*32 + r][k][chunk*8 + 2*p + h],   p = 0..3,
// which are exactly its A operands (row r, reduction index h) of the four v_mfma_f32_32x32x2_f32
// that consume channel pairs (2p, 2p+1) of the chunk.  One 16-byte load per lane therefore feeds
// four MFMAs, and the 1 KiB a wave loads for one (tap, chunk) is contiguous.  cinp rounds cin up
// so every wave of the 4-way channel split owns whole chunks; padding rows/channels are zero.
#define CONV_CK 8          // input channels per staged chunk (per wave)
#define CONV_WAVES 4       // waves per workgroup, each owning a quarter of the channels

extern "C" int ptk_conv_cinp(int cin) {
  const int q = CONV_WAVES * CONV_CK;
  return (cin + q - 1) / q * q;
}
extern "C" size_t ptk_relayout_floats(int M, int K, int cin) {
  const size_t Mp = (size_t) (M + 31) / 32 * 32;
  return Mp * (size_t) K * (size_t) ptk_conv_cinp(cin);
}

// il: 0, or the rows per phase C4 of a stride-4 convT whose rows the MFMA layout interleaves by
// phase: relaid row m is packed row (m & 3) * il + (m >> 2), phase m & 3 of channel m >> 2.
__device__ __forceinline__ int relayout_row(int m, int il) { return il ? (m & 3) * il + (m >> 2) : m; }

__global__ void relayout_kernel(float *__restrict__ dst, const float *__restrict__ wp, int M,
                                int K, int cin, int cinp, long long total, int il) {
  long long i = (long long) blockIdx.x * blockDim.x + threadIdx.x;
  const long long st = (long long) gridDim.x * blockDim.x;
  const int nchunk = cinp / CONV_CK;
  for (; i < total; i += st) {
    const int p = (int) (i & 3);
    const int lane = (int) ((i >> 2) & 63);
    long long r = i >> 8;
    const int chunk = (int) (r % nchunk);
    r /= nchunk;
    const int k = (int) (r % K);
    const int mb = (int) (r / K);
    const int m = mb * 32 + (lane & 31);
    const int ci = chunk * CONV_CK + 2 * p + (lane >> 5);
    float v = 0.0f;
    if (m < M && ci < cin) {
      const int ms = relayout_row(m, il);
      v = wp[(((long long) (ms >> 2) * K + k) * cin + ci) * 4 + (ms & 3)];
    }
    dst[i] = v;
  }
}

static int relayout_il_ok(int M, int il, const char *who) {
  if (il != 0 && (il < 1 || M != 4 * il)) {
    set_err("%s: phase interleave needs M = 4 x rows per phase (M %d, rows per phase %d)", who, M, il);
    return 0;
  }
  return 1;
}

extern "C" int ptk_relayout_il(float *dst, const float *wp, int M, int K, int cin, int il, void *s) {
  if (!relayout_il_ok(M, il, "ptk_relayout_il")) return -1;
  const long long total = (long long) ptk_relayout_floats(M, K, cin);
  long long blocks = (total + 255) / 256;
  if (blocks > 4096) blocks = 4096;
  hipLaunchKernelGGL(relayout_kernel, dim3((unsigned) blocks), dim3(256), 0, (hipStream_t) s, dst,
                     wp, M, K, cin, ptk_conv_cinp(cin), total, il);
  HCHK(hipGetLastError());
  return 0;
}
extern "C" int ptk_relayout(float *dst, const float *wp, int M, int K, int cin, void *s) {
  return ptk_relayout_il(dst, wp, M, K, cin, 0, s);
}

// The same weights for 16-row tiles on v_mfma_f32_16x16x4_f32: [Mp/16][K][cinp/8][64][2] (Mp = M
// rounded up to 16).  Lane l = 16*kq + r holds W[mb*16 + r][k][chunk*8 + 4*s + kq], s = 0, 1: its
// A operands (row r, reduction index kq) of the two MFMAs that consume channels 4s .. 4s + 3 of
// the chunk.  One 8-byte load per lane feeds both, and a wave's (tap, chunk) slice is 512
// contiguous bytes.
extern "C" size_t ptk_relayout16_floats(int M, int K, int cin) {
  const size_t Mp = (size_t) (M + 15) / 16 * 16;
  return Mp * (size_t) K * (size_t) ptk_conv_cinp(cin);
}

__global__ void relayout16_kernel(float *__restrict__ dst, const float *__restrict__ wp, int M,
                                  int K, int cin, int cinp, long long total, int il) {
  long long i = (long long) blockIdx.x * blockDim.x + threadIdx.x;
  const long long st = (long long) gridDim.x * blockDim.x;
  const int nchunk = cinp / CONV_CK;
  for (; i < total; i += st) {
    const int s = (int) (i & 1);
    const int lane = (int) ((i >> 1) & 63);
    long long r = i >> 7;
    const int chunk = (int) (r % nchunk);
    r /= nchunk;
    const int k = (int) (r % K);
    const int mb = (int) (r / K);
    const int m = mb * 16 + (lane & 15);
    const int ci = chunk * CONV_CK + 4 * s + (lane >> 4);
    float v = 0.0f;
    if (m < M && ci < cin) {
      const int ms = relayout_row(m, il);
      v = wp[(((long long) (ms >> 2) * K + k) * cin + ci) * 4 + (ms & 3)];
    }
    dst[i] = v;
  }
}

extern "C" int ptk_relayout16_il(float *dst, const float *wp, int M, int K, int cin, int il, void *s) {
  if (!relayout_il_ok(M, il, "ptk_relayout16_il")) return -1;
  const long long total = (long long) ptk_relayout16_floats(M, K, cin);
  long long blocks = (total + 255) / 256;
  if (blocks > 4096) blocks = 4096;
  hipLaunchKernelGGL(relayout16_kernel, dim3((unsigned) blocks), dim3(256), 0, (hipStream_t) s,
                     dst, wp, M, K, cin, ptk_conv_cinp(cin), total, il);
  HCHK(hipGetLastError());
  return 0;
}
extern "C" int ptk_relayout16(float *dst, const float *wp, int M, int K, int cin, void *s) {
  return ptk_relayout16_il(dst, wp, M, K, cin, 0, s);
}

// ------------------------------------------------------------------------------ fp16 expansion
// binary16 -> binary32 by its bit fields.  Every binary16 value is exact in binary32: normals
// rebias the exponent (15 -> 127), subnormals m * 2^-24 renormalise around their leading one,
// inf / NaN keep sign and payload.  Integer work only, so no float mode (denormal flushing,
// NaN quieting) can change a result.
__device__ __forceinline__ unsigned half_to_float_bits(unsigned h) {
  const unsigned s = (h & 0x8000u) << 16, e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
  if (e == 31u) return s | 0x7f800000u | (m << 13);
  if (e != 0u) return s | ((e + 112u) << 23) | (m << 13);
  if (m == 0u) return s;
  const unsigned p = 31u - (unsigned) __builtin_clz(m);   // leading one at bit p (0..9)
  return s | ((p + 103u) << 23) | ((m << (23u - p)) & 0x7fffffu);
}

__global__ void h2f_kernel(float *__restrict__ dst, const unsigned short *__restrict__ src,
                           long long n) {
  const long long st = (long long) gridDim.x * blockDim.x;
  for (long long i = (long long) blockIdx.x * blockDim.x + threadIdx.x; i < n; i += st)
    dst[i] = __uint_as_float(half_to_float_bits(src[i]));
}

extern "C" int ptk_h2f(float *dst, const uint16_t *src, int64_t n, void *s) {
  if (n <= 0) return 0;
  long long blocks = (n + 255) / 256;
  if (blocks > 8192) blocks = 8192;
  hipLaunchKernelGGL(h2f_kernel, dim3((unsigned) blocks), dim3(256), 0, (hipStream_t) s, dst,
                     (const unsigned short *) src, (long long) n);
  HCHK(hipGetLastError());
  return 0;
}

// ------------------------------------------------------------------------------ epilogue
__device__ __forceinline__ float epi_apply(float v, const ptk_epi &e, int b, int co, long long col) {
  switch (e.op) {
    case PTK_EPI_LEAKY: return v >= 0.0f ? v : e.a * v;
    case PTK_EPI_RELU: return v > 0.0f ? v : 0.0f;
    case PTK_EPI_MULS: return v * e.a;
    case PTK_EPI_ADDS: return v + e.a;
    case PTK_EPI_ADDT: return v + e.t[(long long) b * e.bst + (long long) co * e.ldt + col];
    case PTK_EPI_DIVS: return v / e.a;
    default: return v;
  }
}

// input transform applied as a window element is staged (the reference's separate LeakyReLU node
// in front of a conv, fused): IN is a PTK_IN_* code.
// LeakyReLU as max(v, a*v): identical to (v >= 0 ? v : a*v) for 0 <= a <= 1 (signed zeros
// included), which the launcher enforces, in two instructions instead of three.
template <int IN>
__device__ __forceinline__ float in_xform(float v, float a) {
  if constexpr (IN != PTK_IN_PLAIN) v = fmaxf(v, a * v);
  return v;
}

// ------------------------------------------------------------------------------ MFMA conv kernel
// n / d for 0 <= n < 2^24 as (n * m) >> s, m = ceil(2^s / d), s = 24 + ceil(log2 d): the error
// term n * (m*d - 2^s) / (d * 2^s) stays below 1/d, so the floor is exact.  With n, m and s
// wave-uniform the division is two scalar multiplies and a shift.
struct FastDiv {
  unsigned m;
  int s;
};
static FastDiv fast_div(unsigned d) {
  int l = 0;
  while ((1u << l) < d) l++;
  const int s = 24 + l;
  return FastDiv{(unsigned) (((1ull << s) + d - 1) / d), s};
}
__device__ __forceinline__ int fdiv(int n, FastDiv f) {
  return (int) (((unsigned long long) (unsigned) n * f.m) >> f.s);
}

// Per-problem launch facts computed on the host, 64 bytes: one scalar load at kernel entry.
struct ConvProb {
  int count;                      // workgroups of the problem (grid row blockIdx.y = problem)
  int mt;                         // RB-row blocks
  int nt;                         // column tiles of a middle batch item
  int nt0;                        // of item 0 (its columns start ext_l earlier; one item: all)
  int ntl;                        // of the last item (its columns end ext_r later)
  int nitem;                      // batch items
  FastDiv div_tiles;              // by mt * nt (tiles of a middle batch item)
  FastDiv div_mt;                 // by mt
  FastDiv div_phase;              // by C4 / RB (row blocks per convT phase) when one_phase
  int flags;                      // PROB_ONE_PHASE | PROB_FAST | PROB_PHASE_IL
  int ext_l;                      // item 0's first column is q0 - ext_l
  int addt;                       // the chain's first tensor add, or -1
  int M;                          // GEMM rows
};
// every row block lies inside one phase (conv, or C4 % RB == 0)
#define PROB_ONE_PHASE 1
// output / residual index ranges fit the 32-bit epilogue
#define PROB_FAST 2
// stride-4 convT with its rows interleaved by phase (row m: phase m & 3 of channel m >> 2)
#define PROB_PHASE_IL 4
static_assert(sizeof(ConvProb) == 64, "one 64-byte scalar load");

// What the fast epilogue reads, 128 bytes per problem, fetched in one batch of scalar loads when
// the epilogue starts (field by field from the descriptor, each chain op's fields had been a
// scalar load and a wait of their own).
struct ConvEpi {
  const float *y, *y2, *t;        // output, its LeakyReLU copy (or null), the residual of op addt
  long long bsy, bst;             // batch strides of y / y2 and of t
  int ldy, ldt;                   // row strides (fit 32 bits on the fast path)
  int lout, qend, ext_r, ys, ypad, C4, nepi;   // qend: a middle item's column end
  int ops;                        // op e in bits 4e .. 4e + 3
  float a[PTK_MAX_EPI];
  float a2;
  int pad[7];
};
static_assert(sizeof(ConvEpi) == 128, "two 64-byte scalar loads");

struct ConvGroup {
  ConvProb info[PTK_MAX_GROUP];
  ConvEpi ep[PTK_MAX_GROUP];
  ptk_conv_desc d[PTK_MAX_GROUP];
  int ngroup;
  int split;                      // waves of a workgroup sharing one output block: 1, 2, 4 or 8
  int lg_split;                   // log2(split)
};

// Staged input window of one chunk (8 channels): NB column blocks of 32 outputs need
// (32*NB - 1)*stride + |K-1|*|dil| + 1 columns; the kernel supports up to 64*(NB+1).  LDS holds it
// as two planes h = 0, 1 of float4 columns: plane h, column c = channels h, 2+h, 4+h, 6+h.  The
// four B operands a lane (column, h) needs for one tap are then one 16-byte LDS read, and each
// half-wave reads (and each staging store writes) consecutive 16-byte columns: no bank conflicts.
template <int NB> struct WinGeo {
  static constexpr int NJ = NB + 1;          // 64-column slices a lane loads per row
  static constexpr int XWMAX = 64 * NJ;
};

// 16-row tiles (RB = 16) keep the same window but store it as four planes q = 0..3 of float2
// columns: plane q, column c = channels q, 4 + q, the B operands (reduction index q) of the two
// 16x16x4 MFMAs of a chunk.  A quarter-wave reads 16 consecutive float2 of one plane per tap and
// column block; planes are XWMAX + 16 float2 apart, so the two quarter-waves served together
// fall on different banks.
//
// LDS of one workgroup: per wave its staging area, and the partial-sum area (the staging area
// itself when the partial sums fit in it).
template <int NB, int RB, int NW> struct LdsGeo {
  static constexpr int XWMAX = WinGeo<NB>::XWMAX;
  static constexpr int PS = RB == 32 ? XWMAX : XWMAX + 16;   // plane stride (float4 / float2)
  static constexpr int STG = 8 * PS;                         // staging floats per wave
  static constexpr int NV = RB / 2;                          // accumulators per lane and column block
  static constexpr int RED = NB * NV * 64;                   // partial-sum floats per wave
  static constexpr bool OWN_RED = RED <= STG;
  static constexpr size_t BYTES = (size_t) NW * (STG > RED ? STG : RED) * sizeof(float);
};

// word 3 of a raw buffer resource on gfx9-family parts (gfx950): 32-bit data, range checked
#define PTK_BUF_WORD3 0x00020000
// an offset past every buffer: the load returns 0 (buffer range checking)
#define PTK_OOB 0x80000000u

// Scheduling fence for global loads: every instruction class except vector-memory may be moved
// across it (ALU, VALU, SALU, MFMA, LDS).  Placed right after prefetch loads, it keeps the machine
// scheduler from sinking them towards their use, which it does to shorten register live ranges
// and which would leave no prefetch distance at all.
#define PTK_PIN_VMEM() __builtin_amdgcn_sched_barrier(0x0106)

// voff: per-lane byte offset (PTK_OOB for an element that must read 0); soff: wave-uniform byte
// offset.  Either placement of the range check (with or without soff) leaves PTK_OOB + soff out of
// range for the buffers used here, which stay below 2 GiB.
__device__ __forceinline__ float buf_load(__amdgpu_buffer_rsrc_t r, unsigned voff, unsigned soff) {
  return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, 0));
}

// One workgroup = NW waves (4, or 8 for the 8-way split).  The waves form NW/S column groups of S
// waves; the S waves of a group compute the same RB-row x 32*NB-column output block over disjoint
// eighths/quarters/halves of the input channels (S = 1: each wave its own block over all channels)
// and are reduced through LDS in wave order (deterministic).  NW = 8 runs S = 8 only.  KT > 0:
// every problem of the group has K <= KT and the whole next chunk's A operands (KT float4 / float2
// per lane) are prefetched while the current chunk runs; KT == 0: any K, A loaded per tap.  IN:
// input transform (PTK_IN_*).  RB: rows per tile, 32 (32x32x2 MFMA, weights from d.w) or 16
// (16x16x4 MFMA on two 16-column blocks, weights from d.w16).
template <int KT, int NB, int IN, int RB, int NW>
__global__ void __launch_bounds__(64 * NW) conv_mfma_kernel(const ConvGroup g) {
  extern __shared__ float smem[];
  static_assert(RB == 32 || (RB == 16 && NB == 1), "16-row tiles are built for one column block");
  static_assert(NW == 4 || (NW == 8 && NB == 1), "8-wave workgroups are built for one column block");
  constexpr int NJ = WinGeo<NB>::NJ, XWMAX = WinGeo<NB>::XWMAX;
  using Geo = LdsGeo<NB, RB, NW>;
  constexpr int PS = Geo::PS, NV = Geo::NV;
  // Grid row blockIdx.y is the problem, so every field of it can be fetched at entry; rows are
  // as long as the largest problem's workgroup count, and the excess of a shorter one exits.
  const int p = blockIdx.y;
  const ConvProb pi = g.info[p];
  const ptk_conv_desc &d = g.d[p];
  // The scalar-cache lines of the problem's descriptor fields the prologue reads (x .. q0) and of
  // the split are touched in the same batch of loads as the launch facts: the prologue's later
  // reads of them then hit, instead of each batch waiting out a round trip of its own.
  asm volatile("" ::"s"(pi.count), "s"(d.x), "s"(d.w16), "s"(d.q0), "s"(g.split));
  const int bid = blockIdx.x;
  if (bid >= pi.count) return;
  const int mt = pi.mt;
  // Tiles item after item, column tile after column tile, row block fastest: item 0 has nt0
  // column tiles, the middle items nt, the last one ntl >= nt (all nt for a plain launch).
  // Written as masks and min / max rather than selects, which the compiler turns into branches
  // around the divisions (measured slower on single-wave-per-SIMD launches).
  const int c0 = mt * pi.nt0, t = bid - c0;
  const int past0 = ~(t >> 31);                          // -1 past item 0's tiles, else 0
  const int bq = fdiv(max(t, 0), pi.div_tiles);
  const int b = min(bq + 1, pi.nitem - 1) & past0;      // the last item takes its extra tiles
  const int r = bid - ((c0 + (b - 1) * (mt * pi.nt)) & past0);
  const int tn = fdiv(r, pi.div_mt);
  const int mb = r - tn * mt;
  const bool last_item = b == pi.nitem - 1;
  const long long q0i = d.q0 - (long long) (pi.ext_l & ~past0);   // this item's first column
  const int S = g.split, lgS = g.lg_split, G = NW >> lgS;

  // descriptor fields used in loops, read once (the problem index is dynamic, so the compiler
  // would otherwise re-read them from the kernel arguments)
  const int K = d.K, dil = d.dil, st = d.stride, cin = d.cin;
  const unsigned ldx4 = (unsigned) d.ldx * 4u;
  const long long lim = d.lim;
  const float in_a = d.in_a;
  const int nchunk = d.cinp / CONV_CK;          // chunks over all channels
  const int nch = nchunk >> lgS;                // chunks of this wave

  const int lane = threadIdx.x & 63;
  // wave index: uniform across the wave, which the compiler cannot see on its own (without this
  // the wave-based buffer resources would be treated as divergent)
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int ks = w & (S - 1), cg = w >> lgS;    // channel split index, column group
  // The phase of this row block (convT: row m is phase m / C4 of channel m % C4), when the block
  // lies inside one phase.
  const bool phase_rows = d.C4 != d.M;
  const bool one_phase = (pi.flags & PROB_ONE_PHASE) != 0;
  // rows interleaved by phase: only the 4-tap convT phase form (KT = 4) carries that code, so the
  // other instantiations compile exactly as without it (the launcher refuses it elsewhere)
  const bool phase_il = KT == 4 && (pi.flags & PROB_PHASE_IL) != 0;
  const int r_tile = phase_rows && one_phase ? fdiv(mb, pi.div_phase) : 0;
  // Lane l < RB loads the bias of the block's row l once the first chunk's loads are in flight,
  // and the epilogue fetches each value's bias from the lane of its row (ds_bpermute): the load's
  // latency is spent behind the main loop, and no wave depends on another's write.
  float bias_r = 0.0f;
  auto load_bias = [&]() {
    // the fields read in one batch ahead of any branch (under the kernel's scalar-register
    // pressure the compiler re-reads kernel arguments where they are used, one wait per read)
    const float *bp = d.bias;
    const int nbias = d.nbias, Mr = d.M, C4r = d.C4;
    const int m = mb * RB + lane;
    int co = m - r_tile * C4r;   // conv: r_tile = 0
    if (phase_il) co = m >> 2;
    else if (!one_phase) co = m % C4r;
    if (lane < RB && bp != nullptr && m < Mr && co < nbias) bias_r = bp[co];
  };
  // bias of row `row` of the block (every lane of the wave must be active)
  auto bias_of = [&](int row) {
    return __int_as_float(__builtin_amdgcn_ds_bpermute(row * 4, __float_as_int(bias_r)));
  };
  const int half = lane >> 5;     // RB = 32: which of the two reduction rows this lane feeds
  const int l32 = lane & 31;
  const int quad = lane >> 4;     // RB = 16: the reduction index (and row group) of this lane
  const int l16 = lane & 15;
  const int q0off = (tn * G + cg) * (32 * NB);   // this wave's first column past the item's first
  const long long q0 = q0i + q0off;
  const int kd = (K - 1) * dil;
  const int dmin = kd < 0 ? kd : 0;
  const int XW = (32 * NB - 1) * st + (kd < 0 ? -kd : kd) + 1;
  const long long cmin = q0 * st + dmin - d.shift;
  const int chunk0 = ks * nch;
  float *xsw = smem + w * Geo::STG;   // this wave's staging planes
  float4 *xs = reinterpret_cast<float4 *>(xsw);    // RB = 32: [h][column] float4
  float2 *xs2 = reinterpret_cast<float2 *>(xsw);   // RB = 16: [q][column] float2

  // Window columns this lane stages, fixed for the wave: byte offset in the row, or an offset the
  // buffer range check turns into 0 (columns outside [0, lim), past the window).  The row offset
  // is wave-uniform and goes into the scalar offset.  A row past cin (zero padding of the last
  // chunk when cin is not a multiple of 8) reads row 0 and is zeroed when it is stored.
  const long long xoff = (long long) b * d.bsx;
  const unsigned nrec = (unsigned) cin * ldx4;
  const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc(
      (void *) (d.x + xoff), (short) 0, (int) nrec, PTK_BUF_WORD3);
  unsigned voff[NJ];
#pragma unroll
  for (int jj = 0; jj < NJ; jj++) {
    const int col = lane + 64 * jj;
    const long long c = cmin + col;
    const bool ok = (col < XW) & (c >= 0) & (c < lim);
    const long long pc = d.reflect_l1 ? (c == 0 ? 1 : c - 1) : c;
    voff[jj] = ok ? (unsigned) pc * 4u : PTK_OOB;
  }

  // Staging is split so that all global loads of a chunk are in flight together: the load phase
  // only issues loads, the store phase (one chunk later) transforms and writes LDS.
  // Rows past cin exist only when cin is not a multiple of 32 (cinp > cin); MASK (compile time)
  // selects the chunk code that handles them, so the common case carries no per-row tests.
  // NJU (compile time) of the NJ slices are staged: windows up to 64 columns (every decoder conv
  // but K = 11 at dilation 5) need one, which halves the window loads and LDS stores.
  float pf[CONV_CK][NJ];
  auto load_chunk = [&](int c0, auto mask, auto nju) {
    constexpr bool MASK = decltype(mask)::value;
    constexpr int NJU = decltype(nju)::value;
#pragma unroll
    for (int r = 0; r < CONV_CK; r++) {
      const unsigned rowo = (!MASK || c0 + r < cin) ? (unsigned) (c0 + r) * ldx4 : 0u;
#pragma unroll
      for (int jj = 0; jj < NJU; jj++) {
        pf[r][jj] = buf_load(rx, voff[jj], rowo);
      }
    }
  };
  auto store_chunk = [&](int c0, auto mask, auto nju) {
    constexpr bool MASK = decltype(mask)::value;
    constexpr int NJU = decltype(nju)::value;
    const int nlive = cin - c0;   // rows of this chunk that hold channels
#pragma unroll
    for (int jj = 0; jj < NJU; jj++) {
      float v[CONV_CK];
#pragma unroll
      for (int r = 0; r < CONV_CK; r++) {
        v[r] = in_xform<IN>(pf[r][jj], in_a);
      }
      if constexpr (MASK) {
        if (nlive < CONV_CK) {
#pragma unroll
          for (int r = 0; r < CONV_CK; r++) v[r] = r < nlive ? v[r] : 0.0f;
        }
      }
      if constexpr (RB == 32) {
        xs[lane + 64 * jj] = make_float4(v[0], v[2], v[4], v[6]);
        xs[XWMAX + lane + 64 * jj] = make_float4(v[1], v[3], v[5], v[7]);
      } else {
#pragma unroll
        for (int q = 0; q < 4; q++) xs2[q * PS + lane + 64 * jj] = make_float2(v[q], v[4 + q]);
      }
    }
  };

  // accumulators: RB = 32, one 32x32 block per column block (16 values per lane); RB = 16, two
  // 16x16 blocks per column block (4 values per lane each)
  using AccT = std::conditional_t<RB == 32, f32x16, f32x4>;
  constexpr int NCB = RB == 32 ? 1 : 2;
  AccT acc[NB][NCB];
#pragma unroll
  for (int nb = 0; nb < NB; nb++)
#pragma unroll
    for (int cb = 0; cb < NCB; cb++)
#pragma unroll
      for (int v = 0; v < NV / NCB; v++) acc[nb][cb][v] = 0.0f;

  // A operands: float4 (RB = 16: float2) ((mb*K + k)*nchunk + chunk)*64 + lane of the relaid
  // weights, read through a buffer resource based at this wave's first chunk: the lane offset is
  // fixed and the (tap, chunk) offset is wave-uniform, so a load costs no vector address arithmetic
  using AT = std::conditional_t<RB == 32, float4, float2>;
  constexpr int ABYTES = 64 * (int) sizeof(AT);   // one (tap, chunk) slice of a wave
  const AT *wbase = reinterpret_cast<const AT *>(RB == 32 ? d.w : d.w16) +
                    ((long long) mb * K * nchunk + chunk0) * 64;
  const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc(
      (void *) wbase, (short) 0, (int) ((unsigned) K * (unsigned) nchunk * (unsigned) ABYTES),
      PTK_BUF_WORD3);
  const unsigned wlane = (unsigned) lane * (unsigned) sizeof(AT);
  const int wtap = nchunk * ABYTES;  // bytes between taps
  auto wa = [&](int k, int j) {
    if constexpr (RB == 32)
      return __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(rw, wlane, k * wtap + j * ABYTES, 0));
    else
      return __builtin_bit_cast(float2, __builtin_amdgcn_raw_buffer_load_b64(rw, wlane, k * wtap + j * ABYTES, 0));
  };
  // staging-plane index of tap 0, column block 0 (float4 for RB = 32, float2 for RB = 16)
  const int lbase = RB == 32 ? half * XWMAX + l32 * st - dmin : quad * PS + l16 * st - dmin;

  // the MFMAs of one tap: xr points at this lane's B operands of column block 0 (a float4 of
  // plane h for RB = 32, a float2 of plane quad for RB = 16)
  auto mfma4 = [&](const AT a, const auto *xr) {
    if constexpr (RB == 32) {
#pragma unroll
      for (int nb = 0; nb < NB; nb++) {
        const float4 bq = xr[32 * nb * st];
        acc[nb][0] = __builtin_amdgcn_mfma_f32_32x32x2f32(a.x, bq.x, acc[nb][0], 0, 0, 0);
        acc[nb][0] = __builtin_amdgcn_mfma_f32_32x32x2f32(a.y, bq.y, acc[nb][0], 0, 0, 0);
        acc[nb][0] = __builtin_amdgcn_mfma_f32_32x32x2f32(a.z, bq.z, acc[nb][0], 0, 0, 0);
        acc[nb][0] = __builtin_amdgcn_mfma_f32_32x32x2f32(a.w, bq.w, acc[nb][0], 0, 0, 0);
      }
    } else {
#pragma unroll
      for (int nb = 0; nb < NB; nb++)
#pragma unroll
        for (int cb = 0; cb < 2; cb++) {
          const float2 bq = xr[(32 * nb + 16 * cb) * st];
          acc[nb][cb] = __builtin_amdgcn_mfma_f32_16x16x4f32(a.x, bq.x, acc[nb][cb], 0, 0, 0);
          acc[nb][cb] = __builtin_amdgcn_mfma_f32_16x16x4f32(a.y, bq.y, acc[nb][cb], 0, 0, 0);
        }
    }
  };
  auto tap = [&](const AT a, int k) {
    if constexpr (RB == 32) mfma4(a, xs + lbase + k * dil);
    else mfma4(a, xs2 + lbase + k * dil);
  };
  // The chunk loop, for a compile-time tap count KC (0: runtime K, A operands loaded per tap).
  // Each chunk is straight-line code, so the scheduler can run LDS reads ahead of the MFMAs and
  // count outstanding loads exactly: stage the window loaded one chunk earlier, issue the next
  // chunk's window loads, then per tap four MFMAs on acur[k] followed by the load of that tap's
  // operands for the next chunk into the same registers (prefetch distance about one chunk).  The
  // last chunk is peeled so it issues no loads.
  auto run = [&](auto kc, auto mask, auto nju) {
    constexpr int KC = decltype(kc)::value;
    constexpr int KA = KC > 0 ? KC : 1;
    AT acur[KA];
    auto chunk = [&](int j, auto with_loads) {
      constexpr bool LD = decltype(with_loads)::value;
      __builtin_amdgcn_wave_barrier();
      store_chunk((chunk0 + j) * CONV_CK, mask, nju);
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      if constexpr (KC > 0) {
        // the next chunk's window loads go out behind tap 0's MFMAs, not between the window
        // store and the chunk's first MFMA
#pragma unroll
        for (int k = 0; k < KC; k++) {
          tap(acur[k], k);
          if constexpr (LD) {
            if (k == 0) {
              load_chunk((chunk0 + j + 1) * CONV_CK, mask, nju);
              PTK_PIN_VMEM();
            }
            acur[k] = wa(k, j + 1);
            PTK_PIN_VMEM();
          }
        }
      } else {
        if constexpr (LD) {
          load_chunk((chunk0 + j + 1) * CONV_CK, mask, nju);
          PTK_PIN_VMEM();
        }
        for (int k = 0; k < K; k++) tap(wa(k, j), k);
      }
      __builtin_amdgcn_wave_barrier();
    };
    // window loads first, then the A operands: the same order as inside a chunk, so the wait
    // before the first window store is the same count on entry as on every later trip
    load_chunk(chunk0 * CONV_CK, mask, nju);
    if constexpr (KC > 0) {
#pragma unroll
      for (int k = 0; k < KC; k++) acur[k] = wa(k, 0);
    }
    load_bias();
    for (int j = 0; j + 1 < nch; j++) chunk(j, std::true_type{});
    chunk(nch - 1, std::false_type{});
  };
  constexpr std::false_type nomask{};
  constexpr std::integral_constant<int, 1> one{};
  constexpr std::integral_constant<int, NJ> all{};
  const bool narrow = XW <= 64;
  if (cin == d.cinp) {
    if constexpr (KT > 0) {
      if (K == KT && narrow) run(std::integral_constant<int, KT>{}, nomask, one);
      else if (K == KT) run(std::integral_constant<int, KT>{}, nomask, all);
      else if (KT > 7 && K == 7 && narrow) run(std::integral_constant<int, 7>{}, nomask, one);
      else if (KT > 3 && K == 3 && narrow) run(std::integral_constant<int, 3>{}, nomask, one);
      else run(std::integral_constant<int, 0>{}, nomask, all);
    } else {
      run(std::integral_constant<int, 0>{}, nomask, all);
    }
  } else {
    // channel padding in the last chunks: any K through the generic body
    run(std::integral_constant<int, 0>{}, std::true_type{}, all);
  }

  // Epilogue: the S partial sums of a block are added in wave order through LDS, then bias, the
  // epilogue chain and one store per output.  RB = 32: lane (l32, half) holds, for column block
  // nb, the 16 values v of column q0 + 32*nb + l32 at rows 8*(v >> 2) + 4*half + (v & 3) of the
  // block.  RB = 16: lane (l16, quad) holds 8 values v of column q0 + 32*nb + 16*(v >> 2) + l16 at
  // rows 4*quad + (v & 3).  Wave ks of a column group finishes v in [v0, v0 + NV/S).
  const long long qend = d.q0 + d.nq + (last_item ? d.ext_r : 0);
  const int M = d.M, C4 = d.C4, ys = d.ys, ypad = d.ypad, nepi = d.nepi;
  const long long Lout = d.Lout, ldy = d.ldy;
  float *yb = d.y + (long long) b * d.bsy;
  float *y2b = d.y2 != nullptr ? d.y2 + (long long) b * d.bsy : nullptr;
  const float a2 = d.a2;
  const int addt = pi.addt;   // the chain's residual add, if any
  const int nv = NV >> lgS, v0 = ks * nv, wg0 = cg * S;
  // row and column of value v inside the block, lane parts included
  auto vrow = [&](int v) { return RB == 32 ? 8 * (v >> 2) + 4 * half + (v & 3) : 4 * quad + (v & 3); };
  auto vcol = [&](int nb, int v) { return RB == 32 ? 32 * nb + l32 : 32 * nb + 16 * (v >> 2) + l16; };

  // Each wave writes its partial sums over its own staging area, which only it reads, so no wave
  // waits for the others before writing (a separate region when they do not fit).
  constexpr bool OWN_RED = Geo::OWN_RED;
  auto red_of = [&](int wave) { return OWN_RED ? smem + wave * Geo::STG : smem + wave * Geo::RED; };
  if constexpr (!OWN_RED) __syncthreads();
  {
    float *red = red_of(w);
#pragma unroll
    for (int nb = 0; nb < NB; nb++)
#pragma unroll
      for (int cb = 0; cb < NCB; cb++)
#pragma unroll
        for (int v = 0; v < NV / NCB; v++) red[(nb * NV + cb * (NV / NCB) + v) * 64 + lane] = acc[nb][cb][v];
  }
  auto reduce_wait = [&]() {
    if (S > 1) {
      __syncthreads();
    } else {   // S = 1: a wave reads back only what it wrote
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
  };
  // The S partial sums of a value in wave order.  Every read is issued (a wave past the split
  // re-reads the group's first, in bounds, and is not added), so the reads of all values go out
  // together behind one wait instead of one round trip each behind a branch.
  auto reduced = [&](int nb, int v) {
    const int o = (nb * NV + v) * 64 + lane;
    float part[NW];
#pragma unroll
    for (int i = 0; i < NW; i++) part[i] = red_of(wg0 + (i < S ? i : 0))[o];
    float sum = part[0];
#pragma unroll
    for (int i = 1; i < NW; i++) sum = i < S ? sum + part[i] : sum;
    return sum;
  };
  // Fast path: a full block whose rows are consecutive output channels (conv, or a convT block
  // inside one phase), with every index of the output, its LeakyReLU copy and the residual inside
  // 32 bits (the launcher checks the extents).  Addresses are a wave-uniform row offset, in the
  // scalar offset of a buffer access, plus a lane offset computed once per column; the residual
  // loads are issued before the reduction barrier, at a clamped column so that every lane loads
  // in bounds without a branch (a lane whose column does not exist stores nothing).  The values
  // of a lane are val[i], i < nv: value v0 + i of the block.  The chain runs op by op over all of
  // them, one branch per op.  A convT block with its rows interleaved by phase (phase_il) holds
  // RB / 4 whole channels; its stores are laid out below.
  if ((pi.flags & PROB_FAST) && (one_phase || phase_il) && mb * RB + RB <= pi.M) {
    const ConvEpi ep = g.ep[p];
    // a wave finishes at most NMAX values (NV over the smallest split of its workgroup size),
    // in groups of GRP that share a column block (nv is a multiple of GRP)
    constexpr int NMAX = NW == 8 ? NV / 8 : NV;
    constexpr int GRP = (RB == 32 ? 4 : 2) < NMAX ? (RB == 32 ? 4 : 2) : NMAX, NG = NMAX / GRP;
    const int ngrp = nv / GRP;
    // first channel of the block
    const long long row0 = phase_il ? (long long) mb * (RB / 4) : (long long) mb * RB - (long long) r_tile * ep.C4;
    const int ldy32 = ep.ldy, ldt32 = ep.ldt;
    float *yk = const_cast<float *>(ep.y) + (long long) b * ep.bsy + row0 * ldy32;
    const __amdgpu_buffer_rsrc_t ry = __builtin_amdgcn_make_buffer_rsrc(
        (void *) yk, (short) 0, (int) 0x7fffffff, PTK_BUF_WORD3);
    const __amdgpu_buffer_rsrc_t ry2 = __builtin_amdgcn_make_buffer_rsrc(
        (void *) (ep.y2 != nullptr ? ep.y2 + (long long) b * ep.bsy + row0 * ldy32 : yk), (short) 0,
        (int) 0x7fffffff, PTK_BUF_WORD3);
    const __amdgpu_buffer_rsrc_t rt = __builtin_amdgcn_make_buffer_rsrc(
        (void *) (addt >= 0 ? ep.t + (long long) b * ep.bst + row0 * ldt32 : yk), (short) 0,
        (int) 0x7fffffff, PTK_BUF_WORD3);
    // lane part of the row of value i, and its wave-uniform part
    const int lrow = RB == 32 ? 4 * half : 4 * quad;
    auto urow = [&](int i) { return RB == 32 ? 8 * (((v0 + i) >> 2)) + ((v0 + i) & 3) : ((v0 + i) & 3); };
    const int qend32 = ep.qend + (last_item ? ep.ext_r : 0);
#pragma unroll
    for (int nb = 0; nb < NB; nb++) {
      // columns of this lane: one per column block (RB = 32), two (RB = 16)
      bool ok[NCB], oq[NCB];
      int cl[NCB], cu[NCB];
#pragma unroll
      for (int cb = 0; cb < NCB; cb++) {
        const int q = (int) q0 + 32 * nb + (RB == 32 ? l32 : 16 * cb + l16);
        const int col = q * ep.ys + r_tile - ep.ypad;
        oq[cb] = q < qend32;
        cu[cb] = col;   // phase_il: the sample of phase 0 (r_tile = 0), unclamped
        ok[cb] = oq[cb] && col >= 0 && col < ep.lout;
        cl[cb] = ok[cb] ? col : 0;
      }
      auto cbo = [&](int i) { return RB == 32 ? 0 : ((v0 + i) >> 2); };
      // column / test of column block c as a select (an index into cl / ok that is not a
      // compile-time constant would put the arrays in scratch memory)
      auto clof = [&](int c) { return NCB == 1 || c == 0 ? cl[0] : cl[NCB - 1]; };
      auto okof = [&](int c) { return NCB == 1 || c == 0 ? ok[0] : ok[NCB - 1]; };
      float rv[NMAX], val[NMAX];
      if (addt >= 0) {
#pragma unroll
        for (int gg = 0; gg < NG; gg++)
          if (gg < ngrp)
#pragma unroll
            for (int jj = 0, i = gg * GRP; jj < GRP; jj++, i++)
            rv[i] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(
                rt, (unsigned) (lrow * ldt32 + clof(cbo(i))) * 4u, (unsigned) (urow(i) * ldt32) * 4u, 0));
      }
#pragma unroll
      for (int gg = 0; gg < NG; gg++)
        if (gg < ngrp)
#pragma unroll
          for (int jj = 0, i = gg * GRP; jj < GRP; jj++, i++) val[i] = bias_of(lrow + urow(i));
      if (nb == 0) reduce_wait();
#pragma unroll
      for (int gg = 0; gg < NG; gg++)
        if (gg < ngrp)
#pragma unroll
          for (int jj = 0, i = gg * GRP; jj < GRP; jj++, i++) val[i] += reduced(nb, v0 + i);
      // the chain op by op over the four slots (straight-line: a rolled loop over the ops made the
      // compiler copy the value array at every op); a slot past nepi is skipped by a uniform branch
#pragma unroll
      for (int e = 0; e < PTK_MAX_EPI; e++) {
        if (e >= ep.nepi) break;
        const int op = (ep.ops >> (4 * e)) & 15;
        const float a = ep.a[e];
        if (op == PTK_EPI_LEAKY) {
#pragma unroll
          for (int gg = 0; gg < NG; gg++)
            if (gg < ngrp)
#pragma unroll
              for (int jj = 0, i = gg * GRP; jj < GRP; jj++, i++) val[i] = val[i] >= 0.0f ? val[i] : a * val[i];
        } else if (op == PTK_EPI_RELU) {
#pragma unroll
          for (int gg = 0; gg < NG; gg++)
            if (gg < ngrp)
#pragma unroll
              for (int jj = 0, i = gg * GRP; jj < GRP; jj++, i++) val[i] = val[i] > 0.0f ? val[i] : 0.0f;
        } else if (op == PTK_EPI_MULS) {
#pragma unroll
          for (int gg = 0; gg < NG; gg++)
            if (gg < ngrp)
#pragma unroll
              for (int jj = 0, i = gg * GRP; jj < GRP; jj++, i++) val[i] = val[i] * a;
        } else if (op == PTK_EPI_ADDS) {
#pragma unroll
          for (int gg = 0; gg < NG; gg++)
            if (gg < ngrp)
#pragma unroll
              for (int jj = 0, i = gg * GRP; jj < GRP; jj++, i++) val[i] = val[i] + a;
        } else if (op == PTK_EPI_DIVS) {
#pragma unroll
          for (int gg = 0; gg < NG; gg++)
            if (gg < ngrp)
#pragma unroll
              for (int jj = 0, i = gg * GRP; jj < GRP; jj++, i++) val[i] = val[i] / a;
        } else if (op == PTK_EPI_ADDT) {   // the chain's one tensor add (the launcher's rule)
#pragma unroll
          for (int gg = 0; gg < NG; gg++)
            if (gg < ngrp)
#pragma unroll
              for (int jj = 0, i = gg * GRP; jj < GRP; jj++, i++) val[i] = val[i] + rv[i];
        }
      }
      if (phase_il) {
        // Rows interleaved by phase: the GRP values of a group are consecutive phases p0 .. of one
        // channel at one column (RB = 32: channel 2 * (v >> 2) + half of the block; RB = 16:
        // channel quad, column block v >> 2), so they go to GRP consecutive samples.  Stored in
        // pairs, 8 bytes from one lane, where both samples exist; one by one at the sequence
        // ends.  Every address is formed from an existing sample (0 otherwise).
        const int chl = RB == 32 ? half : quad;
        auto cuof = [&](int c) { return NCB == 1 || c == 0 ? cu[0] : cu[NCB - 1]; };
        auto oqof = [&](int c) { return NCB == 1 || c == 0 ? oq[0] : oq[NCB - 1]; };
        typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
#pragma unroll
        for (int gg = 0; gg < NG; gg++)
          if (gg < ngrp) {
            const int vg = v0 + gg * GRP, cb = cbo(gg * GRP);
            const unsigned so = (unsigned) ((RB == 32 ? 2 * (vg >> 2) : 0) * ldy32) * 4u;
            const bool inq = oqof(cb);
            if constexpr (GRP == 1) {   // one value per wave (16-row tiles, 8-way split)
              const int sa = cuof(cb) + (vg & 3);
              if (inq && sa >= 0 && sa < ep.lout) {
                const unsigned vo = (unsigned) (chl * ldy32 + sa) * 4u;
                __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(val[gg]), ry, vo, so, 0);
                if (ep.y2 != nullptr)
                  __builtin_amdgcn_raw_buffer_store_b32(
                      __float_as_uint(val[gg] >= 0.0f ? val[gg] : ep.a2 * val[gg]), ry2, vo, so, 0);
              }
              continue;
            }
#pragma unroll
            for (int jj = 0; jj < GRP; jj += 2) {
              const int i = gg * GRP + jj;
              const int sa = cuof(cb) + (vg & 3) + jj;   // sample of value i; value i + 1 at sa + 1
              const bool va = inq && sa >= 0 && sa < ep.lout;
              const bool vb = inq && sa + 1 >= 0 && sa + 1 < ep.lout;
              const int sb = va ? sa : (vb ? sa + 1 : 0);
              const unsigned vo = (unsigned) (chl * ldy32 + sb) * 4u;
              const float y2a = val[i] >= 0.0f ? val[i] : ep.a2 * val[i];
              const float y2b = val[i + 1] >= 0.0f ? val[i + 1] : ep.a2 * val[i + 1];
              if (va && vb) {
                __builtin_amdgcn_raw_buffer_store_b64(u32x2{__float_as_uint(val[i]), __float_as_uint(val[i + 1])}, ry, vo, so, 0);
                if (ep.y2 != nullptr)
                  __builtin_amdgcn_raw_buffer_store_b64(u32x2{__float_as_uint(y2a), __float_as_uint(y2b)}, ry2, vo, so, 0);
              } else if (va || vb) {
                const float one = va ? val[i] : val[i + 1];
                __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(one), ry, vo, so, 0);
                if (ep.y2 != nullptr)
                  __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(va ? y2a : y2b), ry2, vo, so, 0);
              }
            }
          }
        continue;
      }
      // a group shares its column block, so one test covers its stores
#pragma unroll
      for (int gg = 0; gg < NG; gg++)
        if (gg < ngrp && okof(cbo(gg * GRP))) {
          const unsigned vo = (unsigned) (lrow * ldy32 + clof(cbo(gg * GRP))) * 4u;
#pragma unroll
          for (int jj = 0, i = gg * GRP; jj < GRP; jj++, i++) {
            const unsigned so = (unsigned) (urow(i) * ldy32) * 4u;
            __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(val[i]), ry, vo, so, 0);
            if (ep.y2 != nullptr)
              __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(val[i] >= 0.0f ? val[i] : ep.a2 * val[i]), ry2, vo, so, 0);
          }
        }
    }
    return;
  }

  // General path (partial row blocks, convT phases that straddle a block, large tensors): per
  // element
  reduce_wait();
  auto emit = [&](int nb, int v, float sum) {
    const int m = mb * RB + vrow(v);
    const long long q = q0 + vcol(nb, v);
    if (m >= M || q >= qend) return;
    int co = m, r = 0;
    if (phase_il) {
      r = m & 3;
      co = m >> 2;
    } else if (phase_rows) {
      r = m / C4;
      co = m - r * C4;
    }
    const long long col = q * ys + r - ypad;
    if (col < 0 || col >= Lout) return;
    float val = sum;
    for (int e = 0; e < nepi; e++) val = epi_apply(val, d.epi[e], b, co, col);
    const long long yi = (long long) co * ldy + col;
    yb[yi] = val;
    if (y2b != nullptr) y2b[yi] = val >= 0.0f ? val : a2 * val;
  };
#pragma unroll
  for (int nb = 0; nb < NB; nb++)
    for (int vv = 0; vv < nv; vv++) {
      const int v = v0 + vv;
      const float bv = bias_of(vrow(v));   // all lanes active here
      emit(nb, v, reduced(nb, v) + bv);
    }
}

static int conv_window(const ptk_conv_desc *d, int nb) {
  const int kd = (d->K - 1) * d->dil;
  return (32 * nb - 1) * d->stride + (kd < 0 ? -kd : kd) + 1;
}
static int win_max(int nb) { return nb == 2 ? WinGeo<2>::XWMAX : WinGeo<1>::XWMAX; }

// Kernel-selection knobs (PTK_*), read from the environment once per process, at the first
// launch that consults them, not per launch: launches come from many serving threads at once, and
// getenv is neither cheap nor safe against a concurrent setenv.  ptk_knobs_reload re-reads them
// (tests that change a knob between calls); each is an atomic int, so a launch running meanwhile
// sees the old or the new value of each knob.
enum KnobId {
  KN_CONV_SPLIT, KN_CONV_RB, KN_CONV_S8, KN_CONV_S8_MAX, KN_CONV_NB, KN_CONV_FAST, KN_TAIL_OUT,
  KN_TAIL_GRID, KN_TAIL_XCD, KN_NARROW, KN_COUNT
};
static const struct {
  const char *name;
  int dflt;
} kKnobs[KN_COUNT] = {{"PTK_CONV_SPLIT", 0}, {"PTK_CONV_RB", 0},    {"PTK_CONV_S8", 1},
                      {"PTK_CONV_S8_MAX", 1536}, {"PTK_CONV_NB", 0}, {"PTK_CONV_FAST", 1},
                      {"PTK_TAIL_OUT", 0},
                      {"PTK_TAIL_GRID", 0},   {"PTK_TAIL_XCD", 1},  {"PTK_NARROW", 1}};
static std::atomic<int> g_knob[KN_COUNT];
static std::once_flag g_knob_once;
static std::mutex g_knob_lock;

static void knobs_read() {
  std::lock_guard<std::mutex> lk(g_knob_lock);
  for (int i = 0; i < KN_COUNT; i++) {
    const char *e = getenv(kKnobs[i].name);
    g_knob[i].store(e ? atoi(e) : kKnobs[i].dflt, std::memory_order_relaxed);
  }
}
static int knob(KnobId k) {
  std::call_once(g_knob_once, knobs_read);
  return g_knob[k].load(std::memory_order_relaxed);
}
extern "C" void ptk_knobs_reload(void) {
  std::call_once(g_knob_once, knobs_read);
  knobs_read();
}

// Tile shape (RB rows, channel split S in {1, 2, 4, 8}; PTK_CONV_RB and PTK_CONV_SPLIT override).
// All waves of a launch usually fit on the chip at once, so a launch lasts as long as its busiest
// SIMD: with W waves over the 1024 SIMDs (256 CUs x 4) that SIMD holds ceil(W / 1024) of them
// while the mean is W / 1024.  Fewer than ~3 waves per SIMD also leave MFMA latency exposed (a
// lone wave keeps its SIMD's matrix pipe ~60 % busy), and each split step costs its LDS reduction
// and a share of the edges.  The model below, fitted to decoder shapes measured on MI355X (batch 1
// and 22, C 128 / 256, K 3-11), picks the shape with the best predicted MFMA occupancy:
//   eff = [mean / max waves per SIMD] x [latency hiding at the mean] x [split cost]
//         x [rows that exist / rows computed] x [16-row tile cost]
// evaluated on ONE batch item's grid (of nq_shape columns when the launch covers a sub-range).
// The shape fixes the order in which a block's partial sums are added, so choosing it without the
// batch size makes a batched item's result bit-identical to the same item decoded alone (and it
// measured faster at batch 8 than a batch-aware choice).
// 16-row tiles double the waves of a grid (and cut the padding of row counts like 72), at twice
// the window staging and epilogue work per MFMA.  They need the 16-row weight copy (w16) and are
// offered to single-problem launches only (PTK_CONV_RB=16 forces them on any launch with the
// copy): the grouped MRF launches at small T ran as fast or faster alone on 16-row tiles, but
// the concurrent serving step, where other streams fill the chip anyway, lost 1.4 % of its
// throughput to their extra work per MFMA.  kRb16Cost = 0.7 puts conv_pre (T 226) and conv_post
// on 16-row tiles and keeps ups.0 / ups.1 on 32-row ones, as measured at batch 1.
static const double kSimds = 1024.0;
static const double kRb16Cost = 0.70;
static double split_eff(long long waves, int S) {
  const double m = (double) waves / kSimds;
  // past residency the extra waves run as one more wave on the SIMDs they land on
  const double busiest = ceil(m);
  const double balance = m / (busiest > 0.0 ? busiest : 1.0);
  const double mh = m < 4.0 ? m : 4.0;
  const double hide = mh >= 2.75 ? 1.0 : 0.45 + 0.2 * mh;
  const double cost = S == 1 ? 1.0 : (S == 2 ? 0.97 : 0.90);
  return balance * hide * cost;
}
static int choose_tiles(const ptk_conv_desc *const *ds, int n, int nb, int *rb_out) {
  const int env_s = knob(KN_CONV_SPLIT), env_rb = knob(KN_CONV_RB);
  bool rb16_ok = nb == 1 && (n == 1 || env_rb == 16);
  for (int i = 0; i < n; i++)
    if (ds[i]->w16 == nullptr) rb16_ok = false;
  int best = 4, best_rb = 32;
  long long best_waves = 0;
  double best_eff = -1.0;
  for (int RB = 32; RB >= 16; RB /= 2) {
    if (RB == 16 && !rb16_ok) continue;
    if ((env_rb == 16 || env_rb == 32) && RB != env_rb && (env_rb == 32 || rb16_ok)) continue;
    for (int S = 1; S <= 4; S *= 2) {
      if ((env_s == 1 || env_s == 2 || env_s == 4) && S != env_s) continue;
      const int G = 4 / S;
      long long waves = 0;
      double rows = 0.0, rows_run = 0.0;
      for (int i = 0; i < n; i++) {
        const ptk_conv_desc *d = ds[i];
        const long long nq = d->nq_shape > 0 ? d->nq_shape : d->nq;
        const long long mt = (d->M + RB - 1) / RB;
        const long long tiles = mt * ((nq + 32LL * nb * G - 1) / (32LL * nb * G));
        waves += 4LL * tiles;
        const double work = (double) nq * d->K * d->cinp;
        rows += work * d->M;
        rows_run += work * (double) (mt * RB);
      }
      const double e = split_eff(waves, S) * (rows_run > 0.0 ? rows / rows_run : 1.0) *
                       (RB == 16 ? kRb16Cost : 1.0);
      if (e > best_eff + 1e-9) {
        best_eff = e;
        best = S;
        best_rb = RB;
        best_waves = waves;
      }
    }
  }
  // The 8-way split (8-wave workgroups over the same tiles): for a single problem on 32-row
  // tiles whose 4-way grid leaves one lone wave on most SIMDs (1 to 1.5 waves per SIMD), it
  // doubles the waves that hide each other's latency at the cost of twice the partial sums.  On
  // 16-row tiles, which already do more staging and epilogue work per MFMA, it measured no faster
  // alone and slower batched.  Needs whole chunks for all eight waves (cinp a multiple of 64).
  // PTK_CONV_SPLIT=8 forces it where it applies, PTK_CONV_S8=0 turns the rule off,
  // PTK_CONV_S8_MAX sets the upper bound in waves (1536).
  const bool s8_ok = nb == 1 && n == 1 && ds[0]->cinp % (8 * CONV_CK) == 0;
  const long long s8_max = knob(KN_CONV_S8_MAX);
  if (s8_ok && (env_s == 8 || (env_s == 0 && knob(KN_CONV_S8) != 0 && best == 4 &&
                               best_rb == 32 && best_waves >= (long long) kSimds &&
                               best_waves < s8_max)))
    best = 8;
  *rb_out = best_rb;
  return best;
}

// column blocks per wave: 1.  Two blocks halve the weight loads per MFMA but double the window
// registers and halve the grid; on MI355X they lost at every decoder shape measured (batch 1 and
// 8), so they are only used when PTK_CONV_NB=2 asks for them.
static int choose_nb(const ptk_conv_desc *d) {
  const int env_nb = knob(KN_CONV_NB);
  if (env_nb == 2 && conv_window(d, 2) <= win_max(2)) return 2;
  return 1;
}

extern "C" int ptk_conv_mfma_ok(const ptk_conv_desc *d) {
  if (d->M < 16 || d->cin < 2 || d->K < 1 || d->stride < 1 || d->dil == 0) return 0;
  if (conv_window(d, 1) > win_max(1)) return 0;
  if (d->cinp != ptk_conv_cinp(d->cin)) return 0;
  // 32-bit buffer offsets: every row offset plus the out-of-range marker must stay below 2^32
  if ((unsigned long long) d->cinp * (unsigned long long) d->ldx * 4ULL >= 0x80000000ULL) return 0;
  return 1;
}

template <int KT, int NB, int IN, int RB, int NW>
static void launch_conv(const ConvGroup &g, dim3 grid, hipStream_t s) {
  constexpr size_t lds = LdsGeo<NB, RB, NW>::BYTES;
  hipLaunchKernelGGL((conv_mfma_kernel<KT, NB, IN, RB, NW>), grid, dim3(64 * NW), lds, s, g);
}

template <int NB, int IN, int RB, int NW>
static void launch_conv_k(int kmax, const ConvGroup &g, dim3 grid, hipStream_t s) {
  if (kmax <= 3) launch_conv<3, NB, IN, RB, NW>(g, grid, s);
  else if (kmax == 4) launch_conv<4, NB, IN, RB, NW>(g, grid, s);
  else if (kmax <= 7) launch_conv<7, NB, IN, RB, NW>(g, grid, s);
  else if (kmax <= 11) launch_conv<11, NB, IN, RB, NW>(g, grid, s);
  else launch_conv<0, NB, IN, RB, NW>(g, grid, s);
}

template <int NB, int RB, int NW>
static void launch_conv_in(int in_op, int kmax, const ConvGroup &g, dim3 grid, hipStream_t s) {
  if (in_op == PTK_IN_LEAKY) launch_conv_k<NB, PTK_IN_LEAKY, RB, NW>(kmax, g, grid, s);
  else launch_conv_k<NB, PTK_IN_PLAIN, RB, NW>(kmax, g, grid, s);
}

extern "C" int ptk_conv_launch(const ptk_conv_desc *dd, int ngroup, void *stream) {
  if (ngroup < 1 || ngroup > PTK_MAX_GROUP) {
    set_err("ptk_conv_launch: ngroup %d out of range", ngroup);
    return -1;
  }
  ConvGroup g;
  memset(&g, 0, sizeof g);
  // heaviest problems first, so their long workgroups start before the short ones
  int order[PTK_MAX_GROUP];
  for (int i = 0; i < ngroup; i++) order[i] = i;
  for (int i = 0; i < ngroup; i++)
    for (int j = i + 1; j < ngroup; j++)
      if ((long long) dd[order[j]].K * dd[order[j]].cinp > (long long) dd[order[i]].K * dd[order[i]].cinp) {
        const int t = order[i];
        order[i] = order[j];
        order[j] = t;
      }
  const int nb = choose_nb(&dd[order[0]]);
  int kmax = 0, in_op = -1;
  int total = 0;
  const ptk_conv_desc *live[PTK_MAX_GROUP];
  for (int i = 0; i < ngroup; i++) {
    const ptk_conv_desc *d = &dd[order[i]];
    if (!ptk_conv_mfma_ok(d) || conv_window(d, nb) > win_max(nb)) {
      set_err("ptk_conv_launch: shape outside the MFMA kernel (M %d cin %d K %d dil %d stride %d)",
              d->M, d->cin, d->K, d->dil, d->stride);
      return -1;
    }
    if (d->nq <= 0 || d->batch <= 0) continue;
    if (d->ext_l < 0 || d->ext_r < 0 || d->nq_shape < 0 || d->ext_l >= (1LL << 30) ||
        d->ext_r >= (1LL << 30)) {
      set_err("ptk_conv_launch: column extension or shape width out of range");
      return -1;
    }
    // a row tile's weight panel is addressed through one buffer resource (the input rows are
    // bounded the same way by ptk_conv_mfma_ok)
    if ((unsigned long long) d->K * (unsigned long long) (d->cinp / CONV_CK) * 1024ull >= (unsigned long long) PTK_OOB) {
      set_err("ptk_conv_launch: weight panel (K %d, cin %d) reaches the 2 GiB range of one buffer "
              "resource", d->K, d->cin);
      return -1;
    }
    if (d->phase_il && !(d->M == 4 * d->C4 && d->ys == 4 && d->dil == -1 && d->stride == 1 &&
                         d->K == 4 && ngroup == 1)) {
      set_err("ptk_conv_launch: rows interleaved by phase need a single stride-4 convT in the "
              "4-tap phase form (M %d, rows per phase %d, %d taps)", d->M, d->C4, d->K);
      return -1;
    }
    if (d->in_op != PTK_IN_PLAIN && !(d->in_a >= 0.0f && d->in_a <= 1.0f)) {
      set_err("ptk_conv_launch: input LeakyReLU slope %g outside [0, 1]", (double) d->in_a);
      return -1;
    }
    if (in_op < 0) in_op = d->in_op;
    if (d->in_op != in_op || d->in_op < PTK_IN_PLAIN || d->in_op > PTK_IN_LEAKY) {
      set_err("ptk_conv_launch: grouped problems need one valid input transform");
      return -1;
    }
    if (d->K > kmax) kmax = d->K;
    g.d[g.ngroup] = *d;
    live[g.ngroup] = d;
    g.ngroup++;
  }
  if (g.ngroup == 0) return 0;
  int rb = 32, maxcount = 0;
  const int S = choose_tiles(live, g.ngroup, nb, &rb), NW = S == 8 ? 8 : 4, G = NW / S;
  g.split = S;
  g.lg_split = S == 8 ? 3 : S == 4 ? 2 : S == 2 ? 1 : 0;
  for (int i = 0; i < g.ngroup; i++) {
    const ptk_conv_desc *d = live[i];
    ConvProb &pi = g.info[i];
    const long long cols = 32LL * nb * G;   // columns of one tile
    pi.mt = (d->M + rb - 1) / rb;
    pi.nt = (int) ((d->nq + cols - 1) / cols);
    pi.nitem = d->batch;
    long long n;
    if (d->batch == 1) {
      pi.nt0 = pi.ntl = (int) ((d->nq + d->ext_l + d->ext_r + cols - 1) / cols);
      n = (long long) pi.mt * pi.nt0;
    } else {
      pi.nt0 = (int) ((d->nq + d->ext_l + cols - 1) / cols);
      pi.ntl = (int) ((d->nq + d->ext_r + cols - 1) / cols);
      n = (long long) pi.mt * (pi.nt0 + (long long) (d->batch - 2) * pi.nt + pi.ntl);
    }
    if (n >= (1LL << 24) || total + n >= (1LL << 31)) {
      set_err("ptk_conv_launch: %lld workgroups for one problem (the tile decode takes < 2^24)", n);
      return -1;
    }
    total += (int) n;
    pi.count = (int) n;
    if (pi.count > maxcount) maxcount = pi.count;
    pi.div_tiles = fast_div((unsigned) (pi.mt * pi.nt));
    pi.div_mt = fast_div((unsigned) pi.mt);
    const bool il = d->phase_il != 0;
    const bool one_phase = !il && (d->C4 == d->M || d->C4 % rb == 0);
    pi.div_phase = fast_div(d->C4 == d->M ? 1u : (unsigned) (d->C4 / rb > 0 ? d->C4 / rb : 1));
    pi.addt = -1;
    int naddt = 0;
    for (int e = 0; e < d->nepi; e++)
      if (d->epi[e].op == PTK_EPI_ADDT && naddt++ == 0) pi.addt = e;
    pi.M = d->M;
    // the fast epilogue's 32-bit indices: columns, and byte offsets from a row block's first row
    const long long lim31 = 1LL << 31, lim30 = 1LL << 30;
    bool fast = (one_phase || il) && d->ldy < (1LL << 23) && d->Lout < lim30 &&
                (d->q0 + d->nq + d->ext_r) * d->ys + d->C4 < lim30 && d->q0 - d->ext_l >= 0 &&
                ((long long) rb * d->ldy + d->Lout) * 4 < lim31;
    // the fast epilogue reads one tensor operand (loaded ahead of the reduction); a chain with two
    // takes the general path
    if (naddt > 1) fast = false;
    // the interleaved-phase stores have no tensor-add operand loads: such a chain takes the
    // general path, and so do outputs where a sample pair is not 8-byte aligned (64-bit stores)
    if (il && (pi.addt >= 0 || ((d->ldy | d->bsy) & 1) != 0 || ((uintptr_t) d->y & 7) != 0 ||
               ((uintptr_t) d->y2 & 7) != 0))
      fast = false;
    // PTK_CONV_FAST=0: every block through the general per-element epilogue (tests compare the
    // two epilogues)
    if (!knob(KN_CONV_FAST)) fast = false;
    if (pi.addt >= 0) {
      const long long ldt = d->epi[pi.addt].ldt;
      fast = fast && ldt >= 0 && ldt < (1LL << 23) && ((long long) rb * ldt + d->Lout) * 4 < lim31;
    }
    pi.flags = (one_phase ? PROB_ONE_PHASE : 0) | (fast ? PROB_FAST : 0) | (il ? PROB_PHASE_IL : 0);
    pi.ext_l = (int) d->ext_l;
    ConvEpi &ep = g.ep[i];
    ep.y = d->y;
    ep.y2 = d->y2;
    ep.bsy = d->bsy;
    ep.t = pi.addt >= 0 ? d->epi[pi.addt].t : nullptr;
    ep.bst = pi.addt >= 0 ? d->epi[pi.addt].bst : 0;
    ep.ldy = (int) d->ldy;
    ep.ldt = pi.addt >= 0 ? (int) d->epi[pi.addt].ldt : 0;
    ep.lout = (int) d->Lout;
    ep.qend = (int) (d->q0 + d->nq);
    ep.ext_r = (int) d->ext_r;
    ep.ys = d->ys;
    ep.ypad = d->ypad;
    ep.C4 = d->C4;
    ep.nepi = d->nepi;
    ep.ops = 0;
    for (int e = 0; e < PTK_MAX_EPI; e++) {
      const int op = e < d->nepi ? d->epi[e].op : PTK_EPI_NONE;
      // codes outside the table are no-ops, as in epi_apply
      ep.ops |= (op >= PTK_EPI_NONE && op <= PTK_EPI_DIVS ? op : PTK_EPI_NONE) << (4 * e);
      ep.a[e] = e < d->nepi ? d->epi[e].a : 0.0f;
    }
    ep.a2 = d->a2;
  }
  if (total == 0) return 0;
  hipStream_t s = (hipStream_t) stream;
  const dim3 grid((unsigned) maxcount, (unsigned) g.ngroup);
  if (nb == 2) launch_conv_in<2, 32, 4>(in_op, kmax, g, grid, s);
  else if (NW == 8 && rb == 16) launch_conv_in<1, 16, 8>(in_op, kmax, g, grid, s);
  else if (NW == 8) launch_conv_in<1, 32, 8>(in_op, kmax, g, grid, s);
  else if (rb == 16) launch_conv_in<1, 16, 4>(in_op, kmax, g, grid, s);
  else launch_conv_in<1, 32, 4>(in_op, kmax, g, grid, s);
  HCHK(hipGetLastError());
  return 0;
}

// ------------------------------------------------------------------------------ narrow convs
// Convs and convTs with few output rows on the reference ABI path (cout4 < 16, channel counts 1,
// 4 or 16: the PQMF synthesis FIR 4 -> 1 K 63; the iSTFT overlap-add 16 -> 1 and window sum
// 1 -> 1, K 16 s 4; the PQMF x4 zero-insert 4 -> 4 K 4 s 4).  A workgroup stages in LDS, once,
// the input window its outputs read, as [column][CIN] (a column's channels in one to four 16-byte
// reads; the column stride padded to CIN + 4 floats for CIN 16, so a wave's reads spread over all
// banks), and the real rows' weights, [row][tap][CIN] (conv) or [row][tap][CIN][s] (convT).  Each
// output is one chain of FMAs in the generic kernels' order (bias, tap ascending, channel
// ascending, taps whose input column is outside the sequence skipped), so the results are the
// same bits.  The chip is nearly empty at these sizes, so the work is spread over many waves: one
// conv output per thread, its taps' operands read one tap ahead into two alternating register
// sets; a convT step's s phases per thread, sharing each input value.  (A first form, a plain loop
// with its reads waiting one at a time, took 14-38 us per launch; four conv outputs per thread
// gave 228 waves each issuing ~4700 instructions one at a time: 19 us.)  The layout's padding rows
// (cout..cout4-1, zero weights and bias) get the epilogue of 0 without the sums.  Other channel
// counts, windows past NARROW_LDS_FLOATS and sizes past 2^31 take the generic kernels below;
// PTK_NARROW=0 forces them everywhere.
#define NARROW_THREADS 256
#define NARROW_LDS_FLOATS 12288   // 48 KB of dynamic LDS per workgroup
#define NARROW_SMAX 4             // convT phases (stride) a thread keeps in registers

// floats per staged window column
template <int CIN>
__host__ __device__ constexpr int narrow_cs() { return CIN >= 16 ? CIN + 4 : CIN; }

// CIN consecutive floats from LDS (16-byte aligned when CIN % 4 == 0) into registers
template <int CIN>
__device__ __forceinline__ void lds_cols(float (&v)[CIN], const float *p) {
  if constexpr (CIN % 4 == 0) {
#pragma unroll
    for (int q = 0; q < CIN / 4; q++) {
      const float4 t = reinterpret_cast<const float4 *>(p)[q];
      v[4 * q] = t.x;
      v[4 * q + 1] = t.y;
      v[4 * q + 2] = t.z;
      v[4 * q + 3] = t.w;
    }
  } else {
#pragma unroll
    for (int i = 0; i < CIN; i++) v[i] = p[i];
  }
}

// Stages columns [0, win) of rows [0, CIN) into xs[col][narrow_cs<CIN>] (column c0 + col of the
// item, 0 outside [0, lim)).  A thread's columns col = tid + p * NARROW_THREADS are taken PG at a
// time, and all PG * CIN loads of a group are issued before its stores, so the window costs about
// one global load latency per group.
template <int CIN>
__device__ __forceinline__ void narrow_stage(float *__restrict__ xs, const float *__restrict__ xb,
                                             long long ldx, int c0, int lim, int win, int tid) {
  constexpr int PG = CIN >= 16 ? 2 : 16 / CIN, CS = narrow_cs<CIN>();
  for (int col0 = tid; col0 < win; col0 += PG * NARROW_THREADS) {
    float v[PG][CIN];
#pragma unroll
    for (int g = 0; g < PG; g++) {
      const int c = c0 + col0 + g * NARROW_THREADS;
      const bool ok = col0 + g * NARROW_THREADS < win && c >= 0 && c < lim;
      const float *src = xb + (ok ? c : 0);
#pragma unroll
      for (int ci = 0; ci < CIN; ci++) v[g][ci] = ok ? src[(long long) ci * ldx] : 0.0f;
    }
#pragma unroll
    for (int g = 0; g < PG; g++) {
      const int col = col0 + g * NARROW_THREADS;
      if (col >= win) break;
      if constexpr (CIN % 4 == 0) {
#pragma unroll
        for (int q = 0; q < CIN / 4; q++)
          reinterpret_cast<float4 *>(xs + col * CS)[q] =
              make_float4(v[g][4 * q], v[g][4 * q + 1], v[g][4 * q + 2], v[g][4 * q + 3]);
      } else {
#pragma unroll
        for (int ci = 0; ci < CIN; ci++) xs[col * CS + ci] = v[g][ci];
      }
    }
  }
}

template <int CIN>
__device__ __forceinline__ float narrow_fma(float acc, const float (&w)[CIN], const float (&x)[CIN]) {
#pragma unroll
  for (int ci = 0; ci < CIN; ci++) acc += w[ci] * x[ci];
  return acc;
}

template <int CIN>
__global__ void __launch_bounds__(NARROW_THREADS) conv_narrow_kernel(
    const float *__restrict__ x, long long ldx, long long bsx, int lim, const float *__restrict__ wp,
    const float *__restrict__ bias, int cout, int K, int st, int dil, int shift,
    float *__restrict__ y, long long ldy, long long bsy, int n, int win, int epi0, float a0,
    int epi1, float a1) {
  constexpr int CS = narrow_cs<CIN>();
  extern __shared__ float4 lds4[];
  float *const xs = reinterpret_cast<float *>(lds4);   // [win][CS]; column 0 = input t0*st - shift
  float *const ws = xs + ((win * CS + 3) & ~3);        // [cout][K][CIN]
  const int tid = threadIdx.x, b = blockIdx.y;
  const int t0 = blockIdx.x * NARROW_THREADS;
  narrow_stage<CIN>(xs, x + (long long) b * bsx, ldx, t0 * st - shift, lim, win, tid);
  for (int i = tid; i < cout * K * CIN; i += NARROW_THREADS) {
    const int m = i / (K * CIN), r = i - m * (K * CIN), k = r / CIN, ci = r - k * CIN;
    ws[i] = wp[((long long) (m >> 2) * K + k) * CIN * 4 + ci * 4 + (m & 3)];
  }
  __syncthreads();
  const int t = t0 + tid;
  if (t >= n) return;
  // taps whose input column t * st + k * dil - shift lies in [0, lim): k in [klo, khi)
  const int base = t * st - shift;
  int klo = base >= 0 ? 0 : (-base + dil - 1) / dil;
  int khi = base >= lim ? 0 : (lim - base + dil - 1) / dil;
  khi = khi < K ? khi : K;
  klo = klo < khi ? klo : khi;
  const int c4 = (cout + 3) & ~3;
  const ptk_epi e0 = {epi0, a0, nullptr, 0, 0}, e1 = {epi1, a1, nullptr, 0, 0};
  const float *const xt = xs + tid * st * CS;
  const int kstep = dil * CS;
  for (int m = 0; m < c4; m++) {
    float v = (bias != nullptr && m < cout) ? bias[m] : 0.0f;
    if (m < cout && klo < khi) {
      const float *const wm = ws + m * K * CIN;
      // operands of the next tap read into the other register set while this tap's FMAs run;
      // the read is unconditional (a tap past the last re-reads the last), so the wait before
      // the FMAs leaves it in flight
      const int klast = khi - 1;
      float wa[CIN], xa[CIN], wb[CIN], xb2[CIN];
      lds_cols<CIN>(wa, wm + klo * CIN);
      lds_cols<CIN>(xa, xt + klo * kstep);
      for (int k = klo;; k += 2) {
        const int k1 = k + 1 < klast ? k + 1 : klast, k2 = k + 2 < klast ? k + 2 : klast;
        lds_cols<CIN>(wb, wm + k1 * CIN);
        lds_cols<CIN>(xb2, xt + k1 * kstep);
        v = narrow_fma<CIN>(v, wa, xa);
        if (k + 1 >= khi) break;
        lds_cols<CIN>(wa, wm + k2 * CIN);
        lds_cols<CIN>(xa, xt + k2 * kstep);
        v = narrow_fma<CIN>(v, wb, xb2);
        if (k + 2 >= khi) break;
      }
    }
    if (epi0) v = epi_apply(v, e0, b, m, t);
    if (epi1) v = epi_apply(v, e1, b, m, t);
    y[(long long) b * bsy + (long long) m * ldy + t] = v;
  }
}

// Thread tid of workgroup bx takes the delay-line step q = qlo + bx * NARROW_THREADS + tid and its
// s outputs oi = q * s + r - pad (r < s) that fall in [0, Lout), all s phases at once (s
// independent sums over the same input values); the window holds input columns
// [q0 - ntap + 1, q0 + NARROW_THREADS) of the workgroup's first step q0.
template <int CIN>
__global__ void __launch_bounds__(NARROW_THREADS) convT_narrow_kernel(
    const float *__restrict__ x, long long ldx, long long bsx, int tin, const float *__restrict__ wp,
    const float *__restrict__ bias, int cout, int s, int pad, int ntap, float *__restrict__ y,
    long long ldy, long long bsy, int Lout, int qlo, int nq, int win) {
  constexpr int CS = narrow_cs<CIN>();
  extern __shared__ float4 lds4[];
  float *const xs = reinterpret_cast<float *>(lds4);   // [win][CS]
  float *const ws = xs + ((win * CS + 3) & ~3);        // [cout][ntap][CIN][NARROW_SMAX]
  const int tid = threadIdx.x, b = blockIdx.y;
  const int c4 = (cout + 3) & ~3;
  const int q0 = qlo + blockIdx.x * NARROW_THREADS;
  narrow_stage<CIN>(xs, x + (long long) b * bsx, ldx, q0 - ntap + 1, tin, win, tid);
  for (int i = tid; i < cout * ntap * CIN * NARROW_SMAX; i += NARROW_THREADS) {
    const int r = i % NARROW_SMAX, rest = i / NARROW_SMAX, ci = rest % CIN, rest2 = rest / CIN;
    const int j = rest2 % ntap, co = rest2 / ntap, row = r * c4 + co;
    ws[i] = r < s ? wp[((long long) (row >> 2) * ntap + j) * CIN * 4 + ci * 4 + (row & 3)] : 0.0f;
  }
  __syncthreads();
  const int q = q0 + tid;
  if (q - qlo >= nq) return;
  // taps whose input column q - j lies in [0, tin): j in [jlo, jhi)
  const int jlo = q >= tin ? q - tin + 1 : 0;
  const int jhi = q + 1 < ntap ? q + 1 : ntap;
  float *yb = y + (long long) b * bsy;
  const float *const xq = xs + (tid + ntap - 1) * CS;   // input column q - j at xq[-j * CS]
  for (int co = 0; co < c4; co++) {
    const float bv = (bias != nullptr && co < cout) ? bias[co] : 0.0f;
    float acc[NARROW_SMAX];
#pragma unroll
    for (int r = 0; r < NARROW_SMAX; r++) acc[r] = bv;
    if (co < cout) {
      const float *const wc = ws + co * ntap * CIN * NARROW_SMAX;
      for (int j = jlo; j < jhi; j++) {
        // the tap's operands all read before its FMAs
        float xv[CIN], w[CIN][NARROW_SMAX];
        lds_cols<CIN>(xv, xq - j * CS);
#pragma unroll
        for (int ci = 0; ci < CIN; ci++) lds_cols<NARROW_SMAX>(w[ci], wc + (j * CIN + ci) * NARROW_SMAX);
#pragma unroll
        for (int ci = 0; ci < CIN; ci++)
#pragma unroll
          for (int r = 0; r < NARROW_SMAX; r++) acc[r] += w[ci][r] * xv[ci];
      }
    }
#pragma unroll
    for (int r = 0; r < NARROW_SMAX; r++) {
      const int oi = q * s + r - pad;
      if (r < s && oi >= 0 && oi < Lout) yb[(long long) co * ldy + oi] = acc[r];
    }
  }
}

// ------------------------------------------------------------------------------ SIMT fallbacks
// Any shape the MFMA and narrow kernels do not take: one thread per output, summing over tap then
// channel onto the bias in the reference's order.
__global__ void conv_simt_kernel(const float *__restrict__ x, long long ldx, long long bsx,
                                 long long lim, int cin, const float *__restrict__ wp,
                                 const float *__restrict__ bias, int cout, int K, int st, int dil,
                                 int shift, float *__restrict__ y, long long ldy, long long bsy,
                                 long long n, int epi0, float a0, int epi1, float a1) {
  const long long t = (long long) blockIdx.x * blockDim.x + threadIdx.x;
  const int m = blockIdx.y, b = blockIdx.z;
  if (t >= n) return;
  const float *xb = x + (long long) b * bsx;
  const float *wq = wp + (long long) (m >> 2) * K * cin * 4 + (m & 3);
  float v = (bias != nullptr && m < cout) ? bias[m] : 0.0f;
  for (int k = 0; k < K; k++) {
    const long long c = t * st + (long long) k * dil - shift;
    if (c < 0 || c >= lim) continue;
    const float *wk = wq + (long long) k * cin * 4;
    for (int ci = 0; ci < cin; ci++) v += wk[ci * 4] * xb[(long long) ci * ldx + c];
  }
  ptk_epi e0 = {epi0, a0, nullptr, 0, 0}, e1 = {epi1, a1, nullptr, 0, 0};
  if (epi0) v = epi_apply(v, e0, b, m, t);
  if (epi1) v = epi_apply(v, e1, b, m, t);
  y[(long long) b * bsy + (long long) m * ldy + t] = v;
}

extern "C" int ptk_conv_simt(const float *x, int64_t ldx, int64_t bsx, int64_t lim, int cin,
                             const float *wp, const float *bias, int cout, int K, int stride,
                             int dil, int shift, float *y, int64_t ldy, int64_t bsy, int64_t n,
                             int batch, int epi0, float a0, int epi1, float a1, void *s) {
  if (n <= 0 || batch <= 0) return 0;
  // no residual tensor reaches these kernels: a tensor add would read through a null pointer
  if (epi0 == PTK_EPI_ADDT || epi1 == PTK_EPI_ADDT) {
    set_err("ptk_conv_simt: epilogue code %d (tensor add) takes no tensor here", PTK_EPI_ADDT);
    return -1;
  }
  const long long per_wg = NARROW_THREADS;
  const long long win = (per_wg - 1) * stride + (long long) (K - 1) * dil + 1;
  const long long cs = cin >= 16 ? cin + 4 : cin;
  const long long lds_floats = ((cs * win + 3) & ~3LL) + (long long) cout * K * cin;
  // 32-bit column arithmetic in the kernel: every window column, output and input index < 2^31
  const bool small = lim < INT32_MAX && (n + per_wg) * stride + win + shift < INT32_MAX;
  if (knob(KN_NARROW) && (cin == 1 || cin == 4 || cin == 16) && dil >= 1 && stride >= 1 && small &&
      lds_floats <= NARROW_LDS_FLOATS) {
    dim3 grid((unsigned) ((n + per_wg - 1) / per_wg), (unsigned) batch);
    const size_t lds = (size_t) lds_floats * sizeof(float);
#define NARROW_CONV_LAUNCH(CINV)                                                                  \
  hipLaunchKernelGGL(conv_narrow_kernel<CINV>, grid, dim3(NARROW_THREADS), lds, (hipStream_t) s, x, \
                     (long long) ldx, (long long) bsx, (int) lim, wp, bias, cout, K, stride, dil,  \
                     shift, y, (long long) ldy, (long long) bsy, (int) n, (int) win, epi0, a0,     \
                     epi1, a1)
    if (cin == 1) NARROW_CONV_LAUNCH(1);
    else if (cin == 4) NARROW_CONV_LAUNCH(4);
    else NARROW_CONV_LAUNCH(16);
#undef NARROW_CONV_LAUNCH
    HCHK(hipGetLastError());
    return 0;
  }
  const int c4 = (cout + 3) / 4 * 4;
  dim3 grid((unsigned) ((n + 255) / 256), (unsigned) c4, (unsigned) batch);
  hipLaunchKernelGGL(conv_simt_kernel, grid, dim3(256), 0, (hipStream_t) s, x, (long long) ldx,
                     (long long) bsx, (long long) lim, cin, wp, bias, cout, K, stride, dil, shift,
                     y, (long long) ldy, (long long) bsy, (long long) n, epi0, a0, epi1, a1);
  HCHK(hipGetLastError());
  return 0;
}

__global__ void convT_simt_kernel(const float *__restrict__ x, long long ldx, long long bsx,
                                  long long tin, int cin, const float *__restrict__ wp,
                                  const float *__restrict__ bias, int cout, int s, int pad, int ntap,
                                  float *__restrict__ y, long long ldy, long long bsy, long long Lout) {
  const long long oi = (long long) blockIdx.x * blockDim.x + threadIdx.x;
  const int co = blockIdx.y, b = blockIdx.z;
  if (oi >= Lout) return;
  const int c4 = (cout + 3) / 4 * 4;
  const long long u = oi + pad;
  const long long q = u / s;
  const int r = (int) (u - q * s);
  const int row = r * c4 + co;
  const float *wq = wp + (long long) (row >> 2) * ntap * cin * 4 + (row & 3);
  const float *xb = x + (long long) b * bsx;
  float v = (bias != nullptr && co < cout) ? bias[co] : 0.0f;
  for (int j = 0; j < ntap; j++) {
    const long long c = q - j;
    if (c < 0 || c >= tin) continue;
    const float *wj = wq + (long long) j * cin * 4;
    for (int ci = 0; ci < cin; ci++) v += wj[ci * 4] * xb[(long long) ci * ldx + c];
  }
  y[(long long) b * bsy + (long long) co * ldy + oi] = v;
}

extern "C" int ptk_convT_simt(const float *x, int64_t ldx, int64_t bsx, int64_t tin, int cin,
                              const float *wp, const float *bias, int cout, int st, int pad, int K,
                              float *y, int64_t ldy, int64_t bsy, int64_t Lout, int batch, void *s) {
  if (Lout <= 0 || batch <= 0) return 0;
  const int c4 = (cout + 3) / 4 * 4;
  const int ntap = (K + st - 1) / st;
  const long long win = NARROW_THREADS + ntap - 1;
  const long long cs = cin >= 16 ? cin + 4 : cin;
  const long long lds_floats = ((cs * win + 3) & ~3LL) + (long long) NARROW_SMAX * cout * ntap * cin;
  const bool small = tin < INT32_MAX - NARROW_THREADS && Lout + pad + (long long) NARROW_THREADS * st < INT32_MAX;
  if (knob(KN_NARROW) && (cin == 1 || cin == 4 || cin == 16) && st >= 1 && st <= NARROW_SMAX &&
      pad >= 0 && small && lds_floats <= NARROW_LDS_FLOATS) {
    // delay-line steps with an output in [0, Lout): u = oi + pad = q * st + r
    const long long qlo = pad / st, nq = (Lout - 1 + pad) / st - qlo + 1;
    dim3 grid((unsigned) ((nq + NARROW_THREADS - 1) / NARROW_THREADS), (unsigned) batch);
    const size_t lds = (size_t) lds_floats * sizeof(float);
#define NARROW_CONVT_LAUNCH(CINV)                                                                 \
  hipLaunchKernelGGL(convT_narrow_kernel<CINV>, grid, dim3(NARROW_THREADS), lds, (hipStream_t) s, \
                     x, (long long) ldx, (long long) bsx, (int) tin, wp, bias, cout, st, pad, ntap, \
                     y, (long long) ldy, (long long) bsy, (int) Lout, (int) qlo, (int) nq, (int) win)
    if (cin == 1) NARROW_CONVT_LAUNCH(1);
    else if (cin == 4) NARROW_CONVT_LAUNCH(4);
    else NARROW_CONVT_LAUNCH(16);
#undef NARROW_CONVT_LAUNCH
    HCHK(hipGetLastError());
    return 0;
  }
  dim3 grid((unsigned) ((Lout + 255) / 256), (unsigned) c4, (unsigned) batch);
  hipLaunchKernelGGL(convT_simt_kernel, grid, dim3(256), 0, (hipStream_t) s, x, (long long) ldx,
                     (long long) bsx, (long long) tin, cin, wp, bias, cout, st, pad, ntap, y,
                     (long long) ldy, (long long) bsy, (long long) Lout);
  HCHK(hipGetLastError());
  return 0;
}

// ------------------------------------------------------------------------------ matmul
// fp32 MFMA matmul, C[m][n] = A[m][k] . B[k][n], all row-major with leading dimensions lda, ldb,
// ldc (the reference's pt_v21_matmul contract).  A workgroup computes a 64x64 block of C, each of
// its four waves a 32x32 tile, walking k in steps of 8: lane (h, r) feeds A[row r][k0 + 2p + h]
// and B[k0 + 2p + h][column r] to the p-th of four v_mfma_f32_32x32x2_f32 (the operand layout of
// the conv kernel).  Loads outside the matrices read as 0, so any m, n, k works.
__global__ void __launch_bounds__(256) matmul_mfma_kernel(const float *__restrict__ A, long long m,
                                                          long long k, long long lda,
                                                          const float *__restrict__ B,
                                                          long long ldb, long long nn,
                                                          float *__restrict__ C, long long ldc) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int h = lane >> 5, l32 = lane & 31;
  const long long r0 = (long long) blockIdx.y * 64 + (w >> 1) * 32;
  const long long c0 = (long long) blockIdx.x * 64 + (w & 1) * 32;
  const long long ra = r0 + l32, cb = c0 + l32;
  const bool rok = ra < m, cok = cb < nn;
  const float *arow = A + (rok ? ra : 0) * lda;
  f32x16 acc;
#pragma unroll
  for (int v = 0; v < 16; v++) acc[v] = 0.0f;
  for (long long k0 = 0; k0 < k; k0 += 8) {
    float av[4], bv[4];
#pragma unroll
    for (int q = 0; q < 4; q++) {
      const long long kk = k0 + 2 * q + h;
      const bool kok = kk < k;
      av[q] = (rok && kok) ? arow[kk] : 0.0f;
      bv[q] = (cok && kok) ? B[kk * ldb + cb] : 0.0f;
    }
#pragma unroll
    for (int q = 0; q < 4; q++) acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av[q], bv[q], acc, 0, 0, 0);
  }
#pragma unroll
  for (int v = 0; v < 16; v++) {
    const long long row = r0 + 8 * (v >> 2) + 4 * h + (v & 3);
    if (row < m && cok) C[row * ldc + cb] = acc[v];
  }
}
extern "C" int ptk_matmul(const float *A, int64_t m, int64_t k, int64_t lda, const float *B,
                          int64_t ldb, int64_t nn, float *C, int64_t ldc, void *s) {
  if (m <= 0 || nn <= 0) return 0;
  const long long gy = (m + 63) / 64, gx = (nn + 63) / 64;
  if (gy > 65535 || gx > 0x7fffffffLL) {
    set_err("ptk_matmul: %lld x %lld outside the grid limits", (long long) m, (long long) nn);
    return -1;
  }
  hipLaunchKernelGGL(matmul_mfma_kernel, dim3((unsigned) gx, (unsigned) gy), dim3(256), 0,
                     (hipStream_t) s, A, (long long) m, (long long) k, (long long) lda, B,
                     (long long) ldb, (long long) nn, C, (long long) ldc);
  HCHK(hipGetLastError());
  return 0;
}

// ------------------------------------------------------------------------------ elementwise
__global__ void add_kernel(const float *__restrict__ a, const float *__restrict__ b,
                           float *__restrict__ y, long long n, int epi, float alpha) {
  long long i = (long long) blockIdx.x * blockDim.x + threadIdx.x;
  const long long st = (long long) gridDim.x * blockDim.x;
  for (; i < n; i += st) {
    float v = a[i] + b[i];
    if (epi == 1) v = v >= 0.0f ? v : alpha * v;
    y[i] = v;
  }
}
__global__ void leaky_kernel(const float *__restrict__ a, float *__restrict__ y, long long n,
                             float alpha) {
  long long i = (long long) blockIdx.x * blockDim.x + threadIdx.x;
  const long long st = (long long) gridDim.x * blockDim.x;
  for (; i < n; i += st) {
    const float v = a[i];
    y[i] = v >= 0.0f ? v : alpha * v;
  }
}
__global__ void avg3_leaky_kernel(const float *__restrict__ a, const float *__restrict__ b,
                                  const float *__restrict__ c, float *__restrict__ y, long long n,
                                  float alpha) {
  long long i = (long long) blockIdx.x * blockDim.x + threadIdx.x;
  const long long st = (long long) gridDim.x * blockDim.x;
  for (; i < n; i += st) {
    const float v = ((a[i] + b[i]) + c[i]) / 3.0f;
    y[i] = v >= 0.0f ? v : alpha * v;
  }
}
static unsigned ew_blocks(long long n) {
  long long b = (n + 255) / 256;
  if (b > 8192) b = 8192;
  return (unsigned) (b < 1 ? 1 : b);
}

// The same elementwise ops four elements per thread, for 16-byte aligned operands (the decoder's
// arena blocks are 256-byte aligned): each element goes through exactly the scalar kernel's
// operations, the n % 4 tail elements through threads 0 .. n % 4 - 1.
__device__ __forceinline__ float leaky1(float v, float a) { return v >= 0.0f ? v : a * v; }
__global__ void avg3_leaky4_kernel(const float *__restrict__ a, const float *__restrict__ b,
                                   const float *__restrict__ c, float *__restrict__ y, long long n,
                                   float alpha) {
  const long long n4 = n >> 2, i0 = (long long) blockIdx.x * blockDim.x + threadIdx.x;
  const long long st = (long long) gridDim.x * blockDim.x;
  for (long long i = i0; i < n4; i += st) {
    const float4 va = reinterpret_cast<const float4 *>(a)[i], vb = reinterpret_cast<const float4 *>(b)[i],
                 vc = reinterpret_cast<const float4 *>(c)[i];
    reinterpret_cast<float4 *>(y)[i] = make_float4(leaky1(((va.x + vb.x) + vc.x) / 3.0f, alpha),
                                                   leaky1(((va.y + vb.y) + vc.y) / 3.0f, alpha),
                                                   leaky1(((va.z + vb.z) + vc.z) / 3.0f, alpha),
                                                   leaky1(((va.w + vb.w) + vc.w) / 3.0f, alpha));
  }
  if (i0 < (n & 3)) {
    const long long e = (n4 << 2) + i0;
    y[e] = leaky1(((a[e] + b[e]) + c[e]) / 3.0f, alpha);
  }
}
__global__ void add4_kernel(const float *__restrict__ a, const float *__restrict__ b,
                            float *__restrict__ y, long long n, int epi, float alpha) {
  const long long n4 = n >> 2, i0 = (long long) blockIdx.x * blockDim.x + threadIdx.x;
  const long long st = (long long) gridDim.x * blockDim.x;
  for (long long i = i0; i < n4; i += st) {
    const float4 va = reinterpret_cast<const float4 *>(a)[i], vb = reinterpret_cast<const float4 *>(b)[i];
    float4 v = make_float4(va.x + vb.x, va.y + vb.y, va.z + vb.z, va.w + vb.w);
    if (epi == 1) v = make_float4(leaky1(v.x, alpha), leaky1(v.y, alpha), leaky1(v.z, alpha), leaky1(v.w, alpha));
    reinterpret_cast<float4 *>(y)[i] = v;
  }
  if (i0 < (n & 3)) {
    const long long e = (n4 << 2) + i0;
    const float v = a[e] + b[e];
    y[e] = epi == 1 ? leaky1(v, alpha) : v;
  }
}
__global__ void leaky4_kernel(const float *__restrict__ a, float *__restrict__ y, long long n, float alpha) {
  const long long n4 = n >> 2, i0 = (long long) blockIdx.x * blockDim.x + threadIdx.x;
  const long long st = (long long) gridDim.x * blockDim.x;
  for (long long i = i0; i < n4; i += st) {
    const float4 va = reinterpret_cast<const float4 *>(a)[i];
    reinterpret_cast<float4 *>(y)[i] = make_float4(leaky1(va.x, alpha), leaky1(va.y, alpha),
                                                   leaky1(va.z, alpha), leaky1(va.w, alpha));
  }
  if (i0 < (n & 3)) y[(n4 << 2) + i0] = leaky1(a[(n4 << 2) + i0], alpha);
}
static bool al16(const void *p) { return ((uintptr_t) p & 15) == 0; }
extern "C" int ptk_add(const float *a, const float *b, float *y, int64_t n, int epi, float alpha,
                       void *s) {
  if (n <= 0) return 0;
  if (al16(a) && al16(b) && al16(y) && n >= 4)
    hipLaunchKernelGGL(add4_kernel, dim3(ew_blocks(n >> 2)), dim3(256), 0, (hipStream_t) s, a, b, y,
                       (long long) n, epi, alpha);
  else
    hipLaunchKernelGGL(add_kernel, dim3(ew_blocks(n)), dim3(256), 0, (hipStream_t) s, a, b, y,
                       (long long) n, epi, alpha);
  HCHK(hipGetLastError());
  return 0;
}
extern "C" int ptk_avg3_leaky(const float *a, const float *b, const float *c, float *y, int64_t n,
                              float alpha, void *s) {
  if (n <= 0) return 0;
  if (al16(a) && al16(b) && al16(c) && al16(y) && n >= 4)
    hipLaunchKernelGGL(avg3_leaky4_kernel, dim3(ew_blocks(n >> 2)), dim3(256), 0, (hipStream_t) s, a,
                       b, c, y, (long long) n, alpha);
  else
    hipLaunchKernelGGL(avg3_leaky_kernel, dim3(ew_blocks(n)), dim3(256), 0, (hipStream_t) s, a, b,
                       c, y, (long long) n, alpha);
  HCHK(hipGetLastError());
  return 0;
}
extern "C" int ptk_leaky(const float *a, float *y, int64_t n, float alpha, void *s) {
  if (n <= 0) return 0;
  if (al16(a) && al16(y) && n >= 4)
    hipLaunchKernelGGL(leaky4_kernel, dim3(ew_blocks(n >> 2)), dim3(256), 0, (hipStream_t) s, a, y,
                       (long long) n, alpha);
  else
    hipLaunchKernelGGL(leaky_kernel, dim3(ew_blocks(n)), dim3(256), 0, (hipStream_t) s, a, y,
                       (long long) n, alpha);
  HCHK(hipGetLastError());
  return 0;
}

// ------------------------------------------------------------------------------ decoder tail
// conv_post output p [72][L] (channel c = band*18 + k) -> waveform, fused:
//   frame[b][n][t] = hann[n] * sum_k (re Bc[k][n] + im Bs[k][n]),  re/im = exp(p_k) cos/sin(pi sin(p_9+k))
//   ola[b][j] = sum_{j-4t in [0,16)} frame[b][j-4t][t];   y[b][i] = ola[b][i+8] / max(wsum[i+8], 1e-9)
//   wav[o] = sum_b sum_m h[b][m] * 4 * y[b][(o+m-31)/4]   over (o+m-31) = 0 mod 4 in range.
// A tile is TOUT consecutive samples of one item, made by one workgroup of four waves that
// recomputes the frames the tile needs, so the whole tail is a single pass over p with no
// intermediates in HBM.  Its two products run on the fp32 16x16x4 MFMA (lane l holds A[l%16][l/16],
// B[l/16][l%16] and result rows 4(l/16)+i of column l%16):
//   - the irfft: 16 frames x 16 samples per product group, the spectrum as A (k = the lane's bin
//     group: re of bin g, im of bin g (bin 0's k group carries re of bin 8 instead: the imaginary
//     parts of bins 0 and 8 meet sin(0) and sin(pi n), which vanish), re and im of bin g + 4), the
//     basis with hann folded in as B;
//   - the PQMF synthesis: samples o0' + 16m + 4q + r of a 256-sample block are
//     sum_b sum_s y_b[64k + 4m + 1 + s] * 4 h_b[3 - r + 4(s - q)], a Hankel product over the 19
//     shifts s with the four bands as the k of each MFMA.
// Wave w makes band w's frames and y values (phases A and B touch only that wave's LDS, so they
// need no barrier), then the waves make one 256-sample block each from all bands' y (phase C).
// A workgroup loops over tiles (tile, tile + gridDim.x, ...); the next tile's reads are issued as
// soon as the current tile's are used and arrive while phases B and C run.
// An angle p (radians) as revolutions in [-1/2, 1/2] for v_sin_f32 / v_cos_f32, whose input
// domain is |x| <= 256 revolutions and which see only the rounded product p / 2 pi.  Cody and
// Waite's two-constant reduction (W. J. Cody, W. Waite, Software Manual for the Elementary
// Functions, 1980): k = rint(p / 2 pi), r = (p - k C1) - k C2 with C1 = fp32(2 pi) and
// C2 = 2 pi - C1, each step one fused multiply-add, so r carries p's own bits to within a few
// units of its last place for |p| up to ~1e7.  For |p| < pi, k = 0 and r = p: the result is the
// plain p / 2 pi.
__device__ __forceinline__ float rev_of(float p) {
  const float k = __builtin_rintf(p * 0.159154943f);
  float r = __builtin_fmaf(-k, 6.28318548f, p);
  r = __builtin_fmaf(-k, -1.74845553e-7f, r);
  return r * 0.159154943f;
}

template <int TOUT>
struct TailGeo {
  static constexpr int NG = ((TOUT / 4 + 27) / 4 + 16) / 16;   // 16-frame groups per band
  static constexpr int P = 64 * NG + 32;     // one overlap-add plane (floats); a multiple of 32
  static constexpr int SLOTS = TOUT / 4 + 16;  // y slots per band: slot u + 1 + j for u < TOUT/4
  static constexpr int YP = TOUT / 4 + 20;   // a band's y row: slot at +3, read 20 at a time
  static constexpr int NB = TOUT / 256;      // 256-sample output blocks
};

// The launch's walk over the tiles.  Tiles are numbered item-major; workgroup b takes tiles
// base, base + stride, ... below its end, passing over those with no kept sample.  With a
// workgroup per tile: base = b, stride = the grid, end = all tiles.  When workgroups loop (the
// grid a multiple of 8), the tiles are split into 8 contiguous runs, one per XCD (workgroup b runs
// on XCD b % 8), and the XCD's workgroups take its run in order: neighbouring tiles, which read
// the same boundary frames, then share that XCD's L2.  The stride steps (item, bx) by sq items
// and sr tiles, so no division per step.  Each item's kept samples are [lo, hi) (clamped to its
// samples; item 0 and the last item have their own bounds: the windows of a long request).
struct TailWalk {
  int nbx, batch, ntiles, xcd_run;   // xcd_run: tiles per XCD run, 0 = no split
  int stride, sq, sr;
  int lo_first, lo, hi, hi_last;
};

template <int TOUT>
__global__ void __launch_bounds__(256) tail_kernel(const float *__restrict__ p, long long ldp,
                                                   long long bsp, int L, float *__restrict__ wav,
                                                   long long bsw, const float *__restrict__ cst,
                                                   TailWalk tw) {
  using G = TailGeo<TOUT>;
  constexpr int NG = G::NG, P = G::P, SLOTS = G::SLOTS, YP = G::YP, NB = G::NB;
  static_assert(NB >= 1 && NB <= 4 && TOUT % 256 == 0, "one 256-sample block per wave");
  // s_pl[band][jt][jr]: sample n = 4 jt + (jr & 3) of relative frame (jr >> 2) - jt, so
  // ola[jr] = sum_jt s_pl[band][jt][jr]; s_y[band][slot + 3]
  __shared__ __align__(16) float s_pl[4 * 4 * P];
  __shared__ __align__(16) float s_y[4 * YP];
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
  const int lm = lane & 15, lg = lane >> 4;
  const float *hann = cst, *bc = cst + 16, *bs = cst + 160, *hp = cst + 304, *hb = cst + 560;
  const int Ly = 4 * (L - 1);

  // this workgroup's tiles (TailWalk); (item, bx) = divmod(tile, nbx)
  const int b0 = (int) blockIdx.x;
  int tile = tw.xcd_run ? (b0 & 7) * tw.xcd_run + (b0 >> 3) : b0;
  const int tend = tw.xcd_run ? min(((b0 & 7) + 1) * tw.xcd_run, tw.ntiles) : tw.ntiles;
  int item = tile / tw.nbx, bx = tile - item * tw.nbx;
  auto step = [&](int &t, int &it, int &b) {
    t += tw.stride;
    it += tw.sq;
    b += tw.sr;
    if (b >= tw.nbx) {
      b -= tw.nbx;
      it++;
    }
  };
  auto kept_lo = [&](int it) { return it == 0 ? tw.lo_first : tw.lo; };
  auto kept_hi = [&](int it) { return it + 1 == tw.batch ? tw.hi_last : tw.hi; };
  auto to_kept = [&](int &t, int &it, int &b) {
    while (t < tend && !(b * TOUT < kept_hi(it) && b * TOUT + TOUT > kept_lo(it))) step(t, it, b);
  };
  to_kept(tile, item, bx);
  if (tile >= tend) return;

  // reads of one tile: for frame group c of band w, lane (m, g) reads frame t_lo + 16c + m of
  // bins g and g + 4 (magnitude and phase) and, in k group 0, bin 8.  The item's 72 rows are one
  // buffer; a frame outside [0, L) gets an offset past it and reads 0 (the host keeps 72 * ldp
  // floats within 2 GiB); the row steps between the reads are scalar offsets.
  const unsigned nrec = (unsigned) (72 * ldp * 4), ldp4 = (unsigned) (ldp * 4);
  const unsigned ro = (unsigned) (18 * w + lg) * ldp4;
  float ld[NG][6];
  auto issue = [&](int it, int b) {
    const int t_lo = b * (TOUT / 16) - 3;
    const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(
        (void *) (p + (long long) it * bsp), (short) 0, (int) nrec, PTK_BUF_WORD3);
#pragma unroll
    for (int c = 0; c < NG; c++) {
      const int tf = t_lo + 16 * c + lm;
      const bool ok = (unsigned) tf < (unsigned) L;
      const unsigned vo = ok ? ro + (unsigned) tf * 4u : PTK_OOB;
      const unsigned vo8 = ok && lg == 0 ? vo + 8u * ldp4 : PTK_OOB;
      ld[c][0] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, vo, 0, 0));
      ld[c][1] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, vo, 9 * ldp4, 0));
      ld[c][2] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, vo, 4 * ldp4, 0));
      ld[c][3] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, vo, 13 * ldp4, 0));
      ld[c][4] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, vo8, 0, 0));
      ld[c][5] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, vo8, 9 * ldp4, 0));
    }
  };
  issue(item, bx);

  // B operands, the same for every tile: the irfft basis of this lane's k group with hann[n]
  // folded in, and the synthesis taps (gain 4 folded in: an exact power-of-two scaling) of band
  // lg for output n = 4q + r at each shift s
  float ba[4], bf[19];
  {
    const float h = hann[lm];
    ba[0] = h * bc[lg * 16 + lm];
    ba[1] = h * (lg == 0 ? bc[8 * 16 + lm] : bs[lg * 16 + lm]);
    ba[2] = h * bc[(lg + 4) * 16 + lm];
    ba[3] = h * bs[(lg + 4) * 16 + lm];
    const int q = lm >> 2, r = lm & 3;
#pragma unroll
    for (int s = 0; s < 19; s++) {
      const int j = s - q;
      bf[s] = j >= 0 && j < 16 ? 4.0f * hp[(lg * 4 + r) * 16 + j] : 0.0f;
    }
  }
  const float bias = hb[0];
  // phase B: lane slot = lane + 64 it has jr & 3 = lane & 3, so its window-sum terms hann^2 are
  // fixed.  Every y is ola * (1 / max(wsum, 1e-9)), wsum summed over the valid terms in tap
  // order: the interior value is computed once here, by the same operations.
  const float eps = 1e-9f;
  float hh[4];
#pragma unroll
  for (int jt = 0; jt < 4; jt++) {
    const float h = hann[(lane & 3) + 4 * jt];
    hh[jt] = h * h;
  }
  float ws_in = 0.0f;
#pragma unroll
  for (int jt = 0; jt < 4; jt++) ws_in += hh[jt];
  const float inv_in = 1.0f / (ws_in > eps ? ws_in : eps);
  float *const pl = s_pl + w * 4 * P;        // this wave's band
  float *const yw = s_y + w * YP + 3;

  for (bool first = true;; first = false) {
    const int o0 = bx * TOUT;
    const int t_lo = o0 / 16 - 3;             // frame of relative index 0
    const int i_lo = o0 / 4 - 8;              // y index of slot 0
    // every frame and y slot of the tile inside the sequence: no range tests
    const bool inner = t_lo >= 0 && t_lo + 16 * NG <= L && i_lo >= 0 && i_lo + SLOTS <= Ly;
    // A) band w's frames, 16 per group: spectra into A, 4 MFMAs, the 16 x 16 result into the
    //    overlap-add planes (row 4 lg + i of column lm is sample lm of frame 16c + 4lg + i)
#pragma unroll
    for (int c = 0; c < NG; c++) {
      const int tf = t_lo + 16 * c + lm;
      // the hardware transcendentals: v_exp_f32 is 2^x, v_sin_f32 / v_cos_f32 take revolutions
      // (sin(2 pi x)).  The phase pi * sin(p) in revolutions is sin(p) / 2, within [-1/2, 1/2],
      // so the outer cos / sin need no range reduction.  The inner sin(p) does: p is an
      // unbounded conv output (reduced by rev_of below).
      const float m0 = __builtin_amdgcn_exp2f(ld[c][0] * 1.44269504f);
      const float r0 = 0.5f * __builtin_amdgcn_sinf(rev_of(ld[c][1]));
      const float m1 = __builtin_amdgcn_exp2f(ld[c][2] * 1.44269504f);
      const float r1 = 0.5f * __builtin_amdgcn_sinf(rev_of(ld[c][3]));
      const float m8 = __builtin_amdgcn_exp2f(ld[c][4] * 1.44269504f);
      const float r8 = 0.5f * __builtin_amdgcn_sinf(rev_of(ld[c][5]));
      float a0 = m0 * __builtin_amdgcn_cosf(r0);
      float a1 = lg == 0 ? m8 * __builtin_amdgcn_cosf(r8) : m0 * __builtin_amdgcn_sinf(r0);
      float a2 = m1 * __builtin_amdgcn_cosf(r1);
      float a3 = m1 * __builtin_amdgcn_sinf(r1);
      if (!inner && (unsigned) tf >= (unsigned) L) {   // frames outside the sequence are zero
        a0 = 0.0f;
        a1 = 0.0f;
        a2 = 0.0f;
        a3 = 0.0f;
      }
      f32x4 d = {0.0f, 0.0f, 0.0f, 0.0f};
      d = __builtin_amdgcn_mfma_f32_16x16x4f32(a0, ba[0], d, 0, 0, 0);
      d = __builtin_amdgcn_mfma_f32_16x16x4f32(a1, ba[1], d, 0, 0, 0);
      d = __builtin_amdgcn_mfma_f32_16x16x4f32(a2, ba[2], d, 0, 0, 0);
      d = __builtin_amdgcn_mfma_f32_16x16x4f32(a3, ba[3], d, 0, 0, 0);
      float *const dst = pl + (lm >> 2) * P + 64 * c + 16 * lg + lm;
#pragma unroll
      for (int i = 0; i < 4; i++) dst[4 * i] = d[i];
    }
    int ntile = tile, nitem = item, nxb = bx;
    step(ntile, nitem, nxb);
    to_kept(ntile, nitem, nxb);
    const bool more = ntile < tend;
    if (more) issue(nitem, nxb);   // in flight through phases B and C
    // the previous tile's phase C read every band's y
    if (!first) __syncthreads();
    // B) band w's y: overlap-add, window-sum normalisation, [8:-8] trim; 0 outside [0, Ly)
    if (inner) {
#pragma unroll
      for (int it = 0; it < (SLOTS + 63) / 64; it++) {
        const int slot = lane + 64 * it, jr = slot + 12;
        if (slot < SLOTS)
          yw[slot] = (((pl[jr] + pl[P + jr]) + pl[2 * P + jr]) + pl[3 * P + jr]) * inv_in;
      }
    } else {
#pragma unroll
      for (int it = 0; it < (SLOTS + 63) / 64; it++) {
        const int slot = lane + 64 * it;
        if (slot < SLOTS) {
          const int jr = slot + 12, i = i_lo + slot;
          float yv = 0.0f;
          if (i >= 0 && i < Ly) {
            const float ola = ((pl[jr] + pl[P + jr]) + pl[2 * P + jr]) + pl[3 * P + jr];
            const int t0 = t_lo + (jr >> 2);    // frame of tap jt is t0 - jt
            float ws = 0.0f;
#pragma unroll
            for (int jt = 0; jt < 4; jt++) ws += (unsigned) (t0 - jt) < (unsigned) L ? hh[jt] : 0.0f;
            yv = ola * (1.0f / (ws > eps ? ws : eps));
          }
          yw[slot] = yv;
        }
      }
    }
    __syncthreads();
    // C) PQMF synthesis of the 256-sample block w: A = y_lg[64w + 4m + 1 + s] (a lane's 20
    //    consecutive values in five 16-byte reads), B = the taps of shift s; the result row
    //    4lg + i, column lm is sample o0 + 256w + 16(4lg + i) + lm
    if (w < NB) {
      const float4 *ya = reinterpret_cast<const float4 *>(s_y + lg * YP + 64 * w + 4 * lm + 4);
      float a[20];
#pragma unroll
      for (int v = 0; v < 5; v++) {
        const float4 x = ya[v];
        a[4 * v] = x.x; a[4 * v + 1] = x.y; a[4 * v + 2] = x.z; a[4 * v + 3] = x.w;
      }
      f32x4 d = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int s = 0; s < 19; s++) d = __builtin_amdgcn_mfma_f32_16x16x4f32(a[s], bf[s], d, 0, 0, 0);
      // samples outside the item's kept range (which lies inside its samples) get an offset past
      // the buffer: the store is dropped by the range check
      const int lo = kept_lo(item), hi = kept_hi(item);
      const unsigned cnt = hi > lo ? (unsigned) (hi - lo) : 0u;
      const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc(
          (void *) (wav + (long long) item * bsw), (short) 0, (int) 0x7fffffff, PTK_BUF_WORD3);
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int o = o0 + 256 * w + 16 * (4 * lg + i) + lm;
        const unsigned vo = (unsigned) (o - lo) < cnt ? (unsigned) o * 4u : PTK_OOB;
        __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(d[i] + bias), rw, vo, 0, 0);
      }
    }
    if (!more) break;
    tile = ntile;
    item = nitem;
    bx = nxb;
  }
}

template <int TOUT>
static int launch_tail(int batch, const float *p, int64_t ldp, int64_t bsp, int64_t L, float *wav,
                       int64_t bsw, const float *consts, const ptk_emit *em, int grid_knob,
                       hipStream_t s) {
  const int nout = (int) (16 * (L - 1));
  const int nbx = (nout + TOUT - 1) / TOUT;
  const long long ntiles = (long long) nbx * batch;
  if (ntiles > INT_MAX / 2) {
    set_err("ptk_tail: %lld tiles exceed the launch's index range", ntiles);
    return -1;
  }
  // A workgroup per tile while the tiles fit on the chip at once; past that, as many workgroups
  // as are resident, each looping over tiles with the next tile's reads in flight (PTK_TAIL_GRID:
  // -1 = a workgroup per tile, n > 0 = n workgroups).
  static const int resident = [] {
    int ncu = 0, per_cu = 0;
    if (hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, 0) != hipSuccess ||
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, tail_kernel<TOUT>, 256, 0) !=
            hipSuccess)
      return 0;
    return ncu * per_cu;
  }();
  long long grid = grid_knob > 0 ? grid_knob : (grid_knob < 0 || resident <= 0 ? ntiles : resident);
  if (grid > ntiles) grid = ntiles;
  // looping workgroups split the tiles into one contiguous run per XCD (PTK_TAIL_XCD=0: no split)
  const int xcd_run = grid < ntiles && grid % 8 == 0 && knob(KN_TAIL_XCD)
      ? (int) ((ntiles + 7) / 8) : 0;
  const int stride = xcd_run ? (int) (grid / 8) : (int) grid;
  auto clamp = [nout](int64_t v) { return (int) (v < 0 ? 0 : (v > nout ? nout : v)); };
  const TailWalk tw = {nbx, batch, (int) ntiles, xcd_run, stride, stride / nbx, stride % nbx,
                       clamp(em->lo_first), clamp(em->lo), clamp(em->hi), clamp(em->hi_last)};
  hipLaunchKernelGGL((tail_kernel<TOUT>), dim3((unsigned) grid), dim3(256), 0, s, p,
                     (long long) ldp, (long long) bsp, (int) L, wav, (long long) bsw, consts, tw);
  HCHK(hipGetLastError());
  return 0;
}

extern "C" int ptk_tail_batched(const float *p, int64_t ldp, int64_t bsp, int64_t L, float *wav,
                                int64_t bsw, int batch, const float *consts, const ptk_emit *emit,
                                void *s) {
  if (L < 2) {
    set_err("ptk_tail: need at least 2 frames (got %lld)", (long long) L);
    return -1;
  }
  // 32-bit buffer offsets: an item's 72 rows and its waveform within 2 GiB each
  if (ldp < L || 72 * ldp * 4 > INT32_MAX || 16 * (L - 1) * 4 > INT32_MAX) {
    set_err("ptk_tail: %lld frames (row stride %lld) past the kernel's 32-bit offsets",
            (long long) L, (long long) ldp);
    return -1;
  }
  if (batch <= 0) return 0;
  const long long nout = 16 * (L - 1);
  const ptk_emit all = {0, 0, nout, nout};
  const ptk_emit em = emit ? *emit : all;
  // Tile size: PTK_TAIL_OUT=256 / 512 / 1024 forces one.
  const int oknob = knob(KN_TAIL_OUT), gknob = knob(KN_TAIL_GRID);
  const long long t1k = (nout + 1023) / 1024 * batch, t512 = (nout + 511) / 512 * batch;
  hipStream_t st = (hipStream_t) s;
  const int tout = oknob == 256 || oknob == 512 || oknob == 1024
      ? oknob : (t1k >= 256 ? 1024 : (t512 >= 256 ? 512 : 256));
  if (tout == 1024)
    return launch_tail<1024>(batch, p, ldp, bsp, L, wav, bsw, consts, &em, gknob, st);
  if (tout == 512)
    return launch_tail<512>(batch, p, ldp, bsp, L, wav, bsw, consts, &em, gknob, st);
  return launch_tail<256>(batch, p, ldp, bsp, L, wav, bsw, consts, &em, gknob, st);
}
extern "C" int ptk_tail(const float *p, int64_t ldp, int64_t L, float *wav, const float *consts,
                        void *s) {
  return ptk_tail_batched(p, ldp, 0, L, wav, 0, 1, consts, NULL, s);
}

// ------------------------------------------------------------------------------ MFMA layout probe
__global__ void mfma_probe_kernel(const float *a, const float *b, float *d) {
  const int lane = threadIdx.x;
  f32x16 acc;
  for (int v = 0; v < 16; v++) acc[v] = 0.0f;
  acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a[(lane & 31) * 2 + (lane >> 5)],
                                             b[(lane >> 5) * 32 + (lane & 31)], acc, 0, 0, 0);
  for (int v = 0; v < 16; v++) {
    const int i = 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3), j = lane & 31;
    d[i * 32 + j] = acc[v];
  }
}
extern "C" int ptk_mfma_probe(const float *a, const float *b, float *d, void *s) {
  hipLaunchKernelGGL(mfma_probe_kernel, dim3(1), dim3(64), 0, (hipStream_t) s, a, b, d);
  HCHK(hipGetLastError());
  return 0;
}

// 16x16x4: lane l holds A[l % 16][l / 16] and B[l / 16][l % 16]; value r of its result is
// D[4*(l / 16) + r][l % 16], the layout the 16-row conv tiles assume
__global__ void mfma16_probe_kernel(const float *a, const float *b, float *d) {
  const int lane = threadIdx.x;
  f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
  acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[(lane & 15) * 4 + (lane >> 4)],
                                             b[(lane >> 4) * 16 + (lane & 15)], acc, 0, 0, 0);
  for (int r = 0; r < 4; r++) d[(4 * (lane >> 4) + r) * 16 + (lane & 15)] = acc[r];
}
extern "C" int ptk_mfma16_probe(const float *a, const float *b, float *d, void *s) {
  hipLaunchKernelGGL(mfma16_probe_kernel, dim3(1), dim3(64), 0, (hipStream_t) s, a, b, d);
  HCHK(hipGetLastError());
  return 0;
}
