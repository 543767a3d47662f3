// runtime.hip -- libmlxq runtime: init, errors, device memory, streams,
// events and the per-device workspace.
//
// Mirrors the contract the reference's FFI layer relies on
// (src/mlx/ffi.ts:3-11, :277-348): int status per call, an error message
// recorded on the calling thread, raw handles passed as u64.
#include <mutex>
#include <string>
#include <vector>

#include "mlxq_internal.h"

namespace mlxq {

static thread_local std::string g_last_error;
static std::mutex g_mu;
static int g_device = -1;
static hipStream_t g_stream = nullptr;
static int g_cu_count = 0;

// Per-device workspace: the live block and the blocks it replaced that a
// captured graph may still reference.
struct DeviceWorkspace {
  void* ptr = nullptr;
  size_t bytes = 0;
  std::vector<void*> retired;
};
static std::vector<DeviceWorkspace> g_ws;  // indexed by device
static int g_live_graphs = 0;              // graph execs made by mlxq_graph_end, not yet destroyed

// The fixed scratch block of the no-allocation entry points: a file-scope
// device array, so every GPU the library runs on holds its own copy for the
// life of the process.  In host code `scratch` names a host-side stand-in,
// not device memory: its per-device address comes from hipGetSymbolAddress
// at mlxq_init (g_scratch_ptr), and only that address reaches kernels.
static __device__ __align__(256) uint8_t scratch[MLXQ_NOALLOC_SCRATCH_BYTES];
static std::vector<void*> g_scratch_ptr;  // indexed by device

void set_error(const std::string& msg) { g_last_error = msg; }

int fail(int code, const std::string& msg) {
  set_error(msg);
  return code;
}

int hip_fail(hipError_t e, const char* what) {
  set_error(std::string(what) + ": " + hipGetErrorName(e) + " (" + hipGetErrorString(e) + ")");
  return MLXQ_ERR_HIP;
}

bool initialised() { return g_device >= 0; }

hipStream_t resolve_stream(void* s) { return s ? (hipStream_t)s : g_stream; }

int device_cu_count() { return g_cu_count; }

// Grows the current device's block to at least `bytes` (caller holds g_mu).
static int grow_locked(size_t bytes, hipStream_t stream) {
  int dev = 0;
  MLXQ_HIP(hipGetDevice(&dev));
  if ((int)g_ws.size() <= dev) g_ws.resize(dev + 1);
  DeviceWorkspace& w = g_ws[dev];
  if (w.bytes >= bytes) return MLXQ_OK;
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  MLXQ_HIP(hipStreamIsCapturing(stream, &cs));
  if (cs != hipStreamCaptureStatusNone)
    return fail(MLXQ_ERR_STATE, "the library workspace must grow to " + std::to_string(bytes) +
                                    " bytes while the stream is being captured: run the call once, or "
                                    "mlxq_workspace_reserve, before capture");
  size_t nb = bytes < ((size_t)1 << 20) ? ((size_t)1 << 20) : bytes;
  nb = (nb + 4095) & ~(size_t)4095;
  void* p = nullptr;
  MLXQ_HIP(hipMalloc(&p, nb));
  if (w.ptr) {
    if (g_live_graphs > 0) {
      w.retired.push_back(w.ptr);  // a replay may still read or write it
    } else {
      MLXQ_HIP(hipStreamSynchronize(stream));
      MLXQ_HIP(hipFree(w.ptr));
    }
  }
  w.ptr = p;
  w.bytes = nb;
  return MLXQ_OK;
}

int workspace(size_t bytes, void** out, hipStream_t stream) {
  std::lock_guard<std::mutex> lk(g_mu);
  int rc = grow_locked(bytes, stream);
  if (rc) return rc;
  int dev = 0;
  MLXQ_HIP(hipGetDevice(&dev));
  *out = g_ws[dev].ptr;
  return MLXQ_OK;
}

int noalloc_scratch(Scratch* out) {
  int dev = 0;
  MLXQ_HIP(hipGetDevice(&dev));
  std::lock_guard<std::mutex> lk(g_mu);
  if (dev >= (int)g_scratch_ptr.size() || !g_scratch_ptr[dev])
    return fail(MLXQ_ERR_STATE, "mlxq_init was not called for the current device");
  out->fixed = g_scratch_ptr[dev];
  out->fixed_bytes = MLXQ_NOALLOC_SCRATCH_BYTES;
  return MLXQ_OK;
}

int Scratch::get(size_t bytes, void** out, hipStream_t stream) const {
  if (!fixed) return workspace(bytes, out, stream);
  if (bytes > fixed_bytes)
    return fail(MLXQ_ERR_UNSUPPORTED, "this call needs " + std::to_string(bytes) + " bytes of scratch, more than the " +
                                          std::to_string(fixed_bytes) + "-byte fixed block");
  *out = fixed;
  return MLXQ_OK;
}

// Frees every retired block once no graph exec can reference one.
static int release_retired_locked() {
  if (g_live_graphs > 0) return MLXQ_OK;
  for (DeviceWorkspace& w : g_ws) {
    for (void* p : w.retired) MLXQ_HIP(hipFree(p));
    w.retired.clear();
  }
  return MLXQ_OK;
}

}  // namespace mlxq

using namespace mlxq;

__global__ void mlxq_fill_zero_kernel(uint4* __restrict__ dst16, uint64_t n16, uint8_t* __restrict__ tail,
                                      uint64_t ntail) {
  uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  for (uint64_t j = i; j < n16; j += stride) dst16[j] = make_uint4(0, 0, 0, 0);
  if (i < ntail) tail[i] = 0;
}

extern "C" {

int mlxq_init(int device) {
  int n = 0;
  MLXQ_HIP(hipGetDeviceCount(&n));
  if (device < 0 || device >= n) return fail(MLXQ_ERR_ARGUMENT, "mlxq_init: device index out of range");
  MLXQ_HIP(hipSetDevice(device));
  hipDeviceProp_t prop;
  MLXQ_HIP(hipGetDeviceProperties(&prop, device));
  std::string arch = prop.gcnArchName;
  if (arch.rfind("gfx950", 0) != 0)
    return fail(MLXQ_ERR_UNSUPPORTED, "libmlxq is built for gfx950 only; device is " + arch);
  std::lock_guard<std::mutex> lk(g_mu);
  if (!g_stream) MLXQ_HIP(hipStreamCreateWithFlags(&g_stream, hipStreamNonBlocking));
  if ((int)g_scratch_ptr.size() <= device) g_scratch_ptr.resize(device + 1, nullptr);
  if (!g_scratch_ptr[device]) {  // this device's copy of the fixed scratch block
    void* p = nullptr;
    MLXQ_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    g_scratch_ptr[device] = p;
  }
  g_cu_count = prop.multiProcessorCount;
  g_device = device;
  return MLXQ_OK;
}

int mlxq_abi_version(void) { return MLXQ_ABI_VERSION; }

const char* mlxq_last_error(void) { return g_last_error.c_str(); }

const char* mlxq_target_arch(void) { return "gfx950"; }

int mlxq_device_count(int* count) {
  if (!count) return fail(MLXQ_ERR_ARGUMENT, "null out-pointer");
  MLXQ_HIP(hipGetDeviceCount(count));
  return MLXQ_OK;
}

int mlxq_malloc(void** ptr, uint64_t nbytes) {
  MLXQ_REQUIRE_INIT();
  if (!ptr) return fail(MLXQ_ERR_ARGUMENT, "null out-pointer");
  *ptr = nullptr;
  if (nbytes == 0) nbytes = 256;  // distinct, freeable pointer for empty arrays
  MLXQ_HIP(hipMalloc(ptr, nbytes));
  return MLXQ_OK;
}

int mlxq_free(void* ptr) {
  MLXQ_REQUIRE_INIT();
  if (ptr) MLXQ_HIP(hipFree(ptr));
  return MLXQ_OK;
}

int mlxq_memcpy_htod(void* dst, const void* src, uint64_t nbytes, void* stream) {
  MLXQ_REQUIRE_INIT();
  if (!nbytes) return MLXQ_OK;
  hipStream_t s = resolve_stream(stream);
  MLXQ_HIP(hipMemcpyAsync(dst, src, nbytes, hipMemcpyHostToDevice, s));
  MLXQ_HIP(hipStreamSynchronize(s));  // src is pageable host memory owned by the caller
  return MLXQ_OK;
}

int mlxq_memcpy_dtoh(void* dst, const void* src, uint64_t nbytes, void* stream) {
  MLXQ_REQUIRE_INIT();
  if (!nbytes) return MLXQ_OK;
  hipStream_t s = resolve_stream(stream);
  MLXQ_HIP(hipMemcpyAsync(dst, src, nbytes, hipMemcpyDeviceToHost, s));
  MLXQ_HIP(hipStreamSynchronize(s));
  return MLXQ_OK;
}

int mlxq_memcpy_dtod(void* dst, const void* src, uint64_t nbytes, void* stream) {
  MLXQ_REQUIRE_INIT();
  if (!nbytes) return MLXQ_OK;
  MLXQ_HIP(hipMemcpyAsync(dst, src, nbytes, hipMemcpyDeviceToDevice, resolve_stream(stream)));
  return MLXQ_OK;
}

int mlxq_fill_zero(void* dst, uint64_t nbytes, void* stream) {
  MLXQ_REQUIRE_INIT();
  if (!nbytes) return MLXQ_OK;
  if ((uintptr_t)dst % 16) return fail(MLXQ_ERR_ARGUMENT, "mlxq_fill_zero: dst must be 16-byte aligned");
  uint64_t n16 = nbytes / 16, ntail = nbytes % 16;
  uint64_t blocks = (n16 + 255) / 256;
  if (blocks < 1) blocks = 1;
  if (blocks > 8192) blocks = 8192;
  hipLaunchKernelGGL(mlxq_fill_zero_kernel, dim3((unsigned)blocks), dim3(256), 0, resolve_stream(stream),
                     (uint4*)dst, n16, (uint8_t*)dst + n16 * 16, ntail);
  MLXQ_LAUNCHED("mlxq_fill_zero_kernel");
  return MLXQ_OK;
}

int mlxq_copy_2d(void* dst, uint64_t dst_pitch, const void* src, uint64_t src_pitch, uint64_t row_bytes,
                 uint64_t rows, void* stream) {
  MLXQ_REQUIRE_INIT();
  if (!rows || !row_bytes) return MLXQ_OK;
  if (row_bytes > dst_pitch || row_bytes > src_pitch)
    return fail(MLXQ_ERR_ARGUMENT, "mlxq_copy_2d: row_bytes exceeds a pitch");
  MLXQ_HIP(hipMemcpy2DAsync(dst, dst_pitch, src, src_pitch, row_bytes, rows, hipMemcpyDeviceToDevice,
                            resolve_stream(stream)));
  return MLXQ_OK;
}

int mlxq_stream_create(void** stream) {
  MLXQ_REQUIRE_INIT();
  if (!stream) return fail(MLXQ_ERR_ARGUMENT, "null out-pointer");
  hipStream_t s;
  MLXQ_HIP(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
  *stream = s;
  return MLXQ_OK;
}

int mlxq_stream_destroy(void* stream) {
  MLXQ_REQUIRE_INIT();
  if (stream) MLXQ_HIP(hipStreamDestroy((hipStream_t)stream));
  return MLXQ_OK;
}

int mlxq_synchronize(void* stream) {
  MLXQ_REQUIRE_INIT();
  MLXQ_HIP(hipStreamSynchronize(resolve_stream(stream)));
  return MLXQ_OK;
}

int mlxq_event_create(void** event) {
  MLXQ_REQUIRE_INIT();
  if (!event) return fail(MLXQ_ERR_ARGUMENT, "null out-pointer");
  hipEvent_t e;
  MLXQ_HIP(hipEventCreate(&e));
  *event = e;
  return MLXQ_OK;
}

int mlxq_event_destroy(void* event) {
  MLXQ_REQUIRE_INIT();
  if (event) MLXQ_HIP(hipEventDestroy((hipEvent_t)event));
  return MLXQ_OK;
}

int mlxq_event_record(void* event, void* stream) {
  MLXQ_REQUIRE_INIT();
  MLXQ_HIP(hipEventRecord((hipEvent_t)event, resolve_stream(stream)));
  return MLXQ_OK;
}

int mlxq_graph_begin(void* stream) {
  MLXQ_REQUIRE_INIT();
  MLXQ_HIP(hipStreamBeginCapture(resolve_stream(stream), hipStreamCaptureModeRelaxed));
  return MLXQ_OK;
}

int mlxq_graph_end(void* stream, void** graph_exec) {
  MLXQ_REQUIRE_INIT();
  if (!graph_exec) return fail(MLXQ_ERR_ARGUMENT, "null out-pointer");
  hipGraph_t g = nullptr;
  MLXQ_HIP(hipStreamEndCapture(resolve_stream(stream), &g));
  hipGraphExec_t ge = nullptr;
  hipError_t e = hipGraphInstantiate(&ge, g, nullptr, nullptr, 0);
  (void)hipGraphDestroy(g);
  if (e != hipSuccess) return hip_fail(e, "hipGraphInstantiate");
  *graph_exec = ge;
  std::lock_guard<std::mutex> lk(g_mu);
  ++g_live_graphs;
  return MLXQ_OK;
}

int mlxq_graph_launch(void* graph_exec, void* stream) {
  MLXQ_REQUIRE_INIT();
  MLXQ_HIP(hipGraphLaunch((hipGraphExec_t)graph_exec, resolve_stream(stream)));
  return MLXQ_OK;
}

int mlxq_graph_destroy(void* graph_exec) {
  MLXQ_REQUIRE_INIT();
  if (!graph_exec) return MLXQ_OK;
  MLXQ_HIP(hipGraphExecDestroy((hipGraphExec_t)graph_exec));
  std::lock_guard<std::mutex> lk(g_mu);
  if (g_live_graphs > 0) --g_live_graphs;
  return release_retired_locked();
}

int mlxq_workspace_reserve(uint64_t nbytes, void* stream) {
  MLXQ_REQUIRE_INIT();
  std::lock_guard<std::mutex> lk(g_mu);
  return grow_locked((size_t)nbytes, resolve_stream(stream));
}

int mlxq_workspace_size(uint64_t* nbytes) {
  MLXQ_REQUIRE_INIT();
  if (!nbytes) return fail(MLXQ_ERR_ARGUMENT, "null out-pointer");
  int dev = 0;
  MLXQ_HIP(hipGetDevice(&dev));
  std::lock_guard<std::mutex> lk(g_mu);
  *nbytes = dev < (int)g_ws.size() ? g_ws[dev].bytes : 0;
  return MLXQ_OK;
}

int mlxq_event_elapsed_ms(void* start, void* stop, float* ms) {
  MLXQ_REQUIRE_INIT();
  if (!ms) return fail(MLXQ_ERR_ARGUMENT, "null out-pointer");
  MLXQ_HIP(hipEventSynchronize((hipEvent_t)stop));
  MLXQ_HIP(hipEventElapsedTime(ms, (hipEvent_t)start, (hipEvent_t)stop));
  return MLXQ_OK;
}

}  // extern "C"
