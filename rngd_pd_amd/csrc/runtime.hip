// Library state, staging memory, streams, events, same-GPU IPC, the greedy
// argmax kernel and a plain copy kernel (traffic-counter calibration).

#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include "pdk_common.h"

namespace pdk {

// Device-visible alias of [host, host + bytes) when the whole range is pinned
// host memory (hipHostMalloc), else null. A failed lookup leaves an error in
// the runtime's last-error slot, which is cleared here.
static void* pinned_alias(void* host, size_t bytes) {
  hipPointerAttribute_t a0{}, a1{};
  char* last = static_cast<char*>(host) + bytes - 1;
  const bool ok = hipPointerGetAttributes(&a0, host) == hipSuccess &&
                  hipPointerGetAttributes(&a1, last) == hipSuccess;
  (void)hipGetLastError();
  // Both ends pinned, and mapped contiguously (one allocation).
  if (!ok || a0.type != hipMemoryTypeHost || a1.type != hipMemoryTypeHost || !a0.devicePointer ||
      static_cast<char*>(a1.devicePointer) != static_cast<char*>(a0.devicePointer) + (bytes - 1))
    return nullptr;
  return a0.devicePointer;
}

int copy_host_device(void* host, void* dev, size_t bytes, bool to_host, hipStream_t st) {
  if (bytes == 0) return PDK_OK;
  // Pinned memory is device-visible: copy on the DMA engines (the "no compute
  // unit" kind), so the transfer takes nothing from kernels on other streams.
  // Through the host kinds some runtimes copy with a blit kernel, which waits
  // for CUs whenever a large kernel (a prefill GEMM) fills the chip.
  if (void* alias = pinned_alias(host, bytes)) {
    PDK_TRY_HIP(hipMemcpyAsync(to_host ? alias : dev, to_host ? dev : alias, bytes,
                               hipMemcpyDeviceToDeviceNoCU, st));
  } else {
    PDK_TRY_HIP(hipMemcpyAsync(to_host ? host : dev, to_host ? dev : host, bytes,
                               to_host ? hipMemcpyDeviceToHost : hipMemcpyHostToDevice, st));
  }
  return PDK_OK;
}


static thread_local char g_err[512] = {0};

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}

void clear_error() { g_err[0] = 0; }

int hip_fail(hipError_t e, const char* what) {
  set_error("%s: %s (%d)", what, hipGetErrorString(e), (int)e);
  return PDK_EHIP;
}

int check_launch(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return hip_fail(e, what);
  return PDK_OK;
}

}  // namespace pdk

namespace {

using pdk::v8;

// First-maximum argmax of one bf16 row; NaN ranks above every number (the
// torch.argmax convention greedy_tokens relies on).
struct Best {
  float v;
  int i;
  int nan;
};

__device__ __forceinline__ bool better(const Best& x, const Best& y) {
  if (x.nan != y.nan) return x.nan > y.nan;
  if (!x.nan && x.v != y.v) return x.v > y.v;
  return x.i < y.i;
}

// One workgroup of 1024 threads per row. kVec: the row is 16-byte aligned
// and V % 8 == 0, read as 8 values per load; otherwise one value per load.
// `better` is a total order (value, then NaN rank, then lower index), so the
// order in which threads visit elements does not matter.
constexpr int kArgThreads = 1024;

__device__ __forceinline__ void consider(Best& best, float x, int i) {
  const Best c{x, i, x != x ? 1 : 0};
  if (better(c, best)) best = c;
}

template <bool kVec>
__global__ __launch_bounds__(kArgThreads) void argmax_kernel(const uint16_t* logits, int V,
                                                             int64_t ld, int32_t* out) {
  __shared__ Best red[kArgThreads / 64];
  const uint16_t* row = logits + (int64_t)blockIdx.x * ld;
  Best best{-INFINITY, 0x7fffffff, 0};
  if (kVec) {
    const int n8 = V >> 3;
#pragma unroll 4
    for (int c = threadIdx.x; c < n8; c += kArgThreads) {
      const v8 v = pdk::ld16(row + 8 * c);
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        consider(best, pdk::bf16_to_f32(v.w[k] & 0xffffu), 8 * c + 2 * k);
        consider(best, pdk::bf16_to_f32(v.w[k] >> 16), 8 * c + 2 * k + 1);
      }
    }
  } else {
    for (int i = threadIdx.x; i < V; i += kArgThreads) consider(best, pdk::bf16_to_f32(row[i]), i);
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    const Best c{__shfl_xor(best.v, o), __shfl_xor(best.i, o), __shfl_xor(best.nan, o)};
    if (better(c, best)) best = c;
  }
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = best;
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int q = 1; q < kArgThreads / 64; ++q)
      if (better(red[q], best)) best = red[q];
    out[blockIdx.x] = best.i;
  }
}

__global__ __launch_bounds__(256) void copy_kernel(uint4* dst, const uint4* src, int64_t n) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
    dst[i] = src[i];
}

// Streaming probes: a linear read, a linear write and a copy of 16-byte
// vectors, four independent vectors in flight per lane (grid-stride), with
// ordinary or non-temporal accesses. The read folds what it loads into an XOR
// and stores a word only where a fold equals `key`, so its loads cannot be
// dropped while in practice it writes nothing.
typedef uint32_t su4 __attribute__((ext_vector_type(4)));

template <bool kNT>
__device__ __forceinline__ su4 probe_ld(const su4* p) {
  if (kNT) return __builtin_nontemporal_load(p);
  return *p;
}

template <bool kNT>
__device__ __forceinline__ void probe_st(su4* p, su4 v) {
  if (kNT) __builtin_nontemporal_store(v, p);
  else *p = v;
}

template <int kKind, bool kNT>
__global__ __launch_bounds__(256) void stream_probe_kernel(su4* dst, const su4* src, int64_t n,
                                                           uint32_t key, uint32_t* sink) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  su4 acc = {0u, 0u, 0u, 0u};
  const su4 fill = {key, key, key, key};
  for (; i + 3 * stride < n; i += 4 * stride) {
    if (kKind == PDK_STREAM_WRITE) {
#pragma unroll
      for (int u = 0; u < 4; ++u) probe_st<kNT>(dst + i + u * stride, fill);
    } else {
      su4 v[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) v[u] = probe_ld<kNT>(src + i + u * stride);
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        if (kKind == PDK_STREAM_COPY) probe_st<kNT>(dst + i + u * stride, v[u]);
        else acc ^= v[u];
      }
    }
  }
  for (; i < n; i += stride) {
    if (kKind == PDK_STREAM_WRITE) probe_st<kNT>(dst + i, fill);
    else if (kKind == PDK_STREAM_COPY) probe_st<kNT>(dst + i, probe_ld<kNT>(src + i));
    else acc ^= probe_ld<kNT>(src + i);
  }
  if (kKind == PDK_STREAM_READ && (acc.x ^ acc.y ^ acc.z ^ acc.w) == key)
    sink[blockIdx.x & 255] = key;
}

// One 16-byte vector per lane, one workgroup per 4 KiB, no loop: every
// workgroup is short-lived, and the dispatcher keeps all CUs fed with fresh
// ones. On MI355X this shape reads and writes HBM faster than any grid-stride
// loop at 4 GiB (about 6.8 TB/s each way against 6.5 / 5.0 TB/s).
template <int kKind, bool kNT>
__global__ __launch_bounds__(256) void stream_once_kernel(su4* dst, const su4* src, int64_t n,
                                                          uint32_t key, uint32_t* sink) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  const su4 fill = {key, key, key, key};
  if (kKind == PDK_STREAM_WRITE) {
    probe_st<kNT>(dst + i, fill);
  } else {
    const su4 v = probe_ld<kNT>(src + i);
    if (kKind == PDK_STREAM_COPY) probe_st<kNT>(dst + i, v);
    else if ((v.x ^ v.y ^ v.z ^ v.w) == key) sink[blockIdx.x & 255] = key;
  }
}

}  // namespace

extern "C" {

int pdk_version(void) { return 100; }

const char* pdk_last_error(void) { return pdk::g_err; }

int pdk_device_count(int* out) {
  pdk::clear_error();
  PDK_REQUIRE(out != nullptr, "out is null");
  PDK_TRY_HIP(hipGetDeviceCount(out));
  return PDK_OK;
}

int pdk_set_device(int device) {
  pdk::clear_error();
  PDK_TRY_HIP(hipSetDevice(device));
  return PDK_OK;
}

int pdk_greedy_argmax(const uint16_t* logits, int B, int V, int64_t ld, int32_t* out,
                      uintptr_t stream) {
  pdk::clear_error();
  PDK_REQUIRE(logits && out, "null pointer argument");
  PDK_REQUIRE(B >= 1 && V >= 1 && ld >= V, "bad shape B=%d V=%d ld=%lld", B, V, (long long)ld);
  const bool vec = pdk::aligned16(logits) && ld % 8 == 0 && V % 8 == 0;
  if (vec)
    hipLaunchKernelGGL(argmax_kernel<true>, dim3(B), dim3(kArgThreads), 0, pdk::as_stream(stream),
                       logits, V, ld, out);
  else
    hipLaunchKernelGGL(argmax_kernel<false>, dim3(B), dim3(kArgThreads), 0, pdk::as_stream(stream),
                       logits, V, ld, out);
  return pdk::check_launch("argmax_kernel");
}

int pdk_host_alloc(size_t bytes, void** out) {
  pdk::clear_error();
  PDK_REQUIRE(out != nullptr && bytes > 0, "bad arguments");
  *out = nullptr;
  const hipError_t e = hipHostMalloc(out, bytes, hipHostMallocDefault);
  if (e != hipSuccess) {
    pdk::hip_fail(e, "hipHostMalloc");
    return PDK_ENOMEM;
  }
  return PDK_OK;
}

int pdk_host_free(void* p) {
  pdk::clear_error();
  if (!p) return PDK_OK;
  PDK_TRY_HIP(hipHostFree(p));
  return PDK_OK;
}

int pdk_dev_alloc(size_t bytes, void** out) {
  pdk::clear_error();
  PDK_REQUIRE(out != nullptr && bytes > 0, "bad arguments");
  *out = nullptr;
  const hipError_t e = hipMalloc(out, bytes);
  if (e != hipSuccess) {
    pdk::hip_fail(e, "hipMalloc");
    return PDK_ENOMEM;
  }
  return PDK_OK;
}

int pdk_dev_free(void* p) {
  pdk::clear_error();
  if (!p) return PDK_OK;
  PDK_TRY_HIP(hipFree(p));
  return PDK_OK;
}

int pdk_memcpy_d2h(void* host_dst, const void* dev_src, size_t bytes, uintptr_t stream) {
  pdk::clear_error();
  PDK_REQUIRE(host_dst && dev_src, "null pointer argument");
  return pdk::copy_host_device(host_dst, const_cast<void*>(dev_src), bytes, true,
                               pdk::as_stream(stream));
}

int pdk_memcpy_h2d(void* dev_dst, const void* host_src, size_t bytes, uintptr_t stream) {
  pdk::clear_error();
  PDK_REQUIRE(dev_dst && host_src, "null pointer argument");
  return pdk::copy_host_device(const_cast<void*>(host_src), dev_dst, bytes, false,
                               pdk::as_stream(stream));
}

int pdk_memcpy_d2d(void* dev_dst, const void* dev_src, size_t bytes, uintptr_t stream) {
  pdk::clear_error();
  PDK_REQUIRE(dev_dst && dev_src, "null pointer argument");
  PDK_TRY_HIP(hipMemcpyAsync(dev_dst, dev_src, bytes, hipMemcpyDeviceToDevice,
                             pdk::as_stream(stream)));
  return PDK_OK;
}

int pdk_copy_kernel(void* dev_dst, const void* dev_src, size_t bytes, uintptr_t stream) {
  pdk::clear_error();
  PDK_REQUIRE(dev_dst && dev_src, "null pointer argument");
  PDK_REQUIRE(bytes % 16 == 0 && pdk::aligned16(dev_dst) && pdk::aligned16(dev_src),
              "copy needs 16-byte aligned pointers and a multiple of 16 bytes");
  const int64_t n = (int64_t)(bytes / 16);
  if (n == 0) return PDK_OK;
  int64_t blocks = (n + 255) / 256;
  if (blocks > 8192) blocks = 8192;
  hipLaunchKernelGGL(copy_kernel, dim3((unsigned)blocks), dim3(256), 0, pdk::as_stream(stream),
                     static_cast<uint4*>(dev_dst), static_cast<const uint4*>(dev_src), n);
  return pdk::check_launch("copy_kernel");
}

int pdk_stream_probe(int kind, void* dev_dst, const void* dev_src, size_t bytes, int flags,
                     int blocks, uint32_t key, uint32_t* dev_sink, uintptr_t stream) {
  pdk::clear_error();
  PDK_REQUIRE(kind == PDK_STREAM_READ || kind == PDK_STREAM_WRITE || kind == PDK_STREAM_COPY,
              "bad kind %d", kind);
  PDK_REQUIRE((flags & ~PDK_STREAM_NONTEMPORAL) == 0, "unknown flags 0x%x", flags);
  PDK_REQUIRE(blocks >= 0 && blocks <= (1 << 20), "blocks must be in [0, 2^20] (got %d)", blocks);
  const bool reads = kind != PDK_STREAM_WRITE, writes = kind != PDK_STREAM_READ;
  PDK_REQUIRE(!reads || (dev_src && pdk::aligned16(dev_src)), "src null or not 16-byte aligned");
  PDK_REQUIRE(!writes || (dev_dst && pdk::aligned16(dev_dst)), "dst null or not 16-byte aligned");
  PDK_REQUIRE(kind != PDK_STREAM_READ || dev_sink, "a read needs a 256-word sink");
  PDK_REQUIRE(bytes % 16 == 0, "bytes must be a multiple of 16");
  const int64_t n = (int64_t)(bytes / 16);
  if (n == 0) return PDK_OK;
  PDK_REQUIRE(blocks > 0 || n <= (1ll << 31), "a one-shot probe moves at most 32 GiB");
  const bool once = blocks == 0;
  const dim3 grid((unsigned)(once ? (n + 255) / 256 : blocks));
  su4* d = static_cast<su4*>(dev_dst);
  const su4* s = static_cast<const su4*>(dev_src);
  hipStream_t st = pdk::as_stream(stream);
  const bool nt = (flags & PDK_STREAM_NONTEMPORAL) != 0;
#define PDK_PROBE_NT(K, NT)                                                                 \
  if (once) hipLaunchKernelGGL((stream_once_kernel<K, NT>), grid, dim3(256), 0, st, d, s, n, key, dev_sink); \
  else hipLaunchKernelGGL((stream_probe_kernel<K, NT>), grid, dim3(256), 0, st, d, s, n, key, dev_sink)
#define PDK_PROBE(K)                                                                        \
  if (nt) { PDK_PROBE_NT(K, true); } else { PDK_PROBE_NT(K, false); }
  if (kind == PDK_STREAM_READ) {
    PDK_PROBE(PDK_STREAM_READ);
  } else if (kind == PDK_STREAM_WRITE) {
    PDK_PROBE(PDK_STREAM_WRITE);
  } else {
    PDK_PROBE(PDK_STREAM_COPY);
  }
#undef PDK_PROBE
#undef PDK_PROBE_NT
  return pdk::check_launch("stream_probe_kernel");
}

int pdk_stream_create(uintptr_t* out) {
  pdk::clear_error();
  PDK_REQUIRE(out != nullptr, "out is null");
  hipStream_t s = nullptr;
  PDK_TRY_HIP(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
  *out = reinterpret_cast<uintptr_t>(s);
  return PDK_OK;
}

int pdk_stream_destroy(uintptr_t stream) {
  pdk::clear_error();
  if (!stream) return PDK_OK;
  PDK_TRY_HIP(hipStreamDestroy(pdk::as_stream(stream)));
  return PDK_OK;
}

int pdk_stream_sync(uintptr_t stream) {
  pdk::clear_error();
  PDK_TRY_HIP(hipStreamSynchronize(pdk::as_stream(stream)));
  return PDK_OK;
}

int pdk_event_create(uintptr_t* out, int flags) {
  pdk::clear_error();
  PDK_REQUIRE(out != nullptr, "out is null");
  PDK_REQUIRE(flags == PDK_EVENT_TIMING || flags == PDK_EVENT_INTERPROCESS ||
                  flags == PDK_EVENT_SYNC,
              "bad flags %d", flags);
  hipEvent_t e = nullptr;
  if (flags == PDK_EVENT_INTERPROCESS) {
    PDK_TRY_HIP(hipEventCreateWithFlags(&e, hipEventInterprocess | hipEventDisableTiming));
  } else if (flags == PDK_EVENT_SYNC) {
    PDK_TRY_HIP(hipEventCreateWithFlags(&e, hipEventDisableTiming));
  } else {
    PDK_TRY_HIP(hipEventCreate(&e));
  }
  *out = reinterpret_cast<uintptr_t>(e);
  return PDK_OK;
}

int pdk_event_destroy(uintptr_t event) {
  pdk::clear_error();
  if (!event) return PDK_OK;
  PDK_TRY_HIP(hipEventDestroy(pdk::as_event(event)));
  return PDK_OK;
}

int pdk_event_record(uintptr_t event, uintptr_t stream) {
  pdk::clear_error();
  PDK_REQUIRE(event != 0, "event is null");
  PDK_TRY_HIP(hipEventRecord(pdk::as_event(event), pdk::as_stream(stream)));
  return PDK_OK;
}

int pdk_event_query(uintptr_t event) {
  pdk::clear_error();
  PDK_REQUIRE(event != 0, "event is null");
  const hipError_t e = hipEventQuery(pdk::as_event(event));
  if (e == hipSuccess) return PDK_OK;
  if (e == hipErrorNotReady) return PDK_EAGAIN;
  return pdk::hip_fail(e, "hipEventQuery");
}

int pdk_event_sync(uintptr_t event) {
  pdk::clear_error();
  PDK_REQUIRE(event != 0, "event is null");
  PDK_TRY_HIP(hipEventSynchronize(pdk::as_event(event)));
  return PDK_OK;
}

int pdk_stream_wait_event(uintptr_t stream, uintptr_t event) {
  pdk::clear_error();
  PDK_REQUIRE(event != 0, "event is null");
  PDK_TRY_HIP(hipStreamWaitEvent(pdk::as_stream(stream), pdk::as_event(event), 0));
  return PDK_OK;
}

int pdk_event_elapsed_ms(uintptr_t start, uintptr_t stop, float* ms) {
  pdk::clear_error();
  PDK_REQUIRE(start && stop && ms, "null argument");
  PDK_TRY_HIP(hipEventElapsedTime(ms, pdk::as_event(start), pdk::as_event(stop)));
  return PDK_OK;
}

int pdk_ipc_export_mem(const void* dev_ptr, void* handle_out) {
  pdk::clear_error();
  PDK_REQUIRE(dev_ptr && handle_out, "null argument");
  static_assert(sizeof(hipIpcMemHandle_t) == PDK_IPC_HANDLE_BYTES, "IPC handle size");
  hipIpcMemHandle_t h;
  PDK_TRY_HIP(hipIpcGetMemHandle(&h, const_cast<void*>(dev_ptr)));
  memcpy(handle_out, &h, sizeof(h));
  return PDK_OK;
}

int pdk_ipc_open_mem(const void* handle, void** dev_ptr_out) {
  pdk::clear_error();
  PDK_REQUIRE(handle && dev_ptr_out, "null argument");
  hipIpcMemHandle_t h;
  memcpy(&h, handle, sizeof(h));
  *dev_ptr_out = nullptr;
  PDK_TRY_HIP(hipIpcOpenMemHandle(dev_ptr_out, h, hipIpcMemLazyEnablePeerAccess));
  return PDK_OK;
}

int pdk_ipc_close_mem(void* dev_ptr) {
  pdk::clear_error();
  PDK_REQUIRE(dev_ptr != nullptr, "null argument");
  PDK_TRY_HIP(hipIpcCloseMemHandle(dev_ptr));
  return PDK_OK;
}

int pdk_ipc_export_event(uintptr_t event, void* handle_out) {
  pdk::clear_error();
  PDK_REQUIRE(event && handle_out, "null argument");
  static_assert(sizeof(hipIpcEventHandle_t) == PDK_IPC_HANDLE_BYTES, "IPC event handle size");
  hipIpcEventHandle_t h;
  PDK_TRY_HIP(hipIpcGetEventHandle(&h, pdk::as_event(event)));
  memcpy(handle_out, &h, sizeof(h));
  return PDK_OK;
}

int pdk_ipc_open_event(const void* handle, uintptr_t* event_out) {
  pdk::clear_error();
  PDK_REQUIRE(handle && event_out, "null argument");
  hipIpcEventHandle_t h;
  memcpy(&h, handle, sizeof(h));
  hipEvent_t e = nullptr;
  PDK_TRY_HIP(hipIpcOpenEventHandle(&e, h));
  *event_out = reinterpret_cast<uintptr_t>(e);
  return PDK_OK;
}

}  // extern "C"
