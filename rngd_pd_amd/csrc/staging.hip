// Layer-wise staging pipeline: per-layer pack, per-layer copies between HBM
// and pinned host memory, per-layer scatter, chained by events across
// streams. Each entry point enqueues all layers in one native loop so the
// host never becomes the bottleneck of a pipeline whose per-layer device work
// is a few microseconds (kernels) to ~40 us (2 MiB over the host link).

#include "pdk_common.h"

namespace {

int check_events(const uintptr_t* ev, int n, const char* what) {
  if (!ev) return PDK_OK;
  for (int i = 0; i < n; ++i)
    PDK_REQUIRE(ev[i] != 0, "%s[%d] is null", what, i);
  return PDK_OK;
}

}  // namespace

extern "C" int pdk_pack_kv_layerwise(const pdk_pack_req* req, int n_layers, int S, int n_kv_heads,
                                     int head_dim, const uintptr_t* done_events,
                                     uintptr_t stream) {
  pdk::clear_error();
  PDK_REQUIRE(req != nullptr && n_layers >= 1, "bad arguments");
  int rc = check_events(done_events, n_layers, "done_events");
  if (rc) return rc;
  const int64_t F = (int64_t)n_kv_heads * head_dim * S;
  for (int l = 0; l < n_layers; ++l) {
    pdk_pack_req r = *req;
    if (r.P > 0) {
      r.src_k += (int64_t)l * req->layer_stride;
      r.src_v += (int64_t)l * req->layer_stride;
    }
    r.frame += (int64_t)l * 2 * F;
    rc = pdk_pack_kv_batch(&r, 1, 1, S, n_kv_heads, head_dim, stream);
    if (rc) return rc;
    if (done_events) PDK_TRY_HIP(hipEventRecord(pdk::as_event(done_events[l]), pdk::as_stream(stream)));
  }
  return PDK_OK;
}

extern "C" int pdk_copy_layers(void* dst, const void* src, size_t layer_bytes, int n_layers,
                               int direction, const uintptr_t* wait_events,
                               const uintptr_t* done_events, uintptr_t stream) {
  pdk::clear_error();
  PDK_REQUIRE(dst && src && n_layers >= 1 && layer_bytes > 0, "bad arguments");
  PDK_REQUIRE(direction >= PDK_COPY_D2H && direction <= PDK_COPY_D2D, "bad direction %d",
              direction);
  int rc = check_events(wait_events, n_layers, "wait_events");
  if (rc) return rc;
  rc = check_events(done_events, n_layers, "done_events");
  if (rc) return rc;
  hipStream_t st = pdk::as_stream(stream);
  for (int l = 0; l < n_layers; ++l) {
    if (wait_events) PDK_TRY_HIP(hipStreamWaitEvent(st, pdk::as_event(wait_events[l]), 0));
    char* d = static_cast<char*>(dst) + (size_t)l * layer_bytes;
    char* s = const_cast<char*>(static_cast<const char*>(src)) + (size_t)l * layer_bytes;
    if (direction == PDK_COPY_D2D) {
      PDK_TRY_HIP(hipMemcpyAsync(d, s, layer_bytes, hipMemcpyDeviceToDevice, st));
    } else {
      const bool to_host = direction == PDK_COPY_D2H;
      rc = pdk::copy_host_device(to_host ? d : s, to_host ? s : d, layer_bytes, to_host, st);
      if (rc) return rc;
    }
    if (done_events) PDK_TRY_HIP(hipEventRecord(pdk::as_event(done_events[l]), st));
  }
  return PDK_OK;
}

extern "C" int pdk_scatter_paged_layerwise(const pdk_scatter_req* req, int n_layers, int S,
                                           int n_kv_heads, int head_dim, uint16_t* cache_k,
                                           uint16_t* cache_v, int64_t cache_layer_stride,
                                           int num_blocks, const uintptr_t* wait_events,
                                           uintptr_t stream) {
  pdk::clear_error();
  PDK_REQUIRE(req != nullptr && n_layers >= 1, "bad arguments");
  PDK_REQUIRE(cache_k && cache_v, "null cache");
  int rc = check_events(wait_events, n_layers, "wait_events");
  if (rc) return rc;
  const int64_t F = (int64_t)n_kv_heads * head_dim * S;
  hipStream_t st = pdk::as_stream(stream);
  for (int l = 0; l < n_layers; ++l) {
    if (wait_events) PDK_TRY_HIP(hipStreamWaitEvent(st, pdk::as_event(wait_events[l]), 0));
    pdk_scatter_req r = *req;
    if (r.frame) r.frame += (int64_t)l * 2 * F;
    rc = pdk_scatter_paged_batch(&r, 1, 1, S, n_kv_heads, head_dim,
                                 cache_k + (int64_t)l * cache_layer_stride,
                                 cache_v + (int64_t)l * cache_layer_stride, cache_layer_stride,
                                 num_blocks, stream);
    if (rc) return rc;
  }
  return PDK_OK;
}
