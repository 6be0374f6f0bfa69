// Runtime of the C ABI: context, stream-ordered pooled allocator, copies, profiler, errors.
// Replaces the WebGPU runtime of app/gpu/device.js (GPU, BufferPool, Profiler).
#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstddef>
#include <cstdio>
#include <cstring>
#include <string>

#include "internal.h"

namespace {
thread_local std::string g_init_error;  // errors of anima_init (no context yet)

// 1/8-power-of-two size buckets, minimum 256 B (the bucketing of app/gpu/device.js:33-39).
size_t bucket(size_t bytes) {
  size_t b = std::max<size_t>(256, bytes);
  size_t p = size_t(1) << (63 - __builtin_clzll(b));
  size_t step = std::max<size_t>(256, p / 8);
  return (b + step - 1) / step * step;
}
}  // namespace

namespace anima {

int fail(anima_ctx* c, int code, const char* fmt, ...) {
  char buf[1024];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  if (c) c->err = buf;
  else g_init_error = buf;
  return code;
}

int hip_fail(anima_ctx* c, hipError_t e, const char* what) {
  if (c && (e == hipErrorIllegalAddress || e == hipErrorLaunchFailure || e == hipErrorAssert))
    c->lost = true;  // the device context is unusable after a fault (device lost)
  return fail(c, e == hipErrorOutOfMemory ? ANIMA_E_OOM : ANIMA_E_HIP, "%s: %s (%d)", what,
              hipGetErrorString(e), (int)e);
}

int workspace(anima_ctx* c, size_t bytes, void** out) {
  if (c->capturing) {
    // A graph's replays keep using the scratch its capture was handed, so the capture gets a pool
    // buffer of the requested size, parked for the graph at once (the graph owns it from
    // anima_graph_end on), and never the context's own workspace, which may have grown far
    // larger for some earlier call.  Later requests of the same capture reuse parked buffers:
    // the stream runs them in order.
    void* p = nullptr;
    int rc = anima_alloc(c, bytes, &p);
    if (rc != ANIMA_OK) return rc;
    anima_free(c, p);
    *out = p;
    return ANIMA_OK;
  }
  if (bytes > c->ws_bytes) {
    if (c->ws) {
      hipError_t e = hipStreamSynchronize(c->stream);
      if (e != hipSuccess) return hip_fail(c, e, "workspace sync");
      hipFree(c->ws);
      c->allocated -= c->ws_bytes;
      c->ws = nullptr;
      c->ws_bytes = 0;
    }
    size_t want = bucket(bytes);
    hipError_t e = hipMalloc(&c->ws, want);
    if (e != hipSuccess) {
      c->ws = nullptr;
      return hip_fail(c, e, "workspace hipMalloc");
    }
    c->ws_bytes = want;
    c->allocated += want;
    c->peak = std::max(c->peak, c->allocated);
  }
  *out = c->ws;
  return ANIMA_OK;
}

static hipEvent_t take_event(anima_ctx* c) {
  if (!c->spare_events.empty()) {
    hipEvent_t e = c->spare_events.back();
    c->spare_events.pop_back();
    return e;
  }
  hipEvent_t e = nullptr;
  if (hipEventCreate(&e) != hipSuccess) return nullptr;
  return e;
}

Launch::Launch(anima_ctx* ctx, const char* name, double flops, double bytes)
    : c(ctx), rec{name, flops, bytes, nullptr, nullptr}, on(ctx->profiling && !ctx->capturing) {
  if (on) {
    rec.a = take_event(c);
    rec.b = take_event(c);
    if (!rec.a || !rec.b) on = false;
    else hipEventRecord(rec.a, c->stream);
  }
}

int Launch::end() {
  hipError_t e = hipGetLastError();
  if (on) {
    hipEventRecord(rec.b, c->stream);
    c->recs.push_back(rec);
  }
  if (e != hipSuccess) return hip_fail(c, e, rec.name);
  return ANIMA_OK;
}

// Resolves pending profiler records into per-name statistics (needs a synchronized stream).
static void collect(anima_ctx* c) {
  for (auto& r : c->recs) {
    float ms = 0;
    hipEventElapsedTime(&ms, r.a, r.b);
    Stat& s = c->stats[r.name];
    s.count++;
    s.ms += ms;
    s.flops += r.flops;
    s.bytes += r.bytes;
    c->spare_events.push_back(r.a);
    c->spare_events.push_back(r.b);
  }
  c->recs.clear();
}

}  // namespace anima

using namespace anima;

#define CHECK_CTX(c)                                                                      \
  do {                                                                                    \
    if (!(c)) return fail(nullptr, ANIMA_E_ARG, "null context");                          \
    if ((c)->lost) return fail((c), ANIMA_E_STATE, "context lost after a device error: %s", \
                               (c)->err.c_str());                                         \
  } while (0)

#define NOT_CAPTURING(c, what)                                                                 \
  do {                                                                                         \
    if ((c)->capturing) return fail((c), ANIMA_E_STATE, "%s: not allowed while capturing a graph", what); \
  } while (0)

static void release_graph(anima_ctx* c, anima_graph* g, bool to_pool) {
  if (g->exec) hipGraphExecDestroy(g->exec);
  if (g->graph) hipGraphDestroy(g->graph);
  for (auto& b : g->owned) {
    if (to_pool) {
      c->free_lists[b.second].push_back(b.first);
      c->pooled += b.second;
    } else {
      hipFree(b.first);
    }
  }
  delete g;
}

// Ends a failed capture: buffers parked for it go back to the pool.
static void drop_capture(anima_ctx* c) {
  for (auto& kv : c->cap_free)
    for (void* p : kv.second) {
      c->free_lists[kv.first].push_back(p);
      c->pooled += kv.first;
    }
  c->cap_free.clear();
  c->capturing = false;
}

// The pinned staging ring of anima_h2d, allocated on first use (4 x 4 MiB of page-locked host
// memory per context).  If the host refuses it, copies stay on the pageable path.
static bool stage_ready(anima_ctx* c) {
  if (c->stage[0]) return true;
  if (c->stage_failed) return false;
  for (int i = 0; i < anima_ctx::kStageSlots; i++) {
    if (hipHostMalloc(&c->stage[i], anima_ctx::kStageBytes, hipHostMallocDefault) != hipSuccess ||
        hipEventCreateWithFlags(&c->stage_ev[i], hipEventDisableTiming) != hipSuccess) {
      for (int j = 0; j <= i; j++) {
        if (c->stage[j]) hipHostFree(c->stage[j]);
        if (c->stage_ev[j]) hipEventDestroy(c->stage_ev[j]);
        c->stage[j] = nullptr;
        c->stage_ev[j] = nullptr;
      }
      hipGetLastError();  // the refusal is not an error of the copy that asked
      c->stage_failed = true;
      return false;
    }
  }
  return true;
}

extern "C" {

int anima_init(int device, anima_ctx** out) {
  if (!out) return fail(nullptr, ANIMA_E_ARG, "anima_init: out is NULL");
  *out = nullptr;
  int n = 0;
  hipError_t e = hipGetDeviceCount(&n);
  if (e != hipSuccess || n == 0) return fail(nullptr, ANIMA_E_HIP, "anima_init: no HIP device (%s)", hipGetErrorString(e));
  if (device < 0 || device >= n) return fail(nullptr, ANIMA_E_ARG, "anima_init: device %d out of range [0,%d)", device, n);
  hipDeviceProp_t prop;
  e = hipGetDeviceProperties(&prop, device);
  if (e != hipSuccess) return fail(nullptr, ANIMA_E_HIP, "hipGetDeviceProperties: %s", hipGetErrorString(e));
  if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0)
    return fail(nullptr, ANIMA_E_UNSUPPORTED, "anima_init: device %d is %s; this library is built for gfx950 (MI355X) only", device, prop.gcnArchName);
  e = hipSetDevice(device);
  if (e != hipSuccess) return fail(nullptr, ANIMA_E_HIP, "hipSetDevice: %s", hipGetErrorString(e));
  anima_ctx* c = new anima_ctx();
  c->device = device;
  c->num_cus = prop.multiProcessorCount > 0 ? prop.multiProcessorCount : 256;
  e = hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking);
  if (e == hipSuccess) e = hipEventCreate(&c->t0);
  if (e == hipSuccess) e = hipEventCreate(&c->t1);
  if (e != hipSuccess) {
    fail(nullptr, ANIMA_E_HIP, "anima_init: %s", hipGetErrorString(e));
    if (c->stream) hipStreamDestroy(c->stream);
    delete c;
    return ANIMA_E_HIP;
  }
  int rc = attention_scratch_init(c);
  if (rc != ANIMA_OK) {
    fail(nullptr, rc, "anima_init: %s", c->err.c_str());
    hipEventDestroy(c->t0);
    hipEventDestroy(c->t1);
    hipStreamDestroy(c->stream);
    delete c;
    return rc;
  }
  *out = c;
  return ANIMA_OK;
}

int anima_destroy(anima_ctx* c) {
  if (!c) return ANIMA_OK;
  hipSetDevice(c->device);
  if (c->capturing) {
    hipGraph_t g = nullptr;
    hipStreamEndCapture(c->stream, &g);
    if (g) hipGraphDestroy(g);
    drop_capture(c);
  }
  hipStreamSynchronize(c->stream);
  for (anima_graph* g : c->graphs) release_graph(c, g, false);
  c->graphs.clear();
  for (auto& kv : c->free_lists)
    for (void* p : kv.second) hipFree(p);
  for (auto& kv : c->live) hipFree(kv.first);
  if (c->ws) hipFree(c->ws);
  for (auto& r : c->recs) {
    hipEventDestroy(r.a);
    hipEventDestroy(r.b);
  }
  for (hipEvent_t e : c->spare_events) hipEventDestroy(e);
  for (int i = 0; i < anima_ctx::kStageSlots; i++) {
    if (c->stage[i]) hipHostFree(c->stage[i]);
    if (c->stage_ev[i]) hipEventDestroy(c->stage_ev[i]);
  }
  for (int i = 0; i < anima_ctx::kMarks; i++)
    if (c->marks[i]) hipEventDestroy(c->marks[i]);
  if (c->t0) hipEventDestroy(c->t0);
  if (c->t1) hipEventDestroy(c->t1);
  hipStreamDestroy(c->stream);
  delete c;
  return ANIMA_OK;
}

const char* anima_last_error(const anima_ctx* c) { return c ? c->err.c_str() : g_init_error.c_str(); }

int anima_sync(anima_ctx* c) {
  CHECK_CTX(c);
  NOT_CAPTURING(c, "anima_sync");
  hipError_t e = hipStreamSynchronize(c->stream);
  if (e != hipSuccess) return hip_fail(c, e, "anima_sync");
  e = hipGetLastError();
  if (e != hipSuccess) return hip_fail(c, e, "anima_sync (deferred)");
  return ANIMA_OK;
}

int anima_flush(anima_ctx* c) {
  CHECK_CTX(c);
  return ANIMA_OK;
}

int anima_mem_stats(anima_ctx* c, uint64_t* allocated, uint64_t* peak, uint64_t* pooled) {
  if (!c) return fail(nullptr, ANIMA_E_ARG, "null context");
  if (allocated) *allocated = c->allocated;
  if (peak) *peak = c->peak;
  if (pooled) *pooled = c->pooled;
  return ANIMA_OK;
}

int anima_device_limits(anima_ctx* c, anima_limits* out) {
  CHECK_CTX(c);
  if (!out) return fail(c, ANIMA_E_ARG, "anima_device_limits: out is NULL");
  hipDeviceProp_t p;
  hipError_t e = hipGetDeviceProperties(&p, c->device);
  if (e != hipSuccess) return hip_fail(c, e, "anima_device_limits (properties)");
  size_t fr = 0, tot = 0;
  e = hipMemGetInfo(&fr, &tot);
  if (e != hipSuccess) return hip_fail(c, e, "anima_device_limits (memory)");
  memset(out, 0, sizeof *out);
  out->max_buffer_size = (int64_t)p.totalGlobalMem;
  out->max_binding_size = (int64_t)p.totalGlobalMem;
  out->total_memory = (int64_t)tot;
  out->free_memory = (int64_t)fr;
  out->workgroup_storage_size = (int32_t)p.sharedMemPerBlock;
  out->max_workgroup_size = p.maxThreadsPerBlock;
  out->max_workgroups_per_dimension = p.maxGridSize[0];
  out->compute_units = p.multiProcessorCount;
  out->wavefront_size = p.warpSize;
  out->clock_khz = p.clockRate;
  snprintf(out->arch, sizeof out->arch, "%s", p.gcnArchName);
  return ANIMA_OK;
}

int anima_alloc(anima_ctx* c, size_t bytes, void** out) {
  CHECK_CTX(c);
  if (!out) return fail(c, ANIMA_E_ARG, "anima_alloc: out is NULL");
  size_t size = bucket(bytes);
  if (c->capturing) {
    auto ct = c->cap_free.find(size);
    if (ct != c->cap_free.end() && !ct->second.empty()) {
      *out = ct->second.back();
      ct->second.pop_back();
      c->live[*out] = size;
      return ANIMA_OK;
    }
  }
  auto it = c->free_lists.find(size);
  if (it != c->free_lists.end() && !it->second.empty()) {
    *out = it->second.back();
    it->second.pop_back();
    c->pooled -= size;
    c->live[*out] = size;
    return ANIMA_OK;
  }
  void* p = nullptr;
  hipError_t e = hipMalloc(&p, size);
  if (e != hipSuccess && c->capturing) return hip_fail(c, e, "anima_alloc (while capturing a graph)");
  if (e != hipSuccess) {
    // release parked buffers and retry once (the pool's trim)
    hipStreamSynchronize(c->stream);
    for (auto& kv : c->free_lists)
      for (void* q : kv.second) {
        hipFree(q);
        c->allocated -= kv.first;
      }
    c->free_lists.clear();
    c->pooled = 0;
    hipGetLastError();
    e = hipMalloc(&p, size);
    if (e != hipSuccess) return hip_fail(c, e, "anima_alloc");
  }
  c->allocated += size;
  c->peak = std::max(c->peak, c->allocated);
  c->live[p] = size;
  *out = p;
  return ANIMA_OK;
}

int anima_free(anima_ctx* c, void* p) {
  if (!c) return fail(nullptr, ANIMA_E_ARG, "null context");
  if (!p) return ANIMA_OK;
  auto it = c->live.find(p);
  if (it == c->live.end()) return fail(c, ANIMA_E_ARG, "anima_free: %p was not allocated by this context (or freed twice)", p);
  if (c->capturing) {  // reserved for the graph being captured
    c->cap_free[it->second].push_back(p);
    c->live.erase(it);
    return ANIMA_OK;
  }
  c->free_lists[it->second].push_back(p);
  c->pooled += it->second;
  c->live.erase(it);
  return ANIMA_OK;
}

int anima_pool_trim(anima_ctx* c) {
  CHECK_CTX(c);
  NOT_CAPTURING(c, "anima_pool_trim");
  hipError_t e = hipStreamSynchronize(c->stream);
  if (e != hipSuccess) return hip_fail(c, e, "anima_pool_trim");
  for (auto& kv : c->free_lists)
    for (void* q : kv.second) {
      hipFree(q);
      c->allocated -= kv.first;
    }
  c->free_lists.clear();
  c->pooled = 0;
  return ANIMA_OK;
}

int anima_h2d(anima_ctx* c, void* dst, const void* src, size_t bytes) {
  CHECK_CTX(c);
  NOT_CAPTURING(c, "anima_h2d");
  if (bytes == 0) return ANIMA_OK;
  if (!dst || !src) return fail(c, ANIMA_E_ARG, "anima_h2d: null pointer");
  hipError_t e;
  if (bytes <= anima_ctx::kStageBytes && stage_ready(c)) {
    // copy into a pinned slot and enqueue the DMA from there: the call returns without waiting
    // for the work already on the stream, and `src` may be reused at once
    const int s = c->stage_next;
    c->stage_next = (s + 1) % anima_ctx::kStageSlots;
    if (c->stage_pending[s]) {
      e = hipEventSynchronize(c->stage_ev[s]);
      if (e != hipSuccess) return hip_fail(c, e, "anima_h2d (staging slot)");
      c->stage_pending[s] = false;
    }
    std::memcpy(c->stage[s], src, bytes);
    e = hipMemcpyAsync(dst, c->stage[s], bytes, hipMemcpyHostToDevice, c->stream);
    if (e == hipSuccess) e = hipEventRecord(c->stage_ev[s], c->stream);
    if (e != hipSuccess) return hip_fail(c, e, "anima_h2d");
    c->stage_pending[s] = true;
    return ANIMA_OK;
  }
  // larger copies: hipMemcpyAsync from pageable memory stages the source before it returns (and
  // waits for the stream to reach the copy), so `src` may be reused
  e = hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, c->stream);
  if (e != hipSuccess) return hip_fail(c, e, "anima_h2d");
  return ANIMA_OK;
}

int anima_mark(anima_ctx* c, uint64_t* ticket) {
  CHECK_CTX(c);
  NOT_CAPTURING(c, "anima_mark");
  if (!ticket) return fail(c, ANIMA_E_ARG, "anima_mark: ticket is NULL");
  const int s = (int)(c->mark_count % anima_ctx::kMarks);
  hipError_t e = hipSuccess;
  if (!c->marks[s]) e = hipEventCreateWithFlags(&c->marks[s], hipEventDisableTiming);
  if (e == hipSuccess) e = hipEventRecord(c->marks[s], c->stream);
  if (e != hipSuccess) return hip_fail(c, e, "anima_mark");
  *ticket = c->mark_count++;
  return ANIMA_OK;
}

int anima_wait_mark(anima_ctx* c, uint64_t ticket) {
  CHECK_CTX(c);
  NOT_CAPTURING(c, "anima_wait_mark");
  if (ticket >= c->mark_count)
    return fail(c, ANIMA_E_ARG, "anima_wait_mark: ticket %llu was not issued (next is %llu)", (unsigned long long)ticket,
                (unsigned long long)c->mark_count);
  // a ticket older than the last kMarks marks shares its slot with a later mark: waiting for that
  // later point also covers the work before the older one
  hipError_t e = hipEventSynchronize(c->marks[ticket % anima_ctx::kMarks]);
  if (e != hipSuccess) return hip_fail(c, e, "anima_wait_mark");
  e = hipGetLastError();
  if (e != hipSuccess) return hip_fail(c, e, "anima_wait_mark (deferred)");
  return ANIMA_OK;
}

int anima_d2h(anima_ctx* c, void* dst, const void* src, size_t bytes) {
  CHECK_CTX(c);
  NOT_CAPTURING(c, "anima_d2h");
  if (bytes == 0) return ANIMA_OK;
  if (!dst || !src) return fail(c, ANIMA_E_ARG, "anima_d2h: null pointer");
  hipError_t e = hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, c->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
  if (e != hipSuccess) return hip_fail(c, e, "anima_d2h");
  return ANIMA_OK;
}

int anima_d2d(anima_ctx* c, void* dst, const void* src, size_t bytes) {
  CHECK_CTX(c);
  if (bytes == 0) return ANIMA_OK;
  if (!dst || !src) return fail(c, ANIMA_E_ARG, "anima_d2d: null pointer");
  hipError_t e = hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, c->stream);
  if (e != hipSuccess) return hip_fail(c, e, "anima_d2d");
  return ANIMA_OK;
}

int anima_profile_enable(anima_ctx* c, int on) {
  CHECK_CTX(c);
  c->profiling = on != 0;
  return ANIMA_OK;
}

int anima_profile_reset(anima_ctx* c) {
  CHECK_CTX(c);
  NOT_CAPTURING(c, "anima_profile_reset");
  hipError_t e = hipStreamSynchronize(c->stream);
  if (e != hipSuccess) return hip_fail(c, e, "anima_profile_reset");
  collect(c);
  c->stats.clear();
  return ANIMA_OK;
}

int anima_profile_report(anima_ctx* c, char* buf, size_t len) {
  CHECK_CTX(c);
  NOT_CAPTURING(c, "anima_profile_report");
  if (!buf || len == 0) return fail(c, ANIMA_E_ARG, "anima_profile_report: empty buffer");
  hipError_t e = hipStreamSynchronize(c->stream);
  if (e != hipSuccess) return hip_fail(c, e, "anima_profile_report");
  collect(c);
  std::vector<std::pair<std::string, Stat>> rows(c->stats.begin(), c->stats.end());
  std::sort(rows.begin(), rows.end(), [](auto& a, auto& b) { return a.second.ms > b.second.ms; });
  std::string s = "[";
  char tmp[512];
  for (size_t i = 0; i < rows.size(); i++) {
    snprintf(tmp, sizeof tmp, "%s{\"name\":\"%s\",\"count\":%lld,\"ms\":%.6f,\"flops\":%.6e,\"bytes\":%.6e}",
             i ? "," : "", rows[i].first.c_str(), (long long)rows[i].second.count, rows[i].second.ms,
             rows[i].second.flops, rows[i].second.bytes);
    s += tmp;
  }
  s += "]";
  if (s.size() + 1 > len) return fail(c, ANIMA_E_ARG, "anima_profile_report: buffer of %zu bytes, need %zu", len, s.size() + 1);
  std::memcpy(buf, s.c_str(), s.size() + 1);
  return ANIMA_OK;
}

int anima_timer_start(anima_ctx* c) {
  CHECK_CTX(c);
  NOT_CAPTURING(c, "anima_timer_start");
  hipError_t e = hipEventRecord(c->t0, c->stream);
  if (e != hipSuccess) return hip_fail(c, e, "anima_timer_start");
  return ANIMA_OK;
}

int anima_timer_stop(anima_ctx* c, float* ms) {
  CHECK_CTX(c);
  NOT_CAPTURING(c, "anima_timer_stop");
  if (!ms) return fail(c, ANIMA_E_ARG, "anima_timer_stop: ms is NULL");
  hipError_t e = hipEventRecord(c->t1, c->stream);
  if (e == hipSuccess) e = hipEventSynchronize(c->t1);
  if (e == hipSuccess) e = hipEventElapsedTime(ms, c->t0, c->t1);
  if (e != hipSuccess) return hip_fail(c, e, "anima_timer_stop");
  return ANIMA_OK;
}

int anima_attention(anima_ctx* c, const anima_attn_desc* d) {
  CHECK_CTX(c);
  if (!d) return fail(c, ANIMA_E_ARG, "anima_attention: null descriptor");
  return attention_launch(c, d);
}

int anima_conv3x3(anima_ctx* c, const anima_conv_desc* d) {
  CHECK_CTX(c);
  return conv3x3_launch(c, d);
}

int anima_channel_norm(anima_ctx* c, const float* x, const float* gamma, float* y, int64_t rows, int cols, int silu) {
  CHECK_CTX(c);
  return channel_norm_launch(c, x, gamma, y, rows, cols, silu);
}

int anima_weight_unpack_w4(anima_ctx* c, const anima_weight* w4, int8_t* grid) {
  CHECK_CTX(c);
  NOT_CAPTURING(c, "anima_weight_unpack_w4");
  return weight_unpack_w4_launch(c, w4, grid);
}

int anima_set_w4_path(anima_ctx* c, int path) {
  CHECK_CTX(c);
  if (path != ANIMA_W4_GRID_SCRATCH && path != ANIMA_W4_IN_GEMM) return fail(c, ANIMA_E_ARG, "anima_set_w4_path: unknown path %d", path);
  c->w4_path = path;
  return ANIMA_OK;
}

int anima_to_rgba(anima_ctx* c, const float* x, int64_t n, uint8_t* out) {
  CHECK_CTX(c);
  return to_rgba_launch(c, x, n, out);
}

int anima_attention_noalloc(anima_ctx* c, const anima_attn_desc* d) {
  CHECK_CTX(c);
  return attention_noalloc_launch(c, d);
}

int64_t anima_attention_noalloc_scratch_bytes(void) { return (int64_t)attention_scratch_bytes(); }

int anima_attention_prepare_kv(anima_ctx* c, const anima_attn_desc* d, void* kv_prep) {
  CHECK_CTX(c);
  return attention_prepare_kv_launch(c, d, kv_prep);
}

int64_t anima_attention_kv_bytes(int B, int Hkv, int Lk, int precision) { return attention_kv_bytes(B, Hkv, Lk, precision); }

int anima_qk_norm_rope(anima_ctx* c, float* qkv, int64_t L, int H, int D, int64_t ld,
                       const float* qn, const float* kn, const float* cs, int64_t sin_off, float eps) {
  CHECK_CTX(c);
  return qk_norm_rope_launch(c, qkv, L, H, D, ld, qn, kn, cs, sin_off, eps);
}

int anima_rmsnorm(anima_ctx* c, const float* x, const float* w, float* y, int64_t rows, int cols, float eps) {
  CHECK_CTX(c);
  return rmsnorm_launch(c, x, w, y, rows, cols, eps);
}

int anima_rope(anima_ctx* c, float* x, const float* cs, int64_t L, int H, int D, int64_t sin_off,
               int64_t row_stride, int64_t col_off) {
  CHECK_CTX(c);
  return rope_launch(c, x, cs, L, H, D, sin_off, row_stride, col_off);
}

int anima_hadamard(anima_ctx* c, const float* x, float* y, int64_t n) {
  CHECK_CTX(c);
  return hadamard_launch(c, x, y, n);
}

int anima_quant_rows(anima_ctx* c, const float* x, int64_t M, int K, int rotate, int8_t* q, float* s) {
  CHECK_CTX(c);
  return quant_rows_launch(c, x, M, K, rotate, ANIMA_ACT_NONE, q, s);
}

int anima_quant_rows_act(anima_ctx* c, const float* x, int64_t M, int K, int act, int rotate, int8_t* q, float* s) {
  CHECK_CTX(c);
  return quant_rows_launch(c, x, M, K, rotate, act, q, s);
}

int anima_quant_rows_bf16(anima_ctx* c, const uint16_t* x, int64_t M, int K, int rotate, int8_t* q, float* s) {
  CHECK_CTX(c);
  return quant_rows_bf16_launch(c, x, M, K, rotate, q, s);
}

int anima_layernorm_mod(anima_ctx* c, const float* x, const float* mod, int64_t shift_off, int64_t scale_off,
                        int64_t rows, int cols, float eps, int rotate, float* y, int8_t* q, float* s) {
  CHECK_CTX(c);
  return layernorm_mod_launch(c, x, mod, shift_off, scale_off, rows, cols, eps, rotate, y, q, s);
}

int anima_elementwise(anima_ctx* c, int op, const float* a, const float* b, float* y, int64_t n) {
  CHECK_CTX(c);
  return elementwise_launch(c, op, a, b, y, n);
}

int anima_zero(anima_ctx* c, float* y, int64_t n) {
  CHECK_CTX(c);
  return zero_launch(c, y, n);
}

int anima_patchify(anima_ctx* c, const float* latents, int B, int h, int w, float* patches) {
  CHECK_CTX(c);
  return patchify_launch(c, latents, patches, B, h, w, false);
}

int anima_unpatchify(anima_ctx* c, const float* o, int B, int h, int w, float* latents) {
  CHECK_CTX(c);
  return patchify_launch(c, o, latents, B, h, w, true);
}

int anima_split3_bf16(anima_ctx* c, const float* src, uint16_t* dst, int64_t n) {
  CHECK_CTX(c);
  return split3_launch(c, src, dst, n);
}

int anima_sampler_step(anima_ctx* c, const anima_sampler_desc* d) {
  CHECK_CTX(c);
  return sampler_step_launch(c, d);
}

int anima_fill_random(anima_ctx* c, void* dst, int64_t n, int kind, uint64_t seed, float lo, float hi) {
  CHECK_CTX(c);
  return fill_random_launch(c, dst, n, kind, seed, lo, hi);
}

int anima_linear(anima_ctx* c, const anima_linear_desc* d) {
  CHECK_CTX(c);
  if (!d) return fail(c, ANIMA_E_ARG, "anima_linear: null descriptor");
  return linear_launch(c, d);
}

int anima_linear_qkv(anima_ctx* c, const anima_linear_desc* d, const anima_qkv_desc* p) {
  CHECK_CTX(c);
  return linear_qkv_launch(c, d, p);
}

int anima_linear_grouped_bf16(anima_ctx* c, int G, int64_t M, int N, int K, const float* x, int64_t ldx,
                              int64_t x_gstride, const uint16_t* w, int64_t w_gstride, const float* bias,
                              int64_t bias_gstride, float* out, int64_t ldc, int64_t out_gstride) {
  CHECK_CTX(c);
  return linear_grouped_bf16_launch(c, G, M, N, K, x, ldx, x_gstride, w, w_gstride, bias, bias_gstride, out, ldc,
                                    out_gstride);
}

int anima_gemv_grouped_f32(anima_ctx* c, int G, int N, int K, const float* x, int64_t x_gstride, const float* w,
                           int64_t w_gstride, float* y, int64_t y_gstride, float alpha, int accumulate) {
  CHECK_CTX(c);
  return gemv_grouped_f32_launch(c, G, N, K, x, x_gstride, w, w_gstride, y, y_gstride, alpha, accumulate);
}

#define ABI_FIELD(T, f) {#T, #f, (int64_t)offsetof(T, f)}
#define ABI_SIZE(T) {#T, nullptr, (int64_t)sizeof(T)}
static const struct {
  const char* type;
  const char* field;
  int64_t value;
} k_abi[] = {
    ABI_SIZE(anima_attn_desc), ABI_FIELD(anima_attn_desc, B), ABI_FIELD(anima_attn_desc, Lq),
    ABI_FIELD(anima_attn_desc, Lk), ABI_FIELD(anima_attn_desc, H), ABI_FIELD(anima_attn_desc, D),
    ABI_FIELD(anima_attn_desc, group), ABI_FIELD(anima_attn_desc, q), ABI_FIELD(anima_attn_desc, ldq),
    ABI_FIELD(anima_attn_desc, q_off), ABI_FIELD(anima_attn_desc, q_bstride), ABI_FIELD(anima_attn_desc, k),
    ABI_FIELD(anima_attn_desc, ldk), ABI_FIELD(anima_attn_desc, k_off), ABI_FIELD(anima_attn_desc, k_bstride),
    ABI_FIELD(anima_attn_desc, v), ABI_FIELD(anima_attn_desc, ldv), ABI_FIELD(anima_attn_desc, v_off),
    ABI_FIELD(anima_attn_desc, v_bstride), ABI_FIELD(anima_attn_desc, o), ABI_FIELD(anima_attn_desc, ldo),
    ABI_FIELD(anima_attn_desc, o_off), ABI_FIELD(anima_attn_desc, o_bstride), ABI_FIELD(anima_attn_desc, scale),
    ABI_FIELD(anima_attn_desc, kv_len), ABI_FIELD(anima_attn_desc, precision), ABI_FIELD(anima_attn_desc, q_norm),
    ABI_FIELD(anima_attn_desc, k_norm), ABI_FIELD(anima_attn_desc, rope_cs), ABI_FIELD(anima_attn_desc, rope_sin_off),
    ABI_FIELD(anima_attn_desc, eps), ABI_FIELD(anima_attn_desc, causal), ABI_FIELD(anima_attn_desc, kv_prep),
    ABI_FIELD(anima_attn_desc, kv_prep_bytes), ABI_FIELD(anima_attn_desc, q_prep), ABI_FIELD(anima_attn_desc, o_bf16),
    ABI_SIZE(anima_weight), ABI_FIELD(anima_weight, kind), ABI_FIELD(anima_weight, N), ABI_FIELD(anima_weight, K),
    ABI_FIELD(anima_weight, w), ABI_FIELD(anima_weight, scale), ABI_FIELD(anima_weight, srel),
    ABI_FIELD(anima_weight, codebook), ABI_FIELD(anima_weight, bias),
    ABI_SIZE(anima_linear_desc), ABI_FIELD(anima_linear_desc, M), ABI_FIELD(anima_linear_desc, W),
    ABI_FIELD(anima_linear_desc, x), ABI_FIELD(anima_linear_desc, ldx), ABI_FIELD(anima_linear_desc, x_rotated),
    ABI_FIELD(anima_linear_desc, xq), ABI_FIELD(anima_linear_desc, xs), ABI_FIELD(anima_linear_desc, out),
    ABI_FIELD(anima_linear_desc, ldc), ABI_FIELD(anima_linear_desc, alpha), ABI_FIELD(anima_linear_desc, act),
    ABI_FIELD(anima_linear_desc, epilogue), ABI_FIELD(anima_linear_desc, gate), ABI_FIELD(anima_linear_desc, gate_off),
    ABI_FIELD(anima_linear_desc, acc_out), ABI_FIELD(anima_linear_desc, add), ABI_FIELD(anima_linear_desc, ld_add),
    ABI_FIELD(anima_linear_desc, lora_xa), ABI_FIELD(anima_linear_desc, ld_lora_xa), ABI_FIELD(anima_linear_desc, lora_b),
    ABI_FIELD(anima_linear_desc, lora_r), ABI_FIELD(anima_linear_desc, lora_cols),
    ABI_SIZE(anima_sampler_desc), ABI_FIELD(anima_sampler_desc, kind), ABI_FIELD(anima_sampler_desc, n),
    ABI_FIELD(anima_sampler_desc, x), ABI_FIELD(anima_sampler_desc, v), ABI_FIELD(anima_sampler_desc, v_uncond),
    ABI_FIELD(anima_sampler_desc, cfg), ABI_FIELD(anima_sampler_desc, sigma), ABI_FIELD(anima_sampler_desc, final_step),
    ABI_FIELD(anima_sampler_desc, stage), ABI_FIELD(anima_sampler_desc, den_out), ABI_FIELD(anima_sampler_desc, old),
    ABI_FIELD(anima_sampler_desc, old_d), ABI_FIELD(anima_sampler_desc, eps), ABI_FIELD(anima_sampler_desc, c),
    ABI_SIZE(anima_conv_desc), ABI_FIELD(anima_conv_desc, B), ABI_FIELD(anima_conv_desc, H), ABI_FIELD(anima_conv_desc, W),
    ABI_FIELD(anima_conv_desc, cin), ABI_FIELD(anima_conv_desc, cout), ABI_FIELD(anima_conv_desc, up),
    ABI_FIELD(anima_conv_desc, x), ABI_FIELD(anima_conv_desc, w), ABI_FIELD(anima_conv_desc, bias),
    ABI_FIELD(anima_conv_desc, out), ABI_FIELD(anima_conv_desc, resid), ABI_FIELD(anima_conv_desc, precision),
    ABI_SIZE(anima_limits), ABI_FIELD(anima_limits, max_buffer_size), ABI_FIELD(anima_limits, max_binding_size),
    ABI_FIELD(anima_limits, total_memory), ABI_FIELD(anima_limits, free_memory),
    ABI_FIELD(anima_limits, workgroup_storage_size), ABI_FIELD(anima_limits, max_workgroup_size),
    ABI_FIELD(anima_limits, max_workgroups_per_dimension), ABI_FIELD(anima_limits, compute_units),
    ABI_FIELD(anima_limits, wavefront_size), ABI_FIELD(anima_limits, clock_khz), ABI_FIELD(anima_limits, arch),
    ABI_SIZE(anima_qkv_desc), ABI_FIELD(anima_qkv_desc, B), ABI_FIELD(anima_qkv_desc, L), ABI_FIELD(anima_qkv_desc, H),
    ABI_FIELD(anima_qkv_desc, k_norm), ABI_FIELD(anima_qkv_desc, rope_cs), ABI_FIELD(anima_qkv_desc, rope_sin_off),
    ABI_FIELD(anima_qkv_desc, eps), ABI_FIELD(anima_qkv_desc, kv_prep), ABI_FIELD(anima_qkv_desc, kv_prep_bytes),
    ABI_FIELD(anima_qkv_desc, q_norm), ABI_FIELD(anima_qkv_desc, q_prep), ABI_FIELD(anima_qkv_desc, q_scale),
};
#undef ABI_FIELD
#undef ABI_SIZE

int64_t anima_abi_offset(const char* type, const char* field) {
  if (!type) return -1;
  for (const auto& e : k_abi)
    if (!strcmp(e.type, type) && ((!field && !e.field) || (field && e.field && !strcmp(field, e.field))))
      return e.value;
  return -1;
}

int anima_graph_begin(anima_ctx* c) {
  CHECK_CTX(c);
  NOT_CAPTURING(c, "anima_graph_begin");
  hipError_t e = hipStreamBeginCapture(c->stream, hipStreamCaptureModeRelaxed);
  if (e != hipSuccess) return hip_fail(c, e, "anima_graph_begin");
  c->capturing = true;
  c->cap_free.clear();
  return ANIMA_OK;
}

int anima_graph_end(anima_ctx* c, anima_graph** out) {
  CHECK_CTX(c);
  if (!out) return fail(c, ANIMA_E_ARG, "anima_graph_end: out is NULL");
  *out = nullptr;
  if (!c->capturing) return fail(c, ANIMA_E_STATE, "anima_graph_end: no capture in progress");
  hipGraph_t graph = nullptr;
  hipError_t e = hipStreamEndCapture(c->stream, &graph);
  if (e != hipSuccess) {
    if (graph) hipGraphDestroy(graph);
    drop_capture(c);
    return hip_fail(c, e, "anima_graph_end (capture)");
  }
  hipGraphExec_t exec = nullptr;
  e = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
  if (e != hipSuccess) {
    hipGraphDestroy(graph);
    drop_capture(c);
    return hip_fail(c, e, "anima_graph_end (instantiate)");
  }
  anima_graph* g = new anima_graph();
  g->graph = graph;
  g->exec = exec;
  for (auto& kv : c->cap_free)
    for (void* p : kv.second) g->owned.emplace_back(p, kv.first);
  c->cap_free.clear();
  c->capturing = false;
  c->graphs.insert(g);
  *out = g;
  return ANIMA_OK;
}

int anima_graph_launch(anima_ctx* c, anima_graph* g) {
  CHECK_CTX(c);
  NOT_CAPTURING(c, "anima_graph_launch");
  if (!g || !c->graphs.count(g)) return fail(c, ANIMA_E_ARG, "anima_graph_launch: not a graph of this context");
  hipError_t e = hipGraphLaunch(g->exec, c->stream);
  if (e != hipSuccess) return hip_fail(c, e, "anima_graph_launch");
  return ANIMA_OK;
}

int anima_graph_destroy(anima_ctx* c, anima_graph* g) {
  if (!c) return fail(nullptr, ANIMA_E_ARG, "null context");
  if (!g) return ANIMA_OK;
  if (!c->graphs.count(g)) return fail(c, ANIMA_E_ARG, "anima_graph_destroy: not a graph of this context (or destroyed twice)");
  c->graphs.erase(g);
  release_graph(c, g, true);
  return ANIMA_OK;
}

}  // extern "C"
