// Internal declarations shared by the runtime and the kernel translation units.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <string>
#include <unordered_map>
#include <unordered_set>
#include <vector>

#include "../../include/anima.h"

namespace anima {

// Per-launch timing record (profiling mode).
struct ProfRec {
  const char* name;
  double flops, bytes;
  hipEvent_t a, b;
};

struct Stat {
  int64_t count = 0;
  double ms = 0, flops = 0, bytes = 0;
};

}  // namespace anima

struct anima_ctx {
  int device = 0;
  int num_cus = 256;  // compute units of the device (grid-size decisions)
  hipStream_t stream = nullptr;
  std::string err;
  bool lost = false;
  // pool: bucket size -> parked device buffers; live pointer -> bucket size
  std::unordered_map<size_t, std::vector<void*>> free_lists;
  std::unordered_map<void*, size_t> live;
  uint64_t allocated = 0, peak = 0, pooled = 0;
  // profiler
  bool profiling = false;
  std::vector<anima::ProfRec> recs;
  std::vector<hipEvent_t> spare_events;
  std::unordered_map<std::string, anima::Stat> stats;
  // timer
  hipEvent_t t0 = nullptr, t1 = nullptr;
  // host -> device staging: a ring of pinned slots, so that anima_h2d of a pageable source
  // returns without waiting for the stream; slot i is reusable once stage_ev[i] has completed
  static constexpr int kStageSlots = 4;
  static constexpr size_t kStageBytes = (size_t)4 << 20;
  void* stage[kStageSlots] = {};
  hipEvent_t stage_ev[kStageSlots] = {};
  bool stage_pending[kStageSlots] = {};
  int stage_next = 0;
  bool stage_failed = false;  // pinned allocation refused once: plain pageable copies from then on
  // queue marks (anima_mark / anima_wait_mark): a ring of events, ticket t in slot t % kMarks
  static constexpr int kMarks = 16;
  hipEvent_t marks[kMarks] = {};
  uint64_t mark_count = 0;
  // attention workspace (K in bf16/fp32, V transposed), grown on demand
  void* ws = nullptr;
  size_t ws_bytes = 0;
  // device address of this device's static K/V scratch (anima_attention_noalloc)
  void* scratch = nullptr;
  // ANIMA_W4_GRID_SCRATCH / ANIMA_W4_IN_GEMM (anima_set_w4_path)
  int w4_path = 0;
  // stream capture (anima_graph_begin .. anima_graph_end): buffers freed while capturing are
  // parked in cap_free, reused only by later allocations of the same capture, and owned by the
  // graph at the end (its replays keep using them); a workspace requested while capturing is such
  // a parked buffer of the requested size
  bool capturing = false;
  std::unordered_map<size_t, std::vector<void*>> cap_free;
  std::unordered_set<anima_graph*> graphs;
};

// A captured, instantiated HIP graph and the device buffers only its replays use.
struct anima_graph {
  hipGraph_t graph = nullptr;
  hipGraphExec_t exec = nullptr;
  std::vector<std::pair<void*, size_t>> owned;
};

namespace anima {

int fail(anima_ctx* c, int code, const char* fmt, ...);
int hip_fail(anima_ctx* c, hipError_t e, const char* what);
// Workspace of at least `bytes` (grows by synchronizing and reallocating).
int workspace(anima_ctx* c, size_t bytes, void** out);

// Launch bracket for the profiler: begin() before a kernel launch, end() after it.
struct Launch {
  anima_ctx* c;
  ProfRec rec;
  bool on;
  Launch(anima_ctx* ctx, const char* name, double flops, double bytes);
  // Checks the launch status; returns ANIMA_OK or a negative status.
  int end();
};

// ---- kernel launchers (attention.hip)
int attention_launch(anima_ctx* c, const anima_attn_desc* d);
int attention_launch_ws(anima_ctx* c, const anima_attn_desc* d, void* scratch);
// Looks up this device's scratch address (once per device; the context's device is current).
int attention_scratch_init(anima_ctx* c);
size_t attention_scratch_bytes();
int attention_noalloc_launch(anima_ctx* c, const anima_attn_desc* d);
int attention_prepare_kv_launch(anima_ctx* c, const anima_attn_desc* d, void* dst);
int64_t attention_kv_bytes(int B, int Hkv, int Lk, int precision);

// ---- kernel launchers (tgemm.hip)
int conv3x3_launch(anima_ctx* c, const anima_conv_desc* d);
int channel_norm_launch(anima_ctx* c, const float* x, const float* gamma, float* y, int64_t rows, int cols, int silu);
int to_rgba_launch(anima_ctx* c, const float* x, int64_t n, uint8_t* out);
int weight_unpack_w4_launch(anima_ctx* c, const anima_weight* W, int8_t* grid);
int attention_chunked_check(anima_ctx* c, const anima_attn_desc* d);
int attention_chunked_launch(anima_ctx* c, const anima_attn_desc* d, const int* kv_len);

// ---- kernel launchers (rowops.hip)
int qk_norm_rope_launch(anima_ctx* c, float* qkv, int64_t L, int H, int D, int64_t ld,
                        const float* qn, const float* kn, const float* cs, int64_t sin_off,
                        float eps);
int rmsnorm_launch(anima_ctx* c, const float* x, const float* w, float* y, int64_t rows,
                   int cols, float eps);
int rope_launch(anima_ctx* c, float* x, const float* cs, int64_t L, int H, int D,
                int64_t sin_off, int64_t row_stride, int64_t col_off);
int hadamard_launch(anima_ctx* c, const float* x, float* y, int64_t n);
int quant_rows_launch(anima_ctx* c, const float* x, int64_t M, int K, int rotate, int act, int8_t* q, float* s);
int quant_rows_bf16_launch(anima_ctx* c, const uint16_t* x, int64_t M, int K, int rotate, int8_t* q, float* s);
int layernorm_mod_launch(anima_ctx* c, const float* x, const float* mod, int64_t shift_off, int64_t scale_off,
                         int64_t rows, int cols, float eps, int rotate, float* y, int8_t* q, float* s);
int elementwise_launch(anima_ctx* c, int op, const float* a, const float* b, float* y, int64_t n);
int zero_launch(anima_ctx* c, float* y, int64_t n);
// forward: src = latents, dst = patches; inverse: src = final-layer output, dst = latents
int patchify_launch(anima_ctx* c, const float* src, float* dst, int B, int h, int w, bool inverse);

int split3_launch(anima_ctx* c, const float* src, uint16_t* dst, int64_t n);

// ---- kernel launchers (sampler.hip)
int sampler_step_launch(anima_ctx* c, const anima_sampler_desc* d);
int fill_random_launch(anima_ctx* c, void* dst, int64_t n, int kind, uint64_t seed, float lo, float hi);

// ---- kernel launchers (gemm.hip)
// s3_plane: split-weight (ANIMA_W_F32S3) plane stride in elements, 0 = N * K (a row block of
// larger planes passes the full planes' stride)
int linear_launch(anima_ctx* c, const anima_linear_desc* d, int64_t s3_plane = 0);
int linear_qkv_launch(anima_ctx* c, const anima_linear_desc* d, const anima_qkv_desc* p);
int linear_grouped_bf16_launch(anima_ctx* c, int G, int64_t M, int N, int K, const float* x, int64_t ldx,
                               int64_t x_gs, const uint16_t* w, int64_t w_gs, const float* bias, int64_t bias_gs,
                               float* out, int64_t ldc, int64_t out_gs);
int gemv_grouped_f32_launch(anima_ctx* c, int G, int N, int K, const float* x, int64_t x_gs, const float* w, int64_t w_gs,
                            float* y, int64_t y_gs, float alpha, int accumulate);

}  // namespace anima
